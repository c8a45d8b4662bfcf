//! Rust side of the drop-in boundary: `libwohper_hip.so` (gfx950 HIP
//! kernels behind `include/wohper_hip.h`) for the engine's DeepSeek-V4 FP8 /
//! FP4 kernel entry points.
//!
//! * [`sys`] is the raw `extern "C"` block.
//! * [`Status`] maps the library's codes; codes 1..=8 are
//!   `DeepSeekV4KernelError` in declaration order (E/deepseek_v4.rs:398-408),
//!   so an engine branch converts them one to one.
//! * [`Context`] is a safe owner of one library context with the slice
//!   (host-buffer) entry points the engine's functions take, plus the
//!   store calls that make weights resident.
//!
//! The engine adds a `rocm` feature and, at the top of each entry point, a
//! branch `#[cfg(feature = "rocm")] if let Some(ctx) = rocm_ctx() { ... }`
//! that calls the matching method here.  Device-pointer (`_async`) entry
//! points stay on [`sys`]: their pointers are the engine's own device
//! buffers.

pub mod sys;

use std::ffi::{CStr, CString};
use std::os::raw::c_int;

pub use sys::{WhExpertPackEntry, WhExpertRoute, WhGemvDesc, WhRouteOptions, WhTensor};

/// Library status codes (`enum wh_status`).
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum Status {
    EmptyShape,
    InvalidShape,
    PackedWeightTooSmall,
    ScaleTooSmall,
    InputTooSmall,
    OutputTooSmall,
    ScratchTooSmall,
    NonFiniteOutput,
    InvalidQuantFormat,
    NotResident,
    OutOfMemory,
    HipError,
    InvalidArgument,
    NonFiniteInput,
    Unsupported,
    TruncatedQuantBlock,
    InvalidQuantBlockMagic,
    UnsupportedQuantBlockVersion,
    InvalidQuantBlock,
    TensorIndexOutOfRange,
    Unaligned,
    Io,
    Unknown(c_int),
}

impl Status {
    pub fn from_code(code: c_int) -> Option<Status> {
        use Status::*;
        Some(match code {
            0 => return None,
            1 => EmptyShape,
            2 => InvalidShape,
            3 => PackedWeightTooSmall,
            4 => ScaleTooSmall,
            5 => InputTooSmall,
            6 => OutputTooSmall,
            7 => ScratchTooSmall,
            8 => NonFiniteOutput,
            9 => InvalidQuantFormat,
            10 => NotResident,
            11 => OutOfMemory,
            12 => HipError,
            13 => InvalidArgument,
            14 => NonFiniteInput,
            15 => Unsupported,
            16 => TruncatedQuantBlock,
            17 => InvalidQuantBlockMagic,
            18 => UnsupportedQuantBlockVersion,
            19 => InvalidQuantBlock,
            20 => TensorIndexOutOfRange,
            21 => Unaligned,
            22 => Io,
            c => Unknown(c),
        })
    }

    /// Codes 1..=8 are the engine's `DeepSeekV4KernelError` variants.
    pub fn is_kernel_error(self) -> bool {
        matches!(
            self,
            Status::EmptyShape
                | Status::InvalidShape
                | Status::PackedWeightTooSmall
                | Status::ScaleTooSmall
                | Status::InputTooSmall
                | Status::OutputTooSmall
                | Status::ScratchTooSmall
                | Status::NonFiniteOutput
        )
    }
}

/// A failed call: its status and the library's text for it (for the block
/// and pack codes, the reference's Display text of the error).
#[derive(Clone, Debug)]
pub struct Error {
    pub status: Status,
    pub message: String,
}

impl std::fmt::Display for Error {
    fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
        write!(f, "{:?}: {}", self.status, self.message)
    }
}

impl std::error::Error for Error {}

pub type Result<T> = std::result::Result<T, Error>;

fn check(code: c_int) -> Result<()> {
    match Status::from_code(code) {
        None => Ok(()),
        Some(status) => Err(Error { status, message: last_error() }),
    }
}

/// The library's text for the last failed call on this thread.
pub fn last_error() -> String {
    // SAFETY: the library returns a NUL-terminated thread-local string.
    unsafe {
        let p = sys::wh_last_error();
        if p.is_null() {
            String::new()
        } else {
            CStr::from_ptr(p).to_string_lossy().into_owned()
        }
    }
}

/// Owns one library context (one GPU, one HIP stream).  Calls are
/// serialised inside the library; the context may move between threads.
pub struct Context {
    raw: *mut sys::WhCtx,
}

unsafe impl Send for Context {}
unsafe impl Sync for Context {}

impl Context {
    pub fn new(device: i32) -> Result<Context> {
        let mut raw = std::ptr::null_mut();
        // SAFETY: `raw` is a valid out pointer.
        check(unsafe { sys::wh_init(device, &mut raw) })?;
        Ok(Context { raw })
    }

    pub fn as_ptr(&self) -> *mut sys::WhCtx {
        self.raw
    }

    // ------------------------------------------------------------- store

    /// An FP8 E4M3 tensor with block scales (f32 when `scales_f32`, else
    /// UE8M0 bytes), resident in HBM.
    pub fn store_fp8(&self, weight: &[u8], rows: usize, cols: usize, scales: &[u8], scales_f32: bool,
                     scale_rows: usize, scale_cols: usize) -> Result<WhTensor> {
        let fmt = if scales_f32 { sys::WH_SCALE_F32 } else { sys::WH_SCALE_UE8M0 };
        let mut t: WhTensor = 0;
        // SAFETY: the slices are valid for their lengths.
        check(unsafe {
            sys::wh_store_fp8(self.raw, weight.as_ptr(), weight.len(), rows, cols, scales.as_ptr().cast(),
                              scales.len(), fmt, scale_rows, scale_cols, &mut t)
        })?;
        Ok(t)
    }

    /// An FP4 E2M1 tensor (two values per byte, low nibble first) with a
    /// UE8M0 scale per group of cols / scale_cols.
    pub fn store_fp4(&self, packed: &[u8], scales: &[u8], rows: usize, cols: usize,
                     scale_cols: usize) -> Result<WhTensor> {
        let mut t: WhTensor = 0;
        // SAFETY: the slices are valid for their lengths.
        check(unsafe {
            sys::wh_store_fp4(self.raw, packed.as_ptr(), packed.len(), scales.as_ptr(), scales.len(), rows, cols,
                              scale_cols, &mut t)
        })?;
        Ok(t)
    }

    /// Keys three resident FP4 tensors as expert (layer, expert).
    pub fn store_expert(&self, layer: u32, expert: u32, w1: WhTensor, w3: WhTensor, w2: WhTensor) -> Result<()> {
        // SAFETY: plain values.
        check(unsafe { sys::wh_store_expert(self.raw, layer, expert, w1, w3, w2) })
    }

    /// Parses a ZCBLK01 expert block once (as
    /// `deepseek_v4_fp4_expert_from_quant_block`) and makes it resident.
    pub fn store_expert_block(&self, layer: u32, expert: u32, block: &[u8]) -> Result<()> {
        // SAFETY: the slice is valid for its length.
        check(unsafe { sys::wh_store_expert_block(self.raw, layer, expert, block.as_ptr(), block.len()) })
    }

    /// Loads the listed experts of a consolidated experts pack; returns how
    /// many were stored.
    pub fn store_expert_pack(&self, path: &str, entries: &[WhExpertPackEntry]) -> Result<usize> {
        let c = CString::new(path).map_err(|_| Error {
            status: Status::InvalidArgument,
            message: "pack path holds a NUL byte".into(),
        })?;
        let mut stored = 0usize;
        // SAFETY: `c` and `entries` outlive the call.
        check(unsafe { sys::wh_store_expert_pack(self.raw, c.as_ptr(), entries.as_ptr(), entries.len(), &mut stored) })?;
        Ok(stored)
    }

    pub fn release(&self, t: WhTensor) -> Result<()> {
        // SAFETY: plain values.
        check(unsafe { sys::wh_store_release(self.raw, t) })
    }

    /// Exact numerics (the default) keep the reference kernels' summation
    /// order bit for bit; off, the MFMA kernels run (each matvec within
    /// 1e-5 * ||w_row|| * ||x|| of the reference kernel).
    pub fn set_exact_numerics(&self, on: bool) -> Result<()> {
        // SAFETY: plain values.
        check(unsafe { sys::wh_set_exact_numerics(self.raw, on as c_int) })
    }

    // ------------------------------------------- the engine's entry points

    /// `gemv_fp8_e4m3_ue8m0_rows` (E/compute.rs:6244; row_start 0 and
    /// row_end rows is `…_tensorwise`, E/compute.rs:6174).  Returns the
    /// count of weights read, as the reference does.
    pub fn fp8_gemv(&self, w: WhTensor, row_start: usize, row_end: usize, input: &[f32],
                    output: &mut [f32]) -> Result<usize> {
        let mut values = 0usize;
        // SAFETY: the slices are valid for their lengths.
        check(unsafe {
            sys::wh_fp8_gemv(self.raw, w, row_start, row_end, input.as_ptr(), input.len(), output.as_mut_ptr(),
                             output.len(), &mut values)
        })?;
        Ok(values)
    }

    /// `gemv_fp8_e4m3_ue8m0_rows_multi` (E/compute.rs:6384): one output per
    /// input.  The slices are packed at the shortest input's and output's
    /// length, so a short one fails with the reference's InputTooSmall /
    /// OutputTooSmall.
    pub fn fp8_gemv_multi(&self, w: WhTensor, row_start: usize, row_end: usize, inputs: &[&[f32]],
                          outputs: &mut [&mut [f32]]) -> Result<usize> {
        if inputs.len() != outputs.len() {
            return Err(Error { status: Status::InvalidShape, message: "inputs and outputs differ in count".into() });
        }
        let n = inputs.len();
        let in_stride = inputs.iter().map(|x| x.len()).min().unwrap_or(0);
        let out_stride = outputs.iter().map(|y| y.len()).min().unwrap_or(0);
        let mut packed_in = Vec::with_capacity(n * in_stride);
        for x in inputs {
            packed_in.extend_from_slice(&x[..in_stride]);
        }
        let mut packed_out = vec![0f32; n * out_stride];
        let mut values = 0usize;
        // SAFETY: the packed buffers hold n strides each.
        check(unsafe {
            sys::wh_fp8_gemv_multi(self.raw, w, row_start, row_end, packed_in.as_ptr(), n, in_stride,
                                   packed_out.as_mut_ptr(), out_stride, &mut values)
        })?;
        let rows = row_end - row_start;
        for (i, y) in outputs.iter_mut().enumerate() {
            y[..rows].copy_from_slice(&packed_out[i * out_stride..i * out_stride + rows]);
        }
        Ok(values)
    }

    /// `fp4_e2m1_ue8m0_matvec_scalar` (E/deepseek_v4.rs:464).
    pub fn fp4_matvec(&self, w: WhTensor, input: &[f32], output: &mut [f32]) -> Result<()> {
        // SAFETY: the slices are valid for their lengths.
        check(unsafe {
            sys::wh_fp4_matvec(self.raw, w, input.as_ptr(), input.len(), output.as_mut_ptr(), output.len())
        })
    }

    /// `deepseek_v4_fp4_expert_forward_scalar` (E/deepseek_v4.rs:561) of a
    /// resident expert; `scratch_len` keeps the reference's ScratchTooSmall.
    pub fn fp4_expert_forward(&self, layer: u32, expert: u32, input: &[f32], output: &mut [f32],
                              scratch_len: usize) -> Result<()> {
        // SAFETY: the slices are valid for their lengths.
        check(unsafe {
            sys::wh_fp4_expert_forward(self.raw, layer, expert, input.as_ptr(), input.len(), output.as_mut_ptr(),
                                       output.len(), scratch_len)
        })
    }

    /// `fp8_act_quant_dequant_in_place` (E/compute.rs:2504).
    pub fn act_quant_dequant(&self, values: &mut [f32], block_size: usize) -> Result<()> {
        // SAFETY: the slice is valid for its length.
        check(unsafe { sys::wh_act_quant_dequant(self.raw, values.as_mut_ptr(), values.len(), block_size) })
    }

    /// `compute_active_experts` (E/compute.rs:1948): the weighted routed sum
    /// into `hidden`.
    pub fn routed_experts(&self, routes: &[WhExpertRoute], hidden: &mut [f32]) -> Result<()> {
        // SAFETY: the slices are valid for their lengths.
        check(unsafe {
            sys::wh_routed_experts(self.raw, routes.as_ptr(), routes.len(), hidden.as_mut_ptr(), hidden.len())
        })
    }

    /// `compute_active_and_shared_experts` (E/compute.rs:1872).
    pub fn routed_and_shared_experts(&self, routes: &[WhExpertRoute], shared_layer: u32, shared_expert: u32,
                                     hidden: &mut [f32]) -> Result<()> {
        // SAFETY: the slices are valid for their lengths.
        check(unsafe {
            sys::wh_routed_and_shared_experts(self.raw, routes.as_ptr(), routes.len(), shared_layer, shared_expert,
                                              hidden.as_mut_ptr(), hidden.len())
        })
    }

    /// The batch prefill MoE (E/server/generation.rs:2487-2569 with
    /// `accumulate_expert_for_positions`, E/compute.rs:1779): `npos`
    /// positions of `topk` routes; `shared` is (layer, expert) of the shared
    /// expert or None.
    pub fn moe_batch(&self, layer: u32, route_ids: &[u32], route_scores: &[f32], npos: usize, topk: usize,
                     shared: Option<(u32, u32)>, x: &[f32], out: &mut [f32]) -> Result<()> {
        if route_ids.len() < npos * topk || route_scores.len() < npos * topk {
            return Err(Error { status: Status::InputTooSmall, message: "route arrays too short".into() });
        }
        let (sl, se) = shared.unwrap_or((sys::WH_NO_SHARED_EXPERT, sys::WH_NO_SHARED_EXPERT));
        // SAFETY: lengths checked above; x and out are checked by the library.
        check(unsafe {
            sys::wh_moe_batch(self.raw, layer, route_ids.as_ptr(), route_scores.as_ptr(), npos, topk, sl, se,
                              x.as_ptr(), x.len(), out.as_mut_ptr(), out.len())
        })
    }

    /// `compute_deepseek_fp8_shared_expert_into_hidden` (E/compute.rs:5545).
    pub fn fp8_shared_expert(&self, w1: WhTensor, w3: WhTensor, w2: WhTensor, input: &[f32],
                             output: &mut [f32]) -> Result<()> {
        // SAFETY: the slices are valid for their lengths.
        check(unsafe {
            sys::wh_fp8_shared_expert(self.raw, w1, w3, w2, input.as_ptr(), input.len(), output.as_mut_ptr(),
                                      output.len())
        })
    }

    /// `route_experts_from_dense_block` (E/compute.rs:2129) on a layer whose
    /// router `wh_store_router` made resident: ids and weights of the
    /// selected experts.
    pub fn route_experts(&self, layer: u32, hidden: &[f32], active: usize, available: &[u32],
                         options: &WhRouteOptions) -> Result<(Vec<u32>, Vec<f32>)> {
        let cap = active.max(1);
        let mut ids = vec![0u32; cap];
        let mut scores = vec![0f32; cap];
        let mut n = 0usize;
        // SAFETY: the buffers hold `cap` entries.
        check(unsafe {
            sys::wh_route_experts(self.raw, layer, hidden.as_ptr(), hidden.len(), active, available.as_ptr(),
                                  available.len(), options, ids.as_mut_ptr(), scores.as_mut_ptr(), cap, &mut n)
        })?;
        ids.truncate(n);
        scores.truncate(n);
        Ok((ids, scores))
    }

    /// Waits for the library stream and reports its kernels' status.
    pub fn synchronize(&self) -> Result<()> {
        // SAFETY: plain value.
        check(unsafe { sys::wh_synchronize(self.raw) })
    }
}

impl Drop for Context {
    fn drop(&mut self) {
        // SAFETY: `raw` came from wh_init and is released once.
        unsafe {
            sys::wh_shutdown(self.raw);
        }
    }
}

#[cfg(test)]
mod tests {
    use super::*;

    #[test]
    fn kernel_error_codes_follow_the_engine_enum() {
        for (code, status) in [
            (1, Status::EmptyShape),
            (2, Status::InvalidShape),
            (3, Status::PackedWeightTooSmall),
            (4, Status::ScaleTooSmall),
            (5, Status::InputTooSmall),
            (6, Status::OutputTooSmall),
            (7, Status::ScratchTooSmall),
            (8, Status::NonFiniteOutput),
        ] {
            assert_eq!(Status::from_code(code), Some(status));
            assert!(status.is_kernel_error());
        }
        assert_eq!(Status::from_code(0), None);
        assert!(!Status::NotResident.is_kernel_error());
    }
}
