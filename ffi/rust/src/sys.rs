//! Raw bindings of `include/wohper_hip.h` (every entry point except the
//! `wh_debug_*` test hooks).  Status codes are `c_int`; see `crate::Status`.
#![allow(non_camel_case_types)]
use std::os::raw::{c_char, c_int, c_void};

/// The library context (one HIP stream and the store views of one GPU).
#[repr(C)]
pub struct WhCtx {
    _p: [u8; 0],
}
/// Handle into the weight store; 0 is none.
pub type WhTensor = u64;

/// One routed expert of a token: `IoBlockPtr{layer_id, expert_id,
/// route_weight}` (E/compute.rs:896-904) without the host pointer.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct WhExpertRoute {
    pub layer_id: u32,
    pub expert_id: u32,
    pub route_weight: f32,
}

/// One FP8 GEMV of `wh_fp8_gemv_batch_async`.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct WhGemvDesc {
    pub weight: WhTensor,
    pub row_start: usize,
    pub row_end: usize,
    pub x_dev: *const f32,
    pub y_dev: *mut f32,
}

/// `RouteOptions` (E/compute.rs:2096-2127); `hash_token_id < 0`: none.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct WhRouteOptions {
    pub math: i32,
    pub route_scale: f32,
    pub hash_token_id: i64,
}

/// One entry of a consolidated experts pack (E/model_format.rs:458-504).
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct WhExpertPackEntry {
    pub layer_id: u32,
    pub expert_id: u32,
    pub offset: u64,
    pub disk_bytes: u64,
    pub payload_bytes: u64,
}

/// One tensor record of a ZCBLK01 block (`QuantTensorLayout`,
/// E/compute.rs:441-451) with absolute byte offsets into the block.
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct WhQuantTensor {
    pub dtype_original: u16,
    pub quant_format: u16,
    pub rank: u32,
    pub flags: u32,
    pub scale: f32,
    pub zero_point: f32,
    pub name_offset: usize,
    pub name_len: usize,
    pub shape_offset: usize,
    pub data_offset: usize,
    pub data_bytes: usize,
}

/// One FP4 projection of an expert block (`Fp4Matvec`,
/// E/deepseek_v4.rs:411-417) as byte ranges of the block.
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct WhFp4View {
    pub rows: usize,
    pub cols: usize,
    pub scale_cols: usize,
    pub weight_offset: usize,
    pub weight_bytes: usize,
    pub scale_offset: usize,
    pub scale_bytes: usize,
}

/// `YarnRope` (E/compute.rs:2558-2572).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct WhYarn {
    pub factor: f32,
    pub beta_fast: f32,
    pub beta_slow: f32,
    pub original_seq_len: usize,
}

/// The resident tensors of one MLA decode layer
/// (`compute_deepseek_v4_mla_attention`, E/compute.rs:3924-4293).
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct WhMlaLayer {
    pub physical_layer: u32,
    pub heads: usize,
    pub nope_dim: usize,
    pub rope_dim: usize,
    pub o_groups: usize,
    pub o_lora_rank: usize,
    pub wq_a: WhTensor,
    pub wq_b: WhTensor,
    pub wkv: WhTensor,
    pub wo_a: WhTensor,
    pub wo_b: WhTensor,
    pub q_norm_bf16: *const u16,
    pub kv_norm_bf16: *const u16,
    pub sink: *const f32,
}

/// One DeepSeek-V4 mHC decode layer on the device (wh_mhc_layer).
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct WhMhcLayer {
    pub hc: usize,
    pub hidden: usize,
    pub sinkhorn_iters: usize,
    pub hc_eps: f32,
    pub hc_attn_fn: *const f32,
    pub hc_attn_scale: *const f32,
    pub hc_attn_base: *const f32,
    pub hc_ffn_fn: *const f32,
    pub hc_ffn_scale: *const f32,
    pub hc_ffn_base: *const f32,
    pub attn_norm_bf16: *const u16,
    pub ffn_norm_bf16: *const u16,
    pub attn: WhMlaLayer,
    pub layer_id: u32,
    pub active: usize,
    pub available_dev: *const u32,
    pub n_available: usize,
    pub route: WhRouteOptions,
    pub shared_layer: u32,
    pub shared_expert: u32,
}

pub const WH_SCALE_UE8M0: c_int = 0;
pub const WH_SCALE_F32: c_int = 1;
pub const WH_ROUTER_RAW_LOGITS: i32 = 0;
pub const WH_ROUTER_SQRT_SOFTPLUS: i32 = 1;
pub const WH_NO_SHARED_EXPERT: u32 = 0xFFFF_FFFF;
pub const WH_NOALLOC_SCRATCH_BYTES: usize = 8 << 20;

extern "C" {
    pub fn wh_init(device: c_int, out_: *mut *mut WhCtx) -> c_int;
    pub fn wh_shutdown(ctx: *mut WhCtx) -> c_int;
    pub fn wh_status_string(status: c_int) -> *const c_char;
    pub fn wh_synchronize(ctx: *mut WhCtx) -> c_int;
    pub fn wh_last_error() -> *const c_char;
    pub fn wh_build_info() -> *const c_char;
    pub fn wh_store_fp8(ctx: *mut WhCtx, weight: *const u8, weight_len: usize, rows: usize, cols: usize,
                        scales: *const c_void, scales_len: usize, scale_format: c_int, scale_rows: usize,
                        scale_cols: usize, out_: *mut WhTensor) -> c_int;
    pub fn wh_store_fp4(ctx: *mut WhCtx, packed: *const u8, packed_len: usize, scales: *const u8,
                        scales_len: usize, rows: usize, cols: usize, scale_cols: usize, out_: *mut WhTensor) -> c_int;
    pub fn wh_store_expert(ctx: *mut WhCtx, layer_id: u32, expert_id: u32, w1: WhTensor, w3: WhTensor,
                           w2: WhTensor) -> c_int;
    pub fn wh_quant_block_header(block: *const u8, block_len: usize, tensor_count: *mut u32,
                                 quant_format: *mut u32, flags: *mut u32) -> c_int;
    pub fn wh_quant_block_tensor(block: *const u8, block_len: usize, index: usize, out_: *mut WhQuantTensor) -> c_int;
    pub fn wh_quant_block_fp4_expert(block: *const u8, block_len: usize, out_: *mut WhFp4View) -> c_int;
    pub fn wh_store_expert_block(ctx: *mut WhCtx, layer_id: u32, expert_id: u32, block: *const u8,
                                 block_len: usize) -> c_int;
    pub fn wh_store_expert_pack(ctx: *mut WhCtx, pack_path: *const c_char, entries: *const WhExpertPackEntry,
                                n: usize, stored: *mut usize) -> c_int;
    pub fn wh_store_router(ctx: *mut WhCtx, layer_id: u32, block: *const u8, block_len: usize,
                           hidden_len: usize, found: *mut c_int) -> c_int;
    pub fn wh_route_experts(ctx: *mut WhCtx, layer_id: u32, hidden: *const f32, hidden_len: usize,
                            active_experts: usize, available: *const u32, n_available: usize,
                            options: *const WhRouteOptions, expert_ids: *mut u32, scores: *mut f32,
                            out_cap: usize, n_out: *mut usize) -> c_int;
    pub fn wh_route_experts_async(ctx: *mut WhCtx, layer_id: u32, x_dev: *const f32, hidden_len: usize,
                                  active_experts: usize, available_dev: *const u32, n_available: usize,
                                  options: *const WhRouteOptions, ids_dev: *mut u32, scores_dev: *mut f32,
                                  count_dev: *mut u32) -> c_int;
    pub fn wh_store_expert_synthetic(ctx: *mut WhCtx, layer_id: u32, expert_id: u32, hidden: usize,
                                     inter: usize, seed: u64, scale_lo: u32, scale_hi: u32) -> c_int;
    pub fn wh_store_fp8_synthetic(ctx: *mut WhCtx, rows: usize, cols: usize, seed: u64, stream: u64,
                                  scales: *const f32, scale_rows: usize, scale_cols: usize,
                                  out_: *mut WhTensor) -> c_int;
    pub fn wh_synth_fp8_host(seed: u64, stream: u64, weight: *mut u8, n: usize);
    pub fn wh_synth_fp4_host(seed: u64, stream: u64, packed: *mut u8, packed_len: usize, scales: *mut u8,
                             scales_len: usize, scale_lo: u32, scale_hi: u32);
    pub fn wh_store_release(ctx: *mut WhCtx, t: WhTensor) -> c_int;
    pub fn wh_store_usage(ctx: *mut WhCtx, device_bytes: *mut usize, tensors: *mut usize, experts: *mut usize) -> c_int;
    pub fn wh_tensor_dequant(ctx: *mut WhCtx, t: WhTensor, out_: *mut f32, out_len: usize) -> c_int;
    pub fn wh_fp8_gemv(ctx: *mut WhCtx, w: WhTensor, row_start: usize, row_end: usize, input: *const f32,
                       input_len: usize, output: *mut f32, output_len: usize, values_out: *mut usize) -> c_int;
    pub fn wh_fp8_gemv_multi(ctx: *mut WhCtx, w: WhTensor, row_start: usize, row_end: usize,
                             inputs: *const f32, n: usize, input_stride: usize, outputs: *mut f32,
                             output_stride: usize, values_out: *mut usize) -> c_int;
    pub fn wh_fp4_matvec(ctx: *mut WhCtx, w: WhTensor, input: *const f32, input_len: usize, output: *mut f32,
                         output_len: usize) -> c_int;
    pub fn wh_fp4_expert_forward(ctx: *mut WhCtx, layer_id: u32, expert_id: u32, input: *const f32,
                                 input_len: usize, output: *mut f32, output_len: usize, scratch_len: usize) -> c_int;
    pub fn wh_act_quant_dequant(ctx: *mut WhCtx, values: *mut f32, n: usize, block_size: usize) -> c_int;
    pub fn wh_routed_experts(ctx: *mut WhCtx, routes: *const WhExpertRoute, n_routes: usize,
                             hidden: *mut f32, hidden_len: usize) -> c_int;
    pub fn wh_routed_and_shared_experts(ctx: *mut WhCtx, routes: *const WhExpertRoute, n_routes: usize,
                                        shared_layer: u32, shared_expert: u32, hidden: *mut f32,
                                        hidden_len: usize) -> c_int;
    pub fn wh_routed_and_shared_experts_async(ctx: *mut WhCtx, routes: *const WhExpertRoute, n_routes: usize,
                                              shared_layer: u32, shared_expert: u32, x_dev: *const c_void,
                                              x_is_bf16: c_int, n_tokens: usize, out_dev: *mut f32) -> c_int;
    pub fn wh_routed_and_shared_experts_dev_async(ctx: *mut WhCtx, layer_id: u32, ids_dev: *const u32,
                                                  weights_dev: *const f32, count_dev: *const u32, n_slots: usize,
                                                  shared_layer: u32, shared_expert: u32, x_dev: *const c_void,
                                                  x_is_bf16: c_int, out_dev: *mut f32) -> c_int;
    pub fn wh_routed_and_shared_experts_noalloc_async(ctx: *mut WhCtx, routes: *const WhExpertRoute,
                                                      n_routes: usize, shared_layer: u32, shared_expert: u32,
                                                      x_dev: *const c_void, x_is_bf16: c_int,
                                                      n_tokens: usize, out_dev: *mut f32) -> c_int;
    pub fn wh_fp8_shared_expert(ctx: *mut WhCtx, w1: WhTensor, w3: WhTensor, w2: WhTensor, input: *const f32,
                                input_len: usize, output: *mut f32, output_len: usize) -> c_int;
    pub fn wh_fp8_shared_expert_async(ctx: *mut WhCtx, w1: WhTensor, w3: WhTensor, w2: WhTensor,
                                      x_dev: *const f32, y_dev: *mut f32) -> c_int;
    pub fn wh_set_exact_numerics(ctx: *mut WhCtx, on: c_int) -> c_int;
    pub fn wh_set_moe_mfma_min(ctx: *mut WhCtx, min_tokens: u32) -> c_int;
    pub fn wh_moe_batch(ctx: *mut WhCtx, layer_id: u32, route_ids: *const u32, route_scores: *const f32,
                        npos: usize, topk: usize, shared_layer: u32, shared_expert: u32, x: *const f32,
                        x_len: usize, out_: *mut f32, out_len: usize) -> c_int;
    pub fn wh_moe_batch_async(ctx: *mut WhCtx, layer_id: u32, route_ids_dev: *const u32,
                              route_scores_dev: *const f32, npos: usize, topk: usize, shared_layer: u32,
                              shared_expert: u32, x_dev: *const c_void, x_is_bf16: c_int, out_dev: *mut f32) -> c_int;
    pub fn wh_routed_experts_async(ctx: *mut WhCtx, routes: *const WhExpertRoute, n_routes: usize,
                                   x_dev: *const c_void, x_is_bf16: c_int, n_tokens: usize, out_dev: *mut f32) -> c_int;
    pub fn wh_fp8_gemv_batch_async(ctx: *mut WhCtx, descs: *const WhGemvDesc, n: usize) -> c_int;
    pub fn wh_fp8_gemv_multi_async(ctx: *mut WhCtx, w: WhTensor, row_start: usize, row_end: usize,
                                   x_dev: *const f32, n: usize, x_stride: usize, y_dev: *mut f32,
                                   y_stride: usize) -> c_int;
    pub fn wh_fp8_gemv_multi_groups_async(ctx: *mut WhCtx, w: WhTensor, row_start: usize, row_end: usize,
                                          group_rows: usize, x_dev: *const f32, x_group_stride: usize,
                                          n: usize, x_stride: usize, y_dev: *mut f32, y_stride: usize) -> c_int;
    pub fn wh_fp8_gemv_multi_pair_async(ctx: *mut WhCtx, w0: WhTensor, row_start0: usize, row_end0: usize,
                                        y0_dev: *mut f32, y0_stride: usize, w1: WhTensor, row_start1: usize,
                                        row_end1: usize, y1_dev: *mut f32, y1_stride: usize, x_dev: *const f32,
                                        n: usize, x_stride: usize) -> c_int;
    pub fn wh_set_fp8_mfma_min(ctx: *mut WhCtx, min_inputs: u32) -> c_int;
    pub fn wh_fp8_gemv_async(ctx: *mut WhCtx, w: WhTensor, row_start: usize, row_end: usize,
                             x_dev: *const f32, y_dev: *mut f32) -> c_int;
    pub fn wh_stream_status(ctx: *mut WhCtx) -> c_int;
    pub fn wh_graph_begin(ctx: *mut WhCtx) -> c_int;
    pub fn wh_graph_end(ctx: *mut WhCtx, out_: *mut u64) -> c_int;
    pub fn wh_graph_launch(ctx: *mut WhCtx, graph: u64) -> c_int;
    pub fn wh_graph_release(ctx: *mut WhCtx, graph: u64) -> c_int;
    pub fn wh_device_alloc(ctx: *mut WhCtx, bytes: usize, out_: *mut *mut c_void) -> c_int;
    pub fn wh_device_free(ctx: *mut WhCtx, ptr: *mut c_void) -> c_int;
    pub fn wh_memcpy(ctx: *mut WhCtx, dst: *mut c_void, src: *const c_void, bytes: usize, kind: c_int) -> c_int;
    pub fn wh_timer_start(ctx: *mut WhCtx) -> c_int;
    pub fn wh_timer_stop(ctx: *mut WhCtx, elapsed_us: *mut f64) -> c_int;
    pub fn wh_probe_read_floor(ctx: *mut WhCtx, buf_dev: *const c_void, buf_bytes: usize, bytes: usize,
                               reps: usize, best_us: *mut f64, best_grid: *mut u32, best_depth: *mut u32,
                               empty_us: *mut f64) -> c_int;
    pub fn wh_profile_routed(ctx: *mut WhCtx, routes: *const WhExpertRoute, n_routes: usize, n_sets: usize,
                             x_dev: *const c_void, x_is_bf16: c_int, out_dev: *mut f32, iters: usize,
                             us_per_launch: *mut f64) -> c_int;
    pub fn wh_profile_token_pipeline(ctx: *mut WhCtx, routes: *const WhExpertRoute, n_routes: usize,
                                     n_sets: usize, x_dev: *const c_void, x_is_bf16: c_int, x_stride: usize,
                                     out_dev: *mut f32, iters: usize, mode: c_int, us_per_token: *mut f64) -> c_int;
    pub fn wh_rope_inv_freqs(rope_dim: usize, theta: f32, yarn: *const WhYarn, out_: *mut f32, out_len: usize) -> c_int;
    pub fn wh_deepseek_rope_for_layer(physical_layer: u32, theta: *mut f32, yarn: *mut WhYarn,
                                      has_yarn: *mut c_int) -> c_int;
    pub fn wh_rms_norm_async(ctx: *mut WhCtx, x_dev: *const f32, out_dev: *mut f32, rows: usize, n: usize,
                             weight_bf16_dev: *const u16) -> c_int;
    pub fn wh_rope_async(ctx: *mut WhCtx, values_dev: *mut f32, rows: usize, row_stride: usize,
                         offset: usize, inv_freqs_dev: *const f32, pairs: usize, position: usize,
                         inverse: c_int) -> c_int;
    pub fn wh_act_quant_dequant_async(ctx: *mut WhCtx, values_dev: *mut f32, n: usize, block_size: usize) -> c_int;
    pub fn wh_window_attention_async(ctx: *mut WhCtx, q_dev: *const f32, heads: usize, head_dim: usize,
                                     nope_dim: usize, window_dev: *const f32, n_window: usize,
                                     window_stride: usize, comp_dev: *const f32, n_comp: usize,
                                     sink_dev: *const f32, inv_freqs_dev: *const f32, pairs: usize,
                                     token_pos: usize, scores_dev: *mut f32, out_dev: *mut f32) -> c_int;
    pub fn wh_mla_attention_decode_async(ctx: *mut WhCtx, layer: *const WhMlaLayer, token_pos: usize,
                                         hidden_dev: *mut f32, kv_cache_dev: *mut f32, kv_stride: usize,
                                         kv_capacity: usize, comp_dev: *const f32, n_comp: usize) -> c_int;
    pub fn wh_hc_split_sinkhorn_async(ctx: *mut WhCtx, mixes_dev: *const f32, scale_dev: *const f32,
                                      base_dev: *const f32, hc: usize, sinkhorn_iters: usize, eps: f32,
                                      pre_dev: *mut f32, post_dev: *mut f32, comb_dev: *mut f32) -> c_int;
    pub fn wh_hc_pre_async(ctx: *mut WhCtx, fn_dev: *const f32, scale_dev: *const f32, base_dev: *const f32,
                           hc: usize, hidden: usize, sinkhorn_iters: usize, eps: f32, x_dev: *const f32,
                           y_dev: *mut f32, post_dev: *mut f32, comb_dev: *mut f32) -> c_int;
    pub fn wh_hc_post_async(ctx: *mut WhCtx, y_dev: *const f32, residual_dev: *const f32,
                            post_dev: *const f32, comb_dev: *const f32, out_dev: *mut f32, hc: usize,
                            hidden: usize) -> c_int;
    pub fn wh_mla_attention_decode_batch_async(ctx: *mut WhCtx, layer: *const WhMlaLayer, positions: *const usize,
                                               npos: usize, hidden_dev: *mut f32, kv_cache_dev: *mut f32,
                                               kv_stride: usize, kv_capacity: usize, comp_dev: *const *const f32,
                                               n_comp: *const usize) -> c_int;
    pub fn wh_deepseek_mhc_layer_async(ctx: *mut WhCtx, layer: *const WhMhcLayer, token_pos: usize,
                                       hidden_dev: *mut f32, kv_cache_dev: *mut f32, kv_stride: usize,
                                       kv_capacity: usize, comp_dev: *const f32, n_comp: usize) -> c_int;
    pub fn wh_deepseek_mhc_layer_batch_async(ctx: *mut WhCtx, layer: *const WhMhcLayer, positions: *const usize,
                                             npos: usize, hidden_dev: *mut f32, kv_cache_dev: *mut f32,
                                             kv_stride: usize, kv_capacity: usize, comp_dev: *const *const f32,
                                             n_comp: *const usize, token_ids: *const i64) -> c_int;
}
