"""wohper_amd - MI355X (gfx950) decode hot path of wohper's DeepSeek-V4 engine.

Host mirror of the reference's kernel interface over the C ABI in
include/wohper_hip.h (libwohper_hip.so, built from wohper_amd/csrc):

  reference (engine/zc_infer_core/src)                this module
  -------------------------------------------------   ---------------------------------
  Fp4Matvec / DeepSeekV4Fp4Expert  deepseek_v4.rs:410-424      Fp4Matvec / DeepSeekV4Fp4Expert
  fp4_e2m1_ue8m0_matvec_scalar     deepseek_v4.rs:464          fp4_e2m1_ue8m0_matvec_scalar
  deepseek_v4_fp4_expert_forward_scalar deepseek_v4.rs:561     deepseek_v4_fp4_expert_forward_scalar
  gemv_fp8_e4m3_ue8m0_tensorwise   compute.rs:6174             gemv_fp8_e4m3_ue8m0_tensorwise
  gemv_fp8_e4m3_ue8m0_rows         compute.rs:6244             gemv_fp8_e4m3_ue8m0_rows
  gemv_fp8_e4m3_ue8m0_rows_multi   compute.rs:6384             gemv_fp8_e4m3_ue8m0_rows_multi
  fp8_act_quant_dequant_in_place   compute.rs:2504             fp8_act_quant_dequant_in_place
  compute_active_experts           compute.rs:1948             Context.routed_experts
  DeepSeekV4KernelError            deepseek_v4.rs:398-408      DeepSeekV4KernelError
  parse_quant_block                compute.rs:1099             quant_block_header / quant_block_tensor
  deepseek_v4_fp4_expert_from_quant_block compute.rs:1249      deepseek_v4_fp4_expert_from_quant_block
  load_optional_expert_pack        model_format.rs:458         model_format.load_optional_expert_pack
  route_experts_from_dense_block   compute.rs:2129             Context.store_router + Context.route_experts

The slice-based functions upload the weights for the call, as the reference
reads them from its I/O buffers; the resident path (Context.store_* plus the
handle-based methods) keeps them in HBM.  There is no CPU fallback: without
the HIP library or a GPU every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from pathlib import Path
from typing import Optional, Sequence

import numpy as np

_PKG = Path(__file__).resolve().parent
LIB_PATH = _PKG / "libwohper_hip.so"

STATUS_NAMES = {
    0: "Ok",
    1: "EmptyShape",
    2: "InvalidShape",
    3: "PackedWeightTooSmall",
    4: "ScaleTooSmall",
    5: "InputTooSmall",
    6: "OutputTooSmall",
    7: "ScratchTooSmall",
    8: "NonFiniteOutput",
    9: "InvalidQuantFormat",
    10: "NotResident",
    11: "OutOfMemory",
    12: "HipError",
    13: "InvalidArgument",
    14: "NonFiniteInput",
    15: "Unsupported",
    16: "TruncatedQuantBlock",
    17: "InvalidQuantBlockMagic",
    18: "UnsupportedQuantBlockVersion",
    19: "InvalidQuantBlock",
    20: "TensorIndexOutOfRange",
    21: "Unaligned",
    22: "Io",
}

# codes whose wh_last_error() text says what failed
_DETAILED = {2, 7, 11, 12, 13, 15, 16, 17, 18, 19, 20, 21, 22}

SCALE_UE8M0 = 0
SCALE_F32 = 1
NO_SHARED_EXPERT = 0xFFFFFFFF

# every symbol include/wohper_hip.h declares
EXPORTED = (
    "wh_init", "wh_shutdown", "wh_status_string", "wh_synchronize", "wh_stream", "wh_build_info",
    "wh_store_fp8", "wh_store_fp4", "wh_store_expert", "wh_store_expert_synthetic",
    "wh_synth_fp4_host", "wh_store_release", "wh_store_usage", "wh_tensor_dequant",
    "wh_fp8_gemv", "wh_fp8_gemv_multi", "wh_fp4_matvec", "wh_fp4_expert_forward",
    "wh_act_quant_dequant", "wh_routed_experts", "wh_routed_experts_async", "wh_fp8_gemv_async",
    "wh_stream_status", "wh_debug_eval", "wh_timer_start", "wh_timer_stop", "wh_profile_routed",
    "wh_probe_read_floor", "wh_profile_token_pipeline",
    "wh_store_fp8_synthetic", "wh_synth_fp8_host", "wh_routed_and_shared_experts", "wh_fp8_gemv_batch_async",
    "wh_routed_and_shared_experts_async", "wh_moe_batch", "wh_moe_batch_async", "wh_set_moe_mfma_min",
    "wh_debug_moe_batch_read", "wh_fp8_gemv_multi_async", "wh_fp8_gemv_multi_groups_async", "wh_fp8_gemv_multi_pair_async", "wh_set_fp8_mfma_min",
    "wh_set_exact_numerics", "wh_debug_moe_token_capture", "wh_debug_token_kernels",
    "wh_debug_moe_token_read", "wh_fp8_shared_expert", "wh_fp8_shared_expert_async",
    "wh_device_alloc", "wh_device_free", "wh_memcpy", "wh_last_error",
    "wh_quant_block_header", "wh_quant_block_tensor", "wh_quant_block_fp4_expert", "wh_store_expert_block",
    "wh_store_expert_pack", "wh_store_router", "wh_route_experts", "wh_route_experts_async",
    "wh_routed_and_shared_experts_noalloc_async",
    "wh_rope_inv_freqs", "wh_deepseek_rope_for_layer", "wh_rms_norm_async", "wh_rope_async",
    "wh_act_quant_dequant_async", "wh_window_attention_async", "wh_mla_attention_decode_async",
    "wh_mla_attention_decode_batch_async",
    "wh_hc_split_sinkhorn_async", "wh_hc_pre_async", "wh_hc_post_async",
    "wh_graph_begin", "wh_graph_end", "wh_graph_launch", "wh_graph_release",
    "wh_routed_and_shared_experts_dev_async", "wh_deepseek_mhc_layer_async", "wh_deepseek_mhc_layer_batch_async",
)

ROUTER_RAW_LOGITS = 0
ROUTER_SQRT_SOFTPLUS = 1


class DeepSeekV4KernelError(RuntimeError):
    """Mirror of the reference's error enum (E/deepseek_v4.rs:398-408) plus
    the store/runtime codes of the C ABI."""

    def __init__(self, code: int, where: str = "", detail: str = ""):
        self.code = int(code)
        self.name = STATUS_NAMES.get(self.code, f"status {code}")
        self.detail = detail
        text = self.name + (f" ({where})" if where else "") + (f": {detail}" if detail else "")
        super().__init__(text)


class WhYarn(ctypes.Structure):
    _fields_ = [("factor", ctypes.c_float), ("beta_fast", ctypes.c_float), ("beta_slow", ctypes.c_float),
                ("original_seq_len", ctypes.c_size_t)]


class WhMlaLayer(ctypes.Structure):
    _fields_ = [("physical_layer", ctypes.c_uint32), ("heads", ctypes.c_size_t), ("nope_dim", ctypes.c_size_t),
                ("rope_dim", ctypes.c_size_t), ("o_groups", ctypes.c_size_t), ("o_lora_rank", ctypes.c_size_t),
                ("wq_a", ctypes.c_uint64), ("wq_b", ctypes.c_uint64), ("wkv", ctypes.c_uint64),
                ("wo_a", ctypes.c_uint64), ("wo_b", ctypes.c_uint64), ("q_norm_bf16", ctypes.c_void_p),
                ("kv_norm_bf16", ctypes.c_void_p), ("sink", ctypes.c_void_p)]


class WhGemvDesc(ctypes.Structure):
    _fields_ = [("weight", ctypes.c_uint64), ("row_start", ctypes.c_size_t), ("row_end", ctypes.c_size_t),
                ("x_dev", ctypes.c_void_p), ("y_dev", ctypes.c_void_p)]


class WhExpertRoute(ctypes.Structure):
    _fields_ = [("layer_id", ctypes.c_uint32), ("expert_id", ctypes.c_uint32),
                ("route_weight", ctypes.c_float)]


class WhQuantTensor(ctypes.Structure):
    _fields_ = [("dtype_original", ctypes.c_uint16), ("quant_format", ctypes.c_uint16), ("rank", ctypes.c_uint32),
                ("flags", ctypes.c_uint32), ("scale", ctypes.c_float), ("zero_point", ctypes.c_float),
                ("name_offset", ctypes.c_size_t), ("name_len", ctypes.c_size_t), ("shape_offset", ctypes.c_size_t),
                ("data_offset", ctypes.c_size_t), ("data_bytes", ctypes.c_size_t)]


class WhFp4View(ctypes.Structure):
    _fields_ = [("rows", ctypes.c_size_t), ("cols", ctypes.c_size_t), ("scale_cols", ctypes.c_size_t),
                ("weight_offset", ctypes.c_size_t), ("weight_bytes", ctypes.c_size_t),
                ("scale_offset", ctypes.c_size_t), ("scale_bytes", ctypes.c_size_t)]


class WhRouteOptions(ctypes.Structure):
    _fields_ = [("math", ctypes.c_int32), ("route_scale", ctypes.c_float), ("hash_token_id", ctypes.c_int64)]


class WhMhcLayer(ctypes.Structure):
    _fields_ = [("hc", ctypes.c_size_t), ("hidden", ctypes.c_size_t), ("sinkhorn_iters", ctypes.c_size_t),
                ("hc_eps", ctypes.c_float), ("hc_attn_fn", ctypes.c_void_p), ("hc_attn_scale", ctypes.c_void_p),
                ("hc_attn_base", ctypes.c_void_p), ("hc_ffn_fn", ctypes.c_void_p), ("hc_ffn_scale", ctypes.c_void_p),
                ("hc_ffn_base", ctypes.c_void_p), ("attn_norm_bf16", ctypes.c_void_p),
                ("ffn_norm_bf16", ctypes.c_void_p), ("attn", WhMlaLayer), ("layer_id", ctypes.c_uint32),
                ("active", ctypes.c_size_t), ("available_dev", ctypes.c_void_p), ("n_available", ctypes.c_size_t),
                ("route", WhRouteOptions), ("shared_layer", ctypes.c_uint32), ("shared_expert", ctypes.c_uint32)]


class WhExpertPackEntry(ctypes.Structure):
    _fields_ = [("layer_id", ctypes.c_uint32), ("expert_id", ctypes.c_uint32), ("offset", ctypes.c_uint64),
                ("disk_bytes", ctypes.c_uint64), ("payload_bytes", ctypes.c_uint64)]


_lib: Optional[ctypes.CDLL] = None


def load_library(path: Optional[os.PathLike] = None) -> ctypes.CDLL:
    """Loads libwohper_hip.so.  Raises if it was not built - there is no
    fallback implementation."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise RuntimeError(f"{p} is missing: run `python -m wohper_amd.build` (no CPU fallback exists)")
    lib = ctypes.CDLL(str(p))
    c = ctypes
    vp, sz, u8p, f32p = c.c_void_p, c.c_size_t, c.POINTER(c.c_uint8), c.POINTER(c.c_float)
    sig = {
        "wh_init": (c.c_int, [c.c_int, c.POINTER(vp)]),
        "wh_shutdown": (c.c_int, [vp]),
        "wh_status_string": (c.c_char_p, [c.c_int]),
        "wh_synchronize": (c.c_int, [vp]),
        "wh_stream": (vp, [vp]),
        "wh_build_info": (c.c_char_p, []),
        "wh_last_error": (c.c_char_p, []),
        "wh_store_fp8": (c.c_int, [vp, u8p, sz, sz, sz, vp, sz, c.c_int, sz, sz, c.POINTER(c.c_uint64)]),
        "wh_store_fp4": (c.c_int, [vp, u8p, sz, u8p, sz, sz, sz, sz, c.POINTER(c.c_uint64)]),
        "wh_store_expert": (c.c_int, [vp, c.c_uint32, c.c_uint32, c.c_uint64, c.c_uint64, c.c_uint64]),
        "wh_store_expert_synthetic": (c.c_int, [vp, c.c_uint32, c.c_uint32, sz, sz, c.c_uint64,
                                                c.c_uint32, c.c_uint32]),
        "wh_synth_fp4_host": (None, [c.c_uint64, c.c_uint64, u8p, sz, u8p, sz, c.c_uint32, c.c_uint32]),
        "wh_store_release": (c.c_int, [vp, c.c_uint64]),
        "wh_store_usage": (c.c_int, [vp, c.POINTER(sz), c.POINTER(sz), c.POINTER(sz)]),
        "wh_tensor_dequant": (c.c_int, [vp, c.c_uint64, f32p, sz]),
        "wh_fp8_gemv": (c.c_int, [vp, c.c_uint64, sz, sz, f32p, sz, f32p, sz, c.POINTER(sz)]),
        "wh_fp8_gemv_multi": (c.c_int, [vp, c.c_uint64, sz, sz, f32p, sz, sz, f32p, sz, c.POINTER(sz)]),
        "wh_fp4_matvec": (c.c_int, [vp, c.c_uint64, f32p, sz, f32p, sz]),
        "wh_fp4_expert_forward": (c.c_int, [vp, c.c_uint32, c.c_uint32, f32p, sz, f32p, sz, sz]),
        "wh_act_quant_dequant": (c.c_int, [vp, f32p, sz, sz]),
        "wh_routed_experts": (c.c_int, [vp, c.POINTER(WhExpertRoute), sz, f32p, sz]),
        "wh_routed_experts_async": (c.c_int, [vp, c.POINTER(WhExpertRoute), sz, vp, c.c_int, sz, vp]),
        "wh_fp8_gemv_async": (c.c_int, [vp, c.c_uint64, sz, sz, vp, vp]),
        "wh_stream_status": (c.c_int, [vp]),
        "wh_routed_and_shared_experts_dev_async": (c.c_int, [vp, c.c_uint32, vp, vp, vp, sz, c.c_uint32, c.c_uint32,
                                                            vp, c.c_int, vp]),
        "wh_deepseek_mhc_layer_async": (c.c_int, [vp, c.POINTER(WhMhcLayer), sz, vp, vp, sz, sz, vp, sz]),
        "wh_deepseek_mhc_layer_batch_async": (c.c_int, [vp, c.POINTER(WhMhcLayer), c.POINTER(sz), sz, vp, vp, sz, sz,
                                                        c.POINTER(vp), c.POINTER(sz), c.POINTER(c.c_int64)]),
        "wh_graph_begin": (c.c_int, [vp]),
        "wh_graph_end": (c.c_int, [vp, c.POINTER(c.c_uint64)]),
        "wh_graph_launch": (c.c_int, [vp, c.c_uint64]),
        "wh_graph_release": (c.c_int, [vp, c.c_uint64]),
        "wh_debug_eval": (c.c_int, [vp, c.c_int, f32p, f32p, sz]),
        "wh_device_alloc": (c.c_int, [vp, sz, c.POINTER(vp)]),
        "wh_device_free": (c.c_int, [vp, vp]),
        "wh_memcpy": (c.c_int, [vp, vp, vp, sz, c.c_int]),
        "wh_timer_start": (c.c_int, [vp]),
        "wh_fp8_gemv_batch_async": (c.c_int, [vp, c.POINTER(WhGemvDesc), sz]),
        "wh_store_fp8_synthetic": (c.c_int, [vp, sz, sz, c.c_uint64, c.c_uint64, f32p, sz, sz,
                                             c.POINTER(c.c_uint64)]),
        "wh_synth_fp8_host": (None, [c.c_uint64, c.c_uint64, u8p, sz]),
        "wh_routed_and_shared_experts": (c.c_int, [vp, c.POINTER(WhExpertRoute), sz, c.c_uint32, c.c_uint32,
                                                   f32p, sz]),
        "wh_routed_and_shared_experts_async": (c.c_int, [vp, c.POINTER(WhExpertRoute), sz, c.c_uint32,
                                                         c.c_uint32, vp, c.c_int, sz, vp]),
        "wh_routed_and_shared_experts_noalloc_async": (c.c_int, [vp, c.POINTER(WhExpertRoute), sz, c.c_uint32,
                                                                 c.c_uint32, vp, c.c_int, sz, vp]),
        "wh_profile_token_pipeline": (c.c_int, [vp, c.POINTER(WhExpertRoute), sz, sz, vp, c.c_int, sz, vp, sz,
                                                c.c_int, c.POINTER(c.c_double)]),
        "wh_profile_routed": (c.c_int, [vp, c.POINTER(WhExpertRoute), sz, sz, vp, c.c_int, vp, sz,
                                        c.POINTER(c.c_double)]),
        "wh_timer_stop": (c.c_int, [vp, c.POINTER(c.c_double)]),
        "wh_probe_read_floor": (c.c_int, [vp, vp, sz, sz, sz, c.POINTER(c.c_double), c.POINTER(c.c_uint32),
                                          c.POINTER(c.c_uint32), c.POINTER(c.c_double)]),
        "wh_moe_batch": (c.c_int, [vp, c.c_uint32, c.POINTER(c.c_uint32), f32p, sz, sz, c.c_uint32, c.c_uint32,
                                   f32p, sz, f32p, sz]),
        "wh_moe_batch_async": (c.c_int, [vp, c.c_uint32, vp, vp, sz, sz, c.c_uint32, c.c_uint32, vp, c.c_int,
                                         vp]),
        "wh_set_moe_mfma_min": (c.c_int, [vp, c.c_uint32]),
        "wh_fp8_gemv_multi_async": (c.c_int, [vp, c.c_uint64, sz, sz, vp, sz, sz, vp, sz]),
        "wh_fp8_gemv_multi_groups_async": (c.c_int, [vp, c.c_uint64, sz, sz, sz, vp, sz, sz, sz, vp, sz]),
        "wh_fp8_gemv_multi_pair_async": (c.c_int, [vp, c.c_uint64, sz, sz, vp, sz, c.c_uint64, sz, sz, vp, sz, vp, sz,
                                                    sz]),
        "wh_set_fp8_mfma_min": (c.c_int, [vp, c.c_uint32]),
        "wh_debug_moe_batch_read": (c.c_int, [vp, c.c_int, vp, sz]),
        "wh_set_exact_numerics": (c.c_int, [vp, c.c_int]),
        "wh_fp8_shared_expert": (c.c_int, [vp, c.c_uint64, c.c_uint64, c.c_uint64, f32p, sz, f32p, sz]),
        "wh_fp8_shared_expert_async": (c.c_int, [vp, c.c_uint64, c.c_uint64, c.c_uint64, vp, vp]),
        "wh_debug_moe_token_capture": (c.c_int, [vp, c.c_int]),
        "wh_debug_token_kernels": (c.c_int, [vp, c.c_int]),
        "wh_debug_moe_token_read": (c.c_int, [vp, c.c_int, vp, sz]),
        "wh_quant_block_header": (c.c_int, [u8p, sz, c.POINTER(c.c_uint32), c.POINTER(c.c_uint32),
                                            c.POINTER(c.c_uint32)]),
        "wh_quant_block_tensor": (c.c_int, [u8p, sz, sz, c.POINTER(WhQuantTensor)]),
        "wh_quant_block_fp4_expert": (c.c_int, [u8p, sz, c.POINTER(WhFp4View)]),
        "wh_store_expert_block": (c.c_int, [vp, c.c_uint32, c.c_uint32, u8p, sz]),
        "wh_store_expert_pack": (c.c_int, [vp, c.c_char_p, c.POINTER(WhExpertPackEntry), sz, c.POINTER(sz)]),
        "wh_store_router": (c.c_int, [vp, c.c_uint32, u8p, sz, sz, c.POINTER(c.c_int)]),
        "wh_route_experts": (c.c_int, [vp, c.c_uint32, f32p, sz, sz, c.POINTER(c.c_uint32), sz,
                                       c.POINTER(WhRouteOptions), c.POINTER(c.c_uint32), f32p, sz, c.POINTER(sz)]),
        "wh_rope_inv_freqs": (c.c_int, [sz, c.c_float, c.POINTER(WhYarn), f32p, sz]),
        "wh_deepseek_rope_for_layer": (c.c_int, [c.c_uint32, c.POINTER(c.c_float), c.POINTER(WhYarn),
                                                 c.POINTER(c.c_int)]),
        "wh_rms_norm_async": (c.c_int, [vp, vp, vp, sz, sz, vp]),
        "wh_rope_async": (c.c_int, [vp, vp, sz, sz, sz, vp, sz, sz, c.c_int]),
        "wh_act_quant_dequant_async": (c.c_int, [vp, vp, sz, sz]),
        "wh_window_attention_async": (c.c_int, [vp, vp, sz, sz, sz, vp, sz, sz, vp, sz, vp, vp, sz, sz, vp, vp]),
        "wh_mla_attention_decode_async": (c.c_int, [vp, c.POINTER(WhMlaLayer), sz, vp, vp, sz, sz, vp, sz]),
        "wh_mla_attention_decode_batch_async": (c.c_int, [vp, c.POINTER(WhMlaLayer), c.POINTER(sz), sz, vp, vp, sz,
                                                          sz, c.POINTER(vp), c.POINTER(sz)]),
        "wh_hc_split_sinkhorn_async": (c.c_int, [vp, vp, vp, vp, sz, sz, c.c_float, vp, vp, vp]),
        "wh_hc_pre_async": (c.c_int, [vp, vp, vp, vp, sz, sz, sz, c.c_float, vp, vp, vp, vp]),
        "wh_hc_post_async": (c.c_int, [vp, vp, vp, vp, vp, vp, sz, sz]),
        "wh_route_experts_async": (c.c_int, [vp, c.c_uint32, vp, sz, sz, vp, sz, c.POINTER(WhRouteOptions), vp, vp,
                                             vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def _u8(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint8)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a: np.ndarray, ct):
    return a.ctypes.data_as(ctypes.POINTER(ct))


def _check(code: int, where: str = ""):
    if code != 0:
        detail = ""
        if code in _DETAILED and _lib is not None:
            detail = _lib.wh_last_error().decode(errors="replace")
        raise DeepSeekV4KernelError(code, where, detail)


class Context:
    """One device context: a HIP stream plus the HBM weight store."""

    def __init__(self, device: int = 0):
        self.lib = load_library()
        h = ctypes.c_void_p()
        _check(self.lib.wh_init(device, ctypes.byref(h)), "wh_init")
        self._h = h

    def close(self):
        if getattr(self, "_h", None):
            self.lib.wh_shutdown(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def stream(self) -> int:
        return self.lib.wh_stream(self._h)

    def synchronize(self):
        _check(self.lib.wh_synchronize(self._h), "deferred kernel status")

    # ------------------------------------------------------------- graphs
    def graph_begin(self):
        """Starts recording this thread's *_async calls into a HIP graph."""
        _check(self.lib.wh_graph_begin(self._h), "graph_begin")

    def graph_end(self) -> int:
        """Ends the recording; returns the graph handle."""
        out = ctypes.c_uint64()
        _check(self.lib.wh_graph_end(self._h, ctypes.byref(out)), "graph_end")
        return out.value

    def graph_capture(self, fn) -> int:
        """Records fn() into a graph; if fn raises, the capture is ended and
        dropped before the exception propagates."""
        self.graph_begin()
        try:
            fn()
        except BaseException:
            out = ctypes.c_uint64()
            if self.lib.wh_graph_end(self._h, ctypes.byref(out)) == 0:
                self.lib.wh_graph_release(self._h, out.value)
            raise
        return self.graph_end()

    def graph_launch(self, graph: int):
        _check(self.lib.wh_graph_launch(self._h, graph), "graph_launch")

    def graph_release(self, graph: int):
        _check(self.lib.wh_graph_release(self._h, graph), "graph_release")

    # ------------------------------------------------------------- store
    def store_fp8(self, weight, rows: int, cols: int, scales, scale_rows: int, scale_cols: int,
                  scale_format: int = SCALE_UE8M0) -> int:
        w = _u8(weight).reshape(-1)
        s = np.ascontiguousarray(scales, dtype=np.float32 if scale_format == SCALE_F32 else np.uint8).reshape(-1)
        out = ctypes.c_uint64()
        _check(self.lib.wh_store_fp8(self._h, _p(w, ctypes.c_uint8), w.size, rows, cols,
                                     s.ctypes.data_as(ctypes.c_void_p), s.nbytes, scale_format,
                                     scale_rows, scale_cols, ctypes.byref(out)), "store_fp8")
        return out.value

    def store_fp4(self, packed, scales, rows: int, cols: int, scale_cols: int) -> int:
        w, s = _u8(packed).reshape(-1), _u8(scales).reshape(-1)
        out = ctypes.c_uint64()
        _check(self.lib.wh_store_fp4(self._h, _p(w, ctypes.c_uint8), w.size, _p(s, ctypes.c_uint8), s.size,
                                     rows, cols, scale_cols, ctypes.byref(out)), "store_fp4")
        return out.value

    def store_expert(self, layer_id: int, expert_id: int, w1: int, w3: int, w2: int):
        _check(self.lib.wh_store_expert(self._h, layer_id, expert_id, w1, w3, w2), "store_expert")

    def store_fp4_expert(self, layer_id: int, expert_id: int, expert: "DeepSeekV4Fp4Expert"):
        hs = [self.store_fp4(m.packed_weight, m.ue8m0_scales, m.rows, m.cols, m.scale_cols)
              for m in (expert.w1, expert.w3, expert.w2)]
        self.store_expert(layer_id, expert_id, *hs)
        return hs

    def store_expert_synthetic(self, layer_id: int, expert_id: int, hidden: int, inter: int,
                               seed: int, scale_lo: int = 119, scale_hi: int = 127):
        _check(self.lib.wh_store_expert_synthetic(self._h, layer_id, expert_id, hidden, inter, seed,
                                                  scale_lo, scale_hi), "store_expert_synthetic")

    def store_expert_block(self, layer_id: int, expert_id: int, block) -> None:
        """Makes the FP4 expert of a ZCBLK01 block (bytes-like) resident under
        (layer_id, expert_id); a malformed block raises the reference's error."""
        b = _block_array(block)
        _check(self.lib.wh_store_expert_block(self._h, layer_id, expert_id, _p(b, ctypes.c_uint8), b.size),
               "store_expert_block")

    def store_expert_pack(self, pack, keys=None) -> int:
        """Loads experts of a consolidated pack (model_format.ExpertPackInfo)
        into the store, all of them or the (layer_id, expert_id) keys given,
        in file order.  Returns the number stored."""
        if keys is None:
            keys = list(pack.entries)
        chosen = sorted(((k, pack.entries[k]) for k in keys), key=lambda kv: kv[1].offset)
        arr = (WhExpertPackEntry * max(1, len(chosen)))(
            *[WhExpertPackEntry(k[0], k[1], e.offset, e.disk_bytes, e.payload_bytes) for k, e in chosen])
        stored = ctypes.c_size_t()
        _check(self.lib.wh_store_expert_pack(self._h, os.fsencode(str(pack.file)), arr, len(chosen),
                                             ctypes.byref(stored)), "store_expert_pack")
        return stored.value

    # ------------------------------------------------------------ router
    def store_router(self, layer_id: int, dense_block, hidden_len: int) -> bool:
        """Makes a layer's router (gate, bias, tid2eid) resident from its
        dense ZCBLK01 block; False when the block has no gate."""
        b = _block_array(dense_block)
        found = ctypes.c_int()
        _check(self.lib.wh_store_router(self._h, layer_id, _p(b, ctypes.c_uint8), b.size, hidden_len,
                                        ctypes.byref(found)), "store_router")
        return bool(found.value)

    @staticmethod
    def route_options(math: int = ROUTER_SQRT_SOFTPLUS, route_scale: float = 1.0, hash_token_id=None):
        return WhRouteOptions(math, route_scale, -1 if hash_token_id is None else int(hash_token_id))

    def route_experts(self, layer_id: int, hidden, active: int, available=None, math: int = ROUTER_SQRT_SOFTPLUS,
                      route_scale: float = 1.0, hash_token_id=None):
        """route_experts_from_dense_block (E/compute.rs:2129-2237) for a
        resident router: returns (expert ids, weights)."""
        h = _f32(hidden)
        av = None if available is None else np.ascontiguousarray(available, dtype=np.uint32)
        cap = max(1, int(active))
        ids = np.zeros(cap, np.uint32)
        sc = np.zeros(cap, np.float32)
        n = ctypes.c_size_t()
        opt = self.route_options(math, route_scale, hash_token_id)
        _check(self.lib.wh_route_experts(self._h, layer_id, _p(h, ctypes.c_float), h.size, active,
                                         None if av is None else _p(av, ctypes.c_uint32), 0 if av is None else av.size,
                                         ctypes.byref(opt), _p(ids, ctypes.c_uint32), _p(sc, ctypes.c_float), cap,
                                         ctypes.byref(n)), "route_experts")
        return ids[:n.value].copy(), sc[:n.value].copy()

    def route_experts_async(self, layer_id: int, x_ptr: int, hidden_len: int, active: int, avail_ptr: int,
                            n_available: int, ids_ptr: int, scores_ptr: int, count_ptr: int,
                            math: int = ROUTER_SQRT_SOFTPLUS, route_scale: float = 1.0, hash_token_id=None):
        opt = self.route_options(math, route_scale, hash_token_id)
        _check(self.lib.wh_route_experts_async(self._h, layer_id, ctypes.c_void_p(x_ptr), hidden_len, active,
                                               ctypes.c_void_p(avail_ptr) if avail_ptr else None, n_available,
                                               ctypes.byref(opt), ctypes.c_void_p(ids_ptr), ctypes.c_void_p(scores_ptr),
                                               ctypes.c_void_p(count_ptr)), "route_experts_async")

    def release(self, t: int):
        _check(self.lib.wh_store_release(self._h, t), "release")

    def usage(self):
        b, t, e = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
        _check(self.lib.wh_store_usage(self._h, ctypes.byref(b), ctypes.byref(t), ctypes.byref(e)))
        return b.value, t.value, e.value

    def dequant(self, t: int, rows: int, cols: int) -> np.ndarray:
        out = np.empty(rows * cols, np.float32)
        _check(self.lib.wh_tensor_dequant(self._h, t, _p(out, ctypes.c_float), out.size), "dequant")
        return out.reshape(rows, cols)

    # ---------------------------------------------------------- hot path
    def fp8_gemv(self, t: int, x, out_rows: int, row_start: int = 0, row_end: Optional[int] = None):
        x = _f32(x)
        if row_end is None:
            row_end = row_start + out_rows
        y = np.empty(out_rows, np.float32)
        vals = ctypes.c_size_t()
        _check(self.lib.wh_fp8_gemv(self._h, t, row_start, row_end, _p(x, ctypes.c_float), x.size,
                                    _p(y, ctypes.c_float), y.size, ctypes.byref(vals)), "fp8_gemv")
        return y, vals.value

    def fp8_gemv_multi(self, t: int, xs, row_start: int, row_end: int):
        xs = _f32(xs)
        n, k = xs.shape
        y = np.empty((n, row_end - row_start), np.float32)
        vals = ctypes.c_size_t()
        _check(self.lib.wh_fp8_gemv_multi(self._h, t, row_start, row_end, _p(xs, ctypes.c_float), n, k,
                                          _p(y, ctypes.c_float), y.shape[1], ctypes.byref(vals)),
               "fp8_gemv_multi")
        return y, vals.value

    def fp4_matvec(self, t: int, x, rows: int):
        x = _f32(x)
        y = np.empty(rows, np.float32)
        _check(self.lib.wh_fp4_matvec(self._h, t, _p(x, ctypes.c_float), x.size, _p(y, ctypes.c_float), y.size),
               "fp4_matvec")
        return y

    def fp4_expert_forward(self, layer_id: int, expert_id: int, x, out_len: int, scratch_len: int):
        x = _f32(x)
        y = np.empty(out_len, np.float32)
        _check(self.lib.wh_fp4_expert_forward(self._h, layer_id, expert_id, _p(x, ctypes.c_float), x.size,
                                              _p(y, ctypes.c_float), y.size, scratch_len), "fp4_expert_forward")
        return y

    def act_quant_dequant(self, values, block_size: int = 64) -> np.ndarray:
        v = _f32(values).copy()
        _check(self.lib.wh_act_quant_dequant(self._h, _p(v, ctypes.c_float), v.size, block_size), "act_quant")
        return v

    def routed_experts(self, routes: Sequence[tuple], hidden) -> np.ndarray:
        """compute_active_experts: routes = [(layer_id, expert_id, weight), ...]."""
        h = _f32(hidden).copy()
        arr = (WhExpertRoute * max(1, len(routes)))(*[WhExpertRoute(int(a), int(b), float(w)) for a, b, w in routes])
        _check(self.lib.wh_routed_experts(self._h, arr, len(routes), _p(h, ctypes.c_float), h.size),
               "routed_experts")
        return h

    def routed_experts_async(self, routes: Sequence[tuple], x_ptr: int, x_is_bf16: bool, n_tokens: int,
                             out_ptr: int):
        arr = (WhExpertRoute * len(routes))(*[WhExpertRoute(int(a), int(b), float(w)) for a, b, w in routes])
        _check(self.lib.wh_routed_experts_async(self._h, arr, len(routes), ctypes.c_void_p(x_ptr),
                                                int(x_is_bf16), n_tokens, ctypes.c_void_p(out_ptr)),
               "routed_experts_async")

    def fp8_gemv_async(self, t: int, row_start: int, row_end: int, x_ptr: int, y_ptr: int):
        _check(self.lib.wh_fp8_gemv_async(self._h, t, row_start, row_end, ctypes.c_void_p(x_ptr),
                                          ctypes.c_void_p(y_ptr)), "fp8_gemv_async")

    def device_alloc(self, nbytes: int) -> int:
        p = ctypes.c_void_p()
        _check(self.lib.wh_device_alloc(self._h, nbytes, ctypes.byref(p)), "device_alloc")
        return p.value or 0

    def device_free(self, ptr: int):
        _check(self.lib.wh_device_free(self._h, ctypes.c_void_p(ptr)), "device_free")

    def to_device(self, ptr: int, arr: np.ndarray):
        a = np.ascontiguousarray(arr)
        _check(self.lib.wh_memcpy(self._h, ctypes.c_void_p(ptr), a.ctypes.data_as(ctypes.c_void_p), a.nbytes, 0),
               "memcpy h2d")

    def from_device(self, arr: np.ndarray, ptr: int):
        assert arr.flags.c_contiguous
        _check(self.lib.wh_memcpy(self._h, arr.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(ptr), arr.nbytes, 1),
               "memcpy d2h")

    def timer_start(self):
        """Records the start event on the library stream."""
        _check(self.lib.wh_timer_start(self._h), "timer_start")

    def profile_routed(self, route_sets, x_dev: int, x_is_bf16: bool, out_dev: int, iters: int):
        """Mean microseconds per launch of (gate/up, down) over `iters`
        back-to-back launches cycling through `route_sets` (lists of
        (layer, expert, weight) of equal length)."""
        n = len(route_sets[0])
        flat = [r for rs in route_sets for r in rs]
        arr = (WhExpertRoute * len(flat))(*[WhExpertRoute(int(l), int(e), float(w)) for l, e, w in flat])
        us = (ctypes.c_double * 2)()
        _check(self.lib.wh_profile_routed(self._h, arr, n, len(route_sets), ctypes.c_void_p(x_dev), int(x_is_bf16),
                                          ctypes.c_void_p(out_dev), iters, us), "profile_routed")
        return us[0], us[1]

    def profile_token_pipeline(self, route_sets, x_dev: int, x_is_bf16: bool, x_stride: int, out_dev: int,
                               iters: int, graph: bool) -> float:
        """Mean microseconds per token of `iters` tokens (gate/up then down)
        enqueued by one library call, token i on route set i % len(route_sets)
        with input / output row i % len(route_sets); graph: replay of a HIP
        graph captured from the same launches."""
        n = len(route_sets[0])
        flat = [r for rs in route_sets for r in rs]
        arr = (WhExpertRoute * len(flat))(*[WhExpertRoute(int(l), int(e), float(w)) for l, e, w in flat])
        us = ctypes.c_double()
        _check(self.lib.wh_profile_token_pipeline(self._h, arr, n, len(route_sets), ctypes.c_void_p(x_dev),
                                                  int(x_is_bf16), x_stride, ctypes.c_void_p(out_dev), iters,
                                                  int(bool(graph)), ctypes.byref(us)), "profile_token_pipeline")
        return us.value

    def probe_read_floor(self, buf_dev: int, buf_bytes: int, nbytes: int, reps: int):
        """Fastest plain streaming read of nbytes per launch (rotating windows
        of the device buffer): (us, grid, depth, empty-launch us)."""
        us, e = ctypes.c_double(), ctypes.c_double()
        g, d = ctypes.c_uint32(), ctypes.c_uint32()
        _check(self.lib.wh_probe_read_floor(self._h, ctypes.c_void_p(buf_dev), buf_bytes, nbytes, reps,
                                            ctypes.byref(us), ctypes.byref(g), ctypes.byref(d), ctypes.byref(e)),
               "probe_read_floor")
        return us.value, g.value, d.value, e.value

    @staticmethod
    def gemv_descs(descs):
        """ctypes array of (tensor, row_start, row_end, x_ptr, y_ptr) descriptors."""
        return (WhGemvDesc * len(descs))(*[WhGemvDesc(t, r0, r1, x, y) for t, r0, r1, x, y in descs])

    @staticmethod
    def route_array(routes):
        """ctypes array of (layer, expert, weight) routes (at least one slot)."""
        return (WhExpertRoute * max(1, len(routes)))(*[WhExpertRoute(int(a), int(b), float(w)) for a, b, w in routes])

    def fp8_gemv_batch_async(self, descs):
        """descs: sequence of (tensor, row_start, row_end, x_ptr, y_ptr), or a
        prebuilt gemv_descs() array."""
        arr = descs if isinstance(descs, ctypes.Array) else self.gemv_descs(descs)
        _check(self.lib.wh_fp8_gemv_batch_async(self._h, arr, len(arr)), "fp8_gemv_batch_async")

    def store_fp8_synthetic(self, rows: int, cols: int, seed: int, stream: int, scales) -> int:
        """Device-generated FP8 tensor (bytes = synth_fp8_host's) with f32
        128x128 block scales `scales` [rows/128][cols/128]."""
        sc = _f32(scales)
        h = ctypes.c_uint64()
        _check(self.lib.wh_store_fp8_synthetic(self._h, rows, cols, seed, stream, _p(sc, ctypes.c_float),
                                               sc.shape[0], sc.shape[1], ctypes.byref(h)), "store_fp8_synthetic")
        return h.value

    def routed_and_shared_experts(self, routes, shared_key, x) -> np.ndarray:
        """out = shared(x) + routed(x) (compute_active_and_shared_experts)."""
        arr = (WhExpertRoute * max(1, len(routes)))(*[WhExpertRoute(int(a), int(b), float(w)) for a, b, w in routes])
        h = _f32(x).copy()
        _check(self.lib.wh_routed_and_shared_experts(self._h, arr, len(routes), shared_key[0], shared_key[1],
                                                     _p(h, ctypes.c_float), h.size), "routed_and_shared_experts")
        return h

    def routed_and_shared_experts_async(self, routes, shared_key, x_ptr: int, x_is_bf16: bool, n_tokens: int,
                                        out_ptr: int, n_routes=None):
        """routes: sequence of (layer, expert, weight), or a prebuilt
        route_array() with n_routes entries."""
        arr = routes if isinstance(routes, ctypes.Array) else self.route_array(routes)
        n = n_routes if n_routes is not None else len(routes)
        _check(self.lib.wh_routed_and_shared_experts_async(self._h, arr, n, shared_key[0], shared_key[1],
                                                           ctypes.c_void_p(x_ptr), int(x_is_bf16), n_tokens,
                                                           ctypes.c_void_p(out_ptr)), "routed_and_shared_experts_async")

    def routed_and_shared_experts_dev_async(self, layer_id: int, ids_ptr: int, weights_ptr: int, count_ptr: int,
                                            n_slots: int, shared_key, x_ptr: int, x_is_bf16: bool, out_ptr: int):
        """One token's experts from a route list in device memory (ids,
        weights, count as route_experts_async writes them); shared_key None:
        no shared expert."""
        sl, se = shared_key if shared_key is not None else (0, NO_SHARED_EXPERT)
        _check(self.lib.wh_routed_and_shared_experts_dev_async(
            self._h, layer_id, ctypes.c_void_p(ids_ptr), ctypes.c_void_p(weights_ptr), ctypes.c_void_p(count_ptr),
            n_slots, sl, se, ctypes.c_void_p(x_ptr), int(x_is_bf16), ctypes.c_void_p(out_ptr)),
            "routed_and_shared_experts_dev_async")

    def routed_and_shared_experts_noalloc_async(self, routes, shared_key, x_ptr: int, x_is_bf16: bool,
                                                n_tokens: int, out_ptr: int):
        """The allocation-free variant of routed_and_shared_experts_async: its
        working memory is the library's fixed per-GPU array."""
        arr = self.route_array(routes)
        _check(self.lib.wh_routed_and_shared_experts_noalloc_async(
            self._h, arr, len(routes), shared_key[0], shared_key[1], ctypes.c_void_p(x_ptr), int(x_is_bf16),
            n_tokens, ctypes.c_void_p(out_ptr)), "routed_and_shared_experts_noalloc_async")

    def moe_batch(self, layer_id: int, route_ids, route_scores, x, shared_key=None) -> np.ndarray:
        """Batched routed experts, expert-major (the batch-prefill MoE of
        E/server/generation.rs:2487-2569 with accumulate_expert_for_positions,
        E/compute.rs:1779-1810).  route_ids / route_scores: [npos, topk];
        x: [npos, hidden] f32.  shared_key: (layer, expert) of the shared
        expert, added as out = shared + routed."""
        ids = np.ascontiguousarray(route_ids, dtype=np.uint32)
        sc = _f32(route_scores)
        x = _f32(x)
        if ids.ndim != 2 or sc.shape != ids.shape or x.ndim != 2 or x.shape[0] != ids.shape[0]:
            raise ValueError("route_ids/route_scores must be [npos, topk] and x [npos, hidden]")
        out = np.zeros_like(x)
        sl, se = shared_key if shared_key is not None else (0, NO_SHARED_EXPERT)
        _check(self.lib.wh_moe_batch(self._h, layer_id, _p(ids, ctypes.c_uint32), _p(sc, ctypes.c_float),
                                     ids.shape[0], ids.shape[1], sl, se, _p(x, ctypes.c_float), x.size,
                                     _p(out, ctypes.c_float), out.size), "moe_batch")
        return out

    def moe_batch_async(self, layer_id: int, ids_ptr: int, scores_ptr: int, npos: int, topk: int, x_ptr: int,
                        x_is_bf16: bool, out_ptr: int, shared_key=None):
        """Device-pointer variant of moe_batch, enqueued on the library stream."""
        sl, se = shared_key if shared_key is not None else (0, NO_SHARED_EXPERT)
        _check(self.lib.wh_moe_batch_async(self._h, layer_id, ctypes.c_void_p(ids_ptr), ctypes.c_void_p(scores_ptr),
                                           npos, topk, sl, se, ctypes.c_void_p(x_ptr), int(x_is_bf16),
                                           ctypes.c_void_p(out_ptr)), "moe_batch_async")

    def fp8_gemv_multi_groups_async(self, t: int, row_start: int, row_end: int, group_rows: int, x_ptr: int,
                                    x_group_stride: int, n: int, x_stride: int, y_ptr: int, y_stride: int):
        """Row groups of group_rows rows, group g reading its n inputs at
        x_ptr + 4 * g * x_group_stride (strides in floats)."""
        _check(self.lib.wh_fp8_gemv_multi_groups_async(self._h, t, row_start, row_end, group_rows,
                                                       ctypes.c_void_p(x_ptr), x_group_stride, n, x_stride,
                                                       ctypes.c_void_p(y_ptr), y_stride), "fp8_gemv_multi_groups_async")

    def fp8_gemv_multi_pair_async(self, t0: int, row_start0: int, row_end0: int, y0_ptr: int, y0_stride: int,
                                  t1: int, row_start1: int, row_end1: int, y1_ptr: int, y1_stride: int, x_ptr: int,
                                  n: int, x_stride: int):
        """Two multi-input GEMVs on the same n inputs (wq_a and wkv), one
        launch where the MFMA path allows it (strides in floats)."""
        _check(self.lib.wh_fp8_gemv_multi_pair_async(self._h, t0, row_start0, row_end0, ctypes.c_void_p(y0_ptr),
                                                     y0_stride, t1, row_start1, row_end1, ctypes.c_void_p(y1_ptr),
                                                     y1_stride, ctypes.c_void_p(x_ptr), n, x_stride),
               "fp8_gemv_multi_pair_async")

    def set_fp8_mfma_min(self, n: int):
        """Multi-input FP8 GEMVs with at least n inputs use MFMA when exact
        numerics are off (0: never)."""
        _check(self.lib.wh_set_fp8_mfma_min(self._h, n), "set_fp8_mfma_min")

    def fp8_gemv_multi_async(self, t: int, row_start: int, row_end: int, x_ptr: int, n: int, x_stride: int,
                             y_ptr: int, y_stride: int):
        """n inputs (f32, stride x_stride floats) through rows [row_start,
        row_end) of an FP8 tensor, outputs at stride y_stride floats."""
        _check(self.lib.wh_fp8_gemv_multi_async(self._h, t, row_start, row_end, ctypes.c_void_p(x_ptr), n, x_stride,
                                                ctypes.c_void_p(y_ptr), y_stride), "fp8_gemv_multi_async")

    def set_moe_mfma_min(self, min_tokens: int):
        """Batch experts with at least min_tokens tokens run on MFMA (0: none)."""
        _check(self.lib.wh_set_moe_mfma_min(self._h, min_tokens), "set_moe_mfma_min")

    def fp8_shared_expert(self, w1: int, w3: int, w2: int, x, out_len: int) -> np.ndarray:
        """compute_deepseek_fp8_shared_expert_into_hidden on resident FP8
        tensors: returns the w2-rows output."""
        x = _f32(x)
        y = np.empty(out_len, np.float32)
        _check(self.lib.wh_fp8_shared_expert(self._h, w1, w3, w2, _p(x, ctypes.c_float), x.size,
                                             _p(y, ctypes.c_float), y.size), "fp8_shared_expert")
        return y

    def fp8_shared_expert_async(self, w1: int, w3: int, w2: int, x_ptr: int, y_ptr: int):
        _check(self.lib.wh_fp8_shared_expert_async(self._h, w1, w3, w2, ctypes.c_void_p(x_ptr),
                                                   ctypes.c_void_p(y_ptr)), "fp8_shared_expert_async")

    # ------------------------------------------------------------ MLA glue
    def rms_norm_async(self, x_ptr: int, out_ptr: int, rows: int, n: int, weight_bf16_ptr: int = 0):
        _check(self.lib.wh_rms_norm_async(self._h, x_ptr, out_ptr, rows, n, weight_bf16_ptr or None),
               "rms_norm_async")

    def rope_async(self, values_ptr: int, rows: int, row_stride: int, offset: int, inv_freqs_ptr: int, pairs: int,
                   position: int, inverse: bool = False):
        _check(self.lib.wh_rope_async(self._h, values_ptr, rows, row_stride, offset, inv_freqs_ptr, pairs, position,
                                      int(bool(inverse))), "rope_async")

    def act_quant_dequant_async(self, values_ptr: int, n: int, block_size: int = 64):
        _check(self.lib.wh_act_quant_dequant_async(self._h, values_ptr, n, block_size), "act_quant_dequant_async")

    def window_attention_async(self, q_ptr: int, heads: int, head_dim: int, nope_dim: int, win_ptr: int,
                               n_window: int, window_stride: int, comp_ptr: int, n_comp: int, sink_ptr: int,
                               inv_freqs_ptr: int, pairs: int, token_pos: int, scores_ptr: int, out_ptr: int):
        _check(self.lib.wh_window_attention_async(self._h, q_ptr, heads, head_dim, nope_dim, win_ptr or None,
                                                  n_window, window_stride, comp_ptr or None, n_comp,
                                                  sink_ptr or None, inv_freqs_ptr or None, pairs, token_pos,
                                                  scores_ptr, out_ptr), "window_attention_async")

    def mla_attention_decode_async(self, layer: "WhMlaLayer", token_pos: int, hidden_ptr: int, kv_ptr: int,
                                   kv_stride: int, kv_capacity: int, comp_ptr: int = 0, n_comp: int = 0):
        _check(self.lib.wh_mla_attention_decode_async(self._h, ctypes.byref(layer), token_pos, hidden_ptr, kv_ptr,
                                                      kv_stride, kv_capacity, comp_ptr or None, n_comp),
               "mla_attention_decode_async")

    def mla_attention_decode_batch_async(self, layer: "WhMlaLayer", positions, hidden_ptr: int, kv_ptr: int,
                                         kv_stride: int, kv_capacity: int, comps=None):
        """compute_deepseek_v4_mla_attention_batch over ascending positions:
        hidden_ptr holds len(positions) rows of hidden floats, overwritten
        with the attention outputs.  comps: None, or one (device pointer,
        row count) of compressed rows per position."""
        n = len(positions)
        pos = (ctypes.c_size_t * n)(*[int(p) for p in positions])
        cp = cn = None
        if comps is not None:
            cp = (ctypes.c_void_p * n)(*[int(p) or None for p, _ in comps])
            cn = (ctypes.c_size_t * n)(*[int(k) for _, k in comps])
        _check(self.lib.wh_mla_attention_decode_batch_async(self._h, ctypes.byref(layer), pos, n, hidden_ptr, kv_ptr,
                                                            kv_stride, kv_capacity, cp, cn),
               "mla_attention_decode_batch_async")

    def deepseek_mhc_layer_async(self, layer: "WhMhcLayer", token_pos: int, hidden_ptr: int, kv_ptr: int,
                                 kv_stride: int, kv_capacity: int, comp_ptr: int = 0, n_comp: int = 0):
        """One decode layer (hc_pre -> norm -> MLA -> hc_post -> hc_pre ->
        norm -> router -> shared + routed experts -> hc_post) on the hc
        copies of the hidden state at hidden_ptr, in place."""
        _check(self.lib.wh_deepseek_mhc_layer_async(self._h, ctypes.byref(layer), token_pos, hidden_ptr, kv_ptr,
                                                    kv_stride, kv_capacity, comp_ptr or None, n_comp),
               "deepseek_mhc_layer_async")

    def deepseek_mhc_layer_batch_async(self, layer: "WhMhcLayer", positions, hidden_ptr: int, kv_ptr: int,
                                       kv_stride: int, kv_capacity: int, comps=None, token_ids=None):
        """The batched layer of prefill and verify over ascending positions:
        hidden_ptr holds len(positions) states of hc * hidden floats, each
        updated in place; the routed experts of all positions run as one
        batch MoE.  comps as in mla_attention_decode_batch_async;
        token_ids: each position's token for a hash layer, or None for the
        layer's route options."""
        n = len(positions)
        pos = (ctypes.c_size_t * n)(*[int(p) for p in positions])
        cp = cn = tk = None
        if comps is not None:
            cp = (ctypes.c_void_p * n)(*[int(p) or None for p, _ in comps])
            cn = (ctypes.c_size_t * n)(*[int(k) for _, k in comps])
        if token_ids is not None:
            tk = (ctypes.c_int64 * n)(*[int(t) for t in token_ids])
        _check(self.lib.wh_deepseek_mhc_layer_batch_async(self._h, ctypes.byref(layer), pos, n, hidden_ptr, kv_ptr,
                                                          kv_stride, kv_capacity, cp, cn, tk),
               "deepseek_mhc_layer_batch_async")

    # ------------------------------------------------------------------ mHC
    def hc_split_sinkhorn_async(self, mixes_ptr: int, scale_ptr: int, base_ptr: int, hc: int, iters: int,
                                eps: float, pre_ptr: int, post_ptr: int, comb_ptr: int):
        _check(self.lib.wh_hc_split_sinkhorn_async(self._h, mixes_ptr, scale_ptr, base_ptr, hc, iters, eps, pre_ptr,
                                                   post_ptr, comb_ptr), "hc_split_sinkhorn_async")

    def hc_pre_async(self, fn_ptr: int, scale_ptr: int, base_ptr: int, hc: int, hidden: int, iters: int, eps: float,
                     x_ptr: int, y_ptr: int, post_ptr: int, comb_ptr: int):
        _check(self.lib.wh_hc_pre_async(self._h, fn_ptr, scale_ptr, base_ptr, hc, hidden, iters, eps, x_ptr, y_ptr,
                                        post_ptr, comb_ptr), "hc_pre_async")

    def hc_post_async(self, y_ptr: int, res_ptr: int, post_ptr: int, comb_ptr: int, out_ptr: int, hc: int,
                      hidden: int):
        _check(self.lib.wh_hc_post_async(self._h, y_ptr, res_ptr, post_ptr, comb_ptr, out_ptr, hc, hidden),
               "hc_post_async")

    def set_exact_numerics(self, on: bool):
        """True (default): routed-expert matvecs in the reference kernel's
        summation order (bit-identical); False: split-K kernels, each matvec
        within 1e-5 * ||w_row|| * ||x|| of it."""
        _check(self.lib.wh_set_exact_numerics(self._h, int(bool(on))), "set_exact_numerics")

    def debug_token_kernels(self, mask: int):
        """MFMA token kernels at hidden 4096 / inter 2048: bit 0 gate/up, bit 1
        down on the LDS-streaming kernels (default 1), else the register-ring
        kernels."""
        _check(self.lib.wh_debug_token_kernels(self._h, int(mask)), "debug_token_kernels")

    def debug_moe_token_capture(self, on: bool):
        _check(self.lib.wh_debug_moe_token_capture(self._h, int(bool(on))), "debug_moe_token_capture")

    def debug_moe_token_read(self, which: int, shape) -> np.ndarray:
        """Last routed-expert call: 0 gate/up [T][n][2][inter], 1 SwiGLU
        [T][n][inter], 2 expert outputs [T][n][hidden] (f32)."""
        out = np.empty(shape, np.float32)
        _check(self.lib.wh_debug_moe_token_read(self._h, which, out.ctypes.data_as(ctypes.c_void_p), out.nbytes),
               "debug_moe_token_read")
        return out

    def debug_moe_batch_read(self, which: int, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype)
        _check(self.lib.wh_debug_moe_batch_read(self._h, which, out.ctypes.data_as(ctypes.c_void_p), out.nbytes),
               "debug_moe_batch_read")
        return out

    def timer_stop(self) -> float:
        """Device microseconds since timer_start (waits for the stream)."""
        us = ctypes.c_double()
        _check(self.lib.wh_timer_stop(self._h, ctypes.byref(us)), "timer_stop")
        return us.value

    def debug_eval(self, fn: int, x) -> np.ndarray:
        x = _f32(x)
        y = np.empty_like(x)
        _check(self.lib.wh_debug_eval(self._h, fn, _p(x, ctypes.c_float), _p(y, ctypes.c_float), x.size),
               "debug_eval")
        return y


# ------------------------------------------- reference-shaped slice API
@dataclass
class Fp4Matvec:
    """E/deepseek_v4.rs:410-417"""
    packed_weight: np.ndarray
    ue8m0_scales: np.ndarray
    rows: int
    cols: int
    scale_cols: int


@dataclass
class DeepSeekV4Fp4Expert:
    """E/deepseek_v4.rs:419-424"""
    w1: Fp4Matvec
    w3: Fp4Matvec
    w2: Fp4Matvec


def _block_array(block) -> np.ndarray:
    if isinstance(block, np.ndarray):
        return np.ascontiguousarray(block, dtype=np.uint8).reshape(-1)
    return np.frombuffer(bytes(block), dtype=np.uint8)


@dataclass
class QuantTensor:
    """QuantTensorLayout (E/compute.rs:441-451) with its name, shape and data
    read out of the block."""
    dtype_original: int
    quant_format: int
    rank: int
    flags: int
    name: bytes
    shape: tuple
    data: np.ndarray
    scale: float
    zero_point: float

    @property
    def role(self) -> int:
        """TensorRole code (E/compute.rs:455-471)."""
        return self.flags & 0xFFFF


def quant_block_header(block):
    """parse_quant_block (E/compute.rs:1099-1148): (tensor_count,
    quant_format, flags).  Host only."""
    lib = load_library()
    b = _block_array(block)
    n, q, f = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint32()
    _check(lib.wh_quant_block_header(_p(b, ctypes.c_uint8), b.size, ctypes.byref(n), ctypes.byref(q),
                                     ctypes.byref(f)), "parse_quant_block")
    return n.value, q.value, f.value


def quant_block_tensor(block, index: int) -> QuantTensor:
    """QuantBlockLayout::tensor (E/compute.rs:545-600).  Host only."""
    lib = load_library()
    b = _block_array(block)
    t = WhQuantTensor()
    _check(lib.wh_quant_block_tensor(_p(b, ctypes.c_uint8), b.size, index, ctypes.byref(t)), "quant_block_tensor")
    dims = b[t.shape_offset + 4:t.shape_offset + 4 + 8 * t.rank].view("<u8") if t.rank else np.zeros(0, np.uint64)
    return QuantTensor(t.dtype_original, t.quant_format, t.rank, t.flags,
                       b[t.name_offset:t.name_offset + t.name_len].tobytes(), tuple(int(d) for d in dims),
                       b[t.data_offset:t.data_offset + t.data_bytes], t.scale, t.zero_point)


def deepseek_v4_fp4_expert_from_quant_block(block) -> DeepSeekV4Fp4Expert:
    """E/compute.rs:1249-1268: the w1/w3/w2 FP4 projections of an expert
    block, as views of the block's bytes.  Host only."""
    lib = load_library()
    b = _block_array(block)
    views = (WhFp4View * 3)()
    _check(lib.wh_quant_block_fp4_expert(_p(b, ctypes.c_uint8), b.size, views),
           "deepseek_v4_fp4_expert_from_quant_block")
    ms = [Fp4Matvec(b[v.weight_offset:v.weight_offset + v.weight_bytes],
                    b[v.scale_offset:v.scale_offset + v.scale_bytes], v.rows, v.cols, v.scale_cols) for v in views]
    return DeepSeekV4Fp4Expert(*ms)


_default_ctx: Optional[Context] = None


def default_context() -> Context:
    global _default_ctx
    if _default_ctx is None:
        _default_ctx = Context(0)
    return _default_ctx


def fp4_e2m1_ue8m0_matvec_scalar(spec: Fp4Matvec, input, output: np.ndarray, ctx: Optional[Context] = None):
    """E/deepseek_v4.rs:464 on the GPU; output[:rows] is written."""
    ctx = ctx or default_context()
    x = _f32(input)
    # validate_fp4_matvec order (E/deepseek_v4.rs:434-462)
    if spec.rows == 0 or spec.cols == 0 or spec.scale_cols == 0:
        raise DeepSeekV4KernelError(1)
    if x.size < spec.cols:
        raise DeepSeekV4KernelError(5)
    if output.size < spec.rows:
        raise DeepSeekV4KernelError(6)
    t = ctx.store_fp4(spec.packed_weight, spec.ue8m0_scales, spec.rows, spec.cols, spec.scale_cols)
    try:
        output[: spec.rows] = ctx.fp4_matvec(t, x[: spec.cols], spec.rows)
    finally:
        ctx.release(t)


def deepseek_v4_fp4_expert_forward_scalar(expert: DeepSeekV4Fp4Expert, input, output: np.ndarray,
                                          scratch_len: int, ctx: Optional[Context] = None,
                                          key=(0xFFFFFFFF, 0xFFFFFFFF)):
    """E/deepseek_v4.rs:561 on the GPU."""
    ctx = ctx or default_context()
    x = _f32(input)
    hs = ctx.store_fp4_expert(key[0], key[1], expert)
    try:
        output[: expert.w2.rows] = ctx.fp4_expert_forward(key[0], key[1], x, output.size, scratch_len)[: expert.w2.rows]
    finally:
        for h in hs:
            ctx.release(h)


def fp8_act_quant_dequant_in_place(values: np.ndarray, block_size: int, ctx: Optional[Context] = None):
    """E/compute.rs:2504 on the GPU (values: float32 array, modified in place)."""
    ctx = ctx or default_context()
    values[...] = ctx.act_quant_dequant(values, block_size).reshape(values.shape)


def gemv_fp8_e4m3_ue8m0_rows(weight, rows: int, cols: int, scales, scale_rows: int, scale_cols: int,
                             row_start: int, row_end: int, input, output: np.ndarray,
                             scale_format: int = SCALE_UE8M0, ctx: Optional[Context] = None) -> int:
    """E/compute.rs:6244 on the GPU; returns the consumed value count."""
    ctx = ctx or default_context()
    t = ctx.store_fp8(weight, rows, cols, scales, scale_rows, scale_cols, scale_format)
    try:
        y, vals = ctx.fp8_gemv(t, input, row_end - row_start, row_start, row_end)
        output[: row_end - row_start] = y
        return vals
    finally:
        ctx.release(t)


def gemv_fp8_e4m3_ue8m0_tensorwise(weight, rows: int, cols: int, scales, scale_rows: int, scale_cols: int,
                                   input, output: np.ndarray, scale_format: int = SCALE_UE8M0,
                                   ctx: Optional[Context] = None) -> int:
    """E/compute.rs:6174 on the GPU."""
    return gemv_fp8_e4m3_ue8m0_rows(weight, rows, cols, scales, scale_rows, scale_cols, 0, rows, input,
                                    output, scale_format, ctx)


def gemv_fp8_e4m3_ue8m0_rows_multi(weight, rows: int, cols: int, scales, scale_rows: int, scale_cols: int,
                                   row_start: int, row_end: int, inputs, scale_format: int = SCALE_UE8M0,
                                   ctx: Optional[Context] = None):
    """E/compute.rs:6384 on the GPU: returns (outputs [n x rows], values)."""
    ctx = ctx or default_context()
    t = ctx.store_fp8(weight, rows, cols, scales, scale_rows, scale_cols, scale_format)
    try:
        return ctx.fp8_gemv_multi(t, inputs, row_start, row_end)
    finally:
        ctx.release(t)


def rope_inv_freqs(rope_dim: int, theta: float, yarn=None) -> np.ndarray:
    """rope_inv_freqs (E/compute.rs:2591-2620): yarn = (factor, beta_fast,
    beta_slow, original_seq_len) or None."""
    lib = load_library()
    out = np.zeros(max(rope_dim // 2, 1), np.float32)
    y = WhYarn(*yarn) if yarn is not None else None
    _check(lib.wh_rope_inv_freqs(rope_dim, theta, ctypes.byref(y) if y is not None else None,
                                 _p(out, ctypes.c_float), out.size), "rope_inv_freqs")
    return out[:rope_dim // 2]


def deepseek_rope_for_layer(physical_layer: int):
    """deepseek_rope_for_layer (E/compute.rs:2575-2586): (theta, yarn or None)."""
    lib = load_library()
    theta, y, has = ctypes.c_float(), WhYarn(), ctypes.c_int()
    _check(lib.wh_deepseek_rope_for_layer(physical_layer, ctypes.byref(theta), ctypes.byref(y), ctypes.byref(has)),
           "deepseek_rope_for_layer")
    return theta.value, ((y.factor, y.beta_fast, y.beta_slow, y.original_seq_len) if has.value else None)
