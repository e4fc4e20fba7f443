"""Loader for libaxk.so, the C-ABI of the gfx950 kernels (declared in include/axk.h).

The library is built in-tree by ``make -C ax-dsl-kernels_amd/csrc``. There is no CPU fallback: if the
library is missing every operator raises, so a test or benchmark can never pass on a substitute path.
"""
from __future__ import annotations

import ctypes
import os
import re

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libaxk.so")
HEADER_PATH = os.path.join(_HERE, "..", "..", "include", "axk.h")

# status codes and dtype codes, kept in step with include/axk.h (tests check the header text)
AXK_OK = 0
STATUS_NAMES = {
    1: "AXK_E_NULL",
    2: "AXK_E_SHAPE",
    3: "AXK_E_ALIGN",
    4: "AXK_E_DTYPE",
    5: "AXK_E_ALIAS",
    6: "AXK_E_WORKSPACE",
    7: "AXK_E_LAUNCH",
    8: "AXK_E_ROLE",
    9: "AXK_E_BUFFER",
    10: "AXK_E_SCRATCH",
}
DT_U8, DT_F32, DT_I32, DT_BF16, DT_F16, DT_FP8E4M3, DT_FP8E5M2, DT_FP4 = 1, 3, 6, 9, 10, 11, 12, 15

TORCH_TO_DT = {
    torch.uint8: DT_U8,
    torch.float32: DT_F32,
    torch.int32: DT_I32,
    torch.bfloat16: DT_BF16,
    torch.float16: DT_F16,
    torch.float8_e4m3fn: DT_FP8E4M3,
    torch.float8_e5m2: DT_FP8E5M2,
}


class AxkError(RuntimeError):
    def __init__(self, fn: str, status: int, text: str):
        super().__init__(f"{fn} failed: {STATUS_NAMES.get(status, status)} ({text})")
        self.status = status


_lib = None

_vp, _i64, _i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int

# argument signatures of every exported entry point (return type is int unless listed in _RESTYPES)
SIGNATURES: dict[str, list] = {
    "axk_version": [],
    "axk_status_string": [_i32],
    "axk_io_table": [ctypes.c_char_p, _vp, _i32, _vp, _i32, _vp],
    "axk_mxfp4_dequant": [_vp, _vp, _vp, _i64, _i64, _vp],
    "axk_mxfp4_gemm": [_vp, _i64, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _vp],
    "axk_fp8_gemm": [_vp, _i64, _vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _vp],
    "axk_mxfp8_gemm": [_vp, _i64, _vp, _vp, _i32, _vp, _vp, _i32, _i64, _i64, _i64, _vp],
    "axk_nvfp4_gemm": [_vp, _i64, _vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _vp],
    "axk_bf16_gemm": [_vp, _i64, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _vp],
    "axk_int8_gemm": [_vp, _i64, _vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _vp],
    "axk_int4_gemm": [_vp, _i64, _vp, _vp, _i64, _vp, _vp, _i32, _i64, _i64, _i64, _vp],
    "axk_paged_decode_workspace_size": [_i64, _i64, _i64, _i64],
    "axk_paged_decode_plan": [_vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp, ctypes.c_size_t, _vp],
    "axk_paged_decode_split": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, ctypes.c_float,
                               _vp, ctypes.c_size_t, _vp],
    "axk_paged_decode_merge": [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp, ctypes.c_size_t, _vp],
    "axk_paged_decode_run": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, ctypes.c_float, _vp,
                             ctypes.c_size_t, _vp],
    "axk_paged_decode": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, ctypes.c_float, _vp,
                         ctypes.c_size_t, _vp],
    "axk_paged_attention_decode": [_vp] * 9 + [_i64] * 6 + [ctypes.c_float, _vp, _vp, ctypes.c_size_t, _vp],
    "axk_paged_decode_noalloc": [_vp] * 6 + [_i64] * 6 + [ctypes.c_float, _vp],
    "axk_paged_kv_write": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp, _vp],
    "axk_paged_decode_fp8": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, ctypes.c_float,
                             ctypes.c_float, _vp, ctypes.c_size_t, _vp],
    "axk_paged_kv_write_fp8": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, ctypes.c_float, _vp, _vp],
    "axk_paged_kv_write_i8": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp, _vp],
    "axk_paged_decode_i8": [_vp] * 7 + [_i64] * 6 + [ctypes.c_float, _vp, ctypes.c_size_t, _vp],
    "axk_paged_prefill": [_vp] * 7 + [_i64] * 7 + [ctypes.c_float, _vp, _vp],
    "axk_gdn_recurrent": [_vp] * 10 + [_i64] * 6 + [_vp],
    "axk_gdn_chunk_workspace_size": [_i64] * 7,
    "axk_gdn_chunk_prefill": [_vp] * 10 + [_i64] * 7 + [_vp, ctypes.c_size_t, _vp],
    "axk_moe_workspace_size": [_i64] * 6,
    "axk_moe_route": [_vp, _vp, _vp, _i64, _i64, _i64, _i32, _vp],
    "axk_moe_experts": [_vp] * 16 + [_i64] * 6 + [_vp, ctypes.c_size_t, _vp],
    "axk_moe_decode": [_vp] * 18 + [_i64] * 6 + [_i32, _vp, ctypes.c_size_t, _vp],
    "axk_rmsnorm": [_vp, _i64, _vp, _vp, _i64, _i64, _i64, ctypes.c_float, _vp],
    "axk_add_rmsnorm": [_vp] * 5 + [_i64, _i64, ctypes.c_float, _vp],
    "axk_gated_rmsnorm_silu": [_vp] * 4 + [_i64, _i64, ctypes.c_float, _vp],
    "axk_causal_conv1d_silu": [_vp] * 5 + [_i64] * 4 + [_vp],
    "axk_qk_norm_rope": [_vp, _i64, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, ctypes.c_float, _vp],
    "axk_sigmoid_mul": [_vp, _vp, _i64, _vp, _i64, _i64, _vp],
    "axk_silu_mul": [_vp, _vp, _vp, _i64, _i64, _vp],
    "axk_add": [_vp, _vp, _vp, _i64, _i64, _vp],
    "axk_gdn_layer_workspace_size": [_i64] * 6,
    "axk_gdn_layer_decode": [_vp] * 28 + [_i64] * 7 + [ctypes.c_float, _i32, _i32, _i32, _vp, ctypes.c_size_t,
                             _vp],
    "axk_attn_layer_workspace_size": [_i64] * 6,
    "axk_gdn_layer_verify_workspace_size": [_i64] * 7,
    "axk_attn_layer_verify_workspace_size": [_i64] * 7,
    "axk_gdn_layer_verify": [_vp] * 30 + [_i64] * 8 + [ctypes.c_float, _i32, _i32, _i32, _vp, ctypes.c_size_t,
                             _vp],
    "axk_attn_layer_verify": [_vp] * 27 + [_i64] * 10 + [ctypes.c_float, ctypes.c_float, _i32, _i32, _vp,
                              ctypes.c_size_t, _vp],
    "axk_attn_layer_decode": [_vp] * 27 + [_i64] * 9 + [ctypes.c_float, ctypes.c_float, _i32, _i32, _vp,
                              ctypes.c_size_t, _vp],
    "axk_gdn_layer_moe_workspace_size": [_i64] * 6 + [_vp],
    "axk_attn_layer_moe_workspace_size": [_i64] * 6 + [_vp],
    "axk_gdn_layer_decode_moe": [_vp] * 29 + [_i64] * 7 + [ctypes.c_float, _i32, _i32, _i32, _vp,
                                 ctypes.c_size_t, _vp],
    "axk_attn_layer_decode_moe": [_vp] * 28 + [_i64] * 9 + [ctypes.c_float, ctypes.c_float, _i32, _i32, _vp,
                                  ctypes.c_size_t, _vp],
    "axk_gdn_layer_prefill_workspace_size": [_i64] * 7,
    "axk_attn_layer_prefill_workspace_size": [_i64] * 7,
    "axk_gdn_layer_prefill": [_vp] * 28 + [_i64] * 8 + [ctypes.c_float, _i32, _i32, _i32, _vp, ctypes.c_size_t,
                              _vp],
    "axk_attn_layer_prefill": [_vp] * 27 + [_i64] * 10 + [ctypes.c_float, ctypes.c_float, _i32, _i32, _vp,
                               ctypes.c_size_t, _vp],
    "axk_gdn_layer_prefill_moe_workspace_size": [_i64] * 7 + [_vp],
    "axk_attn_layer_prefill_moe_workspace_size": [_i64] * 7 + [_vp],
    "axk_gdn_layer_prefill_moe": [_vp] * 29 + [_i64] * 8 + [ctypes.c_float, _i32, _i32, _i32, _vp,
                                  ctypes.c_size_t, _vp],
    "axk_attn_layer_prefill_moe": [_vp] * 28 + [_i64] * 10 + [ctypes.c_float, ctypes.c_float, _i32, _i32, _vp,
                                   ctypes.c_size_t, _vp],
}
_RESTYPES = {
    "axk_version": ctypes.c_char_p,
    "axk_status_string": ctypes.c_char_p,
    "axk_paged_decode_workspace_size": ctypes.c_size_t,
    "axk_moe_workspace_size": ctypes.c_size_t,
    "axk_gdn_chunk_workspace_size": ctypes.c_size_t,
    "axk_gdn_layer_workspace_size": ctypes.c_size_t,
    "axk_attn_layer_workspace_size": ctypes.c_size_t,
    "axk_gdn_layer_verify_workspace_size": ctypes.c_size_t,
    "axk_attn_layer_verify_workspace_size": ctypes.c_size_t,
    "axk_gdn_layer_moe_workspace_size": ctypes.c_size_t,
    "axk_attn_layer_moe_workspace_size": ctypes.c_size_t,
    "axk_gdn_layer_prefill_workspace_size": ctypes.c_size_t,
    "axk_attn_layer_prefill_workspace_size": ctypes.c_size_t,
    "axk_gdn_layer_prefill_moe_workspace_size": ctypes.c_size_t,
    "axk_attn_layer_prefill_moe_workspace_size": ctypes.c_size_t,
}


class Nvfp4Scales(ctypes.Structure):
    """axk_nvfp4_scales of include/axk.h: an NVFP4 weight's E4M3 block scales and fp32 scale2 (device pointers)."""

    _fields_ = [("block_scales", ctypes.c_void_p), ("scale2", ctypes.c_void_p)]


class MoeBlock(ctypes.Structure):
    """axk_moe_block of include/axk.h: the MoE block of the MoE decode layers (device pointers and sizes)."""

    _fields_ = [("w_router", ctypes.c_void_p), ("w_shg", ctypes.c_void_p), ("e_gw", ctypes.c_void_p),
                ("e_gs", ctypes.c_void_p), ("e_dw", ctypes.c_void_p), ("e_ds", ctypes.c_void_p),
                ("num_experts", ctypes.c_int64), ("top_k", ctypes.c_int64), ("expert_inter", ctypes.c_int64),
                ("norm_topk_prob", ctypes.c_int32), ("reserved", ctypes.c_int32), ("logits", ctypes.c_void_p),
                ("topk_ids", ctypes.c_void_p), ("topk_weights", ctypes.c_void_p)]


def header_symbols(path: str = HEADER_PATH) -> list[str]:
    """Names of the functions declared in include/axk.h."""
    with open(path) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(axk_[a-z0-9_]+)\s*\(", text)))


def load() -> ctypes.CDLL:
    """Load libaxk.so once; raise if it is absent (no fallback path exists)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is not built; run `make -C ax-dsl-kernels_amd/csrc` (or __graft_entry__.build())"
        )
    lib = ctypes.CDLL(LIB_PATH)
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _RESTYPES.get(name, ctypes.c_int)
    _lib = lib
    return lib


def call(name: str, *args) -> None:
    """Call an entry point and raise AxkError on a nonzero status."""
    lib = load()
    status = getattr(lib, name)(*args)
    if status != AXK_OK:
        raise AxkError(name, status, lib.axk_status_string(status).decode())


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    """The current torch stream of t's device as a hipStream_t value."""
    return torch.cuda.current_stream(t.device).cuda_stream


def require_device(*tensors: torch.Tensor | None) -> None:
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise ValueError(f"axk operators take device tensors; got a tensor on {t.device}")
