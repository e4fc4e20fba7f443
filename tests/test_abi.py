"""The C-ABI library loads, exports every symbol include/axk.h declares, and rejects contract
violations before touching the GPU (CPU only: no compute call is made)."""
import ctypes
import os
import re

import pytest
import torch

import axk
from axk import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_header_symbols_exported_and_bound():
    lib = _lib.load()
    declared = _lib.header_symbols()
    assert declared, "no declarations parsed from include/axk.h"
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in include/axk.h but not exported by libaxk.so"
    # every declared function has a ctypes signature and vice versa
    assert sorted(_lib.SIGNATURES) == declared


def test_header_status_and_dtype_codes_match_python():
    text = open(_lib.HEADER_PATH).read()
    codes = {m[0]: int(m[1]) for m in re.findall(r"#define (AXK_E_[A-Z]+) (\d+)", text)}
    assert {v: k for k, v in codes.items()} == _lib.STATUS_NAMES
    dts = {m[0]: int(m[1]) for m in re.findall(r"#define AXK_DT_([A-Z0-9]+) (\d+)", text)}
    # AX dtype codes of tools/manifest/onnx_io.py:18-29
    assert dts == {"U8": 1, "F32": 3, "I32": 6, "BF16": 9, "F16": 10, "FP8E4M3": 11, "FP8E5M2": 12, "FP4": 15}


def test_version_and_status_strings():
    lib = _lib.load()
    assert b"gfx950" in lib.axk_version()
    for code in list(_lib.STATUS_NAMES) + [0]:
        assert lib.axk_status_string(code)


def test_contract_violations_return_before_launch():
    lib = _lib.load()
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: every check below fails first
    # NULL codes
    assert lib.axk_mxfp4_dequant(None, fake, fake, 4, 64, None) == 1
    # k not a multiple of 32
    assert lib.axk_mxfp4_dequant(fake, fake, fake, 4, 48, None) == 2
    # misaligned activation
    assert lib.axk_mxfp4_gemm(ctypes.c_void_p(0x1002), 64, fake, fake, None, fake, 9, 1, 16, 64, None) == 3
    # bad output dtype
    assert lib.axk_mxfp4_gemm(fake, 64, fake, fake, None, fake, 15, 1, 16, 64, None) == 4
    # output overlapping the activation
    assert lib.axk_mxfp4_gemm(fake, 64, ctypes.c_void_p(0x9000), fake, None, fake, 9, 1, 16, 64, None) == 5
    # fp8 without its channel scales
    assert lib.axk_fp8_gemm(fake, 64, fake, None, None, None, fake, 9, 1, 16, 64, None) == 1
    # int8: k not a multiple of 16; misaligned leading dimension; bad dtype; missing scale_a
    assert lib.axk_int8_gemm(fake, 64, fake, fake, fake, None, fake, 9, 1, 16, 40, None) == 2
    assert lib.axk_int8_gemm(fake, 72, fake, fake, fake, None, fake, 9, 1, 16, 64, None) == 3
    assert lib.axk_int8_gemm(fake, 64, fake, fake, fake, None, fake, 6, 1, 16, 64, None) == 4
    assert lib.axk_int8_gemm(fake, 64, fake, None, fake, None, fake, 9, 1, 16, 64, None) == 1
    # int4: a group that is not a multiple of 32 or does not divide k; output over the weights
    assert lib.axk_int4_gemm(fake, 64, fake, fake, 16, None, fake, 9, 1, 16, 64, None) == 2
    assert lib.axk_int4_gemm(fake, 96, fake, fake, 64, None, fake, 9, 1, 16, 96, None) == 2
    assert lib.axk_int4_gemm(fake, 64, ctypes.c_void_p(0x9000), fake, 32, None, ctypes.c_void_p(0x9100), 9, 1, 16, 64,
                             None) == 5


def test_python_layer_raises_value_error_on_contract():
    import torch

    a = torch.zeros(2, 64, dtype=torch.bfloat16)
    w = torch.zeros(16, 16, dtype=torch.uint8)
    s = torch.zeros(16, 2, dtype=torch.uint8)
    with pytest.raises(ValueError):
        axk.mxfp4_gemm(a, w, s)  # k/2 mismatch
    with pytest.raises(ValueError):
        axk.mxfp4_gemm(a.float(), torch.zeros(16, 32, dtype=torch.uint8), s)  # fp32 activation
    with pytest.raises(ValueError):
        axk.mxfp4_gemm(a, torch.zeros(16, 32, dtype=torch.uint8), torch.zeros(16, 3, dtype=torch.uint8))
    i8 = torch.zeros(2, 64, dtype=torch.int8)
    with pytest.raises(ValueError):
        axk.int8_gemm(i8, torch.zeros(16, 48, dtype=torch.int8), torch.ones(1), torch.ones(1))  # k mismatch
    with pytest.raises(ValueError):
        axk.int8_gemm(i8, torch.zeros(16, 64, dtype=torch.int8), torch.ones(3), torch.ones(1))  # scale_a size
    with pytest.raises(ValueError):
        axk.int8_gemm(a, torch.zeros(16, 64, dtype=torch.int8), torch.ones(1), torch.ones(1))  # bf16 activation
    with pytest.raises(ValueError):
        axk.int4_gemm(a, torch.zeros(16, 64, dtype=torch.int8), torch.ones(16, 4))  # group 16
    with pytest.raises(ValueError):
        axk.int4_gemm(a, torch.zeros(16, 64, dtype=torch.int8), torch.ones(15, 2))  # scale rows
    with pytest.raises(ValueError):
        axk.int4_gemm(a, torch.zeros(16, 64, dtype=torch.uint8), torch.ones(16, 2))  # unsigned storage


def test_moe_workspace_size_limits():
    lib = _lib.load()
    assert lib.axk_moe_workspace_size(256, 64, 8, 2, 32, 32) > 0
    # above 256 tokens the prefill path needs inter and shared_inter % 64 == 0 (32 passes only the decode path)
    assert lib.axk_moe_workspace_size(257, 64, 8, 2, 32, 32) == 0
    assert lib.axk_moe_workspace_size(257, 64, 8, 2, 64, 64) > 0
    assert lib.axk_moe_workspace_size(4, 64, 1025, 2, 32, 32) == 0  # experts <= 1024
    assert lib.axk_moe_workspace_size(4, 64, 8, 33, 32, 32) == 0   # top_k <= 32
    assert lib.axk_moe_workspace_size(4, 96, 8, 2, 32, 32) == 0     # hidden % 64


@pytest.mark.skipif(torch.cuda.is_available(), reason="drives entry points with host pointers: only on a GPU-less host")
def test_prefill_layer_workspace_limits():
    lib = _lib.load()
    assert lib.axk_gdn_layer_prefill_workspace_size(2, 100, 256, 2, 4, 128, 512) > 0
    assert lib.axk_gdn_layer_prefill_workspace_size(1, 1 << 16, 256, 2, 4, 128, 512) > 0
    assert lib.axk_gdn_layer_prefill_workspace_size(1, (1 << 16) + 1, 256, 2, 4, 128, 512) == 0  # tokens <= 65536
    assert lib.axk_gdn_layer_prefill_workspace_size(3, 1 << 16, 256, 2, 4, 128, 512) == 0  # rows <= 131072
    assert lib.axk_gdn_layer_prefill_workspace_size(2, 100, 256, 2, 4, 64, 512) == 0  # head_dim 128
    assert lib.axk_gdn_layer_prefill_workspace_size(2, 100, 256, 2, 3, 128, 512) == 0  # NV % NK
    assert lib.axk_attn_layer_prefill_workspace_size(2, 100, 256, 4, 2, 256, 512) > 0
    assert lib.axk_attn_layer_prefill_workspace_size(2, 100, 256, 4, 2, 96, 512) == 0  # head_dim 64 / 128 / 256
    assert lib.axk_attn_layer_prefill_workspace_size(2, 100, 256, 5, 2, 256, 512) == 0  # HQ % HKV
    # the attention prefill's workspace is the verify layer's at the same rows
    assert (lib.axk_attn_layer_prefill_workspace_size(4, 16, 256, 4, 2, 256, 512) ==
            lib.axk_attn_layer_verify_workspace_size(4, 16, 256, 4, 2, 256, 512))


def test_entry_points_reach_the_launch_on_a_gpu_less_host():
    """Every host-side step of an entry point (argument checks, the layers' validate-only pass, workspace carving)
    runs on a host without a GPU and ends at the launch with AXK_E_LAUNCH, never a crash."""
    import ctypes

    lib = _lib.load()
    buf = ctypes.create_string_buffer(1 << 24)
    base = (ctypes.addressof(buf) + 4095) // 4096 * 4096
    p = [base + 65536 * i for i in range(200)]
    launch = 7  # AXK_E_LAUNCH
    assert lib.axk_rmsnorm(p[0], 64, p[1], p[2], 64, 1, 64, 1e-6, None) == launch
    assert lib.axk_int8_gemm(p[0], 64, p[1], p[2], p[3], None, p[4], 9, 3, 70, 64, None) == launch
    assert lib.axk_int4_gemm(p[0], 64, p[1], p[2], 32, p[3], p[4], 3, 3, 70, 64, None) == launch
    ws = lib.axk_paged_decode_workspace_size(2, 8, 2, 128)
    assert lib.axk_paged_decode(p[0], p[1], p[2], p[3], p[4], p[5], 2, 8, 2, 128, 32, 4, 0.1, p[100], ws,
                                None) == launch
    assert lib.axk_paged_attention_decode(p[0], p[6], p[7], p[1], p[2], p[3], p[4], p[8], p[5], 2, 8, 2, 128, 32, 4,
                                          0.1, None, p[100], ws, None) == launch
    gws = lib.axk_gdn_layer_workspace_size(1, 256, 1, 2, 128, 256)
    args = [p[10 + i] for i in range(28)]
    assert lib.axk_gdn_layer_decode(*args, 1, 256, 1, 2, 128, 4, 256, 1e-6, 0, 2, 1, p[150], gws, None) == launch
    # a late contract error (misaligned w_out, argument 15) is found by the validate pass before any launch
    bad = list(args)
    bad[14] += 1
    assert lib.axk_gdn_layer_decode(*bad, 1, 256, 1, 2, 128, 4, 256, 1e-6, 0, 2, 1, p[150], gws, None) == 3
    # an unknown weight format is refused before anything else
    assert lib.axk_gdn_layer_decode(*args, 1, 256, 1, 2, 128, 4, 256, 1e-6, 7, 2, 1, p[150], gws, None) == 4
    # an unknown value-head order is refused before any launch
    assert lib.axk_gdn_layer_decode(*args, 1, 256, 1, 2, 128, 4, 256, 1e-6, 0, 2, 2, p[150], gws, None) == 2
    # the prefill layer: 20 tokens of one sequence; a late misaligned w_out found before the conv / state launches
    pws = lib.axk_gdn_layer_prefill_workspace_size(1, 20, 256, 1, 2, 128, 256)
    assert 0 < pws < 65536 * 48
    assert lib.axk_gdn_layer_prefill(*args, 1, 20, 256, 1, 2, 128, 4, 256, 1e-6, 0, 2, 1, p[150], pws, None) == launch
    assert lib.axk_gdn_layer_prefill(*bad, 1, 20, 256, 1, 2, 128, 4, 256, 1e-6, 0, 2, 1, p[150], pws, None) == 3
    assert lib.axk_gdn_layer_prefill(*args, 1, 20, 256, 1, 2, 128, 4, 256, 1e-6, 0, 2, 1, p[150], pws - 1, None) == 6


def test_int8_kv_contract_violations_return_before_launch():
    """The INT8 cache entries reject bad shapes, NULL scales and misaligned scales before any launch; the Python
    wrappers raise ValueError on mismatched scale tensors before touching a device."""
    lib = _lib.load()
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: every check below fails first
    args = lambda scales, hkv, d: (fake, fake, scales, fake, fake, fake, fake, 2, 2 * hkv, hkv, d, 64, 8, 0.0625,
                                   fake, 1 << 20, None)
    assert lib.axk_paged_decode_i8(*args(None, 2, 128)) == 1               # NULL kv_scales
    assert lib.axk_paged_decode_i8(*args(fake, 2, 64)) == 2                # head_dim 64
    assert lib.axk_paged_decode_i8(*args(fake, 17, 128)) == 2              # more than 16 KV heads
    assert lib.axk_paged_decode_i8(*args(ctypes.c_void_p(0x1002), 2, 128)) == 3  # scales not 4-byte aligned
    assert lib.axk_paged_kv_write_i8(fake, fake, fake, None, fake, 2, 2, 128, 64, 8, None, None) == 1
    assert lib.axk_paged_kv_write_i8(fake, fake, fake, fake, fake, 2, 2, 64, 64, 8, None, None) == 2
    assert lib.axk_paged_kv_write_i8(ctypes.c_void_p(0x1008), fake, fake, fake, fake, 2, 2, 128, 64, 8, None,
                                     None) == 3
    q = torch.zeros(2, 4, 128, dtype=torch.bfloat16)
    cache = torch.zeros(8, 2, 64, 2, 128, dtype=torch.int8)
    ip, idx, last = torch.tensor([0, 1, 2], dtype=torch.int32), torch.zeros(2, dtype=torch.int32), \
        torch.ones(2, dtype=torch.int32)
    with pytest.raises(ValueError, match="kv_scales"):
        axk.paged_decode_i8(q, cache, torch.zeros(8, 2, 64, 2, dtype=torch.float32), ip, idx, last)
    with pytest.raises(ValueError, match="kv_scales"):
        axk.store_paged_kv_i8(torch.zeros(2, 2, 128, dtype=torch.bfloat16), torch.zeros(2, 2, 128, dtype=torch.bfloat16),
                              cache, torch.zeros(8, 2, 64, 3, dtype=torch.bfloat16), torch.zeros(2, 2, dtype=torch.int32))
