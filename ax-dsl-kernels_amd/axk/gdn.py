"""Gated DeltaNet (GDN) on gfx950: the recurrent / decode step and the chunked prefill.

Mirrors the GDN primitives of sgl_kernel_axera.attention.gdn (gdn_gate, l2norm_lastdim, gdn_recurrent_step:
models/qwen35_35b_a3b/sgl/python/sgl_kernel_axera/attention/gdn.py:919-989; gdn_stable_chunk and its solve:
gdn.py:992-1212) with the argument order of the reference's golden gdn_reference(q, k, v, a, b, a_log, dt_bias,
state_in) (models/qwen35_35b_a3b/sgl/tests/test_gdn_attn.py:259).
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _lib


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _check_inputs(q, k, v, a, b, a_log, dt_bias, state_in, state_out, output):
    _check(q.dim() == 4 and k.shape == q.shape, "q and k must be [B, T, NK, 128]")
    bsz, t, nk, dk = q.shape
    _check(v.dim() == 4 and v.shape[:2] == (bsz, t), "v must be [B, T, NV, 128]")
    nv, dv = v.shape[2], v.shape[3]
    _check(dk == 128 and dv == 128, "head dims must be 128")
    _check(nv % nk == 0, "num_v_heads must be a multiple of num_k_heads")
    for name, x in (("q", q), ("k", k), ("v", v), ("a", a), ("b", b)):
        _check(x.dtype == torch.bfloat16 and x.is_contiguous(), f"{name} must be contiguous bf16")
    _check(a.shape == (bsz, t, nv) and b.shape == (bsz, t, nv), "a and b must be [B, T, NV]")
    a_log = a_log.reshape(-1).to(torch.float32).contiguous()
    dt_bias = dt_bias.reshape(-1).to(torch.float32).contiguous()
    _check(a_log.numel() == nv and dt_bias.numel() == nv, "a_log and dt_bias must have NV elements")
    _check(state_in.shape == (bsz, nv, dk, dv) and state_in.dtype == torch.float32 and state_in.is_contiguous(),
           "state_in must be contiguous f32 [B, NV, 128, 128]")
    if state_out is None:
        state_out = torch.empty_like(state_in)
    _check(state_out.shape == state_in.shape and state_out.dtype == torch.float32 and state_out.is_contiguous(),
           "bad state_out")
    if output is None:
        output = torch.empty_like(v)
    _check(output.shape == v.shape and output.dtype == torch.bfloat16 and output.is_contiguous(), "bad output")
    _lib.require_device(q, k, v, a, b, a_log, dt_bias, state_in, state_out, output)
    return (bsz, t, nk, nv, dk, dv), a_log, dt_bias, state_out, output


def gdn_recurrent(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    a_log: torch.Tensor,
    dt_bias: torch.Tensor,
    state_in: torch.Tensor,
    state_out: Optional[torch.Tensor] = None,
    output: Optional[torch.Tensor] = None,
):
    """q, k [B, T, NK, 128] bf16; v [B, T, NV, 128] bf16; a, b [B, T, NV] bf16; a_log, dt_bias [NV] f32;
    state_in [B, NV, 128, 128] f32. Returns (output bf16 [B, T, NV, 128], state_out). Pass
    state_out=state_in to update the state in place."""
    dims, a_log, dt_bias, state_out, output = _check_inputs(q, k, v, a, b, a_log, dt_bias, state_in, state_out,
                                                            output)
    _lib.call("axk_gdn_recurrent", q.data_ptr(), k.data_ptr(), v.data_ptr(), a.data_ptr(), b.data_ptr(),
              a_log.data_ptr(), dt_bias.data_ptr(), state_in.data_ptr(), state_out.data_ptr(), output.data_ptr(),
              *dims, _lib.stream_of(q))
    return output, state_out


def gdn_chunk_workspace(batch: int, tokens: int, num_k_heads: int, num_v_heads: int, device,
                        chunk_size: int = 64) -> torch.Tensor:
    n = _lib.load().axk_gdn_chunk_workspace_size(batch, tokens, num_k_heads, num_v_heads, 128, 128, chunk_size)
    _check(n > 0, "unsupported GDN chunk shape")
    return torch.empty(n, dtype=torch.uint8, device=device)


def gdn_chunk_prefill(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    a_log: torch.Tensor,
    dt_bias: torch.Tensor,
    state_in: torch.Tensor,
    state_out: Optional[torch.Tensor] = None,
    output: Optional[torch.Tensor] = None,
    chunk_size: int = 64,
    workspace: Optional[torch.Tensor] = None,
):
    """The same recurrence as gdn_recurrent over all T tokens, in the chunked form of gdn_stable_chunk
    (chunk_size 64). Returns (output bf16 [B, T, NV, 128], state_out)."""
    dims, a_log, dt_bias, state_out, output = _check_inputs(q, k, v, a, b, a_log, dt_bias, state_in, state_out,
                                                            output)
    bsz, t, nk, nv, dk, dv = dims
    if workspace is None:
        workspace = gdn_chunk_workspace(bsz, t, nk, nv, q.device, chunk_size)
    _check(workspace.dtype == torch.uint8 and workspace.is_contiguous(), "workspace must be contiguous uint8")
    _lib.require_device(workspace)
    _lib.call("axk_gdn_chunk_prefill", q.data_ptr(), k.data_ptr(), v.data_ptr(), a.data_ptr(), b.data_ptr(),
              a_log.data_ptr(), dt_bias.data_ptr(), state_in.data_ptr(), state_out.data_ptr(), output.data_ptr(),
              *dims, chunk_size, workspace.data_ptr(), workspace.numel(), _lib.stream_of(q))
    return output, state_out
