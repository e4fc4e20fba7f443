"""Per-layer glue of the Qwen3.5 hybrid decode layer over libaxk.so (include/axk.h).

RMSNorm (plain, fused with the residual add, gated by silu(z)), the stateful causal conv1d + SiLU, q / k norm
with partial NeoX RoPE, and the elementwise gates of models/qwen35_35b_a3b/src/70b0fbc/q35_step.py. Inputs are
bf16 device tensors (weights of the norms fp32, as the reference passes them); outputs are new bf16 tensors
unless `out` is given. Contract violations raise ValueError.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _lib


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _bf16(t: torch.Tensor, name: str) -> None:
    _check(t.dtype == torch.bfloat16, f"{name} must be bfloat16, got {t.dtype}")


def _out(out: Optional[torch.Tensor], shape, like: torch.Tensor) -> torch.Tensor:
    if out is None:
        return torch.empty(shape, dtype=torch.bfloat16, device=like.device)
    _check(out.dtype == torch.bfloat16 and tuple(out.shape) == tuple(shape) and out.is_contiguous(),
           f"out must be contiguous bfloat16 {tuple(shape)}")
    return out


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float = 1e-6, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """x [..., n] bf16 (rows may be strided, last dim contiguous); w f32 [n] (1 + weight for layer / q / k norms)."""
    _bf16(x, "x")
    n = x.shape[-1]
    _check(w.dtype == torch.float32 and w.numel() == n and w.is_contiguous(), "w must be contiguous float32 [n]")
    _check(x.stride(-1) == 1, "x rows must be contiguous")
    x2 = x.reshape(-1, n) if x.is_contiguous() else x
    _check(x2.dim() == 2, "a strided x must be 2-D [rows, n]")
    rows = x2.shape[0]
    o = _out(out, x.shape, x).reshape(rows, n)
    _lib.require_device(x2, w, o)
    _lib.call("axk_rmsnorm", x2.data_ptr(), x2.stride(0), w.data_ptr(), o.data_ptr(), n, rows, n, eps,
              _lib.stream_of(x))
    return o.reshape(x.shape)


def add_rmsnorm(x: torch.Tensor, y: torch.Tensor, w: torch.Tensor, eps: float = 1e-6,
                sum_out: Optional[torch.Tensor] = None, norm_out: Optional[torch.Tensor] = None):
    """(bf16(x + y), rmsnorm(bf16(x + y), w)) for contiguous x, y [..., n]."""
    _bf16(x, "x")
    _bf16(y, "y")
    _check(x.shape == y.shape and x.is_contiguous() and y.is_contiguous(), "x and y must be contiguous, same shape")
    n = x.shape[-1]
    _check(w.dtype == torch.float32 and w.numel() == n, "w must be float32 [n]")
    s = _out(sum_out, x.shape, x)
    o = _out(norm_out, x.shape, x)
    _lib.require_device(x, y, w, s, o)
    _lib.call("axk_add_rmsnorm", x.data_ptr(), y.data_ptr(), w.data_ptr(), s.data_ptr(), o.data_ptr(),
              x.numel() // n, n, eps, _lib.stream_of(x))
    return s, o


def gated_rmsnorm_silu(x: torch.Tensor, w: torch.Tensor, z: torch.Tensor, eps: float = 1e-6,
                       out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """bf16(bf16(rmsnorm(x) * w) * silu(z)) per row of the last dim (the GDN output norm, w = norm_w f32)."""
    _bf16(x, "x")
    _bf16(z, "z")
    _check(x.shape == z.shape and x.is_contiguous() and z.is_contiguous(), "x and z must be contiguous, same shape")
    n = x.shape[-1]
    _check(w.dtype == torch.float32 and w.numel() == n, "w must be float32 [n]")
    o = _out(out, x.shape, x)
    _lib.require_device(x, w, z, o)
    _lib.call("axk_gated_rmsnorm_silu", x.data_ptr(), w.data_ptr(), z.data_ptr(), o.data_ptr(), x.numel() // n, n,
              eps, _lib.stream_of(x))
    return o


def causal_conv1d_silu(x: torch.Tensor, w: torch.Tensor, state_in: torch.Tensor,
                       state_out: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None):
    """x [B, T, C] bf16; w [C, K] bf16 (column 0 multiplies the current token); state [B, K-1, C] bf16.
    Returns (out [B, T, C], state_out); state_out may be state_in (in place)."""
    _bf16(x, "x")
    _bf16(w, "w")
    _check(x.dim() == 3 and x.is_contiguous() and w.dim() == 2 and w.shape[0] == x.shape[2] and w.is_contiguous(),
           "x must be contiguous [B, T, C] and w [C, K]")
    b, t, c = x.shape
    k = w.shape[1]
    _check(tuple(state_in.shape) == (b, k - 1, c) and state_in.dtype == torch.bfloat16 and state_in.is_contiguous(),
           f"state_in must be contiguous bfloat16 [{b}, {k - 1}, {c}]")
    so = torch.empty_like(state_in) if state_out is None else state_out
    _check(so.shape == state_in.shape and so.dtype == torch.bfloat16 and so.is_contiguous(), "bad state_out")
    o = _out(out, x.shape, x)
    _lib.require_device(x, w, state_in, so, o)
    _lib.call("axk_causal_conv1d_silu", x.data_ptr(), w.data_ptr(), state_in.data_ptr(), so.data_ptr(), o.data_ptr(),
              b, t, c, k, _lib.stream_of(x))
    return o, so


def qk_norm_rope(x: torch.Tensor, w: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, rot: int,
                 eps: float = 1e-6, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """x [B, heads, D] bf16 (the head rows may be strided: a [B, heads, 2D] q projection's first halves);
    w f32 [D] (1 + weight); cos, sin bf16 [B, rot/2]. Returns contiguous [B, heads, D]."""
    _bf16(x, "x")
    _check(x.dim() == 3 and x.stride(-1) == 1 and x.stride(0) == x.shape[1] * x.stride(1),
           "x must be [B, heads, D] with unit-stride rows evenly spaced")
    b, h, d = x.shape
    _check(w.dtype == torch.float32 and w.numel() == d, "w must be float32 [D]")
    if rot:
        _check(cos.dtype == torch.bfloat16 and sin.dtype == torch.bfloat16 and tuple(cos.shape) == (b, rot // 2)
               and tuple(sin.shape) == (b, rot // 2) and cos.is_contiguous() and sin.is_contiguous(),
               f"cos and sin must be contiguous bfloat16 [{b}, {rot // 2}]")
    o = _out(out, (b, h, d), x)
    _lib.require_device(x, w, o)
    _lib.call("axk_qk_norm_rope", x.data_ptr(), x.stride(1), w.data_ptr(), _lib.ptr(cos if rot else None),
              _lib.ptr(sin if rot else None), o.data_ptr(), b, h, d, rot, eps, _lib.stream_of(x))
    return o


def sigmoid_mul(x: torch.Tensor, gate: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """bf16(x * sigmoid(gate)): x contiguous [rows, n] (or [..., n]); gate rows may be strided."""
    _bf16(x, "x")
    _bf16(gate, "gate")
    n = x.shape[-1]
    rows = x.numel() // n
    _check(x.is_contiguous() and gate.shape == x.shape and gate.stride(-1) == 1,
           "x must be contiguous and gate of x's shape with unit-stride rows")
    # the gate's rows: its leading dims must collapse into one evenly spaced row index
    ldg = gate.stride(-2) if gate.dim() >= 2 else n
    for i in range(gate.dim() - 2):
        _check(gate.stride(i) == gate.shape[i + 1] * gate.stride(i + 1), "gate rows must be evenly spaced")
    o = _out(out, x.shape, x)
    _lib.require_device(x, gate, o)
    _lib.call("axk_sigmoid_mul", x.data_ptr(), gate.data_ptr(), ldg, o.data_ptr(), rows, n, _lib.stream_of(x))
    return o


def silu_mul(g: torch.Tensor, u: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """bf16(silu(g) * u) for contiguous g, u of one shape."""
    _bf16(g, "g")
    _bf16(u, "u")
    _check(g.shape == u.shape and g.is_contiguous() and u.is_contiguous(), "g and u must be contiguous, same shape")
    n = g.shape[-1]
    o = _out(out, g.shape, g)
    _lib.require_device(g, u, o)
    _lib.call("axk_silu_mul", g.data_ptr(), u.data_ptr(), o.data_ptr(), g.numel() // n, n, _lib.stream_of(g))
    return o


def add(x: torch.Tensor, y: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """bf16(x + y) for contiguous x, y of one shape."""
    _bf16(x, "x")
    _bf16(y, "y")
    _check(x.shape == y.shape and x.is_contiguous() and y.is_contiguous(), "x and y must be contiguous, same shape")
    n = x.shape[-1]
    o = _out(out, x.shape, x)
    _lib.require_device(x, y, o)
    _lib.call("axk_add", x.data_ptr(), y.data_ptr(), o.data_ptr(), x.numel() // n, n, _lib.stream_of(x))
    return o
