"""The oracle's bf16 rounding points, switchable (CPU, test infrastructure only).

The layer and MoE restatements round every intermediate tensor to bf16 where the reference stores one
(q35_step.py rmsnorm / linear outputs, q35_moe.py:96-137 gate / up / act). `fp32()` turns every such point into
an fp32 pass-through, so a composition can be compared at fp32 tolerance with an fp32 formulation of the same
model (transformers' Qwen3.5 modules), which pins the composition itself: op order, operand roles, gate and
residual wiring. The rounding schedule is then pinned separately, as bf16 mode within tolerance of fp32 mode.
"""
from __future__ import annotations

import contextlib

import torch

_ROUND = [True]


def bf(x: torch.Tensor) -> torch.Tensor:
    """bf16(x) at a rounding point; fp32 x when the points are switched off."""
    return x.to(torch.bfloat16) if _ROUND[0] else x.float()


def rounding() -> bool:
    return _ROUND[0]


@contextlib.contextmanager
def fp32():
    """Within the block every rounding point of oracle.layer / oracle.moe is an fp32 pass-through."""
    prev = _ROUND[0]
    _ROUND[0] = False
    try:
        yield
    finally:
        _ROUND[0] = prev
