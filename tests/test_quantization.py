"""The host NVFP4 codec (axk.quantize_nvfp4, the role of sgl_kernel_axera/quantization.py:8-37) against the oracle's
restatement and the reference test's vectors (CPU only)."""
import numpy as np
import pytest
import torch

from axk import quantize_nvfp4
from oracle import mx


@pytest.mark.parametrize("shape,dtype", [((37, 64), torch.float32), ((5, 2048), torch.bfloat16),
                                         ((1100, 48), torch.float16), ((3, 16), torch.float32)])
def test_quantize_nvfp4_matches_oracle(shape, dtype):
    g = torch.Generator().manual_seed(shape[0] * shape[1])
    w = (torch.randn(*shape, generator=g) * torch.logspace(-3, 1, shape[0])[:, None]).to(dtype)
    w[0, :2] = torch.tensor([0.0, -0.0])
    packed, scales, s2 = quantize_nvfp4(w)
    assert packed.dtype == torch.float4_e2m1fn_x2 and packed.shape == (shape[0], shape[1] // 2)
    assert scales.dtype == torch.float8_e4m3fn and scales.shape == (shape[0], shape[1] // 16)
    assert s2.dtype == torch.float32 and s2.shape == (1,)
    rp, rs, r2 = mx.quantize_nvfp4(w.float().numpy())
    assert np.array_equal(packed.view(torch.uint8).numpy(), rp)
    assert np.array_equal(scales.view(torch.uint8).numpy(), rs)
    assert s2.item() == float(r2)


def test_quantize_nvfp4_reference_vectors():
    """test_nvfp4_lm_head.py:19-39: the midpoint row codes to the even neighbours, zero blocks stay zero."""
    src = torch.zeros(3, 32, dtype=torch.bfloat16)
    src[0, 0] = 448 * 6
    src[1, :16] = torch.tensor([0, 0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5, 6, -0.25, -0.75, -1.25, -1.75, -2.5, -3.5, -5])
    packed, scales, s2 = quantize_nvfp4(src)
    expected = torch.tensor([0, 0, 2, 2, 4, 4, 6, 6, 7, 8, 10, 10, 12, 12, 14, 14], dtype=torch.uint8)
    assert torch.equal(packed.view(torch.uint8)[1, :8], expected[::2] | (expected[1::2] << 4))
    assert not packed.view(torch.uint8)[2].any()
    assert scales.float()[1, 0] == 1 and not scales.float()[2].any() and s2.tolist() == [1]
    zp, zs, z2 = quantize_nvfp4(torch.zeros(2, 16))
    assert z2.item() == 1 and not zp.view(torch.uint8).any() and not zs.float().any()


def test_quantize_nvfp4_contract():
    with pytest.raises(ValueError, match="divisible by 16"):
        quantize_nvfp4(torch.zeros(2, 24))
    with pytest.raises(ValueError, match="floating-point"):
        quantize_nvfp4(torch.zeros(2, 32, dtype=torch.int32))
