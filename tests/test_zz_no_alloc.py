"""GPU check of the no-allocation entry point axk_paged_decode_noalloc (called through the C-ABI) against the
workspace entry point axk_paged_decode on the same inputs: bit-identical outputs (the same kernels and partition run
on the library's static scratch instead of a caller workspace), and within the oracle's bar rel 2e-2 / abs 1e-2. Two
calls in a row, the second smaller, so the second runs over what the first left in the scratch. A request beyond the
scratch is rejected with AXK_E_SCRATCH before anything is launched."""
import pytest
import torch

from axk import _lib, attention, configs
from oracle import paged_attn as pa

pytestmark = pytest.mark.gpu
TOL = dict(rtol=2e-2, atol=1e-2)


def _noalloc(c, dev):
    q, cache = c["q"].to(dev), c["cache"].to(dev)
    indptr, indices, last = (c[k].to(dev) for k in ("indptr", "indices", "last_page_len"))
    b, hq, d = q.shape
    p, _, page, hkv, _ = cache.shape
    out = torch.full_like(q, float("nan"))
    _lib.call("axk_paged_decode_noalloc", q.data_ptr(), cache.data_ptr(), indptr.data_ptr(), indices.data_ptr(),
              last.data_ptr(), out.data_ptr(), b, hq, hkv, d, page, p, float(c["scale"]), _lib.stream_of(q))
    ref = attention.paged_decode(q, cache, indptr, indices, last, sm_scale=c["scale"])
    torch.cuda.synchronize()
    return out.cpu(), ref.cpu()


def test_noalloc_matches_workspace_entry_point(dev):
    g = torch.Generator().manual_seed(7)
    cases = [(configs.config1(), "config1"),
             (configs.paged_case([300, 1, 2000, 77], 8, 2, 128, 32, g), "smaller")]
    for c, name in cases:
        print(f"noalloc case {name}", flush=True)
        got, ref = _noalloc(c, dev)
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), name
        want = pa.paged_decode(c["q"], c["cache"], c["indptr"], c["indices"], c["last_page_len"], c["scale"])
        torch.testing.assert_close(got.float(), want.to(torch.bfloat16).float(), **TOL)


def test_noalloc_rejects_requests_beyond_the_scratch(dev):
    """Refused on the host; the buffers are real and every sequence is empty, so no access could leave them."""
    lib = _lib.load()
    b, hq, hkv, d, page = 63, 1024, 64, 256, 64  # the partials of this shape need about 80 MB
    assert lib.axk_paged_decode_workspace_size(b, hq, hkv, d) > (24 << 20)
    q = torch.zeros(b, hq, d, dtype=torch.bfloat16, device=dev)
    cache = torch.zeros(1, 2, page, hkv, d, dtype=torch.bfloat16, device=dev)
    indptr = torch.zeros(b + 1, dtype=torch.int32, device=dev)
    indices = torch.zeros(1, dtype=torch.int32, device=dev)
    last = torch.zeros(b, dtype=torch.int32, device=dev)
    out = torch.full_like(q, 1.0)
    rc = lib.axk_paged_decode_noalloc(q.data_ptr(), cache.data_ptr(), indptr.data_ptr(), indices.data_ptr(),
                                      last.data_ptr(), out.data_ptr(), b, hq, hkv, d, page, 1, 0.0625,
                                      _lib.stream_of(q))
    assert rc == 10  # AXK_E_SCRATCH
    torch.cuda.synchronize()
    assert bool((out == 1.0).all())  # nothing was launched
