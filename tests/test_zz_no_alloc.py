"""GPU check of the no-allocation entry point axk_paged_decode_noalloc (called through the C-ABI) against the
workspace entry point axk_paged_decode on the same inputs: bit-identical outputs (the same kernels and partition run
on the library's static scratch instead of a caller workspace), and within the oracle's bar rel 2e-2 / abs 1e-2. Two
calls in a row, the second smaller, so the second runs over what the first left in the scratch. A request beyond the
scratch is rejected with AXK_E_SCRATCH before anything is launched. After one eager call, a captured call replayed over
page tables rewritten in place equals the workspace entry point on every replay."""
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


def test_noalloc_captured_replays_over_rewritten_page_tables(dev):
    """The no-allocation call captured in a HIP graph (after the eager calls above did the one-time set-up) and replayed
    with the page table rewritten in place between replays (so the partition the kernels derive changes): every replay
    is bit-identical to axk_paged_decode on the same table, with that eager call (on its own workspace) in between."""
    g = torch.Generator().manual_seed(79)
    bsz, hq, hkv, d, page, pool = 5, 16, 2, 256, 64, 400
    cache = (torch.randn(pool, 2, page, hkv, d, generator=g) * 0.5).bfloat16().to(dev)
    q = torch.randn(bsz, hq, d, generator=g).bfloat16().to(dev)
    indptr = torch.zeros(bsz + 1, dtype=torch.int32, device=dev)
    indices = torch.zeros(pool, dtype=torch.int32, device=dev)
    last = torch.ones(bsz, dtype=torch.int32, device=dev)
    out = torch.empty_like(q)
    lib = _lib.load()

    def set_table(lens):
        npg = [(L + page - 1) // page for L in lens]
        ptr = torch.tensor([0] + torch.tensor(npg).cumsum(0).tolist(), dtype=torch.int32)
        perm = torch.randperm(pool, generator=g)[: int(ptr[-1])].to(torch.int32)
        indptr.copy_(ptr.to(dev))
        indices[: len(perm)].copy_(perm.to(dev))
        last.copy_(torch.tensor([L - (n - 1) * page for L, n in zip(lens, npg)], dtype=torch.int32).to(dev))

    def call(stream):
        return lib.axk_paged_decode_noalloc(q.data_ptr(), cache.data_ptr(), indptr.data_ptr(), indices.data_ptr(),
                                            last.data_ptr(), out.data_ptr(), bsz, hq, hkv, d, page, pool, d ** -0.5,
                                            stream)

    tables = [[4000, 130, 6000, 64, 2000], [64, 64, 9000, 3000, 128], [7000, 1, 65, 4500, 2222]]
    set_table(tables[0])
    assert call(_lib.stream_of(q)) == 0  # eager: the one-time set-up on this device
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            rc = call(stream.cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    for rep in range(6):
        set_table(tables[rep % 3])
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        eager = attention.paged_decode(q, cache, indptr, indices, last, sm_scale=d ** -0.5)
        torch.cuda.synchronize()
        print(f"noalloc replay {rep} table {rep % 3}", flush=True)
        assert torch.equal(got.view(torch.int16), eager.view(torch.int16))
