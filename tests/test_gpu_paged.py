"""GPU parity of paged decode attention and the paged KV write against the oracle.

Bar: bf16 outputs within rel 2e-2 / abs 1e-2 of the fp32 golden; the KV write is byte-exact and leaves
every other cache byte untouched; repeated launches are bitwise identical.
"""
import pytest
import torch

import axk
from axk import attention, configs
from oracle import paged_attn as pa

pytestmark = pytest.mark.gpu
TOL = dict(rtol=2e-2, atol=1e-2)


def _run(c, dev, **kw):
    out = attention.paged_decode(
        c["q"].to(dev), c["cache"].to(dev), c["indptr"].to(dev), c["indices"].to(dev),
        c["last_page_len"].to(dev), sm_scale=c["scale"], **kw,
    )
    return out.cpu()


def _ref(c):
    return pa.paged_decode(c["q"], c["cache"], c["indptr"], c["indices"], c["last_page_len"], c["scale"])


@pytest.mark.parametrize(
    "lens,hq,hkv,d,page",
    [
        ([1], 1, 1, 64, 32),
        ([31, 32, 33, 64, 65], 8, 2, 64, 32),
        ([1, 100, 1000], 16, 2, 256, 64),
        ([500, 7, 129], 4, 4, 128, 64),
        ([300, 2000], 16, 1, 128, 256),
        ([64, 0, 65], 8, 1, 256, 64),  # an empty sequence yields zeros
        ([4096] * 3, 32, 4, 256, 64),
        # more than 63 sequences: the partition comes from the plan kernel instead of the run kernels
        ([(37 * i) % 700 for i in range(100)], 8, 1, 128, 32),
        ([1 + (53 * i) % 4000 for i in range(64)], 16, 2, 256, 64),
    ],
)
def test_paged_decode_matches_oracle(dev, lens, hq, hkv, d, page):
    g = torch.Generator().manual_seed(sum(lens) + hq + d)
    c = configs.paged_case(lens, hq, hkv, d, page, g, extra_pages=2)
    print(f"case lens={lens} hq={hq} hkv={hkv} d={d} page={page}", flush=True)
    got = _run(c, dev)
    ref = _ref(c)
    torch.testing.assert_close(got.float(), ref.to(torch.bfloat16).float(), **TOL)
    for b, L in enumerate(lens):
        if L == 0:
            assert not got[b].any()


def test_paged_decode_config1_and_determinism(dev):
    c = configs.config1()
    print(f"config1 lens={c['lens']}", flush=True)
    ws = attention.paged_decode_workspace(16, 16, 2, 256, dev)
    got = _run(c, dev, workspace=ws)
    torch.testing.assert_close(got.float(), _ref(c).to(torch.bfloat16).float(), **TOL)
    again = _run(c, dev, workspace=ws)
    assert torch.equal(got.view(torch.int16), again.view(torch.int16))


def test_paged_decode_ignores_garbage_past_the_tail(dev):
    g = torch.Generator().manual_seed(5)
    c = configs.paged_case([70, 10], 8, 2, 64, 64, g)
    clean = _run(c, dev)
    # poison every slot past each sequence's valid length with NaN: masked slots must not leak
    for b in range(len(c["lens"])):
        last = int(c["indices"][int(c["indptr"][b + 1]) - 1])
        c["cache"][last, :, int(c["last_page_len"][b]):] = float("nan")
    poisoned = _run(c, dev)
    assert torch.equal(clean.view(torch.int16), poisoned.view(torch.int16))


def test_kv_write_then_decode(dev):
    g = torch.Generator().manual_seed(11)
    c = configs.paged_case([65, 128, 1], 8, 2, 128, 64, g, extra_pages=4)
    cache = c["cache"].to(dev)
    before = cache.clone()
    # append one token to each sequence: (page, offset) of token L (a fresh page when L % 64 == 0)
    loc, new_last, new_indices, new_indptr = [], [], [], [0]
    used = set(c["indices"].tolist())
    spare = [p for p in range(c["cache"].shape[0]) if p not in used]
    for b, L in enumerate(c["lens"]):
        pages = c["indices"][int(c["indptr"][b]):int(c["indptr"][b + 1])].tolist()
        if L % 64 == 0:
            pages.append(spare.pop())
        loc.append([pages[-1], L % 64])
        new_indices += pages
        new_indptr.append(len(new_indices))
        new_last.append(L % 64 + 1)
    k = torch.randn(3, 2, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(3, 2, 128, generator=g).to(torch.bfloat16)
    loc_t = torch.tensor(loc, dtype=torch.int32)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    attention.store_paged_kv(k.to(dev), v.to(dev), cache, loc_t.to(dev), status=status)
    ref_cache = pa.store_paged_kv(before.cpu(), k, v, loc_t.numpy())
    assert torch.equal(cache.cpu().view(torch.int16), ref_cache.view(torch.int16))
    assert int(status.item()) == 0
    c2 = dict(c, cache=cache.cpu(), indices=torch.tensor(new_indices, dtype=torch.int32),
              indptr=torch.tensor(new_indptr, dtype=torch.int32), last_page_len=torch.tensor(new_last, dtype=torch.int32),
              lens=[L + 1 for L in c["lens"]])
    got = _run(c2, dev)
    torch.testing.assert_close(got.float(), _ref(c2).to(torch.bfloat16).float(), **TOL)
    # an out-of-pool location is skipped and flagged, the cache stays as it was
    snap = cache.clone()
    attention.store_paged_kv(k[:1].to(dev), v[:1].to(dev), cache,
                             torch.tensor([[10_000, 0]], dtype=torch.int32, device=dev), status=status)
    assert int(status.item()) == 1 and torch.equal(cache, snap)


def test_kv_write_config1(dev):
    # the measured KV write: config 1's current-token rows into its cache, byte-exact, nothing else touched
    c = configs.config1_kv_write()
    cache = c["cache"].to(dev)
    attention.store_paged_kv(c["k"].to(dev), c["v"].to(dev), cache, c["loc"].to(dev))
    ref = pa.store_paged_kv(c["cache"], c["k"], c["v"], c["loc"].numpy())
    assert torch.equal(cache.cpu().view(torch.int16), ref.view(torch.int16))


def test_contract_errors(dev):
    c = configs.paged_case([10], 8, 2, 64, 32, torch.Generator().manual_seed(0))
    with pytest.raises(ValueError):
        attention.paged_decode(c["q"].to(dev), c["cache"].to(dev), c["indptr"].to(dev).long(), c["indices"].to(dev),
                               c["last_page_len"].to(dev))
    small = torch.empty(16, dtype=torch.uint8, device=dev)
    with pytest.raises(axk._lib.AxkError):
        attention.paged_decode(c["q"].to(dev), c["cache"].to(dev), c["indptr"].to(dev), c["indices"].to(dev),
                               c["last_page_len"].to(dev), workspace=small)


@pytest.mark.parametrize("lens", [[100, 3000, 64, 9000], [50 + 13 * i for i in range(70)]])
def test_plan_once_run_many(dev, lens):
    """One plan serves several runs (every attention layer of a step), with the run kernels deriving the
    partition (4 sequences) or reading the plan kernel's (70 sequences)."""
    g = torch.Generator().manual_seed(21)
    bsz = len(lens)
    c = configs.paged_case(lens, 16, 2, 256, 64, g)
    ws = attention.paged_decode_workspace(bsz, 16, 2, 256, dev)
    args = [c[k].to(dev) for k in ("indptr", "indices", "last_page_len")]
    cache = c["cache"].to(dev)
    attention.paged_decode_plan(args[0], args[2], 16, 2, 256, 64, ws)
    for trial in range(3):
        q = torch.randn(bsz, 16, 256, generator=g).to(torch.bfloat16)
        print(f"run {trial}", flush=True)
        got = attention.paged_decode_run(q.to(dev), cache, *args, workspace=ws, sm_scale=c["scale"]).cpu()
        ref = pa.paged_decode(q, c["cache"], c["indptr"], c["indices"], c["last_page_len"], c["scale"])
        torch.testing.assert_close(got.float(), ref.to(torch.bfloat16).float(), **TOL)


# ---- FP8 KV cache (q35_group.py:44-54, KV8=2): stored e4m3(bf16(x * S)), attended stored / S ----
KV_SCALE = 8.0


def _fp8_case(c):
    """c's cache quantised the reference's way, and the bf16 values attention reads from it."""
    codes = pa.quant_kv_fp8(c["cache"], KV_SCALE)
    return codes, pa.dequant_kv_fp8(codes, KV_SCALE)


@pytest.mark.parametrize(
    "lens,hq,hkv,d,page",
    [
        ([1, 100, 1000], 16, 2, 256, 64),
        ([500, 7, 129], 4, 4, 128, 64),
        ([64, 0, 65], 8, 1, 256, 64),  # an empty sequence yields zeros
        ([300, 2000], 16, 1, 128, 256),
        ([(37 * i) % 700 for i in range(70)], 8, 1, 128, 32),  # the plan kernel's partition
    ],
)
def test_paged_decode_fp8(dev, lens, hq, hkv, d, page):
    g = torch.Generator().manual_seed(sum(lens) + hq + d)
    c = configs.paged_case(lens, hq, hkv, d, page, g)
    codes, deq = _fp8_case(c)
    got = axk.paged_decode_fp8(c["q"].to(dev), codes.to(dev), c["indptr"].to(dev), c["indices"].to(dev),
                               c["last_page_len"].to(dev), KV_SCALE, sm_scale=c["scale"]).cpu()
    ref = pa.paged_decode(c["q"], deq, c["indptr"], c["indices"], c["last_page_len"], c["scale"])
    torch.testing.assert_close(got.float(), ref.float(), **TOL)


def test_paged_decode_fp8_config1(dev):
    c = configs.config1()
    codes, deq = _fp8_case(c)
    got = axk.paged_decode_fp8(c["q"].to(dev), codes.to(dev), c["indptr"].to(dev), c["indices"].to(dev),
                               c["last_page_len"].to(dev), KV_SCALE, sm_scale=c["scale"]).cpu()
    ref = pa.paged_decode(c["q"], deq, c["indptr"], c["indices"], c["last_page_len"], c["scale"])
    torch.testing.assert_close(got.float(), ref.float(), **TOL)


def test_kv_write_fp8_bytes(dev):
    """The written bytes equal the reference quantisation (e4m3 of bf16(x * S), round to nearest even; past 464
    after scaling -> NaN), every other byte untouched; includes values at and around the E4M3 ties and limits."""
    g = torch.Generator().manual_seed(5)
    b, hkv, d, page, pages = 6, 2, 128, 32, 9
    k = (torch.randn(b, hkv, d, generator=g) * 4).bfloat16()
    v = (torch.randn(b, hkv, d, generator=g) * 4).bfloat16()
    special = torch.tensor([58.0, 57.0, -58.5, 60.0, -61.0, 0.0, -0.0, 2.0 ** -12, 2.0 ** -13, 3 * 2.0 ** -13,
                            0.1, -0.3, 55.5, 56.0])  # x 8: 464 (tie to 448), 456, -468, 480 (NaN), ...
    k[0, 0, : special.numel()] = special.bfloat16()
    cache = torch.randint(0, 256, (pages, 2, page, hkv, d), generator=g, dtype=torch.uint8)
    loc = torch.tensor([[1, 0], [1, 31], [4, 7], [0, 0], [8, 16], [5, 3]], dtype=torch.int32)
    got = cache.to(dev)
    axk.store_paged_kv_fp8(k.to(dev), v.to(dev), got, loc.to(dev), KV_SCALE)
    ref = cache.clone()
    for i, (p, o) in enumerate(loc.tolist()):
        ref[p, 0, o] = pa.quant_kv_fp8(k[i], KV_SCALE)
        ref[p, 1, o] = pa.quant_kv_fp8(v[i], KV_SCALE)
    assert torch.equal(got.cpu(), ref)


# ---- the local item partition's edge cases (batch <= 63, the kernels derive the plan themselves): many items per
# workgroup, fewer pages than workgroups, tails that are not whole tiles, long sequences split into many items, odd
# KV-head counts ----
@pytest.mark.parametrize(
    "lens,hq,hkv,d,page",
    [
        ([1, 2, 3, 5, 8, 13, 21, 34, 55], 8, 2, 128, 16),   # fewer tiles than workgroups, every tail partial
        ([17] * 63, 4, 1, 64, 16),                            # 63 sequences, units < workgroups
        ([5000, 4097, 16], 12, 3, 128, 16),                  # 313 pages of 16 tokens: two chunk crossings
        ([9000, 1, 0, 700], 16, 1, 256, 32),                 # empty sequence between others
        ([16 * i + 1 for i in range(40)], 32, 16, 64, 16),   # 16 KV heads, many short pairs per workgroup
        ([100000], 16, 2, 256, 64),                          # one long sequence over every workgroup
    ],
)
def test_paged_decode_local_partition(dev, lens, hq, hkv, d, page):
    g = torch.Generator().manual_seed(len(lens) * 7 + hkv)
    c = configs.paged_case(lens, hq, hkv, d, page, g, extra_pages=1)
    print(f"case lens={lens[:6]}.. hq={hq} hkv={hkv} d={d} page={page}", flush=True)
    got = _run(c, dev)
    torch.testing.assert_close(got.float(), _ref(c).to(torch.bfloat16).float(), **TOL)
    for b, L in enumerate(lens):
        if L == 0:
            assert not got[b].any()


def test_local_plan_garbage_workspace_and_changing_partitions(dev):
    """The split and merge keep nothing in the workspace from one call to the next: a workspace of random
    bytes, then calls whose partitions differ (other lengths, so other pieces per pair) on that same workspace, each
    against the oracle and bit-identical to the same call on a fresh zeroed workspace."""
    g = torch.Generator().manual_seed(77)
    ws = attention.paged_decode_workspace(6, 16, 2, 256, dev)
    ws.copy_(torch.randint(0, 256, ws.shape, generator=g, dtype=torch.uint8).to(dev))
    for trial, lens in enumerate([[3000, 17, 900, 4100, 64, 2500], [5, 9000, 1, 0, 700, 300],
                                  [3000, 17, 900, 4100, 64, 2500]]):
        c = configs.paged_case(lens, 16, 2, 256, 64, g)
        print(f"trial {trial} lens={lens}", flush=True)
        got = _run(c, dev, workspace=ws)
        fresh = _run(c, dev, workspace=torch.zeros_like(ws))
        assert torch.equal(got.view(torch.int16), fresh.view(torch.int16))
        torch.testing.assert_close(got.float(), _ref(c).to(torch.bfloat16).float(), **TOL)


def test_local_plan_graph_replays_with_new_page_tables(dev):
    """A captured decode (split + merge) replayed with the page table rewritten in place between replays (lengths
    change, so the partition the kernels derive changes): every replay equals the eager call, with eager calls on the
    same workspace in between."""
    g = torch.Generator().manual_seed(78)
    bsz, hq, hkv, d, page = 5, 16, 2, 256, 64
    pool = 400
    cache = (torch.randn(pool, 2, page, hkv, d, generator=g) * 0.5).bfloat16().to(dev)
    q = torch.randn(bsz, hq, d, generator=g).bfloat16().to(dev)
    ws = attention.paged_decode_workspace(bsz, hq, hkv, d, dev)
    indptr = torch.zeros(bsz + 1, dtype=torch.int32, device=dev)
    indices = torch.zeros(pool, dtype=torch.int32, device=dev)
    last = torch.ones(bsz, dtype=torch.int32, device=dev)
    out = torch.empty_like(q)

    def set_table(lens):
        npg = [(L + page - 1) // page for L in lens]
        ptr = torch.tensor([0] + torch.tensor(npg).cumsum(0).tolist(), dtype=torch.int32)
        perm = torch.randperm(pool, generator=g)[: int(ptr[-1])].to(torch.int32)
        indptr.copy_(ptr.to(dev))
        indices[: len(perm)].copy_(perm.to(dev))
        last.copy_(torch.tensor([L - (n - 1) * page for L, n in zip(lens, npg)], dtype=torch.int32).to(dev))

    tables = [[4000, 130, 6000, 64, 2000], [64, 64, 9000, 3000, 128], [7000, 1, 65, 4500, 2222]]
    set_table(tables[0])
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            attention.paged_decode(q, cache, indptr, indices, last, sm_scale=d ** -0.5, output=out, workspace=ws)
    torch.cuda.synchronize()
    for rep in range(6):
        set_table(tables[rep % 3])
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        eager = attention.paged_decode(q, cache, indptr, indices, last, sm_scale=d ** -0.5, workspace=ws)
        torch.cuda.synchronize()
        print(f"replay {rep} table {rep % 3}", flush=True)
        assert torch.equal(got.view(torch.int16), eager.view(torch.int16))
        if rep < 3:
            ref = pa.paged_decode(q.cpu(), cache.cpu(), indptr.cpu(), indices.cpu(), last.cpu(), d ** -0.5)
            torch.testing.assert_close(got.float().cpu(), ref.to(torch.bfloat16).float(), **TOL)


# ---- the sgl decode convention (flash_attn.py:2335-2357): last_page_len counts history only, may be 0 ----
def _sgl_reference_case(history, g, hq=8, hkv=2, d=256, page=256):
    """The metadata of the reference's own runtime test (test_qwen35_runtime.py:96-118): a 32-page pool of 256-token
    pages, page list [7, 2, 11], page_count = history // 256 + 1, last_page_len = history % 256 and the current token
    at cache_location = [rows[-1], history % 256]."""
    cache = (torch.randn(32, 2, page, hkv, d, generator=g) * 0.05).bfloat16()
    indices = torch.tensor([7, 2, 11] + [0] * 29, dtype=torch.int32)
    page_count = history // page + 1
    rows = indices[:page_count].long()
    q = torch.randn(1, hq, d, generator=g).bfloat16()
    k = torch.randn(1, hkv, d, generator=g).bfloat16()
    v = torch.randn(1, hkv, d, generator=g).bfloat16()
    return dict(cache=cache, indices=indices, rows=rows, q=q, k=k, v=v,
                indptr=torch.tensor([0, page_count], dtype=torch.int32),
                last=torch.tensor([history % page], dtype=torch.int32),
                loc=torch.tensor([[int(rows[-1]), history % page]], dtype=torch.int32))


@pytest.mark.parametrize("history", [0, 1, 255, 256, 514])
def test_paged_attention_decode_sgl_convention(dev, history):
    g = torch.Generator().manual_seed(history)
    c = _sgl_reference_case(history, g)
    hkv, d = c["k"].shape[1], c["k"].shape[2]
    print(f"sgl history={history}", flush=True)
    cache = c["cache"].to(dev)
    got = attention.paged_attention_decode(c["q"].to(dev), c["k"].to(dev), c["v"].to(dev), cache,
                                           c["indptr"].to(dev), c["indices"].to(dev), c["last"].to(dev),
                                           c["loc"].to(dev)).cpu()
    # the reference's golden: SDPA over the gathered history plus the current token (test_qwen35_runtime.py:73-84)
    hk = c["cache"][c["rows"], 0].reshape(-1, hkv, d)[:history]
    hv = c["cache"][c["rows"], 1].reshape(-1, hkv, d)[:history]
    kk = torch.cat((hk, c["k"]), 0).float().transpose(0, 1)[None]
    vv = torch.cat((hv, c["v"]), 0).float().transpose(0, 1)[None]
    ref = torch.nn.functional.scaled_dot_product_attention(c["q"].float()[:, :, None, :], kk, vv, enable_gqa=True)
    torch.testing.assert_close(got.float(), ref[:, :, 0, :].bfloat16().float(), **TOL)
    # the current token's rows written, every other cache byte untouched
    want = c["cache"].clone()
    want[c["rows"][-1], 0, history % 256] = c["k"][0]
    want[c["rows"][-1], 1, history % 256] = c["v"][0]
    assert torch.equal(cache.cpu().view(torch.int16), want.view(torch.int16))


def test_paged_attention_decode_sgl_convention_matches_paged_decode(dev):
    """History-only last_page_len (+ the written current token) == axk_paged_decode with last_page_len + 1, for a
    batch whose kernels derive the partition themselves (16) and one that takes the plan kernel's items (70)."""
    for bsz in (16, 70):
        g = torch.Generator().manual_seed(bsz)
        hist = [int(x) for x in torch.randint(0, 3000, (bsz,), generator=g)]
        hist[0] = 0
        hist[1] = 64
        c = configs.append_token_case(hist, 8, 2, 128, 64, g)
        k = torch.randn(bsz, 2, 128, generator=g).bfloat16()
        v = torch.randn(bsz, 2, 128, generator=g).bfloat16()
        hist_last = (c["last_page_len"] - 1).to(torch.int32)
        print(f"sgl batch={bsz}", flush=True)
        cache = c["cache"].to(dev)
        got = attention.paged_attention_decode(c["q"].to(dev), k.to(dev), v.to(dev), cache, c["indptr"].to(dev),
                                               c["indices"].to(dev), hist_last.to(dev), c["loc"].to(dev)).cpu()
        ref_cache = pa.store_paged_kv(c["cache"], k, v, c["loc"].numpy())
        ref = pa.paged_decode(c["q"], ref_cache, c["indptr"], c["indices"], c["last_page_len"], c["scale"])
        torch.testing.assert_close(got.float(), ref.to(torch.bfloat16).float(), **TOL)
        assert torch.equal(cache.cpu().view(torch.int16), ref_cache.view(torch.int16))


# ---- INT8 KV cache with a bf16 scale per row and KV head (q35_group.py:44-47, 197-221, 250-255; KV8=1) ----
def _i8_case(c):
    """c's cache quantized the reference's way (codes, scales), and the bf16 values attention reads from it."""
    codes, scales = pa.quant_kv_i8(c["cache"])
    return codes, scales, pa.dequant_kv_i8(codes, scales)


@pytest.mark.parametrize(
    "lens,hq,hkv,d,page",
    [
        ([1, 100, 1000], 16, 2, 256, 64),
        ([500, 7, 129], 4, 4, 128, 64),
        ([64, 0, 65], 8, 1, 256, 64),  # an empty sequence yields zeros
        ([300, 2000], 16, 1, 128, 256),
        ([40, 900], 16, 16, 128, 16),  # 16 KV heads: a tile's scales fill every lane of the four waves
        ([(37 * i) % 700 for i in range(70)], 24, 8, 128, 32),  # the plan kernel's partition, 8 KV heads
    ],
)
def test_paged_decode_i8(dev, lens, hq, hkv, d, page):
    g = torch.Generator().manual_seed(sum(lens) + hq + d + hkv)
    c = configs.paged_case(lens, hq, hkv, d, page, g)
    print(f"i8 decode lens={lens[:4]} hq={hq} hkv={hkv} d={d} page={page}", flush=True)
    codes, scales, deq = _i8_case(c)
    got = axk.paged_decode_i8(c["q"].to(dev), codes.to(dev), scales.to(dev), c["indptr"].to(dev),
                              c["indices"].to(dev), c["last_page_len"].to(dev), sm_scale=c["scale"]).cpu()
    ref = pa.paged_decode(c["q"], deq, c["indptr"], c["indices"], c["last_page_len"], c["scale"])
    torch.testing.assert_close(got.float(), ref.float(), **TOL)
    for b, L in enumerate(lens):
        if L == 0:
            assert not got[b].any()


def test_paged_decode_i8_config1(dev):
    c = configs.config1()
    codes, scales, deq = _i8_case(c)
    got = axk.paged_decode_i8(c["q"].to(dev), codes.to(dev), scales.to(dev), c["indptr"].to(dev),
                              c["indices"].to(dev), c["last_page_len"].to(dev), sm_scale=c["scale"]).cpu()
    ref = pa.paged_decode(c["q"], deq, c["indptr"], c["indices"], c["last_page_len"], c["scale"])
    torch.testing.assert_close(got.float(), ref.float(), **TOL)


@pytest.mark.parametrize("d,hkv", [(128, 2), (256, 4)])
def test_kv_write_i8_bytes(dev, d, hkv):
    """The written codes and scales equal the reference quantization bit for bit (incl. a zero row, an outlier and
    rows of mixed magnitude); every other cache and scale byte untouched."""
    g = torch.Generator().manual_seed(7 + d)
    b, page, pages = 6, 32, 9
    k = (torch.randn(b, hkv, d, generator=g) * 4).bfloat16()
    v = (torch.randn(b, hkv, d, generator=g) * torch.logspace(-3, 2, d)).bfloat16()
    k[1, 0] = 0
    k[2, hkv - 1, 5] = 1000.0
    cache = torch.randint(-128, 128, (pages, 2, page, hkv, d), generator=g, dtype=torch.int8)
    scales = torch.randn(pages, 2, page, hkv, generator=g).bfloat16()
    loc = torch.tensor([[1, 0], [1, 31], [4, 7], [0, 0], [8, 16], [5, 3]], dtype=torch.int32)
    gc, gs = cache.to(dev), scales.to(dev)
    axk.store_paged_kv_i8(k.to(dev), v.to(dev), gc, gs, loc.to(dev))
    rc, rs = pa.store_paged_kv_i8(cache, scales, k, v, loc)
    assert torch.equal(gc.cpu(), rc)
    assert torch.equal(gs.cpu().view(torch.int16), rs.view(torch.int16))


def _i8_tie_rows(d):
    """Rows whose scale is exactly 1 (amax 127 or 127.5: bf16(amax * bf16(1 / 127)) = 1), so every code is
    round(x) of an exact product: half-integers x = n + 0.5 (ties), and +-127.5 (past 127: saturation)."""
    rows = []
    half = torch.arange(d, dtype=torch.float32) - d // 2 + 0.5       # ..., -1.5, -0.5, 0.5, 1.5, ... (every tie)
    half = torch.where(half.abs() > 126, half.sign() * 126.5, half)  # inside (-127, 127)
    r = half.clone(); r[0] = 127.0; rows.append(r)                    # amax 127: ties only
    r = -half.clone(); r[1] = -127.0; rows.append(r)                  # negative amax
    r = half.clone(); r[2] = 127.5; r[3] = -127.5; rows.append(r)     # 127.5 -> 128 (saturates to 127); -127.5 -> -128
    return torch.stack(rows)


def test_kv_write_i8_ties_and_saturation(dev):
    """Ties and saturation of the int8 cast, pinned kernel == oracle (round half to even, clamp to [-128, 127]) on rows
    where the products are exact half-integers and +-127.5, for both head dims."""
    for d in (128, 256):
        hkv, page = 3, 16
        rows = _i8_tie_rows(d).bfloat16()
        assert torch.equal(rows.float(), _i8_tie_rows(d))  # every value exactly representable
        k = rows.reshape(1, 3, d)
        v = (-rows).reshape(1, 3, d)
        cache = torch.zeros(2, 2, page, hkv, d, dtype=torch.int8)
        scales = torch.zeros(2, 2, page, hkv).bfloat16()
        loc = torch.tensor([[1, 5]], dtype=torch.int32)
        gc, gs = cache.to(dev), scales.to(dev)
        axk.store_paged_kv_i8(k.to(dev), v.to(dev), gc, gs, loc.to(dev))
        rc, rs = pa.store_paged_kv_i8(cache, scales, k, v, loc)
        assert torch.equal(gc.cpu(), rc) and torch.equal(gs.cpu().view(torch.int16), rs.view(torch.int16))
        assert (rs[1, :, 5].float() == 1.0).all()
        codes = gc.cpu()[1, 0, 5]
        assert codes[0, 0] == 127 and codes[2, 2] == 127 and codes[2, 3] == -128  # saturation
        assert codes[0, d // 2] == 0 and codes[0, d // 2 + 1] == 2 and codes[0, d // 2 - 1] == 0  # 0.5, 1.5, -0.5


def test_kv_write_then_decode_i8(dev):
    """Write the new token of every sequence through axk, then decode over the INT8 cache: equal to the oracle's
    write + decode (the bf16 cache's append case, quantized)."""
    g = torch.Generator().manual_seed(12)
    hq, hkv, d, page = 8, 2, 128, 64
    c = configs.append_token_case([100, 63, 300], hq, hkv, d, page, g)
    codes, scales = pa.quant_kv_i8(c["cache"])
    k = torch.randn(3, hkv, d, generator=g).bfloat16()
    v = torch.randn(3, hkv, d, generator=g).bfloat16()
    q = torch.randn(3, hq, d, generator=g).bfloat16()
    gc, gs = codes.to(dev), scales.to(dev)
    axk.store_paged_kv_i8(k.to(dev), v.to(dev), gc, gs, c["loc"].to(dev))
    got = axk.paged_decode_i8(q.to(dev), gc, gs, c["indptr"].to(dev), c["indices"].to(dev),
                              c["last_page_len"].to(dev)).cpu()
    rc, rs = pa.store_paged_kv_i8(codes, scales, k, v, c["loc"])
    ref = pa.paged_decode(q, pa.dequant_kv_i8(rc, rs), c["indptr"], c["indices"], c["last_page_len"], d ** -0.5)
    torch.testing.assert_close(got.float(), ref.float(), **TOL)
