"""GPU parity of the causal multi-token (prefill / speculative verify) attention over the paged cache.

Bar: bf16 outputs within rel 2e-2 / abs 1e-2 of the fp32 oracle (oracle/paged_attn.py paged_prefill); rows that see
no cached token are exactly zero; repeated launches are bitwise identical; bad page ids raise the status flag.
"""
import pytest
import torch

from axk import attention, configs
from oracle import paged_attn as pa

pytestmark = pytest.mark.gpu
TOL = dict(rtol=2e-2, atol=1e-2)


def _dev(c, dev):
    return {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in c.items()}


def _run(c, dev, **kw):
    d = _dev(c, dev)
    return attention.paged_prefill(d["q"], d["cache"], d["qo_indptr"], d["indptr"], d["indices"],
                                   d["last_page_len"], sm_scale=c["scale"], **kw).cpu()


def _ref(c):
    return pa.paged_prefill(c["q"], c["cache"], c["qo_indptr"], c["indptr"], c["indices"], c["last_page_len"],
                            c["scale"])


@pytest.mark.parametrize(
    "qlens,kv_lens,hq,hkv,d,page",
    [
        ([1], [1], 1, 1, 64, 16),
        ([4, 4, 4], [4, 100, 1000], 16, 2, 256, 64),          # speculative verify: 4 rows per sequence
        ([37, 0, 129], [37, 50, 300], 8, 2, 128, 32),          # ragged, an empty query range, history
        ([256], [256], 16, 2, 256, 64),                        # a pure prefill chunk (no history)
        ([300, 17], [2000, 17], 32, 4, 256, 64),               # a chunk after a long history
        ([64, 65, 1], [64, 700, 5], 4, 4, 64, 16),             # group 1
        ([100], [150], 24, 2, 128, 128),                       # group 12: rows straddle tokens
        ([9, 6], [9, 3], 8, 1, 64, 32),                        # a query longer than the cache: early rows see nothing
        ([64], [5000], 8, 2, 128, 16),                         # 313 pages: the page ids reload past 64 pages
        ([40, 7], [90, 700], 12, 3, 128, 32),                  # 3 KV heads: no whole number of XCDs per head
        ([33], [333], 32, 16, 64, 16),                         # 16 KV heads: the per-head XCD mapping is off
    ],
)
def test_paged_prefill_matches_oracle(dev, qlens, kv_lens, hq, hkv, d, page):
    g = torch.Generator().manual_seed(sum(kv_lens) + hq + d)
    c = configs.prefill_case(qlens, kv_lens, hq, hkv, d, page, g, extra_pages=2)
    print(f"case qlens={qlens} kv_lens={kv_lens} hq={hq} hkv={hkv} d={d} page={page}", flush=True)
    got = _run(c, dev)
    ref = _ref(c)
    torch.testing.assert_close(got.float(), ref.to(torch.bfloat16).float(), **TOL)
    zero_rows = ref.abs().amax(dim=(1, 2)) == 0
    assert not got[zero_rows].any()


def test_paged_prefill_chunk_512_and_determinism(dev):
    # the bench workload's shape at an eighth of its length: one sequence, HQ 16 / HKV 2, D 256, page 64, no history
    g = torch.Generator().manual_seed(3)
    c = configs.prefill_case([512], [512], 16, 2, 256, 64, g)
    print("case prefill 512 tokens hq16 hkv2 d256", flush=True)
    got = _run(c, dev)
    torch.testing.assert_close(got.float(), _ref(c).to(torch.bfloat16).float(), **TOL)
    again = _run(c, dev)
    assert torch.equal(got.view(torch.int16), again.view(torch.int16))


def test_paged_prefill_chunk_4096_matches_oracle_and_determinism(dev):
    """The bench workload itself (paged_prefill): one 4096-token chunk, HQ 16 / HKV 2, D 256, page 64, no history,
    against the fp32 oracle, and bit-identical across launches."""
    g = torch.Generator().manual_seed(4096)
    c = configs.prefill_case([4096], [4096], 16, 2, 256, 64, g)
    print("case prefill 4096 tokens hq16 hkv2 d256", flush=True)
    got = _run(c, dev)
    torch.testing.assert_close(got.float(), _ref(c).to(torch.bfloat16).float(), **TOL)
    again = _run(c, dev)
    assert torch.equal(got.view(torch.int16), again.view(torch.int16))


def test_paged_prefill_one_token_matches_decode_kernel(dev):
    g = torch.Generator().manual_seed(4)
    c = configs.prefill_case([1] * 5, [1, 64, 65, 1000, 3000], 16, 2, 256, 64, g)
    print("case one token per sequence vs the decode kernel", flush=True)
    got = _run(c, dev)
    d = _dev(c, dev)
    dec = attention.paged_decode(d["q"], d["cache"], d["indptr"], d["indices"], d["last_page_len"],
                                 sm_scale=c["scale"]).cpu()
    torch.testing.assert_close(got.float(), dec.float(), **TOL)


def test_paged_prefill_bad_page_sets_status(dev):
    g = torch.Generator().manual_seed(6)
    c = configs.prefill_case([8], [40], 8, 2, 64, 16, g)
    c["indices"] = c["indices"].clone()
    c["indices"][1] = c["cache"].shape[0] + 5  # outside the pool: skipped, flagged
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    print("case bad page id", flush=True)
    _run(c, dev, status=status)
    assert int(status.item()) == 1
