"""The IO-table query (axk_io_table, host only) and the manifest / pack binder (axk.manifest) against the reference's
own manifests: the 9B whole-model manifest (MXFP4 layers, banks, column strips) and the 35B-A3B manifest (MXFP8 layers,
MoE, column blocks), committed as data fixtures by tests/golden/make_manifest_fixtures.py.

The IO table is compared entry by entry (name, bytes, dtype, shape, in order) with the manifests' params and the
output head's IO, the name -> bytes check of models/qwen35_35b_a3b/sgl/scripts/check_adapter_abi.py:20-56 made exact.
The binder is checked on the manifests' real member tables (placement, alignment, byte counts) and by a store -> bind
round trip on host buffers at the manifests' full pack sizes; the column-split byte order is pinned by small cases
written out by hand from the reference's packers (q35_layer_pk.py blocked(): [R, C] -> its column strips stacked;
q35_layer_mc.py pk_packed(): the column blocks one after the other, each [rows, cols] row-major).
"""
import ctypes
import os

import pytest
import torch

from axk import _lib, configs
from axk import manifest as mf

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "manifests")
M9 = os.path.join(HERE, "qwen35_9b_c131072.manifest.json")
M35 = os.path.join(HERE, "qwen35_35b_a3b.manifest.json")
LAYOUT9 = os.path.join(HERE, "qwen35_9b_group16_gggagggagggaggga_mx4_kvc_c16384_npu4.layout")
RUNTIME = {"x", "state_in", "conv_in", "out", "state_out", "conv_out", "cos", "sin", "indptr", "indices",
           "last_page_len", "cache_location", "kv_cache"}


def _params(table):
    return [e for e in table["in"] if e[0] not in RUNTIME]


def _manifest_params(m, kind):
    return [[n, e.bytes, e.dtype, list(e.shape)] for n, e in m.params[kind].items()]


@pytest.fixture(scope="module")
def m9():
    return mf.Manifest.load(M9)


@pytest.fixture(scope="module")
def m35():
    return mf.Manifest.load(M35)


# ---- IO table -------------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("path,k", [(M9, 4096), (M35, 2048)])
def test_io_table_lm_head_matches_manifest(path, k):
    m = mf.Manifest.load(path)
    ref = m.kernel("lm_head").io_table()
    # the manifest's x is [1, K]; the board's row count is the m dimension
    assert mf.io_table("lm_head", n=248320, k=k) == ref


def test_io_table_layer_params_match_the_9b_manifest(m9):
    # Qwen3.5-9B: hidden 4096, GDN 16 / 32 heads, attention 16 / 4 heads of 256, MLP 12288, every weight MXFP4
    g = mf.io_table("layer.gdn", hidden=4096, num_k_heads=16, num_v_heads=32, inter=12288, proj_fmt="mxfp4",
                    mlp_fmt="mxfp4")
    assert _params(g) == _manifest_params(m9, "gdn")
    a = mf.io_table("layer.attn", hidden=4096, num_qo_heads=16, num_kv_heads=4, head_dim=256, inter=12288,
                    proj_fmt="mxfp4", mlp_fmt="mxfp4")
    assert _params(a) == _manifest_params(m9, "attn")


def test_io_table_layer_params_match_the_35b_manifest(m35):
    # Qwen3.5-35B-A3B: hidden 2048, MXFP8 layer weights, shared expert 512 as the dense MLP, 256 routed experts
    g = mf.io_table("layer.gdn", hidden=2048, num_k_heads=16, num_v_heads=32, inter=512, proj_fmt="mxfp8",
                    mlp_fmt="mxfp8", num_experts=256)
    assert _params(g) == _manifest_params(m35, "gdn")
    a = mf.io_table("layer.attn", hidden=2048, num_qo_heads=16, num_kv_heads=2, head_dim=256, inter=512,
                    proj_fmt="mxfp8", mlp_fmt="mxfp8", num_experts=256)
    assert _params(a) == _manifest_params(m35, "attn")
    e = mf.io_table("experts", num_experts=256, hidden=2048, inter=512)
    assert e["in"] == _manifest_params(m35, "experts")


def test_io_table_resident_state_matches_the_groups(m9, m35):
    """The GDN layer's state / conv state are the groups' resident st<j> / cv<j> (35B) bytes, dtype and shape; the
    attention layer's paged cache has the 9B group's kv<j> bytes and dtype ([P, 2, page, HKV D] there,
    [P, 2, page, HKV, D] here)."""
    g = mf.io_table("layer.gdn", hidden=2048, num_k_heads=16, num_v_heads=32, inter=512, proj_fmt="mxfp8",
                    mlp_fmt="mxfp8", num_experts=256)
    outs = {e[0]: e for e in g["out"]}
    grp = m35.kernel("decode.group")
    st, cv = grp.entry("st0"), grp.entry("cv0")
    assert outs["state_out"][1:] == [st.bytes, st.dtype, list(st.shape)]
    assert outs["conv_out"][1:] == [cv.bytes, cv.dtype, list(cv.shape)]
    assert outs["out"][1:] == [grp.entry("out").bytes, 9, [1, 1, 2048]]
    a = mf.io_table("layer.attn", hidden=4096, num_qo_heads=16, num_kv_heads=4, head_dim=256, inter=12288,
                    page_size=256, num_pages=512)
    kv = {e[0]: e for e in a["out"]}["kv_cache"]
    ref = m9.kernel("decode.group").entry("kv3")
    assert kv[1:3] == [ref.bytes, ref.dtype] and kv[3] == [512, 2, 256, 4, 256]


def test_io_table_errors():
    lib = _lib.load()
    count = ctypes.c_int(-1)
    dims = (ctypes.c_int64 * 2)(248320, 2048)
    st = lib.axk_io_table(b"no.such.role", ctypes.addressof(dims), 2, None, 0, ctypes.addressof(count))
    assert st == 8  # AXK_E_ROLE
    st = lib.axk_io_table(b"lm_head", ctypes.addressof(dims), 2, None, 0, ctypes.addressof(count))
    assert st == 9 and count.value == 4  # AXK_E_BUFFER, the number of entries needed
    buf = (mf._IoEntryC * 3)()
    st = lib.axk_io_table(b"lm_head", ctypes.addressof(dims), 2, ctypes.addressof(buf), 3, ctypes.addressof(count))
    assert st == 9 and count.value == 4 and buf[2].name == b"s"  # the first 3 are filled
    bad = (ctypes.c_int64 * 2)(248320, 2047)  # k not a multiple of 32
    assert lib.axk_io_table(b"lm_head", ctypes.addressof(bad), 2, None, 0, ctypes.addressof(count)) == 2
    assert lib.axk_io_table(b"lm_head", ctypes.addressof(dims), 1, None, 0, ctypes.addressof(count)) == 2
    five = (ctypes.c_int64 * 7)(2048, 16, 32, 512, 4, 7, 1)  # weight format 7
    assert lib.axk_io_table(b"layer.gdn", ctypes.addressof(five), 7, None, 0, ctypes.addressof(count)) == 4
    with pytest.raises(ValueError):
        mf.io_table("lm_head", n=8)


# ---- manifests and layouts ------------------------------------------------------------------------------------------
def test_layout_file_matches_the_manifest_members(m9):
    packs, members = mf.parse_layout(open(LAYOUT9).read())
    k = m9.kernel("decode.group")
    assert packs == k.packs
    assert [(m.name, m.pack, m.offset, m.bytes, m.layer, m.param, m.strips) for m in members] == \
        [(m.name, m.pack, m.offset, m.bytes, m.layer, m.param, m.strips) for m in k.members]


@pytest.mark.parametrize("path,role", [(M9, "decode.group"), (M35, "decode.group"), (M35, "prefill256.gdn"),
                                       (M35, "prefill256.attn")])
def test_manifest_members_are_consistent(path, role):
    m = mf.Manifest.load(path)
    m.check_members(role)  # raises on any misplaced, misaligned, overlapping or mis-sized member


def test_group_kinds(m9, m35):
    assert m9.kernel("decode.group").kinds() == ["gdn", "gdn", "gdn", "attn"] * 4
    assert m35.kernel("decode.group").kinds() == ["gdn", "gdn", "gdn", "attn"] * 2


def test_column_split_byte_order_by_hand():
    """The stored order of the reference's packers, written out for small cases."""
    w = torch.arange(2 * 8, dtype=torch.uint8).view(2, 8)  # rows [0..7], [8..15]
    strips = mf.Member("L0.w_out", "p4", 0, 16, "w_out", 0, None, (2, 8, 4))
    # blocked(): cat([w[:, 0:4], w[:, 4:8]], dim=0) -> rows 0:4 of both rows, then 4:8 of both rows
    assert strips.from_row_major(w).tolist() == [0, 1, 2, 3, 8, 9, 10, 11, 4, 5, 6, 7, 12, 13, 14, 15]
    assert torch.equal(strips.to_row_major(strips.from_row_major(w)), w)
    # pk_packed(): the ranges in storage order (here core-major and permuted), each [rows, b - a] row-major
    blocks = mf.Member("L0.w_o", "pw", 0, 16, "w_o", 0, None, None, (2, 8, ((4, 6), (0, 4), (6, 8))))
    assert blocks.from_row_major(w).tolist() == [4, 5, 12, 13, 0, 1, 2, 3, 8, 9, 10, 11, 6, 7, 14, 15]
    assert torch.equal(blocks.to_row_major(blocks.from_row_major(w)), w)


def test_check_buffers_name_to_bytes(m35):
    k = m35.kernel("lm_head")
    bufs = {"x": torch.empty(2048, dtype=torch.bfloat16), "w": torch.empty(248320, 1024, dtype=torch.uint8),
            "s": torch.empty(248320, 64, dtype=torch.uint8), "out": torch.empty(248320)}
    k.check_buffers(bufs)
    bufs["s"] = torch.empty(248320, 63, dtype=torch.uint8)
    with pytest.raises(ValueError, match="s: 15644160 bytes"):
        k.check_buffers(bufs)
    del bufs["out"]
    with pytest.raises(ValueError, match="out: missing"):
        k.check_buffers(bufs)


# ---- store -> bind round trips at the manifests' pack sizes (host buffers, only the bound layers written) ----------
def _buffers(k, names):
    out = {}
    for e in k.inputs:
        if e.name in names:
            out[e.name] = torch.zeros(e.bytes, dtype=torch.uint8)
    return out


def _weights_9b(g, kind):
    if kind == "gdn":
        return configs.gdn_layer_weights(g, 4096, 12288, 16, 32, proj_fmt="mxfp4", mlp_fmt="mxfp4")
    return configs.attn_layer_weights(g, 4096, 12288, 16, 4, 256, proj_fmt="mxfp4", mlp_fmt="mxfp4")


def _same(a, b):
    return a.dtype == b.dtype and a.shape == b.shape and torch.equal(a.view(torch.uint8), b.view(torch.uint8))


@pytest.mark.parametrize("layer", [0, 2, 7])
def test_bind_9b_group_layer_round_trip(m9, layer):
    k = m9.kernel("decode.group")
    kind = k.kinds()[layer]
    names = set(k.packs) | {f"k_b{layer % 4}_{b}" for b in mf.BANKS[kind]}
    bufs = _buffers(k, names)
    w = _weights_9b(torch.Generator().manual_seed(layer), kind)
    w = {n: t.to(torch.float32) if n in ("a_log", "dt_bias") else t for n, t in w.items()}
    m9.store_layer("decode.group", bufs, layer, w)
    b = m9.bind_layer("decode.group", bufs, layer)
    assert b.kind == kind and b.proj_fmt == "mxfp4" and b.mlp_fmt == "mxfp4"
    assert set(b.weights) == set(m9.params[kind])
    for n, t in b.weights.items():
        assert _same(t, w[n]), n
    # plain pack members bind as views of the pack (no copy)
    ln1 = b.weights["ln1"]
    assert ln1.untyped_storage().data_ptr() == bufs["pf"].untyped_storage().data_ptr()


@pytest.mark.parametrize("layer", [1, 3])
def test_bind_35b_group_layer_round_trip(m35, layer):
    k = m35.kernel("decode.group")
    kind = k.kinds()[layer]
    bufs = _buffers(k, set(k.packs))
    g = torch.Generator().manual_seed(100 + layer)
    if kind == "gdn":
        w = configs.gdn_layer_weights(g, 2048, 512, 16, 32, proj_fmt="mxfp8", mlp_fmt="mxfp8")
    else:
        w = configs.attn_layer_weights(g, 2048, 512, 16, 2, 256, proj_fmt="mxfp8", mlp_fmt="mxfp8")
    w["w_router"] = (torch.randn(256, 2048, generator=g) * 0.02).bfloat16()
    w["w_shg"] = (torch.randn(2048, generator=g) * 0.02).bfloat16()
    experts = {}
    for base in mf.EXPERT_IO:
        e = k.entry(f"{base}{layer}")
        experts[e.name] = torch.randint(0, 256, (e.bytes,), generator=g, dtype=torch.uint8)
    bufs.update(experts)
    m35.store_layer("decode.group", bufs, layer, w)
    b = m35.bind_layer("decode.group", bufs, layer)
    assert b.kind == kind and b.proj_fmt == "mxfp8" and b.mlp_fmt == "mxfp8"
    for n in m35.params[kind]:
        assert _same(b.weights[n], w[n]), n
    for base in mf.EXPERT_IO:
        assert b.weights[base].shape == tuple(k.entry(f"{base}{layer}").shape)
        assert torch.equal(b.weights[base].reshape(-1), experts[f"{base}{layer}"])


def test_bind_reports_missing_and_missized_buffers(m35):
    k = m35.kernel("decode.group")
    bufs = _buffers(k, set(k.packs))
    bufs["ps"] = torch.zeros(100, dtype=torch.uint8)
    with pytest.raises(ValueError, match="ps: 100 bytes"):
        m35.bind_layer("decode.group", bufs, 0)
    with pytest.raises(ValueError, match="layer 9"):
        m35.bind_layer("decode.group", bufs, 9)
    with pytest.raises(ValueError, match="no role"):
        m35.kernel("decode.group16")


def test_state_views():
    conv = torch.arange(2 * 3 * 8192).view(2, 3, 8192)
    cq, ck, cv = mf.gdn_conv_views(conv, 16)
    assert cq.shape == (2, 3, 2048) and ck.shape == (2, 3, 2048) and cv.shape == (2, 3, 4096)
    assert cq[1, 2, 0] == conv[1, 2, 0] and ck[0, 0, 0] == conv[0, 0, 2048] and cv[0, 1, 5] == conv[0, 1, 4101]
    kv = torch.zeros(4, 2, 256, 1024, dtype=torch.bfloat16)
    v = mf.paged_cache_view(kv, 4)
    assert v.shape == (4, 2, 256, 4, 256) and v.data_ptr() == kv.data_ptr()


@pytest.mark.parametrize("path", [M9, M35])
def test_every_manifest_dtype_is_handled_or_rejected_by_name(path):
    """Every (name, dtype) of the committed manifests either has a storage size that matches its declared bytes, or
    (the 35B's code 0 KV-cache outputs, absent from the reference's ONNX dtype table) is rejected with a ValueError that
    names the IO, never a bare KeyError."""
    import json

    with open(path, encoding="utf-8") as f:
        raw = json.load(f)
    seen, rejected = set(), set()

    def walk(o):
        if isinstance(o, dict):
            if "dtype" in o and "name" in o and "shape" in o:
                name, dt, shape = o["name"], int(o["dtype"]), o["shape"]
                seen.add(dt)
                if dt in mf.DT_TORCH:
                    assert mf.storage_bytes(dt, shape, name) == int(o["bytes"]), name
                else:
                    with pytest.raises(ValueError, match=name):
                        mf.storage_bytes(dt, shape, name)
                    with pytest.raises(ValueError, match=name):
                        mf._typed(torch.zeros(int(o["bytes"]), dtype=torch.uint8), dt, shape, name)
                    rejected.add(dt)
            for v in o.values():
                walk(v)
        elif isinstance(o, list):
            for v in o:
                walk(v)

    walk(raw)
    assert seen
    if path == M35:
        assert rejected == {0}
