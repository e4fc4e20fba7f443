"""Pins the per-layer glue oracle (CPU only) against transformers' Qwen3.5 modules and torch's conv1d."""
import pytest
import torch
import torch.nn.functional as F

from oracle import layer, rounding


def _g(seed):
    return torch.Generator().manual_seed(seed)


def test_rmsnorm_matches_transformers_one_plus_rmsnorm():
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5RMSNorm

    g = _g(0)
    x = torch.randn(6, 256, generator=g).bfloat16()
    w_raw = (torch.randn(256, generator=g) * 0.1).bfloat16()
    m = Qwen3_5RMSNorm(256, eps=1e-6)
    m.weight.data = w_raw.float()
    ref = m(x)
    got = layer.rmsnorm(x, 1.0 + w_raw.float(), 1e-6)  # the reference passes one_plus(w) at run time
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


def test_gated_norm_against_transformers_rmsnorm_gated():
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5RMSNormGated

    g = _g(1)
    x = torch.randn(8, 128, generator=g).bfloat16()
    z = torch.randn(8, 128, generator=g).bfloat16()
    m = Qwen3_5RMSNormGated(128, eps=1e-6)
    # unit weight: both round the normalised row to bf16 before the gate -> identical
    assert torch.equal(layer.gated_rmsnorm_silu(x, torch.ones(128), z).view(torch.int16), m(x, z).view(torch.int16))
    # a general weight: the reference multiplies before its bf16 rounding, transformers after -> one rounding apart
    w = torch.rand(128, generator=g) + 0.5
    m.weight.data = w
    torch.testing.assert_close(layer.gated_rmsnorm_silu(x, w, z).float(), m(x, z).float(), rtol=1e-2, atol=1e-2)


def _conv_fp32(x, w, state):
    """Independent formulation: torch depthwise conv1d over [state; x] (PyTorch tap order: last tap = now)."""
    b, t, c = x.shape
    k = w.shape[1]
    seq = torch.cat((state, x), 1).float().transpose(1, 2)  # [B, C, K-1+T]
    w_pt = w.float().flip(-1).reshape(c, 1, k)
    return F.silu(F.conv1d(seq, w_pt, groups=c)).transpose(1, 2)


@pytest.mark.parametrize("b,t,c,k", [(2, 1, 64, 4), (3, 7, 40, 4), (1, 5, 16, 2), (2, 3, 24, 1)])
def test_conv1d_silu_against_torch_conv1d(b, t, c, k):
    g = _g(b * 100 + t)
    x = torch.randn(b, t, c, generator=g).bfloat16()
    w = (torch.randn(c, k, generator=g) * 0.5).bfloat16()
    st = torch.randn(b, k - 1, c, generator=g).bfloat16()
    out, st_out = layer.causal_conv1d_silu(x, w, st)
    torch.testing.assert_close(out.float(), _conv_fp32(x, w, st), rtol=3e-2, atol=2e-2)
    seq = torch.cat((st, x), 1)
    assert torch.equal(st_out, seq[:, seq.shape[1] - (k - 1):])


def test_conv1d_single_tap_is_exact_and_state_carries():
    # only tap 2 nonzero: out_t = silu(bf16(x_{t-2} w)); two calls of 3 tokens == one call of 6
    g = _g(7)
    x = torch.randn(1, 6, 8, generator=g).bfloat16()
    w = torch.zeros(8, 4).bfloat16()
    w[:, 2] = 0.75
    st = torch.randn(1, 3, 8, generator=g).bfloat16()
    out, st6 = layer.causal_conv1d_silu(x, w, st)
    seq = torch.cat((st, x), 1).float()
    want = F.silu((seq[:, 1:7] * 0.75).bfloat16().float()).bfloat16()
    assert torch.equal(out, want)
    o1, s1 = layer.causal_conv1d_silu(x[:, :3], w, st)
    o2, s2 = layer.causal_conv1d_silu(x[:, 3:], w, s1)
    assert torch.equal(torch.cat((o1, o2), 1), out) and torch.equal(s2, st6)


def test_rope_matches_transformers_partial_rotary():
    from transformers.models.qwen3_5.modeling_qwen3_5 import apply_rotary_pos_emb

    g = _g(3)
    b, h, d, rot = 3, 4, 256, 64
    q = torch.randn(b, h, d, generator=g).bfloat16()
    pos = torch.tensor([0, 17, 130000])
    cos, sin = layer.rope_cos_sin(pos, rot, 10_000_000.0)
    got = layer.rope(q, cos, sin, rot)
    # transformers: cos / sin over the full rotary width (both halves), q [B, heads, seq, D]
    cf = torch.cat((cos, cos), -1).float()[:, None, :]
    sf = torch.cat((sin, sin), -1).float()[:, None, :]
    ref, _ = apply_rotary_pos_emb(q.float()[:, :, None, :], q.float()[:, :, None, :], cf, sf, unsqueeze_dim=1)
    assert torch.equal(got.view(torch.int16), ref[:, :, 0, :].bfloat16().view(torch.int16))
    # position 0 is the identity; channels past rot pass through; each rotated pair keeps its length
    assert torch.equal(got[0], q[0])
    assert torch.equal(got[..., rot:], q[..., rot:])
    half = rot // 2
    n_in = q.float()[..., :half] ** 2 + q.float()[..., half:rot] ** 2
    n_out = got.float()[..., :half] ** 2 + got.float()[..., half:rot] ** 2
    torch.testing.assert_close(n_out, n_in, rtol=2e-2, atol=2e-2)


def test_elementwise_gates_special_values():
    x = torch.tensor([[1.5, -2.0, 3.0, 0.25]]).bfloat16()
    zero = torch.zeros_like(x)
    assert torch.equal(layer.sigmoid_mul(x, zero), (x.float() * 0.5).bfloat16())  # sigmoid(0) = 1/2
    assert torch.equal(layer.silu_mul(zero, x), zero)  # silu(0) = 0
    assert torch.equal(layer.add(x, zero), x)
    s, n = layer.add_rmsnorm(x, x, torch.ones(4))
    assert torch.equal(s, (2 * x.float()).bfloat16())
    assert torch.equal(n, layer.rmsnorm(s, torch.ones(4)))


# ---------------------------------------------------------------------------------------------
# Whole decode layers against transformers' Qwen3_5DecoderLayer (fp32, the dequantised weights)
# ---------------------------------------------------------------------------------------------
def _deq_fp8(w, s):
    from oracle import mx

    return torch.from_numpy(mx.e4m3_table()[w.numpy()]) * s.float()[:, None]


def _deq_mx(c, s):
    from oracle import mx

    return torch.from_numpy(mx.dequant_mxfp4(c.numpy(), s.numpy()))


def _hf_layer(kind, w, hidden, inter, **kw):
    """transformers' Qwen3_5DecoderLayer (fp32, eager attention) holding the layer's dequantised weights. The
    kernel contract passes norm weights as 1 + weight (q35_step.py:346-348); transformers adds the 1 itself."""
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5DecoderLayer

    cfg = Qwen3_5TextConfig(hidden_size=hidden, intermediate_size=inter, num_hidden_layers=1, hidden_act="silu",
                            layer_types=[kind], rms_norm_eps=1e-6, **kw)
    cfg._attn_implementation = "eager"
    m = Qwen3_5DecoderLayer(cfg, 0).float().eval()
    with torch.no_grad():
        m.input_layernorm.weight.copy_(w["ln1"] - 1)
        m.post_attention_layernorm.weight.copy_(w["ln2"] - 1)
        m.mlp.gate_proj.weight.copy_(_deq_mx(w["w_gate"], w["s_gate"]))
        m.mlp.up_proj.weight.copy_(_deq_mx(w["w_up"], w["s_up"]))
        m.mlp.down_proj.weight.copy_(_deq_mx(w["w_down"], w["s_down"]))
        if kind == "linear_attention":
            la = m.linear_attn
            la.in_proj_qkv.weight.copy_(_deq_fp8(w["w_qkv"], w["s_qkv"]))
            la.in_proj_z.weight.copy_(_deq_fp8(w["w_z"], w["s_z"]))
            la.in_proj_b.weight.copy_(_deq_fp8(w["w_b"], w["s_b"]))
            la.in_proj_a.weight.copy_(_deq_fp8(w["w_a"], w["s_a"]))
            # column 0 of conv_w multiplies the current token; torch's last tap does
            la.conv1d.weight.copy_(w["conv_w"].float().flip(-1)[:, None, :])
            la.A_log.copy_(w["a_log"])
            la.dt_bias.copy_(w["dt_bias"])
            la.norm.weight.copy_(w["norm_w"])
            la.out_proj.weight.copy_(_deq_fp8(w["w_out"], w["s_out"]))
        else:
            sa = m.self_attn
            sa.q_proj.weight.copy_(_deq_fp8(w["w_q"], w["s_q"]))
            sa.k_proj.weight.copy_(_deq_fp8(w["w_k"], w["s_k"]))
            sa.v_proj.weight.copy_(_deq_fp8(w["w_v"], w["s_v"]))
            sa.o_proj.weight.copy_(_deq_fp8(w["w_o"], w["s_o"]))
            sa.q_norm.weight.copy_(w["q_norm"] - 1)
            sa.k_norm.weight.copy_(w["k_norm"] - 1)
    return m, cfg


def _gdn_decode_tokens(x, w, nk, nv, conv_k=4, v_order="grouped"):
    """The oracle's decode layer applied token by token from zero GDN and conv states (in the checkpoint's value-head
    order by default, the order transformers' layer reads its weights in)."""
    b, t, _ = x.shape
    c = (2 * nk + nv) * 128
    st = torch.zeros(b, nv, 128, 128)
    cv = torch.zeros(b, conv_k - 1, c, dtype=x.dtype)
    outs = []
    for i in range(t):
        o, st, cv = layer.gdn_layer_decode(x[:, i], w, st, cv, nk, nv, v_order=v_order)
        outs.append(o.float())
    return torch.stack(outs, 1), st


@pytest.mark.parametrize("b,t,nk,nv", [(2, 5, 1, 2), (1, 9, 2, 4)])
def test_gdn_layer_decode_matches_transformers_decoder_layer(b, t, nk, nv):
    """q35_step.py gdn_layer (149-183) + mlp_block (118-142) decoded token by token == transformers'
    linear-attention decoder layer over the same tokens (its conv over the window and its chunked delta rule:
    an independent formulation). Pins projection roles (qkv | z | b | a), the conv tap order, the q / k / v
    split and the grouped key heads, the gates, the output norm gated by silu(z), and both residuals."""
    from axk import configs

    hidden, inter = 128, 64
    w = configs.gdn_layer_weights(_g(40 + t), hidden, inter, nk, nv)
    m, _ = _hf_layer("linear_attention", w, hidden, inter, linear_num_key_heads=nk, linear_num_value_heads=nv,
                     linear_key_head_dim=128, linear_value_head_dim=128, linear_conv_kernel_dim=4)
    x = torch.randn(b, t, hidden, generator=_g(41 + t))
    dummy = torch.zeros(b, t, 64)
    with torch.no_grad():
        ref = m(x, position_embeddings=(dummy, dummy))
    with rounding.fp32():
        got, _ = _gdn_decode_tokens(x, w, nk, nv)
    torch.testing.assert_close(got, ref, rtol=1e-4, atol=1e-4)
    # the reference's bf16 points keep the composed layer within the fused-layer bar (test_gdn_attn.py:354)
    got_bf, _ = _gdn_decode_tokens(x.bfloat16(), w, nk, nv)
    torch.testing.assert_close(got_bf, ref, rtol=5e-2, atol=0.0625)
    # slips that the pin must catch: z gate off, conv taps in torch order, value heads paired with the other key head
    for name, bad_w in (("z", dict(w, w_z=torch.zeros_like(w["w_z"]))),
                        ("conv", dict(w, conv_w=w["conv_w"].flip(-1).contiguous()))):
        with rounding.fp32():
            bad, _ = _gdn_decode_tokens(x, bad_w, nk, nv)
        assert not torch.allclose(bad, ref, rtol=1e-3, atol=1e-3), name
    if nv > 1 and nk > 1:  # the tiled pairing on checkpoint-order weights
        with rounding.fp32():
            bad, _ = _gdn_decode_tokens(x, w, nk, nv, v_order="tiled")
        assert not torch.allclose(bad, ref, rtol=1e-3, atol=1e-3), "v_order"


def _attn_decode_tokens(x, w, hq, hkv, d, rot, theta, page, g):
    """The oracle's attention decode layer, token by token, over a paged cache that grows by one token per step
    (pages drawn from a shuffled pool, the new token's page appended when it starts)."""
    from oracle import paged_attn  # noqa: F401  (the layer oracle calls it)

    b, t, _ = x.shape
    pages_per_seq = -(-t // page)
    pool = torch.randperm(b * pages_per_seq + 3, generator=g).to(torch.int32)
    cache = torch.randn(pool.numel() + 1, 2, page, hkv, d, generator=g)  # garbage beyond the written rows
    cache = cache.to(x.dtype)
    inv = 1.0 / (theta ** (torch.arange(0, rot, 2, dtype=torch.int64).float() / rot))
    outs = []
    for i in range(t):
        npg = i // page + 1
        indices = torch.cat([pool[s * pages_per_seq: s * pages_per_seq + npg] for s in range(b)])
        indptr = torch.arange(0, b * npg + 1, npg, dtype=torch.int32)
        lpl = torch.full((b,), i % page + 1, dtype=torch.int32)
        loc = torch.tensor([[int(pool[s * pages_per_seq + npg - 1]), i % page] for s in range(b)], dtype=torch.int32)
        f = torch.full((b, 1), float(i)) * inv[None, :]
        cos, sin = rounding.bf(f.cos()), rounding.bf(f.sin())
        o, cache = layer.attn_layer_decode(x[:, i], w, cos, sin, cache, indptr, indices, lpl, loc, hq, rot)
        outs.append(o.float())
    return torch.stack(outs, 1)


@pytest.mark.parametrize("b,t,hq,hkv,page", [(2, 7, 4, 2, 4), (1, 11, 6, 2, 8)])
def test_attn_layer_decode_matches_transformers_decoder_layer(b, t, hq, hkv, page):
    """q35_step.py attn_block (186-293) + mlp_block decoded token by token over the paged cache == transformers'
    full-attention decoder layer with a causal mask over the same tokens. Pins the per-head [q | gate] split of
    the q projection, the (1 + w) q / k norms, partial NeoX RoPE (64 of 256 channels) at each position, GQA
    grouping, the sigmoid output gate, the paged KV write / read and both residuals."""
    from axk import configs

    hidden, inter, d, rot, theta = 128, 64, 256, 64, 10_000_000.0
    w = configs.attn_layer_weights(_g(50 + t), hidden, inter, hq, hkv, d)
    m, cfg = _hf_layer("full_attention", w, hidden, inter, num_attention_heads=hq, num_key_value_heads=hkv,
                       head_dim=d, rope_parameters={"rope_type": "default", "rope_theta": theta,
                                                    "partial_rotary_factor": rot / d})
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5TextRotaryEmbedding

    x = torch.randn(b, t, hidden, generator=_g(51 + t))
    pos = torch.arange(t)[None].expand(b, t)
    cos, sin = Qwen3_5TextRotaryEmbedding(cfg)(x, pos)
    mask = torch.full((t, t), float("-inf")).triu(1)[None, None].expand(b, 1, t, t)
    with torch.no_grad():
        ref = m(x, position_embeddings=(cos, sin), attention_mask=mask)
    with rounding.fp32():
        got = _attn_decode_tokens(x, w, hq, hkv, d, rot, theta, page, _g(52))
    torch.testing.assert_close(got, ref, rtol=1e-4, atol=1e-4)
    got_bf = _attn_decode_tokens(x.bfloat16(), w, hq, hkv, d, rot, theta, page, _g(52))
    torch.testing.assert_close(got_bf, ref, rtol=5e-2, atol=0.0625)
    # slips the pin must catch: [gate | q] instead of [q | gate], RoPE on the wrong channels (no rotation)
    q = w["w_q"].reshape(hq, 2, d, hidden)
    for name, bad_w, bad_rot in (("gate order", dict(w, w_q=q.flip(1).reshape(hq * 2 * d, hidden),
                                                     s_q=w["s_q"].reshape(hq, 2, d).flip(1).reshape(-1)), rot),
                                 ("no rope", w, 0)):
        with rounding.fp32():
            bad = _attn_decode_tokens(x, bad_w, hq, hkv, d, bad_rot, theta, page, _g(52))
        assert not torch.allclose(bad, ref, rtol=1e-3, atol=1e-3), name


def test_attn_verify_oracle_is_causal_and_one_row_is_a_decode_step():
    """attn_layer_verify's per-row page-table prefixes: row t sees the history and rows 0 .. t only (changing later
    rows leaves it unchanged, changing an earlier row moves it), and a single row is exactly one decode step."""
    from axk import configs

    g = torch.Generator().manual_seed(4)
    hq, hkv, d, page, H, F = 4, 2, 64, 16, 128, 128
    w = configs.attn_layer_weights(g, H, F, hq, hkv, d)
    c = configs.verify_rows_case([20, 15], 3, hq, hkv, d, page, g)  # the second sequence's rows cross a page
    x = torch.randn(2, 3, H, generator=g).bfloat16()
    cos, sin = layer.rope_cos_sin(c["pos"].reshape(-1), 32, 10_000_000.0)
    cos, sin = cos.reshape(2, 3, -1), sin.reshape(2, 3, -1)
    args = (c["indptr"], c["indices"], c["last_page_len"], c["loc"], hq, 32)
    out, _ = layer.attn_layer_verify(x, w, cos, sin, c["cache"], *args)
    x2 = x.clone()
    x2[:, 2] = torch.randn(2, H, generator=g).bfloat16()
    out2, _ = layer.attn_layer_verify(x2, w, cos, sin, c["cache"], *args)
    assert torch.equal(out[:, :2], out2[:, :2]) and not torch.equal(out[:, 2], out2[:, 2])
    x3 = x.clone()
    x3[:, 0] = torch.randn(2, H, generator=g).bfloat16()
    out3, _ = layer.attn_layer_verify(x3, w, cos, sin, c["cache"], *args)
    assert not torch.equal(out[:, 1], out3[:, 1])  # row 1 attends row 0's K / V
    c1 = configs.verify_rows_case([20, 15], 1, hq, hkv, d, page, torch.Generator().manual_seed(4))
    one, _ = layer.attn_layer_verify(x[:, :1], w, cos[:, :1], sin[:, :1], c1["cache"], c1["indptr"], c1["indices"],
                                     c1["last_page_len"], c1["loc"], hq, 32)
    dec, _ = layer.attn_layer_decode(x[:, 0], w, cos[:, 0], sin[:, 0], c1["cache"], c1["indptr"], c1["indices"],
                                     c1["last_page_len"], c1["loc"][:, 0], hq, 32)
    assert torch.equal(one[:, 0], dec)


@pytest.mark.parametrize("t,chunk", [(7, 64), (20, 8), (21, 4)])
def test_gdn_prefill_oracle_equals_decode_steps(t, chunk):
    """gdn_layer_prefill (the chunked delta rule over T tokens, conv over the tokens) equals T decode steps of the
    layer (the recurrent form, pinned to transformers' decoder layer) in fp32 arithmetic, for one chunk and for
    several chunks with a ragged last one; and the bf16 schedule stays within the fused bar of it."""
    from axk import configs

    g = torch.Generator().manual_seed(t)
    w = configs.gdn_layer_weights(g, 128, 128, 1, 2)
    x = torch.randn(2, t, 128, generator=g).bfloat16()
    st = torch.randn(2, 2, 128, 128, generator=g) * 0.02
    cv = torch.randn(2, 3, 512, generator=g).bfloat16()
    with rounding.fp32():
        po, ps, pc = layer.gdn_layer_prefill(x, w, st, cv, 1, 2, chunk=chunk)
        ro, rs, rc, _, _ = layer.gdn_layer_verify(x, w, st, cv, 1, 2)
    torch.testing.assert_close(po.float(), ro.float(), rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(ps, rs, rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(pc, rc, rtol=1e-5, atol=1e-6)  # fp32 products over B T rows vs B rows
    bo, bs, _ = layer.gdn_layer_prefill(x, w, st, cv, 1, 2, chunk=chunk)
    torch.testing.assert_close(bo.float(), ro.float(), rtol=5e-2, atol=0.0625)
    torch.testing.assert_close(bs, rs, rtol=5e-2, atol=3e-3)


@pytest.mark.parametrize("fmt", ["fp8", "mxfp8", "mxfp4"])
def test_tiled_value_heads_on_tiled_weights_equal_the_grouped_layer(fmt):
    """The tiled value-head order (q35_step.py:82-85, the reference's layer default) on weights converted as its
    loader converts them (axk.layer.tile_value_heads, q35_step.py v_tiled 351-358) computes the grouped layer on the
    checkpoint's weights: the same outputs (the output projection sums the value heads in another order) and the
    same states with their value heads permuted; decode and chunked prefill."""
    from axk import configs
    from axk.layer import tile_value_heads, v_tiled

    nk, nv, h = 2, 6, 128
    g = torch.Generator().manual_seed(31)
    w = configs.gdn_layer_weights(g, h, 128, nk, nv, proj_fmt=fmt)
    wt = tile_value_heads(w, nk, nv, fmt)
    x = torch.randn(2, 5, h, generator=g).bfloat16()
    st = torch.randn(2, nv, 128, 128, generator=g) * 0.02
    cv = torch.randn(2, 3, (2 * nk + nv) * 128, generator=g).bfloat16()
    kd = 2 * nk * 128
    cvt = torch.cat((cv[..., :kd], v_tiled(cv[..., kd:], 2, nk, nv, 128)), -1)
    stt = v_tiled(st, 1, nk, nv, 1)
    with rounding.fp32():
        o_g, s_g, c_g = layer.gdn_layer_decode(x[:, 0], w, st, cv, nk, nv, proj_fmt=fmt, v_order="grouped")
        o_t, s_t, c_t = layer.gdn_layer_decode(x[:, 0], wt, stt, cvt, nk, nv, proj_fmt=fmt, v_order="tiled")
        p_g, ps_g, _ = layer.gdn_layer_prefill(x, w, st, cv, nk, nv, proj_fmt=fmt, chunk=2, v_order="grouped")
        p_t, ps_t, _ = layer.gdn_layer_prefill(x, wt, stt, cvt, nk, nv, proj_fmt=fmt, chunk=2, v_order="tiled")
    torch.testing.assert_close(o_t, o_g, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(s_t, v_tiled(s_g, 1, nk, nv, 1), rtol=1e-6, atol=1e-7)
    torch.testing.assert_close(c_t, torch.cat((c_g[..., :kd], v_tiled(c_g[..., kd:], 2, nk, nv, 128)), -1),
                               rtol=1e-6, atol=1e-7)
    torch.testing.assert_close(p_t, p_g, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(ps_t, v_tiled(ps_g, 1, nk, nv, 1), rtol=1e-6, atol=1e-7)
    # and the orders differ: the tiled pairing on the checkpoint's weights is another layer
    with rounding.fp32():
        o_x, _, _ = layer.gdn_layer_decode(x[:, 0], w, st, cv, nk, nv, proj_fmt=fmt, v_order="tiled")
    assert not torch.allclose(o_x, o_g, rtol=1e-3, atol=1e-3)


def test_v_tiled_is_the_reference_permutation():
    """v_tiled: value head (vo, kh) of the result is head (kh, vo) of the input, i.e. tiled head vh = vo * NK + kh
    holds grouped head kh * (NV / NK) + vo (q35_step.py:171); identity for NV == NK."""
    from axk.layer import v_tiled

    nk, nv = 3, 12
    t = torch.arange(nv * 2).reshape(nv * 2, 1)
    r = v_tiled(t, 0, nk, nv, 2).reshape(nv, 2)
    for vh in range(nv):
        vo, kh = divmod(vh, nk)
        assert r[vh, 0] == 2 * (kh * (nv // nk) + vo)
    assert torch.equal(v_tiled(t[:6], 0, 3, 3, 2), t[:6])


def test_attn_rows_half_is_the_verify_layer_before_its_mlp():
    """attn_rows_half (the MoE prefill layer's first half) then the MLP residual is attn_layer_verify, exactly."""
    from axk import configs

    g = torch.Generator().manual_seed(8)
    hq, hkv, d, page, H, F = 4, 2, 64, 16, 128, 128
    w = configs.attn_layer_weights(g, H, F, hq, hkv, d)
    c = configs.verify_rows_case([20, 15], 3, hq, hkv, d, page, g)
    x = torch.randn(2, 3, H, generator=g).bfloat16()
    cos, sin = layer.rope_cos_sin(c["pos"].reshape(-1), 32, 10_000_000.0)
    cos, sin = cos.reshape(2, 3, -1), sin.reshape(2, 3, -1)
    args = (c["indptr"], c["indices"], c["last_page_len"], c["loc"], hq, 32)
    out, cache = layer.attn_layer_verify(x, w, cos, sin, c["cache"], *args)
    y, cache2 = layer.attn_rows_half(x, w, cos, sin, c["cache"], *args)
    assert torch.equal(layer.mlp_residual(x.reshape(6, H), y, w, 1e-6).reshape(2, 3, H), out)
    assert torch.equal(cache, cache2)


# ---- the MoE block of the MoE decode layers (moe_full, q35_layer_mc.py:797-853) ----
@pytest.mark.parametrize("fmt", ["fp8", "mxfp8", "mxfp4"])
def test_dequant_weight_is_what_proj_multiplies(fmt):
    """dequant_weight(w, name, fmt) is the weight proj() multiplies (the shared expert's down projection uses it
    unrounded)."""
    from axk import configs

    g = _g(40)
    w = configs.mlp_weights(g, 64, 96, fmt)
    a = torch.randn(5, 96, generator=g).bfloat16()
    ref = layer.proj(a, w, "down", fmt).float()
    got = (a.float() @ layer.dequant_weight(w, "down", fmt).T).bfloat16().float()
    torch.testing.assert_close(got, ref, rtol=1e-6, atol=1e-6)


def _moe_case(seed, fmt="mxfp4"):
    from axk import configs

    g = _g(seed)
    h, f, e, fe, k, b = 64, 96, 8, 32, 3, 5
    w = configs.mlp_weights(g, h, f, fmt)
    w["ln2"] = 1.0 + 0.1 * torch.randn(h, generator=g)
    blk = configs.moe_block(g, h, e, fe, k, router_std=0.2)
    x = torch.randn(b, h, generator=g).bfloat16()
    y = torch.randn(b, h, generator=g).bfloat16()
    return w, blk, x, y


def test_moe_block_with_an_mxfp4_shared_expert_equals_the_moe_oracle():
    """With the shared expert in MXFP4 the block is oracle.moe.moe_layer (pinned against transformers'
    Qwen3_5MoeSparseMoeBlock) on h2 = rmsnorm(x1, ln2) with x1 as the residual: the same routing, and the same
    output with base kept fp32."""
    from oracle import moe as omoe

    w, blk, x, y = _moe_case(41)
    base, routed, slack, logits, ids, wts = layer.moe_block_parts(x, y, w, blk, fmt="mxfp4")
    x1, h2 = layer.add_rmsnorm(x, y, w["ln2"])
    mw = dict(blk, **{n: w[n] for n in ("w_gate", "s_gate", "w_up", "s_up", "w_down", "s_down")})
    ref, rlogits, rids, rwts = omoe.moe_layer(h2, mw, top_k=blk["top_k"], x_res=x1, round_base=False)
    assert torch.equal(ids, rids)
    torch.testing.assert_close(wts, rwts, rtol=0, atol=0)
    torch.testing.assert_close(logits, rlogits, rtol=0, atol=0)
    torch.testing.assert_close((base + routed).bfloat16().float(), ref.float(), rtol=1e-6, atol=1e-6)
    assert (slack > 0).all()


def test_moe_block_pin_detects_plausible_slips():
    """The comparison above fails for a gate / up swap in the shared expert and for a dropped shared gate."""
    from oracle import moe as omoe

    w, blk, x, y = _moe_case(42)
    x1, h2 = layer.add_rmsnorm(x, y, w["ln2"])
    mw = dict(blk, **{n: w[n] for n in ("w_gate", "s_gate", "w_up", "s_up", "w_down", "s_down")})
    ref = omoe.moe_layer(h2, mw, top_k=blk["top_k"], x_res=x1, round_base=False)[0].float()
    swapped = dict(w, w_gate=w["w_up"], s_gate=w["s_up"], w_up=w["w_gate"], s_up=w["s_gate"])
    base, routed, *_ = layer.moe_block_parts(x, y, swapped, blk, fmt="mxfp4")
    assert not torch.allclose((base + routed).bfloat16().float(), ref, rtol=2e-2, atol=1e-2)
    base, routed, *_ = layer.moe_block_parts(x, y, w, dict(blk, w_shg=None), fmt="mxfp4")
    assert not torch.allclose((base + routed).bfloat16().float(), ref, rtol=2e-2, atol=1e-2)
