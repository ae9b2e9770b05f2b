"""Pins of the Qwen3 oracle (CPU): closed forms and invariants of RMSNorm and
RoPE, attention against torch's scaled_dot_product_attention, prefill against
step-by-step decode, and the whole decoder against the transformers library's
Qwen3 implementation loaded with the same (dequantised) weights.
"""

import math

import numpy as np
import pytest
import torch

from oracle import qwen3 as oq
from oracle import w4a16 as ow
from torch2iron_amd import model as gm

F32 = oq._Round("fp32")
B16 = oq._Round("bf16")


def test_rmsnorm_closed_forms():
    w = torch.linspace(0.9, 1.1, 64)
    c = torch.full((2, 64), 3.0)
    out = oq.rmsnorm(c, w, 1e-6, F32)
    assert torch.allclose(out, w.expand(2, 64) * 3.0 / math.sqrt(9.0 + 1e-6), rtol=1e-6)
    x = torch.randn(5, 64, generator=torch.Generator().manual_seed(0))
    assert torch.allclose(oq.rmsnorm(7.0 * x, w, 0.0, F32), oq.rmsnorm(x, w, 0.0, F32), rtol=1e-5, atol=1e-6)
    # bf16 mode only rounds (three roundings of at most 2^-9 each): close to the fp32 result
    assert ((oq.rmsnorm(x, w, 1e-6, B16) - oq.rmsnorm(x, w, 1e-6, F32)).abs()
            <= 3 * 2.0 ** -8 * oq.rmsnorm(x, w, 1e-6, F32).abs() + 1e-6).all()


@pytest.mark.parametrize("style", ["halves", "interleaved"])
def test_rope_invariants(style):
    d = 128
    ang = oq.rope_angles(d, 512, 1e6)
    g = torch.Generator().manual_seed(1)
    q, k = torch.randn(d, generator=g), torch.randn(d, generator=g)
    # position 0 is the identity
    assert torch.equal(oq.apply_rope(q, ang[0], style, F32), q)
    # each rotated pair keeps its norm
    r = oq.apply_rope(q, ang[77], style, F32)
    if style == "halves":
        pairs_in = q[:64] ** 2 + q[64:] ** 2
        pairs_out = r[:64] ** 2 + r[64:] ** 2
    else:
        pairs_in = q[0::2] ** 2 + q[1::2] ** 2
        pairs_out = r[0::2] ** 2 + r[1::2] ** 2
    assert torch.allclose(pairs_in, pairs_out, rtol=1e-5)
    # relative positions: <rope(q, p1), rope(k, p2)> depends on p1 - p2 only
    dots = [torch.dot(oq.apply_rope(q, ang[p + 40], style, F32), oq.apply_rope(k, ang[p], style, F32))
            for p in (0, 100, 300)]
    assert max(dots) - min(dots) < 1e-3 * abs(dots[0]) + 1e-4


def test_rope_styles_are_the_same_rotation_up_to_a_permutation():
    d = 128
    perm = torch.empty(d, dtype=torch.long)       # halves index -> interleaved index
    perm[:64] = torch.arange(0, d, 2)
    perm[64:] = torch.arange(1, d, 2)
    ang = oq.rope_angles(d, 64, 1e6)
    x = torch.randn(3, d, generator=torch.Generator().manual_seed(2))
    xi = torch.empty_like(x)
    xi[:, perm] = x
    a = oq.apply_rope(x, ang[33], "halves", F32)
    b = oq.apply_rope(xi, ang[33], "interleaved", F32)
    assert torch.allclose(b[:, perm], a, atol=1e-6)


def test_decode_attention_matches_sdpa_and_special_cases():
    b, h, hkv, n, d = 2, 8, 2, 37, 128
    g = torch.Generator().manual_seed(3)
    q = torch.randn(b, h, d, generator=g)
    kc = torch.randn(b, hkv, 64, d, generator=g)
    vc = torch.randn(b, hkv, 64, d, generator=g)
    lengths = torch.tensor([n, 64])
    out = oq.decode_attention(q, kc, vc, lengths, hkv)
    for i in range(b):
        L = int(lengths[i])
        k = kc[i, :, :L].repeat_interleave(h // hkv, dim=0)
        v = vc[i, :, :L].repeat_interleave(h // hkv, dim=0)
        ref = torch.nn.functional.scaled_dot_product_attention(q[i][:, None], k, v)[:, 0]
        assert torch.allclose(out[i], ref, atol=1e-5, rtol=1e-5)
    # a single key returns its value; a zero query averages the values
    one = oq.decode_attention(q, kc, vc, torch.tensor([1, 1]), hkv)
    assert torch.allclose(one[0, 0], vc[0, 0, 0], atol=1e-6)
    zero = oq.decode_attention(torch.zeros_like(q), kc, vc, lengths, hkv)
    assert torch.allclose(zero[0, 0], vc[0, 0, :n].mean(0), atol=1e-5)


def _tiny():
    cfg = gm.Qwen3Config(hidden=256, n_heads=4, n_kv_heads=2, head_dim=128, intermediate=512, n_layers=2,
                         vocab=1000)
    ocfg = oq.Qwen3Config(**{k: getattr(cfg, k) for k in oq.Qwen3Config.__dataclass_fields__})
    return cfg, ocfg, gm.random_qwen3_tensors(cfg, seed=4, weights="centered")


def test_prefill_equals_stepwise_decode():
    cfg, ocfg, t = _tiny()
    prompt = torch.randint(0, cfg.vocab, (2, 9), generator=torch.Generator().manual_seed(5))
    m = oq.DenseQwen3(t, ocfg, mode="fp32", ctx_cap=32)
    full = m.prefill(prompt)
    m2 = oq.DenseQwen3(t, ocfg, mode="fp32", ctx_cap=32)
    m2.prefill(prompt[:, :1])
    for j in range(1, 9):
        last = m2.decode_step(prompt[:, j], torch.full((2,), j, dtype=torch.long))
    assert torch.allclose(full, last, rtol=1e-4, atol=1e-3 * full.abs().max())


@pytest.mark.parametrize("tied", [True, False])
def test_decoder_matches_transformers_qwen3(tied):
    """The oracle (fp32 mode, two-halves RoPE) against transformers' Qwen3ForCausalLM
    holding the same dequantised weights, with the tied embedding as lm_head or a
    separate lm_head matrix."""
    transformers = pytest.importorskip("transformers")
    cfg, ocfg, t = _tiny()
    if not tied:
        t = dict(t)
        t["lm_head.weight"] = (torch.randn(cfg.vocab, cfg.hidden, generator=torch.Generator().manual_seed(9))
                               .to(torch.bfloat16).float().numpy())
    hf_cfg = transformers.Qwen3Config(
        vocab_size=cfg.vocab, hidden_size=cfg.hidden, intermediate_size=cfg.intermediate,
        num_hidden_layers=cfg.n_layers, num_attention_heads=cfg.n_heads, num_key_value_heads=cfg.n_kv_heads,
        head_dim=cfg.head_dim, rms_norm_eps=cfg.eps, tie_word_embeddings=tied, max_position_embeddings=64,
        rope_parameters={"rope_theta": cfg.rope_theta, "rope_type": "default"}, attention_bias=False)
    torch.manual_seed(0)
    hf = transformers.Qwen3ForCausalLM(hf_cfg).float().eval()
    sd = {}
    for name in list(t):
        if name.endswith(".qweight"):
            base = name[:-len(".qweight")]
            sd[base + ".weight"] = torch.from_numpy(
                ow.dequantize(t[base + ".qweight"], t[base + ".qzeros"], t[base + ".scales"]))
        elif name.endswith(".weight"):
            sd[name] = torch.as_tensor(np.asarray(t[name], dtype=np.float32))
    if tied:
        sd["lm_head.weight"] = sd["model.embed_tokens.weight"]
    missing, unexpected = hf.load_state_dict(sd, strict=False)
    assert not unexpected and all("rotary" in m for m in missing), (missing, unexpected)
    prompt = torch.randint(0, cfg.vocab, (2, 11), generator=torch.Generator().manual_seed(6))
    with torch.no_grad():
        ref = hf(input_ids=prompt).logits[:, -1, :].float()
    ours = oq.DenseQwen3(t, ocfg, mode="fp32", ctx_cap=32).prefill(prompt)
    assert torch.allclose(ours, ref, rtol=1e-4, atol=1e-3 * ref.abs().max()), (ours - ref).abs().max()
    assert torch.equal(torch.argmax(ours, -1), torch.argmax(ref, -1))


# ---- the bf16 mode against the same formulas run natively in torch.bfloat16 ----
# ``quantized_qwen3/model.py`` with ``compute_dtype=torch.bfloat16`` keeps every
# activation as a bf16 tensor; each torch op then rounds its result to bf16.  The
# oracle's bf16 mode holds bf16 values in fp32 tensors and rounds explicitly; these
# tests run the reference's formulas on bf16 tensors and require the same bits.

BF = torch.bfloat16


def _bf16_randn(*shape, seed=0, scale=1.0):
    return (torch.randn(*shape, generator=torch.Generator().manual_seed(seed)) * scale).to(BF)


@pytest.mark.parametrize("shape", [(4, 1024), (3, 16, 128), (2, 8, 128), (1, 2048)])
def test_bf16_rmsnorm_matches_native_bfloat16(shape):
    """``model.py:176-179``: variance in fp32, rsqrt cast to bf16, two bf16 products."""
    x = _bf16_randn(*shape, seed=shape[-1], scale=3.0)
    w = (torch.rand(shape[-1], generator=torch.Generator().manual_seed(7)) * 0.2 + 0.9).to(BF)
    variance = x.to(torch.float32).pow(2).mean(dim=-1, keepdim=True)
    native = (x * torch.rsqrt(variance + 1e-6).to(x.dtype)) * w
    got = oq.rmsnorm(x.float(), w.float(), 1e-6, B16)
    assert torch.equal(got.to(BF), native)


def test_bf16_rope_interleaved_matches_native_bfloat16():
    """``model.py:184-196``: x * cos + rotate_half(x) * sin, each product and the sum in bf16."""
    d, n = 128, 40
    ang = oq.rope_angles(d, 600, 1e6)
    pos = torch.arange(0, 600, 15)[:n]
    x = _bf16_randn(n, 16, d, seed=3)
    a = ang[pos].to(BF)[:, None, :]                  # the bf16 table (model.py:421-425)
    cos = a[..., ::2].repeat_interleave(2, dim=-1)
    sin = a[..., 1::2].repeat_interleave(2, dim=-1)
    rot = torch.stack((-x[..., 1::2], x[..., ::2]), dim=-1).flatten(-2)
    native = x * cos + rot * sin
    got = oq.apply_rope(x.float(), a.float(), "interleaved", B16)
    assert torch.equal(got.to(BF), native)


def test_bf16_rope_halves_matches_native_bfloat16():
    """The (i, i + d/2) pairing of ``rms_norm_rope/kernel.cc:39-67``, written as the
    same bf16 products and sum."""
    d, n = 128, 40
    ang = oq.rope_angles(d, 600, 1e6)
    pos = torch.arange(0, 600, 15)[:n]
    x = _bf16_randn(n, 8, d, seed=4)
    a = ang[pos].to(BF)[:, None, :]
    cos = torch.cat((a[..., ::2], a[..., ::2]), dim=-1)
    sin = torch.cat((a[..., 1::2], a[..., 1::2]), dim=-1)
    rot = torch.cat((-x[..., d // 2:], x[..., :d // 2]), dim=-1)
    native = x * cos + rot * sin
    got = oq.apply_rope(x.float(), a.float(), "halves", B16)
    assert torch.equal(got.to(BF), native)


def test_bf16_swiglu_and_residual_match_native_bfloat16():
    """``model.py:215-216, 322-327``: silu(gate) * up and the residual adds, each op in bf16."""
    g = _bf16_randn(6, 3072, seed=5, scale=4.0)
    u = _bf16_randn(6, 3072, seed=6, scale=2.0)
    native = torch.nn.functional.silu(g) * u
    got = oq._bf(oq._bf(oq.silu(g.float())) * u.float())
    assert torch.equal(got.to(BF), native)
    r = _bf16_randn(6, 1024, seed=8, scale=30.0)
    o = _bf16_randn(6, 1024, seed=9, scale=0.5)
    assert torch.equal(oq._bf(r.float() + o.float()).to(BF), r + o)


def test_bf16_layer_matches_native_bfloat16_layer():
    """One decode-free layer pass (RMSNorm, projections, q/k-norm, RoPE, causal
    attention, o_proj + residual, RMSNorm, SwiGLU MLP + residual) of the oracle's
    bf16 mode against the same layer written natively in bf16 torch ops, with the
    linears as fp32 matmuls of the exact weights cast back to bf16
    (``model.py:133-146``) and fp32 softmax weights (the oracle's stated departure
    from ``model.py:277``)."""
    cfg = oq.Qwen3Config(hidden=256, n_heads=4, n_kv_heads=2, head_dim=128, intermediate=512, n_layers=1,
                         vocab=64, rope_style="interleaved")
    gcfg = gm.Qwen3Config(**{k: getattr(cfg, k) for k in oq.Qwen3Config.__dataclass_fields__})
    t = gm.random_qwen3_tensors(gcfg, seed=12, weights="centered")
    layer = oq.DenseLayer(t, "model.layers.0", cfg)
    b, n = 2, 9
    x = _bf16_randn(b, n, cfg.hidden, seed=13)
    ang = oq.rope_angles(cfg.head_dim, 64, cfg.rope_theta)
    kc = torch.zeros(b, cfg.n_kv_heads, 64, cfg.head_dim)
    vc = torch.zeros_like(kc)
    got = layer.prefill(x.float(), kc, vc, ang, B16)

    def lin(name, h):
        return (h.float() @ layer.w[name].T).to(BF)

    def norm(h, w):
        var = h.float().pow(2).mean(dim=-1, keepdim=True)
        return (h * torch.rsqrt(var + cfg.eps).to(BF)) * w.to(BF)

    def rope(h):
        a = ang[:n].to(BF)[None, None]
        cos = a[..., ::2].repeat_interleave(2, dim=-1)
        sin = a[..., 1::2].repeat_interleave(2, dim=-1)
        rot = torch.stack((-h[..., 1::2], h[..., ::2]), dim=-1).flatten(-2)
        return h * cos + rot * sin

    xn = norm(x, layer.ln1)
    q = lin("q_proj", xn).view(b, n, cfg.n_heads, cfg.head_dim).transpose(1, 2)
    k = lin("k_proj", xn).view(b, n, cfg.n_kv_heads, cfg.head_dim).transpose(1, 2)
    v = lin("v_proj", xn).view(b, n, cfg.n_kv_heads, cfg.head_dim).transpose(1, 2)
    q = rope(norm(q, layer.q_norm))
    k = rope(norm(k, layer.k_norm))
    kk = k.float().repeat_interleave(2, dim=1)
    vv = v.float().repeat_interleave(2, dim=1)
    s = (q.float() @ kk.transpose(-2, -1)) * cfg.head_dim ** -0.5
    s = s.masked_fill(~torch.ones(n, n, dtype=torch.bool).tril(), torch.finfo(torch.float32).min)
    ctx = (torch.softmax(s, dim=-1) @ vv).to(BF).transpose(1, 2).reshape(b, n, -1)
    h = x + lin("o_proj", ctx)
    hn = norm(h, layer.ln2)
    mlp = torch.nn.functional.silu(lin("gate_proj", hn)) * lin("up_proj", hn)
    native = h + lin("down_proj", mlp)
    assert torch.equal(got.to(BF), native)
