"""Prompt (prefill) path on the MI355X vs the CPU oracle.

Bars: q/k norm + RoPE and the KV-cache rows within one bf16 ulp of the oracle's
bf16 chain (v bit-exact); the causal attention within 1e-2 max relative error,
and elementwise within 2^-8 (sum_j p_j |v_j| + |out|): the softmax weights
enter P . V as bf16 and the output is bf16; the model's prompt pass picks the
oracle's first token except at near-ties, and its KV cache matches the
oracle's within the bf16 rounding of a head vector.
"""

import math

import numpy as np
import pytest
import torch

from oracle import qwen3 as oq
from torch2iron_amd import model as gm
from torch2iron_amd import ops

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16


def _bf(t):
    return t.to(BF16).float()


def ulp_diff(a: torch.Tensor, b: torch.Tensor):
    ai = a.to(BF16).view(torch.int16).to(torch.int32)
    bi = b.to(BF16).view(torch.int16).to(torch.int32)
    d = (ai - bi).abs()
    return (d > 0).float().mean().item(), d.max().item()


def _case(gpu, b, t, p0, hq, hkv, cap, style, seed):
    d = 128
    g = torch.Generator().manual_seed(seed)
    qkv = torch.randn(b * t, (hq + 2 * hkv) * d, generator=g).to(BF16)
    kc = torch.randn(b, hkv, cap, d, generator=g).to(BF16)        # slots < p0: an earlier prompt chunk
    vc = torch.randn(b, hkv, cap, d, generator=g).to(BF16)
    qn = (torch.rand(d, generator=g) * 0.2 + 0.9).to(BF16)
    kn = (torch.rand(d, generator=g) * 0.2 + 0.9).to(BF16)
    rope = gm.rope_table(d, cap, 1e6, "cpu")
    # oracle
    rnd = oq._Round("bf16")
    cs = oq.rope_angles(d, cap, 1e6)[p0:p0 + t].repeat(b, 1)                  # row b*t + i -> position p0 + i
    q = qkv[:, :hq * d].float().view(b * t, hq, d)
    k = qkv[:, hq * d:(hq + hkv) * d].float().view(b * t, hkv, d)
    v = qkv[:, (hq + hkv) * d:].float().view(b * t, hkv, d)
    q = oq.apply_rope(oq.rmsnorm(q, qn.float(), 1e-6, rnd), cs[:, None, :], style, rnd)
    k = oq.apply_rope(oq.rmsnorm(k, kn.float(), 1e-6, rnd), cs[:, None, :], style, rnd)
    kref, vref = kc.float().clone(), vc.float().clone()
    kref[:, :, p0:p0 + t] = k.view(b, t, hkv, d).transpose(1, 2)
    vref[:, :, p0:p0 + t] = v.view(b, t, hkv, d).transpose(1, 2)
    qb = q.view(b, t, hq, d).transpose(1, 2)                                    # [B, Hq, T, D]
    group = hq // hkv
    ref = torch.empty(b, t, hq, d)
    mag = torch.empty(b, t, hq, d)         # sum_j p_j |v_j|: scale of the bf16 rounding of the weights
    for i in range(b):
        keys = kref[i, :, :p0 + t].repeat_interleave(group, dim=0)             # [Hq, L, D]
        vals = vref[i, :, :p0 + t].repeat_interleave(group, dim=0)
        sc = torch.matmul(qb[i], keys.transpose(-2, -1)) / math.sqrt(d)         # [Hq, T, L]
        mask = torch.arange(p0 + t)[None, :] <= (p0 + torch.arange(t))[:, None]
        sc = sc.masked_fill(~mask, float("-inf"))
        pr = torch.softmax(sc, dim=-1)
        ref[i] = torch.matmul(pr, vals).transpose(0, 1)
        mag[i] = torch.matmul(pr, vals.abs()).transpose(0, 1)
    ref = ref.reshape(b * t, hq * d)
    mag = mag.reshape(b * t, hq * d)
    # GPU
    kd, vd = kc.to(gpu), vc.to(gpu)
    qd = ops.prefill_qk_rope_kv(qkv.to(gpu), b, p0, hq, hkv, qn.to(gpu), kn.to(gpu), 1e-6, rope.to(gpu), kd, vd,
                                rope_style=0 if style == "halves" else 1)
    out = ops.prefill_attention(qd, p0, hkv, kd, vd).float().cpu()
    return qd.cpu(), qb, kd.cpu(), vd.cpu(), kref, vref, out, ref, mag


@pytest.mark.parametrize("style", ["halves", "interleaved"])
@pytest.mark.parametrize("b,t,p0,hq,hkv,cap", [
    (2, 100, 0, 16, 8, 128),      # Qwen3-0.6B heads, ragged prompt (not a multiple of the 32-row tile)
    (3, 64, 0, 16, 8, 64),        # prompt fills the cache
    (1, 200, 0, 8, 8, 256),       # one q head per kv head (64-row tiles)
    (2, 37, 0, 16, 4, 64),        # 4 q heads per kv head
    (1, 50, 0, 16, 2, 64),        # 8 q heads per kv head
    (2, 70, 90, 16, 8, 256),      # second prompt chunk: positions 90..159 over 90 cached slots
])
def test_prefill_prep_and_attention_match_oracle(gpu, b, t, p0, hq, hkv, cap, style):
    qd, qb, kd, vd, kref, vref, out, ref, mag = _case(gpu, b, t, p0, hq, hkv, cap, style, seed=b * 100 + t + p0)
    fq, wq = ulp_diff(qd.float(), qb)
    assert wq <= 1 and fq < 0.01, (fq, wq)
    fk, wk = ulp_diff(kd[:, :, p0:p0 + t].float(), kref[:, :, p0:p0 + t])
    assert wk <= 1 and fk < 0.01, (fk, wk)
    assert torch.equal(vd[:, :, p0:p0 + t].float(), vref[:, :, p0:p0 + t])
    # slots outside p0..p0+T-1 untouched
    assert torch.equal(kd[:, :, :p0].float(), kref[:, :, :p0])
    assert torch.equal(kd[:, :, p0 + t:].float(), kref[:, :, p0 + t:])
    err = (out - ref).abs()
    scale = ref.abs().max()
    assert err.max() / scale <= 1e-2, f"max relative error {err.max() / scale:.3e}"
    # each softmax weight is rounded to bf16 (relative 2^-9) before P . V, and the
    # output to bf16 (2^-9): |err| <= 2^-9 (sum_j p_j |v_j| + |ref|), bound taken at 2^-8
    assert (err <= 2.0 ** -8 * (mag + ref.abs()) + 1e-6).all(), (err / (mag + ref.abs())).max()


def _random_prefill_cases(n_cases: int, seed: int):
    """Seeded random prompt chunks: 1-4 sequences of 1-300 rows at a start position of
    0-300 (earlier slots cached), 1/2/4/8 q heads per kv head, a cache with up to 100
    slots past the chunk, both RoPE styles."""
    rs = np.random.RandomState(seed)
    cases = []
    for i in range(n_cases):
        hkv = int(rs.choice([1, 2, 4, 8]))
        hq = hkv * int(rs.choice([1, 2, 4])) if hkv == 8 else hkv * int(rs.choice([1, 2, 4, 8]))
        b, t = int(rs.randint(1, 5)), int(rs.randint(1, 301))
        p0 = 0 if i % 3 == 0 else int(rs.randint(0, 301))
        cases.append((b, t, p0, hq, hkv, p0 + t + int(rs.randint(0, 101)), "halves" if i % 2 else "interleaved"))
    return cases


RANDOM_PREFILL = _random_prefill_cases(12, seed=5)


@pytest.mark.parametrize("b,t,p0,hq,hkv,cap,style", RANDOM_PREFILL,
                         ids=[f"B{c[0]}-T{c[1]}-p{c[2]}-Hq{c[3]}-Hkv{c[4]}-cap{c[5]}-{c[6]}" for c in RANDOM_PREFILL])
def test_prefill_random_shapes(gpu, b, t, p0, hq, hkv, cap, style):
    """The bars of test_prefill_prep_and_attention_match_oracle at seeded random shapes."""
    qd, qb, kd, vd, kref, vref, out, ref, mag = _case(gpu, b, t, p0, hq, hkv, cap, style, seed=7 * b + t + p0)
    fq, wq = ulp_diff(qd.float(), qb)
    assert wq <= 1 and fq < 0.01, (fq, wq)
    fk, wk = ulp_diff(kd[:, :, p0:p0 + t].float(), kref[:, :, p0:p0 + t])
    assert wk <= 1 and fk < 0.01, (fk, wk)
    assert torch.equal(vd[:, :, p0:p0 + t].float(), vref[:, :, p0:p0 + t])
    assert torch.equal(kd[:, :, :p0].float(), kref[:, :, :p0])
    assert torch.equal(kd[:, :, p0 + t:].float(), kref[:, :, p0 + t:])
    err = (out - ref).abs()
    assert err.max() / ref.abs().max() <= 1e-2
    assert (err <= 2.0 ** -8 * (mag + ref.abs()) + 1e-6).all(), (err / (mag + ref.abs())).max()


def _oracle_cfg(cfg):
    return oq.Qwen3Config(**{k: getattr(cfg, k) for k in oq.Qwen3Config.__dataclass_fields__})


def _random_projection_cases(n_cases: int, seed: int):
    """Seeded random fused-projection shapes: 512-1500 prompt rows over 1-8
    sequences, 1/2/4/8 q heads per kv head over 1-8 kv heads, K any multiple of 128 up
    to 3072, a start position of 0-200 and up to 64 slots past the prompt."""
    rs = np.random.RandomState(seed)
    cases = []
    while len(cases) < n_cases:
        b = int(rs.randint(1, 9))
        t = int(rs.randint(-(-512 // b), 1500 // b + 1))
        hkv = int(rs.choice([1, 2, 4, 8]))
        hq = hkv * int(rs.choice([1, 2, 4, 8]))
        k = 128 * int(rs.randint(1, 25))
        p0 = int(rs.randint(0, 201))
        if 512 <= b * t <= 1500 and hq + 2 * hkv <= 40:
            cases.append((b, t, p0, hq, hkv, k, p0 + t + int(rs.randint(0, 65))))
    return cases


@pytest.mark.parametrize("style", [0, 1])
@pytest.mark.parametrize("b,t,p0,hq,hkv,k,cap", [
    (16, 512, 0, 16, 8, 1024, 640),     # the Qwen3-0.6B prompt pass
    (3, 200, 37, 16, 4, 2048, 300),     # 600 rows: a ragged last row tile; 4 q heads a kv head; p0 > 0
    (1, 512, 0, 8, 8, 1024, 512),       # one q head a kv head, the cache exactly full
] + _random_projection_cases(5, seed=8))
def test_fused_prompt_projection_matches_two_launches(gpu, b, t, p0, hq, hkv, k, cap, style):
    """The prompt GEMM with the q/k norm + RoPE + cache write in its epilogue gives
    the bits of the projection followed by t2i_prefill_qk_rope_kv: q rows and both
    caches (slots outside p0 .. p0 + T - 1 untouched)."""
    print(f"fused prompt projection B={b} T={t} p0={p0} Hq={hq} Hkv={hkv} K={k} style={style}", flush=True)
    from oracle import w4a16 as ow
    from torch2iron_amd.formats import W4A16Weight
    d = 128
    n = (hq + 2 * hkv) * d
    w = W4A16Weight.from_numpy(*ow.synthetic_tensors(k, n, seed=b + t + k), device=gpu)
    g = torch.Generator().manual_seed(t + p0)
    x = (torch.randn(b * t, k, generator=g) * 2).to(BF16).to(gpu)
    kc0 = torch.randn(b, hkv, cap, d, generator=g).to(BF16).to(gpu)
    vc0 = torch.randn(b, hkv, cap, d, generator=g).to(BF16).to(gpu)
    qn = (torch.rand(d, generator=g) * 0.2 + 0.9).to(BF16).to(gpu)
    kn = (torch.rand(d, generator=g) * 0.2 + 0.9).to(BF16).to(gpu)
    rope = gm.rope_table(d, cap, 1e6, gpu)
    kc_ref, vc_ref = kc0.clone(), vc0.clone()
    q_ref = ops.prefill_qk_rope_kv(ops.linear(x, w), b, p0, hq, hkv, qn, kn, 1e-6, rope, kc_ref, vc_ref,
                                   rope_style=style)
    kc, vc = kc0.clone(), vc0.clone()
    q = ops.prefill_qkv_rope_kv(x, w, b, p0, hq, hkv, qn, kn, 1e-6, rope, kc, vc, rope_style=style)
    torch.cuda.synchronize()
    assert torch.equal(q, q_ref), "q rows"
    assert torch.equal(kc, kc_ref) and torch.equal(vc, vc_ref), "KV cache"
    assert not torch.equal(kc, kc0)   # the prompt's slots were written


@pytest.mark.parametrize("weights,plen", [("centered", 70), ("uniform", 70), ("centered", 160)],
                         ids=["centered-280rows", "uniform-280rows", "centered-640rows"])
def test_model_prefill_matches_oracle(gpu, weights, plen):
    """Whole prompt pass (3 layers, batch 4): the KV cache and the first greedy token of
    each sequence against the oracle's prefill.  280 rows run the 16-row-tile linear
    and the separate q/k prep; 640 rows the prompt GEMM with the prep in its epilogue
    and every GEMM's row sums handed over by the kernel that wrote its input."""
    cfg = gm.Qwen3Config(n_layers=3, vocab=4096)
    t = gm.random_qwen3_tensors(cfg, seed=41, weights=weights)
    b = 4
    cap = plen + 26
    prompt = torch.randint(0, cfg.vocab, (b, plen), generator=torch.Generator().manual_seed(42))
    m = gm.Qwen3Model(t, cfg, batch=b, ctx_cap=cap, device=gpu)
    assert m._prefill_sums(b * plen) == (b * plen >= ops.PROMPT_GEMM_ROWS)
    m.reset()
    m.history = torch.zeros(b, 4, dtype=torch.int32, device=gpu)
    m.step.zero_()
    m.prefill(prompt)
    first = m.tokens.cpu().long()
    assert int(m.positions.min()) == plen and int(m.positions.max()) == plen
    assert torch.equal(m.history[:, 0].cpu().long(), first)
    o32 = oq.DenseQwen3(t, _oracle_cfg(cfg), mode="fp32", ctx_cap=cap)
    o16 = oq.DenseQwen3(t, _oracle_cfg(cfg), mode="bf16", ctx_cap=cap)
    l32 = o32.prefill(prompt)
    l16 = o16.prefill(prompt)
    noise = (l16 - l32).abs().amax(dim=1)
    top2 = torch.topk(l32, 2, dim=1).values
    margin = top2[:, 0] - top2[:, 1]
    ref = l32.argmax(dim=1)
    for i in range(b):
        if first[i] != ref[i]:
            assert margin[i] <= 2 * noise[i], f"sequence {i}: margin {margin[i]:.3f} > 2 x bf16 noise {noise[i]:.3f}"
    # the cache rows the prompt wrote: layer 0 within a few bf16 roundings of each head
    # vector's scale (RoPE's rotate-and-add cancels, so ulps near zero say nothing);
    # deeper layers drift by the bf16 rounding of the layers before them
    k0 = m.k_cache[0, :, :, :plen].float().cpu()
    r0 = o16.k_cache[0, :, :, :plen]
    assert ((k0 - r0).abs() <= 2.0 ** -7 * r0.abs().amax(dim=-1, keepdim=True)).all()
    for li in range(cfg.n_layers):
        kk = m.k_cache[li, :, :, :plen].float().cpu()
        k16, k32 = o16.k_cache[li, :, :, :plen], o32.k_cache[li, :, :, :plen]
        band = (k16 - k32).abs().max()            # what bf16 rounding alone moves the oracle by
        assert (kk - k16).abs().max() <= 2 * band + 2.0 ** -7 * k16.abs().max(), li


def test_generate_with_prefill_matches_oracle(gpu):
    """4 layers, batch 8: prefill + 24 greedy decode steps vs the fp32 oracle, divergences
    only at near-ties, and teacher-forced logits (prefill, then decode steps) no noisier
    against fp32 than the oracle's bf16 mode."""
    from tests.test_gpu_decode import assert_logit_noise_like_bf16_oracle, assert_near_tie
    cfg = gm.Qwen3Config(n_layers=4, vocab=8192)
    t = gm.random_qwen3_tensors(cfg, seed=21, weights="centered")
    b, plen, new = 8, 40, 24
    prompt = torch.randint(0, cfg.vocab, (b, plen), generator=torch.Generator().manual_seed(23))
    m = gm.Qwen3Model(t, cfg, batch=b, ctx_cap=80, device=gpu)
    got = m.generate(prompt, new, prompt_mode="prefill")
    got_eager = m.generate(prompt, new, prompt_mode="prefill", use_graph=False)
    assert torch.equal(got, got_eager)
    o16 = oq.DenseQwen3(t, _oracle_cfg(cfg), mode="bf16", ctx_cap=80)
    o32 = oq.DenseQwen3(t, _oracle_cfg(cfg), mode="fp32", ctx_cap=80)
    ref, margins = o32.generate(prompt, new, return_margins=True)
    for i in range(b):
        diff = (got[i] != ref[i]).nonzero()
        if len(diff):
            s = int(diff[0])
            assert_near_tie(o16, o32, prompt[i:i + 1], ref[i:i + 1, :s], margins[i, s], f"sequence {i} step {s}")
    assert_logit_noise_like_bf16_oracle(m, o16, o32, prompt, ref[:, :new - 1], "prefill")
