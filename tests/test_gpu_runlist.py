"""The reference's batch-decode runlist on the MI355X, entry for entry.

``runlist.batch_decode_runlist`` writes the per-step runlist of
``quantized_qwen3/batch_decode_fused.py:300-539`` with this build's operators,
constructed with the reference's own arguments: RMSNorm, the q GEMM and the
paired k|v GEMM, RMSNormRoPE on q and k, one attention entry per sequence
(``CopyPresentKVAttention``, for the packet-cache pair), the o GEMM,
ResidualAddRMSNorm, the paired gate|up GEMM, SiLUMul, the down GEMM and
ResidualAddRMSNorm, then the int4 lm_head GEMM.

Checks:
* each standalone operator against the oracle's formula, and against the fused
  kernel it stands for in the decode layer (bit for bit where they round alike);
* the whole runlist (one and two layers, a padded batch, ragged positions) against
  the fp32 oracle, inside the band of the oracle's own bf16 chain, as the decode
  layer test holds the standalone kernels; the written cache rows alike; the
  logits of the int4 lm_head within the linear's 1e-2 of the fp64 product.
"""

import numpy as np
import pytest
import torch

from oracle import qwen3 as oq
from oracle import w4a16 as ow
from torch2iron_amd import model as gm
from torch2iron_amd import ops
from torch2iron_amd import runlist as R
from torch2iron_amd.formats import W4A16Weight, interleave_gate_up

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16


def _ocfg(cfg):
    return oq.Qwen3Config(**{k: getattr(cfg, k) for k in oq.Qwen3Config.__dataclass_fields__})


def _ulps(a, b):
    ai = a.to(BF16).view(torch.int16).to(torch.int32)
    bi = b.to(BF16).view(torch.int16).to(torch.int32)
    d = (ai - bi).abs()
    return (d > 0).float().mean().item(), d.max().item()


@pytest.mark.parametrize("rows,cols,angle_rows,style", [(256, 128, 16, 0), (128, 128, 16, 1), (24, 64, 3, 0),
                                                        (40, 256, 8, 0), (7, 1024, 7, 1)])
def test_rmsnorm_rope_matches_oracle(gpu, rows, cols, angle_rows, style):
    g = torch.Generator().manual_seed(rows + cols)
    x = (torch.randn(rows, cols, generator=g) * 3).to(BF16)
    w = (torch.rand(cols, generator=g) * 0.2 + 0.9).to(BF16)
    pos = torch.randint(0, 4000, (angle_rows,), generator=g)
    ang = oq.rope_angles(cols, 4000, 1e6)[pos].to(BF16)
    eps = 1e-5
    rnd = oq._Round("bf16")
    xs = x.float().view(angle_rows, rows // angle_rows, cols)
    ref = oq.apply_rope(oq.rmsnorm(xs, w.float(), eps, rnd), ang.float()[:, None, :],
                        "halves" if style == 0 else "interleaved", rnd).view(rows, cols)
    xg = x.to(gpu)
    got = ops.rmsnorm_rope(xg, w.to(gpu), ang.to(gpu), eps, rope_style=style)
    frac, worst = _ulps(got.float().cpu(), ref)
    print(f"rmsnorm_rope {rows}x{cols}: {frac:.4f} of values differ from the oracle's bf16 chain, at most {worst} ulp")
    assert worst <= 2 and frac <= 0.02
    # in place (the runlist's "queries" -> "queries") gives the same bits
    ops.rmsnorm_rope(xg, w.to(gpu), ang.to(gpu), eps, rope_style=style, out=xg)
    assert torch.equal(xg, got)


def test_silu_mul_and_residual_add_rmsnorm_match_the_fused_epilogues(gpu):
    g = torch.Generator().manual_seed(3)
    k, n, m = 1024, 3072, 13
    gate, up = ow.synthetic_tensors(k, n, seed=1), ow.synthetic_tensors(k, n, seed=2)
    wp = W4A16Weight.from_numpy(*interleave_gate_up(gate, up), device=gpu)
    x = torch.randn(m, k, generator=g).to(BF16).to(gpu)
    gg, uu = ops.gate_up(x, wp, swiglu=False)
    h = ops.silu_mul(gg, uu)
    assert torch.equal(h, ops.gate_up(x, wp, swiglu=True))           # the SwiGLU epilogue's bits
    ref = oq._bf(oq._bf(oq.silu(gg.float().cpu())) * uu.float().cpu())
    assert torch.equal(h.float().cpu(), ref)
    # residual add + RMSNorm: the o_proj / down residual epilogue, then t2i_rmsnorm
    wo = W4A16Weight.from_numpy(*ow.synthetic_tensors(n, k, seed=4), device=gpu)
    res = torch.randn(m, k, generator=g).to(BF16).to(gpu)
    gamma = (torch.rand(k, generator=g) * 0.2 + 0.9).to(BF16).to(gpu)
    upd = ops.linear(h, wo)
    xo, y = ops.residual_add_rmsnorm(res, upd, gamma, 1e-5)
    assert torch.equal(xo, ops.linear(h, wo, residual=res))
    assert torch.equal(y, ops.rmsnorm(xo, gamma, 1e-5))
    # in place, as the runlist's ("x", "attn_output", W, "x", "x_norm")
    xi = res.clone()
    ops.residual_add_rmsnorm(xi, upd, gamma, 1e-5, x_out=xi, out=torch.empty_like(xi))
    assert torch.equal(xi, xo)


@pytest.mark.parametrize("b,hq,hkv,cap", [(5, 16, 8, 200), (3, 8, 2, 700), (16, 16, 8, 640)])
def test_prepared_attention_equals_the_prologue_form(gpu, b, hq, hkv, cap):
    """RMSNormRoPE on q and k, then the prepared attention, gives the bits of
    t2i_decode_attention (whose prologue norms and rotates), cache rows included."""
    g = torch.Generator().manual_seed(b + cap)
    d = 128
    qkv = torch.randn(b, (hq + 2 * hkv) * d, generator=g).to(BF16).to(gpu)
    qn = (torch.rand(d, generator=g) * 0.2 + 0.9).to(BF16).to(gpu)
    kn = (torch.rand(d, generator=g) * 0.2 + 0.9).to(BF16).to(gpu)
    kc = torch.randn(b, hkv, cap, d, generator=g).to(BF16).to(gpu)
    vc = torch.randn(b, hkv, cap, d, generator=g).to(BF16).to(gpu)
    pos = torch.randint(0, cap, (b,), generator=g, dtype=torch.int32).to(gpu)
    rope = gm.rope_table(d, cap, 1e6, gpu)
    k1, v1 = kc.clone(), vc.clone()
    ref = ops.decode_attention(qkv, pos, hq, hkv, qn, kn, 1e-5, rope, k1, v1)
    q = qkv[:, :hq * d].contiguous()
    k = qkv[:, hq * d:(hq + hkv) * d].contiguous()
    v = qkv[:, (hq + hkv) * d:].contiguous()
    ang = rope[pos.long()].contiguous()
    ops.rmsnorm_rope(q, qn, ang, 1e-5, out=q)
    ops.rmsnorm_rope(k, kn, ang, 1e-5, out=k)
    k2, v2 = kc.clone(), vc.clone()
    got = ops.decode_attention_prepared(q, k, v, pos, hq, hkv, k2, v2)
    torch.cuda.synchronize()
    assert torch.equal(k2, k1) and torch.equal(v2, v1)
    assert torch.equal(got, ref)


def _run_reference_runlist(gpu, cfg, t, batch, cap, positions, lm_head):
    built = R.batch_decode_runlist(cfg, cap, batch, lm_head_out_features=lm_head[2].shape[1])
    rows = built["decode_rows"]
    g = torch.Generator().manual_seed(31)
    x = torch.zeros(rows, cfg.hidden)
    x[:batch] = torch.randn(batch, cfg.hidden, generator=g)
    x = x.to(BF16)
    caches = [(torch.randn(batch, cfg.n_kv_heads, cap, cfg.head_dim, generator=g).to(BF16),
               torch.randn(batch, cfg.n_kv_heads, cap, cfg.head_dim, generator=g).to(BF16))
              for _ in range(cfg.n_layers)]
    pos = torch.tensor(positions, dtype=torch.int32)
    table = gm.rope_table(cfg.head_dim, cap, cfg.rope_theta, gpu)
    angles = torch.zeros(rows, cfg.head_dim, dtype=BF16, device=gpu)
    angles[:batch] = table[pos.long().to(gpu)]
    bufs = {"x": x.to(gpu), "rope_angles": angles, "positions": pos.to(gpu),
            **R.batch_decode_weights(t, cfg, gpu, lm_head=lm_head)}
    for i, (kc, vc) in enumerate(caches):
        bufs[f"k_cache_{i}"], bufs[f"v_cache_{i}"] = kc.to(gpu), vc.to(gpu)
    fused = R.FusedRunlist("quantized_batch_decode_fused_op", built["runlist"], built["input_args"],
                           built["output_args"], bufs, gpu, buffer_sizes=built["buffer_sizes"])
    fused()
    torch.cuda.synchronize()
    return built, fused, x, caches, pos


@pytest.mark.parametrize("layers,batch,positions", [(1, 5, [0, 7, 63, 100, 127]),
                                                    (2, 16, [(37 * i) % 128 for i in range(15)] + [127])])
def test_reference_batch_decode_runlist_matches_oracle(gpu, layers, batch, positions):
    """The reference's runlist (eps 1e-5, the default its RMSNorm operators are built
    with) against the fp32 oracle: final hidden rows and every layer's written k/v
    rows no farther from fp32 than the oracle's bf16 chain (max and RMS, within
    25 %); logits of the int4 lm_head within 1e-2 of the fp64 product."""
    cfg = gm.Qwen3Config(n_layers=layers, vocab=4096, eps=1e-5)
    t = gm.random_qwen3_tensors(cfg, seed=17, weights="centered")
    lm_head = ow.synthetic_tensors(cfg.hidden, cfg.vocab, seed=18)
    cap = 128
    built, fused, x, caches, pos = _run_reference_runlist(gpu, cfg, t, batch, cap, positions, lm_head)
    ocfg = _ocfg(cfg)
    ang = oq.rope_angles(cfg.head_dim, cap, cfg.rope_theta)
    slots, rows = pos.long(), torch.arange(batch)
    refs = {}
    for mode in ("bf16", "fp32"):
        rnd = oq._Round(mode)
        h = x[:batch].float()
        kv = [(kc.float().clone(), vc.float().clone()) for kc, vc in caches]
        for i in range(layers):
            h = oq.DenseLayer(t, f"model.layers.{i}", ocfg).decode(h, kv[i][0], kv[i][1], slots, ang, rnd)
        hn = oq.rmsnorm(h, torch.as_tensor(t["model.norm.weight"], dtype=torch.float32), cfg.eps, rnd)
        refs[mode] = (hn, kv)
    rms = lambda a: a.pow(2).mean().sqrt().item()
    checks = [("hidden_out", fused.get_buffer("hidden_out").view(-1, cfg.hidden)[:batch].float().cpu(),
               refs["bf16"][0], refs["fp32"][0])]
    for i in range(layers):
        for j, kind in enumerate(("k", "v")):
            got = fused.get_buffer(f"{kind}_cache_{i}").cpu()[rows, :, slots].float()
            checks.append((f"layer {i} {kind} row", got, refs["bf16"][1][i][j][rows, :, slots],
                           refs["fp32"][1][i][j][rows, :, slots]))
    failures = []
    for name, got, r16, r32 in checks:
        band_max, band_rms = (r16 - r32).abs().max().item(), rms(r16 - r32)
        dev_max, dev_rms = (got - r32).abs().max().item(), rms(got - r32)
        print(f"{name}: max dev {dev_max:.4f} (bf16 chain {band_max:.4f}), RMS {dev_rms:.5f} ({band_rms:.5f})")
        if dev_max > 1.25 * band_max + 1e-6:
            failures.append(f"{name}: max deviation {dev_max:.4f} vs bf16 chain {band_max:.4f}")
        if dev_rms > 1.25 * band_rms + 1e-7:
            failures.append(f"{name}: RMS deviation {dev_rms:.5f} vs bf16 chain {band_rms:.5f}")
    # untouched cache slots stay as they were
    kc0 = fused.get_buffer("k_cache_0").cpu().clone()
    kc0[rows, :, slots] = caches[0][0][rows, :, slots]
    if not torch.equal(kc0, caches[0][0]):
        failures.append("cache slots other than the current positions changed")
    hid = fused.get_buffer("hidden_out").view(-1, cfg.hidden).float().cpu().numpy()
    logits_ref = ow.linear(hid.astype(np.float64), *lm_head)
    logits = fused.get_buffer("logits").view(-1, cfg.vocab).float().cpu().numpy()
    err = np.abs(logits - logits_ref).max() / np.abs(logits_ref).max()
    print(f"lm_head logits: max rel err {err:.2e} against fp64")
    if err > 1e-2:
        failures.append(f"logits max relative error {err:.3e}")
    assert not failures, "; ".join(failures)
