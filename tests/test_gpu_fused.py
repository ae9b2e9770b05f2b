"""The decode layer's front in one cooperative launch (``t2i_qkv_attention``): the
RMSNorm + q|k|v projection (the decode linear's 16-wave tile) must match
``t2i_w4a16_rmsnorm_linear``, whose plan may split K over 8 waves instead, up to
the order of the fp32 partial sums (within one bf16 rounding, mostly identical;
its tagged words are read back from the workspace); on those projection rows the
KV-cache write must give the bits of ``t2i_decode_attention`` and the context
match it within a bf16 rounding, and the oracle within the attention test's bars.
Repeated launches and graph replays keep working (the tag advances per launch)."""

import pytest
import torch

from oracle import qwen3 as oq
from oracle import w4a16 as ow
from torch2iron_amd import ops
from torch2iron_amd import model as gm
from torch2iron_amd.formats import W4A16Weight

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16
D = 128


def _case(gpu, b, hq, hkv, hidden, cap, positions, seed):
    g = torch.Generator().manual_seed(seed)
    n = (hq + 2 * hkv) * D
    w = W4A16Weight.from_numpy(*ow.synthetic_tensors(hidden, n, seed=seed), device=gpu)
    x = (torch.randn(b, hidden, generator=g) * 2).to(BF16).to(gpu)
    ln = (torch.rand(hidden, generator=g) * 0.2 + 0.9).to(BF16).to(gpu)
    kc = torch.randn(b, hkv, cap, D, generator=g).to(BF16).to(gpu)
    vc = torch.randn(b, hkv, cap, D, generator=g).to(BF16).to(gpu)
    qn = (torch.rand(D, generator=g) * 0.2 + 0.9).to(BF16).to(gpu)
    kn = (torch.rand(D, generator=g) * 0.2 + 0.9).to(BF16).to(gpu)
    pos = torch.tensor(positions, dtype=torch.int32, device=gpu)
    rope = gm.rope_table(D, cap, 1e6, gpu)
    return w, x, ln, kc, vc, qn, kn, pos, rope


def _ll_values(ws, b, n):
    """The projection's bf16 values from the tagged words at the start of the workspace."""
    v = ws[:b * n * 8].view(torch.int64).view(b, n) & 0xFFFF
    return torch.where(v >= 32768, v - 65536, v).to(torch.int16).view(BF16)


@pytest.mark.parametrize("style", [0, 1])
@pytest.mark.parametrize("b,hq,hkv,hidden,cap,positions,normed", [
    (16, 16, 8, 1024, 640, [576] * 8 + [0, 95, 96, 191, 192, 300, 383, 639], False),   # 2 splits a pair
    (8, 16, 8, 1024, 1088, [1024] * 4 + [0, 191, 192, 1087], False),                    # 4 splits, streamed rows
    (3, 16, 8, 2048, 300, [0, 150, 299], False),                                           # 8 splits, K = 2048
    (1, 16, 8, 1024, 2100, [2050], True),                                                  # 16 splits, long context
    (16, 8, 8, 1024, 200, list(range(0, 200, 13))[:16], True),                             # 1 q head per kv head
])
def test_fused_front_matches_unfused_kernels_and_oracle(gpu, b, hq, hkv, hidden, cap, positions, normed, style):
    print(f"fused front B={b} Hq={hq} Hkv={hkv} K={hidden} cap={cap} normed={normed} style={style}", flush=True)
    w, x, ln, kc, vc, qn, kn, pos, rope = _case(gpu, b, hq, hkv, hidden, cap, positions, seed=b + cap)
    n = (hq + 2 * hkv) * D
    kc2, vc2 = kc.clone(), vc.clone()
    ws = ops.Workspace()
    ctx = ops.qkv_attention(x, None if normed else ln, 1e-6, w, pos, hq, hkv, qn, kn, rope, kc2, vc2,
                            rope_style=style, workspace=ws)
    torch.cuda.synchronize()
    assert ops.qkv_attention_errors(b, hq, hkv, gpu, workspace=ws) == 0
    # the projection, up to the order of the partial sums
    unfused = ops.linear(x, w) if normed else ops.rmsnorm_linear(x, ln, 1e-6, w)
    buf = next(iter(ws._bufs.values()))
    qkv = _ll_values(buf, b, n)
    g, r = qkv.float(), unfused.float()
    assert ((g - r).abs() <= 2.0 ** -7 * r.abs() + 1e-3 * r.abs().max()).all()
    assert (g == r).float().mean().item() >= 0.9
    # the unfused attention on the launch's own projection rows
    ref = ops.decode_attention(qkv, pos, hq, hkv, qn, kn, 1e-6, rope, kc, vc, rope_style=style)
    assert torch.equal(kc2, kc) and torch.equal(vc2, vc), "KV-cache writes differ from the unfused kernel"
    diff = (ctx.float() - ref.float()).abs()
    assert (diff <= 2.0 ** -7 * ref.float().abs() + 1e-3 * ref.float().abs().max()).all()
    # and the oracle in its bf16 mode
    rnd = oq._Round("bf16")
    q = qkv.float().cpu()[:, :hq * D].view(b, hq, D)
    k = qkv.float().cpu()[:, hq * D:(hq + hkv) * D].view(b, hkv, D)
    v = qkv.float().cpu()[:, (hq + hkv) * D:].view(b, hkv, D)
    p = pos.long().cpu()
    cs = oq.rope_angles(D, cap, 1e6)[p]
    st = "halves" if style == 0 else "interleaved"
    q = oq.apply_rope(oq.rmsnorm(q, qn.float().cpu(), 1e-6, rnd), cs[:, None, :], st, rnd)
    k = oq.apply_rope(oq.rmsnorm(k, kn.float().cpu(), 1e-6, rnd), cs[:, None, :], st, rnd)
    kref, vref = kc.float().cpu().clone(), vc.float().cpu().clone()   # with the new k / v at each position
    for i in range(b):
        kref[i, :, p[i]] = k[i]
        vref[i, :, p[i]] = v[i]
    out = oq.decode_attention(q, kref, vref, p + 1, hkv).reshape(b, -1)
    err = (ctx.float().cpu() - out).abs().max() / out.abs().max()
    assert err <= 1e-2, f"max relative error {err:.3e}"


def test_fused_front_out_of_range_position(gpu):
    b, hq, hkv, cap = 4, 16, 8, 128
    w, x, ln, kc, vc, qn, kn, _, rope = _case(gpu, b, hq, hkv, 1024, cap, [0] * b, seed=5)
    pos = torch.tensor([cap, -1, 5, cap + 7], dtype=torch.int32, device=gpu)
    kc0, vc0 = kc.clone(), vc.clone()
    ctx = ops.qkv_attention(x, ln, 1e-6, w, pos, hq, hkv, qn, kn, rope, kc, vc, workspace=ops.Workspace())
    torch.cuda.synchronize()
    for i in (0, 1, 3):
        assert torch.count_nonzero(ctx[i]).item() == 0
    assert torch.count_nonzero(ctx[2]).item() > 0
    changed = (kc != kc0).any(dim=-1).any(dim=1)   # [b, cap]
    assert changed[0].sum() == 0 and changed[1].sum() == 0 and changed[3].sum() == 0
    assert bool(changed[2, 5]) and changed[2].sum() == 1


def test_fused_front_repeated_and_graph_replays(gpu):
    """The tag advances per launch: repeated launches on one workspace, and replays
    of a captured launch with eager work in between, all give the first result."""
    b, hq, hkv, cap = 16, 16, 8, 512
    w, x, ln, kc, vc, qn, kn, pos, rope = _case(gpu, b, hq, hkv, 1024, cap, [400] * b, seed=9)
    ws = ops.Workspace()
    out = torch.empty(b, hq * D, dtype=BF16, device=gpu)
    first = ops.qkv_attention(x, ln, 1e-6, w, pos, hq, hkv, qn, kn, rope, kc, vc, out=out, workspace=ws).clone()
    for _ in range(3):
        again = ops.qkv_attention(x, ln, 1e-6, w, pos, hq, hkv, qn, kn, rope, kc, vc, out=out, workspace=ws)
        assert torch.equal(again, first)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            ops.qkv_attention(x, ln, 1e-6, w, pos, hq, hkv, qn, kn, rope, kc, vc, out=out, workspace=ws)
    torch.cuda.current_stream().wait_stream(s)
    for i in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, first), f"replay {i}"
        ops.qkv_attention(x, ln, 1e-6, w, pos, hq, hkv, qn, kn, rope, kc, vc, workspace=ws)   # eager in between
    torch.cuda.synchronize()
    assert ops.qkv_attention_errors(b, hq, hkv, gpu, workspace=ws) == 0


def test_fused_front_rejects_unsupported_shapes(gpu):
    w, x, ln, kc, vc, qn, kn, pos, rope = _case(gpu, 17, 16, 8, 1024, 64, [0] * 17, seed=1)
    with pytest.raises(ValueError):
        ops.qkv_attention(x, ln, 1e-6, w, pos, 16, 8, qn, kn, rope, kc, vc)   # B = 17 > 16


def test_model_decode_with_fused_front_matches_unfused(gpu):
    """A 3-layer model: greedy tokens with the fused front equal the unfused kernels'
    wherever the fp32 oracle's top-2 margin is not a near-tie; logits within bf16 noise."""
    cfg = gm.Qwen3Config(n_layers=3, vocab=4096)
    t = gm.random_qwen3_tensors(cfg, seed=61, weights="centered")
    b, plen, new = 16, 40, 16
    prompt = torch.randint(0, cfg.vocab, (b, plen), generator=torch.Generator().manual_seed(62))
    fused = gm.Qwen3Model(t, cfg, batch=b, ctx_cap=64, device=gpu, fused=True, persistent=False)
    plain = gm.Qwen3Model(t, cfg, batch=b, ctx_cap=64, device=gpu, fused=False, persistent=False)
    assert fused.layers[0].fused and not plain.layers[0].fused
    tf = fused.generate(prompt, new)
    tp = plain.generate(prompt, new)
    same = (tf == tp).all(dim=1).float().mean().item()
    print(f"fused vs unfused front: {same:.2f} of sequences identical over {new} tokens", flush=True)
    assert same >= 0.75
    # logits along the same tokens
    fused.reset()
    plain.reset()
    lf = fused.prefill(prompt, want_logits=True)
    lp = plain.prefill(prompt, want_logits=True)
    _, lf2 = fused.decode_step(tp[:, 0], torch.full((b,), plen), want_logits=True)
    _, lp2 = plain.decode_step(tp[:, 0], torch.full((b,), plen), want_logits=True)
    assert torch.equal(lf, lp)   # the prompt pass does not use the fused front
    rel = ((lf2 - lp2).pow(2).mean().sqrt() / lp2.std()).item()
    assert rel < 2e-2, rel
