"""Row group sums handed to the prompt GEMM (the ``*_sums`` entry points).

The producers (RMSNorm, prefill attention, the gate_up SwiGLU epilogue) write
the same bf16 outputs as their plain forms, bit for bit, and fp32 sums of those
outputs over each 128-wide (or 64-wide half) group within 1e-5 of the sum of the
magnitudes (fp32 rounding of a 128-term sum; the fp64 sum of the bf16 values is
the truth).  The GEMM given the sums meets the oracle bars of the prompt-row
tests (max relative error 1e-2, elementwise one bf16 rounding) and agrees with
the plain GEMM, which forms the sums itself, on at least 99 % of the outputs
and within one bf16 ulp plus 1e-4 of the largest output elsewhere (the
two differ only in the fp32 rounding of the zero-point term).
"""

import numpy as np
import pytest
import torch

from oracle import w4a16 as ow
from torch2iron_amd import ops
from torch2iron_amd.formats import W4A16Weight, interleave_gate_up

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16


def check_linear(y: torch.Tensor, ref: np.ndarray):
    """The prompt-row bars: max relative error 1e-2, elementwise one bf16 rounding."""
    yf = y.float().cpu().numpy().astype(np.float64)
    scale = np.abs(ref).max()
    err = np.abs(yf - ref)
    assert err.max() / scale <= 1e-2, f"max relative error {err.max() / scale:.3e}"
    bad = err > 2.0 ** -8 * np.abs(ref) * 1.01 + 1e-4 * scale
    assert not bad.any(), f"{bad.sum()} elements beyond one bf16 rounding; worst {err.max():.4e}"


def group_sums(y: torch.Tensor, width: int) -> tuple[torch.Tensor, torch.Tensor]:
    """fp64 sums of the rows of ``y`` over ``width``-wide column groups, and of |y|."""
    yf = y.double().cpu()
    m, n = yf.shape
    g = yf.view(m, n // width, width)
    return g.sum(-1), g.abs().sum(-1)


def check_sums(got: torch.Tensor, y: torch.Tensor, width: int):
    """got: the group-major sums [groups, rows] a producer wrote."""
    ref, mag = group_sums(y, width)
    err = (got.double().cpu().view(ref.shape[1], ref.shape[0]).t() - ref).abs()
    assert (err <= 1e-5 * mag + 1e-30).all(), f"worst sum error {(err / (mag + 1e-30)).max():.3e} of |y|"


def check_close_to_plain(y: torch.Tensor, plain: torch.Tensor, head_vectors: bool = False):
    """Within one bf16 ulp of the plain output (2^-7 relative at most) plus 1e-4 of its
    largest value (the zero-point term's fp32 rounding moves outputs near zero by
    more than an ulp of their own), and equal on at least 99 % of the outputs.
    head_vectors (rows normalised and rotated after the product): plus one ulp of
    the row's largest value instead, as RoPE's differences cancel."""
    a, b = y.float().cpu(), plain.float().cpu()
    err = (a - b).abs()
    if head_vectors:
        bound = 2.0 ** -7 * b.abs() + 2.0 ** -7 * b.abs().amax(dim=-1, keepdim=True)
    else:
        bound = 2.0 ** -7 * b.abs() + 1e-4 * b.abs().max()
    frac = (a == b).float().mean().item()
    assert (err <= bound).all(), f"worst difference {(err / bound).max():.3f} of the bound ({frac:.4f} equal)"
    assert frac >= 0.99, f"only {frac:.4f} equal"


def _sums(x: torch.Tensor, parts: int) -> torch.Tensor:
    """Exact (fp64, then fp32) group sums of x, group-major, as a producer hands them over."""
    s, _ = group_sums(x, 128 // parts)
    return s.t().float().contiguous()


@pytest.mark.parametrize("m,h", [(600, 1024), (513, 2048), (64, 3072)])
def test_rmsnorm_sums(gpu, m, h):
    g = torch.Generator().manual_seed(m + h)
    x = (torch.randn(m, h, generator=g) * 3).to(BF16).to(gpu)
    w = (torch.rand(h, generator=g) * 0.2 + 0.9).to(BF16).to(gpu)
    plain = ops.rmsnorm(x, w, 1e-6)
    sums = torch.full((h // 128, m), float("nan"), device=gpu)
    y = ops.rmsnorm(x, w, 1e-6, out_sums=sums)
    assert torch.equal(y, plain)
    check_sums(sums, y, 128)


def test_rmsnorm_sums_gathered_rows(gpu):
    """The embedding gather form: x_out gets the table rows, y and its sums as above."""
    v, h, m = 300, 1024, 520
    g = torch.Generator().manual_seed(11)
    table = torch.randn(v, h, generator=g).to(BF16).to(gpu)
    w = (torch.rand(h, generator=g) * 0.2 + 0.9).to(BF16).to(gpu)
    tok = torch.randint(0, v, (m,), generator=g, dtype=torch.int32).to(gpu)
    x_out = torch.empty(m, h, dtype=BF16, device=gpu)
    sums = torch.empty(h // 128, m, device=gpu)
    y = ops.rmsnorm(table, w, 1e-6, tokens=tok, x_out=x_out, out_sums=sums)
    assert torch.equal(x_out, table[tok.long()])
    assert torch.equal(y, ops.rmsnorm(table[tok.long()].contiguous(), w, 1e-6))
    check_sums(sums, y, 128)


@pytest.mark.parametrize("b,t,hq,hkv", [(2, 300, 16, 8), (1, 70, 8, 8), (3, 64, 16, 4)])
def test_prefill_attention_sums(gpu, b, t, hq, hkv):
    d, cap = 128, t + 16
    g = torch.Generator().manual_seed(b * 1000 + t)
    q = torch.randn(b, hq, t, d, generator=g).to(BF16).to(gpu)
    kc = torch.randn(b, hkv, cap, d, generator=g).to(BF16).to(gpu)
    vc = torch.randn(b, hkv, cap, d, generator=g).to(BF16).to(gpu)
    plain = ops.prefill_attention(q, 0, hkv, kc, vc)
    sums = torch.full((hq, b * t), float("nan"), device=gpu)
    out = ops.prefill_attention(q, 0, hkv, kc, vc, out_sums=sums)
    assert torch.equal(out, plain)
    check_sums(sums, out, 128)


SUM_CASES = [(600, 1024, 4096, 1), (1030, 3072, 1024, 2), (520, 128, 128, 1), (777, 2048, 1024, 2),
             (513, 384, 384, 1)]


@pytest.mark.parametrize("m,k,n,parts", SUM_CASES, ids=[f"M{m}-K{k}-N{n}-p{p}" for m, k, n, p in SUM_CASES])
def test_prompt_linear_with_sums(gpu, m, k, n, parts):
    qw, qz, sc = ow.synthetic_tensors(k, n, seed=3000 + m + k)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m + n)).to(BF16)
    ref = ow.linear(x.float().numpy(), qw, qz, sc, accumulate="fp64")
    w = W4A16Weight.from_numpy(qw, qz, sc, device=gpu)
    xd = x.to(gpu)
    y = ops.linear(xd, w, x_sums=_sums(x, parts).to(gpu), sum_parts=parts)
    check_linear(y, ref)
    check_close_to_plain(y, ops.linear(xd, w))


def test_prompt_linear_with_sums_residual(gpu):
    m, k, n = 700, 2048, 1024
    qw, qz, sc = ow.synthetic_tensors(k, n, seed=51)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(52)).to(BF16)
    res = torch.randn(m, n, generator=torch.Generator().manual_seed(53)).to(BF16).to(gpu)
    w = W4A16Weight.from_numpy(qw, qz, sc, device=gpu)
    xd = x.to(gpu)
    plain = ops.linear(xd, w, residual=res)
    out = res.clone()
    y = ops.linear(xd, w, residual=out, out=out, x_sums=_sums(x, 1).to(gpu))
    # one bf16 ulp of the product (rounded before the residual is added) and one of the sum
    lin = ops.linear(xd, w).float().cpu()
    a, b = y.float().cpu(), plain.float().cpu()
    bound = 2.0 ** -7 * (lin.abs() + b.abs()) + 1e-4 * lin.abs().max()
    assert ((a - b).abs() <= bound).all(), f"worst difference {((a - b).abs() / bound).max():.3f} of the bound"
    assert (a == b).float().mean().item() >= 0.99


def test_gate_up_with_sums(gpu):
    """x_sums in, and the SwiGLU output's half-group sums out (the down projection's input)."""
    m, k, inter = 600, 1024, 3072
    gate = ow.synthetic_tensors(k, inter, seed=61)
    up = ow.synthetic_tensors(k, inter, seed=62)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(63)).to(BF16)
    w = W4A16Weight.from_numpy(*interleave_gate_up(gate, up), device=gpu)
    xd, xs = x.to(gpu), _sums(x, 1).to(gpu)
    g, u = ops.gate_up(xd, w, swiglu=False, x_sums=xs)
    check_linear(g, ow.linear(x.float().numpy(), *gate, accumulate="fp64"))
    check_linear(u, ow.linear(x.float().numpy(), *up, accumulate="fp64"))
    g0, u0 = ops.gate_up(xd, w, swiglu=False)
    check_close_to_plain(g, g0)
    check_close_to_plain(u, u0)
    hs = torch.full((2 * inter // 128, m), float("nan"), device=gpu)
    h = ops.gate_up(xd, w, swiglu=True, x_sums=xs, out_sums=hs).float().cpu()
    # the SwiGLU epilogue on this form's own gate and up, as test_prompt_rows_gate_up
    h_chain = (torch.nn.functional.silu(g.float().cpu()).to(BF16).float() * u.float().cpu()).to(BF16).float()
    assert (h - h_chain).abs().max() <= 2.0 ** -7 * h_chain.abs().max()
    assert (h == h_chain).float().mean() > 0.999
    check_sums(hs, h, 64)
    # the plain input and the sums-out form agree on h too
    hs2 = torch.empty_like(hs)
    assert torch.equal(ops.gate_up(xd, w, swiglu=True, out_sums=hs2), ops.gate_up(xd, w, swiglu=True))
    check_sums(hs2, ops.gate_up(xd, w, swiglu=True), 64)


def test_prefill_projection_with_sums(gpu):
    """The fused qkv projection + q/k norm + RoPE + cache write, given x's sums, against
    the same launch forming them itself: q and the caches as check_close_to_plain."""
    from torch2iron_amd import model as gm
    b, t, hq, hkv, k = 4, 160, 16, 8, 1024
    d, cap = 128, 192
    n = (hq + 2 * hkv) * d
    qw, qz, sc = ow.synthetic_tensors(k, n, seed=71)
    w = W4A16Weight.from_numpy(qw, qz, sc, device=gpu)
    g = torch.Generator().manual_seed(72)
    x = torch.randn(b * t, k, generator=g).to(BF16)
    qn = (torch.rand(d, generator=g) * 0.2 + 0.9).to(BF16).to(gpu)
    kn = (torch.rand(d, generator=g) * 0.2 + 0.9).to(BF16).to(gpu)
    rope = gm.rope_table(d, cap, 1e6, gpu)
    outs = []
    for xs in (None, _sums(x, 1).to(gpu)):
        kc = torch.zeros(b, hkv, cap, d, dtype=BF16, device=gpu)
        vc = torch.zeros_like(kc)
        q = ops.prefill_qkv_rope_kv(x.to(gpu), w, b, 0, hq, hkv, qn, kn, 1e-6, rope, kc, vc, x_sums=xs)
        outs.append((q, kc, vc))
    for a, c in zip(outs[0], outs[1]):
        check_close_to_plain(c.reshape(-1, d), a.reshape(-1, d), head_vectors=True)
