"""W4A16 linear on the MI355X vs the CPU oracle (same seeded inputs).

Bars: the dequantised weights are bit-exact; the linear output is within the
max relative error 1e-2 of the fp64 oracle (max|y - ref| / max|ref|), and
elementwise within one bf16 rounding (2^-8 relative) plus a 1e-4 * max|ref|
accumulation allowance.
"""

import numpy as np
import pytest
import torch

from oracle import w4a16 as ow
from torch2iron_amd import ops
from torch2iron_amd.formats import W4A16Weight, interleave_gate_up

pytestmark = pytest.mark.gpu

QWEN3_06B = [(1024, 4096), (2048, 1024), (1024, 6144), (3072, 1024)]
QWEN3_17B = [(2048, 4096), (2048, 2048), (2048, 12288), (6144, 2048)]

CASES = [(1, 1024, 3072)]
CASES += [(m, k, n) for (k, n) in QWEN3_06B for m in (1, 8, 16, 32, 64)]
CASES += [(m, k, n) for (k, n) in QWEN3_17B for m in (1, 16, 64)]
CASES += [(3, 1024, 3072), (17, 2048, 1024), (50, 1024, 4096), (33, 3072, 1024), (5, 128, 64)]
# row tiles shorter than 16 rows (few column blocks): 4-row tiles with a 1-row last
# tile, 1-row tiles, 2-row tiles
CASES += [(13, 2048, 1024), (16, 1024, 256), (6, 3072, 1024)]
# two 16-row m-tiles a workgroup (64-column blocks needing one to two rounds of the
# CUs): a ragged second tile, and the Qwen3-1.7B gate_up at M = 32
CASES += [(48, 1024, 6144), (32, 2048, 12288)]


def _inputs(m, k, n, seed):
    qw, qz, sc = ow.synthetic_tensors(k, n, seed=seed)
    g = torch.Generator().manual_seed(seed + 1)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    return qw, qz, sc, x


def check_linear(y: torch.Tensor, ref: np.ndarray):
    yf = y.float().cpu().numpy().astype(np.float64)
    scale = np.abs(ref).max()
    err = np.abs(yf - ref)
    assert err.max() / scale <= 1e-2, f"max relative error {err.max() / scale:.3e}"
    bound = 2.0 ** -8 * np.abs(ref) * 1.01 + 1e-4 * scale
    bad = err > bound
    assert not bad.any(), f"{bad.sum()} elements beyond one bf16 rounding; worst {err.max():.4e}"


@pytest.mark.parametrize("m,k,n", CASES, ids=[f"M{m}-K{k}-N{n}" for m, k, n in CASES])
def test_linear_matches_oracle(gpu, m, k, n):
    qw, qz, sc, x = _inputs(m, k, n, seed=1000 + m + k + n)
    ref = ow.linear(x.float().numpy(), qw, qz, sc, accumulate="fp64")
    w = W4A16Weight.from_numpy(qw, qz, sc, device=gpu)
    y = ops.linear(x.to(gpu), w)
    check_linear(y, ref)
    # the in-workgroup reduction has a fixed order: a second call gives the same bits
    y2 = ops.linear(x.to(gpu), w)
    assert torch.equal(y, y2), "repeat call differs"


def test_gemv_vector_input(gpu):
    qw, qz, sc, x = _inputs(1, 1024, 3072, seed=7)
    ref = ow.linear(x.float().numpy(), qw, qz, sc)
    y = ops.linear(x[0].to(gpu), W4A16Weight.from_numpy(qw, qz, sc, device=gpu))
    assert y.shape == (3072,)
    check_linear(y.view(1, -1), ref)


@pytest.mark.parametrize("m,k,n", [(16, 2048, 1024), (64, 1024, 4096), (1, 3072, 1024), (13, 3072, 1024)])
def test_linear_residual(gpu, m, k, n):
    qw, qz, sc, x = _inputs(m, k, n, seed=31 + m)
    res = torch.randn(m, n, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    lin = ow.linear(x.float().numpy(), qw, qz, sc)
    ref = lin + res.float().numpy()
    out = res.clone().to(gpu)
    y = ops.linear(x.to(gpu), W4A16Weight.from_numpy(qw, qz, sc, device=gpu), residual=out, out=out)  # in place
    check_linear_residual = np.abs(y.float().cpu().numpy() - ref)
    # two bf16 roundings (the projection, then the sum)
    bound = 2.0 ** -8 * (np.abs(lin) + np.abs(ref)) * 1.01 + 1e-4 * np.abs(ref).max()
    assert (check_linear_residual <= bound).all()


@pytest.mark.parametrize("k,n", [(1024, 3072), (2048, 1024), (3072, 1024), (128, 64), (6144, 2048)])
def test_dequant_bit_exact(gpu, k, n):
    qw, qz, sc = ow.synthetic_tensors(k, n, seed=k + n)
    ref = ow.dequantize(qw, qz, sc)
    w = ops.dequantize(W4A16Weight.from_numpy(qw, qz, sc, device=gpu)).cpu().numpy()
    assert np.array_equal(w.view(np.uint32), ref.view(np.uint32))


def test_dequant_special_words(gpu):
    """All-zero, all-one and counting words, every zero nibble value."""
    k, n = 128, 64
    qw = np.zeros((k // 8, n), dtype=np.uint32)
    qw[0::3] = 0x76543210
    qw[1::3] = 0xFFFFFFFF
    qw[2::3] = 0xFEDCBA98
    qz = np.tile(np.array([0x76543210, 0xFEDCBA98], dtype=np.uint32), (1, n // 16)).reshape(1, n // 8)
    sc = np.linspace(0.005, 0.02, n, dtype=np.float16).reshape(1, n)
    qw, qz = qw.view(np.int32), qz.view(np.int32)
    ref = ow.dequantize(qw, qz, sc)
    w = ops.dequantize(W4A16Weight.from_numpy(qw, qz, sc, device=gpu)).cpu().numpy()
    assert np.array_equal(w.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("m,k,inter", [(1, 1024, 3072), (16, 1024, 3072), (64, 1024, 3072), (8, 2048, 6144)])
def test_gate_up_paired_and_swiglu(gpu, m, k, inter):
    gate = ow.synthetic_tensors(k, inter, seed=11)
    up = ow.synthetic_tensors(k, inter, seed=12)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(13)).to(torch.bfloat16)
    xf = x.float().numpy()
    g_ref = ow.linear(xf, *gate)
    u_ref = ow.linear(xf, *up)
    w = W4A16Weight.from_numpy(*interleave_gate_up(gate, up), device=gpu)
    g, u = ops.gate_up(x.to(gpu), w, swiglu=False)
    check_linear(g, g_ref)
    check_linear(u, u_ref)
    h = ops.gate_up(x.to(gpu), w, swiglu=True).float().cpu().numpy()
    # h from the GPU's own rounded gate/up must match the reference rounding chain exactly
    gb = g.float().cpu()
    ub = u.float().cpu()
    h_chain = (torch.nn.functional.silu(gb).to(torch.bfloat16).float() * ub).to(torch.bfloat16).float().numpy()
    assert np.abs(h - h_chain).max() <= 2.0 ** -7 * np.abs(h_chain).max()
    assert (h == h_chain).mean() > 0.999
    # and the fp64 truth within tolerance
    truth = (g_ref / (1 + np.exp(-g_ref))) * u_ref
    assert np.abs(h - truth).max() / np.abs(truth).max() <= 1e-2


# Prompt-sized M (at least 512 rows, N a multiple of 128) runs the LDS-tiled GEMM:
# 128 x 128 output tiles, ragged last row tile, one k-tile (an odd count included).
PROMPT_CASES = [(512, 1024, 4096), (600, 2048, 1024), (1030, 3072, 1024), (777, 1024, 256), (520, 128, 128),
                (513, 384, 384)]


@pytest.mark.parametrize("m,k,n", PROMPT_CASES, ids=[f"M{m}-K{k}-N{n}" for m, k, n in PROMPT_CASES])
def test_prompt_rows_match_oracle(gpu, m, k, n):
    qw, qz, sc, x = _inputs(m, k, n, seed=2000 + m + k + n)
    ref = ow.linear(x.float().numpy(), qw, qz, sc, accumulate="fp64")
    w = W4A16Weight.from_numpy(qw, qz, sc, device=gpu)
    y = ops.linear(x.to(gpu), w)
    check_linear(y, ref)
    assert torch.equal(y, ops.linear(x.to(gpu), w)), "repeat call differs"


def test_prompt_rows_residual(gpu):
    m, k, n = 700, 2048, 1024
    qw, qz, sc, x = _inputs(m, k, n, seed=41)
    res = torch.randn(m, n, generator=torch.Generator().manual_seed(42)).to(torch.bfloat16)
    lin = ow.linear(x.float().numpy(), qw, qz, sc, accumulate="fp64")
    ref = lin + res.float().numpy()
    out = res.clone().to(gpu)
    y = ops.linear(x.to(gpu), W4A16Weight.from_numpy(qw, qz, sc, device=gpu), residual=out, out=out)
    err = np.abs(y.float().cpu().numpy() - ref)
    bound = 2.0 ** -8 * (np.abs(lin) + np.abs(ref)) * 1.01 + 1e-4 * np.abs(ref).max()
    assert (err <= bound).all()


def test_prompt_rows_gate_up(gpu):
    m, k, inter = 600, 1024, 3072
    gate = ow.synthetic_tensors(k, inter, seed=43)
    up = ow.synthetic_tensors(k, inter, seed=44)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(45)).to(torch.bfloat16)
    g_ref = ow.linear(x.float().numpy(), *gate, accumulate="fp64")
    u_ref = ow.linear(x.float().numpy(), *up, accumulate="fp64")
    w = W4A16Weight.from_numpy(*interleave_gate_up(gate, up), device=gpu)
    g, u = ops.gate_up(x.to(gpu), w, swiglu=False)
    check_linear(g, g_ref)
    check_linear(u, u_ref)
    h = ops.gate_up(x.to(gpu), w, swiglu=True).float().cpu()
    h_chain = (torch.nn.functional.silu(g.float().cpu()).to(torch.bfloat16).float() * u.float().cpu())
    h_chain = h_chain.to(torch.bfloat16).float()
    assert (h - h_chain).abs().max() <= 2.0 ** -7 * h_chain.abs().max()
    assert (h == h_chain).float().mean() > 0.999


def test_prompt_rows_other_widths(gpu):
    """N not a multiple of 128 stays on the 16-row-tile kernel at any M."""
    m, k, n = 640, 1024, 192
    qw, qz, sc, x = _inputs(m, k, n, seed=46)
    ref = ow.linear(x.float().numpy(), qw, qz, sc, accumulate="fp64")
    check_linear(ops.linear(x.to(gpu), W4A16Weight.from_numpy(qw, qz, sc, device=gpu)), ref)


def test_golden_fixture_on_gpu(gpu):
    """The brute-force fixture (tests/golden/make_golden.py): bit-exact weights, linear within tolerance."""
    from pathlib import Path
    g = np.load(Path(__file__).resolve().parent / "golden" / "w4a16_small.npz")
    w = W4A16Weight.from_numpy(g["qweight"], g["qzeros"], g["scales"], device=gpu)
    assert np.array_equal(ops.dequantize(w).cpu().numpy().view(np.uint32), g["W"].view(np.uint32))
    x = torch.from_numpy(g["x"]).to(torch.bfloat16)
    assert torch.equal(x.float(), torch.from_numpy(g["x"])), "fixture activations are bf16 values"
    check_linear(ops.linear(x.to(gpu), w), g["y"])


NORM_CASES = [(1, 1024, 4096), (8, 1024, 4096), (16, 1024, 6144), (33, 2048, 4096), (64, 1024, 1024),
              (5, 4096, 512), (16, 2048, 12288), (16, 1024, 1024), (7, 1024, 2048),
              (3, 128, 256), (2, 8192, 256)]   # one group (most waves idle); K past the old 4096 limit


def check_rounding_of_activations(fused: torch.Tensor, unfused: torch.Tensor, xn: np.ndarray, w_nk: np.ndarray):
    """The fused kernel multiplies bf16(x * gamma) and scales each row's sums by its
    bf16 1 / rms; the unfused pair multiplies bf16(bf16(x * inv) * gamma).  Both
    activations are within 1.5 bf16 half-units of the same real number x * inv *
    gamma, so the outputs may differ by at most 2^-7 sum_k |xn_k| |W_nk|, plus each
    output's own bf16 rounding (2^-9 relative each).  A bound from the arithmetic,
    with no tolerance fitted to the kernel."""
    f = fused.float().cpu().numpy().astype(np.float64)
    u = unfused.float().cpu().numpy().astype(np.float64)
    budget = 2.0 ** -7 * (np.abs(xn.astype(np.float64)) @ np.abs(w_nk.astype(np.float64)).T)
    bound = budget * 1.01 + 2.0 ** -9 * (np.abs(f) + np.abs(u)) * 1.01 + 1e-6
    err = np.abs(f - u)
    assert (err <= bound).all(), f"{(err > bound).sum()} outputs beyond the rounding budget; worst {err.max():.4e}"


@pytest.mark.parametrize("m,k,n", NORM_CASES, ids=[f"M{m}-K{k}-N{n}" for m, k, n in NORM_CASES])
def test_rmsnorm_linear_fused(gpu, m, k, n):
    """RMSNorm inside the linear kernel: within the linear bar of the oracle (bf16
    RMSNorm chain, fp64 product), and within the activation-rounding budget of the
    unfused rmsnorm-then-linear pair; two calls give the same bits."""
    from oracle import qwen3 as oq
    qw, qz, sc, x = _inputs(m, k, n, seed=77 + m + k)
    x = (x.float() * 3.0).to(torch.bfloat16)           # residual-stream-like magnitude
    gam = (torch.rand(k, generator=torch.Generator().manual_seed(m)) * 0.2 + 0.9).to(torch.bfloat16)
    w = W4A16Weight.from_numpy(qw, qz, sc, device=gpu)
    xd, gd = x.to(gpu), gam.to(gpu)
    fused = ops.rmsnorm_linear(xd, gd, 1e-6, w)
    assert torch.equal(fused, ops.rmsnorm_linear(xd, gd, 1e-6, w)), "repeat call differs"
    unfused = ops.linear(ops.rmsnorm(xd, gd, 1e-6), w)
    xn = oq.rmsnorm(x.float(), gam.float(), 1e-6, oq._Round("bf16")).numpy()
    ref = ow.linear(xn, qw, qz, sc, accumulate="fp64")
    assert np.abs(fused.float().cpu().numpy() - ref).max() / np.abs(ref).max() <= 1e-2
    check_rounding_of_activations(fused, unfused, xn, ow.dequantize(qw, qz, sc))


@pytest.mark.parametrize("m,k,inter", [(1, 1024, 3072), (16, 1024, 3072), (40, 2048, 6144)])
def test_rmsnorm_gate_up_fused(gpu, m, k, inter):
    """Paired outputs within the activation-rounding budget of the unfused pair; the
    SwiGLU output is the bf16 chain of the fused kernel's own gate and up values."""
    from oracle import qwen3 as oq
    gate = ow.synthetic_tensors(k, inter, seed=21)
    up = ow.synthetic_tensors(k, inter, seed=22)
    xc = (torch.randn(m, k, generator=torch.Generator().manual_seed(23)) * 3.0).to(torch.bfloat16)
    gamc = (torch.rand(k, generator=torch.Generator().manual_seed(24)) * 0.2 + 0.9).to(torch.bfloat16)
    x, gam = xc.to(gpu), gamc.to(gpu)
    w = W4A16Weight.from_numpy(*interleave_gate_up(gate, up), device=gpu)
    xn_gpu = ops.rmsnorm(x, gam, 1e-6)
    xn = oq.rmsnorm(xc.float(), gamc.float(), 1e-6, oq._Round("bf16")).numpy()
    g1, u1 = ops.rmsnorm_gate_up(x, gam, 1e-6, w, swiglu=False)
    g2, u2 = ops.gate_up(xn_gpu, w, swiglu=False)
    check_rounding_of_activations(g1, g2, xn, ow.dequantize(*gate))
    check_rounding_of_activations(u1, u2, xn, ow.dequantize(*up))
    h = ops.rmsnorm_gate_up(x, gam, 1e-6, w, swiglu=True).float().cpu()
    gb, ub = g1.float().cpu(), u1.float().cpu()
    h_chain = (torch.nn.functional.silu(gb).to(torch.bfloat16).float() * ub).to(torch.bfloat16).float()
    assert (h - h_chain).abs().max() <= 2.0 ** -7 * h_chain.abs().max()
    assert (h == h_chain).float().mean() > 0.999


def _random_cases(n_cases: int, seed: int):
    """Seeded random shapes for every linear form: M from 1 to 96 (prompt rows from 512
    for the GEMM form), K any multiple of 128 up to 4096, N any multiple of 16 (of 128 for
    the GEMM), within a size each oracle call finishes in
    about a second.  The paired layout interleaves gate and up in 32-column blocks, so a
    paired N is a multiple of 64."""
    rs = np.random.RandomState(seed)
    forms = ["plain", "residual", "norm", "paired", "prompt"]
    cases = []
    while len(cases) < n_cases:
        form = forms[len(cases) % len(forms)]
        k = 128 * int(rs.randint(1, 33))
        if form == "prompt":
            m, n = int(rs.randint(512, 901)), 128 * int(rs.randint(1, 17))
        else:
            m = int(rs.randint(1, 97))
            n = 64 * int(rs.randint(1, 49)) if form == "paired" else 16 * int(rs.randint(1, 257))
        if k * n <= 6 << 20 and m * k * n <= 1536 << 20:
            cases.append((form, m, k, n))
    return cases


RANDOM_CASES = _random_cases(25, seed=2026)


@pytest.mark.parametrize("form,m,k,n", RANDOM_CASES, ids=[f"{f}-M{m}-K{k}-N{n}" for f, m, k, n in RANDOM_CASES])
def test_random_shapes_match_oracle(gpu, form, m, k, n):
    """Shapes off the model's list, each form against the fp64 oracle at the bars above
    (paired: both outputs; residual: two roundings; fused norm: the bf16 RMSNorm chain
    then the linear bar)."""
    seed = 3000 + m + 7 * k + 13 * n
    if form == "paired":
        gate, up = ow.synthetic_tensors(k, n // 2, seed=seed), ow.synthetic_tensors(k, n // 2, seed=seed + 1)
        x = torch.randn(m, k, generator=torch.Generator().manual_seed(seed + 2)).to(torch.bfloat16)
        w = W4A16Weight.from_numpy(*interleave_gate_up(gate, up), device=gpu)
        g, u = ops.gate_up(x.to(gpu), w, swiglu=False)
        check_linear(g, ow.linear(x.float().numpy(), *gate, accumulate="fp64"))
        check_linear(u, ow.linear(x.float().numpy(), *up, accumulate="fp64"))
        return
    qw, qz, sc, x = _inputs(m, k, n, seed=seed)
    w = W4A16Weight.from_numpy(qw, qz, sc, device=gpu)
    if form == "norm":
        from oracle import qwen3 as oq
        x = (x.float() * 3.0).to(torch.bfloat16)
        gam = (torch.rand(k, generator=torch.Generator().manual_seed(seed + 3)) * 0.2 + 0.9).to(torch.bfloat16)
        y = ops.rmsnorm_linear(x.to(gpu), gam.to(gpu), 1e-6, w)
        xn = oq.rmsnorm(x.float(), gam.float(), 1e-6, oq._Round("bf16")).numpy()
        ref = ow.linear(xn, qw, qz, sc, accumulate="fp64")
        assert np.abs(y.float().cpu().numpy() - ref).max() / np.abs(ref).max() <= 1e-2
        check_rounding_of_activations(y, ops.linear(ops.rmsnorm(x.to(gpu), gam.to(gpu), 1e-6), w), xn,
                                      ow.dequantize(qw, qz, sc))
        return
    lin = ow.linear(x.float().numpy(), qw, qz, sc, accumulate="fp64")
    if form == "residual":
        res = torch.randn(m, n, generator=torch.Generator().manual_seed(seed + 4)).to(torch.bfloat16)
        out = res.clone().to(gpu)
        y = ops.linear(x.to(gpu), w, residual=out, out=out)
        ref = lin + res.float().numpy()
        err = np.abs(y.float().cpu().numpy() - ref)
        assert (err <= 2.0 ** -8 * (np.abs(lin) + np.abs(ref)) * 1.01 + 1e-4 * np.abs(ref).max()).all()
        return
    y = ops.linear(x.to(gpu), w)
    check_linear(y, lin)
    assert torch.equal(y, ops.linear(x.to(gpu), w)), "repeat call differs"
