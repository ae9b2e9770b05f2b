"""Decode-linear tiles (t2i_w4a16_tile_qweight / t2i_w4a16_linear_tiles).

The tile layout is the documented permutation of qweight's words (checked by a
reshape and, on a small weight, word by word), and every linear form over tiles
gives the AutoGPTQ entry points' outputs bit for bit: the same kernels and
arithmetic, only the weight words read from another place.  The AutoGPTQ
entry points are themselves held to the fp64 oracle in test_gpu_linear.py.
"""

import numpy as np
import pytest
import torch

from oracle import w4a16 as ow
from torch2iron_amd import _lib, ops
from torch2iron_amd.formats import W4A16Weight, interleave_gate_up

pytestmark = pytest.mark.gpu

QWEN3_06B = [(1024, 4096), (2048, 1024), (1024, 6144), (3072, 1024)]
QWEN3_17B = [(2048, 4096), (2048, 2048), (2048, 12288), (6144, 2048)]

PLAIN = [(m, k, n) for (k, n) in QWEN3_06B for m in (1, 8, 16, 32, 64)]
PLAIN += [(m, k, n) for (k, n) in QWEN3_17B for m in (1, 16, 64)]
# ragged rows, short row tiles, two m-tiles a workgroup, rows up to the prompt GEMM's
PLAIN += [(3, 1024, 3072), (13, 2048, 1024), (6, 3072, 1024), (48, 1024, 6144), (100, 2048, 1024),
          (300, 1024, 4096), (511, 1024, 256), (5, 128, 64), (17, 256, 48)]
NORM = [(1, 1024, 4096), (16, 1024, 4096), (64, 1024, 4096), (16, 2048, 4096), (7, 1024, 2048)]
PAIRED = [(1, 1024, 6144), (16, 1024, 6144), (64, 1024, 6144), (8, 2048, 12288), (33, 1024, 3072)]


def _weight(k, n, seed, dev):
    return W4A16Weight.from_numpy(*ow.synthetic_tensors(k, n, seed=seed), device=dev)


def _tiled(w):
    """A second weight object over the same tensors, with tiles."""
    return ops.tile_weight(W4A16Weight(w.qweight, w.qzeros, w.scales, w.group_size))


def _x(m, k, seed, dev, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(m, k, generator=g) * scale).to(torch.bfloat16).to(dev)


@pytest.mark.parametrize("k,n", [(1024, 4096), (3072, 1024), (2048, 12288), (256, 48)])
def test_tiles_are_the_documented_permutation(gpu, k, n):
    w = ops.tile_weight(_weight(k, n, seed=k + n, dev=gpu))
    t = w.tiles.cpu().numpy().view(np.uint32)
    q = w.qweight.cpu().numpy().view(np.uint32)   # [K/8, N]
    groups = k // 128
    # word row 16 g + 4 j + r, column 16 cb + c  ->  tile (cb, g), word (16 r + c) * 4 + j
    expect = q.reshape(groups, 4, 4, n // 16, 16).transpose(3, 0, 2, 4, 1).reshape(-1)
    assert np.array_equal(t, expect)


def test_tiles_word_by_word_small(gpu):
    k, n = 256, 32
    w = ops.tile_weight(_weight(k, n, seed=5, dev=gpu))
    t = w.tiles.cpu().numpy().view(np.uint32)
    q = w.qweight.cpu().numpy().view(np.uint32)
    groups = k // 128
    for cb in range(n // 16):
        for g in range(groups):
            for r in range(4):
                for c in range(16):
                    for j in range(4):
                        assert t[(cb * groups + g) * 256 + (16 * r + c) * 4 + j] == q[16 * g + 4 * j + r, 16 * cb + c]


@pytest.mark.parametrize("m,k,n", PLAIN, ids=[f"M{m}-K{k}-N{n}" for m, k, n in PLAIN])
def test_linear_over_tiles_is_bit_identical(gpu, m, k, n):
    seed = 7 * m + k + 3 * n
    w = _weight(k, n, seed, gpu)
    wt = _tiled(w)
    x = _x(m, k, seed + 1, gpu)
    assert torch.equal(ops.linear(x, wt), ops.linear(x, w))
    res = _x(m, n, seed + 2, gpu)
    a, b = res.clone(), res.clone()
    assert torch.equal(ops.linear(x, wt, residual=a, out=a), ops.linear(x, w, residual=b, out=b))


@pytest.mark.parametrize("m,k,n", NORM, ids=[f"M{m}-K{k}-N{n}" for m, k, n in NORM])
def test_rmsnorm_linear_over_tiles_is_bit_identical(gpu, m, k, n):
    seed = 11 * m + k + n
    w = _weight(k, n, seed, gpu)
    x = _x(m, k, seed + 1, gpu, scale=3.0)
    gam = (torch.rand(k, generator=torch.Generator().manual_seed(seed + 2)) * 0.2 + 0.9).to(torch.bfloat16).to(gpu)
    assert torch.equal(ops.rmsnorm_linear(x, gam, 1e-6, _tiled(w)), ops.rmsnorm_linear(x, gam, 1e-6, w))


@pytest.mark.parametrize("m,k,n", PAIRED, ids=[f"M{m}-K{k}-N{n}" for m, k, n in PAIRED])
def test_gate_up_over_tiles_is_bit_identical(gpu, m, k, n):
    seed = 13 * m + k + n
    gate, up = ow.synthetic_tensors(k, n // 2, seed=seed), ow.synthetic_tensors(k, n // 2, seed=seed + 1)
    w = W4A16Weight.from_numpy(*interleave_gate_up(gate, up), device=gpu)
    wt = _tiled(w)
    x = _x(m, k, seed + 2, gpu)
    assert torch.equal(ops.gate_up(x, wt, swiglu=True), ops.gate_up(x, w, swiglu=True))
    gt, ut = ops.gate_up(x, wt, swiglu=False)
    g0, u0 = ops.gate_up(x, w, swiglu=False)
    assert torch.equal(gt, g0) and torch.equal(ut, u0)
    gam = (torch.rand(k, generator=torch.Generator().manual_seed(seed + 3)) * 0.2 + 0.9).to(torch.bfloat16).to(gpu)
    assert torch.equal(ops.rmsnorm_gate_up(x, gam, 1e-6, wt, swiglu=True),
                       ops.rmsnorm_gate_up(x, gam, 1e-6, w, swiglu=True))
    gt, ut = ops.rmsnorm_gate_up(x, gam, 1e-6, wt, swiglu=False)
    g0, u0 = ops.rmsnorm_gate_up(x, gam, 1e-6, w, swiglu=False)
    assert torch.equal(gt, g0) and torch.equal(ut, u0)


def test_decode_rows_read_the_tiles_and_prompt_rows_the_autogptq_words(gpu):
    """Which words a call reads: with the AutoGPTQ words zeroed after tiling, a decode-
    sized call of a tile-reading plan (16-column blocks) still gives the original
    outputs and a prompt-sized call changes (it reads qweight)."""
    k, n = 1024, 1024
    w = _weight(k, n, seed=21, dev=gpu)
    x = _x(ops.PROMPT_GEMM_ROWS, k, seed=22, dev=gpu)
    small, big = ops.linear(x[:16], w), ops.linear(x, w)
    wt = _tiled(W4A16Weight(w.qweight.clone(), w.qzeros, w.scales))
    wt.qweight.zero_()
    assert torch.equal(ops.linear(x[:16], wt), small)
    assert not torch.equal(ops.linear(x, wt), big)


def test_tiles_entry_point_without_qweight(gpu):
    """With qweight NULL every decode plan reads the tiles (bit-identical, including
    the plans that would read qweight when given it) and prompt rows are refused."""
    lib = _lib.load()
    for m, k, n, norm in [(16, 1024, 1024, False), (32, 1024, 6144, False), (64, 1024, 4096, False),
                          (16, 1024, 6144, True)]:
        w = ops.tile_weight(_weight(k, n, seed=31 + m, dev=gpu))
        x = _x(m, k, seed=32 + m, dev=gpu)
        gam = torch.full((k,), 1.0, dtype=torch.bfloat16, device=gpu) if norm else None
        y = torch.empty(m, n, dtype=torch.bfloat16, device=gpu)
        rc = lib.t2i_w4a16_linear_tiles(x.data_ptr(), m, _lib.ptr(gam), 1e-6, None, w.tiles.data_ptr(),
                                        w.qzeros.data_ptr(), w.scales.data_ptr(), k, n, 128, _lib.T2I_TILES_STORE,
                                        None, y.data_ptr(), None, _lib.stream_handle(x.device))
        assert rc == 0, _lib.load().t2i_last_error()
        ref = ops.rmsnorm_linear(x, gam, 1e-6, _weight(k, n, seed=31 + m, dev=gpu)) if norm else \
            ops.linear(x, _weight(k, n, seed=31 + m, dev=gpu))
        assert torch.equal(y, ref), (m, k, n, norm)
    k, n = 1024, 1024
    w = ops.tile_weight(_weight(k, n, seed=41, dev=gpu))
    x = _x(ops.PROMPT_GEMM_ROWS, k, seed=42, dev=gpu)
    y = torch.empty(ops.PROMPT_GEMM_ROWS, n, dtype=torch.bfloat16, device=gpu)
    rc = lib.t2i_w4a16_linear_tiles(x.data_ptr(), ops.PROMPT_GEMM_ROWS, None, 0.0, None, w.tiles.data_ptr(),
                                    w.qzeros.data_ptr(), w.scales.data_ptr(), k, n, 128, _lib.T2I_TILES_STORE,
                                    None, y.data_ptr(), None, None)
    assert rc == _lib.T2I_ERR_SHAPE


def _random_cases(n_cases: int, seed: int):
    rs = np.random.RandomState(seed)
    forms = ["plain", "residual", "norm", "paired", "norm_paired"]
    cases = []
    while len(cases) < n_cases:
        form = forms[len(cases) % len(forms)]
        k = 128 * int(rs.randint(1, 25))
        m = int(rs.randint(1, 97))
        n = 64 * int(rs.randint(1, 97)) if "paired" in form else 16 * int(rs.randint(1, 385))
        if k * n <= 6 << 20:
            cases.append((form, m, k, n))
    return cases


RANDOM_CASES = _random_cases(30, seed=77)


@pytest.mark.parametrize("form,m,k,n", RANDOM_CASES, ids=[f"{f}-M{m}-K{k}-N{n}" for f, m, k, n in RANDOM_CASES])
def test_random_shapes_over_tiles_are_bit_identical(gpu, form, m, k, n):
    """Shapes off the model's list (column-block counts that are odd or not multiples of
    8, ragged rows), every form: tiles against the AutoGPTQ words, bit for bit."""
    seed = 5000 + m + 7 * k + 13 * n
    x = _x(m, k, seed, gpu, scale=2.0)
    gam = (torch.rand(k, generator=torch.Generator().manual_seed(seed + 1)) * 0.2 + 0.9).to(torch.bfloat16).to(gpu)
    if "paired" in form:
        gate, up = ow.synthetic_tensors(k, n // 2, seed=seed + 2), ow.synthetic_tensors(k, n // 2, seed=seed + 3)
        w = W4A16Weight.from_numpy(*interleave_gate_up(gate, up), device=gpu)
        wt = _tiled(w)
        if form == "norm_paired":
            assert torch.equal(ops.rmsnorm_gate_up(x, gam, 1e-6, wt, swiglu=True),
                               ops.rmsnorm_gate_up(x, gam, 1e-6, w, swiglu=True))
        else:
            g1, u1 = ops.gate_up(x, wt, swiglu=False)
            g0, u0 = ops.gate_up(x, w, swiglu=False)
            assert torch.equal(g1, g0) and torch.equal(u1, u0)
        return
    w = _weight(k, n, seed + 4, gpu)
    wt = _tiled(w)
    if form == "norm":
        assert torch.equal(ops.rmsnorm_linear(x, gam, 1e-6, wt), ops.rmsnorm_linear(x, gam, 1e-6, w))
    elif form == "residual":
        res = _x(m, n, seed + 5, gpu)
        a, b = res.clone(), res.clone()
        assert torch.equal(ops.linear(x, wt, residual=a, out=a), ops.linear(x, w, residual=b, out=b))
    else:
        assert torch.equal(ops.linear(x, wt), ops.linear(x, w))


# ---- chained RMSNorm between decode linears ----
CHAIN_SHAPES = [(1, 2048, 1024, 1024), (16, 2048, 1024, 4096), (16, 3072, 1024, 1024), (5, 2048, 2048, 4096),
                (13, 3072, 1024, 3072), (8, 3072, 1024, 6144), (32, 2048, 1024, 4096), (32, 2048, 2048, 4096),
                (64, 3072, 1024, 1024)]


@pytest.mark.parametrize("m,kp,h,nc", CHAIN_SHAPES, ids=[f"M{m}-K{kp}-H{h}-N{nc}" for m, kp, h, nc in CHAIN_SHAPES])
def test_chained_norm_matches_the_fused_norm(gpu, m, kp, h, nc):
    """Producer (o_proj/down shape kp -> h, residual) then consumer (h -> nc): the
    producer's y equals the plain residual linear bit for bit, its xg is exactly
    bf16(y * gamma) and its block sums match y**2 (fp32, summation order aside); the
    consumer equals rmsnorm_linear on y except where the order of the squares' sum
    moves the bf16 1/rms by one ulp (a row scaled by 1 +- 2^-8 at most)."""
    if not (ops.chain_supported(m, kp, h, ops.CHAIN_PRODUCER) and ops.chain_supported(m, h, nc, ops.CHAIN_CONSUMER)):
        pytest.skip("no chained form of this plan")
    seed = 31 * m + kp + h + nc
    wp = ops.tile_weight(_weight(kp, h, seed, gpu))
    wc = ops.tile_weight(_weight(h, nc, seed + 1, gpu))
    x = _x(m, kp, seed + 2, gpu)
    res = _x(m, h, seed + 3, gpu, scale=4.0)
    gam = (torch.rand(h, generator=torch.Generator().manual_seed(seed + 4)) * 0.2 + 0.9).to(torch.bfloat16).to(gpu)
    y_ref = ops.linear(x, wp, residual=res.clone(), out=torch.empty(m, h, dtype=torch.bfloat16, device=gpu))
    y = res.clone()
    xg = torch.empty(m, h, dtype=torch.bfloat16, device=gpu)
    ss = torch.full((m, h // 16), float("nan"), dtype=torch.float32, device=gpu)
    ops.linear_residual_next_norm(x, wp, y, y, gam, xg, ss)
    assert torch.equal(y, y_ref)
    assert torch.equal(xg, (y.float() * gam.float()).to(torch.bfloat16))
    ref_ss = (y.double() ** 2).reshape(m, h // 16, 16).sum(-1)
    assert torch.allclose(ss.double(), ref_ss, rtol=1e-6, atol=0)
    z = ops.prenormed_linear(xg, ss, 1e-6, wc)
    z_ref = ops.rmsnorm_linear(y, gam, 1e-6, wc)
    same_rows = (z == z_ref).all(dim=1)
    assert same_rows.float().mean() >= 0.75, f"{int(same_rows.sum())}/{m} rows identical"
    rel = ((z.float() - z_ref.float()).abs() / z_ref.float().abs().clamp_min(1e-3)).max()
    assert rel <= 2.0 ** -7, f"max relative difference {rel:.3e}"


@pytest.mark.parametrize("m", [8, 16])
def test_chained_norm_paired_consumer(gpu, m):
    h, inter = 1024, 3072
    if not ops.chain_supported(m, h, 2 * inter, ops.CHAIN_PAIRED_CONSUMER):
        pytest.skip("no chained form of this plan")
    seed = 4242 + m
    gate, up = ow.synthetic_tensors(h, inter, seed=seed), ow.synthetic_tensors(h, inter, seed=seed + 1)
    w = ops.tile_weight(W4A16Weight.from_numpy(*interleave_gate_up(gate, up), device=gpu))
    y = _x(m, h, seed + 2, gpu, scale=3.0)
    gam = (torch.rand(h, generator=torch.Generator().manual_seed(seed + 3)) * 0.2 + 0.9).to(torch.bfloat16).to(gpu)
    xg = (y.float() * gam.float()).to(torch.bfloat16)
    ss = (y.float() ** 2).reshape(m, h // 16, 16).sum(-1).contiguous()
    for swiglu in (True, False):
        got = ops.prenormed_gate_up(xg, ss, 1e-6, w, swiglu=swiglu)
        ref = ops.rmsnorm_gate_up(y, gam, 1e-6, w, swiglu=swiglu)
        pairs = [(got, ref)] if swiglu else list(zip(got, ref))
        for a, b in pairs:
            rel = ((a.float() - b.float()).abs() / b.float().abs().clamp_min(1e-3)).max()
            assert rel <= 2.0 ** -6, f"swiglu={swiglu}: max relative difference {rel:.3e}"
            assert (a == b).all(dim=1).float().mean() >= 0.75
