"""Pins of the W4A16 oracle (CPU): known answers, the brute-force golden fixture,
exactness of the fp32 dequantisation and properties of the linear.

Each check is chosen so that a plausible slip in the oracle fails it: a wrong
nibble order, a dropped "+1" on the zero point, a transposed operand, a group
index off by one, or an inexact product.
"""

from pathlib import Path

import numpy as np
import pytest

from oracle import w4a16 as ow

GOLDEN = Path(__file__).resolve().parent / "golden" / "w4a16_small.npz"


def test_nibble_order_known_words():
    words = np.array([0x00000000, 0xFFFFFFFF, 0x76543210, 0xFEDCBA98], dtype=np.uint32).view(np.int32)
    nib = ow.unpack_int32_nibbles(words)
    assert nib.tolist() == [[0] * 8, [15] * 8, list(range(8)), list(range(8, 16))]


def test_qweight_layout_known_answer():
    # K = 16, N = 2: column 0 holds k = 0..15 counting up, column 1 counting down
    qweight = np.array([[0x76543210, 0x89ABCDEF], [0xFEDCBA98, 0x01234567]], dtype=np.uint32).view(np.int32)
    q = ow.unpack_qweight(qweight, 16, 2)
    assert q.shape == (2, 16)
    assert q[0].tolist() == list(range(16))
    assert q[1].tolist() == list(range(15, -1, -1))


def test_zero_point_plus_one_convention():
    # stored zero nibble 7 -> z = 8: q = 8 dequantises to exactly 0, q = 9 to +s, q = 7 to -s
    k, n = 128, 8
    q = np.full((n, k), 8, dtype=np.int64)
    q[1, :] = 9
    q[2, :] = 7
    qweight = ow.pack_qweight(q)
    qzeros = np.array([[0x77777777]], dtype=np.uint32).view(np.int32)
    scales = np.full((1, n), 0.0125, dtype=np.float16)
    w = ow.dequantize(qweight, qzeros, scales)
    s = np.float32(np.float16(0.0125))
    assert np.all(w[0] == 0) and np.all(w[1] == s) and np.all(w[2] == -s)
    # zeros span 1..16 for stored 0..15
    z = ow.unpack_qzeros(np.array([[0xF0E1D2C3]], dtype=np.uint32).view(np.int32), 8)
    assert z.tolist() == [[4, 13, 3, 14, 2, 15, 1, 16]]


def test_pack_unpack_roundtrip():
    rng = np.random.default_rng(0)
    q = rng.integers(0, 16, size=(24, 256))
    assert np.array_equal(ow.unpack_qweight(ow.pack_qweight(q), 256, 24), q)
    zs = rng.integers(0, 16, size=(2, 24))
    assert np.array_equal(ow.unpack_qzeros(ow.pack_qzeros(zs), 24), zs + 1)


def test_golden_fixture_dequant_and_linear():
    g = np.load(GOLDEN)
    w = ow.dequantize(g["qweight"], g["qzeros"], g["scales"], int(g["group_size"]))
    assert np.array_equal(w.view(np.uint32), g["W"].view(np.uint32))
    y = ow.linear(g["x"], g["qweight"], g["qzeros"], g["scales"], int(g["group_size"]))
    assert np.allclose(y, g["y"], rtol=1e-12, atol=1e-12 * np.abs(g["y"]).max())


def test_dequant_is_exact_in_fp32():
    qw, qz, sc = ow.synthetic_tensors(1024, 512, seed=5)
    w32 = ow.dequantize(qw, qz, sc)
    q = ow.unpack_qweight(qw, 1024, 512).astype(np.float64)
    z = ow.unpack_qzeros(qz, 512).astype(np.float64)
    s = sc.astype(np.float64)
    w64 = (q.reshape(512, 8, 128) - z.T[:, :, None]) * s.T[:, :, None]
    assert np.array_equal(w32.astype(np.float64), w64.reshape(512, 1024))


def test_scales_stored_transposed_are_accepted():
    qw, qz, sc = ow.synthetic_tensors(256, 64, seed=6)
    assert np.array_equal(ow.dequantize(qw, qz, sc), ow.dequantize(qw, qz, np.ascontiguousarray(sc.T)))
    with pytest.raises(ValueError):
        ow.dequantize(qw, qz, sc[:1])


def test_linear_unit_vectors_pick_columns():
    """x = e_k gives W[:, k]: ties the linear to the dequantised layout (catches a transposed W)."""
    qw, qz, sc = ow.synthetic_tensors(256, 64, seed=7)
    w = ow.dequantize(qw, qz, sc)
    ks = [0, 7, 8, 127, 128, 255]
    x = np.zeros((len(ks), 256), dtype=np.float32)
    x[np.arange(len(ks)), ks] = 1.0
    y = ow.linear(x, qw, qz, sc)
    assert np.array_equal(y, w[:, ks].T.astype(np.float64))


def test_linear_group_loop_and_linearity():
    qw, qz, sc = ow.synthetic_tensors(512, 128, seed=8)
    rng = np.random.default_rng(9)
    # small integers: 2 x1 - 3 x2 is exact in fp32, so linearity must hold to fp64 rounding
    x1 = rng.integers(-8, 9, size=(4, 512)).astype(np.float32)
    x2 = rng.integers(-8, 9, size=(4, 512)).astype(np.float32)
    y1 = ow.linear(x1, qw, qz, sc)
    y2 = ow.linear(x2, qw, qz, sc)
    y12 = ow.linear(2.0 * x1 - 3.0 * x2, qw, qz, sc)
    assert np.allclose(y12, 2 * y1 - 3 * y2, rtol=1e-12, atol=1e-9)
    y32 = ow.linear(x1, qw, qz, sc, accumulate="fp32")      # model.py:133-146 group loop
    assert np.abs(y32 - y1).max() <= 1e-5 * np.abs(y1).max()


def test_bf16_round_matches_torch():
    import torch
    a = np.random.default_rng(10).standard_normal(10000).astype(np.float32) * 100
    a[:3] = [np.inf, -0.0, 1e-40]
    ours = ow.bf16_round(a)
    ref = torch.from_numpy(a).to(torch.bfloat16).float().numpy()
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))
