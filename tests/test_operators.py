"""The reference operator surface: constructor checks and argument order (CPU),
and on the GPU that each operator gives the same bits as the functional layer."""

import pytest
import torch

from oracle import w4a16 as ow
from torch2iron_amd import formats, model as gm, operators as O, ops

BF16 = torch.bfloat16


@pytest.mark.parametrize("ctor", [
    lambda: O.W4A16GEMV(M=3072, K=1000),
    lambda: O.W4A16GEMV(M=3072, K=1024, group_size=64),
    lambda: O.W4A16GEMM(M=0, K=1024, N=4096),
    lambda: O.W4A16GEMM(M=16, K=1024, N=4000),
    lambda: O.W4A16KGroupGEMM(M=16, K=1024, N=4096, k_group=3),
    lambda: O.W4A16PairedKGroupGEMM(M=16, K=640, N=3072),
    lambda: O.Qwen3FusedQKVProjection(in_features=1000, out_features=4096),
    lambda: O.Qwen3FusedUpGateProjection(in_features=1024, out_features=3072, rms_norm_epsilon=0.0),
    lambda: O.Qwen3FusedLinearResidualProjection(in_features=2048, out_features=1000),
])
def test_constructor_checks_raise_value_error(ctor):
    with pytest.raises(ValueError):
        ctor()


def test_argument_order_matches_the_reference():
    gemv = O.W4A16GEMV(M=3072, K=1024).get_arg_spec()
    assert [a.direction for a in gemv] == ["in", "in", "out"] and gemv[1].shape == (1024,)   # (W, x, y)
    gemm = O.W4A16GEMM(M=16, K=1024, N=4096).get_arg_spec()
    assert gemm[0].shape == (16, 1024) and gemm[2].shape == (16, 4096)                       # (A, W, C)
    paired = O.W4A16PairedKGroupGEMM(M=8, K=1024, N=3072).get_arg_spec()
    assert [a.direction for a in paired] == ["in", "in", "out", "out"]                        # (A, W, C0, C1)
    res = O.Qwen3FusedLinearResidualProjection(2048, 1024, rows=8).get_arg_spec()
    assert res[0].shape == (8, 2048) and res[1].shape == (8, 1024)                            # (ctx, residual, W, out)


def test_weight_buffer_is_checked():
    op = O.W4A16GEMM(M=4, K=256, N=64)
    w = formats.W4A16Weight.from_numpy(*ow.synthetic_tensors(256, 128, seed=1))
    with pytest.raises(ValueError):
        op(torch.zeros(4, 256, dtype=BF16), w, torch.zeros(4, 64, dtype=BF16))


@pytest.mark.gpu
def test_operators_match_functional_layer(gpu):
    g = torch.Generator().manual_seed(0)
    w = formats.W4A16Weight.from_numpy(*ow.synthetic_tensors(1024, 3072, seed=2), device=gpu)
    x = torch.randn(1024, generator=g).to(BF16).to(gpu)
    y = torch.empty(3072, dtype=BF16, device=gpu)
    O.W4A16GEMV(M=3072, K=1024)(w, x, y)
    assert torch.equal(y, ops.linear(x, w))
    a = torch.randn(16, 1024, generator=g).to(BF16).to(gpu)
    c = torch.empty(16, 3072, dtype=BF16, device=gpu)
    O.W4A16KGroupGEMM(M=16, K=1024, N=3072, k_group=4)(a, w, c)
    assert torch.equal(c, ops.linear(a, w))
    gate, up = ow.synthetic_tensors(1024, 3072, seed=3), ow.synthetic_tensors(1024, 3072, seed=4)
    wp = formats.W4A16Weight.from_numpy(*formats.interleave_gate_up(gate, up), device=gpu)
    c0, c1 = torch.empty_like(c), torch.empty_like(c)
    O.W4A16PairedKGroupGEMM(M=16, K=1024, N=3072)(a, wp, c0, c1)
    r0, r1 = ops.gate_up(a, wp, swiglu=False)
    assert torch.equal(c0, r0) and torch.equal(c1, r1)
    nw = torch.ones(1024, dtype=BF16, device=gpu)
    h = torch.empty(16, 3072, dtype=BF16, device=gpu)
    O.Qwen3FusedUpGateProjection(1024, 3072, rows=16)(a, nw, wp, h)
    assert torch.equal(h, ops.rmsnorm_gate_up(a, nw, 1e-6, wp, swiglu=True))
    wo = formats.W4A16Weight.from_numpy(*ow.synthetic_tensors(3072, 1024, seed=5), device=gpu)
    res = torch.randn(16, 1024, generator=g).to(BF16).to(gpu)
    out = torch.empty_like(res)
    O.Qwen3FusedLinearResidualProjection(3072, 1024, rows=16)(h, res, wo, out)
    assert torch.equal(out, ops.linear(h, wo, residual=res))
