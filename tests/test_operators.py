"""The reference operator surface: construction with the reference's own call-site
arguments and constructor checks (CPU), and on the GPU that each operator gives
the same bits as the functional layer, and that a decode layer written as a
runlist of ``(op, *buffer_names)`` entries gives the same bits as the layer."""

import numpy as np
import pytest
import torch

from oracle import w4a16 as ow
from torch2iron_amd import formats, model as gm, operators as O, ops
from torch2iron_amd import runlist as R

BF16 = torch.bfloat16

# quantized_qwen3/batch_decode_fused.py:46-52, 74-77 (NPU tiling constants of the batch decoder)
COLUMNS, TILE_M, TILE_K, TILE_N, LM_TILE_N = 8, 8, 128, 64, 64


def _gemm_tile_m(rows):
    return 4 if rows <= 8 else TILE_M


def _n_shard_rows(n, tile_n):
    groups = n // (tile_n * COLUMNS)
    return next(r for r in (4, 3, 2, 1) if groups % r == 0)


@pytest.mark.parametrize("rows", [4, 8, 16, 32])
def test_batch_decode_builder_call_sites_construct(rows):
    """Every W4A16 operator exactly as ``batch_decode_fused.py:170-266`` builds it
    for Qwen3-0.6B (emb 1024, attn 2048, kv 1024, ffn 3072, padded lm_head 152064)."""
    tm = _gemm_tile_m(rows)
    common = dict(num_aie_columns=COLUMNS, num_aie_rows=rows // tm, tile_m=tm, tile_k=TILE_K, tile_n=TILE_N,
                  context=object())
    ops_ = [
        O.W4A16GEMM(M=rows, K=1024, N=2048, **common),
        O.W4A16KGroupGEMM(M=rows, K=1024, N=2048, k_group=4, **common),          # queries
        O.W4A16PairedKGroupGEMM(M=rows, K=1024, N=1024, k_group=2, **common),    # keys / values
        O.W4A16KGroupGEMM(M=rows, K=2048, N=1024, k_group=2, **common),          # attention output
        O.W4A16PairedKGroupGEMM(M=rows, K=1024, N=3072, k_group=2, **common),    # gate / up
        O.W4A16KGroupGEMM(M=rows, K=3072, N=1024, k_group=2, **common),          # down
        O.W4A16NShardGEMM(M=rows, K=1024, N=152064, num_aie_columns=COLUMNS,
                          num_aie_rows=_n_shard_rows(152064, LM_TILE_N), tile_m=tm, tile_k=TILE_K,
                          tile_n=LM_TILE_N, context=object()),
    ]
    for op in ops_:
        specs = op.get_arg_spec()
        assert specs[0].shape == (rows, op.K) and specs[0].direction == "in"       # (A, W, C[, C1])
        assert all(s.direction == "out" for s in specs[2:])


def test_codegen_gemv_call_sites_construct():
    """``W4A16GEMV`` exactly as the codegen factory ``_gemv`` builds it
    (``export/templates/decode_fused.py.j2:93-110``, values of
    ``generated/decode_fused.py:157-333`` for Qwen3-0.6B)."""
    for m, k, tsi, tso in [(2048, 1024, 4, 64), (1024, 1024, 8, 128), (1024, 2048, 2, 128),
                           (3072, 1024, 2, 384), (1024, 3072, 1, 128), (151936, 1024, 8, 128)]:
        op = O.W4A16GEMV(M=m, K=k, num_aie_columns=8, tile_size_input=tsi, tile_size_output=tso,
                         group_size=128, context=object())
        w, x, y = op.get_arg_spec()
        assert (w.direction, x.shape, y.shape) == ("in", (k,), (m,))               # (W, x, y)


def test_q4nx_call_sites_construct():
    """The Q4NX callables with the fields their smokes pass
    (``fast_qwen3/qkv_operator_smoke.py:208``, ``up_gate_operator_smoke.py:178``,
    ``o_projection_operator_smoke.py:127``, ``o_projection_residual_operator_smoke.py:139``)."""
    qkv = O.Q4NXFusedQKVProjection(in_features=1024, output_patches=8, rms_norm_epsilon=1e-6, context=object())
    assert [s.shape for s in qkv.get_arg_spec()] == [(1024,), (1024,), ("W4A16Weight", 1024, 1536), (1536,)]
    ug = O.Q4NXFusedUpGateProjection(in_features=1024, output_patches=4, rms_norm_epsilon=1e-6)
    assert ug.get_arg_spec()[3].shape == (4 * 2 * 64,)
    lin = O.Q4NXFusedLinearProjection(in_features=2048, output_patches=8, context=object())
    assert [s.direction for s in lin.get_arg_spec()] == ["in", "in", "out"]
    res = O.Q4NXFusedLinearResidualProjection(in_features=2048, output_patches=8)
    assert [s.shape for s in res.get_arg_spec()] == [(2048,), (512,), ("W4A16Weight", 2048, 512), (8, 64)]


@pytest.mark.parametrize("ctor", [
    # the reference's own checks
    lambda: O.W4A16GEMV(M=3072, K=1000),
    lambda: O.W4A16GEMV(M=3072, K=1024, kernel_vector_size=16),
    lambda: O.W4A16GEMV(M=3072, K=1024, tile_size_input=4, tile_size_output=6),
    lambda: O.W4A16GEMM(M=12, K=1024, N=4096),                                    # M % (tile_m * rows)
    lambda: O.W4A16GEMM(M=32, K=1024, N=4000),                                    # N % (tile_n * cols)
    lambda: O.W4A16GEMM(M=32, K=1024, N=4096, tile_k=64),                         # tile_k != group_size
    lambda: O.W4A16GEMM(M=36, K=1024, N=4096, tile_m=6, num_aie_rows=1),
    lambda: O.W4A16GEMM(M=32, K=1024, N=4096, tile_n=24),
    lambda: O.W4A16KGroupGEMM(M=32, K=1024, N=4096, k_group=3),
    lambda: O.W4A16PairedKGroupGEMM(M=32, K=640, N=3072),
    lambda: O.W4A16NShardGEMM(M=8, K=1024, N=151936, num_aie_rows=3),
    lambda: O.Q4NXFusedQKVProjection(in_features=1152),
    lambda: O.Q4NXFusedQKVProjection(in_features=1024, out_rows=32),
    lambda: O.Q4NXFusedUpGateProjection(in_features=1024, output_patches=9),
    lambda: O.Q4NXFusedUpGateProjection(in_features=1024, rms_norm_epsilon=0.0),
    lambda: O.Q4NXFusedLinearProjection(in_features=3072),                        # at most 2048 K
    lambda: O.Q4NXFusedLinearResidualProjection(in_features=2048, output_patches=0),
    # the GPU kernels' limits
    lambda: O.W4A16GEMV(M=3000, K=1024),
    lambda: O.W4A16GEMV(M=3072, K=1024, group_size=64),
    lambda: O.Qwen3FusedQKVProjection(in_features=1000, out_features=4096),
    lambda: O.Qwen3FusedUpGateProjection(in_features=1024, out_features=3072, rms_norm_epsilon=0.0),
    lambda: O.Qwen3FusedLinearResidualProjection(in_features=2048, out_features=1000),
    lambda: O.Qwen3DecodeAttention(n_heads=16, n_kv_heads=6),
])
def test_constructor_checks_raise_value_error(ctor):
    with pytest.raises(ValueError):
        ctor()


def test_argument_order_matches_the_reference():
    gemv = O.W4A16GEMV(M=3072, K=1024).get_arg_spec()
    assert [a.direction for a in gemv] == ["in", "in", "out"] and gemv[1].shape == (1024,)   # (W, x, y)
    batched = O.W4A16GEMV(M=3072, K=1024, num_batches=4, shared_qparam=True).get_arg_spec()
    assert batched[1].shape == (4, 1024) and batched[2].shape == (4, 3072)
    gemm = O.W4A16GEMM(M=32, K=1024, N=4096).get_arg_spec()
    assert gemm[0].shape == (32, 1024) and gemm[2].shape == (32, 4096)                       # (A, W, C)
    paired = O.W4A16PairedKGroupGEMM(M=8, K=1024, N=3072, tile_m=4, num_aie_rows=2).get_arg_spec()
    assert [a.direction for a in paired] == ["in", "in", "out", "out"]                        # (A, W, C0, C1)
    res = O.Qwen3FusedLinearResidualProjection(2048, 1024, rows=8).get_arg_spec()
    assert res[0].shape == (8, 2048) and res[1].shape == (8, 1024)                            # (ctx, residual, W, out)


def test_weight_buffer_is_checked():
    op = O.W4A16GEMM(M=4, K=256, N=512, tile_m=4, num_aie_rows=1)
    w = formats.W4A16Weight.from_numpy(*ow.synthetic_tensors(256, 128, seed=1))
    with pytest.raises(ValueError):
        op(torch.zeros(4, 256, dtype=BF16), w, torch.zeros(4, 512, dtype=BF16))


def test_q4nx_patch_weight_is_a_column_permutation():
    """Column (p * 3 + j) * 64 + r of the patch weight is row (first + p) * 64 + r of
    projection j, exactly (the dequantised columns are equal)."""
    parts = [ow.synthetic_tensors(256, n, seed=s) for s, n in ((1, 512), (2, 256), (3, 256))]
    w = formats.q4nx_patch_weight(*parts, output_patches=2, first_patch=1)
    dense = ow.dequantize(*w)
    ref = [ow.dequantize(*p) for p in parts]
    for p in range(2):
        for j in range(3):
            got = dense[(p * 3 + j) * 64:(p * 3 + j + 1) * 64]
            assert np.array_equal(got, ref[j][(1 + p) * 64:(2 + p) * 64])
    with pytest.raises(ValueError):
        formats.q4nx_patch_weight(*parts, output_patches=5)


def test_runlist_checks_entries_against_arg_specs():
    cfg = gm.Qwen3Config(n_layers=1)
    rl = R.qwen3_decode_runlist(cfg, rows=4, ctx_cap=64)
    assert len(rl) == 5 and all(len(bufs) == len(op.get_arg_spec()) for op, *bufs in rl)
    op, *bufs = rl[2]
    with pytest.raises(ValueError, match="Number of buffers"):
        R.FusedRunlist("bad", [(op, *bufs[:-1])], [], [], {}, "cpu")
    with pytest.raises(TypeError):
        R.FusedRunlist("bad", [(op, 1, 2, 3, 4)], [], [], {}, "cpu")
    with pytest.raises(ValueError, match="weight buffer"):
        R.FusedRunlist("bad", [rl[2]], [], [], {}, "cpu")


@pytest.mark.gpu
def test_operators_match_functional_layer(gpu):
    g = torch.Generator().manual_seed(0)
    w = formats.W4A16Weight.from_numpy(*ow.synthetic_tensors(1024, 3072, seed=2), device=gpu)
    x = torch.randn(1024, generator=g).to(BF16).to(gpu)
    y = torch.empty(3072, dtype=BF16, device=gpu)
    O.W4A16GEMV(M=3072, K=1024, num_aie_columns=8, tile_size_input=2, tile_size_output=384)(w, x, y)
    assert torch.equal(y, ops.linear(x, w))
    a = torch.randn(16, 1024, generator=g).to(BF16).to(gpu)
    c = torch.empty(16, 3072, dtype=BF16, device=gpu)
    O.W4A16KGroupGEMM(M=16, K=1024, N=3072, num_aie_rows=2, k_group=4)(a, w, c)
    assert torch.equal(c, ops.linear(a, w))
    gate, up = ow.synthetic_tensors(1024, 3072, seed=3), ow.synthetic_tensors(1024, 3072, seed=4)
    wp = formats.W4A16Weight.from_numpy(*formats.interleave_gate_up(gate, up), device=gpu)
    c0, c1 = torch.empty_like(c), torch.empty_like(c)
    O.W4A16PairedKGroupGEMM(M=16, K=1024, N=3072, num_aie_rows=2)(a, wp, c0, c1)
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
    # several vectors, one weight each (num_batches, not shared)
    ws = [formats.W4A16Weight.from_numpy(*ow.synthetic_tensors(1024, 3072, seed=10 + i), device=gpu) for i in range(3)]
    xb = torch.randn(3, 1024, generator=g).to(BF16).to(gpu)
    yb = torch.empty(3, 3072, dtype=BF16, device=gpu)
    O.W4A16GEMV(M=3072, K=1024, num_batches=3)(ws, xb, yb)
    for i in range(3):
        assert torch.equal(yb[i], ops.linear(xb[i], ws[i]))


@pytest.mark.gpu
def test_q4nx_operators_match_the_patch_reference(gpu):
    """The Q4NX callables against the oracle: out[p][j][r] = projection j row 64 (first + p) + r
    of the RMSNorm'd hidden vector (qkv: q, k, v; up/gate: up, gate), and the plain and
    residual o-projections, with patch-ordered AutoGPTQ weights."""
    g = torch.Generator().manual_seed(5)
    k = 1024
    parts = [ow.synthetic_tensors(k, 1024, seed=20 + j) for j in range(3)]
    hidden = torch.randn(k, generator=g).to(BF16)
    nw = (torch.rand(k, generator=g) * 0.2 + 0.9).to(BF16)
    from oracle import qwen3 as oq
    xn = oq.rmsnorm(hidden.float(), nw.float(), 1e-6, oq._Round("bf16"))
    for cls, nproj in ((O.Q4NXFusedQKVProjection, 3), (O.Q4NXFusedUpGateProjection, 2)):
        op = cls(in_features=k, output_patches=4, rms_norm_epsilon=1e-6)
        wt = formats.q4nx_patch_weight(*parts[:nproj], output_patches=4, first_patch=2)
        out = torch.empty(op.get_arg_spec()[3].shape, dtype=BF16, device=gpu)
        op(hidden.to(gpu), nw.to(gpu), formats.W4A16Weight.from_numpy(*wt, device=gpu), out)
        got = out.float().cpu().view(4, nproj, 64)
        ref = torch.from_numpy(ow.linear(xn.numpy()[None], *wt)).view(4, nproj, 64)
        err = (got - ref).abs().max() / ref.abs().max()
        assert err < 1e-2, (cls.__name__, float(err))
    wo = ow.synthetic_tensors(2048, 512, seed=30)
    ctx = torch.randn(2048, generator=g).to(BF16)
    resid = torch.randn(512, generator=g).to(BF16)
    ref = torch.from_numpy(ow.linear(ctx.float().numpy()[None], *wo)).view(-1)
    lin = O.Q4NXFusedLinearProjection(in_features=2048, output_patches=8)
    out = torch.empty(512, dtype=BF16, device=gpu)
    lin(ctx.to(gpu), formats.W4A16Weight.from_numpy(*wo, device=gpu), out)
    assert ((out.float().cpu() - ref).abs().max() / ref.abs().max()) < 1e-2
    rop = O.Q4NXFusedLinearResidualProjection(in_features=2048, output_patches=8)
    out2 = torch.empty(8, 64, dtype=BF16, device=gpu)
    rop(ctx.to(gpu), resid.to(gpu), formats.W4A16Weight.from_numpy(*wo, device=gpu), out2)
    assert torch.equal(out2.view(-1), (out.float() + resid.to(gpu).float()).to(BF16))


@pytest.mark.gpu
@pytest.mark.parametrize("layers", [1, 2])
def test_runlist_layer_matches_decode_layer(gpu, layers):
    """A decode step's layers written as the reference's ``(op, *buffer_names)``
    runlist (``batch_decode_fused.py:426-539`` form) give the same bits as
    ``Qwen3DecodeLayer``: residual stream and both KV caches."""
    cfg = gm.Qwen3Config(n_layers=layers, vocab=512)
    t = gm.random_qwen3_tensors(cfg, seed=41, weights="centered")
    b, cap = 6, 96
    # the runlist names the separate qkv linear and attention operators, each RMSNorm
    # fused into its consumer as the reference's operators have it: the layers without
    # the chained norm (whose sums of squares run in another order)
    m1 = gm.Qwen3Model(t, cfg, batch=b, ctx_cap=cap, device=gpu, fused=False, chain=False)
    m2 = gm.Qwen3Model(t, cfg, batch=b, ctx_cap=cap, device=gpu, fused=False)
    g = torch.Generator().manual_seed(42)
    x0 = torch.randn(b, cfg.hidden, generator=g).to(BF16).to(gpu)
    kc = torch.randn(m1.k_cache.shape, generator=g).to(BF16).to(gpu)
    vc = torch.randn(m1.v_cache.shape, generator=g).to(BF16).to(gpu)
    pos = torch.tensor([0, 5, 17, 40, 90, 95], dtype=torch.int32, device=gpu)
    for m in (m1, m2):
        m.x.copy_(x0)
        m.k_cache.copy_(kc)
        m.v_cache.copy_(vc)
        m.positions.copy_(pos)
    buf = m1.micro[0].buf
    for i, layer in enumerate(m1.layers):
        layer(buf, m1.positions, m1.k_cache[i], m1.v_cache[i])
    fused = R.FusedRunlist("qwen3_decode_layers", R.qwen3_decode_runlist(cfg, rows=b, ctx_cap=cap),
                           ["x", "positions"], ["x"], R.qwen3_decode_buffers(m2), gpu)
    fused()
    torch.cuda.synchronize()
    assert torch.equal(m2.x, m1.x)
    assert torch.equal(m2.k_cache, m1.k_cache) and torch.equal(m2.v_cache, m1.v_cache)
    assert torch.equal(fused.get_buffer("x"), m1.x)


@pytest.mark.parametrize("batch", [1, 5, 16, 32])
def test_reference_batch_decode_runlist_constructs(batch):
    """The reference's per-step runlist (``batch_decode_fused.py:300-539``) for
    Qwen3-0.6B: its operators are constructed with the reference's own arguments
    (``:336-425``), every entry's buffer count matches its operator's arg spec,
    and the per-layer sequence is the reference's, with one attention entry per
    sequence in place of the packet-cache pair."""
    cfg = gm.QWEN3_0_6B
    built = R.batch_decode_runlist(cfg, 640, batch, lm_head_out_features=152064)
    rl, rows = built["runlist"], built["decode_rows"]
    assert rows == next(r for r in (4, 8, 16, 32) if batch <= r)
    assert len(rl) == 1 + cfg.n_layers * (4 + batch + 6) + 1
    assert all(len(bufs) == len(op.get_arg_spec()) for op, *bufs in rl)
    names = [type(op).__name__ for op, *_ in rl[:5 + batch + 6]]
    assert names == (["RMSNorm", "W4A16KGroupGEMM", "W4A16PairedKGroupGEMM", "RMSNormRoPE", "RMSNormRoPE"]
                     + ["CopyPresentKVAttention"] * batch
                     + ["W4A16KGroupGEMM", "ResidualAddRMSNorm", "W4A16PairedKGroupGEMM", "SiLUMul",
                        "W4A16KGroupGEMM", "ResidualAddRMSNorm"])
    norm, q_gemm, kv_gemm, rope_q, rope_k = (e[0] for e in rl[:5])
    cols = min(8, rows)
    assert (norm.size, norm.num_aie_columns, norm.num_channels, norm.tile_size, norm.weighted, norm.epsilon) == \
        (rows * 1024, cols, 1, 1024, True, 1e-5)
    assert (rope_q.rows, rope_q.cols, rope_q.angle_rows, rope_q.num_aie_columns) == (rows * 16, 128, rows, cols)
    assert (rope_k.rows, rope_k.angle_rows) == (rows * 8, rows)
    assert (q_gemm.M, q_gemm.K, q_gemm.N, q_gemm.k_group) == (rows, 1024, 2048, 4)
    assert (kv_gemm.N, kv_gemm.k_group, kv_gemm.tile_m) == (1024, 2, 4 if rows <= 8 else 8)
    silu = rl[5 + batch + 3][0]
    assert (silu.size, silu.tile_size, silu.num_aie_columns) == (rows * 3072, 384, 8)
    head = rl[-1][0]
    assert type(head).__name__ == "W4A16NShardGEMM" and head.num_aie_rows == _n_shard_rows(152064, 64) and rl[-1][1:] == ("hidden_out",
                                                                                                  "W_out_head_qparam",
                                                                                                  "logits")
    # the last layer's residual norm writes hidden_out with the final norm weight
    assert rl[-2][1:] == ("x", "ffn_output", "W_final_norm", "x", "hidden_out")
    attn = rl[5]
    assert attn[1:] == ("queries[0:4096]", "keys[0:2048]", "values[0:2048]", "positions[0:4]",
                        f"k_cache_0[0:{8 * 640 * 128 * 2}]", f"v_cache_0[0:{8 * 640 * 128 * 2}]",
                        "attn_context[0:4096]")


def test_reference_batch_decode_runlist_binds_on_the_host():
    """A two-layer runlist binds its weight names and sizes every other buffer
    (``FusedRunlist`` with the reference's ``buffer_sizes``), without a GPU."""
    cfg = gm.Qwen3Config(n_layers=2, vocab=512)
    t = gm.random_qwen3_tensors(cfg, seed=3, weights="centered")
    built = R.batch_decode_runlist(cfg, 128, 3)
    bufs = {"x": torch.zeros(4, 1024, dtype=BF16), "rope_angles": torch.zeros(4, 128, dtype=BF16),
            "positions": torch.zeros(3, dtype=torch.int32), **R.batch_decode_weights(t, cfg, "cpu")}
    for i in range(2):
        bufs[f"k_cache_{i}"] = torch.zeros(3, 8, 128, 128, dtype=BF16)
        bufs[f"v_cache_{i}"] = torch.zeros(3, 8, 128, 128, dtype=BF16)
    fr = R.FusedRunlist("step", built["runlist"], built["input_args"], built["output_args"], bufs, "cpu",
                        buffer_sizes=built["buffer_sizes"])
    assert fr.get_buffer("queries").numel() == 4 * 2048 and fr.get_buffer("ffn_hidden").numel() == 4 * 3072
    assert fr.get_buffer("attn_context[4096:8192]").numel() == 2048
    assert fr.get_buffer("W_attn_key_value_1_qparam").N == 2048     # k|v paired
    with pytest.raises(ValueError, match="explicit size"):
        R.FusedRunlist("step", built["runlist"], built["input_args"], built["output_args"], bufs, "cpu")
    with pytest.raises(ValueError):
        R.batch_decode_runlist(cfg, 100, 3)          # max_seq_len % 64
    with pytest.raises(ValueError):
        R.batch_decode_runlist(cfg, 128, 33)         # beyond the 32-row bucket


@pytest.mark.parametrize("ctor", [
    lambda: O.RMSNorm(size=8 * 1000, num_aie_columns=8, num_channels=1, tile_size=1024, weighted=True),
    lambda: O.RMSNorm(size=8 * 1024, num_aie_columns=8, num_channels=1, tile_size=1024, epsilon=0.0),
    lambda: O.RMSNormRoPE(rows=128, cols=100, angle_rows=16),
    lambda: O.RMSNormRoPE(rows=128, cols=128, angle_rows=12),
    lambda: O.RMSNormRoPE(rows=128, cols=128, angle_rows=4),          # angle_rows < num_aie_columns
    lambda: O.RMSNormRoPE(rows=130, cols=128, angle_rows=13, num_aie_columns=8),
    lambda: O.SiLUMul(size=3000, tile_size=384),
    lambda: O.ResidualAddRMSNorm(size=8 * 1024, num_aie_columns=8, tile_size=1000),
    lambda: O.ResidualAddRMSNorm(size=8 * 1024, num_aie_columns=8, tile_size=1024, epsilon=-1.0),
    lambda: O.CopyPresentKVAttention(max_seq_len=100, chunk_size=64),
    lambda: O.CopyPresentKVAttention(max_seq_len=128, head_dim=64),   # the GPU kernel's D = 128
    lambda: O.CopyPresentKVAttention(max_seq_len=128, head_dim=128, q_heads_per_group=3),
])
def test_runlist_operator_checks_raise_value_error(ctor):
    with pytest.raises(ValueError):
        ctor()
