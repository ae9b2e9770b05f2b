"""The reference's operator surface for the W4A16 path, on MI355X kernels.

Each class keeps the name, the constructor fields (with their defaults), the
``ValueError`` checks and the positional buffer order of ``get_arg_spec()`` of
the reference operator it stands in for, so the reference's runlist builders
construct it with the same keyword arguments and a runlist entry
``(op, *buffer_names)`` calls it unchanged.  The one difference is the weight
buffer: the AutoGPTQ tensors of the checkpoint (``W4A16Weight``) instead of an
NPU tile stream.  The NPU tiling fields (``num_aie_columns``, ``num_aie_rows``,
``tile_m``/``tile_k``/``tile_n``, ``tile_size_input``/``tile_size_output``,
``k_group``, ``context``) are accepted and checked as the reference checks
them, and have no effect on the GPU launch, whose tiling is chosen per shape.
Calls are asynchronous on torch's current stream; the caller owns every buffer
(``fusion.py:749-807`` semantics).

Reference operators:

* ``W4A16GEMV``              ``quantized_qwen3/operators/w4a16_gemv/op.py:22-126``, args (W, x, y)
* ``W4A16GEMM``              ``quantized_qwen3/operators/w4a16_gemm/op.py:23-174``, args (A, W, C)
* ``W4A16PairedKGroupGEMM``  ``w4a16_gemm/op.py:178-263``, args (A, W_pair, C0, C1)
* ``W4A16KGroupGEMM``        ``w4a16_gemm/op.py:267-333``, args (A, W, C)
* ``W4A16NShardGEMM``        ``w4a16_gemm/op.py:337-399``, args (A, W, C)
* ``Q4NXFusedQKVProjection``             ``fast_qwen3/operators/q4nx_fused_qkv_projection/op.py:30-136``,
                                         args (hidden, norm_weight, W, out)
* ``Q4NXFusedUpGateProjection``          ``fast_qwen3/operators/q4nx_fused_up_gate_projection/op.py:30-126``,
                                         args (hidden, norm_weight, W, out)
* ``Q4NXFusedLinearProjection``          ``fast_qwen3/operators/q4nx_fused_linear_projection/op.py:31-133``,
                                         args (x, W, out)
* ``Q4NXFusedLinearResidualProjection``  ``fast_qwen3/operators/q4nx_fused_linear_residual_projection/op.py:31-118``,
                                         args (ctx, residual, W, out)

The standalone operators of the reference's batch-decode runlist
(``quantized_qwen3/batch_decode_fused.py:336-425``), one kernel each:

* ``RMSNorm``                ``torch2iron/operators/rms_norm/op.py:20-143``, args (x, [weight,] y)
* ``RMSNormRoPE``            ``torch2iron/operators/rms_norm_rope/op.py:19-96``, args (x, weight, angles, y)
* ``SiLUMul``                ``torch2iron/operators/silu_mul/op.py:20-79``, args (left, right, out)
* ``ResidualAddRMSNorm``     ``torch2iron/operators/residual_add_rms_norm/op.py:19-93``,
                             args (x, update, weight, x_out, y)
* ``CopyPresentKVAttention`` the per-row pair ``CopyPresentPacketKV`` + ``LlamaChunkedAttention``
                             (``copy_present_packet_kv/op.py:18-95``, ``llama_chunked_attention/op.py:20-150``)
                             on the contiguous KV cache, args (q, k, v, positions, k_cache, v_cache, out)

Batch-row forms of the fused projections (one call per decode batch and full
output width, the shapes the GPU decode layer runs):

* ``Qwen3FusedQKVProjection``             (hidden [rows, K], norm_weight, W_qkv, out [rows, N])
* ``Qwen3FusedUpGateProjection``          (hidden, norm_weight, W_gate_up, out = silu(gate) * up)
* ``Qwen3FusedLinearResidualProjection``  (ctx, residual, W, out)
* ``Qwen3DecodeAttention``                (qkv, positions, q_norm, k_norm, rope, k_cache, v_cache, out):
                                          ``RMSNormRoPE`` q/k + ``CopyPresentPacketKV`` +
                                          ``LlamaChunkedAttention`` of ``batch_decode_fused.py:445-479``
* ``Qwen3LayerFused``                     ``fast_qwen3/operators/qwen3_layer_fused/op.py:18-50`` and the
                                          per-layer runlist of ``batch_decode_fused.py:426-530``,
                                          args (hidden, positions, k_cache, v_cache)
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from torch2iron_amd import ops
from torch2iron_amd.formats import W4A16Weight

BF16 = torch.bfloat16
Q4NX_IN_CHUNK = 256          # in_features granularity of the Q4NX operators (q4nx_layout.py:32)
Q4NX_PATCH_OUT_ROWS = 64     # output rows per patch (q4nx_layout.py:33)


@dataclass(frozen=True)
class ArgSpec:
    """Direction, shape and dtype of one positional buffer (``AIERuntimeArgSpec``)."""

    direction: str
    shape: tuple
    dtype: object


def _check_weight(w: W4A16Weight, k: int, n: int):
    if not isinstance(w, W4A16Weight):
        raise ValueError("the weight buffer must be a W4A16Weight (AutoGPTQ qweight/qzeros/scales)")
    if (w.K, w.N) != (k, n):
        raise ValueError(f"weight is K={w.K} N={w.N}, operator expects K={k} N={n}")


def _weight_spec(k: int, n: int) -> ArgSpec:
    return ArgSpec("in", ("W4A16Weight", k, n), W4A16Weight)


def _check_gpu_group(group_size: int):
    if group_size != 128:
        raise ValueError("the MI355X kernels support group_size=128 only")


# ---------------------------------------------------------------------------
# W4A16 GEMV / GEMM (quantized_qwen3 operators)
# ---------------------------------------------------------------------------

@dataclass
class W4A16GEMV:
    """y[M] = W[M, K] . x[K]: M output rows (the AutoGPTQ N), K inputs.

    ``num_batches > 1``: x ``[num_batches, K]`` and y ``[num_batches, M]``; with
    ``shared_qparam`` one weight serves every batch (one launch of
    ``num_batches`` rows), else the weight buffer is a sequence of
    ``num_batches`` weights (``w4a16_gemv/op.py:115-126``).
    """

    M: int
    K: int
    num_aie_columns: int = 1
    tile_size_input: int = 2
    tile_size_output: int | None = None
    num_batches: int = 1
    shared_qparam: bool = False
    group_size: int = 128
    kernel_vector_size: int = field(default=32, repr=False)
    context: object = field(default=None, repr=False)

    def __post_init__(self):
        # the reference's checks (w4a16_gemv/op.py:46-64)
        if self.tile_size_output is None:
            self.tile_size_output = self.tile_size_input
        if self.K % 2 != 0:
            raise ValueError("K must be even for packed int4 weights")
        if self.K % self.group_size != 0:
            raise ValueError("K must be a multiple of group_size")
        if self.kernel_vector_size != 32:
            raise ValueError("W4A16GEMV currently supports kernel_vector_size=32 only")
        if self.group_size % self.kernel_vector_size != 0:
            raise ValueError("group_size must be a multiple of kernel_vector_size")
        if self.K % self.kernel_vector_size != 0:
            raise ValueError("K must be a multiple of kernel_vector_size")
        if not (self.tile_size_output % self.tile_size_input == 0
                and self.tile_size_output >= self.tile_size_input):
            raise ValueError("tile_size_output must be a multiple of tile_size_input")
        # the GPU kernel's own limits
        _check_gpu_group(self.group_size)
        if self.M <= 0 or self.M % 16 != 0:
            raise ValueError("M must be a positive multiple of 16 (16-column MFMA tiles)")
        if self.num_batches < 1:
            raise ValueError("num_batches must be positive")

    def get_arg_spec(self):
        batch_dim = (self.num_batches,) if self.num_batches > 1 else ()
        qparam_dim = () if self.shared_qparam else batch_dim
        return [ArgSpec("in", qparam_dim + ("W4A16Weight", self.K, self.M), W4A16Weight),
                ArgSpec("in", batch_dim + (self.K,), BF16), ArgSpec("out", batch_dim + (self.M,), BF16)]

    def __call__(self, W, x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
        rows = self.num_batches
        if rows > 1 and not self.shared_qparam:
            ws = list(W)
            if len(ws) != rows:
                raise ValueError(f"expected {rows} weights, one per batch")
            xs, ys = x.view(rows, self.K), y.view(rows, self.M)
            for i, w in enumerate(ws):
                _check_weight(w, self.K, self.M)
                ops.linear(xs[i:i + 1], w, out=ys[i:i + 1])
            return y
        _check_weight(W, self.K, self.M)
        ops.linear(x.view(rows, self.K), W, out=y.view(rows, self.M))
        return y


@dataclass
class W4A16GEMM:
    """C[M, N] = A[M, K] . W^T (``w4a16_gemm/op.py:23-174``)."""

    M: int
    K: int
    N: int
    num_aie_columns: int = 8
    num_aie_rows: int = 4
    tile_m: int = 8
    tile_k: int = 128
    tile_n: int = 64
    group_size: int = 128
    context: object = field(default=None, repr=False)

    def _check_tiles(self, n_divisor: int):
        # the reference's checks (w4a16_gemm/op.py:55-74, 343-362)
        if self.tile_k != self.group_size:
            raise ValueError(f"{type(self).__name__} currently requires tile_k == group_size")
        if self.K % self.tile_k != 0:
            raise ValueError("K must be a multiple of tile_k")
        if self.N % n_divisor != 0:
            raise ValueError("N must be divisible by the tile_n * column (* row) product")
        if self.tile_m != 4 and self.tile_m % 8 != 0:
            raise ValueError("tile_m must be 4 or a multiple of 8 for aie::mmul<4,8,8>")
        if self.tile_k % 8 != 0:
            raise ValueError("tile_k must be a multiple of 8 for aie::mmul<4,8,8>")
        if self.tile_n % 16 != 0:
            raise ValueError("tile_n must be a multiple of 16 for 2x2 aie::mmul expansion")
        # the GPU kernel's own limits
        _check_gpu_group(self.group_size)
        if self.M < 1:
            raise ValueError("M must be positive")

    def __post_init__(self):
        if self.M % (self.tile_m * self.num_aie_rows) != 0:
            raise ValueError("M must be divisible by tile_m * num_aie_rows")
        self._check_tiles(self.tile_n * self.num_aie_columns)

    @property
    def k_tiles(self) -> int:
        return self.K // self.tile_k

    def get_arg_spec(self):
        return [ArgSpec("in", (self.M, self.K), BF16), _weight_spec(self.K, self.N),
                ArgSpec("out", (self.M, self.N), BF16)]

    def __call__(self, A: torch.Tensor, W: W4A16Weight, C: torch.Tensor) -> torch.Tensor:
        _check_weight(W, self.K, self.N)
        return ops.linear(A.view(self.M, self.K), W, out=C.view(self.M, self.N))


@dataclass
class W4A16KGroupGEMM(W4A16GEMM):
    """Same contract as ``W4A16GEMM`` (``w4a16_gemm/op.py:267-333``).  The NPU kernel
    rounded C to bf16 every ``k_group`` k-tiles; the GPU kernel accumulates the
    whole K in fp32."""

    k_group: int = 2

    def __post_init__(self):
        super().__post_init__()
        if self.k_tiles % self.k_group != 0:
            raise ValueError("k_tiles must be divisible by k_group")


@dataclass
class W4A16PairedKGroupGEMM(W4A16GEMM):
    """C0, C1 [M, N] from one A stream and one paired weight
    (``formats.interleave_gate_up(first, second)``: pair 0 -> C0, pair 1 -> C1;
    the reference runs gate/up and key/value this way, ``w4a16_gemm/op.py:178-263``)."""

    k_group: int = 2

    def __post_init__(self):
        super().__post_init__()
        if self.k_tiles % self.k_group != 0:
            raise ValueError("k_tiles must be divisible by k_group")

    def get_arg_spec(self):
        return [ArgSpec("in", (self.M, self.K), BF16), _weight_spec(self.K, 2 * self.N),
                ArgSpec("out", (self.M, self.N), BF16), ArgSpec("out", (self.M, self.N), BF16)]

    def __call__(self, A, W_pair: W4A16Weight, C0, C1):
        _check_weight(W_pair, self.K, 2 * self.N)
        return ops.gate_up(A.view(self.M, self.K), W_pair, swiglu=False, out=C0.view(self.M, self.N),
                           out_up=C1.view(self.M, self.N))


@dataclass
class W4A16NShardGEMM(W4A16GEMM):
    """The int4 lm_head GEMM (``w4a16_gemm/op.py:337-399``): N sharded over the
    NPU's core rows there; one GPU launch here."""

    def __post_init__(self):
        if self.M % self.tile_m != 0:
            raise ValueError("M must be divisible by tile_m")
        self._check_tiles(self.tile_n * self.num_aie_columns * self.num_aie_rows)


# ---------------------------------------------------------------------------
# Q4NX fused projections (fast_qwen3 operators), one hidden vector per call
# ---------------------------------------------------------------------------

def _check_q4nx_in(in_features: int):
    if in_features % Q4NX_IN_CHUNK != 0:
        raise ValueError(f"in_features must be divisible by {Q4NX_IN_CHUNK}")


def _check_patches(output_patches: int):
    if not 1 <= output_patches <= 8:
        raise ValueError("output_patches must be in [1, 8]")


@dataclass
class _Q4NXNormedProjection:
    in_features: int = Q4NX_IN_CHUNK
    out_rows: int = Q4NX_PATCH_OUT_ROWS
    output_patches: int = 8
    rms_norm_epsilon: float = 1e-6
    context: object = field(default=None, repr=False)

    projections = 0   # weight rows per patch position: 3 (q, k, v) or 2 (up, gate)

    def __post_init__(self):
        _check_q4nx_in(self.in_features)
        if self.out_rows != Q4NX_PATCH_OUT_ROWS:
            raise ValueError(f"out_rows must be {Q4NX_PATCH_OUT_ROWS}")
        _check_patches(self.output_patches)
        if self.rms_norm_epsilon <= 0:
            raise ValueError("rms_norm_epsilon must be positive")

    @property
    def out_features(self) -> int:
        return self.output_patches * self.projections * self.out_rows

    def get_arg_spec(self):
        return [ArgSpec("in", (self.in_features,), BF16), ArgSpec("in", (self.in_features,), BF16),
                _weight_spec(self.in_features, self.out_features), ArgSpec("out", (self.out_features,), BF16)]

    def __call__(self, hidden, norm_weight, W: W4A16Weight, out):
        _check_weight(W, self.in_features, self.out_features)
        ops.rmsnorm_linear(hidden.view(1, self.in_features), norm_weight.view(self.in_features),
                           self.rms_norm_epsilon, W, out=out.view(1, self.out_features))
        return out


@dataclass
class Q4NXFusedQKVProjection(_Q4NXNormedProjection):
    """RMSNorm + q/k/v projection of one hidden vector over ``output_patches``
    64-row output patches: ``out`` is ``[patch][q, k, v][64]``, as
    ``q4nx_fused_qkv_projection/op.py:128-136``.  The weight holds those rows as
    AutoGPTQ columns in the same order (``formats.q4nx_patch_weight(q, k, v, ...)``)."""

    projections = 3


@dataclass
class Q4NXFusedUpGateProjection(_Q4NXNormedProjection):
    """RMSNorm + up/gate projection of one hidden vector: ``out`` is
    ``[patch][up, gate][64]`` (``q4nx_fused_up_gate_projection/op.py:118-126``;
    weight from ``formats.q4nx_patch_weight(up, gate, ...)``)."""

    projections = 2


@dataclass
class Q4NXFusedLinearProjection:
    """Raw bf16 vector times ``output_patches`` 64-row patches: ``out`` [patches * 64]
    (``q4nx_fused_linear_projection/op.py:31-133``; in_features <= 2048 as there)."""

    in_features: int = 2048
    output_patches: int = 8
    context: object = field(default=None, repr=False)

    def __post_init__(self):
        _check_q4nx_in(self.in_features)
        _check_patches(self.output_patches)
        if self.in_features // Q4NX_IN_CHUNK > 8:
            raise ValueError(f"{type(self).__name__} currently supports at most 2048 K")

    @property
    def output_elements(self) -> int:
        return self.output_patches * Q4NX_PATCH_OUT_ROWS

    def get_arg_spec(self):
        return [ArgSpec("in", (self.in_features,), BF16), _weight_spec(self.in_features, self.output_elements),
                ArgSpec("out", (self.output_elements,), BF16)]

    def __call__(self, x, W: W4A16Weight, out):
        _check_weight(W, self.in_features, self.output_elements)
        ops.linear(x.view(1, self.in_features), W, out=out.view(1, self.output_elements))
        return out


@dataclass
class Q4NXFusedLinearResidualProjection(Q4NXFusedLinearProjection):
    """Projection followed by the residual add, ``out = bf16(bf16(ctx . W^T) + residual)``,
    ``out`` [patches, 64] (``q4nx_fused_linear_residual_projection/op.py:31-118``)."""

    def get_arg_spec(self):
        return [ArgSpec("in", (self.in_features,), BF16), ArgSpec("in", (self.output_elements,), BF16),
                _weight_spec(self.in_features, self.output_elements),
                ArgSpec("out", (self.output_patches, Q4NX_PATCH_OUT_ROWS), BF16)]

    def __call__(self, ctx, residual, W: W4A16Weight, out):
        _check_weight(W, self.in_features, self.output_elements)
        ops.linear(ctx.view(1, self.in_features), W, residual=residual.view(1, self.output_elements),
                   out=out.view(1, self.output_elements))
        return out


# ---------------------------------------------------------------------------
# Batch-row forms used by the GPU decode layer
# ---------------------------------------------------------------------------

@dataclass
class _NormedProjection:
    in_features: int
    out_features: int
    rows: int = 1
    rms_norm_epsilon: float = 1e-6

    def __post_init__(self):
        if self.in_features % 128 != 0:
            raise ValueError("in_features must be divisible by 128")
        if self.out_features % 64 != 0:
            raise ValueError("out_features must be divisible by 64")
        if not 1 <= self.rows <= 64:
            raise ValueError("rows must be in [1, 64]")
        if self.rms_norm_epsilon <= 0:
            raise ValueError("rms_norm_epsilon must be positive")


@dataclass
class Qwen3FusedQKVProjection(_NormedProjection):
    """RMSNorm + fused q|k|v projection in one kernel: out [rows, (Hq + 2 Hkv) * D]."""

    def get_arg_spec(self):
        return [ArgSpec("in", (self.rows, self.in_features), BF16), ArgSpec("in", (self.in_features,), BF16),
                _weight_spec(self.in_features, self.out_features),
                ArgSpec("out", (self.rows, self.out_features), BF16)]

    def __call__(self, hidden, norm_weight, W_qkv: W4A16Weight, out):
        _check_weight(W_qkv, self.in_features, self.out_features)
        return ops.rmsnorm_linear(hidden.view(self.rows, self.in_features), norm_weight, self.rms_norm_epsilon,
                                  W_qkv, out=out.view(self.rows, self.out_features))


@dataclass
class Qwen3FusedUpGateProjection(_NormedProjection):
    """RMSNorm + fused gate|up projection with the SwiGLU epilogue, in one kernel:
    out [rows, out_features] = silu(gate) * up, out_features = intermediate size."""

    def get_arg_spec(self):
        return [ArgSpec("in", (self.rows, self.in_features), BF16), ArgSpec("in", (self.in_features,), BF16),
                _weight_spec(self.in_features, 2 * self.out_features),
                ArgSpec("out", (self.rows, self.out_features), BF16)]

    def __call__(self, hidden, norm_weight, W_up_gate: W4A16Weight, out):
        _check_weight(W_up_gate, self.in_features, 2 * self.out_features)
        return ops.rmsnorm_gate_up(hidden.view(self.rows, self.in_features), norm_weight, self.rms_norm_epsilon,
                                   W_up_gate, swiglu=True, out=out.view(self.rows, self.out_features))


@dataclass
class Qwen3FusedLinearResidualProjection:
    """Projection followed by the residual add: out = residual + ctx . W^T
    (o_projection + residual, and down + residual).  ``out`` may be ``residual``."""

    in_features: int = 2048
    out_features: int = 1024
    rows: int = 1

    def __post_init__(self):
        if self.in_features % 128 != 0:
            raise ValueError("in_features must be divisible by 128")
        if self.out_features % 64 != 0:
            raise ValueError("out_features must be divisible by 64")
        if not 1 <= self.rows <= 64:
            raise ValueError("rows must be in [1, 64]")

    def get_arg_spec(self):
        return [ArgSpec("in", (self.rows, self.in_features), BF16), ArgSpec("in", (self.rows, self.out_features), BF16),
                _weight_spec(self.in_features, self.out_features),
                ArgSpec("out", (self.rows, self.out_features), BF16)]

    def __call__(self, ctx, residual, W: W4A16Weight, out):
        _check_weight(W, self.in_features, self.out_features)
        return ops.linear(ctx.view(self.rows, self.in_features), W, residual=residual.view(self.rows, -1),
                          out=out.view(self.rows, self.out_features))


@dataclass
class Qwen3DecodeAttention:
    """q/k RMSNorm + RoPE, KV-cache write of the current token and GQA attention,
    for ``rows`` sequences (one token each), in one kernel.  Args ``(qkv, positions,
    q_norm, k_norm, rope, k_cache, v_cache, out)``; caches ``[rows, Hkv, ctx_cap, D]``."""

    n_heads: int = 16
    n_kv_heads: int = 8
    head_dim: int = 128
    ctx_cap: int = 1024
    rows: int = 1
    rms_norm_epsilon: float = 1e-6
    rope_style: str = "halves"
    _workspace: object = field(default=None, repr=False)

    def __post_init__(self):
        if self.head_dim != 128:
            raise ValueError("head_dim must be 128")
        if self.n_kv_heads < 1 or self.n_heads % self.n_kv_heads or self.n_heads // self.n_kv_heads > 8:
            raise ValueError("n_heads must be a multiple of n_kv_heads, at most 8 per kv head")
        if not 1 <= self.rows <= 64 or self.ctx_cap < 1:
            raise ValueError("rows must be in [1, 64] and ctx_cap positive")
        if self.rope_style not in ("halves", "interleaved"):
            raise ValueError("rope_style must be 'halves' or 'interleaved'")
        self._workspace = ops.Workspace()

    def get_arg_spec(self):
        qkv = (self.n_heads + 2 * self.n_kv_heads) * self.head_dim
        cache = (self.rows, self.n_kv_heads, self.ctx_cap, self.head_dim)
        return [ArgSpec("in", (self.rows, qkv), BF16), ArgSpec("in", (self.rows,), torch.int32),
                ArgSpec("in", (self.head_dim,), BF16), ArgSpec("in", (self.head_dim,), BF16),
                ArgSpec("in", (self.ctx_cap, self.head_dim), BF16),
                ArgSpec("inout", cache, BF16), ArgSpec("inout", cache, BF16),
                ArgSpec("out", (self.rows, self.n_heads * self.head_dim), BF16)]

    def __call__(self, qkv, positions, q_norm, k_norm, rope, k_cache, v_cache, out):
        style = ops.ROPE_HALVES if self.rope_style == "halves" else ops.ROPE_INTERLEAVED
        return ops.decode_attention(qkv.view(self.rows, -1), positions, self.n_heads, self.n_kv_heads, q_norm,
                                    k_norm, self.rms_norm_epsilon, rope, k_cache, v_cache, rope_style=style,
                                    out=out.view(self.rows, -1), workspace=self._workspace)


@dataclass
class Qwen3LayerFused:
    """The whole decode layer: ``(hidden, positions, k_cache, v_cache)``, hidden updated in place.

    ``weights`` is a ``model.Qwen3LayerWeights``; ``rope`` the bf16 cos/sin table.
    """

    weights: object
    config: object
    rope: torch.Tensor
    rows: int = 1
    _impl: object = field(default=None, repr=False)
    _buf: object = field(default=None, repr=False)

    def __post_init__(self):
        from torch2iron_amd import model as gm
        if not 1 <= self.rows <= 64:
            raise ValueError("rows must be in [1, 64]")
        self._impl = gm.Qwen3DecodeLayer(self.weights, self.config, self.rope)

    def get_arg_spec(self):
        c = self.config
        return [ArgSpec("inout", (self.rows, c.hidden), BF16), ArgSpec("in", (self.rows,), torch.int32),
                ArgSpec("inout", (self.rows, c.n_kv_heads, self.rope.shape[0], c.head_dim), BF16),
                ArgSpec("inout", (self.rows, c.n_kv_heads, self.rope.shape[0], c.head_dim), BF16)]

    def __call__(self, hidden, positions, k_cache, v_cache):
        from torch2iron_amd import model as gm
        if self._buf is None:
            self._buf = gm.DecodeBuffers(self.config, self.rows, hidden.device)
        self._buf.x.copy_(hidden.view(self.rows, -1))
        self._impl(self._buf, positions, k_cache, v_cache)
        hidden.view(self.rows, -1).copy_(self._buf.x)
        return hidden


# ---------------------------------------------------------------------------
# The standalone operators of the batch-decode runlist (torch2iron operators)
# ---------------------------------------------------------------------------
# Their NPU fields (``num_aie_columns``, ``num_channels``, ``tile_size``) keep
# their meaning for the buffer shapes and divisibility checks; the ShimDMA
# channel budget checks of the reference (an NPU resource) have no counterpart.

@dataclass
class RMSNorm:
    """Row-wise RMSNorm over rows of ``tile_size`` (``rms_norm/op.py:20-143``);
    ``weighted`` multiplies by a ``[tile_size]`` weight (the decode runlist's form)."""

    size: int
    num_aie_columns: int
    num_channels: int
    tile_size: int
    weighted: bool = False
    epsilon: float = 1e-5
    context: object = field(default=None, repr=False)
    _ones: object = field(default=None, repr=False)

    def __post_init__(self):
        if self.epsilon <= 0:
            raise ValueError(f"epsilon must be positive, got {self.epsilon}")
        max_multiple = self.num_aie_columns * self.num_channels * self.tile_size
        if self.size % max_multiple != 0:
            raise ValueError(f"size ({self.size}) must be a multiple of "
                             f"num_aie_columns * num_channels * tile_size ({max_multiple})")
        if self.tile_size % 8 != 0 or self.tile_size > 8192:
            raise ValueError("tile_size must be a multiple of 8, at most 8192")

    def get_arg_spec(self):
        rows = (self.size // self.tile_size, self.tile_size)
        specs = [ArgSpec("in", rows, BF16)]
        if self.weighted:
            specs.append(ArgSpec("in", (self.tile_size,), BF16))
        specs.append(ArgSpec("out", rows, BF16))
        return specs

    def __call__(self, x, *rest):
        if self.weighted:
            weight, y = rest
        else:
            (y,) = rest
            if self._ones is None or self._ones.device != x.device:
                self._ones = torch.ones(self.tile_size, dtype=BF16, device=x.device)
            weight = self._ones
        return ops.rmsnorm(x.view(-1, self.tile_size), weight, self.epsilon, out=y.view(-1, self.tile_size))


@dataclass
class RMSNormRoPE:
    """Weighted RMSNorm then two-halves RoPE of ``rows`` head rows of ``cols``
    (``rms_norm_rope/op.py:19-96``, kernel ``kernel.cc:39-67``): row r takes angle
    row ``r // (rows // angle_rows)`` (cos at even, sin at odd columns)."""

    rows: int
    cols: int
    angle_rows: int
    num_aie_columns: int = 8
    epsilon: float = 1e-5
    context: object = field(default=None, repr=False)

    def __post_init__(self):
        # the reference's checks (rms_norm_rope/op.py:35-46)
        if self.cols % 32 != 0:
            raise ValueError("cols must be divisible by 32")
        if self.rows % self.num_aie_columns != 0:
            raise ValueError("rows must be divisible by num_aie_columns")
        if self.angle_rows > self.rows or self.rows % self.angle_rows != 0:
            raise ValueError("angle_rows must divide rows")
        if self.angle_rows < self.num_aie_columns or self.angle_rows % self.num_aie_columns != 0:
            raise ValueError("angle_rows must be divisible by num_aie_columns")
        if self.epsilon <= 0:
            raise ValueError("epsilon must be positive")
        if self.cols > 1024:
            raise ValueError("cols must be at most 1024")

    def get_arg_spec(self):
        return [ArgSpec("in", (self.rows, self.cols), BF16), ArgSpec("in", (self.cols,), BF16),
                ArgSpec("in", (self.angle_rows, self.cols), BF16), ArgSpec("out", (self.rows, self.cols), BF16)]

    def __call__(self, x, weight, angles, y):
        return ops.rmsnorm_rope(x.view(self.rows, self.cols), weight, angles.view(self.angle_rows, self.cols),
                                self.epsilon, rope_style=ops.ROPE_HALVES, out=y.view(self.rows, self.cols))


@dataclass
class SiLUMul:
    """``silu(left) * right`` elementwise (``silu_mul/op.py:20-79``)."""

    size: int
    tile_size: int
    num_aie_columns: int = 8
    context: object = field(default=None, repr=False)

    def __post_init__(self):
        if self.size % (self.num_aie_columns * self.tile_size) != 0:
            raise ValueError(f"size ({self.size}) must be a multiple of "
                             f"num_aie_columns * tile_size ({self.num_aie_columns * self.tile_size})")
        if self.size % 8 != 0:
            raise ValueError("size must be a multiple of 8")

    def get_arg_spec(self):
        return [ArgSpec("in", (self.size,), BF16), ArgSpec("in", (self.size,), BF16),
                ArgSpec("out", (self.size,), BF16)]

    def __call__(self, left, right, out):
        return ops.silu_mul(left.view(-1), right.view(-1), out=out.view(-1))


@dataclass
class ResidualAddRMSNorm:
    """``x_out = x + update``, then the weighted RMSNorm of ``x_out`` over rows of
    ``tile_size`` (``residual_add_rms_norm/op.py:19-93``).  ``x_out`` may be ``x``."""

    size: int
    num_aie_columns: int
    tile_size: int
    epsilon: float = 1e-5
    context: object = field(default=None, repr=False)

    def __post_init__(self):
        if self.epsilon <= 0:
            raise ValueError("epsilon must be positive")
        if self.size % (self.num_aie_columns * self.tile_size) != 0:
            raise ValueError("size must be divisible by num_aie_columns * tile_size")
        if self.tile_size % 8 != 0 or self.tile_size > 8192:
            raise ValueError("tile_size must be a multiple of 8, at most 8192")

    def get_arg_spec(self):
        return [ArgSpec("in", (self.size,), BF16), ArgSpec("in", (self.size,), BF16),
                ArgSpec("in", (self.tile_size,), BF16), ArgSpec("out", (self.size,), BF16),
                ArgSpec("out", (self.size,), BF16)]

    def __call__(self, x, update, weight, x_out, y):
        ops.residual_add_rmsnorm(x.view(-1), update.view(-1), weight, self.epsilon, x_out=x_out.view(-1),
                                 out=y.view(-1))
        return y


@dataclass
class CopyPresentKVAttention:
    """The runlist pair ``CopyPresentPacketKV`` + ``LlamaChunkedAttention``
    (``batch_decode_fused.py:445-479``) on the contiguous KV cache: writes the
    current k and v of ``rows`` sequences at their positions and attends (GQA)
    over slots ``0 .. position``.  q and k arrive normalised and rotated
    (``RMSNormRoPE``).  Constructor fields are ``LlamaChunkedAttention``'s
    (``llama_chunked_attention/op.py:35-63``; ``chunk_size`` is the NPU packet
    size, checked and otherwise unused) plus ``rows``.  Args ``(q [rows, Hq*D],
    k [rows, Hkv*D], v [rows, Hkv*D], positions int32 [rows], k_cache, v_cache,
    out [rows, Hq*D])``, caches ``[rows, Hkv, max_seq_len, D]``."""

    max_seq_len: int
    num_kv_groups: int = 8
    q_heads_per_group: int = 4
    head_dim: int = 64
    chunk_size: int = 64
    rows: int = 1
    kernel_vector_size: int = field(default=32, repr=False)
    context: object = field(default=None, repr=False)
    _workspace: object = field(default=None, repr=False)

    def __post_init__(self):
        # the reference's checks (llama_chunked_attention/op.py:49-63)
        if self.max_seq_len <= 0:
            raise ValueError("max_seq_len must be positive")
        if self.chunk_size <= 0:
            raise ValueError("chunk_size must be positive")
        if self.max_seq_len % self.chunk_size != 0:
            raise ValueError("max_seq_len must be divisible by chunk_size")
        if self.num_kv_groups <= 0:
            raise ValueError("num_kv_groups must be positive")
        if self.q_heads_per_group <= 0:
            raise ValueError("q_heads_per_group must be positive")
        if self.head_dim <= 0:
            raise ValueError("head_dim must be positive")
        if self.head_dim % self.kernel_vector_size != 0:
            raise ValueError("head_dim must be divisible by kernel_vector_size")
        # the GPU kernel's limits
        if self.head_dim != 128:
            raise ValueError("head_dim must be 128")
        if self.q_heads_per_group not in (1, 2, 4, 8):
            raise ValueError("q_heads_per_group must be 1, 2, 4 or 8")
        if self.rows < 1:
            raise ValueError("rows must be positive")
        self._workspace = ops.Workspace()

    def get_arg_spec(self):
        hq = self.num_kv_groups * self.q_heads_per_group
        cache = (self.rows, self.num_kv_groups, self.max_seq_len, self.head_dim)
        return [ArgSpec("in", (self.rows, hq * self.head_dim), BF16),
                ArgSpec("in", (self.rows, self.num_kv_groups * self.head_dim), BF16),
                ArgSpec("in", (self.rows, self.num_kv_groups * self.head_dim), BF16),
                ArgSpec("in", (self.rows,), torch.int32),
                ArgSpec("inout", cache, BF16), ArgSpec("inout", cache, BF16),
                ArgSpec("out", (self.rows, hq * self.head_dim), BF16)]

    def __call__(self, q, k, v, positions, k_cache, v_cache, out):
        hq = self.num_kv_groups * self.q_heads_per_group
        cache = (self.rows, self.num_kv_groups, self.max_seq_len, self.head_dim)
        return ops.decode_attention_prepared(q.view(self.rows, -1), k.view(self.rows, -1), v.view(self.rows, -1),
                                             positions.view(-1), hq, self.num_kv_groups, k_cache.view(cache),
                                             v_cache.view(cache), out=out.view(self.rows, -1),
                                             workspace=self._workspace)
