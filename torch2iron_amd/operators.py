"""The reference's operator surface for the W4A16 path, on MI355X kernels.

Each class keeps the name, the constructor shape arguments, the positional
buffer order of ``get_arg_spec()`` and the ``ValueError`` checks of the
reference operator it stands in for, so a runlist entry
``(op, *buffer_names)`` built for the NPU can call it unchanged apart from the
weight buffer, which is the AutoGPTQ tensors (``W4A16Weight``) instead of an
NPU tile stream.  Calls are asynchronous on torch's current stream; the
caller owns every buffer (``fusion.py:749-807`` semantics).

Reference operators:

* ``W4A16GEMV``             ``quantized_qwen3/operators/w4a16_gemv/op.py:22-126``, args (W, x, y)
* ``W4A16GEMM``             ``quantized_qwen3/operators/w4a16_gemm/op.py:23-174``, args (A, W, C)
* ``W4A16KGroupGEMM``       ``w4a16_gemm/op.py:267-333``, args (A, W, C)
* ``W4A16PairedKGroupGEMM`` ``w4a16_gemm/op.py:178-263``, args (A, W_pair, C_gate, C_up)
* ``Qwen3FusedQKVProjection``      ``fast_qwen3/operators/q4nx_fused_qkv_projection/op.py:30-136``,
                                   args (hidden, norm_weight, W_qkv, out)
* ``Qwen3FusedLinearResidualProjection``
                                   ``fast_qwen3/operators/q4nx_fused_linear_residual_projection/op.py:31-118``,
                                   args (ctx, residual, W, out)   (o_projection + residual, and down + residual)
* ``Qwen3FusedUpGateProjection``   ``fast_qwen3/operators/q4nx_fused_up_gate_projection/op.py:30-126``,
                                   args (hidden, norm_weight, W_up_gate, out)
* ``Qwen3LayerFused``              ``fast_qwen3/operators/qwen3_layer_fused/op.py:18-50`` and the per-layer
                                   runlist of ``quantized_qwen3/batch_decode_fused.py:426-530``,
                                   args (hidden, positions, k_cache, v_cache)
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from torch2iron_amd import ops
from torch2iron_amd.formats import W4A16Weight

BF16 = torch.bfloat16


@dataclass(frozen=True)
class ArgSpec:
    """Direction, shape and dtype of one positional buffer (``AIERuntimeArgSpec``)."""

    direction: str
    shape: tuple
    dtype: object


def _check_group(k: int, group_size: int):
    if group_size != 128:
        raise ValueError("only group_size=128 is supported")
    if k % group_size != 0:
        raise ValueError("K must be a multiple of group_size")


def _weight_specs(k: int, n: int, group_size: int):
    return [ArgSpec("in", (k // 8, n), torch.int32), ArgSpec("in", (k // group_size, n // 8), torch.int32),
            ArgSpec("in", (k // group_size, n), torch.float16)]


def _check_weight(w: W4A16Weight, k: int, n: int):
    if not isinstance(w, W4A16Weight):
        raise ValueError("the weight buffer must be a W4A16Weight (AutoGPTQ qweight/qzeros/scales)")
    if (w.K, w.N) != (k, n):
        raise ValueError(f"weight is K={w.K} N={w.N}, operator expects K={k} N={n}")


@dataclass
class W4A16GEMV:
    """y[M] = W[M, K] . x[K]: M output rows (the AutoGPTQ N), K inputs."""

    M: int
    K: int
    group_size: int = 128

    def __post_init__(self):
        if self.K % 2 != 0:
            raise ValueError("K must be even for packed int4 weights")
        _check_group(self.K, self.group_size)
        if self.M % 64 != 0:
            raise ValueError("M must be a multiple of 64")

    def get_arg_spec(self):
        return [ArgSpec("in", ("W4A16Weight", self.K, self.M), W4A16Weight),
                ArgSpec("in", (self.K,), BF16), ArgSpec("out", (self.M,), BF16)]

    def __call__(self, W: W4A16Weight, x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
        _check_weight(W, self.K, self.M)
        return ops.linear(x.view(1, self.K), W, out=y.view(1, self.M)).view(self.M)


@dataclass
class W4A16GEMM:
    """C[M, N] = A[M, K] . W^T with 1 <= M <= 64 decode rows."""

    M: int
    K: int
    N: int
    group_size: int = 128

    def __post_init__(self):
        if not 1 <= self.M <= 64:
            raise ValueError("M must be in [1, 64]")
        _check_group(self.K, self.group_size)
        if self.N % 64 != 0:
            raise ValueError("N must be a multiple of 64")

    def get_arg_spec(self):
        return [ArgSpec("in", (self.M, self.K), BF16), ArgSpec("in", ("W4A16Weight", self.K, self.N), W4A16Weight),
                ArgSpec("out", (self.M, self.N), BF16)]

    def __call__(self, A: torch.Tensor, W: W4A16Weight, C: torch.Tensor) -> torch.Tensor:
        _check_weight(W, self.K, self.N)
        return ops.linear(A, W, out=C)


@dataclass
class W4A16KGroupGEMM(W4A16GEMM):
    """Same contract as ``W4A16GEMM``.  ``k_group`` is accepted for runlist
    compatibility; the MI355X kernel always accumulates the whole K in fp32
    (the NPU variant rounded C to bf16 every ``k_group`` tiles)."""

    k_group: int = 2

    def __post_init__(self):
        super().__post_init__()
        if (self.K // 128) % self.k_group != 0:
            raise ValueError("k_tiles must be divisible by k_group")


@dataclass
class W4A16PairedKGroupGEMM(W4A16GEMM):
    """C_gate, C_up [M, N] from one A stream and one paired weight
    (``formats.interleave_gate_up``; gate = pair 0, up = pair 1)."""

    k_group: int = 2

    def __post_init__(self):
        super().__post_init__()
        if (self.K // 128) % self.k_group != 0:
            raise ValueError("k_tiles must be divisible by k_group")

    def get_arg_spec(self):
        return [ArgSpec("in", (self.M, self.K), BF16),
                ArgSpec("in", ("W4A16Weight", self.K, 2 * self.N), W4A16Weight),
                ArgSpec("out", (self.M, self.N), BF16), ArgSpec("out", (self.M, self.N), BF16)]

    def __call__(self, A, W_pair: W4A16Weight, C_gate, C_up):
        _check_weight(W_pair, self.K, 2 * self.N)
        return ops.gate_up(A, W_pair, swiglu=False, out=C_gate, out_up=C_up)


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
                ArgSpec("in", ("W4A16Weight", self.in_features, self.out_features), W4A16Weight),
                ArgSpec("out", (self.rows, self.out_features), BF16)]

    def __call__(self, hidden, norm_weight, W_qkv: W4A16Weight, out):
        _check_weight(W_qkv, self.in_features, self.out_features)
        return ops.rmsnorm_linear(hidden.view(self.rows, self.in_features), norm_weight, self.rms_norm_epsilon,
                                  W_qkv, out=out)


@dataclass
class Qwen3FusedUpGateProjection(_NormedProjection):
    """RMSNorm + fused gate|up projection with the SwiGLU epilogue, in one kernel:
    out [rows, out_features] = silu(gate) * up, out_features = intermediate size."""

    def get_arg_spec(self):
        return [ArgSpec("in", (self.rows, self.in_features), BF16), ArgSpec("in", (self.in_features,), BF16),
                ArgSpec("in", ("W4A16Weight", self.in_features, 2 * self.out_features), W4A16Weight),
                ArgSpec("out", (self.rows, self.out_features), BF16)]

    def __call__(self, hidden, norm_weight, W_up_gate: W4A16Weight, out):
        _check_weight(W_up_gate, self.in_features, 2 * self.out_features)
        return ops.rmsnorm_gate_up(hidden.view(self.rows, self.in_features), norm_weight, self.rms_norm_epsilon,
                                   W_up_gate, swiglu=True, out=out)


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
                ArgSpec("in", ("W4A16Weight", self.in_features, self.out_features), W4A16Weight),
                ArgSpec("out", (self.rows, self.out_features), BF16)]

    def __call__(self, ctx, residual, W: W4A16Weight, out):
        _check_weight(W, self.in_features, self.out_features)
        return ops.linear(ctx.view(self.rows, self.in_features), W, residual=residual, out=out)


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
