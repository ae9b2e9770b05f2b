"""numpy restatement of the AutoGPTQ group-wise W4A16 linear. TEST INFRASTRUCTURE ONLY.

Tensors (AutoGPTQ layout, group size ``g``):

* ``qweight``  int32 ``[K/8, N]``; word ``qweight[r, n]`` holds ``q[8r + j, n]``
  in bits ``4j .. 4j+3`` (least-significant nibble first).
* ``qzeros``   int32 ``[K/g, N/8]``; word ``qzeros[t, c]`` holds the stored zero
  of column ``8c + j`` in nibble ``j``.  The effective zero point is the
  stored nibble **plus one** (the AutoGPTQ convention).
* ``scales``   fp16 ``[K/g, N]``.

``W[n, k] = (q[k, n] - z[k // g, n]) * s[k // g, n]``, computed in fp32, where
it is exact: ``|q - z| <= 16`` needs 5 bits and an fp16 scale 11, so the
product fits in fp32's 24-bit significand.

Every function cites the reference line it restates.
"""

from __future__ import annotations

import numpy as np


def unpack_int32_nibbles(packed: np.ndarray, values_per_word: int = 8) -> np.ndarray:
    """``(w >> 4j) & 0xF`` for ``j = 0..7``, appended as a trailing axis.

    Follows ``src/models/quantized_qwen3/packed_format.py:88-91`` (shifts by
    ``arange(0, 32, 4)``, mask ``0xF``, int16 result).  The word is taken as
    its 32-bit pattern, so negative int32 words unpack like their unsigned
    counterparts.
    """
    words = np.asarray(packed).astype(np.int64) & 0xFFFFFFFF
    shifts = np.arange(0, values_per_word * 4, 4, dtype=np.int64)
    return ((words[..., None] >> shifts) & 0xF).astype(np.int16)


def unpack_qweight(qweight: np.ndarray, in_features: int, out_features: int) -> np.ndarray:
    """Return ``q[n, k]`` (int16 ``[N, K]``) from ``qweight [K/8, N]``.

    Follows ``packed_format.py:94-101``: unpack to ``[K/8, N, 8]``, permute to
    ``[N, K/8, 8]``, flatten the last two axes and slice to ``in_features``.
    """
    nib = unpack_int32_nibbles(qweight)                # [K/8, N, 8]
    nib = np.transpose(nib, (1, 0, 2)).reshape(out_features, -1)
    return np.ascontiguousarray(nib[:, :in_features])


def unpack_qzeros(qzeros: np.ndarray, out_features: int) -> np.ndarray:
    """Return the effective zero points ``z[t, n]`` (int16 ``[K/g, N]``).

    Follows ``packed_format.py:104-106``: nibble ``j`` of ``qzeros[t, c]`` is
    the stored zero of column ``8c + j``; the effective zero is stored + 1.
    """
    nib = unpack_int32_nibbles(qzeros).reshape(qzeros.shape[0], -1)
    return np.ascontiguousarray(nib[:, :out_features] + 1).astype(np.int16)


def dequantize(qweight: np.ndarray, qzeros: np.ndarray, scales: np.ndarray,
               group_size: int = 128) -> np.ndarray:
    """Dense fp32 ``W [N, K]`` with ``W[n, k] = (q - z) * s``.

    Follows ``src/models/fast_qwen3/fast_packed_format.py:132-161``
    (``_autogptq_linear_to_dense``): ``in_features = 8 * qweight.shape[0]``,
    scales taken to fp32, transposed when stored ``[N, K/g]``, then the
    group loop ``(q - z) * s`` in fp32.  Vectorised here over groups; the
    result is bit-identical because each element is one exact product.
    """
    in_features = int(qweight.shape[0]) * 8
    out_features = int(qweight.shape[1])
    q = unpack_qweight(qweight, in_features, out_features).astype(np.float32)
    z = unpack_qzeros(qzeros, out_features).astype(np.float32)     # [G, N]
    s = np.asarray(scales).astype(np.float32)
    if s.shape[0] != z.shape[0] and s.shape[1] == z.shape[0]:
        s = np.ascontiguousarray(s.T)
    if s.shape != z.shape:
        raise ValueError(f"scale/zero shape mismatch: scales={s.shape} zeros={z.shape}")
    n_groups = s.shape[0]
    if n_groups * group_size != in_features:
        raise ValueError("in_features must equal groups * group_size")
    qg = q.reshape(out_features, n_groups, group_size)
    w = (qg - z.T[:, :, None]) * s.T[:, :, None]
    return np.ascontiguousarray(w.reshape(out_features, in_features), dtype=np.float32)


def linear(x: np.ndarray, qweight: np.ndarray, qzeros: np.ndarray, scales: np.ndarray,
           group_size: int = 128, accumulate: str = "fp64") -> np.ndarray:
    """``y[M, N] = x[M, K] @ W[N, K]^T`` with the exact fp32 weights.

    ``accumulate="fp64"`` is the high-precision reference used for the
    tolerance checks; ``"fp32"`` restates the group-loop form of
    ``src/models/quantized_qwen3/model.py:133-146`` (fp32 partial product per
    group, summed into an fp32 output).  ``x`` is taken to fp32 first
    (``model.py:135``), so a bf16 activation enters exactly.
    """
    w = dequantize(qweight, qzeros, scales, group_size)
    xf = np.asarray(x, dtype=np.float32)
    if accumulate == "fp64":
        return xf.astype(np.float64) @ w.astype(np.float64).T
    if accumulate != "fp32":
        raise ValueError("accumulate must be 'fp64' or 'fp32'")
    m = xf.shape[0]
    n, k = w.shape
    out = np.zeros((m, n), dtype=np.float32)
    for g0 in range(0, k, group_size):
        out += xf[:, g0:g0 + group_size] @ w[:, g0:g0 + group_size].T
    return out


# --------------------------------------------------------------------------
# Inverse packers.  Used to build test inputs from chosen integer values and
# to check unpack(pack(v)) == v; they are not part of the reference path.
# --------------------------------------------------------------------------

def pack_qweight(q_nk: np.ndarray) -> np.ndarray:
    """Pack ``q[n, k]`` (values 0..15) into AutoGPTQ ``qweight [K/8, N]``."""
    q = np.asarray(q_nk, dtype=np.int64)
    n, k = q.shape
    if k % 8:
        raise ValueError("K must be a multiple of 8")
    q = q.reshape(n, k // 8, 8)
    words = np.zeros((n, k // 8), dtype=np.int64)
    for j in range(8):
        words |= (q[:, :, j] & 0xF) << (4 * j)
    return words.T.astype(np.uint32).view(np.int32).copy()


def pack_qzeros(stored: np.ndarray) -> np.ndarray:
    """Pack stored zero nibbles ``[K/g, N]`` (values 0..15) into ``[K/g, N/8]``."""
    z = np.asarray(stored, dtype=np.int64)
    g, n = z.shape
    if n % 8:
        raise ValueError("N must be a multiple of 8")
    z = z.reshape(g, n // 8, 8)
    words = np.zeros((g, n // 8), dtype=np.int64)
    for j in range(8):
        words |= (z[:, :, j] & 0xF) << (4 * j)
    return words.astype(np.uint32).view(np.int32).copy()


def synthetic_tensors(K: int, N: int, group_size: int = 128, seed: int = 0):
    """Seeded AutoGPTQ tensors with the distributions of the benchmark configs.

    qweight and qzeros are uniform random 32-bit words (every nibble uniform
    in 0..15); scales are uniform in [0.005, 0.02], stored fp16.
    """
    rng = np.random.default_rng(seed)
    qweight = rng.integers(0, 2**32, size=(K // 8, N), dtype=np.uint64).astype(np.uint32).view(np.int32)
    qzeros = rng.integers(0, 2**32, size=(K // group_size, N // 8), dtype=np.uint64).astype(np.uint32).view(np.int32)
    scales = rng.uniform(0.005, 0.02, size=(K // group_size, N)).astype(np.float16)
    return qweight, qzeros, scales


def bf16_round(a: np.ndarray) -> np.ndarray:
    """Round fp32 to the nearest bf16 (ties to even), returned as fp32."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = rounded.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(a), a, out)
