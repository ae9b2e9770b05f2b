"""AutoGPTQ group-128 W4A16 tensors as the MI355X kernels read them.

The kernels consume the checkpoint layout unchanged (``qweight [K/8, N]``,
``qzeros [K/g, N/8]``, fp16 ``scales [K/g, N]``), so a linear is just these
three device tensors.  The only offline repacks are column permutations done
at the nibble level, which are exact:

* ``concat_columns`` fuses q|k|v into one ``N = (Hq + 2 Hkv) * D`` linear;
* ``interleave_gate_up`` fuses gate|up into one linear whose column ``2i``
  is gate ``i`` and column ``2i + 1`` is up ``i``, so a lane that owns two
  consecutive output columns owns a matching gate/up pair (the reference
  pairs gate and up offline the same way, ``packed_format.py:360-369,
  548-582``, gate = pair 0).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

GROUP_SIZE = 128


@dataclass
class W4A16Weight:
    """One AutoGPTQ linear: ``W[n, k] = (q[k, n] - (z[k/g, n] + 1)) * s[k/g, n]``."""

    qweight: torch.Tensor   # int32 [K/8, N]
    qzeros: torch.Tensor    # int32 [K/g, N/8]
    scales: torch.Tensor    # fp16  [K/g, N]
    group_size: int = GROUP_SIZE
    # qweight's words as decode-linear tiles (int32, K/8 * N), set by ops.tile_weight;
    # the decode-sized linears read these instead of qweight when present
    tiles: torch.Tensor | None = field(default=None, repr=False, compare=False)

    def __post_init__(self):
        if self.qweight.dtype != torch.int32 or self.qzeros.dtype != torch.int32:
            raise ValueError("qweight and qzeros must be int32")
        if self.scales.dtype != torch.float16:
            raise ValueError("scales must be float16")
        k8, n = self.qweight.shape
        if self.scales.shape != (k8 * 8 // self.group_size, n):
            raise ValueError(f"scales shape {tuple(self.scales.shape)} does not match qweight {tuple(self.qweight.shape)}")
        if self.qzeros.shape != (self.scales.shape[0], n // 8):
            raise ValueError(f"qzeros shape {tuple(self.qzeros.shape)} does not match qweight {tuple(self.qweight.shape)}")

    @property
    def K(self) -> int:
        return int(self.qweight.shape[0]) * 8

    @property
    def N(self) -> int:
        return int(self.qweight.shape[1])

    @property
    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.qweight, self.qzeros, self.scales))

    def to(self, device) -> "W4A16Weight":
        return W4A16Weight(self.qweight.to(device).contiguous(), self.qzeros.to(device).contiguous(),
                           self.scales.to(device).contiguous(), self.group_size)

    @classmethod
    def from_numpy(cls, qweight, qzeros, scales, device="cpu", group_size: int = GROUP_SIZE) -> "W4A16Weight":
        return cls(torch.from_numpy(np.ascontiguousarray(qweight).view(np.int32)).to(device),
                   torch.from_numpy(np.ascontiguousarray(qzeros).view(np.int32)).to(device),
                   torch.from_numpy(np.ascontiguousarray(scales).astype(np.float16)).to(device),
                   group_size)

    def numpy(self):
        return (self.qweight.cpu().numpy(), self.qzeros.cpu().numpy(), self.scales.cpu().numpy())


def random_tensors(K: int, N: int, seed: int, group_size: int = GROUP_SIZE):
    """Seeded AutoGPTQ arrays: uniform random words (uniform nibbles 0..15),
    fp16 scales uniform in [0.005, 0.02]."""
    rng = np.random.default_rng(seed)
    qweight = rng.integers(0, 2**32, size=(K // 8, N), dtype=np.uint64).astype(np.uint32).view(np.int32)
    qzeros = rng.integers(0, 2**32, size=(K // group_size, N // 8), dtype=np.uint64).astype(np.uint32).view(np.int32)
    scales = rng.uniform(0.005, 0.02, size=(K // group_size, N)).astype(np.float16)
    return qweight, qzeros, scales


def random_weight(K: int, N: int, seed: int, device="cpu") -> W4A16Weight:
    return W4A16Weight.from_numpy(*random_tensors(K, N, seed), device=device)


# ---- nibble-level column permutations (exact repacks) ----

def _words_to_nibbles(words: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(words).view(np.uint32).astype(np.uint64)
    return ((w[..., None] >> (4 * np.arange(8, dtype=np.uint64))) & 0xF).astype(np.uint8)


def _nibbles_to_words(nib: np.ndarray) -> np.ndarray:
    acc = np.zeros(nib.shape[:-1], dtype=np.uint64)
    for j in range(8):
        acc |= nib[..., j].astype(np.uint64) << np.uint64(4 * j)
    return acc.astype(np.uint32).view(np.int32)


def _permute_columns(qweight, qzeros, scales, perm: np.ndarray):
    """New column n takes old column perm[n]."""
    qz_nib = _words_to_nibbles(qzeros).reshape(qzeros.shape[0], -1)[:, perm]
    qzeros_new = _nibbles_to_words(qz_nib.reshape(qzeros.shape[0], -1, 8))
    return (np.ascontiguousarray(np.asarray(qweight)[:, perm]), qzeros_new,
            np.ascontiguousarray(np.asarray(scales)[:, perm]))


def concat_columns(*parts):
    """Concatenate AutoGPTQ linears (numpy triples) along N."""
    qw = np.concatenate([p[0] for p in parts], axis=1)
    qz = np.concatenate([p[1] for p in parts], axis=1)
    sc = np.concatenate([p[2] for p in parts], axis=1)
    return qw, qz, sc


def gate_up_permutation(intermediate: int) -> np.ndarray:
    """Index map of the fused gate|up weight into concat(gate, up) columns."""
    f = np.arange(2 * intermediate)
    return np.where(f % 2 == 0, f // 2, intermediate + f // 2).astype(np.int64)


def interleave_gate_up(gate, up):
    """Fuse gate and up (numpy triples with equal K, N) into the paired layout."""
    inter = int(np.asarray(gate[0]).shape[1])
    if int(np.asarray(up[0]).shape[1]) != inter:
        raise ValueError("gate and up must have the same number of columns")
    if inter % 32:
        raise ValueError("intermediate size must be a multiple of 32")
    cat = concat_columns(gate, up)
    return _permute_columns(*cat, gate_up_permutation(inter))


def q4nx_patch_weight(*parts, output_patches: int, first_patch: int = 0, patch_rows: int = 64):
    """The columns a Q4NX fused projection reads, as one AutoGPTQ linear (numpy triple).

    ``parts`` are the projections whose patches the operator interleaves (q, k, v
    for the fused qkv, up, gate for the up/gate projection).  New column
    ``(p * len(parts) + j) * patch_rows + r`` is row ``(first_patch + p) * patch_rows + r``
    of projection ``j``: the ``[patch][projection][row]`` output order of the
    Q4NX operators (``q4nx_fused_qkv_projection/op.py:128-136``).  Exact (a
    column permutation at the nibble level).
    """
    if output_patches < 1 or not parts:
        raise ValueError("need at least one projection and one patch")
    widths = [int(np.asarray(p[0]).shape[1]) for p in parts]
    if any(w < (first_patch + output_patches) * patch_rows for w in widths):
        raise ValueError("a projection has fewer rows than the requested patches")
    offsets = np.cumsum([0] + widths[:-1])
    perm = [offsets[j] + (first_patch + p) * patch_rows + r
            for p in range(output_patches) for j in range(len(parts)) for r in range(patch_rows)]
    return _permute_columns(*concat_columns(*parts), np.asarray(perm, dtype=np.int64))


def random_weight_on_device(K: int, N: int, generator: torch.Generator, device) -> W4A16Weight:
    """Seeded random AutoGPTQ weight drawn directly on the device (benchmarks).

    Same distributions as ``random_tensors``: uniform 32-bit words, fp16
    scales uniform in [0.005, 0.02].
    """
    g = GROUP_SIZE
    qweight = torch.randint(-2**31, 2**31, (K // 8, N), dtype=torch.int64, device=device,
                            generator=generator).to(torch.int32)
    qzeros = torch.randint(-2**31, 2**31, (K // g, N // 8), dtype=torch.int64, device=device,
                           generator=generator).to(torch.int32)
    scales = (torch.rand((K // g, N), device=device, generator=generator) * 0.015 + 0.005).to(torch.float16)
    return W4A16Weight(qweight, qzeros, scales, g)


def algorithmic_bytes(M: int, K: int, N: int, group_size: int = GROUP_SIZE) -> int:
    """Bytes a W4A16 linear must move at minimum: int4 weights, fp16 scales,
    int32 zero words, bf16 activations in and out."""
    return K * N // 2 + (K // group_size) * N * 2 + (K // group_size) * (N // 8) * 4 + M * K * 2 + M * N * 2
