"""Write the small W4A16 golden fixture (``w4a16_small.npz``).

The expected outputs are computed here by brute force with plain Python
integers and fractions, one weight at a time, directly from the AutoGPTQ
definition -- nibble j of word (r, n) is q[8r + j][n], stored zero + 1 is the
zero point -- and not with the vectorised oracle, so the fixture checks the
oracle (and the GPU path) against an independent computation:

* ``W``: exact dequantised weights (q - z) * s, fp32;
* ``y``: x @ W^T accumulated exactly in rationals, rounded once to fp64.

The reference holds no fixture for this path (its tests need an NPU), so the
inputs are synthetic: a seeded draw plus hand-picked special words.

Run: ``python tests/golden/make_golden.py`` (rewrites the .npz next to it).
"""

from fractions import Fraction
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent / "w4a16_small.npz"
K, N, M, G = 256, 64, 3, 128


def build_inputs():
    rng = np.random.default_rng(20260101)
    qweight = rng.integers(0, 2**32, size=(K // 8, N), dtype=np.uint64).astype(np.uint32)
    qweight[0, :4] = [0x00000000, 0xFFFFFFFF, 0x76543210, 0xFEDCBA98]
    qzeros = rng.integers(0, 2**32, size=(K // G, N // 8), dtype=np.uint64).astype(np.uint32)
    qzeros[0, 0] = 0xF0E1D2C3   # zero nibbles 3,12,2,13,1,14,0,15: every extreme of z - 1
    scales = rng.uniform(0.005, 0.02, size=(K // G, N)).astype(np.float16)
    x = rng.standard_normal((M, K)).astype(np.float32)
    # bf16-representable activations (the kernels take bf16)
    x = (x.view(np.uint32) & 0xFFFF0000).view(np.float32)
    return qweight.view(np.int32), qzeros.view(np.int32), scales, x


def brute_force(qweight, qzeros, scales, x):
    qw = qweight.view(np.uint32)
    qz = qzeros.view(np.uint32)
    W = np.zeros((N, K), dtype=np.float32)
    Wq = [[None] * K for _ in range(N)]
    for n in range(N):
        for k in range(K):
            word = int(qw[k // 8, n])
            q = (word >> (4 * (k % 8))) & 0xF
            zword = int(qz[k // G, n // 8])
            z = ((zword >> (4 * (n % 8))) & 0xF) + 1
            s = Fraction(float(scales[k // G, n]))
            w = (q - z) * s
            Wq[n][k] = w
            W[n, k] = float(w)
    y = np.zeros((M, N), dtype=np.float64)
    for m in range(M):
        xs = [Fraction(float(v)) for v in x[m]]
        for n in range(N):
            y[m, n] = float(sum(xs[k] * Wq[n][k] for k in range(K)))
    return W, y


def main():
    qweight, qzeros, scales, x = build_inputs()
    W, y = brute_force(qweight, qzeros, scales, x)
    np.savez(OUT, qweight=qweight, qzeros=qzeros, scales=scales, x=x, W=W, y=y,
             K=K, N=N, M=M, group_size=G)
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
