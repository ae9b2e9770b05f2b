"""The C ABI library: it loads, exports every declared entry point, and rejects
bad arguments on the host before launching anything (CPU only, no GPU calls)."""

import re

import pytest
import torch

from conftest import ROOT
from torch2iron_amd import _lib
from torch2iron_amd import ops
from torch2iron_amd.formats import W4A16Weight, random_tensors

HEADER = ROOT / "include" / "t2i_hip.h"
FAKE = 0x10000          # an aligned, never-dereferenced address
MISALIGNED = 0x10002


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^(?:const\s+)?\w+\s*\*?\s*(t2i_\w+)\(", text, flags=re.M)))


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_functions()
    assert len(names) >= 12
    for name in names:
        assert hasattr(lib, name), f"{name} declared in t2i_hip.h but not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert lib.t2i_abi_version() == 7
    assert lib.t2i_strerror(-2) == b"unsupported shape"


@pytest.mark.parametrize("M,K,N,group,x,code", [
    (0, 1024, 3072, 128, FAKE, _lib.T2I_ERR_SHAPE),
    (65535 * 16 + 1, 1024, 3072, 128, FAKE, _lib.T2I_ERR_SHAPE),
    (1, 1000, 3072, 128, FAKE, _lib.T2I_ERR_SHAPE),
    (1, 1024, 3000, 128, FAKE, _lib.T2I_ERR_SHAPE),
    (1, 1024, 3072, 64, FAKE, _lib.T2I_ERR_GROUP),
    (1, 1024, 3072, 128, MISALIGNED, _lib.T2I_ERR_ALIGN),
    (1, 1024, 3072, 128, 0, _lib.T2I_ERR_NULL),
])
def test_linear_argument_errors(M, K, N, group, x, code):
    lib = _lib.load()
    rc = lib.t2i_w4a16_linear(x, M, FAKE, FAKE, FAKE, K, N, group, None, FAKE, None)
    assert rc == code
    assert lib.t2i_last_error()


def test_linear_residual_and_pair_validation():
    lib = _lib.load()
    assert lib.t2i_w4a16_linear(FAKE, 1, FAKE, FAKE, FAKE, 2048, 1024, 128, MISALIGNED, FAKE, None) \
        == _lib.T2I_ERR_ALIGN
    assert lib.t2i_w4a16_gate_up(FAKE, 1, FAKE, FAKE, FAKE, 1024, 6144, 128, 0, FAKE, None, None) \
        == _lib.T2I_ERR_NULL
    assert lib.t2i_w4a16_gate_up(FAKE, 1, FAKE, FAKE, FAKE, 1024, 6144, 64, 1, FAKE, None, None) \
        == _lib.T2I_ERR_GROUP


def test_fused_norm_entry_points_validate():
    lib = _lib.load()
    f = lib.t2i_w4a16_rmsnorm_linear
    assert f(FAKE, 16, None, 1e-6, FAKE, FAKE, FAKE, 1024, 4096, 128, FAKE, None) == _lib.T2I_ERR_NULL
    assert f(FAKE, 16, FAKE, 0.0, FAKE, FAKE, FAKE, 1024, 4096, 128, FAKE, None) == _lib.T2I_ERR_VALUE
    assert f(FAKE, 16, FAKE, 1e-6, FAKE, FAKE, FAKE, 1000, 4096, 128, FAKE, None) == _lib.T2I_ERR_SHAPE
    assert f(FAKE, 0, FAKE, 1e-6, FAKE, FAKE, FAKE, 1024, 4096, 128, FAKE, None) == _lib.T2I_ERR_SHAPE
    assert f(FAKE + 2, 16, FAKE, 1e-6, FAKE, FAKE, FAKE, 1024, 4096, 128, FAKE, None) == _lib.T2I_ERR_ALIGN
    g = lib.t2i_w4a16_rmsnorm_gate_up
    assert g(FAKE, 16, FAKE, 1e-6, FAKE, FAKE, FAKE, 1024, 6144, 128, 0, FAKE, None, None) == _lib.T2I_ERR_NULL
    assert g(FAKE, 16, FAKE, 1e-6, FAKE, FAKE, FAKE, 1024, 6144, 64, 1, FAKE, None, None) == _lib.T2I_ERR_GROUP


def test_row_sum_entry_points_validate():
    """The *_sums entry points reject bad sums arguments before launching anything."""
    lib = _lib.load()
    E = _lib
    # sums pointers: NULL where required, misaligned
    assert lib.t2i_w4a16_linear_sums(FAKE, None, 1, 600, FAKE, FAKE, FAKE, 1024, 4096, 128, None, FAKE,
                                     None) == E.T2I_ERR_NULL
    assert lib.t2i_w4a16_linear_sums(FAKE, FAKE + 2, 1, 600, FAKE, FAKE, FAKE, 1024, 4096, 128, None, FAKE,
                                     None) == E.T2I_ERR_ALIGN
    assert lib.t2i_w4a16_linear_sums(FAKE, FAKE, 3, 600, FAKE, FAKE, FAKE, 1024, 4096, 128, None, FAKE,
                                     None) == E.T2I_ERR_VALUE
    # y_sums needs the prompt GEMM (M >= 512) and the SwiGLU epilogue
    assert lib.t2i_w4a16_gate_up_sums(FAKE, None, 1, 16, FAKE, FAKE, FAKE, 1024, 6144, 128, 1, FAKE, None, FAKE,
                                      None) == E.T2I_ERR_SHAPE
    assert lib.t2i_w4a16_gate_up_sums(FAKE, None, 1, 600, FAKE, FAKE, FAKE, 1024, 6144, 128, 0, FAKE, FAKE, FAKE,
                                      None) == E.T2I_ERR_VALUE
    # RMSNorm sums: H a multiple of 128, sums required
    assert lib.t2i_rmsnorm_sums(FAKE, None, 0, 600, 1000, FAKE, 1e-6, None, FAKE, FAKE, None) == E.T2I_ERR_SHAPE
    assert lib.t2i_rmsnorm_sums(FAKE, None, 0, 600, 1024, FAKE, 1e-6, None, FAKE, None, None) == E.T2I_ERR_NULL
    assert lib.t2i_prefill_attention_sums(FAKE, 2, 100, 0, 16, 8, 128, FAKE, FAKE, 128, FAKE, None,
                                          None) == E.T2I_ERR_NULL
    assert lib.t2i_prefill_attention_sums(FAKE, 2, 100, 0, 16, 8, 128, FAKE, FAKE, 128, FAKE, FAKE + 2,
                                          None) == E.T2I_ERR_ALIGN
    qkv = [FAKE, FAKE, 4, 160, 0, FAKE, FAKE, FAKE, 1024, 128, 16, 8, 128, FAKE, FAKE, 1e-6, FAKE, 0, FAKE, FAKE,
           FAKE, 192, None]
    a = list(qkv); a[1] = None
    assert lib.t2i_prefill_qkv_rope_kv_sums(*a) == E.T2I_ERR_NULL
    a = list(qkv); a[1] = FAKE + 2
    assert lib.t2i_prefill_qkv_rope_kv_sums(*a) == E.T2I_ERR_ALIGN
    a = list(qkv); a[3] = 100                                    # B*T = 400 < 512
    assert lib.t2i_prefill_qkv_rope_kv_sums(*a) == E.T2I_ERR_SHAPE


def test_tile_entry_points_validate():
    """The decode-linear tile calls reject bad arguments before launching anything."""
    lib, E = _lib.load(), _lib
    tile = lib.t2i_w4a16_tile_qweight
    assert tile(None, 1024, 1024, FAKE, None) == E.T2I_ERR_NULL
    assert tile(FAKE, 1000, 1024, FAKE + 0x100000, None) == E.T2I_ERR_SHAPE
    assert tile(FAKE, 1024, 1000, FAKE + 0x100000, None) == E.T2I_ERR_SHAPE
    assert tile(FAKE, 1024, 1024, MISALIGNED + 0x100000, None) == E.T2I_ERR_ALIGN
    assert tile(FAKE, 1024, 1024, FAKE + 0x1000, None) == E.T2I_ERR_VALUE     # overlaps qweight (512 KiB)
    lt = lib.t2i_w4a16_linear_tiles
    args = [FAKE, 16, None, 0.0, None, FAKE, FAKE, FAKE, 1024, 4096, 128, E.T2I_TILES_STORE, None, FAKE, None, None]
    a = list(args); a[11] = 7
    assert lt(*a) == E.T2I_ERR_VALUE                                            # unknown epilogue
    a = list(args); a[11] = E.T2I_TILES_SWIGLU; a[12] = FAKE
    assert lt(*a) == E.T2I_ERR_VALUE                                            # residual with SwiGLU
    a = list(args); a[2] = FAKE; a[3] = 1e-6; a[12] = FAKE
    assert lt(*a) == E.T2I_ERR_VALUE                                            # residual with the fused norm
    a = list(args); a[1] = 512
    assert lt(*a) == E.T2I_ERR_SHAPE                                            # prompt rows without qweight
    a = list(args); a[5] = None
    assert lt(*a) == E.T2I_ERR_NULL                                             # no tiles
    a = list(args); a[4] = FAKE; a[5] = MISALIGNED
    assert lt(*a) == E.T2I_ERR_ALIGN                                            # misaligned tiles
    a = list(args); a[11] = E.T2I_TILES_PAIRED
    assert lt(*a) == E.T2I_ERR_NULL                                             # paired needs y1
    a = list(args); a[10] = 64
    assert lt(*a) == E.T2I_ERR_GROUP


def test_prefill_entry_points_validate():
    lib = _lib.load()
    prep = lib.t2i_prefill_qk_rope_kv
    args = [FAKE, 2, 100, 0, 16, 8, 128, FAKE, FAKE, 1e-6, FAKE, 0, FAKE, FAKE, FAKE, 640, None]
    a = list(args); a[6] = 64
    assert prep(*a) == _lib.T2I_ERR_SHAPE                       # head_dim 64
    a = list(args); a[3] = 600
    assert prep(*a) == _lib.T2I_ERR_SHAPE                       # positions 600..699 beyond the 640-slot cache
    a = list(args); a[11] = 2
    assert prep(*a) == _lib.T2I_ERR_VALUE                       # rope style
    a = list(args); a[12] = None
    assert prep(*a) == _lib.T2I_ERR_NULL
    att = lib.t2i_prefill_attention
    args = [FAKE, 2, 100, 0, 16, 8, 128, FAKE, FAKE, 640, FAKE, None]
    a = list(args); a[4] = 12
    assert att(*a) == _lib.T2I_ERR_SHAPE                        # 12 q heads over 8 kv heads
    a = list(args); a[4], a[5] = 32, 2
    assert att(*a) == _lib.T2I_ERR_SHAPE                        # 16 q heads per kv head
    a = list(args); a[10] = FAKE + 2
    assert att(*a) == _lib.T2I_ERR_ALIGN
    a = list(args); a[2], a[3] = 700, 0
    assert att(*a) == _lib.T2I_ERR_SHAPE
    fused = lib.t2i_prefill_qkv_rope_kv
    args = [FAKE, 16, 512, 0, FAKE, FAKE, FAKE, 1024, 128, 16, 8, 128, FAKE, FAKE, 1e-6, FAKE, 0, FAKE, FAKE, FAKE,
            640, None]
    a = list(args); a[1], a[2] = 2, 100
    assert fused(*a) == _lib.T2I_ERR_SHAPE                      # 200 rows: below the prompt GEMM
    a = list(args); a[11] = 64
    assert fused(*a) == _lib.T2I_ERR_SHAPE                      # head_dim 64
    a = list(args); a[20] = 500
    assert fused(*a) == _lib.T2I_ERR_SHAPE                      # positions beyond the cache
    a = list(args); a[8] = 64
    assert fused(*a) == _lib.T2I_ERR_GROUP
    a = list(args); a[17] = FAKE + 2
    assert fused(*a) == _lib.T2I_ERR_ALIGN
    a = list(args); a[12] = None
    assert fused(*a) == _lib.T2I_ERR_NULL


def test_other_entry_points_validate():
    lib = _lib.load()
    assert lib.t2i_rmsnorm(FAKE, None, 0, 4, 1020, FAKE, 1e-6, None, FAKE, None, None) == _lib.T2I_ERR_SHAPE
    assert lib.t2i_rmsnorm(FAKE, None, 0, 4, 1024, FAKE, 0.0, None, FAKE, None, None) == _lib.T2I_ERR_VALUE
    assert lib.t2i_rmsnorm(FAKE, FAKE, 10, 4, 1024, FAKE, 1e-6, None, FAKE, None, None) == _lib.T2I_ERR_NULL
    assert lib.t2i_rmsnorm(FAKE, FAKE, 0, 4, 1024, FAKE, 1e-6, FAKE, FAKE, None, None) == _lib.T2I_ERR_SHAPE
    args = [FAKE, FAKE, 8, 16, 8, 64, FAKE, FAKE, 1e-6, FAKE, 0, FAKE, FAKE, 1088, FAKE, None, 0, None]
    assert lib.t2i_decode_attention(*args) == _lib.T2I_ERR_SHAPE            # head_dim 64
    args[5] = 128
    args[3] = 12                                                             # 12 q heads over 8 kv heads
    assert lib.t2i_decode_attention(*args) == _lib.T2I_ERR_SHAPE
    args[3] = 16
    args[2], args[13] = 2, 4096                                              # 2 sequences, 4096 slots: split
    assert lib.t2i_decode_attention_workspace_bytes(2, 16, 8, 4096) > 0
    assert lib.t2i_decode_attention(*args) == _lib.T2I_ERR_WORKSPACE        # split context needs workspace
    args[15], args[16] = FAKE, 64
    assert lib.t2i_decode_attention(*args) == _lib.T2I_ERR_WORKSPACE        # workspace too small
    assert lib.t2i_lm_head_argmax(FAKE, 16, FAKE, 151930, 1024, None, FAKE, None) == _lib.T2I_ERR_SHAPE
    assert lib.t2i_lm_head_argmax(FAKE, 16, FAKE, 151936, 1024, None, None, None) == _lib.T2I_ERR_NULL
    fused = lib.t2i_rmsnorm_lm_head_argmax
    assert fused(FAKE, 16, None, 1e-6, FAKE, 151936, 1024, None, FAKE, None) == _lib.T2I_ERR_NULL
    assert fused(FAKE, 16, FAKE, 1e-6, FAKE, 151936, 192, None, FAKE, None) == _lib.T2I_ERR_SHAPE   # K not 2^n
    assert fused(FAKE, 16, FAKE, 0.0, FAKE, 151936, 1024, None, FAKE, None) == _lib.T2I_ERR_VALUE
    assert fused(FAKE, 16, FAKE + 2, 1e-6, FAKE, 151936, 1024, None, FAKE, None) == _lib.T2I_ERR_ALIGN
    assert lib.t2i_w4a16_dequant_f32(FAKE, FAKE, FAKE, 1024, 3072, 128, None, None) == _lib.T2I_ERR_NULL
    assert lib.t2i_stream_read(FAKE, 4096, 4, None, None) == _lib.T2I_ERR_NULL
    assert lib.t2i_stream_read(FAKE, 4100, 4, FAKE, None) == _lib.T2I_ERR_SHAPE    # not a multiple of 16
    assert lib.t2i_stream_read(FAKE, 4096, 3, FAKE, None) == _lib.T2I_ERR_VALUE    # loads per thread
    assert lib.t2i_stream_read(FAKE + 8, 4096, 4, FAKE, None) == _lib.T2I_ERR_ALIGN
    assert lib.t2i_stream_read_out_words(4096 * 4 * 3 + 16, 4) == 4 * 4   # 4 workgroups of 16 KB, 4 waves each
    assert lib.t2i_stream_read_out_words(4096, 3) == 0


def test_python_layer_rejects_cpu_tensors_and_bad_shapes():
    w = W4A16Weight.from_numpy(*random_tensors(256, 64, seed=1))
    x = torch.zeros(1, 256, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU tensor"):
        ops.linear(x, w)
    with pytest.raises(ValueError):
        W4A16Weight(w.qweight, w.qzeros, w.scales[:1])


def test_workspace_sizes_are_consistent():
    lib = _lib.load()
    # a context of at most one 128-slot chunk needs no workspace
    assert lib.t2i_decode_attention_workspace_bytes(8, 16, 8, 100) == 0
    assert lib.t2i_decode_attention_workspace_bytes(8, 16, 8, 128) == 0
    # counters + (max, sum) pairs + contexts of every chunk; batch 8 at 1088 slots takes
    # 8 chunks of 136 (512 workgroups, a multiple of the 256 CUs) instead of 9 of 128
    for b, hq, hkv, cap, chunk in ((8, 16, 8, 1088, 136), (2, 16, 8, 4096, 128), (4, 16, 4, 640, 64)):
        units, q, splits = b * hkv, hq // hkv, -(-cap // chunk)
        need = units * 4 + units * splits * q * 2 * 4 + units * splits * q * 128 * 4
        n = lib.t2i_decode_attention_workspace_bytes(b, hq, hkv, cap)
        assert need <= n <= need + 512, (b, hq, hkv, cap, n, need)
    assert lib.t2i_decode_attention_workspace_bytes(0, 16, 8, 640) == 0
    # batch 16 x 8 kv heads at 640 slots: 6 splits (768 workgroups, a multiple of the
    # 256 CUs) instead of 5; batch 8 at 1088 slots: no raise of the 9 splits reaches a
    # multiple (12 would be a third more), so 8 longer chunks of 136 slots (512)
    for b, cap, splits in ((16, 640, 6), (8, 1088, 8), (32, 640, 5)):
        units, q = b * 8, 2
        need = units * 4 + units * splits * q * 2 * 4 + units * splits * q * 128 * 4
        n = lib.t2i_decode_attention_workspace_bytes(b, 16, 8, cap)
        assert need <= n <= need + 512, (b, cap, n, need)


def test_split_batch_covers_rows():
    from torch2iron_amd.model import split_batch
    for batch in (1, 3, 8, 16, 17):
        for parts in (1, 2, 3, 4, 32):
            r = split_batch(batch, parts)
            assert r[0][0] == 0 and r[-1][1] == batch
            assert all(a1 == b0 for (_, a1), (b0, _) in zip(r, r[1:]))
            sizes = [b1 - b0 for b0, b1 in r]
            assert min(sizes) >= 1 and max(sizes) - min(sizes) <= 1
            assert len(r) == min(parts, batch)


def test_runlist_entry_points_validate():
    """The reference runlist's standalone operators and the prepared attention
    reject bad arguments on the host before any launch."""
    lib = _lib.load()
    rr = lib.t2i_rmsnorm_rope
    assert rr(None, 256, 128, FAKE, FAKE, 16, 1e-5, 0, FAKE, None) == _lib.T2I_ERR_NULL
    assert rr(FAKE, 256, 127, FAKE, FAKE, 16, 1e-5, 0, FAKE, None) == _lib.T2I_ERR_SHAPE      # odd cols
    assert rr(FAKE, 256, 2048, FAKE, FAKE, 16, 1e-5, 0, FAKE, None) == _lib.T2I_ERR_SHAPE     # > 1024
    assert rr(FAKE, 256, 128, FAKE, FAKE, 12, 1e-5, 0, FAKE, None) == _lib.T2I_ERR_SHAPE      # 12 does not divide 256
    assert rr(FAKE, 256, 128, FAKE, FAKE, 16, 1e-5, 2, FAKE, None) == _lib.T2I_ERR_VALUE
    assert rr(FAKE, 256, 128, FAKE, FAKE, 16, 0.0, 0, FAKE, None) == _lib.T2I_ERR_VALUE
    sm = lib.t2i_silu_mul
    assert sm(FAKE, None, 3072, FAKE, None) == _lib.T2I_ERR_NULL
    assert sm(FAKE, FAKE, 3070, FAKE, None) == _lib.T2I_ERR_SHAPE
    assert sm(FAKE, MISALIGNED, 3072, FAKE, None) == _lib.T2I_ERR_ALIGN
    ra = lib.t2i_residual_add_rmsnorm
    assert ra(FAKE, FAKE, 8, 1024, FAKE, 1e-5, FAKE, None, None) == _lib.T2I_ERR_NULL
    assert ra(FAKE, FAKE, 8, 1020, FAKE, 1e-5, FAKE, FAKE, None) == _lib.T2I_ERR_SHAPE
    assert ra(FAKE, FAKE, 0, 1024, FAKE, 1e-5, FAKE, FAKE, None) == _lib.T2I_ERR_SHAPE
    assert ra(FAKE, FAKE, 8, 1024, FAKE, -1.0, FAKE, FAKE, None) == _lib.T2I_ERR_VALUE
    assert ra(FAKE, MISALIGNED, 8, 1024, FAKE, 1e-5, FAKE, FAKE, None) == _lib.T2I_ERR_ALIGN
    pa = lib.t2i_decode_attention_prepared
    args = [FAKE, FAKE, FAKE, FAKE, 16, 16, 8, 128, FAKE, FAKE, 640, FAKE, FAKE, 1 << 20, None]
    a = list(args); a[1] = None
    assert pa(*a) == _lib.T2I_ERR_NULL
    a = list(args); a[7] = 64
    assert pa(*a) == _lib.T2I_ERR_SHAPE                          # head_dim 64
    a = list(args); a[5] = 12
    assert pa(*a) == _lib.T2I_ERR_SHAPE                          # 12 q heads over 8 kv heads
    a = list(args); a[2] = MISALIGNED
    assert pa(*a) == _lib.T2I_ERR_ALIGN
    a = list(args); a[12] = None
    assert pa(*a) == _lib.T2I_ERR_WORKSPACE                      # split context needs the workspace
