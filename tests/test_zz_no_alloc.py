"""The allocation-free decode attention (``t2i_decode_attention_noalloc``) against the
workspace entry point (``t2i_decode_attention``), through the C ABI: two calls in a
row on the library's scratch, the second with a smaller input, each bit-identical to
the workspace call on the same inputs."""

import pytest
import torch

from torch2iron_amd import _lib
from torch2iron_amd import model as gm
from torch2iron_amd import ops

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16


def _inputs(b, hq, hkv, cap, seed, dev):
    d = 128
    g = torch.Generator().manual_seed(seed)
    qkv = torch.randn(b, (hq + 2 * hkv) * d, generator=g).to(BF16).to(dev)
    kc = torch.randn(b, hkv, cap, d, generator=g).to(BF16).to(dev)
    vc = torch.randn(b, hkv, cap, d, generator=g).to(BF16).to(dev)
    qn = (torch.rand(d, generator=g) * 0.2 + 0.9).to(BF16).to(dev)
    kn = (torch.rand(d, generator=g) * 0.2 + 0.9).to(BF16).to(dev)
    pos = torch.randint(0, cap, (b,), generator=g, dtype=torch.int32)
    pos[0] = cap - 1
    return qkv, pos.to(dev), qn, kn, kc, vc


def _noalloc(qkv, pos, hq, hkv, qn, kn, rope, kc, vc, out):
    lib = _lib.load()
    rc = lib.t2i_decode_attention_noalloc(qkv.data_ptr(), pos.data_ptr(), pos.numel(), hq, hkv, 128,
                                          qn.data_ptr(), kn.data_ptr(), 1e-6, rope.data_ptr(), 0,
                                          kc.data_ptr(), vc.data_ptr(), kc.shape[2], out.data_ptr(),
                                          _lib.stream_handle(qkv.device))
    _lib.check(rc, "t2i_decode_attention_noalloc")


def test_noalloc_attention_matches_workspace_entry_point(gpu):
    # larger first (16 sequences, context 1088: several chunks per kv head), then smaller
    for b, hq, hkv, cap, seed in ((16, 16, 8, 1088, 1), (3, 16, 8, 300, 2)):
        print(f"noalloc attention B={b} Hq={hq} Hkv={hkv} ctx_cap={cap}", flush=True)
        qkv, pos, qn, kn, kc, vc = _inputs(b, hq, hkv, cap, seed, gpu)
        rope = gm.rope_table(128, cap, 1e6, gpu)
        kc2, vc2 = kc.clone(), vc.clone()
        ref = ops.decode_attention(qkv, pos, hq, hkv, qn, kn, 1e-6, rope, kc, vc, workspace=ops.Workspace())
        out = torch.full_like(ref, 7.0)
        _noalloc(qkv, pos, hq, hkv, qn, kn, rope, kc2, vc2, out)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        assert torch.equal(kc2, kc) and torch.equal(vc2, vc)
        # the same call again on the (now reused) scratch
        out2 = torch.zeros_like(ref)
        _noalloc(qkv, pos, hq, hkv, qn, kn, rope, kc2, vc2, out2)
        torch.cuda.synchronize()
        assert torch.equal(out2, ref)


def test_noalloc_attention_rejects_oversized_calls(gpu):
    """Beyond the scratch's limits the entry point returns T2I_ERR_WORKSPACE before
    launching anything (8193 sequence/kv-head pairs; 16 MiB of chunk states)."""
    lib = _lib.load()
    fake = 0x10000
    for b, hkv, cap in ((8193, 1, 4096), (64, 8, 65536)):
        rc = lib.t2i_decode_attention_noalloc(fake, fake, b, hkv * 2, hkv, 128, fake, fake, 1e-6, fake, 0,
                                              fake, fake, cap, fake, None)
        assert rc == _lib.T2I_ERR_WORKSPACE, (b, hkv, cap, rc)
