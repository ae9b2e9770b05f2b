"""The HBM read-ceiling kernel (``t2i_stream_read``) reads every byte it is given
and nothing else: each wave's XOR word equals the XOR of that wave's 16-byte words
(word i * 256 + t of workgroup g belongs to wave t / 64), computed on the host,
for every loads-per-thread variant, ragged tails and offsets into the buffer."""

import numpy as np
import pytest
import torch

from torch2iron_amd import ops

pytestmark = pytest.mark.gpu


def _expected(buf: np.ndarray, offset: int, nbytes: int, lpt: int) -> np.ndarray:
    words = buf[offset:offset + nbytes].view(np.uint32).reshape(-1, 4)   # 16-byte words
    per_wg = 256 * lpt
    blocks = -(-words.shape[0] // per_wg)
    padded = np.zeros((blocks * per_wg, 4), dtype=np.uint32)   # words past the end read as zero
    padded[:words.shape[0]] = words
    # [workgroup, load i, wave, lane, component] -> one row per wave
    per_wave = padded.reshape(blocks, lpt, 4, 64, 4).transpose(0, 2, 1, 3, 4).reshape(blocks * 4, -1)
    return np.bitwise_xor.reduce(per_wave, axis=1)


@pytest.mark.parametrize("nbytes,offset,lpt", [
    (16, 0, 1),                   # one word: one workgroup, 15 of its 16 KB past the end
    (4096 * 4 + 48, 256, 4),      # a ragged last workgroup, offset into the buffer
    (1 << 20, 0, 1), (1 << 20, 0, 2), (1 << 20, 0, 4), (1 << 20, 0, 8),
    ((3 << 20) + 4080, 1024, 2),
    (2278304, 4096, 8),           # the linear sweep's mean bytes per launch
])
def test_stream_read_xor_words(gpu, nbytes, offset, lpt):
    print(f"stream read {nbytes} bytes at {offset}, {lpt} loads per thread", flush=True)
    g = torch.Generator().manual_seed(nbytes + lpt)
    host = torch.randint(0, 256, (offset + nbytes + 4096,), dtype=torch.uint8, generator=g)
    dev = host.to(gpu)
    got = ops.stream_read(dev, nbytes, offset, lpt)
    torch.cuda.synchronize()
    want = _expected(host.numpy(), offset, nbytes, lpt)
    assert got.numel() == want.size
    assert np.array_equal(got.cpu().numpy().view(np.uint32), want)


def test_stream_read_rejects_bad_ranges(gpu):
    buf = torch.zeros(4096, dtype=torch.uint8, device=gpu)
    with pytest.raises(ValueError):
        ops.stream_read(buf, 4096, 16)        # past the end
    with pytest.raises(ValueError):
        ops.stream_read(buf, 100, 0)          # not a multiple of 16
    with pytest.raises(ValueError):
        ops.stream_read(buf, 4096, 0, loads_per_thread=3)
