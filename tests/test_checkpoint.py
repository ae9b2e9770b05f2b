"""AutoGPTQ safetensors checkpoints: round trip, sharding and the rejected variants.

The reference's loader (``packed_format.py:71-85``) reads ``model.safetensors``
or an index of shards; a synthetic checkpoint in that layout is written here
(no checkpoint can be downloaded) and read back bit for bit.
"""

import json

import numpy as np
import pytest
import torch

from torch2iron_amd import checkpoint as ck
from torch2iron_amd import model as gm

CFG = gm.Qwen3Config(n_layers=2, vocab=512, hidden=256, n_heads=4, n_kv_heads=2, intermediate=512)


def _tensors(seed=3, weights="uniform"):
    return gm.random_qwen3_tensors(CFG, seed=seed, weights=weights)


def _same(a: dict, b: dict):
    assert set(a) == set(b)
    for k in a:
        x, y = np.asarray(a[k]), np.asarray(b[k])
        assert x.shape == y.shape, k
        if k.endswith((".qweight", ".qzeros")):
            assert np.array_equal(x.view(np.uint32), y.view(np.uint32)), k
        else:
            assert np.array_equal(x.astype(np.float32), y.astype(np.float32)), k


@pytest.mark.parametrize("shards", [1, 3])
def test_round_trip(tmp_path, shards):
    t = _tensors()
    ck.write_checkpoint(tmp_path, t, CFG, shards=shards)
    if shards > 1:
        idx = json.loads((tmp_path / ck.INDEX).read_text())
        assert len(set(idx["weight_map"].values())) == shards
        assert not (tmp_path / ck.SINGLE).exists()
    got, cfg = ck.load_checkpoint(tmp_path)
    assert cfg == CFG
    _same(got, t)


def test_untied_lm_head_and_trivial_g_idx(tmp_path):
    from safetensors.torch import load_file, save_file
    t = _tensors()
    t["lm_head.weight"] = torch.randn(CFG.vocab, CFG.hidden).to(torch.bfloat16).float().numpy()
    ck.write_checkpoint(tmp_path, t, CFG)
    f = tmp_path / ck.SINGLE
    raw = load_file(str(f))
    raw["model.layers.0.self_attn.q_proj.g_idx"] = (torch.arange(CFG.hidden) // 128).to(torch.int32)
    save_file(raw, str(f))
    got, _ = ck.load_checkpoint(tmp_path)
    assert "lm_head.weight" in got and not any(k.endswith(".g_idx") for k in got)
    _same(got, t)


def test_config_fields(tmp_path):
    ck.write_checkpoint(tmp_path, _tensors(), CFG)
    hf = json.loads((tmp_path / "config.json").read_text())
    hf.pop("rope_theta")
    hf["rope_parameters"] = {"rope_theta": 5e5}
    hf.pop("head_dim")
    cfg = ck.config_from_hf(hf)
    assert cfg.rope_theta == 5e5 and cfg.head_dim == CFG.hidden // CFG.n_heads


@pytest.mark.parametrize("change,match", [
    (lambda q: q.update(bits=8), "4-bit"),
    (lambda q: q.update(group_size=64), "group_size"),
    (lambda q: q.update(desc_act=True), "act-order"),
])
def test_rejected_quantisation(tmp_path, change, match):
    ck.write_checkpoint(tmp_path, _tensors(), CFG)
    hf = json.loads((tmp_path / "config.json").read_text())
    change(hf["quantization_config"])
    (tmp_path / "config.json").write_text(json.dumps(hf))
    with pytest.raises(ValueError, match=match):
        ck.load_checkpoint(tmp_path)


def test_rejected_act_order_g_idx_and_missing_tensor(tmp_path):
    from safetensors.torch import load_file, save_file
    ck.write_checkpoint(tmp_path, _tensors(), CFG)
    f = tmp_path / ck.SINGLE
    raw = load_file(str(f))
    perm = torch.randperm(CFG.hidden, generator=torch.Generator().manual_seed(0))
    raw["model.layers.0.mlp.gate_proj.g_idx"] = ((torch.arange(CFG.hidden) // 128)[perm]).to(torch.int32)
    save_file(raw, str(f))
    with pytest.raises(ValueError, match="g_idx"):
        ck.load_checkpoint(tmp_path)
    raw.pop("model.layers.0.mlp.gate_proj.g_idx")
    raw.pop("model.layers.1.self_attn.k_norm.weight")
    save_file(raw, str(f))
    with pytest.raises(ValueError, match="missing"):
        ck.load_checkpoint(tmp_path)
    (tmp_path / "empty").mkdir()
    with pytest.raises(FileNotFoundError):
        ck._load_files(tmp_path / "empty")


@pytest.mark.gpu
def test_from_pretrained_generates_like_in_memory(gpu, tmp_path):
    """A model loaded from disk (sharded, untied lm_head) decodes exactly as the same
    tensors handed over in memory, and matches the oracle that holds them."""
    from oracle import qwen3 as oq
    cfg = gm.Qwen3Config(n_layers=2, vocab=2048)
    t = gm.random_qwen3_tensors(cfg, seed=5, weights="centered")
    t["lm_head.weight"] = (torch.randn(cfg.vocab, cfg.hidden, generator=torch.Generator().manual_seed(6))
                           .to(torch.bfloat16).float().numpy())
    ck.write_checkpoint(tmp_path, t, cfg, shards=2)
    prompt = torch.randint(0, cfg.vocab, (4, 20), generator=torch.Generator().manual_seed(7))
    a = gm.Qwen3Model.from_pretrained(tmp_path, batch=4, ctx_cap=48, device=gpu).generate(prompt, 8)
    b = gm.Qwen3Model(t, cfg, batch=4, ctx_cap=48, device=gpu).generate(prompt, 8)
    assert torch.equal(a, b)
    ocfg = oq.Qwen3Config(**{k: getattr(cfg, k) for k in oq.Qwen3Config.__dataclass_fields__})
    ref = oq.DenseQwen3(t, ocfg, mode="fp32", ctx_cap=48).generate(prompt, 8)
    assert (a == ref).all(dim=1).float().mean() >= 0.75
