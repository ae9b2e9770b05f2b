"""AutoGPTQ W4A16 Qwen3 checkpoints on disk (safetensors + config.json).

Reads a Hugging Face-style model directory the way the reference reads it
before packing (``quantized_qwen3/packed_format.py:71-85``: ``model.safetensors``
or the shards listed in ``model.safetensors.index.json``; the config fields of
``quantized_qwen3/model.py:380-390`` and ``qwen_inference_harness.py:40-53``),
and returns the tensors the device model takes, unchanged:

* per linear ``<prefix>.qweight`` int32 ``[K/8, N]``, ``.qzeros`` int32
  ``[K/128, N/8]``, ``.scales`` fp16 ``[K/128, N]``;
* dense tensors (norm weights, the embedding, an untied ``lm_head.weight``)
  as float32 arrays holding their bf16 values.

Unlike the reference's packer (``packed_format.py:414-419``, which requires
``sym``), asymmetric checkpoints are accepted: the kernels keep the zero points.
Rejected with ``ValueError``: bits other than 4, a group size other than 128,
act-order checkpoints (a ``g_idx`` that is not ``k // group_size``, which the
reference also ignores, ``packed_format.py:454``) and a quantised lm_head.
``write_checkpoint`` writes the same layout (tests and conversions).
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import torch

from torch2iron_amd.model import Qwen3Config

SINGLE = "model.safetensors"
INDEX = "model.safetensors.index.json"


def _load_files(model_dir: Path) -> dict:
    from safetensors.torch import load_file

    single = model_dir / SINGLE
    if single.exists():
        return load_file(str(single))
    index = model_dir / INDEX
    if not index.exists():
        raise FileNotFoundError(f"no {SINGLE} or {INDEX} in {model_dir}")
    files = sorted(set(json.loads(index.read_text())["weight_map"].values()))
    tensors: dict = {}
    for name in files:
        tensors.update(load_file(str(model_dir / name)))
    return tensors


def config_from_hf(hf: dict) -> Qwen3Config:
    """``Qwen3Config`` from a Hugging Face ``config.json`` dict (W4A16 AutoGPTQ)."""
    q = hf.get("quantization_config") or {}
    bits = int(q.get("bits", 4))
    if bits != 4:
        raise ValueError(f"only 4-bit (W4A16) checkpoints are supported, got bits={bits}")
    group = int(q.get("group_size", 128))
    if group != 128:
        raise ValueError(f"only group_size 128 is supported, got {group}")
    if q.get("desc_act", False):
        raise ValueError("act-order (desc_act) checkpoints are not supported")
    hidden = int(hf["hidden_size"])
    heads = int(hf["num_attention_heads"])
    rope = hf.get("rope_parameters") or {}
    return Qwen3Config(
        hidden=hidden,
        n_heads=heads,
        n_kv_heads=int(hf["num_key_value_heads"]),
        head_dim=int(hf.get("head_dim", hidden // heads)),
        intermediate=int(hf["intermediate_size"]),
        n_layers=int(hf["num_hidden_layers"]),
        vocab=int(hf["vocab_size"]),
        eps=float(hf.get("rms_norm_eps", 1e-6)),
        rope_theta=float(rope.get("rope_theta", hf.get("rope_theta", 1e6))),
        group_size=group,
    )


def load_checkpoint(model_dir) -> tuple[dict, Qwen3Config]:
    """Tensors (numpy, HF names) and config of an AutoGPTQ W4A16 Qwen3 directory."""
    model_dir = Path(model_dir).expanduser()
    hf = json.loads((model_dir / "config.json").read_text())
    cfg = config_from_hf(hf)
    raw = _load_files(model_dir)
    if "lm_head.qweight" in raw:
        raise ValueError("a quantised lm_head is not supported (the lm_head is a bf16 matrix)")
    out = {}
    for name, t in raw.items():
        if name.endswith(".g_idx"):
            k = t.numel()
            if not torch.equal(t.to(torch.int64), torch.arange(k) // cfg.group_size):
                raise ValueError(f"{name}: act-order (non-sequential g_idx) checkpoints are not supported")
            continue
        if name.endswith((".qweight", ".qzeros")):
            if t.dtype != torch.int32:
                raise ValueError(f"{name} must be int32, got {t.dtype}")
            out[name] = t.numpy()
        elif name.endswith(".scales"):
            out[name] = t.to(torch.float16).numpy()
        else:
            # dense tensors are bf16 in the model; keep their bf16 values
            out[name] = t.to(torch.bfloat16).float().numpy()
    tied = bool(hf.get("tie_word_embeddings", "lm_head.weight" not in out))
    if tied:
        out.pop("lm_head.weight", None)
    _check_complete(out, cfg)
    return out, cfg


def _check_complete(t: dict, cfg: Qwen3Config) -> None:
    need = ["model.embed_tokens.weight", "model.norm.weight"]
    for i in range(cfg.n_layers):
        p = f"model.layers.{i}"
        for lin in ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
                    "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"):
            need += [f"{p}.{lin}.{s}" for s in ("qweight", "qzeros", "scales")]
        need += [f"{p}.input_layernorm.weight", f"{p}.post_attention_layernorm.weight",
                 f"{p}.self_attn.q_norm.weight", f"{p}.self_attn.k_norm.weight"]
    missing = [n for n in need if n not in t]
    if missing:
        raise ValueError(f"checkpoint is missing {len(missing)} tensors, e.g. {missing[:3]}")


def write_checkpoint(model_dir, tensors: dict, cfg: Qwen3Config, shards: int = 1, sym: bool = False) -> None:
    """Write ``tensors`` (the layout ``load_checkpoint`` returns) as an AutoGPTQ
    directory: ``config.json`` plus one safetensors file, or ``shards`` files and
    an index.  Dense tensors are stored as bf16."""
    from safetensors.torch import save_file

    model_dir = Path(model_dir)
    model_dir.mkdir(parents=True, exist_ok=True)
    hf = {
        "architectures": ["Qwen3ForCausalLM"], "model_type": "qwen3",
        "hidden_size": cfg.hidden, "num_attention_heads": cfg.n_heads, "num_key_value_heads": cfg.n_kv_heads,
        "head_dim": cfg.head_dim, "intermediate_size": cfg.intermediate, "num_hidden_layers": cfg.n_layers,
        "vocab_size": cfg.vocab, "rms_norm_eps": cfg.eps, "rope_theta": cfg.rope_theta,
        "tie_word_embeddings": "lm_head.weight" not in tensors,
        "quantization_config": {"quant_method": "gptq", "bits": 4, "group_size": cfg.group_size,
                                "desc_act": False, "sym": sym},
    }
    (model_dir / "config.json").write_text(json.dumps(hf, indent=1))
    tt = {}
    for name, a in tensors.items():
        a = np.ascontiguousarray(a)
        if name.endswith((".qweight", ".qzeros")):
            tt[name] = torch.from_numpy(a.view(np.int32))
        elif name.endswith(".scales"):
            tt[name] = torch.from_numpy(a.astype(np.float16))
        else:
            tt[name] = torch.from_numpy(a.astype(np.float32)).to(torch.bfloat16)
    names = sorted(tt)
    if shards <= 1:
        save_file(tt, str(model_dir / SINGLE))
        return
    weight_map = {}
    for s in range(shards):
        part = names[s::shards]
        fname = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
        save_file({n: tt[n] for n in part}, str(model_dir / fname))
        weight_map.update({n: fname for n in part})
    (model_dir / INDEX).write_text(json.dumps({"metadata": {}, "weight_map": weight_map}, indent=1))
