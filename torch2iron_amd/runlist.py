"""Runlists of ``(operator, *buffer_names)`` entries, executed on the GPU.

The reference assembles a decode step as a runlist of operator entries over
named buffers and hands it to ``FusedMLIROperator``
(``torch2iron/fusion.py:333-510``), which checks every entry against the
operator's ``get_arg_spec()``, sizes the buffers and runs the entries in order
as one NPU dispatch.  ``FusedRunlist`` takes the same runlist form with the
operators of ``torch2iron_amd.operators`` and runs the entries in order on
torch's current stream (capturable into one HIP graph):

* an entry is ``(op, *names)``; ``len(names)`` must equal ``len(op.get_arg_spec())``
  (``fusion.py:466-472``);
* ``"base[start:end]"`` names a byte range of buffer ``base`` (the reference's
  ``_slice``, ``batch_decode_fused.py:59-62``);
* buffers named in ``buffers`` (weights, caches, inputs) are the caller's;
  every other buffer is allocated once from its arg spec, and a buffer named
  twice must have the same number of elements both times (``fusion.py:486-491``).

``qwen3_decode_runlist`` writes the per-layer runlist of
``batch_decode_fused.py:426-539`` for this build's operators, and
``qwen3_decode_buffers`` binds a ``model.Qwen3Model``'s weights and caches to
its names.
"""

from __future__ import annotations

import math

import torch

from torch2iron_amd import operators as O
from torch2iron_amd.formats import W4A16Weight


def _split(name: str):
    if "[" in name and name.endswith("]"):
        base = name[: name.index("[")]
        start, end = map(int, name[name.index("[") + 1: -1].split(":"))
        return base, start, end
    return name, None, None


class FusedRunlist:
    """Checks a runlist against its operators' arg specs and runs it."""

    def __init__(self, name: str, runlist, input_args, output_args, buffers: dict, device):
        for entry in runlist:
            op, *bufs = entry
            if not (hasattr(op, "get_arg_spec") and callable(op) and all(isinstance(b, str) for b in bufs)):
                raise TypeError("runlist entries must be (operator, *str) tuples")
        self.name = name
        self.runlist = list(runlist)
        self.device = torch.device(device)
        self._bufs = dict(buffers)
        sizes: dict = {}
        for op, *bufs in self.runlist:
            specs = op.get_arg_spec()
            if len(specs) != len(bufs):
                raise ValueError(f"Number of buffers ({len(bufs)}) must match operator "
                                 f"argument specification ({len(specs)}) for {op!r}")
            for b, spec in zip(bufs, specs):
                base, start, _ = _split(b)
                if start is not None:
                    if base not in self._bufs and base not in sizes:
                        raise ValueError(f"Sliced buffer {b!r} requires a sized base buffer {base!r}")
                    continue
                if spec.dtype is W4A16Weight:
                    if b not in self._bufs:
                        raise ValueError(f"weight buffer {b!r} must be given")
                    continue
                n = math.prod(spec.shape)
                if b in sizes and sizes[b][0] != n:
                    raise ValueError(f"Buffer {b!r} has conflicting sizes: {sizes[b][0]} vs {n}")
                sizes.setdefault(b, (n, spec.dtype))
        for b, (n, dtype) in sizes.items():
            if b in self._bufs:
                t = self._bufs[b]
                if isinstance(t, torch.Tensor) and t.numel() < n:
                    raise ValueError(f"buffer {b!r} holds {t.numel()} elements, the runlist needs {n}")
            else:
                self._bufs[b] = torch.zeros(n, dtype=dtype, device=self.device)
        names = set(self._bufs) | {_split(b)[0] for _, *bs in self.runlist for b in bs}
        for arg in list(input_args) + list(output_args):
            if arg not in names:
                raise ValueError(f"argument {arg!r} not found in runlist buffers")
        self.input_args = list(input_args)
        self.output_args = list(output_args)

    def get_buffer(self, name: str):
        """The tensor (or weight) a buffer name resolves to; a slice is a view."""
        base, start, end = _split(name)
        t = self._bufs[base]
        if start is None:
            return t
        flat = t.view(-1)
        item = flat.element_size()
        if start % item or end % item or end > flat.numel() * item:
            raise ValueError(f"slice {name!r} is not whole {flat.dtype} elements inside {base!r}")
        return flat[start // item: end // item]

    def __call__(self):
        for op, *bufs in self.runlist:
            op(*[self.get_buffer(b) for b in bufs])


def _slice(name: str, start_elements: int, length_elements: int, itemsize: int = 2) -> str:
    """Byte-range name of ``length_elements`` values from ``start_elements`` (bf16 by default)."""
    return f"{name}[{start_elements * itemsize}:{(start_elements + length_elements) * itemsize}]"


def qwen3_decode_runlist(cfg, rows: int, ctx_cap: int, n_layers: int | None = None):
    """The decode step's runlist over ``n_layers`` layers (default all) for ``rows``
    sequences: per layer the five entries of the GPU decode layer, then the final
    RMSNorm is left to the caller (the model's head).  Buffer names follow the
    reference's (``x``, ``attn_context``, ``ffn_hidden``, ``W_norm1_{i}``, ...)."""
    n_layers = cfg.n_layers if n_layers is None else n_layers
    qkv_op = O.Qwen3FusedQKVProjection(cfg.hidden, cfg.qkv_dim, rows=rows, rms_norm_epsilon=cfg.eps)
    attn_op = O.Qwen3DecodeAttention(cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, ctx_cap, rows=rows,
                                     rms_norm_epsilon=cfg.eps, rope_style=cfg.rope_style)
    o_op = O.Qwen3FusedLinearResidualProjection(cfg.n_heads * cfg.head_dim, cfg.hidden, rows=rows)
    up_gate_op = O.Qwen3FusedUpGateProjection(cfg.hidden, cfg.intermediate, rows=rows, rms_norm_epsilon=cfg.eps)
    down_op = O.Qwen3FusedLinearResidualProjection(cfg.intermediate, cfg.hidden, rows=rows)
    runlist = []
    for i in range(n_layers):
        runlist.extend([
            (qkv_op, "x", f"W_norm1_{i}", f"W_attn_qkv_{i}", "qkv"),
            (attn_op, "qkv", "positions", f"W_attn_query_norm_{i}", f"W_attn_key_norm_{i}", "rope_angles",
             f"k_cache_{i}", f"v_cache_{i}", "attn_context"),
            (o_op, "attn_context", "x", f"W_attn_output_{i}", "x"),
            (up_gate_op, "x", f"W_norm2_{i}", f"W_ffn_gate_up_{i}", "ffn_hidden"),
            (down_op, "ffn_hidden", "x", f"W_ffn_down_{i}", "x"),
        ])
    return runlist


def qwen3_decode_buffers(model, n_layers: int | None = None, batch_rows: slice = slice(None)) -> dict:
    """Bind a ``model.Qwen3Model``'s weights, KV caches, RoPE table and its
    residual stream / positions to the names of ``qwen3_decode_runlist``."""
    n_layers = model.cfg.n_layers if n_layers is None else n_layers
    bufs = {"x": model.x[batch_rows], "positions": model.positions[batch_rows], "rope_angles": model.rope}
    for i in range(n_layers):
        w = model.layers[i].w
        bufs.update({
            f"W_norm1_{i}": w.ln1, f"W_attn_qkv_{i}": w.qkv, f"W_attn_query_norm_{i}": w.q_norm,
            f"W_attn_key_norm_{i}": w.k_norm, f"k_cache_{i}": model.k_cache[i, batch_rows],
            f"v_cache_{i}": model.v_cache[i, batch_rows], f"W_attn_output_{i}": w.o,
            f"W_norm2_{i}": w.ln2, f"W_ffn_gate_up_{i}": w.gate_up, f"W_ffn_down_{i}": w.down,
        })
    return bufs
