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

    def __init__(self, name: str, runlist, input_args, output_args, buffers: dict, device,
                 buffer_sizes: dict | None = None):
        for entry in runlist:
            op, *bufs = entry
            if not (hasattr(op, "get_arg_spec") and callable(op) and all(isinstance(b, str) for b in bufs)):
                raise TypeError("runlist entries must be (operator, *str) tuples")
        self.name = name
        self.runlist = list(runlist)
        self.device = torch.device(device)
        self._bufs = dict(buffers)
        explicit = dict(buffer_sizes or {})   # bytes, as the reference's buffer_sizes
        sizes: dict = {}
        for op, *bufs in self.runlist:
            specs = op.get_arg_spec()
            if len(specs) != len(bufs):
                raise ValueError(f"Number of buffers ({len(bufs)}) must match operator "
                                 f"argument specification ({len(specs)}) for {op!r}")
            for b, spec in zip(bufs, specs):
                base, start, _ = _split(b)
                if start is not None:
                    if base not in self._bufs and base not in sizes and base not in explicit:
                        raise ValueError(f"Sliced buffer {b!r} requires explicit size for base buffer {base!r}")
                    continue
                if spec.dtype is W4A16Weight:
                    if b not in self._bufs:
                        raise ValueError(f"weight buffer {b!r} must be given")
                    continue
                n = math.prod(spec.shape)
                if b in sizes and sizes[b][0] != n:
                    raise ValueError(f"Buffer {b!r} has conflicting sizes: {sizes[b][0]} vs {n}")
                sizes.setdefault(b, (n, spec.dtype))
        for b, nbytes in explicit.items():
            if b in self._bufs or b in sizes:
                continue
            dtype = torch.bfloat16 if nbytes % 2 == 0 else torch.uint8
            sizes[b] = (nbytes // (2 if dtype is torch.bfloat16 else 1), dtype)
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


# ---------------------------------------------------------------------------
# The reference's batch-decode runlist, entry for entry
# ---------------------------------------------------------------------------
# quantized_qwen3/batch_decode_fused.py:44-52 and runtime_config.py: the row
# buckets and NPU tiling constants its operators are constructed with.
BATCH_DECODE_ROW_BUCKETS = (4, 8, 16, 32)
BATCH_DECODE_COLUMNS = 8
BATCH_DECODE_GEMM_TILE_M = 8
BATCH_DECODE_GEMM_TILE_K = 128
BATCH_DECODE_TRANSFORMER_TILE_N = 64
BATCH_DECODE_LM_HEAD_TILE_N = 64
DECODE_ATTN_CHUNK_SIZE = 64


def select_batch_decode_rows(batch_size: int) -> int:
    """The padded row count of a batch (``batch_decode_fused.py:64-70``)."""
    for rows in BATCH_DECODE_ROW_BUCKETS:
        if batch_size <= rows:
            return rows
    raise ValueError(f"batch_size {batch_size} exceeds padded rows {BATCH_DECODE_ROW_BUCKETS[-1]}")


def _gemm_tile_m(rows: int) -> int:
    return 4 if rows <= 8 else BATCH_DECODE_GEMM_TILE_M


def _gemm_fields(rows: int, tile_n: int = BATCH_DECODE_TRANSFORMER_TILE_N) -> dict:
    tm = _gemm_tile_m(rows)
    return dict(num_aie_columns=BATCH_DECODE_COLUMNS, num_aie_rows=rows // tm, tile_m=tm,
                tile_k=BATCH_DECODE_GEMM_TILE_K, tile_n=tile_n)


def _n_shard_rows(n: int, tile_n: int) -> int:
    groups = n // (tile_n * BATCH_DECODE_COLUMNS)
    for rows in (4, 3, 2, 1):
        if groups % rows == 0:
            return rows
    raise ValueError(f"N={n} cannot be sharded across {BATCH_DECODE_COLUMNS} columns")


def batch_decode_runlist(cfg, max_seq_len: int, batch_size: int, lm_head_out_features: int | None = None,
                         context=None) -> dict:
    """The per-step runlist of the reference's batch decoder
    (``batch_decode_fused.py:300-539``) with this build's operators, constructed
    with the reference's own arguments (``:336-425``).  One substitution: the
    per-row pair ``CopyPresentPacketKV`` + ``LlamaChunkedAttention`` over a
    64-slot packet cache becomes one ``CopyPresentKVAttention`` entry per row
    over the contiguous cache ``k_cache_{l}`` / ``v_cache_{l}`` ``[batch, Hkv,
    max_seq_len, D]``, which takes each row's position from ``positions`` (int32
    ``[batch_size]``) instead of a packet mask.

    With ``lm_head_out_features`` the step ends with the int4 lm_head GEMM
    (``W_out_head_qparam`` -> ``logits``), as the reference's does; without it
    the runlist ends at ``hidden_out`` (the final RMSNorm's output), for a caller
    that runs the tied bf16 head (``ops.lm_head_argmax``).

    Returns ``runlist``, ``input_args``, ``output_args``, ``buffer_sizes`` (bytes)
    and ``decode_rows`` (the padded row count every GEMM runs over).
    """
    if batch_size < 1:
        raise ValueError("batch_size must be positive")
    if max_seq_len % DECODE_ATTN_CHUNK_SIZE != 0:
        raise ValueError(f"max_seq_len must be divisible by {DECODE_ATTN_CHUNK_SIZE}")
    decode_rows = select_batch_decode_rows(batch_size)
    emb, hidden = cfg.hidden, cfg.intermediate
    n_heads, n_kv = cfg.n_heads, cfg.n_kv_heads
    head_dim = cfg.head_dim
    attn_dim, kv_dim = n_heads * head_dim, n_kv * head_dim
    x_elements = decode_rows * emb
    ffn_elements = decode_rows * hidden
    norm_columns = min(BATCH_DECODE_COLUMNS, decode_rows)

    rms_norm_op = O.RMSNorm(size=x_elements, num_aie_columns=norm_columns, num_channels=1, tile_size=emb,
                            weighted=True, context=context)
    rope_q_op = O.RMSNormRoPE(rows=decode_rows * n_heads, cols=head_dim, angle_rows=decode_rows,
                              num_aie_columns=norm_columns, context=context)
    rope_k_op = O.RMSNormRoPE(rows=decode_rows * n_kv, cols=head_dim, angle_rows=decode_rows,
                              num_aie_columns=norm_columns, context=context)
    fields = _gemm_fields(decode_rows)
    query_op = O.W4A16KGroupGEMM(M=decode_rows, K=emb, N=attn_dim, k_group=4, context=context, **fields)
    key_value_op = O.W4A16PairedKGroupGEMM(M=decode_rows, K=emb, N=kv_dim, k_group=2, context=context, **fields)
    output_op = O.W4A16KGroupGEMM(M=decode_rows, K=attn_dim, N=emb, k_group=2, context=context, **fields)
    up_gate_op = O.W4A16PairedKGroupGEMM(M=decode_rows, K=emb, N=hidden, k_group=2, context=context, **fields)
    down_op = O.W4A16KGroupGEMM(M=decode_rows, K=hidden, N=emb, k_group=2, context=context, **fields)
    silu_mul_op = O.SiLUMul(size=ffn_elements, tile_size=hidden // BATCH_DECODE_COLUMNS,
                            num_aie_columns=BATCH_DECODE_COLUMNS, context=context)
    residual_norm_op = O.ResidualAddRMSNorm(size=x_elements, tile_size=emb, num_aie_columns=norm_columns,
                                            context=context)
    attention_op = O.CopyPresentKVAttention(max_seq_len=max_seq_len, num_kv_groups=n_kv,
                                            q_heads_per_group=n_heads // n_kv, head_dim=head_dim,
                                            chunk_size=DECODE_ATTN_CHUNK_SIZE, rows=1, context=context)
    cache_elements = n_kv * max_seq_len * head_dim

    runlist = [(rms_norm_op, "x", "W_norm1_0", "x_norm")]
    for i in range(cfg.n_layers):
        runlist.extend([
            (query_op, "x_norm", f"W_attn_query_{i}_qparam", "queries"),
            (key_value_op, "x_norm", f"W_attn_key_value_{i}_qparam", "keys", "values"),
            (rope_q_op, "queries", f"W_attn_query_norm_{i}", "rope_angles", "queries"),
            (rope_k_op, "keys", f"W_attn_key_norm_{i}", "rope_angles", "keys"),
        ])
        for b in range(batch_size):
            runlist.append((attention_op, _slice("queries", b * attn_dim, attn_dim),
                            _slice("keys", b * kv_dim, kv_dim), _slice("values", b * kv_dim, kv_dim),
                            _slice("positions", b, 1, itemsize=4),
                            _slice(f"k_cache_{i}", b * cache_elements, cache_elements),
                            _slice(f"v_cache_{i}", b * cache_elements, cache_elements),
                            _slice("attn_context", b * attn_dim, attn_dim)))
        runlist.extend([
            (output_op, "attn_context", f"W_attn_output_decode_{i}_qparam", "attn_output"),
            (residual_norm_op, "x", "attn_output", f"W_norm2_{i}", "x", "x_norm"),
            (up_gate_op, "x_norm", f"W_ffn_gate_up_{i}_qparam", "ffn_gate", "ffn_up"),
            (silu_mul_op, "ffn_gate", "ffn_up", "ffn_hidden"),
            (down_op, "ffn_hidden", f"W_ffn_down_{i}_qparam", "ffn_output"),
        ])
        last = i + 1 == cfg.n_layers
        runlist.append((residual_norm_op, "x", "ffn_output", "W_final_norm" if last else f"W_norm1_{i + 1}",
                        "x", "hidden_out" if last else "x_norm"))
    output_args = ["hidden_out"]
    if lm_head_out_features is not None:
        lm_head_op = O.W4A16NShardGEMM(M=decode_rows, K=emb, N=lm_head_out_features,
                                       num_aie_columns=BATCH_DECODE_COLUMNS,
                                       num_aie_rows=_n_shard_rows(lm_head_out_features, BATCH_DECODE_LM_HEAD_TILE_N),
                                       tile_m=_gemm_tile_m(decode_rows), tile_k=BATCH_DECODE_GEMM_TILE_K,
                                       tile_n=BATCH_DECODE_LM_HEAD_TILE_N, context=context)
        runlist.append((lm_head_op, "hidden_out", "W_out_head_qparam", "logits"))
        output_args = ["logits"]
    output_args += [f"{kind}_cache_{i}" for kind in ("k", "v") for i in range(cfg.n_layers)]
    buffer_sizes = {"attn_context": decode_rows * attn_dim * 2, "queries": decode_rows * attn_dim * 2,
                    "keys": decode_rows * kv_dim * 2, "values": decode_rows * kv_dim * 2}
    return {"runlist": runlist, "input_args": ["x", "rope_angles", "positions"], "output_args": output_args,
            "buffer_sizes": buffer_sizes, "decode_rows": decode_rows}


def batch_decode_weights(tensors: dict, cfg, device, lm_head: tuple | None = None) -> dict:
    """The weight buffers of ``batch_decode_runlist`` from AutoGPTQ tensors under
    HF names: q alone, k|v and gate|up paired (pair 0 = key / gate), o_proj,
    down, the norm weights; ``lm_head`` an optional AutoGPTQ triple for
    ``W_out_head_qparam``.  On a GPU each linear also gets its decode-linear tiles
    (``ops.tile_weight``)."""
    from torch2iron_amd.formats import interleave_gate_up

    def trip(name):
        return (tensors[f"{name}.qweight"], tensors[f"{name}.qzeros"], tensors[f"{name}.scales"])

    def bf16(a):
        return torch.as_tensor(a, dtype=torch.float32).to(torch.bfloat16).to(device).contiguous()

    out = {"W_final_norm": bf16(tensors["model.norm.weight"])}
    for i in range(cfg.n_layers):
        p = f"model.layers.{i}"
        out.update({
            f"W_norm1_{i}": bf16(tensors[f"{p}.input_layernorm.weight"]),
            f"W_norm2_{i}": bf16(tensors[f"{p}.post_attention_layernorm.weight"]),
            f"W_attn_query_norm_{i}": bf16(tensors[f"{p}.self_attn.q_norm.weight"]),
            f"W_attn_key_norm_{i}": bf16(tensors[f"{p}.self_attn.k_norm.weight"]),
            f"W_attn_query_{i}_qparam": W4A16Weight.from_numpy(*trip(f"{p}.self_attn.q_proj"), device=device),
            f"W_attn_key_value_{i}_qparam": W4A16Weight.from_numpy(
                *interleave_gate_up(trip(f"{p}.self_attn.k_proj"), trip(f"{p}.self_attn.v_proj")), device=device),
            f"W_attn_output_decode_{i}_qparam": W4A16Weight.from_numpy(*trip(f"{p}.self_attn.o_proj"), device=device),
            f"W_ffn_gate_up_{i}_qparam": W4A16Weight.from_numpy(
                *interleave_gate_up(trip(f"{p}.mlp.gate_proj"), trip(f"{p}.mlp.up_proj")), device=device),
            f"W_ffn_down_{i}_qparam": W4A16Weight.from_numpy(*trip(f"{p}.mlp.down_proj"), device=device),
        })
    if lm_head is not None:
        out["W_out_head_qparam"] = W4A16Weight.from_numpy(*lm_head, device=device)
    if torch.device(device).type == "cuda":
        # resident decode weights: their decode-linear tiles too (bit-identical outputs)
        from torch2iron_amd import ops
        for w in out.values():
            if isinstance(w, W4A16Weight):
                ops.tile_weight(w)
    return out
