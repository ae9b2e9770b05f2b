"""W4A16 Qwen3 decoder on one MI355X: the fused decode layer and batched greedy decode.

Per layer and decode step (batch B, one token per sequence), five launches:

1. ``t2i_w4a16_rmsnorm_linear``   input RMSNorm + fused q|k|v projection (N = (Hq + 2 Hkv) * D);
                                  layer 0 instead takes the rows that ``t2i_rmsnorm`` gathered
                                  from the embedding and normalised
2. ``t2i_decode_attention``       q/k RMSNorm + RoPE + KV-cache write + GQA attention
3. ``t2i_w4a16_linear``           o_proj with the residual add folded in (in place)
4. ``t2i_w4a16_rmsnorm_gate_up``  post-attention RMSNorm + fused gate|up projection + SwiGLU
5. ``t2i_w4a16_linear``           down projection with the residual add (in place)

then the final RMSNorm, the tied bf16 lm_head with the fused argmax, and the
device-side token bookkeeping.  This is the per-layer runlist of the
reference's NPU batch decoder (``quantized_qwen3/batch_decode_fused.py:426-539``)
re-cut for the GPU: q/k/v are one linear, gate/up one linear with SwiGLU, the
RMSNorms run inside the linears that consume them, and the RoPE, q/k-norm and
KV write live in the attention prologue.

A whole decode step is captured once into a HIP graph and replayed; token ids,
positions and the output history stay on the device between steps.  The
layers can instead run as one cooperative launch per step (``t2i_decode_step``,
``persistent=True``), whose phases match the separate kernels within one bf16
rounding (16-wave tiles: another order of the fp32 partial sums); it measured
slower (see ``Qwen3Model``) and is off by default.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

from torch2iron_amd import ops
from torch2iron_amd.formats import W4A16Weight, concat_columns, interleave_gate_up

BF16 = torch.bfloat16


@dataclass(frozen=True)
class Qwen3Config:
    """Shape of a Qwen3 decoder (``quantized_qwen3/model.py:330-348`` fields)."""

    hidden: int = 1024
    n_heads: int = 16
    n_kv_heads: int = 8
    head_dim: int = 128
    intermediate: int = 3072
    n_layers: int = 28
    vocab: int = 151936
    eps: float = 1e-6
    rope_theta: float = 1e6
    group_size: int = 128
    rope_style: str = "halves"

    @property
    def qkv_dim(self) -> int:
        return (self.n_heads + 2 * self.n_kv_heads) * self.head_dim


QWEN3_0_6B = Qwen3Config()
QWEN3_1_7B = Qwen3Config(hidden=2048, intermediate=6144)


def _rand_words(rng, shape):
    return rng.integers(0, 2**32, size=shape, dtype=np.uint64).astype(np.uint32).view(np.int32)


def _centered_words(rng, shape):
    nib = rng.integers(1, 16, size=(*shape, 8), dtype=np.uint64)
    acc = np.zeros(shape, dtype=np.uint64)
    for j in range(8):
        acc |= nib[..., j] << np.uint64(4 * j)
    return acc.astype(np.uint32).view(np.int32)


def random_qwen3_tensors(cfg: Qwen3Config, seed: int = 0, embed_std: float = 1.0,
                         weights: str = "uniform") -> dict:
    """Random-init Qwen3 tensors under HF names (numpy).

    Linears: AutoGPTQ group-128, fp16 scales U[0.005, 0.02].
    ``weights="uniform"``: uniform random words (nibbles and stored zeros
    uniform in 0..15, so ``q - z`` has mean -1).
    ``weights="centered"``: symmetric-checkpoint style, stored zero 7 (z = 8)
    and nibbles uniform in 1..15, so ``q - z`` is uniform in [-7, 7]; with
    the uniform draw, the non-zero mean of every weight row makes greedy decode
    collapse onto one token for every prompt, which leaves token parity nearly
    vacuous.
    RMSNorm weights U[0.9, 1.1] (bf16 values).  Embedding (also the tied
    lm_head) N(0, embed_std) rounded to bf16.
    ``weights="hubs"``: the centred linears with an embedding of N(0, 12) rows
    scaled by exp(0.3 N(0, 1)) each (a few large-norm rows), final-norm weights of
    random sign, and q/k norm weights scaled by 0.1 (near-uniform attention): the
    draw whose greedy tokens are both diverse and least disturbed by bf16 rounding
    among those searched for the full-model parity test.
    """
    if weights not in ("uniform", "centered", "hubs"):
        raise ValueError("weights must be 'uniform', 'centered' or 'hubs'")
    if weights == "hubs":
        t = random_qwen3_tensors(cfg, seed=seed, embed_std=12.0, weights="centered")
        r = np.exp(0.3 * np.random.default_rng(seed + 2000).standard_normal(cfg.vocab)).astype(np.float32)
        emb = t["model.embed_tokens.weight"] * r[:, None]
        t["model.embed_tokens.weight"] = torch.from_numpy(emb).to(BF16).float().numpy()
        sign = np.where(np.random.default_rng(seed + 1000).random(cfg.hidden) < 0.5, -1.0, 1.0).astype(np.float32)
        t["model.norm.weight"] = t["model.norm.weight"] * sign
        for i in range(cfg.n_layers):
            for nm in ("q_norm", "k_norm"):
                k = f"model.layers.{i}.self_attn.{nm}.weight"
                t[k] = torch.from_numpy(t[k] * 0.1).to(BF16).float().numpy()
        return t
    rng = np.random.default_rng(seed)
    g = cfg.group_size
    t = {}

    def lin(name, k, n):
        if weights == "uniform":
            t[f"{name}.qweight"] = _rand_words(rng, (k // 8, n))
            t[f"{name}.qzeros"] = _rand_words(rng, (k // g, n // 8))
        else:
            t[f"{name}.qweight"] = _centered_words(rng, (k // 8, n))
            t[f"{name}.qzeros"] = np.full((k // g, n // 8), 0x77777777, dtype=np.int64).astype(np.int32)
        t[f"{name}.scales"] = rng.uniform(0.005, 0.02, size=(k // g, n)).astype(np.float16)

    def bf16_values(a):
        return torch.from_numpy(np.asarray(a, dtype=np.float32)).to(BF16).float().numpy()

    h, d = cfg.hidden, cfg.head_dim
    for i in range(cfg.n_layers):
        p = f"model.layers.{i}"
        lin(f"{p}.self_attn.q_proj", h, cfg.n_heads * d)
        lin(f"{p}.self_attn.k_proj", h, cfg.n_kv_heads * d)
        lin(f"{p}.self_attn.v_proj", h, cfg.n_kv_heads * d)
        lin(f"{p}.self_attn.o_proj", cfg.n_heads * d, h)
        lin(f"{p}.mlp.gate_proj", h, cfg.intermediate)
        lin(f"{p}.mlp.up_proj", h, cfg.intermediate)
        lin(f"{p}.mlp.down_proj", cfg.intermediate, h)
        t[f"{p}.input_layernorm.weight"] = bf16_values(rng.uniform(0.9, 1.1, h))
        t[f"{p}.post_attention_layernorm.weight"] = bf16_values(rng.uniform(0.9, 1.1, h))
        t[f"{p}.self_attn.q_norm.weight"] = bf16_values(rng.uniform(0.9, 1.1, d))
        t[f"{p}.self_attn.k_norm.weight"] = bf16_values(rng.uniform(0.9, 1.1, d))
    t["model.norm.weight"] = bf16_values(rng.uniform(0.9, 1.1, h))
    emb = torch.randn(cfg.vocab, h, generator=torch.Generator().manual_seed(seed + 7)) * embed_std
    t["model.embed_tokens.weight"] = emb.to(BF16).float().numpy()
    return t


def rope_table(head_dim: int, ctx: int, theta: float, device) -> torch.Tensor:
    """bf16 ``[ctx, head_dim]``: cos at even, sin at odd columns of frequency i.

    Angles as ``quantized_qwen3/model.py:351-358`` (fp32 ``inv_freq``, fp32
    outer product), then rounded to bf16 as that runtime does in bf16 compute
    (``model.py:421-425``).
    """
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2).float() / head_dim))
    freqs = torch.outer(torch.arange(ctx).float(), inv_freq)
    ang = torch.empty(ctx, head_dim)
    ang[:, ::2] = torch.cos(freqs)
    ang[:, 1::2] = torch.sin(freqs)
    return ang.to(BF16).to(device)


def _bf16_dev(a, device) -> torch.Tensor:
    return torch.as_tensor(np.asarray(a, dtype=np.float32)).to(BF16).to(device).contiguous()


class Qwen3LayerWeights:
    """Device weights of one layer, fused for the GPU kernels.  On a GPU each linear
    also gets its decode-linear tiles (``ops.tile_weight``), which the decode-sized
    linears read; prompt batches and the one-launch forms read the AutoGPTQ words."""

    def __init__(self, tensors: dict, layer: int, cfg: Qwen3Config, device):
        p = f"model.layers.{layer}"

        def trip(name):
            return (tensors[f"{name}.qweight"], tensors[f"{name}.qzeros"], tensors[f"{name}.scales"])

        qkv = concat_columns(trip(f"{p}.self_attn.q_proj"), trip(f"{p}.self_attn.k_proj"),
                             trip(f"{p}.self_attn.v_proj"))
        self.qkv = W4A16Weight.from_numpy(*qkv, device=device)
        self.o = W4A16Weight.from_numpy(*trip(f"{p}.self_attn.o_proj"), device=device)
        self.gate_up = W4A16Weight.from_numpy(*interleave_gate_up(trip(f"{p}.mlp.gate_proj"),
                                                                 trip(f"{p}.mlp.up_proj")), device=device)
        self.down = W4A16Weight.from_numpy(*trip(f"{p}.mlp.down_proj"), device=device)
        if torch.device(device).type == "cuda":
            for w in (self.qkv, self.o, self.gate_up, self.down):
                ops.tile_weight(w)
        self.ln1 = _bf16_dev(tensors[f"{p}.input_layernorm.weight"], device)
        self.ln2 = _bf16_dev(tensors[f"{p}.post_attention_layernorm.weight"], device)
        self.q_norm = _bf16_dev(tensors[f"{p}.self_attn.q_norm.weight"], device)
        self.k_norm = _bf16_dev(tensors[f"{p}.self_attn.k_norm.weight"], device)


class DecodeBuffers:
    """Activations of one decode step for a batch of B sequences (preallocated, graph-safe).

    ``x`` / ``xn`` may be given as row slices of larger tensors, so several
    micro-batches can write their residual streams into one ``[B, hidden]``
    tensor that the lm_head then reads in one pass.
    """

    def __init__(self, cfg: Qwen3Config, batch: int, device, x: torch.Tensor | None = None,
                 xn: torch.Tensor | None = None):
        h = cfg.hidden
        self.x = torch.zeros(batch, h, dtype=BF16, device=device) if x is None else x      # residual stream
        self.xn = torch.zeros(batch, h, dtype=BF16, device=device) if xn is None else xn   # normed activations
        self.qkv = torch.zeros(batch, cfg.qkv_dim, dtype=BF16, device=device)
        self.ctx = torch.zeros(batch, cfg.n_heads * cfg.head_dim, dtype=BF16, device=device)
        self.hmlp = torch.zeros(batch, cfg.intermediate, dtype=BF16, device=device)
        # the chained RMSNorm's hand-over: the next norm's input (rows times its weight)
        # and the rows' sums of squares per 16-column block
        self.xg = torch.zeros(batch, h, dtype=BF16, device=device)
        self.ssp = torch.zeros(batch, h // 16, dtype=torch.float32, device=device)
        self.workspace = ops.Workspace()


class Qwen3DecodeLayer:
    """The fused decode layer: ``layer(x, positions, k_cache, v_cache)`` updates ``x`` in place.

    ``x`` bf16 ``[B, hidden]`` (the residual stream), ``positions`` int32
    ``[B]``, caches bf16 ``[B, Hkv, ctx_cap, D]``.  Mirrors the per-layer
    sequence of the reference's fused decode runlist
    (``batch_decode_fused.py:426-530``) and the reference layer semantics
    (``quantized_qwen3/model.py:316-327``).
    """

    def __init__(self, weights: Qwen3LayerWeights, cfg: Qwen3Config, rope: torch.Tensor):
        self.w = weights
        self.cfg = cfg
        self.rope = rope
        self.rope_style = ops.ROPE_HALVES if cfg.rope_style == "halves" else ops.ROPE_INTERLEAVED
        self.fused = False   # set by the model: the qkv projection and attention in one launch
        # set by the model: the chained RMSNorm (o_proj and down hand the next norm's input
        # over; qkv and gate_up take it), and the next layer's input-norm weight
        self.chain = False
        self.chain_in = False   # the previous layer's down hands this layer's input norm over
        self.next_ln1 = None

    def attention_half(self, buf: DecodeBuffers, positions, k_cache, v_cache, normed: bool = False):
        """``normed``: ``buf.xn`` already holds the normalised input (layer 0, whose
        RMSNorm is fused with the embedding gather); otherwise the RMSNorm runs
        inside the qkv linear."""
        c, w = self.cfg, self.w
        if self.fused:
            ops.qkv_attention(buf.xn if normed else buf.x, None if normed else w.ln1, c.eps, w.qkv, positions,
                              c.n_heads, c.n_kv_heads, w.q_norm, w.k_norm, self.rope, k_cache, v_cache,
                              rope_style=self.rope_style, out=buf.ctx, workspace=buf.workspace)
        else:
            if normed:
                ops.linear(buf.xn, w.qkv, out=buf.qkv)
            elif self.chain and self.chain_in:   # the previous layer's down left this norm's input in xg / ssp
                ops.prenormed_linear(buf.xg, buf.ssp, c.eps, w.qkv, out=buf.qkv)
            else:
                ops.rmsnorm_linear(buf.x, w.ln1, c.eps, w.qkv, out=buf.qkv)
            ops.decode_attention(buf.qkv, positions, c.n_heads, c.n_kv_heads, w.q_norm, w.k_norm, c.eps, self.rope,
                                 k_cache, v_cache, rope_style=self.rope_style, out=buf.ctx, workspace=buf.workspace)
        if self.chain:
            ops.linear_residual_next_norm(buf.ctx, w.o, buf.x, buf.x, w.ln2, buf.xg, buf.ssp)
        else:
            ops.linear(buf.ctx, w.o, residual=buf.x, out=buf.x)

    def mlp_half(self, buf: DecodeBuffers):
        c, w = self.cfg, self.w
        if self.chain:
            ops.prenormed_gate_up(buf.xg, buf.ssp, c.eps, w.gate_up, swiglu=True, out=buf.hmlp)
        else:
            ops.rmsnorm_gate_up(buf.x, w.ln2, c.eps, w.gate_up, swiglu=True, out=buf.hmlp)
        if self.chain and self.next_ln1 is not None:
            ops.linear_residual_next_norm(buf.hmlp, w.down, buf.x, buf.x, self.next_ln1, buf.xg, buf.ssp)
        else:
            ops.linear(buf.hmlp, w.down, residual=buf.x, out=buf.x)

    def __call__(self, buf: DecodeBuffers, positions, k_cache, v_cache, normed: bool = False):
        self.attention_half(buf, positions, k_cache, v_cache, normed)
        self.mlp_half(buf)


class _Micro:
    """One micro-batch: rows ``b0:b1`` of the batch, its stream, buffers and graphs."""

    def __init__(self, b0: int, b1: int, buf: DecodeBuffers, stream):
        self.b0, self.b1 = b0, b1
        self.buf = buf
        self.stream = stream
        self.done = torch.cuda.Event()
        self.graphs: dict = {}


def split_batch(batch: int, parts: int) -> list[tuple[int, int]]:
    """Contiguous, nearly equal row ranges covering ``range(batch)``."""
    parts = max(1, min(parts, batch))
    base, extra = divmod(batch, parts)
    out, b0 = [], 0
    for i in range(parts):
        b1 = b0 + base + (1 if i < extra else 0)
        out.append((b0, b1))
        b0 = b1
    return out


class Qwen3Model:
    """Random-init (or given) W4A16 Qwen3 with batched greedy decode on the GPU.

    Weights: AutoGPTQ linears (fused per layer), bf16 norms, bf16 tied
    embedding/lm_head.  KV cache: bf16 ``[layers, B, Hkv, ctx_cap, D]``.

    The batch is split into ``streams`` micro-batches of contiguous rows.  Each
    runs its 28-layer step on its own HIP stream (its own activations,
    attention workspace and KV-cache rows), so the fixed start/finish cost of
    one micro-batch's small launches overlaps with another's work on the other
    hardware queues.  The streams join once per step for the final RMSNorm and
    the tied lm_head with its argmax, which read the embedding table once for
    the whole batch.  Sequences never interact, and a linear's K split depends
    on its shape alone up to 16 rows, so the tokens do not depend on the split
    while every micro-batch has at most 16 rows (as does a batch of 16 or fewer
    in one stream).  Above 16 rows the linears split K another way (16 waves,
    or 32-column blocks), so a batch of 32 in one stream and the same batch as
    two 16-row streams sum their fp32 partials in different orders, and a
    near-tie can then pick another token.

    ``chain=True`` (the default, where every decode linear's plan has the form): the
    RMSNorm between o_proj and gate_up, and between a layer's down and the next
    layer's qkv, is handed over: o_proj and down also write the next norm's input
    (the rows times its weight) and the rows' sums of squares per 16 columns, which
    gate_up and qkv take in place of doing the norm themselves (the same bits up to
    the order in which a row's squares are summed; decode step 0.7755 -> 0.7565 ms at
    batch 16).  ``chain=False``: each norm inside its consumer, as the reference's
    fused projection operators do.

    Two one-launch alternatives, both off by default because they measured
    slower than the separate kernels (Qwen3-0.6B, batch 16, context 576):
    ``persistent=True`` runs every layer of a step in one cooperative launch
    (``ops.decode_step``, single stream, shapes with a one-launch plan): 1.33
    against 0.87 ms a step.  ``fused=True`` runs each layer's RMSNorm + qkv
    projection + attention as one cooperative launch (``ops.qkv_attention``):
    38.5 us a layer against 16.0 us for the two kernels, of which about 18 us is
    the cooperative launch itself.
    """

    def __init__(self, tensors: dict, cfg: Qwen3Config, batch: int, ctx_cap: int, device, streams: int = 1,
                 fused: bool = False, persistent: bool = False, chain: bool = True):
        self.cfg = cfg
        self.chain = chain
        self.fused_front = fused
        self.persistent = persistent
        self.batch = batch
        self.ctx_cap = ctx_cap
        self.device = torch.device(device)
        self.rope = rope_table(cfg.head_dim, ctx_cap, cfg.rope_theta, self.device)
        self.embed = _bf16_dev(tensors["model.embed_tokens.weight"], self.device)
        # the tied embedding is the lm_head unless the checkpoint holds its own (model.py:410-420)
        self.lm_head = (_bf16_dev(tensors["lm_head.weight"], self.device) if "lm_head.weight" in tensors
                        else self.embed)
        self.norm = _bf16_dev(tensors["model.norm.weight"], self.device)
        self.layers = [Qwen3DecodeLayer(Qwen3LayerWeights(tensors, i, cfg, self.device), cfg, self.rope)
                       for i in range(cfg.n_layers)]
        shape = (cfg.n_layers, batch, cfg.n_kv_heads, ctx_cap, cfg.head_dim)
        self.k_cache = torch.zeros(shape, dtype=BF16, device=self.device)
        self.v_cache = torch.zeros(shape, dtype=BF16, device=self.device)
        self.x = torch.zeros(batch, cfg.hidden, dtype=BF16, device=self.device)
        self.xn = torch.zeros(batch, cfg.hidden, dtype=BF16, device=self.device)
        self.set_streams(streams)
        self.tokens = torch.zeros(batch, dtype=torch.int32, device=self.device)
        self.positions = torch.zeros(batch, dtype=torch.int32, device=self.device)
        self.keys = torch.zeros(batch, dtype=torch.int64, device=self.device)
        self.step = torch.zeros(1, dtype=torch.int32, device=self.device)
        self.history = None
        self.prompt = None
        self.logits = None

    @classmethod
    def from_pretrained(cls, model_dir, batch: int, ctx_cap: int, device, streams: int = 1) -> "Qwen3Model":
        """Load an AutoGPTQ W4A16 Qwen3 directory (``checkpoint.load_checkpoint``)."""
        from torch2iron_amd.checkpoint import load_checkpoint

        tensors, cfg = load_checkpoint(model_dir)
        return cls(tensors, cfg, batch=batch, ctx_cap=ctx_cap, device=device, streams=streams)

    def fused_front_ok(self, rows: int, streams: int) -> bool:
        """Whether the one-launch qkv + attention front applies: a single stream (the
        launch takes every CU), at most 16 rows, 1 or 2 q heads per kv head, and one
        workgroup per (sequence, kv head) available."""
        c = self.cfg
        q = c.n_heads // c.n_kv_heads
        cus = torch.cuda.get_device_properties(self.device).multi_processor_count
        return (self.fused_front and streams == 1 and rows <= 16 and q in (1, 2) and c.head_dim == 128
                and rows * c.n_kv_heads <= cus)

    def set_streams(self, streams: int) -> None:
        """Split the batch into ``streams`` micro-batches (drops captured graphs)."""
        if streams < 1:
            raise ValueError("streams must be at least 1")
        rows = -(-self.batch // max(1, min(streams, self.batch)))
        fused = self.fused_front_ok(rows, streams)
        chain = self.chain and not fused and self.chain_ok(rows)
        for i, layer in enumerate(self.layers):
            layer.fused = fused
            layer.chain = chain
            layer.chain_in = chain and i > 0
            layer.next_ln1 = self.layers[i + 1].w.ln1 if chain and i + 1 < len(self.layers) else None
        self.micro = []
        for b0, b1 in split_batch(self.batch, streams):
            buf = DecodeBuffers(self.cfg, b1 - b0, self.device, x=self.x[b0:b1], xn=self.xn[b0:b1])
            stream = torch.cuda.Stream(self.device) if streams > 1 else None
            self.micro.append(_Micro(b0, b1, buf, stream))
        self.step_table = self._step_table() if self.persistent and len(self.micro) == 1 else None
        self._head_graph = None
        self._captured = False

    def chain_ok(self, rows: int) -> bool:
        """Whether every decode linear of a ``rows``-row micro-batch has its chained-norm
        form (o_proj and down hand the next RMSNorm's input over, qkv and gate_up take
        it; the layers' weights carry tiles)."""
        c = self.cfg
        if self.device.type != "cuda" or c.hidden not in (1024, 2048):
            return False
        if any(L.w.qkv.tiles is None or L.w.o.tiles is None or L.w.gate_up.tiles is None or L.w.down.tiles is None
               for L in self.layers):
            return False
        return (ops.chain_supported(rows, c.n_heads * c.head_dim, c.hidden, ops.CHAIN_PRODUCER)
                and ops.chain_supported(rows, c.intermediate, c.hidden, ops.CHAIN_PRODUCER)
                and ops.chain_supported(rows, c.hidden, c.qkv_dim, ops.CHAIN_CONSUMER)
                and ops.chain_supported(rows, c.hidden, 2 * c.intermediate, ops.CHAIN_PAIRED_CONSUMER))

    def _step_table(self):
        """The one-launch step's layer table, or None when the shapes have no one-launch plan."""
        c = self.cfg
        if c.head_dim != 128:
            return None
        layers = [dict(qkv=L.w.qkv, o=L.w.o, gate_up=L.w.gate_up, down=L.w.down, ln1=L.w.ln1, ln2=L.w.ln2,
                       q_norm=L.w.q_norm, k_norm=L.w.k_norm, k_cache=self.k_cache[i], v_cache=self.v_cache[i])
                  for i, L in enumerate(self.layers)]
        table = ops.DecodeLayerTable(layers, c.n_heads, c.n_kv_heads, self.device)
        return table if table.workspace_bytes() > 0 else None

    def check_errors(self) -> None:
        """Raise if a wait inside a one-launch path timed out (synchronises).

        The error word is cleared before raising: a launch that finds it set gives
        up every wait early, so it would otherwise spoil every later step."""
        c = self.cfg
        if self.step_table is not None:
            ws = self.micro[0].buf.workspace
            if ops.decode_step_errors(self.step_table, self.device, workspace=ws):
                ops.clear_decode_step_errors(self.step_table, self.device, workspace=ws)
                raise RuntimeError("t2i_decode_step: a wait inside the launch timed out (error word set, now "
                                   "cleared)")
        elif self.layers and self.layers[0].fused:
            m = self.micro[0]
            if ops.qkv_attention_errors(m.b1 - m.b0, c.n_heads, c.n_kv_heads, self.device, workspace=m.buf.workspace):
                ops.clear_qkv_attention_errors(m.b1 - m.b0, c.n_heads, c.n_kv_heads, self.device,
                                               workspace=m.buf.workspace)
                raise RuntimeError("t2i_qkv_attention: a wait inside the launch timed out (error word set, now "
                                   "cleared)")

    @property
    def n_streams(self) -> int:
        return len(self.micro)

    # ---- the pieces of one step ----
    def _micro_layers(self, m: _Micro):
        """Embedding gather + every layer for the rows of one micro-batch (the gather
        also clears the rows' argmax keys for the step's lm_head)."""
        c, b = self.cfg, m.buf
        ops.rmsnorm(self.embed, self.layers[0].w.ln1, c.eps, out=b.xn, tokens=self.tokens[m.b0:m.b1], x_out=b.x,
                    argmax_keys=self.keys[m.b0:m.b1])
        pos = self.positions[m.b0:m.b1]
        if self.step_table is not None:
            ops.decode_step(self.step_table, b.xn, b.x, pos, c.eps, self.rope, rope_style=self.layers[0].rope_style,
                            workspace=b.workspace)
            return
        for i, layer in enumerate(self.layers):
            layer(b, pos, self.k_cache[i, m.b0:m.b1], self.v_cache[i, m.b0:m.b1], normed=(i == 0))

    def _micro_prompt_advance(self, m: _Micro):
        ops.prompt_advance(self.prompt[m.b0:m.b1], self.tokens[m.b0:m.b1], self.positions[m.b0:m.b1])

    def _head(self, want_logits: bool = False):
        """Final RMSNorm of the whole batch and the tied lm_head with the fused argmax,
        in one launch (the keys were cleared by the step's embedding gather); two
        launches when the hidden size is not a power of two."""
        c = self.cfg
        logits = self._logits_out(want_logits)
        if c.hidden & (c.hidden - 1) == 0:
            ops.rmsnorm_lm_head_argmax(self.x, self.norm, c.eps, self.lm_head, self.keys, logits=logits)
            return
        ops.rmsnorm(self.x, self.norm, c.eps, out=self.xn, argmax_keys=self.keys)
        ops.lm_head_argmax(self.xn, self.lm_head, self.keys, logits=logits)

    def _logits_out(self, want_logits: bool):
        """The fp32 ``[batch, vocab]`` logits buffer when logits are wanted, else None."""
        if not want_logits:
            return None
        if self.logits is None:
            self.logits = torch.empty(self.batch, self.cfg.vocab, dtype=torch.float32, device=self.device)
        return self.logits

    def _fork(self, fn):
        """Run ``fn(m)`` for every micro-batch on its stream, joined back to the current stream."""
        if self.n_streams == 1:
            fn(self.micro[0])
            return
        main = torch.cuda.current_stream(self.device)
        for m in self.micro:
            m.stream.wait_stream(main)
            with torch.cuda.stream(m.stream):
                fn(m)
        for m in self.micro:
            main.wait_stream(m.stream)

    # ---- one step, eager ----
    def forward_step(self, with_head: bool = True, want_logits: bool = False):
        """Embed ``self.tokens`` at ``self.positions``, run every layer, and (optionally)
        the final norm + lm_head argmax into ``self.keys``."""
        self._fork(self._micro_layers)
        if with_head:
            self._head(want_logits)

    def decode_step(self, tokens, positions, want_logits: bool = False):
        """One greedy decode step from host token ids/positions; returns ``(next_tokens, logits|None)``
        (the ``decode_step`` contract of ``qwen_npu.py:166-236``)."""
        tokens = torch.as_tensor(tokens, dtype=torch.int32)
        positions = torch.as_tensor(positions, dtype=torch.int32)
        if tokens.numel() != self.batch or positions.numel() != self.batch:
            raise ValueError("token batch size does not match the model batch size")
        if int(positions.max()) >= self.ctx_cap or int(positions.min()) < 0:
            raise ValueError(f"decode position exceeds the cache capacity {self.ctx_cap}")
        if int(tokens.min()) < 0 or int(tokens.max()) >= self.cfg.vocab:
            raise ValueError("token id out of range")
        self.tokens.copy_(tokens.to(self.device))
        self.positions.copy_(positions.to(self.device))
        self.forward_step(with_head=True, want_logits=want_logits)
        nxt = ops.keys_to_tokens(self.keys)
        self.check_errors()
        return nxt.cpu(), (self.logits.clone() if want_logits else None)

    # ---- prompt pass (prefill) ----
    def _prefill_buffers(self, t: int) -> dict:
        """Activations of a prompt pass over ``B * t`` rows (kept for the next prompt of that length)."""
        if getattr(self, "_pf", None) is not None and self._pf["t"] == t:
            return self._pf
        self._pf = None
        c, r = self.cfg, self.batch * t
        dev = self.device
        self._pf = {
            "t": t,
            "x": torch.empty(r, c.hidden, dtype=BF16, device=dev),
            "xn": torch.empty(r, c.hidden, dtype=BF16, device=dev),
            "qkv": torch.empty(r, c.qkv_dim, dtype=BF16, device=dev),
            "q": torch.empty(self.batch, c.n_heads, t, c.head_dim, dtype=BF16, device=dev),
            "ctx": torch.empty(r, c.n_heads * c.head_dim, dtype=BF16, device=dev),
            "h": torch.empty(r, c.intermediate, dtype=BF16, device=dev),
            "last": (torch.arange(self.batch, dtype=torch.int32) * t + (t - 1)).to(dev),
        }
        if self._prefill_sums(r):
            # row group sums that each producer hands to the next prompt GEMM
            # (group-major: [groups, rows])
            self._pf["xn_sums"] = torch.empty(c.hidden // 128, r, dtype=torch.float32, device=dev)
            self._pf["ctx_sums"] = torch.empty(c.n_heads, r, dtype=torch.float32, device=dev)
            self._pf["h_sums"] = torch.empty(c.intermediate // 64, r, dtype=torch.float32, device=dev)
        return self._pf

    def _prefill_sums(self, rows: int) -> bool:
        """Whether the prompt pass hands row group sums to its GEMMs: every GEMM of
        the pass is the prompt GEMM (rows and widths) and a head is one group."""
        c = self.cfg
        return (rows >= ops.PROMPT_GEMM_ROWS and c.head_dim == 128 and c.hidden % 128 == 0
                and (2 * c.intermediate) % 128 == 0 and (c.n_heads * c.head_dim) % 128 == 0)

    def prefill(self, prompt: torch.Tensor, want_logits: bool = False):
        """Consume ``prompt [B, T]`` from position 0 in one pass over all ``B * T`` rows
        (every layer on the whole prompt batch, causal attention over the cache), then
        greedy-pick the first new token from the last prompt row of each sequence:
        afterwards ``tokens`` holds it, ``positions`` is ``T`` and ``history[:, 0]`` it.
        Returns the fp32 logits of the last prompt rows when ``want_logits`` (else None).
        Follows the prompt pass of ``quantized_qwen3/model.py:453-478`` for a batch.
        """
        c = self.cfg
        b, t = prompt.shape
        pf = self._prefill_buffers(t)
        toks = prompt.reshape(-1).to(device=self.device, dtype=torch.int32)   # no copy for a device int32 prompt
        # Each prompt GEMM's input comes with its row group sums from the kernel that
        # wrote it (the norm, the attention, the SwiGLU epilogue), so the GEMM does
        # not form them itself.
        xs_n, xs_ctx, xs_h = pf.get("xn_sums"), pf.get("ctx_sums"), pf.get("h_sums")
        ops.rmsnorm(self.embed, self.layers[0].w.ln1, c.eps, out=pf["xn"], tokens=toks, x_out=pf["x"],
                    out_sums=xs_n)
        # Over prompt-sized batches the norms run as their own pass: the prompt GEMM
        # has no fused-norm form, and the decode kernel's would redo each row's sum
        # of squares once per column block.
        for i, layer in enumerate(self.layers):
            w = layer.w
            if i > 0:
                ops.rmsnorm(pf["x"], w.ln1, c.eps, out=pf["xn"], out_sums=xs_n)
            if b * t >= ops.PROMPT_GEMM_ROWS:
                # the projection's epilogue does the q/k norm, RoPE and cache write
                ops.prefill_qkv_rope_kv(pf["xn"], w.qkv, b, 0, c.n_heads, c.n_kv_heads, w.q_norm, w.k_norm, c.eps,
                                        self.rope, self.k_cache[i], self.v_cache[i], rope_style=layer.rope_style,
                                        q_out=pf["q"], x_sums=xs_n)
            else:
                ops.linear(pf["xn"], w.qkv, out=pf["qkv"])
                ops.prefill_qk_rope_kv(pf["qkv"], b, 0, c.n_heads, c.n_kv_heads, w.q_norm, w.k_norm, c.eps,
                                       self.rope, self.k_cache[i], self.v_cache[i], rope_style=layer.rope_style,
                                       q_out=pf["q"])
            ops.prefill_attention(pf["q"], 0, c.n_kv_heads, self.k_cache[i], self.v_cache[i], out=pf["ctx"],
                                  out_sums=xs_ctx)
            ops.linear(pf["ctx"], w.o, residual=pf["x"], out=pf["x"], x_sums=xs_ctx)
            ops.rmsnorm(pf["x"], w.ln2, c.eps, out=pf["xn"], out_sums=xs_n)
            ops.gate_up(pf["xn"], w.gate_up, swiglu=True, out=pf["h"], x_sums=xs_n, out_sums=xs_h)
            ops.linear(pf["h"], w.down, residual=pf["x"], out=pf["x"], x_sums=xs_h, sum_parts=2)
        # final norm of each sequence's last prompt row, then the tied lm_head + argmax
        ops.rmsnorm(pf["x"], self.norm, c.eps, out=self.xn, tokens=pf["last"], x_out=self.x, argmax_keys=self.keys)
        logits = self._logits_out(want_logits)
        ops.lm_head_argmax(self.xn, self.lm_head, self.keys, logits=logits)
        self.positions.fill_(t - 1)
        self.step.zero_()                  # a prompt pass starts the token record
        ops.greedy_advance(self.keys, self.tokens, self.positions, self.history, self.step)
        return logits.clone() if want_logits else None

    # ---- graph-captured greedy generation ----
    def _capture_graph(self, stream, fn):
        stream.wait_stream(torch.cuda.current_stream(self.device))
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            with torch.cuda.graph(g, stream=stream):
                fn()
        torch.cuda.current_stream(self.device).wait_stream(stream)
        return g

    # decode steps captured in one graph ("steps", one stream): the boundary between
    # two graph replays costs ~6 us, paid once per this many tokens
    STEPS_PER_GRAPH = 8

    def _capture(self):
        """One graph per micro-batch and kind ("prompt": layers + prompt bookkeeping;
        "layers": layers only) and one head graph (norm, lm_head, greedy bookkeeping),
        each captured on, and replayed on, its own stream.  With one stream a decode
        step is one graph ("step": layers, head and bookkeeping): no boundary between
        two graphs in the step (0.789 -> 0.783 ms a step at batch 16); and
        ``STEPS_PER_GRAPH`` steps are one more ("steps"), which ``generate`` replays
        while that many steps remain."""
        if self._captured:
            return

        def head():
            self._head()
            ops.greedy_advance(self.keys, self.tokens, self.positions, self.history, self.step)

        for m in self.micro:
            stream = m.stream if m.stream is not None else torch.cuda.Stream(self.device)
            m.graphs["prompt"] = self._capture_graph(stream, lambda m=m: (self._micro_layers(m),
                                                                          self._micro_prompt_advance(m)))
            if self.n_streams == 1:
                m.graphs["step"] = self._capture_graph(stream, lambda m=m: (self._micro_layers(m), head()))

                def steps(m=m):
                    for _ in range(self.STEPS_PER_GRAPH):
                        self._micro_layers(m)
                        head()

                m.graphs["steps"] = self._capture_graph(stream, steps)
            else:
                m.graphs["layers"] = self._capture_graph(stream, lambda m=m: self._micro_layers(m))
        if self.n_streams > 1:
            self._head_stream = torch.cuda.Stream(self.device)
            self._head_graph = self._capture_graph(self._head_stream, head)
        self._captured = True

    def _replay(self, kind: str):
        """Replay one step: every micro-batch's graph on its stream; for a decode step
        the streams then join on the current stream for the head graph (one stream:
        the step graph, which holds the head)."""
        main = torch.cuda.current_stream(self.device)
        if self.n_streams == 1:
            self.micro[0].graphs["step" if kind == "layers" else kind].replay()
            return
        for m in self.micro:
            m.stream.wait_stream(main)
            with torch.cuda.stream(m.stream):
                m.graphs[kind].replay()
        for m in self.micro:
            main.wait_stream(m.stream)
        if kind == "layers":
            self._head_graph.replay()

    def reset(self):
        self.k_cache.zero_()
        self.v_cache.zero_()

    def generate(self, prompt: torch.Tensor, new_tokens: int, use_graph: bool = True, timings: dict | None = None,
                 prompt_mode: str = "prefill"):
        """Greedy decode as ``qwen_npu.py:309-325``: consume the prompt, then emit
        ``new_tokens`` tokens per sequence (the first from the last prompt position).

        ``prompt_mode="prefill"``: the prompt goes through one prefill pass
        (``prefill``).  ``"decode"``: it is consumed one position at a time
        through the decode step (teacher forcing), as the NPU runner does.
        Returns int64 ``[B, new_tokens]`` on the host.
        """
        if prompt_mode not in ("prefill", "decode"):
            raise ValueError("prompt_mode must be 'prefill' or 'decode'")
        prompt = torch.as_tensor(prompt)
        b, plen = prompt.shape
        if b != self.batch:
            raise ValueError("prompt batch does not match the model batch size")
        if plen + new_tokens - 1 > self.ctx_cap:
            raise ValueError(f"prompt {plen} + {new_tokens} tokens exceed the cache capacity {self.ctx_cap}")
        if int(prompt.min()) < 0 or int(prompt.max()) >= self.cfg.vocab:
            raise ValueError("prompt token id out of range")
        # The KV cache is not cleared: attention reads only slots 0 .. position of a
        # sequence, and the prompt pass (or the decode step, for the current slot)
        # writes every one of them before it is read.
        # One prompt buffer per prompt shape: the captured prompt-bookkeeping graph
        # reads it by address (and its length), so a new shape needs a new capture
        # and a new prompt of the same shape only new contents.
        if self.prompt is None or tuple(self.prompt.shape) != (b, plen):
            self.prompt = torch.empty(b, plen, dtype=torch.int32, device=self.device)
            self._captured = False
        self.prompt.copy_(prompt.to(torch.int32))
        if self.history is None or self.history.shape[1] < new_tokens:
            self.history = torch.zeros(b, new_tokens, dtype=torch.int32, device=self.device)
            self._captured = False      # the head graph holds the history pointer
        self.tokens.copy_(self.prompt[:, 0])
        self.positions.zero_()
        self.step.zero_()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        if use_graph and not self._captured:
            # one eager step first: it allocates the attention workspaces outside the capture
            self.forward_step(with_head=True)
            torch.cuda.synchronize(self.device)
            self._capture()
            # restore the state the prompt pass starts from
            self.tokens.copy_(self.prompt[:, 0])
            self.positions.zero_()
            self.step.zero_()
            torch.cuda.synchronize(self.device)
        ev[0].record()
        if prompt_mode == "prefill":
            self.prefill(self.prompt)      # the device copy: no host transfer inside the pass
        elif use_graph:
            for _ in range(plen - 1):
                self._replay("prompt")
            self._replay("layers")          # last prompt position -> first new token
        else:
            for _ in range(plen - 1):
                self._fork(lambda m: (self._micro_layers(m), self._micro_prompt_advance(m)))
            self.forward_step(with_head=True)
            ops.greedy_advance(self.keys, self.tokens, self.positions, self.history, self.step)
        ev[1].record()
        remaining = new_tokens - 1
        if use_graph and self.n_streams == 1:
            # whole groups of steps as one graph each (the step state lives on the GPU)
            while remaining >= self.STEPS_PER_GRAPH:
                self.micro[0].graphs["steps"].replay()
                remaining -= self.STEPS_PER_GRAPH
        for _ in range(remaining):
            if use_graph:
                self._replay("layers")
            else:
                self.forward_step(with_head=True)
                ops.greedy_advance(self.keys, self.tokens, self.positions, self.history, self.step)
        ev[2].record()
        torch.cuda.synchronize(self.device)
        self.check_errors()
        if timings is not None:
            timings["prompt_ms"] = ev[0].elapsed_time(ev[1])
            timings["decode_ms"] = ev[1].elapsed_time(ev[2])
        return self.history[:, :new_tokens].to(torch.int64).cpu()
