"""torch-CPU restatement of the W4A16 Qwen3 decoder. TEST INFRASTRUCTURE ONLY.

Restates ``src/models/quantized_qwen3/model.py`` (the reference's own PyTorch
runtime) with three changes that the GPU path needs and that do not alter the
arithmetic of a single sequence:

* batch > 1, with a per-sequence position (``model.py:461-462`` allows batch 1
  only; the NPU driver ``qwen_npu.py:166-236`` decodes a batch);
* a contiguous KV cache ``[B, n_kv_heads, ctx_cap, head_dim]`` per layer instead
  of ``torch.cat`` growth (``model.py:256-264``);
* the RoPE pairing is selectable: ``"halves"`` rotates ``(i, i + d/2)`` like the
  NPU kernel ``src/torch2iron/operators/rms_norm_rope/kernel.cc:39-67``;
  ``"interleaved"`` rotates ``(2i, 2i+1)`` like ``model.py:184-196``.

Two arithmetic modes:

``mode="fp32"``  every activation in fp32 (``model.py`` with
                 ``compute_dtype=float32``, its default).  The numeric truth.
``mode="bf16"``  the rounding points of ``model.py`` with
                 ``compute_dtype=bfloat16``: every linear output, norm step,
                 RoPE product/sum, SiLU, gate*up product and residual add is
                 rounded to bf16.  Two documented departures: the softmax
                 weights stay fp32 (``model.py:277`` rounds them to bf16 before
                 the context matmul) and the logits stay fp32 for the argmax
                 (``model.py:477`` would round them to bf16, where ties between
                 the top two logits are common).

Weights are AutoGPTQ tensors (numpy) under HF-style names; they are
dequantised once to exact fp32 dense matrices (``oracle.w4a16.dequantize``),
as ``model.py:122-131`` caches its unpacked weight.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

from oracle import w4a16


@dataclass(frozen=True)
class Qwen3Config:
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
    def q_per_kv(self) -> int:
        return self.n_heads // self.n_kv_heads


LINEARS = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


def _bf(t: torch.Tensor) -> torch.Tensor:
    """Round an fp32 tensor to bf16 and back (round to nearest even)."""
    return t.to(torch.bfloat16).to(torch.float32)


class _Round:
    def __init__(self, mode: str):
        if mode not in ("fp32", "bf16"):
            raise ValueError("mode must be 'fp32' or 'bf16'")
        self.mode = mode

    def __call__(self, t: torch.Tensor) -> torch.Tensor:
        return _bf(t) if self.mode == "bf16" else t


def rope_angles(head_dim: int, context_length: int, theta: float) -> torch.Tensor:
    """``[ctx, head_dim]`` table with ``cos`` at even and ``sin`` at odd columns.

    Follows ``model.py:351-358`` (and ``qwen_inference_harness.py:86-97``):
    ``inv_freq = 1 / theta ** (arange(0, d, 2) / d)`` in fp32,
    ``freqs = outer(pos, inv_freq)``.
    """
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2).float() / head_dim))
    position = torch.arange(context_length).float()
    freqs = torch.outer(position, inv_freq)
    angles = torch.empty(context_length, head_dim)
    angles[:, ::2] = torch.cos(freqs)
    angles[:, 1::2] = torch.sin(freqs)
    return angles


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float, rnd: _Round) -> torch.Tensor:
    """``x * rsqrt(mean(x^2) + eps) * w`` over the last axis.

    Follows ``model.py:172-181``: the variance in fp32, the inverse root cast
    to the compute dtype, then two products in the compute dtype.
    """
    variance = x.pow(2).mean(dim=-1, keepdim=True)
    inv = rnd(torch.rsqrt(variance + eps))
    return rnd(rnd(x * inv) * weight)


def apply_rope(x: torch.Tensor, cos_sin: torch.Tensor, style: str, rnd: _Round) -> torch.Tensor:
    """Rotate ``x [..., d]`` by the per-row ``cos_sin [..., d]`` table rows.

    ``cos_sin`` broadcasts against ``x`` (its even columns are cos, odd are sin
    of frequency ``i``).  ``"interleaved"`` follows ``model.py:184-196``:
    pairs ``(2i, 2i+1)``.  ``"halves"`` follows
    ``rms_norm_rope/kernel.cc:39-67``: pairs ``(i, i + d/2)``, frequency ``i``.
    In bf16 mode the table is rounded to bf16 (``model.py:423``) and each
    product and the sum are rounded (``model.py:196``).
    """
    cos = rnd(cos_sin[..., ::2])
    sin = rnd(cos_sin[..., 1::2])
    if style == "interleaved":
        cos_f = cos.repeat_interleave(2, dim=-1)
        sin_f = sin.repeat_interleave(2, dim=-1)
        even, odd = x[..., ::2], x[..., 1::2]
        rot = torch.stack((-odd, even), dim=-1).flatten(-2)
    elif style == "halves":
        cos_f = torch.cat((cos, cos), dim=-1)
        sin_f = torch.cat((sin, sin), dim=-1)
        half = x.shape[-1] // 2
        rot = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    else:
        raise ValueError("rope style must be 'halves' or 'interleaved'")
    return rnd(rnd(x * cos_f) + rnd(rot * sin_f))


def silu(x: torch.Tensor) -> torch.Tensor:
    """``x * sigmoid(x)`` (``torch.nn.functional.silu``, ``model.py:216``)."""
    return torch.nn.functional.silu(x)


def decode_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                     lengths: torch.Tensor, n_kv_heads: int) -> torch.Tensor:
    """GQA attention of one query token per sequence over its cached keys.

    ``q [B, H, d]``, caches ``[B, Hkv, ctx_cap, d]``, ``lengths [B]`` = number
    of valid cache slots (current token included).  Query head ``h`` reads kv
    head ``h // (H / Hkv)`` (``repeat_interleave``, ``model.py:266-267``);
    scores in fp32 scaled by ``d ** -0.5`` (``model.py:268-269``), softmax in
    fp32 (``model.py:277``), fp32 context.  Slots at or beyond the length are
    masked, which for one query equals the causal mask of ``model.py:271-275``.
    """
    b, h, d = q.shape
    group = h // n_kv_heads
    out = torch.empty(b, h, d, dtype=torch.float32)
    scale = d ** -0.5
    for i in range(b):
        n = int(lengths[i])
        keys = k_cache[i, :, :n, :].float().repeat_interleave(group, dim=0)   # [H, n, d]
        vals = v_cache[i, :, :n, :].float().repeat_interleave(group, dim=0)
        scores = torch.einsum("hd,hnd->hn", q[i].float(), keys) * scale
        weights = torch.softmax(scores, dim=-1)
        out[i] = torch.einsum("hn,hnd->hd", weights, vals)
    return out


def prefill_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, n_kv_heads: int) -> torch.Tensor:
    """Causal attention of ``T`` new tokens over themselves (empty cache).

    ``q [B, H, T, d]``, ``k, v [B, Hkv, T, d]``; the causal mask of
    ``model.py:271-275`` with ``past_len = 0``.
    """
    h = q.shape[1]
    group = h // n_kv_heads
    kk = k.float().repeat_interleave(group, dim=1)
    vv = v.float().repeat_interleave(group, dim=1)
    scores = torch.matmul(q.float(), kk.transpose(-2, -1)) * (q.shape[-1] ** -0.5)
    t = q.shape[2]
    mask = torch.ones(t, t, dtype=torch.bool).tril()
    scores = scores.masked_fill(~mask, torch.finfo(torch.float32).min)
    return torch.matmul(torch.softmax(scores, dim=-1), vv)


class DenseLayer:
    """One decoder layer with exact fp32 dense weights."""

    def __init__(self, tensors: dict, prefix: str, cfg: Qwen3Config):
        self.cfg = cfg
        self.w = {}
        for name in LINEARS:
            sub = "self_attn" if name in ("q_proj", "k_proj", "v_proj", "o_proj") else "mlp"
            p = f"{prefix}.{sub}.{name}"
            self.w[name] = torch.from_numpy(w4a16.dequantize(
                tensors[f"{p}.qweight"], tensors[f"{p}.qzeros"], tensors[f"{p}.scales"], cfg.group_size))
        f = lambda n: torch.as_tensor(np.asarray(tensors[n], dtype=np.float32))
        self.ln1 = f(f"{prefix}.input_layernorm.weight")
        self.ln2 = f(f"{prefix}.post_attention_layernorm.weight")
        self.q_norm = f(f"{prefix}.self_attn.q_norm.weight")
        self.k_norm = f(f"{prefix}.self_attn.k_norm.weight")

    def lin(self, name: str, x: torch.Tensor, rnd: _Round) -> torch.Tensor:
        """fp32 matmul with the exact weight, output in the compute dtype (``model.py:133-146``)."""
        return rnd(x @ self.w[name].T)

    def qkv(self, x: torch.Tensor, cs: torch.Tensor, rnd: _Round):
        """RMSNorm, q/k/v projections, per-head q/k RMSNorm and RoPE (``model.py:246-253, 323``).

        ``x [R, hidden]``, ``cs [R, head_dim]`` the RoPE table row of each row.
        Returns ``q [R, H, d]``, ``k [R, Hkv, d]``, ``v [R, Hkv, d]``.
        """
        c = self.cfg
        xn = rmsnorm(x, self.ln1, c.eps, rnd)
        q = self.lin("q_proj", xn, rnd).view(-1, c.n_heads, c.head_dim)
        k = self.lin("k_proj", xn, rnd).view(-1, c.n_kv_heads, c.head_dim)
        v = self.lin("v_proj", xn, rnd).view(-1, c.n_kv_heads, c.head_dim)
        q = apply_rope(rmsnorm(q, self.q_norm, c.eps, rnd), cs[:, None, :], c.rope_style, rnd)
        k = apply_rope(rmsnorm(k, self.k_norm, c.eps, rnd), cs[:, None, :], c.rope_style, rnd)
        return q, k, v

    def post_attention(self, x: torch.Tensor, ctx: torch.Tensor, rnd: _Round) -> torch.Tensor:
        """o_proj + residual, RMSNorm, SwiGLU MLP + residual (``model.py:215-216, 322-327``)."""
        c = self.cfg
        x = rnd(x + self.lin("o_proj", rnd(ctx), rnd))
        xn = rmsnorm(x, self.ln2, c.eps, rnd)
        g = self.lin("gate_proj", xn, rnd)
        u = self.lin("up_proj", xn, rnd)
        h = rnd(rnd(silu(g)) * u)
        return rnd(x + self.lin("down_proj", h, rnd))

    def decode(self, x: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
               positions: torch.Tensor, angles: torch.Tensor, rnd: _Round) -> torch.Tensor:
        """One decode token per sequence: ``x [B, hidden]`` at ``positions [B]``.

        Writes k/v (in the compute dtype) into the caches at ``positions`` and
        attends over slots ``0..position``, as the NPU runlist does
        (``batch_decode_fused.py:426-530``).
        """
        c = self.cfg
        q, k, v = self.qkv(x, angles[positions], rnd)
        for i in range(x.shape[0]):
            p = int(positions[i])
            k_cache[i, :, p, :] = k[i]
            v_cache[i, :, p, :] = v[i]
        ctx = decode_attention(q, k_cache, v_cache, positions + 1, c.n_kv_heads)
        return self.post_attention(x, ctx.reshape(x.shape[0], -1), rnd)

    def prefill(self, x: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                angles: torch.Tensor, rnd: _Round) -> torch.Tensor:
        """``T`` prompt tokens per sequence from position 0: ``x [B, T, hidden]``."""
        c = self.cfg
        b, t, _ = x.shape
        cs = angles[:t].repeat(b, 1)
        q, k, v = self.qkv(x.reshape(b * t, -1), cs, rnd)
        q = q.view(b, t, c.n_heads, c.head_dim).transpose(1, 2)
        k = k.view(b, t, c.n_kv_heads, c.head_dim).transpose(1, 2)
        v = v.view(b, t, c.n_kv_heads, c.head_dim).transpose(1, 2)
        k_cache[:, :, :t, :] = k
        v_cache[:, :, :t, :] = v
        ctx = prefill_attention(q, k, v, c.n_kv_heads).transpose(1, 2).reshape(b * t, -1)
        return self.post_attention(x.reshape(b * t, -1), ctx, rnd).view(b, t, -1)


class DenseQwen3:
    """Batched greedy Qwen3 decoder (``model.py:361-498`` semantics, batch > 1).

    ``tensors``: ``model.embed_tokens.weight [V, hidden]`` (bf16 values, the
    tied lm_head as in ``model.py:415-420``), ``model.norm.weight`` and the
    per-layer AutoGPTQ tensors and norm weights.
    """

    def __init__(self, tensors: dict, cfg: Qwen3Config, mode: str = "fp32", ctx_cap: int = 2048):
        self.cfg = cfg
        self.rnd = _Round(mode)
        self.embed = torch.as_tensor(np.asarray(tensors["model.embed_tokens.weight"], dtype=np.float32))
        # tied lm_head unless the tensors hold their own (model.py:410-420)
        self.lm_head = (torch.as_tensor(np.asarray(tensors["lm_head.weight"], dtype=np.float32))
                        if "lm_head.weight" in tensors else self.embed)
        self.norm = torch.as_tensor(np.asarray(tensors["model.norm.weight"], dtype=np.float32))
        self.layers = [DenseLayer(tensors, f"model.layers.{i}", cfg) for i in range(cfg.n_layers)]
        self.angles = rope_angles(cfg.head_dim, ctx_cap, cfg.rope_theta)
        self.ctx_cap = ctx_cap
        self.k_cache = self.v_cache = None

    def reset(self, batch: int) -> None:
        c = self.cfg
        shape = (c.n_layers, batch, c.n_kv_heads, self.ctx_cap, c.head_dim)
        self.k_cache = torch.zeros(shape)
        self.v_cache = torch.zeros(shape)

    def logits(self, h: torch.Tensor) -> torch.Tensor:
        """Final RMSNorm then the tied bf16 lm_head, logits in fp32."""
        hn = rmsnorm(h, self.norm, self.cfg.eps, self.rnd)
        return hn @ self.lm_head.T

    @torch.no_grad()
    def prefill(self, tokens: torch.Tensor) -> torch.Tensor:
        """Consume ``tokens [B, T]`` from position 0; returns last-token logits ``[B, V]``."""
        b, t = tokens.shape
        if t > self.ctx_cap:
            raise ValueError("prompt exceeds the cache capacity")
        self.reset(b)
        x = self.embed[tokens]
        for li, layer in enumerate(self.layers):
            x = layer.prefill(x, self.k_cache[li], self.v_cache[li], self.angles, self.rnd)
        return self.logits(x[:, -1, :])

    @torch.no_grad()
    def decode_step(self, tokens: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        """One token per sequence at ``positions``; returns logits ``[B, V]``."""
        if int(positions.max()) >= self.ctx_cap:
            raise ValueError("decode position exceeds the cache capacity")
        x = self.embed[tokens]
        for li, layer in enumerate(self.layers):
            x = layer.decode(x, self.k_cache[li], self.v_cache[li], positions, self.angles, self.rnd)
        return self.logits(x)

    @torch.no_grad()
    def forced_logits(self, prompt: torch.Tensor, forced: torch.Tensor) -> torch.Tensor:
        """Logits after the prompt and after each of the ``forced [B, S]`` tokens
        (teacher forcing): ``[B, S + 1, V]``."""
        b, t = prompt.shape
        out = [self.prefill(prompt)]
        positions = torch.full((b,), t, dtype=torch.long)
        for j in range(forced.shape[1]):
            out.append(self.decode_step(forced[:, j], positions))
            positions = positions + 1
        return torch.stack(out, dim=1)

    @torch.no_grad()
    def generate(self, prompt: torch.Tensor, new_tokens: int, return_margins: bool = False):
        """Greedy decode as ``qwen_npu.py:309-325``: the first new token comes
        from the prompt pass, then ``new_tokens - 1`` decode steps."""
        b, t = prompt.shape
        logits = self.prefill(prompt)
        out, margins = [], []
        positions = torch.full((b,), t, dtype=torch.long)
        for step in range(new_tokens):
            top2 = torch.topk(logits, 2, dim=-1).values
            margins.append((top2[:, 0] - top2[:, 1]).clone())
            nxt = torch.argmax(logits, dim=-1)
            out.append(nxt)
            if step + 1 == new_tokens:
                break
            logits = self.decode_step(nxt, positions)
            positions = positions + 1
        toks = torch.stack(out, dim=1)
        if return_margins:
            return toks, torch.stack(margins, dim=1)
        return toks
