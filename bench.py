#!/usr/bin/env python3
"""Benchmark of the MI355X W4A16 hot path (one GPU).

Workload of the headline (one "step"): the W4A16 group-128 linear over every
Qwen3-0.6B linear shape -- fused qkv K=1024 N=4096, o_proj K=2048 N=1024, fused
gate_up K=1024 N=6144, down K=3072 N=1024 -- at M in {1, 8, 16, 32, 64}
(batched decode).  Each (M, shape) group is one HIP graph that launches the
linear once per weight copy of a pool of more than twice the 256 MB MALL, and
the groups run in the order M, then shape, so a weight copy is used again only
after the whole pool has streamed past: the weights come from HBM (HBM-cold).
Inputs are resident in HBM before the timed region.

``value`` = algorithmic bytes of all launches / wall time of the timed steps
(TB/s).  Algorithmic bytes per launch: K*N/2 (int4) + (K/128)*N*2 (fp16
scales) + (K/128)*(N/8)*4 (int32 zeros) + M*K*2 + M*N*2 (bf16 in/out).

Extra fields: the per-(M, shape) breakdown, the MALL-warm rate (one weight copy
reused), the single GEMV of Qwen3-0.6B's up_proj shape (M=1, K=1024, N=3072;
HBM-cold and MALL-warm), the Qwen3-1.7B sweep, one fused decode layer (batch 8,
context 1024), batch-16 greedy decode of the full random-init Qwen3-0.6B, the
roofline entry for the linear kernel, and the CPU baselines (the oracle on the
host cores, for each configuration).
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = "W4A16 linear achieved HBM TB/s (% of peak); batch-decode tokens/s"
PEAK_GBPS = 8000.0
QWEN3_06B = [("qkv", 1024, 4096), ("o_proj", 2048, 1024), ("gate_up", 1024, 6144), ("down", 3072, 1024)]
QWEN3_17B = [("qkv", 2048, 4096), ("o_proj", 2048, 2048), ("gate_up", 2048, 12288), ("down", 6144, 2048)]
GEMV_06B = [("up_proj", 1024, 3072)]
MALL_BYTES = 256 << 20
COPY_BYTES = 256 << 20
TRAFFIC_FILE = ROOT / "profiles" / "w4a16_linear_qwen3_0.6b_sweep_traffic.json"


def _load_json(path: Path):
    try:
        return json.loads(path.read_text())
    except (OSError, ValueError):
        return None


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--pool-mb", type=int, default=544, help="weight pool per sweep (> 2 x the 256 MB MALL)")
    ap.add_argument("--cpu-seconds", type=float, default=5.0, help="CPU budget per baseline leg")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--skip-extra", action="store_true", help="only the headline sweep")
    ap.add_argument("--skip-decode", action="store_true", help="skip the decode layer / greedy decode runs")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the decode layer and greedy decode (for a kernel trace of the decode step; no headline)")
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--new-tokens", type=int, default=128)
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--streams", default="1,2", help="micro-batch stream counts to measure for batch decode")
    ap.add_argument("--attention-only", action="store_true",
                    help="only the decode attention at the batch-decode shape, HBM-cold (for its kernel trace and "
                         "counters; no headline)")
    ap.add_argument("--prompt-gemm-only", action="store_true",
                    help="only the prompt GEMM at the prompt pass's shapes (16 x 512 rows; for its kernel trace and "
                         "MFMA counters; no headline)")
    ap.add_argument("--eager", action="store_true", help="sweep launches without graphs (for counter collection)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a 256 MiB device copy (the reference kernel for HBM byte counters)")
    return ap.parse_args()


class Sweep:
    """Graph-captured launches of one (M, shape) grid over a weight pool.

    Group (M, shape) launches the linear once per copy of that shape's weights;
    the groups run M-major, so between two uses of one copy the whole pool is
    read (the reuse distance is the pool size)."""

    def __init__(self, shapes, ms, pool_bytes, dev, seed, reps=None, eager=False, tiled=True):
        import torch
        from torch2iron_amd import ops
        from torch2iron_amd.formats import algorithmic_bytes, random_weight_on_device

        self.torch = torch
        gen = torch.Generator(device=dev).manual_seed(seed)
        per_copy = sum(k * n // 2 + (k // 128) * n * 2 + (k // 128) * (n // 8) * 4 for _, k, n in shapes)
        self.per_copy = per_copy
        self.copies = max(1, -(-pool_bytes // per_copy)) if pool_bytes else 1
        # tiled: each copy also gets its decode-linear tiles (ops.tile_weight), which the
        # linear then reads in place of the AutoGPTQ words, as the decode model's do
        self.weights = {name: [random_weight_on_device(k, n, gen, dev) for _ in range(self.copies)]
                        for name, k, n in shapes}
        if tiled:
            for copies in self.weights.values():
                for w in copies:
                    ops.tile_weight(w)
        # launches per graph: one per weight copy (HBM-cold), or ``reps`` of the one copy (MALL-warm)
        self.reps = reps or self.copies
        self.groups = []   # (label, M, K, N, graph, bytes, launches)
        for m in ms:
            for name, k, n in shapes:
                x = torch.randn(m, k, generator=gen, device=dev).to(torch.bfloat16)
                y = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
                ws = [self.weights[name][i % self.copies] for i in range(self.reps)]
                ops.linear(x, ws[0], out=y)
                torch.cuda.synchronize()

                def launch_all(x=x, y=y, ws=ws):
                    for w in ws:
                        ops.linear(x, w, out=y)

                if eager:
                    replay = launch_all
                else:
                    g = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(g):
                        launch_all()
                    replay = g.replay
                self.groups.append(dict(label=f"{name}/M{m}", M=m, K=k, N=n, replay=replay, x=x, y=y,
                                        bytes=algorithmic_bytes(m, k, n) * self.reps, launches=self.reps))
        self.bytes_per_step = sum(gr["bytes"] for gr in self.groups)
        self.launches_per_step = sum(gr["launches"] for gr in self.groups)

    @property
    def pool_mb(self) -> float:
        return self.copies * self.per_copy / 1e6

    def run(self, steps, warmup):
        return run_groups(self.groups, steps, warmup)

    def breakdown(self, per_group):
        return {gr["label"]: {"TBps": round(gr["bytes"] / (t * 1e-3) / 1e12, 4),
                              "us_per_launch": round(t * 1e3 / gr["launches"], 3)}
                for gr, t in zip(self.groups, per_group)}


def run_groups(groups, steps: int, warmup: int):
    """Replay every group's graph in order, ``steps`` times after ``warmup``; returns
    the total ms and the average ms of each group (events between the groups)."""
    import torch
    for _ in range(warmup):
        for gr in groups:
            gr["replay"]()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    marks = [[torch.cuda.Event(enable_timing=True) for _ in groups] for _ in range(steps)]
    start.record()
    for s in range(steps):
        for i, gr in enumerate(groups):
            gr["replay"]()
            marks[s][i].record()
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(marks[-1][-1])
    per_group = [0.0] * len(groups)
    for s in range(steps):
        prev = start if s == 0 else marks[s - 1][-1]
        for i in range(len(groups)):
            per_group[i] += prev.elapsed_time(marks[s][i])
            prev = marks[s][i]
    return total_ms, [t / steps for t in per_group]


def read_ceiling(sweep_groups, pool_bytes: int, dev, steps: int, warmup: int, lpts=(1, 2, 4, 8)):
    """The HBM read ceiling beside the sweep (``t2i_stream_read``, a kernel that only
    streams bytes).  Its twin of the sweep reads, per group, the group's algorithmic
    bytes per launch with the same number of launches, in the same M-major order,
    each launch a fresh slice of a pool larger than twice the MALL (the same reuse
    distance as the weight copies); per group the fastest loads-per-thread variant
    counts.  The bulk leg reads one 1 GiB buffer per launch."""
    import torch
    from torch2iron_amd import ops
    pool = torch.randint(0, 256, (pool_bytes,), dtype=torch.uint8, device=dev,
                         generator=torch.Generator(device=dev).manual_seed(11))
    out = torch.empty(1 << 20, dtype=torch.int32, device=dev)
    best = None
    for lpt in lpts:
        groups, off = [], 0
        for gr in sweep_groups:
            per = -(-(gr["bytes"] // gr["launches"]) // 16) * 16
            slices = []
            for _ in range(gr["launches"]):
                if off + per > pool_bytes:
                    off = 0
                slices.append(off)
                off += -(-per // 256) * 256
            ops.stream_read(pool, per, slices[0], lpt, out=out)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for o in slices:
                    ops.stream_read(pool, per, o, lpt, out=out)
            groups.append(dict(label=gr["label"], replay=g.replay, bytes=per * gr["launches"],
                               launches=gr["launches"], graph=g))
        _, per_group = run_groups(groups, steps, warmup)
        if best is None:
            best = [dict(label=g["label"], bytes=g["bytes"], launches=g["launches"], ms=t, lpt=lpt)
                    for g, t in zip(groups, per_group)]
        else:
            for b, t in zip(best, per_group):
                if t < b["ms"]:
                    b["ms"], b["lpt"] = t, lpt
        del groups
    total_bytes = sum(b["bytes"] for b in best)
    total_ms = sum(b["ms"] for b in best)
    launches = sum(b["launches"] for b in best)
    del pool
    torch.cuda.empty_cache()
    # bulk: one 1 GiB read a launch
    big = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(7)
    bulk = {}
    for lpt in lpts:
        ops.stream_read(big, loads_per_thread=lpt, out=torch.empty(1 << 20, dtype=torch.int32, device=dev))
        bout = torch.empty(1 << 20, dtype=torch.int32, device=dev)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            ops.stream_read(big, loads_per_thread=lpt, out=bout)
        for _ in range(warmup):
            g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        bulk[lpt] = (1 << 30) / (e0.elapsed_time(e1) / steps * 1e-3) / 1e12
        del g, bout
    del big
    torch.cuda.empty_cache()
    bulk_lpt = max(bulk, key=bulk.get)
    return {
        "kernel": "stream_read_kernel (t2i_stream_read: 16-byte non-temporal loads, XOR per wave)",
        "same_launches_TBps": round(total_bytes / (total_ms * 1e-3) / 1e12, 4),
        "same_launches_us_per_launch": round(total_ms * 1e3 / launches, 3),
        "bulk_1GiB_TBps": round(bulk[bulk_lpt], 4),
        "bulk_loads_per_thread": bulk_lpt,
        "bulk_by_loads_per_thread": {str(k): round(v, 4) for k, v in bulk.items()},
        "breakdown": {b["label"]: {"TBps": round(b["bytes"] / (b["ms"] * 1e-3) / 1e12, 4),
                                   "us_per_launch": round(b["ms"] * 1e3 / b["launches"], 3),
                                   "loads_per_thread": b["lpt"]} for b in best},
    }


def rate(sweep: Sweep, steps: int, warmup: int):
    total_ms, per_group = sweep.run(steps, warmup)
    ms_step = total_ms / steps
    return sweep.bytes_per_step / (ms_step * 1e-3) / 1e12, ms_step, per_group


def launch_floor(dev, launches: int, steps: int, warmup: int) -> float:
    """The same number of back-to-back graph launches of a one-element fill: what a
    dependent launch costs on this stream before any kernel does work (us)."""
    import torch
    tiny = torch.zeros(1, device=dev)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(launches):
            tiny.fill_(0.0)
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (steps * launches)


# ---------------------------------------------------------------------------
# decode: config 3 (one fused layer) and config 4 (full model, greedy)
# ---------------------------------------------------------------------------

def bench_decode(dev, steps: int, warmup: int, prompt_len: int, new_tokens: int, batch: int,
                 streams=(1, 2), teacher_forced_leg: bool = True):
    """Config 3 (one fused decode layer, batch 8, 1024 cached tokens) and config 4
    (full Qwen3-0.6B, batch 16 greedy decode) on random-init weights."""
    import numpy as np
    import torch
    from torch2iron_amd import model as gm

    cfg = gm.QWEN3_0_6B
    log("generating random-init Qwen3-0.6B weights (uniform AutoGPTQ words, N(0,1) bf16 embedding)")
    tensors = gm.random_qwen3_tensors(cfg, seed=0)
    out = {}

    # ---- config 3: one decode layer, B = 8, context 1024 (write at 1024) ----
    # 12 distinct layers (weights and caches, 530 MB: past the 256 MB MALL, as the
    # layers of a decode step are) run back to back in one graph, so that every
    # layer reads HBM and the host's replay calls stay off the timed path.
    b3, cap3, n3 = 8, 1088, 12
    rope = gm.rope_table(cfg.head_dim, cap3, cfg.rope_theta, dev)
    buf = gm.DecodeBuffers(cfg, b3, dev)
    gen = torch.Generator(device=dev).manual_seed(5)
    layers3 = []
    for li in range(n3):
        lay = gm.Qwen3DecodeLayer(gm.Qwen3LayerWeights(tensors, li, cfg, dev), cfg, rope)
        kc = torch.randn(b3, cfg.n_kv_heads, cap3, cfg.head_dim, generator=gen, device=dev).to(torch.bfloat16)
        vc = torch.randn(b3, cfg.n_kv_heads, cap3, cfg.head_dim, generator=gen, device=dev).to(torch.bfloat16)
        layers3.append((lay, kc, vc))
    # the layers chained as the model chains them: each o_proj hands the MLP's RMSNorm
    # over to gate_up, each down the next layer's to its qkv (the first layer's qkv and
    # the last layer's down unchained)
    from torch2iron_amd import ops as _ops
    chain3 = (_ops.chain_supported(b3, cfg.n_heads * cfg.head_dim, cfg.hidden, _ops.CHAIN_PRODUCER)
              and _ops.chain_supported(b3, cfg.intermediate, cfg.hidden, _ops.CHAIN_PRODUCER)
              and _ops.chain_supported(b3, cfg.hidden, cfg.qkv_dim, _ops.CHAIN_CONSUMER)
              and _ops.chain_supported(b3, cfg.hidden, 2 * cfg.intermediate, _ops.CHAIN_PAIRED_CONSUMER))
    for li, (lay, _, _) in enumerate(layers3):
        lay.chain = chain3
        lay.chain_in = chain3 and li > 0
        lay.next_ln1 = layers3[li + 1][0].w.ln1 if chain3 and li + 1 < n3 else None
    pos = torch.full((b3,), 1024, dtype=torch.int32, device=dev)
    x0 = torch.randn(b3, cfg.hidden, generator=gen, device=dev).to(torch.bfloat16)
    buf.x.copy_(x0)
    for lay, kc, vc in layers3:
        lay(buf, pos, kc, vc)                    # eager warm-up (allocates the attention workspace)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for lay, kc, vc in layers3:
            lay(buf, pos, kc, vc)
    reps = max(steps, 10)
    for _ in range(warmup):
        buf.x.copy_(x0)
        g.replay()
    torch.cuda.synchronize()
    buf.x.copy_(x0)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    layer_us = e0.elapsed_time(e1) * 1e3 / (reps * n3)
    w = layers3[0][0].w
    layer_bytes = (w.qkv.nbytes + w.o.nbytes + w.gate_up.nbytes + w.down.nbytes + 4 * 2 * cfg.hidden
                   + 2 * 2 * cfg.head_dim + b3 * cfg.n_kv_heads * 1025 * cfg.head_dim * 2 * 2
                   + b3 * cfg.n_kv_heads * cfg.head_dim * 2 * 2 + b3 * cfg.hidden * 2 * 2)
    out["decode_layer"] = {"workload": f"one fused Qwen3-0.6B decode layer, batch 8, context 1024 ({n3} distinct "
                                       "layers back to back in one graph, HBM-cold"
                                       + (", RMSNorms chained as in the model)" if chain3 else ")"),
                           "chained_norm": bool(chain3),
                           "us": round(layer_us, 2), "algorithmic_bytes": layer_bytes,
                           "TBps": round(layer_bytes / (layer_us * 1e-6) / 1e12, 4),
                           "frac_of_8TBps": round(layer_bytes / (layer_us * 1e-6) / 8e12, 4)}
    log(f"decode layer (B=8, ctx 1024): {layer_us:.1f} us, {out['decode_layer']['TBps']} TB/s")
    # each of the layer's five launches on its own: a graph of that launch for all 12
    # layers (HBM-cold as above), event-timed, outside any profiler
    from torch2iron_amd import ops

    def layer_ops(lay, kc, vc):
        # each launch in the form the layer runs it (chained norm: see above)
        c, lw = cfg, lay.w
        if lay.chain_in:
            qkv = lambda: ops.prenormed_linear(buf.xg, buf.ssp, c.eps, lw.qkv, out=buf.qkv)
        else:
            qkv = lambda: ops.rmsnorm_linear(buf.x, lw.ln1, c.eps, lw.qkv, out=buf.qkv)
        if lay.chain:
            o = lambda: ops.linear_residual_next_norm(buf.ctx, lw.o, buf.x, buf.x, lw.ln2, buf.xg, buf.ssp)
            gu = lambda: ops.prenormed_gate_up(buf.xg, buf.ssp, c.eps, lw.gate_up, swiglu=True, out=buf.hmlp)
        else:
            o = lambda: ops.linear(buf.ctx, lw.o, residual=buf.x, out=buf.x)
            gu = lambda: ops.rmsnorm_gate_up(buf.x, lw.ln2, c.eps, lw.gate_up, swiglu=True, out=buf.hmlp)
        if lay.next_ln1 is not None:
            down = lambda: ops.linear_residual_next_norm(buf.hmlp, lw.down, buf.x, buf.x, lay.next_ln1, buf.xg,
                                                         buf.ssp)
        else:
            down = lambda: ops.linear(buf.hmlp, lw.down, residual=buf.x, out=buf.x)
        return [
            ("rmsnorm_qkv", qkv),
            ("attention", lambda: ops.decode_attention(buf.qkv, pos, c.n_heads, c.n_kv_heads, lw.q_norm, lw.k_norm,
                                                       c.eps, lay.rope, kc, vc, rope_style=lay.rope_style,
                                                       out=buf.ctx, workspace=buf.workspace)),
            ("o_proj_residual", o),
            ("rmsnorm_gate_up_swiglu", gu),
            ("down_residual", down),
        ]

    calls = [layer_ops(lay, kc, vc) for lay, kc, vc in layers3]
    per_op = {}
    for j, (name, _) in enumerate(calls[0]):
        gop = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gop):
            for lc in calls:
                lc[j][1]()
        for _ in range(warmup):
            gop.replay()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps):
            gop.replay()
        e1.record()
        torch.cuda.synchronize()
        per_op[name] = round(e0.elapsed_time(e1) * 1e3 / (reps * n3), 2)
        del gop
    out["decode_layer"]["per_op_us"] = per_op
    out["decode_layer"]["per_op_sum_us"] = round(sum(per_op.values()), 2)
    log("decode layer, each launch alone (us): " + ", ".join(f"{k} {v}" for k, v in per_op.items()))
    buf.x.copy_(x0)
    del g, buf, layers3, kc, vc, calls
    torch.cuda.empty_cache()

    # ---- config 4: full model, batch 16, prompt 512, 128 new tokens ----
    cap4 = prompt_len + new_tokens
    model = gm.Qwen3Model(tensors, cfg, batch=batch, ctx_cap=cap4, device=dev)
    prompt = torch.randint(0, cfg.vocab, (batch, prompt_len), generator=torch.Generator().manual_seed(7))
    runs = {}
    toks = None
    for s in streams:
        model.set_streams(s)
        log(f"greedy decode: batch {batch}, prompt {prompt_len} (prefill pass), {new_tokens} new tokens, "
            f"{model.n_streams} micro-batch stream(s) (graph replays)")
        model.generate(prompt[:, :8], new_tokens)     # warm-up and capture
        model.generate(prompt, 2)                     # warm-up of the full-length prompt pass
        model.generate(prompt[:, :8], new_tokens)
        tm = {}
        got = model.generate(prompt, new_tokens, timings=tm)
        if toks is None:
            toks = got
        dec_s = tm["decode_ms"] * 1e-3
        e2e_s = (tm["prompt_ms"] + tm["decode_ms"]) * 1e-3
        step_ms = tm["decode_ms"] / (new_tokens - 1)
        runs[s] = {
            "streams": model.n_streams,
            "decode_tokens_per_s": round(batch * (new_tokens - 1) / dec_s, 1),
            "end_to_end_tokens_per_s": round(batch * new_tokens / e2e_s, 1),
            "ms_per_decode_step": round(step_ms, 4),
            "prompt_ms": round(tm["prompt_ms"], 2),
            "prompt_tokens_per_s": round(batch * prompt_len / (tm["prompt_ms"] * 1e-3), 1),
            "decode_ms": round(tm["decode_ms"], 2),
            "tokens_equal_to_first_run": bool(torch.equal(got, toks)),
        }
        log(f"decode ({model.n_streams} streams): {runs[s]['decode_tokens_per_s']} tok/s, {step_ms:.3f} ms/step; "
            f"prefill {tm['prompt_ms']:.2f} ms; end to end {runs[s]['end_to_end_tokens_per_s']} tok/s")
    # The prompt pass on its own, five passes back to back (no host wait between
    # them), event-timed.  prompt_ms above times one pass inside generate, started
    # from a GPU that was idle while the host prepared it (clocks still rising).
    model.set_streams(1)
    model.prefill(model.prompt)
    torch.cuda.synchronize(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(5):
        model.prefill(model.prompt)
    e1.record()
    torch.cuda.synchronize(dev)
    prefill_steady_ms = e0.elapsed_time(e1) / 5
    log(f"prefill, five passes back to back: {prefill_steady_ms:.2f} ms a pass")
    prefill_kernels = time_prefill_kernels(model, dev)
    log("prefill kernels (us per launch): " + ", ".join(
        f"{k} {v['us_per_launch']}" for k, v in prefill_kernels.items() if isinstance(v, dict))
        + f"; sum {prefill_kernels['sum_ms_per_pass']:.2f} ms per pass")
    # each kernel of the step alone, event-timed outside any profiler, at position 576
    # (the middle of the timed steps' 512..638)
    log("decode step kernels, each alone (graphs of its launches in one step, HBM-cold, events)")
    per_kernel = time_step_kernels(model, dev, max(steps, 10), prompt_len + new_tokens // 2)
    kernel_sum_ms = sum(v["us_per_step"] for v in per_kernel.values() if isinstance(v, dict)) / 1e3
    log("decode step kernels (us per launch): " + ", ".join(
        f"{k} {v['us_per_launch'] if isinstance(v, dict) else v}" for k, v in per_kernel.items())
        + f"; sum {kernel_sum_ms:.3f} ms per step")
    # the prompt consumed one position at a time through the decode step (the NPU runner's way)
    teacher_forced = None
    if teacher_forced_leg:
        model.set_streams(1)
        tm = {}
        tf = model.generate(prompt, new_tokens, timings=tm, prompt_mode="decode")
        teacher_forced = {
            "prompt_ms": round(tm["prompt_ms"], 2),
            "end_to_end_tokens_per_s": round(batch * new_tokens / ((tm["prompt_ms"] + tm["decode_ms"]) * 1e-3), 1),
            "first_token_equal_to_prefill": bool(torch.equal(tf[:, 0], toks[:, 0])),
            "tokens_equal_to_prefill_run": bool(torch.equal(tf, toks))}
        log(f"teacher-forced prompt: {tm['prompt_ms']:.1f} ms")
    # every layer of a step as one cooperative launch (t2i_decode_step): built and
    # tested, off by default because it measures slower; timed here beside the graph
    one_launch = None
    model.persistent = True
    model.set_streams(1)
    if model.step_table is not None:
        model.generate(prompt[:, :8], new_tokens)     # warm-up and capture
        tm = {}
        ol = model.generate(prompt, new_tokens, timings=tm)
        one_launch = {"ms_per_decode_step": round(tm["decode_ms"] / (new_tokens - 1), 4),
                      "decode_tokens_per_s": round(batch * (new_tokens - 1) / (tm["decode_ms"] * 1e-3), 1),
                      "sequences_equal_to_graph_path": int((ol == toks).all(dim=1).sum()), "of": batch}
        log(f"one-launch step (t2i_decode_step): {one_launch['ms_per_decode_step']:.3f} ms/step")
    model.persistent = False
    model.set_streams(1)
    # the fp32 oracle's first 32 tokens for this exact model and prompt (written offline by
    # tests/golden/make_qwen3_greedy_golden.py from the same seeds)
    oracle = {}
    fixture = ROOT / "tests" / "golden" / "qwen3_0.6b_greedy.npz"
    if fixture.exists() and batch == 16 and prompt_len == 512 and new_tokens >= 32:
        with np.load(fixture) as f:
            if np.array_equal(f["prompt"], prompt.numpy()):
                ref = f["uniform_tokens"]
                got32 = toks[:, :ref.shape[1]].numpy()
                oracle = {"sequences_matching_fp32_oracle_32_steps": int((got32 == ref).all(axis=1).sum()),
                          "of": int(ref.shape[0])}
    best = max(runs.values(), key=lambda r: r["decode_tokens_per_s"])
    out["batch_decode"] = {
        "workload": f"random-init Qwen3-0.6B (28 layers, W4A16 g128, bf16 tied lm_head), batch {batch}, "
                    f"prompt {prompt_len} (one prefill pass), {new_tokens} new tokens",
        **best,
        "prefill_ms_steady": round(prefill_steady_ms, 2),
        "prefill_kernels": prefill_kernels,
        "prefill_tokens_per_s_steady": round(batch * prompt_len / (prefill_steady_ms * 1e-3), 1),
        "by_streams": {str(k): v for k, v in runs.items()},
        "step_kernels": {"position": prompt_len + new_tokens // 2, "by_kernel": per_kernel,
                         "sum_ms_per_step": round(kernel_sum_ms, 4),
                         "method": "each kernel's launches of 5 steps in a graph of their own (140 launches, "
                                   "each round on its own weight copies; a per-step kernel 140 times), HBM-cold "
                                   "(a 512 MB read between replays), HIP events per replay on the launch stream, "
                                   "no host wait between replays; wall time per launch; with the chained norm "
                                   "(by_kernel.chained_norm) qkv and gate_up take the norm's input from o_proj and "
                                   "down, which write it (keys as without)"},
        "teacher_forced_prompt": teacher_forced,
        "one_launch_step": one_launch,
        "greedy_parity": oracle,
        "first_tokens": toks[:2, :8].tolist(),
    }
    del model
    torch.cuda.empty_cache()
    return out, tensors, prompt


def time_step_kernels(model, dev, reps: int, pos: int, passes: int = 5) -> dict:
    """Each kernel of the batch-decode step on its own, outside any profiler: per
    kernel a graph of its launches in ``passes`` steps (28 per layer kernel and
    step, a per-step kernel as often) over the model's own weights and caches at
    position ``pos`` for every sequence, replayed ``reps`` times; a read of a 512 MB pool between
    replays (untimed) leaves the MALL without any of the step's bytes, as the
    1.6 GB step itself does, so every replay reads HBM.  HIP events bracket each
    replay on the stream the kernels run on.  Returns microseconds per launch
    (wall time in the graph: launch gaps included, an upper bound on the kernel's
    own duration) and per step, with each kernel's algorithmic bytes."""
    import torch
    from torch2iron_amd import ops
    from torch2iron_amd.formats import algorithmic_bytes
    c, b = model.cfg, model.batch
    buf = model.micro[0].buf
    positions = torch.full((b,), pos, dtype=torch.int32, device=dev)
    adv_positions = positions.clone()   # advanced by every greedy_advance replay
    pool = torch.empty(512 << 20, dtype=torch.uint8, device=dev).fill_(3)
    sink = torch.empty(1 << 20, dtype=torch.int32, device=dev)
    x0 = model.x.clone()
    tokens = model.tokens.clone()
    kv_bytes = b * c.n_kv_heads * (pos + 1) * c.head_dim * 2 * 2
    qkv_n, hq = c.qkv_dim, c.n_heads * c.head_dim
    # ``passes`` rounds over the layers per graph, so that a graph's own start is
    # spread over about as many launches as the step's graph has (143).  Each round
    # reads its own copy of the linear weights (the 28 layers' qkv weights alone,
    # 61 MB, would stay in the 256 MB MALL from one round to the next); the KV
    # caches (1.2 GB) and the 311 MB lm_head table leave it anyway.
    from torch2iron_amd.formats import W4A16Weight

    def copies(get):
        # copies carry tiles like the model's own weights
        return [[get(L.w) if r == 0 else ops.tile_weight(W4A16Weight(get(L.w).qweight.clone(),
                                                                     get(L.w).qzeros.clone(), get(L.w).scales.clone()))
                 for L in model.layers]
                for r in range(passes)]

    wq, wo = copies(lambda w: w.qkv), copies(lambda w: w.o)
    wgu, wd = copies(lambda w: w.gate_up), copies(lambda w: w.down)
    # the layers' own forms: with the chained norm, o_proj and down also write the next
    # norm's input and sums of squares, which qkv and gate_up take (layer 0's qkv and the
    # last layer's down run unchained in the step, counted here in the chained form)
    chain = model.layers[0].chain
    ss_bytes = b * (c.hidden // 16) * 4

    def qkv_op(r, i, L):
        if chain:
            return ops.prenormed_linear(buf.xg, buf.ssp, c.eps, wq[r][i], out=buf.qkv)
        return ops.rmsnorm_linear(buf.x, L.w.ln1, c.eps, wq[r][i], out=buf.qkv)

    def o_op(r, i, L):
        if chain:
            return ops.linear_residual_next_norm(buf.ctx, wo[r][i], buf.x, buf.x, L.w.ln2, buf.xg, buf.ssp)
        return ops.linear(buf.ctx, wo[r][i], residual=buf.x, out=buf.x)

    def gu_op(r, i, L):
        if chain:
            return ops.prenormed_gate_up(buf.xg, buf.ssp, c.eps, wgu[r][i], swiglu=True, out=buf.hmlp)
        return ops.rmsnorm_gate_up(buf.x, L.w.ln2, c.eps, wgu[r][i], swiglu=True, out=buf.hmlp)

    def down_op(r, i, L):
        if chain:
            return ops.linear_residual_next_norm(buf.hmlp, wd[r][i], buf.x, buf.x, L.w.ln1, buf.xg, buf.ssp)
        return ops.linear(buf.hmlp, wd[r][i], residual=buf.x, out=buf.x)

    # a producer's extra bytes: the next norm's weight read, its input and the sums written
    nxt_bytes = (c.hidden * 2 + b * c.hidden * 2 + ss_bytes) if chain else 0
    norm_in_bytes = ss_bytes if chain else c.hidden * 2   # the sums read, or the norm weight
    per_layer = [
        ("rmsnorm_qkv", qkv_op, algorithmic_bytes(b, c.hidden, qkv_n) + norm_in_bytes),
        ("attention", lambda r, i, L: ops.decode_attention(buf.qkv, positions, c.n_heads, c.n_kv_heads, L.w.q_norm,
                                                           L.w.k_norm, c.eps, model.rope, model.k_cache[i],
                                                           model.v_cache[i], rope_style=L.rope_style, out=buf.ctx,
                                                           workspace=buf.workspace),
         kv_bytes + b * qkv_n * 2 + b * c.n_kv_heads * c.head_dim * 2 * 2 + b * hq * 2),
        ("o_proj_residual", o_op, algorithmic_bytes(b, hq, c.hidden) + b * c.hidden * 2 + nxt_bytes),
        ("rmsnorm_gate_up_swiglu", gu_op,
         algorithmic_bytes(b, c.hidden, 2 * c.intermediate) - b * c.intermediate * 2 + norm_in_bytes),
        ("down_residual", down_op, algorithmic_bytes(b, c.intermediate, c.hidden) + b * c.hidden * 2 + nxt_bytes),
    ]
    per_step = [
        ("embedding_gather_rmsnorm", lambda: ops.rmsnorm(model.embed, model.layers[0].w.ln1, c.eps, out=buf.xn,
                                                         tokens=model.tokens, x_out=buf.x, argmax_keys=model.keys),
         b * c.hidden * 2 * 3 + c.hidden * 2 + b * 4),
        ("final_rmsnorm_lm_head_argmax", lambda: model._head(False),
         model.lm_head.numel() * 2 + b * c.hidden * 2 + c.hidden * 2 + b * 8),
        ("greedy_advance", lambda: ops.greedy_advance(model.keys, model.tokens, adv_positions, None, model.step),
         b * 8 + b * 4 * 3),
    ]
    out = {}
    n = len(model.layers) * passes
    # a per-step kernel is launched n times in its graph too, so that every graph
    # spreads its own start over the same number of launches
    jobs = [(name, [lambda r=r, i=i, L=L, f=f: f(r, i, L) for r in range(passes) for i, L in enumerate(model.layers)],
             passes, nb) for name, f, nb in per_layer]
    jobs += [(name, [f] * n, n, nb) for name, f, nb in per_step]
    jobs.append(("graph_floor_one_element_fill", [lambda: sink[:1].fill_(0)] * n, n, 0))
    stream = torch.cuda.current_stream(dev)
    for name, calls, div, nbytes in jobs:
        for fn in calls:
            fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for fn in calls:
                fn()
        marks = []
        for r in range(reps + 1):   # no host wait between replays: the GPU never idles
            model.x.copy_(x0)
            buf.x.copy_(x0)
            model.tokens.copy_(tokens)
            ops.stream_read(pool, out=sink)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            g.replay()
            e1.record(stream)
            marks.append((e0, e1))
        torch.cuda.synchronize()
        total = sum(a.elapsed_time(b) for a, b in marks[1:])   # the first replay is a warm-up
        us = total * 1e3 / (reps * len(calls))
        per_step_launches = len(calls) // div
        out[name] = {"launches_per_step": per_step_launches, "us_per_launch": round(us, 3),
                     "us_per_step": round(us * per_step_launches, 1), "algorithmic_bytes_per_launch": int(nbytes),
                     "TBps": round(nbytes / us / 1e6, 4), "frac_of_8TBps": round(nbytes / us / 1e6 / 8.0, 4)}
        del g
    floor = out.pop("graph_floor_one_element_fill")
    out["graph_floor_us_per_launch"] = floor["us_per_launch"]
    out["chained_norm"] = bool(chain)
    model.x.copy_(x0)
    model.tokens.copy_(tokens)
    del pool, sink
    return out


def time_prefill_kernels(model, dev, reps: int = 5) -> dict:
    """Each kernel of the prompt pass on its own, outside any profiler: per kernel a
    graph of its 28 launches (one per layer, the model's own weights, caches and prompt
    buffers, as ``Qwen3Model.prefill`` last left them), replayed ``reps`` times after a
    warm-up replay, HIP events around each replay on the launch stream.  The products'
    outputs go to spare buffers, so that replays do not feed on themselves.  Returns
    microseconds per launch and per pass, and TFLOP/s (matrix kernels: 2 M K N; the
    attention: its causal half of QK^T and PV) or TB/s (the norms)."""
    import torch
    from torch2iron_amd import ops
    c, b = model.cfg, model.batch
    pf = model._pf
    t = pf["t"]
    r = b * t
    xs_n, xs_ctx, xs_h = pf.get("xn_sums"), pf.get("ctx_sums"), pf.get("h_sums")
    y_h = torch.empty(r, c.hidden, dtype=torch.bfloat16, device=dev)
    q = pf["q"]
    hq = c.n_heads * c.head_dim
    jobs = [
        ("rmsnorm", lambda i, L: ops.rmsnorm(pf["x"], L.w.ln1, c.eps, out=pf["xn"], out_sums=xs_n), 2,
         "TB/s", r * c.hidden * 2 * 2 + (r * c.hidden // 128) * 4),
        ("qkv_prep", lambda i, L: ops.prefill_qkv_rope_kv(pf["xn"], L.w.qkv, b, 0, c.n_heads, c.n_kv_heads,
                                                            L.w.q_norm, L.w.k_norm, c.eps, model.rope,
                                                            model.k_cache[i], model.v_cache[i],
                                                            rope_style=L.rope_style, q_out=q, x_sums=xs_n), 1,
         "TFLOP/s", 2 * r * c.hidden * c.qkv_dim),
        ("attention", lambda i, L: ops.prefill_attention(q, 0, c.n_kv_heads, model.k_cache[i], model.v_cache[i],
                                                         out=pf["ctx"], out_sums=xs_ctx), 1,
         "TFLOP/s", 4 * b * c.n_heads * t * t * c.head_dim // 2),
        ("o_proj_residual", lambda i, L: ops.linear(pf["ctx"], L.w.o, residual=pf["x"], out=y_h, x_sums=xs_ctx), 1,
         "TFLOP/s", 2 * r * hq * c.hidden),
        ("gate_up_swiglu", lambda i, L: ops.gate_up(pf["xn"], L.w.gate_up, swiglu=True, out=pf["h"], x_sums=xs_n,
                                                    out_sums=xs_h), 1,
         "TFLOP/s", 2 * r * c.hidden * 2 * c.intermediate),
        ("down_residual", lambda i, L: ops.linear(pf["h"], L.w.down, residual=pf["x"], out=y_h, x_sums=xs_h,
                                                  sum_parts=2), 1,
         "TFLOP/s", 2 * r * c.intermediate * c.hidden),
    ]
    stream = torch.cuda.current_stream(dev)
    out = {}
    total_ms = 0.0
    for name, f, per_layer, unit, work in jobs:
        calls = [lambda i=i, L=L, f=f: f(i, L) for i, L in enumerate(model.layers)]
        for fn in calls:
            fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for fn in calls:
                fn()
        marks = []
        for _ in range(reps + 1):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            g.replay()
            e1.record(stream)
            marks.append((e0, e1))
        torch.cuda.synchronize()
        us = sum(a.elapsed_time(b2) for a, b2 in marks[1:]) * 1e3 / (reps * len(calls))
        launches = per_layer * len(calls)
        rate = work / us / 1e6
        out[name] = {"launches_per_pass": launches, "us_per_launch": round(us, 2),
                     "us_per_pass": round(us * launches, 1),
                     ("TFLOPs" if unit == "TFLOP/s" else "TBps"): round(rate, 1 if unit == "TFLOP/s" else 3),
                     ("frac_of_2_5PFLOPs" if unit == "TFLOP/s" else "frac_of_8TBps"):
                         round(rate / (2500.0 if unit == "TFLOP/s" else 8.0), 4)}
        total_ms += us * launches / 1e3
        del g
    out["sum_ms_per_pass"] = round(total_ms, 3)
    return out


# ---------------------------------------------------------------------------
# CPU baselines: the oracle on the host cores (bounded samples)
# ---------------------------------------------------------------------------

def bench_attention(dev, steps: int, warmup: int, eager: bool, calibrate: bool) -> dict:
    """Decode attention at the batch-decode shape (16 sequences, 16 q / 8 kv heads, 577
    cached slots each: position 576 of a 640-slot cache), HBM-cold: 28 cache pairs, one
    per layer, cycled (1.2 GB, past the 256 MB MALL).  A step is 28 calls, one graph
    replay (eager launches with ``eager``, for counter runs); event-timed on the stream
    the calls launch on."""
    import torch
    from torch2iron_amd import ops
    from torch2iron_amd import model as gm
    b, hq, hkv, d, cap, pos, layers = 16, 16, 8, 128, 640, 576, 28
    g = torch.Generator(device=dev).manual_seed(6)
    kcs = [torch.randn(b, hkv, cap, d, generator=g, device=dev).to(torch.bfloat16) for _ in range(layers)]
    vcs = [torch.randn(b, hkv, cap, d, generator=g, device=dev).to(torch.bfloat16) for _ in range(layers)]
    qkv = torch.randn(b, (hq + 2 * hkv) * d, generator=g, device=dev).to(torch.bfloat16)
    qn = (torch.rand(d, generator=g, device=dev) * 0.2 + 0.9).to(torch.bfloat16)
    kn = (torch.rand(d, generator=g, device=dev) * 0.2 + 0.9).to(torch.bfloat16)
    rope = gm.rope_table(d, cap, 1e6, dev)
    positions = torch.full((b,), pos, dtype=torch.int32, device=dev)
    out = torch.empty(b, hq * d, dtype=torch.bfloat16, device=dev)
    ws = ops.Workspace()

    def step():
        for i in range(layers):
            ops.decode_attention(qkv, positions, hq, hkv, qn, kn, 1e-6, rope, kcs[i], vcs[i], out=out, workspace=ws)

    step()
    torch.cuda.synchronize()
    run = step
    if not eager:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        run = graph.replay
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        run()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (steps * layers)
    # algorithmic bytes of a call: the K/V rows of the 577 slots, the qkv rows read, the
    # new k/v rows written, the context written
    kv = b * hkv * (pos + 1) * d * 2 * 2
    nbytes = kv + qkv.numel() * 2 + b * hkv * d * 2 * 2 + out.numel() * 2
    if calibrate:
        src = torch.empty(COPY_BYTES, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
    res = {"workload": f"decode attention, batch {b}, {hq} q / {hkv} kv heads, head_dim {d}, {pos + 1} cached "
                       f"slots ({cap}-slot cache), {layers} cache pairs cycled (HBM-cold), "
                       + ("eager launches" if eager else "graph replays"),
           "us_per_call": round(us, 3), "algorithmic_bytes_per_call": nbytes,
           "TBps": round(nbytes / us / 1e6, 4), "frac_of_8TBps": round(nbytes / us / 1e6 / 8.0, 4)}
    log(f"decode attention: {us:.2f} us per call, {nbytes / us / 1e6:.3f} TB/s of {nbytes / 1e6:.1f} MB algorithmic")
    return res


def bench_prompt_gemm(dev, steps: int, warmup: int, eager: bool) -> dict:
    """The prompt pass's four W4A16 GEMMs (Qwen3-0.6B, 16 x 512 = 8192 rows) with their
    epilogues: qkv, o_proj + residual, gate_up + SwiGLU (and its half-group sums), down +
    residual, each given its input's row group sums as the prompt pass hands them over
    (``own_sums_us_per_launch``: the same GEMM forming them itself).  A step runs each 8
    times (one graph replay; eager launches with ``eager``, for counter runs); the weights
    stay MALL-warm, as the GEMMs are bound by their k-loops, not by bytes."""
    import torch
    from torch2iron_amd import ops
    from torch2iron_amd.formats import random_weight_on_device
    m, reps = 8192, 8
    g = torch.Generator(device=dev).manual_seed(9)
    res = {}
    for name, k, n in (("qkv", 1024, 4096), ("o_proj", 2048, 1024), ("gate_up", 1024, 6144), ("down", 3072, 1024)):
        w = random_weight_on_device(k, n, g, dev)
        x = torch.randn(m, k, generator=g, device=dev).to(torch.bfloat16)
        parts = 2 if name == "down" else 1
        xs = x.double().view(m, k * parts // 128, 128 // parts).sum(-1).t().float().contiguous()   # group-major
        if name == "gate_up":
            y = torch.empty(m, n // 2, dtype=torch.bfloat16, device=dev)
            hs = torch.empty(n // 128, m, device=dev)
            forms = {"sums": lambda: ops.gate_up(x, w, swiglu=True, out=y, x_sums=xs, out_sums=hs),
                     "own": lambda: ops.gate_up(x, w, swiglu=True, out=y)}
        elif name == "qkv":
            y = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
            forms = {"sums": lambda: ops.linear(x, w, out=y, x_sums=xs), "own": lambda: ops.linear(x, w, out=y)}
        else:
            r = torch.randn(m, n, generator=g, device=dev).to(torch.bfloat16)
            y = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
            forms = {"sums": lambda: ops.linear(x, w, residual=r, out=y, x_sums=xs, sum_parts=parts),
                     "own": lambda: ops.linear(x, w, residual=r, out=y)}
        us_by = {}
        for form, call in forms.items():
            us_by[form] = _time_prompt_gemm(call, reps, steps, warmup, eager)
        us = us_by["sums"]
        flops = 2 * m * k * n
        res[name] = {"M": m, "K": k, "N": n, "us_per_launch": round(us, 2), "TFLOPs": round(flops / us / 1e6, 1),
                     "frac_of_2_5PFLOPs": round(flops / us / 1e6 / 2500.0, 4),
                     "own_sums_us_per_launch": round(us_by["own"], 2)}
        log(f"prompt GEMM {name} M={m} K={k} N={n}: {us:.1f} us, {flops / us / 1e6:.0f} TFLOP/s "
            f"(forming its own row sums: {us_by['own']:.1f} us)")
        del w, x, y
    # the prompt pass's causal attention: 16 sequences x 512 rows, 16 q / 8 kv heads,
    # head_dim 128, with its head sums; flops 4 B Hq T^2 D / 2 (causal half of QK^T and PV)
    b, t, hq, hkv, d = 16, 512, 16, 8, 128
    q = torch.randn(b, hq, t, d, generator=g, device=dev).to(torch.bfloat16)
    kc = torch.randn(b, hkv, t, d, generator=g, device=dev).to(torch.bfloat16)
    vc = torch.randn(b, hkv, t, d, generator=g, device=dev).to(torch.bfloat16)
    out = torch.empty(b * t, hq * d, dtype=torch.bfloat16, device=dev)
    sums = torch.empty(hq, b * t, device=dev)
    us = _time_prompt_gemm(lambda: ops.prefill_attention(q, 0, hkv, kc, vc, out=out, out_sums=sums), reps, steps,
                           warmup, eager)
    flops = 4 * b * hq * t * t * d / 2
    res["attention"] = {"B": b, "T": t, "Hq": hq, "Hkv": hkv, "D": d, "us_per_launch": round(us, 2),
                        "TFLOPs": round(flops / us / 1e6, 1), "frac_of_2_5PFLOPs": round(flops / us / 1e6 / 2500.0, 4)}
    log(f"prompt attention B={b} T={t} Hq={hq} Hkv={hkv}: {us:.1f} us, {flops / us / 1e6:.0f} TFLOP/s (causal)")
    return res


def _time_prompt_gemm(call, reps: int, steps: int, warmup: int, eager: bool) -> float:
    """Microseconds a launch of ``call``: ``steps`` replays of a graph of ``reps`` launches."""
    import torch
    call()
    torch.cuda.synchronize()

    def step():
        for _ in range(reps):
            call()

    run = step
    if not eager:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        run = graph.replay
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        run()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (steps * reps)


def cpu_info() -> dict:
    import torch
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"cpu_model": model, "os_cpu_count": os.cpu_count(), "torch_threads": torch.get_num_threads()}


def _timed_runs(fn, seconds: float, min_runs: int = 20, max_runs: int = 200):
    """Median wall time (s) of ``fn()`` over at least ``min_runs`` runs, more while
    the budget lasts; one untimed warm-up run first."""
    fn()
    times = []
    t_end = time.perf_counter() + seconds
    while len(times) < max_runs and (len(times) < min_runs or time.perf_counter() < t_end):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def cpu_linear_baselines(seconds: float) -> dict:
    """Configs 0-2 on the host: per call, the oracle's dequant + fp32 group-loop
    matmul (the reference runtime's arithmetic, ``model.py:133-146``), and the
    matmul alone with the dense fp32 weight cached (the reference caches its
    unpacked weight, ``model.py:122-131``)."""
    import numpy as np
    from oracle import w4a16 as ow
    from torch2iron_amd.formats import algorithmic_bytes

    out = {}
    cases = [("config0_gemv", "up_proj", 1, 1024, 3072)]
    cases += [(f"config1_M16_{n}", n, 16, k, nn) for n, k, nn in QWEN3_06B]
    cases += [(f"config2_M16_{n}", n, 16, k, nn) for n, k, nn in QWEN3_17B]
    for i, (label, _, m, k, n) in enumerate(cases):
        qw, qz, sc = ow.synthetic_tensors(k, n, seed=100 + i)
        x = np.random.default_rng(i).standard_normal((m, k)).astype(np.float32)
        b = algorithmic_bytes(m, k, n)
        t_call, n_call = _timed_runs(lambda: ow.linear(x, qw, qz, sc, accumulate="fp32"), seconds / 2)
        w = ow.dequantize(qw, qz, sc)
        t_mm, n_mm = _timed_runs(lambda: x @ w.T, seconds / 2)
        out[label] = {"M": m, "K": k, "N": n,
                      "dequant_matmul_us": round(t_call * 1e6, 1), "dequant_matmul_GBps": round(b / t_call / 1e9, 3),
                      "cached_matmul_us": round(t_mm * 1e6, 1), "cached_matmul_GBps": round(b / t_mm / 1e9, 3),
                      "runs": [n_call, n_mm]}
    return out


def cpu_decode_baselines(tensors, prompt, seconds: float, new_tokens: int) -> dict:
    """Configs 3 and 4 on the host with the fp32 oracle (dense fp32 weights cached):
    one decode layer at batch 8, context 1024; the batch-16 prompt pass over the
    same 512-token prompt as the GPU run, then greedy decode steps from it."""
    import torch
    from oracle import qwen3 as oq
    from torch2iron_amd import model as gm

    cfg = gm.QWEN3_0_6B
    ocfg = oq.Qwen3Config(**{k: getattr(cfg, k) for k in oq.Qwen3Config.__dataclass_fields__})
    out = {}
    # config 3: layer 0 of the same weights, B = 8, 1024 cached positions, write at 1024
    layer = oq.DenseLayer(tensors, "model.layers.0", ocfg)
    g = torch.Generator().manual_seed(5)
    kc = torch.randn(8, cfg.n_kv_heads, 1088, cfg.head_dim, generator=g)
    vc = torch.randn(8, cfg.n_kv_heads, 1088, cfg.head_dim, generator=g)
    x = torch.randn(8, cfg.hidden, generator=g)
    angles = oq.rope_angles(cfg.head_dim, 1088, cfg.rope_theta)
    pos = torch.full((8,), 1024, dtype=torch.long)
    rnd = oq._Round("fp32")
    with torch.no_grad():
        t_layer, n_layer = _timed_runs(lambda: layer.decode(x, kc, vc, pos, angles, rnd), seconds, min_runs=20)
    out["config3_decode_layer"] = {"us": round(t_layer * 1e6, 1), "runs": n_layer,
                                   "sample": "fp32 oracle decode layer, batch 8, context 1024, median"}
    del layer, kc, vc
    # config 4: the whole model
    b, plen = prompt.shape
    m = oq.DenseQwen3(tensors, ocfg, mode="fp32", ctx_cap=plen + new_tokens)
    t0 = time.perf_counter()
    logits = m.prefill(prompt)
    t_prompt = time.perf_counter() - t0
    pos = torch.full((b,), plen, dtype=torch.long)
    step_times = []
    t_end = time.perf_counter() + seconds
    while len(step_times) < 3 or (time.perf_counter() < t_end and len(step_times) < new_tokens - 1):
        nxt = torch.argmax(logits, dim=-1)
        t1 = time.perf_counter()
        logits = m.decode_step(nxt, pos)
        step_times.append(time.perf_counter() - t1)
        pos = pos + 1
    t_step = statistics.median(step_times)
    t_decode = t_step * (new_tokens - 1)
    out["config4_batch_decode"] = {
        "prompt_s": round(t_prompt, 2),
        "prompt_tokens_per_s": round(b * plen / t_prompt, 1),
        "ms_per_decode_step": round(t_step * 1e3, 2),
        "decode_tokens_per_s": round(b / t_step, 2),
        "end_to_end_tokens_per_s": round(b * new_tokens / (t_prompt + t_decode), 2),
        "sample": (f"fp32 oracle: one batch-{b} prompt pass over {plen} tokens (timed), then {len(step_times)} "
                   f"decode steps from position {plen} (median); end to end = prompt + {new_tokens - 1} x the "
                   f"median step"),
    }
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported: the W4A16 path runs "
              "on one GPU (data-parallel decode would replicate the weights and split the batch)",
              file=sys.stderr)
        sys.exit(2)
    import torch
    from torch2iron_amd import _lib
    _lib.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.prompt_gemm_only:
        gemm = bench_prompt_gemm(dev, args.steps, args.warmup, args.eager)
        print(json.dumps({"metric": METRIC, "value": None, "unit": "TB/s", "n_gpus": 1, "note": "prompt GEMM only",
                          "prompt_gemm": gemm}), flush=True)
        return
    if args.attention_only:
        att = bench_attention(dev, args.steps, args.warmup, args.eager, args.calibrate_copy)
        print(json.dumps({"metric": METRIC, "value": None, "unit": "TB/s", "n_gpus": 1, "note": "attention only",
                          "decode_attention": att}), flush=True)
        return
    if args.decode_only:
        decode, _, _ = bench_decode(dev, args.steps, args.warmup, args.prompt, args.new_tokens, args.batch,
                                    [int(v) for v in args.streams.split(",")], teacher_forced_leg=False)
        print(json.dumps({"metric": METRIC, "value": None, "unit": "TB/s", "n_gpus": 1, "note": "decode only",
                          **decode}), flush=True)
        return
    ms = [1, 8, 16, 32, 64]
    log(f"building HBM-cold sweep (pool {args.pool_mb} MB)")
    cold = Sweep(QWEN3_06B, ms, args.pool_mb << 20, dev, seed=1, eager=args.eager)
    log(f"{cold.copies} weight copies ({cold.pool_mb:.0f} MB), {cold.launches_per_step} launches/step, "
        f"{cold.bytes_per_step / 1e6:.1f} MB/step")
    value, ms_per_step, per_group = rate(cold, args.steps, args.warmup)
    avg_launch_us = ms_per_step * 1e3 / cold.launches_per_step
    log(f"HBM-cold sweep: {value:.3f} TB/s, {ms_per_step:.3f} ms/step, avg launch {avg_launch_us:.2f} us")
    floor_us = None if args.eager else launch_floor(dev, cold.launches_per_step, args.steps, args.warmup)
    if floor_us is not None:
        log(f"launch floor (one-element fill, graph): {floor_us:.2f} us per launch")
    breakdown = cold.breakdown(per_group)
    cold_pool_mb = cold.pool_mb
    cold_copies = cold.copies
    cold_bytes = cold.bytes_per_step
    cold_groups = [dict(label=gr["label"], bytes=gr["bytes"], launches=gr["launches"]) for gr in cold.groups]
    cold_launches = cold.launches_per_step

    if args.calibrate_copy:
        src = torch.empty(COPY_BYTES, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    del cold
    torch.cuda.empty_cache()

    ceiling = None
    if not args.eager:
        log("HBM read ceiling: the sweep's byte counts and launches through a read-only kernel, and a 1 GiB read")
        ceiling = read_ceiling(cold_groups, args.pool_mb << 20, dev, args.steps, args.warmup)
        log(f"read ceiling: {ceiling['same_launches_TBps']:.3f} TB/s at the sweep's launches "
            f"({ceiling['same_launches_us_per_launch']:.2f} us per launch); bulk {ceiling['bulk_1GiB_TBps']:.3f} TB/s")
        ceiling["frac_of_same_launches"] = round(value / ceiling["same_launches_TBps"], 4)
        ceiling["frac_of_bulk"] = round(value / ceiling["bulk_1GiB_TBps"], 4)

    extra = {}
    if not args.skip_extra:
        log("HBM-cold sweep over the AutoGPTQ words (the reference-layout entry points, no tiles)")
        flat = Sweep(QWEN3_06B, ms, args.pool_mb << 20, dev, seed=1, eager=args.eager, tiled=False)
        f_rate, f_ms, _ = rate(flat, args.steps, args.warmup)
        extra["autogptq_layout_sweep"] = {"TBps": round(f_rate, 4),
                                          "avg_launch_us": round(f_ms * 1e3 / flat.launches_per_step, 3)}
        log(f"AutoGPTQ-layout sweep: {f_rate:.3f} TB/s")
        del flat
        torch.cuda.empty_cache()
        log("MALL-warm sweep (one weight copy)")
        warm = Sweep(QWEN3_06B, ms, 0, dev, seed=2, reps=cold_copies)
        extra["mall_warm_TBps"] = round(rate(warm, args.steps, args.warmup)[0], 4)
        del warm
        log("single GEMV, M=1 K=1024 N=3072 (HBM-cold and MALL-warm)")
        gv = Sweep(GEMV_06B, [1], args.pool_mb << 20, dev, seed=4)
        gv_rate, gv_ms, _ = rate(gv, args.steps, args.warmup)
        gvw = Sweep(GEMV_06B, [1], 0, dev, seed=5, reps=gv.copies)
        gvw_rate, gvw_ms, _ = rate(gvw, args.steps, args.warmup)
        extra["gemv_m1_k1024_n3072"] = {
            "workload": f"W4A16 GEMV M=1 K=1024 N=3072 (Qwen3-0.6B up_proj), {gv.copies} launches per step",
            "hbm_cold_TBps": round(gv_rate, 4), "hbm_cold_us_per_launch": round(gv_ms * 1e3 / gv.launches_per_step, 3),
            "mall_warm_TBps": round(gvw_rate, 4), "mall_warm_us_per_launch": round(gvw_ms * 1e3 / gvw.launches_per_step, 3),
            "pool_mb": round(gv.pool_mb, 1)}
        del gv, gvw
        log("Qwen3-1.7B sweep (HBM-cold)")
        big = Sweep(QWEN3_17B, [1, 16, 64], args.pool_mb << 20, dev, seed=3)
        b_steps = max(2, args.steps // 2)
        b_rate, _, b_groups = rate(big, b_steps, 1)
        extra["qwen3_1_7b_sweep_TBps"] = round(b_rate, 4)
        extra["qwen3_1_7b_breakdown"] = big.breakdown(b_groups)
        extra["qwen3_1_7b_pool_mb"] = round(big.pool_mb, 1)
        del big
        torch.cuda.empty_cache()
    torch.cuda.synchronize()

    decode = None
    tensors = prompt = None
    if not args.skip_decode:
        decode, tensors, prompt = bench_decode(dev, args.steps, args.warmup, args.prompt, args.new_tokens,
                                               args.batch, [int(v) for v in args.streams.split(",")])
        torch.cuda.synchronize()

    cpu = None
    if not args.skip_cpu:
        log(f"CPU baselines (about {args.cpu_seconds:.0f} s per leg)")
        info = cpu_info()
        lin = cpu_linear_baselines(args.cpu_seconds)
        # the headline's CPU figure: the per-call form over the config-1 shapes at M=16
        c1 = [v for k, v in lin.items() if k.startswith("config1_")]
        c1_bytes = sum(v["dequant_matmul_GBps"] * v["dequant_matmul_us"] for v in c1)   # GB/s * us = kB
        c1_us = sum(v["dequant_matmul_us"] for v in c1)
        c1_cached = sum(v["cached_matmul_GBps"] * v["cached_matmul_us"] for v in c1)
        c1_cached_us = sum(v["cached_matmul_us"] for v in c1)
        cpu = {"value": round(c1_bytes / c1_us / 1e3, 6), "unit": "TB/s", "cores": info["torch_threads"],
               "kind": "port",
               "sample": "oracle dequant + fp32 matmul per call, M=16, the four Qwen3-0.6B shapes, median of >= 20 "
                         "calls each (algorithmic bytes over time)",
               "cached_weights_value": round(c1_cached / c1_cached_us / 1e3, 6),
               **info, "linear": lin}
        if tensors is not None:
            log("CPU decode baselines (config 3 layer, config 4 prompt pass + decode steps)")
            cpu.update(cpu_decode_baselines(tensors, prompt, args.cpu_seconds, args.new_tokens))

    achieved_gbps = value * 1e3
    traffic = _load_json(TRAFFIC_FILE)
    bd = (decode or {}).get("batch_decode") or {}
    line = {
        "metric": METRIC,
        "value": round(value, 4),
        "unit": "TB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "decode_tokens_per_s": bd.get("decode_tokens_per_s"),
        "decode_ms_per_step": bd.get("ms_per_decode_step"),
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "W4A16 group-128 linear sweep, Qwen3-0.6B qkv/o_proj/gate_up/down x M in {1,8,16,32,64}, "
                        f"HBM-cold ({cold_copies}-copy weight pool, {cold_pool_mb:.0f} MB)",
            "weights": "int4 AutoGPTQ (uniform nibbles, fp16 scales U[0.005,0.02])",
            "activations": "bf16 N(0,1)",
            "launches_per_step": len(ms) * len(QWEN3_06B) * cold_copies,
            "bytes_per_step": cold_bytes,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved_gbps, 1),
            "peak": PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved_gbps / PEAK_GBPS, 4),
            "traffic": (traffic or {}).get("hbm_bytes_per_launch"),
            "traffic_source": (traffic or {}).get("source"),
            "kernel": "w4a16_mfma_kernel",
            "avg_launch_us": round(avg_launch_us, 3),
            "launch_floor_us": None if floor_us is None else round(floor_us, 3),
            "read_ceiling": ceiling,
            "kernel_time": {
                "avg_us_per_launch": round(avg_launch_us, 3),
                "algorithmic_bytes_per_launch": round(cold_bytes / cold_launches),
                "frac": round(cold_bytes / cold_launches / (avg_launch_us * 1e-6) / (PEAK_GBPS * 1e9), 4),
                "source": "HIP events around each (shape, M) group's graph of its launches (wall time per launch in "
                          "the graph, an upper bound on the kernel's own duration); rocprofv3 traces are kept for "
                          "kernel names and counters only: their per-dispatch signals stretch the durations"},
        },
        "cpu_baseline": cpu,
        "breakdown": breakdown,
        **extra,
        **(decode or {}),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
