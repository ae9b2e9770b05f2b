#!/usr/bin/env python3
"""Benchmark of the MI355X W4A16 hot path (one GPU).

Workload (one "step"): the W4A16 group-128 linear over every Qwen3-0.6B linear
shape -- fused qkv K=1024 N=4096, o_proj K=2048 N=1024, fused gate_up K=1024
N=6144, down K=3072 N=1024 -- at M in {1, 8, 16, 32, 64} (batched decode), each
(M, shape) pair launched once per weight copy of a pool larger than the
256 MB MALL, so weights stream from HBM (HBM-cold).  The launches are
captured in HIP graphs; inputs are resident in HBM before the timed region.

``value`` = algorithmic bytes of all launches / wall time of the timed steps
(TB/s).  Algorithmic bytes per launch: K*N/2 (int4) + (K/128)*N*2 (fp16
scales) + (K/128)*(N/8)*4 (int32 zeros) + M*K*2 + M*N*2 (bf16 in/out).

Extra fields: the MALL-warm rate (one weight copy reused), the per-(M, shape)
breakdown, the Qwen3-1.7B sweep, a roofline entry for the linear kernel and
the CPU baseline (the oracle's dequant + fp32 matmul on the host cores).
"""

from __future__ import annotations

import argparse
import json
import os
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
MALL_BYTES = 256 << 20
COPY_BYTES = 256 << 20
TRAFFIC_FILE = ROOT / "profiles" / "w4a16_linear_qwen3_0.6b_sweep_traffic.json"


def measured_traffic():
    """HBM bytes per launch of the sweep's linear kernel, from the FETCH_SIZE /
    WRITE_SIZE counter runs summarised in ``TRAFFIC_FILE`` (None if absent)."""
    try:
        return json.loads(TRAFFIC_FILE.read_text())
    except (OSError, ValueError):
        return None


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--pool-mb", type=int, default=320, help="weight pool per sweep (> 256 MB MALL)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--skip-extra", action="store_true", help="only the headline sweep")
    ap.add_argument("--skip-decode", action="store_true", help="skip the decode layer / greedy decode runs")
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--new-tokens", type=int, default=128)
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--streams", default="1,2", help="micro-batch stream counts to measure for batch decode")
    ap.add_argument("--eager", action="store_true", help="sweep launches without graphs (for counter collection)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a 256 MiB device copy (the reference kernel for HBM byte counters)")
    return ap.parse_args()


class Sweep:
    """Graph-captured launches of one (M, shape) grid over a weight pool."""

    def __init__(self, shapes, ms, pool_bytes, dev, seed, reps=None, eager=False):
        import torch
        from torch2iron_amd import ops
        from torch2iron_amd.formats import algorithmic_bytes, random_weight_on_device

        self.torch = torch
        gen = torch.Generator(device=dev).manual_seed(seed)
        per_copy = sum(k * n // 2 + (k // 128) * n * 2 + (k // 128) * (n // 8) * 4 for _, k, n in shapes)
        self.per_copy = per_copy
        self.copies = max(1, -(-pool_bytes // per_copy)) if pool_bytes else 1
        self.weights = {name: [random_weight_on_device(k, n, gen, dev) for _ in range(self.copies)]
                        for name, k, n in shapes}
        # launches per graph: one per weight copy (HBM-cold), or ``reps`` of the one copy (MALL-warm)
        self.reps = reps or self.copies
        self.eager = eager
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

    def run(self, steps, warmup):
        torch = self.torch
        for _ in range(warmup):
            for gr in self.groups:
                gr["replay"]()
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        marks = [[torch.cuda.Event(enable_timing=True) for _ in self.groups] for _ in range(steps)]
        start.record()
        for s in range(steps):
            for i, gr in enumerate(self.groups):
                gr["replay"]()
                marks[s][i].record()
        torch.cuda.synchronize()
        total_ms = start.elapsed_time(marks[-1][-1])
        per_group = [0.0] * len(self.groups)
        for s in range(steps):
            prev = start if s == 0 else marks[s - 1][-1]
            for i in range(len(self.groups)):
                per_group[i] += prev.elapsed_time(marks[s][i])
                prev = marks[s][i]
        per_group = [t / steps for t in per_group]
        return total_ms, per_group


def bench_decode(dev, steps: int, warmup: int, prompt_len: int, new_tokens: int, batch: int,
                 streams=(1, 2, 4)):
    """Config 3 (one fused decode layer, batch 8, 1024 cached tokens) and config 4
    (full Qwen3-0.6B, batch 16 greedy decode) on random-init weights."""
    import torch
    from torch2iron_amd import model as gm

    cfg = gm.QWEN3_0_6B
    log("generating random-init Qwen3-0.6B weights (uniform AutoGPTQ words, N(0,1) bf16 embedding)")
    tensors = gm.random_qwen3_tensors(cfg, seed=0)
    out = {}

    # ---- config 3: one decode layer, B = 8, context 1024 (write at 1024) ----
    b3, cap3 = 8, 1088
    rope = gm.rope_table(cfg.head_dim, cap3, cfg.rope_theta, dev)
    layer = gm.Qwen3DecodeLayer(gm.Qwen3LayerWeights(tensors, 0, cfg, dev), cfg, rope)
    buf = gm.DecodeBuffers(cfg, b3, dev)
    gen = torch.Generator(device=dev).manual_seed(5)
    kc = torch.randn(b3, cfg.n_kv_heads, cap3, cfg.head_dim, generator=gen, device=dev).to(torch.bfloat16)
    vc = torch.randn(b3, cfg.n_kv_heads, cap3, cfg.head_dim, generator=gen, device=dev).to(torch.bfloat16)
    pos = torch.full((b3,), 1024, dtype=torch.int32, device=dev)
    x0 = torch.randn(b3, cfg.hidden, generator=gen, device=dev).to(torch.bfloat16)
    buf.x.copy_(x0)
    layer(buf, pos, kc, vc)                      # eager warm-up (allocates the attention workspace)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        layer(buf, pos, kc, vc)
    reps = max(steps, 10) * 5
    for _ in range(warmup):
        buf.x.copy_(x0)
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    layer_us = e0.elapsed_time(e1) * 1e3 / reps
    w = layer.w
    layer_bytes = (w.qkv.nbytes + w.o.nbytes + w.gate_up.nbytes + w.down.nbytes + 4 * 2 * cfg.hidden
                   + 2 * 2 * cfg.head_dim + b3 * cfg.n_kv_heads * 1025 * cfg.head_dim * 2 * 2
                   + b3 * cfg.n_kv_heads * cfg.head_dim * 2 * 2 + b3 * cfg.hidden * 2 * 2)
    out["decode_layer"] = {"workload": "one fused Qwen3-0.6B decode layer, batch 8, context 1024",
                           "us": round(layer_us, 2), "algorithmic_bytes": layer_bytes,
                           "TBps": round(layer_bytes / (layer_us * 1e-6) / 1e12, 4),
                           "frac_of_8TBps": round(layer_bytes / (layer_us * 1e-6) / 8e12, 4)}
    log(f"decode layer (B=8, ctx 1024): {layer_us:.1f} us, {out['decode_layer']['TBps']} TB/s")
    del g, buf, layer, kc, vc
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
    # the prompt consumed one position at a time through the decode step (the NPU runner's way)
    model.set_streams(1)
    tm = {}
    tf = model.generate(prompt, new_tokens, timings=tm, prompt_mode="decode")
    teacher_forced = {"prompt_ms": round(tm["prompt_ms"], 2),
                      "end_to_end_tokens_per_s": round(batch * new_tokens / ((tm["prompt_ms"] + tm["decode_ms"]) * 1e-3), 1),
                      "first_token_equal_to_prefill": bool(torch.equal(tf[:, 0], toks[:, 0])),
                      "tokens_equal_to_prefill_run": bool(torch.equal(tf, toks))}
    log(f"teacher-forced prompt: {tm['prompt_ms']:.1f} ms")
    best = max(runs.values(), key=lambda r: r["decode_tokens_per_s"])
    out["batch_decode"] = {
        "workload": f"random-init Qwen3-0.6B (28 layers, W4A16 g128, bf16 tied lm_head), batch {batch}, "
                    f"prompt {prompt_len} (one prefill pass), {new_tokens} new tokens",
        **best,
        "by_streams": {str(k): v for k, v in runs.items()},
        "teacher_forced_prompt": teacher_forced,
        "first_tokens": toks[:2, :8].tolist(),
    }
    del model
    torch.cuda.empty_cache()
    return out, tensors, prompt, toks


def cpu_decode_baseline(tensors, seconds: float, batch: int):
    """The oracle (torch fp32 on the host cores) decoding a batch: a bounded sample."""
    import torch
    from oracle import qwen3 as oq
    from torch2iron_amd import model as gm

    cfg = gm.QWEN3_0_6B
    ocfg = oq.Qwen3Config(**{k: getattr(cfg, k) for k in oq.Qwen3Config.__dataclass_fields__})
    torch.set_num_threads(os.cpu_count() or 1)
    m = oq.DenseQwen3(tensors, ocfg, mode="fp32", ctx_cap=640)
    prompt = torch.randint(0, cfg.vocab, (batch, 16), generator=torch.Generator().manual_seed(7))
    logits = m.prefill(prompt)
    pos = torch.full((batch,), 16, dtype=torch.long)
    steps = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        nxt = torch.argmax(logits, dim=-1)
        logits = m.decode_step(nxt, pos)
        pos = pos + 1
        steps += 1
    dt = time.perf_counter() - t0
    return {"value": round(batch * steps / dt, 2), "unit": "tokens/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"{steps} batch-{batch} fp32 decode steps of the oracle after a 16-token prompt, {dt:.1f} s"}


def cpu_baseline(seconds: float):
    """The oracle (numpy) on the host: per-call dequant + fp32 matmul, M=16,
    over the four Qwen3-0.6B shapes in turn, for about ``seconds``."""
    import numpy as np
    from oracle import w4a16 as ow
    from torch2iron_amd.formats import algorithmic_bytes

    try:
        from threadpoolctl import threadpool_info
        cores = max([i.get("num_threads", 1) for i in threadpool_info()] + [1])
    except Exception:  # noqa: BLE001
        cores = os.cpu_count() or 1
    m = 16
    data = []
    for i, (_, k, n) in enumerate(QWEN3_06B):
        qw, qz, sc = ow.synthetic_tensors(k, n, seed=100 + i)
        x = np.random.default_rng(i).standard_normal((m, k)).astype(np.float32)
        data.append((x, qw, qz, sc, algorithmic_bytes(m, k, n)))
    calls, nbytes = 0, 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        x, qw, qz, sc, b = data[calls % len(data)]
        ow.linear(x, qw, qz, sc, accumulate="fp32")
        calls += 1
        nbytes += b
    dt = time.perf_counter() - t0
    # cached dense weights (the reference caches its unpacked weight)
    dense = [(x, ow.dequantize(qw, qz, sc), b) for x, qw, qz, sc, b in data]
    ccalls, cbytes = 0, 0
    t1 = time.perf_counter()
    while time.perf_counter() - t1 < min(seconds, 5.0):
        x, w, b = dense[ccalls % len(dense)]
        _ = x @ w.T
        ccalls += 1
        cbytes += b
    cdt = time.perf_counter() - t1
    return {
        "value": nbytes / dt / 1e12, "unit": "TB/s", "cores": int(cores), "kind": "port",
        "sample": f"{calls} calls of oracle dequant+fp32 matmul (M=16, Qwen3-0.6B shapes in turn) in {dt:.1f} s",
        "cached_weights_value": cbytes / cdt / 1e12,
        "cached_weights_sample": f"{ccalls} fp32 matmuls with cached dense weights in {cdt:.1f} s",
        "cpu_count": os.cpu_count(),
    }


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

    ms = [1, 8, 16, 32, 64]
    log(f"building HBM-cold sweep (pool {args.pool_mb} MB)")
    cold = Sweep(QWEN3_06B, ms, args.pool_mb << 20, dev, seed=1, eager=args.eager)
    log(f"{cold.copies} weight copies, {cold.launches_per_step} launches/step, "
        f"{cold.bytes_per_step / 1e6:.1f} MB/step")
    total_ms, per_group = cold.run(args.steps, args.warmup)
    torch.cuda.synchronize()
    # barrier-equivalent for one process: synchronised on both sides of the timed region
    ms_per_step = total_ms / args.steps
    value = cold.bytes_per_step / (ms_per_step * 1e-3) / 1e12
    avg_launch_us = ms_per_step * 1e3 / cold.launches_per_step
    log(f"HBM-cold sweep: {value:.3f} TB/s, {ms_per_step:.3f} ms/step, avg launch {avg_launch_us:.2f} us")
    floor_us = None
    if not args.eager:
        # the same number of back-to-back graph launches of a one-element fill: what a
        # dependent launch costs on this stream before any kernel does work
        tiny = torch.zeros(1, device=dev)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(cold.launches_per_step):
                tiny.fill_(0.0)
        for _ in range(args.warmup):
            g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        floor_us = e0.elapsed_time(e1) * 1e3 / (args.steps * cold.launches_per_step)
        log(f"launch floor (one-element fill, graph): {floor_us:.2f} us per launch")
        del g, tiny
    breakdown = {}
    for gr, t in zip(cold.groups, per_group):
        breakdown[gr["label"]] = {"TBps": round(gr["bytes"] / (t * 1e-3) / 1e12, 4),
                                  "us_per_launch": round(t * 1e3 / gr["launches"], 3)}

    if args.calibrate_copy:
        src = torch.empty(COPY_BYTES, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    extra = {}
    if not args.skip_extra:
        log("MALL-warm sweep (one weight copy)")
        warm = Sweep(QWEN3_06B, ms, 0, dev, seed=2, reps=cold.copies)
        w_ms, _ = warm.run(args.steps, args.warmup)
        extra["mall_warm_TBps"] = round(warm.bytes_per_step / (w_ms / args.steps * 1e-3) / 1e12, 4)
        del warm
        log("Qwen3-1.7B sweep (HBM-cold)")
        big = Sweep(QWEN3_17B, [1, 16, 64], args.pool_mb << 20, dev, seed=3)
        b_ms, b_groups = big.run(max(2, args.steps // 2), 1)
        extra["qwen3_1_7b_sweep_TBps"] = round(big.bytes_per_step / (b_ms / max(2, args.steps // 2) * 1e-3) / 1e12, 4)
        extra["qwen3_1_7b_breakdown"] = {gr["label"]: round(gr["bytes"] / (t * 1e-3) / 1e12, 4)
                                         for gr, t in zip(big.groups, b_groups)}
        del big
    torch.cuda.synchronize()

    decode = None
    tensors = None
    if not args.skip_decode:
        decode, tensors, _, _ = bench_decode(dev, args.steps, args.warmup, args.prompt, args.new_tokens,
                                             args.batch, [int(v) for v in args.streams.split(",")])
        torch.cuda.synchronize()

    cpu = None
    if not args.skip_cpu:
        log(f"CPU baseline ({args.cpu_seconds:.0f} s)")
        cpu = cpu_baseline(args.cpu_seconds)
        if tensors is not None:
            log(f"CPU decode baseline ({args.cpu_seconds:.0f} s)")
            cpu["decode"] = cpu_decode_baseline(tensors, args.cpu_seconds, args.batch)

    achieved_gbps = value * 1e3
    traffic = measured_traffic()
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
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "W4A16 group-128 linear sweep, Qwen3-0.6B qkv/o_proj/gate_up/down x M in {1,8,16,32,64}, "
                        f"HBM-cold ({cold.copies}-copy weight pool, {cold.copies * cold.per_copy / 1e6:.0f} MB)",
            "weights": "int4 AutoGPTQ (uniform nibbles, fp16 scales U[0.005,0.02])",
            "activations": "bf16 N(0,1)",
            "launches_per_step": cold.launches_per_step,
            "bytes_per_step": cold.bytes_per_step,
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
        },
        "cpu_baseline": cpu,
        "breakdown": breakdown,
        **extra,
        **(decode or {}),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
