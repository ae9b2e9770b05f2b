"""Write the full-size greedy-decode fixture (``qwen3_0.6b_greedy.npz``).

Random-init Qwen3-0.6B (28 layers, hidden 1024, intermediate 3072, vocab
151936, W4A16 group-128 linears, bf16 tied lm_head), batch 16, a 512-token
prompt of uniform random ids, 32 greedy tokens: the oracle's tokens and the
statistics the GPU test needs, so that the GPU box does not have to run a
28-layer fp32 model on its host cores.

For each weight draw (``uniform``: seed 0, the draw the benchmark decodes;
``centered``: seed 1, zero point 8 and nibbles 1..15, which does not collapse
onto one token; ``hubs``: seed 1, the centred linears with large log-normal
embedding rows, final-norm weights of random sign and small q/k norm weights,
whose tokens are diverse and less disturbed by bf16 rounding) the fixture holds:

* ``{draw}_tokens``   int32 [16, 32]  fp32-oracle greedy tokens (the reference
                      runtime's default compute dtype);
* ``{draw}_margins``  fp32 [16, 32]   top-1 minus top-2 logit at each step;
* ``{draw}_noise``    fp32 [16, 32]   largest |bf16-mode - fp32-mode| logit
                      difference at each step along the fp32 tokens (teacher
                      forced): the logit shift bf16 rounding itself causes;
* ``{draw}_tokens16`` int32 [16, 32]  the bf16-mode oracle's own greedy tokens;
* ``{draw}_tf16_top1`` int32 [16, 32] the bf16-mode oracle's top-1 token at each
                      step when teacher-forced along the fp32 tokens;
* ``{draw}_sub``      fp32 [16, 8, 512] fp32 logits at steps 0, 4, .., 28 for
                      the vocabulary entries ``vidx``;
* ``{draw}_rms16``    fp32 scalar      RMS of bf16-mode minus fp32-mode logits
                      over the same entries and steps;
* ``{draw}_check``    fp64 [3]         sums of a few weight tensors, to confirm
                      that the GPU test regenerates the same weights.

The prompt (seed 7, as the benchmark) is stored as ``prompt``.

Run: ``python tests/golden/make_qwen3_greedy_golden.py [draw ...]`` (about two
and a half minutes a draw on 8 cores, 10 GB of memory).  It rewrites the .npz next
to it, recomputing the named draws (default: all) and keeping the others' entries.
"""

from __future__ import annotations

import sys
import time
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

from oracle import qwen3 as oq  # noqa: E402
from torch2iron_amd import model as gm  # noqa: E402

OUT = Path(__file__).resolve().parent / "qwen3_0.6b_greedy.npz"
BATCH, PROMPT, NEW = 16, 512, 32
SUB_STEPS = list(range(0, NEW, 4))
DRAWS = {"uniform": 0, "centered": 1, "hubs": 1}


def weight_check(t: dict) -> np.ndarray:
    return np.array([float(np.asarray(t["model.embed_tokens.weight"], dtype=np.float64).sum()),
                     float(t["model.layers.0.self_attn.q_proj.qweight"].astype(np.int64).sum()),
                     float(t["model.layers.27.mlp.down_proj.scales"].astype(np.float64).sum())])


def path_logits(model: oq.DenseQwen3, prompt: torch.Tensor, forced: torch.Tensor | None):
    """Logits [B, NEW, V] along the greedy path (forced=None) or along ``forced``."""
    b, t = prompt.shape
    logits = model.prefill(prompt)
    out, toks = [], []
    pos = torch.full((b,), t, dtype=torch.long)
    for s in range(NEW):
        out.append(logits.clone())
        nxt = torch.argmax(logits, dim=-1) if forced is None else forced[:, s]
        toks.append(torch.argmax(logits, dim=-1))
        if s + 1 == NEW:
            break
        logits = model.decode_step(nxt, pos)
        pos = pos + 1
    return torch.stack(out, dim=1), torch.stack(toks, dim=1)


def main():
    torch.set_num_threads(max(1, torch.get_num_threads()))
    cfg = gm.QWEN3_0_6B
    ocfg = oq.Qwen3Config(**{k: getattr(cfg, k) for k in oq.Qwen3Config.__dataclass_fields__})
    prompt = torch.randint(0, cfg.vocab, (BATCH, PROMPT), generator=torch.Generator().manual_seed(7))
    vidx = np.sort(np.random.default_rng(99).choice(cfg.vocab, 512, replace=False)).astype(np.int64)
    data = {}
    if OUT.exists():
        with np.load(OUT) as f:
            data = {k: f[k] for k in f.files}
        if not np.array_equal(data["prompt"], prompt.numpy().astype(np.int32)):
            data = {}
    data.update({"prompt": prompt.numpy().astype(np.int32), "vidx": vidx, "sub_steps": np.array(SUB_STEPS)})
    cap = PROMPT + NEW
    todo = sys.argv[1:] or list(DRAWS)
    for draw in todo:
        seed = DRAWS[draw]
        t0 = time.time()
        tensors = gm.random_qwen3_tensors(cfg, seed=seed, weights=draw)
        data[f"{draw}_check"] = weight_check(tensors)
        o32 = oq.DenseQwen3(tensors, ocfg, mode="fp32", ctx_cap=cap)
        l32, tok32 = path_logits(o32, prompt, None)
        del o32
        o16 = oq.DenseQwen3(tensors, ocfg, mode="bf16", ctx_cap=cap)
        l16, tf16 = path_logits(o16, prompt, tok32)
        _, tok16 = path_logits(o16, prompt, None)
        del o16, tensors
        top2 = torch.topk(l32, 2, dim=-1).values
        data[f"{draw}_tokens"] = tok32.numpy().astype(np.int32)
        data[f"{draw}_margins"] = (top2[..., 0] - top2[..., 1]).numpy().astype(np.float32)
        data[f"{draw}_noise"] = (l16 - l32).abs().amax(dim=-1).numpy().astype(np.float32)
        data[f"{draw}_tokens16"] = tok16.numpy().astype(np.int32)
        data[f"{draw}_tf16_top1"] = tf16.numpy().astype(np.int32)
        sub32 = l32[:, SUB_STEPS][..., vidx]
        sub16 = l16[:, SUB_STEPS][..., vidx]
        data[f"{draw}_sub"] = sub32.numpy().astype(np.float32)
        data[f"{draw}_rms16"] = np.float32((sub16 - sub32).pow(2).mean().sqrt().item())
        full = (tok16 == tok32).all(dim=1).sum().item()
        print(f"{draw}: {time.time() - t0:.0f} s; bf16-mode oracle matches fp32 on all {NEW} steps for "
              f"{full}/{BATCH} sequences; teacher-forced top-1 agreement "
              f"{(tf16 == tok32).float().mean().item():.3f}; distinct tokens {len(np.unique(tok32.numpy()))}; "
              f"rms16 {float(data[f'{draw}_rms16']):.4f}; logit std {l32.std().item():.3f}", flush=True)
        del l32, l16
    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
