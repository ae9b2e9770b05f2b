"""Full-size greedy decode against the oracle: random-init Qwen3-0.6B (28 layers,
hidden 1024, intermediate 3072, vocab 151936, W4A16 group-128 linears, bf16 tied
lm_head), batch 16, 512-token prompts, 32 greedy tokens.

The fp32 oracle's tokens, top-2 margins and bf16 logit noise come from
``tests/golden/qwen3_0.6b_greedy.npz`` (written by ``make_qwen3_greedy_golden.py``
from the same seeds), so the 28-layer fp32 model does not run here.  Three weight
draws are checked: ``uniform`` (the benchmark's draw, which collapses onto a couple
of tokens, so every token must match), ``centered`` (diverse tokens, chaotic under
bf16 rounding) and ``hubs`` (diverse tokens -- 2 to 32 distinct per sequence over 32
steps, median 10 -- with 326 of 512 steps clear of near-ties: the bf16-mode oracle
keeps 8 of 16 sequences on all 32 steps; the GPU, which rounds at the same points
with its own fp32 summation order, must keep at least one fewer, every divergence
must be a near-tie, and teacher-forced it must match every one of the 326 clear
steps).

Bars, per sequence, against the fp32 oracle (the reference runtime's default dtype):
* the sequences that match all 32 tokens are counted and reported, and must reach
  the floor written per draw below (all 16 for the uniform draw);
* the tokens matched before each sequence's first divergence, summed over the
  batch, reach at least half of what the bf16-mode oracle's own greedy tokens
  match (its rounding is as legitimate as the GPU's, and this is the scale of
  agreement bf16 compute allows);
* a sequence that diverges does so at a near-tie: the fp32 top-2 margin at its
  first differing step is at most twice the logit shift that bf16 rounding itself
  causes there (the oracle's bf16 mode against its fp32 mode, teacher-forced along
  the same tokens);
* along the oracle's tokens (teacher forcing), where nothing compounds from step
  to step, the GPU's top-1 token equals the fp32 oracle's at every step that is
  not a near-tie, and at least as often overall as the bf16-mode oracle's does,
  less 5 points;
* along the same tokens the GPU logits sit no farther from the fp32 logits (RMS
  over 8 steps x 512 vocabulary entries x 16 sequences) than the bf16-mode
  oracle's do, within 25 %.

The centered draw is chaotic under bf16 rounding: the bf16-mode oracle's own
greedy tokens match its fp32 mode on all 32 steps for only 3 of the 16 sequences
(first divergences 1-21 steps in the others, 197 matched steps of 512), and a
change of fp32 summation order alone moves the GPU between 0 and 1 such
sequences, so its exact-match floor is 0; the matched-prefix, near-tie and
teacher-forced checks carry the weight there.
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from torch2iron_amd import model as gm

pytestmark = pytest.mark.gpu
FIXTURE = Path(__file__).resolve().parent / "golden" / "qwen3_0.6b_greedy.npz"
DRAWS = {"uniform": 0, "centered": 1, "hubs": 1}
# sequences (of 16) that must match the fp32 oracle on all 32 steps; None: the
# bf16-mode oracle's own count less one (which near-ties flip is chance; at the
# first run the GPU kept 7 and the bf16-mode oracle 8)
EXACT_FLOOR = {"uniform": 16, "centered": 0, "hubs": None}


@pytest.fixture(scope="module")
def golden():
    with np.load(FIXTURE) as f:
        return {k: f[k] for k in f.files}


@pytest.mark.parametrize("draw", list(DRAWS))
def test_full_model_greedy_matches_oracle(gpu, golden, draw):
    cfg = gm.QWEN3_0_6B
    print(f"full Qwen3-0.6B greedy parity, {draw} weights (seed {DRAWS[draw]}), batch 16, prompt 512", flush=True)
    t = gm.random_qwen3_tensors(cfg, seed=DRAWS[draw], weights=draw)
    check = np.array([float(np.asarray(t["model.embed_tokens.weight"], dtype=np.float64).sum()),
                      float(t["model.layers.0.self_attn.q_proj.qweight"].astype(np.int64).sum()),
                      float(t["model.layers.27.mlp.down_proj.scales"].astype(np.float64).sum())])
    assert np.array_equal(check, golden[f"{draw}_check"]), "regenerated weights differ from the fixture's"
    prompt = torch.from_numpy(golden["prompt"]).to(torch.int64)
    b, plen = prompt.shape
    new = golden[f"{draw}_tokens"].shape[1]
    model = gm.Qwen3Model(t, cfg, batch=b, ctx_cap=plen + new, device=gpu)
    del t
    got = model.generate(prompt, new).numpy()
    ref = golden[f"{draw}_tokens"]
    margins, noise = golden[f"{draw}_margins"], golden[f"{draw}_noise"]
    exact = int((got == ref).all(axis=1).sum())
    steps_matched = [int(np.argmin(got[i] == ref[i])) if (got[i] != ref[i]).any() else new for i in range(b)]
    print(f"{draw}: {exact}/{b} sequences match the fp32 oracle on all {new} steps; "
          f"first divergence per sequence {steps_matched}", flush=True)
    for i in range(b):
        s = steps_matched[i]
        if s < new:
            assert margins[i, s] <= 2.0 * noise[i, s], \
                f"sequence {i} step {s}: margin {margins[i, s]:.3f} > 2 x bf16 noise {noise[i, s]:.3f}"
    t16 = golden[f"{draw}_tokens16"]
    exact16 = int((t16 == ref).all(axis=1).sum())
    floor = exact16 - 1 if EXACT_FLOOR[draw] is None else EXACT_FLOOR[draw]
    distinct = [len(np.unique(r)) for r in ref]
    print(f"{draw}: {exact}/{b} sequences exact (bf16-mode oracle {exact16}/{b}; floor {floor}); distinct tokens "
          f"per sequence min {min(distinct)} median {int(np.median(distinct))}", flush=True)
    assert exact >= floor, f"{exact} < {floor} sequences match all {new} steps"

    prefix16 = sum(int(np.argmin(t16[i] == ref[i])) if (t16[i] != ref[i]).any() else new for i in range(b))
    print(f"{draw}: {sum(steps_matched)} steps matched before the first divergence (bf16-mode oracle {prefix16})",
          flush=True)
    assert sum(steps_matched) >= 0.5 * prefix16

    # logits along the oracle's tokens (teacher forcing), on the fixture's vocabulary sample
    sub_steps = [int(s) for s in golden["sub_steps"]]
    vidx = torch.from_numpy(golden["vidx"]).to(torch.int64)
    model.reset()
    lg = model.prefill(prompt, want_logits=True)
    rows, top1 = {0: lg.cpu()[:, vidx]}, [lg.argmax(dim=-1).cpu()]
    for j in range(1, new):
        _, lg = model.decode_step(torch.from_numpy(ref[:, j - 1]), torch.full((b,), plen + j - 1), want_logits=True)
        top1.append(lg.argmax(dim=-1).cpu())
        if j in sub_steps:
            rows[j] = lg.cpu()[:, vidx]
    top1 = torch.stack(top1, dim=1).numpy()
    agree = float((top1 == ref).mean())
    agree16 = float((golden[f"{draw}_tf16_top1"] == ref).mean())
    clear = margins > 2.0 * noise
    print(f"{draw}: teacher-forced top-1 agreement with the fp32 oracle {agree:.3f} (bf16-mode oracle "
          f"{agree16:.3f}); {int(clear.sum())} of {clear.size} steps are not near-ties", flush=True)
    assert (top1 == ref)[clear].all(), "the GPU's top-1 differs from the fp32 oracle's at a step that is not a near-tie"
    assert agree >= agree16 - 0.05
    gpu_sub = torch.stack([rows[s] for s in sub_steps], dim=1)
    ref_sub = torch.from_numpy(golden[f"{draw}_sub"])
    rms_gpu = (gpu_sub - ref_sub).pow(2).mean().sqrt().item()
    rms16 = float(golden[f"{draw}_rms16"])
    print(f"{draw}: logit RMS vs fp32 oracle {rms_gpu:.4f} (bf16-mode oracle {rms16:.4f}, "
          f"logit std {ref_sub.std().item():.2f})", flush=True)
    assert rms_gpu <= 1.25 * rms16
