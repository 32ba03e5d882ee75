"""Writes tests/golden/qwen4b_8k_greedy256.npz: the oracle's greedy run of the
Qwen3-4B-shaped workload at full size, for the GPU test that holds the fused
prefill and the captured decode to it (tests/test_model.py).

Workload: the Qwen3-4B architecture (36 layers, hidden 2560, 32 / 8 heads,
head_dim 128, MLP 9728, vocab 151936, tied, q/k-norm, RoPE theta 1e6) with
synth.weights(seed=0), an 8192-token prompt synth.prompt(8192, 151936,
seed=2), f32 caches, then 256 greedy steps (model/model.rs:83-149 and the
temperature-0 pick of model/sampler.rs:21-33, as oracle/cpu_ref.c restates
them). These are the weights and prompt of bench.py's 4B long-context line.

Stored: the 256 picked tokens, the top-2 gap of the logits each was picked
from, and three logit vectors: after the prompt, after the 128th fed token
and after the 256th (the last step's). About 30 minutes on 8 cores.

Run from the repository root: python tests/golden/make_qwen4b_8k.py
"""

from __future__ import annotations

import json
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import ref  # noqa: E402
from titania_amd import QWEN3_4B, synth  # noqa: E402

OUT = Path(__file__).resolve().parent / "qwen4b_8k_greedy256.npz"
SEED, PROMPT_SEED, N_PROMPT, STEPS, MID = 0, 2, 8192, 256, 128


def main() -> None:
    cfg = QWEN3_4B
    t0 = time.time()
    r = ref.RefModel(cfg, synth.weights(cfg, seed=SEED))
    prompt = synth.prompt(N_PROMPT, cfg.vocab_size, seed=PROMPT_SEED)
    st = r.state(N_PROMPT + STEPS)
    logits = r.forward(st, prompt, 0)
    first = logits.copy()
    print(f"prompt done in {time.time() - t0:.0f} s", flush=True)
    toks = np.empty(STEPS, np.uint32)
    gaps = np.empty(STEPS, np.float32)
    mid = None
    for i in range(STEPS):
        t = ref.argmax(logits)
        s = np.partition(logits, -2)[-2:]
        toks[i] = t
        gaps[i] = abs(float(s[1]) - float(s[0]))
        logits = r.forward(st, [t], N_PROMPT + i)
        if i + 1 == MID:
            mid = logits.copy()
        if (i + 1) % 32 == 0:
            print(f"step {i + 1} of {STEPS} ({time.time() - t0:.0f} s)", flush=True)
    meta = {"model": "qwen3-4b", "seed": SEED, "prompt_seed": PROMPT_SEED, "n_prompt": N_PROMPT, "steps": STEPS,
            "mid": MID, "kv": "f32", "oracle_threads": int(ref.lib().ref_get_threads()),
            "seconds": round(time.time() - t0, 1)}
    np.savez_compressed(OUT, meta=json.dumps(meta), tokens=toks, gaps=gaps, logits_prompt=first,
                        logits_mid=mid, logits_last=logits)
    print(f"wrote {OUT.name}: smallest gap {gaps.min():.3e}, {len(set(toks.tolist()))} distinct tokens", flush=True)


if __name__ == "__main__":
    main()
