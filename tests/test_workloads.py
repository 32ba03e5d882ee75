"""Whole workloads against the CPU oracle (model/model.rs:83-149 with the
greedy pick of model/sampler.rs:21-33, restated in oracle/cpu_ref.c).

- The Qwen3-0.6B prefill workload: a 512-token uniform prompt through the
  fused (MFMA) prefill, then 128 greedy decode steps, f32 caches.
- A Qwen3-4B-shaped model of reduced depth (hidden 2560, 32 / 8 heads,
  head_dim 128, MLP 9728, vocab 151936, q/k-norm): every kernel variant that
  exists only at those shapes (GEMV rows of 5 and 19 chunks a lane, the
  group-of-4 q/k/v + attention launch, the 151936 x 2560 output projection)
  meets the oracle, not another device path.
- Group sizes 1, 4 and 8 of query heads per KV head in the captured decode
  step (the 0.6B shape has 2).

Bars: logits within 2e-2 max-abs of the oracle's (measured errors are printed;
with f32 caches they are ~1e-4), and identical greedy token streams.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import ref
from titania_amd import QWEN3_0_6B, QWEN3_4B, TH_KV_F32, TH_PATH_FUSED, synth
from titania_amd.config import Config
from titania_amd.model import Model, State
from util import load_fixture

pytestmark = pytest.mark.gpu

LOGIT_TOL = 2e-2


def oracle_greedy(r: ref.RefModel, prompt, steps: int, max_len: int):
    """The oracle's prompt logits, greedy tokens, top-2 gaps of the logits each
    token was picked from, and the logits after the last fed token."""
    st = r.state(max_len)
    logits = r.forward(st, prompt, 0)
    first = logits.copy()
    toks, gaps = [], []
    for i in range(steps):
        t = ref.argmax(logits)
        s = np.sort(logits)
        toks.append(t)
        gaps.append(float(s[-1] - s[-2]))
        logits = r.forward(st, [t], len(prompt) + i)
    return first, np.array(toks, np.uint32), np.array(gaps), logits


def check_workload(hip, cfg: Config, seed: int, n_prompt: int, steps: int, what: str, split: int = 0):
    """The oracle against the fused forward of the prompt (in two calls, the
    second at position `split`, when split > 0) and the captured decode."""
    w = synth.weights(cfg, seed=seed)
    r = ref.RefModel(cfg, w)
    prompt = synth.prompt(n_prompt, cfg.vocab_size, seed=seed + 1)
    first, rtoks, gaps, last = oracle_greedy(r, prompt, steps, n_prompt + steps)
    m = Model(hip, cfg, w)
    st = State(m, n_prompt + steps, TH_KV_F32)
    if split:
        m.forward(st, prompt[:split], 0, TH_PATH_FUSED, want_logits=False)
        got = m.forward(st, prompt[split:], split, TH_PATH_FUSED)
    else:
        got = m.forward(st, prompt, 0, TH_PATH_FUSED)
    toks, logits = m.decode(st, n_prompt, steps, keep_logits=True)
    st.close()
    m.close()
    # The run is not vacuous: the logits spread and several tokens come out.
    assert 0.3 < float(np.std(first)) < 3.0
    assert len(set(rtoks.tolist())) >= 2
    e_prompt = float(np.max(np.abs(got - first)))
    e_last = float(np.max(np.abs(logits[-1] - last)))
    print(f"{what}: prompt logits max |d| = {e_prompt:.2e}, after {steps} steps {e_last:.2e}; "
          f"smallest top-2 gap {gaps.min():.2e}")
    assert e_prompt <= LOGIT_TOL
    assert e_last <= LOGIT_TOL
    first_diff = next((i for i in range(steps) if toks[i] != rtoks[i]), None)
    assert first_diff is None, (first_diff, gaps[first_diff])


def test_qwen06_prefill512_greedy128(hip):
    """Qwen3-0.6B shape: a 512-token uniform prompt (one fused MFMA prefill
    chunk), then 128 greedy steps (contexts 512..639: ten 64-position
    attention chunks a head in the captured step)."""
    check_workload(hip, QWEN3_0_6B, seed=4, n_prompt=512, steps=128, what="qwen3-0.6b 512+128")


def test_qwen06_two_chunk_prefill(hip):
    """Two layers of the Qwen3-0.6B shape, a 2600-token prompt fed in two
    forward calls, the second at positions 2048.. (its attention reads the
    first call's keys and values through the planes), then 8 greedy steps on
    the split attention path (2608 positions: more than the 16 chunks a head
    a step gives the fused launch)."""
    check_workload(hip, QWEN3_0_6B.with_layers(2), seed=12, n_prompt=2600, steps=8, what="qwen3-0.6b x2 2600+8",
                   split=2048)


def test_qwen4b_shape_reduced_depth(hip):
    """Three layers of the Qwen3-4B shape, a 600-token prompt, 32 greedy steps."""
    check_workload(hip, QWEN3_4B.with_layers(3), seed=9, n_prompt=600, steps=32, what="qwen3-4b x3 600+32")


def test_qwen4b_split_attention_decode(hip):
    """Three layers of the Qwen3-4B shape, a 2600-token prompt fed as 2048 +
    552 tokens, then 16 greedy steps. Past 1024 f32 positions at 32 q heads
    the captured step leaves the fused q/k/v + attention launch for the
    split attention (the register kernel with groups of 4 q heads, one split
    per 64 positions: 41 splits) and its combine, the launches of the 8K
    workload of this shape."""
    check_workload(hip, QWEN3_4B.with_layers(3), seed=31, n_prompt=2600, steps=16, what="qwen3-4b x3 2600+16",
                   split=2048)


# Small models with 1, 4 and 8 query heads per KV head.
GROUPS = {
    1: Config(hidden_size=512, intermediate_size=1536, num_hidden_layers=2, num_attention_heads=4,
              num_key_value_heads=4, vocab_size=1000, head_dim_=128),
    4: Config(hidden_size=1024, intermediate_size=2048, num_hidden_layers=2, num_attention_heads=8,
              num_key_value_heads=2, vocab_size=1000, head_dim_=128),
    8: Config(hidden_size=1024, intermediate_size=1536, num_hidden_layers=2, num_attention_heads=8,
              num_key_value_heads=1, vocab_size=1000, head_dim_=128),
}


@pytest.mark.parametrize("group", sorted(GROUPS))
@pytest.mark.parametrize("n_prompt,steps", [(9, 20), (200, 12), (1100, 6)])
def test_group_sizes_greedy(hip, group, n_prompt, steps):
    """The captured decode step at 1, 4 and 8 query heads per KV head, f32
    caches, against the oracle: logits within 1e-4, identical tokens. Groups
    of 1 and 8 take the split attention kernel; at 1100 positions it runs 18
    splits and the combine."""
    cfg = GROUPS[group]
    w = synth.weights(cfg, seed=20 + group, random_gains=True)
    r = ref.RefModel(cfg, w)
    prompt = synth.prompt(n_prompt, cfg.vocab_size, seed=group)
    _, rtoks, gaps, last = oracle_greedy(r, prompt, steps, n_prompt + steps)
    m = Model(hip, cfg, w)
    st = State(m, n_prompt + steps, TH_KV_F32)
    m.forward(st, prompt, 0, TH_PATH_FUSED, want_logits=False)
    toks, logits = m.decode(st, n_prompt, steps, keep_logits=True)
    st.close()
    m.close()
    assert float(np.std(last)) > 0.05
    assert float(np.max(np.abs(logits[-1] - last))) <= 1e-4
    assert list(toks) == list(rtoks) or float(np.min(gaps)) < 1e-4


def test_untied_fixture_decode_logits(hip):
    """The untied transformers fixture (4 query heads per KV head) through the
    captured decode step: the logits after every fed token against
    transformers' own, an implementation independent of the oracle."""
    cfg, meta, tokens, logits = load_fixture("untied")
    w = synth.weights(cfg, seed=meta["seed"], random_gains=meta["random_gains"])
    m = Model(hip, cfg, w)
    p = meta["prompt_len"]
    st = State(m, len(tokens))
    m.forward(st, tokens[:p], 0, TH_PATH_FUSED, want_logits=False)
    toks, got = m.decode(st, p, len(tokens) - p, keep_logits=True)
    st.close()
    m.close()
    assert list(toks) == [int(t) for t in tokens[p:]]
    # got[i] follows the token fed at position p + i, whose logits the fixture holds at p + i.
    for i in range(len(tokens) - p):
        assert float(np.max(np.abs(got[i] - logits[p + i]))) <= 1e-4, f"position {p + i}"
