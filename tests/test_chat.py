"""Multi-turn conversations with the caches kept between turns (model/chat.rs
`Chat`, at the token level): the oracle's restatement, pinned on the CPU by
the property the reference states for it (the conversation stays in the
caches, so feeding it turn by turn is the same computation as feeding it at
once), and the device's (titania_amd.chat over th_generate) against the
oracle, token for token.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import ref
from titania_amd import QWEN3_0_6B, QWEN3_TINY, InvalidArgument, Sampler, synth
from titania_amd.chat import Chat
from titania_amd.model import Model, State

LOGIT_TOL = 2e-2


def _turns(vocab: int, seed: int, n: int):
    """n (user turn, reply opening) pairs and the closing tokens, seeded."""
    rng = np.random.default_rng(seed)
    turns = [(rng.integers(0, vocab, 9 + 3 * i).astype(np.uint32), rng.integers(0, vocab, 4).astype(np.uint32))
             for i in range(n)]
    end = rng.integers(0, vocab, 2).astype(np.uint32)
    return turns, end


@pytest.fixture(scope="module")
def tiny_ref():
    w = synth.weights(QWEN3_TINY, seed=11, random_gains=True)
    return w, ref.RefModel(QWEN3_TINY, w)


# ---- the oracle (CPU) ----

def test_ref_chat_is_one_forward(tiny_ref):
    """After three turns with stops, the conversation's last logits are those
    of a fresh forward over everything it fed, bit for bit (the oracle's
    results do not depend on how tokens are chunked): so every turn was fed at
    the right positions, and stop tokens were not fed."""
    _, r = tiny_ref
    turns, end = _turns(QWEN3_TINY.vocab_size, 5, 3)
    probe = ref.RefChat(r, 256)
    probe.feed(turns[0][0])
    first = probe.generate(turns[0][1], [QWEN3_TINY.vocab_size], end, 12)  # a stop that never comes
    stop = [int(first[3])]
    chat = ref.RefChat(r, 256)
    fed, hits = [], 0
    for user, opening in turns:
        chat.feed(user)
        reply = chat.generate(opening, stop, end, 12)
        assert 1 <= reply.size <= 12
        assert all(int(t) not in stop for t in reply[:-1])
        stopped = int(reply[-1]) in stop
        hits += stopped
        body = reply[:-1] if stopped else reply
        fed += [*user, *opening, *body, *end]
        assert chat.len == len(fed)
    assert hits >= 1
    fresh = r.forward(r.state(256), np.array(fed, dtype=np.uint32), 0)
    assert np.array_equal(fresh, chat.logits)


def test_ref_chat_first_reply_stops(tiny_ref):
    """The first reply ends at the stop token taken from an unbounded probe,
    at or before the probe's index of it."""
    _, r = tiny_ref
    turns, end = _turns(QWEN3_TINY.vocab_size, 6, 1)
    probe = ref.RefChat(r, 128)
    first = probe.generate(turns[0][1], [QWEN3_TINY.vocab_size], end, 10)
    chat = ref.RefChat(r, 128)
    reply = chat.generate(turns[0][1], [int(first[5])], end, 10)
    k = next(i for i, t in enumerate(first) if int(t) == int(first[5]))
    assert reply.tolist() == first[: k + 1].tolist()
    assert chat.len == turns[0][1].size + k + end.size


# ---- the device against the oracle ----

def _conversation(m, r, cfg, seed, stops_from, n_turns, max_tokens, sampler_args=None, kv_len=384):
    turns, end = _turns(cfg.vocab_size, seed, n_turns)
    probe = ref.RefChat(r, kv_len, ref.Sampler(*sampler_args) if sampler_args else None)
    probe.feed(turns[0][0])
    first = probe.generate(turns[0][1], [cfg.vocab_size], end, max_tokens)  # a stop that never comes
    stop = [int(first[i]) for i in stops_from if i < first.size]
    exp = ref.RefChat(r, kv_len, ref.Sampler(*sampler_args) if sampler_args else None)
    dev_sampler = Sampler(*sampler_args) if sampler_args else None
    got = Chat(m, kv_len, dev_sampler)
    hits = 0
    for user, opening in turns:
        exp.feed(user)
        got.feed(user)
        e = exp.generate(opening, stop, end, max_tokens)
        g = got.generate(opening, stop, end, max_tokens)
        assert g.tolist() == e.tolist()
        assert got.tokens() == exp.len
        hits += int(e[-1]) in stop
    assert hits >= 1  # the stops were reached, not only the bound
    if sampler_args:
        assert dev_sampler.rng == exp.sampler.state
    # The caches hold the conversation: one more token gives the oracle's logits.
    nxt = np.array([7], dtype=np.uint32)
    logits = m.forward(got.state, nxt, got.tokens())
    exp_logits = r.forward(exp.state, nxt, exp.len)
    assert float(np.max(np.abs(logits - exp_logits))) <= LOGIT_TOL
    got.close()


@pytest.fixture(scope="module")
def tiny_dev(hip, tiny_ref):
    w, r = tiny_ref
    m = Model(hip, QWEN3_TINY, w)
    yield m, r
    m.close()


@pytest.mark.gpu
def test_chat_greedy(tiny_dev):
    m, r = tiny_dev
    _conversation(m, r, QWEN3_TINY, seed=1, stops_from=(3, 9), n_turns=3, max_tokens=16)


@pytest.mark.gpu
@pytest.mark.parametrize("t,k,p,seed", [(0.8, 20, 0.9, 3), (1.2, 256, 1.0, 99)])
def test_chat_sampled(tiny_dev, t, k, p, seed):
    m, r = tiny_dev
    _conversation(m, r, QWEN3_TINY, seed=2, stops_from=(2, 5, 8), n_turns=3, max_tokens=14,
                  sampler_args=(t, k, p, seed))


@pytest.mark.gpu
def test_chat_qwen06(hip):
    """Qwen3-0.6B shape (the fused decode step): two greedy turns."""
    w = synth.weights(QWEN3_0_6B, seed=0)
    m = Model(hip, QWEN3_0_6B, w)
    r = ref.RefModel(QWEN3_0_6B, w)
    _conversation(m, r, QWEN3_0_6B, seed=4, stops_from=(2, 4), n_turns=2, max_tokens=8, kv_len=128)
    m.close()


@pytest.mark.gpu
def test_generate_edges(tiny_dev):
    """A stop at the first pick feeds nothing; a stop one past the bound is not
    reached (every returned token fed); bad stop lists are refused."""
    m, r = tiny_dev
    cfg = QWEN3_TINY
    prompt = synth.prompt(12, cfg.vocab_size, seed=18)  # greedy: 165, then 718 (margins > 0.2)
    rtoks, _, _ = r.generate(r.state(64), prompt, 6)

    st = State(m, 64)
    m.forward(st, prompt, 0, want_logits=False)
    toks = m.decode_until(st, 12, 10, [int(rtoks[0])])
    assert toks.tolist() == [int(rtoks[0])]
    # Nothing was fed: the same call again gives the same pick.
    assert m.decode_until(st, 12, 10, [int(rtoks[0])]).tolist() == [int(rtoks[0])]
    # Token j (its first occurrence) as the stop, with room for j: not
    # reached, all j fed; the next call picks it first.
    j = next(j for j in range(1, 6) if int(rtoks[j]) not in rtoks[:j].tolist())
    toks = m.decode_until(st, 12, j, [int(rtoks[j])])
    assert toks.tolist() == rtoks[:j].tolist()
    toks = m.decode_until(st, 12 + j, 3, [int(rtoks[j])])
    assert toks.tolist() == [int(rtoks[j])]
    for bad in ([], list(range(9)), [cfg.vocab_size]):
        with pytest.raises(InvalidArgument):
            m.decode_until(st, 12, 4, bad)
    st.close()
