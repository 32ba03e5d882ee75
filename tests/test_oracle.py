"""Pins the CPU oracle (oracle/cpu_ref.c) before any GPU result is compared
with it.

Each oracle function is checked against something that does not share its
code: a closed form, an independent numpy emulation of the reference's
summation order (bit-exact), float64 brute force with a rounding bound, torch
float64 ops, Hugging Face transformers' Qwen3 (the committed fixtures under
tests/golden/), or an invariant of the algorithm. The checks are chosen so
that the plausible mistakes fail one of them: a transposed operand, a dropped
tail or gain, a sign or pair-index error in RoPE, a wrong GQA head mapping, a
causal off-by-one, an argmax tie broken the wrong way.

Unpinned at the bit level: glibc's expf/powf/sinf/cosf themselves, which the
reference also calls (through Rust's f32 methods) and which no reference test
holds outputs of; the checks involving them are tolerance-based.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ref
from titania_amd import synth
from titania_amd.config import Config
from util import attention_f64, load_fixture


rng = np.random.default_rng(1234)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    return synth.f32_to_bf16(np.asarray(x, dtype=np.float32))


def bf16_f32(bits: np.ndarray) -> np.ndarray:
    return synth.bf16_to_f32(bits)


# ---- embed (model/cpu.rs:38-47) ----

def test_embed_closed_form():
    dim, rows = 24, 50
    table = rng.integers(0, 1 << 16, size=rows * dim, dtype=np.uint16)
    tokens = [0, 49, 7, 7, 31]
    got = ref.embed(table, dim, tokens)
    exp = (table.reshape(rows, dim)[tokens].astype(np.uint32) << 16).view(np.float32).reshape(-1)
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


# ---- matmul (model/cpu.rs:49-77, dot :163-177) ----

def dot_emulation(w_bits: np.ndarray, x: np.ndarray) -> np.ndarray:
    """The reference dot in numpy float32, row-vectorized: eight interleaved
    sums of rounded products, folded left, plus the tail's products folded
    left."""
    w = bf16_f32(w_bits)
    rows, cols = w.shape
    done = cols // 8 * 8
    acc = np.zeros((rows, 8), dtype=np.float32)
    for c in range(0, done, 8):
        acc = acc + (w[:, c:c + 8] * x[c:c + 8]).astype(np.float32)
    s = acc[:, 0].copy()
    for i in range(1, 8):
        s = s + acc[:, i]
    if done < cols:
        p = (w[:, done:] * x[done:]).astype(np.float32)
        rest = p[:, 0].copy()
        for i in range(1, p.shape[1]):
            rest = rest + p[:, i]
        s = s + rest
    return s


@pytest.mark.parametrize("rows,cols,n", [(7, 13, 1), (33, 1027, 2), (64, 1024, 3), (5, 7, 1), (19, 3072, 1)])
def test_matmul_bit_exact(rows, cols, n):
    w = bf16_bits(rng.standard_normal(rows * cols))
    x = rng.standard_normal(n * cols).astype(np.float32)
    got = ref.matmul(w, rows, cols, x).reshape(n, rows)
    for t in range(n):
        exp = dot_emulation(w.reshape(rows, cols), x[t * cols:(t + 1) * cols])
        assert np.array_equal(got[t].view(np.uint32), exp.view(np.uint32)), f"token {t}"


@pytest.mark.parametrize("rows,cols,n", [(3, 5, 2), (2048, 1024, 1), (1024, 3072, 2), (151, 2560, 1)])
def test_matmul_float64_bound(rows, cols, n):
    """|oracle - exact| <= cols * 2^-23 * sum|w x|: a transposed operand or a
    dropped tail misses by far more."""
    w = bf16_bits(rng.standard_normal(rows * cols))
    x = rng.standard_normal(n * cols).astype(np.float32)
    got = ref.matmul(w, rows, cols, x).reshape(n, rows).astype(np.float64)
    W = bf16_f32(w).reshape(rows, cols).astype(np.float64)
    X = x.reshape(n, cols).astype(np.float64)
    exact = X @ W.T
    bound = cols * 2.0 ** -23 * (np.abs(X) @ np.abs(W).T) + 1e-30
    assert np.all(np.abs(got - exact) <= bound)
    lin = torch.nn.functional.linear(torch.from_numpy(X), torch.from_numpy(W)).numpy()
    assert np.all(np.abs(got - lin) <= bound)


# ---- add, copy (model/cpu.rs:79-83, :34-36) ----

def test_add_and_copy():
    x = rng.standard_normal(100).astype(np.float32)
    y = rng.standard_normal(100).astype(np.float32)
    assert np.array_equal(ref.add(x, y), x + y)
    dst = np.zeros(20, dtype=np.float32)
    src = np.arange(30, dtype=np.float32)
    out = ref.copy(dst, 3, src, 10, 8)
    exp = dst.copy()
    exp[3:11] = src[10:18]
    assert np.array_equal(out, exp)


# ---- rmsnorm (model/cpu.rs:85-94) ----

@pytest.mark.parametrize("rows,dim", [(1, 1024), (3, 128), (16, 128), (2, 2560)])
def test_rmsnorm_torch_float64(rows, dim):
    x = rng.standard_normal(rows * dim).astype(np.float32) * 3
    g_bits = bf16_bits(1 + 0.1 * rng.standard_normal(dim))
    got = ref.rmsnorm(x, g_bits, 1e-6).reshape(rows, dim)
    exp = torch.nn.functional.rms_norm(torch.from_numpy(x.reshape(rows, dim).astype(np.float64)), (dim,),
                                       torch.from_numpy(bf16_f32(g_bits).astype(np.float64)), eps=1e-6).numpy()
    np.testing.assert_allclose(got, exp, rtol=2e-6, atol=1e-7)


def test_rmsnorm_constant_row():
    dim, c, eps = 128, 0.75, 1e-6
    g_bits = bf16_bits(np.linspace(-2, 2, dim))
    got = ref.rmsnorm(np.full(dim, c, dtype=np.float32), g_bits, eps)
    exp = c / np.sqrt(c * c + eps) * bf16_f32(g_bits).astype(np.float64)
    np.testing.assert_allclose(got, exp, rtol=1e-6, atol=1e-7)


# ---- rope_table (model/model.rs:239-250) and rope (model/cpu.rs:96-111) ----

def test_rope_table_closed_form():
    max_len, hd, theta = 300, 128, 1e6
    got = ref.rope_table(max_len, hd, theta).reshape(max_len, hd // 2, 2)
    i = np.arange(hd // 2)
    # freq = 1 / theta^(2i/d) is computed in float32 (within a few ulps of the
    # float64 value) and the angle is the float32 product pos * freq, so the
    # angle may differ from the float64 one by pos * freq * ~3 ulps.
    freq = 1.0 / np.power(theta, 2.0 * i / hd)
    pos = np.arange(max_len, dtype=np.float64)[:, None]
    ang = pos * freq[None, :]
    tol = 2e-7 + pos * freq[None, :] * 3.6e-7
    assert np.all(np.abs(got[:, :, 0] - np.cos(ang)) <= tol)
    assert np.all(np.abs(got[:, :, 1] - np.sin(ang)) <= tol)
    # Position 0 is exactly the identity rotation.
    assert np.all(got[0, :, 0] == 1.0) and np.all(got[0, :, 1] == 0.0)


def test_rope_identity_at_pos0():
    hd, heads = 128, 4
    table = ref.rope_table(8, hd, 1e6)
    x = rng.standard_normal(2 * heads * hd).astype(np.float32)
    # Token 0 sits at position 0 (identity); token 1 at position 1 is rotated.
    out = ref.rope(x, table, 0, heads, hd)
    assert np.array_equal(out[:heads * hd], x[:heads * hd])
    assert not np.array_equal(out[heads * hd:], x[heads * hd:])


@pytest.mark.parametrize("pos", [1, 17, 4095])
def test_rope_rotate_half_float64(pos):
    """Against HF's rotate_half form x*cos + rotate_half(x)*sin in float64 on
    the same table; the pair norms are preserved."""
    hd, heads, n = 128, 3, 2
    table = ref.rope_table(pos + n, hd, 1e6)
    x = rng.standard_normal(n * heads * hd).astype(np.float32)
    got = ref.rope(x, table, pos, heads, hd).reshape(n, heads, hd)
    X = x.reshape(n, heads, hd).astype(np.float64)
    half = hd // 2
    for t in range(n):
        ang = table.reshape(-1, half, 2)[pos + t].astype(np.float64)
        cos = np.concatenate([ang[:, 0], ang[:, 0]])
        sin = np.concatenate([ang[:, 1], ang[:, 1]])
        rot = np.concatenate([-X[t, :, half:], X[t, :, :half]], axis=-1)
        exp = X[t] * cos + rot * sin
        np.testing.assert_allclose(got[t], exp, rtol=1e-6, atol=1e-6)
        norm_in = X[t, :, :half] ** 2 + X[t, :, half:] ** 2
        norm_out = got[t, :, :half].astype(np.float64) ** 2 + got[t, :, half:].astype(np.float64) ** 2
        np.testing.assert_allclose(norm_out, norm_in, rtol=1e-5)


# ---- attention (model/cpu.rs:113-149, softmax :183-193) ----

def attention_float64(q, k, v, pos, n_heads, hd, n_kv):
    """Causal GQA attention in float64 over position-major caches."""
    n = q.size // (n_heads * hd)
    group = n_heads // n_kv
    Q = q.reshape(n, n_heads, hd).astype(np.float64)
    K = k.reshape(-1, n_kv, hd).astype(np.float64)
    V = v.reshape(-1, n_kv, hd).astype(np.float64)
    out = np.zeros((n, n_heads, hd))
    for t in range(n):
        ln = pos + t + 1
        for h in range(n_heads):
            kv = h // group
            s = K[:ln, kv] @ Q[t, h] / np.sqrt(hd)
            p = np.exp(s - s.max())
            p /= p.sum()
            out[t, h] = p @ V[:ln, kv]
    return out.reshape(-1)


@pytest.mark.parametrize("pos,n,heads,kv", [(0, 1, 4, 2), (5, 3, 16, 8), (40, 2, 8, 1), (63, 1, 32, 8)])
def test_attention_float64(pos, n, heads, kv):
    hd = 128
    max_len = pos + n
    q = rng.standard_normal(n * heads * hd).astype(np.float32)
    k = rng.standard_normal(max_len * kv * hd).astype(np.float32)
    v = rng.standard_normal(max_len * kv * hd).astype(np.float32)
    got = ref.attention(q, k, v, pos, heads, hd, kv)
    exp = attention_float64(q, k, v, pos, heads, hd, kv)
    np.testing.assert_allclose(got, exp, rtol=1e-5, atol=2e-6)


@pytest.mark.parametrize("pos,n,heads,kv", [(0, 5, 4, 2), (7, 9, 16, 8), (3, 4, 8, 1)])
def test_attention_f64_helper(pos, n, heads, kv):
    """The vectorised float64 attention the GPU tests use past the oracle's
    sizes (head-major caches with rows past the context) agrees with the
    oracle and with the per-row float64 loop above."""
    hd = 128
    q = rng.standard_normal(n * heads * hd).astype(np.float32)
    kc = rng.standard_normal((kv, pos + n + 3, hd)).astype(np.float32)
    vc = rng.standard_normal((kv, pos + n + 3, hd)).astype(np.float32)
    got = attention_f64(q, kc, vc, pos, heads, kv)
    kp = kc[:, :pos + n].transpose(1, 0, 2).copy()
    vp = vc[:, :pos + n].transpose(1, 0, 2).copy()
    np.testing.assert_allclose(got, attention_float64(q, kp, vp, pos, heads, hd, kv), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(ref.attention(q, kp, vp, pos, heads, hd, kv), got, rtol=1e-5, atol=2e-6)


def test_attention_single_position_is_v():
    hd, heads, kv = 128, 4, 2
    q = rng.standard_normal(heads * hd).astype(np.float32)
    k = rng.standard_normal(kv * hd).astype(np.float32)
    v = rng.standard_normal(kv * hd).astype(np.float32)
    got = ref.attention(q, k, v, 0, heads, hd, kv).reshape(heads, hd)
    vv = v.reshape(kv, hd)
    for h in range(heads):
        assert np.array_equal(got[h], vv[h // 2])


def test_attention_equal_keys_average_values():
    hd, heads, kv, pos = 128, 2, 1, 9
    q = rng.standard_normal(heads * hd).astype(np.float32)
    k = np.tile(rng.standard_normal(hd).astype(np.float32), pos + 1)
    v = rng.standard_normal((pos + 1) * hd).astype(np.float32)
    got = ref.attention(q, k, v, pos, heads, hd, kv).reshape(heads, hd)
    mean = v.reshape(pos + 1, hd).astype(np.float64).mean(axis=0)
    for h in range(heads):
        np.testing.assert_allclose(got[h], mean, rtol=1e-5, atol=1e-6)


# ---- silu_mul (model/cpu.rs:151-155) ----

def test_silu_mul():
    g = (rng.standard_normal(4096) * 6).astype(np.float32)
    u = rng.standard_normal(4096).astype(np.float32)
    got = ref.silu_mul(g, u)
    exp = torch.nn.functional.silu(torch.from_numpy(g.astype(np.float64))).numpy() * u
    np.testing.assert_allclose(got, exp, rtol=2e-6, atol=1e-7)
    zero = ref.silu_mul(np.zeros(8, dtype=np.float32), np.ones(8, dtype=np.float32))
    assert np.all(zero == 0.0)


# ---- greedy pick (model/sampler.rs:21-33 at temperature 0) ----

def total_order_key(x: np.ndarray) -> np.ndarray:
    """f32::total_cmp as a signed integer key."""
    b = x.astype(np.float32).view(np.int32).astype(np.int64)
    return np.where(b < 0, b ^ 0x7FFFFFFF, b)


def argmax_brute(x: np.ndarray) -> int:
    key = total_order_key(x)
    return int(np.nonzero(key == key.max())[0][0])


def test_argmax_brute_force():
    for trial in range(50):
        n = int(rng.integers(1, 3000))
        x = rng.standard_normal(n).astype(np.float32)
        if trial % 3 == 0:  # ties: the lowest index wins
            x[rng.integers(0, n, size=5)] = x.max()
        assert ref.argmax(x) == argmax_brute(x)
    # total_cmp: +0.0 > -0.0, +inf beats every finite value, -inf loses.
    assert ref.argmax(np.array([-0.0, 0.0, -0.0], dtype=np.float32)) == 1
    assert ref.argmax(np.array([-np.inf, -1e30, -np.inf], dtype=np.float32)) == 1
    assert ref.argmax(np.array([3.0, np.inf, np.inf], dtype=np.float32)) == 1


# ---- the forward pass (model/model.rs:83-149) ----

@pytest.mark.parametrize("name", ["tied", "untied"])
def test_forward_matches_transformers(name):
    """Logits at every position against transformers' Qwen3ForCausalLM on the
    same weights, and the fixture's greedy tokens. The two implementations sum
    in different orders, so agreement is to float32 rounding (observed
    ~2e-6 on logits of magnitude ~2)."""
    cfg, meta, tokens, logits = load_fixture(name)
    model = ref.RefModel(cfg, synth.weights(cfg, seed=meta["seed"], random_gains=meta["random_gains"]))
    p = meta["prompt_len"]
    st = model.state(len(tokens))
    got = model.forward(st, tokens[:p], 0)
    assert np.max(np.abs(got - logits[p - 1])) <= 2e-5
    for i in range(p, len(tokens)):
        assert ref.argmax(got) == tokens[i], f"greedy token {i}"
        got = model.forward(st, tokens[i:i + 1], i)
        assert np.max(np.abs(got - logits[i])) <= 2e-5, f"position {i}"


def test_forward_batch_chunking_is_exact():
    """BATCH chunking (model.rs:87-89) does not change any bit: each token's
    arithmetic depends only on the cache, not on its batch."""
    cfg = Config(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
                 num_key_value_heads=2, vocab_size=300, head_dim_=64)
    w = synth.weights(cfg, seed=9, random_gains=True)
    prompt = synth.prompt(23, cfg.vocab_size, seed=9)
    a = ref.RefModel(cfg, w, batch=64)
    b = ref.RefModel(cfg, w, batch=5)
    la = a.forward(a.state(32), prompt, 0)
    lb = b.forward(b.state(32), prompt, 0)
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))


def test_generate_is_the_forward_loop():
    cfg = Config(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
                 num_key_value_heads=1, vocab_size=300, head_dim_=64)
    w = synth.weights(cfg, seed=4)
    prompt = synth.prompt(5, cfg.vocab_size, seed=4)
    m = ref.RefModel(cfg, w)
    toks, gaps, last = m.generate(m.state(16), prompt, 8)
    st = m.state(16)
    lg = m.forward(st, prompt, 0)
    for i in range(8):
        t = ref.argmax(lg)
        assert t == toks[i]
        s = np.sort(lg)
        assert gaps[i] == pytest.approx(float(s[-1] - s[-2]))
        lg = m.forward(st, [t], 5 + i)
    assert np.array_equal(lg, last)



@pytest.mark.parametrize("t,k,p,seed", [(0.7, 20, 0.8, 42), (1.0, 300, 1.0, 7), (0.0, 20, 0.8, 3), (1.3, 5, 0.5, 0)])
def test_generate_sampled_is_the_forward_loop(t, k, p, seed):
    """ref_generate_sampled (the checker of the device's sampled decodes) is
    the loop of RefModel.forward and Sampler.sample that chat.rs:149-178
    runs: each token drawn from the previous forward's logits, then fed at
    the next position; the generator ends in the loop's state."""
    cfg = Config(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
                 num_key_value_heads=2, vocab_size=300, head_dim_=64)
    w = synth.weights(cfg, seed=5, random_gains=True)
    prompt = synth.prompt(6, cfg.vocab_size, seed=5)
    m = ref.RefModel(cfg, w)
    a = ref.Sampler(t, k, p, seed)
    toks = m.generate_sampled(m.state(32), prompt, 12, a)
    b = ref.Sampler(t, k, p, seed)
    st = m.state(32)
    lg = m.forward(st, prompt, 0)
    for i in range(12):
        tok = b.sample(lg)
        assert tok == toks[i], f"token {i}"
        lg = m.forward(st, [tok], len(prompt) + i)
    assert a.state == b.state
    if t > 0:
        assert len(set(toks.tolist())) > 1, "a sampled run that never varies pins little"


def test_ref_chat_sampled_is_the_forward_loop():
    """A sampled RefChat reply is the same loop, stopping at a stop token
    without feeding it; its cache then holds exactly the fed tokens (the next
    turn's logits equal a fresh forward over all of them)."""
    cfg = Config(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
                 num_key_value_heads=2, vocab_size=300, head_dim_=64)
    w = synth.weights(cfg, seed=6, random_gains=True)
    m = ref.RefModel(cfg, w)
    prompt = synth.prompt(5, cfg.vocab_size, seed=6)
    free = ref.Sampler(0.9, 30, 0.9, 11)
    probe = m.generate_sampled(m.state(64), prompt, 20, free)
    stop = [int(probe[9])]  # a token the unbounded run draws
    chat = ref.RefChat(m, 64, ref.Sampler(0.9, 30, 0.9, 11))
    end = [1, 2]
    reply = chat.generate(prompt, stop, end, 40)
    b = ref.Sampler(0.9, 30, 0.9, 11)
    st = m.state(64)
    lg = m.forward(st, prompt, 0)
    fed = list(prompt)
    want = []
    while True:
        tok = b.sample(lg)
        want.append(tok)
        if tok in stop:
            break
        lg = m.forward(st, [tok], len(fed))
        fed.append(tok)
    assert reply.tolist() == want and want[-1] == stop[0] and len(want) <= 10
    assert chat.sampler.state == b.state
    fed += end
    assert chat.len == len(fed)
    fresh = m.forward(m.state(64), fed, 0)
    assert np.array_equal(chat.logits.view(np.uint32), fresh.view(np.uint32))


def _patched_forward(cfg, w, tokens, pos, kc, vc, max_len):
    """run_batch of titania_amd/rust/patches/model-model.rs.patch with the
    default methods of model-device.rs.patch, on the oracle's restatements of
    the cpu.rs primitives (one batch of at most 64 tokens): add_rmsnorm =
    add (when set), copy, rmsnorm; qkv_rope_append = matmul x 3, the q/k
    norms, rope x 2, copy x 2; gate_up_silu = matmul x 2, silu_mul."""
    H, hd, I, V = cfg.hidden_size, cfg.head_dim(), cfg.intermediate_size, cfg.vocab_size
    nh, nkv, eps = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.rms_norm_eps
    qd, kvd, n = nh * hd, nkv * hd, len(tokens)
    table = ref.rope_table(max_len, hd, cfg.rope_theta)

    def t(name):
        return w[name].data

    def add_rmsnorm(x, xb, add, gain):
        if add:
            x = ref.add(x, xb)
        xb = ref.copy(xb, 0, x, 0, n * H)
        return x, ref.rmsnorm(xb, gain, eps)

    x = ref.embed(t("model.embed_tokens.weight"), H, tokens)
    xb = np.zeros(n * H, np.float32)
    for i in range(cfg.num_hidden_layers):
        p = f"model.layers.{i}"
        x, xb = add_rmsnorm(x, xb, i > 0, t(f"{p}.input_layernorm.weight"))
        q = ref.matmul(t(f"{p}.self_attn.q_proj.weight"), qd, H, xb)
        k = ref.matmul(t(f"{p}.self_attn.k_proj.weight"), kvd, H, xb)
        v = ref.matmul(t(f"{p}.self_attn.v_proj.weight"), kvd, H, xb)
        if f"{p}.self_attn.q_norm.weight" in w:
            q = ref.rmsnorm(q, t(f"{p}.self_attn.q_norm.weight"), eps)
        if f"{p}.self_attn.k_norm.weight" in w:
            k = ref.rmsnorm(k, t(f"{p}.self_attn.k_norm.weight"), eps)
        q = ref.rope(q, table, pos, nh, hd)
        k = ref.rope(k, table, pos, nkv, hd)
        kc[i] = ref.copy(kc[i], pos * kvd, k, 0, n * kvd)
        vc[i] = ref.copy(vc[i], pos * kvd, v, 0, n * kvd)
        att = ref.attention(q, kc[i], vc[i], pos, nh, hd, nkv)
        xb = ref.matmul(t(f"{p}.self_attn.o_proj.weight"), H, qd, att)
        x, xb = add_rmsnorm(x, xb, True, t(f"{p}.post_attention_layernorm.weight"))
        g = ref.matmul(t(f"{p}.mlp.gate_proj.weight"), I, H, xb)
        u = ref.matmul(t(f"{p}.mlp.up_proj.weight"), I, H, xb)
        g = ref.silu_mul(g, u)
        xb = ref.matmul(t(f"{p}.mlp.down_proj.weight"), H, I, g)
    if cfg.num_hidden_layers:
        x = ref.add(x, xb)
    last = ref.rmsnorm(ref.copy(np.zeros(H, np.float32), 0, x, (n - 1) * H, H), t("model.norm.weight"), eps)
    head = "model.embed_tokens.weight" if cfg.tie_word_embeddings else "lm_head.weight"
    return ref.matmul(t(head), V, H, last)


@pytest.mark.parametrize("kv_heads,tied", [(2, True), (4, False)])
def test_patched_forward_batch_is_bit_identical(kv_heads, tied):
    """The trait-extension patch keeps the reference device's results bit for
    bit: its forward_batch with the default methods gives exactly the logits
    of the original op order (the oracle's forward), for a prompt and then
    two single-token steps at later positions."""
    cfg = Config(hidden_size=256, intermediate_size=512, num_hidden_layers=3, num_attention_heads=4,
                 num_key_value_heads=kv_heads, vocab_size=300, head_dim_=64, tie_word_embeddings=tied)
    w = synth.weights(cfg, seed=13, random_gains=True)
    m = ref.RefModel(cfg, w)
    max_len = 40
    st = m.state(max_len)
    kvd = kv_heads * 64
    kc = [np.zeros(max_len * kvd, np.float32) for _ in range(cfg.num_hidden_layers)]
    vc = [np.zeros(max_len * kvd, np.float32) for _ in range(cfg.num_hidden_layers)]
    prompt = synth.prompt(23, cfg.vocab_size, seed=13)
    calls = [(list(prompt), 0), ([7], 23), ([201], 24)]
    for toks, pos in calls:
        want = m.forward(st, toks, pos)
        got = _patched_forward(cfg, w, toks, pos, kc, vc, max_len)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"tokens at {pos}"


# ---- sampling (model/sampler.rs) ----

M64 = (1 << 64) - 1


def test_xorshift64star_published_recurrence():
    """The generator against Vigna's xorshift64* (2016): the 64-bit state
    recurrence x ^= x >> 12; x ^= x << 25; x ^= x >> 27 and the output
    x * 2685821657736338717 mod 2^64, in Python integers."""
    for seed in (1, 42, 0xDEADBEEFCAFEF00D):
        x = seed
        state = seed
        for _ in range(1000):
            x ^= x >> 12
            x = (x ^ (x << 25)) & M64
            x ^= x >> 27
            out, state = ref.rng_next_u64(state)
            assert state == x
            assert out == (x * 2685821657736338717) & M64


def test_sampler_seed_zero_is_one():
    """Sampler::new seeds with seed.max(1): seeds 0 and 1 draw alike."""
    logits = rng.standard_normal(500).astype(np.float32)
    a, b = ref.Sampler(1.0, 50, 0.95, 0), ref.Sampler(1.0, 50, 0.95, 1)
    assert [a.sample(logits) for _ in range(50)] == [b.sample(logits) for _ in range(50)]


def test_sampler_greedy_cases_are_argmax():
    """Temperature 0, top_k 1 (and 0, clamped to 1), or a top_p below the
    largest probability all return the argmax, lowest index on ties."""
    logits = rng.standard_normal(3000).astype(np.float32)
    logits[[17, 2900]] = logits.max() + 1.0  # a tie for first place
    best = 17
    for t, k, p in [(0.0, 40, 0.9), (0.8, 1, 0.9), (0.8, 0, 0.9), (1.0, 40, 1e-6)]:
        s = ref.Sampler(t, k, p, 7)
        assert {s.sample(logits) for _ in range(30)} == {best}, (t, k, p)


def _softmax64(x: np.ndarray, t: float) -> np.ndarray:
    z = (x.astype(np.float64) - x.max()) / t
    e = np.exp(z)
    return e / e.sum()


@pytest.mark.parametrize("t,k,p", [(0.7, 8, 1.0), (1.3, 20, 0.8), (0.5, 12, 0.6)])
def test_sampler_frequencies_match_float64(t, k, p):
    """Draw frequencies against the float64 softmax of the top k at the
    temperature, restricted to the shortest prefix whose mass reaches top_p
    and renormalised (the draw scales by that prefix's mass). Tokens outside
    the prefix never appear. Logits are spaced so that no prefix boundary is
    within float32 rounding of top_p."""
    logits = (np.linspace(3.0, -2.0, 400) + rng.uniform(-0.01, 0.01, 400)).astype(np.float32)
    order = rng.permutation(400)
    logits = logits[order]
    top = np.argsort(-logits.astype(np.float64), kind="stable")[:k]
    probs = _softmax64(logits[top], t)
    cum = np.cumsum(probs)
    m = int(np.searchsorted(cum, p, side="left")) + 1 if p < 1.0 else k
    m = min(m, k)
    assert p >= 1.0 or abs(cum[m - 1] - p) > 1e-4
    expected = probs[:m] / probs[:m].sum()
    s = ref.Sampler(t, k, p, 1234)
    n = 20000
    draws = np.array([s.sample(logits) for _ in range(n)])
    allowed = set(int(x) for x in top[:m])
    assert set(np.unique(draws).tolist()) <= allowed
    counts = np.array([(draws == tok).sum() for tok in top[:m]], dtype=np.float64)
    chi2 = float((((counts - n * expected) ** 2) / (n * expected)).sum())
    from scipy.stats import chi2 as chi2_dist
    assert chi2_dist.sf(chi2, m - 1) > 1e-4, (chi2, m)
