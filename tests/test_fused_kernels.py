"""Per-kernel parity of the fused kernels against the oracle's composition of
the reference's primitives (model/cpu.rs, in the order model/model.rs:93-149
calls them), at the Qwen3-0.6B and Qwen3-4B shapes, through the test-only
entry points of include/titania_hip_test.h.

Kernels: the decode step's q/k/v GEMV (residual add + RMSNorm prologue), its
gate/up GEMV (SiLU epilogue), its plain GEMV (o, down; 19 chunks a lane at
the 4B down shape), its output projection (argmax epilogue + pick), its fused
q/k/v + attention launch (q/k norm, RoPE, KV append, chunked attention), its
split attention with the combine (the launches of long contexts); the
prefill's q/k/v GEMM (norm + RoPE + KV append epilogue), gate/up GEMM (SiLU
epilogue) and residual-partials + RMSNorm kernel.

Bar: a per-kernel relative error <= 1e-3 (normwise), and an
elementwise bound of a few fp32 rounding steps of each output's magnitude.
"""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from oracle import ref
from titania_amd import Tensor
from titania_amd._lib import LIB_PATH, check
from titania_amd.synth import bf16_to_f32, f32_to_bf16, normal_bf16
from util import assert_close, attention_f64, rel_error

pytestmark = pytest.mark.gpu

_P, _SZ, _F = C.c_void_p, C.c_size_t, C.c_float
TEST_SIGNATURES = {
    "th_test_step_qkv": [_P, _P, _P, _P, _P, _P, _P, _F, _P, _P],
    "th_test_step_gate_up": [_P, _P, _P, _P, _P, _P, _F, _P, _P],
    "th_test_step_gemv": [_P, _P, _P, _P],
    "th_test_step_logits": [_P, _P, _P, _P, _P, _F, _P, C.POINTER(C.c_uint32)],
    "th_test_step_qkv_attn": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _F, _P, _P, _P, _SZ, _SZ, _SZ, _SZ, _P, _P],
    "th_test_step_attention": [_P, _P, _P, _P, _F, _P, _P, _P, _SZ, _SZ, _SZ, _SZ, C.c_int, _P,
                               C.POINTER(C.c_int)],
    "th_test_gemm_qkv": [_P, _P, _P, _P, _P, _P, _P, _F, _P, _P, _P, _SZ, _SZ, _SZ, _SZ, _SZ, _P, _P],
    "th_test_gemm_silu": [_P, _P, _P, _P, _SZ, _P],
    "th_test_add_rmsnorm_parts": [_P, _P, _P, _SZ, _P, _F, _P],
    "th_test_attention_prefill": [_P, _P, _P, _P, _SZ, _SZ, _SZ, _SZ, _SZ, C.c_int, _P],
}
EPS = 1e-6


@pytest.fixture(scope="module")
def tlib(hip):
    L = C.CDLL(str(LIB_PATH))
    for name, args in TEST_SIGNATURES.items():
        f = getattr(L, name)
        f.restype = C.c_int
        f.argtypes = args
    return L


def h(x):
    """The handle of a buffer the caller keeps alive, or NULL."""
    return None if x is None else x.handle


def weight(hip, rows, cols, seed, name, std=0.05):
    bits = normal_bf16(rows * cols, seed, name, std)
    return bits, hip.upload(Tensor((rows, cols), bits))


def gains(hip, n, seed, name):
    g = f32_to_bf16(1.0 + bf16_to_f32(normal_bf16(n, seed, name, 0.1)))
    return g, hip.upload(Tensor((n,), g))


def buf(hip, values):
    values = np.ascontiguousarray(values, np.float32).reshape(-1)
    b = hip.alloc(values.size)
    hip.write(b, values)
    return b


def gemv_bound(wbits, rows, cols, x):
    """Elementwise bound: a few fp32 rounding steps of sum_c |w x|."""
    w = np.abs(bf16_to_f32(wbits).reshape(rows, cols))
    s = (w @ np.abs(np.asarray(x, np.float32).reshape(-1, cols)).T).T.reshape(-1)
    return 3e-5 * s.astype(np.float64) + 1e-6


def split_sigma(wbits, rows, cols, x):
    """6 standard deviations of sum_c w[r, c] d[c] with d[c] uniform in
    +-2^-17 |x[c]| (x rounded to bf16 hi + lo), per output row and x row."""
    w2 = np.square(bf16_to_f32(wbits).reshape(rows, cols))
    x2 = np.square(np.asarray(x, np.float32).reshape(-1, cols))
    return 6 * 2.0 ** -17 / np.sqrt(3) * np.sqrt((x2 @ w2.T).astype(np.float64)).reshape(-1)


SHAPES = {  # hidden, q heads, kv heads, intermediate
    "0.6b": (1024, 16, 8, 3072),
    "4b": (2560, 32, 8, 9728),
}
# q/k/v with few columns, so that 12288 tokens (768 tiles of 256 x 256, the
# q/k/v GEMM's epilogue in registers) stay quick for the oracle.
NARROW = (256, 16, 8, 1024)


@pytest.mark.parametrize("shape", list(SHAPES))
def test_step_qkv(hip, tlib, shape):
    H, nh, nkv, _ = SHAPES[shape]
    qd, kvd = nh * 128, nkv * 128
    wq, Wq = weight(hip, qd, H, 1, "q")
    wk, Wk = weight(hip, kvd, H, 1, "k")
    wv, Wv = weight(hip, kvd, H, 1, "v")
    g, G = gains(hip, H, 1, "g")
    rng = np.random.default_rng(H)
    x, y = rng.standard_normal(H).astype(np.float32), rng.standard_normal(H).astype(np.float32)
    X, Y, xo, qkv = buf(hip, x), buf(hip, y), hip.alloc(H), hip.alloc(qd + 2 * kvd)
    check(tlib.th_test_step_qkv(hip.handle, Wq.handle, Wk.handle, Wv.handle, X.handle, Y.handle,
                                G.handle, EPS, xo.handle, qkv.handle))
    xs = ref.add(x, y)
    xn = ref.rmsnorm(xs, g, EPS)
    exp = np.concatenate([ref.matmul(wq, qd, H, xn), ref.matmul(wk, kvd, H, xn), ref.matmul(wv, kvd, H, xn)])
    assert np.array_equal(hip.read(xo), xs), "x + y is exact"
    got = hip.read(qkv)
    assert rel_error(got, exp) <= 1e-3
    bound = np.concatenate([gemv_bound(wq, qd, H, xn), gemv_bound(wk, kvd, H, xn), gemv_bound(wv, kvd, H, xn)])
    assert np.all(np.abs(got.astype(np.float64) - exp) <= bound + 1e-5 * np.abs(exp))


@pytest.mark.parametrize("shape", list(SHAPES))
def test_step_gate_up(hip, tlib, shape):
    H, _, _, I = SHAPES[shape]
    wg, Wg = weight(hip, I, H, 2, "gate")
    wu, Wu = weight(hip, I, H, 2, "up")
    g, G = gains(hip, H, 2, "g")
    rng = np.random.default_rng(I)
    x1, o = rng.standard_normal(H).astype(np.float32), rng.standard_normal(H).astype(np.float32)
    X1, O, xo, hh = buf(hip, x1), buf(hip, o), hip.alloc(H), hip.alloc(I)
    check(tlib.th_test_step_gate_up(hip.handle, Wg.handle, Wu.handle, X1.handle, O.handle, G.handle,
                                    EPS, xo.handle, hh.handle))
    xs = ref.add(x1, o)
    n = ref.rmsnorm(xs, g, EPS)
    exp = ref.silu_mul(ref.matmul(wg, I, H, n), ref.matmul(wu, I, H, n))
    assert np.array_equal(hip.read(xo), xs)
    got = hip.read(hh)
    assert rel_error(got, exp) <= 1e-3
    assert_close(got, exp, rel=1e-4, abs_=2e-5, what=f"gate/up {shape}")


@pytest.mark.parametrize("name,rows,cols", [("o 0.6b", 1024, 2048), ("down 0.6b", 1024, 3072),
                                            ("o 4b", 2560, 4096), ("down 4b", 2560, 9728)])
def test_step_gemv(hip, tlib, name, rows, cols):
    w, W = weight(hip, rows, cols, 3, name, std=1.0)
    x = np.random.default_rng(rows + cols).standard_normal(cols).astype(np.float32)
    X, out = buf(hip, x), hip.alloc(rows)
    check(tlib.th_test_step_gemv(hip.handle, W.handle, X.handle, out.handle))
    exp = ref.matmul(w, rows, cols, x)
    got = hip.read(out)
    assert rel_error(got, exp) <= 1e-3
    assert np.all(np.abs(got.astype(np.float64) - exp) <= gemv_bound(w, rows, cols, x))


@pytest.mark.parametrize("shape", list(SHAPES))
def test_step_logits(hip, tlib, shape):
    H = SHAPES[shape][0]
    V = 151936
    w, W = weight(hip, V, H, 4, "lm_head", std=0.02)
    g, G = gains(hip, H, 4, "g")
    rng = np.random.default_rng(V + H)
    x, y = rng.standard_normal(H).astype(np.float32), rng.standard_normal(H).astype(np.float32)
    X, Y, lg = buf(hip, x), buf(hip, y), hip.alloc(V)
    tok = C.c_uint32()
    check(tlib.th_test_step_logits(hip.handle, W.handle, X.handle, Y.handle, G.handle, EPS, lg.handle,
                                   C.byref(tok)))
    xn = ref.rmsnorm(ref.add(x, y), g, EPS)
    exp = ref.matmul(w, V, H, xn)
    got = hip.read(lg)
    assert rel_error(got, exp) <= 1e-3
    assert np.all(np.abs(got.astype(np.float64) - exp) <= gemv_bound(w, V, H, xn))
    # The pick is the argmax of the device's own logits; it is the oracle's
    # unless the oracle's top two are closer than the logits' error.
    assert tok.value == int(np.argmax(got))
    s = np.sort(exp)
    if s[-1] - s[-2] > 1e-4:
        assert tok.value == ref.argmax(exp)


def _head_norm_rope(x, gain, table, pos, n_heads):
    """Per-head RMSNorm then RoPE, as model.rs:111-118 applies them."""
    x = ref.rmsnorm(x, gain, EPS) if gain is not None else np.asarray(x, np.float32)
    return ref.rope(x, table, pos, n_heads, 128)


@pytest.mark.parametrize("shape,pos", [("0.6b", 0), ("0.6b", 47), ("0.6b", 300), ("4b", 5), ("4b", 600),
                                       ("0.6b", 1900), ("0.6b", 2100), ("0.6b", 5000), ("4b", 1100), ("4b", 8300)])
def test_step_qkv_attn(hip, tlib, shape, pos):
    """The fused launch against q/k/v GEMV, per-head norms, RoPE, the cache
    append and the attention over positions 0..pos; 300 and 600 positions
    span several 64-position chunks, merged by each head's first chunk, 1900
    the chunked launch's reach (31 chunks, 496 attention blocks); past 32
    chunks a head (0.6B) or 512 attention blocks (4B), the launch holds the
    streaming split attention instead, merged by the combine."""
    H, nh, nkv, _ = SHAPES[shape]
    hd, qd, kvd = 128, nh * 128, nkv * 128
    max_len = pos + 24
    wq, Wq = weight(hip, qd, H, 5, "q")
    wk, Wk = weight(hip, kvd, H, 5, "k")
    wv, Wv = weight(hip, kvd, H, 5, "v")
    g, G = gains(hip, H, 5, "g")
    qn, QN = gains(hip, hd, 5, "qn")
    kn, KN = gains(hip, hd, 5, "kn")
    rng = np.random.default_rng(pos + H)
    x, y = rng.standard_normal(H).astype(np.float32), rng.standard_normal(H).astype(np.float32)
    table = ref.rope_table(max_len, hd, 1e6)
    # Earlier positions' keys and values, device layout [kv head][max_len][128]
    # plus the tail of 128 rows the attention may read past the last head.
    kc = np.zeros((nkv, max_len, hd), np.float32)
    vc = np.zeros((nkv, max_len, hd), np.float32)
    kc[:, :pos] = rng.standard_normal((nkv, pos, hd))
    vc[:, :pos] = rng.standard_normal((nkv, pos, hd))
    tail = np.zeros(128 * hd, np.float32)
    Kc, Vc = buf(hip, np.concatenate([kc.reshape(-1), tail])), buf(hip, np.concatenate([vc.reshape(-1), tail]))
    X, Y, T, xo, att = buf(hip, x), buf(hip, y), buf(hip, table), hip.alloc(H), hip.alloc(qd)
    check(tlib.th_test_step_qkv_attn(hip.handle, Wq.handle, Wk.handle, Wv.handle, X.handle, Y.handle,
                                     G.handle, QN.handle, KN.handle, EPS, T.handle, Kc.handle, Vc.handle,
                                     max_len, pos, nh, nkv, xo.handle, att.handle))
    xs = ref.add(x, y)
    xn = ref.rmsnorm(xs, g, EPS)
    q = _head_norm_rope(ref.matmul(wq, qd, H, xn), qn, table, pos, nh)
    k = _head_norm_rope(ref.matmul(wk, kvd, H, xn), kn, table, pos, nkv)
    v = ref.matmul(wv, kvd, H, xn)
    kc[:, pos], vc[:, pos] = k.reshape(nkv, hd), v.reshape(nkv, hd)
    # The oracle's caches are position-major: [position][kv head][128].
    exp = ref.attention(q, kc.transpose(1, 0, 2).copy(), vc.transpose(1, 0, 2).copy(), pos, nh, hd, nkv)
    assert np.array_equal(hip.read(xo), xs)
    got = hip.read(att)
    assert rel_error(got, exp) <= 1e-3
    assert_close(got, exp, rel=1e-4, abs_=1e-5, what=f"qkv+attention {shape} pos {pos}")
    dk = hip.read(Kc)[: nkv * max_len * hd].reshape(nkv, max_len, hd)
    dv = hip.read(Vc)[: nkv * max_len * hd].reshape(nkv, max_len, hd)
    assert_close(dk[:, pos], kc[:, pos], rel=1e-4, abs_=1e-5, what="appended key")
    assert_close(dv[:, pos], vc[:, pos], rel=1e-4, abs_=1e-5, what="appended value")
    assert np.array_equal(dk[:, :pos], kc[:, :pos]), "earlier keys untouched"


# (q heads, KV heads, context, max_len, bf16 cache): group sizes 1, 2, 4 and 8
# (the LDS-staged kernel for 1 and 8, the register kernel for 2 and 4) at
# contexts of one split (512 positions) to the 256-split cap (32768 f32
# positions take 256 splits of 128), ragged last splits and empty ones.
SPLIT_CASES = [
    (8, 8, 2049, 2049, 0), (8, 8, 4096, 4200, 0), (8, 8, 2049, 2100, 1),
    (16, 8, 500, 512, 0), (16, 8, 2049, 2049, 0), (16, 8, 4096, 4096, 0), (16, 8, 32768, 32768, 0),
    (16, 8, 4096, 4160, 1), (16, 8, 32768, 32768, 1),
    (32, 8, 1025, 1025, 0), (32, 8, 2049, 2080, 0), (32, 8, 8193, 8193, 0), (32, 8, 8448, 8448, 0),
    (32, 8, 3000, 8448, 0), (32, 8, 8448, 8448, 1), (32, 8, 1025, 1100, 1),
    (64, 8, 1025, 1025, 0), (64, 8, 8193, 8200, 0), (64, 8, 2049, 2049, 1),
]


@pytest.mark.parametrize("nh,nkv,ctx,max_len,kv_bf16", SPLIT_CASES)
def test_step_attention_split(hip, tlib, nh, nkv, ctx, max_len, kv_bf16):
    """The decode step's split attention + combine against per-head norms,
    RoPE, the cache append and the oracle's attention over positions 0..pos
    (pos = ctx - 1). With a bf16 cache the oracle attends over the bf16
    values of the earlier rows and the f32 new key and value (the kernel
    attends to the new row from registers and stores it rounded)."""
    hd, qd, kvd = 128, nh * 128, nkv * 128
    pos = ctx - 1
    qn, QN = gains(hip, hd, 9, "qn")
    kn, KN = gains(hip, hd, 9, "kn")
    rng = np.random.default_rng(ctx + 7 * nh + kv_bf16)
    qkv = rng.standard_normal(qd + 2 * kvd).astype(np.float32)
    table = ref.rope_table(max_len, hd, 1e6)
    kc = np.zeros((nkv, max_len, hd), np.float32)
    vc = np.zeros((nkv, max_len, hd), np.float32)
    kc[:, :pos] = rng.standard_normal((nkv, pos, hd))
    vc[:, :pos] = rng.standard_normal((nkv, pos, hd))
    tail = np.zeros(128 * hd, np.float32)
    if kv_bf16:
        # Two bf16 values a float; rows past pos hold NaN, which a read of
        # them would carry to the output.
        kb, vb = f32_to_bf16(kc), f32_to_bf16(vc)
        kb[:, pos:], vb[:, pos:] = 0x7FC0, 0x7FC0
        kc[:, :pos], vc[:, :pos] = bf16_to_f32(kb[:, :pos]), bf16_to_f32(vb[:, :pos])
        dev_k = np.concatenate([kb.reshape(-1).view(np.float32), tail])
        dev_v = np.concatenate([vb.reshape(-1).view(np.float32), tail])
    else:
        kn_ = np.full_like(kc, np.nan)
        vn_ = np.full_like(vc, np.nan)
        kn_[:, :pos], vn_[:, :pos] = kc[:, :pos], vc[:, :pos]
        dev_k, dev_v = np.concatenate([kn_.reshape(-1), tail]), np.concatenate([vn_.reshape(-1), tail])
    Kc, Vc = buf(hip, dev_k), buf(hip, dev_v)
    QKV, T, att = buf(hip, qkv), buf(hip, table), hip.alloc(qd)
    ns = C.c_int()
    check(tlib.th_test_step_attention(hip.handle, QKV.handle, QN.handle, KN.handle, EPS, T.handle, Kc.handle,
                                      Vc.handle, max_len, pos, nh, nkv, kv_bf16, att.handle, C.byref(ns)))
    assert (ns.value > 1) == (max_len > 512), f"{ns.value} splits for {max_len} positions"
    q = _head_norm_rope(qkv[:qd], qn, table, pos, nh)
    k = _head_norm_rope(qkv[qd:qd + kvd], kn, table, pos, nkv)
    v = qkv[qd + kvd:]
    kc[:, pos], vc[:, pos] = k.reshape(nkv, hd), v.reshape(nkv, hd)
    # The oracle's caches are position-major: [position][kv head][128].
    exp = ref.attention(q, kc[:, :ctx].transpose(1, 0, 2).copy(), vc[:, :ctx].transpose(1, 0, 2).copy(),
                        pos, nh, hd, nkv)
    got = hip.read(att)
    assert np.all(np.isfinite(got)), "a row past the context reached the output"
    assert rel_error(got, exp) <= 1e-3
    assert_close(got, exp, rel=1e-4, abs_=1e-5, what=f"split attention {nh}/{nkv} ctx {ctx} max_len {max_len}")
    dk, dv = hip.read(Kc), hip.read(Vc)
    if kv_bf16:
        dk = dk[: nkv * max_len * hd // 2].view(np.uint16).reshape(nkv, max_len, hd)
        dv = dv[: nkv * max_len * hd // 2].view(np.uint16).reshape(nkv, max_len, hd)
        assert np.array_equal(dk[:, :pos], kb[:, :pos]), "earlier keys untouched"
        # The appended row is the kernel's f32 key rounded to bf16: within
        # one bf16 rounding of the oracle's.
        assert_close(bf16_to_f32(dk[:, pos]), kc[:, pos], rel=2 ** -8, abs_=1e-5, what="appended key")
        assert_close(bf16_to_f32(dv[:, pos]), vc[:, pos], rel=2 ** -8, abs_=1e-5, what="appended value")
    else:
        dk = dk[: nkv * max_len * hd].reshape(nkv, max_len, hd)
        dv = dv[: nkv * max_len * hd].reshape(nkv, max_len, hd)
        assert np.array_equal(dk[:, :pos], kc[:, :pos]), "earlier keys untouched"
        assert_close(dk[:, pos], kc[:, pos], rel=1e-4, abs_=1e-5, what="appended key")
        assert_close(dv[:, pos], vc[:, pos], rel=1e-4, abs_=1e-5, what="appended value")
        assert np.all(np.isnan(dk[:, pos + 1:])), "rows past pos untouched"


@pytest.mark.parametrize("shape,n,pos", [("0.6b", 100, 0), ("0.6b", 512, 37), ("0.6b", 512, 64), ("4b", 100, 20),
                                         ("narrow", 12288, 0), ("narrow", 12200, 96)])
def test_gemm_qkv(hip, tlib, shape, n, pos):
    """The head tile (32 tokens x one head) and, for the narrow shape, the
    256 x 256 tile (a wave a head of 64 tokens; 12200 tokens leave the last
    token tile ragged, its last V^T slice partly past the tokens)."""
    H, nh, nkv, _ = NARROW if shape == "narrow" else SHAPES[shape]
    hd, qd, kvd = 128, nh * 128, nkv * 128
    max_len = pos + n + 3
    wq, Wq = weight(hip, qd, H, 6, "q")
    wk, Wk = weight(hip, kvd, H, 6, "k")
    wv, Wv = weight(hip, kvd, H, 6, "v")
    qn, QN = gains(hip, hd, 6, "qn")
    kn, KN = gains(hip, hd, 6, "kn")
    xn = np.random.default_rng(n + H).standard_normal(n * H).astype(np.float32)
    table = ref.rope_table(max_len, hd, 1e6)
    Kc, Vc = hip.alloc(nkv * max_len * hd), hip.alloc(nkv * max_len * hd)
    XN, T, qo = buf(hip, xn), buf(hip, table), hip.alloc(n * qd)
    # The planes, prefilled with bf16 NaN pairs that only the new positions may replace.
    L = (max_len + 63) // 64 * 64
    plane = nkv * 128 * L
    sentinel = np.full(2 * plane, 0x7FC07FC0, np.uint32)
    PL = buf(hip, sentinel.view(np.float32))
    check(tlib.th_test_gemm_qkv(hip.handle, XN.handle, Wq.handle, Wk.handle, Wv.handle, QN.handle, KN.handle,
                                EPS, T.handle, Kc.handle, Vc.handle, max_len, pos, n, nh, nkv, qo.handle,
                                PL.handle))
    q = _head_norm_rope(ref.matmul(wq, qd, H, xn), qn, table, pos, nh)
    k = _head_norm_rope(ref.matmul(wk, kvd, H, xn), kn, table, pos, nkv).reshape(n, nkv, hd)
    v = ref.matmul(wv, kvd, H, xn).reshape(n, nkv, hd)
    got = hip.read(qo)
    assert rel_error(got, q) <= 1e-3
    assert_close(got, q, rel=1e-4, abs_=5e-5, what=f"q {shape} n={n}")
    dk = hip.read(Kc).reshape(nkv, max_len, hd)[:, pos:pos + n].transpose(1, 0, 2)
    dv = hip.read(Vc).reshape(nkv, max_len, hd)[:, pos:pos + n].transpose(1, 0, 2)
    assert rel_error(dk, k) <= 1e-3 and rel_error(dv, v) <= 1e-3
    assert_close(dk, k, rel=1e-4, abs_=5e-5, what="keys")
    assert_close(dv, v, rel=1e-4, abs_=5e-5, what="values")
    _check_planes(hip.read(PL).view(np.uint16), dk, dv, pos, n, nkv, L)


def _check_planes(got, dk, dv, pos, n, nkv, L):
    """The epilogue's planes are the bf16 hi/lo split of the cached keys and
    values, bit for bit, at the new positions only: K rows at their
    positions, V^T columns in the P^T operand order of the prefill attention
    (a slice's column 8 g + i holds key 4 g + i for i < 4, else
    16 + 4 g + i - 4)."""
    hd = 128
    plane = nkv * hd * L
    kh, kl, vh, vl = (got[i * plane:(i + 1) * plane] for i in range(4))

    def split(x):
        h = f32_to_bf16(x)
        return h, f32_to_bf16(x - bf16_to_f32(h))

    key_of_col = [4 * g + i if i < 4 else 16 + 4 * g + i - 4 for g in range(4) for i in range(8)]
    col_of_key = np.argsort(key_of_col)
    assert sorted(key_of_col) == list(range(32))
    want = np.full((4, plane), 0x7FC0, np.uint16)
    k_hi, k_lo = split(dk)  # [n][nkv][hd]
    v_hi, v_lo = split(dv)
    p = np.arange(pos, pos + n)
    cols = (p & ~31) + col_of_key[p & 31]
    for g in range(nkv):
        rows = (g * L + p)[:, None] * hd + np.arange(hd)[None, :]
        want[0][rows] = k_hi[:, g]
        want[1][rows] = k_lo[:, g]
        vt = (g * hd + np.arange(hd))[None, :] * L + cols[:, None]
        want[2][vt] = v_hi[:, g]
        want[3][vt] = v_lo[:, g]
    for i, (name, plane_got) in enumerate(zip(("K hi", "K lo", "V^T hi", "V^T lo"), (kh, kl, vh, vl))):
        bad = np.flatnonzero(plane_got != want[i])
        assert bad.size == 0, f"{name}: {bad.size} entries differ, first at {bad[:4]}"


@pytest.mark.parametrize("H,I,n", [(1024, 3072, 100), (1024, 3072, 512), (2560, 9728, 100), (256, 3072, 8000)])
def test_gemm_silu(hip, tlib, H, I, n):
    """The 0.6B and 4B shapes take the 64 x 64 and 128 x 128 tiles; 8000
    tokens x 2 x 3072 rows, 768 tiles of 256 x 256, the largest tile with its
    SiLU epilogue in registers (against float64 products there: the oracle's
    matmul would take minutes)."""
    wg, Wg = weight(hip, I, H, 7, "gate")
    wu, Wu = weight(hip, I, H, 7, "up")
    xn = np.random.default_rng(n + I).standard_normal(n * H).astype(np.float32)
    XN, ho = buf(hip, xn), hip.alloc(n * I)
    check(tlib.th_test_gemm_silu(hip.handle, XN.handle, Wg.handle, Wu.handle, n, ho.handle))
    if n * H * I <= 1 << 31:
        g, u = ref.matmul(wg, I, H, xn), ref.matmul(wu, I, H, xn)
        exp = ref.silu_mul(g, u)
    else:
        x64 = xn.astype(np.float64).reshape(n, H)
        g = (x64 @ bf16_to_f32(wg).astype(np.float64).reshape(I, H).T).reshape(-1)
        u = (x64 @ bf16_to_f32(wu).astype(np.float64).reshape(I, H).T).reshape(-1)
        exp = g / (1.0 + np.exp(-g)) * u
    got = hip.read(ho)
    assert rel_error(got, exp) <= 1e-3
    # The kernel multiplies x kept as bf16 hi + lo (error <= 2^-17 |x_i|
    # each, independent): gate and up are off by at most 6 standard
    # deviations of that sum, eg and eu; h by |silu(g)| eu + |silu'(g) u| eg,
    # plus its own hi + lo rounding (2^-16 |h|).
    g, u = g.astype(np.float64), u.astype(np.float64)
    eg, eu = split_sigma(wg, I, H, xn), split_sigma(wu, I, H, xn)
    sg = 1.0 / (1.0 + np.exp(-g))
    bound = np.abs(g * sg) * eu + np.abs(sg * (1 + g * (1 - sg)) * u) * eg + 2.0 ** -16 * np.abs(exp) + 1e-6
    err = np.abs(got.astype(np.float64) - exp)
    assert np.all(err <= bound), f"silu(gate) * up {shape} n={n}: worst {np.max(err / bound):.2f} of the bound"


@pytest.mark.parametrize("dim,rows,n_parts", [(1024, 100, 0), (1024, 100, 1), (1024, 64, 3), (2560, 40, 2)])
def test_add_rmsnorm_parts(hip, tlib, dim, rows, n_parts):
    g, G = gains(hip, dim, 8, "g")
    rng = np.random.default_rng(dim + rows + n_parts)
    x = rng.standard_normal(rows * dim).astype(np.float32)
    parts = rng.standard_normal(n_parts * rows * dim).astype(np.float32)
    X, XN = buf(hip, x), hip.alloc(rows * dim)
    P = buf(hip, parts) if n_parts else None
    check(tlib.th_test_add_rmsnorm_parts(hip.handle, X.handle, h(P), n_parts, G.handle, EPS, XN.handle))
    xs = x.copy()
    if n_parts:
        # The partials are summed in order, then added (one rounding each).
        s = parts.reshape(n_parts, -1)[0].copy()
        for p in range(1, n_parts):
            s = ref.add(s, parts.reshape(n_parts, -1)[p])
        xs = ref.add(xs, s)
    exp = ref.rmsnorm(xs, g, EPS)
    assert_close(hip.read(X), xs, rel=1e-6, abs_=1e-6, what="x + partials")
    got = hip.read(XN)
    assert rel_error(got, exp) <= 1e-3
    assert_close(got, exp, rel=2e-5, abs_=1e-6, what="rmsnorm as hi + lo")


@pytest.mark.parametrize("n,pos,H,KVH", [(512, 0, 16, 8), (100, 37, 16, 8), (1500, 600, 16, 8), (300, 20, 32, 8),
                                         (64, 1000, 32, 8), (200, 5, 16, 2), (100, 3, 8, 8), (2048, 0, 32, 8),
                                         (2100, 150, 32, 8), (4096, 0, 16, 8)])
def test_attention_planes(hip, tlib, n, pos, H, KVH):
    """Prefill attention through the bf16 planes (keys and values split once
    per call) gives the per-block-split kernel's output bit for bit, and the
    oracle's within the per-kernel bar (exact float64 attention past the
    oracle's sizes). The last three shapes take the planes kernel's 256-row
    blocks. Cache rows past pos + n hold NaN: a read of them would reach the
    output."""
    hd, max_len = 128, pos + n + 70
    rng = np.random.default_rng(n + pos + H)
    q = rng.standard_normal(n * H * hd).astype(np.float32)
    kc = np.full((KVH, max_len, hd), np.nan, np.float32)
    vc = np.full((KVH, max_len, hd), np.nan, np.float32)
    kc[:, :pos + n] = rng.standard_normal((KVH, pos + n, hd))
    vc[:, :pos + n] = rng.standard_normal((KVH, pos + n, hd))
    Q, K, V = buf(hip, q), buf(hip, kc), buf(hip, vc)
    outs = []
    for planes in (0, 1):
        O = hip.alloc(n * H * hd)
        check(tlib.th_test_attention_prefill(hip.handle, Q.handle, K.handle, V.handle, max_len, pos, n, H, KVH,
                                             planes, O.handle))
        outs.append(hip.read(O))
    assert np.all(np.isfinite(outs[1]))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), "planes differ from the split kernel"
    if n * (pos + n) <= 600_000:
        # The oracle's caches are position-major: [position][kv head][128].
        exp = ref.attention(q, kc[:, :pos + n].transpose(1, 0, 2).copy(), vc[:, :pos + n].transpose(1, 0, 2).copy(),
                            pos, H, hd, KVH)
        assert rel_error(outs[1], exp) <= 1e-3
        assert_close(outs[1], exp, rel=1e-4, abs_=2e-5, what=f"attention n={n} pos={pos} {H}/{KVH}")
    else:
        exp = attention_f64(q, kc, vc, pos, H, KVH)
        assert rel_error(outs[1], exp) <= 1e-3
        assert_close(outs[1], exp, rel=1e-4, abs_=2e-5, what=f"attention n={n} pos={pos} {H}/{KVH} (float64)")
