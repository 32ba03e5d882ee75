"""Per-operation parity of the hip device against the CPU oracle.

The first group restates the reference's own differential tests
(model/titania.rs:268-370): same shapes, same closed-form xorshift inputs, same
tolerance |a - e| <= 1e-5 + 1e-4 |e|. The second runs the Qwen3-0.6B decode
shapes (bf16 weights, f32 activations N(0, 1), seeded) and the GQA decode
attention at contexts 512, 4096 and 32768, against the per-kernel bar of
relative error <= 1e-3 (and tighter elementwise bounds where fp32 rounding
allows).
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import ref
from titania_amd import InvalidArgument, Tensor
from titania_amd.synth import bf16_to_f32, f32_to_bf16, normal_bf16
from util import assert_close, numbers, rel_error, tensor

pytestmark = pytest.mark.gpu


def buffers(hip, n, seed):
    """A buffer on the device and its host copy, holding numbers(n, seed)."""
    values = numbers(n, seed)
    buf = hip.alloc(n)
    hip.write(buf, values)
    return values, buf


# ---- model/titania.rs:268-370 ----

def test_elementwise(hip):
    n = 300
    cx, x = buffers(hip, n, 1)
    cy, y = buffers(hip, n, 2)
    cx = ref.add(cx, cy)
    hip.add(x, y)
    assert_close(hip.read(x), cx, what="add")

    cx = ref.silu_mul(cx, cy)
    hip.silu_mul(x, y)
    assert_close(hip.read(x), cx, what="silu_mul")

    cdst, dst = buffers(hip, n + 10, 3)
    cdst = ref.copy(cdst, 7, cx, 5, n - 5)
    hip.copy(dst, 7, x, 5, n - 5)
    assert_close(hip.read(dst), cdst, what="copy")


def test_resize(hip):
    cx, x = buffers(hip, 300, 1)
    cy, y = buffers(hip, 100, 2)
    hip.resize(x, 100)
    cx = ref.add(cx[:100], cy)
    hip.add(x, y)
    assert_close(hip.read(x), cx, what="resize+add")
    hip.resize(x, 300)
    assert len(hip.read(x)) == 300


def test_embed(hip):
    table = tensor((10, 128), 4)
    tokens = [3, 9, 0]
    _, out = buffers(hip, 3 * 128, 5)
    expected = ref.embed(table.data, 128, tokens)
    w = hip.upload(table)
    hip.embed(out, w, tokens)
    got = hip.read(out)
    assert np.array_equal(got.view(np.uint32), expected.view(np.uint32)), "embed is exact"


@pytest.mark.parametrize("rows,cols,n", [(24, 256, 1), (5, 64, 3), (9, 384, 16), (24, 128, 19)])
def test_matmul(hip, rows, cols, n):
    w = tensor((rows, cols), 6)
    cx, x = buffers(hip, n * cols, 7)
    _, out = buffers(hip, n * rows, 8)
    expected = ref.matmul(w.data, rows, cols, cx)
    hip.matmul(out, hip.upload(w), x)
    assert_close(hip.read(out), expected, what=f"matmul {rows}x{cols} n={n}")


@pytest.mark.parametrize("rows,dim", [(3, 128), (1, 1024), (9, 64)])
def test_rmsnorm(hip, rows, dim):
    weight = tensor((dim,), 9)
    cx, x = buffers(hip, rows * dim, 10)
    expected = ref.rmsnorm(cx, weight.data, 1e-6)
    hip.rmsnorm(x, hip.upload(weight), 1e-6)
    assert_close(hip.read(x), expected, what="rmsnorm")


@pytest.mark.parametrize("n", [1, 3])
def test_rope(hip, n):
    cx, x = buffers(hip, n * 4 * 128, 11)
    ctable, table = buffers(hip, 40 * 128, 16)
    expected = ref.rope(cx, ctable, 37, 4, 128)
    hip.rope(x, table, 37, 4, 128)
    assert_close(hip.read(x), expected, what="rope")


@pytest.mark.parametrize("pos,n", [(0, 1), (6, 1), (32, 1), (39, 1), (0, 5), (30, 10)])
def test_attention(hip, pos, n):
    n_heads, head_dim, n_kv_heads, max_len = 4, 64, 2, 40
    kv_len = max_len * n_kv_heads * head_dim
    cq, q = buffers(hip, n * n_heads * head_dim, 12)
    ck, k = buffers(hip, kv_len, 13)
    cv, v = buffers(hip, kv_len, 14)
    _, out = buffers(hip, n * n_heads * head_dim, 15)
    if pos + n > max_len:
        pytest.skip("past the cache")
    expected = ref.attention(cq, ck, cv, pos, n_heads, head_dim, n_kv_heads)
    hip.attention(out, q, k, v, pos, n_heads, head_dim, n_kv_heads)
    assert_close(hip.read(out), expected, what=f"attention pos={pos} n={n}")


# ---- the reference's panics are errors here ----

def test_misuse_is_an_error(hip):
    x = hip.alloc(10)
    with pytest.raises(InvalidArgument):
        hip.resize(x, 11)
    with pytest.raises(InvalidArgument):
        hip.write(x, np.zeros(9, np.float32))
    w = hip.upload(tensor((4, 8), 1))
    out = hip.alloc(4)
    with pytest.raises(InvalidArgument):
        hip.matmul(out, w, x)  # 10 is not a whole number of 8-long rows
    table = hip.upload(tensor((10, 8), 2))
    e = hip.alloc(8)
    with pytest.raises(InvalidArgument):
        hip.embed(e, table, [10])  # past the table
    rt = hip.alloc(4 * 8)
    q = hip.alloc(2 * 8)
    with pytest.raises(InvalidArgument):
        hip.rope(q, rt, 4, 2, 8)  # position 4 is past a 4-position table
    with pytest.raises(InvalidArgument):
        hip.copy(x, 5, x, 0, 6)


# ---- Qwen3-0.6B decode shapes: bf16 W and f32 x, N(0, 1) ----

QWEN_GEMV = {
    "q": (2048, 1024), "k+v": (1024, 1024), "o": (1024, 2048), "gate+up": (6144, 1024),
    "down": (1024, 3072), "lm_head": (151936, 1024),
}


def _row_bound(wbits, rows, cols, x, n):
    w = bf16_to_f32(wbits).reshape(rows, cols).astype(np.float64)
    xx = np.asarray(x, np.float64).reshape(n, cols)
    return (np.abs(xx) @ np.abs(w).T).reshape(-1)


@pytest.mark.parametrize("name", list(QWEN_GEMV))
@pytest.mark.parametrize("n", [1, 4])
def test_qwen_gemv(hip, name, n):
    rows, cols = QWEN_GEMV[name]
    wbits = normal_bf16(rows * cols, 100, name)
    x = bf16_to_f32(normal_bf16(n * cols, 101, name + "x")) + np.float32(1e-3) * bf16_to_f32(
        normal_bf16(n * cols, 102, name + "x2"))
    expected = ref.matmul(wbits, rows, cols, x)
    xb = hip.alloc(n * cols)
    hip.write(xb, x)
    out = hip.alloc(n * rows)
    hip.matmul(out, hip.upload(Tensor((rows, cols), wbits)), xb)
    got = hip.read(out)
    assert rel_error(got, expected) <= 1e-3
    # fp32 accumulation in another order: within a few ulps of the row's magnitude.
    bound = _row_bound(wbits, rows, cols, x, n)
    assert np.all(np.abs(got.astype(np.float64) - expected) <= 3e-5 * bound + 1e-6)


@pytest.mark.parametrize("n", [16, 64])
def test_qwen_gemm(hip, n):
    rows, cols = 2048, 1024
    wbits = normal_bf16(rows * cols, 103, "gemm")
    x = bf16_to_f32(normal_bf16(n * cols, 104, "gemmx")) * np.float32(1.37)
    expected = ref.matmul(wbits, rows, cols, x)
    xb = hip.alloc(n * cols)
    hip.write(xb, x)
    out = hip.alloc(n * rows)
    hip.matmul(out, hip.upload(Tensor((rows, cols), wbits)), xb)
    got = hip.read(out)
    assert rel_error(got, expected) <= 1e-3
    bound = _row_bound(wbits, rows, cols, x, n)
    assert np.all(np.abs(got.astype(np.float64) - expected) <= 3e-5 * bound + 1e-6)


# The prefill GEMM shapes of Qwen3-0.6B ([n x cols] x [cols x rows]); n = 100 is
# a ragged token tile, n = 512 the 512-token prompt.
QWEN_GEMM = {"q": (2048, 1024), "k/v": (1024, 1024), "o": (1024, 2048), "gate/up": (3072, 1024),
             "down": (1024, 3072)}


@pytest.mark.parametrize("name", list(QWEN_GEMM))
@pytest.mark.parametrize("n", [100, 512])
def test_qwen_prefill_gemm(hip, name, n):
    """MFMA path with f32 activations that bf16 cannot hold exactly: the
    relative error bar and an elementwise bound of a few fp32 ulps of the row.
    The o projection at 512 tokens takes the split-K plan of the small tile."""
    rows, cols = QWEN_GEMM[name]
    rng = np.random.default_rng(n + rows + cols)
    wbits = normal_bf16(rows * cols, 105, name)
    x = rng.standard_normal(n * cols).astype(np.float32)
    if n == 512 and name not in ("q", "down"):
        # A float64 product stands in for the oracle here (faster); both
        # bounds below hold against either.
        w64 = bf16_to_f32(wbits).astype(np.float64).reshape(rows, cols)
        expected = (x.astype(np.float64).reshape(n, cols) @ w64.T).reshape(-1)
    else:
        expected = ref.matmul(wbits, rows, cols, x)
    xb = hip.alloc(n * cols)
    hip.write(xb, x)
    out = hip.alloc(n * rows)
    hip.matmul(out, hip.upload(Tensor((rows, cols), wbits)), xb)
    got = hip.read(out)
    assert rel_error(got, expected) <= 1e-5
    bound = _row_bound(wbits, rows, cols, x, n)
    assert np.all(np.abs(got.astype(np.float64) - expected) <= 3e-5 * bound + 1e-6)


# The prefill GEMM shapes of Qwen3-4B, against a float64 product.
QWEN4B_GEMM = {"q": (4096, 2560), "k/v": (1024, 2560), "o": (2560, 4096), "gate/up": (9728, 2560),
               "down": (2560, 9728)}


@pytest.mark.parametrize("name", list(QWEN4B_GEMM))
@pytest.mark.parametrize("n", [100, 512, 2048])
def test_qwen4b_prefill_gemm(hip, name, n):
    """Every tile plan the Qwen3-4B shapes take: the small tile with and
    without a K split (100 and 512 tokens) and, at 2048 tokens, the large
    tile (gate/up) and the large tile with K split in two (down, 320 tiles
    and 152 K steps)."""
    rows, cols = QWEN4B_GEMM[name]
    rng = np.random.default_rng(n + rows + cols + 7)
    wbits = normal_bf16(rows * cols, 107, name)
    x = rng.standard_normal(n * cols).astype(np.float32)
    w64 = bf16_to_f32(wbits).astype(np.float64).reshape(rows, cols)
    expected = (x.astype(np.float64).reshape(n, cols) @ w64.T).reshape(-1)
    xb = hip.alloc(n * cols)
    hip.write(xb, x)
    out = hip.alloc(n * rows)
    hip.matmul(out, hip.upload(Tensor((rows, cols), wbits)), xb)
    got = hip.read(out)
    assert rel_error(got, expected) <= 1e-5
    bound = (np.abs(x.astype(np.float64).reshape(n, cols)) @ np.abs(w64).T).reshape(-1)
    assert np.all(np.abs(got.astype(np.float64) - expected) <= 3e-5 * bound + 1e-6)


@pytest.mark.parametrize("rows,cols,n", [(6144, 1024, 2000), (4096, 6144, 1024), (6144, 512, 8000),
                                         (2560, 1024, 8000)])
def test_large_tile_gemm(hip, rows, cols, n):
    """The 128 x 128 tile: a launch of 768 tiles with a ragged last token tile,
    and a single matrix of 256 tiles and 96 K steps, which splits K in two;
    the 256 x 256 tile: 768 tiles, the last token tile ragged, and a single
    matrix of 320 tiles, which splits K in two (the Qwen3-4B o and down
    projections at 8192 tokens). Against a float64 product: the relative
    error bar and an elementwise bound of a few fp32 ulps of the row."""
    rng = np.random.default_rng(rows + cols + n)
    wbits = normal_bf16(rows * cols, 106, "large")
    x = rng.standard_normal(n * cols).astype(np.float32)
    w64 = bf16_to_f32(wbits).astype(np.float64).reshape(rows, cols)
    expected = (x.astype(np.float64).reshape(n, cols) @ w64.T).reshape(-1)
    xb = hip.alloc(n * cols)
    hip.write(xb, x)
    out = hip.alloc(n * rows)
    hip.matmul(out, hip.upload(Tensor((rows, cols), wbits)), xb)
    got = hip.read(out)
    assert rel_error(got, expected) <= 1e-5
    bound = (np.abs(x.astype(np.float64).reshape(n, cols)) @ np.abs(w64).T).reshape(-1)
    assert np.all(np.abs(got.astype(np.float64) - expected) <= 3e-5 * bound + 1e-6)


def test_qwen_norms_and_rope(hip):
    # RMSNorm over 1024 and per head over 128 (16 q heads + 8 k heads), gains 1 + N(0, .1).
    for rows, dim, seed in [(1, 1024, 110), (16, 128, 111), (8, 128, 112)]:
        g = f32_to_bf16(1.0 + bf16_to_f32(normal_bf16(dim, seed, "g", 0.1)))
        x = bf16_to_f32(normal_bf16(rows * dim, seed, "x")) * np.float32(3.0)
        expected = ref.rmsnorm(x, g, 1e-6)
        xb = hip.alloc(rows * dim)
        hip.write(xb, x)
        hip.rmsnorm(xb, hip.upload(Tensor((dim,), g)), 1e-6)
        got = hip.read(xb)
        assert rel_error(got, expected) <= 1e-3
        assert_close(got, expected, rel=1e-5, abs_=1e-6, what=f"rmsnorm {rows}x{dim}")
    # RoPE on 16 + 8 heads x 128 with the theta = 1e6 table at a late position.
    table = ref.rope_table(4096, 128, 1e6)
    tb = hip.alloc(table.size)
    hip.write(tb, table)
    for heads in (16, 8):
        x = bf16_to_f32(normal_bf16(heads * 128, 113 + heads, "r"))
        expected = ref.rope(x, table, 4000, heads, 128)
        xb = hip.alloc(x.size)
        hip.write(xb, x)
        hip.rope(xb, tb, 4000, heads, 128)
        assert_close(hip.read(xb), expected, rel=1e-5, abs_=1e-6, what="rope")


@pytest.mark.parametrize("ctx", [512, 4096, 32768])
def test_qwen_decode_attention(hip, ctx):
    """GQA decode: 16 Q heads, 8 KV heads, head_dim 128, caches of bf16-rounded
    N(0, 1), the query at position ctx - 1."""
    H, KVH, hd = 16, 8, 128
    kv = bf16_to_f32(normal_bf16(ctx * KVH * hd, ctx, "k"))
    vv = bf16_to_f32(normal_bf16(ctx * KVH * hd, ctx, "v"))
    q = bf16_to_f32(normal_bf16(H * hd, ctx, "q"))
    expected = ref.attention(q, kv, vv, ctx - 1, H, hd, KVH)
    bk, bv, bq, out = hip.alloc(kv.size), hip.alloc(vv.size), hip.alloc(q.size), hip.alloc(q.size)
    hip.write(bk, kv)
    hip.write(bv, vv)
    hip.write(bq, q)
    hip.attention(out, bq, bk, bv, ctx - 1, H, hd, KVH)
    got = hip.read(out)
    assert rel_error(got, expected) <= 1e-3
    assert_close(got, expected, rel=1e-4, abs_=1e-5, what=f"attention ctx={ctx}")


@pytest.mark.parametrize("n,pos,H,KVH", [(1, 0, 16, 8), (2, 100, 16, 8), (7, 1000, 32, 8), (3, 63, 8, 8),
                                         (5, 200, 16, 2), (1, 17000, 12, 4)])
def test_few_token_attention(hip, n, pos, H, KVH):
    """head_dim 128 with fewer tokens than the matrix-core kernels take: one
    block per (token, KV head, 64-position split), groups of 1 to 8 heads, a
    split boundary inside the context (pos 63, 1000), two passes a split
    (17001 positions: more than 256 splits of 64)."""
    hd = 128
    L = pos + n
    kv = bf16_to_f32(normal_bf16(L * KVH * hd, n + pos, "fk"))
    vv = bf16_to_f32(normal_bf16(L * KVH * hd, n + pos, "fv"))
    q = bf16_to_f32(normal_bf16(n * H * hd, n + pos, "fq"))
    expected = ref.attention(q, kv, vv, pos, H, hd, KVH)
    bk, bv, bq, out = hip.alloc(kv.size), hip.alloc(vv.size), hip.alloc(q.size), hip.alloc(q.size)
    hip.write(bk, kv)
    hip.write(bv, vv)
    hip.write(bq, q)
    hip.attention(out, bq, bk, bv, pos, H, hd, KVH)
    got = hip.read(out)
    assert rel_error(got, expected) <= 1e-5
    assert_close(got, expected, rel=1e-4, abs_=1e-5, what=f"few-token attention n={n} pos={pos}")


def test_prefill_attention(hip):
    """Causal attention of 100 tokens from position 300 (keys split over two blocks)."""
    H, KVH, hd, n, pos = 16, 8, 128, 100, 300
    L = pos + n
    kv = bf16_to_f32(normal_bf16(L * KVH * hd, 7, "pk"))
    vv = bf16_to_f32(normal_bf16(L * KVH * hd, 7, "pv"))
    q = bf16_to_f32(normal_bf16(n * H * hd, 7, "pq"))
    expected = ref.attention(q, kv, vv, pos, H, hd, KVH)
    bk, bv, bq, out = hip.alloc(kv.size), hip.alloc(vv.size), hip.alloc(q.size), hip.alloc(q.size)
    hip.write(bk, kv)
    hip.write(bv, vv)
    hip.write(bq, q)
    hip.attention(out, bq, bk, bv, pos, H, hd, KVH)
    assert_close(hip.read(out), expected, rel=1e-4, abs_=1e-5, what="prefill attention")


@pytest.mark.parametrize("n,pos,H,KVH", [(33, 0, 16, 8), (512, 0, 16, 8), (64, 300, 32, 8), (8, 5, 4, 1),
                                         (77, 40, 8, 8), (50, 90, 16, 2), (300, 700, 32, 8), (20, 0, 12, 4)])
def test_prefill_attention_tiles(hip, n, pos, H, KVH):
    """The query-tiled prefill kernels: a ragged tile, a 512-token prompt, a
    4-query-head group after a long prefix, the smallest tiled launch, groups
    of 1 and 8 query heads, a long prefix split over several blocks, and a
    group of 3 (not a divisor of 8: the one-head-a-block kernel)."""
    hd = 128
    L = pos + n
    kv = bf16_to_f32(normal_bf16(L * KVH * hd, n, "tk"))
    vv = bf16_to_f32(normal_bf16(L * KVH * hd, n, "tv"))
    q = bf16_to_f32(normal_bf16(n * H * hd, n, "tq"))
    expected = ref.attention(q, kv, vv, pos, H, hd, KVH)
    bk, bv, bq, out = hip.alloc(kv.size), hip.alloc(vv.size), hip.alloc(q.size), hip.alloc(q.size)
    hip.write(bk, kv)
    hip.write(bv, vv)
    hip.write(bq, q)
    hip.attention(out, bq, bk, bv, pos, H, hd, KVH)
    got = hip.read(out)
    assert rel_error(got, expected) <= 1e-5
    assert_close(got, expected, rel=1e-4, abs_=1e-5, what=f"prefill attention n={n} pos={pos}")


# ---- fused extensions ----

def test_add_rmsnorm(hip):
    rows, dim = 3, 1024
    g = f32_to_bf16(1.0 + bf16_to_f32(normal_bf16(dim, 120, "g", 0.1)))
    x = numbers(rows * dim, 21)
    y = numbers(rows * dim, 22)
    cx = ref.add(x, y)
    cxb = ref.rmsnorm(cx, g, 1e-6)
    bx, by, bxb = hip.alloc(x.size), hip.alloc(y.size), hip.alloc(x.size)
    hip.write(bx, x)
    hip.write(by, y)
    hip.add_rmsnorm(bx, by, bxb, hip.upload(Tensor((dim,), g)), 1e-6)
    assert_close(hip.read(bx), cx, what="x += y")
    assert_close(hip.read(bxb), cxb, what="rmsnorm(x)")


@pytest.mark.parametrize("n,pos,shape", [(1, 0, "0.6b"), (1, 37, "4b"), (3, 10, "0.6b"), (20, 5, "0.6b"),
                                         (64, 100, "4b"), (5, 2, "tiny")])
def test_qkv_rope_append(hip, n, pos, shape):
    """th_qkv_rope_append (the trait extension's qkv_rope_append) against the
    oracle's matmul x 3, q/k rmsnorm, rope x 2 and cache copies
    (model.rs:108-120) into position-major caches: one token takes the
    three-matrix GEMV, 3 the few-token GEMV, 20 and 64 the MFMA GEMM; the
    tiny shape (head_dim 64, hidden 256) has no q/k norms."""
    H, nh, nkv, hd, norms = {"0.6b": (1024, 16, 8, 128, True), "4b": (2560, 32, 8, 128, True),
                             "tiny": (256, 4, 2, 64, False)}[shape]
    qd, kvd, max_len, eps = nh * hd, nkv * hd, pos + n + 5, 1e-6
    ws = [normal_bf16(r * H, 130 + i, "w", 0.05) for i, r in enumerate((qd, kvd, kvd))]
    W = [hip.upload(Tensor((r, H), w)) for r, w in zip((qd, kvd, kvd), ws)]
    gq = f32_to_bf16(1.0 + bf16_to_f32(normal_bf16(hd, 131, "gq", 0.1)))
    gk = f32_to_bf16(1.0 + bf16_to_f32(normal_bf16(hd, 132, "gk", 0.1)))
    QN, KN = (hip.upload(Tensor((hd,), gq)), hip.upload(Tensor((hd,), gk))) if norms else (None, None)
    rng = np.random.default_rng(n + pos)
    xb = rng.standard_normal(n * H).astype(np.float32)
    kc = rng.standard_normal(max_len * kvd).astype(np.float32)
    vc = rng.standard_normal(max_len * kvd).astype(np.float32)
    table = ref.rope_table(max_len, hd, 1e6)
    bufs = {}
    for name, a in (("xb", xb), ("kc", kc), ("vc", vc), ("rope", table)):
        bufs[name] = hip.alloc(a.size)
        hip.write(bufs[name], a)
    q, k, v = hip.alloc(n * qd), hip.alloc(n * kvd), hip.alloc(n * kvd)
    hip.qkv_rope_append(q, k, v, W[0], W[1], W[2], QN, KN, bufs["xb"], bufs["rope"], bufs["kc"], bufs["vc"], pos,
                        nh, nkv, hd, eps)
    eq = ref.matmul(ws[0], qd, H, xb)
    ek = ref.matmul(ws[1], kvd, H, xb)
    ev = ref.matmul(ws[2], kvd, H, xb)
    if norms:
        eq, ek = ref.rmsnorm(eq, gq, eps), ref.rmsnorm(ek, gk, eps)
    eq, ek = ref.rope(eq, table, pos, nh, hd), ref.rope(ek, table, pos, nkv, hd)
    ekc = ref.copy(kc, pos * kvd, ek, 0, n * kvd)
    evc = ref.copy(vc, pos * kvd, ev, 0, n * kvd)
    for what, got, exp in (("q", hip.read(q), eq), ("k cache", hip.read(bufs["kc"]), ekc),
                           ("v cache", hip.read(bufs["vc"]), evc)):
        assert rel_error(got, exp) <= 1e-3, what
        assert_close(got, exp, rel=1e-4, abs_=5e-5, what=f"{what} n={n} {shape}")
    dk = hip.read(bufs["kc"])
    assert np.array_equal(dk[:pos * kvd], kc[:pos * kvd]) and np.array_equal(dk[(pos + n) * kvd:],
                                                                               kc[(pos + n) * kvd:])


@pytest.mark.parametrize("n,H,I", [(1, 1024, 3072), (1, 2560, 9728), (4, 1024, 3072), (32, 1024, 3072),
                                   (2, 256, 512)])
def test_gate_up_silu(hip, n, H, I):
    """th_gate_up_silu (the trait extension's gate_up_silu) against the
    oracle's matmul x 2 + silu_mul (model.rs:137-139): one token takes the
    GEMV with the SiLU epilogue, 32 the MFMA GEMM."""
    wg, wu = normal_bf16(I * H, 140, "g", 0.05), normal_bf16(I * H, 141, "u", 0.05)
    Wg, Wu = hip.upload(Tensor((I, H), wg)), hip.upload(Tensor((I, H), wu))
    xb = np.random.default_rng(n + H).standard_normal(n * H).astype(np.float32)
    bx, gate, up = hip.alloc(xb.size), hip.alloc(n * I), hip.alloc(n * I)
    hip.write(bx, xb)
    hip.gate_up_silu(gate, up, Wg, Wu, bx)
    exp = ref.silu_mul(ref.matmul(wg, I, H, xb), ref.matmul(wu, I, H, xb))
    got = hip.read(gate)
    assert rel_error(got, exp) <= 1e-3
    assert_close(got, exp, rel=1e-4, abs_=5e-5, what=f"gate_up_silu n={n}")


def test_add_rmsnorm_in_place(hip):
    """y may be xb itself (the trait extension's add_rmsnorm: the projection
    in xb added into x, then x's norm into xb)."""
    rows, dim = 5, 1024
    g = f32_to_bf16(1.0 + bf16_to_f32(normal_bf16(dim, 121, "g", 0.1)))
    x, y = numbers(rows * dim, 23), numbers(rows * dim, 24)
    bx, bxb = hip.alloc(x.size), hip.alloc(y.size)
    hip.write(bx, x)
    hip.write(bxb, y)
    hip.add_rmsnorm(bx, bxb, bxb, hip.upload(Tensor((dim,), g)), 1e-6)
    cx = ref.add(x, y)
    assert_close(hip.read(bx), cx, what="x += xb")
    assert_close(hip.read(bxb), ref.rmsnorm(cx, g, 1e-6), what="xb = rmsnorm(x)")


def test_argmax(hip):
    v = 151936
    x = bf16_to_f32(normal_bf16(v, 130, "logits"))
    b = hip.alloc(v)
    hip.write(b, x)
    assert hip.argmax(b) == ref.argmax(x) == int(np.argmax(x))
    # Ties go to the lowest index; -0.0 < +0.0 under total order.
    y = np.zeros(v, np.float32)
    y[[5000, 70000, 150000]] = 3.0
    hip.write(b, y)
    assert hip.argmax(b) == ref.argmax(y) == 5000
    z = np.full(v, -1.0, np.float32)
    z[10] = -0.0
    z[11] = 0.0
    hip.write(b, z)
    assert hip.argmax(b) == ref.argmax(z) == 11
