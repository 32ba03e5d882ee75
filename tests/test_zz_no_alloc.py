"""th_attention_noalloc: th_attention with its split partials in the
library's fixed per-GPU array. Called through the C ABI (ctypes) and compared
with th_attention on the same inputs, on two calls in a row (the second with
a smaller input, so that it runs over what the first left in the array), and
with the oracle; a call whose partials exceed the array is refused on the
host, before any launch."""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from oracle import ref
from titania_amd import InvalidArgument
from titania_amd._lib import check, lib
from titania_amd.synth import bf16_to_f32, normal_bf16
from util import rel_error

pytestmark = pytest.mark.gpu


def _case(hip, ctx: int, n: int, H: int, KVH: int, seed: int):
    hd = 128
    kv = bf16_to_f32(normal_bf16(ctx * KVH * hd, seed, "nk"))
    vv = bf16_to_f32(normal_bf16(ctx * KVH * hd, seed, "nv"))
    q = bf16_to_f32(normal_bf16(n * H * hd, seed, "nq"))
    bufs = [hip.alloc(a.size) for a in (kv, vv, q)]
    for b, a in zip(bufs, (kv, vv, q)):
        hip.write(b, a)
    return (kv, vv, q), bufs


def _call(fn, hip, out, q, k, v, pos, H, hd, KVH):
    check(fn(C.c_void_p(hip.handle), C.c_void_p(out.handle), C.c_void_p(q.handle), C.c_void_p(k.handle),
             C.c_void_p(v.handle), C.c_size_t(pos), C.c_size_t(H), C.c_size_t(hd), C.c_size_t(KVH)))


@pytest.mark.parametrize("first,second", [((4096, 1, 16, 8), (1000, 1, 16, 8)), ((20000, 1, 32, 8), (600, 3, 8, 2)),
                                          ((16400, 1, 64, 8), (9000, 1, 64, 8))])
def test_noalloc_matches_attention(hip, first, second):
    """The third pair: one token of 64 heads past 16384 positions, 256
    splits (64 x 256 x 130 floats, 8.5 MB of partials)."""
    L = lib()
    for i, (ctx, n, H, KVH) in enumerate((first, second)):
        (kv, vv, q), (bk, bv, bq) = _case(hip, ctx, n, H, KVH, seed=ctx + i)
        pos = ctx - n
        out_a, out_b = hip.alloc(q.size), hip.alloc(q.size)
        _call(L.th_attention_noalloc, hip, out_a, bq, bk, bv, pos, H, 128, KVH)
        got = hip.read(out_a)
        _call(L.th_attention, hip, out_b, bq, bk, bv, pos, H, 128, KVH)
        exp = hip.read(out_b)
        # The same kernels on the same inputs: bit-identical to th_attention.
        assert np.array_equal(got.view(np.uint32), exp.view(np.uint32)), f"call {i}: ctx {ctx}"
        # And the reference's bar against the oracle.
        assert rel_error(got, ref.attention(q, kv, vv, pos, H, 128, KVH)) <= 1e-3


def test_noalloc_refuses_oversized_partials(hip):
    """A 512-token prefill over 8192 positions needs more partials than the
    array holds: refused with an error, nothing launched."""
    H, KVH, hd, n, ctx = 32, 8, 128, 512, 8192
    k, v, q, out = hip.alloc(ctx * KVH * hd), hip.alloc(ctx * KVH * hd), hip.alloc(n * H * hd), hip.alloc(n * H * hd)
    with pytest.raises(InvalidArgument, match="fixed"):
        hip.attention_noalloc(out, q, k, v, ctx - n, H, hd, KVH)
