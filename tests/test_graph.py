"""HIP graphs of the device's stream (th_graph_begin / end / launch): a
captured sequence of the trait's compute calls replays to the same bits as the
same calls run eagerly, replay after replay with other device work between
them, and the calls that cannot be captured are refused while a capture is
open."""

import numpy as np
import pytest

from oracle import ref
from titania_amd import Tensor
from titania_amd.synth import bf16_to_f32, normal_bf16

pytestmark = pytest.mark.gpu

H, KVH, HD = 16, 8, 128
HIDDEN, INTER = 1024, 3072
POS = 1500  # attention over 1501 positions: the keys split over several blocks


def _inputs():
    rng = np.random.default_rng(7)
    return {
        "x": rng.standard_normal(HIDDEN).astype(np.float32),
        "q": bf16_to_f32(normal_bf16(H * HD, 201, "gq")),
        "k": bf16_to_f32(normal_bf16((POS + 1) * KVH * HD, 201, "gk")),
        "v": bf16_to_f32(normal_bf16((POS + 1) * KVH * HD, 201, "gv")),
        "gate": rng.standard_normal(INTER).astype(np.float32),
        "up": rng.standard_normal(INTER).astype(np.float32),
        "table": ref.rope_table(POS + 1, HD, 1e6),
    }


class _Run:
    """Buffers and weights of one sequence: rmsnorm(x), w . x, rope(q), attention, silu_mul."""

    def __init__(self, hip, data, w, gain):
        self.hip, self.data, self.w, self.gain = hip, data, w, gain
        self.b = {k: hip.alloc(v.size) for k, v in data.items()}
        self.y = hip.alloc(2048)
        self.att = hip.alloc(H * HD)

    def load(self):
        for k, v in self.data.items():
            self.hip.write(self.b[k], v)

    def calls(self):
        h, b = self.hip, self.b
        h.rmsnorm(b["x"], self.gain, 1e-6)
        h.matmul(self.y, self.w, b["x"])
        h.rope(b["q"], b["table"], POS, H, HD)
        h.attention(self.att, b["q"], b["k"], b["v"], POS, H, HD, KVH)
        h.silu_mul(b["gate"], b["up"])

    def results(self):
        h = self.hip
        return [h.read(self.b["x"]), h.read(self.y), h.read(self.b["q"]), h.read(self.att), h.read(self.b["gate"])]


def test_graph_replays_match_eager(hip):
    data = _inputs()
    w = hip.upload(Tensor((2048, HIDDEN), normal_bf16(2048 * HIDDEN, 202, "gw")))
    gain = hip.upload(Tensor((HIDDEN,), normal_bf16(HIDDEN, 203, "gg")))
    eager = _Run(hip, data, w, gain)
    eager.load()
    eager.calls()
    want = eager.results()
    # The eager attention agrees with the oracle, so the comparison below pins the replays too.
    q = ref.rope(data["q"], data["table"], POS, H, HD)
    np.testing.assert_allclose(want[3], ref.attention(q, data["k"], data["v"], POS, H, HD, KVH), rtol=1e-4, atol=1e-5)

    run = _Run(hip, data, w, gain)
    hip.graph_begin()
    try:
        run.calls()
    finally:
        graph = hip.graph_end()
    for replay in range(3):
        run.load()  # restores the inputs the sequence overwrites (eager work between replays)
        eager.load()
        eager.calls()
        hip.synchronize()
        graph.launch()
        got = run.results()
        for name, g, e in zip(["rmsnorm", "matmul", "rope", "attention", "silu_mul"], got, want):
            assert np.array_equal(g, e), f"replay {replay}: {name} differs from the eager call"
    graph.free()


def test_capture_refuses_host_and_allocating_calls(hip):
    b = hip.alloc(16)
    hip.graph_begin()
    try:
        for call in (lambda: hip.alloc(4), lambda: hip.read(b), lambda: hip.write(b, np.zeros(16, np.float32)),
                     lambda: hip.synchronize(), lambda: hip.timer_begin(), lambda: hip.argmax(b), lambda: b.free()):
            with pytest.raises(Exception, match="captur"):
                call()
    finally:
        graph = hip.graph_end()
    # Everything works again after the capture: the empty graph replays, b is still valid.
    graph.launch()
    hip.write(b, np.arange(16, dtype=np.float32))
    assert np.array_equal(hip.read(b), np.arange(16, dtype=np.float32))
    graph.free()
    b.free()
