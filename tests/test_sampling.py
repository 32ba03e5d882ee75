"""On-device sampling (th_sample, th_decode_sample) against the oracle's
restatement of model/sampler.rs (pinned in test_oracle.py).

The device runs the reference's arithmetic in its order (one thread, left
folds), so draws and generator states match the oracle exactly; device expf
and glibc expf may differ by an ulp, which could move a draw only when the
uniform lands within ~1e-7 of a cumulative boundary (not for these seeds).
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import ref
from titania_amd import InvalidArgument, Sampler, TH_PATH_FUSED, synth

pytestmark = pytest.mark.gpu


def _logits(n, seed, ties=False):
    x = np.random.default_rng(seed).standard_normal(n).astype(np.float32) * 3.0
    if ties:
        # Equal values inside and at the edge of the top k: lower index first.
        order = np.argsort(-x, kind="stable")
        x[order[1:4]] = x[order[1]]
        x[order[18:22]] = x[order[18]]
    return x


@pytest.mark.parametrize("n,t,k,p,ties", [
    (1000, 0.7, 20, 0.8, False),
    (151936, 0.7, 20, 0.8, False),
    (151936, 1.3, 256, 0.95, False),
    (151936, 0.5, 64, 1.0, True),
    (300, 1.0, 0, 0.9, False),      # top_k 0 clamps to 1
    (200, 1.0, 1000, 0.9, False),   # top_k clamps to the 200 values
    (8192 * 3 + 5, 2.0, 50, 0.3, True),
])
def test_sample_matches_oracle(hip, n, t, k, p, ties):
    x = _logits(n, n + k, ties)
    buf = hip.alloc(n)
    hip.write(buf, x)
    dev, cpu = Sampler(t, k, p, 42), ref.Sampler(t, k, p, 42)
    got = [dev.sample(hip, buf) for _ in range(40)]
    exp = [cpu.sample(x) for _ in range(40)]
    assert got == exp
    assert dev.rng == cpu.state
    buf.free()


def test_sample_temperature_zero_is_argmax(hip):
    x = _logits(5000, 3)
    x[[10, 4000]] = x.max() + 1.0
    buf = hip.alloc(x.size)
    hip.write(buf, x)
    s = Sampler(0.0, 40, 0.9, 9)
    assert s.sample(hip, buf) == 10
    assert s.rng == 9  # no draw at temperature 0
    buf.free()


def test_sample_rejects(hip):
    buf = hip.alloc(1000)
    hip.write(buf, _logits(1000, 1))
    with pytest.raises(InvalidArgument, match="top_k"):
        Sampler(1.0, 257, 0.9, 1).sample(hip, buf)
    with pytest.raises(InvalidArgument, match="top_p"):
        Sampler(1.0, 20, 0.0, 1).sample(hip, buf)
    buf.free()
