"""model/sampler.rs `Sampler`, drawing on the device.

Same parameters and generator as the reference: the top_k most likely tokens,
then the smallest set of those whose probability reaches top_p, at
`temperature` (0: the most likely token), with xorshift64* seeded by
max(seed, 1). `Hip.sample` draws from a logits buffer (th_sample); passing the
sampler to `Model.decode` draws every token of a decode on the device
(th_decode_sample). `rng` is the generator state, advanced by each draw.
"""

from __future__ import annotations


class Sampler:
    def __init__(self, temperature: float, top_k: int, top_p: float, seed: int):
        self.temperature = float(temperature)
        self.top_k = int(top_k)
        self.top_p = float(top_p)
        self.rng = max(int(seed), 1) & 0xFFFFFFFFFFFFFFFF

    def sample(self, hip, logits) -> int:
        """Sampler::sample (model/sampler.rs:21-59) over a device buffer."""
        return hip.sample(logits, self)
