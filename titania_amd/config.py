"""Model architecture (model/config.rs:9-36) and the Qwen3 shapes used here."""

from __future__ import annotations

from dataclasses import dataclass, replace

from ._lib import ThConfig


@dataclass(frozen=True)
class Config:
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    vocab_size: int
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    tie_word_embeddings: bool = True
    head_dim_: int | None = None  # `head_dim` in config.json; None derives it
    qk_norm: bool = True          # whether layers carry q_norm / k_norm (model.rs:55-56)

    def head_dim(self) -> int:
        """model/config.rs:32-35: explicit, or hidden / heads."""
        return self.head_dim_ if self.head_dim_ is not None else self.hidden_size // self.num_attention_heads

    def to_c(self) -> ThConfig:
        return ThConfig(
            self.hidden_size, self.intermediate_size, self.num_hidden_layers, self.num_attention_heads,
            self.num_key_value_heads, self.head_dim(), self.vocab_size, self.rms_norm_eps, self.rope_theta,
            1 if self.tie_word_embeddings else 0,
        )

    @classmethod
    def from_c(cls, c: ThConfig, qk_norm: bool = True) -> "Config":
        return cls(int(c.hidden_size), int(c.intermediate_size), int(c.num_hidden_layers),
                   int(c.num_attention_heads), int(c.num_key_value_heads), int(c.vocab_size),
                   float(c.rms_norm_eps), float(c.rope_theta), bool(c.tie_word_embeddings), int(c.head_dim), qk_norm)

    @classmethod
    def load(cls, path) -> "Config":
        """model/config.rs:29-31 `Config::load` of a Hugging Face config.json
        (th_config_load; no GPU needed)."""
        from ._lib import check, lib
        import ctypes as C
        out = ThConfig()
        check(lib().th_config_load(str(path).encode(), C.byref(out)))
        return cls.from_c(out)

    def with_layers(self, n: int) -> "Config":
        return replace(self, num_hidden_layers=n)

    def weight_bytes_per_token(self) -> int:
        """bf16 weight bytes one decode step streams: every layer, the final norm,
        one embedding row and the output projection."""
        H, I, hd = self.hidden_size, self.intermediate_size, self.head_dim()
        qd, kvd = self.num_attention_heads * hd, self.num_key_value_heads * hd
        per_layer = 2 * (2 * H + qd * H + 2 * kvd * H + H * qd + 3 * I * H)
        if self.qk_norm:
            per_layer += 2 * 2 * hd
        return self.num_hidden_layers * per_layer + 2 * H + 2 * H + 2 * self.vocab_size * H


QWEN3_0_6B = Config(
    hidden_size=1024, intermediate_size=3072, num_hidden_layers=28, num_attention_heads=16,
    num_key_value_heads=8, vocab_size=151936, head_dim_=128,
)

QWEN3_4B = Config(
    hidden_size=2560, intermediate_size=9728, num_hidden_layers=36, num_attention_heads=32,
    num_key_value_heads=8, vocab_size=151936, head_dim_=128,
)

# A small model of the same family for quick end-to-end checks.
QWEN3_TINY = Config(
    hidden_size=512, intermediate_size=1536, num_hidden_layers=2, num_attention_heads=4,
    num_key_value_heads=2, vocab_size=1000, head_dim_=128,
)
