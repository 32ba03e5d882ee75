"""model/chat.rs `Chat` at the token level, on the hip device.

The conversation stays in the state's caches, so each turn runs the model over
its new tokens only (chat.rs:22-23, `feed` at :189-196), and a reply is
generated on the device until a stop token (chat.rs:132-187 through
th_generate): the logits of the decode never leave the device, and the host
learns of the stop a few steps at a time. What `Chat` adds around this (the
tokenizer, ChatML text of the turns, tool-call parsing, streaming text) is host
work the caller keeps; here the caller passes token ids.
"""

from __future__ import annotations

import numpy as np

from ._lib import TH_KV_F32, TH_PATH_FUSED
from .model import Model, State


class Chat:
    """A conversation of up to max_len tokens with `model`; greedy, or drawn by
    `sampler` (titania_amd.Sampler)."""

    def __init__(self, model: Model, max_len: int, sampler=None, kv_dtype: int = TH_KV_F32):
        self.model = model
        self.state = State(model, max_len, kv_dtype)
        self.sampler = sampler
        self.len = 0  # tokens in the conversation so far (chat.rs:30-31)

    def close(self) -> None:
        self.state.close()

    def tokens(self) -> int:
        return self.len

    def feed(self, tokens) -> None:
        """chat.rs:189-196: runs the tokens through the model at the end of the
        conversation (the logits stay on the device for the next reply)."""
        t = np.ascontiguousarray(tokens, dtype=np.uint32).reshape(-1)
        if self.len + t.size > self.state.max_len:
            raise ValueError("the conversation no longer fits in the context window")
        if t.size:
            self.model.forward(self.state, t, self.len, TH_PATH_FUSED, want_logits=False)
        self.len += t.size

    def generate(self, prompt, stop, end, max_tokens: int) -> np.ndarray:
        """chat.rs:132-187: feeds the reply's opening `prompt`, then picks and
        feeds tokens until one in `stop` (not fed), at most max_tokens, then
        feeds `end` (the turn's closing tokens). Returns the reply's tokens,
        the stop token included when one ended it."""
        self.feed(prompt)
        room = self.state.max_len - self.len
        toks = self.model.decode_until(self.state, self.len, min(int(max_tokens), room), stop, self.sampler)
        stopped = toks.size > 0 and int(toks[-1]) in {int(s) for s in np.asarray(stop).reshape(-1)}
        self.len += toks.size - (1 if stopped else 0)
        if not stopped and toks.size < max_tokens:
            # The reply wanted to go on past the end of the cache (chat.rs:190-192).
            raise ValueError("the conversation no longer fits in the context window")
        self.feed(end)
        return toks


__all__ = ["Chat"]
