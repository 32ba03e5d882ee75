"""Writes tests/golden/hf_qwen3_*.npz: logits of Hugging Face transformers'
Qwen3ForCausalLM (an implementation independent of the reference and of this
package) on small Qwen3-shaped models with the synthetic weights of
titania_amd.synth, for pinning the oracle's forward pass.

The model is built from an in-memory Qwen3Config and loaded with our weights
(bf16 values held in float32), run in float32 with eager attention. Greedy
tokens are produced by re-running the whole sequence each step (no cache), and
the logits of every position of the final sequence are stored.

Run from the repository root:  python tests/golden/make_hf_qwen3.py
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from titania_amd import synth  # noqa: E402
from titania_amd.config import Config  # noqa: E402

CASES = {
    # Tied embeddings, random RMSNorm gains (so that every gain is exercised).
    "tied": (Config(hidden_size=512, intermediate_size=1536, num_hidden_layers=2, num_attention_heads=4,
                    num_key_value_heads=2, vocab_size=1000, head_dim_=128), 11, 12, 8),
    # A separate output projection, a wider GQA group and a third layer.
    "untied": (Config(hidden_size=512, intermediate_size=1024, num_hidden_layers=3, num_attention_heads=8,
                      num_key_value_heads=2, vocab_size=777, head_dim_=128, tie_word_embeddings=False), 23, 9, 6),
}


def hf_model(c: Config, tensors: dict):
    from transformers import Qwen3Config, Qwen3ForCausalLM

    hc = Qwen3Config(
        vocab_size=c.vocab_size, hidden_size=c.hidden_size, intermediate_size=c.intermediate_size,
        num_hidden_layers=c.num_hidden_layers, num_attention_heads=c.num_attention_heads,
        num_key_value_heads=c.num_key_value_heads, head_dim=c.head_dim(), hidden_act="silu",
        max_position_embeddings=4096, rms_norm_eps=c.rms_norm_eps, tie_word_embeddings=c.tie_word_embeddings,
        rope_parameters={"rope_type": "default", "rope_theta": c.rope_theta}, attention_bias=False,
        use_sliding_window=False,
    )
    hc._attn_implementation = "eager"
    model = Qwen3ForCausalLM(hc).to(torch.float32).eval()
    state = {name: torch.from_numpy(synth.bf16_to_f32(t.data).reshape(t.shape)) for name, t in tensors.items()}
    if c.tie_word_embeddings:
        state["lm_head.weight"] = state["model.embed_tokens.weight"]
    missing, unexpected = model.load_state_dict(state, strict=False)
    missing = [m for m in missing if "rotary_emb" not in m]
    assert not missing and not unexpected, (missing, unexpected)
    return model


def make(name: str) -> Path:
    c, seed, n_prompt, steps = CASES[name]
    tensors = synth.weights(c, seed=seed, random_gains=True)
    prompt = synth.prompt(n_prompt, c.vocab_size, seed=seed)
    model = hf_model(c, tensors)
    seq = [int(t) for t in prompt]
    with torch.no_grad():
        for _ in range(steps):
            logits = model(torch.tensor([seq])).logits[0, -1]
            seq.append(int(torch.argmax(logits)))
        logits = model(torch.tensor([seq])).logits[0].numpy().astype(np.float32)
    meta = {"config": {k: v for k, v in c.__dict__.items()}, "seed": seed, "random_gains": True,
            "prompt_len": n_prompt, "steps": steps,
            "generator": "transformers Qwen3ForCausalLM, float32, eager attention, no KV cache"}
    out = Path(__file__).with_name(f"hf_qwen3_{name}.npz")
    np.savez_compressed(out, tokens=np.array(seq, dtype=np.uint32), logits=logits, meta=json.dumps(meta))
    return out


if __name__ == "__main__":
    torch.manual_seed(0)
    for case in CASES:
        print(make(case))
