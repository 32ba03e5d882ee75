"""Loading a model from a Hugging Face directory (model/model.rs:40-77,
model/config.rs, model/weights.rs) through th_config_load / th_model_load.

Checkpoints are written here with the `safetensors` package (the format's
reference implementation) from the same seeded weights the other tests
upload directly, so a loaded model must give bit-identical logits to one
built from those tensors, and the transformers fixtures' logits through a
checkpoint directory.
"""

from __future__ import annotations

import json

import numpy as np
import pytest

from oracle import ref
from titania_amd import QWEN3_TINY, InvalidArgument, TH_PATH_FUSED, TH_PATH_OPS, synth
from titania_amd.config import Config
from titania_amd.model import Model, State
from util import load_fixture

# The published config.json of Qwen/Qwen3-0.6B (keys the loader ignores
# included), as a Hugging Face checkpoint directory holds it.
QWEN3_06B_CONFIG = {
    "architectures": ["Qwen3ForCausalLM"], "attention_bias": False, "attention_dropout": 0.0,
    "bos_token_id": 151643, "eos_token_id": 151645, "head_dim": 128, "hidden_act": "silu",
    "hidden_size": 1024, "initializer_range": 0.02, "intermediate_size": 3072,
    "max_position_embeddings": 40960, "max_window_layers": 28, "model_type": "qwen3",
    "num_attention_heads": 16, "num_hidden_layers": 28, "num_key_value_heads": 8, "rms_norm_eps": 1e-06,
    "rope_scaling": None, "rope_theta": 1000000, "sliding_window": None, "tie_word_embeddings": True,
    "torch_dtype": "bfloat16", "transformers_version": "4.51.0", "use_cache": True,
    "use_sliding_window": False, "vocab_size": 151936,
}


def _write_config(path, cfg: dict):
    path.write_text(json.dumps(cfg, indent=2))


def test_config_load_qwen3_06b(tmp_path):
    p = tmp_path / "config.json"
    _write_config(p, QWEN3_06B_CONFIG)
    c = Config.load(p)
    assert (c.hidden_size, c.intermediate_size, c.num_hidden_layers, c.num_attention_heads,
            c.num_key_value_heads, c.head_dim(), c.vocab_size) == (1024, 3072, 28, 16, 8, 128, 151936)
    assert c.tie_word_embeddings
    # f32 fields: the decimal parsed as f64, then rounded to f32 (serde_json).
    assert c.rms_norm_eps == float(np.float32(1e-6)) and c.rope_theta == 1e6


def test_config_load_defaults(tmp_path):
    """head_dim absent or null -> hidden / heads (config.rs:32-35);
    tie_word_embeddings absent -> false (config.rs:22-24)."""
    cfg = {k: v for k, v in QWEN3_06B_CONFIG.items() if k not in ("head_dim", "tie_word_embeddings")}
    cfg["hidden_size"] = 2048
    p = tmp_path / "config.json"
    _write_config(p, cfg)
    c = Config.load(p)
    assert c.head_dim() == 128 and not c.tie_word_embeddings
    cfg["head_dim"] = None
    _write_config(p, cfg)
    assert Config.load(p).head_dim() == 128


def test_config_load_json_forms(tmp_path):
    """Escapes, nesting, exponents and whitespace the JSON grammar allows."""
    text = ('{"_name_or_path": "Qwen\\/Qwen3 \\u00e9\\ud83d\\ude00", "rope_scaling": {"type": "x", "f": [1, 2.5e0]},\n'
            '\t"hidden_size" : 1024, "intermediate_size": 3072, "num_hidden_layers": 28,'
            '"num_attention_heads": 16, "num_key_value_heads": 8, "rms_norm_eps": 1E-6,'
            '"rope_theta": 1.0e6, "vocab_size": 151936, "tie_word_embeddings": false}')
    p = tmp_path / "config.json"
    p.write_text(text)
    c = Config.load(p)
    assert c.rms_norm_eps == float(np.float32(1e-6)) and c.rope_theta == 1e6 and not c.tie_word_embeddings


@pytest.mark.parametrize("edit,match", [
    (lambda c: c.pop("vocab_size"), "missing field `vocab_size`"),
    (lambda c: c.update(hidden_size=1024.0), "`hidden_size` is not an unsigned integer"),
    (lambda c: c.update(num_hidden_layers=-1), "`num_hidden_layers` is not an unsigned integer"),
    (lambda c: c.update(rope_theta="1e6"), "`rope_theta` is not a number"),
    (lambda c: c.update(tie_word_embeddings=1), "`tie_word_embeddings` is not a bool"),
])
def test_config_load_errors(tmp_path, edit, match):
    cfg = dict(QWEN3_06B_CONFIG)
    edit(cfg)
    p = tmp_path / "config.json"
    _write_config(p, cfg)
    with pytest.raises(InvalidArgument, match=match):
        Config.load(p)


@pytest.mark.parametrize("text", ['{"hidden_size": 1024,}', '{"a": tru}', '[1, 2', '{"a": "\\x"}', '{} {}',
                                  '{"a": 01}', '{"a": "\\ud800"}'])
def test_config_load_rejects_malformed_json(tmp_path, text):
    p = tmp_path / "config.json"
    p.write_text(text)
    with pytest.raises(InvalidArgument, match="config.json"):
        Config.load(p)


def test_config_load_missing_file(tmp_path):
    with pytest.raises(InvalidArgument, match="No such file"):
        Config.load(tmp_path / "config.json")


# ---- whole checkpoints (GPU) ----

def _config_dict(c: Config) -> dict:
    return {"hidden_size": c.hidden_size, "intermediate_size": c.intermediate_size,
            "num_hidden_layers": c.num_hidden_layers, "num_attention_heads": c.num_attention_heads,
            "num_key_value_heads": c.num_key_value_heads, "head_dim": c.head_dim(),
            "rms_norm_eps": c.rms_norm_eps, "rope_theta": c.rope_theta, "vocab_size": c.vocab_size,
            "tie_word_embeddings": c.tie_word_embeddings, "model_type": "qwen3"}


def _save_checkpoint(d, cfg: Config, tensors: dict, dtype_override: dict | None = None, drop=()):
    import torch
    from safetensors.torch import save_file

    out = {}
    for name, t in tensors.items():
        if name in drop:
            continue
        bits = np.ascontiguousarray(t.data, dtype=np.uint16).reshape(t.shape)
        x = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)
        if dtype_override and name in dtype_override:
            x = x.to(dtype_override[name])
        out[name] = x
    save_file(out, str(d / "model.safetensors"), metadata={"format": "pt"})
    _write_config(d / "config.json", _config_dict(cfg))


@pytest.mark.gpu
@pytest.mark.parametrize("tied,qk_norm", [(True, True), (False, True), (True, False)])
def test_model_load_matches_uploaded(hip, tmp_path, tied, qk_norm):
    from dataclasses import replace

    cfg = replace(QWEN3_TINY, tie_word_embeddings=tied, qk_norm=qk_norm)
    w = synth.weights(cfg, seed=21, random_gains=True)
    _save_checkpoint(tmp_path, cfg, w)
    loaded = Model.load(hip, tmp_path)
    assert loaded.config.hidden_size == cfg.hidden_size and loaded.config.tie_word_embeddings == tied
    direct = Model(hip, cfg, w)
    prompt = synth.prompt(10, cfg.vocab_size, seed=2)
    for path in (TH_PATH_OPS, TH_PATH_FUSED):
        a, b = State(loaded, 16), State(direct, 16)
        got = loaded.forward(a, prompt, 0, path)
        exp = direct.forward(b, prompt, 0, path)
        assert np.array_equal(got, exp)
        a.close()
        b.close()
    r = ref.RefModel(cfg, w)
    exp = r.forward(r.state(16), prompt, 0)
    st = State(loaded, 16)
    assert float(np.max(np.abs(loaded.forward(st, prompt, 0, TH_PATH_OPS) - exp))) <= 1e-4
    st.close()
    direct.close()
    loaded.close()


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["tied", "untied"])
def test_model_load_transformers_fixture(hip, tmp_path, name):
    """A checkpoint directory of the transformers fixture's weights reproduces
    transformers' logits at every position."""
    cfg, meta, tokens, logits = load_fixture(name)
    w = synth.weights(cfg, seed=meta["seed"], random_gains=meta["random_gains"])
    _save_checkpoint(tmp_path, cfg, w)
    m = Model.load(hip, tmp_path)
    st = State(m, len(tokens))
    for i in range(len(tokens)):
        got = m.forward(st, tokens[i:i + 1], i, TH_PATH_FUSED)
        assert float(np.max(np.abs(got - logits[i]))) <= 1e-4, i
    st.close()
    m.close()


@pytest.mark.gpu
def test_model_load_errors(hip, tmp_path):
    import torch

    cfg = QWEN3_TINY
    w = synth.weights(cfg, seed=1)
    d1 = tmp_path / "f32"
    d1.mkdir()
    _save_checkpoint(d1, cfg, w, dtype_override={"model.layers.1.mlp.up_proj.weight": torch.float32})
    with pytest.raises(InvalidArgument, match="tensor 'model.layers.1.mlp.up_proj.weight' is F32, expected BF16"):
        Model.load(hip, d1)
    d2 = tmp_path / "missing"
    d2.mkdir()
    _save_checkpoint(d2, cfg, w, drop=("model.norm.weight",))
    with pytest.raises(InvalidArgument, match="missing tensor 'model.norm.weight'"):
        Model.load(hip, d2)
    d3 = tmp_path / "truncated"
    d3.mkdir()
    _save_checkpoint(d3, cfg, w)
    blob = (d3 / "model.safetensors").read_bytes()
    (d3 / "model.safetensors").write_bytes(blob[: len(blob) // 2])
    with pytest.raises(InvalidArgument, match="out of range"):
        Model.load(hip, d3)
    d4 = tmp_path / "empty"
    d4.mkdir()
    with pytest.raises(InvalidArgument, match="config.json"):
        Model.load(hip, d4)
