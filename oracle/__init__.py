"""CPU oracle of the Qwen3 forward pass (test infrastructure; see ref.py)."""
