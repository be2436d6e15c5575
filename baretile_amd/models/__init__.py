"""Models on baretile_amd tensors: llama (the Llama family, which SmolLM belongs to)."""
