"""Qwen2-shaped NF4+LoRA decode model and the model-level paged decode loop."""
