"""The GRPO trainer's generation call site (``src/grpo/trainer.py:329-463``)."""
