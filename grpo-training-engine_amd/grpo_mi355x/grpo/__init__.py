"""The GRPO trainer's generation call site (``src/grpo/trainer.py:329-463``).

``generate_responses(trainer, input_ids, attention_mask)`` is a drop-in body
for ``GRPOTrainerLoop.generate_responses``; ``generate_group_token_ids`` is the
same path returning token ids.
"""

from .generation import generate_group_token_ids, generate_responses

__all__ = ["generate_group_token_ids", "generate_responses"]
