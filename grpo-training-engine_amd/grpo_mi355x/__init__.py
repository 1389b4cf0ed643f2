"""grpo_mi355x -- MI355X-native GRPO rollout decode path.

Hand-written HIP kernels for gfx950 (``csrc/``, built into
``_native/libgrpo_hip.so`` and bound through the C ABI of
``include/grpo_hip.h``) behind the reference's operator surface:

* ``grpo_mi355x.kernels``  -- mirror of ``src/triton_kernels`` (registry,
  ``paged_kv_decode``, ``lora_fused_forward``);
* ``grpo_mi355x.core``     -- mirror of ``src/core`` (``ManualLoRALayer``,
  ``inject_lora_layers``, the NF4 weight container, the paged KV block pool);
* ``grpo_mi355x.rollout``  -- a Qwen2-shaped NF4+LoRA decode model and the
  model-level paged decode loop;
* ``grpo_mi355x.grpo``     -- the trainer's generation call site.
"""

__version__ = "0.1.0"
