"""CPU tests of the trainer-shaped generation path (grpo_mi355x.grpo).

The reference trainer (``src/grpo/trainer.py:329-463``) loops micro-batches of
4 rows per prompt and slices ``outputs[j, prompt_len:]``, which drops the first
``prompt_len`` tokens of the paged decode's ``[B, max_new_tokens]`` return.
These tests drive the counterpart with a stand-in decode (no GPU) and check
that every generated token reaches the decoded text, in the reference's order.
"""

from types import SimpleNamespace

import pytest
import torch

from grpo_mi355x.grpo.generation import generate_group_token_ids, generate_responses


class _Tok:
    pad_token_id = 0
    eos_token_id = 2

    def decode(self, ids, skip_special_tokens=True):
        return " ".join(str(int(t)) for t in ids if not (skip_special_tokens and int(t) in (0, 2)))


class _StubDecode:
    """Returns ``[B, max_new_tokens]`` like ``paged_kv_decode_model``: row b
    generates 1000*b + 1, 1000*b + 2, ... and stops after ``stop[b]`` tokens."""

    def __init__(self):
        self.calls = []

    def __call__(self, model, ids, attention_mask=None, max_new_tokens=0, **kw):
        self.calls.append((ids.clone(), attention_mask.clone(), max_new_tokens, kw))
        B = ids.shape[0]
        out = torch.full((B, max_new_tokens), kw["pad_token_id"], dtype=torch.long)
        for b in range(B):
            n = 3 + (b % 4)
            out[b, :n] = torch.arange(1, n + 1) + 1000 * b
        return out


def _batch():
    # two prompts, left padded: lengths 5 and 3
    ids = torch.tensor([[11, 12, 13, 14, 15], [0, 0, 21, 22, 23]])
    mask = torch.tensor([[1, 1, 1, 1, 1], [0, 0, 1, 1, 1]])
    return ids, mask


def test_one_call_for_all_prompts_and_samples_keeps_every_token():
    ids, mask = _batch()
    dec = _StubDecode()
    rows = generate_group_token_ids(None, ids, mask, group_size=8, max_new_tokens=12,
                                    do_sample=True, temperature=0.7, top_p=0.9,
                                    pad_token_id=0, eos_token_id=2, decode_fn=dec)
    assert len(dec.calls) == 1                 # not 2 prompts x 2 micro-batches of 4
    got_ids, got_mask, max_new, kw = dec.calls[0]
    assert got_ids.shape == (16, 5) and max_new == 12
    assert kw["do_sample"] and kw["temperature"] == 0.7 and kw["top_p"] == 0.9
    # prompt-major: rows 0-7 are prompt 0, rows 8-15 prompt 1 (left padding re-applied)
    assert torch.equal(got_ids[:8], ids[0].expand(8, -1))
    assert torch.equal(got_ids[8:, 2:], ids[1, 2:].expand(8, -1))
    assert torch.equal(got_mask[8:], mask[1].expand(8, -1))
    assert len(rows) == 16
    for b, r in enumerate(rows):
        n = 3 + (b % 4)
        assert r[:n].tolist() == [1000 * b + i for i in range(1, n + 1)]
    # the reference's slice would have lost the first prompt_len tokens of every row
    ref_slice = [r[5 if b < 8 else 3:] for b, r in enumerate(rows)]
    assert any(len(s) < len(r) and s.tolist() != r.tolist() for s, r in zip(ref_slice, rows))


def test_generate_responses_reads_the_trainer_fields():
    ids, mask = _batch()
    dec = _StubDecode()
    import grpo_mi355x.grpo.generation as gen

    trainer = SimpleNamespace(
        model=SimpleNamespace(eval=lambda: None), tokenizer=_Tok(), device="cpu",
        group_sampler=SimpleNamespace(group_size=4),
        config=SimpleNamespace(training=SimpleNamespace(
            max_response_length=10, generation_do_sample=True, generation_temperature=0.7,
            generation_top_p=0.9)))
    orig = gen._default_decode
    gen._default_decode = lambda: dec
    try:
        texts = generate_responses(trainer, ids, mask)
    finally:
        gen._default_decode = orig
    assert len(texts) == 8
    assert texts[0] == "1 3"         # 1, 2 (eos skipped), 3
    assert texts[5] == "5001 5002 5003 5004"
    assert dec.calls[0][3]["eos_token_id"] == 2


def test_import_error_falls_back_to_generate_and_slices_the_prompt():
    ids, mask = _batch()

    def no_backend(*a, **k):
        raise ImportError("no HIP")

    class _Gen:
        def generate(self, input_ids, attention_mask, max_new_tokens, **kw):
            n = input_ids.shape[1]
            resp = torch.arange(100, 100 + max_new_tokens).expand(input_ids.shape[0], -1)
            return torch.cat([input_ids, resp + n], dim=1)

    rows = generate_group_token_ids(_Gen(), ids, mask, group_size=2, max_new_tokens=4,
                                    pad_token_id=0, decode_fn=no_backend)
    assert [r.tolist() for r in rows] == [[105, 106, 107, 108]] * 2 + [[103, 104, 105, 106]] * 2


def test_group_size_must_be_positive():
    ids, mask = _batch()
    with pytest.raises(ValueError):
        generate_group_token_ids(None, ids, mask, 0, 4, decode_fn=_StubDecode())


def test_pad_token_id_none_pads_with_zero_and_generate_keeps_none():
    """A tokenizer without a pad id: the paged decode pads stopped rows with 0
    (the left padding's id), and the model.generate fallback still receives
    None so it applies its own default."""
    ids, mask = _batch()
    dec = _StubDecode()
    rows = generate_group_token_ids(None, ids, mask, group_size=2, max_new_tokens=8,
                                    pad_token_id=None, decode_fn=dec)
    assert dec.calls[0][3]["pad_token_id"] == 0
    assert all(int(r[-1]) == 0 for r in rows)
    seen = {}

    def no_backend(*a, **k):
        raise ImportError("no HIP")

    class _Gen:
        def generate(self, input_ids, attention_mask, max_new_tokens, **kw):
            seen.update(kw)
            return torch.cat([input_ids, input_ids[:, :1].expand(-1, max_new_tokens)], dim=1)

    generate_group_token_ids(_Gen(), ids, mask, group_size=2, max_new_tokens=4,
                             pad_token_id=None, decode_fn=no_backend)
    assert "pad_token_id" in seen and seen["pad_token_id"] is None
