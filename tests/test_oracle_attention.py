"""CPU checks that pin the paged-KV oracle (addressing, append, attention, decode loop).

* addressing/append: brute force against a dense reconstruction with shuffled
  block tables and ragged lengths;
* attention: torch ``scaled_dot_product_attention`` in float64 on the gathered
  dense K/V (an independent library routine), plus closed-form special cases;
* decode loop: the dense recompute model of the reference's
  ``tests/test_triton_performance.py:152-219`` must emit the same greedy tokens.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits
from oracle.decode import paged_kv_decode
from oracle.paged import append_kv, gather_kv, paged_attention_decode

from conftest import rng


def make_paged(g, ctx_lens, hkv, d, bs, extra_blocks=3):
    """Dense per-sequence K/V scattered into a shuffled paged pool."""
    nblk = [-(-c // bs) for c in ctx_lens]
    total = sum(nblk) + extra_blocks
    perm = g.permutation(total)
    max_blocks = max(max(nblk), 1) + 1
    tables = np.zeros((len(ctx_lens), max_blocks), np.int32)
    kc = np.zeros((total, hkv, bs, d), np.uint16)
    vc = np.zeros_like(kc)
    dense_k, dense_v = [], []
    cur = 0
    for b, c in enumerate(ctx_lens):
        tables[b, :nblk[b]] = perm[cur:cur + nblk[b]]
        tables[b, nblk[b]:] = perm[cur + nblk[b] - 1] if nblk[b] else 0
        cur += nblk[b]
        k = f32_to_bf16_bits(g.standard_normal((c, hkv, d)))
        v = f32_to_bf16_bits(g.standard_normal((c, hkv, d)))
        for t in range(c):  # scatter one token at a time (brute force)
            kc[tables[b, t // bs], :, t % bs, :] = k[t]
            vc[tables[b, t // bs], :, t % bs, :] = v[t]
        dense_k.append(k)
        dense_v.append(v)
    return kc, vc, tables, dense_k, dense_v


def test_gather_matches_dense():
    g = rng(10)
    ctx = [37, 1, 64, 100]
    kc, vc, tables, dk, dv = make_paged(g, ctx, 2, 8, 16)
    for b, c in enumerate(ctx):
        assert np.array_equal(gather_kv(kc, tables, b, c), dk[b])
        assert np.array_equal(gather_kv(vc, tables, b, c), dv[b])


def test_append_writes_pre_increment_slot():
    g = rng(11)
    ctx = [5, 16, 31]
    kc, vc, tables, dk, dv = make_paged(g, [c + 1 for c in ctx], 2, 8, 16)
    kn = f32_to_bf16_bits(g.standard_normal((3, 2, 8)))
    vn = f32_to_bf16_bits(g.standard_normal((3, 2, 8)))
    before = kc.copy()
    append_kv(kc, vc, kn, vn, tables, np.array(ctx))
    for b, c in enumerate(ctx):
        assert np.array_equal(kc[tables[b, c // 16], :, c % 16], kn[b])
        assert np.array_equal(vc[tables[b, c // 16], :, c % 16], vn[b])
    changed = np.argwhere(np.any(kc != before, axis=-1))
    assert len(changed) <= 3 * 2  # only the three slots (x heads) moved


@pytest.mark.parametrize("hq,hkv", [(2, 2), (12, 2), (28, 4), (8, 1)])
def test_attention_matches_sdpa(hq, hkv):
    g = rng(12 + hq)
    d, bs = 16, 4
    ctx = [1, 9, 23, 40]
    kc, vc, tables, dk, dv = make_paged(g, ctx, hkv, d, bs)
    q = f32_to_bf16_bits(g.standard_normal((len(ctx), hq, d)))
    scale = 1.0 / math.sqrt(d)
    out = paged_attention_decode(q, kc, vc, tables, np.array(ctx), scale)
    for b, c in enumerate(ctx):
        qq = torch.from_numpy(bf16_bits_to_f32(q[b])).double()[:, None, :]      # [hq,1,d]
        kk = torch.from_numpy(bf16_bits_to_f32(dk[b])).double().permute(1, 0, 2)  # [hkv,c,d]
        vv = torch.from_numpy(bf16_bits_to_f32(dv[b])).double().permute(1, 0, 2)
        kk = kk.repeat_interleave(hq // hkv, 0)
        vv = vv.repeat_interleave(hq // hkv, 0)
        ref = F.scaled_dot_product_attention(qq, kk, vv, scale=scale)[:, 0, :].numpy()
        assert np.abs(out[b] - ref).max() <= 1e-6 * max(1.0, np.abs(ref).max())


def test_attention_special_cases():
    g = rng(13)
    d, bs = 8, 4
    kc, vc, tables, dk, dv = make_paged(g, [1, 12, 12, 0], 2, d, bs)
    q = f32_to_bf16_bits(g.standard_normal((4, 4, d)))
    q[2] = 0  # zero query -> uniform weights -> mean of V
    out = paged_attention_decode(q, kc, vc, tables, np.array([1, 12, 12, 0]), 0.5)
    # ctx = 1 -> output = v_0 of the head's KV head
    v0 = bf16_bits_to_f32(dv[0][0])
    assert np.allclose(out[0], np.repeat(v0, 2, axis=0), atol=1e-7)
    mean_v = bf16_bits_to_f32(dv[2]).astype(np.float64).mean(0)
    assert np.allclose(out[2], np.repeat(mean_v, 2, axis=0), atol=1e-6)
    assert np.all(out[3] == 0)  # ctx = 0 -> zeros (masked sum / max(0, 1e-6))


def test_attention_block_permutation_invariance():
    g = rng(14)
    kc, vc, tables, dk, dv = make_paged(g, [50, 33], 2, 8, 4)
    q = f32_to_bf16_bits(g.standard_normal((2, 6, 8)))
    out1 = paged_attention_decode(q, kc, vc, tables, np.array([50, 33]), 0.3)
    # move every block to a new physical slot
    perm = g.permutation(kc.shape[0])
    kc2, vc2 = np.zeros_like(kc), np.zeros_like(vc)
    kc2[perm], vc2[perm] = kc, vc
    out2 = paged_attention_decode(q, kc2, vc2, perm[tables].astype(np.int32),
                                  np.array([50, 33]), 0.3)
    assert np.array_equal(out1, out2)


class TinyPagedModel:
    """The dense recompute model of the reference's
    ``tests/test_triton_performance.py:152-219`` (numpy, float32)."""

    def __init__(self, g, vocab, heads, hd):
        e = heads * hd
        self.embed = g.standard_normal((vocab, e)).astype(np.float32)
        bound = 1 / math.sqrt(e)
        self.wq, self.wk, self.wv = (g.uniform(-bound, bound, (e, e)).astype(np.float32) for _ in range(3))
        self.wo = g.uniform(-bound, bound, (vocab, e)).astype(np.float32)
        self.heads, self.hd = heads, hd

    def project(self, tok):
        x = self.embed[tok]
        sh = x.shape[:-1] + (self.heads, self.hd)
        return (x @ self.wq.T).reshape(sh), (x @ self.wk.T).reshape(sh), (x @ self.wv.T).reshape(sh)

    def qkv_for_decode(self, tok):
        return self.project(tok)

    def logits_from_attn(self, attn):
        return attn.reshape(attn.shape[0], -1) @ self.wo.T

    def generate(self, ids, steps):
        toks = ids.copy()
        out = []
        scale = 1 / math.sqrt(self.hd)
        for _ in range(steps):
            q, k, v = self.project(toks)
            bf = lambda a: bf16_bits_to_f32(f32_to_bf16_bits(a))
            ql, k, v = bf(q[:, -1]), bf(k), bf(v)
            s = (ql[:, None] * k).sum(-1) * scale          # [B, S, H]
            s = s.transpose(0, 2, 1)                         # [B, H, S]
            w = np.exp(s - s.max(-1, keepdims=True))
            w /= w.sum(-1, keepdims=True)
            attn = (w[..., None] * v.transpose(0, 2, 1, 3)).sum(-2)
            nxt = self.logits_from_attn(attn).argmax(-1)
            out.append(nxt)
            toks = np.concatenate([toks, nxt[:, None]], 1)
        return np.stack(out, 1)


def test_decode_loop_matches_dense_generate():
    """Port of test_triton_paged_kv_decode_matches_generate on the oracle."""
    g = rng(7)
    vocab, heads, hd, prompt, new, bs = 32, 2, 8, 3, 3, 4
    m = TinyPagedModel(g, vocab, heads, hd)
    ids = g.integers(0, vocab, (1, prompt))
    max_blocks = math.ceil((prompt - 1 + new + 1) / bs)
    kc = np.zeros((max_blocks, heads, bs, hd), np.uint16)
    vc = np.zeros_like(kc)
    tables = np.arange(max_blocks, dtype=np.int32)[None]
    _, kp, vp = m.project(ids[:, :-1])
    for pos in range(prompt - 1):
        kc[tables[0, pos // bs], :, pos % bs] = f32_to_bf16_bits(kp[0, pos])
        vc[tables[0, pos // bs], :, pos % bs] = f32_to_bf16_bits(vp[0, pos])
    got = paged_kv_decode(ids, kc, vc, tables, np.array([prompt - 1]), m.qkv_for_decode,
                          m.logits_from_attn, max_new_tokens=new, temperature=0.0, top_p=1.0,
                          do_sample=False, eos_token_id=None, pad_token_id=0)
    assert np.array_equal(got, m.generate(ids, new))


def test_decode_loop_finished_rows_emit_first_prompt_token():
    g = rng(8)
    m = TinyPagedModel(g, 16, 2, 8)
    ids = g.integers(0, 16, (2, 3))
    kc = np.zeros((8, 2, 4, 8), np.uint16)
    vc = np.zeros_like(kc)
    tables = np.array([[0, 1, 2, 3], [4, 5, 6, 7]], np.int32)
    first = paged_kv_decode(ids, kc.copy(), vc.copy(), tables, np.array([2, 2]), m.qkv_for_decode,
                            m.logits_from_attn, max_new_tokens=1, do_sample=False)
    eos = int(first[0, 0])
    got = paged_kv_decode(ids, kc, vc, tables, np.array([2, 2]), m.qkv_for_decode,
                          m.logits_from_attn, max_new_tokens=4, do_sample=False,
                          eos_token_id=eos)
    assert got[0, 0] == eos
    assert np.all(got[0, 1:] == ids[0, 0])
