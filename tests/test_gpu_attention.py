"""GPU parity: paged KV append (bit-exact) and paged GQA decode attention.

Attention tolerance: ``max|out - ref| <= 1e-2 * max|ref|`` (north star: bf16
tolerance, fp32 accumulation); the kernels actually land near 1e-6 and the
tests also assert ``<= 1e-4`` to catch partial mistakes (a dropped block, a
wrong head mapping) that could hide under 1e-2.
"""

import math

import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits
from oracle.paged import append_kv, paged_attention_decode as ref_attn

from conftest import from_bf16, rel_err, rng, to_dev_bf16

pytestmark = pytest.mark.gpu


def _ops():
    from grpo_mi355x.kernels import ops

    return ops


def paged_case(seed, ctx_lens, hq, hkv, d, bs, slack_blocks=8, table_width=None):
    """Shuffled paged pool (cfg 1 recipe): Sum ceil(ctx/bs) + slack blocks, randperm."""
    g = rng(seed)
    nblk = [-(-c // bs) for c in ctx_lens]
    total = sum(nblk) + slack_blocks
    perm = g.permutation(total).astype(np.int32)
    width = table_width or max(max(nblk), 1)
    tables = np.zeros((len(ctx_lens), width), np.int32)
    cur = 0
    for b, nb in enumerate(nblk):
        tables[b, :nb] = perm[cur:cur + nb]
        cur += nb
    kc = f32_to_bf16_bits(g.standard_normal((total, hkv, bs, d)))
    vc = f32_to_bf16_bits(g.standard_normal((total, hkv, bs, d)))
    q = f32_to_bf16_bits(g.standard_normal((len(ctx_lens), hq, d)))
    return q, kc, vc, tables, np.array(ctx_lens, np.int32)


def run_attn(dev, q, kc, vc, tables, ctx, scale, out_dtype=torch.float32):
    out = _ops().paged_attention_decode(
        to_dev_bf16(q, dev), to_dev_bf16(kc, dev), to_dev_bf16(vc, dev),
        torch.from_numpy(tables).to(dev), torch.from_numpy(ctx).to(dev), scale,
        out_dtype=out_dtype)
    torch.cuda.synchronize()
    return out


def check(out, ref):
    out = out.cpu().float().numpy() if isinstance(out, torch.Tensor) else out
    assert np.all(np.isfinite(out))
    err = rel_err(out, ref)
    assert err <= 1e-2
    assert err <= 1e-4, err


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_cfg1_paged_attention(dev, seed):
    """4 seqs, ctx U[512,1024], 12 Q / 2 KV heads, D 128, block 16."""
    g = rng(100 + seed)
    ctx = g.integers(512, 1025, 4).tolist()
    q, kc, vc, tables, cl = paged_case(seed, ctx, 12, 2, 128, 16)
    scale = 1 / math.sqrt(128)
    check(run_attn(dev, q, kc, vc, tables, cl, scale), ref_attn(q, kc, vc, tables, cl, scale))


@pytest.mark.parametrize("hq,hkv", [(1, 1), (2, 1), (8, 2), (12, 2), (28, 4), (8, 1), (14, 2),
                                    (40, 8)])
def test_gqa_ratios(dev, hq, hkv):
    g = rng(hq * 10 + hkv)
    ctx = g.integers(1, 300, 5).tolist()
    q, kc, vc, tables, cl = paged_case(hq + hkv, ctx, hq, hkv, 128, 16)
    s = 1 / math.sqrt(128)
    check(run_attn(dev, q, kc, vc, tables, cl, s), ref_attn(q, kc, vc, tables, cl, s))


def test_edge_lengths_and_many_splits(dev):
    ctx = [0, 1, 15, 16, 17, 31, 32, 33, 4096, 1000, 2]
    q, kc, vc, tables, cl = paged_case(5, ctx, 12, 2, 128, 16, table_width=300)
    s = 1 / math.sqrt(128)
    out = run_attn(dev, q, kc, vc, tables, cl, s)
    ref = ref_attn(q, kc, vc, tables, cl, s)
    check(out, ref)
    assert torch.all(out[0] == 0)  # ctx = 0 -> zeros


def test_large_group_cfg5_shape(dev):
    """cfg 5 shape on a reduced batch: 28 Q / 4 KV heads, ctx U[1024,4096]."""
    g = rng(55)
    ctx = g.integers(1024, 4097, 6).tolist()
    q, kc, vc, tables, cl = paged_case(56, ctx, 28, 4, 128, 16)
    s = 1 / math.sqrt(128)
    check(run_attn(dev, q, kc, vc, tables, cl, s), ref_attn(q, kc, vc, tables, cl, s))


def test_bf16_output_is_rounded_fp32_output(dev):
    g = rng(6)
    ctx = g.integers(1, 700, 8).tolist()
    q, kc, vc, tables, cl = paged_case(6, ctx, 12, 2, 128, 16)
    s = 1 / math.sqrt(128)
    o32 = run_attn(dev, q, kc, vc, tables, cl, s)
    o16 = run_attn(dev, q, kc, vc, tables, cl, s, out_dtype=torch.bfloat16)
    assert np.array_equal(from_bf16(o16), f32_to_bf16_bits(o32.cpu().numpy()))


@pytest.mark.parametrize("d,bs,hq,hkv", [(8, 4, 2, 2), (64, 16, 8, 2), (128, 16, 32, 2),
                                         (96, 8, 6, 3), (256, 16, 4, 1)])
def test_generic_path(dev, d, bs, hq, hkv):
    g = rng(d + bs + hq)
    ctx = g.integers(0, 200, 4).tolist()
    q, kc, vc, tables, cl = paged_case(d * bs, ctx, hq, hkv, d, bs)
    s = 1 / math.sqrt(d)
    check(run_attn(dev, q, kc, vc, tables, cl, s), ref_attn(q, kc, vc, tables, cl, s))


@pytest.mark.parametrize("case", ["cfg1", "edges", "gqa8"])
def test_one_launch_equals_split_plus_merge(dev, case, monkeypatch):
    """The one-launch attention (``grpo_paged_attn_decode_merged``, the default
    of ``ops.paged_attention_decode``) against the split kernel + merge launch
    on the same inputs: float32 and bf16 outputs identical bit for bit (the
    last-arriving split merges in the merge kernel's order and formula), over
    three calls in a row through the same counters, which are back at zero,
    with the XCD check word clear (``attention_handover_check``)."""
    ops = _ops()
    if case == "cfg1":
        ctx = rng(3).integers(512, 1025, 4).tolist()
        q, kc, vc, tables, cl = paged_case(11, ctx, 12, 2, 128, 16)
    elif case == "edges":  # ctx 0 and 1, split boundaries, one long row
        ctx = [0, 1, 15, 16, 17, 639, 640, 641, 4096, 1000, 2]
        q, kc, vc, tables, cl = paged_case(12, ctx, 12, 2, 128, 16, table_width=300)
    else:
        ctx = rng(4).integers(1, 2000, 6).tolist()
        q, kc, vc, tables, cl = paged_case(13, ctx, 32, 4, 128, 16)
    s = 1 / math.sqrt(128)
    want = {}
    monkeypatch.setattr(ops, "ATTN_ONE_LAUNCH", False)
    for dt in (torch.float32, torch.bfloat16):
        want[dt] = run_attn(dev, q, kc, vc, tables, cl, s, out_dtype=dt).cpu()
    monkeypatch.setattr(ops, "ATTN_ONE_LAUNCH", True)
    for call in range(3):
        for dt in (torch.float32, torch.bfloat16):
            print(f"one-launch attention {case} call {call} {dt}", flush=True)
            got = run_attn(dev, q, kc, vc, tables, cl, s, out_dtype=dt).cpu()
            assert torch.equal(got.view(torch.int32 if dt == torch.float32 else torch.int16),
                               want[dt].view(torch.int32 if dt == torch.float32 else torch.int16))
    ops.attention_handover_check(dev)
    cnt, err = ops._attn_merge[torch.device(dev)]
    assert int(err.item()) == 0 and not bool((cnt != 0).any())
    check(want[torch.float32], ref_attn(q, kc, vc, tables, cl, s))


def test_invalid_block_ids_are_skipped(dev):
    q, kc, vc, tables, cl = paged_case(7, [40, 40], 12, 2, 128, 16)
    bad = tables.copy()
    bad[1, 1] = -5  # second block of sequence 1 is invalid -> its tokens are ignored
    out = run_attn(dev, q, kc, vc, bad, cl, 0.1).cpu().numpy()
    ref0 = ref_attn(q[:1], kc, vc, tables[:1], cl[:1], 0.1)
    assert rel_err(out[:1], ref0) <= 1e-4
    assert np.all(np.isfinite(out))


def test_append_bit_exact(dev):
    g = rng(8)
    ctx = [0, 15, 16, 100, 511]
    _, kc, vc, tables, cl = paged_case(8, [c + 1 for c in ctx], 12, 2, 128, 16)
    kn = f32_to_bf16_bits(g.standard_normal((5, 2, 128)))
    vn = f32_to_bf16_bits(g.standard_normal((5, 2, 128)))
    kcd, vcd = to_dev_bf16(kc, dev), to_dev_bf16(vc, dev)
    _ops().paged_kv_append(to_dev_bf16(kn, dev), to_dev_bf16(vn, dev), kcd, vcd,
                           torch.from_numpy(tables).to(dev),
                           torch.from_numpy(np.array(ctx, np.int32)).to(dev))
    torch.cuda.synchronize()
    append_kv(kc, vc, kn, vn, tables, np.array(ctx))
    assert np.array_equal(from_bf16(kcd), kc) and np.array_equal(from_bf16(vcd), vc)


def test_append_skips_out_of_table_slots(dev):
    _, kc, vc, tables, _ = paged_case(9, [16, 16], 2, 2, 128, 16)
    kcd, vcd = to_dev_bf16(kc, dev), to_dev_bf16(vc, dev)
    g = rng(9)
    kn = to_dev_bf16(f32_to_bf16_bits(g.standard_normal((2, 2, 128))), dev)
    bad_tables = tables.copy()
    bad_tables[1, 0] = 10_000  # block id outside the pool
    _ops().paged_kv_append(kn, kn, kcd, vcd, torch.from_numpy(bad_tables).to(dev),
                           torch.tensor([16, 3], dtype=torch.int32, device=dev))  # row 0: past table
    torch.cuda.synchronize()
    assert np.array_equal(from_bf16(kcd), kc) and np.array_equal(from_bf16(vcd), vc)


def test_decode_loop_matches_dense_generate(dev):
    """Port of the reference's test_triton_paged_kv_decode_matches_generate
    (tests/test_triton_performance.py:136-271): B=1, H=2, D=8, block 4, greedy."""
    from grpo_mi355x.kernels import paged_kv_decode

    torch.manual_seed(7)
    vocab, heads, hd, prompt, new, bs = 32, 2, 8, 3, 3, 4

    class TinyPagedModel(torch.nn.Module):
        def __init__(self):
            super().__init__()
            e = heads * hd
            self.embed = torch.nn.Embedding(vocab, e)
            self.q_proj = torch.nn.Linear(e, e, bias=False)
            self.k_proj = torch.nn.Linear(e, e, bias=False)
            self.v_proj = torch.nn.Linear(e, e, bias=False)
            self.out_proj = torch.nn.Linear(e, vocab, bias=False)

        def _project(self, ids):
            x = self.embed(ids)
            if x.ndim == 2:
                x = x.unsqueeze(1)
            b, s, _ = x.shape
            sh = (b, s, heads, hd)
            return self.q_proj(x).view(sh), self.k_proj(x).view(sh), self.v_proj(x).view(sh)

        def qkv_for_decode(self, ids):
            q, k, v = self._project(ids)
            return q[:, 0], k[:, 0], v[:, 0]

        def logits_from_attn(self, a):
            return self.out_proj(a.reshape(a.shape[0], -1))

        @torch.no_grad()
        def generate(self, ids, steps):
            toks, out = ids, []
            for _ in range(steps):
                q, k, v = self._project(toks)
                ql = q[:, -1].to(torch.bfloat16).float()
                k, v = k.to(torch.bfloat16).float(), v.to(torch.bfloat16).float()
                sc = ((ql[:, None] * k).sum(-1) / math.sqrt(hd)).transpose(1, 2)
                a = (torch.softmax(sc, -1)[..., None] * v.transpose(1, 2)).sum(-2)
                nxt = torch.argmax(self.logits_from_attn(a), -1)
                out.append(nxt)
                toks = torch.cat([toks, nxt[:, None]], 1)
            return torch.stack(out, 1)

    model = TinyPagedModel().to(dev)
    ids = torch.randint(0, vocab, (1, prompt)).to(dev)
    mb = math.ceil((prompt - 1 + new + 1) / bs)
    kc = torch.zeros((mb, heads, bs, hd), device=dev, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    tables = torch.arange(mb, device=dev, dtype=torch.int32)[None]
    with torch.no_grad():
        _, kp, vp = model._project(ids[:, :-1])
    for pos in range(prompt - 1):
        kc[pos // bs, :, pos % bs] = kp[0, pos].to(torch.bfloat16)
        vc[pos // bs, :, pos % bs] = vp[0, pos].to(torch.bfloat16)
    got = paged_kv_decode(None, input_ids=ids, k_cache=kc, v_cache=vc, block_tables=tables,
                          context_lens=torch.full((1,), prompt - 1, dtype=torch.int32, device=dev),
                          qkv_proj_fn=model.qkv_for_decode, logits_fn=model.logits_from_attn,
                          max_new_tokens=new, temperature=0.0, top_p=1.0, do_sample=False,
                          eos_token_id=None, pad_token_id=0, seed=123)
    assert torch.equal(got, model.generate(ids, new))


def test_decode_loop_gqa_fast_path_matches_oracle(dev):
    """Low-level loop, GQA 12/2, D 128, ragged prompts: tokens equal the oracle loop's."""
    from grpo_mi355x.kernels import paged_kv_decode
    from oracle.decode import paged_kv_decode as ref_decode

    g = rng(12)
    vocab, hq, hkv, d, bs, b = 64, 12, 2, 128, 16, 4
    eq = f32_to_bf16_bits(g.standard_normal((vocab, hq, d)))
    ek = f32_to_bf16_bits(g.standard_normal((vocab, hkv, d)))
    ev = f32_to_bf16_bits(g.standard_normal((vocab, hkv, d)))
    wo = g.standard_normal((vocab, hq * d)).astype(np.float32) / math.sqrt(hq * d)
    prompts = [40, 17, 64, 3]
    steps = 6
    width = -(-(max(prompts) + steps + 1) // bs)
    q0, kc, vc, tables, _ = paged_case(13, [p + steps + 1 for p in prompts], hq, hkv, d, bs,
                                       table_width=width)
    ids = g.integers(0, vocab, (b, 1))
    ctx = np.array(prompts, np.int32)

    ref = ref_decode(ids, kc.copy(), vc.copy(), tables, ctx,
                     lambda t: (bf16_bits_to_f32(eq[t]), bf16_bits_to_f32(ek[t]),
                                bf16_bits_to_f32(ev[t])),
                     lambda a: a.reshape(a.shape[0], -1).astype(np.float64) @ wo.T,
                     max_new_tokens=steps, do_sample=False)
    eqd, ekd, evd = (to_dev_bf16(a, dev) for a in (eq, ek, ev))
    wod = torch.from_numpy(wo).to(dev)
    got = paged_kv_decode(None, input_ids=torch.from_numpy(ids).to(dev),
                          k_cache=to_dev_bf16(kc, dev), v_cache=to_dev_bf16(vc, dev),
                          block_tables=torch.from_numpy(tables).to(dev),
                          context_lens=torch.from_numpy(ctx).to(dev),
                          qkv_proj_fn=lambda t: (eqd[t], ekd[t], evd[t]),
                          logits_fn=lambda a: a.reshape(a.shape[0], -1) @ wod.T,
                          max_new_tokens=steps, do_sample=False)
    assert np.array_equal(got.cpu().numpy(), ref)
