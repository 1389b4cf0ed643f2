"""Chunked paged prefill (``PrefillEngine``, and ``GemmPrefillEngine`` on the
NF4 GEMM for wide chunks) against the oracle.

The reference prefills with one causal forward of ``prompt[:-1]`` and scatters
its K/V into the paged cache (src/triton_kernels/paged_kv.py:547-586).  The
prefill engine runs ``chunk`` prompt positions of one sequence per pass (K/V
of the whole chunk appended before attention, row i attending over i + 1
tokens).  Checked here: the K/V cache it leaves equals, within the bf16 bar
of the decode tests (1e-2 of max|x|), the cache of the oracle's token-by-token
pass over the same prompt, and is no further from it than twice the
teacher-forced decode path's cache; rows past a short last chunk write
nothing; the greedy tokens decoded after a prefill equal the oracle's.  The
GEMM prefill meets the same bars and, at the Qwen2-1.5B shape, leaves the
cache of the 64-token chunked prefill to the decode bar.
"""

import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_bits_to_f32
from oracle.decode import Qwen2DecodeOracle

from conftest import rel_err
from model_export import bits, export

pytestmark = pytest.mark.gpu


def _model(dev, layers=2, seed=3):
    from grpo_mi355x.rollout.qwen2 import Qwen2Config, build_random_model

    cfg = Qwen2Config.tiny(layers=layers, heads=4, kv_heads=2, head_dim=128, inter=1024,
                           vocab=1024)
    return build_random_model(cfg, dev, seed=seed)


def _oracle_cache(oracle, prompt, layers, width):
    """The oracle's K/V caches (blocks 0 .. width-1 in order) after one step per
    token of ``prompt[:-1]``, and their block table."""
    kcs = [np.zeros((width, 2, 16, 128), np.uint16) for _ in range(layers)]
    vcs = [np.zeros_like(k) for k in kcs]
    tab = np.arange(width, dtype=np.int32)[None]
    for t in range(len(prompt) - 1):
        oracle.step(np.array([prompt[t]]), kcs, vcs, tab, np.array([t]))
    return kcs, vcs, tab


def _seq(x, pool, sid, n):
    """[Hkv, n, D] bf16 bits of sequence ``sid``'s first n slots in cache ``x``."""
    return np.concatenate([x[b] for b in pool.blocks[sid]], axis=1)[:, :n]


@pytest.mark.parametrize("chunk", [16, 64])
def test_chunked_prefill_cache_matches_oracle(dev, chunk):
    """Error of the chunked cache against the oracle within the bar and within
    twice that of the teacher-forced decode path (B = 1 engine, one token per
    graph step) on the same prompt, plus 2e-3 of max|x|: the two differ only in
    the split-K summation order of M = chunk versus M = 1 linears."""
    from grpo_mi355x.core.kv_pool import PagedKVPool
    from grpo_mi355x.rollout.decode import DecodeEngine, PrefillEngine, prefill

    layers, width = 2, 4
    model = _model(dev, layers=layers, seed=11)
    w, c = export(model)
    prompt = np.random.default_rng(7).integers(0, 1000, 45).tolist()
    n = len(prompt) - 1  # 44 cached tokens: chunks of 16 give 16 + 16 + 12
    # a decoy sequence first, so the prompt's blocks are not blocks 0..3
    pool = PagedKVPool(layers, 3 * width, 2, 128, 16, device=dev)
    decoy = pool.allocate(width * 16)
    pre = PrefillEngine(model, pool, chunk, width)
    print(f"chunked prefill: {n} tokens, chunk {chunk}", flush=True)
    sid = prefill(pre, pool, tuple(prompt), width)
    torch.cuda.synchronize()
    assert pool.length[sid] == n
    # slots past the prompt and the decoy's blocks are untouched (masked rows)
    for li in range(layers):
        for t in pool.layer(li):
            x = bits(t)
            assert not np.concatenate([x[b] for b in pool.blocks[sid]], axis=1)[:, n:].any()
            assert not x[pool.blocks[decoy]].any()
    pool.free(decoy)
    eng1 = DecodeEngine(model, pool, 1, width)
    eng1.capture()
    tf = prefill(eng1, pool, tuple(prompt), width)
    torch.cuda.synchronize()
    kcs, vcs, _ = _oracle_cache(Qwen2DecodeOracle(w, c), prompt, layers, width)
    for li in range(layers):
        for name, t, ref_c in (("k", pool.layer(li)[0], kcs[li]), ("v", pool.layer(li)[1], vcs[li])):
            x = bits(t)
            ref = bf16_bits_to_f32(np.concatenate(list(ref_c), axis=1)[:, :n])
            e_ch = rel_err(bf16_bits_to_f32(_seq(x, pool, sid, n)), ref)
            e_tf = rel_err(bf16_bits_to_f32(_seq(x, pool, tf, n)), ref)
            print(f"layer {li} {name}: chunked {e_ch:.2e}, teacher-forced {e_tf:.2e}",
                  flush=True)
            assert e_ch <= 1e-2 and e_ch <= 2 * e_tf + 2e-3


@pytest.mark.parametrize("chunk", [128, 192])
def test_gemm_prefill_cache_matches_oracle(dev, chunk):
    """The wide-chunk prefill on the NF4 GEMM (``GemmPrefillEngine``): 149
    cached tokens as 128 + 21 or in one 192-row pass.  Its cache is within the
    bar of the oracle's and within twice the teacher-forced path's error plus
    2e-3; rows past the prompt and another sequence's blocks are untouched."""
    from grpo_mi355x.core.kv_pool import PagedKVPool
    from grpo_mi355x.rollout.decode import DecodeEngine, GemmPrefillEngine, prefill

    layers, width = 3, 10
    model = _model(dev, layers=layers, seed=17)
    w, c = export(model)
    prompt = np.random.default_rng(21).integers(0, 1000, 150).tolist()
    n = len(prompt) - 1
    pool = PagedKVPool(layers, 3 * width, 2, 128, 16, device=dev)
    decoy = pool.allocate(width * 16)
    pre = GemmPrefillEngine(model, pool, chunk, width)
    print(f"GEMM prefill: {n} tokens, chunk {chunk}", flush=True)
    sid = prefill(pre, pool, tuple(prompt), width)
    torch.cuda.synchronize()
    assert pool.length[sid] == n
    for li in range(layers):
        for t in pool.layer(li):
            x = bits(t)
            assert not np.concatenate([x[b] for b in pool.blocks[sid]], axis=1)[:, n:].any()
            assert not x[pool.blocks[decoy]].any()
    pool.free(decoy)
    eng1 = DecodeEngine(model, pool, 1, width)
    eng1.capture()
    tf = prefill(eng1, pool, tuple(prompt), width)
    torch.cuda.synchronize()
    kcs, vcs, _ = _oracle_cache(Qwen2DecodeOracle(w, c), prompt, layers, width)
    for li in range(layers):
        for name, t, ref_c in (("k", pool.layer(li)[0], kcs[li]), ("v", pool.layer(li)[1], vcs[li])):
            x = bits(t)
            ref = bf16_bits_to_f32(np.concatenate(list(ref_c), axis=1)[:, :n])
            e_g = rel_err(bf16_bits_to_f32(_seq(x, pool, sid, n)), ref)
            e_tf = rel_err(bf16_bits_to_f32(_seq(x, pool, tf, n)), ref)
            print(f"layer {li} {name}: GEMM prefill {e_g:.2e}, teacher-forced {e_tf:.2e}",
                  flush=True)
            assert e_g <= 1e-2 and e_g <= 2 * e_tf + 2e-3


def test_gemm_prefill_matches_chunked_prefill_at_qwen2_shape(dev):
    """Qwen2-1.5B layer shapes (2 layers, vocab cut to 4096), a 511-token
    prompt: the one-pass GEMM prefill (512 rows) leaves the cache of the
    64-token chunked prefill to the decode bar, and the factory picks it."""
    from grpo_mi355x.core.kv_pool import PagedKVPool
    from grpo_mi355x.rollout.decode import (GemmPrefillEngine, PrefillEngine, prefill,
                                            prefill_engine)
    from grpo_mi355x.rollout.qwen2 import Qwen2Config, build_random_model

    cfg = Qwen2Config(num_hidden_layers=2, vocab_size=4096)
    model = build_random_model(cfg, dev, seed=2)
    prompt = np.random.default_rng(3).integers(0, 4096, 512).tolist()
    n, width = len(prompt) - 1, 33
    pool = PagedKVPool(2, 2 * width, cfg.num_key_value_heads, cfg.head_dim, 16, device=dev)
    gp = prefill_engine(model, pool, n, width)
    assert isinstance(gp, GemmPrefillEngine) and gp.B == 512
    print("Qwen2-1.5B-shaped prefill, 511 tokens: GEMM (512 rows) and chunked (64)", flush=True)
    a = prefill(gp, pool, tuple(prompt), width)
    b = prefill(PrefillEngine(model, pool, 64, width), pool, tuple(prompt), width)
    torch.cuda.synchronize()
    for li in range(2):
        for t in pool.layer(li):
            x = bits(t)
            e = rel_err(bf16_bits_to_f32(_seq(x, pool, a, n)), bf16_bits_to_f32(_seq(x, pool, b, n)))
            print(f"layer {li}: GEMM vs chunked prefill {e:.2e}", flush=True)
            assert e <= 1e-2


def test_chunked_prefill_across_block_table_width(dev):
    """80 prompt tokens in chunks of 32 (32 + 32 + 16) over six blocks: the
    chunked cache agrees with the teacher-forced one to the decode bar."""
    from grpo_mi355x.core.kv_pool import PagedKVPool
    from grpo_mi355x.rollout.decode import DecodeEngine, PrefillEngine, prefill

    layers, width = 2, 6
    model = _model(dev, layers=layers, seed=13)
    prompt = np.random.default_rng(9).integers(0, 1000, 81).tolist()
    pool = PagedKVPool(layers, 2 * width, 2, 128, 16, device=dev)
    eng1 = DecodeEngine(model, pool, 1, width)
    eng1.capture()
    print("teacher-forced and chunked prefill: 80 tokens", flush=True)
    a = prefill(eng1, pool, tuple(prompt), width)
    b = prefill(PrefillEngine(model, pool, 32, width), pool, tuple(prompt), width)
    torch.cuda.synchronize()
    n = len(prompt) - 1
    for li in range(layers):
        for t in pool.layer(li):
            x = bits(t)
            e = rel_err(bf16_bits_to_f32(_seq(x, pool, b, n)), bf16_bits_to_f32(_seq(x, pool, a, n)))
            print(f"layer {li}: chunked vs teacher-forced {e:.2e}", flush=True)
            assert e <= 1e-2


def test_decode_after_multi_chunk_prefill_matches_oracle(dev):
    """The drop-in with a 150-token prompt (149 cached tokens: one 192-row pass
    of the GEMM prefill), then greedy decode: tokens equal the oracle's
    token-by-token loop."""
    from grpo_mi355x.kernels import paged_kv_decode

    model = _model(dev, layers=2, seed=5)
    w, c = export(model)
    oracle = Qwen2DecodeOracle(w, c)
    prompt = np.random.default_rng(4).integers(0, 1000, 150).tolist()
    new = 6
    ids = torch.tensor([prompt] * 2, device=dev)
    print("paged_kv_decode after a 149-token GEMM prefill", flush=True)
    got = paged_kv_decode(model, ids, attention_mask=torch.ones_like(ids), max_new_tokens=new,
                          do_sample=False, pad_token_id=0, eos_token_id=None).cpu().numpy()
    width = -(-(len(prompt) + new) // 16)
    kcs, vcs, tab = _oracle_cache(oracle, prompt, 2, width)
    tok, ref = prompt[-1], []
    for t in range(len(prompt) - 1, len(prompt) - 1 + new):
        _, nxt = oracle.step(np.array([tok]), kcs, vcs, tab, np.array([t]))
        tok = int(nxt[0])
        ref.append(tok)
    assert np.array_equal(got[0], ref) and np.array_equal(got[1], ref)
