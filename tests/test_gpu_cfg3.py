"""BASELINE config 3 on the GPU at the headline shape: Qwen2-1.5B, G = 8.

Hidden 1536, 12 query / 2 KV heads (GQA ratio 6), head_dim 128, MLP 8960,
vocab 151936, NF4 weights + rank-16 LoRA on q/k/v/o, with two transformer
layers instead of 28 so the numpy oracle stays fast; every kernel of the
benchmarked step runs at its real shape: the fused-prologue split attention at
GQA 6, o_proj merging the attention splits of 12 heads while staging x, the
fused gate|up + SiLU units kernel, the split-K RMSNorm consumers, and the
lm_head GEMV + argmax at V = 151936, all replayed from the captured HIP graph.

1. A 512-token prompt is cached by the chunked ``PrefillEngine`` (511 tokens,
   64-token chunks); the oracle computes the same prefill as one pass of 511
   rows sharing the block table.  Cached K/V within 1e-2 of max|x|.
2. G = 8 rows are forked from it (full prompt blocks shared, the partial last
   block copied) and decoded with ragged stops; each row starts from its own
   input token so the rows' trajectories differ.  The oracle steps the active
   rows from the GPU's own cache and tokens: logits within 1e-2 of max|logit|,
   the fused argmax equals the oracle's wherever its top-2 margin exceeds that
   tolerance, the appended K/V rows match, and rows that stopped write nothing.
"""

import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_bits_to_f32
from oracle.decode import Qwen2DecodeOracle

from conftest import rel_err
from model_export import bits, export

pytestmark = pytest.mark.gpu


def _oracle_prefill(oracle, prompt, table_row, nb, cfg):
    """The oracle's cache after ``prompt[:-1]``: one pass of n rows at positions
    0..n-1 that share the table (every row appends before attention)."""
    n = len(prompt) - 1
    L = cfg.num_hidden_layers
    shape = (nb, cfg.num_key_value_heads, 16, cfg.head_dim)
    kcs = [np.zeros(shape, np.uint16) for _ in range(L)]
    vcs = [np.zeros(shape, np.uint16) for _ in range(L)]
    tables = np.tile(np.asarray(table_row, np.int32), (n, 1))
    oracle.step(np.asarray(prompt[:n]), kcs, vcs, tables, np.arange(n), with_logits=False)
    return kcs, vcs


def test_cfg3_headline_shape_prefill_and_ragged_decode_match_oracle(dev):
    from grpo_mi355x.core.kv_pool import PagedKVPool
    from grpo_mi355x.rollout.decode import DecodeEngine, PrefillEngine, prefill
    from grpo_mi355x.rollout.qwen2 import Qwen2Config, build_random_model

    cfg = Qwen2Config.qwen2_1_5b()
    cfg.num_hidden_layers = 2
    model = build_random_model(cfg, dev, seed=31)
    G, bs, P, steps = 8, 16, 512, 5
    g = np.random.default_rng(12)
    prompt = g.integers(0, cfg.vocab_size, P).tolist()
    width = -(-(P + steps + 1) // bs)
    nb = width * (G + 1) + 8
    pool = PagedKVPool(cfg.num_hidden_layers, nb, cfg.num_key_value_heads, cfg.head_dim, bs,
                       device=dev)
    print("cfg3 shape: chunked prefill of 511 tokens", flush=True)
    pre = PrefillEngine(model, pool, 64, width)
    sid = prefill(pre, pool, tuple(prompt), width)
    torch.cuda.synchronize()
    del pre
    w, c = export(model)
    oracle = Qwen2DecodeOracle(w, c)
    prow = pool.blocks[sid]
    kref, vref = _oracle_prefill(oracle, prompt, prow + [-1] * (width - len(prow)), nb, cfg)
    kg, vg = [bits(pool.k[i]) for i in range(2)], [bits(pool.v[i]) for i in range(2)]
    for li in range(cfg.num_hidden_layers):
        for got, ref in ((kg[li], kref[li]), (vg[li], vref[li])):
            a = bf16_bits_to_f32(got[prow]).reshape(-1, bs, cfg.head_dim)
            r = bf16_bits_to_f32(ref[prow]).reshape(-1, bs, cfg.head_dim)
            e = rel_err(a, r)
            print(f"prefill layer {li}: K/V rel err {e:.2e}", flush=True)
            assert e <= 1e-2

    # G rows forked from the cached prompt, ragged stops
    kids = pool.fork(sid, G, reserve_tokens=P + steps)
    pool.free(sid)
    pool.check_invariants()
    limits = np.array([5, 1, 3, 5, 2, 4, 5, 3])
    toks = np.concatenate([[prompt[-1]], g.integers(0, cfg.vocab_size, G - 1)])
    tables = pool.block_table(kids, width)
    tab_np = tables.cpu().numpy()
    eng = DecodeEngine(model, pool, G, width, keep_logits=True)
    start = dict(tokens=torch.from_numpy(toks).to(dev),
                 positions=torch.full((G,), P - 1, device=dev), block_tables=tables.to(dev),
                 limits=torch.from_numpy(limits).to(dev), max_new_tokens=steps)
    eng.start(**start)
    eng.capture()
    eng.start(**start)
    kcs = [bits(pool.k[i]) for i in range(2)]
    vcs = [bits(pool.v[i]) for i in range(2)]
    pos = np.full(G, P - 1, np.int64)
    worst, agree, total = 0.0, 0, 0
    for t in range(steps):
        act = np.flatnonzero(t < limits)
        print(f"cfg3 shape: decode step {t}, active rows {act.tolist()}", flush=True)
        before = [bits(pool.k[i]) for i in range(2)]
        eng.step()
        torch.cuda.synchronize()
        lg = bf16_bits_to_f32(bits(eng.logits))
        lr_bits, nxt = oracle.step(toks[act], kcs, vcs, tab_np[act], pos[act])
        lr = bf16_bits_to_f32(lr_bits)
        new_toks = eng.tokens.cpu().numpy()
        for j, b in enumerate(act):
            worst = max(worst, rel_err(lg[b], lr[j]))
            assert new_toks[b] == int(np.argmax(lg[b]))  # the fused argmax, first max
            srt = np.sort(lr[j])
            if srt[-1] - srt[-2] > 1e-2 * np.abs(lr[j]).max():
                total += 1
                agree += int(new_toks[b] == nxt[j])
        for li in range(2):
            kga, vga = bits(pool.k[li]), bits(pool.v[li])
            for b in range(G):
                blk, off = tab_np[b, pos[b] // bs], pos[b] % bs
                if b in act:
                    for got, ref in ((kga, kcs[li]), (vga, vcs[li])):
                        assert rel_err(bf16_bits_to_f32(got[blk, :, off]),
                                       bf16_bits_to_f32(ref[blk, :, off])) <= 1e-2
                else:  # a stopped row appends nothing
                    assert np.array_equal(kga[blk, :, off], before[li][blk, :, off])
        toks = new_toks.copy()
        pos[act] += 1
    print(f"cfg3 shape: worst logits rel err {worst:.2e}, argmax agree {agree}/{total}",
          flush=True)
    assert worst <= 1e-2, worst
    assert total >= 10 and agree == total
    gen = eng.generated.cpu().numpy()
    for b in range(G):
        assert np.all(gen[b, limits[b]:] == 0)


def test_cfg3_full_depth_rollouts_keep_the_xcd_check_clear(dev):
    """The benchmarked rollout itself -- 28 layers, G = 8, 512-token prompt,
    512 greedy steps from the captured graph -- twice: both give the same
    tokens, every row generates up to its stop and pads after, and the
    in-kernel hand-over of the default path (o_proj's last K slice of a column
    group finishing it) leaves its counters at zero with the XCD check word
    clear over all 28 x 512 layer-steps (``DecodeEngine.verify_handover``)."""
    from grpo_mi355x.core.kv_pool import PagedKVPool
    from grpo_mi355x.rollout.decode import DecodeEngine, PrefillEngine, prefill, prefill_chunk
    from grpo_mi355x.rollout.qwen2 import Qwen2Config, build_random_model

    cfg = Qwen2Config.qwen2_1_5b()
    model = build_random_model(cfg, dev, seed=0)
    G, P, NEW, bs = 8, 512, 512, 16
    g = np.random.default_rng(0)
    stops = g.integers(64, NEW + 1, G).tolist()
    stops[3] = NEW
    prompt = g.integers(0, cfg.vocab_size, P).tolist()
    width = -(-(P + NEW) // bs)
    pool = PagedKVPool(cfg.num_hidden_layers, width * (G + 2), cfg.num_key_value_heads,
                       cfg.head_dim, bs, device=dev)
    print("cfg3 full depth: prefill", flush=True)
    pre = PrefillEngine(model, pool, prefill_chunk(P - 1), width)
    parent = prefill(pre, pool, tuple(prompt), width)
    del pre
    kids = pool.fork(parent, G, reserve_tokens=P + NEW)
    pool.free(parent)
    eng = DecodeEngine(model, pool, G, width)
    assert eng.attn_fused and eng.o_fin
    start = dict(tokens=torch.full((G,), prompt[-1], dtype=torch.int64, device=dev),
                 positions=torch.full((G,), P - 1, device=dev),
                 block_tables=pool.block_table(kids, width, device=dev),
                 limits=torch.tensor(stops, device=dev), max_new_tokens=NEW)
    eng.start(**start)
    eng.capture()
    outs = []
    for rep in range(2):
        print(f"cfg3 full depth: rollout {rep}", flush=True)
        eng.start(**start)
        eng.run(max(stops))
        torch.cuda.synchronize()
        outs.append(eng.generated.cpu().numpy().copy())
        eng.verify_handover()
    assert np.array_equal(outs[0], outs[1])
    for b, s in enumerate(stops):
        assert np.all(outs[0][b, s:] == 0)
    assert len({tuple(r[:64]) for r in outs[0]}) == 1  # one prompt, greedy: equal prefixes


def test_cfg3_full_depth_logits_within_the_rounding_spread(dev):
    """All 28 layers of the Qwen2-1.5B shape against the oracle, one decode step
    of 4 rows forked from a 128-token prompt (cached by the chunked prefill;
    the oracle starts from the same cache).  The 1e-2 bound of the ops holds
    through 2 layers (the test above); through 28 layers the float32
    summation-order differences of the NF4 linears (products exact, >= 97 %
    of outputs bit-identical per linear) compound, so the yardstick is the
    spread between this build's own kernel families on the same inputs: the
    4-row step (folded down_proj, staged norms, o_proj's in-kernel finish)
    against a 12-row and a 32-row engine (split-K down_proj, separate norm
    launches, other K splits).  The oracle's distance must be within twice the
    largest such spread and below 5e-2 of max|logit| (2.9e-2 and 2.8e-2
    measured; 7.4e-3 and 4.2e-3 at 2 layers, 1.7e-2 and 1.2e-2 at 8), and the
    greedy tokens must equal the oracle's wherever its top-2 margin exceeds
    5e-2 of max|logit|."""
    from grpo_mi355x.core.kv_pool import PagedKVPool
    from grpo_mi355x.rollout.decode import DecodeEngine, PrefillEngine, prefill
    from grpo_mi355x.rollout.qwen2 import Qwen2Config, build_random_model

    cfg = Qwen2Config.qwen2_1_5b()
    L = cfg.num_hidden_layers
    model = build_random_model(cfg, dev, seed=7)
    G, bs, P = 4, 16, 128
    g = np.random.default_rng(3)
    prompt = g.integers(0, cfg.vocab_size, P).tolist()
    width = -(-(P + 4) // bs)
    pool = PagedKVPool(L, width * (G + 1) + 8, cfg.num_key_value_heads, cfg.head_dim, bs,
                       device=dev)
    print("cfg3 full depth: prefill", flush=True)
    pre = PrefillEngine(model, pool, 64, width)
    sid = prefill(pre, pool, tuple(prompt), width)
    torch.cuda.synchronize()
    del pre
    kids = pool.fork(sid, G, reserve_tokens=P + 2)
    pool.free(sid)
    tables = pool.block_table(kids, width).cpu()
    toks = np.concatenate([[prompt[-1]], g.integers(0, cfg.vocab_size, G - 1)])
    kcs = [bits(pool.k[i]) for i in range(L)]
    vcs = [bits(pool.v[i]) for i in range(L)]
    print("cfg3 full depth: oracle step", flush=True)
    w, c = export(model)
    oracle = Qwen2DecodeOracle(w, c)
    lo_bits, nxt = oracle.step(toks, kcs, vcs, tables.numpy(), np.full(G, P - 1))
    lo = bf16_bits_to_f32(lo_bits)

    def step0(B):
        print(f"cfg3 full depth: {B}-row engine", flush=True)
        eng = DecodeEngine(model, pool, B, width, keep_logits=True)
        tok = torch.zeros(B, dtype=torch.int64)
        tok[:G] = torch.from_numpy(toks)
        tbl = torch.full((B, width), -1, dtype=torch.int32)
        tbl[:G] = tables
        lim = torch.zeros(B, dtype=torch.int32)
        lim[:G] = 1  # rows past G idle: no append, length 0
        eng.start(tok.to(dev), torch.full((B,), P - 1, device=dev), tbl.to(dev), lim.to(dev), 1)
        eng.step()
        torch.cuda.synchronize()
        eng.verify_handover()
        return bf16_bits_to_f32(bits(eng.logits))[:G]

    fams = {B: step0(B) for B in (G, 12, 32)}

    def dist(a, b):
        return max(rel_err(a[i], b[i]) for i in range(G))

    spread = max(dist(fams[G], fams[12]), dist(fams[G], fams[32]), dist(fams[12], fams[32]))
    to_oracle = dist(fams[G], lo)
    print(f"cfg3 full depth: oracle distance {to_oracle:.2e}, kernel-family spread {spread:.2e}",
          flush=True)
    assert to_oracle <= 5e-2 and to_oracle <= 2 * spread
    for B, lg in fams.items():
        for i in range(G):
            srt = np.sort(lo[i])
            if srt[-1] - srt[-2] > 5e-2 * np.abs(lo[i]).max():
                assert int(np.argmax(lg[i])) == int(nxt[i]), (B, i)
