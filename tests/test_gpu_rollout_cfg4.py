"""BASELINE config 4 on the GPU: a ragged group with blocks allocated and freed as rows finish.

G = 32 rows = 4 prompts x 8 samples, prompt lengths uniform in [128, 256] (config 4
uses [128, 512]; shortened so the oracle's token-by-token prefill stays quick),
response lengths from a long-tail lognormal (median 20, sigma 0.75, capped at 64;
config 4: median 200, capped at 1024), block size 16, on a tiny Qwen2-shaped
NF4+LoRA model.  Greedy decoding makes the 8 samples of a prompt identical up to
their stops, so the oracle decodes each prompt once.

Checked: every row's tokens equal the oracle's greedy tokens up to its stop
(compared up to the first step whose oracle top-2 logit margin is inside the
bf16 tolerance, after which a near-tie may legitimately flip) and pad after it;
the pool's invariants hold at every chunk; blocks are reserved one chunk ahead
(peak use below an up-front reservation of every row's maximum); every block
is back on the free list at the end.
"""

import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_bits_to_f32
from oracle.decode import Qwen2DecodeOracle

from model_export import bits, export

pytestmark = pytest.mark.gpu

PAD = 0


def _model(dev, seed=9):
    from grpo_mi355x.rollout.qwen2 import Qwen2Config, build_random_model

    cfg = Qwen2Config.tiny(layers=2, heads=4, kv_heads=2, head_dim=128, inter=1024, vocab=1024)
    return build_random_model(cfg, dev, seed=seed)


def _workload(seed=4, prompts=4, samples=8, new=64):
    g = np.random.default_rng(seed)
    lens = g.integers(128, 257, prompts)
    plist = [g.integers(1, 1000, n).tolist() for n in lens]
    stops = np.minimum(new, np.maximum(1, np.round(g.lognormal(np.log(20.0), 0.75,
                                                                prompts * samples)))).astype(int)
    rows = [plist[i // samples] for i in range(prompts * samples)]
    return plist, rows, stops.tolist(), new


def _oracle_greedy(oracle, prompt, new):
    """Greedy tokens after ``prompt`` and whether each step's top-2 margin is safe."""
    width = -(-(len(prompt) + new) // 16)
    kcs = [np.zeros((width, 2, 16, 128), np.uint16) for _ in range(2)]
    vcs = [np.zeros_like(k) for k in kcs]
    tab = np.arange(width, dtype=np.int32)[None]
    tok, out, safe = prompt[0], [], []
    for t in range(len(prompt) - 1 + new):
        tok_in = prompt[t] if t < len(prompt) else tok
        logits, nxt = oracle.step(np.array([tok_in]), kcs, vcs, tab, np.array([t]))
        if t >= len(prompt) - 1:
            lr = bf16_bits_to_f32(logits[0])
            srt = np.sort(lr)
            safe.append(srt[-1] - srt[-2] > 1e-2 * np.abs(lr).max())
            out.append(int(nxt[0]))
            tok = int(nxt[0])
    return np.array(out), np.array(safe)


def test_cfg4_ragged_group_matches_oracle(dev):
    from grpo_mi355x.kernels import paged_kv_decode

    model = _model(dev)
    plist, rows, stops, new = _workload()
    L = max(len(r) for r in rows)
    ids = torch.full((len(rows), L), PAD, dtype=torch.int64)
    mask = torch.zeros_like(ids)
    for b, r in enumerate(rows):  # left padding, as a tokenizer batch would give
        ids[b, L - len(r):] = torch.tensor(r)
        mask[b, L - len(r):] = 1
    got = paged_kv_decode(model, ids.to(dev), attention_mask=mask.to(dev), max_new_tokens=new,
                          do_sample=False, pad_token_id=PAD, eos_token_id=None,
                          stop_lengths=stops).cpu().numpy()
    assert got.shape == (len(rows), new)
    w, c = export(model)
    oracle = Qwen2DecodeOracle(w, c)
    refs = [_oracle_greedy(oracle, p, max(s for r, s in zip(rows, stops) if r is p or r == p))
            for p in plist]
    compared = 0
    for b, (r, stop) in enumerate(zip(rows, stops)):
        ref, safe = refs[plist.index(r)]
        unsafe = np.flatnonzero(~safe[:stop])
        n = int(unsafe[0]) if unsafe.size else stop  # tokens before the first near-tie
        assert np.array_equal(got[b, :n], ref[:n]), (b, got[b, :n], ref[:n])
        assert np.all(got[b, stop:] == PAD)
        compared += n
    # a random tiny model has small top-2 margins: a near-tie ends the comparison of
    # its prompt's rows, so at least half of the tokens must be compared
    assert compared >= 0.5 * sum(stops)


def test_cfg4_blocks_allocated_ahead_and_freed(dev):
    from grpo_mi355x.core.kv_pool import PagedKVPool
    from grpo_mi355x.rollout.decode import DecodeEngine, PrefillEngine, prefill, prefill_chunk

    model = _model(dev)
    plist, rows, stops, new = _workload(seed=5)
    width = -(-(max(len(p) for p in plist) + new) // 16)
    B = len(rows)
    nblocks = len(plist) * width + B * (width + 1)
    pool = PagedKVPool(2, nblocks, 2, 128, 16, device=dev)
    pre = PrefillEngine(model, pool, prefill_chunk(max(len(p) for p in plist) - 1), width)
    parents = [prefill(pre, pool, tuple(p), width) for p in plist]
    sids = [pool.fork(parents[plist.index(r)], 1, reserve_tokens=len(r))[0] for r in rows]
    for p in parents:
        pool.free(p)
    pool.check_invariants()
    upfront = sum(-(-(len(r) + new) // 16) for r in rows)  # private reservation per row
    eng = DecodeEngine(model, pool, B, width)
    start = dict(tokens=torch.tensor([r[-1] for r in rows], device=dev),
                 positions=torch.tensor([len(r) - 1 for r in rows], device=dev),
                 block_tables=pool.block_table(sids, width, device=dev),
                 limits=torch.tensor(stops, device=dev), max_new_tokens=new)
    eng.start(**start)
    eng.capture()
    eng.start(**start)
    stats = eng.run_paged(sids, new, check_invariants=True)
    torch.cuda.synchronize()
    assert stats["steps"] <= max(stops) + 16
    assert stats["peak_blocks"] < upfront
    assert pool.num_free == pool.num_blocks and not pool.blocks
    pool.check_invariants()
    gen = eng.generated.cpu().numpy()
    for b, s in enumerate(stops):
        assert np.all(gen[b, s:] == 0) and np.all(gen[b, :s] >= 0)


@pytest.mark.parametrize("compact", [False, True])
def test_cfg4_headline_shape_ragged_group_matches_oracle(dev, compact):
    """Config 4's recipe on the Qwen2-1.5B shape (two layers): G = 32 rows = 4
    prompts x 8 samples, prompts U[128, 512], lognormal stops (sigma 0.75,
    median scaled to 24 and capped at 48 steps for test time), chunked prefill
    per prompt, rows forked from it, blocks reserved a chunk ahead and freed as
    rows stop (``run_paged``), greedy tokens from the captured graph.

    The oracle follows each prompt's GPU tokens (teacher forcing, the 4 prompts
    batched as 4 rows of one step): at every step of every row the GPU's token
    equals the oracle's argmax wherever the oracle's top-2 margin exceeds 1e-2
    of max|logit|; the 8 samples of a prompt are equal up to their stops and
    pad after; every block returns to the free list.  With ``compact`` the rows
    still decoding move to a 16- and then an 8-row engine once they fit
    (``run_paged(compact=...)``), so their later tokens come from those
    engines' steps."""
    from grpo_mi355x.core.kv_pool import PagedKVPool
    from grpo_mi355x.rollout.decode import DecodeEngine, PrefillEngine, prefill
    from grpo_mi355x.rollout.qwen2 import Qwen2Config, build_random_model

    cfg = Qwen2Config.qwen2_1_5b()
    cfg.num_hidden_layers = 2
    model = build_random_model(cfg, dev, seed=41)
    g = np.random.default_rng(8)
    prompts, samples, new = 4, 8, 48
    lens = g.integers(128, 513, prompts)
    plist = [g.integers(0, cfg.vocab_size, n).tolist() for n in lens]
    stops = np.minimum(new, np.maximum(1, np.round(
        g.lognormal(np.log(24.0), 0.75, prompts * samples)))).astype(int)
    rows = [plist[i // samples] for i in range(prompts * samples)]
    B, bs = len(rows), 16
    width = -(-(int(lens.max()) + new) // bs)
    pool = PagedKVPool(2, prompts * width + B * (width + 1), cfg.num_key_value_heads,
                       cfg.head_dim, bs, device=dev)
    print(f"cfg4 shape: prompts {lens.tolist()}, stops {stops.tolist()}", flush=True)
    pre = PrefillEngine(model, pool, 64, width)
    parents = [prefill(pre, pool, tuple(p), width) for p in plist]
    del pre
    sids = [pool.fork(parents[i // samples], 1, reserve_tokens=len(r))[0]
            for i, r in enumerate(rows)]
    # the oracle's caches: the GPU's prefilled prompt blocks
    ptab = np.full((prompts, width + 4), -1, np.int32)
    for i, p in enumerate(parents):
        bl = pool.blocks[p]
        ptab[i, :len(bl)] = bl
    kcs = [bits(pool.k[li]) for li in range(2)]
    vcs = [bits(pool.v[li]) for li in range(2)]
    for p in parents:
        pool.free(p)
    eng = DecodeEngine(model, pool, B, width)
    start = dict(tokens=torch.tensor([r[-1] for r in rows], device=dev),
                 positions=torch.tensor([len(r) - 1 for r in rows], device=dev),
                 block_tables=pool.block_table(sids, width, device=dev),
                 limits=torch.from_numpy(stops).to(dev), max_new_tokens=new)
    eng.start(**start)
    eng.capture()
    eng.start(**start)
    stats = eng.run_paged(sids, new, check_invariants=True,
                          compact=eng.compaction_engines((16, 8)) if compact else None)
    torch.cuda.synchronize()
    if compact:  # 10 rows left after 32 steps
        assert stats["engines"] == [32, 16]
    assert pool.num_free == pool.num_blocks and not pool.blocks
    gen = eng.generated.cpu().numpy()
    for b in range(B):
        lead = (b // samples) * samples
        s = min(stops[b], stops[lead])
        assert np.array_equal(gen[b, :s], gen[lead, :s])
        assert np.all(gen[b, stops[b]:] == PAD)
    # teacher-forced oracle along each prompt's longest row
    w, c = export(model)
    oracle = Qwen2DecodeOracle(w, c)
    longest = [max(range(i * samples, (i + 1) * samples), key=lambda b: stops[b])
               for i in range(prompts)]
    # oracle tables: the shared full prompt blocks, then fresh blocks past the pool's
    nb_o = pool.num_blocks
    tab = np.full((prompts, width + 4), -1, np.int32)
    extra = nb_o
    for i in range(prompts):
        n = len(plist[i]) - 1
        full = n // bs
        tab[i, :full] = ptab[i, :full]
        for j in range(full, width + 4):
            tab[i, j] = extra
            extra += 1
    for li in range(2):
        pad_blocks = np.zeros((extra - nb_o,) + kcs[li].shape[1:], np.uint16)
        kcs[li] = np.concatenate([kcs[li], pad_blocks])
        vcs[li] = np.concatenate([vcs[li], pad_blocks.copy()])
    for i in range(prompts):  # the partial last prompt block, copied
        n = len(plist[i]) - 1
        if n % bs:
            for li in range(2):
                kcs[li][tab[i, n // bs]] = kcs[li][ptab[i, n // bs]]
                vcs[li][tab[i, n // bs]] = vcs[li][ptab[i, n // bs]]
    pos = np.array([len(p) - 1 for p in plist], np.int64)
    toks = np.array([p[-1] for p in plist])
    compared = agree = 0
    for t in range(int(max(stops[b] for b in longest))):
        act = np.array([i for i in range(prompts) if t < stops[longest[i]]])
        lr_bits, nxt = oracle.step(toks[act], kcs, vcs, tab[act], pos[act])
        lr = bf16_bits_to_f32(lr_bits)
        for j, i in enumerate(act):
            srt = np.sort(lr[j])
            if srt[-1] - srt[-2] > 1e-2 * np.abs(lr[j]).max():
                compared += 1
                agree += int(gen[longest[i], t] == nxt[j])
        toks[act] = gen[[longest[i] for i in act], t]  # teacher forcing on the GPU's tokens
        pos[act] += 1
    print(f"cfg4 shape: {stats}, tokens compared {compared}, agree {agree}", flush=True)
    assert compared >= 0.5 * sum(stops[b] for b in longest)
    assert agree == compared


def _oracle_check_steps(oracle, prompt, gen, steps, width, chunk=256):
    """Teacher-forced oracle at decode steps ``steps`` (increasing) of one row:
    tokens by position are the prompt, then the GPU's generated tokens; the
    oracle caches every position before the checked one by a batched causal
    prefill (rows of one step call sharing the row's block table), then runs
    the checked position with logits.  Returns [(step, oracle next token,
    safe top-2 margin)]."""
    n = len(prompt)
    toks = list(prompt) + [int(t) for t in gen]
    kcs = [np.zeros((width, 2, 16, 128), np.uint16) for _ in range(2)]
    vcs = [np.zeros_like(k) for k in kcs]
    done, out = 0, []
    for s in steps:
        pos = n - 1 + s  # the step's input token and position
        while done < pos:
            j = np.arange(done, min(pos, done + chunk))
            oracle.step(np.array([toks[i] for i in j]), kcs, vcs,
                        np.zeros((len(j), width), np.int32) + np.arange(width, dtype=np.int32),
                        j, with_logits=False)
            done = int(j[-1]) + 1
        logits, nxt = oracle.step(np.array([toks[pos]]), kcs, vcs,
                                  np.arange(width, dtype=np.int32)[None], np.array([pos]))
        done = pos + 1
        lr = bf16_bits_to_f32(logits[0])
        srt = np.sort(lr)
        out.append((s, int(nxt[0]), bool(srt[-1] - srt[-2] > 1e-2 * np.abs(lr).max())))
        print(f"  oracle step {s} (position {pos}): {out[-1]}", flush=True)
    return out


@pytest.mark.timeout(600)
@pytest.mark.parametrize("compact", [False, True])
def test_cfg4_long_tail_rows_match_oracle_at_sampled_steps(dev, compact):
    """Config 4's long tail on the Qwen2-1.5B shape (two layers): G = 32 rows =
    4 prompts x 8 samples, prompts U[128, 512], lognormal stops (median 200,
    sigma 0.75, capped at 1024) with one row of prompt 0 running 1160 tokens, so
    its context grows past 1,500 through blocks reserved a chunk ahead while
    the other rows stop and free theirs (``run_paged``).  Every block is back
    on the free list at the end and the in-kernel hand-overs check clear.  The
    oracle, teacher-forced on the GPU's tokens, recomputes the long row at
    steps 0, 255, 511, 767, 1023 and 1159 and each other prompt's longest row
    at its last step: the GPU's token equals the oracle's argmax wherever the
    oracle's top-2 margin exceeds 1e-2 of max|logit|.  With ``compact`` the
    long row spends its tail on the 8-row engine (``run_paged(compact=...)``)."""
    from grpo_mi355x.core.kv_pool import PagedKVPool
    from grpo_mi355x.rollout.decode import DecodeEngine, PrefillEngine, prefill
    from grpo_mi355x.rollout.qwen2 import Qwen2Config, build_random_model

    cfg = Qwen2Config.qwen2_1_5b()
    cfg.num_hidden_layers = 2
    model = build_random_model(cfg, dev, seed=43)
    g = np.random.default_rng(12)
    prompts, samples, new, long_steps = 4, 8, 1160, 1160
    lens = g.integers(128, 513, prompts)
    plist = [g.integers(0, cfg.vocab_size, n).tolist() for n in lens]
    stops = np.minimum(1024, np.maximum(1, np.round(
        g.lognormal(np.log(200.0), 0.75, prompts * samples)))).astype(int)
    stops[0] = long_steps
    rows = [plist[i // samples] for i in range(prompts * samples)]
    B, bs = len(rows), 16
    width = -(-(int(lens.max()) + new) // bs)
    pool = PagedKVPool(2, prompts * width + B * (width + 1), cfg.num_key_value_heads,
                       cfg.head_dim, bs, device=dev)
    print(f"cfg4 long tail: prompts {lens.tolist()}, stops {stops.tolist()}", flush=True)
    pre = PrefillEngine(model, pool, 64, width)
    parents = [prefill(pre, pool, tuple(p), width) for p in plist]
    del pre
    sids = [pool.fork(parents[i // samples], 1, reserve_tokens=len(r))[0]
            for i, r in enumerate(rows)]
    for p in parents:
        pool.free(p)
    eng = DecodeEngine(model, pool, B, width)
    start = dict(tokens=torch.tensor([r[-1] for r in rows], device=dev),
                 positions=torch.tensor([len(r) - 1 for r in rows], device=dev),
                 block_tables=pool.block_table(sids, width, device=dev),
                 limits=torch.from_numpy(stops).to(dev), max_new_tokens=new)
    eng.start(**start)
    eng.capture()
    eng.start(**start)
    # also checks the hand-overs of every engine used
    stats = eng.run_paged(sids, new, check_invariants=True,
                          compact=eng.compaction_engines((16, 8)) if compact else None)
    torch.cuda.synchronize()
    if compact:
        assert stats["engines"][0] == 32 and stats["engines"][-1] == 8
    assert long_steps <= stats["steps"] <= long_steps + 16
    assert pool.num_free == pool.num_blocks and not pool.blocks
    gen = eng.generated.cpu().numpy()
    for b in range(B):
        lead = (b // samples) * samples
        s = min(stops[b], stops[lead])
        assert np.array_equal(gen[b, :s], gen[lead, :s])
        assert np.all(gen[b, stops[b]:] == PAD)
    print(f"cfg4 long tail: {stats}", flush=True)
    w, c = export(model)
    oracle = Qwen2DecodeOracle(w, c)
    checks = [(0,) + c for c in _oracle_check_steps(oracle, plist[0], gen[0, :long_steps],
                                                    [0, 255, 511, 767, 1023, 1159], width)]
    for i in range(1, prompts):
        b = max(range(i * samples, (i + 1) * samples), key=lambda r: stops[r])
        checks += [(b,) + c for c in _oracle_check_steps(oracle, plist[i], gen[b, :stops[b]],
                                                         [int(stops[b]) - 1], width)]
    safe = [(b, s, nxt) for b, s, nxt, ok in checks if ok]
    assert len(safe) >= len(checks) // 2
    for b, s, nxt in safe:
        assert gen[b, s] == nxt, (b, s, gen[b, s], nxt)
