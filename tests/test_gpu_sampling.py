"""GPU sampling in the model-level decode (the reference's default generation
config: do_sample=True, temperature 0.7, top_p 0.9; src/utils/config.py:135-137).

The sampling runs inside the captured step graph (grpo_sample_advance).  These
tests pin: the same seed gives the same tokens, another seed other tokens, a
vanishing top_p is greedy decoding, and the first sampled token of every row is
the sampling oracle's token for that step's logits and the row's draw.
"""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _model(dev, seed=13):
    from grpo_mi355x.rollout.qwen2 import Qwen2Config, build_random_model

    cfg = Qwen2Config.tiny(layers=2, heads=4, kv_heads=2, head_dim=128, inter=1024, vocab=1024)
    return build_random_model(cfg, dev, seed=seed)


def _ids(dev, G, n=23, seed=1):
    g = np.random.default_rng(seed)
    prompt = g.integers(1, 1000, n).tolist()
    return torch.tensor([prompt] * G, device=dev)


def test_sampling_is_reproducible_and_tiny_top_p_is_greedy(dev):
    from grpo_mi355x.kernels import paged_kv_decode

    model = _model(dev)
    ids = _ids(dev, 6)
    kw = dict(attention_mask=torch.ones_like(ids), max_new_tokens=12, pad_token_id=0,
              eos_token_id=None)
    a = paged_kv_decode(model, ids, do_sample=True, temperature=0.7, top_p=0.9, seed=5, **kw)
    b = paged_kv_decode(model, ids, do_sample=True, temperature=0.7, top_p=0.9, seed=5, **kw)
    c = paged_kv_decode(model, ids, do_sample=True, temperature=0.7, top_p=0.9, seed=6, **kw)
    assert torch.equal(a, b)
    assert not torch.equal(a, c)
    # six identical prompts: sampling makes the rows differ (GRPO's G samples)
    assert len({tuple(r) for r in a.cpu().tolist()}) > 1
    greedy = paged_kv_decode(model, ids, do_sample=False, **kw)
    # temperature 1: bf16(l / 1) = l, so the kept top token is greedy's argmax
    tiny = paged_kv_decode(model, ids, do_sample=True, temperature=1.0, top_p=1e-6, seed=5,
                           **kw)
    assert torch.equal(tiny, greedy)


def test_sampled_first_tokens_match_the_oracle(dev):
    """64 rows of one prompt: every row's first sampled token equals the
    sampling oracle's on the step's bf16 logits with the row's draw
    SplitMix64(seed, row, 0) -- the reference's rule (fused_ops.py:236-248)
    bit for bit -- and the rows spread over the kept set."""
    import numpy as np

    from grpo_mi355x.core.kv_pool import PagedKVPool
    from grpo_mi355x.rollout.decode import DecodeEngine, PrefillEngine, prefill, prefill_chunk
    from oracle import sampling as S

    model = _model(dev, seed=17)
    prompt = _ids(dev, 1, n=31, seed=4)[0].tolist()
    G, width, T, TOP_P, SEED = 64, 4, 0.8, 0.9, 123
    pool = PagedKVPool(2, width * (G + 2), 2, 128, 16, device=dev)
    pre = PrefillEngine(model, pool, prefill_chunk(len(prompt) - 1), width)
    parent = prefill(pre, pool, tuple(prompt), width)
    kids = pool.fork(parent, G, reserve_tokens=len(prompt))
    eng = DecodeEngine(model, pool, G, width, do_sample=True, temperature=T, top_p=TOP_P,
                       seed=SEED)

    def start():
        eng.start(torch.full((G,), prompt[-1], device=dev),
                  torch.full((G,), len(prompt) - 1, device=dev),
                  pool.block_table(kids, width, device=dev), torch.full((G,), 4, device=dev), 4)

    start()
    eng.capture()
    start()
    eng.step()
    torch.cuda.synchronize()
    first = eng.generated[:, 0].cpu().numpy()
    bits = eng.logits.cpu().view(torch.int16).numpy().view(np.uint16)
    assert np.all(bits == bits[0])  # one prompt: every row has the same logits
    draws = np.array([S.step_draw(SEED, b, 0) for b in range(G)], dtype=np.uint64)
    want, kept = S.sample_rows(bits, T, TOP_P, draws)
    assert np.array_equal(first, want)
    assert len(set(first.tolist())) > 1 and kept[0] > 1


def test_sampled_rollout_at_full_vocabulary_matches_the_oracle_twice(dev):
    """The sampled decode at the Qwen2-1.5B shape (two layers, V = 151936,
    T = 0.7, top_p = 0.9, the reference trainer's defaults), G = 8 rows, run as
    two rollouts of graph replays: at every step every active row's token is
    the sampling oracle's on that step's bf16 logits with the row's draw
    SplitMix64(seed, row, step), and the second rollout repeats the first."""
    from grpo_mi355x.core.kv_pool import PagedKVPool
    from grpo_mi355x.rollout.decode import DecodeEngine, PrefillEngine, prefill, prefill_chunk
    from grpo_mi355x.rollout.qwen2 import Qwen2Config, build_random_model
    from oracle import sampling as S

    cfg = Qwen2Config.qwen2_1_5b()
    cfg.num_hidden_layers = 2
    model = build_random_model(cfg, dev, seed=23)
    g = np.random.default_rng(3)
    prompt = g.integers(0, cfg.vocab_size, 40).tolist()
    G, steps, T, TOP_P, SEED = 8, 6, 0.7, 0.9, 77
    width = -(-(len(prompt) + steps) // 16)
    pool = PagedKVPool(2, width * (G + 2), cfg.num_key_value_heads, cfg.head_dim, 16,
                       device=dev)
    pre = PrefillEngine(model, pool, prefill_chunk(len(prompt) - 1), width)
    parent = prefill(pre, pool, tuple(prompt), width)
    del pre
    kids = pool.fork(parent, G, reserve_tokens=len(prompt) + steps)
    eng = DecodeEngine(model, pool, G, width, do_sample=True, temperature=T, top_p=TOP_P,
                       seed=SEED)
    limits = torch.tensor([6, 2, 6, 4, 6, 5, 1, 6], device=dev)

    def start():
        eng.start(torch.full((G,), prompt[-1], device=dev),
                  torch.full((G,), len(prompt) - 1, device=dev),
                  pool.block_table(kids, width, device=dev), limits, steps)

    start()
    eng.capture()
    runs = []
    lim = limits.cpu().numpy()
    for rollout in range(2):
        start()
        for t in range(steps):
            print(f"sampled rollout {rollout}, step {t}", flush=True)
            eng.step()
            torch.cuda.synchronize()
            act = np.flatnonzero(t < lim)
            bits = eng.logits.cpu().view(torch.int16).numpy().view(np.uint16)
            got = eng.generated[:, t].cpu().numpy()
            draws = np.array([S.step_draw(SEED, int(b), t) for b in act], dtype=np.uint64)
            want, kept = S.sample_rows(bits[act], T, TOP_P, draws)
            assert np.array_equal(got[act], want), (rollout, t)
            assert np.all(got[np.flatnonzero(t >= lim)] == 0)
        runs.append(eng.generated.cpu().numpy().copy())
    assert np.array_equal(runs[0], runs[1])
    assert len({tuple(r[:2]) for r in runs[0][lim >= 2]}) > 1
