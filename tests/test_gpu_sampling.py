"""GPU sampling in the model-level decode (the reference's default generation
config: do_sample=True, temperature 0.7, top_p 0.9; src/utils/config.py:135-137).

The sampled tokens depend on the random stream, so these tests pin what the
reference's rule fixes: the same seed gives the same tokens (the sampling runs
inside the captured step graph), a vanishing top_p is greedy decoding, and every
token drawn at a step lies in the kept set the reference's rule
(src/triton_kernels/fused_ops.py:236-248) computes from that step's logits,
with the top token drawn at about its renormalised probability.
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


def test_sampled_first_tokens_follow_the_kept_set(dev):
    """64 rows of one prompt: the first sampled token of every row is in the
    reference's kept set for the prompt's last-position logits, and the most
    likely token is drawn at its renormalised probability (binomial bound)."""
    from grpo_mi355x.core.kv_pool import PagedKVPool
    from grpo_mi355x.rollout.decode import DecodeEngine, prefill

    model = _model(dev, seed=17)
    prompt = _ids(dev, 1, n=31, seed=4)[0].tolist()
    G, width, T, TOP_P = 64, 4, 0.8, 0.9
    pool = PagedKVPool(2, width * (G + 2), 2, 128, 16, device=dev)
    eng1 = DecodeEngine(model, pool, 1, width)
    eng1.capture()
    parent = prefill(eng1, pool, tuple(prompt), width)
    kids = pool.fork(parent, G, reserve_tokens=len(prompt))
    gen = torch.Generator(device=dev)
    gen.manual_seed(123)
    eng = DecodeEngine(model, pool, G, width, do_sample=True, temperature=T, top_p=TOP_P,
                       generator=gen)
    eng.start(torch.full((G,), prompt[-1], device=dev), torch.full((G,), len(prompt) - 1,
                                                                   device=dev),
              pool.block_table(kids, width, device=dev), torch.full((G,), 4, device=dev), 4)
    eng.capture()
    eng.start(torch.full((G,), prompt[-1], device=dev), torch.full((G,), len(prompt) - 1,
                                                                   device=dev),
              pool.block_table(kids, width, device=dev), torch.full((G,), 4, device=dev), 4)
    eng.step()
    torch.cuda.synchronize()
    first = eng.generated[:, 0].cpu()
    logits = eng.logits[0].float().cpu()  # every row has the same logits at this step
    assert torch.allclose(eng.logits.float().cpu(), logits.expand(G, -1))
    # the reference's rule on the same bf16 logits, on the CPU, in float32; its
    # bf16 probabilities and running sum can move the boundary by a token, so
    # the support check allows a running sum up to top_p + 0.02
    scaled = (eng.logits[0].cpu() / T)
    srt, idx = torch.sort(scaled, descending=True)
    cum = torch.softmax(srt.float(), dim=-1).cumsum(-1)
    keep_n = max(1, int((cum <= TOP_P).sum()))
    loose_n = max(1, int((cum <= TOP_P + 0.02).sum()))
    assert set(first.tolist()) <= set(idx[:loose_n].tolist())
    p = torch.softmax(srt[:keep_n].float(), dim=-1)
    top, p0 = int(idx[0]), float(p[0])
    hits = int((first == top).sum())
    sd = (G * p0 * (1 - p0)) ** 0.5
    assert abs(hits - G * p0) <= 4 * sd + 1
