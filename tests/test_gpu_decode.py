"""GPU parity of the model-level decode step (tiny Qwen2-shaped NF4+LoRA model).

The engine's whole step (grouped q|k|v NF4+LoRA, RoPE + append, paged GQA
attention, o_proj, MLP, lm_head, argmax), captured in a HIP graph, is compared
with ``oracle.decode.Qwen2DecodeOracle`` on the same weights, teacher-forced on
the same tokens: logits within the bf16 tolerance (1e-2 of max|logit| after 28
chained bf16 ops is the bar; observed values are far smaller) and greedy tokens
equal wherever the oracle's top-2 margin exceeds that tolerance.
"""

import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_bits_to_f32
from oracle.decode import Qwen2DecodeOracle, rmsnorm, rope_tables

from conftest import rel_err
from model_export import bits, export

pytestmark = pytest.mark.gpu


def _model(dev, layers=2, seed=3):
    from grpo_mi355x.rollout.qwen2 import Qwen2Config, build_random_model

    cfg = Qwen2Config.tiny(layers=layers, heads=4, kv_heads=2, head_dim=128, inter=1024,
                           vocab=1024)  # V % 16 == 0: the fused lm_head + advance path
    return build_random_model(cfg, dev, seed=seed)


def test_rope_tables_match_transformers_formula(dev):
    model = _model(dev, layers=1)
    cos, sin = model.model.rotary_emb.tables(300)
    c_ref, s_ref = rope_tables(np.arange(300), 128, model.config.rope_theta)
    assert np.mean(bits(cos) == c_ref) > 0.999 and np.mean(bits(sin) == s_ref) > 0.999
    assert np.abs(bf16_bits_to_f32(bits(cos)) - bf16_bits_to_f32(c_ref)).max() <= 2 ** -7


def test_add_rmsnorm_matches_oracle(dev):
    from grpo_mi355x import _lib

    lib = _lib.device_library()
    g = torch.Generator().manual_seed(0)
    x = torch.randn(8, 1536, generator=g).to(torch.bfloat16).to(dev)
    res = torch.randn(8, 1536, generator=g).to(torch.bfloat16).to(dev)
    w = (1 + 0.1 * torch.randn(1536, generator=g)).to(torch.bfloat16).to(dev)
    h = res.clone()
    y = torch.empty_like(x)
    _lib.check(lib.grpo_add_rmsnorm(x.data_ptr(), h.data_ptr(), h.data_ptr(), w.data_ptr(),
                                    y.data_ptr(), 8, 1536, 1e-6, _lib.stream_handle(dev)), "n")
    torch.cuda.synchronize()
    hx = (x.float() + res.float()).to(torch.bfloat16)
    assert torch.equal(h, hx)
    ref = rmsnorm(bits(hx), bits(w), 1e-6)
    got = bits(y)
    assert np.mean(got == ref) >= 0.99
    assert rel_err(bf16_bits_to_f32(got), bf16_bits_to_f32(ref)) <= 1e-2


def _oracle_caches(cfg, B, width, bs=16):
    nb = B * width
    shape = (nb, cfg["n_kv"], bs, cfg["head_dim"])
    tables = np.arange(nb, dtype=np.int32).reshape(B, width)
    return ([np.zeros(shape, np.uint16) for _ in range(2)], tables)


# The decode step's attention -> o_proj variants at <= 8 rows: the attention
# merging its splits in the kernel + one-launch o_proj (default); a merge launch
# + one-launch o_proj computing its own LoRA-A product (the path after a failed
# XCD check); o_proj finished by its last K slice (O_TILE off).
PATHS = {"tile_merged": dict(O_TILE=True, ATTN_MERGE=True),
         "tile_merge_launch": dict(O_TILE=True, ATTN_MERGE=False),
         "o_fin": dict(O_TILE=False, ATTN_MERGE=False)}


@pytest.mark.parametrize("layers,path", [(2, "tile_merged"), (2, "tile_merge_launch"),
                                         (2, "o_fin")])
def test_decode_step_matches_oracle(dev, layers, path, monkeypatch):
    from grpo_mi355x.core.kv_pool import PagedKVPool
    from grpo_mi355x.rollout.decode import DecodeEngine

    for k, v in PATHS[path].items():
        monkeypatch.setattr(DecodeEngine, k, v)
    model = _model(dev, layers=layers)
    w, c = export(model)
    oracle = Qwen2DecodeOracle(w, c)
    B, bs, width = 4, 16, 8
    g = np.random.default_rng(1)
    prompts = [g.integers(0, 1000, n).tolist() for n in (5, 17, 33, 1)]
    steps = 6
    # GPU: private blocks per row (no sharing here), teacher-forced prefill in the B-row engine
    pool = PagedKVPool(layers, B * width, 2, 128, bs, device=dev)
    sids = [pool.allocate(width * bs) for _ in range(B)]
    eng = DecodeEngine(model, pool, B, width, keep_logits=True)
    assert eng.o_tile == PATHS[path]["O_TILE"] and eng.attn_merge == PATHS[path]["ATTN_MERGE"]
    assert eng.o_fin == (path == "o_fin")
    tbl = pool.block_table(sids, width, device=dev)
    eng.start(torch.zeros(B, dtype=torch.int64, device=dev), torch.zeros(B, device=dev), tbl,
              torch.full((B,), 100, device=dev), 100)
    eng.capture()
    # oracle state
    kcs = [np.zeros((B * width, 2, bs, 128), np.uint16) for _ in range(layers)]
    vcs = [np.zeros_like(k) for k in kcs]
    otab = np.arange(B * width, dtype=np.int32).reshape(B, width)
    # run prompts token by token (rows with shorter prompts start decoding earlier)
    maxp = max(len(p) for p in prompts)
    feed = [list(p) for p in prompts]
    pos = np.zeros(B, np.int64)
    worst, agree, total = 0.0, 0, 0
    for t in range(maxp + steps):
        toks = np.array([f[t] if t < len(f) else 0 for f in feed])
        eng.tokens.copy_(torch.from_numpy(toks).to(dev))
        eng.pos.copy_(torch.from_numpy(pos.astype(np.int32)).to(dev))
        eng.active.fill_(True)
        eng.count.zero_()
        eng._masks()
        eng.step()
        torch.cuda.synchronize()
        logits_gpu = bf16_bits_to_f32(bits(eng.logits))
        logits_ref, nxt_ref = oracle.step(toks, kcs, vcs, otab, pos)
        lr = bf16_bits_to_f32(logits_ref)
        for b in range(B):
            if t >= len(prompts[b]) - 1:  # this row is decoding: compare
                worst = max(worst, rel_err(logits_gpu[b], lr[b]))
                srt = np.sort(lr[b])
                if srt[-1] - srt[-2] > 1e-2 * np.abs(lr[b]).max():
                    total += 1
                    agree += int(np.argmax(logits_gpu[b]) == nxt_ref[b])
                if t + 1 >= len(feed[b]):
                    feed[b].append(int(nxt_ref[b]))
        pos += 1
    assert worst <= 1e-2, worst
    assert total > 0 and agree == total
    eng.verify_handover()  # counters back to zero, XCD check word clear


def test_paged_kv_decode_model_greedy_matches_oracle(dev):
    """The model-level drop-in (prefill + fork + graph decode) vs the oracle loop."""
    from grpo_mi355x.kernels import paged_kv_decode

    model = _model(dev, layers=2, seed=5)
    w, c = export(model)
    oracle = Qwen2DecodeOracle(w, c)
    g = np.random.default_rng(2)
    prompt = g.integers(0, 1000, 21).tolist()
    G, new = 3, 8
    ids = torch.tensor([prompt] * G, device=dev)
    got = paged_kv_decode(model, ids, attention_mask=torch.ones_like(ids), max_new_tokens=new,
                          do_sample=False, pad_token_id=0, eos_token_id=None,
                          stop_lengths=[8, 3, 5]).cpu().numpy()
    # oracle: prefill by stepping through prompt[:-1], then greedy decode
    width = 4
    kcs = [np.zeros((width, 2, 16, 128), np.uint16) for _ in range(2)]
    vcs = [np.zeros_like(k) for k in kcs]
    tab = np.arange(width, dtype=np.int32)[None]
    tok, ref = prompt[0], []
    for t in range(len(prompt) - 1 + new):
        tok_in = prompt[t] if t < len(prompt) else tok
        logits, nxt = oracle.step(np.array([tok_in]), kcs, vcs, tab, np.array([t]))
        if t >= len(prompt) - 1:
            ref.append(int(nxt[0]))
            tok = int(nxt[0])
    ref = np.array(ref)
    for row, stop in enumerate([8, 3, 5]):
        assert np.array_equal(got[row, :stop], ref[:stop])
        assert np.all(got[row, stop:] == 0)


def test_paged_kv_decode_accepts_transformers_model(dev):
    """The trainer's call (trainer.py:389-400) with a transformers Qwen2 model whose
    linears are NF4 and whose q/k/v/o carry ManualLoRALayer adapters."""
    from hf_model import build_hf_nf4_lora_model

    from grpo_mi355x.kernels import paged_kv_decode
    from grpo_mi355x.rollout.adapt import decode_model_from

    hf = build_hf_nf4_lora_model(seed=4, layers=2, device=dev)  # vocab 1000: hipBLASLt path
    w, c = export(hf, decode_model_from(hf).config)
    oracle = Qwen2DecodeOracle(w, c)
    g = np.random.default_rng(7)
    prompt = g.integers(0, 1000, 19).tolist()
    G, new = 4, 6
    ids = torch.tensor([prompt] * G, device=dev)
    got = paged_kv_decode(hf, input_ids=ids, attention_mask=torch.ones_like(ids),
                          max_new_tokens=new, do_sample=False, pad_token_id=0,
                          eos_token_id=None, use_cache=True).cpu().numpy()
    width = 2
    kcs = [np.zeros((width, 2, 16, 128), np.uint16) for _ in range(2)]
    vcs = [np.zeros_like(k) for k in kcs]
    tab = np.arange(width, dtype=np.int32)[None]
    tok, ref = prompt[0], []
    for t in range(len(prompt) - 1 + new):
        tok_in = prompt[t] if t < len(prompt) else tok
        _, nxt = oracle.step(np.array([tok_in]), kcs, vcs, tab, np.array([t]))
        if t >= len(prompt) - 1:
            ref.append(int(nxt[0]))
            tok = int(nxt[0])
    for row in range(G):
        assert np.array_equal(got[row], np.array(ref))


def test_lm_head_argmax_and_advance(dev):
    """bf16 lm_head GEMV + first-index argmax + the row bookkeeping, vs torch."""
    from grpo_mi355x import _lib

    lib = _lib.device_library()
    st = _lib.stream_handle(dev)
    g = torch.Generator().manual_seed(11)
    M, V, K = 8, 4096, 512
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
    w = (torch.randn(V, K, generator=g) * 0.05).to(torch.bfloat16).to(dev)
    w[100:104] = w[5]  # exact ties: the first index must win
    x[3] = 0.0         # an all-zero row: every logit ties at 0 -> index 0
    logits = torch.empty(M, V, dtype=torch.bfloat16, device=dev)
    ws = torch.empty(int(lib.grpo_lm_head_workspace_bytes(M, V)), dtype=torch.uint8, device=dev)
    _lib.check(lib.grpo_lm_head_argmax(x.data_ptr(), K, w.data_ptr(), V, K, M, logits.data_ptr(),
                                       V, ws.data_ptr(), ws.numel(), st), "lm_head")
    ref = (x.float() @ w.float().t())
    assert rel_err(logits.float().cpu().numpy(), ref.cpu().numpy()) <= 1e-2
    # row state: rows 0..7 with different activity / limits / eos hits
    nxt = torch.full((M,), -5, dtype=torch.int64, device=dev)
    tokens = torch.zeros(M, dtype=torch.int64, device=dev)
    pos = torch.arange(10, 10 + M, dtype=torch.int32, device=dev)
    count = torch.tensor([0, 1, 2, 3, 4, 5, 6, 7], dtype=torch.int32, device=dev)
    limit = torch.tensor([9, 2, 9, 9, 9, 9, 9, 9], dtype=torch.int32, device=dev)
    active = torch.tensor([1, 1, 0, 1, 1, 1, 1, 1], dtype=torch.uint8, device=dev)
    gen = torch.full((M, 9), -1, dtype=torch.int64, device=dev)
    greedy_ref = logits.float().argmax(dim=1)  # torch: first index of the maximum
    eos = torch.tensor([int(greedy_ref[4])], dtype=torch.int64, device=dev)
    app = torch.zeros(M, dtype=torch.int32, device=dev)
    alen = torch.zeros(M, dtype=torch.int32, device=dev)
    _lib.check(lib.grpo_decode_advance(ws.data_ptr(), M, V, nxt.data_ptr(), tokens.data_ptr(),
                                       pos.data_ptr(), count.data_ptr(), limit.data_ptr(),
                                       active.data_ptr(), eos.data_ptr(), gen.data_ptr(), 9,
                                       app.data_ptr(), alen.data_ptr(), st), "advance")
    torch.cuda.synchronize()
    assert torch.equal(nxt, greedy_ref) and int(nxt[3]) == 0
    assert torch.equal(tokens, nxt)
    was = [1, 1, 0, 1, 1, 1, 1, 1]
    for m in range(M):
        c0 = [0, 1, 2, 3, 4, 5, 6, 7][m]
        if was[m]:
            assert int(gen[m, c0]) == int(nxt[m]) and int(count[m]) == c0 + 1
            assert int(pos[m]) == 10 + m + 1
        else:
            assert torch.all(gen[m] == -1) and int(count[m]) == c0 and int(pos[m]) == 10 + m
        still = bool(was[m]) and int(count[m]) < int(limit[m]) and int(nxt[m]) != int(eos[0])
        assert bool(active[m]) == still
        assert int(app[m]) == (int(pos[m]) if still else -1)
        assert int(alen[m]) == (int(pos[m]) + 1 if still else 0)
    assert not bool(active[1]) and not bool(active[4])  # limit reached / EOS


@pytest.mark.parametrize("M,V,K", [(8, 4096, 1536), (32, 2048, 512), (1, 160, 256),
                                   (64, 4096, 3584), (40, 2064, 3584)])
def test_lm_head_weight_tiles_give_the_same_bits(dev, M, V, K):
    """grpo_lm_head_weight_tiles rearranges W so that each wave load reads 1 KiB
    of contiguous memory; the _tiles entry points on it must reproduce the
    row-major entry points bit for bit (logits and per-tile argmax pairs),
    with and without the staged RMSNorm, and the rearrangement must be the
    documented permutation of W's 16-byte chunks.  The last two shapes stage x
    in K chunks (lm_head_argmax_wide: x beyond 160 KiB of LDS)."""
    from grpo_mi355x import _lib

    lib = _lib.device_library()
    st = _lib.stream_handle(dev)
    g = torch.Generator().manual_seed(M + V + K)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
    w = (torch.randn(V, K, generator=g) * 0.05).to(torch.bfloat16).to(dev)
    wt = torch.empty_like(w)
    _lib.check(lib.grpo_lm_head_weight_tiles(w.data_ptr(), V, K, wt.data_ptr(), st), "tiles")
    torch.cuda.synchronize()
    # the layout: chunk ((t * K/256 + s) * 8 + j) * 64 + l = W[16t + l%16][256s + 32j + 8(l//16) ..]
    q = torch.arange(V * K // 8)
    l, j, tk = q % 64, (q // 64) % 8, q // 512
    t, s_ = tk // (K // 256), tk % (K // 256)
    rows = 16 * t + l % 16
    cols = 256 * s_ + 32 * j + 8 * (l // 16)
    want = w.cpu().view(V, K // 8, 8)[rows, cols // 8]
    assert torch.equal(wt.cpu().view(-1, 8), want)
    nws = int(lib.grpo_lm_head_workspace_bytes(M, V))
    outs = []
    for fn, wp in ((lib.grpo_lm_head_argmax, w), (lib.grpo_lm_head_argmax_tiles, wt)):
        logits = torch.empty(M, V, dtype=torch.bfloat16, device=dev)
        ws = torch.empty(nws, dtype=torch.uint8, device=dev)
        _lib.check(fn(x.data_ptr(), K, wp.data_ptr(), V, K, M, logits.data_ptr(), V,
                      ws.data_ptr(), nws, st), "lm_head")
        outs.append((logits, ws))
    if M <= 8:
        ss = (x.float() ** 2).reshape(M, K // 8, 8).sum(-1).contiguous()
        nw = (torch.randn(K, generator=g) * 0.1 + 1).to(torch.bfloat16).to(dev)
        for fn, wp in ((lib.grpo_lm_head_argmax_norm, w), (lib.grpo_lm_head_argmax_norm_tiles, wt)):
            logits = torch.empty(M, V, dtype=torch.bfloat16, device=dev)
            ws = torch.empty(nws, dtype=torch.uint8, device=dev)
            _lib.check(fn(x.data_ptr(), K, ss.data_ptr(), K // 8, nw.data_ptr(), 1e-6,
                          wp.data_ptr(), V, K, M, logits.data_ptr(), V, ws.data_ptr(), nws, st),
                       "lm_head_norm")
            outs.append((logits, ws))
    torch.cuda.synchronize()
    for a_, b_ in ((0, 1), (2, 3)) if M <= 8 else ((0, 1),):
        assert torch.equal(outs[a_][0].view(torch.int16), outs[b_][0].view(torch.int16))
        assert torch.equal(outs[a_][1], outs[b_][1])


@pytest.mark.parametrize("M,K", [(64, 3584), (24, 8192), (64, 1024)])
def test_lm_head_argmax_wide_x_in_k_chunks(dev, M, K):
    """x [M, K] beyond 160 KiB of LDS (Qwen2-7B at G = 64, and a 24-row case
    with a short last chunk): staged in K chunks; logits within the bf16
    tolerance of a float32 product, the per-tile pairs reduce to torch's
    first-index argmax of the returned logits.  [64, 1024] fits LDS whole."""
    from grpo_mi355x import _lib

    lib = _lib.device_library()
    st = _lib.stream_handle(dev)
    g = torch.Generator().manual_seed(M + K)
    V = 2048
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
    w = (torch.randn(V, K, generator=g) * 0.05).to(torch.bfloat16).to(dev)
    w[700:703] = w[9]  # exact ties: the first index must win
    logits = torch.empty(M, V, dtype=torch.bfloat16, device=dev)
    ws = torch.empty(int(lib.grpo_lm_head_workspace_bytes(M, V)), dtype=torch.uint8, device=dev)
    print(f"lm_head wide M={M} K={K}", flush=True)
    _lib.check(lib.grpo_lm_head_argmax(x.data_ptr(), K, w.data_ptr(), V, K, M, logits.data_ptr(),
                                       V, ws.data_ptr(), ws.numel(), st), "lm_head")
    nxt = torch.full((M,), -5, dtype=torch.int64, device=dev)
    _lib.check(lib.grpo_decode_advance(ws.data_ptr(), M, V, nxt.data_ptr(), None, None, None,
                                       None, None, None, None, 0, None, None, st), "argmax")
    torch.cuda.synchronize()
    ref = x.float() @ w.float().t()
    assert rel_err(logits.float().cpu().numpy(), ref.cpu().numpy()) <= 1e-2
    assert torch.equal(nxt, logits.float().argmax(dim=1))


def test_release_decode_caches_frees_the_lm_head_copy(dev):
    """The tile-order lm_head copy lives on the model between rollouts and
    release_decode_caches drops it; the next engine rebuilds the same bits."""
    from grpo_mi355x.core.kv_pool import PagedKVPool
    from grpo_mi355x.kernels import ops
    from grpo_mi355x.rollout.decode import DecodeEngine, release_decode_caches

    model = _model(dev, layers=1)
    pool = PagedKVPool(1, 16, 2, 128, 16, device=dev)
    eng = DecodeEngine(model, pool, 4, 4)
    assert eng.lm_tiled and hasattr(model, "_grpo_lm_tiles")
    assert eng.lm_screen and hasattr(model, "_grpo_lm_q8")
    first = eng.lm_w.clone()
    ops.packed_lora_a(model.model.layers[0].self_attn.o_proj.lora_A.weight)
    assert len(ops._packed_a) > 0
    del eng
    release_decode_caches(model)
    assert not hasattr(model, "_grpo_lm_tiles") and len(ops._packed_a) == 0
    assert not hasattr(model, "_grpo_lm_q8")
    eng = DecodeEngine(model, pool, 4, 4)
    torch.cuda.synchronize()
    assert torch.equal(eng.lm_w.view(torch.int16), first.view(torch.int16))


def test_screened_head_gives_the_tokens_of_the_full_head(dev, monkeypatch):
    """The greedy decode step with the screened lm_head (int8 bounds, exact bf16
    logits of the candidate rows; LM_SCREEN) generates exactly the tokens of
    the step with the full bf16 lm_head, over graph-replayed rollouts with rows
    that stop at different lengths, and leaves its hand-over counters zero."""
    from grpo_mi355x.core.kv_pool import PagedKVPool
    from grpo_mi355x.rollout.decode import DecodeEngine

    model = _model(dev, layers=2)
    B, bs, width, new = 8, 16, 8, 40
    outs = []
    for screen in (True, False):
        monkeypatch.setattr(DecodeEngine, "LM_SCREEN", screen)
        pool = PagedKVPool(2, B * width, 2, 128, bs, device=dev)
        sids = [pool.allocate(width * bs) for _ in range(B)]
        eng = DecodeEngine(model, pool, B, width)
        assert eng.lm_screen == screen
        g = torch.Generator().manual_seed(7)
        tok = torch.randint(0, 1000, (B,), generator=g).to(dev)
        limits = torch.tensor([40, 3, 17, 40, 1, 29, 40, 8], device=dev)
        eng.start(tok, torch.zeros(B, device=dev), pool.block_table(sids, width, device=dev),
                  limits, new)
        eng.capture()
        for _ in range(2):  # two rollouts of graph replays (16-step graphs, then single steps)
            eng.start(tok, torch.zeros(B, device=dev), pool.block_table(sids, width, device=dev),
                      limits, new)
            eng.run(new)
        torch.cuda.synchronize()
        eng.verify_handover()
        outs.append(eng.generated.clone())
    print("generated (screened):", outs[0][:, :8].tolist(), flush=True)
    assert torch.equal(outs[0], outs[1])


def test_live_width_split_plan_gives_the_tokens_of_the_table_width(dev, monkeypatch):
    """run() with the attention splits planned for the live contexts
    (LIVE_WIDTH: each 16-step graph's attention and o_proj plan their splits
    for the blocks its steps can reach) generates exactly the tokens of the
    plan for the whole block table, over rollouts whose contexts grow across
    several plan widths, with rows that stop at different lengths."""
    from grpo_mi355x.core.kv_pool import PagedKVPool
    from grpo_mi355x.rollout.decode import DecodeEngine

    model = _model(dev, layers=2)
    B, bs, width, new = 8, 16, 64, 200
    outs, widths = [], []
    for live in (True, False):
        monkeypatch.setattr(DecodeEngine, "LIVE_WIDTH", live)
        pool = PagedKVPool(2, B * width, 2, 128, bs, device=dev)
        sids = [pool.allocate(width * bs) for _ in range(B)]
        eng = DecodeEngine(model, pool, B, width)
        assert eng.attn_splits > 1
        g = torch.Generator().manual_seed(11)
        tok = torch.randint(0, 1000, (B,), generator=g).to(dev)
        pos = torch.tensor([0, 37, 80, 129, 170, 211, 260, 300], device=dev)
        limits = torch.tensor([200, 3, 117, 200, 1, 29, 160, 64], device=dev)
        table = pool.block_table(sids, width, device=dev)
        eng.start(tok, pos, table, limits, new)
        eng.capture()
        for _ in range(2):
            eng.start(tok, pos, table, limits, new)
            eng.run(new)
        torch.cuda.synchronize()
        eng.verify_handover()
        outs.append(eng.generated.clone())
        widths.append(sorted(eng.graph_multi))
    print("plan widths recorded:", widths, flush=True)
    # positions 300 .. 500: widths 24 and 32 of the 64-block table
    assert widths[0] == [24, 32] and widths[1] == [width]
    assert torch.equal(outs[0], outs[1])
