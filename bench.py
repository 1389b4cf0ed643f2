#!/usr/bin/env python
"""Rollout decode benchmark on one MI355X.

Workload: a random-init Qwen2-1.5B-shaped model (28 layers, hidden 1536, 12 Q / 2
KV heads, head_dim 128, MLP 8960, vocab 151936) with NF4 base weights (blocksize
64, float32 absmax) and rank-16 LoRA (alpha 32) on q/k/v/o; a group of G = 8
samples of one 512-token prompt; greedy decoding with forced per-sequence stop
lengths drawn uniformly from [64, 512] (seeded), so the batch is ragged.

One benchmark "step" is one full ragged rollout: every decode step until the
longest row stops (the prompt's KV is prefilled once before timing, shared by
the 8 rows through the block pool, and excluded from the metric).  The metric is
generated tokens of active rows / wall time of the decode loop.

The JSON line also carries:
* ``roofline`` -- the dominant kernel, the NF4 split-K linear (q|k|v, o,
  gate|up, down): each kind's 28 per-layer launches of the decode step are
  replayed as a HIP graph between HIP events on their stream; achieved =
  algorithmic bytes per launch / average launch duration, peak 8 TB/s;
* ``cpu_baseline`` -- the numpy oracle (a restatement of the reference's
  PyTorch semantics) running one decode step of the same model on the host.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "grpo-training-engine_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_HBM_GBS = 8000.0
METRIC = "rollout decode tok/s (Qwen2-1.5B arch, G=8, NF4+LoRA); % HBM roofline"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3, help="timed rollouts")
    ap.add_argument("--warmup", type=int, default=1, help="untimed rollouts")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--group", type=int, default=8)
    ap.add_argument("--prompt-len", type=int, default=512)
    ap.add_argument("--max-new", type=int, default=512)
    ap.add_argument("--layers", type=int, default=28, help="(smaller only for debugging)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-kernel-timing", action="store_true")
    ap.add_argument("--eager", action="store_true",
                    help="launch every decode step directly instead of replaying a HIP graph "
                         "(for profilers that cannot follow graph launches)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first stream a 256 MiB buffer through a copy-like kernel 3 times "
                         "(scale reference for the HBM FETCH_SIZE/WRITE_SIZE counters)")
    ap.add_argument("--sample", action="store_true",
                    help="config 3 with the reference trainer's default sampling (temperature "
                         "0.7, top-p 0.9) instead of greedy decoding (an extra measurement)")
    ap.add_argument("--grad-x", action="store_true",
                    help="time the backward's NF4 input-gradient product (grpo_nf4_grad_x and "
                         "dequantize + bf16 GEMM) at Qwen2-1.5B training shapes, M = 4096 "
                         "(an extra measurement, not the headline)")
    ap.add_argument("--wide-linear", action="store_true",
                    help="time the NF4+LoRA linear beyond the decode batches (the NF4 GEMM, "
                         "grpo_nf4_gemm, against dequantize + hipBLASLt): the reference "
                         "harness shape and the Qwen2-1.5B projections at 512 and 4096 rows "
                         "(an extra measurement, not the headline)")
    ap.add_argument("--config", type=int, default=3, choices=(1, 2, 3, 4, 5),
                    help="BASELINE config: 3 (default, the headline metric), 1 (one layer of "
                         "paged decode attention), 2 (NF4+LoRA linear at M=8), 4 (G=32 ragged "
                         "group, blocks freed as rows stop) or 5 (Qwen2-7B shape, G=64, "
                         "long contexts); 1, 2, 4 and 5 are extra measurements")
    return ap.parse_args()


def kv_bytes_per_token(cfg) -> int:
    return 2 * cfg.num_key_value_heads * cfg.head_dim * 2 * cfg.num_hidden_layers


def rollout_bytes(cfg, model, stops, prompt_len, group, block_size=16, lm_screen=False):
    """Algorithmic HBM bytes of one rollout (weights once per decode step + KV read).

    KV is counted per active row and step at its full context (logical bytes);
    the physical count reads the shared prompt blocks once per step instead of
    once per row.  With the screened lm_head (lm_screen) the head reads the
    int8 copy (V * H bytes + 8 per vocabulary row) instead of the bf16 weight;
    the candidate rows' bf16 bytes (a few KiB per row) are not counted.
    """
    wb = model.weight_bytes()
    head = wb["lm_head"]
    if lm_screen:
        V = cfg.vocab_size
        head = head // 2 + 8 * V
    per_step_weights = wb["nf4"] + wb["absmax"] + wb["lora"] + head
    kv_tok = kv_bytes_per_token(cfg)
    shared = ((prompt_len - 1) // block_size) * block_size  # tokens in shared full blocks
    steps = max(stops)
    logical = physical = 0
    for s in range(steps):
        ctxs = [prompt_len + s for st in stops if st > s]
        logical += sum(ctxs) * kv_tok
        physical += (shared + sum(c - shared for c in ctxs)) * kv_tok if ctxs else 0
    return dict(weights=per_step_weights * steps, kv_logical=logical, kv_physical=physical,
                steps=steps, weight_per_step=per_step_weights)


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "nf4_linears_traffic_cfg3.md")
PREFILL_REPS = 5  # timed prefills (mean reported)
ATTN_TRAFFIC_FILE = os.path.join(ROOT, "profiles", "paged_attention_cfg1.md")


def measured_traffic(path: str = TRAFFIC_FILE, key: str = "traffic_bytes_per_launch"):
    """HBM bytes per launch (per call for config 1) from a committed rocprofv3
    FETCH_SIZE/WRITE_SIZE summary (two counter passes, scaled by a copy kernel of
    known size), or None."""
    try:
        with open(path) as fh:
            for line in fh:
                if line.startswith(key + ":"):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def kernel_timing(eng, dev, reps: int = 20) -> dict:
    """Average launch duration of every op kind of the decode step.

    The step's own launches of one kind (e.g. the 28 per-layer q|k|v NF4
    launches, with the step's arguments) are captured into a HIP graph; the
    graph is replayed ``reps`` times between two HIP events on the stream it
    runs on, so the average covers back-to-back launches (including the short
    gap between graph nodes) with every layer's weights streamed from HBM.
    Kinds with fewer than 28 launches per step (embedding, lm_head, advance)
    are captured repeatedly up to 28 nodes, so the fixed cost of launching a
    graph is spread as it is for the per-layer kinds.
    """
    import torch

    out = {}
    side = torch.cuda.Stream(device=dev)
    kinds = []
    for k, _ in eng.launches():
        if k not in kinds:
            kinds.append(k)
    for kind in kinds:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            fns = [fn for k, fn in eng.launches() if k == kind]
            fns = fns * -(-28 // len(fns))
            for fn in fns:
                fn()
        g.replay()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        e1.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (reps * len(fns))
        rec = dict(launches=sum(k == kind for k, _ in eng.launches()), avg_us=round(us, 3))
        if kind in eng.NF4_KINDS:
            nb = eng.bytes[kind]
            rec.update(bytes_per_launch=nb, achieved_GBs=round(nb / (us * 1e-6) / 1e9, 1),
                       splits=eng.splits(kind))
        out[kind] = rec
        del g
    return out


def cpu_baseline(model, cfg, group, ctx, seed, timed: int = 2):
    """Decode steps of the numpy oracle on the host (bounded sample: one
    warm-up step, then ``timed`` timed steps; about 10 s each at config 3)."""
    import numpy as np

    from oracle.decode import Qwen2DecodeOracle
    import torch

    def bits(t):
        return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)

    def nf4(lin, bias=None, a=None, b=None):
        d = dict(packed=lin.weight.detach().cpu().numpy().reshape(-1),
                 absmax=lin.weight.quant_state.absmax.detach().cpu().numpy(),
                 n=lin.out_features, k=lin.in_features)
        if bias is not None:
            d["bias"] = bits(bias)
        if a is not None:
            d["A"], d["B"] = bits(a), bits(b)
        return d

    layers = []
    for L in model.model.layers:
        at, mlp = L.self_attn, L.mlp
        e = dict(input_norm=bits(L.input_layernorm.weight),
                 post_norm=bits(L.post_attention_layernorm.weight))
        for n in ("q", "k", "v", "o"):
            m = getattr(at, f"{n}_proj")
            e[n] = nf4(m.base_layer, m.base_layer.bias, m.lora_A.weight, m.lora_B.weight)
        for n in ("gate", "up", "down"):
            e[n] = nf4(getattr(mlp, f"{n}_proj"))
        layers.append(e)
    w = dict(embed=bits(model.model.embed_tokens.weight), norm=bits(model.model.norm.weight),
             lm_head=bits(model.lm_head.weight), layers=layers)
    c = dict(hidden=cfg.hidden_size, n_heads=cfg.num_attention_heads,
             n_kv=cfg.num_key_value_heads, head_dim=cfg.head_dim, eps=cfg.rms_norm_eps,
             theta=cfg.rope_theta, blocksize=cfg.nf4_blocksize,
             scaling=cfg.lora_alpha / cfg.lora_rank)
    oracle = Qwen2DecodeOracle(w, c, cache_dequant=False)
    g = np.random.default_rng(seed)
    width = -(-(ctx + timed + 2) // 16)
    nb = group * width
    kcs = [g.integers(0, 1 << 16, (nb, cfg.num_key_value_heads, 16, cfg.head_dim),
                      dtype=np.uint16) & 0xBFFF for _ in range(cfg.num_hidden_layers)]
    vcs = [k.copy() for k in kcs]
    tables = np.arange(nb, dtype=np.int32).reshape(group, width)
    toks = g.integers(0, cfg.vocab_size, group)
    pos = np.full(group, ctx, dtype=np.int64)
    # one untimed warm-up step (first-touch page faults, BLAS start-up), then
    # `timed` steps, each at the next position
    toks = oracle.step(toks, kcs, vcs, tables, pos)[1]
    pos = pos + 1
    t0 = time.perf_counter()
    for _ in range(timed):
        toks = oracle.step(toks, kcs, vcs, tables, pos)[1]
        pos = pos + 1
    dt = (time.perf_counter() - t0) / timed
    return dict(value=round(group / dt, 4), unit="tok/s", kind="port", **_host_cores(),
                sample=(f"{timed} decode steps of the numpy oracle after 1 warm-up step, G={group} "
                        f"rows at context {ctx + 2}..{ctx + 1 + timed}, all 28 layers + lm_head, "
                        f"NF4 dequantized per call; {dt:.2f} s per step (numpy: elementwise "
                        "single-threaded, BLAS matmuls multi-threaded)"))


def _emit(args, value, unit, ms_step, workload, extra):
    out = {"metric": METRIC, "value": round(value, 2), "unit": unit, "n_gpus": 1,
           "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 3),
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
           "data": "synthetic (random-init weights N(0,0.02) -> NF4, LoRA N(0,0.01); random "
                   "prompts)", "config": dict(workload=workload, parallelism="single GPU")}
    out.update(extra)
    print(json.dumps(out), flush=True)


def run_cfg4(args):
    """G = 32 (4 prompts x 8 samples), prompts U[128, 512],
    responses lognormal (median 200, sigma 0.75) capped at 1024, blocks reserved
    one block ahead and freed as rows stop (DecodeEngine.run_paged), the rows
    still decoding moved to a 16- and then an 8-row engine once they fit.  One
    timed step = one rollout: fork the 8 samples of each prefilled prompt,
    decode until every row stops (blocks released on the way)."""
    import numpy as np
    import torch

    from grpo_mi355x.core.kv_pool import PagedKVPool
    from grpo_mi355x.rollout.decode import DecodeEngine, prefill, prefill_engine
    from grpo_mi355x.rollout.qwen2 import Qwen2Config, build_random_model

    dev = torch.device("cuda:0")
    copy_calibration(args, dev)
    cfg = Qwen2Config.qwen2_1_5b()
    cfg.num_hidden_layers = args.layers
    rng = np.random.default_rng(args.seed)
    P, S, NEW, BS = 4, 8, 1024, 16
    lens = rng.integers(128, 513, P).tolist()
    prompts = [rng.integers(0, cfg.vocab_size, n).tolist() for n in lens]
    stops = np.minimum(NEW, np.maximum(1, np.round(rng.lognormal(np.log(200.0), 0.75, P * S))))
    stops = stops.astype(int).tolist()
    model = build_random_model(cfg, dev, seed=args.seed)
    width = -(-(max(lens) + NEW) // BS)
    G = P * S
    pool = PagedKVPool(cfg.num_hidden_layers, P * width + G * (width + 1),
                       cfg.num_key_value_heads, cfg.head_dim, BS, device=dev)
    pre = prefill_engine(model, pool, max(lens) - 1, width)
    parents = [prefill(pre, pool, tuple(p), width) for p in prompts]
    del pre
    eng = DecodeEngine(model, pool, G, width)
    # row compaction: the rows still decoding move to a 24-, a 16- and then an
    # 8-row engine once they fit (the long tail of the group runs on the
    # cheaper steps)
    ladder = eng.compaction_engines((24, 16, 8))
    rows = [prompts[i // S] for i in range(G)]

    def rollout():
        sids = [pool.fork(parents[i // S], 1, reserve_tokens=len(rows[i]))[0] for i in range(G)]
        eng.start(torch.tensor([r[-1] for r in rows], device=dev),
                  torch.tensor([len(r) - 1 for r in rows], device=dev),
                  pool.block_table(sids, width, device=dev), torch.tensor(stops, device=dev),
                  NEW)
        return sids

    sids = rollout()
    eng.capture()
    peak = 0
    for _ in range(args.warmup):
        eng.run_paged(sids, NEW, compact=ladder)
        sids = rollout()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    nsteps, engines = 0, []
    for i in range(args.steps):
        st = eng.run_paged(sids, NEW, compact=ladder)
        nsteps, peak, engines = st["steps"], st["peak_blocks"], st["engines"]
        if i + 1 < args.steps:
            sids = rollout()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    assert pool.num_free == pool.num_blocks - sum(len(pool.blocks[p]) for p in parents)
    value = sum(stops) * args.steps / elapsed
    log(f"config 4: {value:.1f} tok/s, {nsteps} decode steps per rollout, peak {peak} of "
        f"{pool.num_blocks} blocks")
    _emit(args, value, "tok/s", elapsed / args.steps * 1e3,
          "BASELINE config 4: Qwen2-1.5B-shaped NF4+LoRA decode, G=32 (4 prompts x 8), prompts "
          "U[128,512], responses lognormal(median 200, sigma 0.75) capped at 1024, blocks "
          "freed as rows stop; step = one ragged rollout",
          dict(prompt_lens=lens, response_tokens=sum(stops), decode_steps_per_rollout=nsteps,
               engines_rows=engines,
               us_per_decode_step=round(elapsed / args.steps / max(nsteps, 1) * 1e6, 2),
               peak_blocks=peak, pool_blocks=pool.num_blocks))


def run_cfg5(args):
    """Qwen2-7B shape (28 layers), G = 64, contexts U[1024, 4096]
    over a KV pool pre-filled with N(0, 1) bf16 (decode-only: no 4k prefill).  One
    timed step = one decode step of the 64 rows (graph replay)."""
    import numpy as np
    import torch

    from grpo_mi355x.core.kv_pool import PagedKVPool
    from grpo_mi355x.rollout.decode import DecodeEngine
    from grpo_mi355x.rollout.qwen2 import Qwen2Config, build_random_model

    dev = torch.device("cuda:0")
    copy_calibration(args, dev)
    cfg = Qwen2Config.qwen2_7b()
    cfg.num_hidden_layers = args.layers
    rng = np.random.default_rng(args.seed)
    G, BS = 64, 16
    steps = args.steps * 16
    ctx = rng.integers(1024, 4097, G)
    width = -(-(int(ctx.max()) + steps + (args.warmup + 1) * 16) // BS)
    need = [-(-(int(c) + steps + (args.warmup + 1) * 16) // BS) for c in ctx]
    nb = sum(need)
    model = build_random_model(cfg, dev, seed=args.seed)
    pool = PagedKVPool(cfg.num_hidden_layers, nb, cfg.num_key_value_heads, cfg.head_dim, BS,
                       device=dev)
    gen = torch.Generator(device=dev).manual_seed(args.seed)
    for li in range(cfg.num_hidden_layers):
        pool.k[li].normal_(generator=gen)
        pool.v[li].normal_(generator=gen)
    perm = rng.permutation(nb).astype(np.int32)
    tables = np.full((G, width), -1, np.int32)
    o = 0
    for b in range(G):
        tables[b, :need[b]] = perm[o:o + need[b]]
        o += need[b]
    eng = DecodeEngine(model, pool, G, width)
    start = dict(tokens=torch.from_numpy(rng.integers(0, cfg.vocab_size, G)).to(dev),
                 positions=torch.from_numpy(ctx).to(dev),
                 block_tables=torch.from_numpy(tables).to(dev),
                 limits=torch.full((G,), 1 << 20, device=dev), max_new_tokens=steps + 64)
    eng.start(**start)
    if not args.eager:
        eng.capture()
    eng.start(**start)
    eng.run(16 * args.warmup)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    eng.run(steps)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    value = G * steps / elapsed
    kv = int(eng.attn_len.sum().item()) * cfg.num_key_value_heads * cfg.head_dim * 2 * 2 \
        * cfg.num_hidden_layers
    wb = sum(model.weight_bytes().values())
    step_s = elapsed / steps
    log(f"config 5: {value:.1f} tok/s, {step_s * 1e6:.1f} us/decode step")
    ab = eng.attention_bytes()  # before the timing replays advance the rows
    kernels = {} if args.no_kernel_timing else kernel_timing(eng, dev)
    if kernels:
        kernels["attention"].update(bytes_per_launch=ab, achieved_GBs=round(
            ab / (kernels["attention"]["avg_us"] * 1e-6) / 1e9, 1))
    _emit(args, value, "tok/s", step_s * 1e3,
          "BASELINE config 5: Qwen2-7B-shaped NF4+LoRA decode, G=64, contexts U[1024,4096], KV "
          "pool pre-filled N(0,1) bf16 (decode only); step = one decode step of 64 rows",
          dict(us_per_decode_step=round(step_s * 1e6, 2),
               step_hbm=dict(weight_bytes=wb, kv_bytes=kv,
                             achieved_GBs=round((wb + kv) / step_s / 1e9, 1),
                             frac_of_peak=round((wb + kv) / step_s / 1e9 / PEAK_HBM_GBS, 4)),
               kernels=kernels))


def _graph_time(fns, dev, reps: int) -> float:
    """Average µs per call of ``fns`` (one launch sequence each), captured once
    into a HIP graph and replayed ``reps`` times between HIP events recorded on
    the stream the graph runs on."""
    import torch

    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        for fn in fns:
            fn()  # workspaces sized and per-weight layouts (packed LoRA A) built before capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        for fn in fns:
            fn()
    g.replay()
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(side)
        for _ in range(reps):
            g.replay()
        e1.record(side)
    e1.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * len(fns))


def _eager_time(fns, dev, reps: int) -> float:
    """Average µs per call of ``fns`` launched directly (no graph; for
    profilers whose counter passes cannot follow graph launches)."""
    import torch

    for fn in fns[:2]:
        fn()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        for fn in fns:
            fn()
    e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * len(fns))


def copy_calibration(args, dev) -> None:
    """With --copy-calibration: three float32 multiply kernels that each read and
    write exactly 256 MiB, the scale reference for the FETCH_SIZE / WRITE_SIZE
    counters of the same profiler pass."""
    if not args.copy_calibration:
        return
    import torch

    src = torch.ones(64 << 20, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    log("copy calibration: 3 x (read 268435456 B, write 268435456 B) elementwise kernels")
    del src, dst


def _host_cores() -> dict:
    """Host cores (os.cpu_count()) and the BLAS threads numpy uses."""
    blas = None
    try:
        from threadpoolctl import threadpool_info

        blas = max([i.get("num_threads", 1) for i in threadpool_info()] + [1])
    except Exception:  # pragma: no cover - threadpoolctl is optional
        pass
    return dict(cores=os.cpu_count(), blas_threads=blas)


ROTATE_BYTES = 512 << 20  # config 1/2 working sets fit the 256 MB MALL: rotate >= 512 MB


def run_cfg1(args):
    """one layer of paged GQA decode attention, 4 sequences,
    contexts U[512, 1024], 12 query / 2 KV heads, head_dim 128, block size 16,
    shuffled block tables, q/K/V ~ N(0, 1) bf16, float32 softmax and output.

    R independent instances (own pool, table permutation, q) of >= 512 MB in
    total are launched back to back (``grpo_paged_attn_decode_merged``: one
    launch per call, the last-arriving context split of each (sequence, KV
    head) merging the pair's splits), so no call finds its K/V in the 256 MB
    MALL.  One step = one replay of the R calls."""
    import numpy as np
    import torch

    from grpo_mi355x.kernels import ops

    dev = torch.device("cuda:0")
    copy_calibration(args, dev)
    B, HQ, HKV, D, BS = 4, 12, 2, 128, 16
    rng = np.random.default_rng(args.seed)
    ctx = rng.integers(512, 1025, B).astype(np.int32)
    nblk = [-(-int(c) // BS) for c in ctx]
    nb = sum(nblk) + 8
    kv_bytes = int(ctx.sum()) * HKV * D * 2 * 2
    call_bytes = kv_bytes + B * HQ * D * 2 + B * HQ * D * 4 + sum(nblk) * 4
    R = -(-ROTATE_BYTES // (nb * HKV * BS * D * 2 * 2))
    gen = torch.Generator(device=dev).manual_seed(args.seed)
    inst = []
    for _ in range(R):
        kc = torch.randn((nb, HKV, BS, D), generator=gen, device=dev).to(torch.bfloat16)
        vc = torch.randn((nb, HKV, BS, D), generator=gen, device=dev).to(torch.bfloat16)
        perm = rng.permutation(nb).astype(np.int32)
        tab = np.full((B, max(nblk)), -1, np.int32)
        o = 0
        for b in range(B):
            tab[b, :nblk[b]] = perm[o:o + nblk[b]]
            o += nblk[b]
        q = torch.randn((B, HQ, D), generator=gen, device=dev).to(torch.bfloat16)
        inst.append((q, kc, vc, torch.from_numpy(tab).to(dev)))
    lens = torch.from_numpy(ctx).to(dev)
    out = torch.empty((B, HQ, D), dtype=torch.float32, device=dev)
    scale = 1.0 / math.sqrt(D)
    fns = [lambda i=i: ops.paged_attention_decode(i[0], i[1], i[2], i[3], lens, scale, out=out)
           for i in inst]
    for _ in range(args.warmup):
        _graph_time(fns, dev, 1)
    us = _eager_time(fns, dev, max(args.steps, 1)) if args.eager else \
        _graph_time(fns, dev, max(args.steps, 1) * 5)
    achieved = call_bytes / (us * 1e-6) / 1e9
    ops.attention_handover_check(dev)  # the in-kernel merges ran on one XCD per pair
    log(f"config 1: {R} rotating instances, {us:.2f} us per call, {achieved:.1f} GB/s")
    cpu = None
    if not args.no_cpu_baseline:
        from oracle.paged import paged_attention_decode as oracle_attn

        def bits(t):
            return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)

        q, kc, vc, tab = (bits(inst[0][0]), bits(inst[0][1]), bits(inst[0][2]),
                          inst[0][3].cpu().numpy())
        oracle_attn(q, kc, vc, tab, ctx, scale)
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < 10.0 or n < 5:
            oracle_attn(q, kc, vc, tab, ctx, scale)
            n += 1
        dt = (time.perf_counter() - t0) / n
        cpu = dict(value=round(call_bytes / dt / 1e9, 4), unit="GB/s", kind="port",
                   sample=f"{n} calls of the numpy oracle on one instance, {dt * 1e3:.1f} ms "
                          "per call (algorithmic bytes / time)", **_host_cores())
    print(json.dumps({
        "metric": "paged GQA decode attention GB/s (BASELINE config 1); % HBM roofline",
        "value": round(achieved, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(us * R / 1e3, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (q, K, V ~ N(0,1) bf16; shuffled block tables)",
        "config": {"workload": "BASELINE config 1: one layer of paged decode attention, 4 seqs, "
                               "ctx U[512,1024], 12Q/2KV, D128, block 16, shuffled tables; step = "
                               f"{R} rotating instances (>= 512 MB)",
                   "context_lens": ctx.tolist(), "instances": R, "parallelism": "single GPU"},
        "us_per_call": round(us, 3), "bytes_per_call": call_bytes,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                     "traffic": measured_traffic(ATTN_TRAFFIC_FILE),
                     "kernel": "grpo_paged_attn_decode_merged: paged_attn_split with the "
                               "in-kernel merge (one launch per call)"},
        "cpu_baseline": cpu}), flush=True)


def run_cfg2(args):
    """the NF4-dequant + fused LoRA linear at a decode batch of
    8 tokens: q/o 1536x1536 and k/v 256x1536 (NF4, blocksize 64, float32
    absmax, weights N(0, 0.02) before quantization), LoRA rank 16 / alpha 32
    with A, B ~ N(0, 0.01), bias on q/k/v, x ~ N(0, 1) bf16.

    R independent sets of the four projections (>= 512 MB of weights) are
    launched back to back (``ops.nf4_lora_linear``: at 8 rows the one-launch
    tile kernel, ``grpo_nf4_tile_linear``, with each LoRA A packed once before
    the timed region), so no call finds its weights in the 256 MB MALL.  One
    step = one replay of the R x 4 calls."""
    import numpy as np
    import torch

    from grpo_mi355x.core.nf4 import nf4_code, quantize_nf4
    from grpo_mi355x.kernels import ops

    dev = torch.device("cuda:0")
    copy_calibration(args, dev)
    M, K, R_, BSZ = 8, 1536, 16, 64
    shapes = dict(q=1536, k=256, v=256, o=1536)
    rng = torch.Generator(device=dev).manual_seed(args.seed)
    code = nf4_code(dev)

    def lin_bytes(n, bias):
        return n * K // 2 + n * K // BSZ * 4 + (R_ * K + n * R_) * 2 + M * K * 2 + M * n * 2 \
            + (n * 2 if bias else 0)

    per_set = sum(lin_bytes(n, k != "o") for k, n in shapes.items())
    R = -(-ROTATE_BYTES // per_set)
    sets = []
    for _ in range(R):
        d = {}
        for name, n in shapes.items():
            w = torch.randn((n, K), generator=rng, device=dev) * 0.02
            packed, qs = quantize_nf4(w, BSZ)
            d[name] = dict(
                n=n, packed=packed.view(-1), absmax=qs.absmax,
                bias=(torch.randn(n, generator=rng, device=dev) * 0.02).to(torch.bfloat16)
                if name != "o" else None,
                a=(torch.randn((R_, K), generator=rng, device=dev) * 0.01).to(torch.bfloat16),
                b=(torch.randn((n, R_), generator=rng, device=dev) * 0.01).to(torch.bfloat16),
                x=torch.randn((M, K), generator=rng, device=dev).to(torch.bfloat16),
                y=torch.empty((M, n), dtype=torch.bfloat16, device=dev))
        sets.append(d)
    per_kind = {}
    reps = max(args.steps, 1) * 5
    for name, n in shapes.items():
        fns = [lambda p=s[name]: ops.nf4_lora_linear(p["x"], p["packed"], p["absmax"], code, BSZ,
                                                      p["n"], bias=p["bias"], lora_a=p["a"],
                                                      lora_b=p["b"], scaling=2.0, out=p["y"])
               for s in sets]
        for _ in range(args.warmup):
            _graph_time(fns, dev, 1)
        us = _eager_time(fns, dev, max(args.steps, 1)) if args.eager else \
            _graph_time(fns, dev, reps)
        nb = lin_bytes(n, name != "o")
        per_kind[name] = dict(us_per_call=round(us, 3), bytes_per_call=nb,
                              achieved_GBs=round(nb / (us * 1e-6) / 1e9, 1),
                              launches_per_call=1)
    tot_us = sum(v["us_per_call"] for v in per_kind.values())
    achieved = per_set / (tot_us * 1e-6) / 1e9
    log(f"config 2: {R} rotating sets; {per_kind}")
    cpu = None
    if not args.no_cpu_baseline:
        from oracle.lora_linear import nf4_lora_linear as oracle_linear

        def bits(t):
            return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)

        host = {k: dict(x=bits(p["x"]), packed=p["packed"].cpu().numpy(),
                        absmax=p["absmax"].cpu().numpy(), n=p["n"],
                        bias=None if p["bias"] is None else bits(p["bias"]), a=bits(p["a"]),
                        b=bits(p["b"])) for k, p in sets[0].items()}

        def one_set():
            for p in host.values():
                oracle_linear(p["x"], p["packed"], p["absmax"], p["n"], K, BSZ,
                              bias_bits=p["bias"], a_bits=p["a"], b_bits=p["b"], scaling=2.0)

        one_set()
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < 10.0 or n < 3:
            one_set()
            n += 1
        dt = (time.perf_counter() - t0) / n
        cpu = dict(value=round(per_set / dt / 1e9, 4), unit="GB/s", kind="port",
                   sample=f"{n} sets of the four projections on the numpy oracle (NF4 "
                          f"dequantized per call), {dt * 1e3:.1f} ms per set", **_host_cores())
    print(json.dumps({
        "metric": "NF4+LoRA linear GB/s at M=8 (BASELINE config 2); % HBM roofline",
        "value": round(achieved, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(tot_us * R / 1e3, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (W ~ N(0,0.02) -> NF4, A/B ~ N(0,0.01), x ~ N(0,1), bf16)",
        "config": {"workload": "BASELINE config 2: NF4+LoRA linear, M=8, q/o 1536x1536, k/v "
                               "256x1536, r16 a32, bias on q/k/v; step = "
                               f"{R} rotating sets of q,k,v,o (>= 512 MB)",
                   "sets": R, "parallelism": "single GPU"},
        "bytes_per_set": per_set, "projections": per_kind,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": None,
                     "kernel": "grpo_nf4_tile_linear: nf4_tile_mfma (one launch per call)"},
        "cpu_baseline": cpu}), flush=True)


def run_grad_x(args):
    """grad_x = bf16(g [M, N] @ W_nf4 [N, K]) of the fused linear's backward at the
    Qwen2-1.5B projections' shapes (q/o: 1536 x 1536, gate|up: 8960 x 1536,
    down: 1536 x 8960) for M = 4096 rows, on random bf16 g and random NF4 bytes.
    Both paths the backward uses are timed with HIP events on the stream they
    run on: the fused kernel (below 1024 rows in the backward) and dequantize +
    hipBLASLt GEMM (from 1024 rows).  One JSON line; roofline = MFMA bf16."""
    import torch

    from grpo_mi355x import _lib
    from grpo_mi355x.kernels import ops

    _lib.device_library()
    dev = torch.device("cuda:0")
    M, reps, rows = 4096, max(args.steps, 1) * 10, []
    code = torch.linspace(-1.0, 1.0, 16, device=dev)
    for (n, k) in ((1536, 1536), (8960, 1536), (1536, 8960)):
        g = torch.randn(M, n, device=dev).to(torch.bfloat16)
        packed = torch.randint(0, 256, (n * k // 2,), dtype=torch.uint8, device=dev)
        absmax = torch.rand(n * k // 64, device=dev) * 0.1
        fused = lambda: ops.nf4_grad_x(g, packed, absmax, code, 64, n, k)
        gemm = lambda: torch.matmul(g, ops.nf4_dequant(packed, absmax, code, n * k, 64).view(n, k))
        row = dict(N=n, K=k)
        for name, fn in (("fused_kernel", fused), ("dequant_gemm", gemm)):
            for _ in range(3):
                fn()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                fn()
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) / reps * 1e3
            row[name] = dict(us=round(us, 1), tflops=round(2 * M * n * k / us / 1e6, 1))
        log(f"N={n} K={k}: {row}")
        rows.append(row)
    tot_f = sum(r["fused_kernel"]["us"] for r in rows)
    flops = sum(2 * M * r["N"] * r["K"] for r in rows)
    ach = flops / tot_f / 1e6
    print(json.dumps({
        "metric": "NF4 grad_x TFLOP/s (fused kernel, Qwen2-1.5B projection shapes, M=4096)",
        "value": round(ach, 1), "unit": "TFLOP/s", "n_gpus": 1, "steps": reps, "warmup": 3,
        "higher_is_better": True, "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random bf16 gradients, random NF4 bytes)",
        "config": {"workload": "backward grad_x of the fused NF4+LoRA linear", "M": M,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(ach, 1), "peak": 2500.0,
                     "unit": "TFLOP/s", "frac": round(ach / 2500.0, 4), "traffic": None},
        "shapes": rows}), flush=True)


def run_wide_linear(args):
    """y = the fused NF4 + LoRA linear (bias, r = 16, scaling 2) for more than 64
    rows: the reference harness shape (tools/benchmark_lora_layer.py:68-75:
    4 x 64 rows, 1024 x 1024) and the Qwen2-1.5B projections (q/o 1536 x 1536,
    k/v 256 x 1536, gate/up 8960 x 1536, down 1536 x 8960) at 512 rows (a
    prefill chunk) and 4096 rows (a training batch).  The NF4 GEMM (one
    grpo_nf4_lora_linear call: nf4_gemm_mfma, K slices + nf4_finish when the
    tiles are few) against the weight dequantized + hipBLASLt (the path it
    replaces), both timed with HIP events on the stream they run on.  Random
    bf16 x, random NF4 bytes.  One JSON line; roofline = bf16 MFMA."""
    import torch
    import torch.nn.functional as F

    from grpo_mi355x import _lib
    from grpo_mi355x.kernels import ops
    from grpo_mi355x.kernels.lora_forward import _bf16_scalar

    _lib.device_library()
    dev = torch.device("cuda:0")
    reps = max(args.steps, 1) * 10
    code = torch.linspace(-1.0, 1.0, 16, device=dev)
    shapes = [("harness", 256, 1024, 1024)]
    for m in (512, 4096):
        shapes += [(f"q/o@{m}", m, 1536, 1536), (f"k/v@{m}", m, 256, 1536),
                   (f"gate/up@{m}", m, 8960, 1536), (f"down@{m}", m, 1536, 8960)]
    r, rows = 16, []
    for (name, m, n, k) in shapes:
        g = torch.Generator(device=dev).manual_seed(m + n + k)
        x = torch.randn(m, k, device=dev, generator=g).to(torch.bfloat16)
        packed = torch.randint(0, 256, (n * k // 2,), dtype=torch.uint8, device=dev, generator=g)
        absmax = torch.rand(n * k // 64, device=dev, generator=g) * 0.05
        a = (torch.randn(r, k, device=dev, generator=g) * 0.01).to(torch.bfloat16)
        b = (torch.randn(n, r, device=dev, generator=g) * 0.01).to(torch.bfloat16)
        bias = (torch.randn(n, device=dev, generator=g) * 0.01).to(torch.bfloat16)
        out = torch.empty(m, n, device=dev, dtype=torch.bfloat16)
        fused = lambda: ops.nf4_lora_linear(x, packed, absmax, code, 64, n, bias=bias, lora_a=a,
                                            lora_b=b, scaling=2.0, out=out)

        def dequant_gemm():
            wb = ops.nf4_dequant(packed, absmax, code, n * k, 64).view(n, k)
            acc = F.linear(x, wb) + bias
            return torch.add(acc, F.linear(F.linear(x, a), b) * _bf16_scalar(2.0))

        row = dict(shape=name, M=m, N=n, K=k)
        for key, fn in (("nf4_gemm", fused), ("dequant_gemm", dequant_gemm)):
            for _ in range(3):
                fn()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                fn()
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) / reps * 1e3
            row[key] = dict(us=round(us, 1), tflops=round(2 * m * n * k / us / 1e6, 1))
        log(f"{name} M={m} N={n} K={k}: {row}")
        rows.append(row)
    tot = sum(r_["nf4_gemm"]["us"] for r_ in rows)
    flops = sum(2 * r_["M"] * r_["N"] * r_["K"] for r_ in rows)
    ach = flops / tot / 1e6
    print(json.dumps({
        "metric": "NF4+LoRA linear TFLOP/s beyond 64 rows (NF4 GEMM, all shapes)",
        "value": round(ach, 1), "unit": "TFLOP/s", "n_gpus": 1, "steps": reps, "warmup": 3,
        "higher_is_better": True, "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random bf16 x, random NF4 bytes)",
        "config": {"workload": "fused NF4+LoRA forward at prefill and training batches",
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(ach, 1), "peak": 2500.0,
                     "unit": "TFLOP/s", "frac": round(ach / 2500.0, 4), "traffic": None},
        "shapes": rows}), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build has no "
              "multi-GPU path (rollout groups would shard data-parallel, one group per GPU).",
              file=sys.stderr)
        sys.exit(2)
    if args.grad_x:
        return run_grad_x(args)
    if args.wide_linear:
        return run_wide_linear(args)
    if args.config != 3:
        from grpo_mi355x import _lib

        _lib.device_library()
        return {1: run_cfg1, 2: run_cfg2, 4: run_cfg4, 5: run_cfg5}[args.config](args)
    import numpy as np
    import torch

    from grpo_mi355x import _lib
    from grpo_mi355x.core.kv_pool import PagedKVPool
    from grpo_mi355x.rollout.decode import DecodeEngine, prefill, prefill_engine
    from grpo_mi355x.rollout.qwen2 import Qwen2Config, build_random_model

    _lib.device_library()
    dev = torch.device("cuda:0")
    copy_calibration(args, dev)
    cfg = Qwen2Config.qwen2_1_5b()
    cfg.num_hidden_layers = args.layers
    G, P, NEW, BS = args.group, args.prompt_len, args.max_new, 16
    rng = np.random.default_rng(args.seed)
    stops = rng.integers(min(64, NEW), NEW + 1, G).tolist()
    prompt = rng.integers(0, cfg.vocab_size, P).tolist()
    log(f"building model (layers={cfg.num_hidden_layers}) ...")
    t = time.time()
    model = build_random_model(cfg, dev, seed=args.seed)
    torch.cuda.synchronize()
    log(f"model built in {time.time() - t:.1f}s; weight bytes {model.weight_bytes()}")
    width = -(-(P + NEW) // BS)
    pool = PagedKVPool(cfg.num_hidden_layers, width * (G + 2), cfg.num_key_value_heads,
                       cfg.head_dim, BS, device=dev)
    # chunked prefill of the shared prompt (not part of the timed decode)
    pre = prefill_engine(model, pool, P - 1, width)
    pre.capture()
    torch.cuda.synchronize()
    # one untimed prefill (first use of the pool blocks and of the graph), then
    # the mean of PREFILL_REPS timed ones (each into a fresh pool sequence)
    pool.free(prefill(pre, pool, tuple(prompt), width))
    times = []
    for i in range(PREFILL_REPS):
        torch.cuda.synchronize()
        t = time.perf_counter()
        parent = prefill(pre, pool, tuple(prompt), width)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t)
        if i + 1 < PREFILL_REPS:
            pool.free(parent)
    prefill_s = sum(times) / len(times)
    log(f"prefill of {P - 1} tokens in {prefill_s * 1e3:.1f} ms ({pre.B}-token chunks; mean of "
        f"{PREFILL_REPS}, min {min(times) * 1e3:.1f}, max {max(times) * 1e3:.1f})")
    prefill_info = dict(tokens=P - 1, chunk=pre.B, ms=round(prefill_s * 1e3, 2),
                        ms_min=round(min(times) * 1e3, 2), ms_max=round(max(times) * 1e3, 2),
                        reps=PREFILL_REPS, tokens_per_s=round((P - 1) / prefill_s, 1))
    kids = pool.fork(parent, G, reserve_tokens=P - 1 + NEW + 1)
    pool.free(parent)
    pool.check_invariants()
    del pre
    if args.sample:
        eng = DecodeEngine(model, pool, G, width, do_sample=True, temperature=0.7, top_p=0.9,
                           seed=args.seed)
    else:
        eng = DecodeEngine(model, pool, G, width)
    tables = pool.block_table(kids, width, device=dev)
    start = dict(tokens=torch.full((G,), prompt[-1], dtype=torch.int64, device=dev),
                 positions=torch.full((G,), P - 1, device=dev), block_tables=tables,
                 limits=torch.tensor(stops, device=dev), max_new_tokens=NEW)
    eng.start(**start)
    if not args.eager:
        eng.capture()
    nsteps = max(stops)

    def rollout():
        eng.start(**start)
        eng.run(nsteps)

    for _ in range(args.warmup):
        rollout()
    torch.cuda.synchronize()
    gen = eng.generated.clone()
    lengths = (torch.arange(NEW, device=dev)[None, :] < torch.tensor(stops, device=dev)[:, None])
    log(f"warm-up done; rows stop at {stops}")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        rollout()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    elapsed = t1 - t0
    if args.warmup > 0 and not args.sample:
        assert torch.equal(eng.generated, gen), "rollouts are not deterministic"
    eng.verify_handover()  # the in-kernel hand-overs ran on one XCD (outside the timed region)
    tokens = sum(stops) * args.steps
    value = tokens / elapsed
    ms_rollout = elapsed / args.steps * 1e3
    rb = rollout_bytes(cfg, model, stops, P, G, BS, lm_screen=eng.lm_screen)
    step_ms = ms_rollout / nsteps
    alg = rb["weights"] + rb["kv_logical"]
    log(f"{value:.1f} tok/s, {ms_rollout:.2f} ms/rollout, {step_ms * 1e3:.1f} us/decode step")

    roofline = attention = None
    kernels = {}
    if not args.no_kernel_timing:
        # time the ops at a representative point of the rollout: every row
        # active, context = prompt + 64 generated tokens
        eng.start(**start)
        eng.run(min(64, nsteps))
        torch.cuda.synchronize()
        ab = eng.attention_bytes()  # before the timing replays advance the rows
        kernels = kernel_timing(eng, dev)
        nf4 = [kernels[k] for k in eng.NF4_KINDS]
        tot_us = sum(k["avg_us"] * k["launches"] for k in nf4)
        tot_b = sum(k["bytes_per_launch"] * k["launches"] for k in nf4)
        n = sum(k["launches"] for k in nf4)
        agg = tot_b / (tot_us * 1e-6) / 1e9
        # the dominant kernel of the step (most GPU time per step): gate|up
        dom = max(eng.NF4_KINDS, key=lambda k: kernels[k]["avg_us"] * kernels[k]["launches"])
        dk = kernels[dom]
        achieved = dk["bytes_per_launch"] / (dk["avg_us"] * 1e-6) / 1e9
        roofline = dict(bound="hbm", achieved=round(achieved, 1), peak=PEAK_HBM_GBS, unit="GB/s",
                        frac=round(achieved / PEAK_HBM_GBS, 4),
                        traffic=measured_traffic(key=f"traffic_{dom}"),
                        kernel=f"{dom}: {eng.kernel_name(dom)}", avg_launch_us=dk["avg_us"],
                        bytes_per_launch=dk["bytes_per_launch"],
                        step_share=round(dk["avg_us"] * dk["launches"] / (step_ms * 1e3), 4),
                        nf4_aggregate=dict(
                            kernels={k: eng.kernel_name(k) for k in eng.NF4_KINDS},
                            achieved=round(agg, 1), frac=round(agg / PEAK_HBM_GBS, 4),
                            avg_launch_us=round(tot_us / n, 3), bytes_per_launch=tot_b // n,
                            traffic=measured_traffic()))
        shared = ((P - 1) // BS) * BS  # prompt tokens in the rows' shared full blocks
        ab_phys = ab - (G - 1) * shared * cfg.num_key_value_heads * cfg.head_dim * 2 * 2
        at_us = kernels["attention"]["avg_us"]
        attention = dict(
            kernel="paged_attn_split<6, fused q|k|v finish + RoPE + append> (decode step)",
            context=P + min(64, nsteps), avg_us=at_us, bytes_per_launch_logical=ab,
            bytes_per_launch_physical=ab_phys,
            achieved_GBs_logical=round(ab / (at_us * 1e-6) / 1e9, 1),
            achieved_GBs_physical=round(ab_phys / (at_us * 1e-6) / 1e9, 1),
            frac_logical=round(ab / (at_us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
            frac_physical=round(ab_phys / (at_us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4))
        log(f"kernel timing: {kernels}")

    cpu = None
    if not args.no_cpu_baseline:
        log("CPU baseline (numpy oracle: one warm-up + two timed decode steps) ...")
        try:
            cpu = cpu_baseline(model, cfg, G, P, args.seed)
        except MemoryError as exc:  # pragma: no cover
            cpu = dict(value=None, unit="tok/s", kind="port", sample=f"not run: {exc}",
                       **_host_cores())
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_rollout, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights N(0,0.02) -> NF4, LoRA N(0,0.01); random prompt)",
        "config": {
            "workload": "BASELINE config 3: Qwen2-1.5B-shaped NF4+LoRA decode, G=8, 512-token "
                        "prompt, " + ("sampled (T 0.7, top-p 0.9)" if args.sample else "greedy")
                        + ", per-sequence stops U[64,512]; step = one ragged rollout",
            "group": G, "prompt_len": P, "max_new_tokens": NEW, "stops": stops,
            "layers": cfg.num_hidden_layers, "block_size": BS, "parallelism": "single GPU",
        },
        "decode_steps_per_rollout": nsteps,
        "us_per_decode_step": round(step_ms * 1e3, 2),
        "prefill": prefill_info,
        "step_hbm": {
            "alg_bytes_per_rollout": alg,
            "kv_bytes_logical": rb["kv_logical"], "kv_bytes_physical": rb["kv_physical"],
            "weight_bytes_per_step": rb["weight_per_step"],
            "lm_head": "int8 screen + bf16 candidate rows" if eng.lm_screen else "bf16",
            "achieved_GBs": round(alg / (elapsed / args.steps) / 1e9, 1),
            "frac_of_peak": round(alg / (elapsed / args.steps) / 1e9 / PEAK_HBM_GBS, 4),
        },
        "roofline": roofline,
        "attention": attention,
        "kernels": kernels,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
