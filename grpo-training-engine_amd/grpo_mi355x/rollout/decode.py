"""Model-level paged decode on the HIP kernels.

``DecodeEngine`` runs one decode step of a ``Qwen2ForCausalLM`` (NF4 + LoRA) for
a fixed batch of sequences on a ``PagedKVPool``: the reference's ``_step``
(``src/triton_kernels/paged_kv.py:690-820``) as a fixed list of C-ABI launches.
Up to 8 rows, five per layer --

  q|k|v NF4+LoRA split-K partials (the input RMSNorm staged from h and the
  per-group sums of squares) -> paged GQA attention (finishes q|k|v, RoPE,
  KV append; split partials) -> o_proj split-K (merges the attention splits
  while staging x; the last K slice of each column group adds the epilogue
  and the residual, writes h and its sums of squares) -> gate|up + SiLU*up
  (the post-attention RMSNorm staged) -> down_proj over the whole K per 8
  columns (residual add, h and sums of squares out)

-- after an embedding launch that also writes layer 0's norm statistic, and
followed by the bf16 lm_head GEMV (the final norm staged) with the first
argmax pass and one kernel that finishes the argmax and advances every row's
state.  Wider batches run the norms as launches of their own (add + RMSNorm
of the previous linear's partial sums), the attention merge as a launch, and
down_proj as split-K partials.  A split-K linear writes float32 partial sums
and the op that consumes its output sums them and applies the linear's
epilogue (bias, LoRA, bf16 rounding) itself, so no launch is spent on
finishing a linear.  Lengths, block tables
and the token buffer live on the device, so the whole step (including the
per-row bookkeeping) is captured once into a HIP graph and replayed with no
host synchronisation.  Rows stop at EOS or at a per-row length cap; a stopped
row is masked out of the append (slot -1) and of attention (length 0).

``paged_kv_decode_model`` is the drop-in for ``paged_kv.paged_kv_decode_model``
(``paged_kv.py:589-837``) with the reference's contract (returns
``[B, max_new_tokens]`` new tokens, pad after a row finishes) and per-sequence
block tables instead of the reference's shared ``arange`` table.
"""

from __future__ import annotations

import ctypes
import math
from typing import Optional

import torch

from .. import _lib
from ..core.kv_pool import PagedKVPool
from ..core.nf4 import float_absmax
from ..kernels import ops
from .adapt import decode_model_from
from .qwen2 import Qwen2ForCausalLM


def _vp(x) -> ctypes.c_void_p:
    return ctypes.c_void_p(x)


class DecodeEngine:
    """Static-shape decode step for ``batch`` rows over a KV pool."""

    def __init__(self, model: Qwen2ForCausalLM, pool: PagedKVPool, batch: int, max_blocks: int,
                 max_pos: Optional[int] = None, keep_logits: bool = False,
                 do_sample: bool = False, temperature: float = 1.0, top_p: float = 1.0,
                 seed: int = 0):
        self.lib = _lib.device_library()
        # Greedy decoding needs only each step's argmax; keep_logits also fills
        # self.logits [B, V] (bf16) every step, for callers that inspect them.
        # Sampling (do_sample with temperature > 0) needs the logits too.
        self.sampling = bool(do_sample) and temperature > 0.0
        self.temperature, self.top_p = float(temperature), float(top_p)
        # row b's draw at its n-th token is SplitMix64 of (seed, b, n): fixed by the seed
        self.seed = int(seed) & 0xFFFFFFFFFFFFFFFF
        self.keep_logits = keep_logits or self.sampling
        cfg = model.config
        self.model, self.pool, self.cfg = model, pool, cfg
        self.B, self.max_blocks = batch, max_blocks
        dev = pool.k.device
        self.device = dev
        H, D = cfg.hidden_size, cfg.head_dim
        self.Hq, self.Hkv, self.D, self.H = (cfg.num_attention_heads, cfg.num_key_value_heads, D,
                                             H)
        self.I, self.V = cfg.intermediate_size, cfg.vocab_size
        self.nqkv = (self.Hq + 2 * self.Hkv) * D
        self.max_pos = max_pos or max_blocks * pool.block_size
        self.cos, self.sin = model.model.rotary_emb.tables(self.max_pos)
        bf = dict(dtype=torch.bfloat16, device=dev)
        i32 = dict(dtype=torch.int32, device=dev)
        B = batch
        # device state
        self.tokens = torch.zeros(B, dtype=torch.int64, device=dev)
        self.pos = torch.zeros(B, **i32)          # tokens already cached
        self.append_pos = torch.zeros(B, **i32)   # pos, or -1 for a stopped row
        self.attn_len = torch.zeros(B, **i32)     # pos + 1, or 0 for a stopped row
        self.active = torch.zeros(B, dtype=torch.bool, device=dev)
        self.count = torch.zeros(B, **i32)
        self.limit = torch.zeros(B, **i32)
        self.eos = torch.full((1,), -1, dtype=torch.int64, device=dev)
        self.pad = torch.zeros(1, dtype=torch.int64, device=dev)
        self.block_tables = torch.full((B, max_blocks), -1, **i32)
        self.generated: Optional[torch.Tensor] = None
        # activations
        self.h = torch.zeros(B, H, **bf)
        self.x = torch.zeros(B, H, **bf)
        self.act = torch.zeros(B, self.I, **bf)
        self.logits = torch.zeros(B, self.V, **bf)
        self.attn_out = torch.zeros(B, self.Hq * D, **bf) if B > self.ATTN_STAGE_MAX_ROWS \
            else None
        self.next = torch.zeros(B, dtype=torch.int64, device=dev)
        self._prepare_layers()
        self.graph: Optional[torch.cuda.CUDAGraph] = None
        # MULTI_STEP steps, by the block width the attention splits are planned for
        self.graph_multi: dict = {}

    # ------------------------------------------------------------- set-up --
    def _prepare_layers(self):
        cfg, B, dev = self.cfg, self.B, self.device
        H, I, Hq, D = self.H, self.I, self.Hq, self.D
        bs = cfg.nf4_blocksize
        self.bs = bs
        self.layers = []
        self._keep = []  # ctypes objects referenced by the launches
        r = self.model.model.layers[0].self_attn.q_proj.rank
        shapes = dict(qkv=(self.nqkv, H, r, 3), o=(H, Hq * D, r, 1), gate_up=(2 * I, H, 0, 1),
                      down=(H, I, 0, 1))
        plans = {}
        for kind, (n, k, rr, nseg) in shapes.items():
            plan = ops.nf4_linear_plan(B, n, k, rr, nseg, bs)
            if plan is None:
                raise ValueError(f"{kind} shape [{n}, {k}] (B={B}) is outside the split-K "
                                 "NF4 path")
            plans[kind] = plan
        # Partial-sum buffers: q|k|v, o and down share one (each is consumed by
        # the next kernel before another linear writes it); gate|up has its own,
        # because down_proj reads it while writing its own partial sums.
        self.part = torch.empty(max(p[1] for p in plans.values()) // 4, dtype=torch.float32,
                                device=dev)
        self.part_gu = torch.empty(plans["gate_up"][1] // 4, dtype=torch.float32, device=dev)
        self.tpart = torch.empty(max(max(p[2] for p in plans.values()) // 4, 1),
                                 dtype=torch.float32, device=dev)

        def parts(kind, seg_rows, biases=None, lbs=None, rank=0, scaling=1.0):
            n, k, _, nseg = shapes[kind]
            d = _lib.LinearParts()
            buf = self.part_gu if kind == "gate_up" else self.part
            d.part, d.tpart = buf.data_ptr(), self.tpart.data_ptr()
            d.splits, d.M, d.N, d.K, d.nseg, d.r = plans[kind][0], B, n, k, nseg, rank
            end = 0
            for i, rows in enumerate(seg_rows):
                end += rows
                d.seg_end[i] = end
                d.bias[i] = None if biases is None else biases[i]
                d.lora_b[i] = None if lbs is None else lbs[i]
            d.scaling = scaling
            self._keep.append(d)
            return ctypes.byref(d)

        for layer in self.model.model.layers:
            at, mlp = layer.self_attn, layer.mlp
            qkv = at.qkv
            projs = [at.q_proj, at.k_proj, at.v_proj]
            for p in projs:
                if p.base_layer.weight.data_ptr() < qkv.packed.data_ptr() or \
                        p.base_layer.weight.data_ptr() >= qkv.packed.data_ptr() + qkv.packed.numel():
                    raise ValueError("q/k/v weights are not views of the stacked buffer")
            la = (ctypes.c_void_p * 3)(*[p.lora_A.weight.data_ptr() for p in projs])
            o = at.o_proj
            o_la = (ctypes.c_void_p * 1)(o.lora_A.weight.data_ptr())
            self._keep += [la, o_la]
            oq = o.base_layer.weight.quant_state
            dq = mlp.down_proj.weight.quant_state
            self.layers.append(dict(
                in_norm=layer.input_layernorm.weight, post_norm=layer.post_attention_layernorm.weight,
                eps=float(layer.input_layernorm.variance_epsilon),
                qkv=qkv, la=la,
                qkv_parts=parts("qkv", qkv.seg_rows,
                                [p.base_layer.bias.data_ptr() for p in projs],
                                [p.lora_B.weight.data_ptr() for p in projs], projs[0].rank,
                                float(projs[0].scaling)),
                o_w=o.base_layer.weight, o_absmax=float_absmax(oq), o_code=oq.code, o_la=o_la,
                o_parts=parts("o", [H], None, [o.lora_B.weight.data_ptr()], o.rank,
                              float(o.scaling)),
                gu=mlp.gate_up, gu_parts=parts("gate_up", [2 * I]),
                down_w=mlp.down_proj.weight, down_absmax=float_absmax(dq), down_code=dq.code,
                down_parts=parts("down", [H])))
        self.final_norm = self.model.model.norm.weight
        self.final_eps = float(self.model.model.norm.variance_epsilon)
        self.embed = self.model.model.embed_tokens.weight
        self.lm_head = self.model.lm_head.weight
        # workspaces sized before any graph capture
        self.ws_attn = ops.workspace("paged_attn", max(ops.paged_attention_workspace_bytes(
            B, Hq, self.Hkv, D, self.pool.block_size, self.max_blocks), 1), dev)
        self.attn_splits = int(self.lib.grpo_paged_attn_splits(
            B, Hq, self.Hkv, D, self.pool.block_size, self.max_blocks))
        # the fused attention prologue finishes q|k|v from at most this many K
        # slices; a plan with more takes the unfused launches (append, then
        # attention over the finished q, then o_proj from its bf16 rows)
        self.attn_fused = (self.attn_splits > 0 and plans["qkv"][0]
                           <= int(self.lib.grpo_paged_attn_qkv_max_slices()))
        if not self.attn_fused:
            self.q_rot = torch.zeros(B, Hq, D, dtype=torch.bfloat16, device=dev)
            self.attn_out = torch.zeros(B, Hq * D, dtype=torch.bfloat16, device=dev)
        self.plans = plans
        # bf16 lm_head GEMV with fused argmax + device-side row advance (x staged
        # whole in LDS, or in K chunks past 160 KiB); otherwise hipBLASLt +
        # argmax + torch ops.
        lm_bytes = int(self.lib.grpo_lm_head_workspace_bytes(B, self.V))
        self.lm_fused = self.V % 16 == 0 and H % 256 == 0 and B <= 64
        # lm_head weight in the kernels' tile order (contiguous 1 KiB per load
        # instruction); the weight is frozen during rollouts
        self.lm_w = self.lm_head
        self.lm_tiled = self.LM_TILES and self.lm_fused
        if self.lm_tiled:
            self.lm_w = self._lm_tiles(self.model, self.lm_head, dev)
        self.ws_lm = torch.empty(max(lm_bytes, 16), dtype=torch.uint8, device=dev)
        # the sampler's workspace starts zero-filled and every call leaves it so
        self.ws_smp = None
        if self.sampling:
            self.ws_smp = torch.zeros(int(self.lib.grpo_sample_workspace_bytes(B, self.V)),
                                      dtype=torch.uint8, device=dev)
        # MLP: gate|up and SiLU*up in one kernel that writes the bf16 input of
        # down_proj, when the shape allows; else down_proj stages SiLU(gate)*up
        # from the gate|up partial sums (at most 2 K slices), else a SiLU*mul
        # launch of its own.
        self.gu_fused = bool(self.lib.grpo_nf4_gate_up_silu_supported(B, I, H, bs))
        self.fuse_silu = not self.gu_fused and plans["gate_up"][0] <= 2
        # Decode batches of <= 8 rows: down_proj finishes its own columns (the
        # residual add and per-8-column sums of squares in the same launch), and
        # the next q|k|v kernel stages the input RMSNorm from h and those sums,
        # so the step has no input-norm launch after layer 0.
        # The post-attention norm likewise: o_proj's epilogue + residual add +
        # per-256-column sums of squares over N / 256 workgroups per row, and
        # gate|up stages the norm.
        self.fold = (self.FOLD_DOWN and self.gu_fused and H % 64 == 0
                     and H // 8 <= self.NORM_MAX_GROUPS and H // 64 <= self.GU_NORM_MAX_GROUPS
                     and bool(self.lib.grpo_nf4_linear_residual_supported(B, H, I, bs))
                     and bool(self.lib.grpo_nf4_gate_up_silu_tiles_norm_supported(B, I, H, bs)))
        self.ss = torch.zeros(B, max(H // 8, 1), dtype=torch.float32, device=dev)
        # greedy steps of <= 8 rows: the screened lm_head (int8 bounds, the
        # candidate tiles recomputed in bf16; the same token, half the bytes)
        self.lm_screen = (self.LM_SCREEN and self.lm_tiled and self.fold and not self.sampling
                          and not self.keep_logits and B <= 8 and self.V <= 262144)
        self.lm_q8 = self.ws_scr = None
        if self.lm_screen:
            self.lm_q8 = self._lm_q8(self.model, self.lm_head, dev)
            # its hand-over counters start zero and every call leaves them so
            self.ws_scr = torch.zeros(
                int(self.lib.grpo_lm_head_screen_workspace_bytes(B, self.V)), dtype=torch.uint8,
                device=dev)
        # the post-attention norm's statistic: per-64-column sums of squares of
        # h from grpo_linear_finish_residual (or from the o_proj kernels below)
        self.ss_post = torch.zeros(B, max(H // 64, 1), dtype=torch.float32, device=dev)
        # XCD check word of the in-kernel hand-overs (attention merge, o_proj
        # finish): zero, and zero after every run (verify_handover)
        self.xcd_err = torch.zeros(1, dtype=torch.int32, device=dev)
        self.m_cnt = None
        # o_proj as the one-launch tile linear (grpo_nf4_tile_linear_residual):
        # the epilogue, the residual add and per-column-group sums of squares
        # of h in the same launch, x = the attention's bf16 rows.  With
        # attn_merge the attention merges its context splits in the kernel and
        # also leaves o_proj's LoRA-A product (no launch between them);
        # otherwise a merge launch writes the rows and the tile kernel
        # multiplies by LoRA A itself (packed once per engine).
        self.o_tile = False
        self.attn_merge = False
        if (self.fold and self.O_TILE and self.attn_fused
                and bool(self.lib.grpo_nf4_tile_supported(B, H, Hq * D, r, 1, bs))):
            G = int(self.lib.grpo_nf4_tile_sumsq_groups(B, H, Hq * D, r, bs))
            if 0 < G <= self.GU_NORM_MAX_GROUPS and G % 4 == 0:
                self.o_tile = True
                self.ss_post = torch.zeros(B, G, dtype=torch.float32, device=dev)
                self.attn_out = torch.zeros(B, Hq * D, dtype=torch.bfloat16, device=dev)
                self.attn_merge = self.ATTN_MERGE and self.Hkv <= 4
                if self.attn_merge:
                    self.m_cnt = torch.zeros(
                        int(self.lib.grpo_paged_attn_merge_counter_bytes(B, self.Hkv)) // 4,
                        dtype=torch.int32, device=dev)
                    self.o_lora_t = torch.zeros(B, self.Hkv, 16, dtype=torch.float32,
                                                device=dev)
                for L, layer in zip(self.layers, self.model.model.layers):
                    o = layer.self_attn.o_proj
                    d = _lib.TileLinear()
                    d.M, d.N, d.K, d.nseg, d.r = B, H, Hq * D, 1, o.rank
                    d.seg_end[0] = H
                    d.scaling = float(o.scaling)
                    if o.rank > 0:
                        d.lora_b[0] = o.lora_B.weight.data_ptr()
                        if self.attn_merge:
                            d.lora_t, d.lora_t_parts = self.o_lora_t.data_ptr(), self.Hkv
                        else:
                            L["o_la_packed"] = ops.pack_lora_a(o.lora_A.weight)
                            d.lora_a[0] = L["o_la_packed"].data_ptr()
                    L["o_tile"] = d
                    L["o_la_rows"] = o.lora_A.weight
                    self._keep.append(d)
        # o_proj finishing its own columns (the K slice of each 64-column group
        # that ends last adds the epilogue and the residual, and writes the
        # group's sums of squares): no separate finish launch
        self.o_fin = False
        if (self.fold and self.O_FIN and self.attn_fused and not self.o_tile
                and B <= self.ATTN_STAGE_MAX_ROWS):
            tb, cb = ctypes.c_size_t(0), ctypes.c_size_t(0)
            G = int(self.lib.grpo_nf4_linear_attn_residual_groups(
                B, H, Hq * D, r, bs, ctypes.byref(tb), ctypes.byref(cb)))
            if 0 < G <= self.GU_NORM_MAX_GROUPS:
                self.o_fin = True
                self.o_tpart = torch.zeros(max(tb.value // 4, 1), dtype=torch.float32, device=dev)
                # arrival counters: zero before the first launch, left zero by every launch
                self.o_cnt = torch.zeros(cb.value // 4, dtype=torch.int32, device=dev)
                self.ss_post = torch.zeros(B, G, dtype=torch.float32, device=dev)
        # wide batches (more rows than o_proj's split staging takes) with more
        # than one context split: the attention merges its splits in the kernel
        # and writes the bf16 rows o_proj reads (no merge launch)
        self.wide_merge = False
        if (self.ATTN_MERGE and self.attn_fused and B > self.ATTN_STAGE_MAX_ROWS
                and self.attn_splits > 1):
            self.wide_merge = True
            self.m_cnt = torch.zeros(
                int(self.lib.grpo_paged_attn_merge_counter_bytes(B, self.Hkv)) // 4,
                dtype=torch.int32, device=dev)
        # the embedding's row statistic for layer 0's input norm
        self.ss_embed = torch.zeros(B, int(self.lib.grpo_embedding_sumsq_groups()),
                                    dtype=torch.float32, device=dev)
        # down_proj's input in the fold tile layout (zero-filled: rows >= B and
        # columns >= I stay zero)
        self.act_tiles = torch.zeros(int(self.lib.grpo_fold_tiles_elements(I)) if self.fold
                                     else 1, dtype=torch.bfloat16, device=dev)
        nf4 = lambda n, k: n * k // 2 + n * k // bs * 4
        # Algorithmic HBM bytes of each NF4 launch: packed weight + absmax +
        # LoRA A + x + the float32 partial sums written (the fused gate|up
        # writes the bf16 [B, I] activation instead).
        self.bytes = {kind: nf4(n, k) + nseg * rr * k * 2 + B * k * 2 + plans[kind][1]
                      + plans[kind][2] for kind, (n, k, rr, nseg) in shapes.items()}
        if self.gu_fused:
            self.bytes["gate_up"] = nf4(2 * I, H) + B * H * 2 + B * I * 2
        if self.fold:
            # weight + absmax + x + residual read + h written + sums of squares
            self.bytes["down"] = nf4(H, I) + B * I * 2 + 2 * B * H * 2 + B * (H // 8) * 4
        if self.o_fin or self.o_tile:
            # ... and o_proj's residual read, h written and sums of squares
            self.bytes["o"] += 2 * B * H * 2 + B * self.ss_post.shape[1] * 4
        if self.o_tile:
            # no partial sums: weight + absmax + x + LoRA (A, or its product
            # from the attention) + B + residual, h and sums
            n_, k_, rr, _ = shapes["o"]
            self.bytes["o"] = (nf4(n_, k_) + B * k_ * 2 + rr * n_ * 2
                               + (B * self.Hkv * 16 * 4 if self.attn_merge else rr * k_ * 2)
                               + 2 * B * H * 2 + B * self.ss_post.shape[1] * 4)

    def kernel_name(self, kind: str) -> str:
        """The kernel an NF4 launch kind of this engine runs (for reports)."""
        if kind == "qkv":
            return ("nf4_part_mfma (split-K, input RMSNorm staged)" if self.fold
                    else "nf4_part_mfma (split-K)")
        if kind == "o":
            if self.o_tile:
                return "nf4_tile_mfma (one launch: epilogue + residual)"
            if self.o_fin:
                return ("nf4_part_mfma (split-K, attention splits merged while staging, "
                        "last K slice finishes + residual)")
            return "nf4_part_mfma (split-K)"
        if kind == "gate_up":
            if not self.gu_fused:
                return "nf4_part_mfma (split-K)"
            if self.B <= 8 and (self.H // 256) % 2 == 0:
                return ("nf4_gate_up_units (4+4-column units of two k-steps"
                        + (", input RMSNorm staged" if self.fold else "") + ", SiLU*up fused)")
            if self.B <= 16 or (self.B <= 32 and self.B * (self.H + 8) * 2 <= 120 * 1024):
                return "nf4_gate_up_units (8+8-column units, SiLU*up fused)"
            return "nf4_gate_up_wide (x in 512-column chunks, SiLU*up fused)"
        if kind == "down":
            return ("nf4_fold_residual (whole K per 8 columns, residual)" if self.fold
                    else "nf4_part_mfma (split-K)")
        return kind

    def splits(self, kind: str) -> int:
        """K slices of an NF4 launch kind (1 for the folded down_proj)."""
        return 1 if kind == "down" and self.fold else self.plans[kind][0]

    # -------------------------------------------------------------- launch --
    def attention_bytes(self) -> int:
        """Algorithmic bytes of one attention launch at the current lengths (host sync)."""
        n = int(self.attn_len.sum().item())
        nblk = int(((self.attn_len + self.pool.block_size - 1) // self.pool.block_size).sum())
        return (n * self.Hkv * self.D * 2 * 2 + self.B * self.Hq * self.D * 2 * 2 + nblk * 4)

    NF4_KINDS = ("qkv", "o", "gate_up", "down")
    # Rows up to which o_proj merges the attention splits while staging x.
    ATTN_STAGE_MAX_ROWS = 16
    # grpo_nf4_linear_residual + grpo_nf4_linear_partials_norm for <= 8 rows
    FOLD_DOWN = True
    NORM_MAX_GROUPS = 256  # sums of squares per row the q|k|v norm staging reads
    GU_NORM_MAX_GROUPS = 256  # ... and the gate|up norm staging
    # o_proj as the one-launch tile linear (<= 8 rows, the fold path), after
    # an attention that merges its splits in the kernel (ATTN_MERGE).  Off by
    # default: at config 3 the attention's in-kernel merge and LoRA-A product
    # cost 3.4 us per launch against 1.2 us saved in o_proj (3345 against
    # 3503 tok/s); o_proj merging the splits while it stages x (O_FIN) is
    # faster.  ATTN_MERGE alone applies to wide batches (more than 16 rows),
    # whose o_proj reads merged bf16 rows: the attention merges its splits
    # instead of a merge launch.  The in-kernel hand-overs are checked after
    # every run (verify_handover), which switches ATTN_MERGE and O_FIN off for
    # later engines if one fails.
    O_TILE = False
    ATTN_MERGE = True
    # o_proj + its epilogue + residual add in one launch through the last
    # K slice of each column group (<= 16 rows; used when O_TILE is off)
    O_FIN = True
    # lm_head weight read in the kernel's tile order
    LM_TILES = True
    # greedy lm_head screened by int8 bounds (grpo_lm_head_screen_norm +
    # grpo_lm_head_exact_advance_norm): bit-identical tokens from half the
    # weight bytes (config 3: lm_head + advance 80 -> 60 us per step)
    LM_SCREEN = True

    @staticmethod
    def _lm_tiles(model, w: torch.Tensor, dev) -> torch.Tensor:
        """The tile-order copy of the lm_head weight, built once per model and
        weight version (kept on the model object, V * H * 2 bytes: 0.47 GB at
        Qwen2-1.5B, 1.09 GB at 7B, until ``release_decode_caches(model)``; the
        weight is frozen while rollouts run)."""
        key = (w.data_ptr(), w._version, tuple(w.shape))
        cache = getattr(model, "_grpo_lm_tiles", None)
        if cache is not None and cache[0] == key:
            return cache[1]
        lib = _lib.device_library()
        V, K = w.shape
        wt = torch.empty_like(w)
        _lib.check(lib.grpo_lm_head_weight_tiles(w.data_ptr(), V, K, wt.data_ptr(),
                                                  _lib.stream_handle(dev)), "lm_weight_tiles")
        model._grpo_lm_tiles = (key, wt)
        return wt

    @staticmethod
    def _lm_q8(model, w: torch.Tensor, dev):
        """The int8 copy of the lm_head weight for the screened argmax
        (grpo_lm_head_q8_tiles: V * H bytes + two float32 per vocabulary row),
        built once per model and weight version and kept on the model like the
        tile-order copy (0.23 GB at Qwen2-1.5B) until release_decode_caches."""
        key = (w.data_ptr(), w._version, tuple(w.shape))
        cache = getattr(model, "_grpo_lm_q8", None)
        if cache is not None and cache[0] == key:
            return cache[1]
        lib = _lib.device_library()
        V, K = w.shape
        wq = torch.empty(V * K, dtype=torch.uint8, device=dev)
        scale = torch.empty(V, dtype=torch.float32, device=dev)
        rnorm = torch.empty(V, dtype=torch.float32, device=dev)
        _lib.check(lib.grpo_lm_head_q8_tiles(w.data_ptr(), V, K, wq.data_ptr(), scale.data_ptr(),
                                              rnorm.data_ptr(), _lib.stream_handle(dev)), "lm_q8")
        model._grpo_lm_q8 = (key, (wq, scale, rnorm))
        return model._grpo_lm_q8[1]

    def launches(self) -> list:
        """[(kind, launch())] of one forward pass, in order, bound to torch's
        current stream (call inside the stream/graph context they run in)."""
        lib, st = self.lib, _lib.stream_handle(self.device)
        B, H, I = self.B, self.H, self.I
        chk = _lib.check
        pool = self.pool
        h, x = self.h.data_ptr(), self.x.data_ptr()
        if self.fold:  # the embedding also writes the statistic of layer 0's input norm
            out = [("embedding", lambda: chk(lib.grpo_embedding_sumsq(
                self.tokens.data_ptr(), self.embed.data_ptr(), self.V, H, h, B,
                self.ss_embed.data_ptr(), st), "embedding"))]
        else:
            out = [("embedding", lambda: chk(lib.grpo_embedding(
                self.tokens.data_ptr(), self.embed.data_ptr(), self.V, H, h, B, st),
                "embedding"))]
        prev = None
        for li, L in enumerate(self.layers):
            kc, vc = (t.data_ptr() for t in pool.layer(li))
            q = L["qkv"]
            if not self.fold:
                if prev is None:
                    out.append(("rmsnorm", lambda L=L: chk(lib.grpo_add_rmsnorm(
                        h, None, None, L["in_norm"].data_ptr(), x, B, H, L["eps"], st),
                        "rmsnorm")))
                else:
                    out.append(("rmsnorm", lambda L=L, P=prev: chk(lib.grpo_add_rmsnorm_parts(
                        P["down_parts"], h, h, L["in_norm"].data_ptr(), x, L["eps"], st),
                        "add_rmsnorm")))
            if self.fold:
                # layer 0 from the embedding's statistic, the others from down_proj's
                ss, ng = ((self.ss_embed.data_ptr(), self.ss_embed.shape[1]) if prev is None
                          else (self.ss.data_ptr(), H // 8))
                out.append(("qkv", lambda q=q, L=L, ss=ss, ng=ng: chk(
                    lib.grpo_nf4_linear_partials_norm(
                        h, H, ss, ng, L["in_norm"].data_ptr(), L["eps"], q.packed.data_ptr(),
                        q.absmax.data_ptr(), q.code.data_ptr(), self.bs, L["la"],
                        L["qkv_parts"], st), "qkv")))
            else:
                out.append(("qkv", lambda q=q, L=L: chk(lib.grpo_nf4_linear_partials(
                    x, H, q.packed.data_ptr(), q.absmax.data_ptr(), q.code.data_ptr(), self.bs,
                    L["la"], L["qkv_parts"], st), "qkv")))
            out += self._attn_launches(L, kc, vc, st)
            g = L["gu"]
            if self.fold:
                # o_proj finish + residual (h in place) + sums of squares, then
                # gate|up staging RMSNorm(h) and writing act in the tile layout
                # the folded down_proj loads
                sp = self.ss_post.data_ptr()
                if not (self.o_fin or self.o_tile):
                    out.append(("rmsnorm", lambda L=L, sp=sp: chk(
                        lib.grpo_linear_finish_residual(L["o_parts"], h, h, H, sp, st),
                        "post_finish")))
                out.append(("gate_up", lambda g=g, L=L, sp=sp: chk(
                    lib.grpo_nf4_gate_up_silu_tiles_norm(
                        h, H, sp, self.ss_post.shape[1], L["post_norm"].data_ptr(), L["eps"],
                        g.packed.data_ptr(), g.absmax.data_ptr(), g.code.data_ptr(), self.bs,
                        I, H, B, self.act_tiles.data_ptr(), st), "gate_up")))
            else:
                out.append(("rmsnorm", lambda L=L: chk(lib.grpo_add_rmsnorm_parts(
                    L["o_parts"], h, h, L["post_norm"].data_ptr(), x, L["eps"], st),
                    "post_norm")))
                if self.gu_fused:
                    out.append(("gate_up", lambda g=g: chk(lib.grpo_nf4_gate_up_silu(
                        x, H, g.packed.data_ptr(), g.absmax.data_ptr(), g.code.data_ptr(),
                        self.bs, I, H, B, self.act.data_ptr(), I, st), "gate_up")))
                else:
                    out.append(("gate_up", lambda g=g, L=L: chk(lib.grpo_nf4_linear_partials(
                        x, H, g.packed.data_ptr(), g.absmax.data_ptr(), g.code.data_ptr(),
                        self.bs, None, L["gu_parts"], st), "gate_up")))
            if self.fold:
                out.append(("down", lambda L=L: chk(lib.grpo_nf4_linear_residual(
                    self.act_tiles.data_ptr(), I, 1, L["down_w"].data_ptr(),
                    L["down_absmax"].data_ptr(), L["down_code"].data_ptr(), self.bs, H, I, B,
                    h, H, h, H, self.ss.data_ptr(), st), "down")))
            elif self.gu_fused:
                out.append(("down", lambda L=L: chk(lib.grpo_nf4_linear_partials(
                    self.act.data_ptr(), I, L["down_w"].data_ptr(),
                    L["down_absmax"].data_ptr(), L["down_code"].data_ptr(), self.bs, None,
                    L["down_parts"], st), "down")))
            elif self.fuse_silu:
                out.append(("down", lambda L=L: chk(lib.grpo_nf4_linear_partials_silu(
                    L["gu_parts"], L["down_w"].data_ptr(), L["down_absmax"].data_ptr(),
                    L["down_code"].data_ptr(), self.bs, L["down_parts"], st), "down")))
            else:
                out.append(("silu_mul", lambda L=L: chk(lib.grpo_silu_mul_parts(
                    L["gu_parts"], self.act.data_ptr(), I, st), "silu_mul")))
                out.append(("down", lambda L=L: chk(lib.grpo_nf4_linear_partials(
                    self.act.data_ptr(), I, L["down_w"].data_ptr(),
                    L["down_absmax"].data_ptr(), L["down_code"].data_ptr(), self.bs, None,
                    L["down_parts"], st), "down")))
            prev = L
        return out + self._head_launches(prev, st)

    def _attn_launches(self, L: dict, kc: int, vc: int, st) -> list:
        """Attention of one layer: RoPE + K/V append of the step's token, paged
        GQA attention over pos + 1 tokens (split partials), o_proj NF4+LoRA
        partials merging the splits while staging x."""
        if not self.attn_fused:
            return self._attn_launches_unfused(L, kc, vc, st)
        lib, chk, pool = self.lib, _lib.check, self.pool
        Hq, Hkv, D = self.Hq, self.Hkv, self.D
        wsa, wsa_n = self.ws_attn.data_ptr(), self.ws_attn.numel()
        # context splits planned for pw blocks (>= every row's context in the
        # steps these launches run: _live_width), the same for the attention
        # and the o_proj staging or merge that reads its partials
        pw = self._pw or self.max_blocks
        wide = self.B > self.ATTN_STAGE_MAX_ROWS
        # one context split: the attention writes its bf16 output itself
        direct = wide and self.attn_splits == 1
        ao = self.attn_out.data_ptr() if wide else None
        attention = ("attention", lambda: chk(lib.grpo_paged_attn_decode_qkv(
            L["qkv_parts"], Hq, Hkv, D, self.cos.data_ptr(), self.sin.data_ptr(),
            self.max_pos, self.append_pos.data_ptr(), self.attn_len.data_ptr(), kc, vc,
            pool.num_blocks, self.block_tables.data_ptr(), self.max_blocks,
            pool.block_size, pw, 1.0 / math.sqrt(D), wsa, wsa_n,
            ao if direct else None, st), "attention"))
        if wide:
            # wide batches: o_proj stages the merged bf16 rows as plain x
            # (merging the splits while staging repeats the merge in every
            # workgroup of a K slice: ~0.4 GB of partial-sum reads at 64 rows);
            # the attention merges them itself (wide_merge) or a merge launch does
            if self.wide_merge:
                attention = ("attention", lambda: chk(lib.grpo_paged_attn_decode_qkv_merged(
                    L["qkv_parts"], Hq, Hkv, D, self.cos.data_ptr(), self.sin.data_ptr(),
                    self.max_pos, self.append_pos.data_ptr(), self.attn_len.data_ptr(), kc, vc,
                    pool.num_blocks, self.block_tables.data_ptr(), self.max_blocks,
                    pool.block_size, pw, 1.0 / math.sqrt(D), wsa, wsa_n,
                    self.m_cnt.data_ptr(), self.xcd_err.data_ptr(), ao, None, 0, None, st),
                    "attention"))
            merge = [] if direct or self.wide_merge else [
                ("attn_merge", lambda: chk(lib.grpo_paged_attn_merge(
                    wsa, self.attn_len.data_ptr(), self.B, Hq, Hkv, D, pool.block_size,
                    pw, ao, 1, st), "attn_merge"))]
            return [attention] + merge + [
                ("o", lambda: chk(lib.grpo_nf4_linear_partials(
                    ao, Hq * D, L["o_w"].data_ptr(), L["o_absmax"].data_ptr(),
                    L["o_code"].data_ptr(), self.bs, L["o_la"], L["o_parts"], st), "o_proj"))]
        if self.o_tile:
            h, ao = self.h.data_ptr(), self.attn_out.data_ptr()
            o_tile = ("o", lambda: chk(lib.grpo_nf4_tile_linear_residual(
                ao, Hq * D, L["o_w"].data_ptr(), L["o_absmax"].data_ptr(),
                L["o_code"].data_ptr(), self.bs, ctypes.byref(L["o_tile"]), h, h, self.H,
                self.ss_post.data_ptr(), st), "o_proj"))
            if self.attn_merge:
                la = L["o_la_rows"]
                merged = ("attention", lambda: chk(lib.grpo_paged_attn_decode_qkv_merged(
                    L["qkv_parts"], Hq, Hkv, D, self.cos.data_ptr(), self.sin.data_ptr(),
                    self.max_pos, self.append_pos.data_ptr(), self.attn_len.data_ptr(), kc, vc,
                    pool.num_blocks, self.block_tables.data_ptr(), self.max_blocks,
                    pool.block_size, pw, 1.0 / math.sqrt(D), wsa, wsa_n,
                    self.m_cnt.data_ptr(), self.xcd_err.data_ptr(), ao,
                    la.data_ptr() if L["o_tile"].r > 0 else None, L["o_tile"].r,
                    self.o_lora_t.data_ptr(), st), "attention"))
                return [merged, o_tile]
            merge = ("attn_merge", lambda: chk(lib.grpo_paged_attn_merge(
                wsa, self.attn_len.data_ptr(), self.B, Hq, Hkv, D, pool.block_size,
                pw, ao, 1, st), "attn_merge"))
            return [attention, merge, o_tile]
        if self.o_fin:
            h = self.h.data_ptr()
            return [
                attention,
                ("o", lambda: chk(lib.grpo_nf4_linear_attn_residual(
                    wsa, self.attn_len.data_ptr(), Hq, Hkv, D, pool.block_size, pw,
                    L["o_w"].data_ptr(), L["o_absmax"].data_ptr(), L["o_code"].data_ptr(),
                    self.bs, L["o_la"], L["o_parts"], self.o_tpart.data_ptr(),
                    self.o_cnt.data_ptr(), self.xcd_err.data_ptr(), h, h, self.H,
                    self.ss_post.data_ptr(), st), "o_proj"))]
        return [
            attention,
            ("o", lambda: chk(lib.grpo_nf4_linear_partials_attn(
                wsa, self.attn_len.data_ptr(), Hq, Hkv, D, pool.block_size, pw,
                L["o_w"].data_ptr(), L["o_absmax"].data_ptr(), L["o_code"].data_ptr(), self.bs,
                L["o_la"], L["o_parts"], st), "o_proj"))]

    def _attn_launches_unfused(self, L: dict, kc: int, vc: int, st) -> list:
        """Append (q|k|v finished from the partial sums, RoPE, K/V to the cache)
        as a launch of its own, attention over the rotated q (bf16 rows), o_proj
        partial sums from those rows."""
        lib, chk, pool = self.lib, _lib.check, self.pool
        Hq, Hkv, D = self.Hq, self.Hkv, self.D
        wsa, wsa_n = self.ws_attn.data_ptr(), self.ws_attn.numel()
        q, o = self.q_rot.data_ptr(), self.attn_out.data_ptr()
        return [
            ("append", lambda: chk(lib.grpo_qkv_rope_append_parts(
                L["qkv_parts"], Hq, Hkv, D, self.cos.data_ptr(), self.sin.data_ptr(),
                self.max_pos, self.append_pos.data_ptr(), q, kc, vc, pool.num_blocks,
                self.block_tables.data_ptr(), self.max_blocks, pool.block_size,
                self.max_blocks, st), "append")),
            ("attention", lambda: chk(lib.grpo_paged_attn_decode(
                q, Hq * D, D, kc, vc, pool.num_blocks, self.block_tables.data_ptr(),
                self.max_blocks, self.attn_len.data_ptr(), o, 1, self.B, Hq, Hkv, D,
                pool.block_size, self.max_blocks, 1.0 / math.sqrt(D), wsa, wsa_n, st),
                "attention")),
            ("o", lambda: chk(lib.grpo_nf4_linear_partials(
                o, Hq * D, L["o_w"].data_ptr(), L["o_absmax"].data_ptr(),
                L["o_code"].data_ptr(), self.bs, L["o_la"], L["o_parts"], st), "o_proj"))]

    def _head_launches(self, prev: dict, st) -> list:
        """Final norm, lm_head and the token choice with the row advance."""
        lib, chk, B, H = self.lib, _lib.check, self.B, self.H
        h, x = self.h.data_ptr(), self.x.data_ptr()
        if self.fold and self.lm_fused:
            # the lm_head kernel stages the final norm from h and down_proj's sums
            if self.lm_screen:
                return self._head_launches_screen(st)
            return self._head_launches_norm(st)
        if self.fold:  # h is finished: the final norm reads it alone
            out = [("rmsnorm", lambda: chk(lib.grpo_add_rmsnorm(
                h, None, None, self.final_norm.data_ptr(), x, B, H, self.final_eps, st),
                "final_norm"))]
        else:
            out = [("rmsnorm", lambda P=prev: chk(lib.grpo_add_rmsnorm_parts(
                P["down_parts"], h, h, self.final_norm.data_ptr(), x, self.final_eps, st),
                "final_norm"))]
        if self.sampling:
            if self.lm_fused:
                fn = lib.grpo_lm_head_argmax_tiles if self.lm_tiled else lib.grpo_lm_head_argmax
                out.append(("lm_head", lambda: chk(fn(
                    x, H, self.lm_w.data_ptr(), self.V, H, B, self.logits.data_ptr(), self.V,
                    self.ws_lm.data_ptr(), self.ws_lm.numel(), st), "lm_head")))
            else:
                out.append(("lm_head",
                            lambda: torch.matmul(self.x, self.lm_head.t(), out=self.logits)))
            gen = self.generated
            out.append(("sample", lambda: chk(lib.grpo_sample_advance(
                self.logits.data_ptr(), self.V, B, self.V, self.temperature, self.top_p,
                self.seed, self.next.data_ptr(), self.tokens.data_ptr(), self.pos.data_ptr(),
                self.count.data_ptr(), self.limit.data_ptr(), self.active.data_ptr(),
                self.eos.data_ptr(), None if gen is None else gen.data_ptr(),
                0 if gen is None else gen.shape[1], self.append_pos.data_ptr(),
                self.attn_len.data_ptr(), self.ws_smp.data_ptr(), self.ws_smp.numel(), st),
                "sample")))
        elif self.lm_fused:
            gen = self.generated
            logits = self.logits.data_ptr() if self.keep_logits else None
            fn = lib.grpo_lm_head_argmax_tiles if self.lm_tiled else lib.grpo_lm_head_argmax
            out.append(("lm_head", lambda: chk(fn(
                x, H, self.lm_w.data_ptr(), self.V, H, B, logits, self.V,
                self.ws_lm.data_ptr(), self.ws_lm.numel(), st), "lm_head")))
            out.append(("advance", lambda: chk(lib.grpo_decode_advance(
                self.ws_lm.data_ptr(), B, self.V, self.next.data_ptr(), self.tokens.data_ptr(),
                self.pos.data_ptr(), self.count.data_ptr(), self.limit.data_ptr(),
                self.active.data_ptr(), self.eos.data_ptr(),
                None if gen is None else gen.data_ptr(), 0 if gen is None else gen.shape[1],
                self.append_pos.data_ptr(), self.attn_len.data_ptr(), st), "advance")))
        else:
            out.append(("lm_head",
                        lambda: torch.matmul(self.x, self.lm_head.t(), out=self.logits)))
            out.append(("argmax", lambda: chk(lib.grpo_argmax_bf16(
                self.logits.data_ptr(), self.V, self.V, B, self.next.data_ptr(), st),
                "argmax")))
        return out

    def _head_launches_norm(self, st) -> list:
        """lm_head staging the final RMSNorm from h and the sums of squares of
        the last down_proj, then the sampler or the greedy advance."""
        lib, chk, B, H = self.lib, _lib.check, self.B, self.H
        h, ss = self.h.data_ptr(), self.ss.data_ptr()
        gen = self.generated
        logits = self.logits.data_ptr() if (self.keep_logits or self.sampling) else None
        fn = lib.grpo_lm_head_argmax_norm_tiles if self.lm_tiled else lib.grpo_lm_head_argmax_norm
        out = [("lm_head", lambda: chk(fn(
            h, H, ss, H // 8, self.final_norm.data_ptr(), self.final_eps, self.lm_w.data_ptr(),
            self.V, H, B, logits, self.V, self.ws_lm.data_ptr(), self.ws_lm.numel(), st),
            "lm_head"))]
        if self.sampling:
            out.append(("sample", lambda: chk(lib.grpo_sample_advance(
                self.logits.data_ptr(), self.V, B, self.V, self.temperature, self.top_p,
                self.seed, self.next.data_ptr(), self.tokens.data_ptr(), self.pos.data_ptr(),
                self.count.data_ptr(), self.limit.data_ptr(), self.active.data_ptr(),
                self.eos.data_ptr(), None if gen is None else gen.data_ptr(),
                0 if gen is None else gen.shape[1], self.append_pos.data_ptr(),
                self.attn_len.data_ptr(), self.ws_smp.data_ptr(), self.ws_smp.numel(), st),
                "sample")))
        else:
            out.append(("advance", lambda: chk(lib.grpo_decode_advance(
                self.ws_lm.data_ptr(), B, self.V, self.next.data_ptr(), self.tokens.data_ptr(),
                self.pos.data_ptr(), self.count.data_ptr(), self.limit.data_ptr(),
                self.active.data_ptr(), self.eos.data_ptr(),
                None if gen is None else gen.data_ptr(), 0 if gen is None else gen.shape[1],
                self.append_pos.data_ptr(), self.attn_len.data_ptr(), st), "advance")))
        return out

    def _head_launches_screen(self, st) -> list:
        """The greedy head from the int8 screen: bounds of every logit, then the
        exact bf16 logits of the candidate tiles' candidate rows, the first
        index of the maximum and the row advance (the final norm staged by both
        launches from h and the last down_proj's sums of squares)."""
        lib, chk, B, H = self.lib, _lib.check, self.B, self.H
        h, ss = self.h.data_ptr(), self.ss.data_ptr()
        wq, scale, rnorm = self.lm_q8
        ws, gen = self.ws_scr, self.generated
        return [
            ("lm_head", lambda: chk(lib.grpo_lm_head_screen_norm(
                h, H, ss, H // 8, self.final_norm.data_ptr(), self.final_eps, wq.data_ptr(),
                scale.data_ptr(), rnorm.data_ptr(), self.V, H, B, ws.data_ptr(), ws.numel(), st),
                "lm_screen")),
            ("advance", lambda: chk(lib.grpo_lm_head_exact_advance_norm(
                h, H, ss, H // 8, self.final_norm.data_ptr(), self.final_eps,
                self.lm_w.data_ptr(), self.V, H, B, ws.data_ptr(), ws.numel(),
                self.xcd_err.data_ptr(),
                self.next.data_ptr(), self.tokens.data_ptr(), self.pos.data_ptr(),
                self.count.data_ptr(), self.limit.data_ptr(), self.active.data_ptr(),
                self.eos.data_ptr(), None if gen is None else gen.data_ptr(),
                0 if gen is None else gen.shape[1], self.append_pos.data_ptr(),
                self.attn_len.data_ptr(), st), "lm_exact_advance"))]

    def nf4_launches(self) -> list:
        """[(kind, algorithmic bytes, launch())] of every NF4 linear of one step."""
        return [(k, self.bytes[k], fn) for k, fn in self.launches() if k in self.NF4_KINDS]

    def _forward(self):
        """Embedding -> layers -> final norm -> lm_head -> argmax (device only)."""
        for _, fn in self.launches():
            fn()

    def _advance(self, greedy_tokens: torch.Tensor):
        """Record the step's tokens and move the per-row state (device only)."""
        if self.generated is not None:
            # an active row's token goes to column count[b]; rows that stopped,
            # and columns past the buffer, keep what they hold (the gather and
            # scatter then touch column 0 with its own value)
            col = self.count.to(torch.int64)
            ok = self.active & (col >= 0) & (col < self.generated.shape[1])
            col = torch.where(ok, col, torch.zeros_like(col)).view(-1, 1)
            keep = self.generated.gather(1, col)
            self.generated.scatter_(1, col, torch.where(ok.view(-1, 1),
                                                        greedy_tokens.view(-1, 1), keep))
        act = self.active.to(torch.int32)
        self.pos.add_(act)
        self.count.add_(act)
        still = self.active & (self.count < self.limit) & (greedy_tokens != self.eos)
        self.active.copy_(still)
        self.tokens.copy_(greedy_tokens)
        self._masks()

    def _masks(self):
        self.append_pos.copy_(torch.where(self.active, self.pos, torch.full_like(self.pos, -1)))
        self.attn_len.copy_(torch.where(self.active, self.pos + 1, torch.zeros_like(self.pos)))

    def _step(self):
        self._forward()
        if not self.lm_fused and not self.sampling:  # the fused and sampling paths advanced
            self._advance(self.next)

    # ------------------------------------------------------------ control --
    def start(self, tokens: torch.Tensor, positions: torch.Tensor, block_tables: torch.Tensor,
              limits: torch.Tensor, max_new_tokens: int, eos_token_id: Optional[int] = None,
              pad_token_id: int = 0, record: bool = True):
        """Load a new batch: input tokens at ``positions`` (tokens already cached)."""
        B = self.B
        self.tokens.copy_(tokens.view(B))
        self.pos.copy_(positions.view(B).to(torch.int32))
        self.count.zero_()
        self.limit.copy_(limits.view(B).to(torch.int32))
        self.active.copy_(self.limit > 0)
        self.eos.fill_(-1 if eos_token_id is None else int(eos_token_id))
        self.pad.fill_(int(pad_token_id))
        w = block_tables.shape[1]
        self.block_tables.fill_(-1)
        self.block_tables[:, :w].copy_(block_tables)
        if record:
            if self.generated is None or self.generated.shape[1] != max_new_tokens:
                self.generated = torch.full((B, max_new_tokens), pad_token_id, dtype=torch.int64,
                                            device=self.device)
                self.graph = None  # the recorded step writes into this buffer
                self.graph_multi = {}
            self.generated.fill_(pad_token_id)
        self._masks()
        # bound on every row's position for run()'s choice of split plan (one
        # host sync per batch)
        self._pos_hi = int(positions.max()) if positions.numel() else 0

    def capture(self):
        """Record one step into a HIP graph (after two warm-up steps on a side stream)."""
        # A warm-up step writes K/V only at each active row's slot pos[b], which
        # is not yet valid cache content: the first real step rewrites it before
        # attention reads it.  Row state is saved and restored around them.
        saved = [t.clone() for t in (self.tokens, self.pos, self.count, self.active)]
        s = torch.cuda.Stream(device=self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(s):
            for _ in range(2):
                self._step()
                self._restore(saved)
        torch.cuda.current_stream(self.device).wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            self._step()
        self._restore(saved)
        self.graph = g
        self.graph_multi = {}  # recorded at their first use (run)

    def _restore(self, saved):
        for t, v in zip((self.tokens, self.pos, self.count, self.active), saved):
            t.copy_(v)
        if self.generated is not None:
            self.generated.fill_(int(self.pad.item()))
        self._masks()

    def verify_handover(self):
        """Check the in-kernel hand-overs of the steps run so far (host sync).

        The attention's split merge and o_proj's in-kernel finish hand partial
        results to the last-arriving workgroup of a group through an L2 counter,
        which is correct only when the group's workgroups ran on one XCD.  The
        kernels flag a group that did not (``xcd_err``), and such a group leaves
        its counter non-zero.  Either means the outputs of the run are not
        valid: this raises ``RuntimeError`` and switches the in-kernel
        hand-overs off (``ATTN_MERGE``, ``O_FIN``) for engines built later, which
        then take the launches that need no hand-over."""
        bad = int(self.xcd_err.item()) != 0
        ws_scr = getattr(self, "ws_scr", None)  # the screened lm_head's counters
        lm_cnt = ws_scr[:1024] if ws_scr is not None else None
        for cnt in (self.m_cnt, getattr(self, "o_cnt", None) if self.o_fin else None, lm_cnt):
            if cnt is not None and bool((cnt != 0).any()):
                bad = True
        if bad:
            DecodeEngine.ATTN_MERGE = False
            DecodeEngine.O_FIN = False
            DecodeEngine.LM_SCREEN = False
            raise RuntimeError("decode step: a group of workgroups that hands data over "
                               "through L2 did not run on one XCD; the results of this run "
                               "are not valid (in-kernel hand-overs now off; run again)")

    def step(self):
        if self.graph is not None:
            self.graph.replay()
        else:
            self._step()

    # steps recorded in one graph for run(): one graph launch per 16 steps
    # instead of one per step (7 us per step less at config 3)
    MULTI_STEP = 16

    # Attention splits planned for the live context: the attention and the
    # o_proj that reads its partials plan their context splits for pw blocks
    # instead of the table width, pw covering every row's context in the
    # graph's MULTI_STEP steps (rounded up to a multiple of an eighth of the
    # table: at most 8 recorded graphs).  Fewer split slots for o_proj to
    # stage while the contexts are short.  Where the table width plans 8
    # blocks per split (config 3's 64-block tables), every width does, and
    # the splits, and so the results, are the same as at the full width.
    # Only where every split of every (row, KV head) pair still has a CU of its
    # own (B * Hkv * 8 <= 256): more workgroups than CUs run in two rounds
    # (config 4's 32-row engine: 8867 tok/s planned live against 8927).
    LIVE_WIDTH = True
    _pw: Optional[int] = None  # plan width of the launches being built (None: the table's)
    _pos_hi: Optional[int] = None

    def _live_width(self, ctx: int) -> int:
        """Plan width (blocks) covering contexts of up to ``ctx`` tokens."""
        full = self.max_blocks
        if not (self.LIVE_WIDTH and getattr(self, "attn_fused", False)
                and getattr(self, "attn_splits", 1) > 1 and self.B * self.Hkv * 8 <= 256):
            return full
        unit = max(8, -(-full // 8))
        need = -(-max(ctx, 1) // self.pool.block_size)
        return min(full, -(-need // unit) * unit)

    def _multi_graph(self, pw: Optional[int] = None) -> torch.cuda.CUDAGraph:
        pw = pw or self.max_blocks
        g = self.graph_multi.get(pw)
        if g is None:
            # recording executes nothing: the row state is untouched
            s = torch.cuda.Stream(device=self.device)
            s.wait_stream(torch.cuda.current_stream(self.device))
            g = torch.cuda.CUDAGraph()
            self._pw = pw
            try:
                with torch.cuda.graph(g, stream=s):
                    for _ in range(self.MULTI_STEP):
                        self._step()
            finally:
                self._pw = None
            torch.cuda.current_stream(self.device).wait_stream(s)
            self.graph_multi[pw] = g
        return g

    def run(self, steps: int):
        """``steps`` decode steps: graph replays of MULTI_STEP steps, then
        single steps (rows that stop in between do nothing in later steps).
        Each replay's attention splits are planned for the contexts its steps
        can reach (every row's position advances by at most one per step)."""
        if self.graph is not None and steps >= self.MULTI_STEP:
            while steps >= self.MULTI_STEP:
                pw = (self._live_width(self._pos_hi + self.MULTI_STEP)
                      if self._pos_hi is not None else None)
                self._multi_graph(pw).replay()
                if self._pos_hi is not None:
                    self._pos_hi += self.MULTI_STEP
                steps -= self.MULTI_STEP
        for _ in range(steps):
            self.step()
            if self._pos_hi is not None:
                self._pos_hi += 1

    def compaction_engines(self, sizes=(24, 16, 8)) -> list:
        """Greedy engines of fewer rows (``sizes`` below this engine's) over the
        same model, pool and block-table width, for ``run_paged(...,
        compact=...)``: once the rows still decoding fit a smaller engine,
        their state moves there and the rollout goes on with that engine's
        cheaper step.  Sampling engines are not compacted: a row's draws are
        keyed by its row index, which compaction changes."""
        if self.sampling:
            raise ValueError("row compaction renumbers rows, which changes sampled draws "
                             "(keyed by the row index); it is for greedy decoding")
        return [DecodeEngine(self.model, self.pool, n, self.max_blocks, max_pos=self.max_pos)
                for n in sorted({int(n) for n in sizes if 0 < int(n) < self.B}, reverse=True)]

    def _ready_for(self, width: int) -> None:
        """A generated buffer of ``width`` columns and a captured step, every row idle."""
        if self.graph is not None and self.generated is not None and \
                self.generated.shape[1] == width:
            return
        B, dev = self.B, self.device
        z = torch.zeros(B, dtype=torch.int64, device=dev)
        self.start(z, z, torch.full((B, 1), -1, dtype=torch.int32, device=dev), z, width)
        self.capture()

    def _take_rows(self, src: "DecodeEngine", rows: list) -> None:
        """Rows ``rows`` of ``src`` (state, block tables, tokens generated so
        far) become rows 0 .. len(rows) - 1 of this engine; the others idle."""
        n = len(rows)
        idx = torch.tensor(rows, dtype=torch.long, device=self.device)
        for name in ("tokens", "pos", "count", "limit", "active"):
            dst = getattr(self, name)
            dst.zero_()
            dst[:n].copy_(getattr(src, name).index_select(0, idx))
        self.eos.copy_(src.eos)
        self.pad.copy_(src.pad)
        self.block_tables.fill_(-1)
        self.block_tables[:n].copy_(src.block_tables.index_select(0, idx))
        self.generated.copy_(src.pad.view(1, 1).expand_as(self.generated))
        self.generated[:n].copy_(src.generated.index_select(0, idx))
        self._masks()
        self._pos_hi = src._pos_hi

    def run_paged(self, sids: list, max_steps: int, chunk: Optional[int] = None,
                  check_invariants: bool = False, compact: Optional[list] = None) -> dict:
        """Decode until every row has stopped (or ``max_steps``), allocating each
        row's KV blocks one chunk ahead and releasing them when the row stops.

        ``sids[b]`` is the pool sequence of row ``b`` (its table row already
        loaded by ``start``).  Every ``chunk`` steps (default: the block size,
        so a row needs at most one new block per chunk) the host reads the
        rows' positions and activity -- the only synchronisation -- then
        releases the blocks of rows that stopped (``PagedKVPool.free``: shared
        prompt blocks return to the free list with their last reference),
        reserves blocks for the next ``chunk`` positions of every active row and
        writes the new entries into the device block table.  The steps in
        between are graph replays.  The reference allocates one cache for the
        whole call instead (``paged_kv.py:626-645``); BASELINE config 4 asks
        for blocks allocated and freed as sequences finish.

        ``compact`` (engines from ``compaction_engines``): at a chunk boundary
        where the rows still decoding fit a smaller engine, they move to the
        smallest that holds them (``_take_rows``) and the following steps run
        on it; at the end every row's tokens are back in this engine's
        ``generated``.  A long-tailed group (config 4: lognormal lengths, most
        rows done long before the longest) then spends its tail on the step of
        8 rows instead of 32.  Each row's arithmetic is its own in every
        engine, but the engines' kernels sum in different orders, so a token
        can differ where the top two logits are within rounding.

        Returns ``dict(steps, peak_blocks, engines)``: decode steps run, the
        most blocks in use at once and the row counts of the engines used.
        """
        pool = self.pool
        chunk = chunk or pool.block_size
        if compact and getattr(self, "sampling", False):
            raise ValueError("row compaction is for greedy decoding (sampled draws are keyed "
                             "by the row index)")
        for e in compact or ():
            if e.pool is not pool or e.max_blocks != self.max_blocks or \
                    getattr(e, "sampling", False):
                raise ValueError("compaction engines must be greedy engines over this engine's "
                                 "pool and block-table width (compaction_engines)")
        ladder = sorted((e for e in (compact or ()) if e.B < self.B), key=lambda e: e.B)
        eng, used = self, [self]
        origin = list(range(len(sids)))  # row of eng -> row of this engine
        live = {b: s for b, s in enumerate(sids)}
        steps = peak = 0
        while True:
            pos = eng.pos.cpu().tolist()
            act = eng.active.cpu().tolist()
            for b in [b for b in live if not act[b]]:
                pool.free(live.pop(b))
                eng.block_tables[b].fill_(-1)
            if not live or steps >= max_steps:
                break
            fit = [e for e in ladder if len(live) <= e.B < eng.B]
            if fit:
                dst = fit[0]
                dst._ready_for(self.generated.shape[1])
                if eng is not self:
                    self._put_back(eng, origin)
                rows = sorted(live)
                dst._take_rows(eng, rows)
                eng.active.zero_()  # the moved rows go on in dst only
                eng._masks()
                origin = [origin[b] for b in rows]
                live = {i: live[b] for i, b in enumerate(rows)}
                pos = [pos[b] for b in rows]
                eng = dst
                used.append(dst)
            n = min(chunk, max_steps - steps)
            for b, sid in live.items():
                have = len(pool.blocks[sid])
                pool.set_length(sid, pos[b])
                pool.reserve(sid, pos[b] + n)  # slots pos .. pos + n - 1
                bl = pool.blocks[sid]
                if len(bl) > eng.max_blocks:
                    raise RuntimeError(f"row {b} needs {len(bl)} blocks; the engine's block "
                                       f"table holds {eng.max_blocks}")
                if len(bl) > have:
                    eng.block_tables[b, have:len(bl)].copy_(
                        torch.tensor(bl[have:], dtype=torch.int32))
            if check_invariants:
                pool.check_invariants()
            peak = max(peak, pool.num_blocks - pool.num_free)
            eng._pos_hi = max(pos)
            eng.run(n)
            steps += n
        for b in list(live):  # rows cut off by max_steps
            pool.free(live.pop(b))
            eng.block_tables[b].fill_(-1)
        if eng is not self:
            self._put_back(eng, origin)
        for e in used:
            e.verify_handover()
        return dict(steps=steps, peak_blocks=peak, engines=[e.B for e in used])

    def _put_back(self, eng: "DecodeEngine", origin: list) -> None:
        """Copy rows 0 .. len(origin) - 1 of ``eng.generated`` to this engine's rows ``origin``."""
        idx = torch.tensor(origin, dtype=torch.long, device=self.device)
        self.generated.index_copy_(0, idx, eng.generated[:len(origin)])


class PrefillEngine(DecodeEngine):
    """Chunked paged prefill: ``chunk`` prompt tokens of one sequence per pass,
    as rows at positions p .. p + c - 1 that share the sequence's block table.

    The reference prefills with one transformers forward of ``prompt[:-1]`` and
    a Python scatter of its K/V into the paged cache, one ``.item()`` per
    (layer, row, token) (``paged_kv.py:547-586``).  Here a chunk is one pass of
    the decode layers in which every row's K/V is appended first
    (``grpo_qkv_rope_append_parts``) and attention runs after
    (``grpo_paged_attn_decode``, row i over p + i + 1 tokens), so row i sees
    the chunk's earlier tokens as a causal forward does; o_proj reads the bf16
    attention output.  No final norm or lm_head runs: prefill only fills the
    cache.  The pass is captured once into a HIP graph; rows past the end of a
    short last chunk are masked (slot -1, length 0).
    """
    # o_proj partial sums from the bf16 attention output (no in-kernel finish)
    O_FIN = False
    O_TILE = False

    def __init__(self, model: Qwen2ForCausalLM, pool: PagedKVPool, chunk: int, max_blocks: int,
                 max_pos: Optional[int] = None):
        super().__init__(model, pool, chunk, max_blocks, max_pos=max_pos)
        bf = dict(dtype=torch.bfloat16, device=self.device)
        self.q_rot = torch.zeros(chunk, self.Hq, self.D, **bf)
        self.attn_out = torch.zeros(chunk, self.Hq * self.D, **bf)
        self._rows = torch.arange(chunk, dtype=torch.int32, device=self.device)

    def _attn_launches(self, L: dict, kc: int, vc: int, st) -> list:
        return self._attn_launches_unfused(L, kc, vc, st)

    def _head_launches(self, prev: dict, st) -> list:
        return []

    def _step(self):
        self._forward()

    def run_prompt(self, table: torch.Tensor, prompt: torch.Tensor, n: int):
        """Cache tokens ``prompt[0 .. n-1]`` at positions 0 .. n-1 of the sequence
        whose block table row is ``table`` ([1, w] int32, its blocks reserved)."""
        if self.graph is None:
            self.active.zero_()  # the warm-up passes append nothing
            self.capture()
        w = table.shape[1]
        self.block_tables.fill_(-1)
        self.block_tables[:, :w].copy_(table.view(1, w).expand(self.B, w))
        none = torch.full_like(self._rows, -1)
        for p in range(0, n, self.B):
            c = min(self.B, n - p)
            valid = self._rows < c
            self.tokens.zero_()
            self.tokens[:c].copy_(prompt[p:p + c])
            self.append_pos.copy_(torch.where(valid, self._rows + p, none))
            self.attn_len.copy_(torch.where(valid, self._rows + (p + 1), none + 1))
            self.step()


class GemmPrefillEngine:
    """Chunked paged prefill with wide chunks: up to ``chunk`` (default 512)
    prompt tokens of one sequence per pass, every linear on the NF4 GEMM
    (``grpo_nf4_lora_linear`` beyond 64 rows: ``nf4_gemm_mfma``), so a
    511-token prompt reads each NF4 weight once per row tile of one pass
    instead of once per 64-token chunk.

    The rows are positions p .. p + c - 1 sharing the sequence's block table,
    as in ``PrefillEngine``, and every launch keeps the decode step's rounding
    points: embedding -> per layer RMSNorm (+ the residual add of the previous
    layer's down_proj) -> q|k|v (grouped: one GEMM per projection, bias and
    LoRA in the kernel) -> RoPE + K/V append (``grpo_rope_append``) ->
    attention over p + i + 1 tokens (``grpo_paged_attn_decode``) -> o_proj ->
    residual add + RMSNorm -> gate|up with SiLU*up in its epilogue
    (``grpo_nf4_gate_up_silu``) -> down_proj.  The reference
    prefills with one transformers forward and a per-token scatter of K/V
    (``paged_kv.py:547-586``).  Only the cache is filled: the last layer stops
    after its append (its attention and MLP feed nothing that is kept).  The
    pass is captured once into a HIP graph; rows past the end of a short last
    chunk are masked (slot -1, length 0)."""

    def __init__(self, model: Qwen2ForCausalLM, pool: PagedKVPool, chunk: int, max_blocks: int,
                 max_pos: Optional[int] = None):
        self.lib = _lib.device_library()
        cfg = model.config
        self.model, self.pool, self.cfg = model, pool, cfg
        self.B, self.max_blocks = chunk, max_blocks
        dev = pool.k.device
        self.device = dev
        H, D = cfg.hidden_size, cfg.head_dim
        self.Hq, self.Hkv, self.D, self.H = (cfg.num_attention_heads, cfg.num_key_value_heads, D,
                                             H)
        self.I, self.V = cfg.intermediate_size, cfg.vocab_size
        self.nqkv = (self.Hq + 2 * self.Hkv) * D
        self.bs = cfg.nf4_blocksize
        self.max_pos = max_pos or max_blocks * pool.block_size
        self.cos, self.sin = model.model.rotary_emb.tables(self.max_pos)
        bf = dict(dtype=torch.bfloat16, device=dev)
        i32 = dict(dtype=torch.int32, device=dev)
        B = chunk
        self.tokens = torch.zeros(B, dtype=torch.int64, device=dev)
        self.append_pos = torch.full((B,), -1, **i32)
        self.attn_len = torch.zeros(B, **i32)
        self.block_tables = torch.full((B, max_blocks), -1, **i32)
        self.h = torch.zeros(B, H, **bf)
        self.x = torch.zeros(B, H, **bf)
        self.y = torch.zeros(B, H, **bf)            # o_proj and down_proj outputs
        self.qkv = torch.zeros(B, self.nqkv, **bf)
        self.q_rot = torch.zeros(B, self.Hq, D, **bf)
        self.attn_out = torch.zeros(B, self.Hq * D, **bf)
        self.gu = torch.zeros(B, 2 * self.I, **bf)
        self.act = torch.zeros(B, self.I, **bf)
        self._rows = torch.arange(B, dtype=torch.int32, device=dev)
        self._keep = []
        self.layers = []
        ws = 0
        for layer in model.model.layers:
            at, mlp = layer.self_attn, layer.mlp
            projs = [at.q_proj, at.k_proj, at.v_proj]
            r = projs[0].rank
            arr = ctypes.c_void_p * 4
            bias = arr(*[p.base_layer.bias.data_ptr() if p.base_layer.bias is not None else None
                         for p in projs], None)
            la = arr(*[p.lora_A.weight.data_ptr() if r > 0 else None for p in projs], None)
            lb = arr(*[p.lora_B.weight.data_ptr() if r > 0 else None for p in projs], None)
            seg = (ctypes.c_int * 4)(*at.qkv.seg_rows, 0)
            self._keep += [bias, la, lb, seg]
            o = at.o_proj
            oq = o.base_layer.weight.quant_state
            dq = mlp.down_proj.weight.quant_state
            self.layers.append(dict(
                in_norm=layer.input_layernorm.weight, post_norm=layer.post_attention_layernorm.weight,
                eps=float(layer.input_layernorm.variance_epsilon),
                qkv=at.qkv, bias=bias, la=la, lb=lb, seg=seg, r=r, scaling=float(projs[0].scaling),
                o_w=o.base_layer.weight, o_absmax=float_absmax(oq), o_code=oq.code,
                o_bias=o.base_layer.bias, o_la=o.lora_A.weight, o_lb=o.lora_B.weight,
                o_r=o.rank, o_scaling=float(o.scaling),
                gu=mlp.gate_up, down_w=mlp.down_proj.weight, down_absmax=float_absmax(dq),
                down_code=dq.code))
            for (n, k, rr, nseg) in ((self.nqkv, H, r, 3), (H, self.Hq * D, o.rank, 1),
                                     (2 * self.I, H, 0, 1), (H, self.I, 0, 1)):
                ws = max(ws, int(self.lib.grpo_nf4_lora_linear_workspace_bytes(
                    B, n, k, rr, nseg, self.bs)))
        # one workspace for every linear (they run one after another on one stream)
        self.ws = torch.empty(max(ws, 16), dtype=torch.uint8, device=dev)
        self.ws_attn = ops.workspace("paged_attn_prefill", max(ops.paged_attention_workspace_bytes(
            B, self.Hq, self.Hkv, D, pool.block_size, max_blocks), 1), dev)
        self.embed = model.model.embed_tokens.weight
        self.gu_fused = bool(self.lib.grpo_nf4_gate_up_silu_supported(B, self.I, H, self.bs))
        self.graph: Optional[torch.cuda.CUDAGraph] = None

    def launches(self) -> list:
        """[(kind, launch())] of one pass, bound to torch's current stream."""
        lib, st, chk = self.lib, _lib.stream_handle(self.device), _lib.check
        B, H, I, D, Hq, Hkv = self.B, self.H, self.I, self.D, self.Hq, self.Hkv
        pool, bs = self.pool, self.bs
        h, x, y = self.h.data_ptr(), self.x.data_ptr(), self.y.data_ptr()
        qkv, q, ao = self.qkv.data_ptr(), self.q_rot.data_ptr(), self.attn_out.data_ptr()
        gu, act = self.gu.data_ptr(), self.act.data_ptr()
        ws, ws_n = self.ws.data_ptr(), self.ws.numel()
        wsa, wsa_n = self.ws_attn.data_ptr(), self.ws_attn.numel()
        bt, ap, al = self.block_tables.data_ptr(), self.append_pos.data_ptr(), self.attn_len.data_ptr()
        ptr = _lib.ptr

        def linear(xp, ldx, w, absmax, code, bias, la, lb, r, sc, out, n, k):
            return chk(lib.grpo_nf4_lora_linear(
                xp, ldx, w.data_ptr(), absmax.data_ptr(), code.data_ptr(), bs, ptr(bias),
                ptr(la) if r > 0 else None, ptr(lb) if r > 0 else None, r, sc, out, n, B, n, k,
                ws, ws_n, st), "prefill linear")

        out = [("embedding", lambda: chk(lib.grpo_embedding(
            self.tokens.data_ptr(), self.embed.data_ptr(), self.V, H, h, B, st), "embedding"))]
        last = len(self.layers) - 1
        for li, L in enumerate(self.layers):
            kc, vc = (t.data_ptr() for t in pool.layer(li))
            # h += the previous layer's down_proj output; x = RMSNorm(h)
            res = None if li == 0 else y
            out.append(("rmsnorm", lambda L=L, res=res: chk(lib.grpo_add_rmsnorm(
                res if res is not None else h, h if res is not None else None,
                h if res is not None else None, L["in_norm"].data_ptr(), x, B, H, L["eps"], st),
                "rmsnorm")))
            qs = L["qkv"]
            out.append(("qkv", lambda L=L, qs=qs: chk(lib.grpo_nf4_lora_linear_grouped(
                x, H, qs.packed.data_ptr(), qs.absmax.data_ptr(), qs.code.data_ptr(), bs, 3,
                L["seg"], L["bias"], L["la"], L["lb"], L["r"], L["scaling"], qkv, self.nqkv, B,
                H, ws, ws_n, st), "qkv")))
            out.append(("append", lambda kc=kc, vc=vc: chk(lib.grpo_rope_append(
                qkv, self.nqkv, Hq, Hkv, D, self.cos.data_ptr(), self.sin.data_ptr(),
                self.max_pos, ap, q, kc, vc, pool.num_blocks, bt, self.max_blocks,
                pool.block_size, self.max_blocks, B, st), "append")))
            if li == last:
                break  # the last layer's attention and MLP feed nothing kept
            out.append(("attention", lambda kc=kc, vc=vc: chk(lib.grpo_paged_attn_decode(
                q, Hq * D, D, kc, vc, pool.num_blocks, bt, self.max_blocks, al, ao, 1, B, Hq,
                Hkv, D, pool.block_size, self.max_blocks, 1.0 / math.sqrt(D), wsa, wsa_n, st),
                "attention")))
            out.append(("o", lambda L=L: linear(
                ao, Hq * D, L["o_w"], L["o_absmax"], L["o_code"], L["o_bias"], L["o_la"],
                L["o_lb"], L["o_r"], L["o_scaling"], y, H, Hq * D)))
            out.append(("rmsnorm", lambda L=L: chk(lib.grpo_add_rmsnorm(
                y, h, h, L["post_norm"].data_ptr(), x, B, H, L["eps"], st), "post_norm")))
            g = L["gu"]
            if self.gu_fused:  # gate|up with SiLU*up in the GEMM's epilogue
                out.append(("gate_up", lambda g=g: chk(lib.grpo_nf4_gate_up_silu(
                    x, H, g.packed.data_ptr(), g.absmax.data_ptr(), g.code.data_ptr(), bs, I, H,
                    B, act, I, st), "gate_up")))
            else:
                out.append(("gate_up", lambda g=g: chk(lib.grpo_nf4_lora_linear(
                    x, H, g.packed.data_ptr(), g.absmax.data_ptr(), g.code.data_ptr(), bs, None,
                    None, None, 0, 1.0, gu, 2 * I, B, 2 * I, H, ws, ws_n, st), "gate_up")))
                out.append(("silu_mul", lambda: chk(lib.grpo_silu_mul(
                    gu, 2 * I, I, act, I, B, st), "silu_mul")))
            out.append(("down", lambda L=L: linear(
                act, I, L["down_w"], L["down_absmax"], L["down_code"], None, None, None, 0, 1.0,
                y, H, I)))
        return out

    def _forward(self):
        for _, fn in self.launches():
            fn()

    def capture(self):
        """Record one pass into a HIP graph (after a warm-up pass that appends
        nothing: every row masked)."""
        self.append_pos.fill_(-1)
        self.attn_len.zero_()
        s = torch.cuda.Stream(device=self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(s):
            self._forward()
        torch.cuda.current_stream(self.device).wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            self._forward()
        self.graph = g

    def step(self):
        if self.graph is not None:
            self.graph.replay()
        else:
            self._forward()

    def run_prompt(self, table: torch.Tensor, prompt: torch.Tensor, n: int):
        """Cache tokens ``prompt[0 .. n-1]`` at positions 0 .. n-1 of the sequence
        whose block table row is ``table`` ([1, w] int32, its blocks reserved)."""
        if self.graph is None:
            self.capture()
        w = table.shape[1]
        self.block_tables.fill_(-1)
        self.block_tables[:, :w].copy_(table.view(1, w).expand(self.B, w))
        none = torch.full_like(self._rows, -1)
        for p in range(0, n, self.B):
            c = min(self.B, n - p)
            valid = self._rows < c
            self.tokens.zero_()
            self.tokens[:c].copy_(prompt[p:p + c])
            self.append_pos.copy_(torch.where(valid, self._rows + p, none))
            self.attn_len.copy_(torch.where(valid, self._rows + (p + 1), none + 1))
            self.step()


def release_decode_caches(model=None) -> None:
    """Free what the decode path keeps between rollouts, e.g. before the
    training phase: the tile-order lm_head copy on ``model`` (and on its
    adapted decode view; V * H * 2 bytes) and the packed LoRA A copies of the
    one-launch linear.  The next rollout rebuilds them (one copy kernel each)."""
    from . import adapt

    models = [] if model is None else [model, adapt._cache.get(model)]
    for m in models:
        for attr in ("_grpo_lm_tiles", "_grpo_lm_q8"):
            if m is not None and hasattr(m, attr):
                delattr(m, attr)
    ops._packed_a.clear()


# ------------------------------------------------------------- drop-in ---

def _prompt_rows(input_ids: torch.Tensor, attention_mask: Optional[torch.Tensor]):
    ids = input_ids.detach().cpu()
    mask = None if attention_mask is None else attention_mask.detach().cpu()
    rows = []
    for b in range(ids.shape[0]):
        r = ids[b] if mask is None else ids[b][mask[b].bool()]
        rows.append(tuple(int(t) for t in r.tolist()))
    return rows


def prefill_chunk(n: int, cap: int = 64) -> int:
    """Rows of a ``PrefillEngine`` for prompts of up to ``n`` cached tokens."""
    return max(1, min(cap, n))


# Prompts of more than this many cached tokens prefill on the NF4 GEMM
# (``GemmPrefillEngine``, chunks of up to GEMM_PREFILL_CHUNK rows); shorter ones
# on the decode step's launches (``PrefillEngine``).
GEMM_PREFILL_MIN = 64
GEMM_PREFILL_CHUNK = 512


def prefill_engine(model: Qwen2ForCausalLM, pool: PagedKVPool, n: int, width: int,
                   max_pos: Optional[int] = None):
    """The prefill engine for prompts of up to ``n`` cached tokens over block
    tables of ``width`` entries: ``GemmPrefillEngine`` beyond GEMM_PREFILL_MIN
    tokens (chunk = n rounded up to 64, at most GEMM_PREFILL_CHUNK), else a
    ``PrefillEngine`` of ``prefill_chunk(n)`` rows."""
    if n > GEMM_PREFILL_MIN:
        chunk = min(GEMM_PREFILL_CHUNK, (n + 63) // 64 * 64)
        return GemmPrefillEngine(model, pool, chunk, width, max_pos=max_pos)
    return PrefillEngine(model, pool, prefill_chunk(n), width, max_pos=max_pos)


@torch.no_grad()
def prefill(engine1: DecodeEngine, pool: PagedKVPool, prompt: tuple, width: int) -> int:
    """Prefill of ``prompt[:-1]`` into a new pool sequence: chunked when
    ``engine1`` is a ``PrefillEngine``, else teacher-forced one token per step
    through a B = 1 decode engine."""
    sid = pool.allocate(len(prompt))
    n = len(prompt) - 1
    if n > 0 and isinstance(engine1, (PrefillEngine, GemmPrefillEngine)):
        dev = engine1.device
        engine1.run_prompt(pool.block_table([sid], width, device=dev),
                           torch.tensor(prompt, dtype=torch.int64, device=dev), n)
    elif n > 0:
        dev = engine1.device
        tbl = pool.block_table([sid], width, device=dev)
        engine1.start(torch.tensor([prompt[0]], device=dev), torch.zeros(1, device=dev), tbl,
                      torch.tensor([n], device=dev), n, record=False)
        prompt_t = torch.tensor(prompt, dtype=torch.int64, device=dev)
        for t in range(n):
            engine1.tokens.copy_(prompt_t[t:t + 1])  # teacher forcing
            engine1.step()
    pool.set_length(sid, n)
    return sid


@torch.no_grad()
def paged_kv_decode_model(model: Qwen2ForCausalLM, input_ids: torch.Tensor,
                          attention_mask: Optional[torch.Tensor] = None,
                          max_new_tokens: int = 128, do_sample: bool = False,
                          temperature: float = 1.0, top_p: float = 1.0,
                          pad_token_id: Optional[int] = 0,
                          eos_token_id: Optional[int] = None,
                          seed: Optional[int] = None, block_size: int = 16,
                          use_cache: Optional[bool] = None,
                          stop_lengths: Optional[list[int]] = None) -> torch.Tensor:
    """Drop-in for ``paged_kv.paged_kv_decode_model``: returns ``[B, max_new_tokens]``.

    ``model`` is either this package's ``Qwen2ForCausalLM`` or a transformers
    Qwen2 model in the reference's training layout (NF4 linears, LoRA on
    q/k/v/o), adapted once by ``rollout.adapt.decode_model_from``.

    Rows with identical (unpadded) prompts share one prefill; their full prompt
    blocks are shared through the pool and the partial last block is copied
    per row.  ``stop_lengths`` (an extension) caps each row's generated length.
    Decoding (greedy, or sampled with the reference's temperature / top-p rule,
    draws fixed by ``seed``) runs in the captured graph; every
    block-size steps the host
    gives growing rows their next block and frees the blocks of rows that
    stopped (``DecodeEngine.run_paged``), and decoding ends once every row has
    stopped (the reference's ``finished.all()`` exit, ``paged_kv.py:903``).
    """
    if max_new_tokens <= 0:
        raise ValueError(f"max_new_tokens must be > 0, got {max_new_tokens}.")
    if pad_token_id is None:  # as the low-level entry (paged_kv.py:876-877)
        pad_token_id = 0
    if input_ids.ndim != 2 or input_ids.shape[1] == 0:
        raise ValueError("input_ids must be [batch, seq_len] with at least 1 token.")
    model = decode_model_from(model)
    cfg = model.config
    dev = input_ids.device
    rows = _prompt_rows(input_ids, attention_mask)
    B = len(rows)
    max_ctx = max(len(r) for r in rows) + max_new_tokens
    width = -(-max_ctx // block_size)
    uniq = sorted(set(rows), key=rows.index)
    nblocks = len(uniq) * width + B * (width + 1)
    pool = PagedKVPool(cfg.num_hidden_layers, nblocks, cfg.num_key_value_heads, cfg.head_dim,
                       block_size, device=dev)
    pre = prefill_engine(model, pool, max(len(r) for r in uniq) - 1, width)
    parents = {p: prefill(pre, pool, p, width) for p in uniq}
    del pre
    sids = []
    for r in rows:
        # room for the first decode slot; run_paged grows the row from there
        (cid,) = pool.fork(parents[r], 1, reserve_tokens=len(r))
        sids.append(cid)
    for p in parents.values():
        pool.free(p)
    pool.check_invariants()
    if seed is None:  # paged_kv.py:668-671: unseeded calls draw from torch's global RNG
        seed = int(torch.randint(0, 2 ** 62, (1,)).item())
    eng = DecodeEngine(model, pool, B, width, do_sample=do_sample, temperature=temperature,
                       top_p=top_p, seed=seed)
    limits = torch.tensor(stop_lengths if stop_lengths is not None else [max_new_tokens] * B,
                          dtype=torch.int32, device=dev).clamp(max=max_new_tokens)
    eng.start(torch.tensor([r[-1] for r in rows], device=dev),
              torch.tensor([len(r) - 1 for r in rows], device=dev),
              pool.block_table(sids, width, device=dev), limits, max_new_tokens,
              eos_token_id=eos_token_id, pad_token_id=pad_token_id)
    eng.capture()
    eng.start(torch.tensor([r[-1] for r in rows], device=dev),
              torch.tensor([len(r) - 1 for r in rows], device=dev),
              pool.block_table(sids, width, device=dev), limits, max_new_tokens,
              eos_token_id=eos_token_id, pad_token_id=pad_token_id)
    eng.run_paged(sids, max_new_tokens)
    return eng.generated.clone()


__all__ = ["DecodeEngine", "PrefillEngine", "GemmPrefillEngine", "paged_kv_decode_model",
           "prefill", "prefill_chunk", "prefill_engine", "release_decode_caches"]
