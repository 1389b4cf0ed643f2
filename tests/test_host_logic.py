"""CPU tests of host-side logic: the paged KV block pool and argument validation."""

import pytest
import torch

from grpo_mi355x.core.kv_pool import PagedKVPool


def test_pool_allocate_reserve_free():
    pool = PagedKVPool(2, 10, 2, 8, block_size=4)
    a = pool.allocate(9)  # 3 blocks
    assert len(pool.blocks[a]) == 3 and pool.num_free == 7
    pool.reserve(a, 12)  # still 3 blocks
    assert len(pool.blocks[a]) == 3
    pool.reserve(a, 13)
    assert len(pool.blocks[a]) == 4
    pool.check_invariants()
    pool.free(a)
    assert pool.num_free == 10
    pool.check_invariants()


def test_pool_out_of_blocks_raises():
    pool = PagedKVPool(1, 2, 1, 4, block_size=4)
    pool.allocate(8)
    with pytest.raises(RuntimeError, match="out of memory"):
        pool.allocate(1)


def test_fork_shares_full_blocks_and_copies_partial():
    pool = PagedKVPool(2, 32, 2, 8, block_size=4)
    p = pool.allocate(10)
    pool.set_length(p, 10)  # 2 full blocks + 2 tokens in the third
    pool.k[:, pool.blocks[p][2]] = 7.0
    kids = pool.fork(p, 3, reserve_tokens=20)
    for c in kids:
        assert pool.blocks[c][:2] == pool.blocks[p][:2]           # shared prefix
        assert pool.blocks[c][2] != pool.blocks[p][2]             # private copy of the tail
        assert torch.all(pool.k[:, pool.blocks[c][2]] == 7.0)     # copied content
        assert len(pool.blocks[c]) == 5
    assert pool.refcount[pool.blocks[p][0]] == 4
    pool.check_invariants()
    pool.free(p)
    pool.check_invariants()
    assert pool.refcount[pool.blocks[kids[0]][0]] == 3
    for c in kids:
        pool.free(c)
    assert pool.num_free == 32
    pool.check_invariants()


def test_fork_at_block_boundary_shares_everything():
    pool = PagedKVPool(1, 16, 1, 4, block_size=4)
    p = pool.allocate(8)
    pool.set_length(p, 8)
    (c,) = pool.fork(p, 1, reserve_tokens=12)
    assert pool.blocks[c][:2] == pool.blocks[p][:2] and len(pool.blocks[c]) == 3
    pool.check_invariants()


def test_invariant_checker_catches_shared_writable_block():
    pool = PagedKVPool(1, 8, 1, 4, block_size=4)
    a = pool.allocate(8)
    pool.set_length(a, 5)
    b = pool.allocate(0)
    pool.blocks[b] = [pool.blocks[a][1]]  # b aliases a's writable block
    pool.refcount[pool.blocks[a][1]] += 1
    with pytest.raises(AssertionError, match="shared block"):
        pool.check_invariants()


def test_block_table_padding():
    pool = PagedKVPool(1, 8, 1, 4, block_size=4)
    a, b = pool.allocate(8), pool.allocate(3)
    t = pool.block_table([a, b], 4)
    assert t.dtype == torch.int32 and t.shape == (2, 4)
    assert t[1, 1:].tolist() == [-1, -1, -1]
    with pytest.raises(ValueError):
        pool.block_table([a], 1)


def test_lora_validation_messages_match_reference():
    from grpo_mi355x.kernels.lora_forward import _validate_inputs

    class QS:
        shape = (8, 16)

    x = torch.zeros(2, 16)
    with pytest.raises(ValueError, match=r"x must be \[batch, seq_len, hidden\]"):
        _validate_inputs(x, torch.zeros(1), QS(), torch.zeros(4, 16), torch.zeros(8, 4))
    with pytest.raises(ValueError, match="must be on CUDA"):
        _validate_inputs(torch.zeros(1, 2, 16), torch.zeros(1), QS(), torch.zeros(4, 16),
                         torch.zeros(8, 4))


def test_lora_dropout_rejected_before_any_kernel():
    from grpo_mi355x.kernels.lora_forward import lora_fused_forward

    with pytest.raises(ValueError, match="Dropout"):
        lora_fused_forward(torch.zeros(1, 1, 4), base_layer=object(), lora_A=object(),
                           lora_B=object(), scaling=2.0, dropout=torch.nn.Dropout(0.1))


def test_paged_validation_messages_match_reference():
    from grpo_mi355x.kernels.paged_kv import _validate_inputs

    ids = torch.zeros(2, 3, dtype=torch.long)
    kc = torch.zeros(4, 2, 16, 8, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="input_ids must be"):
        _validate_inputs(torch.zeros(3, dtype=torch.long), kc, kc, torch.zeros(2, 4), torch.zeros(2))
    with pytest.raises(ValueError, match="identical shapes"):
        _validate_inputs(ids, kc, kc[:2], torch.zeros(2, 4), torch.zeros(2))
    with pytest.raises(ValueError, match="batch dimension"):
        _validate_inputs(ids, kc, kc, torch.zeros(3, 4), torch.zeros(2))
    with pytest.raises(ValueError, match="CUDA"):
        _validate_inputs(ids, kc, kc, torch.zeros(2, 4), torch.zeros(2))


def test_manual_lora_layer_surface():
    from grpo_mi355x.core.lora import ManualLoRALayer, get_lora_parameters, inject_lora_layers
    from grpo_mi355x.core.nf4 import Linear4bitNF4

    base = Linear4bitNF4.from_weight(torch.randn(16, 32) * 0.02, torch.zeros(16))
    layer = ManualLoRALayer(base, rank=4, alpha=8)
    assert layer.scaling == 2.0 and layer.rank == 4 and layer.alpha == 8
    assert torch.all(layer.lora_B.weight == 0)
    assert not layer.base_layer.weight.requires_grad
    assert layer.base_layer.weight.quant_state.shape == (16, 32)

    class Tiny(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.q_proj = Linear4bitNF4.from_weight(torch.randn(16, 32))
            self.k_proj = Linear4bitNF4.from_weight(torch.randn(16, 32))
            self.other = torch.nn.Linear(32, 16)

    m = Tiny()
    assert inject_lora_layers(m, ["q_proj", "other"], rank=4, alpha=8) == 1
    assert isinstance(m.q_proj, ManualLoRALayer) and isinstance(m.k_proj, Linear4bitNF4)
    assert len(get_lora_parameters(m)) == 2
    # the quant state survives the dtype cast of inject_lora_layers
    assert m.q_proj.base_layer.weight.quant_state.absmax.dtype == torch.float32


def test_run_paged_reserves_ahead_and_frees_stopped_rows():
    """DecodeEngine.run_paged's block accounting, with a host stand-in for the
    graph step: every slot a row writes is mapped and private when written,
    rows get blocks one chunk ahead, stopped rows release theirs."""
    from grpo_mi355x.core.kv_pool import PagedKVPool
    from grpo_mi355x.rollout.decode import DecodeEngine

    pool = PagedKVPool(1, 64, 1, 8, block_size=4)
    parent = pool.allocate(6)
    pool.set_length(parent, 6)
    sids = pool.fork(parent, 3, reserve_tokens=7)
    pool.free(parent)
    limits = [1, 5, 13]

    class Stand:
        def __init__(self):
            self.pool, self.max_blocks, self.B = pool, 8, 3
            self.pos = torch.full((3,), 6, dtype=torch.int32)
            self.count = torch.zeros(3, dtype=torch.int32)
            self.active = torch.ones(3, dtype=torch.bool)
            self.block_tables = pool.block_table(sids, 8)
            self.in_use = []
            self.verified = 0

        def verify_handover(self):
            self.verified += 1

        def run(self, n):
            for _ in range(n):
                self.step()

        def step(self):
            self.in_use.append(pool.num_blocks - pool.num_free)
            for b in range(3):
                if not self.active[b]:
                    continue
                blk = int(self.block_tables[b, int(self.pos[b]) // 4])
                assert blk >= 0 and pool.refcount[blk] == 1
                self.pos[b] += 1
                self.count[b] += 1
                if int(self.count[b]) >= limits[b]:
                    self.active[b] = False

    s = Stand()
    stats = DecodeEngine.run_paged(s, sids, 50, check_invariants=True)
    assert s.verified == 1  # the in-kernel hand-overs are checked after the run
    assert stats["steps"] == 16  # the longest row stops in the 4th chunk of 4
    assert s.count.tolist() == limits
    # 7 private slots for 6 + 13 tokens: at most one chunk ahead of each live row
    assert stats["peak_blocks"] <= 1 + 3 + 2 + 2 + 5
    assert pool.num_free == pool.num_blocks and not pool.blocks
    assert torch.all(s.block_tables == -1)


def test_run_paged_compaction_moves_live_rows_to_smaller_engines():
    """run_paged with compaction engines (host stand-ins for the graph step,
    whose next token depends only on the row's own token and position): once
    the rows still decoding fit a smaller engine, their state moves to the
    smallest that holds them; every row's tokens end up in the first engine's
    ``generated``, equal to a run without compaction, blocks are still
    reserved one chunk ahead and all freed, and every engine used has its
    hand-overs checked."""
    from grpo_mi355x.core.kv_pool import PagedKVPool
    from grpo_mi355x.rollout.decode import DecodeEngine

    limits = [3, 40, 9, 17, 2, 33, 5, 21]

    class Stand:
        _take_rows = DecodeEngine._take_rows
        _put_back = DecodeEngine._put_back
        _masks = DecodeEngine._masks

        def __init__(self, pool, B):
            self.pool, self.B, self.max_blocks, self.device = pool, B, 16, torch.device("cpu")
            i32 = dict(dtype=torch.int32)
            self.tokens = torch.zeros(B, dtype=torch.int64)
            self.pos, self.count, self.limit = (torch.zeros(B, **i32) for _ in range(3))
            self.append_pos, self.attn_len = torch.zeros(B, **i32), torch.zeros(B, **i32)
            self.active = torch.zeros(B, dtype=torch.bool)
            self.eos = torch.full((1,), -1, dtype=torch.int64)
            self.pad = torch.full((1,), 7, dtype=torch.int64)
            self.block_tables = torch.full((B, 16), -1, **i32)
            self.generated, self.graph = None, None
            self.steps_run = self.verified = 0

        def _ready_for(self, width):
            if self.generated is None:
                self.generated = torch.full((self.B, width), 7, dtype=torch.int64)
            self.graph = True

        def verify_handover(self):
            self.verified += 1

        def run(self, n):
            for _ in range(n):
                self.step()

        def step(self):
            self.steps_run += 1
            for b in range(self.B):
                if not self.active[b]:
                    continue
                blk = int(self.block_tables[b, int(self.pos[b]) // 4])
                assert blk >= 0 and self.pool.refcount[blk] == 1
                nxt = (int(self.tokens[b]) * 31 + int(self.pos[b])) % 1000
                self.generated[b, int(self.count[b])] = nxt
                self.tokens[b] = nxt
                self.pos[b] += 1
                self.count[b] += 1
                if int(self.count[b]) >= int(self.limit[b]):
                    self.active[b] = False
            self._masks()

    def run(compact):
        pool = PagedKVPool(1, 256, 1, 8, block_size=4)
        parent = pool.allocate(6)
        pool.set_length(parent, 6)
        sids = pool.fork(parent, 8, reserve_tokens=7)
        pool.free(parent)
        big = Stand(pool, 8)
        big._ready_for(48)
        big.tokens.copy_(torch.arange(8) + 5)
        big.pos.fill_(6)
        big.limit.copy_(torch.tensor(limits))
        big.active.copy_(big.limit > 0)
        big.block_tables.copy_(pool.block_table(sids, 16))
        big._masks()
        ladder = [Stand(pool, 4), Stand(pool, 2)] if compact else None
        stats = DecodeEngine.run_paged(big, sids, 48, check_invariants=True, compact=ladder)
        assert pool.num_free == pool.num_blocks and not pool.blocks
        return big, stats, ladder

    ref, st0, _ = run(False)
    big, st1, ladder = run(True)
    assert torch.equal(big.generated, ref.generated)
    assert [int((ref.generated[b] != 7).sum()) for b in range(8)] == limits
    assert st0["engines"] == [8] and st1["engines"] == [8, 4, 2]
    assert st1["steps"] == st0["steps"] == 40
    # 4 rows left after 12 steps, 2 after 24: the 2-row engine ran the last 16
    assert (big.steps_run, ladder[0].steps_run, ladder[1].steps_run) == (12, 12, 16)
    assert big.verified == 1 and all(e.verified == 1 for e in ladder)
    # the engines rows moved away from are left idle
    assert not bool(big.active.any()) and not bool(ladder[0].active.any())
    # engines over another pool, or a sampling engine, are refused
    other = Stand(PagedKVPool(1, 16, 1, 8, block_size=4), 4)
    with pytest.raises(ValueError, match="compaction engines"):
        DecodeEngine.run_paged(big, [], 8, compact=[other])
    big.sampling = True
    with pytest.raises(ValueError, match="greedy"):
        DecodeEngine.run_paged(big, [], 8, compact=ladder)


def test_torch_advance_stays_inside_the_generated_buffer():
    """The torch-side step bookkeeping (used with sampling and the unfused
    lm_head) records an active row's token at column count[b] and nothing once
    count reaches the buffer width, as the HIP advance does: replaying the step
    past the width (as a timing loop does) writes no column out of range."""
    import types

    from grpo_mi355x.rollout.decode import DecodeEngine

    B, W = 3, 4
    e = types.SimpleNamespace(
        B=B, generated=torch.full((B, W), 7, dtype=torch.int64),
        count=torch.tensor([0, 2, 0], dtype=torch.int32),
        pos=torch.tensor([10, 20, 30], dtype=torch.int32),
        limit=torch.tensor([100, 100, 1], dtype=torch.int32),
        active=torch.tensor([True, True, False]), eos=torch.tensor([-1]),
        tokens=torch.zeros(B, dtype=torch.int64), pad=torch.tensor([7]),
        append_pos=torch.zeros(B, dtype=torch.int32), attn_len=torch.zeros(B, dtype=torch.int32))
    e._masks = lambda: DecodeEngine._masks(e)
    for step in range(10):
        DecodeEngine._advance(e, torch.tensor([100 + step, 200 + step, 300 + step]))
    assert e.generated.tolist() == [[100, 101, 102, 103], [7, 7, 200, 201], [7, 7, 7, 7]]
    assert e.count.tolist() == [10, 12, 0] and e.pos.tolist() == [20, 30, 30]
    assert e.active.tolist() == [True, True, False]
    assert e.append_pos.tolist() == [20, 30, -1] and e.attn_len.tolist() == [21, 31, 0]


def test_fork_into_a_nearly_full_pool_changes_nothing():
    pool = PagedKVPool(1, 12, 1, 4, block_size=4)
    p = pool.allocate(10)
    pool.set_length(p, 10)          # 2 full blocks + a partial one: 9 blocks free
    refs = list(pool.refcount)
    free = pool.num_free
    # 3 children x (1 private tail + 2 blocks of growth to 20 tokens) = 9: fits
    kids = pool.fork(p, 3, reserve_tokens=20)
    pool.check_invariants()
    for c in kids:
        pool.free(c)
    assert pool.refcount == refs and pool.num_free == free
    # 4 children need 12 > 9 free blocks: refused before any state changes
    with pytest.raises(RuntimeError, match="out of memory"):
        pool.fork(p, 4, reserve_tokens=20)
    assert pool.refcount == refs and pool.num_free == free
    assert set(pool.blocks) == {p}
    pool.check_invariants()


def test_verify_handover_raises_and_switches_the_hand_overs_off():
    """DecodeEngine.verify_handover: a set XCD check word, or a hand-over
    counter left non-zero, raises RuntimeError and turns the in-kernel
    hand-overs (attention merge, o_proj finish, the screened lm_head's exact
    pass) off for engines built later; clear words and counters pass."""
    from types import SimpleNamespace

    from grpo_mi355x.rollout.decode import DecodeEngine

    saved = (DecodeEngine.ATTN_MERGE, DecodeEngine.O_FIN, DecodeEngine.LM_SCREEN)

    def stand(err=0, mcnt=None, ocnt=None, o_fin=False, lmcnt=None):
        ws = None
        if lmcnt is not None:  # the screened lm_head's workspace: counters in its first 1 KiB
            ws = torch.zeros(4096, dtype=torch.uint8)
            ws[:1024].view(torch.int32)[: len(lmcnt)] = torch.tensor(lmcnt, dtype=torch.int32)
        return SimpleNamespace(
            xcd_err=torch.tensor([err], dtype=torch.int32),
            m_cnt=None if mcnt is None else torch.tensor(mcnt, dtype=torch.int32),
            o_cnt=None if ocnt is None else torch.tensor(ocnt, dtype=torch.int32), o_fin=o_fin,
            ws_scr=ws)

    def on():
        DecodeEngine.ATTN_MERGE, DecodeEngine.O_FIN, DecodeEngine.LM_SCREEN = True, True, True

    try:
        on()
        DecodeEngine.verify_handover(stand(mcnt=[0] * 64, ocnt=[0] * 32, o_fin=True,
                                           lmcnt=[0] * 256))
        assert DecodeEngine.ATTN_MERGE and DecodeEngine.O_FIN and DecodeEngine.LM_SCREEN
        # o_proj finish counters are ignored when that path is not in use
        DecodeEngine.verify_handover(stand(ocnt=[5], o_fin=False))
        assert DecodeEngine.ATTN_MERGE and DecodeEngine.O_FIN and DecodeEngine.LM_SCREEN
        for bad in (stand(err=1), stand(mcnt=[0, 0, 0x100, 0]), stand(ocnt=[0, 3], o_fin=True),
                    stand(lmcnt=[0] * 32 + [0x20])):
            on()
            with pytest.raises(RuntimeError, match="XCD"):
                DecodeEngine.verify_handover(bad)
            assert not (DecodeEngine.ATTN_MERGE or DecodeEngine.O_FIN or DecodeEngine.LM_SCREEN)
    finally:
        DecodeEngine.ATTN_MERGE, DecodeEngine.O_FIN, DecodeEngine.LM_SCREEN = saved


def test_attention_handover_check_raises_and_switches_the_one_launch_form_off():
    """ops.attention_handover_check: clear counters and word pass; a set XCD
    word or a counter left non-zero raises RuntimeError, clears the state and
    turns the one-launch attention off for later calls (the split + merge
    launches, which hand nothing over)."""
    from grpo_mi355x.kernels import ops

    saved = (dict(ops._attn_merge), ops.ATTN_ONE_LAUNCH)
    dev = torch.device("cpu")
    try:
        ops._attn_merge.clear()
        ops.ATTN_ONE_LAUNCH = True
        ops._attn_merge[dev] = (torch.zeros(64, dtype=torch.int32),
                                torch.zeros(1, dtype=torch.int32))
        ops.attention_handover_check(dev)
        ops.attention_handover_check()  # every device
        assert ops.ATTN_ONE_LAUNCH
        for cnt, err in (([0] * 63 + [0x10], 0), ([0] * 64, 1)):
            ops.ATTN_ONE_LAUNCH = True
            ops._attn_merge[dev] = (torch.tensor(cnt, dtype=torch.int32),
                                    torch.tensor([err], dtype=torch.int32))
            with pytest.raises(RuntimeError, match="XCD"):
                ops.attention_handover_check(dev)
            assert not ops.ATTN_ONE_LAUNCH
            c, e = ops._attn_merge[dev]
            assert not bool((c != 0).any()) and int(e.item()) == 0
    finally:
        ops._attn_merge.clear()
        ops._attn_merge.update(saved[0])
        ops.ATTN_ONE_LAUNCH = saved[1]


def test_live_width_covers_every_context_of_a_graph_replay():
    """run() picks, for each 16-step graph replay, an attention plan width
    (blocks) that covers every context its steps can reach -- the bound on the
    rows' positions plus 16 tokens -- rounded up to an eighth of the table;
    single steps run the table-width graph; without context splits, with
    more split workgroups than CUs, or with LIVE_WIDTH off the table width is
    kept."""
    from grpo_mi355x.rollout.decode import DecodeEngine

    class Pool:
        block_size = 16

    class Stand:
        LIVE_WIDTH = True
        MULTI_STEP = 16
        _live_width = DecodeEngine._live_width

        def __init__(self, full, splits=8, rows=8):
            self.max_blocks, self.attn_splits, self.attn_fused = full, splits, True
            self.B, self.Hkv = rows, 2
            self.pool, self.graph, self.replayed, self.singles = Pool(), True, [], 0
            self._pos_hi = None

        def _multi_graph(self, pw=None):
            outer = self

            class G:
                def replay(self):
                    outer.replayed.append(pw)
            return G()

        def step(self):
            self.singles += 1

    s = Stand(64)
    assert [s._live_width(c) for c in (1, 128, 129, 512, 513, 1024)] == [8, 8, 16, 32, 40, 64]
    s._pos_hi = 511  # contexts 512 .. 527 in the first replay
    DecodeEngine.run(s, 16 * 9 + 5)
    assert s.replayed == [40] * 8 + [48] and s.singles == 5
    assert s._pos_hi == 511 + 16 * 9 + 5
    # the widths cover the contexts: a replay from position bound P reaches P + 16
    for k, pw in enumerate(s.replayed):
        assert pw * 16 >= 511 + 16 * k + 16
    big = Stand(256)  # unit 32 blocks
    assert [big._live_width(c) for c in (600, 2048, 4096, 5000)] == [64, 128, 256, 256]
    assert Stand(64, splits=1)._live_width(100) == 64
    # 32 rows x 2 KV heads x 8 splits would be two rounds of workgroups
    assert Stand(64, rows=16)._live_width(100) == 8 and Stand(64, rows=32)._live_width(100) == 64
    off = Stand(64)
    off.LIVE_WIDTH = False
    assert off._live_width(100) == 64
    none = Stand(64)  # no position bound (start not called): the table width
    DecodeEngine.run(none, 32)
    assert none.replayed == [None, None]
