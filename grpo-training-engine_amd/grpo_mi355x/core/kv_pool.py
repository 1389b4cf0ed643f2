"""Paged KV block pool: per-layer caches, block allocator, prefix sharing.

The reference has no KV manager (``src/core/memory_manager.py`` only does VRAM
housekeeping); its model-level decode allocates one cache per call and gives
every batch row the same ``arange`` block table (``paged_kv.py:626-645``), so
G samples of one prompt write the same slots once their tokens diverge.  This
pool gives each sequence its own block table:

* a sequence owns a list of physical blocks; ``reserve`` grows it;
* ``fork`` makes G children of a prefilled prompt: FULL prompt blocks are
  shared (reference-counted, read-only), the partially filled last block is
  copied per child (copy-on-write at fork), so no two live sequences can
  write one block;
* ``free`` drops a finished sequence's references; blocks whose count reaches
  zero return to the free list ("blocks allocated and freed
  as sequences finish");
* ``check_invariants`` verifies reference counts, the free list and that every
  block a sequence may still write is exclusively owned.

Storage: ``k``/``v`` are bf16 ``[num_layers, num_blocks, Hkv, block_size, D]``;
``k[layer]`` is the contiguous ``[num_blocks, Hkv, block_size, D]`` cache the
kernels take.
"""

from __future__ import annotations

from collections import deque

import torch


class PagedKVPool:
    def __init__(self, num_layers: int, num_blocks: int, num_kv_heads: int, head_dim: int,
                 block_size: int = 16, device=None, dtype: torch.dtype = torch.bfloat16):
        if num_blocks <= 0 or block_size <= 0:
            raise ValueError("num_blocks and block_size must be positive.")
        self.num_layers = num_layers
        self.num_blocks = num_blocks
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.block_size = block_size
        shape = (num_layers, num_blocks, num_kv_heads, block_size, head_dim)
        self.k = torch.zeros(shape, dtype=dtype, device=device)
        self.v = torch.zeros(shape, dtype=dtype, device=device)
        self.refcount = [0] * num_blocks
        self._free: deque[int] = deque(range(num_blocks))
        self.blocks: dict[int, list[int]] = {}
        self.length: dict[int, int] = {}
        self._next_id = 0

    # ------------------------------------------------------------ queries --
    @property
    def num_free(self) -> int:
        return len(self._free)

    def blocks_for(self, n_tokens: int) -> int:
        return -(-n_tokens // self.block_size)

    def layer(self, i: int) -> tuple[torch.Tensor, torch.Tensor]:
        return self.k[i], self.v[i]

    # ---------------------------------------------------------- allocation --
    def _take(self) -> int:
        if not self._free:
            raise RuntimeError("out of memory: paged KV pool has no free blocks")
        b = self._free.popleft()
        self.refcount[b] = 1
        return b

    def allocate(self, n_tokens: int = 0) -> int:
        """New sequence with room for ``n_tokens`` tokens (length 0)."""
        sid = self._next_id
        self._next_id += 1
        self.blocks[sid] = []
        self.length[sid] = 0
        self.reserve(sid, n_tokens)
        return sid

    def reserve(self, sid: int, n_tokens: int) -> None:
        """Make sure sequence ``sid`` has blocks for ``n_tokens`` positions."""
        need = self.blocks_for(n_tokens) - len(self.blocks[sid])
        if need > len(self._free):
            raise RuntimeError(f"out of memory: need {need} blocks, {len(self._free)} free")
        for _ in range(max(need, 0)):
            self.blocks[sid].append(self._take())

    def set_length(self, sid: int, n_tokens: int) -> None:
        if self.blocks_for(n_tokens) > len(self.blocks[sid]):
            raise ValueError("length exceeds the reserved blocks")
        self.length[sid] = n_tokens

    def fork(self, sid: int, n: int, reserve_tokens: int | None = None) -> list[int]:
        """``n`` children sharing ``sid``'s first ``length`` tokens.

        Full blocks are shared; the partial last block (if any) is copied into a
        private block of each child in every layer.  Children get room for
        ``reserve_tokens`` tokens (default: the parent's length).

        All-or-nothing: the free blocks the children need (the private tail
        plus the reservation's growth, per child) are counted first, and an
        out-of-memory ``RuntimeError`` leaves the pool unchanged.
        """
        length = self.length[sid]
        full = length // self.block_size
        partial = length % self.block_size != 0
        parent = self.blocks[sid]
        own = full + int(partial)
        per_child = int(partial) + max(
            0, (self.blocks_for(reserve_tokens) if reserve_tokens is not None else 0) - own)
        if n * per_child > len(self._free):
            raise RuntimeError(f"out of memory: fork of {n} needs {n * per_child} blocks, "
                               f"{len(self._free)} free")
        children = []
        for _ in range(n):
            cid = self._next_id
            self._next_id += 1
            blocks = list(parent[:full])
            for b in blocks:
                self.refcount[b] += 1
            if partial:
                nb = self._take()
                src = parent[full]
                self.k[:, nb].copy_(self.k[:, src])
                self.v[:, nb].copy_(self.v[:, src])
                blocks.append(nb)
            self.blocks[cid] = blocks
            self.length[cid] = length
            if reserve_tokens is not None:
                self.reserve(cid, reserve_tokens)
            children.append(cid)
        return children

    def free(self, sid: int) -> None:
        """Release a sequence; unreferenced blocks return to the free list."""
        for b in self.blocks.pop(sid):
            self.refcount[b] -= 1
            if self.refcount[b] == 0:
                self._free.append(b)
        self.length.pop(sid)

    # ---------------------------------------------------------- tables ----
    def block_table(self, sids: list[int], width: int | None = None,
                    device=None) -> torch.Tensor:
        """int32 ``[len(sids), width]`` block table; unused entries are -1 (invalid)."""
        width = width or max((len(self.blocks[s]) for s in sids), default=1)
        rows = []
        for s in sids:
            bl = self.blocks[s]
            if len(bl) > width:
                raise ValueError("block table narrower than a sequence")
            rows.append(bl + [-1] * (width - len(bl)))
        t = torch.tensor(rows, dtype=torch.int32)
        return t.to(device if device is not None else self.k.device)

    # -------------------------------------------------------- invariants --
    def check_invariants(self) -> None:
        counts = [0] * self.num_blocks
        for bl in self.blocks.values():
            for b in bl:
                counts[b] += 1
        if counts != self.refcount:
            raise AssertionError("reference counts do not match the block lists")
        free = set(self._free)
        if len(free) != len(self._free):
            raise AssertionError("a block is on the free list twice")
        for b in range(self.num_blocks):
            if (b in free) != (counts[b] == 0):
                raise AssertionError(f"block {b}: free-list membership disagrees with its count")
        for sid, bl in self.blocks.items():
            first_writable = self.length[sid] // self.block_size
            for b in bl[first_writable:]:
                if self.refcount[b] != 1:
                    raise AssertionError(f"sequence {sid} may write shared block {b}")
