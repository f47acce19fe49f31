"""Host-side paged KV cache for the MI355X kernels.

Same public interface, layout and bookkeeping as the reference's
``PagedKVCache`` (superl8serve/engine/kv_cache.py:432-1299) so a caller can
switch to it unchanged:

* storage (kv_cache.py:484-512): int8 ``k_cache`` / ``v_cache``
  ``[L, N, Hkv, bs, D]``, fp32 ``k_scale`` / ``v_scale`` ``[L, N, Hkv, bs]``; or, for
  ``v_quant="lloydmax3"``, ``v_packed`` int32 ``[L, N, Hkv, bs, 3D/32]``,
  ``v_norm`` fp32 ``[L, N, Hkv, bs, D/128]`` and a per-layer ``v_codebook``;
* slots and blocks (kv_cache.py:703-755): LIFO free lists of slots and physical
  blocks, blocks pulled one at a time as a slot grows, reference counts so that
  blocks shared through the prefix cache are freed by their last holder;
* prefix cache (kv_cache.py:757-898): a token trie with entries at every
  block-aligned boundary, a global access counter for LRU, eviction of the
  least recently used entry on an entry-count cap, and a budget on the number of
  distinct blocks the cache pins (default half the pool);
* slot mappings, block tables and pinned staging for graph replays
  (kv_cache.py:900-995, 1118-1127);
* writes and attention through the gfx950 kernels (``ops``): append (int8 and
  fused K8V3), batched paged decode, and multi-query verify.

Beyond the reference: copy-on-write of a shared last block and compaction of
the pool (moving live blocks into free holes) through the block-copy kernel.
"""

from __future__ import annotations

import numpy as np
import torch

from . import ops
from .codebook import gaussian_codebook


def _unpack3(words: torch.Tensor, d: int) -> torch.Tensor:
    """Bit-plane words ``[..., 3d/32]`` -> 3-bit codes ``[..., d]`` (word 3g+b
    holds bit b of codes 32g..32g+31, element 32g+i at bit i)."""
    w = words.reshape(*words.shape[:-1], d // 32, 3).to(torch.int64) & 0xFFFFFFFF
    bit = torch.arange(32, device=words.device)
    planes = (w.unsqueeze(-1) >> bit) & 1  # [..., g, 3, 32]
    codes = planes[..., 0, :] | (planes[..., 1, :] << 1) | (planes[..., 2, :] << 2)
    return codes.reshape(*words.shape[:-1], d)


def block_bytes(num_kv_heads: int, block_size: int, head_dim: int, v_quant: str = "int8",
                lloyd_block: int = 128) -> int:
    """HBM bytes of one block in one layer (kv_cache.py:98-120)."""
    tokens = num_kv_heads * block_size
    k_side = tokens * (head_dim + 4)
    if v_quant == "lloydmax3":
        return k_side + tokens * (head_dim * 3 // 32 * 4 + head_dim // lloyd_block * 4)
    return k_side + tokens * (head_dim + 4)


class _Staging:
    """Pinned host mirrors of device buffers that captured graphs read.  A
    refresh writes the host mirror and issues one non-blocking copy; an event
    recorded after the copy is waited on before the mirror is written again,
    so a pending copy never reads a half-written mirror."""

    def __init__(self, pin: bool):
        self._pin = pin
        self._host: dict[str, torch.Tensor] = {}
        self._done: dict[str, torch.cuda.Event] = {}

    def put(self, dst: torch.Tensor, values: np.ndarray, name: str) -> None:
        n = values.size
        buf = self._host.get(name)
        if buf is None or buf.numel() < n or buf.dtype != dst.dtype:
            buf = torch.empty(max(n, 1), dtype=dst.dtype, pin_memory=self._pin)
            self._host[name] = buf
            self._done.pop(name, None)
        ev = self._done.get(name)
        if ev is not None:
            ev.synchronize()
        host = buf[:n].view(values.shape)
        host.numpy()[...] = values
        dst.copy_(host, non_blocking=self._pin)
        if self._pin and dst.is_cuda:
            ev = torch.cuda.Event()
            ev.record()
            self._done[name] = ev


class _Entry:
    __slots__ = ("blocks", "num_tokens", "lru")

    def __init__(self, blocks: list[int], num_tokens: int, lru: int):
        self.blocks = blocks
        self.num_tokens = num_tokens
        self.lru = lru


class _Node:
    __slots__ = ("children", "entry")

    def __init__(self):
        self.children: dict[int, _Node] = {}
        self.entry: _Entry | None = None


class PagedKVCache:
    def __init__(self, num_layers, num_slots, num_kv_heads, max_len, head_dim, *, device, block_size: int = 16,
                 num_blocks: int | None = None, max_prefix_entries: int | None = None,
                 max_prefix_blocks: int | None = None, max_prefix_block_fraction: float = 0.5,
                 kv_layers: list[int] | None = None, v_quant: str = "int8", lloyd_block: int = 128):
        if v_quant not in ("int8", "lloydmax3"):
            raise ValueError(f"v_quant must be 'int8' or 'lloydmax3', got {v_quant!r}")
        self.block_size = block_size
        self._row_of_layer = None if kv_layers is None else {l: i for i, l in enumerate(kv_layers)}
        self.num_layers = num_layers if kv_layers is None else len(kv_layers)
        self.v_quant = v_quant
        self.lloyd_block = lloyd_block
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.max_len = max_len
        self.max_blocks_per_seq = -(-max_len // block_size)
        self.num_blocks = num_blocks or num_slots * self.max_blocks_per_seq
        self.num_slots = num_slots
        self.device = device
        geom = (self.num_layers, self.num_blocks, num_kv_heads, block_size)
        self.k_cache = torch.zeros(geom + (head_dim,), dtype=torch.int8, device=device)
        self.k_scale = torch.ones(geom, dtype=torch.float32, device=device)
        if v_quant == "lloydmax3":
            self.v_packed = torch.zeros(geom + (head_dim * 3 // 32,), dtype=torch.int32, device=device)
            self.v_norm = torch.zeros(geom + (head_dim // lloyd_block,), dtype=torch.float32, device=device)
            cb = torch.from_numpy(gaussian_codebook(3, lloyd_block)).to(device)
            self.v_codebook = cb.unsqueeze(0).repeat(self.num_layers, 1)
            self.v_cache = None
            self.v_scale = None
        else:
            self.v_cache = torch.zeros(geom + (head_dim,), dtype=torch.int8, device=device)
            self.v_scale = torch.ones(geom, dtype=torch.float32, device=device)
            self.v_packed = self.v_norm = self.v_codebook = None
        # LIFO pools: the next block / slot handed out is the last one returned
        self._free_blocks: list[int] = list(range(self.num_blocks))
        self._free_slots: list[int] = list(range(num_slots))
        self._slot_blocks: list[list[int]] = [[] for _ in range(num_slots)]
        self._block_refcount: dict[int, int] = {}
        # prefix cache
        self._trie = _Node()
        self._lru_clock = 0
        self._max_prefix_entries = max_prefix_entries
        self._prefix_entry_count = 0
        # distinct blocks the prefix cache may pin: explicit, else a fraction of
        # the pool (at least one), else unbounded
        budget = max_prefix_blocks
        if budget is None and max_prefix_block_fraction is not None:
            budget = max(1, int(self.num_blocks * max_prefix_block_fraction))
        self._max_prefix_blocks: int | None = budget
        self._prefix_block_refs: dict[int, int] = {}
        # graph inputs: pinned host mirrors of the device buffers a captured
        # graph reads (decode slot mapping / block table, prefill statics)
        self._pin = device != "cpu" and torch.cuda.is_available()
        self._staging = _Staging(self._pin)
        self._prefill_mapping_static: torch.Tensor | None = None
        self._prefill_positions_static: torch.Tensor | None = None
        self._prefill_blocks_static: torch.Tensor | None = None
        self._graph_prefill_mode = False

    # ------------------------------------------------------------------ layout

    def _layer_row(self, layer: int) -> int:
        if self._row_of_layer is None:
            return layer
        if layer not in self._row_of_layer:
            raise KeyError(f"layer {layer} bears no KV cache")
        return self._row_of_layer[layer]

    def _tensors(self) -> list[torch.Tensor]:
        if self.v_quant == "lloydmax3":
            return [self.k_cache, self.k_scale, self.v_packed, self.v_norm]
        return [self.k_cache, self.k_scale, self.v_cache, self.v_scale]

    # ------------------------------------------------------- slots and blocks

    def alloc(self) -> int:
        if not self._free_slots:
            raise RuntimeError("PagedKVCache: no free slots")
        return self._free_slots.pop()

    def _release_block(self, blk: int) -> None:
        left = self._block_refcount.get(blk, 1) - 1
        if left > 0:
            self._block_refcount[blk] = left
        else:
            self._block_refcount.pop(blk, None)
            self._free_blocks.append(blk)

    def free(self, slot: int) -> None:
        for blk in self._slot_blocks[slot]:
            self._release_block(blk)
        self._slot_blocks[slot] = []
        self._free_slots.append(slot)

    def has_free_slot(self) -> bool:
        return len(self._free_slots) > 0

    def has_free_block(self) -> bool:
        return len(self._free_blocks) > 0

    @property
    def used_blocks(self) -> int:
        return self.num_blocks - len(self._free_blocks)

    def ensure_capacity(self, slots: list[int], lengths: list[int]) -> None:
        for slot, n in zip(slots, lengths):
            owned = self._slot_blocks[slot]
            want = -(-n // self.block_size)
            while len(owned) < want:
                if not self._free_blocks:
                    raise RuntimeError("PagedKVCache: no free blocks")
                blk = self._free_blocks.pop()
                owned.append(blk)
                self._block_refcount[blk] = 1

    def share_blocks(self, slot: int, blocks: list[int]) -> None:
        self._slot_blocks[slot] = list(blocks)
        for blk in blocks:
            self._block_refcount[blk] = self._block_refcount.get(blk, 1) + 1

    # ----------------------------------------------------------- prefix cache

    def _tick_lru(self) -> int:
        self._lru_clock += 1
        return self._lru_clock

    def _oldest_entry(self):
        """(parent, token, node) of the least recently used entry, in trie
        pre-order (first found wins ties), or None."""
        best = None
        stack = [(self._trie, iter(self._trie.children.items()))]
        while stack:
            parent, it = stack[-1]
            nxt = next(it, None)
            if nxt is None:
                stack.pop()
                continue
            tok, node = nxt
            if node.entry is not None and (best is None or node.entry.lru < best[2].entry.lru):
                best = (parent, tok, node)
            stack.append((node, iter(node.children.items())))
        return best

    def _evict_one_prefix(self) -> bool:
        found = self._oldest_entry()
        if found is None:
            return False
        parent, tok, node = found
        entry, node.entry = node.entry, None
        for blk in entry.blocks:
            pins = self._prefix_block_refs.get(blk, 0) - 1
            if pins > 0:
                self._prefix_block_refs[blk] = pins
            else:
                self._prefix_block_refs.pop(blk, None)
            self._release_block(blk)
        self._prefix_entry_count -= 1
        if not node.children:
            del parent.children[tok]
        return True

    def _enforce_prefix_budget(self) -> None:
        if self._max_prefix_blocks is None:
            return
        while len(self._prefix_block_refs) > self._max_prefix_blocks and self._evict_one_prefix():
            pass

    @property
    def pinned_prefix_blocks(self) -> int:
        return len(self._prefix_block_refs)

    def prefix_block_bytes(self) -> int:
        return (len(self._prefix_block_refs) * self.num_layers
                * block_bytes(self.num_kv_heads, self.block_size, self.head_dim, self.v_quant, self.lloyd_block))

    def store_prefix(self, token_ids: list[int], slot: int) -> None:
        bs = self.block_size
        whole = len(token_ids) // bs
        if whole == 0:
            return
        owned = list(self._slot_blocks[slot])
        now = self._tick_lru()
        node = self._trie
        for i, tok in enumerate(token_ids):
            node = node.children.setdefault(tok, _Node())
            n = i + 1
            if n % bs or n // bs > whole:
                continue
            if node.entry is not None:
                node.entry.lru = now
                continue
            if self._max_prefix_entries is not None and self._prefix_entry_count >= self._max_prefix_entries:
                self._evict_one_prefix()
            blocks = owned[: n // bs]
            node.entry = _Entry(blocks, n, now)
            for blk in blocks:
                self._block_refcount[blk] = self._block_refcount.get(blk, 1) + 1
                self._prefix_block_refs[blk] = self._prefix_block_refs.get(blk, 0) + 1
            self._prefix_entry_count += 1
        self._enforce_prefix_budget()

    def lookup_prefix(self, token_ids: list[int]) -> tuple[int, list[int]]:
        now = self._tick_lru()
        node = self._trie
        length, blocks = 0, []
        for i, tok in enumerate(token_ids):
            node = node.children.get(tok)
            if node is None:
                break
            e = node.entry
            if e is not None and i + 1 >= e.num_tokens:
                length, blocks = e.num_tokens, list(e.blocks)
                e.lru = now
        return length, blocks

    # --------------------------------------------- mappings and block tables

    def flat_slot_mapping(self, slot: int, length: int) -> list[int]:
        bs = self.block_size
        owned = self._slot_blocks[slot]
        return [owned[p // bs] * bs + p % bs for p in range(length)]

    def slot_mapping_for(self, slots: list[int], positions: list[int]) -> torch.Tensor:
        """int32 device tensor of the flat slots of (slot, position) pairs
        (kv_cache.py:900-905, 960-961)."""
        return torch.from_numpy(self._flat_slots(slots, positions)).to(self.device)

    _slot_mapping = slot_mapping_for

    def block_table(self, slots: list[int]) -> torch.Tensor:
        """``[B, max_blocks_per_seq]`` int32 block ids, zero padded
        (kv_cache.py:1118-1127)."""
        return torch.from_numpy(self._table_rows(slots, self.max_blocks_per_seq)).to(self.device)

    def _flat_slots(self, slots: list[int], positions: list[int]) -> np.ndarray:
        """int32 flat slots ``block * bs + pos % bs`` of (slot, position) pairs."""
        bs = self.block_size
        blk = np.fromiter((self._slot_blocks[s][p // bs] for s, p in zip(slots, positions)), np.int64,
                          count=len(slots))
        pos = np.asarray(positions, dtype=np.int64)
        return (blk * bs + pos % bs).astype(np.int32)

    def _table_rows(self, slots: list[int], width: int) -> np.ndarray:
        """Zero-padded int32 ``[len(slots), width]`` block ids."""
        table = np.zeros((len(slots), width), dtype=np.int32)
        for i, s in enumerate(slots):
            owned = self._slot_blocks[s]
            table[i, : len(owned)] = owned
        return table

    def fill_slot_mapping(self, dst: torch.Tensor, slots: list[int], positions: list[int]) -> None:
        """Refresh a graph's slot-mapping buffer in place: the values go through
        a pinned host mirror and one non-blocking copy (the role of
        kv_cache.py:971-980)."""
        self._staging.put(dst, self._flat_slots(slots, positions), "slot_mapping")

    def fill_block_table(self, dst: torch.Tensor, slots: list[int]) -> None:
        """Refresh a graph's block-table buffer in place; short rows are zero
        padded (the role of kv_cache.py:982-995)."""
        self._staging.put(dst, self._table_rows(slots, dst.shape[1]), "block_table")

    def enable_graph_prefill(self, max_len: int) -> None:
        """Allocate the device buffers a graph-captured ``write_prefill`` reads
        (kv_cache.py:918-932): the flat slots of ``max_len`` positions and a
        block-id table indexed by ``position // block_size`` (one entry per
        pool block, so no position of a slot can index past it)."""
        self._prefill_mapping_static = torch.zeros(max_len, dtype=torch.int32, device=self.device)
        self._prefill_blocks_static = torch.zeros(self.num_blocks, dtype=torch.int64, device=self.device)
        self._graph_prefill_mode = True

    def bind_graph_write_prefill(self, slot: int, length: int) -> None:
        """Point the graph-prefill buffers at `slot` (kv_cache.py:934-956): its
        first `length` flat slots and its block ids, written in place so a
        captured ``write_prefill`` replays against them.  No-op before
        ``enable_graph_prefill``.

        CHOICE: the mapping entries past `length` become -1, which the append
        skips, so the padding tokens of a prompt shorter than the captured
        bucket write nothing.  The reference rewrites only the first `length`
        entries, leaving the previous binding's slots there (the scratch
        slot's after capture, a previous prompt's slots after a longer one)."""
        if self._prefill_mapping_static is None:
            return
        n = int(length)
        cap = self._prefill_mapping_static.numel()
        if n > cap:
            raise ValueError(f"bind_graph_write_prefill: {n} positions exceed the {cap} enable_graph_prefill allocated")
        mapping = np.full(cap, -1, dtype=np.int32)
        mapping[:n] = self._flat_slots([slot] * n, list(range(n)))
        self._staging.put(self._prefill_mapping_static, mapping, "prefill_mapping")
        owned = self._slot_blocks[slot]
        if owned:
            self._staging.put(self._prefill_blocks_static[: len(owned)], np.asarray(owned, dtype=np.int64),
                              "prefill_blocks")

    # ------------------------------------------------------------------ writes

    def write_prefill_varlen(self, layer: int, slot_mapping: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
        """k, v: fp16 ``[T, Hkv, D]``; one append of every token at its flat slot."""
        row = self._layer_row(layer)
        if self.v_quant == "lloydmax3":
            ops.quantize_kv_write_paged_k8v3(k.contiguous(), v.contiguous(), self.k_cache[row], self.k_scale[row],
                                             self.v_packed[row], self.v_norm[row], self.v_codebook[row],
                                             slot_mapping, self.lloyd_block)
        else:
            ops.quantize_kv_write_paged(k.contiguous(), v.contiguous(), self.k_cache[row], self.k_scale[row],
                                        self.v_cache[row], self.v_scale[row], slot_mapping)

    def write_prefill(self, layer: int, k: torch.Tensor, v: torch.Tensor, *, slot: int, start: int = 0,
                      positions: torch.Tensor | None = None) -> None:
        """k, v: fp16 ``[1, Hkv, S, D]``.  Positions ``[0, S)`` (or `positions`),
        skipping those below `start` (shared-prefix reuse)."""
        s = k.shape[2]
        if s == 0:
            return
        kt = k[0].transpose(0, 1)
        vt = v[0].transpose(0, 1)
        graph = self._graph_prefill_mode
        if positions is None:
            first = min(max(start, 0), s)
            if first == s:
                return
            if graph and self._prefill_mapping_static is not None:  # bound by bind_graph_write_prefill
                mapping = self._prefill_mapping_static[first:s]
            else:
                mapping = torch.from_numpy(self._flat_slots([slot] * (s - first), list(range(first, s)))).to(
                    self.device)
            kt, vt = kt[first:], vt[first:]
        else:
            pos = positions.reshape(-1).to(device=self.device, dtype=torch.int64)
            if start > 0:
                # a shared prefix: one host check that anything is left to write
                keep = pos >= start
                if not bool(keep.any()):
                    return
                pos, kt, vt = pos[keep], kt[keep], vt[keep]
            if graph and self._prefill_blocks_static is not None:
                owned = self._prefill_blocks_static
            else:
                owned = torch.from_numpy(np.asarray(self._slot_blocks[slot], dtype=np.int64)).to(self.device)
            mapping = (owned[pos // self.block_size] * self.block_size + pos % self.block_size).to(torch.int32)
        self.write_prefill_varlen(layer, mapping, kt, vt)

    def write_decode_static(self, layer: int, slot_mapping: torch.Tensor, k_new: torch.Tensor,
                            v_new: torch.Tensor) -> None:
        """k_new, v_new: fp16 ``[B, Hkv, D]``, one token per sequence."""
        self.write_prefill_varlen(layer, slot_mapping, k_new, v_new)

    def write_decode(self, layer: int, slots: list[int], positions: list[int], k_new: torch.Tensor,
                     v_new: torch.Tensor) -> None:
        self.write_decode_static(layer, self.slot_mapping_for(slots, positions), k_new, v_new)

    # --------------------------------------------------------------- attention

    def decode_attn_static(self, layer: int, q: torch.Tensor, block_table: torch.Tensor, context_lens: torch.Tensor,
                           max_context_len: int, *, scale: float, window: int | None = None) -> torch.Tensor:
        """Batched paged decode (kv_cache.py:1148-1201).  ``window``: a
        sliding-window layer attends only each row's last ``window`` tokens
        (what the reference gets from ``read_dense(..., window=)`` plus a dense
        decode per row, gqa_attention.py:191-196)."""
        row = self._layer_row(layer)
        if window is not None:
            if self.v_quant == "lloydmax3":
                return ops.attn_paged_decode_window_k8v3(
                    q, self.k_cache[row], self.k_scale[row], self.v_packed[row], self.v_norm[row],
                    self.v_codebook[row], block_table, context_lens, self.block_size,
                    max_context_len=max_context_len, window=window, scale=scale)
            return ops.attn_paged_decode_window(q, self.k_cache[row], self.k_scale[row], self.v_cache[row],
                                                self.v_scale[row], block_table, context_lens, self.block_size,
                                                max_context_len=max_context_len, window=window, scale=scale)
        if self.v_quant == "lloydmax3":
            return ops.attn_paged_decode_k8v3(q, self.k_cache[row], self.k_scale[row], self.v_packed[row],
                                              self.v_norm[row], self.v_codebook[row], block_table, context_lens,
                                              self.block_size, max_context_len=max_context_len, scale=scale)
        return ops.attn_paged_decode_cached(q, self.k_cache[row], self.k_scale[row], self.v_cache[row],
                                            self.v_scale[row], block_table, context_lens, self.block_size,
                                            max_context_len=max_context_len, scale=scale)

    def decode_attn(self, layer: int, q: torch.Tensor, slots: list[int], lengths: list[int], *,
                    scale: float, window: int | None = None) -> torch.Tensor:
        """`lengths[i]` is the position of the token just written, so row i
        attends `lengths[i] + 1` tokens (kv_cache.py:1129-1146), or the last
        ``window`` of them."""
        ctx = [n + 1 for n in lengths]
        return self.decode_attn_static(layer, q, self.block_table(slots),
                                       torch.tensor(ctx, dtype=torch.int32, device=self.device),
                                       max(ctx) if ctx else 0, scale=scale, window=window)

    def decode_step_plan(self, block_table: torch.Tensor, context_lens: torch.Tensor, max_context_len: int, *,
                         num_q_heads: int) -> torch.Tensor:
        """The slice plan one decode step's ``decode_step_static`` calls can
        share: every layer of a step reads the same ``block_table`` and
        ``context_lens`` (these tensors, with unchanged contents), so the split
        of the rows' tokens over the decode workgroups is computed once, on the
        device, instead of in every layer's launch."""
        return ops.attn_paged_decode_plan(self.k_cache[0], block_table, context_lens, self.block_size,
                                          num_q_heads=num_q_heads, max_context_len=max_context_len,
                                          layout="k8v3" if self.v_quant == "lloydmax3" else "int8")

    def decode_step_static(self, layer: int, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                           block_table: torch.Tensor, context_lens: torch.Tensor, max_context_len: int, *,
                           scale: float, plan: torch.Tensor | None = None) -> torch.Tensor:
        """``write_decode_static`` + ``decode_attn_static`` in one launch (int8
        and K8V3 layouts): row b's new token goes to position ``context_lens[b] - 1``
        of its block table (where the reference's decode step writes it,
        kv_cache.py:1083-1093 with 1129-1146), then the row attends.  Same
        cache bytes and output as the two calls.  ``plan``: the step's
        ``decode_step_plan`` (same results, the launch skips locating its work)."""
        row = self._layer_row(layer)
        if self.v_quant == "lloydmax3":
            return ops.attn_paged_decode_append_k8v3(
                q, k_new, v_new, self.k_cache[row], self.k_scale[row], self.v_packed[row], self.v_norm[row],
                self.v_codebook[row], block_table, context_lens, self.block_size, max_context_len=max_context_len,
                scale=scale, plan=plan)
        return ops.attn_paged_decode_append(q, k_new, v_new, self.k_cache[row], self.k_scale[row],
                                            self.v_cache[row], self.v_scale[row], block_table, context_lens,
                                            self.block_size, max_context_len=max_context_len, scale=scale,
                                            plan=plan)

    def decode_step(self, layer: int, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                    slots: list[int], lengths: list[int], *, scale: float) -> torch.Tensor:
        """``write_decode`` + ``decode_attn`` (write at ``lengths[i]``, attend
        ``lengths[i] + 1`` tokens) in one launch."""
        ctx = [n + 1 for n in lengths]
        return self.decode_step_static(layer, q, k_new, v_new, self.block_table(slots),
                                       torch.tensor(ctx, dtype=torch.int32, device=self.device),
                                       max(ctx) if ctx else 0, scale=scale)

    def verify_attn(self, layer: int, q: torch.Tensor, slots: list[int], prefix_lens: list[int], *, scale: float,
                    query_lens: list[int] | None = None, tree_mask: torch.Tensor | None = None,
                    window: int | None = None, k_draft: torch.Tensor | None = None,
                    v_draft: torch.Tensor | None = None) -> torch.Tensor:
        """Multi-query attention of drafts (already written at positions
        ``prefix_lens[b] ..``): chain / chunk when `tree_mask` is None, else tree.
        ``q``: fp16 ``[B, Hq, S, D]``.  A sliding-window layer (``window``)
        may pass the drafts' fresh K / V ``[B, S, Hkv, D]`` to attend them
        unquantized, as the reference's window verify does."""
        row = self._layer_row(layer)
        s = q.shape[2]
        ql = query_lens if query_lens is not None else [s] * len(slots)
        max_ctx = max((p + n for p, n in zip(prefix_lens, ql)), default=0)
        common = dict(
            query_lens=None if query_lens is None else torch.tensor(query_lens, dtype=torch.int32, device=self.device),
            tree_mask=tree_mask, max_context_len=min(max_ctx, self.max_blocks_per_seq * self.block_size),
            scale=scale, window=window, k_draft=k_draft, v_draft=v_draft)
        bt = self.block_table(slots)
        pl = torch.tensor(prefix_lens, dtype=torch.int32, device=self.device)
        if self.v_quant == "lloydmax3":
            return ops.attn_paged_verify_k8v3(
                q, self.k_cache[row], self.k_scale[row], self.v_packed[row], self.v_norm[row], self.v_codebook[row],
                bt, pl, self.block_size, **common)
        return ops.attn_paged_verify(q, self.k_cache[row], self.k_scale[row], self.v_cache[row], self.v_scale[row],
                                     bt, pl, self.block_size, **common)

    def read_dense(self, layer: int, slot: int, length: int, *, window: int | None = None,
                   dtype: torch.dtype = torch.float16) -> tuple[torch.Tensor, torch.Tensor]:
        """Dequantized fp16 K, V ``[1, Hkv, n, D]`` of one sequence (the
        reference's dense reader, kv_cache.py:1233-1299): K un-rotated."""
        row = self._layer_row(layer)
        first = max(0, length - window) if window is not None else 0
        pos = torch.arange(first, length, device=self.device)
        owned = torch.tensor(self._slot_blocks[slot], dtype=torch.int64, device=self.device)
        blk = owned[pos // self.block_size]
        off = pos % self.block_size
        kq = self.k_cache[row][blk, :, off].float() * self.k_scale[row][blk, :, off].unsqueeze(-1)
        d = self.head_dim
        # the reference's recipe, rotate_last((k_i8 * s_k).to(dtype)), with the
        # rotation on the row kernel: each row's rounding is independent of
        # how many rows are read
        k = ops.rotate_rows(kq.to(dtype))
        if self.v_quant == "lloydmax3":
            codes = _unpack3(self.v_packed[row][blk, :, off], d)
            nb = d // self.lloyd_block
            cbv = self.v_codebook[row][codes.long()].reshape(*codes.shape[:-1], nb, self.lloyd_block)
            v = (cbv * self.v_norm[row][blk, :, off].unsqueeze(-1)).reshape(codes.shape).to(dtype)
        else:
            v = (self.v_cache[row][blk, :, off].float() * self.v_scale[row][blk, :, off].unsqueeze(-1)).to(dtype)
        return k.transpose(0, 1).unsqueeze(0), v.transpose(0, 1).unsqueeze(0)

    # --------------------------------------------- copy-on-write, compaction

    def copy_on_write_last_block(self, slot: int) -> int | None:
        """Give `slot` a private copy of its last block when that block is shared
        (refcount > 1): copy it on the GPU, drop one reference, point the slot's
        table at the copy.  Returns the new block id, or None if nothing to do."""
        owned = self._slot_blocks[slot]
        if not owned or self._block_refcount.get(owned[-1], 1) <= 1:
            return None
        if not self._free_blocks:
            raise RuntimeError("PagedKVCache: no free blocks")
        old = owned[-1]
        new = self._free_blocks.pop()
        ops.copy_blocks(self._tensors(), [old], [new])
        self._block_refcount[new] = 1
        self._block_refcount[old] -= 1
        owned[-1] = new
        return new

    def evict_after_prefill(self, slot: int, seq_len: int, *, eviction_config, num_heads: int,
                            keep_mask: list[int] | None = None, q_last: torch.Tensor | None = None,
                            k_full: torch.Tensor | None = None, logits_full: torch.Tensor | None = None,
                            logits_fn=None) -> dict:
        """Prompt-time eviction of `slot` with this cache's geometry
        (kv_cache.py:1303-1336); see ``eviction.KVEviction.evict``."""
        from .eviction import KVEviction

        return KVEviction.evict(self, slot, seq_len, eviction_config=eviction_config, num_heads=num_heads,
                                num_kv_heads=self.num_kv_heads, head_dim=self.head_dim, q_last=q_last,
                                k_full=k_full, keep_mask=keep_mask, logits_full=logits_full, logits_fn=logits_fn)

    def defragment(self) -> list[tuple[int, int]]:
        """Move every live block above the free watermark into the lowest free
        holes, so the live set occupies blocks ``[0, used_blocks)``.  One GPU
        block copy for all layers and tensors, then every reference (slot
        tables, prefix entries, refcounts, pins) is rewritten.  Returns the
        ``(src, dst)`` moves.

        The live set is every block outside the free list: a block a slot
        holds need not have a refcount entry (``KVEviction.compact`` takes
        its new blocks from the pool without one, as the reference does), so
        the refcount map alone would miss it."""
        used = self.used_blocks
        free = set(self._free_blocks)
        live_high = [b for b in range(used, self.num_blocks) if b not in free]
        holes = sorted(b for b in self._free_blocks if b < used)
        moves = list(zip(live_high, holes))
        if not moves:
            return []
        ops.copy_blocks(self._tensors(), [s for s, _ in moves], [d for _, d in moves])
        remap = dict(moves)
        for owned in self._slot_blocks:
            owned[:] = [remap.get(b, b) for b in owned]
        stack = [self._trie]
        while stack:
            node = stack.pop()
            if node.entry is not None:
                node.entry.blocks = [remap.get(b, b) for b in node.entry.blocks]
            stack.extend(node.children.values())
        self._block_refcount = {remap.get(b, b): c for b, c in self._block_refcount.items()}
        self._prefix_block_refs = {remap.get(b, b): c for b, c in self._prefix_block_refs.items()}
        # the holes are now live; the vacated blocks join the free list (the
        # highest last, so the LIFO pool hands them out high-first as before)
        moved_to = set(remap.values())
        self._free_blocks = [b for b in self._free_blocks if b not in moved_to] + [s for s, _ in moves]
        return moves
