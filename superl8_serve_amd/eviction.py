"""Prompt-time KV eviction: SnapKV selection, Ada-KV budgets, the DuoAttention
split, the recall gate and keep-list compaction, with the interface of the
reference's ``EvictionConfig`` / ``KVEviction`` (superl8serve/engine/kv_cache.py:44-429).

Scoring runs on the gfx950 kernels (``ops.snapkv_scores`` over a dense K as
the reference takes it, or ``ops.snapkv_scores_paged`` straight over a
sequence's int8 K in the paged cache).  Compaction moves the kept tokens'
quantized rows into fresh blocks with one gather launch across every layer
and cache tensor (``ops.gather_slots``): the kept bytes are unchanged, where
the reference dequantizes, un-rotates and re-quantizes each kept token per
layer (kv_cache.py:249-296), which is lossy; it also covers the K8V3 layout,
which the reference's compaction rejects (kv_cache.py:228-232).
"""

from __future__ import annotations

import logging
from dataclasses import dataclass
from typing import Callable

import torch

from . import ops
from .paged_cache import block_bytes as _block_bytes

logger = logging.getLogger(__name__)


@dataclass
class EvictionConfig:
    """Eviction policy knobs (kv_cache.py:44-78): ``policy`` "snapkv" |
    "adakv" | "duoattn"; ``kv_budget`` tokens kept; the recall gate skips an
    eviction whose post-eviction logits fall below ``recall_threshold``
    cosine similarity to the full-KV logits."""

    enabled: bool = False
    policy: str = "snapkv"
    kv_budget: int = 512
    recall_threshold: float = 0.99
    measure_hbm: bool = True
    adakv_min_budget: int = 128
    adakv_max_budget: int = 1024
    duoattn_streaming_heads: float = 0.25
    duoattn_window: int = 128


def _no_op(blocks_after: int, kept: int) -> dict:
    return {"bytes_freed": 0, "blocks_freed": 0, "blocks_after": blocks_after, "tokens_kept": kept}


class KVEviction:
    """Stateless eviction strategies over a ``PagedKVCache``."""

    @staticmethod
    def block_bytes(num_kv_heads: int, block_size: int, head_dim: int, v_quant: str = "int8",
                    lloyd_block: int = 128) -> int:
        """HBM bytes of one block in one layer (kv_cache.py:98-120)."""
        return _block_bytes(num_kv_heads, block_size, head_dim, v_quant, lloyd_block)

    @staticmethod
    def snapkv_selection(q_last: torch.Tensor, k_full: torch.Tensor, budget: int, num_heads: int,
                         num_kv_heads: int) -> list[int]:
        """Sorted positions of the ``budget`` keys the last query attends to
        most, averaged over q heads (kv_cache.py:124-166): ``q_last``
        ``[num_heads, D]`` or ``[1, num_heads, 1, D]``, ``k_full``
        ``[Hkv, S, D]`` or ``[1, Hkv, S, D]`` on the GPU.  Every position when
        ``S <= budget``.

        CHOICE: the logits, softmax and mean are computed in fp32 whatever
        the input dtype; the reference computes them in the input dtype (fp16
        in the engine).  For fp16 inputs, keys whose scores tie within fp16
        rounding may therefore rank differently; the selections recorded from
        the reference (fp32 inputs) are reproduced exactly."""
        seq_len = k_full.shape[-2]
        if seq_len <= budget:
            return list(range(seq_len))
        scores = ops.snapkv_scores(q_last, k_full, num_heads, num_kv_heads)
        return sorted(torch.topk(scores, min(budget, seq_len)).indices.tolist())

    @staticmethod
    def snapkv_selection_paged(cache, layer: int, slot: int, seq_len: int, q_last: torch.Tensor, budget: int,
                               num_heads: int) -> list[int]:
        """``snapkv_selection`` over the slot's own cached K (the first
        ``seq_len`` positions of ``layer``), scored in place in the paged
        int8 store -- no dense K is needed."""
        if seq_len <= budget:
            return list(range(seq_len))
        row = cache._layer_row(layer)
        scores = ops.snapkv_scores_paged(q_last, cache.k_cache[row], cache.k_scale[row], cache._slot_blocks[slot],
                                         seq_len, num_heads)
        return sorted(torch.topk(scores, min(budget, seq_len)).indices.tolist())

    @staticmethod
    def adakv_budgets(num_layers: int, total_budget: int, min_budget: int = 128, max_budget: int = 1024) -> list[int]:
        """Pyramid of per-layer budgets (kv_cache.py:170-186): a linear ramp
        from ``min_budget`` to ``max_budget`` over the layers, rescaled to sum
        to about ``total_budget``, each at least 1."""
        if num_layers <= 1:
            return [total_budget]
        ramp = [int(min_budget + i / (num_layers - 1) * (max_budget - min_budget)) for i in range(num_layers)]
        factor = total_budget / sum(ramp)
        return [max(1, int(b * factor)) for b in ramp]

    @staticmethod
    def duoattn_split(num_heads: int, streaming_fraction: float = 0.25) -> tuple[list[int], list[int]]:
        """``(streaming heads, retrieval heads)``: the first
        ``max(1, int(num_heads * fraction))`` heads stream (kv_cache.py:190-195)."""
        n = max(1, int(num_heads * streaming_fraction))
        return list(range(n)), list(range(n, num_heads))

    @classmethod
    def compact(cls, cache, slot: int, keep_positions: list[int]) -> dict:
        """Keep only ``keep_positions`` of ``slot`` (kv_cache.py:199-313):
        take ``ceil(kept / block_size)`` blocks from the pool (LIFO), move the
        kept tokens there in order -- position ``keep_positions[j]`` becomes
        position ``j`` -- for every layer, then release the old blocks and
        rewrite the slot's block list.  Nothing happens when the keep list
        is empty or would not free a block.

        Returns ``bytes_freed`` (freed blocks x layers x block bytes),
        ``blocks_freed``, ``blocks_after``, ``tokens_kept``.

        CHOICES against the reference: the kept rows are moved byte for byte
        (the reference re-quantizes them); both cache layouts are supported;
        an old block still referenced elsewhere (the prefix cache, another
        slot) loses one reference instead of returning to the pool."""
        old = list(cache._slot_blocks[slot])
        if not old or not keep_positions:
            return _no_op(len(old), 0)
        bs = cache.block_size
        kept = [int(p) for p in keep_positions]
        needed = -(-len(kept) // bs)
        if needed >= len(old):
            return _no_op(len(old), len(kept))
        src = [old[p // bs] * bs + p % bs for p in kept]  # IndexError past the slot's blocks, as the reference
        new: list[int] = []
        for _ in range(needed):
            if not cache._free_blocks:
                raise RuntimeError("PagedKVCache: no free blocks for eviction compaction")
            new.append(cache._free_blocks.pop())
        dst = [new[j // bs] * bs + j % bs for j in range(len(kept))]
        ops.gather_slots(cache._tensors(), src, dst, bs)
        for blk in old:
            if cache._block_refcount.get(blk, 1) > 1:
                cache._block_refcount[blk] -= 1
            else:
                cache._block_refcount.pop(blk, None)
                cache._free_blocks.append(blk)
        cache._slot_blocks[slot] = new
        freed = len(old) - needed
        bb = cls.block_bytes(cache.num_kv_heads, bs, cache.head_dim, cache.v_quant, cache.lloyd_block)
        return {"bytes_freed": freed * cache.num_layers * bb, "blocks_freed": freed, "blocks_after": needed,
                "tokens_kept": len(kept)}

    @classmethod
    def recall_check(cls, logits_full: torch.Tensor, logits_evicted: torch.Tensor, threshold: float = 0.99) -> dict:
        """Cosine similarity of the two logit vectors in fp32 and whether it
        reaches ``threshold`` (kv_cache.py:317-327)."""
        a = logits_full.float().flatten()
        b = logits_evicted.float().flatten()
        cos = (a @ b / (a.norm() * b.norm() + 1e-12)).item()
        return {"cos_sim": cos, "passed": cos >= threshold, "threshold": threshold}

    @classmethod
    def evict(cls, cache, slot: int, seq_len: int, *, eviction_config: EvictionConfig, num_heads: int,
              num_kv_heads: int, head_dim: int, q_last: torch.Tensor | None = None,
              k_full: torch.Tensor | None = None, keep_mask: list[int] | None = None,
              logits_full: torch.Tensor | None = None,
              logits_fn: Callable[[], torch.Tensor] | None = None) -> dict:
        """Choose the positions to keep (explicit ``keep_mask``, or the
        policy), apply the recall gate, compact (kv_cache.py:331-429).
        Returns ``evicted``, ``strategy``, ``metrics`` (compaction metrics
        plus ``budget``) and ``recall``."""
        cfg = eviction_config
        if not cfg.enabled:
            return {"evicted": False, "strategy": None, "metrics": None, "recall": None}
        have_qk = q_last is not None and k_full is not None
        if keep_mask is not None:
            positions = keep_mask
        elif cfg.policy == "snapkv" and have_qk:
            positions = cls.snapkv_selection(q_last, k_full, cfg.kv_budget, num_heads, num_kv_heads)
        elif cfg.policy == "adakv":
            if seq_len <= cfg.kv_budget:
                positions = list(range(seq_len))
            else:
                # the first layer's budget picks the positions for every layer
                budget = cls.adakv_budgets(cache.k_cache.shape[0], cfg.kv_budget, cfg.adakv_min_budget,
                                           cfg.adakv_max_budget)[0]
                positions = (cls.snapkv_selection(q_last, k_full, budget, num_heads, num_kv_heads) if have_qk
                             else list(range(min(budget, seq_len))))
        elif cfg.policy == "duoattn":
            # the streaming heads keep a recent window; the rest keep their top keys
            recent = list(range(max(0, seq_len - cfg.duoattn_window), seq_len))
            top = (cls.snapkv_selection(q_last, k_full, cfg.kv_budget, num_heads, num_kv_heads) if have_qk
                   else list(range(min(cfg.kv_budget, seq_len))))
            positions = sorted(set(recent + top))
        else:
            positions = list(range(min(cfg.kv_budget, seq_len)))
        if len(positions) >= seq_len:
            return {"evicted": False, "strategy": cfg.policy, "metrics": None, "recall": None}
        recall = None
        if cfg.recall_threshold < 1.0 and logits_full is not None and logits_fn is not None:
            recall = cls.recall_check(logits_full, logits_fn(), cfg.recall_threshold)
            if not recall["passed"]:
                logger.warning("Recall gate BLOCKED eviction (cos=%.4f < %.4f)", recall["cos_sim"],
                               recall["threshold"])
                return {"evicted": False, "strategy": cfg.policy, "metrics": None, "recall": recall}
        metrics = cls.compact(cache, slot, positions)
        metrics["budget"] = cfg.kv_budget
        return {"evicted": True, "strategy": cfg.policy, "metrics": metrics, "recall": recall}
