"""GPU parity of the multi-query verify attention (tree verify, chain verify,
chunked prefill) against the float64 oracle, through the C ABI.

Tolerance as for decode: max(|out-ref| / max(1,|ref|)) <= 2e-3 and relative
RMS <= 1e-3 against the oracle over the exactly dequantized cache.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from superl8_serve_amd import ops
from tests.kvcase import make_case, oracle_fill_int8

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def _random_tree(rng, n):
    """Ancestor masks of a random tree over nodes 0..n-1 (parent[i] < i);
    bit i of mask[i] is set (a node sees itself).  int64, two's complement."""
    masks = []
    for i in range(n):
        parent = int(rng.integers(0, i)) if i else -1
        masks.append((masks[parent] if parent >= 0 else 0) | (1 << i))
    return np.array([m - (1 << 64) if m >= 1 << 63 else m for m in masks], dtype=np.int64)


def _verify_case(seed, batch, hq, hkv, d, bs, prefix, nq, *, outliers=0, q_layout="bhsd"):
    """prefix[b] tokens + nq drafts per row, all appended (oracle) to the cache."""
    prefix = np.asarray(prefix)
    lens = prefix + nq
    case = make_case(seed, batch, hq, hkv, d, bs, lens, outlier_channels=outliers)
    cache = oracle_fill_int8(case)
    rng = np.random.default_rng(seed + 1000)
    q = rng.standard_normal((batch, hq, nq, d)).astype(np.float32)
    if outliers:
        ch = rng.choice(d, size=outliers, replace=False)
        q[..., ch] *= 20.0
    q = q.astype(np.float16)
    return case, cache, q, prefix


def _run(case, cache, q, prefix, *, query_lens=None, tree_mask=None, q_layout="bhsd"):
    kc, ks, vc, vs = (_t(x) for x in cache)
    if q_layout == "bshd":  # the verify seam's [B, S, Hq, D] tensor viewed as [B, Hq, S, D]
        qt = _t(np.ascontiguousarray(q.transpose(0, 2, 1, 3))).transpose(1, 2)
    else:
        qt = _t(q)
    max_ctx = int(case.block_table.shape[1] * case.block_size)
    out = ops.attn_paged_verify(
        qt, kc, ks, vc, vs, _t(case.block_table), _t(prefix.astype(np.int32)), case.block_size,
        query_lens=None if query_lens is None else _t(np.asarray(query_lens, np.int32)),
        tree_mask=None if tree_mask is None else _t(tree_mask),
        max_context_len=max_ctx, scale=case.scale)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def _ref(case, cache, q, prefix, *, query_lens=None, tree_mask=None):
    layer = O.LayerCache(*cache)
    return O.paged_verify(q, layer, case.block_table, prefix, case.scale, query_lens=query_lens, tree_mask=tree_mask)


def _close(out, ref, what):
    mx, rel = O.attention_errors(out, ref)
    assert mx <= O.MAX_ABS_TOL and rel <= O.REL_RMS_TOL, f"{what}: max err {mx:.3e}, rel rms {rel:.3e}"


@pytest.mark.parametrize("hq,hkv,d,bs,prefix,nq", [
    (8, 2, 128, 16, [100, 37, 256], 5),        # chain verify, G=4
    (16, 16, 64, 4, [33, 0, 70], 7),           # G=1, empty prefix, tiny blocks
    (32, 2, 128, 256, [300, 511], 9),          # G=16
    (4, 2, 256, 16, [64, 90], 4),              # D=256
    (16, 8, 128, 256, [1000, 2500], 20),       # long prefix: several key sub-ranges
])
def test_chain_verify(hq, hkv, d, bs, prefix, nq):
    case, cache, q, pre = _verify_case(21 + d + bs, len(prefix), hq, hkv, d, bs, prefix, nq)
    _close(_run(case, cache, q, pre), _ref(case, cache, q, pre), "chain verify")


def test_chunked_prefill_bottom_right_causal():
    """A 200-query chunk after a 777-token prefix (several 64-row query blocks,
    diagonal tiles), q as a [B, S, Hq, D] transpose view, outlier channels."""
    case, cache, q, pre = _verify_case(31, 2, 8, 2, 128, 16, [777, 64], 200, outliers=2)
    _close(_run(case, cache, q, pre, q_layout="bshd"), _ref(case, cache, q, pre), "chunk")


@pytest.mark.parametrize("nq", [16, 40, 64])
def test_tree_verify(nq):
    rng = np.random.default_rng(nq)
    case, cache, q, pre = _verify_case(41 + nq, 3, 16, 4, 128, 16, [500, 129, 2048], nq, outliers=1)
    masks = np.stack([_random_tree(rng, nq) for _ in range(3)])
    _close(_run(case, cache, q, pre, tree_mask=masks), _ref(case, cache, q, pre, tree_mask=masks), "tree")


def test_tree_of_a_chain_equals_chain():
    case, cache, q, pre = _verify_case(51, 2, 8, 2, 128, 16, [200, 31], 12)
    chain_masks = np.stack([np.array([(1 << (i + 1)) - 1 for i in range(12)], np.int64)] * 2)  # node i: drafts 0..i
    out_tree = _run(case, cache, q, pre, tree_mask=chain_masks)
    out_chain = _run(case, cache, q, pre)
    assert np.array_equal(out_tree, out_chain)


def test_query_lens_zero_rows():
    case, cache, q, pre = _verify_case(61, 3, 8, 2, 128, 16, [50, 80, 10], 10)
    ql = [10, 3, 0]
    out = _run(case, cache, q, pre, query_lens=ql)
    ref = _ref(case, cache, q, pre, query_lens=ql)
    _close(out, ref, "query_lens")
    assert np.all(out[1, :, 3:] == 0) and np.all(out[2] == 0)


def test_chain_verify_equals_sequential_decodes():
    """The reference's chain verify is S paged decodes with context L+t+1
    (gqa_attention.py:259-277): the verify op must agree with the decode op."""
    case, cache, q, pre = _verify_case(71, 2, 16, 4, 128, 16, [400, 129], 6)
    out = _run(case, cache, q, pre)
    kc, ks, vc, vs = (_t(x) for x in cache)
    bt = _t(case.block_table)
    for t in range(6):
        dec = ops.attn_paged_decode_cached(_t(q[:, :, t:t + 1]), kc, ks, vc, vs, bt, _t((pre + t + 1).astype(np.int32)),
                                           case.block_size, max_context_len=int(pre.max()) + 6, scale=case.scale)
        _close(out[:, :, t], dec[:, :, 0].float().cpu().numpy(), f"decode step {t}")
