"""GPU parity of the multi-query verify attention over the K8V3 cache (int8 K,
3-bit Lloyd-Max V) against the float64 oracle, through the C ABI.

On a k8v3 cache the reference verifies a chain with S sequential
attn_paged_decode_k8v3 calls (gqa_attention.py:259-277, kv_cache.py:1168-1188);
the one-launch verify must agree with that and with the oracle's masked
attention over the exactly dequantized cache.  Tolerance as for decode:
max(|out-ref| / max(1,|ref|)) <= 2e-3 and relative RMS <= 1e-3.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from superl8_serve_amd import ops
from tests.kvcase import make_case, oracle_fill_k8v3

pytestmark = pytest.mark.gpu

DEV = "cuda"
CODEBOOK = O.gaussian_codebook(3, 128)


def _t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def _random_tree(rng, n):
    masks = []
    for i in range(n):
        parent = int(rng.integers(0, i)) if i else -1
        masks.append((masks[parent] if parent >= 0 else 0) | (1 << i))
    return np.array([m - (1 << 64) if m >= 1 << 63 else m for m in masks], dtype=np.int64)


def _case(seed, batch, hq, hkv, d, bs, prefix, nq, *, outliers=0):
    prefix = np.asarray(prefix)
    case = make_case(seed, batch, hq, hkv, d, bs, prefix + nq, outlier_channels=outliers)
    cache = oracle_fill_k8v3(case, CODEBOOK)
    rng = np.random.default_rng(seed + 1000)
    q = rng.standard_normal((batch, hq, nq, d)).astype(np.float32)
    if outliers:
        q[..., rng.choice(d, size=outliers, replace=False)] *= 20.0
    return case, cache, q.astype(np.float16), prefix


def _run(case, cache, q, prefix, *, query_lens=None, tree_mask=None, q_layout="bhsd"):
    kc, ks, vp, vn = (_t(x) for x in cache)
    qt = _t(np.ascontiguousarray(q.transpose(0, 2, 1, 3))).transpose(1, 2) if q_layout == "bshd" else _t(q)
    out = ops.attn_paged_verify_k8v3(
        qt, kc, ks, vp, vn, _t(CODEBOOK), _t(case.block_table), _t(prefix.astype(np.int32)), case.block_size,
        query_lens=None if query_lens is None else _t(np.asarray(query_lens, np.int32)),
        tree_mask=None if tree_mask is None else _t(tree_mask),
        max_context_len=int(case.block_table.shape[1] * case.block_size), scale=case.scale)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def _ref(case, cache, q, prefix, *, query_lens=None, tree_mask=None):
    kc, ks, vp, vn = cache
    layer = O.LayerCache(kc, ks, v_packed=vp, v_norm=vn, v_codebook=CODEBOOK)
    return O.paged_verify(q, layer, case.block_table, prefix, case.scale, query_lens=query_lens, tree_mask=tree_mask)


def _close(out, ref, what):
    mx, rel = O.attention_errors(out, ref)
    assert mx <= O.MAX_ABS_TOL and rel <= O.REL_RMS_TOL, f"{what}: max err {mx:.3e}, rel rms {rel:.3e}"


@pytest.mark.parametrize("hq,hkv,d,bs,prefix,nq", [
    (8, 2, 128, 16, [100, 37, 256], 5),        # chain verify, G=4
    (32, 2, 128, 256, [300, 511], 9),          # G=16
    (4, 2, 256, 16, [64, 90], 4),              # D=256: two V blocks per key
    (16, 8, 128, 256, [1000, 2500], 20),       # long prefix: several key sub-ranges
])
def test_chain_verify_k8v3(hq, hkv, d, bs, prefix, nq):
    case, cache, q, pre = _case(121 + d + bs, len(prefix), hq, hkv, d, bs, prefix, nq, outliers=2)
    _close(_run(case, cache, q, pre), _ref(case, cache, q, pre), "chain verify")


@pytest.mark.parametrize("d", [128, 256])
def test_chunked_prefill_k8v3(d):
    """A 200-query chunk after a 777-token prefix, q as a [B, S, Hq, D]
    transpose view, outlier channels."""
    case, cache, q, pre = _case(131 + d, 2, 8, 2, d, 16, [777, 64], 200, outliers=2)
    _close(_run(case, cache, q, pre, q_layout="bshd"), _ref(case, cache, q, pre), "chunk")


@pytest.mark.parametrize("nq", [16, 64])
def test_tree_verify_k8v3(nq):
    rng = np.random.default_rng(nq + 7)
    case, cache, q, pre = _case(141 + nq, 3, 16, 4, 128, 16, [500, 129, 2048], nq, outliers=1)
    masks = np.stack([_random_tree(rng, nq) for _ in range(3)])
    _close(_run(case, cache, q, pre, tree_mask=masks), _ref(case, cache, q, pre, tree_mask=masks), "tree")


def test_tree_of_a_chain_equals_chain_k8v3():
    case, cache, q, pre = _case(151, 2, 8, 2, 128, 16, [200, 31], 12)
    chain_masks = np.stack([np.array([(1 << (i + 1)) - 1 for i in range(12)], np.int64)] * 2)
    assert np.array_equal(_run(case, cache, q, pre, tree_mask=chain_masks), _run(case, cache, q, pre))


def test_query_lens_zero_rows_k8v3():
    case, cache, q, pre = _case(161, 3, 8, 2, 128, 16, [50, 80, 10], 10)
    ql = [10, 3, 0]
    out = _run(case, cache, q, pre, query_lens=ql)
    _close(out, _ref(case, cache, q, pre, query_lens=ql), "query_lens")
    assert np.all(out[1, :, 3:] == 0) and np.all(out[2] == 0)


@pytest.mark.parametrize("d", [128, 256])
def test_chain_verify_k8v3_equals_sequential_decodes(d):
    """The reference's chain verify on a k8v3 cache is S attn_paged_decode_k8v3
    calls with context L+t+1: the verify op must agree with the decode op."""
    case, cache, q, pre = _case(171 + d, 2, 16, 4, d, 16, [400, 129], 6)
    out = _run(case, cache, q, pre)
    kc, ks, vp, vn = (_t(x) for x in cache)
    bt = _t(case.block_table)
    for t in range(6):
        dec = ops.attn_paged_decode_k8v3(_t(q[:, :, t:t + 1]), kc, ks, vp, vn, _t(CODEBOOK), bt,
                                         _t((pre + t + 1).astype(np.int32)), case.block_size,
                                         max_context_len=int(pre.max()) + 6, scale=case.scale)
        _close(out[:, :, t], dec[:, :, 0].float().cpu().numpy(), f"decode step {t}")


def test_verify_k8v3_rejects_head_dim_64():
    case = make_case(181, 1, 4, 2, 64, 16, [20])
    kc = torch.zeros((case.num_blocks, 2, 16, 64), dtype=torch.int8, device=DEV)
    ks = torch.ones((case.num_blocks, 2, 16), device=DEV)
    vp = torch.zeros((case.num_blocks, 2, 16, 6), dtype=torch.int32, device=DEV)
    vn = torch.ones((case.num_blocks, 2, 16, 1), device=DEV)
    q = torch.zeros((1, 4, 2, 64), dtype=torch.float16, device=DEV)
    with pytest.raises(RuntimeError, match="head_dim 64"):
        ops.attn_paged_verify_k8v3(q, kc, ks, vp, vn, _t(CODEBOOK), _t(case.block_table), _t(np.array([18], np.int32)),
                                   16, max_context_len=20, scale=0.125)
