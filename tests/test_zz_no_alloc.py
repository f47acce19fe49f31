"""GPU test of the allocation-free decode step
(``s8kv_decode_append_int8_noalloc``), called through the C ABI: its output
and cache bytes must equal those of ``s8kv_decode_append_int8`` (the same
kernels with a caller-provided workspace) bit for bit, on two calls in a
row, the second with a smaller batch and shorter rows than the first (the
static scratch keeps the first call's partials and counters)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from superl8_serve_amd import _lib, ops
from tests.kvcase import empty_int8_cache, make_case

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def _inputs(case):
    """Cache holding every token but each row's last, and the rows' last
    tokens [B, Hkv, D] (the ones the decode step appends)."""
    ends = np.cumsum(case.lens)
    keep = np.ones(int(ends[-1]), bool)
    keep[ends - 1] = False
    pre = empty_int8_cache(case)
    O.quantize_kv_write_paged(case.k[keep], case.v[keep], *pre, case.slots[keep])
    return pre, case.k[ends - 1], case.v[ends - 1]


def _noalloc(case, pre, k_new, v_new, max_ctx):
    kc, ks, vc, vs = (_t(x) for x in pre)
    q = _t(case.q)
    kn, vn = _t(k_new), _t(v_new)
    bt, cl = _t(case.block_table), _t(case.lens.astype(np.int32))
    out = torch.empty_like(q)
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.s8kv_decode_append_int8_noalloc(
        q.data_ptr(), case.batch, case.num_q_heads, case.num_kv_heads, case.head_dim, q.stride(0), q.stride(1),
        kn.data_ptr(), kn.stride(0), kn.stride(1), vn.data_ptr(), vn.stride(0), vn.stride(1),
        kc.data_ptr(), ks.data_ptr(), vc.data_ptr(), vs.data_ptr(), case.num_blocks, case.block_size,
        bt.data_ptr(), bt.stride(0), cl.data_ptr(), max_ctx, case.scale, out.data_ptr(), stream)
    _lib.check(rc, "s8kv_decode_append_int8_noalloc")
    torch.cuda.synchronize()
    return out.cpu().numpy(), [x.cpu().numpy() for x in (kc, ks, vc, vs)]


def _with_workspace(case, pre, k_new, v_new, max_ctx):
    kc, ks, vc, vs = (_t(x) for x in pre)
    out = ops.attn_paged_decode_append(_t(case.q), _t(k_new), _t(v_new), kc, ks, vc, vs, _t(case.block_table),
                                       _t(case.lens.astype(np.int32)), case.block_size, max_context_len=max_ctx,
                                       scale=case.scale)
    torch.cuda.synchronize()
    return out.cpu().numpy(), [x.cpu().numpy() for x in (kc, ks, vc, vs)]


def _same(a, b):
    return np.array_equal(np.ascontiguousarray(a).view(np.uint8), np.ascontiguousarray(b).view(np.uint8))


def test_noalloc_equals_workspace_entry_point_on_two_calls():
    rng = np.random.default_rng(91)
    cases = [
        # long rows split across many workgroups, outlier channels x20
        make_case(91, 24, 32, 8, 128, 16, rng.integers(200, 3000, size=24), outlier_channels=2),
        # then a smaller batch of shorter rows: the scratch still holds the
        # first call's partials and counter words
        make_case(92, 5, 32, 8, 128, 16, rng.integers(1, 400, size=5), outlier_channels=2),
    ]
    for i, case in enumerate(cases):
        print(f"noalloc call {i}: batch {case.batch}, max len {int(case.lens.max())}", flush=True)
        pre, k_new, v_new = _inputs(case)
        max_ctx = int(case.lens.max())
        want, want_cache = _with_workspace(case, pre, k_new, v_new, max_ctx)
        got, got_cache = _noalloc(case, pre, k_new, v_new, max_ctx)
        assert _same(got, want), f"call {i}: output differs from s8kv_decode_append_int8"
        for a, b, name in zip(got_cache, want_cache, ("k_cache", "k_scale", "v_cache", "v_scale")):
            assert _same(a, b), f"call {i}: {name} differs from s8kv_decode_append_int8"
        # and the appended bytes are the oracle's
        full = empty_int8_cache(case)
        O.quantize_kv_write_paged(case.k, case.v, *full, case.slots)
        for a, b, name in zip(got_cache, full, ("k_cache", "k_scale", "v_cache", "v_scale")):
            assert _same(a, b), f"call {i}: {name} differs from the oracle's append"


def test_noalloc_rejects_geometry_beyond_the_scratch():
    lib = _lib.load()
    # batch 65535 with 16 q heads on one KV head of head_dim 256 needs ~1 GiB
    rc = lib.s8kv_decode_append_int8_noalloc(
        None, 65535, 16, 1, 256, 0, 0, None, 0, 0, None, 0, 0, None, None, None, None, 4, 16,
        None, 0, None, 16, 0.1, None, None)
    assert rc == -4 and b"static scratch" in lib.s8kv_last_error()
