"""Arrival counters of the decode kernel.

A row split across workgroups is combined by the workgroup whose segment
completes it: every segment stores its partial, then adds its length to the
row's counter word at the end of the workspace; the word carries a tag of the
launch, so the workspace needs no initialisation, and the completing arrival
clears it.  These tests call the C ABI with a workspace of their own: filled
with random bytes and with stale words of other launches, reused across calls,
and replayed in a graph (same tag on every replay).  Outputs must equal the
op's own (fresh workspace) bit for bit and stay within tolerance of the
oracle; after each call every counter word is either zero (a split row, its
word cleared by the completing arrival) or untouched (a row never split).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from superl8_serve_amd import _lib, ops
from tests.kvcase import make_case, oracle_fill_int8

pytestmark = pytest.mark.gpu

DEV = "cuda"
ERR_WORKSPACE = -4
ERR_UNSUPPORTED = -2

# (wg_per_head, ghost): default slicing; long rows over few slices (every row
# split); ghost-free slices that end inside short rows
SLICINGS = [(None, None), (3, 256), (7, 0)]


def _t(x, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(x))
    if dtype is not None:
        t = t.to(dtype)
    return t.to(DEV)


def _case(seed=71):
    return make_case(seed, 6, 8, 2, 128, 16, [700, 33, 0, 1500, 64, 5])


def _decode_abi(case, cache_t, q3, ws, ws_bytes=None, ptr_offset=0, max_context_len=None):
    kc, ks, vc, vs = cache_t
    b, hq, d = q3.shape
    n, hkv, bs, _ = kc.shape
    bt = _t(case.block_table)
    cl = _t(case.lens.astype(np.int32))
    out = torch.empty((b, hq, d), dtype=torch.float16, device=DEV)
    mcl = int(case.lens.max()) if max_context_len is None else max_context_len
    rc = _lib.load().s8kv_decode_int8(
        q3.data_ptr(), b, hq, hkv, d, q3.stride(0), q3.stride(1),
        kc.data_ptr(), ks.data_ptr(), vc.data_ptr(), vs.data_ptr(), n, bs,
        bt.data_ptr(), bt.stride(0), cl.data_ptr(), mcl, float(case.scale),
        out.data_ptr(), ws.data_ptr() + ptr_offset, ws.numel() if ws_bytes is None else ws_bytes,
        torch.cuda.current_stream().cuda_stream)
    return rc, out


def _counters(ws, case):
    b, hkv = case.batch, case.num_kv_heads
    need = ops.decode_workspace_bytes(b, case.num_q_heads, hkv, case.head_dim, int(case.lens.max()))
    return ws[need - hkv * b * 8:need].view(torch.int64)


def _last_error():
    return (_lib.load().s8kv_last_error() or b"").decode(errors="replace")


def _set_slicing(monkeypatch, wg, ghost):
    if wg is not None:
        monkeypatch.setenv("S8KV_DECODE_WG_PER_HEAD", str(wg))
    if ghost is not None:
        monkeypatch.setenv("S8KV_DECODE_GHOST", str(ghost))


@pytest.mark.parametrize("wg,ghost", SLICINGS)
def test_garbage_workspace_and_counters_cleared(wg, ghost, monkeypatch):
    _set_slicing(monkeypatch, wg, ghost)
    case = _case()
    cache = oracle_fill_int8(case)
    cache_t = tuple(_t(x) for x in cache)
    q3 = _t(case.q, torch.float16)
    ref = O.paged_decode(case.q, O.LayerCache(*cache), case.block_table, case.lens, case.scale)
    want = ops.attn_paged_decode_cached(q3[:, :, None, :], *cache_t, _t(case.block_table),
                                        _t(case.lens.astype(np.int32)), case.block_size,
                                        max_context_len=int(case.lens.max()), scale=case.scale)[:, :, 0, :]
    need = ops.decode_workspace_bytes(case.batch, case.num_q_heads, case.num_kv_heads, case.head_dim,
                                      int(case.lens.max()))
    gen = torch.Generator(device=DEV).manual_seed(5)
    ws = torch.randint(0, 256, (need,), dtype=torch.uint8, device=DEV, generator=gen)
    cnt = _counters(ws, case)
    # stale words of other launches: random tags with counts in range
    tags = torch.randint(1, 1 << 40, cnt.shape, dtype=torch.int64, device=DEV, generator=gen)
    cnt[::2] = (tags[::2] << 24) | torch.randint(1, 40, cnt[::2].shape, dtype=torch.int64, device=DEV, generator=gen)
    before = cnt.clone()
    for call in range(3):
        rc, out = _decode_abi(case, cache_t, q3, ws)
        torch.cuda.synchronize()
        assert rc == 0, _last_error()
        assert torch.equal(out, want), f"call {call}: differs from the op's own result"
        changed = cnt != before
        assert bool((cnt[changed] == 0).all()), f"call {call}: a counter word was left mid-count"
        assert int((before[changed] != 0).sum()) > 0, "no row was split: the case does not exercise the counters"
        mx, rel = O.attention_errors(out.float().cpu().numpy(), ref)
        assert mx <= O.MAX_ABS_TOL and rel <= O.REL_RMS_TOL, f"max err {mx:.3e}, rel rms {rel:.3e}"


@pytest.mark.parametrize("wg,ghost", SLICINGS[1:])
def test_graph_replays_same_tag(wg, ghost, monkeypatch):
    """A captured launch keeps its tag on every replay; the completing
    arrivals clear the words, so each replay starts from zero.  Eager calls
    run between the replays."""
    _set_slicing(monkeypatch, wg, ghost)
    case = _case(72)
    cache_t = tuple(_t(x) for x in oracle_fill_int8(case))
    bt = _t(case.block_table)
    cl = _t(case.lens.astype(np.int32))
    q_in = torch.zeros((case.batch, case.num_q_heads, 1, case.head_dim), dtype=torch.float16, device=DEV)

    def run(q):
        return ops.attn_paged_decode_cached(q, *cache_t, bt, cl, case.block_size,
                                            max_context_len=int(case.lens.max()), scale=case.scale)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run(q_in)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out_g = run(q_in)
    gen = torch.Generator(device=DEV).manual_seed(9)
    for r in range(4):
        q = torch.randn(q_in.shape, device=DEV, generator=gen).half()
        eager = run(q)
        torch.cuda.synchronize()
        q_in.copy_(q)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, eager), f"replay {r} differs from the eager call"


def test_workspace_alignment_and_limits():
    case = _case(73)
    cache_t = tuple(_t(x) for x in oracle_fill_int8(case))
    q3 = _t(case.q, torch.float16)
    need = ops.decode_workspace_bytes(case.batch, case.num_q_heads, case.num_kv_heads, case.head_dim,
                                      int(case.lens.max()))
    ws = torch.zeros(need + 16, dtype=torch.uint8, device=DEV)
    rc, _ = _decode_abi(case, cache_t, q3, ws, ws_bytes=need, ptr_offset=4)
    assert rc == ERR_WORKSPACE and "aligned" in _last_error()
    rc, _ = _decode_abi(case, cache_t, q3, ws, ws_bytes=need - 8)
    assert rc == ERR_WORKSPACE
    rc, _ = _decode_abi(case, cache_t, q3, ws, max_context_len=1 << 28)
    assert rc == ERR_UNSUPPORTED
    torch.cuda.synchronize()


@pytest.mark.parametrize("wg,ghost", SLICINGS)
def test_graph_replays_with_changing_lengths(wg, ghost, monkeypatch):
    """Replays of one captured launch (one tag) with the context lengths
    rewritten between them, as a serving loop replays its decode graph: the
    stream's slicing changes from replay to replay (down to an empty stream
    and back).  Every replay equals an eager call on the same lengths bit for
    bit and stays within tolerance of the oracle."""
    _set_slicing(monkeypatch, wg, ghost)
    case = make_case(74, 6, 8, 2, 128, 16, [1500] * 6)
    cache = oracle_fill_int8(case)
    cache_t = tuple(_t(x) for x in cache)
    bt = _t(case.block_table)
    cl = _t(np.asarray(case.lens, dtype=np.int32))
    q_in = _t(case.q, torch.float16)[:, :, None, :]

    def run(lens_t):
        return ops.attn_paged_decode_cached(q_in, *cache_t, bt, lens_t, case.block_size, max_context_len=1500,
                                            scale=case.scale)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run(cl)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out_g = run(cl)
    schedule = [[1500] * 6, [700, 33, 0, 1500, 64, 5], [1, 0, 2, 0, 0, 3], [1499, 1, 900, 1200, 32, 1500],
                [0] * 6, [257, 640, 1023, 96, 1500, 31]]
    for r, lens in enumerate(schedule):
        lens_np = np.asarray(lens, dtype=np.int32)
        cl.copy_(_t(lens_np))
        g.replay()
        torch.cuda.synchronize()
        got = out_g.clone()
        eager = run(_t(lens_np))
        torch.cuda.synchronize()
        assert torch.equal(got, eager), f"replay {r} (lengths {lens}) differs from the eager call"
        ref = O.paged_decode(case.q, O.LayerCache(*cache), case.block_table, lens_np.astype(np.int64), case.scale)
        mx, rel = O.attention_errors(got[:, :, 0, :].float().cpu().numpy(), ref)
        assert mx <= O.MAX_ABS_TOL and rel <= O.REL_RMS_TOL, f"replay {r}: max err {mx:.3e}, rel rms {rel:.3e}"
