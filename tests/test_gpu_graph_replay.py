"""HIP graph capture of the verify and sliding-window decode ops (the
reference captures decode and verify in CUDA graphs, cuda_graph.py:455-637):
each op is captured once, replayed several times with fresh inputs copied into
its static buffers and eager work in between, and every replay must equal the
eager call bit for bit."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from superl8_serve_amd import ops
from tests.kvcase import make_case, oracle_fill_int8, oracle_fill_k8v3

pytestmark = pytest.mark.gpu

DEV = "cuda"
CODEBOOK = O.gaussian_codebook(3, 128)


def _t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def _replays_equal_eager(step, inputs, seed, reps=3):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_static = step()
    rng = np.random.default_rng(seed)
    for rep in range(reps):
        for buf in inputs:
            buf.copy_(torch.from_numpy(rng.standard_normal(tuple(buf.shape)).astype(np.float16)).to(DEV))
        graph.replay()
        torch.cuda.synchronize()
        got = out_static.clone()
        eager = step()
        torch.cuda.synchronize()
        assert torch.equal(got, eager), f"replay {rep} differs from eager"


@pytest.mark.parametrize("k8v3", [False, True])
def test_graph_replay_verify(k8v3):
    case = make_case(501, 3, 16, 4, 128, 16, [300, 77, 1000])
    prefix = _t(np.array([290, 70, 990], np.int32))
    q_in = torch.zeros((3, 16, 10, 128), dtype=torch.float16, device=DEV)
    bt = _t(case.block_table)
    kw = dict(max_context_len=int(case.block_table.shape[1] * case.block_size), scale=case.scale)
    if k8v3:
        kc, ks, vp, vn = (_t(x) for x in oracle_fill_k8v3(case, CODEBOOK))
        cb = _t(CODEBOOK)

        def step():
            return ops.attn_paged_verify_k8v3(q_in, kc, ks, vp, vn, cb, bt, prefix, case.block_size, **kw)
    else:
        kc, ks, vc, vs = (_t(x) for x in oracle_fill_int8(case))

        def step():
            return ops.attn_paged_verify(q_in, kc, ks, vc, vs, bt, prefix, case.block_size, **kw)
    _replays_equal_eager(step, [q_in], 502)


def test_graph_replay_window_decode():
    case = make_case(511, 4, 8, 2, 128, 16, [600, 33, 5, 2000])
    kc, ks, vc, vs = (_t(x) for x in oracle_fill_int8(case))
    bt, cl = _t(case.block_table), _t(case.lens.astype(np.int32))
    q_in = torch.zeros((4, 8, 1, 128), dtype=torch.float16, device=DEV)

    def step():
        return ops.attn_paged_decode_window(q_in, kc, ks, vc, vs, bt, cl, case.block_size, max_context_len=2000,
                                            window=300, scale=case.scale)
    _replays_equal_eager(step, [q_in], 512)
