"""Softmax weights far below the largest, in bulk, against the oracle.

Each row's first token is an attention sink: every query scores it S = 14
(natural log units) while the other keys score ~N(0, 1.2), and V carries a
bias of 1.  Each other key then weighs ~1e-6 of the sink and together they
hold ~5% of the softmax mass in 32K-token rows (~2% in keys below 2^-24).  Their products weight x V
scale (~3e-2) lie below fp16's smallest subnormal, so without the weight
shift the kernels apply (WeightShift in csrc/s8kv_device.h) they would be
dropped from the PV MFMAs while still counted in the normalizer.  Decode runs
with one slice per head (a whole row per workgroup, a quarter per wave) and
with the default slicing; chunk verify reads each row in one workgroup."""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import kv_oracle as O
from tests.kvcase import make_case
from tests.kvgpu import KINDS, alloc, append, assert_close, decode, layer, t, to_np, verify

pytestmark = pytest.mark.gpu

SINK = 14.0
SINK_NORM = 30.0  # |K| of the sink token


def _sink_case(seed, hq, hkv, d, bs, lens, nq=0):
    """make_case with V += 1 and, per row and KV head, the row's first key set
    to SINK_NORM * u (u a random unit vector) and every query of the group
    (decode q, and ``nq`` verify queries) given the component along u that
    scores it SINK."""
    case = make_case(seed, len(lens), hq, hkv, d, bs, lens)
    rng = np.random.default_rng(seed + 1)
    g = hq // hkv
    k = case.k.astype(np.float64)
    v = case.v.astype(np.float64) + 1.0
    q = case.q.astype(np.float64)
    qv = rng.standard_normal((case.batch, hq, nq, d)) if nq else None
    along = SINK * math.sqrt(d) / SINK_NORM  # q . u giving score SINK with scale 1/sqrt(d)
    starts = np.concatenate([[0], np.cumsum(case.lens)[:-1]]).astype(np.int64)
    for b in range(case.batch):
        for j in range(hkv):
            u = rng.standard_normal(d)
            u /= np.linalg.norm(u)
            k[starts[b], j] = SINK_NORM * u
            for h in range(j * g, (j + 1) * g):
                q[b, h] += (along - q[b, h] @ u) * u
                if nq:
                    qv[b, h] += (along - qv[b, h] @ u)[:, None] * u
    case.k, case.v, case.q = k.astype(np.float16), v.astype(np.float16), q.astype(np.float16)
    return case, None if qv is None else qv.astype(np.float16)


def _fill(kind, case):
    cache = alloc(kind, case.num_blocks, case.num_kv_heads, case.block_size, case.head_dim)
    append(kind, t(case.k), t(case.v), cache, t(case.slots))
    return cache, tuple(to_np(x) for x in cache)


def _assert_underflow_regime(lc, case, q):
    """The case exercises what it claims: in row 0, keys whose weight times V
    scale (relative to the row's largest weight) is below 2^-24 hold >= 1% of
    the softmax mass of head 0 (1.9% in these cases; passing their weights
    through fp16 hi + lo unshifted misses the oracle by ~4e-3 rel RMS)."""
    k, v = O.exact_kv(lc, case.block_table[0], int(case.lens[0]))
    s = case.scale * (k[0] @ q.astype(np.float64))
    e = np.exp(s - s.max())
    rows = O.gather_rows(case.block_table[0], case.num_kv_heads, case.block_size, int(case.lens[0]))[:, 0]
    vsc = lc.v_scale.reshape(-1)[rows]
    lost = e[e * vsc < 2.0 ** -24].sum() / e.sum()
    assert lost >= 0.01, f"only {lost:.3%} of the mass is below fp16's range"


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("wg_per_head", [1, None])
def test_sink_decode(kind, wg_per_head, monkeypatch):
    if wg_per_head is not None:
        monkeypatch.setenv("S8KV_DECODE_WG_PER_HEAD", str(wg_per_head))
    hq, hkv, d, bs = 8, 2, 128, 256
    lens = np.array([32768, 20000])
    case, _ = _sink_case(800, hq, hkv, d, bs, lens)
    cache, host = _fill(kind, case)
    lc = layer(kind, host)
    if kind == "int8":  # K8V3's block norms (~1.4 here) keep these weights in fp16's range
        _assert_underflow_regime(lc, case, case.q[0, 0])
    out = decode(kind, t(case.q), cache, t(case.block_table), t(lens.astype(np.int32)), bs, int(lens.max()),
                 case.scale)
    ref = O.paged_decode(case.q, lc, case.block_table, lens, case.scale)
    assert_close(to_np(out.float()), ref, f"{kind} sink decode (wg/head {wg_per_head})")


@pytest.mark.parametrize("kind,d", [("int8", 128), ("int8", 64), ("k8v3", 128), ("k8v3", 256)])
def test_sink_chunk_verify(kind, d):
    hq, hkv, bs, nq = 8, 2, 256, 16
    prefix = np.array([32768, 20000])
    case, qv = _sink_case(810 + d, hq, hkv, d, bs, prefix + nq, nq=nq)
    cache, host = _fill(kind, case)
    lc = layer(kind, host)
    if kind == "int8":
        _assert_underflow_regime(lc, case, qv[0, 0, 0])
    out = verify(kind, t(qv), cache, t(case.block_table), t(prefix.astype(np.int32)), None, bs,
                 int(case.lens.max()), case.scale)
    ref = O.paged_verify(qv, lc, case.block_table, prefix, case.scale)
    assert_close(to_np(out.float()), ref, f"{kind} D={d} sink chunk verify")
