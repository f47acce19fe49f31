"""The closed form behind the whole-pool GPU test, pinned against the oracle
on small pools of the same construction (no GPU): zero keys with a constant
V row, one needle per q head, decode and chain-verify limits."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import kv_oracle as O
from tests.kvcase import make_needle_case, needle_fill, needle_reference


@pytest.mark.parametrize("nblk,bs,d,hq", [(64, 16, 128, 8), (33, 4, 64, 4), (17, 32, 128, 16)])
def test_needle_closed_form_matches_oracle(nblk, bs, d, hq):
    half = nblk // 2
    nc = make_needle_case(50 + nblk, nblk, bs, d, hq, [(0, 0), (half, 0), (half - 1, bs - 1), (3 * half // 2, bs // 2),
                                                       (half // 2, 1)][: hq - 2])
    n = nc.n
    assert nc.rows[0] == nblk * bs - 1, "needle 0 must sit in the pool's last row"
    layer = O.LayerCache(*needle_fill(nc))
    bt = nc.block_table[None]
    dec = O.paged_decode(nc.q[None], layer, bt, np.array([n]), nc.scale)[0]
    np.testing.assert_allclose(needle_reference(nc, n), dec, rtol=1e-10, atol=1e-12)
    # each head weighs its own needle against the background comparably
    w_needle = np.exp(nc.scale * nc.q.astype(np.float64) @ (
        (nc.k_i8.astype(np.float64) * nc.k_scale[:, None]) @ O.hadamard_matrix(d)).T)
    frac = np.diag(w_needle) / (w_needle.sum(axis=1) + n - hq)
    assert np.all((frac > 0.1) & (frac < 0.9)), frac
    nq = 4
    qv = np.ascontiguousarray(np.broadcast_to(nc.q[:, None, :], (hq, nq, d)))[None]
    ver = O.paged_verify(qv, layer, bt, np.array([n - nq]), nc.scale)[0]
    for s in range(nq):
        np.testing.assert_allclose(needle_reference(nc, n - nq + s + 1), ver[:, s], rtol=1e-10, atol=1e-12)
    # a window verify: positions [n - nq - window, n - nq + s] (some needles outside the window)
    window = n // 3
    wver = O.paged_verify(qv, layer, bt, np.array([n - nq]), nc.scale, window=window)[0]
    for s in range(nq):
        np.testing.assert_allclose(needle_reference(nc, n - nq + s + 1, start=n - nq - window), wver[:, s],
                                   rtol=1e-10, atol=1e-12)
    assert ((nc.pos < n - nq - window).any() and (nc.pos >= n - nq - window).any()), "needles on both sides"


def test_needle_reference_detects_a_missing_needle():
    """Dropping one needle (the last row of the pool) moves its head's output
    far outside the attention tolerance."""
    nc = make_needle_case(61, 64, 16, 128, 8, [(0, 0), (32, 0)])
    full = needle_reference(nc, nc.n)
    k = nc.k_i8.copy()
    nc.k_i8[0] = 0  # needle 0 becomes a background key with its own V
    dropped = needle_reference(nc, nc.n)
    nc.k_i8[:] = k
    mx, _ = O.attention_errors(dropped, full)
    assert mx > 100 * O.MAX_ABS_TOL
