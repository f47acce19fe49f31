"""Read-ceiling probes (diagnostics behind the benchmark's read-ceiling
leg): they must read exactly the bytes they claim.  Each workgroup folds the
32-bit words it read into one checksum word; the XOR of all of them equals
the XOR of the K and V words of the listed tiles (each scale word is read by
two lanes and cancels), and of every word of the linear buffer."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from superl8_serve_amd import _lib

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _xor_words(a: np.ndarray) -> int:
    return int(np.bitwise_xor.reduce(np.ascontiguousarray(a).view(np.uint32).ravel(), initial=np.uint32(0)))


@pytest.mark.parametrize("nwg", [1, 7, 64])
def test_probe_read_tiles_reads_every_listed_tile(nwg):
    rng = np.random.default_rng(nwg)
    blocks, hkv, bs, d = 9, 2, 64, 128
    kc = rng.integers(-128, 128, (blocks, hkv, bs, d), dtype=np.int8)
    vc = rng.integers(-128, 128, (blocks, hkv, bs, d), dtype=np.int8)
    ks = rng.standard_normal((blocks, hkv, bs)).astype(np.float32)
    vs = rng.standard_normal((blocks, hkv, bs)).astype(np.float32)
    rows = blocks * hkv * bs
    tiles = rng.choice(rows // 32, 23, replace=False).astype(np.int32) * 32  # 32-row tiles, in any order
    sink = torch.zeros(nwg, dtype=torch.int32, device=DEV)
    t = [torch.from_numpy(x).to(DEV) for x in (kc, ks, vc, vs, tiles)]
    lib = _lib.load()
    rc = lib.s8kv_probe_read_tiles(t[0].data_ptr(), t[1].data_ptr(), t[2].data_ptr(), t[3].data_ptr(), rows, d,
                                   t[4].data_ptr(), len(tiles), nwg, sink.data_ptr(),
                                   torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "s8kv_probe_read_tiles")
    got = _xor_words(sink.cpu().numpy())
    flat_k, flat_v = kc.reshape(rows, d), vc.reshape(rows, d)
    want = 0
    for r0 in tiles:
        want ^= _xor_words(flat_k[r0:r0 + 32]) ^ _xor_words(flat_v[r0:r0 + 32])
    assert got == want


@pytest.mark.parametrize("nbytes,nwg", [(16, 1), (4096 * 16 + 48, 5), (1 << 20, 256)])
def test_probe_read_linear_reads_the_whole_buffer(nbytes, nwg):
    rng = np.random.default_rng(nbytes)
    buf = rng.integers(0, 256, nbytes, dtype=np.uint8)
    t = torch.from_numpy(buf).to(DEV)
    sink = torch.zeros(nwg, dtype=torch.int32, device=DEV)
    lib = _lib.load()
    rc = lib.s8kv_probe_read_linear(t.data_ptr(), nbytes, nwg, sink.data_ptr(), torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "s8kv_probe_read_linear")
    assert _xor_words(sink.cpu().numpy()) == _xor_words(buf)


def test_probe_arguments_are_checked():
    lib = _lib.load()
    rc = lib.s8kv_probe_read_tiles(None, None, None, None, 64, 64, None, 0, 1, None, None)
    assert rc != 0 and b"head_dim" in lib.s8kv_last_error()
    rc = lib.s8kv_probe_read_linear(ctypes.c_void_p(16), 8, 1, ctypes.c_void_p(16), None)
    assert rc != 0
