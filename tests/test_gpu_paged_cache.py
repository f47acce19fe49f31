"""The host paged cache driving the gfx950 kernels end to end (GPU): prefill
and decode writes through slot mappings, batched decode, verify, prefix
sharing with copy-on-write, and pool compaction -- results checked against the
oracle over the cache contents and against reads taken before each move."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from superl8_serve_amd.paged_cache import PagedKVCache

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _layer(c, layer):
    r = c._layer_row(layer)
    if c.v_quant == "lloydmax3":
        return O.LayerCache(c.k_cache[r].cpu().numpy(), c.k_scale[r].cpu().numpy(),
                            v_packed=c.v_packed[r].cpu().numpy(), v_norm=c.v_norm[r].cpu().numpy(),
                            v_codebook=c.v_codebook[r].cpu().numpy())
    return O.LayerCache(c.k_cache[r].cpu().numpy(), c.k_scale[r].cpu().numpy(), c.v_cache[r].cpu().numpy(),
                        c.v_scale[r].cpu().numpy())


def _close(out, ref, what):
    mx, rel = O.attention_errors(out, ref)
    assert mx <= O.MAX_ABS_TOL and rel <= O.REL_RMS_TOL, f"{what}: max err {mx:.3e}, rel rms {rel:.3e}"


@pytest.mark.parametrize("v_quant,block_size", [("int8", 16), ("int8", 256), ("lloydmax3", 16)])
def test_prefill_decode_flow(v_quant, block_size):
    g = torch.Generator(device=DEV).manual_seed(0)
    hq, hkv, d = 16, 4, 128
    c = PagedKVCache(2, 4, hkv, 1024, d, device=DEV, block_size=block_size, v_quant=v_quant)
    lens = [300, 37, 512]
    slots = [c.alloc() for _ in lens]
    c.ensure_capacity(slots, [n + 1 for n in lens])
    for layer in range(2):
        for s, n in zip(slots, lens):
            k = torch.randn(1, hkv, n, d, generator=g, device=DEV).half()
            v = torch.randn(1, hkv, n, d, generator=g, device=DEV).half()
            c.write_prefill(layer, k, v, slot=s)
        kn = torch.randn(len(lens), hkv, d, generator=g, device=DEV).half()
        vn = torch.randn(len(lens), hkv, d, generator=g, device=DEV).half()
        c.write_decode(layer, slots, lens, kn, vn)
    q = torch.randn(len(lens), hq, 1, d, generator=g, device=DEV).half()
    scale = 1.0 / math.sqrt(d)
    out = c.decode_attn(1, q, slots, lens, scale=scale)
    bt = c.block_table(slots).cpu().numpy()
    ref = O.paged_decode(q[:, :, 0].cpu().numpy(), _layer(c, 1), bt, np.array(lens) + 1, scale)
    _close(out[:, :, 0].float().cpu().numpy(), ref, f"decode {v_quant}")
    # the dense reader returns the same tokens the kernels attend
    # the reference's dense reader: bit-exact (K un-rotated row by row, V elementwise)
    k16, v16 = c.read_dense(1, slots[1], lens[1] + 1)
    rk, rv = O.read_dense(_layer(c, 1), bt[1], lens[1] + 1)
    assert np.array_equal(k16.cpu().numpy().view(np.uint16), rk.view(np.uint16))
    assert np.array_equal(v16.cpu().numpy().view(np.uint16), rv.view(np.uint16))


@pytest.mark.parametrize("v_quant", ["int8", "lloydmax3"])
def test_decode_step_equals_write_then_attend(v_quant):
    """decode_step (one launch for int8) leaves the same cache and returns the
    same output as write_decode followed by decode_attn."""
    g = torch.Generator(device=DEV).manual_seed(3)
    hq, hkv, d, bs = 16, 4, 128, 16
    caches = [PagedKVCache(1, 4, hkv, 1024, d, device=DEV, block_size=bs, v_quant=v_quant) for _ in range(2)]
    lens = [300, 0, 47, 512]
    for c in caches:
        slots = [c.alloc() for _ in lens]
        c.ensure_capacity(slots, [n + 1 for n in lens])
    g2 = torch.Generator(device=DEV).manual_seed(4)
    for s, n in zip(slots, lens):
        if n == 0:
            continue
        k = torch.randn(1, hkv, n, d, generator=g2, device=DEV).half()
        v = torch.randn(1, hkv, n, d, generator=g2, device=DEV).half()
        for c in caches:
            c.write_prefill(0, k, v, slot=s)
    kn = torch.randn(len(lens), hkv, d, generator=g, device=DEV).half()
    vn = torch.randn(len(lens), hkv, d, generator=g, device=DEV).half()
    q = torch.randn(len(lens), hq, 1, d, generator=g, device=DEV).half()
    scale = 1.0 / math.sqrt(d)
    caches[0].write_decode(0, slots, lens, kn, vn)
    ref = caches[0].decode_attn(0, q, slots, lens, scale=scale)
    out = caches[1].decode_step(0, q, kn, vn, slots, lens, scale=scale)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    names = ("k_cache", "k_scale", "v_cache", "v_scale") if v_quant == "int8" else ("k_cache", "k_scale", "v_packed", "v_norm")
    for name in names:
        assert torch.equal(getattr(caches[0], name), getattr(caches[1], name)), name


@pytest.mark.parametrize("v_quant", ["int8", "lloydmax3"])
def test_chunked_prefill_positions_and_verify(v_quant):
    g = torch.Generator(device=DEV).manual_seed(1)
    hq, hkv, d, bs = 8, 2, 128, 16
    c = PagedKVCache(1, 2, hkv, 512, d, device=DEV, block_size=bs, v_quant=v_quant)
    s = c.alloc()
    prefix, chunk = 100, 40
    c.ensure_capacity([s], [prefix + chunk])
    kp = torch.randn(1, hkv, prefix, d, generator=g, device=DEV).half()
    c.write_prefill(0, kp, torch.randn_like(kp), slot=s)
    kc = torch.randn(1, hkv, chunk, d, generator=g, device=DEV).half()
    pos = torch.arange(prefix, prefix + chunk, device=DEV)
    c.write_prefill(0, kc, torch.randn_like(kc), slot=s, positions=pos)
    q = torch.randn(1, hq, chunk, d, generator=g, device=DEV).half()
    out = c.verify_attn(0, q, [s], [prefix], scale=0.1)
    bt = c.block_table([s]).cpu().numpy()
    ref = O.paged_verify(q.cpu().numpy(), _layer(c, 0), bt, np.array([prefix]), 0.1)
    _close(out.float().cpu().numpy(), ref, f"{v_quant} chunk via cache")


def test_prefix_share_copy_on_write():
    g = torch.Generator(device=DEV).manual_seed(2)
    hkv, d, bs = 2, 64, 16
    c = PagedKVCache(2, 3, hkv, 256, d, device=DEV, block_size=bs)
    a = c.alloc()
    toks = list(range(40))
    c.ensure_capacity([a], [40])
    for layer in range(2):
        k = torch.randn(1, hkv, 40, d, generator=g, device=DEV).half()
        c.write_prefill(layer, k, torch.randn_like(k), slot=a)
    c.store_prefix(toks, a)
    n, blocks = c.lookup_prefix(toks)
    assert n == 32 and blocks == c._slot_blocks[a][:2]
    b = c.alloc()
    c.share_blocks(b, blocks)
    before = [t.clone() for t in c.read_dense(1, b, 32)]
    new = c.copy_on_write_last_block(b)
    assert new is not None and new != blocks[-1] and c._slot_blocks[b][-1] == new
    after = c.read_dense(1, b, 32)
    assert all(torch.equal(x, y) for x, y in zip(before, after))
    # writing into the private copy leaves the shared original untouched
    k = torch.randn(1, hkv, 1, d, generator=g, device=DEV).half()
    c.write_prefill(1, k, k, slot=b, positions=torch.tensor([31], device=DEV))
    assert torch.equal(c.read_dense(1, a, 32)[0], before[0])


@pytest.mark.parametrize("v_quant", ["int8", "lloydmax3"])
def test_compaction_keeps_every_read(v_quant):
    g = torch.Generator(device=DEV).manual_seed(3)
    hq, hkv, d, bs = 8, 2, 128, 16
    c = PagedKVCache(2, 6, hkv, 256, d, device=DEV, block_size=bs, v_quant=v_quant, num_blocks=64)
    slots = [c.alloc() for _ in range(6)]
    lens = [100, 37, 200, 64, 150, 90]
    c.ensure_capacity(slots, lens)
    for layer in range(2):
        for s, n in zip(slots, lens):
            k = torch.randn(1, hkv, n, d, generator=g, device=DEV).half()
            c.write_prefill(layer, k, torch.randn_like(k), slot=s)
    c.store_prefix(list(range(64)), slots[3])
    for s in (slots[0], slots[2]):                                   # free holes in the middle of the pool
        c.free(s)
    live = [slots[i] for i in (1, 3, 4, 5)]
    live_lens = [lens[i] for i in (1, 3, 4, 5)]
    q = torch.randn(len(live), hq, 1, d, generator=g, device=DEV).half()
    before = c.decode_attn(1, q, live, [n - 1 for n in live_lens], scale=0.1)
    reads = [c.read_dense(0, s, n) for s, n in zip(live, live_lens)]
    moves = c.defragment()
    assert moves and max(b for s in live for b in c._slot_blocks[s]) < c.used_blocks
    assert set(c._block_refcount) == set(range(c.used_blocks))
    after = c.decode_attn(1, q, live, [n - 1 for n in live_lens], scale=0.1)
    assert torch.equal(before, after)
    for (k0, v0), s, n in zip(reads, live, live_lens):
        k1, v1 = c.read_dense(0, s, n)
        assert torch.equal(k0, k1) and torch.equal(v0, v1)
    assert c.lookup_prefix(list(range(64)))[0] == 64
