"""CPU oracle for the quantized paged KV-cache hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports, calls or
links this module.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` use it, and only to check or time results.

This is a numpy restatement of what the reference (jajmangold/superl8-serve)
does on its quantized paged-KV path.  The reference's arithmetic lives in the
un-vendored ``superl8`` package, so its exact rounding choices are not
available; every place where this oracle has to *choose* an operation order or
a rounding rule is marked "CHOICE" and the GPU kernels implement the same
choice.  Each function cites the reference file:line whose behaviour it
restates.

Conventions (all from ``superl8serve/engine/kv_cache.py``):
  * cache tensors are per-layer views ``[N, Hkv, bs, D]`` (int8) and
    ``[N, Hkv, bs]`` (fp32 scales) -- kv_cache.py:484-512;
  * a flat slot ``s = block*bs + pos % bs`` maps to storage row
    ``(block*Hkv + h)*bs + s % bs`` -- kv_cache.py:570-585;
  * K is Hadamard-rotated before quantization, V is not --
    kv_cache.py:587-604, 1286-1298.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

F32 = np.float32
F16 = np.float16

# ---------------------------------------------------------------------------
# Hadamard rotation
# ---------------------------------------------------------------------------


def hadamard_matrix(d: int) -> np.ndarray:
    """Normalized Sylvester Hadamard ``H_d / sqrt(d)`` in float64.

    The reference restates ``rotate_last(x) = (x.float() @ hadamard_matrix(d))
    .to(x.dtype)`` (superl8serve/dist/pipeline.py:51-59) and relies on it being
    an involution (kv_cache.py:274-278), which fixes the normalized,
    symmetric Sylvester form."""
    if d < 1 or d & (d - 1):
        raise ValueError("head_dim must be a power of two")
    h = np.ones((1, 1))
    while h.shape[0] < d:
        h = np.block([[h, h], [h, -h]])
    return h / math.sqrt(d)


def rotate_norm_const(d: int) -> np.float32:
    """CHOICE: the 1/sqrt(D) normalization is one fp32 multiply by
    ``float32(1/sqrt(D))`` (computed in float64, rounded once)."""
    return F32(1.0 / math.sqrt(d))


def fwht_f32(x: np.ndarray) -> np.ndarray:
    """Unnormalized Walsh-Hadamard transform over the last axis in float32.

    CHOICE (fixed op order, matched by the GPU kernels): stages h = 1, 2, 4, ...,
    D/2; at each stage the pair (i, i+h) with bit h of i clear becomes
    ``(x[i] + x[i+h], x[i] - x[i+h])``, each a single IEEE fp32 add/sub."""
    x = np.asarray(x, dtype=F32)
    d = x.shape[-1]
    lead = x.shape[:-1]
    y = x.reshape(-1, d).copy()
    h = 1
    while h < d:
        y = y.reshape(-1, d // (2 * h), 2, h)
        a = y[:, :, 0, :]
        b = y[:, :, 1, :]
        y = np.stack([a + b, a - b], axis=2).reshape(-1, d)
        h *= 2
    return y.reshape(*lead, d)


def rotate_last(x: np.ndarray) -> np.ndarray:
    """``rotate_last`` of the reference (dist/pipeline.py:51-59, used at
    kv_cache.py:597,1272,1297): rotate in fp32, return in the input dtype.

    CHOICE: fp32 FWHT (``fwht_f32``), one fp32 multiply by
    ``rotate_norm_const(D)``, then a single round-to-nearest-even cast."""
    x = np.asarray(x)
    out_dtype = x.dtype
    y = fwht_f32(x.astype(F32)) * rotate_norm_const(x.shape[-1])
    return y.astype(out_dtype)


# ---------------------------------------------------------------------------
# Symmetric per-row RTN int8
# ---------------------------------------------------------------------------


def quantize_i8_rowwise(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-row symmetric round-to-nearest int8 with an fp32 scale.

    Restates ``superl8.quantize_i8_rowwise`` as used at kv_cache.py:601 and the
    reference's own RTN restatements (tests/test_layers.py:31-32,
    tests/test_smoke.py:16-17): ``scale = absmax/127``,
    ``q = round(x/scale)`` clamped to [-127, 127].

    CHOICES: absmax is taken over the fp32 value of each element; the scale
    is one correctly rounded fp32 division by 127; ``x/scale`` is one
    correctly rounded fp32 division followed by round-half-even; an all-zero
    row stores scale 0 and codes 0 (dequantizes to exact zeros)."""
    x = np.asarray(x)
    d = x.shape[-1]
    xf = x.astype(F32).reshape(-1, d)
    amax = np.abs(xf).max(axis=-1)
    scale = (amax / F32(127.0)).astype(F32)
    safe = np.where(scale > 0, scale, F32(1.0)).astype(F32)
    q = np.rint(xf / safe[:, None])
    q = np.clip(q, -127, 127)
    q = np.where(scale[:, None] > 0, q, 0).astype(np.int8)
    return q.reshape(x.shape), scale.reshape(x.shape[:-1])


def dequantize_int8_rowwise(q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """``q * scale`` in fp32 (kv_cache.py:1289-1296 before the dtype cast)."""
    return q.astype(F32) * np.asarray(scale, dtype=F32)[..., None]


# ---------------------------------------------------------------------------
# Paged layout
# ---------------------------------------------------------------------------


def flat_rows(slot_mapping: np.ndarray, num_kv_heads: int, block_size: int) -> np.ndarray:
    """[T] flat slots -> [T, Hkv] storage rows ``(block*Hkv + h)*bs + off``
    (kv_cache.py:570-585)."""
    sm = np.asarray(slot_mapping, dtype=np.int64)
    blk = sm // block_size
    off = sm % block_size
    heads = np.arange(num_kv_heads, dtype=np.int64)
    return (blk[:, None] * num_kv_heads + heads[None, :]) * block_size + off[:, None]


def quantize_kv_write_paged(k, v, k_cache, k_scale, v_cache, v_scale, slot_mapping) -> None:
    """In-place paged int8 append (``superl8.quantize_kv_write_paged``, called at
    kv_cache.py:1073-1081 and 1108-1116).

    ``k, v``: fp16 ``[T, Hkv, D]``.  K: ``rotate_last`` then per-(token, head)
    RTN; V: RTN without rotation (kv_cache.py:587-604 documents the K recipe;
    read_dense at kv_cache.py:1286-1298 un-rotates K only).  Rows whose slot is
    negative are skipped (CHOICE; the reference never passes one)."""
    k = np.asarray(k, dtype=F16)
    v = np.asarray(v, dtype=F16)
    t, hkv, d = k.shape
    bs = k_cache.shape[2]
    sm = np.asarray(slot_mapping, dtype=np.int64)
    keep = sm >= 0
    kq, ks = quantize_i8_rowwise(rotate_last(k))
    vq, vs = quantize_i8_rowwise(v)
    rows = flat_rows(sm[keep], hkv, bs).reshape(-1)
    k_cache.reshape(-1, d)[rows] = kq[keep].reshape(-1, d)
    k_scale.reshape(-1)[rows] = ks[keep].reshape(-1)
    v_cache.reshape(-1, d)[rows] = vq[keep].reshape(-1, d)
    v_scale.reshape(-1)[rows] = vs[keep].reshape(-1)


# ---------------------------------------------------------------------------
# K8V3: 3-bit Lloyd-Max V codec
# ---------------------------------------------------------------------------

# Max (1960), "Quantizing for minimum distortion", 8-level table for N(0,1):
# output levels to four decimals.  The codebook actually used is the converged
# Lloyd iteration below (pinned against this table by the tests).
MAX_1960_GAUSS_8LEVEL = (0.2451, 0.7560, 1.3440, 2.1520)


def lloyd_max_gaussian_levels(levels: int = 8, iters: int = 2000) -> np.ndarray:
    """Lloyd's algorithm for the minimum-MSE ``levels``-point quantizer of a
    standard normal, in float64, from uniform initial levels.  Centroid of an
    interval (a, b) of N(0,1) is ``(phi(a) - phi(b)) / (Phi(b) - Phi(a))``."""
    from math import erf, exp, pi, sqrt

    def phi(x):
        return 0.0 if math.isinf(x) else exp(-0.5 * x * x) / sqrt(2 * pi)

    def cdf(x):
        if math.isinf(x):
            return 1.0 if x > 0 else 0.0
        return 0.5 * (1.0 + erf(x / sqrt(2)))

    c = np.linspace(-2.0, 2.0, levels)
    for _ in range(iters):
        t = np.concatenate([[-math.inf], 0.5 * (c[1:] + c[:-1]), [math.inf]])
        new = np.array([(phi(t[i]) - phi(t[i + 1])) / (cdf(t[i + 1]) - cdf(t[i])) for i in range(levels)])
        if np.max(np.abs(new - c)) < 1e-15:
            c = new
            break
        c = new
    return c


def gaussian_codebook(bits: int = 3, block_size: int = 128) -> np.ndarray:
    """fp32 ``[2**bits]`` ascending codebook for unit-L2-norm blocks of
    ``block_size`` elements: the N(0,1) Lloyd-Max levels divided by
    ``sqrt(block_size)`` (each coordinate of a random unit vector in R^n is
    ~N(0, 1/n)).  Restates ``superl8.quant.lloydmax.gaussian_codebook`` as
    consumed at kv_cache.py:502-507 (CHOICE: values are unpinned upstream)."""
    if bits != 3:
        raise ValueError("only the 3-bit (8-level) codebook is defined")
    return (lloyd_max_gaussian_levels(8) / math.sqrt(block_size)).astype(F32)


def l2_norm_blocks(x: np.ndarray, block_size: int) -> np.ndarray:
    """Per-block fp32 L2 norm over the last axis.

    CHOICE (fixed reduction order, matched by the GPU): squares in fp32 (exact
    for fp16 inputs), then a pairwise tree over neighbours: repeatedly add
    each even-indexed partial sum to the odd one after it
    (``s[0::2] + s[1::2]``) until one element is left, then a correctly
    rounded fp32 sqrt."""
    xf = np.asarray(x, dtype=F32)
    d = xf.shape[-1]
    s = (xf * xf).reshape(*xf.shape[:-1], d // block_size, block_size)
    while s.shape[-1] > 1:
        s = s[..., 0::2] + s[..., 1::2]
    return np.sqrt(s[..., 0]).astype(F32)


def quantize_lloydmax(v: np.ndarray, codebook: np.ndarray, block_size: int = 128):
    """3-bit Lloyd-Max V quantizer (kv_cache.py:606-626, ``quantize_lloydmax``).

    Returns ``(codes uint8 [..., D], norms fp32 [..., D/block])``.
    CHOICES: ``u = v / norm`` is one correctly rounded fp32 division (u = 0
    where norm == 0); the code is the first index minimizing
    ``|u - codebook[j]|`` computed in fp32."""
    vf = np.asarray(v, dtype=F32)
    d = vf.shape[-1]
    nb = d // block_size
    norms = l2_norm_blocks(vf, block_size)
    blocks = vf.reshape(*vf.shape[:-1], nb, block_size)
    safe = np.where(norms > 0, norms, F32(1.0)).astype(F32)
    u = (blocks / safe[..., None]).astype(F32)
    u = np.where(norms[..., None] > 0, u, F32(0.0)).astype(F32)
    cb = np.asarray(codebook, dtype=F32)
    dist = np.abs(u[..., None] - cb).astype(F32)
    codes = np.argmin(dist, axis=-1).astype(np.uint8)
    return codes.reshape(vf.shape), norms


def pack_indices_lowbit(codes: np.ndarray, bits: int = 3) -> np.ndarray:
    """Bit-plane packing of 3-bit codes into int32 words, ``D*3/32`` per row
    (``pack_indices_lowbit``, kv_cache.py:623; "bit-plane" per
    docs/k8v3-qwen38-tq34s-wiring.md:33-34).

    CHOICE: for element group g (elements 32g..32g+31) word ``3g + b`` holds bit
    b of each code, element 32g+i at bit i (LSB first)."""
    if bits != 3:
        raise ValueError("only 3-bit packing is defined")
    c = np.asarray(codes, dtype=np.uint32)
    d = c.shape[-1]
    g = c.reshape(*c.shape[:-1], d // 32, 32)
    shifts = np.arange(32, dtype=np.uint32)
    words = []
    for b in range(3):
        plane = ((g >> np.uint32(b)) & np.uint32(1)) << shifts
        words.append(np.bitwise_or.reduce(plane, axis=-1))
    w = np.stack(words, axis=-1).astype(np.uint32)
    return w.reshape(*c.shape[:-1], d // 32 * 3).view(np.int32)


def unpack_indices_lowbit(packed: np.ndarray, bits: int, d: int) -> np.ndarray:
    """Inverse of ``pack_indices_lowbit`` (kv_cache.py:662)."""
    if bits != 3:
        raise ValueError("only 3-bit packing is defined")
    w = np.asarray(packed).view(np.uint32).reshape(*np.shape(packed)[:-1], d // 32, 3)
    shifts = np.arange(32, dtype=np.uint32)
    codes = np.zeros((*w.shape[:-1], 32), dtype=np.uint32)
    for b in range(3):
        codes |= ((w[..., b, None] >> shifts) & np.uint32(1)) << np.uint32(b)
    return codes.reshape(*w.shape[:-2], d).astype(np.uint8)


def dequantize_lloydmax(codes, norms, codebook, block_size: int = 128) -> np.ndarray:
    """``codebook[code] * norm`` in fp32 (kv_cache.py:663-669)."""
    c = np.asarray(codes)
    d = c.shape[-1]
    cb = np.asarray(codebook, dtype=F32)
    vals = cb[c.astype(np.int64)].reshape(*c.shape[:-1], d // block_size, block_size)
    return (vals * np.asarray(norms, dtype=F32)[..., None]).reshape(c.shape).astype(F32)


def k8v3_write_paged(k, v, k_cache, k_scale, v_packed, v_norm, codebook, slot_mapping, lloyd_block=128) -> None:
    """In-place K8V3 append: K exactly as the int8 path (kv_cache.py:587-604),
    V through the Lloyd-Max codec and bit-plane packing (kv_cache.py:606-626),
    scattered at the same storage rows."""
    k = np.asarray(k, dtype=F16)
    v = np.asarray(v, dtype=F16)
    t, hkv, d = k.shape
    bs = k_cache.shape[2]
    sm = np.asarray(slot_mapping, dtype=np.int64)
    keep = sm >= 0
    kq, ks = quantize_i8_rowwise(rotate_last(k))
    codes, norms = quantize_lloydmax(v, codebook, lloyd_block)
    packed = pack_indices_lowbit(codes, 3)
    rows = flat_rows(sm[keep], hkv, bs).reshape(-1)
    k_cache.reshape(-1, d)[rows] = kq[keep].reshape(-1, d)
    k_scale.reshape(-1)[rows] = ks[keep].reshape(-1)
    v_packed.reshape(-1, packed.shape[-1])[rows] = packed[keep].reshape(-1, packed.shape[-1])
    v_norm.reshape(-1, norms.shape[-1])[rows] = norms[keep].reshape(-1, norms.shape[-1])


# ---------------------------------------------------------------------------
# Readers: the reference's dense dequant, and the exact (fp64) dequant
# ---------------------------------------------------------------------------


def gather_rows(block_row: np.ndarray, num_kv_heads: int, block_size: int, length: int, start: int = 0):
    """Storage rows ``[n, Hkv]`` of positions ``start..length-1`` of a sequence
    whose block list is ``block_row`` (kv_cache.py:1247-1254)."""
    pos = np.arange(start, length, dtype=np.int64)
    blk = np.asarray(block_row, dtype=np.int64)[pos // block_size]
    off = pos % block_size
    heads = np.arange(num_kv_heads, dtype=np.int64)
    return (blk[:, None] * num_kv_heads + heads[None, :]) * block_size + off[:, None]


@dataclass
class LayerCache:
    """One layer's view of the cache (kv_cache.py:484-512)."""

    k_cache: np.ndarray  # int8 [N, Hkv, bs, D]
    k_scale: np.ndarray  # fp32 [N, Hkv, bs]
    v_cache: np.ndarray | None = None  # int8 [N, Hkv, bs, D]
    v_scale: np.ndarray | None = None  # fp32 [N, Hkv, bs]
    v_packed: np.ndarray | None = None  # int32 [N, Hkv, bs, D*3/32]
    v_norm: np.ndarray | None = None  # fp32 [N, Hkv, bs, D/128]
    v_codebook: np.ndarray | None = None  # fp32 [8]
    lloyd_block: int = 128

    @property
    def num_kv_heads(self):
        return self.k_cache.shape[1]

    @property
    def block_size(self):
        return self.k_cache.shape[2]

    @property
    def head_dim(self):
        return self.k_cache.shape[3]

    @property
    def is_k8v3(self):
        return self.v_packed is not None


def read_dense(layer: LayerCache, block_row, length: int, *, window: int | None = None, dtype=F16):
    """The reference's pure-torch dequant reader (kv_cache.py:1233-1299):
    ``K = rotate_last((k_i8 * s_k).to(dtype))``, ``V = (v_i8 * s_v).to(dtype)``
    (int8) or ``codebook[code]*norm`` (k8v3).  Returns ``[1, Hkv, n, D]`` twice."""
    start = max(0, length - window) if window is not None else 0
    hkv, bs, d = layer.num_kv_heads, layer.block_size, layer.head_dim
    rows = gather_rows(block_row, hkv, bs, length, start)  # [n, Hkv]
    kq = layer.k_cache.reshape(-1, d)[rows]
    ks = layer.k_scale.reshape(-1)[rows]
    k = rotate_last((kq.astype(F32) * ks[..., None]).astype(dtype))
    if layer.is_k8v3:
        codes = unpack_indices_lowbit(layer.v_packed.reshape(-1, layer.v_packed.shape[-1])[rows], 3, d)
        norms = layer.v_norm.reshape(-1, layer.v_norm.shape[-1])[rows]
        v = dequantize_lloydmax(codes, norms, layer.v_codebook, layer.lloyd_block).astype(dtype)
    else:
        vq = layer.v_cache.reshape(-1, d)[rows]
        vs = layer.v_scale.reshape(-1)[rows]
        v = (vq.astype(F32) * vs[..., None]).astype(dtype)
    return k.transpose(1, 0, 2)[None], v.transpose(1, 0, 2)[None]


def exact_kv(layer: LayerCache, block_row, length: int):
    """float64 K, V ``[Hkv, n, D]`` of one sequence with no intermediate
    rounding: ``K = H (k_i8 * s_k)``, ``V = v_i8 * s_v`` (or the Lloyd-Max
    dequant).  This is the value the reference's dense reader approximates."""
    hkv, bs, d = layer.num_kv_heads, layer.block_size, layer.head_dim
    rows = gather_rows(block_row, hkv, bs, length)
    kq = layer.k_cache.reshape(-1, d)[rows].astype(np.float64)
    ks = layer.k_scale.reshape(-1)[rows].astype(np.float64)
    k = (kq * ks[..., None]) @ hadamard_matrix(d)
    if layer.is_k8v3:
        codes = unpack_indices_lowbit(layer.v_packed.reshape(-1, layer.v_packed.shape[-1])[rows], 3, d)
        norms = layer.v_norm.reshape(-1, layer.v_norm.shape[-1])[rows].astype(np.float64)
        cb = np.asarray(layer.v_codebook, dtype=np.float64)
        nb = d // layer.lloyd_block
        v = (cb[codes.astype(np.int64)].reshape(*codes.shape[:-1], nb, layer.lloyd_block) * norms[..., None]).reshape(codes.shape)
    else:
        vq = layer.v_cache.reshape(-1, d)[rows].astype(np.float64)
        vs = layer.v_scale.reshape(-1)[rows].astype(np.float64)
        v = vq * vs[..., None]
    return k.transpose(1, 0, 2), v.transpose(1, 0, 2)


# ---------------------------------------------------------------------------
# Attention oracles (float64)
# ---------------------------------------------------------------------------


def _softmax_attend(q, k, v, scale, visible=None):
    """q [R, D], k/v [n, D] float64 -> [R, D]."""
    s = (q @ k.T) * scale
    if visible is not None:
        s = np.where(visible, s, -np.inf)
    m = s.max(axis=-1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    p = np.exp(s - m)
    if visible is not None:
        p = np.where(visible, p, 0.0)
    den = p.sum(axis=-1, keepdims=True)
    out = (p @ v) / np.where(den > 0, den, 1.0)
    return out


def paged_decode(q, layer: LayerCache, block_table, context_lens, scale, window=None) -> np.ndarray:
    """Ragged-batch GQA decode over the paged cache in float64
    (``attn_paged_decode_cached`` / ``attn_paged_decode_k8v3`` semantics,
    kv_cache.py:1167-1201): row b attends its first ``context_lens[b]``
    tokens; q head h reads KV head ``h // (Hq/Hkv)`` (gqa_attention.py:208-212).
    ``window``: only the last ``window`` of them, positions
    ``[max(0, n - window), n)`` -- the reference's sliding-window decode reads
    that range back dense (``first = max(0, length - window)`` in
    kv_cache.py:1233-1299, called at gqa_attention.py:191-196).

    q: ``[B, Hq, D]`` (any float) -> float64 ``[B, Hq, D]``."""
    q = np.asarray(q, dtype=np.float64)
    b_, hq, d = q.shape
    hkv = layer.num_kv_heads
    g = hq // hkv
    out = np.zeros((b_, hq, d))
    for b in range(b_):
        n = int(context_lens[b])
        if n <= 0:
            continue
        k, v = exact_kv(layer, block_table[b], n)
        if window is not None:
            first = max(0, n - int(window))
            k, v = k[:, first:], v[:, first:]
        for h in range(hkv):
            out[b, h * g:(h + 1) * g] = _softmax_attend(q[b, h * g:(h + 1) * g], k[h], v[h], scale)
    return out


def paged_verify(q, layer: LayerCache, block_table, prefix_lens, scale, *, query_lens=None, tree_mask=None,
                 window=None, fresh_drafts=None) -> np.ndarray:
    """Multi-query verify attention over the paged cache in float64.

    Query s of row b sees every prefix key ``j < prefix_lens[b]`` plus draft key
    ``prefix_lens[b] + i`` when bit i of ``tree_mask[b, s]`` is set (its
    ancestors and itself).  With ``tree_mask`` None the drafts form a chain and
    query s sees drafts 0..s -- exactly the reference's chain verify, which runs
    S decode steps with context ``L + t + 1`` (gqa_attention.py:259-277), and
    the bottom-right-aligned causal chunk of chunked prefill
    (gqa_attention.py:117-126, gated_gqa_attention.py:167-185).
    Queries ``s >= query_lens[b]`` produce zeros.  ``window``: a sliding-window
    layer sees only the last ``window`` prefix keys, ``[max(0, p - window), p)``,
    plus its drafts -- the reference reads that prefix window back dense and
    appends the drafts (gqa_attention.py:305-314 with kv_cache.py:1233-1299).
    ``fresh_drafts`` = (k, v) fp16 ``[B, S, Hkv, D]``: the drafts enter with
    these values instead of their cache rows -- the reference's window verify
    concatenates the layer's fresh fp16 draft K / V to the dequantized prefix
    window (gqa_attention.py:298-303).

    q: ``[B, Hq, S, D]`` -> float64 ``[B, Hq, S, D]``."""
    q = np.asarray(q, dtype=np.float64)
    b_, hq, s_, d = q.shape
    hkv = layer.num_kv_heads
    g = hq // hkv
    out = np.zeros_like(q)
    for b in range(b_):
        nq = s_ if query_lens is None else int(query_lens[b])
        p = int(prefix_lens[b])
        if nq <= 0:
            continue
        total = p + nq
        k, v = exact_kv(layer, block_table[b], total)
        if fresh_drafts is not None:
            k[:, p:] = np.asarray(fresh_drafts[0], dtype=np.float64)[b, :nq].transpose(1, 0, 2)
            v[:, p:] = np.asarray(fresh_drafts[1], dtype=np.float64)[b, :nq].transpose(1, 0, 2)
        j = np.arange(total)
        vis = np.zeros((nq, total), dtype=bool)
        for s in range(nq):
            if tree_mask is None:
                vis[s] = j <= p + s
            else:
                bits = int(np.asarray(tree_mask)[b, s]) & ((1 << 64) - 1)
                draft = np.array([(bits >> i) & 1 for i in range(nq)], dtype=bool)
                vis[s] = (j < p) | np.concatenate([np.zeros(p, dtype=bool), draft])
        if window is not None:
            vis &= (j >= max(0, p - int(window)))[None, :]
        for h in range(hkv):
            for gg in range(g):
                hh = h * g + gg
                out[b, hh, :nq] = _softmax_attend(q[b, hh, :nq], k[h], v[h], scale, vis)
    return out


def dense_varlen_attention(q, k, v, cu_q, cu_k, scale, causal=True, window_left=None) -> np.ndarray:
    """Prefill attention over fresh K / V in float64 (the role of
    ``superl8.attn_int8_varlen``, gqa_attention.py:81-104): q ``[Tq, Hq, D]``,
    k, v ``[Tk, Hkv, D]``; sequence b = query tokens ``cu_q[b] ..``, key tokens
    ``cu_k[b] ..``; causal is bottom-right aligned (query s sees keys
    ``j <= s + nk - nq``; a query that sees none gives zeros).  The reference's
    kernel is absent (the superl8 package), so this is the exact attention the
    reference's int8 kernel approximates.  CHOICE: ``window_left >= 1``
    (causal only) lets query i (aligned bottom-right) see its last
    ``window_left`` keys, ``i - window_left + 1 .. i`` -- the window the
    reference's decode side attends for the same layer (``_window`` keeps the
    last ``window_left`` keys, gqa_attention.py:150-154; ``read_dense(window=)``
    starts at ``length - window``, kv_cache.py:1251), so a token sees the same
    keys at prefill and at decode.  Returns float64 ``[Tq, Hq, D]``."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    hq, hkv = q.shape[1], k.shape[1]
    g = hq // hkv
    out = np.zeros_like(q)
    for b in range(len(cu_q) - 1):
        qs, qe, ks_, ke = int(cu_q[b]), int(cu_q[b + 1]), int(cu_k[b]), int(cu_k[b + 1])
        nq, nk = qe - qs, ke - ks_
        if nq <= 0 or nk <= 0:
            continue
        j = np.arange(nk)
        vis = (j[None, :] <= np.arange(nq)[:, None] + nk - nq) if causal else np.ones((nq, nk), bool)
        if window_left is not None:
            if int(window_left) < 1:
                raise ValueError("window_left must be >= 1")
            vis &= j[None, :] > np.arange(nq)[:, None] + nk - nq - int(window_left)
        live = vis.any(axis=1)
        for h in range(hq):
            kv = h // g
            o = _softmax_attend(q[qs:qe, h][live], k[ks_:ke, kv], v[ks_:ke, kv], scale, vis[live])
            out[np.arange(qs, qe)[live], h] = o
    return out


# ---------------------------------------------------------------------------
# Block copy (copy-on-write / compaction)
# ---------------------------------------------------------------------------


def copy_blocks(tensors: list[np.ndarray], src: list[int], dst: list[int]) -> None:
    """Byte copy of whole blocks: for every tensor ``[NL, N, ...]`` set
    ``t[:, dst[i]] = t[:, src[i]]``.  The reference has no raw block copy; its
    prefix sharing is refcounted (kv_cache.py:751-755) and its compaction is a
    lossy dequant/requant (kv_cache.py:199-313).  Copying the quantized bytes
    is the closed form that leaves every ``read_dense`` unchanged."""
    if len(set(src) & set(dst)):
        raise ValueError("source and destination blocks overlap")
    for t in tensors:
        t[:, list(dst)] = t[:, list(src)]


def snapkv_scores(q, k, num_heads: int, num_kv_heads: int, scale: float | None = None) -> np.ndarray:
    """SnapKV ranking in float64 (``KVEviction.snapkv_selection``,
    kv_cache.py:149-163): q ``[num_heads, D]``, k ``[Hkv, S, D]``; q head h
    reads KV head ``h // (num_heads / num_kv_heads)`` (the reference's
    expand + reshape repeat); ``softmax_t(q_h . k_t * scale)`` averaged over
    the heads, ``scale`` 1/sqrt(D) by default."""
    q = np.asarray(q, dtype=np.float64).reshape(num_heads, -1)
    k = np.asarray(k, dtype=np.float64)
    if k.ndim == 4:
        k = k[0]
    g = num_heads // num_kv_heads
    d = q.shape[1]
    sc = 1.0 / math.sqrt(d) if scale is None else scale
    logits = np.einsum("hd,hsd->hs", q, np.repeat(k, g, axis=0)) * sc
    logits -= logits.max(axis=1, keepdims=True)
    p = np.exp(logits)
    return (p / p.sum(axis=1, keepdims=True)).mean(axis=0)


def snapkv_scores_paged(q, layer: "LayerCache", block_row, length: int, num_heads: int) -> np.ndarray:
    """``snapkv_scores`` over a sequence's exactly dequantized cached K
    (``H (k_i8 * s_k)`` in float64, as ``exact_kv``; only K is read)."""
    hkv, bs, d = layer.num_kv_heads, layer.block_size, layer.head_dim
    rows = gather_rows(block_row, hkv, bs, length)
    kq = layer.k_cache.reshape(-1, d)[rows].astype(np.float64)
    ks = layer.k_scale.reshape(-1)[rows].astype(np.float64)
    k = ((kq * ks[..., None]) @ hadamard_matrix(d)).transpose(1, 0, 2)
    return snapkv_scores(q, k, num_heads, hkv)


def snapkv_select(scores, budget: int) -> list[int]:
    """Sorted positions of the ``budget`` largest scores (all of them when
    there are at most ``budget``; kv_cache.py:145-147, 165-166).  CHOICE:
    equal scores keep the lower position (the reference leaves ties to
    ``torch.topk``)."""
    s = np.asarray(scores, dtype=np.float64)
    if s.size <= budget:
        return list(range(s.size))
    order = np.lexsort((np.arange(s.size), -s))
    return sorted(int(i) for i in order[:budget])


def gather_slots(tensors: list[np.ndarray], src: list[int], dst: list[int]) -> None:
    """Keep-list compaction as a byte move: for every tensor ``[NL, N, Hkv,
    bs, ...]`` the rows of flat slot ``src[j]`` go to flat slot ``dst[j]``
    in every layer and head (the closed form of moving kept tokens without
    re-quantizing them; the reference's KVEviction.compact re-quantizes,
    kv_cache.py:249-296)."""
    if set(src) & set(dst):
        raise ValueError("source and destination slots overlap")
    for t in tensors:
        bs = t.shape[3]
        sb, so = np.asarray(src) // bs, np.asarray(src) % bs
        db, do = np.asarray(dst) // bs, np.asarray(dst) % bs
        t[:, db, :, do] = t[:, sb, :, so]


def block_bytes(num_kv_heads, block_size, head_dim, v_quant="int8", lloyd_block=128) -> int:
    """HBM bytes of one block per layer (kv_cache.py:98-120)."""
    n = num_kv_heads * block_size
    if v_quant == "lloydmax3":
        return n * (head_dim + 4) + n * (head_dim * 3 // 8 + head_dim // lloyd_block * 4)
    return 2 * n * head_dim + 2 * n * 4


# ---------------------------------------------------------------------------
# Tolerance used for attention outputs
# ---------------------------------------------------------------------------


def attention_errors(out, ref) -> tuple[float, float]:
    """(max scaled abs error, relative RMS error) of ``out`` against ``ref``.

    The abs error is divided by ``max(1, |ref|)`` elementwise: plain absolute
    error where |ref| <= 1, relative error above it, because an fp16 output
    cannot hold more than ~11 significant bits of a large value."""
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    err = np.abs(out - ref)
    mx = float(np.max(err / np.maximum(1.0, np.abs(ref)))) if err.size else 0.0
    den = float(np.sqrt(np.mean(ref * ref))) if ref.size else 0.0
    rel = float(np.sqrt(np.mean((out - ref) ** 2)) / den) if den > 0 else float(np.sqrt(np.mean(err ** 2)))
    return mx, rel


MAX_ABS_TOL = 2e-3
REL_RMS_TOL = 1e-3
