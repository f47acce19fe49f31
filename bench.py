#!/usr/bin/env python3
"""Paged int8 decode-attention + append throughput at Qwen3-8B shapes, batch 64.

Workload (one "step" = one decode step of the whole model's KV path):
  * 36 layers, 32 query heads, 8 KV heads, head_dim 128, block size 256;
  * 64 sequences with context lengths lognormal(median 2048, sigma 0.75),
    clipped to [256, 8192], seed 1; each step appends one token per sequence
    (its position is the last one of the context) and then attends;
  * a pool of 1111 physical blocks per layer (40,000 block-layer slots over 36
    layers), blocks dealt from a seeded permutation (fragmented tables);
  * fp16 K/V/q ~ N(0,1) with 1% (2 of 128) outlier channels scaled 20x;
  * distinct cache storage per layer, so the 256 MB Infinity Cache cannot
    serve one layer's KV to the next.
Each layer runs as one launch that appends the new tokens and attends
(attn_paged_decode_append; cache bytes and outputs identical to the
reference's append-then-decode pair, which --separate-append runs instead).
Inputs are resident in HBM before the timed region.  The 36-layer step is
captured once in a HIP graph and replayed.  Every timed step re-appends at the
same positions, so all steps do identical work.

Prints one JSON line.  `value` = algorithmic bytes of one step / step time.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import platform
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0  # MI355X published HBM3E bandwidth
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X published dense fp16 / bf16 MFMA rate


def roofline_max(hbm_bytes: float, flops: float, sec: float, **extra) -> dict:
    """Roofline of a launch that both streams `hbm_bytes` and does `flops`
    useful work in `sec`: its bound is whichever term takes longer at the
    published peaks, and frac = max(bytes / BW, flops / peak) / sec.  Both
    terms are reported."""
    t_mem = hbm_bytes / (HBM_PEAK_GBPS * 1e9)
    t_mfma = flops / (MFMA_F16_PEAK_TFLOPS * 1e12)
    gbps = hbm_bytes / sec / 1e9
    tflops = flops / sec / 1e12
    hbm_bound = t_mem >= t_mfma
    return {"bound": "hbm" if hbm_bound else "mfma",
            "achieved": round(gbps if hbm_bound else tflops, 2),
            "peak": HBM_PEAK_GBPS if hbm_bound else MFMA_F16_PEAK_TFLOPS,
            "unit": "GB/s" if hbm_bound else "TFLOP/s",
            "frac": round(max(t_mem, t_mfma) / sec, 4),
            "hbm_term": {"bytes": int(hbm_bytes), "gbps": round(gbps, 1), "frac": round(t_mem / sec, 4)},
            "mfma_term": {"flops": int(flops), "tflops": round(tflops, 2), "frac": round(t_mfma / sec, 4)},
            **extra}

NUM_LAYERS = 36
BATCH = 64
HQ, HKV, D, BS = 32, 8, 128, 256
POOL_BLOCKS = 1111
MAX_LEN = 8192
SIGMA = 0.75
SEED = 1
OUTLIER_CH = 2
OUTLIER_SCALE = 20.0
BYTES_PER_TOKEN_HEAD = 2 * D + 8  # int8 K + V + two fp32 scales


def workload_lengths():
    rng = np.random.default_rng(SEED)
    lens = np.clip(np.round(np.exp(rng.normal(math.log(2048), SIGMA, BATCH))), 256, MAX_LEN).astype(np.int64)
    need = (lens + BS - 1) // BS
    perm = rng.permutation(POOL_BLOCKS)
    assert need.sum() <= POOL_BLOCKS
    bt = np.zeros((BATCH, MAX_LEN // BS), dtype=np.int32)
    pos = 0
    for b in range(BATCH):
        bt[b, : need[b]] = perm[pos: pos + need[b]]
        pos += need[b]
    return lens, bt, rng


def step_bytes(lens: np.ndarray) -> dict:
    """Algorithmic HBM bytes of one step (each logical byte counted once)."""
    t = BATCH
    append = t * HKV * D * 2 * 2 + 4 * t + t * HKV * BYTES_PER_TOKEN_HEAD
    blocks = int(((lens + BS - 1) // BS).sum())
    decode = int(lens.sum()) * HKV * BYTES_PER_TOKEN_HEAD + 2 * BATCH * HQ * D * 2 + 4 * blocks + 4 * BATCH
    # the one-launch step reads no slot mapping (the slot comes from the block table, counted in decode)
    fused = append - 4 * t + decode
    return {"append_layer": append, "decode_layer": decode, "fused_layer": fused, "step": NUM_LAYERS * (append + decode)}


def _fp16_outliers(gen, shape, ch, device):
    import torch

    x = torch.randn(shape, generator=gen, device=device, dtype=torch.float32)
    x[..., ch] *= OUTLIER_SCALE
    return x.half()


def build(device, layers: int = NUM_LAYERS, keep_prefix: bool = False):
    """The decode-step workload of `layers` layers (distinct storage each):
    the prefix of every row appended, and per layer the new tokens' K/V and
    q.  `keep_prefix`: also return the appended prefix K/V (fp16, per layer)."""
    import torch

    from superl8_serve_amd import ops

    lens, bt_np, rng = workload_lengths()
    prefix = lens - 1
    # flat slots of every prefix token and of the appended token, per sequence
    pre_slots = np.concatenate([bt_np[b, np.arange(prefix[b]) // BS] * BS + np.arange(prefix[b]) % BS
                                for b in range(BATCH)]).astype(np.int32)
    new_slots = np.array([bt_np[b, prefix[b] // BS] * BS + prefix[b] % BS for b in range(BATCH)], dtype=np.int32)

    shape = (layers, POOL_BLOCKS, HKV, BS, D)
    kc = torch.zeros(shape, dtype=torch.int8, device=device)
    vc = torch.zeros(shape, dtype=torch.int8, device=device)
    ks = torch.ones(shape[:4], dtype=torch.float32, device=device)
    vs = torch.ones(shape[:4], dtype=torch.float32, device=device)
    gen = torch.Generator(device=device)
    gen.manual_seed(SEED)
    pre_sm = torch.from_numpy(pre_slots).to(device)
    chans, kept = [], []
    for layer in range(layers):
        ch = torch.from_numpy(rng.choice(D, OUTLIER_CH, replace=False)).to(device)
        chans.append(ch)
        kp = _fp16_outliers(gen, (pre_slots.size, HKV, D), ch, device)
        vp = _fp16_outliers(gen, (pre_slots.size, HKV, D), ch, device)
        ops.quantize_kv_write_paged(kp, vp, kc[layer], ks[layer], vc[layer], vs[layer], pre_sm)
        if keep_prefix:
            kept.append((kp, vp))
        del kp, vp
    k_new = [_fp16_outliers(gen, (BATCH, HKV, D), chans[l], device) for l in range(layers)]
    v_new = [_fp16_outliers(gen, (BATCH, HKV, D), chans[l], device) for l in range(layers)]
    # q as the attention seam passes it: a [B,1,Hq,D] -> [B,Hq,1,D] transpose view
    q = [_fp16_outliers(gen, (BATCH, 1, HQ, D), chans[l], device).transpose(1, 2) for l in range(layers)]
    torch.cuda.synchronize()
    return {
        "lens": lens, "kc": kc, "vc": vc, "ks": ks, "vs": vs,
        "bt": torch.from_numpy(bt_np).to(device), "bt_np": bt_np,
        "cl": torch.from_numpy(lens.astype(np.int32)).to(device),
        "new_sm": torch.from_numpy(new_slots).to(device), "new_slots": new_slots, "pre_slots": pre_slots,
        "k_new": k_new, "v_new": v_new, "q": q, "prefix": kept,
    }


def decode_layer(w, layer: int, fused: bool, plan=None):
    """One layer of the decode step: append the new token of every row, then
    attend.  fused: one launch (attn_paged_decode_append, reading the step's
    slice plan when one is given); otherwise the reference's two calls
    (quantize_kv_write_paged, attn_paged_decode_cached)."""
    from superl8_serve_amd import ops

    scale = 1.0 / math.sqrt(D)
    if fused:
        return ops.attn_paged_decode_append(
            w["q"][layer], w["k_new"][layer], w["v_new"][layer], w["kc"][layer], w["ks"][layer], w["vc"][layer],
            w["vs"][layer], w["bt"], w["cl"], BS, max_context_len=MAX_LEN, scale=scale, plan=plan)
    ops.quantize_kv_write_paged(w["k_new"][layer], w["v_new"][layer], w["kc"][layer], w["ks"][layer],
                                w["vc"][layer], w["vs"][layer], w["new_sm"])
    return ops.attn_paged_decode_cached(w["q"][layer], w["kc"][layer], w["ks"][layer], w["vc"][layer], w["vs"][layer],
                                        w["bt"], w["cl"], BS, max_context_len=MAX_LEN, scale=scale)


def step_plan(w, adaptive: bool = False):
    """The step's slice plan: one launch, shared by the 36 layers' launches
    (every layer decodes the same rows).  `adaptive`: made into the
    workload's one plan tensor, whose slice bounds follow the last step's
    measured workgroup times (two launches: bounds, then plan)."""
    from superl8_serve_amd import ops

    if not adaptive:
        return ops.attn_paged_decode_plan(w["kc"][0], w["bt"], w["cl"], BS, num_q_heads=HQ, max_context_len=MAX_LEN)
    w["plan"] = ops.attn_paged_decode_plan(w["kc"][0], w["bt"], w["cl"], BS, num_q_heads=HQ, max_context_len=MAX_LEN,
                                           adaptive=True, plan=w.get("plan"))
    return w["plan"]


def make_step(w, fused: bool, planned: bool = True, adaptive: bool = False):
    """The 36-layer step; the fused form starts with the step's plan launch
    when `planned` (adaptive slice bounds when `adaptive`)."""
    outs = [None] * NUM_LAYERS

    def step():
        plan = step_plan(w, adaptive) if fused and planned else None
        for layer in range(NUM_LAYERS):
            outs[layer] = decode_layer(w, layer, fused, plan)
        return outs

    return step


def time_decode_kernel(w, reps: int, fused: bool, planned: bool = True, adaptive: bool = False) -> dict:
    """Average duration of the decode attention kernel (which also combines
    the partials of rows split across workgroups), from HIP events the library
    records on the launch stream around each launch (s8kv_timing_begin/end),
    over `reps` eager passes of the 36
    decode calls (the one-launch step when `fused`: its append rewrites the
    same bytes; an adaptive plan is made again before each pass).  A
    preceding spin kernel keeps the GPU ahead of the host so host launch
    latency never enters an interval."""
    import ctypes

    import torch

    from superl8_serve_amd import _lib, ops

    lib = _lib.load()
    scale = 1.0 / math.sqrt(D)
    plan = step_plan(w, adaptive) if fused and planned else None
    torch.cuda.synchronize()
    torch.cuda._sleep(int(2e8))  # ~0.1 s of GPU spin while the host enqueues
    _lib.check(lib.s8kv_timing_begin(), "s8kv_timing_begin")
    for _ in range(reps):
        if fused and planned and adaptive:
            plan = step_plan(w, True)
        for layer in range(NUM_LAYERS):
            if fused:
                decode_layer(w, layer, True, plan)
            else:
                ops.attn_paged_decode_cached(w["q"][layer], w["kc"][layer], w["ks"][layer], w["vc"][layer],
                                             w["vs"][layer], w["bt"], w["cl"], BS, max_context_len=MAX_LEN,
                                             scale=scale)
    n = ctypes.c_int(0)
    dk, mk = ctypes.c_double(0.0), ctypes.c_double(0.0)
    _lib.check(lib.s8kv_timing_end(ctypes.byref(n), ctypes.byref(dk), ctypes.byref(mk)), "s8kv_timing_end")
    torch.cuda.synchronize()
    launches = max(n.value, 1)
    return {"decode_s": dk.value * 1e-3 / launches, "launches": n.value}


def decode_tiles(lens: np.ndarray, bt_np: np.ndarray, slices_per_head: int) -> np.ndarray:
    """First storage row of every 32-token tile the decode step reads, one
    list per KV head (rows concatenated), each cut into `slices_per_head`
    equal slices and the slices dealt as the decode kernel deals its
    workgroups (workgroup j * HKV + h takes slice j of head h)."""
    per_head = []
    for h in range(HKV):
        rows = []
        for b in range(BATCH):
            t0 = np.arange(0, int(lens[b]), 32)
            rows.append((bt_np[b, t0 // BS].astype(np.int64) * HKV + h) * BS + t0 % BS)
        per_head.append(np.concatenate(rows))
    out = []
    for j in range(slices_per_head):
        for h in range(HKV):
            n = per_head[h].size
            out.append(per_head[h][n * j // slices_per_head: n * (j + 1) // slices_per_head])
    return np.concatenate(out).astype(np.int32)


def _time_graph(fn, steps: int, warmup: int) -> float:
    """Seconds per replay of a graph holding `fn`'s launches, from HIP events
    around `steps` back-to-back replays."""
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e-3 / max(steps, 1)


def _spin_ahead(warm=None, per_call_s: float = 0.0, warm_s: float = 0.03) -> None:
    """Keep the GPU ahead of the host for an eager timed loop: a ~0.1 s spin
    kernel runs while the host enqueues the timed calls, so host launch
    overhead never opens a gap between them (the start event, recorded
    after the spin, is stamped when the spin ends).  The spin is one wave,
    so the engine clock may fall while it runs: with `warm` (a call of the
    timed workload, ~per_call_s of GPU time) about warm_s of untimed calls
    follow it, so the timed calls start at the clock a busy GPU holds."""
    import torch

    torch.cuda._sleep(int(2e8))
    if warm is not None and per_call_s > 0:
        for i in range(min(4000, max(1, math.ceil(warm_s / per_call_s)))):
            warm(i)


def _timed_warmup(fn, calls: int) -> float:
    """Run `calls` untimed calls fn(i) and return their GPU seconds per call
    (HIP events; the first timing pass of a process warms the clocks too)."""
    import torch

    st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    st.record()
    for i in range(calls):
        fn(i)
    en.record()
    torch.cuda.synchronize()
    return st.elapsed_time(en) * 1e-3 / max(calls, 1)


def read_ceiling(w, steps: int) -> dict:
    """What a read-only kernel reaches on the decode step's bytes, with the
    step's shape: 36 launches, one per layer's storage, in a graph.
      tiles : exactly the K/V rows and scales of the decode's 32-token
              tiles (s8kv_probe_read_tiles), for several grid sizes;
      linear: one layer's whole int8 K tensor per launch, contiguous
              (s8kv_probe_read_linear), for several grid sizes.
    GB/s = the probe's own bytes per launch / its average launch time."""
    import torch

    from superl8_serve_amd import _lib

    lib = _lib.load()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    stream = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)  # noqa: E731
    nrows = POOL_BLOCKS * HKV * BS
    sink = torch.zeros(cus * 16, dtype=torch.int32, device="cuda")
    res = {"tiles": {}, "linear": {}}
    for per_cu in (2, 3, 4, 6):
        nwg = cus * per_cu
        tiles = torch.from_numpy(decode_tiles(w["lens"], w["bt_np"], nwg // HKV)).cuda()
        nt = int(tiles.numel())

        def probe(tiles=tiles, nt=nt, nwg=nwg):
            for layer in range(NUM_LAYERS):
                _lib.check(lib.s8kv_probe_read_tiles(
                    w["kc"][layer].data_ptr(), w["ks"][layer].data_ptr(), w["vc"][layer].data_ptr(),
                    w["vs"][layer].data_ptr(), nrows, D, tiles.data_ptr(), nt, nwg, sink.data_ptr(), stream()),
                    "s8kv_probe_read_tiles")

        sec = _time_graph(probe, steps, 2) / NUM_LAYERS
        nbytes = nt * 32 * (2 * D + 8)
        res["tiles"][f"{per_cu}/CU"] = {"gbps": round(nbytes / sec / 1e9, 1), "launch_us": round(sec * 1e6, 2),
                                        "bytes": nbytes}
    for per_cu in (4, 8):
        nwg = cus * per_cu
        nbytes = w["kc"][0].numel()

        def probe(nwg=nwg, nbytes=nbytes):
            for layer in range(NUM_LAYERS):
                _lib.check(lib.s8kv_probe_read_linear(w["kc"][layer].data_ptr(), nbytes, nwg, sink.data_ptr(),
                                                      stream()), "s8kv_probe_read_linear")

        sec = _time_graph(probe, steps, 2) / NUM_LAYERS
        res["linear"][f"{per_cu}/CU"] = {"gbps": round(nbytes / sec / 1e9, 1), "launch_us": round(sec * 1e6, 2),
                                         "bytes": nbytes}
    res["tiles_best_gbps"] = max(v["gbps"] for v in res["tiles"].values())
    res["linear_best_gbps"] = max(v["gbps"] for v in res["linear"].values())
    return res


TRACE_WORDS = 16  # per-workgroup record of the decode trace build


def trace_decode(steps: int, warmup: int, adaptive: bool = False) -> dict:
    """Per-launch breakdown of the one-launch decode step from the trace
    build of the library (libsuperl8_kv_trace.so: the same kernels, the decode
    kernel stamping the device's 100 MHz clock at fixed points of each
    workgroup).  The 36-layer step is captured with the trace on (each layer's
    launch writing its own slot), replayed, and the last replay's records are
    summarised: phase times are medians over workgroups and launches, spreads
    are per launch (then the median over launches), all in us from the
    launch's first workgroup start."""
    import ctypes

    import torch

    from superl8_serve_amd import _lib

    lib = _lib.load()
    fn = lib.s8kv_decode_trace_set
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64]
    w = build("cuda")
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    stride = cus * 8 * TRACE_WORDS  # the largest grid the decode launches (8 workgroups per CU)
    buf = torch.zeros(NUM_LAYERS * stride, dtype=torch.int64, device="cuda")
    _lib.check(fn(buf.data_ptr(), stride, NUM_LAYERS), "s8kv_decode_trace_set")
    step = make_step(w, True, True, adaptive)
    sec = _time_graph(step, steps, warmup)
    _lib.check(fn(None, 0, 0), "s8kv_decode_trace_set")
    rec = buf.view(NUM_LAYERS, cus * 8, TRACE_WORDS).cpu().numpy().view(np.uint64)
    us = lambda x: x.astype(np.float64) * 0.01  # noqa: E731  (100 MHz ticks)
    med = lambda x: float(np.median(x)) if len(x) else None  # noqa: E731
    phases = {k: [] for k in ("lengths_staged", "first_segment_found", "first_q_and_blocks_loaded",
                              "first_q_published", "first_full_tile_done")}
    per_launch = {k: [] for k in ("span", "tiles_end_min", "tiles_end_median", "tiles_end_p90", "tiles_end_max",
                                  "exit_median", "exit_p90", "exit_max", "balanced_tiles_end")}
    tails = {"whole_row": [], "split_row": [], "split_row_combining": []}
    starts, ends = [], []
    for layer in range(NUM_LAYERS):
        r = rec[layer]
        r = r[(r[:, 9] & np.uint64(1)) == 1]
        t0 = r[:, 0].min()
        rel = lambda c: us(r[:, c] - t0)  # noqa: E731
        starts.append(int(t0))
        ends.append(int(r[:, 7].max()))
        for i, k in enumerate(phases, start=1):
            v = r[:, i]
            phases[k].extend(us(v[v > 0] - r[v > 0, 0]))
        te, ex = rel(6), rel(7)
        per_launch["span"].append(us(r[:, 7].max() - t0))
        for k, q in (("tiles_end_min", 0), ("tiles_end_median", 50), ("tiles_end_p90", 90), ("tiles_end_max", 100)):
            per_launch[k].append(np.percentile(te, q))
        for k, q in (("exit_median", 50), ("exit_p90", 90), ("exit_max", 100)):
            per_launch[k].append(np.percentile(ex, q))
        # finish time if every workgroup kept its measured token rate and
        # the work were spread so that all tile loops end together
        tok = (r[:, 8] & np.uint64(0xFFFFFFFF)).astype(np.float64)
        start_tiles = rel(3)
        rate = tok / np.maximum(te - start_tiles, 1e-3)
        per_launch["balanced_tiles_end"].append(float((tok.sum() + (rate * start_tiles).sum()) / rate.sum()))
        whole = (r[:, 9] >> np.uint64(8)) & np.uint64(1)
        comb = (r[:, 9] >> np.uint64(9)) & np.uint64(1)
        tails["whole_row"].extend(ex[whole == 1] - te[whole == 1])
        tails["split_row"].extend(ex[(whole == 0) & (comb == 0)] - te[(whole == 0) & (comb == 0)])
        tails["split_row_combining"].extend(ex[comb == 1] - te[comb == 1])
    gaps = [us(np.uint64(starts[i + 1] - ends[i])) for i in range(NUM_LAYERS - 1)]
    return {
        "trace": "decode_kernel<128, int8, fused append>, Qwen3-8B batch-64 step, trace build",
        "slice_plan": "adaptive" if adaptive else "fixed split",
        "step_ms_trace_build": round(sec * 1e3, 4),
        "workgroups_per_launch": int(((rec[0][:, 9] & np.uint64(1)) == 1).sum()),
        "prologue_us_from_workgroup_start": {k: round(med(v), 2) for k, v in phases.items()},
        "per_launch_us": {k: round(float(np.median(v)), 2) for k, v in per_launch.items()},
        "tail_us_exit_minus_tiles_end": {k: round(med(v), 2) if len(v) else None for k, v in tails.items()},
        "gap_between_launches_us": round(float(np.median(gaps)), 2),
    }


def cpu_baseline(lens: np.ndarray, bt_np: np.ndarray, layers: int) -> dict:
    """The reference's host path restated in PyTorch-CPU (oracle/cpu_path.py),
    timed on this host's cores over `layers` layers of the same step."""
    import torch

    from oracle import cpu_path

    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        threads = min(threads, int(os.environ["OMP_NUM_THREADS"]))
    torch.set_num_threads(threads)
    gen = torch.Generator().manual_seed(SEED)
    h = cpu_path.hadamard(D)
    nb = int(bt_np.max()) + 1
    kc = torch.zeros((nb, HKV, BS, D), dtype=torch.int8)
    vc = torch.zeros_like(kc)
    ks = torch.ones((nb, HKV, BS))
    vs = torch.ones_like(ks)
    blocks = [[int(x) for x in bt_np[b, : (lens[b] + BS - 1) // BS]] for b in range(BATCH)]
    new_sm = torch.tensor([blocks[b][(lens[b] - 1) // BS] * BS + (lens[b] - 1) % BS for b in range(BATCH)],
                          dtype=torch.int32)
    k_new = torch.randn((BATCH, HKV, D), generator=gen).half()
    v_new = torch.randn((BATCH, HKV, D), generator=gen).half()
    q = torch.randn((BATCH, HQ, D), generator=gen).half()
    t0 = time.perf_counter()
    for _ in range(layers):
        cpu_path.append(k_new, v_new, kc, ks, vc, vs, new_sm, h)
        cpu_path.decode(q, kc, ks, vc, vs, blocks, lens.tolist(), 1.0 / math.sqrt(D), h)
    dt = time.perf_counter() - t0
    b = step_bytes(lens)
    gbps = layers * (b["append_layer"] + b["decode_layer"]) / dt / 1e9
    model = ""
    try:
        out = subprocess.run(["lscpu"], stdout=subprocess.PIPE, text=True, timeout=10).stdout
        model = next((l.split(":", 1)[1].strip() for l in out.splitlines() if l.startswith("Model name")), "")
    except Exception:
        pass
    return {"value": round(gbps, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{layers} of 36 layers of the same batch-64 step (append + per-slot dense decode), "
                      f"{dt:.2f} s on {threads} threads of {model or platform.processor()}"}


def calibrate_copy(mib: int) -> None:
    """Plain copy of a known size with s8kv_copy_blocks (PMC calibration run)."""
    import torch

    from superl8_serve_amd import ops

    t = torch.zeros((1, 8, mib * 1024 * 1024 // 32), dtype=torch.int32, device="cuda")  # 8 blocks, mib MiB
    torch.cuda.synchronize()
    for _ in range(3):
        ops.copy_blocks([t], [0, 1, 2, 3], [4, 5, 6, 7])
    torch.cuda.synchronize()
    moved = 4 * t[0, 0].numel() * 4
    print(json.dumps({"calibration_copy_bytes_read": moved, "calibration_copy_bytes_written": moved}))


# ---------------------------------------------------------------------------
# Verify workloads (not the headline metric): chunked prefill and tree verify
# ---------------------------------------------------------------------------

VERIFY_LAYERS = 4  # distinct per-layer storage, rotated so no layer is served from the Infinity Cache


def verify_workload(kind: str, device, k8v3: bool = False, layers: int = VERIFY_LAYERS, keep_prefix: bool = False):
    """Chunked prefill: 16 sequences sharing a 4096-token prefix (the prefix
    blocks appear in every block table) each append a 512-token chunk and
    attend bottom-right causally.  Tree verify: 32 sequences with 8192-token
    prefixes each append 16..64 draft nodes of a random tree (BFS, 1-4
    children per expanded node) and attend prefix + ancestors; tree_b1: one
    sequence, a 32768-token prefix and a 32-node tree.  Seeds 3 / 4 / 5.
    `k8v3`: the same over the K8V3 cache (int8 K, 3-bit Lloyd-Max V)."""
    import torch

    from superl8_serve_amd import ops
    from superl8_serve_amd.codebook import gaussian_codebook

    rng = np.random.default_rng({"chunk": 3, "tree": 4}.get(kind, 5))
    if kind == "chunk":
        b_, prefix_len, nq_max = 16, 4096, 512
        nq = np.full(b_, nq_max)
        shared = prefix_len // BS
        own = (nq_max + BS - 1) // BS
        n_blocks = shared + b_ * own + 4
        perm = rng.permutation(n_blocks)
        bt = np.zeros((b_, shared + own), np.int32)
        for i in range(b_):
            bt[i, :shared] = perm[:shared]
            bt[i, shared:] = perm[shared + i * own: shared + (i + 1) * own]
        prefix = np.full(b_, prefix_len)
        tree = None
    else:
        if kind == "tree_b1":  # batch-1 speculative decoding: one long context, one 32-node tree
            b_, prefix_len = 1, 32768
            nq = np.full(1, 32)
            nq_max = 32
        else:
            b_, prefix_len = 32, 8192
            nq = rng.integers(16, 65, size=b_)
            nq_max = 64
        per = (prefix_len + nq_max + BS - 1) // BS
        n_blocks = b_ * per + 4
        perm = rng.permutation(n_blocks)
        bt = perm[: b_ * per].reshape(b_, per).astype(np.int32)
        prefix = np.full(b_, prefix_len)
        tree = np.zeros((b_, nq_max), np.int64)
        for i in range(b_):
            masks, frontier, nxt = [1], [0], 1
            while nxt < nq[i]:
                parent = frontier.pop(0)
                for _ in range(int(rng.integers(1, 5))):
                    if nxt >= nq[i]:
                        break
                    masks.append(masks[parent] | (1 << nxt))
                    frontier.append(nxt)
                    nxt += 1
            tree[i, : nq[i]] = [m - (1 << 64) if m >= 1 << 63 else m for m in masks]
    width = bt.shape[1]
    shape = (layers, n_blocks, HKV, BS, D)
    kc = torch.zeros(shape, dtype=torch.int8, device=device)
    ks = torch.ones(shape[:4], dtype=torch.float32, device=device)
    cb = torch.from_numpy(gaussian_codebook()).to(device)
    if k8v3:  # vc / vs hold the packed codes and the block norms
        vc = torch.zeros(shape[:4] + (D * 3 // 32,), dtype=torch.int32, device=device)
        vs = torch.zeros(shape[:4] + (D // 128,), dtype=torch.float32, device=device)
    else:
        vc = torch.zeros(shape, dtype=torch.int8, device=device)
        vs = torch.ones(shape[:4], dtype=torch.float32, device=device)

    def append(k, v, layer, slots):
        if k8v3:
            ops.quantize_kv_write_paged_k8v3(k, v, kc[layer], ks[layer], vc[layer], vs[layer], cb, slots)
        else:
            ops.quantize_kv_write_paged(k, v, kc[layer], ks[layer], vc[layer], vs[layer], slots)
    gen = torch.Generator(device=device)
    gen.manual_seed({"chunk": 3, "tree": 4}.get(kind, 5))
    # prefix tokens (the shared prefix once for the chunk workload)
    rows = range(1) if kind == "chunk" else range(b_)
    pre_slots = np.concatenate([bt[i, np.arange(prefix_len) // BS] * BS + np.arange(prefix_len) % BS for i in rows])
    new_slots = np.concatenate([bt[i, (prefix_len + np.arange(nq[i])) // BS] * BS + (prefix_len + np.arange(nq[i])) % BS
                                for i in range(b_)]).astype(np.int32)
    ch = [torch.from_numpy(rng.choice(D, OUTLIER_CH, replace=False)).to(device) for _ in range(layers)]
    sm = torch.from_numpy(pre_slots.astype(np.int32)).to(device)
    kept = []
    for layer in range(layers):
        kp = _fp16_outliers(gen, (pre_slots.size, HKV, D), ch[layer], device)
        vp = _fp16_outliers(gen, (pre_slots.size, HKV, D), ch[layer], device)
        append(kp, vp, layer, sm)
        if keep_prefix:
            kept.append((kp, vp))
    t_new = int(new_slots.size)
    k_new = [_fp16_outliers(gen, (t_new, HKV, D), ch[l], device) for l in range(layers)]
    v_new = [_fp16_outliers(gen, (t_new, HKV, D), ch[l], device) for l in range(layers)]
    q = [_fp16_outliers(gen, (b_, nq_max, HQ, D), ch[l], device).transpose(1, 2) for l in range(layers)]
    w = {"kc": kc, "vc": vc, "ks": ks, "vs": vs, "bt": torch.from_numpy(bt).to(device), "bt_np": bt,
         "prefix_np": prefix, "nq_np": nq, "tree_np": tree, "pre_slots": pre_slots.astype(np.int32),
         "new_slots": new_slots, "prefix_kv": kept,
         "prefix": torch.from_numpy(prefix.astype(np.int32)).to(device),
         "ql": torch.from_numpy(nq.astype(np.int32)).to(device),
         "tree": None if tree is None else torch.from_numpy(tree).to(device),
         "new_sm": torch.from_numpy(new_slots).to(device), "k_new": k_new, "v_new": v_new, "q": q,
         "max_ctx": width * BS, "cb": cb, "append": append}
    # useful work: every query attends prefix + its visible drafts
    if kind == "chunk":
        ctx = [prefix_len + s + 1 for i in range(b_) for s in range(nq[i])]
        kv_tokens = prefix_len + int(nq.sum())  # distinct keys read (shared prefix once)
    else:
        ctx = [prefix_len + bin(int(m) & ((1 << 64) - 1)).count("1") for i in range(b_) for m in tree[i, : nq[i]]]
        kv_tokens = int((prefix + nq).sum())
    flops = 4 * D * HQ * int(np.sum(ctx))
    per_head = K8V3_BYTES_PER_TOKEN_HEAD if k8v3 else BYTES_PER_TOKEN_HEAD
    hbm = kv_tokens * HKV * per_head + 2 * 2 * b_ * HQ * nq_max * D
    append_bytes = t_new * HKV * (D * 4 + per_head) + 4 * t_new
    torch.cuda.synchronize()
    return w, {"batch": b_, "prefix": prefix_len, "queries": int(nq.sum()), "flops_layer": flops,
               "kv_bytes_layer": hbm, "append_bytes_layer": append_bytes}


def run_verify(kind: str, steps: int, warmup: int, k8v3: bool = False) -> None:
    import torch

    from superl8_serve_amd import ops

    w, info = verify_workload(kind, "cuda", k8v3)
    scale = 1.0 / math.sqrt(D)

    def layer_ops(layer, append=True):
        if append:
            w["append"](w["k_new"][layer], w["v_new"][layer], layer, w["new_sm"])
        kw = dict(query_lens=w["ql"], tree_mask=w["tree"], max_context_len=w["max_ctx"], scale=scale)
        if k8v3:
            return ops.attn_paged_verify_k8v3(w["q"][layer], w["kc"][layer], w["ks"][layer], w["vc"][layer],
                                              w["vs"][layer], w["cb"], w["bt"], w["prefix"], BS, **kw)
        return ops.attn_paged_verify(w["q"][layer], w["kc"][layer], w["ks"][layer], w["vc"][layer], w["vs"][layer],
                                     w["bt"], w["prefix"], BS, **kw)

    per_call = _timed_warmup(lambda i: layer_ops(i % VERIFY_LAYERS), max(warmup, 1) * VERIFY_LAYERS)
    warm = lambda i: layer_ops(i % VERIFY_LAYERS, append=False)  # noqa: E731
    st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # attention alone
    _spin_ahead(warm, per_call)
    st.record()
    for i in range(steps * VERIFY_LAYERS):
        layer_ops(i % VERIFY_LAYERS, append=False)
    en.record()
    torch.cuda.synchronize()
    t_attn = st.elapsed_time(en) * 1e-3 / (steps * VERIFY_LAYERS)
    _spin_ahead(warm, per_call)
    st.record()
    for i in range(steps * VERIFY_LAYERS):
        layer_ops(i % VERIFY_LAYERS)
    en.record()
    torch.cuda.synchronize()
    t_layer = st.elapsed_time(en) * 1e-3 / (steps * VERIFY_LAYERS)
    tflops = info["flops_layer"] / t_attn / 1e12
    name = {"chunk": "chunked prefill (16 x (4096 shared prefix + 512 chunk))",
            "tree": "tree verify (32 x (8192 prefix + 16..64 draft tree))",
            "tree_b1": "tree verify (1 x (32768 prefix + 32 draft tree))"}[kind]
    split = {}
    if kind == "tree_b1":  # the same call with the key-range split switched off
        from superl8_serve_amd import _lib

        _lib.check(_lib.load().s8kv_verify_set_splits(1), "s8kv_verify_set_splits")
        _spin_ahead(warm, _timed_warmup(warm, 2))
        st.record()
        for i in range(steps * VERIFY_LAYERS):
            layer_ops(i % VERIFY_LAYERS, append=False)
        en.record()
        torch.cuda.synchronize()
        _lib.check(_lib.load().s8kv_verify_set_splits(0), "s8kv_verify_set_splits")
        t_one = st.elapsed_time(en) * 1e-3 / (steps * VERIFY_LAYERS)
        split = {"ms_per_layer_attention_unsplit": round(t_one * 1e3, 4), "split_speedup": round(t_one / t_attn, 2)}
    print(json.dumps({
        "metric": f"paged {'k8v3' if k8v3 else 'int8'} verify attention TFLOP/s, {name}, Qwen3-8B heads",
        "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_layer_attention": round(t_attn * 1e3, 4), "ms_per_layer_append_plus_attention": round(t_layer * 1e3, 4),
        **split, "higher_is_better": True,
        "dtype": f"{'int8 K / 3-bit V' if k8v3 else 'int8'} cache, fp16 MFMA (hi+lo split operands)",
        "data": "synthetic (fp16 N(0,1), 2 of 128 channels x20)",
        "config": {"workload": name, "num_q_heads": HQ, "num_kv_heads": HKV, "head_dim": D, "block_size": BS,
                   "layers_rotated": VERIFY_LAYERS, **info},
        "roofline": roofline_max(info["kv_bytes_layer"], info["flops_layer"], t_attn,
                                 note="useful flops (4*D*Hq per visible key); the kernel issues 2x MFMAs "
                                      "(hi+lo operands)"),
    }))


# ---------------------------------------------------------------------------
# K8V3 decode step (int8 K, 3-bit Lloyd-Max V) and block copy
# ---------------------------------------------------------------------------

K8V3_BATCH = 32
K8V3_BYTES_PER_TOKEN_HEAD = D + 4 + D * 3 // 8 + 4 * (D // 128)  # 184 B


def k8v3_workload(dev, layers: int = NUM_LAYERS, keep_rows=()):
    """The K8V3 decode-step workload (batch 32, contexts U{8192..32768},
    seed 2) over `layers` layers of distinct storage: every row's prefix
    appended, and per layer the new tokens' K/V and q.  `keep_rows`: rows whose
    layer-0 prefix K/V (fp16) are returned too, as (row, first position, k, v)
    chunks."""
    import torch

    from superl8_serve_amd import ops
    from superl8_serve_amd.codebook import gaussian_codebook

    rng = np.random.default_rng(2)
    lens = rng.integers(8192, 32769, size=K8V3_BATCH)
    need = (lens + BS - 1) // BS
    n_blocks = int(math.ceil(1.2 * need.sum()))
    perm = rng.permutation(n_blocks)
    width = int(need.max())
    bt = np.zeros((K8V3_BATCH, width), np.int32)
    pos = 0
    for b in range(K8V3_BATCH):
        bt[b, : need[b]] = perm[pos: pos + need[b]]
        pos += need[b]
    prefix = lens - 1
    shape = (layers, n_blocks, HKV, BS, D)
    kc = torch.zeros(shape, dtype=torch.int8, device=dev)
    ks = torch.ones(shape[:4], dtype=torch.float32, device=dev)
    vp = torch.zeros(shape[:4] + (D * 3 // 32,), dtype=torch.int32, device=dev)
    vn = torch.zeros(shape[:4] + (D // 128,), dtype=torch.float32, device=dev)
    cb = torch.from_numpy(gaussian_codebook(3, 128)).to(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(2)
    chunk = 65536
    kept = []
    for layer in range(layers):
        ch = torch.from_numpy(rng.choice(D, OUTLIER_CH, replace=False)).to(dev)
        for b in range(K8V3_BATCH):
            for c0 in range(0, int(prefix[b]), chunk):
                n = min(chunk, int(prefix[b]) - c0)
                p_ = np.arange(c0, c0 + n)
                sm = torch.from_numpy((bt[b, p_ // BS] * BS + p_ % BS).astype(np.int32)).to(dev)
                kp = _fp16_outliers(gen, (n, HKV, D), ch, dev)
                vq = _fp16_outliers(gen, (n, HKV, D), ch, dev)
                ops.quantize_kv_write_paged_k8v3(kp, vq, kc[layer], ks[layer], vp[layer], vn[layer], cb, sm)
                if layer == 0 and b in keep_rows:
                    kept.append((b, c0, kp, vq))
    new_slots = np.array([bt[b, prefix[b] // BS] * BS + prefix[b] % BS for b in range(K8V3_BATCH)], np.int32)
    k_new = [torch.randn((K8V3_BATCH, HKV, D), generator=gen, device=dev).half() for _ in range(layers)]
    v_new = [torch.randn((K8V3_BATCH, HKV, D), generator=gen, device=dev).half() for _ in range(layers)]
    q = [torch.randn((K8V3_BATCH, 1, HQ, D), generator=gen, device=dev).half().transpose(1, 2) for _ in range(layers)]
    torch.cuda.synchronize()
    return {"lens": lens, "need": need, "bt_np": bt, "n_blocks": n_blocks, "kc": kc, "ks": ks, "vp": vp, "vn": vn,
            "cb": cb, "new_slots": new_slots, "new_sm": torch.from_numpy(new_slots).to(dev), "k_new": k_new,
            "v_new": v_new, "q": q, "bt": torch.from_numpy(bt).to(dev),
            "cl": torch.from_numpy(lens.astype(np.int32)).to(dev), "max_ctx": int(need.max()) * BS,
            "prefix_kv": kept}


def run_k8v3(steps: int, warmup: int, fused: bool, planned: bool = True, adaptive: bool = False) -> None:
    """Qwen3-8B K8V3 decode step, batch 32, contexts U{8192..32768} (seed 2):
    36 layers x (append 1 token per sequence + decode), pool 1.2x the blocks
    needed, distinct storage per layer; one launch per layer
    (attn_paged_decode_append_k8v3, after the step's one plan launch when
    `planned`, adaptive when `adaptive`) unless `fused` is False."""
    import torch

    from superl8_serve_amd import ops

    w = k8v3_workload("cuda")
    lens, need, n_blocks = w["lens"], w["need"], w["n_blocks"]
    kc, ks, vp, vn, cb = w["kc"], w["ks"], w["vp"], w["vn"], w["cb"]
    new_sm, k_new, v_new, q, btd, cl, max_ctx = (w[k] for k in ("new_sm", "k_new", "v_new", "q", "bt", "cl",
                                                                 "max_ctx"))
    scale = 1.0 / math.sqrt(D)

    def step():
        plan = None
        if fused and planned:
            plan = ops.attn_paged_decode_plan(kc[0], btd, cl, BS, num_q_heads=HQ, max_context_len=max_ctx,
                                              layout="k8v3", adaptive=adaptive, plan=w.get("plan"))
            if adaptive:
                w["plan"] = plan
        for layer in range(NUM_LAYERS):
            if fused:
                ops.attn_paged_decode_append_k8v3(q[layer], k_new[layer], v_new[layer], kc[layer], ks[layer],
                                                  vp[layer], vn[layer], cb, btd, cl, BS, max_context_len=max_ctx,
                                                  scale=scale, plan=plan)
                continue
            ops.quantize_kv_write_paged_k8v3(k_new[layer], v_new[layer], kc[layer], ks[layer], vp[layer], vn[layer],
                                             cb, new_sm)
            ops.attn_paged_decode_k8v3(q[layer], kc[layer], ks[layer], vp[layer], vn[layer], cb, btd, cl, BS,
                                       max_context_len=max_ctx, scale=scale)

    torch.cuda.synchronize()
    step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        graph.replay()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / max(steps, 1) * 1e3
    t = K8V3_BATCH
    append = t * HKV * D * 4 + 4 * t + t * HKV * K8V3_BYTES_PER_TOKEN_HEAD
    decode = int(lens.sum()) * HKV * K8V3_BYTES_PER_TOKEN_HEAD + 2 * t * HQ * D * 2 + 4 * int(need.sum()) + 4 * t + 32
    step_b = NUM_LAYERS * (append + decode)
    value = step_b / (ms * 1e-3) / 1e9
    print(json.dumps({
        "metric": "paged k8v3 decode-attn+append HBM GB/s (% of peak) at Qwen3-8B shapes, b=32, 8k-32k context",
        "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "dtype": "int8 K / 3-bit V",
        "data": "synthetic (fp16 N(0,1), 2 of 128 channels x20, seed 2)",
        "config": {"workload": "Qwen3-8B K8V3 decode step: 36 layers x (append 1 token/seq + decode)",
                   "batch": t, "sum_context_tokens": int(lens.sum()), "pool_blocks_per_layer": n_blocks,
                   "bytes_per_step": step_b,
                   "append": "in the decode launch (attn_paged_decode_append_k8v3)" if fused
                             else "separate kernel (quantize_kv_write_paged_k8v3)",
                   "slice_plan": ("none" if not (fused and planned) else
                                  "adaptive (bounds from the last step's workgroup times)" if adaptive
                                  else "fixed split")},
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBPS, 2)}))


def run_append(steps: int, warmup: int, k8v3: bool = False) -> None:
    """Prefill append: 64 sequences x 2048 new tokens (131,072 tokens) of
    Qwen3-8B K/V (8 KV heads, head_dim 128, fp16) quantized into a paged
    cache (block 256) by one quantize_kv_write_paged call (K8V3:
    quantize_kv_write_paged_k8v3), as one layer of the reference's
    write_prefill_varlen does; each sequence's slots are contiguous over
    blocks dealt from a seeded permutation of the pool.  The inputs (537 MB)
    exceed the 256 MB Infinity Cache, so every call reads them from HBM."""
    import torch

    from superl8_serve_amd import ops

    seqs, per_seq = 64, 2048
    T = seqs * per_seq
    nblk = per_seq // BS
    pool = seqs * nblk + 64
    perm = np.random.default_rng(7).permutation(pool)
    off = np.arange(per_seq)
    slots = np.concatenate([perm[s * nblk + off // BS] * BS + off % BS for s in range(seqs)]).astype(np.int32)
    gen = torch.Generator(device="cuda").manual_seed(7)
    k = torch.randn((T, HKV, D), device="cuda", generator=gen).half()
    v = torch.randn((T, HKV, D), device="cuda", generator=gen).half()
    kc = torch.zeros((pool, HKV, BS, D), dtype=torch.int8, device="cuda")
    ks = torch.zeros((pool, HKV, BS), dtype=torch.float32, device="cuda")
    sm = torch.from_numpy(slots).cuda()
    if k8v3:
        from superl8_serve_amd.codebook import gaussian_codebook

        vc = torch.zeros((pool, HKV, BS, D * 3 // 32), dtype=torch.int32, device="cuda")
        vs = torch.zeros((pool, HKV, BS, D // 128), dtype=torch.float32, device="cuda")
        cb = torch.from_numpy(gaussian_codebook(3, 128)).cuda()

        def call():
            ops.quantize_kv_write_paged_k8v3(k, v, kc, ks, vc, vs, cb, sm)

        out_bytes = D + 4 + D * 3 // 8 + 4 * (D // 128)  # int8 K + scale, packed 3-bit V + norms
    else:
        vc = torch.zeros_like(kc)
        vs = torch.zeros_like(ks)

        def call():
            ops.quantize_kv_write_paged(k, v, kc, ks, vc, vs, sm)

        out_bytes = 2 * D + 2 * 4  # int8 K, V and two fp32 scales
    for _ in range(max(warmup, 1)):
        call()
    torch.cuda.synchronize()
    st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    _spin_ahead()
    st.record()
    for _ in range(steps):
        call()
    en.record()
    torch.cuda.synchronize()
    sec = st.elapsed_time(en) * 1e-3 / steps
    # the same call timed alone: idle GPU before each call, events on either side
    alone = []
    for _ in range(steps):
        torch.cuda.synchronize()
        st.record()
        call()
        en.record()
        torch.cuda.synchronize()
        alone.append(st.elapsed_time(en) * 1e-3)
    sec_alone = float(np.median(alone))
    moved = T * HKV * (2 * D * 2 + out_bytes)  # fp16 K, V in; the cache bytes out
    fmt = "k8v3: int8 K + 3-bit V" if k8v3 else "int8 + scales"
    print(json.dumps({"metric": f"prefill append GB/s (fp16 K/V in, {fmt} out), 131,072 tokens x 8 KV heads",
                      "value": round(moved / sec / 1e9, 1), "unit": "GB/s", "us_per_call": round(sec * 1e6, 1),
                      "us_per_call_alone_median": round(sec_alone * 1e6, 1),
                      "bytes_per_call": moved, "pct_of_hbm_peak": round(100 * moved / sec / 1e9 / HBM_PEAK_GBPS, 1)}))


PREFILL_SEQS, PREFILL_LEN = 16, 4096


def run_prefill(steps: int, warmup: int) -> None:
    """Dense causal prefill attention over fresh fp16 K / V (attn_varlen):
    16 prompts of 4096 tokens, Qwen3-8B heads (Hq 32, Hkv 8, D 128), four
    rotated layers of distinct inputs.  Useful flops: 4*D*Hq per visible
    (query, key) pair."""
    import torch

    from superl8_serve_amd import ops

    dev = "cuda"
    gen = torch.Generator(device=dev)
    gen.manual_seed(6)
    rng = np.random.default_rng(6)
    t = PREFILL_SEQS * PREFILL_LEN
    cu = torch.arange(0, t + 1, PREFILL_LEN, dtype=torch.int32, device=dev)
    layers = []
    for _ in range(4):
        ch = torch.from_numpy(rng.choice(D, OUTLIER_CH, replace=False)).to(dev)
        layers.append((_fp16_outliers(gen, (t, HQ, D), ch, dev), _fp16_outliers(gen, (t, HKV, D), ch, dev),
                       _fp16_outliers(gen, (t, HKV, D), ch, dev)))
    scale = 1.0 / math.sqrt(D)

    def attend(i):
        q, k, v = layers[i % 4]
        return ops.attn_varlen(q, k, v, cu, cu, PREFILL_LEN, PREFILL_LEN, causal=True, scale=scale)

    per_call = _timed_warmup(attend, max(warmup, 1) * 4)
    st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    _spin_ahead(attend, per_call)
    st.record()
    for i in range(steps * 4):
        attend(i)
    en.record()
    torch.cuda.synchronize()
    sec = st.elapsed_time(en) * 1e-3 / (steps * 4)
    flops = 4 * D * HQ * PREFILL_SEQS * PREFILL_LEN * (PREFILL_LEN + 1) // 2
    prefill_bytes = PREFILL_SEQS * PREFILL_LEN * (2 * HQ + 2 * HKV) * D * 2
    tflops = flops / sec / 1e12
    print(json.dumps({
        "metric": "dense causal prefill attention TFLOP/s (fresh fp16 K/V), 16 x 4096 tokens, Qwen3-8B heads",
        "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_layer": round(sec * 1e3, 4), "higher_is_better": True,
        "dtype": "fp16 inputs, fp16 MFMA (exact fp16 q, hi+lo split P), fp32 accumulate",
        "data": "synthetic (fp16 N(0,1), 2 of 128 channels x20, seed 6)",
        "config": {"workload": "dense varlen prefill attention", "sequences": PREFILL_SEQS, "tokens": PREFILL_LEN,
                   "num_q_heads": HQ, "num_kv_heads": HKV, "head_dim": D, "flops_layer": flops},
        "roofline": roofline_max(prefill_bytes, flops, sec,
                                 note="useful flops; fp16 q, k, v read and o written once"),
    }))


WINDOW = 4096
WINDOW_LAYERS = 4  # distinct storage, rotated so no layer is served from the Infinity Cache


def run_window(steps: int, warmup: int) -> None:
    """Sliding-window decode (attn_paged_decode_window): Qwen3-8B int8 heads,
    batch 64, contexts U{8192..32768} (seed 5), window 4096 -- each row reads
    its last 4096 tokens.  Only the windowed positions (and the rest of the
    32-token tile holding a window start) are filled; earlier positions are
    never read.  Four layers of distinct storage, rotated."""
    import torch

    from superl8_serve_amd import ops

    dev = "cuda"
    rng = np.random.default_rng(5)
    lens = rng.integers(8192, 32769, size=BATCH)
    need = (lens + BS - 1) // BS
    n_blocks = int(need.sum()) + 4
    perm = rng.permutation(n_blocks)
    width = int(need.max())
    bt = np.zeros((BATCH, width), np.int32)
    pos = 0
    for b in range(BATCH):
        bt[b, : need[b]] = perm[pos: pos + need[b]]
        pos += need[b]
    first = [(max(0, int(n) - WINDOW)) & ~31 for n in lens]
    slots = np.concatenate([bt[b, np.arange(first[b], lens[b]) // BS] * BS + np.arange(first[b], lens[b]) % BS
                            for b in range(BATCH)]).astype(np.int32)
    shape = (n_blocks, HKV, BS, D)
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    sm = torch.from_numpy(slots).to(dev)
    layers = []
    for layer in range(WINDOW_LAYERS):
        kc = torch.zeros(shape, dtype=torch.int8, device=dev)
        vc = torch.zeros(shape, dtype=torch.int8, device=dev)
        ks = torch.zeros(shape[:3], dtype=torch.float32, device=dev)
        vs = torch.zeros(shape[:3], dtype=torch.float32, device=dev)
        ch = torch.from_numpy(rng.choice(D, OUTLIER_CH, replace=False)).to(dev)
        for c0 in range(0, slots.size, 65536):
            n = min(65536, slots.size - c0)
            kp = _fp16_outliers(gen, (n, HKV, D), ch, dev)
            vp = _fp16_outliers(gen, (n, HKV, D), ch, dev)
            ops.quantize_kv_write_paged(kp, vp, kc, ks, vc, vs, sm[c0:c0 + n])
        q = _fp16_outliers(gen, (BATCH, HQ, 1, D), ch, dev)
        layers.append((q, kc, ks, vc, vs))
    btd = torch.from_numpy(bt).to(dev)
    cl = torch.from_numpy(lens.astype(np.int32)).to(dev)
    scale = 1.0 / math.sqrt(D)

    def attend(i):
        q, kc, ks, vc, vs = layers[i % WINDOW_LAYERS]
        return ops.attn_paged_decode_window(q, kc, ks, vc, vs, btd, cl, BS, max_context_len=width * BS,
                                            window=WINDOW, scale=scale)

    per_call = _timed_warmup(attend, max(warmup, 1) * WINDOW_LAYERS)
    st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    _spin_ahead(attend, per_call)
    st.record()
    for i in range(steps * WINDOW_LAYERS):
        attend(i)
    en.record()
    torch.cuda.synchronize()
    t = st.elapsed_time(en) * 1e-3 / (steps * WINDOW_LAYERS)
    tokens = int(np.minimum(lens, WINDOW).sum())
    nbytes = tokens * HKV * BYTES_PER_TOKEN_HEAD + 2 * 2 * BATCH * HQ * D + 4 * BATCH * (1 + WINDOW // BS + 1)
    print(json.dumps({
        "metric": f"paged int8 sliding-window decode HBM GB/s, Qwen3-8B shapes, b={BATCH}, window {WINDOW}, "
                  "8k-32k contexts",
        "value": round(nbytes / t / 1e9, 2), "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "us_per_launch": round(t * 1e6, 2), "higher_is_better": True, "dtype": "int8",
        "data": "synthetic (fp16 N(0,1), 2 of 128 channels x20, seed 5)",
        "config": {"workload": "sliding-window decode", "batch": BATCH, "window": WINDOW,
                   "sum_window_tokens": tokens, "bytes_per_launch": nbytes, "layers_rotated": WINDOW_LAYERS},
        "pct_of_hbm_peak": round(nbytes / t / 1e9 / 8000.0 * 100, 2),
    }))


def run_copy(steps: int) -> None:
    """copy_blocks over a 4096-block synthetic pool (Qwen3-8B int8 block: K, V,
    two scale tensors; 1 layer): 1024 random source blocks moved to 1024 other
    random blocks, as a compaction pass does."""
    import torch

    from superl8_serve_amd import ops

    rng = np.random.default_rng(5)
    n = 4096
    t = [torch.randint(-127, 128, (1, n, HKV, BS, D), dtype=torch.int8, device="cuda") for _ in range(2)]
    t += [torch.rand((1, n, HKV, BS), device="cuda") for _ in range(2)]
    perm = rng.permutation(n)
    # block ids already on the device, as a serving loop hands them over
    src = torch.tensor(perm[:1024], dtype=torch.int32, device="cuda")
    dst = torch.tensor(perm[1024:2048], dtype=torch.int32, device="cuda")
    ops.copy_blocks(t, src, dst)
    torch.cuda.synchronize()
    st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    _spin_ahead()
    st.record()
    for _ in range(steps):
        ops.copy_blocks(t, src, dst)
    en.record()
    torch.cuda.synchronize()
    sec = st.elapsed_time(en) * 1e-3 / steps
    moved = 1024 * (2 * HKV * BS * D + 2 * HKV * BS * 4)
    print(json.dumps({"metric": "copy_blocks GB/s (read + write), 1024 random blocks of a 4096-block pool",
                      "value": round(2 * moved / sec / 1e9, 1), "unit": "GB/s", "us_per_call": round(sec * 1e6, 1),
                      "bytes_moved": moved, "pct_of_hbm_peak": round(100 * 2 * moved / sec / 1e9 / HBM_PEAK_GBPS, 1)}))


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=50,
                    help="untimed steps first (50 graph replays of the decode step take ~0.12 s; with 5 the "
                         "timed steps start before the engine clock settles and read ~1 %% lower)")
    ap.add_argument("--cpu-layers", type=int, default=NUM_LAYERS, help="layers in the CPU-baseline sample (0 = skip)")
    ap.add_argument("--traffic-json", default=os.path.join(ROOT, "profiles", "decode_traffic.json"),
                    help="measured HBM bytes per decode launch (from the PMC runs) to report as roofline.traffic")
    ap.add_argument("--kernel-reps", type=int, default=3,
                    help="eager event-timed decode passes over the 36 layers (0 = skip, one-launch step only)")
    ap.add_argument("--ceiling-steps", type=int, default=5,
                    help="graph replays per read-ceiling probe (0 = skip the read-ceiling leg)")
    ap.add_argument("--no-plan", action="store_true",
                    help="fused step without the per-step slice plan (every launch locates its own work)")
    ap.add_argument("--adaptive-split", action="store_true",
                    help="the step's plan with adaptive slice bounds that follow the last step's measured "
                         "workgroup times (default: the fixed split)")
    ap.add_argument("--separate-append", action="store_true",
                    help="decode step as the reference's two calls per layer (append kernel, then decode) instead "
                         "of the one-launch append + decode")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0, help="only run a plain copy of this size")
    ap.add_argument("--trace-decode", action="store_true",
                    help="only print the per-launch breakdown of the decode step from the trace build "
                         "(superl8_serve_amd/libsuperl8_kv_trace.so)")
    ap.add_argument("--workload", choices=["decode", "chunk", "tree", "tree_b1", "chunk_k8v3", "tree_k8v3", "k8v3",
                                           "window", "prefill", "copy", "append", "append_k8v3"],
                    default="decode",
                    help="decode: the Qwen3-8B batch-64 int8 decode step (headline); chunk / tree: verify "
                         "attention (chunk_k8v3 / tree_k8v3: over the K8V3 cache; tree_b1: one sequence, "
                         "32768-token prefix, 32-node tree); k8v3: the K8V3 decode step "
                         "(batch 32, 8k-32k); window: sliding-window decode (batch 64, window 4096); prefill: dense "
                         "causal prefill attention (16 x 4096 tokens); copy: "
                         "copy_blocks; append / append_k8v3: prefill append of 131,072 tokens")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: measures one GPU only; --gpus {args.gpus} is not supported "
              "(the path shards by sequence or KV head with no exchange; see the design notes)", file=sys.stderr)
        sys.exit(2)

    import torch

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    from superl8_serve_amd import _lib

    if args.trace_decode:
        from superl8_serve_amd import build_ext

        _lib.LIB_PATH = build_ext.TRACE_LIB_PATH
        print(json.dumps(trace_decode(args.steps, args.warmup, args.adaptive_split)))
        return
    _lib.load()
    if args.calibrate_copy_mib:
        calibrate_copy(args.calibrate_copy_mib)
        return
    if args.workload in ("chunk", "tree", "tree_b1", "chunk_k8v3", "tree_k8v3"):
        run_verify(args.workload.removesuffix("_k8v3"), args.steps, args.warmup, k8v3=args.workload.endswith("_k8v3"))
        return
    if args.workload == "k8v3":
        run_k8v3(args.steps, args.warmup, not args.separate_append, not args.no_plan, args.adaptive_split)
        return
    if args.workload == "copy":
        run_copy(args.steps)
        return
    if args.workload == "window":
        run_window(args.steps, args.warmup)
        return
    if args.workload == "prefill":
        run_prefill(args.steps, args.warmup)
        return
    if args.workload in ("append", "append_k8v3"):
        run_append(args.steps, args.warmup, k8v3=args.workload == "append_k8v3")
        return

    device = "cuda"
    w = build(device)
    fused = not args.separate_append
    planned = fused and not args.no_plan
    adaptive = planned and args.adaptive_split
    step = make_step(w, fused, planned, adaptive)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    # HIP events on the replay stream bracket the timed replays as well
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(args.steps):
        graph.replay()
    ev1.record()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms = dt / max(args.steps, 1) * 1e3
    ev_launch_s = ev0.elapsed_time(ev1) * 1e-3 / (max(args.steps, 1) * NUM_LAYERS)

    b = step_bytes(w["lens"])
    value = b["step"] / (ms * 1e-3) / 1e9
    # eager per-launch timing: required for the two-call step, a cross-check otherwise
    kt = (time_decode_kernel(w, args.kernel_reps, fused, planned, adaptive) if args.kernel_reps > 0 or not fused
          else {"decode_s": None, "launches": 0})
    kernel = "decode_kernel<128, int8, fused append>" if fused else "decode_kernel<128, int8>"
    kernel_bytes = b["fused_layer"] if fused else b["decode_layer"]
    # The one-launch step graph holds NUM_LAYERS decode_kernel launches and
    # (planned) the step's one plan launch, so the events around the timed
    # replays give the kernel's average launch duration over the timed region
    # (gaps between the back-to-back launches and the plan launch's share
    # included).  The two-call step also runs the append
    # kernel, so there the library's per-launch events over eager passes time
    # the decode kernel alone.
    dec_s = ev_launch_s if fused else kt["decode_s"]
    achieved = kernel_bytes / dec_s / 1e9
    traffic = None
    if args.traffic_json and os.path.exists(args.traffic_json):
        with open(args.traffic_json) as f:
            tj = json.load(f)
        if tj.get("kernel") == kernel:  # measured for this kernel
            traffic = tj.get("decode_kernel_hbm_bytes_per_launch")
    result = {
        "metric": "paged int8 decode-attn+append HBM GB/s (% of peak) at Qwen3-8B shapes, b=64",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (fp16 N(0,1) K/V/q, 2 of 128 channels x20, seed 1)",
        "config": {
            "workload": "Qwen3-8B int8 paged KV decode step: 36 layers x (append 1 token/seq + GQA decode)",
            "batch": BATCH, "num_q_heads": HQ, "num_kv_heads": HKV, "head_dim": D, "block_size": BS,
            "layers": NUM_LAYERS, "context": f"lognormal(median 2048, sigma {SIGMA}) clipped [256, 8192], seed {SEED}",
            "sum_context_tokens": int(w["lens"].sum()), "pool_blocks_per_layer": POOL_BLOCKS,
            "bytes_per_step": b["step"],
            "append": "in the decode launch (attn_paged_decode_append)" if fused
                      else "separate kernel (quantize_kv_write_paged)",
            "slice_plan": ("none (every launch locates its own work)" if not planned else
                           "one adaptive attn_paged_decode_plan per step (slice bounds from the last step's "
                           "workgroup times), read by the 36 launches" if adaptive else
                           "one attn_paged_decode_plan launch per step (fixed split), read by the 36 launches"),
        },
        "pct_of_hbm_peak": round(100.0 * value / HBM_PEAK_GBPS, 2),
        "roofline": {
            "kernel": kernel,
            "bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
            "avg_launch_us": round(dec_s * 1e6, 2), "algorithmic_bytes_per_launch": kernel_bytes,
            "avg_launch_from": ("HIP events around the timed graph replays / launches" if fused
                                else "library HIP events per eager launch"),
            "timed_launches": args.steps * NUM_LAYERS if fused else kt["launches"],
            "eager_avg_launch_us": round(kt["decode_s"] * 1e6, 2) if kt["decode_s"] else None,
        },
    }
    if args.ceiling_steps > 0:
        rc = read_ceiling(w, args.ceiling_steps)
        rc["decode_frac_of_tiles_best"] = round(achieved / rc["tiles_best_gbps"], 4)
        rc["decode_frac_of_linear_best"] = round(achieved / rc["linear_best_gbps"], 4)
        result["read_ceiling"] = rc
    if args.cpu_layers > 0:
        result["cpu_baseline"] = cpu_baseline(w["lens"], w["bt_np"], args.cpu_layers)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
