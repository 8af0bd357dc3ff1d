#!/usr/bin/env python3
"""Token-mixer benchmark on one MI355X (gfx950).

Headline line (one JSON object on stdout): Gated-DeltaNet prefill of one
2048-token sequence through one layer (16 k-heads, 32 v-heads, dk = dv = 128,
conv 4, zero state, fp32), tokens/s, with the roofline of its dominant kernel
and the CPU restatement timed beside it.  The same line carries the decode
mixers (one DeltaNet layer at batch 1; one GQA layer at 8193 cached rows), the
GQA prefill at T = 2048 and the 32-layer mixer stack (24 DeltaNet + 8 GQA
layers, 8 sequences at context 32768, 128 decode steps) under "workloads".

A step is one pass of the measured mixer over its synthetic inputs, which are
resident in HBM before the timed region.  Timing uses HIP events on the
library's own stream; per-kernel durations come from the library's event
timers in a second, separately timed pass.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "qwen3.5sharp_amd"))

import q35mix  # noqa: E402
import synth  # noqa: E402

HBM_PEAK = 8.0e12          # B/s, MI355X datasheet
FP32_PEAK = 157.3e12       # FLOP/s, MI355X dense fp32 (matrix = vector)
INT8_PEAK = 5.0e15         # OP/s, MI355X dense int8 matrix
NK, NV, DK = 16, 32, 128
NH, NKV, HD = 16, 4, 256
CONV_DIM = 2 * NK * DK + NV * DK
VALUE_DIM = NV * DK
Q_DIM, KV_DIM = NH * HD, NKV * HD

# Algorithmic work per unit.
DN_DECODE_BYTES = 4_588_544               # 1 token, 1 layer, 1 sequence


def attn_decode_bytes(kv_len: int) -> int:
    return 8192 * kv_len + 59_648          # K+V rows + q|gate, new k/v, out, norms, RoPE row


DN_PREFILL_FLOP = 11_811_160_064           # T=2048, chunked WY form (32 heads x 32 chunks)
# Per-kernel algorithmic work of one T=2048 DeltaNet prefill (C = 64, 32 chunks,
# 16 k-heads, 32 v-heads), as (bound, amount, description):
DN_PREFILL_KERNELS = {
    "dn_chunk_scan": ("mfma", 32 * 32 * 3 * (2 * 64 * DK * DK),
                      "W S, K^T D and Q S, 3 x 2*64*128*128 FLOP per (v-head, chunk), 32 x 32"),
    "dn_chunk_out": ("hbm", 4 * 32 * 32 * (10 * 16 * 16 + 4 * 64 * DK),
                     "M o QK^T causal blocks (10 x 16x16 floats), inter-chunk output, D and z "
                     "(64x128 floats each) read, out (64x128) written, per (v-head, chunk)"),
    "dn_chunk_prep": ("mfma", 32 * 16 * 2 * 2 * 64 * 64 * DK + 32 * 32 * 2 * 2 * 64 * 64 * DK,
                      "K K^T, Q K^T (2 x 2*64*64*128 per k-head chunk) + W, U (2 x 2*64*64*128 "
                      "per v-head chunk); also the conv, gates and norms of the inputs"),
}
ATTN_PREFILL_FLOP = 4 * HD * NH * 2048 * 2049 // 2
PROFILES = os.path.join(ROOT, "profiles")


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed PMC summary
    (profiles/<kernel>_traffic.txt, line 'bytes_per_launch: N'), or None."""
    path = os.path.join(PROFILES, f"{kernel}_traffic.txt")
    try:
        for line in open(path):
            if line.startswith("bytes_per_launch:"):
                return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def time_calls(ctx, fn, steps, warmup):
    for i in range(warmup):
        fn(i)
    ctx.sync()
    e0, e1 = q35mix.Event(), q35mix.Event()
    e0.record(ctx.stream)
    for i in range(steps):
        fn(warmup + i)
    e1.record(ctx.stream)
    ms = e0.elapsed_ms(e1)
    return ms / steps


def time_calls_median(ctx, fn, steps, warmup, group=10):
    """Per-call time of back-to-back calls: `steps` calls in groups of
    `group`, one event pair around each group (an event recorded between
    single calls would add its own few microseconds to every call), the
    median over the groups of the per-call mean: (median ms, mean ms)."""
    for i in range(warmup):
        fn(i)
    ctx.sync()
    groups = max(1, steps // group)
    ev = [q35mix.Event() for _ in range(groups + 1)]
    ev[0].record(ctx.stream)
    for g in range(groups):
        for j in range(group):
            fn(warmup + g * group + j)
        ev[g + 1].record(ctx.stream)
    ev[-1].synchronize()
    per = [ev[g].elapsed_ms(ev[g + 1]) / group for g in range(groups)]
    return float(np.median(per)), float(np.mean(per))


def kernel_times(ctx, fn, steps):
    ctx.profile(True)
    for i in range(steps):
        fn(i)
    res = ctx.profile_read()
    ctx.profile(False)
    return {k: (ms / n, n) for k, (ms, n) in res.items()}


def dominant(ktimes):
    name = max(ktimes, key=lambda k: ktimes[k][0] * ktimes[k][1])
    return name, ktimes[name][0]


# --------------------------------------------------------------------------
# workloads
# --------------------------------------------------------------------------

def bench_dn_prefill(steps, warmup, T=2048):
    ctx = q35mix.Context(q35mix.qwen35_config(num_layers=1, is_recurrent=[1]), 1, 16)
    ctx.set_deltanet_weights(0, synth.deltanet_weights(NK, NV, DK))
    x = synth.deltanet_inputs(T, NK, NV, DK)
    qkv, z = ctx.array((T, CONV_DIM), x["qkv"]), ctx.array((T, VALUE_DIM), x["z"])
    b, a = ctx.array((T, NV), x["b"]), ctx.array((T, NV), x["a"])
    out = ctx.array((T, VALUE_DIM))

    def step(i):
        ctx.deltanet_prefill(0, 0, T, qkv, z, b, a, out)

    ms = time_calls(ctx, step, steps, warmup)
    # Per-kernel times (the roofline) over at least 50 layers: one pass of 10
    # varies by up to 10 % between runs, 50 agree with a kernel trace.  As
    # time per step: (per-launch ms x launches) / steps profiled.
    n_prof = max(steps, 50)
    kt = kernel_times(ctx, step, n_prof)
    kt = {k: (v[0] * v[1] / n_prof, 1) for k, v in kt.items()}
    ctx.close()
    return ms, kt, x


def bench_dn_decode(steps, warmup, n_layers=160):
    """Batch 1; rotates over n_layers distinct states (> MALL) between calls."""
    ctx = q35mix.Context(q35mix.qwen35_config(num_layers=n_layers, is_recurrent=[1] * n_layers),
                         1, 16)
    w = synth.deltanet_weights(NK, NV, DK)
    for layer in range(n_layers):
        ctx.set_deltanet_weights(layer, w)
    x = synth.deltanet_inputs(1, NK, NV, DK)
    qkv, z = ctx.array((1, CONV_DIM), x["qkv"]), ctx.array((1, VALUE_DIM), x["z"])
    b, a = ctx.array((1, NV), x["b"]), ctx.array((1, NV), x["a"])
    out = ctx.array((1, VALUE_DIM))

    def step(i):
        ctx.deltanet_decode(i % n_layers, [0], qkv, z, b, a, out)

    ms = time_calls_median(ctx, step, steps, warmup)
    kt = kernel_times(ctx, step, steps)
    ctx.close()
    return ms, kt


def bench_attn_decode(steps, warmup, n_layers=8, pos=8192):
    """One token at position 8192 (8193 rows); rotates over 8 distinct caches."""
    ctx = q35mix.Context(q35mix.qwen35_config(num_layers=n_layers, is_recurrent=[0] * n_layers),
                         1, pos + 1)
    wts = synth.attn_weights(HD)
    k, v = synth.kv_prefill(pos, KV_DIM)
    for layer in range(n_layers):
        ctx.set_attn_weights(layer, wts)
        ctx.state_write(layer, 0, q35mix.STATE_KEYS, k)
        ctx.state_write(layer, 0, q35mix.STATE_VALUES, v)
    ctx.advance(0, pos)
    x = synth.attn_inputs(1, NH, NKV, HD)
    qg, kk, vv = ctx.array((1, 2 * Q_DIM), x["q_gate"]), ctx.array((1, KV_DIM), x["k"]), \
        ctx.array((1, KV_DIM), x["v"])
    out = ctx.array((1, Q_DIM))

    def step(i):
        ctx.attn_decode(i % n_layers, [0], qg, kk, vv, out)

    ms = time_calls_median(ctx, step, steps, warmup)
    kt = kernel_times(ctx, step, steps)
    ctx.close()
    return ms, kt


def bench_attn_prefill(steps, warmup, T=2048):
    ctx = q35mix.Context(q35mix.qwen35_config(num_layers=1, is_recurrent=[0]), 1, T)
    ctx.set_attn_weights(0, synth.attn_weights(HD))
    x = synth.attn_inputs(T, NH, NKV, HD)
    qg, kk, vv = ctx.array((T, 2 * Q_DIM), x["q_gate"]), ctx.array((T, KV_DIM), x["k"]), \
        ctx.array((T, KV_DIM), x["v"])
    out = ctx.array((T, Q_DIM))

    def step(i):
        ctx.attn_prefill(0, 0, T, qg, kk, vv, out)

    ms = time_calls(ctx, step, steps, warmup)
    kt = kernel_times(ctx, step, steps)
    ctx.close()
    return ms, kt


def bench_linear_q(qtype, n_in, n_out, steps, warmup, copies, tokens=1, order=0):
    """Projection of `tokens` rows (1: the decode GEMV) rotating over `copies`
    weight copies, more bytes than the 256 MB MALL; `order` is the
    projection order (q35m_set_projection_order)."""
    ctx = q35mix.Context(q35mix.qwen35_config(num_layers=1, is_recurrent=[1]), 1, 16)
    ctx.set_projection_order(order)
    w = synth.quant_weights(qtype, n_out, n_in)
    ws = [ctx.bytes_array(w) for _ in range(copies)]
    x = ctx.array((tokens, n_in), synth.normal(310, tokens * n_in))
    y = ctx.array((tokens, n_out))

    def step(i):
        ctx.linear_q(qtype, ws[i % copies], x, y, n_in, n_out, tokens)

    ms = time_calls(ctx, step, steps, warmup)
    kt = kernel_times(ctx, step, steps)
    ctx.close()
    return ms, kt, w.nbytes + 4 * (n_in + n_out)


def bench_boundary(dim, tokens, steps, warmup):
    """The layer boundary: hidden += delta, y = RmsNormZeroCentered(hidden, w)
    and its Q8_K blocks, over `tokens` rows of dim."""
    ctx = q35mix.Context(q35mix.qwen35_config(num_layers=1, is_recurrent=[1]), 1, 16)
    h = ctx.array((tokens, dim), synth.normal(41, tokens * dim))
    d = ctx.array((tokens, dim), synth.normal(42, tokens * dim))
    w = ctx.array((dim,), 0.02 * synth.normal(43, dim))
    y = ctx.array((tokens, dim))
    q8 = q35mix.DeviceBytes(ctx, np.zeros(q35mix.lib().q35m_q8k_bytes(dim, tokens), np.uint8))

    def step(i):
        ctx.add_rmsnorm(h, d, w, y, q8, dim, tokens, 1e-6)

    ms = time_calls(ctx, step, steps, warmup)
    kt = kernel_times(ctx, step, steps)
    ctx.close()
    # read hidden, delta and w; write hidden, y and the Q8_K blocks
    return ms, kt, 16 * tokens * dim + 4 * dim + q35mix.lib().q35m_q8k_bytes(dim, tokens)


def memcpy_d2d(ctx, dst_ptr, src_ptr, nbytes):
    hip = q35mix.hip()
    hip.hipMemcpyAsync.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
                                   ctypes.c_void_p]
    r = hip.hipMemcpyAsync(ctypes.c_void_p(dst_ptr), ctypes.c_void_p(src_ptr), nbytes, 3,
                           ctypes.c_void_p(ctx.stream))
    if r != 0:
        raise RuntimeError(f"hipMemcpyAsync failed: {r}")


def bench_decode_stack(is_rec, n_seqs, start, n_steps, warmup=4, eager=True, n_sets=8):
    """Decode steps of a mixer stack (layer l is Gated-DeltaNet when is_rec[l],
    GQA otherwise) for n_seqs sequences from context `start`, n_steps tokens.

    Timed two ways over the same inputs: (1) the whole step captured once as
    a decode graph (q35m_decode_graph_create) and replayed per token; its
    inputs sit in one fixed staging block, and each step first copies one of
    n_sets pre-generated input images into it (one device-to-device copy of
    every layer's inputs, inside the timed region; timed alone too); (2) the
    per-layer entry points called one by one (q35m_deltanet_decode /
    q35m_attn_decode, then q35m_advance per sequence), reading the images
    directly.  Lengths are put back to `start` before each timed pass."""
    L = len(is_rec)
    cap = start + n_steps
    ctx = q35mix.Context(q35mix.qwen35_config(num_layers=L, is_recurrent=is_rec), n_seqs, cap)
    block = synth.normal(1234, 4 << 20)       # KV rows ~N(0,1): a 16 MiB block of normals tiled
    wd, wa = synth.deltanet_weights(NK, NV, DK), synth.attn_weights(HD)
    st = synth.deltanet_state(NK, NV, DK)
    for layer in range(L):
        if is_rec[layer]:
            ctx.set_deltanet_weights(layer, wd)
            for s in range(n_seqs):
                ctx.state_write(layer, s, q35mix.STATE_RECURRENT, st["state"])
                ctx.state_write(layer, s, q35mix.STATE_CONV, st["conv_state"])
        else:
            ctx.set_attn_weights(layer, wa)
            for s in range(n_seqs):
                for kind in (q35mix.STATE_KEYS, q35mix.STATE_VALUES):
                    # the whole head-major [kv_heads][capacity][256] block of the (layer, seq)
                    ptr, nbytes = ctx.state_device_ptr(layer, s, kind)
                    off = 0
                    while off < nbytes:
                        n = min(block.nbytes, nbytes - off)
                        q35mix.check(q35mix.lib().q35m_copy_h2d(ctx.handle, ptr + off, block.ctypes.data, n))
                        off += n
    # One input image: every layer's inputs, contiguous.
    shapes = []
    for layer in range(L):
        if is_rec[layer]:
            shapes.append([(n_seqs, CONV_DIM), (n_seqs, VALUE_DIM), (n_seqs, NV), (n_seqs, NV)])
        else:
            shapes.append([(n_seqs, 2 * Q_DIM), (n_seqs, KV_DIM), (n_seqs, KV_DIM)])
    offs, total = [], 0
    for shp in shapes:
        o = []
        for sh in shp:
            o.append(total)
            total += int(np.prod(sh))
        offs.append(o)
    sets = []
    for j in range(n_sets):
        xd = synth.deltanet_inputs(n_seqs, NK, NV, DK, salt=500 + j)
        xa = synth.attn_inputs(n_seqs, NH, NKV, HD, salt=600 + j)
        sets.append(([xd["qkv"], xd["z"], xd["b"], xd["a"]], [xa["q_gate"], xa["k"], xa["v"]]))
    images = []
    for j in range(n_sets):
        host = np.empty(total, np.float32)
        for layer in range(L):
            xs = sets[(j * L + layer) % n_sets][0 if is_rec[layer] else 1]
            for o, x in zip(offs[layer], xs):
                host[o:o + x.size] = x.ravel()
        images.append(ctx.array((total,), host))
    stage = ctx.array((total,))
    outs = [ctx.array((n_seqs, VALUE_DIM if is_rec[layer] else Q_DIM)) for layer in range(L)]

    def views(img):
        return [[q35mix.DeviceView(img, o, sh) for o, sh in zip(offs[layer], shapes[layer])]
                for layer in range(L)]
    stage_v = views(stage)
    img_v = [views(img) for img in images]
    io = [tuple(stage_v[layer]) + ((None,) if not is_rec[layer] else ()) + (outs[layer],) for layer in range(L)]
    seqs = list(range(n_seqs))
    for s in seqs:
        ctx.advance(s, start)

    def rewind():
        ctx.sync()
        for s in seqs:
            ctx.truncate(s, start)

    g = q35mix.DecodeGraph(ctx, seqs, io, cap)

    def graph_step(i):
        memcpy_d2d(ctx, stage.ptr, images[i % n_sets].ptr, total * 4)
        g.run(replay=True)

    def eager_step(i):
        v = img_v[i % n_sets]
        for layer in range(L):
            if is_rec[layer]:
                ctx.deltanet_decode(layer, seqs, *v[layer], outs[layer])
            else:
                ctx.attn_decode(layer, seqs, *v[layer], outs[layer])
        for s in seqs:
            ctx.advance(s, 1)

    def timed(fn):
        for i in range(warmup):
            fn(i)
        rewind()
        e0, e1 = q35mix.Event(), q35mix.Event()
        e0.record(ctx.stream)
        for i in range(n_steps):
            fn(i)
        e1.record(ctx.stream)
        ms = e0.elapsed_ms(e1)
        rewind()
        return ms

    res = {"graph_ms": timed(graph_step)}
    # the staging copies alone
    e0, e1 = q35mix.Event(), q35mix.Event()
    e0.record(ctx.stream)
    for i in range(n_steps):
        memcpy_d2d(ctx, stage.ptr, images[i % n_sets].ptr, total * 4)
    e1.record(ctx.stream)
    res["staging_ms"] = e0.elapsed_ms(e1)
    res["staging_bytes_per_step"] = 2 * total * 4
    if eager:
        res["eager_ms"] = timed(eager_step)
    # Per-kernel times: the graph's launches issued one by one with the timers on.
    ctx.profile(True)
    for i in range(4):
        g.run(replay=False)
    kt = ctx.profile_read()
    ctx.profile(False)
    rewind()
    res["kernels"] = {k: (ms / n, n / 4) for k, (ms, n) in kt.items()}
    g.close()
    ctx.close()
    by = 0
    n_dn = sum(1 for r in is_rec if r)
    n_at = L - n_dn
    for i in range(n_steps):
        by += n_seqs * (n_dn * DN_DECODE_BYTES + n_at * attn_decode_bytes(start + i + 1))
    res["bytes"] = by
    return res


def bench_stack(n_steps=128, warmup=4, n_seqs=8, ctx_len=32768, n_layers=32):
    """32-layer mixer stack, 8 sequences decoding from context 32640 to 32768."""
    is_rec = [(i + 1) % 4 != 0 for i in range(n_layers)]
    return bench_decode_stack(is_rec, n_seqs, ctx_len - n_steps, n_steps, warmup)


# --------------------------------------------------------------------------
# CPU restatement timed beside the GPU
# --------------------------------------------------------------------------

def _oracle():
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    return oracle


def cpu_threads():
    """Worker threads for the CPU attention: the reference's pool default, one
    per physical core (CpuThreadPool.cs:27-29), of the cores this process may
    use, at most 16 (work is split by q head).  Returns (threads, logical
    CPUs available, hardware threads per core)."""
    avail = len(os.sched_getaffinity(0))
    tpc = 1
    try:
        sib = cores = None
        for line in open("/proc/cpuinfo"):
            if line.startswith("siblings") and sib is None:
                sib = int(line.split(":")[1])
            elif line.startswith("cpu cores") and cores is None:
                cores = int(line.split(":")[1])
        if sib and cores:
            tpc = max(1, sib // cores)
    except (OSError, ValueError):
        pass
    return max(1, min(16, avail // tpc)), avail, tpc


def _median_s(fn, reps=20, warm=3):
    for _ in range(warm):
        fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts))


def cpu_baseline_dn_decode():
    """One DeltaNet decode token through one layer on one thread (the
    reference passes no pool to the recurrence, GatedDeltaNetOps.cs:107-120):
    median of 20 after 3 warm-up runs, in microseconds."""
    oracle = _oracle()
    d = oracle.dims()
    w = synth.deltanet_weights(NK, NV, DK)
    st = synth.deltanet_state(NK, NV, DK)
    x = synth.deltanet_inputs(1, NK, NV, DK)
    sec = _median_s(lambda: oracle.deltanet_decode(d, x["qkv"][0], x["z"][0], x["b"][0], x["a"][0], w,
                                                   st["conv_state"], st["state"]))
    return sec * 1e6


def cpu_baseline_attn_decode(threads, pos=8192):
    """One GQA decode token at 8193 rows, scores/softmax/combine on `threads`
    workers (Ops.cs:353-356): median of 20 after 3 warm-up runs, in us."""
    oracle = _oracle()
    d = oracle.dims()
    k, v = synth.kv_prefill(pos, KV_DIM)
    ck = np.zeros((pos + 1, KV_DIM), np.float32)
    cv = np.zeros_like(ck)
    ck[:pos], cv[:pos] = k, v
    x = synth.attn_inputs(1, NH, NKV, HD)
    wts = synth.attn_weights(HD)
    sec = _median_s(lambda: oracle.attn_decode(d, pos, x["q_gate"][0], x["k"][0], x["v"][0], wts, ck, cv,
                                               n_threads=threads, inplace=True))
    return sec * 1e6


def cpu_baseline_attn_prefill(threads, T=2048):
    """One causal GQA prefill of 2048 tokens on `threads` workers, one run:
    tokens/s and seconds."""
    oracle = _oracle()
    d = oracle.dims()
    x = synth.attn_inputs(T, NH, NKV, HD)
    wts = synth.attn_weights(HD)
    z = np.zeros((T, KV_DIM), np.float32)
    t0 = time.perf_counter()
    oracle.attn_prefill(d, 0, T, x["q_gate"], x["k"], x["v"], wts, z, z, n_threads=threads)
    dt = time.perf_counter() - t0
    return T / dt, dt


def cpu_baseline_stack(threads, n_steps=4, n_seqs=8, ctx_len=32768, n_layers=32, total_steps=128):
    """The 32-layer mixer stack on the CPU restatement: n_steps decode steps of
    8 sequences (24 DeltaNet layers on one thread, 8 GQA layers on `threads`
    workers over caches of ~32K rows), extrapolated linearly to 128 steps.
    One K/V cache pair is shared by every (layer, sequence): the CPU cost does
    not depend on the values.  Returns (us per token, seconds measured)."""
    oracle = _oracle()
    d = oracle.dims()
    start = ctx_len - total_steps
    block = synth.normal(1234, 4 << 20)
    ck = np.resize(block, (ctx_len, KV_DIM)).astype(np.float32)
    cv = np.ascontiguousarray(ck[::-1])
    wd, wa = synth.deltanet_weights(NK, NV, DK), synth.attn_weights(HD)
    st = synth.deltanet_state(NK, NV, DK)
    xd = synth.deltanet_inputs(n_seqs, NK, NV, DK, salt=500)
    xa = synth.attn_inputs(n_seqs, NH, NKV, HD, salt=600)
    t0 = time.perf_counter()
    for step in range(n_steps):
        for layer in range(n_layers):
            for s in range(n_seqs):
                if (layer + 1) % 4 != 0:
                    oracle.deltanet_decode(d, xd["qkv"][s], xd["z"][s], xd["b"][s], xd["a"][s], wd,
                                           st["conv_state"], st["state"])
                else:
                    oracle.attn_decode(d, start + step, xa["q_gate"][s], xa["k"][s], xa["v"][s], wa, ck, cv,
                                       n_threads=threads, inplace=True)
    dt = time.perf_counter() - t0
    return dt / n_steps * total_steps / (total_steps * n_seqs) * 1e6, dt


def cpu_baseline_prefill(x, T=2048):
    oracle = _oracle()
    d = oracle.dims()
    w = synth.deltanet_weights(NK, NV, DK)
    st = np.zeros((NV, DK, DK), np.float32)
    t0 = time.perf_counter()
    oracle.deltanet_prefill(d, T, x["qkv"], x["z"], x["b"], x["a"], w, st)
    dt = time.perf_counter() - t0
    return T / dt, dt


def measured_peaks():
    """Ceilings measured on this GPU by libq35probe.so (grid-stride streaming
    read and copy kernels, with plain and with non-temporal accesses, and an
    fp32 MFMA loop), reported beside the datasheet peaks."""
    path = os.path.join(ROOT, "qwen3.5sharp_amd", "libq35probe.so")
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(path)
    out = {}
    for name, fn, args in (("hbm_read_GBps", lib.q35p_hbm_read_gbs, (ctypes.c_size_t(1 << 31), 10, 0)),
                           ("hbm_read_nt_GBps", lib.q35p_hbm_read_gbs, (ctypes.c_size_t(1 << 31), 10, 1)),
                           ("hbm_copy_rw_GBps", lib.q35p_hbm_copy_gbs, (ctypes.c_size_t(1 << 30), 10, 0)),
                           ("hbm_copy_rw_nt_GBps", lib.q35p_hbm_copy_gbs, (ctypes.c_size_t(1 << 30), 10, 1)),
                           ("mfma_f32_TFLOPs", lib.q35p_mfma_f32_tflops, (20000,))):
        v = ctypes.c_double(0.0)
        r = fn(*args, ctypes.byref(v))
        if r != 0:
            raise RuntimeError(f"{name} probe failed ({r})")
        out[name] = v.value
    out["datasheet"] = {"hbm_GBps": HBM_PEAK / 1e9, "mfma_f32_TFLOPs": FP32_PEAK / 1e12}
    return out


def cpu_info():
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return model, os.cpu_count()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", default="", help="comma list of: dn_prefill,dn_decode,attn_decode,"
                                               "attn_prefill,linear_q,boundary,stack,stack_b1,peaks")
    ap.add_argument("--stack-steps", type=int, default=128,
                    help="decode steps of the mixer-stack workload (the context ends at 32768 rows)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="also run one device-to-device copy of MIB MiB (a plain copy kernel "
                         "of known traffic, to scale FETCH_SIZE/WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X only; --gpus {args.gpus} is not supported "
              "(the mixers shard with no exchange inside the layer; see the sharding design)",
              file=sys.stderr)
        sys.exit(2)
    only = set(filter(None, args.only.split(",")))

    def want(name):
        return not only or name in only

    K, W = args.steps, args.warmup
    workloads = {}
    result = None

    if args.copy_calibration:
        nbytes = args.copy_calibration << 20
        ctx = q35mix.Context(q35mix.qwen35_config(num_layers=1, is_recurrent=[1]), 1, 16)
        src, dst = ctx.array((nbytes // 4,)), ctx.array((nbytes // 4,))
        hip = q35mix.hip()
        hip.hipMemcpyAsync.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                       ctypes.c_int, ctypes.c_void_p]
        r = hip.hipMemcpyAsync(ctypes.c_void_p(dst.ptr), ctypes.c_void_p(src.ptr), nbytes, 3,
                               ctypes.c_void_p(ctx.stream))
        if r != 0:
            raise RuntimeError(f"hipMemcpyAsync failed: {r}")
        ctx.sync()
        log(f"[bench] calibration copy: {nbytes} bytes device to device")
        ctx.close()

    if want("dn_prefill"):
        log("[bench] DeltaNet prefill T=2048 ...")
        ms, kt, x = bench_dn_prefill(K, W)      # kt: per-step kernel times
        tok_s = 2048 / (ms / 1e3)
        kname, kms = dominant(kt)
        log(f"[bench] DeltaNet prefill: {ms:.3f} ms/step, {tok_s:.0f} tok/s; kernels {kt}")
        if kname not in DN_PREFILL_KERNELS:
            raise RuntimeError(f"no algorithmic work count for dominant kernel {kname}")
        bound, work, what = DN_PREFILL_KERNELS[kname]
        if bound == "mfma":
            achieved, peak, unit = work / (kms / 1e3) / 1e12, FP32_PEAK / 1e12, "TFLOP/s"
            algo = f"{work} FLOP per launch: {what}"
        else:
            achieved, peak, unit = work / (kms / 1e3) / 1e9, HBM_PEAK / 1e9, "GB/s"
            algo = f"{work} bytes per launch: {what}"
        roof = {"bound": bound, "achieved": achieved, "peak": peak, "unit": unit,
                "frac": achieved / peak, "traffic": measured_traffic(kname),
                "kernel": kname, "kernel_ms": kms, "algorithmic": algo,
                "kernels_ms": {k: v[0] for k, v in kt.items()},
                "kernels_frac": {k: (DN_PREFILL_KERNELS[k][1] / (v[0] / 1e3) /
                                     (FP32_PEAK if DN_PREFILL_KERNELS[k][0] == "mfma" else HBM_PEAK))
                                 for k, v in kt.items() if k in DN_PREFILL_KERNELS}}
        cpu = None
        if not args.no_cpu:
            log("[bench] CPU restatement, one 2048-token DeltaNet prefill layer ...")
            cpu_tok_s, cpu_s = cpu_baseline_prefill(x)
            model, ncpu = cpu_info()
            cpu = {"value": cpu_tok_s, "unit": "tokens/s", "cores": 1, "kind": "port",
                   "sample": f"one full 2048-token DeltaNet prefill layer ({cpu_s:.2f} s, "
                             f"single thread as the reference, {model}, {ncpu} logical CPUs)"}
        result = {"metric": "token-mixer µs/token decode + % HBM peak; prefill tokens/s @T=2048",
                  "value": tok_s, "unit": "tokens/s", "n_gpus": 1, "steps": K, "warmup": W,
                  "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
                  "vs_baseline": None, "dtype": "f32", "data": "synthetic",
                  "config": {"workload": "Gated-DeltaNet prefill, 1 layer, T=2048, batch 1, "
                                         "16 k / 32 v heads, dk=dv=128, conv 4, zero state",
                             "global_batch": 1, "seq_len": 2048, "parallelism": "none"},
                  "roofline": roof, "cpu_baseline": cpu,
                  "prefill_dn_mflop_frac": DN_PREFILL_FLOP / (ms / 1e3) / FP32_PEAK}

    threads, avail, tpc = cpu_threads()
    model, _ = cpu_info()
    cpu_desc = f"{model}, {avail} logical CPUs available, {tpc} threads per core"

    if want("dn_decode"):
        log("[bench] DeltaNet decode batch 1 ...")
        (ms, mean_ms), kt = bench_dn_decode(max(K, 200), max(W, 20))
        kname, kms = dominant(kt)
        workloads["deltanet_decode_b1"] = {
            "us_per_token": ms * 1e3, "us_per_token_mean": mean_ms * 1e3,
            "timing": "median over 20 groups of 10 back-to-back calls",
            "hbm_frac_call": DN_DECODE_BYTES / (ms / 1e3) / HBM_PEAK,
            "kernel": kname, "kernel_us": kms * 1e3,
            "hbm_frac_kernel": DN_DECODE_BYTES / (kms / 1e3) / HBM_PEAK}
        if not args.no_cpu:
            us = cpu_baseline_dn_decode()
            workloads["deltanet_decode_b1"]["cpu_baseline"] = {
                "value": us, "unit": "us/token", "cores": 1, "kind": "port",
                "sample": f"median of 20 single-token decodes of one layer, one thread as the reference "
                          f"({cpu_desc})"}
        log(f"[bench] DeltaNet decode: {workloads['deltanet_decode_b1']}")

    if want("attn_decode"):
        log("[bench] GQA decode at 8193 rows ...")
        (ms, mean_ms), kt = bench_attn_decode(max(K, 200), max(W, 20))
        by = attn_decode_bytes(8193)
        workloads["attn_decode_8193"] = {
            "us_per_token": ms * 1e3, "us_per_token_mean": mean_ms * 1e3,
            "timing": "median over 20 groups of 10 back-to-back calls",
            "hbm_frac_call": by / (ms / 1e3) / HBM_PEAK,
            "kernels_us": {k: v[0] * 1e3 for k, v in kt.items()}}
        if not args.no_cpu:
            us = cpu_baseline_attn_decode(threads)
            workloads["attn_decode_8193"]["cpu_baseline"] = {
                "value": us, "unit": "us/token", "cores": threads, "kind": "port",
                "sample": f"median of 20 single-token decodes at 8193 rows, attention on {threads} "
                          f"workers, one per physical core as the reference's pool ({cpu_desc})"}
        log(f"[bench] GQA decode: {workloads['attn_decode_8193']}")

    if want("attn_prefill"):
        log("[bench] GQA prefill T=2048 ...")
        ms, kt = bench_attn_prefill(K, W)
        workloads["attn_prefill_2048"] = {
            "tokens_per_s": 2048 / (ms / 1e3), "ms": ms,
            "mfma_frac": ATTN_PREFILL_FLOP / (ms / 1e3) / FP32_PEAK,
            "kernels_ms": {k: v[0] for k, v in kt.items()}}
        if not args.no_cpu:
            tok_s_cpu, sec = cpu_baseline_attn_prefill(threads)
            workloads["attn_prefill_2048"]["cpu_baseline"] = {
                "value": tok_s_cpu, "unit": "tokens/s", "cores": threads, "kind": "port",
                "sample": f"one causal 2048-token prefill of one layer ({sec:.2f} s) on {threads} "
                          f"workers ({cpu_desc})"}
        log(f"[bench] GQA prefill: {workloads['attn_prefill_2048']}")

    if want("linear_q"):
        log("[bench] Q4_K projection 2560 -> 8192, 2048 tokens ...")
        ms, kt, by = bench_linear_q(4, 2560, 8192, K, W, 1, tokens=2048)
        macs = 2048 * 2560 * 8192
        workloads["linear_q4k_2560x8192_t2048"] = {
            "ms": ms, "tokens_per_s": 2048 / (ms / 1e3),
            "int8_mfma_frac": 2 * macs / (ms / 1e3) / INT8_PEAK,
            "kernels_ms": {k: v[0] for k, v in kt.items()}}
        log(f"[bench] linear_q4k_2560x8192_t2048: {workloads['linear_q4k_2560x8192_t2048']}")
        log("[bench] Q6_K projection 4096 -> 2560, 2048 tokens ...")
        ms, kt, by = bench_linear_q(6, 4096, 2560, K, W, 1, tokens=2048)
        macs = 2048 * 4096 * 2560
        msb, ktb, _ = bench_linear_q(6, 4096, 2560, K, W, 1, tokens=2048, order=q35mix.PROJ_BLOCK)
        workloads["linear_q6k_4096x2560_t2048"] = {
            "ms": ms, "tokens_per_s": 2048 / (ms / 1e3),
            "int8_mfma_frac": 2 * macs / (ms / 1e3) / INT8_PEAK,
            "kernels_ms": {k: v[0] for k, v in kt.items()},
            "block_order_ms": msb, "block_order_tokens_per_s": 2048 / (msb / 1e3),
            "block_order_int8_mfma_frac": 2 * macs / (msb / 1e3) / INT8_PEAK,
            "block_order_kernels_ms": {k: v[0] for k, v in ktb.items()}}
        log(f"[bench] linear_q6k_4096x2560_t2048: {workloads['linear_q6k_4096x2560_t2048']}")
    if want("boundary"):
        log("[bench] layer boundary (add + RMSNorm + Q8_K), 2048 x 2560 ...")
        ms, kt, by = bench_boundary(2560, 2048, K, W)
        workloads["boundary_2048x2560"] = {
            "us": ms * 1e3, "bytes": by, "hbm_frac_call": by / (ms / 1e3) / HBM_PEAK,
            "kernels_us": {k: v[0] * 1e3 for k, v in kt.items()}}
        log(f"[bench] boundary_2048x2560: {workloads['boundary_2048x2560']}")
    qnames = {1: "stq1_0", 2: "q2_0c", 4: "q4k", 5: "q5k", 6: "q6k", 14: "iq4xs"}
    gemv_kernel = {1: "linear_qt<1>", 2: "linear_qt<2>", 4: "linear_q<4>", 5: "linear_qs<5>",
                   6: "linear_q<6>", 14: "linear_qs<14>"}
    for qtype, n_in, n_out, copies in ((4, 2560, 8192, 32), (6, 4096, 2560, 40), (5, 2560, 8192, 28),
                                       (14, 2560, 8192, 40), (2, 2560, 8192, 60), (1, 2560, 8192, 90)):
        if not want("linear_q"):
            break
        name = f"linear_{qnames[qtype]}_{n_in}x{n_out}"
        log(f"[bench] {qnames[qtype]} projection {n_in} -> {n_out}, one token ...")
        ms, kt, by = bench_linear_q(qtype, n_in, n_out, max(K, 200), max(W, 20), copies)
        kus = {k: v[0] * 1e3 for k, v in kt.items()}
        gemv = gemv_kernel[qtype]
        workloads[name] = {
            "us_per_call": ms * 1e3, "bytes": by, "hbm_frac_call": by / (ms / 1e3) / HBM_PEAK,
            "kernels_us": kus, "hbm_frac_kernel": by / (kus[gemv] / 1e6) / HBM_PEAK}
        log(f"[bench] {name}: {workloads[name]}")

    if want("stack"):
        ns = args.stack_steps
        log(f"[bench] 32-layer mixer stack, 8 seqs x ctx 32768, {ns} decode steps ...")
        r = bench_stack(n_steps=ns)
        ms, by = r["graph_ms"], r["bytes"]
        workloads["stack_decode_8x32k"] = {
            "us_per_token": ms * 1e3 / (ns * 8), "ms_per_step": ms / ns, "steps": ns,
            "timing": "one decode graph (24 DeltaNet + 8 GQA mixers and the length advance) captured once and "
                      "replayed per token; each step first copies its inputs into the graph's staging block "
                      "(included; staging_us_per_step alone)",
            "hbm_frac": by / (ms / 1e3) / HBM_PEAK, "gb_per_step": by / ns / 1e9,
            "staging_us_per_step": r["staging_ms"] * 1e3 / ns,
            "eager_us_per_token": r["eager_ms"] * 1e3 / (ns * 8),
            "eager_hbm_frac": by / (r["eager_ms"] / 1e3) / HBM_PEAK,
            "kernels_us": {k: v[0] * 1e3 for k, v in r["kernels"].items()}}
        if not args.no_cpu:
            log("[bench] CPU restatement, 4 steps of the stack ...")
            us, sec = cpu_baseline_stack(threads)
            workloads["stack_decode_8x32k"]["cpu_baseline"] = {
                "value": us, "unit": "us/token", "cores": threads, "kind": "port",
                "sample": f"4 decode steps of the 32-layer stack x 8 sequences at ~32K rows ({sec:.1f} s), "
                          f"extrapolated linearly to 128 steps; DeltaNet on one thread, attention on "
                          f"{threads} workers ({cpu_desc})"}
        log(f"[bench] stack: {workloads['stack_decode_8x32k']}")

    if want("stack_b1"):
        ns = args.stack_steps
        is_rec = [(i + 1) % 4 != 0 for i in range(32)]
        log(f"[bench] 32-layer mixer stack, batch 1 from ctx 8192, {ns} decode steps ...")
        r = bench_decode_stack(is_rec, 1, 8192, ns)
        ms, by = r["graph_ms"], r["bytes"]
        workloads["stack_decode_b1_8k"] = {
            "us_per_token": ms * 1e3 / ns, "steps": ns,
            "timing": "decode graph of the 32 layers replayed per token (staging copy included), contexts "
                      "8193 to 8320 rows",
            "hbm_frac": by / (ms / 1e3) / HBM_PEAK, "mb_per_token": by / ns / 1e6,
            "staging_us_per_step": r["staging_ms"] * 1e3 / ns,
            "eager_us_per_token": r["eager_ms"] * 1e3 / ns,
            "eager_hbm_frac": by / (r["eager_ms"] / 1e3) / HBM_PEAK,
            "kernels_us": {k: v[0] * 1e3 for k, v in r["kernels"].items()}}
        log(f"[bench] stack b1: {workloads['stack_decode_b1_8k']}")
        # One mixer kind per graph, per layer: DeltaNet decode (160 layers, so
        # the states exceed the MALL) and GQA decode at 8193-8320 rows.
        log("[bench] per-layer decode in a graph: 160 DeltaNet layers, batch 1 ...")
        r = bench_decode_stack([True] * 160, 1, 0, ns)
        per = (r["graph_ms"] - r["staging_ms"]) * 1e3 / (ns * 160)
        workloads.setdefault("deltanet_decode_b1", {}).update({
            "graph_us_per_layer": per, "graph_hbm_frac": DN_DECODE_BYTES / (per / 1e6) / HBM_PEAK,
            "graph_timing": "160-layer decode graph replayed 128 times; (time - staging copies) / 160 layers",
            "eager_us_per_layer_in_loop": r["eager_ms"] * 1e3 / (ns * 160)})
        log(f"[bench] DeltaNet decode per layer in a graph: {per:.2f} us")
        log("[bench] per-layer decode in a graph: 8 GQA layers at 8193-8320 rows, batch 1 ...")
        r = bench_decode_stack([False] * 8, 1, 8192, ns)
        per = (r["graph_ms"] - r["staging_ms"]) * 1e3 / (ns * 8)
        workloads.setdefault("attn_decode_8193", {}).update({
            "graph_us_per_layer": per,
            "graph_hbm_frac": (r["bytes"] / (ns * 8)) / (per / 1e6) / HBM_PEAK,
            "graph_timing": "8-layer decode graph replayed 128 times (rows 8193-8320); "
                            "(time - staging copies) / 8 layers",
            "eager_us_per_layer_in_loop": r["eager_ms"] * 1e3 / (ns * 8)})
        log(f"[bench] GQA decode per layer in a graph: {per:.2f} us")

    if result is None:
        result = {"metric": "token-mixer µs/token decode + % HBM peak; prefill tokens/s @T=2048",
                  "value": None, "unit": "tokens/s", "n_gpus": 1, "steps": K, "warmup": W,
                  "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
                  "dtype": "f32", "data": "synthetic", "config": {"workload": "partial run"}}
    result["workloads"] = workloads
    if not only or "peaks" in only:
        log("[bench] measured device ceilings ...")
        result["measured_peaks"] = measured_peaks()
        log(f"[bench] measured: {result['measured_peaks']}")
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
