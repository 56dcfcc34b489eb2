#!/usr/bin/env python3
"""Benchmark of the MXFP4 routed-expert FFN on one MI355X (gfx950).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-sweep] [--no-cpu]
    python bench.py --only {decode,single,verify,prefill,fp8,grouped,producers,dropin,pack,remote,copy}   # one workload (for profilers), one JSON line

A step is one routed-expert FFN over one batch of synthetic tokens: softmax top-6 routing of [T, 256] logits,
dispatch, fp8 input transform, w1/w3 grouped GEMV with the SwiGLU epilogue, w2 grouped GEMV, combine to bf16
[T, 4096] -- everything uh_mx_moe_forward enqueues. The headline workload is BASELINE configs[1] (decode, T = 8
tokens, 256 experts of MXFP4 w1/w3 [2048, 4096] + w2 [4096, 2048]); inputs and weights are resident in HBM before
the timed region. Each step takes the next of R rotating (x, logits) sets, so consecutive steps route to different
experts and the touched weights (~590 MB per step) do not stay in the 256 MB Infinity Cache.

Prints ONE JSON line (rank 0, N = 1). `roofline` is for the dominant kernel (the w1/w3 + SwiGLU grouped GEMV),
timed with HIP events on the launch stream inside the timed region; `cpu_baseline` is the repository's CPU oracle
(oracle/, the reference arithmetic) on a bounded sample of the same workload. `workloads` adds the other BASELINE
configurations (single GEMV, verify M = 64, prefill M = 4096, fp8 dense M = 1 / 64 / 4096), each timed the same way.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

D, I, E, TOPK = 4096, 2048, 256, 6
MAT_BYTES = I * D // 2 + I * D // 32  # 4,456,448: codes + e8m0 scales of one MXFP4 [2048, 4096] matrix
EXPERT_BYTES = 3 * MAT_BYTES
LIMIT = 10.0
HBM_PEAK_GBS = 8000.0
# HBM bytes per launch of the dominant kernel (w1/w3 GEMV, this seeded workload): FETCH_SIZE + WRITE_SIZE from two
# rocprofv3 --pmc runs, scaled by the same counters on a 1 GiB device copy (profiles/hbm_traffic_pmc.md).
GEMV_TRAFFIC_BYTES = 383.9e6
BF16_PEAK_TFLOPS = 2500.0
GW_G, GW_R, GW_K = 8, 1024, 4096  # the DSV4 wo_a shape (o_groups, o_lora_rank, heads x head_dim / o_groups)
FP8_PEAK_TFLOPS = 5000.0  # the block-scaled fp8 x fp4 MFMA runs at the fp8 rate (4.29 PFLOP/s sustained, measured)


def to_bf16(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


class Weights:
    """256 experts of synthetic MXFP4 weights in the tile-major layout: code bytes uniform over 0..255 (every
    nibble uniform over the 16 e2m1 codes), e8m0 scales uniform in [119, 125] (2^-8 .. 2^-2), written on the device."""

    def __init__(self, seed=0):
        from unholy_amd.device import DeviceBuffer, fill_random_bytes, pointer_table
        self.buf = DeviceBuffer(E * EXPERT_BYTES)
        base = self.buf.ptr
        shapes = [(I, D), (I, D), (D, I)]
        tab = [[None] * E for _ in range(6)]
        off = 0
        for e in range(E):
            for m, (n, k) in enumerate(shapes):
                cb, sb = n * k // 2, n * k // 32
                tab[2 * m][e] = base + off
                tab[2 * m + 1][e] = base + off + cb
                off += cb + sb
        fill_random_bytes(self.buf, E * EXPERT_BYTES, seed, 0, 255)
        for e in range(E):  # scales
            for m in range(3):
                fill_random_bytes(tab[2 * m + 1][e], shapes[m][0] * shapes[m][1] // 32, seed + 1 + 3 * e + m, 119, 125)
        self.ptrs = tab
        self.table = pointer_table([p for row in tab for p in row])


def routing_sets(rng, T, R, bias_scale=0.0, disjoint=False):
    """R (x, logits) sets for rotating steps. disjoint: consecutive sets (the last and the first included) route to
    disjoint experts -- the logits of the experts the neighbouring sets pick are lowered below every other logit
    -- so no step's weights can come from a cache the step before it filled (the 256 MB Infinity Cache holds part
    of a ~595 MB decode step)."""
    sets = []
    bias = rng.standard_normal(E).astype(np.float32) * np.float32(bias_scale) if bias_scale else None
    picked = []
    for i in range(R):
        x = to_bf16(rng.standard_normal((T, D), dtype=np.float32))
        logits = rng.standard_normal((T, E), dtype=np.float32)
        if bias is not None:
            logits = logits + bias
        if disjoint:
            avoid = set(picked[-1]) if picked else set()
            if i == R - 1 and picked:
                avoid |= set(picked[0])
            if avoid:
                logits[:, sorted(avoid)] -= np.float32(1000.0)
            picked.append(set(distinct_experts(logits)[1].ravel().tolist()))
        sets.append((x, logits))
    return sets


def distinct_experts(logits):
    """Experts a softmax top-6 step touches (selection by logit, as the router)."""
    sel = np.argsort(-logits, axis=1, kind="stable")[:, :TOPK]
    return len(np.unique(sel)), sel


class MoeRunner:
    def __init__(self, w, sets):
        from unholy_amd import call
        from unholy_amd.device import DeviceBuffer, Event
        self.call, self.w = call, w
        self.T = sets[0][0].shape[0]
        self.dev = [(DeviceBuffer.from_array(x), DeviceBuffer.from_array(l)) for x, l in sets]
        self.U = [distinct_experts(l)[0] for _, l in sets]
        self.ws_bytes = call("uh_mx_moe_workspace_size", self.T, TOPK, E, D, I)
        self.ws = DeviceBuffer(self.ws_bytes)
        self.out = DeviceBuffer(self.T * D * 2)
        self.ev = []  # per timed step: events around the w1/w3 + SwiGLU GEMV
        self.evarr = (ctypes.c_void_p * 6)()
        self.Event = Event

    def step(self, i, stage_events=False):
        x, l = self.dev[i % len(self.dev)]
        if stage_events:
            while len(self.ev) <= i:
                self.ev.append((self.Event(), self.Event()))
            self.evarr[2], self.evarr[3] = self.ev[i][0].handle, self.ev[i][1].handle
        self.call("uh_mx_moe_forward_ev", x, l, self.T, TOPK, E, D, I, self.w.table, LIMIT, self.ws, self.ws_bytes,
                  self.out, None, None, None, self.evarr if stage_events else None)


def bench_moe_graph(w, T, steps, warmup, rng, R=8, bias=0.0):
    """ms per step of the same routed-expert FFN with the R rotating steps captured as one HIP graph and replayed
    (the serving loop's form: every kernel of every step runs, the host enqueues one graph per R steps)."""
    sets = routing_sets(rng, T, R, bias, disjoint=T <= 8)
    r = MoeRunner(w, sets)

    def fn(i, stream):
        x, l = r.dev[i % len(r.dev)]
        r.call("uh_mx_moe_forward", x, l, r.T, TOPK, E, D, I, r.w.table, LIMIT, r.ws, r.ws_bytes, r.out, None, None,
               stream.handle)

    return dict(ms=time_graph(fn, steps, warmup, per_graph=R), U=float(np.mean(r.U)))


def time_steps(fn, steps, warmup, timed_fn=None):
    """Total ms of `steps` calls after `warmup` (timed_fn, if given, is the form used inside the timed region)."""
    from unholy_amd.device import Event, synchronize
    for i in range(warmup):
        fn(i)
    synchronize()
    a, b = Event(), Event()
    a.record()
    for i in range(steps):
        (timed_fn or fn)(i)
    b.record()
    b.synchronize()
    return a.elapsed_ms(b)


def time_graph(fn, steps, warmup, per_graph=32):
    """Per-step ms of short steps: `per_graph` steps fn(i, stream) captured as one HIP graph (the host enqueues a
    graph, not one launch per kernel, so the timing is the GPU's), replayed to cover `steps` (rounded up to whole
    graphs) after `warmup` steps' worth of replays; events on the capture stream."""
    from unholy_amd.device import Event, Graph, Stream
    st = Stream()
    for i in range(per_graph):  # one eager pass first: an entry point may allocate its workspace (not under capture)
        fn(i, st)
    st.synchronize()
    g = Graph(st, lambda: [fn(i, st) for i in range(per_graph)])
    reps = max(1, -(-steps // per_graph))
    for _ in range(max(1, -(-warmup // per_graph))):
        g.launch()
    st.synchronize()
    a, b = Event(), Event()
    a.record(st)
    for _ in range(reps):
        g.launch()
    b.record(st)
    b.synchronize()
    return a.elapsed_ms(b) / (reps * per_graph)


def bench_moe(w, T, steps, warmup, rng, R=8, bias=0.0, stage=False):
    from unholy_amd.device import synchronize
    sets = routing_sets(rng, T, R, bias, disjoint=T <= 8)
    r = MoeRunner(w, sets)
    ms = time_steps(lambda i: r.step(i), steps, warmup, (lambda i: r.step(i, True)) if stage else None)
    synchronize()
    stage_ms = [(r.ev[i][0].elapsed_ms(r.ev[i][1]), r.U[i % R]) for i in range(steps)] if stage else []
    u_mean = float(np.mean([r.U[i % R] for i in range(steps)]))
    return dict(ms=ms / steps, U=u_mean, stage=stage_ms, runner=r)


class DropinRunner:
    """The reference's own call sequence for the native MXFP4 experts (src/model/forward_ref.hip:455-470, with
    UNHOLY_MX_GEMV_TOKENS unset: a GEMV step for T <= 8 tokens) through the drop-in entry points: routing
    (uh_route_softmax), dispatch (uh_moe_dispatch_small for T <= 32, else count / plan / scatter; tiles of
    kMxGemvTileRows = 8 rows for a GEMV step, else 128), mx_xform_in (the pair rows gathered and fake-quantized to
    bf16), then
      - T <= 8: mx_grouped_gemv for w1 / w3 with the SwiGLU epilogue writing hh (MxGlu), mx_grouped_gemv for w2;
      - larger T, glu (the reference's gfx11 order): mx_grouped_gemm_glu, then mx_grouped_gemm for w2;
      - larger T, not glu (its gfx12 order): mx_grouped_gemm for w1 and w3 (two outputs), mx_swiglu, mx_grouped_gemm
        for w2;
    each grouped call with max_rows = min(T, 128) (an expert has at most one row per token); then moe_combine."""

    def __init__(self, w, sets, glu=True):
        from unholy_amd import call
        from unholy_amd.device import DeviceBuffer, pointer_table
        self.call, self.w = call, w
        T = self.T = sets[0][0].shape[0]
        P = self.P = T * TOPK
        self.gemv, self.glu = T <= 8, glu
        self.tile_rows = 8 if self.gemv else 128
        self.max_tiles = min(P, E + P // self.tile_rows + 1)
        self.dev = [(DeviceBuffer.from_array(x), DeviceBuffer.from_array(l)) for x, l in sets]
        self.U = [distinct_experts(l)[0] for _, l in sets]
        B = DeviceBuffer
        self.sel, self.wt = B(P * 4), B(P * 4)
        self.plan, self.tiles = B(20), B(self.max_tiles * 12)
        self.eidx, self.ewt, self.row_expert, self.pidx = B(P * 4), B(P * 4), B(P * 4), B(P * 4)
        self.count, self.off, self.fill = B(E * 4), B(E * 4), B(E * 4)
        self.xa, self.hh, self.pair = B(P * D * 2), B(P * I * 2), B(P * D * 2)
        self.g, self.u = (B(P * I * 2), B(P * I * 2)) if not (self.gemv or glu) else (None, None)
        self.out = B(T * D * 2)
        t = w.ptrs
        self.tab = [pointer_table(t[i]) for i in range(6)]

    def step(self, i, stream=None):
        c, T, P, st = self.call, self.T, self.P, (stream.handle if stream is not None else None)
        x, l = self.dev[i % len(self.dev)]
        w1, s1, w3, s3, w2, s2 = self.tab
        ntd = self.plan.ptr + 8  # MoePlan::n_local_tiles
        c("uh_route_softmax", l, self.sel, self.wt, T, E, TOPK, st)
        if T <= 32:
            c("uh_moe_dispatch_small", self.sel, self.wt, T, TOPK, E, P, self.max_tiles, self.tile_rows, self.plan,
              self.tiles, self.eidx, self.ewt, self.row_expert, self.pidx, None, None, None, 0.0, None, None, None,
              None, None, 0, st)
        else:
            self.count.zero(st)
            c("uh_moe_count", self.sel, T, TOPK, self.count, E, st, None)
            c("uh_moe_plan", self.count, None, E, P, self.plan, self.tiles, None, self.off, self.fill, self.max_tiles,
              st, self.tile_rows)
            c("uh_moe_scatter", self.sel, self.wt, T, TOPK, self.off, self.fill, self.eidx, self.ewt, self.row_expert,
              self.pidx, st)
        c("uh_mx_xform_in", x, D, self.row_expert, s1, self.xa, P, D, st, self.eidx)
        rows = min(T, 128)
        if self.gemv:
            c("uh_mx_grouped_gemv", self.xa, D, self.tiles, self.max_tiles, w1, s1, None, I, I, st, ntd, w3, s3, None,
              rows, self.ewt, self.row_expert, s2, self.hh, LIMIT, None)
            c("uh_mx_grouped_gemv", self.hh, I, self.tiles, self.max_tiles, w2, s2, self.pair, D, D, st, ntd, None,
              None, None, rows, None, None, None, None, 0.0, None)
        else:
            if self.glu:
                c("uh_mx_grouped_gemm_glu", self.xa, D, self.tiles, self.max_tiles, w1, s1, w3, s3, I, self.ewt,
                  self.row_expert, s2, self.hh, LIMIT, st, ntd)
            else:
                c("uh_mx_grouped_gemm", self.xa, D, self.tiles, self.max_tiles, w1, s1, self.g, I, I, st, ntd, w3, s3,
                  self.u, rows)
                c("uh_mx_swiglu", self.g, self.u, self.ewt, self.row_expert, s2, self.hh, P, I, LIMIT, st)
            c("uh_mx_grouped_gemm", self.hh, I, self.tiles, self.max_tiles, w2, s2, self.pair, D, D, st, ntd, None,
              None, None, rows)
        c("uh_moe_combine", self.pair, self.pidx, None, self.out, T, TOPK, D, st)


def bench_dropin(w, T, steps, warmup, rng, R=8, bias=0.0, glu=True):
    """ms per step of the reference's call sequence (DropinRunner); T <= 32 as HIP-graph replays (the GPU's time, not
    the host's launch rate of seven ctypes calls), larger T eagerly (memsets are not captured)."""
    sets = routing_sets(rng, T, R, bias, disjoint=T <= 8)
    r = DropinRunner(w, sets, glu)
    if T <= 32:
        return dict(ms=time_graph(lambda i, st: r.step(i, st), steps, warmup, per_graph=R), U=float(np.mean(r.U)))
    return dict(ms=time_steps(lambda i: r.step(i), steps, warmup) / steps, U=float(np.mean(r.U)))


def bench_single_gemv(w, steps, warmup, rng):
    """x [1, 4096] through act_quant, one MXFP4 [2048, 4096] matrix (a 1-row tile), rotating
    over the 256 experts' w1 matrices (1.1 GB) so the weights come from HBM."""
    from unholy_amd import call
    from unholy_amd.device import DeviceBuffer
    x = to_bf16(rng.standard_normal((1, D), dtype=np.float32))
    dx = DeviceBuffer.from_array(x)
    q, qs = DeviceBuffer(D), DeviceBuffer(D // 128)
    call("uh_act_quant_fp8", dx, D, q, qs, 1, D, 128, None)
    tiles = [DeviceBuffer.from_array(np.array([[e, 0, 1]], np.int32)) for e in range(E)]
    out = DeviceBuffer(I * 2)
    wt, st = w.table.ptr, w.table.ptr + 8 * E

    def fn(i, stream):
        call("uh_mx_grouped_gemv_q", q, qs, D, tiles[i % E], 1, wt, st, out, I, I, stream.handle, None, None, None, None,
             1, None, None, None, None, None, None, 0.0)

    return time_graph(fn, steps, warmup, per_graph=64)


def bench_fp8_dense(M, steps, warmup, rng, copies, form="fused"):
    """A bf16 [M, 4096] -> e4m3 per 1x128 with fp32 scales (in the step); W e4m3 [4096, 4096]
    with fp32 128x128 scales (quantized once from N(0, 0.02)); rotating over `copies` weight copies. form "fused":
    for M <= 16 the quantization inside the GEMV launch (uh_gemm_fp8_f32s_x), otherwise as "two"; "two":
    act_quant_fp8_f32s then uh_gemm_fp8_f32s (the reference's call sequence)."""
    from unholy_amd import call
    from unholy_amd.device import DeviceBuffer
    N = K = 4096
    wf = DeviceBuffer.from_array(rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
    wq = [DeviceBuffer(N * K) for _ in range(copies)]
    ws = DeviceBuffer((N // 128) * (K // 128) * 4)
    for c in wq:
        call("uh_quant_weight_fp8_f32s", wf, c, ws, N, K, None)
    del wf
    x = DeviceBuffer.from_array(to_bf16(rng.standard_normal((M, K), dtype=np.float32)))
    q, sa = DeviceBuffer(M * K), DeviceBuffer(M * (K // 128) * 4)
    c = DeviceBuffer(M * N * 2)

    def fn(i, stream):
        if form == "fused" and M <= 16:
            call("uh_gemm_fp8_f32s_x", x, K, wq[i % copies], ws, c, N, M, N, K, stream.handle)
            return
        call("uh_act_quant_fp8_f32s", x, K, q, sa, M, K, 128, stream.handle)
        call("uh_gemm_fp8_f32s", q, sa, wq[i % copies], ws, c, N, M, N, K, stream.handle)

    return time_graph(fn, steps, warmup, per_graph=copies)


def bench_grouped_fp8w(M, steps, warmup, rng, copies):
    """The reference's wo_a projection (forward_ref.hip:1012-1022), grouped "mgk,grk->mgr" at the DSV4 shape: a bf16
    [M, 8, 4096], w e4m3 [8 x 1024, 4096] (32 MiB) with 128 x 128 e8m0 scales, c bf16 [M, 8, 1024]; through
    uh_gemm_grouped_fp8w_wmma (the GEMV for M <= 16, the row-tile kernel for 16 < M <= 160, the tiled MFMA GEMM above),
    rotating over `copies` weight copies
    so that they are read from HBM."""
    from unholy_amd import call
    from unholy_amd.device import DeviceBuffer
    G, R, K = GW_G, GW_R, GW_K
    wq = [DeviceBuffer(G * R * K) for _ in range(copies)]
    for i, c in enumerate(wq):
        call("uh_fill_random_bytes", c, G * R * K, 100 + i, 0, 126, None)  # finite e4m3 codes
    sw = DeviceBuffer.from_array(rng.integers(118, 126, (G * R // 128, K // 128), dtype=np.uint8))
    a = DeviceBuffer.from_array(to_bf16(rng.standard_normal((M, G, K), dtype=np.float32)))
    c = DeviceBuffer(M * G * R * 2)

    def fn(i, stream):
        call("uh_gemm_grouped_fp8w_wmma", a, wq[i % copies], sw, c, M, G, R, K, stream.handle)

    return time_graph(fn, steps, warmup, per_graph=copies)


def bench_producers(rows, steps, warmup, rng):
    """The fused activation producers at D = 4096: rmsnorm_quant_slices (rmsnorm + act_quant_fp8 of its output) of
    `rows` rows, and quant_remote_tokens of `rows` gathered rows (every token remote). Returns ms per call of each."""
    import ctypes
    from unholy_amd import call
    from unholy_amd.device import DeviceBuffer
    x = DeviceBuffer.from_array(to_bf16(rng.standard_normal((rows, D), dtype=np.float32)))
    w = DeviceBuffer.from_array(to_bf16(rng.standard_normal(D, dtype=np.float32)))
    y, q, qs = DeviceBuffer(rows * D * 2), DeviceBuffer(rows * D), DeviceBuffer(rows * D // 128)
    u2t = DeviceBuffer.from_array(rng.permutation(rows).astype(np.int32))
    plan = DeviceBuffer.from_array(np.array([6 * rows, 0, 0, 0, rows], np.int32))
    done = ctypes.c_int(0)
    t_norm = time_graph(lambda i, st: call("uh_rmsnorm_quant_slices", x, D, w, y, D, q, qs, rows, D, 1e-6,
                                           ctypes.byref(done), st.handle), steps, warmup)
    t_rq = time_graph(lambda i, st: call("uh_quant_remote_tokens", x, D, u2t, plan, q, qs, rows, st.handle),
                      steps, warmup)
    return t_norm, t_rq


def producers_entry(rows, t_norm, t_rq):
    b_norm = rows * D * (2 + 2 + 1) + rows * D // 128 + D * 2  # x in, y out, codes, scales, weights
    b_rq = rows * D * (2 + 1) + rows * D // 128
    return {"rmsnorm_quant_slices": {"ms": t_norm, "GBps": b_norm / (t_norm * 1e-3) / 1e9},
            "quant_remote_tokens": {"ms": t_rq, "GBps": b_rq / (t_rq * 1e-3) / 1e9}}


def bench_remote(T, steps, warmup, rng):
    """The remote-expert transport kernels at D = 4096, K = 6, E = 256 with every other expert held elsewhere (the
    remote side's buffers are device buffers on one GPU). T <= 32: moe_dispatch_small with every remote-side output
    (staging, compact tokens, their bf16 rows and fp8 codes). All T: remote_tokens, remote_combine and
    moe_combine_partial_link. Returns ms per call and algorithmic bytes per call of each."""
    import oracle
    from unholy_amd import call
    from unholy_amd.device import DeviceBuffer
    E_, K_ = 256, 6
    P = T * K_
    sel = np.stack([rng.permutation(E_)[:K_] for _ in range(T)]).astype(np.int32)
    wt = rng.random((T, K_)).astype(np.float32)
    resident = (np.arange(E_) % 2).astype(np.uint8)
    d = oracle.dispatch(sel, wt, E_, 8 if T <= 32 else 128, resident)
    rt = oracle.remote_tokens(d["pidx"], d["eidx"], d["plan"][1])
    U, r0 = rt["U"], int(d["plan"][1])
    plan = d["plan"].copy()
    plan[4] = U
    dv = DeviceBuffer.from_array
    dplan, dpidx, deidx, dtok2u = dv(plan), dv(d["pidx"]), dv(d["eidx"]), dv(rt["tok2u"])
    tok2u, u2t, p2u, u2p = DeviceBuffer(T * 4), DeviceBuffer(T * 4), DeviceBuffer(P * 4), DeviceBuffer(P * 4)
    pair_out = dv(to_bf16(rng.standard_normal((P, D), dtype=np.float32)))
    shared = dv(to_bf16(rng.standard_normal((T, D), dtype=np.float32)))
    partial, out = DeviceBuffer(T * D * 2), DeviceBuffer(T * D * 2)
    du2p = dv(rt["u2p"] if U else np.full((1, K_), -1, np.int32))
    res = {"T": T, "remote0": r0, "remote_tokens_U": U}
    # remote_tokens rewrites plan[4] with the same U, so the later kernels see the oracle's count
    t = time_graph(lambda i, st: call("uh_remote_tokens", dpidx, deidx, T, K_, dplan, tok2u, u2t, p2u, u2p,
                                      st.handle), steps, warmup)
    res["remote_tokens"] = {"ms": t, "bytes": P * 4 * 2 + T * 4 * 2 + (P - r0) * 4 + U * K_ * 4}
    t = time_graph(lambda i, st: call("uh_remote_combine", pair_out, du2p, dplan, partial, K_, D, T, st.handle),
                   steps, warmup)
    b = (P - r0) * D * 2 + U * D * 2
    res["remote_combine"] = {"ms": t, "bytes": b, "GBps": b / (t * 1e-3) / 1e9}
    t = time_graph(lambda i, st: call("uh_moe_combine_partial_link", pair_out, dpidx, dplan, dtok2u, partial, shared,
                                      out, T, K_, D, None, None, None, 0, st.handle), steps, warmup)
    b = r0 * D * 2 + U * D * 2 + T * D * 2 * 2
    res["moe_combine_partial_link"] = {"ms": t, "bytes": b, "GBps": b / (t * 1e-3) / 1e9}
    if T <= 32:
        mt = P + E_
        o = [DeviceBuffer(n) for n in (20, mt * 12, mt * 12, P * 4, P * 4, P * 4, P * 4, 20, mt * 12, P * 4,
                                       P * 4, T * D * 2, T * D, T * D // 128, 4)]
        x, dsel, dwt, dres = dv(to_bf16(rng.standard_normal((T, D), dtype=np.float32))), dv(sel), dv(wt), \
            dv(resident)
        t = time_graph(lambda i, st: call(
            "uh_moe_dispatch_small_remote", dsel, dwt, T, K_, E_, P, mt, 8, o[0], o[1], o[2], o[3], o[4], o[5], o[6],
            dres, None, None, 0.0, 1, 1, tok2u, u2t, p2u, u2p, o[7], o[8], o[9], o[10], x, D, o[11], o[12], o[13],
            o[14], i + 1, st.handle), steps, warmup)
        res["moe_dispatch_small_remote"] = {"ms": t}
    return res


def bench_pack(n_experts=16, reps=3):
    """The expert pack's loader: a pack of n_experts experts of the headline shape (13.4 MB each) written to a
    temporary file (its pages stay in the host's page cache), then its slots loaded into device memory by the
    loader's reader threads through pinned staging, with and without the per-slot xxh64 check. Returns GB/s of slot bytes (best of
    reps), host page cache to HBM."""
    import ctypes
    import tempfile
    from unholy_amd import call
    from unholy_amd.device import DeviceBuffer, synchronize
    rng = np.random.default_rng(77)
    parts = []
    for _ in range(n_experts):
        for rows, cols in ((I, D), (I, D), (D, I)):
            parts.append(rng.integers(0, 256, rows * cols // 2, dtype=np.uint8))
            parts.append(rng.integers(119, 126, rows * cols // 32, dtype=np.uint8))
    ptrs = (ctypes.c_void_p * len(parts))(*[a.ctypes.data for a in parts])
    with tempfile.TemporaryDirectory() as tmp:
        path = (tmp + "/experts.pack").encode()
        call("uh_pack_write", path, 1, 0, n_experts, I, D, D, I, ptrs, 0, 0)
        del parts
        dst = DeviceBuffer(n_experts * EXPERT_BYTES)
        out = {"experts": n_experts, "bytes": n_experts * EXPERT_BYTES}
        for verify in (0, 1):
            best = None
            for _ in range(reps):
                t0 = time.perf_counter()
                call("uh_pack_load", path, 0, n_experts, dst, EXPERT_BYTES, verify, 0, None)
                synchronize()
                dt = time.perf_counter() - t0
                best = dt if best is None else min(best, dt)
            out["GBps_verified" if verify else "GBps"] = n_experts * EXPERT_BYTES / best / 1e9
        return out


def grouped_entry(M, ms):
    G, R, K = GW_G, GW_R, GW_K
    wbytes = G * R * K + (G * R // 128) * (K // 128)
    e = {"ms": ms, "tokens_per_s": M / (ms * 1e-3), "TFLOPs": 2 * M * G * R * K / (ms * 1e-3) / 1e12,
         "GBps_weights": wbytes / (ms * 1e-3) / 1e9}
    # 2 M flop per weight byte: below the bf16 ridge (~312 flop/B) the weight stream bounds the call
    if 2 * M * G * R * K / wbytes < BF16_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9):
        e["frac_hbm_peak"] = e["GBps_weights"] / HBM_PEAK_GBS
    else:
        e["frac_bf16_mfma_peak"] = e["TFLOPs"] / BF16_PEAK_TFLOPS
    return e


def cpu_model():
    """The host CPU as /proc/cpuinfo names it: model name, family / model / stepping, logical CPUs, the clock the
    kernel reports, and this process's CPU affinity."""
    info = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k = k.strip()
                if k in ("model name", "cpu family", "model", "stepping", "cpu MHz") and k not in info:
                    info[k] = v.strip()
                if k == "processor":
                    info["logical"] = info.get("logical", 0) + 1
    except OSError:
        return "unknown"
    try:
        aff = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        aff = os.cpu_count() or 1
    return (f"{info.get('model name', 'unknown')} (family {info.get('cpu family', '?')}, model "
            f"{info.get('model', '?')}, stepping {info.get('stepping', '?')}; {info.get('logical', '?')} logical CPUs, "
            f"{aff} in this process's affinity; {info.get('cpu MHz', '?')} MHz reported)")


def cpu_threads():
    """Host threads for the CPU oracle: the cores this process may run on, at most 16 (a one-GPU box's CPU share)."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def _host_experts(rng, touched):
    experts = [None] * E
    for e in touched:
        ex = {}
        for (wn, sn), (n, k) in ((("w1", "s1"), (I, D)), (("w3", "s3"), (I, D)), (("w2", "s2"), (D, I))):
            ex[wn] = rng.integers(0, 256, n * k // 2, dtype=np.uint8)
            ex[sn] = rng.integers(119, 126, n * k // 32, dtype=np.uint8)
        experts[e] = ex
    return experts


def _timed(fn, min_s, max_reps=50):
    """(reps, seconds) of back-to-back calls until min_s seconds or max_reps calls."""
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= min_s or reps >= max_reps:
            return reps, dt


def cpu_baselines(min_s=1.0):
    """The CPU oracle (oracle/uh_oracle.cpp: the reference's arithmetic restated in C++, the same code the parity
    tests check against) on every BASELINE configuration, at 1 thread and at cpu_threads() threads, on the same
    kind of seeded synthetic inputs as the GPU workloads. Each figure is tokens (rows) per second of the whole
    workload. configs[3] (T = 4096) and configs[4] at M = 4096 run a sample (4 experts' rows; 64 rows) and are
    extrapolated linearly in rows, labelled so. About 20-30 s of CPU time in all."""
    import oracle
    rng = np.random.default_rng(1234)
    nt = cpu_threads()
    out = {"cpu_model": cpu_model(), "threads": nt, "kind": "port"}

    def both(name, fn, tokens, note, scale=1.0):
        e = {"sample": note}
        for th in (1, nt):
            reps, dt = _timed(lambda: fn(th), min_s)
            one = th == 1 and nt > 1
            e["tokens_per_s_1t" if one else "tokens_per_s"] = tokens * reps / (dt * scale)
            e["seconds_per_step_1t" if one else "seconds_per_step"] = dt * scale / reps
        e["threads"] = nt
        out[name] = e

    # one MXFP4 GEMV (act_quant of x, then [2048, 4096] weights)
    x1 = to_bf16(rng.standard_normal((1, D), dtype=np.float32))
    w0 = rng.integers(0, 256, (I, D // 2), dtype=np.uint8)
    s0 = rng.integers(119, 126, (I, D // 32), dtype=np.uint8)

    def gemv0(th):
        q, qs = oracle.act_quant_fp8(x1)
        oracle.gemm_a8w4(q, qs, w0, s0, I, threads=th)

    both("configs0_single_gemv_M1", gemv0, 1, "act_quant + one [2048, 4096] MXFP4 GEMV")
    # configs[1], [2]: the whole routed-expert FFN step (routing, dispatch, act_quant, w1/w3, SwiGLU, w2, combine)
    for name, T, bias in (("configs1_moe_decode_T8", 8, 0.0), ("configs2_moe_verify_T64", 64, 0.5)):
        x = to_bf16(rng.standard_normal((T, D), dtype=np.float32))
        logits = rng.standard_normal((T, E), dtype=np.float32)
        if bias:
            logits = logits + rng.standard_normal(E, dtype=np.float32) * np.float32(bias)
        sel, wt = oracle.route_softmax(logits, TOPK)
        touched = sorted(set(sel.ravel().tolist()))
        experts = _host_experts(rng, touched)
        both(name, lambda th: oracle.moe_forward(x, *oracle.route_softmax(logits, TOPK), experts, D, I, LIMIT,
                                                 threads=th),
             T, f"whole step, {len(touched)} experts touched")
        del experts
    # T = 4096 routed over 256 experts; the sample runs 4 experts' rows, scaled by P / sample rows
    T = 4096
    x = to_bf16(rng.standard_normal((T, D), dtype=np.float32))
    logits = rng.standard_normal((T, E), dtype=np.float32)
    sel, wt = oracle.route_softmax(logits, TOPK)
    cnt = np.bincount(sel.ravel(), minlength=E)
    sample = [int(e) for e in rng.choice(E, 4, replace=False)]
    experts = _host_experts(rng, sample)
    rows = int(cnt[sample].sum())
    both("configs3_moe_prefill_T4096", lambda th: oracle.moe_forward(x, sel, wt, experts, D, I, LIMIT, threads=th,
                                                                     subset=sample),
         T, f"4 of 256 experts ({rows} of {T * TOPK} pair rows), extrapolated linearly in rows",
         scale=T * TOPK / rows)
    del experts
    # fp8 dense 4096 x 4096 with fp32 scales (act_quant_fp8_f32s + gemm_w8a8)
    wq = rng.integers(0, 256, (D, D), dtype=np.uint8)
    wq[(wq & 0x7F) == 0x7F] = 0
    wsc = (rng.random((D // 128, D // 128), dtype=np.float32) * np.float32(1e-3)).astype(np.float32)
    for M, rows_s in ((1, 1), (64, 64), (4096, 64)):
        xm = to_bf16(rng.standard_normal((rows_s, D), dtype=np.float32))

        def fp8(th, xm=xm):
            q, sa = oracle.act_quant_fp8_f32s(xm)
            oracle.gemm_w8a8(q, sa, wq, wsc, threads=th)

        both(f"configs4_fp8_dense_M{M}", fp8, M, "whole GEMM" if rows_s == M else
             f"{rows_s} of {M} rows, extrapolated linearly in rows", scale=M / rows_s)
    return out


def run_only(name, args, rng):
    """One workload alone, so that a profiler's kernel table holds only its kernels (plus weight generation)."""
    if name == "copy":  # 1 GiB device-to-device copies: the reference for FETCH_SIZE / WRITE_SIZE counters
        from unholy_amd.device import DeviceBuffer, synchronize
        from unholy_amd._lib import call
        n = 1 << 30
        src, dst = DeviceBuffer(n), DeviceBuffer(n)
        call("uh_fill_random_bytes", src, n, 1, 0, 255, None)
        for _ in range(4):
            call("uh_memcpy_d2d", dst, src, n, None)
        synchronize()
        return {"workload": "copy", "bytes_per_copy": n, "copies": 4}
    if name == "remote":
        rng = np.random.default_rng(5)
        return {"remote_transport_T8": bench_remote(8, args.steps, args.warmup, rng),
                "remote_transport_T4096": bench_remote(4096, args.steps, args.warmup, rng)}
    if name == "pack":
        return {"expert_pack_load": bench_pack()}
    if name == "producers":
        return {f"producers_rows{r}": producers_entry(r, *bench_producers(r, 64, 16, rng)) for r in (8, 4096)}
    if name == "grouped":
        return {f"grouped_fp8w_M{M}": bench_grouped_fp8w(M, 100 if M < 4096 else 10, 10 if M < 4096 else 2, rng, c)
                for M, c in ((1, 16), (64, 16), (4096, 2))}
    if name == "fp8_m64":  # configs[4] at M = 64
        return {"fp8_dense_M64": bench_fp8_dense(64, 40, 5, rng, 16)}
    if name == "fp8":
        return {f"fp8_dense_M{M}": bench_fp8_dense(M, 100 if M < 4096 else 10, 10 if M < 4096 else 2, rng, c)
                for M, c in ((1, 64), (64, 64), (4096, 4))}
    w = Weights(seed=0)
    if name == "single":
        return {"single_gemv_M1_ms": bench_single_gemv(w, 500, 50, rng)}
    if name == "decode":
        d = bench_moe(w, 8, args.steps, args.warmup, rng)
        g = bench_moe_graph(w, 8, args.steps, args.warmup, np.random.default_rng(0))
        return {"moe_decode_T8_ms": d["ms"], "moe_decode_T8_graph_ms": g["ms"], "distinct_experts": d["U"]}
    if name == "dropin":
        d8 = bench_dropin(w, 8, args.steps, args.warmup, rng)
        d64 = bench_dropin(w, 64, 50, 5, rng, bias=0.5, glu=False)
        d4 = bench_dropin(w, 4096, 5, 1, rng)
        return {"dropin_T8_ms": d8["ms"], "dropin_T64_ms": d64["ms"], "dropin_T4096_ms": d4["ms"]}
    if name == "verify":
        d = bench_moe(w, 64, 50, 5, rng, bias=0.5)
        return {"moe_verify_T64_ms": d["ms"], "distinct_experts": d["U"]}
    d = bench_moe(w, 4096, 5, 1, rng, R=2)
    return {"moe_prefill_T4096_ms": d["ms"]}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", choices=["decode", "single", "verify", "prefill", "fp8", "fp8_m64", "grouped", "producers",
                                       "dropin", "pack", "remote", "copy"])
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the MoE expert path runs on a single MI355X in this build "
              "(expert-parallel sharding is a design note, not implemented); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    from unholy_amd.device import device_name

    rng = np.random.default_rng(0)
    if args.only:
        print(json.dumps(run_only(args.only, args, rng)))
        return
    w = Weights(seed=0)
    dec = bench_moe(w, 8, args.steps, args.warmup, rng, stage=True)
    ms = dec["ms"]
    U = dec["U"]
    # dominant kernel: the w1/w3 + SwiGLU grouped GEMV; algorithmic bytes = touched experts' w1 + w3 (codes +
    # scales) + the pair rows' fp8 inputs (P x 4096 + scales) + hh out (P x 2048 codes + scales)
    P = 8 * TOPK
    gemv_ms = [m for m, _ in dec["stage"]]
    gemv_bytes = [u * 2 * MAT_BYTES + P * (D + D // 128) + P * (I + I // 128) for _, u in dec["stage"]]
    g_ms = float(np.mean(gemv_ms))
    achieved = float(np.mean(gemv_bytes)) / (g_ms * 1e-3) / 1e9
    step_bytes = U * EXPERT_BYTES + 8 * D * 2 * 2
    result = {
        "metric": "MoE expert-FFN tokens/s (decode, BASELINE configs[1])",
        "value": 8 / (ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "mxfp4 weights x e4m3 activations, exact bf16 dequant, bf16 MFMA, fp32 accumulate",
        "data": "synthetic (device splitmix64 weights, numpy PCG64 activations/logits)",
        "config": {"workload": "moe_decode_T8 (BASELINE configs[1])", "tokens": 8, "experts": E, "top_k": TOPK,
                   "dim": D, "moe_inter": I, "swiglu_limit": LIMIT, "rotating_sets": 8,
                   "distinct_experts_per_step": U, "step_algorithmic_bytes": step_bytes,
                   "step_GBps": step_bytes / (ms * 1e-3) / 1e9, "device": device_name()},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": GEMV_TRAFFIC_BYTES,
                     "traffic_source": "profiles/hbm_traffic_pmc.md (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE)",
                     "kernel": "mx_gemv_kernel<2, 2, 2, 8, false, true> (w1/w3 grouped GEMV, SwiGLU epilogue)", "avg_launch_ms": g_ms,
                     "algorithmic_bytes_per_launch": float(np.mean(gemv_bytes))},
    }
    if not args.no_sweep:
        wl = {}
        s0 = bench_single_gemv(w, 500, 50, rng)
        b0 = MAT_BYTES + D + D // 128 + I * 2  # weights (codes + scales), the row's codes + scales in, bf16 out
        wl["single_gemv_M1 (configs[0])"] = {"ms": s0, "algorithmic_bytes": b0, "GBps": b0 / (s0 * 1e-3) / 1e9,
                                             "bound": "hbm", "frac_hbm_peak": b0 / (s0 * 1e-3) / 1e9 / HBM_PEAK_GBS}
        v = bench_moe(w, 64, 50, 5, rng, bias=0.5)
        bv = v["U"] * EXPERT_BYTES + 64 * D * 2 * 2  # touched experts' w1 + w3 + w2, x in and out (bf16)
        wl["moe_verify_T64 (configs[2])"] = {"ms": v["ms"], "tokens_per_s": 64 / (v["ms"] * 1e-3),
                                              "distinct_experts": v["U"], "step_algorithmic_bytes": bv,
                                              "GBps": bv / (v["ms"] * 1e-3) / 1e9, "bound": "hbm",
                                              "frac_hbm_peak": bv / (v["ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS,
                                              "GBps_weights": v["U"] * EXPERT_BYTES / (v["ms"] * 1e-3) / 1e9}
        from unholy_amd import call
        flops = 4096 * TOPK * 3 * 2 * D * I
        p = bench_moe(w, 4096, 5, 1, rng, R=2)
        prev = call("uh_mx_gemm_set_exact", 0)
        try:
            ps = bench_moe(w, 4096, 5, 1, rng, R=2)
        finally:
            call("uh_mx_gemm_set_exact", prev)
        roof_ms = E * EXPERT_BYTES / (HBM_PEAK_GBS * 1e9) * 1e3
        wl["moe_prefill_T4096 (configs[3])"] = {
            "ms": p["ms"], "tokens_per_s": 4096 / (p["ms"] * 1e-3),
            "TFLOPs": flops / (p["ms"] * 1e-3) / 1e12,
            "mfma": "v_mfma_f32_16x16x32_bf16 on exactly dequantized operands (one MFMA per 32-input block)",
            "frac_bf16_mfma_peak": flops / (p["ms"] * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
            "hbm_roof_ms": roof_ms, "frac_hbm_roof": roof_ms / p["ms"],
            "GBps_weights": E * EXPERT_BYTES / (p["ms"] * 1e-3) / 1e9,
            "speed_mode_block_scaled_not_parity": {
                "ms": ps["ms"], "TFLOPs": flops / (ps["ms"] * 1e-3) / 1e12,
                "mfma": "v_mfma_scale_f32_16x16x128_f8f6f4 (e4m3 x e2m1, e8m0 block scales); sums below fp32 "
                        "precision, outside the per-element tolerance",
                "frac_fp8_mfma_peak": flops / (ps["ms"] * 1e-3) / 1e12 / FP8_PEAK_TFLOPS}}
        for T, stp, wu, bias, glu in ((8, 200, 16, 0.0, True), (64, 50, 5, 0.5, False), (4096, 5, 1, 0.0, True)):
            dr = bench_dropin(w, T, stp, wu, rng, bias=bias, glu=glu)
            wl[f"dropin_sequence_T{T}"] = {
                "ms": dr["ms"], "tokens_per_s": T / (dr["ms"] * 1e-3), "distinct_experts": dr["U"],
                "sequence": "route_softmax, dispatch, mx_xform_in, " + (
                    "mx_grouped_gemv (MxGlu hh), mx_grouped_gemv (tiles of 8 rows)" if T <= 8 else
                    "mx_grouped_gemm (w1 and w3, max_rows = T), mx_swiglu, mx_grouped_gemm (w2, max_rows = T)"
                    if not glu else "mx_grouped_gemm_glu, mx_grouped_gemm") +
                ", moe_combine (forward_ref.hip:455-470; UNHOLY_MX_GEMV_TOKENS unset)"}
        for M, copies in ((1, 64), (64, 64), (4096, 4)):
            t = bench_fp8_dense(M, 100 if M < 4096 else 10, 10 if M < 4096 else 2, rng, copies)
            wl[f"fp8_dense_M{M} (configs[4])"] = {"ms": t, "tokens_per_s": M / (t * 1e-3),
                                                  "TFLOPs": 2 * M * D * D / (t * 1e-3) / 1e12,
                                                  "GBps_weights": D * D / (t * 1e-3) / 1e9}
            e = wl[f"fp8_dense_M{M} (configs[4])"]
            # 2 M flop per weight byte against the bf16 ridge (the operands are dequantized to bf16)
            if 2 * M < BF16_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9):
                e["frac_hbm_peak"] = e["GBps_weights"] / HBM_PEAK_GBS
            else:
                e["frac_bf16_mfma_peak"] = e["TFLOPs"] / BF16_PEAK_TFLOPS
            if M <= 16:  # the two-call form beside the fused one
                e["ms_act_quant_then_gemm"] = bench_fp8_dense(M, 100, 10, rng, copies, form="two")
        for M, copies in ((1, 16), (64, 16), (4096, 2)):
            t = bench_grouped_fp8w(M, 100 if M < 4096 else 10, 10 if M < 4096 else 2, rng, copies)
            wl[f"grouped_fp8w_wo_a_M{M}"] = grouped_entry(M, t)
        for r in (8, 4096):
            wl[f"producers_rows{r}"] = producers_entry(r, *bench_producers(r, 64, 16, rng))
        wl["expert_pack_load"] = bench_pack()
        wl["remote_transport_T8"] = bench_remote(8, 64, 16, rng)
        wl["remote_transport_T4096"] = bench_remote(4096, 64, 16, rng)
        result["workloads"] = wl
    if not args.no_cpu:
        cb = cpu_baselines()
        head = cb["configs1_moe_decode_T8"]
        result["cpu_baseline"] = {
            "value": head["tokens_per_s"], "unit": "tokens/s", "cores": cb["threads"], "kind": "port",
            "sample": "one decode step of configs[1] (T=8, 256 experts, top-6; " + head["sample"] + ") through the "
                      "CPU oracle, repeated for >= 1 s; per_config holds every BASELINE configuration at 1 thread "
                      "and at `cores` threads",
            "value_1_thread": head["tokens_per_s_1t"], "cpu_model": cb["cpu_model"],
            "per_config": {k: v for k, v in cb.items() if k.startswith("configs")}}
    print(json.dumps(result))


if __name__ == "__main__":
    main()
