#!/usr/bin/env python3
"""Benchmark: fused GDN decode step with INT8 state + packed-INT4 EF residual.

Workload ("C3", at its headline batch): one
single-layer decode step at batch 64 over 32 value heads (H = HV = 32) with
K = V = 128, int8 per-V-row state, packed int4 residual with a per-head
scale, fp32 activations, vLLM paged layout, in place through
``quantized_gated_delta_rule_packed_decode`` (one kernel launch per step).

Synthetic data of the config's distributions: alpha = exp(g),
g ~ U(log 0.9, log 0.995) per (request, head), beta = sigmoid(U(-2, 2)); q, k
L2-normalised N(0,1) (normalised on the host, kernel flag off, scale 1.0);
v ~ N(0,1). The gates reach the kernel as A_log = 0, dt_bias = 0,
a = log(expm1(-g)), b = logit(beta). The initial state is 64 fp32 warm-up
steps from zero (on the GPU, fp32 state arm), then quantized into the pool.

Each step takes the next group of 64 slots of a 1025-slot pool (about 0.8 GB,
larger than the 256 MB Infinity Cache), so state reads come from HBM as they
do when 24 layers share the cache between two steps of one layer.

Prints ONE JSON line (rank 0). ``value`` is algorithmic GB/s over the timed
steps; ``ms_per_step`` is the device time per step from HIP events on the
launch stream.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
if HERE not in sys.path:
    sys.path.insert(0, HERE)

from carrykernel_amd.statequant import kernel as sq  # noqa: E402
from carrykernel_amd.vllm_integration import quantized_packed_decode as qpd  # noqa: E402

HBM_PEAK_GBPS = 8000.0
METRIC = "\u00b5s per GDN decode step and achieved HBM GB/s (% roofline) at batch 64, 1 GPU"
H = HV = 32
K = V = 128


def algorithmic_bytes(B, H, HV, K, V, resid_fmt, per_head, act_bytes=4):
    """Unique bytes read + written by one step.

    Per (request, value-head): state codes 2*K*V; residual 2*K*V (int8) or
    K*V (int4); state scale 2*4*V; residual scale 2*4*V (per row) or 2*4
    (per head); v and o 2*act*V; the two gate inputs a, b 2*act. Per
    (request, QK head): q and k 2*act*K. Per request: the 4-byte slot id.
    """
    resid = 2 * K * V if resid_fmt == qpd.RESID_INT8 else K * V
    rscale = 2 * 4 if per_head else 2 * 4 * V
    per_vhead = 2 * K * V + resid + 2 * 4 * V + rscale + 2 * act_bytes * V + 2 * act_bytes
    per_qkhead = 2 * act_bytes * K
    return B * (HV * per_vhead + H * per_qkhead + 4)


def float_state_bytes(B, H, HV, K, V, esz, act_bytes=4):
    """Same step with an unquantized state of `esz` bytes per element."""
    per_vhead = 2 * esz * K * V + 2 * act_bytes * V + 2 * act_bytes
    return B * (HV * per_vhead + H * 2 * act_bytes * K + 4)


def bf16_state_bytes(B, H, HV, K, V, act_bytes=4):
    """Same step with vLLM's default bf16 state (the comparison arm)."""
    return float_state_bytes(B, H, HV, K, V, 2, act_bytes)


def make_step_inputs(B, n_sets, device, seed):
    """Synthetic activations in the config's distributions (see module doc)."""
    g = torch.Generator().manual_seed(seed)
    sets = []
    for _ in range(n_sets):
        q = torch.randn(B, H, K, generator=g)
        k = torch.randn(B, H, K, generator=g)
        q = q / q.norm(dim=-1, keepdim=True)
        k = k / k.norm(dim=-1, keepdim=True)
        v = torch.randn(B, HV, V, generator=g)
        lg = torch.empty(B, HV).uniform_(math.log(0.9), math.log(0.995), generator=g)
        a = torch.log(torch.expm1(-lg))
        b = torch.empty(B, HV).uniform_(-2.0, 2.0, generator=g)
        mixed = torch.cat([q.reshape(B, -1), k.reshape(B, -1), v.reshape(B, -1)], dim=1).contiguous()
        sets.append(tuple(x.to(device) for x in (mixed, a.contiguous(), b.contiguous())))
    A_log = torch.zeros(HV, device=device)
    dt_bias = torch.zeros(HV, device=device)
    return sets, A_log, dt_bias


def warm_state(S, device, seed):
    """64 fp32 warm-up steps from zero on slots 1..S-1, then quantize."""
    from carrykernel_amd import _native
    state = torch.zeros(S, HV, V, K, device=device)
    sets, A_log, dt_bias = make_step_inputs(S - 1, 4, device, seed + 17)
    idx = torch.arange(1, S, dtype=torch.int32, device=device)
    out = torch.empty(S - 1, 1, HV, V, device=device)
    L = _native.lib()
    for t in range(64):
        mixed, a, b = sets[t % len(sets)]
        st = L.ck_gdn_packed_decode_float_state(
            mixed.data_ptr(), 0, mixed.stride(0), a.data_ptr(), 0, a.stride(0), b.data_ptr(), 0, b.stride(0),
            A_log.data_ptr(), 0, dt_bias.data_ptr(), 0, 1.0, state.data_ptr(), 0, state.stride(0),
            out.data_ptr(), 0, idx.data_ptr(), 1, S, S - 1, H, HV, K, V, 0,
            _native.stream_handle(state.device))
        _native.check(st, "warm-up")
    return state


def cpu_baseline(B, resid_fmt, per_head, seconds=12.0):
    """The CPU oracle (C, OpenMP over (request, head)) on the same workload
    shape, timed on this host for about `seconds`."""
    import numpy as np
    import oracle
    nthreads = len(os.sched_getaffinity(0))
    nthreads = min(nthreads, 16)
    S = B + 1
    rng = np.random.default_rng(0)
    h0 = (rng.standard_normal((S, HV, V, K)) * 0.1).astype(np.float32)
    sc, ss = oracle.quantize_rows(h0)
    rc = np.zeros((S, HV, V, K // 2 if resid_fmt == qpd.RESID_INT4 else K), np.int8)
    rs = np.zeros((S, HV) if per_head else (S, HV, V), np.float32)
    sets, A_log, dt_bias = make_step_inputs(B, 2, "cpu", 5)
    idx = np.arange(1, B + 1, dtype=np.int32)
    steps = 0
    t0 = time.perf_counter()
    while True:
        mixed, a, b = sets[steps % 2]
        oracle.packed_decode(mixed.numpy(), a.numpy(), b.numpy(), A_log.numpy(), dt_bias.numpy(), 1.0,
                             sc, ss, rc, rs, idx, H, resid_fmt=resid_fmt, per_head=per_head,
                             nthreads=nthreads)
        steps += 1
        el = time.perf_counter() - t0
        if el >= seconds or steps >= 5000:
            break
    us = el / steps * 1e6
    gbps = algorithmic_bytes(B, H, HV, K, V, resid_fmt, per_head) / (us * 1e-6) / 1e9
    return {"value": round(gbps, 3), "unit": "GB/s", "us_per_step": round(us, 1), "cores": nthreads,
            "kind": "port",
            "sample": f"{steps} steps of the B={B} workload through the C oracle (oracle/gdn_oracle.c, "
                      f"OpenMP, {nthreads} threads), {el:.1f} s"}


class Timer:
    """HIP events on the launch stream (torch's current stream)."""

    def __init__(self, device):
        self.s = torch.cuda.Event(enable_timing=True)
        self.e = torch.cuda.Event(enable_timing=True)
        self.stream = torch.cuda.current_stream(device)

    def start(self):
        self.s.record(self.stream)

    def stop_ms(self):
        self.e.record(self.stream)
        self.e.synchronize()
        return self.s.elapsed_time(self.e)


def run_config(device, B, resid_fmt, per_head, steps, warmup, groups, quant_mode="fast", seed=0,
               act_dtype=torch.float32):
    """Returns (device ms per step from a replayed graph, host-inclusive ms per
    eager call). The graph holds one step per slot group. `act_dtype` is the
    dtype of mixed_qkv, a, b and out (vLLM runs bf16 activations)."""
    S = B * groups + 1
    state = warm_state(S, device, seed)
    pool = qpd.init_quantized_state(S, HV, V, K, device, h0=state, resid_fmt=resid_fmt,
                                    per_head_resid_scale=per_head)
    del state
    torch.cuda.empty_cache()
    sets, A_log, dt_bias = make_step_inputs(B, 8, device, seed + 1)
    sets = [tuple(x.to(act_dtype) for x in st) for st in sets]
    perm = torch.randperm(S - 1, generator=torch.Generator().manual_seed(seed)) + 1
    idx_groups = [perm[i * B:(i + 1) * B].to(torch.int32).to(device) for i in range(groups)]
    out = torch.empty(B, 1, HV, V, device=device, dtype=act_dtype)

    def step(t):
        mixed, a, b = sets[t % len(sets)]
        qpd.quantized_gated_delta_rule_packed_decode(
            mixed, a, b, A_log, dt_bias, 1.0, *pool, out, idx_groups[t % groups],
            resid_fmt=resid_fmt, quant_mode=quant_mode)

    # eager calls: host-inclusive latency per call
    for t in range(min(warmup, 50)):
        step(t)
    torch.cuda.synchronize()
    n_eager = 50
    t0 = time.perf_counter()
    for t in range(n_eager):
        step(t)
    torch.cuda.synchronize()
    host_ms = (time.perf_counter() - t0) * 1e3 / n_eager

    # graph of `groups` consecutive steps, replayed
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            for t in range(groups):
                step(t)
    torch.cuda.current_stream(device).wait_stream(side)
    torch.cuda.synchronize()
    reps_w = max(1, -(-warmup // groups))
    reps = max(1, -(-steps // groups))
    for _ in range(reps_w):
        graph.replay()
    torch.cuda.synchronize()
    timer = Timer(device)
    timer.start()
    for _ in range(reps):
        graph.replay()
    ms = timer.stop_ms() / (reps * groups)
    torch.cuda.synchronize()
    if not torch.isfinite(out).all():
        raise RuntimeError("non-finite output in the timed run")
    del graph, pool
    torch.cuda.empty_cache()
    return ms, host_ms


def _graph_time(device, step, n_steps, warmup, reps_cap=None):
    """Device ms per step of `step(t)` captured as n_steps consecutive launches
    in one HIP graph and replayed (warm-up replays first; median of three
    timed batches)."""
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        for t in range(n_steps):
            step(t)
    torch.cuda.current_stream(device).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        for t in range(n_steps):
            step(t)
    torch.cuda.synchronize()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    reps = reps_cap or 20
    trials = []
    for _ in range(3):   # median of three timed batches of replays
        timer = Timer(device)
        timer.start()
        for _ in range(reps):
            graph.replay()
        trials.append(timer.stop_ms() / (reps * n_steps))
    del graph
    return sorted(trials)[1]


def multilayer_token(device, layers=24, B=64, live=None, tokens=20, seed=7):
    """Config C5's decode shape as a serving engine runs it: one token through
    `layers` GDN layers at batch B (int4 residual, per-head scale), each layer
    with its own pool, called eagerly (host-inclusive time per token: one
    Python call and one launch per layer) and captured once in a HIP graph and
    replayed (device time per token). With live < B the batch is padded with
    NULL-block ids, as a capture at a fixed batch size is
    (quantized_packed_decode.py:24-26,132-136); bytes count live requests."""
    live = B if live is None else live
    S = B + 1
    pools = [qpd.init_quantized_state(S, HV, V, K, device, resid_fmt=qpd.RESID_INT4, per_head_resid_scale=True)
             for _ in range(layers)]
    sets, A_log, dt_bias = make_step_inputs(B, 1, device, seed)
    mixed, a, b = sets[0]
    idx = torch.arange(1, B + 1, dtype=torch.int32, device=device)
    idx[live:] = 0
    outs = [torch.empty(B, 1, HV, V, device=device) for _ in range(layers)]

    def token(_t=0):
        for layer in range(layers):
            qpd.quantized_gated_delta_rule_packed_decode(mixed, a, b, A_log, dt_bias, 1.0, *pools[layer],
                                                         outs[layer], idx, resid_fmt=qpd.RESID_INT4)

    for _ in range(3):
        token()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(tokens):
        token()
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) * 1e3 / tokens
    graph_ms = _graph_time(device, token, 1, 10, max(3, tokens))
    nb = layers * algorithmic_bytes(live, H, HV, K, V, qpd.RESID_INT4, True)
    del pools, outs
    torch.cuda.empty_cache()
    return {"layers": layers, "batch": B, "live_requests": live,
            "eager_host_us_per_token": round(eager_ms * 1e3, 2),
            "graph_us_per_token": round(graph_ms * 1e3, 2),
            "graph_us_per_layer": round(graph_ms * 1e3 / layers, 3),
            "GBps": round(nb / (graph_ms * 1e-3) / 1e9, 1),
            "frac": round(nb / (graph_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}


def ingest_arm(device, slots=257):
    """State ingest (init_quantized_state's quantization, ck_quantize_rows) of a
    [slots, HV, V, K] prefill state in fp32 and bf16: reads the state, writes
    int8 codes and one fp32 scale per row. Buffers rotate over > 256 MB."""
    from carrykernel_amd import _native
    L = _native.lib()
    res = {}
    rows = slots * HV * V
    for name, dt, esz in (("ingest_rows_fp32", torch.float32, 4), ("ingest_rows_bf16", torch.bfloat16, 2)):
        x = torch.randn(slots, HV, V, K, device=device).to(dt)
        codes = torch.empty(slots, HV, V, K, dtype=torch.int8, device=device)
        scale = torch.empty(slots, HV, V, device=device)
        code = _native.dtype_code(x, "x")

        def step(_t, x=x, codes=codes, scale=scale, code=code):
            _native.check(L.ck_quantize_rows(x.data_ptr(), code, K, rows, K, 127.0, codes.data_ptr(),
                                             scale.data_ptr(), _native.stream_handle(device)), "ck_quantize_rows")

        ms = _graph_time(device, step, 1, 20, 20)
        nb = rows * K * (esz + 1) + rows * 4
        res[name] = {"us": round(ms * 1e3, 2), "bytes": nb, "GBps": round(nb / (ms * 1e-3) / 1e9, 1),
                     "frac": round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}
        del x, codes, scale
        torch.cuda.empty_cache()
    # the statequant layout's per-V-column quantization (per_v_channel_quantize,
    # ck_quantize_cols) of a [slots, HV, K, V] fp32 state
    x = torch.randn(slots, HV, K, V, device=device)
    codes = torch.empty(slots, HV, K, V, dtype=torch.int8, device=device)
    scale = torch.empty(slots, HV, V, device=device)

    def cstep(_t):
        _native.check(L.ck_quantize_cols(x.data_ptr(), slots * HV, K, V, 127.0, codes.data_ptr(), scale.data_ptr(),
                                         _native.stream_handle(device)), "ck_quantize_cols")

    ms = _graph_time(device, cstep, 1, 20, 20)
    nb = slots * HV * K * V * 5 + slots * HV * V * 4
    res["ingest_cols_fp32"] = {"us": round(ms * 1e3, 2), "bytes": nb, "GBps": round(nb / (ms * 1e-3) / 1e9, 1),
                               "frac": round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}
    del x, codes, scale
    torch.cuda.empty_cache()
    return res


def slot_ops_arm(device, n=256):
    """The engine-side slot operations (ck_pool_copy_slots, ck_pool_reset_slots)
    on an int4 / per-head pool of HV=32, K=V=128: copy n random slots to n
    others of a 4n+1-slot pool (slot bytes read and written), reset n slots
    (written)."""
    res = {}
    S = 4 * n + 1
    pool = qpd.init_quantized_state(S, HV, V, K, device, resid_fmt=qpd.RESID_INT4, per_head_resid_scale=True)
    slot_bytes = qpd.state_bytes_per_slot(HV, V, K, True, resid_fmt=qpd.RESID_INT4, per_head_resid_scale=True)
    perm = torch.randperm(S - 1, generator=torch.Generator().manual_seed(11)) + 1
    groups = [perm[i * n:(i + 1) * n].to(torch.int32).to(device) for i in range(4)]

    def copy_step(t):
        qpd.copy_quantized_state(pool, groups[t % 4], pool, groups[(t + 1) % 4])

    def reset_step(t):
        qpd.reset_quantized_state(pool, groups[t % 4])

    ms = _graph_time(device, copy_step, 3, 20, 20)
    nb = 2 * n * slot_bytes
    res["pool_copy_slots"] = {"us": round(ms * 1e3, 2), "bytes": nb, "GBps": round(nb / (ms * 1e-3) / 1e9, 1),
                              "frac": round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}
    ms = _graph_time(device, reset_step, 4, 20, 20)
    nb = n * slot_bytes
    res["pool_reset_slots"] = {"us": round(ms * 1e3, 2), "bytes": nb, "GBps": round(nb / (ms * 1e-3) / 1e9, 1),
                               "frac": round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}
    del pool
    torch.cuda.empty_cache()
    return res


def statequant_bytes(B, HV, K, V, res_fmt):
    """Unique bytes of one statequant-layout step (statequant/kernel.py:379-408):
    int8 codes in/out, residual in/out, per-column state scale in/out (and the
    int8 residual's per-column scale in/out), q/k/v/o fp32, alpha/beta."""
    rb = {sq.RES_FP32: 4, sq.RES_FP16: 2, sq.RES_FP8: 1, sq.RES_INT8: 1}[res_fmt]
    per = 2 * K * V + 2 * K * V * rb + 2 * 4 * V + (2 * 4 * V if res_fmt == sq.RES_INT8 else 0)
    per += 2 * 4 * K + 2 * 4 * V + 2 * 4
    return B * HV * per


def arms(device, batches=(8, 64), steps=800):
    """The other entry points at config shapes (HV=32, K=V=128, fp32
    activations): the statequant-layout step for each residual format, its fp32
    baseline, and the unquantized fp32 / bf16 state arms of the vLLM-layout
    decode. Out-of-place steps ping-pong between buffer sets whose total exceeds
    the 256 MB MALL. Returns {name: {us, GBps, frac}}."""
    from carrykernel_amd import _native
    L = _native.lib()
    res = {}
    gen = torch.Generator(device=device).manual_seed(3)

    def rec(name, ms, nbytes):
        res[name] = {"us": round(ms * 1e3, 3), "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1),
                     "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}

    for B in batches:
        q = torch.randn(B, HV, K, device=device, generator=gen)
        k = torch.randn(B, HV, K, device=device, generator=gen)
        k = k / k.norm(dim=-1, keepdim=True)
        v = torch.randn(B, HV, V, device=device, generator=gen)
        al = torch.full((B, HV), 0.99, device=device)
        be = torch.full((B, HV), 0.5, device=device)
        o = torch.empty(B, HV, V, device=device)
        for res_fmt in (sq.RES_FP32, sq.RES_FP16, sq.RES_FP8, sq.RES_INT8):
            per_set = B * HV * K * V * (1 + sq.residual_bytes(res_fmt))
            nsets = max(2, min(64, -(-(512 << 20) // per_set)))
            h0 = torch.randn(B, HV, K, V, device=device, generator=gen) * 0.1
            sets = []
            for _ in range(nsets):
                hs = sq.init_quant_state(h0, 8, res_fmt)
                es = hs[3] if hs[3] is not None else torch.zeros(B, HV, V, device=device)
                sets.append((hs[0], hs[1], hs[2], es))
            del h0

            def step(t, sets=sets, res_fmt=res_fmt):
                a_, b_ = sets[t % nsets], sets[(t + 1) % nsets]
                st = L.ck_gdn_quant_step(a_[0].data_ptr(), a_[1].data_ptr(), a_[2].data_ptr(), a_[3].data_ptr(),
                                         q.data_ptr(), k.data_ptr(), v.data_ptr(), al.data_ptr(), be.data_ptr(),
                                         o.data_ptr(), b_[0].data_ptr(), b_[1].data_ptr(), b_[2].data_ptr(),
                                         b_[3].data_ptr(), B, HV, K, V, 127.0, res_fmt, 0,
                                         _native.stream_handle(device))
                _native.check(st, "statequant step")
            ms = _graph_time(device, step, nsets, -(-200 // nsets), max(2, steps // nsets))
            rec(f"statequant_B{B}_{sq.residual_label(res_fmt)}", ms, statequant_bytes(B, HV, K, V, res_fmt))
            del sets
        # fp32 baseline step, ping-pong between state buffers
        nsets = max(2, min(64, -(-(512 << 20) // (B * HV * K * V * 4))))
        hsets = [torch.randn(B, HV, K, V, device=device, generator=gen) * 0.1 for _ in range(nsets)]

        def fstep(t):
            st = L.ck_gdn_fp32_step(hsets[t % nsets].data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                    al.data_ptr(), be.data_ptr(), o.data_ptr(), hsets[(t + 1) % nsets].data_ptr(),
                                    B, HV, K, V, _native.stream_handle(device))
            _native.check(st, "fp32 step")
        ms = _graph_time(device, fstep, nsets, -(-200 // nsets), max(2, steps // nsets))
        rec(f"fp32_step_B{B}", ms, B * HV * (2 * 4 * K * V + 2 * 4 * K + 2 * 4 * V + 8))
        del hsets
        torch.cuda.empty_cache()
    # vLLM-layout unquantized arms at B=64 (in place, slot groups rotated)
    B = 64
    sets_in, A_log, dt_bias = make_step_inputs(B, 4, device, 9)
    for dtype, name, esz in ((torch.float32, "fp32", 4), (torch.bfloat16, "bf16", 2)):
        groups = max(2, min(64, -(-(512 << 20) // (B * HV * V * K * esz))))
        S = B * groups + 1
        state = (torch.randn(S, HV, V, K, device=device, generator=gen) * 0.1).to(dtype)
        idxs = [torch.arange(1 + g * B, 1 + (g + 1) * B, dtype=torch.int32, device=device) for g in range(groups)]
        out = torch.empty(B, 1, HV, V, device=device)

        def vstep(t, state=state, idxs=idxs, dtype=dtype, out=out, S=S):
            mixed, a, b = sets_in[t % len(sets_in)]
            st = L.ck_gdn_packed_decode_float_state(
                mixed.data_ptr(), 0, mixed.stride(0), a.data_ptr(), 0, a.stride(0), b.data_ptr(), 0, b.stride(0),
                A_log.data_ptr(), 0, dt_bias.data_ptr(), 0, 1.0, state.data_ptr(),
                0 if dtype == torch.float32 else 1, state.stride(0), out.data_ptr(), 0,
                idxs[t % len(idxs)].data_ptr(), 1, S, B, H, HV, K, V, 0, _native.stream_handle(device))
            _native.check(st, "float-state step")
        ms = _graph_time(device, vstep, groups, -(-200 // groups), max(2, steps // groups))
        rec(f"vllm_{name}_state_B{B}", ms, float_state_bytes(B, H, HV, K, V, esz))
        del state
        torch.cuda.empty_cache()
    return res


def copy_peak(device, mib, reps):
    """Device-to-device copy of `mib` MiB (read + write), reps times."""
    n = mib * (1 << 20) // 4
    src = torch.randn(n, device=device)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    timer = Timer(device)
    timer.start()
    for _ in range(reps):
        dst.copy_(src)
    ms = timer.stop_ms() / reps
    moved = 2 * n * 4
    return {"copy_mib": mib, "bytes_per_copy": moved, "us_per_copy": round(ms * 1e3, 3),
            "GBps": round(moved / (ms * 1e-3) / 1e9, 1)}


def hbm_copy_peak(device, total_bytes, pool_bytes=1 << 31, grids=(512, 2048, 4096)):
    """Measured HBM ceiling beside the spec-sheet one: the library's streaming
    copy (ck_hbm_copy) moving `total_bytes` per launch (half read, half
    written), timed like the decode (graph-replayed, rotating over buffer
    pairs that together exceed the 256 MB MALL); best of a few grid sizes."""
    from carrykernel_amd import _native
    L = _native.lib()
    half = (total_bytes // 2) // 4096 * 4096
    groups = int(max(2, min(64, pool_bytes // (2 * half))))
    src = [torch.empty(half, dtype=torch.uint8, device=device).fill_(t + 1) for t in range(groups)]
    dst = [torch.empty(half, dtype=torch.uint8, device=device) for _ in range(groups)]
    best = None
    for grid in grids:
        def step(t, grid=grid):
            _native.check(L.ck_hbm_copy(src[t % groups].data_ptr(), dst[t % groups].data_ptr(), half, grid,
                                        _native.stream_handle(device)), "hbm copy")
        ms = _graph_time(device, step, groups, -(-200 // groups))
        if best is None or ms < best[0]:
            best = (ms, grid)
    if not all(bool((d[:4096] == t + 1).all()) for t, d in enumerate(dst)):
        raise RuntimeError("hbm copy produced wrong bytes")
    del src, dst
    torch.cuda.empty_cache()
    ms, grid = best
    return {"bytes_per_launch": 2 * half, "us": round(ms * 1e3, 3), "GBps": round(2 * half / (ms * 1e-3) / 1e9, 1),
            "grid": grid}


def float_state_step(state, mixed, a, b, A_log, dt_bias, scale, out, idx, l2norm):
    """One step of the unquantized fp32 state arm (ck_gdn_packed_decode_float_state)."""
    from carrykernel_amd import _native
    S, hv, v, k = state.shape
    st = _native.lib().ck_gdn_packed_decode_float_state(
        mixed.data_ptr(), 0, mixed.stride(0), a.data_ptr(), 0, a.stride(0), b.data_ptr(), 0, b.stride(0),
        A_log.data_ptr(), 0, dt_bias.data_ptr(), 0, float(scale), state.data_ptr(), 0, state.stride(0),
        out.data_ptr(), 0, idx.data_ptr(), idx.stride(0), S, mixed.shape[0], (mixed.shape[1] - hv * v) // (2 * k),
        hv, k, v, int(l2norm),
        _native.stream_handle(state.device))
    _native.check(st, "float-state step")


def dequant_pool(pool, resid_fmt, with_residual):
    """codes * scale (+ the dequantized residual) of a vLLM pool, fp32 [S, HV, V, K]."""
    sc, ss, rc, rs = pool
    h = sc.float() * ss[..., None]
    if not with_residual:
        return h
    if resid_fmt == qpd.RESID_INT4:
        x = rc.to(torch.int32) & 0xFF
        lo = ((x & 0xF) ^ 8) - 8
        hi = ((x >> 4) ^ 8) - 8
        e = torch.stack([lo, hi], dim=-1).reshape(*rc.shape[:-1], 2 * rc.shape[-1]).float()
    else:
        e = rc.float()
    es = rs[..., None, None] if rs.dim() == 2 else rs[..., None]
    return h + e * es


def drift_c5(device, bits, tokens=2048, layers=24, B=64, every=256, resid_fmt=None, per_head=True,
             seed=0, log=None):
    """Config C5: `layers` GDN layers per token at batch B, fresh q/k/v per layer
    and token, heads 0..HV/2-1 at alpha 0.995 and the rest at 0.9, beta =
    sigmoid(U(-2, 2)), q/k L2-normalised in the kernel. The quantized pool
    (int8 or int6 state, int4 residual with a per-head scale by default) and an
    unquantized fp32 pool (the float-state arm, on the GPU) start from zero and
    see identical inputs. Every `every` tokens: relative error of the
    dequantized state (codes*scale, and with the residual added back) and of
    the outputs, over all layers and requests."""
    resid_fmt = qpd.RESID_INT4 if resid_fmt is None else resid_fmt
    gen = torch.Generator(device=device).manual_seed(seed)
    S = B + 1
    idx = torch.arange(1, S, dtype=torch.int32, device=device)
    pools = [qpd.init_quantized_state(S, HV, V, K, device, resid_fmt=resid_fmt, per_head_resid_scale=per_head,
                                      state_bits=bits) for _ in range(layers)]
    refs = [torch.zeros(S, HV, V, K, device=device) for _ in range(layers)]
    alpha = torch.tensor([0.995] * (HV // 2) + [0.9] * (HV - HV // 2), dtype=torch.float64)
    a = torch.log(torch.expm1(-torch.log(alpha))).float().to(device).expand(B, HV).contiguous()
    A_log = torch.zeros(HV, device=device)
    dt_bias = torch.zeros(HV, device=device)
    out_q = torch.empty(B, 1, HV, V, device=device)
    out_r = torch.empty(B, 1, HV, V, device=device)
    width = 2 * H * K + HV * V
    rows = []
    for t in range(tokens):
        report = (t + 1) % every == 0 or t == tokens - 1
        do2 = dn2 = 0.0
        for layer in range(layers):
            mixed = torch.randn(B, width, generator=gen, device=device)
            b = torch.rand(B, HV, generator=gen, device=device) * 4.0 - 2.0
            qpd.quantized_gated_delta_rule_packed_decode(
                mixed, a, b, A_log, dt_bias, 1.0, *pools[layer], out_q, idx, use_qk_l2norm_in_kernel=True,
                resid_fmt=resid_fmt, state_bits=bits)
            float_state_step(refs[layer], mixed, a, b, A_log, dt_bias, 1.0, out_r, idx, True)
            if report:
                do2 += float((out_q - out_r).double().square().sum())
                dn2 += float(out_r.double().square().sum())
        if report:
            dh2 = dhe2 = hn2 = 0.0
            for layer in range(layers):
                ref = refs[layer][1:].double()
                dh2 += float((dequant_pool(pools[layer], resid_fmt, False)[1:].double() - ref).square().sum())
                dhe2 += float((dequant_pool(pools[layer], resid_fmt, True)[1:].double() - ref).square().sum())
                hn2 += float(ref.square().sum())
            row = {"token": t + 1, "state_rel": round(math.sqrt(dh2 / hn2), 6),
                   "state_plus_residual_rel": round(math.sqrt(dhe2 / hn2), 6),
                   "o_rel": round(math.sqrt(do2 / dn2), 6)}
            rows.append(row)
            if log:
                log(row)
    return rows


def timeline_report(device, B, resid_fmt, per_head, groups, launches=20):
    """Per-workgroup timeline of one launch of the headline step, from the
    timestamped measurement build (libcarrykernel_gdn_timeline.so): the last
    of `launches` back-to-back eager launches writes, for every workgroup, its
    start, and per item the times its processing began, its loads had all
    landed, and its stores were issued (s_memrealtime, 100 MHz), plus the CU
    it ran on. Returns per-age statistics (age = dispatch order among the
    workgroups that share a CU)."""
    import numpy as np
    from carrykernel_amd import _native
    L = _native.use_timeline_build()
    S = B * groups + 1
    state = warm_state(S, device, 0)
    pool = qpd.init_quantized_state(S, HV, V, K, device, h0=state, resid_fmt=resid_fmt,
                                    per_head_resid_scale=per_head)
    del state
    sets, A_log, dt_bias = make_step_inputs(B, 8, device, 1)
    perm = torch.randperm(S - 1, generator=torch.Generator().manual_seed(0)) + 1
    ids = [perm[i * B:(i + 1) * B].to(torch.int32).to(device) for i in range(groups)]
    out = torch.empty(B, 1, HV, V, device=device)

    def step(t):
        mixed, a, b = sets[t % len(sets)]
        qpd.quantized_gated_delta_rule_packed_decode(mixed, a, b, A_log, dt_bias, 1.0, *pool, out, ids[t % groups],
                                                    resid_fmt=resid_fmt)

    for t in range(200):
        step(t)
    torch.cuda.synchronize()
    slots, max_wg = 40, 2048
    buf = torch.zeros(max_wg * slots, dtype=torch.int64, device=device)
    _native.check(L.ck_timeline_set(buf.data_ptr()), "ck_timeline_set")
    for t in range(launches - 1):
        step(t)
    buf.zero_()                      # on the launch stream, between the last two launches
    step(launches - 1)
    torch.cuda.synchronize()
    _native.check(L.ck_timeline_set(None), "ck_timeline_set")
    ts = buf.cpu().numpy().view(np.uint64).reshape(max_wg, slots)
    nwg = int(np.count_nonzero(ts[:, 0]))
    t = ts[:nwg, :31].astype(np.int64)
    t0 = t[:, 0].min()
    rel = np.where(t > 0, (t - t0) * 1e-2, np.nan)          # us
    su = ts[:nwg, 32:35].astype(np.int64)
    start = np.where(su > 0, (su - t0) * 1e-2, np.nan)       # slot id known, item 0 issued, gates done
    hw = (ts[:nwg, 31] & 0xffffffff).astype(np.int64)
    xcc = (ts[:nwg, 31] >> 32).astype(np.int64) & 0xf
    cu_id = xcc * 1024 + ((hw >> 13) & 7) * 64 + ((hw >> 12) & 1) * 16 + ((hw >> 8) & 0xf)
    per_cu = int(np.bincount(np.unique(cu_id, return_inverse=True)[1]).max())
    begin, data, end = rel[:, 1:31:3], rel[:, 2:31:3], rel[:, 3:31:3]
    n_rec = np.sum(~np.isnan(end), axis=1)
    last_end = np.array([end[i, n_rec[i] - 1] for i in range(nwg)])
    comp = np.nansum(end - data, axis=1) / n_rec
    wait = np.nansum(data - begin, axis=1) / n_rec
    # from one item's stores to the next item's start: the loop's bookkeeping, the
    # slot-id load of the item after next and the issue of its prefetch
    gap = np.nanmedian(begin[:, 1:] - end[:, :-1], axis=1)
    m = nwg // per_cu
    # do the workgroups q, q + m, ... share a CU (for every q)?
    groups_ok = sum(1 for q in range(m) if len({int(cu_id[q + a * m]) for a in range(per_cu)}) == 1
                    and int(np.count_nonzero(cu_id == cu_id[q])) == per_cu)
    ages = []
    for a in range(per_cu):
        sel = slice(a * m, (a + 1) * m)
        ages.append({"age": a, "items_median": float(np.median(n_rec[sel])),
                     "start_us": round(float(np.median(rel[sel, 0])), 2),
                     "slot_id_known_us": round(float(np.nanmedian(start[sel, 0])), 2),
                     "item0_loads_issued_us": round(float(np.nanmedian(start[sel, 1])), 2),
                     "gates_done_us": round(float(np.nanmedian(start[sel, 2])), 2),
                     "first_data_us": round(float(np.median(data[sel, 0])), 2),
                     "compute_us_per_item": round(float(np.median(comp[sel])), 2),
                     "wait_us_per_item": round(float(np.median(wait[sel])), 2),
                     "between_items_us": round(float(np.nanmedian(gap[sel])), 2),
                     "end_us_median": round(float(np.median(last_end[sel])), 2),
                     "end_us_max": round(float(np.max(last_end[sel])), 2)})
    return {"timeline": {"workload": f"B={B} {'int4' if resid_fmt == qpd.RESID_INT4 else 'int8'} residual, "
                                     f"{'per-head' if per_head else 'per-row'} scale",
                         "workgroups": nwg, "workgroups_per_cu": per_cu,
                         "cu_groups_in_dispatch_order": f"{groups_ok} of {m}",
                         "span_us": round(float(np.nanmax(last_end)), 2),
                         "end_us_median": round(float(np.median(last_end)), 2),
                         "end_us_p90": round(float(np.percentile(last_end, 90)), 2),
                         "ages": ages,
                         "note": "items >= 10 per workgroup are counted as 10 (the buffer keeps 10 item slots)"}}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--groups", type=int, default=16, help="disjoint slot groups rotated over")
    ap.add_argument("--resid", choices=("int4", "int8"), default="int4")
    ap.add_argument("--rscale", choices=("head", "row"), default="head")
    ap.add_argument("--quant-mode", choices=("fast", "exact"), default="fast")
    ap.add_argument("--sweep", action="store_true",
                    help="time every B in {1, 8, 64, 256} x residual format x scale granularity (default: "
                         "the headline format at B in {1, 8, 64, 256} and the C2 / C4 steps)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-sweep", action="store_true",
                    help="time only the headline configuration (no batch sweep, no other entry points)")
    ap.add_argument("--drift", action="store_true",
                    help="instead: config C5 drift (24 layers x B=64 x 2048 tokens, int8 and int6 state) "
                         "against the fp32 state arm; prints one JSON line")
    ap.add_argument("--drift-tokens", type=int, default=2048)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--timeline", action="store_true",
                    help="instead: per-workgroup timeline of one launch of the chosen step from the "
                         "timestamped measurement build (prints one JSON line)")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="instead: time a plain device copy of this many MiB (HBM copy peak, and the "
                         "byte-count calibration for the FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the decode step shards with no exchange between GPUs "
              "(requests or value heads per GPU), so only --gpus 1 is run here.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    device = torch.device("cuda", 0)
    if args.copy_mib:
        print(json.dumps(copy_peak(device, args.copy_mib, args.steps)), flush=True)
        return
    if args.drift:
        res = {}
        for bits in (8, 6):
            t0 = time.perf_counter()
            rows = drift_c5(device, bits, tokens=args.drift_tokens,
                            log=lambda r, bits=bits: print(f"int{bits}", json.dumps(r), file=sys.stderr, flush=True))
            res[f"int{bits}"] = {"rows": rows, "seconds": round(time.perf_counter() - t0, 1)}
        print(json.dumps({"config": "C5: 24 layers x B=64 x HV=32 x K=V=128, int4 residual (per-head scale), "
                                    "alpha 0.995 (heads 0-15) / 0.9 (16-31), drift vs the fp32 state arm",
                          "tokens": args.drift_tokens, "drift": res}), flush=True)
        return
    resid_fmt = qpd.RESID_INT4 if args.resid == "int4" else qpd.RESID_INT8
    per_head = args.rscale == "head"
    B = args.batch
    if args.timeline:
        print(json.dumps(timeline_report(device, B, resid_fmt, per_head, max(2, min(64, 1024 // B)))), flush=True)
        return

    ms, host_ms = run_config(device, B, resid_fmt, per_head, args.steps, args.warmup, args.groups,
                             args.quant_mode)
    nbytes = algorithmic_bytes(B, H, HV, K, V, resid_fmt, per_head)
    gbps = nbytes / (ms * 1e-3) / 1e9
    line = {
        "metric": METRIC,
        "value": round(gbps, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "us_per_step": round(ms * 1e3, 3),
        "host_us_per_eager_call": round(host_ms * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 state / int4 residual, fp32 arithmetic",
        "data": "synthetic (config distributions; state from 64 fp32 warm-up steps)",
        "config": {"workload": "C3: single-layer fused decode, int8 per-V state + packed int4 EF residual "
                               "(per-head scale), vLLM [slots,HV,V,K] layout",
                   "batch": B, "value_heads": HV, "qk_heads": H, "K": K, "V": V,
                   "resid": args.resid, "resid_scale": args.rscale, "quant_mode": args.quant_mode,
                   "pool_slots": B * args.groups + 1},
        "roofline": {"bound": "hbm", "achieved": round(gbps, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None,
                     "bytes_per_launch": nbytes},
        "bytes_vs_bf16_state": round(bf16_state_bytes(B, H, HV, K, V) / nbytes, 4),
    }
    traffic_path = os.path.join(HERE, "profiles", "traffic_packed_decode_b64.json")
    if os.path.exists(traffic_path):
        with open(traffic_path) as f:
            line["roofline"]["traffic"] = json.load(f).get("traffic_bytes_per_launch")
    # batch sweep of the same format (config C3), plus config C2's (B=8, int8
    # residual, per-head scale) and C4's (B=128, int4, per-row scale) steps;
    # --sweep adds every batch x residual format x scale granularity
    formats = {"int4_head": (qpd.RESID_INT4, True), "int4_row": (qpd.RESID_INT4, False),
               "int8_head": (qpd.RESID_INT8, True), "int8_row": (qpd.RESID_INT8, False)}
    if args.no_sweep:
        cases = []
    elif args.sweep:
        cases = [(bb, f) for bb in (1, 8, 64, 256) for f in formats] + [(128, "int4_row")]
    else:
        cases = [(bb, "int4_head") for bb in (1, 8, 256)] + [(8, "int8_head"), (128, "int4_row")]
    sweep = {}
    if args.batch == 64 and args.resid == "int4" and args.rscale == "head":
        sweep["B64_int4_head"] = {"us": line["us_per_step"], "host_us": line["host_us_per_eager_call"],
                                  "GBps": line["value"], "frac": line["roofline"]["frac"]}
    for bb, fmt_name in cases:
        if f"B{bb}_{fmt_name}" in sweep:
            continue
        fmt, ph = formats[fmt_name]
        groups = max(2, min(64, 1024 // bb))
        m, hm = run_config(device, bb, fmt, ph, args.steps, args.warmup, groups, args.quant_mode)
        nb = algorithmic_bytes(bb, H, HV, K, V, fmt, ph)
        sweep[f"B{bb}_{fmt_name}"] = {"us": round(m * 1e3, 3), "host_us": round(hm * 1e3, 3),
                                     "GBps": round(nb / (m * 1e-3) / 1e9, 1),
                                     "frac": round(nb / (m * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}
    if not args.no_sweep:   # the headline step with vLLM's bf16 activations and output
        m, hm = run_config(device, 64, qpd.RESID_INT4, True, args.steps, args.warmup, 16, args.quant_mode,
                           act_dtype=torch.bfloat16)
        nb = algorithmic_bytes(64, H, HV, K, V, qpd.RESID_INT4, True, act_bytes=2)
        sweep["B64_int4_head_bf16act"] = {"us": round(m * 1e3, 3), "host_us": round(hm * 1e3, 3),
                                          "GBps": round(nb / (m * 1e-3) / 1e9, 1),
                                          "frac": round(nb / (m * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}
    line["sweep"] = dict(sorted(sweep.items(), key=lambda kv: (int(kv[0][1:kv[0].index("_")]), kv[0])))
    if not args.no_sweep:
        # the C5 shape through 24 layers per token: eager vs one graph per token,
        # full and NULL-padded (48 live requests in a batch-64 capture)
        line["multilayer_c5"] = {"full": multilayer_token(device),
                                 "padded": multilayer_token(device, live=48)}
        line["arms"] = arms(device)
        line["arms"].update(ingest_arm(device))
        line["arms"].update(slot_ops_arm(device))
        # measured copy ceiling at the headline's byte count and for a 1 GiB copy
        at = hbm_copy_peak(device, nbytes)
        big = hbm_copy_peak(device, 1 << 30)
        line["copy_peak"] = {"kernel": "ck_hbm_copy (16 B non-temporal load + store per lane, grid-stride)",
                             "at_workload_bytes": at, "large": big,
                             "frac_of_copy_at_workload": round(gbps / at["GBps"], 4),
                             "frac_of_copy_large": round(gbps / big["GBps"], 4)}
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(B, resid_fmt, per_head, args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
