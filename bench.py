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
launch stream. The headline times exactly --steps after exactly --warmup
steps; each ``sweep`` line records the steps and warm-up it timed, at least
those and at least 1 ms / 0.4 ms of work (``sweep_window``).
"""

from __future__ import annotations

import argparse
import ctypes
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
# Sweep lines (not the headline) time a window of at least SWEEP_WINDOW_US of
# device work after at least SWEEP_WARM_US of warm-up steps: each follows the
# CPU leg's check of that line, which leaves the GPU idle, and a 20-step window
# of a 6 us step then reads the clocks' ramp rather than the step.
SWEEP_WINDOW_US = 1000.0
SWEEP_WARM_US = 400.0
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


class CpuLeg:
    """The CPU leg of the bench, the only part of it that loads oracle/.

    * The reference's CPU path timed on this host: oracle/torch_path.py, a
      torch restatement of gdn_quant_step_torch (statequant/kernel.py:149-178)
      in the vLLM layout with int4 nibble packing, on the same workload shape,
      with torch using every core this process may run on.
    * Every timed GPU configuration checked before it is timed: one GPU step on
      the configuration's own buffers and code path, its touched slots and
      outputs compared bit for bit with the C oracle on host copies of the
      same inputs (as experiments/kernel_bench.py:77-91,158-163 checks each
      configuration against its torch path). A mismatch makes the bench fail.
    """

    def __init__(self, seconds_per_batch):
        import numpy as np
        import oracle
        from oracle import torch_path
        self.np = np
        self.oracle = oracle
        self.tp = torch_path
        self.cores = len(os.sched_getaffinity(0))
        self.seconds = seconds_per_batch
        self.checked = []

    # -- the reference CPU path, timed --------------------------------------
    def time_torch_path(self, B, resid_fmt=qpd.RESID_INT4, per_head=True):
        """us per step of the torch restatement at batch B (HV=32, K=V=128,
        fp32, the configs' input distributions), over about `seconds` of
        steps after one untimed step; torch threads = this process's cores."""
        prev = torch.get_num_threads()
        torch.set_num_threads(self.cores)
        try:
            S = B + 1
            g = torch.Generator().manual_seed(B)
            h0 = torch.randn(S, HV, V, K, generator=g) * 0.1
            sc, ss = (torch.from_numpy(x) for x in self.oracle.quantize_rows(h0.numpy()))
            rc = torch.zeros(S, HV, V, K // 2 if resid_fmt == qpd.RESID_INT4 else K, dtype=torch.int8)
            rs = torch.zeros((S, HV) if per_head else (S, HV, V))
            sets, A_log, dt_bias = make_step_inputs(B, 2, "cpu", 5)
            idx = torch.arange(1, S, dtype=torch.int32)

            def step(t):
                mixed, a, b = sets[t % 2]
                self.tp.packed_decode_torch(mixed, a, b, A_log, dt_bias, 1.0, sc, ss, rc, rs, idx, H,
                                            resid_fmt=resid_fmt, per_head=per_head)

            step(0)
            n = 0
            t0 = time.perf_counter()
            while True:
                step(n)
                n += 1
                el = time.perf_counter() - t0
                if el >= self.seconds or n >= 2000:
                    break
        finally:
            torch.set_num_threads(prev)
        us = el / n * 1e6
        nb = algorithmic_bytes(B, H, HV, K, V, resid_fmt, per_head)
        return {"us": round(us, 1), "GBps": round(nb / (us * 1e-6) / 1e9, 3), "steps": n, "seconds": round(el, 2)}

    def time_c_oracle(self, B, resid_fmt=qpd.RESID_INT4, per_head=True, seconds=3.0):
        """us per step of the C oracle (OpenMP over (request, head), every
        core) on the same workload: a second CPU figure beside the torch path."""
        np = self.np
        S = B + 1
        rng = np.random.default_rng(0)
        h0 = (rng.standard_normal((S, HV, V, K)) * 0.1).astype(np.float32)
        sc, ss = self.oracle.quantize_rows(h0)
        rc = np.zeros((S, HV, V, K // 2 if resid_fmt == qpd.RESID_INT4 else K), np.int8)
        rs = np.zeros((S, HV) if per_head else (S, HV, V), np.float32)
        sets, A_log, dt_bias = make_step_inputs(B, 2, "cpu", 5)
        idx = np.arange(1, S, dtype=np.int32)
        n = 0
        t0 = time.perf_counter()
        while True:
            mixed, a, b = sets[n % 2]
            self.oracle.packed_decode(mixed.numpy(), a.numpy(), b.numpy(), A_log.numpy(), dt_bias.numpy(), 1.0,
                                      sc, ss, rc, rs, idx, H, resid_fmt=resid_fmt, per_head=per_head,
                                      nthreads=self.cores)
            n += 1
            el = time.perf_counter() - t0
            if el >= seconds or n >= 2000:
                break
        return {"us": round(el / n * 1e6, 1), "steps": n, "threads": self.cores}

    # -- checks of the GPU steps that are timed -------------------------------
    def _record(self, name, ok, detail=""):
        self.checked.append({"line": name, "ok": bool(ok), **({"detail": detail} if detail else {})})
        if not ok:
            raise RuntimeError(f"bench: the GPU result of {name} differs from the oracle ({detail})")
        return True

    @staticmethod
    def _host(t):
        return t.detach().float().cpu().numpy() if t.dtype in (torch.bfloat16, torch.float16) \
            else t.detach().cpu().numpy().copy()

    def check_packed_decode(self, name, run, pool, ids, inputs, out, resid_fmt, per_head, quant_mode="fast",
                            l2norm=False, scale=1.0, bits=8, Hq=H):
        """run() launches one GPU decode step that reads and writes the slots
        `ids` of `pool` and writes `out`."""
        np, orc = self.np, self.oracle
        torch.cuda.synchronize()
        li = ids.long()
        live = li > 0
        gather = li.clamp(min=0)
        compact = [np.concatenate([np.zeros_like(self._host(x[:1])), self._host(x[gather])]) for x in pool]
        run()
        torch.cuda.synchronize()
        B = ids.shape[0]
        cidx = np.where(live.cpu().numpy(), np.arange(1, B + 1), 0).astype(np.int32)
        mode = orc.MODE_EXACT if quant_mode == "exact" else orc.MODE_FAST
        ref = orc.packed_decode(*(self._host(x).astype(np.float32) for x in inputs), scale, *compact, cidx, Hq,
                                use_qk_l2norm=l2norm, resid_fmt=resid_fmt, per_head=per_head,
                                state_bits=bits, mode=mode)
        got = self._host(out)[:, 0]
        if out.dtype == torch.bfloat16:
            ref = orc.bf16_round(ref)
        ok = np.array_equal(got, ref)
        lv = live.cpu().numpy()
        for x, c in zip(pool, compact):
            ok = ok and np.array_equal(self._host(x[gather])[lv], c[1:][lv])
        return self._record(name, ok, "" if ok else "outputs or state differ")

    def check_quant_step(self, name, run, ins, outs, res_fmt, bits=8):
        """statequant layout: ins = (h_int8, scale, e, e_scale, q, k, v, alpha,
        beta), outs = (o, h_int8, scale, e, e_scale) written by run()."""
        np, orc = self.np, self.oracle

        def resid_store(t):   # the residual as the oracle stores it (fp16 / e5m2 as raw bits)
            if res_fmt == sq.RES_FP16:
                return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)
            if res_fmt == sq.RES_FP8:
                return t.detach().cpu().view(torch.uint8).numpy()
            return self._host(t)

        torch.cuda.synchronize()
        hin = [None if x is None else (resid_store(x) if i == 2 else self._host(x)) for i, x in enumerate(ins)]
        run()
        torch.cuda.synchronize()
        ref = orc.quant_step_kv(hin[0], hin[1], hin[2], hin[3] if res_fmt == sq.RES_INT8 else None, *hin[4:],
                                bits=bits, res_fmt=res_fmt)
        ok = True
        for i, (g, r) in enumerate(zip(outs, ref)):
            if r is None:
                continue
            ok = ok and np.array_equal(resid_store(g) if i == 3 else self._host(g), r)
        return self._record(name, ok, "" if ok else "statequant step differs")

    def check_fp32_step(self, name, run, h, q, k, v, al, be, o, h_out):
        np, orc = self.np, self.oracle
        torch.cuda.synchronize()
        hh = [self._host(x) for x in (h, q, k, v, al, be)]
        run()
        torch.cuda.synchronize()
        h_ref, o_ref = orc.fp32_step_kv(*hh)
        ok = np.array_equal(self._host(o), o_ref) and np.array_equal(self._host(h_out), h_ref)
        return self._record(name, ok, "" if ok else "fp32 step differs")

    def check_float_state(self, name, run, state, ids, inputs, out, Hq=H, l2norm=False, scale=1.0):
        np, orc = self.np, self.oracle
        torch.cuda.synchronize()
        li = ids.long()
        B = ids.shape[0]
        compact = np.concatenate([np.zeros_like(self._host(state[:1])), self._host(state[li])]).astype(np.float32)
        run()
        torch.cuda.synchronize()
        ref = orc.packed_decode_float_state(*(self._host(x).astype(np.float32) for x in inputs), scale, compact,
                                            np.arange(1, B + 1, dtype=np.int32), Hq,
                                            bf16=state.dtype == torch.bfloat16, use_qk_l2norm=l2norm)
        ok = np.array_equal(self._host(out)[:, 0], ref) and np.array_equal(self._host(state[li]), compact[1:])
        return self._record(name, ok, "" if ok else "float-state step differs")

    def check_quantize_rows(self, name, run, x, codes, scale, qmax=127.0, rows=4096):
        np, orc = self.np, self.oracle
        run()
        torch.cuda.synchronize()
        xk = self._host(x.reshape(-1, x.shape[-1])[:rows])
        name_of = {torch.float32: "float32", torch.bfloat16: "bfloat16", torch.float16: "float16"}
        c_ref, s_ref = orc.quantize_rows_in_dtype(xk, name_of[x.dtype], qmax)
        ok = np.array_equal(self._host(codes.reshape(-1, x.shape[-1])[:rows]), c_ref) and \
            np.array_equal(self._host(scale.reshape(-1)[:rows]), s_ref)
        return self._record(name, ok, "" if ok else "row ingest differs")

    def check_quantize_cols(self, name, run, x, codes, scale, qmax=127.0, mats=8):
        np, orc = self.np, self.oracle
        run()
        torch.cuda.synchronize()
        Kx, Vx = x.shape[-2:]
        xk = self._host(x.reshape(-1, Kx, Vx)[:mats])
        c_ref, s_ref = orc.quantize_cols(xk, qmax)
        ok = np.array_equal(self._host(codes.reshape(-1, Kx, Vx)[:mats]), c_ref) and \
            np.array_equal(self._host(scale.reshape(-1, Vx)[:mats]), s_ref)
        return self._record(name, ok, "" if ok else "column ingest differs")


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


def _capture(device, step, ts):
    """One HIP graph holding step(t) for t in ts, captured on a side stream."""
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            for t in ts:
                step(t)
    torch.cuda.current_stream(device).wait_stream(side)
    torch.cuda.synchronize()
    return graph


_hip_runtime = None


def _graph_upload(graph, device):
    """hipGraphUpload of an instantiated graph on the launch stream: puts the
    graph's launch packets and kernel arguments on the device without running
    it, so its first replay costs what every later one does."""
    global _hip_runtime
    if _hip_runtime is None:
        # the HIP runtime already mapped into this process (the one torch
        # uses): opening that same file returns the loaded library's handle
        with open("/proc/self/maps") as maps:
            paths = [ln.split()[-1] for ln in maps if "/libamdhip64.so" in ln]
        if not paths:
            raise RuntimeError("the HIP runtime is not loaded in this process")
        hip = ctypes.CDLL(paths[0])
        hip.hipGraphUpload.restype = ctypes.c_int
        hip.hipGraphUpload.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        _hip_runtime = hip
    st = _hip_runtime.hipGraphUpload(graph.raw_cuda_graph_exec(),
                                     torch.cuda.current_stream(device).cuda_stream)
    if st != 0:
        raise RuntimeError(f"hipGraphUpload failed with status {st}")
    return graph


class StepReplayer:
    """Exactly `warmup` untimed launches of step(t), then exactly `steps`
    timed ones, all graph-replayed, with t running on from the warm-up into
    the timed region: the warm-up runs t = 0 .. warmup-1 and the timed steps
    t = warmup .. warmup+steps-1 (step(t) depends on t only modulo `period`),
    so every timed step's slot group was last touched `period` steps earlier,
    never a few steps earlier by the warm-up. Every graph is captured and
    uploaded when the replayer is built, so nothing is captured between the
    warm-up and the timed region and no graph's first replay is timed. The
    warm-up is warmup // period replays of a graph of steps 0 .. period-1 plus
    one graph of the remainder; the timed steps are replays of one graph of
    at most MAX_GRAPH_STEPS steps (a multiple of `period` when there is more
    than one replay, so each replay ends where the next begins in the
    rotation) plus one graph of the remainder, so a short run is one graph
    launch."""

    MAX_GRAPH_STEPS = 1024

    def __init__(self, device, step, period, steps, warmup):
        self.device, self.steps, self.warmup = device, steps, warmup

        def graph(t0, n):
            return _graph_upload(_capture(device, step, range(t0, t0 + n)), device) if n > 0 else None

        self.warm_full = graph(0, period) if warmup >= period else None
        self.warm_reps = warmup // period
        self.warm_tail = graph(0, warmup % period)
        if steps <= self.MAX_GRAPH_STEPS:
            n_big = steps
        else:
            n_big = max(period, self.MAX_GRAPH_STEPS - self.MAX_GRAPH_STEPS % period)
        self.big = graph(warmup, n_big)
        self.big_reps = steps // n_big if n_big > 0 else 0
        self.tail = graph(warmup + self.big_reps * n_big, steps - self.big_reps * n_big)

    def time_ms_per_step(self):
        """The warm-up, a synchronize, then the timed steps between two HIP
        events on the launch stream, and a synchronize."""
        for _ in range(self.warm_reps):
            self.warm_full.replay()
        if self.warm_tail is not None:
            self.warm_tail.replay()
        torch.cuda.synchronize()
        timer = Timer(self.device)
        timer.start()
        for _ in range(self.big_reps):
            self.big.replay()
        if self.tail is not None:
            self.tail.replay()
        ms = timer.stop_ms() / self.steps
        torch.cuda.synchronize()
        return ms


SLOT_ORDERS = ("random", "sorted", "dense")


def slot_groups(S, B, groups, order, seed=0):
    """The slot ids of each step's batch, `groups` disjoint groups of B ids
    from 1 .. S-1 (slot 0 is the NULL block). random: a random permutation of
    the pool cut into groups, request n reading a random slot (a long-running
    server's slot map); sorted: the same groups, each in ascending slot
    order; dense: group g is the consecutive slots g*B+1 .. (g+1)*B in
    order (a freshly filled pool)."""
    if order == "dense":
        perm = torch.arange(1, S)
    else:
        perm = torch.randperm(S - 1, generator=torch.Generator().manual_seed(seed)) + 1
    out = [perm[i * B:(i + 1) * B] for i in range(groups)]
    if order == "sorted":
        out = [torch.sort(g).values for g in out]
    return [g.to(torch.int32) for g in out]


def sweep_window(nbytes, steps, warmup):
    """(steps, warmup) for a sweep line moving `nbytes` per step: at least the
    driver's K and W, and enough steps, at a step time estimated from the
    bytes at 5 TB/s (5 us at least), for SWEEP_WINDOW_US of timed and
    SWEEP_WARM_US of warm-up work."""
    est_us = max(5.0, nbytes / 5.0e6)
    return max(steps, math.ceil(SWEEP_WINDOW_US / est_us)), max(warmup, math.ceil(SWEEP_WARM_US / est_us))


def run_config(device, B, resid_fmt, per_head, steps, warmup, groups, quant_mode="fast", seed=0,
               act_dtype=torch.float32, cpu=None, name=None, slot_order="random"):
    """One configuration of the decode step: a pool of B * groups + 1 slots
    (state from 64 fp32 warm-up steps), each step on the next group of B
    slots (slot_groups: random by default). Returns {ms: device ms per step
    over exactly `steps` graph-replayed steps, host_ms: host-inclusive ms per
    eager call, validated: the CPU leg's bit-exact check of one step of this
    very configuration (None without a CPU leg)}. `act_dtype` is the dtype of
    mixed_qkv, a, b and out (vLLM runs bf16 activations)."""
    S = B * groups + 1
    state = warm_state(S, device, seed)
    pool = qpd.init_quantized_state(S, HV, V, K, device, h0=state, resid_fmt=resid_fmt,
                                    per_head_resid_scale=per_head)
    del state
    torch.cuda.empty_cache()
    sets, A_log, dt_bias = make_step_inputs(B, 8, device, seed + 1)
    sets = [tuple(x.to(act_dtype) for x in st) for st in sets]
    idx_groups = [g.to(device) for g in slot_groups(S, B, groups, slot_order, seed)]
    out = torch.empty(B, 1, HV, V, device=device, dtype=act_dtype)

    def step(t):
        mixed, a, b = sets[t % len(sets)]
        qpd.quantized_gated_delta_rule_packed_decode(
            mixed, a, b, A_log, dt_bias, 1.0, *pool, out, idx_groups[t % groups],
            resid_fmt=resid_fmt, quant_mode=quant_mode)

    validated = None
    if cpu is not None:
        mixed, a, b = sets[0]
        validated = cpu.check_packed_decode(name or f"B{B}", lambda: step(0), pool, idx_groups[0],
                                            (mixed, a, b, A_log, dt_bias), out, resid_fmt, per_head, quant_mode)

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

    # captured after the eager calls: a short timed run straight after them
    # (graphs captured first) runs up to 15 % slower per step at B=256
    rep = StepReplayer(device, step, groups, steps, warmup)
    ms = rep.time_ms_per_step()
    if not torch.isfinite(out.float()).all():
        raise RuntimeError("non-finite output in the timed run")
    del rep, pool
    torch.cuda.empty_cache()
    return {"ms": ms, "host_ms": host_ms, "validated": validated}


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


def multilayer_token(device, layers=24, B=64, live=None, tokens=20, seed=7, cpu=None):
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

    validated = None
    if cpu is not None:   # layer 0's step of this shape, NULL padding included
        validated = cpu.check_packed_decode(
            f"multilayer_c5_live{live}",
            lambda: qpd.quantized_gated_delta_rule_packed_decode(mixed, a, b, A_log, dt_bias, 1.0, *pools[0],
                                                                 outs[0], idx, resid_fmt=qpd.RESID_INT4),
            pools[0], idx, (mixed, a, b, A_log, dt_bias), outs[0], qpd.RESID_INT4, True)
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
            "graph_us_per_layer": round(graph_ms * 1e3 / layers, 3), "validated": validated,
            "GBps": round(nb / (graph_ms * 1e-3) / 1e9, 1),
            "frac": round(nb / (graph_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}


def ingest_arm(device, slots=257, cpu=None):
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

        validated = cpu.check_quantize_rows(name, lambda: step(0), x, codes, scale) if cpu else None
        ms = _graph_time(device, step, 1, 20, 20)
        nb = rows * K * (esz + 1) + rows * 4
        res[name] = {"us": round(ms * 1e3, 2), "bytes": nb, "GBps": round(nb / (ms * 1e-3) / 1e9, 1),
                     "frac": round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4), "validated": validated}
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

    validated = cpu.check_quantize_cols("ingest_cols_fp32", lambda: cstep(0), x, codes, scale) if cpu else None
    ms = _graph_time(device, cstep, 1, 20, 20)
    nb = slots * HV * K * V * 5 + slots * HV * V * 4
    res["ingest_cols_fp32"] = {"us": round(ms * 1e3, 2), "bytes": nb, "GBps": round(nb / (ms * 1e-3) / 1e9, 1),
                               "frac": round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4), "validated": validated}
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

    # each operation checked once on these buffers, byte for byte against
    # torch's own gather of the same slots (random pool contents first)
    for t in pool:
        t.copy_(torch.randint(-100, 100, t.shape, device=device).to(t.dtype))
    src_before = [t[groups[0].long()].clone() for t in pool]
    copy_step(0)
    ok_copy = all(torch.equal(t[groups[1].long()], b) for t, b in zip(pool, src_before))
    reset_step(1)
    ok_reset = all(bool((t[groups[1].long()] == 0).all()) for t in pool)
    del src_before
    if not (ok_copy and ok_reset):
        raise RuntimeError("bench: slot copy / reset moved the wrong bytes")
    ms = _graph_time(device, copy_step, 3, 20, 20)
    nb = 2 * n * slot_bytes
    res["pool_copy_slots"] = {"us": round(ms * 1e3, 2), "bytes": nb, "GBps": round(nb / (ms * 1e-3) / 1e9, 1),
                              "frac": round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4), "validated": ok_copy}
    ms = _graph_time(device, reset_step, 4, 20, 20)
    nb = n * slot_bytes
    res["pool_reset_slots"] = {"us": round(ms * 1e3, 2), "bytes": nb, "GBps": round(nb / (ms * 1e-3) / 1e9, 1),
                               "frac": round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4), "validated": ok_reset}
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


def arms(device, batches=(8, 64), steps=800, cpu=None):
    """The other entry points at config shapes (HV=32, K=V=128, fp32
    activations): the statequant-layout step for each residual format, its fp32
    baseline, and the unquantized fp32 / bf16 state arms of the vLLM-layout
    decode. Out-of-place steps ping-pong between buffer sets whose total exceeds
    the 256 MB MALL. Returns {name: {us, GBps, frac}}."""
    from carrykernel_amd import _native
    L = _native.lib()
    res = {}
    gen = torch.Generator(device=device).manual_seed(3)

    def rec(name, ms, nbytes, validated=None):
        res[name] = {"us": round(ms * 1e3, 3), "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1),
                     "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4), "validated": validated}

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
            name = f"statequant_B{B}_{sq.residual_label(res_fmt)}"
            validated = None
            if cpu is not None:
                a_, b_ = sets[0], sets[1]
                validated = cpu.check_quant_step(name, lambda: step(0), (*a_, q, k, v, al, be),
                                                 (o, *b_), res_fmt)
            ms = _graph_time(device, step, nsets, -(-200 // nsets), max(2, steps // nsets))
            rec(name, ms, statequant_bytes(B, HV, K, V, res_fmt), validated)
            del sets
        # fp32 baseline step, ping-pong between state buffers
        nsets = max(2, min(64, -(-(512 << 20) // (B * HV * K * V * 4))))
        hsets = [torch.randn(B, HV, K, V, device=device, generator=gen) * 0.1 for _ in range(nsets)]

        def fstep(t):
            st = L.ck_gdn_fp32_step(hsets[t % nsets].data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                    al.data_ptr(), be.data_ptr(), o.data_ptr(), hsets[(t + 1) % nsets].data_ptr(),
                                    B, HV, K, V, _native.stream_handle(device))
            _native.check(st, "fp32 step")
        validated = cpu.check_fp32_step(f"fp32_step_B{B}", lambda: fstep(0), hsets[0], q, k, v, al, be, o,
                                        hsets[1]) if cpu else None
        ms = _graph_time(device, fstep, nsets, -(-200 // nsets), max(2, steps // nsets))
        rec(f"fp32_step_B{B}", ms, B * HV * (2 * 4 * K * V + 2 * 4 * K + 2 * 4 * V + 8), validated)
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
        validated = None
        if cpu is not None:
            mixed, a, b = sets_in[0]
            validated = cpu.check_float_state(f"vllm_{name}_state_B{B}", lambda: vstep(0), state, idxs[0],
                                              (mixed, a, b, A_log, dt_bias), out)
        ms = _graph_time(device, vstep, groups, -(-200 // groups), max(2, steps // groups))
        rec(f"vllm_{name}_state_B{B}", ms, float_state_bytes(B, H, HV, K, V, esz), validated)
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
    """One step of the unquantized state arm (ck_gdn_packed_decode_float_state)
    on an fp32 or bf16 state pool; every tensor's dtype code is its own (the
    kernel addresses the pool by the state dtype it is given)."""
    from carrykernel_amd import _native
    if state.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"the state arm takes a float32 or bfloat16 pool, got {state.dtype}")
    for t, nm in ((mixed, "mixed_qkv"), (a, "a"), (b, "b"), (A_log, "A_log"), (dt_bias, "dt_bias"), (out, "out")):
        _native.dtype_code(t, nm)
    S, hv, v, k = state.shape
    dc = _native.dtype_code
    st = _native.lib().ck_gdn_packed_decode_float_state(
        mixed.data_ptr(), dc(mixed, "mixed_qkv"), mixed.stride(0), a.data_ptr(), dc(a, "a"), a.stride(0),
        b.data_ptr(), dc(b, "b"), b.stride(0), A_log.data_ptr(), dc(A_log, "A_log"), dt_bias.data_ptr(),
        dc(dt_bias, "dt_bias"), float(scale), state.data_ptr(), dc(state, "state"), state.stride(0),
        out.data_ptr(), dc(out, "out"), idx.data_ptr(), idx.stride(0), S, mixed.shape[0],
        (mixed.shape[1] - hv * v) // (2 * k), hv, k, v, int(l2norm),
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


def _single_item_timeline(B, resid_fmt, per_head, rel, start, begin, data, end, cu_id):
    """Timeline summary of a launch of the one-item kernel (one workgroup per
    item, started by the dispatcher as CU slots free): when workgroups start,
    each one's chain from its start to its end, and when each CU finishes."""
    import numpy as np
    st = rel[:, 0]
    cus = np.unique(cu_id)
    first_wave = np.array([int(np.count_nonzero((cu_id == c) & (st < np.nanmin(st) + 0.5))) for c in cus])
    cu_end = np.array([np.nanmax(end[cu_id == c]) for c in cus])
    pct = lambda x, q: round(float(np.nanpercentile(x, q)), 2)   # noqa: E731
    return {"workload": f"B={B} {'int4' if resid_fmt == qpd.RESID_INT4 else 'int8'} residual, "
                        f"{'per-head' if per_head else 'per-row'} scale",
            "kernel": "packed_decode_single_kernel (one item per workgroup)",
            "workgroups": int(len(st)), "cus": int(len(cus)),
            "started_within_0.5us_per_cu_median": float(np.median(first_wave)),
            "start_us": {"p50": pct(st, 50), "p90": pct(st, 90), "max": pct(st, 100)},
            "from_start_us": {"slot_id_known": pct(start[:, 0] - st, 50),
                              "loads_issued": pct(start[:, 1] - st, 50),
                              "gates_done": pct(start[:, 2] - st, 50),
                              "data_in": pct(data - st, 50), "end": pct(end - st, 50),
                              "end_p10": pct(end - st, 10), "end_p90": pct(end - st, 90)},
            "compute_us": {"p50": pct(end - data, 50), "p90": pct(end - data, 90)},
            "cu_last_end_us": {"p50": round(float(np.median(cu_end)), 2), "p90": round(float(np.percentile(cu_end, 90)), 2),
                               "max": round(float(cu_end.max()), 2)},
            "span_us": round(float(np.nanmax(end)), 2)}


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
    slots, max_wg = 40, 8192
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
    if int(n_rec.max()) == 1:
        return {"timeline": _single_item_timeline(B, resid_fmt, per_head, rel, start, begin[:, 0], data[:, 0],
                                                  end[:, 0], cu_id)}
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
    ap.add_argument("--slot-order", choices=SLOT_ORDERS, default="random",
                    help="slot ids of each step's batch (slot_groups): random (default), sorted, dense")
    ap.add_argument("--resid", choices=("int4", "int8"), default="int4")
    ap.add_argument("--rscale", choices=("head", "row"), default="head")
    ap.add_argument("--quant-mode", choices=("fast", "exact"), default="fast")
    ap.add_argument("--sweep", action="store_true",
                    help="time every B in {1, 8, 64, 256} x residual format x scale granularity (default: "
                         "the headline format at B in {1, 8, 64, 256} and the C2 / C4 steps)")
    ap.add_argument("--no-cpu", action="store_true",
                    help="skip the CPU leg (the reference CPU path timing and the oracle checks of each line)")
    ap.add_argument("--no-sweep", action="store_true",
                    help="time only the headline configuration (no batch sweep, no other entry points)")
    ap.add_argument("--drift", action="store_true",
                    help="instead: config C5 drift (24 layers x B=64 x 2048 tokens, int8 and int6 state) "
                         "against the fp32 state arm; prints one JSON line")
    ap.add_argument("--drift-tokens", type=int, default=2048)
    ap.add_argument("--cpu-seconds", type=float, default=4.0,
                    help="seconds of CPU-path steps timed per batch in the CPU leg")
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

    cpu = None if args.no_cpu else CpuLeg(args.cpu_seconds)
    r = run_config(device, B, resid_fmt, per_head, args.steps, args.warmup, args.groups, args.quant_mode,
                   cpu=cpu, name=f"B{B}_{args.resid}_{args.rscale}_{args.quant_mode}", slot_order=args.slot_order)
    ms, host_ms = r["ms"], r["host_ms"]
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
        "dtype": "f32",   # the arithmetic; storage: int8 state codes, int4 / int8 residual codes (config)
        "data": "synthetic (config distributions; state from 64 fp32 warm-up steps)",
        "config": {"workload": "C3: single-layer fused decode, int8 per-V state + packed int4 EF residual "
                               "(per-head scale), vLLM [slots,HV,V,K] layout",
                   "batch": B, "value_heads": HV, "qk_heads": H, "K": K, "V": V, "state": "int8",
                   "resid": args.resid, "resid_scale": args.rscale, "quant_mode": args.quant_mode,
                   "pool_slots": B * args.groups + 1, "slot_order": args.slot_order},
        "validated": r["validated"],
        "roofline": {"bound": "hbm", "achieved": round(gbps, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None,
                     "bytes_per_launch": nbytes},
        "bytes_vs_bf16_state": round(bf16_state_bytes(B, H, HV, K, V) / nbytes, 4),
    }
    traffic_path = os.path.join(HERE, "profiles", "traffic_packed_decode_b64.json")
    # the measured traffic belongs to the headline configuration only
    headline = (B == 64 and args.resid == "int4" and args.rscale == "head" and args.quant_mode == "fast")
    if headline and os.path.exists(traffic_path):
        with open(traffic_path) as f:
            line["roofline"]["traffic"] = json.load(f).get("traffic_bytes_per_launch")
    # batch sweep of the same format (config C3) in both arithmetic modes at
    # B = 64 and 256, plus config C2's (B=8, int8 residual, per-head scale)
    # and C4's (B=128, int4, per-row scale) steps; --sweep adds every batch x
    # residual format x scale granularity. Every entry is checked by the CPU
    # leg before it is timed, and the C3 batches carry the reference CPU
    # path's time at the same batch.
    formats = {"int4_head": (qpd.RESID_INT4, True), "int4_row": (qpd.RESID_INT4, False),
               "int8_head": (qpd.RESID_INT8, True), "int8_row": (qpd.RESID_INT8, False)}
    if args.no_sweep:
        cases = []
    elif args.sweep:
        cases = [(bb, f, "fast") for bb in (1, 8, 64, 256) for f in formats] + [(128, "int4_row", "fast")]
    else:
        cases = [(bb, "int4_head", "fast") for bb in (1, 8, 256)] + [(8, "int8_head", "fast"),
                                                                      (1, "int4_row", "fast"),
                                                                      (128, "int4_row", "fast")]
    if not args.no_sweep:
        cases += [(64, "int4_head", "exact"), (256, "int4_head", "exact")]
    sweep = {}

    def key(bb, fmt_name, mode):
        return f"B{bb}_{fmt_name}" + ("" if mode == "fast" else "_exact")

    if args.batch == 64 and args.resid == "int4" and args.rscale == "head":
        sweep[key(64, "int4_head", args.quant_mode)] = {
            "us": line["us_per_step"], "host_us": line["host_us_per_eager_call"], "GBps": line["value"],
            "frac": line["roofline"]["frac"], "steps": args.steps, "warmup": args.warmup,
            "validated": r["validated"]}
    for bb, fmt_name, mode in cases:
        if key(bb, fmt_name, mode) in sweep:
            continue
        fmt, ph = formats[fmt_name]
        groups = max(2, min(64, 1024 // bb))
        nb = algorithmic_bytes(bb, H, HV, K, V, fmt, ph)
        st, wu = sweep_window(nb, args.steps, args.warmup)
        rr = run_config(device, bb, fmt, ph, st, wu, groups, mode, cpu=cpu, name=key(bb, fmt_name, mode))
        sweep[key(bb, fmt_name, mode)] = {"us": round(rr["ms"] * 1e3, 3), "host_us": round(rr["host_ms"] * 1e3, 3),
                                          "GBps": round(nb / (rr["ms"] * 1e-3) / 1e9, 1),
                                          "frac": round(nb / (rr["ms"] * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                                          "steps": st, "warmup": wu, "validated": rr["validated"]}
    if not args.no_sweep:   # the headline step with vLLM's bf16 activations and output
        nb = algorithmic_bytes(64, H, HV, K, V, qpd.RESID_INT4, True, act_bytes=2)
        st, wu = sweep_window(nb, args.steps, args.warmup)
        rr = run_config(device, 64, qpd.RESID_INT4, True, st, wu, 16, args.quant_mode,
                        act_dtype=torch.bfloat16, cpu=cpu, name="B64_int4_head_bf16act")
        sweep["B64_int4_head_bf16act"] = {"us": round(rr["ms"] * 1e3, 3), "host_us": round(rr["host_ms"] * 1e3, 3),
                                          "GBps": round(nb / (rr["ms"] * 1e-3) / 1e9, 1),
                                          "frac": round(nb / (rr["ms"] * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                                          "steps": st, "warmup": wu, "validated": rr["validated"]}
    if not args.no_sweep:
        # the C5 shape through 24 layers per token: eager vs one graph per token,
        # full and NULL-padded (48 live requests in a batch-64 capture)
        line["multilayer_c5"] = {"full": multilayer_token(device, cpu=cpu),
                                 "padded": multilayer_token(device, live=48, cpu=cpu)}
        line["arms"] = arms(device, cpu=cpu)
        line["arms"].update(ingest_arm(device, cpu=cpu))
        line["arms"].update(slot_ops_arm(device))
        # measured copy ceiling at the headline's byte count and for a 1 GiB copy
        at = hbm_copy_peak(device, nbytes)
        big = hbm_copy_peak(device, 1 << 30)
        line["copy_peak"] = {"kernel": "ck_hbm_copy (16 B non-temporal load + store per lane, grid-stride)",
                             "at_workload_bytes": at, "large": big,
                             "frac_of_copy_at_workload": round(gbps / at["GBps"], 4),
                             "frac_of_copy_large": round(gbps / big["GBps"], 4)}
    if cpu is not None:
        # the reference CPU path at every C3 batch the sweep times (and the
        # headline's), on this host's cores; bytes per step as on the GPU
        by_batch = {}
        for bb in sorted({B} | ({1, 8, 64, 256} if not args.no_sweep else set())):
            by_batch[bb] = cpu.time_torch_path(bb, resid_fmt if bb == B else qpd.RESID_INT4,
                                               per_head if bb == B else True)
            k_ = key(bb, "int4_head", "fast")
            if k_ in sweep:
                sweep[k_]["cpu_us"] = by_batch[bb]["us"]
                sweep[k_]["gpu_vs_cpu"] = round(by_batch[bb]["us"] / sweep[k_]["us"], 1)
        head = by_batch[B]
        line["cpu_baseline"] = {
            "value": head["GBps"], "unit": "GB/s", "us_per_step": head["us"],
            "cores": cpu.cores, "threads": cpu.cores, "kind": "port",
            "sample": (f"{head['steps']} steps of the B={B} workload ({head['seconds']} s) through "
                       "oracle/torch_path.py, a torch restatement of the reference CPU path "
                       "(statequant/kernel.py:149-178) in the vLLM layout, torch threads = "
                       f"{cpu.cores} = the cores this process may run on"),
            "by_batch": {str(bb): v for bb, v in by_batch.items()},
            "c_oracle_us_per_step": cpu.time_c_oracle(B, resid_fmt, per_head),
            "validated_lines": len(cpu.checked),
        }
    line["sweep"] = dict(sorted(sweep.items(), key=lambda kv: (int(kv[0][1:kv[0].index("_")]), kv[0])))
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
