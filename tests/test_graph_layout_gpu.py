"""GPU tests of how callers use the decode: captured in a HIP graph over a
multi-layer loop with NULL-slot padding, and on pools whose slots are views
with padding between them (a cache that interleaves other per-slot state)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from carrykernel_amd.vllm_integration import quantized_packed_decode as qpd
from tests._helpers import make_packed_inputs, make_pool

pytestmark = pytest.mark.gpu


def _layer_pools(layers, S, HV, V, K, device, resid_fmt, per_head, seed):
    g = torch.Generator().manual_seed(seed)
    return [list(qpd.init_quantized_state(S, HV, V, K, device, h0=(torch.randn(S, HV, V, K, generator=g) * 0.1)
                                          .to(device), resid_fmt=resid_fmt, per_head_resid_scale=per_head))
            for _ in range(layers)]


@pytest.mark.parametrize("resid_fmt,per_head", [(qpd.RESID_INT4, True), (qpd.RESID_INT8, False)])
def test_graph_captured_multilayer_decode(device, resid_fmt, per_head, layers=4, H=8, HV=16, K=64, V=64):
    """A decode step over `layers` layers captured once and replayed, with the
    batch padded by NULL-block ids (the padding a captured batch size needs).
    Each replay (new activations copied into the static inputs, eager work
    and synchronizations between replays) must equal the same step run
    eagerly on a copy of the pools, bit for bit."""
    B, S = 8, 12
    idx = torch.tensor([3, 0, 7, 1, 0, 11, 5, 0], dtype=torch.int32, device=device)
    pools = _layer_pools(layers, S, HV, V, K, device, resid_fmt, per_head, seed=21)
    ref_pools = [[t.clone() for t in p] for p in pools]
    static_in = [[x.to(device) for x in make_packed_inputs(B, H, HV, K, V, seed=100 + l)] for l in range(layers)]
    outs = [torch.empty(B, 1, HV, V, device=device) for _ in range(layers)]

    def step(pool_set, out_set):
        for l in range(layers):
            mixed, a, b, A_log, dt_bias = static_in[l]
            qpd.quantized_gated_delta_rule_packed_decode(mixed, a, b, A_log, dt_bias, K ** -0.5, *pool_set[l],
                                                         out_set[l], idx, use_qk_l2norm_in_kernel=True,
                                                         resid_fmt=resid_fmt)

    # capture on a side stream (the warm-up call settles the occupancy query)
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        warm = [[t.clone() for t in p] for p in pools]
        step(warm, [torch.empty_like(o) for o in outs])
    torch.cuda.current_stream(device).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        step(pools, outs)
    torch.cuda.synchronize()
    # capture does not execute: the pools are still the initial state
    for p, r in zip(pools, ref_pools):
        for t, u in zip(p, r):
            assert torch.equal(t, u)

    ref_outs = [torch.empty_like(o) for o in outs]
    for rep in range(3):
        print(f"case graph replay {rep} resid={resid_fmt} per_head={per_head}", flush=True)
        for l in range(layers):
            fresh = make_packed_inputs(B, H, HV, K, V, seed=1000 * rep + l)
            for dst, src in zip(static_in[l][:3], fresh[:3]):
                dst.copy_(src.to(device))
        graph.replay()
        torch.cuda.synchronize()
        step(ref_pools, ref_outs)          # eager, same inputs, on the copies
        torch.cuda.synchronize()
        _ = torch.randn(1000, device=device).sum().item()   # unrelated eager work between replays
        for l in range(layers):
            assert torch.equal(outs[l], ref_outs[l]), f"layer {l} output differs on replay {rep}"
            assert torch.all(outs[l][1] == 0) and torch.all(outs[l][4] == 0) and torch.all(outs[l][7] == 0)
            for t, u in zip(pools[l], ref_pools[l]):
                assert torch.equal(t, u), f"layer {l} pool differs on replay {rep}"


@pytest.mark.parametrize("resid_fmt,per_head", [(qpd.RESID_INT4, True), (qpd.RESID_INT4, False),
                                                (qpd.RESID_INT8, True)])
def test_padded_slot_strides(device, resid_fmt, per_head, H=4, HV=8, K=128, V=128):
    """Pool tensors that are views with 256 spare bytes (64 floats for the
    scales) after every slot: results equal the oracle's on the unpadded
    pool and the padding is never written."""
    B, S = 3, 5
    pool = make_pool(S, HV, V, K, resid_fmt, per_head, seed=9)
    padded = []
    for arr, pad in zip(pool, (256, 64, 256, 64)):
        flat = torch.from_numpy(np.ascontiguousarray(arr)).reshape(S, -1)
        big = torch.full((S, flat.shape[1] + pad), 77 if arr.dtype == np.int8 else -5.0,
                         dtype=flat.dtype)
        big[:, :flat.shape[1]] = flat
        big = big.to(device)
        padded.append((big, big[:, :flat.shape[1]].view(arr.shape)))
    views = [v for _, v in padded]
    assert views[0].stride(0) == HV * V * K + 256
    idx = np.array([4, 0, 2], np.int32)
    mixed, a, b, A_log, dt_bias = make_packed_inputs(B, H, HV, K, V, seed=31)
    out = torch.empty(B, 1, HV, V, device=device)
    print(f"case padded strides resid={resid_fmt} per_head={per_head}", flush=True)
    qpd.quantized_gated_delta_rule_packed_decode(
        mixed.to(device), a.to(device), b.to(device), A_log.to(device), dt_bias.to(device), K ** -0.5, *views,
        out, torch.from_numpy(idx).to(device), use_qk_l2norm_in_kernel=True, resid_fmt=resid_fmt)
    torch.cuda.synchronize()
    host = [x.copy() for x in pool]
    o_ref = oracle.packed_decode(mixed.numpy(), a.numpy(), b.numpy(), A_log.numpy(), dt_bias.numpy(), K ** -0.5,
                                 *host, idx, H, use_qk_l2norm=True, resid_fmt=resid_fmt, per_head=per_head)
    np.testing.assert_array_equal(out[:, 0].cpu().numpy(), o_ref)
    for (big, view), h, pad in zip(padded, host, (256, 64, 256, 64)):
        np.testing.assert_array_equal(view.cpu().numpy(), h)
        tail = big[:, big.shape[1] - pad:].cpu()
        assert torch.all(tail == (77 if big.dtype == torch.int8 else -5.0)), "padding between slots was written"


def test_concurrent_calls_from_two_threads(device, H=8, HV=16, K=128, V=128, B=16, T=12):
    """The C ABI keeps no per-call state outside its arguments (the occupancy
    cache is filled once under a lock): two host threads, each driving its own
    pool on its own stream, give the same results as the same steps run one
    after the other."""
    import threading

    def run(pool_h, seed, stream, outs):
        pool = [torch.from_numpy(np.array(x, copy=True)).to(device) for x in pool_h]
        idx = torch.arange(1, B + 1, dtype=torch.int32, device=device)
        steps = [[x.to(device) for x in make_packed_inputs(B, H, HV, K, V, seed=seed + t)] for t in range(T)]
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            for mixed, a, b, A_log, dt_bias in steps:
                out = torch.empty(B, 1, HV, V, device=device)
                qpd.quantized_gated_delta_rule_packed_decode(mixed, a, b, A_log, dt_bias, 0.1, *pool, out, idx,
                                                             resid_fmt=qpd.RESID_INT4)
                outs.append(out)
        stream.synchronize()
        outs.extend(pool)

    pools = [make_pool(B + 1, HV, V, K, qpd.RESID_INT4, True, seed=s) for s in (81, 82)]
    # sequential reference
    ref = [[], []]
    for i in range(2):
        run(pools[i], 100 * i, torch.cuda.Stream(device), ref[i])
    print("case two host threads, two streams", flush=True)
    got = [[], []]
    threads = [threading.Thread(target=run, args=(pools[i], 100 * i, torch.cuda.Stream(device), got[i]))
               for i in range(2)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=60)
        assert not th.is_alive()
    for i in range(2):
        assert len(got[i]) == len(ref[i])
        for x, y in zip(got[i], ref[i]):
            assert torch.equal(x, y)
