"""Host-side tests without a GPU: the C ABI library loads and exports every
declared symbol, argument errors come back as status codes, the Python
front ends raise the reference's errors, and nothing falls back to the CPU."""

from __future__ import annotations

import ctypes
import os
import re

import pytest
import torch

from carrykernel_amd import _native, build
from carrykernel_amd.statequant import kernel as sq
from carrykernel_amd.vllm_integration import quantized_packed_decode as qpd

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "carrykernel_gdn.h")


def _declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(ck_\w+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def L():
    if not _native.library_available():
        pytest.skip("library not built")
    return _native.lib()


def test_library_exports_every_declared_symbol(L):
    declared = _declared_symbols()
    assert len(declared) >= 8
    raw = ctypes.CDLL(_native.LIB_PATH)
    for name in declared:
        assert hasattr(raw, name), f"{name} declared in include/carrykernel_gdn.h but not exported"
    assert set(declared) == set(_native.exported_symbols())
    assert L.ck_abi_version() == _native.ABI_VERSION


def _pd_args(**over):
    """Argument list of ck_gdn_packed_decode with dummy (never dereferenced) pointers."""
    p = ctypes.c_void_p(16)
    a = dict(mixed=p, qkv_dtype=0, stride_qkv=384, a=p, a_dtype=0, stride_a=2, b=p, b_dtype=0, stride_b=2,
             A_log=p, A_log_dtype=0, dt_bias=p, dt_bias_dtype=0, scale=1.0,
             state=p, stride_state=2 * 64 * 128, sscale=p, stride_sscale=128, resid=p,
             stride_resid=2 * 64 * 64, rscale=p, stride_rscale=2, out=p, out_dtype=0, idx=p, stride_idx=1,
             num_slots=4, B=1, H=1, HV=2, K=128, V=64, l2=0, resid_fmt=1, rscale_mode=1, bits=8, mode=0,
             stream=None)
    a.update(over)
    return list(a.values())


@pytest.mark.parametrize("over,status,msg", [
    (dict(K=1030), _native.CK_EUNSUPPORTED, "K must be at most 1024"),
    # a per-head residual scale keeps a whole head in one workgroup: 64 rows of 1024 codes at most
    (dict(K=1024, V=128, stride_state=2 * 128 * 1024, stride_sscale=256, stride_resid=2 * 128 * 512),
     _native.CK_EUNSUPPORTED, "per-head residual scale supports V <= 64 at K=1024, got V=128"),
    (dict(K=25), _native.CK_EINVAL, "even K"),
    (dict(HV=3, H=2), _native.CK_EINVAL, "multiple of H"),
    (dict(qkv_dtype=7), _native.CK_EINVAL, "dtype"),
    (dict(resid_fmt=5), _native.CK_EINVAL, "resid_fmt"),
    (dict(rscale_mode=9), _native.CK_EINVAL, "rscale_mode"),
    (dict(mode=4), _native.CK_EINVAL, "quant_mode"),
    (dict(bits=9), _native.CK_EINVAL, "state_bits"),
    (dict(num_slots=0), _native.CK_EINVAL, "num_slots"),
    (dict(mixed=None), _native.CK_EINVAL, "null pointer"),
    (dict(stride_state=-1), _native.CK_EUNSUPPORTED, "strides must be"),
])
def test_packed_decode_argument_errors(L, over, status, msg):
    rc = L.ck_gdn_packed_decode(*_pd_args(**over))
    assert rc == status
    assert msg in L.ck_last_error().decode()


def test_packed_decode_empty_batch_is_ok(L):
    assert L.ck_gdn_packed_decode(*_pd_args(B=0)) == _native.CK_OK
    assert L.ck_last_error().decode() == ""


def test_packed_decode_empty_batch_with_null_pointers(L):
    """B = 0 with every pointer NULL (an empty tensor's data pointer): the
    in-place and the out-of-place step return CK_OK and launch nothing; with
    B > 0 a NULL destination id array is refused."""
    nulls = {k: None for k in ("mixed", "a", "b", "A_log", "dt_bias", "state", "sscale", "resid", "rscale",
                               "out", "idx")}
    at = 26   # ck_gdn_packed_decode_to takes (dst ids, stride) after (ids, stride)
    args = _pd_args(B=0, **nulls)
    assert L.ck_gdn_packed_decode(*args) == _native.CK_OK
    assert L.ck_gdn_packed_decode_to(*args[:at], None, 1, *args[at:]) == _native.CK_OK
    args = _pd_args()
    assert L.ck_gdn_packed_decode_to(*args[:at], None, 1, *args[at:]) == _native.CK_EINVAL
    assert "dst_state_indices is NULL" in L.ck_last_error().decode()


def test_other_entry_points_argument_errors(L):
    p = ctypes.c_void_p(16)
    # the statequant step takes any K in 1..256 (rows zero-padded to a power of two); B = 0 checks and
    # launches nothing, so these run without a GPU
    for k_ok in (1, 24, 48, 96, 100, 256):
        assert L.ck_gdn_quant_step(p, p, p, p, p, p, p, p, p, p, p, p, p, p, 0, 1, k_ok, 6, 127.0, 0, 0, None) == 0
        assert L.ck_gdn_fp32_step(p, p, p, p, p, p, p, p, 0, 1, k_ok, 6, None) == 0
    for k_bad in (257, 512):
        rc = L.ck_gdn_quant_step(p, p, p, p, p, p, p, p, p, p, p, p, p, p, 1, 1, k_bad, 6, 127.0, 0, 0, None)
        assert rc == _native.CK_EUNSUPPORTED and "K must be in 1..256" in L.ck_last_error().decode()
        rc = L.ck_gdn_fp32_step(p, p, p, p, p, p, p, p, 1, 1, k_bad, 6, None)
        assert rc == _native.CK_EUNSUPPORTED and "K must be in 1..256" in L.ck_last_error().decode()
    odd = ctypes.c_void_p(17)   # an fp16 residual at an odd address
    rc = L.ck_gdn_quant_step(p, p, odd, p, p, p, p, p, p, p, p, p, p, p, 1, 1, 32, 6, 127.0, 1, 0, None)
    assert rc == _native.CK_EINVAL and "2-byte aligned" in L.ck_last_error().decode()
    rc = L.ck_gdn_quant_step(p, p, p, p, p, p, p, p, p, p, p, p, p, p, 1, 1, 32, 8, 12.5, 0, 0, None)
    assert rc == _native.CK_EINVAL and "qmax" in L.ck_last_error().decode()
    rc = L.ck_gdn_quant_step(p, p, p, None, p, p, p, p, p, p, p, p, p, None, 1, 1, 32, 8, 127.0, 3, 0, None)
    assert rc == _native.CK_EINVAL and "e_scale" in L.ck_last_error().decode()
    rc = L.ck_gdn_fp32_step(p, p, p, p, p, p, p, p, 1, 1, 300, 8, None)
    assert rc == _native.CK_EUNSUPPORTED
    rc = L.ck_quantize_rows(p, 9, 128, 4, 128, 127.0, p, p, None)
    assert rc == _native.CK_EINVAL
    rc = L.ck_set_max_items_per_launch(-1)
    assert rc == _native.CK_EINVAL and "item limit" in L.ck_last_error().decode()
    assert L.ck_set_max_items_per_launch(0) == _native.CK_OK
    for bad in (-1, 3):
        rc = L.ck_set_decode_kernel(bad)
        assert rc == _native.CK_EINVAL and "decode kernel" in L.ck_last_error().decode()
    assert L.ck_set_decode_kernel(_native.DECODE_KERNEL_AUTO) == _native.CK_OK
    rc = L.ck_quantize_cols(p, 1, 32, 8, 300.0, p, p, None)
    assert rc == _native.CK_EINVAL
    rc = L.ck_gdn_packed_decode_float_state(p, 0, 384, p, 0, 2, p, 0, 2, p, 0, p, 0, 1.0, p, 2, 100, p, 0, p, 1,
                                            4, 1, 1, 2, 128, 64, 0, None)
    assert rc == _native.CK_EINVAL and "float32 or bfloat16" in L.ck_last_error().decode()
    rc = L.ck_hbm_copy(p, p, 24, 0, None)
    assert rc == _native.CK_EINVAL and "multiple of 16" in L.ck_last_error().decode()
    rc = L.ck_hbm_copy(ctypes.c_void_p(8), p, 32, 0, None)
    assert rc == _native.CK_EINVAL and "aligned" in L.ck_last_error().decode()
    assert L.ck_hbm_copy(None, None, 0, 0, None) == _native.CK_OK


# ---------------------------------------------------------------------------
# Python front ends: the reference's ValueErrors (quantized_packed_decode.py:268-309)
# ---------------------------------------------------------------------------

def _cpu_case(B=2, H=2, HV=4, K=64, V=32, resid_fmt=qpd.RESID_INT4):
    S = 3
    rk = K // 2 if resid_fmt == qpd.RESID_INT4 else K
    return dict(mixed_qkv=torch.zeros(B, 2 * H * K + HV * V), a=torch.zeros(B, HV), b=torch.zeros(B, HV),
                A_log=torch.zeros(HV), dt_bias=torch.zeros(HV), scale=1.0,
                state_codes=torch.zeros(S, HV, V, K, dtype=torch.int8), state_scale=torch.zeros(S, HV, V),
                resid_codes=torch.zeros(S, HV, V, rk, dtype=torch.int8), resid_scale=torch.zeros(S, HV, V),
                out=torch.zeros(B, 1, HV, V), ssm_state_indices=torch.tensor([1, 2], dtype=torch.int32),
                resid_fmt=resid_fmt)


@pytest.mark.parametrize("mutate,msg", [
    (lambda c: c.update(mixed_qkv=torch.zeros(2, 3, 4)), "mixed_qkv must be 2-D"),
    (lambda c: c.update(mixed_qkv=torch.zeros(512, 2).t()), "contiguous in its last dimension"),
    (lambda c: c.update(state_codes=torch.zeros(3, 4, 32, dtype=torch.int8)), "state_codes must be 4-D"),
    (lambda c: c.update(state_codes=torch.zeros(3, 4, 64, 32, dtype=torch.int8).transpose(2, 3)),
     "state_codes must be contiguous in its last dimension"),
    (lambda c: c.update(resid_codes=c["resid_codes"].float()), "must be int8 storage"),
    (lambda c: c.update(resid_codes=torch.zeros(3, 4, 32, 64, dtype=torch.int8)), "packed two codes per byte"),
    (lambda c: c.update(resid_fmt=qpd.RESID_INT8), "same shape as the state"),
    (lambda c: c.update(ssm_state_indices=torch.tensor([[1, 2]], dtype=torch.int32)), "must be 1-D"),
    (lambda c: c.update(ssm_state_indices=torch.tensor([1, 2])), "must be int32"),
    (lambda c: c.update(out=torch.zeros(2, 4, 32)), "out must be"),
    (lambda c: c.update(out=torch.zeros(2, 1, 32, 4).transpose(2, 3)), "out must be contiguous"),
    (lambda c: c.update(mixed_qkv=torch.zeros(2, 4 * 32 + 1)), "cannot infer H"),
    (lambda c: c.update(resid_scale=torch.zeros(3, 5)), "resid_scale must be"),
    (lambda c: c.update(state_scale=torch.zeros(3, 4, 32, dtype=torch.float16)), "state_scale must be"),
])
def test_qpd_value_errors(mutate, msg):
    c = _cpu_case()
    mutate(c)
    with pytest.raises(ValueError, match=re.escape(msg)):
        qpd.quantized_gated_delta_rule_packed_decode(**c)


def test_qpd_k_limits():
    """K above 1024 is refused; an odd K cannot hold an int4 residual (two
    codes per byte: the reference's packing check, quantized_packed_decode.py:
    278-281, fires before its even-K check at :306-307, which the C ABI keeps);
    any other K is accepted and, on CPU tensors, stops at the missing GPU (no
    host path)."""
    c = _cpu_case(K=1040, resid_fmt=qpd.RESID_INT8)
    with pytest.raises(ValueError, match="packed decode supports K <= 1024"):
        qpd.quantized_gated_delta_rule_packed_decode(**c)
    c = _cpu_case(K=24, resid_fmt=qpd.RESID_INT4)
    c.update(mixed_qkv=torch.zeros(2, 2 * 2 * 25 + 4 * 32),
             state_codes=torch.zeros(3, 4, 32, 25, dtype=torch.int8),
             resid_codes=torch.zeros(3, 4, 32, 12, dtype=torch.int8))
    with pytest.raises(ValueError, match="packed two codes per byte"):
        qpd.quantized_gated_delta_rule_packed_decode(**c)
    for K, fmt in ((48, qpd.RESID_INT8), (7, qpd.RESID_INT8), (100, qpd.RESID_INT4), (264, qpd.RESID_INT8),
                   (1024, qpd.RESID_INT4)):
        with pytest.raises(_native.HipUnavailable):
            qpd.quantized_gated_delta_rule_packed_decode(**_cpu_case(K=K, resid_fmt=fmt))


def test_qpd_no_cpu_fallback():
    """Valid arguments on CPU tensors: the op refuses (HipUnavailable, a
    RuntimeError) instead of computing anything on the host."""
    with pytest.raises(_native.HipUnavailable):
        qpd.quantized_gated_delta_rule_packed_decode(**_cpu_case())
    with pytest.raises(_native.HipUnavailable):
        qpd.init_quantized_state(2, 4, 32, 64, "cpu")
    B, HV, K, V = 1, 2, 32, 8
    z = torch.zeros
    with pytest.raises(_native.HipUnavailable):
        sq.gdn_quant_step_fused(z(B, HV, K, V, dtype=torch.int8), z(B, HV, V), z(B, HV, K, V), None, z(B, HV, K),
                                z(B, HV, K), z(B, HV, V), z(B, HV), z(B, HV))
    with pytest.raises(_native.HipUnavailable):
        sq.gdn_step_fused_fp32(z(B, HV, K, V), z(B, HV, K), z(B, HV, K), z(B, HV, V), z(B, HV), z(B, HV))
    with pytest.raises(_native.HipUnavailable):
        sq.per_v_channel_quantize(z(2, K, V))


def test_statequant_shape_errors():
    B, HV, K, V = 1, 2, 32, 8
    z = torch.zeros
    for bad in (z(5), z(2, 0, V), z(2, K, 0)):
        with pytest.raises(ValueError):
            sq.per_v_channel_quantize(bad)
    with pytest.raises(AssertionError):
        sq.gdn_quant_step_fused(z(B, HV, K, V), z(B, HV, V), z(B, HV, K, V), None, z(B, HV, K), z(B, HV, K),
                                z(B, HV, V), z(B, HV), z(B, HV))
    with pytest.raises(ValueError, match="e must be"):
        sq.gdn_quant_step_fused(z(B, HV, K, V, dtype=torch.int8), z(B, HV, V), z(B, HV, K, V), None, z(B, HV, K),
                                z(B, HV, K), z(B, HV, V), z(B, HV), z(B, HV), res_fmt=sq.RES_FP16)
    with pytest.raises(ValueError, match="e_scale"):
        sq.gdn_quant_step_fused(z(B, HV, K, V, dtype=torch.int8), z(B, HV, V), z(B, HV, K, V, dtype=torch.int8),
                                None, z(B, HV, K), z(B, HV, K), z(B, HV, V), z(B, HV), z(B, HV),
                                res_fmt=sq.RES_INT8)
    with pytest.raises(ValueError, match="k must be"):
        sq.gdn_quant_step_fused(z(B, HV, K, V, dtype=torch.int8), z(B, HV, V), z(B, HV, K, V), None, z(B, HV, K),
                                z(B, HV, K + 1), z(B, HV, V), z(B, HV), z(B, HV))


def test_native_module_host_checks():
    """cuda/binding.py's contract without a GPU: load_extension raises
    CudaUnavailable (binding.py:31,49-50); the module's launchers reject a host
    state with the check_state message (gdn_state_kernel.cu:299-302) before
    touching the library."""
    from carrykernel_amd.hip import binding
    if torch.cuda.is_available():
        pytest.skip("checks the no-GPU path")
    with pytest.raises(binding.CudaUnavailable, match="no GPU"):
        binding.load_extension()
    with pytest.raises(binding.CudaUnavailable):
        binding.gdn_fp32_step_cuda(*(torch.zeros(1) for _ in range(6)))
    ext = binding.HipModule(None)
    z = torch.zeros
    with pytest.raises(RuntimeError, match="h_in must be a CUDA tensor"):
        ext.gdn_quant_step(z(1, 1, 4, 4, dtype=torch.int8), *(z(1) for _ in range(13)), 127.0, 0, 128)
    with pytest.raises(RuntimeError, match="h_in must be a CUDA tensor"):
        ext.gdn_fp32_step(z(1, 1, 4, 4), *(z(1) for _ in range(7)), 128)


def test_debug_index_checks():
    qpd._check_indices_host(torch.tensor([0, 2, 3, 0], dtype=torch.int32), 4)
    with pytest.raises(ValueError, match="duplicate"):
        qpd._check_indices_host(torch.tensor([1, 2, 1], dtype=torch.int32), 4)
    with pytest.raises(ValueError, match=">= num_slots"):
        qpd._check_indices_host(torch.tensor([1, 4], dtype=torch.int32), 4)


def test_reference_constants():
    """quantized_packed_decode.py:73-83 and statequant/kernel.py:56-66."""
    assert (qpd.QMAX_INT8, qpd.QMAX_INT4, qpd.EPS, qpd.SOFTPLUS_THRESHOLD, qpd.NULL_BLOCK_ID) == (
        127.0, 7.0, 1e-12, 20.0, 0)
    assert (qpd.RESID_INT8, qpd.RESID_INT4) == (0, 1)
    assert (sq.RES_FP32, sq.RES_FP16, sq.RES_FP8, sq.RES_INT8) == (0, 1, 2, 3)
    assert [sq.residual_bytes(f) for f in range(4)] == [4, 2, 1, 1]
    assert [sq.residual_label(f) for f in range(4)] == ["fp32", "fp16", "fp8", "int8"]
    assert sq.residual_dtype(sq.RES_FP8) == torch.float8_e5m2


def test_product_never_imports_the_oracle():
    pkg = os.path.join(REPO, "carrykernel_amd")
    for root, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp")):
                text = open(os.path.join(root, f)).read()
                assert not re.search(r"^\s*(import|from)\s+oracle\b", text, re.M), f
                assert "gdn_oracle" not in text, f


def test_build_flags():
    flags = " ".join(build.HIPCC_FLAGS)
    assert "--offload-arch=gfx950" in flags
    assert "-packed-fp32-ops" in flags and "-ffp-contract=off" in flags


def test_slot_contiguity_check_matches_its_definition():
    """The per-call check (dense fast paths, general loop otherwise) against a
    restatement of the rule: every dim after the slot dim is row-major dense,
    size-1 dims may have any stride."""
    def rule(t):
        expect = 1
        for size, stride in zip(reversed(t.shape[1:]), reversed(t.stride()[1:])):
            if size != 1 and stride != expect:
                return False
            expect *= size
        return True

    g = torch.Generator().manual_seed(0)
    cases = []
    for shape in [(5, 4, 3, 8), (5, 1, 3, 8), (5, 4, 1, 8), (5, 4, 3, 1), (3, 6, 7), (3, 1, 7), (4, 9), (4, 1)]:
        base = torch.empty(shape)
        cases += [base, base[:, ...]]
        back = torch.empty((shape[0], base[0].numel() + 5))       # padded slots (a view per slot row)
        cases.append(back[:, :base[0].numel()].view(shape))
        if len(shape) >= 3:
            cases.append(base.transpose(-1, -2))                    # not row-major inside a slot
            cases.append(torch.empty(shape[:-1] + (shape[-1] * 2,))[..., ::2])  # strided last dim
    for _ in range(40):                                             # random size-1 dims with odd strides
        shape = tuple(int(x) for x in torch.randint(1, 4, (4,), generator=g))
        strides = tuple(int(x) for x in torch.randint(1, 50, (4,), generator=g))
        cases.append(torch.empty(1000).as_strided(shape, strides))
    for t in cases:
        assert qpd._slot_contiguous(t) == rule(t), (tuple(t.shape), t.stride())


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU and says so for --gpus N > 1 (exit status 2)."""
    import subprocess
    import sys
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 2
    assert "only --gpus 1" in r.stderr and r.stdout == ""


@pytest.mark.parametrize("steps,warmup,period", [(20, 5, 16), (2000, 200, 16), (1, 0, 16), (1024, 16, 16),
                                                 (1025, 17, 16), (3000, 3, 8), (16, 15, 16), (3000, 7, 12),
                                                 (2100, 30, 100)])
def test_bench_times_exactly_k_steps(monkeypatch, steps, warmup, period):
    """The bench's replayer runs exactly `warmup` steps before the start
    event, exactly `steps` steps between the two events and nothing after; the
    timed steps are at most ceil(steps / 1024) + 1 graph launches, and every
    graph is captured (and uploaded) before the warm-up. The step indices
    run on from the warm-up into the timed region, modulo the rotation
    period: the warm-up replays t = 0 .. warmup-1 and the timed region
    t = warmup .. warmup+steps-1, so no timed step re-reads a slot group that
    the warm-up touched fewer than `period` steps before."""
    import bench
    log, marks = [], {}

    class FakeGraph:
        def __init__(self, ts):
            self.ts = list(ts)
            marks.setdefault("captures_at", []).append(len(log))

        def replay(self):
            log.extend(self.ts)

    class FakeTimer:
        def __init__(self, device):
            pass

        def start(self):
            marks["start"] = len(log)

        def stop_ms(self):
            marks["stop"] = len(log)
            return 1.0

    launches = []
    real_replay = FakeGraph.replay

    def counting_replay(self):
        launches.append(len(log))
        real_replay(self)

    FakeGraph.replay = counting_replay
    monkeypatch.setattr(bench, "_capture", lambda device, step, ts: FakeGraph(ts))
    monkeypatch.setattr(bench, "_graph_upload", lambda graph, device: graph)
    monkeypatch.setattr(bench, "Timer", FakeTimer)
    monkeypatch.setattr(bench.torch.cuda, "synchronize", lambda *a, **k: None)
    rep = bench.StepReplayer("cpu", None, period, steps, warmup)
    ms = rep.time_ms_per_step()
    assert all(at == 0 for at in marks["captures_at"])
    assert marks["start"] == warmup
    assert marks["stop"] - marks["start"] == steps
    assert len(log) == marks["stop"]
    assert [t % period for t in log] == [t % period for t in range(warmup + steps)]
    timed_launches = sum(1 for at in launches if at >= marks["start"])
    assert timed_launches <= -(-steps // bench.StepReplayer.MAX_GRAPH_STEPS) + 1
    assert ms == pytest.approx(1.0 / steps)


def test_init_quantized_state_checks_h0_before_allocating():
    """init_quantized_state rejects an h0 of the wrong shape or a non-float
    dtype with ValueError before it touches a device; a float h0 on the host
    is accepted (it is copied to the pool's GPU, which this host lacks)."""
    from carrykernel_amd import _native
    from carrykernel_amd.vllm_integration import quantized_packed_decode as qpd
    with pytest.raises(ValueError, match="h0 must be"):
        qpd.init_quantized_state(2, 1, 16, 16, "cuda", h0=torch.zeros(2, 1, 16, 8))
    with pytest.raises(ValueError, match="floating-point"):
        qpd.init_quantized_state(2, 1, 16, 16, "cuda", h0=torch.zeros(2, 1, 16, 16, dtype=torch.int32))
    with pytest.raises(_native.HipUnavailable):
        qpd.init_quantized_state(2, 1, 16, 16, "cpu", h0=torch.zeros(2, 1, 16, 16, dtype=torch.float64))


def test_bench_float_state_step_passes_each_dtype_code(monkeypatch):
    """bench.float_state_step hands the state arm the pool's own dtype code
    (a bf16 pool addressed as fp32 would be read and written at twice its
    size), and refuses pools of other dtypes before any call."""
    import bench
    calls = []

    class FakeLib:
        def ck_gdn_packed_decode_float_state(self, *args):
            calls.append(args)
            return 0

    monkeypatch.setattr(_native, "lib", lambda: FakeLib())
    monkeypatch.setattr(_native, "stream_handle", lambda dev: None)
    B, H_, HV_, K_, V_ = 2, 1, 2, 16, 16
    mixed = torch.zeros(B, 2 * H_ * K_ + HV_ * V_, dtype=torch.bfloat16)
    a = torch.zeros(B, HV_)
    b = torch.zeros(B, HV_, dtype=torch.float16)
    A_log = torch.zeros(HV_)
    dt = torch.zeros(HV_)
    out = torch.zeros(B, 1, HV_, V_)
    idx = torch.tensor([1, 2], dtype=torch.int32)
    for sdt, code in ((torch.float32, 0), (torch.bfloat16, 1)):
        state = torch.zeros(3, HV_, V_, K_, dtype=sdt)
        bench.float_state_step(state, mixed, a, b, A_log, dt, 1.0, out, idx, False)
        args = calls[-1]
        assert args[15] == code                        # state dtype
        assert (args[1], args[4], args[7], args[10], args[12], args[18]) == (1, 0, 2, 0, 0, 0)
    with pytest.raises(ValueError, match="float32 or bfloat16"):
        bench.float_state_step(torch.zeros(3, HV_, V_, K_, dtype=torch.float16), mixed, a, b, A_log, dt, 1.0,
                               out, idx, False)
    assert len(calls) == 2


def test_bench_slot_groups_orders():
    """bench.slot_groups: every order gives `groups` disjoint batches of B
    slot ids from 1 .. S-1 (never the NULL block 0); sorted holds the random
    order's groups in ascending order; dense holds consecutive slots."""
    import bench
    S, B, groups = 4 * 16 + 1, 16, 4
    rnd = bench.slot_groups(S, B, groups, "random", seed=3)
    srt = bench.slot_groups(S, B, groups, "sorted", seed=3)
    dns = bench.slot_groups(S, B, groups, "dense")
    for gs in (rnd, srt, dns):
        ids = torch.cat(gs).tolist()
        assert len(gs) == groups and all(len(g) == B and g.dtype == torch.int32 for g in gs)
        assert len(set(ids)) == len(ids) and min(ids) >= 1 and max(ids) <= S - 1
    for a, b in zip(rnd, srt):
        assert sorted(a.tolist()) == b.tolist()
    assert any(a.tolist() != b.tolist() for a, b in zip(rnd, srt))
    assert [g.tolist() for g in dns] == [list(range(1 + i * B, 1 + (i + 1) * B)) for i in range(groups)]


def test_bench_sweep_window():
    """bench.sweep_window: never fewer than the driver's K / W; small steps
    get enough steps for 1 ms of timed and 0.4 ms of warm-up work at the
    5 us floor; a step estimated above 1 ms keeps K and W."""
    import bench
    assert bench.sweep_window(1, 20, 5) == (200, 80)              # 5 us floor
    nb64 = bench.algorithmic_bytes(64, 32, 32, 128, 128, qpd.RESID_INT4, True)
    assert bench.sweep_window(nb64, 20, 5) == (47, 19)            # ~21.4 us at 5 TB/s
    assert bench.sweep_window(nb64, 100, 50) == (100, 50)
    assert bench.sweep_window(10 * 5.0e9, 20, 5) == (20, 5)       # 10 ms estimate
