"""GPU parity of the any-K decode path (packed_decode_masked.h): pool rows
whose K is not a power of two from 16 to 256 (K = 1 ... 1024: byte-granular
accesses, 4-byte state and 2- or 4-byte residual accesses when K is a
multiple of 4, or whole 16-byte lanes when K is a multiple of 16), and
power-of-two K whose pool rows are not aligned for the bandwidth kernel's
16-byte lane loads (byte-granular). The reference computes such rows as if
zero-padded to its power-of-two lane count (quantized_packed_decode.py:
123-127,158,165-166,196-202); the oracle does the same. Each case runs
consecutive steps on one pool through the drop-in front end and compares the
output and all four pool tensors bit for bit with the oracle after every
step."""

from __future__ import annotations

import zlib

import numpy as np
import pytest
import torch

import oracle
from carrykernel_amd.vllm_integration import quantized_packed_decode as qpd
from tests._helpers import make_packed_inputs, make_pool

pytestmark = pytest.mark.gpu

I8, I4 = qpd.RESID_INT8, qpd.RESID_INT4
F32, BF16, F16 = torch.float32, torch.bfloat16, torch.float16

# name: K, B, H, HV, V, resid, per_head, mode, act, out, l2norm, NULL fraction, out-of-range id,
#       out-of-place, state bits, steps, pool misaligned by one element
CASES = {
    "k24_int8_row": (24, 4, 2, 4, 40, I8, False, "fast", F32, F32, True, 0.0, False, False, 8, 2, False),
    "k24_int4_head": (24, 4, 2, 4, 40, I4, True, "fast", F32, F32, True, 0.0, False, False, 8, 2, False),
    "k7_int8_head_exact": (7, 3, 1, 2, 33, I8, True, "exact", F32, F32, True, 0.0, False, False, 8, 2, False),
    "k2_int4_row": (2, 5, 2, 2, 17, I4, False, "fast", F32, F32, False, 0.0, False, False, 8, 3, False),
    # the smallest shapes: one code per row, one row per head
    "k1_v1_int8_row": (1, 3, 1, 2, 1, I8, False, "fast", F32, F32, True, 0.0, False, False, 8, 3, False),
    "k1_v3_int8_head_exact": (1, 4, 2, 2, 3, I8, True, "exact", F32, F32, False, 0.25, False, False, 8, 2, False),
    "k100_int8_row_bf16_nulls": (100, 8, 2, 4, 64, I8, False, "fast", BF16, BF16, True, 0.25, True, False, 8, 2,
                                 False),
    "k200_int4_head_gqa": (200, 4, 2, 6, 96, I4, True, "fast", F32, F32, True, 0.0, False, False, 8, 2, False),
    "k96_int8_head_out_of_place": (96, 6, 2, 4, 128, I8, True, "fast", F32, F32, True, 0.0, False, True, 8, 2,
                                   False),
    "k48_f16_int6_exact": (48, 4, 1, 3, 50, I4, False, "exact", F16, F16, True, 0.0, False, False, 6, 2, False),
    "k130_int8_row_many": (130, 40, 2, 8, 128, I8, False, "fast", F32, F32, True, 0.1, False, False, 8, 2, False),
    "k80_int4_head_lanes": (80, 6, 2, 4, 128, I4, True, "fast", F32, F32, True, 0.1, True, False, 8, 2, False),
    "k112_int8_row_exact_lanes": (112, 5, 1, 2, 70, I8, False, "exact", BF16, BF16, True, 0.0, False, False, 8, 2,
                                  False),
    "k192_int4_row_lanes_out_of_place": (192, 6, 2, 4, 128, I4, False, "fast", F16, F32, True, 0.0, False, True, 8,
                                         2, False),
    # 64 x 8 x 4 = 2048 tiles of 32 rows: the one-wave, 4-rows-per-lane shape
    "k96_int4_row_lanes_many_tiles": (96, 64, 2, 8, 128, I4, False, "fast", F32, F32, True, 0.1, True, False, 8, 2,
                                      False),
    "k240_int8_head_lanes": (240, 3, 1, 3, 100, I8, True, "fast", F32, F32, False, 0.0, False, False, 6, 2, False),
    # K a multiple of 4: word accesses; int4 residual rows of K / 2 = 50 and 10 bytes are 2-byte aligned
    "k100_int4_row_words": (100, 6, 2, 4, 64, I4, False, "fast", F32, F32, True, 0.0, False, False, 8, 2, False),
    "k100_int4_head_words_gqa": (100, 4, 2, 8, 120, I4, True, "fast", BF16, F32, True, 0.2, True, False, 8, 2, False),
    "k20_int4_head_words_exact": (20, 4, 1, 2, 40, I4, True, "exact", F32, F32, True, 0.1, True, False, 8, 2, False),
    "k128_misaligned_int4_head": (128, 8, 4, 8, 128, I4, True, "fast", F32, F32, True, 0.1, True, False, 8, 2,
                                  True),
    "k64_misaligned_int8_row_exact": (64, 8, 2, 4, 100, I8, False, "exact", BF16, F32, False, 0.0, False, False, 8,
                                      2, True),
    "k256_misaligned_int4_row_out_of_place": (256, 4, 1, 2, 64, I4, False, "fast", F32, F32, True, 0.0, False,
                                              True, 8, 2, True),
    # K above 256: rows padded to 512 lanes (32 lanes per row) or 1024 (a whole wave per row)
    "k384_int8_row_lanes": (384, 4, 2, 4, 64, I8, False, "fast", F32, F32, True, 0.1, True, False, 8, 2, False),
    "k512_int4_head_lanes_v128": (512, 3, 1, 2, 128, I4, True, "fast", F32, F32, True, 0.0, False, False, 8, 2,
                                  False),
    "k300_int4_row_words_exact": (300, 4, 2, 4, 50, I4, False, "exact", BF16, F32, True, 0.0, False, False, 8, 2,
                                  False),
    "k333_int8_head_bytes_exact": (333, 3, 1, 2, 20, I8, True, "exact", F32, F32, True, 0.0, False, False, 8, 2,
                                   False),
    "k1000_int8_head_words_gqa": (1000, 3, 1, 3, 64, I8, True, "fast", F32, F32, True, 0.0, True, False, 8, 2,
                                  False),
    # 16 x 4 x 32 = 2048 tiles of 4 rows: the one-wave, 4-rows-per-lane shape at 1024 lanes
    "k1024_int4_row_lanes_many_tiles_exact": (1024, 16, 2, 4, 128, I4, False, "exact", F16, F16, True, 0.1, False,
                                              False, 8, 2, False),
    "k520_misaligned_int4_row_out_of_place": (520, 4, 1, 2, 40, I4, False, "fast", F32, F32, True, 0.0, False, True,
                                              8, 2, True),
}


def _dev(arr, device, misalign):
    """A device copy of arr; misaligned: starting one element past an
    allocation boundary, so rows are not 16-byte aligned."""
    t = torch.from_numpy(np.array(arr, copy=True))
    if not misalign:
        return t.to(device)
    buf = torch.empty(t.numel() + 1, dtype=t.dtype, device=device)
    view = buf[1:].view(t.shape)
    view.copy_(t.to(device))
    return view


def _expected_out(o_ref, out_dt):
    if out_dt == BF16:
        return oracle.bf16_round(o_ref)
    if out_dt == F16:
        return o_ref.astype(np.float16).astype(np.float32)
    return o_ref


@pytest.mark.parametrize("name", list(CASES))
def test_masked_decode_bit_exact(device, name):
    K, B, H, HV, V, resid, per_head, mode, act, out_dt, l2norm, null_frac, bad_id, dst_mode, bits, steps, mis = \
        CASES[name]
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    S = 2 * B + 3 if dst_mode else B + 3
    pool = make_pool(S, HV, V, K, resid, per_head, seed=K, bits=bits)
    dpool = [_dev(x, device, mis) for x in pool]
    if mis:
        assert dpool[0].data_ptr() % 16 and dpool[2].data_ptr() % 8
    perm = (rng.permutation(S - 1) + 1).astype(np.int32)
    src = perm[:B].copy()
    src[rng.random(B) < null_frac] = 0
    if bad_id:
        src[int(rng.integers(B))] = S + 2
    dst = perm[B:2 * B].copy() if dst_mode else None
    print(f"case {name}", flush=True)
    for t in range(steps):
        mixed, a, b, A_log, dt_bias = make_packed_inputs(B, H, HV, K, V, seed=7 * K + t, dtype=act)
        scale = K ** -0.5
        out = torch.empty(B, 1, HV, V, dtype=out_dt, device=device)
        qpd.quantized_gated_delta_rule_packed_decode(
            mixed.to(device), a.to(device), b.to(device), A_log.to(device), dt_bias.to(device), scale, *dpool, out,
            torch.from_numpy(src).to(device), use_qk_l2norm_in_kernel=l2norm, resid_fmt=resid, state_bits=bits,
            quant_mode=mode, dst_state_indices=None if dst is None else torch.from_numpy(dst).to(device))
        torch.cuda.synchronize()
        o_ref = oracle.packed_decode(
            mixed.float().numpy(), a.float().numpy(), b.float().numpy(), A_log.float().numpy(),
            dt_bias.float().numpy(), scale, *pool, src, H, use_qk_l2norm=l2norm, resid_fmt=resid,
            per_head=per_head, state_bits=bits, mode=oracle.MODE_EXACT if mode == "exact" else oracle.MODE_FAST,
            dst_indices=dst)
        got = out[:, 0].float().cpu().numpy()
        want = _expected_out(o_ref, out_dt)
        live = (src > 0) & (src < S)
        np.testing.assert_array_equal(got[live], want[live], err_msg=f"{name}: out differs at step {t}")
        assert np.all(got[src == 0] == 0) and np.all(np.isnan(got[src >= S]))
        for tname, d, h in zip(("state_codes", "state_scale", "resid_codes", "resid_scale"), dpool, pool):
            np.testing.assert_array_equal(d.cpu().numpy(), h, err_msg=f"{name}: {tname} differs at step {t}")
        if dst is not None:
            src, dst = dst, src                       # read back what was written
            src = np.where((src > 0) & (src < S), src, 0).astype(np.int32)
            dst = np.where((dst > 0) & (dst < S), dst, 0).astype(np.int32)
