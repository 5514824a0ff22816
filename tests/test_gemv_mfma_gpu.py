"""Linears of 3..8 rows on MFMA (the reference's gemm8 range, Shaders.swift:110-283; the
DiT's M = 6 and the VAE's M = 4): every M on ragged shapes -- K with 32-k block tails and K
past the 2048-k LDS chunk, N not a multiple of the 16-feature tile -- every epilogue flag,
the fused RMSNorm, all activation and weight types; against the fp32 reference loop and the
fp64 recomputation, against the lane-group GEMV (same contract, another kernel), and re-run
bit for bit."""
import numpy as np
import pytest
import torch

import mingtts as mt
import oracle as O
from _gpu_util import assert_linear_parity, dev16, dev_x, expected, run_linear, say

pytestmark = pytest.mark.gpu

SHAPES = [  # (N, K, flags, bias)
    (100, 1000, O.GELU, True),            # N past the tile, K with a 32-k tail (1000 = 31 blocks + 8)
    (1024, 4096, O.ACCUM, True),          # DiT ff2: two LDS chunks
    (3072, 1024, 0, True),                # DiT qkv
    (896, 4864, O.SILU_GATE, False),      # a gated op with 3 chunks (the last one 768 k)
    (16, 64, O.SILU, False),              # one tile, two 32-k blocks
    (64, 2056, O.ACCUM, False),           # the second chunk holds one 8-k piece
]


def _id(s):
    return f"N{s[0]}_K{s[1]}_f{s[2]}"


@pytest.mark.parametrize("M", [3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("shape", SHAPES, ids=_id)
def test_rows_3_to_8(gpu, M, shape):
    N, K, flags, bias = shape
    say(f"gemv_mfma M={M} {_id(shape)}")
    c = O.gemv_case(M, N, K, flags, bias, 1.0, wt=O.BF16)
    got, xu = run_linear(c, O.F32, gpu)
    assert_linear_parity(got, *expected(c, xu), K, f"M={M} {_id(shape)}")
    again, _ = run_linear(c, O.F32, gpu)
    np.testing.assert_array_equal(again, got)
    old = mt.set_tuning(mt.TUNE_GEMV_MFMA, 1)
    try:
        lane, _ = run_linear(c, O.F32, gpu)
    finally:
        mt.set_tuning(mt.TUNE_GEMV_MFMA, old)
    # another kernel and summation order (fp32 FMA dot products; here hi + lo halves on MFMA)
    assert O.normwise_rel_err(got, lane.astype(np.float64)) <= 1e-5


@pytest.mark.parametrize("wt", [O.F16, O.BF16], ids=["wf16", "wbf16"])
@pytest.mark.parametrize("xt", [O.F32, O.F16, O.BF16], ids=["xf32", "xf16", "xbf16"])
def test_types(gpu, xt, wt):
    say(f"gemv_mfma types x{xt} w{wt}")
    c = O.gemv_case(6, 200, 1024, O.GELU, True, 1.0, wt=wt)
    got, xu = run_linear(c, xt, gpu)
    assert_linear_parity(got, *expected(c, xu), 1024, f"x{xt} w{wt}")


@pytest.mark.parametrize("M,N,K,flags", [(6, 3072, 1024, O.BIAS), (6, 4096, 1024, O.GELU | O.BIAS),
                                         (4, 4864, 896, O.SILU_GATE), (5, 96, 4096, 0)])
def test_fused_rmsnorm(gpu, M, N, K, flags):
    """rmsnorm then linear in one pass at 3..8 rows (the DiT's norm1 + qkv, norm2 + ff1)."""
    gated = bool(flags & O.SILU_GATE)
    c = O.gemv_case(M, N, K, flags & ~O.BIAS, bool(flags & O.BIAS), 1.0, wt=O.BF16)
    x = np.ascontiguousarray(c["x"][:M]) * np.float32(4.0)   # without the NaN sentinel rows
    gbits, _ = O.round16(1.0 + 0.1 * O.gaussian(77 + N, K), O.BF16)
    x_d, xu = dev_x(x, O.F32, gpu)
    y_d = torch.from_numpy(c["y0"].copy()).to(gpu)
    say(f"gemv_mfma rmsnorm M={M} N={N} K={K}")
    rc = mt.linear_rmsnorm_raw(x_d, O.F32, dev16(gbits, O.BF16, gpu), dev16(c["w"], O.BF16, gpu),
                               dev16(c["w2"], O.BF16, gpu) if gated else None, O.BF16,
                               dev16(c["bias"], O.BF16, gpu) if c["bias"] is not None else None, y_d,
                               M, N, K, K, N, c["flags"], 1e-6, None)
    assert rc == 0, mt.last_error()
    torch.cuda.synchronize()
    got = y_d.cpu().numpy()
    want64 = O.linear_np64(O.rmsnorm_f64(xu, gbits, O.BF16), c["w"], c["w2"] if gated else None, O.BF16,
                           c["bias"], c["y0"], c["flags"])
    normed32 = O.rmsnorm_f32(xu, gbits, O.BF16)
    want32 = O.linear_f32(normed32, c["w"], c["w2"] if gated else None, O.BF16, c["bias"], c["y0"], M, N, K,
                          c["flags"])
    assert_linear_parity(got, want32, want64, K, f"rmsnorm M={M} N={N} K={K}")


def test_rows_past_m_are_not_read(gpu):
    """x rows past M hold NaN: the staged rows stop at M."""
    M, N, K = 5, 64, 512
    c = O.gemv_case(M, N, K, 0, False, 1.0, wt=O.F16)
    x = np.full((M + 3, K), np.nan, np.float32)
    x[:M] = c["x"][:M]
    x_d = torch.from_numpy(x).to(gpu)
    y_d = torch.zeros(M, N, device=gpu)
    say("gemv_mfma NaN rows past M")
    rc = mt.linear_raw(x_d, O.F32, dev16(c["w"], O.F16, gpu), None, O.F16, None, y_d, M, N, K, K, N, 0, None)
    assert rc == 0, mt.last_error()
    torch.cuda.synchronize()
    got = y_d.cpu().numpy()
    assert np.all(np.isfinite(got))
    assert O.normwise_rel_err(got, O.linear_f64(c["x"][:M], c["w"], None, O.F16, None, None, M, N, K, 0)) <= 1e-5


@pytest.mark.parametrize("splits", [1, 2, 3, 7])
@pytest.mark.parametrize("M,N,K,flags,norm", [(6, 1024, 4096, O.ACCUM, False), (4, 96, 1000, O.SILU_GATE, True),
                                              (8, 300, 2056, O.GELU, True)])
def test_forced_splits_bit_exact_reruns(gpu, splits, M, N, K, flags, norm):
    """Split-K counts forced through MT_TUNE_GEMM_SPLITK (the x^2 sums of a fused norm travel
    with the partial sums): parity, and a re-run bit for bit (the arrival counters re-arm and
    the splits are added in split order)."""
    gated = bool(flags & O.SILU_GATE)
    c = O.gemv_case(M, N, K, flags, False, 1.0, wt=O.F16)
    x = np.ascontiguousarray(c["x"][:M]) * np.float32(3.0)
    gbits, _ = O.round16(1.0 + 0.1 * O.gaussian(5 + K, K), O.F16)
    x_d, xu = dev_x(x, O.F32, gpu)
    say(f"gemv_mfma splits={splits} M={M} N={N} K={K} norm={norm}")
    old = mt.set_tuning(mt.TUNE_GEMM_SPLITK, splits)
    try:
        outs = []
        for _ in range(2):
            y_d = torch.from_numpy(c["y0"].copy()).to(gpu)
            args = (dev16(c["w"], O.F16, gpu), dev16(c["w2"], O.F16, gpu) if gated else None, O.F16, None, y_d,
                    M, N, K, K, N, c["flags"])
            if norm:
                rc = mt.linear_rmsnorm_raw(x_d, O.F32, dev16(gbits, O.F16, gpu), *args, 1e-6, None)
            else:
                rc = mt.linear_raw(x_d, O.F32, *args, None)
            assert rc == 0, mt.last_error()
            torch.cuda.synchronize()
            outs.append(y_d.cpu().numpy())
    finally:
        mt.set_tuning(mt.TUNE_GEMM_SPLITK, old)
    np.testing.assert_array_equal(outs[1], outs[0])
    w2 = c["w2"] if gated else None
    if norm:
        want64 = O.linear_np64(O.rmsnorm_f64(xu, gbits, O.F16), c["w"], w2, O.F16, None, c["y0"], c["flags"])
        want32 = O.linear_f32(O.rmsnorm_f32(xu, gbits, O.F16), c["w"], w2, O.F16, None, c["y0"], M, N, K, c["flags"])
    else:
        want64 = O.linear_f64(xu, c["w"], w2, O.F16, None, c["y0"], M, N, K, c["flags"])
        want32 = O.linear_f32(xu, c["w"], w2, O.F16, None, c["y0"], M, N, K, c["flags"])
    assert_linear_parity(outs[0], want32, want64, K, f"splits {splits} M={M} N={N} K={K}")


@pytest.mark.parametrize("M,xt", [(9, O.F16), (16, O.F16), (33, O.BF16), (64, O.F16), (12, O.F32), (32, O.F32)])
@pytest.mark.parametrize("shape", [(100, 1000, O.GELU, True), (896, 4864, O.SILU_GATE, False),
                                   (1152, 896, O.ACCUM, False)], ids=_id)
def test_skinny_rows_forced(gpu, M, xt, shape):
    """MT_TUNE_GEMV_MFMA = 2: M > 8 on the same kernel with 2 or 4 column groups (x of the
    weights' type staged as it is, other x as hi + lo halves)."""
    N, K, flags, bias = shape
    wt = O.BF16 if xt == O.BF16 else O.F16
    say(f"gemv_mfma skinny M={M} x{xt} {_id(shape)}")
    c = O.gemv_case(M, N, K, flags, bias, 1.0, wt=wt)
    old = mt.set_tuning(mt.TUNE_GEMV_MFMA, 2)
    old_r = mt.set_tuning(mt.TUNE_GEMV_ROWS_MAX, 0)
    try:
        got, xu = run_linear(c, xt, gpu)
        again, _ = run_linear(c, xt, gpu)
    finally:
        mt.set_tuning(mt.TUNE_GEMV_MFMA, old)
        mt.set_tuning(mt.TUNE_GEMV_ROWS_MAX, old_r)
    assert_linear_parity(got, *expected(c, xu), K, f"skinny M={M} {_id(shape)}")
    np.testing.assert_array_equal(again, got)
