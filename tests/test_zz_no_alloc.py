"""mt_linear_static (the allocation-free mt_linear): through the C ABI, on linears whose K is
split (the pipelined GEMM, with 16-bit and with fp32 x, and the small-row MFMA kernel, whose
partial sums then live in the library's fixed device array), against mt_linear on the same
inputs -- bit for bit, since the kernels and their summation order are the same -- on
consecutive calls, each later one smaller, so a call that found the array dirty from the one
before would show it."""
import numpy as np
import pytest
import torch

import mingtts as mt
import oracle as O
from _gpu_util import say

pytestmark = pytest.mark.gpu


def _case(M, N, K, xt, seed, gpu):
    rng = np.random.default_rng(seed)
    wb, wr = O.round16(rng.standard_normal((N, K)).astype(np.float32) * np.float32(0.05), O.F16)
    w = torch.from_numpy(wb.view(np.int16)).to(gpu).view(torch.float16)
    xf = rng.standard_normal((M, K)).astype(np.float32)
    if xt == mt.F16:
        xb, xr = O.round16(xf, O.F16)
        x = torch.from_numpy(xb.view(np.int16)).to(gpu).view(torch.float16)
    else:
        x, xr = torch.from_numpy(xf).to(gpu), xf
    bias_b, _ = O.round16(rng.standard_normal(N).astype(np.float32) * np.float32(0.1), O.F16)
    bias = torch.from_numpy(bias_b.view(np.int16)).to(gpu).view(torch.float16)
    y0 = rng.standard_normal((M, N)).astype(np.float32)
    return x, xr, w, wb, bias, bias_b, y0


@pytest.mark.parametrize("rounds", [2])
def test_static_linear_matches_mt_linear(gpu, rounds):
    cases = [(64, 896, 4864, mt.F16, mt.KERNEL_GEMM),        # pipelined GEMM, K split
             (64, 896, 4864, mt.F32, mt.KERNEL_GEMM),        # its fp32-x (hi + lo) path, K split in 8
             (6, 1024, 4096, mt.F32, mt.KERNEL_GEMV_MFMA),   # small-row MFMA kernel, K split
             (3, 512, 1024, mt.F32, mt.KERNEL_GEMV_MFMA)]    # smaller again
    for r in range(rounds):
        for M, N, K, xt, fam in cases:
            say(f"static linear round {r} M={M} N={N} K={K}")
            assert mt.linear_kernel(M, N, K, xt=xt, wt=mt.F16) == fam
            x, xr, w, wb, bias, bias_b, y0 = _case(M, N, K, xt, 7 * M + r, gpu)
            flags = mt.GemvFlags.bias | mt.GemvFlags.accumulate
            ys = torch.from_numpy(y0.copy()).to(gpu)
            yd = torch.from_numpy(y0.copy()).to(gpu)
            assert mt.linear_static_raw(x, xt, w, None, mt.F16, bias, ys, M, N, K, K, N, flags) == 0, mt.last_error()
            assert mt.linear_raw(x, xt, w, None, mt.F16, bias, yd, M, N, K, K, N, flags) == 0, mt.last_error()
            torch.cuda.synchronize()
            got, ref = ys.cpu().numpy(), yd.cpu().numpy()
            np.testing.assert_array_equal(got, ref)
            want = O.linear_f64(xr, wb, None, O.F16, bias_b, y0, M, N, K, O.BIAS | O.ACCUM)
            assert O.normwise_rel_err(got, want) <= 1e-5


def test_static_linear_refuses_a_split_beyond_its_scratch(gpu):
    """Forced to 64 K splits, a 512-row linear needs far more partial sums than the fixed
    array holds: refused with MT_ENOTSUP before anything is launched (mt_linear runs it)."""
    M, N, K = 512, 896, 4864
    x, xr, w, wb, bias, bias_b, y0 = _case(M, N, K, mt.F16, 3, gpu)
    y = torch.zeros(M, N, device=gpu)
    old = mt.set_tuning(mt.TUNE_GEMM_SPLITK, 64)
    try:
        say("static linear refusal")
        rc = mt.linear_static_raw(x, mt.F16, w, None, mt.F16, None, y, M, N, K, K, N, 0)
    finally:
        mt.set_tuning(mt.TUNE_GEMM_SPLITK, old)
    assert rc == mt.ENOTSUP and "static scratch" in mt.last_error()
    torch.cuda.synchronize()
    assert float(y.abs().max()) == 0.0
