"""Helpers of the GPU tests: upload oracle inputs, run through the C ABI, compare."""
import sys

import numpy as np
import torch

import mingtts as mt
import oracle as O

TORCH_T = {O.F32: torch.float32, O.F16: torch.float16, O.BF16: torch.bfloat16}


def say(msg: str) -> None:
    """Names the case about to run on the GPU (flushed, so a fault still leaves it)."""
    print(msg, flush=True)
    sys.stdout.flush()


def dev16(bits: np.ndarray, t: int, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(device).view(TORCH_T[t])


def dev_x(xf32: np.ndarray, xt: int, device) -> tuple[torch.Tensor, np.ndarray]:
    """x on the device in type xt, and the fp32 values the kernel sees."""
    if xt == O.F32:
        return torch.from_numpy(np.ascontiguousarray(xf32)).to(device), xf32
    bits, rounded = O.round16(xf32, xt)
    return dev16(bits, xt, device), rounded


def run_linear(c: dict, xt: int, device, stream=None) -> tuple[np.ndarray, np.ndarray]:
    """Runs a gemv_case dict through mt_linear; returns (gpu y, fp32 x values used)."""
    m, n, k, flags, wt = c["m"], c["n"], c["k"], c["flags"], c["wt"]
    x_d, x_used = dev_x(c["x"], xt, device)
    w_d = dev16(c["w"], wt, device)
    w2_d = dev16(c["w2"], wt, device) if flags & O.SILU_GATE else None
    b_d = dev16(c["bias"], wt, device) if c["bias"] is not None else None
    y_d = torch.from_numpy(c["y0"].copy()).to(device)
    rc = mt.linear_raw(x_d, xt, w_d, w2_d, wt, b_d, y_d, m, n, k, k, n, flags, stream)
    assert rc == 0, mt.last_error()
    torch.cuda.synchronize()
    return y_d.cpu().numpy(), x_used


def expected(c: dict, x_used: np.ndarray):
    """(fp32 reference loop, fp64 recomputation) on the inputs the kernel consumed."""
    m, n, k, flags, wt = c["m"], c["n"], c["k"], c["flags"], c["wt"]
    gw2 = c["w2"] if flags & O.SILU_GATE else None
    want32 = O.linear_f32(x_used[:m], c["w"], gw2, wt, c["bias"], c["y0"], m, n, k, flags)
    want64 = O.linear_f64(x_used[:m], c["w"], gw2, wt, c["bias"], c["y0"], m, n, k, flags)
    return want32, want64


def assert_linear_parity(got: np.ndarray, want32: np.ndarray, want64: np.ndarray, k: int, what: str) -> None:
    """The precision gate: the reference's per-element tolerance (atol 2e-4 sqrt(K)/30,
    rtol 1e-4, KernelTests.swift:58-68, 102) against the fp32 reference loop, and the
    normwise max|y - y64| / max|y64| <= 1e-3 against the fp64 recomputation."""
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    ex, i, g, w = O.worst_violation(got, want32, O.kat_atol(k))
    assert ex <= 0, f"{what}: index {i} got {g} want {w} (excess {ex:.3g})"
    rel = O.normwise_rel_err(got, want64)
    assert rel <= 1e-3, f"{what}: normwise error {rel:.3g} > 1e-3"
