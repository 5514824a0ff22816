"""The 24-layer prefill chain of backbone linears (QwenForward.dispatches at M prompt rows,
Qwen.swift:72-97): each layer's rmsnorm + qkv, o +=, rmsnorm + gate|up, down += issued as
mt_linear / mt_linear_rmsnorm launches on one stream, fp32 activations chained from op to op
as in the reference, against the same chain in fp64 per op (fp32 between ops).  At M = 64
and 512 every op runs on the MFMA GEMM families."""
import numpy as np
import pytest
import torch

import mingtts as mt
import oracle as O
from _gpu_util import say
from test_seq_gpu import H, INTER, QKV, make_stack

pytestmark = pytest.mark.gpu


def oracle_chain_np(ws, x0):
    """The chain with numpy's fp64 matmul for every op (fp32 activations between ops)."""
    resid = x0.astype(np.float32).copy()
    qkv = mlp = None
    for p in ws:
        qkv = O.linear_np64(O.rmsnorm_f64(resid, p["norm1"], O.F16), p["qkv"], None, O.F16, p["qkv_b"], None,
                            O.BIAS).astype(np.float32)
        resid = O.linear_np64(qkv[:, :H], p["o"], None, O.F16, None, resid, O.ACCUM).astype(np.float32)
        mlp = O.linear_np64(O.rmsnorm_f64(resid, p["norm2"], O.F16), p["gate"], p["up"], O.F16, None, None,
                            O.SILU_GATE).astype(np.float32)
        resid = O.linear_np64(mlp, p["down"], None, O.F16, None, resid, O.ACCUM).astype(np.float32)
    return resid, qkv, mlp


@pytest.mark.parametrize("M", [64, 512])
def test_prefill_chain_matches_fp64(gpu, M):
    ws, x0 = make_stack(24, M, 71 + M, gpu)
    resid = torch.from_numpy(x0.copy()).to(gpu)
    qkv = torch.zeros(M, QKV, device=gpu)
    mlp = torch.zeros(M, INTER, device=gpu)
    assert mt.linear_kernel(M, INTER, H, xt=mt.F32, wt=mt.F16) == mt.KERNEL_GEMM
    say(f"prefill chain 24 layers M={M}")
    for p in ws:
        d = p["dev"]
        mt.linear(resid, d["qkv"], qkv, M, bias=d["qkv_b"], norm=d["norm1"])
        mt.linear(qkv, d["o"], resid, M, flags=mt.GemvFlags.accumulate, ldx=QKV)
        mt.linear(resid, d["gate"], mlp, M, flags=mt.GemvFlags.siluGate, w2=d["up"], norm=d["norm2"])
        mt.linear(mlp, d["down"], resid, M, flags=mt.GemvFlags.accumulate)
    torch.cuda.synchronize()
    want = oracle_chain_np(ws, x0)
    for g, w, what in zip((resid, qkv, mlp), want, ("resid", "qkv", "mlp")):
        got = g.cpu().numpy()
        assert np.all(np.isfinite(got)), what
        rel = O.normwise_rel_err(got, w)
        assert rel <= 1e-3, f"{what}: normwise {rel:.3g}"
