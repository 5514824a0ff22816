"""The persistent linear sequence (mt_seq_*) on the GPU: the decode step's chain of backbone
linears (Qwen.swift:85-91 per layer) against an fp64 oracle chain, against the same ops
issued one mt_linear at a time, across re-runs (bit for bit) and workgroup counts."""
import numpy as np
import pytest
import torch

import mingtts as mt
import oracle as O
from _gpu_util import dev16, say

pytestmark = pytest.mark.gpu

H, QKV, INTER = 896, 1152, 4864


def make_stack(layers: int, M: int, seed: int, device, wt=O.F16):
    """Per-layer 16-bit weights of type wt ~ N(0, 0.02^2) (qkv with bias, o, gate, up, down)
    and RMSNorm gains ~ 1 + N(0, 0.1^2), seeded per layer from the SplitMix64 normal stream."""
    ws = []
    for l in range(layers):
        n = QKV * H + QKV + H * H + 2 * INTER * H + H * INTER
        z = O.gaussian(seed * 1000 + l, n, 0.02)
        bits, _ = O.round16(z, wt)
        o = 0
        parts = {}
        for name, size, shape in (("qkv", QKV * H, (QKV, H)), ("qkv_b", QKV, (QKV,)), ("o", H * H, (H, H)),
                                  ("gate", INTER * H, (INTER, H)), ("up", INTER * H, (INTER, H)),
                                  ("down", H * INTER, (H, INTER))):
            parts[name] = bits[o:o + size].reshape(shape)
            o += size
        gains = 1.0 + O.gaussian(seed * 1000 + 500 + l, 2 * H, 0.1)
        parts["norm1"], _ = O.round16(gains[:H], wt)
        parts["norm2"], _ = O.round16(gains[H:], wt)
        parts["dev"] = {k: dev16(v, wt, device) for k, v in parts.items()}
        ws.append(parts)
    x0 = O.gaussian(seed + 7, M * H)
    return ws, x0.reshape(M, H)


def chain_ops(ws, M, resid, qkv, mlp):
    """The decode chain of one Qwen layer's linears (Qwen.swift:84-91) with the RMSNorms fused:
    qkv = rmsnorm(resid; g1) Wqkv^T + b; resid += qkv[:, :896] Wo^T (the attention output
    stand-in); mlp = silu(n Wg^T) * (n Wu^T) with n = rmsnorm(resid; g2); resid += mlp Wd^T."""
    ops = []
    for p in ws:
        d = p["dev"]
        ops.append(mt.op(resid, d["qkv"], qkv, M, bias=d["qkv_b"], norm=d["norm1"]))
        ops.append(mt.op(qkv, d["o"], resid, M, flags=mt.GemvFlags.accumulate, ldx=QKV))
        ops.append(mt.op(resid, d["gate"], mlp, M, flags=mt.GemvFlags.siluGate, w2=d["up"], norm=d["norm2"]))
        ops.append(mt.op(mlp, d["down"], resid, M, flags=mt.GemvFlags.accumulate))
    return ops


def oracle_chain(ws, x0, M, wt=O.F16):
    """The same chain in fp64 per op, activations stored as fp32 between ops (as on the GPU)."""
    resid = x0.astype(np.float32).copy()
    qkv = mlp = None
    for p in ws:
        qkv = O.linear_np64(O.rmsnorm_f64(resid, p["norm1"], wt), p["qkv"], None, wt, p["qkv_b"], None,
                            0).astype(np.float32)
        resid = O.linear_f64(np.ascontiguousarray(qkv[:, :H]), p["o"], None, wt, None, resid, M, H, H,
                             O.ACCUM).astype(np.float32)
        mlp = O.linear_np64(O.rmsnorm_f64(resid, p["norm2"], wt), p["gate"], p["up"], wt, None, None,
                            O.SILU_GATE).astype(np.float32)
        resid = O.linear_f64(mlp, p["down"], None, wt, None, resid, M, H, INTER, O.ACCUM).astype(np.float32)
    return resid, qkv, mlp


def buffers(M, x0, device):
    resid = torch.from_numpy(x0.copy()).to(device)
    qkv = torch.zeros(M, QKV, device=device)
    mlp = torch.zeros(M, INTER, device=device)
    return resid, qkv, mlp


@pytest.mark.parametrize("layers,M", [(4, 2), (24, 2), (3, 1)])
def test_decode_chain_matches_fp64_oracle(gpu, layers, M):
    say(f"seq chain layers={layers} M={M}")
    ws, x0 = make_stack(layers, M, 11 + M, gpu)
    resid, qkv, mlp = buffers(M, x0, gpu)
    seq = mt.Seq(chain_ops(ws, M, resid, qkv, mlp))
    seq.run()
    torch.cuda.synchronize()
    seq.check()
    want_r, want_q, want_m = oracle_chain(ws, x0, M)
    for got, want, what in ((resid, want_r, "resid"), (qkv, want_q, "qkv"), (mlp, want_m, "mlp")):
        g = got.cpu().numpy()
        assert np.all(np.isfinite(g)), what
        rel = O.normwise_rel_err(g, want)
        assert rel <= 1e-3, f"{what}: normwise {rel:.3g}"
    seq.close()


@pytest.mark.parametrize("layers,M", [(24, 2), (4, 1), (3, 4)])
def test_decode_layer_kernel_matches_general_kernel(gpu, layers, M):
    """A plan that repeats the Qwen2-0.5B decode layer runs the kernel specialised for its
    shapes; MT_TUNE_SEQ_LAYER = 1 runs the same plan on the general sequence kernel.  Each is
    bit-exact from run to run; they split K differently, so they agree to fp32 rounding, and
    both meet the fp64 oracle chain.  (M = 4, the VAE stack's rows, exceeds the general
    kernel's activation staging at K = 4864: there the oracle alone is the reference.)"""
    ws, x0 = make_stack(layers, M, 31 + M, gpu)
    resid, qkv, mlp = buffers(M, x0, gpu)
    ops = chain_ops(ws, M, resid, qkv, mlp)
    outs = {}
    for mode in ((0, 1) if M <= 2 else (0,)):
        old = mt.set_tuning(mt.TUNE_SEQ_LAYER, mode)
        try:
            seq = mt.Seq(ops)
        finally:
            mt.set_tuning(mt.TUNE_SEQ_LAYER, old)
        say(f"seq layers={layers} M={M} layer-kernel mode {mode} kernel {seq.kernel} groups {seq.groups}")
        assert seq.kernel == (mt.SEQ_DECODE_LAYER if mode == 0 else mt.SEQ_GENERAL)
        runs = []
        for _ in range(2):
            resid.copy_(torch.from_numpy(x0))
            qkv.zero_()
            mlp.zero_()
            seq.run()
            torch.cuda.synchronize()
            runs.append([t.cpu().numpy().copy() for t in (resid, qkv, mlp)])
        seq.check()
        seq.close()
        for a, b in zip(runs[0], runs[1]):
            np.testing.assert_array_equal(a, b)
        outs[mode] = runs[0]
    want = oracle_chain(ws, x0, M)
    for j, what in enumerate(("resid", "qkv", "mlp")):
        g = outs[0][j]
        assert np.all(np.isfinite(g)), what
        assert O.normwise_rel_err(g, want[j]) <= 1e-3, what
        if 1 in outs:
            assert O.normwise_rel_err(g, outs[1][j].astype(np.float64)) <= 1e-5, what


def test_layer_shapes_with_other_dataflow_run_the_general_kernel(gpu):
    """A plan with the decode layer's shapes whose downs accumulate into a buffer of their own
    (each layer's down reads the previous down's output as its old y, while o accumulates
    into the residual): the decode-layer kernel splits down over K into two planes that only
    qkv's x and o's old y add, so the plan compiler must give this plan to the general
    kernel, whose result matches the fp64 chain of the same dataflow."""
    M, layers = 2, 3
    ws, x0 = make_stack(layers, M, 71, gpu)
    resid, qkv, mlp = buffers(M, x0, gpu)
    side0 = O.gaussian(73, M * H).reshape(M, H).astype(np.float32)
    side = torch.from_numpy(side0.copy()).to(gpu)
    ops = []
    for p in ws:
        d = p["dev"]
        ops.append(mt.op(resid, d["qkv"], qkv, M, bias=d["qkv_b"], norm=d["norm1"]))
        ops.append(mt.op(qkv, d["o"], resid, M, flags=mt.GemvFlags.accumulate, ldx=QKV))
        ops.append(mt.op(resid, d["gate"], mlp, M, flags=mt.GemvFlags.siluGate, w2=d["up"], norm=d["norm2"]))
        ops.append(mt.op(mlp, d["down"], side, M, flags=mt.GemvFlags.accumulate))
    seq = mt.Seq(ops)
    say(f"seq other-dataflow layers={layers} M={M} kernel {seq.kernel}")
    assert seq.kernel == mt.SEQ_GENERAL
    seq.run()
    torch.cuda.synchronize()
    seq.check()
    seq.close()
    r, s = x0.astype(np.float32).copy(), side0.copy()
    q = m = None
    for p in ws:
        q = O.linear_np64(O.rmsnorm_f64(r, p["norm1"], O.F16), p["qkv"], None, O.F16, p["qkv_b"], None,
                          0).astype(np.float32)
        r = O.linear_f64(np.ascontiguousarray(q[:, :H]), p["o"], None, O.F16, None, r, M, H, H,
                         O.ACCUM).astype(np.float32)
        m = O.linear_np64(O.rmsnorm_f64(r, p["norm2"], O.F16), p["gate"], p["up"], O.F16, None, None,
                          O.SILU_GATE).astype(np.float32)
        s = O.linear_f64(m, p["down"], None, O.F16, None, s, M, H, INTER, O.ACCUM).astype(np.float32)
    for got, want, what in ((resid, r, "resid"), (side, s, "side"), (qkv, q, "qkv"), (mlp, m, "mlp")):
        g = got.cpu().numpy()
        assert np.all(np.isfinite(g)), what
        assert O.normwise_rel_err(g, want) <= 1e-3, what


@pytest.mark.parametrize("M", [1, 2, 4])
def test_decode_layer_kernel_with_bf16_weights(gpu, M):
    """The reference's checkpoints hold bf16 weights (Weights.swift): the decode-layer kernel's
    bf16 instantiation (bf16 MFMA, the hi + lo split of x in bf16) against the fp64 chain on
    the same bf16 weights and, at M <= 2, against the general kernel."""
    ws, x0 = make_stack(3, M, 61 + M, gpu, wt=O.BF16)
    resid, qkv, mlp = buffers(M, x0, gpu)
    ops = chain_ops(ws, M, resid, qkv, mlp)
    outs = {}
    for mode in ((0, 1) if M <= 2 else (0,)):
        old = mt.set_tuning(mt.TUNE_SEQ_LAYER, mode)
        try:
            seq = mt.Seq(ops)
        finally:
            mt.set_tuning(mt.TUNE_SEQ_LAYER, old)
        say(f"seq bf16 M={M} mode {mode} kernel {seq.kernel}")
        assert seq.kernel == (mt.SEQ_DECODE_LAYER if mode == 0 else mt.SEQ_GENERAL)
        resid.copy_(torch.from_numpy(x0))
        seq.run()
        torch.cuda.synchronize()
        seq.check()
        seq.close()
        outs[mode] = [t.cpu().numpy().copy() for t in (resid, qkv, mlp)]
    want = oracle_chain(ws, x0, M, wt=O.BF16)
    for j, what in enumerate(("resid", "qkv", "mlp")):
        assert O.normwise_rel_err(outs[0][j], want[j]) <= 1e-3, what
        if 1 in outs:
            # The two kernels split K differently and carry x as bf16 hi + lo halves (2^-17
            # relative), so their chains agree to about 1e-5 (1.04e-5 measured for mlp at M = 1).
            assert O.normwise_rel_err(outs[0][j], outs[1][j].astype(np.float64)) <= 2e-5, what


def test_seq_deterministic_and_equal_to_per_op_launches(gpu):
    """Re-runs of one plan are bit-identical; the 16 same ops as separate mt_linear launches
    (fp32 FMA dot products, another summation order) agree to fp32 rounding."""
    layers, M = 4, 2
    say("seq vs per-op")
    ws, x0 = make_stack(layers, M, 5, gpu)
    resid, qkv, mlp = buffers(M, x0, gpu)
    ops = chain_ops(ws, M, resid, qkv, mlp)
    _seq_vs_per_op(ops, resid, x0)


def _seq_vs_per_op(ops, resid, x0):
    for o in ops:
        if o.norm:
            rc = mt.linear_rmsnorm_raw(o.x, o.xt, o.norm, o.w, o.w2, o.wt, o.bias, o.y, o.p.M, o.p.N, o.p.K,
                                       o.p.ldx, o.p.ldy, o.p.flags, o.p.eps, None)
        else:
            rc = mt.linear_raw(o.x, o.xt, o.w, o.w2, o.wt, o.bias, o.y, o.p.M, o.p.N, o.p.K, o.p.ldx, o.p.ldy,
                               o.p.flags, None)
        assert rc == 0, mt.last_error()
    torch.cuda.synchronize()
    ref = resid.cpu().numpy().copy()
    results = []
    seq = mt.Seq(ops)
    say(f"seq groups={seq.groups}")
    for _ in range(3):   # the plan's run epoch advances by itself between runs
        resid.copy_(torch.from_numpy(x0))
        seq.run()
        torch.cuda.synchronize()
        results.append(resid.cpu().numpy().copy())
    seq.check()
    seq.close()
    # One plan is bit-exact from run to run; separate launches (other code and summation
    # order; the sequence splits each fp32 activation into a hi + lo 16-bit pair, good to
    # about 2^-22 relative) agree to fp32 rounding.
    for r in results:
        np.testing.assert_array_equal(r, results[0])
    assert O.normwise_rel_err(results[0], ref.astype(np.float64)) <= 1e-5


def test_seq_general_dataflow(gpu):
    """Inputs from an op two back, a column slice of an earlier output, an accumulate into a
    buffer written earlier, and a buffer written twice (only the last write reaches it):
    the sequence equals the same ops issued one at a time, at several workgroup counts
    (each count tiles the ops differently) and bit for bit across re-runs."""
    rng = np.random.default_rng(21)
    M = 3

    def w(n, k):
        b, _ = O.round16(rng.standard_normal((n, k)).astype(np.float32) * np.float32(0.1), O.BF16)
        return dev16(b, O.BF16, gpu)

    x0 = torch.from_numpy(rng.standard_normal((M, 64)).astype(np.float32)).to(gpu)
    A = torch.zeros(M, 96, device=gpu)
    B = torch.zeros(M, 128, device=gpu)
    C = torch.zeros(M, 40, device=gpu)
    D = torch.from_numpy(rng.standard_normal((M, 96)).astype(np.float32)).to(gpu)
    W0, W1, W2, W3, W4 = w(96, 64), w(128, 96), w(96, 128), w(40, 32), w(96, 40)
    ops = [
        mt.op(x0, W0, A, M),                                         # A = x0 W0
        mt.op(A, W1, B, M, flags=mt.GemvFlags.silu),                 # B = silu(A W1)
        mt.op(B, W2, A, M, flags=mt.GemvFlags.accumulate),           # A += B W2 (old A from op 0)
        mt.op(A[:, 16:], W3, C, M, ldx=96),                          # C = A[:, 16:48] W3 (op 2)
        mt.op(C, W4, D, M, flags=mt.GemvFlags.accumulate | mt.GemvFlags.gelu),  # D += gelu(C W4)
    ]
    d0 = D.clone()
    runs = []
    for groups in (0, 64, 7):   # each feature's sum runs in one order at any workgroup count
        old = mt.set_tuning(mt.TUNE_SEQ_GROUPS, groups)
        try:
            seq = mt.Seq(ops)
        finally:
            mt.set_tuning(mt.TUNE_SEQ_GROUPS, old)
        say(f"seq general dataflow groups={seq.groups}")
        again = []
        for _ in range(2):
            A.zero_(), B.zero_(), C.zero_(), D.copy_(d0)
            seq.run()
            torch.cuda.synchronize()
            again.append([t.cpu().numpy().copy() for t in (A, B, C, D)])
        seq.check()
        seq.close()
        for a, b in zip(again[0], again[1]):
            np.testing.assert_array_equal(a, b)
        runs.append(again[0])
    A.zero_(), B.zero_(), C.zero_(), D.copy_(d0)
    for o in ops:
        assert mt.linear_raw(o.x, o.xt, o.w, o.w2, o.wt, o.bias, o.y, o.p.M, o.p.N, o.p.K, o.p.ldx, o.p.ldy,
                             o.p.flags, None) == 0, mt.last_error()
    torch.cuda.synchronize()
    for got in runs:
        for g, t, name in zip(got, (A, B, C, D), "ABCD"):
            assert O.normwise_rel_err(g, t.cpu().numpy().astype(np.float64)) <= 1e-5, name


def test_seq_with_bf16_weights_and_fp16_activations(gpu):
    """A short chain in other dtypes: bf16 W, fp16 x (activations rounded between ops by the
    caller's buffer type is not possible for an fp32 y, so x here is a fixed fp16 input)."""
    M, N, K = 2, 512, 256
    rng = np.random.default_rng(3)
    wb, _ = O.round16(rng.standard_normal((N, K)).astype(np.float32) * np.float32(0.05), O.BF16)
    xb, xr = O.round16(rng.standard_normal((M, K)).astype(np.float32), O.F16)
    w = dev16(wb, O.BF16, gpu)
    x = dev16(xb, O.F16, gpu)
    y = torch.zeros(M, N, device=gpu)
    y2 = torch.zeros(M, N, device=gpu)
    say("seq bf16/f16")
    seq = mt.Seq([mt.op(x, w, y, M), mt.op(x, w, y2, M, flags=mt.GemvFlags.gelu)])
    seq.run()
    torch.cuda.synchronize()
    seq.check()
    want = O.linear_f64(xr, wb, None, O.BF16, None, None, M, N, K, 0)
    want2 = O.linear_f64(xr, wb, None, O.BF16, None, None, M, N, K, O.GELU)
    assert O.normwise_rel_err(y.cpu().numpy(), want) <= 1e-5
    assert O.normwise_rel_err(y2.cpu().numpy(), want2) <= 1e-5
    seq.close()


def test_seq_flags_activations_beyond_fp16_range(gpu):
    """fp16 weights: an activation beyond 65504 cannot take the hi + lo fp16 split; the run
    raises the plan's range flag and mt_seq_check reports MT_ERANGE."""
    M, N, K = 2, 64, 64
    rng = np.random.default_rng(9)
    wb, _ = O.round16(rng.standard_normal((N, K)).astype(np.float32) * np.float32(0.05), O.F16)
    w = dev16(wb, O.F16, gpu)
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(gpu)
    y = torch.zeros(M, N, device=gpu)
    say("seq fp16 range ok")
    seq = mt.Seq([mt.op(x, w, y, M)])
    seq.run()
    torch.cuda.synchronize()
    seq.check()
    x[1, 5] = 1.0e5
    say("seq fp16 range exceeded")
    seq.run()
    torch.cuda.synchronize()
    with pytest.raises(mt.MingTTSError) as e:
        seq.check()
    assert e.value.code == mt.ERANGE
    seq.close()


def test_seq_ordinary_launch_matches_cooperative(gpu):
    """The cooperative launch and the ordinary one (the default) run the same plan to the same
    bits on an idle device."""
    layers, M = 2, 2
    ws, x0 = make_stack(layers, M, 8, gpu)
    resid, qkv, mlp = buffers(M, x0, gpu)
    seq = mt.Seq(chain_ops(ws, M, resid, qkv, mlp))
    out = []
    for mode in (0, 1):
        old = mt.set_tuning(mt.TUNE_SEQ_LAUNCH, mode)
        try:
            say(f"seq launch mode {mode}")
            resid.copy_(torch.from_numpy(x0))
            seq.run()
            torch.cuda.synchronize()
        finally:
            mt.set_tuning(mt.TUNE_SEQ_LAUNCH, old)
        seq.check()
        out.append(resid.cpu().numpy().copy())
    seq.close()
    np.testing.assert_array_equal(out[0], out[1])
