"""mt_linear on the GPU against the oracle: the reference's known-answer tests (restated bit
for bit), every kernel family and dtype combination, the BASELINE shapes, and
size-independent properties at full size."""
import json
import os

import numpy as np
import pytest
import torch

import mingtts as mt
import oracle as O
from _gpu_util import assert_linear_parity, dev16, dev_x, expected, run_linear, say

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _id(c):
    m, n, k, flags, bias, xs = c
    return f"m{m}-n{n}-k{k}-f{flags}-b{int(bias)}-s{xs:g}"


@pytest.mark.parametrize("case", O.KAT_ALL, ids=_id)
def test_reference_kats_bf16_weights_fp32_activations(gpu, case):
    """The reference's own semantics: bf16 W, fp32 x, fp32 y, default kernel choice."""
    m, n, k, flags, bias, xs = case
    say(f"kat bf16/f32 {_id(case)} kernel {mt.linear_kernel(m, n, k)}")
    c = O.gemv_case(m, n, k, flags, bias, xs, wt=O.BF16)
    got, xu = run_linear(c, O.F32, gpu)
    assert_linear_parity(got, *expected(c, xu), k, _id(case))


@pytest.mark.parametrize("case", O.KAT_ALL, ids=_id)
def test_reference_kats_forced_gemm(gpu, case):
    """Every KAT shape through the register-staged MFMA GEMM, fp32 x split into hi + lo halves
    (the small-row MFMA kernel switched off)."""
    m, n, k, flags, bias, xs = case
    old = mt.set_tuning(mt.TUNE_GEMV_ROWS_MAX, 0)
    old_m = mt.set_tuning(mt.TUNE_GEMV_MFMA, 1)
    try:
        say(f"kat forced gemm {_id(case)}")
        c = O.gemv_case(m, n, k, flags, bias, xs, wt=O.BF16)
        got, xu = run_linear(c, O.F32, gpu)
    finally:
        mt.set_tuning(mt.TUNE_GEMV_ROWS_MAX, old)
        mt.set_tuning(mt.TUNE_GEMV_MFMA, old_m)
    assert_linear_parity(got, *expected(c, xu), k, "gemm " + _id(case))


@pytest.mark.parametrize("lanes", [8, 16, 32, 64])
@pytest.mark.parametrize("case", [c for c in O.KAT_ALL if c[0] <= 8], ids=_id)
def test_reference_kats_gemv_lane_splits(gpu, case, lanes):
    """The lane-group GEMV at every lane split (the analogue of the reference's kSplit /
    columnTiles sweep), also for the 3..8 rows that go to the MFMA kernel by default."""
    m, n, k, flags, bias, xs = case
    old = mt.set_tuning(mt.TUNE_GEMV_LANES, lanes)
    old_mfma = mt.set_tuning(mt.TUNE_GEMV_MFMA, 1)
    try:
        say(f"kat gemv lanes {lanes} {_id(case)}")
        c = O.gemv_case(m, n, k, flags, bias, xs, wt=O.F16)
        got, xu = run_linear(c, O.F32, gpu)
    finally:
        mt.set_tuning(mt.TUNE_GEMV_LANES, old)
        mt.set_tuning(mt.TUNE_GEMV_MFMA, old_mfma)
    assert_linear_parity(got, *expected(c, xu), k, f"lanes {lanes} " + _id(case))


DTYPE_CASES = [(6, 1024, 1024, O.GELU, True, 1.0), (4, 896, 896, O.SILU_GATE, False, 1.0),
               (33, 4864, 896, O.SILU_GATE, False, 1.0), (40, 896, 4864, O.ACCUM, False, 1.0),
               (2, 1152, 896, 0, True, 1.0), (65, 128, 64, O.SILU, True, 1.0)]


@pytest.mark.parametrize("wt", [O.F16, O.BF16], ids=["wf16", "wbf16"])
@pytest.mark.parametrize("xt", [O.F32, O.F16, O.BF16], ids=["xf32", "xf16", "xbf16"])
@pytest.mark.parametrize("case", DTYPE_CASES, ids=_id)
def test_dtype_combinations(gpu, case, xt, wt):
    m, n, k, flags, bias, xs = case
    say(f"dtypes x{xt} w{wt} {_id(case)}")
    c = O.gemv_case(m, n, k, flags, bias, xs, wt=wt)
    got, xu = run_linear(c, xt, gpu)
    assert_linear_parity(got, *expected(c, xu), k, f"x{xt} w{wt} " + _id(case))


def test_single_gemv_config_seed0(gpu):
    """W fp16 [4864 x 896] ~ N(0, 0.02^2), x fp16 [896] ~ N(0, 1), seed 0 (the single-GEMV
    configuration), against the committed fp32-reference-loop fixture and fp64."""
    import make_fixtures
    wb, xb, xr = make_fixtures.c1_inputs()
    with open(os.path.join(GOLDEN, "c1_gemv.json")) as f:
        fx = json.load(f)
    assert make_fixtures.digest(wb) == fx["w_digest"] and make_fixtures.digest(xb) == fx["x_digest"]
    say("c1 gemv 4864x896 fp16 seed 0")
    w_d = dev16(wb, O.F16, gpu)
    x_d = dev16(xb, O.F16, gpu)
    y_d = torch.zeros(1, 4864, device=gpu)
    mt.linear(x_d, w_d, y_d, M=1)
    torch.cuda.synchronize()
    got = y_d.cpu().numpy()
    want32 = O.linear_f32(xr, wb, None, O.F16, None, None, 1, 4864, 896, 0)
    np.testing.assert_array_equal(want32[0, :16], np.array(fx["y_head"], np.float32))
    want64 = O.linear_f64(xr, wb, None, O.F16, None, None, 1, 4864, 896, 0)
    assert_linear_parity(got, want32, want64, 896, "c1")


BACKBONE = [  # (label, N, K, flags, bias, gated) of one Qwen layer (Qwen.swift:85-91, Weights.swift:121-125)
    ("qkv", 1152, 896, 0, True, False), ("o", 896, 896, O.ACCUM, False, False),
    ("gate|up", 4864, 896, O.SILU_GATE, False, True), ("down", 896, 4864, O.ACCUM, False, False),
]
DIT = [  # BASELINE DiT head: MLP 896 -> 3584 (GELU) -> 896, adaLN 896 -> 6 x 896 (M = 2)
    ("dit ff1", 3584, 896, O.GELU, True, False), ("dit ff2", 896, 3584, O.ACCUM, True, False),
    ("dit adaLN", 5376, 896, 0, True, False),
]


def _baseline_case(seed, M, N, K, flags, bias, gated, xt=O.F16):
    """Seeded BASELINE-style inputs: W fp16 ~ N(0, 0.02^2), x ~ N(0, 1), y0 ~ N(0, 1)."""
    z = O.gaussian(seed, N * K * (2 if gated else 1) + N + M * K + M * N)
    o = 0
    wb, _ = O.round16(z[o:o + N * K] * np.float32(0.02), O.F16); o += N * K
    w2b = None
    if gated:
        w2b, _ = O.round16(z[o:o + N * K] * np.float32(0.02), O.F16); o += N * K
    bb, _ = O.round16(z[o:o + N] * np.float32(0.02), O.F16); o += N
    x = z[o:o + M * K].reshape(M, K).copy(); o += M * K
    y0 = z[o:o + M * N].reshape(M, N).copy()
    return dict(m=M, n=N, k=K, flags=flags | (O.BIAS if bias else 0), x=x, w=wb.reshape(N, K),
                w2=w2b.reshape(N, K) if gated else wb.reshape(N, K), bias=bb if bias else None, y0=y0, wt=O.F16)


@pytest.mark.parametrize("M", [64, 256, 512])
@pytest.mark.parametrize("layer", BACKBONE, ids=[b[0] for b in BACKBONE])
def test_prefill_backbone_shapes(gpu, M, layer):
    label, N, K, flags, bias, gated = layer
    say(f"prefill {label} M={M}")
    c = _baseline_case(1000 + M + N + K, M, N, K, flags, bias, gated)
    got, xu = run_linear(c, O.F16, gpu)
    assert_linear_parity(got, *expected(c, xu), K, f"prefill {label} M={M}")


@pytest.mark.parametrize("layer", DIT, ids=[d[0] for d in DIT])
def test_dit_head_shapes(gpu, layer):
    label, N, K, flags, bias, gated = layer
    M = 2 if label == "dit adaLN" else 64
    say(f"{label} M={M}")
    c = _baseline_case(2000 + N + K, M, N, K, flags, bias, gated)
    got, xu = run_linear(c, O.F16, gpu)
    assert_linear_parity(got, *expected(c, xu), K, label)


@pytest.mark.parametrize("M", [1, 2, 4, 8])
@pytest.mark.parametrize("layer", BACKBONE, ids=[b[0] for b in BACKBONE])
def test_decode_backbone_shapes_fp32_activations(gpu, M, layer):
    label, N, K, flags, bias, gated = layer
    say(f"decode {label} M={M}")
    c = _baseline_case(3000 + M + N, M, N, K, flags, bias, gated)
    got, xu = run_linear(c, O.F32, gpu)
    assert_linear_parity(got, *expected(c, xu), K, f"decode {label} M={M}")


@pytest.mark.parametrize("M", [2, 64])
def test_deterministic_and_exactly_homogeneous(gpu, M):
    """Two runs are bit-identical, and y(2x) == 2 y(x) bit for bit (scaling by a power of two
    is exact in every fp32 / fp16 step, including the hi/lo split) -- at the full gate|up size."""
    N, K = 4864, 896
    say(f"determinism M={M}")
    c = _baseline_case(77, M, N, K, 0, False, False)
    # Not (fp32 x, fp16 w) in the GEMM: there the low half of x is rounded on fp16's
    # subnormal grid, where doubling does not commute with rounding.
    combos = [(O.F16, O.F16), (O.F32, O.BF16)] + ([(O.F32, O.F16)] if M <= 8 else [])
    for xt, wt in combos:
        x_d, _ = dev_x(c["x"], xt, gpu)
        wb, _ = O.round16(O.decode16(c["w"], O.F16), wt)
        w_d = dev16(wb, wt, gpu)
        ys = []
        for scale in (1.0, 1.0, 2.0):
            y_d = torch.zeros(M, N, device=gpu)
            mt.linear(x_d * scale, w_d, y_d, M=M)
            torch.cuda.synchronize()
            ys.append(y_d.cpu().numpy())
        np.testing.assert_array_equal(ys[0], ys[1])
        np.testing.assert_array_equal(ys[2], 2 * ys[0])


def test_strided_views_and_edges(gpu):
    """ldx > K and ldy > N (row views like ActView.row/column), N = 1, K = 8, rows past M."""
    rng = np.random.default_rng(8)
    for (M, N, K, ldx, ldy) in ((1, 1, 8, 8, 1), (3, 5, 16, 24, 9), (2, 1152, 896, 1152, 1200),
                                (20, 70, 40, 48, 80)):
        say(f"strided M={M} N={N} K={K} ldx={ldx} ldy={ldy}")
        x = rng.standard_normal((M + 8, ldx)).astype(np.float32)
        x[M:] = np.nan
        wb, _ = O.round16(rng.standard_normal((N, K)).astype(np.float32) * np.float32(0.1), O.BF16)
        y0 = rng.standard_normal((M, ldy)).astype(np.float32)
        x_d = torch.from_numpy(x).to(gpu)
        y_d = torch.from_numpy(y0.copy()).to(gpu)
        rc = mt.linear_raw(x_d, O.F32, dev16(wb, O.BF16, gpu), None, O.BF16, None, y_d, M, N, K, ldx, ldy,
                           O.ACCUM, None)
        assert rc == 0, mt.last_error()
        torch.cuda.synchronize()
        got = y_d.cpu().numpy()
        want64 = O.linear_f64(np.ascontiguousarray(x[:M, :K]), wb, None, O.BF16, None,
                              np.ascontiguousarray(y0[:, :N]), M, N, K, O.ACCUM)
        assert O.normwise_rel_err(got[:, :N], want64) <= 1e-5
        np.testing.assert_array_equal(got[:, N:], y0[:, N:])   # columns past N untouched


@pytest.mark.parametrize("rows_max,mfma", [(8, 0), (8, 1), (0, 1)], ids=["mfma", "gemv", "gemm"])
def test_reference_rmsnorm_kat_through_identity_weights(gpu, rows_max, mfma):
    """KernelTests.testRMSNorm (KernelTests.swift:187-203) through the fused prologue: with
    W = I (exact in bf16) the linear returns the normalised rows themselves."""
    rows, k = 5, 896
    rng = O.LCG(3)
    x = rng.floats(rows * k, 3.0).reshape(rows, k)
    gb, _ = O.round16(rng.floats(k), O.BF16)
    eye, _ = O.round16(np.eye(k, dtype=np.float32), O.BF16)
    want = O.rmsnorm_f32(x, gb, O.BF16)
    x_d = torch.from_numpy(np.concatenate([x, np.full((8, k), np.nan, np.float32)])).to(gpu)
    y_d = torch.zeros(rows, k, device=gpu)
    old = mt.set_tuning(mt.TUNE_GEMV_ROWS_MAX, rows_max)
    old_m = mt.set_tuning(mt.TUNE_GEMV_MFMA, mfma)
    try:
        say(f"rmsnorm kat rows_max={rows_max} mfma={mfma}")
        mt.linear(x_d, dev16(eye, O.BF16, gpu), y_d, M=rows, norm=dev16(gb, O.BF16, gpu), eps=1e-6)
        torch.cuda.synchronize()
    finally:
        mt.set_tuning(mt.TUNE_GEMV_ROWS_MAX, old)
        mt.set_tuning(mt.TUNE_GEMV_MFMA, old_m)
    ex, i, g, w = O.worst_violation(y_d.cpu().numpy(), want, 1e-5)   # atol 1e-5 as the reference
    assert ex <= 0, f"index {i} got {g} want {w}"


@pytest.mark.parametrize("M", [1, 2, 5, 64, 174])
@pytest.mark.parametrize("layer", [BACKBONE[0], BACKBONE[2]], ids=["qkv", "gate|up"])
@pytest.mark.parametrize("xt", [O.F32, O.F16], ids=["xf32", "xf16"])
def test_fused_rmsnorm_prologue(gpu, M, layer, xt):
    """rmsnorm then linear (Qwen.swift:84-85, 89-90) as one pass, against the fp64 composition
    and against the reference's two fp32 loops (norm, then linear on the stored fp32 row)."""
    label, N, K, flags, bias, gated = layer
    c = _baseline_case(4000 + M + N, M, N, K, flags, bias, gated)
    x = c["x"] * np.float32(5.0)       # off-unit scale: the norm must actually rescale
    gbits, _ = O.round16(1.0 + 0.1 * O.gaussian(4100 + N, K), O.F16)
    x_d, xu = dev_x(x, xt, gpu)
    y_d = torch.from_numpy(c["y0"].copy()).to(gpu)
    say(f"fused rmsnorm {label} M={M} x{xt}")
    rc = mt.linear_rmsnorm_raw(x_d, xt, dev16(gbits, O.F16, gpu), dev16(c["w"], O.F16, gpu),
                               dev16(c["w2"], O.F16, gpu) if gated else None, O.F16,
                               dev16(c["bias"], O.F16, gpu) if c["bias"] is not None else None, y_d,
                               M, N, K, K, N, flags, 1e-6, None)
    assert rc == 0, mt.last_error()
    torch.cuda.synchronize()
    got = y_d.cpu().numpy()
    want64 = O.linear_np64(O.rmsnorm_f64(xu, gbits, O.F16), c["w"], c["w2"] if gated else None, O.F16,
                           c["bias"], c["y0"], c["flags"])
    normed32 = O.rmsnorm_f32(xu, gbits, O.F16)
    want32 = O.linear_f32(normed32, c["w"], c["w2"] if gated else None, O.F16, c["bias"], c["y0"], M, N, K, c["flags"])
    assert_linear_parity(got, want32, want64, K, f"fused rmsnorm {label} M={M}")


def test_encoder_mirror_reads_like_the_reference(gpu):
    """Encoder.linear with Linear / ActView / GPUTensor (Kernels.swift:7-44, 132-161)."""
    c = O.gemv_case(2, 2, 896, 0, True)
    wt = O.BF16
    e = mt.Encoder()
    w = mt.GPUTensor(dev16(c["w"], wt, gpu))
    b = mt.GPUTensor(dev16(c["bias"], wt, gpu))
    xb = torch.from_numpy(c["x"]).to(gpu)
    yb = torch.from_numpy(c["y0"].copy()).to(gpu)
    say("encoder mirror")
    e.linear(mt.ActView(xb, ld=896), 2, mt.Linear(w, b, 2, 896), mt.ActView(yb, ld=2))
    torch.cuda.synchronize()
    assert_linear_parity(yb.cpu().numpy(), *expected(c, c["x"]), 896, "encoder")
