"""The pipelined MFMA GEMM under every tile shape and forced split-K count, on ragged shapes,
against the oracle's fp32 reference loop and fp64 recomputation: activations of the weights'
type, and fp32 activations split into hi + lo planes (with and without the fused RMSNorm);
split-K runs are re-run to show the arrival counters re-arm and the partial sums are added
in a fixed order (bit-identical results)."""
import numpy as np
import pytest
import torch

import mingtts as mt
import oracle as O
from _gpu_util import assert_linear_parity, dev16, expected, run_linear, say

pytestmark = pytest.mark.gpu

SHAPES = [  # (M, N, K, flags, bias)
    (77, 100, 200, O.GELU, True),         # ragged everywhere; K tail inside a 64-k stage
    (130, 260, 136, O.ACCUM, False),      # two x-row tiles of 128 plus 2 rows
    (64, 70, 896, O.SILU_GATE, True),     # gated, features past N inside the tile
    (9, 896, 4864, O.ACCUM, False),       # long K, 9 rows
    (512, 1152, 896, O.BIAS, True),
    (33, 4864, 896, O.SILU_GATE | O.ACCUM, False),
    (200, 64, 8, O.SILU, True),           # K = 8: one chunk of one stage
]


def _case(seed, M, N, K, flags, bias, wt):
    rng = np.random.default_rng(seed)
    gated = bool(flags & O.SILU_GATE)
    wb, _ = O.round16(rng.standard_normal((N, K)).astype(np.float32) * np.float32(0.05), wt)
    w2b = O.round16(rng.standard_normal((N, K)).astype(np.float32) * np.float32(0.05), wt)[0] if gated else wb
    bb = O.round16(rng.standard_normal(N).astype(np.float32) * np.float32(0.05), wt)[0] if bias else None
    x = rng.standard_normal((M, K)).astype(np.float32)
    y0 = rng.standard_normal((M, N)).astype(np.float32)
    return dict(m=M, n=N, k=K, flags=flags | (O.BIAS if bias else 0), x=x, w=wb, w2=w2b, bias=bb, y0=y0, wt=wt)


def _with_tuning(tile, splits, fn, stages=0):
    """Runs fn on the pipelined GEMM (the small-row MFMA kernel switched off, every M a GEMM)."""
    old_t = mt.set_tuning(mt.TUNE_GEMM_TILE, tile)
    old_s = mt.set_tuning(mt.TUNE_GEMM_SPLITK, splits)
    old_p = mt.set_tuning(mt.TUNE_GEMM_STAGES, stages)
    old_r = mt.set_tuning(mt.TUNE_GEMV_ROWS_MAX, 0)
    old_m = mt.set_tuning(mt.TUNE_GEMV_MFMA, 1)
    try:
        return fn()
    finally:
        mt.set_tuning(mt.TUNE_GEMM_TILE, old_t)
        mt.set_tuning(mt.TUNE_GEMM_SPLITK, old_s)
        mt.set_tuning(mt.TUNE_GEMM_STAGES, old_p)
        mt.set_tuning(mt.TUNE_GEMV_ROWS_MAX, old_r)
        mt.set_tuning(mt.TUNE_GEMV_MFMA, old_m)


def _ids(s):
    return f"M{s[0]}_N{s[1]}_K{s[2]}_f{s[3]}"


@pytest.mark.parametrize("splits", [0, 1, 3, 8])
@pytest.mark.parametrize("tile", [1, 2, 3])
@pytest.mark.parametrize("shape", SHAPES, ids=_ids)
def test_tiles_and_splits(gpu, shape, tile, splits):
    M, N, K, flags, bias = shape
    if flags & O.SILU_GATE and tile == 3:
        pytest.skip("a gated tile always has 128 weight rows")
    say(f"tiled tile={tile} splits={splits} {_ids(shape)}")
    c = _case(M * 7 + N + K, M, N, K, flags, bias, O.F16)
    got, xu = _with_tuning(tile, splits, lambda: run_linear(c, O.F16, gpu))
    assert_linear_parity(got, *expected(c, xu), K, f"tile {tile} splits {splits} {_ids(shape)}")
    if splits != 1:
        again, _ = _with_tuning(tile, splits, lambda: run_linear(c, O.F16, gpu))
        np.testing.assert_array_equal(again, got)


@pytest.mark.parametrize("stages", [1, 2, 3, 4])
@pytest.mark.parametrize("tile", [1, 2, 3])
@pytest.mark.parametrize("shape", SHAPES, ids=_ids)
def test_pipeline_depths(gpu, shape, tile, stages):
    """Every load pipeline (register-staged, 2-4 direct-to-LDS stages) on every tile, with a
    split of 2 where K allows it."""
    M, N, K, flags, bias = shape
    if flags & O.SILU_GATE and tile == 3:
        pytest.skip("a gated tile always has 128 weight rows")
    say(f"tiled stages={stages} tile={tile} {_ids(shape)}")
    c = _case(M * 11 + N + K, M, N, K, flags, bias, O.F16)
    got, xu = _with_tuning(tile, 2, lambda: run_linear(c, O.F16, gpu), stages=stages)
    assert_linear_parity(got, *expected(c, xu), K, f"stages {stages} tile {tile} {_ids(shape)}")


@pytest.mark.parametrize("shape", SHAPES[:4], ids=_ids)
def test_bf16(gpu, shape):
    M, N, K, flags, bias = shape
    say(f"tiled bf16 {_ids(shape)}")
    c = _case(M + 3 * N + K, M, N, K, flags, bias, O.BF16)
    got, xu = _with_tuning(0, 0, lambda: run_linear(c, O.BF16, gpu))
    assert_linear_parity(got, *expected(c, xu), K, f"bf16 {_ids(shape)}")


# fp32 x split into hi + lo halves represents x to 2^-22 (fp16) / 2^-17 (bf16) relative, so the
# products stay within fp32 accumulation error of fp64; x rounded to 16 bits alone would sit
# near 3e-4 and fail this bound.
SPLIT_TOL = 2e-5


@pytest.mark.parametrize("wt", [O.F16, O.BF16], ids=["wf16", "wbf16"])
@pytest.mark.parametrize("splits", [0, 3])
@pytest.mark.parametrize("tile", [1, 2, 3])
@pytest.mark.parametrize("shape", SHAPES, ids=_ids)
def test_fp32_activations_split_into_hi_and_lo(gpu, shape, tile, splits, wt):
    M, N, K, flags, bias = shape
    if flags & O.SILU_GATE and tile == 3:
        pytest.skip("a gated tile always has 128 weight rows")
    say(f"tiled fp32 x w{wt} tile={tile} splits={splits} {_ids(shape)}")
    c = _case(M * 13 + N + K + wt, M, N, K, flags, bias, wt)
    # Larger x gives the lo half more to carry; with bf16 halves (2^-17) unit-scale x keeps a
    # gated product inside the reference's per-element tolerance.
    c["x"] = c["x"] * np.float32(3.0 if wt == O.F16 else 1.0)
    got, xu = _with_tuning(tile, splits, lambda: run_linear(c, O.F32, gpu))
    want32, want64 = expected(c, xu)
    assert_linear_parity(got, want32, want64, K, f"fp32 x tile {tile} splits {splits} {_ids(shape)}")
    rel = O.normwise_rel_err(got, want64)
    assert rel <= SPLIT_TOL, f"fp32 x: normwise {rel:.3g} > {SPLIT_TOL} (lo half lost?)"
    if splits != 1:
        again, _ = _with_tuning(tile, splits, lambda: run_linear(c, O.F32, gpu))
        np.testing.assert_array_equal(again, got)


@pytest.mark.parametrize("wt", [O.F16, O.BF16], ids=["wf16", "wbf16"])
@pytest.mark.parametrize("tile", [1, 2, 3])
@pytest.mark.parametrize("shape", SHAPES, ids=_ids)
def test_fp32_activations_with_fused_rmsnorm(gpu, shape, tile, wt):
    """rmsnorm(x) * gain then the linear, one pass: the row sums of x^2 come from the staged
    loads and scale the epilogue; under a forced split of 3 each split's partial row sums
    travel with its partial tile (re-run: bit-identical)."""
    M, N, K, flags, bias = shape
    if flags & O.SILU_GATE and tile == 3:
        pytest.skip("a gated tile always has 128 weight rows")
    say(f"tiled fp32 x rmsnorm w{wt} tile={tile} {_ids(shape)}")
    c = _case(M * 17 + N + K + wt, M, N, K, flags, bias, wt)
    x = c["x"] * np.float32(4.0)
    gbits, _ = O.round16(1.0 + 0.1 * O.gaussian(4200 + N, K), wt)
    gated = bool(flags & O.SILU_GATE)
    x_d = torch.from_numpy(x).to(gpu)
    y_d = torch.from_numpy(c["y0"].copy()).to(gpu)

    def go():
        rc = mt.linear_rmsnorm_raw(x_d, O.F32, dev16(gbits, wt, gpu), dev16(c["w"], wt, gpu),
                                   dev16(c["w2"], wt, gpu) if gated else None, wt,
                                   dev16(c["bias"], wt, gpu) if c["bias"] is not None else None, y_d,
                                   M, N, K, K, N, flags | (O.BIAS if bias else 0), 1e-6, None)
        assert rc == 0, mt.last_error()
        torch.cuda.synchronize()

    _with_tuning(tile, 3, go)
    got = y_d.cpu().numpy()
    y_d.copy_(torch.from_numpy(c["y0"]))
    _with_tuning(tile, 3, go)
    np.testing.assert_array_equal(y_d.cpu().numpy(), got)
    want64 = O.linear_np64(O.rmsnorm_f64(x, gbits, wt), c["w"], c["w2"] if gated else None, wt, c["bias"],
                           c["y0"], c["flags"])
    want32 = O.linear_f32(O.rmsnorm_f32(x, gbits, wt), c["w"], c["w2"] if gated else None, wt, c["bias"],
                          c["y0"], M, N, K, c["flags"])
    assert_linear_parity(got, want32, want64, K, f"fp32 x rmsnorm tile {tile} {_ids(shape)}")
    rel = O.normwise_rel_err(got, want64)
    assert rel <= SPLIT_TOL, f"fp32 x rmsnorm: normwise {rel:.3g} > {SPLIT_TOL}"


@pytest.mark.parametrize("norm", [False, True], ids=["plain", "rmsnorm"])
@pytest.mark.parametrize("splits", [0, 3])
@pytest.mark.parametrize("tile", [1, 2, 3])
@pytest.mark.parametrize("shape", SHAPES, ids=_ids)
def test_fp32_activation_loops_agree_bit_for_bit(gpu, shape, tile, splits, norm):
    """The fp32-x path's two K loops (stages 1: commits only the split's stages; 2: branch-free,
    the stages past the split staged and never multiplied, their x^2 not summed) multiply the
    same stages in the same order: the same bits, with and without the fused RMSNorm, and the
    branch-free loop against fp64."""
    M, N, K, flags, bias = shape
    if flags & O.SILU_GATE and tile == 3:
        pytest.skip("a gated tile always has 128 weight rows")
    say(f"tiled fp32 x loops tile={tile} splits={splits} norm={norm} {_ids(shape)}")
    wt = O.F16
    c = _case(M * 19 + N + K, M, N, K, flags, bias, wt)
    x = c["x"] * np.float32(3.0)
    gbits, _ = O.round16(1.0 + 0.1 * O.gaussian(4300 + N, K), wt)
    gated = bool(flags & O.SILU_GATE)
    x_d = torch.from_numpy(x).to(gpu)
    y_d = torch.from_numpy(c["y0"].copy()).to(gpu)
    g_d = dev16(gbits, wt, gpu)
    w_d, w2_d = dev16(c["w"], wt, gpu), dev16(c["w2"], wt, gpu) if gated else None
    b_d = dev16(c["bias"], wt, gpu) if c["bias"] is not None else None

    def go():
        y_d.copy_(torch.from_numpy(c["y0"]))
        if norm:
            rc = mt.linear_rmsnorm_raw(x_d, O.F32, g_d, w_d, w2_d, wt, b_d, y_d, M, N, K, K, N, c["flags"], 1e-6)
        else:
            rc = mt.linear_raw(x_d, O.F32, w_d, w2_d, wt, b_d, y_d, M, N, K, K, N, c["flags"])
        assert rc == 0, mt.last_error()
        torch.cuda.synchronize()
        return y_d.cpu().numpy()

    got = {st: _with_tuning(tile, splits, go, stages=st) for st in (1, 2)}
    np.testing.assert_array_equal(got[2], got[1])
    xin64 = O.rmsnorm_f64(x, gbits, wt) if norm else x.astype(np.float64)
    xin32 = O.rmsnorm_f32(x, gbits, wt) if norm else x
    want64 = O.linear_np64(xin64, c["w"], c["w2"] if gated else None, wt, c["bias"], c["y0"], c["flags"])
    want32 = O.linear_f32(xin32, c["w"], c["w2"] if gated else None, wt, c["bias"], c["y0"], M, N, K, c["flags"])
    assert_linear_parity(got[2], want32, want64, K, f"fp32 x loops tile {tile} {_ids(shape)}")
    rel = O.normwise_rel_err(got[2], want64)
    assert rel <= SPLIT_TOL, f"fp32 x loops: normwise {rel:.3g} > {SPLIT_TOL}"


def test_workspace_grows_and_streams_are_independent(gpu):
    """A small split launch, a much larger one (the workspace grows), then both again on a
    second stream: every result matches the first run of the same case bit for bit."""
    small = _case(5, 64, 256, 4864, O.ACCUM, False, O.F16)
    large = _case(6, 256, 4864, 896, O.SILU_GATE, False, O.F16)
    say("tiled workspace growth")
    r_small, xs = _with_tuning(3, 16, lambda: run_linear(small, O.F16, gpu))
    r_large, xl = _with_tuning(1, 4, lambda: run_linear(large, O.F16, gpu))
    assert_linear_parity(r_small, *expected(small, xs), 4864, "small split")
    assert_linear_parity(r_large, *expected(large, xl), 896, "large split")
    s = torch.cuda.Stream(device=gpu)
    with torch.cuda.stream(s):
        again_small, _ = _with_tuning(3, 16, lambda: run_linear(small, O.F16, gpu, stream=s.cuda_stream))
        again_large, _ = _with_tuning(1, 4, lambda: run_linear(large, O.F16, gpu, stream=s.cuda_stream))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(again_small, r_small)
    np.testing.assert_array_equal(again_large, r_large)


def test_nan_rows_past_m_are_not_read(gpu):
    """x rows past M hold NaN in memory: the tile's zero-filled rows keep them out."""
    M, N, K = 70, 96, 192
    rng = np.random.default_rng(11)
    x = rng.standard_normal((M + 64, K)).astype(np.float32)
    x[M:] = np.nan
    wb, _ = O.round16(rng.standard_normal((N, K)).astype(np.float32) * np.float32(0.05), O.F16)
    xb, xr = O.round16(x, O.F16)
    from _gpu_util import dev16
    x_d = dev16(xb, O.F16, gpu)
    y_d = torch.zeros(M, N, device=gpu)
    say("tiled NaN rows past M")

    def go():
        rc = mt.linear_raw(x_d, O.F16, dev16(wb, O.F16, gpu), None, O.F16, None, y_d, M, N, K, K, N, 0, None)
        assert rc == 0, mt.last_error()
        torch.cuda.synchronize()
        return y_d.cpu().numpy()

    got = _with_tuning(1, 2, go)
    want64 = O.linear_f64(xr[:M], wb, None, O.F16, None, None, M, N, K, 0)
    assert np.all(np.isfinite(got))
    assert O.normwise_rel_err(got, want64) <= 1e-5


def _ring_auto(M, N, gpu):
    """Whether the automatic tile choice takes the gated ring kernel: its tiles (128 rows x 96
    features, one workgroup a CU) fill at least three quarters of their last wave."""
    cus = torch.cuda.get_device_properties(gpu).multi_processor_count
    t = -(-M // 128) * -(-N // 96)
    waves = -(-t // cus)
    return 4 * t >= 3 * waves * cus


RING_SHAPES = [  # gated (M, N, K, flags, bias) for the ring kernel of 96-feature tiles
    (512, 4864, 896, O.SILU_GATE, False),             # gate|up at the prefill's 512 rows
    (130, 100, 200, O.SILU_GATE, True),               # ragged: rows, features and K past the tiles
    (384, 300, 136, O.SILU_GATE | O.ACCUM, False),    # K tail inside a stage, accumulate
    (33, 4864, 896, O.SILU_GATE | O.ACCUM, True),
    (200, 96, 8, O.SILU_GATE | O.SILU, True),         # K = 8: one chunk of one stage
    (257, 192, 320, O.SILU_GATE | O.GELU, False),     # GELU after the gate (flag order)
]


@pytest.mark.parametrize("wt", [O.F16, O.BF16], ids=["wf16", "wbf16"])
@pytest.mark.parametrize("shape", RING_SHAPES, ids=_ids)
def test_gated_ring_kernel(gpu, shape, wt):
    """The gated ring kernel (MT_TUNE_GEMM_TILE = 5; the auto choice for gated linears whose ring
    tiles fill at least 3/4 of their last wave) against the oracle's fp32 loop and fp64, re-run
    bit-identical; where the default routing takes it (gate|up at 512 rows) it gives the same
    bits."""
    M, N, K, flags, bias = shape
    say(f"ring w{wt} {_ids(shape)}")
    c = _case(M * 19 + N + K + wt, M, N, K, flags, bias, wt)
    got, xu = _with_tuning(5, 0, lambda: run_linear(c, wt, gpu))
    assert_linear_parity(got, *expected(c, xu), K, f"ring w{wt} {_ids(shape)}")
    again, _ = _with_tuning(5, 0, lambda: run_linear(c, wt, gpu))
    np.testing.assert_array_equal(again, got)
    if _ring_auto(M, N, gpu):
        auto, _ = _with_tuning(0, 0, lambda: run_linear(c, wt, gpu))
        np.testing.assert_array_equal(auto, got)


def test_ring_tile_refuses_ungated_linears(gpu):
    c = _case(5, 128, 64, 64, 0, False, O.F16)
    old = mt.set_tuning(mt.TUNE_GEMM_TILE, 5)
    try:
        x_d = dev16(O.round16(c["x"], O.F16)[0], O.F16, gpu)
        w_d = dev16(c["w"], O.F16, gpu)
        y_d = torch.zeros(128, 64, device=gpu)
        rc = mt.linear_raw(x_d, O.F16, w_d, None, O.F16, None, y_d, 128, 64, 64, 64, 64, 0)
    finally:
        mt.set_tuning(mt.TUNE_GEMM_TILE, old)
    assert rc == mt.EINVAL, rc
    assert "ring" in mt.last_error()


@pytest.mark.parametrize("norm", [False, True], ids=["plain", "rmsnorm"])
@pytest.mark.parametrize("wt", [O.F16, O.BF16], ids=["wf16", "wbf16"])
@pytest.mark.parametrize("shape", RING_SHAPES, ids=_ids)
def test_gated_ring_kernel_fp32_activations(gpu, shape, wt, norm):
    """The gated ring kernel for fp32 x (hi + lo halves, MT_TUNE_GEMM_TILE = 5; the auto choice
    for gated linears whose ring tiles fill at least 3/4 of their last wave), with and without
    the fused RMSNorm, against the oracle's fp32 loop and fp64 within the split bound; re-run
    bit-identical, and where the default routing takes it (gate|up at 512 rows) the same bits."""
    M, N, K, flags, bias = shape
    say(f"ring fp32 x w{wt} norm={norm} {_ids(shape)}")
    c = _case(M * 23 + N + K + wt, M, N, K, flags, bias, wt)
    c["x"] = c["x"] * np.float32(3.0 if wt == O.F16 else 1.0)
    if not norm:
        got, xu = _with_tuning(5, 0, lambda: run_linear(c, O.F32, gpu))
        want32, want64 = expected(c, xu)
        assert_linear_parity(got, want32, want64, K, f"ring fp32 x {_ids(shape)}")
        rel = O.normwise_rel_err(got, want64)
        assert rel <= SPLIT_TOL, f"ring fp32 x: normwise {rel:.3g} > {SPLIT_TOL}"
        again, _ = _with_tuning(5, 0, lambda: run_linear(c, O.F32, gpu))
        np.testing.assert_array_equal(again, got)
        if _ring_auto(M, N, gpu):
            auto, _ = _with_tuning(0, 0, lambda: run_linear(c, O.F32, gpu))
            np.testing.assert_array_equal(auto, got)
        return
    x = c["x"]
    gbits, _ = O.round16(1.0 + 0.1 * O.gaussian(4300 + N, K), wt)
    x_d = torch.from_numpy(x).to(gpu)
    y_d = torch.from_numpy(c["y0"].copy()).to(gpu)

    def go():
        rc = mt.linear_rmsnorm_raw(x_d, O.F32, dev16(gbits, wt, gpu), dev16(c["w"], wt, gpu), dev16(c["w2"], wt, gpu), wt,
                                   dev16(c["bias"], wt, gpu) if c["bias"] is not None else None, y_d,
                                   M, N, K, K, N, c["flags"], 1e-6, None)
        assert rc == 0, mt.last_error()
        torch.cuda.synchronize()
        return y_d.cpu().numpy().copy()

    got = _with_tuning(5, 0, go)
    y_d.copy_(torch.from_numpy(c["y0"]))
    again = _with_tuning(5, 0, go)
    np.testing.assert_array_equal(again, got)
    want64 = O.linear_np64(O.rmsnorm_f64(x, gbits, wt), c["w"], c["w2"], wt, c["bias"], c["y0"], c["flags"])
    want32 = O.linear_f32(O.rmsnorm_f32(x, gbits, wt), c["w"], c["w2"], wt, c["bias"], c["y0"], M, N, K, c["flags"])
    assert_linear_parity(got, want32, want64, K, f"ring fp32 x rmsnorm {_ids(shape)}")
    rel = O.normwise_rel_err(got, want64)
    assert rel <= SPLIT_TOL, f"ring fp32 x rmsnorm: normwise {rel:.3g} > {SPLIT_TOL}"
    if _ring_auto(M, N, gpu):
        y_d.copy_(torch.from_numpy(c["y0"]))
        auto = _with_tuning(0, 0, go)
        np.testing.assert_array_equal(auto, got)
