"""mt_rmsnorm, the reference's Encoder.rmsnorm (Kernels.swift:163-171, Shaders.swift:414-440)
on its own: the reference's known-answer test and other shapes, strides, gain types and in
place, against the oracle's restatement of the reference CPU loop and an fp64 recomputation."""
import numpy as np
import pytest
import torch

import mingtts as mt
import oracle as O
from _gpu_util import dev16, say

pytestmark = pytest.mark.gpu


def test_reference_rmsnorm_kat(gpu):
    """KernelTests.testRMSNorm (KernelTests.swift:187-203): 5 rows of 896, x from the KAT RNG
    (state 3) at scale 3, bf16 gain from the same stream; atol 1e-5 as the reference."""
    rows, k = 5, 896
    rng = O.LCG(3)
    x = rng.floats(rows * k, 3.0).reshape(rows, k)
    gb, _ = O.round16(rng.floats(k), O.BF16)
    y = torch.zeros(rows, k, device=gpu)
    say("rmsnorm kat")
    mt.rmsnorm(torch.from_numpy(x).to(gpu), dev16(gb, O.BF16, gpu), y)
    torch.cuda.synchronize()
    ex, i, g, w = O.worst_violation(y.cpu().numpy(), O.rmsnorm_f32(x, gb, O.BF16), 1e-5)
    assert ex <= 0, f"index {i} got {g} want {w}"


@pytest.mark.parametrize("rows,width,ldx,ldy,wt,inplace", [
    (1, 4, 4, 4, O.BF16, False), (7, 1028, 1032, 1036, O.F16, False), (64, 896, 896, 896, O.BF16, True),
    (3, 4864, 4864, 4864, O.F16, False), (9, 256, 260, 256, O.BF16, False)])
def test_rmsnorm_shapes(gpu, rows, width, ldx, ldy, wt, inplace):
    rng = np.random.default_rng(rows * 1000 + width)
    x = (rng.standard_normal((rows, ldx)) * 2.0).astype(np.float32)
    gb, _ = O.round16((1.0 + 0.1 * rng.standard_normal(width)).astype(np.float32), wt)
    x_d = torch.from_numpy(x).to(gpu)
    if inplace:
        y_d, ldy = x_d, ldx
    else:
        y_d = torch.full((rows, ldy), -7.0, device=gpu)
    say(f"rmsnorm rows={rows} width={width} ldx={ldx} ldy={ldy} wt={wt} inplace={inplace}")
    assert mt.rmsnorm_raw(x_d, ldx, rows, width, dev16(gb, wt, gpu), wt, y_d, ldy, 1e-6) == 0, mt.last_error()
    torch.cuda.synchronize()
    got = y_d.cpu().numpy()
    xs = np.ascontiguousarray(x[:, :width])
    ex, i, g, w = O.worst_violation(got[:, :width], O.rmsnorm_f32(xs, gb, wt), 1e-5)
    assert ex <= 0, f"index {i} got {g} want {w}"
    assert O.normwise_rel_err(got[:, :width], O.rmsnorm_f64(xs, gb, wt)) <= 1e-6
    if inplace:
        np.testing.assert_array_equal(got[:, width:], x[:, width:])
    else:
        assert np.all(got[:, width:] == -7.0)
