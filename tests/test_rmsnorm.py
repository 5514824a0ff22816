"""mt_rmsnorm's refusals, through the C ABI on the CPU: each call is rejected by the
argument checks before anything reaches the GPU (the pointers are never dereferenced)."""
import pytest

import mingtts as mt

X, G, Y = 0x10000, 0x20000, 0x30000


@pytest.mark.parametrize("args,what", [
    ((X, 896, 2, 6, G, mt.BF16, Y, 896), "multiple of 4"),
    ((X, 892, 2, 896, G, mt.BF16, Y, 896), "strides"),
    ((X, 898, 2, 896, G, mt.BF16, Y, 896), "strides"),
    ((X + 4, 896, 2, 896, G, mt.BF16, Y, 896), "16-byte"),
    ((X, 896, 2, 896, G + 2, mt.BF16, Y, 896), "8-byte"),
    ((X, 896, 2, 896, G, mt.F32, Y, 896), "f16 or bf16"),
    ((X, 896, 2, 896, G, mt.BF16, X + 16, 896), "overlaps"),
    ((X, 896, 2, 896, G, mt.BF16, X, 900), "in place"),
    ((None, 896, 2, 896, G, mt.BF16, Y, 896), "null"),
])
def test_rmsnorm_refusals(args, what):
    x, ldx, rows, width, g, wt, y, ldy = args
    assert mt.rmsnorm_raw(x, ldx, rows, width, g, wt, y, ldy, 1e-6, stream=0) == mt.EINVAL
    assert what in mt.last_error()


def test_rmsnorm_of_no_rows_is_a_no_op():
    assert mt.rmsnorm_raw(X, 896, 0, 896, G, mt.BF16, Y, 896, 1e-6, stream=0) == mt.OK
