"""Writes the committed fixtures of tests/golden/ from the oracle.

The reference holds no stored vectors for the linear path: its known-answer tests
compute inputs from an LCG and expected values from a CPU loop at test time
(Tests/MingTTSTests/KernelTests.swift:21-103).  These fixtures record what the oracle
regenerates for those cases (input digests, the first expected values and their sum),
so a later change to the RNG, the rounding or the loop is caught.  Also recorded: the
single-GEMV configuration (W fp16 [4864 x 896] ~ N(0, 0.02^2), x fp16 [896] ~ N(0, 1),
seed 0) as computed by the fp32 reference loop.

    python tests/golden/make_fixtures.py
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import oracle as O  # noqa: E402


def digest(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        if a is not None:
            h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()[:24]


def c1_inputs():
    """C1: one normal stream, seed 0: the first N*K draws x 0.02 are W, the next K are x."""
    N, K = 4864, 896
    z = O.gaussian(0, N * K + K)
    wb, _ = O.round16(z[:N * K] * np.float32(0.02), O.F16)
    xb, xr = O.round16(z[N * K:], O.F16)
    return wb.reshape(N, K), xb.reshape(1, K), xr.reshape(1, K)


def main():
    kat = {}
    for (m, n, k, flags, bias, xs) in O.KAT_ALL:
        if m * n * k > 4 * 1152 * 896:
            continue
        c = O.gemv_case(m, n, k, flags, bias, xs)
        key = f"{m}x{n}x{k}:f{flags}:b{int(bias)}:s{xs}"
        kat[key] = dict(
            inputs=digest(c["x"][:m], c["w"], c["w2"] if flags & O.SILU_GATE else None, c["bias"], c["y0"]),
            want_head=[float(v) for v in c["want"].ravel()[:8]],
            want_sum=float(np.sum(c["want"].astype(np.float64))),
        )
    with open(os.path.join(HERE, "kat_digests.json"), "w") as f:
        json.dump(kat, f, indent=1, sort_keys=True)

    wb, xb, xr = c1_inputs()
    y = O.linear_f32(xr, wb, None, O.F16, None, None, 1, 4864, 896, 0)
    y64 = O.linear_f64(xr, wb, None, O.F16, None, None, 1, 4864, 896, 0)
    c1 = dict(w_digest=digest(wb), x_digest=digest(xb), y_head=[float(v) for v in y[0, :16]],
              y_sum=float(np.sum(y.astype(np.float64))), y64_absmax=float(np.max(np.abs(y64))))
    with open(os.path.join(HERE, "c1_gemv.json"), "w") as f:
        json.dump(c1, f, indent=1, sort_keys=True)
    print(f"wrote {len(kat)} KAT digests and the C1 fixture")


if __name__ == "__main__":
    main()
