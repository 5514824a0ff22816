"""The oracle pinned against library routines, closed forms and invariants (CPU only).

Each check is chosen so that a plausible slip in the oracle (a dropped epilogue term, a
wrong rounding, a transposed operand, a wrong RoPE pairing) fails it; none re-types the
oracle's own formula.
"""
import hashlib
import json
import math
import os

import numpy as np
import pytest
import scipy.special
import scipy.stats
import torch
import torch.nn.functional as F

import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ------------------------------------------------------------------ 16-bit types --

def test_f16_decode_matches_numpy_all_patterns():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.decode16(bits, O.F16)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f16_encode_matches_numpy_rne():
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(3.0),
        (rng.standard_normal(50000) * 1e-5).astype(np.float32),          # subnormal range
        (rng.standard_normal(50000) * 3e4).astype(np.float32),           # near overflow
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, np.inf, -np.inf,
                  2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -14, 1.0 + 2.0 ** -11,
                  1.0 + 3 * 2.0 ** -11], np.float32),
    ])
    # every exact tie between neighbouring halves: midpoints of random half pairs
    h = rng.integers(0, 0x7BFF, 20000).astype(np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).astype(np.uint16).view(np.float16).astype(np.float64)
    x = np.concatenate([x, ((lo + hi) / 2).astype(np.float32)])
    bits, rounded = O.round16(x, O.F16)
    want = x.astype(np.float16)
    assert np.array_equal(bits, want.view(np.uint16))
    assert np.array_equal(rounded, want.astype(np.float32))


def test_bf16_round_matches_torch_rne():
    rng = np.random.default_rng(2)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32),
        (rng.standard_normal(20000) * 1e-38).astype(np.float32),
        np.array([1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, -1.0 - 2.0 ** -8, 3.0e38, 0.0, -0.0], np.float32),
    ])
    bits, rounded = O.round16(x, O.BF16)
    want = torch.from_numpy(x).to(torch.bfloat16)
    assert np.array_equal(bits, want.view(torch.int16).numpy().view(np.uint16))
    assert np.array_equal(rounded, want.float().numpy())
    # decode agrees with torch's widening on every pattern that is not NaN
    allb = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    dec = O.decode16(allb, O.BF16)
    tw = torch.from_numpy(allb.view(np.int16)).view(torch.bfloat16).float().numpy()
    ok = ~np.isnan(tw)
    assert np.array_equal(dec[ok].view(np.uint32), tw[ok].view(np.uint32))


# ---------------------------------------------------------------------- RNGs --

def _lcg_skip(state: int, n: int) -> int:
    """State after n steps by the closed form s_n = a^n s_0 + c (a^n - 1) / (a - 1) mod 2^64,
    evaluated by repeated squaring of the affine map (an algorithm independent of the fill loop)."""
    a, c, mod = 6364136223846793005, 1442695040888963407, 1 << 64
    acc_a, acc_c = 1, 0
    cur_a, cur_c = a, c
    while n:
        if n & 1:
            acc_a, acc_c = (acc_a * cur_a) % mod, (acc_c * cur_a + cur_c) % mod
        cur_a, cur_c = (cur_a * cur_a) % mod, (cur_c * cur_a + cur_c) % mod
        n >>= 1
    return (acc_a * state + acc_c) % mod


def test_lcg_is_the_affine_recurrence_and_uniform():
    rng = O.LCG(12345)
    v = rng.floats(100000)
    assert rng.state == _lcg_skip(12345, 100000)
    # value t is determined by the state after t+1 steps: top 24 bits scaled to [-1, 1)
    for t in (0, 1, 977, 99999):
        s = _lcg_skip(12345, t + 1)
        assert v[t] == np.float32((s >> 40) / 2.0 ** 24 * 2 - 1)
    assert v.min() >= -1.0 and v.max() < 1.0
    assert abs(v.mean()) < 0.01 and abs(v.var() - 1 / 3) < 0.01
    # Hull-Dobell: c odd and a - 1 divisible by 4, so the period is the full 2^64
    assert 1442695040888963407 % 2 == 1 and (6364136223846793005 - 1) % 4 == 0


PHI64 = 0x9E3779B97F4A7C15  # SplitMix64 state increment


def test_splitmix64_matches_published_reference_outputs():
    """SplitMix64 seeded with 1234567 (state += golden before each output) starts
    6457827717110365317, 3203168211198807973, 9817491932198370423, 4593380528125082431,
    16408922859458223821 (the published reference outputs of Rosetta Code's
    "Pseudo-random numbers/Splitmix64" task).  The reference's stream starts its state one
    golden step later (Engine.swift:434), so its seed for that stream is 1234567 - golden."""
    want = [6457827717110365317, 3203168211198807973, 9817491932198370423, 4593380528125082431,
            16408922859458223821]
    seed = (1234567 - PHI64) % 2**64
    assert [O.splitmix64(seed, t) for t in range(1, 6)] == want


def test_gaussian_pairs_are_box_muller_of_the_stream():
    """Pair j of ``gaussian`` is Box-Muller of draws 2j+1 and 2j+2, each taken as its top 53
    bits / 2^53 (Engine.swift:435-450): z0 = sqrt(-2 ln u1) cos(2 pi u2), z1 = ... sin, both
    rounded to fp32, then scaled in fp32."""
    seed = 11
    z = O.gaussian(seed, 8)
    zs = O.gaussian(seed, 8, 0.02)
    for j in range(4):
        u1 = max((O.splitmix64(seed, 2 * j + 1) >> 11) / 2.0**53, 1e-300)
        u2 = (O.splitmix64(seed, 2 * j + 2) >> 11) / 2.0**53
        r = np.sqrt(-2.0 * np.log(u1))
        z0, z1 = np.float32(r * np.cos(2 * np.pi * u2)), np.float32(r * np.sin(2 * np.pi * u2))
        assert z[2 * j] == z0 and z[2 * j + 1] == z1
        assert zs[2 * j] == np.float32(z0 * np.float32(0.02)) and zs[2 * j + 1] == np.float32(z1 * np.float32(0.02))


def test_gaussian_is_standard_normal_and_seeded():
    z = O.gaussian(0, 400000)
    assert scipy.stats.kstest(z.astype(np.float64), "norm").pvalue > 1e-3
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01
    # pairs are (r cos, r sin) of one radius: z0^2 + z1^2 = -2 ln u1 >= 0 and the angle is uniform
    ang = np.arctan2(z[1::2], z[0::2])
    assert scipy.stats.kstest((ang + np.pi) / (2 * np.pi), "uniform").pvalue > 1e-3
    assert np.array_equal(O.gaussian(0, 1001), O.gaussian(0, 1001))
    assert np.array_equal(O.gaussian(7, 1000)[:999], O.gaussian(7, 999))   # prefix-stable
    assert not np.array_equal(O.gaussian(1, 1000), O.gaussian(0, 1000))
    s = O.gaussian(3, 1000, 0.02)
    assert np.array_equal(s, (O.gaussian(3, 1000) * np.float32(0.02)).astype(np.float32))


# -------------------------------------------------------------------- linear --

def _lib_linear64(x, w, w2, b, y0, flags):
    """The linear from library routines: numpy fp64 matmul, scipy's expit for SiLU, torch's
    tanh-approximate GELU, in the epilogue order of the reference kernels."""
    acc = x.astype(np.float64) @ w.astype(np.float64).T
    v = acc + (b.astype(np.float64) if b is not None else 0.0)
    if flags & O.SILU_GATE:
        v = v * scipy.special.expit(v) * (x.astype(np.float64) @ w2.astype(np.float64).T)
    if flags & O.GELU:
        v = F.gelu(torch.from_numpy(v), approximate="tanh").numpy()
    if flags & O.SILU:
        v = v * scipy.special.expit(v)
    if flags & O.ACCUM:
        v = v + y0.astype(np.float64)
    return v


def _random_linear(seed, M, N, K, wt, x_scale=1.0):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((M, K)) * x_scale).astype(np.float32)
    wb, w = O.round16(rng.standard_normal((N, K)).astype(np.float32) * np.float32(0.05), wt)
    w2b, w2 = O.round16(rng.standard_normal((N, K)).astype(np.float32) * np.float32(0.05), wt)
    bb, b = O.round16(rng.standard_normal(N).astype(np.float32), wt)
    y0 = rng.standard_normal((M, N)).astype(np.float32)
    return x, wb, w, w2b, w2, bb, b, y0


FLAG_SETS = [0, O.ACCUM, O.GELU, O.SILU, O.SILU_GATE, O.SILU_GATE | O.ACCUM, O.GELU | O.ACCUM,
             O.GELU | O.SILU, O.SILU_GATE | O.GELU | O.SILU | O.ACCUM]


@pytest.mark.parametrize("flags", FLAG_SETS)
@pytest.mark.parametrize("wt", [O.F16, O.BF16])
def test_linear_f64_matches_library_routines(flags, wt):
    M, N, K = 3, 37, 72
    x, wb, w, w2b, w2, bb, b, y0 = _random_linear(flags * 10 + wt, M, N, K, wt, x_scale=2.0)
    for use_bias in (False, True):
        got = O.linear_f64(x, wb, w2b if flags & O.SILU_GATE else None, wt, bb if use_bias else None, y0,
                           M, N, K, flags)
        want = _lib_linear64(x, w, w2, b if use_bias else None, y0, flags)
        np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("flags", FLAG_SETS)
def test_linear_np64_agrees_with_linear_f64(flags):
    M, N, K = 3, 40, 96
    x, wb, w, w2b, w2, bb, b, y0 = _random_linear(300 + flags, M, N, K, O.BF16, x_scale=3.0)
    gw2 = w2b if flags & O.SILU_GATE else None
    np.testing.assert_allclose(O.linear_np64(x, wb, gw2, O.BF16, bb, y0, flags | O.BIAS),
                               O.linear_f64(x, wb, gw2, O.BF16, bb, y0, M, N, K, flags), rtol=1e-12, atol=1e-12)


def test_rmsnorm_matches_torch_rms_norm():
    rng = np.random.default_rng(12)
    x = (rng.standard_normal((5, 896)) * 3).astype(np.float32)
    gb, g = O.round16(rng.standard_normal(896).astype(np.float32), O.BF16)
    want = F.rms_norm(torch.from_numpy(x.astype(np.float64)), (896,), torch.from_numpy(g.astype(np.float64)),
                      eps=float(np.float32(1e-6))).numpy()
    np.testing.assert_allclose(O.rmsnorm_f64(x, gb, O.BF16), want, rtol=1e-12, atol=1e-12)
    # the fp32 reference loop sits within fp32 rounding of it
    np.testing.assert_allclose(O.rmsnorm_f32(x, gb, O.BF16), want, rtol=2e-6, atol=1e-6)
    # scale invariance: rmsnorm(c x) == rmsnorm(x) up to eps
    np.testing.assert_allclose(O.rmsnorm_f64(x * 4, gb, O.BF16, 0.0), O.rmsnorm_f64(x, gb, O.BF16, 0.0), rtol=1e-12)


def test_linear_f64_brute_force_tiny():
    """2 x 3 x 8 against explicit triple loops over the decoded weights."""
    M, N, K = 2, 3, 8
    x, wb, w, w2b, w2, bb, b, y0 = _random_linear(5, M, N, K, O.BF16)
    got = O.linear_f64(x, wb, None, O.BF16, bb, None, M, N, K, 0)
    for m in range(M):
        for n in range(N):
            s = 0.0
            for k in range(K):
                s += float(x[m, k]) * float(w[n, k])
            assert abs(got[m, n] - (s + float(b[n]))) < 1e-12


def test_linear_selects_rows_and_columns():
    """One-hot x picks a weight column; one-hot-row W picks an x column (catches a transpose)."""
    M, N, K = 4, 16, 32
    _, wb, w, *_ = _random_linear(9, M, N, K, O.F16)
    x = np.zeros((M, K), np.float32)
    for m in range(M):
        x[m, 3 * m + 1] = 1.0
    got = O.linear_f64(x, wb, None, O.F16, None, None, M, N, K, 0)
    for m in range(M):
        np.testing.assert_array_equal(got[m], w[:, 3 * m + 1].astype(np.float64))
    eye = np.zeros((N, K), np.float32)
    eye[np.arange(N), (np.arange(N) * 5) % K] = 1.0
    eb, _ = O.round16(eye, O.F16)
    xr = np.random.default_rng(3).standard_normal((M, K)).astype(np.float32)
    got = O.linear_f64(xr, eb, None, O.F16, None, None, M, N, K, 0)
    np.testing.assert_array_equal(got, xr[:, (np.arange(N) * 5) % K].astype(np.float64))


@pytest.mark.parametrize("flags", FLAG_SETS)
def test_linear_f32_and_fast_within_fp32_bound(flags):
    """The fp32 reference loop and the split-sum baseline sit within the fp32 summation bound
    of the fp64 recomputation: |y32 - y64| <= 2 K u sum_k |x||w| (+ epilogue slack)."""
    M, N, K = 2, 64, 896
    x, wb, w, w2b, w2, bb, b, y0 = _random_linear(100 + flags, M, N, K, O.F16)
    gw2 = w2b if flags & O.SILU_GATE else None
    want = O.linear_f64(x, wb, gw2, O.F16, bb, y0, M, N, K, flags)
    mag = np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64).T
    if flags & O.SILU_GATE:
        mag = mag * (1 + np.abs(x).astype(np.float64) @ np.abs(w2).astype(np.float64).T)
    bound = 2 * K * 2.0 ** -24 * (mag + np.abs(b)) + 1e-5 * (1 + np.abs(want))
    for fn in (O.linear_f32, O.linear_fast):
        got = fn(x, wb, gw2, O.F16, bb, y0, M, N, K, flags)
        assert np.all(np.abs(got - want) <= bound), fn.__name__


def test_epilogue_special_cases():
    """x = 0 reduces every output to act(bias) (+ y0): closed forms for each flag."""
    M, N, K = 2, 64, 16
    x = np.zeros((M, K), np.float32)
    bb, b = O.round16(np.linspace(-12, 12, N).astype(np.float32), O.F16)
    wb, _ = O.round16(np.ones((N, K), np.float32), O.F16)
    y0 = np.full((M, N), 0.5, np.float32)
    b64 = b.astype(np.float64)
    gelu_erf = 0.5 * b64 * (1 + scipy.special.erf(b64 / math.sqrt(2)))
    cases = {
        0: b64,
        O.SILU: b64 * scipy.special.expit(b64),
        O.GELU: F.gelu(torch.from_numpy(b64), approximate="tanh").numpy(),
        O.GELU | O.ACCUM: F.gelu(torch.from_numpy(b64), approximate="tanh").numpy() + 0.5,
        O.SILU_GATE: np.zeros(N),                     # silu(b) * (x . w2) = silu(b) * 0
    }
    for flags, want in cases.items():
        got = O.linear_f64(x, wb, wb, O.F16, bb, y0, M, N, K, flags)
        # atol 1e-11: the reference clamps the tanh argument to +-15 (Shaders.swift:21-27), which
        # leaves 0.5 v (1 + tanh(-15)) ~ -1e-12 at v = -12 where the unclamped form gives 0.
        np.testing.assert_allclose(got, np.broadcast_to(want, (M, N)), rtol=1e-12, atol=1e-11)
    # the tanh form stays within 1e-3 of the exact (erf) GELU: a dropped cubic term would not
    got = O.linear_f64(x, wb, None, O.F16, bb, None, M, N, K, O.GELU)[0]
    assert np.max(np.abs(got - gelu_erf)) < 1e-3
    # accumulate comes last: gelu(b) + y0, not gelu(b + y0)
    got = O.linear_f64(x, wb, None, O.F16, bb, y0, M, N, K, O.GELU | O.ACCUM)[0]
    assert np.max(np.abs(got - (gelu_erf + 0.5))) < 1e-3


# ------------------------------------------------------------ known answers --

def _digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        if a is not None:
            h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()[:24]


def test_kat_cases_match_committed_digests():
    """The regenerated known-answer cases (inputs and fp32 expected outputs) are the ones the
    committed fixture recorded, so a drift in the RNG, the rounding or the loop shows up."""
    with open(os.path.join(GOLDEN, "kat_digests.json")) as f:
        golden = json.load(f)
    small = [c for c in O.KAT_ALL if c[0] * c[1] * c[2] <= 4 * 1152 * 896]
    for (m, n, k, flags, bias, xs) in small:
        c = O.gemv_case(m, n, k, flags, bias, xs)
        key = f"{m}x{n}x{k}:f{flags}:b{int(bias)}:s{xs}"
        assert key in golden, key
        g = golden[key]
        assert _digest(c["x"][:m], c["w"], c["w2"] if flags & O.SILU_GATE else None, c["bias"], c["y0"]) == g["inputs"]
        np.testing.assert_allclose(c["want"].ravel()[:8], np.array(g["want_head"], np.float32), rtol=0, atol=0)
        assert abs(float(np.sum(c["want"].astype(np.float64))) - g["want_sum"]) <= 1e-6 * max(1.0, abs(g["want_sum"]))


def test_kat_tolerance_separates_a_planted_mistake():
    """The reference's per-element tolerance rejects a plausible oracle slip (bias dropped,
    accumulate applied before GELU), so the KAT comparison has teeth."""
    c = O.gemv_case(6, 256, 1024, O.GELU, True, 1.0)
    m, n, k = 6, 256, 1024
    atol = O.kat_atol(k)
    ok, *_ = O.worst_violation(O.linear_f64(c["x"][:m], c["w"], None, O.BF16, c["bias"], None, m, n, k, O.GELU),
                               c["want"], atol)
    assert ok <= 0
    no_bias = O.linear_f64(c["x"][:m], c["w"], None, O.BF16, None, None, m, n, k, O.GELU)
    assert O.worst_violation(no_bias, c["want"], atol)[0] > 0
    c2 = O.gemv_case(1, 256, 896, O.GELU | O.ACCUM, False, 8.0)
    x = c2["x"][:1].astype(np.float64)
    v = x @ c2["w"].astype(np.float64).T
    wrong = F.gelu(torch.from_numpy(v + c2["y0"]), approximate="tanh").numpy()
    assert O.worst_violation(wrong, c2["want"], O.kat_atol(896))[0] > 0


def test_nan_sentinel_rows_are_outside_the_oracle():
    c = O.gemv_case(2, 2, 896, 0, True)
    assert np.all(np.isnan(c["x"][2:])) and np.all(np.isfinite(c["want"]))


# --------------------------------------------------------- rope / attention --

def test_inv_freq_and_rope_invariants():
    invf = O.inv_freq(1e6)
    assert invf[0] == 1.0 and abs(invf[31] - 1e6 ** (-62 / 64)) < 1e-9
    rng = np.random.default_rng(4)
    q = rng.standard_normal((5, 64))
    k = rng.standard_normal((5, 64))
    np.testing.assert_allclose(O.rope_neox(q, 0, invf), q, atol=0)          # position 0 is the identity
    for p in (1, 17, 511):
        r = O.rope_neox(q, p, invf)
        np.testing.assert_allclose(np.linalg.norm(r, axis=-1), np.linalg.norm(q, axis=-1), rtol=1e-12)
    # relative position: <R(a) q, R(b) k> depends on b - a only (pairs (i, i+32) rotate together)
    d1 = np.sum(O.rope_neox(q, 10, invf, False) * O.rope_neox(k, 13, invf, False), -1)
    d2 = np.sum(O.rope_neox(q, 100, invf, False) * O.rope_neox(k, 103, invf, False), -1)
    np.testing.assert_allclose(d1, d2, rtol=1e-9)
    # the fp32 angle (the reference's) is within one fp32 rounding of the exact angle
    r32, r64 = O.rope_neox(q, 511, invf), O.rope_neox(q, 511, invf, False)
    assert np.max(np.abs(r32 - r64)) <= 511 * 2.0 ** -24 * np.max(np.abs(q)) * 2
    # pairing is (i, i+32): a vector living only in dims {0, 32} stays there
    e = np.zeros(64)
    e[0] = 1.0
    r = O.rope_neox(e, 5, invf)
    assert np.count_nonzero(np.abs(r) > 1e-15) == 2 and abs(r[0] - math.cos(5.0)) < 1e-12 and abs(r[32] - math.sin(5.0)) < 1e-12


def test_attention_matches_torch_sdpa():
    """Causal GQA over a cache against torch's scaled_dot_product_attention in fp64."""
    rng = np.random.default_rng(6)
    hq, hkv, cap = 14, 2, 96
    k = rng.standard_normal((hkv, cap, 64))
    v = rng.standard_normal((hkv, cap, 64))
    q = rng.standard_normal((hq, 64))
    for qpos, window in ((0, 0), (40, 0), (95, 0), (95, 64), (30, 64)):
        got = O.attention_f64(q, k, v, qpos, window, 0.125)
        start = qpos + 1 - window if window and qpos + 1 > window else 0
        kk = torch.from_numpy(np.repeat(k[:, start:qpos + 1], hq // hkv, axis=0))[None]
        vv = torch.from_numpy(np.repeat(v[:, start:qpos + 1], hq // hkv, axis=0))[None]
        want = F.scaled_dot_product_attention(torch.from_numpy(q)[None, :, None, :], kk, vv, scale=0.125)
        np.testing.assert_allclose(got, want[0, :, 0].numpy(), rtol=1e-10, atol=1e-12)


def test_interleaved_rope_invariants():
    """x_transformers rotary (Shaders.swift:605-608): identity at position 0, norm-preserving,
    relative-position dot products, and pairs (2p, 2p + 1) rotating together."""
    invf = (1.0 / np.power(np.float32(1e4), np.float32(2.0) * np.arange(32, dtype=np.float32) / np.float32(64))).astype(np.float32)
    rng = np.random.default_rng(8)
    q = rng.standard_normal((4, 64))
    k = rng.standard_normal((4, 64))
    np.testing.assert_allclose(O.rope_interleaved(q, 0, invf), q, atol=0)
    for p in (1, 2, 7):
        np.testing.assert_allclose(np.linalg.norm(O.rope_interleaved(q, p, invf), axis=-1), np.linalg.norm(q, axis=-1),
                                   rtol=1e-12)
    d1 = np.sum(O.rope_interleaved(q, 2, invf) * O.rope_interleaved(k, 5, invf), -1)
    d2 = np.sum(O.rope_interleaved(q, 4, invf) * O.rope_interleaved(k, 7, invf), -1)
    # equal up to the fp32 rounding of the angles (the reference forms them in fp32)
    np.testing.assert_allclose(d1, d2, rtol=0, atol=1e-5)
    e = np.zeros(64)
    e[2] = 1.0   # dim 2 pairs with dim 3 at frequency invf[1]
    r = O.rope_interleaved(e, 3, invf)
    a = float(np.float32(3) * invf[1])
    assert np.count_nonzero(np.abs(r) > 1e-15) == 2
    assert abs(r[2] - math.cos(a)) < 1e-12 and abs(r[3] - math.sin(a)) < 1e-12


def test_dit_attention_matches_torch_sdpa():
    """Full attention per sequence on the rotated q / k against torch's fp64 SDPA; one row
    per sequence returns v; NeoX pairing in place of the interleaved one is caught."""
    B, S, H = 2, 3, 4
    D = H * 64
    invf = (1.0 / np.power(np.float32(1e4), np.float32(2.0) * np.arange(32, dtype=np.float32) / np.float32(64))).astype(np.float32)
    qkv = O.LCG(11).floats(B * S * 3 * D).reshape(B * S, 3 * D).astype(np.float64)
    got = O.dit_attention_f64(qkv, B, S, H, invf)
    pos = np.arange(S)
    for b in range(B):
        rows = qkv[b * S:(b + 1) * S]
        q = np.stack([O.rope_interleaved(rows[:, h * 64:(h + 1) * 64], pos, invf) for h in range(H)])
        k = np.stack([O.rope_interleaved(rows[:, D + h * 64:D + (h + 1) * 64], pos, invf) for h in range(H)])
        v = np.stack([rows[:, 2 * D + h * 64:2 * D + (h + 1) * 64] for h in range(H)])
        want = F.scaled_dot_product_attention(torch.from_numpy(q)[None], torch.from_numpy(k)[None],
                                              torch.from_numpy(v)[None], scale=0.125)[0].numpy()
        np.testing.assert_allclose(got[b * S:(b + 1) * S].reshape(S, H, 64), want.transpose(1, 0, 2), rtol=1e-10,
                                   atol=1e-12)
    one = O.dit_attention_f64(qkv[:2], 2, 1, H, invf)   # S = 1: softmax of one key
    np.testing.assert_array_equal(one, qkv[:2, 2 * D:])
    # a plausible mistake: NeoX pairs (i, i + 32) in place of interleaved (2p, 2p + 1)
    neox = np.empty_like(got)
    for b in range(B):
        rows = qkv[b * S:(b + 1) * S]
        for h in range(H):
            q = O.rope_neox(rows[:, h * 64:(h + 1) * 64], pos, invf)
            k = O.rope_neox(rows[:, D + h * 64:D + (h + 1) * 64], pos, invf)
            sc = q @ k.T * 0.125
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            neox[b * S:(b + 1) * S, h * 64:(h + 1) * 64] = (p / p.sum(1, keepdims=True)) @ rows[:, 2 * D + h * 64:2 * D + (h + 1) * 64]
    assert np.max(np.abs(neox - got)) > 100 * 2e-5   # far outside the reference test's atol


def test_flow_assemble_and_euler_closed_forms():
    """Flow input rows against torch's fp64 linear and the slot layout; the Euler step at cfg
    0 and 1."""
    rng = np.random.default_rng(12)
    hidden, latent = 96, 64
    w, _ = O.round16(rng.standard_normal((hidden, latent)).astype(np.float32) * np.float32(0.05), O.BF16)
    xb, _ = O.round16(rng.standard_normal(hidden).astype(np.float32) * np.float32(0.05), O.BF16)
    cb, _ = O.round16(rng.standard_normal(hidden).astype(np.float32), O.BF16)
    y, hist = rng.standard_normal(latent), rng.standard_normal(latent)
    cemb, temb = rng.standard_normal(hidden), rng.standard_normal(hidden)
    x = O.flow_assemble_f64(y, hist, cemb, cb, temb, w, xb, O.BF16)
    wt = torch.from_numpy(O.decode16(w, O.BF16).astype(np.float64))
    bt = torch.from_numpy(O.decode16(xb, O.BF16).astype(np.float64))
    np.testing.assert_allclose(x[1], F.linear(torch.from_numpy(hist), wt, bt).numpy(), rtol=1e-12)
    np.testing.assert_allclose(x[2], F.linear(torch.from_numpy(y), wt, bt).numpy(), rtol=1e-12)
    np.testing.assert_array_equal(x[4], x[1])
    np.testing.assert_array_equal(x[5], x[2])
    np.testing.assert_allclose(x[0], temb + cemb, rtol=1e-15)
    np.testing.assert_allclose(x[3], temb + O.decode16(cb, O.BF16), rtol=1e-15)
    pred = rng.standard_normal((6, latent))
    y0 = rng.standard_normal(latent)
    y1, cap = O.flow_euler_f64(y0, pred, 2, 5, 0.0, 0.25)
    np.testing.assert_allclose(y1, y0 + pred[2] * 0.25, rtol=1e-15)
    y2, _ = O.flow_euler_f64(y0, pred, 2, 5, 1.0, 0.5)
    np.testing.assert_allclose(y2, y0 + (2 * pred[2] - pred[5]) * 0.5, rtol=1e-14)
    np.testing.assert_array_equal(cap, np.concatenate([pred[2], pred[5]]))


def test_istft_frame_matches_a_direct_dft_and_upsample_matches_torch():
    """The frame synthesis against the reference's direct double loop (KernelTests.swift:
    361-374) at a small N, with a planted sign mistake caught; the upsample against torch's
    linear interpolation (align_corners = False, scale 4; KernelTests.swift:384-398)."""
    N = 24
    bins = N // 2 + 1
    rng = np.random.default_rng(13)
    row = np.concatenate([rng.uniform(-1, 1, bins), rng.uniform(0, 3, bins)])
    win = 0.5 - 0.5 * np.cos(2 * np.pi * np.arange(N) / N)
    got = O.istft_frame_f64(row, N, win)
    mag = np.minimum(np.exp(row[:bins]), 100.0)
    re, im = mag * np.cos(row[bins:]), mag * np.sin(row[bins:])
    want = np.empty(N)
    for t in range(N):
        acc = re[0] + (re[N // 2] if t % 2 == 0 else -re[N // 2])
        for k in range(1, N // 2):
            a = 2 * np.pi * (k * t % N) / N
            acc += 2 * (re[k] * np.cos(a) - im[k] * np.sin(a))
        want[t] = acc / N * win[t]
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-14)
    planted = O.istft_frame_f64(np.concatenate([row[:bins], -row[bins:]]), N, win)   # conjugate phase
    assert np.max(np.abs(planted - want)) > 1e-3
    h = O.LCG(9).floats(5 * 32).reshape(5, 32).astype(np.float64)
    frames = np.concatenate([O.upsample4_f64(h[i - 1] if i else None, h[i], h[i + 1] if i < 4 else None)
                             for i in range(5)])
    ref = F.interpolate(torch.from_numpy(h.T[None]), scale_factor=4, mode="linear", align_corners=False)[0].T.numpy()
    np.testing.assert_allclose(frames, ref, rtol=1e-12, atol=1e-12)


def test_istft_emit_reconstructs_a_stream():
    """Frames cut from a known signal with a Hann analysis window, times the synthesis window
    (as istft_frames applies it), overlap-added with the window^2 envelope give the signal
    back: the identity the emit step relies on."""
    N, hop = 32, 8
    rng = np.random.default_rng(14)
    sig = rng.standard_normal(12 * hop + N)
    win = 0.5 - 0.5 * np.cos(2 * np.pi * np.arange(N) / N)
    frames = [sig[f * hop:f * hop + N] * win * win for f in range(12)]
    pad = (N - hop) // 2
    out = O.istft_emit_f64(frames, win, N, hop, 0, 8 * hop, 11)
    np.testing.assert_allclose(out, sig[pad:pad + 8 * hop], rtol=1e-12)
