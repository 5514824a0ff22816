"""CPU oracle for the MingTTS linear hot path.

TEST INFRASTRUCTURE, NOT PRODUCT CODE.  Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker (or as the timed CPU baseline).  The HIP library never calls it.

Contents (reference paths relative to the reference checkout):

* ``LCG`` -- the known-answer-test RNG of Tests/MingTTSTests/KernelTests.swift:21-28.
* ``round16`` / ``decode16`` -- bf16 rounding of KernelTests.swift:30-36, and IEEE fp16.
* ``gaussian`` -- SplitMix64 + Box-Muller of Sources/MingTTS/Engine/Engine.swift:432-453.
* ``linear_f32`` -- the reference CPU loop of one linear, KernelTests.swift:86-101, with
  the kernels' epilogue order (Sources/MingTTS/Engine/Shaders.swift:21-29, 92-103).
* ``linear_f64`` -- fp64 recomputation on the same rounded inputs (the precision gate).
* ``linear_fast`` -- the same linear with a 16-way split K sum (timed CPU baseline).
* ``rope_neox`` / ``attention_f64`` -- NeoX RoPE and causal GQA attention over a cache,
  restating Shaders.swift:451-596 and the CPU reference of KernelTests.swift:207-268.
* ``gemv_case`` -- regenerates the reference's linear known-answer tests bit for bit
  (KernelTests.swift:72-103).
* ``rope_interleaved`` / ``dit_attention_f64`` / ``flow_assemble_f64`` / ``flow_euler_f64``
  -- the DiT flow step around its linears: Shaders.swift:598-693 and the CPU reference of
  KernelTests.swift:282-318.
* ``flow_timesteps_f64`` / ``sinusoid_f64`` / ``time_mlp_f64`` -- the flow sampler's
  schedule and timestep embedding (Sources/MingTTS/Engine/DiT.swift:55-80) and the time-MLP
  precompute (Sources/MingTTS/Engine/Engine.swift:186-198), in fp64 closed form.
* ``upsample4_f64`` / ``istft_frame_f64`` / ``istft_emit_f64`` -- the VAE decoder's tail:
  Shaders.swift:697-790 and the CPU references of KernelTests.swift:322-398.
"""
from __future__ import annotations

import ctypes
import math
import os

import numpy as np

F32, F16, BF16 = 0, 1, 2
BIAS, ACCUM, GELU, SILU_GATE, SILU = 1, 2, 4, 8, 16

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def lib() -> ctypes.CDLL:
    """The compiled oracle (oracle/libmt_oracle.so, built by ``make -C oracle``)."""
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "libmt_oracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"oracle library missing: {path} (run make -C oracle)")
        L = ctypes.CDLL(path)
        vp, i64, i32, u32, u64, f32 = (ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                                       ctypes.c_uint32, ctypes.c_uint64, ctypes.c_float)
        L.mto_lcg_fill.argtypes = [u64, vp, i64, f32]
        L.mto_lcg_fill.restype = u64
        L.mto_gaussian_fill.argtypes = [u64, vp, i64, f32]
        L.mto_gaussian_fill.restype = None
        L.mto_splitmix64.argtypes = [u64, u64]
        L.mto_splitmix64.restype = u64
        L.mto_bf16_bits.argtypes = [f32]
        L.mto_bf16_bits.restype = ctypes.c_uint16
        L.mto_f16_bits.argtypes = [f32]
        L.mto_f16_bits.restype = ctypes.c_uint16
        L.mto_round16.argtypes = [vp, i64, i32, vp, vp]
        L.mto_round16.restype = None
        L.mto_decode16.argtypes = [vp, i64, i32, vp]
        L.mto_decode16.restype = None
        sig = [vp, i64, vp, vp, i32, vp, vp, vp, i64, i32, i32, i32, u32, i32]
        L.mto_linear_f32.argtypes = sig
        L.mto_linear_f32.restype = i32
        L.mto_linear_fast.argtypes = sig
        L.mto_linear_fast.restype = i32
        L.mto_linear_f64.argtypes = [vp, i64, vp, vp, i32, vp, vp, i64, vp, i64, i32, i32, i32, u32, i32]
        L.mto_linear_f64.restype = i32
        L.mto_max_threads.argtypes = []
        L.mto_max_threads.restype = i32
        _LIB = L
    return _LIB


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


# ---------------------------------------------------------------- RNGs --

class LCG:
    """KernelTests.swift:21-28: uniforms in [-1, 1) from a 64-bit LCG, fp32 arithmetic."""

    def __init__(self, state: int):
        self.state = state & 0xFFFFFFFFFFFFFFFF

    def floats(self, n: int, scale: float = 1.0) -> np.ndarray:
        out = np.empty(n, np.float32)
        self.state = lib().mto_lcg_fill(self.state, _p(out), n, scale)
        return out


def splitmix64(seed: int, t: int) -> int:
    """The t-th 64-bit draw (t >= 1) of the SplitMix64 stream behind ``gaussian`` for ``seed``
    (Engine.swift:432-441: state = seed + golden, then state += golden per draw)."""
    return int(lib().mto_splitmix64(seed & 0xFFFFFFFFFFFFFFFF, t & 0xFFFFFFFFFFFFFFFF))


def gaussian(seed: int, n: int, scale: float = 1.0) -> np.ndarray:
    """Engine.swift:432-453: standard normals (times ``scale``) from SplitMix64 + Box-Muller."""
    out = np.empty(n, np.float32)
    lib().mto_gaussian_fill(seed & 0xFFFFFFFFFFFFFFFF, _p(out), n, scale)
    return out


# ------------------------------------------------------------ rounding --

def round16(x: np.ndarray, dtype: int) -> tuple[np.ndarray, np.ndarray]:
    """Round fp32 values to bf16 (KernelTests.swift:30-36) or fp16 (IEEE RNE).

    Returns (uint16 bits, the rounded values as fp32)."""
    x = np.ascontiguousarray(x, np.float32)
    bits = np.empty(x.shape, np.uint16)
    rounded = np.empty(x.shape, np.float32)
    lib().mto_round16(_p(x), x.size, dtype, _p(bits), _p(rounded))
    return bits, rounded


def decode16(bits: np.ndarray, dtype: int) -> np.ndarray:
    bits = np.ascontiguousarray(bits, np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().mto_decode16(_p(bits), bits.size, dtype, _p(out))
    return out


# -------------------------------------------------------------- linear --

def _linear_args(x, w, w2, bias, y0, M, N, K):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.uint16)
    w2 = None if w2 is None else np.ascontiguousarray(w2, np.uint16)
    bias = None if bias is None else np.ascontiguousarray(bias, np.uint16)
    y0 = None if y0 is None else np.ascontiguousarray(y0, np.float32)
    assert x.size >= M * K and w.size >= N * K
    return x, w, w2, bias, y0


def linear_f32(x, w, w2, wt, bias, y0, M, N, K, flags, threads=0) -> np.ndarray:
    """The reference CPU loop (KernelTests.swift:86-101): fp32, natural K order.

    x: fp32 [M, K] (rounded values if the kernel reads 16-bit x); w, w2: uint16 [N, K];
    bias: uint16 [N] or None (passing a bias sets BIAS, as Kernels.swift:135 does);
    y0: fp32 [M, N] read under ACCUM.  Returns fp32 [M, N]."""
    x, w, w2, bias, y0 = _linear_args(x, w, w2, bias, y0, M, N, K)
    if bias is not None:
        flags |= BIAS
    y = np.empty((M, N), np.float32)
    rc = lib().mto_linear_f32(_p(x), K, _p(w), _p(w2), wt, _p(bias), _p(y0), _p(y), N, M, N, K, flags, threads)
    assert rc == 0, rc
    return y


def linear_fast(x, w, w2, wt, bias, y0, M, N, K, flags, threads=0) -> np.ndarray:
    """linear_f32 with the K sum split 16 ways (vectorised); the timed CPU baseline."""
    x, w, w2, bias, y0 = _linear_args(x, w, w2, bias, y0, M, N, K)
    if bias is not None:
        flags |= BIAS
    y = np.empty((M, N), np.float32)
    rc = lib().mto_linear_fast(_p(x), K, _p(w), _p(w2), wt, _p(bias), _p(y0), _p(y), N, M, N, K, flags, threads)
    assert rc == 0, rc
    return y


def linear_f64(x, w, w2, wt, bias, y0, M, N, K, flags, threads=0) -> np.ndarray:
    """fp64 recomputation of the linear on the same inputs; returns float64 [M, N]."""
    x, w, w2, bias, y0 = _linear_args(x, w, w2, bias, y0, M, N, K)
    if bias is not None:
        flags |= BIAS
    y = np.empty((M, N), np.float64)
    rc = lib().mto_linear_f64(_p(x), K, _p(w), _p(w2), wt, _p(bias), _p(y0), N, _p(y), N, M, N, K, flags, threads)
    assert rc == 0, rc
    return y


def max_threads() -> int:
    return lib().mto_max_threads()


def _gelu64(v: np.ndarray) -> np.ndarray:
    u = np.clip(0.7978845608028654 * (v + 0.044715 * v ** 3), -15.0, 15.0)
    return 0.5 * v * (1.0 + np.tanh(u))


def linear_np64(x64, w, w2, wt, bias, y0, flags) -> np.ndarray:
    """The linear in fp64 from numpy's matmul (x64: float [M, K] in any precision, w / w2 /
    bias as 16-bit storage), epilogue in the reference order.  Used where x is itself an
    fp64 intermediate (the RMSNorm prologue)."""
    x64 = np.asarray(x64, np.float64)
    acc = x64 @ decode16(w, wt).astype(np.float64).T
    v = acc + (decode16(bias, wt).astype(np.float64) if bias is not None else 0.0)
    if flags & SILU_GATE:
        acc2 = x64 @ decode16(w2, wt).astype(np.float64).T
        v = v / (1.0 + np.exp(-v)) * acc2
    if flags & GELU:
        v = _gelu64(v)
    if flags & SILU:
        v = v / (1.0 + np.exp(-v))
    if flags & ACCUM:
        v = v + np.asarray(y0, np.float64)
    return v


def rmsnorm_f64(x, g, wt, eps: float = 1e-6) -> np.ndarray:
    """RMSNorm of rows, x * rsqrt(mean(x^2) + eps) * g (Shaders.swift:414-441;
    KernelTests.swift:187-203), in fp64.  g: 16-bit storage of type wt."""
    x64 = np.asarray(x, np.float64)
    s = 1.0 / np.sqrt(np.mean(x64 * x64, axis=-1, keepdims=True) + np.float64(np.float32(eps)))
    return x64 * s * decode16(g, wt).astype(np.float64)


def rmsnorm_f32(x, g, wt, eps: float = 1e-6) -> np.ndarray:
    """The reference's CPU RMSNorm loop (KernelTests.swift:193-199): fp32 sum of squares in
    natural order, s = 1 / sqrt(ss / k + eps), y = x * s * g, all fp32."""
    x = np.asarray(x, np.float32)
    gf = decode16(g, wt)
    out = np.empty_like(x)
    k = x.shape[-1]
    for r in range(x.shape[0]):
        ss = np.float32(0.0)
        for v in x[r]:
            ss = np.float32(ss + v * v)
        s = np.float32(1.0) / np.sqrt(np.float32(ss / np.float32(k) + np.float32(eps)))
        out[r] = x[r] * s * gf
    return out


# ---------------------------------------------------------- tolerances --

def kat_atol(k: int) -> float:
    """Per-element absolute tolerance of the reference's linear tests (KernelTests.swift:102)."""
    return 2e-4 * math.sqrt(k) / 30


def worst_violation(got: np.ndarray, want: np.ndarray, atol: float, rtol: float = 1e-4):
    """assertClose of KernelTests.swift:58-68: the element with the largest |d| - tol.

    Returns (excess, index, got, want); excess <= 0 means every element passed."""
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    assert got.shape == want.shape
    d = np.abs(got - want)
    tol = atol + rtol * np.abs(want)
    ex = d - tol
    ex = np.where(np.isnan(ex), np.inf, ex)
    i = int(np.argmax(ex))
    return float(ex[i]), i, float(got[i]), float(want[i])


def normwise_rel_err(got: np.ndarray, want64: np.ndarray) -> float:
    """max |y - y_hat| / max |y_hat|, the 1e-3 precision gate against fp64."""
    got = np.asarray(got, np.float64)
    want64 = np.asarray(want64, np.float64)
    den = float(np.max(np.abs(want64))) if want64.size else 0.0
    num = float(np.max(np.abs(got - want64))) if want64.size else 0.0
    if not np.all(np.isfinite(got)):
        return float("inf")
    return num / den if den > 0 else num


# ----------------------------------------------------- known answers --

def gemv_case(m: int, n: int, k: int, flags: int, bias: bool, x_scale: float = 1.0, wt: int = BF16) -> dict:
    """Inputs and expected output of KernelTests.gemvCase (KernelTests.swift:72-103).

    Draw order from one LCG seeded m*1000 + n*7 + k: x (m*k, scale x_scale), w (n*k, 0.1),
    w2 (n*k, 0.1), b (n), y0 (m*n).  Weights and bias are rounded to ``wt`` (the reference
    uses bf16); x stays fp32.  ``x`` carries 8 extra NaN rows the kernel must never read."""
    rng = LCG(m * 1000 + n * 7 + k)
    x = rng.floats(m * k, x_scale)
    w = rng.floats(n * k, 0.1)
    w2 = rng.floats(n * k, 0.1)
    b = rng.floats(n)
    y0 = rng.floats(m * n)
    wb, _ = round16(w, wt)
    w2b, _ = round16(w2, wt)
    bb, _ = round16(b, wt)
    xs = np.concatenate([x, np.full(8 * k, np.nan, np.float32)]).reshape(m + 8, k)
    gated = bool(flags & SILU_GATE)
    want = linear_f32(xs[:m], wb.reshape(n, k), w2b.reshape(n, k) if gated else None, wt,
                      bb if bias else None, y0.reshape(m, n), m, n, k, flags)
    return dict(m=m, n=n, k=k, flags=flags | (BIAS if bias else 0), x=xs, w=wb.reshape(n, k),
                w2=w2b.reshape(n, k), bias=bb if bias else None, y0=y0.reshape(m, n), want=want, wt=wt)


# Linear known-answer cases of the reference (KernelTests.swift:127-183), (m, n, k, flags, bias, xScale).
KAT_GEMV_SHAPES = [  # testGemvShapes, KernelTests.swift:127-137
    (1, 1152, 896, 0, True, 1.0), (2, 2, 896, 0, True, 1.0), (4, 896, 4864, ACCUM, False, 1.0),
    (6, 4096, 1024, GELU, True, 1.0), (3, 64, 1024, 0, True, 1.0), (21, 300, 896, 0, False, 1.0),
    (4, 3530, 896, 0, True, 1.0), (1, 896, 64, 0, True, 1.0), (8, 2, 896, 0, True, 1.0),
]
KAT_GEMM8_TILES = [  # testGemm8ColumnTiles, KernelTests.swift:142-160
    (6, 1024, 1024, GELU, True, 1.0), (4, 896, 896, SILU_GATE, False, 1.0), (3, 1152, 896, ACCUM, False, 1.0),
    (6, 1024, 4096, ACCUM, False, 1.0), (4, 896, 4864, ACCUM, False, 1.0),
]
KAT_GEMM_PREFILL = [  # testGemmPrefillShapes, KernelTests.swift:164-172
    (174, 1152, 896, 0, True, 1.0), (40, 896, 4864, ACCUM, False, 1.0), (33, 4864, 896, SILU_GATE, False, 1.0),
    (16, 64, 32, GELU, True, 1.0), (65, 128, 64, SILU, True, 1.0),
]
KAT_LARGE_INPUTS = [  # testGemvGeluLargeInputs, KernelTests.swift:175-178
    (6, 256, 1024, GELU, True, 8.0), (1, 256, 896, SILU, False, 8.0),
]
KAT_SILU_GATE = [  # testGemvSiluGate, KernelTests.swift:180-183
    (1, 4864, 896, SILU_GATE, False, 1.0), (5, 256, 896, SILU_GATE, False, 1.0),
]
KAT_ALL = KAT_GEMV_SHAPES + KAT_GEMM8_TILES + KAT_GEMM_PREFILL + KAT_LARGE_INPUTS + KAT_SILU_GATE


# ------------------------------------------------- rope and attention --

def inv_freq(theta: float = 1e6, dim: int = 64) -> np.ndarray:
    """1 / theta^(2i / dim) in fp32 as the reference builds it (Qwen.swift:60)."""
    i = np.arange(dim // 2, dtype=np.float32)
    return (np.float32(1.0) / np.power(np.float32(theta), np.float32(2.0) * i / np.float32(dim))).astype(np.float32)


def rope_neox(v: np.ndarray, pos, invf: np.ndarray, fp32_angle: bool = True) -> np.ndarray:
    """NeoX rotation of 64-wide heads, pairs (i, i + 32), angle pos * inv_freq[i]
    (Shaders.swift:472-478; KernelTests.swift:207-217).  The angle is formed in fp32 as the
    reference forms it (``float(pos) * invFreq[i]``); cos, sin and the rotation are fp64.
    v: [..., 64]."""
    v = np.asarray(v, np.float64)
    if fp32_angle:
        a = (np.asarray(pos, np.float32)[..., None] * invf.astype(np.float32)).astype(np.float64)
    else:
        a = np.asarray(pos, np.float64)[..., None] * invf.astype(np.float64)
    c, s = np.cos(a), np.sin(a)
    x0, x1 = v[..., :32], v[..., 32:]
    return np.concatenate([x0 * c - x1 * s, x1 * c + x0 * s], axis=-1)


def attention_f64(q: np.ndarray, k: np.ndarray, v: np.ndarray, qpos: int, window: int, scale: float) -> np.ndarray:
    """Causal attention of one query row (hq heads of 64) over keys [start, qpos] of a
    cache k, v: [hkv, >= qpos + 1, 64]; start = max(0, qpos + 1 - window) (window 0 =
    all); GQA kv head = h // (hq // hkv) (Shaders.swift:511-520).  fp64.  Returns [hq, 64]."""
    hq = q.shape[0]
    hkv = k.shape[0]
    start = qpos + 1 - window if (window > 0 and qpos + 1 > window) else 0
    out = np.zeros((hq, 64), np.float64)
    for h in range(hq):
        kvh = h // (hq // hkv)
        kk = k[kvh, start:qpos + 1].astype(np.float64)
        vv = v[kvh, start:qpos + 1].astype(np.float64)
        s = kk @ q[h].astype(np.float64) * scale
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ vv
    return out


# ---------------------------------------------------- DiT flow step --

def rope_interleaved(v: np.ndarray, pos, invf: np.ndarray) -> np.ndarray:
    """x_transformers interleaved rotary of 64-wide heads: pairs (2p, 2p + 1), angle pos *
    inv_freq[p], formed in fp32 as the reference forms it (Shaders.swift:605-608, 627;
    KernelTests.swift:291-300); cos, sin and the rotation in fp64.  v: [..., 64]."""
    v = np.asarray(v, np.float64)
    a = (np.asarray(pos, np.float32)[..., None] * invf.astype(np.float32)).astype(np.float64)
    c, s = np.cos(a), np.sin(a)
    x, y = v[..., 0::2], v[..., 1::2]
    out = np.empty_like(v)
    out[..., 0::2] = x * c - y * s
    out[..., 1::2] = y * c + x * s
    return out


def dit_attention_f64(qkv: np.ndarray, B: int, S: int, H: int, invf: np.ndarray, scale: float = 0.125) -> np.ndarray:
    """Full (non-causal) attention inside each of B sequences of S rows (Shaders.swift:612-648,
    KernelTests.swift:301-316): qkv rows [q | k | v] of H heads; q and k of row i rotated at
    position i; max-subtracted softmax of q.k * scale over the sequence's S keys; out = sum p v.
    fp64.  Returns [B * S, H * 64]."""
    D = H * 64
    qkv = np.asarray(qkv, np.float64)
    out = np.zeros((B * S, D), np.float64)
    pos = np.arange(S)
    for b in range(B):
        rows = qkv[b * S:(b + 1) * S]
        for h in range(H):
            q = rope_interleaved(rows[:, h * 64:(h + 1) * 64], pos, invf)
            k = rope_interleaved(rows[:, D + h * 64:D + (h + 1) * 64], pos, invf)
            v = rows[:, 2 * D + h * 64:2 * D + (h + 1) * 64]
            sc = q @ k.T * scale
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            out[b * S:(b + 1) * S, h * 64:(h + 1) * 64] = (p / p.sum(axis=1, keepdims=True)) @ v
    return out


def flow_assemble_f64(y, history, cemb, cbias_bits, temb, xw_bits, xb_bits, wt: int) -> np.ndarray:
    """The six flow-input rows (Shaders.swift:650-676): row r, slot r % 3 = 0: temb + cemb
    (rows 0-2) or temb + the cond embedder's bias (rows 3-5); 1: x_b + x_w history; 2: x_b +
    x_w y.  16-bit weights decoded exactly; fp64 sums.  Returns [6, hidden]."""
    w = decode16(xw_bits, wt).astype(np.float64)
    b = decode16(xb_bits, wt).astype(np.float64)
    cb = decode16(cbias_bits, wt).astype(np.float64)
    t = np.asarray(temb, np.float64)
    rows = [t + np.asarray(cemb, np.float64), b + w @ np.asarray(history, np.float64), b + w @ np.asarray(y, np.float64)]
    rows += [t + cb, rows[1], rows[2]]
    return np.stack(rows)


def flow_euler_f64(y, pred, pred_row: int, null_row: int, cfg: float, dt: float):
    """The CFG Euler step of the flow sampler (Shaders.swift:678-693): c = pred[pred_row], u =
    pred[null_row]; y + (c + (c - u) cfg) dt, and the capture [c, u].  fp64."""
    c = np.asarray(pred[pred_row], np.float64)
    u = np.asarray(pred[null_row], np.float64)
    return np.asarray(y, np.float64) + (c + (c - u) * cfg) * dt, np.concatenate([c, u])


# ------------------------------------------------ flow schedule --

# EPSS base timesteps in 32nds per step count, DiT.swift:58-62.
EPSS_32NDS = {
    5: (0, 2, 4, 8, 16, 32), 6: (0, 2, 4, 6, 8, 16, 32), 7: (0, 2, 4, 6, 8, 16, 24, 32),
    10: (0, 2, 4, 6, 8, 12, 16, 20, 24, 28, 32), 12: (0, 2, 4, 6, 8, 10, 12, 14, 16, 20, 24, 28, 32),
    16: (0, 1, 2, 3, 4, 5, 6, 7, 8, 10, 12, 14, 16, 20, 24, 28, 32),
}


def flow_timesteps_f64(steps: int) -> np.ndarray:
    """FlowSchedule.timesteps (DiT.swift:57-65) in fp64 closed form: the sway -1 map
    t - (cos(pi/2 t) - 1 + t) equals 1 - cos(pi/2 t), applied to the EPSS grid for the
    listed step counts and to the uniform grid k / steps otherwise."""
    if steps in EPSS_32NDS:
        base = np.asarray(EPSS_32NDS[steps], np.float64) / 32.0
    else:
        base = np.arange(steps + 1, dtype=np.float64) / steps
    return 1.0 - np.cos(np.pi / 2 * base)


def sinusoid_f64(t: float, width: int = 256, scale: float = 1000.0) -> np.ndarray:
    """FlowSchedule.sinusoid (DiT.swift:67-79) in fp64: [sin(a_i), cos(a_i)] for
    a_i = scale t exp(-i ln(1e4) / (width/2 - 1)), i < width / 2."""
    half = width // 2
    a = scale * float(t) * np.exp(-np.arange(half, dtype=np.float64) * math.log(10000.0) / (half - 1))
    return np.concatenate([np.sin(a), np.cos(a)])


def time_mlp_f64(sinus, w1, b1, w2, b2, wt: int) -> np.ndarray:
    """The time MLP of precomputeTimeEmbeddings (Engine.swift:186-198) on given sinusoid rows:
    SiLU(x W1^T + b1) into an fp32 buffer, then W2^T + b2; fp64 per op.  Returns float64."""
    mid = linear_np64(np.asarray(sinus, np.float64), w1, None, wt, b1, None, BIAS | SILU).astype(np.float32)
    return linear_np64(mid, w2, None, wt, b2, None, BIAS)


# --------------------------------------------------------- VAE tail --

def upsample4_f64(prev, cur, nxt) -> np.ndarray:
    """The four frames of a latent (Shaders.swift:700-718): torch's linear x4 upsample weights
    with an absent neighbour (None) clamped to cur.  fp64.  Returns [4, hidden]."""
    c = np.asarray(cur, np.float64)
    p = c if prev is None else np.asarray(prev, np.float64)
    n = c if nxt is None else np.asarray(nxt, np.float64)
    return np.stack([0.625 * c + 0.375 * p, 0.875 * c + 0.125 * p, 0.875 * c + 0.125 * n, 0.625 * c + 0.375 * n])


def istft_frame_f64(row, nfft: int, window) -> np.ndarray:
    """One synthesis frame (Shaders.swift:720-759, KernelTests.swift:361-374): bins k <=
    nfft / 2 of magnitude min(e^row[k], 100) and phase row[bins + k]; the real inverse DFT
    with 1 / nfft scaling (the imaginary parts of bins 0 and nfft / 2 drop out), times the
    window.  fp64."""
    bins = nfft // 2 + 1
    row = np.asarray(row, np.float64)
    mag = np.minimum(np.exp(row[:bins]), 100.0)
    spec = mag * np.exp(1j * row[bins:2 * bins])
    return np.fft.irfft(spec, n=nfft) * np.asarray(window, np.float64)


def istft_emit_f64(frames, window, nfft: int, hop: int, s0: int, count: int, last_frame: int) -> np.ndarray:
    """Overlap-add of frames[0 .. last_frame] (KernelTests.swift:375-380, Shaders.swift:761-787):
    out[i] for s = s0 + i + (nfft - hop) / 2 is the sum of frame f's sample s - f hop over the
    frames covering s, divided by the sum of window^2 there.  fp64."""
    pad = (nfft - hop) // 2
    w2 = np.asarray(window, np.float64) ** 2
    out = np.zeros(count, np.float64)
    for i in range(count):
        s = s0 + i + pad
        acc = env = 0.0
        for f in range(0, last_frame + 1):
            t = s - f * hop
            if 0 <= t < nfft:
                acc += frames[f][t]
                env += w2[t]
        out[i] = acc / env
    return out
