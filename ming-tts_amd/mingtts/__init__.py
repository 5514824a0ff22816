"""Python binding of libmingtts_hip.so (the gfx950 linear hot path of MingTTS).

The library is the product; this module only loads it with ctypes and forwards
device pointers.  It raises if the library is missing: there is no CPU fallback.

The classes ``Linear``, ``ActView``, ``GemvFlags`` and ``Encoder`` mirror the
reference's operator layer (Sources/MingTTS/Engine/Kernels.swift:7-44, 128-206) so
callers and tests read like the reference's own: ``Encoder.linear(x, rows, linear, y,
flags, gate)`` forwards to ``mt_linear`` with the same argument meaning.  Tensors are
torch device tensors (plumbing for memory and streams only).
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from typing import Optional, Sequence

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.normpath(os.path.join(_HERE, "..", "csrc", "libmingtts_hip.so"))

F32, F16, BF16 = 0, 1, 2
OK, EHIP, ENOMEM, EINVAL, ERANGE, ENOTSUP = 0, -5, -12, -22, -34, -95
KERNEL_GEMV, KERNEL_GEMM, KERNEL_GEMV_MFMA = 1, 2, 3
(TUNE_GEMV_ROWS_MAX, TUNE_GEMV_LANES, TUNE_GEMM_SPLITK, TUNE_SEQ_GROUPS, TUNE_SEQ_LAUNCH, TUNE_GEMM_TILE,
 TUNE_GEMM_STAGES, TUNE_GEMV_MFMA, TUNE_SEQ_LAYER) = 1, 2, 3, 4, 5, 6, 7, 8, 9
SEQ_GENERAL, SEQ_DECODE_LAYER, SEQ_DIT_BLOCK = 0, 1, 2

# Every symbol include/mingtts_hip.h declares.
EXPORTS = (
    "mt_linear", "mt_linear_static", "mt_linear_rmsnorm", "mt_rmsnorm", "mt_linear_kernel", "mt_set_tuning", "mt_seq_create",
    "mt_seq_create_items", "mt_seq_run",
    "mt_seq_destroy", "mt_seq_groups", "mt_seq_kernel", "mt_seq_check", "mt_rope_cache", "mt_rope_cache_decode",
    "mt_attention", "mt_attention_decode", "mt_rope_attention", "mt_dit_attention", "mt_dit_attention_linear", "mt_flow_assemble",
    "mt_flow_euler", "mt_flow_euler_assemble",
    "mt_upsample4", "mt_istft_frames", "mt_istft_emit", "mt_st_open", "mt_st_close", "mt_st_count", "mt_st_name", "mt_st_find", "mt_arena_create", "mt_arena_tensor",
    "mt_arena_padded", "mt_arena_bytes", "mt_arena_upload", "mt_arena_audit", "mt_arena_destroy",
    "mt_last_error", "mt_version",
)


class GemvFlags:
    """GemvFlags, Kernels.swift:21-28."""
    bias = 1
    accumulate = 2
    gelu = 4
    siluGate = 8
    silu = 16


class MingTTSError(RuntimeError):
    """An error code returned by the library, with mt_last_error()'s text."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class GemvParams(ctypes.Structure):
    """mt_gemv_params == GemvParams (Shaders.swift:39)."""
    _fields_ = [("M", ctypes.c_uint32), ("N", ctypes.c_uint32), ("K", ctypes.c_uint32),
                ("ldx", ctypes.c_uint32), ("ldy", ctypes.c_uint32), ("flags", ctypes.c_uint32),
                ("eps", ctypes.c_float)]


class LinearOp(ctypes.Structure):
    """mt_linear_op: one op of a persistent sequence."""
    _fields_ = [("x", ctypes.c_void_p), ("w", ctypes.c_void_p), ("w2", ctypes.c_void_p),
                ("bias", ctypes.c_void_p), ("norm", ctypes.c_void_p), ("y", ctypes.c_void_p),
                ("p", GemvParams), ("xt", ctypes.c_int32), ("wt", ctypes.c_int32)]


class AttnOp(ctypes.Structure):
    """mt_attn_op: the decode attention of one layer as an item of a sequence."""
    _fields_ = [("qkv", ctypes.c_void_p), ("ldq", ctypes.c_uint32), ("B", ctypes.c_uint32),
                ("hq", ctypes.c_uint32), ("hkv", ctypes.c_uint32), ("pos", ctypes.c_void_p),
                ("k_cache", ctypes.c_void_p), ("v_cache", ctypes.c_void_p), ("cache_t", ctypes.c_int32),
                ("cache_len", ctypes.c_uint32), ("cache_stride", ctypes.c_uint64), ("inv_freq", ctypes.c_void_p),
                ("out", ctypes.c_void_p), ("ldo", ctypes.c_uint32), ("window", ctypes.c_uint32),
                ("scale", ctypes.c_float)]


class DitAttnOp(ctypes.Structure):
    """mt_dit_attn_op: the DiT's full attention (mt_dit_attention) as an item of a sequence."""
    _fields_ = [("qkv", ctypes.c_void_p), ("ldq", ctypes.c_uint32), ("B", ctypes.c_uint32), ("S", ctypes.c_uint32),
                ("H", ctypes.c_uint32), ("inv_freq", ctypes.c_void_p), ("out", ctypes.c_void_p),
                ("ldo", ctypes.c_uint32), ("scale", ctypes.c_float)]


SEQ_LINEAR, SEQ_ATTENTION, SEQ_DIT_ATTENTION = 0, 1, 2


class SeqItem(ctypes.Structure):
    """mt_seq_item: a linear, a decode attention or a DiT attention item of a sequence."""
    _fields_ = [("kind", ctypes.c_int32), ("linear", LinearOp), ("attn", AttnOp), ("dit", DitAttnOp)]


class StEntry(ctypes.Structure):
    """mt_st_entry: one tensor of a .safetensors file."""
    _fields_ = [("dtype", ctypes.c_int32), ("ndim", ctypes.c_uint32), ("shape", ctypes.c_uint64 * 8),
                ("bytes", ctypes.c_uint64), ("host", ctypes.c_void_p)]


_lib: Optional[ctypes.CDLL] = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Loads libmingtts_hip.so (raises if it is not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"libmingtts_hip.so is not built at {path}; run __graft_entry__.build()")
    L = ctypes.CDLL(path)
    vp, u32, u64, i32, f32 = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int, ctypes.c_float
    L.mt_linear.argtypes = [vp, i32, vp, vp, i32, vp, vp, GemvParams, vp]
    L.mt_linear.restype = i32
    L.mt_linear_static.argtypes = [vp, i32, vp, vp, i32, vp, vp, GemvParams, vp]
    L.mt_linear_static.restype = i32
    L.mt_linear_rmsnorm.argtypes = [vp, i32, vp, vp, vp, i32, vp, vp, GemvParams, vp]
    L.mt_linear_rmsnorm.restype = i32
    L.mt_rmsnorm.argtypes = [vp, u32, u32, u32, vp, i32, vp, u32, f32, vp]
    L.mt_rmsnorm.restype = i32
    L.mt_linear_kernel.argtypes = [u32, u32, u32, i32, i32]
    L.mt_linear_kernel.restype = i32
    L.mt_set_tuning.argtypes = [i32, i32]
    L.mt_set_tuning.restype = i32
    L.mt_seq_create.argtypes = [ctypes.POINTER(LinearOp), u32, ctypes.POINTER(vp)]
    L.mt_seq_create.restype = i32
    L.mt_seq_create_items.argtypes = [ctypes.POINTER(SeqItem), u32, ctypes.POINTER(vp)]
    L.mt_seq_create_items.restype = i32
    L.mt_seq_run.argtypes = [vp, vp]
    L.mt_seq_run.restype = i32
    L.mt_seq_destroy.argtypes = [vp]
    L.mt_seq_destroy.restype = i32
    L.mt_seq_groups.argtypes = [vp]
    L.mt_seq_groups.restype = i32
    L.mt_seq_kernel.argtypes = [vp]
    L.mt_seq_kernel.restype = i32
    L.mt_seq_check.argtypes = [vp]
    L.mt_seq_check.restype = i32
    L.mt_rope_cache.argtypes = [vp, u32, u32, u32, u32, u32, vp, vp, i32, u32, vp, vp]
    L.mt_rope_cache.restype = i32
    L.mt_rope_cache_decode.argtypes = [vp, u32, u32, u32, u32, vp, vp, vp, i32, u32, u64, vp, vp]
    L.mt_rope_cache_decode.restype = i32
    L.mt_attention.argtypes = [vp, u32, u32, u32, u32, u32, u32, vp, vp, i32, u32, vp, u32, f32, vp]
    L.mt_rope_attention.argtypes = [vp, u32, u32, u32, u32, u32, u32, vp, vp, i32, u32, vp, vp, u32, f32, vp]
    L.mt_rope_attention.restype = i32
    L.mt_attention.restype = i32
    L.mt_attention_decode.argtypes = [vp, u32, u32, u32, u32, vp, u32, vp, vp, i32, u32, u64, vp, u32, f32, vp]
    L.mt_attention_decode.restype = i32
    L.mt_dit_attention.argtypes = [vp, u32, u32, u32, u32, vp, vp, u32, f32, vp]
    L.mt_dit_attention.restype = i32
    L.mt_dit_attention_linear.argtypes = [vp, u32, u32, u32, vp, f32, vp, i32, vp, vp, GemvParams, vp]
    L.mt_dit_attention_linear.restype = i32
    L.mt_flow_assemble.argtypes = [vp, vp, vp, vp, vp, vp, vp, i32, vp, u32, u32, u32, vp]
    L.mt_flow_assemble.restype = i32
    L.mt_flow_euler.argtypes = [vp, vp, u32, u32, u32, vp, u32, f32, f32, vp]
    L.mt_flow_euler.restype = i32
    L.mt_flow_euler_assemble.argtypes = [vp, vp, u32, u32, u32, vp, f32, f32, vp, vp, vp, vp, vp, vp, i32, vp, u32, u32,
                                         u32, vp]
    L.mt_flow_euler_assemble.restype = i32
    L.mt_upsample4.argtypes = [vp, vp, vp, vp, u32, u32, vp]
    L.mt_upsample4.restype = i32
    L.mt_istft_frames.argtypes = [vp, u32, u32, u32, vp, vp, vp, u32, u32, vp]
    L.mt_istft_frames.restype = i32
    L.mt_istft_emit.argtypes = [vp, vp, u32, u32, u32, u32, u32, u32, vp, vp]
    L.mt_istft_emit.restype = i32
    cp = ctypes.c_char_p
    L.mt_st_open.argtypes = [cp, ctypes.POINTER(vp)]
    L.mt_st_open.restype = i32
    L.mt_st_close.argtypes = [vp]
    L.mt_st_close.restype = i32
    L.mt_st_count.argtypes = [vp]
    L.mt_st_count.restype = i32
    L.mt_st_name.argtypes = [vp, u32, ctypes.POINTER(cp)]
    L.mt_st_name.restype = i32
    L.mt_st_find.argtypes = [vp, cp, ctypes.POINTER(StEntry)]
    L.mt_st_find.restype = i32
    L.mt_arena_create.argtypes = [vp, i32, ctypes.POINTER(vp)]
    L.mt_arena_create.restype = i32
    L.mt_arena_tensor.argtypes = [vp, ctypes.POINTER(cp), u32, ctypes.POINTER(u64), ctypes.POINTER(u64)]
    L.mt_arena_tensor.restype = i32
    L.mt_arena_padded.argtypes = [vp, cp, u32, u32, u32, ctypes.POINTER(u64)]
    L.mt_arena_padded.restype = i32
    L.mt_arena_bytes.argtypes = [vp]
    L.mt_arena_bytes.restype = u64
    L.mt_arena_upload.argtypes = [vp, vp, vp]
    L.mt_arena_upload.restype = i32
    L.mt_arena_audit.argtypes = [vp, ctypes.POINTER(u64), ctypes.POINTER(u64)]
    L.mt_arena_audit.restype = i32
    L.mt_arena_destroy.argtypes = [vp]
    L.mt_arena_destroy.restype = i32
    L.mt_last_error.argtypes = []
    L.mt_last_error.restype = ctypes.c_char_p
    L.mt_version.argtypes = []
    L.mt_version.restype = ctypes.c_char_p
    _lib = L
    return L


def last_error() -> str:
    return load().mt_last_error().decode()


def check(rc: int) -> int:
    if rc < 0:
        raise MingTTSError(rc, last_error())
    return rc


def _ptr(t) -> Optional[int]:
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _stream(stream) -> Optional[int]:
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def dtype_code(t) -> int:
    import torch
    return {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}[t.dtype]


# ------------------------------------------------------------ raw calls --

def linear_raw(x, xt, w, w2, wt, bias, y, M, N, K, ldx, ldy, flags, stream=None) -> int:
    """mt_linear on raw pointers / tensors; returns the raw return code."""
    p = GemvParams(M, N, K, ldx, ldy, flags, 0.0)
    return load().mt_linear(_ptr(x), xt, _ptr(w), _ptr(w2), wt, _ptr(bias), _ptr(y), p, _stream(stream))


def linear_static_raw(x, xt, w, w2, wt, bias, y, M, N, K, ldx, ldy, flags, stream=None) -> int:
    """mt_linear_static on raw pointers / tensors; returns the raw return code."""
    p = GemvParams(M, N, K, ldx, ldy, flags, 0.0)
    return load().mt_linear_static(_ptr(x), xt, _ptr(w), _ptr(w2), wt, _ptr(bias), _ptr(y), p, _stream(stream))


def linear_rmsnorm_raw(x, xt, norm, w, w2, wt, bias, y, M, N, K, ldx, ldy, flags, eps=1e-6, stream=None) -> int:
    """mt_linear_rmsnorm on raw pointers / tensors; returns the raw return code."""
    p = GemvParams(M, N, K, ldx, ldy, flags, eps)
    return load().mt_linear_rmsnorm(_ptr(x), xt, _ptr(norm), _ptr(w), _ptr(w2), wt, _ptr(bias), _ptr(y), p,
                                    _stream(stream))


def linear(x, w, y, M=None, flags=0, w2=None, bias=None, ldx=None, ldy=None, norm=None, eps=1e-6,
           stream=None) -> None:
    """y[:M] (op)= x[:M] @ w.T with the epilogue in ``flags``; torch tensors, w: [N, K].
    With ``norm`` (gain [K]) x is RMS-normalised first (mt_linear_rmsnorm)."""
    N, K = w.shape
    M = x.shape[0] if M is None else M
    ldx = x.stride(0) if ldx is None else ldx
    ldy = y.stride(0) if ldy is None else ldy
    if norm is not None:
        check(linear_rmsnorm_raw(x, dtype_code(x), norm, w, w2, dtype_code(w), bias, y, M, N, K, ldx, ldy, flags,
                                 eps, stream))
    else:
        check(linear_raw(x, dtype_code(x), w, w2, dtype_code(w), bias, y, M, N, K, ldx, ldy, flags, stream))


def rmsnorm_raw(x, ldx, rows, width, g, wt, y, ldy, eps=1e-6, stream=None) -> int:
    """mt_rmsnorm on raw pointers / tensors; returns the raw return code."""
    return load().mt_rmsnorm(_ptr(x), ldx, rows, width, _ptr(g), wt, _ptr(y), ldy, eps, _stream(stream))


def rmsnorm(x, g, y, rows=None, eps=1e-6, stream=None) -> None:
    """y[:rows] = x[:rows] * rsqrt(mean(x^2) + eps) * g (mt_rmsnorm); torch tensors, g [width]."""
    rows = x.shape[0] if rows is None else rows
    check(rmsnorm_raw(x, x.stride(0), rows, g.shape[0], g, dtype_code(g), y, y.stride(0), eps, stream))


def linear_kernel(M, N, K, xt=F32, wt=BF16) -> int:
    return load().mt_linear_kernel(M, N, K, xt, wt)


def set_tuning(key: int, value: int) -> int:
    return check(load().mt_set_tuning(key, value))


class Seq:
    """A persistent sequence plan (mt_seq_*) of linears (``LinearOp``) and, optionally,
    decode attention items (``AttnOp``) or DiT attention items (``DitAttnOp``)."""

    def __init__(self, ops: Sequence):
        h = ctypes.c_void_p()
        if all(isinstance(o, LinearOp) for o in ops):
            arr = (LinearOp * len(ops))(*ops)
            check(load().mt_seq_create(arr, len(ops), ctypes.byref(h)))
        else:
            items = (SeqItem * len(ops))()
            for i, o in enumerate(ops):
                if isinstance(o, AttnOp):
                    items[i].kind = SEQ_ATTENTION
                    items[i].attn = o
                elif isinstance(o, DitAttnOp):
                    items[i].kind = SEQ_DIT_ATTENTION
                    items[i].dit = o
                else:
                    items[i].kind = SEQ_LINEAR
                    items[i].linear = o
            check(load().mt_seq_create_items(items, len(ops), ctypes.byref(h)))
        self.handle = h
        self.n_ops = len(ops)

    def run(self, stream=None) -> None:
        check(load().mt_seq_run(self.handle, _stream(stream)))

    def check(self) -> None:
        check(load().mt_seq_check(self.handle))

    @property
    def groups(self) -> int:
        return check(load().mt_seq_groups(self.handle))

    @property
    def kernel(self) -> int:
        """SEQ_DECODE_LAYER when the plan runs the kernel specialised for Qwen2-0.5B decode
        layers, SEQ_DIT_BLOCK for the flow head's DiT blocks, else SEQ_GENERAL."""
        return check(load().mt_seq_kernel(self.handle))

    def close(self) -> None:
        if self.handle:
            load().mt_seq_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def op(x, w, y, M, flags=0, w2=None, bias=None, ldx=None, ldy=None, xt=None, wt=None, norm=None,
       eps=1e-6) -> LinearOp:
    """An mt_linear_op over torch tensors (w: [N, K]); ``norm`` fuses an RMSNorm prologue."""
    N, K = w.shape
    if bias is not None:
        flags |= GemvFlags.bias
    return LinearOp(_ptr(x), _ptr(w), _ptr(w2), _ptr(bias), _ptr(norm), _ptr(y),
                    GemvParams(M, N, K, x.stride(0) if ldx is None else ldx, y.stride(0) if ldy is None else ldy,
                               flags, eps if norm is not None else 0.0),
                    dtype_code(x) if xt is None else xt, dtype_code(w) if wt is None else wt)


def dit_attn_op(qkv, B, S, H, inv_freq, out, ldq=None, ldo=None, scale=0.125) -> DitAttnOp:
    """An mt_dit_attn_op over torch tensors: B sequences of S rows of qkv ([B S, 3 H 64] at
    stride ldq), out [B S, H 64]."""
    return DitAttnOp(_ptr(qkv), qkv.stride(0) if ldq is None else ldq, B, S, H, _ptr(inv_freq), _ptr(out),
                     out.stride(0) if ldo is None else ldo, scale)


def attn_op(qkv, B, hq, hkv, pos, kc, vc, cache_len, cache_stride, inv_freq, out, ldq=None, ldo=None,
            window=0, scale=0.125) -> AttnOp:
    """An mt_attn_op over torch tensors: rows b < B of qkv ([B, (hq + 2 hkv) 64] at stride
    ldq), positions pos (device uint32/int32 [B]), caches kc / vc ([B, hkv, cache_len, 64]
    at cache_stride elements per row), out [B, hq 64]."""
    return AttnOp(_ptr(qkv), qkv.stride(0) if ldq is None else ldq, B, hq, hkv, _ptr(pos), _ptr(kc), _ptr(vc),
                  dtype_code(kc), cache_len, cache_stride, _ptr(inv_freq), _ptr(out),
                  out.stride(0) if ldo is None else ldo, window, scale)


def rope_cache(qkv, ldq, M, hq, hkv, pos0, kc, vc, cache_len, inv_freq, stream=None) -> None:
    check(load().mt_rope_cache(_ptr(qkv), ldq, M, hq, hkv, pos0, _ptr(kc), _ptr(vc), dtype_code(kc), cache_len,
                               _ptr(inv_freq), _stream(stream)))


def rope_cache_decode(qkv, ldq, B, hq, hkv, pos, kc, vc, cache_len, cache_stride, inv_freq, stream=None) -> None:
    check(load().mt_rope_cache_decode(_ptr(qkv), ldq, B, hq, hkv, _ptr(pos), _ptr(kc), _ptr(vc), dtype_code(kc),
                                      cache_len, cache_stride, _ptr(inv_freq), _stream(stream)))


def attention(q, ldq, M, hq, hkv, pos0, window, kc, vc, cache_len, out, ldo, scale=0.125, stream=None) -> None:
    check(load().mt_attention(_ptr(q), ldq, M, hq, hkv, pos0, window, _ptr(kc), _ptr(vc), dtype_code(kc),
                              cache_len, _ptr(out), ldo, scale, _stream(stream)))


def rope_attention(qkv, ldq, M, hq, hkv, pos0, window, kc, vc, cache_len, inv_freq, out, ldo, scale=0.125,
                   stream=None) -> None:
    """rope_cache then attention over the same M rows in one launch (mt_rope_attention)."""
    check(load().mt_rope_attention(_ptr(qkv), ldq, M, hq, hkv, pos0, window, _ptr(kc), _ptr(vc), dtype_code(kc),
                                   cache_len, _ptr(inv_freq), _ptr(out), ldo, scale, _stream(stream)))


def attention_decode(q, ldq, B, hq, hkv, lens, window, kc, vc, cache_len, cache_stride, out, ldo, scale=0.125,
                     stream=None) -> None:
    check(load().mt_attention_decode(_ptr(q), ldq, B, hq, hkv, _ptr(lens), window, _ptr(kc), _ptr(vc),
                                     dtype_code(kc), cache_len, cache_stride, _ptr(out), ldo, scale,
                                     _stream(stream)))


def dit_attention(qkv, B, S, H, inv_freq, out, ld=None, ldo=None, scale=0.125, stream=None) -> None:
    """Encoder.ditAttention: full attention with interleaved RoPE inside each of B sequences
    of S rows (Kernels.swift:208-220)."""
    check(load().mt_dit_attention(_ptr(qkv), qkv.stride(0) if ld is None else ld, B, S, H, _ptr(inv_freq), _ptr(out),
                                  out.stride(0) if ldo is None else ldo, scale, _stream(stream)))


def dit_attention_linear(qkv, B, S, H, inv_freq, w, y, flags=0, bias=None, scale=0.125, ldq=None, ldy=None,
                         stream=None) -> None:
    """Encoder.ditAttention then Encoder.linear of its output (DiT.swift:44-45) in one launch:
    y[:B S] (op)= dit_attention(qkv) @ w.T with the epilogue in ``flags``; w: [N, 64 H]."""
    N, K = w.shape
    p = GemvParams(B * S, N, K, qkv.stride(0) if ldq is None else ldq, y.stride(0) if ldy is None else ldy, flags, 0.0)
    check(load().mt_dit_attention_linear(_ptr(qkv), B, S, H, _ptr(inv_freq), scale, _ptr(w), dtype_code(w), _ptr(bias),
                                         _ptr(y), p, _stream(stream)))


def flow_assemble(y, history, cemb, cond_bias, temb, x_w, x_b, x, ldx=None, stream=None) -> None:
    """Encoder.flowAssemble: the six flow-input rows (Kernels.swift:222-235); x_w [hidden,
    latent_dim] of the weights' 16-bit type."""
    hidden, latent = x_w.shape
    check(load().mt_flow_assemble(_ptr(y), _ptr(history), _ptr(cemb), _ptr(cond_bias), _ptr(temb), _ptr(x_w),
                                  _ptr(x_b), dtype_code(x_w), _ptr(x), x.stride(0) if ldx is None else ldx, hidden,
                                  latent, _stream(stream)))


def flow_euler(y, pred, pred_row, null_row, cfg, dt, capture=None, ldp=None, stream=None) -> None:
    """Encoder.flowEuler: y += (c + (c - u) cfg) dt with c, u rows of pred (Kernels.swift:237-246)."""
    latent = y.numel()
    check(load().mt_flow_euler(_ptr(y), _ptr(pred), pred.stride(0) if ldp is None else ldp, pred_row, null_row,
                               _ptr(capture), latent, cfg, dt, _stream(stream)))


def flow_euler_assemble(y, pred, pred_row, null_row, cfg, dt, history, cemb, cond_bias, temb, x_w, x_b, x,
                        capture=None, ldp=None, ldx=None, stream=None) -> None:
    """flow_euler of one ODE step then flow_assemble of the next, in one launch."""
    hidden, latent = x_w.shape
    check(load().mt_flow_euler_assemble(_ptr(y), _ptr(pred), pred.stride(0) if ldp is None else ldp, pred_row, null_row,
                                        _ptr(capture), cfg, dt, _ptr(history), _ptr(cemb), _ptr(cond_bias), _ptr(temb),
                                        _ptr(x_w), _ptr(x_b), dtype_code(x_w), _ptr(x),
                                        x.stride(0) if ldx is None else ldx, hidden, latent, _stream(stream)))


def upsample4(prev, cur, nxt, frames, ldf=None, stream=None) -> None:
    """Encoder.upsample4 (Kernels.swift:247-257): prev / nxt None when absent."""
    check(load().mt_upsample4(_ptr(prev), _ptr(cur), _ptr(nxt), _ptr(frames), frames.stride(0) if ldf is None else ldf,
                              cur.numel(), _stream(stream)))


def istft_frames(spec, count, nfft, cos_table, window, ring_frames, frame0, ring, ld_spec=None, stream=None) -> None:
    """Encoder.istftFrames (Kernels.swift:259-270)."""
    check(load().mt_istft_frames(_ptr(spec), spec.stride(0) if ld_spec is None else ld_spec, count, nfft, _ptr(cos_table),
                                 _ptr(window), _ptr(ring_frames), frame0, ring, _stream(stream)))


def istft_emit(ring_frames, window, nfft, hop, s0, count, last_frame, ring, out, stream=None) -> None:
    """Encoder.istftEmit (Kernels.swift:272-283)."""
    check(load().mt_istft_emit(_ptr(ring_frames), _ptr(window), nfft, hop, s0, count, last_frame, ring, _ptr(out),
                               _stream(stream)))


# ------------------------------------------- mirror of the reference types --

@dataclass
class GPUTensor:
    """GPUTensor (Kernels.swift:7-11): a tensor at an element offset of a buffer, ``count``
    elements long; ``dtype`` names the element type when the buffer is a byte arena (a
    WeightArena's tensors sit at byte offsets of one uint8 buffer)."""
    buffer: object
    offset: int = 0
    count: int = 0
    dtype: Optional[int] = None

    def ptr(self) -> int:
        return self.buffer.data_ptr() + self.offset * self.buffer.element_size()

    def elem_type(self) -> int:
        return self.dtype if self.dtype is not None else dtype_code(self.buffer)


@dataclass
class Linear:
    """Linear (Kernels.swift:13-19): y = x W^T (+ bias), w [n, k] row-major."""
    w: GPUTensor
    bias: Optional[GPUTensor]
    n: int
    k: int


@dataclass
class ActView:
    """ActView (Kernels.swift:30-44): a view of rows at an element offset, stride ``ld``."""
    buffer: object
    offset: int = 0
    ld: int = 0

    def row(self, r: int) -> "ActView":
        return ActView(self.buffer, self.offset + r * self.ld, self.ld)

    def column(self, c: int) -> "ActView":
        return ActView(self.buffer, self.offset + c, self.ld)

    def ptr(self) -> int:
        return self.buffer.data_ptr() + self.offset * self.buffer.element_size()


class Encoder:
    """The reference's Encoder (Kernels.swift:89-206) over the C ABI, on one stream."""

    def __init__(self, stream=None):
        self.stream = stream

    def linear(self, x: ActView, rows: int, linear: Linear, y: ActView, flags: int = 0,
               gate: Optional[GPUTensor] = None) -> None:
        """Encoder.linear (Kernels.swift:132-161)."""
        wt = linear.w.elem_type()
        check(linear_raw(x.ptr(), dtype_code(x.buffer), linear.w.ptr(), gate.ptr() if gate else None, wt,
                         linear.bias.ptr() if linear.bias else None, y.ptr(), rows, linear.n, linear.k, x.ld, y.ld,
                         flags, self.stream))

    def rmsnorm(self, x: ActView, rows: int, width: int, weight: GPUTensor, y: ActView, eps: float = 1e-6) -> None:
        """Encoder.rmsnorm (Kernels.swift:163-171)."""
        check(rmsnorm_raw(x.ptr(), x.ld, rows, width, weight.ptr(), weight.elem_type(), y.ptr(), y.ld, eps,
                          self.stream))


# ----------------------------------------------------------- weight path --

class SafeTensors:
    """SafeTensors (SafeTensors.swift:7-87): a memory-mapped .safetensors file (mt_st_*).
    ``entries`` maps names (header order) to (dtype code or -1, shape, byte count)."""

    def __init__(self, path: str):
        h = ctypes.c_void_p()
        check(load().mt_st_open(os.fsencode(path), ctypes.byref(h)))
        self.handle = h
        L = load()
        self.entries = {}
        for i in range(check(L.mt_st_count(h))):
            name = ctypes.c_char_p()
            check(L.mt_st_name(h, i, ctypes.byref(name)))
            e = self.entry(name.value.decode())
            self.entries[name.value.decode()] = (e.dtype, tuple(e.shape[:e.ndim]), e.bytes)

    def entry(self, name: str) -> StEntry:
        e = StEntry()
        check(load().mt_st_find(self.handle, name.encode(), ctypes.byref(e)))
        return e

    def raw(self, name: str) -> bytes:
        """The tensor's bytes as stored."""
        e = self.entry(name)
        return ctypes.string_at(e.host, e.bytes)

    def close(self) -> None:
        if self.handle:
            load().mt_st_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class WeightArena:
    """WeightArena (Weights.swift:8-79) over mt_arena_*: plan tensors (``tensor``, ``linear``,
    ``padded_linear``), then ``upload`` into one 256-byte-aligned device buffer (a torch uint8
    tensor this object owns); the planned GPUTensor / Linear objects are bound to it then.
    ``convert_to`` F16 converts the bf16 weights to fp16 at upload (``audit`` gives the
    overflow and flush-to-zero counts)."""

    def __init__(self, st: SafeTensors, convert_to: int = BF16):
        h = ctypes.c_void_p()
        check(load().mt_arena_create(st.handle, convert_to, ctypes.byref(h)))
        self.handle, self.st, self.dtype = h, st, convert_to
        self.buffer = None
        self._planned = []

    def tensor(self, *names: str) -> "GPUTensor":
        arr = (ctypes.c_char_p * len(names))(*[n.encode() for n in names])
        off, cnt = ctypes.c_uint64(), ctypes.c_uint64()
        check(load().mt_arena_tensor(self.handle, arr, len(names), ctypes.byref(off), ctypes.byref(cnt)))
        t = GPUTensor(None, off.value, cnt.value)
        self._planned.append(t)
        return t

    def linear(self, prefix: str, n: int, k: int, bias: bool) -> "Linear":
        w = self.tensor(prefix + ".weight")
        if w.count != n * k:
            raise MingTTSError(EINVAL, f"bad checkpoint: {prefix}.weight has {w.count} elements, expected {n}x{k}")
        return Linear(w, self.tensor(prefix + ".bias") if bias else None, n, k)

    def padded_linear(self, prefix: str, n: int, k: int, stored_k: int) -> "Linear":
        off = ctypes.c_uint64()
        check(load().mt_arena_padded(self.handle, (prefix + ".weight").encode(), n, k, stored_k, ctypes.byref(off)))
        t = GPUTensor(None, off.value, n * k)
        self._planned.append(t)
        return Linear(t, None, n, k)

    @property
    def nbytes(self) -> int:
        return load().mt_arena_bytes(self.handle)

    def upload(self, device=None, stream=None) -> None:
        import torch
        dev = torch.device("cuda", 0) if device is None else device
        self.buffer = torch.empty(max(self.nbytes, 256), dtype=torch.uint8, device=dev)
        check(load().mt_arena_upload(self.handle, self.buffer.data_ptr(), _stream(stream)))
        for t in self._planned:
            t.buffer, t.dtype = self.buffer, self.dtype

    def audit(self) -> tuple:
        ov, un = ctypes.c_uint64(), ctypes.c_uint64()
        check(load().mt_arena_audit(self.handle, ctypes.byref(ov), ctypes.byref(un)))
        return ov.value, un.value

    def close(self) -> None:
        if self.handle:
            load().mt_arena_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @staticmethod
    def load(st: SafeTensors, build, convert_to: int = BF16, device=None):
        """WeightArena.load (Weights.swift:15-22): plans with ``build(arena)``, allocates and
        uploads, and returns the build's result bound to the arena (kept on ``result``'s
        arena attribute by the caller as needed)."""
        arena = WeightArena(st, convert_to)
        result = build(arena)
        arena.upload(device)
        return result, arena


from .flow import FlowSchedule, time_embeddings  # noqa: E402  (host side of the flow sampler)
