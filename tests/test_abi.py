"""The C ABI without a GPU: the library loads, exports every symbol the header declares,
and rejects bad arguments with MT_EINVAL before touching the device (the reference turns
the same shape violations into preconditionFailure, Kernels.swift:105, 147)."""
import os
import re
import subprocess

import pytest

import mingtts as mt

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mingtts_hip.h")

ALIGNED = 1 << 20          # fake 16-byte-aligned "device" addresses: never dereferenced,
W_ADDR = 2 << 20           # every call below fails validation before any HIP call
Y_ADDR = 8 << 20


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mt_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert header_functions() == sorted(mt.EXPORTS)


def test_library_exports_every_declared_symbol():
    mt.load()
    out = subprocess.run(["nm", "-D", "--defined-only", mt.LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (mt_[a-z0-9_]+)$", out, flags=re.M))
    missing = set(header_functions()) - exported
    assert not missing, missing
    assert mt.load().mt_version().decode().startswith("mingtts_hip")


def lin(M=2, N=64, K=64, ldx=None, ldy=None, flags=0, x=ALIGNED, w=W_ADDR, w2=None, bias=None, y=Y_ADDR,
        xt=mt.F32, wt=mt.F16):
    return mt.linear_raw(x, xt, w, w2, wt, bias, y, M, N, K, K if ldx is None else ldx, N if ldy is None else ldy,
                         flags, stream=0)


@pytest.mark.parametrize("kwargs,needle", [
    (dict(K=60, ldx=64), "multiple of 8"),
    (dict(K=0), "multiple of 8"),
    (dict(ldx=32), "ldx"),
    (dict(ldy=32), "ldy"),
    (dict(wt=mt.F32), "weights must be f16 or bf16"),
    (dict(xt=7), "activation dtype"),
    (dict(flags=mt.GemvFlags.bias), "MT_BIAS without a bias"),
    (dict(flags=mt.GemvFlags.siluGate), "without w2"),
    (dict(flags=64), "unknown flag"),
    (dict(x=ALIGNED + 4), "16-byte aligned"),
    (dict(ldx=66, K=64), "16-byte"),
    (dict(w=W_ADDR + 8), "w / w2"),
    (dict(flags=mt.GemvFlags.siluGate, w2=W_ADDR + 8), "w / w2"),
    (dict(y=Y_ADDR + 2), "y must be"),
    (dict(x=None), "null"),
    (dict(y=ALIGNED + 64), "overlaps"),
])
def test_linear_rejects_bad_arguments(kwargs, needle):
    rc = lin(**kwargs)
    assert rc == mt.EINVAL
    assert needle in mt.last_error()


def test_empty_linear_is_a_no_op():
    assert lin(M=0) == mt.OK
    assert lin(N=0) == mt.OK


def test_linear_rmsnorm_rejects_bad_arguments():
    def call(norm=W_ADDR, eps=1e-6, K=64):
        return mt.linear_rmsnorm_raw(ALIGNED, mt.F32, norm, W_ADDR, None, mt.F16, None, Y_ADDR, 2, 64, K, 64, 64, 0,
                                     eps, stream=0)
    assert call(norm=None) == mt.EINVAL and "null norm" in mt.last_error()
    assert call(norm=W_ADDR + 2) == mt.EINVAL and "norm must be 16-byte" in mt.last_error()
    assert call(eps=-1e-3) == mt.EINVAL and "eps" in mt.last_error()
    assert call(eps=float("nan")) == mt.EINVAL
    assert call(K=12) == mt.EINVAL


def test_kernel_choice_and_tuning_round_trip():
    """The analogue of Kernels.usesGemm / scalarRowsMax (KernelTests.swift:155-157, 165-166):
    the family mt_linear actually launches, under each tuning."""
    assert mt.linear_kernel(1, 1152, 896) == mt.KERNEL_GEMV
    assert mt.linear_kernel(2, 4864, 896) == mt.KERNEL_GEMV
    assert mt.linear_kernel(3, 1152, 896) == mt.KERNEL_GEMV_MFMA
    assert mt.linear_kernel(8, 2, 896) == mt.KERNEL_GEMV_MFMA
    assert mt.linear_kernel(16, 64, 32) == mt.KERNEL_GEMV_MFMA
    assert mt.linear_kernel(17, 64, 32) == mt.KERNEL_GEMM
    assert mt.linear_kernel(174, 1152, 896) == mt.KERNEL_GEMM
    old = mt.set_tuning(mt.TUNE_GEMV_ROWS_MAX, 2)
    try:
        assert mt.linear_kernel(3, 1152, 896) == mt.KERNEL_GEMV_MFMA   # past the GEMV rows: <= 16 rows
        assert mt.linear_kernel(2, 1152, 896) == mt.KERNEL_GEMV
    finally:
        mt.set_tuning(mt.TUNE_GEMV_ROWS_MAX, old)
    old = mt.set_tuning(mt.TUNE_GEMV_MFMA, 1)
    try:
        assert mt.linear_kernel(3, 1152, 896) == mt.KERNEL_GEMV
        assert mt.linear_kernel(16, 64, 32) == mt.KERNEL_GEMM
    finally:
        mt.set_tuning(mt.TUNE_GEMV_MFMA, old)
    old = mt.set_tuning(mt.TUNE_GEMV_MFMA, 2)
    try:
        assert mt.linear_kernel(64, 1152, 896, xt=mt.BF16, wt=mt.BF16) == mt.KERNEL_GEMV_MFMA   # 64 columns
        assert mt.linear_kernel(33, 1152, 896) == mt.KERNEL_GEMM       # fp32 x: 2 M = 66 columns > 64
    finally:
        mt.set_tuning(mt.TUNE_GEMV_MFMA, old)
    assert mt.load().mt_set_tuning(99, 0) == mt.EINVAL
    assert mt.load().mt_set_tuning(mt.TUNE_GEMV_ROWS_MAX, 9) == mt.EINVAL
    assert mt.load().mt_set_tuning(mt.TUNE_SEQ_LAUNCH, 2) == mt.EINVAL
    assert mt.set_tuning(mt.TUNE_SEQ_LAUNCH, 0) == 1   # the ordinary launch is the default
    assert mt.set_tuning(mt.TUNE_SEQ_LAUNCH, -1) == 0


def test_seq_create_validates_every_op_before_the_device():
    import ctypes
    def op(M=2, K=64, wt=mt.F16, norm=None, eps=0.0):
        return mt.LinearOp(ALIGNED, W_ADDR, None, None, norm, Y_ADDR, mt.GemvParams(M, 64, K, 64, 64, 0, eps), mt.F32, wt)

    ok, bad_m, bad_t, bad_k = op(), op(M=9), op(wt=mt.BF16), op(K=60)
    bad_norm = op(norm=W_ADDR + 8)
    bad_eps = op(norm=W_ADDR, eps=-1.0)
    L = mt.load()
    h = ctypes.c_void_p()
    for ops, needle in (([ok, bad_m], "op 1: a sequence takes M <= 8"), ([ok, bad_t], "share the weight"),
                        ([bad_k], "op 0: K must"), ([bad_norm], "norm must be 16-byte"),
                        ([ok, ok, bad_eps], "op 2: RMSNorm eps")):
        arr = (mt.LinearOp * len(ops))(*ops)
        assert L.mt_seq_create(arr, len(ops), ctypes.byref(h)) == mt.EINVAL
        assert needle in mt.last_error()
    assert L.mt_seq_create(None, 1, ctypes.byref(h)) == mt.EINVAL
    assert L.mt_seq_run(None, None) == mt.EINVAL


def test_seq_plan_refuses_what_dataflow_cannot_order():
    """The plan compiler runs before any device call: layouts it cannot map and hazards it
    cannot prove ordered are refused with MT_ENOTSUP."""
    import ctypes
    L = mt.load()
    h = ctypes.c_void_p()
    A, B, C, D = 1 << 20, 2 << 20, 3 << 20, 4 << 20
    W = 8 << 20

    def op(x, y, ldx=64, ldy=64, K=64, N=64, M=2, flags=0):
        return mt.LinearOp(x, W, None, None, None, y, mt.GemvParams(M, N, K, ldx, ldy, flags, 0.0), mt.F32, mt.F16)

    cases = [
        ([op(A, B), op(B, C, ldx=32, K=32)], "another layout"),                 # B read at stride 32, written at 64
        ([op(A, B, ldy=128), op(C, B + 128, ldy=128)], "partly overwrites"),    # columns 32..95 over 0..63
        ([op(A, B), op(D, A)], "read from the user buffer"),                    # A overwritten, no dependency
        ([op(A, B), op(B, C), op(B, C, flags=mt.GemvFlags.accumulate, ldy=32, N=32)],
         "accumulates into op 1's output at another layout"),
    ]
    for ops, needle in cases:
        arr = (mt.LinearOp * len(ops))(*ops)
        assert L.mt_seq_create(arr, len(ops), ctypes.byref(h)) == mt.ENOTSUP, needle
        assert needle in mt.last_error(), mt.last_error()


def test_rope_and_attention_reject_bad_arguments():
    L = mt.load()
    A = ALIGNED
    # hq not a multiple of hkv
    assert L.mt_attention(A, 1152, 1, 14, 3, 0, 0, A, A, mt.F32, 512, A, 896, 0.125, None) == mt.EINVAL
    # positions past the cache
    assert L.mt_attention(A, 1152, 4, 14, 2, 510, 0, A, A, mt.F32, 512, A, 896, 0.125, None) == mt.EINVAL
    assert "past cache_len" in mt.last_error()
    # cache too long for the score buffer
    assert L.mt_attention(A, 1152, 1, 14, 2, 0, 0, A, A, mt.F32, 5000, A, 896, 0.125, None) == mt.EINVAL
    # bf16 caches are not supported
    assert L.mt_attention_decode(A, 1152, 2, 14, 2, A, 0, A, A, mt.BF16, 512, 65536, A, 896, 0.125, None) == mt.EINVAL
    # overlapping per-sequence caches
    assert L.mt_attention_decode(A, 1152, 2, 14, 2, A, 0, A, A, mt.F16, 512, 100, A, 896, 0.125, None) == mt.EINVAL
    assert L.mt_rope_cache(A, 896, 1, 14, 2, 0, A, A, mt.F32, 512, A, None) == mt.EINVAL   # ldq too small
    assert L.mt_rope_cache(A, 1152, 2, 14, 2, 511, A, A, mt.F32, 512, A, None) == mt.EINVAL
    assert L.mt_rope_cache_decode(A, 1152, 2, 14, 2, None, A, A, mt.F16, 512, 65536, A, None) == mt.EINVAL
    assert L.mt_attention(A, 1152, 0, 14, 2, 0, 0, A, A, mt.F32, 512, A, 896, 0.125, None) == mt.OK  # empty


def test_dit_attention_linear_rejects_bad_arguments():
    """mt_dit_attention_linear checks its attention shape on top of mt_linear's checks."""
    L = mt.load()
    A = ALIGNED

    def call(B=2, S=3, H=16, M=6, N=1024, K=1024, ldq=3072, flags=0, inv=A, y=Y_ADDR):
        p = mt.GemvParams(M, N, K, ldq, N, flags, 0.0)
        return L.mt_dit_attention_linear(A, B, S, H, inv, 0.125, W_ADDR, mt.BF16, None, y, p, None)

    assert call(S=9, M=18) == mt.EINVAL and "at most 8 rows" in mt.last_error()
    assert call(M=5) == mt.EINVAL and "is not B" in mt.last_error()
    assert call(K=960) == mt.EINVAL and "64 H" in mt.last_error()
    assert call(flags=mt.GemvFlags.siluGate) == mt.EINVAL and "gate partner" in mt.last_error()
    assert call(ldq=2048) == mt.EINVAL and "< 3 K" in mt.last_error()
    assert call(inv=None) == mt.EINVAL and "inv_freq" in mt.last_error()
    assert call(y=A + 4096) == mt.EINVAL and "overlaps y" in mt.last_error()   # y inside qkv's k span
    assert call(B=6, S=8, M=48) == mt.ENOTSUP and "at most 32 rows" in mt.last_error()
    assert call(B=0, M=0) == mt.OK   # empty


def test_flow_euler_assemble_rejects_bad_arguments():
    L = mt.load()
    A = ALIGNED

    def call(hidden=1024, latent=64, ldp=64, ldx=1024, wt=mt.BF16, xw=W_ADDR, y=A):
        return L.mt_flow_euler_assemble(y, A, ldp, 2, 5, None, 2.0, 0.0625, A, A, A, A, xw, A, wt, Y_ADDR, ldx,
                                        hidden, latent, None)

    assert call(hidden=0) == mt.EINVAL and "empty" in mt.last_error()
    assert call(wt=mt.F32) == mt.EINVAL and "f16 or bf16" in mt.last_error()
    assert call(y=None) == mt.EINVAL and "null pointer" in mt.last_error()
    assert call(latent=60, ldp=60) == mt.EINVAL and "multiple of 8" in mt.last_error()
    assert call(latent=2056, ldp=2056) == mt.EINVAL and "up to 2048" in mt.last_error()
    assert call(xw=W_ADDR + 2) == mt.EINVAL and "aligned" in mt.last_error()
    assert call(ldp=32) == mt.EINVAL and "ldp" in mt.last_error()
    assert call(ldx=1000) == mt.EINVAL and "ldx" in mt.last_error()


def test_seq_item_layout_matches_the_header(tmp_path):
    """The ctypes mirrors of mt_attn_op, mt_dit_attn_op and mt_seq_item have the C compiler's
    sizes and offsets."""
    import ctypes
    src = tmp_path / "layout.c"
    src.write_text('#include <stddef.h>\n#include <stdio.h>\n#include "mingtts_hip.h"\n'
                   'int main(void) { printf("%zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu\\n", sizeof(mt_attn_op), '
                   'offsetof(mt_attn_op, cache_stride), offsetof(mt_attn_op, scale), sizeof(mt_seq_item), '
                   'offsetof(mt_seq_item, linear), offsetof(mt_seq_item, attn), sizeof(mt_linear_op), '
                   'sizeof(mt_dit_attn_op), offsetof(mt_dit_attn_op, inv_freq), offsetof(mt_dit_attn_op, scale), '
                   'offsetof(mt_seq_item, dit)); return 0; }\n')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    got = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    want = [ctypes.sizeof(mt.AttnOp), mt.AttnOp.cache_stride.offset, mt.AttnOp.scale.offset,
            ctypes.sizeof(mt.SeqItem), mt.SeqItem.linear.offset, mt.SeqItem.attn.offset, ctypes.sizeof(mt.LinearOp),
            ctypes.sizeof(mt.DitAttnOp), mt.DitAttnOp.inv_freq.offset, mt.DitAttnOp.scale.offset,
            mt.SeqItem.dit.offset]
    assert got == want


def _items(ops):
    import ctypes
    items = (mt.SeqItem * len(ops))()
    for i, o in enumerate(ops):
        if isinstance(o, mt.AttnOp):
            items[i].kind, items[i].attn = mt.SEQ_ATTENTION, o
        elif isinstance(o, mt.DitAttnOp):
            items[i].kind, items[i].dit = mt.SEQ_DIT_ATTENTION, o
        else:
            items[i].kind, items[i].linear = mt.SEQ_LINEAR, o
    return items


def test_seq_attention_items_are_checked_before_the_device():
    """Attention items: argument errors are MT_EINVAL, cache aliasing is MT_ENOTSUP, both
    before any device call (a valid list gets as far as the device query)."""
    import ctypes
    L = mt.load()
    h = ctypes.c_void_p()
    QKV, OUT, KC, VC, RES, POS, INV = (k << 20 for k in (1, 2, 4, 6, 8, 10, 11))
    W = 16 << 20
    stride = 2 * 512 * 64

    def attn(**kw):
        a = dict(qkv=QKV, ldq=1152, B=2, hq=14, hkv=2, pos=POS, k_cache=KC, v_cache=VC, cache_t=mt.F16,
                 cache_len=512, cache_stride=stride, inv_freq=INV, out=OUT, ldo=896, window=0, scale=0.125)
        a.update(kw)
        return mt.AttnOp(*(a[f[0]] for f in mt.AttnOp._fields_))

    def lin(x, y, N=1152, K=896, ldx=None, ldy=None, flags=0):
        return mt.LinearOp(x, W, None, None, None, y,
                           mt.GemvParams(2, N, K, K if ldx is None else ldx, N if ldy is None else ldy, flags, 0.0),
                           mt.F32, mt.F16)

    layer = [lin(RES, QKV), attn(), lin(OUT, RES, N=896, flags=mt.GemvFlags.accumulate)]
    rc = L.mt_seq_create_items(_items(layer), len(layer), ctypes.byref(h))
    assert rc not in (mt.EINVAL, mt.ENOTSUP), mt.last_error()   # planned; the device query fails here
    for bad, needle in ((attn(B=9), "1 <= B <= 8"), (attn(hkv=3), "multiple of hkv"),
                        (attn(cache_t=mt.BF16), "cache dtype"), (attn(cache_len=5000), "cache_len"),
                        (attn(ldq=1024), "ldq"), (attn(k_cache=KC + 8), "16-byte aligned"),
                        (attn(pos=None), "null pointer"), (attn(cache_stride=1000), "cache_stride")):
        ops = [lin(RES, QKV), bad]
        assert L.mt_seq_create_items(_items(ops), 2, ctypes.byref(h)) == mt.EINVAL, needle
        assert needle in mt.last_error(), mt.last_error()
    for ops, needle in (([lin(RES, QKV), attn(v_cache=KC)], "attention caches overlap"),
                        ([lin(RES, KC), attn()], "overlaps an attention cache"),
                        ([attn(), attn(out=RES)], "attention caches overlap")):
        assert L.mt_seq_create_items(_items(ops), len(ops), ctypes.byref(h)) == mt.ENOTSUP, needle
        assert needle in mt.last_error(), mt.last_error()
    items = _items([lin(RES, QKV)])
    items[0].kind = 7
    assert L.mt_seq_create_items(items, 1, ctypes.byref(h)) == mt.EINVAL
    assert "unknown kind" in mt.last_error()


def test_dit_attention_items_are_checked_before_the_device():
    """DiT attention items: argument errors are MT_EINVAL; a sequence with one outside the
    DiT-block pattern (shape, wiring, frequencies, the general kernel forced) is MT_ENOTSUP,
    both before any device call; the pattern itself gets as far as the device query."""
    import ctypes
    L = mt.load()
    h = ctypes.c_void_p()
    X, QKV, ATT, FF, INV, INV2 = (k << 22 for k in (1, 2, 3, 4, 5, 6))
    W, B16 = 64 << 22, 96 << 22

    def lin(x, y, N, K, flags, norm=True, M=6):
        return mt.LinearOp(x, W, None, B16, B16 if norm else None, y,
                           mt.GemvParams(M, N, K, K, N, flags | mt.GemvFlags.bias, 1e-6 if norm else 0.0),
                           mt.F32, mt.BF16)

    def dit(**kw):
        a = dict(qkv=QKV, ldq=3072, B=2, S=3, H=16, inv_freq=INV, out=ATT, ldo=1024, scale=0.125)
        a.update(kw)
        return mt.DitAttnOp(*(a[f[0]] for f in mt.DitAttnOp._fields_))

    def block(att=None, out_x=ATT, ff1_flags=mt.GemvFlags.gelu):
        return [lin(X, QKV, 3072, 1024, 0), dit() if att is None else att,
                lin(out_x, X, 1024, 1024, mt.GemvFlags.accumulate, norm=False),
                lin(X, FF, 4096, 1024, ff1_flags), lin(FF, X, 1024, 4096, mt.GemvFlags.accumulate, norm=False)]

    good = block() + block()
    rc = L.mt_seq_create_items(_items(good), len(good), ctypes.byref(h))
    assert rc not in (mt.EINVAL, mt.ENOTSUP), mt.last_error()   # planned; the device query fails here
    # the aggregator's shape, batch 1 x seq 2
    agg = [lin(X, QKV, 3072, 1024, 0, M=2), dit(B=1, S=2), lin(ATT, X, 1024, 1024, mt.GemvFlags.accumulate, False, 2),
           lin(X, FF, 4096, 1024, mt.GemvFlags.gelu, M=2), lin(FF, X, 1024, 4096, mt.GemvFlags.accumulate, False, 2)]
    rc = L.mt_seq_create_items(_items(agg), len(agg), ctypes.byref(h))
    assert rc not in (mt.EINVAL, mt.ENOTSUP), mt.last_error()
    odd = [lin(X, QKV, 3072, 1024, 0, M=4), dit(B=2, S=2), lin(ATT, X, 1024, 1024, mt.GemvFlags.accumulate, False, 4),
           lin(X, FF, 4096, 1024, mt.GemvFlags.gelu, M=4), lin(FF, X, 1024, 4096, mt.GemvFlags.accumulate, False, 4)]
    assert L.mt_seq_create_items(_items(odd), len(odd), ctypes.byref(h)) == mt.ENOTSUP   # B 2 x S 2: no kernel
    assert "DiT-block kernel" in mt.last_error(), mt.last_error()
    for bad, needle in ((dit(B=0), "B, S, H >= 1"), (dit(S=9), "S <= 8"), (dit(B=3, S=3), "B S <= 8"),
                        (dit(inv_freq=None), "null pointer"), (dit(ldq=2048), "ldq"),
                        (dit(out=ATT + 4), "16-byte aligned")):
        ops = block(att=bad)
        assert L.mt_seq_create_items(_items(ops), len(ops), ctypes.byref(h)) == mt.EINVAL, needle
        assert needle in mt.last_error(), mt.last_error()
    for ops in (block(ff1_flags=0),                                  # ff1 without GELU
                block(att=dit(scale=0.25)) + block(),                # scales differ between items
                block() + block(att=dit(inv_freq=INV2)),             # frequencies differ between items
                block()[:4]):                                        # not whole blocks
        assert L.mt_seq_create_items(_items(ops), len(ops), ctypes.byref(h)) == mt.ENOTSUP
        assert "DiT-block kernel" in mt.last_error(), mt.last_error()
    ops = block(att=dit(H=8))                                        # not the flow head's heads: out reads
    assert L.mt_seq_create_items(_items(ops), len(ops), ctypes.byref(h)) == mt.ENOTSUP   # past its output
    mt.set_tuning(mt.TUNE_SEQ_LAYER, 1)
    try:
        assert L.mt_seq_create_items(_items(good), len(good), ctypes.byref(h)) == mt.ENOTSUP
    finally:
        mt.set_tuning(mt.TUNE_SEQ_LAYER, 0)
