"""Attention items over rows of one sequence (a shared cache: cache_stride 0, rows at
consecutive positions), the VAE decoder's sliding-window layers (VAEDecoder.decodeDispatches,
VAEDecoder.swift:81-107: rmsnorm + qkv, ropeCache + attention over the last 65 keys, o +=,
rmsnorm + gate|up, down +=, at M = 4 rows per latent) as one persistent launch: against the
same layers as separate mt_linear / mt_rope_attention launches, against an fp64 chain, and
on the general sequence kernel at other shapes."""
import numpy as np
import pytest
import torch

import mingtts as mt
import oracle as O
from _gpu_util import dev16, say
from test_seq_gpu import H, INTER, QKV, make_stack

pytestmark = pytest.mark.gpu

HQ, HKV = 14, 2


def _caches(layers, cap, seed, gpu):
    out = []
    for l in range(layers):
        z = O.gaussian(seed * 100 + l, 2 * HKV * cap * 64).reshape(2, HKV, cap, 64).astype(np.float16)
        out.append((torch.from_numpy(z[0].copy()).to(gpu), torch.from_numpy(z[1].copy()).to(gpu)))
    return out


def _oracle(ws, x0, caches0, pos0, window, invf):
    """fp64 per op, fp32 between ops; the rows' new k (rotated) and v rounded to fp16 go into
    the cache at pos0 + m before row m attends over [pos0 + m + 1 - window, pos0 + m]."""
    M = x0.shape[0]
    x = x0.astype(np.float32).copy()
    att = None
    caches = [(k.copy(), v.copy()) for k, v in caches0]
    for p, (kc, vc) in zip(ws, caches):
        qkv = O.linear_np64(O.rmsnorm_f64(x, p["norm1"], O.F16), p["qkv"], None, O.F16, p["qkv_b"], None,
                            O.BIAS).astype(np.float32)
        for m in range(M):
            k = O.rope_neox(qkv[m, HQ * 64:(HQ + HKV) * 64].reshape(HKV, 64), pos0 + m, invf)
            kc[:, pos0 + m] = k.astype(np.float16)
            vc[:, pos0 + m] = qkv[m, (HQ + HKV) * 64:].reshape(HKV, 64).astype(np.float16)
        att = np.zeros((M, HQ * 64), np.float32)
        for m in range(M):
            q = O.rope_neox(qkv[m, :HQ * 64].reshape(HQ, 64), pos0 + m, invf)
            att[m] = O.attention_f64(q, kc.astype(np.float64), vc.astype(np.float64), pos0 + m, window,
                                     0.125).reshape(-1)
        x = O.linear_np64(att, p["o"], None, O.F16, None, x, O.ACCUM).astype(np.float32)
        mlp = O.linear_np64(O.rmsnorm_f64(x, p["norm2"], O.F16), p["gate"], p["up"], O.F16, None, None,
                            O.SILU_GATE).astype(np.float32)
        x = O.linear_np64(mlp, p["down"], None, O.F16, None, x, O.ACCUM).astype(np.float32)
    return x, att, caches


@pytest.mark.parametrize("layers,pos0,window,cap", [(4, 200, 65, 512), (2, 30, 65, 512), (3, 0, 65, 128),
                                                    (2, 508, 0, 512)])
def test_vae_rows_persistent_matches_launches_and_fp64(gpu, layers, pos0, window, cap):
    M = 4
    ws, x0 = make_stack(layers, M, 90 + layers, gpu)
    caches = _caches(layers, cap, 5 + layers, gpu)
    k0 = [(k.cpu().numpy().copy(), v.cpu().numpy().copy()) for k, v in caches]
    invf = O.inv_freq(1e6)
    invf_d = torch.from_numpy(invf).to(gpu)
    pos_d = torch.from_numpy(np.arange(pos0, pos0 + M, dtype=np.int32)).to(gpu)
    frames = torch.from_numpy(x0.copy()).to(gpu)
    qkv = torch.zeros(M, QKV, device=gpu)
    att = torch.zeros(M, HQ * 64, device=gpu)
    mlp = torch.zeros(M, INTER, device=gpu)

    def reset():
        frames.copy_(torch.from_numpy(x0))
        for (k, v), (a, b) in zip(caches, k0):
            k.copy_(torch.from_numpy(a))
            v.copy_(torch.from_numpy(b))

    say(f"vae rows: separate launches layers={layers} pos0={pos0} window={window}")
    for p, (kc, vc) in zip(ws, caches):
        d = p["dev"]
        mt.linear(frames, d["qkv"], qkv, M, bias=d["qkv_b"], norm=d["norm1"])
        mt.rope_attention(qkv, QKV, M, HQ, HKV, pos0, window, kc, vc, cap, invf_d, att, HQ * 64)
        mt.linear(att, d["o"], frames, M, flags=mt.GemvFlags.accumulate)
        mt.linear(frames, d["gate"], mlp, M, flags=mt.GemvFlags.siluGate, w2=d["up"], norm=d["norm2"])
        mt.linear(mlp, d["down"], frames, M, flags=mt.GemvFlags.accumulate)
    torch.cuda.synchronize()
    ref = (frames.cpu().numpy().copy(), att.cpu().numpy().copy(),
           [(k.cpu().numpy().astype(np.float64), v.cpu().numpy().astype(np.float64)) for k, v in caches])

    items = []
    for p, (kc, vc) in zip(ws, caches):
        d = p["dev"]
        items.append(mt.op(frames, d["qkv"], qkv, M, bias=d["qkv_b"], norm=d["norm1"]))
        items.append(mt.attn_op(qkv, M, HQ, HKV, pos_d, kc, vc, cap, 0, invf_d, att, window=window))
        items.append(mt.op(att, d["o"], frames, M, flags=mt.GemvFlags.accumulate))
        items.append(mt.op(frames, d["gate"], mlp, M, flags=mt.GemvFlags.siluGate, w2=d["up"], norm=d["norm2"]))
        items.append(mt.op(mlp, d["down"], frames, M, flags=mt.GemvFlags.accumulate))
    seq = mt.Seq(items)
    assert seq.kernel == mt.SEQ_DECODE_LAYER
    runs = []
    for r in range(2):
        reset()
        say(f"vae rows: persistent run {r}")
        seq.run()
        torch.cuda.synchronize()
        runs.append((frames.cpu().numpy().copy(), att.cpu().numpy().copy(),
                     [(k.cpu().numpy().astype(np.float64), v.cpu().numpy().astype(np.float64)) for k, v in caches]))
    seq.check()
    seq.close()
    np.testing.assert_array_equal(runs[0][0], runs[1][0])
    got_f, got_a, got_c = runs[0]
    assert O.normwise_rel_err(got_f, ref[0].astype(np.float64)) <= 1e-4
    assert O.normwise_rel_err(got_a, ref[1].astype(np.float64)) <= 1e-4
    for (gk, gv), (rk, rv) in zip(got_c, ref[2]):
        np.testing.assert_allclose(gk, rk, rtol=2e-3, atol=2e-3)
        np.testing.assert_allclose(gv, rv, rtol=2e-3, atol=2e-3)
    want_f, want_a, want_c = _oracle(ws, x0, k0, pos0, window, invf)
    assert O.normwise_rel_err(got_f, want_f) <= 1e-3
    assert O.normwise_rel_err(got_a, want_a) <= 1e-3
    for (gk, gv), (wk, wv), (ik, iv) in zip(got_c, want_c, k0):
        # the rows written, to fp16 rounding; every other row untouched
        np.testing.assert_allclose(gk[:, pos0:pos0 + M], wk[:, pos0:pos0 + M].astype(np.float64), rtol=2e-3, atol=2e-3)
        keep = np.ones(cap, bool)
        keep[pos0:pos0 + M] = False
        np.testing.assert_array_equal(gk[:, keep], ik[:, keep].astype(np.float64))
        np.testing.assert_array_equal(gv[:, keep], iv[:, keep].astype(np.float64))


def test_rows_of_one_sequence_on_the_general_kernel(gpu):
    """The same shared-cache attention item on the general sequence kernel (shapes outside
    the decode-layer kernel: hidden 256, 4 q / 2 kv heads, 3 rows): qkv linear, attention,
    out linear, against mt_linear + mt_rope_attention launches."""
    M, Hd, hq, hkv, cap, pos0, window = 3, 256, 4, 2, 64, 10, 8
    n_qkv = (hq + 2 * hkv) * 64
    rng = np.random.default_rng(8)
    w_qkv, _ = O.round16(rng.standard_normal((n_qkv, Hd)).astype(np.float32) * np.float32(0.05), O.F16)
    w_o, _ = O.round16(rng.standard_normal((Hd, hq * 64)).astype(np.float32) * np.float32(0.05), O.F16)
    x = torch.from_numpy(rng.standard_normal((M, Hd)).astype(np.float32)).to(gpu)
    k0 = rng.standard_normal((hkv, cap, 64)).astype(np.float16)
    v0 = rng.standard_normal((hkv, cap, 64)).astype(np.float16)
    kc, vc = torch.from_numpy(k0.copy()).to(gpu), torch.from_numpy(v0.copy()).to(gpu)
    invf_d = torch.from_numpy(O.inv_freq(1e6)).to(gpu)
    pos_d = torch.from_numpy(np.arange(pos0, pos0 + M, dtype=np.int32)).to(gpu)
    qkv = torch.zeros(M, n_qkv, device=gpu)
    att = torch.zeros(M, hq * 64, device=gpu)
    y = torch.zeros(M, Hd, device=gpu)
    wq_d, wo_d = dev16(w_qkv, O.F16, gpu), dev16(w_o, O.F16, gpu)
    say("rows of one sequence, general kernel: separate launches")
    mt.linear(x, wq_d, qkv, M)
    mt.rope_attention(qkv, n_qkv, M, hq, hkv, pos0, window, kc, vc, cap, invf_d, att, hq * 64)
    mt.linear(att, wo_d, y, M)
    torch.cuda.synchronize()
    ref_y, ref_att, ref_k = y.cpu().numpy().copy(), att.cpu().numpy().copy(), kc.cpu().numpy().astype(np.float64)
    kc.copy_(torch.from_numpy(k0))
    vc.copy_(torch.from_numpy(v0))
    y.zero_()
    seq = mt.Seq([mt.op(x, wq_d, qkv, M),
                  mt.attn_op(qkv, M, hq, hkv, pos_d, kc, vc, cap, 0, invf_d, att, window=window),
                  mt.op(att, wo_d, y, M)])
    assert seq.kernel == mt.SEQ_GENERAL
    say("rows of one sequence, general kernel: persistent")
    seq.run()
    torch.cuda.synchronize()
    seq.check()
    seq.close()
    assert O.normwise_rel_err(att.cpu().numpy(), ref_att.astype(np.float64)) <= 1e-5
    assert O.normwise_rel_err(y.cpu().numpy(), ref_y.astype(np.float64)) <= 1e-5
    np.testing.assert_allclose(kc.cpu().numpy().astype(np.float64), ref_k, rtol=2e-3, atol=2e-3)
