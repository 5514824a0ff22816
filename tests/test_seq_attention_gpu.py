"""Whole decode layers (Qwen.swift:84-91: rmsnorm, qkv, rope_cache, attention, o, rmsnorm,
gate|up, down) as one persistent launch: linears plus decode attention items
(mt_seq_create_items) against an fp64 oracle layer, against the same step issued as
separate launches (mt_linear, mt_rope_cache_decode, mt_attention_decode), across re-runs,
and at the attention edges (fp32 cache, sliding window, one row, a position past the
cache)."""
import numpy as np
import pytest
import torch

import mingtts as mt
import oracle as O
from _gpu_util import say
from test_seq_gpu import H, INTER, QKV, make_stack

pytestmark = pytest.mark.gpu

HQ, HKV = 14, 2


def make_caches(layers, B, cap, seed, cache_np, device):
    """Per-layer K / V caches [B, hkv, cap, 64] ~ N(0, 1) in the cache type."""
    ks, vs = [], []
    for l in range(layers):
        z = O.gaussian(seed * 100 + l, 2 * B * HKV * cap * 64).reshape(2, B, HKV, cap, 64).astype(cache_np)
        ks.append(torch.from_numpy(z[0].copy()).to(device))
        vs.append(torch.from_numpy(z[1].copy()).to(device))
    return ks, vs


def layer_items(ws, B, resid, qkv, att, mlp, ks, vs, pos_d, invf_d, cap, window=0):
    items = []
    for p, kc, vc in zip(ws, ks, vs):
        d = p["dev"]
        items.append(mt.op(resid, d["qkv"], qkv, B, bias=d["qkv_b"], norm=d["norm1"]))
        items.append(mt.attn_op(qkv, B, HQ, HKV, pos_d, kc, vc, cap, HKV * cap * 64, invf_d, att, window=window))
        items.append(mt.op(att, d["o"], resid, B, flags=mt.GemvFlags.accumulate))
        items.append(mt.op(resid, d["gate"], mlp, B, flags=mt.GemvFlags.siluGate, w2=d["up"], norm=d["norm2"]))
        items.append(mt.op(mlp, d["down"], resid, B, flags=mt.GemvFlags.accumulate))
    return items


def oracle_layers(ws, x0, B, kcs, vcs, pos, invf, window, cache_np):
    """The same layers in fp64 per op; activations stored as fp32 between ops; the new cache
    row of each layer is the rotated k and the v rounded to the cache type, and attention
    runs over the stored cache values (KernelTests.swift:207-268 restated in the oracle)."""
    resid = x0.astype(np.float32).copy()
    cap = kcs[0].shape[2]
    rows = []
    qkv = att = mlp = None
    for p, kc0, vc0 in zip(ws, kcs, vcs):
        qkv = O.linear_np64(O.rmsnorm_f64(resid, p["norm1"], O.F16), p["qkv"], None, O.F16, p["qkv_b"], None,
                            0).astype(np.float32)
        att = np.zeros((B, HQ * 64), np.float32)
        new_rows = []
        for b in range(B):
            kc = kc0[b].astype(np.float64)
            vc = vc0[b].astype(np.float64)
            q = O.rope_neox(qkv[b, :HQ * 64].reshape(HQ, 64), int(pos[b]), invf)
            k = O.rope_neox(qkv[b, HQ * 64:(HQ + HKV) * 64].reshape(HKV, 64), int(pos[b]), invf)
            v = qkv[b, (HQ + HKV) * 64:].reshape(HKV, 64)
            if pos[b] < cap:
                kc[:, pos[b]] = k.astype(cache_np)
                vc[:, pos[b]] = v.astype(cache_np)
                qpos = int(pos[b])
            else:
                qpos = cap - 1
            new_rows.append((k.astype(cache_np), v.astype(cache_np)))
            att[b] = O.attention_f64(q, kc, vc, qpos, window, 0.125).reshape(-1)
        rows.append(new_rows)
        resid = O.linear_f64(att, p["o"], None, O.F16, None, resid, B, H, H, O.ACCUM).astype(np.float32)
        mlp = O.linear_np64(O.rmsnorm_f64(resid, p["norm2"], O.F16), p["gate"], p["up"], O.F16, None, None,
                            O.SILU_GATE).astype(np.float32)
        resid = O.linear_f64(mlp, p["down"], None, O.F16, None, resid, B, H, INTER, O.ACCUM).astype(np.float32)
    return resid, qkv, att, mlp, rows


def _setup(layers, B, cap, seed, cache_np, gpu, pos):
    ws, x0 = make_stack(layers, B, seed, gpu)
    kcs, vcs = make_caches(layers, B, cap, seed, cache_np, gpu)
    k0 = [k.cpu().numpy().copy() for k in kcs]
    v0 = [v.cpu().numpy().copy() for v in vcs]
    resid = torch.from_numpy(x0.copy()).to(gpu)
    qkv = torch.zeros(B, QKV, device=gpu)
    att = torch.zeros(B, HQ * 64, device=gpu)
    mlp = torch.zeros(B, INTER, device=gpu)
    pos_d = torch.from_numpy(np.asarray(pos, np.int32)).to(gpu)
    invf = O.inv_freq(1e6)
    invf_d = torch.from_numpy(invf).to(gpu)
    return ws, x0, kcs, vcs, k0, v0, resid, qkv, att, mlp, pos_d, invf, invf_d


@pytest.mark.parametrize("layers,B,cap,cache_np,window,pos", [
    (4, 2, 512, np.float16, 0, [441, 338]),       # the decode configuration, lengths in [32, 512]
    (24, 2, 512, np.float16, 0, [100, 511]),      # 24 layers; the last cache slot
    (2, 2, 128, np.float32, 64, [127, 130]),      # fp32 cache, window 64, row 1 past the cache
    (3, 1, 256, np.float16, 0, [0]),              # one row at position 0 (one key)
    (3, 4, 256, np.float16, 0, [10, 200, 255, 77]),   # four independent sequences (M = 4)
])
def test_layers_match_fp64_oracle(gpu, layers, B, cap, cache_np, window, pos):
    say(f"seq+attention layers={layers} B={B} cap={cap} cache={np.dtype(cache_np).name} window={window} pos={pos}")
    ws, x0, kcs, vcs, k0, v0, resid, qkv, att, mlp, pos_d, invf, invf_d = _setup(layers, B, cap, 31 + layers, cache_np,
                                                                                gpu, pos)
    seq = mt.Seq(layer_items(ws, B, resid, qkv, att, mlp, kcs, vcs, pos_d, invf_d, cap, window))
    seq.run()
    torch.cuda.synchronize()
    seq.check()
    seq.close()
    want_r, want_q, want_a, want_m, rows = oracle_layers(ws, x0, B, k0, v0, pos, invf, window, cache_np)
    for got, want, what in ((resid, want_r, "resid"), (qkv, want_q, "qkv"), (att, want_a, "attention"),
                            (mlp, want_m, "mlp")):
        g = got.cpu().numpy()
        assert np.all(np.isfinite(g)), what
        rel = O.normwise_rel_err(g, want)
        assert rel <= 1e-3, f"{what}: normwise {rel:.3g}"
    # The caches: row pos of each layer holds the new k (rotated) and v; all else untouched.
    for l in range(layers):
        kg, vg = kcs[l].cpu().numpy(), vcs[l].cpu().numpy()
        for b in range(B):
            p = pos[b]
            keep = np.ones(cap, bool)
            if p < cap:
                keep[p] = False
                kn, vn = rows[l][b]
                tol = 2e-3 if cache_np == np.float16 else 1e-5
                np.testing.assert_allclose(kg[b, :, p].astype(np.float64), kn.astype(np.float64), rtol=tol, atol=tol)
                np.testing.assert_allclose(vg[b, :, p].astype(np.float64), vn.astype(np.float64), rtol=tol, atol=tol)
            np.testing.assert_array_equal(kg[b][:, keep], k0[l][b][:, keep])
            np.testing.assert_array_equal(vg[b][:, keep], v0[l][b][:, keep])


@pytest.mark.parametrize("B,cache_np", [(2, np.float16), (1, np.float32)])
def test_decode_layer_kernel_with_attention_matches_general_kernel(gpu, B, cache_np):
    """Whole decode layers at the backbone's shapes run the decode-layer kernel with its
    attention items; MT_TUNE_SEQ_LAYER = 1 runs the same plan on the general kernel.  They
    split K and sum the attention's key groups differently (7 waves against 8), so they agree
    to fp32 rounding; the new cache rows agree to the cache type's rounding."""
    layers, cap = 6, 512
    pos = [441, 338][:B]
    outs = {}
    for mode in (0, 1):
        ws, x0, kcs, vcs, k0, v0, resid, qkv, att, mlp, pos_d, invf, invf_d = _setup(layers, B, cap, 53, cache_np,
                                                                                    gpu, pos)
        old = mt.set_tuning(mt.TUNE_SEQ_LAYER, mode)
        try:
            seq = mt.Seq(layer_items(ws, B, resid, qkv, att, mlp, kcs, vcs, pos_d, invf_d, cap))
        finally:
            mt.set_tuning(mt.TUNE_SEQ_LAYER, old)
        say(f"seq+attention B={B} mode {mode} kernel {seq.kernel} groups {seq.groups}")
        assert seq.kernel == (mt.SEQ_DECODE_LAYER if mode == 0 else mt.SEQ_GENERAL)
        runs = []
        for _ in range(2):
            for l in range(layers):
                kcs[l].copy_(torch.from_numpy(k0[l]))
                vcs[l].copy_(torch.from_numpy(v0[l]))
            resid.copy_(torch.from_numpy(x0))
            seq.run()
            torch.cuda.synchronize()
            runs.append([t.cpu().numpy().copy() for t in (resid, qkv, att, mlp)] +
                        [np.stack([k.cpu().numpy() for k in kcs]).astype(np.float64)])
        seq.check()
        seq.close()
        for a, b in zip(runs[0], runs[1]):
            np.testing.assert_array_equal(a, b)
        outs[mode] = runs[0]
    want = oracle_layers(ws, x0, B, k0, v0, pos, invf, 0, cache_np)
    for j, what in enumerate(("resid", "qkv", "attention", "mlp")):
        assert O.normwise_rel_err(outs[0][j], want[j]) <= 1e-3, what
        assert O.normwise_rel_err(outs[0][j], outs[1][j].astype(np.float64)) <= 1e-4, what
    tol = 2e-3 if cache_np == np.float16 else 1e-5
    np.testing.assert_allclose(outs[0][4], outs[1][4], rtol=tol, atol=tol)


def test_layers_equal_separate_launches_and_rerun_bit_exact(gpu):
    """The fused layers against the same step as separate launches (another kernel and
    summation order for every part: fp32 rounding apart), and re-runs of the plan bit for
    bit (the cache rows it writes are the same each run)."""
    layers, B, cap = 4, 2, 512
    pos = [300, 47]
    say("seq+attention vs separate launches")
    ws, x0, kcs, vcs, k0, v0, resid, qkv, att, mlp, pos_d, invf, invf_d = _setup(layers, B, cap, 77, np.float16,
                                                                                gpu, pos)
    lens_d = pos_d + 1
    stride = HKV * cap * 64
    for p, kc, vc in zip(ws, kcs, vcs):
        d = p["dev"]
        for o in (mt.op(resid, d["qkv"], qkv, B, bias=d["qkv_b"], norm=d["norm1"]),):
            assert mt.linear_rmsnorm_raw(o.x, o.xt, o.norm, o.w, o.w2, o.wt, o.bias, o.y, o.p.M, o.p.N, o.p.K,
                                         o.p.ldx, o.p.ldy, o.p.flags, o.p.eps, None) == 0, mt.last_error()
        mt.rope_cache_decode(qkv, QKV, B, HQ, HKV, pos_d, kc, vc, cap, stride, invf_d)
        mt.attention_decode(qkv, QKV, B, HQ, HKV, lens_d, 0, kc, vc, cap, stride, att, HQ * 64, 0.125)
        for o in (mt.op(att, d["o"], resid, B, flags=mt.GemvFlags.accumulate),
                  mt.op(resid, d["gate"], mlp, B, flags=mt.GemvFlags.siluGate, w2=d["up"], norm=d["norm2"]),
                  mt.op(mlp, d["down"], resid, B, flags=mt.GemvFlags.accumulate)):
            if o.norm:
                rc = mt.linear_rmsnorm_raw(o.x, o.xt, o.norm, o.w, o.w2, o.wt, o.bias, o.y, o.p.M, o.p.N, o.p.K,
                                           o.p.ldx, o.p.ldy, o.p.flags, o.p.eps, None)
            else:
                rc = mt.linear_raw(o.x, o.xt, o.w, o.w2, o.wt, o.bias, o.y, o.p.M, o.p.N, o.p.K, o.p.ldx, o.p.ldy,
                                   o.p.flags, None)
            assert rc == 0, mt.last_error()
    torch.cuda.synchronize()
    ref_resid = resid.cpu().numpy().copy()
    ref_att = att.cpu().numpy().copy()
    ref_k = [k.cpu().numpy().copy() for k in kcs]
    for l in range(layers):   # back to the initial caches
        kcs[l].copy_(torch.from_numpy(k0[l]))
        vcs[l].copy_(torch.from_numpy(v0[l]))
    seq = mt.Seq(layer_items(ws, B, resid, qkv, att, mlp, kcs, vcs, pos_d, invf_d, cap))
    results = []
    for _ in range(3):
        resid.copy_(torch.from_numpy(x0))
        seq.run()
        torch.cuda.synchronize()
        results.append((resid.cpu().numpy().copy(), att.cpu().numpy().copy()))
    seq.check()
    seq.close()
    for r, a in results:
        np.testing.assert_array_equal(r, results[0][0])
        np.testing.assert_array_equal(a, results[0][1])
    assert O.normwise_rel_err(results[0][0], ref_resid.astype(np.float64)) <= 1e-5
    # The last layer's attention reads a residual that the two paths rounded differently
    # (about 1e-6 apart); its softmax scales that relative difference by the size of the
    # scores, so the two fp32 results agree to 1e-4 (the fp64 precision gate of 1e-3 is
    # checked against the oracle layer).
    assert O.normwise_rel_err(results[0][1], ref_att.astype(np.float64)) <= 1e-4
    for l in range(layers):   # the same cache rows (the rotation of k, rounded to fp16)
        got = kcs[l].cpu().numpy().astype(np.float64)
        np.testing.assert_allclose(got, ref_k[l].astype(np.float64), rtol=2e-3, atol=2e-3)


def test_linear_after_early_attention_item_reads_no_stale_scratch(gpu):
    """An attention item at position 5 (six keys: half the workgroup's waves see none) uses
    the activation staging as scratch; the next linear (M = 1, K = 776, so its staged x ends
    before that scratch does) over-reads the staging past K against zero weights.  The result
    must be the fp64 linear of the attention output, with no NaN from the item's leftovers."""
    cap, B, N, K = 64, 1, 64, 776
    say("seq attention item then M=1 K=776 linear")
    rng = np.random.default_rng(4)
    qkv = torch.from_numpy(rng.standard_normal((B, QKV)).astype(np.float32)).to(gpu)
    kc = torch.from_numpy(rng.standard_normal((B, HKV, cap, 64)).astype(np.float16)).to(gpu)
    vc = torch.from_numpy(rng.standard_normal((B, HKV, cap, 64)).astype(np.float16)).to(gpu)
    att = torch.zeros(B, HQ * 64, device=gpu)
    y = torch.zeros(B, N, device=gpu)
    pos_d = torch.tensor([5], dtype=torch.int32, device=gpu)
    invf_d = torch.from_numpy(O.inv_freq(1e6)).to(gpu)
    wb, _ = O.round16(rng.standard_normal((N, K)).astype(np.float32) * np.float32(0.05), O.F16)
    w = torch.from_numpy(wb.view(np.int16)).to(gpu).view(torch.float16)
    seq = mt.Seq([mt.attn_op(qkv, B, HQ, HKV, pos_d, kc, vc, cap, HKV * cap * 64, invf_d, att),
                  mt.op(att, w, y, B, ldx=HQ * 64)])
    for _ in range(2):
        seq.run()
        torch.cuda.synchronize()
        seq.check()
        a = att.cpu().numpy()
        got = y.cpu().numpy()
        assert np.all(np.isfinite(a)) and np.all(np.isfinite(got))
        want = O.linear_f64(np.ascontiguousarray(a[:, :K]), wb, None, O.F16, None, None, B, N, K, 0)
        assert O.normwise_rel_err(got, want) <= 1e-5
    seq.close()


@pytest.mark.parametrize("B", [1, 2])
def test_token_with_final_norm_and_stop_head_matches_fp64(gpu, B):
    """The llm stage's token (Engine.swift:381-385): the decode layers with attention in one
    launch, then the final RMSNorm of the last hidden rows (Qwen.swift:94) and the stop head, a
    2 x 896 linear with bias (Engine.swift:385), against the fp64 chain of the same token."""
    layers, cap = 4, 512
    pos = [441, 338][:B]
    say(f"token + final norm + stop head B={B}")
    ws, x0, kcs, vcs, k0, v0, resid, qkv, att, mlp, pos_d, invf, invf_d = _setup(layers, B, cap, 61, np.float16, gpu, pos)
    fin = 1.0 + O.gaussian(63, H, 0.1)
    fin_bits, _ = O.round16(fin, O.F16)
    stop = O.gaussian(64, 2 * H + 2, 0.02)
    stop_bits, _ = O.round16(stop, O.F16)
    stop_w, stop_b = stop_bits[:2 * H].reshape(2, H), stop_bits[2 * H:]
    from _gpu_util import dev16
    fin_d, stop_w_d, stop_b_d = dev16(fin_bits, O.F16, gpu), dev16(stop_w, O.F16, gpu), dev16(stop_b, O.F16, gpu)
    z = torch.zeros(B, H, device=gpu)
    logits = torch.zeros(B, 2, device=gpu)
    seq = mt.Seq(layer_items(ws, B, resid, qkv, att, mlp, kcs, vcs, pos_d, invf_d, cap))
    seq.run()
    mt.rmsnorm(resid, fin_d, z, rows=B)
    mt.linear(z, stop_w_d, logits, B, bias=stop_b_d)
    torch.cuda.synchronize()
    seq.check()
    seq.close()
    want_r = oracle_layers(ws, x0, B, k0, v0, pos, invf, 0, np.float16)[0]
    want_z = O.rmsnorm_f64(want_r, fin_bits, O.F16).astype(np.float32)
    want_l = O.linear_np64(want_z, stop_w, None, O.F16, stop_b, None, 0)
    for got, want, what in ((z, want_z, "final norm"), (logits, want_l, "stop logits")):
        g = got.cpu().numpy()
        assert np.all(np.isfinite(g)), what
        rel = O.normwise_rel_err(g, want)
        assert rel <= 1e-3, f"{what}: normwise {rel:.3g}"
