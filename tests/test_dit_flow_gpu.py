"""The DiT flow step around its linears on the GPU (Shaders.swift:598-693): dit_attention on
the reference's own known-answer case (KernelTests.swift:282-318) and other shapes,
flow_assemble and flow_euler against the oracle, and one whole flow step (assembly, DiT
blocks of the reference's flow head shape -- hidden 1024, 16 heads, 2 x 3 rows -- final
layer, Euler update; Engine.swift:395-402, DiT.swift:35-52) against an fp64 chain, the time
MLP precompute (Engine.swift:186-198), and the whole 10-step ODE loop of the EPSS schedule."""
import numpy as np
import pytest
import torch

import mingtts as mt
import oracle as O
from _gpu_util import assert_linear_parity, dev16, say

pytestmark = pytest.mark.gpu


def invf_1e4():
    """The reference test's frequencies: 1 / powf(1e4, 2n / 64) in fp32 (KernelTests.swift:286)."""
    n = np.arange(32, dtype=np.float32)
    return (np.float32(1.0) / np.power(np.float32(1e4), np.float32(2.0) * n / np.float32(64))).astype(np.float32)


def test_dit_attention_reference_kat(gpu):
    """testDitAttention: B 2, S 3, H 16, qkv from the KAT RNG (state 11), atol 2e-5."""
    B, S, H = 2, 3, 16
    D = H * 64
    ld = 3 * D
    qkv = O.LCG(11).floats(B * S * ld)
    invf = invf_1e4()
    out = torch.zeros(B * S, D, device=gpu)
    say("dit_attention KAT")
    mt.dit_attention(torch.from_numpy(qkv.reshape(B * S, ld)).to(gpu), B, S, H, torch.from_numpy(invf).to(gpu), out)
    torch.cuda.synchronize()
    want = O.dit_attention_f64(qkv.reshape(B * S, ld), B, S, H, invf)
    np.testing.assert_allclose(out.cpu().numpy(), want, rtol=0, atol=2e-5)


@pytest.mark.parametrize("B,S,H,pad", [(1, 1, 1, 0), (3, 8, 16, 0), (2, 5, 2, 64), (4, 2, 3, 2)])
def test_dit_attention_shapes(gpu, B, S, H, pad):
    D = H * 64
    ld = 3 * D + pad
    rng = np.random.default_rng(B * 100 + S * 10 + H)
    qkv = rng.standard_normal((B * S, ld)).astype(np.float32)
    invf = invf_1e4()
    out = torch.full((B * S, D + pad), 7.0, device=gpu)
    say(f"dit_attention B={B} S={S} H={H} pad={pad}")
    mt.dit_attention(torch.from_numpy(qkv).to(gpu), B, S, H, torch.from_numpy(invf).to(gpu), out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    want = O.dit_attention_f64(qkv, B, S, H, invf)
    np.testing.assert_allclose(got[:, :D], want, rtol=0, atol=2e-5)
    assert np.all(got[:, D:] == 7.0)   # the row padding is not written


def test_dit_attention_rejects_long_sequences():
    assert mt.load().mt_dit_attention(1 << 20, 3072, 1, 9, 16, 1 << 20, 2 << 20, 1024, 0.125, None) == mt.EINVAL
    assert "at most 8 rows" in mt.last_error()


@pytest.mark.parametrize("B,S,H,N,wt,flags,bias,pad", [
    (2, 3, 16, 1024, O.BF16, O.ACCUM, True, 0),    # the flow head's out projection (split K)
    (2, 3, 16, 4096, O.F16, 0, False, 64),         # 256 tiles, no split; padded qkv rows
    (1, 1, 1, 64, O.F16, 0, True, 0),              # one row
    (4, 2, 3, 300, O.BF16, O.GELU, True, 8),       # ragged N, K = 192
    (2, 8, 2, 200, O.F16, O.ACCUM, False, 0),      # 16 rows: two column groups
    (4, 8, 1, 96, O.BF16, 0, True, 4),             # 32 rows: four column groups
])
def test_dit_attention_linear(gpu, B, S, H, N, wt, flags, bias, pad):
    """mt_dit_attention_linear against the fp64 chain (dit attention, then the linear) to the
    linear precision gate, and against mt_dit_attention into a buffer followed by mt_linear:
    the same bits wherever that linear runs the same small-row MFMA kernel and split (3..16
    rows), else within 1e-5."""
    M, K = B * S, 64 * H
    ldq = 3 * K + pad
    rng = np.random.default_rng(M * 1000 + N + H)
    qkv = rng.standard_normal((M, ldq)).astype(np.float32)
    w, _ = O.round16(rng.standard_normal((N, K)).astype(np.float32) * np.float32(0.02), wt)
    b16 = O.round16(rng.standard_normal(N).astype(np.float32) * np.float32(0.02), wt)[0] if bias else None
    y0 = rng.standard_normal((M, N)).astype(np.float32)
    invf = invf_1e4()
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    qkv_d, invf_d, w_d = t(qkv), t(invf), dev16(w, wt, gpu)
    b_d = dev16(b16, wt, gpu) if bias else None
    y = t(y0)
    say(f"dit_attention_linear B={B} S={S} H={H} N={N} wt={wt} flags={flags} bias={bias} pad={pad}")
    mt.dit_attention_linear(qkv_d, B, S, H, invf_d, w_d, y, flags=flags, bias=b_d)
    att = torch.zeros(M, K, device=gpu)
    mt.dit_attention(qkv_d, B, S, H, invf_d, att)
    y2 = t(y0)
    mt.linear(att, w_d, y2, M, flags=flags, bias=b_d)
    torch.cuda.synchronize()
    got, sep = y.cpu().numpy(), y2.cpu().numpy()
    x_used = O.dit_attention_f64(qkv, B, S, H, invf).astype(np.float32)
    want32 = O.linear_f32(x_used, w, None, wt, b16, y0, M, N, K, flags)
    want64 = O.linear_f64(x_used, w, None, wt, b16, y0, M, N, K, flags)
    assert_linear_parity(got, want32, want64, K, "fused")
    if 3 <= M <= 16:
        np.testing.assert_array_equal(got, sep)
    else:
        np.testing.assert_allclose(got, sep, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("wt,hidden,ldx", [(O.BF16, 1024, 1024), (O.F16, 96, 100), (O.BF16, 300, 304)])
def test_flow_assemble(gpu, wt, hidden, ldx):
    latent = 64
    rng = np.random.default_rng(hidden + wt)
    w, _ = O.round16(rng.standard_normal((hidden, latent)).astype(np.float32) * np.float32(0.05), wt)
    xb, _ = O.round16(rng.standard_normal(hidden).astype(np.float32) * np.float32(0.05), wt)
    cb, _ = O.round16(rng.standard_normal(hidden).astype(np.float32), wt)
    y, hist = rng.standard_normal(latent).astype(np.float32), rng.standard_normal(latent).astype(np.float32)
    cemb, temb = rng.standard_normal(hidden).astype(np.float32), rng.standard_normal(hidden).astype(np.float32)
    x = torch.full((6, ldx), -3.0, device=gpu)
    say(f"flow_assemble wt={wt} hidden={hidden}")
    t = lambda a: torch.from_numpy(a).to(gpu)
    mt.flow_assemble(t(y), t(hist), t(cemb), dev16(cb, wt, gpu), t(temb), dev16(w, wt, gpu), dev16(xb, wt, gpu), x)
    torch.cuda.synchronize()
    got = x.cpu().numpy()
    want = O.flow_assemble_f64(y, hist, cemb, cb, temb, w, xb, wt)
    np.testing.assert_allclose(got[:, :hidden], want, rtol=1e-6, atol=1e-6)
    assert np.all(got[:, hidden:] == -3.0)


def test_flow_euler(gpu):
    latent = 64
    rng = np.random.default_rng(3)
    pred = rng.standard_normal((6, latent)).astype(np.float32)
    y0 = rng.standard_normal(latent).astype(np.float32)
    for cfg, dt, capture in ((2.0, 0.0625, True), (0.0, 0.125, False)):
        y = torch.from_numpy(y0.copy()).to(gpu)
        cap = torch.zeros(2 * latent, device=gpu) if capture else None
        say(f"flow_euler cfg={cfg}")
        mt.flow_euler(y, torch.from_numpy(pred).to(gpu), 2, 5, cfg, dt, capture=cap)
        torch.cuda.synchronize()
        want, want_cap = O.flow_euler_f64(y0, pred, 2, 5, cfg, dt)
        np.testing.assert_allclose(y.cpu().numpy(), want, rtol=1e-6, atol=1e-7)
        if capture:
            np.testing.assert_array_equal(cap.cpu().numpy(), want_cap.astype(np.float32))


@pytest.mark.parametrize("wt,hidden,latent,ldx", [(O.BF16, 1024, 64, 1024), (O.F16, 1000, 72, 1008)])
def test_flow_euler_assemble_matches_the_two_launches(gpu, wt, hidden, latent, ldx):
    """mt_flow_euler_assemble = mt_flow_euler then mt_flow_assemble of the next ODE step: y, the
    six rows of x (row stride ldx) and the captured velocities, bit for bit."""
    rng = np.random.default_rng(17 + latent)
    f32 = lambda *shape: rng.standard_normal(shape).astype(np.float32)
    w16 = lambda *shape, s=0.05: dev16(O.round16(f32(*shape) * np.float32(s), wt)[0], wt, gpu)
    pred = torch.from_numpy(f32(6, latent)).to(gpu)
    y0, hist = f32(latent), torch.from_numpy(f32(latent)).to(gpu)
    cemb, temb = torch.from_numpy(f32(hidden)).to(gpu), torch.from_numpy(f32(hidden)).to(gpu)
    cbias, xw, xb = w16(hidden, s=1.0), w16(hidden, latent), w16(hidden)
    outs = []
    for fused in (False, True):
        y = torch.from_numpy(y0.copy()).to(gpu)
        x = torch.zeros(6, ldx, device=gpu)
        cap = torch.zeros(2 * latent, device=gpu)
        say(f"flow_euler_assemble fused={fused} w{wt} hidden={hidden} latent={latent}")
        if fused:
            mt.flow_euler_assemble(y, pred, 2, 5, 2.0, 0.0625, hist, cemb, cbias, temb, xw, xb, x, capture=cap)
        else:
            mt.flow_euler(y, pred, 2, 5, 2.0, 0.0625, capture=cap)
            mt.flow_assemble(y, hist, cemb, cbias, temb, xw, xb, x)
        torch.cuda.synchronize()
        outs.append([t.cpu().numpy() for t in (y, x, cap)])
    for a, b, what in zip(outs[0], outs[1], ("y", "x", "capture")):
        np.testing.assert_array_equal(b, a, err_msg=what)
    assert np.all(outs[1][1][:, hidden:] == 0.0)  # past hidden in each row: untouched


HID, HEADS, LAT = 1024, 16, 64


def dit_weights(blocks, seed):
    """bf16 weights ~ N(0, 0.02^2) of the flow head's DiT blocks (Weights.swift:146-172) and
    gains ~ 1 + N(0, 0.1^2), seeded per block."""
    out = []
    for i in range(blocks):
        rng = np.random.default_rng(seed * 100 + i)
        def w(*shape):
            return O.round16(rng.standard_normal(shape).astype(np.float32) * np.float32(0.02), O.BF16)[0]
        def g(n):
            return O.round16((1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32), O.BF16)[0]
        out.append(dict(norm1=g(HID), qkv=w(3 * HID, HID), qkv_b=w(3 * HID), out=w(HID, HID), out_b=w(HID),
                        norm2=g(HID), ff1=w(4 * HID, HID), ff1_b=w(4 * HID), ff2=w(HID, 4 * HID), ff2_b=w(HID)))
    return out


def oracle_flow_step(blocks, final, x0, invf, y0, cfg, dt):
    """DiTForward.encode over the six assembled rows (batch 2 x seq 3) then the Euler update,
    fp64 per op with fp32 activations between ops."""
    x = x0.astype(np.float32).copy()
    M = 6
    for p in blocks:
        qkv = O.linear_np64(O.rmsnorm_f64(x, p["norm1"], O.BF16), p["qkv"], None, O.BF16, p["qkv_b"], None,
                            O.BIAS).astype(np.float32)
        att = O.dit_attention_f64(qkv, 2, 3, HEADS, invf).astype(np.float32)
        x = O.linear_f64(att, p["out"], None, O.BF16, p["out_b"], x, M, HID, HID, O.ACCUM).astype(np.float32)
        ff = O.linear_np64(O.rmsnorm_f64(x, p["norm2"], O.BF16), p["ff1"], None, O.BF16, p["ff1_b"], None,
                           O.BIAS | O.GELU).astype(np.float32)
        x = O.linear_f64(ff, p["ff2"], None, O.BF16, p["ff2_b"], x, M, HID, 4 * HID, O.ACCUM).astype(np.float32)
    pred = O.linear_np64(O.rmsnorm_f64(x, final["norm"], O.BF16), final["w"], None, O.BF16, final["b"], None,
                         O.BIAS).astype(np.float32)
    y1, _ = O.flow_euler_f64(y0, pred, 2, 5, cfg, dt)
    return x, pred, y1


@pytest.mark.parametrize("fused", [False, True])
def test_flow_step_matches_fp64_chain(gpu, fused):
    """One ODE step of the flow head: assemble, 2 DiT blocks, final norm + linear, Euler;
    with ``fused`` the attention runs inside the out projection (mt_dit_attention_linear)."""
    rng = np.random.default_rng(21)
    blocks = dit_weights(2, 21)
    final = dict(norm=O.round16((1.0 + 0.1 * rng.standard_normal(HID)).astype(np.float32), O.BF16)[0],
                 w=O.round16(rng.standard_normal((LAT, HID)).astype(np.float32) * np.float32(0.02), O.BF16)[0],
                 b=O.round16(rng.standard_normal(LAT).astype(np.float32) * np.float32(0.02), O.BF16)[0])
    xw = O.round16(rng.standard_normal((HID, LAT)).astype(np.float32) * np.float32(0.05), O.BF16)[0]
    xb = O.round16(rng.standard_normal(HID).astype(np.float32) * np.float32(0.05), O.BF16)[0]
    cb = O.round16(rng.standard_normal(HID).astype(np.float32), O.BF16)[0]
    y0 = rng.standard_normal(LAT).astype(np.float32)
    hist = rng.standard_normal(LAT).astype(np.float32)
    cemb = rng.standard_normal(HID).astype(np.float32)
    temb = rng.standard_normal(HID).astype(np.float32)
    invf = invf_1e4()
    cfg, dt = 2.0, 0.0625
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    b16 = lambda a: dev16(a, O.BF16, gpu)
    dw = [{k: b16(v) for k, v in p.items()} for p in blocks]
    x = torch.zeros(6, HID, device=gpu)
    qkv = torch.zeros(6, 3 * HID, device=gpu)
    att = torch.zeros(6, HID, device=gpu)
    ff = torch.zeros(6, 4 * HID, device=gpu)
    pred = torch.zeros(6, LAT, device=gpu)
    y = t(y0.copy())
    invf_d = t(invf)
    say(f"flow step: assemble, 2 DiT blocks, final, euler (fused attention: {fused})")
    mt.flow_assemble(y, t(hist), t(cemb), b16(cb), t(temb), b16(xw), b16(xb), x)
    lin = lambda xx, w, out, flags=0, bias=None, norm=None: mt.linear(xx, w, out, 6, flags=flags, bias=bias, norm=norm)
    for d in dw:
        lin(x, d["qkv"], qkv, bias=d["qkv_b"], norm=d["norm1"])
        if fused:
            mt.dit_attention_linear(qkv, 2, 3, HEADS, invf_d, d["out"], x, flags=mt.GemvFlags.accumulate,
                                    bias=d["out_b"])
        else:
            mt.dit_attention(qkv, 2, 3, HEADS, invf_d, att)
            lin(att, d["out"], x, flags=mt.GemvFlags.accumulate, bias=d["out_b"])
        lin(x, d["ff1"], ff, flags=mt.GemvFlags.gelu, bias=d["ff1_b"], norm=d["norm2"])
        lin(ff, d["ff2"], x, flags=mt.GemvFlags.accumulate, bias=d["ff2_b"])
    lin(x, b16(final["w"]), pred, bias=b16(final["b"]), norm=b16(final["norm"]))
    mt.flow_euler(y, pred, 2, 5, cfg, dt)
    torch.cuda.synchronize()
    x0 = O.flow_assemble_f64(y0, hist, cemb, cb, temb, xw, xb, O.BF16)
    want_x, want_pred, want_y = oracle_flow_step(blocks, final, x0, invf, y0, cfg, dt)
    for got, want, what in ((x, want_x, "hidden"), (pred, want_pred, "velocity"), (y, want_y, "latent")):
        g = got.cpu().numpy()
        assert np.all(np.isfinite(g)), what
        rel = O.normwise_rel_err(g, want)
        assert rel <= 1e-3, f"{what}: normwise {rel:.3g}"


def dit_block_items(dw, x, qkv, att, ff, invf_d, B=2, S=3):
    """The items of DiTForward.encode's blocks (DiT.swift:35-52) over the B S rows x, as a
    persistent sequence: per block rmsnorm+qkv, the DiT attention, out +=, rmsnorm+ff1 GELU,
    ff2 +=."""
    M = B * S
    items = []
    for d in dw:
        items += [mt.op(x, d["qkv"], qkv, M, bias=d["qkv_b"], norm=d["norm1"]),
                  mt.dit_attn_op(qkv, B, S, HEADS, invf_d, att),
                  mt.op(att, d["out"], x, M, flags=mt.GemvFlags.accumulate, bias=d["out_b"]),
                  mt.op(x, d["ff1"], ff, M, flags=mt.GemvFlags.gelu, bias=d["ff1_b"], norm=d["norm2"]),
                  mt.op(ff, d["ff2"], x, M, flags=mt.GemvFlags.accumulate, bias=d["ff2_b"])]
    return items


@pytest.mark.parametrize("B,S,blocks_n", [(2, 3, 1), (2, 3, 8), (1, 2, 1), (1, 2, 8)])
def test_dit_blocks_as_one_persistent_launch(gpu, B, S, blocks_n):
    """The DiT blocks of one ODE step (B 2 x S 3) or of the aggregator (B 1 x S 2) as one
    launch of the DiT-block kernel: the hidden rows within 1e-3 (normwise) of the fp64 chain
    and within 1e-5 of the same blocks as separate launches; the last attention item's output
    written; two runs in a row give the same bits."""
    M = B * S
    rng = np.random.default_rng(51)
    blocks = dit_weights(blocks_n, 51)
    x0 = rng.standard_normal((M, HID)).astype(np.float32)
    invf = invf_1e4()
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    dw = [{k: dev16(v, O.BF16, gpu) for k, v in p.items()} for p in blocks]
    x = t(x0.copy())
    qkv = torch.zeros(M, 3 * HID, device=gpu)
    att = torch.zeros(M, HID, device=gpu)
    ff = torch.zeros(M, 4 * HID, device=gpu)
    invf_d = t(invf)
    say(f"DiT-block kernel: {blocks_n} blocks at B {B} x S {S}")
    seq = mt.Seq(dit_block_items(dw, x, qkv, att, ff, invf_d, B, S))
    assert seq.kernel == mt.SEQ_DIT_BLOCK and seq.groups == 256
    runs = []
    for _ in range(2):
        x.copy_(t(x0))
        seq.run()
        torch.cuda.synchronize()
        seq.check()
        runs.append((x.cpu().numpy().copy(), att.cpu().numpy().copy()))
    np.testing.assert_array_equal(runs[1][0], runs[0][0])
    got, got_att = runs[1]
    # the same blocks as separate launches
    xs = t(x0.copy())
    for d in dw:
        mt.linear(xs, d["qkv"], qkv, M, bias=d["qkv_b"], norm=d["norm1"])
        mt.dit_attention(qkv, B, S, HEADS, invf_d, att)
        mt.linear(att, d["out"], xs, M, flags=mt.GemvFlags.accumulate, bias=d["out_b"])
        mt.linear(xs, d["ff1"], ff, M, flags=mt.GemvFlags.gelu, bias=d["ff1_b"], norm=d["norm2"])
        mt.linear(ff, d["ff2"], xs, M, flags=mt.GemvFlags.accumulate, bias=d["ff2_b"])
    torch.cuda.synchronize()
    assert O.normwise_rel_err(got, xs.cpu().numpy()) <= 1e-5
    assert O.normwise_rel_err(got_att, att.cpu().numpy()) <= 1e-5
    # the fp64 chain
    want = x0.copy()
    for p in blocks:
        q = O.linear_np64(O.rmsnorm_f64(want, p["norm1"], O.BF16), p["qkv"], None, O.BF16, p["qkv_b"], None,
                          O.BIAS).astype(np.float32)
        a = O.dit_attention_f64(q, B, S, HEADS, invf).astype(np.float32)
        want = O.linear_f64(a, p["out"], None, O.BF16, p["out_b"], want, M, HID, HID, O.ACCUM).astype(np.float32)
        f = O.linear_np64(O.rmsnorm_f64(want, p["norm2"], O.BF16), p["ff1"], None, O.BF16, p["ff1_b"], None,
                          O.BIAS | O.GELU).astype(np.float32)
        want = O.linear_f64(f, p["ff2"], None, O.BF16, p["ff2_b"], want, M, HID, 4 * HID, O.ACCUM).astype(np.float32)
    rel = O.normwise_rel_err(got, want)
    assert rel <= 1e-3, f"normwise {rel:.3g}"
    seq.close()


def test_time_embeddings_match_fp64(gpu):
    """MingEngine.precomputeTimeEmbeddings (Engine.swift:186-198): the 10-step schedule's
    sinusoids through time1 (256 -> 1024, SiLU) and time2 (1024 -> 1024) at M = 10, on the
    GPU through mt.time_embeddings, against the fp64 time MLP on the same sinusoid rows."""
    rng = np.random.default_rng(31)
    w1 = O.round16(rng.standard_normal((HID, 256)).astype(np.float32) * np.float32(0.02), O.BF16)[0]
    b1 = O.round16(rng.standard_normal(HID).astype(np.float32) * np.float32(0.02), O.BF16)[0]
    w2 = O.round16(rng.standard_normal((HID, HID)).astype(np.float32) * np.float32(0.02), O.BF16)[0]
    b2 = O.round16(rng.standard_normal(HID).astype(np.float32) * np.float32(0.02), O.BF16)[0]
    ts = mt.FlowSchedule.timesteps(10)
    b16 = lambda a: dev16(a, O.BF16, gpu)
    say("time embeddings: 10 sinusoids through the time MLP")
    temb = mt.time_embeddings((b16(w1), b16(b1)), (b16(w2), b16(b2)), ts)
    torch.cuda.synchronize()
    got = temb.cpu().numpy()
    assert got.shape == (10, HID)
    want = O.time_mlp_f64(mt.FlowSchedule.sinusoids(ts[:10]), w1, b1, w2, b2, O.BF16)
    assert O.normwise_rel_err(got, want) <= 1e-5


def test_flow_ode_loop_matches_fp64_chain(gpu):
    """The flow stage of one generation step (MingEngine.encodeStep, Engine.swift:387-402): the
    cond embedder on the LLM row (896 -> 1024, M = 1), then the 10 ODE steps of the EPSS
    schedule with sway -- assemble with that step's time embedding, 2 DiT blocks of the flow
    head's shape, final norm + linear, the CFG Euler step with dt = t[k+1] - t[k] and the
    velocity captured per step -- against the same loop as an fp64 chain (fp32 between ops)."""
    rng = np.random.default_rng(41)
    blocks = dit_weights(2, 41)
    bf = lambda *shape, s=0.02: O.round16(rng.standard_normal(shape).astype(np.float32) * np.float32(s), O.BF16)[0]
    final = dict(norm=O.round16((1.0 + 0.1 * rng.standard_normal(HID)).astype(np.float32), O.BF16)[0],
                 w=bf(LAT, HID), b=bf(LAT))
    xw, xb = bf(HID, LAT, s=0.05), bf(HID, s=0.05)
    cw, cbias = bf(HID, 896), bf(HID, s=1.0)
    w1, b1, w2, b2 = bf(HID, 256), bf(HID), bf(HID, HID), bf(HID)
    z = rng.standard_normal((1, 896)).astype(np.float32)
    y0 = rng.standard_normal(LAT).astype(np.float32)
    hist = rng.standard_normal(LAT).astype(np.float32)
    invf = invf_1e4()
    cfg = 2.0
    ts = mt.FlowSchedule.timesteps(10)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    b16 = lambda a: dev16(a, O.BF16, gpu)
    dw = [{k: b16(v) for k, v in p.items()} for p in blocks]
    x = torch.zeros(6, HID, device=gpu)
    qkv = torch.zeros(6, 3 * HID, device=gpu)
    ff = torch.zeros(6, 4 * HID, device=gpu)
    pred = torch.zeros(6, LAT, device=gpu)
    cemb = torch.zeros(1, HID, device=gpu)
    vel = torch.zeros(10, 2 * LAT, device=gpu)
    y = t(y0.copy())
    invf_d = t(invf)
    say("flow ODE loop: time MLP, cond embedder, 10 steps x (assemble, 2 DiT blocks, final, euler)")
    temb = mt.time_embeddings((b16(w1), b16(b1)), (b16(w2), b16(b2)), ts)
    mt.linear(t(z), b16(cw), cemb, 1, bias=b16(cbias))
    lin = lambda xx, w, out, flags=0, bias=None, norm=None: mt.linear(xx, w, out, 6, flags=flags, bias=bias, norm=norm)
    for k in range(10):
        mt.flow_assemble(y, t(hist), cemb[0], b16(cbias), temb[k], b16(xw), b16(xb), x)
        for d in dw:
            lin(x, d["qkv"], qkv, bias=d["qkv_b"], norm=d["norm1"])
            mt.dit_attention_linear(qkv, 2, 3, HEADS, invf_d, d["out"], x, flags=mt.GemvFlags.accumulate,
                                    bias=d["out_b"])
            lin(x, d["ff1"], ff, flags=mt.GemvFlags.gelu, bias=d["ff1_b"], norm=d["norm2"])
            lin(ff, d["ff2"], x, flags=mt.GemvFlags.accumulate, bias=d["ff2_b"])
        lin(x, b16(final["w"]), pred, bias=b16(final["b"]), norm=b16(final["norm"]))
        mt.flow_euler(y, pred, 2, 5, cfg, float(ts[k + 1] - ts[k]), capture=vel[k])
    torch.cuda.synchronize()

    temb_o = O.time_mlp_f64(mt.FlowSchedule.sinusoids(ts[:10]), w1, b1, w2, b2, O.BF16).astype(np.float32)
    cemb_o = O.linear_np64(z, cw, None, O.BF16, cbias, None, O.BIAS).astype(np.float32)[0]
    yo = y0.copy()
    vel_o = []
    for k in range(10):
        x0 = O.flow_assemble_f64(yo, hist, cemb_o, cbias, temb_o[k], xw, xb, O.BF16)
        _, pred_o, _ = oracle_flow_step(blocks, final, x0, invf, yo, cfg, 0.0)
        y1, cap = O.flow_euler_f64(yo, pred_o, 2, 5, cfg, float(ts[k + 1] - ts[k]))
        yo = y1.astype(np.float32)
        vel_o.append(cap)
    for got, want, what in ((temb, temb_o, "temb"), (cemb, cemb_o[None], "cemb"), (vel, np.stack(vel_o), "velocity"),
                            (y, yo, "latent")):
        g = got.cpu().numpy()
        assert np.all(np.isfinite(g)), what
        rel = O.normwise_rel_err(g, want)
        assert rel <= 1e-3, f"{what}: normwise {rel:.3g}"


def oracle_dit_stack(blocks, x0, B, S, invf):
    """DiTForward.encode's block loop (DiT.swift:41-49) at B x S rows, fp64 per op with fp32
    activations between ops."""
    x = x0.astype(np.float32).copy()
    M = B * S
    for p in blocks:
        qkv = O.linear_np64(O.rmsnorm_f64(x, p["norm1"], O.BF16), p["qkv"], None, O.BF16, p["qkv_b"], None,
                            O.BIAS).astype(np.float32)
        att = O.dit_attention_f64(qkv, B, S, HEADS, invf).astype(np.float32)
        x = O.linear_f64(att, p["out"], None, O.BF16, p["out_b"], x, M, HID, HID, O.ACCUM).astype(np.float32)
        ff = O.linear_np64(O.rmsnorm_f64(x, p["norm2"], O.BF16), p["ff1"], None, O.BF16, p["ff1_b"], None,
                           O.BIAS | O.GELU).astype(np.float32)
        x = O.linear_f64(ff, p["ff2"], None, O.BF16, p["ff2_b"], x, M, HID, 4 * HID, O.ACCUM).astype(np.float32)
    return x


@pytest.mark.parametrize("P", [1, 3])
def test_aggregator_stage_matches_fp64(gpu, P):
    """The aggregator (linear_proj_audio): one latent per generation step (MingEngine.encodeStep,
    Engine.swift:405-410: row 0 the cls embedding, row 1 x_embedder(latent), the 8-block DiT at
    batch 1 x seq 2, the final norm + 896 x 1024 linear of row 0), or a clone prompt's P
    reference latents at once (Engine.swift:234-250: rows [cls, x_embedder(latent_p)] per
    latent at row stride 2 hidden, batch P x seq 2, the final layer of every row), against the
    fp64 chain."""
    rng = np.random.default_rng(51 + P)
    blocks = dit_weights(8, 51 + P)
    bf = lambda *shape, s=0.02: O.round16(rng.standard_normal(shape).astype(np.float32) * np.float32(s), O.BF16)[0]
    xw, xb = bf(HID, LAT, s=0.05), bf(HID, s=0.05)
    fin_norm = O.round16((1.0 + 0.1 * rng.standard_normal(HID)).astype(np.float32), O.BF16)[0]
    fin_w, fin_b = bf(896, HID), bf(896)
    cls = rng.standard_normal(HID).astype(np.float32)
    latents = rng.standard_normal((P, LAT)).astype(np.float32)
    invf = invf_1e4()
    M = 2 * P
    out_rows = 1 if P == 1 else M
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    b16 = lambda a: dev16(a, O.BF16, gpu)
    dw = [{k: b16(v) for k, v in p.items()} for p in blocks]
    x = t(np.tile(cls, (M, 1)))
    qkv = torch.zeros(M, 3 * HID, device=gpu)
    ff = torch.zeros(M, 4 * HID, device=gpu)
    out = torch.zeros(out_rows, 896, device=gpu)
    invf_d = t(invf)
    say(f"aggregator: {P} latent(s), x_embedder, 8 DiT blocks at batch {P} x seq 2, final layer of {out_rows} row(s)")
    # x_embedder(latent_p) into row 2 p + 1 (row stride 2 hidden), over the cls rows.
    mt.linear(t(latents), b16(xw), x[1:], P, bias=b16(xb), ldy=2 * HID)
    for d in dw:
        mt.linear(x, d["qkv"], qkv, M, bias=d["qkv_b"], norm=d["norm1"])
        mt.dit_attention_linear(qkv, P, 2, HEADS, invf_d, d["out"], x, flags=mt.GemvFlags.accumulate, bias=d["out_b"])
        mt.linear(x, d["ff1"], ff, M, flags=mt.GemvFlags.gelu, bias=d["ff1_b"], norm=d["norm2"])
        mt.linear(ff, d["ff2"], x, M, flags=mt.GemvFlags.accumulate, bias=d["ff2_b"])
    mt.linear(x, b16(fin_w), out, out_rows, bias=b16(fin_b), norm=b16(fin_norm))
    torch.cuda.synchronize()

    x0 = np.tile(cls, (M, 1)).astype(np.float32)
    x0[1::2] = O.linear_np64(latents, xw, None, O.BF16, xb, None, O.BIAS).astype(np.float32)
    want_x = oracle_dit_stack(blocks, x0, P, 2, invf)
    want_out = O.linear_np64(O.rmsnorm_f64(want_x[:out_rows], fin_norm, O.BF16), fin_w, None, O.BF16, fin_b, None,
                             O.BIAS)
    for got, want, what in ((x, want_x, "hidden"), (out, want_out, "LLM row(s)")):
        g = got.cpu().numpy()
        assert np.all(np.isfinite(g)), what
        rel = O.normwise_rel_err(g, want)
        assert rel <= 1e-3, f"{what}: normwise {rel:.3g}"
