"""mt_rope_cache / mt_attention on the GPU against the fp64 oracle: the reference's attention
known-answer tests (KernelTests.swift:219-278, restated bit for bit) and the batch-2 decode
configuration (fp16 caches, lengths ~ U[32, 512], RoPE base 1e6)."""
import numpy as np
import pytest
import torch

import mingtts as mt
import oracle as O
from _gpu_util import say

pytestmark = pytest.mark.gpu
HQ, HKV, LD, CAP = 14, 2, (14 + 2 * 2) * 64, 512


def _kat(t0, m, window, device):
    """KernelTests.attentionCase: prefill t0 rows then m decode rows, fp32 cache."""
    rng = O.LCG(t0 * 31 + m + window)
    total = t0 + m
    qkv = rng.floats((total + 8) * LD).reshape(total + 8, LD)
    invf = O.inv_freq(1e6)
    qkv_d = torch.from_numpy(qkv.copy()).to(device)
    kc = torch.zeros(HKV, CAP, 64, device=device)
    vc = torch.zeros(HKV, CAP, 64, device=device)
    out = torch.zeros(total, HQ * 64, device=device)
    invf_d = torch.from_numpy(invf).to(device)
    for pos0, rows in ((0, t0), (t0, m)):
        if rows == 0:
            continue
        view = qkv_d[pos0:]
        mt.rope_cache(view, LD, rows, HQ, HKV, pos0, kc, vc, CAP, invf_d)
        mt.attention(view, LD, rows, HQ, HKV, pos0, window, kc, vc, CAP, out[pos0:], HQ * 64, 0.125)
    torch.cuda.synchronize()
    # CPU: rotate every k and q in fp64, attend over the full sequence.
    ks = np.stack([O.rope_neox(qkv[:total, (HQ + h) * 64:(HQ + h + 1) * 64], np.arange(total), invf)
                   for h in range(HKV)])
    vs = np.stack([qkv[:total, (HQ + HKV + h) * 64:(HQ + HKV + h + 1) * 64] for h in range(HKV)])
    want = np.zeros((total, HQ, 64))
    for pos in range(total):
        q = O.rope_neox(qkv[pos, :HQ * 64].reshape(HQ, 64), pos, invf)
        want[pos] = O.attention_f64(q, ks, vs, pos, window, 0.125)
    return out.cpu().numpy().reshape(total, HQ, 64), want, kc.cpu().numpy(), ks


@pytest.mark.parametrize("t0,m,window", [(37, 1, 0), (130, 4, 0), (100, 4, 64), (20, 4, 64)])
def test_reference_attention_kats(gpu, t0, m, window):
    say(f"attention kat t0={t0} m={m} window={window}")
    got, want, kc, ks = _kat(t0, m, window, gpu)
    # atol 2e-5 as the reference (KernelTests.swift:267), rtol 1e-4 (assertClose default)
    ex, i, g, w = O.worst_violation(got, want, 2e-5)
    assert ex <= 0, f"index {i} got {g} want {w}"
    np.testing.assert_allclose(kc[:, :t0 + m], ks, atol=2e-6, rtol=1e-5)


def test_batched_decode_fp16_cache(gpu):
    """Batch 2 (CFG pair) decode over 512-position fp16 caches, lengths drawn from U[32, 512],
    RoPE base 1e6: rope + append the new row at len - 1, then attention over [0, len)."""
    B = 2
    rs = np.random.default_rng(2024)
    lens = rs.integers(32, 513, B).astype(np.uint32)
    invf = O.inv_freq(1e6)
    z = O.gaussian(4, B * HKV * CAP * 64 * 2 + B * LD)
    kc0 = z[:B * HKV * CAP * 64].reshape(B, HKV, CAP, 64).astype(np.float16)
    vc0 = z[B * HKV * CAP * 64:2 * B * HKV * CAP * 64].reshape(B, HKV, CAP, 64).astype(np.float16)
    qkv = z[2 * B * HKV * CAP * 64:].reshape(B, LD).copy()
    kc = torch.from_numpy(kc0.copy()).to(gpu)
    vc = torch.from_numpy(vc0.copy()).to(gpu)
    qkv_d = torch.from_numpy(qkv.copy()).to(gpu)
    pos_d = torch.from_numpy((lens - 1).astype(np.int32)).to(gpu)
    lens_d = torch.from_numpy(lens.astype(np.int32)).to(gpu)
    out = torch.zeros(B, HQ * 64, device=gpu)
    say(f"batched decode lens={lens.tolist()}")
    stride = HKV * CAP * 64
    mt.rope_cache_decode(qkv_d, LD, B, HQ, HKV, pos_d, kc, vc, CAP, stride, torch.from_numpy(invf).to(gpu))
    mt.attention_decode(qkv_d, LD, B, HQ, HKV, lens_d, 0, kc, vc, CAP, stride, out, HQ * 64, 0.125)
    torch.cuda.synchronize()
    kcg = kc.cpu().numpy().astype(np.float64)
    vcg = vc.cpu().numpy().astype(np.float64)
    got = out.cpu().numpy().reshape(B, HQ, 64)
    for b in range(B):
        p = int(lens[b]) - 1
        knew = O.rope_neox(qkv[b, HQ * 64:(HQ + HKV) * 64].reshape(HKV, 64), p, invf)
        np.testing.assert_allclose(kcg[b, :, p], knew, rtol=2e-3, atol=2e-3)      # fp16 storage
        np.testing.assert_array_equal(vcg[b, :, p], qkv[b, (HQ + HKV) * 64:].reshape(HKV, 64).astype(np.float16))
        # untouched positions keep the old cache
        np.testing.assert_array_equal(kcg[b, :, :p], kc0[b, :, :p].astype(np.float64))
        q = O.rope_neox(qkv[b, :HQ * 64].reshape(HQ, 64), p, invf)
        want = O.attention_f64(q, kcg[b], vcg[b], p, 0, 0.125)    # on the stored fp16 values
        ex, i, g, w = O.worst_violation(got[b], want, 2e-5)
        assert ex <= 0, f"b={b} index {i} got {g} want {w}"


def test_decode_window_and_length_edges(gpu):
    """Length 1 (a single key), a window shorter than the length, and a length equal to the cache."""
    B = 3
    lens = np.array([1, 300, 512], np.uint32)
    z = O.gaussian(9, B * HKV * CAP * 64 * 2 + B * HQ * 64)
    kc0 = z[:B * HKV * CAP * 64].reshape(B, HKV, CAP, 64)
    vc0 = z[B * HKV * CAP * 64:2 * B * HKV * CAP * 64].reshape(B, HKV, CAP, 64)
    q = z[2 * B * HKV * CAP * 64:].reshape(B, HQ * 64)
    kc = torch.from_numpy(kc0.copy()).to(gpu)
    vc = torch.from_numpy(vc0.copy()).to(gpu)
    qd = torch.from_numpy(q.copy()).to(gpu)
    lens_d = torch.from_numpy(lens.astype(np.int32)).to(gpu)
    out = torch.zeros(B, HQ * 64, device=gpu)
    for window in (0, 65):
        say(f"decode edges window={window}")
        mt.attention_decode(qd, HQ * 64, B, HQ, HKV, lens_d, window, kc, vc, CAP, HKV * CAP * 64, out, HQ * 64,
                            0.125)
        torch.cuda.synchronize()
        got = out.cpu().numpy().reshape(B, HQ, 64)
        for b in range(B):
            want = O.attention_f64(q[b].reshape(HQ, 64), kc0[b], vc0[b], int(lens[b]) - 1, window, 0.125)
            ex, i, g, w = O.worst_violation(got[b], want, 2e-5)
            assert ex <= 0, f"window {window} b={b} index {i} got {g} want {w}"


@pytest.mark.parametrize("ct,cap,window", [(np.float32, 512, 0), (np.float16, 512, 65), (np.float16, 2048, 0),
                                           (np.float32, 4096, 200), (np.float16, 4096, 0)])
def test_decode_lengths_caches_and_windows(gpu, ct, cap, window):
    """mt_attention_decode over 8 sequences whose lengths straddle the kernel's 32-key score
    passes and 512-key rounds (0, 1, 63 .. 129, the cache's end) on caches of 512 to 4096
    positions, with and without a window; a sequence without keys gets zeros.  Against the
    fp64 oracle on the stored cache values; a second run gives the same bits."""
    lens = np.array([0, 1, 63, 64, 65, 129, cap - 1, cap], np.uint32)
    B = len(lens)
    z = O.gaussian(cap + window, B * HKV * cap * 64 * 2 + B * HQ * 64)
    kc0 = z[:B * HKV * cap * 64].reshape(B, HKV, cap, 64).astype(ct)
    vc0 = z[B * HKV * cap * 64:2 * B * HKV * cap * 64].reshape(B, HKV, cap, 64).astype(ct)
    q = z[2 * B * HKV * cap * 64:].reshape(B, HQ * 64)
    kc = torch.from_numpy(kc0.copy()).to(gpu)
    vc = torch.from_numpy(vc0.copy()).to(gpu)
    qd = torch.from_numpy(q.copy()).to(gpu)
    lens_d = torch.from_numpy(lens.astype(np.int32)).to(gpu)
    runs = []
    for r in range(2):
        out = torch.full((B, HQ * 64), 7.0, device=gpu)
        say(f"decode lengths ct={np.dtype(ct).name} cap={cap} window={window} run {r}")
        mt.attention_decode(qd, HQ * 64, B, HQ, HKV, lens_d, window, kc, vc, cap, HKV * cap * 64, out, HQ * 64, 0.125)
        torch.cuda.synchronize()
        runs.append(out.cpu().numpy().reshape(B, HQ, 64))
    np.testing.assert_array_equal(runs[0], runs[1])
    got = runs[0]
    for b in range(B):
        if lens[b] == 0:
            np.testing.assert_array_equal(got[b], np.zeros((HQ, 64), np.float32))
            continue
        want = O.attention_f64(q[b].reshape(HQ, 64), kc0[b].astype(np.float64), vc0[b].astype(np.float64),
                               int(lens[b]) - 1, window, 0.125)
        ex, i, g, w = O.worst_violation(got[b], want, 2e-5)
        assert ex <= 0, f"len {lens[b]} index {i} got {g} want {w}"


@pytest.mark.parametrize("ct,M,pos0,window,cap", [
    (torch.float16, 4, 200, 65, 512),    # one VAE latent's sliding-window rows
    (torch.float32, 4, 200, 65, 512),
    (torch.float16, 3, 0, 0, 64),        # no cached keys yet, unlimited window
    (torch.float32, 1, 37, 1, 64),       # a window of the row itself
    (torch.float16, 16, 100, 0, 256),    # 16 rows, unlimited window
    (torch.float16, 8, 504, 9, 512),     # positions up to the cache's end, window inside the chunk
])
def test_rope_attention_equals_rope_cache_then_attention(gpu, ct, M, pos0, window, cap):
    """mt_rope_attention against mt_rope_cache then mt_attention on copies of the same qkv and
    caches: the same out, the same rotated q in qkv, the same cache rows, bit for bit."""
    rng = np.random.default_rng(M * 1000 + pos0 + window)
    qkv = rng.standard_normal((M, LD)).astype(np.float32)
    kc0 = rng.standard_normal((HKV, cap, 64)).astype(np.float32)
    vc0 = rng.standard_normal((HKV, cap, 64)).astype(np.float32)
    invf = torch.from_numpy(O.inv_freq(1e6)).to(gpu)
    t = lambda a, dt=torch.float32: torch.from_numpy(a.copy()).to(gpu).to(dt)
    q1, k1, v1 = t(qkv), t(kc0, ct), t(vc0, ct)
    q2, k2, v2 = t(qkv), t(kc0, ct), t(vc0, ct)
    o1 = torch.full((M, HQ * 64), 5.0, device=gpu)
    o2 = torch.full((M, HQ * 64), 5.0, device=gpu)
    say(f"rope_attention ct={ct} M={M} pos0={pos0} window={window} cap={cap}")
    mt.rope_cache(q1, LD, M, HQ, HKV, pos0, k1, v1, cap, invf)
    mt.attention(q1, LD, M, HQ, HKV, pos0, window, k1, v1, cap, o1, HQ * 64, 0.125)
    mt.rope_attention(q2, LD, M, HQ, HKV, pos0, window, k2, v2, cap, invf, o2, HQ * 64, 0.125)
    torch.cuda.synchronize()
    for a, b, what in ((o1, o2, "out"), (q1, q2, "qkv"), (k1, k2, "k cache"), (v1, v2, "v cache")):
        np.testing.assert_array_equal(a.cpu().numpy(), b.cpu().numpy(), err_msg=what)


@pytest.mark.parametrize("ct,M,pos0,window", [
    (torch.float16, 174, 0, 0),     # the reference's prefill prompt
    (torch.float32, 174, 0, 0),
    (torch.float16, 8, 0, 0),       # the fewest rows that go by blocks
    (torch.float32, 13, 37, 0),     # a ragged last block after cached keys
    (torch.float16, 301, 700, 0),   # rows of up to 1001 keys: four sum slots a thread
    (torch.float32, 61, 3, 64),     # a window longer than every row's span
    (torch.float16, 124, 900, 0),   # pos0 + M = 1024, the most keys that go by blocks
    (torch.float32, 40, 50, 70),    # a window shorter than the last rows' spans: row by row
])
def test_row_blocks_equal_rows_one_at_a_time(gpu, ct, M, pos0, window):
    """mt_attention over M rows of one sequence (a workgroup per head and block of rows)
    against the same rows attended one call each (a workgroup per row and head): the same
    bits; and sampled rows against the fp64 oracle on the stored cache values."""
    cap = 1024
    rng = np.random.default_rng(M * 7 + pos0)
    q = rng.standard_normal((M, HQ * 64)).astype(np.float32)
    kc = torch.from_numpy(rng.standard_normal((HKV, cap, 64)).astype(np.float32)).to(gpu).to(ct)
    vc = torch.from_numpy(rng.standard_normal((HKV, cap, 64)).astype(np.float32)).to(gpu).to(ct)
    qd = torch.from_numpy(q).to(gpu)
    o1 = torch.full((M, HQ * 64), 7.0, device=gpu)
    o2 = torch.full((M, HQ * 64), 7.0, device=gpu)
    say(f"row blocks ct={ct} M={M} pos0={pos0} window={window}")
    mt.attention(qd, HQ * 64, M, HQ, HKV, pos0, window, kc, vc, cap, o1, HQ * 64, 0.125)
    for m in range(M):
        mt.attention(qd[m:], HQ * 64, 1, HQ, HKV, pos0 + m, window, kc, vc, cap, o2[m:], HQ * 64, 0.125)
    torch.cuda.synchronize()
    got = o1.cpu().numpy()
    np.testing.assert_array_equal(got, o2.cpu().numpy())
    kcg = kc.double().cpu().numpy()
    vcg = vc.double().cpu().numpy()
    for m in sorted({0, 1, M // 2, M - 2, M - 1}):
        want = O.attention_f64(q[m].reshape(HQ, 64), kcg, vcg, pos0 + m, window, 0.125)
        ex, i, g, w = O.worst_violation(got[m].reshape(HQ, 64), want, 2e-5)
        assert ex <= 0, f"row {m} index {i} got {g} want {w}"


def test_rope_attention_rejects_bad_arguments():
    L = mt.load()
    A = 1 << 20
    assert L.mt_rope_attention(A, LD, 65, HQ, HKV, 0, 0, A, A, mt.F16, 512, A, A + (1 << 24), HQ * 64, 0.125, None) \
        == mt.EINVAL and "at most 64 rows" in mt.last_error()
    assert L.mt_rope_attention(A, LD, 4, HQ, HKV, 510, 0, A, A, mt.F16, 512, A, A + (1 << 24), HQ * 64, 0.125, None) \
        == mt.EINVAL and "past cache_len" in mt.last_error()
    assert L.mt_rope_attention(A, LD, 4, HQ, HKV, 0, 0, A, A, mt.F16, 512, A, A + 64, HQ * 64, 0.125, None) \
        == mt.EINVAL and "overlaps" in mt.last_error()
    assert L.mt_rope_attention(A, LD, 0, HQ, HKV, 0, 0, A, A, mt.F16, 512, A, A, HQ * 64, 0.125, None) == mt.OK
