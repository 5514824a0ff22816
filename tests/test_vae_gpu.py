"""The VAE decoder's tail on the GPU (Shaders.swift:697-790): the reference's own known-answer
tests (KernelTests.testIstftMatchesDirectOverlapAdd and testUpsampleMatchesTorchLinear,
KernelTests.swift:322-398) regenerated bit for bit from the KAT RNG, and the frame ring
wrapping around."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import mingtts as mt
import oracle as O
from _gpu_util import say

pytestmark = pytest.mark.gpu

NFFT, HOP = 3528, 882
BINS = NFFT // 2 + 1


def _tables():
    window = np.array([0.5 - 0.5 * np.cos(2 * np.pi * t / NFFT) for t in range(NFFT)], np.float32)
    cos_table = np.array([np.cos(2 * np.pi * t / NFFT) for t in range(NFFT)], np.float32)
    return window, cos_table


def _spec(frames, state):
    rng = O.LCG(state)
    spec = np.zeros((frames, 2 * BINS), np.float32)
    for f in range(frames):   # the reference's draw order: per frame, per bin, magnitude then phase
        for k in range(BINS):
            spec[f, k] = rng.floats(1)[0] * 2 - 1
            spec[f, BINS + k] = rng.floats(1)[0] * 3
    return spec


def test_istft_reference_kat(gpu):
    """8 frames from the KAT RNG (state 5) through two frame calls and three emit calls, as the
    reference test drives them, against the direct overlap-add; atol 2e-5 x scale, rtol 1e-4."""
    frames, ring = 8, 8
    spec = _spec(frames, 5)
    window, cos_table = _tables()
    d = lambda a: torch.from_numpy(a).to(gpu)
    spec_d, win_d, cos_d = d(spec), d(window), d(cos_table)
    ring_d = torch.zeros(ring, NFFT, device=gpu)
    pad = (NFFT - HOP) // 2
    total = frames * HOP
    out = torch.zeros(total, device=gpu)
    say("istft KAT")
    mt.istft_frames(spec_d[0:4], 4, NFFT, cos_d, win_d, ring_d, 0, ring)
    mt.istft_emit(ring_d, win_d, NFFT, HOP, 0, 4 * HOP - pad, 3, ring, out[0:])
    mt.istft_frames(spec_d[4:8], 4, NFFT, cos_d, win_d, ring_d, 4, ring)
    mt.istft_emit(ring_d, win_d, NFFT, HOP, 4 * HOP - pad, 4 * HOP, 7, ring, out[4 * HOP - pad:])
    mt.istft_emit(ring_d, win_d, NFFT, HOP, 8 * HOP - pad, pad, 7, ring, out[8 * HOP - pad:])
    torch.cuda.synchronize()
    fr = [O.istft_frame_f64(spec[f], NFFT, window) for f in range(frames)]
    want = O.istft_emit_f64(fr, window, NFFT, HOP, 0, total, frames - 1)
    got = out.cpu().numpy()
    scale = np.max(np.abs(want))
    ex, i, g, w = O.worst_violation(got, want, 2e-5 * scale, 1e-4)
    assert ex <= 0, f"index {i} got {g} want {w}"
    # the frames themselves, before the overlap-add
    np.testing.assert_allclose(ring_d.cpu().numpy()[7], fr[7], rtol=0, atol=2e-5 * np.max(np.abs(fr[7])))


def test_istft_ring_wraps(gpu):
    """Frames 6..9 of an 8-slot ring land in slots 6, 7, 0, 1."""
    spec = _spec(4, 21)
    window, cos_table = _tables()
    d = lambda a: torch.from_numpy(a).to(gpu)
    ring_d = torch.full((8, NFFT), 5.0, device=gpu)
    say("istft ring wrap")
    mt.istft_frames(d(spec), 4, NFFT, d(cos_table), d(window), ring_d, 6, 8)
    torch.cuda.synchronize()
    got = ring_d.cpu().numpy()
    for f, slot in enumerate((6, 7, 0, 1)):
        want = O.istft_frame_f64(spec[f], NFFT, window)
        np.testing.assert_allclose(got[slot], want, rtol=0, atol=2e-5 * np.max(np.abs(want)))
    assert np.all(got[2:6] == 5.0)


def test_upsample_reference_kat(gpu):
    """testUpsampleMatchesTorchLinear: 5 latents of 896 (KAT RNG state 9), each upsampled with
    its neighbours, against torch's linear interpolation over the whole sequence."""
    hidden, n = 896, 5
    rng = O.LCG(9)
    h = [rng.floats(hidden) for _ in range(n)]
    hb = [torch.from_numpy(x).to(gpu) for x in h]
    out = torch.zeros(n * 4, hidden, device=gpu)
    say("upsample KAT")
    for i in range(n):
        mt.upsample4(hb[i - 1] if i > 0 else None, hb[i], hb[i + 1] if i + 1 < n else None, out[4 * i:4 * i + 4])
    torch.cuda.synchronize()
    seq = torch.from_numpy(np.stack(h).T[None].astype(np.float64))
    want = F.interpolate(seq, scale_factor=4, mode="linear", align_corners=False)[0].T.numpy()
    np.testing.assert_allclose(out.cpu().numpy(), want, rtol=1e-6, atol=1e-6)
    one = torch.zeros(4, hidden, device=gpu)
    mt.upsample4(None, hb[0], None, one)   # a lone latent: four copies
    torch.cuda.synchronize()
    np.testing.assert_array_equal(one.cpu().numpy(), np.stack([h[0]] * 4))
