"""The flow sampler's host arithmetic (FlowSchedule, DiT.swift:55-80): the product's fp32
schedule and sinusoid against the oracle's fp64 closed forms, the oracle against textbook
values, and the sinusoid against torch's SinusPositionEmbedding formula."""
import math

import numpy as np
import pytest
import torch

import mingtts as mt
import oracle as O

STEP_COUNTS = [1, 3, 5, 6, 7, 8, 10, 12, 16]


def test_oracle_timesteps_are_one_minus_cos_of_the_grid():
    """The sway -1 map t - (cos(pi/2 t) - 1 + t) is 1 - cos(pi/2 t): at the 10-step EPSS grid
    points 1/4, 1/2 and 3/4 that is 1 - cos(pi/8), 1 - cos(pi/4), 1 - cos(3 pi/8), whose
    values follow from the half-angle formulas.  A flipped sway sign (2t + cos - 1) would give
    0.707 at t = 1/2 instead of 0.293."""
    ts = O.flow_timesteps_f64(10)
    assert ts[0] == 0.0 and abs(ts[-1] - 1.0) < 1e-15
    assert ts[4] == pytest.approx(1 - math.sqrt(2 + math.sqrt(2)) / 2, abs=1e-15)   # grid 8/32
    assert ts[6] == pytest.approx(1 - math.sqrt(2) / 2, abs=1e-15)                 # grid 16/32
    assert ts[8] == pytest.approx(1 - math.sqrt(2 - math.sqrt(2)) / 2, abs=1e-15)  # grid 24/32
    u = O.flow_timesteps_f64(8)  # not in the EPSS table: uniform grid k / 8
    assert u[4] == pytest.approx(1 - math.sqrt(2) / 2, abs=1e-15)
    assert u[2] == pytest.approx(1 - math.sqrt(2 + math.sqrt(2)) / 2, abs=1e-15)


@pytest.mark.parametrize("steps", STEP_COUNTS)
def test_timesteps_match_the_closed_form(steps):
    got = mt.FlowSchedule.timesteps(steps)
    want = O.flow_timesteps_f64(steps)
    assert got.dtype == np.float32 and got.shape == (steps + 1,)
    assert got[0] == 0.0 and got[-1] == 1.0
    assert np.all(np.diff(got) > 0)
    np.testing.assert_allclose(got, want, rtol=0, atol=3e-7)


def test_timesteps_refuse_no_steps():
    with pytest.raises(ValueError):
        mt.FlowSchedule.timesteps(0)


def test_oracle_sinusoid_closed_form():
    """Slot 0 has frequency 1 and slot 127 frequency 1e-4: sin(1000 t) and sin(0.1 t), with the
    cosines 128 slots later; every sin/cos pair lies on the unit circle."""
    for t in (0.0, 0.004815, 0.5, 1.0):
        s = O.sinusoid_f64(t)
        assert s.shape == (256,)
        assert s[0] == pytest.approx(math.sin(1000 * t), abs=1e-12)
        assert s[128] == pytest.approx(math.cos(1000 * t), abs=1e-12)
        assert s[127] == pytest.approx(math.sin(0.1 * t), abs=1e-12)
        np.testing.assert_allclose(s[:128] ** 2 + s[128:] ** 2, 1.0, rtol=0, atol=1e-12)


def _torch_sinusoid(t: float) -> np.ndarray:
    """The SinusPositionEmbedding formula the reference restates, in torch fp32 on the CPU:
    exp(arange(half) * -(ln(1e4) / (half - 1))), scaled by 1000 t, then [sin, cos]."""
    half = 128
    emb = math.log(10000) / (half - 1)
    emb = torch.exp(torch.arange(half, dtype=torch.float32) * -emb)
    emb = 1000.0 * torch.tensor([t], dtype=torch.float32).unsqueeze(1) * emb.unsqueeze(0)
    return torch.cat((emb.sin(), emb.cos()), dim=-1)[0].numpy()


@pytest.mark.parametrize("k", range(10))
def test_sinusoid_matches_torch_and_fp64(k):
    """At the 10-step schedule's times.  The argument reaches 1000, where one fp32 rounding of
    it moves sin by up to 6e-5, so the bound is 2e-4; a wrong frequency denominator (128 for
    127) or scale moves slots by O(1)."""
    t = float(mt.FlowSchedule.timesteps(10)[k])
    got = mt.FlowSchedule.sinusoid(t)
    assert got.dtype == np.float32 and got.shape == (256,)
    np.testing.assert_allclose(got, O.sinusoid_f64(t), rtol=0, atol=2e-4)
    np.testing.assert_allclose(got, _torch_sinusoid(t), rtol=0, atol=2e-4)
    if t == 0.0:
        assert np.all(got[:128] == 0.0) and np.all(got[128:] == 1.0)


def test_oracle_fails_a_planted_sinusoid_mistake():
    """The comparison above has teeth: the oracle with the frequency denominator 128 instead
    of 127 differs from the product by far more than the bound at t = 0.5."""
    t = 0.5
    a = 1000 * t * np.exp(-np.arange(128) * math.log(10000.0) / 128)
    wrong = np.concatenate([np.sin(a), np.cos(a)])
    assert np.max(np.abs(mt.FlowSchedule.sinusoid(t) - wrong)) > 0.1
