"""Host side of the flow sampler around the DiT linears: the CFM timestep schedule and the
timestep embedding (FlowSchedule, Sources/MingTTS/Engine/DiT.swift:55-80), and the time-MLP
precompute that turns the embeddings into the per-step ``temb`` rows
(MingEngine.precomputeTimeEmbeddings, Sources/MingTTS/Engine/Engine.swift:186-198).

The schedule and the sinusoid are host arithmetic in the reference too (fp32, computed once
per engine); the two time-MLP linears run on the GPU through mt_linear.
"""
from __future__ import annotations

import math

import numpy as np


class FlowSchedule:
    """FlowSchedule (DiT.swift:55-80)."""

    # EPSS base timesteps in 32nds, per step count (the reference's table, DiT.swift:58-62);
    # other step counts use a uniform grid.
    EPSS = {
        5: (0, 2, 4, 8, 16, 32),
        6: (0, 2, 4, 6, 8, 16, 32),
        7: (0, 2, 4, 6, 8, 16, 24, 32),
        10: (0, 2, 4, 6, 8, 12, 16, 20, 24, 28, 32),
        12: (0, 2, 4, 6, 8, 10, 12, 14, 16, 20, 24, 28, 32),
        16: (0, 1, 2, 3, 4, 5, 6, 7, 8, 10, 12, 14, 16, 20, 24, 28, 32),
    }
    WIDTH = 256  # SinusPositionEmbedding(256)
    SCALE = 1000.0

    @staticmethod
    def timesteps(steps: int) -> np.ndarray:
        """steps + 1 fp32 times from 0 to 1: the EPSS grid (or a uniform one) bent by the sway
        coefficient -1, t - (cos(pi/2 t) - 1 + t), evaluated in fp32 in that order
        (DiT.swift:57-65)."""
        if steps < 1:
            raise ValueError(f"FlowSchedule.timesteps: steps {steps} < 1")
        if steps in FlowSchedule.EPSS:
            base = np.asarray(FlowSchedule.EPSS[steps], np.float32) / np.float32(32)
        else:
            base = np.arange(steps + 1, dtype=np.float32) / np.float32(steps)
        half_pi = np.float32(math.pi / 2)
        inner = (np.cos(half_pi * base) - np.float32(1)) + base
        return (base - inner).astype(np.float32)

    @staticmethod
    def sinusoid(t: float) -> np.ndarray:
        """The 256-wide timestep embedding at scale 1000 (DiT.swift:67-79): frequencies
        exp(-i ln(1e4) / 127) in fp32, argument (1000 t) * freq in fp32, sines in the first
        128 slots and cosines in the last 128, each evaluated in double and rounded."""
        half = FlowSchedule.WIDTH // 2
        step = np.float32(math.log(10000.0) / (half - 1))
        freq = np.exp(np.arange(half, dtype=np.float32) * -step).astype(np.float32)
        arg = (np.float32(FlowSchedule.SCALE) * np.float32(t)) * freq
        a64 = arg.astype(np.float64)
        return np.concatenate([np.sin(a64), np.cos(a64)]).astype(np.float32)

    @staticmethod
    def sinusoids(times) -> np.ndarray:
        """sinusoid of each time, one row each: [len(times), 256] fp32."""
        return np.stack([FlowSchedule.sinusoid(float(t)) for t in times]).astype(np.float32)


def time_embeddings(time1, time2, timesteps, stream=None):
    """MingEngine.precomputeTimeEmbeddings (Engine.swift:186-198): the sinusoid of each flow
    timestep but the last (one row per ODE step) through ``time1`` (256 -> 1024, SiLU) and
    ``time2`` (1024 -> 1024) on the GPU, two mt_linear launches at M = steps.  ``time1`` and
    ``time2`` are (w [N, K], bias [N]) pairs of device tensors; returns temb [steps, N2] fp32
    on the weights' device, enqueued on ``stream``."""
    import torch

    from . import GemvFlags, linear

    (w1, b1), (w2, b2) = time1, time2
    steps = len(timesteps) - 1
    dev = w1.device
    sinus = torch.from_numpy(FlowSchedule.sinusoids(timesteps[:steps])).to(dev)
    mid = torch.empty(steps, w1.shape[0], device=dev, dtype=torch.float32)
    temb = torch.empty(steps, w2.shape[0], device=dev, dtype=torch.float32)
    linear(sinus, w1, mid, steps, flags=GemvFlags.silu, bias=b1, stream=stream)
    linear(mid, w2, temb, steps, bias=b2, stream=stream)
    return temb
