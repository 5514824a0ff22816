"""The LLM decode step paired with a VAE latent (MingEngine.encodeStep, Engine.swift:377-385;
QwenForward.encodePaired, Qwen.swift:103-115): the persistent decode sequence on one stream
and a VAE latent's launches (upsample4, the M = 4 sliding-window layers, captured in a HIP
graph) on a second stream at the same time give the same bits as the two run one after the
other, on every round, and the decode part matches its fp64 chain."""
import numpy as np
import pytest
import torch

import mingtts as mt
import oracle as O
from _gpu_util import say

pytestmark = pytest.mark.gpu

H, QKV, INTER, HQ, HKV, CAP = 896, 1152, 4864, 14, 2, 512


def _layers(g, dev, n):
    w = lambda *s: (torch.randn(*s, generator=g, device=dev) * 0.02).half()
    gain = lambda k: (1.0 + 0.1 * torch.randn(k, generator=g, device=dev)).half()
    return [dict(qkv=w(QKV, H), qkv_b=w(QKV), o=w(H, H), gate=w(INTER, H), up=w(INTER, H), down=w(H, INTER),
                 norm1=gain(H), norm2=gain(H)) for _ in range(n)]


def test_decode_paired_with_vae_latent_matches_serial(gpu):
    g = torch.Generator(device=gpu)
    g.manual_seed(17)
    llm, vae = _layers(g, gpu, 2), _layers(g, gpu, 2)
    M = 2
    resid = torch.randn(M, H, generator=g, device=gpu)
    x0 = resid.clone()
    qkv = torch.zeros(M, QKV, device=gpu)
    mlp = torch.zeros(M, INTER, device=gpu)
    ops = []
    for p in llm:
        ops.append(mt.op(resid, p["qkv"], qkv, M, bias=p["qkv_b"], norm=p["norm1"]))
        ops.append(mt.op(qkv, p["o"], resid, M, flags=mt.GemvFlags.accumulate, ldx=QKV))
        ops.append(mt.op(resid, p["gate"], mlp, M, flags=mt.GemvFlags.siluGate, w2=p["up"], norm=p["norm2"]))
        ops.append(mt.op(mlp, p["down"], resid, M, flags=mt.GemvFlags.accumulate))
    seq = mt.Seq(ops)

    # The VAE latent: 4 frames from three fc1 rows, then the layers at M = 4.
    hrows = [torch.randn(H, generator=g, device=gpu) for _ in range(3)]
    frames = torch.zeros(4, H, device=gpu)
    vqkv = torch.zeros(4, QKV, device=gpu)
    att = torch.zeros(4, HQ * 64, device=gpu)
    vmlp = torch.zeros(4, INTER, device=gpu)
    caches = [(torch.randn(HKV, CAP, 64, generator=g, device=gpu).half(),
               torch.randn(HKV, CAP, 64, generator=g, device=gpu).half()) for _ in vae]
    i = torch.arange(32, device=gpu, dtype=torch.float32)
    invf = (1.0 / torch.pow(torch.tensor(1e6, device=gpu), 2.0 * i / 64.0)).float()
    sv = torch.cuda.Stream(device=gpu)

    def latent():
        s = sv.cuda_stream
        mt.upsample4(hrows[0], hrows[1], hrows[2], frames, stream=s)
        for p, (kc, vc) in zip(vae, caches):
            mt.linear(frames, p["qkv"], vqkv, 4, bias=p["qkv_b"], norm=p["norm1"], stream=s)
            mt.rope_attention(vqkv, QKV, 4, HQ, HKV, 200, 65, kc, vc, CAP, invf, att, HQ * 64, stream=s)
            mt.linear(att, p["o"], frames, 4, flags=mt.GemvFlags.accumulate, stream=s)
            mt.linear(frames, p["gate"], vmlp, 4, flags=mt.GemvFlags.siluGate, w2=p["up"], norm=p["norm2"], stream=s)
            mt.linear(vmlp, p["down"], frames, 4, flags=mt.GemvFlags.accumulate, stream=s)

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(sv):
        latent()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=sv):
            latent()
    torch.cuda.synchronize()
    sa = torch.cuda.Stream(device=gpu)

    def run(paired: bool):
        with torch.cuda.stream(sa):
            resid.copy_(x0)
            start = torch.cuda.Event()
            start.record()
            if paired:
                sv.wait_event(start)
                seq.run(sa)
                with torch.cuda.stream(sv):
                    graph.replay()
                    done = torch.cuda.Event()
                    done.record()
                sa.wait_event(done)
            else:
                seq.run(sa)
                graph.replay()
        torch.cuda.synchronize()
        seq.check()
        return resid.cpu().numpy(), frames.cpu().numpy()

    say("pairing: serial reference run")
    want_r, want_f = run(False)
    for r in range(3):
        say(f"pairing: paired round {r}")
        got_r, got_f = run(True)
        np.testing.assert_array_equal(got_r, want_r)
        np.testing.assert_array_equal(got_f, want_f)

    # The decode part against its fp64 chain (fp32 between ops).
    hw = [{k: v.cpu().numpy().view(np.uint16) for k, v in p.items()} for p in llm]
    x = x0.cpu().numpy()
    for p in hw:
        q = O.linear_np64(O.rmsnorm_f64(x, p["norm1"], O.F16), p["qkv"], None, O.F16, p["qkv_b"], None,
                          O.BIAS).astype(np.float32)
        x = O.linear_f64(np.ascontiguousarray(q[:, :H]), p["o"], None, O.F16, None, x, M, H, H,
                         O.ACCUM).astype(np.float32)
        m = O.linear_np64(O.rmsnorm_f64(x, p["norm2"], O.F16), p["gate"], p["up"], O.F16, None, None,
                          O.SILU_GATE).astype(np.float32)
        x = O.linear_f64(m, p["down"], None, O.F16, None, x, M, H, INTER, O.ACCUM).astype(np.float32)
    assert O.normwise_rel_err(want_r, x) <= 1e-3
    seq.close()
    del graph
