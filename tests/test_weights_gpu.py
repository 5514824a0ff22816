"""The weight path on the GPU: a WeightArena uploaded from a .safetensors file holds every
planned tensor's bytes at its offset (concatenations in order, padded columns and
placement gaps zero); converted to fp16 it holds torch's round-to-nearest-even conversion
of the bf16 values bit for bit, with the audit counting the values that became +-inf and
the nonzero values that became zero; and a Qwen layer loaded the reference's way
(QwenWeights, Weights.swift:115-130) runs through Encoder.linear against the oracle."""
import numpy as np
import pytest
import torch
from safetensors.torch import save_file

import mingtts as mt
import oracle as O
from _gpu_util import say

pytestmark = pytest.mark.gpu


def _bytes(t):
    return t.contiguous().view(torch.uint8).reshape(-1).cpu().numpy()


def test_upload_places_every_tensor(gpu, tmp_path):
    g = torch.Generator().manual_seed(2)
    ts = {"q": torch.randn(24, 64, generator=g).bfloat16(), "k": torch.randn(8, 64, generator=g).bfloat16(),
          "v": torch.randn(8, 64, generator=g).bfloat16(), "b": torch.randn(40, generator=g).bfloat16(),
          "pad.weight": torch.randn(5, 20, generator=g).bfloat16()}
    path = str(tmp_path / "w.safetensors")
    save_file(ts, path)
    st = mt.SafeTensors(path)
    arena = mt.WeightArena(st)
    qkv = arena.tensor("q", "k", "v")
    b = arena.tensor("b")
    pad = arena.padded_linear("pad", 5, 24, 20)
    say("arena upload bf16")
    arena.upload(gpu)
    dev = arena.buffer.cpu().numpy()
    want = np.zeros(arena.nbytes, np.uint8)
    cat = np.concatenate([_bytes(ts["q"]), _bytes(ts["k"]), _bytes(ts["v"])])
    want[qkv.offset:qkv.offset + cat.size] = cat
    want[b.offset:b.offset + 80] = _bytes(ts["b"])
    padded = np.zeros((5, 24), np.uint16)
    padded[:, :20] = ts["pad.weight"].view(torch.int16).numpy().view(np.uint16)
    want[pad.w.offset:pad.w.offset + padded.nbytes] = padded.view(np.uint8).reshape(-1)
    np.testing.assert_array_equal(dev[:arena.nbytes], want)
    assert arena.audit() == (0, 0)
    arena.close()
    st.close()


def test_fp16_conversion_and_audit(gpu, tmp_path):
    """bf16 -> fp16 in place: bit-identical to torch's conversion; the audit counts finite
    values past the fp16 range and nonzero values below half its smallest subnormal."""
    rng = np.random.default_rng(9)
    vals = np.concatenate([rng.standard_normal(5000) * 0.05, [7e4, -1e5, 65504.0, 65520.0, 3e38, np.inf, -np.inf],
                           [1e-8, -3e-8, 5.96e-8, 2.9e-8, 1e-30, 0.0, -0.0], rng.standard_normal(997) * 300.0])
    t = torch.from_numpy(vals.astype(np.float32)).bfloat16()
    path = str(tmp_path / "c.safetensors")
    save_file({"w": t.reshape(-1)}, path)
    st = mt.SafeTensors(path)
    arena = mt.WeightArena(st, convert_to=mt.F16)
    w = arena.tensor("w")
    say("arena upload bf16 -> fp16")
    arena.upload(gpu)
    got = arena.buffer[w.offset:w.offset + 2 * w.count].view(torch.float16).cpu()
    want = t.to(torch.float16)
    np.testing.assert_array_equal(got.view(torch.int16).numpy(), want.view(torch.int16).numpy())
    tf = t.float()
    wf = want.float()
    overflow = int((torch.isfinite(tf) & torch.isinf(wf)).sum())
    underflow = int(((tf != 0) & (wf == 0)).sum())
    assert arena.audit() == (overflow, underflow) and overflow >= 4 and underflow >= 3
    arena.close()
    st.close()


def test_qwen_layer_from_a_checkpoint_file(gpu, tmp_path):
    """One Qwen2 layer's tensors under the checkpoint's names, loaded as QwenWeights does
    (q, k, v rows and biases concatenated), then qkv through Encoder.linear."""
    H, KV, I = 896, 128, 4864
    g = torch.Generator().manual_seed(4)
    p = "model.layers.0"
    names = {f"{p}.self_attn.q_proj.weight": (H, H), f"{p}.self_attn.k_proj.weight": (KV, H),
             f"{p}.self_attn.v_proj.weight": (KV, H), f"{p}.self_attn.q_proj.bias": (H,),
             f"{p}.self_attn.k_proj.bias": (KV,), f"{p}.self_attn.v_proj.bias": (KV,),
             f"{p}.self_attn.o_proj.weight": (H, H), f"{p}.mlp.gate_proj.weight": (I, H),
             f"{p}.mlp.up_proj.weight": (I, H), f"{p}.mlp.down_proj.weight": (H, I),
             f"{p}.input_layernorm.weight": (H,), f"{p}.post_attention_layernorm.weight": (H,)}
    ts = {n: (torch.randn(*s, generator=g) * 0.02).bfloat16() for n, s in names.items()}
    path = str(tmp_path / "qwen.safetensors")
    save_file(ts, path)
    st = mt.SafeTensors(path)

    def build(a):
        qkv_w = a.tensor(f"{p}.self_attn.q_proj.weight", f"{p}.self_attn.k_proj.weight", f"{p}.self_attn.v_proj.weight")
        qkv_b = a.tensor(f"{p}.self_attn.q_proj.bias", f"{p}.self_attn.k_proj.bias", f"{p}.self_attn.v_proj.bias")
        return dict(qkv=mt.Linear(qkv_w, qkv_b, H + 2 * KV, H), o=a.linear(f"{p}.self_attn.o_proj", H, H, False),
                    gate=a.linear(f"{p}.mlp.gate_proj", I, H, False), up=a.linear(f"{p}.mlp.up_proj", I, H, False),
                    down=a.linear(f"{p}.mlp.down_proj", H, I, False))

    say("qwen layer from a checkpoint file")
    layer, arena = mt.WeightArena.load(st, build, device=gpu)
    x = O.LCG(5).floats(2 * H).reshape(2, H)
    xb = torch.from_numpy(x).to(gpu)
    y = torch.zeros(2, H + 2 * KV, device=gpu)
    mt.Encoder().linear(mt.ActView(xb, ld=H), 2, layer["qkv"], mt.ActView(y, ld=H + 2 * KV))
    torch.cuda.synchronize()
    w = torch.cat([ts[f"{p}.self_attn.{n}_proj.weight"] for n in "qkv"]).view(torch.int16).numpy().view(np.uint16)
    b = torch.cat([ts[f"{p}.self_attn.{n}_proj.bias"] for n in "qkv"]).view(torch.int16).numpy().view(np.uint16)
    want = O.linear_f64(x, w, None, O.BF16, b, None, 2, H + 2 * KV, H, 0)
    assert O.normwise_rel_err(y.cpu().numpy(), want) <= 1e-5
    arena.close()
    st.close()
