"""Writes tests/golden/checkpoint_small.safetensors: a small two-layer hybrid decoder's W4 linears in the two
on-disk forms the checkpoint reader takes, plus ineligible linears (one per check) and a dense tensor.

hidden 256, intermediate 256, 2 q heads / 1 kv head of 128, GDN 1 key head / 2 value heads of 128;
layer 0 Gated-DeltaNet, layer 1 attention (attn_every 2). GPTQ tensors (AutoGPTQ layout, "gptq" v1
zero - 1 storage, group 128, symmetric) for every linear of the two layers; comfy-kitchen-style W4A8
tensors (codes int8 [N, K/2], fp8 e4m3 group-16 scales, s_channel, codebook) under `w4a8.*`.
Seeded; run from the repository root: python tests/golden/make_checkpoint_fixture.py"""
import os

import torch
from safetensors.torch import save_file

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "checkpoint_small.safetensors")


def pack_int32(codes, axis):
    """int codes 0..15 -> int32 words of 8 codes (code j of a word in bits 4 j..4 j + 3) along `axis`."""
    c = codes.to(torch.int64)
    if axis == 0:
        c = c.reshape(c.shape[0] // 8, 8, c.shape[1])
        w = sum(c[:, j, :] << (4 * j) for j in range(8))
    else:
        c = c.reshape(c.shape[0], c.shape[1] // 8, 8)
        w = sum(c[:, :, j] << (4 * j) for j in range(8))
    return ((w + 2 ** 31) % 2 ** 32 - 2 ** 31).to(torch.int32)


def gptq(g, N, K, G=128, zero=8, act_order=False):
    codes = torch.randint(0, 16, (K, N), generator=g)
    scales = (torch.rand(K // G, N, generator=g) * 0.015 + 0.005).half()
    zeros = torch.full((K // G, N), zero - 1)  # v1 storage: zero - 1
    g_idx = torch.arange(K, dtype=torch.int32) // G
    if act_order:
        g_idx = g_idx[torch.randperm(K, generator=g)]
    return {"qweight": pack_int32(codes, 0), "qzeros": pack_int32(zeros, 1), "scales": scales, "g_idx": g_idx}


def w4a8(g, N, K, bad_scale=False):
    codes = torch.randint(-128, 128, (N, K // 2), generator=g).to(torch.int8)
    scale = (torch.rand(N, K // 16, generator=g) * 2 + 0.25).to(torch.float8_e4m3fn)
    if bad_scale:
        scale[0, 0] = -1.0
    return {"weight": codes, "weight_scale": scale, "s_channel": torch.rand(N, generator=g) * 0.01 + 0.001,
            "codebook": torch.arange(-8, 8, dtype=torch.float32)}


def main():
    g = torch.Generator().manual_seed(20)
    H, I, qd, kd, ch, hv = 256, 256, 256, 128, 512, 256
    t = {}

    def put(prefix, d):
        for k, v in d.items():
            t[f"{prefix}.{k}"] = v.contiguous()

    for name, (N, K) in {"linear_attn.in_proj_qkv": (ch, H), "linear_attn.in_proj_z": (hv, H),
                         "linear_attn.out_proj": (H, hv), "mlp.gate_proj": (I, H), "mlp.up_proj": (I, H),
                         "mlp.down_proj": (H, I)}.items():
        put(f"model.layers.0.{name}", gptq(g, N, K))
    for name, (N, K) in {"self_attn.q_proj": (qd, H), "self_attn.k_proj": (kd, H), "self_attn.v_proj": (kd, H),
                         "self_attn.o_proj": (H, qd), "mlp.gate_proj": (I, H), "mlp.up_proj": (I, H),
                         "mlp.down_proj": (H, I)}.items():
        put(f"model.layers.1.{name}", gptq(g, N, K))
    put("model.layers.5.mlp.gate_proj", gptq(g, 16, 256))         # a layer past the configured depth
    put("extra.act_order", gptq(g, 16, 256, act_order=True))       # desc_act: permuted groups
    put("extra.asym", gptq(g, 16, 256, zero=7))                    # asymmetric zeros
    put("w4a8.a", w4a8(g, 32, 256))
    put("w4a8.b", w4a8(g, 16, 512))
    put("w4a8.bias", dict(w4a8(g, 16, 256), bias=torch.zeros(16)))  # a bias
    put("w4a8.bad_scale", w4a8(g, 16, 256, bad_scale=True))        # a negative fp8 group scale
    t["lm_head.weight"] = (torch.randn(64, H, generator=g) * 0.02).bfloat16()  # dense
    save_file(t, OUT, metadata={"bits": "4", "group_size": "128", "sym": "true", "checkpoint_format": "gptq"})
    print(f"wrote {OUT}: {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
