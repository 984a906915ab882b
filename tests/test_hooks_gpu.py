"""The host hooks with libmdx on the GPU: the wrapped W4A8 linear against the oracle bit for bit; the
wrapped MLP block against a host forward written in float32 torch (dequantised ConvRot weights, the
activations rotated by H256, no quantisation) within the activation quantisation's error; the wrapped
attention block against the same libmdx operators called directly, bit for bit (KV rows and x)."""
import types

import numpy as np
import pytest
import torch

from conftest import assert_bits_equal, bits
from oracle import ref

pytestmark = pytest.mark.gpu


def _kitchen(g, N, K, dev):
    q = torch.randint(-128, 128, (N, K // 2), generator=g, dtype=torch.int8)
    s = (torch.rand(N, K // 16, generator=g) * 2 + 0.5).to(torch.float8_e4m3fn)
    sc = torch.rand(N, generator=g) * 2e-3 + 1e-3
    cb = torch.arange(-8, 8, dtype=torch.float32)
    p = types.SimpleNamespace(scale=s.to(dev), s_channel=sc.to(dev), codebook=cb.to(dev), group_size=16,
                              convrot_groupsize=256, mma_packed=False, transposed=False, correction=None)
    return types.SimpleNamespace(weight=types.SimpleNamespace(_qdata=q.to(dev), _params=p), bias=None)


def _dense(lin):
    """float32 [N, K] weights of a packed linear: rint(cb[code] * s_rel) * s_channel (the contract)."""
    w = lin.weight
    s = ref.fp8e4m3_to_f32(w._params.scale.view(torch.uint8).cpu().numpy())
    w8 = ref.decode_w8(w._qdata.cpu().numpy(), s, w._params.codebook.cpu().numpy(), 16).astype(np.float32)
    return torch.from_numpy(w8 * w._params.s_channel.cpu().numpy()[:, None])


def test_w4_hook_matches_the_oracle(C, dev, monkeypatch):
    from mdx import guard, hooks
    guard.BOARD.clear()
    hooks.reset_stats()
    g = torch.Generator().manual_seed(2)
    lin = _kitchen(g, 1024, 4096, dev)
    p = lin.weight._params
    f = hooks.wrap_linear(lambda *a: pytest.fail("the host path must not run"))
    for rows in (1, 5, 16):
        print(f"case w4 hook rows={rows}", flush=True)
        x = torch.randint(-128, 128, (rows, 4096), generator=g, dtype=torch.int8)
        xs = torch.rand(rows, 1, generator=g) * 0.05
        out = f(x.to(dev), xs.to(dev), lin.weight._qdata, p.scale, p.s_channel, p.codebook, None, 16, torch.bfloat16)
        want = ref.w4a8_linear(x.numpy(), xs.numpy(), lin.weight._qdata.cpu().numpy(),
                               ref.fp8e4m3_to_f32(p.scale.view(torch.uint8).cpu().numpy()), p.s_channel.cpu().numpy(),
                               p.codebook.cpu().numpy(), 16)
        assert_bits_equal(bits(out), want, f"rows={rows}")


def test_mlp_hook_against_a_float32_host_forward(C, dev, monkeypatch):
    from mdx import guard, hooks, layout
    guard.BOARD.clear()
    hooks.reset_stats()
    g = torch.Generator().manual_seed(3)
    I = 2048
    mlp = types.SimpleNamespace(gate_proj=_kitchen(g, I, 4096, dev), up_proj=_kitchen(g, I, 4096, dev),
                                down_proj=_kitchen(g, 4096, I, dev))
    dense = [_dense(l).to(dev) for l in (mlp.gate_proj, mlp.up_proj, mlp.down_proj)]
    h = layout.regular_hadamard(dev, torch.float32)
    rot = lambda t: (t.reshape(t.shape[0], -1, 256) @ h).reshape(t.shape)
    nw = (1 + 0.05 * torch.randn(4096, generator=g)).bfloat16().to(dev)

    def norm(x):
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6) * nw.float()).bfloat16()

    def host(self, x, norm=None):
        xn = norm(x).reshape(-1, 4096).float()
        gg, uu = rot(xn) @ dense[0].T, rot(xn) @ dense[1].T
        return (rot(torch.nn.functional.silu(gg) * uu) @ dense[2].T).reshape(*x.shape[:-1], 4096)

    fwd = hooks.wrap_mlp(host)
    for rows in (1, 8):
        print(f"case mlp hook rows={rows}", flush=True)
        x = torch.randn(1, rows, 4096, generator=g).bfloat16().to(dev)
        got = fwd(mlp, x, norm).float()
        want = host(mlp, x, norm)
        rel = ((got - want).norm() / want.norm()).item()
        assert rel < 3e-2, rel  # int8 activations (2 quantisations) against float32
        assert hooks.stats()["mono"]["fallback"] == {}
    assert hooks.stats()["mono"]["fast"] >= 2 and guard.BOARD.allows("mono")


def test_attention_block_hook_equals_the_operators(C, dev, monkeypatch):
    from mdx import guard, hooks, layout
    guard.BOARD.clear()
    hooks.reset_stats()
    g = torch.Generator().manual_seed(4)
    S, H, Hk, D, cap, L = 4, 32, 8, 128, 256, 100
    mix = types.SimpleNamespace(q_proj=_kitchen(g, 2 * H * D, 4096, dev), k_proj=_kitchen(g, Hk * D, 4096, dev),
                                v_proj=_kitchen(g, Hk * D, 4096, dev), o_proj=_kitchen(g, 4096, H * D, dev),
                                q_norm=types.SimpleNamespace(weight=(1 + 0.1 * torch.randn(D, generator=g)).bfloat16().to(dev), eps=1e-6),
                                k_norm=types.SimpleNamespace(weight=(1 + 0.1 * torch.randn(D, generator=g)).bfloat16().to(dev), eps=1e-6),
                                num_heads=H, num_kv_heads=Hk, head_dim=D, rotary_dim=64)
    norm = lambda: types.SimpleNamespace(weight=(1 + 0.05 * torch.randn(4096, generator=g)).bfloat16().to(dev), eps=1e-6)

    class Block:
        layer_type = "full_attention"

        def forward(self, *a, **k):
            pytest.fail("the host path must not run")

    blk = Block()
    blk.self_attn = mix
    blk.mlp = types.SimpleNamespace(gate_proj=_kitchen(g, 4096, 4096, dev), up_proj=_kitchen(g, 4096, 4096, dev),
                                    down_proj=_kitchen(g, 4096, 4096, dev))
    blk.mlp.up_proj.weight._params.codebook = blk.mlp.gate_proj.weight._params.codebook
    blk.mlp.down_proj.weight._params.codebook = blk.mlp.gate_proj.weight._params.codebook
    blk.input_layernorm, blk.post_attention_layernorm = norm(), norm()
    freqs = torch.randn(S, 32, 2, 2, generator=g).to(dev)
    parents = [-1, 0, 1, 0]
    mask = torch.tensor(ref.tree_mask(parents), dtype=torch.int32, device=dev)

    def kv():
        gk = torch.Generator().manual_seed(9)
        return types.SimpleNamespace(key=torch.randn(1, Hk, cap, D, generator=gk).bfloat16().to(dev),
                                     value=torch.randn(1, Hk, cap, D, generator=gk).bfloat16().to(dev),
                                     position=torch.arange(L, L + S, device=dev),
                                     seqlen=torch.tensor([L], dtype=torch.int32, device=dev), mask=mask)

    x0 = torch.randn(1, S, 4096, generator=g).bfloat16().to(dev)
    # the hooked block
    x1, kv1 = x0.clone(), kv()
    out = hooks.wrap_block(Block.forward)(blk, x1, freqs_cis=freqs, past_key_value=kv1)
    assert out[0] is x1 and hooks.stats()["layer"]["fast"] == 1
    # the same operators called directly
    x2, kv2 = x0.clone(), kv()
    h, silu, sig = layout.regular_hadamard(dev), layout.silu_lut(dev), layout.sigmoid_lut(dev)
    w = lambda l: [l.weight._qdata, l.weight._params.scale, l.weight._params.s_channel, l.weight._params.codebook]
    xv = x2.view(S, 4096)
    outs = C.layer_pre(xv, blk.input_layernorm.weight, 1e-6, h, w(mix.q_proj) + w(mix.k_proj) + w(mix.v_proj), 0, False)
    rawq = outs[1].view(1, S, H, 2 * D)[..., :D]
    vv = outs[3].view(1, S, Hk, D)
    qo, ko = C.qk_norm_rope_kv(rawq, outs[2].view(1, S, Hk, D), vv, mix.q_norm.weight, mix.k_norm.weight, freqs,
                               kv2.key, kv2.value, kv2.position, 1e-6, 1e-6, 64)
    y = C.attn_dpas(qo, kv2.key, kv2.value, kv2.seqlen, ko, vv.transpose(1, 2), mask, 0).view(S, H * D)
    gate = outs[1].view(S, H, 2, D)[:, :, 1].reshape(S, H * D).contiguous()
    C.layer_post(xv, y.contiguous(), gate, sig, *w(mix.o_proj), blk.post_attention_layernorm.weight, 1e-6, h, silu,
                 *w(blk.mlp.gate_proj), *w(blk.mlp.up_proj), *w(blk.mlp.down_proj), 0, 6, False)
    assert_bits_equal(bits(x1), bits(x2), "x")
    assert_bits_equal(bits(kv1.key), bits(kv2.key), "KV rows")
    assert_bits_equal(bits(kv1.value), bits(kv2.value), "V rows")
