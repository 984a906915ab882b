"""The oracle's C restatement of the MLP chain (oracle/cpu_mlp.c, the bench's CPU baseline) against the
numpy oracle (ref.rmsnorm + ref.mono_mlp, rotation none), bit for bit, single- and multi-threaded, on
faithful fp16-ratio scales, integral scales, a zero row and rows that saturate the codes. CPU only."""
import numpy as np
import pytest
import torch

from oracle import cpu_port, ref


def _weights(N, K, gen, integral=False):
    from mdx import layout
    q = torch.randint(-8, 8, (N, K), generator=gen)
    sg = (torch.rand(N, K // 128, generator=gen) * 0.015 + 0.005).half()
    packed, s_rel, sch, _ = layout.gptq_pack(q, sg, 128, integral=integral)  # row-major codes [N, K / 2]
    return dict(packed=packed.numpy(), s=s_rel.float().numpy(), sch=sch.numpy(), cb=None, G=128)


@pytest.mark.parametrize("rows,H,I,integral,threads", [(1, 512, 1024, False, 1), (3, 512, 768, False, 4),
                                                       (8, 256, 512, True, 3), (2, 1024, 512, False, 8)])
def test_cpu_port_matches_oracle(rows, H, I, integral, threads):
    from mdx import layout
    gen = torch.Generator().manual_seed(rows * 7 + H)
    gate, up, down = _weights(I, H, gen, integral), _weights(I, H, gen, integral), _weights(H, I, gen, integral)
    x = (torch.randn(rows, H, generator=gen) * 2).bfloat16()
    if rows > 1:
        x[1] = 0  # a zero row: scale 1e-30, every code 0
    if rows > 2:
        x[2, :4] = 3e4  # saturating values
    xb = x.view(torch.int16).numpy().view(np.uint16)
    nwb = (1 + 0.05 * torch.randn(H, generator=gen)).bfloat16().view(torch.int16).numpy().view(np.uint16)
    lutb = layout.silu_lut(torch.device("cpu")).view(torch.int16).numpy().view(np.uint16)
    want = ref.mono_mlp(ref.rmsnorm(xb, nwb, 1e-6), "none", None, lutb, dict(gate), dict(up), dict(down))
    got = cpu_port.mlp(xb, nwb, 1e-6, lutb, gate, up, down, threads=threads)
    assert np.array_equal(got, want)
