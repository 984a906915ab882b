"""The host hook layer (mdx/hooks.py, mdx/guard.py) on the CPU against a fake backend: routing of the
W4A8 linear, the MLP block and the decoder block, the fallback reasons, stats, and the failure rules
of the reference (comfy_mono_decode_xpu/guard.py; tests/test_runtime.py:13-67): a failure before any
state write falls back to the host's forward and switches the piece off; a failure after a KV / x write
re-raises without replaying the block; a sub-path failure leaves the piece on; an interrupt passes through;
install switches, idempotence and isolation of a piece that fails to install."""
import logging
import types

import pytest
import torch


@pytest.fixture
def hk(monkeypatch):
    from mdx import guard, hooks
    monkeypatch.setattr(hooks, "DEVICE_TYPE", "cpu")
    guard.BOARD.clear()
    hooks.reset_stats()
    fake = types.SimpleNamespace(calls=[])
    monkeypatch.setattr(hooks, "_lib_C", lambda: fake)
    yield hooks, guard, fake
    guard.BOARD.clear()


def _linear_args(rows=2, N=32, K=256, G=16):
    g = torch.Generator().manual_seed(1)
    x = torch.randint(-128, 128, (rows, K), generator=g, dtype=torch.int8)
    xs = torch.rand(rows, 1)
    packed = torch.randint(-128, 128, (N, K // 2), generator=g, dtype=torch.int8)
    s_rel = torch.rand(N, K // G).to(torch.float8_e4m3fn)
    return [x, xs, packed, s_rel, torch.rand(N), torch.arange(-8, 8, dtype=torch.float32), None, G, torch.bfloat16]


def test_linear_routes_the_contract_and_counts_reasons(hk):
    hooks, guard, fake = hk
    host = []
    original = lambda *a: host.append(a) or "host"
    fake.w4a8_decode_linear = lambda x, xs, q, s, sc, cb, res, G, code: torch.full((x.shape[0], q.shape[0]), 7.0)
    f = hooks.wrap_linear(original)
    assert getattr(f, hooks.CLAIM) and f.__wrapped__ is original
    out = f(*_linear_args())
    assert out.shape == (2, 32) and (out == 7).all() and not host
    cases = {
        "bias": dict(i=6, v=torch.zeros(32)),
        "out_dtype": dict(i=8, v=torch.float16),
        "x": dict(i=0, v=torch.zeros(2, 256, dtype=torch.int16)),
        "rows": dict(i=0, v=torch.zeros(17, 256, dtype=torch.int8)),
        "shape": dict(i=7, v=24),
        "packed": dict(i=2, v=torch.zeros(40, 128, dtype=torch.int8)),
        "s_rel": dict(i=3, v=torch.rand(32, 8)),
        "s_channel": dict(i=4, v=torch.rand(31)),
        "codebook": dict(i=5, v=torch.arange(8, dtype=torch.float32)),
        "operands": dict(i=1, v=torch.rand(3)),
    }
    for why, c in cases.items():
        a = _linear_args()
        a[c["i"]] = c["v"]
        assert f(*a) == "host", why
    st = hooks.stats()["w4"]
    assert st["fast"] == 1 and st["fallback"] == {k: 1 for k in cases}
    assert guard.BOARD.allows("w4")


def test_linear_failure_falls_back_and_switches_off(hk, caplog):
    hooks, guard, fake = hk
    n = {"fast": 0}

    def broken(*a):
        n["fast"] += 1
        raise RuntimeError("launch failed")

    fake.w4a8_decode_linear = broken
    f = hooks.wrap_linear(lambda *a: "host")
    with caplog.at_level(logging.WARNING):
        assert f(*_linear_args()) == "host"
        assert f(*_linear_args()) == "host"
    assert not guard.BOARD.allows("w4") and n["fast"] == 1
    assert caplog.text.count("w4 path failed") == 1


def test_interrupt_passes_through_and_switches_nothing_off(hk):
    hooks, guard, fake = hk

    def interrupted(*a):
        raise KeyboardInterrupt()

    fake.w4a8_decode_linear = interrupted
    f = hooks.wrap_linear(lambda *a: "host")
    with pytest.raises(KeyboardInterrupt):
        f(*_linear_args())
    assert guard.BOARD.allows("w4")
    # an interrupt-type exception that reaches the board is re-raised unchanged
    with pytest.raises(KeyboardInterrupt):
        guard.BOARD.trip("w4", KeyboardInterrupt())
    assert guard.BOARD.allows("w4")


class _P:
    def __init__(self, N, K, cb=None, **kw):
        g = torch.Generator().manual_seed(N + K)
        self.scale = (torch.rand(N, K // 16, generator=g) + 0.5).to(torch.float8_e4m3fn)
        self.s_channel = torch.rand(N, generator=g)
        self.codebook = torch.arange(-8, 8, dtype=torch.float32) if cb is None else cb
        self.group_size, self.convrot_groupsize, self.mma_packed, self.transposed, self.correction = 16, 256, False, \
            False, None
        self.__dict__.update(kw)


class _QT:
    def __init__(self, N, K, **kw):
        self._qdata = torch.zeros(N, K // 2, dtype=torch.int8)
        self._params = _P(N, K, **kw)


def _lin(N, K, **kw):
    return types.SimpleNamespace(weight=_QT(N, K, **kw), bias=None)


class _MLP:
    def __init__(self, I=256, **kw):
        self.gate_proj, self.up_proj, self.down_proj = _lin(I, 4096, **kw), _lin(I, 4096), _lin(4096, I)

    def forward(self, x, norm=None):
        return "host"


def test_mlp_block_routes_and_falls_back(hk):
    hooks, guard, fake = hk
    fake.mono_mlp = lambda xn, h, lut, *a: (fake.calls.append(len(a)), torch.ones(xn.shape[0], 4096))[1]
    fwd = hooks.wrap_mlp(_MLP.forward)
    x = torch.zeros(1, 3, 4096, dtype=torch.bfloat16)
    norm = lambda t: t
    out = fwd(_MLP(), x, norm)
    assert out.shape == (1, 3, 4096) and fake.calls == [15]  # 12 weight tensors + nwg, stop, tiled
    assert fwd(_MLP(), x, None) == "host"                      # no norm: the host's MLP
    assert fwd(_MLP(), x[:, :, :2048].contiguous(), norm) == "host"
    assert fwd(_MLP(mma_packed=True), x, norm) == "host"
    assert fwd(_MLP(cb=torch.arange(16, dtype=torch.float32)), x, norm) == "host"
    st = hooks.stats()["mono"]
    assert st["fast"] == 1 and st["fallback"] == {"weights": 1, "codebook": 1}

    def broken(*a):
        raise RuntimeError("LDS overflow")

    fake.mono_mlp = broken
    assert fwd(_MLP(), x, norm) == "host" and not guard.BOARD.allows("mono")
    fake.mono_mlp = lambda *a: pytest.fail("a piece that is off must not be called")
    assert fwd(_MLP(), x, norm) == "host"


class _Norm:
    eps = 1e-6

    def __init__(self, n=4096):
        self.weight = torch.ones(n, dtype=torch.bfloat16)


def _attn_block():
    mix = types.SimpleNamespace(q_proj=_lin(8192, 4096), k_proj=_lin(1024, 4096), v_proj=_lin(1024, 4096),
                                o_proj=_lin(4096, 4096), q_norm=_Norm(128), k_norm=_Norm(128), num_heads=32,
                                num_kv_heads=8, head_dim=128, rotary_dim=64)
    return mix


class _Block:
    layer_type = "full_attention"

    def __init__(self, gdn=False):
        self.host_calls = 0
        self.mlp = _MLP(256)
        self.input_layernorm, self.post_attention_layernorm = _Norm(), _Norm()
        if gdn:
            self.layer_type = "linear_attention"
            self.linear_attn = types.SimpleNamespace(
                in_proj_qkv=_lin(8192, 4096), in_proj_z=_lin(4096, 4096), out_proj=_lin(4096, 4096),
                in_proj_a=types.SimpleNamespace(weight=torch.zeros(32, 4096)),
                in_proj_b=types.SimpleNamespace(weight=torch.zeros(32, 4096)),
                conv1d=types.SimpleNamespace(weight=torch.zeros(8192, 1, 4), bias=None), norm=_Norm(128),
                key_head_dim=128, num_key_heads=16)
        else:
            self.self_attn = _attn_block()

    def forward(self, x, attention_mask=None, freqs_cis=None, optimized_attention=None, past_key_value=None):
        self.host_calls += 1
        return "host"


def _kv(S=3):
    return types.SimpleNamespace(key=torch.zeros(1, 8, 64, 128, dtype=torch.bfloat16),
                                 value=torch.zeros(1, 8, 64, 128, dtype=torch.bfloat16),
                                 position=torch.arange(S), seqlen=torch.tensor([10], dtype=torch.int32),
                                 mask=torch.tensor([1, 3, 7][:S], dtype=torch.int32), writes=0)


def _fake_layer(fake, S, x, failure=None):
    fake.layer_pre = lambda x2, nw, eps, h, mats, nwg, tiled: (
        fake.calls.append(("pre", len(mats))),
        [x2, torch.zeros(S, 8192, dtype=torch.bfloat16), torch.zeros(S, 1024, dtype=torch.bfloat16),
         torch.zeros(S, 1024, dtype=torch.bfloat16)])[1]
    if failure == "pre":
        def pre(*a):
            raise RuntimeError("contract")
        fake.layer_pre = pre

    def rope(rawq, rawk, vv, wq, wk, freqs, key, value, pos, eq, ek, rd):
        key.add_(1)  # the KV write
        if failure == "kv":
            raise RuntimeError("after state write")
        return torch.zeros(1, 32, S, 128, dtype=torch.bfloat16), torch.zeros(1, 8, S, 128, dtype=torch.bfloat16)

    def attn(qo, key, value, seqlen, ko, xv, mask, hint):
        if failure == "subpath":
            raise __import__("mdx.hooks", fromlist=["_"]).SubpathError("after state write")
        return torch.zeros(1, S, 4096, dtype=torch.bfloat16)

    def post(x2, y, gate, sig, *a):
        fake.calls.append(("post", gate is not None, len(a)))
        x2.add_(1)  # x in place
        if failure == "x":
            raise RuntimeError("after state write")
        return x2

    fake.qk_norm_rope_kv, fake.attn_dpas, fake.layer_post = rope, attn, post


@pytest.mark.parametrize("failure", [None, "pre", "kv", "x", "subpath"])
def test_decoder_block_state_writes_are_not_replayed(hk, failure):
    hooks, guard, fake = hk
    S = 3
    x = torch.zeros(1, S, 4096, dtype=torch.bfloat16)
    kv = _kv(S)
    _fake_layer(fake, S, x, failure)
    blk = _Block()
    fwd = hooks.wrap_block(_Block.forward)
    if failure in (None, "pre"):
        out = fwd(blk, x, past_key_value=kv)
        if failure is None:
            assert out[0] is x and out[1] is kv and blk.host_calls == 0
            assert fake.calls == [("pre", 12), ("post", True, 4 + 2 + 2 + 12 + 3)]  # gated q: the gate goes in
            assert hooks.stats()["layer"]["fast"] == 1 and guard.BOARD.allows("layer")
            assert kv.key.max().item() == 1 and x.max().item() == 1
        else:
            assert out == "host" and blk.host_calls == 1 and not guard.BOARD.allows("layer")
            assert kv.key.max().item() == 0
        return
    with pytest.raises(RuntimeError, match="after state write"):
        fwd(blk, x, past_key_value=kv)
    assert blk.host_calls == 0 and kv.key.max().item() == 1  # written once, never replayed
    assert x.max().item() == int(failure == "x")
    assert (not guard.BOARD.allows("layer")) == (failure != "subpath")


def test_decoder_block_inputs_outside_the_contract_run_the_host(hk):
    hooks, guard, fake = hk
    fwd = hooks.wrap_block(_Block.forward)
    blk = _Block()
    kv = _kv()
    for x, kw in ((torch.zeros(2, 3, 4096, dtype=torch.bfloat16), {}),
                  (torch.zeros(1, 17, 4096, dtype=torch.bfloat16), {}),
                  (torch.zeros(1, 3, 4096), {}),
                  (torch.zeros(1, 3, 2048, dtype=torch.bfloat16), {}),
                  (torch.zeros(1, 3, 4096, dtype=torch.bfloat16), {"attention_mask": torch.zeros(3, 3)}),
                  (torch.zeros(1, 3, 4096, dtype=torch.bfloat16), {"past_key_value": None})):
        kw.setdefault("past_key_value", kv)
        assert fwd(blk, x, **kw) == "host"
    assert blk.host_calls == 6 and hooks.stats()["layer"] == {"fast": 0, "fallback": {}}
    bad = _Block()
    bad.self_attn.o_proj = _lin(4096, 4096, group_size=32)
    assert fwd(bad, torch.zeros(1, 3, 4096, dtype=torch.bfloat16), past_key_value=kv) == "host"
    assert hooks.stats()["layer"]["fallback"] == {"weights": 1}


def test_gdn_block_runs_layer_gdn(hk):
    hooks, guard, fake = hk
    seen = {}

    def layer_gdn(*a):
        seen["n"] = len(a)
        seen["w4"] = len(a[4])
        seen["conv_w"] = tuple(a[7].shape)
        a[0].add_(1)

    fake.layer_gdn = layer_gdn
    blk = _Block(gdn=True)
    kv = types.SimpleNamespace(decode_step=lambda S: S <= 8, conv_state=None, proj_buf=None, qkv_buf=None, ctl=None,
                               dt_bias=None, g_decay=None, recurrent_state=None, gates_buf=None, sumsq_buf=None,
                               norm_weight=None)
    fwd = hooks.wrap_block(_Block.forward)
    x = torch.zeros(1, 2, 4096, dtype=torch.bfloat16)
    out = fwd(blk, x, past_key_value=kv)
    assert out[0] is x and x.max().item() == 1 and seen == {"n": 27, "w4": 24, "conv_w": (8192, 4)}
    assert fwd(blk, torch.zeros(1, 9, 4096, dtype=torch.bfloat16), past_key_value=kv) == "host"  # not a decode step


def test_install_switches_idempotence_and_isolation(hk, monkeypatch, caplog):
    hooks, guard, fake = hk
    mod = types.SimpleNamespace(w4a8_linear_prequantized=lambda *a: "host")

    class MLP(_MLP):
        pass

    class Block(_Block):
        pass

    assert hooks.install(mod, MLP, Block, env={}) == {"W4": True, "MONO": True, "LAYER": True}
    assert getattr(mod.w4a8_linear_prequantized, hooks.CLAIM) and MLP.forward.__wrapped__ is _MLP.forward
    assert hooks.install(mod, MLP, Block, env={}) == {"W4": False, "MONO": False, "LAYER": False}

    class MLP2(_MLP):
        pass

    mod2 = types.SimpleNamespace(w4a8_linear_prequantized=lambda *a: "host")
    assert hooks.install(mod2, MLP2, None, env={"MDX_DECODE": "0"}) == {}
    assert hooks.install(mod2, MLP2, None, env={"MDX_DECODE": "0", "MDX_DECODE_MONO": "1"}) == {"MONO": True}
    assert not getattr(mod2.w4a8_linear_prequantized, hooks.CLAIM, False)

    class NoForward:
        pass

    mod3 = types.SimpleNamespace(w4a8_linear_prequantized=lambda *a: "host")
    with caplog.at_level(logging.ERROR):
        res = hooks.install(mod3, NoForward, None, env={})
    assert res["W4"] is True and res["MONO"].startswith("AttributeError")
    # without the library nothing is installed
    monkeypatch.setattr(hooks, "_lib_C", lambda: (_ for _ in ()).throw(OSError("libmdx.so: not found")))
    mod4 = types.SimpleNamespace(w4a8_linear_prequantized=lambda *a: "host")
    assert hooks.install(mod4, None, None, env={}) == {}
    assert not getattr(mod4.w4a8_linear_prequantized, hooks.CLAIM, False)


def test_board_rule_directly(caplog):
    """The breaker rule on its own: a failure before a write answers from the host and trips the piece, one
    log line per piece however often it fails; after a write the error propagates (still tripping); a
    PassThrough error and an interrupt trip nothing; clear() switches a piece back on."""
    from mdx import guard
    board = guard.Board()
    calls = []

    def fails(wrote, exc=RuntimeError("boom")):
        def fast(progress):
            if wrote:
                progress.wrote()
            raise exc
        return fast

    host = lambda: calls.append("host") or "host"  # noqa: E731
    with caplog.at_level(logging.WARNING):
        assert guard.shielded("p", fails(False), host, board) == "host"
        assert guard.shielded("p", fails(False), host, board) == "host"
        with pytest.raises(RuntimeError, match="boom"):
            guard.shielded("q", fails(True), host, board)
    assert calls == ["host", "host"] and board.failures("p") == 2 and board.failures("q") == 1
    assert caplog.text.count("p path failed") == 1 and caplog.text.count("q path failed") == 1
    assert set(board.tripped()) == {"p", "q"} and not board.allows("p")
    for exc in (guard.PassThrough("sub-path already off"), KeyboardInterrupt()):
        with pytest.raises(type(exc)):
            guard.shielded("r", fails(True, exc), host, board)
    assert board.allows("r") and calls == ["host", "host"]
    board.clear("p")
    assert board.allows("p") and not board.allows("q")
    assert guard.shielded("p", lambda progress: "fast", host, board) == "fast"
