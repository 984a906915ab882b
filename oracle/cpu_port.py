"""Loader of the oracle's C restatement of the MLP chain (cpu_mlp.c, built by oracle/Makefile into
oracle/_build/libmdx_cpu.so): the CPU baseline of the MLP bench line, checked bit for bit against
ref.rmsnorm + ref.mono_mlp (tests/test_oracle_cpu_port.py). Test infrastructure, not the library."""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "_build", "libmdx_cpu.so")
_lib = None


def load(build=True):
    """The ctypes library; built with make when missing (and `build`)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB) and build:
            subprocess.run(["make", "-s", "-C", HERE], check=True)
        lib = ctypes.CDLL(LIB)
        p = ctypes.c_void_p
        lib.cpu_mlp.argtypes = [p, p, ctypes.c_float, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                p, p, p, p, p, p, p, p, p, p, p, ctypes.c_int]
        lib.cpu_mlp.restype = ctypes.c_int
        _lib = lib
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def mlp(x_bits, nw_bits, eps, lut_bits, gate, up, down, threads=1):
    """bf16 bits [rows, H] of mono_mlp(rmsnorm(x, nw, eps)) (rotation none); gate/up/down: dicts with
    packed (uint8 [N, K / 2], row-major codes), s (float32 [N, K / G]), sch (float32 [N]), G."""
    lib = load()
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    rows, H = x.shape
    I = gate["packed"].shape[0]
    G = int(gate["G"])
    arrs = []
    for d in (gate, up, down):
        # (the codes are reinterpreted as bytes, not converted: no copy of the weights per call)
        arrs += [np.ascontiguousarray(d["packed"]).view(np.uint8), np.ascontiguousarray(d["s"], dtype=np.float32),
                 np.ascontiguousarray(d["sch"], dtype=np.float32)]
    nw = np.ascontiguousarray(nw_bits, dtype=np.uint16)
    lut = np.ascontiguousarray(lut_bits, dtype=np.uint16)
    out = np.empty((rows, H), dtype=np.uint16)
    rc = lib.cpu_mlp(_ptr(x), _ptr(nw), float(eps), rows, H, I, G, *[_ptr(a) for a in arrs], _ptr(lut), _ptr(out),
                     int(threads))
    if rc != 0:
        raise ValueError("cpu_mlp: shapes (H, I multiples of 256 and of G)")
    return out
