"""ctypes binding of liboracle.so (the CPU restatement) and of _ref/libref_q8.so
(the reference's own phonon_q8.c, compiled from its sources).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker. The product never imports it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libref_q8.so")

Q8_BLOCK = np.dtype([("scale_bits", "<u2"), ("values", "i1", (32,))], align=False)
assert Q8_BLOCK.itemsize == 34

_f32p = ctypes.POINTER(ctypes.c_float)
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t


class OracleLayer(ctypes.Structure):
    _fields_ = [(n, _f32p) for n in (
        "qkv", "out", "mlp_in", "mlp_out",
        "norm1_weight", "norm1_bias", "norm2_weight", "norm2_bias")]


def build() -> None:
    """Compile liboracle.so (and _ref/ when the reference tree is present)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def _ptr(a: np.ndarray, kind=_f32p):
    return a.ctypes.data_as(kind)


class Oracle:
    def __init__(self, path: str = LIB_PATH):
        if not os.path.exists(path):
            build()
        lib = ctypes.CDLL(path)
        self.lib = lib
        lib.oracle_half_to_float.restype = ctypes.c_float
        lib.oracle_half_to_float.argtypes = [ctypes.c_uint16]
        sigs = {
            "oracle_bf16_to_float": [_vp, _sz, _f32p],
            "oracle_q8_dot": [_vp, _f32p, _sz, _f32p],
            "oracle_q8_matvec": [_vp, _f32p, _sz, _sz, _f32p],
            "oracle_q8_expand": [_vp, _sz, _sz, _f32p],
            "oracle_linear_batch": [_f32p, _f32p, _sz, _sz, _f32p, _f32p, _sz],
            "oracle_rms_norm": [_f32p, _f32p, _sz, ctypes.c_float, _f32p],
            "oracle_layer_norm": [_f32p, _f32p, _f32p, _sz, ctypes.c_float, _f32p],
            "oracle_erf_gelu": [_f32p, _sz],
            "oracle_rope_interleaved": [_f32p, _sz, _sz, _sz, ctypes.c_float],
            "oracle_attention": [_f32p, _f32p, _f32p, _sz, _sz, _f32p],
            "oracle_kv_append": [_f32p, _f32p, _sz, _sz, _sz, _sz, _f32p, _f32p],
            "oracle_layer_step": [ctypes.POINTER(OracleLayer), _f32p, _f32p, _sz, _sz, _sz, _sz,
                                  _f32p, ctypes.c_float, _f32p],
            "oracle_stack_step": [ctypes.POINTER(OracleLayer), _sz, _f32p, _f32p, _sz, _sz,
                                  _f32p, ctypes.c_float, _f32p],
            "oracle_stack_step_streams": [ctypes.POINTER(OracleLayer), _sz, _f32p, _f32p, _sz,
                                          _sz, ctypes.POINTER(_sz), _f32p, ctypes.c_float,
                                          _f32p, _sz],
        }
        for name, args in sigs.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int

    # -- scalar / vector primitives -------------------------------------------------
    def half_to_float(self, bits: int) -> float:
        return self.lib.oracle_half_to_float(bits)

    def q8_dot(self, blocks: np.ndarray, x: np.ndarray):
        out = np.zeros(1, np.float32)
        ok = self.lib.oracle_q8_dot(blocks.ctypes.data, _ptr(x), x.size, _ptr(out))
        return bool(ok), out[0]

    def q8_matvec(self, blocks: np.ndarray, x: np.ndarray, rows: int, cols: int):
        y = np.zeros(rows, np.float32)
        ok = self.lib.oracle_q8_matvec(blocks.ctypes.data, _ptr(x), rows, cols, _ptr(y))
        return bool(ok), y

    def q8_expand(self, blocks: np.ndarray, rows: int, cols: int):
        w = np.zeros((rows, cols), np.float32)
        ok = self.lib.oracle_q8_expand(blocks.ctypes.data, rows, cols, _ptr(w))
        return bool(ok), w

    def bf16_to_float(self, bits: np.ndarray):
        bits = np.ascontiguousarray(bits, np.uint16)
        out = np.zeros(bits.size, np.float32)
        ok = self.lib.oracle_bf16_to_float(bits.ctypes.data, bits.size, _ptr(out))
        return bool(ok), out

    def linear_batch(self, w: np.ndarray, x: np.ndarray, bias=None):
        rows, cols = w.shape
        x = np.ascontiguousarray(x, np.float32).reshape(-1, cols)
        out = np.zeros((x.shape[0], rows), np.float32)
        b = None if bias is None else _ptr(np.ascontiguousarray(bias, np.float32))
        ok = self.lib.oracle_linear_batch(_ptr(np.ascontiguousarray(w, np.float32)), _ptr(x),
                                          rows, cols, b, _ptr(out), x.shape[0])
        return bool(ok), out

    def layer_norm(self, x, w, b, eps=1e-5):
        x, w, b = (np.ascontiguousarray(a, np.float32) for a in (x, w, b))
        out = np.zeros_like(x)
        ok = self.lib.oracle_layer_norm(_ptr(x), _ptr(w), _ptr(b), x.size, eps, _ptr(out))
        return bool(ok), out

    def rms_norm(self, x, w, eps=1e-5):
        x, w = (np.ascontiguousarray(a, np.float32) for a in (x, w))
        out = np.zeros_like(x)
        ok = self.lib.oracle_rms_norm(_ptr(x), _ptr(w), x.size, eps, _ptr(out))
        return bool(ok), out

    def erf_gelu(self, x):
        v = np.array(x, np.float32, copy=True)
        ok = self.lib.oracle_erf_gelu(_ptr(v), v.size)
        return bool(ok), v

    def rope(self, x, heads: int, position: int, theta: float = 10000.0):
        v = np.array(x, np.float32, copy=True)
        ok = self.lib.oracle_rope_interleaved(_ptr(v), v.size, heads, position, theta)
        return bool(ok), v

    def attention(self, q, keys, values, count: int, stride: int):
        q = np.ascontiguousarray(q, np.float32)
        out = np.zeros(64, np.float32)
        ok = self.lib.oracle_attention(_ptr(q), _ptr(keys), _ptr(values), count, stride, _ptr(out))
        return bool(ok), out


class OracleModel:
    """Expanded fp32 weights of L layers, kept alive for the OracleLayer pointers."""

    def __init__(self, oracle: Oracle, layers):
        """`layers`: list of dicts with fp32 arrays qkv, out, mlp_in, mlp_out and
        norm1_weight, norm1_bias, norm2_weight, norm2_bias."""
        self.oracle = oracle
        self.arrays = []
        self.structs = (OracleLayer * len(layers))()
        for i, layer in enumerate(layers):
            fields = {}
            for name, _ in OracleLayer._fields_:
                a = np.ascontiguousarray(layer[name], np.float32)
                self.arrays.append(a)
                fields[name] = _ptr(a)
            self.structs[i] = OracleLayer(**fields)
        self.layers = len(layers)

    def layer_step(self, keys, values, capacity, layer, position, x, theta=10000.0):
        out = np.zeros(512, np.float32)
        ok = self.oracle.lib.oracle_layer_step(
            ctypes.byref(self.structs[layer]), _ptr(keys), _ptr(values), self.layers, capacity,
            layer, position, _ptr(np.ascontiguousarray(x, np.float32)), theta, _ptr(out))
        return bool(ok), out

    def stack_step(self, keys, values, capacity, position, x, theta=10000.0):
        out = np.zeros(512, np.float32)
        ok = self.oracle.lib.oracle_stack_step(
            self.structs, self.layers, _ptr(keys), _ptr(values), capacity, position,
            _ptr(np.ascontiguousarray(x, np.float32)), theta, _ptr(out))
        return bool(ok), out

    def stack_step_streams(self, keys, values, capacity, positions, inputs, threads,
                           theta=10000.0):
        streams = len(positions)
        pos = (_sz * streams)(*[int(p) for p in positions])
        inputs = np.ascontiguousarray(inputs, np.float32)
        out = np.zeros((streams, 512), np.float32)
        ok = self.oracle.lib.oracle_stack_step_streams(
            self.structs, self.layers, _ptr(keys), _ptr(values), capacity, streams, pos,
            _ptr(inputs), theta, _ptr(out), threads)
        return bool(ok), out


class ReferenceQ8:
    """The reference's phonon_q8.c, compiled from its own source into _ref/."""

    def __init__(self, path: str = REF_PATH):
        lib = ctypes.CDLL(path)
        lib.phonon_q8_dot.argtypes = [_vp, _f32p, _sz, _f32p]
        lib.phonon_q8_dot.restype = ctypes.c_int
        lib.phonon_q8_matvec.argtypes = [_vp, _f32p, _sz, _sz, _f32p]
        lib.phonon_q8_matvec.restype = ctypes.c_int
        self.lib = lib

    @staticmethod
    def available() -> bool:
        return os.path.exists(REF_PATH)

    def q8_matvec(self, blocks: np.ndarray, x: np.ndarray, rows: int, cols: int):
        y = np.zeros(rows, np.float32)
        ok = self.lib.phonon_q8_matvec(blocks.ctypes.data, _ptr(x), rows, cols, _ptr(y))
        return bool(ok), y

    def q8_dot(self, blocks: np.ndarray, x: np.ndarray):
        out = np.zeros(1, np.float32)
        ok = self.lib.phonon_q8_dot(blocks.ctypes.data, _ptr(x), x.size, _ptr(out))
        return bool(ok), out[0]
