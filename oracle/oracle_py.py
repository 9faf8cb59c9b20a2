"""ctypes binding of liboracle.so (the CPU restatement) and of _ref/libref_q8.so
(the reference's own phonon_q8.c, compiled from its sources).

TEST INFRASTRUCTURE ONLY: imported by tests/ and __graft_entry__.smoke(), which
check the GPU results against it, and by the cpu_baseline leg of bench.py, which
times it. The product never imports it.
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


HEAD_BLOCKS = 6


class OracleFlowHead(ctypes.Structure):
    """OracleFlowHead (oracle.h): fp32 weights of the flow head."""
    _fields_ = ([("input_weight", _f32p), ("input_bias", _f32p), ("cond_weight", _f32p),
                 ("cond_bias", _f32p), ("time_weight", (_f32p * 2) * 2),
                 ("time_bias", (_f32p * 2) * 2), ("time_freqs", _f32p * 2),
                 ("time_alpha", _f32p * 2), ("block_ada_weight", _f32p * HEAD_BLOCKS),
                 ("block_ada_bias", _f32p * HEAD_BLOCKS),
                 ("block_norm_weight", _f32p * HEAD_BLOCKS),
                 ("block_norm_bias", _f32p * HEAD_BLOCKS),
                 ("block_mlp_weight", (_f32p * 2) * HEAD_BLOCKS),
                 ("block_mlp_bias", (_f32p * 2) * HEAD_BLOCKS),
                 ("final_ada_weight", _f32p), ("final_ada_bias", _f32p),
                 ("final_weight", _f32p), ("final_bias", _f32p)])


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
            "oracle_flow_layer_norm": [_f32p, _f32p, _f32p, _f32p],
            "oracle_silu": [_f32p, _sz],
            "oracle_time_embedding": [ctypes.POINTER(OracleFlowHead), _sz, ctypes.c_float, _f32p],
            "oracle_flow_head_forward": [ctypes.POINTER(OracleFlowHead), _f32p, _f32p,
                                         ctypes.c_float, ctypes.c_float, _f32p],
            "oracle_lsd_one_step": [ctypes.POINTER(OracleFlowHead), _f32p, _f32p,
                                    ctypes.c_float, _f32p],
            "oracle_eos_logit": [_f32p, _f32p, _f32p, _f32p],
        }
        lib.oracle_mean_512.restype = ctypes.c_float
        lib.oracle_mean_512.argtypes = [_f32p]
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


    # -- flow head --------------------------------------------------------------------
    def mean_512(self, x) -> float:
        return self.lib.oracle_mean_512(_ptr(np.ascontiguousarray(x, np.float32)))

    def flow_layer_norm(self, x, w=None, b=None):
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros(512, np.float32)
        wp = None if w is None else _ptr(np.ascontiguousarray(w, np.float32))
        bp = None if b is None else _ptr(np.ascontiguousarray(b, np.float32))
        ok = self.lib.oracle_flow_layer_norm(_ptr(x), wp, bp, _ptr(out))
        return bool(ok), out

    def silu(self, x):
        v = np.array(x, np.float32, copy=True)
        ok = self.lib.oracle_silu(_ptr(v), v.size)
        return bool(ok), v


class OracleHead:
    """fp32 weights of one flow head, kept alive for the OracleFlowHead pointers.
    `head` maps the reference's tensor roles to arrays (see flow_head_arrays)."""

    def __init__(self, oracle: Oracle, head: dict):
        self.oracle = oracle
        keep = {k: np.ascontiguousarray(v, np.float32) for k, v in head.items()}
        self.keep = keep
        h = OracleFlowHead()
        for name in ("input_weight", "input_bias", "cond_weight", "cond_bias", "final_ada_weight",
                     "final_ada_bias", "final_weight", "final_bias"):
            setattr(h, name, _ptr(keep[name]))
        for i in range(2):
            for j in range(2):
                h.time_weight[i][j] = _ptr(keep[f"time_weight_{i}_{j}"])
                h.time_bias[i][j] = _ptr(keep[f"time_bias_{i}_{j}"])
            h.time_freqs[i] = _ptr(keep[f"time_freqs_{i}"])
            h.time_alpha[i] = _ptr(keep[f"time_alpha_{i}"])
        for b in range(HEAD_BLOCKS):
            h.block_ada_weight[b] = _ptr(keep[f"block_ada_weight_{b}"])
            h.block_ada_bias[b] = _ptr(keep[f"block_ada_bias_{b}"])
            h.block_norm_weight[b] = _ptr(keep[f"block_norm_weight_{b}"])
            h.block_norm_bias[b] = _ptr(keep[f"block_norm_bias_{b}"])
            for j in range(2):
                h.block_mlp_weight[b][j] = _ptr(keep[f"block_mlp_weight_{b}_{j}"])
                h.block_mlp_bias[b][j] = _ptr(keep[f"block_mlp_bias_{b}_{j}"])
        self.h = h

    def time_embedding(self, which: int, value: float):
        out = np.zeros(512, np.float32)
        ok = self.oracle.lib.oracle_time_embedding(ctypes.byref(self.h), which, value, _ptr(out))
        return bool(ok), out

    def forward(self, condition, state, s: float, t: float):
        c = np.ascontiguousarray(condition, np.float32)
        x = np.ascontiguousarray(state, np.float32)
        out = np.zeros(32, np.float32)
        ok = self.oracle.lib.oracle_flow_head_forward(ctypes.byref(self.h), _ptr(c), _ptr(x), s,
                                                      t, _ptr(out))
        return bool(ok), out

    def lsd_one_step(self, condition, raw_noise, temperature: float):
        c = np.ascontiguousarray(condition, np.float32)
        n = np.ascontiguousarray(raw_noise, np.float32)
        out = np.zeros(32, np.float32)
        ok = self.oracle.lib.oracle_lsd_one_step(ctypes.byref(self.h), _ptr(c), _ptr(n),
                                                 temperature, _ptr(out))
        return bool(ok), out

    def eos_logit(self, weight, bias, state):
        w = np.ascontiguousarray(weight, np.float32)
        b = np.ascontiguousarray(bias, np.float32)
        x = np.ascontiguousarray(state, np.float32)
        out = np.zeros(1, np.float32)
        ok = self.oracle.lib.oracle_eos_logit(_ptr(w), _ptr(b), _ptr(x), _ptr(out))
        return bool(ok), float(out[0])


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


# ------------------------------------------------------------ audio decoder
class OracleMimi(ctypes.Structure):
    """OracleMimi (oracle.h): fp32 weights of the Mimi latent transformer."""
    _fields_ = [("projection", _f32p), ("upsample", _f32p), ("qkv", _f32p * 2),
                ("out", _f32p * 2), ("mlp_in", _f32p * 2), ("mlp_out", _f32p * 2),
                ("norm1_weight", _f32p * 2), ("norm1_bias", _f32p * 2),
                ("norm2_weight", _f32p * 2), ("norm2_bias", _f32p * 2),
                ("scale1", _f32p * 2), ("scale2", _f32p * 2), ("rope_theta", ctypes.c_float)]


def _audio_lib(oracle: Oracle):
    lib = oracle.lib
    if getattr(lib, "_audio_ready", False):
        return lib
    sigs = {
        "oracle_mimi_upsample_frame": (ctypes.c_int, [_f32p, _f32p, _f32p, _sz, _sz, _f32p]),
        "oracle_mimi_create": (_vp, [ctypes.POINTER(OracleMimi)]),
        "oracle_mimi_destroy": (None, [_vp]),
        "oracle_mimi_positions": (_sz, [_vp]),
        "oracle_mimi_process": (ctypes.c_int, [_vp, _f32p, _sz, _f32p]),
        "oracle_conv_create": (_vp, [_f32p, _f32p, _sz, _sz, _sz, _sz, ctypes.c_int]),
        "oracle_conv_destroy": (None, [_vp]),
        "oracle_conv_process": (ctypes.c_int, [_vp, _f32p, _sz, _f32p]),
        "oracle_conv_elu": (None, [_f32p, _sz]),
        "oracle_residual_process": (ctypes.c_int, [_vp, _vp, _f32p, _sz, _f32p]),
        "oracle_pcm_process": (ctypes.c_int, [_vp, _vp * 11, _f32p, _sz, _f32p]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    lib._audio_ready = True
    return lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


class MimiOracle:
    """A Mimi request state over fp32 weights: `weights` holds projection
    [512,32], upsample [512,32] and per layer l the keys qkv, out, mlp_in,
    mlp_out, norm1_w, norm1_b, norm2_w, norm2_b, scale1, scale2 as
    weights[l][key]."""

    KEYS = ("qkv", "out", "mlp_in", "mlp_out", "norm1_w", "norm1_b", "norm2_w", "norm2_b",
            "scale1", "scale2")

    def __init__(self, oracle: Oracle, weights: dict, theta: float = 10000.0):
        self.lib = _audio_lib(oracle)
        self._keep = {k: _f32(weights[k]) for k in ("projection", "upsample")}
        m = OracleMimi()
        m.projection = _ptr(self._keep["projection"])
        m.upsample = _ptr(self._keep["upsample"])
        names = {"qkv": "qkv", "out": "out", "mlp_in": "mlp_in", "mlp_out": "mlp_out",
                 "norm1_w": "norm1_weight", "norm1_b": "norm1_bias",
                 "norm2_w": "norm2_weight", "norm2_b": "norm2_bias",
                 "scale1": "scale1", "scale2": "scale2"}
        for l in range(2):
            for key, field in names.items():
                arr = _f32(weights[l][key])
                self._keep[(l, key)] = arr
                getattr(m, field)[l] = _ptr(arr)
        m.rope_theta = theta
        self.model = m
        self.state = self.lib.oracle_mimi_create(ctypes.byref(m))
        assert self.state

    def positions(self) -> int:
        return self.lib.oracle_mimi_positions(self.state)

    def process(self, latents):
        x = _f32(latents).reshape(-1, 32)
        out = np.zeros((x.shape[0] * 16, 512), np.float32)
        ok = self.lib.oracle_mimi_process(self.state, _ptr(x), x.shape[0], _ptr(out))
        return bool(ok), out

    def close(self):
        if self.state:
            self.lib.oracle_mimi_destroy(self.state)
            self.state = None


class ConvOracle:
    """A causal Conv1d (weight [out,in,kernel]) or transposed conv (weight
    [in,out,kernel], stride s, kernel 2s) with its history."""

    def __init__(self, oracle: Oracle, weight, bias, stride: int, transpose: bool):
        self.lib = _audio_lib(oracle)
        w = _f32(weight)
        self.w, self.b = w, _f32(bias)
        if transpose:
            self.cin, self.cout, self.kernel = w.shape
        else:
            self.cout, self.cin, self.kernel = w.shape
        self.stride = stride
        self.conv = self.lib.oracle_conv_create(_ptr(self.w), _ptr(self.b), self.cin, self.cout,
                                                self.kernel, stride, int(transpose))
        assert self.conv

    def process(self, x):
        x = _f32(x).reshape(-1, self.cin)
        y = np.zeros((x.shape[0] * self.stride, self.cout), np.float32)
        ok = self.lib.oracle_conv_process(self.conv, _ptr(x), x.shape[0], _ptr(y))
        return bool(ok), y

    def close(self):
        if self.conv:
            self.lib.oracle_conv_destroy(self.conv)
            self.conv = None


def conv_elu(oracle: Oracle, x):
    lib = _audio_lib(oracle)
    y = _f32(x).copy()
    lib.oracle_conv_elu(_ptr(y), y.size)
    return y


def residual_process(oracle: Oracle, conv3: ConvOracle, conv1: ConvOracle, x):
    lib = _audio_lib(oracle)
    x = _f32(x).reshape(-1, conv3.cin)
    y = np.zeros_like(x)
    ok = lib.oracle_residual_process(conv3.conv, conv1.conv, _ptr(x), x.shape[0], _ptr(y))
    return bool(ok), y


def mimi_upsample_frame(oracle: Oracle, kernel, x, previous, channels: int, stride: int):
    lib = _audio_lib(oracle)
    k, x, p = _f32(kernel), _f32(x), _f32(previous)
    out = np.zeros(stride * channels, np.float32)
    ok = lib.oracle_mimi_upsample_frame(_ptr(k), _ptr(x), _ptr(p), channels, stride, _ptr(out))
    return bool(ok), out


def pcm_process(oracle: Oracle, mimi: MimiOracle, convs, latents):
    """convs: the eleven ConvOracle of the reference's model.conv[] order."""
    lib = _audio_lib(oracle)
    x = _f32(latents).reshape(-1, 32)
    out = np.zeros(x.shape[0] * 1920, np.float32)
    arr = (_vp * 11)(*[c.conv for c in convs])
    ok = lib.oracle_pcm_process(mimi.state, arr, _ptr(x), x.shape[0], _ptr(out))
    return bool(ok), out
