"""Shared test plumbing: imports of the product package (by path) and of the
CPU oracle, and conversions of synthetic weights for the oracle."""
from __future__ import annotations

import ctypes
import importlib.util
import os
import sys

import numpy as np
from scipy.special import erf

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "speech-mac_amd")
ORACLE_DIR = os.path.join(ROOT, "oracle")
GOLDEN_DIR = os.path.join(ROOT, "tests", "golden")


def package():
    if "speech_mac_amd" in sys.modules:
        return sys.modules["speech_mac_amd"]
    spec = importlib.util.spec_from_file_location(
        "speech_mac_amd", os.path.join(PKG_DIR, "__init__.py"),
        submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["speech_mac_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def synthetic():
    package()
    import speech_mac_amd.synthetic as syn  # noqa: E402
    return syn


def oracle_module():
    if ORACLE_DIR not in sys.path:
        sys.path.insert(0, ORACLE_DIR)
    import oracle_py  # noqa: E402
    return oracle_py


SHAPES = {"qkv": (1536, 512), "out": (512, 512), "mlp_in": (2048, 512), "mlp_out": (512, 2048)}


def oracle_layers(oracle, model):
    """Synthetic layer dicts -> fp32 expansions made by the oracle's own
    restatement of the reference expansion (src/phonon_pack.c:372-411)."""
    pkg = package()
    out = []
    for layer in model:
        d = {}
        for name, (r, c) in SHAPES.items():
            w = layer[name]
            if w.dtype == pkg.Q8_BLOCK:
                ok, e = oracle.q8_expand(w, r, c)
                assert ok
            else:
                ok, e = oracle.bf16_to_float(w.reshape(-1))
                assert ok
                e = e.reshape(r, c)
            d[name] = e
        for k in ("norm1_weight", "norm1_bias", "norm2_weight", "norm2_bias"):
            ok, d[k] = oracle.bf16_to_float(layer[k])
            assert ok
        out.append(d)
    return out


def scaled_model(syn, seed, layers, factor=0.1):
    """The synthetic benchmark model with every Q8 scale multiplied by
    `factor` (rounded to fp16 again): a well-conditioned stack for tight
    multi-layer, multi-step parity."""
    model = syn.flow_model(seed, layers)
    for layer in model:
        for name in SHAPES:
            sc = layer[name]["scale_bits"].view(np.float16).astype(np.float32) * factor
            layer[name]["scale_bits"] = sc.astype(np.float16).view(np.uint16)
    return model


def normwise(a, b) -> float:
    """max|a-b| / max|b| (the parity metric; 0 when both are zero)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    scale = np.max(np.abs(b))
    err = np.max(np.abs(a - b))
    return float(err / scale) if scale > 0 else float(err)


def elementwise_ok(a, b, atol=1e-5, rtol=1e-3) -> bool:
    """The reference's own gate |a-b| <= 1e-5 + 1e-3|b| (tests/test_phonon_pack.c:446)."""
    return bool(np.all(np.abs(np.asarray(a, np.float64) - b) <= atol + rtol * np.abs(b)))


# ------------------------------------------------------------------ flow head

HEAD_BLOCKS = 6


def bf16_bits(values) -> np.ndarray:
    """Upper 16 bits of the fp32 values (exact for values bf16 can hold)."""
    return (np.asarray(values, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def bf16_float(bits) -> np.ndarray:
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def reference_flow_head_bits() -> dict:
    """The synthetic BF16 flow head of tests/test_phonon_sampler.c:104-180 as
    arrays of bf16 bits: one shared matrix pattern ((5i mod 7) - 3) / 128 that
    every weight view starts inside at its own element offset, and bias /
    norm / frequency / alpha vectors of four patterns."""
    n = 1536 * 512 + 32
    i = np.arange(n, dtype=np.int64)
    matrix = bf16_bits((((i * 5) % 7) - 3).astype(np.float32) / 128.0)

    def mat(rows, cols, offset):
        return matrix[offset: offset + rows * cols].reshape(rows, cols)

    def vec(count, pattern, kind):
        k = np.arange(count, dtype=np.int64)
        if kind in (1, 2):
            v = 1.0 + ((((k * 3 + pattern * 5) % 7) - 3).astype(np.float32) / 128.0)
        elif kind == 3:
            v = ((k % 8) + 1).astype(np.float32) / 128.0
        else:
            v = (((k * 3 + pattern * 5) % 11) - 5).astype(np.float32) / 128.0
        return bf16_bits(v)

    h = {"input_weight": mat(512, 32, 1), "input_bias": vec(512, 1, 0),
         "cond_weight": mat(512, 512, 2), "cond_bias": vec(512, 2, 0)}
    for t in range(2):
        h[f"time_weight_{t}_0"] = mat(512, 256, t + 1)
        h[f"time_bias_{t}_0"] = vec(512, t + 3, 0)
        h[f"time_weight_{t}_1"] = mat(512, 512, t + 4)
        h[f"time_bias_{t}_1"] = vec(512, t + 5, 0)
        h[f"time_freqs_{t}"] = vec(128, 30 + t, 3)
        h[f"time_alpha_{t}"] = vec(512, 32 + t, 2)
    for b in range(HEAD_BLOCKS):
        h[f"block_ada_weight_{b}"] = mat(1536, 512, b + 3)
        h[f"block_ada_bias_{b}"] = vec(1536, b + 4, 0)
        h[f"block_norm_weight_{b}"] = vec(512, 10 + b, 1)
        h[f"block_norm_bias_{b}"] = vec(512, 16 + b, 0)
        h[f"block_mlp_weight_{b}_0"] = mat(512, 512, b + 9)
        h[f"block_mlp_bias_{b}_0"] = vec(512, b + 10, 0)
        h[f"block_mlp_weight_{b}_1"] = mat(512, 512, b + 11)
        h[f"block_mlp_bias_{b}_1"] = vec(512, b + 12, 0)
    h["final_ada_weight"] = mat(1024, 512, 22)
    h["final_ada_bias"] = vec(1024, 23, 0)
    h["final_weight"] = mat(32, 512, 24)
    h["final_bias"] = vec(32, 25, 0)
    return h


def flow_head_checkpoint_names() -> dict:
    """Checkpoint tensor name of each role of the head builders above (the
    names src/phonon_sampler.c:163-212 reads)."""
    net = "flow_lm.flow_net"
    names = {"input_weight": f"{net}.input_proj.weight", "input_bias": f"{net}.input_proj.bias",
             "cond_weight": f"{net}.cond_embed.weight", "cond_bias": f"{net}.cond_embed.bias",
             "final_ada_weight": f"{net}.final_layer.adaLN_modulation.1.weight",
             "final_ada_bias": f"{net}.final_layer.adaLN_modulation.1.bias",
             "final_weight": f"{net}.final_layer.linear.weight",
             "final_bias": f"{net}.final_layer.linear.bias"}
    for t in range(2):
        for j, layer in ((0, 0), (1, 2)):
            names[f"time_weight_{t}_{j}"] = f"{net}.time_embed.{t}.mlp.{layer}.weight"
            names[f"time_bias_{t}_{j}"] = f"{net}.time_embed.{t}.mlp.{layer}.bias"
        names[f"time_freqs_{t}"] = f"{net}.time_embed.{t}.freqs"
        names[f"time_alpha_{t}"] = f"{net}.time_embed.{t}.mlp.3.alpha"
    for b in range(HEAD_BLOCKS):
        blk = f"{net}.res_blocks.{b}"
        names[f"block_ada_weight_{b}"] = f"{blk}.adaLN_modulation.1.weight"
        names[f"block_ada_bias_{b}"] = f"{blk}.adaLN_modulation.1.bias"
        names[f"block_norm_weight_{b}"] = f"{blk}.in_ln.weight"
        names[f"block_norm_bias_{b}"] = f"{blk}.in_ln.bias"
        for j in range(2):
            names[f"block_mlp_weight_{b}_{j}"] = f"{blk}.mlp.{2 * j}.weight"
            names[f"block_mlp_bias_{b}_{j}"] = f"{blk}.mlp.{2 * j}.bias"
    return names


def reference_flow_head_inputs():
    """condition and state of tests/test_phonon_sampler.c:185-188."""
    i = np.arange(512)
    condition = (((i * 7) % 13) - 6).astype(np.float32) / 8.0
    j = np.arange(32)
    state = (((j * 11 + 3) % 17) - 8).astype(np.float32) / 16.0
    return condition, state


def random_flow_head_bits(seed: int, scale: float = 0.04) -> dict:
    """A random BF16 head of the same shapes (N(0, scale) weights, small
    biases, norm weights near 1, time frequencies in (0, 1])."""
    rng = np.random.default_rng(seed)
    ref = reference_flow_head_bits()
    out = {}
    for name, bits in ref.items():
        shape = bits.shape
        if "freqs" in name:
            v = rng.uniform(0.001, 1.0, shape)
        elif "alpha" in name or "norm_weight" in name:
            v = 1.0 + 0.1 * rng.standard_normal(shape)
        elif "bias" in name:
            v = 0.05 * rng.standard_normal(shape)
        else:
            v = scale * rng.standard_normal(shape)
        out[name] = bf16_bits(np.asarray(v, np.float32))
    return out


# ------------------------------------------------- float64 restatements
# Textbook float64 forms of the layer step, independent of the oracle's and
# the GPU's operation orders: both fp32 implementations are measured
# against them.

def rope_phases(pos, theta=10000.0):
    """fp32 phases pos*freq with freq = 1/powf(theta, 2i/64), powf taken as
    correctly rounded (float64 pow rounded once to fp32)."""
    expo = (np.arange(32, dtype=np.float32) * 2) / np.float32(64)
    powed = np.power(np.float64(np.float32(theta)), expo.astype(np.float64)).astype(np.float32)
    freq = np.float32(1.0) / powed
    return (np.float32(pos) * freq).astype(np.float64)


def softmax_attention_f64(q, k, v):
    s = (k.astype(np.float64) @ q.astype(np.float64)) * 0.125
    p = np.exp(s - s.max())
    return (p @ v.astype(np.float64)) / p.sum()


def f64_layer(w, x, keys, values, pos, theta=10000.0):
    """Float64 textbook layer step (pre-LN, interleaved RoPE, causal SDPA,
    erf-GELU MLP), independent of the oracle's operation order."""
    def ln(v, g, b):
        return (v - v.mean()) / np.sqrt(v.var() + 1e-5) * g + b

    def rope(v):
        ph = rope_phases(pos, theta)
        h = v.reshape(8, 32, 2)
        c, s = np.cos(ph), np.sin(ph)
        return np.stack([h[..., 0] * c - h[..., 1] * s, h[..., 0] * s + h[..., 1] * c],
                        -1).reshape(-1)

    f = {k: np.asarray(a, np.float64) for k, a in w.items()}
    qkv = f["qkv"] @ ln(x, f["norm1_weight"], f["norm1_bias"])
    q, k, v = rope(qkv[:512]), rope(qkv[512:1024]), qkv[1024:]
    keys[pos], values[pos] = k, v
    att = np.concatenate([softmax_attention_f64(q[h * 64:(h + 1) * 64],
                                                keys[:pos + 1, h * 64:(h + 1) * 64],
                                                values[:pos + 1, h * 64:(h + 1) * 64])
                          for h in range(8)])
    r = x + f["out"] @ att
    m = f["mlp_in"] @ ln(r, f["norm2_weight"], f["norm2_bias"])
    m = 0.5 * m * (1 + erf(m / np.sqrt(2)))
    return r + f["mlp_out"] @ m


# ------------------------------------------------------------ kpack v1 files
KPACK_SOURCE = "f6acc8f43cb296be31341b4428a6f01b6402659cd0039b624c4aea224936cf95"
KPACK_CONFIG = "3e89e90b9e7ae5a74c6b4e694960c37fd2ec85906d84adfcc1440c64307aa4f1"
KPACK_Q8, KPACK_BF16 = 1, 2


def kpack_bytes(tensors) -> bytes:
    """A kpack v1 file image (the layout src/phonon_pack.c:87-290 reads):
    `tensors` is a list of (name, dtype, shape, payload bytes). Payload
    ranges are 8-byte aligned; the metadata is padded with spaces so the
    payload starts 8-byte aligned; digests are SHA-256 (hashlib)."""
    import hashlib
    import struct
    index, payload = bytearray(), bytearray()
    for name, dtype, shape, data in tensors:
        payload += b"\0" * (-len(payload) % 8)
        nb = name.encode()
        index += struct.pack("<HBB", len(nb), dtype, len(shape))
        index += b"".join(struct.pack("<Q", d) for d in shape)
        index += struct.pack("<QQ", len(payload), len(data)) + nb
        payload += data
    meta = (f'{{"config_sha256":"{KPACK_CONFIG}","model":"gradium/phonon-40m-en",'
            f'"revision":"cc738b7e4d182c2ba1bafb8062aa4846af000637","source":"model.q8.gguf",'
            f'"source_sha256":"{KPACK_SOURCE}","tensors":209}}').encode()
    meta += b" " * (-(192 + 4 + len(meta) + len(index)) % 8)
    header = bytearray(192)
    header[0:8] = b"PHNQ8P1\0"
    header[8:32] = struct.pack("<IIQQ", 1, len(tensors), len(index), len(payload))
    header[32:64] = bytes.fromhex(KPACK_SOURCE)
    header[64:96] = bytes.fromhex(KPACK_CONFIG)
    header[96:128] = hashlib.sha256(bytes(index)).digest()
    header[128:160] = hashlib.sha256(bytes(payload)).digest()
    header[160:192] = hashlib.sha256(meta).digest()
    return bytes(header) + struct.pack("<I", len(meta)) + meta + bytes(index) + bytes(payload)


def kpack_synthetic():
    """The reference's synthetic pack (tests/test_phonon_pack.c:56-133): 36
    Q8_0 [1, 32] tensors of 32 ones at scale 1.0 (fp16 0x3c00), then 173 BF16
    [1] tensors holding 1.0."""
    q8 = b"\x00\x3c" + b"\x01" * 32
    return [(f"flow_lm.fixture_{i:03d}.weight", KPACK_Q8, (1, 32), q8) if i < 36 else
            (f"mimi.fixture_{i:03d}.weight", KPACK_BF16, (1,), b"\x80\x3f") for i in range(209)]


# ------------------------------------------------------ audio decoder models
def mimi_identity_model(route_only: bool = False) -> dict:
    """fp32 weights of the reference tests' synthetic Mimi models.

    route_only=False: tests/test_phonon_mimi.c:74-98 - projection routes
    channel i to latent i % 32, upsample taps 1 (current) and .5 (previous),
    per layer V = identity, Q = K = 0, out = identity, LayerNorm weights 1,
    layer_scale_1 = .5 / .25, MLP and layer_scale_2 zero.
    route_only=True: tests/test_phonon_pcm.c:65-77 - only channel 0 carries
    latent 0 through 16 current taps; every layer weight is zero."""
    proj = np.zeros((512, 32), np.float32)
    up = np.zeros((512, 32), np.float32)
    if route_only:
        proj[0, 0] = 1.0
        up[0, :16] = 1.0
    else:
        proj[np.arange(512), np.arange(512) % 32] = 1.0
        up[:, :16] = 1.0
        up[:, 16:] = 0.5
    model = {"projection": proj, "upsample": up}
    for l in range(2):
        layer = {"qkv": np.zeros((1536, 512), np.float32), "out": np.zeros((512, 512), np.float32),
                 "mlp_in": np.zeros((2048, 512), np.float32),
                 "mlp_out": np.zeros((512, 2048), np.float32)}
        for key in ("norm1_w", "norm1_b", "norm2_w", "norm2_b", "scale1", "scale2"):
            layer[key] = np.zeros(512, np.float32)
        if not route_only:
            layer["qkv"][1024 + np.arange(512), np.arange(512)] = 1.0
            layer["out"][np.arange(512), np.arange(512)] = 1.0
            layer["norm1_w"][:] = 1.0
            layer["norm2_w"][:] = 1.0
            layer["scale1"][:] = 0.25 if l else 0.5
        model[l] = layer
    return model


def pcm_scalar_convs():
    """The eleven convolutions of tests/test_phonon_pcm.c:31-49,78-86 as
    (weight, bias, stride, transposed), in the reference's model.conv[]
    order: conv0, then per stride 6, 5, 4 the transposed conv (channel-0
    route: taps 1 for the current position, .5 for the overlap) and a zero
    residual pair, then the final conv (taps 1 and .25)."""
    def conv(cin, cout, kernel, stride, route):
        trans = stride > 1
        w = np.zeros((cin, cout, kernel) if trans else (cout, cin, kernel), np.float32)
        flat = w.reshape(-1)
        if route:
            flat[0 if trans else kernel - 1] = 1.0
            if trans:
                flat[1:stride] = 1.0
                flat[stride:kernel] = 0.5
            elif cout == 1:
                flat[kernel - 2] = 0.25
        return w, np.zeros(cout, np.float32), stride, trans

    out = [conv(512, 512, 7, 1, True)]
    ch = 512
    for s in (6, 5, 4):
        out += [conv(ch, ch // 2, 2 * s, s, True), conv(ch // 2, ch // 4, 3, 1, False),
                conv(ch // 4, ch // 2, 1, 1, False)]
        ch //= 2
    out.append(conv(64, 1, 3, 1, True))
    return out


def pcm_scalar_expected(x: np.ndarray) -> np.ndarray:
    """tests/test_phonon_pcm.c:92-118: the sparse scalar graph's samples
    (float32 arithmetic, ELU through expf)."""
    f32 = np.float32
    elu = lambda v: v if v > 0 else f32(np.expm1(np.float64(v)))  # noqa: E731
    prev = [f32(0), f32(0), f32(0)]
    last = f32(0)
    out = []
    for t in range(x.shape[0] * 16):
        a = elu(f32(x[t // 16, 0]))
        for _ in range(6):
            b = elu(f32(a + prev[0]))
            for _ in range(5):
                d = elu(f32(b + prev[1]))
                for _ in range(4):
                    e = elu(f32(d + prev[2]))
                    out.append(f32(e + f32(0.25) * last))
                    last = e
                prev[2] = f32(0.5) * d
            prev[1] = f32(0.5) * b
        prev[0] = f32(0.5) * a
    return np.array(out, np.float32)


# ------------------------------------------------- audio decoder weights

MIMI_KEYS = ("qkv", "out", "mlp_in", "mlp_out", "norm1_w", "norm1_b", "norm2_w", "norm2_b",
             "scale1", "scale2")


def rounded(w):
    """fp32 weights -> the values bf16 holds (what both sides compute with)."""
    if isinstance(w, dict):
        return {k: rounded(v) for k, v in w.items()}
    return bf16_float(bf16_bits(w)).reshape(np.shape(w))


def random_mimi(seed):
    """Random Mimi weights of the real shapes (bf16-representable), scaled so
    that activations stay O(1) through both layers."""
    rng = np.random.default_rng(seed)
    n = lambda shape, s: (rng.standard_normal(shape) * s).astype(np.float32)  # noqa: E731
    w = {"projection": n((512, 32), 0.3), "upsample": n((512, 32), 0.3)}
    for l in range(2):
        w[l] = {"qkv": n((1536, 512), 512 ** -0.5), "out": n((512, 512), 512 ** -0.5),
                "mlp_in": n((2048, 512), 512 ** -0.5), "mlp_out": n((512, 2048), 2048 ** -0.5),
                "norm1_w": 1 + n(512, 0.1), "norm1_b": n(512, 0.1),
                "norm2_w": 1 + n(512, 0.1), "norm2_b": n(512, 0.1),
                "scale1": n(512, 0.3), "scale2": n(512, 0.3)}
    return rounded(w)


def mimi_model(lib, pkg, views, w):
    """fp32 Mimi weights (bf16-representable) -> PhononMimiModel of BF16 views
    kept alive by `views`."""
    m = pkg.PhononMimiModel()
    m.config = lib.phonon_mimi_config()
    m.stride = 16
    m.projection = views.bf16(bf16_bits(w["projection"]), (512, 32, 1))
    m.upsample = views.bf16(bf16_bits(w["upsample"]), (512, 1, 32))
    for l in range(2):
        for f, key in enumerate(MIMI_KEYS):
            arr = w[l][key]
            m.layers[l][f] = views.bf16(bf16_bits(arr), arr.shape)
    return m


def conv_model(lib, views, w, b, stride, trans):
    """A PhononConvModel handle from fp32 weight/bias (bf16-representable)."""
    wv = views.bf16(bf16_bits(w), w.shape)
    bv = views.bf16(bf16_bits(b), b.shape)
    h = ctypes.c_void_p()
    assert lib.phonon_conv_model_create(ctypes.byref(wv), ctypes.byref(bv), stride, int(trans),
                                        ctypes.byref(h)) == 1
    return h


def random_pcm_convs(seed):
    """Random weights for the eleven SEANet convolutions (the shapes and
    order of pcm_scalar_convs), scaled so that activations stay O(1)."""
    rng = np.random.default_rng(seed)
    out = []
    for (w, b, s, t) in pcm_scalar_convs():
        if t:
            cin, cout, k = w.shape
        else:
            cout, cin, k = w.shape
        gain = 0.5 if k > 1 and not t and cout != 1 and cin == cout else 1.0
        w = rounded((rng.standard_normal(w.shape) * gain * (cin * k / s) ** -0.5)
                    .astype(np.float32))
        b = rounded((rng.standard_normal(cout) * 0.05).astype(np.float32))
        out.append((w, b, s, t))
    return out


def pcm_model(lib, pkg, views, mimi_w, convs):
    """(PhononMimiModel, PhononPCMModel handle) from Mimi weights and the
    eleven (weight, bias, stride, transposed) convolutions."""
    mimi = mimi_model(lib, pkg, views, mimi_w)
    arr = (ctypes.c_void_p * 11)(*[conv_model(lib, views, w, b, s, t).value
                                   for (w, b, s, t) in convs])
    model = ctypes.c_void_p()
    assert lib.phonon_pcm_model_from_parts(ctypes.byref(mimi), arr, ctypes.byref(model)) == 1
    return mimi, model
