"""Pins the CPU oracle (oracle/oracle.c) before GPU results are checked against it:
against the reference's own golden vectors and known answers, against the
reference's phonon_q8.c compiled from its source (oracle/_ref), and against
closed forms, exact special cases and float64 brute force."""
import json
import os

import numpy as np
import pytest
from scipy.special import erf

import helpers
from helpers import f64_layer, rope_phases, softmax_attention_f64

GOLDEN = json.load(open(os.path.join(helpers.GOLDEN_DIR, "reference_vectors.json")))
Q8GOLD = np.load(os.path.join(helpers.GOLDEN_DIR, "q8_reference_vectors.npz"))


def bits(x):
    return np.asarray(x, np.float32).view(np.uint32)


# ------------------------------------------------------------------ fp16 / Q8
def test_half_to_float_all_patterns(oracle):
    """Brute force: all 65,536 binary16 patterns vs numpy's IEEE conversion."""
    pats = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = pats.view(np.float16).astype(np.float32)
    got = np.array([oracle.half_to_float(int(p)) for p in pats], np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(bits(got)[finite], bits(want)[finite])
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(got[np.isinf(want)], want[np.isinf(want)])


def q8_blocks(pkg, scales, values):
    b = np.zeros(len(scales), pkg.Q8_BLOCK)
    b["scale_bits"] = scales
    b["values"] = values
    return b


def test_q8_known_answers(oracle, pkg):
    """tests/test_phonon_q8.c:9-56."""
    k = GOLDEN["q8_known"]
    blocks = q8_blocks(pkg, [0x3800, 0x4000], [np.arange(32) - 16, np.ones(32)])
    x = np.ones(64, np.float32)
    ok, v = oracle.q8_dot(blocks, x)
    assert ok and v == k["dot_two_blocks"]
    matrix = np.concatenate([blocks, blocks[::-1]])
    ok, y = oracle.q8_matvec(matrix, x, 2, 64)
    assert ok and list(y) == k["matvec_rows"]
    assert not oracle.q8_dot(blocks, x[:63])[0]
    rows = q8_blocks(pkg, [0x3800, 0x4000, 0x3800, 0x4000],
                     [np.ones(32), 2 * np.ones(32), -np.ones(32), 3 * np.ones(32)])
    asym = np.concatenate([np.ones(32), 2 * np.ones(32)]).astype(np.float32)
    ok, y = oracle.q8_matvec(rows, asym, 2, 64)
    assert ok and list(y) == k["asymmetric_rows"]
    inf_scale = q8_blocks(pkg, [0x7C00], [np.ones(32)])
    assert not oracle.q8_dot(inf_scale, np.ones(32, np.float32))[0]
    sub = q8_blocks(pkg, [0x0001], [np.ones(32)])
    ok, v = oracle.q8_dot(sub, np.ones(32, np.float32))
    assert ok and v == k["subnormal_scale_dot"]
    xi = np.ones(32, np.float32)
    xi[0] = np.inf
    assert not oracle.q8_dot(sub, xi)[0]


def test_q8_matches_reference_golden_full(oracle, syn):
    """2048x512 seeded matvec: bit-identical to the compiled reference source."""
    import hashlib
    rng = np.random.default_rng(int(Q8GOLD["full_seed"][0]))
    w = syn.q8_matrix(rng, 2048, 512)
    x = rng.standard_normal(512).astype(np.float32)
    assert hashlib.sha256(w.tobytes()).digest() == Q8GOLD["full_sha256_w"].tobytes()
    assert hashlib.sha256(x.tobytes()).digest() == Q8GOLD["full_sha256_x"].tobytes()
    ok, y = oracle.q8_matvec(w, x, 2048, 512)
    assert ok
    assert np.array_equal(bits(y), bits(Q8GOLD["full_y"]))


def test_q8_matches_reference_golden_small(oracle, pkg):
    w = Q8GOLD["small_blocks"].view(pkg.Q8_BLOCK)
    ok, y = oracle.q8_matvec(w, Q8GOLD["small_x"], 64, 512)
    assert ok
    assert np.array_equal(bits(y), bits(Q8GOLD["small_y"]))


def test_q8_matches_compiled_reference_live(oracle, oracle_mod, syn):
    if not oracle_mod.ReferenceQ8.available():
        pytest.skip("oracle/_ref/libref_q8.so not built (reference tree absent)")
    ref = oracle_mod.ReferenceQ8()
    for seed in (11, 12, 13):
        rng = np.random.default_rng(seed)
        rows = int(rng.integers(1, 40)) * 16
        cols = int(rng.integers(1, 40)) * 32
        w = syn.q8_matrix(rng, rows, cols)
        x = rng.standard_normal(cols).astype(np.float32)
        ok1, y1 = oracle.q8_matvec(w, x, rows, cols)
        ok2, y2 = ref.q8_matvec(w, x, rows, cols)
        assert ok1 and ok2 and np.array_equal(bits(y1), bits(y2))


def test_q8_exact_on_representable_inputs(oracle, pkg):
    """Integer inputs and power-of-two scales: every partial sum is an exact
    integer below 2^24, so the result equals the float64 value exactly."""
    rng = np.random.default_rng(3)
    rows, cols = 32, 256
    scales = rng.choice([0x3800, 0x3C00, 0x4000, 0x3400], size=rows * cols // 32)
    values = rng.integers(-127, 128, size=(rows * cols // 32, 32))
    w = q8_blocks(pkg, scales, values)
    x = rng.integers(-8, 9, size=cols).astype(np.float32)
    ok, y = oracle.q8_matvec(w, x, rows, cols)
    sc = scales.astype(np.uint16).view(np.float16).astype(np.float64)
    dense = (values.astype(np.float64) * sc[:, None]).reshape(rows, cols)
    assert ok and np.array_equal(y.astype(np.float64), dense @ x.astype(np.float64))


def test_q8_float64_bound(oracle, syn):
    rng = np.random.default_rng(5)
    w = syn.q8_matrix(rng, 256, 512)
    x = rng.standard_normal(512).astype(np.float32)
    ok, y = oracle.q8_matvec(w, x, 256, 512)
    sc = w["scale_bits"].view(np.float16).astype(np.float64)
    dense = (w["values"].astype(np.float64) * sc[:, None]).reshape(256, 512)
    exact = dense @ x.astype(np.float64)
    assert ok and helpers.normwise(y, exact) < 1e-6


# ------------------------------------------------------------------- linear
def test_linear_known_answers(oracle):
    g = GOLDEN["linear_bf16"]
    ok, w = oracle.bf16_to_float(np.array(g["weight_bits"], np.uint16))
    ok2, y = oracle.linear_batch(w.reshape(g["shape"]), np.array(g["input"], np.float32))
    assert ok and ok2 and list(y[0]) == g["expected"]
    assert not oracle.bf16_to_float(np.array([0x7F80], np.uint16))[0]


def test_linear_q8_scale_special_cases(oracle, pkg):
    g = GOLDEN["linear_q8_scales"]
    blocks = q8_blocks(pkg, g["scale_bits"], [np.ones(32), np.ones(32)])
    ok, w = oracle.q8_expand(blocks, 2, 32)
    ok2, y = oracle.linear_batch(w, np.ones(32, np.float32))
    assert ok and ok2 and list(y[0]) == g["expected"]
    for bad in g["rejected_scale_bits"]:
        blocks["scale_bits"][0] = bad
        assert not oracle.q8_expand(blocks, 2, 32)[0]


def test_linear_bias_is_added_after_the_dot(oracle):
    """Bias is the beta*C term of one SGEMM: y = dot + bias (so a bias that
    dwarfs the dot does not change the dot's own rounding)."""
    w = np.ones((1, 4), np.float32)
    x = np.array([1.0, 2.0 ** -24, 2.0 ** -24, 0.0], np.float32)
    ok, y = oracle.linear_batch(w, x, bias=np.array([1.0], np.float32))
    # dot = 1 + 2^-24 + 2^-24 -> 1 (serial fp32), then + 1 -> 2
    assert ok and y[0][0] == 2.0
    assert not oracle.linear_batch(w, x, bias=np.array([np.nan], np.float32))[0]


def test_linear_float64_bound_batch(oracle):
    rng = np.random.default_rng(9)
    w = rng.standard_normal((64, 96)).astype(np.float32)
    x = rng.standard_normal((5, 96)).astype(np.float32)
    b = rng.standard_normal(64).astype(np.float32)
    ok, y = oracle.linear_batch(w, x, bias=b)
    exact = x.astype(np.float64) @ w.astype(np.float64).T + b
    assert ok and helpers.normwise(y, exact) < 1e-6


# --------------------------------------------------------------------- norms
def test_layer_norm_bit_regression(oracle):
    g = GOLDEN["layer_norm_regression"]
    x = np.array(g["input_bits"], np.uint32).view(np.float32)
    ok, y = oracle.layer_norm(x, np.ones(512, np.float32), np.zeros(512, np.float32))
    assert ok and int(bits(y[:1])[0]) == g["expected_first_bits"]


def test_layer_norm_closed_form_and_float64(oracle):
    """tests/test_phonon_transformer.c:547-551, then width 512 vs float64."""
    x = np.array([1.0, -2.0, 3.0], np.float32)
    ok, y = oracle.layer_norm(x, np.array([1.0, 2.0, 0.5], np.float32),
                              np.array([0.0, 0.1, -0.1], np.float32))
    d = np.sqrt(38.0 / 9.0 + 1e-5)
    assert ok and np.allclose(y, [(1 / 3) / d, (-8 / 3) / d * 2 + 0.1, (7 / 3) / d * 0.5 - 0.1],
                              atol=1e-5)
    rng = np.random.default_rng(2)
    for scale in (1e-3, 1.0, 1e3):
        x = (rng.standard_normal(512) * scale + 0.3 * scale).astype(np.float32)
        w = rng.standard_normal(512).astype(np.float32)
        b = rng.standard_normal(512).astype(np.float32)
        ok, y = oracle.layer_norm(x, w, b)
        x64 = x.astype(np.float64)
        ref = (x64 - x64.mean()) / np.sqrt(x64.var() + 1e-5) * w + b
        assert ok and helpers.normwise(y, ref) < 1e-5


def test_rms_norm_closed_form(oracle):
    x = np.array([1.0, -2.0, 3.0], np.float32)
    ok, y = oracle.rms_norm(x, np.array([2.0, 0.5, -1.0], np.float32))
    inv = 1.0 / np.sqrt(14.0 / 3.0 + 1e-5)
    assert ok and np.allclose(y, [2 * inv, -inv, -3 * inv], atol=1e-6)


# ---------------------------------------------------------------------- GELU
def test_gelu_golden_bits(oracle):
    g = GOLDEN["gelu"]
    ok, y = oracle.erf_gelu(np.array(g["inputs"], np.float32))
    assert ok and list(bits(y)) == g["expected_bits"]
    cf = g["closed_form"]
    ok, y = oracle.erf_gelu(np.array(cf["inputs"], np.float32))
    assert ok and np.allclose(y, cf["expected"], atol=cf["tolerance"])


def test_gelu_float64_bound(oracle):
    x = np.linspace(-8, 8, 4096).astype(np.float32)
    ok, y = oracle.erf_gelu(x)
    ref = 0.5 * x.astype(np.float64) * (1 + erf(x.astype(np.float64) / np.sqrt(2)))
    # A&S 7.1.26 has absolute error <= 1.5e-7 in erf.
    assert ok and np.max(np.abs(y - ref) / np.maximum(np.abs(x), 1.0)) < 4e-7
    assert not oracle.erf_gelu(np.array([np.inf], np.float32))[0]


# ---------------------------------------------------------------------- RoPE
def test_rope_golden(oracle):
    g = GOLDEN["rope"]
    for pos, want in zip(g["positions"], g["expected"]):
        row = np.zeros(64, np.float32)
        row[2:4] = g["pair_in"]
        ok, r = oracle.rope(row, 1, pos, g["theta"])
        assert ok and np.all(np.abs(r[2:4] - want) < g["tolerance"])
    q = np.array([1, 0, 0, 1], np.float32)
    ok, r = oracle.rope(q, 1, 1)
    assert ok and np.allclose(r, [np.cos(1), np.sin(1), -np.sin(0.01), np.cos(0.01)], atol=1e-6)
    assert not oracle.rope(q, 3, 0)[0]


def test_rope_float64_rotation(oracle):
    rng = np.random.default_rng(4)
    v = rng.standard_normal(512).astype(np.float32)
    for pos in (0, 5, 777, 8191):
        ok, r = oracle.rope(v, 8, pos)
        phase = rope_phases(pos)
        c, s = np.cos(phase), np.sin(phase)
        h = v.astype(np.float64).reshape(8, 32, 2)
        ref = np.stack([h[..., 0] * c - h[..., 1] * s, h[..., 0] * s + h[..., 1] * c], -1)
        assert ok and np.max(np.abs(r - ref.reshape(-1))) < 1e-6


# ----------------------------------------------------------------- attention
def attention_case(count, middle, tail):
    q = np.zeros(64, np.float32)
    q[0] = 8
    k = np.zeros((count, 64), np.float32)
    v = np.zeros((count, 64), np.float32)
    k[0, 0] = 2
    k[count - 1, 0] = tail
    v[0, 0] = v[count - 1, 0] = 0.01
    if middle:
        k[512, 0] = middle
    return q, k, v


def test_attention_golden_bits(oracle):
    """Five exact-bit cases of tests/test_speech.c:120-168 (512-key block
    boundaries, K=1 tail blocks, max rescale)."""
    for c in GOLDEN["attention_cases"]["cases"]:
        q, k, v = attention_case(c["count"], c["middle"], c["tail"])
        ok, out = oracle.attention(q, k, v, c["count"], 64)
        assert ok and int(bits(out[:1])[0]) == c["expected_bits"]
        assert np.all(out[1:] == 0)


def test_attention_special_cases(oracle):
    rng = np.random.default_rng(6)
    q = rng.standard_normal(64).astype(np.float32)
    k = rng.standard_normal((1, 64)).astype(np.float32)
    v = rng.standard_normal((1, 64)).astype(np.float32)
    ok, out = oracle.attention(q, k, v, 1, 64)
    assert ok and np.array_equal(out, v[0])  # one key: softmax weight exactly 1
    kk = np.repeat(k, 700, axis=0)
    vv = rng.standard_normal((700, 64)).astype(np.float32)
    ok, out = oracle.attention(q, kk, vv, 700, 64)
    assert ok and np.allclose(out, vv.astype(np.float64).mean(0), atol=1e-5)


def test_attention_float64_bound_strided(oracle):
    rng = np.random.default_rng(8)
    for count in (2, 511, 512, 513, 1500, 2049):
        rows = rng.standard_normal((count, 512)).astype(np.float32)
        vals = rng.standard_normal((count, 512)).astype(np.float32)
        q = rng.standard_normal(64).astype(np.float32) * 3
        h = 3
        ok, out = oracle.attention(q, rows[:, h * 64:], vals[:, h * 64:], count, 512)
        ref = softmax_attention_f64(q, rows[:, h * 64:(h + 1) * 64], vals[:, h * 64:(h + 1) * 64])
        assert ok and helpers.normwise(out, ref) < 1e-5


# ------------------------------------------------------------ layer / stack
def test_stack_step_matches_float64(oracle, oracle_mod, syn):
    layers, steps = 2, 6
    model = syn.flow_model(21, layers)
    ol = helpers.oracle_layers(oracle, model)
    om = oracle_mod.OracleModel(oracle, ol)
    cap = steps
    keys = np.zeros((layers, cap, 512), np.float32)
    vals = np.zeros_like(keys)
    k64 = np.zeros((layers, cap, 512))
    v64 = np.zeros_like(k64)
    rng = np.random.default_rng(22)
    for pos in range(steps):
        x = rng.standard_normal(512).astype(np.float32)
        ok, y = om.stack_step(keys, vals, cap, pos, x)
        ref = x.astype(np.float64)
        for l in range(layers):
            ref = f64_layer(ol[l], ref, k64[l], v64[l], pos)
        assert ok
        assert helpers.normwise(y, ref) < 1e-4, (pos, helpers.normwise(y, ref))


def zero_layer(pkg):
    """All-zero BF16 matrices, unit LN weight, zero bias."""
    z = {name: np.zeros(r * c, np.uint16) for name, (r, c) in helpers.SHAPES.items()}
    z["norm1_weight"] = z["norm2_weight"] = np.full(512, 0x3F80, np.uint16)
    z["norm1_bias"] = z["norm2_bias"] = np.zeros(512, np.uint16)
    return z


def test_stack_step_invariants(oracle, oracle_mod, pkg):
    """tests/test_phonon_transformer.c:707-855: zero projections are the
    identity; a nonzero V/out path makes the output depend on the cache."""
    zl = zero_layer(pkg)
    ol = helpers.oracle_layers(oracle, [zl] * 3)
    om = oracle_mod.OracleModel(oracle, ol)
    keys = np.zeros((3, 2, 512), np.float32)
    vals = np.zeros_like(keys)
    x = (np.arange(512) / 512).astype(np.float32)
    ok, y = om.stack_step(keys, vals, 2, 0, x)
    assert ok and np.array_equal(y, x)
    zl2 = dict(zl)
    zl2["qkv"] = zl["qkv"].copy()
    zl2["qkv"][1024 * 512] = 0x3F80  # V[0] <- x[0]
    zl2["out"] = zl["out"].copy()
    zl2["out"][0] = 0x3F80  # out[0] <- attended[0]
    om2 = oracle_mod.OracleModel(oracle, helpers.oracle_layers(oracle, [zl2] * 3))
    keys[:] = 0
    vals[:] = 0
    first = np.zeros(512, np.float32)
    first[0] = 1
    second = np.zeros(512, np.float32)
    second[0] = 3
    ok0, out0 = om2.stack_step(keys, vals, 2, 0, first)
    ok1, out1 = om2.stack_step(keys, vals, 2, 1, second)
    assert ok0 and ok1 and out0[0] > 1 and out1[0] > 3


def test_kv_append_layout(oracle):
    g = GOLDEN["kv_layout"]
    layers, cap = 9, g["capacity"]
    keys = np.zeros((layers, cap, 512), np.float32)
    vals = np.zeros_like(keys)
    k = np.arange(512, dtype=np.float32)
    ok = oracle.lib.oracle_kv_append(
        keys.ctypes.data_as(oracle_ptr()), vals.ctypes.data_as(oracle_ptr()), layers, cap,
        g["layer"], g["position"], k.ctypes.data_as(oracle_ptr()),
        (-k).ctypes.data_as(oracle_ptr()))
    flat = keys.reshape(-1)
    assert ok and flat[(g["layer"] * cap + g["position"]) * 512 + g["probe_column"]] == 7.0
    assert not oracle.lib.oracle_kv_append(
        keys.ctypes.data_as(oracle_ptr()), vals.ctypes.data_as(oracle_ptr()), layers, cap, 9, 0,
        k.ctypes.data_as(oracle_ptr()), k.ctypes.data_as(oracle_ptr()))


def oracle_ptr():
    import ctypes
    return ctypes.POINTER(ctypes.c_float)


def test_stack_step_streams_equals_single_stream_steps(oracle, oracle_mod, syn):
    """oracle_stack_step_streams (the threaded CPU baseline) runs, per stream,
    exactly oracle_stack_step on that stream's own cache: outputs and appended
    K/V rows are bit-identical, for any thread count, over several steps."""
    layers, streams, cap, steps = 2, 5, 40, 3
    om = oracle_mod.OracleModel(oracle, helpers.oracle_layers(oracle, syn.flow_model(23, layers)))
    rng = np.random.default_rng(24)
    positions = np.array([0, 3, 17, 31, 36])
    keys = rng.standard_normal((streams, layers, cap, 512)).astype(np.float32)
    vals = rng.standard_normal((streams, layers, cap, 512)).astype(np.float32)
    xs = rng.standard_normal((steps, streams, 512)).astype(np.float32)
    single_k, single_v = keys.copy(), vals.copy()
    want = np.zeros((steps, streams, 512), np.float32)
    for t in range(steps):
        for s in range(streams):
            ok, want[t, s] = om.stack_step(single_k[s], single_v[s], cap, positions[s] + t,
                                           xs[t, s])
            assert ok
    for threads in (1, 2, 5, 8):
        k, v = keys.copy(), vals.copy()
        for t in range(steps):
            ok, got = om.stack_step_streams(k, v, cap, positions + t, xs[t], threads)
            assert ok
            assert np.array_equal(bits(got), bits(want[t])), (threads, t)
        assert np.array_equal(bits(k), bits(single_k)) and np.array_equal(bits(v), bits(single_v))
    # A failing stream (position past the capacity) fails the whole call.
    ok, _ = om.stack_step_streams(keys.copy(), vals.copy(), cap, np.array([0, 1, 2, 3, cap]),
                                  xs[0], 3)
    assert not ok
