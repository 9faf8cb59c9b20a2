"""GPU parity of the decode-step primitives, through the C-ABI, against the
CPU oracle (and the reference's golden vectors where they exist).

Tolerances: fp32 matvec / linear / attention / norms: normwise
max|gpu-oracle| <= 1e-4 * max|oracle| and the reference's elementwise gate
|d| <= 1e-5 + 1e-3|oracle| (tests/test_phonon_pack.c:446). Data movement
(KV append/gather, block indexing) and the RoPE rotation: bit-exact."""
import ctypes
import json
import os

import numpy as np
import pytest

import helpers

pytestmark = pytest.mark.gpu

GOLDEN = json.load(open(os.path.join(helpers.GOLDEN_DIR, "reference_vectors.json")))
Q8GOLD = np.load(os.path.join(helpers.GOLDEN_DIR, "q8_reference_vectors.npz"))
TOL = 1e-4


def bits(x):
    return np.asarray(x, np.float32).view(np.uint32)


def fp(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def test_device_is_gfx950(lib):
    buf = ctypes.create_string_buffer(256)
    assert lib.pgpu_device_name(buf, 256) == 1
    print("device:", buf.value.decode())
    assert b"gfx950" in buf.value


# ---------------------------------------------------------------- Q8 matvec
def gpu_q8_matvec(lib, blocks, x, rows, cols):
    y = np.full(rows, np.nan, np.float32)
    ok = lib.phonon_q8_matvec(blocks.ctypes.data, fp(x), rows, cols, fp(y))
    return bool(ok), y


def test_q8_matvec_config1_vs_reference_golden(lib, oracle, syn):
    """2048x512 seeded (the matvec benchmark input) vs the reference's own
    phonon_q8.c output committed as a golden vector, and vs the oracle: the
    drop-in runs the reference's arithmetic on the vector units, so every
    output has the reference's bits."""
    rng = np.random.default_rng(int(Q8GOLD["full_seed"][0]))
    w = syn.q8_matrix(rng, 2048, 512)
    x = rng.standard_normal(512).astype(np.float32)
    ok, y = gpu_q8_matvec(lib, w, x, 2048, 512)
    assert ok
    ref = Q8GOLD["full_y"]
    print("normwise vs reference:", helpers.normwise(y, ref))
    assert np.array_equal(bits(y), bits(ref))
    ok, yo = oracle.q8_matvec(w, x, 2048, 512)
    assert ok and np.array_equal(bits(y), bits(yo))


def test_q8_matvec_wide_dynamic_range(lib, pkg):
    w = Q8GOLD["small_blocks"].view(pkg.Q8_BLOCK)
    ok, y = gpu_q8_matvec(lib, w, Q8GOLD["small_x"], 64, 512)
    assert ok and np.array_equal(bits(y), bits(Q8GOLD["small_y"]))


def q8_blocks(pkg, scales, values):
    b = np.zeros(len(scales), pkg.Q8_BLOCK)
    b["scale_bits"] = scales
    b["values"] = values
    return b


def test_q8_known_answers(lib, pkg):
    """tests/test_phonon_q8.c:9-56 through the drop-in entry points."""
    k = GOLDEN["q8_known"]
    blocks = q8_blocks(pkg, [0x3800, 0x4000], [np.arange(32) - 16, np.ones(32)])
    x = np.ones(64, np.float32)
    out = np.zeros(1, np.float32)
    assert lib.phonon_q8_dot(blocks.ctypes.data, fp(x), 64, fp(out)) and out[0] == 56.0
    matrix = np.concatenate([blocks, blocks[::-1]])
    ok, y = gpu_q8_matvec(lib, matrix, x, 2, 64)
    assert ok and list(y) == k["matvec_rows"]
    assert not lib.phonon_q8_dot(blocks.ctypes.data, fp(x), 63, fp(out))
    assert not lib.phonon_q8_matvec(blocks.ctypes.data, fp(x), 1, 63, fp(out))
    assert not lib.phonon_q8_dot(None, fp(x), 32, fp(out))
    rows = q8_blocks(pkg, [0x3800, 0x4000, 0x3800, 0x4000],
                     [np.ones(32), 2 * np.ones(32), -np.ones(32), 3 * np.ones(32)])
    asym = np.concatenate([np.ones(32), 2 * np.ones(32)]).astype(np.float32)
    ok, y = gpu_q8_matvec(lib, rows, asym, 2, 64)
    assert ok and list(y) == k["asymmetric_rows"]
    # Overlapping output and input / weights are rejected.
    assert not lib.phonon_q8_matvec(rows.ctypes.data, fp(asym), 2, 64, fp(asym))
    assert not lib.phonon_q8_matvec(rows.ctypes.data, fp(asym), 2, 64,
                                    ctypes.cast(rows.ctypes.data, ctypes.POINTER(ctypes.c_float)))
    inf_scale = q8_blocks(pkg, [0x7C00], [np.ones(32)])
    assert not lib.phonon_q8_dot(inf_scale.ctypes.data, fp(np.ones(32, np.float32)), 32, fp(out))
    sub = q8_blocks(pkg, [0x0001], [np.ones(32)])
    ones = np.ones(32, np.float32)
    assert lib.phonon_q8_dot(sub.ctypes.data, fp(ones), 32, fp(out))
    assert out[0] == k["subnormal_scale_dot"]
    ones[0] = np.inf
    assert not lib.phonon_q8_dot(sub.ctypes.data, fp(ones), 32, fp(out))


@pytest.mark.parametrize("batch", [1, 3, 16, 17, 64])
def test_q8_device_matvec_batches(lib, oracle, syn, pkg, batch):
    rng = np.random.default_rng(100 + batch)
    rows, cols = 512, 2048
    w = syn.q8_matrix(rng, rows, cols)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    handle = ctypes.c_void_p()
    assert lib.phonon_q8_device_create(w.ctypes.data, rows, cols, 2, ctypes.byref(handle))
    dx = pkg.DeviceBuffer(lib, x.nbytes)
    dy = pkg.DeviceBuffer(lib, batch * rows * 4)
    dx.upload(x)
    for copy in (0, 1):
        assert lib.phonon_q8_device_matvec(handle, copy, dx.ptr, dy.ptr, batch, None)
        assert lib.phonon_q8_device_status(handle, None)
        y = dy.download((batch, rows))
        for b in range(batch):
            ok, yo = oracle.q8_matvec(w, x[b], rows, cols)
            assert ok and helpers.normwise(y[b], yo) <= TOL, (copy, b)
    lib.phonon_q8_device_destroy(handle)


@pytest.mark.parametrize("batch", [1, 5, 17, 64])
def test_q8_device_matvec_512_columns_rows_path(lib, oracle, syn, pkg, batch):
    """The config-1 shape (2048 x 512): 512-column matrices take the one-launch
    path that splits the fp32 rows inside the projection; against the oracle
    from an input at a 16-byte offset into its buffer. An input or output
    that is not 16-byte aligned is rejected before any launch."""
    rng = np.random.default_rng(300 + batch)
    rows, cols = 2048, 512
    w = syn.q8_matrix(rng, rows, cols)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    handle = ctypes.c_void_p()
    assert lib.phonon_q8_device_create(w.ctypes.data, rows, cols, 1, ctypes.byref(handle))
    padded = np.concatenate([np.zeros(4, np.float32), x.ravel()])  # x at byte 16 and at 4
    dx = pkg.DeviceBuffer(lib, padded.nbytes)
    dx.upload(padded)
    dy = pkg.DeviceBuffer(lib, batch * rows * 4)
    assert lib.phonon_q8_device_matvec(handle, 0, dx.ptr + 16, dy.ptr, batch, None)
    assert lib.phonon_q8_device_status(handle, None)
    y = dy.download((batch, rows))
    for b in range(batch):
        ok, yo = oracle.q8_matvec(w, x[b], rows, cols)
        assert ok and helpers.normwise(y[b], yo) <= TOL, b
    assert not lib.phonon_q8_device_matvec(handle, 0, dx.ptr + 12, dy.ptr, batch, None)
    assert not lib.phonon_q8_device_matvec(handle, 0, dx.ptr + 16, dy.ptr + 4, batch, None)
    lib.phonon_q8_device_destroy(handle)


@pytest.mark.parametrize("rows,cols", [(2048, 512), (512, 2048), (48, 64)])
@pytest.mark.parametrize("batch", [1, 2, 5, 8])
def test_q8_device_matvec_valu_bits(lib, oracle, syn, pkg, rows, cols, batch):
    """phonon_q8_device_matvec_valu (pgpu_q8_gemv, vector units, batch <= 8)
    gives the oracle's bits (the reference's arithmetic) for every stream;
    batch 9, a column count that is not 32 x a divisor of 64, and a
    misaligned input are rejected."""
    rng = np.random.default_rng(rows + cols + batch)
    w = syn.q8_matrix(rng, rows, cols)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    handle = ctypes.c_void_p()
    assert lib.phonon_q8_device_create(w.ctypes.data, rows, cols, 2, ctypes.byref(handle))
    dx = pkg.DeviceBuffer(lib, x.nbytes + 16)
    dx.upload(x)
    dy = pkg.DeviceBuffer(lib, 8 * rows * 4)
    for copy in (0, 1):
        assert lib.phonon_q8_device_matvec_valu(handle, copy, dx.ptr, dy.ptr, batch, None)
        assert lib.phonon_q8_device_status(handle, None)
        y = dy.download((batch, rows))
        for b in range(batch):
            ok, yo = oracle.q8_matvec(w, x[b], rows, cols)
            assert ok and np.array_equal(bits(y[b]), bits(yo)), (copy, b)
    assert not lib.phonon_q8_device_matvec_valu(handle, 0, dx.ptr, dy.ptr, 9, None)
    assert not lib.phonon_q8_device_matvec_valu(handle, 0, dx.ptr + 4, dy.ptr, 1, None)
    lib.phonon_q8_device_destroy(handle)
    if cols == 64:
        w96 = syn.q8_matrix(rng, 16, 96)
        h96 = ctypes.c_void_p()
        assert lib.phonon_q8_device_create(w96.ctypes.data, 16, 96, 1, ctypes.byref(h96))
        assert not lib.phonon_q8_device_matvec_valu(h96, 0, dx.ptr, dy.ptr, 1, None)
        lib.phonon_q8_device_destroy(h96)


def test_q8_matvec_valu_flags_nonfinite(lib, syn, pkg):
    """A non-finite input reaching the vector-unit kernel is reported."""
    rng = np.random.default_rng(7)
    w = syn.q8_matrix(rng, 64, 512)
    x = rng.standard_normal((2, 512)).astype(np.float32)
    x[1, 100] = np.nan
    handle = ctypes.c_void_p()
    assert lib.phonon_q8_device_create(w.ctypes.data, 64, 512, 1, ctypes.byref(handle))
    dx = pkg.DeviceBuffer(lib, x.nbytes)
    dx.upload(x)
    dy = pkg.DeviceBuffer(lib, 2 * 64 * 4)
    assert lib.phonon_q8_device_matvec_valu(handle, 0, dx.ptr, dy.ptr, 2, None)
    assert not lib.phonon_q8_device_status(handle, None)
    assert lib.phonon_q8_device_status(handle, None)  # the record was cleared
    lib.phonon_q8_device_destroy(handle)


# ------------------------------------------------------------------- linear
def test_linear_bf16_known_answer(lib, pkg):
    g = GOLDEN["linear_bf16"]
    v = pkg.Views()
    view = v.bf16(np.array(g["weight_bits"], np.uint16), g["shape"])
    y = np.zeros(2, np.float32)
    x = np.array(g["input"], np.float32)
    assert lib.phonon_linear(ctypes.byref(view), fp(x), 2, 2, None, fp(y))
    assert list(y) == g["expected"]


def test_linear_q8_scale_cases(lib, pkg):
    g = GOLDEN["linear_q8_scales"]
    blocks = q8_blocks(pkg, g["scale_bits"], [np.ones(32), np.ones(32)])
    v = pkg.Views()
    view = v.q8(blocks, 2, 32)
    y = np.zeros(2, np.float32)
    x = np.ones(32, np.float32)
    assert lib.phonon_linear(ctypes.byref(view), fp(x), 2, 32, None, fp(y))
    assert list(y) == g["expected"]
    for bad in g["rejected_scale_bits"]:
        blocks["scale_bits"][0] = bad
        view = v.q8(blocks, 2, 32)
        assert not lib.phonon_linear(ctypes.byref(view), fp(x), 2, 32, None, fp(y))


@pytest.mark.parametrize("kind", ["q8", "bf16"])
def test_linear_batch_random_vs_oracle(lib, oracle, syn, pkg, kind):
    rng = np.random.default_rng(31)
    rows, cols, batch = 1536, 512, 7
    v = pkg.Views()
    if kind == "q8":
        w = syn.q8_matrix(rng, rows, cols)
        view = v.q8(w, rows, cols)
        ok, dense = oracle.q8_expand(w, rows, cols)
    else:
        wb = syn.bf16_bits(rng.standard_normal((rows, cols)).astype(np.float32) * 0.05)
        view = v.bf16(wb, (rows, cols))
        ok, dense = oracle.bf16_to_float(wb.reshape(-1))
        dense = dense.reshape(rows, cols)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    bias = rng.standard_normal(rows).astype(np.float32)
    y = np.zeros((batch, rows), np.float32)
    assert lib.phonon_linear_batch(ctypes.byref(view), fp(x), rows, cols, fp(bias), fp(y), batch)
    ok, yo = oracle.linear_batch(dense, x, bias)
    for b in range(batch):
        assert helpers.normwise(y[b], yo[b]) <= TOL
        assert helpers.elementwise_ok(y[b], yo[b])


def test_linear_odd_shapes_pad_correctly(lib, oracle, syn, pkg):
    """rows not a multiple of 16, BF16 columns not a multiple of 32."""
    rng = np.random.default_rng(32)
    rows, cols, batch = 37, 45, 3
    wb = syn.bf16_bits(rng.standard_normal((rows, cols)).astype(np.float32))
    v = pkg.Views()
    view = v.bf16(wb, (rows, cols))
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    y = np.zeros((batch, rows), np.float32)
    assert lib.phonon_linear_batch(ctypes.byref(view), fp(x), rows, cols, None, fp(y), batch)
    ok, dense = oracle.bf16_to_float(wb.reshape(-1))
    ok, yo = oracle.linear_batch(dense.reshape(rows, cols), x)
    assert helpers.normwise(y, yo) <= TOL


# -------------------------------------------------------------- norms / GELU
def test_layer_norm_regression_and_random(lib, oracle):
    g = GOLDEN["layer_norm_regression"]
    x = np.array(g["input_bits"], np.uint32).view(np.float32)
    w = np.ones(512, np.float32)
    b = np.zeros(512, np.float32)
    y = np.zeros(512, np.float32)
    assert lib.phonon_layer_norm(fp(x), fp(w), fp(b), 512, 1e-5, fp(y))
    ok, yo = oracle.layer_norm(x, w, b)
    assert helpers.normwise(y, yo) <= 1e-6
    rng = np.random.default_rng(41)
    for width in (3, 512, 1000):
        x = (rng.standard_normal(width) * 7 + 2).astype(np.float32)
        w = rng.standard_normal(width).astype(np.float32)
        b = rng.standard_normal(width).astype(np.float32)
        y = np.zeros(width, np.float32)
        assert lib.phonon_layer_norm(fp(x), fp(w), fp(b), width, 1e-5, fp(y))
        ok, yo = oracle.layer_norm(x, w, b)
        assert helpers.normwise(y, yo) <= 1e-5
        assert lib.phonon_rms_norm(fp(x), fp(w), width, 1e-5, fp(y))
        ok, yo = oracle.rms_norm(x, w)
        assert helpers.normwise(y, yo) <= 1e-6
    x[0] = np.nan
    assert not lib.phonon_layer_norm(fp(x), fp(w), fp(b), width, 1e-5, fp(y))


def test_gelu_golden_and_random(lib, oracle):
    g = GOLDEN["gelu"]
    v = np.array(g["inputs"], np.float32)
    assert lib.phonon_erf_gelu(fp(v), v.size)
    want = np.array(g["expected_bits"], np.uint32).view(np.float32)
    assert np.max(np.abs(v - want)) <= 2e-7
    x = np.linspace(-9, 9, 20011).astype(np.float32)
    v = x.copy()
    assert lib.phonon_erf_gelu(fp(v), v.size)
    ok, yo = oracle.erf_gelu(x)
    assert np.max(np.abs(v - yo) / np.maximum(np.abs(yo), 1.0)) <= 2e-6
    bad = np.array([1.0, np.inf], np.float32)
    assert not lib.phonon_erf_gelu(fp(bad), 2)
    assert lib.phonon_erf_gelu(None, 0)


def test_rope_bit_exact_vs_oracle(lib, oracle):
    g = GOLDEN["rope"]
    for pos, want in zip(g["positions"], g["expected"]):
        row = np.zeros(64, np.float32)
        row[2:4] = g["pair_in"]
        assert lib.phonon_rope_interleaved(fp(row), 64, 1, pos, g["theta"])
        assert np.all(np.abs(row[2:4] - want) < g["tolerance"])
    rng = np.random.default_rng(43)
    for pos in (0, 1, 139, 4096, 8191):
        v = rng.standard_normal(512).astype(np.float32)
        ok, ro = oracle.rope(v, 8, pos)
        assert lib.phonon_rope_interleaved(fp(v), 512, 8, pos, 10000.0)
        assert np.array_equal(bits(v), bits(ro)), pos
    assert not lib.phonon_rope_interleaved(fp(v), 4, 3, 0, 10000.0)


# ---------------------------------------------------------------- attention
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


def gpu_attention(lib, q, k, v, count, stride):
    out = np.full(64, np.nan, np.float32)
    ok = lib.phonon_attention_test(fp(q), fp(k), fp(v), count, stride, fp(out))
    return bool(ok), out


def test_attention_golden_cases(lib):
    for c in GOLDEN["attention_cases"]["cases"]:
        q, k, v = attention_case(c["count"], c["middle"], c["tail"])
        ok, out = gpu_attention(lib, q, k, v, c["count"], 64)
        want = np.array([c["expected_bits"]], np.uint32).view(np.float32)[0]
        assert ok and abs(out[0] - want) <= TOL * abs(want), (c, out[0], want)
        assert np.all(out[1:] == 0)


def test_attention_single_key_is_exact(lib):
    rng = np.random.default_rng(51)
    q = rng.standard_normal(64).astype(np.float32)
    k = rng.standard_normal((1, 64)).astype(np.float32)
    v = rng.standard_normal((1, 64)).astype(np.float32)
    ok, out = gpu_attention(lib, q, k, v, 1, 64)
    assert ok and np.array_equal(out, v[0])


@pytest.mark.parametrize("count", [1, 2, 15, 16, 17, 63, 64, 65, 255, 256, 257, 511, 512, 513,
                                   1024, 2047, 2048, 2049, 4100, 8192])
def test_attention_vs_oracle(lib, oracle, count):
    rng = np.random.default_rng(1000 + count)
    stride = 512
    k = rng.standard_normal((count, stride)).astype(np.float32)
    v = rng.standard_normal((count, stride)).astype(np.float32)
    q = (rng.standard_normal(64) * 2).astype(np.float32)
    h = 5
    # Head 5 of 512-wide rows: row i of the head starts at i*512 + 320.
    kh = k.reshape(-1)[h * 64:]
    vh = v.reshape(-1)[h * 64:]
    ok, out = gpu_attention(lib, q, kh, vh, count, stride)
    ok2, ref = oracle.attention(q, kh, vh, count, stride)
    assert ok and ok2
    assert helpers.normwise(out, ref) <= TOL and helpers.elementwise_ok(out, ref)


def test_attention_rejects_bad_arguments(lib):
    q = np.zeros(64, np.float32)
    k = np.zeros((4, 64), np.float32)
    out = np.zeros(64, np.float32)
    assert not lib.phonon_attention_test(fp(q), fp(k), fp(k), 0, 64, fp(out))
    assert not lib.phonon_attention_test(fp(q), fp(k), fp(k), 4, 63, fp(out))
    assert not lib.phonon_attention_test(fp(q), fp(k), fp(k), 8193, 64, fp(out))
    k[1, 3] = np.nan
    assert not lib.phonon_attention_test(fp(q), fp(k), fp(k), 4, 64, fp(out))


@pytest.mark.parametrize("rows,width", [(1, 1), (7, 300), (4096, 512)])
def test_gather_rows_copy(lib, pkg, rows, width):
    """The table gather of a batched prefill: row r of dst is row map[r] of
    src, and the same launch copies one value per row (the positions)."""
    rng = np.random.default_rng(rows + width)
    src_rows = 16
    src = rng.integers(-2**31, 2**31 - 1, size=(src_rows, width), dtype=np.int64).astype(np.int32)
    mp = rng.integers(0, src_rows, size=rows).astype(np.int32)
    vals = rng.integers(0, 8192, size=rows).astype(np.int32)
    d_src, d_map, d_vals = (pkg.DeviceBuffer(lib, a.nbytes) for a in (src, mp, vals))
    d_src.upload(src), d_map.upload(mp), d_vals.upload(vals)
    d_dst = pkg.DeviceBuffer(lib, rows * width * 4)
    d_copy = pkg.DeviceBuffer(lib, rows * 4)
    assert lib.pgpu_gather_rows_copy(None, d_dst.ptr, d_src.ptr, d_map.ptr, rows, width,
                                     d_copy.ptr, d_vals.ptr), pkg.last_error(lib)
    assert np.array_equal(d_dst.download((rows, width), np.int32), src[mp])
    assert np.array_equal(d_copy.download(rows, np.int32), vals)
    # Without the copy pair it is pgpu_gather_rows; half a pair is refused.
    assert lib.pgpu_gather_rows(None, d_dst.ptr, d_src.ptr, d_map.ptr, rows, width)
    assert not lib.pgpu_gather_rows_copy(None, d_dst.ptr, d_src.ptr, d_map.ptr, rows, width,
                                         d_copy.ptr, None)
    for b in (d_src, d_map, d_vals, d_dst, d_copy):
        b.free()
