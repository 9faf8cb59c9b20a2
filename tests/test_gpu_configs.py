"""GPU parity at the benchmark workloads themselves, through the C-ABI:

- B=1, 12 layers: a 256-position prefill (batched prefill entry point, and
  separately the 9-layer drop-in phonon_flow_stack_prefill) followed by 16
  decode steps, every output against the oracle;
- the large-batch workload's prefill leg: 16 fresh streams x 256 positions
  (4096 pseudo-streams) through one batched prefill, every position against
  the oracle, and two streams bit for bit against single decode steps;
- the benchmark weight distribution through all 12 layers: at 1e-4 of the
  oracle in the decode benchmark's regime (N(0,1) contexts), and as close
  to float64 as the oracle is where the model's own context makes the
  stack ill-conditioned (the oracle itself ~1e-3 from float64 there);
- the closed per-frame loop (decode step, output norm, flow head LSD step,
  EOS logit, latent embedding into the next step's input) over several
  frames, on the batch's stream and on the head's own stream with events.

Tolerances: 1e-4 normwise relative (fp32 paths); bit-exact where the same
arithmetic runs twice."""
import ctypes

import numpy as np
import pytest

import helpers
from test_gpu_decode import Batch, Cache, fp, i32p, set_step_mode

pytestmark = pytest.mark.gpu
TOL = 1e-4
SZP = ctypes.POINTER(ctypes.c_size_t)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# ------------------------------------------------------------ B=1, 12 layers
C3_LAYERS, C3_PREFILL, C3_STEPS = 12, 256, 16


@pytest.fixture(scope="module")
def config3(oracle, oracle_mod, syn):
    """The oracle's run of the B=1 workload: 256 prefill positions then 16
    decode steps through 12 layers, layer by layer, so the outputs after the
    first 9 layers (the drop-in's PHONON_FLOW_LAYERS model: the same first
    nine layers) come from the same run. The K/V of layers 0..8 are the
    same in both models."""
    model = helpers.scaled_model(syn, 301, C3_LAYERS)
    om = oracle_mod.OracleModel(oracle, helpers.oracle_layers(oracle, model))
    rng = np.random.default_rng(302)
    total = C3_PREFILL + C3_STEPS
    xs = rng.standard_normal((total, 512)).astype(np.float32)
    keys = np.zeros((C3_LAYERS, total, 512), np.float32)
    vals = np.zeros_like(keys)
    out9 = np.zeros((total, 512), np.float32)
    out12 = np.zeros((total, 512), np.float32)
    for p in range(total):
        a = xs[p]
        for layer in range(C3_LAYERS):
            ok, a = om.layer_step(keys, vals, total, layer, p, a)
            assert ok
            if layer == 8:
                out9[p] = a
        out12[p] = a
    return {"model": model, "xs": xs, "keys": keys, "vals": vals, "out9": out9,
            "out12": out12, "total": total}


def test_config3_batched_prefill_then_decode_vs_oracle(lib, pkg, config3):
    """phonon_flow_batch_prefill_device over the 256-position prompt, then 16
    decode steps in the library's default mode (one launch at B=1): every
    prefill position, every step and the whole appended cache at 1e-4."""
    c = config3
    views = pkg.Views()
    w = views.layers(c["model"])
    total = c["total"]
    table_len = (total + 15) // 16
    blocks = table_len + 7
    bt = Batch(lib, w, C3_LAYERS, C3_PREFILL, total, blocks)
    ids = np.zeros(blocks, np.int32)
    assert lib.phonon_kv_pool_alloc(bt.pool, blocks, i32p(ids))
    table = np.ascontiguousarray(np.random.default_rng(303).permutation(ids)[:table_len])
    din = pkg.DeviceBuffer(lib, C3_PREFILL * 512 * 4)
    dout = pkg.DeviceBuffer(lib, C3_PREFILL * 512 * 4)
    din.upload(c["xs"][:C3_PREFILL])
    first = np.array([0], np.uintp)
    counts = np.array([C3_PREFILL], np.uintp)
    assert lib.phonon_flow_batch_prefill_device(
        bt.batch, 1, first.ctypes.data_as(SZP), counts.ctypes.data_as(SZP), i32p(table),
        table_len, din.ptr, 10000.0, dout.ptr), pkg.last_error(lib)
    assert lib.phonon_flow_batch_sync(bt.batch)
    got = dout.download((C3_PREFILL, 512))
    errs = [helpers.normwise(got[p], c["out12"][p]) for p in range(C3_PREFILL)]
    print("config 3 prefill: max normwise error", max(errs), "at", int(np.argmax(errs)))
    assert max(errs) <= TOL
    pos = np.array([C3_PREFILL], np.uintp)
    assert lib.phonon_flow_batch_set_streams(bt.batch, 1, pos.ctypes.data_as(SZP), i32p(table),
                                             table_len)
    worst = 0.0
    for t in range(C3_STEPS):
        p = C3_PREFILL + t
        y = np.zeros((1, 512), np.float32)
        assert lib.phonon_flow_batch_step(bt.batch, fp(np.ascontiguousarray(c["xs"][p:p + 1])),
                                          10000.0, fp(y)), pkg.last_error(lib)
        err = helpers.normwise(y[0], c["out12"][p])
        worst = max(worst, err)
        assert err <= TOL, (t, err)
    print("config 3 decode steps: max normwise error", worst)
    k = np.zeros((C3_LAYERS, total, 512), np.float32)
    v = np.zeros_like(k)
    assert lib.phonon_kv_pool_read(bt.pool, i32p(table), table_len, 0, total, fp(k), fp(v),
                                   total)
    assert helpers.normwise(k, c["keys"]) <= TOL and helpers.normwise(v, c["vals"]) <= TOL
    din.free()
    dout.free()
    bt.close()


def test_config3_dropin_prefill_then_steps_vs_oracle(lib, pkg, config3):
    """The reference-signature path: phonon_flow_stack_prefill of the same
    256 positions into a PhononKvCache (PHONON_FLOW_LAYERS = 9), then 16
    phonon_flow_stack_step calls; the returned output, every step and the
    host cache mirror at 1e-4."""
    c = config3
    views = pkg.Views()
    w = views.layers(c["model"][:9])
    total = c["total"]
    cache = Cache(lib, total)
    out = np.zeros(512, np.float32)
    assert lib.phonon_flow_stack_prefill(w, cache.ref(), fp(np.ascontiguousarray(
        c["xs"][:C3_PREFILL])), C3_PREFILL, 10000.0, fp(out)), pkg.last_error(lib)
    assert cache.c.length == C3_PREFILL
    err = helpers.normwise(out, c["out9"][C3_PREFILL - 1])
    print("config 3 drop-in prefill: normwise error", err)
    assert err <= TOL
    for t in range(C3_STEPS):
        p = C3_PREFILL + t
        y = np.zeros(512, np.float32)
        assert lib.phonon_flow_stack_step(w, cache.ref(), p, fp(np.ascontiguousarray(c["xs"][p])),
                                          10000.0, fp(y)), pkg.last_error(lib)
        assert cache.c.length == p + 1
        assert helpers.normwise(y, c["out9"][p]) <= TOL, (t, helpers.normwise(y, c["out9"][p]))
    assert helpers.normwise(cache.keys(), c["keys"][:9]) <= TOL
    assert helpers.normwise(cache.values(), c["vals"][:9]) <= TOL
    cache.destroy()


# ------------------------------------------- the large-batch prefill leg
C5_LAYERS, C5_STREAMS, C5_CHUNK = 12, 16, 256


def test_config5_prefill_leg_vs_oracle(lib, pkg, oracle, oracle_mod, syn):
    """The large-batch workload's prefill: 16 newly admitted streams x 256
    positions through all 12 layers in one batched prefill (4096
    pseudo-streams; the benchmark's batch shape, 8192-position tables,
    shuffled pool blocks). With the default (matrix-core) prefill attention,
    every position of every stream and the appended K/V of two streams
    against the oracle at 1e-4. With the exact prefill attention, those two
    streams decoded one position at a time give the same bits (outputs and
    K/V); the matrix-core and the lane-per-query runs (projections on two
    fp16 split terms; the matrix-core attention on fp16 pairs too) stay
    within 1e-4 of the exact one everywhere."""
    model = helpers.scaled_model(syn, 311, C5_LAYERS)
    views = pkg.Views()
    w = views.layers(model)
    max_pos, n = 8192, C5_STREAMS * C5_CHUNK
    table_len = max_pos // 16
    used = C5_CHUNK // 16
    rng = np.random.default_rng(312)
    xs = rng.standard_normal((C5_STREAMS, C5_CHUNK, 512)).astype(np.float32)
    blocks = C5_STREAMS * used
    tables = np.zeros((C5_STREAMS, table_len), np.int32)
    checked = (0, C5_STREAMS - 1)

    def prefill(exact):
        print(f"config 5 prefill leg: exact={exact}", flush=True)
        bt = Batch(lib, w, C5_LAYERS, n, max_pos, blocks)
        assert lib.phonon_flow_batch_set_prefill_exact(bt.batch, exact)
        ids = np.zeros(blocks, np.int32)
        assert lib.phonon_kv_pool_alloc(bt.pool, blocks, i32p(ids))
        tables[:, :used] = np.random.default_rng(313).permutation(ids).reshape(C5_STREAMS, used)
        din = pkg.DeviceBuffer(lib, n * 512 * 4)
        dout = pkg.DeviceBuffer(lib, n * 512 * 4)
        din.upload(xs.reshape(n, 512))
        first = np.zeros(C5_STREAMS, np.uintp)
        counts = np.full(C5_STREAMS, C5_CHUNK, np.uintp)
        assert lib.phonon_flow_batch_prefill_device(
            bt.batch, C5_STREAMS, first.ctypes.data_as(SZP), counts.ctypes.data_as(SZP),
            i32p(tables), table_len, din.ptr, 10000.0, dout.ptr), pkg.last_error(lib)
        assert lib.phonon_flow_batch_sync(bt.batch)
        got = dout.download((C5_STREAMS, C5_CHUNK, 512))
        kv_got = {}
        for s in checked:
            k = np.zeros((C5_LAYERS, C5_CHUNK, 512), np.float32)
            v = np.zeros_like(k)
            assert lib.phonon_kv_pool_read(bt.pool, i32p(tables[s]), table_len, 0, C5_CHUNK,
                                           fp(k), fp(v), C5_CHUNK)
            kv_got[s] = (k, v)
        din.free()
        dout.free()
        bt.close()
        return got, kv_got

    got, kv_got = prefill(0)
    exact, kv_exact = prefill(1)
    rows, _ = prefill(2)
    for name, other in (("matrix-core", got), ("lane-per-query", rows)):
        fast_vs_exact = max(helpers.normwise(other[s, p], exact[s, p])
                            for s in range(C5_STREAMS) for p in range(C5_CHUNK))
        print(f"config 5 prefill leg: {name} vs exact attention, max normwise", fast_vs_exact)
        assert fast_vs_exact <= 1e-4

    # The oracle: every stream's positions in order, streams on host threads.
    om = oracle_mod.OracleModel(oracle, helpers.oracle_layers(oracle, model))
    okeys = np.zeros((C5_STREAMS, C5_LAYERS, C5_CHUNK, 512), np.float32)
    ovals = np.zeros_like(okeys)
    worst = 0.0
    for p in range(C5_CHUNK):
        ok, ref = om.stack_step_streams(okeys, ovals, C5_CHUNK, np.full(C5_STREAMS, p),
                                        xs[:, p], 16)
        assert ok
        for s in range(C5_STREAMS):
            err = helpers.normwise(got[s, p], ref[s])
            worst = max(worst, err)
            assert err <= TOL, (s, p, err)
    print("config 5 prefill leg: max normwise error over 4096 positions", worst)
    for s in checked:
        assert helpers.normwise(kv_got[s][0], okeys[s]) <= TOL
        assert helpers.normwise(kv_got[s][1], ovals[s]) <= TOL

    # Single decode steps of the same two streams: the exact prefill's bits
    # (with the merge in the out projection: the one-stream default, the
    # fused MLP, orders the MLP-out sums differently).
    bt = Batch(lib, w, C5_LAYERS, 1, max_pos, blocks)
    assert lib.phonon_flow_batch_set_handoff(bt.batch, 3)
    ids = np.zeros(blocks, np.int32)
    assert lib.phonon_kv_pool_alloc(bt.pool, blocks, i32p(ids))
    for s in checked:
        table = np.ascontiguousarray(tables[s])
        pos = np.array([0], np.uintp)
        assert lib.phonon_flow_batch_set_streams(bt.batch, 1, pos.ctypes.data_as(SZP),
                                                 i32p(table), table_len)
        for p in range(C5_CHUNK):
            y = np.zeros((1, 512), np.float32)
            assert lib.phonon_flow_batch_step(bt.batch, fp(np.ascontiguousarray(xs[s, p:p + 1])),
                                              10000.0, fp(y)), pkg.last_error(lib)
            assert np.array_equal(bits(y[0]), bits(exact[s, p])), (s, p)
        k = np.zeros((C5_LAYERS, C5_CHUNK, 512), np.float32)
        v = np.zeros_like(k)
        assert lib.phonon_kv_pool_read(bt.pool, i32p(table), table_len, 0, C5_CHUNK, fp(k),
                                       fp(v), C5_CHUNK)
        assert np.array_equal(bits(k), bits(kv_exact[s][0]))
        assert np.array_equal(bits(v), bits(kv_exact[s][1]))
    bt.close()


def test_config5_prefill_at_benchmark_weights_vs_float64(lib, pkg, oracle, oracle_mod, syn):
    """The prefill the large-batch benchmark runs: 16 streams x 256
    positions through all 12 layers with the benchmark's own (unscaled)
    weights and N(0,1) inputs, in the default mode (matrix-core attention;
    every projection reads the three bf16 terms of each activation).

    At these weights the 12-layer stack over its own K/V is ill-conditioned:
    the oracle (fp32 in the reference's order) drifts up to ~5e-2 from a
    float64 restatement within 64 positions, so no fp32 order can be held to
    1e-2 of another everywhere. For eight streams' first 128 positions,
    replayed in float64: the GPU's worst and mean distance from float64 at
    most 3x the oracle's; and wherever the oracle is itself within 1e-3 of
    float64, the GPU within 1e-2 of the oracle (the tolerance of the bf16
    matrix-core path)."""
    layers, streams, chunk, checked = 12, 16, 256, 128
    model = syn.flow_model(2026, layers)
    ol = helpers.oracle_layers(oracle, model)
    om = oracle_mod.OracleModel(oracle, ol)
    views = pkg.Views()
    w = views.layers(model)
    max_pos, n = 8192, streams * chunk
    table_len = max_pos // 16
    used = chunk // 16
    rng = np.random.default_rng(2026 + 54)
    xs = rng.standard_normal((streams, chunk, 512)).astype(np.float32)
    blocks = streams * used
    tables = np.zeros((streams, table_len), np.int32)
    print("benchmark-weight prefill: 16 x 256 positions, 12 layers", flush=True)
    bt = Batch(lib, w, layers, n, max_pos, blocks)
    ids = np.zeros(blocks, np.int32)
    assert lib.phonon_kv_pool_alloc(bt.pool, blocks, i32p(ids))
    tables[:, :used] = np.random.default_rng(2026 + 52).permutation(ids).reshape(streams, used)
    din = pkg.DeviceBuffer(lib, n * 512 * 4)
    dout = pkg.DeviceBuffer(lib, n * 512 * 4)
    din.upload(xs.reshape(n, 512))
    first = np.zeros(streams, np.uintp)
    counts = np.full(streams, chunk, np.uintp)
    assert lib.phonon_flow_batch_prefill_device(
        bt.batch, streams, first.ctypes.data_as(SZP), counts.ctypes.data_as(SZP),
        i32p(tables), table_len, din.ptr, 10000.0, dout.ptr), pkg.last_error(lib)
    assert lib.phonon_flow_batch_sync(bt.batch)
    got = dout.download((streams, chunk, 512))
    din.free()
    dout.free()
    bt.close()
    assert np.all(np.isfinite(got))

    okeys = np.zeros((streams, layers, checked, 512), np.float32)
    ovals = np.zeros_like(okeys)
    ref = np.zeros((streams, checked, 512), np.float32)
    for p in range(checked):
        ok, ref[:, p] = om.stack_step_streams(okeys, ovals, checked, np.full(streams, p),
                                              xs[:, p], 16)
        assert ok

    ol64 = [{k: np.asarray(a, np.float64) for k, a in layer.items()} for layer in ol]
    e_gpu, e_oracle, tight = [], [], []
    for s in range(0, streams, 2):
        k64 = np.zeros((layers, checked, 512))
        v64 = np.zeros_like(k64)
        for p in range(checked):
            exact = xs[s, p].astype(np.float64)
            for layer in range(layers):
                exact = helpers.f64_layer(ol64[layer], exact, k64[layer], v64[layer], p)
            e_gpu.append(helpers.normwise(got[s, p], exact))
            e_oracle.append(helpers.normwise(ref[s, p], exact))
            if e_oracle[-1] <= 1e-3:
                tight.append(helpers.normwise(got[s, p], ref[s, p]))
    e_gpu, e_oracle, tight = np.array(e_gpu), np.array(e_oracle), np.array(tight)
    print(f"benchmark-weight prefill: from float64 worst GPU {e_gpu.max():.2e} oracle "
          f"{e_oracle.max():.2e}; mean GPU {e_gpu.mean():.2e} oracle {e_oracle.mean():.2e}; "
          f"{len(tight)} positions where the oracle is within 1e-3 of float64: GPU vs oracle "
          f"max {tight.max():.2e}")
    assert e_gpu.max() <= 3.0 * e_oracle.max()
    assert e_gpu.mean() <= 3.0 * e_oracle.mean()
    assert len(tight) >= 64 and tight.max() <= 1e-2


# ------------------------------------------------ benchmark weights, 12 layers
def test_benchmark_weights_full_stack_vs_oracle(lib, pkg, oracle, oracle_mod, syn):
    """The benchmark's own weight distribution (Q8 scales U[1e-3, 1e-2],
    unscaled) through all 12 layers at N(0,1) contexts U{1..2048} (the
    decode benchmark's regime): every stream at 1e-4 of the oracle; both are
    also printed against a float64 restatement of the stack."""
    layers, streams = 12, 12
    model = syn.flow_model(2026, layers)
    ol = helpers.oracle_layers(oracle, model)
    om = oracle_mod.OracleModel(oracle, ol)
    views = pkg.Views()
    w = views.layers(model)
    rng = np.random.default_rng(321)
    lengths = np.sort(rng.integers(1, 2049, size=streams) - 1)   # positions
    lengths[0] = 0
    max_pos = int(lengths.max()) + 1
    table_len = (max_pos + 15) // 16
    keys = rng.standard_normal((layers, max_pos, 512)).astype(np.float32)
    vals = rng.standard_normal((layers, max_pos, 512)).astype(np.float32)
    blocks = streams * table_len
    bt = Batch(lib, w, layers, streams, max_pos, blocks)
    ids = np.zeros(blocks, np.int32)
    assert lib.phonon_kv_pool_alloc(bt.pool, blocks, i32p(ids))
    tables = np.ascontiguousarray(rng.permutation(ids).reshape(streams, table_len))
    for s in range(streams):
        if lengths[s]:
            assert lib.phonon_kv_pool_write(bt.pool, i32p(tables[s]), table_len, 0,
                                            int(lengths[s]), fp(keys), fp(vals), max_pos)
    pos = lengths.astype(np.uintp)
    assert lib.phonon_flow_batch_set_streams(bt.batch, streams, pos.ctypes.data_as(SZP),
                                             i32p(tables), table_len)
    x = rng.standard_normal((streams, 512)).astype(np.float32)
    y = np.zeros_like(x)
    assert lib.phonon_flow_batch_step(bt.batch, fp(x), 10000.0, fp(y)), pkg.last_error(lib)
    bt.close()
    k64 = keys.astype(np.float64)
    v64 = vals.astype(np.float64)
    for s in range(streams):
        p = int(lengths[s])
        row_k, row_v = keys[:, p].copy(), vals[:, p].copy()
        ok, ref = om.stack_step(keys, vals, max_pos, p, x[s])
        keys[:, p], vals[:, p] = row_k, row_v
        assert ok
        exact = x[s].astype(np.float64)
        for layer in range(layers):
            exact = helpers.f64_layer(ol[layer], exact, k64[layer], v64[layer], p)
        k64[:, p], v64[:, p] = row_k, row_v
        err = helpers.normwise(y[s], ref)
        print(f"stream {s} position {p}: GPU vs oracle {err:.2e}; from float64: GPU "
              f"{helpers.normwise(y[s], exact):.2e}, oracle {helpers.normwise(ref, exact):.2e}")
        assert err <= TOL, (s, p, err)


def test_benchmark_weights_self_generated_context_vs_float64(lib, pkg, oracle, oracle_mod,
                                                             syn):
    """The same weights over 24 steps from position 0, each step's input
    N(0,1): the context is the model's own K/V, softmax saturates and the
    stack amplifies fp32 rounding, so the oracle itself is ~1e-3 from a
    float64 restatement. Neither fp32 order is the exact one; the GPU must
    be as close to float64 as the oracle is: over all steps of 4 streams,
    its worst and mean distances at most 3x the oracle's."""
    layers, streams, steps = 12, 4, 24
    model = syn.flow_model(81, layers)
    ol = helpers.oracle_layers(oracle, model)
    om = oracle_mod.OracleModel(oracle, ol)
    views = pkg.Views()
    w = views.layers(model)
    table_len = (steps + 15) // 16
    blocks = streams * table_len
    bt = Batch(lib, w, layers, streams, steps, blocks)
    ids = np.zeros(blocks, np.int32)
    assert lib.phonon_kv_pool_alloc(bt.pool, blocks, i32p(ids))
    tables = np.ascontiguousarray(np.random.default_rng(341).permutation(ids).reshape(
        streams, table_len))
    pos = np.zeros(streams, np.uintp)
    assert lib.phonon_flow_batch_set_streams(bt.batch, streams, pos.ctypes.data_as(SZP),
                                             i32p(tables), table_len)
    xs = np.random.default_rng(342).standard_normal((steps, streams, 512)).astype(np.float32)
    ys = np.zeros_like(xs)
    for t in range(steps):
        assert lib.phonon_flow_batch_step(bt.batch, fp(np.ascontiguousarray(xs[t])), 10000.0,
                                          fp(ys[t])), pkg.last_error(lib)
    bt.close()
    e_gpu, e_oracle = [], []
    for s in range(streams):
        keys = np.zeros((layers, steps, 512), np.float32)
        vals = np.zeros_like(keys)
        k64 = np.zeros((layers, steps, 512))
        v64 = np.zeros_like(k64)
        for t in range(steps):
            ok, ref = om.stack_step(keys, vals, steps, t, xs[t, s])
            assert ok
            exact = xs[t, s].astype(np.float64)
            for layer in range(layers):
                exact = helpers.f64_layer(ol[layer], exact, k64[layer], v64[layer], t)
            e_gpu.append(helpers.normwise(ys[t, s], exact))
            e_oracle.append(helpers.normwise(ref, exact))
    e_gpu, e_oracle = np.array(e_gpu), np.array(e_oracle)
    print(f"self-generated context, 12 layers: from float64 worst GPU {e_gpu.max():.2e} oracle "
          f"{e_oracle.max():.2e}; mean GPU {e_gpu.mean():.2e} oracle {e_oracle.mean():.2e}")
    assert e_gpu.max() <= 3.0 * e_oracle.max()
    assert e_gpu.mean() <= 3.0 * e_oracle.mean()


# ------------------------------------------------------- closed frame loop
def frame_head(pkg, lib, views, streams, seed):
    rng = np.random.default_rng(seed)
    bits_ = helpers.random_flow_head_bits(seed + 1)
    eos_w = helpers.bf16_bits(rng.standard_normal(512).astype(np.float32) * 0.05)
    eos_b = helpers.bf16_bits(np.array([0.125], np.float32))
    norm_w = helpers.bf16_bits(1.0 + 0.1 * rng.standard_normal(512).astype(np.float32))
    norm_b = helpers.bf16_bits(0.1 * rng.standard_normal(512).astype(np.float32))
    lin = helpers.bf16_bits(rng.standard_normal((512, 32)).astype(np.float32) * 0.2)
    head = views.flow_head(bits_)
    ew, eb = views.bf16(eos_w.reshape(1, 512), (1, 512)), views.bf16(eos_b, (1,))
    nw, nb = views.bf16(norm_w, (512,)), views.bf16(norm_b, (512,))
    lv = views.bf16(lin, (512, 32))
    dev = ctypes.c_void_p()
    assert lib.phonon_flow_head_device_create(ctypes.byref(head), ctypes.byref(ew),
                                              ctypes.byref(eb), streams, ctypes.byref(dev))
    assert lib.phonon_flow_head_device_set_frame(dev, ctypes.byref(nw), ctypes.byref(nb),
                                                 ctypes.byref(lv)), pkg.last_error(lib)
    floats = {k: helpers.bf16_float(v) for k, v in bits_.items()}
    return dev, (head, ew, eb, nw, nb, lv), {
        "head": floats, "eos_w": helpers.bf16_float(eos_w), "eos_b": helpers.bf16_float(eos_b),
        "norm_w": helpers.bf16_float(norm_w), "norm_b": helpers.bf16_float(norm_b),
        "lin": helpers.bf16_float(lin)}


@pytest.mark.parametrize("shared_stream", [True, False])
def test_closed_frame_loop_vs_oracle(lib, pkg, oracle, oracle_mod, syn, shared_stream):
    """Several frames of the generation loop (src/phonon_sampler.c:447-483)
    on the GPU with no host synchronisation between them: the decode step
    (phonon_flow_batch_step_device), then phonon_flow_head_device_frame
    (output norm, LSD step with that frame's raw noise, EOS logit, and the
    next step's input = input_linear . latent + condition). The head runs on
    the batch's stream, or on its own stream with events handing each frame
    over both ways. Each frame's decode output, latent, EOS logit and next
    input are kept in their own buffers and compared, per stream, with the
    oracle's own closed loop (stack step, LayerNorm, LSD step, EOS logit,
    linear + condition) at 1e-4; positions advance by one per frame."""
    layers, streams, frames, temp = 2, 21, 4, 0.7
    model = helpers.scaled_model(syn, 331, layers)
    om = oracle_mod.OracleModel(oracle, helpers.oracle_layers(oracle, model))
    views = pkg.Views()
    w = views.layers(model)
    rng = np.random.default_rng(332)
    lengths = rng.integers(0, 300, size=streams)
    lengths[0] = 0
    max_pos = int(lengths.max()) + frames
    table_len = (max_pos + 15) // 16
    blocks = streams * table_len
    bt = Batch(lib, w, layers, streams, max_pos, blocks)
    ids = np.zeros(blocks, np.int32)
    assert lib.phonon_kv_pool_alloc(bt.pool, blocks, i32p(ids))
    tables = np.ascontiguousarray(rng.permutation(ids).reshape(streams, table_len))
    okeys = np.zeros((streams, layers, max_pos, 512), np.float32)
    ovals = np.zeros_like(okeys)
    for s in range(streams):
        n = int(lengths[s])
        if n:
            okeys[s, :, :n] = rng.standard_normal((layers, n, 512))
            ovals[s, :, :n] = rng.standard_normal((layers, n, 512))
            assert lib.phonon_kv_pool_write(bt.pool, i32p(tables[s]), table_len, 0, n,
                                            fp(okeys[s]), fp(ovals[s]), max_pos)
    pos = lengths.astype(np.uintp)
    assert lib.phonon_flow_batch_set_streams(bt.batch, streams, pos.ctypes.data_as(SZP),
                                             i32p(tables), table_len)
    dev, keep, hw = frame_head(pkg, lib, views, streams, 333)
    bstream = lib.phonon_flow_batch_stream(bt.batch)
    if shared_stream:
        assert lib.phonon_flow_head_device_set_stream(dev, bstream)
    hstream = lib.phonon_flow_head_device_stream(dev)
    assert (hstream == bstream) == shared_stream
    x0 = rng.standard_normal((streams, 512)).astype(np.float32)
    cond = rng.standard_normal((streams, 512)).astype(np.float32)
    raw = rng.standard_normal((frames, streams, 32)).astype(np.float32)
    row = streams * 512 * 4
    ins = [pkg.DeviceBuffer(lib, row) for _ in range(frames + 1)]
    outs = [pkg.DeviceBuffer(lib, row) for _ in range(frames)]
    lats = [pkg.DeviceBuffer(lib, streams * 32 * 4) for _ in range(frames)]
    eoss = [pkg.DeviceBuffer(lib, streams * 4) for _ in range(frames)]
    raws = [pkg.DeviceBuffer(lib, streams * 32 * 4) for _ in range(frames)]
    dcond = pkg.DeviceBuffer(lib, row)
    ins[0].upload(x0)
    dcond.upload(cond)
    for f in range(frames):
        raws[f].upload(raw[f])
    assert lib.pgpu_stream_sync(None)
    decoded, framed = ctypes.c_void_p(), ctypes.c_void_p()
    assert lib.pgpu_event_create(ctypes.byref(decoded))
    assert lib.pgpu_event_create(ctypes.byref(framed))
    for f in range(frames):
        assert lib.phonon_flow_batch_step_device(bt.batch, ins[f].ptr, 10000.0, outs[f].ptr)
        if not shared_stream:
            assert lib.pgpu_event_record(decoded, bstream)
            assert lib.pgpu_stream_wait_event(hstream, decoded)
        assert lib.phonon_flow_head_device_frame(dev, streams, outs[f].ptr, dcond.ptr,
                                                 raws[f].ptr, temp, lats[f].ptr, eoss[f].ptr,
                                                 ins[f + 1].ptr), pkg.last_error(lib)
        if not shared_stream:
            assert lib.pgpu_event_record(framed, hstream)
            assert lib.pgpu_stream_wait_event(bstream, framed)
    assert lib.phonon_flow_batch_sync(bt.batch) and lib.phonon_flow_head_device_sync(dev)
    got = {"out": [b.download((streams, 512)) for b in outs],
           "lat": [b.download((streams, 32)) for b in lats],
           "eos": [b.download((streams,)) for b in eoss],
           "next": [b.download((streams, 512)) for b in ins[1:]]}
    now = np.zeros(streams, np.uintp)
    assert lib.phonon_flow_batch_positions(bt.batch, now.ctypes.data_as(SZP))
    assert np.array_equal(now, lengths + frames)

    oh = oracle_mod.OracleHead(oracle, hw["head"])
    worst = 0.0
    for s in range(streams):
        x = x0[s]
        for f in range(frames):
            ok, y = om.stack_step(okeys[s], ovals[s], max_pos, int(lengths[s]) + f, x)
            assert ok
            ok, state = oracle.layer_norm(y, hw["norm_w"], hw["norm_b"], 1e-5)
            assert ok
            ok, lat = oh.lsd_one_step(state, raw[f, s], temp)
            assert ok
            ok, eos = oh.eos_logit(hw["eos_w"], hw["eos_b"], state)
            assert ok
            ok, emb = oracle.linear_batch(hw["lin"], lat)
            assert ok
            x = (emb[0] + cond[s]).astype(np.float32)
            errs = (helpers.normwise(got["out"][f][s], y), helpers.normwise(got["lat"][f][s], lat),
                    abs(float(got["eos"][f][s]) - eos) / max(1.0, abs(eos)),
                    helpers.normwise(got["next"][f][s], x))
            worst = max(worst, *errs)
            assert max(errs) <= TOL, (s, f, errs)
    print(f"closed frame loop ({'shared' if shared_stream else 'own'} stream): max error {worst:.2e}")
    for b in ins + outs + lats + eoss + raws + [dcond]:
        b.free()
    lib.pgpu_event_destroy(decoded)
    lib.pgpu_event_destroy(framed)
    lib.phonon_flow_head_device_destroy(dev)
    bt.close()
    del keep
