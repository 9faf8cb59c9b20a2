"""GPU parity of the flow head (phonon_sampler.h) through the C-ABI: the
reference-signature functions against the reference's own synthetic-head
golden vector and the oracle, and the batched device LSD step (with the EOS
logit) against the oracle per stream. Tolerance: 1e-4 normwise relative
(fp32-accurate projections; device expf/sincosf vs libm)."""
import ctypes

import numpy as np
import pytest

import helpers

pytestmark = pytest.mark.gpu
TOL = 1e-4
GOLD = __import__("json").load(open(helpers.GOLDEN_DIR + "/reference_vectors.json"))


def fp(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def float_head(bits):
    return {k: helpers.bf16_float(v) for k, v in bits.items()}


def rel(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - b)) / max(np.max(np.abs(b)), 1e-30))


def test_head_forward_matches_reference_golden(lib, pkg, oracle, oracle_mod):
    """The reference's synthetic head (tests/test_phonon_sampler.c:148-195):
    velocity at (s, t) = (0, 1) within the reference test's 2e-4 of its
    PyTorch values, and within 1e-4 of the oracle."""
    g = GOLD["flow_head_synthetic"]
    bits = helpers.reference_flow_head_bits()
    views = pkg.Views()
    head = views.flow_head(bits)
    condition, state = helpers.reference_flow_head_inputs()
    out = np.zeros(32, np.float32)
    assert lib.phonon_flow_head_forward(ctypes.byref(head), fp(condition), fp(state), 0.0, 1.0,
                                        fp(out)), pkg.last_error(lib)
    assert np.max(np.abs(out - np.asarray(g["expected"], np.float32))) < g["tolerance"]
    ok, ref = oracle_mod.OracleHead(oracle, float_head(bits)).forward(condition, state, 0.0, 1.0)
    assert ok and rel(out, ref) < TOL
    lib.phonon_flow_head_release(ctypes.byref(head))


def test_head_forward_other_flow_times(lib, pkg, oracle, oracle_mod):
    bits = helpers.random_flow_head_bits(21)
    views = pkg.Views()
    head = views.flow_head(bits)
    oh = oracle_mod.OracleHead(oracle, float_head(bits))
    rng = np.random.default_rng(22)
    for s, t in ((0.0, 1.0), (0.25, 0.75), (0.9, 0.1), (0.0, 1.0)):
        condition = rng.standard_normal(512).astype(np.float32)
        state = rng.standard_normal(32).astype(np.float32)
        out = np.zeros(32, np.float32)
        assert lib.phonon_flow_head_forward(ctypes.byref(head), fp(condition), fp(state), s, t,
                                            fp(out)), pkg.last_error(lib)
        ok, ref = oh.forward(condition, state, s, t)
        assert ok and rel(out, ref) < TOL, (s, t, rel(out, ref))
    lib.phonon_flow_head_release(ctypes.byref(head))


def test_lsd_one_step_and_cancel(lib, pkg, oracle, oracle_mod):
    """phonon_flow_lsd_one_step against the oracle; the cancel variant
    returns 0 when its poll fires (here at the 4th of 7 polls) and succeeds
    when it never does; a non-positive temperature or a non-finite noise
    value fails."""
    bits = helpers.random_flow_head_bits(23)
    views = pkg.Views()
    head = views.flow_head(bits)
    oh = oracle_mod.OracleHead(oracle, float_head(bits))
    rng = np.random.default_rng(24)
    condition = rng.standard_normal(512).astype(np.float32)
    raw = rng.standard_normal(32).astype(np.float32)
    out = np.zeros(32, np.float32)
    assert lib.phonon_flow_lsd_one_step(ctypes.byref(head), fp(condition), fp(raw), 0.8, fp(out))
    ok, ref = oh.lsd_one_step(condition, raw, 0.8)
    assert ok and rel(out, ref) < TOL

    CANCEL = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p)
    polls = []

    def poll(_ctx):
        polls.append(1)
        return 1 if len(polls) == 4 else 0

    cancel = CANCEL(poll)
    out2 = np.full(32, 7.0, np.float32)
    assert not lib.phonon_flow_lsd_one_step_cancel(ctypes.byref(head), fp(condition), fp(raw),
                                                   0.8, fp(out2), cancel, None)
    assert np.all(out2 == 7.0)  # nothing published
    never = CANCEL(lambda _ctx: 0)
    assert lib.phonon_flow_lsd_one_step_cancel(ctypes.byref(head), fp(condition), fp(raw), 0.8,
                                               fp(out2), never, None)
    assert np.array_equal(out2, out)
    assert not lib.phonon_flow_lsd_one_step(ctypes.byref(head), fp(condition), fp(raw), 0.0,
                                            fp(out))
    bad = raw.copy()
    bad[5] = np.nan
    assert not lib.phonon_flow_lsd_one_step(ctypes.byref(head), fp(condition), fp(bad), 0.8,
                                            fp(out))
    lib.phonon_flow_head_release(ctypes.byref(head))


@pytest.mark.parametrize("streams,graph", [(1, 1), (5, 1), (16, 0), (17, 1), (64, 1), (64, 0)])
def test_batched_lsd_and_eos_vs_oracle(lib, pkg, oracle, oracle_mod, streams, graph):
    """The device LSD step of B streams with the EOS logit, replayed from a
    graph or launched kernel by kernel, against the oracle per stream; then a
    NaN in one stream's noise is reported by sync, and the same buffers with
    finite noise again give the first results (a graph replayed with new
    input contents)."""
    bits = helpers.random_flow_head_bits(25)
    rng = np.random.default_rng(26)
    eos_w = helpers.bf16_bits(rng.standard_normal(512).astype(np.float32) * 0.05)
    eos_b = helpers.bf16_bits(np.array([0.125], np.float32))
    views = pkg.Views()
    head = views.flow_head(bits)
    ew, eb = views.bf16(eos_w.reshape(1, 512), (1, 512)), views.bf16(eos_b, (1,))
    dev = ctypes.c_void_p()
    assert lib.phonon_flow_head_device_create(ctypes.byref(head), ctypes.byref(ew),
                                              ctypes.byref(eb), 64, ctypes.byref(dev)), \
        pkg.last_error(lib)
    assert lib.phonon_flow_head_device_set_graph(dev, graph)
    stream = lib.phonon_flow_head_device_stream(dev)
    cond = rng.standard_normal((streams, 512)).astype(np.float32)
    raw = rng.standard_normal((streams, 32)).astype(np.float32)
    dc, dr = pkg.DeviceBuffer(lib, cond.nbytes), pkg.DeviceBuffer(lib, raw.nbytes)
    dl, de = pkg.DeviceBuffer(lib, raw.nbytes), pkg.DeviceBuffer(lib, streams * 4)
    dc.upload(cond)
    dr.upload(raw)
    assert lib.phonon_flow_head_device_lsd(dev, streams, dc.ptr, dr.ptr, 0.7, dl.ptr, de.ptr)
    assert lib.phonon_flow_head_device_sync(dev), pkg.last_error(lib)
    lat = np.zeros((streams, 32), np.float32)
    eos = np.zeros(streams, np.float32)
    assert lib.pgpu_copy_d2h(stream, lat.ctypes.data, dl.ptr, lat.nbytes)
    assert lib.pgpu_copy_d2h(stream, eos.ctypes.data, de.ptr, eos.nbytes)
    assert lib.pgpu_stream_sync(stream)
    oh = oracle_mod.OracleHead(oracle, float_head(bits))
    for s in range(streams):
        ok, ref = oh.lsd_one_step(cond[s], raw[s], 0.7)
        assert ok and rel(lat[s], ref) < TOL, (s, rel(lat[s], ref))
        ok, e = oh.eos_logit(helpers.bf16_float(eos_w), helpers.bf16_float(eos_b), cond[s])
        assert ok and abs(eos[s] - e) <= TOL * max(1.0, abs(e)), (s, eos[s], e)
    bad = raw.copy()
    bad[streams // 2, 3] = np.inf
    dr.upload(bad)
    assert lib.phonon_flow_head_device_lsd(dev, streams, dc.ptr, dr.ptr, 0.7, dl.ptr, None)
    assert not lib.phonon_flow_head_device_sync(dev)
    assert lib.phonon_flow_head_device_sync(dev)  # the record was cleared
    dr.upload(raw)
    for _ in range(3):
        assert lib.phonon_flow_head_device_lsd(dev, streams, dc.ptr, dr.ptr, 0.7, dl.ptr, de.ptr)
        assert lib.phonon_flow_head_device_sync(dev)
        again = np.zeros_like(lat)
        again_eos = np.zeros_like(eos)
        assert lib.pgpu_copy_d2h(stream, again.ctypes.data, dl.ptr, again.nbytes)
        assert lib.pgpu_copy_d2h(stream, again_eos.ctypes.data, de.ptr, again_eos.nbytes)
        assert lib.pgpu_stream_sync(stream)
        assert np.array_equal(again, lat) and np.array_equal(again_eos, eos)
    for b in (dc, dr, dl, de):
        b.free()
    lib.phonon_flow_head_device_destroy(dev)


@pytest.mark.parametrize("streams,graph", [(5, 1), (64, 1), (64, 0)])
def test_frame_vs_oracle(lib, pkg, oracle, oracle_mod, streams, graph):
    """One frame after the decode step (phonon_flow_head_device_frame): the
    output norm (LayerNorm eps 1e-5, src/phonon_transformer.c:904-914), the
    LSD step and EOS logit at the normalized state, and the next step's
    input = input_linear . latent + condition (src/phonon_transformer.c:
    860-874), against the oracle's LayerNorm, head and linear per stream."""
    bits = helpers.random_flow_head_bits(31)
    rng = np.random.default_rng(32)
    eos_w = helpers.bf16_bits(rng.standard_normal(512).astype(np.float32) * 0.05)
    eos_b = helpers.bf16_bits(np.array([-0.25], np.float32))
    norm_w = helpers.bf16_bits(1.0 + 0.1 * rng.standard_normal(512).astype(np.float32))
    norm_b = helpers.bf16_bits(0.1 * rng.standard_normal(512).astype(np.float32))
    lin = helpers.bf16_bits(rng.standard_normal((512, 32)).astype(np.float32) * 0.2)
    views = pkg.Views()
    head = views.flow_head(bits)
    ew, eb = views.bf16(eos_w.reshape(1, 512), (1, 512)), views.bf16(eos_b, (1,))
    nw, nb = views.bf16(norm_w, (512,)), views.bf16(norm_b, (512,))
    lv = views.bf16(lin, (512, 32))
    dev = ctypes.c_void_p()
    assert lib.phonon_flow_head_device_create(ctypes.byref(head), ctypes.byref(ew),
                                              ctypes.byref(eb), 64, ctypes.byref(dev))
    assert lib.phonon_flow_head_device_set_frame(dev, ctypes.byref(nw), ctypes.byref(nb),
                                                 ctypes.byref(lv)), pkg.last_error(lib)
    assert not lib.phonon_flow_head_device_set_frame(dev, ctypes.byref(nw), ctypes.byref(nb),
                                                     ctypes.byref(lv))  # once per head
    assert lib.phonon_flow_head_device_set_graph(dev, graph)
    stream = lib.phonon_flow_head_device_stream(dev)
    outputs = (rng.standard_normal((streams, 512)) * 3 + 0.5).astype(np.float32)
    cond = rng.standard_normal((streams, 512)).astype(np.float32)
    raw = rng.standard_normal((streams, 32)).astype(np.float32)
    bufs = [pkg.DeviceBuffer(lib, n) for n in (outputs.nbytes, cond.nbytes, raw.nbytes,
                                               raw.nbytes, streams * 4, cond.nbytes)]
    do, dc, dr, dl, de, dn = bufs
    do.upload(outputs)
    dc.upload(cond)
    dr.upload(raw)
    # Rows are moved 16 bytes at a time: misaligned device rows are rejected.
    assert not lib.phonon_flow_head_device_frame(dev, streams, do.ptr, dc.ptr + 4, dr.ptr, 0.6,
                                                 dl.ptr, de.ptr, dn.ptr)
    assert not lib.phonon_flow_head_device_frame(dev, streams, do.ptr, dc.ptr, dr.ptr, 0.6,
                                                 dl.ptr, de.ptr, dn.ptr + 8)
    for _ in range(2):  # a replayed graph gives the same frame
        assert lib.phonon_flow_head_device_frame(dev, streams, do.ptr, dc.ptr, dr.ptr, 0.6,
                                                 dl.ptr, de.ptr, dn.ptr)
        assert lib.phonon_flow_head_device_sync(dev), pkg.last_error(lib)
        lat = dl.download((streams, 32), stream=stream)
        eos = de.download((streams,), stream=stream)
        nxt = dn.download((streams, 512), stream=stream)
        oh = oracle_mod.OracleHead(oracle, float_head(bits))
        wl = helpers.bf16_float(lin)
        for s in range(streams):
            ok, state = oracle.layer_norm(outputs[s], helpers.bf16_float(norm_w),
                                          helpers.bf16_float(norm_b), 1e-5)
            assert ok
            ok, ref = oh.lsd_one_step(state, raw[s], 0.6)
            assert ok and rel(lat[s], ref) < TOL, (s, rel(lat[s], ref))
            ok, e = oh.eos_logit(helpers.bf16_float(eos_w), helpers.bf16_float(eos_b), state)
            assert ok and abs(eos[s] - e) <= TOL * max(1.0, abs(e)), (s, eos[s], e)
            ok, emb = oracle.linear_batch(wl, lat[s])
            assert ok and rel(nxt[s], emb[0] + cond[s]) < TOL, s
    for b in bufs:
        b.free()
    lib.phonon_flow_head_device_destroy(dev)


def test_head_on_a_callers_stream(lib, pkg):
    """phonon_flow_head_device_set_stream: the LSD step enqueued on a
    caller's stream (graph re-captured there) gives the bits it gives on the
    head's own stream; NULL switches back."""
    bits = helpers.random_flow_head_bits(41)
    rng = np.random.default_rng(42)
    views = pkg.Views()
    head = views.flow_head(bits)
    dev = ctypes.c_void_p()
    assert lib.phonon_flow_head_device_create(ctypes.byref(head), None, None, 16,
                                              ctypes.byref(dev))
    cond = rng.standard_normal((16, 512)).astype(np.float32)
    raw = rng.standard_normal((16, 32)).astype(np.float32)
    dc, dr, dl = (pkg.DeviceBuffer(lib, n) for n in (cond.nbytes, raw.nbytes, raw.nbytes))
    dc.upload(cond)
    dr.upload(raw)
    mine = ctypes.c_void_p()
    assert lib.pgpu_stream_create(ctypes.byref(mine))
    own = lib.phonon_flow_head_device_stream(dev)  # the head's own stream
    assert own and own != mine.value
    outs = []
    for stream in (None, mine.value, None):
        assert lib.phonon_flow_head_device_set_stream(dev, stream)
        # NULL restores the head's own stream.
        assert lib.phonon_flow_head_device_stream(dev) == (stream or own)
        assert lib.phonon_flow_head_device_lsd(dev, 16, dc.ptr, dr.ptr, 0.9, dl.ptr, None)
        assert lib.phonon_flow_head_device_sync(dev)
        outs.append(dl.download((16, 32)))
    if mine.value:
        assert lib.phonon_flow_head_device_stream(dev) != mine.value
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])
    for b in (dc, dr, dl):
        b.free()
    lib.phonon_flow_head_device_destroy(dev)
    lib.pgpu_stream_destroy(mine)


def _head_with_frame(lib, pkg, views, seed, max_streams=64):
    """A device head with the EOS row and the frame's output norm and
    latent embedding, random BF16 weights."""
    rng = np.random.default_rng(seed)
    head = views.flow_head(helpers.random_flow_head_bits(seed))
    ew = views.bf16(helpers.bf16_bits(rng.standard_normal((1, 512)).astype(np.float32) * 0.05),
                    (1, 512))
    eb = views.bf16(helpers.bf16_bits(np.array([0.0625], np.float32)), (1,))
    nw = views.bf16(helpers.bf16_bits(1.0 + 0.1 * rng.standard_normal(512).astype(np.float32)),
                    (512,))
    nb = views.bf16(helpers.bf16_bits(0.1 * rng.standard_normal(512).astype(np.float32)),
                    (512,))
    lv = views.bf16(helpers.bf16_bits(rng.standard_normal((512, 32)).astype(np.float32) * 0.2),
                    (512, 32))
    dev = ctypes.c_void_p()
    assert lib.phonon_flow_head_device_create(ctypes.byref(head), ctypes.byref(ew),
                                              ctypes.byref(eb), max_streams, ctypes.byref(dev))
    assert lib.phonon_flow_head_device_set_frame(dev, ctypes.byref(nw), ctypes.byref(nb),
                                                 ctypes.byref(lv))
    return dev


@pytest.mark.parametrize("streams", [1, 5, 17, 64])
def test_one_launch_head_equals_the_chain(lib, pkg, streams):
    """The three forms of the LSD step (with and without the EOS logit) and
    of the frame give the same bits, from a replayed graph and launched
    directly, each twice in a row:
    - the two-launch-per-block chain (phonon_flow_head_device_set_fused_mlp
      0);
    - the fused chain (set to 1, and the default -1, which fuses at most 2
      streams: one launch per residual block, whose MLP-out product reaches
      the next launch as 8 partials added in the MLP-out projection's
      order);
    - the one dataflow launch (phonon_flow_head_device_set_one_launch 1;
      the counters are reset after each launch), and the same launch with
      tagged hand-offs along the chain (2; each launch has its own tag);
    - the library's defaults (-1, -1): the tagged launch for at most 2
      streams, the chain otherwise."""
    views = pkg.Views()
    dev = _head_with_frame(lib, pkg, views, 51 + streams)
    stream = lib.phonon_flow_head_device_stream(dev)
    rng = np.random.default_rng(52)
    outputs = (rng.standard_normal((streams, 512)) * 2).astype(np.float32)
    cond = rng.standard_normal((streams, 512)).astype(np.float32)
    raw = rng.standard_normal((streams, 32)).astype(np.float32)
    bufs = [pkg.DeviceBuffer(lib, n) for n in (outputs.nbytes, cond.nbytes, raw.nbytes,
                                               raw.nbytes, streams * 4, cond.nbytes)]
    do, dc, dr, dl, de, dn = bufs
    do.upload(outputs)
    dc.upload(cond)
    dr.upload(raw)

    def run(mode):
        got = {}
        for eos in (True, False):
            assert lib.phonon_flow_head_device_lsd(dev, streams, dc.ptr, dr.ptr, 0.8, dl.ptr,
                                                   de.ptr if eos else None)
            assert lib.phonon_flow_head_device_sync(dev), (mode, pkg.last_error(lib))
            got[f"lat{int(eos)}"] = dl.download((streams, 32), stream=stream)
            if eos:
                got["eos"] = de.download((streams,), stream=stream)
        assert lib.phonon_flow_head_device_frame(dev, streams, do.ptr, dc.ptr, dr.ptr, 0.6,
                                                 dl.ptr, de.ptr, dn.ptr)
        assert lib.phonon_flow_head_device_sync(dev), (mode, pkg.last_error(lib))
        got["frame_lat"] = dl.download((streams, 32), stream=stream)
        got["frame_eos"] = de.download((streams,), stream=stream)
        got["next"] = dn.download((streams, 512), stream=stream)
        return got

    assert lib.phonon_flow_head_device_set_one_launch(dev, 0)
    assert not lib.phonon_flow_head_device_set_fused_mlp(dev, 2)  # -1, 0 or 1
    assert not lib.phonon_flow_head_device_set_one_launch(dev, 3)  # -1, 0, 1 or 2
    assert lib.phonon_flow_head_device_set_fused_mlp(dev, 0)
    chain = run("chain")
    for graph in (1, 0):
        assert lib.phonon_flow_head_device_set_graph(dev, graph)
        for fused, one_launch in ((1, 0), (-1, 0), (0, 1), (0, 2), (-1, -1)):
            assert lib.phonon_flow_head_device_set_fused_mlp(dev, fused)
            assert lib.phonon_flow_head_device_set_one_launch(dev, one_launch)
            for rep in range(2):
                mode = f"fused={fused} one launch={one_launch} graph={graph} rep={rep}"
                got = run(mode)
                for k in chain:
                    assert np.array_equal(got[k], chain[k]), (k, mode)
    for b in bufs:
        b.free()
    lib.phonon_flow_head_device_destroy(dev)


@pytest.mark.parametrize("one_launch", [1, 2])
def test_one_launch_head_forced_wait_timeout_recovers(lib, pkg, one_launch):
    """A 1 us wait limit, set from the host, makes the one-launch head's
    waiting tasks give up (counter waits, and with tagged hand-offs the
    polls of the tagged rows): the launch ends, sync reports failure; with
    the limit lifted the same call gives the chain's bits again (the next
    launch's tag differs from the abandoned one's)."""
    streams = 64
    views = pkg.Views()
    dev = _head_with_frame(lib, pkg, views, 61)
    stream = lib.phonon_flow_head_device_stream(dev)
    rng = np.random.default_rng(62)
    cond = rng.standard_normal((streams, 512)).astype(np.float32)
    raw = rng.standard_normal((streams, 32)).astype(np.float32)
    dc, dr, dl, de = (pkg.DeviceBuffer(lib, n) for n in (cond.nbytes, raw.nbytes, raw.nbytes,
                                                          streams * 4))
    dc.upload(cond)
    dr.upload(raw)
    assert lib.phonon_flow_head_device_lsd(dev, streams, dc.ptr, dr.ptr, 0.8, dl.ptr, de.ptr)
    assert lib.phonon_flow_head_device_sync(dev)
    want = dl.download((streams, 32), stream=stream)
    assert lib.phonon_flow_head_device_set_one_launch(dev, one_launch)
    assert lib.phonon_flow_head_device_set_wait_limit(dev, 1)
    assert lib.phonon_flow_head_device_lsd(dev, streams, dc.ptr, dr.ptr, 0.8, dl.ptr, de.ptr)
    assert not lib.phonon_flow_head_device_sync(dev)
    assert lib.phonon_flow_head_device_set_wait_limit(dev, 0)
    assert lib.phonon_flow_head_device_lsd(dev, streams, dc.ptr, dr.ptr, 0.8, dl.ptr, de.ptr)
    assert lib.phonon_flow_head_device_sync(dev), pkg.last_error(lib)
    assert np.array_equal(dl.download((streams, 32), stream=stream), want)
    for b in (dc, dr, dl, de):
        b.free()
    lib.phonon_flow_head_device_destroy(dev)
