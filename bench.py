"""Decode-step throughput of the Flow transformer on one MI355X.

Workload (the headline line): batched decode, B=64 independent streams,
12 layers, d=512, 8x64 heads, FFN 2048, Q8_0 weights (per-row scales),
per-stream contexts c ~ U{1..2048} (keys attended, including the appended
one), paged fp32 KV with block size 16 and shuffled block tables. One "step"
advances every stream by one frame. Inputs and KV are resident in HBM when
the timed region starts; data is synthetic (seeded).

Also reported in the same JSON line: B=1 decode (12 layers, context 256 ->
256+steps), the single Q8 matvec (2048x512, rotating >256 MB of weight
copies), one attention layer vs context length, the roofline of the
dominant kernel (the one-launch step kernel at B=64) timed with HIP events
on its stream, and the CPU baseline (the C restatement of the reference
step, on host cores).

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--batch 64] [--layers 12]
"""
from __future__ import annotations

import argparse
import ctypes
import importlib.util
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(ROOT, "speech-mac_amd")

HBM_PEAK_GBS = 8000.0
KV_BYTES_PER_KEY = 2 * 512 * 4          # K + V fp32 per key per layer
Q8_LAYER_BYTES = (1536 + 512 + 2048) * 512 * 34 // 32 + 512 * 2048 * 34 // 32


def package():
    spec = importlib.util.spec_from_file_location(
        "speech_mac_amd", os.path.join(PKG_DIR, "__init__.py"),
        submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["speech_mac_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


P_I32 = ctypes.POINTER(ctypes.c_int32)
P_F32 = ctypes.POINTER(ctypes.c_float)
P_SZ = ctypes.POINTER(ctypes.c_size_t)


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def last_error(lib):
    """The library's last recorded error (pgpu_last_error), for assert messages."""
    msg = lib.pgpu_last_error()
    return msg.decode(errors="replace") if msg else ""


class Timer:
    def __init__(self, lib, stream):
        self.lib, self.stream = lib, stream
        self.a, self.b = ctypes.c_void_p(), ctypes.c_void_p()
        assert lib.pgpu_event_create(ctypes.byref(self.a)), last_error(lib)
        assert lib.pgpu_event_create(ctypes.byref(self.b)), last_error(lib)

    def start(self):
        assert self.lib.pgpu_event_record(self.a, self.stream), last_error(self.lib)

    def stop_ms(self) -> float:
        assert self.lib.pgpu_event_record(self.b, self.stream), last_error(self.lib)
        ms = ctypes.c_float()
        assert self.lib.pgpu_event_elapsed_ms(self.a, self.b, ctypes.byref(ms)), \
            last_error(self.lib)
        return ms.value


class DecodeSetup:
    """Model + pool + batch with synthetic contexts, ready to step."""

    def __init__(self, pkg, lib, layers, streams, lengths, headroom, seed):
        import speech_mac_amd.synthetic as syn
        self.lib, self.layers, self.streams = lib, layers, streams
        self.lengths = np.asarray(lengths, np.int64)
        self.max_positions = int(self.lengths.max()) + headroom
        assert self.max_positions <= 8192
        self.table_len = (self.max_positions + 15) // 16
        blocks = streams * self.table_len
        views = pkg.Views()
        self.views = views
        weights = views.layers(syn.flow_model(seed, layers))
        self.model, self.pool, self.batch = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
        assert lib.phonon_flow_model_create(weights, layers, ctypes.byref(self.model)), \
            last_error(lib)
        assert lib.phonon_kv_pool_create(layers, blocks, ctypes.byref(self.pool)), last_error(lib)
        assert lib.phonon_kv_pool_fill_normal(self.pool, seed + 1), last_error(lib)
        ids = np.zeros(blocks, np.int32)
        assert lib.phonon_kv_pool_alloc(self.pool, blocks, ids.ctypes.data_as(P_I32)), \
            last_error(lib)
        perm = np.random.default_rng(seed + 2).permutation(ids)   # shuffled tables
        self.tables = np.ascontiguousarray(perm.reshape(streams, self.table_len).astype(np.int32))
        assert lib.phonon_flow_batch_create(self.model, self.pool, streams, self.max_positions,
                                            ctypes.byref(self.batch)), last_error(lib)
        self.stream = lib.phonon_flow_batch_stream(self.batch)
        self.din = lib.phonon_flow_batch_device_inputs(self.batch)
        self.dout = lib.phonon_flow_batch_device_outputs(self.batch)
        x = np.random.default_rng(seed + 3).standard_normal((streams, 512)).astype(np.float32)
        assert lib.pgpu_copy_h2d(self.stream, self.din, x.ctypes.data, x.nbytes), last_error(lib)
        self.reset()

    def reset(self):
        pos = self.lengths.astype(np.uintp)
        assert self.lib.phonon_flow_batch_set_streams(
            self.batch, self.streams, pos.ctypes.data_as(P_SZ), self.tables.ctypes.data_as(P_I32),
            self.table_len), last_error(self.lib)

    def step(self):
        # Output feeds the next step's input: a closed-loop decode.
        assert self.lib.phonon_flow_batch_step_device(self.batch, self.din, 10000.0, self.dout), \
            last_error(self.lib)
        self.din, self.dout = self.dout, self.din

    def positions(self):
        out = np.zeros(self.streams, np.uintp)
        assert self.lib.phonon_flow_batch_positions(self.batch, out.ctypes.data_as(P_SZ)), \
            last_error(self.lib)
        return out.astype(np.int64)

    def close(self):
        self.lib.phonon_flow_batch_destroy(self.batch)
        self.lib.phonon_kv_pool_destroy(self.pool)
        self.lib.phonon_flow_model_destroy(self.model)


def step_bytes(layers, contexts):
    """Algorithmic HBM bytes of one step: Q8 weights once, every attended
    key's K+V once per layer, one appended K+V row per stream per layer."""
    contexts = np.asarray(contexts, np.int64)
    return layers * Q8_LAYER_BYTES + int(layers * np.sum(KV_BYTES_PER_KEY * contexts
                                                         + KV_BYTES_PER_KEY))


# Untimed steps before the warmup. Two things slow the first steps of a run
# (measured on MI355X at B=64): the GPU's clock ramps up over the first
# ~150 ms of load after an idle spell (20-step blocks at 688.6, 688.9, 683.3
# and then 673-674 us for the next 8 s), and a run that starts right after
# another process freed a large allocation (a 103 GB KV pool) steps at
# 688-690 us for ~1.1 s, then at 670-674 us from one block to the next. The
# settle runs rounds of SETTLE_ROUND steps, the positions back at the
# configured contexts after each, until SETTLE_SECONDS have passed, so the
# timed steps measure the settled GPU. A serving loop runs at the settled
# clock.
SETTLE_ROUND = 80
SETTLE_SECONDS = 2.0


def run_decode(pkg, lib, layers, streams, lengths, steps, warmup, seed, groups=None,
               eager=False, settle_s=SETTLE_SECONDS):
    # headroom: a settling round, or the timed steps and then the
    # roofline's timed launches
    d = DecodeSetup(pkg, lib, layers, streams, lengths,
                    max(SETTLE_ROUND, steps + warmup + 41) + 8, seed)
    if groups:
        assert lib.phonon_flow_batch_set_groups(d.batch, groups), last_error(lib)
    if eager:
        assert lib.phonon_flow_batch_set_graph(d.batch, 0), last_error(lib)
    # Settle the clock, then back to the configured contexts: the warmup and
    # timed steps attend exactly the keys they would from a cold start.
    settled = 0
    t_settle = time.perf_counter()
    while settle_s > 0 and time.perf_counter() - t_settle < settle_s:
        for i in range(SETTLE_ROUND):
            d.step()
            if i % 10 == 9:
                assert lib.pgpu_stream_sync(d.stream), last_error(lib)
        settled += SETTLE_ROUND
        assert lib.phonon_flow_batch_sync(d.batch), "non-finite value while settling"
        d.reset()
    for _ in range(warmup):
        d.step()
    assert lib.phonon_flow_batch_sync(d.batch), "non-finite value during warmup"
    first = d.positions()
    timer = Timer(lib, d.stream)
    assert lib.pgpu_stream_sync(d.stream), last_error(lib)
    t0 = time.perf_counter()
    timer.start()
    for _ in range(steps):
        d.step()
    ms = timer.stop_ms()
    assert lib.pgpu_stream_sync(d.stream), last_error(lib)
    wall = time.perf_counter() - t0
    clean = lib.phonon_flow_batch_sync(d.batch)
    # keys attended at step i = position + 1
    total_bytes = sum(step_bytes(layers, first + i + 1) for i in range(steps))
    return d, {"ms": ms, "wall_s": wall, "clean": bool(clean), "bytes": total_bytes,
               "first_positions": first, "settle_steps": settled}


PMC_SUMMARY = "profiles/k_attention_b64_hbm_traffic.md"
FLOW_PMC_SUMMARY = "profiles/k_flow_step_b64_hbm_traffic.md"


def pmc_traffic(summary=PMC_SUMMARY):
    """(traffic, algorithmic) bytes per launch recorded from the rocprofv3
    --pmc passes in `summary`, or None if the summary is absent."""
    try:
        with open(os.path.join(ROOT, summary)) as f:
            fields = dict(line.split(":", 1) for line in f if line.startswith(
                ("traffic_bytes_per_launch:", "algorithmic_bytes_per_launch:")))
        return (int(fields["traffic_bytes_per_launch"]),
                int(fields["algorithmic_bytes_per_launch"]))
    except (OSError, KeyError, ValueError):
        return None


def attention_roofline(pkg, lib, d, iterations=20):
    """Average duration of the split-attention kernel alone on the decode
    workload (the layers of the pool in turn, the streams' current contexts),
    timed with HIP events on the stream it is launched on."""
    pos = d.positions()
    view = pkg.PgpuPagedKv()
    assert lib.phonon_kv_pool_view(d.pool, ctypes.byref(view)), last_error(lib)
    streams = d.streams
    max_splits = (d.max_positions + 255) // 256
    q = pkg.DeviceBuffer(lib, streams * 512 * 4)
    q.upload(np.random.default_rng(5).standard_normal((streams, 512)).astype(np.float32) * 0.125)
    tables = pkg.DeviceBuffer(lib, d.tables.nbytes)
    tables.upload(d.tables)
    positions = pkg.DeviceBuffer(lib, streams * 4)
    positions.upload(pos.astype(np.int32))
    slots = streams * 8 * max_splits
    part = pkg.DeviceBuffer(lib, slots * 66 * 4)
    words = pkg.DeviceBuffer(lib, 4)
    lib.pgpu_memset(d.stream, words.ptr, 0, 4)
    scratch = pkg.PgpuAttentionScratch(part.ptr, part.ptr + slots * 64 * 4, streams, max_splits)
    status = words.ptr

    def launch(layer):
        assert lib.pgpu_attention(d.stream, q.ptr, ctypes.byref(view), layer, tables.ptr,
                                  d.table_len, positions.ptr, streams, 8, max_splits,
                                  ctypes.byref(scratch), status), last_error(lib)

    # Layers in turn, as in a decode step: a launch never finds the previous
    # launch's keys in the last-level cache.
    for i in range(3):
        launch(i % d.layers)
    timer = Timer(lib, d.stream)
    timer.start()
    for i in range(iterations):
        launch((i + 3) % d.layers)
    ms = timer.stop_ms() / iterations
    contexts = pos + 1
    kv_bytes = int(KV_BYTES_PER_KEY * contexts.sum())
    traffic = kv_bytes + streams * 512 * 4 * 2
    achieved = kv_bytes / (ms * 1e-3) / 1e9
    st = np.zeros(1, np.int32)
    lib.pgpu_copy_d2h(d.stream, st.ctypes.data, status, 4)
    for b in (q, tables, positions, part, words):
        b.free()
    measured = pmc_traffic()
    traffic_bytes = None
    if measured:
        # Counter passes are a separate run (bench.py --pmc-program): their
        # traffic/algorithmic ratio applied to this launch's contexts.
        traffic_bytes = int(round(kv_bytes * measured[0] / measured[1]))
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_bytes,
            "traffic_source": f"{PMC_SUMMARY} (FETCH_SIZE/WRITE_SIZE, copy-calibrated): "
                              f"{measured[0]} B for {measured[1]} B algorithmic"
                              if measured else None,
            "kernel": "pgpu::k_attention", "us_per_launch": round(ms * 1e3, 2),
            "algorithmic_bytes_per_launch": kv_bytes, "read_bytes_incl_q_out": traffic,
            "status_clean": int(st[0]) == 0}


def flow_roofline(pkg, lib, d, steps=20):
    """Average duration of the one-launch step kernel (k_flow_step: every
    layer's projections, K/V appends and attention of one decode step) on
    the decode workload, timed with HIP events recorded on the batch's stream
    right before and after each launch (the step is that one launch: its
    work-groups clear the next step's counters themselves). Continues the decode from where the timed run left it. Returns
    None if the batch does not run its step as one launch."""
    events = []
    for _ in range(2 * steps):
        e = ctypes.c_void_p()
        assert lib.pgpu_event_create(ctypes.byref(e)), last_error(lib)
        events.append(e)
    step_bytes_sum = 0
    for i in range(steps):
        step_bytes_sum += step_bytes(d.layers, d.positions() + 1)
        assert lib.phonon_flow_batch_set_timing(d.batch, events[2 * i], events[2 * i + 1]), \
            last_error(lib)
        d.step()
    assert lib.phonon_flow_batch_set_timing(d.batch, None, None), last_error(lib)
    assert lib.pgpu_stream_sync(d.stream), last_error(lib)
    clean = bool(lib.phonon_flow_batch_sync(d.batch))
    total_ms = 0.0
    for i in range(steps):
        ms = ctypes.c_float()
        if not lib.pgpu_event_elapsed_ms(events[2 * i], events[2 * i + 1], ctypes.byref(ms)):
            total_ms = None   # events never recorded: the step ran phase by phase
            break
        total_ms += ms.value
    for e in events:
        lib.pgpu_event_destroy(e)
    if total_ms is None:
        return None
    us = total_ms / steps * 1e3
    per_launch = step_bytes_sum / steps
    achieved = step_bytes_sum / (total_ms * 1e-3) / 1e9
    measured = pmc_traffic(FLOW_PMC_SUMMARY)
    traffic_bytes = None
    if measured:
        # Counter passes are a separate run (bench.py --pmc-program): their
        # traffic/algorithmic ratio applied to this run's contexts.
        traffic_bytes = int(round(per_launch * measured[0] / measured[1]))
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_bytes,
            "traffic_source": f"{FLOW_PMC_SUMMARY} (FETCH_SIZE/WRITE_SIZE, copy-calibrated): "
                              f"{measured[0]} B for {measured[1]} B algorithmic"
                              if measured else None,
            "kernel": "pgpu::k_flow_step<true, 0, false, 1>", "us_per_launch": round(us, 2),
            "launches": steps, "algorithmic_bytes_per_launch": int(per_launch),
            "algorithmic_bytes": "Q8 weights of 12 layers once + K/V of every attended key "
                                 "per layer + the appended K/V row per stream per layer",
            "status_clean": clean}


def calibration_copy(pkg, lib, d, repeats=5):
    """A plain copy of known size for scaling hardware byte counters: all
    layers of positions [0, n) of stream 0 from the pool to contiguous rows
    (pgpu_kv_copy, 16 KiB-aligned 4 KiB tiles). Returns bytes read (= bytes
    written) per launch."""
    view = pkg.PgpuPagedKv()
    assert lib.phonon_kv_pool_view(d.pool, ctypes.byref(view)), last_error(lib)
    n = (d.max_positions // 16) * 16
    row_bytes = 512 * 4
    keys = pkg.DeviceBuffer(lib, d.layers * n * row_bytes)
    values = pkg.DeviceBuffer(lib, d.layers * n * row_bytes)
    tables = pkg.DeviceBuffer(lib, d.tables.nbytes)
    tables.upload(d.tables)
    words = pkg.DeviceBuffer(lib, 4)
    lib.pgpu_memset(d.stream, words.ptr, 0, 4)
    for _ in range(repeats):
        assert lib.pgpu_kv_copy(d.stream, ctypes.byref(view), tables.ptr, 0, n, 0, d.layers,
                                keys.ptr, values.ptr, n, 1, words.ptr), last_error(lib)
    assert lib.pgpu_stream_sync(d.stream), last_error(lib)
    for b in (keys, values, tables, words):
        b.free()
    return 2 * d.layers * n * row_bytes


def pmc_program(pkg, lib, args):
    """Short program for hardware-counter passes: the B=64 decode contexts,
    20 launches of the split-attention kernel alone, 10 decode steps (one
    k_flow_step launch each), then a calibration copy of known size. Prints
    the algorithmic bytes of each."""
    lengths = np.random.default_rng(args.seed).integers(1, 2049, size=args.batch) - 1
    d = DecodeSetup(pkg, lib, args.layers, args.batch, lengths, 64, args.seed)
    roof = attention_roofline(pkg, lib, d)
    for _ in range(3):
        d.step()
    flow = flow_roofline(pkg, lib, d, steps=10)
    copied = calibration_copy(pkg, lib, d)
    d.close()
    print(json.dumps({"k_attention_algorithmic_bytes": roof["algorithmic_bytes_per_launch"],
                      "k_attention_us": roof["us_per_launch"],
                      "k_flow_step_algorithmic_bytes": flow["algorithmic_bytes_per_launch"]
                      if flow else None,
                      "k_flow_step_us": flow["us_per_launch"] if flow else None,
                      "k_kv_copy_bytes_read": copied, "k_kv_copy_bytes_written": copied}),
          flush=True)


def prefill_mfma_work(layers, new_streams, chunk, terms=3, attn16=False):
    """(16-bit MFMA flops, fp32 MFMA flops) of a batched prefill of
    new_streams fresh prompts of `chunk` positions: the projections as issued
    (one MFMA product per multiply-add and split term: 3 bf16 terms in the
    exact mode, 2 fp16 terms in the fast ones) and the causal attention's Q.K
    and P.V (2 flops per multiply-add, every (query, key) pair with key <=
    query, 8 heads x 64 dimensions): in fp32, or with attn16 on the 16-bit
    matrix cores as issued (6 products per Q.K multiply-add, bf16 terms; 3
    per P.V multiply-add, fp16 pairs), counted with the projections."""
    rows = new_streams * chunk
    proj = rows * layers * (1536 + 512 + 2048 + 2048) * 512 * 2 * terms
    pairs = new_streams * chunk * (chunk + 1) // 2
    mac = layers * pairs * 8 * 64 * 2
    if attn16:
        return proj + mac * (6 + 3), 0
    return proj, mac * 2


def prefill_mfma_fraction(layers, new_streams, chunk, ms, terms, attn16=False):
    """The prefill's matrix-core work against the time it took: bf16 / fp16
    flops at 2.5 PFLOP/s plus fp32 flops at 157.3 TFLOP/s (dense peaks), as
    a fraction of the measured time."""
    proj, attn = prefill_mfma_work(layers, new_streams, chunk, terms, attn16)
    secs = ms * 1e-3
    return {"projection_operands": "three bf16 terms" if terms == 3 else "two fp16 terms",
            "attention": ("16-bit matrix cores (bf16 x3 scores, fp16-pair values; counted "
                          "with the projections)" if attn16 else "fp32"),
            "proj_tflop": round(proj / 1e12, 2), "fp32_gflop": round(attn / 1e9, 2),
            "proj_TFLOPs": round(proj / secs / 1e12, 1),
            "frac": round((proj / 2.5e15 + attn / 157.3e12) / secs, 4)}


def large_batch_with_prefill(pkg, lib, seed, layers=12, streams=256, new_streams=16, chunk=256,
                             iterations=4, warmup=1, prefill_attention=0):
    """Large-batch decode with interleaved prefill: every iteration advances
    `streams` streams (contexts U{256..8192-headroom}, paged KV block 16,
    shuffled tables) by one decode step and prefills a `chunk`-position prompt
    for each of `new_streams` newly admitted streams (batched causal prefill:
    all their positions through all layers in one pass)."""
    import speech_mac_amd.synthetic as syn
    rng = np.random.default_rng(seed + 50)
    steps = iterations + warmup
    max_positions = 8192
    lengths = rng.integers(256, max_positions - steps, size=streams) - 1  # positions
    table_len = max_positions // 16
    decode_blocks = int(np.sum((lengths + steps + 16) // 16))
    prefill_blocks = new_streams * (chunk // 16)
    views = pkg.Views()
    weights = views.layers(syn.flow_model(seed, layers))
    model, pool, dec, pre = (ctypes.c_void_p() for _ in range(4))
    assert lib.phonon_flow_model_create(weights, layers, ctypes.byref(model)), last_error(lib)
    assert lib.phonon_kv_pool_create(layers, decode_blocks + prefill_blocks, ctypes.byref(pool)), \
        last_error(lib)
    assert lib.phonon_kv_pool_fill_normal(pool, seed + 51), last_error(lib)
    ids = np.zeros(decode_blocks + prefill_blocks, np.int32)
    assert lib.phonon_kv_pool_alloc(pool, ids.size, ids.ctypes.data_as(P_I32)), last_error(lib)
    ids = np.random.default_rng(seed + 52).permutation(ids).astype(np.int32)
    tables = np.zeros((streams, table_len), np.int32)
    at = 0
    for s_i in range(streams):
        need = int((lengths[s_i] + steps + 16) // 16)
        tables[s_i, :need] = ids[at:at + need]
        at += need
    pre_tables = np.zeros((new_streams, table_len), np.int32)
    pre_tables[:, :chunk // 16] = ids[at:at + prefill_blocks].reshape(new_streams, chunk // 16)
    assert lib.phonon_flow_batch_create(model, pool, streams, max_positions, ctypes.byref(dec)), \
        last_error(lib)
    assert lib.phonon_flow_batch_create(model, pool, new_streams * chunk, max_positions,
                                        ctypes.byref(pre)), last_error(lib)
    assert lib.phonon_flow_batch_set_prefill_exact(pre, prefill_attention), last_error(lib)
    pos = lengths.astype(np.uintp)
    assert lib.phonon_flow_batch_set_streams(dec, streams, pos.ctypes.data_as(P_SZ),
                                             tables.ctypes.data_as(P_I32), table_len), \
                                                 last_error(lib)
    stream = lib.phonon_flow_batch_stream(dec)
    pstream = lib.phonon_flow_batch_stream(pre)
    din, dout = lib.phonon_flow_batch_device_inputs(dec), lib.phonon_flow_batch_device_outputs(dec)
    pin, pout = lib.phonon_flow_batch_device_inputs(pre), lib.phonon_flow_batch_device_outputs(pre)
    x = np.random.default_rng(seed + 53).standard_normal((streams, 512)).astype(np.float32)
    assert lib.pgpu_copy_h2d(stream, din, x.ctypes.data, x.nbytes), last_error(lib)
    px = np.random.default_rng(seed + 54).standard_normal((new_streams * chunk, 512))
    px = px.astype(np.float32)
    assert lib.pgpu_copy_h2d(pstream, pin, px.ctypes.data, px.nbytes), last_error(lib)
    first = np.zeros(new_streams, np.uintp)
    counts = np.full(new_streams, chunk, np.uintp)
    dec_t, pre_t = Timer(lib, stream), Timer(lib, pstream)
    dec_ms = pre_ms = 0.0
    for it in range(steps):
        dec_t.start()
        assert lib.phonon_flow_batch_step_device(dec, din, 10000.0, dout), last_error(lib)
        d_ms = dec_t.stop_ms()
        din, dout = dout, din
        pre_t.start()
        assert lib.phonon_flow_batch_prefill_device(
            pre, new_streams, first.ctypes.data_as(P_SZ), counts.ctypes.data_as(P_SZ),
            pre_tables.ctypes.data_as(P_I32), table_len, pin, 10000.0, pout), last_error(lib)
        p_ms = pre_t.stop_ms()
        if it >= warmup:
            dec_ms += d_ms
            pre_ms += p_ms
    # The prefill set alone: back to back, after three untimed sets (each
    # set above directly follows an 8.9 ms HBM-bound decode step).
    for it in range(13):
        if it == 3:
            pre_t.start()
        assert lib.phonon_flow_batch_prefill_device(
            pre, new_streams, first.ctypes.data_as(P_SZ), counts.ctypes.data_as(P_SZ),
            pre_tables.ctypes.data_as(P_I32), table_len, pin, 10000.0, pout), last_error(lib)
    alone_ms = pre_t.stop_ms() / 10
    clean = bool(lib.phonon_flow_batch_sync(dec)) and bool(lib.phonon_flow_batch_sync(pre))
    lib.phonon_flow_batch_destroy(pre)
    lib.phonon_flow_batch_destroy(dec)
    lib.phonon_kv_pool_destroy(pool)
    lib.phonon_flow_model_destroy(model)
    keys = sum(int(np.sum(lengths + warmup + i + 1)) for i in range(iterations)) / iterations
    dec_bytes = layers * Q8_LAYER_BYTES + layers * KV_BYTES_PER_KEY * (keys + streams)
    per_it_ms = (dec_ms + pre_ms) / iterations
    return {"workload": f"B={streams} decode, contexts U{{256..{max_positions - steps}}}, "
                        f"{layers} layers; plus {new_streams} x {chunk}-position prefills per "
                        f"iteration (batched causal prefill)",
            "iteration_ms": round(per_it_ms, 3),
            "decode_ms": round(dec_ms / iterations, 3),
            "decode_frames_per_s": round(streams / (dec_ms / iterations * 1e-3), 1),
            "decode_GBps": round(dec_bytes / (dec_ms / iterations * 1e-3) / 1e9, 1),
            "decode_frac_of_hbm": round(dec_bytes / (dec_ms / iterations * 1e-3) / 1e9
                                        / HBM_PEAK_GBS, 4),
            "prefill_ms": round(pre_ms / iterations, 3),
            "prefill_alone_ms": round(alone_ms, 3),
            "prefill_tokens_per_s": round(new_streams * chunk / (pre_ms / iterations * 1e-3), 1),
            "prefill_attention": ["matrix cores", "exact (decode arithmetic)",
                                  "lane per query"][prefill_attention],
            # the exact attention keeps three bf16 split terms; the fast
            # modes take two fp16 terms (Q8 weights)
            "prefill_mfma": prefill_mfma_fraction(layers, new_streams, chunk,
                                                  pre_ms / iterations,
                                                  3 if prefill_attention == 1 else 2,
                                                  attn16=prefill_attention == 0),
            "frames_per_s_incl_prefill": round(streams / (per_it_ms * 1e-3), 1),
            "clean": clean}


def task_trace_summary(sched, trace):
    """Per-phase timing of one traced one-launch step (phonon_flow_batch_set_trace:
    start, inputs ready and end of every task on the 100 MHz constant clock),
    averaged over the layers past the first: for each phase, when its first
    task saw its inputs, when its last task ended, the median task body
    (inputs ready -> end) and the gap from the previous phase's last end to
    this phase's first inputs-ready (microseconds)."""
    names = ["QKV", "ATTN", "OUT", "MLP_IN", "MLP_OUT"]
    kind, layer = sched & 7, (sched >> 3) & 63
    tr = trace.astype(np.int64)
    done = (tr[:, 0] > 0) & (tr[:, 2] > 0)
    t0 = tr[done, 0].min()
    ready, end = (tr[:, 1] - t0) / 100.0, (tr[:, 2] - t0) / 100.0
    layers = int(layer[done].max()) + 1
    rows = {n: {"body_us": [], "gap_us": [], "span_us": []} for n in names}
    per_layer = []
    prev_end = None
    for l in range(layers):
        for k, n in enumerate(names):
            m = done & (layer == l) & (kind == k)
            if not m.any():
                continue
            r0, e1 = float(ready[m].min()), float(end[m].max())
            if l > 0:
                rows[n]["body_us"].append(float(np.median(end[m] - ready[m])))
                rows[n]["span_us"].append(e1 - r0)
                if prev_end is not None:
                    rows[n]["gap_us"].append(r0 - prev_end)
            prev_end = e1
        per_layer.append(prev_end)
    out = {n: {key: round(float(np.mean(v)), 2) for key, v in d.items() if v}
           for n, d in rows.items()}
    out["us_per_layer"] = round((per_layer[-1] - per_layer[0]) / (layers - 1), 2)
    out["step_span_us"] = round(float(end[done].max()), 1)
    return out


def b1_with_prefill(pkg, lib, layers, seed, prompt=256, frames=750, warmup=10, mode=None,
                    trace_steps=0, handoff=None):
    """B=1: one stream, `layers` layers. A `prompt`-position prefill (the
    batched causal prefill, positions 0..prompt-1 through every layer in one
    pass), then `frames` decode steps, each step's output fed back as the
    next input. Run once untimed (prefill + `warmup` steps), then again from
    position 0: prefill and decode timed separately with HIP events. `mode`:
    the step's pipeline mode (None: the library's default); `handoff`: the
    one-launch step's hand-off mode (None: the library's default)."""
    import speech_mac_amd.synthetic as syn
    max_pos = prompt + frames + 16
    table_len = (max_pos + 15) // 16
    blocks = table_len + 3
    views = pkg.Views()
    weights = views.layers(syn.flow_model(seed, layers))
    model, pool, batch = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
    assert lib.phonon_flow_model_create(weights, layers, ctypes.byref(model)), last_error(lib)
    assert lib.phonon_kv_pool_create(layers, blocks, ctypes.byref(pool)), last_error(lib)
    ids = np.zeros(blocks, np.int32)
    assert lib.phonon_kv_pool_alloc(pool, blocks, ids.ctypes.data_as(P_I32)), last_error(lib)
    table = np.ascontiguousarray(np.random.default_rng(seed + 60).permutation(ids)[:table_len])
    assert lib.phonon_flow_batch_create(model, pool, prompt, max_pos, ctypes.byref(batch)), \
        last_error(lib)
    if mode is not None:
        assert lib.phonon_flow_batch_set_pipeline(batch, mode), last_error(lib)
    if handoff is not None:
        assert lib.phonon_flow_batch_set_handoff(batch, handoff), last_error(lib)
    stream = lib.phonon_flow_batch_stream(batch)
    rng = np.random.default_rng(seed + 61)
    pin = pkg.DeviceBuffer(lib, prompt * 512 * 4)
    pout = pkg.DeviceBuffer(lib, prompt * 512 * 4)
    pin.upload(rng.standard_normal((prompt, 512)).astype(np.float32))
    x0 = rng.standard_normal(512).astype(np.float32)
    din, dout = lib.phonon_flow_batch_device_inputs(batch), lib.phonon_flow_batch_device_outputs(
        batch)
    first = np.zeros(1, np.uintp)
    counts = np.full(1, prompt, np.uintp)
    timer = Timer(lib, stream)

    def run(steps):
        nonlocal din, dout
        assert lib.pgpu_copy_h2d(stream, din, x0.ctypes.data, x0.nbytes), last_error(lib)
        timer.start()
        assert lib.phonon_flow_batch_prefill_device(
            batch, 1, first.ctypes.data_as(P_SZ), counts.ctypes.data_as(P_SZ),
            table.ctypes.data_as(P_I32), table_len, pin.ptr, 10000.0, pout.ptr), last_error(lib)
        pre_ms = timer.stop_ms()
        pos = np.array([prompt], np.uintp)
        assert lib.phonon_flow_batch_set_streams(batch, 1, pos.ctypes.data_as(P_SZ),
                                                 table.ctypes.data_as(P_I32), table_len), \
                                                     last_error(lib)
        timer.start()
        for _ in range(steps):
            assert lib.phonon_flow_batch_step_device(batch, din, 10000.0, dout), last_error(lib)
            din, dout = dout, din
        dec_ms = timer.stop_ms()
        return pre_ms, dec_ms

    run(warmup)
    clean = bool(lib.phonon_flow_batch_sync(batch))
    pre_ms, dec_ms = run(frames)
    clean = clean and bool(lib.phonon_flow_batch_sync(batch))
    traced = None
    if trace_steps:
        # One more traced step at the end of the run (context prompt + frames).
        ntask = lib.phonon_flow_batch_schedule(batch, None, 0)
        sched = np.zeros(ntask, np.uint32)
        lib.phonon_flow_batch_schedule(batch, sched.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
                                       ntask)
        buf = pkg.DeviceBuffer(lib, ntask * 4 * 8)
        assert lib.phonon_flow_batch_set_trace(batch, buf.ptr, ntask), last_error(lib)
        summaries = []
        for _ in range(trace_steps):
            assert lib.phonon_flow_batch_step_device(batch, din, 10000.0, dout), last_error(lib)
            din, dout = dout, din
            assert lib.pgpu_stream_sync(stream), last_error(lib)
            tr = np.zeros((ntask, 4), np.uint64)
            assert lib.pgpu_copy_d2h(stream, tr.ctypes.data, buf.ptr, tr.nbytes), last_error(lib)
            assert lib.pgpu_stream_sync(stream), last_error(lib)
            summaries.append(task_trace_summary(sched, tr))
        assert lib.phonon_flow_batch_set_trace(batch, None, 0), last_error(lib)
        buf.free()
        traced = {"context": prompt + frames + 1, "tasks": int(ntask), "steps": summaries}
        clean = clean and bool(lib.phonon_flow_batch_sync(batch))
    pin.free()
    pout.free()
    lib.phonon_flow_batch_destroy(batch)
    lib.phonon_kv_pool_destroy(pool)
    lib.phonon_flow_model_destroy(model)
    total_bytes = sum(step_bytes(layers, [prompt + i + 1]) for i in range(frames))
    return {"frames_per_s": round(frames / (dec_ms * 1e-3), 1),
            "us_per_step": round(dec_ms * 1e3 / frames, 2),
            "effective_GBps": round(total_bytes / (dec_ms * 1e-3) / 1e9, 1),
            "prefill_ms": round(pre_ms, 3),
            "prefill_tokens_per_s": round(prompt / (pre_ms * 1e-3), 1),
            "workload": f"B=1, {layers} layers: a {prompt}-position prompt through the batched "
                        f"prefill, then {frames} decode frames (contexts {prompt + 1}.."
                        f"{prompt + frames}), each output fed back as the next input; "
                        + ("the library's default step mode" if mode is None
                           else f"step pipeline mode {mode}")
                        + ("" if handoff is None else f", hand-off mode {handoff}"),
            "clean": clean, **({"task_trace": traced} if traced else {})}


def q8_matvec_bench(pkg, lib, seed=1, calls=2000):
    """Config: single Q8 matvec 2048x512; 300 rotating weight copies (>256 MB)."""
    import speech_mac_amd.synthetic as syn
    rng = np.random.default_rng(seed)
    w = syn.q8_matrix(rng, 2048, 512)
    x = rng.standard_normal(512).astype(np.float32)
    copies = 300
    h = ctypes.c_void_p()
    assert lib.phonon_q8_device_create(w.ctypes.data, 2048, 512, copies, ctypes.byref(h)), \
        last_error(lib)
    stream = ctypes.c_void_p()
    assert lib.pgpu_stream_create(ctypes.byref(stream)), last_error(lib)
    dx = pkg.DeviceBuffer(lib, 512 * 4)
    dx.upload(x)
    dy = pkg.DeviceBuffer(lib, 2048 * 4)
    for i in range(20):
        assert lib.phonon_q8_device_matvec(h, i % copies, dx.ptr, dy.ptr, 1, stream), \
            last_error(lib)
    timer = Timer(lib, stream)
    res = {}
    for label, rotate in (("rotating_300_copies", True), ("same_copy_cache_resident", False)):
        timer.start()
        for i in range(calls):
            assert lib.phonon_q8_device_matvec(h, i % copies if rotate else 0, dx.ptr, dy.ptr, 1,
                                               stream), last_error(lib)
        ms = timer.stop_ms() / calls
        nbytes = lib.phonon_q8_device_bytes_per_call(h, 1)
        res[label] = {"us_per_call": round(ms * 1e3, 3),
                      "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1)}
    assert lib.phonon_q8_device_status(h, stream), last_error(lib)
    res["bytes_per_call"] = int(lib.phonon_q8_device_bytes_per_call(h, 1))
    res["launches_per_call"] = 1  # 512 columns: the projection splits the fp32 rows itself
    dx.free()
    dy.free()
    lib.phonon_q8_device_destroy(h)
    lib.pgpu_stream_destroy(stream)
    return res


def gemv_valu_vs_mfma(pkg, lib, seed=3, calls=400, copies=300):
    """Small-batch Q8 products, vector units (phonon_q8_device_matvec_valu:
    pgpu_q8_gemv, the reference's arithmetic, one lane per 32-column block)
    against the matrix cores (phonon_q8_device_matvec: the projection task,
    exact split MFMA), for batch 1, 2, 4, 8 at the two projection shapes of
    the decode step; each call reads one of `copies` weight copies in turn
    (more bytes than the 256 MB Infinity Cache holds). Kernel time from HIP
    events over `calls` back-to-back calls on one stream."""
    import speech_mac_amd.synthetic as syn
    stream = ctypes.c_void_p()
    assert lib.pgpu_stream_create(ctypes.byref(stream)), last_error(lib)
    timer = Timer(lib, stream)
    out = {}
    for rows, cols in ((2048, 512), (512, 2048)):
        rng = np.random.default_rng(seed + rows)
        w = syn.q8_matrix(rng, rows, cols)
        h = ctypes.c_void_p()
        assert lib.phonon_q8_device_create(w.ctypes.data, rows, cols, copies, ctypes.byref(h)), \
            last_error(lib)
        x = rng.standard_normal((8, cols)).astype(np.float32)
        dx = pkg.DeviceBuffer(lib, x.nbytes)
        dx.upload(x)
        dy = pkg.DeviceBuffer(lib, 8 * rows * 4)
        shape = {}
        for batch in (1, 2, 4, 8):
            row = {}
            for name, fn in (("valu", lib.phonon_q8_device_matvec_valu),
                             ("mfma", lib.phonon_q8_device_matvec)):
                for i in range(20):
                    assert fn(h, i % copies, dx.ptr, dy.ptr, batch, stream)
                timer.start()
                for i in range(calls):
                    fn(h, i % copies, dx.ptr, dy.ptr, batch, stream)
                ms = timer.stop_ms() / calls
                nbytes = lib.phonon_q8_device_bytes_per_call(h, batch)
                row[name] = {"us_per_call": round(ms * 1e3, 2),
                             "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1)}
            shape[f"batch_{batch}"] = row
        assert lib.phonon_q8_device_status(h, stream), last_error(lib)
        out[f"{rows}x{cols}"] = shape
        dx.free()
        dy.free()
        lib.phonon_q8_device_destroy(h)
    lib.pgpu_stream_destroy(stream)
    out["note"] = ("kernel time per call from HIP events (back-to-back calls, rotating "
                   f"{copies} weight copies); valu = vector-unit GEMV with the reference's "
                   "rounding order (bit-exact), mfma = the exact-split projection task")
    return out


def flow_head_bench(pkg, lib, streams=64, calls=200, seed=11, graph=-1, one_launch=-1,
                    fused=-1):
    """The flow head's batched LSD step (phonon_flow_head_device_lsd: noise
    scaling, input/condition projections, seven adaLN projections as one, six
    residual MLP blocks, final layer, EOS logit) for `streams` streams, on a
    random BF16 head of the reference's shapes; and the reference-signature
    phonon_flow_lsd_one_step (one stream, host buffers, synchronous)."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import helpers
    bits = helpers.random_flow_head_bits(seed)
    rng = np.random.default_rng(seed + 1)
    eos_w = helpers.bf16_bits(rng.standard_normal(512).astype(np.float32) * 0.05)
    eos_b = helpers.bf16_bits(np.array([0.1], np.float32))
    views = pkg.Views()
    head = views.flow_head(bits)
    ew, eb = views.bf16(eos_w.reshape(1, 512), (1, 512)), views.bf16(eos_b, (1,))
    dev = ctypes.c_void_p()
    assert lib.phonon_flow_head_device_create(ctypes.byref(head), ctypes.byref(ew),
                                              ctypes.byref(eb), streams, ctypes.byref(dev)), \
                                                  last_error(lib)
    assert lib.phonon_flow_head_device_set_graph(dev, graph), last_error(lib)
    assert lib.phonon_flow_head_device_set_one_launch(dev, one_launch), last_error(lib)
    assert lib.phonon_flow_head_device_set_fused_mlp(dev, fused), last_error(lib)
    stream = lib.phonon_flow_head_device_stream(dev)
    cond = pkg.DeviceBuffer(lib, streams * 512 * 4)
    raw = pkg.DeviceBuffer(lib, streams * 32 * 4)
    lat = pkg.DeviceBuffer(lib, streams * 32 * 4)
    eos = pkg.DeviceBuffer(lib, streams * 4)
    cond.upload(rng.standard_normal((streams, 512)).astype(np.float32))
    raw.upload(rng.standard_normal((streams, 32)).astype(np.float32))
    for _ in range(5):
        assert lib.phonon_flow_head_device_lsd(dev, streams, cond.ptr, raw.ptr, 0.7, lat.ptr,
                                               eos.ptr), last_error(lib)
    assert lib.phonon_flow_head_device_sync(dev), last_error(lib)
    timer = Timer(lib, stream)
    timer.start()
    for _ in range(calls):
        lib.phonon_flow_head_device_lsd(dev, streams, cond.ptr, raw.ptr, 0.7, lat.ptr, eos.ptr)
    ms = timer.stop_ms() / calls
    clean = bool(lib.phonon_flow_head_device_sync(dev))
    weight_bytes = 2 * (512 * 32 + 512 * 512 + 10240 * 512 + 12 * 512 * 512 + 32 * 512 + 512)
    c1 = np.random.default_rng(seed + 2).standard_normal(512).astype(np.float32)
    n1 = np.random.default_rng(seed + 3).standard_normal(32).astype(np.float32)
    o1 = np.zeros(32, np.float32)
    fpp = lambda a: a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))  # noqa: E731
    assert lib.phonon_flow_lsd_one_step(ctypes.byref(head), fpp(c1), fpp(n1), 0.7, fpp(o1)), \
        last_error(lib)
    t0 = time.perf_counter()
    reps = 100
    for _ in range(reps):
        lib.phonon_flow_lsd_one_step(ctypes.byref(head), fpp(c1), fpp(n1), 0.7, fpp(o1))
    single_us = (time.perf_counter() - t0) / reps * 1e6
    lib.phonon_flow_head_release(ctypes.byref(head))
    for b in (cond, raw, lat, eos):
        b.free()
    lib.phonon_flow_head_device_destroy(dev)
    # The library's defaults (-1): steps of at most 2 streams run as one
    # launch with tagged hand-offs, larger ones as the chain (whose blocks
    # the fused mode -1 would fuse at most 2 streams).
    mode = one_launch if one_launch >= 0 else (2 if streams <= 2 else 0)
    fused_chain = not mode and (fused == 1 or (fused == -1 and streams <= 2))
    return {"workload": f"flow head LSD step + EOS logit, B={streams} streams, BF16 head of the "
                        f"reference's shapes (6 adaLN blocks, 8.68 M weights per step)",
            "us_per_step": round(ms * 1e3, 2),
            "frames_per_s": round(streams / (ms * 1e-3), 1),
            "launches_per_step": 2 if mode else 9 if fused_chain else 15,
            "one_launch": bool(mode),
            "tagged_handoffs": mode == 2,
            "fused_mlp": fused_chain,
            "weight_bytes_per_step": weight_bytes,
            "weight_GBps": round(weight_bytes / (ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(weight_bytes / (ms * 1e-3) / 8e12, 4),
            "single_stream_api_us": round(single_us, 1),
            "single_stream_api": "phonon_flow_lsd_one_step: host buffers in and out, "
                                 "synchronous",
            "clean": clean}


def frame_loop_bench(pkg, lib, layers=12, streams=64, frames=30, warmup=3, seed=2026,
                     shared_stream=True, graph=-1, one_launch=-1, fused=-1):
    """The whole per-frame loop of B streams on the GPU: the decode step
    (library default mode), then phonon_flow_head_device_frame (output norm,
    LSD step + EOS logit, latent embedding + condition) writing the next
    step's inputs; the head runs on the batch's stream (shared_stream) or on
    its own, handed over through events. Random BF16 head, out_norm and
    input_linear of the reference's shapes."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import helpers
    rng = np.random.default_rng(seed + 5)
    lengths = np.random.default_rng(seed).integers(1, 2049, size=streams) - 1
    d = DecodeSetup(pkg, lib, layers, streams, lengths, frames + warmup + 8, seed)
    views = pkg.Views()
    head = views.flow_head(helpers.random_flow_head_bits(seed + 6))
    eos_w = helpers.bf16_bits(rng.standard_normal(512).astype(np.float32) * 0.05)
    ew, eb = views.bf16(eos_w.reshape(1, 512), (1, 512)), views.bf16(
        helpers.bf16_bits(np.array([0.0], np.float32)), (1,))
    nw = views.bf16(helpers.bf16_bits(np.ones(512, np.float32)), (512,))
    nb = views.bf16(helpers.bf16_bits(np.zeros(512, np.float32)), (512,))
    lv = views.bf16(helpers.bf16_bits(rng.standard_normal((512, 32)).astype(np.float32) * 0.1),
                    (512, 32))
    h = ctypes.c_void_p()
    assert lib.phonon_flow_head_device_create(ctypes.byref(head), ctypes.byref(ew),
                                              ctypes.byref(eb), streams, ctypes.byref(h)), \
                                                  last_error(lib)
    assert lib.phonon_flow_head_device_set_frame(h, ctypes.byref(nw), ctypes.byref(nb),
                                                 ctypes.byref(lv)), last_error(lib)
    if shared_stream:
        assert lib.phonon_flow_head_device_set_stream(h, d.stream), last_error(lib)
    assert lib.phonon_flow_head_device_set_graph(h, graph), last_error(lib)
    assert lib.phonon_flow_head_device_set_one_launch(h, one_launch), last_error(lib)
    assert lib.phonon_flow_head_device_set_fused_mlp(h, fused), last_error(lib)
    hs = lib.phonon_flow_head_device_stream(h)
    cond = pkg.DeviceBuffer(lib, streams * 512 * 4)
    raw = pkg.DeviceBuffer(lib, streams * 32 * 4)
    lat = pkg.DeviceBuffer(lib, streams * 32 * 4)
    eos = pkg.DeviceBuffer(lib, streams * 4)
    cond.upload(rng.standard_normal((streams, 512)).astype(np.float32))
    raw.upload(rng.standard_normal((streams, 32)).astype(np.float32))
    decoded, framed = ctypes.c_void_p(), ctypes.c_void_p()
    assert lib.pgpu_event_create(ctypes.byref(decoded)), last_error(lib)
    assert lib.pgpu_event_create(ctypes.byref(framed)), last_error(lib)
    din, dout = d.din, d.dout

    def frame():
        assert lib.phonon_flow_batch_step_device(d.batch, din, 10000.0, dout), last_error(lib)
        if not shared_stream:
            assert lib.pgpu_event_record(decoded, d.stream), last_error(lib)
            assert lib.pgpu_stream_wait_event(hs, decoded), last_error(lib)
        assert lib.phonon_flow_head_device_frame(h, streams, dout, cond.ptr, raw.ptr, 0.7, lat.ptr,
                                                 eos.ptr, din), last_error(lib)
        if not shared_stream:
            assert lib.pgpu_event_record(framed, hs), last_error(lib)
            assert lib.pgpu_stream_wait_event(d.stream, framed), last_error(lib)

    for _ in range(warmup):
        frame()
    assert lib.pgpu_stream_sync(d.stream), last_error(lib)
    timer = Timer(lib, d.stream)
    timer.start()
    for _ in range(frames):
        frame()
    ms = timer.stop_ms() / frames
    clean = bool(lib.phonon_flow_batch_sync(d.batch)) and bool(
        lib.phonon_flow_head_device_sync(h))
    for b in (cond, raw, lat, eos):
        b.free()
    lib.pgpu_event_destroy(decoded)
    lib.pgpu_event_destroy(framed)
    lib.phonon_flow_head_device_destroy(h)
    d.close()
    return {"workload": f"closed per-frame loop, B={streams}: {layers}-layer decode step + "
                        f"output norm + flow head LSD step + EOS + latent embedding into the "
                        f"next step's input, contexts U{{1..2048}}",
            "head_stream": "the batch's" if shared_stream else "its own, events between",
            # -1: the library's default (a graph for the chain of launches)
            "head_graph": graph == 1 or (graph == -1 and not (one_launch > 0 or
                                                             (one_launch == -1 and streams <= 2))),
            "head_one_launch": one_launch > 0 or (one_launch == -1 and streams <= 2),
            "head_tagged": one_launch == 2 or (one_launch == -1 and streams <= 2),
            "head_fused_mlp": one_launch == 0 and (fused == 1 or (fused == -1 and streams <= 2)),
            "us_per_frame": round(ms * 1e3, 1), "frames_per_s": round(streams / (ms * 1e-3), 1),
            "clean": clean}


def pcm_flops_per_frame():
    """Algorithmic flops (2 per multiply-add) of one latent frame through
    Mimi (16 rows, 2 layers, full 250-key window) and the SEANet decoder."""
    mimi_rows = 16 * 2 * 2 * (1536 * 512 + 512 * 512 + 2048 * 512 + 512 * 2048)
    mimi_attention = 16 * 2 * 2 * 2 * 250 * 512
    mimi_input = 2 * 512 * 32 + 16 * 512 * 2 * 2
    seanet = 16 * 2 * 512 * 512 * 7
    positions, ch = 16, 512
    for s in (6, 5, 4):
        seanet += positions * 2 * ch * (ch // 2) * 2 * s      # transposed conv, 2s taps
        positions *= s
        ch //= 2
        seanet += positions * 2 * (ch * (ch // 2) * 3 + (ch // 2) * ch)  # residual k3 + k1
    seanet += positions * 2 * 64 * 3
    return mimi_rows + mimi_attention + mimi_input + seanet


def pcm_bench(pkg, lib, seed=31, frames=256, stream_frames=40):
    """Latent frames -> 24 kHz PCM through phonon_pcm_process (Mimi and the
    SEANet decoder on the GPU), random weights of the real shapes: one
    request of `frames` frames, then frame-by-frame calls (streaming). Host
    buffers go in and out inside each call, as the drop-in's contract has
    it; the call returns when the samples are in host memory."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import helpers
    views = pkg.Views()
    mimi, model = helpers.pcm_model(lib, pkg, views, helpers.random_mimi(seed),
                                    helpers.random_pcm_convs(seed + 1))
    h = ctypes.c_void_p()
    assert lib.phonon_pcm_state_create(model, ctypes.byref(h)), last_error(lib)
    x = np.random.default_rng(seed + 2).standard_normal((frames, 32)).astype(np.float32)
    raw = np.zeros(frames * 1920, np.float32)
    fpp = lambda a: a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))  # noqa: E731
    assert lib.phonon_pcm_process(h, fpp(x), 32, fpp(raw), raw.size, None, 0), last_error(lib)
    lib.phonon_pcm_state_reset(h)
    t0 = time.perf_counter()
    assert lib.phonon_pcm_process(h, fpp(x), frames, fpp(raw), raw.size, None, 0), last_error(lib)
    bulk = time.perf_counter() - t0
    lib.phonon_pcm_state_reset(h)
    one = np.zeros(1920, np.float32)
    per = []
    for f in range(stream_frames):
        xf = np.ascontiguousarray(x[f:f + 1])
        t0 = time.perf_counter()
        assert lib.phonon_pcm_process(h, fpp(xf), 1, fpp(one), one.size, None, 0), last_error(lib)
        per.append(time.perf_counter() - t0)
    lib.phonon_pcm_state_destroy(h)
    lib.phonon_pcm_model_destroy(model)
    flops = pcm_flops_per_frame()
    audio_s = frames / 12.5
    return {"workload": f"latent -> PCM decoding (Mimi 2 layers + SEANet, 1920 samples per "
                        f"frame), random BF16 weights of the real shapes; one request of "
                        f"{frames} frames ({audio_s:.1f} s of audio), then {stream_frames} "
                        f"one-frame calls",
            "bulk_ms": round(bulk * 1e3, 2),
            "bulk_frames_per_s": round(frames / bulk, 1),
            "bulk_realtime_factor": round(audio_s / bulk, 1),
            "stream_ms_per_frame_median": round(float(np.median(per)) * 1e3, 3),
            "stream_ms_per_frame_p90": round(float(np.percentile(per, 90)) * 1e3, 3),
            "flops_per_frame": flops,
            "bulk_TFLOPs": round(flops * frames / bulk / 1e12, 2),
            "note": "wall clock around the synchronous host-buffer call (PCIe copies "
                    "included); the real-time budget is 80 ms of audio per frame"}


def cpu_pcm(seed=31, budget_s=10.0):
    """The oracle's latent -> PCM chain (Mimi and SEANet restated in C from
    the reference's sequential code) on one thread, 2-frame calls."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_py
    import helpers
    oracle = oracle_py.Oracle()
    om = oracle_py.MimiOracle(oracle, helpers.random_mimi(seed))
    oc = [oracle_py.ConvOracle(oracle, w, b, s, t)
          for (w, b, s, t) in helpers.random_pcm_convs(seed + 1)]
    x = np.random.default_rng(seed + 2).standard_normal((4096, 32)).astype(np.float32)
    frames, elapsed = 0, 0.0
    while elapsed < budget_s:
        t0 = time.perf_counter()
        ok, _ = oracle_py.pcm_process(oracle, om, oc, x[frames:frames + 2])
        elapsed += time.perf_counter() - t0
        assert ok
        frames += 2
    for c in oc:
        c.close()
    om.close()
    return {"value": round(frames / elapsed, 2), "unit": "frames/s", "cores": 1, "kind": "port",
            "realtime_factor": round(frames / 12.5 / elapsed, 2),
            "sample": f"{frames} latent frames through the oracle's Mimi + SEANet chain in "
                      f"2-frame calls, {elapsed:.1f} s"}


def attention_curve(pkg, lib, seed=9):
    """One attention layer decode (H=8, dh=64): append + attention per step,
    vs context length, as one 1-layer batched step of one stream."""
    out = {}
    reps = 20
    for c in (1, 2, 16, 128, 511, 512, 513, 1024, 2048):
        d = DecodeSetup(pkg, lib, 1, 1, [c - 1], reps + 8, seed)
        for _ in range(3):
            d.step()
        d.reset()
        timer = Timer(lib, d.stream)
        timer.start()
        for _ in range(reps):
            d.step()
        ms = timer.stop_ms() / reps
        d.close()
        out[str(c)] = round(ms * 1e3, 2)
    return {"us_per_layer_step_vs_context": out,
            "note": f"one stream, one layer (LN, QKV+RoPE+append, attention, out, MLP) in "
                    f"the library's default step mode; contexts c .. c+{reps - 1}"}


def cpu_flow_head(seed=11, budget_s=2.0):
    """The oracle's LSD step of the flow head (the reference's per-frame CPU
    head restated in C), one stream per call on one thread."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_py
    import helpers
    bits = helpers.random_flow_head_bits(seed)
    oh = oracle_py.OracleHead(oracle_py.Oracle(), {k: helpers.bf16_float(v)
                                                   for k, v in bits.items()})
    rng = np.random.default_rng(seed + 2)
    cond = rng.standard_normal(512).astype(np.float32)
    raw = rng.standard_normal(32).astype(np.float32)
    frames, elapsed = 0, 0.0
    while elapsed < budget_s:
        t0 = time.perf_counter()
        ok, _ = oh.lsd_one_step(cond, raw, 0.7)
        elapsed += time.perf_counter() - t0
        assert ok
        frames += 1
    return {"value": round(frames / elapsed, 1), "unit": "frames/s", "cores": 1, "kind": "port",
            "sample": f"{frames} LSD steps of one stream (flow head forward at (0, 1), "
                      f"{elapsed:.1f} s)"}


def cpu_host():
    """What the CPU baselines ran on: nproc, the CPUs this process may use,
    the CPU model and whether SMT is on, read from /proc/cpuinfo and sysfs
    (no child process)."""
    info = {"nproc": os.cpu_count(), "usable_cpus": len(os.sched_getaffinity(0))}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                key, _, value = line.partition(":")
                if key.strip() == "model name":
                    info["model"] = value.strip()
                    break
    except OSError:
        pass
    try:
        with open("/sys/devices/system/cpu/cpu0/topology/thread_siblings_list") as f:
            # a cpulist ("0,64", "0-1"): the logical CPUs sharing cpu0's core
            count = 0
            for part in f.read().strip().split(","):
                first, _, last = part.partition("-")
                count += int(last or first) - int(first) + 1
            info["threads_per_core"] = count
    except (OSError, ValueError):
        pass
    try:
        with open("/sys/devices/system/cpu/smt/active") as f:
            info["smt_active"] = f.read().strip() == "1"
    except OSError:
        pass
    return info


def cpu_threads():
    """Host threads for the batched CPU leg: every CPU this process may use,
    at most 16 (the GPU box's CPU share for one GPU)."""
    return max(1, min(16, len(os.sched_getaffinity(0))))


def cpu_q8_matvec(seed=1, budget_s=2.0):
    """The single Q8 matvec (2048x512) on one core: the reference's own
    phonon_q8.c, compiled from its source into oracle/_ref when that build
    exists (kind "reference"), else the oracle's restatement, bit-identical
    to it (kind "port")."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle_py
    import speech_mac_amd.synthetic as syn
    rng = np.random.default_rng(seed)
    w = syn.q8_matrix(rng, 2048, 512)
    x = rng.standard_normal(512).astype(np.float32)
    if oracle_py.ReferenceQ8.available():
        impl, kind = oracle_py.ReferenceQ8(), "reference"
    else:
        impl, kind = oracle_py.Oracle(), "port"
    calls, elapsed = 0, 0.0
    while elapsed < budget_s:
        t0 = time.perf_counter()
        for _ in range(50):
            ok, _ = impl.q8_matvec(w, x, 2048, 512)
        elapsed += time.perf_counter() - t0
        assert ok
        calls += 50
    us = elapsed / calls * 1e6
    return {"value": round(us, 2), "unit": "us/call", "cores": 1, "kind": kind,
            "GBps": round(1124352 / (us * 1e-6) / 1e9, 2),
            "sample": f"{calls} calls of phonon_q8_matvec 2048x512 (same weights every call), "
                      f"{elapsed:.1f} s"}


def cpu_b1_stack(layers, seed, budget_s=4.0):
    """B=1 decode on one core: the oracle's 12-layer stack step at the B=1
    workload's positions (256 .. 1005 after the 256-position prefill)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_py
    import helpers
    import speech_mac_amd.synthetic as syn
    oracle = oracle_py.Oracle()
    om = oracle_py.OracleModel(oracle, helpers.oracle_layers(oracle, syn.flow_model(seed, layers)))
    cap = 1006
    tile = np.random.default_rng(seed).standard_normal(1 << 16).astype(np.float32)
    keys = np.resize(tile, layers * cap * 512).reshape(layers, cap, 512)
    vals = np.resize(tile[::-1].copy(), layers * cap * 512).reshape(layers, cap, 512)
    x = np.random.default_rng(seed + 1).standard_normal(512).astype(np.float32)
    positions = np.random.default_rng(seed + 2).integers(256, cap, size=10000)
    steps, elapsed = 0, 0.0
    while elapsed < budget_s:
        t0 = time.perf_counter()
        ok, _ = om.stack_step(keys, vals, cap, int(positions[steps]), x)
        elapsed += time.perf_counter() - t0
        assert ok
        steps += 1
    return {"value": round(steps / elapsed, 2), "unit": "frames/s", "cores": 1, "kind": "port",
            "us_per_step": round(elapsed / steps * 1e6, 1),
            "sample": f"{steps} single-stream {layers}-layer decode steps (the oracle's stack "
                      f"step) at positions drawn from 256..1005, {elapsed:.1f} s"}


def cpu_baseline(pkg, lib, layers, lengths, seed, budget_s=10.0):
    """The C restatement of the reference step (oracle) for all B streams of
    the headline workload, one pthread per stream of a group: streams run
    in groups of `threads`, one decode step each, at their own contexts;
    reported in frames/s over the whole batch."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_py
    import helpers
    import speech_mac_amd.synthetic as syn
    oracle = oracle_py.Oracle()
    om = oracle_py.OracleModel(oracle, helpers.oracle_layers(oracle, syn.flow_model(seed, layers)))
    threads = cpu_threads()
    lengths = np.asarray(lengths, np.int64)
    groups = [lengths[i:i + threads] for i in range(0, len(lengths), threads)]
    # Every repetition is the same decode step (append at each stream's
    # position, attend position+1 keys), so the cache needs one free slot.
    cap = int(lengths.max()) + 1
    tile = np.random.default_rng(seed).standard_normal(1 << 16).astype(np.float32)
    total = threads * layers * cap * 512
    keys = np.resize(tile, total).reshape(threads, layers, cap, 512)
    vals = np.resize(tile[::-1].copy(), total).reshape(threads, layers, cap, 512)
    x = np.random.default_rng(seed + 1).standard_normal((threads, 512)).astype(np.float32)
    reps, frames, elapsed = 0, 0, 0.0
    while elapsed < budget_s:
        for g in groups:
            n = len(g)
            t0 = time.perf_counter()
            ok, _ = om.stack_step_streams(keys[:n], vals[:n], cap, g, x[:n], n)
            elapsed += time.perf_counter() - t0
            assert ok
            frames += n
        reps += 1
    return {"value": round(frames / elapsed, 2), "unit": "frames/s", "cores": threads,
            "kind": "port", "host": cpu_host(),
            "sample": f"all {len(lengths)} streams of the headline workload (contexts "
                      f"U{{1..2048}}), {reps} repetitions of one {layers}-layer decode step each "
                      f"(the oracle's stack step), {threads} pthreads (one per stream of a group "
                      f"of {threads}), {elapsed:.1f} s"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--layers", type=int, default=12)
    ap.add_argument("--seed", type=int, default=2026)
    ap.add_argument("--groups", type=int, default=0,
                    help="concurrent stream groups of the step (0 = library default)")
    ap.add_argument("--eager", action="store_true",
                    help="launch the step's kernels directly instead of a graph replay")
    ap.add_argument("--skip-extras", action="store_true",
                    help="only the headline B=64 line (no B=1, matvec, curve, CPU)")
    ap.add_argument("--large-batch", action="store_true",
                    help="run only the B=256 decode + batched prefill workload")
    ap.add_argument("--flow-head", action="store_true",
                    help="run only the flow head LSD step measurement")
    ap.add_argument("--gemv", action="store_true",
                    help="run only the small-batch Q8 GEMV comparison (vector units vs MFMA)")
    ap.add_argument("--pcm", action="store_true",
                    help="run only the latent -> PCM decoding measurement")
    ap.add_argument("--pmc-program", action="store_true",
                    help="run only the attention kernel and a calibration copy, for "
                         "rocprofv3 --pmc passes")
    ap.add_argument("--b1-trace", action="store_true",
                    help="run only the B=1 prefill + decode workload, then trace three "
                         "one-launch steps task by task and print each phase's timing")
    ap.add_argument("--b1-handoff", type=int, default=None,
                    help="the one-launch hand-off mode of the --b1-trace run (default: the "
                         "library's)")
    ap.add_argument("--b1-handoffs", type=str, default="",
                    help="run only the B=1 prefill + decode workload, once per listed "
                         "one-launch hand-off mode (comma-separated, e.g. 3,4)")
    ap.add_argument("--b1-modes", type=str, default="",
                    help="run only the B=1 prefill + decode workload, once per listed step "
                         "pipeline mode (comma-separated, e.g. 0,2)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU: streams are independent and "
                          "would shard across GPUs with no collectives; --gpus must be 1"}))
        sys.exit(2)
    pkg = package()
    lib = pkg.load()
    if lib.pgpu_device_init() != 1:
        raise SystemExit("no gfx950 device: " + pkg.last_error(lib))
    name = ctypes.create_string_buffer(256)
    lib.pgpu_device_name(name, 256)
    log(f"device: {name.value.decode()}")
    if args.pmc_program:
        pmc_program(pkg, lib, args)
        return
    if args.large_batch:
        for kind in (0, 2):
            print(json.dumps(large_batch_with_prefill(pkg, lib, args.seed,
                                                      prefill_attention=kind)), flush=True)
        return
    if args.b1_trace:
        print(json.dumps(b1_with_prefill(pkg, lib, args.layers, args.seed, trace_steps=3,
                                         handoff=args.b1_handoff)), flush=True)
        return
    if args.b1_handoffs:
        for rep_i in range(2):
            for h in (int(m) for m in args.b1_handoffs.split(",")):
                print(json.dumps(dict(b1_with_prefill(pkg, lib, args.layers, args.seed,
                                                      handoff=h), handoff=h, repeat=rep_i)),
                      flush=True)
        return
    if args.b1_modes:
        for mode in (int(m) for m in args.b1_modes.split(",")):
            print(json.dumps(dict(b1_with_prefill(pkg, lib, args.layers, args.seed, mode=mode),
                                  mode=mode)), flush=True)
        return
    if args.pcm:
        print(json.dumps(pcm_bench(pkg, lib)), flush=True)
        return
    if args.gemv:
        print(json.dumps(gemv_valu_vs_mfma(pkg, lib)), flush=True)
        return
    if args.flow_head:
        # (one launch, fused chain): the dataflow launch with tagged and with
        # counted hand-offs, the fused chain, the two-launch-per-block chain.
        modes = ((2, 0), (1, 0), (0, 1), (0, 0))
        for one, fused in modes:
            for graph in (1, 0):
                print(json.dumps(frame_loop_bench(pkg, lib, shared_stream=True, graph=graph,
                                                  one_launch=one, fused=fused)), flush=True)
        for streams in (64, 16, 1):
            for one, fused in modes:
                for graph in (1, 0):
                    r = flow_head_bench(pkg, lib, streams=streams, graph=graph, one_launch=one,
                                        fused=fused)
                    print(json.dumps(dict(r, graph=graph)), flush=True)
        return

    lengths = np.random.default_rng(args.seed).integers(1, 2049, size=args.batch) - 1
    log(f"B={args.batch} L={args.layers}: contexts {lengths.min() + 1}..{lengths.max() + 1}")
    d, r = run_decode(pkg, lib, args.layers, args.batch, lengths, args.steps, args.warmup,
                      args.seed, args.groups, args.eager)
    ms_step = r["ms"] / args.steps
    value = args.batch * args.steps / (r["ms"] * 1e-3)
    gbs = r["bytes"] / (r["ms"] * 1e-3) / 1e9
    log(f"B={args.batch}: {ms_step * 1e3:.1f} us/step, {value:.0f} frames/s, {gbs:.0f} GB/s "
        f"({gbs / HBM_PEAK_GBS:.1%} of HBM), clean={r['clean']}")
    # The dominant kernel: the one-launch step kernel where the batch runs
    # its step as one launch (B=64), else the split-attention kernel.
    roof = flow_roofline(pkg, lib, d) or attention_roofline(pkg, lib, d)
    log(f"{roof['kernel']}: {roof['us_per_launch']} us/launch, {roof['achieved']} GB/s")
    d.close()

    line = {
        "metric": "decode frames/sec at B=64 (12L d512 Q8); achieved HBM GB/s vs peak",
        "value": round(value, 1), "unit": "frames/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "settle_steps": r["settle_steps"],
        "ms_per_step": round(ms_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp32",
        "data": "synthetic (seeded Q8 weights, N(0,1) KV contexts)",
        "config": {"workload": f"batched decode B={args.batch}, {args.layers} layers d512 "
                               "8x64 FFN2048, Q8_0 per-row scales, contexts U{1..2048}, paged fp32 "
                               "KV block 16, shuffled tables",
                   "global_batch": args.batch, "seq_len": 2048, "parallelism": "none (1 GPU)"},
        "hbm": {"algorithmic_bytes_per_step": int(r["bytes"] / args.steps),
                "achieved_GBps": round(gbs, 1), "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4),
                "all_steps_finite": r["clean"]},
        "roofline": roof,
    }
    if not args.skip_extras:
        line["b1"] = b1_with_prefill(pkg, lib, args.layers, args.seed)
        log(f"B=1: {line['b1']}")
        line["b256_with_prefill"] = large_batch_with_prefill(pkg, lib, args.seed)
        log(f"B=256 + prefill: {line['b256_with_prefill']}")
        line["q8_matvec_2048x512"] = q8_matvec_bench(pkg, lib)
        log(f"q8 matvec: {line['q8_matvec_2048x512']}")
        line["q8_gemv_valu_vs_mfma"] = gemv_valu_vs_mfma(pkg, lib)
        log(f"q8 gemv valu vs mfma: {line['q8_gemv_valu_vs_mfma']}")
        line["flow_head"] = {"b64": flow_head_bench(pkg, lib, streams=64),
                             "b1": flow_head_bench(pkg, lib, streams=1),
                             "frame_loop_b64": frame_loop_bench(pkg, lib)}
        log(f"flow head: {line['flow_head']}")
        line["pcm_decode"] = pcm_bench(pkg, lib)
        log(f"pcm decode: {line['pcm_decode']}")
        line["attention_layer_curve"] = attention_curve(pkg, lib)
        log(f"attention curve: {line['attention_layer_curve']}")
        line["cpu_baseline"] = cpu_baseline(pkg, lib, args.layers, lengths, args.seed)
        line["cpu_baseline"]["b1_one_core"] = cpu_b1_stack(args.layers, args.seed)
        line["cpu_baseline"]["q8_matvec_one_core"] = cpu_q8_matvec()
        line["cpu_baseline"]["flow_head"] = cpu_flow_head()
        line["cpu_baseline"]["pcm_decode"] = cpu_pcm()
        log(f"cpu baseline: {line['cpu_baseline']}")
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
