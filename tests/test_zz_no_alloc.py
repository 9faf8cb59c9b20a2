"""pgpu_attention_static, the entry point that allocates nothing: the split
partials live in the library's fixed device array instead of a caller's
pgpu_attention_scratch. Its output must equal, bit for bit, pgpu_attention
followed by pgpu_attention_merge on the same inputs (the same kernels), on
two calls in a row (the second smaller, over the partials the first left
behind); sizes past the array's limit are rejected before any launch. The
call can be captured into a HIP graph in global capture mode (where any
allocation call during the capture fails it) and replayed."""
import ctypes

import numpy as np
import pytest

import helpers

pytestmark = pytest.mark.gpu
SLOTS = 16384  # PGPU_ATTENTION_STATIC_SLOTS


def i32p(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))


def fp(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


class Case:
    """A pool with random K/V, shuffled tables and ragged positions; q, the
    outputs and a caller-owned pgpu_attention_scratch in device memory."""

    def __init__(self, pkg, lib, layers, streams, positions, seed):
        self.lib, self.streams = lib, streams
        rng = np.random.default_rng(seed)
        self.positions = np.asarray(positions, np.int32)
        max_pos = int(self.positions.max()) + 1
        self.table_len = (max_pos + 15) // 16
        self.max_splits = (max_pos + 255) // 256
        blocks = streams * self.table_len
        self.pool = ctypes.c_void_p()
        assert lib.phonon_kv_pool_create(layers, blocks, ctypes.byref(self.pool))
        ids = np.zeros(blocks, np.int32)
        assert lib.phonon_kv_pool_alloc(self.pool, blocks, i32p(ids))
        self.tables = np.ascontiguousarray(rng.permutation(ids).reshape(streams, self.table_len))
        keys = rng.standard_normal((layers, max_pos, 512)).astype(np.float32)
        vals = rng.standard_normal((layers, max_pos, 512)).astype(np.float32)
        for s in range(streams):
            assert lib.phonon_kv_pool_write(self.pool, i32p(self.tables[s]), self.table_len, 0,
                                            int(self.positions[s]) + 1, fp(keys), fp(vals),
                                            max_pos)
        self.kv = pkg.PgpuPagedKv()
        assert lib.phonon_kv_pool_view(self.pool, ctypes.byref(self.kv))
        self.q = pkg.DeviceBuffer(lib, streams * 512 * 4)
        self.q.upload((rng.standard_normal((streams, 512)) * 0.125).astype(np.float32))
        self.dtab = pkg.DeviceBuffer(lib, self.tables.nbytes)
        self.dtab.upload(self.tables)
        self.dpos = pkg.DeviceBuffer(lib, self.positions.nbytes)
        self.dpos.upload(self.positions)
        self.status = pkg.DeviceBuffer(lib, 4)
        self.status.upload(np.zeros(1, np.int32))
        slots = streams * 8 * self.max_splits
        self.acc = pkg.DeviceBuffer(lib, slots * 64 * 4)
        self.ml = pkg.DeviceBuffer(lib, slots * 2 * 4)
        self.work = pkg.PgpuAttentionScratch(self.acc.ptr, self.ml.ptr, streams, self.max_splits)
        self.out = [pkg.DeviceBuffer(lib, streams * 512 * 4) for _ in range(2)]

    def existing(self, layer):
        """pgpu_attention + pgpu_attention_merge with the caller's scratch."""
        lib = self.lib
        assert lib.pgpu_attention(None, self.q.ptr, ctypes.byref(self.kv), layer, self.dtab.ptr,
                                  self.table_len, self.dpos.ptr, self.streams, 8,
                                  self.max_splits, ctypes.byref(self.work), self.status.ptr)
        assert lib.pgpu_attention_merge(None, ctypes.byref(self.work), self.dpos.ptr,
                                        self.streams, 8, self.max_splits, self.out[0].ptr, None,
                                        self.status.ptr)
        assert lib.pgpu_stream_sync(None)
        return self.out[0].download((self.streams, 512))

    def enqueue_static(self, layer, max_splits=None, stream=None, table_len=None):
        return self.lib.pgpu_attention_static(
            stream, self.q.ptr, ctypes.byref(self.kv), layer, self.dtab.ptr,
            self.table_len if table_len is None else table_len, self.dpos.ptr, self.streams, 8,
            max_splits or self.max_splits, self.out[1].ptr, None, self.status.ptr)

    def static(self, layer, max_splits=None):
        if not self.enqueue_static(layer, max_splits):
            return None
        assert self.lib.pgpu_stream_sync(None)
        return self.out[1].download((self.streams, 512))

    def clean(self):
        return int(self.status.download((1,), np.int32)[0]) == 0

    def close(self):
        for b in [self.q, self.dtab, self.dpos, self.status, self.acc, self.ml] + self.out:
            b.free()
        self.lib.phonon_kv_pool_destroy(self.pool)


def test_static_attention_equals_the_scratch_path(lib, pkg):
    # First call: 40 streams, contexts up to 2048 keys (8 splits); second:
    # 7 streams, up to 600 keys (3 splits), over what the first left behind.
    rng = np.random.default_rng(901)
    first = Case(pkg, lib, 2, 40, rng.integers(0, 2048, size=40), 902)
    second = Case(pkg, lib, 3, 7, rng.integers(0, 600, size=7), 903)
    try:
        for case, layer in ((first, 1), (second, 2)):
            got = case.static(layer)
            assert got is not None, pkg.last_error(lib)
            want = case.existing(layer)
            assert np.isfinite(want).all() and case.clean()
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        # The first case again, after the second: the same bits.
        got = first.static(1)
        assert np.array_equal(got.view(np.uint32), first.existing(1).view(np.uint32))
        # Past the limit: rejected on the host, with the reason.
        assert first.static(1, max_splits=SLOTS // (8 * 40) + 1) is None
        assert b"partial slots" in lib.pgpu_last_error()
    finally:
        first.close()
        second.close()


def test_static_attention_replays_from_a_graph_captured_in_global_mode(lib, pkg):
    """One pgpu_attention_static call captured on a stream in global capture
    mode: had the call allocated (hipMalloc and the like), the capture would
    fail. The graph, replayed three times over a NaN-filled output with the
    scratch path run eagerly in between, gives its bits every time. A table
    stride below 1 is rejected."""
    rng = np.random.default_rng(911)
    case = Case(pkg, lib, 2, 24, rng.integers(0, 1500, size=24), 912)
    stream, exec_ = ctypes.c_void_p(), ctypes.c_void_p()
    assert lib.pgpu_stream_create(ctypes.byref(stream))
    try:
        assert not case.enqueue_static(1, table_len=0)
        assert b"invalid arguments" in lib.pgpu_last_error()
        want = case.existing(1)
        assert lib.pgpu_graph_begin_global(stream), pkg.last_error(lib)
        enqueued = case.enqueue_static(1, stream=stream)
        ended = lib.pgpu_graph_end(stream, ctypes.byref(exec_))
        assert enqueued and ended, pkg.last_error(lib)
        nan = np.full((case.streams, 512), np.nan, np.float32)
        for replay in range(3):
            case.out[1].upload(nan)
            assert lib.pgpu_graph_launch(exec_, stream), pkg.last_error(lib)
            assert lib.pgpu_stream_sync(stream)
            got = case.out[1].download((case.streams, 512))
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), replay
            assert np.array_equal(case.existing(1).view(np.uint32), want.view(np.uint32))
        assert case.clean()
    finally:
        lib.pgpu_graph_destroy(exec_)
        lib.pgpu_stream_destroy(stream)
        case.close()
