"""The KV pool's N(0,1) fill (pgpu_fill_normal): its dispatch plan on the CPU,
and on the GPU a pool of the B=256, 8192-position, 12-layer shape (103 GB,
12.9 G value pairs), whose first and last blocks are checked against the
fill's own formula. A dispatch packet counts work-items in 32 bits, so the
plan must split such a pool into dispatches of at most 2^31 work-items."""
import ctypes

import numpy as np
import pytest

FILL_MAX_GROUPS = 1 << 23            # PGPU_FILL_MAX_GROUPS (phonon_gpu.h)
BLOCK_FLOATS = 8 * 2 * 16 * 64       # heads x (K, V) x positions x head width


def plan(lib, count):
    n = lib.pgpu_fill_normal_plan(count, 0, None, None)
    out = []
    for i in range(n):
        first, pairs = ctypes.c_size_t(), ctypes.c_size_t()
        assert lib.pgpu_fill_normal_plan(count, i, ctypes.byref(first), ctypes.byref(pairs)) == n
        out.append((first.value, pairs.value))
    return out


@pytest.mark.parametrize("count", [2, 512, 514, 2 * 256 * FILL_MAX_GROUPS,
                                   2 * 256 * FILL_MAX_GROUPS + 2, 2 ** 33 + 6,
                                   12 * 131072 * BLOCK_FLOATS, 12 * 67840 * BLOCK_FLOATS])
def test_fill_plan_covers_every_pair_in_dispatches_below_2_31_work_items(pkg, count):
    lib = pkg.load()
    dispatches = plan(lib, count)
    end = 0
    for first, pairs in dispatches:
        assert first == end                        # contiguous, no overlap
        assert 0 < pairs <= 256 * FILL_MAX_GROUPS  # one work-item per pair
        groups = -(-pairs // 256)
        assert groups <= FILL_MAX_GROUPS and groups * 256 < 2 ** 32
        end += pairs
    assert end == count // 2
    # every dispatch but the last is full: the fewest dispatches
    assert all(p == 256 * FILL_MAX_GROUPS for _, p in dispatches[:-1])


def test_fill_plan_of_the_failing_pool(pkg):
    """The 12-layer pool of 256 streams x 512 blocks (8192 positions): one
    dispatch of 12.9 G work-items before; now 6 of 2^31 (12 x 2^30 pairs)."""
    dispatches = plan(pkg.load(), 12 * 131072 * BLOCK_FLOATS)
    assert len(dispatches) == 6


def _mix64(z):
    z = (z + np.uint64(0x9E3779B97F4A7C15))
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def expected_fill(seed, first_float, count):
    """Values [first_float, first_float + count) of the fill (even first,
    even count), restated from k_fill_normal in float32 with numpy."""
    with np.errstate(over="ignore"):
        i = np.arange(first_float // 2, (first_float + count) // 2, dtype=np.uint64)
        r = _mix64(np.uint64(seed) ^ _mix64(i))
    u1 = ((r >> np.uint64(40)).astype(np.uint32) + np.uint32(1)).astype(np.float32) * \
        np.float32(1.0 / 16777217.0)
    u2 = (r & np.uint64(0xFFFFFF)).astype(np.uint32).astype(np.float32) * \
        np.float32(1.0 / 16777216.0)
    rad = np.sqrt(np.float32(-2.0) * np.log(u1))
    ang = np.float32(6.283185307179586) * u2
    out = np.empty(count, np.float32)
    out[0::2] = rad * np.cos(ang)
    out[1::2] = rad * np.sin(ang)
    return out


@pytest.mark.gpu
def test_pool_fill_of_a_103_gb_pool(lib, pkg):
    layers, blocks, seed = 12, 256 * 512, 2027
    print(f"pool fill: {layers} layers x {blocks} blocks", flush=True)
    pool = ctypes.c_void_p()
    assert lib.phonon_kv_pool_create(layers, blocks, ctypes.byref(pool)), pkg.last_error(lib)
    try:
        assert lib.phonon_kv_pool_fill_normal(pool, seed), pkg.last_error(lib)
        i32p = ctypes.POINTER(ctypes.c_int32)
        fp = ctypes.POINTER(ctypes.c_float)
        for block in (0, blocks - 1):
            table = np.array([block], np.int32)
            k = np.zeros((layers, 16, 512), np.float32)
            v = np.zeros((layers, 16, 512), np.float32)
            assert lib.phonon_kv_pool_read(pool, table.ctypes.data_as(i32p), 1, 0, 16,
                                           k.ctypes.data_as(fp), v.ctypes.data_as(fp), 16)
            for layer in (0, layers - 1):
                # pool layout per layer: [block][head][K | V][16 positions][64]
                base = layer * blocks * BLOCK_FLOATS + block * BLOCK_FLOATS
                want = expected_fill(seed, base, BLOCK_FLOATS).reshape(8, 2, 16, 64)
                got_k = k[layer].reshape(16, 8, 64).transpose(1, 0, 2)
                got_v = v[layer].reshape(16, 8, 64).transpose(1, 0, 2)
                assert np.all(np.abs(got_k) > 0) and np.all(np.abs(got_v) > 0)
                np.testing.assert_allclose(got_k, want[:, 0], rtol=0, atol=2e-5)
                np.testing.assert_allclose(got_v, want[:, 1], rtol=0, atol=2e-5)
    finally:
        lib.phonon_kv_pool_destroy(pool)
