"""CPU checks of the one-launch step's task list (pgpu_flow_schedule).

The launch cannot deadlock if every task is listed after every task it
waits for (work-groups are dispatched in list order, so the lowest unfinished
task always has its inputs done). These tests decode the descriptors the
library builds and replay the waits of pgpu_flow.hip against the list order.
"""
import ctypes

import numpy as np
import pytest

QKV, ATTN, OUT, MLP_IN, MLP_OUT = range(5)
TASKS = {QKV: 24, OUT: 8, MLP_IN: 32, MLP_OUT: 32}
FUSED_OUT_TASKS = 8          # PGPU_FLOW_FUSED_OUT_TASKS
PREFILL, FUSED = 1, 2        # pgpu_flow_schedule flags


PLACEMENTS = [None, (0.024, (4.0, 10.0, 16.0, 22.0)), (0.001, (0.0, 0.0, 0.0, 0.0)),
              (1.0, (50.0, 20.0, 900.0, 1e6)), (0.05, (1e9, 1e9, 1e9, 1e9))]


def build(lib, splits, layers, place=None, prefill=0):
    splits = np.ascontiguousarray(splits, dtype=np.uintp)
    szp = splits.ctypes.data_as(ctypes.POINTER(ctypes.c_size_t))
    pp = None
    if place is not None:
        import speech_mac_amd as pkg
        pl = pkg.PgpuFlowPlacement(place[0], (ctypes.c_float * 4)(*place[1]))
        pp = ctypes.byref(pl)
    n = lib.pgpu_flow_schedule(len(splits), layers, szp, pp, prefill, None, 0)
    out = np.zeros(n, np.uint32)
    got = lib.pgpu_flow_schedule(len(splits), layers, szp, pp, prefill,
                                 out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), n)
    assert got == n
    return out


def decode(d):
    d = d.astype(np.int64)
    return d & 7, (d >> 3) & 63, (d >> 9) & 255, d >> 17


def check_order(sched, splits, layers, prefill=False, fused=False):
    """Replays the step: each task must find its waits satisfied by the tasks
    listed before it. Raises AssertionError at the first violation. fused:
    the fused MLP's list (no MLP_OUT phase; a layer's QKV tasks sum the
    previous layer's MLP_IN partials and read its r; the last layer's 8
    MLP_OUT tasks write the output from them)."""
    streams = len(splits)
    tiles = (streams + 15) // 16
    kind, layer, tile, index = decode(sched)
    done = np.zeros((layers, tiles, 5), np.int64)
    qkv_head = np.zeros((layers, tiles, 8), np.int64)  # QKV tasks done per head (q, k, v)
    merged = np.zeros((layers, streams, 8), np.int64)   # ATTN tasks seen per (s, head)
    seen = set()
    for i in range(len(sched)):
        k, l, t, x = int(kind[i]), int(layer[i]), int(tile[i]), int(index[i])
        key = (k, l, t, x)
        assert key not in seen, f"task {key} listed twice"
        seen.add(key)
        assert l < layers and t < tiles
        live = min(16, streams - 16 * t)
        if k == QKV:
            assert x < TASKS[QKV]
            if l > 0 and fused:
                assert done[l - 1, t, MLP_IN] == TASKS[MLP_IN], f"QKV({l},{t}) before MLP_IN"
                assert done[l - 1, t, OUT] == TASKS[OUT], f"QKV({l},{t}) before OUT"
            elif l > 0:
                assert done[l - 1, t, MLP_OUT] == TASKS[MLP_OUT], f"QKV({l},{t}) before MLP_OUT"
            qkv_head[l, t, x % 8] += 1   # rows [64x, 64x + 64): q, k or v of head x % 8
        elif k == ATTN:
            h, j, n = x & 7, (x >> 3) & 255, x >> 11
            assert n < live and j < splits[16 * t + n]
            # decode: the head's q, k and v tasks of its tile (pgpu_flow.hip
            # waits on PGPU_FLOW_QKV_HEAD + h); prefill: every QKV task of
            # every tile (PGPU_FLOW_QKV_ALL)
            if prefill:
                for t2 in range(tiles):
                    assert done[l, t2, QKV] == TASKS[QKV], f"ATTN({l},{t}) before QKV({l},{t2})"
            else:
                assert qkv_head[l, t, h] == 3, f"ATTN({l},{t},head {h}) before its QKV tasks"
            merged[l, 16 * t + n, h] += 1
            if merged[l, 16 * t + n, h] == splits[16 * t + n]:
                done[l, t, ATTN] += 1   # the (stream, head) is merged
        elif k == OUT:
            assert x < TASKS[OUT]
            assert done[l, t, ATTN] == 8 * live, f"OUT({l},{t}) before its attention"
        elif k == MLP_IN:
            assert x < TASKS[MLP_IN]
            assert done[l, t, OUT] == TASKS[OUT], f"MLP_IN({l},{t}) before OUT"
        elif k == MLP_OUT:
            assert x < (FUSED_OUT_TASKS if fused else TASKS[MLP_OUT])
            assert not fused or l == layers - 1, f"fused MLP_OUT({l},{t}) before the last layer"
            assert done[l, t, MLP_IN] == TASKS[MLP_IN], f"MLP_OUT({l},{t}) before MLP_IN"
        else:
            raise AssertionError(f"bad kind {k}")
        if k != ATTN:
            done[l, t, k] += 1
    # every task of the step is listed
    for l in range(layers):
        for t in range(tiles):
            live = min(16, streams - 16 * t)
            for k, n in TASKS.items():
                if fused and k == MLP_OUT:
                    n = FUSED_OUT_TASKS if l == layers - 1 else 0
                assert done[l, t, k] == n, (l, t, k)
            assert done[l, t, ATTN] == 8 * live
    return True


@pytest.mark.parametrize("streams,layers", [(1, 1), (1, 12), (5, 3), (16, 2), (17, 4),
                                            (40, 12), (64, 12), (256, 2)])
@pytest.mark.parametrize("place", range(len(PLACEMENTS)))
def test_schedule_lists_every_task_after_its_inputs(pkg, streams, layers, place):
    lib = pkg.load()
    rng = np.random.default_rng(streams * 100 + layers)
    splits = rng.integers(1, 33, size=streams)
    chain = sum(TASKS.values())
    count = layers * ((streams + 15) // 16) * chain + layers * 8 * int(splits.sum())
    sched = build(lib, splits, layers, PLACEMENTS[place])
    assert len(sched) == count
    assert check_order(sched, splits, layers)
    pre = build(lib, splits, layers, PLACEMENTS[place], prefill=1)
    assert len(pre) == count
    assert check_order(pre, splits, layers, prefill=True)


def test_schedule_puts_each_chain_behind_its_own_attention(pkg):
    """Tile t's OUT tasks follow its last ATTN task directly, ahead of tile
    t+1's attention (the overlap the order exists for)."""
    lib = pkg.load()
    splits = np.full(48, 3)
    sched = build(lib, splits, 2)
    kind, layer, tile, _ = decode(sched)
    for l in range(2):
        for t in range(3):
            attn = np.flatnonzero((kind == ATTN) & (layer == l) & (tile == t))
            outs = np.flatnonzero((kind == OUT) & (layer == l) & (tile == t))
            assert outs[0] == attn[-1] + 1
            if t < 2:
                nxt = np.flatnonzero((kind == ATTN) & (layer == l) & (tile == t + 1))
                assert nxt[0] > outs[-1]


def test_order_checker_rejects_planted_mistakes(pkg):
    """The replay is not vacuous: moving one task ahead of an input, dropping
    a task, or listing one twice each fail it."""
    lib = pkg.load()
    splits = np.array([2, 1, 3, 1, 2] * 4)
    sched = build(lib, splits, 2)
    kind, layer, tile, _ = decode(sched)
    cases = []
    # an OUT task moved in front of the last ATTN of its tile
    o = int(np.flatnonzero((kind == OUT) & (layer == 1) & (tile == 0))[0])
    a = int(np.flatnonzero((kind == ATTN) & (layer == 1) & (tile == 0))[-1])
    bad = sched.copy()
    bad[a], bad[o] = sched[o], sched[a]
    cases.append(bad)
    # a QKV of layer 1 moved in front of the last MLP_OUT of layer 0
    q = int(np.flatnonzero((kind == QKV) & (layer == 1) & (tile == 1))[0])
    m = int(np.flatnonzero((kind == MLP_OUT) & (layer == 0) & (tile == 1))[-1])
    bad = sched.copy()
    bad[m], bad[q] = sched[q], sched[m]
    cases.append(bad)
    cases.append(np.delete(sched, len(sched) // 2))          # a task missing
    cases.append(np.insert(sched, 10, sched[3]))             # a task twice
    # the first ATTN task of (layer 1, tile 0) moved in front of the v task
    # of its own head
    kind, layer, tile, index = decode(sched)
    a = int(np.flatnonzero((kind == ATTN) & (layer == 1) & (tile == 0))[0])
    h = int(index[a]) & 7
    v = int(np.flatnonzero((kind == QKV) & (layer == 1) & (tile == 0) & (index == 16 + h))[0])
    bad = np.insert(np.delete(sched, a), v, sched[a])
    cases.append(bad)
    for bad in cases:
        with pytest.raises(AssertionError):
            check_order(bad, splits, 2)


def test_order_checker_allows_attention_after_its_own_head(pkg):
    """The per-head rule is what the kernel waits for: an ATTN task of head
    h may run before another head's QKV tasks of its tile (the checker
    accepts it), but not before its own head's (rejected above)."""
    lib = pkg.load()
    splits = np.array([1] * 16)
    sched = build(lib, splits, 1)
    kind, layer, tile, index = decode(sched)
    qkv = np.flatnonzero(kind == QKV)
    assert list(index[qkv]) == [(i % 3) * 8 + i // 3 for i in range(24)]  # head by head
    a = int(np.flatnonzero((kind == ATTN) & ((index & 7) == 0))[0])
    # move it right behind head 0's three QKV tasks, ahead of heads 1..7
    moved = np.insert(np.delete(sched, a), int(qkv[2]) + 1, sched[a])
    assert check_order(moved, splits, 1)


@pytest.mark.parametrize("streams,layers", [(1, 1), (1, 12), (3, 5), (4, 12)])
@pytest.mark.parametrize("place", range(len(PLACEMENTS)))
def test_fused_mlp_schedule_lists_every_task_after_its_inputs(pkg, streams, layers, place):
    """The fused MLP's list (PGPU_FLOW_SCHEDULE_FUSED_MLP): no MLP_OUT phase
    but the last layer's output tasks, every task after its inputs; with the
    prefill flag as well the fused flag is ignored."""
    lib = pkg.load()
    rng = np.random.default_rng(streams * 10 + layers)
    splits = rng.integers(1, 33, size=streams)
    count = layers * (24 + 8 + 32) + FUSED_OUT_TASKS + layers * 8 * int(splits.sum())
    sched = build(lib, splits, layers, PLACEMENTS[place], prefill=FUSED)
    assert len(sched) == count
    assert check_order(sched, splits, layers, fused=True)
    # the fused list fails the unfused replay (its QKV tasks follow no MLP_OUT)
    if layers > 1:
        with pytest.raises(AssertionError):
            check_order(sched, splits, layers)
    pre = build(lib, splits, layers, PLACEMENTS[place], prefill=PREFILL | FUSED)
    assert np.array_equal(pre, build(lib, splits, layers, PLACEMENTS[place], prefill=PREFILL))
    assert check_order(pre, splits, layers, prefill=True)


def test_fused_order_checker_rejects_planted_mistakes(pkg):
    """A QKV task of layer 1 moved in front of the last MLP_IN task of layer
    0, or an output task in front of the last layer's last MLP_IN task,
    fails the fused replay."""
    lib = pkg.load()
    splits = np.array([3, 1, 2])
    sched = build(lib, splits, 2, prefill=FUSED)
    kind, layer, _, _ = decode(sched)
    cases = []
    q = int(np.flatnonzero((kind == QKV) & (layer == 1))[0])
    m = int(np.flatnonzero((kind == MLP_IN) & (layer == 0))[-1])
    bad = sched.copy()
    bad[m], bad[q] = sched[q], sched[m]
    cases.append(bad)
    o = int(np.flatnonzero(kind == MLP_OUT)[0])
    m = int(np.flatnonzero((kind == MLP_IN) & (layer == 1))[-1])
    bad = sched.copy()
    bad[m], bad[o] = sched[o], sched[m]
    cases.append(bad)
    for bad in cases:
        with pytest.raises(AssertionError):
            check_order(bad, splits, 2, fused=True)


def test_schedule_rejects_unknown_flags(pkg):
    lib = pkg.load()
    splits = np.ascontiguousarray([1], dtype=np.uintp)
    szp = splits.ctypes.data_as(ctypes.POINTER(ctypes.c_size_t))
    assert lib.pgpu_flow_schedule(1, 1, szp, None, 4, None, 0) == 0
