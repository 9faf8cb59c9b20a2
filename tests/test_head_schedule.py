"""CPU checks of the one-launch flow head's task list (pgpu_head_flow_schedule).

The launch cannot deadlock if every task is listed after every task it
waits for (work-groups are dispatched in list order). These tests decode the
descriptors the library builds and replay the waits of k_head_flow
(pgpu_head.hip) against the list order: every task exactly once, every wait
satisfied by the tasks listed before it. A planted mistake (a task moved
ahead of one it waits for) must fail the replay."""
import ctypes

import numpy as np
import pytest

COND, EOS, NOISE, INPUT, ADA, MLP_IN, MLP_OUT, FINAL, EMBED = range(9)
BLOCKS = 6
GROUPS512, ROWS512 = 8, 32          # 64-row groups / 16-row tiles of a 512-row projection
ADA_BLOCK, ADA_FINAL = 24, 16       # 64-row groups of one block's / the final layer's rows


def build(lib, tiles, eos, embed):
    n = lib.pgpu_head_flow_schedule(None, 0, tiles, eos, embed)
    out = np.zeros(n, np.uint32)
    got = lib.pgpu_head_flow_schedule(out.ctypes.data_as(ctypes.c_void_p), n, tiles, eos, embed)
    assert got == n
    return out


def decode(d):
    d = d.astype(np.int64)
    return d & 15, (d >> 4) & 15, (d >> 8) & 255, d >> 16


def expected_tasks(tiles, eos, embed):
    per_tile = (GROUPS512 + eos + 1 + ROWS512 + BLOCKS * ADA_BLOCK + ADA_FINAL +
                BLOCKS * (GROUPS512 + ROWS512) + 1 + embed * ROWS512)
    return tiles * per_tile


def check_order(sched, tiles, eos, embed):
    kind, block, tile, index = decode(sched)
    # counters as k_head_flow counts them, per tile
    cond = np.zeros(tiles, int)
    eosc = np.zeros(tiles, int)
    noise = np.zeros(tiles, int)
    ada = np.zeros((tiles, BLOCKS + 1), int)
    u = np.zeros((tiles, BLOCKS), int)
    x = np.zeros((tiles, BLOCKS + 1), int)
    final = np.zeros(tiles, int)
    seen = set()
    for i in range(len(sched)):
        k, b, t, j = int(kind[i]), int(block[i]), int(tile[i]), int(index[i])
        key = (k, b, t, j)
        assert key not in seen, f"task {key} listed twice"
        seen.add(key)
        assert t < tiles
        if k == COND:
            assert j < GROUPS512
            cond[t] += 1
        elif k == EOS:
            assert eos and j == 0
            eosc[t] += 1
        elif k == NOISE:
            noise[t] += 1
        elif k == INPUT:
            assert noise[t] >= 1, f"INPUT {key} before its noise"
            x[t, 0] += 1
        elif k == ADA:
            assert j < BLOCKS * ADA_BLOCK + ADA_FINAL
            assert cond[t] >= GROUPS512, f"ADA {key} before its condition"
            ada[t, j // ADA_BLOCK] += 1
        elif k == MLP_IN:
            assert b < BLOCKS and j < GROUPS512
            assert x[t, b] >= ROWS512, f"MLP_IN {key} before x_{b}"
            assert ada[t, b] >= ADA_BLOCK, f"MLP_IN {key} before block {b}'s modulation"
            u[t, b] += 1
        elif k == MLP_OUT:
            assert b < BLOCKS and j < ROWS512
            assert u[t, b] >= GROUPS512, f"MLP_OUT {key} before its MLP_IN"
            x[t, b + 1] += 1
        elif k == FINAL:
            assert x[t, BLOCKS] >= ROWS512 and ada[t, BLOCKS] >= ADA_FINAL
            assert not eos or eosc[t] >= 1
            final[t] += 1
        elif k == EMBED:
            assert embed and final[t] >= 1
        else:
            raise AssertionError(f"unknown kind {k}")
    assert len(seen) == expected_tasks(tiles, eos, embed)
    assert np.all(final == 1)


@pytest.mark.parametrize("tiles", [1, 2, 4, 5, 16, 64])
@pytest.mark.parametrize("eos,embed", [(0, 0), (1, 0), (1, 1), (0, 1)])
def test_head_schedule_is_complete_and_ordered(pkg, tiles, eos, embed):
    lib = pkg.load()
    sched = build(lib, tiles, eos, embed)
    assert len(sched) == expected_tasks(tiles, eos, embed)
    check_order(sched, tiles, eos, embed)


def test_head_schedule_capacity(pkg):
    lib = pkg.load()
    n = lib.pgpu_head_flow_schedule(None, 0, 4, 1, 1)
    out = np.zeros(n, np.uint32)
    assert lib.pgpu_head_flow_schedule(out.ctypes.data_as(ctypes.c_void_p), n - 1, 4, 1, 1) == 0
    assert lib.pgpu_head_flow_schedule(None, 0, 0, 1, 1) == 0
    assert lib.pgpu_head_flow_schedule(None, 0, 256, 1, 1) == 0


@pytest.mark.parametrize("mistake", ["mlp_out_first", "ada_late", "final_early"])
def test_replay_catches_planted_mistakes(pkg, mistake):
    lib = pkg.load()
    sched = list(build(lib, 4, 1, 1))
    kind, block, tile, index = decode(np.array(sched, np.uint32))
    if mistake == "mlp_out_first":      # block 2's first MLP_OUT ahead of everything
        i = next(i for i in range(len(sched)) if kind[i] == MLP_OUT and block[i] == 2)
        sched.insert(0, sched.pop(i))
    elif mistake == "ada_late":         # block 3's last modulation task moved to the end
        i = max(i for i in range(len(sched)) if kind[i] == ADA and index[i] // ADA_BLOCK == 3)
        sched.append(sched.pop(i))
    else:                               # a FINAL task before the last MLP_OUT of its tile
        i = next(i for i in range(len(sched)) if kind[i] == FINAL)
        j = next(j for j in range(len(sched)) if kind[j] == MLP_OUT and block[j] == 5
                 and tile[j] == tile[i])
        sched.insert(j, sched.pop(i))
    with pytest.raises(AssertionError):
        check_order(np.array(sched, np.uint32), 4, 1, 1)
