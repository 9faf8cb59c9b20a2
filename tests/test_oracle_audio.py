"""The audio-decoder oracle (oracle/oracle_audio.c: Mimi, SEANet, PCM) pinned
by the reference's own known-answer tests, restated here as the closed forms
those tests compute (no reference code runs):

- tests/test_phonon_mimi.c:43-62     depthwise upsample, overlap and startup
- tests/test_phonon_mimi.c:74-178    synthetic two-layer Mimi: Q = K = 0 gives a
                                     uniform causal mean over min(t + 1, 250)
                                     value rows; learned scales .5 / .25
- tests/test_phonon_conv.c:48-98     Conv1d (kernel 3) and ConvTranspose1d
                                     (strides 4, 5, 6) on exact binary
                                     fractions: bit-exact, and chunking-invariant
- tests/test_phonon_conv.c:147-183   residual block closed form
- tests/test_phonon_pcm.c:65-118     the complete decoder's sparse scalar graph
                                     (NRMSE <= 1e-3, max-abs <= 2e-3)
"""
import sys
import os

import numpy as np
import pytest

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "oracle"))
import oracle_py  # noqa: E402

from helpers import mimi_identity_model, pcm_scalar_convs, pcm_scalar_expected  # noqa: E402


@pytest.fixture(scope="module")
def orc():
    return oracle_py.Oracle()


def test_upsample_known_answers(orc):
    k = np.arange(1, 9, dtype=np.float32).reshape(2, 4)
    ok, out = oracle_py.mimi_upsample_frame(orc, k, [2, 3], [5, 7], 2, 2)
    assert ok and out.tolist() == [17, 64, 24, 74]
    ok, out = oracle_py.mimi_upsample_frame(orc, k, [2, 3], [0, 0], 2, 2)
    assert ok and out.tolist() == [2, 15, 4, 18]
    ok, _ = oracle_py.mimi_upsample_frame(orc, k, [np.nan, 3], [0, 0], 2, 2)
    assert not ok


def mimi_synthetic_expected(x, frames):
    """tests/test_phonon_mimi.c:113-136 as numpy (float64 sums)."""
    positions = frames * 16
    t = np.arange(positions)
    i = np.arange(512)
    e = x[t[:, None] // 16, i[None, :] % 32].astype(np.float32)
    prev = np.where((t >= 16)[:, None], 0.5 * x[np.maximum(t // 16 - 1, 0)[:, None], i[None, :] % 32], 0)
    e = (e + prev.astype(np.float32)).astype(np.float32)
    for scale in (0.5, 0.25):
        mean = e.astype(np.float64).mean(axis=1, keepdims=True)
        var = ((e.astype(np.float64) - mean) ** 2).mean(axis=1, keepdims=True)
        s = (1.0 / np.sqrt(np.float32(var / 1) + np.float32(1e-5))).astype(np.float32)
        norm = ((e.astype(np.float64) - mean).astype(np.float32) * s).astype(np.float32)
        csum = np.cumsum(norm.astype(np.float64), axis=0)
        add = np.zeros_like(e)
        for p in range(positions):
            first = p - 249 if p >= 249 else 0
            total = csum[p] - (csum[first - 1] if first > 0 else 0)
            add[p] = (np.float32(scale) * (total / (p + 1 - first)).astype(np.float32))
        e = (e + add).astype(np.float32)
    return e


def test_mimi_synthetic_ring_and_scales(orc):
    frames = 19
    w = mimi_identity_model()
    x = np.sin((np.arange(frames)[:, None] * 7 + np.arange(32)[None, :]).astype(np.float32)
               * np.float32(0.17)).astype(np.float32)
    expected = mimi_synthetic_expected(x, frames)
    m = oracle_py.MimiOracle(orc, w)
    ok, got = m.process(x)
    assert ok and m.positions() == frames * 16
    assert np.max(np.abs(got - expected)) <= 4e-6
    m.close()
    # Frame by frame from a fresh state: the same bits.
    m = oracle_py.MimiOracle(orc, w)
    parts = [m.process(x[f:f + 1])[1] for f in range(frames)]
    m.close()
    assert np.array_equal(np.concatenate(parts), got)


def tiny_conv_expected(trans, stride):
    """tests/test_phonon_conv.c:48-82: exact binary fractions."""
    kernel = 2 * stride if trans else 3
    cin = cout = 2
    n = 7
    wf = np.array([((i % 11) - 5) * 0.125 for i in range(cin * cout * kernel)], np.float32)
    bf = np.array([0.25, -0.5], np.float32)
    x = np.array([((i % 9) - 4) * 0.25 for i in range(n * cin)], np.float32)
    x[12] = x[13] = 0
    exp = np.tile(bf, n * stride).astype(np.float64)
    if trans:
        for t in range(n):
            for c in range(cin):
                for o in range(cout):
                    for k in range(kernel):
                        if t * stride + k < n * stride:
                            exp[(t * stride + k) * cout + o] += x[t * cin + c] * wf[(c * cout + o) * kernel + k]
    else:
        for t in range(n):
            for o in range(cout):
                for c in range(cin):
                    for k in range(kernel):
                        if t + k >= kernel - 1:
                            exp[t * cout + o] += x[(t + k - (kernel - 1)) * cin + c] * wf[(o * cin + c) * kernel + k]
    shape = (cin, cout, kernel) if trans else (cout, cin, kernel)
    return wf.reshape(shape), bf, x.reshape(n, cin), exp.astype(np.float32).reshape(-1, cout)


@pytest.mark.parametrize("trans,stride", [(0, 1), (1, 4), (1, 5), (1, 6)])
def test_conv_tiny_exact_and_chunking(orc, trans, stride):
    w, b, x, exp = tiny_conv_expected(trans, stride)
    c = oracle_py.ConvOracle(orc, w, b, stride, bool(trans))
    ok, y = c.process(x)
    assert ok and np.array_equal(y, exp)
    c.close()
    c = oracle_py.ConvOracle(orc, w, b, stride, bool(trans))
    parts = []
    off = 0
    for count in (1, 2, 1, 3):
        parts.append(c.process(x[off:off + count])[1])
        off += count
    c.close()
    assert np.array_equal(np.concatenate(parts), y)


def test_residual_tiny_closed_form(orc):
    weights = np.array([0.5, -0.25, 0.125, -0.5, 0.75, 0.25], np.float32)
    c3 = oracle_py.ConvOracle(orc, weights.reshape(1, 2, 3), np.array([0.25], np.float32), 1, False)
    c1 = oracle_py.ConvOracle(orc, np.array([0.5, -0.25], np.float32).reshape(2, 1, 1),
                              np.array([0.125, -0.25], np.float32), 1, False)
    x = np.array([-1, 0.5, 2, -0.25, -0.5, -2, 0, 1, 0, 0], np.float32).reshape(5, 2)
    elu = lambda v: np.where(v <= 0, np.expm1(v), v)  # noqa: E731
    exp = np.zeros((5, 2))
    for t in range(5):
        hidden = 0.25
        for c in range(2):
            for k in range(3):
                if t + k >= 2:
                    hidden += elu(float(x[t + k - 2, c])) * weights[c * 3 + k]
        exp[t, 0] = x[t, 0] + elu(hidden) * 0.5 + 0.125
        exp[t, 1] = x[t, 1] - elu(hidden) * 0.25 - 0.25
    ok, y = oracle_py.residual_process(orc, c3, c1, x)
    assert ok
    assert np.all(np.abs(y - exp) <= 1e-5 + 1e-3 * np.abs(exp))


def test_pcm_scalar_graph(orc):
    mimi_w = mimi_identity_model(route_only=True)
    mimi = oracle_py.MimiOracle(orc, mimi_w)
    convs = [oracle_py.ConvOracle(orc, w, b, s, t) for (w, b, s, t) in pcm_scalar_convs()]
    x = np.zeros((3, 32), np.float32)
    x[0, 0], x[1, 0] = -0.5, 0.25
    ok, pcm = oracle_py.pcm_process(orc, mimi, convs, x)
    assert ok and pcm.size == 3 * 1920
    exp = pcm_scalar_expected(x)
    d = pcm.astype(np.float64) - exp
    nrmse = np.sqrt(np.sum(d * d) / np.sum(exp.astype(np.float64) ** 2))
    assert nrmse <= 1e-3 and np.max(np.abs(d)) <= 2e-3
    for c in convs:
        c.close()
    mimi.close()
