"""GPU parity of the audio decoder drop-ins (phonon_mimi.h, phonon_conv.h,
phonon_pcm.h) through the C-ABI, against the reference's own closed forms
and against the oracle (oracle/oracle_audio.c):

- tests/test_phonon_mimi.c:43-62     depthwise upsample known answers
- tests/test_phonon_mimi.c:74-178    the synthetic two-layer Mimi (uniform
                                     causal means over a 250-key window,
                                     learned scales .5 / .25), max-abs 4e-6
- tests/test_phonon_conv.c:48-98     Conv1d / ConvTranspose1d on exact binary
                                     fractions: bit-exact, chunking-invariant
- tests/test_phonon_conv.c:147-183   residual closed form
- tests/test_phonon_pcm.c:65-118     the decoder's sparse scalar graph
                                     (NRMSE <= 1e-3, max-abs <= 2e-3)

and on random weights at the real shapes (512 channels, the 6/5/4 strides,
ring wrap past 1024 positions, requests longer than one device pass): the
oracle at 1e-5 normwise relative (the error is printed), and the GPU against
itself bit for bit however a request is split into calls. Convolutions
whose input channels are not a multiple of 32 (the reference tests' tiny
ones) run the sequential path: the same fp32 operations in the same order
as the oracle, so they are compared bit for bit."""
import ctypes

import numpy as np
import pytest

import helpers
from helpers import bf16_bits, conv_model, mimi_identity_model, mimi_model, pcm_scalar_convs, \
    pcm_scalar_expected, random_mimi, random_pcm_convs, rounded

pytestmark = pytest.mark.gpu
TOL = 1e-5


def fp(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


class Mimi:
    def __init__(self, lib, model):
        self.lib, self.model = lib, model
        self.h = ctypes.c_void_p()
        assert lib.phonon_mimi_state_create(ctypes.byref(model), ctypes.byref(self.h)) == 1

    def process(self, x):
        x = np.ascontiguousarray(x, np.float32)
        out = np.full((x.shape[0] * 16, 512), np.nan, np.float32)
        ok = self.lib.phonon_mimi_process(self.h, fp(x), x.shape[0], fp(out), out.shape[0])
        return ok, out

    def close(self):
        self.lib.phonon_mimi_state_destroy(self.h)


class Conv:
    def __init__(self, lib, model):
        self.lib, self.model = lib, model
        self.h = ctypes.c_void_p()
        assert lib.phonon_conv_state_create(model, ctypes.byref(self.h)) == 1
        self.cout = lib.phonon_conv_output_channels(model)
        self.stride = lib.phonon_conv_stride(model)

    def process(self, x):
        x = np.ascontiguousarray(x, np.float32)
        out = np.full((x.shape[0] * self.stride, self.cout), np.nan, np.float32)
        ok = self.lib.phonon_conv_process(self.h, fp(x), x.shape[0], fp(out), out.shape[0])
        return ok, out

    def close(self):
        self.lib.phonon_conv_state_destroy(self.h)


def normwise(a, b):
    return helpers.normwise(np.asarray(a, np.float64), np.asarray(b, np.float64))


# ------------------------------------------------------------------- Mimi


def test_upsample_known_answers(lib, pkg):
    views = pkg.Views()
    k = views.bf16(bf16_bits(np.arange(1, 9, dtype=np.float32)), (2, 1, 4))
    out = np.zeros(4, np.float32)
    x = np.array([2, 3], np.float32)
    for prev, exp in (([5, 7], [17, 64, 24, 74]), ([0, 0], [2, 15, 4, 18])):
        p = np.array(prev, np.float32)
        assert lib.phonon_mimi_upsample_frame(ctypes.byref(k), fp(x), fp(p), 2, 2, fp(out)) == 1
        assert out.tolist() == exp
    bad = np.array([np.nan, 3], np.float32)
    assert lib.phonon_mimi_upsample_frame(ctypes.byref(k), fp(bad), fp(p), 2, 2, fp(out)) == 0


def test_mimi_synthetic_ring_and_scales(lib, pkg):
    from test_oracle_audio import mimi_synthetic_expected
    frames = 19
    views = pkg.Views()
    model = mimi_model(lib, pkg, views, mimi_identity_model())
    x = np.sin((np.arange(frames)[:, None] * 7 + np.arange(32)[None, :]).astype(np.float32)
               * np.float32(0.17)).astype(np.float32)
    expected = mimi_synthetic_expected(x, frames)
    m = Mimi(lib, model)
    ok, got = m.process(x)
    assert ok == 1 and lib.phonon_mimi_positions(m.h) == frames * 16
    err = float(np.max(np.abs(got - expected)))
    print(f"mimi synthetic max-abs {err:.3g}")
    assert err <= 4e-6
    # Frame by frame from a reset state: the same bits.
    lib.phonon_mimi_state_reset(m.h)
    assert lib.phonon_mimi_positions(m.h) == 0
    parts = []
    for f in range(frames):
        ok, y = m.process(x[f:f + 1])
        assert ok == 1
        parts.append(y)
    assert np.array_equal(np.concatenate(parts), got)
    m.close()


def test_mimi_random_weights_ring_wrap_against_oracle(lib, pkg, oracle, oracle_mod):
    """70 frames = 1120 positions: past the 1024-row device ring, past one
    32-frame device pass, and every row against the oracle; then the same
    request in uneven calls, bit for bit."""
    frames = 70
    w = random_mimi(811)
    x = np.random.default_rng(812).standard_normal((frames, 32)).astype(np.float32)
    om = oracle_mod.MimiOracle(oracle, w)
    ok, exp = om.process(x)
    om.close()
    assert ok
    views = pkg.Views()
    model = mimi_model(lib, pkg, views, w)
    m = Mimi(lib, model)
    ok, got = m.process(x)
    assert ok == 1
    err = normwise(got, exp)
    rows = [normwise(got[r * 16:(r + 1) * 16], exp[r * 16:(r + 1) * 16]) for r in range(frames)]
    print(f"mimi random normwise {err:.3g}, worst frame {max(rows):.3g}")
    assert err <= TOL and max(rows) <= TOL
    lib.phonon_mimi_state_reset(m.h)
    parts, off = [], 0
    for count in (1, 33, 5, 31):
        ok, y = m.process(x[off:off + count])
        assert ok == 1
        parts.append(y)
        off += count
    assert off == frames and np.array_equal(np.concatenate(parts), got)
    m.close()


def test_mimi_rejects_bad_requests(lib, pkg):
    views = pkg.Views()
    model = mimi_model(lib, pkg, views, mimi_identity_model())
    m = Mimi(lib, model)
    x = np.zeros((2, 32), np.float32)
    out = np.zeros((32, 512), np.float32)
    assert lib.phonon_mimi_process(m.h, fp(x), 2, fp(out), 31) == 0   # capacity
    x[1, 3] = np.inf
    assert lib.phonon_mimi_process(m.h, fp(x), 2, fp(out), 32) == 0   # non-finite
    assert lib.phonon_mimi_positions(m.h) == 0
    x[1, 3] = 0
    assert lib.phonon_mimi_process(m.h, fp(x), 0, fp(out), 0) == 0   # no frames
    assert lib.phonon_mimi_process(m.h, fp(x), 2, fp(out), 32) == 1
    assert lib.phonon_mimi_positions(m.h) == 32
    m.close()


# ------------------------------------------------------------- convolutions


@pytest.mark.parametrize("trans,stride", [(0, 1), (1, 4), (1, 5), (1, 6)])
def test_conv_tiny_exact_and_chunking(lib, pkg, trans, stride):
    from test_oracle_audio import tiny_conv_expected
    w, b, x, exp = tiny_conv_expected(trans, stride)
    views = pkg.Views()
    model = conv_model(lib, views, w, b, stride, trans)
    c = Conv(lib, model)
    ok, y = c.process(x)
    assert ok == 1 and np.array_equal(y, exp)
    c.process(x)  # history now holds x; reset must clear it
    lib.phonon_conv_state_reset(c.h)
    parts, off = [], 0
    for count in (1, 2, 1, 3):
        ok, p = c.process(x[off:off + count])
        assert ok == 1
        parts.append(p)
        off += count
    assert np.array_equal(np.concatenate(parts), y)
    c.close()
    lib.phonon_conv_model_destroy(model)


SEANET = [  # (cin, cout, kernel, stride) of each distinct SEANet convolution
    (512, 512, 7, 1), (512, 256, 12, 6), (256, 128, 3, 1), (128, 256, 1, 1),
    (256, 128, 10, 5), (128, 64, 8, 4), (64, 1, 3, 1)]


@pytest.mark.parametrize("cin,cout,kernel,stride", SEANET)
def test_conv_random_against_oracle(lib, pkg, oracle, oracle_mod, cin, cout, kernel, stride):
    trans = stride > 1
    rng = np.random.default_rng(cin * 7 + cout + kernel)
    shape = (cin, cout, kernel) if trans else (cout, cin, kernel)
    w = rounded((rng.standard_normal(shape) * (cin * kernel / stride) ** -0.5).astype(np.float32))
    b = rounded((rng.standard_normal(cout) * 0.1).astype(np.float32))
    positions = 97
    x = rng.standard_normal((positions, cin)).astype(np.float32)
    oc = oracle_mod.ConvOracle(oracle, w, b, stride, trans)
    ok, exp = oc.process(x)
    oc.close()
    assert ok
    views = pkg.Views()
    model = conv_model(lib, views, w, b, stride, trans)
    assert lib.phonon_conv_input_channels(model) == cin
    c = Conv(lib, model)
    ok, y = c.process(x)
    assert ok == 1
    err = normwise(y, exp)
    print(f"conv {cin}->{cout} k{kernel} s{stride} normwise {err:.3g}")
    if cin % 32:
        assert np.array_equal(y, exp)      # sequential path
    else:
        assert err <= TOL                  # MFMA path
    lib.phonon_conv_state_reset(c.h)
    parts, off = [], 0
    for count in (5, 1, 60, 31):
        ok, p = c.process(x[off:off + count])
        assert ok == 1
        parts.append(p)
        off += count
    assert np.array_equal(np.concatenate(parts), y)
    c.close()
    lib.phonon_conv_model_destroy(model)


def test_conv_elu(lib):
    x = np.linspace(-6, 3, 1001).astype(np.float32)
    y = x.copy()
    lib.phonon_conv_elu(fp(y), y.size)
    exp = np.where(x <= 0, np.expm1(x.astype(np.float64)), x)
    assert np.max(np.abs(y - exp)) <= 2e-7
    assert np.array_equal(y[x > 0], x[x > 0])


def test_residual_tiny_closed_form(lib, pkg):
    views = pkg.Views()
    weights = np.array([0.5, -0.25, 0.125, -0.5, 0.75, 0.25], np.float32)
    c3 = conv_model(lib, views, weights.reshape(1, 2, 3), np.array([0.25], np.float32), 1, False)
    c1 = conv_model(lib, views, np.array([0.5, -0.25], np.float32).reshape(2, 1, 1),
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
    h = ctypes.c_void_p()
    assert lib.phonon_residual_state_create(c3, c1, ctypes.byref(h)) == 1
    y = np.zeros_like(x)
    assert lib.phonon_residual_process(h, fp(x), 5, fp(y), 5) == 1
    assert np.all(np.abs(y - exp) <= 1e-5 + 1e-3 * np.abs(exp))
    assert lib.phonon_residual_process(h, fp(x), 5, fp(y), 4) == 0  # capacity
    lib.phonon_residual_state_destroy(h)
    lib.phonon_conv_model_destroy(c3)
    lib.phonon_conv_model_destroy(c1)


@pytest.mark.parametrize("channels", [512, 256, 128])
def test_residual_random_against_oracle(lib, pkg, oracle, oracle_mod, channels):
    rng = np.random.default_rng(channels)
    half = channels // 2
    w3 = rounded((rng.standard_normal((half, channels, 3)) * (3 * channels) ** -0.5)
                 .astype(np.float32))
    b3 = rounded((rng.standard_normal(half) * 0.1).astype(np.float32))
    w1 = rounded((rng.standard_normal((channels, half, 1)) * half ** -0.5).astype(np.float32))
    b1 = rounded((rng.standard_normal(channels) * 0.1).astype(np.float32))
    x = rng.standard_normal((83, channels)).astype(np.float32)
    o3 = oracle_mod.ConvOracle(oracle, w3, b3, 1, False)
    o1 = oracle_mod.ConvOracle(oracle, w1, b1, 1, False)
    ok, exp = oracle_mod.residual_process(oracle, o3, o1, x)
    o3.close()
    o1.close()
    assert ok
    views = pkg.Views()
    c3 = conv_model(lib, views, w3, b3, 1, False)
    c1 = conv_model(lib, views, w1, b1, 1, False)
    h = ctypes.c_void_p()
    assert lib.phonon_residual_state_create(c3, c1, ctypes.byref(h)) == 1
    y = np.full_like(x, np.nan)
    assert lib.phonon_residual_process(h, fp(x), x.shape[0], fp(y), x.shape[0]) == 1
    err = normwise(y, exp)
    print(f"residual {channels} normwise {err:.3g}")
    assert err <= TOL
    lib.phonon_residual_state_reset(h)
    parts, off = [], 0
    for count in (40, 1, 42):
        p = np.full((count, channels), np.nan, np.float32)
        assert lib.phonon_residual_process(h, fp(x[off:off + count].copy()), count, fp(p),
                                           count) == 1
        parts.append(p)
        off += count
    assert np.array_equal(np.concatenate(parts), y)
    lib.phonon_residual_state_destroy(h)
    lib.phonon_conv_model_destroy(c3)
    lib.phonon_conv_model_destroy(c1)


# --------------------------------------------------------------------- PCM


class Pcm:
    def __init__(self, lib, pkg, views, mimi_w, convs):
        self.lib = lib
        self.mimi, self.model = helpers.pcm_model(lib, pkg, views, mimi_w, convs)
        self.h = ctypes.c_void_p()
        assert lib.phonon_pcm_state_create(self.model, ctypes.byref(self.h)) == 1

    def process(self, x, final=False):
        x = np.ascontiguousarray(x, np.float32)
        raw = np.full(x.shape[0] * 1920, np.nan, np.float32)
        fin = np.full_like(raw, np.nan) if final else None
        ok = self.lib.phonon_pcm_process(self.h, fp(x), x.shape[0], fp(raw), raw.size,
                                         fp(fin) if final else None, raw.size if final else 0)
        return ok, raw, fin

    def close(self):
        self.lib.phonon_pcm_state_destroy(self.h)
        self.lib.phonon_pcm_model_destroy(self.model)


def test_pcm_scalar_graph(lib, pkg):
    views = pkg.Views()
    p = Pcm(lib, pkg, views, mimi_identity_model(route_only=True), pcm_scalar_convs())
    x = np.zeros((3, 32), np.float32)
    x[0, 0], x[1, 0] = -0.5, 0.25
    ok, raw, fin = p.process(x, final=True)
    assert ok == 1 and lib.phonon_pcm_samples(p.h) == 3 * 1920
    assert np.array_equal(raw, fin)
    exp = pcm_scalar_expected(x)
    d = raw.astype(np.float64) - exp
    nrmse = np.sqrt(np.sum(d * d) / np.sum(exp.astype(np.float64) ** 2))
    print(f"pcm scalar nrmse {nrmse:.3g} max-abs {np.max(np.abs(d)):.3g}")
    assert nrmse <= 1e-3 and np.max(np.abs(d)) <= 2e-3
    assert lib.phonon_pcm_finish(p.h) == 1
    assert lib.phonon_pcm_process(p.h, fp(x), 3, fp(raw), raw.size, None, 0) == 0
    assert lib.phonon_pcm_finish(p.h) == 0
    lib.phonon_pcm_state_reset(p.h)
    assert lib.phonon_pcm_samples(p.h) == 0
    ok, raw2, _ = p.process(x)
    assert ok == 1 and np.array_equal(raw2, raw)
    p.close()


def test_pcm_random_weights_against_oracle(lib, pkg, oracle, oracle_mod):
    """Random weights through the whole decoder: 35 frames (one full 32-frame
    device pass and a partial one) against the oracle, then the same frames
    in uneven calls, bit for bit."""
    frames = 35
    mimi_w = random_mimi(901)
    convs = random_pcm_convs(902)
    x = np.random.default_rng(903).standard_normal((frames, 32)).astype(np.float32)
    om = oracle_mod.MimiOracle(oracle, mimi_w)
    oc = [oracle_mod.ConvOracle(oracle, w, b, s, t) for (w, b, s, t) in convs]
    ok, exp = oracle_mod.pcm_process(oracle, om, oc, x)
    for c in oc:
        c.close()
    om.close()
    assert ok and np.all(np.isfinite(exp))
    views = pkg.Views()
    p = Pcm(lib, pkg, views, mimi_w, convs)
    ok, raw, _ = p.process(x)
    assert ok == 1
    err = normwise(raw, exp)
    frame_err = max(normwise(raw[f * 1920:(f + 1) * 1920], exp[f * 1920:(f + 1) * 1920])
                    for f in range(frames))
    print(f"pcm random normwise {err:.3g}, worst frame {frame_err:.3g}, rms {np.std(exp):.3g}")
    assert err <= TOL and frame_err <= TOL
    lib.phonon_pcm_state_reset(p.h)
    parts, off = [], 0
    for count in (2, 31, 2):
        ok, r, _ = p.process(x[off:off + count])
        assert ok == 1
        parts.append(r)
        off += count
    assert np.array_equal(np.concatenate(parts), raw)
    p.close()


def test_pcm_rejects_bad_requests(lib, pkg):
    views = pkg.Views()
    p = Pcm(lib, pkg, views, mimi_identity_model(route_only=True), pcm_scalar_convs())
    x = np.zeros((2, 32), np.float32)
    raw = np.zeros(2 * 1920, np.float32)
    assert lib.phonon_pcm_process(p.h, fp(x), 2, fp(raw), raw.size - 1, None, 0) == 0
    x[0, 5] = np.nan
    assert lib.phonon_pcm_process(p.h, fp(x), 2, fp(raw), raw.size, None, 0) == 0
    x[0, 5] = 0
    assert lib.phonon_pcm_samples(p.h) == 0
    assert lib.phonon_pcm_process(p.h, fp(x), 2, fp(raw), raw.size, None, 0) == 1
    assert lib.phonon_pcm_samples(p.h) == 2 * 1920
    p.close()
