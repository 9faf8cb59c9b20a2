"""Pins the oracle's flow head (oracle/oracle.c, src/phonon_sampler.c:229-401)
before GPU results are checked against it: the reference's own synthetic-head
golden vector (an independent PyTorch 2.7.1 run), closed forms and float64
restatements of each stage, and the exact cascade of mean_512."""
import json
import os

import numpy as np

import helpers

GOLDEN = json.load(open(os.path.join(helpers.GOLDEN_DIR, "reference_vectors.json")))


def float_head(bits: dict) -> dict:
    return {k: helpers.bf16_float(v) for k, v in bits.items()}


def oracle_head(oracle, oracle_mod, bits):
    return oracle_mod.OracleHead(oracle, float_head(bits))


def test_flow_head_matches_reference_golden(oracle, oracle_mod):
    g = GOLDEN["flow_head_synthetic"]
    head = oracle_head(oracle, oracle_mod, helpers.reference_flow_head_bits())
    condition, state = helpers.reference_flow_head_inputs()
    ok, velocity = head.forward(condition, state, g["s"], g["t"])
    assert ok
    assert np.max(np.abs(velocity - np.asarray(g["expected"], np.float32))) < g["tolerance"]


def test_flow_head_golden_catches_a_planted_mistake(oracle, oracle_mod):
    """The golden vector is not vacuous: dropping the second time embedding
    (t) or the final adaLN shift moves the output past the tolerance."""
    g = GOLDEN["flow_head_synthetic"]
    condition, state = helpers.reference_flow_head_inputs()
    expected = np.asarray(g["expected"], np.float32)
    for name in ("time_alpha_1", "final_ada_bias"):
        bits = helpers.reference_flow_head_bits()
        bits[name] = np.zeros_like(bits[name])
        ok, velocity = oracle_head(oracle, oracle_mod, bits).forward(condition, state, 0.0, 1.0)
        assert ok and np.max(np.abs(velocity - expected)) > 10 * g["tolerance"], name


def test_mean_512_cascade(oracle):
    """Exact on integers (every partial sum exact); within float32 rounding of
    the float64 mean otherwise; and the cascade order itself: a value that
    one order loses and the other keeps."""
    rng = np.random.default_rng(3)
    x = rng.integers(-1000, 1000, 512).astype(np.float32)
    assert oracle.mean_512(x) == np.float32(x.astype(np.float64).mean())
    for _ in range(5):
        x = rng.standard_normal(512).astype(np.float32) * 10
        assert abs(oracle.mean_512(x) - x.astype(np.float64).mean()) < 1e-5
    # 1 in lane 0 of vector 0, -2^24 then +2^24 in lane 0 of vector 1 of the
    # same groups: vector-wise partial sums keep the 1 exactly.
    x = np.zeros(512, np.float32)
    x[0] = 1.0
    x[4] = 2.0 ** 24
    x[20] = -(2.0 ** 24)
    assert oracle.mean_512(x) == np.float32(1.0 / 512.0)


def test_flow_layer_norm_float64(oracle):
    rng = np.random.default_rng(4)
    for affine in (False, True):
        x = (rng.standard_normal(512) * 3 + 1).astype(np.float32)
        w = (1 + 0.1 * rng.standard_normal(512)).astype(np.float32) if affine else None
        b = (0.1 * rng.standard_normal(512)).astype(np.float32) if affine else None
        ok, y = oracle.flow_layer_norm(x, w, b)
        assert ok
        xd = x.astype(np.float64)
        ref = (xd - xd.mean()) / np.sqrt(xd.var() + 1e-6)
        if affine:
            ref = ref * w + b
        assert np.max(np.abs(y - ref)) < 2e-5
    ok, _ = oracle.flow_layer_norm(np.full(512, np.nan, np.float32))
    assert not ok


def test_silu_closed_form(oracle):
    x = np.linspace(-20, 20, 4001).astype(np.float32)
    ok, y = oracle.silu(x)
    xd = x.astype(np.float64)
    assert ok and np.max(np.abs(y - xd / (1 + np.exp(-xd))) / (1 + np.abs(xd))) < 1e-6


def float64_time_embedding(head: dict, which: int, value: float) -> np.ndarray:
    phase = np.float32(value) * head[f"time_freqs_{which}"].astype(np.float32)
    emb = np.concatenate([np.cos(phase.astype(np.float64)), np.sin(phase.astype(np.float64))])
    hid = head[f"time_weight_{which}_0"].astype(np.float64) @ emb + head[f"time_bias_{which}_0"]
    hid = hid / (1 + np.exp(-hid))
    out = head[f"time_weight_{which}_1"].astype(np.float64) @ hid + head[f"time_bias_{which}_1"]
    return head[f"time_alpha_{which}"] * out / np.sqrt(np.mean(out * out) + 1e-5)


def float64_head_forward(head: dict, condition, state, s, t) -> np.ndarray:
    f = {k: v.astype(np.float64) for k, v in head.items()}
    silu = lambda v: v / (1 + np.exp(-v))  # noqa: E731

    def ln(v, w=None, b=None):
        out = (v - v.mean()) / np.sqrt(v.var() + 1e-6)
        return out if w is None else out * w + b

    x = f["input_weight"] @ state + f["input_bias"]
    y = f["cond_weight"] @ condition + f["cond_bias"]
    y = y + 0.5 * (float64_time_embedding(head, 0, s) + float64_time_embedding(head, 1, t))
    for blk in range(helpers.HEAD_BLOCKS):
        mod = f[f"block_ada_weight_{blk}"] @ silu(y) + f[f"block_ada_bias_{blk}"]
        h = ln(x, f[f"block_norm_weight_{blk}"], f[f"block_norm_bias_{blk}"])
        h = h * (1 + mod[512:1024]) + mod[:512]
        first = silu(f[f"block_mlp_weight_{blk}_0"] @ h + f[f"block_mlp_bias_{blk}_0"])
        second = f[f"block_mlp_weight_{blk}_1"] @ first + f[f"block_mlp_bias_{blk}_1"]
        x = x + mod[1024:] * second
    mod = f["final_ada_weight"] @ silu(y) + f["final_ada_bias"]
    h = ln(x) * (1 + mod[512:]) + mod[:512]
    return f["final_weight"] @ h + f["final_bias"]


def test_time_embedding_float64(oracle, oracle_mod):
    head = float_head(helpers.random_flow_head_bits(5))
    oh = oracle_mod.OracleHead(oracle, head)
    for which, value in ((0, 0.0), (1, 1.0), (0, 0.37), (1, -2.5)):
        ok, out = oh.time_embedding(which, value)
        ref = float64_time_embedding(head, which, value)
        assert ok and np.max(np.abs(out - ref)) / np.max(np.abs(ref)) < 1e-5


def test_flow_head_float64_and_lsd_step(oracle, oracle_mod):
    """The whole head against a float64 restatement on a random head; the LSD
    step is noise * sqrt(T) plus the head's velocity at (s, t) = (0, 1), and
    rejects a non-positive temperature."""
    head = float_head(helpers.random_flow_head_bits(6))
    oh = oracle_mod.OracleHead(oracle, head)
    rng = np.random.default_rng(7)
    for _ in range(3):
        condition = rng.standard_normal(512).astype(np.float32)
        raw = rng.standard_normal(32).astype(np.float32)
        ok, v = oh.forward(condition, raw, 0.0, 1.0)
        ref = float64_head_forward(head, condition.astype(np.float64), raw.astype(np.float64),
                                   0.0, 1.0)
        assert ok and np.max(np.abs(v - ref)) / np.max(np.abs(ref)) < 1e-4
        ok, out = oh.lsd_one_step(condition, raw, 0.64)
        noise = raw * np.float32(np.sqrt(np.float32(0.64)))
        ok2, v2 = oh.forward(condition, noise, 0.0, 1.0)
        assert ok and ok2 and np.array_equal(out, noise + v2)
    assert not oh.lsd_one_step(condition, raw, 0.0)[0]
    assert not oh.lsd_one_step(condition, raw, -1.0)[0]


def test_eos_logit_closed_form(oracle, oracle_mod):
    rng = np.random.default_rng(8)
    w = helpers.bf16_float(helpers.bf16_bits(rng.standard_normal(512).astype(np.float32) * 0.05))
    b = np.array([0.25], np.float32)
    x = rng.standard_normal(512).astype(np.float32)
    oh = oracle_mod.OracleHead(oracle, float_head(helpers.random_flow_head_bits(9)))
    ok, logit = oh.eos_logit(w, b, x)
    assert ok and abs(logit - (w.astype(np.float64) @ x + 0.25)) < 1e-5
