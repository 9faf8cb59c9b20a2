"""The device path fed from a kpack (phonon_pack.h + phonon_transformer.h's
pack-side helpers), through the C-ABI: a model-shaped synthetic pack (the
nine Flow layers under their checkpoint names, Q8_0; BF16 norms, out_norm,
input_linear, bos_emb, latent statistics) is opened, its layers loaded by
name and registered for the device (phonon_flow_prepare_weights), then
decoded with phonon_flow_stack_step against the oracle; the helpers that run
on the device (embed_latent, embed_bos, output_norm, voice projection,
speaker/duration conditioning) against the oracle's linear / LayerNorm.
Tolerance 1e-4 normwise."""
import ctypes

import numpy as np
import pytest

import helpers
from test_pack import model_pack_tensors, opened

pytestmark = pytest.mark.gpu
TOL = 1e-4


def f32(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


@pytest.fixture(scope="module")
def scaled_pack(syn, tmp_path_factory):
    model, extra, tensors = model_pack_tensors(syn, seed=405, factor=0.1)
    path = tmp_path_factory.mktemp("kpack") / "model.kpack"
    path.write_bytes(helpers.kpack_bytes(tensors))
    return model, extra, str(path).encode()


def test_pack_layers_decode_vs_oracle(lib, pkg, oracle, oracle_mod, syn, scaled_pack):
    model, _, path = scaled_pack
    ok, pack = opened(lib, path)
    assert ok
    storage = (pkg.PhononTensorView * (9 * 8))()
    weights = (pkg.PhononFlowLayerWeights * 9)()
    assert lib.phonon_flow_load_layers(pack, storage, weights)
    assert lib.phonon_flow_prepare_weights(weights, 9), pkg.last_error(lib)
    om = oracle_mod.OracleModel(oracle, helpers.oracle_layers(oracle, model))
    steps = 12
    cache = lib.phonon_kv_cache_init.argtypes[0]._type_()
    assert lib.phonon_kv_cache_init(ctypes.byref(cache), steps)
    okeys = np.zeros((9, steps, 512), np.float32)
    ovals = np.zeros_like(okeys)
    rng = np.random.default_rng(406)
    for pos in range(steps):
        x = rng.standard_normal(512).astype(np.float32)
        y = np.zeros(512, np.float32)
        assert lib.phonon_flow_stack_step(weights, ctypes.byref(cache), pos, f32(x), 10000.0,
                                          f32(y)), pkg.last_error(lib)
        ok, ref = om.stack_step(okeys, ovals, steps, pos, x)
        assert ok and helpers.normwise(y, ref) <= TOL, (pos, helpers.normwise(y, ref))
    lib.phonon_kv_cache_destroy(ctypes.byref(cache))
    lib.phonon_flow_release_weights(weights)
    lib.phonon_pack_close(pack)


def test_pack_embeddings_and_output_norm_vs_oracle(lib, pkg, oracle, syn, scaled_pack):
    """phonon_flow_embed_latent / embed_bos (input_linear . latent +
    condition, src/phonon_transformer.c:842-874) and phonon_flow_output_norm
    (LayerNorm eps 1e-5 in place, :904-914) with the pack's tensors."""
    _, extra, path = scaled_pack
    ok, pack = opened(lib, path)
    assert ok
    lin = syn.bf16_to_f32(extra["flow_lm.input_linear.weight"]).reshape(512, 32)
    rng = np.random.default_rng(407)
    latent = rng.standard_normal(32).astype(np.float32)
    cond = rng.standard_normal(512).astype(np.float32)
    out = np.zeros(512, np.float32)
    assert lib.phonon_flow_embed_latent(pack, f32(latent), f32(cond), f32(out)), \
        pkg.last_error(lib)
    ok, emb = oracle.linear_batch(lin, latent)
    assert ok and helpers.normwise(out, emb[0] + cond) <= TOL
    bos = syn.bf16_to_f32(extra["flow_lm.bos_emb"])
    assert lib.phonon_flow_embed_bos(pack, f32(cond), f32(out))
    ok, emb = oracle.linear_batch(lin, bos)
    assert ok and helpers.normwise(out, emb[0] + cond) <= TOL
    v = (rng.standard_normal(512) * 4 + 1).astype(np.float32)
    got = v.copy()
    assert lib.phonon_flow_output_norm(pack, f32(got))
    ok, ref = oracle.layer_norm(v, syn.bf16_to_f32(extra["flow_lm.out_norm.weight"]),
                                syn.bf16_to_f32(extra["flow_lm.out_norm.bias"]), 1e-5)
    assert ok and helpers.normwise(got, ref) <= TOL
    bad = cond.copy()
    bad[7] = np.inf
    assert not lib.phonon_flow_embed_latent(pack, f32(latent), f32(bad), f32(out))
    lib.phonon_pack_close(pack)


def test_voice_projection_and_condition_vs_oracle(lib, pkg, oracle):
    """phonon_voice_project (a 512x512 linear over voice frames) and
    phonon_flow_condition (speaker embedding row through its projection plus
    the [cos | sin] duration features through theirs,
    src/phonon_transformer.c:711-757)."""
    rng = np.random.default_rng(408)
    views = pkg.Views()
    proj_bits = helpers.bf16_bits(rng.standard_normal((512, 512)).astype(np.float32) * 0.04)
    proj = views.bf16(proj_bits, (512, 512))
    frames = 5
    voice = rng.standard_normal((frames, 512)).astype(np.float32)
    out = np.zeros((frames, 512), np.float32)
    assert lib.phonon_voice_project(f32(voice), frames, ctypes.byref(proj), f32(out))
    ok, ref = oracle.linear_batch(helpers.bf16_float(proj_bits), voice)
    assert ok and helpers.normwise(out, ref) <= TOL
    assert not lib.phonon_voice_project(f32(voice), 0, ctypes.byref(proj), f32(out))
    table_bits = helpers.bf16_bits(rng.standard_normal((4, 16)).astype(np.float32))
    sp_bits = helpers.bf16_bits(rng.standard_normal((512, 16)).astype(np.float32) * 0.2)
    du_bits = helpers.bf16_bits(rng.standard_normal((512, 128)).astype(np.float32) * 0.1)
    table, sp, du = (views.bf16(table_bits, (4, 16)), views.bf16(sp_bits, (512, 16)),
                     views.bf16(du_bits, (512, 128)))
    cond = np.zeros(512, np.float32)
    delta = 0.37
    assert lib.phonon_flow_condition(ctypes.byref(table), ctypes.byref(sp), ctypes.byref(du), 2,
                                     delta, f32(cond)), pkg.last_error(lib)
    phase = 1000.0 * np.float64(np.float32(delta)) / np.power(10000.0, np.arange(64) / 63.0)
    feats = np.concatenate([np.cos(phase), np.sin(phase)]).astype(np.float32)
    ok, a = oracle.linear_batch(helpers.bf16_float(sp_bits), helpers.bf16_float(table_bits[2]))
    ok2, b = oracle.linear_batch(helpers.bf16_float(du_bits), feats)
    assert ok and ok2 and helpers.normwise(cond, a[0] + b[0]) <= TOL
    assert not lib.phonon_flow_condition(ctypes.byref(table), ctypes.byref(sp), ctypes.byref(du),
                                         4, delta, f32(cond))   # speaker out of range


def test_pack_flow_head_and_eos_vs_golden_and_oracle(lib, pkg, oracle, oracle_mod, syn,
                                                     scaled_pack):
    """The flow head loaded from the pack by its checkpoint names
    (phonon_flow_head_load) drives phonon_flow_head_forward to the reference
    test's golden velocity (tests/test_phonon_sampler.c:148-195, its 2e-4)
    and to the oracle within 1e-4, so every view is wired to its role; the
    pack's EOS row (phonon_flow_eos_logit, on the device linear) against the
    oracle's dot product within 1e-4 relative; bad arguments rejected."""
    _, extra, path = scaled_pack
    ok, pack = opened(lib, path)
    assert ok
    head = pkg.PhononFlowHead()
    assert lib.phonon_flow_head_load(pack, ctypes.byref(head))
    g = __import__("json").load(open(helpers.GOLDEN_DIR + "/reference_vectors.json"))
    g = g["flow_head_synthetic"]
    condition, state = helpers.reference_flow_head_inputs()
    out = np.zeros(32, np.float32)
    assert lib.phonon_flow_head_forward(ctypes.byref(head), f32(condition), f32(state), 0.0, 1.0,
                                        f32(out)), pkg.last_error(lib)
    assert np.max(np.abs(out - np.asarray(g["expected"], np.float32))) < g["tolerance"]
    floats = {k: helpers.bf16_float(v) for k, v in helpers.reference_flow_head_bits().items()}
    oh = oracle_mod.OracleHead(oracle, floats)
    ok, ref = oh.forward(condition, state, 0.0, 1.0)
    assert ok and helpers.normwise(out, ref) <= TOL
    lib.phonon_flow_head_release(ctypes.byref(head))

    w = syn.bf16_to_f32(extra["flow_lm.out_eos.weight"]).reshape(512)
    b = syn.bf16_to_f32(extra["flow_lm.out_eos.bias"])
    rng = np.random.default_rng(417)
    for _ in range(3):
        x = rng.standard_normal(512).astype(np.float32)
        logit = np.zeros(1, np.float32)
        assert lib.phonon_flow_eos_logit(pack, f32(x), f32(logit)), pkg.last_error(lib)
        ok, want = oh.eos_logit(w, b, x)
        assert ok
        assert abs(float(logit[0]) - want) <= TOL * max(abs(want), float(np.abs(w * x).sum()))
    assert not lib.phonon_flow_eos_logit(None, f32(x), f32(logit))
    x[0] = np.nan
    assert not lib.phonon_flow_eos_logit(pack, f32(x), f32(logit))
    lib.phonon_pack_close(pack)
