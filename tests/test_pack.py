"""The kpack v1 reader of phonon_pack.h on the CPU (no GPU needed), against
a synthetic 209-tensor pack written here with hashlib digests, following
tests/test_phonon_pack.c:56-360 of the reference: open and count, every
rejected mutation, the pinned index, BF16 decode, Q8/BF16 expansion,
bounded fp32 materialization with rollback; then the pack-side helpers of
phonon_transformer.h that need no device (layer views by name, token
embeddings, latent normalization, prefix rows)."""
import ctypes
import struct

import numpy as np
import pytest

import helpers


@pytest.fixture(scope="module")
def lib(pkg):
    return pkg.load()


def write(tmp_path, data, name="p.kpack"):
    p = tmp_path / name
    p.write_bytes(data)
    return str(p).encode()


def opened(lib, path, pinned=False):
    pack = ctypes.c_void_p()
    fn = lib.phonon_pack_open if pinned else lib.phonon_pack_open_for_tests
    ok = fn(path, ctypes.byref(pack))
    return ok, pack


def rehash(data, index=False, meta=False):
    """Recompute the index or metadata digest after a mutation inside it (as
    the reference test does), so only the mutated field can reject."""
    import hashlib
    b = bytearray(data)
    meta_size = struct.unpack_from("<I", b, 192)[0]
    index_at = 196 + meta_size
    index_size = struct.unpack_from("<Q", b, 16)[0]
    if index:
        b[96:128] = hashlib.sha256(bytes(b[index_at:index_at + index_size])).digest()
    if meta:
        b[160:192] = hashlib.sha256(bytes(b[196:index_at])).digest()
    return bytes(b)


def test_synthetic_pack_opens_and_names_resolve(lib, pkg, tmp_path):
    path = write(tmp_path, helpers.kpack_bytes(helpers.kpack_synthetic()))
    ok, pack = opened(lib, path)
    assert ok and lib.phonon_pack_tensor_count(pack) == 209
    v = pkg.PhononTensorView()
    assert lib.phonon_pack_tensor(pack, b"flow_lm.fixture_000.weight", ctypes.byref(v))
    assert v.dtype == 1 and v.rank == 2 and list(v.shape[:2]) == [1, 32] and v.byte_count == 34
    raw = ctypes.string_at(v.data, 34)
    assert raw == b"\x00\x3c" + b"\x01" * 32
    assert not lib.phonon_pack_tensor(pack, b"flow_lm.missing.weight", ctypes.byref(v))
    name, length = ctypes.c_char_p(), ctypes.c_size_t()
    assert lib.phonon_pack_tensor_at(pack, 208, ctypes.byref(name), ctypes.byref(length),
                                     ctypes.byref(v))
    assert ctypes.string_at(name, length.value) == b"mimi.fixture_208.weight"
    assert not lib.phonon_pack_tensor_at(pack, 209, ctypes.byref(name), ctypes.byref(length),
                                         ctypes.byref(v))
    # The published model's index digest is pinned: the synthetic index is not it.
    ok_pinned, _ = opened(lib, path, pinned=True)
    assert not ok_pinned
    lib.phonon_pack_close(pack)
    for _ in range(8):  # open/close cycles
        ok, pack = opened(lib, path)
        assert ok
        lib.phonon_pack_close(pack)


def index_offsets(data):
    meta = struct.unpack_from("<I", data, 192)[0]
    first = 196 + meta
    name_size, _, rank = struct.unpack_from("<HBB", data, first)
    second = first + 4 + rank * 8 + 16 + name_size
    return first, rank, second, data[second + 3]


@pytest.mark.parametrize("what", ["truncated", "version", "source", "config", "metadata",
                                  "overflow", "overlap", "dtype", "length", "row_shape",
                                  "payload", "name", "count", "trailing_index", "meta_pad",
                                  "duplicate_name", "misaligned_offset"])
def test_rejected_pack_variants(lib, tmp_path, what):
    """tests/test_phonon_pack.c:171-244 (each mutation alone must reject),
    plus a wrong tensor count, trailing index bytes, non-space metadata
    padding, a duplicate name and a misaligned payload offset."""
    tensors = helpers.kpack_synthetic()
    data = bytearray(helpers.kpack_bytes(tensors))
    first, rank, second, second_rank = index_offsets(bytes(data))
    payload_size = struct.unpack_from("<Q", data, 24)[0]
    if what == "truncated":
        data = data[:-1]
    elif what == "version":
        data[8:12] = struct.pack("<I", 2)
    elif what == "source":
        data[32] ^= 1
    elif what == "config":
        data[64] ^= 1
    elif what == "metadata":
        data[196 + 20] = ord("X")
        data = bytearray(rehash(bytes(data), meta=True))
    elif what == "overflow":
        data[first + 4:first + 12] = b"\xff" * 8
        data = bytearray(rehash(bytes(data), index=True))
    elif what == "overlap":
        data[second + 4 + second_rank * 8:second + 12 + second_rank * 8] = b"\0" * 8
        data = bytearray(rehash(bytes(data), index=True))
    elif what == "dtype":
        data[first + 2] = 9
        data = bytearray(rehash(bytes(data), index=True))
    elif what == "length":
        at = first + 4 + rank * 8 + 8
        data[at:at + 8] = b"\0" * 8
        data = bytearray(rehash(bytes(data), index=True))
    elif what == "row_shape":
        data[first + 4:first + 20] = struct.pack("<QQ", 2, 16)
        data = bytearray(rehash(bytes(data), index=True))
    elif what == "payload":
        data[len(data) - payload_size] ^= 1
    elif what == "name":
        data[first + 4 + rank * 8 + 16] = ord("/")
        data = bytearray(rehash(bytes(data), index=True))
    elif what == "count":
        data = bytearray(helpers.kpack_bytes(tensors[:208]))
    elif what == "trailing_index":
        # one more (well-formed) entry than the header counts
        data = bytearray(helpers.kpack_bytes(tensors + [("mimi.extra.weight", 2, (1,),
                                                          b"\x80\x3f")]))
        data[12:16] = struct.pack("<I", 209)
    elif what == "meta_pad":
        meta = struct.unpack_from("<I", data, 192)[0]
        if meta and data[196 + meta - 1] == ord(" "):
            data[196 + meta - 1] = ord("x")
        else:
            data[196 + 5] = ord("x")
        data = bytearray(rehash(bytes(data), meta=True))
    elif what == "duplicate_name":
        tensors[1] = (tensors[0][0],) + tensors[1][1:]
        data = bytearray(helpers.kpack_bytes(tensors))
    elif what == "misaligned_offset":
        at = second + 4 + second_rank * 8
        off = struct.unpack_from("<Q", data, at)[0]
        data[at:at + 8] = struct.pack("<Q", off + 1)
        data = bytearray(rehash(bytes(data), index=True))
    ok, pack = opened(lib, write(tmp_path, bytes(data), what + ".kpack"))
    assert not ok and not pack.value
    assert not lib.phonon_pack_open_for_tests(write(tmp_path, helpers.kpack_bytes(
        helpers.kpack_synthetic()), "ok.kpack"), None)


def test_bf16_decode_and_expansion(lib, pkg, tmp_path):
    ok, pack = opened(lib, write(tmp_path, helpers.kpack_bytes(helpers.kpack_synthetic())))
    assert ok
    v = pkg.PhononTensorView()
    assert lib.phonon_pack_tensor(pack, b"mimi.fixture_036.weight", ctypes.byref(v))
    out = np.zeros(1, np.float32)
    # Overlapping buffers are rejected; otherwise the bits decode exactly.
    assert not lib.phonon_bf16_to_float(v.data, 1, ctypes.cast(v.data, ctypes.POINTER(
        ctypes.c_float)))
    assert lib.phonon_bf16_to_float(v.data, 1, out.ctypes.data_as(ctypes.POINTER(
        ctypes.c_float))) and out[0] == 1.0
    inf = np.array([0x7F80], np.uint16)
    assert not lib.phonon_bf16_to_float(inf.ctypes.data, 1, out.ctypes.data_as(
        ctypes.POINTER(ctypes.c_float)))
    lib.phonon_pack_close(pack)
    # tests/test_phonon_pack.c:331-345: [1, -2] from bf16, an inf rejected
    # with the output left NULL; Q8 values times the block scale.
    views = pkg.Views()
    small = views.bf16(np.array([0x3F80, 0xC000], np.uint16), (1, 2))
    f = ctypes.POINTER(ctypes.c_float)()
    assert lib.phonon_tensor_expand_linear(ctypes.byref(small), ctypes.byref(f))
    assert f[0] == 1.0 and f[1] == -2.0
    bad = views.bf16(np.array([0x7F80], np.uint16), (1, 1))
    g = ctypes.cast(1, ctypes.POINTER(ctypes.c_float))
    assert not lib.phonon_tensor_expand_linear(ctypes.byref(bad), ctypes.byref(g)) and not g
    blocks = np.zeros(2, pkg.Q8_BLOCK)
    blocks["scale_bits"] = [0x3800, 0xC000]   # 0.5, -2.0
    blocks["values"][0] = np.arange(32) - 16
    blocks["values"][1] = 3
    q = views.q8(blocks, 1, 64)
    h = ctypes.POINTER(ctypes.c_float)()
    assert lib.phonon_tensor_expand_linear(ctypes.byref(q), ctypes.byref(h))
    got = np.ctypeslib.as_array(h, shape=(64,))
    want = np.concatenate([(np.arange(32) - 16) * 0.5, np.full(32, -6.0)]).astype(np.float32)
    assert np.array_equal(got, want)


def test_prepare_linears_bounded_with_rollback(lib, pkg, tmp_path):
    """tests/test_phonon_pack.c:300-327: a limit that fails after one
    expansion keeps none; the real call materializes (values 1), is
    idempotent, and each pack owns its own materialization."""
    path = write(tmp_path, helpers.kpack_bytes(helpers.kpack_synthetic()))
    ok, pack = opened(lib, path)
    assert ok
    v = pkg.PhononTensorView()
    assert lib.phonon_pack_tensor(pack, b"flow_lm.fixture_000.weight", ctypes.byref(v))
    data_before = v.data
    assert not v.linear_data
    assert not lib.phonon_pack_prepare_linears_for_tests(pack, 32 * 4)
    assert lib.phonon_pack_tensor(pack, b"flow_lm.fixture_000.weight", ctypes.byref(v))
    assert not v.linear_data
    assert lib.phonon_pack_prepare_linears(pack)
    assert lib.phonon_pack_tensor(pack, b"flow_lm.fixture_000.weight", ctypes.byref(v))
    assert v.linear_data and v.data == data_before
    lin = ctypes.cast(v.linear_data, ctypes.POINTER(ctypes.c_float))
    assert all(lin[i] == 1.0 for i in range(32))
    first = ctypes.cast(v.linear_data, ctypes.c_void_p).value
    assert lib.phonon_pack_prepare_linears(pack)
    assert lib.phonon_pack_tensor(pack, b"flow_lm.fixture_000.weight", ctypes.byref(v))
    assert ctypes.cast(v.linear_data, ctypes.c_void_p).value == first
    ok, other = opened(lib, path)
    assert ok and lib.phonon_pack_prepare_linears(other)
    w = pkg.PhononTensorView()
    assert lib.phonon_pack_tensor(other, b"flow_lm.fixture_000.weight", ctypes.byref(w))
    assert ctypes.cast(w.linear_data, ctypes.c_void_p).value != first
    # rank-1 tensors are never materialized
    assert lib.phonon_pack_tensor(pack, b"mimi.fixture_100.weight", ctypes.byref(w))
    assert not w.linear_data
    lib.phonon_pack_close(other)
    lib.phonon_pack_close(pack)
    assert not lib.phonon_pack_prepare_linears(None)


# ----------------------------------------------- a model-shaped synthetic pack
def model_pack_tensors(syn, seed=404, vocab=48, factor=1.0):
    """A 209-tensor pack holding the nine Flow layers under their checkpoint
    names (36 Q8_0), their norms, the decoder's out_norm, input_linear,
    bos_emb, emb_mean/emb_std, a transcript embedding table, the flow head
    (the reference test's synthetic head, tests/test_phonon_sampler.c:104-180,
    68 tensors) and out_eos (BF16), filled up to 173 BF16 tensors with small
    vectors."""
    rng = np.random.default_rng(seed)
    model = helpers.scaled_model(syn, seed, 9, factor) if factor != 1.0 else syn.flow_model(seed, 9)
    t = []
    names = {"qkv": "self_attn.in_proj.weight", "out": "self_attn.out_proj.weight",
             "mlp_in": "linear1.weight", "mlp_out": "linear2.weight"}
    for l, layer in enumerate(model):
        for key, suffix in names.items():
            r, c = helpers.SHAPES[key]
            t.append((f"flow_lm.transformer.layers.{l}.{suffix}", helpers.KPACK_Q8, (r, c),
                      layer[key].tobytes()))
    extra = {}
    for l, layer in enumerate(model):
        for key in ("norm1_weight", "norm1_bias", "norm2_weight", "norm2_bias"):
            t.append((f"flow_lm.transformer.layers.{l}.{key.replace('_', '.')}",
                      helpers.KPACK_BF16, (512,), layer[key].tobytes()))
    bf = lambda a: syn.bf16_bits(np.asarray(a, np.float32))  # noqa: E731
    extra["flow_lm.out_norm.weight"] = ((512,), bf(1 + 0.1 * rng.standard_normal(512)))
    extra["flow_lm.out_norm.bias"] = ((512,), bf(0.1 * rng.standard_normal(512)))
    extra["flow_lm.input_linear.weight"] = ((512, 32), bf(0.2 * rng.standard_normal((512, 32))))
    extra["flow_lm.bos_emb"] = ((32,), bf(rng.standard_normal(32)))
    extra["flow_lm.emb_mean"] = ((32,), bf(rng.standard_normal(32)))
    extra["flow_lm.emb_std"] = ((32,), bf(rng.uniform(0.5, 2.0, 32)))
    extra["flow_lm.condition_provider.conditioners.transcript_in_segment.embed.weight"] = (
        (vocab, 512), bf(rng.standard_normal((vocab, 512))))
    extra["flow_lm.out_eos.weight"] = ((1, 512), bf(0.05 * rng.standard_normal((1, 512))))
    extra["flow_lm.out_eos.bias"] = ((1,), bf([0.125]))
    names = helpers.flow_head_checkpoint_names()
    for key, bits in helpers.reference_flow_head_bits().items():
        extra[names[key]] = (bits.shape, bits)
    for name, (shape, bits) in extra.items():
        t.append((name, helpers.KPACK_BF16, shape, bits.tobytes()))
    i = 0
    while len(t) < 209:
        t.append((f"mimi.filler_{i:03d}.weight", helpers.KPACK_BF16, (4,),
                  bf(rng.standard_normal(4)).tobytes()))
        i += 1
    return model, {k: v[1] for k, v in extra.items()}, t


@pytest.fixture(scope="module")
def model_pack(syn, tmp_path_factory):
    model, extra, tensors = model_pack_tensors(syn)
    path = tmp_path_factory.mktemp("kpack") / "model.kpack"
    path.write_bytes(helpers.kpack_bytes(tensors))
    return model, extra, str(path).encode()


def test_load_layers_gives_the_checkpoint_views(lib, pkg, model_pack):
    model, _, path = model_pack
    ok, pack = opened(lib, path)
    assert ok
    storage = (pkg.PhononTensorView * (9 * 8))()
    weights = (pkg.PhononFlowLayerWeights * 9)()
    assert lib.phonon_flow_load_layers(pack, storage, weights)
    for l in range(9):
        w = weights[l]
        qkv = w.qkv.contents
        assert qkv.dtype == 1 and list(qkv.shape[:2]) == [1536, 512]
        assert ctypes.string_at(qkv.data, qkv.byte_count) == model[l]["qkv"].tobytes()
        mo = w.mlp_out.contents
        assert list(mo.shape[:2]) == [512, 2048]
        assert ctypes.string_at(mo.data, mo.byte_count) == model[l]["mlp_out"].tobytes()
        n2 = w.norm2_bias.contents
        assert ctypes.string_at(n2.data, 1024) == model[l]["norm2_bias"].tobytes()
    # A pack without the layers fails.
    ok, other = opened(lib, path)
    lib.phonon_pack_close(pack)
    lib.phonon_pack_close(other)


def test_pack_helpers_without_the_device(lib, pkg, syn, model_pack):
    """embed_tokens (table rows), normalize_latent ((x - mean) / std per
    channel) and prepare_prefix (voice rows for prompt ids, the BOS row,
    token rows otherwise), against numpy; bad ids and counts rejected."""
    _, extra, path = model_pack
    ok, pack = opened(lib, path)
    assert ok
    f32 = lambda a: a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))  # noqa: E731
    i32 = lambda a: a.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))  # noqa: E731
    table = syn.bf16_to_f32(extra["flow_lm.condition_provider.conditioners."
                                  "transcript_in_segment.embed.weight"]).reshape(48, 512)
    ids = np.array([3, 0, 47, 3], np.int32)
    emb = np.zeros((4, 512), np.float32)
    assert lib.phonon_flow_embed_tokens(pack, i32(ids), 4, f32(emb))
    assert np.array_equal(emb, table[ids])
    assert not lib.phonon_flow_embed_tokens(pack, i32(np.array([48], np.int32)), 1, f32(emb))
    assert not lib.phonon_flow_embed_tokens(pack, i32(np.array([-1], np.int32)), 1, f32(emb))
    mean = syn.bf16_to_f32(extra["flow_lm.emb_mean"])
    std = syn.bf16_to_f32(extra["flow_lm.emb_std"])
    x = np.random.default_rng(5).standard_normal(32).astype(np.float32)
    y = np.zeros(32, np.float32)
    assert lib.phonon_flow_normalize_latent(pack, f32(x), f32(y))
    assert np.array_equal(y, ((x - mean) / std).astype(np.float32))
    x[3] = np.nan
    assert not lib.phonon_flow_normalize_latent(pack, f32(x), f32(y))
    lib.phonon_pack_close(pack)
    # prepare_prefix: ids 7 = prompt, 9 = bos
    rng = np.random.default_rng(6)
    pid = np.array([1, 7, 7, 9, 2], np.int32)
    tok = rng.standard_normal((5, 512)).astype(np.float32)
    voice = rng.standard_normal((2, 512)).astype(np.float32)
    bos = rng.standard_normal(512).astype(np.float32)
    out = np.zeros((5, 512), np.float32)
    assert lib.phonon_flow_prepare_prefix(i32(pid), 5, f32(tok), 7, 9, f32(voice), 2, f32(bos),
                                          f32(out))
    want = np.stack([tok[0], voice[0], voice[1], bos, tok[4]])
    assert np.array_equal(out, want)
    assert not lib.phonon_flow_prepare_prefix(i32(pid), 5, f32(tok), 7, 9, f32(voice), 1,
                                              f32(bos), f32(out))   # 2 prompts, 1 voice frame
    two_bos = np.array([9, 7, 7, 9, 2], np.int32)
    assert not lib.phonon_flow_prepare_prefix(i32(two_bos), 5, f32(tok), 7, 9, f32(voice), 2,
                                              f32(bos), f32(out))


def test_flow_head_load_gives_the_checkpoint_views(lib, pkg, syn, model_pack, tmp_path):
    """phonon_flow_head_load fills every PhononFlowHead view with its
    checkpoint tensor (bytes and shapes), and fails when a tensor is missing
    or has another shape."""
    _, extra, path = model_pack
    ok, pack = opened(lib, path)
    assert ok
    head = pkg.PhononFlowHead()
    assert lib.phonon_flow_head_load(pack, ctypes.byref(head))
    names = helpers.flow_head_checkpoint_names()
    bits = helpers.reference_flow_head_bits()

    def view(key):
        parts = key.split("_")
        if key.startswith(("time_weight", "time_bias", "block_mlp")):
            field = "_".join(parts[:-2])
            return getattr(head, field)[int(parts[-2])][int(parts[-1])]
        if key.startswith(("time_freqs", "time_alpha", "block_")):
            return getattr(head, "_".join(parts[:-1]))[int(parts[-1])]
        return getattr(head, key)

    for key, want in bits.items():
        v = view(key)
        assert v.dtype == 2 and list(v.shape[:v.rank]) == list(want.shape), key
        assert ctypes.string_at(v.data, v.byte_count) == want.tobytes(), key
    lib.phonon_pack_close(pack)
    assert not lib.phonon_flow_head_load(None, ctypes.byref(head))

    # A missing tensor, or one of another shape: the load fails.
    model, _, tensors = model_pack_tensors(syn)
    for mutate in ("missing", "shape"):
        bad = []
        for name, dtype, shape, data in tensors:
            if name == names["time_freqs_1"]:
                if mutate == "missing":
                    name = "flow_lm.flow_net.time_embed.1.freq"
                else:
                    shape, data = (127,), data[:254]
            bad.append((name, dtype, shape, data))
        p = tmp_path / f"{mutate}.kpack"
        p.write_bytes(helpers.kpack_bytes(bad))
        ok, other = opened(lib, str(p).encode())
        assert ok, mutate
        assert not lib.phonon_flow_head_load(other, ctypes.byref(head)), mutate
        lib.phonon_pack_close(other)


def test_denormalize_latent_without_the_device(lib, pkg, syn, model_pack):
    """x * emb_std + emb_mean per channel, as float32 rounds it (two
    operations, no contraction); a non-finite result fails."""
    _, extra, path = model_pack
    ok, pack = opened(lib, path)
    assert ok
    f32 = lambda a: a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))  # noqa: E731
    mean = syn.bf16_to_f32(extra["flow_lm.emb_mean"])
    std = syn.bf16_to_f32(extra["flow_lm.emb_std"])
    x = np.random.default_rng(7).standard_normal(32).astype(np.float32)
    y = np.zeros(32, np.float32)
    assert lib.phonon_flow_denormalize_latent(pack, f32(x), f32(y))
    assert np.array_equal(y, (x * std).astype(np.float32) + mean)
    # normalize then denormalize: back within a few ulps
    z = np.zeros(32, np.float32)
    assert lib.phonon_flow_normalize_latent(pack, f32(y), f32(z))
    np.testing.assert_allclose(z, x, rtol=1e-6, atol=1e-6)
    x[5] = np.inf
    assert not lib.phonon_flow_denormalize_latent(pack, f32(x), f32(y))
    assert not lib.phonon_flow_denormalize_latent(None, f32(x), f32(y))
    lib.phonon_pack_close(pack)
