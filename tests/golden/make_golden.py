"""Writes the golden fixtures of tests/golden/ (run in a tree that has the
reference at /root/reference and oracle/_ref built: `make -C oracle`).

reference_vectors.json
    Known answers the reference's own C tests hold for the decode-step
    functions, as data: expected bits/values, plus the 512 input floats of
    the LayerNorm bit regression (tests/phonon_layer_norm_regression.inc).
q8_reference_vectors.npz
    phonon_q8_matvec outputs of the reference's own src/phonon_q8.c,
    compiled from its source into oracle/_ref/libref_q8.so (gcc -std=c17 -O2
    -ffp-contract=off), on seeded synthetic matrices.
"""
from __future__ import annotations

import json
import os
import re
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REFERENCE = "/root/reference"
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

import helpers  # noqa: E402
import oracle_py  # noqa: E402


def hexf(s: str) -> float:
    return float.fromhex(s)


def f32_bits(x: float) -> int:
    return int(np.array([x], np.float32).view(np.uint32)[0])


def layer_norm_input_bits() -> list:
    path = os.path.join(REFERENCE, "tests", "phonon_layer_norm_regression.inc")
    text = open(path).read()
    body = text[text.index("{") + 1: text.rindex("}")]
    bits = [int(h, 16) for h in re.findall(r"0x([0-9a-fA-F]{8})U", body)]
    assert len(bits) == 512
    return bits


def reference_vectors() -> dict:
    return {
        "layer_norm_regression": {
            "source": "tests/phonon_layer_norm_regression.inc:7-71; tests/test_speech.c:108-119",
            "input_bits": layer_norm_input_bits(),
            "weight": 1.0, "bias": 0.0, "epsilon": 1e-5,
            "expected_first_bits": 0x3F31CD52,
        },
        "attention_cases": {
            "source": "tests/test_speech.c:120-168 (query[0]=8, k[0]=2, k[n-1]=tail, "
                      "k[512]=middle, v[0]=v[n-1]=0.01, stride 64)",
            "cases": [
                {"count": 513, "middle": 0, "tail": 1, "expected_bits": 0x394B6175},
                {"count": 513, "middle": 0, "tail": 3, "expected_bits": 0x3A05C0FA},
                {"count": 1025, "middle": 3, "tail": 1, "expected_bits": 0x38C973B4},
                {"count": 1025, "middle": 1, "tail": 1, "expected_bits": 0x38CCD53A},
                {"count": 1537, "middle": 3, "tail": 1, "expected_bits": 0x388782FA},
            ],
        },
        "gelu": {
            "source": "tests/test_phonon_transformer.c:552-563",
            "closed_form": {"inputs": [-1.0, 0.0, 1.0],
                            "expected": [-0.15865526, 0.0, 0.8413447], "tolerance": 1e-6},
            "inputs": [-1.2345, 0.12345, 2.34567, -0.75, 1.0, -1.0, 0.0, 0.5, 0.25],
            "expected_bits": [f32_bits(hexf(s)) for s in (
                "-0x1.125648p-3", "0x1.15aa60p-4", "0x1.2964fep+1", "-0x1.5c197ap-3",
                "0x1.aec4bcp-1", "-0x1.44ed10p-3", "0x0p+0", "0x1.62075cp-2", "0x1.3289a2p-3")],
        },
        "rope": {
            "source": "tests/test_phonon_transformer.c:564-584",
            "head_width": 64, "theta": 10000.0, "pair_in": [1.0, -0.5], "pair_index": 1,
            "positions": [1, 139, 8191],
            "expected": [[1.072541714, 0.315680861], [-1.112550020, -0.110599607],
                         [-1.111756921, -0.118306905]],
            "tolerance": 3e-7,
        },
        "sincos_sleef": {
            "source": "tests/test_phonon_math.c:30-44 (pinned Torch/SLEEF u10 values; "
                      "the host RoPE table uses libm, compared within 1 ulp)",
            "phases": [hexf(s) for s in (
                "-0x1.ff7p+2", "-0x1.ff9cp+2", "0x1p+0", "-0x1p-1", "0x1.fffp+12",
                "0x1.0624dep-10", "0x1.4p+3", "-0x1.9p+6", "0x1.f9a6b6p-4")],
            "cos": [hexf(s) for s in (
                "-0x1.182a12p-3", "-0x1.1d9c92p-3", "0x1.14a282p-1", "0x1.c1528p-1",
                "-0x1.4af3b2p-1", "0x1.fffffp-1", "-0x1.ad9ac8p-1", "0x1.b981dcp-1",
                "0x1.fc1a82p-1")],
            "sin": [hexf(s) for s in (
                "-0x1.fb2fc6p-1", "-0x1.faff26p-1", "0x1.aed548p-1", "-0x1.eaee88p-2",
                "-0x1.86a8d4p-1", "0x1.0624dcp-10", "-0x1.1689fp-1", "0x1.03425cp-1",
                "0x1.f85e2cp-4")],
        },
        "q8_known": {
            "source": "tests/test_phonon_q8.c:9-56",
            "dot_two_blocks": 56.0, "matvec_rows": [56.0, 56.0],
            "asymmetric_rows": [272.0, 368.0], "subnormal_scale_dot": hexf("0x1p-19"),
        },
        "linear_bf16": {
            "source": "tests/test_phonon_transformer.c:603-607",
            "weight_bits": [0x3F80, 0xC000, 0x4000, 0x3F00], "shape": [2, 2],
            "input": [3.0, 2.0], "expected": [-1.0, 7.0],
        },
        "linear_q8_scales": {
            "source": "tests/test_phonon_transformer.c:641-650",
            "scale_bits": [0x0001, 0x8000], "expected": [hexf("0x1p-19"), 0.0],
            "rejected_scale_bits": [0x7C00, 0x7E00],
        },
        "kv_layout": {
            "source": "tests/test_phonon_transformer.c:586-607",
            "capacity": 2, "layer": 8, "position": 1, "probe_column": 7,
        },
        "flow_head_synthetic": {
            "source": "tests/test_phonon_sampler.c:104-195 (the synthetic BF16 head that "
                      "tests/helpers.py reference_flow_head_bits rebuilds; condition[i] = "
                      "((7i mod 13) - 6) / 8, state[i] = ((11i + 3 mod 17) - 8) / 16; "
                      "s = 0, t = 1; expected from an independent PyTorch 2.7.1 run)",
            "s": 0.0, "t": 1.0, "tolerance": 2e-4,
            "expected": [
                6.749069214, -2.760953903, -6.280110359, 1.966097355, 3.173623323,
                -1.909553528, -0.930359602, 6.741256714, -2.768766403, -6.287922859,
                1.958284855, 3.165810823, -1.917366028, -0.852234602, 6.733444214,
                -2.776578903, -6.295735359, 1.950472355, 3.157998323, -1.925178528,
                -0.860047102, 6.725631714, -2.784391403, -6.303547859, 2.028597355,
                3.150185823, -1.932991028, -0.867859602, 6.717819214, -2.792203903,
                -6.311360359, 2.020784855],
        },
    }


def q8_vectors(ref) -> dict:
    syn = helpers.synthetic()
    out = {}
    # Config of the matvec benchmark: 2048 x 512, seed 1. Inputs regenerate
    # from the seed (numpy PCG64); their SHA-256 is stored to detect drift.
    import hashlib
    rng = np.random.default_rng(1)
    w = syn.q8_matrix(rng, 2048, 512)
    x = rng.standard_normal(512).astype(np.float32)
    ok, y = ref.q8_matvec(w, x, 2048, 512)
    assert ok
    out["full_seed"] = np.array([1])
    out["full_sha256_w"] = np.frombuffer(hashlib.sha256(w.tobytes()).digest(), np.uint8)
    out["full_sha256_x"] = np.frombuffer(hashlib.sha256(x.tobytes()).digest(), np.uint8)
    out["full_y"] = y
    # A small case with inputs committed, including large dynamic range.
    rng = np.random.default_rng(7)
    w = syn.q8_matrix(rng, 64, 512)
    x = (rng.standard_normal(512) * np.exp(rng.uniform(-6, 6, 512))).astype(np.float32)
    ok, y = ref.q8_matvec(w, x, 64, 512)
    assert ok
    out["small_blocks"] = w.view(np.uint8)
    out["small_x"] = x
    out["small_y"] = y
    return out


def main():
    with open(os.path.join(HERE, "reference_vectors.json"), "w") as f:
        json.dump(reference_vectors(), f, indent=1)
    if "--json-only" not in sys.argv:
        ref = oracle_py.ReferenceQ8()
        np.savez(os.path.join(HERE, "q8_reference_vectors.npz"), **q8_vectors(ref))
    print("wrote", os.listdir(HERE))


if __name__ == "__main__":
    main()
