"""Shared test plumbing: imports of the product package (by path) and of the
CPU oracle, and conversions of synthetic weights for the oracle."""
from __future__ import annotations

import importlib.util
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "speech-mac_amd")
ORACLE_DIR = os.path.join(ROOT, "oracle")
GOLDEN_DIR = os.path.join(ROOT, "tests", "golden")


def package():
    if "speech_mac_amd" in sys.modules:
        return sys.modules["speech_mac_amd"]
    spec = importlib.util.spec_from_file_location(
        "speech_mac_amd", os.path.join(PKG_DIR, "__init__.py"),
        submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["speech_mac_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def synthetic():
    package()
    import speech_mac_amd.synthetic as syn  # noqa: E402
    return syn


def oracle_module():
    if ORACLE_DIR not in sys.path:
        sys.path.insert(0, ORACLE_DIR)
    import oracle_py  # noqa: E402
    return oracle_py


SHAPES = {"qkv": (1536, 512), "out": (512, 512), "mlp_in": (2048, 512), "mlp_out": (512, 2048)}


def oracle_layers(oracle, model):
    """Synthetic layer dicts -> fp32 expansions made by the oracle's own
    restatement of the reference expansion (src/phonon_pack.c:372-411)."""
    pkg = package()
    out = []
    for layer in model:
        d = {}
        for name, (r, c) in SHAPES.items():
            w = layer[name]
            if w.dtype == pkg.Q8_BLOCK:
                ok, e = oracle.q8_expand(w, r, c)
                assert ok
            else:
                ok, e = oracle.bf16_to_float(w.reshape(-1))
                assert ok
                e = e.reshape(r, c)
            d[name] = e
        for k in ("norm1_weight", "norm1_bias", "norm2_weight", "norm2_bias"):
            ok, d[k] = oracle.bf16_to_float(layer[k])
            assert ok
        out.append(d)
    return out


def normwise(a, b) -> float:
    """max|a-b| / max|b| (the parity metric; 0 when both are zero)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    scale = np.max(np.abs(b))
    err = np.max(np.abs(a - b))
    return float(err / scale) if scale > 0 else float(err)


def elementwise_ok(a, b, atol=1e-5, rtol=1e-3) -> bool:
    """The reference's own gate |a-b| <= 1e-5 + 1e-3|b| (tests/test_phonon_pack.c:446)."""
    return bool(np.all(np.abs(np.asarray(a, np.float64) - b) <= atol + rtol * np.abs(b)))
