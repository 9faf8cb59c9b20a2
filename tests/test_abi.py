"""CPU checks of the C-ABI boundary: the library loads without a GPU, exports
every function include/*.h declares, keeps the reference's struct layouts,
and the Python binding declares exactly those functions."""
import ctypes
import os
import re
import subprocess

import helpers

INCLUDE = os.path.join(helpers.ROOT, "include")


def declared_functions():
    names = set()
    for header in sorted(os.listdir(INCLUDE)):
        text = open(os.path.join(INCLUDE, header)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"typedef[^;]*;", "", text)
        for m in re.finditer(r"\b([a-z_][a-z0-9_]*)\s*\(", text):
            name = m.group(1)
            if name.startswith(("phonon_", "pgpu_")):
                names.add(name)
    return names


def test_headers_declare_the_reference_entry_points():
    names = declared_functions()
    # src/phonon_q8.h:19-21 and the decode-step part of src/phonon_transformer.h:33-73
    for n in ("phonon_q8_dot", "phonon_q8_matvec", "phonon_kv_cache_init",
              "phonon_kv_cache_reset", "phonon_kv_cache_destroy", "phonon_kv_cache_append",
              "phonon_kv_cache_commit_position", "phonon_rms_norm", "phonon_layer_norm",
              "phonon_erf_gelu", "phonon_rope_interleaved", "phonon_linear",
              "phonon_linear_batch", "phonon_flow_layer_step", "phonon_flow_stack_step",
              "phonon_flow_stack_step_cancel", "phonon_flow_stack_prefill",
              "phonon_flow_stack_prefill_cancel", "phonon_attention_test",
              # src/phonon_mimi.h:27-46, src/phonon_conv.h:11-44, src/phonon_pcm.h:10-36
              "phonon_mimi_config", "phonon_mimi_model_load", "phonon_mimi_state_create",
              "phonon_mimi_state_reset", "phonon_mimi_state_destroy", "phonon_mimi_positions",
              "phonon_mimi_process", "phonon_mimi_upsample_frame", "phonon_conv_model_create",
              "phonon_conv_model_destroy", "phonon_conv_input_channels",
              "phonon_conv_output_channels", "phonon_conv_stride", "phonon_conv_state_create",
              "phonon_conv_state_destroy", "phonon_conv_state_reset", "phonon_conv_process",
              "phonon_conv_elu", "phonon_residual_state_create",
              "phonon_residual_state_destroy", "phonon_residual_state_reset",
              "phonon_residual_process", "phonon_pcm_model_create", "phonon_pcm_model_destroy",
              "phonon_pcm_state_create", "phonon_pcm_state_destroy", "phonon_pcm_state_reset",
              "phonon_pcm_samples", "phonon_pcm_process", "phonon_pcm_finish"):
        assert n in names, n


def test_library_exports_every_declared_symbol(pkg):
    lib = pkg.load()
    names = declared_functions()
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing
    assert set(pkg.EXPORTS) == names, (set(pkg.EXPORTS) ^ names)
    out = subprocess.run(["nm", "-D", "--defined-only", pkg.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert names <= exported


def test_struct_layouts_match_the_reference(pkg):
    # PhononQ8Block is 34 packed bytes (src/phonon_q8.h:17).
    assert pkg.Q8_BLOCK.itemsize == 34
    # PhononKvCache / PhononTensorView / PhononFlowLayerWeights keep the
    # reference field order (src/phonon_transformer.h:16-31, src/phonon_pack.h:10-19).
    assert ctypes.sizeof(pkg.PhononKvCache) == 32
    assert pkg.PhononTensorView.data.offset == 8 + 64
    assert ctypes.sizeof(pkg.PhononFlowLayerWeights) == 64
    # PhononFlowHead: 68 PhononTensorView (96 B each) in the reference's field
    # order (src/phonon_sampler.h:51-60).
    assert ctypes.sizeof(pkg.PhononTensorView) == 96
    assert ctypes.sizeof(pkg.PhononFlowHead) == 68 * 96
    assert pkg.PhononFlowHead.block_ada_weight.offset == 16 * 96
    assert pkg.PhononFlowHead.final_ada_weight.offset == 64 * 96
    # PhononMimiConfig {unsigned, float, unsigned[3], size_t, float} and
    # PhononMimiModel {config, size_t stride, 2 views, 2 x 10 views}
    # (src/phonon_mimi.h:10-24) on LP64.
    assert ctypes.sizeof(pkg.PhononMimiConfig) == 40
    assert pkg.PhononMimiConfig.context.offset == 24
    assert pkg.PhononMimiConfig.rope_theta.offset == 32
    assert pkg.PhononMimiModel.stride.offset == 40
    assert pkg.PhononMimiModel.projection.offset == 48
    assert pkg.PhononMimiModel.layers.offset == 48 + 2 * 96
    assert ctypes.sizeof(pkg.PhononMimiModel) == 48 + 22 * 96


def test_c_layouts_of_the_audio_headers(tmp_path):
    """The C compiler's layout of include/phonon_mimi.h agrees with the
    reference's field order (checked by static assertions)."""
    src = tmp_path / "mimi.c"
    src.write_text(
        '#include <stddef.h>\n#include "phonon_pcm.h"\n'
        '_Static_assert(sizeof(PhononMimiConfig) == 40, "config");\n'
        '_Static_assert(offsetof(PhononMimiConfig, context) == 24, "context");\n'
        '_Static_assert(offsetof(PhononMimiModel, stride) == 40, "stride");\n'
        '_Static_assert(offsetof(PhononMimiModel, layers) == 48 + 2 * 96, "layers");\n'
        '_Static_assert(sizeof(PhononMimiModel) == 48 + 22 * 96, "model");\n'
        'int main(void){return 0;}\n')
    subprocess.run(["gcc", "-std=c17", "-Wall", "-Wextra", "-Wpedantic", "-Werror",
                    "-I", INCLUDE, "-fsyntax-only", str(src)], check=True)


def test_library_has_no_cpu_compute_symbols(pkg):
    """The product links no oracle code (no oracle_* symbols) and no BLAS."""
    out = subprocess.run(["nm", "-D", pkg.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    assert "oracle_" not in out
    assert "cblas" not in out and "sgemm" not in out


def test_c_header_compiles_as_c17(tmp_path):
    src = tmp_path / "use.c"
    src.write_text('#include "phonon_flow_batch.h"\n#include "phonon_q8_device.h"\n'
                   '#include "phonon_gpu.h"\nint main(void){return 0;}\n')
    subprocess.run(["gcc", "-std=c17", "-Wall", "-Wextra", "-Wpedantic", "-Werror",
                    "-I", INCLUDE, "-fsyntax-only", str(src)], check=True)
