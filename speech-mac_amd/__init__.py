"""speech-mac Flow-transformer decode step on the MI355X.

Python binding (ctypes) of libphonon_mi355x.so, the C-ABI library built from
csrc/ (gfx950 HIP kernels) and host/ (C17 host layer). The numerical work
always runs in that library on the GPU; this module only declares the C
signatures and moves numpy arrays in and out. It never computes results
itself and has no CPU fallback: loading fails loudly when the library is
missing.

The directory name is not an identifier, so import it by path::

    spec = importlib.util.spec_from_file_location(
        "speech_mac_amd", "speech-mac_amd/__init__.py",
        submodule_search_locations=["speech-mac_amd"])
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libphonon_mi355x.so")
INCLUDE_DIR = os.path.join(os.path.dirname(HERE), "include")

WIDTH, HEADS, HEAD_DIM, FFN = 512, 8, 64, 2048
REFERENCE_LAYERS = 9
BLOCK_POSITIONS = 16
MAX_POSITIONS = 8192
PACK_Q8_0, PACK_BF16 = 1, 2

Q8_BLOCK = np.dtype([("scale_bits", "<u2"), ("values", "i1", (32,))], align=False)
assert Q8_BLOCK.itemsize == 34


def build(jobs: int = 8) -> None:
    """Compile every HIP and C source of the library for gfx950 (always)."""
    subprocess.run(["make", "-s", "-B", "-C", HERE, f"-j{jobs}"], check=True)


# --------------------------------------------------------------------- C types
_sz = ctypes.c_size_t
_i = ctypes.c_int
_vp = ctypes.c_void_p
_f = ctypes.c_float
_fp = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)
_szp = ctypes.POINTER(ctypes.c_size_t)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_ip = ctypes.POINTER(ctypes.c_int)


class PhononTensorView(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int), ("rank", ctypes.c_uint),
                ("shape", ctypes.c_uint64 * 8), ("data", _vp),
                ("byte_count", _sz), ("linear_data", _vp)]


class PhononFlowLayerWeights(ctypes.Structure):
    _fields_ = [(n, ctypes.POINTER(PhononTensorView)) for n in (
        "qkv", "attention_out", "mlp_in", "mlp_out",
        "norm1_weight", "norm1_bias", "norm2_weight", "norm2_bias")]


HEAD_BLOCKS = 6
_TV = PhononTensorView


class PhononFlowHead(ctypes.Structure):
    """PhononFlowHead (phonon_sampler.h, src/phonon_sampler.h:48-60)."""
    _fields_ = [("input_weight", _TV), ("input_bias", _TV), ("cond_weight", _TV),
                ("cond_bias", _TV), ("time_weight", (_TV * 2) * 2), ("time_bias", (_TV * 2) * 2),
                ("time_freqs", _TV * 2), ("time_alpha", _TV * 2),
                ("block_ada_weight", _TV * HEAD_BLOCKS), ("block_ada_bias", _TV * HEAD_BLOCKS),
                ("block_norm_weight", _TV * HEAD_BLOCKS), ("block_norm_bias", _TV * HEAD_BLOCKS),
                ("block_mlp_weight", (_TV * 2) * HEAD_BLOCKS),
                ("block_mlp_bias", (_TV * 2) * HEAD_BLOCKS),
                ("final_ada_weight", _TV), ("final_ada_bias", _TV), ("final_weight", _TV),
                ("final_bias", _TV)]


class PhononKvCache(ctypes.Structure):
    _fields_ = [("capacity", _sz), ("length", _sz), ("keys", _fp), ("values", _fp)]


class PgpuMatrix(ctypes.Structure):
    _fields_ = [("q8", _i), ("rows", _sz), ("columns", _sz), ("values", _vp), ("scales", _vp)]


class PgpuPagedKv(ctypes.Structure):
    _fields_ = [("base", _vp), ("layers", _i), ("blocks", _sz), ("layer_stride", _sz)]


class PgpuAttentionScratch(ctypes.Structure):
    _fields_ = [("part_acc", _vp), ("part_ml", _vp), ("max_streams", _i), ("max_splits", _i)]


class PgpuGemmInput(ctypes.Structure):
    _fields_ = [("split", _vp), ("ln_rows", _vp), ("ln_weight", _vp), ("ln_bias", _vp),
                ("ln_epsilon", _f), ("attn_acc", _vp), ("attn_ml", _vp),
                ("attn_positions", _vp), ("attn_max_splits", _i), ("rows", _vp)]


class PgpuConvLayer(ctypes.Structure):
    """pgpu_conv_layer (phonon_gpu.h)."""
    _fields_ = [("cin", _i), ("cout", _i), ("kernel", _i), ("stride", _i), ("transpose", _i),
                ("taps", _i), ("ncols", _i), ("fragments", _vp), ("weight", _vp), ("bias", _vp)]


class PhononMimiConfig(ctypes.Structure):
    """PhononMimiConfig (phonon_mimi.h, src/phonon_mimi.h:10-16)."""
    _fields_ = [("sample_rate", ctypes.c_uint), ("frame_rate", _f),
                ("ratios", ctypes.c_uint * 3), ("context", _sz), ("rope_theta", _f)]


class PhononMimiModel(ctypes.Structure):
    """PhononMimiModel (phonon_mimi.h, src/phonon_mimi.h:17-24)."""
    _fields_ = [("config", PhononMimiConfig), ("stride", _sz), ("projection", _TV),
                ("upsample", _TV), ("layers", (_TV * 10) * 2)]


CANCEL_POLL = ctypes.CFUNCTYPE(ctypes.c_int, _vp)
_wp = ctypes.POINTER(PhononFlowLayerWeights)
_cachep = ctypes.POINTER(PhononKvCache)
_viewp = ctypes.POINTER(PhononTensorView)
_mp = ctypes.POINTER(PgpuMatrix)
_kvp = ctypes.POINTER(PgpuPagedKv)
_scp = ctypes.POINTER(PgpuAttentionScratch)
_gip = ctypes.POINTER(PgpuGemmInput)
_pp = ctypes.POINTER(_vp)

# Every function declared in include/*.h: name -> (restype, argtypes).
EXPORTS = {
    # phonon_q8.h
    "phonon_q8_dot": (_i, [_vp, _fp, _sz, _fp]),
    "phonon_q8_matvec": (_i, [_vp, _fp, _sz, _sz, _fp]),
    # phonon_q8_device.h
    "phonon_q8_device_create": (_i, [_vp, _sz, _sz, _sz, _pp]),
    "phonon_q8_device_destroy": (None, [_vp]),
    "phonon_q8_device_matvec": (_i, [_vp, _sz, _vp, _vp, _sz, _vp]),
    "phonon_q8_device_status": (_i, [_vp, _vp]),
    "phonon_q8_device_bytes_per_call": (_sz, [_vp, _sz]),
    # phonon_transformer.h
    "phonon_kv_cache_init": (_i, [_cachep, _sz]),
    "phonon_kv_cache_reset": (None, [_cachep]),
    "phonon_kv_cache_destroy": (None, [_cachep]),
    "phonon_kv_cache_append": (_i, [_cachep, _sz, _sz, _fp, _fp, _sz]),
    "phonon_kv_cache_commit_position": (_i, [_cachep, _sz]),
    "phonon_rms_norm": (_i, [_fp, _fp, _sz, _f, _fp]),
    "phonon_layer_norm": (_i, [_fp, _fp, _fp, _sz, _f, _fp]),
    "phonon_erf_gelu": (_i, [_fp, _sz]),
    "phonon_rope_interleaved": (_i, [_fp, _sz, _sz, _sz, _f]),
    "phonon_linear": (_i, [_viewp, _fp, _sz, _sz, _fp, _fp]),
    "phonon_linear_batch": (_i, [_viewp, _fp, _sz, _sz, _fp, _fp, _sz]),
    "phonon_flow_layer_step": (_i, [_wp, _cachep, _sz, _sz, _fp, _f, _fp]),
    "phonon_flow_stack_step": (_i, [_wp, _cachep, _sz, _fp, _f, _fp]),
    "phonon_flow_stack_step_cancel": (_i, [_wp, _cachep, _sz, _fp, _f, _fp, CANCEL_POLL, _vp]),
    "phonon_flow_stack_prefill_cancel": (_i, [_wp, _cachep, _fp, _sz, _f, _fp, CANCEL_POLL,
                                              _vp]),
    "phonon_flow_stack_prefill": (_i, [_wp, _cachep, _fp, _sz, _f, _fp]),
    "phonon_attention_test": (_i, [_fp, _fp, _fp, _sz, _sz, _fp]),
    "phonon_voice_project": (_i, [_fp, _sz, _viewp, _fp]),
    "phonon_flow_condition": (_i, [_viewp, _viewp, _viewp, _sz, _f, _fp]),
    "phonon_flow_prepare_prefix": (_i, [_i32p, _sz, _fp, _sz, _sz, _fp, _sz, _fp, _fp]),
    "phonon_flow_load_layers": (_i, [_vp, _vp, _vp]),
    "phonon_flow_embed_tokens": (_i, [_vp, _i32p, _sz, _fp]),
    "phonon_flow_embed_bos": (_i, [_vp, _fp, _fp]),
    "phonon_flow_embed_latent": (_i, [_vp, _fp, _fp, _fp]),
    "phonon_flow_normalize_latent": (_i, [_vp, _fp, _fp]),
    "phonon_flow_output_norm": (_i, [_vp, _fp]),
    # phonon_pack.h
    "phonon_pack_open": (_i, [ctypes.c_char_p, _pp]),
    "phonon_pack_open_for_tests": (_i, [ctypes.c_char_p, _pp]),
    "phonon_pack_close": (None, [_vp]),
    "phonon_pack_prepare_linears": (_i, [_vp]),
    "phonon_pack_prepare_linears_for_tests": (_i, [_vp, _sz]),
    "phonon_tensor_expand_linear": (_i, [_viewp, ctypes.POINTER(_fp)]),
    "phonon_pack_tensor_count": (_sz, [_vp]),
    "phonon_pack_tensor": (_i, [_vp, ctypes.c_char_p, _viewp]),
    "phonon_pack_tensor_at": (_i, [_vp, _sz, ctypes.POINTER(ctypes.c_char_p), _szp, _viewp]),
    "phonon_bf16_to_float": (_i, [_vp, _sz, _fp]),
    # phonon_flow_batch.h
    "phonon_flow_model_create": (_i, [_wp, _sz, _pp]),
    "phonon_flow_model_destroy": (None, [_vp]),
    "phonon_flow_model_layers": (_sz, [_vp]),
    "phonon_flow_model_device_bytes": (_sz, [_vp]),
    "phonon_kv_pool_create": (_i, [_sz, _sz, _pp]),
    "phonon_kv_pool_destroy": (None, [_vp]),
    "phonon_kv_pool_free_blocks": (_sz, [_vp]),
    "phonon_kv_pool_alloc": (_i, [_vp, _sz, _i32p]),
    "phonon_kv_pool_release": (_i, [_vp, _sz, _i32p]),
    "phonon_kv_pool_fill_normal": (_i, [_vp, ctypes.c_uint64]),
    "phonon_kv_pool_write": (_i, [_vp, _i32p, _sz, _sz, _sz, _fp, _fp, _sz]),
    "phonon_kv_pool_read": (_i, [_vp, _i32p, _sz, _sz, _sz, _fp, _fp, _sz]),
    "phonon_kv_pool_view": (_i, [_vp, _kvp]),
    "phonon_flow_batch_create": (_i, [_vp, _vp, _sz, _sz, _pp]),
    "phonon_flow_batch_destroy": (None, [_vp]),
    "phonon_flow_batch_set_streams": (_i, [_vp, _sz, _szp, _i32p, _sz]),
    "phonon_flow_batch_step": (_i, [_vp, _fp, _f, _fp]),
    "phonon_flow_batch_step_device": (_i, [_vp, _vp, _f, _vp]),
    "phonon_flow_batch_set_pipeline": (_i, [_vp, _i]),
    "phonon_flow_batch_set_trace": (_i, [_vp, _vp, _sz]),
    "phonon_flow_batch_set_placement": (_i, [_vp, _vp]),
    "phonon_flow_batch_schedule": (_sz, [_vp, ctypes.POINTER(ctypes.c_uint32), _sz]),
    "phonon_flow_batch_set_handoff": (_i, [_vp, _i]),
    "phonon_flow_batch_prefill_device": (_i, [_vp, _sz, _vp, _vp, _vp, _sz, _vp, _f, _vp]),
    "phonon_flow_batch_sync": (_i, [_vp]),
    "phonon_flow_batch_status": (_i, [_vp, _vp]),
    "phonon_flow_batch_set_groups": (_i, [_vp, _sz]),
    "phonon_flow_batch_set_graph": (_i, [_vp, _i]),
    "phonon_flow_batch_set_timing": (_i, [_vp, _vp, _vp]),
    "phonon_flow_batch_set_attention_rounds": (_i, [_vp, _i]),
    "phonon_flow_batch_positions": (_i, [_vp, _szp]),
    "phonon_flow_batch_stream": (_vp, [_vp]),
    "phonon_flow_batch_device_inputs": (_vp, [_vp]),
    "phonon_flow_batch_device_outputs": (_vp, [_vp]),
    "phonon_flow_prepare_weights": (_i, [_wp, _sz]),
    "phonon_flow_release_weights": (None, [_wp]),
    # phonon_gpu.h
    "pgpu_last_error": (ctypes.c_char_p, []),
    "pgpu_record_error": (None, [ctypes.c_char_p]),
    "pgpu_device_init": (_i, []),
    "pgpu_device_name": (_i, [ctypes.c_char_p, _sz]),
    "pgpu_malloc": (_vp, [_sz]),
    "pgpu_free": (None, [_vp]),
    "pgpu_memset": (_i, [_vp, _vp, _i, _sz]),
    "pgpu_copy_h2d": (_i, [_vp, _vp, _vp, _sz]),
    "pgpu_host_malloc": (_vp, [_sz]),
    "pgpu_host_free": (None, [_vp]),
    "pgpu_copy_h2d_async": (_i, [_vp, _vp, _vp, _sz]),
    "pgpu_copy_d2h": (_i, [_vp, _vp, _vp, _sz]),
    "pgpu_copy_d2d": (_i, [_vp, _vp, _vp, _sz]),
    "pgpu_stream_create": (_i, [_pp]),
    "pgpu_stream_destroy": (None, [_vp]),
    "pgpu_stream_sync": (_i, [_vp]),
    "pgpu_event_create": (_i, [_pp]),
    "pgpu_event_destroy": (None, [_vp]),
    "pgpu_event_record": (_i, [_vp, _vp]),
    "pgpu_event_elapsed_ms": (_i, [_vp, _vp, _fp]),
    "pgpu_stream_wait_event": (_i, [_vp, _vp]),
    "pgpu_graph_begin": (_i, [_vp]),
    "pgpu_graph_begin_global": (_i, [_vp]),
    "pgpu_graph_end": (_i, [_vp, _pp]),
    "pgpu_graph_launch": (_i, [_vp, _vp]),
    "pgpu_graph_destroy": (None, [_vp]),
    "pgpu_check_launch": (_i, []),
    "pgpu_gemm_store": (_i, [_vp, _mp, _gip, _i, _vp, _vp, _i, _vp]),
    "pgpu_gemm_residual": (_i, [_vp, _mp, _gip, _i, _vp, _vp, _vp]),
    "pgpu_gemm_gelu_split": (_i, [_vp, _mp, _gip, _i, _vp, _vp]),
    "pgpu_gemm_qkv": (_i, [_vp, _mp, _gip, _i, _kvp, _i, _vp, _i, _vp, _vp, _vp, _vp]),
    "pgpu_attention": (_i, [_vp, _vp, _kvp, _i, _vp, _i, _vp, _i, _i, _i, _scp, _vp]),
    "pgpu_attention_merge": (_i, [_vp, _scp, _vp, _i, _i, _i, _vp, _vp, _vp]),
    "pgpu_rows_split_ln": (_i, [_vp, _vp, _vp, _vp, ctypes.c_float, _i, _i, _vp, _vp]),
    "pgpu_rows_split_attention": (_i, [_vp, _scp, _vp, _i, _i, _vp, _vp]),
    "pgpu_wide_from_matrix": (_i, [_vp, _mp, _vp, _vp, _vp]),
    "pgpu_prefill_gemm_qkv": (_i, [_vp, _vp, _vp, _i, _i, _kvp, _i, _vp, _i, _vp, _vp, _vp,
                                    _vp]),
    "pgpu_prefill_gemm_residual": (_i, [_vp, _vp, _vp, _i, _i, _vp, _vp, _vp]),
    "pgpu_prefill_gemm_gelu_split": (_i, [_vp, _vp, _vp, _i, _i, _vp, _vp]),
    "pgpu_prefill_attention_rows": (_i, [_vp, _vp, _kvp, _i, _vp, _i, _vp, _i, _vp, _i, _vp,
                                         _i, _vp]),
    "pgpu_prefill_attention_mfma": (_i, [_vp, _vp, _kvp, _i, _vp, _i, _vp, _i, _vp, _i, _vp,
                                         _i, _vp]),
    "phonon_flow_batch_set_prefill_exact": (_i, [_vp, _i]),
    "phonon_flow_batch_set_wait_limit": (_i, [_vp, ctypes.c_uint]),
    "pgpu_prefill_attention": (_i, [_vp, _vp, _kvp, _i, _vp, _i, _vp, _i, _i, _i, _vp, _i,
                                    _scp, _vp]),
    "pgpu_attention_static": (_i, [_vp, _vp, _kvp, _i, _vp, _i, _vp, _i, _i, _i, _vp, _vp,
                                   _vp]),
    "pgpu_ln_split": (_i, [_vp, _vp, _i, _vp, _vp, _f, _vp, _vp, _vp]),
    "pgpu_split_rows": (_i, [_vp, _vp, _i, _i, _vp, _vp]),
    "pgpu_norm_row": (_i, [_vp, _vp, _i, _vp, _vp, _f, _i, _vp, _vp]),
    "pgpu_gelu": (_i, [_vp, _vp, _sz, _vp]),
    "pgpu_rope": (_i, [_vp, _vp, _i, _i, _vp, _vp]),
    "pgpu_kv_copy": (_i, [_vp, _kvp, _vp, _i, _i, _i, _i, _vp, _vp, _sz, _i, _vp]),
    "pgpu_fill_normal": (_i, [_vp, _vp, _sz, ctypes.c_uint64]),
    "pgpu_advance_positions": (_i, [_vp, _vp, _i, _i]),
    "pgpu_fill_normal_plan": (_sz, [_sz, _sz, _szp, _szp]),
    "pgpu_gather_rows": (_i, [_vp, _vp, _vp, _vp, _i, _i]),
    "pgpu_gather_rows_copy": (_i, [_vp, _vp, _vp, _vp, _i, _i, _vp, _vp]),
    "pgpu_fill_u32": (_i, [_vp, _vp, _sz, ctypes.c_uint32]),
    "pgpu_flow_schedule": (_sz, [_sz, _sz, _szp, _vp, _i, ctypes.POINTER(ctypes.c_uint32),
                                 _sz]),
    "pgpu_flow_launch": (_i, [_vp, _vp, _kvp]),
    "pgpu_gemm_silu_split": (_i, [_vp, _vp, _vp, _i, _vp, _vp, _vp, _vp]),
    "pgpu_gemm_gated": (_i, [_vp, _vp, _vp, _i, _vp, _vp, _i, _vp, _vp, _vp]),
    "pgpu_head_front": (_i, [_vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i,
                             _vp, _f, _vp, _vp, _vp]),
    "pgpu_head_mod": (_i, [_vp, _vp, _vp, _i, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp]),
    "pgpu_head_mlp_in": (_i, [_vp, _vp, _vp, _i, _vp, _vp, _f, _vp, _i, _vp, _vp, _vp]),
    "pgpu_head_block": (_i, [_vp, _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _f, _vp, _i, _vp,
                             _vp, _i, _vp]),
    "pgpu_head_final": (_i, [_vp, _vp, _vp, _i, _vp, _f, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp,
                             _i, _vp, _vp]),
    "pgpu_head_time_phase": (_i, [_vp, _vp, _f, _vp, _vp]),
    "pgpu_head_time_sum": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "phonon_flow_head_forward": (_i, [_vp, _vp, _vp, _f, _f, _vp]),
    "phonon_flow_head_load": (_i, [_vp, _vp]),
    "phonon_flow_eos_logit": (_i, [_vp, _vp, _vp]),
    "phonon_flow_denormalize_latent": (_i, [_vp, _vp, _vp]),
    "phonon_flow_lsd_one_step": (_i, [_vp, _vp, _vp, _f, _vp]),
    "phonon_flow_lsd_one_step_cancel": (_i, [_vp, _vp, _vp, _f, _vp, _vp, _vp]),
    "phonon_flow_head_prepare": (_i, [_vp]),
    "phonon_flow_head_release": (None, [_vp]),
    "phonon_flow_head_device_create": (_i, [_vp, _vp, _vp, _sz, _pp]),
    # phonon_mimi.h / phonon_conv.h / phonon_pcm.h
    "phonon_mimi_config": (PhononMimiConfig, []),
    "phonon_mimi_model_load": (_i, [_vp, ctypes.POINTER(PhononMimiConfig),
                                    ctypes.POINTER(PhononMimiModel)]),
    "phonon_mimi_state_create": (_i, [ctypes.POINTER(PhononMimiModel), _pp]),
    "phonon_mimi_state_reset": (None, [_vp]),
    "phonon_mimi_state_destroy": (None, [_vp]),
    "phonon_mimi_positions": (_sz, [_vp]),
    "phonon_mimi_process": (_i, [_vp, _fp, _sz, _fp, _sz]),
    "phonon_mimi_upsample_frame": (_i, [_viewp, _fp, _fp, _sz, _sz, _fp]),
    "phonon_conv_model_create": (_i, [_viewp, _viewp, _sz, _i, _pp]),
    "phonon_conv_model_destroy": (None, [_vp]),
    "phonon_conv_input_channels": (_sz, [_vp]),
    "phonon_conv_output_channels": (_sz, [_vp]),
    "phonon_conv_stride": (_sz, [_vp]),
    "phonon_conv_state_create": (_i, [_vp, _pp]),
    "phonon_conv_state_destroy": (None, [_vp]),
    "phonon_conv_state_reset": (None, [_vp]),
    "phonon_conv_process": (_i, [_vp, _fp, _sz, _fp, _sz]),
    "phonon_conv_elu": (None, [_fp, _sz]),
    "phonon_residual_state_create": (_i, [_vp, _vp, _pp]),
    "phonon_residual_state_destroy": (None, [_vp]),
    "phonon_residual_state_reset": (None, [_vp]),
    "phonon_residual_process": (_i, [_vp, _fp, _sz, _fp, _sz]),
    "phonon_pcm_model_create": (_i, [_vp, _pp]),
    "phonon_pcm_model_destroy": (None, [_vp]),
    "phonon_pcm_state_create": (_i, [_vp, _pp]),
    "phonon_pcm_state_destroy": (None, [_vp]),
    "phonon_pcm_state_reset": (None, [_vp]),
    "phonon_pcm_samples": (_sz, [_vp]),
    "phonon_pcm_process": (_i, [_vp, _fp, _sz, _fp, _sz, _fp, _sz]),
    "phonon_pcm_finish": (_i, [_vp]),
    "phonon_pcm_model_from_parts": (_i, [ctypes.POINTER(PhononMimiModel), _vp * 11, _pp]),
    "pgpu_mimi_input": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _vp, _vp]),
    "pgpu_mimi_rope_store": (_i, [_vp, _vp, _i, ctypes.c_longlong, _vp, ctypes.c_longlong, _vp,
                                  _vp, _i]),
    "pgpu_mimi_attention": (_i, [_vp, _vp, _i, ctypes.c_longlong, _vp, _vp, _i, _i, _vp,
                                 _vp]),
    "pgpu_head_flow_schedule": (_i, [_vp, _i, _i, _i, _i]),
    "pgpu_head_flow_launch": (_i, [_vp, _vp]),
    "pgpu_head_flow_reset": (_i, [_vp, _vp, _sz, _vp]),
    "phonon_flow_head_device_set_one_launch": (_i, [_vp, _i]),
    "phonon_flow_head_device_set_fused_mlp": (_i, [_vp, _i]),
    "phonon_flow_head_device_set_wait_limit": (_i, [_vp, ctypes.c_uint]),
    "pgpu_q8_gemv": (_i, [_vp, _vp, _vp, _i, _i, _vp, _i, _vp, _vp]),
    "phonon_q8_device_matvec_valu": (_i, [_vp, _sz, _vp, _vp, _sz, _vp]),
    "pgpu_conv_rows": (_i, [_vp, ctypes.POINTER(PgpuConvLayer), _vp, _i, _vp, _vp, _vp, _i, _vp,
                            _vp]),
    "pgpu_upsample_frame": (_i, [_vp, _vp, _vp, _vp, _i, _i, _vp, _vp]),
    "pgpu_elu": (_i, [_vp, _vp, _vp, _sz]),
    "phonon_flow_head_device_destroy": (None, [_vp]),
    "phonon_flow_head_device_lsd": (_i, [_vp, _sz, _vp, _vp, _f, _vp, _vp]),
    "phonon_flow_head_device_set_graph": (_i, [_vp, _i]),
    "phonon_flow_head_device_set_frame": (_i, [_vp, _vp, _vp, _vp]),
    "phonon_flow_head_device_set_stream": (_i, [_vp, _vp]),
    "phonon_flow_head_device_frame": (_i, [_vp, _sz, _vp, _vp, _vp, _f, _vp, _vp, _vp]),
    "phonon_flow_head_device_stream": (_vp, [_vp]),
    "phonon_flow_head_device_sync": (_i, [_vp]),
}

_LIB = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load libphonon_mi355x.so and declare every exported signature.
    Raises when the library is not built: there is no fallback."""
    global _LIB
    if _LIB is not None and path == LIB_PATH:
        return _LIB
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: build it with __graft_entry__.build() "
                           "(make -C speech-mac_amd)")
    lib = ctypes.CDLL(path)
    for name, (restype, argtypes) in EXPORTS.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    if path == LIB_PATH:
        _LIB = lib
    return lib


def last_error(lib) -> str:
    msg = lib.pgpu_last_error()
    return msg.decode() if msg else ""


def fptr(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_fp)


def vptr(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data)


# ------------------------------------------------------------- host helpers
class Views:
    """Keeps numpy buffers and PhononTensorView structs alive together."""

    def __init__(self):
        self.keep = []

    def q8(self, blocks: np.ndarray, rows: int, cols: int) -> PhononTensorView:
        assert blocks.dtype == Q8_BLOCK and blocks.size == rows * cols // 32
        blocks = np.ascontiguousarray(blocks)
        self.keep.append(blocks)
        v = PhononTensorView(PACK_Q8_0, 2, (ctypes.c_uint64 * 8)(rows, cols), blocks.ctypes.data,
                             blocks.nbytes, None)
        self.keep.append(v)
        return v

    def bf16(self, bits: np.ndarray, shape) -> PhononTensorView:
        bits = np.ascontiguousarray(bits, np.uint16)
        self.keep.append(bits)
        v = PhononTensorView(PACK_BF16, len(shape), (ctypes.c_uint64 * 8)(*shape),
                             bits.ctypes.data, bits.nbytes, None)
        self.keep.append(v)
        return v

    def flow_head(self, bits: dict) -> "PhononFlowHead":
        """bf16-bit arrays by role (the keys of tests' flow-head builders) ->
        PhononFlowHead of BF16 views."""
        h = PhononFlowHead()
        v = lambda key: self.bf16(bits[key], bits[key].shape)  # noqa: E731
        for name in ("input_weight", "input_bias", "cond_weight", "cond_bias",
                     "final_ada_weight", "final_ada_bias", "final_weight", "final_bias"):
            setattr(h, name, v(name))
        for i in range(2):
            for j in range(2):
                h.time_weight[i][j] = v(f"time_weight_{i}_{j}")
                h.time_bias[i][j] = v(f"time_bias_{i}_{j}")
            h.time_freqs[i] = v(f"time_freqs_{i}")
            h.time_alpha[i] = v(f"time_alpha_{i}")
        for b in range(HEAD_BLOCKS):
            h.block_ada_weight[b] = v(f"block_ada_weight_{b}")
            h.block_ada_bias[b] = v(f"block_ada_bias_{b}")
            h.block_norm_weight[b] = v(f"block_norm_weight_{b}")
            h.block_norm_bias[b] = v(f"block_norm_bias_{b}")
            for j in range(2):
                h.block_mlp_weight[b][j] = v(f"block_mlp_weight_{b}_{j}")
                h.block_mlp_bias[b][j] = v(f"block_mlp_bias_{b}_{j}")
        self.keep.append(h)
        return h

    def layers(self, layer_dicts) -> ctypes.Array:
        """layer dicts (see synthetic.flow_layer) -> PhononFlowLayerWeights[L]."""
        arr = (PhononFlowLayerWeights * len(layer_dicts))()
        for i, d in enumerate(layer_dicts):
            def mat(key, rows, cols):
                if d[key].dtype == Q8_BLOCK:
                    return self.q8(d[key], rows, cols)
                return self.bf16(d[key], (rows, cols))
            views = [mat("qkv", 3 * WIDTH, WIDTH), mat("out", WIDTH, WIDTH),
                     mat("mlp_in", FFN, WIDTH), mat("mlp_out", WIDTH, FFN)]
            views += [self.bf16(d[k], (WIDTH,)) for k in
                      ("norm1_weight", "norm1_bias", "norm2_weight", "norm2_bias")]
            arr[i] = PhononFlowLayerWeights(*[ctypes.pointer(v) for v in views])
        self.keep.append(arr)
        return arr


class PgpuFlowPlacement(ctypes.Structure):
    """pgpu_flow_placement (phonon_gpu.h)."""
    _fields_ = [("unit_us", ctypes.c_float), ("after_us", ctypes.c_float * 4)]


class DeviceBuffer:
    """Device allocation through the library's pgpu_malloc (no torch)."""

    def __init__(self, lib, nbytes: int):
        self.lib = lib
        self.nbytes = int(nbytes)
        self.ptr = lib.pgpu_malloc(self.nbytes)
        if not self.ptr:
            raise MemoryError(f"pgpu_malloc({nbytes}): {last_error(lib)}")

    def upload(self, a: np.ndarray, stream=None):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        if not self.lib.pgpu_copy_h2d(stream, self.ptr, a.ctypes.data, a.nbytes):
            raise RuntimeError(last_error(self.lib))

    def download(self, shape, dtype=np.float32, stream=None) -> np.ndarray:
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes
        if not self.lib.pgpu_copy_d2h(stream, out.ctypes.data, self.ptr, out.nbytes):
            raise RuntimeError(last_error(self.lib))
        return out

    def free(self):
        if self.ptr:
            self.lib.pgpu_stream_sync(None)
            self.lib.pgpu_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
