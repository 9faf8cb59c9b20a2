// Single-phase projection kernels: one projection of B streams per launch,
// one task (pgpu_gemm.hpp) per 512-thread work-group. Used by the primitives
// of phonon_transformer.h / phonon_q8.h and by the batched step when it runs
// phase by phase; the one-launch step (pgpu_flow.hip) runs the same tasks.
#include "pgpu_gemm.hpp"
#include "phonon_gpu.h"

namespace pgpu {

template <int EPI, bool Q8>
__global__ __launch_bounds__(kTaskThreads) void k_gemm(GemmArgs a) {
    __shared__ f32x4 lds4[kTaskWaves * 64];
    gemm_split_task<EPI, Q8>(a, blockIdx.x, blockIdx.y, (uint16_t *)lds4, NoWait{});
}

template <int SRC, int EPI, bool Q8>
__global__ __launch_bounds__(kTaskThreads) void k_gemm_wide(GemmArgs a) {
    __shared__ uint4 bsh4[kTaskLds / 8];
    gemm_wide_task<SRC, EPI, Q8>(a, blockIdx.x, blockIdx.y, (uint16_t *)bsh4, NoWait{});
}

template <int SRC, int EPI, bool Q8>
static int launch(const GemmArgs &a, hipStream_t stream) {
    if (a.n_rows <= 0 || a.n_rows % 16 || a.k_cols <= 0 || a.k_cols % 32 || a.streams <= 0 ||
        (SRC != SRC_SPLIT && a.k_cols != kWidth))
        return bad_arguments("pgpu_gemm");
    if constexpr (SRC != SRC_SPLIT) {
        const dim3 grid((a.n_rows / 16 + 3) / 4, (a.streams + 15) / 16);
        hipLaunchKernelGGL((k_gemm_wide<SRC, EPI, Q8>), grid, dim3(kTaskThreads), 0, stream, a);
    } else {
        const dim3 grid(a.n_rows / 16, (a.streams + 15) / 16);
        hipLaunchKernelGGL((k_gemm<EPI, Q8>), grid, dim3(kTaskThreads), 0, stream, a);
    }
    return launch_ok("pgpu_gemm");
}

template <int EPI>
static int dispatch(const GemmArgs &a, int q8, hipStream_t stream) {
    if (a.plain_rows)
        return q8 ? launch<SRC_ROWS, EPI, true>(a, stream)
                  : launch<SRC_ROWS, EPI, false>(a, stream);
    const int src = a.ln_x ? SRC_LN : (a.part_acc ? SRC_ATTN : SRC_SPLIT);
    if (src == SRC_LN)
        return q8 ? launch<SRC_LN, EPI, true>(a, stream) : launch<SRC_LN, EPI, false>(a, stream);
    if (src == SRC_ATTN)
        return q8 ? launch<SRC_ATTN, EPI, true>(a, stream)
                  : launch<SRC_ATTN, EPI, false>(a, stream);
    return q8 ? launch<SRC_SPLIT, EPI, true>(a, stream)
              : launch<SRC_SPLIT, EPI, false>(a, stream);
}

// Fills the operand-source fields from a pgpu_gemm_input.
static bool set_input(GemmArgs &a, const pgpu_gemm_input *in) {
    if (!in) return false;
    const int kinds = (in->split != nullptr) + (in->ln_rows != nullptr) +
                      (in->attn_acc != nullptr) + (in->rows != nullptr);
    if (kinds != 1) return false;
    a.xs = in->split;
    a.ln_x = in->rows ? in->rows : in->ln_rows;
    a.plain_rows = in->rows != nullptr;
    a.ln_w = in->ln_weight;
    a.ln_b = in->ln_bias;
    a.ln_eps = in->ln_epsilon;
    a.part_acc = in->attn_acc;
    a.part_ml = in->attn_ml;
    a.max_splits = in->attn_max_splits;
    if (in->ln_rows && (!a.ln_w || !a.ln_b)) return false;
    if (a.part_acc && (!a.part_ml || a.max_splits <= 0 || !in->attn_positions)) return false;
    if (a.part_acc) a.positions = in->attn_positions;
    return true;
}

static bool base_args(GemmArgs &a, const pgpu_matrix *w, const pgpu_gemm_input *in, int streams,
                      int *status) {
    a = GemmArgs{};
    a.w = w->values;
    a.wscale = w->scales;
    a.n_rows = (int)w->rows;
    a.k_cols = (int)w->columns;
    a.streams = streams;
    a.status = status;
    return set_input(a, in);
}

}  // namespace pgpu

using namespace pgpu;

extern "C" int pgpu_gemm_store(void *stream, const pgpu_matrix *w, const pgpu_gemm_input *in,
                               int streams, const float *bias, float *out, int ld_out,
                               int *status) {
    GemmArgs a;
    if (!base_args(a, w, in, streams, status)) return bad_arguments("pgpu_gemm_store");
    a.out = out;
    a.ld_out = ld_out;
    a.bias = bias;
    return dispatch<EPI_STORE>(a, w->q8, (hipStream_t)stream);
}

extern "C" int pgpu_gemm_residual(void *stream, const pgpu_matrix *w, const pgpu_gemm_input *in,
                                  int streams, const float *residual, float *out, int *status) {
    GemmArgs a;
    if (!base_args(a, w, in, streams, status)) return bad_arguments("pgpu_gemm_residual");
    a.out = out;
    a.ld_out = (int)w->rows;
    a.residual = residual;
    return dispatch<EPI_RESIDUAL>(a, w->q8, (hipStream_t)stream);
}

extern "C" int pgpu_gemm_gelu_split(void *stream, const pgpu_matrix *w,
                                    const pgpu_gemm_input *in, int streams, uint16_t *out_split,
                                    int *status) {
    GemmArgs a;
    if (!base_args(a, w, in, streams, status)) return bad_arguments("pgpu_gemm_gelu_split");
    a.out_split = out_split;
    a.out_kb = (int)w->rows / 32;
    return dispatch<EPI_GELU_SPLIT>(a, w->q8, (hipStream_t)stream);
}

extern "C" int pgpu_gemm_silu_split(void *stream, const pgpu_matrix *w,
                                    const pgpu_gemm_input *in, int streams, const float *bias,
                                    const float *bias2, uint16_t *out_split, int *status) {
    GemmArgs a;
    if (w->rows % 32 || !base_args(a, w, in, streams, status))
        return bad_arguments("pgpu_gemm_silu_split");
    a.bias = bias;
    a.bias2 = bias2;
    a.out_split = out_split;
    a.out_kb = (int)w->rows / 32;
    return dispatch<EPI_SILU_SPLIT>(a, w->q8, (hipStream_t)stream);
}

extern "C" int pgpu_gemm_gated(void *stream, const pgpu_matrix *w, const pgpu_gemm_input *in,
                               int streams, const float *bias, const float *gate, int ld_gate,
                               const float *residual, float *out, int *status) {
    GemmArgs a;
    if (!gate || !residual || (ld_gate != 0 && ld_gate < (int)w->rows) || ld_gate % 4 ||
        !base_args(a, w, in, streams, status))
        return bad_arguments("pgpu_gemm_gated");
    a.bias = bias;
    a.gate = gate;
    a.ld_gate = ld_gate;
    a.residual = residual;
    a.out = out;
    a.ld_out = (int)w->rows;
    return dispatch<EPI_GATED>(a, w->q8, (hipStream_t)stream);
}

extern "C" int pgpu_gemm_qkv(void *stream, const pgpu_matrix *w, const pgpu_gemm_input *in,
                             int streams, const pgpu_paged_kv *kv, int layer,
                             const int32_t *tables, int table_stride, const int32_t *positions,
                             const float *rope, float *q_out, int *status) {
    GemmArgs a;
    if (w->rows != 3 * kWidth || w->columns != kWidth || layer < 0 || layer >= kv->layers ||
        !base_args(a, w, in, streams, status) || a.part_acc)
        return bad_arguments("pgpu_gemm_qkv");
    a.q_out = q_out;
    a.kv = kv->base;
    a.layer_stride = kv->layer_stride;
    a.blocks = (unsigned)kv->blocks;
    a.layer = layer;
    a.tables = tables;
    a.table_stride = table_stride;
    a.positions = positions;
    a.rope = (const float2 *)rope;
    return dispatch<EPI_QKV>(a, w->q8, (hipStream_t)stream);
}
