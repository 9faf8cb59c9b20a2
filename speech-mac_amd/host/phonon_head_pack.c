/* The pack-side functions of the flow head (src/phonon_sampler.h:62-71):
 * the head's tensors found by their checkpoint names (phonon_flow_head_load,
 * src/phonon_sampler.c:163-212), the EOS logit of a decoder state
 * (src/phonon_sampler.c:395-401) and the latent's denormalization
 * (src/phonon_sampler.c:403-418). The EOS row runs on the library's own
 * linear (the device); the views stay borrowed from the pack. */
#include "ph_internal.h"
#include "phonon_pack.h"
#include "phonon_sampler.h"

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

/* One tensor of the head: its checkpoint name, its shape and the field of
 * PhononFlowHead it fills. Rank 2 is a linear's weight [rows][cols] (any
 * dtype the linear accepts), rank 1 a BF16 vector of `rows` values. */
typedef struct {
    char name[96];
    unsigned rank;
    uint64_t rows, cols;
    PhononTensorView *view;
} HeadTensor;

/* input, cond, 2 x (two linears, freqs, alpha), 6 x (adaLN, norm weight and
 * bias, two linears), final adaLN, final linear: 68 tensors. */
enum { HEAD_TENSORS = 68 };

typedef struct {
    HeadTensor t[HEAD_TENSORS];
    size_t n;
    int overflow;
} HeadList;

static void add(HeadList *l, PhononTensorView *view, unsigned rank, uint64_t rows,
                uint64_t cols, const char *fmt, ...) {
    if (l->n == HEAD_TENSORS) {
        l->overflow = 1;
        return;
    }
    HeadTensor *t = &l->t[l->n++];
    va_list ap;
    va_start(ap, fmt);
    const int len = vsnprintf(t->name, sizeof(t->name), fmt, ap);
    va_end(ap);
    if (len < 0 || len >= (int)sizeof(t->name))
        l->overflow = 1;
    t->rank = rank;
    t->rows = rows;
    t->cols = cols;
    t->view = view;
}

/* A linear "<prefix>.weight" [rows][cols] with its "<prefix>.bias" [rows]. */
static void add_linear(HeadList *l, PhononTensorView *w, PhononTensorView *b, uint64_t rows,
                       uint64_t cols, const char *prefix) {
    add(l, w, 2, rows, cols, "flow_lm.flow_net.%s.weight", prefix);
    add(l, b, 1, rows, 0, "flow_lm.flow_net.%s.bias", prefix);
}

static void head_tensors(PhononFlowHead *h, HeadList *l) {
    char p[64];
    add_linear(l, &h->input_weight, &h->input_bias, 512, 32, "input_proj");
    add_linear(l, &h->cond_weight, &h->cond_bias, 512, 512, "cond_embed");
    for (size_t i = 0; i < 2; i++) {
        snprintf(p, sizeof(p), "time_embed.%zu.mlp.0", i);
        add_linear(l, &h->time_weight[i][0], &h->time_bias[i][0], 512, 256, p);
        snprintf(p, sizeof(p), "time_embed.%zu.mlp.2", i);
        add_linear(l, &h->time_weight[i][1], &h->time_bias[i][1], 512, 512, p);
        add(l, &h->time_freqs[i], 1, 128, 0, "flow_lm.flow_net.time_embed.%zu.freqs", i);
        add(l, &h->time_alpha[i], 1, 512, 0, "flow_lm.flow_net.time_embed.%zu.mlp.3.alpha", i);
    }
    for (size_t b = 0; b < PHONON_FLOW_HEAD_BLOCKS; b++) {
        snprintf(p, sizeof(p), "res_blocks.%zu.adaLN_modulation.1", b);
        add_linear(l, &h->block_ada_weight[b], &h->block_ada_bias[b], 1536, 512, p);
        add(l, &h->block_norm_weight[b], 1, 512, 0, "flow_lm.flow_net.res_blocks.%zu.in_ln.weight",
            b);
        add(l, &h->block_norm_bias[b], 1, 512, 0, "flow_lm.flow_net.res_blocks.%zu.in_ln.bias",
            b);
        for (size_t j = 0; j < 2; j++) {
            snprintf(p, sizeof(p), "res_blocks.%zu.mlp.%zu", b, 2 * j);
            add_linear(l, &h->block_mlp_weight[b][j], &h->block_mlp_bias[b][j], 512, 512, p);
        }
    }
    add_linear(l, &h->final_ada_weight, &h->final_ada_bias, 1024, 512,
               "final_layer.adaLN_modulation.1");
    add_linear(l, &h->final_weight, &h->final_bias, 32, 512, "final_layer.linear");
}

static int fetch(const PhononPack *pack, const HeadTensor *t) {
    PhononTensorView v;
    if (!phonon_pack_tensor(pack, t->name, &v) || v.rank != t->rank || v.shape[0] != t->rows ||
        (t->rank == 2 && v.shape[1] != t->cols) || (t->rank == 1 && v.dtype != PHONON_PACK_BF16))
        return 0;
    *t->view = v;
    return 1;
}

int phonon_flow_head_load(const PhononPack *pack, PhononFlowHead *head) {
    if (!pack || !head)
        return 0;
    memset(head, 0, sizeof(*head));
    HeadList list = {.n = 0, .overflow = 0};
    head_tensors(head, &list);
    if (list.overflow || list.n != HEAD_TENSORS)
        return 0;
    for (size_t i = 0; i < list.n; i++)
        if (!fetch(pack, &list.t[i]))
            return 0;
    return 1;
}

int phonon_flow_eos_logit(const PhononPack *pack, const float state[512], float *raw_logit) {
    PhononTensorView w, b;
    float bias;
    if (!pack || !state || !raw_logit ||
        !phonon_pack_tensor(pack, "flow_lm.out_eos.weight", &w) || w.rank != 2 ||
        w.shape[0] != 1 || w.shape[1] != 512 ||
        !phonon_pack_tensor(pack, "flow_lm.out_eos.bias", &b) || !ph_vector_decode(&b, 1, &bias))
        return 0;
    return phonon_linear(&w, state, 1, 512, &bias, raw_logit);
}

/* x * std + mean per latent channel (the inverse of
 * phonon_flow_normalize_latent); a non-finite result fails. */
int phonon_flow_denormalize_latent(const PhononPack *pack, const float normalized[32],
                                   float denormalized[32]) {
    PhononTensorView mv, sv;
    float mean[32], std[32];
    if (!pack || !normalized || !denormalized ||
        !phonon_pack_tensor(pack, "flow_lm.emb_mean", &mv) || !ph_vector_decode(&mv, 32, mean) ||
        !phonon_pack_tensor(pack, "flow_lm.emb_std", &sv) || !ph_vector_decode(&sv, 32, std))
        return 0;
    for (size_t i = 0; i < 32; i++) {
        denormalized[i] = normalized[i] * std[i] + mean[i];
        if (!isfinite(denormalized[i]))
            return 0;
    }
    return 1;
}
