/* The pack-side helpers of phonon_transformer.h (src/phonon_transformer.c:
 * 711-914): weights and vectors looked up by tensor name in a kpack, the
 * step's input built from a latent (embed_latent, embed_bos) or tokens, the
 * output norm, voice projection and speaker/duration conditioning. They run
 * on the library's own linear and LayerNorm (the device), and with the
 * batched flow head's frame (phonon_flow_head_device_frame) bracket each
 * decode step as src/phonon_sampler.c:447-483 does. */
#include "ph_internal.h"
#include "phonon_pack.h"

#include <math.h>
#include <stdio.h>
#include <string.h>

#define W PHONON_FLOW_WIDTH

/* A BF16 [count] vector of the pack, decoded (finite values only). */
static int pack_vector(const PhononPack *pack, const char *name, size_t count, float *out) {
    PhononTensorView v;
    return phonon_pack_tensor(pack, name, &v) && ph_vector_decode(&v, count, out);
}

static int add_condition(float *output, const float *condition) {
    for (size_t i = 0; i < W; i++) {
        output[i] += condition[i];
        if (!isfinite(output[i]))
            return 0;
    }
    return 1;
}

/* src/phonon_transformer.c:711-717. */
int phonon_voice_project(const float *voice_latents, size_t frames,
                         const PhononTensorView *projection, float *projected) {
    if (!voice_latents || !projection || !projected || !frames || frames > 8192)
        return 0;
    return phonon_linear_batch(projection, voice_latents, W, W, NULL, projected, frames);
}

/* src/phonon_transformer.c:719-757: speaker embedding row through its
 * projection, plus the duration features [cos | sin](1000 d / 10000^(i/63))
 * through theirs. */
int phonon_flow_condition(const PhononTensorView *speaker_embeddings,
                          const PhononTensorView *speaker_projection,
                          const PhononTensorView *duration_projection, size_t speaker_count,
                          float duration_delta, float output[PHONON_FLOW_WIDTH]) {
    if (!speaker_embeddings || !speaker_embeddings->data || !speaker_projection ||
        !duration_projection || !output || speaker_embeddings->rank != 2 ||
        speaker_embeddings->shape[1] != 16 || speaker_count >= speaker_embeddings->shape[0] ||
        !isfinite(duration_delta) || speaker_embeddings->dtype != PHONON_PACK_BF16 ||
        speaker_embeddings->byte_count != speaker_embeddings->shape[0] * 16 * sizeof(uint16_t))
        return 0;
    const uint16_t *row = (const uint16_t *)speaker_embeddings->data + speaker_count * 16;
    float speaker_in[16], duration[128], speaker[W], from_duration[W];
    for (size_t i = 0; i < 16; i++)
        speaker_in[i] = ph_bf16_to_float(row[i]);
    const double scale = 1000.0 * (double)duration_delta;
    for (size_t i = 0; i < 64; i++) {
        const double phase = scale / pow(10000.0, (double)i / 63.0);
        duration[i] = (float)cos(phase);
        duration[64 + i] = (float)sin(phase);
    }
    if (!phonon_linear(speaker_projection, speaker_in, W, 16, NULL, speaker) ||
        !phonon_linear(duration_projection, duration, W, 128, NULL, from_duration))
        return 0;
    for (size_t i = 0; i < W; i++) {
        output[i] = speaker[i] + from_duration[i];
        if (!isfinite(output[i]))
            return 0;
    }
    return 1;
}

/* src/phonon_transformer.c:759-790: the prefix rows: a projected voice
 * frame for each prompt id (in order), the BOS projection for the one BOS
 * id, the token's embedding otherwise. */
int phonon_flow_prepare_prefix(const int32_t *ids, size_t tokens, const float *token_embeddings,
                               size_t prompt_id, size_t bos_id, const float *projected_voice,
                               size_t voice_frames, const float *bos_latent_projection,
                               float *prefix_embeddings) {
    if (!ids || !tokens || !token_embeddings || !projected_voice || !voice_frames ||
        !bos_latent_projection || !prefix_embeddings || tokens > 8192 || voice_frames > tokens ||
        prompt_id > INT32_MAX || bos_id > INT32_MAX)
        return 0;
    size_t prompts = 0, boses = 0;
    for (size_t i = 0; i < tokens; i++) {
        prompts += ids[i] == (int32_t)prompt_id;
        boses += ids[i] == (int32_t)bos_id;
    }
    if (prompts != voice_frames || boses != 1)
        return 0;
    for (size_t i = 0, voice = 0; i < tokens; i++) {
        const float *src = ids[i] == (int32_t)prompt_id ? projected_voice + W * voice++
                           : ids[i] == (int32_t)bos_id  ? bos_latent_projection
                                                         : token_embeddings + W * i;
        float *dst = prefix_embeddings + W * i;
        memcpy(dst, src, W * sizeof(float));
        if (!ph_all_finite(dst, W))
            return 0;
    }
    return 1;
}

/* src/phonon_transformer.c:796-820: the eight views of each of the nine
 * layers, by their checkpoint names. */
int phonon_flow_load_layers(const PhononPack *pack,
                            PhononTensorView storage[PHONON_FLOW_LAYERS][8],
                            PhononFlowLayerWeights weights[PHONON_FLOW_LAYERS]) {
    static const char *const suffix[8] = {
        "self_attn.in_proj.weight", "self_attn.out_proj.weight", "linear1.weight",
        "linear2.weight",           "norm1.weight",              "norm1.bias",
        "norm2.weight",             "norm2.bias"};
    if (!pack || !storage || !weights)
        return 0;
    for (size_t l = 0; l < PHONON_FLOW_LAYERS; l++) {
        for (size_t k = 0; k < 8; k++) {
            char name[160];
            snprintf(name, sizeof(name), "flow_lm.transformer.layers.%zu.%s", l, suffix[k]);
            if (!phonon_pack_tensor(pack, name, &storage[l][k]))
                return 0;
        }
        weights[l] = (PhononFlowLayerWeights){
            .qkv = &storage[l][0], .attention_out = &storage[l][1], .mlp_in = &storage[l][2],
            .mlp_out = &storage[l][3], .norm1_weight = &storage[l][4],
            .norm1_bias = &storage[l][5], .norm2_weight = &storage[l][6],
            .norm2_bias = &storage[l][7]};
    }
    return 1;
}

/* src/phonon_transformer.c:822-840: rows of the transcript embedding table. */
int phonon_flow_embed_tokens(const PhononPack *pack, const int32_t *ids, size_t count,
                             float *embeddings) {
    PhononTensorView t;
    if (!pack || !ids || !count || !embeddings || count > 8192 ||
        !phonon_pack_tensor(
            pack, "flow_lm.condition_provider.conditioners.transcript_in_segment.embed.weight",
            &t) ||
        t.rank != 2 || t.shape[1] != W || t.dtype != PHONON_PACK_BF16 ||
        t.byte_count != t.shape[0] * W * sizeof(uint16_t))
        return 0;
    for (size_t i = 0; i < count; i++)
        if (ids[i] < 0 || (uint64_t)ids[i] >= t.shape[0] ||
            !phonon_bf16_to_float((const uint16_t *)t.data + (size_t)ids[i] * W, W,
                                  embeddings + W * i))
            return 0;
    return 1;
}

/* src/phonon_transformer.c:842-858: input_linear . bos_emb + condition. */
int phonon_flow_embed_bos(const PhononPack *pack, const float condition[PHONON_FLOW_WIDTH],
                          float output[PHONON_FLOW_WIDTH]) {
    PhononTensorView bos, lin;
    float latent[32];
    if (!pack || !condition || !output || !phonon_pack_tensor(pack, "flow_lm.bos_emb", &bos) ||
        bos.rank != 1 || bos.shape[0] != 32 || bos.dtype != PHONON_PACK_BF16 ||
        !phonon_pack_tensor(pack, "flow_lm.input_linear.weight", &lin) ||
        !phonon_bf16_to_float(bos.data, 32, latent) ||
        !phonon_linear(&lin, latent, W, 32, NULL, output))
        return 0;
    return add_condition(output, condition);
}

/* src/phonon_transformer.c:860-874: the next step's input from a latent,
 * input_linear . latent + condition. */
int phonon_flow_embed_latent(const PhononPack *pack, const float latent[32],
                             const float condition[PHONON_FLOW_WIDTH],
                             float output[PHONON_FLOW_WIDTH]) {
    PhononTensorView lin;
    if (!pack || !latent || !condition || !output ||
        !phonon_pack_tensor(pack, "flow_lm.input_linear.weight", &lin) ||
        !phonon_linear(&lin, latent, W, 32, NULL, output))
        return 0;
    return add_condition(output, condition);
}

/* src/phonon_transformer.c:876-902: (x - mean) / std per latent channel. */
int phonon_flow_normalize_latent(const PhononPack *pack, const float denormalized[32],
                                 float normalized[32]) {
    float mean[32], std[32];
    if (!pack || !denormalized || !normalized ||
        !pack_vector(pack, "flow_lm.emb_mean", 32, mean) ||
        !pack_vector(pack, "flow_lm.emb_std", 32, std))
        return 0;
    for (size_t i = 0; i < 32; i++) {
        if (!isfinite(denormalized[i]) || !(std[i] > 0.0f))
            return 0;
        normalized[i] = (denormalized[i] - mean[i]) / std[i];
        if (!isfinite(normalized[i]))
            return 0;
    }
    return 1;
}

/* src/phonon_transformer.c:904-914: the decoder's final LayerNorm (eps
 * 1e-5), in place. */
int phonon_flow_output_norm(const PhononPack *pack, float values[PHONON_FLOW_WIDTH]) {
    float w[W], b[W], y[W];
    if (!pack || !values || !pack_vector(pack, "flow_lm.out_norm.weight", W, w) ||
        !pack_vector(pack, "flow_lm.out_norm.bias", W, b) ||
        !phonon_layer_norm(values, w, b, W, 1e-5f, y))
        return 0;
    memcpy(values, y, sizeof(y));
    return 1;
}
