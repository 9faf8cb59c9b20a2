/* kpack v1 reader and tensor views (phonon_pack.h), replacing
 * src/phonon_pack.c:87-452 of speech-mac, so that real weights reach the
 * device path: the views it returns feed phonon_flow_model_create /
 * phonon_flow_prepare_weights (device upload, Q8_0 repacked into MFMA
 * fragment order) and the reference-signature functions.
 *
 * File layout (little-endian), as the reference's loader accepts it:
 *   [0, 192)    header: magic "PHNQ8P1\0", u32 version (1), u32 tensor
 *               count (209), u64 index bytes, u64 payload bytes, then five
 *               32-byte digests: source model, model config, SHA-256 of the
 *               index, of the payload and of the metadata;
 *   [192, 196)  u32 metadata bytes, then the metadata: the model's pinned
 *               JSON line, padded with spaces;
 *   index       per tensor: u16 name bytes, u8 dtype, u8 rank, rank u64
 *               dimensions, u64 payload offset, u64 bytes, the name;
 *   payload     starts 8-byte aligned; tensors at 8-byte aligned,
 *               non-overlapping offsets.
 * A pack holds 36 Q8_0 tensors (rank 2, 34 bytes per 32 values) and 173
 * BF16 tensors. phonon_pack_open also pins the index digest of the
 * published model; the test seam phonon_pack_open_for_tests does not.
 *
 * SHA-256 is FIPS 180-4, written here (the reference calls CommonCrypto). */
#include "ph_internal.h"
#include "phonon_pack.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------- SHA-256 -- */

static const uint32_t sha_k[64] = {
    0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4,
    0xab1c5ed5, 0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe,
    0x9bdc06a7, 0xc19bf174, 0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f,
    0x4a7484aa, 0x5cb0a9dc, 0x76f988da, 0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7,
    0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967, 0x27b70a85, 0x2e1b2138, 0x4d2c6dfc,
    0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85, 0xa2bfe8a1, 0xa81a664b,
    0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070, 0x19a4c116,
    0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
    0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7,
    0xc67178f2};

static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

static void sha_block(uint32_t h[8], const unsigned char *p) {
    uint32_t w[64];
    for (int i = 0; i < 16; i++)
        w[i] = (uint32_t)p[4 * i] << 24 | (uint32_t)p[4 * i + 1] << 16 |
               (uint32_t)p[4 * i + 2] << 8 | (uint32_t)p[4 * i + 3];
    for (int i = 16; i < 64; i++) {
        const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
        const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
        w[i] = w[i - 16] + s0 + w[i - 7] + s1;
    }
    uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], k = h[7];
    for (int i = 0; i < 64; i++) {
        const uint32_t t1 = k + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) +
                            sha_k[i] + w[i];
        const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
        k = g;
        g = f;
        f = e;
        e = d + t1;
        d = c;
        c = b;
        b = a;
        a = t1 + t2;
    }
    h[0] += a;
    h[1] += b;
    h[2] += c;
    h[3] += d;
    h[4] += e;
    h[5] += f;
    h[6] += g;
    h[7] += k;
}

/* SHA-256 of `size` bytes into 32 bytes. */
static void sha256(const unsigned char *data, size_t size, unsigned char out[32]) {
    uint32_t h[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a,
                     0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    size_t done = 0;
    for (; size - done >= 64; done += 64)
        sha_block(h, data + done);
    unsigned char tail[128] = {0};
    const size_t rest = size - done;
    memcpy(tail, data + done, rest);
    tail[rest] = 0x80;
    const size_t blocks = rest + 9 <= 64 ? 1 : 2;
    const uint64_t bits = (uint64_t)size * 8;
    for (int i = 0; i < 8; i++)
        tail[blocks * 64 - 1 - i] = (unsigned char)(bits >> (8 * i));
    for (size_t i = 0; i < blocks; i++)
        sha_block(h, tail + 64 * i);
    for (int i = 0; i < 8; i++)
        for (int j = 0; j < 4; j++)
            out[4 * i + j] = (unsigned char)(h[i] >> (24 - 8 * j));
}

/* ---------------------------------------------------------- the format -- */

enum { KP_HEADER = 192, KP_TENSORS = 209, KP_Q8 = 36, KP_BF16 = 173 };
#define KP_MAX_BYTES ((size_t)512 * 1024 * 1024)
#define KP_PREPARE_LIMIT ((size_t)256 * 1024 * 1024)

/* The published model the reference pins (src/phonon_pack.c:12-19). */
static const char kp_source_digest[] =
    "f6acc8f43cb296be31341b4428a6f01b6402659cd0039b624c4aea224936cf95";
static const char kp_config_digest[] =
    "3e89e90b9e7ae5a74c6b4e694960c37fd2ec85906d84adfcc1440c64307aa4f1";
static const char kp_index_digest[] =
    "97512628c18e7532f1c3fd5fa53bd45e58cdd46175b304d3125bea6833cff254";

typedef struct {
    const char *name;
    size_t name_length;
    uint64_t offset;
    PhononTensorView view;
} KpEntry;

struct PhononPack {
    unsigned char *file;
    size_t size;
    KpEntry *entries;
    size_t count;
};

static uint32_t le32(const unsigned char *p) {
    return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
}

static uint64_t le64(const unsigned char *p) { return le32(p) | (uint64_t)le32(p + 4) << 32; }

static int hex_digit(char c) {
    return c >= '0' && c <= '9' ? c - '0' : (c >= 'a' && c <= 'f' ? c - 'a' + 10 : -1);
}

/* The 32 raw bytes equal the 64-digit lowercase hex string. */
static int digest_is(const unsigned char *raw, const char *hex) {
    for (int i = 0; i < 32; i++)
        if (raw[i] != (unsigned char)(hex_digit(hex[2 * i]) << 4 | hex_digit(hex[2 * i + 1])))
            return 0;
    return 1;
}

static int hash_is(const unsigned char *data, size_t size, const unsigned char *expected) {
    unsigned char got[32];
    sha256(data, size, got);
    return memcmp(got, expected, 32) == 0;
}

static int name_char(unsigned char c) {
    return (c >= 'a' && c <= 'z') || (c >= 'A' && c <= 'Z') || (c >= '0' && c <= '9') ||
           c == '_' || c == '.';
}

static void pack_free(PhononPack *pack) {
    if (!pack)
        return;
    for (size_t i = 0; pack->entries && i < pack->count; i++)
        free((void *)pack->entries[i].view.linear_data);
    free(pack->entries);
    free(pack->file);
    free(pack);
}

/* Elements of a shape, 0 on a zero dimension or overflow. */
static size_t elements_of(const uint64_t *shape, unsigned rank) {
    size_t n = 1;
    for (unsigned i = 0; i < rank; i++) {
        if (!shape[i] || shape[i] > SIZE_MAX || n > SIZE_MAX / (size_t)shape[i])
            return 0;
        n *= (size_t)shape[i];
    }
    return n;
}

static unsigned char *read_file(const char *path, size_t *size) {
    FILE *f = fopen(path, "rb");
    if (!f)
        return NULL;
    unsigned char *data = NULL;
    long length = -1;
    if (fseek(f, 0, SEEK_END) == 0)
        length = ftell(f);
    if (length >= KP_HEADER + 4 && (unsigned long)length <= KP_MAX_BYTES &&
        fseek(f, 0, SEEK_SET) == 0) {
        data = malloc((size_t)length);
        if (data && fread(data, 1, (size_t)length, f) != (size_t)length) {
            free(data);
            data = NULL;
        }
    }
    fclose(f);
    if (data)
        *size = (size_t)length;
    return data;
}

/* Header, metadata and digests; on success the index and payload ranges. */
static int check_header(const unsigned char *b, size_t size, int pinned, size_t *index_at,
                        size_t *index_size, size_t *payload_at) {
    static const unsigned char magic[8] = {'P', 'H', 'N', 'Q', '8', 'P', '1', 0};
    if (memcmp(b, magic, 8) || le32(b + 8) != 1 || le32(b + 12) != KP_TENSORS ||
        !digest_is(b + 32, kp_source_digest) || !digest_is(b + 64, kp_config_digest))
        return 0;
    const uint64_t index_bytes = le64(b + 16), payload_bytes = le64(b + 24);
    const size_t meta_size = le32(b + KP_HEADER);
    if (meta_size > size - KP_HEADER - 4)
        return 0;
    const size_t index_start = KP_HEADER + 4 + meta_size;
    if (index_bytes > size - index_start)
        return 0;
    const size_t payload_start = index_start + (size_t)index_bytes;
    if (payload_bytes != size - payload_start || payload_start % 8)
        return 0;
    const unsigned char *meta = b + KP_HEADER + 4;
    if (!hash_is(b + index_start, (size_t)index_bytes, b + 96) ||
        (pinned && !digest_is(b + 96, kp_index_digest)) || !hash_is(meta, meta_size, b + 160) ||
        !hash_is(b + payload_start, (size_t)payload_bytes, b + 128))
        return 0;
    /* The metadata is the model's JSON line (src/phonon_pack.c:166-171),
     * then spaces only. */
    char line[512];
    const int n = snprintf(line, sizeof(line),
                           "{\"config_sha256\":\"%s\",\"model\":\"gradium/phonon-40m-en\","
                           "\"revision\":\"cc738b7e4d182c2ba1bafb8062aa4846af000637\","
                           "\"source\":\"model.q8.gguf\",\"source_sha256\":\"%s\","
                           "\"tensors\":209}",
                           kp_config_digest, kp_source_digest);
    if (n <= 0 || (size_t)n > meta_size || memcmp(meta, line, (size_t)n))
        return 0;
    for (size_t i = (size_t)n; i < meta_size; i++)
        if (meta[i] != ' ')
            return 0;
    *index_at = index_start;
    *index_size = (size_t)index_bytes;
    *payload_at = payload_start;
    return 1;
}

/* One index entry at b[*at, end); advances *at. */
static int read_entry(const unsigned char *b, size_t *at, size_t end, const unsigned char *payload,
                      size_t payload_size, KpEntry *e) {
    if (end - *at < 4)
        return 0;
    const unsigned char *p = b + *at;
    const size_t name_size = (size_t)p[0] | (size_t)p[1] << 8;
    const unsigned dtype = p[2], rank = p[3];
    if (!name_size || name_size > 1024 || !rank || rank > PHONON_PACK_MAX_RANK ||
        end - *at - 4 < (size_t)rank * 8 + 16 + name_size)
        return 0;
    p += 4;
    memset(e, 0, sizeof(*e));
    e->view.rank = rank;
    for (unsigned d = 0; d < rank; d++)
        e->view.shape[d] = le64(p + 8 * d);
    p += 8 * rank;
    e->offset = le64(p);
    const uint64_t bytes = le64(p + 8);
    e->name = (const char *)(p + 16);
    e->name_length = name_size;
    *at += 4 + (size_t)rank * 8 + 16 + name_size;
    int dot = 0;
    for (size_t i = 0; i < name_size; i++) {
        if (!name_char((unsigned char)e->name[i]))
            return 0;
        dot |= e->name[i] == '.';
    }
    if (!dot)
        return 0;
    const size_t n = elements_of(e->view.shape, rank);
    size_t want;
    if (!n)
        return 0;
    if (dtype == PHONON_PACK_Q8_0) {
        if (rank != 2 || e->view.shape[1] % 32 || n / 32 > SIZE_MAX / sizeof(PhononQ8Block))
            return 0;
        want = n / 32 * sizeof(PhononQ8Block);
    } else if (dtype == PHONON_PACK_BF16) {
        if (n > SIZE_MAX / 2)
            return 0;
        want = n * 2;
    } else {
        return 0;
    }
    if (bytes != want || e->offset % 8 || e->offset > payload_size ||
        bytes > payload_size - e->offset)
        return 0;
    e->view.dtype = (PhononPackDType)dtype;
    e->view.data = payload + e->offset;
    e->view.byte_count = (size_t)bytes;
    return 1;
}

static int pack_open(const char *path, PhononPack **result, int pinned) {
    if (!path || !result)
        return 0;
    *result = NULL;
    PhononPack *pack = calloc(1, sizeof(*pack));
    if (!pack)
        return 0;
    pack->file = read_file(path, &pack->size);
    size_t index_at = 0, index_size = 0, payload_at = 0;
    if (!pack->file ||
        !check_header(pack->file, pack->size, pinned, &index_at, &index_size, &payload_at) ||
        !(pack->entries = calloc(KP_TENSORS, sizeof(KpEntry)))) {
        pack_free(pack);
        return 0;
    }
    const unsigned char *payload = pack->file + payload_at;
    const size_t payload_size = pack->size - payload_at;
    size_t at = index_at, q8 = 0, bf16 = 0;
    const size_t end = index_at + index_size;
    for (size_t i = 0; i < KP_TENSORS; i++) {
        KpEntry *e = &pack->entries[i];
        if (!read_entry(pack->file, &at, end, payload, payload_size, e)) {
            pack_free(pack);
            return 0;
        }
        pack->count = i + 1;
        q8 += e->view.dtype == PHONON_PACK_Q8_0;
        bf16 += e->view.dtype == PHONON_PACK_BF16;
        /* Names are unique and tensors do not overlap. */
        for (size_t j = 0; j < i; j++) {
            const KpEntry *o = &pack->entries[j];
            if ((o->name_length == e->name_length && !memcmp(o->name, e->name, e->name_length)) ||
                (e->offset < o->offset + o->view.byte_count &&
                 o->offset < e->offset + e->view.byte_count)) {
                pack_free(pack);
                return 0;
            }
        }
    }
    if (at != end || q8 != KP_Q8 || bf16 != KP_BF16) {
        pack_free(pack);
        return 0;
    }
    *result = pack;
    return 1;
}

int phonon_pack_open(const char *path, PhononPack **pack) { return pack_open(path, pack, 1); }

int phonon_pack_open_for_tests(const char *path, PhononPack **pack) {
    return pack_open(path, pack, 0);
}

void phonon_pack_close(PhononPack *pack) { pack_free(pack); }

size_t phonon_pack_tensor_count(const PhononPack *pack) { return pack ? pack->count : 0; }

int phonon_pack_tensor_at(const PhononPack *pack, size_t index, const char **name,
                          size_t *name_length, PhononTensorView *view) {
    if (!pack || index >= pack->count || !name || !name_length || !view)
        return 0;
    *name = pack->entries[index].name;
    *name_length = pack->entries[index].name_length;
    *view = pack->entries[index].view;
    return 1;
}

int phonon_pack_tensor(const PhononPack *pack, const char *name, PhononTensorView *view) {
    if (!pack || !name || !view)
        return 0;
    const size_t n = strlen(name);
    for (size_t i = 0; i < pack->count; i++)
        if (pack->entries[i].name_length == n && !memcmp(pack->entries[i].name, name, n)) {
            *view = pack->entries[i].view;
            return 1;
        }
    return 0;
}

/* ------------------------------------------------- values and expansion -- */

int phonon_bf16_to_float(const uint16_t *values, size_t count, float *output) {
    if (!values || !output || !count || count > SIZE_MAX / sizeof(float) ||
        ph_overlap(values, count * sizeof(uint16_t), output, count * sizeof(float)))
        return 0;
    for (size_t i = 0; i < count; i++) {
        if (!ph_bf16_finite(values[i]))
            return 0;
        output[i] = ph_bf16_to_float(values[i]);
    }
    return 1;
}

/* src/phonon_pack.c:372-411: BF16 values, or Q8_0 values times their
 * block's scale (scale * (float)q, one product per weight). */
int phonon_tensor_expand_linear(const PhononTensorView *view, float **output) {
    if (!output)
        return 0;
    *output = NULL;
    if (!view || !view->data || view->rank != 2)
        return 0;
    const size_t n = elements_of(view->shape, 2);
    if (!n || n > SIZE_MAX / sizeof(float))
        return 0;
    if (view->dtype == PHONON_PACK_BF16) {
        if (view->byte_count != n * sizeof(uint16_t))
            return 0;
    } else if (view->dtype != PHONON_PACK_Q8_0 || view->shape[1] % 32 ||
               view->byte_count != n / 32 * sizeof(PhononQ8Block)) {
        return 0;
    }
    float *f = malloc(n * sizeof(float));
    if (!f)
        return 0;
    int ok = 1;
    if (view->dtype == PHONON_PACK_BF16) {
        ok = phonon_bf16_to_float(view->data, n, f);
    } else {
        const PhononQ8Block *q = view->data;
        for (size_t b = 0; ok && b < n / 32; b++) {
            const float scale = ph_half_to_float(q[b].scale_bits);
            ok = isfinite(scale);
            for (size_t i = 0; ok && i < 32; i++)
                f[b * 32 + i] = scale * (float)q[b].values[i];
        }
    }
    if (!ok) {
        free(f);
        return 0;
    }
    *output = f;
    return 1;
}

static int has(const char *name, size_t length, const char *part) {
    const size_t m = strlen(part);
    for (size_t i = 0; m <= length && i + m <= length; i++)
        if (!memcmp(name + i, part, m))
            return 1;
    return 0;
}

/* src/phonon_pack.c:413-448: fp32 expansions of every rank-2 linear (not
 * the lookup tables, not the unused flow.w_s_t branch), at most `limit`
 * bytes in all; on failure none is kept. Idempotent. */
static int prepare(PhononPack *pack, size_t limit) {
    if (!pack)
        return 0;
    size_t total = 0;
    int ok = 1;
    for (size_t i = 0; ok && i < pack->count; i++) {
        KpEntry *e = &pack->entries[i];
        if (e->view.rank != 2 || has(e->name, e->name_length, ".embed.weight") ||
            has(e->name, e->name_length, "flow_lm.flow.w_s_t."))
            continue;
        const size_t n = elements_of(e->view.shape, 2);
        if (!n || n > (limit - total) / sizeof(float)) {
            ok = 0;
            break;
        }
        total += n * sizeof(float);
        if (!e->view.linear_data) {
            float *f = NULL;
            ok = phonon_tensor_expand_linear(&e->view, &f);
            e->view.linear_data = f;
        }
    }
    if (!ok)
        for (size_t i = 0; i < pack->count; i++) {
            free((void *)pack->entries[i].view.linear_data);
            pack->entries[i].view.linear_data = NULL;
        }
    return ok;
}

int phonon_pack_prepare_linears(PhononPack *pack) { return prepare(pack, KP_PREPARE_LIMIT); }

int phonon_pack_prepare_linears_for_tests(PhononPack *pack, size_t limit) {
    return prepare(pack, limit);
}
