/*
 * g4img.c -- the gemma4.c model image: validating loader and seeded
 * synthetic-model writer in the exact layout exporter.py produces.
 *
 * The synthetic writer stands in for exporter.py (which needs the real HF
 * checkpoint): same record table, same data order and alignment, same packing
 * and the same weight quantizer, with seeded N(0, 0.02) matrices instead of
 * checkpoint weights.
 */
#define _POSIX_C_SOURCE 200809L
#include "g4img.h"

#include <fcntl.h>
#include <math.h>
#include <omp.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

static char g_error[256] = "no error";

static int fail(const char *msg, int record) {
    if (record >= 0)
        snprintf(g_error, sizeof(g_error), "%s (record %d)", msg, record);
    else
        snprintf(g_error, sizeof(g_error), "%s", msg);
    return -1;
}

const char *g4img_last_error(void) { return g_error; }

static size_t align64(size_t v) { return (v + 63) & ~(size_t)63; }

/* ------------------------------------------------------------------------- */
/* fp16 conversions (round to nearest even, as numpy's astype("<f2")).        */

static uint16_t f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u, exponent = (x >> 23) & 0xffu, mantissa = x & 0x7fffffu;
    if (exponent == 0xff) return (uint16_t)(sign | 0x7c00u | (mantissa ? 0x200u : 0));
    int e = (int)exponent - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t full = mantissa | 0x800000u;
        int shift = 14 - e;
        uint32_t half = full >> shift, rest = full & ((1u << shift) - 1), mid = 1u << (shift - 1);
        if (rest > mid || (rest == mid && (half & 1u))) half++;
        return (uint16_t)(sign | half);
    }
    uint32_t half = ((uint32_t)e << 10) | (mantissa >> 13), rest = mantissa & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (half & 1u))) half++;
    return (uint16_t)(sign | half);
}

static float f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exponent = (h >> 10) & 0x1fu, mantissa = h & 0x3ffu;
    if (exponent == 0) {
        float f = (float)mantissa * 5.9604644775390625e-8f;
        return sign ? -f : f;
    }
    uint32_t bits = exponent == 31 ? (sign | 0x7f800000u | (mantissa << 13))
                                   : (sign | ((exponent + 112u) << 23) | (mantissa << 13));
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* Round to bfloat16 (nearest, ties to even), kept as fp32: what a BF16
 * checkpoint holds for a value (finite inputs). */
static float round_bf16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    x = (x + 0x7fffu + ((x >> 16) & 1u)) & 0xffff0000u;
    memcpy(&f, &x, 4);
    return f;
}

/* ------------------------------------------------------------------------- */
/* Layout plan: the exporter's tensor() call order (exporter.py:95-150).       */

enum {
    K_QUANT = G4IMG_KIND_QUANT,
    K_VECTOR = G4IMG_KIND_VECTOR,
    K_SCALAR = G4IMG_KIND_SCALAR,
    K_ROPE_COS = G4IMG_KIND_ROPE_COS,
    K_ROPE_SIN = G4IMG_KIND_ROPE_SIN,
    K_GELU = G4IMG_KIND_GELU
};

typedef struct {
    int record;  /* first record that references the item (also the RNG key) */
    int kind;
    int rows, cols;
    int global_rope;
    uint64_t data, scales;
} item;

typedef struct {
    uint64_t rec_data[G4_RECORDS], rec_scales[G4_RECORDS];
    int32_t rec_shape[G4_RECORDS][4];
    item items[700];
    int count;
    size_t cursor;
} plan;

static int add(plan *p, int record, int kind, int rows, int cols, int global_rope) {
    item *it = &p->items[p->count];
    it->record = record;
    it->kind = kind;
    it->rows = rows;
    it->cols = cols;
    it->global_rope = global_rope;
    it->data = p->cursor;
    it->scales = 0;
    size_t count = (size_t)rows * (size_t)cols;
    if (kind == K_QUANT) {
        p->cursor = align64(p->cursor + count);
        it->scales = p->cursor;
        p->cursor = align64(p->cursor + count / 64 * 2);
    } else {
        p->cursor = align64(p->cursor + count * 4);
    }
    p->rec_data[record] = it->data;
    p->rec_scales[record] = it->scales;
    if (kind == K_QUANT || kind == K_ROPE_COS || kind == K_ROPE_SIN) {
        p->rec_shape[record][0] = rows;
        p->rec_shape[record][1] = cols;
    } else if (kind == K_GELU) {
        p->rec_shape[record][0] = rows;
        p->rec_shape[record][1] = -8; /* exporter.py:143: (4096, lo, hi) */
        p->rec_shape[record][2] = 8;
    } else {
        p->rec_shape[record][0] = rows;
    }
    return p->count++;
}

static void point(plan *p, int record, int item_index) {
    const item *it = &p->items[item_index];
    p->rec_data[record] = it->data;
    p->rec_scales[record] = it->scales;
    p->rec_shape[record][0] = it->rows;
    p->rec_shape[record][1] = it->cols;
}

static void make_plan(plan *p, unsigned flags) {
    memset(p, 0, sizeof(*p));
    p->cursor = G4IMG_DATA_START;
    add(p, G4IMG_EMBED, K_QUANT, G4_VOCAB, G4_HIDDEN, 0);
    add(p, G4IMG_EMBED_PER_LAYER, K_QUANT, G4_VOCAB, G4_LAYERS * G4_PLE, 0);
    int rope_items[4] = {-1, -1, -1, -1};
    for (int l = 0; l < G4_LAYERS; l++) {
        const int full = l % 5 == 4, kv = l < 15;
        const int hd = full ? 512 : 256, ffn = (flags & G4IMG_FFN_6144) || l < 15 ? 6144 : 12288;
        add(p, G4IMG_LAYER(l, G4F_INPUT_LAYERNORM), K_VECTOR, G4_HIDDEN, 1, 0);
        add(p, G4IMG_LAYER(l, G4F_LAYER_SCALAR), K_SCALAR, 1, 1, 0);
        add(p, G4IMG_LAYER(l, G4F_PRE_FFN_LAYERNORM), K_VECTOR, G4_HIDDEN, 1, 0);
        add(p, G4IMG_LAYER(l, G4F_POST_ATTN_LAYERNORM), K_VECTOR, G4_HIDDEN, 1, 0);
        add(p, G4IMG_LAYER(l, G4F_POST_FFN_LAYERNORM), K_VECTOR, G4_HIDDEN, 1, 0);
        add(p, G4IMG_LAYER(l, G4F_POST_PER_LAYER_INPUT_NORM), K_VECTOR, G4_HIDDEN, 1, 0);
        add(p, G4IMG_LAYER(l, G4F_PER_LAYER_INPUT_GATE), K_QUANT, G4_PLE, G4_HIDDEN, 0);
        add(p, G4IMG_LAYER(l, G4F_PER_LAYER_PROJECTION), K_QUANT, G4_HIDDEN, G4_PLE, 0);
        add(p, G4IMG_LAYER(l, G4F_Q_NORM), K_VECTOR, hd, 1, 0);
        if (kv) add(p, G4IMG_LAYER(l, G4F_K_NORM), K_VECTOR, hd, 1, 0);
        add(p, G4IMG_LAYER(l, G4F_Q_PROJ), K_QUANT, G4_HEADS * hd, G4_HIDDEN, 0);
        if (kv) add(p, G4IMG_LAYER(l, G4F_K_PROJ), K_QUANT, hd, G4_HIDDEN, 0);
        if (kv) add(p, G4IMG_LAYER(l, G4F_V_PROJ), K_QUANT, hd, G4_HIDDEN, 0);
        add(p, G4IMG_LAYER(l, G4F_O_PROJ), K_QUANT, G4_HIDDEN, G4_HEADS * hd, 0);
        add(p, G4IMG_LAYER(l, G4F_GATE_PROJ), K_QUANT, ffn, G4_HIDDEN, 0);
        add(p, G4IMG_LAYER(l, G4F_UP_PROJ), K_QUANT, ffn, G4_HIDDEN, 0);
        add(p, G4IMG_LAYER(l, G4F_DOWN_PROJ), K_QUANT, G4_HIDDEN, ffn, 0);
        /* Shared RoPE tables: written once, every layer of a type points at them
         * (exporter.py:97-102, 129, 350-356). */
        const int base = full ? 2 : 0, pairs = full ? 64 : 128;
        for (int t = 0; t < 2; t++) {
            int rec = G4IMG_LAYER(l, t ? G4F_ROPE_SIN : G4F_ROPE_COS);
            if (rope_items[base + t] < 0)
                rope_items[base + t] = add(p, rec, t ? K_ROPE_SIN : K_ROPE_COS, G4_MAX_CONTEXT, pairs, full);
            else
                point(p, rec, rope_items[base + t]);
        }
    }
    add(p, G4IMG_GELU_TABLE, K_GELU, 4096, 1, 0);
    add(p, G4IMG_NORM, K_VECTOR, G4_HIDDEN, 1, 0);
    add(p, G4IMG_PER_LAYER_MODEL_PROJECTION, K_QUANT, G4_LAYERS * G4_PLE, G4_HIDDEN, 0);
    add(p, G4IMG_PER_LAYER_PROJECTION_NORM, K_VECTOR, G4_PLE, 1, 0);
}

size_t g4img_size(unsigned flags) {
    plan *p = malloc(sizeof(plan));
    if (!p) return 0;
    make_plan(p, flags);
    size_t size = p->cursor;
    free(p);
    return size;
}

/* ------------------------------------------------------------------------- */
/* Seeded values                                                              */

static inline uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static inline uint64_t key_of(uint64_t seed, int record, uint64_t index) {
    return mix64(seed ^ mix64(((uint64_t)(uint32_t)record << 40) ^ index));
}

/* 64 values N(0, sigma) (Box-Muller) for one (record, group) key, from IEEE
 * basic operations only, so the weights are the same on every host and the
 * loops vectorize:
 *   log u1: u1 = m * 2^e, m in [sqrt(1/2), sqrt(2)), log m = 2 atanh(s) with
 *           s = (m - 1) / (m + 1), |s| < 0.172, series to s^11;
 *   sin/cos(2 pi u2): quadrant from u2, Taylor on [0, pi/2) to a^15 / a^16. */
static void normals64(uint64_t key, float sigma, float *v) {
    float u1[32], u2[32], r[32], sn[32], cs[32];
    for (int i = 0; i < 32; i++) {
        uint64_t x = mix64(key + (uint64_t)i * 0xD1B54A32D192ED03ull);
        u1[i] = (float)(int32_t)((x >> 40) + 1) * 5.9604644775390625e-8f; /* (0, 1] */
        u2[i] = (float)(int32_t)((x >> 16) & 0xffffffu) * 5.9604644775390625e-8f;
    }
#pragma omp simd
    for (int i = 0; i < 32; i++) {
        uint32_t b;
        memcpy(&b, &u1[i], 4);
        int e = (int)((b >> 23) & 0xffu) - 127;
        uint32_t mb = (b & 0x7fffffu) | 0x3f800000u;
        float m;
        memcpy(&m, &mb, 4);
        float big = (float)(m > 1.41421356f);
        m = m * (1.0f - 0.5f * big);
        float exponent = (float)e + big;
        float s = (m - 1.0f) / (m + 1.0f), s2 = s * s;
        float p = s2 * (1.0f / 3 + s2 * (1.0f / 5 + s2 * (1.0f / 7 + s2 * (1.0f / 9 + s2 * (1.0f / 11)))));
        float log_u1 = exponent * 0.693147180559945f + 2.0f * (s + s * p);
        r[i] = sigma * sqrtf(-2.0f * log_u1);
        float f = u2[i] * 4.0f;
        int quadrant = (int)f;
        float a = (f - (float)quadrant) * 1.57079632679489662f, a2 = a * a;
        float sa = a * (1 - a2 * (1.0f / 6) * (1 - a2 * (1.0f / 20) * (1 - a2 * (1.0f / 42) *
                   (1 - a2 * (1.0f / 72) * (1 - a2 * (1.0f / 110) * (1 - a2 * (1.0f / 156) *
                   (1 - a2 * (1.0f / 210))))))));
        float ca = 1 - a2 * 0.5f * (1 - a2 * (1.0f / 12) * (1 - a2 * (1.0f / 30) * (1 - a2 * (1.0f / 56) *
                   (1 - a2 * (1.0f / 90) * (1 - a2 * (1.0f / 132) * (1 - a2 * (1.0f / 182) *
                   (1 - a2 * (1.0f / 240))))))));
        /* quadrant 0..3: (sin, cos) = (s, c), (c, -s), (-s, -c), (-c, s) */
        float odd = (float)(quadrant & 1);
        float sign_s = 1.0f - 2.0f * (float)(quadrant >> 1);
        float sign_c = 1.0f - 2.0f * (float)(((quadrant + 1) >> 1) & 1);
        sn[i] = sign_s * (odd * ca + (1.0f - odd) * sa);
        cs[i] = sign_c * (odd * sa + (1.0f - odd) * ca);
    }
    for (int i = 0; i < 32; i++) {
        v[2 * i] = r[i] * cs[i];
        v[2 * i + 1] = r[i] * sn[i];
    }
}

static float uniform(uint64_t key, float lo, float hi) {
    float u = (float)(mix64(key) >> 40) * 5.9604644775390625e-8f;
    return lo + (hi - lo) * u;
}

/* exporter.py:267-273 for one 64-group: fp16 scale floored at 6.104e-05, then
 * rint(x / scale) clipped to [-127, 127]. */
static uint16_t quantize_group(const float *v, int8_t *q) {
    float max_abs = 0.0f;
    for (int j = 0; j < 64; j++) max_abs = fmaxf(max_abs, fabsf(v[j]));
    float s = max_abs / 127.0f;
    if (s < 6.104e-05f) s = 6.104e-05f;
    uint16_t h = f32_to_f16(s);
    float wide = f16_to_f32(h);
    for (int j = 0; j < 64; j++) {
        float r = rintf(v[j] / wide);
        q[j] = (int8_t)(r > 127.0f ? 127.0f : (r < -127.0f ? -127.0f : r));
    }
    return h;
}

static void fill_quant(uint8_t *base, const item *it, uint64_t seed, unsigned flags, int threads) {
    const size_t cols = (size_t)it->cols, groups = cols / 64, blocks = (size_t)it->rows / 16;
    int8_t *data = (int8_t *)(base + it->data);
    uint16_t *scales = (uint16_t *)(base + it->scales);
    /* One 1024-byte tile (16 rows x one 64-column group) per work item, built
     * locally and stored once; values are keyed by (row, group). */
#pragma omp parallel for schedule(static) num_threads(threads)
    for (size_t ti = 0; ti < blocks * groups; ti++) {
        const size_t block = ti / groups, g = ti % groups;
        int8_t tile[1024];
        uint16_t tile_scales[16];
        for (int r = 0; r < 16; r++) {
            float v[64];
            int8_t q[64];
            normals64(key_of(seed, it->record, (block * 16 + (size_t)r) * groups + g), 0.02f, v);
            if (flags & G4IMG_BF16_VALUES)
                for (int j = 0; j < 64; j++) v[j] = round_bf16(v[j]);
            tile_scales[r] = quantize_group(v, q);
            for (int c = 0; c < 16; c++) memcpy(tile + c * 64 + r * 4, q + c * 4, 4);
        }
        memcpy(data + block * 16 * cols + g * 1024, tile, sizeof(tile));
        memcpy(scales + (block * groups + g) * 16, tile_scales, sizeof(tile_scales));
    }
}

/* exporter.py:78-92: angle = pos * theta^(-2j/head_dim), fp32 throughout. */
static void fill_rope(uint8_t *base, const item *it, int threads) {
    const int pairs = it->cols, hd = it->global_rope ? 512 : 256;
    const float theta = it->global_rope ? 1000000.0f : 10000.0f;
    float frequency[128];
    for (int j = 0; j < pairs; j++) frequency[j] = 1.0f / powf(theta, (2.0f * (float)j) / (float)hd);
    float *out = (float *)(base + it->data);
    const int sine = it->kind == K_ROPE_SIN;
#pragma omp parallel for schedule(static) num_threads(threads)
    for (int pos = 0; pos < it->rows; pos++)
        for (int j = 0; j < pairs; j++) {
            float a = (float)pos * frequency[j];
            out[(size_t)pos * pairs + j] = sine ? sinf(a) : cosf(a);
        }
}

/* exporter.py:73-75: tanh-form GELU on linspace(-8, 8, 4096). */
static void fill_gelu(uint8_t *base, const item *it) {
    float *out = (float *)(base + it->data);
    for (int i = 0; i < it->rows; i++) {
        float x = i == it->rows - 1 ? 8.0f : (float)((double)i * (16.0 / 4095.0) - 8.0);
        float cubic = 0.044715f * x * x * x;
        out[i] = 0.5f * x * (1.0f + tanhf(0.7978845608f * (x + cubic)));
    }
}

int g4img_generate(void *buf, size_t size, uint64_t seed, unsigned flags, int threads) {
    plan *p = malloc(sizeof(plan));
    if (!p) return fail("out of memory", -1);
    make_plan(p, flags);
    if (!buf || size < p->cursor || ((uintptr_t)buf & 63)) {
        free(p);
        return fail("buffer too small or not 64-byte aligned", -1);
    }
    if (threads <= 0) threads = omp_get_num_procs();
    uint8_t *base = buf;
    memset(base, 0, G4IMG_DATA_START);
    memcpy(base, "MOG", 4);
    for (int r = 0; r < G4_RECORDS; r++) {
        uint8_t *rec = base + G4IMG_RECORDS_OFFSET + (size_t)r * 32;
        memcpy(rec, &p->rec_data[r], 8);
        memcpy(rec + 8, &p->rec_scales[r], 8);
        memcpy(rec + 16, p->rec_shape[r], 16);
    }
    for (int i = 0; i < p->count; i++) {
        const item *it = &p->items[i];
        /* zero the alignment padding after the item's data (and scales) */
        size_t end = i + 1 < p->count ? p->items[i + 1].data : p->cursor;
        size_t count = (size_t)it->rows * (size_t)it->cols;
        if (it->kind == K_QUANT) {
            memset(base + it->data + count, 0, it->scales - (it->data + count));
            memset(base + it->scales + count / 32, 0, end - (it->scales + count / 32));
        } else {
            memset(base + it->data + count * 4, 0, end - (it->data + count * 4));
        }
        switch (it->kind) {
        case K_QUANT: fill_quant(base, it, seed, flags, threads); break;
        case K_ROPE_COS:
        case K_ROPE_SIN: fill_rope(base, it, threads); break;
        case K_GELU: fill_gelu(base, it); break;
        case K_SCALAR:
        case K_VECTOR: {
            float *out = (float *)(base + it->data);
            const int scalar = it->kind == K_SCALAR;
            for (int j = 0; j < it->rows; j++) {
                out[j] = (flags & G4IMG_UNIT_NORMS)
                             ? 1.0f
                             : uniform(key_of(seed, it->record, (uint64_t)j),
                                       scalar ? 0.9f : 0.75f, scalar ? 1.1f : 1.25f);
                if (flags & G4IMG_BF16_VALUES) out[j] = round_bf16(out[j]);
            }
            break;
        }
        }
    }
    free(p);
    return 0;
}

int g4img_write_file(const char *path, uint64_t seed, unsigned flags, int threads) {
    size_t size = g4img_size(flags);
    int fd = open(path, O_RDWR | O_CREAT | O_TRUNC, 0644);
    if (fd < 0) return fail("cannot create output file", -1);
    if (ftruncate(fd, (off_t)size) != 0) {
        close(fd);
        return fail("cannot size output file", -1);
    }
    void *map = mmap(NULL, size, PROT_READ | PROT_WRITE, MAP_SHARED, fd, 0);
    close(fd);
    if (map == MAP_FAILED) return fail("cannot map output file", -1);
    int rc = g4img_generate(map, size, seed, flags, threads);
    if (msync(map, size, MS_SYNC) != 0 && rc == 0) rc = fail("msync failed", -1);
    munmap(map, size);
    return rc;
}

/* ------------------------------------------------------------------------- */
/* Pieces of the image for a checkpoint writer (gemma4.c_amd/export.py): the
 * layout, the header, the quantize-and-pack step and the tables, so that the
 * writer fills the same bytes from a checkpoint's weights that the synthetic
 * generator fills from its seeded ones.                                      */

int g4img_layout(unsigned flags, g4img_item *out, int max_items) {
    plan *p = malloc(sizeof(plan));
    if (!p) return fail("out of memory", -1);
    make_plan(p, flags);
    const int n = p->count;
    if (!out || max_items < n) {
        free(p);
        return fail("item buffer too small", -1);
    }
    for (int i = 0; i < n; i++) {
        const item *it = &p->items[i];
        out[i].record = it->record;
        out[i].kind = it->kind;
        out[i].rows = it->rows;
        out[i].cols = it->cols;
        out[i].global_rope = it->global_rope;
        out[i].data = it->data;
        out[i].scales = it->scales;
    }
    free(p);
    return n;
}

int g4img_write_header(void *buf, size_t size, unsigned flags) {
    plan *p = malloc(sizeof(plan));
    if (!p) return fail("out of memory", -1);
    make_plan(p, flags);
    if (!buf || size < G4IMG_DATA_START) {
        free(p);
        return fail("buffer smaller than the header", -1);
    }
    uint8_t *base = buf;
    memset(base, 0, G4IMG_DATA_START);
    memcpy(base, "MOG", 4);
    for (int r = 0; r < G4_RECORDS; r++) {
        uint8_t *rec = base + G4IMG_RECORDS_OFFSET + (size_t)r * 32;
        memcpy(rec, &p->rec_data[r], 8);
        memcpy(rec + 8, &p->rec_scales[r], 8);
        memcpy(rec + 16, p->rec_shape[r], 16);
    }
    free(p);
    return 0;
}

static float bf16_to_f32(uint16_t h) {
    const uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static float load_value(const uint8_t *src, int dtype, size_t index) {
    if (dtype == G4IMG_F32) {
        float f;
        memcpy(&f, src + index * 4, 4);
        return f;
    }
    uint16_t h;
    memcpy(&h, src + index * 2, 2);
    return dtype == G4IMG_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
}

int g4img_pack_matrix(const void *src, int dtype, int rows, int cols, void *data, void *scales,
                      int threads) {
    if (!src || !data || !scales || rows <= 0 || cols <= 0 || rows % 16 || cols % 64 ||
        (dtype != G4IMG_F32 && dtype != G4IMG_BF16 && dtype != G4IMG_F16))
        return fail("pack: bad matrix", -1);
    if (threads <= 0) threads = omp_get_num_procs();
    const size_t ncols = (size_t)cols, groups = ncols / 64, blocks = (size_t)rows / 16;
    const uint8_t *in = src;
    int8_t *out = data;
    uint16_t *out_scales = scales;
    int bad = 0;
#pragma omp parallel for schedule(static) num_threads(threads) reduction(| : bad)
    for (size_t ti = 0; ti < blocks * groups; ti++) {
        const size_t block = ti / groups, g = ti % groups;
        int8_t tile[1024];
        uint16_t tile_scales[16];
        for (int r = 0; r < 16; r++) {
            float v[64];
            int8_t q[64];
            const size_t row = block * 16 + (size_t)r;
            for (int j = 0; j < 64; j++) {
                v[j] = load_value(in, dtype, row * ncols + g * 64 + (size_t)j);
                bad |= !(fabsf(v[j]) <= 3.40282347e38f); /* NaN or inf: no scale can hold it */
            }
            tile_scales[r] = quantize_group(v, q);
            for (int c = 0; c < 16; c++) memcpy(tile + c * 64 + r * 4, q + c * 4, 4);
        }
        memcpy(out + block * 16 * ncols + g * 1024, tile, sizeof(tile));
        memcpy(out_scales + (block * groups + g) * 16, tile_scales, sizeof(tile_scales));
    }
    return bad ? fail("pack: the matrix holds a NaN or an infinity", -1) : 0;
}

int g4img_fill_table(void *base, size_t size, const g4img_item *it, int threads) {
    if (!base || !it || it->data + (size_t)it->rows * (size_t)it->cols * 4 > size)
        return fail("table: item outside the buffer", -1);
    if (threads <= 0) threads = omp_get_num_procs();
    item local = {it->record, it->kind, it->rows, it->cols, it->global_rope, it->data, it->scales};
    if (it->kind == K_ROPE_COS || it->kind == K_ROPE_SIN)
        fill_rope(base, &local, threads);
    else if (it->kind == K_GELU)
        fill_gelu(base, &local);
    else
        return fail("table: not a table item", it->record);
    return 0;
}

static void store_value(void *out, int dtype, size_t index, float v) {
    if (dtype == G4IMG_F32) {
        memcpy((uint8_t *)out + index * 4, &v, 4);
    } else {  /* G4IMG_BF16: v is already a bfloat16 value */
        uint32_t x;
        memcpy(&x, &v, 4);
        const uint16_t h = (uint16_t)(x >> 16);
        memcpy((uint8_t *)out + index * 2, &h, 2);
    }
}

int g4img_draw(uint64_t seed, unsigned flags, const g4img_item *it, void *out, int dtype, int threads) {
    if (!it || !out || (dtype != G4IMG_F32 && dtype != G4IMG_BF16) ||
        (dtype == G4IMG_BF16 && !(flags & G4IMG_BF16_VALUES)))
        return fail("draw: bad arguments (BF16 output needs G4IMG_BF16_VALUES)", -1);
    if (threads <= 0) threads = omp_get_num_procs();
    if (it->kind == K_QUANT) {
        const size_t cols = (size_t)it->cols, groups = cols / 64, rows = (size_t)it->rows;
#pragma omp parallel for schedule(static) num_threads(threads)
        for (size_t rg = 0; rg < rows * groups; rg++) {
            float v[64];
            normals64(key_of(seed, it->record, rg), 0.02f, v);
            const size_t at = (rg / groups) * cols + (rg % groups) * 64;
            for (int j = 0; j < 64; j++)
                store_value(out, dtype, at + (size_t)j, (flags & G4IMG_BF16_VALUES) ? round_bf16(v[j]) : v[j]);
        }
        return 0;
    }
    if (it->kind == K_VECTOR || it->kind == K_SCALAR) {
        const int scalar = it->kind == K_SCALAR;
        for (int j = 0; j < it->rows; j++) {
            float v = (flags & G4IMG_UNIT_NORMS) ? 1.0f
                                                 : uniform(key_of(seed, it->record, (uint64_t)j),
                                                           scalar ? 0.9f : 0.75f, scalar ? 1.1f : 1.25f);
            if (flags & G4IMG_BF16_VALUES) v = round_bf16(v);
            store_value(out, dtype, (size_t)j, v);
        }
        return 0;
    }
    return fail("draw: a table item has no draws", it->record);
}

/* ------------------------------------------------------------------------- */
/* Loader                                                                     */

static int read_records(const uint8_t *base, size_t size, uint64_t *data, uint64_t *scales,
                        int32_t (*shape)[4]) {
    if (!base) return fail("null image", -1);
    if (size < (size_t)G4IMG_RECORDS_OFFSET + (size_t)G4_RECORDS * 32)
        return fail("image smaller than its header and record table", -1);
    if (memcmp(base, "MOG", 4) != 0) return fail("bad model file", -1); /* gemma4.c:680 */
    for (int r = 0; r < G4_RECORDS; r++) {
        const uint8_t *rec = base + G4IMG_RECORDS_OFFSET + (size_t)r * 32;
        memcpy(&data[r], rec, 8);
        memcpy(&scales[r], rec + 8, 8);
        memcpy(shape[r], rec + 16, 16);
    }
    for (int r = 0; r < G4_RECORDS; r++) {
        if (!data[r]) {
            if (scales[r]) return fail("record has scales but no data", r);
            continue;
        }
        const int32_t *s = shape[r];
        size_t bytes;
        if (scales[r]) {
            if (s[0] <= 0 || s[1] <= 0 || s[0] % 16 || s[1] % 64)
                return fail("quantized record shape is not packable", r);
            size_t count = (size_t)s[0] * (size_t)s[1];
            if (scales[r] > size || count / 32 > size - scales[r])
                return fail("record scales lie outside the image", r);
            bytes = count;
        } else if (r == G4IMG_GELU_TABLE) {
            if (s[0] < 2 || s[2] <= s[1]) return fail("bad GELU table record", r);
            bytes = (size_t)s[0] * 4;
        } else {
            if (s[0] <= 0 || s[1] < 0) return fail("bad fp32 record shape", r);
            bytes = (size_t)s[0] * (size_t)(s[1] > 0 ? s[1] : 1) * 4;
        }
        if (data[r] > size || bytes > size - data[r]) return fail("record data lies outside the image", r);
    }
    return 0;
}

int g4img_records(const void *base, size_t size, g4_tensor *out) {
    uint64_t data[G4_RECORDS], scales[G4_RECORDS];
    int32_t shape[G4_RECORDS][4];
    if (read_records(base, size, data, scales, shape) != 0) return -1;
    const uint8_t *b = base;
    for (int r = 0; r < G4_RECORDS; r++) {
        out[r].data = data[r] ? (void *)(b + data[r]) : NULL;
        out[r].scales = scales[r] ? (uint16_t *)(b + scales[r]) : NULL;
        memcpy(out[r].shape, shape[r], 16);
    }
    return 0;
}

int g4img_fixup_inplace(void *base, size_t size) {
    g4_tensor records[G4_RECORDS];
    if (g4img_records(base, size, records) != 0) return -1;
    memcpy((uint8_t *)base + G4IMG_RECORDS_OFFSET, records, sizeof(records));
    return 0;
}
