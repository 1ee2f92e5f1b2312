/*
 * oracle.c -- CPU restatement of gemma4.c's W8A8 forward path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker for the HIP path and the timed
 * CPU baseline.  The product library never links this file.
 *
 * Parity pins (each function is checked by tests/test_oracle*.py):
 *   - against the compiled reference (oracle/_ref, built from the reference
 *     sources by oracle/Makefile) on identical inputs, bit for bit, for every
 *     kernel below and for forward()/logits() on a full synthetic model;
 *   - against the committed golden vectors in tests/golden/ (written by the
 *     compiled reference), so the pin holds where the reference is absent;
 *   - against closed forms: brute-force integer dot products, the quantizer's
 *     +-127 / zero-group cases, the GELU-table and RoPE formulas.
 *   Functions that call libm (expf in softmax, tanhf in logits, sqrtf in
 *   rmsnorm) are bit-exact against the reference only for the same libm; the
 *   GPU side is held to tolerances there.
 *
 * Build: gcc -std=c11 -O3 -ffp-contract=off -fopenmp (oracle/Makefile).  With
 * contraction off, every a*b+c below rounds twice; fmaf() marks the places the
 * reference uses an explicit fused multiply-add intrinsic.
 */
#define _POSIX_C_SOURCE 200809L
#include "oracle.h"

#include <cpuid.h>
#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

#if defined(__x86_64__)
#include <immintrin.h>
#endif

/* ------------------------------------------------------------------------- */
/* State                                                                      */

struct orc_state {
    float *residual;         /* [BATCH x HIDDEN] */
    float *hidden;           /* [BATCH x 8*HIDDEN]; also the VOCAB logits row */
    float *aux;              /* [BATCH x 8*HIDDEN] */
    int8_t *quantized;       /* [BATCH x 8*HIDDEN] */
    float *act_scales;       /* one per 64 quantized values */
    float *per_layer_inputs; /* [BATCH x LAYERS x PLE] */
    int32_t *xsum;           /* VNNI correction scratch [BATCH x 8*HIDDEN/64] */
    float *cache[15];        /* owner layers 0..14: K ring then V ring */
};

static const size_t kWide = (size_t)ORC_BATCH * 8 * ORC_HIDDEN;

static int owner_is_full(int layer) { return layer % 5 == 4; }
static int ring_len(int full) { return full ? ORC_MAX_CONTEXT : ORC_SLIDING_RING; }
static int ring_dim(int full) { return full ? 512 : 256; }

static size_t cache_floats(int layer) {
    int full = owner_is_full(layer);
    return 2 * (size_t)ring_len(full) * (size_t)ring_dim(full);
}

orc_state *orc_state_new(void) {
    orc_state *s = calloc(1, sizeof(*s));
    if (!s) return NULL;
    s->residual = calloc((size_t)ORC_BATCH * ORC_HIDDEN, sizeof(float));
    s->hidden = calloc(kWide, sizeof(float));
    s->aux = calloc(kWide, sizeof(float));
    s->quantized = calloc(kWide, 1);
    s->act_scales = calloc(kWide / 64, sizeof(float));
    s->per_layer_inputs = calloc((size_t)ORC_BATCH * ORC_LAYERS * ORC_PLE, sizeof(float));
    s->xsum = calloc(kWide / 64, sizeof(int32_t));
    int ok = s->residual && s->hidden && s->aux && s->quantized && s->act_scales &&
             s->per_layer_inputs && s->xsum;
    for (int l = 0; l < 15; l++) {
        s->cache[l] = calloc(cache_floats(l), sizeof(float)); /* lazily paged in */
        ok = ok && s->cache[l];
    }
    if (!ok) {
        orc_state_free(s);
        return NULL;
    }
    return s;
}

void orc_state_free(orc_state *s) {
    if (!s) return;
    free(s->residual);
    free(s->hidden);
    free(s->aux);
    free(s->quantized);
    free(s->act_scales);
    free(s->per_layer_inputs);
    free(s->xsum);
    for (int l = 0; l < 15; l++) free(s->cache[l]);
    free(s);
}

void orc_state_reset(orc_state *s) {
    for (int l = 0; l < 15; l++) {
        free(s->cache[l]);
        s->cache[l] = calloc(cache_floats(l), sizeof(float));
    }
    memset(s->residual, 0, (size_t)ORC_BATCH * ORC_HIDDEN * sizeof(float));
}

float *orc_state_cache(orc_state *s, int layer, int *cache_len, int *head_dim) {
    if (layer < 0 || layer >= 15) return NULL;
    int full = owner_is_full(layer);
    if (cache_len) *cache_len = ring_len(full);
    if (head_dim) *head_dim = ring_dim(full);
    return s->cache[layer];
}

float *orc_state_residual(orc_state *s) { return s->residual; }
float *orc_state_hidden(orc_state *s) { return s->hidden; }

/* ------------------------------------------------------------------------- */
/* Threads and dispatch                                                       */

static int g_threads = 0;
static int g_fast = 1;

void orc_set_threads(int n) { g_threads = n > 0 ? n : 0; }

/* One thread per physical core unless OMP_NUM_THREADS is set (gemma4.c:182-188). */
int orc_threads(void) {
    if (g_threads > 0) return g_threads;
    if (getenv("OMP_NUM_THREADS")) return omp_get_max_threads();
    unsigned int eax = 0, ebx = 0, ecx = 0, edx = 0;
    int per_core = 1;
    if (__get_cpuid_max(0, NULL) >= 0xB) {
        __cpuid_count(0xB, 0, eax, ebx, ecx, edx);
        per_core = (int)(ebx & 0xffff);
        if (per_core <= 0) per_core = 1;
    }
    int n = omp_get_num_procs() / per_core;
    return n > 0 ? n : 1;
}

int orc_fast_available(void) {
#if defined(__x86_64__)
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
           __builtin_cpu_supports("avx512vnni");
#else
    return 0;
#endif
}

void orc_set_fast(int on) { g_fast = on; }

/* fp16 bit pattern -> fp32, exact (the _cvtsh_ss of gemma4.c:350 and the
 * vcvtph2ps of gemma4.c:216). */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exponent = (h >> 10) & 0x1fu, mantissa = h & 0x3ffu;
    if (exponent == 0) {
        float f = (float)mantissa * 5.9604644775390625e-8f; /* m * 2^-24, exact */
        return sign ? -f : f;
    }
    uint32_t bits = exponent == 31 ? (sign | 0x7f800000u | (mantissa << 13))
                                   : (sign | ((exponent + 112u) << 23) | (mantissa << 13));
    float f;
    memcpy(&f, &bits, sizeof(f));
    return f;
}

/* ------------------------------------------------------------------------- */
/* Kernel bodies: orphaned work-sharing loops, called inside a parallel team. */

/* gemma4.c:265-279. */
static void quantize_body(int8_t *q, float *scales, const float *x, size_t rows, size_t width) {
    size_t groups = rows * (width / 64);
#pragma omp for schedule(static)
    for (size_t gi = 0; gi < groups; gi++) {
        const float *v = x + gi * 64;
        float max_abs = 0.0f;
        for (int j = 0; j < 64; j++) {
            float a = fabsf(v[j]);
            if (a > max_abs) max_abs = a;
        }
        float scale = max_abs / 127.0f;
        float inverse = scale > 0.0f ? 1.0f / scale : 0.0f;
        for (int j = 0; j < 64; j++) q[gi * 64 + j] = (int8_t)rintf(v[j] * inverse);
        scales[gi] = scale;
    }
}

/* One 16-row output block, scalar: per 64-group exact int32 dot, then the fold
 * acc = fma((float)dot, f32(ws) * xs, acc) over groups in ascending order
 * (gemma4.c:202-218 / 235-248).  Packed tile layout: tile (block, g) is 1024
 * bytes at ((block * G + g) * 1024), byte (chunk c, row r, j) at c*64 + r*4 + j,
 * holding W[block*16 + r][g*64 + c*4 + j]. */
static void matmul_block_scalar(float *out, const int8_t *xq, const float *xs,
                                const orc_tensor *w, size_t rows, size_t block) {
    const size_t n_out = (size_t)w->shape[0], k = (size_t)w->shape[1], groups = k / 64;
    const int8_t *tiles = (const int8_t *)w->data + block * 16 * k;
    const uint16_t *ws = w->scales + block * groups * 16;
    for (size_t m = 0; m < rows; m++) {
        const int8_t *x = xq + m * k;
        for (int r = 0; r < 16; r++) {
            float acc = 0.0f;
            for (size_t g = 0; g < groups; g++) {
                const int8_t *tile = tiles + g * 1024;
                int32_t dot = 0;
                for (int c = 0; c < 16; c++)
                    for (int j = 0; j < 4; j++)
                        dot += (int32_t)x[g * 64 + c * 4 + j] * (int32_t)tile[c * 64 + r * 4 + j];
                float p = orc_f16_to_f32(ws[g * 16 + r]) * xs[m * groups + g];
                acc = fmaf((float)dot, p, acc);
            }
            out[m * n_out + block * 16 + r] = acc;
        }
    }
}

#if defined(__x86_64__)
/* Same block with AVX-512 VNNI.  vpdpbusd wants unsigned x signed bytes, so the
 * weights are offset to w+128 (an xor with 0x80) and the exact correction
 * 128 * sum(x over the group) is subtracted afterwards; the int32 dot is then
 * identical to the scalar one, and the fold is the same fma, so results are
 * bit-identical. */
__attribute__((target("avx512f,avx512bw,avx512vl,avx512vnni,fma,f16c"))) static void
matmul_block_vnni(float *out, const int8_t *xq, const float *xs, const int32_t *xsum,
                  const orc_tensor *w, size_t rows, size_t block) {
    const size_t n_out = (size_t)w->shape[0], k = (size_t)w->shape[1], groups = k / 64;
    const int8_t *tiles = (const int8_t *)w->data + block * 16 * k;
    const uint16_t *ws = w->scales + block * groups * 16;
    const __m512i flip = _mm512_set1_epi8((char)0x80);
    for (size_t m0 = 0; m0 < rows; m0 += 8) {
        size_t live = rows - m0 < 8 ? rows - m0 : 8;
        __m512 acc[8];
        for (int i = 0; i < 8; i++) acc[i] = _mm512_setzero_ps();
        for (size_t g = 0; g < groups; g++) {
            __m512i dot[8];
            for (int i = 0; i < 8; i++) dot[i] = _mm512_setzero_si512();
            const int8_t *tile = tiles + g * 1024;
            for (int c = 0; c < 16; c++) {
                __m512i wu = _mm512_xor_si512(_mm512_loadu_si512((const void *)(tile + c * 64)), flip);
                for (size_t i = 0; i < live; i++) {
                    int32_t x4;
                    memcpy(&x4, xq + (m0 + i) * k + g * 64 + c * 4, 4);
                    dot[i] = _mm512_dpbusd_epi32(dot[i], wu, _mm512_set1_epi32(x4));
                }
            }
            __m512 wscale = _mm512_cvtph_ps(_mm256_loadu_si256((const __m256i *)(ws + g * 16)));
            for (size_t i = 0; i < live; i++) {
                size_t m = m0 + i;
                __m512i exact = _mm512_sub_epi32(dot[i], _mm512_set1_epi32(128 * xsum[m * groups + g]));
                __m512 p = _mm512_mul_ps(wscale, _mm512_set1_ps(xs[m * groups + g]));
                acc[i] = _mm512_fmadd_ps(_mm512_cvtepi32_ps(exact), p, acc[i]);
            }
        }
        for (size_t i = 0; i < live; i++)
            _mm512_storeu_ps(out + (m0 + i) * n_out + block * 16, acc[i]);
    }
}
#endif

/* gemma4.c:257-262: one work item per 16-row output block. */
static void matmul_body(float *out, const int8_t *xq, const float *xs, const orc_tensor *w,
                        size_t rows, int32_t *xsum) {
    const size_t blocks = (size_t)w->shape[0] / 16;
    const size_t k = (size_t)w->shape[1], groups = k / 64;
#if defined(__x86_64__)
    if (g_fast && xsum && orc_fast_available()) {
#pragma omp for schedule(static)
        for (size_t gi = 0; gi < rows * groups; gi++) {
            int32_t s = 0;
            for (int j = 0; j < 64; j++) s += xq[gi * 64 + j];
            xsum[gi] = s;
        }
#pragma omp for schedule(static)
        for (size_t b = 0; b < blocks; b++) matmul_block_vnni(out, xq, xs, xsum, w, rows, b);
        return;
    }
#endif
    (void)xsum;
#pragma omp for schedule(static)
    for (size_t b = 0; b < blocks; b++) matmul_block_scalar(out, xq, xs, w, rows, b);
}

/* gemma4.c:281-294: 16 fma lanes over j = lane (mod 16), then the fixed tree
 * ((l0..7 + l8..15) -> 4 -> (s0 + s2) + (s1 + s3)). */
static float score_one(const float *q, const float *key, int head_dim) {
    float lane[16] = {0};
#if defined(__AVX2__) && defined(__FMA__)
    /* the 16 lanes in two registers (lanes 0-7, 8-15), so the chains stay in
     * registers; each lane's fma chain is the scalar one */
    __m256 lo = _mm256_setzero_ps(), hi = _mm256_setzero_ps();
    for (int j = 0; j < head_dim; j += 16) {
        lo = _mm256_fmadd_ps(_mm256_loadu_ps(q + j), _mm256_loadu_ps(key + j), lo);
        hi = _mm256_fmadd_ps(_mm256_loadu_ps(q + j + 8), _mm256_loadu_ps(key + j + 8), hi);
    }
    _mm256_storeu_ps(lane, lo);
    _mm256_storeu_ps(lane + 8, hi);
#else
    for (int j = 0; j < head_dim; j += 16)
        for (int l = 0; l < 16; l++) lane[l] = fmaf(q[j + l], key[j + l], lane[l]);
#endif
    float s8[8], s4[4];
    for (int l = 0; l < 8; l++) s8[l] = lane[l] + lane[l + 8];
    for (int l = 0; l < 4; l++) s4[l] = s8[l] + s8[l + 4];
    return (s4[0] + s4[2]) + (s4[1] + s4[3]);
}

static void scores_serial(float *scores, const float *q, const float *kc, int first, int n,
                          int mask, int head_dim) {
    for (int i = 0; i < n; i++)
        scores[i] = score_one(q, kc + (size_t)((first + i) & mask) * head_dim, head_dim);
}

/* gemma4.c:400-408. */
static void softmax_serial(float *v, int n) {
    float max = v[0], sum = 1.0f;
    for (int i = 1; i < n; i++) {
        if (v[i] > max) {
            sum = sum * expf(max - v[i]) + 1.0f;
            max = v[i];
        } else {
            sum += expf(v[i] - max);
        }
    }
    for (int i = 0; i < n; i++) v[i] = expf(v[i] - max) / sum;
}

/* gemma4.c:296-307: per output channel, an fma chain over keys in order. */
static void value_sum_serial(float *out, const float *p, const float *vc, int first, int n,
                             int mask, int head_dim) {
#if defined(__AVX2__) && defined(__FMA__)
    /* 64 channels at a time, their chains held in eight registers (kept in
     * memory, the chains are store-forwarding bound: ~5x slower) */
    for (int j = 0; j < head_dim; j += 64) {
        __m256 acc[8];
        for (int r = 0; r < 8; r++) acc[r] = _mm256_setzero_ps();
        for (int i = 0; i < n; i++) {
            const float *v = vc + (size_t)((first + i) & mask) * head_dim + j;
            const __m256 pi = _mm256_broadcast_ss(p + i);
            for (int r = 0; r < 8; r++) acc[r] = _mm256_fmadd_ps(pi, _mm256_loadu_ps(v + 8 * r), acc[r]);
        }
        for (int r = 0; r < 8; r++) _mm256_storeu_ps(out + j + 8 * r, acc[r]);
    }
#else
    for (int j = 0; j < head_dim; j += 64) {
        float acc[64] = {0};
        for (int i = 0; i < n; i++) {
            const float *v = vc + (size_t)((first + i) & mask) * head_dim + j;
            for (int u = 0; u < 64; u++) acc[u] = fmaf(p[i], v[u], acc[u]);
        }
        memcpy(out + j, acc, sizeof(acc));
    }
#endif
}

/* gemma4.c:310-331: table GELU with linear interpolation, times up. */
static void geglu_body(float *gate, const float *up, int rows, int width, int up_stride,
                       const orc_tensor *gelu_table) {
    const float *table = (const float *)gelu_table->data;
    const int size = gelu_table->shape[0];
    const float lower = (float)gelu_table->shape[1];
    const float upper = (float)gelu_table->shape[2];
    const float scale = (float)(size - 1) / (upper - lower);
#pragma omp for collapse(2) schedule(static)
    for (int r = 0; r < rows; r++) {
        for (int i = 0; i < width; i++) {
            float x = gate[(size_t)r * width + i];
            if (x <= lower) {
                x = table[0];
            } else if (!(x >= upper)) {
                float position = (x - lower) * scale;
                int index = (int)position;
                float fraction = position - (float)index;
                x = table[index] + fraction * (table[index + 1] - table[index]);
            }
            gate[(size_t)r * width + i] = x * up[(size_t)r * up_stride + i];
        }
    }
}

/* gemma4.c:337-358: gather one packed int8 row per token and dequantize. */
static void embedding_body(float *out, const orc_tensor *table, const int *tokens, size_t n,
                           float multiplier) {
    const int width = table->shape[1], groups = width / 64;
#pragma omp for schedule(static)
    for (size_t t = 0; t < n; t++) {
        size_t block = (size_t)(tokens[t] / 16);
        int row = tokens[t] % 16;
        float *v = out + t * width;
        const int8_t *data = (const int8_t *)table->data + block * 16 * (size_t)width;
        const uint16_t *sc = table->scales + block * (size_t)groups * 16;
        for (int g = 0; g < groups; g++) {
            const int8_t *tile = data + (size_t)g * 1024;
            float s = orc_f16_to_f32(sc[g * 16 + row]) * multiplier;
            for (int j = 0; j < 64; j++) v[g * 64 + j] = (float)tile[(j / 4) * 64 + row * 4 + j % 4] * s;
        }
    }
}

/* gemma4.c:360-373: sequential fp32 sum of squares. */
static void rmsnorm_body(float *out, const float *in, const orc_tensor *weight, int width,
                         float epsilon, size_t rows) {
    const float *w = weight ? (const float *)weight->data : NULL;
#pragma omp for schedule(static)
    for (size_t r = 0; r < rows; r++) {
        const float *x = in + r * width;
        float *y = out + r * width;
        float sum = 0.0f;
        for (int i = 0; i < width; i++) sum += x[i] * x[i];
        float inverse = 1.0f / sqrtf(sum / (float)width + epsilon);
        for (int i = 0; i < width; i++) y[i] = (w ? w[i] : 1.0f) * (inverse * x[i]);
    }
}

/* gemma4.c:375-378. */
static void add_and_scale_body(float *out, const float *add, size_t n, float scale) {
#pragma omp for schedule(static)
    for (size_t i = 0; i < n; i++) out[i] = (out[i] + add[i]) * scale;
}

/* gemma4.c:381-398: half-split rotation of the first `pairs` channel pairs. */
static void rope_body(const orc_tensor *cosines, const orc_tensor *sines, float *v, int heads,
                      int head_dim, int start_pos, size_t n) {
    const int pairs = cosines->shape[1];
#pragma omp for schedule(static)
    for (size_t t = 0; t < n; t++) {
        const float *c = (const float *)cosines->data + ((size_t)start_pos + t) * pairs;
        const float *s = (const float *)sines->data + ((size_t)start_pos + t) * pairs;
        for (int h = 0; h < heads; h++) {
            float *x = v + (t * heads + h) * (size_t)head_dim;
            for (int j = 0; j < pairs; j++) {
                float a = x[j], b = x[j + head_dim / 2];
                x[j] = a * c[j] - b * s[j];
                x[j + head_dim / 2] = b * c[j] + a * s[j];
            }
        }
    }
}

/* gemma4.c:443-456: every (head, token) scores, softmaxes and sums values. */
static void attend_body(float *out, const float *q, const float *kc, const float *vc,
                        int cache_len, int head_dim, int heads, int full, int start_pos,
                        size_t n, float *scores) {
    const int mask = cache_len - 1;
    const size_t width = (size_t)heads * head_dim;
#pragma omp for collapse(2) schedule(dynamic, 1)
    for (size_t h = 0; h < (size_t)heads; h++) {
        for (size_t t = 0; t < n; t++) {
            int pos = start_pos + (int)t;
            int first = !full && pos + 1 > ORC_WINDOW ? pos + 1 - ORC_WINDOW : 0;
            int keys = pos + 1 - first;
            scores_serial(scores, q + t * width + h * head_dim, kc, first, keys, mask, head_dim);
            softmax_serial(scores, keys);
            value_sum_serial(out + t * width + h * head_dim, scores, vc, first, keys, mask,
                             head_dim);
        }
    }
}

/* gemma4.c:411-461. */
static void attention_body(orc_state *s, const orc_layer *layers, int layer, int start_pos,
                           size_t n, float *scores) {
    const orc_layer *w = &layers[layer];
    const int full = owner_is_full(layer);
    const int cache_len = ring_len(full), mask = cache_len - 1;
    const int head_dim = w->q_norm.shape[0];
    const int query_width = w->q_proj.shape[0];
    int owner = layer;
    while (!layers[owner].k_proj.data || owner_is_full(owner) != full) owner--;
    float *kc = s->cache[owner];
    float *vc = kc + (size_t)cache_len * head_dim;

    quantize_body(s->quantized, s->act_scales, s->hidden, n, (size_t)w->q_proj.shape[1]);
    matmul_body(s->aux, s->quantized, s->act_scales, &w->q_proj, n, s->xsum);
    rmsnorm_body(s->aux, s->aux, &w->q_norm, head_dim, 1e-6f, n * (size_t)(query_width / head_dim));
    rope_body(&w->rope_cos, &w->rope_sin, s->aux, query_width / head_dim, head_dim, start_pos, n);

    if (w->k_proj.data) {
        float *new_keys = kc + ((size_t)start_pos & (size_t)mask) * head_dim;
        float *new_values = vc + ((size_t)start_pos & (size_t)mask) * head_dim;
        matmul_body(new_keys, s->quantized, s->act_scales, &w->k_proj, n, s->xsum);
        matmul_body(new_values, s->quantized, s->act_scales, &w->v_proj, n, s->xsum);
        rmsnorm_body(new_keys, new_keys, &w->k_norm, head_dim, 1e-6f, n);
        rmsnorm_body(new_values, new_values, NULL, head_dim, 1e-6f, n);
        rope_body(&w->rope_cos, &w->rope_sin, new_keys, 1, head_dim, start_pos, n);
    }

    attend_body(s->hidden, s->aux, kc, vc, cache_len, head_dim, query_width / head_dim, full,
                start_pos, n, scores);

    quantize_body(s->quantized, s->act_scales, s->hidden, n, (size_t)w->o_proj.shape[1]);
    matmul_body(s->hidden, s->quantized, s->act_scales, &w->o_proj, n, s->xsum);
}

/* ------------------------------------------------------------------------- */
/* Parallel entry points                                                      */

void orc_quantize(int8_t *q, float *scales, const float *x, size_t rows, size_t width) {
#pragma omp parallel num_threads(orc_threads())
    quantize_body(q, scales, x, rows, width);
}

void orc_matmul_int8(float *out, const int8_t *xq, const float *xs, const orc_tensor *w,
                     size_t rows) {
    size_t groups = rows * ((size_t)w->shape[1] / 64);
    int32_t *xsum = malloc(groups * sizeof(int32_t));
#pragma omp parallel num_threads(orc_threads())
    matmul_body(out, xq, xs, w, rows, xsum);
    free(xsum);
}

void orc_attention_scores(float *scores, const float *query, const float *key_cache,
                          int first_key, int num_keys, int cache_mask, int head_dim) {
    scores_serial(scores, query, key_cache, first_key, num_keys, cache_mask, head_dim);
}

void orc_softmax(float *values, int count) { softmax_serial(values, count); }

void orc_weighted_value_sum(float *out, const float *p, const float *value_cache,
                            int first_key, int num_keys, int cache_mask, int head_dim) {
    value_sum_serial(out, p, value_cache, first_key, num_keys, cache_mask, head_dim);
}

void orc_geglu(float *gate, const float *up, int rows, int width, int up_stride,
               const orc_tensor *gelu_table) {
#pragma omp parallel num_threads(orc_threads())
    geglu_body(gate, up, rows, width, up_stride, gelu_table);
}

void orc_embedding(float *out, const orc_tensor *table, const int *tokens, size_t n,
                   float multiplier) {
#pragma omp parallel num_threads(orc_threads())
    embedding_body(out, table, tokens, n, multiplier);
}

void orc_rmsnorm(float *out, const float *in, const orc_tensor *weight, int width,
                 float epsilon, size_t rows) {
#pragma omp parallel num_threads(orc_threads())
    rmsnorm_body(out, in, weight, width, epsilon, rows);
}

void orc_add_and_scale(float *out, const float *add, size_t n, float scale) {
#pragma omp parallel num_threads(orc_threads())
    add_and_scale_body(out, add, n, scale);
}

void orc_apply_rope(const orc_tensor *cosines, const orc_tensor *sines, float *v, int heads,
                    int head_dim, int start_pos, size_t n) {
#pragma omp parallel num_threads(orc_threads())
    rope_body(cosines, sines, v, heads, head_dim, start_pos, n);
}

void orc_attend(float *out, const float *q, const float *key_cache, const float *value_cache,
                int cache_len, int head_dim, int heads, int full_attention, int start_pos,
                size_t n) {
#pragma omp parallel num_threads(orc_threads())
    {
        float *scores = malloc(((size_t)start_pos + n) * sizeof(float));
        attend_body(out, q, key_cache, value_cache, cache_len, head_dim, heads, full_attention,
                    start_pos, n, scores);
        free(scores);
    }
}

/* gemma4.c:411-461: attention() of one layer alone, over the first n rows of
 * the state's hidden buffer (in: the normalized rows, gemma4.c:483; out: the
 * o projection's rows), reading and writing the state's caches. */
void orc_attention_layer(const orc_weights *w, orc_state *s, int layer, int start_pos, size_t n) {
#pragma omp parallel num_threads(orc_threads())
    {
        float *scores = malloc(((size_t)start_pos + n) * sizeof(float));
        attention_body(s, w->layers, layer, start_pos, n, scores);
        free(scores);
    }
}

/* gemma4.c:463-509: one team for the whole step; every kernel shares its loop. */
void orc_forward(const orc_weights *w, orc_state *s, const int *tokens, size_t n,
                 int start_pos) {
    const int ple = w->per_layer_projection_norm.shape[0];
#pragma omp parallel num_threads(orc_threads())
    {
        float *scores = malloc(((size_t)start_pos + n) * sizeof(float));
        embedding_body(s->residual, &w->embed, tokens, n, sqrtf((float)ORC_HIDDEN));

        quantize_body(s->quantized, s->act_scales, s->residual, n, ORC_HIDDEN);
        matmul_body(s->per_layer_inputs, s->quantized, s->act_scales,
                    &w->per_layer_model_projection, n, s->xsum);
        rmsnorm_body(s->per_layer_inputs, s->per_layer_inputs, &w->per_layer_projection_norm, ple,
                     1e-6f * ORC_HIDDEN, n * ORC_LAYERS);
        embedding_body(s->hidden, &w->embed_per_layer, tokens, n, sqrtf((float)ple));
        add_and_scale_body(s->per_layer_inputs, s->hidden, n * ORC_LAYERS * (size_t)ple,
                           1.0f / sqrtf(2.0f));

        for (int layer = 0; layer < ORC_LAYERS; layer++) {
            const orc_layer *lw = &w->layers[layer];
            rmsnorm_body(s->hidden, s->residual, &lw->input_layernorm, ORC_HIDDEN, 1e-6f, n);
            attention_body(s, w->layers, layer, start_pos, n, scores);
            rmsnorm_body(s->hidden, s->hidden, &lw->post_attn_layernorm, ORC_HIDDEN, 1e-6f, n);
            add_and_scale_body(s->residual, s->hidden, n * ORC_HIDDEN, 1.0f);

            rmsnorm_body(s->hidden, s->residual, &lw->pre_ffn_layernorm, ORC_HIDDEN, 1e-6f, n);
            quantize_body(s->quantized, s->act_scales, s->hidden, n, (size_t)lw->gate_proj.shape[1]);
            matmul_body(s->hidden, s->quantized, s->act_scales, &lw->gate_proj, n, s->xsum);
            matmul_body(s->aux, s->quantized, s->act_scales, &lw->up_proj, n, s->xsum);
            geglu_body(s->hidden, s->aux, (int)n, lw->gate_proj.shape[0], lw->gate_proj.shape[0],
                       &w->gelu_table);
            quantize_body(s->quantized, s->act_scales, s->hidden, n, (size_t)lw->down_proj.shape[1]);
            matmul_body(s->hidden, s->quantized, s->act_scales, &lw->down_proj, n, s->xsum);
            rmsnorm_body(s->hidden, s->hidden, &lw->post_ffn_layernorm, ORC_HIDDEN, 1e-6f, n);
            add_and_scale_body(s->residual, s->hidden, n * ORC_HIDDEN, 1.0f);

            quantize_body(s->quantized, s->act_scales, s->residual, n, ORC_HIDDEN);
            matmul_body(s->hidden, s->quantized, s->act_scales, &lw->per_layer_input_gate, n,
                        s->xsum);
            geglu_body(s->hidden, s->per_layer_inputs + (size_t)layer * ple, (int)n, ple,
                       ORC_LAYERS * ple, &w->gelu_table);
            quantize_body(s->quantized, s->act_scales, s->hidden, n,
                          (size_t)lw->per_layer_projection.shape[1]);
            matmul_body(s->hidden, s->quantized, s->act_scales, &lw->per_layer_projection, n,
                        s->xsum);
            rmsnorm_body(s->hidden, s->hidden, &lw->post_per_layer_input_norm, ORC_HIDDEN, 1e-6f, n);
            add_and_scale_body(s->residual, s->hidden, n * ORC_HIDDEN,
                               ((const float *)lw->layer_scalar.data)[0]);
        }
        free(scores);
    }
}

/* gemma4.c:512-522: final norm, tied int8 lm_head, 30*tanh(x/30) soft cap. */
float *orc_logits(const orc_weights *w, orc_state *s, size_t row) {
#pragma omp parallel num_threads(orc_threads())
    {
        rmsnorm_body(s->hidden, s->residual + row * ORC_HIDDEN, &w->norm, ORC_HIDDEN, 1e-6f, 1);
        quantize_body(s->quantized, s->act_scales, s->hidden, 1, ORC_HIDDEN);
        matmul_body(s->hidden, s->quantized, s->act_scales, &w->embed, 1, s->xsum);
#pragma omp for schedule(static)
        for (int i = 0; i < ORC_VOCAB; i++) s->hidden[i] = 30.0f * tanhf(s->hidden[i] / 30.0f);
    }
    return s->hidden;
}

/* ------------------------------------------------------------------------- */
/* Sampling (gemma4.c:527-561), the generator state passed explicitly.        */

/* gemma4.c:529-534: one xorshift64* step; the top 24 bits of the scrambled
 * state as a float in [0, 1). */
static float orc_uniform(uint64_t *state) {
    uint64_t x = *state;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *state = x;
    return (float)((x * 0x2545F4914F6CDD1DULL) >> 40) / 16777216.0f;
}

/* gemma4.c:536-561.  temperature <= 0: the first maximum.  Otherwise the 64
 * highest logits kept in a list sorted by score (a later equal score goes
 * after an earlier one; a score equal to the 64th does not enter), softmax
 * over them at the temperature (sum accumulated in list order), the smallest
 * prefix holding 95% of that sum, one uniform draw scaled by the prefix mass
 * and walked down the prefix. */
int orc_sample(const float *logits, int vocab, float temperature, uint64_t *rng_state) {
    if (temperature <= 0.0f) {
        int best = 0;
        for (int i = 1; i < vocab; i++)
            if (logits[i] > logits[best]) best = i;
        return best;
    }
    float score[64];
    int token[64];
    for (int i = 0; i < 64; i++) {
        score[i] = -INFINITY;
        token[i] = 0;
    }
    for (int t = 0; t < vocab; t++) {
        const float x = logits[t];
        if (x <= score[63]) continue;
        int i = 63;
        for (; i > 0 && x > score[i - 1]; i--) {
            score[i] = score[i - 1];
            token[i] = token[i - 1];
        }
        score[i] = x;
        token[i] = t;
    }
    const float max = score[0] / temperature;
    float sum = 0.0f;
    for (int i = 0; i < 64; i++) {
        score[i] = expf(score[i] / temperature - max);
        sum += score[i];
    }
    float mass = 0.0f;
    int count = 0;
    while (count < 64 && mass < 0.95f * sum) mass += score[count++];
    float threshold = orc_uniform(rng_state) * mass;
    for (int i = 0; i < count; i++)
        if ((threshold -= score[i]) <= 0.0f) return token[i];
    return token[count > 0 ? count - 1 : 0];
}
