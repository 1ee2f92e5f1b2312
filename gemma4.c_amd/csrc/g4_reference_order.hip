// g4_reference_order.hip -- rmsnorm and attention in the reference's own
// summation order, so their results are bit-identical to gemma4.c.
//
// Why: every linear input is re-quantized to int8 (gemma4.c:264-279).  A
// last-bit difference in an rmsnorm or attention output moves a few values
// across an int8 rounding boundary, and each such flip is a perturbation
// ~10^4 times larger than the ulp that caused it; over 35 layers the step's
// logits then drift by 1e-2..1e0 on a random-init model.  Reproducing the
// reference's order is the only way to keep logits within 1e-3.
//
// What is sequential and what is not:
//   rmsnorm (gemma4.c:366-368): squares in parallel, one lane adds them in
//     index order (fp32, no contraction);
//   softmax (gemma4.c:400-408): the running maximum is a prefix maximum, so
//     every expf term is computed in parallel; only the sum recurrence
//     s = s*e + 1 (new maximum) / s = s + e runs on one lane per (token, head);
//   value sums (gemma4.c:296-307): one lane per output channel runs the fma
//     chain over keys in order;
//   scores (gemma4.c:281-294): already order-exact in the parallel kernels'
//     16-lane trees, reused here.
//   expf is the host libm's: the table-driven exp2 method of ARM's
//   optimized-routines (32-entry 2^(i/32) table, degree-3 polynomial, double
//   evaluation with the range reduction fused), which glibc >= 2.28 ships.
//   Checked against the host libm on every input of its main path.
#include <math.h>

#include "g4_internal.h"

namespace g4 {

static int g_order = G4_ORDER_REFERENCE;
int order() { return g_order; }

// 2^(i/32) correctly rounded to double, minus i << 47 (so that adding k << 47
// for k = 32 q + i yields 2^(k/32)).
__constant__ uint64_t kExp2Table[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

__device__ __forceinline__ float expf_libm(float x) {
    const uint32_t ux = __float_as_uint(x);
    const uint32_t abstop = (ux >> 20) & 0x7ff;
    if (abstop >= 0x42b) {                          // |x| >= 88 or not finite
        if (ux == 0xff800000u) return 0.0f;         // -inf
        if (abstop >= 0x7f8) return x + x;          // +inf, nan
        if (x > 0x1.62e42ep6f) return __builtin_inff();
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = (double)x;
    double kd = fma(inv_ln2_n, xd, shift);  // round(x * 32 / ln 2), ties to even
    const uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd -= shift;
    const double r = fma(inv_ln2_n, xd, -kd);
    const uint64_t t = kExp2Table[ki & 31] + (ki << 47);
    const double s = __longlong_as_double((long long)t);
    const double z = fma(c0, r, c1);
    const double r2 = r * r;
    double y = fma(c2, r, 1.0);
    y = fma(z, r2, y);
    return (float)(y * s);
}

// ---------------------------------------------------------------------------
// rmsnorm, reference order: one wave per row.

constexpr int kNormMaxWidth = 1536;

__global__ __launch_bounds__(256) void k_rmsnorm_reference(float *out, const float *in,
                                                           const float *__restrict__ weight,
                                                           int width, float eps, size_t rows) {
    __shared__ __attribute__((aligned(16))) float s_sq[4][kNormMaxWidth];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const size_t row = (size_t)blockIdx.x * 4 + wave;
    const bool valid = row < rows;
    const float *x = in + row * width;
    float *y = out + row * width;
    const bool staged = width <= kNormMaxWidth;
    if (valid && staged)
        for (int i = lane; i < width; i += 64) s_sq[wave][i] = x[i] * x[i];
    __syncthreads();
    float sum = 0.0f;
    if (valid && lane == 0) {
        if (staged) {
            // Batches of 64 squares are read into registers ahead of the add
            // chain that consumes them (two alternating buffers), so the chain
            // never waits on LDS.
            const float4 *sq = reinterpret_cast<const float4 *>(s_sq[wave]);
            const int batches = width / 64;
            float4 ba[16], bb[16];
            if (batches > 0) {
#pragma unroll
                for (int j = 0; j < 16; j++) ba[j] = sq[j];
            }
            for (int b = 0; b < batches; b += 2) {
                if (b + 1 < batches) {
#pragma unroll
                    for (int j = 0; j < 16; j++) bb[j] = sq[(b + 1) * 16 + j];
                }
#pragma unroll
                for (int j = 0; j < 16; j++) {
                    sum += ba[j].x;
                    sum += ba[j].y;
                    sum += ba[j].z;
                    sum += ba[j].w;
                }
                if (b + 2 < batches) {
#pragma unroll
                    for (int j = 0; j < 16; j++) ba[j] = sq[(b + 2) * 16 + j];
                }
                if (b + 1 < batches) {
#pragma unroll
                    for (int j = 0; j < 16; j++) {
                        sum += bb[j].x;
                        sum += bb[j].y;
                        sum += bb[j].z;
                        sum += bb[j].w;
                    }
                }
            }
            for (int i = batches * 64; i < width; i++) sum += s_sq[wave][i];
        } else {
            for (int i = 0; i < width; i++) sum += x[i] * x[i];
        }
    }
    sum = __shfl(sum, 0);
    if (!valid) return;
    const float inverse = 1.0f / sqrtf(sum / (float)width + eps);
    for (int i = lane; i < width; i += 64) y[i] = (weight ? weight[i] : 1.0f) * (inverse * x[i]);
}

void launch_rmsnorm_reference(hipStream_t s, float *out, const float *in, const float *weight,
                              int width, float eps, size_t rows) {
    if (!rows) return;
    hipLaunchKernelGGL(k_rmsnorm_reference, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, out,
                       in, weight, width, eps, rows);
}

void launch_rmsnorm(hipStream_t s, float *out, const float *in, const float *weight, int width,
                    float eps, size_t rows) {
    if (g_order == G4_ORDER_REFERENCE)
        launch_rmsnorm_reference(s, out, in, weight, width, eps, rows);
    else
        launch_rmsnorm_parallel(s, out, in, weight, width, eps, rows);
}

// ---------------------------------------------------------------------------
// Attention, reference order.

__device__ __forceinline__ int first_visible(int pos, int full) {
    return !full && pos + 1 > G4_WINDOW ? pos + 1 - G4_WINDOW : 0;
}

// Scores of every (token, head, visible key), exact (gemma4.c:281-294): 16
// lanes per key, lane m an fma chain over channels m, m+16, ... (s ascending),
// then the fixed tree.  A block takes TQ tokens x 8 heads against 64 keys: each
// 16-lane group keeps its key's channel slice in registers and reads the query
// rows from LDS, stored [row][m][s] (padded) so a lane's chain is contiguous
// (16-byte LDS loads, bank-conflict free).  scores[(t * 8 + h) * stride + (p - first(t))] for key position p.
template <int HD, int TQ>
__global__ __launch_bounds__(256) void k_attn_scores(const float *__restrict__ q,
                                                     const float *__restrict__ key_cache,
                                                     int cache_len, int full, int start_pos, int n,
                                                     size_t stride, float *__restrict__ scores) {
    constexpr int S = HD / 16, SP = S + 4;  // +4 floats: the 16 lanes' 16-byte reads hit distinct banks
    __shared__ __attribute__((aligned(16))) float s_q[TQ * 8][16][SP];
    const int t0 = blockIdx.y * TQ;
    const int tn = n - t0 < TQ ? n - t0 : TQ;
    const int pos_last = start_pos + t0 + tn - 1;
    const int kbase = first_visible(start_pos + t0, full) + blockIdx.x * 64;
    if (kbase > pos_last) return;
    const int mask = cache_len - 1, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float *qt = q + (size_t)t0 * 8 * HD;
    for (int i = tid; i < tn * 8 * HD; i += 256) {
        const int row = i / HD, j = i % HD;
        s_q[row][j & 15][j >> 4] = qt[i];
    }
    __syncthreads();
    const int m = lane & 15, kg = lane >> 4;
    for (int kk = wave * 4 + kg; kk < 64; kk += 16) {
        const int p = kbase + kk;
        if (p > pos_last) break;  // uniform within the 16-lane group
        const float *kr = key_cache + (size_t)(p & mask) * HD + m;
        float kv[S];
#pragma unroll
        for (int s = 0; s < S; s++) kv[s] = kr[16 * s];
        for (int row = 0; row < tn * 8; row++) {
            const int t = t0 + row / 8, pos = start_pos + t, first = first_visible(pos, full);
            const float4 *qv = reinterpret_cast<const float4 *>(s_q[row][m]);
            float acc = 0.0f;
#pragma unroll
            for (int s4 = 0; s4 < S / 4; s4++) {
                const float4 qq = qv[s4];
                acc = fmaf(qq.x, kv[4 * s4 + 0], acc);
                acc = fmaf(qq.y, kv[4 * s4 + 1], acc);
                acc = fmaf(qq.z, kv[4 * s4 + 2], acc);
                acc = fmaf(qq.w, kv[4 * s4 + 3], acc);
            }
            acc += __shfl_down(acc, 8, 16);
            acc += __shfl_down(acc, 4, 16);
            acc += __shfl_down(acc, 2, 16);
            acc += __shfl_down(acc, 1, 16);
            if (m == 0 && p >= first && p <= pos)
                scores[((size_t)t * 8 + (row & 7)) * stride + (p - first)] = acc;
        }
    }
}

// Softmax of one row in place (gemma4.c:400-408), by one wave.  Per block of
// 64 values: a prefix-max scan gives each value the maximum m seen before it;
// a value above m contributes expf(m - v) as a rescale factor (the sum becomes
// s * e + 1), any other value expf(v - m) as an addend.  Lane 0 applies the
// recurrence in index order, reading its operands from LDS in batches so the
// chain never waits on memory; the next block's values are loaded meanwhile.
// Then p = expf(v - max) / sum.
__device__ void softmax_row_reference(float *v, int count, float *s_e, int *s_new) {
    const int lane = threadIdx.x & 63;
    float carry = v[0];  // max = values[0], sum = 1 (gemma4.c:401)
    float sum = 1.0f;
    float x_next = 1 + lane < count ? v[1 + lane] : -INFINITY;
    for (int base = 1; base < count; base += 64) {
        const float x = x_next;
        const int j_next = base + 64 + lane;
        x_next = j_next < count ? v[j_next] : -INFINITY;
        float incl = x;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float y = __shfl_up(incl, o);
            if (lane >= o) incl = fmaxf(incl, y);
        }
        incl = fmaxf(incl, carry);
        float before = __shfl_up(incl, 1);
        if (lane == 0) before = carry;
        const int is_new = x > before;
        s_e[lane] = is_new ? expf_libm(before - x) : expf_libm(x - before);
        s_new[lane] = is_new;
        const int any_new = __any(is_new);
        __syncthreads();
        if (lane == 0) {
            const int n = count - base < 64 ? count - base : 64;
            if (!any_new && n == 64) {
                const float4 *e4 = reinterpret_cast<const float4 *>(s_e);
                float4 e[16];
#pragma unroll
                for (int i = 0; i < 16; i++) e[i] = e4[i];
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    sum += e[i].x;
                    sum += e[i].y;
                    sum += e[i].z;
                    sum += e[i].w;
                }
            } else {
                for (int jj = 0; jj < n; jj++) {
                    if (s_new[jj])
                        sum = sum * s_e[jj] + 1.0f;
                    else
                        sum += s_e[jj];
                }
            }
        }
        carry = __shfl(incl, 63);
        __syncthreads();
    }
    sum = __shfl(sum, 0);
    const float max = carry;
    for (int i = lane; i < count; i += 64) v[i] = expf_libm(v[i] - max) / sum;
}

// Attention probabilities of every (token, head) row, one wave each.
__global__ __launch_bounds__(64) void k_attn_softmax_reference(float *__restrict__ scores,
                                                               int heads, int full, int start_pos,
                                                               size_t stride) {
    __shared__ float s_e[64];
    __shared__ int s_new[64];
    const int h = blockIdx.x, t = blockIdx.y;
    const int pos = start_pos + t, keys = pos + 1 - first_visible(pos, full);
    softmax_row_reference(scores + ((size_t)t * heads + h) * stride, keys, s_e, s_new);
}

// Independent rows of `count` values at `stride` (the per-op entry point).
__global__ __launch_bounds__(64) void k_softmax_rows(float *values, int count, size_t stride) {
    __shared__ float s_e[64];
    __shared__ int s_new[64];
    softmax_row_reference(values + (size_t)blockIdx.x * stride, count, s_e, s_new);
}

// out[t][h][d] = fma chain over keys in order (gemma4.c:296-307): one lane
// per output channel and (token, head) chain.  A block takes a 64-channel
// slice for WAVES waves; wave w runs the chains of token t0 + w / (8 / HPW)
// for HPW heads.  V rows are staged in LDS 64 keys at a time, transposed to
// [channel][key] so a lane reads four keys with one 16-byte load, and DEPTH
// tiles are prefetched into registers ahead of the chains.  A key outside a
// token's window is skipped by that token's chains (the order of the keys it
// does see is unchanged).
template <int HD, int WAVES, int HPW, int DEPTH>
__global__ __launch_bounds__(WAVES * 64) void k_attn_values(float *__restrict__ out,
                                                            const float *__restrict__ probs,
                                                            const float *__restrict__ value_cache,
                                                            int cache_len, int full, int start_pos,
                                                            int n, size_t stride) {
    constexpr int THREADS = WAVES * 64;
    constexpr int TOKENS = WAVES * HPW / 8;     // tokens per block
    constexpr int F4 = 64 * 64 / 4 / THREADS;   // float4 per thread per tile
    __shared__ __attribute__((aligned(16))) float s_v[64][64 + 4];
    // wave is made provably uniform so the probability loads below are scalar
    // loads: vector loads would retire in order behind the V prefetch ring.
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int d0 = blockIdx.x * 64, t0 = blockIdx.y * TOKENS;
    const int tn = n - t0 < TOKENS ? n - t0 : TOKENS;
    const int mask = cache_len - 1;
    const int pos_last = start_pos + t0 + tn - 1;
    const int kfirst = first_visible(start_pos + t0, full);
    const int tiles = (pos_last - kfirst + 64) / 64;

    const int my_t = t0 + wave / (8 / HPW), h0 = (wave % (8 / HPW)) * HPW;
    const bool active = my_t < t0 + tn;
    const int my_pos = start_pos + my_t, my_first = first_visible(my_pos, full);
    const float *prow = probs + ((size_t)my_t * 8 + h0) * stride;

    // tile loader: thread covers float4 (key kr, channels 4 cc .. 4 cc + 3)
    auto load_tile = [&](int tile, float4 (&r)[F4]) {
#pragma unroll
        for (int i = 0; i < F4; i++) {
            const int idx = i * THREADS + tid, kr = idx >> 4, cc = idx & 15;
            // keys past the block's last position are never consumed; loading a
            // valid row instead keeps the loads unconditional (no drain)
            const int p = min(kfirst + tile * 64 + kr, pos_last);
            r[i] = *reinterpret_cast<const float4 *>(value_cache + (size_t)(p & mask) * HD + d0 + 4 * cc);
        }
    };
    float4 ring[DEPTH][F4];
#pragma unroll
    for (int s = 0; s < DEPTH; s++) load_tile(min(s, tiles - 1), ring[s]);

    float o[HPW];
#pragma unroll
    for (int e = 0; e < HPW; e++) o[e] = 0.0f;

    // One tile: stage ring slot `s` in LDS, refill the slot DEPTH tiles ahead,
    // then run this wave's chains over the tile.  The loop below is unrolled by
    // DEPTH so every slot index is a compile-time constant (precise waits).
    auto step = [&](int tile, float4 (&slot)[F4]) {
        __syncthreads();  // previous tile fully consumed
#pragma unroll
        for (int i = 0; i < F4; i++) {
            const int idx = i * THREADS + tid, kr = idx >> 4, cc = idx & 15;
            s_v[4 * cc + 0][kr] = slot[i].x;
            s_v[4 * cc + 1][kr] = slot[i].y;
            s_v[4 * cc + 2][kr] = slot[i].z;
            s_v[4 * cc + 3][kr] = slot[i].w;
        }
        load_tile(min(tile + DEPTH, tiles - 1), slot);  // unconditional refill
        __syncthreads();
        if (!active || tile >= tiles) return;
        const int p0 = kfirst + tile * 64;
        int k_lo = my_first - p0, k_hi = my_pos - p0 + 1;  // this token's keys in the tile
        if (k_lo < 0) k_lo = 0;
        if (k_hi > 64) k_hi = 64;
        if (k_lo == 0 && k_hi == 64) {
            const float4 *vr = reinterpret_cast<const float4 *>(s_v[lane]);
#pragma unroll 4
            for (int k4 = 0; k4 < 16; k4++) {
                const float4 v4 = vr[k4];
                const int pk = p0 + 4 * k4 - my_first;
#pragma unroll
                for (int e = 0; e < HPW; e++) {
                    const float *pe = prow + (size_t)e * stride + pk;
                    o[e] = fmaf(pe[0], v4.x, o[e]);
                    o[e] = fmaf(pe[1], v4.y, o[e]);
                    o[e] = fmaf(pe[2], v4.z, o[e]);
                    o[e] = fmaf(pe[3], v4.w, o[e]);
                }
            }
        } else {
            for (int k = k_lo; k < k_hi; k++) {
                const float vv = s_v[lane][k];
                const int pk = p0 + k - my_first;
#pragma unroll
                for (int e = 0; e < HPW; e++) o[e] = fmaf(prow[(size_t)e * stride + pk], vv, o[e]);
            }
        }
    };
    for (int tile = 0; tile < tiles; tile += DEPTH) {
#pragma unroll
        for (int s = 0; s < DEPTH; s++) step(tile + s, ring[s]);
    }
    if (active) {
#pragma unroll
        for (int e = 0; e < HPW; e++) out[((size_t)my_t * 8 + h0 + e) * HD + d0 + lane] = o[e];
    }
}

int launch_attend_reference(hipStream_t s, float *out, const float *q, const float *key_cache,
                            const float *value_cache, int cache_len, int head_dim, int heads,
                            int full, int start_pos, size_t n) {
    if (!n) return G4_OK;
    if (heads != 8) return set_error(G4_ERR_ARG, "reference-order attention needs 8 query heads");
    const int last_pos = start_pos + (int)n - 1;
    const int max_keys = full ? last_pos + 1 : (last_pos + 1 < G4_WINDOW ? last_pos + 1 : G4_WINDOW);
    const size_t stride = ((size_t)max_keys + 63) & ~(size_t)63;
    int rc = scratch_reserve(0, n * heads * stride * sizeof(float));
    if (rc) return rc;
    float *scores = scratch().attn;
    // keys spanned by one block of tokens: its first token's window start to
    // its last token
    auto span = [&](int tq) {
        const int tokens = (int)n < tq ? (int)n : tq;
        const int widest = full ? last_pos + 1 : G4_WINDOW - 1 + tokens;
        return widest < last_pos + 1 ? widest : last_pos + 1;
    };
    const unsigned nn = (unsigned)n;
    if (head_dim == 256) {
        constexpr int TQ = 6;
        dim3 grid((unsigned)((span(TQ) + 63) / 64), (nn + TQ - 1) / TQ);
        hipLaunchKernelGGL((k_attn_scores<256, TQ>), grid, dim3(256), 0, s, q, key_cache, cache_len,
                           full, start_pos, (int)n, stride, scores);
    } else {
        constexpr int TQ = 3;
        dim3 grid((unsigned)((span(TQ) + 63) / 64), (nn + TQ - 1) / TQ);
        hipLaunchKernelGGL((k_attn_scores<512, TQ>), grid, dim3(256), 0, s, q, key_cache, cache_len,
                           full, start_pos, (int)n, stride, scores);
    }
    hipLaunchKernelGGL(k_attn_softmax_reference, dim3((unsigned)heads, nn), dim3(64), 0, s, scores,
                       heads, full, start_pos, stride);
    const unsigned slices = (unsigned)(head_dim / 64);
    if (n <= 4) {  // decode: one token per block, 2 heads per lane, deep prefetch
        dim3 grid(slices, nn);
        if (head_dim == 256)
            hipLaunchKernelGGL((k_attn_values<256, 4, 2, 8>), grid, dim3(256), 0, s, out, scores,
                               value_cache, cache_len, full, start_pos, (int)n, stride);
        else
            hipLaunchKernelGGL((k_attn_values<512, 4, 2, 8>), grid, dim3(256), 0, s, out, scores,
                               value_cache, cache_len, full, start_pos, (int)n, stride);
    } else {  // prefill: 16 tokens x 8 heads per block share each V tile
        dim3 grid(slices, (nn + 15) / 16);
        if (head_dim == 256)
            hipLaunchKernelGGL((k_attn_values<256, 16, 8, 2>), grid, dim3(1024), 0, s, out, scores,
                               value_cache, cache_len, full, start_pos, (int)n, stride);
        else
            hipLaunchKernelGGL((k_attn_values<512, 16, 8, 2>), grid, dim3(1024), 0, s, out, scores,
                               value_cache, cache_len, full, start_pos, (int)n, stride);
    }
    return G4_OK;
}

int launch_attend(hipStream_t s, float *out, const float *q, const float *key_cache,
                  const float *value_cache, int cache_len, int head_dim, int heads, int full,
                  int start_pos, size_t n) {
    if (g_order == G4_ORDER_REFERENCE)
        return launch_attend_reference(s, out, q, key_cache, value_cache, cache_len, head_dim,
                                       heads, full, start_pos, n);
    return launch_attend_parallel(s, out, q, key_cache, value_cache, cache_len, head_dim, heads,
                                  full, start_pos, n);
}

}  // namespace g4

extern "C" int g4_set_order(int order) {
    if (order != G4_ORDER_REFERENCE && order != G4_ORDER_PARALLEL) {
        g4::set_error(G4_ERR_ARG, "g4_set_order: unknown order %d", order);
        return -1;
    }
    const int previous = g4::g_order;
    g4::g_order = order;
    return previous;
}

extern "C" int g4_softmax(void *stream, float *values, int count, size_t rows) {
    G4_CHECK(values && count > 0, "g4_softmax: bad arguments");
    if (!rows) return G4_OK;
    hipLaunchKernelGGL(g4::k_softmax_rows, dim3((unsigned)rows), dim3(64), 0, (hipStream_t)stream,
                       values, count, (size_t)count);
    G4_HIP(hipGetLastError());
    return G4_OK;
}
