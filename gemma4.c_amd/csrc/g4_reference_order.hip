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
            const float4 *sq = reinterpret_cast<const float4 *>(s_sq[wave]);
            for (int i = 0; i < width / 4; i++) {
                const float4 q = sq[i];
                sum += q.x;
                sum += q.y;
                sum += q.z;
                sum += q.w;
            }
            for (int i = width & ~3; i < width; i++) sum += s_sq[wave][i];
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
// lanes per key, lane m an fma chain over channels m, m+16, ..., then the fixed
// tree.  scores[(t * heads + h) * stride + k], k relative to the first key.
template <int HD>
__global__ __launch_bounds__(256) void k_attn_scores(const float *__restrict__ q,
                                                     const float *__restrict__ key_cache,
                                                     int cache_len, int heads, int full,
                                                     int start_pos, size_t stride,
                                                     float *__restrict__ scores) {
    __shared__ float s_q[8][HD];
    const int t = blockIdx.y;
    const int pos = start_pos + t, first = first_visible(pos, full), keys = pos + 1 - first;
    const int k0 = blockIdx.x * 64;
    if (k0 >= keys) return;
    const int kn = keys - k0 < 64 ? keys - k0 : 64;
    const int mask = cache_len - 1, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float *qt = q + (size_t)t * heads * HD;
    for (int i = tid; i < heads * HD; i += 256) s_q[i / HD][i % HD] = qt[i];
    __syncthreads();
    const int m16 = lane & 15, kg = lane >> 4;
    for (int kk = wave * 4 + kg; kk < kn; kk += 16) {
        const float *kr = key_cache + (size_t)((first + k0 + kk) & mask) * HD;
        float acc[8];
#pragma unroll
        for (int h = 0; h < 8; h++) acc[h] = 0.0f;
        for (int j = m16; j < HD; j += 16) {
            const float kv = kr[j];
#pragma unroll
            for (int h = 0; h < 8; h++)
                if (h < heads) acc[h] = fmaf(s_q[h][j], kv, acc[h]);
        }
#pragma unroll
        for (int h = 0; h < 8; h++) {
            float v = acc[h];
            v += __shfl_down(v, 8, 16);
            v += __shfl_down(v, 4, 16);
            v += __shfl_down(v, 2, 16);
            v += __shfl_down(v, 1, 16);
            if (m16 == 0 && h < heads) scores[((size_t)t * heads + h) * stride + k0 + kk] = v;
        }
    }
}

// Softmax of one row in place (gemma4.c:400-408), by one wave.  Per block of
// 64 values: a prefix-max scan gives each value the maximum m seen before it;
// a value above m contributes expf(m - v) as a rescale factor (the sum becomes
// s * e + 1), any other value expf(v - m) as an addend.  Lane 0 applies the
// recurrence in index order.  Then p = expf(v - max) / sum.
__device__ void softmax_row_reference(float *v, int count, float *s_e, int *s_new) {
    const int lane = threadIdx.x & 63;
    float carry = v[0];  // max = values[0], sum = 1 (gemma4.c:401)
    float sum = 1.0f;
    for (int base = 1; base < count; base += 64) {
        const int j = base + lane;
        const float x = j < count ? v[j] : -INFINITY;
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
            if (!any_new) {
                for (int jj = 0; jj < n; jj++) sum += s_e[jj];
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
// per output channel; the probabilities are wave-uniform.
__global__ __launch_bounds__(64) void k_attn_values_reference(float *__restrict__ out,
                                                              const float *__restrict__ probs,
                                                              const float *__restrict__ value_cache,
                                                              int cache_len, int head_dim, int heads,
                                                              int full, int start_pos, size_t stride) {
    const int d = blockIdx.x * 64 + threadIdx.x, h = blockIdx.y, t = blockIdx.z;
    const int pos = start_pos + t, first = first_visible(pos, full), keys = pos + 1 - first;
    const int mask = cache_len - 1;
    const float *p = probs + ((size_t)t * heads + h) * stride;
    const float *vc = value_cache + d;
    float o = 0.0f;
    int k = 0;
    for (; k + 4 <= keys; k += 4) {
        const float v0 = vc[(size_t)((first + k) & mask) * head_dim];
        const float v1 = vc[(size_t)((first + k + 1) & mask) * head_dim];
        const float v2 = vc[(size_t)((first + k + 2) & mask) * head_dim];
        const float v3 = vc[(size_t)((first + k + 3) & mask) * head_dim];
        o = fmaf(p[k], v0, o);
        o = fmaf(p[k + 1], v1, o);
        o = fmaf(p[k + 2], v2, o);
        o = fmaf(p[k + 3], v3, o);
    }
    for (; k < keys; k++) o = fmaf(p[k], vc[(size_t)((first + k) & mask) * head_dim], o);
    out[((size_t)t * heads + h) * head_dim + d] = o;
}

int launch_attend_reference(hipStream_t s, float *out, const float *q, const float *key_cache,
                            const float *value_cache, int cache_len, int head_dim, int heads,
                            int full, int start_pos, size_t n) {
    if (!n) return G4_OK;
    const int last_pos = start_pos + (int)n - 1;
    const int max_keys = full ? last_pos + 1 : (last_pos + 1 < G4_WINDOW ? last_pos + 1 : G4_WINDOW);
    const size_t stride = ((size_t)max_keys + 63) & ~(size_t)63;
    int rc = scratch_reserve(0, 0, n * heads * stride * sizeof(float));
    if (rc) return rc;
    float *scores = scratch().attn;
    const dim3 grid1((unsigned)((max_keys + 63) / 64), (unsigned)n);
    if (head_dim == 256)
        hipLaunchKernelGGL(k_attn_scores<256>, grid1, dim3(256), 0, s, q, key_cache, cache_len,
                           heads, full, start_pos, stride, scores);
    else
        hipLaunchKernelGGL(k_attn_scores<512>, grid1, dim3(256), 0, s, q, key_cache, cache_len,
                           heads, full, start_pos, stride, scores);
    hipLaunchKernelGGL(k_attn_softmax_reference, dim3((unsigned)heads, (unsigned)n), dim3(64), 0, s,
                       scores, heads, full, start_pos, stride);
    hipLaunchKernelGGL(k_attn_values_reference, dim3((unsigned)(head_dim / 64), (unsigned)heads, (unsigned)n),
                       dim3(64), 0, s, out, scores, value_cache, cache_len, head_dim, heads, full,
                       start_pos, stride);
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
