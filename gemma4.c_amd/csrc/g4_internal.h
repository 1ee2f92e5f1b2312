// g4_internal.h -- shared between the HIP translation units of libg4.so.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "g4.h"

namespace g4 {

// ---- errors ---------------------------------------------------------------

// Records a message for g4_last_error() and returns `status`.
int set_error(int status, const char *fmt, ...);

#define G4_HIP(call)                                                                    \
    do {                                                                                \
        hipError_t e_ = (call);                                                         \
        if (e_ != hipSuccess)                                                           \
            return ::g4::set_error(G4_ERR_DEVICE, "%s: %s (%s:%d)", #call,              \
                                   hipGetErrorString(e_), __FILE__, __LINE__);          \
    } while (0)

#define G4_CHECK(cond, ...)                                                             \
    do {                                                                                \
        if (!(cond)) return ::g4::set_error(G4_ERR_ARG, __VA_ARGS__);                   \
    } while (0)

// Returns a nonzero status from a call that already recorded its message.
#define G4_TRY(x)                                                                       \
    do {                                                                                \
        int rc_ = (x);                                                                  \
        if (rc_) return rc_;                                                            \
    } while (0)

// ---- device helpers ---------------------------------------------------------

__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
    return __half2float(__ushort_as_half(h));  // exact
}

// The reference's table GELU (gemma4.c:319-327): linear interpolation inside
// (lower, upper), table[0] at or below lower, identity at or above upper (and
// NaN for NaN).  Branch-free: both table loads are issued for every x, at an
// index clamped into the table, so that the loads of many lookups go out
// together instead of one branch -- and one wait -- per lookup.
__device__ __forceinline__ float gelu_table_lookup(float x, const float *table, int size,
                                                   float lower, float upper) {
    const float scale = (float)(size - 1) / (upper - lower);
    // inside (lower, upper) xc == x: the position and index are the reference's
    const float xc = fminf(fmaxf(x, lower), upper);  // NaN -> lower
    const float position = (xc - lower) * scale;     // 0 .. size - 1
    const int index = (int)position;
    const int at = min(index, size - 2);
    const float t0 = table[at], t1 = table[at + 1];  // t0 = table[0] for x <= lower
    const float fraction = position - (float)index;
    // x just below `upper` can round to position == size - 1 (x + 8 -> 16);
    // the fraction is then 0 and the reference's result is table[size - 1]
    const float inside = index >= size - 1 ? t1 : t0 + fraction * (t1 - t0);
    return x <= lower ? t0 : (x >= upper || x != x) ? x : inside;
}

// The exact int32 group dots of one packed 1 KB weight tile (16 rows x 64
// columns, byte (chunk c, row r, j) at c*64 + r*4 + j) against M activation
// rows.  Lane l holds the 16-byte unit l (chunk l/4, rows 4(l%4)..+3) and
// x4[m], row m's activation dword for chunk l/4.  Four v_dot4_i32_i8 give the
// lane's partial dots; a transposing butterfly over the 16 lanes that share
// l%4 leaves the dot of row 4(l%4) + 2 b2 + b3 (b2, b3 = bits 2, 3 of l) in
// lanes 0..15.
template <int M>
__device__ __forceinline__ void gemv_group_dots(const uint4 t, const int (&x4)[M], int b2, int b3,
                                                int (&d)[M]) {
#pragma unroll
    for (int m = 0; m < M; m++) {
        const int p0 = __builtin_amdgcn_sdot4((int)t.x, x4[m], 0, false);
        const int p1 = __builtin_amdgcn_sdot4((int)t.y, x4[m], 0, false);
        const int p2 = __builtin_amdgcn_sdot4((int)t.z, x4[m], 0, false);
        const int p3 = __builtin_amdgcn_sdot4((int)t.w, x4[m], 0, false);
        int k0 = b2 ? p2 : p0, k1 = b2 ? p3 : p1;
        const int s0 = b2 ? p0 : p2, s1 = b2 ? p1 : p3;
        k0 += __shfl_xor(s0, 4);
        k1 += __shfl_xor(s1, 4);
        int kk = b3 ? k1 : k0;
        const int ss = b3 ? k0 : k1;
        kk += __shfl_xor(ss, 8);
        kk += __shfl_xor(kk, 16);
        kk += __shfl_xor(kk, 32);
        d[m] = kk;
    }
}

// ---- scratch owned by the library ------------------------------------------

// Device scratch for split-K matmul dot products and attention partials or
// scores.  Grows on demand (allocation happens outside any kernel sequence
// that a caller might capture).
struct Scratch {
    int32_t *dots = nullptr;  // split-K exact group dot products
    size_t dots_bytes = 0;
    float *attn = nullptr;    // attention partials (m, l, o per chunk) or scores
    size_t attn_bytes = 0;
    unsigned generation = 0;  // bumped whenever a buffer moves (captured graphs hold the old one)
};
Scratch &scratch();
int scratch_reserve(size_t dots_bytes, size_t attn_bytes);
// Frees both buffers (after the device has finished with them); the next
// reservation allocates afresh and bumps the generation.
void scratch_release();
// Frees the per-op attention layer's intermediate buffers (g4_attention_layer).
void layer_buffers_release();

// ---- launchers (asynchronous on `stream`; shapes validated by callers) -------

// gemma4.c:265-279
void launch_quantize(hipStream_t s, int8_t *q, float *scales, const float *x, size_t groups);

// gemma4.c:257-262; rows <= 8 takes the split-K GEMV, larger the MFMA GEMM.
// out row stride is out_stride (>= N).
int launch_matmul(hipStream_t s, float *out, size_t out_stride, const int8_t *xq,
                  const float *xs, const int8_t *w, const uint16_t *ws, int n_out, int k,
                  int rows);

// Reduction order of rmsnorm and attention (g4_set_order).
int order();

// gemma4.c:360-373 (weight may be null); dispatches on order().
void launch_rmsnorm(hipStream_t s, float *out, const float *in, const float *weight, int width,
                    float eps, size_t rows);
void launch_rmsnorm_parallel(hipStream_t s, float *out, const float *in, const float *weight,
                             int width, float eps, size_t rows);
void launch_rmsnorm_reference(hipStream_t s, float *out, const float *in, const float *weight,
                              int width, float eps, size_t rows);
// gemma4.c:375-378
void launch_add_and_scale(hipStream_t s, float *out, const float *add, size_t n, float scale);
// Fused row tail for hidden rows of 1536, reference order (see k_row_tail):
// optional rmsnorm of h, residual = (residual + h') * scale, optional rmsnorm
// of the residual, optional quantize; y (may be null) receives the last value.
// Supported flag sets: (1,1,1,1), (1,1,0,1), (1,1,0,0), (0,0,1,1).
void launch_row_tail(hipStream_t s, const float *h, const float *w_in, float *residual, float scale,
                     const float *w_out, float *y, int8_t *q8, float *qs, float eps, size_t rows,
                     int norm_in, int add, int norm_out, int quant);
// Position-dependent launchers take start_pos and pos_dev: when pos_dev is
// non-null the kernels read the position from that device int instead (so a
// captured decode graph can be replayed at every position), and the grid no
// longer depends on the position.
// gemma4.c:381-398 (rows of v are heads*head_dim wide)
void launch_rope(hipStream_t s, const float *cosines, const float *sines, int pairs, float *v,
                 int heads, int head_dim, int start_pos, const int *pos_dev, size_t n);
// gemma4.c:310-331
// One token's products (k_gemv_tail): up to three matrices on one input,
// GELU epilogues that also write the next product's quantized input.
struct GemvMat {
    const int8_t *w;
    const uint16_t *ws;
    float *out;
    int strips;  // output rows / 16
};
struct GemvJob {
    GemvMat m[3];
    int count;
    const float *mul;  // EPI_GELU_MUL
    const float *gelu_table;
    int gelu_size;
    float gelu_lower, gelu_upper;
    int8_t *q_out;  // GELU epilogues: the output, quantized
    float *qs_out;
    int k;
};
enum { EPI_PLAIN = 0, EPI_GELU_PAIR = 1, EPI_GELU_MUL = 2 };
// The row tail that feeds a decode product (k_row_tail's arithmetic for one
// 1536-wide row), run inside the product's launch (k_gemv_tail).
struct RowTailJob {
    const float *h;        // the sublayer's output (tails that add)
    const float *w_in;     // its norm weight
    const float *res_in;   // the residual before the add (read by every block)
    float *res_out;        // after it (written by block 0; must differ from res_in)
    float scale;           // residual = (residual + norm(h)) * scale
    const float *w_out;    // the norm of the updated residual (tails 1, 3)
    float eps;
};
// tail 1: norm h, add, norm, quantize; 2: norm h, add, quantize the residual;
// 3: norm the residual, quantize.  K must be 1536.  epi/W pairs with a kernel:
// EPI_PLAIN with tails 1, 2, 3; EPI_GELU_PAIR with 1; EPI_GELU_MUL with 2.
int launch_gemv_tail(hipStream_t s, const GemvJob &job, int epi, const RowTailJob &tj, int tail);

// One token's product of K = 256 whose input is quantize(gelu(a) * b)
// (gemma4.c:309-331 then 265-279; b = the per-layer input), computed by the
// product's blocks themselves (k_gemv1).  Returns G4_ERR_ARG for other K.
int launch_gemv_gelu(hipStream_t s, float *out, const float *a, const float *b, const float *gelu_table,
                     int gelu_size, float gelu_lower, float gelu_upper, const int8_t *w, const uint16_t *ws,
                     int n_out, int k);

// Prefill products with a GELU epilogue (k_gemm_dma<EPI_GELU_*>): the output
// is written quantized only (q_out [rows][n_out], qs_out [rows][n_out / 64]).
struct GemmEpilogue {
    const int8_t *w2;     // EPI_GELU_PAIR: the second operand (up) and its scales
    const uint16_t *ws2;
    const float *mul;     // EPI_GELU_MUL: mul[m * mul_stride + n]
    size_t mul_stride;
    const float *gelu_table;
    int gelu_size;
    float gelu_lower, gelu_upper;
    int8_t *q_out;
    float *qs_out;
    // EPI_PLAIN with up to two more products of the same input (q, k, v):
    // column blocks [0, cols[0]) are the launch's own matrix, the next
    // cols[1] matrix 1, the next cols[2] matrix 2
    int cols[3];
    const int8_t *gw[2];
    const uint16_t *gws[2];
    float *gout[2];
    size_t gstride[2];
    int gn[2];
};
// Returns G4_ERR_ARG (and launches nothing) when the shape does not fit the
// fused kernel (rows <= 8, K not a multiple of 512, N not of 64).
// Up to three products of the same many-row input in one launch (K equal,
// groups % 8 == 0, rows > 8): out[i] = x W[i]^T at out_stride[i].  Returns
// G4_ERR_ARG (and launches nothing) when they do not fit.
int launch_matmul_group(hipStream_t s, const int8_t *xq, const float *xs, int rows, int k, int count,
                        const int8_t *const *w, const uint16_t *const *ws, float *const *out,
                        const size_t *out_stride, const int *n_out);
int launch_matmul_gelu(hipStream_t s, const int8_t *xq, const float *xs, const int8_t *w,
                       const uint16_t *ws, int n_out, int k, int rows, int epi,
                       const GemmEpilogue &ep);

void launch_geglu(hipStream_t s, float *gate, const float *up, int rows, int width,
                  int up_stride, const float *table, int table_size, float lower, float upper);
// gemma4.c:337-358
// Tokens outside [0, table_rows) produce NaN rows instead of reading outside.
void launch_embedding(hipStream_t s, float *out, const int8_t *table, const uint16_t *scales,
                      int width, int table_rows, const int *tokens, size_t n, float multiplier);
// A device buffer the caller owns, used by attention in place of the
// library's growing scratch (the allocation-free entry point): a call that
// needs more than `bytes` fails with G4_ERR_ARG before it launches anything.
struct FixedScratch {
    void *ptr;
    size_t bytes;
};
// gemma4.c:443-456: attention over a ring cache; dispatches on order().
// pos_dev requires reference order and n == 1.
// With q8 set, the output is also written quantized (k_quantize's groups).
int launch_attend(hipStream_t s, float *out, const float *q, const float *key_cache,
                  const float *value_cache, int cache_len, int head_dim, int heads, int full,
                  int start_pos, const int *pos_dev, size_t n, int8_t *q8 = nullptr,
                  float *qs = nullptr, const FixedScratch *fixed = nullptr);
// Scratch bytes launch_attend needs for n query rows (8 heads, head_dim <= 512)
// whose last position is last_pos, in the current summation order.
size_t attend_scratch_bytes(size_t n, int last_pos);
// Device bytes of the split softmax's terms, flags and per-row results for
// `rows` decode rows of `stride` values (they follow the scores in the
// attention scratch).  Decode rows longer than kSoftmaxSplitMin take the split.
constexpr int kSoftmaxSplitMin = 8192;
size_t softmax_split_bytes(size_t rows, size_t stride);
int launch_attend_parallel(hipStream_t s, float *out, const float *q, const float *key_cache,
                           const float *value_cache, int cache_len, int head_dim, int heads,
                           int full, int start_pos, size_t n, const FixedScratch *fixed = nullptr);
int launch_attend_reference(hipStream_t s, float *out, const float *q, const float *key_cache,
                            const float *value_cache, int cache_len, int head_dim, int heads,
                            int full, int start_pos, const int *pos_dev, size_t n,
                            int8_t *q8 = nullptr, float *qs = nullptr,
                            const FixedScratch *fixed = nullptr);
// Argument checks of g4_attend (shared by its allocation-free variant).
int check_attend_args(const char *who, float *out, const float *q, const float *key_cache,
                      const float *value_cache, int cache_len, int head_dim, int heads,
                      int full_attention, int start_pos, size_t n);
// Fused tail of the K/V projections (gemma4.c:437-440): rmsnorm+rope of the n
// new keys and rmsnorm of the new values, written into the rings at
// (start_pos + t) & (cache_len - 1).
void launch_kv_finish(hipStream_t s, float *key_cache, float *value_cache, const float *k_new,
                      const float *v_new, const float *k_norm, const float *cosines,
                      const float *sines, int pairs, int head_dim, int cache_len, int start_pos,
                      const int *pos_dev, size_t n);
// Reference order, one launch for the row-local tail of the attention
// projections (gemma4.c:427-428, 437-440): rmsnorm + RoPE of every query head
// in place, and, when k_new is set, launch_kv_finish's work on the new key and
// value.  head_dim 256 or 512.
void launch_qkv_finish(hipStream_t s, float *q, int heads, const float *q_norm, const float *k_new,
                       const float *v_new, const float *k_norm, float *key_cache, float *value_cache,
                       const float *cosines, const float *sines, int pairs, int head_dim,
                       int cache_len, int start_pos, const int *pos_dev, size_t n);
// gemma4.c:518-519: 30 * tanh(x / 30) in place.
void launch_softcap(hipStream_t s, float *x, size_t n);
// First index of the maximum (gemma4.c:537-541) of each of `rows` rows.
void launch_argmax(hipStream_t s, int *out, const float *x, size_t rows, size_t width);
// sample() (gemma4.c:536-561) over `vocab` device logits; *result points into
// the scratch buffer: [0] the token, [1] the advanced generator state.
int launch_sample(hipStream_t s, const float *logits, int vocab, float temperature, uint64_t state,
                  uint64_t **result);
// Copies that result back (synchronizing the stream); the state only when
// temperature > 0 (the reference draws only then).
int finish_sample(hipStream_t s, const uint64_t *result, float temperature, uint64_t *rng_state,
                  int *out_token);

}  // namespace g4
