// g4_kernels.hip -- gfx950 kernels of the W8A8 forward path and the per-op
// entry points of include/g4.h.
//
// Arithmetic contract (parity with gemma4.c):
//   quantize, the matmul (exact int32 group dots + the group-ordered fp32
//   fold), rope, geglu, embedding and add_and_scale are bit-identical to the
//   reference on identical inputs.  The rmsnorm, softmax and attention kernels
//   here are the parallel summation order (G4_ORDER_PARALLEL: tree sums,
//   split-KV flash decoding, the device expf), equal to within fp32 rounding;
//   the default order's kernels, bit-identical to the reference, are in
//   g4_reference_order.hip.  The final soft cap's tanhf restates the host
//   libm's method (tanhf_libm), bit-identical.
//   Built with -ffp-contract=off: a*b+c rounds twice unless fmaf() is written.
#include <float.h>
#include <math.h>

#include <type_traits>

#include "g4_internal.h"

namespace g4 {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------------------
// Scratch

static Scratch g_scratch;
Scratch &scratch() { return g_scratch; }

int scratch_reserve(size_t dots_bytes, size_t attn_bytes) {
    Scratch &s = g_scratch;
    if (dots_bytes > s.dots_bytes) {
        if (s.dots) G4_HIP(hipFree(s.dots));
        s.dots = nullptr;
        s.dots_bytes = 0;
        G4_HIP(hipMalloc(&s.dots, dots_bytes));
        s.dots_bytes = dots_bytes;
        s.generation++;
    }
    if (attn_bytes > s.attn_bytes) {
        if (s.attn) G4_HIP(hipFree(s.attn));
        s.attn = nullptr;
        s.attn_bytes = 0;
        G4_HIP(hipMalloc(&s.attn, attn_bytes));
        s.attn_bytes = attn_bytes;
        s.generation++;
    }
    return G4_OK;
}

void scratch_release() {
    Scratch &s = g_scratch;
    if (s.dots || s.attn) (void)hipDeviceSynchronize();
    if (s.dots) (void)hipFree(s.dots);
    if (s.attn) (void)hipFree(s.attn);
    s.dots = nullptr;
    s.attn = nullptr;
    s.dots_bytes = s.attn_bytes = 0;
    s.generation++;
}

// ---------------------------------------------------------------------------
// Reductions

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

// Sum over a 256-thread block; every thread gets the result.
__device__ __forceinline__ float block_sum256(float v, float *red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// ---------------------------------------------------------------------------
// Quantize (gemma4.c:265-279): 16 lanes per 64-value group, 4 values a lane.

__global__ __launch_bounds__(256) void k_quantize(int8_t *__restrict__ q, float *__restrict__ scales,
                                                  const float *__restrict__ x, size_t groups) {
    const size_t gid = (size_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    const int sub = threadIdx.x & 15;
    if (gid >= groups) return;  // all 16 lanes of a group leave together
    const float4 v = reinterpret_cast<const float4 *>(x + gid * 64)[sub];
    float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 16));
    const float scale = m / 127.0f;
    const float inverse = scale > 0.0f ? 1.0f / scale : 0.0f;
    char4 out;
    out.x = (signed char)(int)rintf(v.x * inverse);
    out.y = (signed char)(int)rintf(v.y * inverse);
    out.z = (signed char)(int)rintf(v.z * inverse);
    out.w = (signed char)(int)rintf(v.w * inverse);
    reinterpret_cast<char4 *>(q + gid * 64)[sub] = out;
    if (sub == 0) scales[gid] = scale;
}

void launch_quantize(hipStream_t s, int8_t *q, float *scales, const float *x, size_t groups) {
    if (!groups) return;
    hipLaunchKernelGGL(k_quantize, dim3((unsigned)((groups + 15) / 16)), dim3(256), 0, s, q, scales,
                       x, groups);
}

// ---------------------------------------------------------------------------
// W8A8 matmul, few rows (decode): split-K GEMV, one wave per (16-row block,
// group range).
//
// A wave reads one 1024-byte tile per group with one 16-byte load per lane:
// lane l holds chunk c = l/4 (k = 4c..4c+3) of rows 4(l%4)..4(l%4)+3.  Four
// v_dot4_i32_i8 give the lane's partial dots; a transposing butterfly over the
// 16 lanes that share l%4 leaves the exact int32 group dot of row
// 4(l%4) + 2 b2 + b3 (b2, b3 = bits 2, 3 of l) in lanes 0..15.
//
// Memory-level parallelism: a wave issues a batch of U tiles (U KB) with the
// activation dwords and weight scales interleaved in the order they are
// consumed, so each group waits only for its own loads.
//
// Fold: acc = fma((float)dot, f32(ws) * xs, acc) over groups in ascending
// order (gemma4.c:216-218), so results are bit-identical.  With one split per
// block the wave folds as it goes; with several, each wave stores its exact
// dots and k_gemv_fold (the next launch on the stream) folds all groups in
// order -- the kernel boundary orders the two, no device-scope fences needed.

// One wave's share of a one-strip GEMV: groups [g_begin, g_end) of the strip
// at `tiles` / `wscale`, for M activation rows; `emit(g, d[M], wsr, xsv[M])`
// gets each group's exact dots (in lanes 0..15, row `row`), raw weight scale
// and -- with XS -- the rows' activation scales (else zeros).  Loads for a
// batch of up to U groups are issued before any is consumed: full batches of
// U, then one batch of the n < U left (n is the same in the whole wave; the
// launchers pick U to suit a wave's share); slots past n reload the batch's
// last group -- unconditional loads, so no wait at branch joins -- and are
// not consumed.
template <int M, int U, bool XS, typename Emit>
__device__ __forceinline__ void gemv_strip_groups(const uint4 *tiles, const uint16_t *wscale, const int *xrow,
                                                  const float *xs, int k, int rows, int g_begin, int g_end,
                                                  int b2, int b3, Emit emit) {
    const int groups = k >> 6;
    auto batch = [&](int g0, int n) __attribute__((always_inline)) {
        uint4 t[U];
        int x4[U][M];
        uint16_t wsr[U];
        float xsv[U][M];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int gu = g0 + min(u, n - 1);
            t[u] = tiles[(size_t)gu * 64];
#pragma unroll
            for (int m = 0; m < M; m++) {  // rows past `rows` reread the last row (unused)
                const int mm = min(m, rows - 1);
                x4[u][m] = xrow[((size_t)mm * k + (size_t)gu * 64) >> 2];
                xsv[u][m] = XS ? xs[(size_t)mm * groups + gu] : 0.0f;
            }
            wsr[u] = wscale[gu * 16];
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (u < n) {
                int d[M];
                gemv_group_dots<M>(t[u], x4[u], b2, b3, d);
                emit(g0 + u, d, wsr[u], xsv[u]);
            }
        }
    };
    int g = g_begin;
    for (; g + U <= g_end; g += U) batch(g, U);
    if (g < g_end) batch(g, g_end - g);
}

// Batch size for a wave's share of `count` groups: the fewest batches of at
// most `cap`, each rounded up to a multiple of 4.
inline int gemv_batch(int count, int cap) {
    const int batches = (count + cap - 1) / cap;
    const int u = (count + batches - 1) / batches;
    return (u + 3) & ~3;
}

template <int M, int U>
__global__ __launch_bounds__(64) void k_gemv(float *__restrict__ out, size_t out_stride,
                                             const int8_t *__restrict__ xq,
                                             const float *__restrict__ xs,
                                             const int8_t *__restrict__ w,
                                             const uint16_t *__restrict__ ws, int k, int splits,
                                             int rows, int32_t *__restrict__ dots) {
    const int groups = k >> 6;
    const int block = blockIdx.x / splits, split = blockIdx.x % splits;
    const int g_begin = (int)((long)split * groups / splits);
    const int g_end = (int)((long)(split + 1) * groups / splits);
    const int lane = threadIdx.x;
    const int chunk = lane >> 2, b2 = (lane >> 2) & 1, b3 = (lane >> 3) & 1;
    const int row = 4 * (lane & 3) + 2 * b2 + b3;
    const uint4 *tiles = reinterpret_cast<const uint4 *>(w + (size_t)block * 16 * k) + lane;
    const uint16_t *wscale = ws + (size_t)block * groups * 16 + row;
    const int *xrow = reinterpret_cast<const int *>(xq) + chunk;

    if (splits == 1) {  // the wave folds as it goes
        float acc[M];
#pragma unroll
        for (int m = 0; m < M; m++) acc[m] = 0.0f;
        gemv_strip_groups<M, U, true>(
            tiles, wscale, xrow, xs, k, rows, g_begin, g_end, b2, b3,
            [&](int, const int (&d)[M], uint16_t wsr, const float (&xsv)[M]) __attribute__((always_inline)) {
                const float wsf = half_bits_to_float(wsr);
#pragma unroll
                for (int m = 0; m < M; m++) acc[m] = fmaf((float)d[m], wsf * xsv[m], acc[m]);
            });
        if (lane < 16) {
#pragma unroll
            for (int m = 0; m < M; m++)
                if (m < rows) out[(size_t)m * out_stride + (size_t)block * 16 + row] = acc[m];
        }
        return;
    }
    gemv_strip_groups<M, U, false>(
        tiles, wscale, xrow, xs, k, rows, g_begin, g_end, b2, b3,
        [&](int gg, const int (&d)[M], uint16_t, const float (&)[M]) __attribute__((always_inline)) {
            if (lane < 16) {
#pragma unroll
                for (int m = 0; m < M; m++) dots[(((size_t)block * groups + gg) * M + m) * 16 + row] = d[m];
            }
        });
}

// The in-order fold of G groups for one output from LDS rows (16-byte
// aligned, readable up to the next multiple of 4 plus 4): the exact dots `d`,
// the weight scales `w` (fp16 widened to fp32, exact) and the activation
// scales `x`; c = w * x is the reference's scale product (one rounding) and
// acc = fma(d, c, acc) its fold step.  Quads are read one quad ahead of the
// fma chain, so the chain never waits on LDS.
__device__ __forceinline__ float fold_lds_row(const float *d, const float *w, const float *x, int groups,
                                              float acc) {
    const float4 *d4 = reinterpret_cast<const float4 *>(d), *w4 = reinterpret_cast<const float4 *>(w),
                 *x4 = reinterpret_cast<const float4 *>(x);
    const int quads = groups >> 2;
    float4 dq = d4[0], wq = w4[0], xq = x4[0];
    for (int i = 0; i < quads; i++) {
        const float4 dn = d4[i + 1], wn = w4[i + 1], xn = x4[i + 1];
        acc = fmaf(dq.x, wq.x * xq.x, acc);
        acc = fmaf(dq.y, wq.y * xq.y, acc);
        acc = fmaf(dq.z, wq.z * xq.z, acc);
        acc = fmaf(dq.w, wq.w * xq.w, acc);
        dq = dn, wq = wn, xq = xn;
    }
    const int rest = groups & 3;  // the last partial quad, in dq / wq / xq now
    if (rest > 0) acc = fmaf(dq.x, wq.x * xq.x, acc);
    if (rest > 1) acc = fmaf(dq.y, wq.y * xq.y, acc);
    if (rest > 2) acc = fmaf(dq.z, wq.z * xq.z, acc);
    return acc;
}
// LDS row length (floats) for fold_lds_row over `groups` groups
__host__ __device__ constexpr int fold_row_floats(int groups) { return ((groups + 3) & ~3) + 4; }

// Few rows, split K inside one block: W = blockDim.x / 64 waves share one
// 16-row weight strip, wave w taking groups [w G / W, (w + 1) G / W).  Each
// group's exact dots and weight scale go to LDS (one row per output (m, r),
// one per weight row r), the activation scales too (loaded first, stored
// after the weight loads); after one barrier, thread (m, r) folds its
// output's groups in order (the reference's order, one fma each).  No second
// kernel.  Dynamic LDS: (16 M + 16 + M) x fold_row_floats(G) floats; M x G
// <= 4 x blockDim.x.
template <int M, int U>
__global__ __launch_bounds__(1024) void k_gemv_split(float *__restrict__ out, size_t out_stride,
                                                     const int8_t *__restrict__ xq,
                                                     const float *__restrict__ xs,
                                                     const int8_t *__restrict__ w,
                                                     const uint16_t *__restrict__ ws, int k,
                                                     int rows) {
    extern __shared__ __attribute__((aligned(16))) float s_fold[];
    const int groups = k >> 6, waves = blockDim.x >> 6, gp = fold_row_floats(groups);
    float *s_d = s_fold;                         // [m][r][g]
    float *s_w = s_d + (size_t)M * 16 * gp;      // [r][g]
    float *s_x = s_w + (size_t)16 * gp;          // [m][g]
    const int block = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int g_begin = (int)((long)wave * groups / waves);
    const int g_end = (int)((long)(wave + 1) * groups / waves);
    const int chunk = lane >> 2, b2 = (lane >> 2) & 1, b3 = (lane >> 3) & 1;
    const int row = 4 * (lane & 3) + 2 * b2 + b3;
    const uint4 *tiles = reinterpret_cast<const uint4 *>(w + (size_t)block * 16 * k) + lane;
    const uint16_t *wscale = ws + (size_t)block * groups * 16 + row;
    const int *xrow = reinterpret_cast<const int *>(xq) + chunk;
    float xsv[4];  // this thread's activation scales, stored to LDS after the weight loads
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int i = min((int)threadIdx.x + j * (int)blockDim.x, M * groups - 1);
        xsv[j] = M == 1 ? xs[i] : xs[(size_t)min(i / groups, rows - 1) * groups + i % groups];
    }
    gemv_strip_groups<M, U, false>(tiles, wscale, xrow, xs, k, rows, g_begin, g_end, b2, b3,
                            [&](int gg, const int (&d)[M], uint16_t wsr, const float (&)[M]) __attribute__((always_inline)) {
                                if (lane < 16) {
#pragma unroll
                                    for (int m = 0; m < M; m++) s_d[(m * 16 + row) * gp + gg] = (float)d[m];
                                    s_w[row * gp + gg] = half_bits_to_float(wsr);
                                }
                            });
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int i = threadIdx.x + j * blockDim.x;
        if (i < M * groups) s_x[M == 1 ? i : (i / groups) * gp + i % groups] = xsv[j];
    }
    __syncthreads();
    const int tid = threadIdx.x;
    if (tid < 16 * M) {
        const int m = tid >> 4, r = tid & 15;
        const float acc = fold_lds_row(s_d + (size_t)tid * gp, s_w + (size_t)r * gp, s_x + (size_t)m * gp, groups, 0.0f);
        if (m < rows) out[(size_t)m * out_stride + (size_t)block * 16 + r] = acc;
    }
}

// One token (M = 1) with every CU streaming weight tiles.  A block covers one
// 16-row strip and GB = W * U consecutive groups of it -- all of its groups
// (SPLIT false), or one of `parts` slices of them (SPLIT true) -- and wave
// w takes U of those groups.  Each thread first loads its share of the
// block's activation dwords (and, without SPLIT, of its (group, row) weight
// and activation scales), then the wave issues its U tile loads; the dwords
// and the scales go to LDS while the tiles are in flight (vector-memory loads
// complete in order, so the staging waits only for the first loads).  The
// exact group dots (gemv_group_dots) then go to LDS, and 16 threads fold the
// strip's groups in order (gemma4.c:216-218); with SPLIT they go to dots
// [strip][group][16] and k_gemv1_fold folds them.  The scale product is the
// reference's f16(ws) * xs, one rounding.
//
// IN = GEMV_GELU_MUL (U a multiple of 4): the input is not given
// quantized but as two fp32 rows a, b; the block quantizes its own groups of
// gelu(a) * b on the way in -- geglu (gemma4.c:309-331) then quantize
// (gemma4.c:265-279), k_quantize's arithmetic, four values a thread, a
// group's 16 threads in one wave -- so the product that makes a and b needs
// no GELU epilogue.  Every block that reads a group computes the same bits.
enum { GEMV_X = 0, GEMV_GELU_MUL = 1 };
struct GemvInput {
    const float *a, *b;  // gelu(a) * b
    const float *gelu_table;
    int gelu_size;
    float gelu_lower, gelu_upper;
};

template <int W, int U, bool SPLIT, int IN = GEMV_X>
__global__ __launch_bounds__(64 * W) void k_gemv1(float *__restrict__ out, const int8_t *__restrict__ xq,
                                                  const float *__restrict__ xs,
                                                  const int8_t *__restrict__ w,
                                                  const uint16_t *__restrict__ ws, int k, int parts,
                                                  int32_t *__restrict__ dots, GemvInput in) {
    constexpr int GB = W * U, XD = (U + 3) / 4;  // groups a block; staged entries a thread
    static_assert(IN == GEMV_X || (U % 4 == 0 && !SPLIT), "GELU inputs: groups of four values, one block a strip");
    constexpr int RF = fold_row_floats(GB);  // fold rows [16][RF] (k_gemv1 without SPLIT)
    __shared__ int s_x[GB * 16];
    __shared__ __attribute__((aligned(16))) float s_d[SPLIT ? 1 : 16][SPLIT ? 4 : RF],
        s_w[SPLIT ? 1 : 16][SPLIT ? 4 : RF], s_xs[SPLIT ? 4 : RF];
    const int groups = k >> 6;
    int strip = blockIdx.x / parts, part = blockIdx.x % parts;
    if (SPLIT) {
        // the parts of strip s run on one XCD (blocks are dealt to the 8 XCDs
        // in turn): block x + 8 (parts q + p) is part p of strip 8 q + x
        // (strips % 8 == 0), so the fold kernel's block for s -- on the same
        // XCD -- finds the strip's dots in its own L2
        const int x = blockIdx.x & 7, j = blockIdx.x >> 3;
        strip = 8 * (j / parts) + x;
        part = j % parts;
    }
    const int gb0 = part * GB;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    // GB * 16 entries to stage (the block's activation dwords; without SPLIT
    // also the (group, row) weight scales and the group scales), XD a thread
    int xv[XD];
    uint16_t wsv[XD];
    float xsv[XD];
    float4 av[XD], bv[XD];
#pragma unroll
    for (int i = 0; i < XD; i++) {
        const int e = min(tid + i * 64 * W, GB * 16 - 1);
        if (IN == GEMV_X) {
            xv[i] = reinterpret_cast<const int *>(xq)[gb0 * 16 + e];
            xsv[i] = SPLIT ? 0.0f : xs[gb0 + e / 16];
        } else {
            av[i] = reinterpret_cast<const float4 *>(in.a)[gb0 * 16 + e];
            bv[i] = reinterpret_cast<const float4 *>(in.b)[gb0 * 16 + e];
        }
        wsv[i] = SPLIT ? 0 : ws[((size_t)strip * groups + gb0) * 16 + e];
    }
    const uint4 *tiles = reinterpret_cast<const uint4 *>(w + (size_t)strip * 16 * k) + lane;
    const int gw = gb0 + wave * U;
    uint4 t[U];
#pragma unroll
    for (int u = 0; u < U; u++) t[u] = tiles[(size_t)(gw + u) * 64];
    if (IN != GEMV_X) {  // dword e: values 4 e .. 4 e + 3 of the block's groups
#pragma unroll
        for (int i = 0; i < XD; i++) {
            const float va[4] = {av[i].x, av[i].y, av[i].z, av[i].w}, vb[4] = {bv[i].x, bv[i].y, bv[i].z, bv[i].w};
            float v[4], m = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                v[j] = gelu_table_lookup(va[j], in.gelu_table, in.gelu_size, in.gelu_lower, in.gelu_upper) * vb[j];
                m = fmaxf(m, fabsf(v[j]));
            }
#pragma unroll
            for (int o = 8; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 16));
            const float scale = m / 127.0f;
            const float inverse = scale > 0.0f ? 1.0f / scale : 0.0f;
            char4 q;
            q.x = (signed char)(int)rintf(v[0] * inverse);
            q.y = (signed char)(int)rintf(v[1] * inverse);
            q.z = (signed char)(int)rintf(v[2] * inverse);
            q.w = (signed char)(int)rintf(v[3] * inverse);
            xv[i] = __builtin_bit_cast(int, q);
            xsv[i] = scale;
        }
    }
#pragma unroll
    for (int i = 0; i < XD; i++) {
        const int e = tid + i * 64 * W;
        if (e < GB * 16) {
            s_x[e] = xv[i];
            if (!SPLIT) {
                s_w[e % 16][e / 16] = half_bits_to_float(wsv[i]);
                if (e % 16 == 0) s_xs[e / 16] = xsv[i];
            }
        }
    }
    __syncthreads();
    const int chunk = lane >> 2, b2 = (lane >> 2) & 1, b3 = (lane >> 3) & 1;
    const int row = 4 * (lane & 3) + 2 * b2 + b3;
#pragma unroll
    for (int u = 0; u < U; u++) {
        int d[1];
        const int x4[1] = {s_x[(wave * U + u) * 16 + chunk]};
        gemv_group_dots<1>(t[u], x4, b2, b3, d);
        if (lane < 16) {
            if (SPLIT)
                dots[((size_t)strip * groups + gw + u) * 16 + row] = d[0];
            else
                s_d[row][wave * U + u] = (float)d[0];
        }
    }
    if (SPLIT) return;
    __syncthreads();
    if (tid < 16) out[(size_t)strip * 16 + tid] = fold_lds_row(s_d[tid], s_w[tid], s_xs, GB, 0.0f);
}

// The in-order fold of k_gemv1's split dots (M = 1): one block per 16-row
// strip.  Its 256 threads load the strip's dots and weight scales (and the
// activation scales) into row-major LDS rows with all loads in flight at
// once; then 16 threads fold the groups in order (gemma4.c:216-218) with
// fold_lds_row.  G <= 256.
__global__ __launch_bounds__(256) void k_gemv1_fold(float *__restrict__ out, const int32_t *__restrict__ dots,
                                                    const float *__restrict__ xs,
                                                    const uint16_t *__restrict__ ws, int groups) {
    constexpr int RF = fold_row_floats(256);
    __shared__ __attribute__((aligned(16))) float s_d[16][RF], s_w[16][RF], s_x[RF];
    const int strip = blockIdx.x, tid = threadIdx.x;
    const int4 *d4 = reinterpret_cast<const int4 *>(dots + (size_t)strip * groups * 16);
    const uint2 *s4 = reinterpret_cast<const uint2 *>(ws + (size_t)strip * groups * 16);
    // groups * 4 units of four (group, row) entries, 256 a pass
    constexpr int P = 4;
    int4 dv[P];
    uint2 sv[P];
#pragma unroll
    for (int p = 0; p < P; p++) {
        const int i = min(tid + 256 * p, groups * 4 - 1);
        dv[p] = d4[i];
        sv[p] = s4[i];
    }
    const float xv = xs[min(tid, groups - 1)];
#pragma unroll
    for (int p = 0; p < P; p++) {
        const int i = tid + 256 * p;
        if (i < groups * 4) {
            const int g = i >> 2, r = 4 * (i & 3);
            s_d[r][g] = (float)dv[p].x, s_d[r + 1][g] = (float)dv[p].y;
            s_d[r + 2][g] = (float)dv[p].z, s_d[r + 3][g] = (float)dv[p].w;
            s_w[r][g] = half_bits_to_float((uint16_t)(sv[p].x & 0xFFFF));
            s_w[r + 1][g] = half_bits_to_float((uint16_t)(sv[p].x >> 16));
            s_w[r + 2][g] = half_bits_to_float((uint16_t)(sv[p].y & 0xFFFF));
            s_w[r + 3][g] = half_bits_to_float((uint16_t)(sv[p].y >> 16));
        }
    }
    if (tid < groups) s_x[tid] = xv;
    __syncthreads();
    if (tid < 16) out[(size_t)strip * 16 + tid] = fold_lds_row(s_d[tid], s_w[tid], s_x, groups, 0.0f);
}

// One token's product through k_gemv1 where that was measured faster than
// k_gemv / k_gemv_split (graph replay, weights rotated past the Infinity
// Cache): K = 1536 (24 groups) in one block of 12 waves x 2 groups (up to 384
// strips) or 8 waves x 3 groups (more); K = 2048 in 16 waves x 2 groups;
// K = 4096 in 16 waves x 4 groups; K = 12288 split over blocks of 8 groups
// and folded by k_gemv1_fold.  Returns false (nothing launched) for other
// shapes (K = 256 and K = 6144 among them: the older kernels are faster).
static bool launch_gemv1(hipStream_t s, float *out, const int8_t *xq, const float *xs, const int8_t *w,
                         const uint16_t *ws, int n_out, int k) {
    const int strips = n_out / 16, groups = k / 64;
    const dim3 grid((unsigned)strips);
    switch (groups) {
    case 24:
        if (strips <= 384)
            hipLaunchKernelGGL((k_gemv1<12, 2, false>), grid, dim3(768), 0, s, out, xq, xs, w, ws, k, 1, nullptr,
                               GemvInput{});
        else
            hipLaunchKernelGGL((k_gemv1<8, 3, false>), grid, dim3(512), 0, s, out, xq, xs, w, ws, k, 1, nullptr,
                               GemvInput{});
        return true;
    case 32:
        hipLaunchKernelGGL((k_gemv1<16, 2, false>), grid, dim3(1024), 0, s, out, xq, xs, w, ws, k, 1, nullptr,
                           GemvInput{});
        return true;
    case 64:
        hipLaunchKernelGGL((k_gemv1<16, 4, false>), grid, dim3(1024), 0, s, out, xq, xs, w, ws, k, 1, nullptr,
                           GemvInput{});
        return true;
    case 192: {
        if (strips % 8) return false;
        const int parts = groups / 8;
        if (scratch_reserve((size_t)n_out * groups * sizeof(int32_t), 0)) return false;
        int32_t *dots = scratch().dots;
        hipLaunchKernelGGL((k_gemv1<2, 4, true>), dim3((unsigned)(strips * parts)), dim3(128), 0, s, out, xq, xs, w,
                           ws, k, parts, dots, GemvInput{});
        hipLaunchKernelGGL(k_gemv1_fold, grid, dim3(256), 0, s, out, dots, xs, ws, groups);
        return true;
    }
    default:
        return false;
    }
}

int launch_gemv_gelu(hipStream_t s, float *out, const float *a, const float *b, const float *gelu_table,
                     int gelu_size, float gelu_lower, float gelu_upper, const int8_t *w, const uint16_t *ws,
                     int n_out, int k) {
    if (n_out <= 0 || n_out % 16 || k != 256)
        return set_error(G4_ERR_ARG, "one-token GELU product: shape %d x %d does not fit", n_out, k);
    const GemvInput in{a, b, gelu_table, gelu_size, gelu_lower, gelu_upper};
    hipLaunchKernelGGL((k_gemv1<1, 4, false, GEMV_GELU_MUL>), dim3((unsigned)(n_out / 16)), dim3(64), 0, s, out,
                       nullptr, nullptr, w, ws, k, 1, nullptr, in);
    return G4_OK;
}

// The group-ordered fold of split GEMV dots: one thread per output row.
template <int M>
__global__ __launch_bounds__(256) void k_gemv_fold(float *__restrict__ out, size_t out_stride,
                                                   const int32_t *__restrict__ dots,
                                                   const float *__restrict__ xs,
                                                   const uint16_t *__restrict__ ws, int n_out,
                                                   int groups, int rows) {
    const int n = blockIdx.x * 256 + threadIdx.x;
    if (n >= n_out) return;
    const int block = n >> 4, r = n & 15;
    const int32_t *d = dots + (size_t)block * groups * M * 16 + r;
    const uint16_t *s = ws + (size_t)block * groups * 16 + r;
    float acc[M];
#pragma unroll
    for (int m = 0; m < M; m++) acc[m] = 0.0f;
    // Loads for a batch of B groups are issued before the fma chain that
    // consumes them, so the chain is not serialized on memory latency.
    constexpr int B = 16;
    int g = 0;
    for (; g + B <= groups; g += B) {
        int dv[B][M];
        float xv[B][M];
        uint16_t sv[B];
#pragma unroll
        for (int u = 0; u < B; u++) {
            sv[u] = s[(g + u) * 16];
#pragma unroll
            for (int m = 0; m < M; m++) {
                const int mm = min(m, rows - 1);
                dv[u][m] = d[((size_t)(g + u) * M + mm) * 16];
                xv[u][m] = xs[(size_t)mm * groups + g + u];
            }
        }
#pragma unroll
        for (int u = 0; u < B; u++) {
            const float wsf = half_bits_to_float(sv[u]);
#pragma unroll
            for (int m = 0; m < M; m++)
                if (m < rows) acc[m] = fmaf((float)dv[u][m], wsf * xv[u][m], acc[m]);
        }
    }
    for (; g < groups; g++) {
        const float wsf = half_bits_to_float(s[g * 16]);
#pragma unroll
        for (int m = 0; m < M; m++)
            if (m < rows)
                acc[m] = fmaf((float)d[((size_t)g * M + m) * 16], wsf * xs[(size_t)m * groups + g], acc[m]);
    }
#pragma unroll
    for (int m = 0; m < M; m++)
        if (m < rows) out[(size_t)m * out_stride + n] = acc[m];
}

// ---------------------------------------------------------------------------
// W8A8 matmul, many rows (prefill): int8 MFMA GEMM, 64 x BN output tile per
// 256-thread block (2 x 2 waves of 32 x BN/2), one 64-deep K step per
// quantization group.
//
// v_mfma_i32_16x16x64_i8: lane l supplies 16 bytes of A row (l%16) and of B
// column (l%16), both for k-slots 16(l/16)..16(l/16)+15; output element
// (i, j) = (4(l/16)+v, l%16) comes back in lane l, register v.  Every MFMA
// covers exactly one group, so the group-ordered fp32 fold is the reference's
// (bit-identical).
//
// Pipeline: KG groups per stage, one barrier per stage.  LDS holds two
// stages (double-buffered); while the waves multiply and fold the stage in
// one buffer, the next stage (loaded from global memory during the previous
// iteration) is stored into the other and the one after it is loaded into
// registers.  Within a stage the fold of one group can overlap the MFMAs of
// the next.  The B tiles are reordered on the way into LDS from the packed
// [chunk][row][4] layout to row-major rows of 64 bytes, so each lane reads its
// B operand with one 16-byte load; rows are padded to 80 bytes.

template <int BN, int KG>
__global__ __launch_bounds__(256) void k_gemm(float *__restrict__ out, size_t out_stride,
                                              const int8_t *__restrict__ xq,
                                              const float *__restrict__ xs,
                                              const int8_t *__restrict__ w,
                                              const uint16_t *__restrict__ ws, int rows,
                                              int n_out, int k) {
    constexpr int BM = 64, NT = BN / 16, WN = BN / 2, NI = WN / 16, RS = 80;
    constexpr int BV = NT / 4;  // 16-byte B loads per thread per group
    __shared__ __attribute__((aligned(16))) int8_t s_a[2][KG][BM * RS];
    __shared__ __attribute__((aligned(16))) int8_t s_b[2][KG][BN * RS];
    __shared__ __attribute__((aligned(16))) float s_xs[2][KG][BM];
    __shared__ __attribute__((aligned(16))) float s_ws[2][KG][BN];
    const int groups = k >> 6, stages = (groups + KG - 1) / KG;
    const int m0 = blockIdx.y * BM, nb0 = blockIdx.x * NT, n_blocks = n_out >> 4;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1, q = lane >> 4, l16 = lane & 15;
    const v4i zero = {0, 0, 0, 0};

    // Rows past `rows`, tiles past n_out and groups past the last are loaded
    // from the last valid one instead (their results are never used), so
    // every load is unconditional.
    const int a_row = tid >> 2, a_part = tid & 3;
    const int8_t *a_src = xq + (size_t)min(m0 + a_row, rows - 1) * k + a_part * 16;
    const float *x_src = xs + (size_t)min(m0 + (tid & (BM - 1)), rows - 1) * groups;
    const int w_n = (tid - BM) & (BN - 1);
    const uint16_t *w_src = ws + (size_t)min(nb0 + (w_n >> 4), n_blocks - 1) * groups * 16 + (w_n & 15);

    struct Stage {
        v4i a[KG], b[KG][BV];
        float x[KG];
        uint16_t w[KG];
    };
    auto gload = [&](int st, Stage &r) {
#pragma unroll
        for (int kg = 0; kg < KG; kg++) {
            const int g = min(st * KG + kg, groups - 1);
            r.a[kg] = *reinterpret_cast<const v4i *>(a_src + g * 64);
#pragma unroll
            for (int j = 0; j < BV; j++) {
                const int idx = j * 256 + tid, t = min(nb0 + (idx >> 6), n_blocks - 1);
                r.b[kg][j] = *reinterpret_cast<const v4i *>(w + ((size_t)t * groups + g) * 1024 + (idx & 63) * 16);
            }
            r.x[kg] = x_src[g];  // every thread loads a scale; threads < BM + BN keep theirs
            r.w[kg] = w_src[g * 16];
        }
    };
    auto sstore = [&](int buf, const Stage &r) {
#pragma unroll
        for (int kg = 0; kg < KG; kg++) {
            *reinterpret_cast<v4i *>(s_a[buf][kg] + a_row * RS + a_part * 16) = r.a[kg];
#pragma unroll
            for (int j = 0; j < BV; j++) {
                const int idx = j * 256 + tid, t = idx >> 6, i = idx & 63, c = i >> 2, rq = i & 3;
#pragma unroll
                for (int jj = 0; jj < 4; jj++)
                    *reinterpret_cast<int *>(s_b[buf][kg] + (t * 16 + rq * 4 + jj) * RS + c * 4) = r.b[kg][j][jj];
            }
            if (tid < BM)
                s_xs[buf][kg][tid] = r.x[kg];
            else if (tid < BM + BN)
                s_ws[buf][kg][tid - BM] = half_bits_to_float(r.w[kg]);
        }
    };

    float acc[2][NI][4];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < NI; j++)
#pragma unroll
            for (int v = 0; v < 4; v++) acc[i][j][v] = 0.0f;

    auto compute = [&](int buf, int kg) {
        v4i a[2];
        float4 xv[2];
#pragma unroll
        for (int mi = 0; mi < 2; mi++) {
            const int r = wm * 32 + mi * 16;
            a[mi] = *reinterpret_cast<const v4i *>(s_a[buf][kg] + (r + l16) * RS + q * 16);
            xv[mi] = *reinterpret_cast<const float4 *>(&s_xs[buf][kg][r + 4 * q]);
        }
#pragma unroll
        for (int ni = 0; ni < NI; ni++) {
            const int c = wn * WN + ni * 16 + l16;
            const v4i b = *reinterpret_cast<const v4i *>(s_b[buf][kg] + c * RS + q * 16);
            const float wsf = s_ws[buf][kg][c];
#pragma unroll
            for (int mi = 0; mi < 2; mi++) {
                const v4i d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[mi], b, zero, 0, 0, 0);
                acc[mi][ni][0] = fmaf((float)d[0], wsf * xv[mi].x, acc[mi][ni][0]);
                acc[mi][ni][1] = fmaf((float)d[1], wsf * xv[mi].y, acc[mi][ni][1]);
                acc[mi][ni][2] = fmaf((float)d[2], wsf * xv[mi].z, acc[mi][ni][2]);
                acc[mi][ni][3] = fmaf((float)d[3], wsf * xv[mi].w, acc[mi][ni][3]);
            }
        }
    };

    Stage r;
    gload(0, r);
    sstore(0, r);
    gload(1, r);
    __syncthreads();
    for (int st = 0; st < stages; st++) {
        const int buf = st & 1;
#pragma unroll
        for (int kg = 0; kg < KG; kg++)
            if (st * KG + kg < groups) compute(buf, kg);  // uniform across the block
        if (st + 1 < stages) {
            sstore(buf ^ 1, r);
            gload(st + 2, r);
        }
        __syncthreads();
    }
#pragma unroll
    for (int mi = 0; mi < 2; mi++)
#pragma unroll
        for (int ni = 0; ni < NI; ni++) {
            const int col = wn * WN + ni * 16;
            if (nb0 + (col >> 4) >= n_blocks) continue;
            const size_t n = (size_t)nb0 * 16 + col + l16;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int m = m0 + wm * 32 + mi * 16 + 4 * q + v;
                if (m < rows) out[(size_t)m * out_stride + n] = acc[mi][ni][v];
            }
        }
}

// s_waitcnt immediate (gfx9 encoding) that waits until at most n vector-memory
// operations are outstanding and leaves the LDS and export counters alone:
// vmcnt bits 3:0 and 15:14, expcnt 6:4 = 7, lgkmcnt 11:8 = 15.
constexpr int waitcnt_vm(int n) { return 0x0F70 | (n & 15) | ((n >> 4) << 14); }

// Prefill W8A8 GEMM with every operand brought into LDS by the gfx950 LDS-DMA
// loads (global_load_lds): no registers hold tiles in flight, and the number
// of vector-memory instructions is kept low: each wave issues two 1-KB loads
// per group (three with a second B operand), plus one 1-KB load of scales
// every 8 groups.  Four LDS stages: group g is read while groups g + 1 ..
// g + 3 are in flight.  64 x 64 outputs per block of 4 waves (2 x 2 waves of
// 32 x 32), or of 8 waves (2 x 4 waves of 32 x 16; waves 0-3 then fetch A,
// waves 4-7 the B tiles, one load each per group), or 64 x 48 outputs per
// block of 6 waves (2 x 3 of 32 x 16; waves 0-3 fetch A, waves 4, 5 and 0 the
// three B tiles), one 64-deep K step per
// quantization group, the group-ordered fp32 fold of the reference
// (bit-identical).  Requires groups % 8 == 0.
//   A  64 rows x 64 B per group: wave w fetches rows 16w .. 16w + 15, lane L
//      the 16-byte part (L & 3) ^ ((row >> 1) & 3) of row 16w + L / 4, so the
//      parts of a row are stored XOR-swizzled and a lane's 16-byte operand
//      read (row, part q) is bank-conflict free: the LDS serves a 16-byte
//      read 8 lanes (128 bytes) a cycle, and rows r .. r + 7 then fall on 8
//      distinct 16-byte bank groups (with (row >> 2) & 3, rows r and r + 2
//      shared one: 4 conflict cycles a read, SQ_LDS_BANK_CONFLICT);
//   B  4 packed tiles per group: wave w fetches tile w; LDS slot s holds the
//      tile's 16-byte unit s ^ (4 (s / 16) & 12), so the four 4-byte reads of
//      a lane's operand are conflict free;
//   scales, per 8 groups: waves 0, 1 fetch the activation scales of groups
//      0-3, 4-7 (16 bytes per row), wave 2 the weight scales of the 4 tiles
//      (256 bytes per tile), wave 3 the second B operand's (or repeats
//      wave 2's into padding).
// k-slots: lane (l%16, l/16) covers k = 16 (l/16) + 0..15 -- for B that is
// chunks 4 (l/16) .. + 3 of weight row l%16.
// The fold takes two VALU operations per output: the int32 dot converted to
// fp32 (exact: |dot| <= 64 * 127 * 127 < 2^24) and the fma -- both 4-byte
// VOP1/VOP2 encodings (a subtraction of a 32-bit literal would be an 8-byte
// instruction, measurably slower to issue); the scale products
// xs[m] * ws[n] of the wave's four 16 x 16 tiles come from one fp32 MFMA with
// K = 1 (16x16x1, four blocks), whose products are rounded exactly as a VALU
// multiply, subnormals included.  Block b = 2 mi + ni takes its 16 row
// scales and 16 column scales from lanes 16 b .. 16 b + 15, and its result
// lands in the int8 MFMA's output layout (outputs 4 b .. 4 b + 3); a wave of
// 32 x 16 uses blocks 0 and 2.
template <int EPI, int WAVES, int NT = 4, int S = 4>
__global__ __launch_bounds__(64 * WAVES) void k_gemm_dma(float *__restrict__ out, size_t out_stride,
                                                         const int8_t *__restrict__ xq,
                                                         const float *__restrict__ xs,
                                                         const int8_t *__restrict__ w,
                                                         const uint16_t *__restrict__ ws, int rows,
                                                         int n_out, int k, GemmEpilogue ep) {
    // WAVES = 4: 2 x 2 waves of 32 x 32 outputs; WAVES = 8: 2 x 4 waves of
    // 32 x 16 (two waves a SIMD from one block, for grids of one block a CU)
    // NT = 3 (6 waves, 2 x 3 of 32 x 16): 64 x 48 tiles, so that a 1536-wide
    // product is 32 column blocks -- 256 blocks at 512 rows, one per CU
    constexpr int NWN = WAVES / 2, BM = 64, BN = 16 * NT, WN = BN / NWN, NI = WN / 16;
    constexpr int NB = EPI == EPI_GELU_PAIR ? 2 : 1;  // B operands: (gate, up) or one
    static_assert((WAVES == 4 && NT == 4) || (WAVES == 8 && NT == 4 && NB == 1) ||
                      (WAVES == 6 && NT == 3 && EPI == EPI_PLAIN),
                  "4 or 8 waves of a 64-wide tile, or 6 waves of a 48-wide plain one");
    // vector-memory loads a wave issues per group: A and B (and B2) parts
    // with 4 waves, one of A or B with 8
    constexpr int LOADS = WAVES == 4 ? 1 + NB : 1;
    struct alignas(16) Stage {
        int8_t a[BM * 64];
        int8_t b[NB][NT * 1024];
    };
    struct alignas(16) Scales {  // 8 groups
        float x[2][BM][4];          // [group / 4][row][group % 4]
        uint16_t s[2][4][8][16];    // [0]: [tile][group][row]; [1]: padding (1 KB each)
    };
    // One __shared__ object per stage: the compiler then tells a read of one
    // stage from the DMA writes still landing in the others (with one array
    // it would wait for every DMA before every LDS read).  S = 3 stages (K =
    // 1536 only) for the gate/up pair: 45.6 KB of LDS, three blocks a CU
    // instead of two, so its 768- and 1536-block grids run in whole rounds.
    static_assert(S == 4 || (S == 3 && EPI == EPI_GELU_PAIR), "4 LDS stages, or 3 for the gate/up pair");
    __shared__ Stage st0, st1, st2;
    __shared__ typename std::conditional<S == 4, Stage, char>::type st3;
    __shared__ Scales sc0, sc1;
    auto stage = [&](int i) __attribute__((always_inline)) -> Stage & {
        if constexpr (S == 4)
            return i == 0 ? st0 : i == 1 ? st1 : i == 2 ? st2 : st3;
        else
            return i == 0 ? st0 : i == 1 ? st1 : st2;
    };
    const int groups = k >> 6;
    int bx = blockIdx.x;
    if (EPI == EPI_PLAIN && bx >= ep.cols[0]) {  // a grouped launch's matrix 1 or 2 (uniform)
        const int i = bx - ep.cols[0] < ep.cols[1] ? 0 : 1;
        bx -= ep.cols[0] + (i ? ep.cols[1] : 0);
        w = ep.gw[i];
        ws = ep.gws[i];
        out = ep.gout[i];
        out_stride = ep.gstride[i];
        n_out = ep.gn[i];
    }
    const int m0 = blockIdx.y * BM, nb0 = bx * NT, n_blocks = n_out >> 4;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / NWN, wn = wave % NWN, q = lane >> 4, l16 = lane & 15;
    const v4i zero4 = {0, 0, 0, 0};
    const v16f zero16 = {};

    // DMA sources (group 0, chunk 0); the builtin wants plain void pointers
    // (8 waves: waves 0-3 fetch A, waves 4-7 B)
    const int part = wave & 3;
    const int a_row = 16 * part + (lane >> 2);
    const int8_t *a_src = xq + (size_t)min(m0 + a_row, rows - 1) * k +
                          16 * ((lane & 3) ^ ((a_row >> 1) & 3));
    const int unit = lane ^ ((lane >> 4) << 2);
    const size_t b_at = (size_t)min(nb0 + part, n_blocks - 1) * groups * 1024 + unit * 16;
    const int8_t *b_src = w + b_at, *b2_src = NB == 2 ? ep.w2 + b_at : nullptr;
    // 6 waves: the third B tile is wave 0's second load
    const int8_t *b_third = WAVES == 6 ? w + (size_t)min(nb0 + 2, n_blocks - 1) * groups * 1024 + unit * 16 : nullptr;
    const char *c_src;  // scales: 16 bytes a lane, advancing 8 groups per chunk
    size_t c_step;
    if (wave < 2) {
        c_src = (const char *)(xs + (size_t)min(m0 + lane, rows - 1) * groups + 4 * wave);
        c_step = 8 * sizeof(float);
    } else {  // wave 2: the weight scales; wave 3: the second operand's (or
              // again the first's into the padding, as do waves 4-7)
        const uint16_t *scales = NB == 2 && wave == 3 ? ep.ws2 : ws;
        c_src = (const char *)(scales + (size_t)min(nb0 + (lane >> 4), n_blocks - 1) * groups * 16 + 8 * l16);
        c_step = 8 * 16 * sizeof(uint16_t);
    }
    const int c_dst = wave < 2 ? wave * (BM * 16) : 2 * BM * 16 + min(wave - 2, 1) * 1024;
    // 6 or 8 waves: one source, step and stage offset per wave, chosen once
    const int8_t *dma_src = wave < 4 ? a_src : b_src;
    const int dma_step = wave < 4 ? 64 : 1024;
    const int dma_dst = (wave < 4 ? 0 : (int)offsetof(Stage, b)) + part * 1024;
    // third: std::true_type in wave 0 of 6 (it also loads the third B
    // tile), else std::false_type -- chosen once, around the whole loop
    auto issue = [&](int g, Stage &d, auto third) __attribute__((always_inline)) {
        g = min(g, groups - 1);  // past the end: reload the last group (never read)
        if (WAVES >= 6) {
            __builtin_amdgcn_global_load_lds((const void *)(dma_src + (size_t)g * dma_step),
                                             (void *)((char *)&d + dma_dst), 16, 0, 0);
            if constexpr (decltype(third)::value)
                __builtin_amdgcn_global_load_lds((const void *)(b_third + (size_t)g * 1024),
                                                 (void *)(d.b[0] + 2 * 1024), 16, 0, 0);
            return;
        }
        __builtin_amdgcn_global_load_lds((const void *)(a_src + g * 64), (void *)(d.a + wave * 1024), 16, 0, 0);
        __builtin_amdgcn_global_load_lds((const void *)(b_src + (size_t)g * 1024), (void *)(d.b[0] + wave * 1024), 16, 0, 0);
        if constexpr (NB == 2)
            __builtin_amdgcn_global_load_lds((const void *)(b2_src + (size_t)g * 1024), (void *)(d.b[1] + wave * 1024), 16, 0, 0);
    };
    auto issue_scales = [&](int chunk, Scales &d) __attribute__((always_inline)) {
        chunk = min(chunk, groups / 8 - 1);
        __builtin_amdgcn_global_load_lds((const void *)(c_src + (size_t)chunk * c_step),
                                         (void *)((char *)&d + c_dst), 16, 0, 0);
    };
    // LDS read addresses (loop invariant)
    int a_off[2];
#pragma unroll
    for (int mi = 0; mi < 2; mi++) {
        const int r = wm * 32 + mi * 16 + l16;
        a_off[mi] = r * 64 + 16 * (q ^ ((r >> 1) & 3));
    }
    int b_off[NI][4];
#pragma unroll
    for (int ni = 0; ni < NI; ni++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            // chunk c = 4q + i of row l16 is global unit u = 4c + l16 / 4,
            // stored at slot u ^ (4 (u / 16) & 12)
            const int u = 4 * (4 * q + i) + (l16 >> 2), slot = u ^ ((u >> 4) << 2);
            b_off[ni][i] = (wn * NI + ni) * 1024 + slot * 16 + (l16 & 3) * 4;
        }

    float acc[NB][2][NI][4];
#pragma unroll
    for (int o = 0; o < NB; o++)
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < NI; j++)
#pragma unroll
                for (int v = 0; v < 4; v++) acc[o][i][j][v] = 0.0f;

    // A group's MFMAs are issued together into their own registers and
    // folded one step later, while the next group's MFMAs run: the fold never
    // waits on a fresh MFMA result.  The fetch only issues LDS reads (the
    // weight scale stays raw fp16 bits until the multiply step converts it).
    // (with NI = 1 only its blocks 0 and 2 are used)
    struct Dots {
        v4i d[NB][2][NI];  // the exact int32 group dots
        v16f c[NB];        // xs * ws, tile (mi, ni) at outputs 4 (2 mi + ni) ..
    };
    struct Frags {
        v4i a[2], b[NB][NI];
        float xs;          // row scale of lane l's block (tile row l / 32)
        uint16_t ws[NB];   // column scale of lane l's block (tile column (l / 16) % 2)
    };
    const int xs_row = wm * 32 + (lane >> 5) * 16 + l16;
    const int ws_tile = NI == 2 ? wn * NI + ((lane >> 4) & 1) : wn;
    auto fetch = [&](const Stage &d, const Scales &s, int j, Frags &f) __attribute__((always_inline)) {
#pragma unroll
        for (int mi = 0; mi < 2; mi++) f.a[mi] = *reinterpret_cast<const v4i *>(d.a + a_off[mi]);
        f.xs = s.x[j >> 2][xs_row][j & 3];
#pragma unroll
        for (int ob = 0; ob < NB; ob++) {
#pragma unroll
            for (int ni = 0; ni < NI; ni++)
#pragma unroll
                for (int i = 0; i < 4; i++) f.b[ob][ni][i] = *reinterpret_cast<const int *>(d.b[ob] + b_off[ni][i]);
            f.ws[ob] = s.s[ob][ws_tile][j][l16];
        }
    };
    auto multiply = [&](const Frags &f, Dots &o) __attribute__((always_inline)) {
#pragma unroll
        for (int ob = 0; ob < NB; ob++) {
#pragma unroll
            for (int ni = 0; ni < NI; ni++)
#pragma unroll
                for (int mi = 0; mi < 2; mi++)
                    o.d[ob][mi][ni] = __builtin_amdgcn_mfma_i32_16x16x64_i8(f.a[mi], f.b[ob][ni], zero4, 0, 0, 0);
            o.c[ob] = __builtin_amdgcn_mfma_f32_16x16x1f32(f.xs, half_bits_to_float(f.ws[ob]), zero16, 0, 0, 0);
        }
    };
    auto fold = [&](const Dots &o) __attribute__((always_inline)) {
#pragma unroll
        for (int ob = 0; ob < NB; ob++)
#pragma unroll
            for (int ni = 0; ni < NI; ni++)
#pragma unroll
                for (int mi = 0; mi < 2; mi++)
#pragma unroll
                    for (int v = 0; v < 4; v++)
                        acc[ob][mi][ni][v] = fmaf((float)o.d[ob][mi][ni][v],
                                                  o.c[ob][4 * (2 * mi + ni) + v], acc[ob][mi][ni][v]);
    };

    // Step g (j = g % 8): wait until group g (and its chunk's scales) has
    // landed -- groups g + 1 .. g + S - 2 may still be in flight -- and let
    // the barrier publish it; then issue group g + S - 1 into the stage of
    // group g - 1 (every wave finished reading it before the barrier), plus
    // the next chunk's scales when g + S - 1 starts one; read group g's
    // operands, fold group g - 1 and issue group g's MFMAs.
    auto step = [&](int g, int j, Stage &fill, const Stage &use, const Scales &sc_use,
                    Scales &sc_fill, Dots &cur, const Dots &prev, auto third) __attribute__((always_inline)) {
        // loads of groups g + 1 .. g + S - 2
        constexpr int in_flight = (S - 2) * (LOADS + (decltype(third)::value ? 1 : 0));
        // the next chunk's scales (issued right after its first group) are
        // also in flight once that group is among g + 1 .. g + S - 2
        if (j + S - 2 >= 8)
            __builtin_amdgcn_s_waitcnt(waitcnt_vm(in_flight + 1));
        else
            __builtin_amdgcn_s_waitcnt(waitcnt_vm(in_flight));
        __builtin_amdgcn_s_barrier();
        issue(g + S - 1, fill, third);
        if (j == (9 - S) % 8) issue_scales(g / 8 + 1, sc_fill);
        Frags f;
        fetch(use, sc_use, j, f);       // LDS reads in flight ...
        __builtin_amdgcn_sched_barrier(0);
        fold(prev);                     // ... while group g - 1 is folded
        __builtin_amdgcn_sched_barrier(0);
        multiply(f, cur);               // results are folded one step later
        // (kept here: moved past the next barrier, the MFMAs would sit right
        // before the fold that reads them)
        __builtin_amdgcn_sched_barrier(0);
    };
    auto run = [&](auto third) __attribute__((always_inline)) {
    Dots d0, d1;  // d1 starts as dots 0, products 0: fmaf(0, 0, acc) = acc
#pragma unroll
    for (int ob = 0; ob < NB; ob++) {
        d1.c[ob] = zero16;
#pragma unroll
        for (int ni = 0; ni < NI; ni++)
#pragma unroll
            for (int mi = 0; mi < 2; mi++) d1.d[ob][mi][ni] = zero4;
    }
    issue(0, st0, third);
    issue_scales(0, sc0);
#pragma unroll
    for (int i = 1; i < S - 1; i++) issue(i, stage(i), third);
    // Passes of 16 groups (S = 4) or 24 (S = 3) so that every stage and
    // scale buffer is a fixed object: group g in stage g % S (off = g % S at
    // each call), chunk c = g / 8 in sc0 for even c, sc1 for odd c
    auto eight = [&](int g, int off, Scales &sc_use, Scales &sc_next) __attribute__((always_inline)) {
        step(g + 0, 0, stage((off + S - 1) % S), stage((off + 0) % S), sc_use, sc_next, d0, d1, third);
        step(g + 1, 1, stage((off + S + 0) % S), stage((off + 1) % S), sc_use, sc_next, d1, d0, third);
        step(g + 2, 2, stage((off + S + 1) % S), stage((off + 2) % S), sc_use, sc_next, d0, d1, third);
        step(g + 3, 3, stage((off + S + 2) % S), stage((off + 3) % S), sc_use, sc_next, d1, d0, third);
        step(g + 4, 4, stage((off + S + 3) % S), stage((off + 4) % S), sc_use, sc_next, d0, d1, third);
        step(g + 5, 5, stage((off + S + 4) % S), stage((off + 5) % S), sc_use, sc_next, d1, d0, third);
        step(g + 6, 6, stage((off + S + 5) % S), stage((off + 6) % S), sc_use, sc_next, d0, d1, third);
        step(g + 7, 7, stage((off + S + 6) % S), stage((off + 7) % S), sc_use, sc_next, d1, d0, third);
    };
    if constexpr (S == 3) {
        // groups == 24 (the launcher's condition): one pass, written as a
        // loop so that it stays one scheduling region of its own
        for (int g = 0; g < groups; g += 24) {
            eight(g, 0, sc0, sc1);
            eight(g + 8, 2, sc1, sc0);
            eight(g + 16, 1, sc0, sc1);
        }
    } else {
        int g = 0;
        for (; g + 16 <= groups; g += 16) {
            eight(g, 0, sc0, sc1);
            eight(g + 8, 0, sc1, sc0);
        }
        if (g < groups) eight(g, 0, sc0, sc1);  // uniform: groups % 16 == 8
    }
    fold(d1);  // the last group (groups % 8 == 0: it went to d1)
    };
    // EPI_GELU_MUL: the multipliers do not depend on the products; loaded
    // before the group loop, they arrive during it (memory operations retire
    // in order, so the loop's vmcnt waits still cover the DMA they count)
    float mulv[2][NI][4];
    if constexpr (EPI == EPI_GELU_MUL) {
#pragma unroll
        for (int mi = 0; mi < 2; mi++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int m = min(m0 + wm * 32 + mi * 16 + 4 * q + v, rows - 1);
#pragma unroll
                for (int ni = 0; ni < NI; ni++)
                    mulv[mi][ni][v] = ep.mul[(size_t)m * ep.mul_stride + nb0 * 16 + wn * WN + ni * 16 + l16];
            }
    }
    if (WAVES == 6 && wave == 0)
        run(std::true_type{});
    else
        run(std::false_type{});
    __builtin_amdgcn_s_waitcnt(0xF70);  // vmcnt(0): no DMA outlives the block
    if (EPI == EPI_PLAIN) {
#pragma unroll
        for (int mi = 0; mi < 2; mi++)
#pragma unroll
            for (int ni = 0; ni < NI; ni++) {
                const int col = wn * WN + ni * 16;
                if (nb0 + (col >> 4) >= n_blocks) continue;
                const size_t n = (size_t)nb0 * 16 + col + l16;
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int m = m0 + wm * 32 + mi * 16 + 4 * q + v;
                    if (m < rows) out[(size_t)m * out_stride + n] = acc[0][mi][ni][v];
                }
            }
        return;
    }
    // GELU epilogues: the block's 64 columns are one quantization group of
    // each of its rows.  gelu(gate) * up (or * mul), then k_quantize's
    // arithmetic: row absmax over the 64 columns (16 lanes x NI tiles in this
    // wave, and the other N-half's wave through LDS), scale = absmax / 127.
    __shared__ float s_rowmax[NWN][BM];  // [wn][row]
    float val[2][NI][4], rmax[2][4];
    // every lookup first, so that their loads go out together
#pragma unroll
    for (int mi = 0; mi < 2; mi++)
#pragma unroll
        for (int v = 0; v < 4; v++) {
#pragma unroll
            for (int ni = 0; ni < NI; ni++) {
                const float gl = gelu_table_lookup(acc[0][mi][ni][v], ep.gelu_table, ep.gelu_size,
                                                   ep.gelu_lower, ep.gelu_upper);
                val[mi][ni][v] = EPI == EPI_GELU_PAIR ? gl * acc[NB - 1][mi][ni][v] : gl * mulv[mi][ni][v];
            }
        }
#pragma unroll
    for (int mi = 0; mi < 2; mi++)
#pragma unroll
        for (int v = 0; v < 4; v++) {
            float mx = 0.0f;
#pragma unroll
            for (int ni = 0; ni < NI; ni++) mx = fmaxf(mx, fabsf(val[mi][ni][v]));
#pragma unroll
            for (int o = 8; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 16));
            rmax[mi][v] = mx;
            if (l16 == 0) s_rowmax[wn][wm * 32 + mi * 16 + 4 * q + v] = mx;
        }
    __syncthreads();
    const int groups_out = n_out >> 6;
#pragma unroll
    for (int mi = 0; mi < 2; mi++)
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int r = wm * 32 + mi * 16 + 4 * q + v, m = m0 + r;
            float mx = rmax[mi][v];
#pragma unroll
            for (int o = 1; o < NWN; o++) mx = fmaxf(mx, s_rowmax[(wn + o) % NWN][r]);
            const float scale = mx / 127.0f;
            const float inverse = scale > 0.0f ? 1.0f / scale : 0.0f;
            if (m >= rows) continue;
#pragma unroll
            for (int ni = 0; ni < NI; ni++) {
                const int n = nb0 * 16 + wn * WN + ni * 16 + l16;
                ep.q_out[(size_t)m * n_out + n] = (int8_t)(int)rintf(val[mi][ni][v] * inverse);
            }
            if (wn == 0 && l16 == 0) ep.qs_out[(size_t)m * groups_out + bx] = scale;
        }
}


// Grids of at most one block a CU (256 CUs) take 8-wave blocks: a lone
// block's step is bound by latency, which two waves a SIMD partly hide.
static bool small_grid(unsigned blocks) { return blocks <= 256; }

int launch_matmul_gelu(hipStream_t s, const int8_t *xq, const float *xs, const int8_t *w,
                       const uint16_t *ws, int n_out, int k, int rows, int epi,
                       const GemmEpilogue &ep) {
    if (rows <= 8 || k % 512 || n_out % 64 || (epi != EPI_GELU_PAIR && epi != EPI_GELU_MUL))
        return set_error(G4_ERR_ARG, "fused GEMM: shape %d x %d x %d does not fit", rows, n_out, k);
    const dim3 grid((unsigned)(n_out / 64), (unsigned)((rows + 63) / 64));
    // the pair at K = 1536 (every gate/up): 3 LDS stages, three blocks a CU
    if (epi == EPI_GELU_PAIR && k == 1536)
        hipLaunchKernelGGL((k_gemm_dma<EPI_GELU_PAIR, 4, 4, 3>), grid, dim3(256), 0, s, nullptr, (size_t)0,
                           xq, xs, w, ws, rows, n_out, k, ep);
    else if (epi == EPI_GELU_PAIR)
        hipLaunchKernelGGL((k_gemm_dma<EPI_GELU_PAIR, 4>), grid, dim3(256), 0, s, nullptr, (size_t)0,
                           xq, xs, w, ws, rows, n_out, k, ep);
    else if (small_grid(grid.x * grid.y))
        hipLaunchKernelGGL((k_gemm_dma<EPI_GELU_MUL, 8>), grid, dim3(512), 0, s, nullptr,
                           (size_t)0, xq, xs, w, ws, rows, n_out, k, ep);
    else
        hipLaunchKernelGGL((k_gemm_dma<EPI_GELU_MUL, 4>), grid, dim3(256), 0, s, nullptr, (size_t)0,
                           xq, xs, w, ws, rows, n_out, k, ep);
    return G4_OK;
}

int launch_matmul_group(hipStream_t s, const int8_t *xq, const float *xs, int rows, int k, int count,
                        const int8_t *const *w, const uint16_t *const *ws, float *const *out,
                        const size_t *out_stride, const int *n_out) {
    if (rows <= 8 || k % 512 || count < 1 || count > 3)
        return set_error(G4_ERR_ARG, "grouped GEMM: %d products of %d rows x K %d do not fit", count, rows, k);
    GemmEpilogue ep{};
    unsigned cols = 0;
    for (int i = 0; i < count; i++) {
        if (n_out[i] <= 0 || n_out[i] % 16)
            return set_error(G4_ERR_ARG, "grouped GEMM: N %d is not a multiple of 16", n_out[i]);
        ep.cols[i] = (n_out[i] / 16 + 3) / 4;
        cols += (unsigned)ep.cols[i];
        if (i) {
            ep.gw[i - 1] = w[i];
            ep.gws[i - 1] = ws[i];
            ep.gout[i - 1] = out[i];
            ep.gstride[i - 1] = out_stride[i];
            ep.gn[i - 1] = n_out[i];
        }
    }
    const dim3 grid(cols, (unsigned)((rows + 63) / 64));
    if (small_grid(grid.x * grid.y))
        hipLaunchKernelGGL((k_gemm_dma<EPI_PLAIN, 8>), grid, dim3(512), 0, s, out[0], out_stride[0], xq, xs,
                           w[0], ws[0], rows, n_out[0], k, ep);
    else
        hipLaunchKernelGGL((k_gemm_dma<EPI_PLAIN, 4>), grid, dim3(256), 0, s, out[0], out_stride[0], xq, xs,
                           w[0], ws[0], rows, n_out[0], k, ep);
    return G4_OK;
}

int launch_matmul(hipStream_t s, float *out, size_t out_stride, const int8_t *xq, const float *xs,
                  const int8_t *w, const uint16_t *ws, int n_out, int k, int rows) {
    if (rows <= 0) return G4_OK;
    const int blocks = n_out / 16, groups = k / 64;
    if (rows > 8) {
        const unsigned mb = (unsigned)((rows + 63) / 64);
        const dim3 grid((unsigned)((blocks + 3) / 4), mb), grid48((unsigned)(blocks / 3), mb);
        GemmEpilogue ep{};
        ep.cols[0] = (int)grid.x;
        if (groups % 8 == 0 && blocks % 3 == 0 && grid.x * grid.y < 256 && grid48.x * grid48.y <= 256) {
            // 48-wide tiles fill more of the 256 CUs (N = 1536 at 512 rows: 256 blocks, not 192)
            ep.cols[0] = (int)grid48.x;
            hipLaunchKernelGGL((k_gemm_dma<EPI_PLAIN, 6, 3>), grid48, dim3(384), 0, s, out, out_stride, xq,
                               xs, w, ws, rows, n_out, k, ep);
        } else if (groups % 8 == 0 && small_grid(grid.x * grid.y))
            hipLaunchKernelGGL((k_gemm_dma<EPI_PLAIN, 8>), grid, dim3(512), 0, s, out,
                               out_stride, xq, xs, w, ws, rows, n_out, k, ep);
        else if (groups % 8 == 0)
            hipLaunchKernelGGL((k_gemm_dma<EPI_PLAIN, 4>), grid, dim3(256), 0, s, out, out_stride, xq,
                               xs, w, ws, rows, n_out, k, ep);
        else  // K not a multiple of 512 (the per-layer-embedding projection, K = 256):
              // the register-staged kernel, two groups per barrier
            hipLaunchKernelGGL((k_gemm<64, 2>), dim3((unsigned)((blocks + 3) / 4), mb), dim3(256), 0, s,
                               out, out_stride, xq, xs, w, ws, rows, n_out, k);
        return G4_OK;
    }
    if (rows == 1 && launch_gemv1(s, out, xq, xs, w, ws, n_out, k)) return G4_OK;
    const int m_pad = rows <= 1 ? 1 : rows <= 2 ? 2 : rows <= 4 ? 4 : 8;
    // Enough waves to keep ~16 KB in flight on every CU: aim for >= 2048 waves,
    // each covering at least 8 groups (8 KB of weights).
    int splits = 1;
    if (blocks < 2048) {
        splits = (2048 + blocks - 1) / blocks;
        const int max_splits = groups / 8 > 0 ? groups / 8 : 1;
        if (splits > max_splits) splits = max_splits;
    }
    // Split K inside one block when the per-group dots fit in LDS: no fold kernel.
    const int split_waves = splits < 16 ? splits : 16;
    const size_t fold_lds = (size_t)(16 * m_pad + 16 + m_pad) * fold_row_floats(groups) * sizeof(float);
    if (splits > 1 && fold_lds <= 64 * 1024 && m_pad * groups <= 4 * 64 * split_waves) {
        // one batch of loads per wave where the registers allow it
        const int per_wave = (groups + split_waves - 1) / split_waves;
#define G4_GEMV_SPLIT(MM, UU)                                                                   \
    hipLaunchKernelGGL((k_gemv_split<MM, UU>), dim3((unsigned)blocks), dim3(64 * split_waves), fold_lds, s, \
                       out, out_stride, xq, xs, w, ws, k, rows)
        switch (m_pad) {
        case 1:  // batches of at most 12 (16 would spill with 16 waves a block)
            switch (gemv_batch(per_wave, 12)) {
            case 4: G4_GEMV_SPLIT(1, 4); break;
            case 8: G4_GEMV_SPLIT(1, 8); break;
            default: G4_GEMV_SPLIT(1, 12); break;
            }
            break;
        case 2: G4_GEMV_SPLIT(2, 8); break;
        case 4: G4_GEMV_SPLIT(4, 4); break;
        default: G4_GEMV_SPLIT(8, 4); break;
        }
#undef G4_GEMV_SPLIT
        return G4_OK;
    }
    int32_t *dots = nullptr;
    if (splits > 1) {
        const size_t need = (size_t)n_out * groups * m_pad * sizeof(int32_t);
        int rc = scratch_reserve(need, 0);
        if (rc) return rc;
        dots = scratch().dots;
    }
    dim3 grid((unsigned)(blocks * splits));
#define G4_GEMV(MM, UU)                                                                        \
    hipLaunchKernelGGL((k_gemv<MM, UU>), grid, dim3(64), 0, s, out, out_stride, xq, xs, w, ws, \
                       k, splits, rows, dots)
    switch (m_pad) {
    case 1:
        switch (gemv_batch((groups + splits - 1) / splits, 16)) {
        case 4: G4_GEMV(1, 4); break;
        case 8: G4_GEMV(1, 8); break;
        case 12: G4_GEMV(1, 12); break;
        default: G4_GEMV(1, 16); break;
        }
        break;
    case 2: G4_GEMV(2, 8); break;
    case 4: G4_GEMV(4, 4); break;
    default: G4_GEMV(8, 4); break;
    }
#undef G4_GEMV
    if (splits > 1) {
        dim3 fgrid((unsigned)((n_out + 255) / 256));
#define G4_FOLD(MM)                                                                            \
    hipLaunchKernelGGL((k_gemv_fold<MM>), fgrid, dim3(256), 0, s, out, out_stride, dots, xs, ws, \
                       n_out, groups, rows)
        switch (m_pad) {
        case 1: G4_FOLD(1); break;
        case 2: G4_FOLD(2); break;
        case 4: G4_FOLD(4); break;
        default: G4_FOLD(8); break;
        }
#undef G4_FOLD
    }
    return G4_OK;
}

// ---------------------------------------------------------------------------
// Elementwise kernels

// gemma4.c:360-373, one block per row.  Parallel sum of squares (each square
// rounded, then added, as the reference does; only the order differs).
__global__ __launch_bounds__(256) void k_rmsnorm(float *out, const float *in,
                                                 const float *__restrict__ weight, int width,
                                                 float eps) {
    __shared__ float red[4];
    const float *x = in + (size_t)blockIdx.x * width;
    float *y = out + (size_t)blockIdx.x * width;
    float s = 0.0f;
    for (int i = threadIdx.x; i < width; i += 256) s += x[i] * x[i];
    s = block_sum256(s, red);
    const float inverse = 1.0f / sqrtf(s / (float)width + eps);
    for (int i = threadIdx.x; i < width; i += 256)
        y[i] = (weight ? weight[i] : 1.0f) * (inverse * x[i]);
}

void launch_rmsnorm_parallel(hipStream_t s, float *out, const float *in, const float *weight,
                             int width, float eps, size_t rows) {
    if (!rows) return;
    hipLaunchKernelGGL(k_rmsnorm, dim3((unsigned)rows), dim3(256), 0, s, out, in, weight, width, eps);
}

__global__ __launch_bounds__(256) void k_add_and_scale(float *out, const float *add, size_t n,
                                                       float scale) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = (out[i] + add[i]) * scale;
}

void launch_add_and_scale(hipStream_t s, float *out, const float *add, size_t n, float scale) {
    if (!n) return;
    hipLaunchKernelGGL(k_add_and_scale, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, out,
                       add, n, scale);
}

// gemma4.c:381-398, one thread per (token, head, pair).
__global__ __launch_bounds__(256) void k_rope(const float *__restrict__ cosines,
                                              const float *__restrict__ sines, int pairs, float *v,
                                              int heads, int head_dim, int start_pos,
                                              const int *__restrict__ pos_dev, size_t total) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    if (pos_dev) start_pos = *pos_dev;
    const int j = (int)(i % pairs);
    const size_t th = i / pairs;  // token * heads + head
    const size_t t = th / heads;
    const float c = cosines[((size_t)start_pos + t) * pairs + j];
    const float s = sines[((size_t)start_pos + t) * pairs + j];
    float *x = v + th * head_dim;
    const float a = x[j], b = x[j + head_dim / 2];
    x[j] = a * c - b * s;
    x[j + head_dim / 2] = b * c + a * s;
}

void launch_rope(hipStream_t s, const float *cosines, const float *sines, int pairs, float *v,
                 int heads, int head_dim, int start_pos, const int *pos_dev, size_t n) {
    const size_t total = n * (size_t)heads * pairs;
    if (!total) return;
    hipLaunchKernelGGL(k_rope, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, cosines,
                       sines, pairs, v, heads, head_dim, start_pos, pos_dev, total);
}

// gemma4.c:310-331.
__global__ __launch_bounds__(256) void k_geglu(float *gate, const float *up, int width, int up_stride,
                                               size_t total, const float *__restrict__ table,
                                               int size, float lower, float upper) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const size_t r = i / width, c = i % width;
    const float x = gelu_table_lookup(gate[i], table, size, lower, upper);
    gate[i] = x * up[r * up_stride + c];
}

void launch_geglu(hipStream_t s, float *gate, const float *up, int rows, int width, int up_stride,
                  const float *table, int table_size, float lower, float upper) {
    const size_t total = (size_t)rows * width;
    if (!total) return;
    hipLaunchKernelGGL(k_geglu, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, gate, up,
                       width, up_stride, total, table, table_size, lower, upper);
}

// gemma4.c:337-358, one thread per output value.
__global__ __launch_bounds__(256) void k_embedding(float *out, const int8_t *__restrict__ table,
                                                   const uint16_t *__restrict__ scales, int width,
                                                   int table_rows, const int *__restrict__ tokens,
                                                   size_t total, float multiplier) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const size_t t = i / width;
    const int e = (int)(i % width), g = e >> 6, j = e & 63;
    const int token = tokens[t];
    if (token < 0 || token >= table_rows) {  // never read outside the table
        out[i] = __int_as_float(0x7fc00000);
        return;
    }
    const size_t block = (size_t)(token / 16);
    const int row = token % 16, groups = width / 64;
    const int8_t qv = table[block * 16 * width + (size_t)g * 1024 + (j / 4) * 64 + row * 4 + (j & 3)];
    const float s = half_bits_to_float(scales[(block * groups + g) * 16 + row]) * multiplier;
    out[i] = (float)qv * s;
}

void launch_embedding(hipStream_t s, float *out, const int8_t *table, const uint16_t *scales,
                      int width, int table_rows, const int *tokens, size_t n, float multiplier) {
    const size_t total = n * (size_t)width;
    if (!total) return;
    hipLaunchKernelGGL(k_embedding, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, out,
                       table, scales, width, table_rows, tokens, total, multiplier);
}

// gemma4.c:437-440: new keys get rmsnorm(k_norm) then RoPE, new values a
// weightless rmsnorm; rows land in the rings at (start_pos + t) & mask.
__global__ __launch_bounds__(256) void k_kv_finish(float *key_cache, float *value_cache,
                                                   const float *k_new, const float *v_new,
                                                   const float *__restrict__ k_norm,
                                                   const float *__restrict__ cosines,
                                                   const float *__restrict__ sines, int pairs,
                                                   int head_dim, int cache_len, int start_pos,
                                                   const int *__restrict__ pos_dev,
                                                   int reference_order) {
    __shared__ float red[4];
    if (pos_dev) start_pos = *pos_dev;
    __shared__ float row[512];
    const int t = blockIdx.x, is_value = blockIdx.y;
    const float *x = (is_value ? v_new : k_new) + (size_t)t * head_dim;
    const float *weight = is_value ? nullptr : k_norm;
    float s = 0.0f;
    if (reference_order) {
        // the reference's sequential sum (gemma4.c:367-368): squares in
        // parallel, one lane adds them in index order
        for (int i = threadIdx.x; i < head_dim; i += 256) row[i] = x[i] * x[i];
        __syncthreads();
        if (threadIdx.x == 0) {
            for (int i = 0; i < head_dim; i++) s += row[i];
            red[0] = s;
        }
        __syncthreads();
        s = red[0];
        __syncthreads();
    } else {
        for (int i = threadIdx.x; i < head_dim; i += 256) s += x[i] * x[i];
        s = block_sum256(s, red);
    }
    const float inverse = 1.0f / sqrtf(s / (float)head_dim + 1e-6f);
    for (int i = threadIdx.x; i < head_dim; i += 256)
        row[i] = (weight ? weight[i] : 1.0f) * (inverse * x[i]);
    __syncthreads();
    const int pos = start_pos + t;
    float *dst = (is_value ? value_cache : key_cache) + (size_t)(pos & (cache_len - 1)) * head_dim;
    if (!is_value) {
        const float *c = cosines + (size_t)pos * pairs, *sn = sines + (size_t)pos * pairs;
        for (int i = threadIdx.x; i < head_dim; i += 256) {
            float v = row[i];
            const int half = head_dim / 2;
            if (i < pairs) {
                v = row[i] * c[i] - row[i + half] * sn[i];
            } else if (i >= half && i - half < pairs) {
                const int j = i - half;
                v = row[i] * c[j] + row[j] * sn[j];
            }
            dst[i] = v;
        }
    } else {
        for (int i = threadIdx.x; i < head_dim; i += 256) dst[i] = row[i];
    }
}

void launch_kv_finish(hipStream_t s, float *key_cache, float *value_cache, const float *k_new,
                      const float *v_new, const float *k_norm, const float *cosines,
                      const float *sines, int pairs, int head_dim, int cache_len, int start_pos,
                      const int *pos_dev, size_t n) {
    if (!n) return;
    hipLaunchKernelGGL(k_kv_finish, dim3((unsigned)n, 2), dim3(256), 0, s, key_cache, value_cache,
                       k_new, v_new, k_norm, cosines, sines, pairs, head_dim, cache_len, start_pos,
                       pos_dev, order() == G4_ORDER_REFERENCE ? 1 : 0);
}

// The host libm's tanhf, restated: glibc's single-precision tanh
// (sysdeps/ieee754/flt-32/s_tanhf.c, from Sun's fdlibm) on its expm1f
// (s_expm1f.c).  Every step is one rounded fp32 operation (this file is built
// with -ffp-contract=off; division is correctly rounded), so the results are
// the host's bit for bit: tests/csrc/tanhf_method_check.c runs the same steps
// against the host libm on every float below 22 in magnitude.
//   expm1(x) = 2^k (1 + r + r^2/2 ...) - 1, x = k ln2 + r (ln2 in a high part
//   exact in 24 bits times k, and a low part), with the rational form
//   r1 = 1 + h (Q1 + h (Q2 + h (Q3 + h (Q4 + h Q5)))), h = r^2 / 2, and the
//   reconstruction arranged by the size of k.  Arguments here: |x| < 44.
__device__ __forceinline__ float expm1f_libm(float x) {
    constexpr uint32_t kQ1 = 0xbd088889u, kQ2 = 0x3ad00d01u, kQ3 = 0xb8a670cdu, kQ4 = 0x36867e54u,
                       kQ5 = 0xb457edbbu, kLn2Hi = 0x3f317180u, kLn2Lo = 0x3717f7d1u,
                       kInvLn2 = 0x3fb8aa3bu;
    const float Q1 = __uint_as_float(kQ1), Q2 = __uint_as_float(kQ2), Q3 = __uint_as_float(kQ3),
                Q4 = __uint_as_float(kQ4), Q5 = __uint_as_float(kQ5);
    const float ln2_hi = __uint_as_float(kLn2Hi), ln2_lo = __uint_as_float(kLn2Lo),
                invln2 = __uint_as_float(kInvLn2);
    const uint32_t ux = __float_as_uint(x), ax = ux & 0x7fffffffu;
    const bool negative = ux >> 31;
    if (negative && ax >= 0x4195b844u) return -1.0f;  // x <= -27 ln2
    int k;
    float c = 0.0f;
    if (ax > 0x3eb17218u) {       // |x| > ln2 / 2
        float hi, lo;
        if (ax < 0x3f851592u) {  // |x| < 3 ln2 / 2
            hi = negative ? x + ln2_hi : x - ln2_hi;
            lo = negative ? -ln2_lo : ln2_lo;
            k = negative ? -1 : 1;
        } else {
            k = (int)(invln2 * x + (negative ? -0.5f : 0.5f));
            const float t = (float)k;
            hi = x - t * ln2_hi;  // exact
            lo = t * ln2_lo;
        }
        x = hi - lo;
        c = (hi - x) - lo;
    } else if (ax < 0x33000000u) {  // |x| < 2^-25
        return x;
    } else {
        k = 0;
    }
    const float hfx = 0.5f * x, hxs = x * hfx;
    const float r1 = 1.0f + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
    float t = 3.0f - r1 * hfx;
    float e = hxs * ((r1 - t) / (6.0f - x * t));
    if (k == 0) return x - (x * e - hxs);
    e = x * (e - c) - c;
    e -= hxs;
    if (k == -1) return 0.5f * (x - e) - 0.5f;
    if (k == 1) return x < -0.25f ? -2.0f * (e - (x + 0.5f)) : 1.0f + 2.0f * (x - e);
    float y;
    if (k <= -2 || k > 56) {
        y = 1.0f - (e - x);
        y = __uint_as_float(__float_as_uint(y) + ((uint32_t)k << 23));
        return y - 1.0f;
    }
    if (k < 23) {
        t = __uint_as_float(0x3f800000u - (0x1000000u >> k));  // 1 - 2^-k
        y = t - (e - x);
    } else {
        t = __uint_as_float((uint32_t)(0x7f - k) << 23);  // 2^-k
        y = x - (e + t);
        y += 1.0f;
    }
    return __uint_as_float(__float_as_uint(y) + ((uint32_t)k << 23));
}
__device__ __forceinline__ float tanhf_libm(float x) {
    const uint32_t ux = __float_as_uint(x), ax = ux & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (ux >> 31) ? 1.0f / x - 1.0f : 1.0f / x + 1.0f;  // +-1, NaN
    float z;
    if (ax < 0x41b00000u) {  // |x| < 22
        if (ax == 0) return x;
        if (ax < 0x24000000u) return x * (1.0f + x);  // |x| < 2^-55
        const float a = __uint_as_float(ax);
        if (ax >= 0x3f800000u) {  // |x| >= 1
            const float t = expm1f_libm(2.0f * a);
            z = 1.0f - 2.0f / (t + 2.0f);
        } else {
            const float t = expm1f_libm(-2.0f * a);
            z = -t / (t + 2.0f);
        }
    } else {
        z = 1.0f;
    }
    return (ux >> 31) ? -z : z;
}

// gemma4.c:518-519: 30 tanh(x / 30), bit-identical to the host's.
__global__ __launch_bounds__(256) void k_softcap(float *x, size_t n) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) x[i] = 30.0f * tanhf_libm(x[i] / 30.0f);
}

void launch_softcap(hipStream_t s, float *x, size_t n) {
    if (!n) return;
    hipLaunchKernelGGL(k_softcap, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, n);
}

// First index of the row maximum (strict '>' scan of gemma4.c:537-541).
__global__ __launch_bounds__(256) void k_argmax(int *out, const float *x, size_t width) {
    const float *r = x + (size_t)blockIdx.x * width;
    float best = -INFINITY;
    int index = -1;
    for (size_t i = threadIdx.x; i < width; i += 256)
        if (index < 0 || r[i] > best) {
            best = r[i];
            index = (int)i;
        }
    __shared__ float sv[256];
    __shared__ int si[256];
    sv[threadIdx.x] = best;
    si[threadIdx.x] = index;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (threadIdx.x < o) {
            const float v2 = sv[threadIdx.x + o];
            const int i2 = si[threadIdx.x + o];
            const float v1 = sv[threadIdx.x];
            const int i1 = si[threadIdx.x];
            if (i2 >= 0 && (i1 < 0 || v2 > v1 || (v2 == v1 && i2 < i1))) {
                sv[threadIdx.x] = v2;
                si[threadIdx.x] = i2;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) out[blockIdx.x] = si[0];
}

void launch_argmax(hipStream_t s, int *out, const float *x, size_t rows, size_t width) {
    if (!rows) return;
    hipLaunchKernelGGL(k_argmax, dim3((unsigned)rows), dim3(256), 0, s, out, x, width);
}

// ---------------------------------------------------------------------------
// Attention (gemma4.c:443-456) as split-KV flash decoding over the ring cache.
//
// Phase 1: one 256-thread block per (query token, chunk of 64 visible keys),
// all heads at once so every K/V row is read once per block.  Scores follow the
// reference bit for bit: lane m of a 16-lane group accumulates fma(q_j, k_j)
// over j = m, m+16, ... and the group sums with the fixed tree
// ((l + l^8) -> +4 -> +2 -> +1).  Each head's chunk keeps its max m, the sum l
// of expf(s - m) and o = sum of expf(s - m) * v.
// Phase 2: per (token, head), rescale the chunks to the global max and divide.

constexpr int kAttnChunk = 64;
constexpr int kMaxHeads = 8;

template <int HD>
__global__ __launch_bounds__(256) void k_attn_partial(const float *__restrict__ q,
                                                      const float *__restrict__ key_cache,
                                                      const float *__restrict__ value_cache,
                                                      int cache_len, int heads, int full,
                                                      int start_pos, int max_chunks,
                                                      float *__restrict__ part_o,
                                                      float *__restrict__ part_ml) {
    __shared__ float s_q[kMaxHeads][HD];
    __shared__ float s_p[kMaxHeads][kAttnChunk];
    const int t = blockIdx.y, chunk = blockIdx.x;
    const int pos = start_pos + t;
    const int first = !full && pos + 1 > G4_WINDOW ? pos + 1 - G4_WINDOW : 0;
    const int keys = pos + 1 - first;
    const int k0 = chunk * kAttnChunk;
    if (k0 >= keys) return;
    const int kn = keys - k0 < kAttnChunk ? keys - k0 : kAttnChunk;
    const int mask = cache_len - 1;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float *qt = q + (size_t)t * heads * HD;
    for (int i = tid; i < heads * HD; i += 256) s_q[i / HD][i % HD] = qt[i];
    __syncthreads();

    // Scores: 16 lanes per key, 16 keys in flight per block.
    const int m16 = lane & 15, kg = lane >> 4;
    for (int kk = wave * 4 + kg; kk < kn; kk += 16) {
        const float *kr = key_cache + (size_t)((first + k0 + kk) & mask) * HD;
        float acc[kMaxHeads];
#pragma unroll
        for (int h = 0; h < kMaxHeads; h++) acc[h] = 0.0f;
        for (int j = m16; j < HD; j += 16) {
            const float kv = kr[j];
#pragma unroll
            for (int h = 0; h < kMaxHeads; h++)
                if (h < heads) acc[h] = fmaf(s_q[h][j], kv, acc[h]);
        }
#pragma unroll
        for (int h = 0; h < kMaxHeads; h++) {
            float v = acc[h];
            v += __shfl_down(v, 8, 16);
            v += __shfl_down(v, 4, 16);
            v += __shfl_down(v, 2, 16);
            v += __shfl_down(v, 1, 16);
            if (m16 == 0 && h < heads) s_p[h][kk] = v;
        }
    }
    __syncthreads();

    // Chunk softmax statistics: wave w takes heads w, w+4.
    for (int h = wave; h < heads; h += 4) {
        float m = -INFINITY;
        for (int i = lane; i < kn; i += 64) m = fmaxf(m, s_p[h][i]);
        m = wave_max(m);
        float l = 0.0f;
        for (int i = lane; i < kn; i += 64) {
            const float p = expf(s_p[h][i] - m);
            s_p[h][i] = p;
            l += p;
        }
        l = wave_sum(l);
        if (lane == 0) {
            float *ml = part_ml + (((size_t)t * max_chunks + chunk) * heads + h) * 2;
            ml[0] = m;
            ml[1] = l;
        }
    }
    __syncthreads();

    // Values: thread owns channels tid, tid+256, ... for every head.
    constexpr int PER = (HD + 255) / 256;
    float o[kMaxHeads][PER];
#pragma unroll
    for (int h = 0; h < kMaxHeads; h++)
#pragma unroll
        for (int e = 0; e < PER; e++) o[h][e] = 0.0f;
    for (int k = 0; k < kn; k++) {
        const float *vr = value_cache + (size_t)((first + k0 + k) & mask) * HD;
#pragma unroll
        for (int e = 0; e < PER; e++) {
            const int d = tid + e * 256;
            if (d < HD) {
                const float vv = vr[d];
#pragma unroll
                for (int h = 0; h < kMaxHeads; h++)
                    if (h < heads) o[h][e] = fmaf(s_p[h][k], vv, o[h][e]);
            }
        }
    }
#pragma unroll
    for (int h = 0; h < kMaxHeads; h++) {
        if (h >= heads) break;
        float *dst = part_o + (((size_t)t * max_chunks + chunk) * heads + h) * HD;
#pragma unroll
        for (int e = 0; e < PER; e++) {
            const int d = tid + e * 256;
            if (d < HD) dst[d] = o[h][e];
        }
    }
}

__global__ __launch_bounds__(256) void k_attn_combine(float *__restrict__ out,
                                                      const float *__restrict__ part_o,
                                                      const float *__restrict__ part_ml,
                                                      int head_dim, int heads, int full,
                                                      int start_pos, int max_chunks) {
    extern __shared__ float s_w[];
    __shared__ float red[4];
    const int h = blockIdx.x, t = blockIdx.y;
    const int pos = start_pos + t;
    const int first = !full && pos + 1 > G4_WINDOW ? pos + 1 - G4_WINDOW : 0;
    const int keys = pos + 1 - first;
    const int chunks = (keys + kAttnChunk - 1) / kAttnChunk;
    const float *ml = part_ml + ((size_t)t * max_chunks * heads + h) * 2;
    float m = -INFINITY;
    for (int c = threadIdx.x; c < chunks; c += 256) m = fmaxf(m, ml[(size_t)c * heads * 2]);
    m = wave_max(m);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float l = 0.0f;
    for (int c = threadIdx.x; c < chunks; c += 256) {
        const float wgt = expf(ml[(size_t)c * heads * 2] - m);
        s_w[c] = wgt;
        l += ml[(size_t)c * heads * 2 + 1] * wgt;
    }
    l = block_sum256(l, red);
    for (int d = threadIdx.x; d < head_dim; d += 256) {
        float acc = 0.0f;
        for (int c = 0; c < chunks; c++)
            acc = fmaf(part_o[(((size_t)t * max_chunks + c) * heads + h) * head_dim + d], s_w[c], acc);
        out[((size_t)t * heads + h) * head_dim + d] = acc / l;
    }
}

size_t attend_scratch_bytes(size_t n, int last_pos) {
    const size_t keys = (size_t)last_pos + 1, heads = 8;
    if (order() == G4_ORDER_REFERENCE) {  // the scores, and the split softmax of long decode rows
        const size_t stride = (keys + 63) & ~(size_t)63;
        const size_t scores = (n * heads * stride * sizeof(float) + 255) & ~(size_t)255;
        return scores + (n <= 4 && keys > (size_t)kSoftmaxSplitMin ? softmax_split_bytes(n * heads, stride) : 0);
    }
    return n * ((keys + kAttnChunk - 1) / kAttnChunk) * heads * (512 + 2) * sizeof(float);  // partials
}

int launch_attend_parallel(hipStream_t s, float *out, const float *q, const float *key_cache,
                           const float *value_cache, int cache_len, int head_dim, int heads,
                           int full, int start_pos, size_t n, const FixedScratch *fixed) {
    if (!n) return G4_OK;
    const int last_pos = start_pos + (int)n - 1;
    const int max_keys = full ? last_pos + 1 : (last_pos + 1 < G4_WINDOW ? last_pos + 1 : G4_WINDOW);
    const int max_chunks = (max_keys + kAttnChunk - 1) / kAttnChunk;
    const size_t o_floats = n * (size_t)max_chunks * heads * head_dim;
    const size_t ml_floats = n * (size_t)max_chunks * heads * 2;
    const size_t need = (o_floats + ml_floats) * sizeof(float);
    float *part_o = nullptr;
    if (fixed) {
        if (need > fixed->bytes)
            return set_error(G4_ERR_ARG, "attention needs %zu bytes of scratch, more than the fixed %zu",
                             need, fixed->bytes);
        part_o = (float *)fixed->ptr;
    } else {
        int rc = scratch_reserve(0, need);
        if (rc) return rc;
        part_o = scratch().attn;
    }
    float *part_ml = part_o + o_floats;
    dim3 grid1((unsigned)max_chunks, (unsigned)n);
    if (head_dim == 256)
        hipLaunchKernelGGL(k_attn_partial<256>, grid1, dim3(256), 0, s, q, key_cache, value_cache,
                           cache_len, heads, full, start_pos, max_chunks, part_o, part_ml);
    else
        hipLaunchKernelGGL(k_attn_partial<512>, grid1, dim3(256), 0, s, q, key_cache, value_cache,
                           cache_len, heads, full, start_pos, max_chunks, part_o, part_ml);
    hipLaunchKernelGGL(k_attn_combine, dim3((unsigned)heads, (unsigned)n), dim3(256),
                       (size_t)max_chunks * sizeof(float), s, out, part_o, part_ml, head_dim,
                       heads, full, start_pos, max_chunks);
    return G4_OK;
}

}  // namespace g4

// ---------------------------------------------------------------------------
// Per-op entry points (include/g4.h)

using namespace g4;

static bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

extern "C" int g4_quantize(void *stream, int8_t *q, float *scales, const float *x, size_t rows,
                           size_t width) {
    G4_CHECK(q && scales && x, "g4_quantize: null pointer");
    G4_CHECK(width % 64 == 0, "g4_quantize: width %zu is not a multiple of 64", width);
    G4_CHECK(aligned16(x) && aligned16(q), "g4_quantize: x and q must be 16-byte aligned");
    launch_quantize((hipStream_t)stream, q, scales, x, rows * (width / 64));
    G4_HIP(hipGetLastError());
    return G4_OK;
}

extern "C" int g4_matmul_int8(void *stream, float *out, const int8_t *xq, const float *xs,
                              const g4_tensor *w, size_t rows) {
    G4_CHECK(out && xq && xs && w && w->data && w->scales, "g4_matmul_int8: null pointer");
    const int n = w->shape[0], k = w->shape[1];
    G4_CHECK(n > 0 && k > 0 && n % 16 == 0 && k % 64 == 0,
             "g4_matmul_int8: weight shape %d x %d is not packable", n, k);
    G4_CHECK(rows <= (size_t)1 << 24, "g4_matmul_int8: too many rows");
    G4_CHECK(aligned16(xq) && aligned16(w->data), "g4_matmul_int8: xq and data must be 16-byte aligned");
    int rc = launch_matmul((hipStream_t)stream, out, (size_t)n, xq, xs, (const int8_t *)w->data,
                           w->scales, n, k, (int)rows);
    if (rc) return rc;
    G4_HIP(hipGetLastError());
    return G4_OK;
}

extern "C" int g4_rmsnorm(void *stream, float *out, const float *in, const float *weight,
                          int width, float epsilon, size_t rows) {
    G4_CHECK(out && in && width > 0, "g4_rmsnorm: bad arguments");
    launch_rmsnorm((hipStream_t)stream, out, in, weight, width, epsilon, rows);
    G4_HIP(hipGetLastError());
    return G4_OK;
}

extern "C" int g4_add_and_scale(void *stream, float *out, const float *add, size_t n, float scale) {
    G4_CHECK(out && add, "g4_add_and_scale: null pointer");
    launch_add_and_scale((hipStream_t)stream, out, add, n, scale);
    G4_HIP(hipGetLastError());
    return G4_OK;
}

extern "C" int g4_apply_rope(void *stream, const float *cosines, const float *sines, int pairs,
                             float *v, int heads, int head_dim, int start_pos, size_t n) {
    G4_CHECK(cosines && sines && v, "g4_apply_rope: null pointer");
    G4_CHECK(heads > 0 && head_dim > 0 && head_dim % 2 == 0 && pairs >= 0 && pairs <= head_dim / 2,
             "g4_apply_rope: bad geometry");
    G4_CHECK(start_pos >= 0, "g4_apply_rope: negative position");
    launch_rope((hipStream_t)stream, cosines, sines, pairs, v, heads, head_dim, start_pos, nullptr, n);
    G4_HIP(hipGetLastError());
    return G4_OK;
}

extern "C" int g4_geglu(void *stream, float *gate, const float *up, int rows, int width,
                        int up_stride, const float *table, int table_size, float lower,
                        float upper) {
    G4_CHECK(gate && up && table, "g4_geglu: null pointer");
    G4_CHECK(rows >= 0 && width >= 0 && up_stride >= width && table_size >= 2 && upper > lower,
             "g4_geglu: bad arguments");
    launch_geglu((hipStream_t)stream, gate, up, rows, width, up_stride, table, table_size, lower,
                 upper);
    G4_HIP(hipGetLastError());
    return G4_OK;
}

extern "C" int g4_embedding(void *stream, float *out, const g4_tensor *table, const int *tokens,
                            size_t n, float multiplier) {
    G4_CHECK(out && table && table->data && table->scales && tokens, "g4_embedding: null pointer");
    G4_CHECK(table->shape[0] % 16 == 0 && table->shape[1] % 64 == 0 && table->shape[1] > 0,
             "g4_embedding: table is not packed");
    launch_embedding((hipStream_t)stream, out, (const int8_t *)table->data, table->scales,
                     table->shape[1], table->shape[0], tokens, n, multiplier);
    G4_HIP(hipGetLastError());
    return G4_OK;
}

int g4::check_attend_args(const char *who, float *out, const float *q, const float *key_cache,
                          const float *value_cache, int cache_len, int head_dim, int heads,
                          int full_attention, int start_pos, size_t n) {
    G4_CHECK(out && q && key_cache && value_cache, "%s: null pointer", who);
    G4_CHECK(head_dim == 256 || head_dim == 512, "%s: head_dim must be 256 or 512", who);
    // the reference-order kernels take the model's 8 query heads; the parallel
    // order any count up to 8
    G4_CHECK(order() == G4_ORDER_REFERENCE ? heads == 8 : heads >= 1 && heads <= 8,
             "%s: heads must be 8 (1..8 in the parallel order)", who);
    G4_CHECK(cache_len > 0 && (cache_len & (cache_len - 1)) == 0, "%s: cache_len must be a power of two", who);
    G4_CHECK(start_pos >= 0, "%s: negative position", who);
    G4_CHECK(n <= (size_t)G4_MAX_CONTEXT, "%s: %zu tokens exceed the context", who, n);
    // Keys visible to the batch span positions max(0, start_pos - 511) ..
    // start_pos + n - 1 (sliding) or 0 .. start_pos + n - 1 (full); the ring
    // must hold them all.
    const long span = full_attention ? (long)start_pos + (long)n
                                     : (long)(start_pos < G4_WINDOW - 1 ? start_pos : G4_WINDOW - 1) + (long)n;
    G4_CHECK(span <= cache_len, "%s: %ld visible keys exceed the %d-row ring", who, span, cache_len);
    return G4_OK;
}

extern "C" int g4_attend(void *stream, float *out, const float *q, const float *key_cache,
                         const float *value_cache, int cache_len, int head_dim, int heads,
                         int full_attention, int start_pos, size_t n) {
    int rc = check_attend_args("g4_attend", out, q, key_cache, value_cache, cache_len, head_dim, heads,
                               full_attention, start_pos, n);
    if (rc) return rc;
    rc = launch_attend((hipStream_t)stream, out, q, key_cache, value_cache, cache_len, head_dim,
                       heads, full_attention, start_pos, nullptr, n);
    if (rc) return rc;
    G4_HIP(hipGetLastError());
    return G4_OK;
}
