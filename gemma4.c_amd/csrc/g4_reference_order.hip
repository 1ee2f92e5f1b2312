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
//   value sums (gemma4.c:296-307): one fma chain per output channel over the
//     keys in order (a lane per chain in decode; in prefill an output of the
//     fp32 matrix cores' K = 1 products, which round once a step like fmaf);
//   scores (gemma4.c:281-294): 16 fma chains per score and a fixed tree (16
//     lanes per score in decode, matrix-core outputs in prefill).
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
// rmsnorm, reference order: one wave per row.  The sum of squares is the
// reference's sequential fp32 chain (gemma4.c:366-368); the squares are
// computed in parallel (each is rounded on its own in the reference too), so
// only the dependent adds run on one lane.

constexpr int kNormMaxWidth = 1536;

// Runtime length (any width): 64 squares per step, loaded just before use.
__device__ __forceinline__ float chain_lds(const float4 *sq, int batches) {
    float sum = 0.0f;
    for (int b = 0; b < batches; b++) {
        float4 v[16];
#pragma unroll
        for (int j = 0; j < 16; j++) v[j] = sq[b * 16 + j];
#pragma unroll
        for (int j = 0; j < 16; j++) {
            sum += v[j].x;
            sum += v[j].y;
            sum += v[j].z;
            sum += v[j].w;
        }
    }
    return sum;
}

// ---------------------------------------------------------------------------
// The sequential fp32 sum of non-negative terms, computed in parallel and bit
// for bit.  s_0 = 0, s_k = RN(s_{k-1} + t_k) in order (the reference's loop).
// While s stays inside one binade [2^e, 2^(e+1)) every partial sum is a
// multiple of u = 2^(e-23), and adding t_k rounds it to the nearest multiple:
// s_k = s_{k-1} + R_k u with R_k = rint(t_k / u) -- independent of s_{k-1}
// except at an exact half (a tie, where round-to-even looks at s_{k-1}).  So a
// run of steps is an integer prefix sum over the wave; the run ends at the
// first step that reaches 2^(e+1) (the grid changes) or is a tie, and that
// one step is done as the plain fp32 add before the next run starts.  The
// terms are held "block-major": t[b] in lane l is term 64 b + l.
__device__ __forceinline__ int wave_add_scan(int x) {  // inclusive, over 64 lanes
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31
    return x;
}

// Advance the running sum s over the 64 terms of one block (lane l holds
// term l), from term p0 to the end of the block, in order.  Lanes flagged in
// `special` are a new running maximum of a softmax: s = s * t + 1 there
// (two roundings, gemma4.c:403) instead of s + t.  Terms must be >= 0; with
// no special lanes s must start >= 0, with special lanes s >= 1.
__device__ __forceinline__ float block_advance(float s, float tb, int p0, uint64_t special) {
    const int lane = threadIdx.x & 63;
    int p = p0;
    while (p < 64) {  // uniform
        const uint32_t bits = __float_as_uint(s);
        const int e = (int)((bits >> 23) & 0xff) - 127;  // exponent of s (s >= 0)
        if (e < -100 || e > 100) {  // zero, tiny, huge, inf, nan: one plain step
            const float t = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(tb), p));
            s = (special >> p) & 1 ? s * t + 1.0f : s + t;
            p++;
            continue;
        }
        const int ue = e - 23;                     // log2 of the grid u
        const int S = (int)ldexpf(s, -ue);         // s / u, exact, in [2^23, 2^24)
        const bool active = lane >= p;
        // t / u, exact; clamped at 2^24 (such a term ends the run anyway), so
        // 64 of them cannot overflow the int prefix sum
        const float T = active ? fminf(ldexpf(tb, -ue), 16777216.0f) : 0.0f;
        const bool tie = active && (T - floorf(T) == 0.5f);
        const int P = wave_add_scan((int)rintf(T));  // nearest, ties to even
        const bool stop = active && (tie || ((special >> lane) & 1) || S + P >= (1 << 24));
        const uint64_t mask = __ballot(stop);
        if (mask == 0) {  // the run covers the rest of the block
            s = ldexpf((float)(S + __builtin_amdgcn_readlane(P, 63)), ue);
            break;
        }
        // the run ends before term L, which is applied plainly
        const int L = (int)__builtin_ctzll(mask);
        const int before = L > 0 ? __builtin_amdgcn_readlane(P, L - 1) : 0;
        s = ldexpf((float)(S + before), ue);
        const float t = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(tb), L));
        s = (special >> L) & 1 ? s * t + 1.0f : s + t;
        p = L + 1;
    }
    return s;
}

// ---------------------------------------------------------------------------
// The same sequential sum over a whole row at once, with the binades
// predicted.  NW waves of a block own 64 NW J consecutive terms, lane-major:
// t[j] of thread T = 64 w + l is term k = J T + j.  A pass
//  1. predicts every partial sum with a cheap fp32 prefix (thread-serial
//     sums, then scans over lanes and waves; only its binade is used);
//  2. marks as an event every step that is not a grid step under that
//     prediction: the predicted binade changes, a tie, a softmax new maximum,
//     a term or partial sum outside the normal range.  Every step of a run
//     must be on the run's one grid, also where the run passes from one
//     thread to the next, whose start comes from the scans (another order)
//     and can lie on the other side of a power of two: a thread's first step
//     takes the binade the previous thread's prediction ends in;
//  3. takes R_k = rint(t_k / u), u from the predicted binade, for every
//     other step, and the prefix sums of R within each run between events;
//  4. lists the events in order in LDS: the run sum before each, its term,
//     the binade predicted after it;
//  5. resolves them in order.  Run i adds exactly d_i u_i when the exact sum
//     is in the predicted binade at its start and stays in it (the add is
//     then exact); the event is the plain fp32 step.  The chain is computed
//     first and the checks afterwards, all runs at once.
// Where a prediction was wrong a check fails.  s is exact at the start of the
// first failing run.  A run that leaves its binade early is advanced exactly
// up to the step that does, which is taken plainly; the next pass starts
// there.  A pass resolves at most kEsumEvents events.  Terms must be >= 0 (a
// NaN or inf term is an event, so it propagates as in the plain loop), s >= 0.
constexpr int kEsumEvents = 63;  // the table's last lane holds the final run
constexpr int kEsumMaxWaves = 16;
struct EsumEvent {
    int d;     // run sum (in the run's grid) before the event
    float t;   // the event's term
    int k;     // its index
    int meta;  // bit 0: new maximum; bits 8..15: predicted biased exponent after it
};
struct EsumShared {  // one per block (per wave when NW = 1)
    EsumEvent table[kEsumEvents];
    float wave_a[kEsumMaxWaves], wave_b[kEsumMaxWaves];  // predicted map of each wave
    int wave_seg[kEsumMaxWaves], wave_count[kEsumMaxWaves];
    int last_d;
    int found_k[kEsumMaxWaves], found_before[kEsumMaxWaves];
    float found_t[kEsumMaxWaves];
};

__device__ __forceinline__ int biased_exponent(float x) {
    return (int)((__float_as_uint(x) >> 23) & 0xff);
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_float(float x, float old) {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(x), CTRL, ROW_MASK, 0xf, false));
}
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int dpp_int(int x, int old) {
    return __builtin_amdgcn_update_dpp(old, x, CTRL, ROW_MASK, 0xf, false);
}

// Inclusive scan of fp32 adds over the wave (any association: a prediction).
__device__ __forceinline__ float wave_fadd_inclusive(float x) {
    x += dpp_float<0x111, 0xf>(x, 0.0f);
    x += dpp_float<0x112, 0xf>(x, 0.0f);
    x += dpp_float<0x114, 0xf>(x, 0.0f);
    x += dpp_float<0x118, 0xf>(x, 0.0f);
    x += dpp_float<0x142, 0xa>(x, 0.0f);
    x += dpp_float<0x143, 0xc>(x, 0.0f);
    return x;
}

// Inclusive scan of affine maps x -> a x + b (lower lanes applied first).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ void affine_step(float &a, float &b) {
    const float pa = dpp_float<CTRL, ROW_MASK>(a, 1.0f), pb = dpp_float<CTRL, ROW_MASK>(b, 0.0f);
    b = fmaf(pb, a, b);
    a = pa * a;
}
__device__ __forceinline__ void wave_affine_inclusive(float &a, float &b) {
    affine_step<0x111, 0xf>(a, b);
    affine_step<0x112, 0xf>(a, b);
    affine_step<0x114, 0xf>(a, b);
    affine_step<0x118, 0xf>(a, b);
    affine_step<0x142, 0xa>(a, b);
    affine_step<0x143, 0xc>(a, b);
}

// Run sums saturate at kEsumCap (any sum that large already leaves a binade);
// kEsumFlag marks "a run starts inside" in the segmented scan.
constexpr int kEsumCap = 1 << 29, kEsumFlag = 1 << 30;
__device__ __forceinline__ int segmented_join(int left, int x) {
    return (x & kEsumFlag) ? x : ((left & kEsumFlag) | min(x + (left & (kEsumFlag - 1)), kEsumCap));
}
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int segmented_step(int x) {
    return segmented_join(dpp_int<CTRL, ROW_MASK>(x, 0), x);
}
__device__ __forceinline__ int wave_segmented_inclusive(int x) {
    x = segmented_step<0x111, 0xf>(x);
    x = segmented_step<0x112, 0xf>(x);
    x = segmented_step<0x114, 0xf>(x);
    x = segmented_step<0x118, 0xf>(x);
    x = segmented_step<0x142, 0xa>(x);
    x = segmented_step<0x143, 0xc>(x);
    return x;
}

// The same scans within each 16-lane row: the per-wave values of a block
// (at most kEsumMaxWaves = 16), one a lane, combined by every wave at once
// instead of one wave value after another (blocks of 8 or 16 waves).
__device__ __forceinline__ int row16_segmented_inclusive(int x) {
    x = segmented_step<0x111, 0xf>(x);
    x = segmented_step<0x112, 0xf>(x);
    x = segmented_step<0x114, 0xf>(x);
    x = segmented_step<0x118, 0xf>(x);
    return x;
}
__device__ __forceinline__ int row16_add_inclusive(int x) {
    x += dpp_int<0x111, 0xf>(x, 0);
    x += dpp_int<0x112, 0xf>(x, 0);
    x += dpp_int<0x114, 0xf>(x, 0);
    x += dpp_int<0x118, 0xf>(x, 0);
    return x;
}
__device__ __forceinline__ float row16_fadd_inclusive(float x) {
    x += dpp_float<0x111, 0xf>(x, 0.0f);
    x += dpp_float<0x112, 0xf>(x, 0.0f);
    x += dpp_float<0x114, 0xf>(x, 0.0f);
    x += dpp_float<0x118, 0xf>(x, 0.0f);
    return x;
}
__device__ __forceinline__ void row16_affine_inclusive(float &a, float &b) {
    affine_step<0x111, 0xf>(a, b);
    affine_step<0x112, 0xf>(a, b);
    affine_step<0x114, 0xf>(a, b);
    affine_step<0x118, 0xf>(a, b);
}

template <int NW>
__device__ __forceinline__ void esum_barrier() {
    if constexpr (NW > 1) __syncthreads();
}

// One pass from term k0 with the exact sum s before it.  Returns true when
// every term is summed (s is then the result); otherwise s and k0 are the
// exact state the next pass starts from.  Every thread of the NW waves calls
// it (all lanes active); s and k0 are the same in all of them.
// Phases 1-4 of a pass from term k0 with the sum s before it: the event
// table in sh (its first kEsumEvents entries, sh.last_d the final run) and,
// for each thread, P (the run sum through each of its terms) and carry (the
// run sum coming into its first term).  Returns the number of events.
template <int NW, int J, bool SPECIAL>
__device__ __forceinline__ int esum_table(const float (&t)[J], uint32_t spec, float s, int k0, EsumShared &sh,
                                          int (&P)[J], int &carry) {
    static_assert(NW >= 1 && NW <= kEsumMaxWaves && J <= 32, "esum shape");
    const int lane = threadIdx.x & 63, wave = NW > 1 ? (int)(threadIdx.x >> 6) : 0;
    const int kb = (wave * 64 + lane) * J;
    // 1. the predicted prefix before this thread's first term
    float c;
    {
        float la = 1.0f, lb = 0.0f;
#pragma unroll
        for (int j = 0; j < J; j++) {
            const bool act = kb + j >= k0, sp = SPECIAL && ((spec >> j) & 1);
            if (SPECIAL) {
                const float a = act && sp ? t[j] : 1.0f, b = act ? (sp ? 1.0f : t[j]) : 0.0f;
                lb = fmaf(lb, a, b);
                la *= a;
            } else {
                lb += act ? t[j] : 0.0f;
            }
        }
        float x = s;  // the sum before this wave's first term
        // (the maps of the earlier waves; from 8 waves on, lane w of every row
        // holds wave w's, scanned within the row, and this wave takes lane
        // wave - 1's -- fewer waves run the loop, which measured faster there)
        if (SPECIAL) {
            wave_affine_inclusive(la, lb);
            if constexpr (NW > 1) {
                if (lane == 63) {
                    sh.wave_a[wave] = la;
                    sh.wave_b[wave] = lb;
                }
                esum_barrier<NW>();
                if constexpr (NW >= 8) {
                    const int r = lane & 15;
                    float pa = r < NW ? sh.wave_a[r] : 1.0f, pb = r < NW ? sh.wave_b[r] : 0.0f;
                    row16_affine_inclusive(pa, pb);
                    if (wave > 0)
                        x = fmaf(x, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pa), wave - 1)),
                                 __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pb), wave - 1)));
                } else {
                    for (int w = 0; w < wave; w++) x = fmaf(x, sh.wave_a[w], sh.wave_b[w]);
                }
            }
            c = fmaf(x, dpp_float<0x138, 0xf>(la, 1.0f), dpp_float<0x138, 0xf>(lb, 0.0f));
        } else {
            lb = wave_fadd_inclusive(lb);
            if constexpr (NW > 1) {
                if (lane == 63) sh.wave_b[wave] = lb;
                esum_barrier<NW>();
                if constexpr (NW >= 8) {
                    const int r = lane & 15;
                    const float pb = row16_fadd_inclusive(r < NW ? sh.wave_b[r] : 0.0f);
                    if (wave > 0) x += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pb), wave - 1));
                } else {
                    for (int w = 0; w < wave; w++) x += sh.wave_b[w];
                }
            }
            c = x + dpp_float<0x138, 0xf>(lb, 0.0f);
        }
    }
    // 2. events, grid steps and this thread's run sums, each step on the grid
    // of the binade its prediction is in before it.  A run that goes on from
    // the previous thread must keep that thread's grid: the binade the
    // previous thread's prediction ends in, lane l - 1's over DPP.  Where that
    // is not c's, the first step (taken on c's grid in the loop) becomes an
    // event instead, and its R leaves the run sums up to the next event.
    // Lane 0 of a later wave cannot see the previous wave's end before the
    // next barrier; there c and that end are two fp32 evaluations of the same
    // prefix with nonnegative operands (+, x, fma) and at most 2J + 23
    // roundings on any path, so each is within (2J + 23) 2^-24 of the exact
    // prefix and the two are apart by less than 2^-16 of it (J <= 32): unless
    // c lies within 2^-12 of a power of two they share a binade, c's.  Within
    // that margin the first step is an event -- except just above 1 in a
    // softmax sum, where s >= 1 and every step keeps the sum >= 1.  Where
    // every term before the thread is inactive, c is s itself.
    uint32_t evbits = 0;
    {
        float A = c;
        int run = 0, R0 = 0;
#pragma unroll
        for (int j = 0; j < J; j++) {
            const bool act = kb + j >= k0, sp = SPECIAL && ((spec >> j) & 1);
            const float prev = A;
            if (act) A = sp ? fmaf(A, t[j], 1.0f) : A + t[j];
            const int ep = biased_exponent(prev), ec = biased_exponent(A);
            const float T = fminf(ldexpf(t[j], 150 - ep), 16777216.0f);
            const float R = rintf(T);  // nearest, ties to even
            const bool ev = act && (sp || ep != ec || (unsigned)(ep - 27) > 200u ||
                                    fabsf(T - R) == 0.5f || !(t[j] <= 3.40282347e38f));
            if (j == 0) R0 = act ? (int)R : 0;
            run = ev ? 0 : min(run + (act ? (int)R : 0), kEsumCap);
            P[j] = run;
            evbits |= (uint32_t)ev << j;
        }
        const int ec = biased_exponent(c);
        int e_first = ec;  // wave 0's lane 0: c is s
        if constexpr (NW > 1) {
            const uint32_t m = __float_as_uint(c) & 0x7fffffu;
            const bool near_low = m < (1u << 11) && !(SPECIAL && ec == 127);
            if (wave > 0 && kb > k0 && (near_low || m >= (1u << 23) - (1u << 12))) e_first = -1;
        }
        const int e_in = dpp_int<0x138, 0xf>(biased_exponent(A), e_first);
        if (e_in != ec && kb >= k0 && !(evbits & 1u)) {
            // (sums below 2^24 are exact after the subtraction; larger ones,
            // saturated or not, stay above it and fail the checks either way)
            const int stop = (int)__builtin_ctzll((uint64_t)evbits | 1ull << J);  // J: no later event
#pragma unroll
            for (int j = 0; j < J; j++)
                if (j < stop) P[j] -= R0;
            evbits |= 1u;
        }
    }
    // 3. run sums across threads, event numbering
    const int seg = wave_segmented_inclusive((evbits ? kEsumFlag : 0) | P[J - 1]);
    carry = dpp_int<0x138, 0xf>(seg, 0);  // through the previous thread, flagged if a run starts
    const int count = __popc(evbits), numbered = wave_add_scan(count);
    int idx = numbered - count, total;
    if constexpr (NW > 1) {
        if (lane == 63) {
            sh.wave_seg[wave] = seg;
            sh.wave_count[wave] = numbered;
        }
        esum_barrier<NW>();
        int incoming = 0;
        if constexpr (NW >= 8) {
            const int r = lane & 15;  // (as for the maps above)
            const int vs = row16_segmented_inclusive(r < NW ? sh.wave_seg[r] : 0);
            const int vc = row16_add_inclusive(r < NW ? sh.wave_count[r] : 0);
            if (wave > 0) {
                incoming = __builtin_amdgcn_readlane(vs, wave - 1);
                idx += __builtin_amdgcn_readlane(vc, wave - 1);
            }
            total = __builtin_amdgcn_readlane(vc, NW - 1);
        } else {
            total = 0;
#pragma unroll
            for (int w = 0; w < NW; w++) {
                if (w < wave) {
                    incoming = segmented_join(incoming, sh.wave_seg[w]);
                    idx += sh.wave_count[w];
                }
                total += sh.wave_count[w];
            }
        }
        carry = segmented_join(incoming, carry);
    } else {
        total = __builtin_amdgcn_readlane(numbered, 63);
    }
    carry &= kEsumFlag - 1;
    // 4. the event table; P becomes the run sum through each term
    {
        float A = c;
        int before = carry;
        bool open = true;  // no event yet in this thread: the carry continues its run
#pragma unroll
        for (int j = 0; j < J; j++) {
            const bool act = kb + j >= k0, sp = SPECIAL && ((spec >> j) & 1);
            if (act) A = sp ? fmaf(A, t[j], 1.0f) : A + t[j];
            if ((evbits >> j) & 1) {
                if (idx < kEsumEvents)
                    sh.table[idx] = EsumEvent{before, t[j], kb + j, (int)sp | biased_exponent(A) << 8};
                idx++;
                open = false;
            }
            if (open) P[j] = min(P[j] + carry, kEsumCap);
            before = P[j];
        }
        if (wave == NW - 1 && lane == 63) sh.last_d = P[J - 1];
    }
    esum_barrier<NW>();
    return total;
}

template <int NW, int J, bool SPECIAL>
__device__ bool esum_pass(const float (&t)[J], uint32_t spec, float &s, int &k0, EsumShared &sh) {
    constexpr int N = 64 * NW * J;
    const int lane = threadIdx.x & 63, wave = NW > 1 ? (int)(threadIdx.x >> 6) : 0;
    const int kb = (wave * 64 + lane) * J;
    int P[J], carry;
    const int total = esum_table<NW, J, SPECIAL>(t, spec, s, k0, sh, P, carry);
    // 5. resolve: entry i (lane i) is the run before event i and the event; the
    // final run is one more entry, with no step
    const bool more = total > kEsumEvents;
    const int events = more ? kEsumEvents : total, entries = more ? events : events + 1;
    const EsumEvent e = lane < events ? sh.table[lane] : EsumEvent{sh.last_d, 0.0f, N, 0};
    const int prev_meta = dpp_int<0x138, 0xf>(e.meta, 0), prev_k = dpp_int<0x138, 0xf>(e.k, 0);
    const int e_run = lane == 0 ? biased_exponent(s) : (prev_meta >> 8) & 0xff;
    const int start = lane == 0 ? k0 : prev_k + 1;
    const bool nonempty = e.k > start;
    const float du = nonempty ? ldexpf((float)e.d, e_run - 150) : 0.0f;
    const bool sp = e.meta & 1;
    const float fa = sp ? e.t : 1.0f, fb = sp ? 1.0f : e.t;
    // The chain through the entries in order: entry i's start reaches lane i
    // from lane i - 1's end by a DPP wave shift, so a step is the run's add,
    // the event's step and one move for the whole wave (lane 0 keeps the
    // pass's start).  After step i lane i holds its entry's exact start and
    // its run's end for good (its input no longer changes), so steps past the
    // entry count change nothing and the count is rounded up to fours.
    // entries is the same in every lane (a count read back from LDS, which
    // the compiler cannot see): made scalar, the loop runs on scalar branches.
    const int n_entries = __builtin_amdgcn_readfirstlane(entries);
    float at_start = s, at_end = s, outv = s;
    auto chain_step = [&]() __attribute__((always_inline)) {
        at_end = at_start + du;
        if constexpr (SPECIAL)  // s t + 1 at a new maximum, s + t (t * 1 exact) otherwise
            outv = at_end * fa + fb;
        else
            outv = at_end + fb;
        at_start = dpp_float<0x138, 0xf>(outv, at_start);  // wave_shr:1, lane 0 keeps its own
    };
    for (int i = 0; i < n_entries; i += 4) {
        chain_step();
        chain_step();
        chain_step();
        chain_step();
    }
    const float sv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(outv), n_entries - 1));
    const int e0 = biased_exponent(at_start), e1 = biased_exponent(at_end);
    const uint64_t bad = __ballot(lane < entries && nonempty &&
                                  (e0 != e_run || (unsigned)(e0 - 27) > 200u || e1 != e_run));
    if (!bad) {
        s = sv;
        if (more) {
            k0 = __builtin_amdgcn_readlane(e.k, entries - 1) + 1;
            return false;
        }
        k0 = N;
        return true;
    }
    const int i = (int)__builtin_ctzll(bad);
    const float sb = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(at_start), i));
    const int st = __builtin_amdgcn_readlane(start, i), kend = __builtin_amdgcn_readlane(e.k, i);
    const int eb = biased_exponent(sb);
    if (eb != __builtin_amdgcn_readlane(e_run, i) || (unsigned)(eb - 27) > 200u) {
        s = sb;  // the predicted binade was wrong: start over from this run
        k0 = st;
        return false;
    }
    // the run leaves its binade early: find the first step that does
    const int S = (int)ldexpf(sb, 150 - eb);  // in [2^23, 2^24)
    int found = J, before_found = 0, prevP = carry;
    float t_found = 0.0f;
#pragma unroll
    for (int j = 0; j < J; j++) {
        const int k = kb + j;
        if (found == J && k >= st && k < kend && S + P[j] >= (1 << 24)) {
            found = j;
            before_found = prevP;
            t_found = t[j];
        }
        prevP = P[j];
    }
    const uint64_t hit = __ballot(found < J);
    int kf = N, bf = 0;
    float tf = 0.0f;
    if (hit) {
        const int L = (int)__builtin_ctzll(hit);
        kf = (wave * 64 + L) * J + __builtin_amdgcn_readlane(found, L);
        bf = __builtin_amdgcn_readlane(before_found, L);
        tf = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t_found), L));
    }
    if constexpr (NW > 1) {
        if (lane == 0) {
            sh.found_k[wave] = kf;
            sh.found_before[wave] = bf;
            sh.found_t[wave] = tf;
        }
        esum_barrier<NW>();
        kf = N;
#pragma unroll
        for (int w = NW - 1; w >= 0; w--) {
            if (sh.found_k[w] < N) {
                kf = sh.found_k[w];
                bf = sh.found_before[w];
                tf = sh.found_t[w];
            }
        }
        esum_barrier<NW>();  // the slots are free for the next pass's search
    }
    s = ldexpf((float)(S + bf), eb - 150) + tf;
    k0 = kf + 1;
    return false;
}

// The sequential sum s_init + t_0 + ... (or, for flagged terms, s = s t + 1)
// of the block's 64 NW J terms, lane-major.  Every thread of the NW waves
// calls it; all get the result.
template <int NW, int J, bool SPECIAL>
__device__ __forceinline__ float exact_sum_events(const float (&t)[J], uint32_t spec, float s,
                                                  EsumShared &sh) {
    int k0 = 0;
    while (!esum_pass<NW, J, SPECIAL>(t, spec, s, k0, sh)) {
    }
    return s;
}

// A hidden row of 1536 held by a block of 4 waves, lane-major: thread T
// holds elements 6 T .. 6 T + 5 (three 8-byte loads), the layout the
// exact-sum engine takes (thread T's J terms are terms J T .. J T + J - 1).
// Of the block shapes that split 1536 (waves x terms a thread: 1 x 24, 2 x
// 12, 3 x 8, 4 x 6, 6 x 4, 8 x 3, 12 x 2), 4 x 6 took the least time for a
// fused row tail, alone (decode) and 512 rows at once (prefill): fewer terms
// a thread shorten each wave's serial loops, more waves lengthen the block's
// barriers.
constexpr int kRowWaves = 4, kRowJ = 1536 / (64 * kRowWaves);
__device__ __forceinline__ void load_row6(const float *row, float (&v)[kRowJ]) {
    const float2 *p = reinterpret_cast<const float2 *>(row) + 3 * threadIdx.x;
#pragma unroll
    for (int i = 0; i < 3; i++) {
        const float2 f = p[i];
        v[2 * i] = f.x, v[2 * i + 1] = f.y;
    }
}
__device__ __forceinline__ void store_row6(float *row, const float (&v)[kRowJ]) {
    float2 *p = reinterpret_cast<float2 *>(row) + 3 * threadIdx.x;
#pragma unroll
    for (int i = 0; i < 3; i++) p[i] = make_float2(v[2 * i], v[2 * i + 1]);
}
// The reference's sequential sum of squares (gemma4.c:366-368) of such a row:
// each square rounded on its own, then the in-order fp32 chain through the
// engine.  Every thread of the block calls it and gets the sum.
__device__ __forceinline__ float row6_sum_squares(const float (&x)[kRowJ], EsumShared &sh) {
    float t[kRowJ];
#pragma unroll
    for (int j = 0; j < kRowJ; j++) t[j] = x[j] * x[j];
    return exact_sum_events<kRowWaves, kRowJ, false>(t, 0u, 0.0f, sh);
}
// y = w * (inverse * x) (gemma4.c:371-372).
__device__ __forceinline__ void row6_scale(float (&y)[kRowJ], const float (&w)[kRowJ], float inverse,
                                           const float (&x)[kRowJ]) {
#pragma unroll
    for (int j = 0; j < kRowJ; j++) y[j] = w[j] * (inverse * x[j]);
}

// The reference's sequential sum of squares (gemma4.c:366-368) of a row held
// by a wave as xv[v] = elements 256 v + 4 lane .. + 3.  Squares are computed
// in parallel (each is rounded on its own in the reference too); the chain
// walks the row in order, element k = 256 v + 4 l + c living in lane l,
// register (v, c): each square is broadcast with v_readlane into a scalar
// register and added by the whole wave, so every lane ends with the same sum
// and no LDS or barrier is involved.  The readlanes do not depend on the
// chain and fill its dependent-add stalls.
template <int V>
__device__ __forceinline__ float row_sum_squares(const float4 (&xv)[V]) {
    float sq[V][4];
#pragma unroll
    for (int v = 0; v < V; v++) {
        sq[v][0] = xv[v].x * xv[v].x;
        sq[v][1] = xv[v].y * xv[v].y;
        sq[v][2] = xv[v].z * xv[v].z;
        sq[v][3] = xv[v].w * xv[v].w;
    }
    float sum = 0.0f;
#pragma unroll
    for (int v = 0; v < V; v++)
#pragma unroll
        for (int l = 0; l < 64; l++)
#pragma unroll
            for (int c = 0; c < 4; c++)
                sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sq[v][c]), l));
    return sum;
}

// Widths 256 * V (V = 1, 2: per-head norms of 256 and 512).  Every lane
// holds its 4V values and weights in registers (loaded once, all loads in
// flight); the sum is row_sum_squares.
template <int V>
__global__ __launch_bounds__(256) void k_rmsnorm_reference_v(float *out, const float *in,
                                                             const float *__restrict__ weight,
                                                             float eps, size_t rows) {
    constexpr int W = 256 * V;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const size_t wave_row = (size_t)blockIdx.x * 4 + wave;
    if (wave_row >= rows) return;  // uniform per wave; no block-level barrier follows
    const float4 *x4 = reinterpret_cast<const float4 *>(in + wave_row * W);
    float4 xv[V], wv[V];
#pragma unroll
    for (int v = 0; v < V; v++) xv[v] = x4[v * 64 + lane];
    if (weight) {
        const float4 *w4 = reinterpret_cast<const float4 *>(weight);
#pragma unroll
        for (int v = 0; v < V; v++) wv[v] = w4[v * 64 + lane];
    } else {
#pragma unroll
        for (int v = 0; v < V; v++) wv[v] = make_float4(1.0f, 1.0f, 1.0f, 1.0f);
    }
    const float inverse = 1.0f / sqrtf(row_sum_squares<V>(xv) / (float)W + eps);
    float4 *y4 = reinterpret_cast<float4 *>(out + wave_row * W);
#pragma unroll
    for (int v = 0; v < V; v++)
        y4[v * 64 + lane] = make_float4(wv[v].x * (inverse * xv[v].x), wv[v].y * (inverse * xv[v].y),
                                        wv[v].z * (inverse * xv[v].z), wv[v].w * (inverse * xv[v].w));
}

// Rows of 1536 (the hidden width): one row per block (row6 layout).
__global__ __launch_bounds__(256) void k_rmsnorm_1536(float *out, const float *in,
                                                      const float *__restrict__ weight, float eps) {
    __shared__ EsumShared sh;
    const size_t row = blockIdx.x;
    float x[kRowJ], w[kRowJ];
    load_row6(in + row * 1536, x);
    if (weight) {
        load_row6(weight, w);
    } else {
#pragma unroll
        for (int j = 0; j < kRowJ; j++) w[j] = 1.0f;
    }
    const float inverse = 1.0f / sqrtf(row6_sum_squares(x, sh) / 1536.0f + eps);
    float y[kRowJ];
    row6_scale(y, w, inverse, x);
    store_row6(out + row * 1536, y);
}

// The row-local tail of a sublayer, fused for hidden rows of 1536, reference
// order throughout, one row per block (row6 layout):
//   a = NORM_IN ? rmsnorm(h, w_in) : h                 (gemma4.c:360-373)
//   if ADD:  residual = (residual + a) * scale         (gemma4.c:375-378)
//   b = NORM_OUT ? rmsnorm(residual, w_out) : residual
//   if QUANT: q8, qs = quantize(b)                     (gemma4.c:265-279)
//   if y:     y = b
// It replaces, e.g., rmsnorm + add_and_scale + rmsnorm + quantize between two
// matmuls by one launch.  In-place use (y == h or y == residual) is allowed:
// each thread reads only the elements it writes.  The quantization groups (64
// values) do not align with the threads' 6, so b goes through an LDS row and
// comes back in k_quantize's layout: 16 lanes per group, four values a lane.
template <bool NORM_IN, bool ADD, bool NORM_OUT, bool QUANT>
__global__ __launch_bounds__(256) void k_row_tail(const float *h, const float *__restrict__ w_in,
                                                  float *residual, float scale,
                                                  const float *__restrict__ w_out, float *y,
                                                  int8_t *__restrict__ q8, float *__restrict__ qs,
                                                  float eps) {
    constexpr int W = 1536;
    __shared__ EsumShared sh;
    __shared__ __attribute__((aligned(16))) float s_b[QUANT ? W : 4];
    const int T = threadIdx.x;
    const size_t row = blockIdx.x;
    float r[kRowJ], wi[kRowJ], wo[kRowJ], a[kRowJ];
    // every load first: the weights' and the residual's arrive during the sums
    load_row6(residual + row * W, r);
    if (ADD) load_row6(h + row * W, a);
    if (NORM_IN) load_row6(w_in, wi);
    if (NORM_OUT) load_row6(w_out, wo);
    if (ADD) {
        if (NORM_IN) {
            const float inverse = 1.0f / sqrtf(row6_sum_squares(a, sh) / (float)W + eps);
            row6_scale(a, wi, inverse, a);
        }
#pragma unroll
        for (int j = 0; j < kRowJ; j++) r[j] = (r[j] + a[j]) * scale;
        store_row6(residual + row * W, r);
    }
    if (NORM_OUT) {
        const float inverse = 1.0f / sqrtf(row6_sum_squares(r, sh) / (float)W + eps);
        row6_scale(r, wo, inverse, r);
    }
    if (y) store_row6(y + row * W, r);
    if (QUANT) {
#pragma unroll
        for (int i = 0; i < 3; i++) reinterpret_cast<float2 *>(s_b)[3 * T + i] = make_float2(r[2 * i], r[2 * i + 1]);
        __syncthreads();
        const int lane = T & 63;
        for (int i = T; i < W / 4; i += 256) {  // group i / 16: the 16 lanes of one DPP row
            const float4 x = reinterpret_cast<const float4 *>(s_b)[i];
            float m = fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w)));
#pragma unroll
            for (int o = 8; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 16));
            const float gscale = m / 127.0f;
            const float inverse = gscale > 0.0f ? 1.0f / gscale : 0.0f;
            char4 out;
            out.x = (signed char)(int)rintf(x.x * inverse);
            out.y = (signed char)(int)rintf(x.y * inverse);
            out.z = (signed char)(int)rintf(x.z * inverse);
            out.w = (signed char)(int)rintf(x.w * inverse);
            reinterpret_cast<char4 *>(q8 + row * W)[i] = out;
            if ((lane & 15) == 0) qs[row * (W / 64) + i / 16] = gscale;
        }
    }
}

void launch_row_tail(hipStream_t s, const float *h, const float *w_in, float *residual, float scale,
                     const float *w_out, float *y, int8_t *q8, float *qs, float eps, size_t rows,
                     int norm_in, int add, int norm_out, int quant) {
    if (!rows) return;
    const dim3 grid((unsigned)rows), block(64 * kRowWaves);
#define G4_TAIL(A, B, C, D)                                                                    \
    if (norm_in == A && add == B && norm_out == C && quant == D) {                             \
        hipLaunchKernelGGL((k_row_tail<A, B, C, D>), grid, block, 0, s, h, w_in, residual, scale, \
                           w_out, y, q8, qs, eps);                                       \
        return;                                                                                \
    }
    G4_TAIL(true, true, true, true)     // post-norm, residual add, pre-norm, quantize
    G4_TAIL(true, true, false, true)    // post-norm, residual add, quantize the residual
    G4_TAIL(true, true, false, false)   // post-norm, residual add
    G4_TAIL(false, false, true, true)   // norm, quantize
#undef G4_TAIL
}

// ---------------------------------------------------------------------------
// One token's products fused with the row tail that feeds them (decode,
// reference order).  The tail of the previous sublayer -- k_row_tail's
// arithmetic on a 1536-wide hidden row -- runs at the start of every block,
// all of the block's waves taking part in the exact sums, and leaves the
// quantized row in LDS; the blocks compute it from the same inputs with the
// same code, so every block holds the same bits.  Before the tail, each wave
// has already issued the loads of all of its weight tiles, so the tail runs
// while they are in flight and one launch (and its gap) per tail is saved.
// Block 0 writes the updated residual to res_out; every block reads res_in,
// so the two must differ (the caller alternates two buffers).
// The products (one token, K = 1536, 24 groups): a block covers S 16-row
// strips of each of its NM matrices (S = 1 for EPI_PLAIN: up to three
// matrices that read the same input, blocks taken in matrix order; S = 4 for
// the GELU epilogues: 64 outputs per block, one quantization group), W waves
// per strip-matrix, each taking 24 / W groups; the exact group dots and scale
// products go through LDS and 16 lanes per strip-matrix fold them in group
// order (gemma4.c:216-218).  Epilogues:
//   EPI_PLAIN      out = x W^T
//   EPI_GELU_PAIR  gelu(gate) * up (gemma4.c:309-331), quantized
//   EPI_GELU_MUL   gelu(x W^T) * mul (the per-layer-embedding gate), quantized
// (k_quantize's arithmetic over each block's 64 outputs).
constexpr int kTailGroups = 1536 / 64;

// J = 24 / NW consecutive elements per thread, thread T holding J T ..
// J T + J - 1: the lane-major layout of exact_sum_events.
template <int J>
__device__ __forceinline__ void load_row_j(const float *row, float (&v)[J]) {
    if constexpr (J == 4) {
        const float4 f = reinterpret_cast<const float4 *>(row)[threadIdx.x];
        v[0] = f.x, v[1] = f.y, v[2] = f.z, v[3] = f.w;
    } else if constexpr (J == 2) {
        const float2 f = reinterpret_cast<const float2 *>(row)[threadIdx.x];
        v[0] = f.x, v[1] = f.y;
    } else {
#pragma unroll
        for (int j = 0; j < J; j++) v[j] = row[J * threadIdx.x + j];
    }
}
template <int J>
__device__ __forceinline__ void store_row_j(float *row, const float (&v)[J]) {
    if constexpr (J == 4) {
        reinterpret_cast<float4 *>(row)[threadIdx.x] = make_float4(v[0], v[1], v[2], v[3]);
    } else if constexpr (J == 2) {
        reinterpret_cast<float2 *>(row)[threadIdx.x] = make_float2(v[0], v[1]);
    } else {
#pragma unroll
        for (int j = 0; j < J; j++) row[J * threadIdx.x + j] = v[j];
    }
}

// y = w * (inverse * x), inverse = 1 / sqrt(sum x^2 / 1536 + eps) with the
// sum in index order (gemma4.c:366-372); all NW waves of the block call it.
template <int NW, int J>
__device__ __forceinline__ void tail_rmsnorm(float (&x)[J], const float (&w)[J], float eps,
                                             EsumShared &sh) {
    float t[J];
#pragma unroll
    for (int j = 0; j < J; j++) t[j] = x[j] * x[j];
    const float sum = exact_sum_events<NW, J, false>(t, 0u, 0.0f, sh);
    const float inverse = 1.0f / sqrtf(sum / 1536.0f + eps);
#pragma unroll
    for (int j = 0; j < J; j++) x[j] = w[j] * (inverse * x[j]);
}

// k_row_tail<NORM_IN, ADD, NORM_OUT, QUANT = true> for one row, by the NW
// waves of the block, into LDS: s_q8 (1536 int8 as 384 dwords) and s_qs (24
// group scales).  The loads are split from the arithmetic so that a caller
// can issue them before its own (vector-memory loads complete in order: a
// tail whose inputs queue behind a wave's weight tiles would wait for all of
// them).  compute() ends with a block barrier.
template <int NW, bool NORM_IN, bool ADD, bool NORM_OUT>
struct RowTail {
    static constexpr int J = kTailGroups / NW;
    static_assert(J * NW == kTailGroups, "NW divides 24");
    float r[J], a[J], wi[J], wo[J];
    __device__ __forceinline__ void load(const RowTailJob &tj) {
        load_row_j<J>(tj.res_in, r);
        if (ADD) load_row_j<J>(tj.h, a);
        if (NORM_IN) load_row_j<J>(tj.w_in, wi);
        if (NORM_OUT) load_row_j<J>(tj.w_out, wo);
    }
    __device__ __forceinline__ void compute(const RowTailJob &tj, float *s_row, int *s_q8, float *s_qs,
                                            EsumShared &sh) {
        if (ADD) {
            if (NORM_IN) tail_rmsnorm<NW, J>(a, wi, tj.eps, sh);
#pragma unroll
            for (int j = 0; j < J; j++) r[j] = (r[j] + a[j]) * tj.scale;
            if (blockIdx.x == 0) store_row_j<J>(tj.res_out, r);
        }
        if (NORM_OUT) tail_rmsnorm<NW, J>(r, wo, tj.eps, sh);
        store_row_j<J>(s_row, r);
        __syncthreads();
        // quantize (gemma4.c:265-279) in k_quantize's layout: 16 lanes per
        // group of 64, four values a lane, the block's threads striding over
        // the 384 float4s (a group's 16 lanes are always in one wave)
        for (int T = threadIdx.x; T < 384; T += 64 * NW) {
            const float4 x = reinterpret_cast<const float4 *>(s_row)[T];
            float m = fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w)));
#pragma unroll
            for (int o = 8; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 16));
            const float gscale = m / 127.0f;
            const float inverse = gscale > 0.0f ? 1.0f / gscale : 0.0f;
            char4 q;
            q.x = (signed char)(int)rintf(x.x * inverse);
            q.y = (signed char)(int)rintf(x.y * inverse);
            q.z = (signed char)(int)rintf(x.z * inverse);
            q.w = (signed char)(int)rintf(x.w * inverse);
            reinterpret_cast<char4 *>(s_q8)[T] = q;
            if ((T & 15) == 0) s_qs[T >> 4] = gscale;
        }
        __syncthreads();
    }
};

template <int EPI, int W, int TAIL>
__global__ __launch_bounds__(64 * W * (EPI == EPI_PLAIN ? 1 : EPI == EPI_GELU_PAIR ? 8 : 4))
void k_gemv_tail(GemvJob job, RowTailJob tj) {
    constexpr int NM = EPI == EPI_GELU_PAIR ? 2 : 1, S = EPI == EPI_PLAIN ? 1 : 4, SM = NM * S;
    constexpr int NW = W * SM, NG = kTailGroups / W;
    static_assert(NG * W == kTailGroups, "W divides 24");
    __shared__ EsumShared sh;
    __shared__ __attribute__((aligned(16))) float s_row[1536];
    __shared__ int s_q8[384];
    __shared__ float s_qs[kTailGroups];
    __shared__ float s_d[SM][kTailGroups][16], s_c[SM][kTailGroups][16], s_e[NM][64];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int sm = wave / W, wv = wave % W;
    int mi = EPI == EPI_GELU_PAIR ? sm / S : 0, strip = blockIdx.x * S + sm % S;
    if (EPI == EPI_PLAIN)
        while (mi + 1 < job.count && strip >= job.m[mi].strips) strip -= job.m[mi++].strips;
    const GemvMat mat = job.m[mi];
    const int g0 = wv * NG;
    const int chunk = lane >> 2, b2 = (lane >> 2) & 1, b3 = (lane >> 3) & 1;
    const int row = 4 * (lane & 3) + 2 * b2 + b3;
    const uint4 *tiles = reinterpret_cast<const uint4 *>(mat.w + (size_t)strip * 16 * 1536) + lane;
    const uint16_t *wscale = mat.ws + (size_t)strip * kTailGroups * 16 + row;
    // the tail's inputs first, then the first PRE of this wave's weight tiles,
    // in flight while the tail runs (more would stall the wave at issue: the
    // memory pipeline takes only so many requests, and the tail would then
    // start after the tiles' data instead of beside it); the rest after it
    constexpr int PRE = NG < 4 ? NG : 4;
    RowTail<NW, TAIL != 3, TAIL != 3, TAIL != 2> tail;
    tail.load(tj);
    __builtin_amdgcn_sched_barrier(0);  // keep the tail's loads ahead of the tiles'
    uint4 t[NG];
    uint16_t wsr[NG];
#pragma unroll
    for (int u = 0; u < PRE; u++) {
        t[u] = tiles[(size_t)(g0 + u) * 64];
        wsr[u] = wscale[(g0 + u) * 16];
    }
    __builtin_amdgcn_sched_barrier(0);
    tail.compute(tj, s_row, s_q8, s_qs, sh);
#pragma unroll
    for (int u = PRE; u < NG; u++) {
        t[u] = tiles[(size_t)(g0 + u) * 64];
        wsr[u] = wscale[(g0 + u) * 16];
    }
    // every group's dot first (their butterflies interleave), then the stores
    int d[NG];
#pragma unroll
    for (int u = 0; u < NG; u++) {
        int dd[1];
        const int xx[1] = {s_q8[(g0 + u) * 16 + chunk]};
        gemv_group_dots<1>(t[u], xx, b2, b3, dd);
        d[u] = dd[0];
    }
    if (lane < 16) {
#pragma unroll
        for (int u = 0; u < NG; u++) {
            s_d[sm][g0 + u][row] = (float)d[u];
            s_c[sm][g0 + u][row] = half_bits_to_float(wsr[u]) * s_qs[g0 + u];
        }
    }
    __syncthreads();
    const int tid = threadIdx.x;
    float acc = 0.0f;
    if (tid < 16 * SM) {  // strip-matrix tid / 16, row tid % 16
        const int m = tid >> 4, r = tid & 15;
        for (int g = 0; g < kTailGroups; g++) acc = fmaf(s_d[m][g][r], s_c[m][g][r], acc);
    }
    if (EPI == EPI_PLAIN) {
        if (tid < 16) mat.out[strip * 16 + tid] = acc;
        return;
    }
    if (tid < 16 * SM) s_e[tid >> 6][tid & 63] = acc;
    __syncthreads();
    if (tid >= 64) return;
    const int n = blockIdx.x * 64 + tid;
    const float gl = gelu_table_lookup(s_e[0][tid], job.gelu_table, job.gelu_size, job.gelu_lower,
                                       job.gelu_upper);
    const float v = EPI == EPI_GELU_PAIR ? gl * s_e[NM - 1][tid] : gl * job.mul[n];
    float m = fabsf(v);  // k_quantize's arithmetic over the block's 64 outputs
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    const float scale = m / 127.0f;
    const float inverse = scale > 0.0f ? 1.0f / scale : 0.0f;
    job.q_out[n] = (int8_t)(int)rintf(v * inverse);
    if (tid == 0) job.qs_out[blockIdx.x] = scale;
}

int launch_gemv_tail(hipStream_t s, const GemvJob &job, int epi, const RowTailJob &tj, int tail) {
    int strips = 0;
    for (int i = 0; i < job.count; i++) strips += job.m[i].strips;
    if (job.k != 1536 || job.count < 1 || job.count > 3 || (epi != EPI_PLAIN && job.count != (epi == EPI_GELU_PAIR ? 2 : 1)) ||
        (epi != EPI_PLAIN && (job.m[0].strips % 4 || !job.q_out)) ||
        (epi == EPI_GELU_PAIR && job.m[1].strips != job.m[0].strips) || tail < 1 || tail > 3 ||
        (tail != 3 && tj.res_out == tj.res_in))
        return set_error(G4_ERR_ARG, "fused tail product: bad shape");
    const unsigned blocks = (unsigned)(epi == EPI_PLAIN ? strips : job.m[0].strips / 4);
#define G4_GT(E, WW, T)                                                                     \
    if (epi == E && tail == T) {                                                            \
        constexpr int SM_ = (E == EPI_PLAIN ? 1 : E == EPI_GELU_PAIR ? 8 : 4);              \
        hipLaunchKernelGGL((k_gemv_tail<E, WW, T>), dim3(blocks), dim3(64 * WW * SM_), 0, s, job, tj); \
        return G4_OK;                                                                       \
    }
    // q, k and v: 6 waves a strip (4 groups each); the GELU pair: 8 strip-
    // matrices of one wave (24 groups); the per-layer-embedding gate: 4 strips
    // of 2 waves (12 groups)
    G4_GT(EPI_PLAIN, 6, 1)
    G4_GT(EPI_PLAIN, 6, 2)
    G4_GT(EPI_PLAIN, 6, 3)
    G4_GT(EPI_GELU_PAIR, 1, 1)
    G4_GT(EPI_GELU_MUL, 2, 2)
#undef G4_GT
    return set_error(G4_ERR_ARG, "fused tail product: no kernel for epilogue %d with tail %d", epi, tail);
}

// Any other width (per-op entry point): the same order, plainer loads.
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
            const int batches = width / 64;
            if (batches > 0) sum = chain_lds(reinterpret_cast<const float4 *>(s_sq[wave]), batches);
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
    const dim3 grid((unsigned)((rows + 3) / 4)), block(256);
    // float4 paths need 16-byte aligned rows and weights
    const bool aligned = ((uintptr_t)in % 16 == 0) && ((uintptr_t)out % 16 == 0) &&
                         ((uintptr_t)weight % 16 == 0);
    if (aligned && width == 1536)
        hipLaunchKernelGGL(k_rmsnorm_1536, dim3((unsigned)rows), dim3(64 * kRowWaves), 0, s, out, in, weight, eps);
    else if (aligned && width == 512)
        hipLaunchKernelGGL(k_rmsnorm_reference_v<2>, grid, block, 0, s, out, in, weight, eps, rows);
    else if (aligned && width == 256)
        hipLaunchKernelGGL(k_rmsnorm_reference_v<1>, grid, block, 0, s, out, in, weight, eps, rows);
    else
        hipLaunchKernelGGL(k_rmsnorm_reference, grid, block, 0, s, out, in, weight, width, eps, rows);
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

// Lane l of each 16-lane row receives x from lane l + N of the same row
// (DPP row_shl; lanes past the row's end receive 0).
template <int N>
__device__ __forceinline__ float row_shl(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x100 + N, 0xf, 0xf, true));
}

// Scores of every (token, head, visible key), exact (gemma4.c:281-294): 16
// lanes per key, lane m an fma chain over channels m, m+16, ... (s ascending),
// then the fixed tree.  A block takes TQ tokens x 8 heads against 64 keys: each
// 16-lane group keeps its key's channel slice in registers and reads the query
// rows from LDS, stored [row][m][s] (padded) so a lane's chain is contiguous
// (16-byte LDS loads, bank-conflict free).  scores[(t * 8 + h) * stride + (p - first(t))] for key position p.
// x[0..C) in every lane of a 16-lane row; partner = lane ^ D.  Afterwards
// x[0..C/2) holds x[j] + partner's x[j] for the half of the indices this lane
// keeps: the lower half if bit D of the lane is clear, else the upper half.
template <int D>
__device__ __forceinline__ float row_xor(float v) {
    if constexpr (D == 8) {  // row_ror:8
        return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xf, 0xf, false));
    } else if constexpr (D == 4) {  // row_ror:4 reaches l - 4, row_ror:12 reaches l + 4
        const float down = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xf, 0xf, false));
        const float up = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x12c, 0xf, 0xf, false));
        return (threadIdx.x & 4) ? down : up;
    } else if constexpr (D == 2) {  // quad_perm [2, 3, 0, 1]
        return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4e, 0xf, 0xf, false));
    } else {  // quad_perm [1, 0, 3, 2]
        return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xb1, 0xf, 0xf, false));
    }
}
template <int C, int D, int N>
__device__ __forceinline__ void butterfly_level(float (&x)[N], int lane16) {
    const bool upper = lane16 & D;
#pragma unroll
    for (int j = 0; j < C / 2; j++) {
        const float lo = x[j], hi = x[j + C / 2];
        const float keep = upper ? hi : lo, give = upper ? lo : hi;
        x[j] = keep + row_xor<D>(give);
    }
}

template <int HD, int TQ, int KG>
__global__ __launch_bounds__(256) void k_attn_scores(const float *__restrict__ q,
                                                     const float *__restrict__ key_cache,
                                                     int cache_len, int full, int start_pos, int n,
                                                     const int *__restrict__ pos_dev, size_t stride,
                                                     float *__restrict__ scores) {
    static_assert(KG >= 2, "the butterfly leaves 8 KG / 16 scores a lane: KG = 1 would store none");
    constexpr int S = HD / 16, SP = S + 4;  // +4 floats: the 16 lanes' 16-byte reads hit distinct banks
    __shared__ __attribute__((aligned(16))) float s_q[TQ * 8][16][SP];
    const int t0 = blockIdx.y * TQ;
    const int tn = n - t0 < TQ ? n - t0 : TQ;
    if (pos_dev) start_pos = *pos_dev;
    const int pos_last = start_pos + t0 + tn - 1;
    constexpr int KB = 16 * KG;  // keys per block pass: 16 groups of KG
    const int kfirst = first_visible(start_pos + t0, full);
    if (kfirst + (int)blockIdx.x * KB > pos_last) return;
    const int mask = cache_len - 1, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float *qt = q + (size_t)t0 * 8 * HD;
    {
        // every thread's 16-byte query loads go out before its first LDS
        // write (one load, wait and write at a time would cost a memory
        // latency per float)
        constexpr int QV = TQ * 8 * HD / 4 / 256;
        static_assert(TQ * 8 * HD % 1024 == 0, "whole float4s per thread");
        const int count = tn * 8 * HD;
        float4 qv[QV];
#pragma unroll
        for (int u = 0; u < QV; u++) {
            const int i = 4 * (tid + 256 * u);
            qv[u] = i < count ? *reinterpret_cast<const float4 *>(qt + i) : make_float4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < QV; u++) {
            const int i = 4 * (tid + 256 * u), row = i / HD, j = i % HD;
            if (i < count) {
                s_q[row][(j + 0) & 15][(j + 0) >> 4] = qv[u].x;
                s_q[row][(j + 1) & 15][(j + 1) >> 4] = qv[u].y;
                s_q[row][(j + 2) & 15][(j + 2) >> 4] = qv[u].z;
                s_q[row][(j + 3) & 15][(j + 3) >> 4] = qv[u].w;
            }
        }
    }
    __syncthreads();
    const int m = lane & 15, kg = lane >> 4;
    // A 16-lane group takes KG keys at once, so each q value read from LDS
    // feeds KG fmas (one key per group would make the kernel LDS-bound).
    // Key blocks blockIdx.x, blockIdx.x + gridDim.x, ... (one per block when
    // the grid spans the keys; a fixed grid strides when the position is read
    // from the device)
    for (int kbase = kfirst + blockIdx.x * KB; kbase <= pos_last; kbase += gridDim.x * KB) {
        const int k0 = (wave * 4 + kg) * KG;
        if (kbase + k0 > pos_last) continue;  // uniform within the 16-lane group
        float kv[KG][S];
#pragma unroll
        for (int i = 0; i < KG; i++) {
            const int p = min(kbase + k0 + i, pos_last);  // past the end: a valid row, not written
            const float *kr = key_cache + (size_t)(p & mask) * HD + m;
#pragma unroll
            for (int s = 0; s < S; s++) kv[i][s] = kr[16 * s];
        }
        // The 8 heads x KG keys of a token are independent chains:
        // interleaving them hides the fma latency.
        for (int tt = 0; tt < tn; tt++) {
            const int t = t0 + tt, pos = start_pos + t, first = first_visible(pos, full);
            float acc[8][KG];
#pragma unroll
            for (int h = 0; h < 8; h++)
#pragma unroll
                for (int i = 0; i < KG; i++) acc[h][i] = 0.0f;
#pragma unroll
            for (int s4 = 0; s4 < S / 4; s4++) {
#pragma unroll
                for (int h = 0; h < 8; h++) {
                    const float4 qq = reinterpret_cast<const float4 *>(s_q[tt * 8 + h][m])[s4];
#pragma unroll
                    for (int i = 0; i < KG; i++) {
                        acc[h][i] = fmaf(qq.x, kv[i][4 * s4 + 0], acc[h][i]);
                        acc[h][i] = fmaf(qq.y, kv[i][4 * s4 + 1], acc[h][i]);
                        acc[h][i] = fmaf(qq.z, kv[i][4 * s4 + 2], acc[h][i]);
                        acc[h][i] = fmaf(qq.w, kv[i][4 * s4 + 3], acc[h][i]);
                    }
                }
            }
            // The reference's tree over the 16 lanes -- (l, l+8), then
            // (l, l+4), then (0+2) + (1+3) -- as a transposing butterfly: at
            // each level a lane adds its partner's (lane ^ d) partial sums of
            // one half of the scores and keeps that half, so the same pairs are
            // added (fp addition is commutative) and lane l ends with scores
            // V l / 16 .. of the list v = h KG + i, all lanes storing.
            constexpr int V = 8 * KG;
            float x[V];
#pragma unroll
            for (int h = 0; h < 8; h++)
#pragma unroll
                for (int i = 0; i < KG; i++) x[h * KG + i] = acc[h][i];
            butterfly_level<V, 8>(x, m);
            butterfly_level<V / 2, 4>(x, m);
            butterfly_level<V / 4, 2>(x, m);
            butterfly_level<V / 8, 1>(x, m);
#pragma unroll
            for (int j = 0; j < V / 16; j++) {
                const int v = (V / 16) * m + j, h = v / KG, p = kbase + k0 + v % KG;
                if (p >= first && p <= pos) scores[((size_t)t * 8 + h) * stride + (p - first)] = x[j];
            }
        }
    }
}

// The same scores for many tokens on the fp32 matrix cores (gemma4.c:281-294).
// v_mfma_f32_16x16x1_4b adds one product to each of its 4 x 16 x 16 outputs
// with a single rounding -- fmaf(a, b, c) bit for bit, subnormals, signed
// zeros and overflow included (checked on the chip against the host's fmaf
// over 3.7 M outputs of one and of 16 chained steps) -- so each output can
// carry one of the 16 fma chains the reference runs per score.  A wave holds
// 32 (token, head) rows x 16 keys: lane (b, i) supplies row i of block b's A
// operand and key i of its B operand, so block b of product g steps chain
// m = 4 b + g by channel 16 s + m.  For each s the lane reads one float4 of its
// key (channels 16 s + 4 b .. + 3, components g = 0..3) and one float4 of each
// 16-row half of the queries from LDS, and issues 8 products into 8
// accumulators (2 row halves x 4 g).  Output (block b, register v, lane l) is
// row 4 (l / 16) + v, key l % 16; the reference's tree -- chains (m, m + 8),
// then (m, m + 4), then (0 + 2) + (1 + 3) -- pairs blocks 0/2 and 1/3 of one
// product, then products, all in the same lane and register.
//
// A block stages the 32 query rows of 4 tokens in LDS (the first pass's keys
// already loading) and its 4 waves take 16 keys each per pass; the next pass's
// first keys load while the tree and the stores run.  The grid holds about 512
// blocks (two a CU), each striding over several 64-key passes: with one pass
// a block, staging and pipeline fill cost more than the products.
template <int HD>
__global__ __launch_bounds__(256, 2) void k_attn_scores_mfma(const float *__restrict__ q,
                                                             const float *__restrict__ key_cache,
                                                             int cache_len, int full, int start_pos,
                                                             int n, size_t stride,
                                                             float *__restrict__ scores) {
    typedef float v16 __attribute__((ext_vector_type(16)));
    // CH channel steps of the key per load batch, two batches in flight; QP:
    // the query rows' LDS pitch, +4 floats so the 8 rows one 16-byte read
    // serves per cycle fall on 8 bank groups
    constexpr int S = HD / 16, CH = 2, NCH = S / CH, QP = HD + 4;
    static_assert(NCH % 2 == 0, "the next pass's first batch lands in buffer 0");
    __shared__ __attribute__((aligned(16))) float s_q[32][QP];
    const int t0 = blockIdx.y * 4;
    const int tn = n - t0 < 4 ? n - t0 : 4;
    const int pos_last = start_pos + t0 + tn - 1;
    const int kfirst = first_visible(start_pos + t0, full);
    if (kfirst + (int)blockIdx.x * 64 > pos_last) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, mask = cache_len - 1;
    const int b = lane >> 4, i16 = lane & 15;
    // lane (b, i16)'s slice of key kb + i16 (past the last key: a valid row,
    // never stored)
    auto key_row = [&](int kb) {
        const int p = min(kb + i16, pos_last);
        return key_cache + (size_t)(p & mask) * HD + 4 * b;
    };
    float4 kv[2][CH];
    int kb = kfirst + blockIdx.x * 64 + 16 * wave;
    {
        const float *kr = key_row(kb);
#pragma unroll
        for (int s = 0; s < CH; s++) kv[0][s] = *reinterpret_cast<const float4 *>(kr + 16 * s);
    }
    {
        constexpr int QV = 32 * HD / 4 / 256;
        const float *qt = q + (size_t)t0 * 8 * HD;
        const int count = tn * 8 * HD;
        float4 qv[QV];
#pragma unroll
        for (int u = 0; u < QV; u++) {
            const int i = 4 * (tid + 256 * u);
            qv[u] = i < count ? *reinterpret_cast<const float4 *>(qt + i) : make_float4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < QV; u++) {
            const int i = 4 * (tid + 256 * u);
            *reinterpret_cast<float4 *>(&s_q[i / HD][i % HD]) = qv[u];
        }
    }
    __syncthreads();
    const int kstep = gridDim.x * 64;
    for (; kb <= pos_last; kb += kstep) {  // uniform per wave
        const float *kr = key_row(kb);
        const float *kn = key_row(kb + kstep <= pos_last ? kb + kstep : kb);
        v16 acc[2][4];
#pragma unroll
        for (int r = 0; r < 2; r++)
#pragma unroll
            for (int g = 0; g < 4; g++)
#pragma unroll
                for (int v = 0; v < 16; v++) acc[r][g][v] = 0.0f;
        // batch c from `use` while `fill` receives batch c + 1, or the next
        // pass's first batch after the last one
        auto batch = [&](int c, const float4 (&use)[CH], float4 (&fill)[CH]) __attribute__((always_inline)) {
            const float *src = c + 1 < NCH ? kr + 16 * CH * (c + 1) : kn;
#pragma unroll
            for (int s = 0; s < CH; s++) fill[s] = *reinterpret_cast<const float4 *>(src + 16 * s);
#pragma unroll
            for (int s = 0; s < CH; s++) {
                const int d = 16 * (CH * c + s) + 4 * b;
                const float4 k4 = use[s];
                const float4 qa = *reinterpret_cast<const float4 *>(&s_q[i16][d]);
                const float4 qb = *reinterpret_cast<const float4 *>(&s_q[16 + i16][d]);
                acc[0][0] = __builtin_amdgcn_mfma_f32_16x16x1f32(qa.x, k4.x, acc[0][0], 0, 0, 0);
                acc[1][0] = __builtin_amdgcn_mfma_f32_16x16x1f32(qb.x, k4.x, acc[1][0], 0, 0, 0);
                acc[0][1] = __builtin_amdgcn_mfma_f32_16x16x1f32(qa.y, k4.y, acc[0][1], 0, 0, 0);
                acc[1][1] = __builtin_amdgcn_mfma_f32_16x16x1f32(qb.y, k4.y, acc[1][1], 0, 0, 0);
                acc[0][2] = __builtin_amdgcn_mfma_f32_16x16x1f32(qa.z, k4.z, acc[0][2], 0, 0, 0);
                acc[1][2] = __builtin_amdgcn_mfma_f32_16x16x1f32(qb.z, k4.z, acc[1][2], 0, 0, 0);
                acc[0][3] = __builtin_amdgcn_mfma_f32_16x16x1f32(qa.w, k4.w, acc[0][3], 0, 0, 0);
                acc[1][3] = __builtin_amdgcn_mfma_f32_16x16x1f32(qb.w, k4.w, acc[1][3], 0, 0, 0);
            }
        };
        // a rolled loop: unrolled whole, the compiler hoists every LDS read of
        // the pass and spills
#pragma unroll 1
        for (int c = 0; c < NCH; c += 2) {
            batch(c, kv[0], kv[1]);
            batch(c + 1, kv[1], kv[0]);
        }
        const int key = kb + i16;
#pragma unroll
        for (int r = 0; r < 2; r++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                float u[4];
#pragma unroll
                for (int g = 0; g < 4; g++)
                    u[g] = (acc[r][g][v] + acc[r][g][8 + v]) + (acc[r][g][4 + v] + acc[r][g][12 + v]);
                const float x = (u[0] + u[2]) + (u[1] + u[3]);
                const int row = 16 * r + 4 * b + v, t = t0 + row / 8, h = row % 8;
                const int pos = start_pos + t, first = first_visible(pos, full);
                if (t < n && key >= first && key <= pos)
                    scores[((size_t)t * 8 + h) * stride + (key - first)] = x;
            }
    }
}

// Inclusive max-scan over the 64 lanes (max is exact in any order): DPP row
// shifts within each 16-lane row, then row broadcasts across rows.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_max_step(float x) {
    const float y = __int_as_float(
        __builtin_amdgcn_update_dpp(__float_as_int(-INFINITY), __float_as_int(x), CTRL, ROW_MASK, 0xf, false));
    return fmaxf(x, y);
}
__device__ __forceinline__ float wave_max_scan(float x) {
    x = dpp_max_step<0x111, 0xf>(x);  // row_shr:1
    x = dpp_max_step<0x112, 0xf>(x);  // row_shr:2
    x = dpp_max_step<0x114, 0xf>(x);  // row_shr:4
    x = dpp_max_step<0x118, 0xf>(x);  // row_shr:8
    x = dpp_max_step<0x142, 0xa>(x);  // row_bcast:15 into rows 1 and 3
    x = dpp_max_step<0x143, 0xc>(x);  // row_bcast:31 into rows 2 and 3
    return x;
}
// Lane l receives lane l - 1's value (wave_shr:1; lane 0 receives 0).
__device__ __forceinline__ float wave_shr1(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x138, 0xf, 0xf, false));
}

__device__ void softmax_row_reference(float *v, int count) {
    const int lane = threadIdx.x & 63;
    float carry = v[0];  // max = values[0], sum = 1 (gemma4.c:401)
    float sum = 1.0f;
    float x_next = 1 + lane < count ? v[1 + lane] : -INFINITY;
    for (int base = 1; base < count; base += 64) {
        const float x = x_next;
        const int j_next = base + 64 + lane;
        x_next = j_next < count ? v[j_next] : -INFINITY;
        const float incl = fmaxf(wave_max_scan(x), carry);
        // DPP reads inactive lanes as 0: shift with every lane active, then select
        const float shifted = wave_shr1(incl);
        const float before = lane == 0 ? carry : shifted;
        const bool is_new = x > before;
        // lanes past the end hold x = -inf: their term is expf(-inf) = 0 and
        // adding +0 leaves the (positive) sum unchanged
        const float e = is_new ? expf_libm(before - x) : expf_libm(x - before);
        const uint64_t new_mask = __ballot(is_new);
        // the running sum over this block, in order (exact, see block_advance)
        sum = block_advance(sum, e, 0, new_mask);
        carry = __shfl(incl, 63);
    }
    const float max = carry;
    // four values per lane per pass, loads issued together
    for (int i0 = 0; i0 < count; i0 += 256) {
        float r[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int i = i0 + u * 64 + lane;
            r[u] = v[min(i, count - 1)];
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int i = i0 + u * 64 + lane;
            if (i < count) v[i] = expf_libm(r[u] - max) / sum;
        }
    }
}

// ---------------------------------------------------------------------------
// Long rows (deep-context decode, few rows): one block of NW waves per row,
// in chunks of 64 NW J values, thread T holding values J T .. J T + J - 1 of
// the chunk.  Per chunk:
//   before_i = max(v_0 .. v_{i-1}) (thread-serial, then across lanes and
//   waves, and the maximum of the earlier chunks); a new maximum when
//   v_i > before_i, e_i = expf(before_i - v_i) then, else expf(v_i - before_i)
//   (v_0 is the starting maximum, not a term);
//   the reference's running sum over the e_i in order (sum = sum * e + 1 at a
//   new maximum, else sum += e) through exact_sum_events.
// Then v_i = expf(v_i - max) / sum.  Each value of the result equals the
// one-wave kernel's bit for bit.

// Which values a row holds: a fixed count, or an attention row (t, head)
// whose visible keys follow from the position.  pad64: the row's stride
// leaves room to round the count up to a multiple of 64, and the values
// between are written as 0 (the decode P.V kernel reads whole 64-key tiles).
struct SoftmaxRows {
    int heads, full, start_pos, fixed_count;
    const int *pos_dev;
    int pad64;
    __device__ __forceinline__ int count(int row) const {
        if (fixed_count > 0) return fixed_count;
        const int pos = (pos_dev ? *pos_dev : start_pos) + row / heads;
        return pos + 1 - first_visible(pos, full);
    }
};

// One row of `count` values at x, by the whole block (s_max: NW floats of LDS).
template <int NW, int J>
__device__ __forceinline__ void softmax_row_block(float *x, int count, int pad64, EsumShared &sh, float *s_max) {
    constexpr int C = 64 * NW * J;
    const int T = threadIdx.x, lane = T & 63, wave = T >> 6;
    float run_max = x[0], sum = 1.0f;  // gemma4.c:401
    // 16-byte loads of a thread's J consecutive values when the row allows it
    // (each lane then touches a quarter of the cache lines)
    const bool wide = J % 4 == 0 && ((uintptr_t)x & 15) == 0;
    for (int base = 0; base < count; base += C) {
        float val[J];
#pragma unroll
        for (int j = 0; j < J; j += 4) {
            const int i = base + J * T + j;
            if (J % 4 == 0 && wide && i + 3 < count) {
                const float4 f = *reinterpret_cast<const float4 *>(x + i);
                val[j] = f.x, val[j + 1] = f.y, val[j + 2] = f.z, val[j + 3] = f.w;
            } else {
#pragma unroll
                for (int e = 0; e < 4 && j + e < J; e++)
                    val[j + e] = i + e < count ? x[i + e] : -INFINITY;  // -inf: a zero term
            }
            if (i == 0) val[j] = -INFINITY;  // v_0 is the starting maximum, not a term
        }
        float m = -INFINITY;
#pragma unroll
        for (int j = 0; j < J; j++) m = fmaxf(m, val[j]);
        const float incl = wave_max_scan(m);
        if (lane == 63) s_max[wave] = incl;
        __syncthreads();
        float before = run_max, chunk_max = run_max;
        for (int w = 0; w < NW; w++) {
            if (w < wave) before = fmaxf(before, s_max[w]);
            chunk_max = fmaxf(chunk_max, s_max[w]);
        }
        before = fmaxf(before, dpp_float<0x138, 0xf>(incl, -INFINITY));  // lanes below
        float t[J];
        uint32_t fresh = 0;
#pragma unroll
        for (int j = 0; j < J; j++) {
            const bool is_new = val[j] > before;
            t[j] = is_new ? expf_libm(before - val[j]) : expf_libm(val[j] - before);
            fresh |= (uint32_t)is_new << j;
            before = fmaxf(before, val[j]);
        }
        // (the engine's barriers also order these s_max reads before the next
        // chunk's writes)
        sum = exact_sum_events<NW, J, true>(t, fresh, sum, sh);
        run_max = chunk_max;
    }
    const int end = pad64 ? (count + 63) & ~63 : count;
    if (count <= C) {  // one chunk: a value a lane at a time (short rows skip lanes)
        for (int i = T; i < end; i += 64 * NW) x[i] = i < count ? expf_libm(x[i] - run_max) / sum : 0.0f;
        return;
    }
    // Longer rows chunk by chunk, a chunk's loads all issued first (a value a
    // lane at a time waits out a memory round trip per value: 8K keys on 4
    // waves, 32 of them): each thread rewrites the J values it read in the
    // first pass, every read of which came before the engine's barriers.
    for (int base = 0; base < end; base += C) {
        float v[J];
#pragma unroll
        for (int j = 0; j < J; j += 4) {
            const int i = base + J * T + j;
            if (J % 4 == 0 && wide && i + 3 < count) {
                const float4 f = *reinterpret_cast<const float4 *>(x + i);
                v[j] = f.x, v[j + 1] = f.y, v[j + 2] = f.z, v[j + 3] = f.w;
            } else {
#pragma unroll
                for (int e = 0; e < 4 && j + e < J; e++) v[j + e] = i + e < count ? x[i + e] : 0.0f;
            }
        }
#pragma unroll
        for (int j = 0; j < J; j += 4) {
            const int i = base + J * T + j;
            float o[4];
#pragma unroll
            for (int e = 0; e < 4 && j + e < J; e++)
                o[e] = i + e < count ? expf_libm(v[j + e] - run_max) / sum : 0.0f;
            if (J % 4 == 0 && wide && i + 3 < end) {
                *reinterpret_cast<float4 *>(x + i) = make_float4(o[0], o[1], o[2], o[3]);
            } else {
#pragma unroll
                for (int e = 0; e < 4 && j + e < J; e++)
                    if (i + e < end) x[i + e] = o[e];
            }
        }
    }
}

template <int NW, int J>
__global__ __launch_bounds__(64 * NW) void k_softmax_block(float *__restrict__ v, size_t stride,
                                                           SoftmaxRows spec) {
    __shared__ EsumShared sh;
    __shared__ float s_max[NW];
    const int row = blockIdx.x;
    softmax_row_block<NW, J>(v + (size_t)row * stride, spec.count(row), spec.pad64, sh, s_max);
}

// Softmax of `rows` rows (attention rows (t, head) or rows of a fixed count)
// with at most max_count values, one block per row.
static void launch_softmax_block(hipStream_t s, float *v, size_t stride, int max_count,
                                 SoftmaxRows spec, unsigned rows) {
    if (max_count <= 512)
        hipLaunchKernelGGL((k_softmax_block<8, 1>), dim3(rows), dim3(512), 0, s, v, stride, spec);
    else if (max_count <= 4096)
        hipLaunchKernelGGL((k_softmax_block<16, 4>), dim3(rows), dim3(1024), 0, s, v, stride, spec);
    else  // chunks of 8192 (16384 in one chunk was 1% slower on the decode step at 16K keys)
        hipLaunchKernelGGL((k_softmax_block<16, 8>), dim3(rows), dim3(1024), 0, s, v, stride, spec);
}

// ---------------------------------------------------------------------------
// Long rows of a decode step, in three launches so that only the sequential
// sum stays on one block per row (k_softmax_block, same results bit for bit):
//   k_softmax_terms (every CU): a row is cut into kSplitBlocks ranges of whole
//     64-value tiles; each block takes the maximum before its range (x_0, the
//     starting maximum, and every value before the range: a maximum is the
//     same in any order), then runs k_softmax_block's per-chunk scan over its
//     range and writes each term e_i and whether v_i is a new maximum; the
//     block holding the row's last value writes the row's maximum;
//   k_softmax_sum (a block per row): the reference's running sum over those
//     terms in order (exact_sum_events, which is exact whatever the chunks);
//   k_softmax_norm (every CU): v_i = expf(v_i - max) / sum, and the zeros up
//     to the tile end.
// A row of at most kSplitMin values (known on the device only, with a
// device-side position) is done whole by k_softmax_sum's block, as
// k_softmax_block does it, and the other two launches leave it alone.
constexpr int kSplitBlocks = 32;  // blocks per row: 8 rows of a decode step fill 256 CUs
constexpr int kSplitMin = kSoftmaxSplitMin;

// The running sum is cut into chunks of kSumChunk terms.  Each chunk's
// events and runs (esum_table's, from a predicted start) become entries of a
// list; one wave then walks the list in order from the exact start.
constexpr int kSumChunk = 512;            // 4 waves x 64 lanes x 2 terms
constexpr int kSumFlat = 1024;            // entries the walk holds at once (32 KB of LDS)
struct SumEntry {
    int d;      // run sum in the run's grid (units of its predicted ulp)
    float t;    // the step after the run: its term
    int start;  // the run's first term
    int k;      // the step's term (the chunk's end for a final run, which has no step)
    int meta;   // bit 0: a new maximum (s t + 1); bit 1: no step (a chunk's final run);
                // bit 2: a chunk of too many events (taken by the exact engine);
                // bits 8..15: the run's predicted biased exponent
    int pad[3];
};

struct SoftmaxSplit {
    float *terms;    // [row][stride] the terms e_i (+0 for v_0 and the padding)
    uint8_t *fresh;  // [row][stride] 1 where v_i is a new maximum
    float *max, *sum;  // [row]
    float2 *maps;    // [row][chunks] each chunk's map s -> A s + B (fp32, a prediction)
    SumEntry *ent;   // [row][chunks][64] each chunk's entries
    int *nent;       // [row][chunks] their count, -1 for more than kEsumEvents events
    int chunks;      // per row: stride / kSumChunk, rounded up
};

// Device bytes the split needs for `rows` rows of `stride` values (each part
// 256-byte aligned).
size_t softmax_split_bytes(size_t rows, size_t stride) {
    auto up = [](size_t b) { return (b + 255) & ~(size_t)255; };
    const size_t chunks = (stride + kSumChunk - 1) / kSumChunk;
    return up(rows * stride * sizeof(float)) + up(rows * stride) + 2 * up(rows * sizeof(float)) +
           up(rows * chunks * sizeof(float2)) + up(rows * chunks * 64 * sizeof(SumEntry)) +
           up(rows * chunks * sizeof(int));
}

static SoftmaxSplit softmax_split_carve(void *work, size_t rows, size_t stride) {
    auto up = [](size_t b) { return (b + 255) & ~(size_t)255; };
    const size_t chunks = (stride + kSumChunk - 1) / kSumChunk;
    char *p = static_cast<char *>(work);
    SoftmaxSplit w;
    w.terms = reinterpret_cast<float *>(p);
    p += up(rows * stride * sizeof(float));
    w.fresh = reinterpret_cast<uint8_t *>(p);
    p += up(rows * stride);
    w.max = reinterpret_cast<float *>(p);
    p += up(rows * sizeof(float));
    w.sum = reinterpret_cast<float *>(p);
    p += up(rows * sizeof(float));
    w.maps = reinterpret_cast<float2 *>(p);
    p += up(rows * chunks * sizeof(float2));
    w.ent = reinterpret_cast<SumEntry *>(p);
    p += up(rows * chunks * 64 * sizeof(SumEntry));
    w.nent = reinterpret_cast<int *>(p);
    w.chunks = (int)chunks;
    return w;
}

// The block's range of row values: whole chunks of kSumChunk, the row's
// chunks spread over the grid's x blocks (the last range ends at the row's
// last 64-value tile).
__device__ __forceinline__ void split_range(int count, int &lo, int &hi) {
    const int chunks = (count + kSumChunk - 1) / kSumChunk;
    const int per = (chunks + (int)gridDim.x - 1) / (int)gridDim.x;
    lo = (int)blockIdx.x * per * kSumChunk;
    hi = min(lo + per * kSumChunk, (count + 63) & ~63);
}

template <int J>
__global__ __launch_bounds__(256) void k_softmax_terms(const float *__restrict__ v, size_t stride,
                                                       SoftmaxRows spec, SoftmaxSplit w) {
    constexpr int NW = 4, C = 64 * NW * J;
    static_assert(C == kSumChunk, "a pass of the loop below is one chunk of the running sum");
    __shared__ float s_max[NW], s_ma[NW], s_mb[NW];
    const int row = blockIdx.y, count = spec.count(row);
    const int T = threadIdx.x, lane = T & 63, wave = T >> 6;
    int lo, hi;
    split_range(count, lo, hi);
    if (count <= kSplitMin || lo >= hi) return;  // uniform
    static_assert(J == 2, "a thread's two values are one 8-byte load and store");
    const float *x = v + (size_t)row * stride;
    // values past the row (and v_0, the starting maximum) are -inf: a zero
    // term; values past the range belong to the next block and only follow
    // this block's values
    auto load_chunk = [&](int base, float (&val)[J]) __attribute__((always_inline)) {
        const int i = base + J * T;  // even, and lo, hi, count's tile end are multiples of 64
        const float2 f = i < hi ? *reinterpret_cast<const float2 *>(x + i) : make_float2(0.0f, 0.0f);
        val[0] = i > 0 && i < count && i < hi ? f.x : -INFINITY;
        val[1] = i + 1 < count && i < hi ? f.y : -INFINITY;
    };
    float val[J];
    load_chunk(lo, val);  // in flight with the maximum's loads
    // the maximum before the range (lo is a multiple of 64: 16-byte loads,
    // eight a thread in flight per pass)
    float m = x[0];
    constexpr int PASS = 8 * 4 * 64 * NW;
    for (int i0 = 0; i0 < lo; i0 += PASS) {
        float4 f[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int i = i0 + (k * 64 * NW + T) * 4;
            f[k] = i < lo ? *reinterpret_cast<const float4 *>(x + i) : make_float4(m, m, m, m);
        }
#pragma unroll
        for (int k = 0; k < 8; k++) m = fmaxf(m, fmaxf(fmaxf(f[k].x, f[k].y), fmaxf(f[k].z, f[k].w)));
    }
    m = wave_max_scan(m);
    if (lane == 63) s_max[wave] = m;
    __syncthreads();
    float pre = s_max[0];
#pragma unroll
    for (int k = 1; k < NW; k++) pre = fmaxf(pre, s_max[k]);
    __syncthreads();
    float *terms = w.terms + (size_t)row * stride;
    uint8_t *fresh_out = w.fresh + (size_t)row * stride;
    for (int base = lo; base < hi; base += C) {
        if (base > lo) load_chunk(base, val);
        float mt = -INFINITY;
#pragma unroll
        for (int j = 0; j < J; j++) mt = fmaxf(mt, val[j]);
        const float incl = wave_max_scan(mt);
        if (lane == 63) s_max[wave] = incl;
        __syncthreads();
        float before = pre, chunk_max = pre;
#pragma unroll
        for (int k = 0; k < NW; k++) {
            if (k < wave) before = fmaxf(before, s_max[k]);
            chunk_max = fmaxf(chunk_max, s_max[k]);
        }
        before = fmaxf(before, dpp_float<0x138, 0xf>(incl, -INFINITY));  // lanes below
        float t[J];
        uint32_t fresh = 0;
#pragma unroll
        for (int j = 0; j < J; j++) {
            const bool is_new = val[j] > before;
            t[j] = is_new ? expf_libm(before - val[j]) : expf_libm(val[j] - before);
            fresh |= (uint32_t)is_new << (8 * j);
            before = fmaxf(before, val[j]);
        }
        const int i = base + J * T;
        if (i < hi) {
            *reinterpret_cast<float2 *>(terms + i) = make_float2(t[0], t[1]);
            *reinterpret_cast<uint16_t *>(fresh_out + i) = (uint16_t)fresh;
        }
        // the chunk's map s -> A s + B, in fp32 (the running sum's prediction)
        float la = 1.0f, lb = 0.0f;
#pragma unroll
        for (int j = 0; j < J; j++) {
            const bool f = (fresh >> (8 * j)) & 1;
            const float a = f ? t[j] : 1.0f, b = f ? 1.0f : t[j];
            lb = fmaf(lb, a, b);
            la *= a;
        }
        wave_affine_inclusive(la, lb);
        if (lane == 63) {
            s_ma[wave] = la;
            s_mb[wave] = lb;
        }
        pre = chunk_max;
        __syncthreads();  // s_max is rewritten by the next chunk, s_ma after its first barrier
        if (T == 0) {
            float A = 1.0f, B = 0.0f;
#pragma unroll
            for (int k = 0; k < NW; k++) {
                B = fmaf(s_ma[k], B, s_mb[k]);
                A *= s_ma[k];
            }
            w.maps[(size_t)row * w.chunks + base / kSumChunk] = make_float2(A, B);
        }
    }
    if (hi >= count && T == 0) w.max[row] = pre;
}

// Each chunk of a long row's running sum (every CU): esum_table from the
// chunk's predicted start -- the fp32 maps of the chunks before it composed
// and applied to the sum's start, 1 -- its events and runs written as
// entries; a chunk of more than kEsumEvents events is marked for the exact
// engine.  A run's sum d is in the grid of its predicted binade, which the
// walk checks against the exact sums.
__global__ __launch_bounds__(256) void k_softmax_chunks(SoftmaxRows spec, size_t stride, SoftmaxSplit w) {
    constexpr int NW = 4, J = 2;
    static_assert(64 * NW * J == kSumChunk, "one pass of the engine a chunk");
    __shared__ EsumShared sh;
    __shared__ float s_a[NW], s_b[NW], s_start;
    const int row = blockIdx.y, count = spec.count(row);
    const int T = threadIdx.x, lane = T & 63, wave = T >> 6;
    int lo, hi;
    split_range(count, lo, hi);
    if (count <= kSplitMin || lo >= hi) return;  // uniform
    const float2 *maps = w.maps + (size_t)row * w.chunks;
    const int c0 = lo / kSumChunk, c1 = (hi + kSumChunk - 1) / kSumChunk;
    {  // the predicted start of chunk c0 (c0 < 256: one map a thread)
        float a = 1.0f, b = 0.0f;
        if (T < c0) {
            const float2 m = maps[T];
            a = m.x;
            b = m.y;
        }
        wave_affine_inclusive(a, b);
        if (lane == 63) {
            s_a[wave] = a;
            s_b[wave] = b;
        }
        __syncthreads();
        if (T == max(c0 - 1, 0)) {
            float x = 1.0f;  // gemma4.c:401
            if (c0 > 0) {
                for (int k = 0; k < wave; k++) x = fmaf(s_a[k], x, s_b[k]);
                x = fmaf(a, x, b);
            }
            s_start = x;
        }
        __syncthreads();
    }
    float s_hat = s_start;
    const float *terms = w.terms + (size_t)row * stride;
    const uint8_t *fresh_in = w.fresh + (size_t)row * stride;
    for (int c = c0; c < c1; c++) {
        const int base = c * kSumChunk, i = base + J * T;
        float t[J];
        uint32_t fresh = 0;
#pragma unroll
        for (int j = 0; j < J; j++) {
            t[j] = i + j < count ? terms[i + j] : 0.0f;  // past the row: a zero term
            fresh |= (i + j < count ? (uint32_t)(fresh_in[i + j] & 1) : 0u) << j;
        }
        int P[J], carry;
        const int total = esum_table<NW, J, true>(t, fresh, s_hat, 0, sh, P, carry);
        const int events = min(total, kEsumEvents);
        SumEntry *out = w.ent + ((size_t)row * w.chunks + c) * 64;
        if (T <= events) {  // entry T: the run before event T and the event, or the final run
            const int erun = T == 0 ? biased_exponent(s_hat) : (sh.table[T - 1].meta >> 8) & 0xff;
            SumEntry e;
            e.start = base + (T == 0 ? 0 : sh.table[T - 1].k + 1);
            if (T < events) {
                const EsumEvent x = sh.table[T];
                e.d = x.d;
                e.t = x.t;
                e.k = base + x.k;
                e.meta = (x.meta & 1) | erun << 8;
            } else {
                e.d = sh.last_d;
                e.t = 0.0f;
                e.k = base + kSumChunk;
                e.meta = 2 | erun << 8;
            }
            e.pad[0] = e.pad[1] = e.pad[2] = 0;
            out[T] = e;
        }
        if (T == 0) w.nent[(size_t)row * w.chunks + c] = total > kEsumEvents ? -1 : events + 1;
        const float2 m = maps[c];
        s_hat = fmaf(m.x, s_hat, m.y);
        __syncthreads();  // the table is rewritten by the next chunk
    }
}

// The running sum of a long row from its chunks' entries, or the whole
// softmax of a short one (a block per row).  The entries go to LDS in order
// (at most kSumFlat; beyond that the whole row takes the exact engine); wave
// 0 walks them 64 at a time from the exact sum as esum_pass's resolve does:
// a run adds d u exactly where the exact sum is in the run's predicted binade
// at its start and end, an event is the plain step.  At the first entry whose
// check fails (or a marked chunk), the exact sum before it is known: the
// block runs the exact engine from that run's start to its chunk's end, and
// the walk goes on from the next chunk's first entry.
template <int NW, int J>
__global__ __launch_bounds__(64 * NW) void k_softmax_sum(float *__restrict__ v, SoftmaxRows spec, size_t stride,
                                                         SoftmaxSplit w) {
    static_assert(NW == 16 && J == 8, "the walk's exact engine fills the chunk into 16 waves x 64 lanes");
    constexpr int C = 64 * NW * J;
    __shared__ EsumShared sh;
    __shared__ float s_max[NW];
    __shared__ SumEntry s_flat[kSumFlat];
    __shared__ int s_off[257], s_pos, s_fall;
    __shared__ float s_sum;
    const int row = blockIdx.x, count = spec.count(row);
    const int T = threadIdx.x, lane = T & 63, wave = T >> 6;
    if (count <= kSplitMin) {  // a short row: all of it here
        softmax_row_block<NW, J>(v + (size_t)row * stride, count, spec.pad64, sh, s_max);
        return;
    }
    const float *terms = w.terms + (size_t)row * stride;
    const uint8_t *fresh_in = w.fresh + (size_t)row * stride;
    const int nch = (count + kSumChunk - 1) / kSumChunk;  // <= 256
    const int *nent = w.nent + (size_t)row * w.chunks;
    // entry offsets: chunk c at s_off[c] (a marked chunk takes one entry)
    if (wave == 0) {
        int n[4], tot = 0;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int c = 4 * lane + q;
            n[q] = c < nch ? max(nent[c], 1) : 0;
            tot += n[q];
        }
        int off = wave_add_scan(tot) - tot;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            s_off[4 * lane + q] = off;
            off += n[q];
        }
        if (lane == 63) s_off[256] = off;
    }
    __syncthreads();
    const int total = s_off[nch];
    if (total <= kSumFlat) {
        for (int c = wave; c < nch; c += NW) {  // a wave a chunk
            const int n = nent[c], at = s_off[c];
            const SumEntry *src = w.ent + ((size_t)row * w.chunks + c) * 64;
            if (n < 0) {
                if (lane == 0) {
                    SumEntry e = {};
                    e.start = c * kSumChunk;
                    e.k = (c + 1) * kSumChunk;
                    e.meta = 4;
                    s_flat[at] = e;
                }
            } else if (lane < n) {
                s_flat[at + lane] = src[lane];
            }
        }
        if (T == 0) {
            s_sum = 1.0f;  // gemma4.c:401
            s_pos = 0;
        }
        __syncthreads();
        while (true) {
            if (wave == 0) {
                float s = s_sum;
                int p = s_pos, fall = -1;
                const int m = min(64, total - p);
                if (m > 0) {
                    SumEntry e = {};
                    e.meta = 2;
                    if (lane < m) e = s_flat[p + lane];
                    const int erun = (e.meta >> 8) & 0xff;
                    const bool nonempty = e.k > e.start;
                    const float du = nonempty ? ldexpf((float)e.d, erun - 150) : 0.0f;
                    const bool sp = e.meta & 1, nostep = (e.meta & 6) != 0;
                    const float fa = sp ? e.t : 1.0f, fb = sp ? 1.0f : nostep ? 0.0f : e.t;
                    const int n_entries = __builtin_amdgcn_readfirstlane(m);
                    float at_start = s, at_end = s, outv = s;
                    auto chain_step = [&]() __attribute__((always_inline)) {
                        at_end = at_start + du;
                        outv = at_end * fa + fb;  // s t + 1 at a new maximum, s + t otherwise
                        at_start = dpp_float<0x138, 0xf>(outv, at_start);  // wave_shr:1, lane 0 keeps its own
                    };
                    for (int i = 0; i < n_entries; i += 4) {
                        chain_step();
                        chain_step();
                        chain_step();
                        chain_step();
                    }
                    const int e0 = biased_exponent(at_start), e1 = biased_exponent(at_end);
                    const uint64_t bad = __ballot(lane < m && ((e.meta & 4) || (nonempty && (e0 != erun || (unsigned)(e0 - 27) > 200u || e1 != erun))));
                    if (!bad) {
                        s = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(outv), n_entries - 1));
                        p += m;
                    } else {
                        const int i = (int)__builtin_ctzll(bad);
                        s = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(at_start), i));
                        fall = __builtin_amdgcn_readlane(e.start, i);
                    }
                }
                if (lane == 0) {
                    s_sum = s;
                    s_pos = p;
                    s_fall = fall;
                }
            }
            __syncthreads();
            const int fall = s_fall, pos = s_pos;
            __syncthreads();  // read by every wave before wave 0 writes them again
            if (fall < 0 && pos >= total) break;  // uniform
            if (fall >= 0) {  // the exact engine from term fall to its chunk's end
                const int cb = fall / kSumChunk, base = cb * kSumChunk, i = base + T;
                float t1[1];
                t1[0] = T < kSumChunk && i < count ? terms[i] : 0.0f;  // past the chunk: zero terms
                const uint32_t f1 = T < kSumChunk && i < count ? (uint32_t)(fresh_in[i] & 1) : 0u;
                float s = s_sum;
                int k0 = fall - base;
                while (!esum_pass<NW, 1, true>(t1, f1, s, k0, sh)) {
                }
                __syncthreads();  // every thread has s before it is stored
                if (T == 0) {
                    s_sum = s;
                    s_pos = s_off[cb + 1];
                }
                __syncthreads();
            }
        }
        if (T == 0) w.sum[row] = s_sum;
        return;
    }
    // more entries than the walk holds: the exact engine over the whole row
    auto load = [&](int base, float (&t)[J], uint32_t &fresh) __attribute__((always_inline)) {
        const int i0 = base + J * T;
        fresh = 0;
        if (i0 + J <= count) {
            const float4 a = *reinterpret_cast<const float4 *>(terms + i0);
            const float4 b = *reinterpret_cast<const float4 *>(terms + i0 + 4);
            const uint2 f = *reinterpret_cast<const uint2 *>(fresh_in + i0);
            t[0] = a.x, t[1] = a.y, t[2] = a.z, t[3] = a.w, t[4] = b.x, t[5] = b.y, t[6] = b.z, t[7] = b.w;
#pragma unroll
            for (int j = 0; j < 4; j++) fresh |= ((f.x >> (8 * j)) & 1u) << j | ((f.y >> (8 * j)) & 1u) << (j + 4);
        } else {
#pragma unroll
            for (int j = 0; j < J; j++) {
                const int i = i0 + j;
                t[j] = i < count ? terms[i] : 0.0f;  // past the row: a zero term
                fresh |= (i < count ? (uint32_t)fresh_in[i] : 0u) << j;
            }
        }
    };
    float sum = 1.0f;  // gemma4.c:401
    float t[J];
    uint32_t fresh;
    load(0, t, fresh);
    for (int base = 0; base < count; base += C) {
        // the next chunk's terms are loaded while this one is summed
        float t_next[J] = {};
        uint32_t fresh_next = 0;
        if (base + C < count) load(base + C, t_next, fresh_next);
        sum = exact_sum_events<NW, J, true>(t, fresh, sum, sh);
#pragma unroll
        for (int j = 0; j < J; j++) t[j] = t_next[j];
        fresh = fresh_next;
    }
    if (T == 0) w.sum[row] = sum;
}

__global__ __launch_bounds__(256) void k_softmax_norm(float *__restrict__ v, size_t stride, SoftmaxRows spec,
                                                      SoftmaxSplit w) {
    const int row = blockIdx.y, count = spec.count(row);
    int lo, hi;
    split_range(count, lo, hi);
    const int end = spec.pad64 ? hi : min(hi, count);
    if (count <= kSplitMin || lo >= end) return;
    const float mx = w.max[row], sum = w.sum[row];
    float *x = v + (size_t)row * stride;
    for (int i = lo + (int)threadIdx.x; i < end; i += 256) x[i] = i < count ? expf_libm(x[i] - mx) / sum : 0.0f;
}

// The three launches over `rows` rows; `work` holds softmax_split_bytes(rows, stride).
static void launch_softmax_split(hipStream_t s, float *v, size_t stride, SoftmaxRows spec, unsigned rows,
                                 void *work) {
    const SoftmaxSplit w = softmax_split_carve(work, rows, stride);
    hipLaunchKernelGGL(k_softmax_terms<2>, dim3(kSplitBlocks, rows), dim3(256), 0, s, v, stride, spec, w);
    hipLaunchKernelGGL(k_softmax_chunks, dim3(kSplitBlocks, rows), dim3(256), 0, s, spec, stride, w);
    hipLaunchKernelGGL((k_softmax_sum<16, 8>), dim3(rows), dim3(1024), 0, s, v, spec, stride, w);
    hipLaunchKernelGGL(k_softmax_norm, dim3(kSplitBlocks, rows), dim3(256), 0, s, v, stride, spec, w);
}

// Attention probabilities of every (token, head) row of a prefill pass, a
// block of NW waves per row running softmax_row_block in chunks of 512 NW
// values: one wave for rows of at most a window (a 64-value step at a time
// took 20.7 against 16.6 us for 4096 rows at the start of a prefill), four
// for the long rows of a global layer deep in a prefill (181 against 249 us
// for 4096 rows of 7681-8192 values).
template <int NW>
__global__ __launch_bounds__(64 * NW) void k_attn_softmax_reference(float *__restrict__ scores,
                                                                    int heads, int full, int start_pos,
                                                                    const int *__restrict__ pos_dev,
                                                                    size_t stride) {
    __shared__ EsumShared sh;
    __shared__ float s_max[NW];
    if (pos_dev) start_pos = *pos_dev;
    // last token first: rows grow with the token (causal), so the longest
    // start first and the short ones fill in behind them
    const int h = blockIdx.x, t = gridDim.y - 1 - blockIdx.y;
    const int pos = start_pos + t, keys = pos + 1 - first_visible(pos, full);
    float *row = scores + ((size_t)t * heads + h) * stride;
    if constexpr (NW == 1) {
        // the fewest terms a lane that hold the row in one chunk: the engine's
        // per-term phases shrink with them (a causal chunk's early tokens have
        // short rows; 512 tokens x 8 heads from position 0: 14.2 against
        // 15.6 us with 8 terms a lane)
        if (keys <= 64)
            softmax_row_block<1, 1>(row, keys, 0, sh, s_max);
        else if (keys <= 128)
            softmax_row_block<1, 2>(row, keys, 0, sh, s_max);
        else if (keys <= 256)
            softmax_row_block<1, 4>(row, keys, 0, sh, s_max);
        else
            softmax_row_block<1, 8>(row, keys, 0, sh, s_max);
    } else {
        softmax_row_block<NW, 8>(row, keys, 0, sh, s_max);
    }
}

// Independent rows of `count` values at `stride` (the per-op entry point).
__global__ __launch_bounds__(64) void k_softmax_rows(float *values, int count, size_t stride) {
    softmax_row_reference(values + (size_t)blockIdx.x * stride, count);
}

// out[t][h][d] = fma chain over keys in order (gemma4.c:296-307), on the fp32
// matrix cores: v_mfma_f32_4x4x1_16b adds one product to each output with a
// single rounding (fmaf bit for bit), so one product per key steps 256 chains.
// A wave holds one token's 8 heads x 64 channels as two accumulators of 4
// heads: its 16 blocks are 4-channel groups, lane l supplying channel d0 + l
// of V (operand B) and, as row l % 4 of its block, the probability of head
// h0 + l % 4 (operand A); lane l's output register v is then head h0 + v,
// channel d0 + l.  All 8 heads of a token see the same keys, so a product per
// key visible to the token and none for any other keeps every chain the
// reference's.  A block takes a 64-channel slice for WAVES tokens (one a
// wave); per 64-key tile, V rows are staged in LDS transposed to
// [channel][key] (a lane reads four keys' operand with one 16-byte load) and
// each wave's probabilities [head][key] beside them (rows padded by 4 floats,
// so the 4 heads one read serves sit on different banks); both are prefetched
// DEPTH tiles ahead in registers with unconditional loads.
template <int HD, int WAVES, int DEPTH>
__global__ __launch_bounds__(WAVES * 64) void k_attn_values(float *__restrict__ out,
                                                            const float *__restrict__ probs,
                                                            const float *__restrict__ value_cache,
                                                            int cache_len, int full, int start_pos,
                                                            int n, const int *__restrict__ pos_dev,
                                                            size_t stride, int8_t *__restrict__ q8,
                                                            float *__restrict__ qs) {
    typedef float v4 __attribute__((ext_vector_type(4)));
    constexpr int HEADS = 8;
    constexpr int THREADS = WAVES * 64;
    if (pos_dev) start_pos = *pos_dev;
    constexpr int F4 = 64 * 64 / 4 / THREADS;   // float4 per thread per tile
    __shared__ __attribute__((aligned(16))) float s_v[64][64 + 4];
    __shared__ __attribute__((aligned(16))) float s_p[WAVES][HEADS][64 + 4];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // last tokens first: their windows hold the most tiles
    const int d0 = blockIdx.x * 64, t0 = (gridDim.y - 1 - blockIdx.y) * WAVES;
    const int tn = n - t0 < WAVES ? n - t0 : WAVES;
    const int mask = cache_len - 1;
    const int pos_last = start_pos + t0 + tn - 1;
    const int kfirst = first_visible(start_pos + t0, full);
    const int tiles = (pos_last - kfirst + 64) / 64;

    const int my_t = t0 + wave;
    const bool active = my_t < t0 + tn;
    const int ld_t = active ? my_t : t0 + tn - 1;  // inactive waves load a valid row
    const int my_pos = start_pos + ld_t, my_first = first_visible(my_pos, full);
    const int my_keys = my_pos - my_first + 1;
    const float *prow = probs + (size_t)ld_t * HEADS * stride;

    // V tile loader: thread (kq, cc) covers keys 4 kq .. 4 kq + 3 of channels
    // d0 + 4 cc .. + 3, stored transposed as four 16-byte rows (bank-conflict
    // free: the 8 lanes of an LDS cycle write 8 different key quads)
    static_assert(F4 == 4 && THREADS == 256, "one key quad x channel quad per thread");
    const int kq = tid & 15, cc = tid >> 4;
    auto load_tile = [&](int tile, float4 (&r)[F4]) {
#pragma unroll
        for (int i = 0; i < F4; i++) {
            // keys past the block's last position are never consumed; loading a
            // valid row instead keeps the loads unconditional (no drain)
            const int p = min(kfirst + tile * 64 + 4 * kq + i, pos_last);
            r[i] = *reinterpret_cast<const float4 *>(value_cache + (size_t)(p & mask) * HD + d0 + 4 * cc);
        }
    };
    // probability loader: lane covers key kfirst + 64 tile + lane of its heads
    auto load_p = [&](int tile, float (&r)[HEADS]) {
        const int j = min(max(kfirst + tile * 64 + lane - my_first, 0), my_keys - 1);
#pragma unroll
        for (int e = 0; e < HEADS; e++) r[e] = prow[(size_t)e * stride + j];
    };
    float4 ring[DEPTH][F4];
    float pring[DEPTH][HEADS];
#pragma unroll
    for (int s = 0; s < DEPTH; s++) {
        load_tile(min(s, tiles - 1), ring[s]);
        load_p(min(s, tiles - 1), pring[s]);
    }

    v4 acc_lo = {0.0f, 0.0f, 0.0f, 0.0f}, acc_hi = {0.0f, 0.0f, 0.0f, 0.0f};  // heads 0-3, 4-7

    // One tile: stage ring slot `s` in LDS, refill the slot DEPTH tiles ahead,
    // then run this wave's chains over the tile.  The loop below is unrolled by
    // DEPTH so every slot index is a compile-time constant (precise waits).
    auto step = [&](int tile, float4 (&slot)[F4], float (&pslot)[HEADS]) {
        __syncthreads();  // previous tile fully consumed
        *reinterpret_cast<float4 *>(&s_v[4 * cc + 0][4 * kq]) = make_float4(slot[0].x, slot[1].x, slot[2].x, slot[3].x);
        *reinterpret_cast<float4 *>(&s_v[4 * cc + 1][4 * kq]) = make_float4(slot[0].y, slot[1].y, slot[2].y, slot[3].y);
        *reinterpret_cast<float4 *>(&s_v[4 * cc + 2][4 * kq]) = make_float4(slot[0].z, slot[1].z, slot[2].z, slot[3].z);
        *reinterpret_cast<float4 *>(&s_v[4 * cc + 3][4 * kq]) = make_float4(slot[0].w, slot[1].w, slot[2].w, slot[3].w);
#pragma unroll
        for (int e = 0; e < HEADS; e++) s_p[wave][e][lane] = pslot[e];
        load_tile(min(tile + DEPTH, tiles - 1), slot);  // unconditional refill
        load_p(min(tile + DEPTH, tiles - 1), pslot);
        __syncthreads();
        if (!active || tile >= tiles) return;
        const int p0 = kfirst + tile * 64;
        int k_lo = my_first - p0, k_hi = my_pos - p0 + 1;  // this token's keys in the tile
        if (k_lo < 0) k_lo = 0;
        if (k_hi > 64) k_hi = 64;
        const float *vr = s_v[lane];
        const float *pa = s_p[wave][lane & 3], *pb = s_p[wave][4 + (lane & 3)];
        if (k_lo == 0 && k_hi == 64) {
#pragma unroll
            for (int k4 = 0; k4 < 16; k4++) {
                const v4 v = reinterpret_cast<const v4 *>(vr)[k4];
                const v4 a = reinterpret_cast<const v4 *>(pa)[k4], b = reinterpret_cast<const v4 *>(pb)[k4];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    acc_lo = __builtin_amdgcn_mfma_f32_4x4x1f32(a[j], v[j], acc_lo, 0, 0, 0);
                    acc_hi = __builtin_amdgcn_mfma_f32_4x4x1f32(b[j], v[j], acc_hi, 0, 0, 0);
                }
            }
        } else {
            for (int k = k_lo; k < k_hi; k++) {
                acc_lo = __builtin_amdgcn_mfma_f32_4x4x1f32(pa[k], vr[k], acc_lo, 0, 0, 0);
                acc_hi = __builtin_amdgcn_mfma_f32_4x4x1f32(pb[k], vr[k], acc_hi, 0, 0, 0);
            }
        }
    };
    for (int tile = 0; tile < tiles; tile += DEPTH) {
#pragma unroll
        for (int s = 0; s < DEPTH; s++) step(tile + s, ring[s], pring[s]);
    }
    if (!active) return;
    float o[HEADS];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        o[e] = acc_lo[e];
        o[4 + e] = acc_hi[e];
    }
    if (!q8) {
#pragma unroll
        for (int e = 0; e < HEADS; e++) out[((size_t)my_t * HEADS + e) * HD + d0 + lane] = o[e];
        return;
    }
    // the o projection's input quantized here (k_quantize's arithmetic): the
    // wave's 64 lanes of head e are one 64-channel group of the row
#pragma unroll
    for (int e = 0; e < HEADS; e++) {
        float m = fabsf(o[e]);
#pragma unroll
        for (int x = 32; x > 0; x >>= 1) m = fmaxf(m, __shfl_xor(m, x));
        const float gscale = m / 127.0f;
        const float inverse = gscale > 0.0f ? 1.0f / gscale : 0.0f;
        const size_t at = ((size_t)my_t * HEADS + e) * HD + d0;
        q8[at + lane] = (int8_t)(int)rintf(o[e] * inverse);
        if (lane == 0) qs[at / 64] = gscale;
    }
}

// The row-local tail of the attention projections, one wave per row, in
// reference order (gemma4.c:427-428 for the queries, 437-440 for a new key and
// value): rmsnorm of each query head (q_norm) then RoPE in place; rmsnorm of
// the new key (k_norm) then RoPE, and the weightless rmsnorm of the new value,
// both written into the rings at (start_pos + t) & (cache_len - 1).  Block
// (r, t): r < heads a query head of token t, r = heads its key, heads + 1 its
// value.  Lane l holds elements J l .. J l + J - 1 (J = HD / 64); the sum of
// squares is the sequential one (exact_sum_events on one wave), and element
// e's RoPE partner e + HD / 2 sits in lane l + 32, same register.
template <int HD>
__global__ __launch_bounds__(64) void k_qkv_finish(float *q, int heads, const float *__restrict__ q_norm,
                                                   const float *__restrict__ k_new,
                                                   const float *__restrict__ v_new,
                                                   const float *__restrict__ k_norm, float *key_cache,
                                                   float *value_cache, const float *__restrict__ cosines,
                                                   const float *__restrict__ sines, int pairs,
                                                   int cache_len, int start_pos,
                                                   const int *__restrict__ pos_dev) {
    constexpr int J = HD / 64;
    __shared__ EsumShared sh;
    if (pos_dev) start_pos = *pos_dev;
    const int r = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
    const int pos = start_pos + t;
    const bool is_q = r < heads, is_v = r == heads + 1;
    const float *src = is_q ? q + ((size_t)t * heads + r) * HD : (is_v ? v_new : k_new) + (size_t)t * HD;
    const float *weight = is_q ? q_norm : is_v ? nullptr : k_norm;
    float x[J], w[J], sq[J];
#pragma unroll
    for (int i = 0; i < J; i += 4) {
        const float4 a = *reinterpret_cast<const float4 *>(src + J * lane + i);
        const float4 b = weight ? *reinterpret_cast<const float4 *>(weight + J * lane + i)
                                : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
        x[i] = a.x, x[i + 1] = a.y, x[i + 2] = a.z, x[i + 3] = a.w;
        w[i] = b.x, w[i + 1] = b.y, w[i + 2] = b.z, w[i + 3] = b.w;
    }
#pragma unroll
    for (int i = 0; i < J; i++) sq[i] = x[i] * x[i];
    const float inverse = 1.0f / sqrtf(exact_sum_events<1, J, false>(sq, 0u, 0.0f, sh) / (float)HD + 1e-6f);
#pragma unroll
    for (int i = 0; i < J; i++) x[i] = w[i] * (inverse * x[i]);
    if (!is_v) {
        const bool upper = lane >= 32;
        const float *c = cosines + (size_t)pos * pairs, *sn = sines + (size_t)pos * pairs;
#pragma unroll
        for (int i = 0; i < J; i++) {
            const float other = __shfl_xor(x[i], 32);
            const int jj = J * (lane & 31) + i;  // the pair index
            if (jj < pairs) {
                const float cj = c[jj], sj = sn[jj];
                // first = element jj (lower lane), second = jj + HD / 2 (upper lane)
                x[i] = upper ? x[i] * cj + other * sj : x[i] * cj - other * sj;
            }
        }
    }
    float *dst = is_q ? q + ((size_t)t * heads + r) * HD
                      : (is_v ? value_cache : key_cache) + (size_t)(pos & (cache_len - 1)) * HD;
#pragma unroll
    for (int i = 0; i < J; i += 4)
        *reinterpret_cast<float4 *>(dst + J * lane + i) = make_float4(x[i], x[i + 1], x[i + 2], x[i + 3]);
}

void launch_qkv_finish(hipStream_t s, float *q, int heads, const float *q_norm, const float *k_new,
                       const float *v_new, const float *k_norm, float *key_cache, float *value_cache,
                       const float *cosines, const float *sines, int pairs, int head_dim,
                       int cache_len, int start_pos, const int *pos_dev, size_t n) {
    if (!n) return;
    const dim3 grid((unsigned)(heads + (k_new ? 2 : 0)), (unsigned)n);
    if (head_dim == 256)
        hipLaunchKernelGGL(k_qkv_finish<256>, grid, dim3(64), 0, s, q, heads, q_norm, k_new, v_new,
                           k_norm, key_cache, value_cache, cosines, sines, pairs, cache_len, start_pos,
                           pos_dev);
    else
        hipLaunchKernelGGL(k_qkv_finish<512>, grid, dim3(64), 0, s, q, heads, q_norm, k_new, v_new,
                           k_norm, key_cache, value_cache, cosines, sines, pairs, cache_len, start_pos,
                           pos_dev);
}

// P.V for one token (decode): one wave per block, four heads per wave.  Lane
// 16 r + j runs the fma chain of head 4 g + r over channel c0 + j (block
// (c0 / 16, g, token)), keys in order (gemma4.c:296-307).  Per 64-key tile
// the wave stages V[64 keys][16 channels] in its own LDS as [channel][key]
// rows, so a lane reads its channel with 16-byte loads; the four heads share
// them (the four lanes of a channel read the same address).  Within a row
// key 4 kq + i sits at position 16 i + kq: the loading lane's sixteen values
// then go out as eight two-address writes with no register shuffling, and
// column register m component u holds key 16 (m % 4) + 4 u + m / 4.  Lane
// 16 r + j holds head 4 g + r's probabilities of keys 4 j .. 4 j + 3 (one
// 16-byte load); key 4 J + e reaches every lane of row r as the DPP source of
// its fma (component e, row_newbcast:J).  A tile's 64 fmas are one asm block:
// nothing inside writes a DPP source, so they issue back to back.  With one
// wave per SIMD every instruction costs the chain its issue slot, so loads
// take at most one add of per-lane address arithmetic: V and the
// probabilities are read through buffer descriptors.
//   FULL (a global layer: keys 0 .. pos are cache rows 0 .. pos, no wrap):
//   the V descriptor ends at row `keys`, so rows past the end read as 0.
//   Sliding windows wrap around the ring; their keys are clamped to the last
//   one (a valid row).
// V is prefetched DEPTH tiles ahead, the probabilities DEPTH - 1, in register
// rings by unconditional loads (5 per tile, all countable by vmcnt; past the
// end the probability loads reread the last tile).  The softmax writes 0 for
// the keys between the row's end and its last whole tile, fma(0, v, o) = o
// exactly (o is never -0, v finite or 0), and steps past the last tile skip
// the chain.

template <int HD, int DEPTH, bool FULL, bool QUANT>
__global__ __launch_bounds__(QUANT ? 256 : 64) void k_attn_values_decode(float *__restrict__ out,
                                                                         const float *__restrict__ probs,
                                                                         const float *__restrict__ value_cache,
                                                                         int cache_len, int full, int start_pos,
                                                                         const int *__restrict__ pos_dev,
                                                                         size_t stride, int8_t *__restrict__ q8,
                                                                         float *__restrict__ qs) {
    constexpr int WPB = QUANT ? 4 : 1;  // waves a block; each stages its own tiles
    __shared__ __attribute__((aligned(16))) float s_vw[WPB][2][16][68];  // [wave][slot][channel][position]
    if (pos_dev) start_pos = *pos_dev;
    const int wave = WPB > 1 ? __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) : 0;
    auto &s_v = s_vw[wave];
    const int lane = threadIdx.x & 63, r = lane >> 4, j = lane & 15;
    const int c0 = (blockIdx.x * WPB + wave) * 16, t = blockIdx.z;
    const int pos = start_pos + t, first = FULL ? 0 : first_visible(pos, full);
    const int keys = pos - first + 1, tiles = (keys + 63) / 64, mask = cache_len - 1;
    constexpr uint32_t ROW = HD * 4, TILE = 64 * ROW;  // bytes
    // V loads: lane (kq, cc) = (lane >> 2, lane & 3) takes keys 4 kq .. 4 kq + 3
    // of channels c0 + 4 cc .. + 3
    const int kq = lane >> 2, cc = lane & 3;
    const uint32_t chan = (uint32_t)(c0 + 4 * cc) * 4;
    const int v_rows = FULL ? min(keys, cache_len) : cache_len;
    const __amdgpu_buffer_rsrc_t v_desc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(value_cache), 0, (int)((uint32_t)v_rows * ROW), 0x00020000);
    // probabilities of heads 4 g .. 4 g + 3 (rows `stride` floats apart), up
    // to the last tile of the fourth
    const float *prows = probs + ((size_t)t * 8 + 4 * blockIdx.y) * stride;
    const __amdgpu_buffer_rsrc_t p_desc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(prows), 0, (int)((3 * stride + (size_t)tiles * 64) * 4), 0x00020000);
    const uint32_t p_lane = (uint32_t)((r * stride + 4 * j) * 4);
    typedef float f4 __attribute__((ext_vector_type(4)));  // SROA-friendly (HIP's float4 is not)
    struct VTile {
        f4 v[4];
    };
    auto load16 = [](__amdgpu_buffer_rsrc_t d, uint32_t offset) __attribute__((always_inline)) {
        return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(d, offset, 0, 0));
    };
    auto load_v = [&](int tile, VTile &st) __attribute__((always_inline)) {
        if constexpr (FULL) {
            const uint32_t base = (uint32_t)(4 * kq) * ROW + chan + (uint32_t)tile * TILE;
#pragma unroll
            for (int i = 0; i < 4; i++) st.v[i] = load16(v_desc, base + i * ROW);
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int key = min(tile * 64 + 4 * kq + i, keys - 1);
                st.v[i] = load16(v_desc, (uint32_t)((first + key) & mask) * ROW + chan);
            }
        }
    };
    auto load_p = [&](int tile) __attribute__((always_inline)) {
        return load16(p_desc, p_lane + (uint32_t)min(tile, tiles - 1) * 256);
    };
    auto store_v = [&](int slot, const VTile &st) __attribute__((always_inline)) {
        float *row = &s_v[slot][4 * cc][kq];
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) row[e * 68 + 16 * i] = st.v[i][e];
    };
    float o = 0.0f;
    // The tile's 64 fmas, keys in order: key 4 J + e is p component e of row
    // lane J times column register 4 e + J / 4, component J % 4 (asm operand
    // 5 + 16 e + J).  s_nop 1 first: p may have been written by the VALU just
    // before (the DPP source read hazard).
#define G4_PV_FMA(J, E, C) \
    "v_fmac_f32_dpp %0, %" #E ", %" #C " row_newbcast:" #J " row_mask:0xf bank_mask:0xf\n"
#define G4_PV_KEYS(J, A, B, C, D) G4_PV_FMA(J, 1, A) G4_PV_FMA(J, 2, B) G4_PV_FMA(J, 3, C) G4_PV_FMA(J, 4, D)
#define G4_PV_COL(M) "v"(col[M].x), "v"(col[M].y), "v"(col[M].z), "v"(col[M].w)
    auto chain64 = [&](const f4 (&col)[16], f4 p) __attribute__((always_inline)) {
        asm volatile("s_nop 1\n"
                     G4_PV_KEYS(0, 5, 21, 37, 53) G4_PV_KEYS(1, 6, 22, 38, 54)
                     G4_PV_KEYS(2, 7, 23, 39, 55) G4_PV_KEYS(3, 8, 24, 40, 56)
                     G4_PV_KEYS(4, 9, 25, 41, 57) G4_PV_KEYS(5, 10, 26, 42, 58)
                     G4_PV_KEYS(6, 11, 27, 43, 59) G4_PV_KEYS(7, 12, 28, 44, 60)
                     G4_PV_KEYS(8, 13, 29, 45, 61) G4_PV_KEYS(9, 14, 30, 46, 62)
                     G4_PV_KEYS(10, 15, 31, 47, 63) G4_PV_KEYS(11, 16, 32, 48, 64)
                     G4_PV_KEYS(12, 17, 33, 49, 65) G4_PV_KEYS(13, 18, 34, 50, 66)
                     G4_PV_KEYS(14, 19, 35, 51, 67) G4_PV_KEYS(15, 20, 36, 52, 68)
                     : "+v"(o)
                     : "v"(p.x), "v"(p.y), "v"(p.z), "v"(p.w), G4_PV_COL(0), G4_PV_COL(1),
                       G4_PV_COL(2), G4_PV_COL(3), G4_PV_COL(4), G4_PV_COL(5), G4_PV_COL(6),
                       G4_PV_COL(7), G4_PV_COL(8), G4_PV_COL(9), G4_PV_COL(10), G4_PV_COL(11),
                       G4_PV_COL(12), G4_PV_COL(13), G4_PV_COL(14), G4_PV_COL(15));
    };
#undef G4_PV_COL
#undef G4_PV_KEYS
#undef G4_PV_FMA
    // V of tile u in v_ring[u % DEPTH], its probabilities in p_ring[u % DEPTH]
    VTile v_ring[DEPTH];
    f4 p_ring[DEPTH];
#pragma unroll
    for (int s = 0; s < DEPTH; s++) {
        load_v(s, v_ring[s]);
        p_ring[s] = load_p(s);
    }
    store_v(0, v_ring[0]);
    load_v(DEPTH, v_ring[0]);
    // step s of a round (tile u = base + s, u % DEPTH = s): tile u is in LDS
    // slot u & 1; its column is read, then tile u + 1 goes to the other slot
    // (last read by tile u - 1: a wave's LDS accesses complete in order) and
    // its ring slot is refilled with tile u + 1 + DEPTH; after the chain, p_ring[s]
    // is refilled with tile u + DEPTH's probabilities.  always_inline: the
    // rings must stay in registers.
    auto step = [&](int tile, VTile &next, f4 &p) __attribute__((always_inline)) {
        f4 col[16];  // this lane's channel, the tile's 64 keys: all reads issued first
        const f4 *src = reinterpret_cast<const f4 *>(&s_v[tile & 1][j][0]);
#pragma unroll
        for (int i = 0; i < 16; i++) col[i] = src[i];
        store_v((tile + 1) & 1, next);
        load_v(tile + 1 + DEPTH, next);  // unconditional: past the end, valid memory
        if (tile < tiles) chain64(col, p);
        p = load_p(tile + DEPTH);
    };
    // The steps are written out (a dynamically indexed ring would live in
    // scratch memory).
    static_assert(DEPTH == 8, "the steps below are written out for 8 ring slots");
    for (int tile = 0; tile < tiles; tile += DEPTH) {
        step(tile + 0, v_ring[1], p_ring[0]);
        step(tile + 1, v_ring[2], p_ring[1]);
        step(tile + 2, v_ring[3], p_ring[2]);
        step(tile + 3, v_ring[4], p_ring[3]);
        step(tile + 4, v_ring[5], p_ring[4]);
        step(tile + 5, v_ring[6], p_ring[5]);
        step(tile + 6, v_ring[7], p_ring[6]);
        step(tile + 7, v_ring[0], p_ring[7]);
    }
    if constexpr (!QUANT) {
        out[((size_t)t * 8 + 4 * blockIdx.y + r) * HD + c0 + j] = o;
    } else {
        // The block holds channels 64 x .. 64 x + 63 of four heads: one
        // quantization group each (gemma4.c:264-279, k_quantize's arithmetic),
        // wave w taking head 4 y + w.  Only the quantized rows are written.
        __shared__ float s_o[4][64];  // [head][channel]
        s_o[r][wave * 16 + j] = o;
        __syncthreads();
        const float x = s_o[wave][lane];
        float m = fabsf(x);
#pragma unroll
        for (int d = 32; d > 0; d >>= 1) m = fmaxf(m, __shfl_xor(m, d));
        const float scale = m / 127.0f;
        const float inverse = scale > 0.0f ? 1.0f / scale : 0.0f;
        const size_t at = ((size_t)t * 8 + 4 * blockIdx.y + wave) * HD + (size_t)blockIdx.x * 64;
        q8[at + lane] = (int8_t)(int)rintf(x * inverse);
        if (lane == 0) qs[at / 64] = scale;
    }
}

// k_attn_values_decode over a global layer (FULL, fp32 out) with the tile
// staging on a second wave.  Wave 1 (the producer, on another SIMD) loads the
// 64-key V tiles of its 16 channels DEPTH tiles ahead in registers and
// writes each, transposed and permuted as above, into LDS slot tile & 3;
// wave 0 (the chain) only reads each tile's column and runs its 64 DPP fmas,
// so the staging no longer takes the chain's issue slots.  The chain reads
// tile u + 1 while it runs tile u.  One barrier every two tiles: before the
// first the producer has written tiles 0-2, and the chain reads tile 0
// between it and a second; barrier m + 2 comes after the chain's tiles 2m
// and 2m + 1 (it then has read, and waited for, tiles up to 2m + 2), and the
// producer writes tiles 2m + 3 and 2m + 4 before it, into the slots of
// tiles 2m - 1 and 2m, which the chain finished reading before barrier
// m + 1.  Both waves pass the same 2 + tiles / 2 barriers.
constexpr int kWaitLgkm0 = 0xC07F;  // s_waitcnt lgkmcnt(0), vmcnt and expcnt untouched

template <int HD, int DEPTH>
__global__ __launch_bounds__(128) void k_attn_values_decode_pc(float *__restrict__ out,
                                                               const float *__restrict__ probs,
                                                               const float *__restrict__ value_cache,
                                                               int cache_len, int start_pos,
                                                               const int *__restrict__ pos_dev,
                                                               size_t stride) {
    __shared__ __attribute__((aligned(16))) float s_v[4][16][68];  // [slot][channel][position]
    if (pos_dev) start_pos = *pos_dev;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, r = lane >> 4, j = lane & 15;
    const int c0 = blockIdx.x * 16, t = blockIdx.z;
    const int pos = start_pos + t, keys = pos + 1, tiles = (keys + 63) / 64;
    constexpr uint32_t ROW = HD * 4, TILE = 64 * ROW;  // bytes
    typedef float f4 __attribute__((ext_vector_type(4)));
    auto load16 = [](__amdgpu_buffer_rsrc_t d, uint32_t offset) __attribute__((always_inline)) {
        return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(d, offset, 0, 0));
    };
    static_assert(DEPTH == 8, "the steps below are written out for 8 ring slots");
    if (wave == 1) {
        // V loads: lane (kq, cc) takes keys 4 kq .. 4 kq + 3 of channels
        // c0 + 4 cc .. + 3; the descriptor ends at row `keys`, so rows past
        // the end (and whole tiles past the last) read as 0
        const int kq = lane >> 2, cc = lane & 3;
        const uint32_t chan = (uint32_t)(c0 + 4 * cc) * 4;
        const int v_rows = min(keys, cache_len);
        const __amdgpu_buffer_rsrc_t v_desc = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float *>(value_cache), 0, (int)((uint32_t)v_rows * ROW), 0x00020000);
        struct VTile {
            f4 v[4];
        };
        auto load_v = [&](int tile, VTile &st) __attribute__((always_inline)) {
            const uint32_t base = (uint32_t)(4 * kq) * ROW + chan + (uint32_t)tile * TILE;
#pragma unroll
            for (int i = 0; i < 4; i++) st.v[i] = load16(v_desc, base + i * ROW);
        };
        auto store_v = [&](int slot, const VTile &st) __attribute__((always_inline)) {
            float *row = &s_v[slot][4 * cc][kq];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int e = 0; e < 4; e++) row[e * 68 + 16 * i] = st.v[i][e];
        };
        VTile ring[DEPTH];  // tile u in ring[u % DEPTH]
#pragma unroll
        for (int s = 0; s < DEPTH; s++) load_v(s, ring[s]);
        // tile u into LDS slot u & 3, its ring slot refilled with tile u + DEPTH
        auto put = [&](int slot, int u, VTile &st) __attribute__((always_inline)) {
            store_v(slot, st);
            load_v(u + DEPTH, st);
        };
        put(0, 0, ring[0]);
        put(1, 1, ring[1]);
        put(2, 2, ring[2]);
        __syncthreads();
        __syncthreads();  // the chain has read tile 0: slot 0 is free
        // One barrier per pair of tiles: pair m puts tiles 2m + 3 and 2m + 4.
        // Whole passes of four pairs run in a loop with no exit inside, so that
        // the compiler keeps each refill where it is written and waits for a
        // tile's own loads only (an early exit made it sink the refills past
        // the exits and wait for nearly every load in flight); the last pairs
        // follow the loop.
        const int pairs = tiles / 2;
        int m = 0;
        for (; m + 4 <= pairs; m += 4) {
            put(3, 2 * m + 3, ring[3]);
            put(0, 2 * m + 4, ring[4]);
            __syncthreads();
            put(1, 2 * m + 5, ring[5]);
            put(2, 2 * m + 6, ring[6]);
            __syncthreads();
            put(3, 2 * m + 7, ring[7]);
            put(0, 2 * m + 8, ring[0]);
            __syncthreads();
            put(1, 2 * m + 9, ring[1]);
            put(2, 2 * m + 10, ring[2]);
            __syncthreads();
        }
        const int rest = pairs - m;
        if (rest > 0) {
            put(3, 2 * m + 3, ring[3]);
            put(0, 2 * m + 4, ring[4]);
            __syncthreads();
        }
        if (rest > 1) {
            put(1, 2 * m + 5, ring[5]);
            put(2, 2 * m + 6, ring[6]);
            __syncthreads();
        }
        if (rest > 2) {
            put(3, 2 * m + 7, ring[7]);
            put(0, 2 * m + 8, ring[0]);
            __syncthreads();
        }
        return;
    }
    // the chain: probabilities of heads 4 y .. 4 y + 3 (rows `stride` floats
    // apart), up to the last tile of the fourth, DEPTH tiles ahead
    const float *prows = probs + ((size_t)t * 8 + 4 * blockIdx.y) * stride;
    const __amdgpu_buffer_rsrc_t p_desc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(prows), 0, (int)((3 * stride + (size_t)tiles * 64) * 4), 0x00020000);
    const uint32_t p_lane = (uint32_t)((r * stride + 4 * j) * 4);
    auto load_p = [&](int tile) __attribute__((always_inline)) {
        return load16(p_desc, p_lane + (uint32_t)min(tile, tiles - 1) * 256);
    };
    float o = 0.0f;
#define G4_PV_FMA(J, E, C) \
    "v_fmac_f32_dpp %0, %" #E ", %" #C " row_newbcast:" #J " row_mask:0xf bank_mask:0xf\n"
#define G4_PV_KEYS(J, A, B, C, D) G4_PV_FMA(J, 1, A) G4_PV_FMA(J, 2, B) G4_PV_FMA(J, 3, C) G4_PV_FMA(J, 4, D)
#define G4_PV_COL(M) "v"(col[M].x), "v"(col[M].y), "v"(col[M].z), "v"(col[M].w)
    auto chain64 = [&](const f4 (&col)[16], f4 p) __attribute__((always_inline)) {
        asm volatile("s_nop 1\n"
                     G4_PV_KEYS(0, 5, 21, 37, 53) G4_PV_KEYS(1, 6, 22, 38, 54)
                     G4_PV_KEYS(2, 7, 23, 39, 55) G4_PV_KEYS(3, 8, 24, 40, 56)
                     G4_PV_KEYS(4, 9, 25, 41, 57) G4_PV_KEYS(5, 10, 26, 42, 58)
                     G4_PV_KEYS(6, 11, 27, 43, 59) G4_PV_KEYS(7, 12, 28, 44, 60)
                     G4_PV_KEYS(8, 13, 29, 45, 61) G4_PV_KEYS(9, 14, 30, 46, 62)
                     G4_PV_KEYS(10, 15, 31, 47, 63) G4_PV_KEYS(11, 16, 32, 48, 64)
                     G4_PV_KEYS(12, 17, 33, 49, 65) G4_PV_KEYS(13, 18, 34, 50, 66)
                     G4_PV_KEYS(14, 19, 35, 51, 67) G4_PV_KEYS(15, 20, 36, 52, 68)
                     : "+v"(o)
                     : "v"(p.x), "v"(p.y), "v"(p.z), "v"(p.w), G4_PV_COL(0), G4_PV_COL(1),
                       G4_PV_COL(2), G4_PV_COL(3), G4_PV_COL(4), G4_PV_COL(5), G4_PV_COL(6),
                       G4_PV_COL(7), G4_PV_COL(8), G4_PV_COL(9), G4_PV_COL(10), G4_PV_COL(11),
                       G4_PV_COL(12), G4_PV_COL(13), G4_PV_COL(14), G4_PV_COL(15));
    };
#undef G4_PV_COL
#undef G4_PV_KEYS
#undef G4_PV_FMA
    f4 p_ring[DEPTH];  // tile u's probabilities in p_ring[u % DEPTH]
#pragma unroll
    for (int s = 0; s < DEPTH; s++) p_ring[s] = load_p(s);
    auto read_col = [&](int slot, f4 (&col)[16]) __attribute__((always_inline)) {
        const f4 *src = reinterpret_cast<const f4 *>(&s_v[slot][j][0]);
#pragma unroll
        for (int i = 0; i < 16; i++) col[i] = src[i];
    };
    // The reads of a column must be complete before the barrier that lets the
    // producer overwrite its slot, and the compiler would otherwise sink LDS
    // loads past a barrier to their first use: an empty asm that takes the
    // registers keeps them (and the wait for them) ahead of it.
    auto pin = [](f4 (&col)[16]) __attribute__((always_inline)) {
        asm volatile("" : "+v"(col[0]), "+v"(col[1]), "+v"(col[2]), "+v"(col[3]), "+v"(col[4]), "+v"(col[5]),
                          "+v"(col[6]), "+v"(col[7]), "+v"(col[8]), "+v"(col[9]), "+v"(col[10]), "+v"(col[11]),
                          "+v"(col[12]), "+v"(col[13]), "+v"(col[14]), "+v"(col[15]));
    };
    f4 col_a[16], col_b[16];  // tile u's column: col_a for even u, col_b for odd
    __syncthreads();  // tiles 0-2 are in slots 0-2
    read_col(0, col_a);
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    pin(col_a);
    __syncthreads();  // slot 0 may take tile 4
    // step u: read tile u + 1 (slot (u + 1) & 3) while tile u's chain runs,
    // then wait for those reads; a barrier after each odd u
    auto step = [&](int slot, int u, const f4 (&cur)[16], f4 (&next)[16], f4 &p) __attribute__((always_inline)) {
        read_col(slot, next);
        chain64(cur, p);
        p = load_p(u + DEPTH);
        __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
        pin(next);
    };
    // whole passes of 8 tiles with no exit inside (exact waits, as for the
    // producer), then the last 0-7 tiles; a barrier after every odd tile
    int u = 0;
    for (; u + DEPTH <= tiles; u += DEPTH) {
        step(1, u + 0, col_a, col_b, p_ring[0]);
        step(2, u + 1, col_b, col_a, p_ring[1]);
        __syncthreads();
        step(3, u + 2, col_a, col_b, p_ring[2]);
        step(0, u + 3, col_b, col_a, p_ring[3]);
        __syncthreads();
        step(1, u + 4, col_a, col_b, p_ring[4]);
        step(2, u + 5, col_b, col_a, p_ring[5]);
        __syncthreads();
        step(3, u + 6, col_a, col_b, p_ring[6]);
        step(0, u + 7, col_b, col_a, p_ring[7]);
        __syncthreads();
    }
    const int rem = tiles - u;
    if (rem > 0) step(1, u + 0, col_a, col_b, p_ring[0]);
    if (rem > 1) {
        step(2, u + 1, col_b, col_a, p_ring[1]);
        __syncthreads();
    }
    if (rem > 2) step(3, u + 2, col_a, col_b, p_ring[2]);
    if (rem > 3) {
        step(0, u + 3, col_b, col_a, p_ring[3]);
        __syncthreads();
    }
    if (rem > 4) step(1, u + 4, col_a, col_b, p_ring[4]);
    if (rem > 5) {
        step(2, u + 5, col_b, col_a, p_ring[5]);
        __syncthreads();
    }
    if (rem > 6) step(3, u + 6, col_a, col_b, p_ring[6]);
    out[((size_t)t * 8 + 4 * blockIdx.y + r) * HD + c0 + j] = o;
}

int launch_attend_reference(hipStream_t s, float *out, const float *q, const float *key_cache,
                            const float *value_cache, int cache_len, int head_dim, int heads,
                            int full, int start_pos, const int *pos_dev, size_t n, int8_t *q8,
                            float *qs, const FixedScratch *fixed) {
    if (!n) return G4_OK;
    if (heads != 8) return set_error(G4_ERR_ARG, "reference-order attention needs 8 query heads");
    if (pos_dev && n != 1) return set_error(G4_ERR_ARG, "device-side positions are for one token");
    const int last_pos = start_pos + (int)n - 1;
    // Keys a row can see, at most; with a device-side position the bound must
    // hold for every position, so it is the cache's.
    const int max_keys = pos_dev ? (full ? G4_MAX_CONTEXT : G4_WINDOW)
                                 : full ? last_pos + 1 : (last_pos + 1 < G4_WINDOW ? last_pos + 1 : G4_WINDOW);
    const size_t stride = ((size_t)max_keys + 63) & ~(size_t)63;
    const size_t score_floats = n * heads * stride;
    // decode rows that may be long: the softmax split over the CUs, its
    // buffers after the scores
    const bool split = n <= 4 && max_keys > kSplitMin;
    const size_t score_bytes = (score_floats * sizeof(float) + 255) & ~(size_t)255;
    const size_t need = score_bytes + (split ? softmax_split_bytes(n * heads, stride) : 0);
    float *scores = nullptr;
    if (fixed) {
        if (need > fixed->bytes)
            return set_error(G4_ERR_ARG, "attention needs %zu bytes of scratch, more than the fixed %zu",
                             need, fixed->bytes);
        scores = (float *)fixed->ptr;
    } else {
        int rc = scratch_reserve(0, need);
        if (rc) return rc;
        scores = scratch().attn;
    }
    // key blocks spanned by one block of tokens: its first token's window
    // start to its last token (a fixed count with a device-side position:
    // the kernel then strides over the blocks it needs)
    // blocks of kb keys
    auto key_blocks = [&](int tq, int kb) -> unsigned {
        if (pos_dev) return full ? 512u : (unsigned)((G4_WINDOW + kb - 1) / kb);
        const int tokens = (int)n < tq ? (int)n : tq;
        const int widest = full ? last_pos + 1 : G4_WINDOW - 1 + tokens;
        const int span = widest < last_pos + 1 ? widest : last_pos + 1;
        const unsigned blocks = (unsigned)((span + kb - 1) / kb);
        // many tokens over a long context: a block strides over several key
        // blocks, so its staged queries serve more keys
        const unsigned cap = (unsigned)(1024 / kb);
        return n > 4 && blocks > cap ? cap : blocks;
    };
    const unsigned nn = (unsigned)n;
    // Decode (at most 4 tokens) on the VALU kernel: 2 keys per 16-lane group
    // over the window, where the 512 keys then span 16 blocks instead of 8; 4
    // over a long context.  The matrix-core kernel's 32-row tiles would be
    // three quarters empty there.
#define G4_SCORES(HD, TQ, KG)                                                                     \
    hipLaunchKernelGGL((k_attn_scores<HD, TQ, KG>), dim3(key_blocks(TQ, 16 * KG), (nn + TQ - 1) / TQ), \
                       dim3(256), 0, s, q, key_cache, cache_len, full, start_pos, (int)n, pos_dev,  \
                       stride, scores)
    if (n > 4) {
        // many tokens: the matrix-core kernel, 4 tokens a block; about 512
        // blocks (two a CU), each striding over the rest of its key blocks
        const unsigned ty = (nn + 3) / 4;
        unsigned bx = key_blocks(4, 64);
        const unsigned fit = 512u / ty > 1u ? 512u / ty : 1u;
        if (bx > fit) bx = fit;
        if (head_dim == 256)
            hipLaunchKernelGGL(k_attn_scores_mfma<256>, dim3(bx, ty), dim3(256), 0, s, q, key_cache,
                               cache_len, full, start_pos, (int)n, stride, scores);
        else
            hipLaunchKernelGGL(k_attn_scores_mfma<512>, dim3(bx, ty), dim3(256), 0, s, q, key_cache,
                               cache_len, full, start_pos, (int)n, stride, scores);
    } else if (head_dim == 256) {
        G4_SCORES(256, 6, 2);  // decode: 32-key blocks, twice the blocks over the window
    } else {
        G4_SCORES(512, 1, 4);
    }
#undef G4_SCORES
    if (n <= 4) {  // decode: few rows, a block per row (the sum's block, when split)
        const SoftmaxRows spec{heads, full, start_pos, 0, pos_dev, 1};
        if (split)
            launch_softmax_split(s, scores, stride, spec, (unsigned)(n * heads),
                                 reinterpret_cast<char *>(scores) + score_bytes);
        else
            launch_softmax_block(s, scores, stride, max_keys, spec, (unsigned)(n * heads));
    } else if (max_keys <= 1024) {
        hipLaunchKernelGGL(k_attn_softmax_reference<1>, dim3((unsigned)heads, nn), dim3(64), 0, s,
                           scores, heads, full, start_pos, pos_dev, stride);
    } else {
        hipLaunchKernelGGL(k_attn_softmax_reference<4>, dim3((unsigned)heads, nn), dim3(256), 0, s,
                           scores, heads, full, start_pos, pos_dev, stride);
    }
    const unsigned slices = (unsigned)(head_dim / 64);
    if (n <= 4) {  // decode: a wave per (16 channels, 4 heads, token), deep prefetch; with
                   // q8 over a window, blocks of 4 such waves (64 channels) quantize their
                   // rows in place of the fp32 ones.  (Over a long context, four chains
                   // sharing a CU run at half speed: those waves keep a CU each and the
                   // rows are quantized after.)
        const bool fuse = q8 && !full;
        const unsigned wpb = fuse ? 4u : 1u;
        dim3 grid((unsigned)(head_dim / 16) / wpb, 2, nn);
#define G4_PV_DECODE(HD, FULL, QUANT)                                                                 \
    hipLaunchKernelGGL((k_attn_values_decode<HD, 8, FULL, QUANT>), grid, dim3(64 * wpb), 0, s, out,   \
                       scores, value_cache, cache_len, full, start_pos, pos_dev, stride, q8, qs)
#define G4_PV_DECODE_Q(HD, FULL)  \
    if (fuse)                     \
        G4_PV_DECODE(HD, FULL, true); \
    else                          \
        G4_PV_DECODE(HD, FULL, false)
        // a global layer: the staging on a second wave of each block
#define G4_PV_DECODE_PC(HD)                                                                        \
    hipLaunchKernelGGL((k_attn_values_decode_pc<HD, 8>), dim3((unsigned)(head_dim / 16), 2, nn),    \
                       dim3(128), 0, s, out, scores, value_cache, cache_len, start_pos, pos_dev, stride)
        if (head_dim == 256) {
            if (full) G4_PV_DECODE_PC(256);
            else G4_PV_DECODE_Q(256, false);
        } else {
            if (full) G4_PV_DECODE_PC(512);
            else G4_PV_DECODE_Q(512, false);
        }
#undef G4_PV_DECODE_PC
#undef G4_PV_DECODE_Q
#undef G4_PV_DECODE
        if (q8 && !fuse) launch_quantize(s, q8, qs, out, n * heads * head_dim / 64);
        return G4_OK;
    } else {  // prefill: 4 tokens x 8 heads per block share each V tile; one
              // tile of prefetch (two or three measured no faster)
        dim3 grid(slices, (nn + 3) / 4);
        // with q8 the kernel writes the quantized rows (and no fp32 ones)
        if (head_dim == 256)
            hipLaunchKernelGGL((k_attn_values<256, 4, 1>), grid, dim3(256), 0, s, out, scores,
                               value_cache, cache_len, full, start_pos, (int)n, pos_dev, stride, q8, qs);
        else
            hipLaunchKernelGGL((k_attn_values<512, 4, 1>), grid, dim3(256), 0, s, out, scores,
                               value_cache, cache_len, full, start_pos, (int)n, pos_dev, stride, q8, qs);
        return G4_OK;
    }
}

int launch_attend(hipStream_t s, float *out, const float *q, const float *key_cache,
                  const float *value_cache, int cache_len, int head_dim, int heads, int full,
                  int start_pos, const int *pos_dev, size_t n, int8_t *q8, float *qs,
                  const FixedScratch *fixed) {
    if (g_order == G4_ORDER_REFERENCE)
        return launch_attend_reference(s, out, q, key_cache, value_cache, cache_len, head_dim,
                                       heads, full, start_pos, pos_dev, n, q8, qs, fixed);
    if (pos_dev) return set_error(G4_ERR_ARG, "device-side positions need reference order");
    const int rc = launch_attend_parallel(s, out, q, key_cache, value_cache, cache_len, head_dim,
                                          heads, full, start_pos, n, fixed);
    if (!rc && q8) launch_quantize(s, q8, qs, out, n * heads * head_dim / 64);
    return rc;
}

// ---------------------------------------------------------------------------
// Sampling (gemma4.c:527-561) on the device.
//
// The reference keeps the 64 highest logits in a list sorted by score: a
// later equal score goes after an earlier one, and a score equal to the 64th
// does not enter.  That list is the first 64 of the order (score descending,
// index ascending) over the logits above -inf.  Each logit becomes a 64-bit
// key that sorts that way: its bits made monotone in the high word (-0 taken
// as +0, which the reference's comparisons treat as equal), the complemented
// index in the low word; -inf and NaN get key 0 and never lead.  Blocks keep
// the 64 largest keys of every 1024 (a bitonic sort in LDS), twice, and one
// block sorts the last 1024 and runs the reference's arithmetic on the 64 in
// one lane, in its order (glibc's expf through expf_libm).  A NaN logit makes
// the list depend on where it falls, so then that lane runs the reference's
// own insertion loop over the whole row.

__device__ __forceinline__ uint64_t sample_key(float x, int index) {
    if (!(x > -INFINITY)) return 0;
    if (x == 0.0f) x = 0.0f;  // -0 -> +0
    const uint32_t b = __float_as_uint(x);
    const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return (uint64_t)o << 32 | (uint32_t)(0xFFFFFFFFu - (uint32_t)index);
}

// Bitonic sort of s[0 .. 1024) into descending order, by a block of 256
// threads (the caller has published s with a barrier).
__device__ void sort1024_descending(uint64_t *s) {
    for (int k = 2; k <= 1024; k <<= 1)
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < 1024; i += 256) {
                const int p = i ^ j;
                if (p > i) {
                    const uint64_t a = s[i], b = s[p];
                    if ((i & k) == 0 ? a < b : a > b) {
                        s[i] = b;
                        s[p] = a;
                    }
                }
            }
            __syncthreads();
        }
}

// Block b: the 64 largest keys of logits [1024 b, 1024 b + 1024) (LOGITS) or
// of keys [1024 b, ...) of a previous pass; flags[b] = a NaN logit was seen.
template <bool LOGITS>
__global__ __launch_bounds__(256) void k_sample_top(uint64_t *__restrict__ top,
                                                    int *__restrict__ flags,
                                                    const void *__restrict__ in, int n) {
    __shared__ uint64_t s[1024];
    const int base = blockIdx.x * 1024;
    bool nan = false;
    for (int i = threadIdx.x; i < 1024; i += 256) {
        const int g = base + i;
        if (LOGITS) {
            const float v = g < n ? static_cast<const float *>(in)[g] : -INFINITY;
            nan |= v != v;
            s[i] = sample_key(v, g);
        } else {
            s[i] = g < n ? static_cast<const uint64_t *>(in)[g] : 0;
        }
    }
    nan = __syncthreads_or(nan);
    sort1024_descending(s);
    if (threadIdx.x < 64) top[blockIdx.x * 64 + threadIdx.x] = s[threadIdx.x];
    if (LOGITS && threadIdx.x == 0) flags[blockIdx.x] = nan;
}

// The last 1024 candidates (n of them), then sample() on lane 0:
// result[0] = the token, result[1] = the advanced generator state.
__global__ __launch_bounds__(256) void k_sample_draw(uint64_t *__restrict__ result,
                                                     const uint64_t *__restrict__ keys, int n,
                                                     const int *__restrict__ flags, int flag_count,
                                                     const float *__restrict__ logits, int vocab,
                                                     float temperature, uint64_t state) {
    __shared__ uint64_t s[1024];
    for (int i = threadIdx.x; i < 1024; i += 256) s[i] = i < n ? keys[i] : 0;
    __syncthreads();
    sort1024_descending(s);
    if (threadIdx.x != 0) return;
    bool nan = false;
    for (int i = 0; i < flag_count; i++) nan |= flags[i] != 0;
    float score[64];
    int token[64];
    if (!nan) {
        for (int i = 0; i < 64; i++) {
            const uint32_t o = (uint32_t)(s[i] >> 32);
            score[i] = s[i] ? __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o) : -INFINITY;
            token[i] = s[i] ? (int)(0xFFFFFFFFu - (uint32_t)s[i]) : 0;
        }
    } else {  // gemma4.c:546-550 as written
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
    }
    // gemma4.c:552-560
    const float max = score[0] / temperature;
    float sum = 0.0f;
    for (int i = 0; i < 64; i++) {
        score[i] = expf_libm(score[i] / temperature - max);
        sum += score[i];
    }
    float mass = 0.0f;
    int count = 0;
    while (count < 64 && mass < 0.95f * sum) mass += score[count++];
    // gemma4.c:529-533: xorshift64*
    state ^= state >> 12;
    state ^= state << 25;
    state ^= state >> 27;
    float threshold = (float)((state * 0x2545F4914F6CDD1DULL) >> 40) / 16777216.0f * mass;
    int chosen = token[count > 0 ? count - 1 : 0];
    for (int i = 0; i < count; i++)
        if ((threshold -= score[i]) <= 0.0f) {
            chosen = token[i];
            break;
        }
    result[0] = (uint64_t)(uint32_t)chosen;
    result[1] = state;
}

// sample() over `vocab` device logits; *result (device, in the scratch
// buffer): [0] the token, [1] the advanced generator state (temperature > 0).
int launch_sample(hipStream_t s, const float *logits, int vocab, float temperature, uint64_t state,
                  uint64_t **result) {
    if (vocab < 64 || vocab > G4_VOCAB)
        return set_error(G4_ERR_ARG, "sample: vocabulary %d not in [64, %d]", vocab, G4_VOCAB);
    const int blocks1 = (vocab + 1023) / 1024, n1 = blocks1 * 64;
    const int blocks2 = (n1 + 1023) / 1024, n2 = blocks2 * 64;  // <= 1024
    const size_t flag_words = ((size_t)blocks1 + 1) / 2;        // ints, in 8-byte words
    const size_t need = ((size_t)n1 + n2 + flag_words + 2) * sizeof(uint64_t);
    int rc = scratch_reserve(need, 0);
    if (rc) return rc;
    uint64_t *top1 = reinterpret_cast<uint64_t *>(scratch().dots), *top2 = top1 + n1;
    int *flags = reinterpret_cast<int *>(top2 + n2);
    uint64_t *out = top2 + n2 + flag_words;
    *result = out;
    if (temperature <= 0.0f) {  // gemma4.c:537-541: the first maximum
        launch_argmax(s, reinterpret_cast<int *>(out), logits, 1, (size_t)vocab);
    } else {
        hipLaunchKernelGGL(k_sample_top<true>, dim3((unsigned)blocks1), dim3(256), 0, s, top1, flags,
                           static_cast<const void *>(logits), vocab);
        hipLaunchKernelGGL(k_sample_top<false>, dim3((unsigned)blocks2), dim3(256), 0, s, top2,
                           static_cast<int *>(nullptr), static_cast<const void *>(top1), n1);
        hipLaunchKernelGGL(k_sample_draw, dim3(1), dim3(256), 0, s, out, top2, n2, flags, blocks1,
                           logits, vocab, temperature, state);
    }
    G4_HIP(hipGetLastError());
    return G4_OK;
}

// Copies a launch_sample result back (synchronizing the stream): the token,
// and the generator state when temperature > 0.
int finish_sample(hipStream_t s, const uint64_t *result, float temperature, uint64_t *rng_state,
                  int *out_token) {
    uint64_t host[2] = {0, 0};
    G4_HIP(hipMemcpyAsync(host, result, sizeof(host), hipMemcpyDeviceToHost, s));
    G4_HIP(hipStreamSynchronize(s));
    *out_token = (int)(uint32_t)host[0];
    if (temperature > 0.0f) *rng_state = host[1];
    return G4_OK;
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
    if (count > 1024 && rows <= 64) {  // few long rows: a block per row
        const g4::SoftmaxRows spec{1, 1, 0, count, nullptr, 0};
        g4::launch_softmax_block((hipStream_t)stream, values, (size_t)count, count, spec,
                                 (unsigned)rows);
    } else {
        hipLaunchKernelGGL(g4::k_softmax_rows, dim3((unsigned)rows), dim3(64), 0, (hipStream_t)stream,
                           values, count, (size_t)count);
    }
    G4_HIP(hipGetLastError());
    return G4_OK;
}

extern "C" int g4_sample_logits(void *stream, const float *logits, int vocab, float temperature,
                                uint64_t *rng_state, int *out_token) {
    G4_CHECK(logits && rng_state && out_token, "g4_sample_logits: null argument");
    uint64_t *result = nullptr;
    const int rc = g4::launch_sample((hipStream_t)stream, logits, vocab, temperature, *rng_state, &result);
    if (rc) return rc;
    return g4::finish_sample((hipStream_t)stream, result, temperature, rng_state, out_token);
}
