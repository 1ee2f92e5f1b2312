// The exact-sum engine (esum_pass in gemma4.c_amd/csrc/g4_reference_order.hip)
// against the plain sequential fp32 loop it replaces -- the rmsnorm sum of
// squares (gemma4.c:366-368) and the softmax running sum with its new-maximum
// step s = s t + 1 (gemma4.c:400-408) -- in every block shape the kernels use
// (waves x terms a thread), one row of 64 NW J terms a block, bit for bit.
//
// Test infrastructure: built by build() into tests/_bin/, run by
// tests/test_gpu_exact_sum.py.  It includes the engine's source file, so it
// runs the library's code as compiled with the library's flags.
//
// Rows, by family (row index mod 8): random magnitudes over several spreads;
// sums that pass a power of two a few ulps a term, with terms that the
// prediction leads, wanders around or lags (three families); tiny terms on a
// sum near 1 or 0; a new maximum at every step (or rising squares); exact
// ties; zeros, subnormal and huge terms.  The pass loop is bounded (a correct
// engine needs at most one pass per term plus one), so a lost pass ends as a
// reported failure, not a hang.  Exit status 0 when every row matches.
#include "g4_reference_order.hip"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

namespace g4 {
constexpr int kFuzzPassBound = 20000;

template <int NW, int J, bool SP>
__global__ __launch_bounds__(64 * NW) void k_esum_fuzz(const float *terms, const uint8_t *spec, const float *s0,
                                                       float *out, int *passes) {
    __shared__ EsumShared sh;
    constexpr int N = 64 * NW * J;
    const int row = blockIdx.x, T = threadIdx.x;
    float t[J];
    uint32_t sp = 0;
#pragma unroll
    for (int j = 0; j < J; j++) {
        t[j] = terms[(size_t)row * N + J * T + j];
        if (SP) sp |= (uint32_t)(spec[(size_t)row * N + J * T + j] & 1) << j;
    }
    float s = s0[row];
    int k0 = 0, n = 0;
    while (n < kFuzzPassBound && !esum_pass<NW, J, SP>(t, sp, s, k0, sh)) n++;
    if (T == 0) {
        out[row] = s;
        passes[row] = n + 1;
    }
}
}  // namespace g4

using namespace g4;

// The reference's loop: s + t, or at a new maximum s t + 1 with two roundings.
static float sequential(const float *t, const uint8_t *sp, int n, float s) {
    for (int k = 0; k < n; k++) {
        if (sp[k]) {
            volatile float p = s * t[k];
            s = p + 1.0f;
        } else {
            s = s + t[k];
        }
    }
    return s;
}

static std::mt19937 gen(2026);
static float uni(float a, float b) { return std::uniform_real_distribution<float>(a, b)(gen); }
static double normal() { return std::normal_distribution<double>(0, 1)(gen); }

// One row of n terms of family f % 8 (softmax mode: sum from 1); returns the start.
static float make_row(int f, bool softmax, int n, float *t, uint8_t *sp) {
    std::fill(sp, sp + n, 0);
    float s = softmax ? 1.0f : 0.0f;
    const int fam = f % 8;
    if (fam == 0) {  // random magnitudes
        const double spread[3] = {1, 5, 20};
        const double sig = spread[f / 8 % 3];
        for (int k = 0; k < n; k++) t[k] = (float)std::exp(normal() * sig - (softmax ? 3 : 0));
    } else if (fam <= 3) {  // a sum passing a power of two B a few ulps a term
        const float bounds[4] = {2.f, 4.f, 1024.f, 0.0009765625f};
        const float B = bounds[f / 8 % 4];
        if (softmax && B < 2) return make_row(f + 8, softmax, n, t, sp);
        // terms of r ulps (u: the ulp just below B), each rounding to R ulps
        // there and to another count above B
        const float lo = fam == 1 ? 2.05f : fam == 2 ? 1.55f : 0.55f;
        const float hi = fam == 3 ? 0.95f : 2.45f;
        const int R = (int)std::lround((lo + hi) / 2);
        const double u = B * std::ldexp(1.0, -24);
        const int cross = (int)uni(n * 0.1f, n * 0.9f);
        for (int k = 0; k < n; k++) t[k] = (float)(uni(lo, hi) * u);
        t[0] = (float)(B - R * (double)(cross - 1) * u - s);
        if (softmax)  // a few new maxima that barely move the sum
            for (int e = 0; e < 3; e++) {
                const int k = (int)uni(1, n - 1);
                sp[k] = 1;
                t[k] = uni(0.999f, 1.0f);
            }
    } else if (fam == 4) {  // tiny terms: a peaked softmax row near 1, or tiny squares
        for (int k = 0; k < n; k++) t[k] = (float)std::exp(normal() * 3 - 14);
        if (softmax)
            for (int e = 0; e < 5; e++) {
                const int k = (int)uni(1, n - 1);
                sp[k] = 1;
                t[k] = uni(0.0f, 1e-3f);
            }
    } else if (fam == 5) {  // a new maximum at every step (or rising squares)
        for (int k = 0; k < n; k++) {
            t[k] = softmax ? uni(0.3f, 1.0f) : (float)(k + 1) * 1e-3f;
            sp[k] = softmax;
        }
    } else if (fam == 6) {  // exact ties: odd multiples of half an ulp
        if (!softmax) s = (float)std::ldexp(1.0, 20);  // ulp 2^-3
        for (int k = 0; k < n; k++) t[k] = (float)((int)uni(0, 8) * (softmax ? std::ldexp(1.0, -24) : 0.0625));
    } else {  // zeros, subnormals, huge terms
        for (int k = 0; k < n; k++) {
            const float r = uni(0, 1);
            t[k] = r < 0.3f ? 0.0f : r < 0.5f ? 1e-40f * uni(1, 100) : r < 0.55f ? uni(1e30f, 1e32f) : uni(0, 2);
        }
        if (softmax)
            for (int e = 0; e < 4; e++) {
                const int k = (int)uni(1, n - 1);
                sp[k] = 1;
                t[k] = uni(0, 1);
            }
    }
    return s;
}

#define CHECK_HIP(x)                                                                   \
    do {                                                                               \
        if ((x) != hipSuccess) {                                                       \
            fprintf(stderr, "HIP error %s at %s:%d\n", hipGetErrorString(x), __FILE__, __LINE__); \
            exit(2);                                                                   \
        }                                                                              \
    } while (0)

template <int NW, int J, bool SP>
static int run(int rows) {
    constexpr int N = 64 * NW * J;
    std::vector<float> t((size_t)rows * N), s0(rows), out(rows), ref(rows);
    std::vector<uint8_t> sp((size_t)rows * N);
    std::vector<int> passes(rows);
    for (int r = 0; r < rows; r++) {
        s0[r] = make_row(r, SP, N, &t[(size_t)r * N], &sp[(size_t)r * N]);
        ref[r] = sequential(&t[(size_t)r * N], &sp[(size_t)r * N], N, s0[r]);
    }
    float *dt, *ds, *dout;
    uint8_t *dsp;
    int *dp;
    CHECK_HIP(hipMalloc(&dt, t.size() * 4));
    CHECK_HIP(hipMalloc(&dsp, sp.size()));
    CHECK_HIP(hipMalloc(&ds, rows * 4));
    CHECK_HIP(hipMalloc(&dout, rows * 4));
    CHECK_HIP(hipMalloc(&dp, rows * 4));
    CHECK_HIP(hipMemcpy(dt, t.data(), t.size() * 4, hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(dsp, sp.data(), sp.size(), hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(ds, s0.data(), rows * 4, hipMemcpyHostToDevice));
    hipLaunchKernelGGL((k_esum_fuzz<NW, J, SP>), dim3(rows), dim3(64 * NW), 0, 0, dt, dsp, ds, dout, dp);
    CHECK_HIP(hipGetLastError());
    CHECK_HIP(hipDeviceSynchronize());
    CHECK_HIP(hipMemcpy(out.data(), dout, rows * 4, hipMemcpyDeviceToHost));
    CHECK_HIP(hipMemcpy(passes.data(), dp, rows * 4, hipMemcpyDeviceToHost));
    int bad = 0, bound = 0, most = 0;
    for (int r = 0; r < rows; r++) {
        const bool same = memcmp(&out[r], &ref[r], 4) == 0 || (std::isnan(out[r]) && std::isnan(ref[r]));
        if (!same && bad < 3)
            printf("    row %d (family %d): engine %.9g, sequential %.9g, %d passes\n", r, r % 8, out[r], ref[r],
                   passes[r]);
        bad += !same;
        bound += passes[r] > kFuzzPassBound;
        most = passes[r] > most ? passes[r] : most;
    }
    printf("esum %2d waves x %2d terms, %s: %d rows, %d differ, %d at the pass bound, at most %d passes\n", NW, J,
           SP ? "softmax" : "plain  ", rows, bad, bound, most);
    fflush(stdout);
    CHECK_HIP(hipFree(dt));
    CHECK_HIP(hipFree(dsp));
    CHECK_HIP(hipFree(ds));
    CHECK_HIP(hipFree(dout));
    CHECK_HIP(hipFree(dp));
    return bad + bound;
}

int main() {
    const int R = 2400;
    int bad = 0;
    bad += run<1, 1, false>(R);  // q/k norms (one wave a row), decode softmax rows
    bad += run<1, 1, true>(R);
    bad += run<1, 4, false>(R);
    bad += run<1, 4, true>(R);
    bad += run<1, 8, false>(R);
    bad += run<1, 8, true>(R);
    bad += run<2, 12, false>(R);
    bad += run<3, 8, false>(R);
    bad += run<4, 2, true>(R);   // the split softmax's 512-term chunks
    bad += run<4, 6, false>(R);  // row tails
    bad += run<4, 8, false>(R);
    bad += run<4, 8, true>(R);   // prefill softmax, long rows
    bad += run<6, 4, false>(R);  // one-token products' row tails
    bad += run<8, 1, false>(R);
    bad += run<8, 1, true>(R);   // window softmax in decode
    bad += run<8, 3, false>(R);  // the gate.up row tail
    bad += run<12, 2, false>(R);
    bad += run<16, 4, true>(R);  // per-op softmax rows
    bad += run<16, 8, false>(R / 2);
    bad += run<16, 8, true>(R / 2);  // long decode rows
    printf("%s\n", bad ? "MISMATCH" : "all rows equal");
    return bad ? 1 : 0;
}
