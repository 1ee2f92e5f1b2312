// g4_attention_layer (include/g4.h): one layer's attention() (gemma4.c:411-461)
// as a per-op entry point, on device buffers the caller owns, so that the whole
// layer -- projections, norms, RoPE, the cache write, attention and the output
// projection -- is checked alone against the reference's attention().  The
// model step runs the same launchers in the same order (g4_model.hip).

#include "g4_internal.h"

namespace g4 {
namespace {

// Intermediate rows of the per-op layer, grown on demand: the query heads,
// the new key/value rows before their norms, the attention output (fp32,
// where the kernels write one) and the quantized activations.
struct LayerBuffers {
    float *aux = nullptr, *att = nullptr, *k_new = nullptr, *v_new = nullptr, *qs = nullptr;
    int8_t *q8 = nullptr;
    size_t rows = 0;
};
LayerBuffers g_lb;

constexpr int kMaxQueryWidth = 8 * 512;  // heads x head_dim

void free_buffers(LayerBuffers &b) {
    (void)hipFree(b.aux);
    (void)hipFree(b.att);
    (void)hipFree(b.k_new);
    (void)hipFree(b.v_new);
    (void)hipFree(b.qs);
    (void)hipFree(b.q8);
    b = LayerBuffers{};
}

int reserve_buffers(size_t rows) {
    LayerBuffers &b = g_lb;
    if (rows <= b.rows) return G4_OK;
    if (b.rows) {
        G4_HIP(hipDeviceSynchronize());  // earlier calls may still read the old buffers
        free_buffers(b);
    }
    const size_t wide = rows * kMaxQueryWidth;
    hipError_t e = hipMalloc(&b.aux, wide * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&b.att, wide * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&b.k_new, rows * 512 * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&b.v_new, rows * 512 * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&b.q8, wide);
    if (e == hipSuccess) e = hipMalloc(&b.qs, wide / 64 * sizeof(float));
    if (e != hipSuccess) {
        free_buffers(b);  // whatever did get allocated
        return set_error(G4_ERR_DEVICE, "g4_attention_layer: hipMalloc: %s", hipGetErrorString(e));
    }
    b.rows = rows;
    return G4_OK;
}

bool packed(const g4_tensor &t, int n, int k) {
    return t.data && t.scales && t.shape[0] == n && t.shape[1] == k &&
           ((uintptr_t)t.data & 15) == 0;
}

}  // namespace

void layer_buffers_release() {
    if (!g_lb.rows) return;  // nothing allocated (no HIP call)
    (void)hipDeviceSynchronize();
    free_buffers(g_lb);
}

}  // namespace g4

using namespace g4;

extern "C" int g4_attention_layer(void *stream, float *hidden, size_t n, int start_pos,
                                  const g4_tensor *layer, float *cache, int cache_len,
                                  int full_attention) {
    G4_CHECK(hidden && layer && cache, "g4_attention_layer: null pointer");
    G4_CHECK(n >= 1 && n <= G4_BATCH, "g4_attention_layer: %zu rows (1..%d)", n, G4_BATCH);
    G4_CHECK(((uintptr_t)hidden & 15) == 0, "g4_attention_layer: hidden must be 16-byte aligned");
    // the layer's records in LayerWeights order (gemma4.c:125-155)
    const g4_tensor &q_norm = layer[8], &k_norm = layer[9], &q = layer[10], &k = layer[11],
                    &v = layer[12], &o = layer[13], &cosines = layer[17], &sines = layer[18];
    const int hd = q_norm.shape[0], qw = q.shape[0];
    G4_CHECK(q_norm.data && (hd == 256 || hd == 512), "g4_attention_layer: head_dim %d (q_norm) is not 256 or 512", hd);
    G4_CHECK(qw == 8 * hd, "g4_attention_layer: q_proj has %d rows, not 8 heads of %d", qw, hd);
    G4_CHECK(packed(q, qw, G4_HIDDEN) && packed(o, G4_HIDDEN, qw),
             "g4_attention_layer: q_proj / o_proj missing, misshapen or unaligned");
    const bool writes = k.data != nullptr;  // shared layers read an earlier layer's cache
    if (writes)
        G4_CHECK(packed(k, hd, G4_HIDDEN) && packed(v, hd, G4_HIDDEN) && k_norm.data && k_norm.shape[0] == hd,
                 "g4_attention_layer: k_proj / v_proj / k_norm missing or misshapen");
    const int pairs = cosines.shape[1];
    G4_CHECK(cosines.data && sines.data && pairs > 0 && pairs <= hd / 2 && sines.shape[1] == pairs &&
                 cosines.shape[0] >= start_pos + (long)n && sines.shape[0] >= start_pos + (long)n,
             "g4_attention_layer: RoPE tables do not cover positions %d..%ld", start_pos,
             start_pos + (long)n - 1);
    float *keys = cache, *values = cache + (size_t)cache_len * hd;
    int rc = check_attend_args("g4_attention_layer", hidden, hidden, keys, values, cache_len, hd, 8,
                               full_attention, start_pos, n);
    if (rc) return rc;
    G4_TRY(reserve_buffers(n));

    const hipStream_t s = (hipStream_t)stream;
    const LayerBuffers &b = g_lb;
    const float *qn = (const float *)q_norm.data, *kn = (const float *)k_norm.data;
    const float *cs = (const float *)cosines.data, *sn = (const float *)sines.data;
    // gemma4.c:425-426, 435-436: the queries, and the new keys and values
    launch_quantize(s, b.q8, b.qs, hidden, n * (G4_HIDDEN / 64));
    if (writes && n > 8) {  // one launch for the three products of the same rows
        const int8_t *w[3] = {(const int8_t *)q.data, (const int8_t *)k.data, (const int8_t *)v.data};
        const uint16_t *ws[3] = {q.scales, k.scales, v.scales};
        float *out[3] = {b.aux, b.k_new, b.v_new};
        const size_t strides[3] = {(size_t)qw, (size_t)hd, (size_t)hd};
        const int ns[3] = {qw, hd, hd};
        G4_TRY(launch_matmul_group(s, b.q8, b.qs, (int)n, G4_HIDDEN, 3, w, ws, out, strides, ns));
    } else {
        G4_TRY(launch_matmul(s, b.aux, qw, b.q8, b.qs, (const int8_t *)q.data, q.scales, qw, G4_HIDDEN, (int)n));
        if (writes) {
            G4_TRY(launch_matmul(s, b.k_new, hd, b.q8, b.qs, (const int8_t *)k.data, k.scales, hd, G4_HIDDEN, (int)n));
            G4_TRY(launch_matmul(s, b.v_new, hd, b.q8, b.qs, (const int8_t *)v.data, v.scales, hd, G4_HIDDEN, (int)n));
        }
    }
    // gemma4.c:427-428, 437-440: norms and RoPE, the new rows into the ring
    if (order() == G4_ORDER_REFERENCE) {
        launch_qkv_finish(s, b.aux, 8, qn, writes ? b.k_new : nullptr, b.v_new, kn, keys, values, cs, sn,
                          pairs, hd, cache_len, start_pos, nullptr, n);
    } else {
        launch_rmsnorm(s, b.aux, b.aux, qn, hd, 1e-6f, n * 8);
        launch_rope(s, cs, sn, pairs, b.aux, 8, hd, start_pos, nullptr, n);
        if (writes)
            launch_kv_finish(s, keys, values, b.k_new, b.v_new, kn, cs, sn, pairs, hd, cache_len,
                             start_pos, nullptr, n);
    }
    // gemma4.c:443-456, 459-460: attention, quantized for the output projection
    G4_TRY(launch_attend(s, b.att, b.aux, keys, values, cache_len, hd, 8, full_attention, start_pos,
                         nullptr, n, b.q8, b.qs));
    G4_TRY(launch_matmul(s, hidden, G4_HIDDEN, b.q8, b.qs, (const int8_t *)o.data, o.scales, G4_HIDDEN,
                         qw, (int)n));
    G4_HIP(hipGetLastError());
    return G4_OK;
}
