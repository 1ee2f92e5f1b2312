// g4_model.hip -- the device-resident model context behind g4_init /
// g4_forward / g4_logits (include/g4.h).
//
// Weights are uploaded once into one HBM arena in the exporter's packed layout
// (the same bytes as the .bin); the fp32 KV rings (3 global owners x 512
// channels, growing from 4096 to at most 131072 positions with the context;
// 12 sliding owners x 4096 x 256; keys then values) and every activation live
// on the device, so a token step moves only token ids in and one logits row
// (or one sampled token) out.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <condition_variable>
#include <map>
#include <mutex>
#include <system_error>
#include <thread>
#include <vector>

#include "g4_internal.h"

namespace g4 {

static char g_error[512] = "no error";

int set_error(int status, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
    return status;
}

struct Weight {
    const int8_t *data = nullptr;
    const uint16_t *scales = nullptr;
    int n = 0, k = 0;
};

struct Layer {
    const float *input_ln, *post_attn_ln, *pre_ffn_ln, *post_ffn_ln, *post_ple_ln, *q_norm, *k_norm;
    Weight q, k, v, o, gate, up, down, ple_gate, ple_proj;
    const float *rope_cos, *rope_sin;
    int pairs, head_dim, query_width, full, owner, ffn;
    float layer_scalar;
};

// Many-token passes in flight at once (struct Lane).
constexpr int kLanes = 4;

// The activation buffers of a lane beyond the first.
struct LaneBuffers {
    hipStream_t stream = nullptr;
    float *residual = nullptr, *hidden = nullptr, *aux = nullptr, *ple = nullptr;
    float *k_new = nullptr, *v_new = nullptr, *qs = nullptr, *qsb = nullptr;
    int8_t *q8 = nullptr, *q8b = nullptr;
    int *tokens_dev = nullptr, *tokens_pinned = nullptr;
};

struct Context {
    bool ready = false;
    int device = 0;
    hipStream_t stream = nullptr;
    // Lanes 1 .. kLanes - 1 (struct Lane): the streams and activation buffers
    // of the passes that run beside lane 0's; kv_written[lane][l] is recorded
    // once a lane's pass has written layer l's key/value rows.
    LaneBuffers extra[kLanes - 1];
    hipEvent_t kv_written[kLanes][15] = {};
    void *lane_attn[kLanes] = {};  // each lane's attention scratch
    size_t lane_attn_bytes[kLanes] = {};
    int pending = -1;    // the lane whose last pass may still run (-1: none)
    int next_pos = 0;    // the position after that pass
    int last_lane = 0;   // the lane holding the last pass's residual rows
    char *arena = nullptr;
    Layer layers[G4_LAYERS];
    Weight embed, embed_ple, ple_model_proj;
    const float *final_norm = nullptr, *ple_norm = nullptr, *gelu = nullptr;
    int gelu_size = 0;
    float gelu_lower = 0, gelu_upper = 0;
    float *residual = nullptr, *hidden = nullptr, *aux = nullptr, *ple = nullptr;
    float *residual_alt = nullptr;  // one token: the row tails alternate residual rows
    float *k_new = nullptr, *v_new = nullptr, *logits = nullptr, *logits_all = nullptr;
    int8_t *q8 = nullptr, *q8b = nullptr;  // quantized activations; q8b: written by a
    float *qs = nullptr, *qsb = nullptr;   // product that reads q8 (the GELU epilogues)
    float *cache[15] = {};
    int cache_len[15] = {}, cache_dim[15] = {};
    int *tokens_dev = nullptr, *argmax_dev = nullptr;
    int *tokens_pinned = nullptr;
    int *pos_dev = nullptr, *pos_pinned = nullptr;
    float *logits_pinned = nullptr;  // one logits row: the copy out is a direct DMA
    // many rows (g4_logits_all): pieces through two pinned buffers, the DMA of
    // one overlapping the host copy (several threads) of the other
    char *pieces_pinned[2] = {};
    hipEvent_t piece_done[2] = {};
    int last_n = 0;
    // One-token steps replay a captured graph of the whole forward pass; the
    // position is read from pos_dev.  Recaptured when the scratch buffers move
    // or the summation order changes.
    hipGraphExec_t decode_graph = nullptr;
    unsigned graph_generation = 0;
    int graph_order = -1;
    // The global layers' rings grow with the context (ensure_kv): a move bumps
    // kv_generation, and the captured graph (which holds the old pointers and
    // lengths) is captured again.
    unsigned kv_generation = 0, graph_kv_generation = 0;
};

static Context g_ctx;

// Bytes of one piece of a many-row logits copy (g4_logits_all), and the host
// threads that copy a piece out of its pinned buffer.
constexpr size_t kCopyPiece = (size_t)32 << 20;
constexpr int kCopyThreads = 8;

// memcpy split over kCopyThreads threads (one copy alone runs at ~20 GB/s).
// kCopyThreads - 1 workers live from the first copy until g4_shutdown (or
// process exit): starting threads for every 32 MiB piece cost more than the
// copy's own time.  Each copy is a numbered job: a worker takes its part of
// every job after the one it last saw (a worker starts knowing the number
// before its first job), the caller takes part 0 and the parts of workers
// that could not start, then waits until every worker's part is done.
class CopyPool {
  public:
    ~CopyPool() { stop(); }
    void copy(char *dst, const char *src, size_t bytes) {
        std::unique_lock<std::mutex> lock(m_);
        if (!started_) start_locked();
        dst_ = dst;
        src_ = src;
        bytes_ = bytes;
        part_ = ((bytes + kCopyThreads - 1) / kCopyThreads + 4095) & ~(size_t)4095;  // > 0 for any bytes > 0
        pending_ = running_;
        ++job_;
        lock.unlock();
        work_.notify_all();
        for (int t = 1 + running_; t < kCopyThreads; t++) take(t);
        take(0);
        lock.lock();
        done_.wait(lock, [&] { return pending_ == 0; });
    }
    void stop() {
        {
            std::lock_guard<std::mutex> guard(m_);
            stopping_ = true;
        }
        work_.notify_all();
        for (std::thread &t : threads_)
            if (t.joinable()) t.join();
        threads_.clear();
        started_ = stopping_ = false;
        running_ = 0;
    }

  private:
    void take(int t) {
        const size_t lo = t * part_ < bytes_ ? t * part_ : bytes_;
        const size_t hi = lo + part_ < bytes_ ? lo + part_ : bytes_;
        if (lo < hi) memcpy(dst_ + lo, src_ + lo, hi - lo);
    }
    void start_locked() {  // m_ held
        started_ = true;
        for (int t = 1; t < kCopyThreads; t++) {
            try {
                threads_.emplace_back([this, t, seen = job_] { work(t, seen); });
            } catch (const std::system_error &) {
                break;  // the caller takes this part and the ones after it
            }
            running_++;
        }
    }
    void work(int t, unsigned seen) {
        std::unique_lock<std::mutex> lock(m_);
        for (;;) {
            work_.wait(lock, [&] { return stopping_ || job_ != seen; });
            if (stopping_) return;
            seen = job_;
            lock.unlock();
            take(t);
            lock.lock();
            if (--pending_ == 0) done_.notify_one();
        }
    }
    std::mutex m_;
    std::condition_variable work_, done_;
    std::vector<std::thread> threads_;
    char *dst_ = nullptr;
    const char *src_ = nullptr;
    size_t bytes_ = 0, part_ = 0;
    unsigned job_ = 0;
    int pending_ = 0, running_ = 0;
    bool started_ = false, stopping_ = false;
};
static CopyPool g_copy_pool;

static void copy_parallel(char *dst, const char *src, size_t bytes) { g_copy_pool.copy(dst, src, bytes); }

// Initial positions of a global-attention ring (a power of two).
constexpr int kGlobalStart = 4096;
// Positions of a sliding-window ring: a pass of G4_BATCH tokens reads the
// G4_WINDOW - 1 positions before it, and the kLanes - 1 passes after it may
// write their own G4_BATCH positions meanwhile (they run concurrently, struct
// Lane), so kLanes * G4_BATCH + G4_WINDOW - 1 positions must not share a slot
// (rounded up to a power of two for the ring mask).
constexpr int kWindowRing = 4096;
static_assert(kWindowRing >= kLanes * G4_BATCH + G4_WINDOW - 1 && (kWindowRing & (kWindowRing - 1)) == 0,
              "sliding ring too short for the passes in flight");

static size_t record_bytes(const g4_tensor &t, int index, size_t *scale_bytes) {
    *scale_bytes = 0;
    if (!t.data) return 0;
    if (t.scales) {
        const size_t count = (size_t)t.shape[0] * (size_t)t.shape[1];
        *scale_bytes = count / 64 * 2;
        return count;
    }
    if (index == G4_RECORDS - 1) return (size_t)t.shape[0] * 4;  // GELU table (4096, lo, hi)
    return (size_t)t.shape[0] * (size_t)(t.shape[1] > 0 ? t.shape[1] : 1) * 4;
}

static size_t round256(size_t v) { return (v + 255) & ~(size_t)255; }

static void release(void *p) {
    if (p) (void)hipFree(p);
}

static void free_all(Context &c) {
    g_copy_pool.stop();
    for (LaneBuffers &b : c.extra)
        if (b.stream) (void)hipStreamSynchronize(b.stream);
    if (c.stream) (void)hipStreamSynchronize(c.stream);
    for (void *p : c.lane_attn) release(p);
    release(c.arena);
    release(c.residual);
    release(c.residual_alt);
    release(c.hidden);
    release(c.aux);
    release(c.ple);
    release(c.k_new);
    release(c.v_new);
    release(c.logits);
    release(c.logits_all);
    release(c.q8);
    release(c.qs);
    release(c.q8b);
    release(c.qsb);
    for (int i = 0; i < 15; i++) release(c.cache[i]);
    release(c.tokens_dev);
    release(c.argmax_dev);
    release(c.pos_dev);
    if (c.tokens_pinned) (void)hipHostFree(c.tokens_pinned);
    if (c.pos_pinned) (void)hipHostFree(c.pos_pinned);
    if (c.logits_pinned) (void)hipHostFree(c.logits_pinned);
    for (char *p : c.pieces_pinned)
        if (p) (void)hipHostFree(p);
    for (hipEvent_t e : c.piece_done)
        if (e) (void)hipEventDestroy(e);
    if (c.decode_graph) (void)hipGraphExecDestroy(c.decode_graph);
    for (auto &lane : c.kv_written)
        for (hipEvent_t e : lane)
            if (e) (void)hipEventDestroy(e);
    for (LaneBuffers &b : c.extra) {
        if (b.stream) (void)hipStreamDestroy(b.stream);
        for (float *p : {b.residual, b.hidden, b.aux, b.ple, b.k_new, b.v_new, b.qs, b.qsb}) release(p);
        release(b.q8);
        release(b.q8b);
        release(b.tokens_dev);
        if (b.tokens_pinned) (void)hipHostFree(b.tokens_pinned);
    }
    if (c.stream) (void)hipStreamDestroy(c.stream);
    scratch_release();  // the model's reservation (and anything per-op calls grew)
    layer_buffers_release();
    c = Context();
}

static int check_weight(const g4_tensor &t, int n, int k, const char *what, int layer) {
    if (!t.data || !t.scales || t.shape[0] != n || t.shape[1] != k)
        return set_error(G4_ERR_ARG, "g4_init: %s of layer %d must be an int8 [%d x %d] record (got %d x %d)",
                         what, layer, n, k, t.shape[0], t.shape[1]);
    return G4_OK;
}

static int check_vector(const g4_tensor &t, int n, const char *what, int layer) {
    if (!t.data || t.scales || t.shape[0] != n)
        return set_error(G4_ERR_ARG, "g4_init: %s of layer %d must be fp32 [%d]", what, layer, n);
    return G4_OK;
}

// Shape checks for everything the forward pass relies on (the reference trusts
// the image; gemma4.c:414-421, 464, 131-140 of exporter.py).
static int validate(const g4_tensor *r) {
    G4_TRY(check_weight(r[0], G4_VOCAB, G4_HIDDEN, "embed", -1));
    G4_TRY(check_weight(r[1], G4_VOCAB, G4_LAYERS * G4_PLE, "embed_per_layer", -1));
    G4_TRY(check_vector(r[667], G4_HIDDEN, "norm", -1));
    G4_TRY(check_weight(r[668], G4_LAYERS * G4_PLE, G4_HIDDEN, "per_layer_model_projection", -1));
    G4_TRY(check_vector(r[669], G4_PLE, "per_layer_projection_norm", -1));
    const g4_tensor &gelu = r[670];
    if (!gelu.data || gelu.scales || gelu.shape[0] < 2 || gelu.shape[2] <= gelu.shape[1])
        return set_error(G4_ERR_ARG, "g4_init: bad GELU table record");
    bool have_sliding_owner = false, have_full_owner = false;
    for (int l = 0; l < G4_LAYERS; l++) {
        const g4_tensor *f = r + 2 + l * 19;
        const int full = l % 5 == 4;
        const int hd = f[8].shape[0];
        if (hd != (full ? 512 : 256))
            return set_error(G4_ERR_ARG, "g4_init: q_norm of layer %d has width %d", l, hd);
        G4_TRY(check_vector(f[0], G4_HIDDEN, "input_layernorm", l));
        if (!f[1].data) return set_error(G4_ERR_ARG, "g4_init: layer %d has no layer_scalar", l);
        G4_TRY(check_vector(f[2], G4_HIDDEN, "pre_ffn_layernorm", l));
        G4_TRY(check_vector(f[3], G4_HIDDEN, "post_attn_layernorm", l));
        G4_TRY(check_vector(f[4], G4_HIDDEN, "post_ffn_layernorm", l));
        G4_TRY(check_vector(f[5], G4_HIDDEN, "post_per_layer_input_norm", l));
        G4_TRY(check_weight(f[6], G4_PLE, G4_HIDDEN, "per_layer_input_gate", l));
        G4_TRY(check_weight(f[7], G4_HIDDEN, G4_PLE, "per_layer_projection", l));
        G4_TRY(check_vector(f[8], hd, "q_norm", l));
        G4_TRY(check_weight(f[10], G4_HEADS * hd, G4_HIDDEN, "q_proj", l));
        if (f[11].data) {
            G4_TRY(check_vector(f[9], hd, "k_norm", l));
            G4_TRY(check_weight(f[11], hd, G4_HIDDEN, "k_proj", l));
            G4_TRY(check_weight(f[12], hd, G4_HIDDEN, "v_proj", l));
            if (l >= 15) return set_error(G4_ERR_ARG, "g4_init: layer %d owns K/V; only layers 0-14 may", l);
            (full ? have_full_owner : have_sliding_owner) = true;
        } else if (!(full ? have_full_owner : have_sliding_owner)) {
            return set_error(G4_ERR_ARG, "g4_init: layer %d has no earlier K/V owner of its type", l);
        }
        G4_TRY(check_weight(f[13], G4_HIDDEN, G4_HEADS * hd, "o_proj", l));
        const int ffn = f[14].shape[0];
        G4_TRY(check_weight(f[14], ffn, G4_HIDDEN, "gate_proj", l));
        G4_TRY(check_weight(f[15], ffn, G4_HIDDEN, "up_proj", l));
        G4_TRY(check_weight(f[16], G4_HIDDEN, ffn, "down_proj", l));
        if (ffn > 8 * G4_HIDDEN || ffn % 64)
            return set_error(G4_ERR_ARG, "g4_init: FFN width %d of layer %d unsupported", ffn, l);
        const int pairs = f[17].shape[1];
        if (!f[17].data || !f[18].data || f[17].shape[0] < G4_MAX_CONTEXT || pairs <= 0 || pairs > hd / 2 ||
            f[18].shape[1] != pairs)
            return set_error(G4_ERR_ARG, "g4_init: bad RoPE tables for layer %d", l);
    }
    return G4_OK;
}

static int init(const g4_tensor *records, int device) {
    Context &c = g_ctx;
    int count = 0;
    G4_HIP(hipGetDeviceCount(&count));
    G4_CHECK(device >= 0 && device < count, "g4_init: device %d not present (%d devices)", device, count);
    G4_TRY(validate(records));
    c.device = device;
    G4_HIP(hipSetDevice(device));
    G4_HIP(hipStreamCreateWithFlags(&c.stream, hipStreamNonBlocking));
    for (LaneBuffers &b : c.extra) G4_HIP(hipStreamCreateWithFlags(&b.stream, hipStreamNonBlocking));
    for (auto &lane : c.kv_written)
        for (hipEvent_t &e : lane) G4_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));

    // One arena for all weights; records that share host data (the RoPE
    // tables) share device data.
    std::map<const void *, size_t> offsets;
    size_t total = 0;
    for (int i = 0; i < G4_RECORDS; i++) {
        size_t sb = 0, db = record_bytes(records[i], i, &sb);
        if (!db || offsets.count(records[i].data)) continue;
        offsets[records[i].data] = total;
        total += round256(db);
        if (sb) {
            offsets[records[i].scales] = total;
            total += round256(sb);
        }
    }
    G4_HIP(hipMalloc(&c.arena, total));
    for (int i = 0; i < G4_RECORDS; i++) {
        size_t sb = 0, db = record_bytes(records[i], i, &sb);
        if (!db) continue;
        G4_HIP(hipMemcpy(c.arena + offsets[records[i].data], records[i].data, db, hipMemcpyHostToDevice));
        if (sb)
            G4_HIP(hipMemcpy(c.arena + offsets[records[i].scales], records[i].scales, sb,
                             hipMemcpyHostToDevice));
    }
    auto dev_f = [&](const g4_tensor &t) -> const float * {
        return t.data ? (const float *)(c.arena + offsets[t.data]) : nullptr;
    };
    auto dev_w = [&](const g4_tensor &t) {
        Weight w;
        if (!t.data) return w;
        w.data = (const int8_t *)(c.arena + offsets[t.data]);
        w.scales = (const uint16_t *)(c.arena + offsets[t.scales]);
        w.n = t.shape[0];
        w.k = t.shape[1];
        return w;
    };
    c.embed = dev_w(records[0]);
    c.embed_ple = dev_w(records[1]);
    c.final_norm = dev_f(records[667]);
    c.ple_model_proj = dev_w(records[668]);
    c.ple_norm = dev_f(records[669]);
    c.gelu = dev_f(records[670]);
    c.gelu_size = records[670].shape[0];
    c.gelu_lower = (float)records[670].shape[1];
    c.gelu_upper = (float)records[670].shape[2];
    for (int l = 0; l < G4_LAYERS; l++) {
        const g4_tensor *f = records + 2 + l * 19;
        Layer &L = c.layers[l];
        L.input_ln = dev_f(f[0]);
        L.layer_scalar = ((const float *)f[1].data)[0];
        L.pre_ffn_ln = dev_f(f[2]);
        L.post_attn_ln = dev_f(f[3]);
        L.post_ffn_ln = dev_f(f[4]);
        L.post_ple_ln = dev_f(f[5]);
        L.ple_gate = dev_w(f[6]);
        L.ple_proj = dev_w(f[7]);
        L.q_norm = dev_f(f[8]);
        L.k_norm = dev_f(f[9]);
        L.q = dev_w(f[10]);
        L.k = dev_w(f[11]);
        L.v = dev_w(f[12]);
        L.o = dev_w(f[13]);
        L.gate = dev_w(f[14]);
        L.up = dev_w(f[15]);
        L.down = dev_w(f[16]);
        L.rope_cos = dev_f(f[17]);
        L.rope_sin = dev_f(f[18]);
        L.pairs = f[17].shape[1];
        L.head_dim = f[8].shape[0];
        L.query_width = f[10].shape[0];
        L.full = l % 5 == 4;
        L.ffn = f[14].shape[0];
        int owner = l;  // gemma4.c:419-420
        while (!records[2 + owner * 19 + 11].data || (owner % 5 == 4) != L.full) owner--;
        L.owner = owner;
    }

    const size_t wide = (size_t)G4_BATCH * 8 * G4_HIDDEN;
    G4_HIP(hipMalloc(&c.residual, (size_t)G4_BATCH * G4_HIDDEN * sizeof(float)));
    G4_HIP(hipMalloc(&c.residual_alt, (size_t)G4_HIDDEN * sizeof(float)));
    G4_HIP(hipMalloc(&c.hidden, wide * sizeof(float)));
    G4_HIP(hipMalloc(&c.aux, wide * sizeof(float)));
    G4_HIP(hipMalloc(&c.ple, (size_t)G4_BATCH * G4_LAYERS * G4_PLE * sizeof(float)));
    G4_HIP(hipMalloc(&c.k_new, (size_t)G4_BATCH * 512 * sizeof(float)));
    G4_HIP(hipMalloc(&c.v_new, (size_t)G4_BATCH * 512 * sizeof(float)));
    G4_HIP(hipMalloc(&c.logits, (size_t)G4_VOCAB * sizeof(float)));
    G4_HIP(hipMalloc(&c.q8, wide));
    G4_HIP(hipMalloc(&c.qs, wide / 64 * sizeof(float)));
    G4_HIP(hipMalloc(&c.q8b, wide));
    G4_HIP(hipMalloc(&c.qsb, wide / 64 * sizeof(float)));
    for (int l = 0; l < 15; l++) {
        if (!records[2 + l * 19 + 11].data) continue;
        const int full = l % 5 == 4;
        // global rings start at kGlobalStart positions and grow on demand
        c.cache_len[l] = full ? kGlobalStart : kWindowRing;
        c.cache_dim[l] = full ? 512 : 256;
        const size_t bytes = 2 * (size_t)c.cache_len[l] * c.cache_dim[l] * sizeof(float);
        G4_HIP(hipMalloc(&c.cache[l], bytes));
        G4_HIP(hipMemset(c.cache[l], 0, bytes));
    }
    G4_HIP(hipMalloc(&c.tokens_dev, G4_BATCH * sizeof(int)));
    G4_HIP(hipMalloc(&c.argmax_dev, G4_BATCH * sizeof(int)));
    G4_HIP(hipHostMalloc((void **)&c.tokens_pinned, G4_BATCH * sizeof(int), hipHostMallocDefault));
    G4_HIP(hipMalloc(&c.pos_dev, sizeof(int)));
    G4_HIP(hipHostMalloc((void **)&c.pos_pinned, sizeof(int), hipHostMallocDefault));
    G4_HIP(hipHostMalloc((void **)&c.logits_pinned, G4_VOCAB * sizeof(float), hipHostMallocDefault));
    for (char *&p : c.pieces_pinned) G4_HIP(hipHostMalloc((void **)&p, kCopyPiece, hipHostMallocDefault));
    for (hipEvent_t &e : c.piece_done) G4_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    // Split-K scratch for the widest few-row product (1536 x 12288), and the
    // one-token attention scratch at full context (8 score rows and their
    // split softmax), so that a captured decode step never needs a larger
    // buffer.
    G4_TRY(scratch_reserve((size_t)G4_VOCAB * (G4_HIDDEN / 64) * sizeof(int32_t),
                           attend_scratch_bytes(1, G4_MAX_CONTEXT - 1)));
    // the other lanes' buffers (struct Lane)
    for (LaneBuffers &b : c.extra) {
        G4_HIP(hipMalloc(&b.residual, (size_t)G4_BATCH * G4_HIDDEN * sizeof(float)));
        G4_HIP(hipMalloc(&b.hidden, wide * sizeof(float)));
        G4_HIP(hipMalloc(&b.aux, wide * sizeof(float)));
        G4_HIP(hipMalloc(&b.ple, (size_t)G4_BATCH * G4_LAYERS * G4_PLE * sizeof(float)));
        G4_HIP(hipMalloc(&b.k_new, (size_t)G4_BATCH * 512 * sizeof(float)));
        G4_HIP(hipMalloc(&b.v_new, (size_t)G4_BATCH * 512 * sizeof(float)));
        G4_HIP(hipMalloc(&b.q8, wide));
        G4_HIP(hipMalloc(&b.qs, wide / 64 * sizeof(float)));
        G4_HIP(hipMalloc(&b.q8b, wide));
        G4_HIP(hipMalloc(&b.qsb, wide / 64 * sizeof(float)));
        G4_HIP(hipMalloc(&b.tokens_dev, G4_BATCH * sizeof(int)));
        G4_HIP(hipHostMalloc((void **)&b.tokens_pinned, G4_BATCH * sizeof(int), hipHostMallocDefault));
    }
    G4_HIP(hipDeviceSynchronize());
    c.ready = true;
    return G4_OK;
}

static int matmul(Context &c, float *out, size_t stride, const Weight &w, int rows,
                  bool second = false) {
    return launch_matmul(c.stream, out, stride, second ? c.q8b : c.q8, second ? c.qsb : c.qs,
                         w.data, w.scales, w.n, w.k, rows);
}

// A stream and the activation buffers one forward pass runs on.  Lane 0 is
// c.stream with the context's first set of buffers (every one-token step and
// every other entry point uses it); lanes 1 .. kLanes - 1 have their own
// streams and sets (c.extra).  Consecutive many-token passes over consecutive
// positions (the chunks of a long prefill, gemma4.c:563-566) take the lanes
// in turn and run concurrently: a pass's attention at layer l reads the
// key/value rows the passes before it wrote at layer l, so it waits for the
// previous pass's event (wait_kv[l]) and then records its own (record_kv[l]),
// which thereby covers every earlier pass too.  Every other op is local to
// the pass's rows.  The window rings are long enough that the passes in
// flight never share a slot (kWindowRing).
struct Lane {
    hipStream_t stream = nullptr;
    float *residual = nullptr, *hidden = nullptr, *aux = nullptr, *ple = nullptr;
    float *k_new = nullptr, *v_new = nullptr;
    int8_t *q8 = nullptr, *q8b = nullptr;
    float *qs = nullptr, *qsb = nullptr;
    int *tokens_dev = nullptr, *tokens_pinned = nullptr;
    const FixedScratch *attn_scratch = nullptr;  // null: the library's attention scratch
    hipEvent_t *record_kv = nullptr;             // record [l] after layer l's key/value rows
    hipEvent_t *wait_kv = nullptr;               // wait for [l] before layer l's attention
};

static Lane make_lane(Context &c, int index) {
    Lane ln;
    if (index == 0) {
        ln.stream = c.stream;
        ln.residual = c.residual, ln.hidden = c.hidden, ln.aux = c.aux, ln.ple = c.ple;
        ln.k_new = c.k_new, ln.v_new = c.v_new;
        ln.q8 = c.q8, ln.q8b = c.q8b, ln.qs = c.qs, ln.qsb = c.qsb;
        ln.tokens_dev = c.tokens_dev, ln.tokens_pinned = c.tokens_pinned;
    } else {
        const LaneBuffers &b = c.extra[index - 1];
        ln.stream = b.stream;
        ln.residual = b.residual, ln.hidden = b.hidden, ln.aux = b.aux, ln.ple = b.ple;
        ln.k_new = b.k_new, ln.v_new = b.v_new;
        ln.q8 = b.q8, ln.q8b = b.q8b, ln.qs = b.qs, ln.qsb = b.qsb;
        ln.tokens_dev = b.tokens_dev, ln.tokens_pinned = b.tokens_pinned;
    }
    return ln;
}

// Wait for every lane; afterwards lane 0's buffers and stream serve any call.
static int drain(Context &c) {
    if (c.pending < 0) return G4_OK;
    c.pending = -1;
    for (LaneBuffers &b : c.extra) G4_HIP(hipStreamSynchronize(b.stream));
    G4_HIP(hipStreamSynchronize(c.stream));
    return G4_OK;
}

// The sequence of gemma4.c:463-509 (attention: 411-461) for the n tokens in
// ln.tokens_dev (at positions from start_pos), as launches on ln.stream over
// the lane's buffers.  With pos_dev non-null (n == 1) the
// position-dependent kernels read the position from the device, so the
// launches can be captured once and replayed at every position.
static int enqueue_forward(Context &c, const Lane &ln, int n, int start_pos, const int *pos_dev) {
    hipStream_t s = ln.stream;
    auto matmul = [&](float *out, size_t stride, const Weight &w, int rows, bool second = false) {
        return launch_matmul(s, out, stride, second ? ln.q8b : ln.q8, second ? ln.qsb : ln.qs, w.data,
                             w.scales, w.n, w.k, rows);
    };
    const int ple_width = G4_LAYERS * G4_PLE;

    launch_embedding(s, ln.residual, c.embed.data, c.embed.scales, G4_HIDDEN, c.embed.n, ln.tokens_dev,
                     n, sqrtf((float)G4_HIDDEN));
    launch_quantize(s, ln.q8, ln.qs, ln.residual, (size_t)n * G4_HIDDEN / 64);
    G4_TRY(matmul(ln.ple, ple_width, c.ple_model_proj, n));
    launch_rmsnorm(s, ln.ple, ln.ple, c.ple_norm, G4_PLE, 1e-6f * G4_HIDDEN, (size_t)n * G4_LAYERS);
    launch_embedding(s, ln.hidden, c.embed_ple.data, c.embed_ple.scales, ple_width, c.embed_ple.n,
                     ln.tokens_dev, n, sqrtf((float)G4_PLE));
    launch_add_and_scale(s, ln.ple, ln.hidden, (size_t)n * ple_width, 1.0f / sqrtf(2.0f));

    // In reference order the row-local ops between matmuls run fused
    // (launch_row_tail): the same arithmetic in one launch instead of up to four.
    const bool fused = order() == G4_ORDER_REFERENCE;
    // One token in reference order: the products fused with their neighbours
    // (k_gemv_tail): each row tail runs inside the product it feeds (q, k and
    // v in one launch; gate/up with geglu and the quantize that follows it,
    // into q8b; the per-layer-embedding gate, whose geglu with the per-layer
    // input and quantize run inside the projection that reads it).  The tails alternate
    // two residual rows, since every block of a product reads the residual
    // that block 0 updates: 104 updates a step, so the step ends in
    // ln.residual again.
    const bool one = fused && n == 1;
    float *res[2] = {ln.residual, c.residual_alt};
    int p = 0;  // res[p] holds the residual
    auto tail_job = [&](const float *h, const float *w_in, float scale, const float *w_out) {
        RowTailJob tj{};
        tj.h = h;
        tj.w_in = w_in;
        tj.res_in = res[p];
        tj.res_out = h ? res[p ^ 1] : nullptr;
        tj.scale = scale;
        tj.w_out = w_out;
        tj.eps = 1e-6f;
        if (h) p ^= 1;
        return tj;
    };
    if (fused && !one)  // layer 0's input norm + quantize
        launch_row_tail(s, nullptr, nullptr, ln.residual, 1.0f, c.layers[0].input_ln, nullptr, ln.q8,
                        ln.qs, 1e-6f, n, 0, 0, 1, 1);
    auto job_on = [&]() {
        GemvJob job{};
        job.gelu_table = c.gelu;
        job.gelu_size = c.gelu_size;
        job.gelu_lower = c.gelu_lower;
        job.gelu_upper = c.gelu_upper;
        return job;
    };
    for (int l = 0; l < G4_LAYERS; l++) {
        const Layer &L = c.layers[l];
        const int hd = L.head_dim, qw = L.query_width, heads = qw / hd;
        if (!fused) {
            launch_rmsnorm(s, ln.hidden, ln.residual, L.input_ln, G4_HIDDEN, 1e-6f, n);
            launch_quantize(s, ln.q8, ln.qs, ln.hidden, (size_t)n * G4_HIDDEN / 64);
        }

        // attention
        float *keys = c.cache[L.owner];
        const int cache_len = c.cache_len[L.owner];
        float *values = keys + (size_t)cache_len * hd;
        if (one) {
            GemvJob job = job_on();
            job.k = G4_HIDDEN;
            job.m[0] = GemvMat{L.q.data, L.q.scales, ln.aux, qw / 16};
            job.count = 1;
            if (L.k.data) {
                job.m[1] = GemvMat{L.k.data, L.k.scales, ln.k_new, hd / 16};
                job.m[2] = GemvMat{L.v.data, L.v.scales, ln.v_new, hd / 16};
                job.count = 3;
            }
            // the previous layer's last tail + this layer's input norm (layer
            // 0: the input norm alone)
            const RowTailJob tj = l == 0 ? tail_job(nullptr, nullptr, 1.0f, L.input_ln)
                                         : tail_job(ln.hidden, c.layers[l - 1].post_ple_ln,
                                                    c.layers[l - 1].layer_scalar, L.input_ln);
            G4_TRY(launch_gemv_tail(s, job, EPI_PLAIN, tj, l == 0 ? 3 : 1));
        } else if (L.k.data && n > 8 && G4_HIDDEN % 512 == 0) {
            // q, k and v read the same rows: one launch fills the chip
            const int8_t *w[3] = {L.q.data, L.k.data, L.v.data};
            const uint16_t *ws[3] = {L.q.scales, L.k.scales, L.v.scales};
            float *out[3] = {ln.aux, ln.k_new, ln.v_new};
            const size_t strides[3] = {(size_t)qw, (size_t)hd, (size_t)hd};
            const int ns[3] = {L.q.n, L.k.n, L.v.n};
            G4_TRY(launch_matmul_group(s, ln.q8, ln.qs, n, G4_HIDDEN, 3, w, ws, out, strides, ns));
        } else {
            G4_TRY(matmul(ln.aux, qw, L.q, n));
            if (L.k.data) {
                G4_TRY(matmul(ln.k_new, hd, L.k, n));
                G4_TRY(matmul(ln.v_new, hd, L.v, n));
            }
        }
        if (fused) {  // query norms + RoPE and the new key/value rows: one launch
            launch_qkv_finish(s, ln.aux, heads, L.q_norm, L.k.data ? ln.k_new : nullptr, ln.v_new,
                              L.k_norm, keys, values, L.rope_cos, L.rope_sin, L.pairs, hd, cache_len,
                              start_pos, pos_dev, n);
        } else {
            launch_rmsnorm(s, ln.aux, ln.aux, L.q_norm, hd, 1e-6f, (size_t)n * heads);
            launch_rope(s, L.rope_cos, L.rope_sin, L.pairs, ln.aux, heads, hd, start_pos, pos_dev, n);
            if (L.k.data)
                launch_kv_finish(s, keys, values, ln.k_new, ln.v_new, L.k_norm, L.rope_cos, L.rope_sin,
                                 L.pairs, hd, cache_len, start_pos, pos_dev, n);
        }
        // after the wait: the event then also stands for every earlier pass's
        // rows of this layer (a pass two back is on another stream)
        if (L.k.data && ln.wait_kv) G4_HIP(hipStreamWaitEvent(s, ln.wait_kv[l], 0));
        if (L.k.data && ln.record_kv) G4_HIP(hipEventRecord(ln.record_kv[l], s));
        G4_TRY(launch_attend(s, ln.hidden, ln.aux, keys, values, cache_len, hd, heads, L.full,
                             start_pos, pos_dev, n, ln.q8, ln.qs, ln.attn_scratch));
        G4_TRY(matmul(ln.hidden, G4_HIDDEN, L.o, n));

        // feed-forward
        if (one) {
            // the tail runs inside the gate/up product below
        } else if (fused) {
            launch_row_tail(s, ln.hidden, L.post_attn_ln, ln.residual, 1.0f, L.pre_ffn_ln, nullptr,
                            ln.q8, ln.qs, 1e-6f, n, 1, 1, 1, 1);
        } else {
            launch_rmsnorm(s, ln.hidden, ln.hidden, L.post_attn_ln, G4_HIDDEN, 1e-6f, n);
            launch_add_and_scale(s, ln.residual, ln.hidden, (size_t)n * G4_HIDDEN, 1.0f);
            launch_rmsnorm(s, ln.hidden, ln.residual, L.pre_ffn_ln, G4_HIDDEN, 1e-6f, n);
            launch_quantize(s, ln.q8, ln.qs, ln.hidden, (size_t)n * G4_HIDDEN / 64);
        }
        // many rows: gate and up in one GEMM whose epilogue applies geglu and
        // quantizes (into q8b)
        const bool gemm_fused = n > 8;
        auto gelu_epilogue = [&]() {
            GemmEpilogue ep{};
            ep.gelu_table = c.gelu;
            ep.gelu_size = c.gelu_size;
            ep.gelu_lower = c.gelu_lower;
            ep.gelu_upper = c.gelu_upper;
            ep.q_out = ln.q8b;
            ep.qs_out = ln.qsb;
            return ep;
        };
        if (gemm_fused) {
            GemmEpilogue ep = gelu_epilogue();
            ep.w2 = L.up.data;
            ep.ws2 = L.up.scales;
            G4_TRY(launch_matmul_gelu(s, ln.q8, ln.qs, L.gate.data, L.gate.scales, L.ffn, G4_HIDDEN, n,
                                      EPI_GELU_PAIR, ep));
        } else if (one) {
            GemvJob job = job_on();
            job.k = G4_HIDDEN;
            job.m[0] = GemvMat{L.gate.data, L.gate.scales, nullptr, L.ffn / 16};
            job.m[1] = GemvMat{L.up.data, L.up.scales, nullptr, L.ffn / 16};
            job.count = 2;
            job.q_out = ln.q8b;
            job.qs_out = ln.qsb;
            const RowTailJob tj = tail_job(ln.hidden, L.post_attn_ln, 1.0f, L.pre_ffn_ln);
            G4_TRY(launch_gemv_tail(s, job, EPI_GELU_PAIR, tj, 1));
        } else {
            G4_TRY(matmul(ln.hidden, L.ffn, L.gate, n));
            G4_TRY(matmul(ln.aux, L.ffn, L.up, n));
            launch_geglu(s, ln.hidden, ln.aux, n, L.ffn, L.ffn, c.gelu, c.gelu_size, c.gelu_lower,
                         c.gelu_upper);
            launch_quantize(s, ln.q8, ln.qs, ln.hidden, (size_t)n * L.ffn / 64);
        }
        G4_TRY(matmul(ln.hidden, G4_HIDDEN, L.down, n, one || gemm_fused));

        // per-layer embedding
        if (one) {
            // the tail runs inside the per-layer-embedding gate below
        } else if (fused) {
            launch_row_tail(s, ln.hidden, L.post_ffn_ln, ln.residual, 1.0f, nullptr, nullptr, ln.q8,
                            ln.qs, 1e-6f, n, 1, 1, 0, 1);
        } else {
            launch_rmsnorm(s, ln.hidden, ln.hidden, L.post_ffn_ln, G4_HIDDEN, 1e-6f, n);
            launch_add_and_scale(s, ln.residual, ln.hidden, (size_t)n * G4_HIDDEN, 1.0f);
            launch_quantize(s, ln.q8, ln.qs, ln.residual, (size_t)n * G4_HIDDEN / 64);
        }
        if (gemm_fused) {
            GemmEpilogue ep = gelu_epilogue();
            ep.mul = ln.ple + (size_t)l * G4_PLE;
            ep.mul_stride = ple_width;
            G4_TRY(launch_matmul_gelu(s, ln.q8, ln.qs, L.ple_gate.data, L.ple_gate.scales, G4_PLE,
                                      G4_HIDDEN, n, EPI_GELU_MUL, ep));
        } else if (one) {
            // the gate as a plain product of the tail's row; geglu with the
            // per-layer input and its quantize run inside the projection
            GemvJob job = job_on();
            job.k = G4_HIDDEN;
            job.m[0] = GemvMat{L.ple_gate.data, L.ple_gate.scales, ln.aux, G4_PLE / 16};
            job.count = 1;
            const RowTailJob tj = tail_job(ln.hidden, L.post_ffn_ln, 1.0f, nullptr);
            G4_TRY(launch_gemv_tail(s, job, EPI_PLAIN, tj, 2));
        } else {
            G4_TRY(matmul(ln.hidden, G4_PLE, L.ple_gate, n));
            launch_geglu(s, ln.hidden, ln.ple + (size_t)l * G4_PLE, n, G4_PLE, ple_width, c.gelu,
                         c.gelu_size, c.gelu_lower, c.gelu_upper);
            launch_quantize(s, ln.q8, ln.qs, ln.hidden, (size_t)n * G4_PLE / 64);
        }
        if (one)
            G4_TRY(launch_gemv_gelu(s, ln.hidden, ln.aux, ln.ple + (size_t)l * G4_PLE, c.gelu, c.gelu_size,
                                    c.gelu_lower, c.gelu_upper, L.ple_proj.data, L.ple_proj.scales, G4_HIDDEN,
                                    G4_PLE));
        else
            G4_TRY(matmul(ln.hidden, G4_HIDDEN, L.ple_proj, n, gemm_fused));
        if (one) {
            if (l + 1 == G4_LAYERS)  // the last tail, in place (the others run in the next q/k/v)
                launch_row_tail(s, ln.hidden, L.post_ple_ln, res[p], L.layer_scalar, nullptr, nullptr,
                                nullptr, nullptr, 1e-6f, n, 1, 1, 0, 0);
        } else if (fused) {
            if (l + 1 < G4_LAYERS)  // + the next layer's input norm and quantize
                launch_row_tail(s, ln.hidden, L.post_ple_ln, ln.residual, L.layer_scalar,
                                c.layers[l + 1].input_ln, nullptr, ln.q8, ln.qs, 1e-6f, n, 1, 1, 1, 1);
            else
                launch_row_tail(s, ln.hidden, L.post_ple_ln, ln.residual, L.layer_scalar, nullptr,
                                nullptr, nullptr, nullptr, 1e-6f, n, 1, 1, 0, 0);
        } else {
            launch_rmsnorm(s, ln.hidden, ln.hidden, L.post_ple_ln, G4_HIDDEN, 1e-6f, n);
            launch_add_and_scale(s, ln.residual, ln.hidden, (size_t)n * G4_HIDDEN, L.layer_scalar);
        }
    }
    if (p != 0) return set_error(G4_ERR_STATE, "one-token step ended in the alternate residual row");
    G4_HIP(hipGetLastError());
    return G4_OK;
}

// Capture the one-token forward pass into c.decode_graph.
static int capture_decode(Context &c) {
    if (c.decode_graph) {
        G4_HIP(hipGraphExecDestroy(c.decode_graph));
        c.decode_graph = nullptr;
    }
    hipGraph_t graph = nullptr;
    G4_HIP(hipStreamBeginCapture(c.stream, hipStreamCaptureModeRelaxed));
    const int rc = enqueue_forward(c, make_lane(c, 0), 1, 0, c.pos_dev);
    hipError_t end = hipStreamEndCapture(c.stream, &graph);
    if (rc) {
        if (graph) (void)hipGraphDestroy(graph);
        return rc;
    }
    G4_HIP(end);
    hipError_t inst = hipGraphInstantiate(&c.decode_graph, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    G4_HIP(inst);
    c.graph_generation = scratch().generation;
    c.graph_order = order();
    c.graph_kv_generation = c.kv_generation;
    return G4_OK;
}

// Global-attention rings hold every position from 0, so they must cover the
// last position of a forward pass.  They start at kGlobalStart positions and
// double (to G4_MAX_CONTEXT at most), keys and values copied to the new
// buffer, the new rows zeroed: a short context does not pay for 131072
// positions of fp32 keys and values per ring (gemma4.c:164-165 allocates
// them all).  A ring grows once it would hold less than one more batch past
// the pass, so a prefill leaves room for the decode steps that follow (they
// do not stop to grow it).  Runs between forward passes, outside any graph
// capture.
static int ensure_kv(Context &c, int last_pos) {
    const int need = last_pos + G4_BATCH < G4_MAX_CONTEXT ? last_pos + G4_BATCH : G4_MAX_CONTEXT - 1;
    for (int l = 0; l < 15; l++) {
        if (!c.cache[l] || c.cache_dim[l] != 512 || need < c.cache_len[l]) continue;
        G4_TRY(drain(c));  // a pass in flight may read the ring
        int len = c.cache_len[l];
        while (len <= need && len < G4_MAX_CONTEXT) len *= 2;
        const size_t hd = (size_t)c.cache_dim[l], old_len = (size_t)c.cache_len[l];
        float *grown = nullptr;
        G4_HIP(hipMalloc(&grown, 2 * (size_t)len * hd * sizeof(float)));
        const size_t old_bytes = old_len * hd * sizeof(float), new_bytes = (size_t)len * hd * sizeof(float);
        hipError_t e = hipMemcpyAsync(grown, c.cache[l], old_bytes, hipMemcpyDeviceToDevice, c.stream);
        if (e == hipSuccess)
            e = hipMemcpyAsync(grown + (size_t)len * hd, c.cache[l] + old_len * hd, old_bytes,
                               hipMemcpyDeviceToDevice, c.stream);
        if (e == hipSuccess) e = hipMemsetAsync((char *)grown + old_bytes, 0, new_bytes - old_bytes, c.stream);
        if (e == hipSuccess)
            e = hipMemsetAsync((char *)(grown + (size_t)len * hd) + old_bytes, 0, new_bytes - old_bytes, c.stream);
        if (e == hipSuccess) e = hipStreamSynchronize(c.stream);
        if (e != hipSuccess) {
            (void)hipFree(grown);
            return set_error(G4_ERR_DEVICE, "growing the KV ring of layer %d: %s", l, hipGetErrorString(e));
        }
        G4_HIP(hipFree(c.cache[l]));
        c.cache[l] = grown;
        c.cache_len[l] = len;
        c.kv_generation++;
    }
    return G4_OK;
}

// A lane's attention scratch, grown to `bytes` once the lane's previous pass
// has finished.  Each lane grows its own when it runs, so a prefill run one
// chunk at a time holds one lane's score rows, not four.
static int reserve_lane_attn(Context &c, int lane, hipStream_t stream, size_t bytes) {
    if (bytes <= c.lane_attn_bytes[lane]) return G4_OK;
    G4_HIP(hipStreamSynchronize(stream));
    release(c.lane_attn[lane]);
    c.lane_attn[lane] = nullptr;
    c.lane_attn_bytes[lane] = 0;
    G4_HIP(hipMalloc(&c.lane_attn[lane], bytes));
    c.lane_attn_bytes[lane] = bytes;
    return G4_OK;
}

// gemma4.c:463 for n tokens at start_pos.  A pass of more than 8 tokens is
// enqueued and left running on a lane (struct Lane): when it continues the
// pass before it (start_pos where that one ended) the two run concurrently;
// every entry point that reads results, and any other pass, waits for the
// lanes first (drain).  At most one pass per lane is in flight.  Shorter
// passes (decode steps) run on lane 0 and return finished.
static int forward(Context &c, const int *tokens, int n, int start_pos) {
    const int last_pos = start_pos + n - 1;
    if (n <= 8) {  // their products take the split-K GEMV, whose scratch is shared
        G4_TRY(drain(c));
        G4_TRY(ensure_kv(c, last_pos));
        hipStream_t s = c.stream;
        memcpy(c.tokens_pinned, tokens, (size_t)n * sizeof(int));
        G4_HIP(hipMemcpyAsync(c.tokens_dev, c.tokens_pinned, (size_t)n * sizeof(int),
                              hipMemcpyHostToDevice, s));
        if (n == 1 && order() == G4_ORDER_REFERENCE) {
            *c.pos_pinned = start_pos;
            G4_HIP(hipMemcpyAsync(c.pos_dev, c.pos_pinned, sizeof(int), hipMemcpyHostToDevice, s));
            if (!c.decode_graph || c.graph_generation != scratch().generation ||
                c.graph_order != order() || c.graph_kv_generation != c.kv_generation)
                G4_TRY(capture_decode(c));
            G4_HIP(hipGraphLaunch(c.decode_graph, s));
        } else {
            G4_TRY(enqueue_forward(c, make_lane(c, 0), n, start_pos, nullptr));
        }
        // finished before returning: these passes use the library's shared
        // scratch (split-K dots, one-token attention rows), which the per-op
        // entry points also use, on the caller's streams
        G4_HIP(hipStreamSynchronize(s));
        c.last_n = n;
        c.last_lane = 0;
        return G4_OK;
    }
    G4_TRY(ensure_kv(c, last_pos));  // drains before it moves a buffer
    const bool follow = c.pending >= 0 && start_pos == c.next_pos;
    if (!follow) G4_TRY(drain(c));
    const int lane = follow ? (c.pending + 1) % kLanes : 0;
    Lane ln = make_lane(c, lane);
    G4_HIP(hipStreamSynchronize(ln.stream));  // the lane's previous pass: its buffers are free
    G4_TRY(reserve_lane_attn(c, lane, ln.stream, attend_scratch_bytes(G4_BATCH, last_pos)));
    const FixedScratch attn{c.lane_attn[lane], c.lane_attn_bytes[lane]};
    ln.attn_scratch = &attn;
    ln.record_kv = c.kv_written[lane];
    ln.wait_kv = follow ? c.kv_written[c.pending] : nullptr;
    memcpy(ln.tokens_pinned, tokens, (size_t)n * sizeof(int));
    G4_HIP(hipMemcpyAsync(ln.tokens_dev, ln.tokens_pinned, (size_t)n * sizeof(int), hipMemcpyHostToDevice,
                          ln.stream));
    c.pending = lane;
    c.next_pos = start_pos + n;
    c.last_lane = lane;
    c.last_n = n;
    const int rc = enqueue_forward(c, ln, n, start_pos, nullptr);
    if (rc) {
        char saved[sizeof(g_error)];
        memcpy(saved, g_error, sizeof(saved));
        (void)drain(c);
        memcpy(g_error, saved, sizeof(saved));
        c.last_n = 0;
    }
    return rc;
}

// gemma4.c:512-522 for `rows` consecutive rows starting at `row`, into dst.
// The rows are the last pass's (on its lane); the work runs on lane 0 once
// every lane has finished.
static int logits_rows(Context &c, float *dst, size_t row, int rows) {
    G4_TRY(drain(c));
    hipStream_t s = c.stream;
    float *residual = make_lane(c, c.last_lane).residual + row * G4_HIDDEN;
    if (order() == G4_ORDER_REFERENCE) {
        launch_row_tail(s, nullptr, nullptr, residual, 1.0f, c.final_norm, nullptr, c.q8, c.qs, 1e-6f,
                        rows, 0, 0, 1, 1);
    } else {
        launch_rmsnorm(s, c.aux, residual, c.final_norm, G4_HIDDEN, 1e-6f, rows);
        launch_quantize(s, c.q8, c.qs, c.aux, (size_t)rows * G4_HIDDEN / 64);
    }
    G4_TRY(matmul(c, dst, G4_VOCAB, c.embed, rows));
    launch_softcap(s, dst, (size_t)rows * G4_VOCAB);
    G4_HIP(hipGetLastError());
    return G4_OK;
}

}  // namespace g4

using namespace g4;

extern "C" const char *g4_last_error(void) { return g4::g_error; }

extern "C" int g4_init(const g4_tensor *records, int device) {
    G4_CHECK(records, "g4_init: null records");
    if (g_ctx.ready) return set_error(G4_ERR_STATE, "g4_init: already initialised (call g4_shutdown first)");
    int rc = init(records, device);
    if (rc) {
        char saved[sizeof(g_error)];
        memcpy(saved, g_error, sizeof(saved));
        free_all(g_ctx);
        memcpy(g_error, saved, sizeof(saved));
    }
    return rc;
}

extern "C" int g4_forward(const int *tokens, size_t token_count, int start_pos) {
    Context &c = g_ctx;
    if (!c.ready) return set_error(G4_ERR_STATE, "g4_forward: g4_init has not succeeded");
    G4_CHECK(tokens, "g4_forward: null tokens");
    G4_CHECK(token_count >= 1 && token_count <= G4_BATCH, "g4_forward: token_count %zu not in 1..%d",
             token_count, G4_BATCH);
    G4_CHECK(start_pos >= 0 && (long)start_pos + (long)token_count <= G4_MAX_CONTEXT,
             "g4_forward: positions %d..%ld exceed the %d-token context", start_pos,
             (long)start_pos + (long)token_count - 1, G4_MAX_CONTEXT);
    for (size_t i = 0; i < token_count; i++)
        G4_CHECK(tokens[i] >= 0 && tokens[i] < G4_VOCAB, "g4_forward: token %d at index %zu out of range",
                 tokens[i], i);
    G4_HIP(hipSetDevice(c.device));
    return forward(c, tokens, (int)token_count, start_pos);
}

extern "C" int g4_logits(size_t token, float *out) {
    Context &c = g_ctx;
    if (!c.ready || !c.last_n) return set_error(G4_ERR_STATE, "g4_logits: no forward pass yet");
    G4_CHECK(out, "g4_logits: null output");
    G4_CHECK(token < (size_t)c.last_n, "g4_logits: row %zu not in the last forward (%d rows)", token,
             c.last_n);
    G4_HIP(hipSetDevice(c.device));
    G4_TRY(logits_rows(c, c.logits, token, 1));
    G4_HIP(hipMemcpyAsync(c.logits_pinned, c.logits, G4_VOCAB * sizeof(float), hipMemcpyDeviceToHost,
                          c.stream));
    G4_HIP(hipStreamSynchronize(c.stream));
    memcpy(out, c.logits_pinned, G4_VOCAB * sizeof(float));
    return G4_OK;
}

extern "C" int g4_logits_all(float *out) {
    Context &c = g_ctx;
    if (!c.ready || !c.last_n) return set_error(G4_ERR_STATE, "g4_logits_all: no forward pass yet");
    G4_CHECK(out, "g4_logits_all: null output");
    G4_HIP(hipSetDevice(c.device));
    if (!c.logits_all) G4_HIP(hipMalloc(&c.logits_all, (size_t)G4_BATCH * G4_VOCAB * sizeof(float)));
    G4_TRY(logits_rows(c, c.logits_all, 0, c.last_n));
    // piece i goes to pinned buffer i % 2 by DMA; while piece i + 1's DMA
    // runs, the host copies piece i out (buffer i % 2 is reused only after
    // that copy returned)
    const size_t total = (size_t)c.last_n * G4_VOCAB * sizeof(float);
    const size_t pieces = (total + kCopyPiece - 1) / kCopyPiece;
    const char *src = (const char *)c.logits_all;
    auto size_of = [&](size_t i) { return i + 1 < pieces ? kCopyPiece : total - i * kCopyPiece; };
    G4_HIP(hipMemcpyAsync(c.pieces_pinned[0], src, size_of(0), hipMemcpyDeviceToHost, c.stream));
    G4_HIP(hipEventRecord(c.piece_done[0], c.stream));
    for (size_t i = 0; i < pieces; i++) {
        if (i + 1 < pieces) {
            G4_HIP(hipMemcpyAsync(c.pieces_pinned[(i + 1) & 1], src + (i + 1) * kCopyPiece, size_of(i + 1),
                                  hipMemcpyDeviceToHost, c.stream));
            G4_HIP(hipEventRecord(c.piece_done[(i + 1) & 1], c.stream));
        }
        G4_HIP(hipEventSynchronize(c.piece_done[i & 1]));
        copy_parallel((char *)out + i * kCopyPiece, c.pieces_pinned[i & 1], size_of(i));
    }
    return G4_OK;
}

extern "C" int g4_argmax(size_t token, int *out_token) {
    Context &c = g_ctx;
    if (!c.ready || !c.last_n) return set_error(G4_ERR_STATE, "g4_argmax: no forward pass yet");
    G4_CHECK(out_token, "g4_argmax: null output");
    G4_CHECK(token < (size_t)c.last_n, "g4_argmax: row %zu not in the last forward", token);
    G4_HIP(hipSetDevice(c.device));
    G4_TRY(logits_rows(c, c.logits, token, 1));
    launch_argmax(c.stream, c.argmax_dev, c.logits, 1, G4_VOCAB);
    G4_HIP(hipMemcpyAsync(out_token, c.argmax_dev, sizeof(int), hipMemcpyDeviceToHost, c.stream));
    G4_HIP(hipStreamSynchronize(c.stream));
    return G4_OK;
}

extern "C" int g4_sample(size_t token, float temperature, uint64_t *rng_state, int *out_token) {
    Context &c = g_ctx;
    if (!c.ready || !c.last_n) return set_error(G4_ERR_STATE, "g4_sample: no forward pass yet");
    G4_CHECK(out_token && rng_state, "g4_sample: null output");
    G4_CHECK(token < (size_t)c.last_n, "g4_sample: row %zu not in the last forward", token);
    G4_HIP(hipSetDevice(c.device));
    G4_TRY(logits_rows(c, c.logits, token, 1));
    uint64_t *result = nullptr;
    G4_TRY(launch_sample(c.stream, c.logits, G4_VOCAB, temperature, *rng_state, &result));
    return finish_sample(c.stream, result, temperature, rng_state, out_token);
}

extern "C" void g4_shutdown(void) {
    if (g_ctx.ready || g_ctx.arena) {
        free_all(g_ctx);
    } else {  // per-op use only: the buffers those calls grew
        scratch_release();
        layer_buffers_release();
    }
}

extern "C" void *g4_stream(void) { return g_ctx.stream; }
