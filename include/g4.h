/*
 * g4.h -- C ABI of the MI355X (gfx950) W8A8 forward path for gemma4.c.
 *
 * Drop-in boundary.  The reference's inference path is a set of plain C
 * functions called from serial host code (gemma4.c:566, 569, 600, 605, 632-633,
 * 640-641).  The model-level entry points below replace forward() and logits();
 * the per-op entry points replace the kernels underneath them and exist so the
 * parity tests can check each one in isolation.
 *
 * Conventions:
 *   - every function returns G4_OK (0) or a nonzero status; g4_last_error()
 *     then holds a one-line message (the reference's error style is a message
 *     on stderr plus exit(1) in its main(); the host keeps that);
 *   - per-op entry points take DEVICE pointers and a hipStream_t passed as
 *     void* (NULL = the null stream), and are asynchronous on that stream;
 *   - model-level entry points take host pointers, run on the library's own
 *     stream and return when their result is ready;
 *   - one model context per process, not thread-safe (the reference likewise
 *     has one Model and one InferenceState).
 */
#ifndef G4_H
#define G4_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Shape constants of the reference (gemma4.c:26-31) and its exporter. */
#define G4_LAYERS 35
#define G4_HIDDEN 1536
#define G4_VOCAB 262144
#define G4_MAX_CONTEXT 131072
#define G4_WINDOW 512
#define G4_BATCH 512
#define G4_PLE 256
#define G4_HEADS 8
#define G4_RECORDS 671 /* 2 + 35*19 + 4 tensor records */

#define G4_OK 0
#define G4_ERR_ARG 1    /* invalid argument (shape, size, null pointer, range) */
#define G4_ERR_DEVICE 2 /* HIP runtime error or no device */
#define G4_ERR_STATE 3  /* call order (e.g. forward before init) */

/* One tensor record of the memory image: identical layout to the reference's
 * Tensor (gemma4.c:119-123), 32 bytes.  Quantized matrices [rows x cols] keep
 * int8 data in 1024-byte tiles (16 rows x 64 columns; byte (chunk c, row r, j)
 * at c*64 + r*4 + j) in row-block-major order, and fp16 scales per (row,
 * 64-column group) ordered [row block][group][16] (exporter.py:304-316).
 * fp32 tensors have scales == NULL. */
typedef struct {
    void *data;
    uint16_t *scales;
    int32_t shape[4];
} g4_tensor;

/* Message for the last nonzero status (never NULL). */
const char *g4_last_error(void);

/* ---- Model-level entry points ------------------------------------------ */

/* Upload the model once.  `records` is the reference's ModelWeights viewed as
 * G4_RECORDS tensors (gemma4.c:147-155) with data/scales already turned into
 * host pointers (gemma4.c:681-685).  Allocates the device KV caches (fp32) and
 * activations.  Replaces nothing in the reference: it is the new init step a
 * host calls after its loader (gemma4.c:686). `device` is the HIP ordinal. */
int g4_init(const g4_tensor *records, int device);

/* Replaces forward() (gemma4.c:463): runs token_count (1..G4_BATCH) tokens at
 * positions start_pos.. through all 35 layers, updating the device KV caches.
 * Requires start_pos + token_count <= G4_MAX_CONTEXT.  `tokens` is copied
 * before the call returns.  A pass of more than 8 tokens may still be running
 * on the device when it returns: the next pass, if it starts where this one
 * ended (the reference's prefill chunks, gemma4.c:563-566), runs concurrently
 * with it (up to four passes at once), and every other entry point below
 * waits for all of them first; errors the device raises in such a pass
 * surface at a later call.  Shorter passes (decode steps) return finished. */
int g4_forward(const int *tokens, size_t token_count, int start_pos);

/* Replaces logits() (gemma4.c:512): final norm, tied lm_head and soft cap for
 * row `token` (< last token_count) of the last forward; writes G4_VOCAB floats
 * to host memory `out`. */
int g4_logits(size_t token, float *out);

/* Logits of every row of the last forward in one batched lm_head pass:
 * writes token_count x G4_VOCAB floats (row-major) to host memory `out`.  Same
 * values as calling g4_logits(i, ...) for each row (the --dump-logits loop,
 * gemma4.c:567-570). */
int g4_logits_all(float *out);

/* Greedy next token for row `token` (first maximum, gemma4.c:537-541),
 * computed on the device so only one int crosses the bus. */
int g4_argmax(size_t token, int *out_token);

/* sample() (gemma4.c:536-561) of row `token` of the last forward pass, on the
 * device: temperature <= 0 is the first maximum; otherwise the 64 highest
 * logits, the smallest prefix holding 95% of their softmax at `temperature`,
 * and one xorshift64* draw (random_uniform, gemma4.c:529-534) from
 * *rng_state -- the reference's global rng_state (gemma4.c:527), passed in
 * and advanced in place exactly as the reference advances it.  Replaces
 * logits() + sample() in generate() (gemma4.c:600): only the token and the
 * state cross the bus. */
int g4_sample(size_t token, float temperature, uint64_t *rng_state, int *out_token);

/* Free every device resource of the model context. */
void g4_shutdown(void);

/* The library's HIP stream (a hipStream_t) for timing with HIP events: the
 * stream of every entry point here, except that consecutive many-token passes
 * (g4_forward) take this and three more streams in turn; the next
 * g4_logits / g4_argmax / g4_sample / one-token g4_forward waits for all. */
void *g4_stream(void);

/* Summation order of rmsnorm and attention, for every later call (model and
 * per-op).  G4_ORDER_REFERENCE (the default) reproduces the reference's
 * sequential fp32 sums (gemma4.c:366-368, 400-408, 296-307) and its libm expf
 * bit for bit, so the whole step is bit-identical to gemma4.c up to the final
 * tanhf.  G4_ORDER_PARALLEL uses tree sums and split-KV flash decoding:
 * faster, equal to within fp32 rounding per op.  Returns the previous order. */
#define G4_ORDER_REFERENCE 0
#define G4_ORDER_PARALLEL 1
int g4_set_order(int order);

/* ---- Per-op entry points (device pointers) ------------------------------ */

/* gemma4.c:265-279: per 64-value group, scale = max|x|/127, q = rint(x/scale). */
int g4_quantize(void *stream, int8_t *q, float *scales, const float *x, size_t rows,
                size_t width);

/* gemma4.c:257-262: out[rows x N] = W8A8 product of the quantized rows with the
 * packed matrix w (N = w->shape[0], K = w->shape[1]; data/scales are device
 * pointers).  Output row stride is N. */
int g4_matmul_int8(void *stream, float *out, const int8_t *xq, const float *xs,
                   const g4_tensor *w, size_t rows);

/* gemma4.c:360-373: y = w * (x / sqrt(mean(x^2) + eps)); weight may be NULL. */
int g4_rmsnorm(void *stream, float *out, const float *in, const float *weight, int width,
               float epsilon, size_t rows);

/* gemma4.c:375-378: out = (out + add) * scale. */
int g4_add_and_scale(void *stream, float *out, const float *add, size_t n, float scale);

/* gemma4.c:381-398: rotate channel pairs (j, j + head_dim/2), j < pairs, with
 * rows start_pos.. of the [positions x pairs] cos/sin tables. */
int g4_apply_rope(void *stream, const float *cosines, const float *sines, int pairs, float *v,
                  int heads, int head_dim, int start_pos, size_t n);

/* gemma4.c:310-331: gate = GELU_table(gate) * up (row stride of up: up_stride). */
int g4_geglu(void *stream, float *gate, const float *up, int rows, int width, int up_stride,
             const float *table, int table_size, float lower, float upper);

/* gemma4.c:337-358: gather and dequantize packed rows; tokens is a device array. */
int g4_embedding(void *stream, float *out, const g4_tensor *table, const int *tokens,
                 size_t n, float multiplier);

/* gemma4.c:400-408: softmax of `rows` independent rows of `count` values in
 * place, in the reference's order with its libm expf (bit-identical). */
int g4_softmax(void *stream, float *values, int count, size_t rows);

/* gemma4.c:536-561: sample() over `vocab` (64 .. G4_VOCAB) device logits with
 * the generator state in *rng_state (advanced in place when temperature > 0).
 * Synchronizes `stream`. */
int g4_sample_logits(void *stream, const float *logits, int vocab, float temperature,
                     uint64_t *rng_state, int *out_token);

/* gemma4.c:443-456: causal attention of n query tokens (heads x head_dim each,
 * row-major) at positions start_pos.. over a ring KV cache of cache_len rows;
 * sliding layers (full_attention = 0) see the last G4_WINDOW positions.
 * head_dim 256 or 512; heads must be 8 (the model's) in G4_ORDER_REFERENCE,
 * 1..8 in G4_ORDER_PARALLEL.  Grows a library-owned device scratch buffer
 * (hipMalloc) when a call needs more than it holds. */
int g4_attend(void *stream, float *out, const float *q, const float *key_cache,
              const float *value_cache, int cache_len, int head_dim, int heads,
              int full_attention, int start_pos, size_t n);

/* gemma4.c:411-461 (attention()): one layer's attention in place over the n
 * rows (1..G4_BATCH) of `hidden` ([n x G4_HIDDEN] fp32, device, 16-byte
 * aligned): they come in as attention()'s input (the input norm applied,
 * gemma4.c:483) and leave as the o projection's output.  `layer` holds the
 * layer's 19 records in LayerWeights order (gemma4.c:125-155) with device
 * data; a layer whose k_proj has no data reads the cache without writing it
 * (the shared layers, gemma4.c:419-421, 432).  `cache` is the cache owner's
 * keys [cache_len x head_dim] followed by its values (gemma4.c:421-422); new rows
 * go to (start_pos + t) & (cache_len - 1).  head_dim is q_norm's length (256
 * or 512), 8 query heads; sliding layers (full_attention = 0) see the last
 * G4_WINDOW positions.  Grows library-owned device buffers (hipMalloc) when a
 * call has more rows than they hold; g4_shutdown frees them.  Those buffers
 * (the query heads, the new key/value rows, the quantized activations) are
 * one set for the process: calls that overlap in time, e.g. on two streams,
 * race on them, so a caller orders its calls on one stream or waits between
 * them. */
int g4_attention_layer(void *stream, float *hidden, size_t n, int start_pos, const g4_tensor *layer,
                       float *cache, int cache_len, int full_attention);

/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  g4_attend with the same arguments and results, its
 * scratch (the score rows, or the split-KV partials in G4_ORDER_PARALLEL)
 * taken from a fixed array of G4_ATTEND_NOALLOC_SCRATCH_BYTES that the
 * library holds on every device it runs on until the process ends.  Allocates
 * nothing.  Returns G4_ERR_ARG, launching nothing, when a call needs more:
 * reference order needs n * 8 * align64(visible keys) floats (e.g. one token
 * at the full 131072-token context, or a 512-token chunk whose keys reach
 * position 2047); parallel order n * ceil(keys / 64) * heads * (head_dim + 2)
 * floats.  Every call on a device shares that device's array: calls that
 * overlap in time on one device race. */
#define G4_ATTEND_NOALLOC_SCRATCH_BYTES (32u << 20)
int g4_attend_noalloc(void *stream, float *out, const float *q, const float *key_cache,
                      const float *value_cache, int cache_len, int head_dim, int heads,
                      int full_attention, int start_pos, size_t n);

#ifdef __cplusplus
}
#endif
#endif
