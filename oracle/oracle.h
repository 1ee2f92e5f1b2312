/*
 * oracle.h -- CPU restatement of gemma4.c's W8A8 forward path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * path and the timed CPU baseline beside it.  Only tests/, the smoke check in
 * __graft_entry__.py and the cpu_baseline leg of bench.py may load it.  The
 * product library (libg4.so) never links or calls it.
 *
 * Every function restates one reference function with the same arithmetic
 * order (citations are gemma4.c:line of the reference).  The library is built
 * with -std=c11 -ffp-contract=off, so a*b+c is two roundings unless the code
 * says fmaf(), exactly as the reference's gcc -std=c11 build behaves.
 */
#ifndef G4_ORACLE_H
#define G4_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Compile-time model shape (gemma4.c:26-31). */
enum {
    ORC_LAYERS = 35,
    ORC_HIDDEN = 1536,
    ORC_VOCAB = 262144,
    ORC_MAX_CONTEXT = 131072,
    ORC_WINDOW = 512,
    ORC_BATCH = 512,
    ORC_PLE = 256,          /* per-layer embedding width */
    ORC_HEADS = 8,          /* query heads; one KV head */
    ORC_SLIDING_RING = ORC_WINDOW + ORC_BATCH,
};

/* One 32-byte tensor record of the memory image (gemma4.c:119-123).
 * data/scales are host pointers (already fixed up from file offsets). */
typedef struct {
    void *data;
    uint16_t *scales;
    int32_t shape[4];
} orc_tensor;

/* Per-layer record block, field order of gemma4.c:125-145. */
typedef struct {
    orc_tensor input_layernorm, layer_scalar, pre_ffn_layernorm, post_attn_layernorm,
        post_ffn_layernorm, post_per_layer_input_norm, per_layer_input_gate,
        per_layer_projection, q_norm, k_norm, q_proj, k_proj, v_proj, o_proj, gate_proj,
        up_proj, down_proj, rope_cos, rope_sin;
} orc_layer;

/* Whole record table, field order of gemma4.c:147-155 (671 records). */
typedef struct {
    orc_tensor embed, embed_per_layer;
    orc_layer layers[ORC_LAYERS];
    orc_tensor norm, per_layer_model_projection, per_layer_projection_norm, gelu_table;
} orc_weights;

/* Activation scratch and fp32 KV caches (the buffers of gemma4.c:157-167). */
typedef struct orc_state orc_state;

orc_state *orc_state_new(void);
void orc_state_free(orc_state *s);
/* Zero the KV caches and activations (a fresh sequence). */
void orc_state_reset(orc_state *s);
/* Cache of the owner layer `layer` (0..14): returns the K half, V follows at
 * +cache_len*head_dim.  *cache_len / *head_dim receive the ring geometry. */
float *orc_state_cache(orc_state *s, int layer, int *cache_len, int *head_dim);
float *orc_state_residual(orc_state *s);
float *orc_state_hidden(orc_state *s);
/* gemma4.c:411-461: one layer's attention() over the state's first n hidden rows. */
void orc_attention_layer(const orc_weights *w, orc_state *s, int layer, int start_pos, size_t n);

/* Threads for the parallel entry points (0 = one per physical core, the rule of
 * gemma4.c:182-188; OMP_NUM_THREADS overrides as there). */
void orc_set_threads(int n);
int orc_threads(void);
/* 1 = VNNI fast matmul when the CPU has it (bit-identical), 0 = scalar only. */
void orc_set_fast(int on);
int orc_fast_available(void);

float orc_f16_to_f32(uint16_t h);

/* Kernels.  Each runs its own parallel team of orc_threads() threads. */
void orc_quantize(int8_t *q, float *scales, const float *x, size_t rows, size_t width);
void orc_matmul_int8(float *out, const int8_t *xq, const float *xs, const orc_tensor *w,
                     size_t rows);
void orc_attention_scores(float *scores, const float *query, const float *key_cache,
                          int first_key, int num_keys, int cache_mask, int head_dim);
void orc_softmax(float *values, int count);
void orc_weighted_value_sum(float *out, const float *p, const float *value_cache,
                            int first_key, int num_keys, int cache_mask, int head_dim);
void orc_geglu(float *gate, const float *up, int rows, int width, int up_stride,
               const orc_tensor *gelu_table);
void orc_embedding(float *out, const orc_tensor *table, const int *tokens, size_t n,
                   float multiplier);
void orc_rmsnorm(float *out, const float *in, const orc_tensor *weight, int width,
                 float epsilon, size_t rows);
void orc_add_and_scale(float *out, const float *add, size_t n, float scale);
void orc_apply_rope(const orc_tensor *cosines, const orc_tensor *sines, float *v,
                    int heads, int head_dim, int start_pos, size_t n);
/* The per-(head, token) loop of gemma4.c:443-456 over an explicit cache:
 * out[token*heads*hd + head*hd] from q laid out the same way. */
void orc_attend(float *out, const float *q, const float *key_cache, const float *value_cache,
                int cache_len, int head_dim, int heads, int full_attention, int start_pos,
                size_t n);

/* Transformer step (gemma4.c:463-509) and logits (gemma4.c:512-522). */
void orc_forward(const orc_weights *w, orc_state *s, const int *tokens, size_t n,
                 int start_pos);
/* Returns a pointer to VOCAB floats inside the state, valid until the next call. */
float *orc_logits(const orc_weights *w, orc_state *s, size_t row);

/* gemma4.c:527-561: sample() with the generator state (the reference's global
 * rng_state) passed in and advanced in place. */
int orc_sample(const float *logits, int vocab, float temperature, uint64_t *rng_state);

#ifdef __cplusplus
}
#endif
#endif
