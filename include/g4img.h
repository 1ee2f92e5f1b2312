/*
 * g4img.h -- the gemma4.c model image (".bin" written by exporter.py): layout
 * constants, a validating loader and a seeded synthetic-model writer.
 *
 * Layout (exporter.py:29-37, 42-70, 262-273, 304-367; gemma4.c:169-176):
 *   "MOG\0" | tokenizer block (33,429,932 B) | 671 tensor records (32 B each)
 *   | data from align64(4 + 33,429,932 + 55,008), every tensor 64-B aligned;
 *   a quantized matrix is its packed int8 tiles then its fp16 scales.
 */
#ifndef G4IMG_H
#define G4IMG_H

#include <stddef.h>
#include <stdint.h>

#include "g4.h"

#ifdef __cplusplus
extern "C" {
#endif

#define G4IMG_TOKENIZER_SPAN 33429932u
#define G4IMG_RECORDS_OFFSET (4u + G4IMG_TOKENIZER_SPAN) /* offsetof(Model, weights) */
#define G4IMG_TEXT_TENSOR_SPAN 55008u
#define G4IMG_DATA_START 33484992u

/* Record indices (the field order of gemma4.c:125-155). */
#define G4IMG_EMBED 0
#define G4IMG_EMBED_PER_LAYER 1
#define G4IMG_LAYER(l, field) (2 + (l) * 19 + (field))
#define G4IMG_NORM 667
#define G4IMG_PER_LAYER_MODEL_PROJECTION 668
#define G4IMG_PER_LAYER_PROJECTION_NORM 669
#define G4IMG_GELU_TABLE 670
enum {
    G4F_INPUT_LAYERNORM, G4F_LAYER_SCALAR, G4F_PRE_FFN_LAYERNORM, G4F_POST_ATTN_LAYERNORM,
    G4F_POST_FFN_LAYERNORM, G4F_POST_PER_LAYER_INPUT_NORM, G4F_PER_LAYER_INPUT_GATE,
    G4F_PER_LAYER_PROJECTION, G4F_Q_NORM, G4F_K_NORM, G4F_Q_PROJ, G4F_K_PROJ, G4F_V_PROJ,
    G4F_O_PROJ, G4F_GATE_PROJ, G4F_UP_PROJ, G4F_DOWN_PROJ, G4F_ROPE_COS, G4F_ROPE_SIN
};

/* Synthetic-model options. */
#define G4IMG_FFN_6144 1u   /* FFN width 6144 in every layer (E2B: 12288 in layers 15-34) */
#define G4IMG_UNIT_NORMS 2u /* norm weights and layer_scalar exactly 1.0 */
#define G4IMG_BF16_VALUES 4u /* every seeded value rounded to bfloat16 first: the image a
                                BF16 checkpoint of the same values exports to */

/* Bytes of the image for these options. */
size_t g4img_size(unsigned flags);

/* Write the whole image into buf (>= g4img_size(flags) bytes, 64-B aligned).
 * Matrices are N(0, 0.02) from a counter-based generator keyed by (seed,
 * record, 64-value group), quantized with the exporter's rule
 * (exporter.py:267-273); norm weights U[0.75, 1.25] and layer_scalar
 * U[0.9, 1.1] unless G4IMG_UNIT_NORMS; RoPE and GELU tables from the
 * exporter's formulas (exporter.py:73-92).  The result depends only on seed
 * and flags, not on thread count.  Returns 0, or -1 on bad arguments. */
int g4img_generate(void *buf, size_t size, uint64_t seed, unsigned flags, int threads);

/* Generate straight into a file (for the command-line host). */
int g4img_write_file(const char *path, uint64_t seed, unsigned flags, int threads);

/* Validate an image (magic, every record's data and scales inside the image,
 * shapes consistent with the packing) and write its records, with offsets
 * turned into pointers into `base`, to out[G4_RECORDS]; the image itself is
 * not modified.  Returns 0, or -1 with a message in g4img_last_error(). */
int g4img_records(const void *base, size_t size, g4_tensor *out);

/* The reference loader's in-place fix-up (gemma4.c:681-685), for hosts that
 * hand the image itself to code expecting a fixed-up Model. */
int g4img_fixup_inplace(void *base, size_t size);

/* ---- pieces for a checkpoint writer (gemma4.c_amd/export.py) ---- */

/* One distinct tensor of the image, in file order (shared RoPE tables appear
 * once, under the first record that uses them). */
typedef struct {
    int record;      /* first record that references it */
    int kind;        /* G4IMG_KIND_* */
    int rows, cols;  /* matrix shape; vectors cols = 1; tables (pos x pairs) or (4096 x 1) */
    int global_rope; /* RoPE tables: 1 for the global layers' */
    uint64_t data, scales; /* file offsets (scales 0 unless quantized) */
} g4img_item;
enum { G4IMG_KIND_QUANT, G4IMG_KIND_VECTOR, G4IMG_KIND_SCALAR, G4IMG_KIND_ROPE_COS,
       G4IMG_KIND_ROPE_SIN, G4IMG_KIND_GELU };
enum { G4IMG_F32, G4IMG_BF16, G4IMG_F16 }; /* source dtypes of g4img_pack_matrix */

/* The image's items (exporter.py:95-150's tensor() order and cursor walk) into
 * out[max_items]; returns the count (<= 700), or -1. */
int g4img_layout(unsigned flags, g4img_item *out, int max_items);

/* "MOG\0", a zero tokenizer block and the 671 records (file offsets) into the
 * first G4IMG_DATA_START bytes of buf. */
int g4img_write_header(void *buf, size_t size, unsigned flags);

/* A rows x cols row-major matrix (rows % 16 == 0, cols % 64 == 0) of dtype
 * G4IMG_F32/BF16/F16, quantized with the exporter's rule (exporter.py:267-273)
 * and packed into 16-row x 64-column tiles (exporter.py:304-316): data gets
 * rows * cols bytes, scales rows * cols / 64 fp16.  -1 if a value is NaN/inf. */
int g4img_pack_matrix(const void *src, int dtype, int rows, int cols, void *data, void *scales,
                      int threads);

/* A RoPE or GELU table item's values (exporter.py:73-92) at base + it->data. */
int g4img_fill_table(void *base, size_t size, const g4img_item *it, int threads);

/* The synthetic generator's values of a matrix or vector item before
 * quantization, row-major (rows * cols values) as G4IMG_F32 or -- with
 * G4IMG_BF16_VALUES -- G4IMG_BF16: what g4img_generate quantizes for it.  For
 * fabricating a checkpoint that must export to the synthetic image. */
int g4img_draw(uint64_t seed, unsigned flags, const g4img_item *it, void *out, int dtype, int threads);

const char *g4img_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
