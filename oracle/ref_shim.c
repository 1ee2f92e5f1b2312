/*
 * ref_shim.c -- builds the reference's own gemma4.c, unmodified, into a shared
 * library for the parity tests (TEST INFRASTRUCTURE ONLY).
 *
 * The reference source is #included from where it lies (-I points at the
 * reference checkout; nothing is copied).  Its main() is renamed so the file
 * links as a library; every kernel keeps its external linkage, so ctypes can
 * call quantize(), matmul_int8(), attention(), forward() and logits() directly.
 * The helpers below only report the layout of the reference's InferenceState so
 * a harness can allocate one and find its KV caches.
 */
#define main gemma4_reference_main
#include "gemma4.c"
#undef main

size_t ref_state_size(void) { return sizeof(InferenceState); }
size_t ref_off_residual(void) { return offsetof(InferenceState, residual); }
size_t ref_off_hidden(void) { return offsetof(InferenceState, hidden); }
size_t ref_off_auxiliary(void) { return offsetof(InferenceState, auxiliary); }
size_t ref_off_sliding(void) { return offsetof(InferenceState, sliding_cache); }
size_t ref_off_full(void) { return offsetof(InferenceState, full_cache); }
size_t ref_model_weights_offset(void) { return offsetof(Model, weights); }
size_t ref_model_size(void) { return sizeof(Model); }
int ref_thread_count(void) { return thread_count(); }
