/*
 * yalm_host.h -- C-ABI of the host library (libyalm_host.so): a loaded model, its inference state
 * and sampler behind one opaque session, for callers that are not C++ (Python via ctypes).
 *
 * A session is the C++ `Model` + `InferenceState` + `Sampler` trio of the reference's decode driver
 * (src/main.cpp:121-211) with the model moved to the HIP device by yalm_session_hip().
 * All functions return 0 on success and -1 on failure; yalm_session_error() describes the failure.
 */
#ifndef YALM_HOST_H
#define YALM_HOST_H

#include <stddef.h>
#include <stdint.h>

#include "yalm_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct yalm_session yalm_session;

typedef struct {
  int dim, hidden_dim, head_dim, n_layers, n_heads, n_kv_heads, vocab_size, max_seq_len;
  float rope_theta, norm_eps, std;
  uint64_t seed;
  int tied_embeddings;
} yalm_synth_spec;

/* Opens a .yalm file (mmapped) and builds the Model (reference Model::Model, src/model.cpp:392-435);
 * context > 0 overrides max_seq_len like the reference -T flag. */
int yalm_session_open(const char* path, int context, yalm_session** out);
/* Builds a synthetic seeded random-init model in host memory (no file). */
int yalm_session_synthetic(const yalm_synth_spec* spec, int context, yalm_session** out);
/* Writes the session's checkpoint image as a .yalm file. */
int yalm_session_write(const yalm_session* s, const char* path);
/* Model::hip() + InferenceState::hip(): uploads the weights to device `device_ordinal`. */
int yalm_session_hip(yalm_session* s, int device_ordinal);
void yalm_session_close(yalm_session* s);
const char* yalm_session_error(const yalm_session* s);

/* The decode-relevant config (as the HIP context sees it). */
int yalm_session_config(const yalm_session* s, yhip_config* out);
/* Host tensor view by .yalm name: data pointer, byte size, dtype code (0 F32, 1 F16, ..., 8 U8)
 * and shape[4]. */
int yalm_session_tensor(const yalm_session* s, const char* name, const void** data, size_t* bytes, int* dtype,
                        int shape[4]);
/* The HIP context (after yalm_session_hip), e.g. for yhip_kv_write. */
yhip_ctx* yalm_session_hip_ctx(yalm_session* s);

/* Model::forward(state, token, pos, mode); logits (vocab floats) copied to `logits` when non-NULL
 * in YHIP_MODE_LOGITS. */
int yalm_session_forward(yalm_session* s, int token, int pos, int mode, float* logits);

/* Model::prefill(state, tokens, n, start_pos): the tokens in one batched pass; the last token's
 * logits (vocab floats) are copied to `logits` when non-NULL. No reference counterpart: the
 * reference hydrates a prompt one token at a time (src/main.cpp:169-177). */
int yalm_session_prefill(yalm_session* s, const int* tokens, int n, int start_pos, float* logits);

/* The reference completion loop (src/main.cpp:144-192) on token ids: warm-up forward(0, 0), prompt
 * hydrate (all but the last token in HYDRATE mode; one batched Model::prefill instead when
 * `batched_prefill` != 0), then n_steps x [sample -> forward]. Greedy when temperature == 0 (sampled
 * on the device when `device_argmax` != 0, else from host logits). Stops early at eos when
 * stop_at_eos != 0. Writes the generated ids to out_tokens[n_steps] and, per step, the wall time of
 * sample+forward in seconds to step_seconds[n_steps] (either may be NULL); *hydrate_seconds gets the
 * prompt time. Returns the number of generated tokens (>= 0) or -1. */
int yalm_session_generate(yalm_session* s, const int* prompt, int n_prompt, int n_steps, float temperature,
                          int device_argmax, int batched_prefill, int stop_at_eos, int* out_tokens,
                          double* step_seconds, double* hydrate_seconds);

/* Config::active_bytes(pos) of the reference (src/model.cpp:73-98). */
size_t yalm_session_active_bytes(const yalm_session* s, size_t pos);

/* Utilities shared with tests: seeded token ids and bit-exact fp16 conversion (RNE). */
void yalm_uniform_ids(int* out, size_t n, uint64_t seed, int hi);
void yalm_fill_normal_f16(uint16_t* out, size_t n, uint64_t seed, const char* stream_name, float std);
void yalm_f32_to_f16(const float* in, uint16_t* out, size_t n);
void yalm_f16_to_f32(const uint16_t* in, float* out, size_t n);

#ifdef __cplusplus
}
#endif
#endif /* YALM_HOST_H */
