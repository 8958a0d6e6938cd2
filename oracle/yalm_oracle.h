/*
 * CPU oracle for the fp16 batch-1 decode path -- TEST INFRASTRUCTURE ONLY.
 *
 * This library restates the reference's `-d cpu` forward pass (src/infer.cpp, src/model.h,
 * src/model.cpp, src/sampler.cpp of allbilly/yalm) so that the HIP path can be checked against
 * it. Only the test suite, the smoke check and the benchmark's CPU-baseline leg may load it.
 * The product (libyalm_hip.so, libyalm_host.so, the yalm binary) never links or calls it.
 *
 * Every function names the reference lines it follows. How each one is pinned (known answers,
 * closed forms, a float64 brute-force model) is written in the header comment of oracle.cpp.
 *
 * Conventions: activations fp32, weights fp16 (IEEE binary16 bit patterns in uint16_t) in
 * row-major (out, in) layout, KV caches fp16 in the reference's layout (model.h:14-17):
 *   K[g][ (j/16)*16*msl + t*16 + j%16 ],  V[g][ j*msl + t ]  for kv head g, dim j, position t.
 */
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
  int dim, hidden_dim, head_dim, n_layers, n_heads, n_kv_heads, vocab_size, max_seq_len, rotary_dim;
  float rope_theta, norm_eps, qkv_clip;
  int act; /* 0 = gelu, 1 = silu (model.h:19-22) */
} oracle_config;

typedef struct oracle_model oracle_model;

/* fp16 <-> fp32 with round-to-nearest-even (infer.cpp:10-16). */
float oracle_h2f(uint16_t h);
uint16_t oracle_f2h(float f);
void oracle_h2f_array(const uint16_t* in, float* out, size_t n);
void oracle_f2h_array(const float* in, uint16_t* out, size_t n);

/* Kernels (infer.cpp). Each is the reference function restated. */
void oracle_matmul_f16(float* xout, const float* x, const uint16_t* w, int n, int d); /* infer.cpp:63-100 */
void oracle_matmul_f32(float* xout, const float* x, const float* w, int n, int d);    /* infer.cpp:48-59 */
void oracle_rmsnorm(float* o, const float* x, const float* weight, int size, float eps); /* infer.cpp:136-146 */
void oracle_softmax(float* o, const float* x, int size);                             /* infer.cpp:172-187 */
float oracle_silu(float x);                                                          /* infer.cpp:193-195 */
float oracle_gelu(float x);                                                          /* infer.cpp:189-191 */
void oracle_rope(float* vec, int d, int head_dim, int pos, float theta, int rotary_dim); /* infer.cpp:202-215 */
int oracle_k_cache_idx(int hi, int t, int max_seq_len);                              /* model.h:15-17 */
void oracle_attn(float* xout, float* atth, const float* qh, const uint16_t* kh, const uint16_t* vh,
                 int head_dim, int n_kv_heads, int max_seq_len, int kv_len);         /* infer.cpp:218-250 */
void oracle_mha(float* xout, float* att, const uint16_t* kb, const uint16_t* vb, const float* q,
                int head_dim, int kv_len, int max_seq_len, int n_heads, int n_kv_heads); /* infer.cpp:394-415 */
void oracle_ffn(float* xout, const float* x, const uint16_t* w1, const uint16_t* w2, const uint16_t* w3,
                int hidden_dim, int dim, int act);                                   /* infer.cpp:424-455 (fp16 weights) */
int oracle_argmax(const float* logits, int n);                                       /* sampler.cpp:27-38 */
/* position math of infer.cpp:489-494: writes kv_sink, kv_pos, kv_len */
void oracle_positions(int pos, int max_seq_len, int* kv_sink, int* kv_pos, int* kv_len);

/* Whole-model forward (infer.cpp:256-392, 460-527). Weight pointers are borrowed, not copied. */
int oracle_create(const oracle_config* cfg, oracle_model** out);
void oracle_destroy(oracle_model* m);
int oracle_set_layer(oracle_model* m, int layer, const float* rms_att, const float* rms_ffn,
                     const uint16_t* wq, const uint16_t* wk, const uint16_t* wv, const uint16_t* wo,
                     const uint16_t* w1, const uint16_t* w2, const uint16_t* w3);
int oracle_set_globals(oracle_model* m, const uint16_t* embed, const float* rms_final, const uint16_t* wcls);
/* mode 0 = hydrate KV cache only, 1 = output logits (model.h:43-46). logits may be NULL in mode 0. */
int oracle_forward(oracle_model* m, int token, int pos, int mode, float* logits);
/* Direct pointers to layer `layer`'s K and V caches (n_kv_heads*head_dim*max_seq_len fp16 each). */
uint16_t* oracle_key_cache(oracle_model* m, int layer);
uint16_t* oracle_value_cache(oracle_model* m, int layer);
/* The fp32 residual stream x after the last forward (dim floats). */
const float* oracle_x(oracle_model* m);
/* Test hook: the model rotates with these head_dim / 2 frequencies instead of the reference's
 * 1 / powf(theta, j / rotary_dim) (n = 0 restores it). */
int oracle_set_rope_freqs(oracle_model* m, const float* freqs, int n);

#ifdef __cplusplus
}
#endif
