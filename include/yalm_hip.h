/*
 * yalm_hip.h -- C-ABI of the MI355X (gfx950) fp16 batch-1 decode path.
 *
 * This is the drop-in boundary behind the reference's C++ model API (allbilly/yalm):
 * a host `Model`/`InferenceState` pair moved to `Device::HIP` owns one `yhip_ctx` and calls
 * `yhip_forward` from `Model::forward`. Plain C types only: no HIP, torch or C++ types cross it.
 *
 * Conventions
 *   - fp16 values travel as IEEE binary16 bit patterns in uint16_t.
 *   - Weight matrices are row-major (out, in), exactly as stored in a .yalm file.
 *   - KV caches use the reference layout (src/model.h:14-17, 266-268), per layer and kv head g:
 *       K[g*hd*msl + (j/16)*16*msl + t*16 + j%16],   V[g*hd*msl + j*msl + t].
 *   - Every entry point returns 0 on success and a negative code on failure; the library never
 *     aborts. yhip_last_error() then describes the failure (thread-local for calls without a ctx).
 *   - One context belongs to one host thread; all its work runs on the context's own stream.
 *     Contexts on the same device are independent.
 */
#ifndef YALM_HIP_H
#define YALM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define YHIP_OK 0
#define YHIP_EINVAL (-1)   /* bad argument or unsupported shape */
#define YHIP_EDEVICE (-2)  /* HIP runtime error */
#define YHIP_ESTATE (-3)   /* missing upload or wrong call order */

#define YHIP_MODE_HYDRATE 0 /* InferenceMode::HYDRATE_KV_CACHE (src/model.h:43-46) */
#define YHIP_MODE_LOGITS 1  /* InferenceMode::OUTPUT_LOGITS */

#define YHIP_ACT_GELU 0
#define YHIP_ACT_SILU 1

/* Launch structure of one decode step (yhip_step_plan). */
#define YHIP_STEP_SEPARATE 0 /* QKV, attention, O + residual, W1/W3, W2: each its own launch */
#define YHIP_STEP_ATTN_O 1   /* attention and O in one launch (each workgroup repeats its kv head's attention) */
#define YHIP_STEP_SPLIT_O 2  /* split-KV attention storing every slice's partial; the O launch merges them */
#define YHIP_STEP_SINGLE 3   /* the whole step as one launch (option "single_launch") */

typedef struct yhip_ctx yhip_ctx;

/* Mirrors the decode-relevant fields of the reference Config (src/model.h:56-82). */
typedef struct {
  int dim, hidden_dim, head_dim, n_layers, n_heads, n_kv_heads, vocab_size, max_seq_len, rotary_dim;
  float rope_theta, norm_eps, qkv_clip;
  int act; /* YHIP_ACT_* */
} yhip_config;

/* Context: device memory for weights, KV caches (zeroed) and activations, one stream.
 * Replaces Model::cuda() + InferenceState::cuda() (src/model.cpp:342-361, 437-451) and the
 * device-memory ABI upload_cuda/register_cuda_host/set_cuda_device/init_cuda_stream
 * (src/model.h:48-54, src/infer.cu:60-91). */
int yhip_create(const yhip_config* cfg, int device_ordinal, yhip_ctx** out);
int yhip_destroy(yhip_ctx* ctx);

/* Weight upload (host -> HBM), replaces Block::cuda() (src/model.cpp:217-241) and its
 * upload_cuda copies (src/infer.cu:34-39). The sources may be pageable (e.g. an mmapped .yalm):
 * large tensors move through pinned staging chunks (option "upload_stage_mb"). Returns after the
 * copies have completed, so the caller may release the host memory.
 * Shapes: rms_* [dim] fp32; wq [n_heads*hd][dim]; wk, wv [n_kv_heads*hd][dim]; wo [dim][n_heads*hd];
 * w1, w3 [hidden][dim]; w2 [dim][hidden]. */
int yhip_upload_layer(yhip_ctx* ctx, int layer, const float* rms_att, const float* rms_ffn,
                      const uint16_t* wq, const uint16_t* wk, const uint16_t* wv, const uint16_t* wo,
                      const uint16_t* w1, const uint16_t* w2, const uint16_t* w3);
/* embed [vocab][dim]; rms_final [dim]; wcls [vocab][dim] or NULL for a tied lm_head
 * (src/model.cpp:425-434). Replaces the global part of Model::cuda(). */
int yhip_upload_globals(yhip_ctx* ctx, const uint16_t* embed, const float* rms_final, const uint16_t* wcls);

/* One decode step: Model::forward(s, token, pos, mode) (src/model.cpp:479-494,
 * src/infer.cu:1274-1294). Writes K/V of `pos` into every layer's cache. In YHIP_MODE_LOGITS it
 * returns after `logits_host` [vocab] holds the next-token logits; in YHIP_MODE_HYDRATE it may
 * return before the device finishes (stream order keeps later calls correct) and logits_host is
 * ignored. `logits_host` may be the pointer from yhip_logits_host() (no extra host copy). */
int yhip_forward(yhip_ctx* ctx, int token, int pos, int mode, float* logits_host);

/* Greedy decode step: like yhip_forward(LOGITS) but returns only the argmax token id computed on
 * the device with the reference tie rule (src/sampler.cpp:27-38). */
int yhip_forward_argmax(yhip_ctx* ctx, int token, int pos, int* next_token);

/* Batched prompt prefill: tokens[0..n) at positions start_pos .. start_pos+n-1 go through every
 * layer together (MFMA GEMMs with fused epilogues, causal MFMA attention) and their K/V land in the
 * caches, as n calls of yhip_forward(YHIP_MODE_HYDRATE) would leave them (src/main.cpp:169-177,
 * src/infer.cpp:256-392). If logits_host is not NULL the call returns after it holds the last
 * token's logits; otherwise it may return before the device finishes. Ring positions
 * (start_pos + n > max_seq_len) and shapes without the batched kernels (head_dim not 32/64/128;
 * dim, hidden_dim, n_heads*head_dim or max_seq_len not a multiple of 32) run token by token.
 * No reference counterpart: the reference hydrates one token per forward. */
int yhip_prefill(yhip_ctx* ctx, const int* tokens, int n, int start_pos, float* logits_host);

/* Pinned host buffer [vocab] that yhip_forward fills without an extra copy when passed back. */
float* yhip_logits_host(yhip_ctx* ctx);

/* KV cache copies in the reference layout (n_kv_heads*hd*max_seq_len fp16 each). */
int yhip_kv_read(yhip_ctx* ctx, int layer, uint16_t* k_host, uint16_t* v_host);
int yhip_kv_write(yhip_ctx* ctx, int layer, const uint16_t* k_host, const uint16_t* v_host);

/* Fills every layer's K and V cache with fp16 draws of N(0, 1) (a counter hash of `seed` and the
 * element index) at positions below n_positions and zeros above, on the device: the set-up of the
 * attention-heavy workload (a KV cache pre-filled to 16384 positions). No reference counterpart. */
int yhip_kv_fill_normal(yhip_ctx* ctx, int n_positions, unsigned long long seed);

/* Options: "single_launch" (1 = the whole step as one cooperative launch, one workgroup per CU
 * walking the step's phases with a grid barrier between them, where the kernel has an
 * instantiation: head_dim 128 with 4 q heads per kv head, and the test shapes, on at most 256 CUs;
 * 0 = per-op kernels, the default), "step_atto_max" (single launch: attention and the O projection
 * as one phase for steps with at most this many cached tokens, below max_seq_len, default 192;
 * 0 = always two phases), "step_spin_limit" (single launch: polls before a grid barrier wait gives
 * up and the step fails with YHIP_EDEVICE; 0 = the default, about a second; small values exercise
 * that error path), "graph" (per-op kernels: 1 = replay
 * a captured hipGraph per step, default; 0 = direct launches), "attn_splits" (most KV slices per
 * kv head, default 7/8 of compute units / n_kv_heads clamped to [1,64]),
 * "attn_min_slice" (fewest tokens per KV slice, a multiple of 64; 0 = the kernel's default: for
 * the MFMA attention one slice up to 320 cached tokens, then 64 up to 2048, 128 up to 6144 and 384
 * beyond; 64 for the SIMT one; a set floor, and the SIMT one's, at least 128 from 1024 cached
 * tokens on), "attn_mfma" (1 = decode
 * attention on the matrix cores where head_dim % 32 == 0 and max_seq_len % 32 == 0, default;
 * 0 = the SIMT kernel), "bpc_qkv" / "bpc_o" / "bpc_w13" / "bpc_w2" / "bpc_lm" (workgroups per CU
 * of the decode matvecs, 0..16; 0 = the default: 2 for QKV, O and the lm_head, 12 for W1/W3, 1 for
 * W2; the results do not depend on it), "stats" (1 = time every synchronised step on the device
 * with HIP events and reset the totals; 0 = off), "attn_o" (1 = default: for steps with at most
 * "attn_o_max" cached tokens (default 512), below max_seq_len, on the matrix-core attention's
 * shapes with at most 8 kv heads, attention and the O projection run in one launch whose
 * workgroups each repeat their kv head's attention and combine their rows of Wo . attention in
 * per-row integer words, bit-reproducibly; 0 = separate launches), "split_o" (1 = default: beyond
 * that, the split-KV attention stores every slice's partial and the O launch merges them, with at
 * most 32 slices per kv head; 0 = the attention launch merges its own slices). The results of
 * every option setting agree to fp32 rounding; each is tested against the CPU reference. With
 * ctx == NULL it sets process-wide options: "test_bpc" (workgroups per CU used by the yhip_test_*
 * hooks; 0 = the decode path's default), "attn_mfma" (attention kernel of the yhip_test_* /
 * yhip_bench_* hooks, as above), "gemm_stages" / "gemm_bk" / "gemm_bm" / "gemm_ksplit" (prefill
 * GEMM variant: stages -1 = chosen per shape (default), 2..4 = the LDS pipeline's depth (4 with
 * 32-deep k-steps, 2 or 3 with 64-deep ones), 6 = the eight-wave 256 x 256 kernel; k-step 32 or
 * 64; workgroup rows 128 or 256; K splits of the LDS pipeline, 0 = per shape), "gemm_ppsplit" (1 =
 * default: the eight-wave kernel splits its last, partial round of tiles along K where that pays;
 * 0 = whole tiles only), "upload_stage_mb" (yhip_upload_layer / yhip_upload_globals copy tensors
 * of 64 KB and more through a ring of three pinned staging chunks of this many MB, default 64;
 * 0 = direct copies from the caller's pageable memory as the reference's upload_cuda,
 * src/infer.cu:34-39) and "upload_threads" (host threads filling a staging chunk, default 8). */
int yhip_set_option(yhip_ctx* ctx, const char* key, int value);

/* The launch plan of the decode step at `pos` under the context's current options: *variant one
 * of YHIP_STEP_*, *slices the KV slices per kv head that hold keys and *slice_len their length in
 * keys (YHIP_STEP_ATTN_O, and YHIP_STEP_SINGLE with attention and O as one phase: 1 and the
 * context length, every workgroup attends to the whole context). Any output may be NULL. No
 * reference counterpart (a test and diagnostics hook). */
int yhip_step_plan(yhip_ctx* ctx, int pos, int* variant, int* slices, int* slice_len);

/* Device time of the steps timed since "stats" was set: total microseconds between HIP events
 * recorded on the context's stream around each LOGITS/argmax step's kernels, and the step count.
 * No reference counterpart (the reference times whole steps on the host, src/main.cpp:195-210). */
int yhip_step_stats(const yhip_ctx* ctx, double* us_total, int* steps);

/* Debug read of a device activation after the last forward: which = 0 x [dim], 1 q [nh*hd],
 * 2 attention output [nh*hd], 3 hb [hidden], 4 logits [vocab]; 5 the rotary frequencies the
 * step uses [head_dim / 2] (fp32, 1 / powf(theta, j / rotary_dim) rounded on the host). Mirrors the reference's
 * DEBUG_MODEL tensor dumps (src/infer.cu:93-109). */
int yhip_debug_read(yhip_ctx* ctx, int which, float* host, size_t n);

const char* yhip_last_error(const yhip_ctx* ctx);

/* ---- kernel-level hooks, mirroring matmul_cuda / mha_cuda / ffn_cuda (src/model.h:328-374).
 * Host pointers in and out; each call allocates device buffers, launches, syncs and frees. ---- */

/* out[d] = W[d][n] . xn, where xn = rmsnorm(x, gain, eps) if gain != NULL else x
 * (src/infer.cpp:63-100 and 136-146). If resid != NULL, out = resid + W.xn. */
int yhip_test_matvec(const float* x, const float* gain, float eps, const uint16_t* w, int n, int d,
                     const float* resid, float* out);
/* Gated FFN with fused pre-norm: hb = act(W1 xn) * (W3 xn); out = resid + W2 hb (resid may be
 * NULL -> out = W2 hb). gain NULL disables the norm (src/infer.cpp:346-391, 424-455). */
int yhip_test_ffn(const float* x, const float* gain, float eps, const uint16_t* w1, const uint16_t* w2,
                  const uint16_t* w3, int hidden_dim, int dim, int act, const float* resid, float* out);
/* GQA attention over reference-layout caches (src/infer.cpp:218-250, 394-415); `nsplit` KV slices
 * per kv head of at least 64 keys, or 0 = the decode step's own slice plan (7/8 of the compute
 * units over the kv heads; the MFMA kernel's length rule, as option "attn_min_slice" 0).
 * The slices are merged inside the launch (the decode step beyond 512 keys defers that merge to
 * its O launch instead). att_out [n_heads*hd]. pos >= max_seq_len exercises sink rotation, which
 * rewrites kcache (the updated K cache is copied back). kv_len is derived from pos. */
int yhip_test_attention(const float* q, uint16_t* kcache, const uint16_t* vcache, int head_dim, int pos,
                        int max_seq_len, int n_heads, int n_kv_heads, int nsplit, float rope_theta,
                        int rotary_dim, float* att_out);
/* yhip_test_attention without any allocation, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference. q, kcache, vcache and att_out are DEVICE pointers (layouts as in
 * yhip_test_attention; kcache is rewritten in sink mode, pos >= max_seq_len); the work is enqueued
 * on `stream` (a hipStream_t, NULL = the default stream) and the call returns without waiting.
 * The split-KV partials, tickets, step parameters and rotary frequencies live in a fixed device
 * array of the library (1 MiB of partials + 4 KiB, one per GPU, held until the process ends): the
 * call fails with YHIP_EINVAL when n_heads * nsplit * (head_dim + 2) floats exceed 1 MiB (nsplit 0 =
 * the default, as yhip_test_attention). Every call on a GPU shares that array, so calls that
 * overlap on one GPU (other streams, other threads) race; calls in order on one stream do not. */
int yhip_attention_noalloc(const float* q, uint16_t* kcache, const uint16_t* vcache, int head_dim, int pos,
                           int max_seq_len, int n_heads, int n_kv_heads, int nsplit, float rope_theta,
                           int rotary_dim, float* att_out, void* stream);
/* Fused pre-norm + QKV matvec + clip + RoPE + KV-cache write (src/infer.cpp:267-305).
 * q_out [nh*hd]; kcache/vcache [n_kv*hd*msl] updated in place at kv_pos(pos). */
int yhip_test_qkv(const float* x, const float* gain, float eps, const uint16_t* wq, const uint16_t* wk,
                  const uint16_t* wv, int dim, int n_heads, int n_kv_heads, int head_dim, int max_seq_len,
                  int rotary_dim, float rope_theta, float qkv_clip, int pos, float* q_out, uint16_t* kcache,
                  uint16_t* vcache);
/* The prefill GEMM: A [M][K], B and B3 [N][K] fp16, K a multiple of 32. mode 0: c = A B^T;
 * mode 1: c += A B^T (c holds the addend on entry); mode 2: h = fp16(act(A B^T) * (A B3^T)) with
 * act 1 silu, 0 gelu (the SwiGLU of src/infer.cpp:362-382). c [M][N] fp32, h [M][N] fp16. */
int yhip_test_gemm(const uint16_t* a, const uint16_t* b, const uint16_t* b3, int M, int N, int K, int mode, int act,
                   float* c, uint16_t* h);
/* The prefill GEMM variant yhip_prefill runs for this shape and mode (as yhip_test_gemm), under the
 * current process-wide options: stages 6 = the eight-wave 256 x 256 kernel, 2..4 = the LDS
 * pipeline's depth; bk the k-step; bm the workgroup's rows. No
 * reference counterpart (the reference has no batched prefill). */
int yhip_gemm_variant(int M, int N, int K, int mode, int* stages, int* bk, int* bm);
/* Greedy argmax on the device with the reference tie rule. */
int yhip_test_argmax(const float* logits, int n, int* out);

/* ---- microbenchmark: one fused decode kernel at a given shape, weights rotated over `copies`
 * device-resident copies (to keep the 256 MB last-level cache from serving them), timed with HIP
 * events on the launching stream. kind: 0 = rmsnorm+QKV+RoPE (rows = q+k+v dims, head_dim 128: 8 kv
 * heads from 2048 rows on, one below, e.g. 768 = one kv head's share of an 8-way split), 1 = O-proj +
 * residual, 2 = rmsnorm + W1/W3 + SwiGLU, 3 = W2 + residual (row pairs below 8192 columns, even
 * rows), 4 = rmsnorm + lm_head, 5 = plain
 * device copy of rows*cols fp16 (the reference point for hardware byte counters).
 * blocks_per_cu caps the grid at blocks_per_cu x CUs workgroups (0 = the decode path's default).
 * Writes the mean kernel time in microseconds. ---- */
int yhip_bench_kernel(int kind, int rows, int cols, int copies, int warmup, int reps, int blocks_per_cu,
                      float* us_per_launch);

/* Memory-only ceiling of one decode step at this config: its weight bytes read by pure streaming
 * launches in the order and sizes of the decode launches (per layer [Wq;Wk;Wv], Wo, W1 and W3,
 * W2; then the lm_head; every launch over fresh memory, the matvecs' access pattern), and the
 * same bytes as one launch. Writes milliseconds per token for both. Needs device memory for one
 * copy of the weights. No reference counterpart (a measurement hook). */
int yhip_bench_stream(const yhip_config* cfg, int reps, float* ms_launches, float* ms_one_launch);

/* Times one prefill GEMM launch (mode as yhip_test_gemm) on device-filled operands: average
 * microseconds over `reps` launches after `warmup`, with HIP events on a private stream. No
 * reference counterpart (the reference has no batched prefill). */
int yhip_bench_gemm(int M, int N, int K, int mode, int warmup, int reps, float* us_per_launch);

/* ---- microbenchmark of the split-KV attention kernel over `copies` rotating KV caches (random
 * fp16), at position kv_len - 1, `nsplit` slices of at least `min_slice` tokens, or nsplit 0 = the
 * decode step's own slice plan (as yhip_test_attention). Mean microseconds. */
int yhip_bench_attention(int head_dim, int n_heads, int n_kv_heads, int max_seq_len, int kv_len, int nsplit,
                         int min_slice, int copies, int warmup, int reps, float* us_per_launch);

#ifdef __cplusplus
}
#endif
#endif /* YALM_HIP_H */
