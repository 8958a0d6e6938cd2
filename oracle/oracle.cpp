/*
 * CPU oracle: restatement of the reference `-d cpu` decode path -- TEST INFRASTRUCTURE ONLY.
 *
 * Loaded only by tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg, as the reference
 * that results are compared against.
 * Built like the reference CPU path (Makefile:32-36 of the reference): -O3 -ffast-math -fopenmp
 * -mf16c -mavx2 -mfma.
 *
 * What the reference's own build cannot give us: src/model.h:4 includes cuda_runtime_api.h and
 * the link needs symbols defined only in .cu files, so src/infer.cpp is not buildable in this
 * image. This file therefore restates it, function by function, with the same arithmetic order
 * (16-wide two-accumulator F16C matvec with the same horizontal reduction, sequential fp32
 * rmsnorm/softmax loops, fp32 powf/cosf/sinf RoPE, RNE fp16 stores).
 *
 * How each function is pinned (tests/test_oracle.py):
 *   - oracle_attn / oracle_mha: the reference's known-answer test (test.cpp:67-125), the
 *     kv_len = 1 closed form (output = V[:,0]), and a float64 NumPy evaluation.
 *   - oracle_matmul_f16/f32: one-hot x returns a column of W exactly; float64 NumPy dot.
 *   - oracle_rmsnorm: constant-vector closed form sign(c)/sqrt(1+eps/c^2); float64 NumPy.
 *   - oracle_rope: identity at pos 0, pair-norm preservation, RoPE(a) o RoPE(b) = RoPE(a+b),
 *     and float64 NumPy.
 *   - oracle_softmax: sums to one, shift invariance, float64 NumPy.
 *   - oracle_silu / oracle_gelu: float64 NumPy of the textbook formulas.
 *   - oracle_h2f / oracle_f2h: NumPy float16 conversion (IEEE RNE) over all 65536 bit patterns
 *     and random floats.
 *   - oracle_k_cache_idx / oracle_positions: brute-force enumeration of the closed forms.
 *   - oracle_argmax: first-index tie rule cases.
 *   - oracle_forward: float64 NumPy brute-force model of the whole forward pass (tiny shapes,
 *     tests/npref.py), compared on logits and on the KV caches.
 * The exact fp32 summation order that the reference's -ffast-math build produced and glibc's
 * powf/cosf/sinf/expf ulp behaviour are pinned only to tolerance (logits rel-L2 <= 1e-2 is the
 * contract); no bit-exact claim depends on them.
 */
#include "yalm_oracle.h"

#include <cfloat>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <immintrin.h>
#include <new>
#include <vector>

// ---------------------------------------------------------------------------------------------
// fp16 conversion: hardware F16C, round-to-nearest-even (infer.cpp:10-16: _cvtsh_ss/_cvtss_sh(x,0))
// ---------------------------------------------------------------------------------------------
extern "C" float oracle_h2f(uint16_t h) { return _cvtsh_ss(h); }
extern "C" uint16_t oracle_f2h(float f) { return (uint16_t)_cvtss_sh(f, 0); }

extern "C" void oracle_h2f_array(const uint16_t* in, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = _cvtsh_ss(in[i]);
}
extern "C" void oracle_f2h_array(const float* in, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = (uint16_t)_cvtss_sh(in[i], 0);
}

// ---------------------------------------------------------------------------------------------
// matvec (infer.cpp:48-59 fp32, infer.cpp:63-100 fp16): W (d, n) row-major times x (n) -> (d)
// ---------------------------------------------------------------------------------------------
extern "C" void oracle_matmul_f32(float* xout, const float* x, const float* w, int n, int d) {
  int i;
#pragma omp parallel for private(i)
  for (i = 0; i < d; i++) {
    float acc = 0.0f;
    const float* row = w + (size_t)i * n;
    for (int j = 0; j < n; j++) acc += row[j] * x[j];
    xout[i] = acc;
  }
}

// Same accumulation structure as the reference: per 16 columns, the low 8 and the high 8
// products go to two 8-lane FMA accumulators; at the end the two are added lane-wise, the
// upper 4 lanes are folded onto the lower 4, and the 4 lanes are summed with DPPS.
static inline float dot_f16_row(const uint16_t* row, const float* x, int n) {
  __m256 acc_a = _mm256_setzero_ps();
  __m256 acc_b = _mm256_setzero_ps();
  for (int j = 0; j < n; j += 16) {
    __m256i h16 = _mm256_loadu_si256(reinterpret_cast<const __m256i*>(row + j));
    __m256 wa = _mm256_cvtph_ps(_mm256_castsi256_si128(h16));
    __m256 wb = _mm256_cvtph_ps(_mm256_extractf128_si256(h16, 1));
    acc_a = _mm256_fmadd_ps(wa, _mm256_loadu_ps(x + j), acc_a);
    acc_b = _mm256_fmadd_ps(wb, _mm256_loadu_ps(x + j + 8), acc_b);
  }
  __m256 s8 = _mm256_add_ps(acc_a, acc_b);
  __m128 s4 = _mm_add_ps(_mm256_castps256_ps128(s8), _mm256_extractf128_ps(s8, 1));
  return _mm_cvtss_f32(_mm_dp_ps(s4, _mm_set1_ps(1.0f), 0xf1));
}

extern "C" void oracle_matmul_f16(float* xout, const float* x, const uint16_t* w, int n, int d) {
  if (n % 16 != 0) {  // infer.cpp:66 asserts this
    std::abort();
  }
  int i;
#pragma omp parallel for private(i)
  for (i = 0; i < d; i++) xout[i] = dot_f16_row(w + (size_t)i * n, x, n);
}

// ---------------------------------------------------------------------------------------------
// rmsnorm (infer.cpp:136-146), softmax (172-187), silu (193-195), gelu (189-191), clip (197-199)
// ---------------------------------------------------------------------------------------------
extern "C" void oracle_rmsnorm(float* o, const float* x, const float* weight, int size, float eps) {
  float ss = 0.0f;
  for (int i = 0; i < size; ++i) ss += x[i] * x[i];
  float inv = 1.0f / sqrtf(ss / size + eps);
  for (int i = 0; i < size; ++i) o[i] = x[i] * inv * weight[i];
}

extern "C" void oracle_softmax(float* o, const float* x, int size) {
  float mx = -FLT_MAX;
  for (int i = 0; i < size; ++i) mx = x[i] > mx ? x[i] : mx;
  float sum = 0.0f;
  for (int i = 0; i < size; ++i) {
    o[i] = expf(x[i] - mx);
    sum += o[i];
  }
  for (int i = 0; i < size; ++i) o[i] /= sum;
}

extern "C" float oracle_silu(float x) { return x / (1.0f + expf(-x)); }
extern "C" float oracle_gelu(float x) {
  return 0.5f * x * (1.0f + tanhf(0.797885f * (x + 0.044715f * x * x * x)));
}
static inline float clampf(float x, float v) { return x < -v ? -v : (x > v ? v : x); }

// ---------------------------------------------------------------------------------------------
// RoPE on interleaved pairs (infer.cpp:202-215)
// ---------------------------------------------------------------------------------------------
extern "C" void oracle_rope(float* vec, int d, int head_dim, int pos, float theta, int rotary_dim) {
  for (int i = 0; i < d; i += 2) {
    int j = i % head_dim;
    float freq = j >= rotary_dim ? 0.0f : 1.0f / powf(theta, (float)j / (float)rotary_dim);
    float ang = pos * freq;
    float c = cosf(ang), s = sinf(ang);
    float a = vec[i], b = vec[i + 1];
    vec[i] = a * c - b * s;
    vec[i + 1] = a * s + b * c;
  }
}

// ---------------------------------------------------------------------------------------------
// KV cache layout (model.h:12-17) and position math (infer.cpp:489-494)
// ---------------------------------------------------------------------------------------------
static const int kKvSinks = 2;  // model.h:12

extern "C" int oracle_k_cache_idx(int hi, int t, int max_seq_len) {
  return (hi / 16) * (16 * max_seq_len) + t * 16 + (hi % 16);
}

extern "C" void oracle_positions(int pos, int max_seq_len, int* kv_sink, int* kv_pos, int* kv_len) {
  int sink = pos >= max_seq_len ? kKvSinks : 0;
  *kv_sink = sink;
  *kv_pos = sink + (pos - sink) % (max_seq_len - sink);
  *kv_len = pos >= max_seq_len ? max_seq_len : pos + 1;
}

// ---------------------------------------------------------------------------------------------
// Attention for one query head over one kv head's cache slice (infer.cpp:218-250)
// ---------------------------------------------------------------------------------------------
extern "C" void oracle_attn(float* xout, float* atth, const float* qh, const uint16_t* kh, const uint16_t* vh,
                            int head_dim, int n_kv_heads, int max_seq_len, int kv_len) {
  (void)n_kv_heads;
  for (int t = 0; t < kv_len; ++t) {
    float s = 0.0f;
    for (int i = 0; i < head_dim; ++i) s += qh[i] * _cvtsh_ss(kh[oracle_k_cache_idx(i, t, max_seq_len)]);
    s /= sqrtf((float)head_dim);
    atth[t] = s;
  }
  oracle_softmax(atth, atth, kv_len);
  for (int i = 0; i < head_dim; ++i) {
    float acc = 0.0f;
    const uint16_t* vrow = vh + (size_t)i * max_seq_len;
    for (int t = 0; t < kv_len; ++t) acc += atth[t] * _cvtsh_ss(vrow[t]);
    xout[i] = acc;
  }
}

// GQA over all query heads (infer.cpp:394-415 and the head loop at 327-336)
extern "C" void oracle_mha(float* xout, float* att, const uint16_t* kb, const uint16_t* vb, const float* q,
                           int head_dim, int kv_len, int max_seq_len, int n_heads, int n_kv_heads) {
  int group = n_heads / n_kv_heads;
  int h;
#pragma omp parallel for private(h)
  for (h = 0; h < n_heads; h++) {
    int g = h / group;
    size_t off = (size_t)g * head_dim * max_seq_len;
    oracle_attn(xout + (size_t)head_dim * h, att + (size_t)max_seq_len * h, q + (size_t)head_dim * h,
                kb + off, vb + off, head_dim, n_kv_heads, max_seq_len, kv_len);
  }
}

static inline float act_fn(float x, int act) { return act == 1 ? oracle_silu(x) : oracle_gelu(x); }

// Gated FFN with fp16 weights (infer.cpp:424-455, restated for f16 weights as the path uses them)
extern "C" void oracle_ffn(float* xout, const float* x, const uint16_t* w1, const uint16_t* w2, const uint16_t* w3,
                           int hidden_dim, int dim, int act) {
  std::vector<float> hb(hidden_dim), hb2(hidden_dim);
  oracle_matmul_f16(hb.data(), x, w1, dim, hidden_dim);
  oracle_matmul_f16(hb2.data(), x, w3, dim, hidden_dim);
  for (int i = 0; i < hidden_dim; ++i) hb[i] = act_fn(hb[i], act) * hb2[i];
  oracle_matmul_f16(xout, hb.data(), w2, hidden_dim, dim);
}

// Greedy sampling: first index of the strict maximum (sampler.cpp:27-38)
extern "C" int oracle_argmax(const float* logits, int n) {
  int best = 0;
  float mx = -FLT_MAX;
  for (int i = 0; i < n; ++i) {
    if (logits[i] > mx) {
      mx = logits[i];
      best = i;
    }
  }
  return best;
}

// ---------------------------------------------------------------------------------------------
// Whole model (model.cpp:130-205, 291-307, 392-435; infer.cpp:256-392, 460-527)
// ---------------------------------------------------------------------------------------------
struct OracleLayer {
  const float* rms_att = nullptr;
  const float* rms_ffn = nullptr;
  const uint16_t *wq = nullptr, *wk = nullptr, *wv = nullptr, *wo = nullptr;
  const uint16_t *w1 = nullptr, *w2 = nullptr, *w3 = nullptr;
  std::vector<uint16_t> kcache, vcache;  // zero-initialised (model.cpp:203-204)
};

struct oracle_model {
  oracle_config c;
  std::vector<OracleLayer> layers;
  const uint16_t* embed = nullptr;
  const float* rms_final = nullptr;
  const uint16_t* wcls = nullptr;
  // InferenceState workspace (model.cpp:291-307)
  std::vector<float> x, xb, xb2, hb, hb2, q, k, v, att;
  // Rotary frequencies set from outside (oracle_set_rope_freqs), one per pair of a head; empty:
  // each rotation computes them as the reference does (infer.cpp:205)
  std::vector<float> rope_freqs;
};

// The model's RoPE: oracle_rope, or the same rotation with the frequencies set from outside.
static void model_rope(const oracle_model* m, float* vec, int d, int pos) {
  const oracle_config& c = m->c;
  if (m->rope_freqs.empty()) {
    oracle_rope(vec, d, c.head_dim, pos, c.rope_theta, c.rotary_dim);
    return;
  }
  for (int i = 0; i < d; i += 2) {
    float ang = pos * m->rope_freqs[(i % c.head_dim) / 2];
    float cs = cosf(ang), sn = sinf(ang);
    float a = vec[i], b = vec[i + 1];
    vec[i] = a * cs - b * sn;
    vec[i + 1] = a * sn + b * cs;
  }
}

// Test hook: rotate with these frequencies (head_dim / 2 of them) instead of the reference's
// 1 / powf(theta, j / rotary_dim), which a -ffast-math build may round an ulp away from the
// correctly rounded value. n = 0 restores the reference's expression.
extern "C" int oracle_set_rope_freqs(oracle_model* m, const float* freqs, int n) {
  if (!m || n < 0 || (n > 0 && (!freqs || n != m->c.head_dim / 2))) return -1;
  m->rope_freqs.assign(freqs, freqs + n);
  return 0;
}

extern "C" int oracle_create(const oracle_config* cfg, oracle_model** out) {
  if (!cfg || !out) return -1;
  const oracle_config& c = *cfg;
  if (c.dim <= 0 || c.head_dim <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 || c.n_heads % c.n_kv_heads != 0 ||
      c.max_seq_len <= kKvSinks || c.n_layers < 0 || c.dim % 16 != 0 || c.hidden_dim % 16 != 0 ||
      (c.n_heads * c.head_dim) % 16 != 0)
    return -1;
  oracle_model* m = new (std::nothrow) oracle_model();
  if (!m) return -1;
  m->c = c;
  m->layers.resize(c.n_layers);
  size_t kv = (size_t)c.max_seq_len * c.n_kv_heads * c.head_dim;
  for (auto& L : m->layers) {
    L.kcache.assign(kv, 0);
    L.vcache.assign(kv, 0);
  }
  int qd = c.n_heads * c.head_dim, kvd = c.n_kv_heads * c.head_dim;
  m->x.assign(c.dim, 0.f);
  m->xb.assign(c.dim, 0.f);
  m->xb2.assign(c.dim > qd ? c.dim : qd, 0.f);
  m->hb.assign(c.hidden_dim > c.dim ? c.hidden_dim : c.dim, 0.f);
  m->hb2.assign(c.hidden_dim, 0.f);
  m->q.assign(qd, 0.f);
  m->k.assign(kvd, 0.f);
  m->v.assign(kvd, 0.f);
  m->att.assign((size_t)c.n_heads * c.max_seq_len * 2, 0.f);
  *out = m;
  return 0;
}

extern "C" void oracle_destroy(oracle_model* m) { delete m; }

extern "C" int oracle_set_layer(oracle_model* m, int layer, const float* rms_att, const float* rms_ffn,
                                const uint16_t* wq, const uint16_t* wk, const uint16_t* wv, const uint16_t* wo,
                                const uint16_t* w1, const uint16_t* w2, const uint16_t* w3) {
  if (!m || layer < 0 || layer >= m->c.n_layers) return -1;
  OracleLayer& L = m->layers[layer];
  L.rms_att = rms_att;
  L.rms_ffn = rms_ffn;
  L.wq = wq;
  L.wk = wk;
  L.wv = wv;
  L.wo = wo;
  L.w1 = w1;
  L.w2 = w2;
  L.w3 = w3;
  return 0;
}

extern "C" int oracle_set_globals(oracle_model* m, const uint16_t* embed, const float* rms_final, const uint16_t* wcls) {
  if (!m) return -1;
  m->embed = embed;
  m->rms_final = rms_final;
  m->wcls = wcls ? wcls : embed;  // tied lm_head when model.output.weight is absent (model.cpp:425-434)
  return 0;
}

// One transformer block (infer.cpp:256-392), dense FFN (expert weight 1.0, infer.cpp:358).
static void block_forward(oracle_model* m, OracleLayer& L, int pos, int kv_sink, int kv_pos, int kv_len) {
  const oracle_config& c = m->c;
  float* x = m->x.data();
  float* xb = m->xb.data();
  float* q = m->q.data();
  float* k = m->k.data();
  float* v = m->v.data();
  int qd = c.n_heads * c.head_dim, kvd = c.n_kv_heads * c.head_dim;
  size_t msl = (size_t)c.max_seq_len;

  oracle_rmsnorm(xb, x, L.rms_att, c.dim, c.norm_eps);  // :270
  oracle_matmul_f16(q, xb, L.wq, c.dim, qd);            // :279-281
  oracle_matmul_f16(k, xb, L.wk, c.dim, kvd);
  oracle_matmul_f16(v, xb, L.wv, c.dim, kvd);
  for (int i = 0; i < qd; ++i) q[i] = clampf(q[i], c.qkv_clip);  // :284-290
  for (int i = 0; i < kvd; ++i) {
    k[i] = clampf(k[i], c.qkv_clip);
    v[i] = clampf(v[i], c.qkv_clip);
  }
  model_rope(m, q, qd, pos);  // :293-294
  model_rope(m, k, kvd, pos);

  uint16_t* kb = L.kcache.data();
  uint16_t* vb = L.vcache.data();
  for (int i = 0; i < kvd; ++i) {  // :300-305
    int g = i / c.head_dim, j = i % c.head_dim;
    kb[g * c.head_dim * msl + oracle_k_cache_idx(j, kv_pos, c.max_seq_len)] = oracle_f2h(k[i]);
    vb[g * c.head_dim * msl + (size_t)j * msl + kv_pos] = oracle_f2h(v[i]);
  }
  for (int r = 0; r < kv_sink; ++r) {  // sink re-rotation by one position (:311-325)
    for (int i = 0; i < kvd; ++i) {
      int g = i / c.head_dim, j = i % c.head_dim;
      k[i] = oracle_h2f(kb[g * c.head_dim * msl + oracle_k_cache_idx(j, r, c.max_seq_len)]);
    }
    model_rope(m, k, kvd, 1);
    for (int i = 0; i < kvd; ++i) {
      int g = i / c.head_dim, j = i % c.head_dim;
      kb[g * c.head_dim * msl + oracle_k_cache_idx(j, r, c.max_seq_len)] = oracle_f2h(k[i]);
    }
  }
  oracle_mha(m->xb2.data(), m->att.data(), kb, vb, q, c.head_dim, kv_len, c.max_seq_len, c.n_heads,
             c.n_kv_heads);                                  // :327-336
  oracle_matmul_f16(m->hb.data(), m->xb2.data(), L.wo, qd, c.dim);  // :339
  for (int i = 0; i < c.dim; ++i) x[i] += m->hb[i];          // :342-344
  oracle_rmsnorm(xb, x, L.rms_ffn, c.dim, c.norm_eps);       // :349
  oracle_matmul_f16(m->hb.data(), xb, L.w1, c.dim, c.hidden_dim);   // :367
  oracle_matmul_f16(m->hb2.data(), xb, L.w3, c.dim, c.hidden_dim);  // :368
  for (int i = 0; i < c.hidden_dim; ++i) m->hb[i] = act_fn(m->hb[i], c.act) * m->hb2[i];  // :369-382
  oracle_matmul_f16(m->xb2.data(), m->hb.data(), L.w2, c.hidden_dim, c.dim);  // :384
  for (int i = 0; i < c.dim; ++i) x[i] += m->xb2[i] * 1.0f;                 // :386-390
}

extern "C" int oracle_forward(oracle_model* m, int token, int pos, int mode, float* logits) {
  if (!m || !m->embed || token < 0 || token >= m->c.vocab_size || pos < 0) return -1;
  const oracle_config& c = m->c;
  for (auto& L : m->layers)
    if (!L.wq || !L.w1 || !L.rms_att) return -1;
  for (int i = 0; i < c.dim; ++i) m->x[i] = oracle_h2f(m->embed[(size_t)token * c.dim + i]);  // :460-481
  int kv_sink, kv_pos, kv_len;
  oracle_positions(pos, c.max_seq_len, &kv_sink, &kv_pos, &kv_len);  // :489-494
  for (auto& L : m->layers) block_forward(m, L, pos, kv_sink, kv_pos, kv_len);
  if (mode == 0) return 0;  // HYDRATE_KV_CACHE (:501-504)
  if (!logits || !m->rms_final) return -1;
  oracle_rmsnorm(m->x.data(), m->x.data(), m->rms_final, c.dim, c.norm_eps);  // :509
  oracle_matmul_f16(logits, m->x.data(), m->wcls, c.dim, c.vocab_size);     // :521
  return 0;
}

extern "C" uint16_t* oracle_key_cache(oracle_model* m, int layer) {
  return (m && layer >= 0 && layer < m->c.n_layers) ? m->layers[layer].kcache.data() : nullptr;
}
extern "C" uint16_t* oracle_value_cache(oracle_model* m, int layer) {
  return (m && layer >= 0 && layer < m->c.n_layers) ? m->layers[layer].vcache.data() : nullptr;
}
extern "C" const float* oracle_x(oracle_model* m) { return m ? m->x.data() : nullptr; }
