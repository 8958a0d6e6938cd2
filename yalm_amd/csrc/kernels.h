// CDNA4 (gfx950) device code for the fp16 batch-1 decode step.
//
// Data layout in HBM (all row-major, as in the .yalm file):
//   weights fp16 [rows][K]; activations fp32; KV caches fp16 per layer
//   K[g][(j/16)*16*msl + t*16 + j%16], V[g][j*msl + t]   (reference src/model.h:14-17, 266-268)
//
// Every kernel runs 256-thread workgroups (four 64-lane wavefronts). Matvecs stream weight rows
// with 16-byte loads: lane l of a wave reads bytes [16*(l + 64u), +16) of each row it owns, so a
// wave-wide load instruction covers 1 KiB of one row and every HBM line is read exactly once.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace yk {

typedef _Float16 f16;
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBlock = 256;
constexpr int kWave = 64;
constexpr int kWavesPerBlock = kBlock / kWave;
constexpr int kKvSinks = 2;  // reference src/model.h:12
constexpr float kNegBig = -3.402823466e38f;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// 2^x as the hardware's v_exp_f32 (about 1 ulp on the range the softmaxes use, x <= 0; results
// below 2^-126 flush to zero, which is nothing next to the running maximum's own term of 1). The
// attention kernels keep scores in log2 units (scaled by log2 e) so that every exponential is this
// one instruction instead of the ~13 of expf.
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Per-token parameters, resident on the device so that a captured graph stays static.
struct StepParams {
  int token;
  int pos;
  int pad[2];
};

// Position arithmetic of reference src/infer.cpp:489-494.
struct Positions {
  int kv_sink, kv_pos, kv_len;
};
__device__ __forceinline__ Positions positions(int pos, int msl) {
  Positions p;
  p.kv_sink = pos >= msl ? kKvSinks : 0;
  p.kv_pos = p.kv_sink + (pos - p.kv_sink) % (msl - p.kv_sink);
  p.kv_len = pos >= msl ? msl : pos + 1;
  return p;
}

__device__ __forceinline__ int k_cache_idx(int j, int t, int msl) {
  return (j >> 4) * (16 * msl) + t * 16 + (j & 15);
}

// Wavefront reductions on DPP: an inclusive row scan (row_shr 1,2,4,8) leaves each 16-lane row's
// total in its lane 15; row_bcast:15 and row_bcast:31 fold the rows so that lane 63 holds the
// wave total, which readlane returns uniformly to every lane. No LDS traffic.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_src(float old, float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old), __builtin_bit_cast(int, v),
                                                               CTRL, ROW_MASK, 0xf, false));
}
__device__ __forceinline__ float lane_read(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
__device__ __forceinline__ float lane63(float v) { return lane_read(v, 63); }
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_src<0x111, 0xf>(0.f, v);  // row_shr:1
  v += dpp_src<0x112, 0xf>(0.f, v);  // row_shr:2
  v += dpp_src<0x114, 0xf>(0.f, v);  // row_shr:4
  v += dpp_src<0x118, 0xf>(0.f, v);  // row_shr:8
  v += dpp_src<0x142, 0xa>(0.f, v);  // row_bcast:15 into rows 1 and 3
  v += dpp_src<0x143, 0xc>(0.f, v);  // row_bcast:31 into rows 2 and 3
  return lane63(v);
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_src<0x111, 0xf>(v, v));
  v = fmaxf(v, dpp_src<0x112, 0xf>(v, v));
  v = fmaxf(v, dpp_src<0x114, 0xf>(v, v));
  v = fmaxf(v, dpp_src<0x118, 0xf>(v, v));
  v = fmaxf(v, dpp_src<0x142, 0xa>(v, v));
  v = fmaxf(v, dpp_src<0x143, 0xc>(v, v));
  return lane63(v);
}

// Block-wide sum; `red` is kWavesPerBlock floats of LDS. All threads get the result.
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int wave = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) red[wave] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int w = 0; w < kWavesPerBlock; ++w) s += red[w];
  return s;
}

// Power-of-two exponent that brings a head's largest |q| (amax) into [2^14, 2^15): q * 2^e is then
// finite in fp16 (also as hi/lo parts) for any finite fp32 q, and the head's scores are multiplied
// by 2^-e. Clamped so that neither factor leaves the normal fp32 range; amax 0, inf or NaN leaves q
// as it is.
__device__ __forceinline__ int q_range_exp(float amax) {
  if (!(amax > 0.f) || !(amax < 3.402823466e38f)) return 0;
  const int e = 15 - __builtin_amdgcn_frexp_expf(amax);  // amax = m 2^E, m in [0.5, 1)
  return e < -60 ? -60 : (e > 100 ? 100 : e);
}

__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }
__device__ __forceinline__ float gelu(float x) {
  return 0.5f * x * (1.0f + tanhf(0.797885f * (x + 0.044715f * x * x * x)));
}
__device__ __forceinline__ float clipf(float x, float v) { return x < -v ? -v : (x > v ? v : x); }

// 8 fp16 weights (one 16-byte load) dotted with 8 fp32 activations from LDS.
__device__ __forceinline__ float dot8(u32x4 wbits, const float* xs, float acc) {
  f16x8 w = __builtin_bit_cast(f16x8, wbits);
  f32x4 a = *reinterpret_cast<const f32x4*>(xs);
  f32x4 b = *reinterpret_cast<const f32x4*>(xs + 4);
  acc = fmaf((float)w[0], a[0], acc);
  acc = fmaf((float)w[1], a[1], acc);
  acc = fmaf((float)w[2], a[2], acc);
  acc = fmaf((float)w[3], a[3], acc);
  acc = fmaf((float)w[4], b[0], acc);
  acc = fmaf((float)w[5], b[1], acc);
  acc = fmaf((float)w[6], b[2], acc);
  acc = fmaf((float)w[7], b[3], acc);
  return acc;
}

// ------------------------------------------------------------------------------------------
// Cross-workgroup hand-off without cache-wide fences.
//
// On a multi-XCD part each XCD has its own L2; an agent-scope fence would write back and
// invalidate the whole L2 of every workgroup that executes it. Data that one workgroup hands to
// another within a launch is instead written and read with agent-scope relaxed atomics (coherent,
// written through past the XCD's L2), and `publish()` waits until this thread's stores have
// completed before the workgroup signals.
// ------------------------------------------------------------------------------------------
__device__ __forceinline__ void store_shared(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_shared(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_shared_u32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void publish() { __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// The value, opaque to the compiler: whatever is computed from it is computed where it is used. In
// the single-launch decode (one loop over the layers) this keeps per-use address arithmetic from
// being hoisted out of the loop and held, in registers or scratch, across every phase.
__device__ __forceinline__ int opaque_v(int v) {
  __asm__ volatile("" : "+v"(v));
  return v;
}
__device__ __forceinline__ int opaque_s(int v) {
  __asm__ volatile("" : "+s"(v));
  return v;
}

constexpr unsigned kSpinLimit = 1u << 20;  // polls before a wait gives up (about a second)

// Thread 0 polls until *f == value (bounded: a time-out sets the abort flag, after which every
// wait returns at once and the host reports the error); the workgroup waits at the barrier.
__device__ __forceinline__ void wait_flag(const unsigned* f, unsigned value, unsigned* abort_flag) {
  if (threadIdx.x == 0) {
    unsigned spins = 0;
    while (__hip_atomic_load(const_cast<unsigned*>(f), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != value) {
      __builtin_amdgcn_s_sleep(1);
      if ((++spins & 255u) == 0 &&
          (spins >= kSpinLimit || __hip_atomic_load(abort_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))) {
        __hip_atomic_store(abort_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
  }
  __syncthreads();
}

constexpr int kBufferConfig = 0x00020000;  // raw buffer descriptor word 3 on gfx9-family GPUs
constexpr int kCpolSc1 = 16;               // cache-policy operand: sc1, the agent-scope coherent load
constexpr int kCpolSc0 = 1;                // cache-policy operand: sc0, served by the XCD's L2 (not the CU's L1)

// 16 bytes that another workgroup of the same launch wrote with store_shared: one dwordx4 load
// with the agent-coherence bit (the access load_shared makes per float).
__device__ __forceinline__ f32x4 load_shared4(__amdgpu_buffer_rsrc_t r, int byte_off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kCpolSc1));
}

// An activation store: plain, or agent-coherent (COH) when a later workgroup of the same launch
// consumes the value.
template <bool COH>
__device__ __forceinline__ void st_act(float* p, float v) {
  if constexpr (COH) store_shared(p, v);
  else *p = v;
}

// ------------------------------------------------------------------------------------------
// Fused matvec family.
//
// A "group" is R weight rows that one wavefront streams together. Groups are dealt to waves
// round-robin over the grid. The input vector (K fp32) is staged once per workgroup into LDS,
// optionally RMS-normalised on the way (reference src/infer.cpp:136-146). The first group's
// weight loads are issued before the staging so that HBM latency overlaps the staging.
// ------------------------------------------------------------------------------------------
enum EpiKind : int {
  kEpiStore = 0,    // out[row] = acc
  kEpiResidual = 1, // out[row] += acc            (x += W v)
  kEpiSwiGLU = 2,   // out[p] = act(acc0) * acc1   (rows p of W1 and W3)
  kEpiQkvRope = 3,  // q / K-cache / V-cache with clip and RoPE on row pairs
};

struct MatvecArgs {
  const uint16_t* w0;  // group p, row r: w0 + p*row_step + r*r_step   (or w1 for r==1 in SwiGLU)
  const uint16_t* w1;
  long row_step, r_step;
  int groups;  // number of groups
  int K;       // row length (elements), multiple of 8
  const float* x;      // input vector [K]
  const uint16_t* emb; // or, when not null, row `token` of this fp16 embedding table [vocab][K]
  float* emb_out;      // if not null, workgroup 0 also writes that row to it as fp32 (the residual stream)
  int token;           // token id, or -1 to read params->token
  const float* gain;   // rmsnorm gain [K] or nullptr (no norm)
  float eps;
  float* out;
  int act;  // 1 silu, 0 gelu (SwiGLU epilogue)
  // QKV epilogue
  int q_dim, kv_dim, head_dim, msl;
  float qkv_clip;
  uint16_t* kcache;
  uint16_t* vcache;
  const StepParams* params;
  int pos;               // position, or -1 to read params->pos
  const float* rope_cs;  // [head_dim]: (cos, sin) per rotary pair at this step's position
  // row-loop statistics for the lm_head: running (max, index) of the outputs, tie rule of
  // src/sampler.cpp:27-38, kept per wave (argmax fused into the last matvec)
  int track_max;
};

// Loads of one row segment for this lane: chunk c = lane + 64*u, u < KC (KC = K/512 when > 0).
template <int KC, int R>
__device__ __forceinline__ void load_group(u32x4 (&wv)[R][KC > 0 ? KC : 1], const uint16_t* const (&rows)[R], int lane) {
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int u = 0; u < KC; ++u)
      wv[r][u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(rows[r]) + lane + kWave * u);
}

// The same loads when the row pointers are wave-uniform (scalar registers): one buffer descriptor
// per row in scalar registers and one shared lane offset, so no per-lane 64-bit addresses are
// formed. Only for call sites whose group index is uniform by construction (readfirstlane).
constexpr int kCpolNt = 2;  // cache-policy operand: nt (streaming)
// valid == false: the descriptors cover no bytes and every load returns zero without a memory
// access (the loads are still issued, so the caller's wait counts do not depend on a branch).
template <int KC, int R>
__device__ __forceinline__ void load_group_uniform(u32x4 (&wv)[R][KC], const uint16_t* const (&rows)[R], int lane,
                                                   bool valid = true) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(rows[r]), 0, valid ? KC * 1024 : 0, kBufferConfig);
#pragma unroll
    for (int u = 0; u < KC; ++u)
      wv[r][u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, lane * 16, u * 1024, kCpolNt));
  }
}

template <int R>
__device__ __forceinline__ void group_rows(const MatvecArgs& a, int p, const uint16_t* (&rows)[R]) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint16_t* base = (r == 1 && a.w1) ? a.w1 : a.w0;
    long off = (long)p * a.row_step + ((r == 1 && a.w1) ? 0 : (long)r * a.r_step);
    rows[r] = base + off;
  }
}

__device__ __forceinline__ void better(float& bv, int& bi, float v, int i) {
  if (v > bv || (v == bv && i < bi)) {
    bv = v;
    bi = i;
  }
}

// Epilogues run on every lane of the wave (all operands are wave-uniform after the reductions);
// only lane 0 stores. Keeping the computation outside a lane-0 branch keeps the row loop's control
// flow simple.
// Operands an epilogue needs from memory, loaded together with the group's weights so that their
// latency is not paid at the end of the group.
template <int R, EpiKind EPI>
__device__ __forceinline__ void epilogue_prefetch(const MatvecArgs& a, int p, float (&pre)[R]) {
  if constexpr (EPI == kEpiResidual) {
#pragma unroll
    for (int r = 0; r < R; ++r) pre[r] = a.out[(long)p * R + r];
  }
}

template <int R, EpiKind EPI>
__device__ __forceinline__ void epilogue(const MatvecArgs& a, int p, const float (&acc)[R], const float (&pre)[R],
                                         int pos, const float* rope_cs, bool store) {
  if constexpr (EPI == kEpiStore) {
    if (store)
#pragma unroll
      for (int r = 0; r < R; ++r) a.out[(long)p * R + r] = acc[r];
  } else if constexpr (EPI == kEpiResidual) {
    if (store)
#pragma unroll
      for (int r = 0; r < R; ++r) a.out[(long)p * R + r] = pre[r] + acc[r];
  } else if constexpr (EPI == kEpiSwiGLU) {
    const float h = a.act == 1 ? silu(acc[0]) : gelu(acc[0]);
    const float v = h * acc[R - 1];
    if (store) a.out[p] = v;
  } else {  // kEpiQkvRope: rows i = 2p, 2p+1 of [Wq; Wk; Wv]  (reference src/infer.cpp:279-305)
    const int i = 2 * p;
    float v0 = clipf(acc[0], a.qkv_clip);
    float v1 = clipf(acc[R - 1], a.qkv_clip);
    if (i < a.q_dim + a.kv_dim) {  // RoPE on q and k (reference src/infer.cpp:202-215)
      // (cos, sin) of pos * freq_j for this step, staged into LDS with the input vector
      const int j = i % a.head_dim;
      const float c = rope_cs[j], s = rope_cs[j + 1];
      const float r0 = v0 * c - v1 * s;
      const float r1 = v0 * s + v1 * c;
      v0 = r0;
      v1 = r1;
    }
    if (!store) return;
    if (i < a.q_dim) {
      a.out[i] = v0;
      a.out[i + 1] = v1;
    } else {
      const Positions ps = positions(pos, a.msl);
      const bool is_k = i < a.q_dim + a.kv_dim;
      const int ik = i - a.q_dim - (is_k ? 0 : a.kv_dim);
      const int g = ik / a.head_dim, j = ik % a.head_dim;
      const long head = (long)g * a.head_dim * a.msl;
      const uint16_t h0 = __builtin_bit_cast(uint16_t, (f16)v0);  // RNE, as _cvtss_sh(x, 0)
      const uint16_t h1 = __builtin_bit_cast(uint16_t, (f16)v1);
      if (is_k) {
        a.kcache[head + k_cache_idx(j, ps.kv_pos, a.msl)] = h0;
        a.kcache[head + k_cache_idx(j + 1, ps.kv_pos, a.msl)] = h1;
      } else {
        a.vcache[head + (long)j * a.msl + ps.kv_pos] = h0;
        a.vcache[head + (long)(j + 1) * a.msl + ps.kv_pos] = h1;
      }
    }
  }
}

// Stage the (optionally RMS-normalised) input vector into LDS: xs[i] = x[i] * inv * g[i] with
// inv = 1/sqrt(mean(x^2) + eps) (reference src/infer.cpp:136-146), for any K % 4 == 0 (the
// unrolled kernels stage through stage_load / stage_store below). x16: the fp16 embedding row as
// the input instead of x. The step's RoPE table (head_dim floats) goes to LDS right after the vector.
__device__ __forceinline__ void stage_input(const MatvecArgs& a, float* xs, float* red, const uint16_t* x16) {
  if (a.rope_cs)
    for (int i = threadIdx.x; i < a.head_dim; i += kBlock) xs[a.K + i] = a.rope_cs[i];
  f32x4* o4 = reinterpret_cast<f32x4*>(xs);
  const int n4 = a.K >> 2;
  auto src4 = [&](int i) {
    f32x4 v;
    if (!x16) {
      v = reinterpret_cast<const f32x4*>(a.x)[i];
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = (float)__builtin_bit_cast(f16, x16[4 * i + e]);
    }
    return v;
  };
  if (a.gain) {
    const f32x4* g4 = reinterpret_cast<const f32x4*>(a.gain);
    float ss = 0.f;
    for (int i = threadIdx.x; i < n4; i += kBlock) {
      f32x4 v = src4(i);
      ss += v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
    }
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)a.K + a.eps);
    for (int i = threadIdx.x; i < n4; i += kBlock) {
      f32x4 v = src4(i), g = g4[i];
      f32x4 o;
      o[0] = v[0] * inv * g[0];
      o[1] = v[1] * inv * g[1];
      o[2] = v[2] * inv * g[2];
      o[3] = v[3] * inv * g[3];
      o4[i] = o;
    }
  } else {
    for (int i = threadIdx.x; i < n4; i += kBlock) o4[i] = src4(i);
  }
  __syncthreads();
}

// The same staging in two halves, for the pipelined matvec (K == 1024*NPT, plain accesses):
// stage_load issues every global read the staging needs (x or the raw fp16 embedding row, the
// gains, the RoPE table) into registers; the caller then issues its first weight loads, and
// stage_store normalises, fills LDS and synchronises the workgroup. Loads complete in issue order,
// so consuming reads issued before the weights does not wait for the weights, and the first row
// group stays in flight across the staging barrier. GAIN / EMB: whether the call site can have an
// RMS gain / an embedding-row input (the residual epilogue has neither), which keeps registers for
// the other cases out of the kernel.
// Which inputs an epilogue kind's call sites can have (the host rejects the others).
template <EpiKind EPI>
constexpr bool kEpiGain = EPI != kEpiResidual;
template <EpiKind EPI>
constexpr bool kEpiEmb = EPI == kEpiQkvRope || EPI == kEpiStore;

template <int NPT, bool GAIN, bool EMB>
struct StagedInput {
  f32x4 xv[NPT], gv[GAIN ? NPT : 1];
  unsigned long long hv[EMB ? NPT : 1];  // four fp16 of the embedding row
  float rc;
};

template <int NPT, bool GAIN, bool EMB>
__device__ __forceinline__ void stage_load(const MatvecArgs& a, StagedInput<NPT, GAIN, EMB>& st, const uint16_t* x16) {
  if (EMB && x16) {
    const unsigned long long* h4 = reinterpret_cast<const unsigned long long*>(x16);
#pragma unroll
    for (int k = 0; k < NPT; ++k) st.hv[k] = h4[threadIdx.x + kBlock * k];
  } else {
    const f32x4* x4 = reinterpret_cast<const f32x4*>(a.x);
#pragma unroll
    for (int k = 0; k < NPT; ++k) st.xv[k] = x4[threadIdx.x + kBlock * k];
  }
  if (GAIN && a.gain) {
    const f32x4* g4 = reinterpret_cast<const f32x4*>(a.gain);
#pragma unroll
    for (int k = 0; k < NPT; ++k) st.gv[k] = g4[threadIdx.x + kBlock * k];
  }
  st.rc = a.rope_cs && (int)threadIdx.x < a.head_dim ? a.rope_cs[threadIdx.x] : 0.f;
}

template <int NPT, bool GAIN, bool EMB>
__device__ __forceinline__ void stage_store(const MatvecArgs& a, StagedInput<NPT, GAIN, EMB>& st, float* xs, float* red,
                                            int pos, const uint16_t* x16) {
  if (a.rope_cs && (int)threadIdx.x < a.head_dim) xs[a.K + threadIdx.x] = st.rc;
  if (EMB && x16) {
#pragma unroll
    for (int k = 0; k < NPT; ++k)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        st.xv[k][e] = (float)__builtin_bit_cast(f16, (uint16_t)(st.hv[k] >> (16 * e)));
  }
  f32x4* o4 = reinterpret_cast<f32x4*>(xs);
  if (GAIN && a.gain) {
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < NPT; ++k)
      ss += st.xv[k][0] * st.xv[k][0] + st.xv[k][1] * st.xv[k][1] + st.xv[k][2] * st.xv[k][2] + st.xv[k][3] * st.xv[k][3];
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)a.K + a.eps);
#pragma unroll
    for (int k = 0; k < NPT; ++k) {
      f32x4 o;
      o[0] = st.xv[k][0] * inv * st.gv[k][0];
      o[1] = st.xv[k][1] * inv * st.gv[k][1];
      o[2] = st.xv[k][2] * inv * st.gv[k][2];
      o[3] = st.xv[k][3] * inv * st.gv[k][3];
      o4[threadIdx.x + kBlock * k] = o;
    }
  } else {
#pragma unroll
    for (int k = 0; k < NPT; ++k) o4[threadIdx.x + kBlock * k] = st.xv[k];
  }
  __syncthreads();
}

// Per-wave running maximum for the fused argmax (track_max); every lane holds the same values.
struct RowMax {
  float v = kNegBig;
  int i = 0x7fffffff;
};

template <int R, EpiKind EPI>
__device__ __forceinline__ void track_rows(const MatvecArgs& a, int p, const float (&acc)[R], RowMax& m) {
  if constexpr (EPI == kEpiStore) {
    if (a.track_max)
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (acc[r] > kNegBig) better(m.v, m.i, acc[r], p * R + r);
  }
}

// The fused matvec over groups p = blk*4 + wave + k*(nblk*4).
// KC > 0: K == 512*KC*H, fully unrolled row streaming. KC == 0: any K % 8 == 0.
// H == 2 (R == 1 only): each row is streamed as two pieces of K/2 (see below).
template <int KC, int R, EpiKind EPI, int H = 1>
__device__ __forceinline__ RowMax matvec_body(const MatvecArgs& a, int blk, int nblk, float* lds) {
  float* red = lds;      // kWavesPerBlock floats (padded to 16)
  float* xs = lds + 16;  // K floats (+ the RoPE table)
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int wave_stride = nblk * kWavesPerBlock;
  int p = blk * kWavesPerBlock + wave;
  RowMax mx;
  // embedding row as the input (reference src/infer.cpp:460-481: exact fp16 -> fp32)
  const uint16_t* x16 = nullptr;
  if (a.emb) {
    x16 = a.emb + (long)(a.token >= 0 ? a.token : a.params->token) * a.K;
    if (a.emb_out && blk == 0)
      for (int i = threadIdx.x; i < a.K; i += kBlock) a.emb_out[i] = (float)__builtin_bit_cast(f16, x16[i]);
  }

  static_assert(H == 1 || (H == 2 && R == 1 && KC > 0), "two-piece rows: one row per group, unrolled");
  if constexpr (H == 2) {
    // Long rows (W2: 28 KB) in two pieces through the two register buffers: piece 0 of a group in
    // wa, piece 1 in wb, so each buffer holds half a row and the pair fits the register file with
    // room to spare (two whole-row buffers need ~250 VGPRs, and the compiler then reuses buffer
    // registers as address temporaries, which forces a wait for the older buffer before every
    // issue). Piece 1 is issued before piece 0 is used and the next group's piece 0 before piece 1
    // is used; the loop has a single exit and a peeled last group, as below.
    const int w_id = __builtin_amdgcn_readfirstlane(wave);
    const int p0 = blk * kWavesPerBlock + w_id;
    const int n = p0 < a.groups ? (a.groups - 1 - p0) / wave_stride + 1 : 0;  // this wave's groups
    const int half = a.K / 2;
    u32x4 wa[1][KC], wb[1][KC];
    float pre[1];
    auto issue = [&](u32x4 (&wv)[1][KC], int i, int piece, bool valid = true) {
      const uint16_t* rows[1];
      group_rows<1>(a, valid ? p0 + i * wave_stride : 0, rows);
      rows[0] += piece * half;
      load_group_uniform<KC, 1>(wv, rows, lane, valid);
      if (piece == 1) epilogue_prefetch<1, EPI>(a, p0 + i * wave_stride, pre);
    };
    StagedInput<KC, kEpiGain<EPI>, kEpiEmb<EPI>> st;  // K = 1024*KC -> KC float4 per thread
    stage_load(a, st, x16);
    __builtin_amdgcn_sched_barrier(0);
    issue(wa, 0, 0, n > 0);  // unconditional: a branch here would make the staging wait for it
    const int pos = EPI == kEpiQkvRope ? (a.pos >= 0 ? a.pos : a.params->pos) : 0;
    stage_store(a, st, xs, red, pos, x16);
    float carry = 0.f;
    auto use = [&](const u32x4 (&wv)[1][KC], int i, int piece) {
      const float* xp = xs + piece * half;
      float acc = 0.f;
#pragma unroll
      for (int u = 0; u < KC; ++u) {
        acc = dot8(wv[0][u], xp + 8 * (lane + kWave * u), acc);
        if ((u & 3) == 3) __builtin_amdgcn_sched_barrier(0);
      }
      if (piece == 0) {
        carry = acc;
        return;
      }
      float accs[1] = {wave_sum(carry + acc)};
      const int pg = p0 + i * wave_stride;
      epilogue<1, EPI>(a, pg, accs, pre, pos, xs + a.K, lane == 0);
      track_rows<1, EPI>(a, pg, accs, mx);
    };
    int i = 0;
    for (; i + 1 < n; ++i) {
      issue(wb, i, 1);
      __builtin_amdgcn_sched_barrier(0);
      use(wa, i, 0);
      issue(wa, i + 1, 0);
      __builtin_amdgcn_sched_barrier(0);
      use(wb, i, 1);
    }
    if (i < n) {
      issue(wb, i, 1);
      __builtin_amdgcn_sched_barrier(0);
      use(wa, i, 0);
      use(wb, i, 1);
    }
  } else if constexpr (KC > 0) {
    // Two register buffers, one group in flight: group i + 1's loads are issued as soon as group
    // i's have landed and before group i's dot products, reduction and epilogue, so a wave's
    // arithmetic overlaps its next memory round trip. (Two groups in flight per wave measured
    // slower: the memory queues saturate.) The loop is unrolled by two with a single exit and a
    // peeled tail so that every load inside it is unconditional and the compiler's wait for the
    // older buffer stays "at most one group outstanding".
    const int w_id = __builtin_amdgcn_readfirstlane(wave);
    const int p0 = blk * kWavesPerBlock + w_id;
    const int n = p0 < a.groups ? (a.groups - 1 - p0) / wave_stride + 1 : 0;  // this wave's groups
    u32x4 wa[R][KC], wb[R][KC];
    float prea[R], preb[R];
    auto issue = [&](u32x4 (&wv)[R][KC], float (&pre)[R], int i, bool valid = true) {
      const uint16_t* rows[R];
      const int g = valid ? p0 + i * wave_stride : 0;
      group_rows<R>(a, g, rows);
      load_group_uniform<KC, R>(wv, rows, lane, valid);
      epilogue_prefetch<R, EPI>(a, g, pre);
    };
    StagedInput<KC / 2, kEpiGain<EPI>, kEpiEmb<EPI>> st;  // K = 512*KC -> KC/2 float4 per thread
    stage_load(a, st, x16);
    __builtin_amdgcn_sched_barrier(0);
    issue(wa, prea, 0, n > 0);  // unconditional: a branch here would make the staging wait for it
    const int pos = EPI == kEpiQkvRope ? (a.pos >= 0 ? a.pos : a.params->pos) : 0;
    stage_store(a, st, xs, red, pos, x16);
    auto use = [&](const u32x4 (&wv)[R][KC], const float (&pre)[R], int i) {
      const int pg = p0 + i * wave_stride;
      float acc[R];
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] = 0.f;
#pragma unroll
      for (int u = 0; u < KC; ++u) {
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = dot8(wv[r][u], xs + 8 * (lane + kWave * u), acc[r]);
        if ((u & 3) == 3) __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);
      epilogue<R, EPI>(a, pg, acc, pre, pos, xs + a.K, lane == 0);
      track_rows<R, EPI>(a, pg, acc, mx);
    };
    int i = 0;
    for (; i + 2 < n; i += 2) {
      issue(wb, preb, i + 1);
      __builtin_amdgcn_sched_barrier(0);
      use(wa, prea, i);
      issue(wa, prea, i + 2);
      __builtin_amdgcn_sched_barrier(0);
      use(wb, preb, i + 1);
    }
    if (i + 2 == n) {
      issue(wb, preb, i + 1);
      __builtin_amdgcn_sched_barrier(0);
      use(wa, prea, i);
      use(wb, preb, i + 1);
    } else if (i + 1 == n) {
      use(wa, prea, i);
    }
  } else {
    const int pos = EPI == kEpiQkvRope ? (a.pos >= 0 ? a.pos : a.params->pos) : 0;
    stage_input(a, xs, red, x16);
    const int nch = a.K >> 3;
    for (; p < a.groups; p += wave_stride) {
      const uint16_t* rows[R];
      group_rows<R>(a, p, rows);
      float pre[R];
      epilogue_prefetch<R, EPI>(a, p, pre);
      float acc[R];
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] = 0.f;
      for (int c = lane; c < nch; c += kWave) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(rows[r]) + c);
          acc[r] = dot8(w, xs + 8 * c, acc[r]);
        }
      }
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);
      epilogue<R, EPI>(a, p, acc, pre, pos, xs + a.K, lane == 0);
      track_rows<R, EPI>(a, p, acc, mx);
    }
  }
  return mx;
}

template <int KC, int R, EpiKind EPI, int H = 1>
__global__ void __launch_bounds__(kBlock) matvec_kernel(MatvecArgs a) {
  extern __shared__ float lds[];
  matvec_body<KC, R, EPI, H>(a, blockIdx.x, gridDim.x, lds);
}

// Packed (logit, index) whose unsigned order is the argmax order with the reference's tie rule
// (src/sampler.cpp:27-38: the first index of the maximum): the float's bits made monotonic in the
// high word (negative values complemented, positive ones with the sign bit set), the complement of
// the index in the low word. NaN and -inf never reach it (track_rows keeps only v > kNegBig).
__device__ __forceinline__ unsigned long long argmax_key(float v, int i) {
  const unsigned u = __float_as_uint(v == 0.f ? 0.f : v);  // -0 == +0 for the comparison
  const unsigned ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)ord << 32) | (unsigned)(~i);
}

// Workgroup best of the waves' maxima (wave-uniform), posted with one 64-bit atomic max. The atomic
// returns nothing, so no workgroup waits on it; the key is zeroed before each step by the step-
// parameter kernel and read back after the launch.
__device__ __forceinline__ void argmax_post(RowMax mx, unsigned long long* key) {
  __shared__ float sv[kWavesPerBlock];
  __shared__ int si[kWavesPerBlock];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  if (lane == 0) {
    sv[wave] = mx.v;
    si[wave] = mx.i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    RowMax r;
    for (int w = 0; w < kWavesPerBlock; ++w) better(r.v, r.i, sv[w], si[w]);
    if (r.i != 0x7fffffff) __hip_atomic_fetch_max(key, argmax_key(r.v, r.i), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Final rmsnorm + lm_head with the greedy argmax fused in (a.track_max set).
template <int KC>
__global__ void __launch_bounds__(kBlock) lm_head_argmax_kernel(MatvecArgs a, unsigned long long* key) {
  extern __shared__ float lds[];
  const RowMax mx = matvec_body<KC, 2, kEpiStore>(a, blockIdx.x, gridDim.x, lds);
  argmax_post(mx, key);
}

// ------------------------------------------------------------------------------------------
// Per-step RoPE table: rope_cs[2k], rope_cs[2k+1] = cos, sin of (float)pos * inv_freq[k], the angle
// of rotary pair k (reference src/infer.cpp:205-208: fp32 angle pos * freq, then cosf / sinf).
// inv_freq[k] = 1 / powf(theta, 2k / rotary_dim), or 0 past rotary_dim, is computed on the host.
// ------------------------------------------------------------------------------------------
__device__ __forceinline__ void fill_rope_table(const float* inv_freq, float* rope_cs, int half, int pos) {
  for (int k = threadIdx.x; k < half; k += blockDim.x) {
    const float ang = (float)pos * inv_freq[k];
    rope_cs[2 * k] = cosf(ang);
    rope_cs[2 * k + 1] = sinf(ang);
  }
}

__global__ void rope_table_kernel(const float* inv_freq, float* rope_cs, int half, const StepParams* params) {
  fill_rope_table(inv_freq, rope_cs, half, params->pos);
}

// ------------------------------------------------------------------------------------------
// Split-KV GQA decode attention (reference src/infer.cpp:218-250, 327-336).
//
// Workgroup (g, s) handles kv head g and the s-th slice of [0, kv_len) for all G query heads
// that share g, so each K/V byte is read once per token. Slices are at least min_slice tokens
// (128 from kv_len 1024 on):
//   chunk = max(floor, roundup(ceil(kv_len / nsplit), 64)),  active = ceil(kv_len / chunk)
// Workgroups past `active` exit at once. With one active slice the workgroup writes the output
// directly; otherwise each writes (max, sum, acc) per head and the last to finish (atomic ticket)
// merges them. Scores for a 256-token tile go to LDS; an online softmax keeps (max, sum, acc).
// In sink mode (pos >= msl) slice 0 first re-rotates the two sink keys by one position
// (reference src/infer.cpp:307-325).
// ------------------------------------------------------------------------------------------
struct AttnArgs {
  const float* q;        // [nh][hd]
  uint16_t* kcache;      // layer base
  const uint16_t* vcache;
  float* partial;        // [nh][nsplit][hd + 2]
  unsigned* tickets;     // [nkv]
  float* out;            // [nh][hd]
  int head_dim, n_heads, n_kv_heads, msl, nsplit;
  int min_slice;          // smallest KV slice per workgroup (multiple of 64; MFMA kernel: 0 = by length)
  int defer_merge = 0;    // MFMA kernel: every slice (one included) stores its partial and the slices are
                          // merged by the next launch (merge_o_kernel) instead of the last slice
  const float* inv_freq;  // [head_dim / 2] rotary frequencies (sink re-rotation by one position)
  const StepParams* params;
};

constexpr int kMaxGroup = 8;

// Tokens per KV slice, a multiple of `gran` (the kernel's tile). From 1024 cached tokens on,
// slices are at least 128 tokens (fewer, longer slices: the merge and the per-workgroup start cost
// outweigh the extra parallelism there).
__host__ __device__ __forceinline__ int attn_chunk(int kv_len, int nsplit, int min_slice, int gran = 64) {
  int chunk = (kv_len + nsplit - 1) / nsplit;
  chunk = (chunk + gran - 1) / gran * gran;
  const int floor = (kv_len >= 1024 && min_slice < 128) ? 128 : min_slice;
  return chunk < floor ? floor : chunk;
}

// Slice length of the MFMA decode attention: min_slice > 0 is a fixed floor; 0 picks it by context
// length, from sweeps on MI355X (Mistral shape, 24 slices per kv head):
//   - up to 320 keys one slice per kv head, no cross-workgroup merge (300 keys: 7.8 against 9.7 µs
//     per layer with two 256-key slices);
//   - up to 2048 keys slices of 64: the merge of many short slices costs less than two or three
//     long ones (400 keys: 8.4 against 9.7; 1024: 8.9 against 10.1 µs per layer; with the merge in
//     the O launch, µs per decode step against 128-key slices at 1100 / 1300 / 1500 / 2000 keys:
//     2672 / 2682 / 2693 / 2715 against 2684 / 2691 / 2695 / 2719);
//   - up to 6144 keys slices of 128 (the slice merge runs in the O launch there: µs per decode
//     step against 256-key slices, 1600 keys 2683 / 2735, 2400: 2704 / 2748, 3216: 2766 / 2775;
//     with 28 slices per kv head against 384-key ones, 4500: 2821 / 2821, 5200: 2836 / 2870,
//     5600: 2850 / 2875, 6000: 2856 / 2876), beyond that 384 (6500: 2913 / 2882, 7500: 2889 /
//     2894, 9000: 2924 / 2919); from ~10K keys the slice count (nsplit) decides.
__host__ __device__ __forceinline__ int attn_mfma_chunk(int kv_len, int nsplit, int min_slice) {
  if (min_slice > 0) return attn_chunk(kv_len, nsplit, min_slice, 32);
  if (kv_len <= 320) return (kv_len + 31) / 32 * 32;
  const int floor = kv_len <= 2048 ? 64 : (kv_len <= 6144 ? 128 : 384);
  const int chunk = ((kv_len + nsplit - 1) / nsplit + 31) / 32 * 32;
  return chunk < floor ? floor : chunk;
}

// Sum over groups of N adjacent lanes (N = 1, 2, 4, 8, 16, 32, 64); every lane of a group gets the
// group total. DPP quad permutes and row mirrors, one cross-row swap for N = 32 and two lane reads
// for the whole wave.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
template <int N>
__device__ __forceinline__ float lane_group_sum(float v) {
  if constexpr (N >= 2) v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
  if constexpr (N >= 4) v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
  if constexpr (N >= 8) v += dpp_mov<0x141>(v);  // row_half_mirror
  if constexpr (N >= 16) v += dpp_mov<0x140>(v); // row_mirror
  if constexpr (N >= 32) v += __shfl_xor(v, 16, kWave);
  if constexpr (N >= 64) v = lane_read(v, 0) + lane_read(v, 32);
  return v;
}

// Tile geometry of the attention workgroup for head_dim HD and NT threads.
//   Score phase: LPT lanes per token, each owning CPL 16-dim chunks of K; TT tokens per tile.
//   Value phase: LPD adjacent lanes cover one V row's TT tokens (8 tokens = 16 bytes each, so a
//   wave instruction reads whole 128-byte lines); a thread owns DPT rows d = dgrp + NDG*m and
//   tokens 8*oct .. 8*oct+7 of the tile.
// Each lane keeps the query values of its CPL chunks for all G heads in registers (16*CPL*G
// floats); the 512-thread layout gives every lane a single chunk (LPT = HD/16) to keep that small.
template <int HD, int NT>
struct AttnGeom {
  static constexpr int NW = NT / kWave;
  static constexpr int LPT = (NT >= 512 || HD < 64) ? HD / 16 : 4;
  static constexpr int CPL = HD / 16 / LPT;
  static constexpr int TT = NT / LPT;
  static constexpr int LPD = TT / 8;
  static constexpr int NDG = NT / LPD;
  static constexpr int DPT = HD / NDG;
  static_assert(DPT >= 1 && NDG * DPT == HD && LPD <= kWave, "attention tile layout");
};

// LDS of one attention workgroup.
constexpr int kMaxSplits = 64;  // KV slices per kv head (the partial buffer holds this many)

template <int HD, int G, int NT>
struct AttnSmem {
  float qs[G * HD];
  __attribute__((aligned(16))) float ps[G][AttnGeom<HD, NT>::TT];
  float red[2][G][NT / kWave];
  float mrg[G][kMaxSplits][2];  // merge: per slice (weight, sum), then 1/L per head in red
  unsigned last_flag;
};

// Cross-workgroup merge of the slices of kv head g, after this workgroup stored its partial
// (unnormalised output, running max m, sum l) for each of its G heads with coherent stores: the
// last slice to finish computes out = sum_s w_s o_s / sum_s w_s l_s with w_s = exp(m_s - max m).
// Every load of a round is issued before any is used: (m, l) of all slices first, then each
// output's slices eight at a time (addresses clamped to the last slice, surplus dropped).
// mrg: LDS [G][kMaxSplits][2]; Ls: LDS, G floats; last_flag: LDS word.
template <int HD, int G, int NT, bool COH>
__device__ __forceinline__ void attn_merge_slices(const AttnArgs& a, int g, int active, int tid,
                                                  float (&mrg)[G][kMaxSplits][2], float* Ls, unsigned& last_flag) {
  const int stride = HD + 2;
  tid = opaque_v(tid);
  publish();
  __syncthreads();
  if (tid == 0) {
    const unsigned t = __hip_atomic_fetch_add(&a.tickets[g], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_flag = (t == (unsigned)(active - 1)) ? 1u : 0u;
  }
  __syncthreads();
  if (!last_flag) return;
  // One round trip: the (m, l) of every slice and this thread's first RND slices of its outputs
  // are all requested before anything waits ((m, l) first, so waiting for them leaves the rest in
  // flight); later rounds only when there are more than RND slices.
  constexpr int MLPT = (kMaxGroup * kMaxSplits + NT - 1) / NT;
  constexpr int OPT = (G * HD + NT - 1) / NT;  // outputs per thread
  constexpr int RND = OPT == 1 ? 32 : (OPT == 2 ? 16 : 8);  // slices per round (<= 32 loads per thread)
  float ml[MLPT][2];
#pragma unroll
  for (int i = 0; i < MLPT; ++i) {
    const int e = tid + i * NT;
    if (e < G * active) {
      const int h = e / active, sp = e - h * active;
      const float* pp = a.partial + ((long)(g * G + h) * a.nsplit + sp) * stride;
      ml[i][0] = load_shared(pp + HD);
      ml[i][1] = load_shared(pp + HD + 1);
    }
  }
  auto load_round = [&](int sp0, float (&v)[OPT][RND]) {
#pragma unroll
    for (int j = 0; j < OPT; ++j) {
      const int e = min(tid + j * NT, G * HD - 1);
      const float* src = a.partial + (long)(g * G + e / HD) * a.nsplit * stride + e % HD;
#pragma unroll
      for (int k = 0; k < RND; ++k) v[j][k] = sp0 + k < active ? load_shared(src + (long)(sp0 + k) * stride) : 0.f;
    }
  };
  float v[OPT][RND];
  load_round(0, v);
#pragma unroll
  for (int i = 0; i < MLPT; ++i) {
    const int e = tid + i * NT;
    if (e < G * active) {
      const int h = e / active, sp = e - h * active;
      mrg[h][sp][0] = ml[i][0];
      mrg[h][sp][1] = ml[i][1];
    }
  }
  __syncthreads();
  // per head: wave h, lane sp (active <= 64 slices), reduced across the wave instead of a serial
  // loop over the slices on one lane
  for (int h = tid / kWave; h < G; h += NT / kWave) {
    const int sp = tid & (kWave - 1);
    const float m = sp < active ? mrg[h][sp][0] : kNegBig;
    const float M = wave_max(m);
    const float w = sp < active ? expf(m - M) : 0.f;
    const float L = wave_sum(sp < active ? mrg[h][sp][1] * w : 0.f);
    if (sp < active) mrg[h][sp][0] = w;
    if (sp == 0) Ls[h] = L;
  }
  __syncthreads();
  float Ov[OPT];
#pragma unroll
  for (int j = 0; j < OPT; ++j) Ov[j] = 0.f;
  for (int sp0 = 0;;) {
#pragma unroll
    for (int j = 0; j < OPT; ++j) {
      const int h = min(tid + j * NT, G * HD - 1) / HD;
#pragma unroll
      for (int k = 0; k < RND; ++k)
        if (sp0 + k < active) Ov[j] = fmaf(v[j][k], mrg[h][sp0 + k][0], Ov[j]);
    }
    sp0 += RND;
    if (sp0 >= active) break;
    load_round(sp0, v);
  }
#pragma unroll
  for (int j = 0; j < OPT; ++j) {
    const int e = tid + j * NT;
    if (e < G * HD) {
      const int h = e / HD;
      float* o = a.out + (long)(g * G + h) * HD + e % HD;
      if constexpr (COH) store_shared(o, Ov[j] / Ls[h]);
      else *o = Ov[j] / Ls[h];
    }
  }
  if (tid == 0) __hip_atomic_store(&a.tickets[g], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Re-rotates the K of the sink tokens r < kv_sink by angle freq*1 in place, fp16 round trip as
// the reference (src/infer.cpp:307-325); kh is the kv head's K cache. COH: the entries are read
// and written with agent-coherent accesses and written through before the function returns (the
// caller's coherent K loads then see them).
template <int HD, int NT, bool COH = false>
__device__ __forceinline__ void rotate_sinks(const AttnArgs& a, uint16_t* kh, int kv_sink, int tid) {
  for (int e = tid; e < kv_sink * (HD / 2); e += NT) {
    const int r = e / (HD / 2);
    const int j = 2 * (e % (HD / 2));
    const float freq = a.inv_freq[j / 2];
    const float c = cosf(freq), s = sinf(freq);
    uint16_t* p0 = kh + k_cache_idx(j, r, a.msl);
    uint16_t* p1 = kh + k_cache_idx(j + 1, r, a.msl);
    uint16_t h0, h1;
    if constexpr (COH) {
      h0 = __hip_atomic_load(p0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      h1 = __hip_atomic_load(p1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      h0 = *p0;
      h1 = *p1;
    }
    const float v0 = (float)__builtin_bit_cast(f16, h0), v1 = (float)__builtin_bit_cast(f16, h1);
    const uint16_t r0 = __builtin_bit_cast(uint16_t, (f16)(v0 * c - v1 * s));
    const uint16_t r1 = __builtin_bit_cast(uint16_t, (f16)(v0 * s + v1 * c));
    if constexpr (COH) {
      __hip_atomic_store(p0, r0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(p1, r1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      *p0 = r0;
      *p1 = r1;
    }
  }
  if constexpr (COH) publish();
}

// K and V registers for one tile of one thread (loaded one tile ahead of use).
template <int CPL, int DPT>
struct AttnTileRegs {
  u32x4 k[CPL][2];  // this thread's 16-dim K chunks of its token
  u32x4 v[DPT];     // 8 consecutive tokens of each of this thread's V rows
};

// One attention workgroup: kv head g, KV slice `split`, all G query heads of g; tid is the thread
// index (passed in so that a caller's loop can keep lane-derived values from being hoisted).
// HD: head_dim; G: query heads per kv head; NT: threads.
// Partial sums stay per lane and are reduced over the LPD lanes once, after the last tile. Every
// tile issues the same loads (addresses clamped into the cache, results masked), so the compiler
// waits only for the tile it is about to use.
template <int HD, int G, int NT>
__device__ __forceinline__ void attn_run(const AttnArgs& a, int g, int split, int pos, AttnSmem<HD, G, NT>& sm, int tid) {
  using Geo = AttnGeom<HD, NT>;
  constexpr int LPT = Geo::LPT, CPL = Geo::CPL, TT = Geo::TT, LPD = Geo::LPD, NDG = Geo::NDG, DPT = Geo::DPT;
  constexpr int NW = Geo::NW;
  static_assert(G >= 1 && G <= kMaxGroup, "query heads per kv head");
  const int lane = tid & (kWave - 1), wave = tid / kWave;
  const Positions pss = positions(pos, a.msl);
  const int kv_len = pss.kv_len;
  const int chunk = attn_chunk(kv_len, a.nsplit, a.min_slice);
  const int active = (kv_len + chunk - 1) / chunk;
  if (split >= active) return;
  const int t_begin = split * chunk;
  const int t_end = min(kv_len, t_begin + chunk);
  const long head_off = (long)g * HD * a.msl;
  uint16_t* kh = a.kcache + head_off;
  const uint16_t* vh = a.vcache + head_off;

  if (pss.kv_sink > 0 && split == 0) {
    rotate_sinks<HD, NT>(a, kh, pss.kv_sink, tid);
    __syncthreads();
  }

  const int tok_l = tid / LPT, sub = tid % LPT;
  const int oct = tid % LPD, dgrp = tid / LPD;
  const bool vec_ok = (a.msl & 7) == 0;
  const int vmax = vec_ok ? a.msl - 8 : 0;

  auto load_tile = [&](int t0, AttnTileRegs<CPL, DPT>& r) {
    const int tok = min(t0 + tok_l, a.msl - 1);
#pragma unroll
    for (int cc = 0; cc < CPL; ++cc) {
      const u32x4* kp = reinterpret_cast<const u32x4*>(kh + (long)(sub * CPL + cc) * 16 * a.msl + (long)tok * 16);
      r.k[cc][0] = kp[0];
      r.k[cc][1] = kp[1];
    }
    if (vec_ok) {
      const int tv = min(t0 + 8 * oct, vmax);
#pragma unroll
      for (int m = 0; m < DPT; ++m)
        r.v[m] = *reinterpret_cast<const u32x4*>(vh + (long)(dgrp + NDG * m) * a.msl + tv);
    }
  };

  // The first K/V tile does not depend on q: its loads go out first, then all of this thread's q
  // loads, and only then does anything wait.
  AttnTileRegs<CPL, DPT> cur, nxt;
  load_tile(t_begin, cur);
  {
    constexpr int QPT = (G * HD + NT - 1) / NT;
    float qv[QPT];
#pragma unroll
    for (int i = 0; i < QPT; ++i) {
      const int e = min(tid + i * NT, G * HD - 1);
      qv[i] = a.q[(long)g * G * HD + e];
    }
#pragma unroll
    for (int i = 0; i < QPT; ++i)
      if (tid + i * NT < G * HD) sm.qs[tid + i * NT] = qv[i];
  }
  float m_run[G], l_run[G], acc[DPT][G];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m_run[h] = kNegBig;
    l_run[h] = 0.f;
#pragma unroll
    for (int m = 0; m < DPT; ++m) acc[m][h] = 0.f;
  }
  const float inv_sqrt_hd = 1.0f / sqrtf((float)HD);
  __syncthreads();

  for (int t0 = t_begin; t0 < t_end; t0 += TT) {
    load_tile(t0 + TT < t_end ? t0 + TT : t0, nxt);  // next tile (or this one again) in flight
    const int tok = t0 + tok_l;
    const bool valid = tok < t_end;
    const int tv = t0 + 8 * oct;
    // scores: partial dots over this lane's chunks, then summed over the LPT lanes of the token
    float s[G];
#pragma unroll
    for (int h = 0; h < G; ++h) s[h] = 0.f;
#pragma unroll
    for (int cc = 0; cc < CPL; ++cc) {
      const f16x8 k0 = __builtin_bit_cast(f16x8, cur.k[cc][0]);
      const f16x8 k1 = __builtin_bit_cast(f16x8, cur.k[cc][1]);
      const int c = sub * CPL + cc;
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float* qh = sm.qs + h * HD + c * 16;
        float d = s[h];
#pragma unroll
        for (int e = 0; e < 8; ++e) d = fmaf(qh[e], (float)k0[e], d);
#pragma unroll
        for (int e = 0; e < 8; ++e) d = fmaf(qh[8 + e], (float)k1[e], d);
        s[h] = d;
      }
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
      s[h] = lane_group_sum<LPT>(s[h]);
      s[h] = valid ? s[h] * inv_sqrt_hd : kNegBig;
      const float m = wave_max(s[h]);
      if (lane == 0) sm.red[0][h][wave] = m;
    }
    __syncthreads();
    float corr[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float m = sm.red[0][h][0];
#pragma unroll
      for (int w = 1; w < NW; ++w) m = fmaxf(m, sm.red[0][h][w]);
      const float m_new = fmaxf(m_run[h], m);
      corr[h] = expf(m_run[h] - m_new);
      m_run[h] = m_new;
      const float p = valid ? expf(s[h] - m_new) : 0.f;
      const bool mine = sub == (h % LPT);  // each (token, head) probability stored and summed once
      if (mine) sm.ps[h][tok_l] = p;
      const float t = wave_sum(mine ? p : 0.f);
      if (lane == 0) sm.red[1][h][wave] = t;
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float t = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) t += sm.red[1][h][w];
      l_run[h] = l_run[h] * corr[h] + t;
#pragma unroll
      for (int m = 0; m < DPT; ++m) acc[m][h] *= corr[h];
    }
    // values: acc[m][h] += sum over this lane's 8 tokens of p[h][t] * V[d_m][t]
    if (vec_ok && tv + 8 <= t_end) {
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const f32x4 p0 = *reinterpret_cast<const f32x4*>(&sm.ps[h][8 * oct]);
        const f32x4 p1 = *reinterpret_cast<const f32x4*>(&sm.ps[h][8 * oct + 4]);
#pragma unroll
        for (int m = 0; m < DPT; ++m) {
          const f16x8 v8 = __builtin_bit_cast(f16x8, cur.v[m]);
          float d = acc[m][h];
          d = fmaf(p0[0], (float)v8[0], d);
          d = fmaf(p0[1], (float)v8[1], d);
          d = fmaf(p0[2], (float)v8[2], d);
          d = fmaf(p0[3], (float)v8[3], d);
          d = fmaf(p1[0], (float)v8[4], d);
          d = fmaf(p1[1], (float)v8[5], d);
          d = fmaf(p1[2], (float)v8[6], d);
          d = fmaf(p1[3], (float)v8[7], d);
          acc[m][h] = d;
        }
      }
    } else if (tv < t_end) {  // partial run at the end of the slice: element by element
      for (int e = 0; e < 8; ++e) {
        const int t = tv + e;
        if (t < t_end) {
#pragma unroll
          for (int m = 0; m < DPT; ++m) {
            const int d = dgrp + NDG * m;
            const float v = (float)__builtin_bit_cast(f16, vh[(long)d * a.msl + t]);
#pragma unroll
            for (int h = 0; h < G; ++h) acc[m][h] = fmaf(sm.ps[h][8 * oct + e], v, acc[m][h]);
          }
        }
      }
    }
    cur = nxt;
    __syncthreads();  // ps / red are rewritten by the next tile
  }

  // Reduce the value sums over the LPD lanes of each row group (adjacent lanes).
#pragma unroll
  for (int m = 0; m < DPT; ++m)
#pragma unroll
    for (int h = 0; h < G; ++h) acc[m][h] = lane_group_sum<LPD>(acc[m][h]);
  const bool writer = oct == 0;
  if (active == 1) {  // the only slice: final normalisation here
    if (writer)
#pragma unroll
      for (int m = 0; m < DPT; ++m)
#pragma unroll
        for (int h = 0; h < G; ++h) {
          a.out[(long)(g * G + h) * HD + dgrp + NDG * m] = acc[m][h] / l_run[h];
        }
    return;
  }
  const int stride = HD + 2;
  if (writer) {
#pragma unroll
    for (int m = 0; m < DPT; ++m)
#pragma unroll
      for (int h = 0; h < G; ++h)
        store_shared(a.partial + ((long)(g * G + h) * a.nsplit + split) * stride + dgrp + NDG * m, acc[m][h]);
  }
  if (tid < G) {
#pragma unroll
    for (int h = 0; h < G; ++h)
      if (h == tid) {
        float* dst = a.partial + ((long)(g * G + h) * a.nsplit + split) * stride;
        store_shared(dst + HD, m_run[h]);
        store_shared(dst + HD + 1, l_run[h]);
      }
  }
  attn_merge_slices<HD, G, NT, false>(a, g, active, tid, sm.mrg, &sm.red[0][0][0], sm.last_flag);
}

// Split-KV attention as its own launch: grid (n_kv_heads, nsplit) of 256-thread workgroups.
template <int HD, int G>
__global__ void __launch_bounds__(kBlock) attention_kernel(AttnArgs a) {
  __shared__ AttnSmem<HD, G, kBlock> sm;
  attn_run<HD, G, kBlock>(a, blockIdx.x, blockIdx.y, a.params->pos, sm, threadIdx.x);
}

// ------------------------------------------------------------------------------------------
// Greedy argmax over logits with the reference tie rule (first index of the strict maximum,
// src/sampler.cpp:27-38). One workgroup of kArgmaxThreads; every thread issues its float4 loads
// up front (n = 32000 -> 8 per thread).
// ------------------------------------------------------------------------------------------
constexpr int kArgmaxThreads = 1024;

__global__ void __launch_bounds__(kArgmaxThreads) argmax_kernel(const float* logits, int n, int* out) {
  __shared__ float sv[kArgmaxThreads / kWave];
  __shared__ int si[kArgmaxThreads / kWave];
  float bv = kNegBig;
  int bi = 0x7fffffff;
  const int n4 = n >> 2;
  const f32x4* l4 = reinterpret_cast<const f32x4*>(logits);
  constexpr int kBatch = 8;
  for (int base = 0; base < n4; base += kArgmaxThreads * kBatch) {
    f32x4 v[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int idx = base + k * kArgmaxThreads + threadIdx.x;
      v[k] = idx < n4 ? l4[idx] : f32x4{kNegBig, kNegBig, kNegBig, kNegBig};
    }
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int idx = base + k * kArgmaxThreads + threadIdx.x;
      if (idx < n4)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (v[k][e] > kNegBig) better(bv, bi, v[k][e], 4 * idx + e);
    }
  }
  for (int i = 4 * n4 + threadIdx.x; i < n; i += kArgmaxThreads)
    if (logits[i] > kNegBig) better(bv, bi, logits[i], i);
  // wave reduce (value, index) with the tie rule
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, kWave);
    const int oi = __shfl_xor(bi, o, kWave);
    better(bv, bi, ov, oi);
  }
  const int wave = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float v = sv[0];
    int i = si[0];
    for (int w = 1; w < kArgmaxThreads / kWave; ++w) better(v, i, sv[w], si[w]);
    out[0] = i == 0x7fffffff ? 0 : i;
  }
}

}  // namespace yk
