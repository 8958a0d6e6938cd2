// Decode attention on the matrix cores: one query position, GQA, split-KV over workgroups.
//
// Same result as the split-KV kernel in kernels.h (reference src/infer.cpp:218-250: scores over
// keys 0..kv_len-1 read back from the fp16 caches, max-subtracted softmax, weighted sum of V), but
// both products run on MFMA and every wave streams its own keys:
//   - workgroup (kv head g, slice s) of NW waves; wave w takes the 32-key tiles w, w + NW, ... of
//     the slice and keeps its own online softmax (no workgroup barrier per tile); the next tile's
//     loads are in flight while the current one is used; a wave with no tile issues no loads;
//   - scores S^T = K Q^T with v_mfma_f32_16x16x32_f16, two 16-key groups per tile: A = 16 keys x
//     32 dims of K straight from the 16-tiled cache (16 bytes per lane), B = the G query heads as
//     columns. Each head's fp32 q is first scaled by a power of two that maps its largest |q| into
//     [2^14, 2^15) (undone exactly in the score scale), then split into q_hi = fp16(q) and
//     q_lo = fp16(q - q_hi) in columns h and G + h, so the sum of the two columns carries ~22 bits
//     of q relative to the head's largest entry, for any finite fp32 q (fp16 products are exact in
//     the fp32 accumulate);
//   - the keys of group j are ordered so that row 4 i + r is key 8 i + 4 j + r of the tile: the
//     accumulators then leave lane l (column l % 16) with keys 8 (l / 16) .. +7 of the tile, which
//     is exactly the B operand layout of O^T += V^T P^T on v_mfma_f32_16x16x32_f16, and the A
//     operand is one 16-byte load per lane of 8 consecutive keys of a V row ([dim][key] cache,
//     64 contiguous bytes per row per instruction). p is scaled by kPScale into the fp16 normal
//     range and split into hi/lo columns like q (undone at the end);
//   - the waves' (m, l, o) are merged in LDS; slices of one kv head are merged by the last one
//     to finish (attn_merge_slices).
// Needs head_dim % 16 == 0 (head_dim 16: the k-step's upper 16 dims of K lie past the head's K
// region and read as zero, those of q are masked to zero) and max_seq_len % 8 == 0 (16-byte V
// reads; keys past the context are read clamped and masked). The per-op launches keep to
// max_seq_len % 32 == 0.
//
// COH (the single-launch decode, where q and the current position's K/V were written by other
// workgroups of the same launch with write-through stores): q, K and V are read with the
// agent-coherence bit (sc1), so no line this XCD's L2 may still hold is used.
#pragma once

#include "kernels.h"

namespace yk {


constexpr float kPScale = 4096.f;

__device__ __forceinline__ f32x4 mfma_16x16x32(const u32x4& a, const u32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                0, 0);
}

// K and V fragments of one wave for one 32-key tile starting at t0 (lane = 16 q + m).
template <int HD>
constexpr int kKSteps = (HD + 31) / 32;  // 32-dim k-steps of the score product

template <int HD>
struct KvFrag {
  u32x4 k[2][kKSteps<HD>];  // group j, k step ks: key t0 + 8 (m / 4) + 4 j + m % 4, dims 32 ks + 8 q .. +7
  u32x4 v[HD / 16];     // dim 16 dt + m, keys t0 + 8 q .. +7
};

// Buffer loads: the K/V regions of the kv head are addressed by a descriptor in scalar registers,
// so each load takes one 32-bit lane offset plus a wave-uniform scalar offset (the dims / k-step
// strides) instead of a 64-bit address per load; reads past the region return zero.
template <bool COH = false>
__device__ __forceinline__ u32x4 buffer_load16(__amdgpu_buffer_rsrc_t rsrc, int voff, int soff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, voff, soff, COH ? kCpolSc1 : 0));
}

template <int HD, bool COH = false>
__device__ __forceinline__ void load_kv_frag(__amdgpu_buffer_rsrc_t kr, __amdgpu_buffer_rsrc_t vr, int msl, int t0,
                                             int m, int q, KvFrag<HD>& f) {
  // K byte offset: (2 ks + q / 2) * 16 msl * 2 + key * 32 + 16 (q % 2)
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int tk = min(t0 + 8 * (m >> 2) + 4 * j + (m & 3), msl - 1);
    const int vo = (q >> 1) * 32 * msl + tk * 32 + 16 * (q & 1);
#pragma unroll
    for (int ks = 0; ks < kKSteps<HD>; ++ks) f.k[j][ks] = buffer_load16<COH>(kr, vo, ks * 64 * msl);
  }
  // V byte offset: (16 dt + m) * msl * 2 + key * 2
  const int vo = m * 2 * msl + 2 * min(t0 + 8 * q, msl - 8);
#pragma unroll
  for (int dt = 0; dt < HD / 16; ++dt) f.v[dt] = buffer_load16<COH>(vr, vo, dt * 32 * msl);
}

template <int HD, int G, int NW>
struct AttnMfmaSmem {
  float om[NW][G][HD];  // per-wave unnormalised outputs
  float oml[NW][G][2];  // per-wave (max, sum)
  float mrg[G][kMaxSplits][2];
  float Ls[G];
  unsigned last_flag;
};

// The per-wave part of the MFMA attention over keys [t_begin, t_end) of kv head g, for all G
// query heads of g, in a workgroup of NW waves: every wave's (m, l, o) lands in sm.om / sm.oml,
// then a workgroup barrier.
// NB: tile buffers per wave -- 1 (each tile loaded after the previous one is used) or 2 (the next
// tile's loads in flight while the current one is used). `issue()` runs once in every wave, right
// after the wave's first
// K/V tile and its q loads are issued (at once in a wave without a tile): loads it issues are
// younger than those, and loads retire in issue order, so waiting for the tile and q does not wait
// for them.
// COH: coherent q, K and V loads (see the file comment).
template <int HD, int G, int NW, int NB, bool COH = false, class Issue>
__device__ __forceinline__ void attn_mfma_waves(const AttnArgs& a, int g, int t_begin, int t_end,
                                                AttnMfmaSmem<HD, G, NW>& sm, Issue issue) {
  static_assert(HD % 16 == 0 && G >= 1 && G <= 8, "head_dim % 16, 1..8 query heads per kv head");
  static_assert(NB == 1 || NB == 2, "tile buffers per wave");
  constexpr int KS = kKSteps<HD>, DT = HD / 16;
  constexpr int TS = 32;  // keys per wave tile
  auto& om = sm.om;
  auto& oml = sm.oml;

  // the wave index in a scalar register: per-wave tile bounds and loop exits are then uniform
  // branches rather than exec-masked ones
  // (tid opaque: the lane's offsets are computed here, where they are used; see opaque_v)
  const int tid = opaque_v(threadIdx.x), lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, grp = lane >> 4;
  const long head_off = (long)g * HD * a.msl;
  const int head_bytes = HD * a.msl * 2;
  const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(a.kcache + head_off, 0, head_bytes, kBufferConfig);
  const __amdgpu_buffer_rsrc_t vr =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.vcache + head_off), 0, head_bytes, kBufferConfig);

  float m_run = kNegBig, l_run = 0.f;
  f32x4 acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  // A wave past the slice's end loads nothing and computes nothing (not even q): it enters the
  // workgroup merge with (m, l, o) = (-inf, 0, 0). At short context most waves are such, and
  // keeping their loads out of the memory queues shortens the working waves' round trips.
  int t0 = t_begin + TS * wave;
  if (t0 < t_end) {
    // first tile in flight before q is read
    KvFrag<HD> cur;
    [[maybe_unused]] KvFrag<HD> nxt;
    load_kv_frag<HD, COH>(kr, vr, a.msl, t0, col, grp, cur);

    // q as the B operand: column col is head col (hi part) or head col - G (lo part); others zero
    u32x4 qf[KS];
    float smul;  // score scale of this lane's head: 1/sqrt(hd) in log2 units, times 2^-e of the head
    {
      const bool used = col < 2 * G;
      const bool lo = col >= G;
      const int h = used ? (lo ? col - G : col) : 0;
      f32x4 q4[KS][2];
      if constexpr (COH) {  // the kv head's G query rows through one descriptor; dims past HD are zero
        const __amdgpu_buffer_rsrc_t qr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(a.q + (long)g * G * HD), 0, G * HD * (int)sizeof(float), kBufferConfig);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const int d = 32 * ks + 8 * grp;
          const int off = 4 * (h * HD + (d < HD ? d : 0));
#pragma unroll
          for (int hf = 0; hf < 2; ++hf) {
            const f32x4 v = load_shared4(qr, off + 16 * hf);
            q4[ks][hf] = d < HD ? v : f32x4{0.f, 0.f, 0.f, 0.f};
          }
        }
      } else {
        static_assert(COH || HD % 32 == 0, "head_dim 16 only with coherent (masked) q loads");
        const float* qp = a.q + (long)(g * G + h) * HD + 8 * grp;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          q4[ks][0] = *reinterpret_cast<const f32x4*>(qp + 32 * ks);
          q4[ks][1] = *reinterpret_cast<const f32x4*>(qp + 32 * ks + 4);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      issue();
      __builtin_amdgcn_sched_barrier(0);
      // the head's largest |q| over the four lanes of the column (each holds 8 of every 32 dims)
      float amax = 0.f;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(q4[ks][e >> 2][e & 3]));
      amax = fmaxf(amax, __shfl_xor(amax, 16));
      amax = fmaxf(amax, __shfl_xor(amax, 32));
      const int qe = q_range_exp(amax);
      const float qmul = __builtin_ldexpf(1.0f, qe);
      smul = __builtin_ldexpf(kLog2e / sqrtf((float)HD), -qe);  // scores in log2 units (exp2_fast)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        f16x8 v;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x = q4[ks][e >> 2][e & 3] * qmul;
          const f16 hi = (f16)x;
          v[e] = !used ? (f16)0.f : (lo ? (f16)(x - (float)hi) : hi);
        }
        qf[ks] = __builtin_bit_cast(u32x4, v);
      }
    }

    // one 32-key tile: scores, online softmax (per column = head), values
    auto tile = [&](const KvFrag<HD>& f, int t0) {
      f32x4 s[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        s[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) s[j] = mfma_16x16x32(f.k[j][ks], qf[ks], s[j]);
      }
      float sv[8];  // keys t0 + 8 grp + e
      float mt = kNegBig;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float raw = s[e >> 2][e & 3];
        const float v = raw + __shfl_xor(raw, G, 16);  // hi + lo columns (both partners get the sum)
        sv[e] = (t0 + 8 * grp + e < t_end) ? v * smul : kNegBig;
        mt = fmaxf(mt, sv[e]);
      }
      mt = fmaxf(mt, __shfl_xor(mt, 16));
      mt = fmaxf(mt, __shfl_xor(mt, 32));
      const float m_new = fmaxf(m_run, mt);
      const float corr = exp2_fast(m_run - m_new);
      m_run = m_new;
      f16x8 pf;
      float psum = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float p = sv[e] > kNegBig ? exp2_fast(sv[e] - m_new) : 0.f;
        psum += p;
        const float ps = p * kPScale;
        const f16 hi = (f16)ps;
        pf[e] = col < G ? hi : (col < 2 * G ? (f16)(ps - (float)hi) : (f16)0.f);
      }
      l_run = l_run * corr + psum;
      const u32x4 pb = __builtin_bit_cast(u32x4, pf);
      // rescale only when some column's running maximum moved
      if (__any(corr != 1.f))
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[dt] *= corr;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) acc[dt] = mfma_16x16x32(f.v[dt], pb, acc[dt]);
    };
    // NB = 2: two register buffers used alternately (unrolled by two, no copies between them):
    // while one tile is used the next one's loads are in flight, and the scheduling barrier keeps
    // them at the top. The explicit wait for the current tile is free in the steady state and keeps
    // the compiler from waiting on the in-flight tile inside the current one. NB = 1: one buffer,
    // each tile loaded after the previous one is used (fewer registers, for short slices).
    if constexpr (NB == 1) {
      for (;;) {
        tile(cur, t0);
        t0 += TS * NW;
        if (t0 >= t_end) break;
        load_kv_frag<HD, COH>(kr, vr, a.msl, t0, col, grp, cur);
      }
    } else for (;;) {
      int tn = t0 + TS * NW;
      if (tn >= t_end) {
        tile(cur, t0);
        break;
      }
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0); expcnt and lgkmcnt unconstrained
      load_kv_frag<HD, COH>(kr, vr, a.msl, tn, col, grp, nxt);
      __builtin_amdgcn_sched_barrier(0);
      tile(cur, t0);
      t0 = tn;
      tn = t0 + TS * NW;
      if (tn >= t_end) {
        tile(nxt, t0);
        break;
      }
      __builtin_amdgcn_s_waitcnt(0x0F70);
      load_kv_frag<HD, COH>(kr, vr, a.msl, tn, col, grp, cur);
      __builtin_amdgcn_sched_barrier(0);
      tile(nxt, t0);
      t0 = tn;
    }
  } else {
    issue();
  }

  // this wave's (m, l, o): l summed over the four lane groups, o over the hi/lo columns
  float lsum = l_run + __shfl_xor(l_run, 16);
  lsum += __shfl_xor(lsum, 32);
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[dt][r] += __shfl_xor(acc[dt][r], G, 16);
  if (col < G) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) om[wave][col][dt * 16 + 4 * grp + r] = acc[dt][r] * (1.0f / kPScale);
    if (grp == 0) {
      oml[wave][col][0] = m_run;
      oml[wave][col][1] = lsum;
    }
  }
  __syncthreads();
}

// One workgroup of NW waves: kv head g, KV slice `split`, all G query heads of g (NB as
// attn_mfma_waves; COH: coherent loads, and the output and the sink keys written through).
template <int HD, int G, int NW, int NB = 2, bool COH = false>
__device__ __forceinline__ void attn_mfma_body(const AttnArgs& a, int g, int split, const Positions& pss,
                                               AttnMfmaSmem<HD, G, NW>& sm) {
  constexpr int NT = 64 * NW;
  const int tid = opaque_v(threadIdx.x);
  const int kv_len = pss.kv_len;
  const int chunk = attn_mfma_chunk(kv_len, a.nsplit, a.min_slice);
  const int active = (kv_len + chunk - 1) / chunk;
  if (split >= active) return;
  const int t_begin = split * chunk;
  const int t_end = min(kv_len, t_begin + chunk);
  if (pss.kv_sink > 0 && split == 0) {
    rotate_sinks<HD, NT, COH>(a, a.kcache + (long)g * HD * a.msl, pss.kv_sink, tid);
    __syncthreads();
  }
  attn_mfma_waves<HD, G, NW, NB, COH>(a, g, t_begin, t_end, sm, [] {});
  auto& om = sm.om;
  auto& oml = sm.oml;

  // the workgroup's (m, l, o) per head: final output, or this slice's partial for the merge
  const int stride = HD + 2;
  for (int e = tid; e < G * HD; e += NT) {
    const int h = e / HD, d = e % HD;
    float M = kNegBig;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, oml[w][h][0]);
    float O = 0.f, L = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float wt = exp2_fast(oml[w][h][0] - M);
      O = fmaf(om[w][h][d], wt, O);
      L = fmaf(oml[w][h][1], wt, L);
    }
    if (active == 1 && !a.defer_merge) {
      st_act<COH>(a.out + (long)(g * G + h) * HD + d, O / L);
    } else {
      float* dst = a.partial + ((long)(g * G + h) * a.nsplit + split) * stride;
      store_shared(dst + d, O);
      if (d == 0) {
        store_shared(dst + HD, M * kLn2);  // the slice merge works in natural units
        store_shared(dst + HD + 1, L);
      }
    }
  }
  if (active == 1 || a.defer_merge) return;
  attn_merge_slices<HD, G, NT, COH>(a, g, active, tid, sm.mrg, sm.Ls, sm.last_flag);
}

template <int HD, int G, int NW, int NB = 2>
__global__ void __launch_bounds__(64 * NW) attn_mfma_kernel(AttnArgs a) {
  __shared__ AttnMfmaSmem<HD, G, NW> sm;
  attn_mfma_body<HD, G, NW, NB>(a, blockIdx.x, blockIdx.y, positions(a.params->pos, a.msl), sm);
}

// ------------------------------------------------------------------------------------------
// Decode attention and the O projection in one launch (short contexts, no sink rotation),
// reference src/infer.cpp:327-344: x += Wo . concat_h attn_h.
//
// The product splits over kv heads: Wo . attn = sum_g Wo[:, cols(g)] . attn(g), where cols(g) are
// the G * HD columns of the G query heads of kv head g. Workgroup b takes kv head g = b % nkv and
// the RB output rows starting at rb * RB (rb = b / nkv); with nkv = 8 every workgroup of kv head g
// runs on the same XCD (b mod 8), so that head's K/V lines are fetched into one L2 only. Each
// workgroup
//   1. issues its K/V tile and q loads, then its Wo block (RB rows x G*HD columns, 16 bytes per
//      lane per row segment, streaming loads) while the attention runs;
//   2. runs the whole-context MFMA attention of kv head g for its G query heads (every workgroup of
//      g repeats it: a few hundred keys are a few hundred KB from L2, against the separate launch's
//      boundary and start-up);
//   3. multiplies its Wo block by that attention output (LDS) and combines each row's sum with the
//      other kv heads' in a 64-bit word per row (below); the workgroup that completes a row writes
//      x[row] once.
// Wo loads: chunk c = lane + 64 u (u < U) of the wave's block is row c / CPR, column chunk c % CPR
// (CPR = G*HD/8 16-byte chunks per row segment); a wave covers U * 64 / CPR rows.
//
// The per-row word: bits 0..55 hold the sum of the terms 2^52 + round(p 2^32) added so far (p: one
// workgroup's fp32 partial product for that row with |p| < 2^20 - 1, so |p 2^32| <= 2^52 - 2^32;
// each term is below 2^53, so up to 8 of them never carry into bit 56), bits 56..59 count the
// partials outside that range and bits 60..63 all additions. Every workgroup adds its term plus
// 2^60 with one returning 64-bit atomic; the one whose addition brings the count to nkv holds all
// terms in (returned value + its own), writes x[row] += (sum - n_in 2^52) 2^-32 and clears the word
// for the next launch. Integer addition is associative, so x does not depend on the order in which
// the workgroups' atomics land: the step is bit-reproducible. The fixed-point resolution is 2^-32
// (2.3e-10) per partial, absolute.
// A partial outside the range (|p| >= 2^20 - 1, inf or NaN) is not clamped: it goes into a float
// side sum per row (ovf, an fp32 atomic add) and its term is 2^60 + 2^56 only, added with release
// ordering; the completing workgroup of such a row acquires and adds the side sum too, so large
// values arrive exactly as fp32 sums (order-dependent in that case only) and inf and NaN reach x as
// the reference's fp32 O projection gives them (src/infer.cpp:339-344).
// ------------------------------------------------------------------------------------------
struct AttnOArgs {
  const uint16_t* wo;        // [dim][q_dim]
  float* x;                  // [dim], x += Wo . attn
  unsigned long long* rowacc;  // [dim] combining words, zero between launches
  float* ovf;                  // [dim] fp32 side sums of out-of-range partials, zero between launches
  int dim, q_dim;
};

constexpr int kRowAccCountShift = 60;
constexpr int kRowAccOvfShift = 56;
constexpr unsigned long long kRowAccValueMask = (1ull << kRowAccOvfShift) - 1;
constexpr unsigned long long kRowAccBias = 1ull << 52;
constexpr float kRowAccScale = 4294967296.0f;  // 2^32
constexpr float kRowAccRange = 1048575.0f;      // 2^20 - 1: |p| below it keeps |p 2^32| <= 2^52 - 2^32
constexpr int kRowAccMaxTerms = 8;

__device__ __forceinline__ bool rowacc_in_range(float p) { return fabsf(p) < kRowAccRange; }  // false for NaN
// This workgroup's term for one row: 2^60 (the count) + 2^52 + round(p 2^32) for an in-range
// partial, 2^60 + 2^56 (the out-of-range count) otherwise.
__device__ __forceinline__ unsigned long long rowacc_term(float p) {
  if (!rowacc_in_range(p)) return (1ull << kRowAccCountShift) + (1ull << kRowAccOvfShift);
  return (1ull << kRowAccCountShift) + kRowAccBias + (unsigned long long)(long long)rintf(p * kRowAccScale);
}
// The in-range partials' fp32 sum from a completed word of n terms: (value bits - n_in 2^52) 2^-32.
__device__ __forceinline__ float rowacc_sum(unsigned long long w, int n) {
  const int n_in = n - (int)((w >> kRowAccOvfShift) & 0xf);
  const long long v = (long long)(w & kRowAccValueMask) - (long long)n_in * (long long)kRowAccBias;
  return (float)v * (1.0f / kRowAccScale);
}

template <int HD, int G, int NW, int U>
struct AttnOGeom {
  static constexpr int CPR = G * HD / 8;
  static constexpr int UPR = CPR >= 64 ? CPR / 64 : 1;   // loads per row (CPR >= 64)
  static constexpr int RPL = CPR >= 64 ? 1 : 64 / CPR;   // rows per load (CPR < 64)
  static constexpr int RW = CPR >= 64 ? U / UPR : U * RPL;  // rows per wave
  static constexpr int RB = RW * NW;                     // rows per workgroup
  static_assert(RW >= 1 && RW <= 64 && (CPR >= 64 ? U % UPR == 0 : true), "attention + O row layout");
};

// The O part shared by attn_o_kernel and merge_o_kernel: this wave's Wo rows (wv, columns of kv
// head g) times the G heads' attention output ao (LDS), each row's sum combined with the other kv
// heads' in the row words; the workgroup completing a row writes x[row].
template <int HD, int G, int NW, int U>
__device__ __forceinline__ void attn_o_rows(const AttnOArgs& o, const float* ao, float (&rs)[NW][AttnOGeom<HD, G, NW, U>::RW],
                                            const u32x4 (&wv)[U], int row0, int lane, int wave, int nkv) {
  using Geo = AttnOGeom<HD, G, NW, U>;
  constexpr int CPR = Geo::CPR, RW = Geo::RW;
  // Wo block . attention output; row sums to lanes 0 .. RW-1, then one atomic per row
  float mine = 0.f;
  if constexpr (CPR >= 64) {
#pragma unroll
    for (int j = 0; j < RW; ++j) {
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < Geo::UPR; ++k) {
        const int c = lane + 64 * (j * Geo::UPR + k);
        acc = dot8(wv[j * Geo::UPR + k], ao + 8 * (c % CPR), acc);
      }
      const float s = wave_sum(acc);
      if (lane == j) mine = s;
    }
  } else {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float s = lane_group_sum<CPR>(dot8(wv[u], ao + 8 * (lane % CPR), 0.f));
      if (lane % CPR == 0) rs[wave][u * Geo::RPL + lane / CPR] = s;
    }
    __syncthreads();
    mine = lane < RW ? rs[wave][lane] : 0.f;
  }
  const int row = row0 + lane;
  if (lane < RW && row < o.dim) {
    const float xr = o.x[row];
    const unsigned long long term = rowacc_term(mine);
    unsigned long long old;
    if (rowacc_in_range(mine)) {
      old = __hip_atomic_fetch_add(o.rowacc + row, term, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {  // the side sum first, published by the word's release
      __hip_atomic_fetch_add(o.ovf + row, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      old = __hip_atomic_fetch_add(o.rowacc + row, term, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    }
    const unsigned long long w = old + term;
    if ((int)(w >> kRowAccCountShift) == nkv) {  // the last of the row's nkv terms
      float v = rowacc_sum(w, nkv);
      if ((w >> kRowAccOvfShift) & 0xf) {  // some partial went to the side sum
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        v += __hip_atomic_load(o.ovf + row, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(o.ovf + row, 0.f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      o.x[row] = xr + v;
      __hip_atomic_store(o.rowacc + row, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}
// This wave's Wo rows, columns of kv head g, into registers (streaming loads); rows past dim read as
// zero (descriptor bound).
template <int HD, int G, int NW, int U>
__device__ __forceinline__ void attn_o_issue(const AttnOArgs& o, int g, int row0, int lane, u32x4 (&wv)[U]) {
  constexpr int CPR = AttnOGeom<HD, G, NW, U>::CPR;
  const long row_bytes = (long)o.q_dim * 2;
  const int valid_bytes = row0 < o.dim ? (int)min((long)(o.dim - row0) * row_bytes, (long)0x7fffffff) : 0;
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(o.wo + (long)(row0 < o.dim ? row0 : 0) * o.q_dim + (long)g * G * HD), 0, valid_bytes,
      kBufferConfig);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int c = lane + 64 * u;
    const int voff = (c / CPR) * (int)row_bytes + (c % CPR) * 16;
    wv[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, voff, 0, kCpolNt));
  }
}

template <int HD, int G, int NW, int U>
__global__ void __launch_bounds__(64 * NW) attn_o_kernel(AttnArgs a, AttnOArgs o) {
  using Geo = AttnOGeom<HD, G, NW, U>;
  constexpr int RW = Geo::RW;
  __shared__ AttnMfmaSmem<HD, G, NW> sm;
  __shared__ __attribute__((aligned(16))) float ao[G * HD];
  __shared__ float rs[NW][RW];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = (int)blockIdx.x % a.n_kv_heads, rb = (int)blockIdx.x / a.n_kv_heads;
  const int row0 = rb * Geo::RB + wave * RW;
  const int kv_len = min(a.params->pos + 1, a.msl);  // the host runs this kernel only for pos < msl

  u32x4 wv[U];
  attn_mfma_waves<HD, G, NW, 1>(a, g, 0, kv_len, sm, [&] { attn_o_issue<HD, G, NW, U>(o, g, row0, lane, wv); });

  // the workgroup's attention output for the G heads of g, normalised, into LDS
  for (int e = tid; e < G * HD; e += 64 * NW) {
    const int h = e / HD, d = e % HD;
    float M = kNegBig;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, sm.oml[w][h][0]);
    float O = 0.f, L = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float wt = exp2_fast(sm.oml[w][h][0] - M);
      O = fmaf(sm.om[w][h][d], wt, O);
      L = fmaf(sm.oml[w][h][1], wt, L);
    }
    ao[e] = O / L;
  }
  __syncthreads();

  attn_o_rows<HD, G, NW, U>(o, ao, rs, wv, row0, lane, wave, a.n_kv_heads);
}

// ------------------------------------------------------------------------------------------
// Slice merge and the O projection in one launch (contexts beyond attn_o's): the split-KV attention
// launch before it stores every slice's partial (unnormalised output o_s, running maximum m_s in
// natural units, sum l_s; AttnArgs::defer_merge) and skips its own last-slice merge. Workgroup b
// (kv head g = b % nkv, rows as attn_o_kernel) issues its Wo block at entry (its addresses depend
// on nothing), then reads the step parameters and requests kv head g's partial block (G heads x
// nsplit slices x (HD + 2) floats, at most kMergeOMaxSplits slices) into registers, merges
// out_h = sum_s w_s o_s / sum_s w_s l_s with w_s = exp(m_s - max_s m_s) (reference
// src/infer.cpp:172-187,218-250: one softmax over all keys, restated over slices), then multiplies
// and combines rows as attn_o_kernel.
// ------------------------------------------------------------------------------------------
constexpr int kMergeOMaxSplits = 32;

template <int HD, int G, int NW, int U>
__global__ void __launch_bounds__(64 * NW) merge_o_kernel(AttnArgs a, AttnOArgs o) {
  using Geo = AttnOGeom<HD, G, NW, U>;
  constexpr int RW = Geo::RW, NT = 64 * NW;
  constexpr int EPT = (G * HD + NT - 1) / NT;  // output elements per thread
  constexpr int NS = kMergeOMaxSplits;
  static_assert(G <= NW && NS <= 64, "one wave per head for the slice weights");
  __shared__ float wts[G][NS];
  __shared__ float linv[G];
  __shared__ __attribute__((aligned(16))) float ao[G * HD];
  __shared__ float rs[NW][RW];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = (int)blockIdx.x % a.n_kv_heads, rb = (int)blockIdx.x / a.n_kv_heads;
  const int row0 = rb * Geo::RB + wave * RW;
  // The Wo stream starts before the step parameters' round trip. Loads return in order, so the
  // partials below arrive with the Wo block; issuing the partials first instead (so that the merge
  // could run under the Wo stream) measured 0.8% slower per decode step at 1K-16K keys.
  u32x4 wv[U];
  attn_o_issue<HD, G, NW, U>(o, g, row0, lane, wv);
  __builtin_amdgcn_sched_barrier(0);
  const Positions pss = positions(a.params->pos, a.msl);
  const int chunk = attn_mfma_chunk(pss.kv_len, a.nsplit, a.min_slice);
  const int active = (pss.kv_len + chunk - 1) / chunk;  // as the attention launch counted them

  // kv head g's partials: rows (g G + h) nsplit + s of HD + 2 floats, one block (reads past it
  // return zero), straight into registers: wave h < G takes (m, l) of slice s in lane s; every
  // thread takes, for its output element (h, d), the d column of head h's active slices.
  const int rowf = HD + 2;
  const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
      a.partial + (long)g * G * a.nsplit * rowf, 0, G * a.nsplit * rowf * (int)sizeof(float), kBufferConfig);
  float pm = kNegBig, pl = 0.f;
  if (wave < G && lane < active) {
    const int off = 4 * ((wave * a.nsplit + lane) * rowf + HD);
    pm = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(pr, off, 0, 0));
    pl = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(pr, off + 4, 0, 0));
  }
  float po[EPT][NS];
#pragma unroll
  for (int i = 0; i < EPT; ++i) {
    const int e = tid + NT * i, h = e / HD, d = e % HD;
    const int base = 4 * (h * a.nsplit * rowf + d);
    if (e < G * HD) {
#pragma unroll
      for (int s = 0; s < NS; ++s)
        if (s < active)  // active is wave-uniform: a scalar branch
          po[i][s] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(pr, base + 4 * s * rowf, 0, 0));
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // per head: the slices' weights relative to the largest maximum, and 1 / sum_s w_s l_s
  if (wave < G) {
    const float M = wave_max(pm);
    const float w = lane < active ? expf(pm - M) : 0.f;
    const float L = wave_sum(w * pl);
    if (lane < NS) wts[wave][lane] = w;
    if (lane == 0) linv[wave] = 1.0f / L;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < EPT; ++i) {
    const int e = tid + NT * i, h = e / HD;
    if (e < G * HD) {
      float O = 0.f;
#pragma unroll
      for (int s = 0; s < NS; ++s)
        if (s < active) O = fmaf(wts[h][s], po[i][s], O);
      ao[e] = O * linv[h];
    }
  }
  __syncthreads();
  attn_o_rows<HD, G, NW, U>(o, ao, rs, wv, row0, lane, wave, a.n_kv_heads);
}
}  // namespace yk
