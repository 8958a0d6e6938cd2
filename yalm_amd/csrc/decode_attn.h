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
// Needs head_dim % 32 == 0 and max_seq_len % 32 == 0.
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
struct KvFrag {
  u32x4 k[2][HD / 32];  // group j, k step ks: key t0 + 8 (m / 4) + 4 j + m % 4, dims 32 ks + 8 q .. +7
  u32x4 v[HD / 16];     // dim 16 dt + m, keys t0 + 8 q .. +7
};

// Buffer loads: the K/V regions of the kv head are addressed by a descriptor in scalar registers,
// so each load takes one 32-bit lane offset plus a wave-uniform scalar offset (the dims / k-step
// strides) instead of a 64-bit address per load; reads past the region return zero.
// CPOL kCpolSc1: agent-coherent reads, for entries written by other workgroups of the same launch.
template <int CPOL = 0>
__device__ __forceinline__ u32x4 buffer_load16(__amdgpu_buffer_rsrc_t rsrc, int voff, int soff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, voff, soff, CPOL));
}

template <int HD, int CPOL = 0>
__device__ __forceinline__ void load_kv_frag(__amdgpu_buffer_rsrc_t kr, __amdgpu_buffer_rsrc_t vr, int msl, int t0,
                                             int m, int q, KvFrag<HD>& f) {
  // K byte offset: (2 ks + q / 2) * 16 msl * 2 + key * 32 + 16 (q % 2)
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int tk = min(t0 + 8 * (m >> 2) + 4 * j + (m & 3), msl - 1);
    const int vo = (q >> 1) * 32 * msl + tk * 32 + 16 * (q & 1);
#pragma unroll
    for (int ks = 0; ks < HD / 32; ++ks) f.k[j][ks] = buffer_load16<CPOL>(kr, vo, ks * 64 * msl);
  }
  // V byte offset: (16 dt + m) * msl * 2 + key * 2
  const int vo = m * 2 * msl + 2 * min(t0 + 8 * q, msl - 8);
#pragma unroll
  for (int dt = 0; dt < HD / 16; ++dt) f.v[dt] = buffer_load16<CPOL>(vr, vo, dt * 32 * msl);
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
// then a workgroup barrier. COH: q and the K/V entries are read with agent-coherent loads (they
// were written by other workgroups of the same launch: the QKV kernel with the attention fused in).
// NB: tile buffers per wave -- 1 (each tile loaded after the previous one is used) or 2 (the next
// tile's loads in flight while the current one is used). `issue()` runs once in every wave, right
// after the wave's first
// K/V tile and its q loads are issued (at once in a wave without a tile): loads it issues are
// younger than those, and loads retire in issue order, so waiting for the tile and q does not wait
// for them.
// LCPOL (with COH false): cache policy of the q and K/V loads, kCpolSc0 when q and this position's
// K/V were written earlier in the same launch by workgroups on the same XCD (served by its L2).
template <int HD, int G, int NW, bool COH, int NB, int LCPOL = 0, class Issue>
__device__ __forceinline__ void attn_mfma_waves(const AttnArgs& a, int g, int t_begin, int t_end,
                                                AttnMfmaSmem<HD, G, NW>& sm, Issue issue) {
  static_assert(HD % 32 == 0 && G >= 1 && G <= 8, "head_dim % 32, 1..8 query heads per kv head");
  static_assert(NB == 1 || NB == 2, "tile buffers per wave");
  constexpr int KS = HD / 32, DT = HD / 16;
  constexpr int TS = 32;  // keys per wave tile
  constexpr int CPOL = COH ? kCpolSc1 : LCPOL;
  auto& om = sm.om;
  auto& oml = sm.oml;

  // the wave index in a scalar register: per-wave tile bounds and loop exits are then uniform
  // branches rather than exec-masked ones
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
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
    load_kv_frag<HD, CPOL>(kr, vr, a.msl, t0, col, grp, cur);

    // q as the B operand: column col is head col (hi part) or head col - G (lo part); others zero
    u32x4 qf[KS];
    float smul;  // score scale of this lane's head: 1/sqrt(hd) in log2 units, times 2^-e of the head
    {
      const bool used = col < 2 * G;
      const bool lo = col >= G;
      const int h = used ? (lo ? col - G : col) : 0;
      const float* qp = a.q + (long)(g * G + h) * HD + 8 * grp;
      f32x4 q4[KS][2];
      if constexpr (COH) {
        // descriptor on the kv head's q block (wave-uniform), per-lane byte offsets
        const __amdgpu_buffer_rsrc_t qr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(a.q + (long)g * G * HD), 0, G * HD * (int)sizeof(float), kBufferConfig);
        const int qoff = (h * HD + 8 * grp) * (int)sizeof(float);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          q4[ks][0] = load_shared4(qr, qoff + 128 * ks);
          q4[ks][1] = load_shared4(qr, qoff + 128 * ks + 16);
        }
      } else if constexpr (LCPOL != 0) {
        const __amdgpu_buffer_rsrc_t qr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(a.q + (long)g * G * HD), 0, G * HD * (int)sizeof(float), kBufferConfig);
        const int qoff = (h * HD + 8 * grp) * (int)sizeof(float);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          q4[ks][0] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(qr, qoff + 128 * ks, 0, LCPOL));
          q4[ks][1] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(qr, qoff + 128 * ks + 16, 0, LCPOL));
        }
      } else {
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
        load_kv_frag<HD, CPOL>(kr, vr, a.msl, t0, col, grp, cur);
      }
    } else for (;;) {
      int tn = t0 + TS * NW;
      if (tn >= t_end) {
        tile(cur, t0);
        break;
      }
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0); expcnt and lgkmcnt unconstrained
      load_kv_frag<HD, CPOL>(kr, vr, a.msl, tn, col, grp, nxt);
      __builtin_amdgcn_sched_barrier(0);
      tile(cur, t0);
      t0 = tn;
      tn = t0 + TS * NW;
      if (tn >= t_end) {
        tile(nxt, t0);
        break;
      }
      __builtin_amdgcn_s_waitcnt(0x0F70);
      load_kv_frag<HD, CPOL>(kr, vr, a.msl, tn, col, grp, cur);
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

// One workgroup of NW waves: kv head g, KV slice `split`, all G query heads of g (COH, NB as
// attn_mfma_waves).
template <int HD, int G, int NW, bool COH, int NB = 2>
__device__ __forceinline__ void attn_mfma_body(const AttnArgs& a, int g, int split, const Positions& pss,
                                               AttnMfmaSmem<HD, G, NW>& sm) {
  constexpr int NT = 64 * NW;
  const int tid = threadIdx.x;
  const int kv_len = pss.kv_len;
  const int chunk = attn_mfma_chunk(kv_len, a.nsplit, a.min_slice);
  const int active = (kv_len + chunk - 1) / chunk;
  if (split >= active) return;
  const int t_begin = split * chunk;
  const int t_end = min(kv_len, t_begin + chunk);
  if (pss.kv_sink > 0 && split == 0) {
    rotate_sinks<HD, NT>(a, a.kcache + (long)g * HD * a.msl, pss.kv_sink, tid);
    __syncthreads();
  }
  attn_mfma_waves<HD, G, NW, COH, NB>(a, g, t_begin, t_end, sm, [] {});
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
      a.out[(long)(g * G + h) * HD + d] = O / L;
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
  attn_merge_slices<HD, G, NT, false>(a, g, active, tid, sm.mrg, sm.Ls, sm.last_flag);
}

template <int HD, int G, int NW, int NB = 2>
__global__ void __launch_bounds__(64 * NW) attn_mfma_kernel(AttnArgs a) {
  if ((int)blockIdx.y >= a.nsplit) {
    const int j = ((int)blockIdx.y - a.nsplit) * (int)gridDim.x + (int)blockIdx.x;
    if (j < a.pf.blocks) prefetch_worker<64 * NW>(a.pf, j);
    return;
  }
  __shared__ AttnMfmaSmem<HD, G, NW> sm;
  attn_mfma_body<HD, G, NW, false, NB>(a, blockIdx.x, blockIdx.y, positions(a.params->pos, a.msl), sm);
}

// ------------------------------------------------------------------------------------------
// QKV matvec with the decode attention fused in (short contexts, no sink rotation). Every
// workgroup first streams its rows of [Wq;Wk;Wv] (RMSNorm, clip, RoPE, fp16 K/V at kv_pos;
// q and the K/V entries written through to memory), waits until its stores are complete and counts
// itself done. The attention items -- kv head i % n_kv_heads, slice i / n_kv_heads -- belong to the
// last workgroups of the grid (item i to workgroup nblk - 1 - i): with the rows dealt round-robin
// those hold one row group per wave and finish first. They wait until every workgroup has counted
// itself done (bounded wait: a time-out sets *abort_flag and the host reports an error), then run
// their item. This removes the attention launch, its boundary and its start-up latency.
// done: kQkvDoneParts zeroed counters kQkvDoneStride words apart; workgroup b counts itself on
// counter b % kQkvDoneParts (its XCD), so the completions do not queue behind one address.
// ------------------------------------------------------------------------------------------
constexpr int kQkvDoneParts = 8, kQkvDoneStride = 64;

// Thread 0 polls until the parts of a split counter sum to `target` (bounded, as wait_count).
__device__ __forceinline__ void wait_split_count(const unsigned* c, unsigned target, unsigned* abort_flag) {
  if (threadIdx.x == 0) {
    unsigned spins = 0;
    for (;;) {
      unsigned sum = 0;
#pragma unroll
      for (int k = 0; k < kQkvDoneParts; ++k)
        sum += __hip_atomic_load(const_cast<unsigned*>(c + k * kQkvDoneStride), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (sum >= target) break;
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

template <int KC, int HD, int G>
__global__ void __launch_bounds__(kBlock) qkv_attn_kernel(MatvecArgs m, AttnArgs a, unsigned* done,
                                                          unsigned* abort_flag) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  __shared__ AttnMfmaSmem<HD, G, kWavesPerBlock> sm;
  matvec_body<KC, 2, kEpiQkvRope, false>(m, blockIdx.x, gridDim.x, lds, [] {});
  publish();  // this thread's q / K / V stores have completed
  __syncthreads();
  if (threadIdx.x == 0)
    __hip_atomic_fetch_add(done + (blockIdx.x % kQkvDoneParts) * kQkvDoneStride, 1u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  const Positions pss = positions(a.params->pos, a.msl);
  const int chunk = attn_mfma_chunk(pss.kv_len, a.nsplit, a.min_slice);
  const int items = a.n_kv_heads * ((pss.kv_len + chunk - 1) / chunk);
  const int item = (int)gridDim.x - 1 - (int)blockIdx.x;
  if (item >= items) return;
  wait_split_count(done, gridDim.x, abort_flag);  // every row of q, K and V is written
  attn_mfma_body<HD, G, kWavesPerBlock, true, 1>(a, item % a.n_kv_heads, item / a.n_kv_heads, pss, sm);
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
// The per-row word: bits 0..59 hold the sum of the terms 2^55 + round(p 2^32) added so far (p: one
// workgroup's fp32 partial product for that row, clamped to |p 2^32| <= 2^55 - 2^32, i.e. |p| just
// under 2^23; each term is below 2^56, so up to 15 of them never carry into bit 60), bits 60..63
// count the additions. Every workgroup adds
// its term plus 2^60 with one returning 64-bit atomic; the one whose addition brings the count to
// nkv holds all terms in (returned value + its own), writes x[row] += (sum - nkv 2^55) 2^-32 and
// clears the word for the next launch. Integer addition is associative, so x does not depend on the
// order in which the workgroups' atomics land: the step is bit-reproducible. The fixed-point
// resolution is 2^-32 (2.3e-10) per partial, absolute.
// ------------------------------------------------------------------------------------------
struct AttnOArgs {
  const uint16_t* wo;        // [dim][q_dim]
  float* x;                  // [dim], x += Wo . attn
  unsigned long long* rowacc;  // [dim] combining words, zero between launches
  int dim, q_dim;
  // when not null: the residual stream is row params->token of this fp16 embedding table instead of
  // x (the first layer of the QKV + attention + O launch, which writes x only once, at the end)
  const uint16_t* emb = nullptr;
  const StepParams* params = nullptr;
};

constexpr int kRowAccCountShift = 60;
constexpr unsigned long long kRowAccMask = (1ull << kRowAccCountShift) - 1;
constexpr unsigned long long kRowAccBias = 1ull << 55;
constexpr float kRowAccScale = 4294967296.0f;  // 2^32
constexpr int kRowAccMaxTerms = 15;

// This workgroup's term for one row: 2^60 (the count) + 2^55 + round(p 2^32).
__device__ __forceinline__ unsigned long long rowacc_term(float p) {
  constexpr float kLim = 36028792723996672.0f;  // 2^55 - 2^32, the largest float below 2^55
  float v = rintf(p * kRowAccScale);
  v = fminf(fmaxf(v, -kLim), kLim);
  return (1ull << kRowAccCountShift) + kRowAccBias + (unsigned long long)(long long)v;
}
// The row's fp32 sum from a completed word (count n): (value bits - n 2^55) 2^-32.
__device__ __forceinline__ float rowacc_sum(unsigned long long w, int n) {
  const long long v = (long long)(w & kRowAccMask) - (long long)n * (long long)kRowAccBias;
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
    const float xr = o.emb ? (float)__builtin_bit_cast(f16, o.emb[(long)o.params->token * o.dim + row]) : o.x[row];
    const unsigned long long term = rowacc_term(mine);
    const unsigned long long old =
        __hip_atomic_fetch_add(o.rowacc + row, term, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const unsigned long long w = old + term;
    if ((int)(w >> kRowAccCountShift) == nkv) {  // the last of the row's nkv terms
      o.x[row] = xr + rowacc_sum(w, nkv);
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
  attn_mfma_waves<HD, G, NW, false, 1>(a, g, 0, kv_len, sm, [&] { attn_o_issue<HD, G, NW, U>(o, g, row0, lane, wv); });

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
// (kv head g = b % nkv, rows as attn_o_kernel) requests kv head g's partial block (G heads x nsplit
// slices x (HD + 2) floats, at most kMergeOMaxSplits slices) into registers before its Wo block,
// merges out_h = sum_s w_s o_s / sum_s w_s l_s with w_s = exp(m_s - max_s m_s) while the Wo
// stream is in flight (reference src/infer.cpp:172-187,218-250: one softmax over all keys,
// restated over slices), then multiplies and combines rows as attn_o_kernel.
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
  const Positions pss = positions(a.params->pos, a.msl);
  const int chunk = attn_mfma_chunk(pss.kv_len, a.nsplit, a.min_slice);
  const int active = (pss.kv_len + chunk - 1) / chunk;  // as the attention launch counted them

  // kv head g's partials: rows (g G + h) nsplit + s of HD + 2 floats, one block (reads past it
  // return zero). Straight into registers, before the Wo loads, so waiting for them leaves the Wo
  // stream in flight: wave h < G takes (m, l) of slice s in lane s; every thread takes, for its
  // output element (h, d), the d column of head h's active slices.
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
  u32x4 wv[U];
  attn_o_issue<HD, G, NW, U>(o, g, row0, lane, wv);
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

namespace yk {
// ------------------------------------------------------------------------------------------
// QKV, attention and the O projection in one launch (short contexts, no sink rotation),
// reference src/infer.cpp:279-344, for shapes with one kv head per XCD (n_kv_heads == 8): the
// dispatcher deals a launch's workgroups to the 8 XCDs round-robin, workgroup b to XCD (s + b) % 8
// for a start s that depends on earlier launches.
//
// Workgroup b takes kv head g = b % nkv and row block rb = b / nkv, so all of kv head g's
// workgroups run on one XCD and what they hand to each other stays in that XCD's L2. Twelve waves in
// two roles:
//   - waves 8..11 issue their 32 Wo row segments (kv head g's columns of rows rb*128 + 32(w-8) ..)
//     early and hold them in registers; they take part in the workgroup barriers until the
//     attention output is in LDS, then multiply and combine the rows as attn_o_kernel does;
//   - waves 0..7 stage x (RMSNorm, reference src/infer.cpp:136-146; the embedding row in the
//     first layer) and stream rb's share of kv head g's rows of [Wq;Wk;Wv] (G*HD q rows, HD k and
//     HD v rows, as row pairs: up to two per wave, the second issued once x is staged) with the
//     matvec's QKV epilogue
//     (clip, RoPE, q and this position's fp16 K/V). A workgroup whose rows are stored counts itself
//     on kv head g's counter; once all of kv head g's workgroups have (bounded wait), waves 0..7 run
//     the whole-context MFMA attention of kv head g, reading q and the caches through the XCD's L2
//     (sc0 loads), and put the normalised output into LDS.
// The roles keep each wave's loads in one stream: loads return in issue order, so attention loads
// queued behind Wo loads would wait for the Wo block, and a wave that stored rows could not wait
// for its stores without also waiting for Wo loads issued before them.
// Each workgroup counts itself as 2^(6 x) on its kv head's 64-bit counter (x: the XCD it runs on,
// from the XCC_ID register) and waits for exactly 2^(6 x) times the head's workgroup count, so a
// head whose workgroups are not all on the waiting workgroup's XCD never completes the wait: it
// times out and the host reports an error for the step instead of reading another L2's data. The
// host enables the launch only after a probe launch of the same grid found the round-robin order,
// and only when the grid fits the GPU at one workgroup per CU (every workgroup of a kv head must be
// resident while the others wait for it).
// ------------------------------------------------------------------------------------------
constexpr int kQaoRowWaves = 8, kQaoWoWaves = 4, kQaoWoLoads = 32, kQaoPairsPerWave = 2, kQaoXcds = 8;

struct QaoArgs {
  // kv head g: 64-bit count of its workgroups whose rows are stored, 2^(6 XCD) each, at
  // done[g * kQkvDoneStride] (zeroed every step)
  unsigned* done;
  unsigned* abort_flag;  // a wait timed out
  int blocks_per_head;   // workgroups per kv head (Wo row blocks), below 64
  int wo_after;          // the Wo waves issue their loads after this many of the workgroup's barriers (0..5)
};

// Thread 0 polls until the 64-bit word *c equals target (bounded, as wait_count); the workgroup
// waits at the barrier.
__device__ __forceinline__ void wait_word(const unsigned long long* c, unsigned long long target, unsigned* abort_flag) {
  if (threadIdx.x == 0) {
    unsigned spins = 0;
    while (__hip_atomic_load(const_cast<unsigned long long*>(c), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != target) {
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

__device__ __forceinline__ unsigned xcc_id() {
  unsigned v;
  __asm__ volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return v & 0xfu;
}

// LDS writes of this wave complete, then the workgroup barrier (no wait for global accesses).
__device__ __forceinline__ void lds_barrier() {
  __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  __asm__ volatile("" ::: "memory");
}

template <int HD, int G>
__global__ void __launch_bounds__(64 * (kQaoRowWaves + kQaoWoWaves)) qao_kernel(MatvecArgs m, AttnArgs a, AttnOArgs o,
                                                                                 QaoArgs z) {
  constexpr int NR = kQaoRowWaves, NT = 64 * NR, KC = 8, K = 512 * KC, NPT = K / (4 * NT);  // K 4096: 2 float4 per row thread
  constexpr int QP = G * HD / 2, KP = HD / 2, NP = QP + 2 * KP;                          // row pairs of one kv head
  using Geo = AttnOGeom<HD, G, kQaoWoWaves, kQaoWoLoads>;
  static_assert(NPT * 4 * NT == K, "x staging: whole float4 per row thread");
  __shared__ AttnMfmaSmem<HD, G, NR> sm;
  __shared__ __attribute__((aligned(16))) float xs[K + HD];  // normalised x, then the step's RoPE table
  __shared__ __attribute__((aligned(16))) float ao[G * HD];
  __shared__ float red[NR];
  __shared__ float rs[kQaoWoWaves][Geo::RW];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nkv = a.n_kv_heads;
  const int g = (int)blockIdx.x % nkv, rb = (int)blockIdx.x / nkv;

  if (wave >= NR) {  // Wo waves
    const int ww = wave - NR;
    const int row0 = rb * Geo::RB + ww * Geo::RW;
    u32x4 wv[kQaoWoLoads];
    // the row waves' six barriers (staging sums, staged input, rows stored, kv head's rows
    // complete, attention outputs, normalised output); the Wo loads go out after wo_after of them
    // (the row waves' first loads then meet fewer bytes ahead of them) and stay in flight
#pragma unroll
    for (int k = 0; k < 6; ++k) {
      if (k == z.wo_after) attn_o_issue<HD, G, kQaoWoWaves, kQaoWoLoads>(o, g, row0, lane, wv);
      __builtin_amdgcn_s_barrier();
    }
    __asm__ volatile("" ::: "memory");
    attn_o_rows<HD, G, kQaoWoWaves, kQaoWoLoads>(o, ao, rs, wv, row0, lane, ww, nkv);
    return;
  }

  // row waves: the staging reads first, then the first two row pairs' weight loads
  const int pos = m.params->pos;
  const uint16_t* x16 = m.emb ? m.emb + (long)m.params->token * K : nullptr;
  f32x4 xv[NPT], gv[NPT];
  unsigned long long hv[NPT];
  if (x16) {
    const unsigned long long* h4 = reinterpret_cast<const unsigned long long*>(x16);
#pragma unroll
    for (int k = 0; k < NPT; ++k) hv[k] = h4[tid + NT * k];
  } else {
    const f32x4* x4 = reinterpret_cast<const f32x4*>(m.x);
#pragma unroll
    for (int k = 0; k < NPT; ++k) xv[k] = x4[tid + NT * k];
  }
  const f32x4* g4 = reinterpret_cast<const f32x4*>(m.gain);
#pragma unroll
  for (int k = 0; k < NPT; ++k) gv[k] = g4[tid + NT * k];
  const float rc = tid < HD ? m.rope_cs[tid] : 0.f;

  const int ppb = (NP + z.blocks_per_head - 1) / z.blocks_per_head;
  auto pair_of = [&](int k, bool& valid) {  // this workgroup's k-th row pair of kv head g, as a [Wq;Wk;Wv] pair
    const int j = rb * ppb + k;
    valid = k < ppb && j < NP;
    if (!valid) return 0;
    if (j < QP) return g * QP + j;
    if (j < QP + KP) return m.q_dim / 2 + g * KP + (j - QP);
    return (m.q_dim + m.kv_dim) / 2 + g * KP + (j - QP - KP);
  };
  bool v0, v1;
  const int p0 = pair_of(wave, v0), p1 = pair_of(wave + NR, v1);
  u32x4 wa[2][KC], wb[2][KC];
  auto issue = [&](u32x4 (&wv)[2][KC], int p, bool valid) {
    const uint16_t* rows[2];
    group_rows<2>(m, p, rows);
    load_group_uniform<KC, 2>(wv, rows, lane, valid);
  };
  issue(wa, p0, v0);

  // RMSNorm into LDS
  if (x16) {
#pragma unroll
    for (int k = 0; k < NPT; ++k)
#pragma unroll
      for (int e = 0; e < 4; ++e) xv[k][e] = (float)__builtin_bit_cast(f16, (uint16_t)(hv[k] >> (16 * e)));
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < NPT; ++k)
    ss += xv[k][0] * xv[k][0] + xv[k][1] * xv[k][1] + xv[k][2] * xv[k][2] + xv[k][3] * xv[k][3];
  ss = wave_sum(ss);
  if (lane == 0) red[wave] = ss;
  lds_barrier();  // 1
  ss = 0.f;
#pragma unroll
  for (int w = 0; w < NR; ++w) ss += red[w];
  const float inv = 1.0f / sqrtf(ss / (float)K + m.eps);
  f32x4* o4 = reinterpret_cast<f32x4*>(xs);
#pragma unroll
  for (int k = 0; k < NPT; ++k) {
    f32x4 v;
    v[0] = xv[k][0] * inv * gv[k][0];
    v[1] = xv[k][1] * inv * gv[k][1];
    v[2] = xv[k][2] * inv * gv[k][2];
    v[3] = xv[k][3] * inv * gv[k][3];
    o4[tid + NT * k] = v;
  }
  if (tid < HD) xs[K + tid] = rc;
  lds_barrier();  // 2
  issue(wb, p1, v1);  // the second pair after the staging: its reads then queue behind fewer bytes

  const float none[2] = {0.f, 0.f};
  auto use = [&](const u32x4 (&wv)[2][KC], int p, bool valid) {
    float acc[2] = {0.f, 0.f};
#pragma unroll
    for (int u = 0; u < KC; ++u) {
#pragma unroll
      for (int r = 0; r < 2; ++r) acc[r] = dot8(wv[r][u], xs + 8 * (lane + kWave * u), acc[r]);
      if ((u & 3) == 3) __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) acc[r] = wave_sum(acc[r]);
    epilogue<2, kEpiQkvRope, false>(m, p, acc, none, pos, xs + K, valid && lane == 0);
  };
  use(wa, p0, v0);
  use(wb, p1, v1);
  publish();  // this thread's q / K / V stores are in the L2
  __builtin_amdgcn_s_barrier();  // 3
  __asm__ volatile("" ::: "memory");
  unsigned long long* done = reinterpret_cast<unsigned long long*>(z.done + (long)g * kQkvDoneStride);
  const unsigned long long mine = 1ull << (6 * xcc_id());
  if (tid == 0) __hip_atomic_fetch_add(done, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  wait_word(done, mine * (unsigned)z.blocks_per_head, z.abort_flag);  // 4: every row of kv head g is stored

  attn_mfma_waves<HD, G, NR, false, 1, kCpolSc0>(a, g, 0, pos + 1, sm, [] {});  // 5 (its closing barrier)
  for (int e = tid; e < G * HD; e += NT) {
    const int h = e / HD, d = e % HD;
    float M = kNegBig;
#pragma unroll
    for (int w = 0; w < NR; ++w) M = fmaxf(M, sm.oml[w][h][0]);
    float O = 0.f, L = 0.f;
#pragma unroll
    for (int w = 0; w < NR; ++w) {
      const float wt = exp2_fast(sm.oml[w][h][0] - M);
      O = fmaf(sm.om[w][h][d], wt, O);
      L = fmaf(sm.oml[w][h][1], wt, L);
    }
    ao[e] = O / L;
  }
  lds_barrier();  // 6
}

// Workgroup b records the XCD it runs on (the round-robin order qao_kernel relies on).
__global__ void __launch_bounds__(512) xcc_probe_kernel(unsigned* out) {
  if (threadIdx.x == 0) out[blockIdx.x] = xcc_id();
}
}  // namespace yk

namespace yk {
// ------------------------------------------------------------------------------------------
// Split-KV attention, slice merge and the O projection in one launch (contexts beyond attn_o's,
// no sink rotation; reference src/infer.cpp:218-250, 327-344), for shapes with one kv head per
// XCD (n_kv_heads == 8, the dispatcher's round-robin order as qao_kernel relies on it).
//
// Workgroup b takes kv head g = b % nkv and Wo row block rb = b / nkv, as attn_o_kernel; the
// workgroups also take one KV slice each (keys [rb c, rb c + c), c = kv_len / NS rounded up to
// the 32-key tile, NS = the head's workgroup count; the last ones may hold no keys). All of kv
// head g's workgroups run on one XCD, so what they hand to each other meets in its L2. A slice
// workgroup (one whose slice holds keys) issues its first K/V tile and q, then its Wo block, runs
// the MFMA attention over its slice and stores the slice's (o, m, l) (m in natural units, as the
// split-KV partials) with plain stores, then counts itself on kv head g's counter with
// qao_kernel's XCD-weighted term (2^(6 x); the wait is for exactly the slice count times the own
// term, so a head split across XCDs times out and the host reports an error). Every workgroup reads
// the head's NS partials with sc0 loads into LDS, merges them (out_h = sum_s w_s o_s /
// sum_s w_s l_s, w_s = exp(m_s - max m)) and multiplies and combines its Wo rows as
// attn_o_kernel. The wait for a slice's partial stores also waits for the wave's Wo loads issued
// before them (loads and stores retire in issue order); by then the Wo stream has mostly landed.
// ------------------------------------------------------------------------------------------
constexpr int kSliceOMaxSlices = 32;  // KV slices per kv head (the partial block in LDS holds this many)

struct SliceOArgs {
  unsigned* done;        // kv head g: 64-bit XCD-weighted count at done[g * kQkvDoneStride] (zeroed every step)
  unsigned* abort_flag;  // a wait timed out
  int slices;            // KV slices per kv head: the head's workgroup count, at most kSliceOMaxSlices
};

template <int HD, int G, int NW, int U>
__global__ void __launch_bounds__(64 * NW) slice_o_kernel(AttnArgs a, AttnOArgs o, SliceOArgs z) {
  using Geo = AttnOGeom<HD, G, NW, U>;
  constexpr int RW = Geo::RW, NT = 64 * NW, NSMAX = kSliceOMaxSlices, ST = HD + 2;
  constexpr int PB = G * NSMAX * ST, PPT = (PB / 4 + NT - 1) / NT;  // partial block floats, float4 per thread
  static_assert(ST % 2 == 0 && NSMAX <= 64, "partial rows");
  __shared__ AttnMfmaSmem<HD, G, NW> sm;
  __shared__ __attribute__((aligned(16))) float pb[PB];
  __shared__ float wts[G][NSMAX];
  __shared__ float linv[G];
  __shared__ __attribute__((aligned(16))) float ao[G * HD];
  __shared__ float rs[NW][RW];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nkv = a.n_kv_heads;
  const int g = (int)blockIdx.x % nkv, rb = (int)blockIdx.x / nkv;
  const int row0 = rb * Geo::RB + wave * RW;
  const int kv_len = min(a.params->pos + 1, a.msl);  // the host runs this kernel only for pos < msl
  const int ns = z.slices;
  const int chunk = ((kv_len + ns - 1) / ns + 31) / 32 * 32;
  const int active = (kv_len + chunk - 1) / chunk;  // slices holding keys (at most ns)
  float* part = a.partial + (long)g * G * a.nsplit * ST;  // rows (h nsplit + s) of ST floats
  unsigned long long* done = reinterpret_cast<unsigned long long*>(z.done + (long)g * kQkvDoneStride);
  const unsigned long long mine = 1ull << (6 * xcc_id());

  u32x4 wv[U];
  if (rb < active) {
    const int t_begin = rb * chunk, t_end = min(kv_len, t_begin + chunk);
    attn_mfma_waves<HD, G, NW, false, 1>(a, g, t_begin, t_end, sm,
                                         [&] { attn_o_issue<HD, G, NW, U>(o, g, row0, lane, wv); });
    // this slice's partial: the waves' (m, l, o) combined
    for (int e = tid; e < G * HD; e += NT) {
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
      float* dst = part + (long)(h * a.nsplit + rb) * ST;
      dst[d] = O;
      if (d == 0) {
        dst[HD] = M * kLn2;  // natural units, as the split-KV partials
        dst[HD + 1] = L;
      }
    }
    publish();  // this thread's partial stores are in the L2 (and its Wo loads have landed)
    __syncthreads();
    if (tid == 0) __hip_atomic_fetch_add(done, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    attn_o_issue<HD, G, NW, U>(o, g, row0, lane, wv);
  }
  wait_word(done, mine * (unsigned)active, z.abort_flag);  // every slice of kv head g is stored

  // kv head g's partial block (rows h nsplit + s, s < active), read through the L2 into LDS:
  // every load issued before the first use
  const int nfl = G * a.nsplit * ST;
  const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(part, 0, nfl * (int)sizeof(float), kBufferConfig);
  f32x4 pv[PPT];
#pragma unroll
  for (int k = 0; k < PPT; ++k) {
    const int f = 4 * (tid + NT * k);  // float index in the block; chunks wholly in slices >= active are not read
    const bool want = f < nfl && ((f / ST) % a.nsplit < active || ((f + 3) / ST) % a.nsplit < active);
    pv[k] = want ? __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(pr, 4 * f, 0, kCpolSc0))
                 : f32x4{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int k = 0; k < PPT; ++k)
    if (4 * (tid + NT * k) < nfl) *reinterpret_cast<f32x4*>(pb + 4 * (tid + NT * k)) = pv[k];
  __syncthreads();
  // per head (one wave each): the slices' weights relative to the largest maximum, 1 / sum_s w_s l_s
  for (int i = tid; i < G * 64; i += NT) {
    const int h = i / 64, s = i % 64;
    const float* row = pb + (h * a.nsplit + s) * ST;
    const float m = s < active ? row[HD] : kNegBig;
    const float M = wave_max(m);
    const float w = s < active ? expf(m - M) : 0.f;
    const float L = wave_sum(s < active ? w * row[HD + 1] : 0.f);
    if (s < NSMAX) wts[h][s] = w;
    if (s == 0) linv[h] = 1.0f / L;
  }
  __syncthreads();
  for (int e = tid; e < G * HD; e += NT) {
    const int h = e / HD, d = e % HD;
    float O = 0.f;
    for (int s = 0; s < active; ++s) O = fmaf(wts[h][s], pb[(h * a.nsplit + s) * ST + d], O);
    ao[e] = O * linv[h];
  }
  __syncthreads();
  attn_o_rows<HD, G, NW, U>(o, ao, rs, wv, row0, lane, wave, nkv);
}
}  // namespace yk
