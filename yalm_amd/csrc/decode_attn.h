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

// One workgroup of NW waves: kv head g, KV slice `split`, all G query heads of g. COH: q and the
// K/V entries are read with agent-coherent loads (they were written by other workgroups of the same
// launch: the QKV kernel with the attention fused in). DB: two tile buffers per wave.
template <int HD, int G, int NW, bool COH, bool DB = true>
__device__ __forceinline__ void attn_mfma_body(const AttnArgs& a, int g, int split, const Positions& pss,
                                               AttnMfmaSmem<HD, G, NW>& sm) {
  static_assert(HD % 32 == 0 && G >= 1 && G <= 8, "head_dim % 32, 1..8 query heads per kv head");
  constexpr int NT = 64 * NW;
  constexpr int KS = HD / 32, DT = HD / 16;
  constexpr int TS = 32;  // keys per wave tile
  constexpr int CPOL = COH ? kCpolSc1 : 0;
  auto& om = sm.om;
  auto& oml = sm.oml;

  // the wave index in a scalar register: per-wave tile bounds and loop exits are then uniform
  // branches rather than exec-masked ones
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, grp = lane >> 4;
  const int kv_len = pss.kv_len;
  const int chunk = attn_mfma_chunk(kv_len, a.nsplit, a.min_slice);
  const int active = (kv_len + chunk - 1) / chunk;
  if (split >= active) return;
  const int t_begin = split * chunk;
  const int t_end = min(kv_len, t_begin + chunk);
  const long head_off = (long)g * HD * a.msl;
  uint16_t* kh = a.kcache + head_off;
  const uint16_t* vh = a.vcache + head_off;
  const int head_bytes = HD * a.msl * 2;
  const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(kh, 0, head_bytes, kBufferConfig);
  const __amdgpu_buffer_rsrc_t vr =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(vh), 0, head_bytes, kBufferConfig);
  if (pss.kv_sink > 0 && split == 0) {
    rotate_sinks<HD, NT>(a, kh, pss.kv_sink, tid);
    __syncthreads();
  }

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
      } else {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          q4[ks][0] = *reinterpret_cast<const f32x4*>(qp + 32 * ks);
          q4[ks][1] = *reinterpret_cast<const f32x4*>(qp + 32 * ks + 4);
        }
      }
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
    // Two register buffers used alternately (unrolled by two, no copies between them): while one
    // tile is used the next one's loads are in flight, and the scheduling barrier keeps them at the
    // top. The explicit wait for the current tile is free in the steady state and keeps the
    // compiler from waiting on the in-flight tile inside the current one. DB false: one buffer,
    // each tile loaded after the previous one is used (fewer registers, for short slices).
    if constexpr (!DB) {
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
    if (active == 1) {
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
  if (active == 1) return;
  attn_merge_slices<HD, G, NT, false>(a, g, active, tid, sm.mrg, sm.Ls, sm.last_flag);
}

template <int HD, int G, int NW>
__global__ void __launch_bounds__(64 * NW) attn_mfma_kernel(AttnArgs a) {
  if ((int)blockIdx.y >= a.nsplit) {
    const int j = ((int)blockIdx.y - a.nsplit) * (int)gridDim.x + (int)blockIdx.x;
    if (j < a.pf.blocks) prefetch_worker<64 * NW>(a.pf, j);
    return;
  }
  __shared__ AttnMfmaSmem<HD, G, NW> sm;
  attn_mfma_body<HD, G, NW, false>(a, blockIdx.x, blockIdx.y, positions(a.params->pos, a.msl), sm);
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
  attn_mfma_body<HD, G, kWavesPerBlock, true, false>(a, item % a.n_kv_heads, item / a.n_kv_heads, pss, sm);
}
}  // namespace yk
