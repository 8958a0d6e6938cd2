// Single-launch decode step for gfx950: one persistent launch computes a whole token.
//
// One workgroup per CU, eight waves each, all resident at once (a cooperative launch). The
// workgroups walk the step's phases together, with a grid barrier between phases:
//   per layer  QKV   rmsnorm(x) -> [Wq;Wk;Wv] -> clip, RoPE -> q, fp16 K/V into the cache
//              ATT   split-KV GQA attention on the matrix cores, one (kv head, slice) per workgroup
//              O     x += Wo att
//              W13   rmsnorm(x) -> act(W1 x) * (W3 x) -> hb
//              W2    x += W2 hb
//   then       LM    final rmsnorm, logits, greedy argmax (a packed key, one atomic max per workgroup)
// Arithmetic follows reference src/infer.cpp:256-527; what one step launches, src/infer.cu:1274-1378
// and src/coop.cu:179-322 (the reference's own one-launch step).
//
// Rows. A matvec phase's rows come in groups of two pieces of at most 16 KB: two rows (QKV, O,
// lm_head: the row pair p = 2i, 2i+1 that RoPE rotates together), row i of W1 and of W3 (W13), or
// the two halves of row i (W2). The groups are dealt to the workgroups in turn (b, b + nb, ...)
// and a workgroup's to its waves in turn (every CU gets the same share of bytes). A piece is PL
// buffer loads of 16 bytes per lane (1 KB per wave instruction, streaming), and a wave holds two:
// the next piece's loads go out before the current one is used, so each wave keeps one piece in
// flight while it computes.
//
// Barrier. Each workgroup owns one arrival flag. After its last group a wave issues the loads of
// its first group of the next matvec phase (weights depend on nothing), waits only until its own
// stores of this phase have completed (loads and stores retire in issue order), and arrives at the
// workgroup barrier. Wave 7 (the poll wave) then writes the workgroup's flag with a write-through
// store, reads all flags with coherent loads until every one shows the phase, stages the next
// phase's input vector into LDS (coherent direct-to-LDS loads, then the RMS normalisation in
// place), and releases the workgroup. The streaming waves' next loads stay in flight across the
// barrier; the poll wave issues its own first group after staging. No atomics: 256 arrivals on one
// counter serialise at the memory side (~12 ns each), flags do not. Every wait is bounded; a
// time-out sets the abort word, after which no barrier waits, and the host reports the error.
//
// Coherence (each XCD has its own L2): everything one workgroup hands to another within the launch
// (x, q, att, hb, the current position's K/V, the attention partials) is written with write-through
// (agent-scope) stores and read with agent-coherent (sc1) loads. K/V of earlier positions and the
// weights were written before the launch.
#pragma once
#include "decode_attn.h"

namespace yk {

// All layers share one layout: layer l's weights start at wbase + l * stride, its K cache at
// kv + 2 l kv_elems and its V cache right after.
struct LayerLayout {
  const char* wbase;
  long stride;
  long o_qkv, o_wo, o_w1, o_w3, o_w2, o_ra, o_rf;
  uint16_t* kv;
  long kv_elems;
};

constexpr int kStepWaves = 8;
constexpr int kStepThreads = kStepWaves * kWave;
constexpr int kPollWave = kStepWaves - 1;
constexpr int kStepMaxBlocks = 256;  // arrival flags: one 16-byte load per lane reads them all
constexpr int kStepPhaseStride = 1024;  // flag values one launch may use (phases + 1)

// Sync words: the abort word, then the arrival flags (one per workgroup, packed).
constexpr int kSyncAbort = 0, kSyncFlags = 64;
constexpr int kSyncWords = kSyncFlags + kStepMaxBlocks;

struct StepArgs {
  LayerLayout layers;
  const uint16_t* embed;
  const uint16_t* wcls;
  const float* rms_final;
  const float* inv_freq;  // [head_dim / 2]
  float* x;
  float* q;
  float* att;
  float* hb;
  float* logits;
  float* partial;
  unsigned* tickets;         // attention merge tickets [n_kv_heads], zero between launches
  unsigned long long* rowacc;  // [dim] combining words of the fused attention + O phase, zero between phases
  float* rowovf;               // [dim] their fp32 side sums, zero between phases
  unsigned* sync;            // kSyncWords
  unsigned long long* keys;  // [2] packed argmax keys: launch e posts to keys[e & 1], zeroes the other
  int n_layers, dim, hidden, q_dim, kv_dim, n_heads, n_kv_heads, vocab, msl;
  int token, pos, mode, nsplit;
  int act;
  float eps, qkv_clip;
  unsigned base;   // flag value before this launch's first phase (increases by kStepPhaseStride)
  unsigned spin_limit;  // polls before a barrier wait gives up (sets the abort word)
  unsigned parity; // launch parity (argmax key)
};

// ---- the matvec phases ----------------------------------------------------------------------

enum StepPhase : int { kPhQkv = 0, kPhAtt = 1, kPhO = 2, kPhW13 = 3, kPhW2 = 4, kPhasesPerLayer = 5, kPhLm = 5 };

// Where a phase's groups lie: group i's piece 0 starts at w0 + i gstride, piece 1 at
// w1 + i gstride; each piece is pbytes long and multiplies the staged input at offset 0 (piece 0)
// or xo1 (piece 1). pre: the residual operand of group i (2 floats of x at pre_base + i pre_step,
// or, in layer 0, 2 fp16 of the embedding row, which x equals there), or none.
struct PhaseMap {
  const uint16_t* w0;
  const uint16_t* w1;
  long gstride;
  int pbytes;
  int xo1;
  int groups;
  const void* pre_base;
  int pre_step;   // bytes per group
  int pre_bytes;  // 0: no residual operand
  int pre_half;   // the operand is fp16 (embedding row)
};

// Two pieces and the residual operand of one group of one wave.
template <int PLMAX>
struct GroupRegs {
  u32x4 a[PLMAX], b[PLMAX];
  uint32_t pre[2];
};

// A buffer descriptor for bytes [off, n) of p (none past n).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_from(const void* p, int off, int n) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(static_cast<const char*>(p)) + off, 0, n > off ? n - off : 0,
                                           kBufferConfig);
}

// PL loads of 16 bytes per lane from a piece of `bytes` bytes at p (load u: bytes 1024 u + 16 lane).
// Loads past the piece read zero without a memory access: the range check covers the vector and
// instruction offsets only (not the scalar one), so each 4 KB of the piece gets its own descriptor
// and the offsets within it stay in the checked fields.
template <int PL>
__device__ __forceinline__ void issue_piece(u32x4* w, const uint16_t* p, int bytes, int lane) {
#pragma unroll
  for (int k = 0; k < (PL + 3) / 4; ++k) {
    const __amdgpu_buffer_rsrc_t rs = rsrc_from(p, 4096 * k, bytes);
#pragma unroll
    for (int u = 4 * k; u < PL && u < 4 * k + 4; ++u)
      w[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, lane * 16 + (u - 4 * k) * 1024, 0, kCpolNt));
  }
}

// The residual operand: the two dwords at pre_base + g pre_step (coherent loads; each returns zero
// past pre_bytes, and both when there is no operand).
constexpr int kPreLoads = 2;
__device__ __forceinline__ void issue_pre(const PhaseMap& m, int g, bool valid, uint32_t (&pre)[2]) {
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(m.pre_base), 0, valid ? m.pre_bytes : 0, kBufferConfig);
  const int off = valid ? g * m.pre_step : 0;
  pre[0] = __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, kCpolSc1);
  pre[1] = __builtin_amdgcn_raw_buffer_load_b32(rs, off + 4, 0, kCpolSc1);
}

// Piece 0, the residual operand, piece 1 of group g (in this order); all loads are issued (zero-size
// descriptors when !valid), so the compiler's wait counts do not depend on a branch.
template <int PL, int PLMAX>
__device__ __forceinline__ void issue_group(const PhaseMap& m, int g, bool valid, GroupRegs<PLMAX>& r, int lane) {
  const long off = valid ? (long)g * m.gstride : 0;
  issue_piece<PL>(r.a, m.w0 + off, valid ? m.pbytes : 0, lane);
  issue_pre(m, g, valid, r.pre);
  issue_piece<PL>(r.b, m.w1 + off, valid ? m.pbytes : 0, lane);
}

// The groups of wave w of workgroup b: g0, g0 + step, ... (n of them). The groups are dealt to the
// workgroups in turn (b, b + nb, b + 2 nb, ...) and a workgroup's to its waves in turn, so every
// workgroup gets the same number of groups to within one (contiguous row blocks per workgroup
// measured 3.32 against 3.24 ms per token).
struct WaveShare {
  int g0, step, n;
};
__device__ __forceinline__ WaveShare wave_share(int groups, int b, int nb, int wave) {
  WaveShare s;
  s.g0 = b + nb * wave;
  s.step = nb * kStepWaves;
  s.n = s.g0 < groups ? (groups - 1 - s.g0) / s.step + 1 : 0;
  return s;
}

// The first group of this wave in phase m (issued when `want` and the wave has one).
template <int PL, int PLMAX>
__device__ __forceinline__ void issue_first(const PhaseMap& m, bool want, GroupRegs<PLMAX>& r, int b, int nb, int wave,
                                            int lane) {
  const WaveShare ws = wave_share(m.groups, b, nb, wave);
  issue_group<PL>(m, ws.g0, want && ws.n > 0, r, lane);
}

// This lane's share of one piece's dot product with the staged input.
template <int PL, int PLMAX>
__device__ __forceinline__ float piece_dot(const u32x4 (&w)[PLMAX], const float* xs, int lane) {
  float acc = 0.f;
#pragma unroll
  for (int u = 0; u < PL; ++u) {
    acc = dot8(w[u], xs + 8 * (lane + kWave * u), acc);
    __builtin_amdgcn_sched_barrier(0);  // one slice of x in registers at a time
  }
  return acc;
}

// s_waitcnt vmcnt(n), other counters unconstrained (gfx9 encoding: vmcnt bits 3:0 and 15:14).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

// Workgroup barrier without the memory fences of __syncthreads (which would wait for every
// outstanding load): LDS writes are complete first; the clobber keeps the compiler from moving
// memory accesses across it.
__device__ __forceinline__ void wg_barrier() { __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

struct StepEpi {
  int layer;
  int hd;
  Positions ps;
  uint16_t* kc;
  uint16_t* vc;
};

// Epilogue of group g of phase KIND with the wave totals: rows 2g, 2g+1 (QKV, O, lm_head), hb[g]
// (W13), x[g] (W2). Every lane computes, lane 0 stores.
template <int KIND>
__device__ __forceinline__ void step_epilogue(const StepArgs& a, const StepEpi& e, int g, float s0, float s1,
                                              const uint32_t (&pre)[2], const float* rope_cs, RowMax& mx,
                                              int lane) {
  const bool st = lane == 0;
  switch (KIND) {
    case kPhQkv: {  // reference src/infer.cpp:279-305
      const int i = 2 * g;
      float v0 = clipf(s0, a.qkv_clip), v1 = clipf(s1, a.qkv_clip);
      if (i < a.q_dim + a.kv_dim) {  // RoPE on q and k (reference src/infer.cpp:202-215)
        const int j = i % e.hd;
        const float c = rope_cs[j], s = rope_cs[j + 1];
        const float r0 = v0 * c - v1 * s;
        const float r1 = v0 * s + v1 * c;
        v0 = r0;
        v1 = r1;
      }
      if (!st) return;
      if (i < a.q_dim) {
        store_shared(a.q + i, v0);
        store_shared(a.q + i + 1, v1);
        return;
      }
      const int hd = e.hd;
      const bool is_k = i < a.q_dim + a.kv_dim;
      const int ik = i - a.q_dim - (is_k ? 0 : a.kv_dim);
      const int kh = ik / hd, j = ik % hd;
      const long head = (long)kh * hd * a.msl;
      const uint16_t h0 = __builtin_bit_cast(uint16_t, (f16)v0);  // RNE, as _cvtss_sh(x, 0)
      const uint16_t h1 = __builtin_bit_cast(uint16_t, (f16)v1);
      if (is_k) {  // j, j + 1 are adjacent in the 16-dim tile: one 32-bit store
        store_shared_u32(reinterpret_cast<uint32_t*>(e.kc + head + k_cache_idx(j, e.ps.kv_pos, a.msl)),
                         (uint32_t)h0 | ((uint32_t)h1 << 16));
      } else {
        __hip_atomic_store(e.vc + head + (long)j * a.msl + e.ps.kv_pos, h0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(e.vc + head + (long)(j + 1) * a.msl + e.ps.kv_pos, h1, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
      return;
    }
    case kPhO: {  // reference src/infer.cpp:339-344
      float x0, x1;
      if (e.layer == 0) {  // x is the embedding row there (src/infer.cpp:460-481)
        x0 = (float)__builtin_bit_cast(f16, (uint16_t)(pre[0] & 0xffff));
        x1 = (float)__builtin_bit_cast(f16, (uint16_t)(pre[0] >> 16));
      } else {
        x0 = __uint_as_float(pre[0]);
        x1 = __uint_as_float(pre[1]);
      }
      if (st) {
        store_shared(a.x + 2 * g, x0 + s0);
        store_shared(a.x + 2 * g + 1, x1 + s1);
      }
      return;
    }
    case kPhW13: {  // reference src/infer.cpp:349-382
      const float h = a.act == 1 ? silu(s0) : gelu(s0);
      if (st) store_shared(a.hb + g, h * s1);
      return;
    }
    case kPhW2:  // reference src/infer.cpp:384-390 (s0: the whole row's sum)
      if (st) store_shared(a.x + g, __uint_as_float(pre[0]) + s0);
      return;
    default:  // lm_head (src/infer.cpp:523-527) and the argmax's running maximum (src/sampler.cpp:27-38)
      if (st) {
        a.logits[2 * g] = s0;
        a.logits[2 * g + 1] = s1;
      }
      if (s0 > kNegBig) better(mx.v, mx.i, s0, 2 * g);
      if (s1 > kNegBig) better(mx.v, mx.i, s1, 2 * g + 1);
      return;
  }
}

// One wave's part of a matvec phase. `primed`: the first group's loads were issued before the
// barrier (by the previous phase); otherwise they are issued here. Each iteration issues the next
// group's piece 0 before using piece 1 and its piece 1 after the epilogue (zero-size loads past the
// wave's last group, so that every iteration issues the same loads and the compiler's waits stay
// "the older piece only"); after the loop the first group of `next` goes out (zero-size when
// !next_valid) behind this phase's stores, and the wave waits for those stores only. Loads are
// issued PLI = max(PL, PLN) per piece (the extra ones read zero past the piece), so that the
// prefetched group covers the next phase's pieces.
template <int KIND, int PL, int PLN, int PLMAX>
__device__ __forceinline__ void step_matvec(const StepArgs& a, const PhaseMap& m, const StepEpi& e, const PhaseMap& nm,
                                            bool next_valid, bool primed, GroupRegs<PLMAX>& r, const float* xs,
                                            const float* rope_cs, RowMax& mx, int b, int nb, int wave, int lane) {
  constexpr int PLI = PL > PLN ? PL : PLN;
  const WaveShare ws = wave_share(m.groups, b, nb, wave);
  const int n = ws.n;
  if (!primed) issue_group<PLI>(m, ws.g0, n > 0, r, lane);
  __builtin_amdgcn_sched_barrier(0);
  for (int i = 0; i < n; ++i) {
    const int g = ws.g0 + i * ws.step;
    const bool more = i + 1 < n;
    const long noff = more ? (long)(g + ws.step) * m.gstride : 0;
    const float p0 = piece_dot<PL>(r.a, xs, lane);
    issue_piece<PLI>(r.a, m.w0 + noff, more ? m.pbytes : 0, lane);
    __builtin_amdgcn_sched_barrier(0);
    const float p1 = piece_dot<PL>(r.b, xs + m.xo1, lane);
    float s0, s1;
    if constexpr (KIND == kPhW2) {  // the two pieces are one row: one reduction
      s0 = wave_sum(p0 + p1);
      s1 = 0.f;
    } else {
      s0 = wave_sum(p0);
      s1 = wave_sum(p1);
    }
    step_epilogue<KIND>(a, e, g, s0, s1, r.pre, rope_cs, mx, lane);
    issue_pre(m, g + ws.step, more, r.pre);
    issue_piece<PLI>(r.b, m.w1 + noff, more ? m.pbytes : 0, lane);
    __builtin_amdgcn_sched_barrier(0);
  }
  // the next phase's first group of this wave, then this phase's stores complete
  issue_first<PLI>(nm, next_valid, r, b, nb, wave, lane);
  wait_vm<2 * PLI + kPreLoads>();
}

// ---- attention and the O projection in one phase (short contexts) ---------------------------
//
// Reference src/infer.cpp:218-250, 327-344 as one phase, the way attn_o_kernel does it between two
// launches: Wo . attn = sum_g Wo[:, cols(g)] . attn(g). Workgroup b takes kv head g = b % nkv and
// the 128 output rows of block b / nkv (16 per wave); it computes the whole-context attention of
// kv head g itself (every workgroup of g repeats it: a few hundred keys, against a grid barrier
// and the attention's own round trips), multiplies its Wo block (loaded before the barrier) by the
// G heads' outputs and combines each row's sum with the other kv heads' in the integer row words
// (decode_attn.h); the workgroup completing a row writes x[row] = x[row] + sum. Needs
// n_kv_heads * ceil(dim / 128) workgroups and pos < max_seq_len (no sink rotation).

// Wo loads per lane of one wave's block: 16 rows of the G*HD columns of its kv head.
template <int HD, int G>
constexpr int kAttOLoads = G * HD / 32;
template <int HD, int G>
using AttOGeom = AttnOGeom<HD, G, kStepWaves, kAttOLoads<HD, G>>;
constexpr int kAttORows = 16 * kStepWaves;  // output rows per workgroup

// The wave's Wo block (rows row0 .. row0 + 15, columns of kv head g) into r.a (first half of the
// loads) and r.b; rows past dim read zero. Load u covers chunk c = lane + 64 u of the block (row
// c / CPR, 16-byte column chunk c % CPR): its row offset goes into a per-load descriptor (scalar),
// so the only vector offset is the lane's own, which does not depend on u.
template <int HD, int G, int PLMAX>
__device__ __forceinline__ void atto_issue(const StepArgs& a, const uint16_t* wo, int g, int row0, bool valid,
                                           GroupRegs<PLMAX>& r, int lane) {
  constexpr int U = kAttOLoads<HD, G>, UA = (U + 1) / 2, CPR = G * HD / 8;
  static_assert(UA <= PLMAX, "the Wo block fits the piece registers");
  static_assert(CPR % kWave == 0 || kWave % CPR == 0, "whole rows per load, or whole loads per row");
  const int row_bytes = opaque_s(a.q_dim * 2);
  const int n_rows = valid && row0 < a.dim ? a.dim - row0 : 0;  // rows of the block inside the matrix
  lane = opaque_v(lane);
  const char* base = reinterpret_cast<const char*>(wo + (long)(n_rows ? row0 : 0) * a.q_dim + (long)g * G * HD);
  // per lane: CPR >= 64: column chunk 64 (u % UPR) + lane of row u / UPR; else row u RPL + lane / CPR,
  // chunk lane % CPR
  constexpr int UPR = CPR >= kWave ? CPR / kWave : 1, RPL = CPR >= kWave ? 1 : kWave / CPR;
  const int voff = CPR >= kWave ? lane * 16 : (lane / CPR) * row_bytes + (lane % CPR) * 16;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int row = CPR >= kWave ? u / UPR : u * RPL;  // first row of this load
    const int col = CPR >= kWave ? (u % UPR) * 1024 : 0;
    const int left = (n_rows - row) * row_bytes - col;  // bytes of the block from this load's start on
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(base + (long)row * row_bytes + col), 0, left > 0 ? left : 0, kBufferConfig);
    const u32x4 w = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, voff, 0, kCpolNt));
    if (u < UA) r.a[u < UA ? u : 0] = w;
    else r.b[u < UA ? 0 : u - UA] = w;
  }
}

template <int HD, int G, int PLMAX>
__device__ __forceinline__ void step_atto(const StepArgs& a, const AttnArgs& at, const uint16_t* wo, int g, int rb,
                                          int layer, const Positions& ps, bool primed, GroupRegs<PLMAX>& r,
                                          float* lds_f, int wave, int lane) {
  using Geo = AttOGeom<HD, G>;
  constexpr int U = kAttOLoads<HD, G>, UA = (U + 1) / 2, CPR = Geo::CPR, RW = Geo::RW;
  static_assert(Geo::RB == kAttORows, "16 rows per wave");
  using Smem = AttnMfmaSmem<HD, G, kStepWaves>;
  auto& sm = *reinterpret_cast<Smem*>(lds_f);
  float* ao = lds_f + (sizeof(Smem) + 15) / 16 * 4;  // G*HD floats, 16-byte aligned
  auto& rs = *reinterpret_cast<float(*)[kStepWaves][RW]>(ao + G * HD);
  const int tid = opaque_v(threadIdx.x);
  const int row0 = rb * kAttORows + wave * RW;
  if (!primed) atto_issue<HD, G>(a, wo, g, row0, true, r, lane);
  __builtin_amdgcn_sched_barrier(0);
  attn_mfma_waves<HD, G, kStepWaves, 1, true>(at, g, 0, ps.kv_len, sm, [] {});
  // the G heads' attention outputs, normalised, into LDS (the waves' (m, l, o) merged)
  for (int e = tid; e < G * HD; e += kStepThreads) {
    const int h = e / HD, d = e % HD;
    float M = kNegBig;
#pragma unroll
    for (int w = 0; w < kStepWaves; ++w) M = fmaxf(M, sm.oml[w][h][0]);
    float O = 0.f, L = 0.f;
#pragma unroll
    for (int w = 0; w < kStepWaves; ++w) {
      const float wt = exp2_fast(sm.oml[w][h][0] - M);
      O = fmaf(sm.om[w][h][d], wt, O);
      L = fmaf(sm.oml[w][h][1], wt, L);
    }
    ao[e] = O / L;
  }
  __syncthreads();
  // this wave's Wo rows times the attention output; the row's sum to lane j
  u32x4 wv[U];
#pragma unroll
  for (int u = 0; u < U; ++u) wv[u] = u < UA ? r.a[u < UA ? u : 0] : r.b[u < UA ? 0 : u - UA];
  float mine = 0.f;
  if constexpr (CPR >= 64) {
#pragma unroll
    for (int j = 0; j < RW; ++j) {
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < Geo::UPR; ++k) {
        const int c = lane + kWave * (j * Geo::UPR + k);
        acc = dot8(wv[j * Geo::UPR + k], ao + 8 * (c % CPR), acc);
      }
      const float sum = wave_sum(acc);
      if (lane == j) mine = sum;
    }
  } else {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float sum = lane_group_sum<CPR>(dot8(wv[u], ao + 8 * (lane % CPR), 0.f));
      if (lane % CPR == 0) rs[wave][u * Geo::RPL + lane / CPR] = sum;
    }
    __syncthreads();
    mine = lane < RW ? rs[wave][lane] : 0.f;
  }
  // combine with the other kv heads' partial sums (row words); the completing workgroup writes x
  const int row = row0 + lane;
  if (lane < RW && row < a.dim) {
    // x[row] before this phase: the embedding row in layer 0 (src/infer.cpp:460-481), else coherent
    const float xr = layer == 0 ? (float)__builtin_bit_cast(f16, a.embed[(long)a.token * a.dim + row])
                                : load_shared(a.x + row);
    const unsigned long long term = rowacc_term(mine);
    unsigned long long old;
    if (rowacc_in_range(mine)) {
      old = __hip_atomic_fetch_add(a.rowacc + row, term, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {  // the side sum first, published by the word's release
      __hip_atomic_fetch_add(a.rowovf + row, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      old = __hip_atomic_fetch_add(a.rowacc + row, term, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    }
    const unsigned long long w = old + term;
    if ((int)(w >> kRowAccCountShift) == a.n_kv_heads) {  // the last of the row's terms
      float v = rowacc_sum(w, a.n_kv_heads);
      if ((w >> kRowAccOvfShift) & 0xf) {
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        v += __hip_atomic_load(a.rowovf + row, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.rowovf + row, 0.f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      store_shared(a.x + row, xr + v);
      __hip_atomic_store(a.rowacc + row, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ---- staging (poll wave) --------------------------------------------------------------------

// nbytes from src into LDS at dst through direct-to-LDS buffer loads (1 KB per instruction; lane i's
// 16 bytes land at dst + 16 i); `total` bytes (rounded up to 1 KB) are written, those past nbytes as
// zeros (the offsets are vector offsets, which the descriptor's range check covers).
template <int CPOL>
__device__ __forceinline__ void lds_fill(float* dst, const void* src, int nbytes, int total, int lane) {
  for (int off = 0; off < total; off += 1024)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_from(src, off, nbytes),
                                             (__attribute__((address_space(3))) void*)((char*)dst + off), 16, lane * 16, 0,
                                             0, CPOL);
}

__device__ __forceinline__ int lds_span(int floats) { return (floats * 4 + 2048 + 1023) / 1024 * 1024; }

// xs[0, K) = src (coherent), zeros after it up to the 1 KB boundary past K + 512.
__device__ __forceinline__ void stage_vec(float* xs, const float* src, int K, int lane) {
  lds_fill<kCpolSc1>(xs, src, K * 4, lds_span(K), lane);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
}

// The residual stream x (coherent loads straight into registers, NPL float4 per lane: K <= 256 NPL),
// RMS-normalised with the staged gain, into xs[0, K); zeros after it up to the 1 KB boundary past
// K + 512 (as stage_vec leaves them).
template <int NPL>
__device__ __forceinline__ void stage_x_norm(const StepArgs& a, float* xs, const float* gain, int lane) {
  const int K = a.dim, n4 = K / 4;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(a.x, 0, K * 4, kBufferConfig);
  f32x4 v[NPL];
#pragma unroll
  for (int u = 0; u < NPL; ++u) v[u] = load_shared4(xr, 16 * (lane + kWave * u));  // zero past K
  float ss = 0.f;
#pragma unroll
  for (int u = 0; u < NPL; ++u) ss += v[u][0] * v[u][0] + v[u][1] * v[u][1] + v[u][2] * v[u][2] + v[u][3] * v[u][3];
  ss = wave_sum(ss);
  const float inv = 1.0f / sqrtf(ss / (float)K + a.eps);
  f32x4* x4 = reinterpret_cast<f32x4*>(xs);
  const f32x4* g4 = reinterpret_cast<const f32x4*>(gain);
  // four float4 of the gain per round, read unconditionally (clamped) so that each round's reads are
  // in flight together
  constexpr int B = 4;
#pragma unroll
  for (int u0 = 0; u0 < NPL; u0 += B) {
    f32x4 g[B];
#pragma unroll
    for (int k = 0; k < B && u0 + k < NPL; ++k) g[k] = g4[min(lane + kWave * (u0 + k), n4 - 1)];
#pragma unroll
    for (int k = 0; k < B && u0 + k < NPL; ++k) {
      const int i = lane + kWave * (u0 + k);
      f32x4 o;
      o[0] = v[u0 + k][0] * inv * g[k][0];
      o[1] = v[u0 + k][1] * inv * g[k][1];
      o[2] = v[u0 + k][2] * inv * g[k][2];
      o[3] = v[u0 + k][3] * inv * g[k][3];
      if (i < n4) x4[i] = o;
    }
  }
  const int zend = lds_span(K) / 16;  // float4 units
  for (int i = n4 + lane; i < zend; i += kWave) x4[i] = f32x4{0.f, 0.f, 0.f, 0.f};
}

// The embedding row (fp16) as the input: exact fp16 -> fp32 (reference src/infer.cpp:460-481),
// normalised with the staged gain; x_out (workgroup 0 with no layers) also receives the raw row.
__device__ __forceinline__ void stage_emb(const StepArgs& a, float* xs, const float* g, float* x_out, int lane) {
  const int K = a.dim;
  const uint16_t* row = a.embed + (long)a.token * K;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(row), 0, K * 2, kBufferConfig);
  float ss = 0.f;
  for (int c = lane; c * 8 < K; c += kWave) {
    const u32x4 h = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, c * 16, 0, 0));
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float lo = (float)__builtin_bit_cast(f16, (uint16_t)(h[k] & 0xffff));
      const float hi = (float)__builtin_bit_cast(f16, (uint16_t)(h[k] >> 16));
      xs[8 * c + 2 * k] = lo;
      xs[8 * c + 2 * k + 1] = hi;
      ss += lo * lo + hi * hi;
      if (x_out) {
        store_shared(x_out + 8 * c + 2 * k, lo);
        store_shared(x_out + 8 * c + 2 * k + 1, hi);
      }
    }
  }
  for (int i = K + lane; i < K + 512; i += kWave) xs[i] = 0.f;
  ss = wave_sum(ss);
  const float inv = 1.0f / sqrtf(ss / (float)K + a.eps);
  for (int i = lane; i < K; i += kWave) xs[i] = xs[i] * inv * g[i];
}

// The grid barrier for phase `done` (0-based index within the launch), poll wave only; then
// `stage` fills LDS for the next phase.
__device__ __forceinline__ void grid_wait(const StepArgs& a, unsigned target, int b, int nb, int lane) {
  unsigned* flags = a.sync + kSyncFlags;
  unsigned* abort_word = a.sync + kSyncAbort;
  if (lane == 0) __hip_atomic_store(flags + b, target, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // all flags in one load per lane (four each); two polls in flight, the older one checked while
  // the newer one travels, so a flag is seen about one load latency after it lands
  const __amdgpu_buffer_rsrc_t fr = __builtin_amdgcn_make_buffer_rsrc(flags, 0, (nb + 3) / 4 * 16, kBufferConfig);
  auto poll = [&] { return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(fr, 16 * lane, 0, kCpolSc1)); };
  auto done = [&](const u32x4& f) {
    bool ok = true;
#pragma unroll
    for (int k = 0; k < 4; ++k) ok &= (4 * lane + k >= nb) || f[k] >= target;
    return __all(ok);
  };
  u32x4 older = poll();
  for (unsigned spins = 0;; ++spins) {
    __builtin_amdgcn_s_sleep(1);
    const u32x4 newer = poll();
    if (done(older)) return;
    older = newer;
    if ((spins & 63u) == 63u || spins >= a.spin_limit) {
      const unsigned ab = __hip_atomic_load(abort_word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (ab || spins >= a.spin_limit) {
        if (lane == 0) __hip_atomic_store(abort_word, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
      }
    }
  }
}

// ---- the kernel -----------------------------------------------------------------------------

// HD: head_dim; G: query heads per kv head; PLD / PLH: loads per piece of the dim-long rows (QKV,
// O, W13, lm_head) and of the W2 half rows.
// ATTO: attention and O as one phase (short contexts, step_atto) or as two (the split-KV attention
// with its slice merge, then the O matvec); the host picks the instantiation per launch.
template <int HD, int G, int PLD, int PLH, bool ATTO>
__global__ void __launch_bounds__(kStepThreads) decode_step_kernel(StepArgs a) {
  constexpr int PLA = (kAttOLoads<HD, G> + 1) / 2;
  constexpr int PLMAX = PLD > PLH ? (PLD > PLA ? PLD : PLA) : (PLH > PLA ? PLH : PLA);
  // LDS: the staged input (rows of up to 1024 PLH floats, dim and q_dim up to 512 PLD, and the zeros
  // after them), overlapped by the attention's workspace in the ATT phase; the RMS gain of the next
  // normalisation in its own region, so that it is fetched a phase ahead
  constexpr int kXs = 1024 * (PLH > (PLD + 1) / 2 ? PLH : (PLD + 1) / 2) + 1024;
  constexpr int kAtt = (int)(sizeof(AttnMfmaSmem<HD, G, kStepWaves>) + 15) / 16 * 4 + G * HD +
                       kStepWaves * AttOGeom<HD, G>::RW;
  __shared__ __attribute__((aligned(16))) float xs[kXs > kAtt ? kXs : kAtt];
  __shared__ __attribute__((aligned(16))) float gain[512 * PLD];
  __shared__ float rope_cs[HD];
  __shared__ float bv[kStepWaves];
  __shared__ int bi[kStepWaves];
  auto& asm_ = *reinterpret_cast<AttnMfmaSmem<HD, G, kStepWaves>*>(xs);  // ATT phase only

  const int tid = threadIdx.x, lane0 = tid & (kWave - 1);
  const int wave0 = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int lane = lane0, wave = wave0;
  const int b = blockIdx.x, nb = gridDim.x;
  const int L = a.n_layers;
  const bool poll = wave == kPollWave;
  const Positions ps = positions(a.pos, a.msl);

  // the step's RoPE table (reference src/infer.cpp:205-208); the other parity's argmax key
  for (int k = tid; k < HD / 2; k += kStepThreads) {
    const float ang = (float)a.pos * a.inv_freq[k];
    rope_cs[2 * k] = cosf(ang);
    rope_cs[2 * k + 1] = sinf(ang);
  }
  if (b == 0 && tid == 0) __hip_atomic_store(a.keys + (a.parity ^ 1u), 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // the gain of the next normalisation into LDS (poll wave; lands a phase before its use)
  auto fetch_gain = [&](const float* g) { lds_fill<0>(gain, g, 4 * a.dim, 4 * a.dim, lane); };

  auto layer_w = [&](int l, long off) {
    return reinterpret_cast<const uint16_t*>(a.layers.wbase + (long)l * a.layers.stride + off);
  };
  auto layer_g = [&](int l, long off) {
    return reinterpret_cast<const float*>(a.layers.wbase + (long)l * a.layers.stride + off);
  };
  // phase maps
  auto map_qkv = [&](int l) {
    PhaseMap m{};
    m.w0 = layer_w(l, a.layers.o_qkv);
    m.w1 = m.w0 + a.dim;
    m.gstride = 2L * a.dim;
    m.pbytes = 2 * a.dim;
    m.groups = (a.q_dim + 2 * a.kv_dim) / 2;
    m.pre_base = a.x;
    return m;
  };
  auto map_o = [&](int l) {
    PhaseMap m{};
    m.w0 = layer_w(l, a.layers.o_wo);
    m.w1 = m.w0 + a.q_dim;
    m.gstride = 2L * a.q_dim;
    m.pbytes = 2 * a.q_dim;
    m.groups = a.dim / 2;
    if (l == 0) {
      m.pre_base = a.embed + (long)a.token * a.dim;
      m.pre_step = 4;
      m.pre_bytes = 2 * a.dim;
      m.pre_half = 1;
    } else {
      m.pre_base = a.x;
      m.pre_step = 8;
      m.pre_bytes = 4 * a.dim;
    }
    return m;
  };
  auto map_w13 = [&](int l) {
    PhaseMap m{};
    m.w0 = layer_w(l, a.layers.o_w1);
    m.w1 = layer_w(l, a.layers.o_w3);
    m.gstride = a.dim;
    m.pbytes = 2 * a.dim;
    m.groups = a.hidden;
    m.pre_base = a.x;
    return m;
  };
  auto map_w2 = [&](int l) {
    PhaseMap m{};
    m.w0 = layer_w(l, a.layers.o_w2);
    m.w1 = m.w0 + a.hidden / 2;
    m.gstride = a.hidden;
    m.pbytes = a.hidden;  // half a row
    m.xo1 = a.hidden / 2;
    m.groups = a.dim;
    m.pre_base = a.x;
    m.pre_step = 4;
    m.pre_bytes = 4 * a.dim;
    return m;
  };
  auto map_lm = [&]() {
    PhaseMap m{};
    m.w0 = a.wcls;
    m.w1 = a.wcls + a.dim;
    m.gstride = 2L * a.dim;
    m.pbytes = 2 * a.dim;
    m.groups = a.vocab / 2;
    m.pre_base = a.x;
    return m;
  };
  auto epi = [&](int l) {
    StepEpi e;
    e.layer = l;
    e.hd = HD;
    e.ps = ps;
    e.kc = a.layers.kv + 2L * l * a.layers.kv_elems;
    e.vc = e.kc + a.layers.kv_elems;
    return e;
  };

  GroupRegs<PLMAX> r;
  RowMax mx;
  unsigned target = a.base;
  const bool lm = a.mode != 0;

  // first phase: no grid wait; its input is the embedding row
  {
    const PhaseMap m0 = L > 0 ? map_qkv(0) : map_lm();
    if (!poll) issue_first<PLD>(m0, L > 0 || lm, r, b, nb, wave, lane);
    wg_barrier();  // the RoPE table
    if (poll) {
      fetch_gain(L > 0 ? layer_g(0, a.layers.o_ra) : a.rms_final);
      __builtin_amdgcn_s_waitcnt(0x0F70);
      stage_emb(a, xs, gain, (L == 0 && b == 0) ? a.x : nullptr, lane);
      if (L > 0) fetch_gain(layer_g(0, a.layers.o_rf));
    }
    wg_barrier();
  }
  if (L == 0 && !lm) return;  // nothing to compute beyond the embedding row

  for (int l = 0; l < L; ++l) {
    const bool last = l + 1 == L;
    // this iteration's lane and wave, opaque (see opaque_v): what the phases derive from them is
    // computed in the phase that uses it
    const int lane = opaque_v(lane0), wave = opaque_s(wave0);
    // QKV (reference src/infer.cpp:270-305)
    const int g_att = b % a.n_kv_heads, s_att = b / a.n_kv_heads;
    const int kv_len = ps.kv_len;
    const int chunk = attn_mfma_chunk(kv_len, a.nsplit, 0);
    const int active = (kv_len + chunk - 1) / chunk;
    const bool att_wg = !ATTO && s_att < active;       // separate attention phase: (kv head, slice)
    const bool atto_wg = ATTO && s_att * kAttORows < a.dim;  // fused phase: (kv head, row block)
    const PhaseMap mo = map_o(l);
    const uint16_t* wo = layer_w(l, a.layers.o_wo);
    AttnArgs at{};
    at.q = a.q;
    at.kcache = a.layers.kv + 2L * l * a.layers.kv_elems;
    at.vcache = at.kcache + a.layers.kv_elems;
    at.partial = a.partial;
    at.tickets = a.tickets;
    at.out = a.att;
    at.head_dim = HD;
    at.n_heads = a.n_heads;
    at.n_kv_heads = a.n_kv_heads;
    at.msl = a.msl;
    at.nsplit = a.nsplit;
    at.min_slice = 0;
    at.inv_freq = a.inv_freq;
    step_matvec<kPhQkv, PLD, PLD>(a, map_qkv(l), epi(l), mo, !ATTO && !att_wg && !poll, !poll, r, xs, rope_cs, mx, b,
                                  nb, wave, lane);
    if constexpr (ATTO) atto_issue<HD, G>(a, wo, g_att, s_att * kAttORows + wave * 16, atto_wg && !poll, r, lane);
    wg_barrier();
    if (poll) grid_wait(a, ++target, b, nb, lane);
    wg_barrier();
    const PhaseMap m13 = map_w13(l);
    if constexpr (ATTO) {
      // attention + O (reference src/infer.cpp:218-250, 327-344), then the W13 phase's first group
      if (atto_wg) step_atto<HD, G>(a, at, wo, g_att, s_att, l, ps, !poll, r, xs, wave, lane);
      issue_first<PLD>(m13, !poll, r, b, nb, wave, lane);
      wait_vm<2 * PLD + kPreLoads>();
    } else {
      // ATT (reference src/infer.cpp:218-250, 307-336)
      if (att_wg) {
        // one tile buffer per wave: the kernel's registers go to the weight pieces, and at the slice
        // lengths the grid gives (at most ~3 tiles per wave at 16K keys) the second buffer matters little
        attn_mfma_body<HD, G, kStepWaves, 1, true>(at, g_att, s_att, ps, asm_);
        // the O phase's first group of this wave, then the attention's stores complete
        issue_first<PLD>(mo, !poll, r, b, nb, wave, lane);
        wait_vm<2 * PLD + kPreLoads>();
      }
      wg_barrier();
      if (poll) {
        grid_wait(a, ++target, b, nb, lane);
        stage_vec(xs, a.att, a.q_dim, lane);
      }
      wg_barrier();
      // O (reference src/infer.cpp:339-344)
      step_matvec<kPhO, PLD, PLD>(a, mo, epi(l), m13, !poll, !poll, r, xs, rope_cs, mx, b, nb, wave, lane);
    }
    wg_barrier();
    if (poll) {
      grid_wait(a, ++target, b, nb, lane);
      stage_x_norm<2 * PLD>(a, xs, gain, lane);
      if (!last || lm) fetch_gain(last ? a.rms_final : layer_g(l + 1, a.layers.o_ra));
    }
    wg_barrier();
    // W13 (reference src/infer.cpp:349-382)
    const PhaseMap m2 = map_w2(l);
    step_matvec<kPhW13, PLD, PLH>(a, m13, epi(l), m2, !poll, !poll, r, xs, rope_cs, mx, b, nb, wave, lane);
    wg_barrier();
    if (poll) {
      grid_wait(a, ++target, b, nb, lane);
      stage_vec(xs, a.hb, a.hidden, lane);
    }
    wg_barrier();
    // W2 (reference src/infer.cpp:384-390), then the next layer's QKV or the lm_head
    const PhaseMap mn = last ? map_lm() : map_qkv(l + 1);
    step_matvec<kPhW2, PLH, PLD>(a, m2, epi(l), mn, (!last || lm) && !poll, !poll, r, xs, rope_cs, mx, b, nb, wave,
                          lane);
    if (last && !lm) break;
    wg_barrier();
    if (poll) {
      grid_wait(a, ++target, b, nb, lane);
      stage_x_norm<2 * PLD>(a, xs, gain, lane);
      if (!last) fetch_gain(layer_g(l + 1, a.layers.o_rf));
    }
    wg_barrier();
  }
  if (!lm) return;
  // final rmsnorm + lm_head (reference src/infer.cpp:501-527), argmax (src/sampler.cpp:27-38)
  {
    const PhaseMap mlm = map_lm();
    PhaseMap none{};
    none.w0 = none.w1 = a.wcls;
    none.pre_base = a.x;
    step_matvec<kPhLm, PLD, PLD>(a, mlm, epi(0), none, false, !poll, r, xs, rope_cs, mx, b, nb, wave, lane);
  }
  // the workgroup's best (the waves' maxima are wave-uniform), posted with one 64-bit atomic max
  if (lane == 0) {
    bv[wave] = mx.v;
    bi[wave] = mx.i;
  }
  __syncthreads();
  if (tid == 0) {
    RowMax best;
    for (int w = 0; w < kStepWaves; ++w) better(best.v, best.i, bv[w], bi[w]);
    if (best.i != 0x7fffffff)
      __hip_atomic_fetch_max(a.keys + a.parity, argmax_key(best.v, best.i), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace yk
