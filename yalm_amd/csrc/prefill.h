// Batched prompt prefill on the CDNA4 matrix cores (gfx950).
//
// A prompt of n tokens goes through each layer as n rows at once, so the decode matvecs become
// GEMMs (reference semantics: the sequential hydrate of src/main.cpp:169-177 through
// src/infer.cpp:256-392, one token at a time; prefill computes the same K/V cache entries and the
// last token's logits):
//   X [n][dim] fp32 residual stream      -> rmsnorm rows -> Xn [n][dim] fp16
//   Xn . Wqkv^T (MFMA)                    -> C [n][q+2kv] fp32 -> clip, RoPE -> Q fp16, K/V cache
//   causal GQA attention (MFMA)           -> A [n][q] fp16
//   X += A . Wo^T (MFMA, residual epilogue)
//   rmsnorm rows -> Xn; H = act(Xn W1^T) * (Xn W3^T) (MFMA, SwiGLU epilogue) -> H [n][hidden] fp16
//   X += H . W2^T (MFMA, residual epilogue)
// Activations enter the matrix cores in fp16 and accumulate in fp32.
//
// MFMA operand layout (v_mfma_f32_32x32x16_f16, one wave): lane l holds row l%32 of A and column
// l%32 of B, eight k values each, group l/32; which eight k a lane holds is free as long as A and
// B agree. Accumulator register r of lane l is row 8(r/4) + 4(l/32) + r%4, column l%32.
#pragma once
#include "kernels.h"

namespace yk {

typedef f16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0, 0, 0);
}
__device__ __forceinline__ int acc_row(int r, int lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }
// Prefill attention's K rows in LDS: row i of a 32-key tile holds key key_row(i) (bits 2 and 3
// swapped, an involution), so a lane's 8 probabilities of MFMA step kk (score rows
// 16 kk + 8 a + 4 half + c, a in {0, 1}, c in 0..3) are keys 16 kk + 8 half + 0..7 in order: the
// value MFMA's B fragment is one contiguous 16-byte read of a V row.
__device__ __forceinline__ int key_row(int i) { return (i & ~12) | ((i & 4) << 1) | ((i & 8) >> 1); }

// x of the partner lane in the other half-wave (lane ^ 32): v_permlane32_swap exchanges lanes 32-63
// of its first operand with lanes 0-31 of its second, both x here. The second operand is passed
// through an empty asm so the compiler cannot treat the two results as equal (it folded a max of
// them to the first one).
__device__ __forceinline__ float half_swap_other(float x) {
  unsigned y = __builtin_bit_cast(unsigned, x);
  __asm__ volatile("" : "+v"(y));
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, x), y, false, false);
  return __builtin_bit_cast(float, (threadIdx.x & 32) ? r[0] : r[1]);
}
__device__ __forceinline__ float half_swap_max(float x) { return fmaxf(x, half_swap_other(x)); }
// Max of 16 MFMA results in 8 v_max3_f32. Written out because fmaxf first quiets each input that
// the compiler cannot prove canonical (an extra v_max_f32 x, x per MFMA result); scores from finite
// fp16 operands are never signalling NaNs.
__device__ __forceinline__ float max3f(float a, float b, float c) {
  float r;
  __asm__("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
__device__ __forceinline__ float max16(const f32x16& s) {
  const float a = max3f(s[0], s[1], s[2]), b = max3f(s[3], s[4], s[5]), c = max3f(s[6], s[7], s[8]);
  const float d = max3f(s[9], s[10], s[11]), e = max3f(s[12], s[13], s[14]);
  return max3f(max3f(a, b, c), max3f(d, e, s[15]), s[15]);
}

// ------------------------------------------------------------------------------------------
// GEMM C[M][N] = A[M][K] . B[N][K]^T, A and B fp16 row-major (both K-contiguous, as activations
// and .yalm weights are), on 32x32x16 MFMA tiles. Rows past M and columns past N are clamped on
// load and masked on store. K must be a multiple of 32.
// Epilogues: STORE C = acc; RESID C += acc; SWIGLU: a tile's B rows are rows of W1 and the same
// rows of W3, interleaved by 32, so each lane holds act(w1) and w3 of one output;
// H[m][j] = fp16(act(w1) * w3) with N counting output columns.
// ------------------------------------------------------------------------------------------
enum GemmEpi : int { kGemmStore = 0, kGemmResid = 1, kGemmSwiGLU = 2 };

// SiLU of the SwiGLU epilogues, x * 1 / (1 + 2^(-x log2 e)) with the hardware exponential and
// reciprocal (each within about an ulp): the epilogue stores fp16 (2^-11 relative), far coarser
// than the few-ulp difference from the reference form x / (1 + expf(-x)) (src/infer.cpp:362-382),
// whose range-reduced expf and IEEE divide take ~25 instructions per output, about 8% of a W1/W3
// tile at 3200 rows. Both limits hold: 2^(+inf) makes the product -0, 2^(-inf) leaves x.
__device__ __forceinline__ float silu_fast(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + exp2_fast(-x * kLog2e));
}

struct GemmArgs {
  const uint16_t* A;
  long lda;
  const uint16_t* B;   // [N][K] (SwiGLU: W1)
  const uint16_t* B3;  // SwiGLU: W3 [N][K]
  long ldb;
  float* C;            // STORE / RESID target [M][ldc]
  long ldc;
  uint16_t* H;         // SwiGLU target [M][ldh] fp16
  long ldh;
  int M, N, K;
  int act;  // SwiGLU: 1 silu, 0 gelu
  // Split-K (LDS-pipeline kernel): ksplit > 1 workgroups share an output tile, each over K / ksplit,
  // and store fp32 partials to P ([ksplit][M][N], SwiGLU [ksplit][M][2][N]: W1 then W3 sums);
  // gemm_splitk_reduce sums them in split order and applies the epilogue.
  float* P;
  long p_floats;  // capacity of P
  int ksplit;     // 0 or 1: no split
  // Split last round of the eight-wave kernel: one flag per partial slot (kSkFlagStride words
  // apart, zeroed once) and the word a timed-out wait sets.
  unsigned* sk_flags;
  unsigned* abort_flag;
};

constexpr int kGBM = 128, kGBN = 128, kGBK = 32;

// ------------------------------------------------------------------------------------------
// 128-row tiles (BM 128 with four waves in 2 x 2, or 256 with eight), each wave a 64 x 64 block of
// four 32x32 MFMA tiles, in an S-stage LDS pipeline fed by direct-to-LDS loads (global_load_lds_dwordx4:
// lane l of a wave instruction writes 16 bytes at the instruction's LDS address + 16 l). A stage
// holds one BK-deep k-step of both operands, 128 rows x 2 BK bytes each, with the 16-byte k-chunk
// c of row r stored at position c ^ ((r / RPW) % CPR) (CPR = BK / 8 chunks per row, RPW = rows per
// 256 bytes): a fragment read (one chunk of 32 rows) is served 16 lanes at a time from 64 banks
// (a 256-byte period), and the swizzle puts the 16 rows of each pass in distinct banks (measured:
// no LDS bank conflicts). S - 1 k-steps are in flight while one is used; nothing passes through
// registers on the way to LDS, and each 16-deep slice's fragments are read while the previous
// slice's MFMAs run.
// ------------------------------------------------------------------------------------------
// Tile order of the pipelined GEMMs (one-dimensional grid of 8 * ceil(tiles / 8) workgroups).
// Workgroups are handed to the eight XCDs in turn (workgroup b runs on XCD b % 8), and each XCD
// takes a contiguous run of tiles in M-fastest order: the row panels of A (the activations, a few
// tens of MB) are walked for one column panel of B (the weights) after another, so each weight
// panel is fetched by one XCD and reused from its L2 across the row panels, and the whole weight
// matrix is read from HBM about once. Returns false for the surplus workgroups.
__device__ __forceinline__ bool gemm_tile(int mt, int nt, int& tm, int& tn) {
  const int tiles = mt * nt, per = (tiles + 7) / 8;
  const int t = (int)(blockIdx.x % 8) * per + (int)(blockIdx.x / 8);
  if (t >= tiles) return false;
  tm = t % mt;
  tn = t / mt;
  return true;
}

// The same order over (tile, K split) units: tiles M-fastest, then the splits of the whole tile grid.
__device__ __forceinline__ bool gemm_unit(int mt, int nt, int ks, int& tm, int& tn, int& split) {
  const int units = mt * nt * ks, per = (units + 7) / 8;
  const int t = (int)(blockIdx.x % 8) * per + (int)(blockIdx.x / 8);
  if (t >= units) return false;
  tm = t % mt;
  tn = (t / mt) % nt;
  split = t / (mt * nt);
  return true;
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {  // s_waitcnt vmcnt(N), expcnt and lgkmcnt unconstrained
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ void load_lds16(const uint16_t* src, uint16_t* lds_dst) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                   (__attribute__((address_space(3))) void*)lds_dst, 16, 0, 0);
}

// BM = 128 (four waves, 2 x 2) or 256 (eight waves, 4 x 2); every wave computes 64 x 64.
template <int EPI, int S, int BK, int BM>
__global__ void __launch_bounds__(BM * 2) gemm_lds_kernel(GemmArgs g) {
  static_assert(S >= 2 && (BK == 32 || BK == 64) && (BM == 128 || BM == 256), "stages, k-step, tile");
  constexpr int NW = BM / 32;               // waves
  constexpr int ATILE = BM * BK;            // halves of the A operand per stage
  constexpr int BTILE = kGBN * BK;          // halves of the B operand per stage
  constexpr int CPR = BK / 8;               // 16-byte chunks per row
  constexpr int RPI = 1024 / (2 * BK);      // rows per 1 KB load instruction
  constexpr int RPW = 256 / (2 * BK);       // rows per 256-byte bank period
  constexpr int IA = BM / RPI / NW;         // A load instructions per wave per stage
  constexpr int IB = kGBN / RPI / NW;       // B load instructions per wave per stage
  constexpr int LPS = IA + IB;              // loads per wave per stage
  constexpr int KK = BK / 16;               // MFMA k-slices per stage
  static_assert(IA >= 1 && IB >= 1, "load split");
  __shared__ __attribute__((aligned(1024))) uint16_t smem[S][ATILE + BTILE];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  constexpr int NC = EPI == kGemmSwiGLU ? kGBN / 2 : kGBN;  // output columns per tile
  const int ks = g.ksplit > 1 ? g.ksplit : 1;
  int tm, tn, split;
  if (!gemm_unit((g.M + BM - 1) / BM, (g.N + NC - 1) / NC, ks, tm, tn, split)) return;
  const int m0 = tm * BM, n0 = tn * NC;
  const int kspan = g.K / ks, kbeg = split * kspan;  // this workgroup's K range (a multiple of BK)
  auto swz = [](int r) { return (r / RPW) % CPR; };

  // wave w fills the 1 KB pieces w, w + NW, ... of each operand tile
  const uint16_t* arow[IA];
  const uint16_t* brow[IB];
#pragma unroll
  for (int j = 0; j < IA; ++j) {
    const int r = RPI * (wave + NW * j) + lane / CPR;
    const int c = (lane % CPR) ^ swz(r);  // the global k-chunk this lane's LDS slot holds
    arow[j] = g.A + (long)min(m0 + r, g.M - 1) * g.lda + kbeg + 8 * c;
  }
#pragma unroll
  for (int j = 0; j < IB; ++j) {
    const int r = RPI * (wave + NW * j) + lane / CPR;
    const int c = (lane % CPR) ^ swz(r);
    if constexpr (EPI == kGemmSwiGLU) {
      const int col = n0 + (r >> 6) * 32 + (r & 31);
      const uint16_t* base = ((r >> 5) & 1) ? g.B3 : g.B;
      brow[j] = base + (long)min(col, g.N - 1) * g.ldb + kbeg + 8 * c;
    } else {
      brow[j] = g.B + (long)min(n0 + r, g.N - 1) * g.ldb + kbeg + 8 * c;
    }
  }
  auto issue = [&](int kt, int kdata) {  // stage slot of k-step kt, filled with k-step kdata
    const int st = kt % S, k0 = kdata * BK;
#pragma unroll
    for (int j = 0; j < IA; ++j) load_lds16(arow[j] + k0, &smem[st][(wave + NW * j) * 512]);
#pragma unroll
    for (int j = 0; j < IB; ++j) load_lds16(brow[j] + k0, &smem[st][ATILE + (wave + NW * j) * 512]);
  };
  auto read_frags = [&](const uint16_t* As, const uint16_t* Bs, int kk, u32x4 (&fa)[2], u32x4 (&fb)[2]) {
    const int c = 2 * kk + (lane >> 5);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int ra = wm * 64 + t * 32 + (lane & 31);
      const int rb = wn * 64 + t * 32 + (lane & 31);
      fa[t] = *reinterpret_cast<const u32x4*>(As + ra * BK + 8 * (c ^ swz(ra)));
      fb[t] = *reinterpret_cast<const u32x4*>(Bs + rb * BK + 8 * (c ^ swz(rb)));
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

  const int nk = kspan / BK;
#pragma unroll
  for (int kt = 0; kt < S - 1; ++kt)
    if (kt < nk) issue(kt, kt);
  for (int kt = 0; kt < nk; ++kt) {
    // k-step kt has landed once at most S - 2 later stages (LPS loads each) are outstanding
    if (kt + S - 2 < nk) wait_vmcnt<LPS * (S - 2)>();
    else wait_vmcnt<0>();
    // Every wave's part of stage kt is in and stage kt - 1 is no longer read. A bare barrier: the
    // wait above already covers this wave's loads, and a fence here would also wait for the
    // later stages still in flight.
    __asm__ volatile("" ::: "memory");  // no LDS access moves across the barrier
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
    if (kt + S - 1 < nk) issue(kt + S - 1, kt + S - 1);
    const uint16_t* As = smem[kt % S];
    const uint16_t* Bs = smem[kt % S] + ATILE;
    u32x4 fa[2][2], fb[2][2];
    read_frags(As, Bs, 0, fa[0], fb[0]);
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      if (kk + 1 < KK) read_frags(As, Bs, kk + 1, fa[(kk + 1) & 1], fb[(kk + 1) & 1]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma32(fa[kk & 1][i], fb[kk & 1][j], acc[i][j]);
    }
  }

  if (ks > 1) {  // raw partial sums; gemm_splitk_reduce applies the epilogue
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * 64 + i * 32 + acc_row(r, lane);
        if (m >= g.M) continue;
        if constexpr (EPI == kGemmSwiGLU) {
          const int j = n0 + wn * 32 + (lane & 31);
          if (j < g.N) {
            float* pp = g.P + ((long)split * g.M + m) * (2L * g.N) + j;
            pp[0] = acc[i][0][r];
            pp[g.N] = acc[i][1][r];
          }
        } else {
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const int n = n0 + wn * 64 + j * 32 + (lane & 31);
            if (n < g.N) g.P[((long)split * g.M + m) * g.N + n] = acc[i][j][r];
          }
        }
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = m0 + wm * 64 + i * 32 + acc_row(r, lane);
      if (m >= g.M) continue;
      if constexpr (EPI == kGemmSwiGLU) {
        const int j = n0 + wn * 32 + (lane & 31);
        if (j < g.N) {
          const float a1 = acc[i][0][r], a3 = acc[i][1][r];
          const float h = g.act == 1 ? silu_fast(a1) : gelu(a1);
          g.H[(long)m * g.ldh + j] = __builtin_bit_cast(uint16_t, (f16)(h * a3));
        }
      } else {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int n = n0 + wn * 64 + j * 32 + (lane & 31);
          if (n >= g.N) continue;
          float* cp = g.C + (long)m * g.ldc + n;
          if constexpr (EPI == kGemmResid) *cp += acc[i][j][r];
          else *cp = acc[i][j][r];
        }
      }
    }
  }
}

// Sum of the split-K partials in split order (deterministic), then the GEMM's epilogue: C = sum,
// C += sum, or H = fp16(act(sum W1) * sum W3). One thread per output element.
template <int EPI>
__global__ void __launch_bounds__(256) gemm_splitk_reduce(GemmArgs g) {
  const long total = (long)g.M * g.N;
  for (long e = (long)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (long)gridDim.x * blockDim.x) {
    const int m = (int)(e / g.N), n = (int)(e % g.N);
    if constexpr (EPI == kGemmSwiGLU) {
      float a1 = 0.f, a3 = 0.f;
      for (int sp = 0; sp < g.ksplit; ++sp) {
        const float* pp = g.P + ((long)sp * g.M + m) * (2L * g.N) + n;
        a1 += pp[0];
        a3 += pp[g.N];
      }
      const float h = g.act == 1 ? silu_fast(a1) : gelu(a1);
      g.H[(long)m * g.ldh + n] = __builtin_bit_cast(uint16_t, (f16)(h * a3));
    } else {
      float v = 0.f;
      for (int sp = 0; sp < g.ksplit; ++sp) v += g.P[((long)sp * g.M + m) * g.N + n];
      float* cp = g.C + (long)m * g.ldc + n;
      if constexpr (EPI == kGemmResid) *cp += v;
      else *cp = v;
    }
  }
}

constexpr int kBigM = 256, kBigN = 256;

// Partial slots and flags of the eight-wave kernel's split round: a slot holds one 256 x 256 fp32
// tile, flags are kSkFlagStride words apart.
constexpr int kSkSlotFloats = kBigM * kBigN;
constexpr int kSkFlagStride = 64;

// ------------------------------------------------------------------------------------------
// Eight-wave large-tile GEMM ("ping-pong"): 256 x 256 per workgroup, two waves per SIMD. Each wave owns a 128 x 64 block of the tile (2 x 4 layout, accumulators 4 x 2
// tiles of 32 x 32) and alternates a memory phase (the LDS fragment reads of its next 32-deep
// half-step, then copies) with a compute phase (that half-step's 16 MFMAs on registers only). Waves
// 0-3 and 4-7 form two groups; group 1 runs one phase behind group 0 and a workgroup barrier ends
// every phase, so while one wave of a SIMD (waves w and w + 4 share one) issues MFMAs the other one
// fetches.
// k-steps are 64 deep (K % 64 == 0): the copies move 128 B row pieces, whole cache lines (measured:
// 1.6x the copy rate of 64 B pieces). LDS is a ring of five 32 KB slots holding k-panels as items
// A_s = 2s and B_s = 2s + 1 (slot = item % 5). Stage s is read in phases 4s .. 4s + 3 (group 0 half 0,
// group 1 half 0, group 0 half 1, group 1 half 1). Every memory phase first reads its fragments and
// then copies a quarter of a stage: the first one of stage s the wave's share of B_{s+1}, the second
// one its share of A_{s+2} (their slots held A_{s-1} and B_{s-1}, last read in phase 4s - 1). So each
// phase carries 16 KB of copies, which the CU's address unit drains well within the phase (a
// memory phase that issued its copies before its reads, or carried a whole stage, stalled on them:
// measured), and every copy has at least three phases to land. A_{s+1} and B_{s+1} are waited for
// at the end of phase 4s + 3 (group 0 after its last compute phase of the stage, group 1 after its
// last memory phase), before the barrier after which group 0 reads stage s + 1.
// Copies past the last k-step re-read it into a slot that is not read again, so every phase has
// the same shape.
// SwiGLU: the B rows of a tile are 128 rows of W1 and the same 128 rows of W3 interleaved by 32, so
// a wave's two column tiles are W1 and W3 of the same 32 outputs.
// ------------------------------------------------------------------------------------------
template <int EPI>
struct PPTile {
  static constexpr int BK = 64, SLOTS = 5;
  static constexpr int CPR = BK / 8, RPI = 1024 / (2 * BK), RPW = 256 / (2 * BK);
  static constexpr int PANEL = kBigM * BK;                // halves per slot (an A or a B k-panel)
  static constexpr int LPI = kBigM / RPI / 8;             // copies per wave per panel
  static constexpr int NC = EPI == kGemmSwiGLU ? kBigN / 2 : kBigN;  // output columns per tile
  static_assert(kBigM == kBigN, "A and B panels share the ring slots");
  static __device__ __forceinline__ int swz(int r) { return (r / RPW) % CPR; }
};

// The last, partial round of tiles (R tiles, fewer than the CUs) split along K so every CU has
// work: each of those tiles has a main part over k-steps [0, kd) and np tail pieces that split
// [kd, KI) near-evenly. Main parts run in lockstep (all at the same k-step, sharing the A and B
// panels in L2 like whole tiles), and so do the tail pieces. A tail piece stores its fp32
// accumulators (agent-coherent) to its partial slot and sets the slot's flag to the launch epoch;
// the main part adds the pieces' partials in piece order (deterministic) and applies the epilogue.
// Workgroups: dp whole tiles (XCD-contiguous), then mains main parts (R used), then tails
// workgroups dealing the R x np pieces to nt workers.
struct PPSplit {
  int dp;     // whole-tile workgroups (8 * ceil(tiles / 8) without a split)
  int mains;  // main-part workgroups (8 * ceil(R / 8)); 0: no split
  int R;      // tiles of the split round (tiles dp .. dp + R - 1)
  int kd;     // main parts: k-steps [0, kd)
  int np;     // tail pieces per tile
  int tails;  // tail workgroups (8 * ceil(nt / 8))
  int nt;     // tail workers: worker j takes pieces j, j + nt, ...
};

template <int EPI>
__global__ void __launch_bounds__(512) gemm_pp_kernel(GemmArgs g, PPSplit sp, unsigned epoch) {
  using T = PPTile<EPI>;
  constexpr int BK = T::BK;
  __shared__ __attribute__((aligned(1024))) uint16_t smem[T::SLOTS * T::PANEL];
  const int mt = (g.M + kBigM - 1) / kBigM, ntl = (g.N + T::NC - 1) / T::NC;
  const int KI = g.K / BK;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2, wm = wave & 1, wn = wave >> 1;
  f32x16 acc[4][2];

  // acc = A[m0 .. m0 + 256) . B[n0 ...]^T over k-steps [k0, k1), every wave taking part; the LDS
  // ring is free again on return
  auto mainloop = [&](int m0, int n0, int k0, int k1) {
    const uint16_t* arow[T::LPI];
    const uint16_t* brow[T::LPI];
#pragma unroll
    for (int j = 0; j < T::LPI; ++j) {
      const int r = T::RPI * (wave + 8 * j) + lane / T::CPR;
      const int c = (lane % T::CPR) ^ T::swz(r);
      arow[j] = g.A + (long)min(m0 + r, g.M - 1) * g.lda + 8 * c;
      if constexpr (EPI == kGemmSwiGLU) {
        const int col = n0 + (r >> 6) * 32 + (r & 31);
        const uint16_t* base = ((r >> 5) & 1) ? g.B3 : g.B;
        brow[j] = base + (long)min(col, g.N - 1) * g.ldb + 8 * c;
      } else {
        brow[j] = g.B + (long)min(n0 + r, g.N - 1) * g.ldb + 8 * c;
      }
    }
    // item 2s (the A panel) or 2s + 1 (the B panel) of the ring, filled with k-step kdata
    auto issue_item = [&](int item, int kdata) {
      uint16_t* st = smem + (item % T::SLOTS) * T::PANEL;
      const int koff = kdata * BK;
      if (item & 1) {
#pragma unroll
        for (int j = 0; j < T::LPI; ++j) load_lds16(brow[j] + koff, st + (wave + 8 * j) * 512);
      } else {
#pragma unroll
        for (int j = 0; j < T::LPI; ++j) load_lds16(arow[j] + koff, st + (wave + 8 * j) * 512);
      }
    };
    // the fragments of 32-deep half-step hs (0, 1) of ring stage s
    u32x4 fa[2][4], fb[2][2];
    auto read_frags = [&](int st, int hs) {
      const uint16_t* As = smem + ((2 * st) % T::SLOTS) * T::PANEL;
      const uint16_t* Bs = smem + ((2 * st + 1) % T::SLOTS) * T::PANEL;
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const int c = 4 * hs + 2 * kk + (lane >> 5);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int ra = wm * 128 + t * 32 + (lane & 31);
          fa[kk][t] = *reinterpret_cast<const u32x4*>(As + ra * BK + 8 * (c ^ T::swz(ra)));
        }
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int rb = wn * 64 + t * 32 + (lane & 31);
          fb[kk][t] = *reinterpret_cast<const u32x4*>(Bs + rb * BK + 8 * (c ^ T::swz(rb)));
        }
      }
    };
    auto barrier = [] {
      __builtin_amdgcn_sched_barrier(0);
      __asm__ volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      __asm__ volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
    };
    auto compute = [&] {
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) acc[i][j] = mfma32(fa[kk][i], fb[kk][j], acc[i][j]);
    };
    constexpr unsigned kLgkm0 = 0xc07f;  // s_waitcnt lgkmcnt(0): the fragments are in registers
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};
    const int ns = k1 - k0;  // ring stage st holds k-step k0 + st
    issue_item(0, k0);
    issue_item(1, k0);
    issue_item(2, k0 + min(1, ns - 1));
    wait_vmcnt<T::LPI>();  // A_0 and B_0 have landed
    barrier();             // stage 0 is in for every wave
    if (grp == 1) barrier();
    for (int st = 0; st < ns; ++st) {
      read_frags(st, 0);
      __builtin_amdgcn_sched_barrier(0);
      issue_item(2 * st + 3, k0 + min(st + 1, ns - 1));  // B_{st+1}
      __builtin_amdgcn_s_waitcnt(kLgkm0);
      barrier();
      compute();
      barrier();
      read_frags(st, 1);
      __builtin_amdgcn_sched_barrier(0);
      issue_item(2 * st + 4, k0 + min(st + 2, ns - 1));  // A_{st+2}
      __builtin_amdgcn_s_waitcnt(kLgkm0);
      if (grp == 1) wait_vmcnt<T::LPI>();  // this wave's copies of A_{st+1} and B_{st+1} have landed
      barrier();
      compute();
      if (grp == 0) wait_vmcnt<T::LPI>();
      barrier();
    }
    wait_vmcnt<0>();  // the copies past the end have landed before the ring is refilled
    if (grp == 0) barrier();
  };

  // Epilogue through buffer accesses bounded to the tile's rows (rows past M fall outside the
  // buffer, columns past N get an offset outside it: the hardware drops those accesses), so it has
  // no per-element branches and the residual's loads go out 32 at a time ahead of their stores
  // (per-element guarded read-modify-writes serialised into one memory round trip each: 40 us of
  // a 3200 x 4096 tile round).
  auto epilogue = [&](int m0, int n0) {
    const int rows = min(kBigM, g.M - m0);
    constexpr unsigned kOut = 0x80000000u;  // a byte offset past any tile's buffer
    if constexpr (EPI == kGemmSwiGLU) {
      const __amdgpu_buffer_rsrc_t hr = __builtin_amdgcn_make_buffer_rsrc(
          g.H + (long)m0 * g.ldh, 0, (int)((long)rows * g.ldh * 2), kBufferConfig);
      const int j = n0 + wn * 32 + (lane & 31);
      const unsigned col = j < g.N ? 2u * j : kOut;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = wm * 128 + i * 32 + acc_row(r, lane);
          const float a1 = acc[i][0][r], a3 = acc[i][1][r];
          const float h = g.act == 1 ? silu_fast(a1) : gelu(a1);
          const unsigned off = col == kOut ? kOut : (unsigned)(m * g.ldh * 2) + col;
          __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, (f16)(h * a3)), hr, off, 0, 0);
        }
    } else {
      const __amdgpu_buffer_rsrc_t cr = __builtin_amdgcn_make_buffer_rsrc(
          g.C + (long)m0 * g.ldc, 0, (int)((long)rows * g.ldc * 4), kBufferConfig);
      unsigned col[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int n = n0 + wn * 64 + j * 32 + (lane & 31);
        col[j] = n < g.N ? 4u * n : kOut;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        unsigned off[2][16];
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            off[j][r] = col[j] == kOut ? kOut : (unsigned)((wm * 128 + i * 32 + acc_row(r, lane)) * g.ldc * 4) + col[j];
        float v[2][16];
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            v[j][r] = acc[i][j][r];
            if constexpr (EPI == kGemmResid)
              v[j][r] += __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(cr, off[j][r], 0, 0));
          }
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v[j][r]), cr, off[j][r], 0, 0);
      }
    }
  };
  // partial slot layout: 16-byte chunks, lane-contiguous (each access moves 1 KB of whole lines)
  auto slot_byte = [&](int i, int j, int r4) { return ((((wave * 8 + 2 * i + j) * 4 + r4) * 64) + lane) * 16; };
  auto slot_rsrc = [&](int s) {
    return __builtin_amdgcn_make_buffer_rsrc(g.P + (long)s * kSkSlotFloats, 0, kSkSlotFloats * (int)sizeof(float),
                                             kBufferConfig);
  };

  const int b = blockIdx.x;
  if (b < sp.dp) {  // a whole tile
    const int t = (b % 8) * (sp.dp / 8) + b / 8;
    if (t >= mt * ntl) return;
    const int m0 = (t % mt) * kBigM, n0 = (t / mt) * T::NC;
    mainloop(m0, n0, 0, KI);
    epilogue(m0, n0);
    return;
  }
  if (b < sp.dp + sp.mains) {  // the main part of a split tile
    const int bb = b - sp.dp, r = (bb % 8) * (sp.mains / 8) + bb / 8;
    if (r >= sp.R) return;
    const int t = sp.dp + r, m0 = (t % mt) * kBigM, n0 = (t / mt) * T::NC;
    mainloop(m0, n0, 0, sp.kd);
    for (int p = 0; p < sp.np; ++p) {
      const int s = r * sp.np + p;
      wait_flag(g.sk_flags + (long)s * kSkFlagStride, epoch, g.abort_flag);
      const __amdgpu_buffer_rsrc_t sr = slot_rsrc(s);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) {
            const f32x4 v = load_shared4(sr, slot_byte(i, j, r4));
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[i][j][4 * r4 + e] += v[e];
          }
    }
    epilogue(m0, n0);
    return;
  }
  // tail pieces
  const int bb = b - sp.dp - sp.mains, j0 = (bb % 8) * (sp.tails / 8) + bb / 8;
  if (j0 >= sp.nt) return;
  const int KT = KI - sp.kd;
  for (int s = j0; s < sp.R * sp.np; s += sp.nt) {
    const int r = s / sp.np, p = s % sp.np;
    const int t = sp.dp + r, m0 = (t % mt) * kBigM, n0 = (t / mt) * T::NC;
    mainloop(m0, n0, sp.kd + p * KT / sp.np, sp.kd + (p + 1) * KT / sp.np);
    const __amdgpu_buffer_rsrc_t sr = slot_rsrc(s);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const f32x4 v = {acc[i][j][4 * r4], acc[i][j][4 * r4 + 1], acc[i][j][4 * r4 + 2], acc[i][j][4 * r4 + 3]};
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), sr, slot_byte(i, j, r4), 0, kCpolSc1);
        }
    publish();
    __syncthreads();
    if (tid == 0)
      __hip_atomic_store(g.sk_flags + (long)s * kSkFlagStride, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}


// ------------------------------------------------------------------------------------------
// Row kernels of the prefill (one workgroup per row).
// ------------------------------------------------------------------------------------------
// X[t][i] = fp32(E[tokens[t]][i]) (reference src/infer.cpp:460-481, exact)
__global__ void __launch_bounds__(kBlock) embed_rows_kernel(const uint16_t* emb, const int* tokens, float* X, int dim) {
  const int t = blockIdx.x;
  const uint16_t* e = emb + (long)tokens[t] * dim;
  for (int i = threadIdx.x; i < dim; i += kBlock) X[(long)t * dim + i] = (float)__builtin_bit_cast(f16, e[i]);
}

// Xn[t] = fp16(X[t] * inv * g), inv = 1/sqrt(mean(X[t]^2) + eps) (reference src/infer.cpp:136-146)
// Rows up to 8192 long (dim % 4 == 0) stay in registers as float4 between the sum and the output
// (one read of X, 16-byte loads and 8-byte stores); longer rows take the two-pass loop.
__global__ void __launch_bounds__(kBlock) rmsnorm_rows_kernel(const float* X, const float* gain, float eps, int dim,
                                                              uint16_t* Xn) {
  __shared__ float red[kWavesPerBlock];
  const float* x = X + (long)blockIdx.x * dim;
  uint16_t* o = Xn + (long)blockIdx.x * dim;
  constexpr int kMax4 = 8;  // float4 per thread: 8192 / (4 * 256)
  const int n4 = dim / 4;
  if (dim % 4 == 0 && n4 <= kMax4 * kBlock) {
    const f32x4* x4 = reinterpret_cast<const f32x4*>(x);
    f32x4 v[kMax4];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < kMax4; ++k) {
      const int i = threadIdx.x + kBlock * k;
      v[k] = i < n4 ? x4[i] : f32x4{0.f, 0.f, 0.f, 0.f};
      ss += v[k][0] * v[k][0] + v[k][1] * v[k][1] + v[k][2] * v[k][2] + v[k][3] * v[k][3];
    }
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
    const f32x4* g4 = reinterpret_cast<const f32x4*>(gain);
#pragma unroll
    for (int k = 0; k < kMax4; ++k) {
      const int i = threadIdx.x + kBlock * k;
      if (i < n4) {
        const f32x4 g = g4[i];
        unsigned long long h = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          h |= (unsigned long long)__builtin_bit_cast(uint16_t, (f16)(v[k][e] * inv * g[e])) << (16 * e);
        reinterpret_cast<unsigned long long*>(o)[i] = h;
      }
    }
    return;
  }
  float ss = 0.f;
  for (int i = threadIdx.x; i < dim; i += kBlock) ss += x[i] * x[i];
  ss = block_sum(ss, red);
  const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
  for (int i = threadIdx.x; i < dim; i += kBlock) o[i] = __builtin_bit_cast(uint16_t, (f16)(x[i] * inv * gain[i]));
}

// Max over an aligned group of n lanes (n in {8, 16, 32}) by DPP moves inside the vector ALU (quad
// permutes for xor 1 and 2, then the 8- and 16-lane mirrors, each pairing the two halves of the
// previous group), plus one cross-row shuffle for 32; __shfl_xor took an LDS round trip per step.
template <int CTRL>
__device__ __forceinline__ float dpp_max(float x) {
  return fmaxf(x, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf,
                                                                        false)));
}
__device__ __forceinline__ float group_max(float x, int n) {
  x = dpp_max<0xb1>(x);   // quad_perm [1, 0, 3, 2]
  x = dpp_max<0x4e>(x);   // quad_perm [2, 3, 0, 1]
  x = dpp_max<0x141>(x);  // row_half_mirror
  if (n >= 16) x = dpp_max<0x140>(x);  // row_mirror
  if (n >= 32) x = fmaxf(x, __shfl_xor(x, 16, 64));
  return x;
}

// Row t of the QKV GEMM output (position start + t): clip, RoPE on q and k pairs
// (reference src/infer.cpp:197-215, 284-305), q as fp16 into Q, k as fp16 into the cache at the
// row's position (no ring: start + n <= max_seq_len). The v columns go to v_rows_kernel.
// Each query head of the row is stored scaled by the power of two that maps its largest |q| into
// [2^14, 2^15) (q_range_exp), so any finite fp32 q fits fp16 with the same relative precision;
// qscale[t][h] receives the inverse factor, which the attention applies to the head's scores.
__global__ void __launch_bounds__(kBlock) qkv_rows_kernel(const float* C, int ldc, int q_dim, int kv_dim, int head_dim,
                                                          float qkv_clip, const float* inv_freq, int start, int msl,
                                                          uint16_t* Q, float* qscale, uint16_t* kcache) {
  // (cos, sin) of pos * freq_k once per rotary pair k of the row, shared by all q and k heads
  __shared__ float rope[128];  // head_dim <= 128 on the batched path (prefill_supported)
  const int t = blockIdx.x, pos = start + t;
  for (int k = threadIdx.x; k < head_dim / 2; k += kBlock) {
    const float ang = (float)pos * inv_freq[k];
    rope[2 * k] = cosf(ang);
    rope[2 * k + 1] = sinf(ang);
  }
  __syncthreads();
  const float* c = C + (long)t * ldc;
  // a lane takes 4 consecutive values (two rotary pairs): 16-byte loads, 8-byte stores (the 4 dims
  // lie in one 16-dim chunk of the K layout); a head is an aligned group of head_dim / 4 lanes
  // (a power of two, head_dim in {32, 64, 128}), and q_dim, kv_dim are multiples of 32
  const int quads = (q_dim + kv_dim) / 4;  // q and k; v goes through v_rows_kernel
  const int hq = head_dim / 4;
  // every thread runs the same number of iterations, so the head-wide maximum below can use
  // cross-lane shuffles; a head's group of lanes is all live or all dead
  for (int p0 = 0; p0 < quads; p0 += kBlock) {
    const int p = p0 + threadIdx.x;
    const bool live = p < quads;
    const int i = 4 * p;
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (live) {
      v = *reinterpret_cast<const f32x4*>(c + i);
      const int j = i % head_dim;
#pragma unroll
      for (int e = 0; e < 4; e += 2) {
        const float v0 = clipf(v[e], qkv_clip), v1 = clipf(v[e + 1], qkv_clip);
        const float cs = rope[j + e], sn = rope[j + e + 1];
        v[e] = v0 * cs - v1 * sn;
        v[e + 1] = v0 * sn + v1 * cs;
      }
    }
    const float amax = group_max(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))), hq);
    if (!live) continue;
    if (i < q_dim) {
      const int qe = q_range_exp(amax);
      const float qmul = __builtin_ldexpf(1.0f, qe);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] *= qmul;
      if (p % hq == 0) qscale[(long)t * (q_dim / head_dim) + i / head_dim] = __builtin_ldexpf(1.0f, -qe);
    }
    unsigned long long h = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) h |= (unsigned long long)__builtin_bit_cast(uint16_t, (f16)v[e]) << (16 * e);
    if (i < q_dim) {
      *reinterpret_cast<unsigned long long*>(Q + (long)t * q_dim + i) = h;
    } else {  // k: dims j .. j+3 (j % 4 == 0) are adjacent in a 16-dim chunk of the K layout
      const int ik = i - q_dim;
      const int g = ik / head_dim, j = ik % head_dim;
      *reinterpret_cast<unsigned long long*>(kcache + (long)g * head_dim * msl + k_cache_idx(j, pos, msl)) = h;
    }
  }
}

// The v columns of the QKV GEMM output into the V cache (clip, fp16 RNE; reference
// src/infer.cpp:284-305): V[g][d][pos] is position-contiguous, so a workgroup transposes a tile of
// 64 positions x 64 value dims through LDS: 16-byte loads of 4 dims of a row, and, when the tile's
// first position is a multiple of 8 and the tile is full, 16-byte stores of 8 positions of a dim
// (otherwise 2-byte stores). kv_dim % 4 == 0.
__global__ void __launch_bounds__(kBlock) v_rows_kernel(const float* C, int ldc, int q_dim, int kv_dim, int n,
                                                        float qkv_clip, int start, int msl, uint16_t* vcache) {
  __shared__ __attribute__((aligned(16))) uint16_t tile[64][64 + 8];  // [dim][position]
  const int p0 = blockIdx.x * 64, d0 = blockIdx.y * 64;  // positions (rows of C), value dims
  const int tid = threadIdx.x;
#pragma unroll
  for (int k = 0; k < 4; ++k) {  // read: 16 lanes cover a row's 64 dims
    const int r = (tid >> 4) + 16 * k, d = d0 + 4 * (tid & 15), t = p0 + r;
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (t < n && d < kv_dim) v = *reinterpret_cast<const f32x4*>(C + (long)t * ldc + q_dim + kv_dim + d);
#pragma unroll
    for (int e = 0; e < 4; ++e) tile[4 * (tid & 15) + e][r] = __builtin_bit_cast(uint16_t, (f16)clipf(v[e], qkv_clip));
  }
  __syncthreads();
  if ((start + p0) % 8 == 0 && p0 + 64 <= n) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {  // write: 8 lanes cover a dim's 64 positions
      const int r = (tid >> 3) + 32 * k, w = tid & 7, d = d0 + r;
      if (d < kv_dim)
        *reinterpret_cast<u32x4*>(vcache + (long)d * msl + start + p0 + 8 * w) =
            *reinterpret_cast<const u32x4*>(&tile[r][8 * w]);
    }
  } else {
    const int tx = tid & 63, ty = tid >> 6;
    for (int r = ty; r < 64; r += kBlock / 64) {  // write: a dim's 64 positions, coalesced
      const int d = d0 + r, t = p0 + tx;
      if (t < n && d < kv_dim) vcache[(long)d * msl + start + t] = tile[r][tx];
    }
  }
}

// ------------------------------------------------------------------------------------------
// Causal GQA prefill attention on MFMA (reference src/infer.cpp:218-250 per query position:
// scores over keys 0..pos read back from the fp16 cache, softmax with max subtraction, weighted
// sum of V). A workgroup serves kv head g and QT consecutive 32-query tiles: wave (qs, gh) handles
// query tile qs for query head g*G + gh. Each 32-key tile of K and V is staged once into LDS (a
// ring of four tiles) and read by all the workgroup's waves, so K/V reaches the CU once per
// workgroup instead of once per wave.
// Ping-pong: a wave alternates an MFMA phase (the value MFMAs of tile j - 1, then the score MFMAs
// of tile j) with a softmax phase (tile j's online softmax, staging tile j + 2 from registers into
// the ring, requesting tile j + 3). The waves form two groups, the second one phase behind, with a
// workgroup barrier ending every phase, so the two waves of a SIMD (w and w + NW/2) keep the matrix
// core and the vector ALU busy at the same time (with one barrier per tile both waves of a SIMD
// reached the same phase together: measured 28% slower). Tile j sits in buffer j % 4: read in
// phases 2j .. 2j + 3, written in phases 2j - 3 and 2j - 2, rewritten (tile j + 4) from phase 2j + 5.
// Per key tile a wave computes S^T = K Q^T (keys as rows), so each lane holds 16 scores of one query
// (its partner lane l^32 the other 16) and runs the online softmax for that query with one
// cross-half exchange; then O^T += V^T P^T, whose B operand is exactly the lane's own
// probabilities (the K rows are stored permuted so that they are 8 consecutive keys: key_row).
// O^T keeps the query in the column, so the softmax rescale and the final 1/sum are lane-local.
// Queries are at positions start + t; keys are the cache entries 0 .. position.
// Requires HD % 32 == 0, max_seq_len % 32 == 0 and 64 * G * QT threads <= 1024.
// ------------------------------------------------------------------------------------------
struct PrefillAttnArgs {
  const uint16_t* Q;   // [n][n_heads * HD] fp16, each (row, head) scaled by a power of two
  const float* qscale; // [n][n_heads]: the factor that undoes it, applied to the scores
  const uint16_t* kcache;
  const uint16_t* vcache;
  uint16_t* out;       // [n][n_heads * HD] fp16
  int n, start, msl, n_heads, n_kv_heads, n_blocks;  // n_blocks: workgroups per kv head
};

template <int HD, int G, int QT>
__global__ void __launch_bounds__(64 * G * QT) prefill_attn_kernel(PrefillAttnArgs a) {
  static_assert(HD % 32 == 0, "head_dim must be a multiple of 32");
  constexpr int NT = 64 * G * QT, NW = G * QT;
  static_assert(NW % 2 == 0, "two wave groups");
  constexpr int KS = HD / 16;   // k steps of the score MFMA
  constexpr int DT = HD / 32;   // 32-dim tiles of the output
  constexpr int KLD = HD + 8;   // LDS row of a key (halves), padded
  constexpr int VLD = 32 + 8;   // LDS row of a V dim (halves), padded
  constexpr int NB = 4;         // key tiles in the LDS ring
  __shared__ __attribute__((aligned(16))) uint16_t Ks[NB][32 * KLD];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[NB][HD * VLD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int grp = __builtin_amdgcn_readfirstlane(wave / (NW / 2));
  const int gh = wave % G, qs = wave / G;
  // latest (longest) query tiles first, of every kv head: the dispatcher starts the workgroups in
  // order, so the long ones of all heads start in the first round and the short ones fill in
  const int qb = a.n_blocks - 1 - (int)blockIdx.x / a.n_kv_heads;
  const int g = (int)blockIdx.x % a.n_kv_heads;
  const int h = g * G + gh;
  const int q0 = (qb * QT + qs) * 32;
  const int qd = a.n_heads * HD;
  const int my_q = q0 + (lane & 31);
  const int q_pos = a.start + my_q;
  const int block_last = a.start + min((qb + 1) * QT * 32 - 1, a.n - 1);  // last query position of the workgroup
  const uint16_t* kh = a.kcache + (long)g * HD * a.msl;
  const uint16_t* vh = a.vcache + (long)g * HD * a.msl;
  const int half = lane >> 5;

  u32x4 qf[KS];
  {
    const uint16_t* qrow = a.Q + (long)min(my_q, a.n - 1) * qd + h * HD + 8 * half;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = *reinterpret_cast<const u32x4*>(qrow + 16 * ks);
    // kept in registers for the whole loop (left alone, the compiler reloads them from memory for
    // every key tile and waits for each load in front of its MFMA)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) __asm__ volatile("" : "+v"(qf[ks]));
  }
  f32x16 o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) o[t] = f32x16{};
  float m_run = kNegBig, l_run = 0.f;
  // scores in log2 units (exp2_fast), with this query's q scale undone
  const float scale = kLog2e / sqrtf((float)HD) * a.qscale[(long)min(my_q, a.n - 1) * a.n_heads + h];

  // staging of a key tile: K (32 keys x HD dims, 16-byte pieces) and V (HD dims x 32 keys)
  constexpr int KPIECES = 32 * HD / 8, VPIECES = HD * 32 / 8;
  constexpr int KPT = (KPIECES + NT - 1) / NT, VPT = (VPIECES + NT - 1) / NT;
  u32x4 kst[KPT], vst[VPT];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      // piece: chunk c, LDS row (of key key_row(row)), 8-dim half hh of the chunk; consecutive lanes
      // take consecutive rows with the same half, so each 16-lane LDS store pass hits distinct banks
      const int pc = min(tid + NT * i, KPIECES - 1);
      const int c = pc / 64, row = pc & 31, hh = (pc >> 5) & 1;
      kst[i] = *reinterpret_cast<const u32x4*>(kh + (long)c * 16 * a.msl + (long)(k0 + key_row(row)) * 16 + 8 * hh);
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      // piece: dim d, 8 consecutive keys (part); 16 consecutive lanes take 16 dims of one part (row
      // stride 5 banks-of-4 apart, distinct modulo 16) for conflict-free LDS stores
      const int pc = min(tid + NT * i, VPIECES - 1);
      const int d = (pc & 15) + 16 * (pc >> 6), part = (pc >> 4) & 3;
      vst[i] = *reinterpret_cast<const u32x4*>(vh + (long)d * a.msl + k0 + 8 * part);
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int pc = tid + NT * i;
      if (pc < KPIECES) {
        const int c = pc / 64, row = pc & 31, hh = (pc >> 5) & 1;
        *reinterpret_cast<u32x4*>(&Ks[buf][row * KLD + c * 16 + 8 * hh]) = kst[i];
      }
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int pc = tid + NT * i;
      if (pc < VPIECES) {
        const int d = (pc & 15) + 16 * (pc >> 6), part = (pc >> 4) & 3;
        *reinterpret_cast<u32x4*>(&Vs[buf][d * VLD + 8 * part]) = vst[i];
      }
    }
  };

  auto barrier = [] {
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS stores are done
    __builtin_amdgcn_sched_barrier(0);
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };

  const int nkt = block_last / 32 + 1;
  // the V buffer the first MFMA phase reads (as tile -1, with P = 0) holds zeros, not stale bits
  // that could be Inf or NaN; tile NB - 1 overwrites it later
  for (int i = tid; i < HD * VLD / 8; i += NT) reinterpret_cast<u32x4*>(Vs[NB - 1])[i] = u32x4{0u, 0u, 0u, 0u};
  gload(0);
  lstore(0);
  if (1 < nkt) {
    gload(32);
    lstore(1);
  }
  if (2 < nkt) gload(64);
  __syncthreads();  // tiles 0 and 1 are in
  if (grp == 1) barrier();
  u32x4 pf[2] = {u32x4{0u, 0u, 0u, 0u}, u32x4{0u, 0u, 0u, 0u}};  // P of the previous tile
  for (int j = 0; j <= nkt; ++j) {
    // MFMA phase: O^T += V^T P^T of tile j - 1 and S^T = K Q^T of tile j. Every fragment read is
    // issued first (left to itself the compiler waits for each read in front of its MFMA), then
    // the MFMAs alternate between the two products, so each score MFMA's wait on its predecessor
    // is covered by an independent value MFMA. One shape for every iteration: at j = 0 the value
    // MFMAs read the zeroed buffer NB - 1 with P = 0, at j = nkt the scores of a stale tile are
    // computed and not used.
    u32x4 vf[DT][2], kf[KS];
    {
      const uint16_t* vb = Vs[(j + NB - 1) % NB];
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        // k order of step kk: keys 16 kk + 8 half + 0..7 of the tile (the permuted score rows)
        const uint16_t* vrow = vb + (t * 32 + (lane & 31)) * VLD + 8 * half;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) vf[t][kk] = *reinterpret_cast<const u32x4*>(vrow + 16 * kk);
      }
      const uint16_t* krow = &Ks[j % NB][(lane & 31) * KLD + 8 * half];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) kf[ks] = *reinterpret_cast<const u32x4*>(krow + 16 * ks);
    }
    __builtin_amdgcn_sched_barrier(0);
    f32x16 s = f32x16{};
    static_assert(KS == 2 * DT, "one value MFMA per score MFMA");
#pragma unroll
    for (int i = 0; i < KS; ++i) {
      s = mfma32(kf[i], qf[i], s);
      o[i >> 1] = mfma32(vf[i >> 1][i & 1], pf[i & 1], o[i >> 1]);
    }
    barrier();
    // softmax phase: the online softmax of tile j (O rescaled here, its P added in the next MFMA
    // phase), then tile j + 2 into the ring and tile j + 3 requested
    if (j < nkt) {
      const int k0 = j * 32;
      if (k0 + 31 > a.start + q0) {  // some key of the tile follows the wave's first query
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = k0 + key_row(acc_row(r, lane));
          s[r] = key <= q_pos ? s[r] : kNegBig;
        }
      }
      // tile max in raw score units (the scale is positive, so the max commutes with it), a tree,
      // combined with the other half-wave's rows of the same query
      // the running max moves only when it would grow by more than 8 in log2 units (softmax is
      // invariant to it; p stays below 2^8, well within fp16), so O is rarely rescaled: with a
      // plain running max, some query of the wave moved it on about half the tiles
      const float m_cand = fmaxf(m_run, half_swap_max(max16(s)));
      const bool grow = (m_cand - m_run) * scale > 8.f;
      const float m_new = grow ? m_cand : m_run;
      const float corr = exp2_fast((m_run - m_new) * scale);
      // p = 2^(scale s - scale m): tile 0 holds key 0, which precedes every query, so m_new is
      // finite from the first tile on and a masked score (kNegBig) underflows to p = 0 with no test
      const float ms = m_new * scale;
      float pv[16];
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        half8 p8;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int r = 8 * kk + e;
          pv[r] = exp2_fast(fmaf(s[r], scale, -ms));
          p8[e] = (f16)pv[r];
        }
        pf[kk] = __builtin_bit_cast(u32x4, p8);
      }
#pragma unroll
      for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
        for (int r = 0; r < w; ++r) pv[r] += pv[r + w];
      // this lane's rows only: the two half-waves' sums are added once, after the last tile
      l_run = l_run * corr + pv[0];
      m_run = m_new;
      if (__any(grow)) {
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[t][r] *= corr;
      }
    }
    if (j + 2 < nkt) lstore((j + 2) % NB);
    if (j + 3 < nkt) gload(32 * (j + 3));
    barrier();
  }
  if (grp == 0) barrier();
  l_run += half_swap_other(l_run);
  if (my_q < a.n) {
    const float inv = 1.0f / l_run;
    uint16_t* orow = a.out + (long)my_q * qd + h * HD;
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) orow[t * 32 + acc_row(r, lane)] = __builtin_bit_cast(uint16_t, (f16)(o[t][r] * inv));
  }
}

}  // namespace yk
