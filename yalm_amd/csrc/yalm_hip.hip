// libyalm_hip.so: the C-ABI in include/yalm_hip.h over the gfx950 kernels in kernels.h.
//
// One decode step (reference src/infer.cu:1274-1378 in structure, src/infer.cpp:483-527 in
// semantics) is enqueued as:
//   embed -> 32 x [ rmsnorm+QKV+RoPE+KV-write | split-KV attention (+merge) | O-proj+residual |
//                   rmsnorm+W1/W3+SwiGLU | W2+residual ] -> rmsnorm+lm_head [-> argmax]
// Token and position live in a device-side parameter block written by a one-thread kernel
// before each step, so the whole step is captured once per mode into a hipGraph and replayed.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <algorithm>
#include <atomic>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/yalm_hip.h"
#include "decode_flow.h"
#include "prefill.h"
#include "kernels.h"
#include "decode_attn.h"

using namespace yk;

namespace {

thread_local std::string g_thread_err;
// Workgroups per CU for the kernel-level test hooks (0 = the decode path's default); set with
// yhip_set_option(NULL, "test_bpc", n) so tests can force many row groups per wave.
int g_test_bpc = 0;
bool g_attn_mfma = true;  // attention kernel of the kernel-level entry points (process-wide option)
// Large-tile prefill GEMM k-step schedule (BigTile::mainloop<IL>): 0 = the compiler's own order,
// 1 = copies and fragment reads placed between the MFMAs by scheduling groups, 2 = fenced phases;
// -1 (default) = per shape: 2 for K >= 8192, else 1. Same box, 3200 rows (us): W1/W3 962 / 890 /
// 905, W2 510 / 488 / 463.
int g_gemm_ppsplit = 1;   // eight-wave prefill GEMM: split the last, partial round of tiles along K
int g_gemm_stages = 4;    // prefill GEMM: LDS pipeline depth 2..4, or 6 = the eight-wave kernel
int g_gemm_bk = 32;       // prefill GEMM: k-step of the LDS pipeline (32 or 64)
int g_gemm_bm = 128;      // prefill GEMM: rows of A per workgroup with the 64-deep k-step (128 or 256)
bool g_gemm_auto = true;  // prefill GEMM variant chosen per shape (cleared by forcing one)
int g_gemm_ksplit = 0;    // prefill GEMM K splits on the LDS-pipeline kernel (0 = chosen per shape)
std::atomic<unsigned> g_sk_epoch{0};  // split-round GEMM launches so far (each launch's flag value)
int g_upload_stage_mb = 64;  // weight upload: pinned staging chunk in MB (0 = direct pageable copies)
int g_upload_threads = 8;    // weight upload: host threads filling a staging chunk

struct LayerW {
  uint16_t* wqkv = nullptr;  // [q_dim + 2*kv_dim][dim]
  uint16_t* wo = nullptr;    // [dim][q_dim]
  uint16_t* w1 = nullptr;    // [hidden][dim]
  uint16_t* w3 = nullptr;    // [hidden][dim]
  uint16_t* w2 = nullptr;    // [dim][hidden]
  float* rms_att = nullptr;
  float* rms_ffn = nullptr;
  bool loaded = false;
};

// The step's token and position, and its RoPE table (cos, sin of pos * inv_freq per rotary pair,
// reference src/infer.cpp:205-208), written before each step so that a captured graph stays static.
// It also zeroes the packed key the fused lm_head argmax posts to.
__global__ void set_params_kernel(StepParams* p, int token, int pos, const float* inv_freq, float* rope_cs, int half,
                                  unsigned long long* argmax_key) {
  if (threadIdx.x == 0) {
    p->token = token;
    p->pos = pos;
    *argmax_key = 0ull;
  }
  fill_rope_table(inv_freq, rope_cs, half, pos);
}

}  // namespace

struct yhip_ctx {
  yhip_config c{};
  int device = 0;
  int num_cus = 256;
  hipStream_t stream = nullptr;
  std::string err;

  // weight upload staging: a ring of pinned chunks (hipHostMalloc) with an event per chunk
  static constexpr int kStageBufs = 3;
  char* stage[kStageBufs] = {};
  hipEvent_t stage_ev[kStageBufs] = {};
  size_t stage_bytes = 0;
  int stage_next = 0;

  char* wbase = nullptr;
  size_t wbytes = 0;
  std::vector<LayerW> layers;
  uint16_t* embed = nullptr;
  float* rms_final = nullptr;
  uint16_t* wcls = nullptr;
  bool globals_loaded = false;

  uint16_t* kv = nullptr;  // layer l: K at kv + 2*l*kv_elems, V at kv + (2*l+1)*kv_elems
  size_t kv_elems = 0;

  char* abase = nullptr;  // activations
  float* x = nullptr;
  float* q = nullptr;
  float* att = nullptr;
  float* hb = nullptr;
  float* logits = nullptr;
  float* partial = nullptr;
  unsigned* tickets = nullptr;
  int* argmax_dev = nullptr;
  unsigned long long* argmax_key = nullptr;  // packed (logit, index) of the fused lm_head argmax
  StepParams* params = nullptr;
  float* inv_freq = nullptr;  // [head_dim / 2]
  float* rope_cs = nullptr;   // [head_dim], refreshed every step

  float* logits_host = nullptr;  // pinned
  int* argmax_host = nullptr;    // pinned

  bool use_graph = true;
  // workgroups per CU of the decode matvecs: QKV, O, W1/W3, W2, lm_head (0: default_bpc)
  int mv_bpc[5] = {0, 0, 0, 0, 0};
  int attn_splits = 1;       // most KV slices per kv head; set at creation (default_attn_splits)
  int attn_min_slice = 0;  // 0: the kernel's own default (attn_min_slice_for)
  bool attn_mfma = true;  // MFMA decode attention where the shape allows it
  // captured steps: [mode: hydrate, logits, argmax][step variant: kStepSeparate, kStepAttnO,
  // kStepSplitO]
  hipGraphExec_t graph[3][3] = {};

  // attention and the O projection in one launch (attn_o_kernel) for contexts up to attn_o_max
  // tokens. Against the split-KV attention with its slice merge in the O launch (merge_o_kernel),
  // µs per decode step (Mistral-7B shape on MI355X, same box): 100 keys 2512 / 2648, 300 2573 /
  // 2689, 430 2617 / 2636, 490 2635 / 2638, 520 2643 / 2639, 580 2662 / 2643, 690 2676 / 2645
  bool attn_o = true;
  int attn_o_max = 512;
  // beyond that, the split-KV attention leaves its slice merge to merge_o_kernel, which merges and
  // runs the O projection in one launch
  bool split_o = true;
  unsigned* step_abort = nullptr;  // a bounded wait of the prefill GEMM's split round timed out
  unsigned long long* rowacc = nullptr;  // [dim] attn_o_kernel's per-row combining words (zero between launches)
  float* rowovf = nullptr;               // [dim] their fp32 side sums of out-of-range partials (zero between launches)

  // single-launch decode (decode_flow.h)
  const void* step_fn = nullptr;       // instantiation for this shape (attention and O as two phases), or null
  const void* step_fn_atto = nullptr;  // the same with attention and O as one phase (short contexts)
  bool use_flow = false;
  unsigned step_launches = 0;
  unsigned step_base = 0;  // arrival-flag value before the next launch (flags count up across launches)
  LayerLayout layout{};       // weight and KV addresses of every layer
  unsigned* sync = nullptr;   // kSyncWords: abort word, arrival flags
  unsigned long long* step_keys = nullptr;  // [2] packed argmax keys (by launch parity)
  // attention and the O projection as one phase of the single launch up to this many keys (0: never)
  int step_atto_max = 192;
  unsigned step_spin_limit = kSpinLimit;  // polls before a grid barrier wait gives up

  // batched prefill workspace (grown on demand, prefill.h)
  int pf_cap = 0;
  char* pf_base = nullptr;
  float* pf_X = nullptr;     // [n][dim]
  uint16_t* pf_Xn = nullptr; // [n][dim] fp16 normalised rows
  uint16_t* pf_H = nullptr;  // [n][hidden] fp16 SwiGLU output
  float* pf_C = nullptr;     // [n][q + 2kv]
  uint16_t* pf_Q = nullptr;  // [n][q]
  float* pf_qs = nullptr;    // [n][n_heads] score factors of the scaled query heads
  uint16_t* pf_A = nullptr;  // [n][q]
  int* pf_tok = nullptr;     // [n]
  float* pf_P = nullptr;     // split-K partials of the prefill GEMMs (and of the split last round)
  long pf_Pn = 0;            // its capacity in floats
  unsigned* pf_flags = nullptr;  // split-last-round flags (zeroed when the workspace is allocated)

  // device timing of synchronised steps ("stats" option)
  bool stats = false;
  bool stats_pending = false;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  double stats_us = 0.0;
  int stats_steps = 0;

  int q_dim() const { return c.n_heads * c.head_dim; }
  int kv_dim() const { return c.n_kv_heads * c.head_dim; }
  uint16_t* kcache(int l) const { return kv + (size_t)2 * l * kv_elems; }
  uint16_t* vcache(int l) const { return kv + (size_t)(2 * l + 1) * kv_elems; }
};

namespace {

int fail(yhip_ctx* ctx, int code, const std::string& msg) {
  if (ctx)
    ctx->err = msg;
  else
    g_thread_err = msg;
  return code;
}

#define HIP_TRY(ctx, expr)                                                                           \
  do {                                                                                               \
    hipError_t e_ = (expr);                                                                          \
    if (e_ != hipSuccess)                                                                            \
      return fail(ctx, YHIP_EDEVICE, std::string(#expr) + ": " + hipGetErrorString(e_));             \
  } while (0)

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Rotary inverse frequencies, one per pair: 1 / powf(theta, j / rotary_dim) for even j < rotary_dim,
// 0 beyond it (reference src/infer.cpp:205), computed once on the host in fp32.
void fill_inv_freq(float* f, int head_dim, int rotary_dim, float theta) {
  for (int k = 0; k < head_dim / 2; ++k) {
    const int j = 2 * k;
    f[k] = j >= rotary_dim ? 0.f : 1.0f / powf(theta, (float)j / (float)rotary_dim);
  }
}
std::vector<float> make_inv_freq(int head_dim, int rotary_dim, float theta) {
  std::vector<float> f(head_dim / 2);
  fill_inv_freq(f.data(), head_dim, rotary_dim, theta);
  return f;
}

// ---- matvec launch -------------------------------------------------------------------------
// Workgroups per CU, measured best on MI355X in the decode step: 2 for 4096-long rows (QKV, O,
// lm_head), 1 for 14336-long rows (W2, whose 57 KB LDS input already limits residency), and 12 for
// W1/W3 + SwiGLU. With 149 VGPRs three of its workgroups fit a CU, so a 12-per-CU grid (about one
// row pair per wave) leaves most workgroups queued, and the hardware dispatcher hands each CU a new
// one as soon as one finishes: the CUs whose loads are served late simply take fewer. That
// balances the launch's tail (2.621 -> 2.570 ms per token); 2-8 per CU are in between, 14 and 16
// no better.
int default_bpc(int K, int kind = -1) {
  if (kind == kEpiSwiGLU) return 12;
  return K >= 8192 ? 1 : 2;
}

template <int KC, int R, EpiKind EPI, int H = 1>
void launch_mv(const MatvecArgs& a, int blocks, hipStream_t s) {
  // reduction scratch + input vector (+ the RoPE table for the QKV epilogue)
  const size_t lds = (16 + (size_t)a.K + (a.rope_cs ? (size_t)a.head_dim : 0)) * sizeof(float);
  hipLaunchKernelGGL((matvec_kernel<KC, R, EPI, H>), dim3(blocks), dim3(kBlock), lds, s, a);
}

template <EpiKind EPI>
void launch_by_shape(const MatvecArgs& a, int R, int blocks, hipStream_t s) {
  if (R == 1) {
    if (a.K == 4096) launch_mv<8, 1, EPI>(a, blocks, s);
    else if (a.K == 14336) launch_mv<14, 1, EPI, 2>(a, blocks, s);  // two 7168-long pieces per row
    else launch_mv<0, 1, EPI>(a, blocks, s);
  } else {
    if (a.K == 4096) launch_mv<8, 2, EPI>(a, blocks, s);
    else launch_mv<0, 2, EPI>(a, blocks, s);
  }
}

int device_cus();  // compute units of the current device (defined with the test hooks)

// KV slices per kv head of the decode attention: seven eighths of a workgroup per CU over all kv
// heads, clamped to [1, 64]. Swept on MI355X (Mistral shape, slices merged in the O launch, µs per
// decode step with 16 / 20 / 24 / 28 / 32 slices): equal up to 2048 keys; 3216 keys 2776 / 2772 /
// 2784 / 2769 / 2769; 4500 2831 / 2850 / 2815 / 2816 / 2838; 8000 2982 / 2910 / 2898 / 2902 / 2897;
// 12000 3042 / 2972 / 3049 / 2966 / 2981; 16384 3164 / 3071 / 3051 / 3026 / 3026. More than one
// workgroup per CU does not fit.
int default_attn_splits(int cus, int n_kv_heads) {
  return std::max(1, std::min(64, 7 * cus / (8 * std::max(1, n_kv_heads))));
}

// Split-K workspace bound: tiles x splits never exceed one workgroup per CU, and a 128 x 128 tile
// (or 128 x 64 of W1 and of W3) holds 16384 partial sums; the eight-wave GEMM's split last round
// keeps one 256 x 256 fp32 slot per CU.
long splitk_ws_floats(int cus) { return (long)cus * kSkSlotFloats; }
// Split-last-round flags: one word per CU slot, kSkFlagStride words apart.
size_t sk_flag_bytes(int cus) { return (size_t)cus * kSkFlagStride * sizeof(unsigned); }

// Chooses the instantiation for row length K, rows-per-group R and epilogue kind.
int launch_matvec(yhip_ctx* ctx, MatvecArgs a, int kind, int R, int num_cus, hipStream_t s, int bpc = 0) {
  if (a.K % 8 != 0 || (16 + (size_t)a.K + 128) * sizeof(float) > 65536)
    return fail(ctx, YHIP_EINVAL, "matvec: row length must be a multiple of 8 and at most 16240");
  if (R != 1 && R != 2) return fail(ctx, YHIP_EINVAL, "matvec: R must be 1 or 2");
  if (kind == kEpiResidual && (a.gain || a.emb)) return fail(ctx, YHIP_EINVAL, "matvec: the residual epilogue takes no gain or embedding input");
  if (kind == kEpiSwiGLU && a.emb) return fail(ctx, YHIP_EINVAL, "matvec: the SwiGLU epilogue takes no embedding input");
  if (kind == kEpiQkvRope && !a.rope_cs) return fail(ctx, YHIP_EINVAL, "matvec: the RoPE epilogue takes a precomputed table (rope_cs)");
  if (bpc <= 0) bpc = default_bpc(a.K, kind);
  int blocks = (a.groups + kWavesPerBlock - 1) / kWavesPerBlock;
  blocks = std::max(1, std::min(blocks, num_cus * bpc));
  switch (kind) {
    case kEpiStore: launch_by_shape<kEpiStore>(a, R, blocks, s); break;
    case kEpiResidual: launch_by_shape<kEpiResidual>(a, R, blocks, s); break;
    case kEpiSwiGLU: launch_by_shape<kEpiSwiGLU>(a, R, blocks, s); break;
    case kEpiQkvRope: launch_by_shape<kEpiQkvRope>(a, R, blocks, s); break;
    default: return fail(ctx, YHIP_EINVAL, "matvec: unknown epilogue");
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(ctx, YHIP_EDEVICE, std::string("matvec launch: ") + hipGetErrorString(e));
  return YHIP_OK;
}

MatvecArgs mv_base() {
  MatvecArgs a;
  memset(&a, 0, sizeof(a));
  a.qkv_clip = 3.402823466e38f;
  a.pos = -1;
  a.token = -1;
  return a;
}

// The MFMA kernel (decode_attn.h) where the shape allows it (head_dim % 32 == 0, max_seq_len % 32
// == 0) unless `mfma` is off; otherwise the SIMT split-KV kernel. Workgroups of 512 and 256 threads.
// Waves per MFMA attention workgroup. Measured on MI355X: 4 waves (a workgroup per 128 keys) is
// faster at a few hundred keys but slower from ~16K keys on, where 8 waves keep twice the bytes in
// flight per CU.
constexpr int kAttnWaves = 8;

template <int HD>
bool launch_attention_hd(const AttnArgs& a, bool mfma, hipStream_t s) {
  const dim3 grid(a.n_kv_heads, a.nsplit);
  if constexpr (HD % 32 == 0) {
    if (mfma && a.msl % 32 == 0) {
      switch (a.n_heads / a.n_kv_heads) {
        case 1: hipLaunchKernelGGL((attn_mfma_kernel<HD, 1, kAttnWaves>), grid, dim3(64 * kAttnWaves), 0, s, a); return true;
        case 2: hipLaunchKernelGGL((attn_mfma_kernel<HD, 2, kAttnWaves>), grid, dim3(64 * kAttnWaves), 0, s, a); return true;
        case 4: hipLaunchKernelGGL((attn_mfma_kernel<HD, 4, kAttnWaves>), grid, dim3(64 * kAttnWaves), 0, s, a); return true;
        case 8: hipLaunchKernelGGL((attn_mfma_kernel<HD, 8, kAttnWaves>), grid, dim3(64 * kAttnWaves), 0, s, a); return true;
        default: return false;
      }
    }
  }
  switch (a.n_heads / a.n_kv_heads) {
    case 1: hipLaunchKernelGGL((attention_kernel<HD, 1>), grid, dim3(kBlock), 0, s, a); return true;
    case 2: hipLaunchKernelGGL((attention_kernel<HD, 2>), grid, dim3(kBlock), 0, s, a); return true;
    case 4: hipLaunchKernelGGL((attention_kernel<HD, 4>), grid, dim3(kBlock), 0, s, a); return true;
    case 8: hipLaunchKernelGGL((attention_kernel<HD, 8>), grid, dim3(kBlock), 0, s, a); return true;
    default: return false;
  }
}

// Fewest tokens per KV slice: the option's value, else for the MFMA kernel 0 (the kernel picks it
// from the context length, attn_mfma_chunk) and 64 for the SIMT kernel.
int attn_min_slice_for(const yhip_ctx* ctx, bool mfma) {
  if (ctx->attn_min_slice > 0) return ctx->attn_min_slice;
  return mfma ? 0 : 64;
}

bool attn_uses_mfma(const yhip_ctx* ctx) {
  return ctx->attn_mfma && ctx->c.head_dim % 32 == 0 && ctx->c.max_seq_len % 32 == 0;
}

int launch_attention(yhip_ctx* ctx, const AttnArgs& a, hipStream_t s) {
  bool ok = false;
  const bool mfma = ctx ? ctx->attn_mfma : g_attn_mfma;
  switch (a.head_dim) {
    case 16: ok = launch_attention_hd<16>(a, mfma, s); break;
    case 32: ok = launch_attention_hd<32>(a, mfma, s); break;
    case 64: ok = launch_attention_hd<64>(a, mfma, s); break;
    case 128: ok = launch_attention_hd<128>(a, mfma, s); break;
    default: break;
  }
  if (!ok) return fail(ctx, YHIP_EINVAL, "unsupported attention shape (head_dim 16/32/64/128, 1/2/4/8 q heads per kv head)");
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(ctx, YHIP_EDEVICE, std::string("attention launch: ") + hipGetErrorString(e));
  return YHIP_OK;
}

int check_attn_shape(yhip_ctx* ctx, int hd, int nh, int nkv) {
  if (!(hd == 16 || hd == 32 || hd == 64 || hd == 128))
    return fail(ctx, YHIP_EINVAL, "head_dim must be 16, 32, 64 or 128");
  if (nkv <= 0 || nkv > 64 || nh % nkv != 0)
    return fail(ctx, YHIP_EINVAL, "n_heads must be a multiple of n_kv_heads (at most 64)");
  const int G = nh / nkv;
  if (G != 1 && G != 2 && G != 4 && G != 8)
    return fail(ctx, YHIP_EINVAL, "query heads per kv head must be 1, 2, 4 or 8");
  return YHIP_OK;
}

// ---- attention + O projection in one launch ------------------------------------------------------
// Waves per attn_o_kernel workgroup, and its Wo loads per wave: 16 row segments of G*HD columns
// (whole rows of 16-byte chunks), or CPR when a segment has fewer than 64 chunks, so that a wave's
// rows fit its 64 lanes.
constexpr int kAttnOWaves = 8;
template <int HD, int G>
constexpr int attn_o_loads() {
  return G * HD / 8 >= 16 ? 16 : G * HD / 8;
}
template <int HD, int G>
int attn_o_blocks(const yhip_config& c) {
  constexpr int RB = AttnOGeom<HD, G, kAttnOWaves, attn_o_loads<HD, G>()>::RB;
  return c.n_kv_heads * ((c.dim + RB - 1) / RB);
}

template <int HD, int G>
void go_attn_o(const yhip_config& c, const AttnArgs& t, const AttnOArgs& o, hipStream_t s) {
  hipLaunchKernelGGL((attn_o_kernel<HD, G, kAttnOWaves, attn_o_loads<HD, G>()>), dim3(attn_o_blocks<HD, G>(c)),
                     dim3(64 * kAttnOWaves), 0, s, t, o);
}

bool attn_o_shape(const yhip_config& c) {
  const int G = c.n_kv_heads > 0 ? c.n_heads / c.n_kv_heads : 0;
  return (c.head_dim == 32 || c.head_dim == 64 || c.head_dim == 128) && (G == 1 || G == 2 || G == 4 || G == 8) &&
         c.n_kv_heads <= kRowAccMaxTerms;
}

// The step at pos runs attention and O in one launch when the option is on, the MFMA attention
// applies, there is no sink rotation (pos < max_seq_len) and the context is at most attn_o_max.
bool attn_o_at(const yhip_ctx* ctx, int pos) {
  return ctx->attn_o && attn_uses_mfma(ctx) && attn_o_shape(ctx->c) && pos < ctx->c.max_seq_len &&
         pos + 1 <= ctx->attn_o_max;
}

template <int HD, int G>
void go_merge_o(const yhip_config& c, const AttnArgs& t, const AttnOArgs& o, hipStream_t s) {
  hipLaunchKernelGGL((merge_o_kernel<HD, G, kAttnOWaves, attn_o_loads<HD, G>()>), dim3(attn_o_blocks<HD, G>(c)),
                     dim3(64 * kAttnOWaves), 0, s, t, o);
}

// The step at pos leaves the split-KV attention's slice merge to merge_o_kernel when the option is on,
// the MFMA attention applies and the slices fit the merge kernel's partial block.
bool split_o_at(const yhip_ctx* ctx, int pos) {
  return ctx->split_o && attn_uses_mfma(ctx) && attn_o_shape(ctx->c) && ctx->attn_splits <= kMergeOMaxSplits &&
         !attn_o_at(ctx, pos);
}

// merge: false = attn_o_kernel (attention inside), true = merge_o_kernel (partials from the attention
// launch)
int launch_attn_o(yhip_ctx* ctx, const AttnArgs& t, const AttnOArgs& o, hipStream_t s, bool merge = false) {
  const yhip_config& c = ctx->c;
#define YK_AO(HD, G) (merge ? go_merge_o<HD, G>(c, t, o, s) : go_attn_o<HD, G>(c, t, o, s))
  switch (t.head_dim * 16 + t.n_heads / t.n_kv_heads) {
    case 32 * 16 + 1: YK_AO(32, 1); break;
    case 32 * 16 + 2: YK_AO(32, 2); break;
    case 32 * 16 + 4: YK_AO(32, 4); break;
    case 32 * 16 + 8: YK_AO(32, 8); break;
    case 64 * 16 + 1: YK_AO(64, 1); break;
    case 64 * 16 + 2: YK_AO(64, 2); break;
    case 64 * 16 + 4: YK_AO(64, 4); break;
    case 64 * 16 + 8: YK_AO(64, 8); break;
    case 128 * 16 + 1: YK_AO(128, 1); break;
    case 128 * 16 + 2: YK_AO(128, 2); break;
    case 128 * 16 + 4: YK_AO(128, 4); break;
    case 128 * 16 + 8: YK_AO(128, 8); break;
    default: return fail(ctx, YHIP_EINVAL, "attention + O: unsupported shape");
  }
#undef YK_AO
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(ctx, YHIP_EDEVICE, std::string("attention + O launch: ") + hipGetErrorString(e));
  return YHIP_OK;
}

// ---- one decode step ------------------------------------------------------------------------
// mode: 0 hydrate, 1 logits (device logits + D2H copy into the pinned buffer), 2 argmax.
// variant: kStepSeparate (every kernel its own launch), kStepAttnO (attention and O in one launch,
// attn_o_at) or kStepSplitO (split-KV attention, then slice merge and O in one launch, split_o_at);
// the values are the header's YHIP_STEP_* codes.
enum StepVariant : int { kStepSeparate = YHIP_STEP_SEPARATE, kStepAttnO = YHIP_STEP_ATTN_O, kStepSplitO = YHIP_STEP_SPLIT_O };
int step_variant(const yhip_ctx* ctx, int pos) {
  if (attn_o_at(ctx, pos)) return kStepAttnO;
  return split_o_at(ctx, pos) ? kStepSplitO : kStepSeparate;
}

int enqueue_step(yhip_ctx* ctx, int mode, int variant) {
  const yhip_config& c = ctx->c;
  hipStream_t s = ctx->stream;
  const int qd = ctx->q_dim(), kvd = ctx->kv_dim();
  for (int l = 0; l < c.n_layers; ++l) {
    const LayerW& L = ctx->layers[l];
    int rc;
    // 1. rmsnorm + QKV + clip + RoPE + KV write
    MatvecArgs a = mv_base();
    a.w0 = L.wqkv;
    a.row_step = 2L * c.dim;
    a.r_step = c.dim;
    a.groups = (qd + 2 * kvd) / 2;
    a.K = c.dim;
    a.x = ctx->x;
    a.gain = L.rms_att;
    a.eps = c.norm_eps;
    a.out = ctx->q;
    a.q_dim = qd;
    a.kv_dim = kvd;
    a.head_dim = c.head_dim;
    a.msl = c.max_seq_len;
    a.qkv_clip = c.qkv_clip;
    a.kcache = ctx->kcache(l);
    a.vcache = ctx->vcache(l);
    a.params = ctx->params;
    a.rope_cs = ctx->rope_cs;  // the step's RoPE table, written by set_params_kernel
    if (l == 0) {  // the residual stream starts as the token's embedding row (src/infer.cpp:460-481)
      a.emb = ctx->embed;
      a.emb_out = ctx->x;
    }
    // 2. attention
    AttnArgs t;
    t.q = ctx->q;
    t.kcache = ctx->kcache(l);
    t.vcache = ctx->vcache(l);
    t.partial = ctx->partial;
    t.tickets = ctx->tickets;
    t.out = ctx->att;
    t.head_dim = c.head_dim;
    t.n_heads = c.n_heads;
    t.n_kv_heads = c.n_kv_heads;
    t.msl = c.max_seq_len;
    t.nsplit = ctx->attn_splits;
    t.min_slice = attn_min_slice_for(ctx, attn_uses_mfma(ctx));
    t.inv_freq = ctx->inv_freq;
    t.params = ctx->params;
    if ((rc = launch_matvec(ctx, a, kEpiQkvRope, 2, ctx->num_cus, s, ctx->mv_bpc[0]))) return rc;
    if (variant == kStepSplitO) {  // 2. attention, its slices merged by the O launch
      t.defer_merge = 1;
      if ((rc = launch_attention(ctx, t, s))) return rc;
    }
    if (variant == kStepAttnO || variant == kStepSplitO) {
      // 2 + 3. attention (or its slice merge) and O-proj + residual in one launch
      AttnOArgs o;
      o.wo = L.wo;
      o.x = ctx->x;
      o.rowacc = ctx->rowacc;
      o.ovf = ctx->rowovf;
      o.dim = c.dim;
      o.q_dim = qd;
      if ((rc = launch_attn_o(ctx, t, o, s, variant == kStepSplitO))) return rc;
    }
    if (variant == kStepSeparate && (rc = launch_attention(ctx, t, s))) return rc;
    // 3. O-proj + residual
    if (variant == kStepSeparate) {
      a = mv_base();
      a.w0 = L.wo;
      a.row_step = 2L * qd;
      a.r_step = qd;
      a.groups = c.dim / 2;
      a.K = qd;
      a.x = ctx->att;
      a.out = ctx->x;
      if ((rc = launch_matvec(ctx, a, kEpiResidual, 2, ctx->num_cus, s, ctx->mv_bpc[1]))) return rc;
    }
    // 4. rmsnorm + W1/W3 + SwiGLU
    a = mv_base();
    a.w0 = L.w1;
    a.w1 = L.w3;
    a.row_step = c.dim;
    a.groups = c.hidden_dim;
    a.K = c.dim;
    a.x = ctx->x;
    a.gain = L.rms_ffn;
    a.eps = c.norm_eps;
    a.out = ctx->hb;
    a.act = c.act;
    if ((rc = launch_matvec(ctx, a, kEpiSwiGLU, 2, ctx->num_cus, s, ctx->mv_bpc[2]))) return rc;
    // 5. W2 + residual
    a = mv_base();
    a.w0 = L.w2;
    a.row_step = c.hidden_dim;
    a.r_step = c.hidden_dim;
    a.groups = c.dim;
    a.K = c.hidden_dim;
    a.x = ctx->hb;
    a.out = ctx->x;
    if ((rc = launch_matvec(ctx, a, kEpiResidual, 1, ctx->num_cus, s, ctx->mv_bpc[3]))) return rc;
  }
  if (mode == 0) return YHIP_OK;
  const int Rc = (c.vocab_size % 2 == 0) ? 2 : 1;
  MatvecArgs a = mv_base();
  a.w0 = ctx->wcls;
  a.row_step = (long)Rc * c.dim;
  a.r_step = c.dim;
  a.groups = c.vocab_size / Rc;
  a.K = c.dim;
  a.x = ctx->x;
  a.gain = ctx->rms_final;
  a.eps = c.norm_eps;
  a.out = ctx->logits;
  a.params = ctx->params;
  if (c.n_layers == 0) {
    a.emb = ctx->embed;
    a.emb_out = ctx->x;
  }
  if (mode == 1 || Rc != 2) {
    if (int rc = launch_matvec(ctx, a, kEpiStore, Rc, ctx->num_cus, s, ctx->mv_bpc[4])) return rc;
    if (mode == 2)
      hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(kArgmaxThreads), 0, s, (const float*)ctx->logits, c.vocab_size,
                         ctx->argmax_dev);
  } else {  // lm_head with the argmax fused in
    a.track_max = 1;
    const int bpc = ctx->mv_bpc[4] > 0 ? ctx->mv_bpc[4] : default_bpc(a.K);
    const int blocks = std::max(1, std::min((a.groups + kWavesPerBlock - 1) / kWavesPerBlock, ctx->num_cus * bpc));
    const size_t lds = (16 + (size_t)a.K) * sizeof(float);
    if (a.K == 4096)
      hipLaunchKernelGGL(lm_head_argmax_kernel<8>, dim3(blocks), dim3(kBlock), lds, s, a, ctx->argmax_key);
    else
      hipLaunchKernelGGL(lm_head_argmax_kernel<0>, dim3(blocks), dim3(kBlock), lds, s, a, ctx->argmax_key);
    HIP_TRY(ctx, hipGetLastError());
  }
  if (mode == 1) {
    HIP_TRY(ctx, hipMemcpyAsync(ctx->logits_host, ctx->logits, (size_t)c.vocab_size * sizeof(float),
                                hipMemcpyDeviceToHost, s));
  } else if (Rc == 2) {  // the packed key, decoded on the host (argmax_host[2..3])
    HIP_TRY(ctx, hipMemcpyAsync(ctx->argmax_host + 2, ctx->argmax_key, 8, hipMemcpyDeviceToHost, s));
  } else {
    HIP_TRY(ctx, hipMemcpyAsync(ctx->argmax_host, ctx->argmax_dev, sizeof(int), hipMemcpyDeviceToHost, s));
  }
  return YHIP_OK;
}

void drop_graphs(yhip_ctx* ctx) {
  for (auto& per_mode : ctx->graph)
    for (auto& g : per_mode) {
      if (g) hipGraphExecDestroy(g);
      g = nullptr;
    }
}

// ---- single-launch decode ---------------------------------------------------------------------
// Instantiations of decode_step_kernel (head_dim, query heads per kv head, 1 KB loads per piece of
// a dim-long row and of half a hidden-long row): the Mistral-7B shape and the small test shapes;
// other shapes run the per-op kernels.
const void* select_step_kernel(const yhip_config& c, int q_dim, bool atto) {
  // the MFMA attention's 16-byte V reads need max_seq_len % 8 == 0 (keys past the context are read
  // clamped and masked, so 32-key tiles need no further alignment)
  if (c.vocab_size % 2 || c.n_kv_heads <= 0 || c.n_heads % c.n_kv_heads || c.max_seq_len % 8 || c.dim % 8 ||
      c.hidden_dim % 16 || q_dim % 8 || c.n_layers * kPhasesPerLayer + 1 >= kStepPhaseStride)
    return nullptr;
  const int G = c.n_heads / c.n_kv_heads;
  const int pld = (2 * std::max(c.dim, q_dim) + 1023) / 1024, plh = (c.hidden_dim + 1023) / 1024;
#define YK_STEP_KERNEL(HD, G, PLD, PLH)                                                                    \
  (atto ? reinterpret_cast<const void*>(&decode_step_kernel<HD, G, PLD, PLH, true>)                           \
        : reinterpret_cast<const void*>(&decode_step_kernel<HD, G, PLD, PLH, false>))
  if (c.head_dim == 128 && G == 4 && pld == 8 && plh == 14) return YK_STEP_KERNEL(128, 4, 8, 14);
  if (c.head_dim == 32 && G == 4 && pld == 1 && plh == 1) return YK_STEP_KERNEL(32, 4, 1, 1);
  if (c.head_dim == 16 && G == 2 && pld == 1 && plh == 1) return YK_STEP_KERNEL(16, 2, 1, 1);
#undef YK_STEP_KERNEL
  return nullptr;
}

// Arrival flags and argmax keys back to zero (context creation, and after an aborted launch).
int reset_step_sync(yhip_ctx* ctx) {
  HIP_TRY(ctx, hipMemsetAsync(ctx->sync, 0, (size_t)kSyncWords * sizeof(unsigned), ctx->stream));
  HIP_TRY(ctx, hipMemsetAsync(ctx->step_keys, 0, 2 * sizeof(unsigned long long), ctx->stream));
  ctx->step_base = 0;
  return YHIP_OK;
}

// KV slices per kv head of the single launch's attention phase: every (kv head, slice) pair needs a
// workgroup of the grid.
int step_nsplit(const yhip_ctx* ctx) {
  return std::max(1, std::min({ctx->attn_splits, ctx->num_cus / ctx->c.n_kv_heads, kMaxSplits}));
}

// Whether the single launch runs attention and O as one phase at this position: every (kv head,
// 128-row block) needs a workgroup, the row words hold up to kRowAccMaxTerms kv heads, no sink
// rotation.
bool step_atto(const yhip_ctx* ctx, int pos) {
  const yhip_config& c = ctx->c;
  const int kv_len = pos >= c.max_seq_len ? c.max_seq_len : pos + 1;
  return ctx->step_fn_atto && pos < c.max_seq_len && kv_len <= ctx->step_atto_max &&
         c.n_kv_heads <= kRowAccMaxTerms && c.n_kv_heads * ((c.dim + kAttORows - 1) / kAttORows) <= ctx->num_cus;
}

int launch_flow_step(yhip_ctx* ctx, int token, int pos, int mode) {
  const yhip_config& c = ctx->c;
  if (ctx->step_base > 0x7fffffffu - 2u * kStepPhaseStride)  // flag values stay far from wrapping
    if (int rc = reset_step_sync(ctx)) return rc;
  StepArgs d;
  memset(&d, 0, sizeof(d));
  d.layers = ctx->layout;
  d.embed = ctx->embed;
  d.wcls = ctx->wcls;
  d.rms_final = ctx->rms_final;
  d.inv_freq = ctx->inv_freq;
  d.x = ctx->x;
  d.q = ctx->q;
  d.att = ctx->att;
  d.hb = ctx->hb;
  d.logits = ctx->logits;
  d.partial = ctx->partial;
  d.tickets = ctx->tickets;
  d.rowacc = ctx->rowacc;
  d.rowovf = ctx->rowovf;
  d.sync = ctx->sync;
  d.keys = ctx->step_keys;
  d.n_layers = c.n_layers;
  d.dim = c.dim;
  d.hidden = c.hidden_dim;
  d.q_dim = ctx->q_dim();
  d.kv_dim = ctx->kv_dim();
  d.n_heads = c.n_heads;
  d.n_kv_heads = c.n_kv_heads;
  d.vocab = c.vocab_size;
  d.msl = c.max_seq_len;
  d.token = token;
  d.pos = pos;
  d.mode = mode;
  const int nb = ctx->num_cus;
  d.nsplit = step_nsplit(ctx);
  const bool atto = step_atto(ctx, pos);
  d.act = c.act;
  d.eps = c.norm_eps;
  d.qkv_clip = c.qkv_clip;
  d.base = ctx->step_base;
  d.spin_limit = ctx->step_spin_limit;
  d.parity = ctx->step_launches & 1u;
  ctx->step_base += kStepPhaseStride;
  ctx->step_launches++;
  void* args[] = {&d};
  HIP_TRY(ctx, hipLaunchCooperativeKernel(atto ? ctx->step_fn_atto : ctx->step_fn, dim3(nb), dim3(kStepThreads), args,
                                          0, ctx->stream));
  if (ctx->stats && mode != 0) HIP_TRY(ctx, hipEventRecord(ctx->ev1, ctx->stream));  // the kernel alone
  if (mode == 1)
    HIP_TRY(ctx, hipMemcpyAsync(ctx->logits_host, ctx->logits, (size_t)c.vocab_size * sizeof(float),
                                hipMemcpyDeviceToHost, ctx->stream));
  else if (mode == 2)
    HIP_TRY(ctx, hipMemcpyAsync(ctx->argmax_host + 2, ctx->step_keys + d.parity, 8, hipMemcpyDeviceToHost, ctx->stream));
  if (mode != 0)  // wait time-out word, checked after the caller's synchronisation
    HIP_TRY(ctx, hipMemcpyAsync(ctx->argmax_host + 1, ctx->sync + kSyncAbort, sizeof(int), hipMemcpyDeviceToHost,
                                ctx->stream));
  return YHIP_OK;
}

// After a synchronised prefill: a bounded wait of a prefill GEMM's split round that timed out
// poisons the result.
int check_step_abort(yhip_ctx* ctx) {
  if (ctx->argmax_host[4] == 0) return YHIP_OK;
  ctx->argmax_host[4] = 0;
  hipMemsetAsync(ctx->step_abort, 0, sizeof(unsigned), ctx->stream);
  hipStreamSynchronize(ctx->stream);
  return fail(ctx, YHIP_EDEVICE, "prefill GEMM: a wait for a partial tile timed out");
}

// After a synchronised single-launch step: a wait that timed out poisons the step.
int check_flow_status(yhip_ctx* ctx) {
  if (!ctx->use_flow || ctx->argmax_host[1] == 0) return YHIP_OK;
  ctx->argmax_host[1] = 0;
  reset_step_sync(ctx);
  hipStreamSynchronize(ctx->stream);
  return fail(ctx, YHIP_EDEVICE, "single-launch decode: a grid barrier wait timed out");
}

int run_step_inner(yhip_ctx* ctx, int token, int pos, int mode);

// One step, bracketed by HIP events on the context's stream when "stats" is on (synchronised
// modes only; the elapsed time is collected after the caller's synchronisation).
int run_step(yhip_ctx* ctx, int token, int pos, int mode) {
  const bool timed = ctx->stats && mode != 0;
  if (timed) HIP_TRY(ctx, hipEventRecord(ctx->ev0, ctx->stream));
  if (int rc = run_step_inner(ctx, token, pos, mode)) return rc;
  if (timed) {
    if (!ctx->use_flow) HIP_TRY(ctx, hipEventRecord(ctx->ev1, ctx->stream));
    ctx->stats_pending = true;
  }
  return YHIP_OK;
}

void collect_stats(yhip_ctx* ctx) {
  if (!ctx->stats_pending) return;
  ctx->stats_pending = false;
  float ms = 0.f;
  if (hipEventElapsedTime(&ms, ctx->ev0, ctx->ev1) == hipSuccess) {
    ctx->stats_us += 1000.0 * ms;
    ctx->stats_steps += 1;
  }
}

int run_step_inner(yhip_ctx* ctx, int token, int pos, int mode) {
  const yhip_config& c = ctx->c;
  if (token < 0 || token >= c.vocab_size) return fail(ctx, YHIP_EINVAL, "token id out of range");
  if (pos < 0) return fail(ctx, YHIP_EINVAL, "negative position");
  if (!ctx->globals_loaded) return fail(ctx, YHIP_ESTATE, "globals not uploaded");
  for (int l = 0; l < c.n_layers; ++l)
    if (!ctx->layers[l].loaded) return fail(ctx, YHIP_ESTATE, "layer " + std::to_string(l) + " not uploaded");
  HIP_TRY(ctx, hipSetDevice(ctx->device));
  if (ctx->use_flow) return launch_flow_step(ctx, token, pos, mode);
  hipLaunchKernelGGL(set_params_kernel, dim3(1), dim3(64), 0, ctx->stream, ctx->params, token, pos,
                     (const float*)ctx->inv_freq, ctx->rope_cs, c.head_dim / 2, ctx->argmax_key);
  HIP_TRY(ctx, hipGetLastError());
  const int variant = step_variant(ctx, pos);
  if (!ctx->use_graph) return enqueue_step(ctx, mode, variant);
  hipGraphExec_t& ge = ctx->graph[mode][variant];
  if (!ge) {
    hipGraph_t g = nullptr;
    HIP_TRY(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    int rc = enqueue_step(ctx, mode, variant);
    hipError_t e = hipStreamEndCapture(ctx->stream, &g);
    if (rc) {
      if (g) hipGraphDestroy(g);
      return rc;
    }
    if (e != hipSuccess) return fail(ctx, YHIP_EDEVICE, std::string("graph capture: ") + hipGetErrorString(e));
    e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
    if (e != hipSuccess) {
      ge = nullptr;
      return fail(ctx, YHIP_EDEVICE, std::string("graph instantiate: ") + hipGetErrorString(e));
    }
  }
  HIP_TRY(ctx, hipGraphLaunch(ge, ctx->stream));
  return YHIP_OK;
}

// ---- batched prefill ---------------------------------------------------------------------------
// The prefill GEMM variant for an epilogue and shape (stages 1 = the 256 x 256 kernel, 2..4 the
// LDS pipeline's depth, 0 the register-staged kernel), or the forced process-wide one.
// Split of the eight-wave GEMM's last, partial round (tiles % CUs of them; the kernel's PPSplit):
// with more of those tiles than half the CUs, one tail piece per tile, the idle CUs taking q of
// them each and the main parts' k-range kd balancing the two (W1/W3 at 3200 rows: 176 tiles after
// five whole rounds, 80 tail workers of up to 3 pieces, kd 48 of 64 k-steps); with fewer, S parts
// per tile (S = CUs / tiles, at most 8, pieces of at least 8 k-steps) run side by side (QKV at
// 3200 rows: 56 tiles, 4 parts each). A grid of fewer tiles than CUs but more than half of them
// (W2 and O at 3200 rows: 208) is not split: filling the idle CUs slowed every main part by ~10%
// (the GPU is at its power limit), measured neutral for W2 and 16% slower for O. No split without
// the partial workspace, when the round is full, or when the pieces would be too small or too
// many per worker.
PPSplit pp_split_plan(long tiles, int KI, int P, bool workspace) {
  PPSplit sp{};
  sp.dp = 8 * (int)((tiles + 7) / 8);
  const long R = tiles % P;
  if (!g_gemm_ppsplit || !workspace || P % 8 != 0 || R == 0) return sp;
  if (tiles < P && 2 * R > P) return sp;
  int kd = 0, np = 0, nt = 0;
  if (2 * R > P) {
    nt = P - (int)R;
    const int q = (int)((R + nt - 1) / nt);
    kd = (q * KI + q) / (q + 1);  // ceil(q KI / (q + 1))
    np = 1;
    if (q > 8 || KI - kd < 2) return sp;
  } else {
    const int S = std::min({(int)(P / R), KI / 8, 8});
    if (S < 2) return sp;
    kd = KI / S;
    np = S - 1;
    nt = (int)R * np;
  }
  sp.dp = (int)(tiles - R);
  sp.R = (int)R;
  sp.mains = 8 * (int)((R + 7) / 8);
  sp.kd = kd;
  sp.np = np;
  sp.nt = nt;
  sp.tails = 8 * ((nt + 7) / 8);
  return sp;
}

void gemm_choice(int epi, int M, int N, int K, int cus, int& stages, int& bk, int& bm) {
  stages = g_gemm_stages;
  bk = g_gemm_bk;
  bm = g_gemm_bm;
  if (!g_gemm_auto) return;
  // Variant per shape, from sweeps of the Mistral-7B shapes over M = 256..4096 on MI355X: the
  // eight-wave 256 x 256 kernel wins once its tile grid covers 9/16 of the CUs (W1/W3 from 512
  // rows, QKV from 1536, O and W2 from 2560); below that the 128-row LDS pipeline wins (it splits K
  // when its own grid is short: W2 at 256 rows 55 us against 284), with 256-row workgroups in
  // between for W1/W3 and W2.
  const long big_tiles = (long)((M + kBigM - 1) / kBigM) * ((N + (epi == kGemmSwiGLU ? kBigN / 2 : kBigN) - 1) /
                                                            (epi == kGemmSwiGLU ? kBigN / 2 : kBigN));
  if (K % 64 == 0 && big_tiles * 16 >= (long)cus * 9) {
    stages = 6;
    bk = 64;
    bm = kBigM;
    return;
  }
  const bool big_rows = epi == kGemmSwiGLU || K >= 8192;
  stages = K % 64 == 0 ? 2 : 4;
  bk = K % 64 == 0 ? 64 : 32;
  bm = 128;
  if (big_rows && K % 64 == 0 && M >= (epi == kGemmSwiGLU ? 192 : 1536)) bm = 256;
}

// The variant launch_gemm runs: gemm_choice, then the kernels' own limits. The eight-wave kernel
// needs K % 64 == 0; the LDS pipeline exists with 4 stages of 32-deep k-steps on 128 rows, or 2..3
// stages of 64-deep ones on 128 or 256 rows (a forced eight-wave kernel with K % 64 != 0 lands there).
void gemm_resolve(int epi, int M, int N, int K, int cus, int& stages, int& bk, int& bm) {
  gemm_choice(epi, M, N, K, cus, stages, bk, bm);
  if (stages == 6 && K % 64 == 0) {
    bk = 64;
    bm = kBigM;
    return;
  }
  if (K % 64 != 0) bk = 32;
  if (bk != 64) {
    bm = 128;
    stages = 4;
  } else {
    stages = std::min(std::max(stages, 2), 3);
  }
}

// Prefill GEMM launch. The variant is chosen per shape (gemm_choice) unless forced with the
// process-wide options.
template <int EPI>
int launch_gemm(yhip_ctx* ctx, const GemmArgs& g, hipStream_t s) {
  if (g.K % kGBK != 0 || g.M <= 0 || g.N <= 0) return fail(ctx, YHIP_EINVAL, "gemm: K must be a multiple of 32");
  int stages, bk, bm;
  gemm_resolve(EPI, g.M, g.N, g.K, ctx ? ctx->num_cus : device_cus(), stages, bk, bm);
  if (stages == 6) {  // 256 x 256 tiles, eight waves in two alternating groups
    const int nc = EPI == kGemmSwiGLU ? kBigN / 2 : kBigN;
    const int P = ctx ? ctx->num_cus : device_cus();
    const PPSplit sp = pp_split_plan((long)((g.M + kBigM - 1) / kBigM) * ((g.N + nc - 1) / nc), g.K / 64, P,
                                     g.P && g.sk_flags && g.abort_flag && g.p_floats >= (long)P * kSkSlotFloats);
    const unsigned epoch = sp.mains ? ++g_sk_epoch : 0;
    hipLaunchKernelGGL(gemm_pp_kernel<EPI>, dim3(sp.dp + sp.mains + sp.tails), dim3(512), 0, s, g, sp, epoch);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(ctx, YHIP_EDEVICE, std::string("gemm launch: ") + hipGetErrorString(e));
    return YHIP_OK;
  }
  const int ncols = EPI == kGemmSwiGLU ? kGBN / 2 : kGBN;
  // Split-K when the output has too few tiles to fill the GPU (short prompts): the largest power of
  // two that keeps tiles x splits within one workgroup per CU, divides the k-steps and leaves each
  // split at least two of them; the partials go to the caller's workspace (none: no split).
  GemmArgs ga = g;
  ga.ksplit = 1;
  const long tiles = (long)((g.M + bm - 1) / bm) * ((g.N + ncols - 1) / ncols);
  const long part_floats = (long)g.M * g.N * (EPI == kGemmSwiGLU ? 2 : 1);  // per split
  const int ksteps = g.K / bk;
  if (stages >= 2 && g.P) {
    if (g_gemm_ksplit > 0) {
      ga.ksplit = g_gemm_ksplit;
      if (ksteps % ga.ksplit != 0) return fail(ctx, YHIP_EINVAL, "gemm_ksplit must divide the k-steps");
    } else {
      const long cus = ctx ? ctx->num_cus : device_cus();
      while (tiles * ga.ksplit * 2 <= cus && ksteps % (ga.ksplit * 2) == 0 && ksteps / (ga.ksplit * 2) >= 2 &&
             part_floats * ga.ksplit * 2 <= g.p_floats)
        ga.ksplit *= 2;
    }
    if (ga.ksplit > 1 && part_floats * ga.ksplit > g.p_floats)
      return fail(ctx, YHIP_EINVAL, "gemm: split-K workspace too small");
  }
  const dim3 grid(8 * (unsigned)((tiles * ga.ksplit + 7) / 8));
  switch (stages * 10000 + bk * 1000 / 8 + bm) {
    case 4 * 10000 + 4000 + 128: hipLaunchKernelGGL((gemm_lds_kernel<EPI, 4, 32, 128>), grid, dim3(256), 0, s, ga); break;
    case 2 * 10000 + 8000 + 128: hipLaunchKernelGGL((gemm_lds_kernel<EPI, 2, 64, 128>), grid, dim3(256), 0, s, ga); break;
    case 3 * 10000 + 8000 + 128: hipLaunchKernelGGL((gemm_lds_kernel<EPI, 3, 64, 128>), grid, dim3(256), 0, s, ga); break;
    case 2 * 10000 + 8000 + 256: hipLaunchKernelGGL((gemm_lds_kernel<EPI, 2, 64, 256>), grid, dim3(512), 0, s, ga); break;
    case 3 * 10000 + 8000 + 256: hipLaunchKernelGGL((gemm_lds_kernel<EPI, 3, 64, 256>), grid, dim3(512), 0, s, ga); break;
    default: return fail(ctx, YHIP_EINVAL, "gemm: no LDS-pipeline kernel for this variant");
  }
  if (ga.ksplit > 1) {
    const long total = (long)g.M * g.N;
    hipLaunchKernelGGL(gemm_splitk_reduce<EPI>, dim3((unsigned)std::min<long>(4096, (total + 255) / 256)), dim3(256), 0,
                       s, ga);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(ctx, YHIP_EDEVICE, std::string("gemm launch: ") + hipGetErrorString(e));
  return YHIP_OK;
}

// Workgroups of 64 * G * QT threads: G query heads x QT query tiles of 32 sharing each K/V tile.
template <int HD>
bool launch_prefill_attn_hd(PrefillAttnArgs p, int G, int n_qtiles, hipStream_t s) {
  auto go = [&](auto kernel, int qt, int threads) {
    p.n_blocks = (n_qtiles + qt - 1) / qt;
    hipLaunchKernelGGL(kernel, dim3(p.n_blocks * p.n_kv_heads), dim3(threads), 0, s, p);
  };
  switch (G) {
    case 1: go(prefill_attn_kernel<HD, 1, 4>, 4, 256); return true;
    case 2: go(prefill_attn_kernel<HD, 2, 4>, 4, 512); return true;
    case 4: go(prefill_attn_kernel<HD, 4, 2>, 2, 512); return true;
    case 8: go(prefill_attn_kernel<HD, 8, 1>, 1, 512); return true;
    default: return false;
  }
}

// The batched path needs head_dim a multiple of 32, row lengths multiples of 32 and a context
// that is a multiple of 32; other shapes prefill token by token.
bool prefill_supported(const yhip_config& c, int q_dim) {
  const int G = c.n_heads / c.n_kv_heads;
  return (c.head_dim == 32 || c.head_dim == 64 || c.head_dim == 128) && (G == 1 || G == 2 || G == 4 || G == 8) &&
         c.dim % 32 == 0 && c.hidden_dim % 32 == 0 && q_dim % 32 == 0 && c.max_seq_len % 32 == 0;
}

int ensure_prefill_ws(yhip_ctx* ctx, int n) {
  if (n <= ctx->pf_cap) return YHIP_OK;
  const yhip_config& c = ctx->c;
  const size_t qd = ctx->q_dim(), kvd = ctx->kv_dim(), N = (size_t)n;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off = align_up(off + bytes, 256);
    return o;
  };
  const size_t oX = take(N * c.dim * 4), oXn = take(N * c.dim * 2), oH = take(N * c.hidden_dim * 2),
               oC = take(N * (qd + 2 * kvd) * 4), oQ = take(N * qd * 2), oQs = take(N * c.n_heads * 4),
               oA = take(N * qd * 2), oT = take(N * 4),
               oP = take((size_t)splitk_ws_floats(ctx->num_cus) * 4), oF = take(sk_flag_bytes(ctx->num_cus));
  if (ctx->pf_base) hipFree(ctx->pf_base);
  ctx->pf_base = nullptr;
  ctx->pf_cap = 0;
  if (hipMalloc(&ctx->pf_base, off) != hipSuccess) return fail(ctx, YHIP_EDEVICE, "out of device memory for prefill");
  ctx->pf_X = (float*)(ctx->pf_base + oX);
  ctx->pf_Xn = (uint16_t*)(ctx->pf_base + oXn);
  ctx->pf_H = (uint16_t*)(ctx->pf_base + oH);
  ctx->pf_C = (float*)(ctx->pf_base + oC);
  ctx->pf_Q = (uint16_t*)(ctx->pf_base + oQ);
  ctx->pf_qs = (float*)(ctx->pf_base + oQs);
  ctx->pf_A = (uint16_t*)(ctx->pf_base + oA);
  ctx->pf_tok = (int*)(ctx->pf_base + oT);
  ctx->pf_P = (float*)(ctx->pf_base + oP);
  ctx->pf_Pn = splitk_ws_floats(ctx->num_cus);
  ctx->pf_flags = (unsigned*)(ctx->pf_base + oF);
  if (hipMemset(ctx->pf_flags, 0, sk_flag_bytes(ctx->num_cus)) != hipSuccess)
    return fail(ctx, YHIP_EDEVICE, "prefill workspace: flag reset failed");
  ctx->pf_cap = n;
  return YHIP_OK;
}

int run_prefill(yhip_ctx* ctx, const int* tokens, int n, int start, float* logits_host) {
  const yhip_config& c = ctx->c;
  hipStream_t s = ctx->stream;
  const int qd = ctx->q_dim(), kvd = ctx->kv_dim(), G = c.n_heads / c.n_kv_heads;
  if (int rc = ensure_prefill_ws(ctx, n)) return rc;
  HIP_TRY(ctx, hipMemcpyAsync(ctx->pf_tok, tokens, (size_t)n * sizeof(int), hipMemcpyHostToDevice, s));
  hipLaunchKernelGGL(embed_rows_kernel, dim3(n), dim3(kBlock), 0, s, (const uint16_t*)ctx->embed,
                     (const int*)ctx->pf_tok, ctx->pf_X, c.dim);
  for (int l = 0; l < c.n_layers; ++l) {
    const LayerW& L = ctx->layers[l];
    int rc;
    hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(n), dim3(kBlock), 0, s, (const float*)ctx->pf_X,
                       (const float*)L.rms_att, c.norm_eps, c.dim, ctx->pf_Xn);
    GemmArgs g;
    memset(&g, 0, sizeof(g));
    g.A = ctx->pf_Xn;
    g.lda = c.dim;
    g.B = L.wqkv;
    g.ldb = c.dim;
    g.C = ctx->pf_C;
    g.ldc = qd + 2 * kvd;
    g.M = n;
    g.N = qd + 2 * kvd;
    g.K = c.dim;
    g.P = ctx->pf_P;
    g.p_floats = ctx->pf_Pn;
    g.sk_flags = ctx->pf_flags;
    g.abort_flag = ctx->step_abort;
    if ((rc = launch_gemm<kGemmStore>(ctx, g, s))) return rc;
    hipLaunchKernelGGL(qkv_rows_kernel, dim3(n), dim3(kBlock), 0, s, (const float*)ctx->pf_C, qd + 2 * kvd, qd, kvd,
                       c.head_dim, c.qkv_clip, (const float*)ctx->inv_freq, start, c.max_seq_len, ctx->pf_Q,
                       ctx->pf_qs, ctx->kcache(l));
    // the V cache of kv head g at (g * head_dim + d) * msl: one [kv_dim][msl] matrix
    hipLaunchKernelGGL(v_rows_kernel, dim3((n + 63) / 64, (kvd + 63) / 64), dim3(kBlock), 0, s, (const float*)ctx->pf_C,
                       qd + 2 * kvd, qd, kvd, n, c.qkv_clip, start, c.max_seq_len, ctx->vcache(l));
    PrefillAttnArgs pa;
    pa.Q = ctx->pf_Q;
    pa.qscale = ctx->pf_qs;
    pa.kcache = ctx->kcache(l);
    pa.vcache = ctx->vcache(l);
    pa.out = ctx->pf_A;
    pa.n = n;
    pa.start = start;
    pa.msl = c.max_seq_len;
    pa.n_heads = c.n_heads;
    pa.n_kv_heads = c.n_kv_heads;
    const int nqt = (n + 31) / 32;
    bool ok = false;
    switch (c.head_dim) {
      case 32: ok = launch_prefill_attn_hd<32>(pa, G, nqt, s); break;
      case 64: ok = launch_prefill_attn_hd<64>(pa, G, nqt, s); break;
      case 128: ok = launch_prefill_attn_hd<128>(pa, G, nqt, s); break;
      default: break;
    }
    if (!ok) return fail(ctx, YHIP_EINVAL, "prefill: unsupported attention shape");
    memset(&g, 0, sizeof(g));
    g.A = ctx->pf_A;
    g.lda = qd;
    g.B = L.wo;
    g.ldb = qd;
    g.C = ctx->pf_X;
    g.ldc = c.dim;
    g.M = n;
    g.N = c.dim;
    g.K = qd;
    g.P = ctx->pf_P;
    g.p_floats = ctx->pf_Pn;
    g.sk_flags = ctx->pf_flags;
    g.abort_flag = ctx->step_abort;
    if ((rc = launch_gemm<kGemmResid>(ctx, g, s))) return rc;
    hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(n), dim3(kBlock), 0, s, (const float*)ctx->pf_X,
                       (const float*)L.rms_ffn, c.norm_eps, c.dim, ctx->pf_Xn);
    memset(&g, 0, sizeof(g));
    g.A = ctx->pf_Xn;
    g.lda = c.dim;
    g.B = L.w1;
    g.B3 = L.w3;
    g.ldb = c.dim;
    g.H = ctx->pf_H;
    g.ldh = c.hidden_dim;
    g.M = n;
    g.N = c.hidden_dim;
    g.K = c.dim;
    g.act = c.act;
    g.P = ctx->pf_P;
    g.p_floats = ctx->pf_Pn;
    g.sk_flags = ctx->pf_flags;
    g.abort_flag = ctx->step_abort;
    if ((rc = launch_gemm<kGemmSwiGLU>(ctx, g, s))) return rc;
    memset(&g, 0, sizeof(g));
    g.A = ctx->pf_H;
    g.lda = c.hidden_dim;
    g.B = L.w2;
    g.ldb = c.hidden_dim;
    g.C = ctx->pf_X;
    g.ldc = c.dim;
    g.M = n;
    g.N = c.dim;
    g.K = c.hidden_dim;
    g.P = ctx->pf_P;
    g.p_floats = ctx->pf_Pn;
    g.sk_flags = ctx->pf_flags;
    g.abort_flag = ctx->step_abort;
    if ((rc = launch_gemm<kGemmResid>(ctx, g, s))) return rc;
  }
  HIP_TRY(ctx, hipGetLastError());
  // a timed-out wait of a split-last-round GEMM, checked after the next synchronisation
  HIP_TRY(ctx, hipMemcpyAsync(ctx->argmax_host + 4, ctx->step_abort, sizeof(int), hipMemcpyDeviceToHost, s));
  if (!logits_host) return YHIP_OK;
  // last token: final rmsnorm + lm_head (reference src/infer.cpp:501-527)
  const int Rc = (c.vocab_size % 2 == 0) ? 2 : 1;
  MatvecArgs a = mv_base();
  a.w0 = ctx->wcls;
  a.row_step = (long)Rc * c.dim;
  a.r_step = c.dim;
  a.groups = c.vocab_size / Rc;
  a.K = c.dim;
  a.x = ctx->pf_X + (size_t)(n - 1) * c.dim;
  a.gain = ctx->rms_final;
  a.eps = c.norm_eps;
  a.out = ctx->logits;
  if (int rc = launch_matvec(ctx, a, kEpiStore, Rc, ctx->num_cus, s)) return rc;
  HIP_TRY(ctx, hipMemcpyAsync(ctx->logits_host, ctx->logits, (size_t)c.vocab_size * sizeof(float),
                              hipMemcpyDeviceToHost, s));
  HIP_TRY(ctx, hipStreamSynchronize(s));
  if (int rc = check_step_abort(ctx)) return rc;
  if (logits_host != ctx->logits_host) memcpy(logits_host, ctx->logits_host, (size_t)c.vocab_size * 4);
  return YHIP_OK;
}

}  // namespace

// ============================================================================================
// C-ABI
// ============================================================================================
extern "C" int yhip_create(const yhip_config* cfg, int device_ordinal, yhip_ctx** out) {
  if (!cfg || !out) return fail(nullptr, YHIP_EINVAL, "null argument");
  *out = nullptr;
  const yhip_config& c = *cfg;
  if (c.dim <= 0 || c.hidden_dim <= 0 || c.n_layers < 0 || c.vocab_size <= 0 || c.max_seq_len <= kKvSinks ||
      c.rotary_dim < 0 || c.rotary_dim > c.head_dim)
    return fail(nullptr, YHIP_EINVAL, "invalid config dimensions");
  if (c.dim % 8 || c.hidden_dim % 8 || (c.n_heads * c.head_dim) % 8)
    return fail(nullptr, YHIP_EINVAL, "dim, hidden_dim and n_heads*head_dim must be multiples of 8");
  if (c.dim > 16240 || c.hidden_dim > 16240 || c.n_heads * c.head_dim > 16240)
    return fail(nullptr, YHIP_EINVAL, "row lengths above 16240 are not supported");
  if (c.act != YHIP_ACT_GELU && c.act != YHIP_ACT_SILU) return fail(nullptr, YHIP_EINVAL, "unknown activation");
  if (int rc = check_attn_shape(nullptr, c.head_dim, c.n_heads, c.n_kv_heads)) return rc;
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || device_ordinal < 0 || device_ordinal >= ndev)
    return fail(nullptr, YHIP_EDEVICE, "no such HIP device");
  yhip_ctx* ctx = new yhip_ctx();
  ctx->c = c;
  ctx->device = device_ordinal;
  auto bail = [&](int rc) {
    yhip_destroy(ctx);
    return rc;
  };
  if (hipSetDevice(device_ordinal) != hipSuccess) return bail(fail(nullptr, YHIP_EDEVICE, "hipSetDevice failed"));
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device_ordinal) == hipSuccess && prop.multiProcessorCount > 0)
    ctx->num_cus = prop.multiProcessorCount;
  ctx->attn_splits = default_attn_splits(ctx->num_cus, c.n_kv_heads);
  if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess)
    return bail(fail(nullptr, YHIP_EDEVICE, "stream create failed"));

  // Weights: one allocation, 256-byte aligned sub-buffers.
  const size_t dim = c.dim, hid = c.hidden_dim, qd = ctx->q_dim(), kvd = ctx->kv_dim(), V = c.vocab_size;
  size_t per_layer = 0;
  auto take = [&](size_t bytes) {
    size_t off = per_layer;
    per_layer = align_up(per_layer + bytes, 256);
    return off;
  };
  const size_t o_qkv = take((qd + 2 * kvd) * dim * 2), o_wo = take(dim * qd * 2), o_w1 = take(hid * dim * 2),
               o_w3 = take(hid * dim * 2), o_w2 = take(dim * hid * 2), o_ra = take(dim * 4), o_rf = take(dim * 4);
  const size_t g_emb = align_up(V * dim * 2, 256), g_cls = align_up(V * dim * 2, 256), g_rf = align_up(dim * 4, 256);
  ctx->wbytes = per_layer * c.n_layers + g_emb + g_cls + g_rf;
  if (hipMalloc(&ctx->wbase, ctx->wbytes) != hipSuccess)
    return bail(fail(nullptr, YHIP_EDEVICE, "out of device memory for weights"));
  ctx->layers.resize(c.n_layers);
  for (int l = 0; l < c.n_layers; ++l) {
    char* b = ctx->wbase + per_layer * l;
    LayerW& L = ctx->layers[l];
    L.wqkv = (uint16_t*)(b + o_qkv);
    L.wo = (uint16_t*)(b + o_wo);
    L.w1 = (uint16_t*)(b + o_w1);
    L.w3 = (uint16_t*)(b + o_w3);
    L.w2 = (uint16_t*)(b + o_w2);
    L.rms_att = (float*)(b + o_ra);
    L.rms_ffn = (float*)(b + o_rf);
  }
  char* gb = ctx->wbase + per_layer * c.n_layers;
  ctx->embed = (uint16_t*)gb;
  ctx->wcls = (uint16_t*)(gb + g_emb);
  ctx->rms_final = (float*)(gb + g_emb + g_cls);

  // KV caches, zeroed (reference src/model.cpp:203-204).
  ctx->kv_elems = (size_t)c.n_kv_heads * c.head_dim * c.max_seq_len;
  const size_t kv_bytes = ctx->kv_elems * 2 * 2 * std::max(1, c.n_layers);
  if (hipMalloc(&ctx->kv, kv_bytes) != hipSuccess) return bail(fail(nullptr, YHIP_EDEVICE, "out of device memory for KV"));
  if (hipMemset(ctx->kv, 0, kv_bytes) != hipSuccess) return bail(fail(nullptr, YHIP_EDEVICE, "KV memset failed"));

  // Activations.
  size_t ab = 0;
  auto atake = [&](size_t bytes) {
    size_t off = ab;
    ab = align_up(ab + bytes, 256);
    return off;
  };
  const size_t a_x = atake(dim * 4), a_q = atake(qd * 4), a_att = atake(qd * 4), a_hb = atake(hid * 4),
               a_lg = atake(V * 4), a_part = atake((size_t)c.n_heads * 64 * (c.head_dim + 2) * 4),
               a_tk = atake(64 * 4), a_am = atake(64), a_key = atake(64), a_par = atake(sizeof(StepParams)),
               a_if = atake((size_t)c.head_dim / 2 * 4), a_cs = atake((size_t)c.head_dim * 4),
               a_sync = atake((size_t)kSyncWords * sizeof(unsigned)), a_skey = atake(2 * sizeof(unsigned long long)),
               a_sa = atake(256), a_racc = atake(dim * sizeof(unsigned long long)),
               a_ovf = atake(dim * sizeof(float));
  if (hipMalloc(&ctx->abase, ab) != hipSuccess) return bail(fail(nullptr, YHIP_EDEVICE, "out of device memory"));
  if (hipMemset(ctx->abase, 0, ab) != hipSuccess) return bail(fail(nullptr, YHIP_EDEVICE, "memset failed"));
  ctx->x = (float*)(ctx->abase + a_x);
  ctx->q = (float*)(ctx->abase + a_q);
  ctx->att = (float*)(ctx->abase + a_att);
  ctx->hb = (float*)(ctx->abase + a_hb);
  ctx->logits = (float*)(ctx->abase + a_lg);
  ctx->partial = (float*)(ctx->abase + a_part);
  ctx->tickets = (unsigned*)(ctx->abase + a_tk);
  ctx->argmax_dev = (int*)(ctx->abase + a_am);
  ctx->argmax_key = (unsigned long long*)(ctx->abase + a_key);
  ctx->params = (StepParams*)(ctx->abase + a_par);
  ctx->inv_freq = (float*)(ctx->abase + a_if);
  ctx->rope_cs = (float*)(ctx->abase + a_cs);
  ctx->sync = (unsigned*)(ctx->abase + a_sync);
  ctx->step_keys = (unsigned long long*)(ctx->abase + a_skey);
  ctx->step_abort = (unsigned*)(ctx->abase + a_sa);
  ctx->rowacc = (unsigned long long*)(ctx->abase + a_racc);
  ctx->rowovf = (float*)(ctx->abase + a_ovf);
  {
    const std::vector<float> f = make_inv_freq(c.head_dim, c.rotary_dim, c.rope_theta);
    if (hipMemcpy(ctx->inv_freq, f.data(), f.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
      return bail(fail(nullptr, YHIP_EDEVICE, "upload of rotary frequencies failed"));
  }
  if (hipHostMalloc((void**)&ctx->logits_host, V * 4, hipHostMallocDefault) != hipSuccess ||
      hipHostMalloc((void**)&ctx->argmax_host, 64, hipHostMallocDefault) != hipSuccess)
    return bail(fail(nullptr, YHIP_EDEVICE, "pinned host allocation failed"));
  memset(ctx->argmax_host, 0, 64);

  // Single-launch decode: one workgroup per CU, all co-resident (cooperative launch).
  ctx->layout = LayerLayout{ctx->wbase, (long)per_layer, (long)o_qkv, (long)o_wo, (long)o_w1, (long)o_w3,
                            (long)o_w2, (long)o_ra, (long)o_rf, ctx->kv, (long)ctx->kv_elems};
  // every (kv head, KV slice) of the attention phase needs a workgroup of the grid
  if (ctx->num_cus <= kStepMaxBlocks && ctx->num_cus >= c.n_kv_heads) {
    ctx->step_fn = select_step_kernel(c, ctx->q_dim(), false);
    ctx->step_fn_atto = select_step_kernel(c, ctx->q_dim(), true);
  }
  for (const void** fn : {&ctx->step_fn, &ctx->step_fn_atto}) {  // one resident workgroup per CU at least
    int per_cu = 0;
    if (*fn && (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, *fn, kStepThreads, 0) != hipSuccess || per_cu < 1))
      *fn = nullptr;
  }
  if (!ctx->step_fn) ctx->step_fn_atto = nullptr;  // available as an option; the per-op graph is the default
  *out = ctx;
  return YHIP_OK;
}

extern "C" int yhip_destroy(yhip_ctx* ctx) {
  if (!ctx) return YHIP_OK;
  hipSetDevice(ctx->device);
  if (ctx->stream) hipStreamSynchronize(ctx->stream);
  drop_graphs(ctx);
  if (ctx->pf_base) hipFree(ctx->pf_base);
  if (ctx->ev0) hipEventDestroy(ctx->ev0);
  if (ctx->ev1) hipEventDestroy(ctx->ev1);
  if (ctx->wbase) hipFree(ctx->wbase);
  if (ctx->kv) hipFree(ctx->kv);
  if (ctx->abase) hipFree(ctx->abase);
  if (ctx->logits_host) hipHostFree(ctx->logits_host);
  for (int k = 0; k < yhip_ctx::kStageBufs; ++k) {
    if (ctx->stage[k]) hipHostFree(ctx->stage[k]);
    if (ctx->stage_ev[k]) hipEventDestroy(ctx->stage_ev[k]);
  }
  if (ctx->argmax_host) hipHostFree(ctx->argmax_host);
  if (ctx->stream) hipStreamDestroy(ctx->stream);
  delete ctx;
  return YHIP_OK;
}

// ---- weight upload -------------------------------------------------------------------------
// A copy from pageable memory makes the runtime bounce every byte through its own small pinned
// buffers one piece at a time. Large tensors instead go through a ring of kStageBufs pinned chunks:
// host threads fill chunk k from the source (an mmapped checkpoint or any host buffer) while the DMA
// engine drains the chunks filled before it; a chunk is refilled once the event recorded after its
// copy has completed. Tensors under 64 KB (norm gains) are copied directly.
namespace {
void parallel_copy(char* dst, const char* src, size_t n, int threads) {
  constexpr size_t kMinPerThread = 4u << 20;
  const int t = (int)std::max<size_t>(1, std::min<size_t>((size_t)std::max(threads, 1), n / kMinPerThread));
  if (t == 1) {
    memcpy(dst, src, n);
    return;
  }
  const size_t per = (n / t + 4095) & ~(size_t)4095;
  std::vector<std::thread> pool;
  pool.reserve(t);
  for (int i = 0; i < t; ++i) {
    const size_t b = std::min(n, (size_t)i * per), e = std::min(n, b + per);
    if (b < e) pool.emplace_back([=] { memcpy(dst + b, src + b, e - b); });
  }
  for (std::thread& th : pool) th.join();
}
}  // namespace

static int ensure_stage(yhip_ctx* ctx, size_t chunk) {
  if (ctx->stage_bytes == chunk) return YHIP_OK;
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  for (int k = 0; k < yhip_ctx::kStageBufs; ++k) {
    if (ctx->stage[k]) HIP_TRY(ctx, hipHostFree(ctx->stage[k]));
    ctx->stage[k] = nullptr;
  }
  ctx->stage_bytes = 0;
  for (int k = 0; k < yhip_ctx::kStageBufs; ++k) {
    if (hipHostMalloc((void**)&ctx->stage[k], chunk, hipHostMallocDefault) != hipSuccess) {
      ctx->stage[k] = nullptr;
      return fail(ctx, YHIP_EDEVICE, "pinned staging buffer allocation failed");
    }
    if (!ctx->stage_ev[k]) HIP_TRY(ctx, hipEventCreateWithFlags(&ctx->stage_ev[k], hipEventDisableTiming));
  }
  ctx->stage_bytes = chunk;
  return YHIP_OK;
}

// Enqueues the host → device copy of `bytes` bytes on the context's stream. The source may be
// released once the stream has been synchronised.
static int upload_h2d(yhip_ctx* ctx, void* dst, const void* src, size_t bytes) {
  const size_t chunk = (size_t)g_upload_stage_mb << 20;
  if (chunk == 0 || bytes < ((size_t)64 << 10)) {
    HIP_TRY(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    return YHIP_OK;
  }
  if (int rc = ensure_stage(ctx, chunk)) return rc;
  const char* s = static_cast<const char*>(src);
  char* d = static_cast<char*>(dst);
  for (size_t off = 0; off < bytes; off += chunk) {
    const size_t n = std::min(chunk, bytes - off);
    const int k = ctx->stage_next;
    ctx->stage_next = (k + 1) % yhip_ctx::kStageBufs;
    HIP_TRY(ctx, hipEventSynchronize(ctx->stage_ev[k]));  // chunk k's previous copy has drained
    parallel_copy(ctx->stage[k], s + off, n, g_upload_threads);
    HIP_TRY(ctx, hipMemcpyAsync(d + off, ctx->stage[k], n, hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(ctx, hipEventRecord(ctx->stage_ev[k], ctx->stream));
  }
  return YHIP_OK;
}

extern "C" int yhip_upload_layer(yhip_ctx* ctx, int layer, const float* rms_att, const float* rms_ffn,
                                 const uint16_t* wq, const uint16_t* wk, const uint16_t* wv, const uint16_t* wo,
                                 const uint16_t* w1, const uint16_t* w2, const uint16_t* w3) {
  if (!ctx) return fail(nullptr, YHIP_EINVAL, "null context");
  if (layer < 0 || layer >= ctx->c.n_layers) return fail(ctx, YHIP_EINVAL, "layer index out of range");
  if (!rms_att || !rms_ffn || !wq || !wk || !wv || !wo || !w1 || !w2 || !w3)
    return fail(ctx, YHIP_EINVAL, "null weight pointer");
  const yhip_config& c = ctx->c;
  const size_t dim = c.dim, hid = c.hidden_dim, qd = ctx->q_dim(), kvd = ctx->kv_dim();
  LayerW& L = ctx->layers[layer];
  hipStream_t s = ctx->stream;
  HIP_TRY(ctx, hipSetDevice(ctx->device));
  int rc = 0;
  if ((rc = upload_h2d(ctx, L.wqkv, wq, qd * dim * 2)) || (rc = upload_h2d(ctx, L.wqkv + qd * dim, wk, kvd * dim * 2)) ||
      (rc = upload_h2d(ctx, L.wqkv + (qd + kvd) * dim, wv, kvd * dim * 2)) ||
      (rc = upload_h2d(ctx, L.wo, wo, dim * qd * 2)) || (rc = upload_h2d(ctx, L.w1, w1, hid * dim * 2)) ||
      (rc = upload_h2d(ctx, L.w3, w3, hid * dim * 2)) || (rc = upload_h2d(ctx, L.w2, w2, dim * hid * 2)) ||
      (rc = upload_h2d(ctx, L.rms_att, rms_att, dim * 4)) || (rc = upload_h2d(ctx, L.rms_ffn, rms_ffn, dim * 4))) {
    hipStreamSynchronize(s);
    return rc;
  }
  HIP_TRY(ctx, hipStreamSynchronize(s));  // host buffers may be released after return
  L.loaded = true;
  return YHIP_OK;
}

extern "C" int yhip_upload_globals(yhip_ctx* ctx, const uint16_t* embed, const float* rms_final, const uint16_t* wcls) {
  if (!ctx) return fail(nullptr, YHIP_EINVAL, "null context");
  if (!embed || !rms_final) return fail(ctx, YHIP_EINVAL, "null weight pointer");
  const yhip_config& c = ctx->c;
  const size_t n = (size_t)c.vocab_size * c.dim;
  HIP_TRY(ctx, hipSetDevice(ctx->device));
  int rc = 0;
  if ((rc = upload_h2d(ctx, ctx->embed, embed, n * 2)) || (rc = upload_h2d(ctx, ctx->wcls, wcls ? wcls : embed, n * 2)) ||
      (rc = upload_h2d(ctx, ctx->rms_final, rms_final, (size_t)c.dim * 4))) {
    hipStreamSynchronize(ctx->stream);
    return rc;
  }
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  ctx->globals_loaded = true;
  return YHIP_OK;
}

extern "C" int yhip_forward(yhip_ctx* ctx, int token, int pos, int mode, float* logits_host) {
  if (!ctx) return fail(nullptr, YHIP_EINVAL, "null context");
  if (mode != YHIP_MODE_HYDRATE && mode != YHIP_MODE_LOGITS) return fail(ctx, YHIP_EINVAL, "unknown mode");
  if (mode == YHIP_MODE_LOGITS && !logits_host) return fail(ctx, YHIP_EINVAL, "null logits buffer");
  if (int rc = run_step(ctx, token, pos, mode)) return rc;
  if (mode == YHIP_MODE_HYDRATE) return YHIP_OK;
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  collect_stats(ctx);
  if (int rc = check_flow_status(ctx)) return rc;
  if (int rc = check_step_abort(ctx)) return rc;
  if (logits_host != ctx->logits_host) memcpy(logits_host, ctx->logits_host, (size_t)ctx->c.vocab_size * 4);
  return YHIP_OK;
}

extern "C" int yhip_forward_argmax(yhip_ctx* ctx, int token, int pos, int* next_token) {
  if (!ctx) return fail(nullptr, YHIP_EINVAL, "null context");
  if (!next_token) return fail(ctx, YHIP_EINVAL, "null output");
  if (int rc = run_step(ctx, token, pos, 2)) return rc;
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  collect_stats(ctx);
  if (int rc = check_flow_status(ctx)) return rc;
  if (int rc = check_step_abort(ctx)) return rc;
  if (ctx->c.vocab_size % 2 == 0) {  // the fused lm_head's packed key (argmax_key, or the single launch's)
    unsigned long long key;
    memcpy(&key, ctx->argmax_host + 2, sizeof(key));
    *next_token = key == 0 ? 0 : (int)~(unsigned)(key & 0xffffffffull);
  } else {
    *next_token = *ctx->argmax_host;
  }
  return YHIP_OK;
}

extern "C" int yhip_prefill(yhip_ctx* ctx, const int* tokens, int n, int start_pos, float* logits_host) {
  if (!ctx) return fail(nullptr, YHIP_EINVAL, "null context");
  if (!tokens || n <= 0 || start_pos < 0) return fail(ctx, YHIP_EINVAL, "bad prefill arguments");
  const yhip_config& c = ctx->c;
  for (int i = 0; i < n; ++i)
    if (tokens[i] < 0 || tokens[i] >= c.vocab_size) return fail(ctx, YHIP_EINVAL, "token id out of range");
  if (!ctx->globals_loaded) return fail(ctx, YHIP_ESTATE, "globals not uploaded");
  for (int l = 0; l < c.n_layers; ++l)
    if (!ctx->layers[l].loaded) return fail(ctx, YHIP_ESTATE, "layer " + std::to_string(l) + " not uploaded");
  HIP_TRY(ctx, hipSetDevice(ctx->device));
  if ((long)start_pos + n <= c.max_seq_len && prefill_supported(c, ctx->q_dim()))
    return run_prefill(ctx, tokens, n, start_pos, logits_host);
  // token by token through the decode path (ring positions, or shapes without the batched kernels)
  for (int i = 0; i < n; ++i) {
    const bool last = i == n - 1 && logits_host;
    if (int rc = yhip_forward(ctx, tokens[i], start_pos + i, last ? YHIP_MODE_LOGITS : YHIP_MODE_HYDRATE,
                              last ? logits_host : nullptr))
      return rc;
  }
  return YHIP_OK;
}

extern "C" float* yhip_logits_host(yhip_ctx* ctx) { return ctx ? ctx->logits_host : nullptr; }

extern "C" int yhip_kv_read(yhip_ctx* ctx, int layer, uint16_t* k_host, uint16_t* v_host) {
  if (!ctx) return fail(nullptr, YHIP_EINVAL, "null context");
  if (layer < 0 || layer >= ctx->c.n_layers) return fail(ctx, YHIP_EINVAL, "layer index out of range");
  HIP_TRY(ctx, hipSetDevice(ctx->device));
  const size_t bytes = ctx->kv_elems * 2;
  if (k_host) HIP_TRY(ctx, hipMemcpyAsync(k_host, ctx->kcache(layer), bytes, hipMemcpyDeviceToHost, ctx->stream));
  if (v_host) HIP_TRY(ctx, hipMemcpyAsync(v_host, ctx->vcache(layer), bytes, hipMemcpyDeviceToHost, ctx->stream));
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  return YHIP_OK;
}

extern "C" int yhip_kv_write(yhip_ctx* ctx, int layer, const uint16_t* k_host, const uint16_t* v_host) {
  if (!ctx) return fail(nullptr, YHIP_EINVAL, "null context");
  if (layer < 0 || layer >= ctx->c.n_layers) return fail(ctx, YHIP_EINVAL, "layer index out of range");
  HIP_TRY(ctx, hipSetDevice(ctx->device));
  const size_t bytes = ctx->kv_elems * 2;
  if (k_host) HIP_TRY(ctx, hipMemcpyAsync(ctx->kcache(layer), k_host, bytes, hipMemcpyHostToDevice, ctx->stream));
  if (v_host) HIP_TRY(ctx, hipMemcpyAsync(ctx->vcache(layer), v_host, bytes, hipMemcpyHostToDevice, ctx->stream));
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  return YHIP_OK;
}

// ---- KV cache fill for the attention-heavy workload -------------------------------------------
namespace {
__device__ __forceinline__ unsigned long long mix64(unsigned long long z) {  // splitmix64 finaliser
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
// Every K and V entry of every layer: fp16 of N(0, 1) (Box-Muller on two 24-bit uniforms of a
// counter hash) at positions below n_pos, zero above; positions follow the reference layouts
// (K [g][d/16][t][16], V [g][d][t]).
__global__ void kv_fill_normal_kernel(uint16_t* kv, size_t kv_elems, size_t total, int msl, int n_pos,
                                      unsigned long long seed) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const size_t within = i % kv_elems;        // element of this layer's K or V
    const bool is_v = (i / kv_elems) % 2 == 1;  // layer l: K at 2 l, V at 2 l + 1
    const int t = is_v ? (int)(within % msl) : (int)((within % (16 * (size_t)msl)) / 16);
    uint16_t h = 0;
    if (t < n_pos) {
      const unsigned long long r = mix64(seed + 0x9E3779B97F4A7C15ull * (i + 1));
      const float u1 = ((float)(r >> 40) + 1.0f) * (1.0f / 16777216.0f);  // (0, 1]
      const float u2 = (float)((r >> 16) & 0xFFFFFF) * (1.0f / 16777216.0f);
      const float z = sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2);
      h = __builtin_bit_cast(uint16_t, (f16)z);
    }
    kv[i] = h;
  }
}
}  // namespace

extern "C" int yhip_kv_fill_normal(yhip_ctx* ctx, int n_positions, unsigned long long seed) {
  if (!ctx) return fail(nullptr, YHIP_EINVAL, "null context");
  if (n_positions < 0 || n_positions > ctx->c.max_seq_len) return fail(ctx, YHIP_EINVAL, "n_positions out of range");
  HIP_TRY(ctx, hipSetDevice(ctx->device));
  const size_t total = ctx->kv_elems * 2 * (size_t)std::max(1, ctx->c.n_layers);
  hipLaunchKernelGGL(kv_fill_normal_kernel, dim3(ctx->num_cus * 8), dim3(256), 0, ctx->stream, ctx->kv, ctx->kv_elems,
                     total, ctx->c.max_seq_len, n_positions, seed);
  HIP_TRY(ctx, hipGetLastError());
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  return YHIP_OK;
}

extern "C" int yhip_set_option(yhip_ctx* ctx, const char* key, int value) {
  if (!key) return fail(ctx, YHIP_EINVAL, "null argument");
  if (!ctx) {
    if (!strcmp(key, "test_bpc")) {
      if (value < 0 || value > 64) return fail(nullptr, YHIP_EINVAL, "test_bpc must be in [0, 64]");
      g_test_bpc = value;
      return YHIP_OK;
    }
    if (!strcmp(key, "attn_mfma")) {
      g_attn_mfma = value != 0;
      return YHIP_OK;
    }
    if (!strcmp(key, "gemm_stages")) {  // -1: chosen per shape; 2..4 LDS stages; 6 eight-wave large tiles
      if (value < -1 || (value >= 0 && value < 2) || value == 5 || value > 6)
        return fail(nullptr, YHIP_EINVAL, "gemm_stages must be -1, 2, 3, 4 or 6");
      g_gemm_auto = value < 0;
      if (value >= 0) g_gemm_stages = value;
      return YHIP_OK;
    }
    if (!strcmp(key, "gemm_ppsplit")) {
      g_gemm_ppsplit = value != 0;
      return YHIP_OK;
    }
    if (!strcmp(key, "gemm_bk")) {
      if (value != 32 && value != 64) return fail(nullptr, YHIP_EINVAL, "gemm_bk must be 32 or 64");
      g_gemm_bk = value;
      return YHIP_OK;
    }
    if (!strcmp(key, "gemm_ksplit")) {  // 0: chosen per shape; n >= 1: forced where the kernel allows
      if (value < 0 || value > 64) return fail(nullptr, YHIP_EINVAL, "gemm_ksplit must be in [0, 64]");
      g_gemm_ksplit = value;
      return YHIP_OK;
    }
    if (!strcmp(key, "upload_stage_mb")) {
      if (value < 0 || value > 1024) return fail(nullptr, YHIP_EINVAL, "upload_stage_mb must be in [0, 1024]");
      g_upload_stage_mb = value;
      return YHIP_OK;
    }
    if (!strcmp(key, "upload_threads")) {
      if (value < 1 || value > 64) return fail(nullptr, YHIP_EINVAL, "upload_threads must be in [1, 64]");
      g_upload_threads = value;
      return YHIP_OK;
    }
    if (!strcmp(key, "gemm_bm")) {
      if (value != 128 && value != 256) return fail(nullptr, YHIP_EINVAL, "gemm_bm must be 128 or 256");
      g_gemm_bm = value;
      return YHIP_OK;
    }
    return fail(nullptr, YHIP_EINVAL, std::string("unknown process-wide option ") + key);
  }
  hipSetDevice(ctx->device);
  hipStreamSynchronize(ctx->stream);
  if (!strcmp(key, "graph")) {
    ctx->use_graph = value != 0;
  } else if (!strcmp(key, "stats")) {
    if (value && !ctx->ev0) {
      HIP_TRY(ctx, hipEventCreate(&ctx->ev0));
      HIP_TRY(ctx, hipEventCreate(&ctx->ev1));
    }
    ctx->stats = value != 0;
    ctx->stats_pending = false;
    ctx->stats_us = 0.0;
    ctx->stats_steps = 0;
    return YHIP_OK;  // graphs stay valid: the events are recorded outside them
  } else if (!strcmp(key, "single_launch")) {
    if (value && !ctx->step_fn) return fail(ctx, YHIP_EINVAL, "no single-launch decode kernel for this shape");
    ctx->use_flow = value != 0;
  } else if (!strcmp(key, "step_spin_limit")) {
    if (value < 0) return fail(ctx, YHIP_EINVAL, "step_spin_limit must be >= 0");
    ctx->step_spin_limit = value ? (unsigned)value : kSpinLimit;
  } else if (!strcmp(key, "step_atto_max")) {
    if (value < 0) return fail(ctx, YHIP_EINVAL, "step_atto_max must be >= 0");
    ctx->step_atto_max = value;
  } else if (!strcmp(key, "attn_splits")) {
    if (value < 1 || value > 64) return fail(ctx, YHIP_EINVAL, "attn_splits must be in [1, 64]");
    ctx->attn_splits = value;
  } else if (!strcmp(key, "attn_mfma")) {
    ctx->attn_mfma = value != 0;
  } else if (!strcmp(key, "split_o")) {
    ctx->split_o = value != 0;
  } else if (!strcmp(key, "attn_o")) {
    ctx->attn_o = value != 0;
  } else if (!strcmp(key, "attn_o_max")) {
    if (value < 0) return fail(ctx, YHIP_EINVAL, "attn_o_max must be >= 0");
    ctx->attn_o_max = value;
  } else if (!strncmp(key, "bpc_", 4)) {
    static const char* names[5] = {"bpc_qkv", "bpc_o", "bpc_w13", "bpc_w2", "bpc_lm"};
    int i = 0;
    while (i < 5 && strcmp(key, names[i])) ++i;
    if (i == 5) return fail(ctx, YHIP_EINVAL, std::string("unknown option ") + key);
    if (value < 0 || value > 16) return fail(ctx, YHIP_EINVAL, "workgroups per CU must be in [0, 16]");
    ctx->mv_bpc[i] = value;
  } else if (!strcmp(key, "attn_min_slice")) {
    if (value < 0 || value % 64) return fail(ctx, YHIP_EINVAL, "attn_min_slice must be 0 or a positive multiple of 64");
    ctx->attn_min_slice = value;
  } else {
    return fail(ctx, YHIP_EINVAL, std::string("unknown option ") + key);
  }
  drop_graphs(ctx);
  return YHIP_OK;
}

extern "C" int yhip_debug_read(yhip_ctx* ctx, int which, float* host, size_t n) {
  if (!ctx || !host) return fail(ctx, YHIP_EINVAL, "null argument");
  const yhip_config& c = ctx->c;
  const float* src = nullptr;
  size_t cap = 0;
  switch (which) {
    case 0: src = ctx->x; cap = c.dim; break;
    case 1: src = ctx->q; cap = ctx->q_dim(); break;
    case 2: src = ctx->att; cap = ctx->q_dim(); break;
    case 3: src = ctx->hb; cap = c.hidden_dim; break;
    case 4: src = ctx->logits; cap = c.vocab_size; break;
    case 5: src = ctx->inv_freq; cap = (size_t)c.head_dim / 2; break;
    default: return fail(ctx, YHIP_EINVAL, "unknown buffer");
  }
  if (n > cap) return fail(ctx, YHIP_EINVAL, "read larger than buffer");
  HIP_TRY(ctx, hipSetDevice(ctx->device));
  HIP_TRY(ctx, hipMemcpyAsync(host, src, n * 4, hipMemcpyDeviceToHost, ctx->stream));
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  return YHIP_OK;
}

extern "C" int yhip_step_plan(yhip_ctx* ctx, int pos, int* variant, int* slices, int* slice_len) {
  if (!ctx) return fail(nullptr, YHIP_EINVAL, "null context");
  if (pos < 0) return fail(ctx, YHIP_EINVAL, "negative position");
  const int kv_len = std::min(pos + 1, ctx->c.max_seq_len);
  int v = ctx->use_flow ? YHIP_STEP_SINGLE : step_variant(ctx, pos);
  int ns = 1, len = kv_len;
  if (ctx->use_flow) {  // the single launch: the whole context per workgroup when attention and O are one phase
    if (!step_atto(ctx, pos)) {
      len = attn_mfma_chunk(kv_len, step_nsplit(ctx), 0);
      ns = (kv_len + len - 1) / len;
    }
  } else if (v != YHIP_STEP_ATTN_O) {
    // the same rules the launches apply (the SIMT kernel in 64-key granules)
    const bool mfma = attn_uses_mfma(ctx);
    const int ms = attn_min_slice_for(ctx, mfma);
    len = mfma ? attn_mfma_chunk(kv_len, ctx->attn_splits, ms) : attn_chunk(kv_len, ctx->attn_splits, ms);
    ns = (kv_len + len - 1) / len;
  }
  if (variant) *variant = v;
  if (slices) *slices = ns;
  if (slice_len) *slice_len = len;
  return YHIP_OK;
}

extern "C" int yhip_step_stats(const yhip_ctx* ctx, double* us_total, int* steps) {
  if (!ctx || !us_total || !steps) return fail(nullptr, YHIP_EINVAL, "null argument");
  *us_total = ctx->stats_us;
  *steps = ctx->stats_steps;
  return YHIP_OK;
}

extern "C" const char* yhip_last_error(const yhip_ctx* ctx) { return ctx ? ctx->err.c_str() : g_thread_err.c_str(); }

// ============================================================================================
// Kernel-level hooks (test only; allocate per call).
// ============================================================================================
namespace {

struct DevBufs {
  std::vector<void*> ptrs;
  ~DevBufs() {
    for (void* p : ptrs) hipFree(p);
  }
  template <class T>
  T* alloc(size_t n, const void* init = nullptr) {
    void* p = nullptr;
    if (hipMalloc(&p, std::max<size_t>(n, 1) * sizeof(T)) != hipSuccess) return nullptr;
    ptrs.push_back(p);
    if (init) {
      if (hipMemcpy(p, init, n * sizeof(T), hipMemcpyHostToDevice) != hipSuccess) return nullptr;
    } else {
      hipMemset(p, 0, std::max<size_t>(n, 1) * sizeof(T));
    }
    return (T*)p;
  }
};

int device_cus() {
  static std::atomic<int> cached[64] = {};  // per device, looked up once
  int dev = 0;
  hipGetDevice(&dev);
  if (dev >= 0 && dev < 64 && cached[dev].load(std::memory_order_relaxed) > 0)
    return cached[dev].load(std::memory_order_relaxed);
  int cus = 256;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) == hipSuccess && prop.multiProcessorCount > 0) cus = prop.multiProcessorCount;
  if (dev >= 0 && dev < 64) cached[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

// The attention hooks' slice plan. nsplit 0: the decode step's own (default_attn_splits slices per
// kv head; the matrix-core kernel picks the slice length from the context length, attn_mfma_chunk;
// the SIMT kernel takes slices of at least 64 keys). nsplit > 0: that many slices of at least 64.
void hook_slice_plan(int head_dim, int max_seq_len, int n_kv_heads, int& nsplit, int& min_slice) {
  const bool mfma = g_attn_mfma && head_dim % 32 == 0 && max_seq_len % 32 == 0;
  if (nsplit <= 0) {
    nsplit = default_attn_splits(device_cus(), n_kv_heads);
    min_slice = mfma ? 0 : 64;
  } else {
    min_slice = 64;
  }
}

#define TRY_ALLOC(p) \
  if (!(p)) return fail(nullptr, YHIP_EDEVICE, "device allocation failed")

}  // namespace

extern "C" int yhip_test_matvec(const float* x, const float* gain, float eps, const uint16_t* w, int n, int d,
                                const float* resid, float* out) {
  if (!x || !w || !out || n <= 0 || d <= 0) return fail(nullptr, YHIP_EINVAL, "bad argument");
  DevBufs b;
  float* dx = b.alloc<float>(n, x);
  TRY_ALLOC(dx);
  float* dg = gain ? b.alloc<float>(n, gain) : nullptr;
  if (gain) TRY_ALLOC(dg);
  uint16_t* dw = b.alloc<uint16_t>((size_t)n * d, w);
  TRY_ALLOC(dw);
  float* dout = b.alloc<float>(d, resid);
  TRY_ALLOC(dout);
  MatvecArgs a = mv_base();
  a.w0 = dw;
  a.K = n;
  a.x = dx;
  a.gain = dg;
  a.eps = eps;
  a.out = dout;
  const int R = (d % 2 == 0) ? 2 : 1;
  a.row_step = (long)R * n;
  a.r_step = n;
  a.groups = d / R;
  if (int rc = launch_matvec(nullptr, a, resid ? kEpiResidual : kEpiStore, R, device_cus(), nullptr, g_test_bpc))
    return rc;
  HIP_TRY(nullptr, hipDeviceSynchronize());
  HIP_TRY(nullptr, hipMemcpy(out, dout, (size_t)d * 4, hipMemcpyDeviceToHost));
  return YHIP_OK;
}

extern "C" int yhip_test_ffn(const float* x, const float* gain, float eps, const uint16_t* w1, const uint16_t* w2,
                             const uint16_t* w3, int hidden_dim, int dim, int act, const float* resid, float* out) {
  if (!x || !w1 || !w2 || !w3 || !out || hidden_dim <= 0 || dim <= 0) return fail(nullptr, YHIP_EINVAL, "bad argument");
  DevBufs b;
  float* dx = b.alloc<float>(dim, x);
  TRY_ALLOC(dx);
  float* dg = gain ? b.alloc<float>(dim, gain) : nullptr;
  if (gain) TRY_ALLOC(dg);
  uint16_t* d1 = b.alloc<uint16_t>((size_t)hidden_dim * dim, w1);
  uint16_t* d2 = b.alloc<uint16_t>((size_t)hidden_dim * dim, w2);
  uint16_t* d3 = b.alloc<uint16_t>((size_t)hidden_dim * dim, w3);
  float* dh = b.alloc<float>(hidden_dim);
  float* dout = b.alloc<float>(dim, resid);
  TRY_ALLOC(d1);
  TRY_ALLOC(d2);
  TRY_ALLOC(d3);
  TRY_ALLOC(dh);
  TRY_ALLOC(dout);
  const int cus = device_cus();
  MatvecArgs a = mv_base();
  a.w0 = d1;
  a.w1 = d3;
  a.row_step = dim;
  a.groups = hidden_dim;
  a.K = dim;
  a.x = dx;
  a.gain = dg;
  a.eps = eps;
  a.out = dh;
  a.act = act;
  if (int rc = launch_matvec(nullptr, a, kEpiSwiGLU, 2, cus, nullptr, g_test_bpc)) return rc;
  a = mv_base();
  a.w0 = d2;
  a.row_step = hidden_dim;
  a.r_step = hidden_dim;
  a.groups = dim;
  a.K = hidden_dim;
  a.x = dh;
  a.out = dout;
  if (int rc = launch_matvec(nullptr, a, resid ? kEpiResidual : kEpiStore, 1, cus, nullptr, g_test_bpc))
    return rc;
  HIP_TRY(nullptr, hipDeviceSynchronize());
  HIP_TRY(nullptr, hipMemcpy(out, dout, (size_t)dim * 4, hipMemcpyDeviceToHost));
  return YHIP_OK;
}

extern "C" int yhip_test_attention(const float* q, uint16_t* kcache, const uint16_t* vcache, int head_dim, int pos,
                                   int max_seq_len, int n_heads, int n_kv_heads, int nsplit, float rope_theta,
                                   int rotary_dim, float* att_out) {
  if (!q || !kcache || !vcache || !att_out || pos < 0 || max_seq_len <= kKvSinks)
    return fail(nullptr, YHIP_EINVAL, "bad argument");
  if (int rc = check_attn_shape(nullptr, head_dim, n_heads, n_kv_heads)) return rc;
  int min_slice = 64;
  hook_slice_plan(head_dim, max_seq_len, n_kv_heads, nsplit, min_slice);
  if (nsplit > 64) return fail(nullptr, YHIP_EINVAL, "nsplit must be at most 64");
  const size_t kv = (size_t)n_kv_heads * head_dim * max_seq_len;
  DevBufs b;
  float* dq = b.alloc<float>((size_t)n_heads * head_dim, q);
  uint16_t* dk = b.alloc<uint16_t>(kv, kcache);
  uint16_t* dv = b.alloc<uint16_t>(kv, vcache);
  float* dpart = b.alloc<float>((size_t)n_heads * nsplit * (head_dim + 2));
  unsigned* dt = b.alloc<unsigned>(64);
  float* dout = b.alloc<float>((size_t)n_heads * head_dim);
  StepParams hp{0, pos, {0, 0}};
  StepParams* dp = b.alloc<StepParams>(1, &hp);
  const std::vector<float> freqs = make_inv_freq(head_dim, rotary_dim, rope_theta);
  float* dfreq = b.alloc<float>(freqs.size(), freqs.data());
  TRY_ALLOC(dq);
  TRY_ALLOC(dk);
  TRY_ALLOC(dv);
  TRY_ALLOC(dpart);
  TRY_ALLOC(dt);
  TRY_ALLOC(dout);
  TRY_ALLOC(dp);
  TRY_ALLOC(dfreq);
  AttnArgs t;
  t.q = dq;
  t.kcache = dk;
  t.vcache = dv;
  t.partial = dpart;
  t.tickets = dt;
  t.out = dout;
  t.head_dim = head_dim;
  t.n_heads = n_heads;
  t.n_kv_heads = n_kv_heads;
  t.msl = max_seq_len;
  t.nsplit = nsplit;
  t.min_slice = min_slice;
  t.inv_freq = dfreq;
  t.params = dp;
  if (int rc = launch_attention(nullptr, t, nullptr)) return rc;
  HIP_TRY(nullptr, hipDeviceSynchronize());
  HIP_TRY(nullptr, hipMemcpy(att_out, dout, (size_t)n_heads * head_dim * 4, hipMemcpyDeviceToHost));
  HIP_TRY(nullptr, hipMemcpy(kcache, dk, kv * 2, hipMemcpyDeviceToHost));
  return YHIP_OK;
}

// ---- attention without allocation ----------------------------------------------------------
// The split-KV attention's working memory (per-slice partials, per-kv-head tickets, the step
// parameters and the rotary frequencies) in one file-scope device array: each GPU the library runs
// on holds its own copy until the process ends. Header: tickets at 0 (64 words), StepParams at
// 256, rotary frequencies at 512 (64 floats); partials from 4096.
namespace {
constexpr size_t kNaHeaderBytes = 4096;
constexpr size_t kNaPartialBytes = (size_t)1 << 20;
constexpr size_t kNaScratchBytes = kNaHeaderBytes + kNaPartialBytes;
constexpr int kNaMaxDevices = 64;
}  // namespace

static __device__ __align__(256) unsigned char scratch[kNaScratchBytes];

namespace {
std::mutex g_scratch_mu;
unsigned char* g_scratch_dev[kNaMaxDevices] = {};  // device address of `scratch` on each GPU

// The scratch array's address on the current device, looked up once per device. In host code the
// array's name is only a stand-in: kernels and copies take this address.
unsigned char* noalloc_scratch() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kNaMaxDevices) {
    fail(nullptr, YHIP_EDEVICE, "no current HIP device (or device index above 63)");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      fail(nullptr, YHIP_EDEVICE, std::string("scratch symbol lookup: ") + hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_dev[dev] = static_cast<unsigned char*>(p);
  }
  return g_scratch_dev[dev];
}

struct NaSetup {
  int pos, n_freq;
  float inv_freq[64];
};

// Clears the tickets (the merge expects zero) and writes the step parameters and frequencies: a
// kernel rather than memsets or copies, so the sequence also records cleanly into a graph.
__global__ void noalloc_setup_kernel(unsigned char* base, NaSetup su) {
  unsigned* tickets = reinterpret_cast<unsigned*>(base);
  StepParams* params = reinterpret_cast<StepParams*>(base + 256);
  float* freq = reinterpret_cast<float*>(base + 512);
  const int t = threadIdx.x;
  tickets[t] = 0u;
  if (t < su.n_freq) freq[t] = su.inv_freq[t];
  if (t == 0) {
    params->token = 0;
    params->pos = su.pos;
    params->pad[0] = params->pad[1] = 0;
  }
}
}  // namespace

extern "C" int yhip_attention_noalloc(const float* q, uint16_t* kcache, const uint16_t* vcache, int head_dim, int pos,
                                      int max_seq_len, int n_heads, int n_kv_heads, int nsplit, float rope_theta,
                                      int rotary_dim, float* att_out, void* stream) {
  if (!q || !kcache || !vcache || !att_out || pos < 0 || max_seq_len <= kKvSinks || rotary_dim < 0 ||
      rotary_dim > head_dim)
    return fail(nullptr, YHIP_EINVAL, "bad argument");
  if (int rc = check_attn_shape(nullptr, head_dim, n_heads, n_kv_heads)) return rc;
  int min_slice = 64;
  hook_slice_plan(head_dim, max_seq_len, n_kv_heads, nsplit, min_slice);  // as yhip_test_attention
  if (nsplit > 64) return fail(nullptr, YHIP_EINVAL, "nsplit must be at most 64");
  const size_t part_bytes = (size_t)n_heads * nsplit * (head_dim + 2) * sizeof(float);
  if (part_bytes > kNaPartialBytes)
    return fail(nullptr, YHIP_EINVAL, "n_heads * nsplit * (head_dim + 2) floats exceed the 1 MiB attention scratch");
  unsigned char* base = noalloc_scratch();
  if (!base) return YHIP_EDEVICE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  NaSetup su;
  su.pos = pos;
  su.n_freq = head_dim / 2;
  fill_inv_freq(su.inv_freq, head_dim, rotary_dim, rope_theta);
  hipLaunchKernelGGL(noalloc_setup_kernel, dim3(1), dim3(64), 0, s, base, su);
  HIP_TRY(nullptr, hipGetLastError());
  AttnArgs t;
  t.q = q;
  t.kcache = kcache;
  t.vcache = vcache;
  t.partial = reinterpret_cast<float*>(base + kNaHeaderBytes);
  t.tickets = reinterpret_cast<unsigned*>(base);
  t.out = att_out;
  t.head_dim = head_dim;
  t.n_heads = n_heads;
  t.n_kv_heads = n_kv_heads;
  t.msl = max_seq_len;
  t.nsplit = nsplit;
  t.min_slice = min_slice;
  t.inv_freq = reinterpret_cast<const float*>(base + 512);
  t.params = reinterpret_cast<const StepParams*>(base + 256);
  return launch_attention(nullptr, t, s);
}

extern "C" int yhip_test_qkv(const float* x, const float* gain, float eps, const uint16_t* wq, const uint16_t* wk,
                             const uint16_t* wv, int dim, int n_heads, int n_kv_heads, int head_dim, int max_seq_len,
                             int rotary_dim, float rope_theta, float qkv_clip, int pos, float* q_out,
                             uint16_t* kcache, uint16_t* vcache) {
  if (!x || !wq || !wk || !wv || !q_out || !kcache || !vcache || dim <= 0 || head_dim <= 0 || head_dim % 2 ||
      n_heads <= 0 || n_kv_heads <= 0 || max_seq_len <= kKvSinks || pos < 0)
    return fail(nullptr, YHIP_EINVAL, "bad argument");
  const size_t qd = (size_t)n_heads * head_dim, kvd = (size_t)n_kv_heads * head_dim;
  const size_t kv = kvd * max_seq_len;
  DevBufs b;
  float* dx = b.alloc<float>(dim, x);
  float* dg = gain ? b.alloc<float>(dim, gain) : nullptr;
  uint16_t* dw = b.alloc<uint16_t>((qd + 2 * kvd) * dim);
  TRY_ALLOC(dx);
  if (gain) TRY_ALLOC(dg);
  TRY_ALLOC(dw);
  HIP_TRY(nullptr, hipMemcpy(dw, wq, qd * dim * 2, hipMemcpyHostToDevice));
  HIP_TRY(nullptr, hipMemcpy(dw + qd * dim, wk, kvd * dim * 2, hipMemcpyHostToDevice));
  HIP_TRY(nullptr, hipMemcpy(dw + (qd + kvd) * dim, wv, kvd * dim * 2, hipMemcpyHostToDevice));
  float* dq = b.alloc<float>(qd);
  uint16_t* dk = b.alloc<uint16_t>(kv, kcache);
  uint16_t* dv = b.alloc<uint16_t>(kv, vcache);
  StepParams hp{0, pos, {0, 0}};
  StepParams* dp = b.alloc<StepParams>(1, &hp);
  const std::vector<float> freqs = make_inv_freq(head_dim, rotary_dim, rope_theta);
  float* dfreq = b.alloc<float>(freqs.size(), freqs.data());
  float* dcs = b.alloc<float>(head_dim);
  TRY_ALLOC(dq);
  TRY_ALLOC(dk);
  TRY_ALLOC(dv);
  TRY_ALLOC(dp);
  TRY_ALLOC(dfreq);
  TRY_ALLOC(dcs);
  hipLaunchKernelGGL(rope_table_kernel, dim3(1), dim3(kBlock), 0, nullptr, (const float*)dfreq, dcs, head_dim / 2,
                     (const StepParams*)dp);
  HIP_TRY(nullptr, hipGetLastError());
  MatvecArgs a = mv_base();
  a.w0 = dw;
  a.row_step = 2L * dim;
  a.r_step = dim;
  a.groups = (int)((qd + 2 * kvd) / 2);
  a.K = dim;
  a.x = dx;
  a.gain = dg;
  a.eps = eps;
  a.out = dq;
  a.q_dim = (int)qd;
  a.kv_dim = (int)kvd;
  a.head_dim = head_dim;
  a.msl = max_seq_len;
  a.qkv_clip = qkv_clip;
  a.kcache = dk;
  a.vcache = dv;
  a.params = dp;
  a.rope_cs = dcs;
  if (int rc = launch_matvec(nullptr, a, kEpiQkvRope, 2, device_cus(), nullptr, g_test_bpc)) return rc;
  HIP_TRY(nullptr, hipDeviceSynchronize());
  HIP_TRY(nullptr, hipMemcpy(q_out, dq, qd * 4, hipMemcpyDeviceToHost));
  HIP_TRY(nullptr, hipMemcpy(kcache, dk, kv * 2, hipMemcpyDeviceToHost));
  HIP_TRY(nullptr, hipMemcpy(vcache, dv, kv * 2, hipMemcpyDeviceToHost));
  return YHIP_OK;
}

extern "C" int yhip_test_gemm(const uint16_t* a, const uint16_t* b, const uint16_t* b3, int M, int N, int K, int mode,
                              int act, float* c, uint16_t* h) {
  if (!a || !b || M <= 0 || N <= 0 || K <= 0 || mode < 0 || mode > 2) return fail(nullptr, YHIP_EINVAL, "bad argument");
  if (mode == kGemmSwiGLU ? (!b3 || !h) : !c) return fail(nullptr, YHIP_EINVAL, "bad argument");
  DevBufs d;
  const uint16_t* da = d.alloc<uint16_t>((size_t)M * K, a);
  const uint16_t* db = d.alloc<uint16_t>((size_t)N * K, b);
  const uint16_t* db3 = mode == kGemmSwiGLU ? d.alloc<uint16_t>((size_t)N * K, b3) : nullptr;
  float* dc = mode != kGemmSwiGLU ? d.alloc<float>((size_t)M * N, mode == kGemmResid ? c : nullptr) : nullptr;
  uint16_t* dh = mode == kGemmSwiGLU ? d.alloc<uint16_t>((size_t)M * N) : nullptr;
  const long pf = splitk_ws_floats(device_cus());
  float* dp = d.alloc<float>((size_t)pf);
  unsigned* dflags = d.alloc<unsigned>(sk_flag_bytes(device_cus()) / sizeof(unsigned));  // zeroed
  unsigned* dabort = d.alloc<unsigned>(1);
  TRY_ALLOC(da);
  TRY_ALLOC(db);
  TRY_ALLOC(dp);
  TRY_ALLOC(dflags);
  TRY_ALLOC(dabort);
  if (mode == kGemmSwiGLU) {
    TRY_ALLOC(db3);
    TRY_ALLOC(dh);
  } else {
    TRY_ALLOC(dc);
  }
  GemmArgs g;
  memset(&g, 0, sizeof(g));
  g.A = da;
  g.lda = K;
  g.B = db;
  g.B3 = db3;
  g.ldb = K;
  g.C = dc;
  g.ldc = N;
  g.H = dh;
  g.ldh = N;
  g.M = M;
  g.N = N;
  g.K = K;
  g.act = act;
  g.P = dp;
  g.p_floats = pf;
  g.sk_flags = dflags;
  g.abort_flag = dabort;
  int rc = mode == kGemmStore ? launch_gemm<kGemmStore>(nullptr, g, nullptr)
           : mode == kGemmResid ? launch_gemm<kGemmResid>(nullptr, g, nullptr)
                                : launch_gemm<kGemmSwiGLU>(nullptr, g, nullptr);
  if (rc) return rc;
  HIP_TRY(nullptr, hipDeviceSynchronize());
  unsigned aborted = 0;
  HIP_TRY(nullptr, hipMemcpy(&aborted, dabort, sizeof(aborted), hipMemcpyDeviceToHost));
  if (aborted) return fail(nullptr, YHIP_EDEVICE, "gemm: a split-last-round wait timed out");
  if (mode == kGemmSwiGLU) HIP_TRY(nullptr, hipMemcpy(h, dh, (size_t)M * N * 2, hipMemcpyDeviceToHost));
  else HIP_TRY(nullptr, hipMemcpy(c, dc, (size_t)M * N * 4, hipMemcpyDeviceToHost));
  return YHIP_OK;
}

extern "C" int yhip_gemm_variant(int M, int N, int K, int mode, int* stages, int* bk, int* bm) {
  if (!stages || !bk || !bm || M <= 0 || N <= 0 || K <= 0 || mode < 0 || mode > 2)
    return fail(nullptr, YHIP_EINVAL, "bad argument");
  int s = 0, k = 0, m = 0;
  gemm_resolve(mode, M, N, K, device_cus(), s, k, m);
  *stages = s;
  *bk = k;
  *bm = m;
  return YHIP_OK;
}

extern "C" int yhip_test_argmax(const float* logits, int n, int* out) {
  if (!logits || !out || n <= 0) return fail(nullptr, YHIP_EINVAL, "bad argument");
  DevBufs b;
  float* dl = b.alloc<float>(n, logits);
  int* dout = b.alloc<int>(1);
  TRY_ALLOC(dl);
  TRY_ALLOC(dout);
  hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(kArgmaxThreads), 0, nullptr, (const float*)dl, n, dout);
  HIP_TRY(nullptr, hipGetLastError());
  HIP_TRY(nullptr, hipDeviceSynchronize());
  HIP_TRY(nullptr, hipMemcpy(out, dout, sizeof(int), hipMemcpyDeviceToHost));
  return YHIP_OK;
}

// ============================================================================================
// Microbenchmark of one fused kernel with rotating weight copies.
// ============================================================================================
namespace {
__global__ void fill_weights_kernel(uint16_t* w, size_t n, uint32_t seed) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    uint32_t h = (uint32_t)i * 2654435761u ^ seed;
    h ^= h >> 15;
    h *= 2246822519u;
    h ^= h >> 13;
    // uniform in [-0.03, 0.03): small, finite fp16
    const float u = ((h >> 8) * (1.0f / 16777216.0f) - 0.5f) * 0.06f;
    w[i] = __builtin_bit_cast(uint16_t, (f16)u);
  }
}
// Plain streaming copy: the counter calibration reference (reads and writes exactly n16*16 bytes).
__global__ void copy_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst, size_t n16) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (size_t)gridDim.x * blockDim.x)
    dst[i] = src[i];
}
// Memory-only read of `groups` 16 KB groups at base with the decode matvecs' access pattern: a
// wave takes groups round-robin and reads each as 16 buffer loads of 1 KB (16 bytes per lane,
// streaming); the loaded words are folded into one value that is stored only if it matches an
// impossible pattern, so the loads cannot be dropped.
__global__ void __launch_bounds__(256) stream_read_kernel(const unsigned char* base, long groups, unsigned* sink) {
  const int lane = threadIdx.x & 63;
  const long gw = __builtin_amdgcn_readfirstlane((int)(blockIdx.x * 4 + (threadIdx.x >> 6)));
  const long nw = (long)gridDim.x * 4;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (long g = gw; g < groups; g += nw) {
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char*>(base + g * 16384), 0, 16384, kBufferConfig);
    u32x4 v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u)
      v[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, lane * 16, u * 1024, kCpolNt));
#pragma unroll
    for (int u = 0; u < 16; ++u) acc ^= v[u];
  }
  if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == 0x9E3779B9u && acc[0] == 0x7F4A7C15u) sink[0] = 1u;
}
__global__ void fill_float_kernel(float* p, size_t n, float base, float step) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    p[i] = base + step * (float)((i * 7919u) % 1000u);
}
}  // namespace

extern "C" int yhip_bench_kernel(int kind, int rows, int cols, int copies, int warmup, int reps, int blocks_per_cu,
                                 float* us_per_launch) {
  if (!us_per_launch || rows <= 0 || cols <= 0 || copies <= 0 || reps <= 0 || warmup < 0 || kind < 0 || kind > 5)
    return fail(nullptr, YHIP_EINVAL, "bad argument");
  // W2 rows one per group when they are long (14336: two pieces of 14 KB), in pairs otherwise
  const int R = (kind == 3 && cols >= 8192) ? 1 : 2;
  if (kind != 2 && kind != 5 && R == 2 && rows % 2) return fail(nullptr, YHIP_EINVAL, "rows must be even");
  const int nmat = (kind == 2) ? 2 : 1;
  const size_t per = (size_t)rows * cols * nmat;
  DevBufs b;
  uint16_t* w = b.alloc<uint16_t>(per * copies);
  float* x = b.alloc<float>(cols);
  float* g = b.alloc<float>(cols);
  float* out = b.alloc<float>(std::max(rows, 1 << 16));
  // attention-shaped KV for the QKV epilogue: kv heads of 128 at msl 4096, 8 of them from 2048 rows
  // on (the Mistral-7B shape at 6144 rows), else one (768 rows: one kv head and its 4 query heads,
  // a GPU's share of an 8-way tensor-parallel split)
  const int hd = 128, nkv = rows >= 2048 ? 8 : 1, msl = 4096;
  uint16_t* kc = b.alloc<uint16_t>((size_t)nkv * hd * msl);
  uint16_t* vc = b.alloc<uint16_t>((size_t)nkv * hd * msl);
  StepParams hp{0, 7, {0, 0}};
  StepParams* dp = b.alloc<StepParams>(1, &hp);
  const std::vector<float> freqs = make_inv_freq(hd, hd, 1e6f);
  float* dfreq = b.alloc<float>(freqs.size(), freqs.data());
  float* dcs = b.alloc<float>(hd);
  TRY_ALLOC(dfreq);
  TRY_ALLOC(dcs);
  TRY_ALLOC(w);
  TRY_ALLOC(x);
  TRY_ALLOC(g);
  TRY_ALLOC(out);
  TRY_ALLOC(kc);
  TRY_ALLOC(vc);
  TRY_ALLOC(dp);
  hipLaunchKernelGGL(fill_weights_kernel, dim3(4096), dim3(256), 0, nullptr, w, per * copies, 12345u);
  hipLaunchKernelGGL(fill_float_kernel, dim3(64), dim3(256), 0, nullptr, x, (size_t)cols, -1.0f, 0.002f);
  hipLaunchKernelGGL(fill_float_kernel, dim3(64), dim3(256), 0, nullptr, g, (size_t)cols, 0.9f, 0.0002f);
  hipLaunchKernelGGL(rope_table_kernel, dim3(1), dim3(kBlock), 0, nullptr, (const float*)dfreq, dcs, hd / 2,
                     (const StepParams*)dp);
  uint16_t* copy_dst = nullptr;
  if (kind == 5) {
    if (per % 8) return fail(nullptr, YHIP_EINVAL, "copy size must be a multiple of 16 bytes");
    copy_dst = b.alloc<uint16_t>(per);
    TRY_ALLOC(copy_dst);
  }
  HIP_TRY(nullptr, hipDeviceSynchronize());
  hipStream_t s;
  HIP_TRY(nullptr, hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  const int cus = device_cus();
  auto launch = [&](int it) -> int {
    const uint16_t* base = w + per * (it % copies);
    if (kind == 5) {
      hipLaunchKernelGGL(copy_kernel, dim3(cus * 8), dim3(256), 0, s, (const u32x4*)base, (u32x4*)copy_dst,
                         per * 2 / 16);
      return hipGetLastError() == hipSuccess ? YHIP_OK : fail(nullptr, YHIP_EDEVICE, "copy launch failed");
    }
    MatvecArgs a = mv_base();
    a.K = cols;
    a.x = x;
    a.out = out;
    int ek = kEpiStore;
    switch (kind) {
      case 0:
        a.w0 = base; a.row_step = 2L * cols; a.r_step = cols; a.groups = rows / 2; a.gain = g; a.eps = 1e-5f;
        a.q_dim = rows - 2 * nkv * hd; a.kv_dim = nkv * hd; a.head_dim = hd; a.msl = msl;
        a.kcache = kc; a.vcache = vc; a.params = dp; a.rope_cs = dcs; ek = kEpiQkvRope;
        if (a.q_dim <= 0 || a.q_dim % hd) return fail(nullptr, YHIP_EINVAL, "QKV bench: rows - 2 kv heads x 128 must be whole query heads");
        break;
      case 1:
        a.w0 = base; a.row_step = 2L * cols; a.r_step = cols; a.groups = rows / 2; ek = kEpiResidual;
        break;
      case 2:
        a.w0 = base; a.w1 = base + (size_t)rows * cols; a.row_step = cols; a.groups = rows; a.gain = g;
        a.eps = 1e-5f; a.act = 1; ek = kEpiSwiGLU;
        break;
      case 3:
        a.w0 = base; a.row_step = (long)R * cols; a.r_step = cols; a.groups = rows / R; ek = kEpiResidual;
        break;
      default:
        a.w0 = base; a.row_step = 2L * cols; a.r_step = cols; a.groups = rows / 2; a.gain = g; a.eps = 1e-5f;
        break;
    }
    return launch_matvec(nullptr, a, ek, R, cus, s, blocks_per_cu);
  };
  int rc = 0;
  for (int i = 0; i < warmup && !rc; ++i) rc = launch(i);
  hipEvent_t e0, e1;
  hipEventCreate(&e0);
  hipEventCreate(&e1);
  hipEventRecord(e0, s);
  for (int i = 0; i < reps && !rc; ++i) rc = launch(warmup + i);
  hipEventRecord(e1, s);
  hipError_t e = hipEventSynchronize(e1);
  float ms = 0.f;
  hipEventElapsedTime(&ms, e0, e1);
  hipEventDestroy(e0);
  hipEventDestroy(e1);
  hipStreamDestroy(s);
  if (rc) return rc;
  if (e != hipSuccess) return fail(nullptr, YHIP_EDEVICE, hipGetErrorString(e));
  *us_per_launch = ms * 1000.0f / reps;
  return YHIP_OK;
}

extern "C" int yhip_bench_attention(int head_dim, int n_heads, int n_kv_heads, int max_seq_len, int kv_len, int nsplit,
                                    int min_slice, int copies, int warmup, int reps, float* us_per_launch) {
  if (!us_per_launch || kv_len <= 0 || kv_len > max_seq_len || copies <= 0 || reps <= 0 || warmup < 0 || nsplit < 0 ||
      nsplit > 64 || min_slice < 0 || min_slice % 64)
    return fail(nullptr, YHIP_EINVAL, "bad argument");
  if (int rc = check_attn_shape(nullptr, head_dim, n_heads, n_kv_heads)) return rc;
  if (nsplit == 0) hook_slice_plan(head_dim, max_seq_len, n_kv_heads, nsplit, min_slice);  // the decode step's plan
  const size_t kv = (size_t)n_kv_heads * head_dim * max_seq_len;
  DevBufs b;
  uint16_t* caches = b.alloc<uint16_t>(kv * 2 * copies);
  float* dq = b.alloc<float>((size_t)n_heads * head_dim);
  float* dpart = b.alloc<float>((size_t)n_heads * 64 * (head_dim + 2));
  unsigned* dt = b.alloc<unsigned>(64);
  float* dout = b.alloc<float>((size_t)n_heads * head_dim);
  StepParams hp{0, kv_len - 1, {0, 0}};
  StepParams* dp = b.alloc<StepParams>(1, &hp);
  const std::vector<float> freqs = make_inv_freq(head_dim, head_dim, 1e6f);
  float* dfreq = b.alloc<float>(freqs.size(), freqs.data());
  TRY_ALLOC(caches);
  TRY_ALLOC(dq);
  TRY_ALLOC(dpart);
  TRY_ALLOC(dt);
  TRY_ALLOC(dout);
  TRY_ALLOC(dp);
  TRY_ALLOC(dfreq);
  hipLaunchKernelGGL(fill_weights_kernel, dim3(4096), dim3(256), 0, nullptr, caches, kv * 2 * copies, 777u);
  hipLaunchKernelGGL(fill_float_kernel, dim3(64), dim3(256), 0, nullptr, dq, (size_t)n_heads * head_dim, -1.0f, 0.002f);
  HIP_TRY(nullptr, hipDeviceSynchronize());
  hipStream_t s;
  HIP_TRY(nullptr, hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  int rc = 0;
  auto launch = [&](int it) {
    AttnArgs t;
    t.q = dq;
    t.kcache = caches + kv * 2 * (it % copies);
    t.vcache = t.kcache + kv;
    t.partial = dpart;
    t.tickets = dt;
    t.out = dout;
    t.head_dim = head_dim;
    t.n_heads = n_heads;
    t.n_kv_heads = n_kv_heads;
    t.msl = max_seq_len;
    t.nsplit = nsplit;
    t.min_slice = min_slice;
    t.inv_freq = dfreq;
    t.params = dp;
    return launch_attention(nullptr, t, s);
  };
  for (int i = 0; i < warmup && !rc; ++i) rc = launch(i);
  hipEvent_t e0, e1;
  hipEventCreate(&e0);
  hipEventCreate(&e1);
  hipEventRecord(e0, s);
  for (int i = 0; i < reps && !rc; ++i) rc = launch(warmup + i);
  hipEventRecord(e1, s);
  hipError_t e = hipEventSynchronize(e1);
  float ms = 0.f;
  hipEventElapsedTime(&ms, e0, e1);
  hipEventDestroy(e0);
  hipEventDestroy(e1);
  hipStreamDestroy(s);
  if (rc) return rc;
  if (e != hipSuccess) return fail(nullptr, YHIP_EDEVICE, hipGetErrorString(e));
  *us_per_launch = ms * 1000.0f / reps;
  return YHIP_OK;
}

// The memory-only ceiling of one decode step (no reference counterpart; a measurement hook): the
// step's weight bytes read by streaming launches in the order and sizes of the decode launches
// (per layer: [Wq;Wk;Wv], Wo, W1 and W3, W2; then the lm_head), every launch over fresh memory,
// with the matvecs' access pattern and 12 workgroups per CU; and the same bytes as one launch.
// Writes milliseconds per token for both (HIP events, mean over reps after one warm-up token).
extern "C" int yhip_bench_stream(const yhip_config* cfg, int reps, float* ms_launches, float* ms_one_launch) {
  if (!cfg || !ms_launches || !ms_one_launch || reps <= 0 || cfg->n_layers < 1 || cfg->dim <= 0)
    return fail(nullptr, YHIP_EINVAL, "bad argument");
  const long dim = cfg->dim, hid = cfg->hidden_dim, qd = (long)cfg->n_heads * cfg->head_dim,
             kvd = (long)cfg->n_kv_heads * cfg->head_dim;
  const long layer_bytes[4] = {(qd + 2 * kvd) * dim * 2, dim * qd * 2, 2 * hid * dim * 2, dim * hid * 2};
  const long lm_bytes = (long)cfg->vocab_size * dim * 2;
  long total = lm_bytes;
  for (long b : layer_bytes) total += b * cfg->n_layers;
  DevBufs bufs;
  unsigned char* w = bufs.alloc<unsigned char>((size_t)total);
  unsigned* sink = bufs.alloc<unsigned>(1);
  TRY_ALLOC(w);
  TRY_ALLOC(sink);
  hipLaunchKernelGGL(fill_weights_kernel, dim3(4096), dim3(256), 0, nullptr, (uint16_t*)w, (size_t)total / 2, 777u);
  HIP_TRY(nullptr, hipDeviceSynchronize());
  hipStream_t s;
  HIP_TRY(nullptr, hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  const long cap = 12L * device_cus();
  auto go = [&](long off, long bytes) {
    const long groups = bytes / 16384;
    hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)std::max(1L, std::min((groups + 3) / 4, cap))), dim3(256), 0,
                       s, (const unsigned char*)w + off, groups, sink);
  };
  auto token = [&] {
    long off = 0;
    for (int l = 0; l < cfg->n_layers; ++l)
      for (long b : layer_bytes) {
        go(off, b);
        off += b;
      }
    go(off, lm_bytes);
  };
  hipEvent_t e0 = nullptr, e1 = nullptr;
  int rc = YHIP_OK;
  float ms = 0.f;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) rc = fail(nullptr, YHIP_EDEVICE, "event create failed");
  if (!rc) {
    token();
    hipEventRecord(e0, s);
    for (int r = 0; r < reps; ++r) token();
    hipEventRecord(e1, s);
    if (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess)
      rc = fail(nullptr, YHIP_EDEVICE, "stream bench failed");
    *ms_launches = ms / reps;
  }
  if (!rc) {
    go(0, total);
    hipEventRecord(e0, s);
    for (int r = 0; r < reps; ++r) go(0, total);
    hipEventRecord(e1, s);
    if (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess)
      rc = fail(nullptr, YHIP_EDEVICE, "stream bench failed");
    *ms_one_launch = ms / reps;
  }
  if (e0) hipEventDestroy(e0);
  if (e1) hipEventDestroy(e1);
  hipStreamDestroy(s);
  return rc;
}

extern "C" int yhip_bench_gemm(int M, int N, int K, int mode, int warmup, int reps, float* us_per_launch) {
  if (!us_per_launch || M <= 0 || N <= 0 || K <= 0 || mode < 0 || mode > 2 || reps <= 0 || warmup < 0)
    return fail(nullptr, YHIP_EINVAL, "bad argument");
  DevBufs d;
  uint16_t* da = d.alloc<uint16_t>((size_t)M * K);
  uint16_t* db = d.alloc<uint16_t>((size_t)N * K);
  uint16_t* db3 = d.alloc<uint16_t>((size_t)N * K);
  float* dc = d.alloc<float>((size_t)M * N);
  uint16_t* dh = d.alloc<uint16_t>((size_t)M * N);
  const long pf = splitk_ws_floats(device_cus());
  float* dp = d.alloc<float>((size_t)pf);
  unsigned* dflags = d.alloc<unsigned>(sk_flag_bytes(device_cus()) / sizeof(unsigned));  // zeroed
  unsigned* dabort = d.alloc<unsigned>(1);
  TRY_ALLOC(da);
  TRY_ALLOC(db);
  TRY_ALLOC(db3);
  TRY_ALLOC(dc);
  TRY_ALLOC(dh);
  TRY_ALLOC(dp);
  TRY_ALLOC(dflags);
  TRY_ALLOC(dabort);
  hipLaunchKernelGGL(fill_weights_kernel, dim3(1024), dim3(256), 0, nullptr, da, (size_t)M * K, 11u);
  hipLaunchKernelGGL(fill_weights_kernel, dim3(1024), dim3(256), 0, nullptr, db, (size_t)N * K, 12u);
  hipLaunchKernelGGL(fill_weights_kernel, dim3(1024), dim3(256), 0, nullptr, db3, (size_t)N * K, 13u);
  HIP_TRY(nullptr, hipMemset(dc, 0, (size_t)M * N * 4));
  HIP_TRY(nullptr, hipDeviceSynchronize());
  GemmArgs g;
  memset(&g, 0, sizeof(g));
  g.A = da;
  g.lda = K;
  g.B = db;
  g.B3 = db3;
  g.ldb = K;
  g.C = dc;
  g.ldc = N;
  g.H = dh;
  g.ldh = N;
  g.M = M;
  g.N = N;
  g.K = K;
  g.act = 1;
  g.P = dp;
  g.p_floats = pf;
  g.sk_flags = dflags;
  g.abort_flag = dabort;
  hipStream_t s;
  HIP_TRY(nullptr, hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  auto launch = [&] {
    return mode == kGemmStore ? launch_gemm<kGemmStore>(nullptr, g, s)
           : mode == kGemmResid ? launch_gemm<kGemmResid>(nullptr, g, s)
                                : launch_gemm<kGemmSwiGLU>(nullptr, g, s);
  };
  int rc = 0;
  for (int i = 0; i < warmup && !rc; ++i) rc = launch();
  hipEvent_t e0, e1;
  hipEventCreate(&e0);
  hipEventCreate(&e1);
  hipEventRecord(e0, s);
  for (int i = 0; i < reps && !rc; ++i) rc = launch();
  hipEventRecord(e1, s);
  hipError_t e = hipEventSynchronize(e1);
  float ms = 0.f;
  hipEventElapsedTime(&ms, e0, e1);
  hipEventDestroy(e0);
  hipEventDestroy(e1);
  hipStreamDestroy(s);
  if (rc) return rc;
  if (e != hipSuccess) return fail(nullptr, YHIP_EDEVICE, std::string("gemm bench: ") + hipGetErrorString(e));
  unsigned aborted = 0;
  HIP_TRY(nullptr, hipMemcpy(&aborted, dabort, sizeof(aborted), hipMemcpyDeviceToHost));
  if (aborted) return fail(nullptr, YHIP_EDEVICE, "gemm bench: a split-last-round wait timed out");
  *us_per_launch = 1000.f * ms / reps;
  return YHIP_OK;
}
