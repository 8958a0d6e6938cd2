// Single-launch decode step for gfx950: one launch computes a whole token as a dataflow of
// workgroups.
//
// The grid holds, per layer, the workgroups of five phases in order
//   QKV   rmsnorm(x) -> [Wq;Wk;Wv] -> clip, RoPE -> q, fp16 K/V into the cache and a side buffer
//   ATT   split-KV GQA attention, one workgroup per (kv head, active slice), ticket merge -> att
//   O     x += Wo att
//   W13   rmsnorm(x) -> act(W1 x) * (W3 x) -> hb
//   W2    x += W2 hb
// and then the lm_head workgroups (final rmsnorm, logits, fused argmax). Arithmetic follows
// reference src/infer.cpp:256-527; what one step launches, src/infer.cu:1274-1378 and
// src/coop.cu:179-322.
//
// Every workgroup takes a ticket when it starts; the ticket, not the hardware workgroup id, names
// its work, so tickets are handed out in start order. A workgroup first issues the weight loads of
// its first row group (weights never depend on other workgroups), then waits until every workgroup
// of the previous phase has counted itself done, then stages its input vector and finishes its
// rows. It only ever waits for workgroups holding smaller tickets, which have all started, so the
// dataflow always drains, whatever the residency; the hardware dispatcher balances the work, and
// the next phase's weight loads overlap the current phase's tail instead of waiting for a kernel
// boundary.
//
// Coherence across workgroups (each XCD has its own L2): activations handed from one phase to the
// next (x, q, att, hb, logits, the current position's K/V) are written and read with agent-scope
// relaxed atomics, and every thread waits for its stores to complete (`publish`) before its
// workgroup counts itself done. KV-cache entries of earlier positions were written by earlier
// launches and are read with plain loads; the current position comes from the coherent side buffer.
#pragma once
#include "kernels.h"

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

enum FlowPhase : int { kPhQkv = 0, kPhAtt = 1, kPhO = 2, kPhW13 = 3, kPhW2 = 4, kPhasesPerLayer = 5, kPhLm = 5 };

// Sync words (unsigned), each on its own 256-byte line: the start tickets of even and odd
// launches, the abort flag (a wait timed out), the argmax ticket, then per launch parity one
// completion counter per phase instance. A launch zeroes the other parity's words, which the
// previous launch used and nothing else touches.
constexpr int kLine = 64;
constexpr int kSyncTicket0 = 0, kSyncTicket1 = kLine, kSyncAbort = 2 * kLine, kSyncArgmax = 3 * kLine,
              kSyncCounters = 4 * kLine;
__host__ __device__ constexpr int flow_counters(int n_layers) { return n_layers * kPhasesPerLayer + 1; }
__host__ __device__ constexpr int flow_sync_words(int n_layers) { return kSyncCounters + 2 * flow_counters(n_layers) * kLine; }

struct FlowArgs {
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
  unsigned* tickets;  // attention merge tickets [n_kv_heads]
  uint32_t* kvcur;    // [K pairs | V pairs] of the current position, fp16x2
  unsigned* sync;     // flow_sync_words(n_layers)
  float* best_v;      // [nb_lm]
  int* best_i;        // [nb_lm]
  int* result;        // [0] argmax token
  int n_layers, dim, hidden, q_dim, kv_dim, head_dim, n_heads, n_kv_heads, vocab, msl;
  int token, pos, mode, nsplit, min_slice, act;
  float eps, qkv_clip;
  unsigned launch;
  int nb[6];  // workgroups per phase: QKV, ATT, O, W13, W2, lm_head
};

// Matvec phase with the row-length specialisations the model shapes use.
template <int R, EpiKind EPI, class Wait>
__device__ __forceinline__ RowMax flow_matvec(const MatvecArgs& m, int blk, int nblk, float* lds, Wait wait) {
  if constexpr (R == 2) {
    if (m.K == 4096) return matvec_body<8, 2, EPI, true>(m, blk, nblk, lds, wait);
    return matvec_body<0, 2, EPI, true>(m, blk, nblk, lds, wait);
  } else {
    if (m.K == 14336) return matvec_body<28, 1, EPI, true>(m, blk, nblk, lds, wait);
    return matvec_body<0, 1, EPI, true>(m, blk, nblk, lds, wait);
  }
}

// HD: head_dim; G: query heads per kv head.
template <int HD, int G>
__global__ void __launch_bounds__(kBlock) decode_flow_kernel(FlowArgs a) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  __shared__ int s_bid;
  const int tid = threadIdx.x;
  const unsigned par = a.launch & 1u;
  const int ncnt = flow_counters(a.n_layers);
  unsigned* counters = a.sync + kSyncCounters + par * ncnt * kLine;
  unsigned* abort_flag = a.sync + kSyncAbort;
  if (tid == 0)
    s_bid = (int)__hip_atomic_fetch_add(a.sync + (par ? kSyncTicket1 : kSyncTicket0), 1u, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  const int bid = s_bid;
  if (bid == 0) {  // reset the other parity (the launch that used it has ended)
    unsigned* other = a.sync + kSyncCounters + (par ^ 1u) * ncnt * kLine;
    for (int c = tid; c < ncnt; c += kBlock)
      __hip_atomic_store(other + c * kLine, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (tid == 0)
      __hip_atomic_store(a.sync + (par ? kSyncTicket0 : kSyncTicket1), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // ticket -> (layer, phase, workgroup within the phase)
  const int per_layer = a.nb[0] + a.nb[1] + a.nb[2] + a.nb[3] + a.nb[4];
  int layer, phase, local;
  if (bid < a.n_layers * per_layer) {
    layer = bid / per_layer;
    local = bid - layer * per_layer;
    phase = 0;
    while (local >= a.nb[phase]) local -= a.nb[phase++];
  } else {
    layer = a.n_layers;
    phase = kPhLm;
    local = bid - a.n_layers * per_layer;
  }
  // this phase's counter, in [0, flow_counters): layer * 5 + phase, the lm_head's is n_layers * 5;
  // the previous one (cidx - 1) belongs to the phase before (for QKV and the lm_head, a W2)
  const int cidx = phase == kPhLm ? a.n_layers * kPhasesPerLayer : layer * kPhasesPerLayer + phase;
  const int prev_nb = (phase == kPhQkv || phase == kPhLm) ? a.nb[kPhW2] : a.nb[phase - 1];
  auto wait = [&] {
    if (cidx > 0) wait_count(counters + (cidx - 1) * kLine, (unsigned)prev_nb, abort_flag);
  };

  const char* lb = a.layers.wbase + (long)(layer < a.n_layers ? layer : 0) * a.layers.stride;
  uint16_t* kc = a.layers.kv + 2L * layer * a.layers.kv_elems;
  uint16_t* vc = kc + a.layers.kv_elems;

  MatvecArgs m;
  memset(&m, 0, sizeof(m));
  m.qkv_clip = a.qkv_clip;
  m.pos = a.pos;
  m.eps = a.eps;

  switch (phase) {
    case kPhQkv: {  // reference src/infer.cpp:270-305
      m.w0 = reinterpret_cast<const uint16_t*>(lb + a.layers.o_qkv);
      m.row_step = 2L * a.dim;
      m.r_step = a.dim;
      m.groups = (a.q_dim + 2 * a.kv_dim) / 2;
      m.K = a.dim;
      m.x = a.x;
      if (layer == 0) {  // the residual stream starts as the embedding row (src/infer.cpp:460-481)
        m.emb = a.embed;
        m.emb_out = a.x;
        m.token = a.token;
      }
      m.gain = reinterpret_cast<const float*>(lb + a.layers.o_ra);
      m.out = a.q;
      m.q_dim = a.q_dim;
      m.kv_dim = a.kv_dim;
      m.head_dim = a.head_dim;
      m.msl = a.msl;
      m.kcache = kc;
      m.vcache = vc;
      m.kvcur = a.kvcur;
      m.inv_freq = a.inv_freq;
      flow_matvec<2, kEpiQkvRope>(m, local, a.nb[kPhQkv], lds, wait);
      break;
    }
    case kPhAtt: {  // reference src/infer.cpp:218-250, 307-336
      wait();
      AttnArgs at;
      at.q = a.q;
      at.kcache = kc;
      at.vcache = vc;
      at.partial = a.partial;
      at.tickets = a.tickets;
      at.out = a.att;
      at.head_dim = HD;
      at.n_heads = a.n_heads;
      at.n_kv_heads = a.n_kv_heads;
      at.msl = a.msl;
      at.nsplit = a.nsplit;
      at.min_slice = a.min_slice;
      at.inv_freq = a.inv_freq;
      at.params = nullptr;
      auto& sm = *reinterpret_cast<AttnSmem<HD, G, kBlock>*>(lds);
      attn_run<HD, G, kBlock, true, true>(at, local % a.n_kv_heads, local / a.n_kv_heads, a.pos, sm, a.kvcur, tid);
      break;
    }
    case kPhO: {  // reference src/infer.cpp:339-344
      m.w0 = reinterpret_cast<const uint16_t*>(lb + a.layers.o_wo);
      m.row_step = 2L * a.q_dim;
      m.r_step = a.q_dim;
      m.groups = a.dim / 2;
      m.K = a.q_dim;
      m.x = a.att;
      m.out = a.x;
      flow_matvec<2, kEpiResidual>(m, local, a.nb[kPhO], lds, wait);
      break;
    }
    case kPhW13: {  // reference src/infer.cpp:349-382
      m.w0 = reinterpret_cast<const uint16_t*>(lb + a.layers.o_w1);
      m.w1 = reinterpret_cast<const uint16_t*>(lb + a.layers.o_w3);
      m.row_step = a.dim;
      m.groups = a.hidden;
      m.K = a.dim;
      m.x = a.x;
      m.gain = reinterpret_cast<const float*>(lb + a.layers.o_rf);
      m.out = a.hb;
      m.act = a.act;
      flow_matvec<2, kEpiSwiGLU>(m, local, a.nb[kPhW13], lds, wait);
      break;
    }
    case kPhW2: {  // reference src/infer.cpp:384-390
      m.w0 = reinterpret_cast<const uint16_t*>(lb + a.layers.o_w2);
      m.row_step = a.hidden;
      m.r_step = a.hidden;
      m.groups = a.dim;
      m.K = a.hidden;
      m.x = a.hb;
      m.out = a.x;
      flow_matvec<1, kEpiResidual>(m, local, a.nb[kPhW2], lds, wait);
      break;
    }
    default: {  // final rmsnorm + lm_head (reference src/infer.cpp:501-527) + argmax (src/sampler.cpp:27-38)
      m.w0 = a.wcls;
      m.row_step = 2L * a.dim;
      m.r_step = a.dim;
      m.groups = a.vocab / 2;
      m.K = a.dim;
      m.x = a.x;
      if (a.n_layers == 0) {
        m.emb = a.embed;
        m.emb_out = a.x;
        m.token = a.token;
      }
      m.gain = a.rms_final;
      m.out = a.logits;
      m.track_max = 1;
      const RowMax mx = flow_matvec<2, kEpiStore>(m, local, a.nb[kPhLm], lds, wait);
      argmax_finish(mx, local, a.nb[kPhLm], a.best_v, a.best_i, a.sync + kSyncArgmax, a.result);
      return;  // nothing waits for the lm_head
    }
  }
  publish();  // this thread's outputs are complete
  __syncthreads();
  if (tid == 0) __hip_atomic_fetch_add(counters + cidx * kLine, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace yk
