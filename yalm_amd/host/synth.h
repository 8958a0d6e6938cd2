// Synthetic Mistral/Llama-architecture checkpoints: seeded random-init fp16 weights with the
// tensor names, shapes and metadata keys that the reference converter emits (convert.py:58-81,
// 174-207), built in memory or written as a .yalm file.
//
// Randomness is counter based, so any element can be generated independently (in parallel, in any
// order) and the same seed always gives the same bytes:
//   stream  = FNV-1a 64 of the tensor name
//   pair p  = splitmix64-mix(seed ^ mix(stream) + p * golden) -> two 24-bit uniforms -> Box-Muller
// giving elements 2p and 2p+1 of N(0, std), rounded to fp16 (RNE).
#pragma once
#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "codec.h"

namespace yalm {

struct SynthSpec {
  int dim, hidden_dim, head_dim, n_layers, n_heads, n_kv_heads, vocab_size, max_seq_len;
  float rope_theta = 1e6f;
  float norm_eps = 1e-5f;
  float std = 0.02f;
  uint64_t seed = 0x59414C4Dull;
  bool tied_embeddings = false;
};

uint64_t fnv1a64(const std::string& s);
uint64_t mix64(uint64_t x);
// N(0, std) fp16 for elements [0, n) of the stream named `name`.
void fill_normal_f16(f16_t* out, size_t n, uint64_t seed, const std::string& name, float std);
// Uniform integers in [0, hi) (token ids): element i of stream `seed`.
void fill_uniform_ids(int* out, size_t n, uint64_t seed, int hi);

// In-memory file image (header + payload) of a synthetic model. The block is malloc'd and owned by
// `out` afterwards. Tensor order: embed, per layer (norms, wq, wk, wv, wo, w1, w2, w3), final norm,
// output, tokenizer.tokens.
int synth_build(const SynthSpec& spec, YALMData& out, std::string* err = nullptr);
std::map<std::string, std::string> synth_metadata(const SynthSpec& spec);

}  // namespace yalm
