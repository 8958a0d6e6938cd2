// Host-side model API with a HIP device behind it.
//
// Mirrors the reference C++ surface (src/model.h:56-302): Config parsed from .yalm metadata,
// an InferenceState per decode stream, and Model::forward(s, token, pos, mode). Moving a model to
// the GPU (`Model::hip()` + `InferenceState::hip()`, the counterparts of the reference's
// `cuda()` calls) creates one yhip_ctx (include/yalm_hip.h) that holds the weights, KV caches and
// activations in HBM; forward() is then a single C-ABI call.
//
// Unlike the reference, the Model keeps its host tensor pointers after the move (the mmapped file
// stays the source of truth), and errors are reported as exceptions rather than assert/abort.
#pragma once
#include <cstddef>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "codec.h"
#include "yalm_hip.h"

namespace yalm {

constexpr int KV_SINKS = 2;  // reference src/model.h:12

// calm-style 16-element K tiling (reference src/model.h:15-17)
inline int k_cache_idx(int hi, int t, int max_seq_len) { return (hi / 16) * (16 * max_seq_len) + t * 16 + (hi % 16); }

enum class ActivationType { GELU, SILU };
enum class LayerNormType { RMSNorm };
enum class Device { CPU, HIP };
enum class InferenceMode { HYDRATE_KV_CACHE, OUTPUT_LOGITS };

struct Error : std::runtime_error {
  using std::runtime_error::runtime_error;
};

struct Config {
  int dim = 0, hidden_dim = 0, head_dim = 0, n_layers = 0, n_heads = 0, n_kv_heads = 0, vocab_size = 0;
  int max_seq_len = 0;
  float rope_theta = 10000.f;
  int rotary_dim = 0;
  float norm_eps = 1e-5f;
  ActivationType act = ActivationType::GELU;
  LayerNormType norm_type = LayerNormType::RMSNorm;
  float qkv_clip = 3.402823466e38f;
  int n_experts = 0, n_experts_active = 0;
  DType weight_dtype = DType::F16;

  // Metadata keys and defaults of the reference (src/model.cpp:18-71): max_seq_len is capped at
  // 4096 unless `context` (the -T flag) overrides it.
  void from_yalm(const YALMData& yalm, int context = 0);
  // Bytes one decode step at `pos` reads, counted like the reference (src/model.cpp:73-98).
  size_t active_bytes(size_t pos) const;
  yhip_config to_hip() const;
};

struct InferenceState {
  explicit InferenceState(std::shared_ptr<Config> config);
  ~InferenceState();
  InferenceState(const InferenceState&) = delete;
  InferenceState& operator=(const InferenceState&) = delete;

  float* logits() const { return _logits; }  // (vocab_size,) host
  void hip();
  Device device() const { return _device; }
  InferenceMode mode() const { return _mode; }
  void set_mode(InferenceMode m) { _mode = m; }

 private:
  friend struct Model;
  std::shared_ptr<Config> _config;
  Device _device = Device::CPU;
  InferenceMode _mode = InferenceMode::OUTPUT_LOGITS;
  std::vector<float> _own_logits;
  float* _logits = nullptr;
};

struct Block {
  // Host views of one transformer layer's tensors (shape- and dtype-checked like the reference,
  // src/model.cpp:130-205).
  const float* rms_att_weight = nullptr;
  const float* rms_ffn_weight = nullptr;
  const f16_t *wq = nullptr, *wk = nullptr, *wv = nullptr, *wo = nullptr, *w1 = nullptr, *w2 = nullptr,
              *w3 = nullptr;
};

struct Model {
  std::shared_ptr<Config> config;
  std::vector<Block> blocks;
  const f16_t* token_embedding_table = nullptr;  // (vocab_size, dim)
  const float* rms_final_weight = nullptr;       // (dim,)
  const f16_t* wcls = nullptr;                   // (vocab_size, dim); the embedding when tied

  Model(const YALMData& yalm, int context = 0);
  ~Model();
  Model(const Model&) = delete;
  Model& operator=(const Model&) = delete;

  // Uploads weights to HIP device `device_ordinal` (reference Model::cuda, src/model.cpp:437-451).
  void hip(int device_ordinal = 0);
  void forward(InferenceState& s, int token, int pos, InferenceMode mode = InferenceMode::OUTPUT_LOGITS);
  // Greedy step on the device: returns argmax of the next-token logits (reference tie rule).
  int forward_argmax(InferenceState& s, int token, int pos);
  // Ingests tokens[0..n) at positions start_pos.. in one batched pass (MFMA GEMMs and causal
  // attention) and leaves the last token's logits in s.logits(). The reference has no batched form:
  // it feeds a prompt one token at a time in HYDRATE mode (src/main.cpp:169-177), which this equals
  // within fp16-activation tolerance; positions past the context fall back to that loop.
  void prefill(InferenceState& s, const int* tokens, int n, int start_pos = 0);
  Device device() const { return _device; }
  yhip_ctx* hip_context() const { return _ctx; }

 private:
  Device _device = Device::CPU;
  yhip_ctx* _ctx = nullptr;
  void check(int rc, const char* what) const;
};

struct Sampler {
  int vocab_size;
  Sampler(std::shared_ptr<Config> config, uint64_t seed);
  float sample_prob(int index, const InferenceState& s);  // reference src/sampler.cpp:11-25
  int sample_argmax(const InferenceState& s);             // first index of the strict max (:27-38)
  int sample(const InferenceState& s, float temperature = 1.0f);  // (:40-65)
};

struct Tokenizer {
  std::vector<std::string> vocab;
  int bos_id = -1, eos_id = -1, eot_id = -1;
  int byte_fallback_start = -1;

  explicit Tokenizer(const YALMData& data);
  ~Tokenizer();
  std::vector<int> encode(const std::string& text, bool encode_bos) const;
  std::string decode_one(int prev_token, int token) const;
  std::string encoding_to_debug_string(const std::vector<int>& encoding) const;

 private:
  struct Trie;
  Trie* _root = nullptr;
};

}  // namespace yalm
