#include "model.h"

#include <algorithm>
#include <cfloat>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <unordered_map>

namespace yalm {

namespace {

int meta_int(const YALMData& y, const char* key) {
  if (!y.has_meta(key)) throw Error(std::string("missing metadata key: ") + key);
  try {
    return std::stoi(y.meta(key));
  } catch (const std::exception&) {
    throw Error(std::string("bad integer metadata: ") + key);
  }
}

float meta_float(const YALMData& y, const char* key, const char* fallback) {
  std::string v = y.has_meta(key) ? y.meta(key) : std::string(fallback ? fallback : "");
  if (v.empty()) throw Error(std::string("missing metadata key: ") + key);
  try {
    return std::stof(v);
  } catch (const std::exception&) {
    throw Error(std::string("bad float metadata: ") + key);
  }
}

const Tensor& get_tensor(const YALMData& y, const std::string& name) {
  const Tensor* t = y.find(name);
  if (!t) throw Error("missing tensor: " + name);
  return *t;
}

// dtype/shape check of src/model.cpp:100-117
const void* check_tensor(const Tensor& t, DType dtype, std::array<int, 4> shape) {
  if (t.dtype != dtype || t.shape != shape) {
    char buf[512];
    snprintf(buf, sizeof(buf), "tensor mismatch for %s: expected %s [%d,%d,%d,%d], got %s [%d,%d,%d,%d]",
             t.name.c_str(), dtype_to_string(dtype).c_str(), shape[0], shape[1], shape[2], shape[3],
             dtype_to_string(t.dtype).c_str(), t.shape[0], t.shape[1], t.shape[2], t.shape[3]);
    throw Error(buf);
  }
  return t.data;
}

}  // namespace

// ---- Config (reference src/model.cpp:18-98) ---------------------------------------------------
void Config::from_yalm(const YALMData& y, int context) {
  dim = meta_int(y, "dim");
  hidden_dim = meta_int(y, "hidden_dim");
  head_dim = meta_int(y, "head_dim");
  n_layers = meta_int(y, "n_layers");
  n_heads = meta_int(y, "n_heads");
  n_kv_heads = meta_int(y, "n_kv_heads");
  vocab_size = meta_int(y, "vocab_size");
  n_experts = y.has_meta("n_experts") ? meta_int(y, "n_experts") : 0;
  n_experts_active = y.has_meta("n_experts_active") ? meta_int(y, "n_experts_active") : 0;
  max_seq_len = std::min(meta_int(y, "max_seq_len"), 4096);
  if (context) max_seq_len = context;
  rope_theta = meta_float(y, "rope_theta", nullptr);
  rotary_dim = meta_int(y, "rotary_dim");
  norm_eps = meta_float(y, "norm_eps", "1e-5");
  const std::string a = y.meta("act_type", "gelu");
  act = a == "silu" ? ActivationType::SILU : ActivationType::GELU;
  if (a != "silu" && a != "gelu") fprintf(stderr, "unsupported act_type, defaulting to gelu\n");
  norm_type = LayerNormType::RMSNorm;
  qkv_clip = y.has_meta("qkv_clip") ? meta_float(y, "qkv_clip", nullptr) : FLT_MAX;
  const std::string dt = y.meta("dtype");
  if (dt == "fp16")
    weight_dtype = DType::F16;
  else if (dt == "fp32")
    weight_dtype = DType::F32;
  else
    throw Error("unsupported dtype: " + dt);
}

size_t Config::active_bytes(size_t pos) const {
  const size_t ws = dtype_size(weight_dtype);
  size_t per_block = 2 * (size_t)dim * sizeof(float);
  per_block += (size_t)n_heads * head_dim * dim * ws;
  per_block += 2 * (size_t)n_kv_heads * head_dim * dim * ws;
  per_block += (size_t)n_heads * head_dim * dim * ws;
  if (n_experts > 0) {
    per_block += (size_t)n_experts * dim * ws;
    per_block += (size_t)n_experts_active * 3 * dim * hidden_dim * ws;
  } else {
    per_block += 3 * (size_t)dim * hidden_dim * ws;
  }
  const size_t kv_len = std::min((size_t)max_seq_len, pos + 1);
  per_block += 2 * kv_len * n_kv_heads * head_dim * sizeof(f16_t);
  size_t bytes = (size_t)dim * ws + n_layers * per_block + dim * sizeof(float);
  bytes += (size_t)vocab_size * dim * sizeof(float);  // the reference counts wcls at 4 bytes
  return bytes;
}

yhip_config Config::to_hip() const {
  yhip_config c;
  c.dim = dim;
  c.hidden_dim = hidden_dim;
  c.head_dim = head_dim;
  c.n_layers = n_layers;
  c.n_heads = n_heads;
  c.n_kv_heads = n_kv_heads;
  c.vocab_size = vocab_size;
  c.max_seq_len = max_seq_len;
  c.rotary_dim = rotary_dim;
  c.rope_theta = rope_theta;
  c.norm_eps = norm_eps;
  c.qkv_clip = qkv_clip;
  c.act = act == ActivationType::SILU ? YHIP_ACT_SILU : YHIP_ACT_GELU;
  return c;
}

// ---- InferenceState (reference src/model.cpp:291-361) ----------------------------------------
InferenceState::InferenceState(std::shared_ptr<Config> config) : _config(std::move(config)) {
  if (!_config) throw Error("null config");
  _own_logits.assign(_config->vocab_size, 0.f);
  _logits = _own_logits.data();
}

InferenceState::~InferenceState() = default;

void InferenceState::hip() { _device = Device::HIP; }

// ---- Model (reference src/model.cpp:392-494) ---------------------------------------------------
Model::Model(const YALMData& yalm, int context) {
  config = std::make_shared<Config>();
  config->from_yalm(yalm, context);
  const Config& c = *config;
  if (c.n_experts > 0) throw Error("mixture-of-experts models are not supported by the HIP decode path");
  if (c.weight_dtype != DType::F16) throw Error("the HIP decode path needs fp16 weights (dtype=fp16)");
  token_embedding_table =
      (const f16_t*)check_tensor(get_tensor(yalm, "model.embed.weight"), c.weight_dtype, {c.vocab_size, c.dim, 0, 0});
  const int qd = c.n_heads * c.head_dim, kvd = c.n_kv_heads * c.head_dim;
  for (int i = 0; i < c.n_layers; ++i) {
    const std::string p = "model.layers." + std::to_string(i) + ".";
    Block b;
    b.rms_att_weight = (const float*)check_tensor(get_tensor(yalm, p + "attn.norm.weight"), DType::F32, {c.dim, 0, 0, 0});
    b.rms_ffn_weight = (const float*)check_tensor(get_tensor(yalm, p + "mlp.norm.weight"), DType::F32, {c.dim, 0, 0, 0});
    b.wq = (const f16_t*)check_tensor(get_tensor(yalm, p + "attn.wq.weight"), c.weight_dtype, {qd, c.dim, 0, 0});
    b.wk = (const f16_t*)check_tensor(get_tensor(yalm, p + "attn.wk.weight"), c.weight_dtype, {kvd, c.dim, 0, 0});
    b.wv = (const f16_t*)check_tensor(get_tensor(yalm, p + "attn.wv.weight"), c.weight_dtype, {kvd, c.dim, 0, 0});
    b.wo = (const f16_t*)check_tensor(get_tensor(yalm, p + "attn.wo.weight"), c.weight_dtype, {c.dim, qd, 0, 0});
    b.w1 = (const f16_t*)check_tensor(get_tensor(yalm, p + "mlp.w1.weight"), c.weight_dtype, {c.hidden_dim, c.dim, 0, 0});
    b.w2 = (const f16_t*)check_tensor(get_tensor(yalm, p + "mlp.w2.weight"), c.weight_dtype, {c.dim, c.hidden_dim, 0, 0});
    b.w3 = (const f16_t*)check_tensor(get_tensor(yalm, p + "mlp.w3.weight"), c.weight_dtype, {c.hidden_dim, c.dim, 0, 0});
    blocks.push_back(b);
  }
  rms_final_weight = (const float*)check_tensor(get_tensor(yalm, "model.norm.weight"), DType::F32, {c.dim, 0, 0, 0});
  if (yalm.find("model.output.weight"))
    wcls = (const f16_t*)check_tensor(get_tensor(yalm, "model.output.weight"), c.weight_dtype, {c.vocab_size, c.dim, 0, 0});
  else
    wcls = token_embedding_table;
}

Model::~Model() {
  if (_ctx) yhip_destroy(_ctx);
}

void Model::check(int rc, const char* what) const {
  if (rc != YHIP_OK) throw Error(std::string(what) + ": " + yhip_last_error(_ctx));
}

void Model::hip(int device_ordinal) {
  if (_device == Device::HIP) return;
  yhip_config hc = config->to_hip();
  yhip_ctx* ctx = nullptr;
  if (yhip_create(&hc, device_ordinal, &ctx) != YHIP_OK) throw Error(std::string("yhip_create: ") + yhip_last_error(nullptr));
  _ctx = ctx;
  for (int i = 0; i < config->n_layers; ++i) {
    const Block& b = blocks[i];
    check(yhip_upload_layer(_ctx, i, b.rms_att_weight, b.rms_ffn_weight, b.wq, b.wk, b.wv, b.wo, b.w1, b.w2, b.w3),
          "yhip_upload_layer");
  }
  check(yhip_upload_globals(_ctx, token_embedding_table, rms_final_weight,
                            wcls == token_embedding_table ? nullptr : wcls),
        "yhip_upload_globals");
  _device = Device::HIP;
}

void Model::forward(InferenceState& s, int token, int pos, InferenceMode mode) {
  if (s.device() != _device) throw Error("inference state device mismatch");
  if (_device != Device::HIP)
    throw Error("this library implements the HIP device only; move the model and state with hip()");
  // Logits land directly in the context's pinned buffer (the counterpart of the reference's
  // host-registered logits, src/model.cpp:357).
  s._logits = yhip_logits_host(_ctx);
  s._mode = mode;
  check(yhip_forward(_ctx, token, pos, mode == InferenceMode::OUTPUT_LOGITS ? YHIP_MODE_LOGITS : YHIP_MODE_HYDRATE,
                     s._logits),
        "yhip_forward");
}

int Model::forward_argmax(InferenceState& s, int token, int pos) {
  if (s.device() != _device || _device != Device::HIP) throw Error("forward_argmax needs a HIP model and state");
  int next = 0;
  check(yhip_forward_argmax(_ctx, token, pos, &next), "yhip_forward_argmax");
  return next;
}

void Model::prefill(InferenceState& s, const int* tokens, int n, int start_pos) {
  if (s.device() != _device || _device != Device::HIP) throw Error("prefill needs a HIP model and state");
  s._logits = yhip_logits_host(_ctx);
  s._mode = InferenceMode::OUTPUT_LOGITS;
  check(yhip_prefill(_ctx, tokens, n, start_pos, s._logits), "yhip_prefill");
}

// ---- Sampler (reference src/sampler.cpp) -------------------------------------------------------
Sampler::Sampler(std::shared_ptr<Config> config, uint64_t seed) : vocab_size(config->vocab_size) {
  std::srand((unsigned)seed);
}

float Sampler::sample_prob(int index, const InferenceState& s) {
  const float* lg = s.logits();
  float mx = -FLT_MAX;
  for (int i = 0; i < vocab_size; ++i) mx = lg[i] > mx ? lg[i] : mx;
  float sum = 0.f;
  for (int i = 0; i < vocab_size; ++i) sum += expf(lg[i] - mx);
  return expf(lg[index] - mx) / sum;
}

int Sampler::sample_argmax(const InferenceState& s) {
  const float* lg = s.logits();
  int best = 0;
  float mx = -FLT_MAX;
  for (int i = 0; i < vocab_size; ++i)
    if (lg[i] > mx) {
      mx = lg[i];
      best = i;
    }
  return best;
}

int Sampler::sample(const InferenceState& s, float temperature) {
  if (temperature == 0.0f) return sample_argmax(s);
  const float* lg = s.logits();
  float mx = -FLT_MAX;
  for (int i = 0; i < vocab_size; ++i) mx = lg[i] > mx ? lg[i] : mx;
  float sum = 0.f;
  for (int i = 0; i < vocab_size; ++i) sum += expf((lg[i] - mx) / temperature);
  const float r = std::rand() / (float)RAND_MAX;
  float cum = 0.f;
  for (int i = 0; i < vocab_size; ++i) {
    cum += expf((lg[i] - mx) / temperature) / sum;
    if (cum >= r) return i;
  }
  return vocab_size - 1;
}

// ---- Tokenizer (reference src/tokenizer.cpp) ---------------------------------------------------
struct Tokenizer::Trie {
  std::unordered_map<char, std::unique_ptr<Trie>> next;
  int token_id = -1;
};

Tokenizer::Tokenizer(const YALMData& data) {
  bos_id = std::stoi(data.meta("bos_token_id", "-1"));
  eos_id = std::stoi(data.meta("eos_token_id", "-1"));
  const Tensor* t = data.find("tokenizer.tokens");
  if (!t) throw Error("missing tensor: tokenizer.tokens");
  const char* p = (const char*)t->data;
  const char* end = p + t->size;
  while (p < end) {  // NUL-separated strings
    const char* s = p;
    while (p < end && *p != '\0') ++p;
    vocab.emplace_back(s, p - s);
    ++p;
  }
  for (size_t i = 0; i < vocab.size(); ++i) {
    if (vocab[i] == "<0x00>")
      byte_fallback_start = (int)i;
    else if (vocab[i] == "<|eot_id|>" || vocab[i] == "<|end|>" || vocab[i] == "<|im_end|>")
      eot_id = (int)i;
  }
  _root = new Trie();
  for (size_t i = 0; i < vocab.size(); ++i) {
    Trie* n = _root;
    for (char c : vocab[i]) {
      auto& child = n->next[c];
      if (!child) child = std::make_unique<Trie>();
      n = child.get();
    }
    n->token_id = (int)i;
  }
}

Tokenizer::~Tokenizer() { delete _root; }

std::vector<int> Tokenizer::encode(const std::string& text, bool encode_bos) const {
  std::vector<int> out;
  if (encode_bos) out.push_back(bos_id);
  for (size_t i = 0; i < text.size();) {
    // greedy longest match over the vocabulary trie, byte fallback otherwise
    const Trie* n = _root;
    size_t len = 0, best_len = 0;
    int best = -1;
    while (i + len < text.size()) {
      auto it = n->next.find(text[i + len]);
      if (it == n->next.end()) break;
      n = it->second.get();
      ++len;
      if (n->token_id >= 0) {
        best = n->token_id;
        best_len = len;
      }
    }
    if (best < 0) {
      if (byte_fallback_start >= 0) out.push_back((unsigned char)text[i] + byte_fallback_start);
      i += 1;
    } else {
      out.push_back(best);
      i += best_len;
    }
  }
  return out;
}

std::string Tokenizer::decode_one(int prev_token, int token) const {
  if (token < 0 || token >= (int)vocab.size()) return "";
  const std::string& piece = vocab[token];
  if (prev_token == bos_id && !piece.empty() && piece[0] == ' ') return piece.substr(1);
  if (byte_fallback_start >= 0 && token >= byte_fallback_start && token - byte_fallback_start < 256)
    return std::string(1, (char)(token - byte_fallback_start));
  return piece;
}

std::string Tokenizer::encoding_to_debug_string(const std::vector<int>& encoding) const {
  std::string s;
  for (int id : encoding) {
    if (id == bos_id)
      s += "[<s>:" + std::to_string(id) + "]";
    else if (id == eos_id)
      s += "[</s>:" + std::to_string(id) + "]";
    else if (id >= 0 && id < (int)vocab.size())
      s += "[" + vocab[id] + ":" + std::to_string(id) + "]";
    else
      s += "[?:" + std::to_string(id) + "]";
  }
  return s;
}

}  // namespace yalm
