#include "synth.h"

#include <cmath>
#include <cstdlib>
#include <cstring>

namespace yalm {

uint64_t fnv1a64(const std::string& s) {
  uint64_t h = 0xcbf29ce484222325ull;
  for (unsigned char c : s) {
    h ^= c;
    h *= 0x100000001b3ull;
  }
  return h;
}

uint64_t mix64(uint64_t x) {
  x ^= x >> 30;
  x *= 0xbf58476d1ce4e5b9ull;
  x ^= x >> 27;
  x *= 0x94d049bb133111ebull;
  x ^= x >> 31;
  return x;
}

void fill_normal_f16(f16_t* out, size_t n, uint64_t seed, const std::string& name, float std) {
  const uint64_t base = seed ^ mix64(fnv1a64(name));
  const size_t pairs = (n + 1) / 2;
  const float two_pi = 6.28318530717958647692f;
#pragma omp parallel for schedule(static)
  for (size_t p = 0; p < pairs; ++p) {
    const uint64_t r = mix64(base + (uint64_t)p * 0x9e3779b97f4a7c15ull);
    const float u1 = ((float)(r >> 40) + 1.0f) * (1.0f / 16777216.0f);  // (0, 1]
    const float u2 = (float)((r >> 16) & 0xffffff) * (1.0f / 16777216.0f);
    const float rad = sqrtf(-2.0f * logf(u1)) * std;
    const float a = two_pi * u2;
    out[2 * p] = float_to_half(rad * cosf(a));
    if (2 * p + 1 < n) out[2 * p + 1] = float_to_half(rad * sinf(a));
  }
}

void fill_uniform_ids(int* out, size_t n, uint64_t seed, int hi) {
  for (size_t i = 0; i < n; ++i) out[i] = (int)(mix64(mix64(seed) + i * 0x9e3779b97f4a7c15ull) % (uint64_t)hi);
}

std::map<std::string, std::string> synth_metadata(const SynthSpec& s) {
  auto num = [](double v) {
    char b[64];
    snprintf(b, sizeof(b), "%.9g", v);
    return std::string(b);
  };
  return {
      {"arch", "MistralForCausalLM"},
      {"dtype", "fp16"},
      {"dim", std::to_string(s.dim)},
      {"hidden_dim", std::to_string(s.hidden_dim)},
      {"head_dim", std::to_string(s.head_dim)},
      {"n_layers", std::to_string(s.n_layers)},
      {"n_heads", std::to_string(s.n_heads)},
      {"n_kv_heads", std::to_string(s.n_kv_heads)},
      {"vocab_size", std::to_string(s.vocab_size)},
      {"max_seq_len", std::to_string(s.max_seq_len)},
      {"bos_token_id", "1"},
      {"eos_token_id", "2"},
      {"rope_theta", num(s.rope_theta)},
      {"rotary_dim", std::to_string(s.head_dim)},
      {"norm_eps", num(s.norm_eps)},
      {"norm_type", "rmsnorm"},
      {"act_type", "silu"},
  };
}

int synth_build(const SynthSpec& s, YALMData& out, std::string* err) {
  if (s.dim <= 0 || s.hidden_dim <= 0 || s.head_dim <= 0 || s.n_layers < 0 || s.n_heads <= 0 || s.n_kv_heads <= 0 ||
      s.vocab_size <= 3) {
    if (err) *err = "invalid synthetic model shape";
    return -1;
  }
  struct Item {
    std::string name;
    DType dtype;
    std::vector<int> shape;
    size_t size;
    int kind;  // 0 normal fp16, 1 ones fp32, 2 vocab bytes
  };
  std::vector<Item> items;
  auto w = [&](const std::string& n, int a, int b) { items.push_back({n, DType::F16, {a, b}, (size_t)a * b * 2, 0}); };
  auto g = [&](const std::string& n) { items.push_back({n, DType::F32, {s.dim}, (size_t)s.dim * 4, 1}); };
  const int qd = s.n_heads * s.head_dim, kvd = s.n_kv_heads * s.head_dim;
  w("model.embed.weight", s.vocab_size, s.dim);
  for (int l = 0; l < s.n_layers; ++l) {
    const std::string p = "model.layers." + std::to_string(l) + ".";
    g(p + "attn.norm.weight");
    g(p + "mlp.norm.weight");
    w(p + "attn.wq.weight", qd, s.dim);
    w(p + "attn.wk.weight", kvd, s.dim);
    w(p + "attn.wv.weight", kvd, s.dim);
    w(p + "attn.wo.weight", s.dim, qd);
    w(p + "mlp.w1.weight", s.hidden_dim, s.dim);
    w(p + "mlp.w2.weight", s.dim, s.hidden_dim);
    w(p + "mlp.w3.weight", s.hidden_dim, s.dim);
  }
  g("model.norm.weight");
  if (!s.tied_embeddings) w("model.output.weight", s.vocab_size, s.dim);
  // A loader-compatible vocabulary: <unk>, <s>, </s>, 256 byte-fallback pieces, then "t<i>".
  std::string vocab_bytes;
  for (int i = 0; i < s.vocab_size; ++i) {
    std::string piece;
    if (i == 0) piece = "<unk>";
    else if (i == 1) piece = "<s>";
    else if (i == 2) piece = "</s>";
    else if (i < 3 + 256) {
      char b[8];
      snprintf(b, sizeof(b), "<0x%02X>", i - 3);
      piece = b;
    } else {
      piece = " t" + std::to_string(i);
    }
    vocab_bytes += piece;
    vocab_bytes += '\0';
  }
  items.push_back({"tokenizer.tokens", DType::U8, {(int)vocab_bytes.size()}, vocab_bytes.size(), 2});

  std::vector<TensorSpec> specs;
  for (const auto& it : items) specs.push_back({it.name, it.dtype, it.shape, nullptr, it.size});
  std::vector<size_t> offs;
  size_t payload = 0;
  const std::string head = yalm_header(synth_metadata(s), specs, &offs, &payload);
  const size_t total = head.size() + payload;
  char* block = (char*)aligned_alloc(4096, (total + 4095) / 4096 * 4096);
  if (!block) {
    if (err) *err = "out of host memory for the synthetic model";
    return -1;
  }
  memcpy(block, head.data(), head.size());
  char* pay = block + head.size();
  for (size_t i = 0; i < items.size(); ++i) {
    const Item& it = items[i];
    char* dst = pay + offs[i];
    if (it.kind == 0) {
      fill_normal_f16((f16_t*)dst, it.size / 2, s.seed, it.name, s.std);
    } else if (it.kind == 1) {
      float* f = (float*)dst;
      for (int k = 0; k < s.dim; ++k) f[k] = 1.0f;
    } else {
      memcpy(dst, vocab_bytes.data(), vocab_bytes.size());
    }
  }
  if (out.from_memory(block, total, true) != 0) {
    if (err) *err = out.error;
    return -1;
  }
  return 0;
}

}  // namespace yalm
