// libyalm_host.so C-ABI (include/yalm_host.h) over the C++ host classes.
#include <chrono>
#include <cstring>
#include <memory>
#include <string>

#include "model.h"
#include "synth.h"
#include "yalm_host.h"

using namespace yalm;

struct yalm_session {
  std::unique_ptr<YALMData> data;
  std::unique_ptr<Model> model;
  std::unique_ptr<InferenceState> state;
  std::unique_ptr<Sampler> sampler;
  int eos_id = -1;
  std::string err;
};

namespace {
thread_local std::string g_err;

int set_err(yalm_session* s, const std::string& m) {
  if (s)
    s->err = m;
  else
    g_err = m;
  return -1;
}

int finish_open(std::unique_ptr<yalm_session>& s, int context, yalm_session** out) {
  try {
    s->model = std::make_unique<Model>(*s->data, context);
  } catch (const std::exception& e) {
    g_err = e.what();
    return -1;
  }
  s->state = std::make_unique<InferenceState>(s->model->config);
  s->sampler = std::make_unique<Sampler>(s->model->config, 0x5eed);
  s->eos_id = std::stoi(s->data->meta("eos_token_id", "-1"));
  *out = s.release();
  return 0;
}
}  // namespace

extern "C" int yalm_session_open(const char* path, int context, yalm_session** out) {
  if (!path || !out) return set_err(nullptr, "null argument");
  auto s = std::make_unique<yalm_session>();
  s->data = std::make_unique<YALMData>();
  if (s->data->from_file(path) != 0) return set_err(nullptr, s->data->error);
  return finish_open(s, context, out);
}

extern "C" int yalm_session_synthetic(const yalm_synth_spec* spec, int context, yalm_session** out) {
  if (!spec || !out) return set_err(nullptr, "null argument");
  SynthSpec ss;
  ss.dim = spec->dim;
  ss.hidden_dim = spec->hidden_dim;
  ss.head_dim = spec->head_dim;
  ss.n_layers = spec->n_layers;
  ss.n_heads = spec->n_heads;
  ss.n_kv_heads = spec->n_kv_heads;
  ss.vocab_size = spec->vocab_size;
  ss.max_seq_len = spec->max_seq_len;
  ss.rope_theta = spec->rope_theta;
  ss.norm_eps = spec->norm_eps;
  ss.std = spec->std;
  ss.seed = spec->seed;
  ss.tied_embeddings = spec->tied_embeddings != 0;
  auto s = std::make_unique<yalm_session>();
  s->data = std::make_unique<YALMData>();
  std::string e;
  if (synth_build(ss, *s->data, &e) != 0) return set_err(nullptr, e);
  return finish_open(s, context, out);
}

extern "C" int yalm_session_write(const yalm_session* s, const char* path) {
  if (!s || !path) return set_err(nullptr, "null argument");
  FILE* f = fopen(path, "wb");
  if (!f) return set_err(const_cast<yalm_session*>(s), std::string("cannot create ") + path);
  const bool ok = fwrite(s->data->data, 1, s->data->size, f) == s->data->size;
  if (fclose(f) != 0 || !ok) return set_err(const_cast<yalm_session*>(s), "write failed");
  return 0;
}

extern "C" int yalm_session_hip(yalm_session* s, int device_ordinal) {
  if (!s) return set_err(nullptr, "null session");
  try {
    s->model->hip(device_ordinal);
    s->state->hip();
  } catch (const std::exception& e) {
    return set_err(s, e.what());
  }
  return 0;
}

extern "C" void yalm_session_close(yalm_session* s) { delete s; }

extern "C" const char* yalm_session_error(const yalm_session* s) { return s ? s->err.c_str() : g_err.c_str(); }

extern "C" int yalm_session_config(const yalm_session* s, yhip_config* out) {
  if (!s || !out) return set_err(nullptr, "null argument");
  *out = s->model->config->to_hip();
  return 0;
}

extern "C" int yalm_session_tensor(const yalm_session* s, const char* name, const void** data, size_t* bytes, int* dtype,
                                   int shape[4]) {
  if (!s || !name) return set_err(nullptr, "null argument");
  const Tensor* t = s->data->find(name);
  if (!t) return set_err(const_cast<yalm_session*>(s), std::string("no tensor ") + name);
  if (data) *data = t->data;
  if (bytes) *bytes = t->size;
  if (dtype) *dtype = (int)t->dtype;
  if (shape)
    for (int i = 0; i < 4; ++i) shape[i] = t->shape[i];
  return 0;
}

extern "C" yhip_ctx* yalm_session_hip_ctx(yalm_session* s) { return s && s->model ? s->model->hip_context() : nullptr; }

extern "C" int yalm_session_forward(yalm_session* s, int token, int pos, int mode, float* logits) {
  if (!s) return set_err(nullptr, "null session");
  try {
    s->model->forward(*s->state, token, pos,
                      mode == YHIP_MODE_LOGITS ? InferenceMode::OUTPUT_LOGITS : InferenceMode::HYDRATE_KV_CACHE);
  } catch (const std::exception& e) {
    return set_err(s, e.what());
  }
  if (logits && mode == YHIP_MODE_LOGITS)
    memcpy(logits, s->state->logits(), sizeof(float) * (size_t)s->model->config->vocab_size);
  return 0;
}

extern "C" int yalm_session_prefill(yalm_session* s, const int* tokens, int n, int start_pos, float* logits) {
  if (!s || !tokens || n <= 0) return set_err(s, "bad argument");
  try {
    s->model->prefill(*s->state, tokens, n, start_pos);
  } catch (const std::exception& e) {
    return set_err(s, e.what());
  }
  if (logits) memcpy(logits, s->state->logits(), sizeof(float) * (size_t)s->model->config->vocab_size);
  return 0;
}

extern "C" int yalm_session_generate(yalm_session* s, const int* prompt, int n_prompt, int n_steps, float temperature,
                                     int device_argmax, int batched_prefill, int stop_at_eos, int* out_tokens,
                                     double* step_seconds, double* hydrate_seconds) {
  if (!s || !prompt || n_prompt <= 0 || n_steps < 0) return set_err(s, "bad argument");
  using clk = std::chrono::steady_clock;
  Model& m = *s->model;
  InferenceState& st = *s->state;
  const bool greedy_dev = device_argmax && temperature == 0.0f;
  try {
    m.forward(st, 0, 0);  // warm-up (reference src/main.cpp:144-148)
    auto t0 = clk::now();
    int pos = 0;
    int next = -1;
    if (batched_prefill) {
      m.prefill(st, prompt, n_prompt, 0);
      pos = n_prompt;
      if (greedy_dev) next = s->sampler->sample_argmax(st);
    } else {
      for (int i = 0; i < n_prompt; ++i, ++pos) {
        const bool last = i + 1 == n_prompt;
        if (last && greedy_dev)
          next = m.forward_argmax(st, prompt[i], pos);
        else
          m.forward(st, prompt[i], pos, last ? InferenceMode::OUTPUT_LOGITS : InferenceMode::HYDRATE_KV_CACHE);
      }
    }
    if (hydrate_seconds) *hydrate_seconds = std::chrono::duration<double>(clk::now() - t0).count();
    int produced = 0;
    for (int i = 0; i < n_steps; ++i) {
      auto ts = clk::now();
      const int tok = greedy_dev ? next : s->sampler->sample(st, temperature);
      if (out_tokens) out_tokens[i] = tok;
      ++produced;
      if (stop_at_eos && tok == s->eos_id) {
        if (step_seconds) step_seconds[i] = std::chrono::duration<double>(clk::now() - ts).count();
        break;
      }
      if (greedy_dev)
        next = m.forward_argmax(st, tok, pos);
      else
        m.forward(st, tok, pos);
      ++pos;
      if (step_seconds) step_seconds[i] = std::chrono::duration<double>(clk::now() - ts).count();
    }
    return produced;
  } catch (const std::exception& e) {
    return set_err(s, e.what());
  }
}

extern "C" size_t yalm_session_active_bytes(const yalm_session* s, size_t pos) {
  return s ? s->model->config->active_bytes(pos) : 0;
}

extern "C" void yalm_uniform_ids(int* out, size_t n, uint64_t seed, int hi) { fill_uniform_ids(out, n, seed, hi); }

extern "C" void yalm_fill_normal_f16(uint16_t* out, size_t n, uint64_t seed, const char* stream_name, float std) {
  fill_normal_f16(out, n, seed, stream_name ? stream_name : "", std);
}

extern "C" void yalm_f32_to_f16(const float* in, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = float_to_half(in[i]);
}

extern "C" void yalm_f16_to_f32(const uint16_t* in, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = half_to_float(in[i]);
}
