// yalm: command-line driver with the reference's contract (src/main.cpp:20-544) on the HIP device.
//
//   yalm <checkpoint.yalm> [-d hip] [-m completion|perplexity|passkey] [-i prompt | -f file | -p ids]
//        [-n steps] [-t temperature] [-T context] [-l passkey_pos] [-b 0|1]
//   yalm --synth <out.yalm> <tiny|mistral-7b> [seed]     write a seeded random-init model
//
// `-p 5,17,900` feeds token ids directly (no tokenizer, no BOS), for synthetic checkpoints.
// `-d cpu` is the reference's own CPU backend and is not part of this library.
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iostream>
#include <sstream>
#include <string>
#include <vector>

#include "model.h"
#include "synth.h"

using namespace yalm;

static void usage() {
  fprintf(stderr,
          "Usage:   yalm <checkpoint> [options]\n"
          "         yalm --synth <out.yalm> <tiny|mistral-7b> [seed]\n"
          "Options:\n"
          "  -h          help\n"
          "  -d hip      device (hip; 'gpu' is an alias)\n"
          "  -m mode     completion (default), perplexity or passkey\n"
          "  -T <int>    context length (0 = metadata value capped at 4096)\n"
          "  -i <str>    prompt text\n"
          "  -f <path>   prompt file\n"
          "  -p <ids>    comma-separated prompt token ids (no BOS added)\n"
          "  -n <int>    steps (completion, default 256; 0 = max_seq_len; -1 = until EOS) or junk lines (passkey)\n"
          "  -t <float>  temperature (default 1.0; 0 = greedy)\n"
          "  -l <int>    passkey position (-1 = random)\n"
          "  -b <0|1>    1: ingest the prompt in one batched prefill instead of token by token (default 0)\n");
  exit(1);
}

static double now_s() {
  return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

static uint64_t now_ms() { return (uint64_t)(now_s() * 1000.0); }

static int synth_main(int argc, char** argv) {
  if (argc < 4) usage();
  SynthSpec s{};
  const std::string which = argv[3];
  if (which == "tiny") {
    s = SynthSpec{256, 768, 32, 4, 8, 2, 32000, 512};
  } else if (which == "mistral-7b") {
    s = SynthSpec{4096, 14336, 128, 32, 32, 8, 32000, 32768};
  } else {
    usage();
  }
  if (argc > 4) s.seed = strtoull(argv[4], nullptr, 0);
  YALMData d;
  std::string err;
  if (synth_build(s, d, &err) != 0) {
    fprintf(stderr, "synth failed: %s\n", err.c_str());
    return 1;
  }
  FILE* f = fopen(argv[2], "wb");
  if (!f || fwrite(d.data, 1, d.size, f) != d.size || fclose(f) != 0) {
    fprintf(stderr, "cannot write %s\n", argv[2]);
    return 1;
  }
  printf("wrote %s (%zu bytes)\n", argv[2], d.size);
  return 0;
}

struct Session {
  YALMData data;
  std::unique_ptr<Model> model;
  std::unique_ptr<InferenceState> state;
  std::unique_ptr<Sampler> sampler;
  std::unique_ptr<Tokenizer> tokenizer;
};

static void open_session(Session& s, const std::string& path, int context, const std::string& device) {
  if (s.data.from_file(path) != 0) throw Error("cannot load " + path + ": " + s.data.error);
  s.model = std::make_unique<Model>(s.data, context);
  s.state = std::make_unique<InferenceState>(s.model->config);
  s.sampler = std::make_unique<Sampler>(s.model->config, now_ms());
  s.tokenizer = std::make_unique<Tokenizer>(s.data);
  std::cout << "Model active bytes with full context window: " << s.model->config->active_bytes(s.model->config->max_seq_len)
            << std::endl;
  if (device == "hip") {
    std::cout << "Using HIP" << std::endl;
    s.model->hip(0);
    s.state->hip();
  }
}

static std::vector<int> parse_ids(const std::string& s) {
  std::vector<int> out;
  std::stringstream ss(s);
  std::string tok;
  while (std::getline(ss, tok, ','))
    if (!tok.empty()) out.push_back(std::stoi(tok));
  return out;
}

// Prompt ingestion: one token at a time in HYDRATE mode as the reference does (src/main.cpp:169-177),
// the last one with logits; or one batched Model::prefill when `batched`.
static void ingest(Session& s, const std::vector<int>& enc, bool batched) {
  Model& m = *s.model;
  if (batched) {
    m.prefill(*s.state, enc.data(), (int)enc.size(), 0);
    return;
  }
  for (size_t pos = 0; pos < enc.size(); ++pos)
    m.forward(*s.state, enc[pos], (int)pos,
              pos + 1 == enc.size() ? InferenceMode::OUTPUT_LOGITS : InferenceMode::HYDRATE_KV_CACHE);
}

static void run_completion(Session& s, const std::string& prompt, const std::string& ids, int num_steps, float temp,
                           bool batched) {
  Model& m = *s.model;
  if (num_steps == 0) num_steps = m.config->max_seq_len;
  m.forward(*s.state, 0, 0);  // warm-up: loads weights, captures the step graph
  std::vector<int> enc;
  {
    const uint64_t t0 = now_ms();
    enc = ids.empty() ? s.tokenizer->encode(prompt, true) : parse_ids(ids);
    const double secs = (now_ms() - t0) / 1000.0;
    std::cout << s.tokenizer->encoding_to_debug_string(enc) << std::endl;
    printf("Encoding stats: (%zu tokens, throughput: %.5gtok/s, latency: %.5gs/tok, total: %.5gs)\n\n", enc.size(),
           enc.size() / std::max(secs, 1e-9), secs / enc.size(), secs);
  }
  if (enc.empty()) throw Error("empty prompt");
  for (int t : enc)
    if (t < 0 || t >= m.config->vocab_size) throw Error("prompt token id out of range");
  const double start = now_s();
  size_t read_bytes = 0;
  ingest(s, enc, batched);
  for (size_t pos = 0; pos < enc.size(); ++pos) read_bytes += m.config->active_bytes(pos);
  const double end_hydrate = now_s();
  for (int i = 0; i < num_steps || num_steps == -1; ++i) {
    const int tok = s.sampler->sample(*s.state, temp);
    std::cout << s.tokenizer->decode_one(enc.back(), tok) << std::flush;
    enc.push_back(tok);
    if (tok == s.tokenizer->eos_id || tok == s.tokenizer->eot_id) break;
    m.forward(*s.state, tok, (int)enc.size() - 1);
    read_bytes += m.config->active_bytes(enc.size() - 1);
  }
  std::cout << "\n" << std::endl;
  const double elapsed = now_s() - start;
  printf(
      "Generation stats:\n  %zu tokens\n  throughput: %.5gtok/s\n  latency: %.5gs/tok\n  hydrate: %.5gs\n"
      "  bandwidth: %.5gGB/s\n  total: %.5gs\n\n",
      enc.size(), enc.size() / elapsed, elapsed / enc.size(), end_hydrate - start, (double)read_bytes / 1e9 / elapsed,
      elapsed);
  printf("tokens:");
  for (int t : enc) printf(" %d", t);
  printf("\n");
}

static void run_perplexity(Session& s, const std::string& prompt, const std::string& ids) {
  Model& m = *s.model;
  m.forward(*s.state, 0, 0);
  std::vector<int> enc = ids.empty() ? s.tokenizer->encode(prompt, true) : parse_ids(ids);
  if (enc.size() < 2) throw Error("perplexity needs at least two tokens");
  double sum = 0, ss = 0;
  const double start = now_s();
  size_t read_bytes = 0;
  const size_t N = enc.size() - 1;
  for (size_t pos = 0; pos + 1 < enc.size(); ++pos) {
    std::cout << "\r Computing perplexity..." << pos + 1 << "/" << N << std::flush;
    m.forward(*s.state, enc[pos], (int)pos);
    read_bytes += m.config->active_bytes(pos);
    const double lp = std::log(s.sampler->sample_prob(enc[pos + 1], *s.state));
    sum += lp;
    ss += lp * lp;
  }
  std::cout << std::endl;
  const double elapsed = now_s() - start;
  const double ppl = std::exp(-sum / N);
  const double err = ppl * std::sqrt((ss - sum * sum / N) / N / N);
  printf("Stats:\n  %zu tokens\n  perplexity: %.5g ± %.5g\n  throughput: %.5gtok/s\n  latency: %.5gs/tok\n"
         "  bandwidth: %.5gGB/s\n  total: %.5gs\n\n",
         N, ppl, err, N / elapsed, elapsed / N, (double)read_bytes / 1e9 / elapsed, elapsed);
}

static void run_passkey(Session& s, int n_junk, int passkey_pos, bool batched) {
  Model& m = *s.model;
  m.forward(*s.state, 0, 0);
  const std::string prefix =
      "There is an important info hidden inside a lot of irrelevant text. "
      "Find it and memorize them. I will quiz you about the important information there.";
  const std::string suffix = " What is the pass key? The pass key is";
  const int passkey = std::rand() % 50000 + 1;
  const int at = passkey_pos == -1 ? std::rand() % n_junk : passkey_pos;
  std::string prompt = prefix;
  for (int i = 0; i < n_junk; ++i) {
    if (i % n_junk == at)
      prompt += " The pass key is " + std::to_string(passkey) + ". Remember it. " + std::to_string(passkey) +
                " is the pass key.";
    prompt += " The grass is green. The sky is blue. The sun is yellow. Here we go. There and back again.";
  }
  prompt += suffix;
  std::vector<int> enc = s.tokenizer->encode(prompt, true);
  printf("Passkey test:\n  prompt: %zu tokens\n  passkey: %d\n  passkey token index: ~%d\n\n", enc.size(), passkey,
         (int)((float)at / n_junk * enc.size()));
  const size_t N = enc.size();
  if (batched) {
    ingest(s, enc, true);
  } else {
    for (size_t pos = 0; pos < N; ++pos) {
      std::cout << "\r Running passkey test..." << pos + 1 << "/" << N << std::flush;
      m.forward(*s.state, enc[pos], (int)pos,
                pos + 1 == N ? InferenceMode::OUTPUT_LOGITS : InferenceMode::HYDRATE_KV_CACHE);
    }
  }
  std::cout << std::endl << suffix << std::flush;
  for (size_t pos = N; pos < N + 16; ++pos) {
    const int tok = s.sampler->sample_argmax(*s.state);
    std::cout << s.tokenizer->decode_one(enc.back(), tok) << std::flush;
    enc.push_back(tok);
    if (tok == s.tokenizer->eos_id || tok == s.tokenizer->eot_id) break;
    m.forward(*s.state, tok, (int)pos);
  }
  std::cout << std::endl;
}

int main(int argc, char** argv) {
  if (argc >= 2 && std::string(argv[1]) == "--synth") return synth_main(argc, argv);
  if (argc < 2) usage();
  std::string path = argv[1], device = "hip", mode = "completion", prompt, prompt_path, ids;
  int context = 0, num_steps = 256, n_junk = 250, passkey_pos = -1, batched = 0;
  float temperature = 1.0f;
  for (int i = 2; i < argc; i += 2) {
    if (i + 1 >= argc || argv[i][0] != '-' || strlen(argv[i]) != 2) usage();
    const char f = argv[i][1];
    const std::string v = argv[i + 1];
    switch (f) {
      case 'm':
        if (std::string("completion").starts_with(v)) mode = "completion";
        else if (std::string("passkey").starts_with(v)) mode = "passkey";
        else if (std::string("perplexity").starts_with(v)) mode = "perplexity";
        else usage();
        break;
      case 'd':
        if (v == "hip" || v == "gpu") device = "hip";
        else if (std::string("cpu").starts_with(v)) {
          fprintf(stderr, "-d cpu is the reference's own CPU backend; this binary runs the HIP device (-d hip)\n");
          return 1;
        } else usage();
        break;
      case 'i': prompt = v; break;
      case 'f': prompt_path = v; break;
      case 'p': ids = v; break;
      case 't': temperature = std::stof(v); break;
      case 'T': context = std::stoi(v); break;
      case 'l': passkey_pos = std::stoi(v); break;
      case 'b': batched = std::stoi(v); break;
      case 'n':
        num_steps = std::stoi(v);
        n_junk = num_steps;
        break;
      default: usage();
    }
  }
  if (mode == "completion" || mode == "perplexity") {
    const int n = (int)!prompt.empty() + (int)!prompt_path.empty() + (int)!ids.empty();
    if (n != 1) usage();
    if (!prompt_path.empty()) {
      std::ifstream fin(prompt_path);
      if (!fin) {
        std::cerr << "Error: could not open file " << prompt_path << std::endl;
        return 1;
      }
      std::stringstream b;
      b << fin.rdbuf();
      prompt = b.str();
    }
  } else if (passkey_pos != -1 && (passkey_pos >= n_junk || passkey_pos < 0)) {
    std::cerr << "Error: passkey position must be between 0 and " << n_junk - 1 << std::endl;
    return 1;
  }
  try {
    Session s;
    open_session(s, path, context, device);
    if (mode == "completion")
      run_completion(s, prompt, ids, num_steps, temperature, batched != 0);
    else if (mode == "perplexity")
      run_perplexity(s, prompt, ids);
    else
      run_passkey(s, n_junk, passkey_pos, batched != 0);
  } catch (const std::exception& e) {
    fprintf(stderr, "error: %s\n", e.what());
    return 1;
  }
  return 0;
}
