#include "codec.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "json.h"

namespace yalm {

std::string dtype_to_string(DType d) {
  switch (d) {
    case DType::F32: return "F32";
    case DType::F16: return "F16";
    case DType::BF16: return "BF16";
    case DType::F8E5M2: return "F8_E5M2";
    case DType::F8E4M3: return "F8_E4M3";
    case DType::I32: return "I32";
    case DType::I16: return "I16";
    case DType::I8: return "I8";
    case DType::U8: return "U8";
  }
  return "UNKNOWN";
}

size_t dtype_size(DType d) {
  switch (d) {
    case DType::F32:
    case DType::I32: return 4;
    case DType::F16:
    case DType::BF16:
    case DType::I16: return 2;
    case DType::F8E5M2:
    case DType::F8E4M3:
    case DType::I8:
    case DType::U8: return 1;
  }
  return 0;
}

bool dtype_from_string(const std::string& s, DType& out) {
  static const std::pair<const char*, DType> table[] = {
      {"F32", DType::F32},       {"F16", DType::F16},         {"BF16", DType::BF16},
      {"F8_E5M2", DType::F8E5M2}, {"F8_E4M3", DType::F8E4M3}, {"I32", DType::I32},
      {"I16", DType::I16},       {"I8", DType::I8},           {"U8", DType::U8}};
  for (const auto& e : table)
    if (s == e.first) {
      out = e.second;
      return true;
    }
  return false;
}

YALMData::~YALMData() {
  if (!data) return;
  if (mapped_)
    munmap(data, size);
  else if (owned_)
    free(data);
}

int YALMData::from_file(const std::string& path) {
  int fd = open(path.c_str(), O_RDONLY);
  if (fd < 0) {
    error = "cannot open " + path;
    return -1;
  }
  struct stat st;
  if (fstat(fd, &st) != 0) {
    close(fd);
    error = "cannot stat " + path;
    return -1;
  }
  size = (size_t)st.st_size;
  if (size < sizeof(uint64_t)) {
    close(fd);
    error = "file too short for a header length";
    return -1;
  }
  void* p = mmap(nullptr, size, PROT_READ | PROT_WRITE, MAP_PRIVATE, fd, 0);
  if (p == MAP_FAILED) {
    close(fd);
    error = "mmap failed";
    return -1;
  }
#ifdef __linux__
  posix_fadvise(fd, 0, size, POSIX_FADV_SEQUENTIAL);
#endif
  close(fd);
  data = p;
  mapped_ = true;
  return parse();
}

int YALMData::from_memory(void* block, size_t n, bool owned) {
  data = block;
  size = n;
  owned_ = owned;
  return parse();
}

int YALMData::parse() {
  uint64_t hlen = 0;
  memcpy(&hlen, data, sizeof(hlen));
  if (hlen == 0 || hlen > size - sizeof(uint64_t)) {
    error = "bad header length";
    return -1;
  }
  const char* hp = (const char*)data + sizeof(uint64_t);
  char* payload = (char*)data + sizeof(uint64_t) + hlen;
  const size_t payload_size = size - sizeof(uint64_t) - hlen;
  Json header;
  std::string perr;
  if (!json_parse(std::string(hp, hlen), header, perr) || !header.is_object()) {
    error = "bad JSON header: " + perr;
    return -1;
  }
  for (const auto& kv : header.obj) {
    const std::string& key = kv.first;
    const Json& val = kv.second;
    if (key == "__metadata__") {
      if (!val.is_object()) {
        error = "__metadata__ is not an object";
        return -1;
      }
      for (const auto& m : val.obj)
        if (m.second.is_string()) metadata[m.first] = m.second.str;
      continue;
    }
    Tensor t;
    t.name = key;
    const Json* dt = val.find("dtype");
    const Json* sh = val.find("shape");
    const Json* off = val.find("data_offsets");
    if (!dt || !dt->is_string() || !dtype_from_string(dt->str, t.dtype)) {
      error = "bad dtype for " + key;
      return -1;
    }
    if (!sh || !sh->is_array()) {
      error = "bad shape for " + key;
      return -1;
    }
    size_t numel = 1;
    for (size_t i = 0; i < sh->arr.size() && i < 4; ++i) {
      const Json& d = sh->arr[i];
      if (!d.is_number() || !d.is_integer || d.i64 < 0 || d.i64 > 0x7fffffff) {
        error = "bad shape for " + key;
        return -1;
      }
      t.shape[i] = (int)d.i64;
      numel *= (size_t)d.i64;
    }
    if (sh->arr.size() > 4) fprintf(stderr, "warning: %s has more than 4 dimensions\n", key.c_str());
    if (!off || !off->is_array() || off->arr.size() != 2 || !off->arr[0].is_integer || !off->arr[1].is_integer) {
      error = "bad data_offsets for " + key;
      return -1;
    }
    const int64_t s0 = off->arr[0].i64, s1 = off->arr[1].i64;
    if (s0 < 0 || s1 <= s0 || (uint64_t)s1 > payload_size) {
      error = "bad offsets for " + key;
      return -1;
    }
    t.data = payload + s0;
    t.size = (size_t)(s1 - s0);
    if (numel * dtype_size(t.dtype) != t.size) {
      error = "size of " + key + " does not match its shape";
      return -1;
    }
    tensors[key] = t;
  }
  return 0;
}

const Tensor* YALMData::find(const std::string& name) const {
  auto it = tensors.find(name);
  return it == tensors.end() ? nullptr : &it->second;
}

std::string YALMData::meta(const std::string& key, const std::string& fallback) const {
  auto it = metadata.find(key);
  return it == metadata.end() ? fallback : it->second;
}

std::string yalm_header(const std::map<std::string, std::string>& metadata, const std::vector<TensorSpec>& tensors,
                        std::vector<size_t>* offsets_out, size_t* payload_out) {
  std::string h = "{";
  bool first = true;
  if (!metadata.empty()) {
    h += "\"__metadata__\":{";
    bool f2 = true;
    for (const auto& kv : metadata) {
      if (!f2) h += ",";
      f2 = false;
      h += json_quote(kv.first) + ":" + json_quote(kv.second);
    }
    h += "}";
    first = false;
  }
  size_t off = 0;
  if (offsets_out) offsets_out->clear();
  for (const auto& t : tensors) {
    if (!first) h += ",";
    first = false;
    h += json_quote(t.name) + ":{\"dtype\":\"" + dtype_to_string(t.dtype) + "\",\"shape\":[";
    for (size_t i = 0; i < t.shape.size(); ++i) h += (i ? "," : "") + std::to_string(t.shape[i]);
    h += "],\"data_offsets\":[" + std::to_string(off) + "," + std::to_string(off + t.size) + "]}";
    if (offsets_out) offsets_out->push_back(off);
    off += t.size;
  }
  h += "}";
  while ((h.size() + 8) % 8) h += ' ';  // keep the payload 8-byte aligned, as safetensors does
  uint64_t n = h.size();
  std::string out(8, '\0');
  memcpy(&out[0], &n, 8);
  if (payload_out) *payload_out = off;
  return out + h;
}

int yalm_write(const std::string& path, const std::map<std::string, std::string>& metadata,
               const std::vector<TensorSpec>& tensors, std::string* err) {
  std::string head = yalm_header(metadata, tensors);
  FILE* f = fopen(path.c_str(), "wb");
  if (!f) {
    if (err) *err = "cannot create " + path;
    return -1;
  }
  bool ok = fwrite(head.data(), 1, head.size(), f) == head.size();
  for (const auto& t : tensors) ok = ok && fwrite(t.data, 1, t.size, f) == t.size;
  ok = (fclose(f) == 0) && ok;
  if (!ok && err) *err = "write failed for " + path;
  return ok ? 0 : -1;
}

float half_to_float(f16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000) << 16;
  uint32_t exp = (h >> 10) & 0x1f;
  uint32_t man = h & 0x3ff;
  uint32_t bits;
  if (exp == 0x1f) {
    bits = sign | 0x7f800000u | (man << 13);
  } else if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {  // subnormal: normalise
      int e = -1;
      do {
        man <<= 1;
        ++e;
      } while (!(man & 0x400));
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ff) << 13);
    }
  } else {
    bits = sign | ((exp + 112) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

f16_t float_to_half(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000);
  const uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return sign | (ax > 0x7f800000u ? 0x7e00 : 0x7c00);  // NaN / Inf
  if (ax >= 0x477ff000u) return sign | 0x7c00;  // rounds to >= 65520 -> Inf
  if (ax < 0x38800000u) {                       // below the smallest normal half: subnormal or zero
    if (ax < 0x33000000u) return sign;          // < 2^-25 rounds to zero (ties at 2^-25 go to even 0)
    const uint32_t e = ax >> 23;
    const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    const int shift = 126 - (int)e;  // value = m * 2^(e-150); half subnormal unit 2^-24
    uint32_t q = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1))) ++q;
    return sign | (uint16_t)q;
  }
  uint32_t r = ax - ((127 - 15) << 23);  // rebias
  const uint32_t lsb = (r >> 13) & 1;
  r += 0xfff + lsb;  // round to nearest even on the 13 dropped bits
  return sign | (uint16_t)(r >> 13);
}

}  // namespace yalm
