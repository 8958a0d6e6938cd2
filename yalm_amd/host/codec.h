// .yalm checkpoint codec (safetensors container): 8-byte little-endian header length, a JSON
// header with "__metadata__" (string values) and per-tensor {dtype, shape, data_offsets}, then the
// raw tensor bytes. Format and validation rules follow the reference reader (src/codec.h:15-50,
// src/codec.cpp:39-156); the implementation is this project's own.
#pragma once
#include <array>
#include <cstddef>
#include <cstdint>
#include <map>
#include <string>
#include <unordered_map>
#include <vector>

namespace yalm {

typedef uint16_t f16_t;

enum class DType { F32, F16, BF16, F8E5M2, F8E4M3, I32, I16, I8, U8 };

std::string dtype_to_string(DType d);
size_t dtype_size(DType d);
bool dtype_from_string(const std::string& s, DType& out);

struct Tensor {
  std::string name;
  DType dtype = DType::F32;
  std::array<int, 4> shape = {0, 0, 0, 0};
  void* data = nullptr;
  size_t size = 0;  // bytes
};

struct YALMData {
  void* data = nullptr;  // mapping (file) or heap block (synthetic)
  size_t size = 0;
  std::map<std::string, std::string> metadata;
  std::unordered_map<std::string, Tensor> tensors;
  std::string error;

  YALMData() = default;
  YALMData(const YALMData&) = delete;
  YALMData& operator=(const YALMData&) = delete;
  ~YALMData();

  // Maps a .yalm file (MAP_PRIVATE, read-ahead advised). Returns 0 on success, -1 on failure with
  // `error` set. Rejected like the reference: files shorter than 8 bytes, a zero or oversized header
  // length, unknown dtypes, data_offsets that are not two values with start < end <= payload size,
  // and tensors whose byte size differs from prod(shape) * dtype size.
  int from_file(const std::string& path);
  // Adopts a heap block laid out like a file image (used by the synthetic-model writer).
  int from_memory(void* block, size_t size, bool owned);

  const Tensor* find(const std::string& name) const;
  std::string meta(const std::string& key, const std::string& fallback = "") const;
  bool has_meta(const std::string& key) const { return metadata.count(key) != 0; }

 private:
  bool mapped_ = false;
  bool owned_ = false;
  int parse();
};

// One tensor to write: name, dtype, shape (up to 4 dims, trailing zeros ignored), bytes.
struct TensorSpec {
  std::string name;
  DType dtype;
  std::vector<int> shape;
  const void* data;
  size_t size;
};

// Builds the header for `tensors` in the given order (offsets assigned contiguously, 8-byte aligned
// header). Returns the header bytes including the 8-byte length prefix.
std::string yalm_header(const std::map<std::string, std::string>& metadata, const std::vector<TensorSpec>& tensors,
                        std::vector<size_t>* offsets_out = nullptr, size_t* payload_out = nullptr);
// Writes a .yalm file. Returns 0 on success.
int yalm_write(const std::string& path, const std::map<std::string, std::string>& metadata,
               const std::vector<TensorSpec>& tensors, std::string* err = nullptr);

// fp16 <-> fp32, round-to-nearest-even (bit-level, no ISA extension required).
float half_to_float(f16_t h);
f16_t float_to_half(float f);

}  // namespace yalm
