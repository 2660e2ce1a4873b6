// Internal representation of an open safetensors file (dq8_st), shared by the
// reader (dq8_safetensors.cpp) and the device load path (dq8_api.hip).  Host only.
#pragma once
#include <stddef.h>
#include <stdint.h>

#include <string>
#include <vector>

struct dq8_st_tensor {
  std::string name;
  std::string dtype;          // as written in the header
  int bits = 0;               // element size in bits
  std::vector<size_t> shape;
  uint64_t begin = 0, end = 0;  // data_offsets, relative to the data section
};

struct dq8_st {
  int fd = -1;
  uint64_t length = 0;                 // file length
  uint64_t data_start = 0;             // 8 + header size
  std::vector<dq8_st_tensor> tensors;  // ascending data offsets
};

namespace dq8 {
// kDtype* code of a readable weight dtype (F32, BF16, F16), -1 for any other.
int st_dtype_code(const std::string& dtype);
// Reads count bytes of the file at absolute offset `at`; false on error or EOF.
bool st_pread(const dq8_st* st, void* dst, size_t count, uint64_t at);
// Data::read's value check (weights.rs:170-187): every element finite.
bool st_all_finite(int code, const void* data, size_t bytes);
}  // namespace dq8
