// safetensors container: header parsing and validation.
//
// Layout: u64 little-endian header length N, N bytes of UTF-8 JSON (an object
// of tensor name -> {"dtype", "shape", "data_offsets"} plus an optional
// "__metadata__" object of string values), then the packed tensor bytes.
// The checks follow the format's published rules as the reference reads them
// through `SafeTensors::read_metadata` (crates/ltx-weights/src/store.rs:137,
// src/lora.rs:68; the `safetensors` crate pinned in Cargo.lock).
#pragma once

#include <stdint.h>

#include <map>
#include <string>
#include <vector>

namespace ltxw {
namespace st {

// Element types; values are the C ABI's ltxw_dtype (include/ltxw_store.h).
enum Dtype : int32_t {
  BOOL = 0, U8 = 1, I8 = 2, F8_E5M2 = 3, F8_E4M3 = 4, I16 = 5, U16 = 6, F16 = 7, BF16 = 8,
  I32 = 9, U32 = 10, F32 = 11, F64 = 12, I64 = 13, U64 = 14, F8_E8M0 = 15, F4 = 16,
  F6_E2M3 = 17, F6_E3M2 = 18, C64 = 19, N_DTYPES = 20
};

const char* dtype_name(int32_t d);
bool dtype_from_name(const std::string& s, int32_t* d);
int dtype_bits(int32_t d);
inline bool is_fp8(int32_t d) { return d == F8_E4M3 || d == F8_E5M2; }

struct TensorInfo {
  int32_t dtype = 0;
  std::vector<uint64_t> shape;
  uint64_t begin = 0, end = 0;  // relative to the data section
  uint64_t numel() const {
    uint64_t n = 1;
    for (uint64_t s : shape) n *= s;
    return n;
  }
};

struct Header {
  uint64_t data_start = 0;  // 8 + N
  std::vector<std::pair<std::string, TensorInfo>> tensors;  // in header order
  std::map<std::string, std::string> metadata;
};

// Error classes: the safetensors crate's error kinds that reach the reference
// as `WeightError::Safetensors`.
enum ParseError { OK = 0, HEADER_TOO_SMALL, HEADER_TOO_LARGE, INVALID_HEADER_LENGTH, INVALID_HEADER,
                  INVALID_HEADER_START, INVALID_HEADER_DESERIALIZATION, INVALID_OFFSET,
                  VALIDATION_OVERFLOW, MISALIGNED_SLICE, TENSOR_INVALID_INFO,
                  METADATA_INCOMPLETE_BUFFER };

// Parses and validates the container in buf[0, len). On failure returns the
// error kind and fills *msg.
ParseError parse(const uint8_t* buf, uint64_t len, Header* out, std::string* msg);

}  // namespace st
}  // namespace ltxw
