// safetensors header parsing and validation (see safetensors.h).
#include "safetensors.h"

#include <string.h>

#include <algorithm>

#include "json.h"

namespace ltxw {
namespace st {

namespace {

struct DtypeRow {
  const char* name;
  int bits;
};
// Indexed by Dtype.
const DtypeRow kDtypes[N_DTYPES] = {
    {"BOOL", 8}, {"U8", 8}, {"I8", 8}, {"F8_E5M2", 8}, {"F8_E4M3", 8}, {"I16", 16}, {"U16", 16},
    {"F16", 16}, {"BF16", 16}, {"I32", 32}, {"U32", 32}, {"F32", 32}, {"F64", 64}, {"I64", 64},
    {"U64", 64}, {"F8_E8M0", 8}, {"F4", 4}, {"F6_E2M3", 6}, {"F6_E3M2", 6}, {"C64", 64},
};

// Largest header the format accepts (100 MB).
constexpr uint64_t kMaxHeader = 100000000ull;

ParseError bad(ParseError e, std::string* msg, const std::string& m) {
  *msg = m;
  return e;
}

}  // namespace

const char* dtype_name(int32_t d) { return (d >= 0 && d < N_DTYPES) ? kDtypes[d].name : "?"; }

bool dtype_from_name(const std::string& s, int32_t* d) {
  for (int32_t k = 0; k < N_DTYPES; ++k)
    if (s == kDtypes[k].name) { *d = k; return true; }
  return false;
}

int dtype_bits(int32_t d) { return (d >= 0 && d < N_DTYPES) ? kDtypes[d].bits : 0; }

ParseError parse(const uint8_t* buf, uint64_t len, Header* out, std::string* msg) {
  *out = Header();
  if (len < 8) return bad(HEADER_TOO_SMALL, msg, "file is shorter than the 8-byte header length");
  uint64_t n = 0;
  for (int k = 7; k >= 0; --k) n = (n << 8) | buf[k];
  if (n > kMaxHeader) return bad(HEADER_TOO_LARGE, msg, "header length " + std::to_string(n) + " exceeds 100 MB");
  if (n > len - 8) return bad(INVALID_HEADER_LENGTH, msg, "header length " + std::to_string(n) + " runs past the file");
  const char* h = (const char*)buf + 8;
  if (!json::valid_utf8((const unsigned char*)h, (size_t)n)) return bad(INVALID_HEADER, msg, "header is not UTF-8");
  if (n == 0 || h[0] != '{') return bad(INVALID_HEADER_START, msg, "header does not start with '{'");
  json::Value root;
  std::string jerr;
  json::Parser p(h, (size_t)n);
  if (!p.parse(&root, &jerr)) return bad(INVALID_HEADER_DESERIALIZATION, msg, "header JSON: " + jerr);
  if (root.kind != json::Value::Object) return bad(INVALID_HEADER_DESERIALIZATION, msg, "header is not an object");

  for (const auto& m : root.members) {
    const std::string& name = m.first;
    const json::Value& v = m.second;
    if (name == "__metadata__") {
      if (v.kind == json::Value::Null) continue;
      if (v.kind != json::Value::Object)
        return bad(INVALID_HEADER_DESERIALIZATION, msg, "__metadata__ is not an object");
      for (const auto& kv : v.members) {
        if (kv.second.kind != json::Value::String)
          return bad(INVALID_HEADER_DESERIALIZATION, msg, "__metadata__ value of '" + kv.first + "' is not a string");
        out->metadata[kv.first] = kv.second.text;
      }
      continue;
    }
    auto field_err = [&](const char* what) {
      return bad(INVALID_HEADER_DESERIALIZATION, msg, "tensor '" + name + "': " + what);
    };
    if (v.kind != json::Value::Object) return field_err("entry is not an object");
    const json::Value* dt = v.get("dtype");
    const json::Value* sh = v.get("shape");
    const json::Value* off = v.get("data_offsets");
    if (!dt || dt->kind != json::Value::String) return field_err("missing or non-string dtype");
    if (!sh || sh->kind != json::Value::Array) return field_err("missing or non-array shape");
    if (!off || off->kind != json::Value::Array || off->items.size() != 2)
      return field_err("data_offsets is not a pair");
    TensorInfo ti;
    if (!dtype_from_name(dt->text, &ti.dtype)) return field_err(("unknown dtype " + dt->text).c_str());
    for (const auto& s : sh->items) {
      uint64_t d;
      if (!s.as_u64(&d)) return field_err("shape entry is not a non-negative integer");
      ti.shape.push_back(d);
    }
    if (!off->items[0].as_u64(&ti.begin) || !off->items[1].as_u64(&ti.end))
      return field_err("data_offsets entry is not a non-negative integer");
    for (const auto& t : out->tensors)
      if (t.first == name) return field_err("duplicate tensor name");
    out->tensors.emplace_back(name, ti);
  }

  // Offsets must tile the data section contiguously from 0, each range
  // exactly the tensor's byte size.
  std::vector<size_t> order(out->tensors.size());
  for (size_t k = 0; k < order.size(); ++k) order[k] = k;
  std::stable_sort(order.begin(), order.end(), [&](size_t a, size_t b) {
    const TensorInfo& x = out->tensors[a].second;
    const TensorInfo& y = out->tensors[b].second;
    return x.begin != y.begin ? x.begin < y.begin : x.end < y.end;
  });
  uint64_t pos = 0;
  for (size_t k : order) {
    const std::string& name = out->tensors[k].first;
    const TensorInfo& t = out->tensors[k].second;
    if (t.begin != pos || t.end < t.begin)
      return bad(INVALID_OFFSET, msg, "tensor '" + name + "' has invalid data_offsets");
    pos = t.end;
    uint64_t nel = 1;
    for (uint64_t s : t.shape) {
      if (s != 0 && nel > UINT64_MAX / s) return bad(VALIDATION_OVERFLOW, msg, "tensor '" + name + "' size overflows");
      nel *= s;
    }
    uint64_t bits = (uint64_t)dtype_bits(t.dtype);
    if (nel > UINT64_MAX / bits) return bad(VALIDATION_OVERFLOW, msg, "tensor '" + name + "' size overflows");
    if ((nel * bits) % 8 != 0) return bad(MISALIGNED_SLICE, msg, "tensor '" + name + "' is not a whole number of bytes");
    if (nel * bits / 8 != t.end - t.begin)
      return bad(TENSOR_INVALID_INFO, msg, "tensor '" + name + "': data_offsets span " +
                 std::to_string(t.end - t.begin) + " bytes, dtype and shape need " + std::to_string(nel * bits / 8));
  }
  if (pos != len - 8 - n)
    return bad(METADATA_INCOMPLETE_BUFFER, msg, "data section holds " + std::to_string(len - 8 - n) +
               " bytes, the tensors cover " + std::to_string(pos));
  out->data_start = 8 + n;
  return OK;
}

}  // namespace st
}  // namespace ltxw
