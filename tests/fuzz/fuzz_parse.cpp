// Mutation fuzz driver for the safetensors header parser (safetensors.cpp),
// built with AddressSanitizer and UndefinedBehaviorSanitizer by
// tests/test_store_fuzz.py. Seeded mutations of a valid header: bit flips,
// JSON-significant characters, header-length changes, truncation, extension.
// Any out-of-bounds access or undefined behaviour aborts the run.
#include <cstdio>
#include <cstdint>
#include <cstring>
#include <random>
#include <string>
#include <vector>
#include "safetensors.h"
using namespace ltxw::st;
static std::vector<uint8_t> make_valid() {
  std::string h = "{\"__metadata__\":{\"format\":\"pt\",\"n\\u00e9\":\"x\\\"y\"},"
                  "\"a.weight\":{\"dtype\":\"F8_E4M3\",\"shape\":[4,8],\"data_offsets\":[0,32]},"
                  "\"a.weight_scale\":{\"dtype\":\"F32\",\"shape\":[4],\"data_offsets\":[32,48]},"
                  "\"b\":{\"dtype\":\"BF16\",\"shape\":[2,3],\"data_offsets\":[48,60]},"
                  "\"e\":{\"dtype\":\"F16\",\"shape\":[0,3],\"data_offsets\":[60,60]}}";
  while (h.size() % 8) h += ' ';
  std::vector<uint8_t> f(8 + h.size() + 60, 0);
  uint64_t n = h.size();
  memcpy(f.data(), &n, 8);
  memcpy(f.data() + 8, h.data(), h.size());
  for (size_t i = 0; i < 60; ++i) f[8 + h.size() + i] = (uint8_t)(i * 7);
  return f;
}
int main(int argc, char** argv) {
  const int iters = argc > 1 ? atoi(argv[1]) : 200000;
  std::mt19937_64 g(12345);
  const std::vector<uint8_t> base = make_valid();
  const char* sig = "{}[],:\"0123456789-.eE\\ u";
  int ok = 0, bad = 0;
  for (int it = 0; it < iters; ++it) {
    std::vector<uint8_t> b = base;
    const uint64_t hlen = b.size() - 8 - 60;
    int nm = 1 + (int)(g() % 4);
    for (int m = 0; m < nm; ++m) {
      switch (g() % 6) {
        case 0: b[8 + g() % hlen] ^= (uint8_t)(1u << (g() % 8)); break;
        case 1: b[8 + g() % hlen] = (uint8_t)sig[g() % strlen(sig)]; break;
        case 2: { uint64_t n = hlen + (g() % 33) - 16; if (g() % 5 == 0) n = g() % (1ull << 40); memcpy(b.data(), &n, 8); break; }
        case 3: b.resize(g() % b.size()); break;
        case 4: b.resize(b.size() + 1 + g() % 64, 0); break;
        default: { size_t i = 8 + g() % hlen; if (i < b.size()) b[i] = (uint8_t)('0' + g() % 10); }
      }
      if (b.size() < 8) break;
    }
    Header h;
    std::string err;
    int rc = parse(b.data(), b.size(), &h, &err);
    if (rc == 0) {
      ++ok;
      for (auto& t : h.tensors) { volatile uint64_t s = t.first.size() + t.second.shape.size() + t.second.numel(); (void)s; }
    } else {
      ++bad;
    }
  }
  printf("ok %d bad %d\n", ok, bad);
  return 0;
}
