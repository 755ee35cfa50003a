// Seeded synthetic LTX-2.5 DiT checkpoints and LoRA adapters as safetensors
// files, written by many threads. Every value is a pure function of
// (seed, tensor name, element index), the same functions ltx_weights/synth.py
// restates in numpy, so any row of any tensor can be regenerated to check a
// materialised result without keeping expected data.
//
// Generator: splitmix64's finaliser over a per-tensor key,
//   key(t)     = mix(seed ^ mix(fnv1a64(name)))
//   word(t, j) = mix(key(t) + (j + 1) * 0x9E3779B97F4A7C15)
// FP8 byte e    : byte e % 8 of word(t, e / 8), mapped onto the format's
//                 finite codes as codes[(b * n_codes) >> 8]
// f32 scale o   : (float)(1e-3 + u * (0.1 - 1e-3)), u = (word(t, o) >> 11) * 2^-53
// bf16 factor e : 0.02 * (sum of the twelve 16-bit lanes of words 3e..3e+2
//                 / 65536 - 6) in f64 (Irwin-Hall approximation of N(0, 1)),
//                 rounded to f32, then to bf16 (nearest even)
// Compiled with -ffp-contract=off so that the f64 arithmetic matches numpy's.
#include <fcntl.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <string>
#include <thread>
#include <vector>

namespace {

constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ull;

inline uint64_t mix(uint64_t x) {
  x ^= x >> 30;
  x *= 0xBF58476D1CE4E5B9ull;
  x ^= x >> 27;
  x *= 0x94D049BB133111EBull;
  x ^= x >> 31;
  return x;
}

uint64_t fnv1a64(const std::string& s) {
  uint64_t h = 0xCBF29CE484222325ull;
  for (unsigned char c : s) {
    h ^= c;
    h *= 0x100000001B3ull;
  }
  return h;
}

inline uint64_t word(uint64_t key, uint64_t j) { return mix(key + (j + 1) * kGolden); }

enum Kind { FP8_E4M3 = 0, FP8_E5M2 = 1, F32_SCALE = 2, BF16_FACTOR = 3 };

struct Tensor {
  std::string name;
  int kind;
  std::vector<uint64_t> shape;
  uint64_t bytes = 0, begin = 0;
  uint64_t key = 0;
};

// Finite codes: e4m3fn without 0x7F/0xFF (254); e5m2 without Inf/NaN (248).
struct Codes {
  uint8_t c[256];
  int n = 0;
  uint8_t map[256];  // random byte b -> c[(b * n) >> 8]
};
Codes make_codes(int kind) {
  Codes k;
  for (int b = 0; b < 256; ++b) {
    bool ok = kind == FP8_E4M3 ? (b & 0x7F) != 0x7F : (b & 0x7F) < 0x7C;
    if (ok) k.c[k.n++] = (uint8_t)b;
  }
  for (int b = 0; b < 256; ++b) k.map[b] = k.c[(b * k.n) >> 8];
  return k;
}

uint16_t bf16_rne(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float scale_value(uint64_t key, uint64_t o) {
  double u = (double)(word(key, o) >> 11) * 0x1p-53;
  return (float)(1e-3 + u * (0.1 - 1e-3));
}

uint16_t factor_value(uint64_t key, uint64_t e) {
  uint64_t sum = 0;
  for (int q = 0; q < 3; ++q) {
    uint64_t w = word(key, 3 * e + (uint64_t)q);
    for (int l = 0; l < 4; ++l) sum += (w >> (16 * l)) & 0xFFFF;
  }
  double z = (double)sum / 65536.0 - 6.0;
  double x = 0.02 * z;
  return bf16_rne((float)x);
}

// Bytes [b0, b1) of tensor t into dst.
void gen(const Tensor& t, const Codes* codes, uint64_t b0, uint64_t b1, uint8_t* dst) {
  if (t.kind == FP8_E4M3 || t.kind == FP8_E5M2) {
    const Codes& cd = codes[t.kind];
    uint64_t e = b0;
    while (e < b1 && (e & 7)) {  // head up to a word boundary
      uint64_t w = word(t.key, e >> 3);
      *dst++ = cd.map[(w >> (8 * (e & 7))) & 0xFF];
      ++e;
    }
    for (; e + 8 <= b1; e += 8, dst += 8) {  // whole words
      uint64_t w = word(t.key, e >> 3), v = 0;
      for (int k = 0; k < 8; ++k) v |= (uint64_t)cd.map[(w >> (8 * k)) & 0xFF] << (8 * k);
      memcpy(dst, &v, 8);
    }
    for (; e < b1; ++e) *dst++ = cd.map[(word(t.key, e >> 3) >> (8 * (e & 7))) & 0xFF];
    return;
  }
  const uint64_t es = t.kind == F32_SCALE ? 4 : 2;
  for (uint64_t e = b0 / es; e * es < b1; ++e) {
    uint8_t v[4];
    if (t.kind == F32_SCALE) {
      float f = scale_value(t.key, e);
      memcpy(v, &f, 4);
    } else {
      uint16_t h = factor_value(t.key, e);
      memcpy(v, &h, 2);
    }
    for (uint64_t k = 0; k < es; ++k) {
      uint64_t b = e * es + k;
      if (b >= b0 && b < b1) *dst++ = v[k];
    }
  }
}

const char* dtype_of(int kind) {
  switch (kind) {
    case FP8_E4M3: return "F8_E4M3";
    case FP8_E5M2: return "F8_E5M2";
    case F32_SCALE: return "F32";
    default: return "BF16";
  }
}

// Writes the safetensors file: header (padded to 8 bytes), then the data
// section generated in 16 MB chunks by `threads` threads.
int write_file(const char* path, std::vector<Tensor>& ts, uint64_t seed, const char* meta_json, int threads) {
  uint64_t off = 0;
  for (auto& t : ts) {
    uint64_t n = 1;
    for (uint64_t s : t.shape) n *= s;
    t.bytes = n * (t.kind == F32_SCALE ? 4 : t.kind == BF16_FACTOR ? 2 : 1);
    t.begin = off;
    off += t.bytes;
    t.key = mix(seed ^ mix(fnv1a64(t.name)));
  }
  const uint64_t data_bytes = off;
  std::string h = "{\"__metadata__\":";
  h += meta_json;
  for (const auto& t : ts) {
    h += ",\"" + t.name + "\":{\"dtype\":\"" + dtype_of(t.kind) + "\",\"shape\":[";
    for (size_t k = 0; k < t.shape.size(); ++k) h += (k ? "," : "") + std::to_string(t.shape[k]);
    h += "],\"data_offsets\":[" + std::to_string(t.begin) + "," + std::to_string(t.begin + t.bytes) + "]}";
  }
  h += "}";
  while (h.size() % 8) h += ' ';
  int fd = open(path, O_CREAT | O_TRUNC | O_WRONLY | O_CLOEXEC, 0644);
  if (fd < 0) return -1;
  uint8_t len8[8];
  for (int k = 0; k < 8; ++k) len8[k] = (uint8_t)((uint64_t)h.size() >> (8 * k));
  if (pwrite(fd, len8, 8, 0) != 8 || pwrite(fd, h.data(), h.size(), 8) != (ssize_t)h.size()) {
    close(fd);
    return -2;
  }
  const uint64_t base = 8 + h.size();
  if (ftruncate(fd, (off_t)(base + data_bytes)) != 0) {
    close(fd);
    return -3;
  }
  Codes codes[2] = {make_codes(FP8_E4M3), make_codes(FP8_E5M2)};
  const uint64_t chunk = 16ull << 20;
  const uint64_t n_chunks = (data_bytes + chunk - 1) / chunk;
  std::atomic<uint64_t> next{0};
  std::atomic<int> bad{0};
  auto worker = [&]() {
    std::vector<uint8_t> buf(chunk);
    size_t ti = 0;
    for (;;) {
      uint64_t c = next.fetch_add(1);
      if (c >= n_chunks || bad.load()) return;
      uint64_t b0 = c * chunk, b1 = std::min(data_bytes, b0 + chunk);
      // first tensor overlapping b0 (tensors are in offset order)
      ti = (size_t)(std::upper_bound(ts.begin(), ts.end(), b0,
                                     [](uint64_t v, const Tensor& t) { return v < t.begin; }) - ts.begin());
      ti = ti ? ti - 1 : 0;
      for (size_t k = ti; k < ts.size() && ts[k].begin < b1; ++k) {
        const Tensor& t = ts[k];
        uint64_t s0 = std::max(b0, t.begin), s1 = std::min(b1, t.begin + t.bytes);
        if (s0 < s1) gen(t, codes, s0 - t.begin, s1 - t.begin, buf.data() + (s0 - b0));
      }
      const uint8_t* p = buf.data();
      uint64_t left = b1 - b0, at = base + b0;
      while (left) {
        ssize_t w = pwrite(fd, p, left, (off_t)at);
        if (w <= 0) {
          bad.store(1);
          return;
        }
        p += w;
        at += (uint64_t)w;
        left -= (uint64_t)w;
      }
    }
  };
  std::vector<std::thread> th;
  for (int k = 0; k < std::max(1, threads); ++k) th.emplace_back(worker);
  for (auto& t : th) t.join();
  if (close(fd) != 0 || bad.load()) return -4;
  return 0;
}

// One DiT block's LoRA-targeted linears: (name, out, in).
struct Linear {
  const char* name;
  uint64_t out, in;
};
const Linear kBlock[] = {
    {"attn1.to_q", 4096, 4096},     {"attn1.to_k", 4096, 4096},     {"attn1.to_v", 4096, 4096},
    {"attn1.to_out.0", 4096, 4096}, {"attn2.to_q", 4096, 4096},     {"attn2.to_k", 4096, 4096},
    {"attn2.to_v", 4096, 4096},     {"attn2.to_out.0", 4096, 4096}, {"ff.net.0.proj", 16384, 4096},
    {"ff.net.2", 4096, 16384},
};
// Tail tensors of the mixed-format set (widths that are not multiples of 64).
const Linear kEdge[] = {{"edge.proj_a", 4096, 4104}, {"edge.proj_b", 4104, 16384}};

bool is_ffn(const char* name) { return strncmp(name, "ff.", 3) == 0; }

}  // namespace

extern "C" {

// Model file. variant 0: every linear e4m3fn with per-row f32 scales.
// variant 1 (mixed): FFN e5m2 with per-row scales, attention e4m3fn with one
// scale (shape []), plus the two edge tensors (e4m3fn/one scale, e5m2/row
// scales). Keys carry the "model.diffusion_model." prefix of LTX checkpoints.
// Returns 0 or a negative error.
int ltxs_write_model(const char* path, uint64_t seed, int n_blocks, int variant, int threads) {
  std::vector<Tensor> ts;
  const std::string pre = "model.diffusion_model.";
  auto add = [&](const std::string& base, const Linear& L, bool e5m2, bool row_scales) {
    ts.push_back({pre + base + ".weight", e5m2 ? FP8_E5M2 : FP8_E4M3, {L.out, L.in}});
    if (row_scales) ts.push_back({pre + base + ".weight_scale", F32_SCALE, {L.out}});
    else ts.push_back({pre + base + ".weight_scale", F32_SCALE, {}});
  };
  for (int b = 0; b < n_blocks; ++b)
    for (const Linear& L : kBlock) {
      std::string base = "transformer_blocks." + std::to_string(b) + "." + L.name;
      if (variant == 0) add(base, L, false, true);
      else add(base, L, is_ffn(L.name), is_ffn(L.name));
    }
  if (variant == 1) {
    add(kEdge[0].name, kEdge[0], false, false);
    add(kEdge[1].name, kEdge[1], true, true);
  }
  std::string meta = "{\"format\":\"pt\",\"generator\":\"ltxw-synth\",\"seed\":\"" + std::to_string(seed) +
                     "\",\"blocks\":\"" + std::to_string(n_blocks) + "\",\"variant\":\"" + std::to_string(variant) + "\"}";
  return write_file(path, ts, seed, meta.c_str(), threads);
}

// LoRA file of rank `rank` over the same linears (keys without the
// checkpoint prefix, as the store sees them after renaming):
// P.lora_A.weight [rank, in] and P.lora_B.weight [out, rank], bf16, no alpha.
int ltxs_write_lora(const char* path, uint64_t seed, int n_blocks, int variant, int rank, int threads) {
  std::vector<Tensor> ts;
  auto add = [&](const std::string& base, const Linear& L) {
    ts.push_back({base + ".lora_A.weight", BF16_FACTOR, {(uint64_t)rank, L.in}});
    ts.push_back({base + ".lora_B.weight", BF16_FACTOR, {L.out, (uint64_t)rank}});
  };
  for (int b = 0; b < n_blocks; ++b)
    for (const Linear& L : kBlock) add("transformer_blocks." + std::to_string(b) + "." + L.name, L);
  if (variant == 1)
    for (const Linear& L : kEdge) add(L.name, L);
  std::string meta = "{\"format\":\"pt\",\"generator\":\"ltxw-synth\",\"rank\":\"" + std::to_string(rank) + "\"}";
  return write_file(path, ts, seed, meta.c_str(), threads);
}

}  // extern "C"
