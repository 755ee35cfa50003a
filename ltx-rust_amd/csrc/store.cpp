// Weight store (include/ltxw_store.h): memory-mapped safetensors files, key
// renaming, LoRA files and merge bookkeeping, and the staged
// host -> HBM materialisation pipeline that feeds the dequant / LoRA kernels.
//
// Reference: crates/ltx-weights/src/store.rs (WeightStore), src/lora.rs
// (LoraFile, MergeReport), src/key_map.rs (KeyMap::apply_key).
#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#include <immintrin.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "ctx.h"
#include "ltxw_store.h"
#include "safetensors.h"

namespace st = ltxw::st;

namespace {

thread_local std::string g_err;

int sfail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int sfail(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

// Copies mapped tensor bytes into the pinned staging block. The block is read
// next by the copy engine, never by the CPU, so 32-byte streaming stores are
// used where the CPU has them: they skip the read-for-ownership of ordinary
// stores, and with it a third of the host memory traffic the fill adds next
// to the copy engine's own reads. The fence makes the stores visible before the
// piece is handed to the copy engine.
__attribute__((target("avx2"))) void copy_stream_avx2(char* d, const char* s, size_t len) {
  while (len && ((uintptr_t)d & 31)) {
    *d++ = *s++;
    --len;
  }
  for (; len >= 128; len -= 128, d += 128, s += 128) {
    const __m256i a = _mm256_loadu_si256((const __m256i*)s);
    const __m256i b = _mm256_loadu_si256((const __m256i*)(s + 32));
    const __m256i c = _mm256_loadu_si256((const __m256i*)(s + 64));
    const __m256i e = _mm256_loadu_si256((const __m256i*)(s + 96));
    _mm256_stream_si256((__m256i*)d, a);
    _mm256_stream_si256((__m256i*)(d + 32), b);
    _mm256_stream_si256((__m256i*)(d + 64), c);
    _mm256_stream_si256((__m256i*)(d + 96), e);
  }
  memcpy(d, s, len);
  _mm_sfence();
}

void copy_to_staging(void* dst, const void* src, size_t len) {
  static const bool avx2 = __builtin_cpu_supports("avx2");
  if (avx2) copy_stream_avx2((char*)dst, (const char*)src, len);
  else memcpy(dst, src, len);
}

// ---------------------------------------------------------------------------
// Mapped files.
// ---------------------------------------------------------------------------
struct MappedFile {
  std::string path;
  int fd = -1;
  const uint8_t* base = nullptr;
  uint64_t size = 0;
  ~MappedFile() {
    if (base) munmap(const_cast<uint8_t*>(base), size);
    if (fd >= 0) close(fd);
  }
};

// Opens and maps `path` read-only; the mapping lives as long as any holder
// (store.rs:131-133 keeps its Mmaps for the store's lifetime).
int map_file(const char* path, std::shared_ptr<MappedFile>* out) {
  auto f = std::make_shared<MappedFile>();
  f->path = path;
  f->fd = open(path, O_RDONLY | O_CLOEXEC);
  if (f->fd < 0) return sfail(LTXW_ERR_IO, "%s: %s", path, strerror(errno));
  struct stat sb;
  if (fstat(f->fd, &sb) != 0) return sfail(LTXW_ERR_IO, "%s: %s", path, strerror(errno));
  f->size = (uint64_t)sb.st_size;
  if (f->size > 0) {
    void* p = mmap(nullptr, f->size, PROT_READ, MAP_SHARED, f->fd, 0);
    if (p == MAP_FAILED) return sfail(LTXW_ERR_IO, "%s: mmap: %s", path, strerror(errno));
    f->base = (const uint8_t*)p;
  }
  *out = std::move(f);
  return LTXW_OK;
}

int parse_file(const MappedFile& f, st::Header* h) {
  std::string msg;
  if (st::parse(f.base, f.size, h, &msg) != st::OK)
    return sfail(LTXW_ERR_FORMAT, "%s: safetensors: %s", f.path.c_str(), msg.c_str());
  return LTXW_OK;
}

// ---------------------------------------------------------------------------
// Exact host widening of small tensors (scales, alpha, LoRA factors read on
// the host), per element type: src/store.rs:672-729, src/lora.rs:176-209.
// ---------------------------------------------------------------------------
float f_bits(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

float with_sign(uint32_t sign, float mag) {
  uint32_t u;
  memcpy(&u, &mag, 4);
  return f_bits(sign | u);
}

float e4m3fn_f32(uint8_t b) {  // src/fp8.rs:90-120
  if ((b & 0x7F) == 0x7F) return f_bits(0x7FC00000u);  // f32::NAN for both signs
  uint32_t sign = (uint32_t)(b & 0x80) << 24, e = (b >> 3) & 0xF, m = b & 7;
  if (e == 0) return with_sign(sign, std::ldexp((float)m, -9));  // exact
  return f_bits(sign | (e + 120) << 23 | m << 20);
}

float e5m2_f32(uint8_t b) {  // src/fp8.rs:127-158
  uint32_t sign = (uint32_t)(b & 0x80) << 24, e = (b >> 2) & 0x1F, m = b & 3;
  if (e == 31) return m ? f_bits(0x7FC00000u) : f_bits(sign | 0x7F800000u);
  if (e == 0) return with_sign(sign, std::ldexp((float)m, -16));
  return f_bits(sign | (e + 112) << 23 | m << 21);
}

float f16_f32(uint16_t h) {  // half's f16::to_f32: exact; NaN quiet, payload kept
  uint32_t sign = (uint32_t)(h & 0x8000) << 16, e = (h >> 10) & 0x1F, m = h & 0x3FF;
  if (e == 31) return f_bits(sign | (m ? 0x7FC00000u | m << 13 : 0x7F800000u));
  if (e == 0) return with_sign(sign, std::ldexp((float)m, -24));
  return f_bits(sign | (e + 112) << 23 | m << 13);
}

bool decodable(int32_t dt) {
  return dt == st::F32 || dt == st::F16 || dt == st::BF16 || dt == st::F8_E4M3 || dt == st::F8_E5M2;
}

// Little-endian, unaligned-safe.
void decode_host(const uint8_t* p, int32_t dt, uint64_t n, float* out) {
  for (uint64_t k = 0; k < n; ++k) {
    switch (dt) {
      case st::F8_E4M3: out[k] = e4m3fn_f32(p[k]); break;
      case st::F8_E5M2: out[k] = e5m2_f32(p[k]); break;
      case st::BF16: out[k] = f_bits((uint32_t)(p[2 * k] | p[2 * k + 1] << 8) << 16); break;
      case st::F16: out[k] = f16_f32((uint16_t)(p[2 * k] | p[2 * k + 1] << 8)); break;
      default: {
        uint32_t u;
        memcpy(&u, p + 4 * k, 4);
        out[k] = f_bits(u);
      }
    }
  }
}

// Base formats the device path takes (ltxw_format), or -1.
int device_format(int32_t dt) {
  switch (dt) {
    case st::F8_E4M3: return LTXW_FMT_E4M3FN;
    case st::F8_E5M2: return LTXW_FMT_E5M2;
    case st::BF16: return LTXW_FMT_BF16;
    case st::F16: return LTXW_FMT_F16;
    case st::F32: return LTXW_FMT_F32;
    default: return -1;
  }
}

// LoRA factor element types the device path takes (ltxw_factor_dtype); the
// store only merges decodable ones.
int factor_dtype(int32_t dt) {
  switch (dt) {
    case st::F32: return LTXW_FACTOR_F32;
    case st::F16: return LTXW_FACTOR_F16;
    case st::F8_E4M3: return LTXW_FACTOR_E4M3FN;
    case st::F8_E5M2: return LTXW_FACTOR_E5M2;
    default: return LTXW_FACTOR_BF16;
  }
}

uint64_t factor_size(int fdt) {
  return fdt == LTXW_FACTOR_F32 ? 4 : (fdt == LTXW_FACTOR_E4M3FN || fdt == LTXW_FACTOR_E5M2) ? 1 : 2;
}

uint64_t dim_or(const std::vector<uint64_t>& s, size_t i, uint64_t dflt) { return i < s.size() ? s[i] : dflt; }

// `usize_to_f32` (src/store.rs:745-750).
float rank_f32(uint64_t r) { return r > UINT32_MAX ? 3.40282347e38f : (float)(uint32_t)r; }

bool ends_with(const std::string& s, const std::string& t) {
  return s.size() >= t.size() && s.compare(s.size() - t.size(), t.size(), t) == 0;
}
bool starts_with(const std::string& s, const std::string& t) { return s.compare(0, t.size(), t) == 0; }

// ---------------------------------------------------------------------------
// Key rules (`KeyMap::apply_key`, src/key_map.rs:237-268).
// ---------------------------------------------------------------------------
struct Rule {
  int32_t kind;
  std::vector<std::string> s;
};

bool apply_key(const std::vector<Rule>& rules, std::string* key) {
  for (const Rule& r : rules) {
    switch (r.kind) {
      case LTXW_RULE_REQUIRE_ANY_PREFIX: {
        if (r.s.empty()) break;
        bool any = false;
        for (const auto& p : r.s) any = any || starts_with(*key, p);
        if (!any) return false;
        break;
      }
      case LTXW_RULE_REPLACE: {
        const std::string& f = r.s[0];
        if (f.empty() || key->find(f) == std::string::npos) {
          // An empty pattern matches before every character and at the end
          // (Rust's str::replace), so the replacement is inserted there.
          if (f.empty()) {
            std::string out = r.s[1];
            size_t i = 0;
            while (i < key->size()) {
              // step over one UTF-8 character
              size_t len = 1;
              unsigned char c = (unsigned char)(*key)[i];
              if (c >= 0xF0) len = 4; else if (c >= 0xE0) len = 3; else if (c >= 0xC0) len = 2;
              out.append(*key, i, len);
              out += r.s[1];
              i += len;
            }
            *key = out;
          }
          break;
        }
        std::string out;
        size_t pos = 0, hit;
        while ((hit = key->find(f, pos)) != std::string::npos) {
          out.append(*key, pos, hit - pos);
          out += r.s[1];
          pos = hit + f.size();
        }
        out.append(*key, pos, std::string::npos);
        *key = out;
        break;
      }
      case LTXW_RULE_RENAME_EXACT:
        if (starts_with(*key, r.s[0])) *key = r.s[1] + key->substr(r.s[0].size());
        break;
      case LTXW_RULE_DROP_PREFIX:
        if (starts_with(*key, r.s[0])) return false;
        break;
      case LTXW_RULE_DROP_SUFFIX:
        if (ends_with(*key, r.s[0])) return false;
        break;
      default: break;
    }
  }
  return true;
}

}  // namespace

// ---------------------------------------------------------------------------
// Objects behind the opaque handles.
// ---------------------------------------------------------------------------
struct LoraData {
  std::shared_ptr<MappedFile> file;
  std::unordered_map<std::string, st::TensorInfo> tensors;  // offsets absolute in the file
  std::vector<std::string> names;                           // sorted
  std::map<std::string, std::string> metadata;
};

struct ltxw_lora_file {
  std::shared_ptr<LoraData> d;
};

struct ltxw_merge_report {
  std::vector<std::string> matched, unmatched;
};

namespace {

// Value transform of an entry made at open by the video-decoder key map
// (store.rs:217-419); the reference materialises these eagerly as host f32.
enum Xform : int32_t {
  XF_NONE = 0,
  XF_SPLIT = 1,  // QKV split part: the parent's bytes, scale as fma(s, v, 0) when has_scale
  XF_GATE = 2,   // gate fold: (v [* scale]) * gate, plain multiplies
  XF_OWNED = 3,  // host-owned f32 bytes (synthesised zero type_emb)
};

struct Entry {
  int32_t dtype;      // as reported (F32 for transformed entries, like the reference)
  std::vector<uint64_t> shape;
  uint32_t file;
  uint64_t start, end;  // absolute in the file (unused for XF_OWNED)
  uint64_t numel;
  int32_t src_dtype;   // element type of the stored bytes
  int32_t xform = XF_NONE;
  bool has_scale = false;
  float scale = 1.0f;  // XF_SPLIT / XF_GATE
  float gate = 1.0f;   // XF_GATE
  std::shared_ptr<std::vector<uint8_t>> owned;  // XF_OWNED
};

// One merged low-rank delta (src/store.rs:751-763), kept as the adapter's
// own bytes: the LoRA file stays mapped while the store holds the delta.
struct Delta {
  std::shared_ptr<LoraData> lora;
  std::string key_a, key_b;
  uint64_t rank, out, in;
  float coeff;
};

}  // namespace

struct ltxw_store {
  std::vector<std::shared_ptr<MappedFile>> files;
  std::unordered_map<std::string, Entry> entries;
  std::unordered_set<std::string> scale_keys;
  std::map<std::string, std::string> metadata;
  std::unordered_map<std::string, std::vector<Delta>> deltas;
  std::vector<std::string> visible;  // sorted
};

namespace {

int tensor_info_out(int32_t dtype, const std::vector<uint64_t>& shape, int32_t* dt, int32_t* ndim,
                    int64_t* dims, int32_t max_dims) {
  if (dt) *dt = dtype;
  if (ndim) *ndim = (int32_t)shape.size();
  if (dims)
    for (int32_t k = 0; k < max_dims && k < (int32_t)shape.size(); ++k) dims[k] = (int64_t)shape[(size_t)k];
  return LTXW_OK;
}

// ---------------------------------------------------------------------------
// Materialisation plan of one key.
// ---------------------------------------------------------------------------
constexpr uint64_t kAlign = 256;
uint64_t align_up(uint64_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

struct Plan {
  const std::string* key;
  const Entry* e;
  const uint8_t* wsrc;  // mapped weight bytes
  void* out;
  int fmt, esize;
  uint64_t rows, cols, numel;
  int scale_mode;
  std::vector<float> scales;
  std::vector<const Delta*> deltas;
  std::vector<const uint8_t*> fb, fa;  // mapped factor bytes, per delta
  std::vector<int> fdt;                // ltxw_factor_dtype, per delta
  ltxw::DescEx ex;                     // gate-fold extras
  // Offsets inside the batch's device slot.
  uint64_t off_w, off_s, bytes;
  std::vector<uint64_t> off_b, off_a;
};

const uint8_t* entry_bytes(const ltxw_store* s, const Entry& e);

int make_plan(const ltxw_store* s, const std::string& key, uint32_t flags, int out_dtype, void* out, Plan* p) {
  auto it = s->entries.find(key);
  if (it == s->entries.end()) return sfail(LTXW_ERR_MISSING_KEY, "missing key: \"%s\"", key.c_str());
  const Entry& e = it->second;
  p->key = &it->first;
  p->e = &e;
  p->wsrc = entry_bytes(s, e);
  p->out = out;
  p->fmt = device_format(e.src_dtype);
  if (p->fmt < 0)
    return sfail(LTXW_ERR_UNSUPPORTED, "unsupported dtype %s for key \"%s\"", st::dtype_name(e.src_dtype), key.c_str());
  p->esize = ltxw::format_bytes(p->fmt);
  p->numel = e.numel;
  p->rows = e.shape.empty() ? 1 : e.shape[0];
  p->cols = p->rows ? p->numel / p->rows : 0;
  if (p->numel && !out) return sfail(LTXW_ERR_INVALID_ARG, "null output buffer for key \"%s\"", key.c_str());
  (void)out_dtype;

  // FP8 scale sibling (store.rs:498-508), or the scale an open-time
  // transform carried over from its source.
  p->scale_mode = LTXW_SCALE_NONE;
  if (e.xform == XF_SPLIT || e.xform == XF_GATE) {
    if (e.has_scale) {
      p->scales.assign(1, e.scale);
      p->scale_mode = LTXW_SCALE_TENSOR;
    }
    if (e.xform == XF_GATE) {
      p->ex.plain_scale = 1;
      p->ex.has_post = 1;
      p->ex.post_mul = e.gate;
    }
  } else if (st::is_fp8(e.dtype)) {
    auto sc = s->entries.find(key + "_scale");
    if (sc != s->entries.end()) {
      const Entry& se = sc->second;
      if (!decodable(se.dtype))
        return sfail(LTXW_ERR_UNSUPPORTED, "unsupported dtype %s for key \"%s_scale\"", st::dtype_name(se.dtype),
                     key.c_str());
      const uint8_t* base = s->files[se.file]->base + se.start;
      const bool rows = !(flags & LTXW_MAT_SCALE_FIRST) && e.shape.size() >= 2 && e.shape[0] > 1 &&
                        se.numel == e.shape[0];
      if (rows) {
        p->scales.resize(se.numel);
        decode_host(base, se.dtype, se.numel, p->scales.data());
        p->scale_mode = LTXW_SCALE_ROW;
      } else {
        // decode_scalar_f32 (store.rs:732-735): element 0, or 1.0 when empty.
        float v = 1.0f;
        if (se.numel) decode_host(base, se.dtype, 1, &v);
        p->scales.assign(1, v);
        p->scale_mode = LTXW_SCALE_TENSOR;
      }
    }
  }

  // Merged deltas (store.rs:510-515, add_to's checks at :767-779).
  auto dl = s->deltas.find(key);
  if (dl != s->deltas.end()) {
    for (const Delta& d : dl->second) {
      const uint64_t out_in = d.out * d.in;
      if ((d.in && out_in / d.in != d.out) || out_in != p->numel || d.in == 0 || d.rank == 0)
        return sfail(LTXW_ERR_LORA_SHAPE, "LoRA shape mismatch for key \"%s\"", key.c_str());
      const st::TensorInfo& ta = d.lora->tensors.at(d.key_a);
      const st::TensorInfo& tb = d.lora->tensors.at(d.key_b);
      if (ta.dtype != tb.dtype)
        return sfail(LTXW_ERR_UNSUPPORTED, "LoRA factors of \"%s\" mix %s (B) and %s (A)", key.c_str(),
                     st::dtype_name(tb.dtype), st::dtype_name(ta.dtype));
      if (d.rank > (1u << 20))
        return sfail(LTXW_ERR_UNSUPPORTED, "LoRA rank %llu of \"%s\" is too large", (unsigned long long)d.rank,
                     key.c_str());
      p->fb.push_back(d.lora->file->base + tb.begin);
      p->fa.push_back(d.lora->file->base + ta.begin);
      p->fdt.push_back(factor_dtype(ta.dtype));
      p->deltas.push_back(&d);
    }
    if (!p->deltas.empty()) {
      p->rows = p->deltas[0]->out;
      p->cols = p->deltas[0]->in;
    }
  }

  // Device layout of the payload: weight, scales, then (B, A) per delta.
  uint64_t off = 0;
  p->off_w = off;
  off = align_up(off + p->numel * (uint64_t)p->esize);
  p->off_s = off;
  off = align_up(off + 4 * (uint64_t)p->scales.size());
  p->off_b.resize(p->deltas.size());
  p->off_a.resize(p->deltas.size());
  for (size_t l = 0; l < p->deltas.size(); ++l) {
    const Delta& d = *p->deltas[l];
    const uint64_t fs = factor_size(p->fdt[l]);
    p->off_b[l] = off;
    off = align_up(off + fs * d.out * d.rank);
    p->off_a[l] = off;
    off = align_up(off + fs * d.rank * d.in);
  }
  p->bytes = off;
  return LTXW_OK;
}


// One host->device copy of the pipeline: at most one staging buffer.
// One mapped source range and where it lands in its batch's device slot.
struct Seg {
  const uint8_t* src;
  uint64_t len;
  uint64_t dst;  // offset in the batch's device slot
};

// A staging slot's worth of a batch's device-slot layout: bytes
// [dst, dst + len) of the slot, filled from the segments [seg_lo, seg_hi)
// that overlap it. Small segments (scales, LoRA factors) share a piece with
// their neighbours, so a batch goes out in ceil(bytes / slot) copies rather
// than one or more per segment.
struct Piece {
  uint64_t dst;
  uint64_t len;
  size_t seg_lo, seg_hi;
};

struct Batch {
  size_t first_plan, n_plans;
  size_t first_piece, end_piece;
};

// Creates the three-slot device ring (or grows it to `need` bytes per slot).
int ensure_ring(ltxw_ctx* ctx, uint64_t need) {
  hipError_t he;
  if (ctx->ring_free.empty()) {
    for (int k = 0; k < 3; ++k) {
      hipEvent_t a = nullptr, b = nullptr;
      if ((he = hipEventCreateWithFlags(&a, hipEventDisableTiming)) != hipSuccess)
        return sfail(LTXW_ERR_HIP, "ring event: %s", hipGetErrorString(he));
      ctx->ring_free.push_back(a);
      if ((he = hipEventCreateWithFlags(&b, hipEventDisableTiming)) != hipSuccess)
        return sfail(LTXW_ERR_HIP, "ring event: %s", hipGetErrorString(he));
      ctx->ring_ready.push_back(b);
    }
  }
  if (!ctx->ring.empty() && ctx->ring_bytes >= need) return LTXW_OK;
  if (!ctx->ring.empty()) {
    if ((he = hipStreamSynchronize(ctx->copy)) != hipSuccess || (he = hipStreamSynchronize(ctx->compute)) != hipSuccess)
      return sfail(LTXW_ERR_HIP, "device ring resize: %s", hipGetErrorString(he));
    for (void* q : ctx->ring) (void)hipFree(q);
    ctx->ring.clear();
    ctx->ring_bytes = 0;
  }
  for (int k = 0; k < 3; ++k) {
    void* q = nullptr;
    if (hipMalloc(&q, need) != hipSuccess) {
      (void)hipGetLastError();
      for (void* x : ctx->ring) (void)hipFree(x);
      ctx->ring.clear();
      return sfail(LTXW_ERR_OOM, "device staging ring of 3 x %llu bytes", (unsigned long long)need);
    }
    ctx->ring.push_back(q);
  }
  ctx->ring_bytes = need;
  for (int k = 0; k < 3; ++k)  // nothing reads the fresh slots
    if ((he = hipEventRecord(ctx->ring_free[(size_t)k], ctx->compute)) != hipSuccess)
      return sfail(LTXW_ERR_HIP, "ring event record: %s", hipGetErrorString(he));
  return LTXW_OK;
}

// Grows the context's device scratch (the chained passes' f32 accumulator)
// to `need` bytes; work already queued may still use the old buffer.
int ensure_tmp(ltxw_ctx* ctx, uint64_t need) {
  if (need <= ctx->tmp_bytes) return LTXW_OK;
  hipError_t he;
  if (ctx->tmp) {
    if ((he = hipStreamSynchronize(ctx->compute)) != hipSuccess)
      return sfail(LTXW_ERR_HIP, "scratch resize: %s", hipGetErrorString(he));
    (void)hipFree(ctx->tmp);
    ctx->tmp = nullptr;
    ctx->tmp_bytes = 0;
  }
  if (hipMalloc(&ctx->tmp, need) != hipSuccess) {
    (void)hipGetLastError();
    ctx->tmp = nullptr;
    return sfail(LTXW_ERR_OOM, "device scratch of %llu bytes", (unsigned long long)need);
  }
  ctx->tmp_bytes = need;
  return LTXW_OK;
}

// Host copy granularity: a staging slot is filled in sub-chunks of this size
// by whichever host threads are free, so one slot fills at the threads'
// combined rate.
constexpr uint64_t kSubChunk = 8ull << 20;
// Largest single host -> device copy: neighbouring filled slots that continue
// one tensor segment go out as one copy (fewer, larger DMA transfers).
constexpr uint64_t kMaxRun = 256ull << 20;

// Staged pipeline over `plans` (each with numel > 0):
//   host threads: mapped bytes -> pinned staging slot (slot p % S for piece p,
//                 refilled once the copy of piece p - S has completed), in
//                 sub-chunks claimed in order;
//   this thread:  filled slots -> device ring slot on the copy stream, in
//                 piece order; after a batch's last piece, the compute stream
//                 waits for the copies and runs the batch's kernels.
// Host reads finish before return; device work completes in stream order.
int run_pipeline(ltxw_ctx* ctx, std::vector<Plan>& plans, int out_dtype, uint32_t flags) {
  if (plans.empty()) return LTXW_OK;
  hipError_t he;
  if ((he = hipSetDevice(ctx->device)) != hipSuccess)
    return sfail(LTXW_ERR_HIP, "hipSetDevice: %s", hipGetErrorString(he));
  if (int rc = ltxw::ensure_staging(ctx)) return sfail(rc, "%s", ctx->err.c_str());
  uint64_t need = 512ull << 20;
  for (const Plan& p : plans) need = std::max(need, p.bytes);
  if (int rc = ensure_ring(ctx, need)) return rc;
  // f32 accumulator of keys with more than LTXW_MAX_LORAS deltas and bf16
  // output (their passes run in stream order, so one buffer serves all).
  uint64_t tmp_need = 0;
  if (out_dtype == LTXW_OUT_BF16)
    for (const Plan& p : plans)
      if (p.deltas.size() > (size_t)LTXW_MAX_LORAS) tmp_need = std::max(tmp_need, 4 * p.numel);
  if (int rc = ensure_tmp(ctx, tmp_need)) return rc;
  const uint64_t stage = ctx->stage_bytes;
  const size_t S = ctx->stage.size(), R = ctx->ring.size();

  std::vector<Batch> batches;
  std::vector<Seg> segs;
  std::vector<Piece> pieces;
  auto add = [&](const void* src, uint64_t len, uint64_t dst) {
    if (len) segs.push_back({(const uint8_t*)src, len, dst});
  };
  for (size_t k = 0; k < plans.size();) {
    Batch b{k, 0, pieces.size(), 0};
    const size_t seg0 = segs.size();
    uint64_t used = 0;
    while (k < plans.size() && (b.n_plans == 0 || used + plans[k].bytes <= ctx->ring_bytes)) {
      Plan& p = plans[k];
      p.off_w += used;
      p.off_s += used;
      for (size_t l = 0; l < p.deltas.size(); ++l) {
        p.off_b[l] += used;
        p.off_a[l] += used;
      }
      add(p.wsrc, p.numel * (uint64_t)p.esize, p.off_w);
      if (!p.scales.empty()) add(p.scales.data(), 4 * p.scales.size(), p.off_s);
      for (size_t l = 0; l < p.deltas.size(); ++l) {
        const Delta& d = *p.deltas[l];
        const uint64_t fs = factor_size(p.fdt[l]);
        add(p.fb[l], fs * d.out * d.rank, p.off_b[l]);
        add(p.fa[l], fs * d.rank * d.in, p.off_a[l]);
      }
      used += p.bytes;
      ++b.n_plans;
      ++k;
    }
    // Cut the batch's layout into staging-slot pieces; the padding between
    // segments travels as it is (nothing reads it).
    std::sort(segs.begin() + (ptrdiff_t)seg0, segs.end(), [](const Seg& x, const Seg& y) { return x.dst < y.dst; });
    size_t lo = seg0;
    for (uint64_t o = 0; o < used; o += stage) {
      const uint64_t len = std::min(stage, used - o);
      while (lo < segs.size() && segs[lo].dst + segs[lo].len <= o) ++lo;
      size_t hi = lo;
      while (hi < segs.size() && segs[hi].dst < o + len) ++hi;
      pieces.push_back({o, len, lo, hi});
    }
    b.end_piece = pieces.size();
    batches.push_back(b);
  }

  // Host copy work: (piece, offset) sub-chunks in piece order.
  std::vector<std::pair<size_t, uint64_t>> chunks;
  std::vector<std::atomic<int>> remaining(pieces.size());
  for (size_t p = 0; p < pieces.size(); ++p) {
    int n = 0;
    for (uint64_t o = 0; o < pieces[p].len; o += kSubChunk, ++n) chunks.push_back({p, o});
    remaining[p].store(n);
  }

  // Shared state of the host copy threads.
  std::mutex mu;
  std::condition_variable cv;
  std::vector<uint8_t> filled(pieces.size(), 0);
  size_t recorded = 0;  // pieces whose copy-done event has been recorded
  bool abort = false;
  std::string worker_err;
  std::atomic<size_t> next{0};
  const int device = ctx->device;

  auto worker = [&]() {
    (void)hipSetDevice(device);
    for (;;) {
      const size_t c = next.fetch_add(1);
      if (c >= chunks.size()) return;
      const size_t p = chunks[c].first;
      const uint64_t off = chunks[c].second, len = std::min(kSubChunk, pieces[p].len - off);
      const size_t s = p % S;
      {
        std::unique_lock<std::mutex> lk(mu);
        cv.wait(lk, [&] { return abort || p < recorded + S; });
        if (abort) return;
      }
      // The slot's previous copy (piece p - S, or an earlier call's) is done.
      hipError_t e = hipEventSynchronize(ctx->stage_done[s]);
      if (e != hipSuccess) {
        std::lock_guard<std::mutex> lk(mu);
        abort = true;
        worker_err = std::string("staging wait: ") + hipGetErrorString(e);
        cv.notify_all();
        return;
      }
      const Piece& pc = pieces[p];
      const uint64_t c0 = pc.dst + off, c1 = c0 + len;
      for (size_t g = pc.seg_lo; g < pc.seg_hi; ++g) {
        const Seg& sg = segs[g];
        const uint64_t s0 = std::max(c0, sg.dst), s1 = std::min(c1, sg.dst + sg.len);
        if (s0 < s1) copy_to_staging((char*)ctx->stage[s] + (s0 - pc.dst), sg.src + (s0 - sg.dst), s1 - s0);
      }
      if (remaining[p].fetch_sub(1) == 1) {
        {
          std::lock_guard<std::mutex> lk(mu);
          filled[p] = 1;
        }
        cv.notify_all();
      }
    }
  };
  const int nt = std::max(1, std::min<int>(ctx->host_threads, (int)chunks.size()));
  std::vector<std::thread> threads;
  threads.reserve((size_t)nt);
  for (int t = 0; t < nt; ++t) threads.emplace_back(worker);

  int rc = LTXW_OK;
  std::vector<ltxw_tensor_desc> descs;
  std::vector<ltxw::DescEx> exs;
  for (size_t bi = 0; bi < batches.size() && rc == LTXW_OK; ++bi) {
    const Batch& b = batches[bi];
    const size_t slot = bi % R;
    char* base = (char*)ctx->ring[slot];
    // Copies into the slot wait for the kernels that last read it.
    if ((he = hipStreamWaitEvent(ctx->copy, ctx->ring_free[slot], 0)) != hipSuccess) {
      rc = sfail(LTXW_ERR_HIP, "copy stream wait: %s", hipGetErrorString(he));
      break;
    }
    for (size_t p = b.first_piece; p < b.end_piece;) {
      // Copy [p, q): piece p and the filled pieces that continue it in both
      // the staging block (no wrap) and the device slot.
      size_t q = p + 1;
      uint64_t len = pieces[p].len;
      {
        std::unique_lock<std::mutex> lk(mu);
        cv.wait(lk, [&] { return abort || filled[p]; });
        if (abort) {
          rc = sfail(LTXW_ERR_HIP, "%s", worker_err.c_str());
          break;
        }
        while (q < b.end_piece && filled[q] && q % S != 0 && pieces[q - 1].len == stage &&
               pieces[q].dst == pieces[q - 1].dst + stage && len + pieces[q].len <= kMaxRun) {
          len += pieces[q].len;
          ++q;
        }
      }
      if ((he = hipMemcpyAsync(base + pieces[p].dst, ctx->stage[p % S], len, hipMemcpyHostToDevice, ctx->copy)) !=
          hipSuccess) {
        rc = sfail(LTXW_ERR_HIP, "staged copy: %s", hipGetErrorString(he));
        break;
      }
      for (size_t k = p; k < q && rc == LTXW_OK; ++k)
        if ((he = hipEventRecord(ctx->stage_done[k % S], ctx->copy)) != hipSuccess)
          rc = sfail(LTXW_ERR_HIP, "staged copy event: %s", hipGetErrorString(he));
      if (rc) break;
      {
        std::lock_guard<std::mutex> lk(mu);
        recorded = q;
      }
      cv.notify_all();
      p = q;
    }
    if (rc) break;
    if ((he = hipEventRecord(ctx->ring_ready[slot], ctx->copy)) != hipSuccess ||
        (he = hipStreamWaitEvent(ctx->compute, ctx->ring_ready[slot], 0)) != hipSuccess) {
      rc = sfail(LTXW_ERR_HIP, "batch hand-off: %s", hipGetErrorString(he));
      break;
    }
    descs.clear();
    exs.clear();
    for (size_t k = b.first_plan; k < b.first_plan + b.n_plans; ++k) {
      const Plan& p = plans[k];
      const size_t nd = p.deltas.size();
      // Up to LTXW_MAX_LORAS deltas: one descriptor. More: passes of up to
      // LTXW_MAX_LORAS deltas each, in merge order and in the reference's
      // operation order, through an f32 accumulator (the output itself for
      // f32, else the context's scratch): each pass continues the previous
      // pass's per-element FMA chain, so the result equals one long chain
      // (store.rs:510-515).
      const bool chained = nd > (size_t)LTXW_MAX_LORAS;
      void* acc = out_dtype == LTXW_OUT_F32 ? p.out : ctx->tmp;
      for (size_t l0 = 0; l0 == 0 || l0 < nd; l0 += LTXW_MAX_LORAS) {
        const size_t l1 = std::min(nd, l0 + (size_t)LTXW_MAX_LORAS);
        const bool first = l0 == 0, last = l1 == nd;
        ltxw_tensor_desc d{};
        d.w = first ? (const uint8_t*)(base + p.off_w) : (const uint8_t*)acc;
        d.out = last ? p.out : acc;
        d.scales = (first && !p.scales.empty()) ? (const float*)(base + p.off_s) : nullptr;
        d.rows = (int64_t)p.rows;
        d.cols = (int64_t)p.cols;
        d.fmt = first ? p.fmt : LTXW_FMT_F32;
        d.scale_mode = first ? p.scale_mode : LTXW_SCALE_NONE;
        d.out_dtype = last ? out_dtype : LTXW_OUT_F32;
        d.n_loras = (int32_t)(l1 - l0);
        d.flags = (chained || (flags & LTXW_MAT_EXACT)) ? LTXW_DESC_EXACT : 0;
        for (size_t l = l0; l < l1; ++l)
          d.loras[l - l0] = {base + p.off_b[l], base + p.off_a[l], (int32_t)p.deltas[l]->rank, p.deltas[l]->coeff,
                             p.fdt[l], 0};
        ltxw::DescEx ex = first ? p.ex : ltxw::DescEx{};
        // FP8 sources keep the reference's one NaN through every pass.
        ex.canon_nan = chained && ltxw::format_bytes(p.fmt) == 1 ? 1 : 0;
        descs.push_back(d);
        exs.push_back(ex);
      }
    }
    if (int r2 = ltxw::run_descs(ctx, descs.data(), (int)descs.size(), exs.data())) {
      rc = sfail(r2, "%s", ctx->err.c_str());
      break;
    }
    if ((he = hipEventRecord(ctx->ring_free[slot], ctx->compute)) != hipSuccess) {
      rc = sfail(LTXW_ERR_HIP, "ring event record: %s", hipGetErrorString(he));
      break;
    }
  }
  {
    std::lock_guard<std::mutex> lk(mu);
    if (rc) abort = true;
  }
  cv.notify_all();
  for (auto& t : threads) t.join();
  return rc;
}

int check_flags(uint32_t flags) {
  const uint32_t all = LTXW_MAT_SCALE_FIRST | LTXW_MAT_EXACT | LTXW_MAT_ROW_SCALES | LTXW_MAT_MFMA;
  if (flags & ~all) return sfail(LTXW_ERR_INVALID_ARG, "unknown flags 0x%x", flags);
  if ((flags & LTXW_MAT_SCALE_FIRST) && (flags & LTXW_MAT_ROW_SCALES))
    return sfail(LTXW_ERR_INVALID_ARG, "LTXW_MAT_SCALE_FIRST and LTXW_MAT_ROW_SCALES together");
  if ((flags & LTXW_MAT_EXACT) && (flags & LTXW_MAT_MFMA))
    return sfail(LTXW_ERR_INVALID_ARG, "LTXW_MAT_EXACT and LTXW_MAT_MFMA together");
  return LTXW_OK;
}

int materialize(ltxw_store* s, ltxw_ctx* ctx, const char* const* keys, int64_t n_keys, int32_t out_dtype,
                uint32_t flags, void* const* outs) {
  if (!s || !ctx) return sfail(LTXW_ERR_INVALID_ARG, "null store or context");
  if (n_keys < 0 || (n_keys > 0 && (!keys || !outs)))
    return sfail(LTXW_ERR_INVALID_ARG, "invalid key or output array");
  if (out_dtype != LTXW_OUT_BF16 && out_dtype != LTXW_OUT_F32)
    return sfail(LTXW_ERR_INVALID_ARG, "invalid output dtype %d", out_dtype);
  if (int rc = check_flags(flags)) return rc;
  // Per-row scales are materialize's default; the deltas run in the
  // reference's operation order unless the MFMA kernels are asked for (the
  // host -> HBM copies hide either).
  if (!(flags & LTXW_MAT_MFMA)) flags |= LTXW_MAT_EXACT;
  flags &= ~(LTXW_MAT_ROW_SCALES | LTXW_MAT_MFMA);
  // Resolve and check every key before any work is queued.
  std::vector<Plan> plans;
  plans.reserve((size_t)n_keys);
  for (int64_t k = 0; k < n_keys; ++k) {
    if (!keys[k]) return sfail(LTXW_ERR_INVALID_ARG, "null key at index %lld", (long long)k);
    Plan p{};
    if (int rc = make_plan(s, keys[k], flags, out_dtype, outs[k], &p)) return rc;
    if (p.numel) plans.push_back(std::move(p));
  }
  return run_pipeline(ctx, plans, out_dtype, flags);
}

}  // namespace

// ---------------------------------------------------------------------------
// Open-time value transforms of the video-decoder key map.
// ---------------------------------------------------------------------------
namespace {

// Gate-fold targets and their gates (key_map.rs:276-283).
const char* const kGateTargets[][2] = {
    {".attn.proj.weight", ".gate_msa"},   {".attn.proj.bias", ".gate_msa"},
    {".mlp.w_down.weight", ".gate_mlp"},  {".mlp.w_down.bias", ".gate_mlp"},
    {".context_proj.weight", ".gate_ctx"}, {".context_proj.bias", ".gate_ctx"},
};
const char* const kGateSuffixes[] = {".gate_msa", ".gate_mlp", ".gate_ctx"};

const uint8_t* entry_bytes(const ltxw_store* s, const Entry& e) {
  return e.xform == XF_OWNED ? e.owned->data() : s->files[e.file]->base + e.start;
}

// decode_scalar_f32 (store.rs:732-735): element 0, or 1.0 when empty.
int scalar_of(const ltxw_store* s, const std::string& key, const Entry& e, float* v) {
  if (!decodable(e.src_dtype))
    return sfail(LTXW_ERR_UNSUPPORTED, "unsupported dtype %s for key \"%s\"", st::dtype_name(e.src_dtype), key.c_str());
  *v = 1.0f;
  if (e.numel) decode_host(entry_bytes(s, e), e.src_dtype, 1, v);
  return LTXW_OK;
}

// store.rs:217-293. Gates must be scalars; every target with a gate becomes
// f32 (v [* scale]) * gate, computed on the device at materialisation; the
// target's scale sibling and the gate entries go away.
int apply_gate_fold(ltxw_store* s) {
  std::vector<std::string> gate_keys;
  for (const auto& kv : s->entries)
    for (const char* suf : kGateSuffixes)
      if (ends_with(kv.first, suf)) gate_keys.push_back(kv.first);
  std::unordered_map<std::string, float> gates;
  for (const std::string& gk : gate_keys) {
    const Entry& e = s->entries.at(gk);
    const bool scalar = e.shape.empty() || (e.shape.size() == 1 && e.shape[0] == 1);
    if (!scalar) {
      std::string shp;
      for (size_t k = 0; k < e.shape.size(); ++k) shp += (k ? ", " : "") + std::to_string(e.shape[k]);
      return sfail(LTXW_ERR_GATE_NOT_SCALAR, "gate fold: expected scalar gate for key \"%s\", got shape [%s]",
                   gk.c_str(), shp.c_str());
    }
    float g;
    if (int rc = scalar_of(s, gk, e, &g)) return rc;
    gates[gk] = g;
  }
  std::vector<std::string> params;
  for (const auto& kv : s->entries) params.push_back(kv.first);
  for (const std::string& pk : params) {
    std::string gk;
    for (const auto& t : kGateTargets)
      if (ends_with(pk, t[0])) {
        gk = pk.substr(0, pk.size() - strlen(t[0])) + t[1];
        break;
      }
    if (gk.empty() || !gates.count(gk)) continue;
    Entry& e = s->entries.at(pk);
    if (!decodable(e.src_dtype) || e.xform != XF_NONE)
      return sfail(LTXW_ERR_UNSUPPORTED, "unsupported dtype %s for key \"%s\"", st::dtype_name(e.src_dtype),
                   pk.c_str());
    if (st::is_fp8(e.src_dtype)) {
      const std::string sk = pk + "_scale";
      auto si = s->entries.find(sk);
      if (si != s->entries.end()) {
        float sc;
        if (int rc = scalar_of(s, sk, si->second, &sc)) return rc;
        e.has_scale = true;
        e.scale = sc;
      }
      s->entries.erase(sk);
      s->scale_keys.erase(sk);
    }
    e.xform = XF_GATE;
    e.gate = gates[gk];
    e.dtype = st::F32;
  }
  for (const std::string& gk : gate_keys) s->entries.erase(gk);
  return LTXW_OK;
}

// store.rs:302-390. `P.qkv.{weight,bias}` with leading dim 3d becomes
// P.to_q / P.to_k / P.to_v of leading dim d: each a contiguous third of the
// parent's bytes, scaled (FP8) as the parent would be, reported as f32.
int apply_qkv_split(ltxw_store* s) {
  std::vector<std::string> keys;
  for (const auto& kv : s->entries)
    if (ends_with(kv.first, ".qkv.weight") || ends_with(kv.first, ".qkv.bias")) keys.push_back(kv.first);
  std::sort(keys.begin(), keys.end());
  for (const std::string& qk : keys) {
    const Entry parent = s->entries.at(qk);
    const uint64_t leading = parent.shape.empty() ? 0 : parent.shape[0];
    if (leading % 3 != 0)
      return sfail(LTXW_ERR_QKV_SPLIT_DIM, "QKV split: leading dim %llu for key \"%s\" is not divisible by 3",
                   (unsigned long long)leading, qk.c_str());
    if (!decodable(parent.src_dtype) || parent.xform != XF_NONE)
      return sfail(LTXW_ERR_UNSUPPORTED, "unsupported dtype %s for key \"%s\"", st::dtype_name(parent.src_dtype),
                   qk.c_str());
    bool has_scale = false;
    float sc = 1.0f;
    const std::string sk = qk + "_scale";
    if (st::is_fp8(parent.src_dtype)) {
      auto si = s->entries.find(sk);
      if (si != s->entries.end()) {
        if (int rc = scalar_of(s, sk, si->second, &sc)) return rc;
        has_scale = true;
      }
    }
    const uint64_t per = parent.numel / 3;
    const uint64_t esize = (uint64_t)st::dtype_bits(parent.src_dtype) / 8;
    const bool weight = ends_with(qk, ".weight");
    const std::string base = qk.substr(0, qk.rfind(".qkv."));
    const char* parts[3] = {".to_q.", ".to_k.", ".to_v."};
    for (int k = 0; k < 3; ++k) {
      const std::string name = base + parts[k] + (weight ? "weight" : "bias");
      if (s->entries.count(name)) return sfail(LTXW_ERR_DUPLICATE_KEY, "duplicate key \"%s\"", name.c_str());
      Entry e = parent;
      if (!e.shape.empty()) e.shape[0] = leading / 3;
      e.numel = per;
      e.start = parent.start + (uint64_t)k * per * esize;
      e.end = e.start + per * esize;
      e.xform = XF_SPLIT;
      e.has_scale = has_scale;
      e.scale = sc;
      e.dtype = st::F32;
      s->entries.emplace(name, std::move(e));
    }
    s->entries.erase(qk);
    s->entries.erase(sk);
    s->scale_keys.erase(sk);
  }
  return LTXW_OK;
}

// store.rs:398-419: a zero f32 `type_emb` of conv_in.weight's in-channels
// when the checkpoint has none.
void apply_zero_type_emb(ltxw_store* s) {
  if (s->entries.count("type_emb")) return;
  auto it = s->entries.find("conv_in.weight");
  if (it == s->entries.end() || it->second.shape.size() < 2 || it->second.shape[1] == 0) return;
  const uint64_t n = it->second.shape[1];
  Entry e{st::F32, {n}, 0, 0, 0, n, st::F32};
  e.xform = XF_OWNED;
  e.owned = std::make_shared<std::vector<uint8_t>>(4 * n, 0);
  s->entries.emplace("type_emb", std::move(e));
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI.
// ---------------------------------------------------------------------------
extern "C" {

const char* ltxw_store_last_error(void) { return g_err.c_str(); }

int ltxw_store_open(const char* const* paths, int n_paths, const ltxw_key_rule* rules, int n_rules,
                    ltxw_store** out) {
  if (!out) return sfail(LTXW_ERR_INVALID_ARG, "null output pointer");
  *out = nullptr;
  if (n_paths < 0 || (n_paths > 0 && !paths) || n_rules < 0 || (n_rules > 0 && !rules))
    return sfail(LTXW_ERR_INVALID_ARG, "invalid path or rule array");
  std::vector<Rule> rs;
  bool want_split = false, want_fold = false, want_type_emb = false;
  for (int k = 0; k < n_rules; ++k) {
    const ltxw_key_rule& r = rules[k];
    int want = -1;
    switch (r.kind) {
      case LTXW_RULE_REQUIRE_ANY_PREFIX: want = -2; break;
      case LTXW_RULE_REPLACE:
      case LTXW_RULE_RENAME_EXACT: want = 2; break;
      case LTXW_RULE_DROP_PREFIX:
      case LTXW_RULE_DROP_SUFFIX: want = 1; break;
      case LTXW_RULE_SPLIT_QKV: want_split = true; want = 0; break;
      case LTXW_RULE_FOLD_GATES: want_fold = true; want = 0; break;
      case LTXW_RULE_SYNTH_ZERO_TYPE_EMB: want_type_emb = true; want = 0; break;
      default: return sfail(LTXW_ERR_INVALID_ARG, "unknown key rule kind %d", r.kind);
    }
    if (r.n < 0 || (want >= 0 && r.n != want) || (r.n > 0 && !r.strs))
      return sfail(LTXW_ERR_INVALID_ARG, "key rule %d: kind %d takes %d strings, got %d", k, r.kind, want, r.n);
    Rule x{r.kind, {}};
    for (int j = 0; j < r.n; ++j) {
      if (!r.strs[j]) return sfail(LTXW_ERR_INVALID_ARG, "key rule %d: null string", k);
      x.s.emplace_back(r.strs[j]);
    }
    rs.push_back(std::move(x));
  }
  std::unique_ptr<ltxw_store> s(new (std::nothrow) ltxw_store());
  if (!s) return sfail(LTXW_ERR_OOM, "store allocation");
  for (int fi = 0; fi < n_paths; ++fi) {
    if (!paths[fi]) return sfail(LTXW_ERR_INVALID_ARG, "null path at index %d", fi);
    std::shared_ptr<MappedFile> f;
    if (int rc = map_file(paths[fi], &f)) return rc;
    st::Header h;
    if (int rc = parse_file(*f, &h)) return rc;
    for (const auto& kv : h.metadata) s->metadata.emplace(kv.first, kv.second);  // first file wins
    for (const auto& t : h.tensors) {
      std::string name = t.first;
      if (!apply_key(rs, &name)) continue;
      if (s->entries.count(name)) return sfail(LTXW_ERR_DUPLICATE_KEY, "duplicate key \"%s\" across checkpoint files",
                                               name.c_str());
      Entry e{t.second.dtype, t.second.shape, (uint32_t)s->files.size(), h.data_start + t.second.begin,
              h.data_start + t.second.end, t.second.numel(), t.second.dtype};
      s->entries.emplace(std::move(name), std::move(e));
    }
    s->files.push_back(std::move(f));
  }
  // `{key}_scale` of an FP8 `key` is internal (store.rs:174-187).
  for (const auto& kv : s->entries) {
    const std::string& k = kv.first;
    if (!ends_with(k, "_scale")) continue;
    auto it = s->entries.find(k.substr(0, k.size() - 6));
    if (it != s->entries.end() && st::is_fp8(it->second.dtype)) s->scale_keys.insert(k);
  }
  // Open-time value transforms, in the reference's order (store.rs:190-198).
  if (want_fold)
    if (int rc = apply_gate_fold(s.get())) return rc;
  if (want_split)
    if (int rc = apply_qkv_split(s.get())) return rc;
  if (want_type_emb) apply_zero_type_emb(s.get());
  for (const auto& kv : s->entries)
    if (!s->scale_keys.count(kv.first)) s->visible.push_back(kv.first);
  std::sort(s->visible.begin(), s->visible.end());
  *out = s.release();
  return LTXW_OK;
}

void ltxw_store_close(ltxw_store* s) { delete s; }

int64_t ltxw_store_n_keys(const ltxw_store* s) { return s ? (int64_t)s->visible.size() : 0; }

const char* ltxw_store_key(const ltxw_store* s, int64_t index) {
  if (!s || index < 0 || index >= (int64_t)s->visible.size()) return nullptr;
  return s->visible[(size_t)index].c_str();
}

int ltxw_store_contains(const ltxw_store* s, const char* key) {
  if (!s || !key) return 0;
  return s->entries.count(key) && !s->scale_keys.count(key) ? 1 : 0;
}

int ltxw_store_tensor_info(const ltxw_store* s, const char* key, int32_t* dtype, int32_t* ndim, int64_t* shape,
                           int32_t max_dims) {
  if (!s || !key) return sfail(LTXW_ERR_INVALID_ARG, "null store or key");
  auto it = s->entries.find(key);
  if (it == s->entries.end()) return sfail(LTXW_ERR_MISSING_KEY, "missing key: \"%s\"", key);
  return tensor_info_out(it->second.dtype, it->second.shape, dtype, ndim, shape, max_dims);
}

const char* ltxw_store_metadata(const ltxw_store* s, const char* key) {
  if (!s || !key) return nullptr;
  auto it = s->metadata.find(key);
  return it == s->metadata.end() ? nullptr : it->second.c_str();
}

int ltxw_lora_open(const char* path, ltxw_lora_file** out) {
  if (!out || !path) return sfail(LTXW_ERR_INVALID_ARG, "null path or output pointer");
  *out = nullptr;
  auto d = std::make_shared<LoraData>();
  if (int rc = map_file(path, &d->file)) return rc;
  st::Header h;
  if (int rc = parse_file(*d->file, &h)) return rc;
  d->metadata = h.metadata;
  for (auto& t : h.tensors) {
    st::TensorInfo ti = t.second;
    ti.begin += h.data_start;
    ti.end += h.data_start;
    d->names.push_back(t.first);
    d->tensors.emplace(t.first, ti);
  }
  std::sort(d->names.begin(), d->names.end());
  ltxw_lora_file* f = new (std::nothrow) ltxw_lora_file();
  if (!f) return sfail(LTXW_ERR_OOM, "LoRA file allocation");
  f->d = std::move(d);
  *out = f;
  return LTXW_OK;
}

void ltxw_lora_close(ltxw_lora_file* f) { delete f; }

int64_t ltxw_lora_n_tensors(const ltxw_lora_file* f) { return f ? (int64_t)f->d->names.size() : 0; }

const char* ltxw_lora_tensor_name(const ltxw_lora_file* f, int64_t index) {
  if (!f || index < 0 || index >= (int64_t)f->d->names.size()) return nullptr;
  return f->d->names[(size_t)index].c_str();
}

int ltxw_lora_tensor_info(const ltxw_lora_file* f, const char* name, int32_t* dtype, int32_t* ndim, int64_t* shape,
                          int32_t max_dims) {
  if (!f || !name) return sfail(LTXW_ERR_INVALID_ARG, "null LoRA file or name");
  auto it = f->d->tensors.find(name);
  if (it == f->d->tensors.end()) return sfail(LTXW_ERR_MISSING_KEY, "missing key: \"%s\"", name);
  return tensor_info_out(it->second.dtype, it->second.shape, dtype, ndim, shape, max_dims);
}

const char* ltxw_lora_metadata(const ltxw_lora_file* f, const char* key) {
  if (!f || !key) return nullptr;
  auto it = f->d->metadata.find(key);
  return it == f->d->metadata.end() ? nullptr : it->second.c_str();
}

int ltxw_lora_ic_layout(const ltxw_lora_file* f, uint32_t* downscale, uint32_t* temporal) {
  if (!f || !downscale || !temporal) return sfail(LTXW_ERR_INVALID_ARG, "null argument");
  // parse_u32_meta (lora.rs:211-213): trimmed, an optional '+', decimal digits.
  auto parse = [&](const char* key) -> uint32_t {
    auto it = f->d->metadata.find(key);
    if (it == f->d->metadata.end()) return 1;
    const std::string& v = it->second;
    size_t a = 0, b = v.size();
    while (a < b && isspace((unsigned char)v[a])) ++a;
    while (b > a && isspace((unsigned char)v[b - 1])) --b;
    if (a < b && v[a] == '+') ++a;
    if (a == b) return 1;
    uint64_t x = 0;
    for (size_t i = a; i < b; ++i) {
      if (v[i] < '0' || v[i] > '9') return 1;
      x = x * 10 + (uint64_t)(v[i] - '0');
      if (x > UINT32_MAX) return 1;
    }
    return (uint32_t)x;
  };
  uint32_t d = parse("reference_downscale_factor"), t = parse("reference_temporal_scale_factor");
  // IcLoraLayout::new (ltx-shape src/lib.rs:228-242) rejects a zero factor.
  if (d == 0) return sfail(LTXW_ERR_INVALID_ARG, "shape error: reference scale factor %u", d);
  if (t == 0) return sfail(LTXW_ERR_INVALID_ARG, "shape error: reference scale factor %u", t);
  *downscale = d;
  *temporal = t;
  return LTXW_OK;
}

int ltxw_lora_read_f32(const ltxw_lora_file* f, const char* name, float* out, int64_t n) {
  if (!f || !name) return sfail(LTXW_ERR_INVALID_ARG, "null LoRA file or name");
  auto it = f->d->tensors.find(name);
  if (it == f->d->tensors.end()) return sfail(LTXW_ERR_MISSING_KEY, "missing key: \"%s\"", name);
  const st::TensorInfo& t = it->second;
  if (!decodable(t.dtype))
    return sfail(LTXW_ERR_UNSUPPORTED, "unsupported dtype %s for key \"%s\"", st::dtype_name(t.dtype), name);
  if (n < 0 || (uint64_t)n != t.numel())
    return sfail(LTXW_ERR_INVALID_ARG, "\"%s\" holds %llu elements, the buffer %lld", name,
                 (unsigned long long)t.numel(), (long long)n);
  if (n && !out) return sfail(LTXW_ERR_INVALID_ARG, "null output buffer");
  decode_host(f->d->file->base + t.begin, t.dtype, (uint64_t)n, out);
  return LTXW_OK;
}

int ltxw_store_merge_lora(ltxw_store* s, const ltxw_lora_file* f, float strength, ltxw_merge_report** report) {
  if (report) *report = nullptr;
  if (!s || !f) return sfail(LTXW_ERR_INVALID_ARG, "null store or LoRA file");
  const LoraData& L = *f->d;
  static const std::string kA = ".lora_A.weight";
  std::unique_ptr<ltxw_merge_report> rep(new ltxw_merge_report());
  std::vector<std::pair<std::string, Delta>> pending;
  for (const std::string& key_a : L.names) {  // store.rs:549-560
    if (!ends_with(key_a, kA)) continue;
    const std::string prefix = key_a.substr(0, key_a.size() - kA.size());
    const std::string base = prefix + ".weight", key_b = prefix + ".lora_B.weight";
    auto be = s->entries.find(base);
    if (be == s->entries.end()) {
      rep->unmatched.push_back(key_a);
      continue;
    }
    const st::TensorInfo& ta = L.tensors.at(key_a);
    if (!decodable(ta.dtype))
      return sfail(LTXW_ERR_UNSUPPORTED, "unsupported dtype %s for key \"%s\"", st::dtype_name(ta.dtype), key_a.c_str());
    auto tb_it = L.tensors.find(key_b);
    if (tb_it == L.tensors.end()) {
      rep->unmatched.push_back(key_a);
      continue;
    }
    const st::TensorInfo& tb = tb_it->second;
    if (!decodable(tb.dtype))
      return sfail(LTXW_ERR_UNSUPPORTED, "unsupported dtype %s for key \"%s\"", st::dtype_name(tb.dtype), key_b.c_str());
    // store.rs:578-603
    const uint64_t rank_a = dim_or(ta.shape, 0, 0), rank_b = dim_or(tb.shape, 1, 0);
    if (rank_a != rank_b || rank_a == 0)
      return sfail(LTXW_ERR_LORA_RANK, "LoRA inner rank mismatch for key \"%s\": A inner %llu, B inner %llu",
                   base.c_str(), (unsigned long long)rank_a, (unsigned long long)rank_b);
    const uint64_t out_f = dim_or(be->second.shape, 0, 0), in_f = dim_or(be->second.shape, 1, 1);
    if (dim_or(tb.shape, 0, 0) != out_f || dim_or(ta.shape, 1, 0) != in_f)
      return sfail(LTXW_ERR_LORA_SHAPE, "LoRA shape mismatch for key \"%s\"", base.c_str());
    // store.rs:605-615: alpha defaults to rank; coeff = strength.mul_add(alpha / rank, 0).
    float alpha = rank_f32(rank_a);
    auto al = L.tensors.find(prefix + ".alpha");
    if (al != L.tensors.end()) {
      if (!decodable(al->second.dtype))
        return sfail(LTXW_ERR_UNSUPPORTED, "unsupported dtype %s for key \"%s.alpha\"",
                     st::dtype_name(al->second.dtype), prefix.c_str());
      if (al->second.numel() > 0) decode_host(L.file->base + al->second.begin, al->second.dtype, 1, &alpha);
    }
    const float coeff = std::fma(strength, alpha / rank_f32(rank_a), 0.0f);
    pending.emplace_back(base, Delta{f->d, key_a, key_b, rank_a, out_f, in_f, coeff});
    rep->matched.push_back(base);
  }
  if (rep->matched.empty() && !rep->unmatched.empty())
    return sfail(LTXW_ERR_NO_LORA_MATCHES, "LoRA file did not match any base weight keys");
  for (auto& pd : pending) s->deltas[pd.first].push_back(std::move(pd.second));
  std::sort(rep->matched.begin(), rep->matched.end());
  std::sort(rep->unmatched.begin(), rep->unmatched.end());
  if (report) *report = rep.release();
  return LTXW_OK;
}

int64_t ltxw_report_n_matched(const ltxw_merge_report* r) { return r ? (int64_t)r->matched.size() : 0; }
const char* ltxw_report_matched(const ltxw_merge_report* r, int64_t i) {
  return (r && i >= 0 && i < (int64_t)r->matched.size()) ? r->matched[(size_t)i].c_str() : nullptr;
}
int64_t ltxw_report_n_unmatched(const ltxw_merge_report* r) { return r ? (int64_t)r->unmatched.size() : 0; }
const char* ltxw_report_unmatched(const ltxw_merge_report* r, int64_t i) {
  return (r && i >= 0 && i < (int64_t)r->unmatched.size()) ? r->unmatched[(size_t)i].c_str() : nullptr;
}
void ltxw_report_free(ltxw_merge_report* r) { delete r; }

int ltxw_store_n_deltas(const ltxw_store* s, const char* key) {
  if (!s || !key) return 0;
  auto it = s->deltas.find(key);
  return it == s->deltas.end() ? 0 : (int)it->second.size();
}

int ltxw_store_delta(const ltxw_store* s, const char* key, int index, int32_t* rank, float* coeff) {
  if (!s || !key) return sfail(LTXW_ERR_INVALID_ARG, "null store or key");
  auto it = s->deltas.find(key);
  if (it == s->deltas.end() || index < 0 || index >= (int)it->second.size())
    return sfail(LTXW_ERR_INVALID_ARG, "key \"%s\" has no delta %d", key, index);
  const Delta& d = it->second[(size_t)index];
  if (rank) *rank = d.rank > INT32_MAX ? INT32_MAX : (int32_t)d.rank;
  if (coeff) *coeff = d.coeff;
  return LTXW_OK;
}

int ltxw_store_materialize(ltxw_store* s, ltxw_ctx* ctx, const char* const* keys, int64_t n_keys,
                           int32_t out_dtype, uint32_t flags, void* const* outs) {
  return materialize(s, ctx, keys, n_keys, out_dtype, flags, outs);
}

int ltxw_store_read(ltxw_store* s, ltxw_ctx* ctx, const char* key, uint32_t flags, float* out, int64_t n) {
  if (!s || !ctx || !key) return sfail(LTXW_ERR_INVALID_ARG, "null store, context or key");
  if (int rc = check_flags(flags)) return rc;
  // The reference's rules unless the caller opts into an extension.
  flags = (flags & LTXW_MAT_ROW_SCALES ? 0u : LTXW_MAT_SCALE_FIRST) | (flags & LTXW_MAT_MFMA ? 0u : LTXW_MAT_EXACT);
  auto it = s->entries.find(key);
  if (it == s->entries.end()) return sfail(LTXW_ERR_MISSING_KEY, "missing key: \"%s\"", key);
  const uint64_t numel = it->second.numel;
  if (n < 0 || (uint64_t)n != numel)
    return sfail(LTXW_ERR_INVALID_ARG, "\"%s\" holds %llu elements, the buffer %lld", key,
                 (unsigned long long)numel, (long long)n);
  if (numel == 0) {  // validate the key as `read` would, nothing to compute
    void* none = nullptr;
    return materialize(s, ctx, &key, 1, LTXW_OUT_F32, flags, &none);
  }
  if (!out) return sfail(LTXW_ERR_INVALID_ARG, "null output buffer");
  void* dev = nullptr;
  if (int rc = ltxw_alloc(ctx, numel * 4, &dev)) return sfail(rc, "%s", ltxw_last_error(ctx));
  int rc = materialize(s, ctx, &key, 1, LTXW_OUT_F32, flags, &dev);
  if (rc == LTXW_OK && (rc = ltxw_download(ctx, dev, numel * 4, out)) != LTXW_OK)
    sfail(rc, "%s", ltxw_last_error(ctx));
  int rf = ltxw_free(ctx, dev);
  if (rc == LTXW_OK && rf != LTXW_OK) rc = sfail(rf, "%s", ltxw_last_error(ctx));
  return rc;
}

}  // extern "C"
