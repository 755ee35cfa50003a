// C ABI of ltxw (include/ltxw.h): context, device memory, staged uploads and
// the dequant / fused dequant + LoRA entry points.
//
// Validation mirrors the reference's error conventions (crates/ltx-weights/
// src/error.rs:7-100): every failure is a status code plus a message, nothing
// throws or aborts across the boundary.
#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <map>
#include <mutex>
#include <thread>
#include <tuple>
#include <new>
#include <string>
#include <vector>

#include "ctx.h"
#include "kernels.h"
#include "ltxw.h"

namespace {
thread_local std::string g_create_err;
}  // namespace

int ltxw::fail(ltxw_ctx* ctx, int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (ctx) ctx->err = buf; else g_create_err = buf;
  return code;
}

namespace {

using ltxw::fail;

int hip_fail(ltxw_ctx* ctx, hipError_t e, const char* what) {
  return fail(ctx, LTXW_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

#define HIP_TRY(ctx, expr, what)                    \
  do {                                              \
    hipError_t e_ = (expr);                         \
    if (e_ != hipSuccess) return hip_fail(ctx, e_, what); \
  } while (0)

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

// Bytes per LoRA factor element (ltxw_factor_dtype); 0 for an unknown type.
int factor_bytes(int dt) {
  switch (dt) {
    case LTXW_FACTOR_BF16:
    case LTXW_FACTOR_F16: return 2;
    case LTXW_FACTOR_F32: return 4;
    case LTXW_FACTOR_E4M3FN:
    case LTXW_FACTOR_E5M2: return 1;
    default: return 0;
  }
}

// rows * cols without overflow; false when either is negative or it overflows.
bool elem_count(int64_t rows, int64_t cols, uint64_t* n) {
  if (rows < 0 || cols < 0) return false;
  if (rows != 0 && (uint64_t)cols > UINT64_MAX / (uint64_t)rows) return false;
  *n = (uint64_t)rows * (uint64_t)cols;
  return *n <= (uint64_t)INT64_MAX / 4;
}

// When the runtime knows the device allocation containing `p`, the launch's
// byte extent [p, p + bytes) must lie inside it: a wrong or undersized
// buffer is then an INVALID_ARG instead of a GPU memory fault. Pointers the
// runtime does not track (other allocators) cannot be checked and pass.
// Mirrors the byte-range check of `Entry::read_raw` (src/store.rs:52-73).
int check_extent(ltxw_ctx* ctx, const void* p, uint64_t bytes, const char* what) {
  hipDeviceptr_t base = nullptr;
  size_t size = 0;
  if (hipMemGetAddressRange(&base, &size, const_cast<void*>(p)) != hipSuccess) {
    (void)hipGetLastError();
    return LTXW_OK;
  }
  uintptr_t b = (uintptr_t)base, q = (uintptr_t)p;
  uint64_t have = (q >= b && q - b <= size) ? size - (q - b) : 0;
  if (bytes > have)
    return fail(ctx, LTXW_ERR_INVALID_ARG, "%s buffer holds %llu bytes from the pointer, the tensor needs %llu",
                what, (unsigned long long)have, (unsigned long long)bytes);
  return LTXW_OK;
}

// Common checks of one tensor description; message names the offending field.
int check_desc(ltxw_ctx* ctx, const ltxw_tensor_desc& d, uint64_t* n) {
  if (!elem_count(d.rows, d.cols, n))
    return fail(ctx, LTXW_ERR_INVALID_ARG, "invalid shape [%lld, %lld]", (long long)d.rows, (long long)d.cols);
  const int esize = ltxw::format_bytes(d.fmt);
  if (esize == 0) return fail(ctx, LTXW_ERR_UNSUPPORTED, "unsupported weight format %d", d.fmt);
  if (d.scale_mode < LTXW_SCALE_NONE || d.scale_mode > LTXW_SCALE_ROW)
    return fail(ctx, LTXW_ERR_INVALID_ARG, "invalid scale mode %d", d.scale_mode);
  // store.rs:500: the `{key}_scale` sibling applies to FP8 tensors only.
  if (esize != 1 && d.scale_mode != LTXW_SCALE_NONE)
    return fail(ctx, LTXW_ERR_INVALID_ARG, "scales apply to FP8 formats only (format %d)", d.fmt);
  if (d.out_dtype != LTXW_OUT_BF16 && d.out_dtype != LTXW_OUT_F32)
    return fail(ctx, LTXW_ERR_INVALID_ARG, "invalid output dtype %d", d.out_dtype);
  if (d.n_loras < 0 || d.n_loras > LTXW_MAX_LORAS)
    return fail(ctx, LTXW_ERR_INVALID_ARG, "n_loras %d outside [0, %d]", d.n_loras, LTXW_MAX_LORAS);
  if (d.flags & ~LTXW_DESC_EXACT) return fail(ctx, LTXW_ERR_INVALID_ARG, "unknown descriptor flags 0x%x", d.flags);
  if (*n == 0) return LTXW_OK;
  if (!d.w || !d.out) return fail(ctx, LTXW_ERR_INVALID_ARG, "null weight or output pointer");
  if (!aligned(d.w, (size_t)esize))
    return fail(ctx, LTXW_ERR_INVALID_ARG, "weight pointer is not aligned to its %d-byte elements", esize);
  if (d.scale_mode != LTXW_SCALE_NONE && !d.scales)
    return fail(ctx, LTXW_ERR_INVALID_ARG, "scale mode %d needs a scales pointer", d.scale_mode);
  for (int l = 0; l < d.n_loras; ++l) {
    const ltxw_lora& L = d.loras[l];
    // store.rs:578-587: a zero rank is a rank mismatch.
    if (L.rank <= 0)
      return fail(ctx, LTXW_ERR_LORA_RANK, "LoRA %d has rank %d", l, L.rank);
    if (L.rank > (1 << 20)) return fail(ctx, LTXW_ERR_INVALID_ARG, "LoRA %d rank %d is too large", l, L.rank);
    if (!L.a || !L.b) return fail(ctx, LTXW_ERR_INVALID_ARG, "LoRA %d has a null factor", l);
    const int fs = factor_bytes(L.dtype);
    if (fs == 0) return fail(ctx, LTXW_ERR_UNSUPPORTED, "LoRA %d has unsupported factor type %d", l, L.dtype);
    if (!aligned(L.a, (size_t)fs) || !aligned(L.b, (size_t)fs))
      return fail(ctx, LTXW_ERR_INVALID_ARG, "LoRA %d factors are not aligned to their %d-byte elements", l, fs);
  }
  int rc;
  if ((rc = check_extent(ctx, d.w, *n * (uint64_t)esize, "weight"))) return rc;
  if ((rc = check_extent(ctx, d.out, *n * (d.out_dtype == LTXW_OUT_F32 ? 4 : 2), "output"))) return rc;
  if (d.scale_mode != LTXW_SCALE_NONE &&
      (rc = check_extent(ctx, d.scales, 4 * (d.scale_mode == LTXW_SCALE_ROW ? (uint64_t)d.rows : 1), "scales")))
    return rc;
  for (int l = 0; l < d.n_loras; ++l) {
    const ltxw_lora& L = d.loras[l];
    const uint64_t fs = (uint64_t)factor_bytes(L.dtype);
    if ((rc = check_extent(ctx, L.b, fs * (uint64_t)d.rows * (uint64_t)L.rank, "LoRA B"))) return rc;
    if ((rc = check_extent(ctx, L.a, fs * (uint64_t)L.rank * (uint64_t)d.cols, "LoRA A"))) return rc;
  }
  return LTXW_OK;
}

ltxw::JobDev to_job(const ltxw_tensor_desc& d) {
  ltxw::JobDev j{};
  j.w = d.w;
  j.out = d.out;
  j.scales = d.scales;
  j.rows = d.rows;
  j.cols = d.cols;
  j.fmt = d.fmt;
  j.scale_mode = d.scale_mode;
  j.n_loras = d.n_loras;
  for (int l = 0; l < d.n_loras; ++l)
    j.lora[l] = {(const uint16_t*)d.loras[l].b, (const uint16_t*)d.loras[l].a, d.loras[l].rank, d.loras[l].coeff,
                 d.loras[l].dtype, 0};
  j.bands_n = (int32_t)((d.cols + ltxw::kBandCols - 1) / ltxw::kBandCols);
  return j;
}

// The tiled MFMA kernel's layout requirements (else: generic kernel).
bool fused_ok(const ltxw_tensor_desc& d) {
  // FP8 bases; bf16 / f16 bases (no scale) when every factor is bf16.
  const int fb = ltxw::format_bytes(d.fmt);
  if (fb != 1 && !(fb == 2 && d.n_loras > 0 && d.loras[0].dtype == LTXW_FACTOR_BF16)) return false;
  if (d.cols % 8 != 0 || !aligned(d.w, 16) || !aligned(d.out, 16)) return false;
  if (d.scale_mode == LTXW_SCALE_ROW && !aligned(d.scales, 16)) return false;  // read 4 rows at a time
  // The kernel addresses every buffer with 32-bit byte offsets.
  const uint64_t lim = UINT32_MAX - 64;
  if ((uint64_t)d.rows * (uint64_t)d.cols * 4 > lim) return false;
  int k = 0;
  for (int l = 0; l < d.n_loras; ++l) {
    const uint64_t r = (uint64_t)d.loras[l].rank;
    // bf16, f16 and FP8 factors, the same type for all of a tensor's LoRAs
    // (one compiled factor type per launch); f32 factors keep the reference
    // order.
    const int dt = d.loras[l].dtype;
    if (dt == LTXW_FACTOR_F32 || dt != d.loras[0].dtype) return false;
    // 8 consecutive elements per load: 16 bytes (16-bit types) or 8 (FP8).
    const size_t vec = 8 * (size_t)factor_bytes(dt);
    if (r % 8 != 0 || !aligned(d.loras[l].a, vec) || !aligned(d.loras[l].b, vec)) return false;
    if (2 * r * (uint64_t)d.rows > lim || 2 * r * (uint64_t)d.cols > lim) return false;
    // Several LoRAs share one accumulator, rescaled by c_l / c_{l+1} between
    // them: keep those ratios and the rescaled partial sums far from f32
    // overflow and underflow.
    const float c = std::fabs(d.loras[l].coeff);
    if (d.n_loras > 1 && !(c >= 0x1p-24f && c <= 0x1p24f)) return false;
    k += ltxw::pad_rank(d.loras[l].rank);
  }
  return k <= ltxw::kRankMax;
}

// Fills the fused kernels' per-K-step table and coefficient fields of a job
// that fused_ok accepted (JobDev::qmask, cmul, coeff_out, step).
void plan_fused(ltxw::JobDev& j) {
  int t = 0;
  for (int l = 0; l < j.n_loras; ++l) {
    const ltxw::LoraDev& L = j.lora[l];
    const int nks = ltxw::pad_rank(L.rank) / 32;
    const size_t esz = (size_t)factor_bytes(L.dtype);
    // B rows whose 64-byte K-step pieces all fall at one offset of their
    // 128-byte lines: pair the steps for the B-fragment swap.
    const bool swap = esz == 2 && (L.rank * esz) % 128 == 0;
    for (int kt = 0; kt < nks && t < ltxw::kMaxSteps; ++kt, ++t) {
      ltxw::StepDev& s = j.step[t];
      s.a = (const char*)L.a + esz * 32 * kt * (size_t)j.cols;
      s.b = (const char*)L.b + esz * 32 * kt;
      s.rank = (uint32_t)L.rank;
      s.klim = (uint32_t)(L.rank - 32 * kt);
      s.q = 1.0f;
      s.pair = swap && kt % 2 == 0 && kt + 1 < nks ? 1u : 0u;
    }
    if (l + 1 < j.n_loras && t >= 1) {
      j.step[t - 1].q = L.coeff / j.lora[l + 1].coeff;
      if (j.step[t - 1].q != 1.0f) j.qmask |= 1u << (t - 1);
    }
  }
  j.coeff_out = j.n_loras > 0 ? j.lora[j.n_loras - 1].coeff : 1.0f;
  j.cmul = j.coeff_out != 1.0f ? 1u : 0u;
}

int run_generic(ltxw_ctx* ctx, const ltxw_tensor_desc& d, uint64_t begin, uint64_t count,
                const ltxw::DescEx* ex = nullptr) {
  ltxw::GenericArgs g{};
  g.job = to_job(d);
  g.elem_begin = begin;
  g.elem_count = count;
  if (ex) {
    g.plain_scale = ex->plain_scale;
    g.has_post = ex->has_post;
    g.post_mul = ex->post_mul;
  }
  HIP_TRY(ctx, ltxw::launch_generic(g, d.out_dtype == LTXW_OUT_F32, ctx->compute), "generic kernel launch");
  return LTXW_OK;
}

// Reference-order tiled kernel over the whole tensor (LoRA deltas in the
// reference's order, any factor type, base format, shape and alignment).
int run_exact(ltxw_ctx* ctx, const ltxw_tensor_desc& d, const ltxw::DescEx* ex) {
  ltxw::ExactArgs a{};
  a.job = to_job(d);
  if (ex) {
    a.plain_scale = ex->plain_scale;
    a.has_post = ex->has_post;
    a.post_mul = ex->post_mul;
    a.canon_nan = ex->canon_nan;
  }
  a.bands_n = (uint32_t)((d.cols + ltxw::kExactCols - 1) / ltxw::kExactCols);
  HIP_TRY(ctx, ltxw::launch_exact(a, d.out_dtype == LTXW_OUT_F32, ctx->compute), "exact kernel launch");
  return LTXW_OK;
}

// Dequant without LoRA: vector kernel on 16-element chunks, generic on the rest.
int run_dequant(ltxw_ctx* ctx, const ltxw_tensor_desc& d, uint64_t n) {
  // Tensors up to an FFN matrix: the tiled kernel.
  if (n <= ltxw::kTileMaxElems && d.cols % 8 == 0 && aligned(d.w, 16) && aligned(d.out, 16) &&
      (d.scale_mode != LTXW_SCALE_ROW || aligned(d.scales, 16))) {
    const uint32_t bands = (uint32_t)((d.cols + ltxw::kBandCols - 1) / ltxw::kBandCols);
    ltxw::DequantTileArgs a{d.w, d.out, d.scales, (uint32_t)d.rows, (uint32_t)d.cols, bands};
    HIP_TRY(ctx, ltxw::launch_dequant_tile(a, d.fmt, d.scale_mode, d.out_dtype == LTXW_OUT_F32, ctx->compute),
            "tiled dequant kernel launch");
    return LTXW_OK;
  }
  bool vec = aligned(d.w, 16) && aligned(d.out, 16) && (d.scale_mode != LTXW_SCALE_ROW || d.cols >= 16);
  uint64_t chunks = vec ? n / 16 : 0;
  if (chunks) {
    ltxw::DequantArgs a{d.w, d.out, d.scales, n, (uint64_t)d.cols, chunks};
    HIP_TRY(ctx, ltxw::launch_dequant(a, d.fmt, d.scale_mode, d.out_dtype == LTXW_OUT_F32, ctx->compute),
            "dequant kernel launch");
  }
  if (chunks * 16 < n) return run_generic(ctx, d, chunks * 16, n - chunks * 16);
  return LTXW_OK;
}

}  // namespace

namespace {

// Job-table slots go in groups of kTableGroup: an event is recorded after the
// upload into a group's last slot only, and the host waits for it before it
// rewrites the group's first slot. An event record per grouped launch
// measured 2-4.5 us of GPU time per launch (DiT block, mixed block).
constexpr size_t kTableGroup = 8;

// Next job-table slot with room for `bytes`. Its host mirror is reusable once
// the slot's previous upload has completed; the device copy is ordered on the
// compute stream after every earlier kernel that read it.
int take_table(ltxw_ctx* ctx, size_t bytes, ltxw_ctx::TableSlot** out, bool* record) {
  const size_t k = ctx->next_table;
  ltxw_ctx::TableSlot& t = ctx->tables[k];
  ctx->next_table = (k + 1) % ctx->tables.size();
  if (k % kTableGroup == 0)  // every upload of the group's previous round precedes this event
    HIP_TRY(ctx, hipEventSynchronize(ctx->tables[k + kTableGroup - 1].copied), "job table wait");
  *record = k % kTableGroup == kTableGroup - 1;
  if (bytes > t.cap) {
    HIP_TRY(ctx, hipStreamSynchronize(ctx->compute), "job table resize");
    if (t.host) (void)hipHostFree(t.host);
    if (t.dev) (void)hipFree(t.dev);
    t.host = t.dev = nullptr;
    t.cap = 0;
    size_t cap = std::max<size_t>(bytes, 64 * 1024);
    if (hipHostMalloc(&t.host, cap, hipHostMallocDefault) != hipSuccess)
      return fail(ctx, LTXW_ERR_OOM, "pinned job table of %zu bytes", cap);
    if (hipMalloc(&t.dev, cap) != hipSuccess) return fail(ctx, LTXW_ERR_OOM, "device job table of %zu bytes", cap);
    t.cap = cap;
  }
  *out = &t;
  return LTXW_OK;
}

// Bytes of one fused launch's job record with ks K-steps.
constexpr size_t record_bytes(int ks) { return sizeof(ltxw::FusedJob) + (size_t)ks * sizeof(ltxw::StepDev); }
static_assert(LTXW_NOALLOC_MAX_DESCS * record_bytes(ltxw::kMaxSteps) <= ltxw::kScratchBytes,
              "the largest allocation-free call's job table fits the scratch array");

// Writes the records of jobs [first, first + count) (plan_fused done) to dst.
void write_records(const std::vector<ltxw::JobDev>& jobs, size_t first, size_t count, int ks, unsigned char* dst) {
  for (size_t k = 0; k < count; ++k) {
    const ltxw::JobDev& j = jobs[first + k];
    ltxw::FusedJob h{};
    h.w = j.w;
    h.out = j.out;
    h.scales = j.scales;
    h.rows = (uint32_t)j.rows;
    h.cols = (uint32_t)j.cols;
    h.bands_n = (uint32_t)j.bands_n;
    h.unit_begin = (uint32_t)j.unit_begin;
    h.fmt = (uint32_t)j.fmt;
    h.scale_mode = (uint32_t)j.scale_mode;
    h.qmask = j.qmask;
    h.cmul = j.cmul;
    h.coeff_out = j.coeff_out;
    h.single = j.single;
    unsigned char* r = dst + k * record_bytes(ks);
    memcpy(r, &h, sizeof(h));
    memcpy(r + sizeof(h), j.step, (size_t)ks * sizeof(ltxw::StepDev));
  }
}

// Total padded LoRA rank of a job (its K extent in the LDS stage).
int job_k(const ltxw::JobDev& j) {
  int k = 0;
  for (int l = 0; l < j.n_loras; ++l) k += ltxw::pad_rank(j.lora[l].rank);
  return k;
}

// Large launches: the last job's last rows (about kTailPairs pair
// workgroups' worth, whole row pairs) become a job of single-unit workgroups
// at the launch's end, so that the launch drains in narrow units: a DiT block
// (8192 workgroups) 144.4-145.6 -> 141.7-142.2 us, with 256 pairs' worth
// 143.1-144.0, with 1024 141.6-142.5 (alternating runs on one machine). Only
// where the records stay in the kernel arguments.
void split_tail(std::vector<ltxw::JobDev>& jobs, int64_t pairs, bool f32out, size_t rec) {
  if (pairs <= (int64_t)ltxw::kRemapMinGrid || jobs.empty()) return;
  if ((jobs.size() + 1) * rec > (size_t)ltxw::kInlineTableBytes || jobs.size() + 1 > (size_t)ltxw::kInlineBegins)
    return;
  ltxw::JobDev& L = jobs.back();
  const int64_t row_pairs = (L.rows + ltxw::kPairRows - 1) / ltxw::kPairRows;
  const int64_t take = std::min<int64_t>(row_pairs - 1, (ltxw::kTailPairs + L.bands_n - 1) / L.bands_n);
  if (take <= 0) return;
  const int64_t r1 = (row_pairs - take) * ltxw::kPairRows;
  ltxw::JobDev T = L;
  T.rows = L.rows - r1;
  T.single = 1;
  T.w = L.w + r1 * L.cols * ltxw::format_bytes(L.fmt);
  T.out = (char*)L.out + r1 * L.cols * (f32out ? 4 : 2);
  if (L.scale_mode == LTXW_SCALE_ROW) T.scales = L.scales + r1;
  for (int l = 0; l < L.n_loras; ++l)
    T.lora[l].b = (const uint16_t*)((const char*)L.lora[l].b +
                                    r1 * (int64_t)L.lora[l].rank * factor_bytes(L.lora[l].dtype));
  L.rows = r1;
  jobs.push_back(T);
}

// One fused launch over `jobs` (all fused_ok, same out dtype, kernel, factor
// type and K-steps): one workgroup per 128-column band and 256 rows of every
// job (128 rows in a split launch's single-unit job).
int run_fused(ltxw_ctx* ctx, std::vector<ltxw::JobDev>& jobs, bool f32out, bool multi, int fdt, bool base16,
              bool noalloc) {
  if (jobs.empty()) return LTXW_OK;
  int kmax = 0;
  for (auto& j : jobs) kmax = std::max(kmax, job_k(j));
  // Every job of the launch has the same K-steps (the launches are bucketed by them).
  const int ks = kmax / 32;
  const size_t rec = record_bytes(ks);
  int64_t pairs = 0;
  for (auto& j : jobs) pairs += (int64_t)j.bands_n * ((j.rows + ltxw::kPairRows - 1) / ltxw::kPairRows);
  // Several-LoRA launches split up to 2 K-steps (a DiT block with r32 + r32
  // LoRAs 151.3-153.1 -> 147.0-147.6 us) and keep pairs to the end above: a
  // mixed DiT block (5 K-steps) measured 251.6-251.9 -> 254.8-255.4 us with
  // single units.
  if (!multi || ks <= 2) split_tail(jobs, pairs, f32out, rec);
  int64_t units = 0;  // workgroups (unit pairs; single units in a split launch's last job)
  int64_t main_groups = -1;
  for (auto& j : jobs) {
    plan_fused(j);
    j.unit_begin = units;
    if (j.single && main_groups < 0) main_groups = units;
    const int64_t group_rows = j.single ? ltxw::kUnitRows : ltxw::kPairRows;
    units += (int64_t)j.bands_n * ((j.rows + group_rows - 1) / group_rows);
  }
  if (main_groups < 0) main_groups = units;
  if (units > INT32_MAX) return fail(ctx, LTXW_ERR_INVALID_ARG, "launch of %lld work units is too large", (long long)units);
  const size_t bytes = jobs.size() * rec;
  ltxw::JobTable t{};
  t.n_jobs = (int32_t)jobs.size();
  t.total_units = units;
  t.lds_ld = kmax + 8;
  t.rec_bytes = (int32_t)rec;
  t.main_groups = (uint32_t)main_groups;
  for (int k = 0; k < ltxw::kInlineBegins; ++k)
    t.begins[k] = (size_t)k < jobs.size() ? (uint32_t)jobs[(size_t)k].unit_begin : UINT32_MAX;
  // The single-LoRA kernel reads a one-job launch's JobDev from its fixed
  // place in the arguments; the several-LoRA kernel reads the record.
  if (jobs.size() == 1) t.one = jobs[0];
  if (bytes <= (size_t)ltxw::kInlineTableBytes) {
    // In the kernel arguments: no upload (a DiT block's 10 tensors fit).
    write_records(jobs, 0, jobs.size(), ks, t.inl);
    t.table = nullptr;
  } else if (noalloc) {
    // The device scratch array, written by fill launches queued just before
    // this launch: launches on this stream run in order, so the previous
    // reader of the scratch has finished by then.
    if (bytes > ltxw::kScratchBytes || !ctx->scratch)
      return fail(ctx, LTXW_ERR_INVALID_ARG, "job table of %zu bytes exceeds the %zu-byte scratch", bytes,
                  ltxw::kScratchBytes);
    alignas(16) unsigned char buf[ltxw::kInlineTableBytes];
    const size_t per = (size_t)ltxw::kInlineTableBytes / rec;
    for (size_t k = 0; k < jobs.size(); k += per) {
      const size_t cnt = std::min(per, jobs.size() - k);
      write_records(jobs, k, cnt, ks, buf);
      HIP_TRY(ctx, ltxw::launch_fill_words((char*)ctx->scratch + k * rec, buf, cnt * rec, ctx->compute),
              "job table fill");
    }
    t.table = ctx->scratch;
  } else {
    ltxw_ctx::TableSlot* slot = nullptr;
    bool record = false;
    int rc = take_table(ctx, bytes, &slot, &record);
    if (rc) return rc;
    write_records(jobs, 0, jobs.size(), ks, (unsigned char*)slot->host);
    hipError_t e = hipMemcpyAsync(slot->dev, slot->host, bytes, hipMemcpyHostToDevice, ctx->compute);
    if (e == hipSuccess && record) e = hipEventRecord(slot->copied, ctx->compute);
    if (e != hipSuccess) {
      // The group's event may now be missing for this round: drain the stream
      // so that no queued upload still reads a host slot the next round rewrites.
      (void)hipStreamSynchronize(ctx->compute);
      return hip_fail(ctx, e, "job table upload");
    }
    t.table = slot->dev;
  }
  HIP_TRY(ctx, ltxw::launch_fused(t, f32out, multi, fdt, base16, ctx->compute), "fused kernel launch");
  return LTXW_OK;
}

}  // namespace

int ltxw::run_descs(ltxw_ctx* ctx, const ltxw_tensor_desc* descs, int n, const DescEx* ex, bool noalloc) {
  // Job tables are allocated on the calling thread's current device.
  HIP_TRY(ctx, hipSetDevice(ctx->device), "hipSetDevice");
  // Validate everything before queuing anything.
  std::vector<uint64_t> counts((size_t)n);
  for (int k = 0; k < n; ++k) {
    int rc = check_desc(ctx, descs[k], &counts[(size_t)k]);
    if (rc) return rc;
  }
  // Fused launches are bucketed by (f32 out, kernel, K-steps, factor type,
  // 16-bit base), so that the register arrays of each launch are sized for
  // its own jobs' rank, not for the largest rank of the call. One bf16 LoRA
  // on an FP8 base takes the single-LoRA kernel; several LoRAs, other factor
  // types or bf16 / f16 bases the several-LoRA one.
  std::map<std::tuple<int, int, int, int, int>, std::vector<ltxw::JobDev>> buckets;
  for (int k = 0; k < n; ++k) {
    const ltxw_tensor_desc& d = descs[k];
    uint64_t cnt = counts[(size_t)k];
    if (cnt == 0) continue;
    int rc = LTXW_OK;
    const bool extras = ex && (ex[k].plain_scale || ex[k].has_post || ex[k].canon_nan);
    if (extras || (d.n_loras > 0 && ((d.flags & LTXW_DESC_EXACT) || !fused_ok(d)))) {
      rc = run_exact(ctx, d, extras ? &ex[k] : nullptr);
    } else if (d.n_loras == 0) {
      rc = ltxw::format_bytes(d.fmt) == 1 ? run_dequant(ctx, d, cnt) : run_generic(ctx, d, 0, cnt);
    } else {
      ltxw::JobDev j = to_job(d);
      const int fdt = d.loras[0].dtype;
      const bool base16 = ltxw::format_bytes(d.fmt) == 2;
      const bool multi = d.n_loras > 1 || fdt != LTXW_FACTOR_BF16 || base16;
      buckets[{d.out_dtype == LTXW_OUT_F32, multi, job_k(j) / 32, fdt, base16}].push_back(j);
    }
    if (rc) return rc;
  }
  for (auto& kv : buckets) {
    int rc = run_fused(ctx, kv.second, std::get<0>(kv.first) == 1, std::get<1>(kv.first) == 1, std::get<3>(kv.first),
                       std::get<4>(kv.first) == 1, noalloc);
    if (rc) return rc;
  }
  return LTXW_OK;
}

int ltxw::ensure_staging(ltxw_ctx* ctx) {
  if (!ctx->stage.empty()) return LTXW_OK;
  // One contiguous pinned block, so that neighbouring slots can go out in a
  // single copy.
  void* block = nullptr;
  const size_t total = ctx->stage_bytes * (size_t)ctx->n_stage;
  if (hipHostMalloc(&block, total, hipHostMallocDefault) != hipSuccess) {
    (void)hipGetLastError();
    return fail(ctx, LTXW_ERR_OOM, "pinned staging ring of %zu bytes", total);
  }
  std::vector<hipEvent_t> evs;
  for (int k = 0; k < ctx->n_stage; ++k) {
    hipEvent_t ev = nullptr;
    hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e != hipSuccess) {
      for (hipEvent_t x : evs) (void)hipEventDestroy(x);
      (void)hipHostFree(block);
      return hip_fail(ctx, e, "staging event");
    }
    evs.push_back(ev);
  }
  ctx->stage_block = block;
  for (int k = 0; k < ctx->n_stage; ++k) ctx->stage.push_back((char*)block + (size_t)k * ctx->stage_bytes);
  ctx->stage_done = std::move(evs);
  ctx->next_stage = 0;
  return LTXW_OK;
}

extern "C" {

int ltxw_ctx_create(int device, size_t staging_bytes, int n_staging, ltxw_ctx** out) {
  if (!out) return fail(nullptr, LTXW_ERR_INVALID_ARG, "null output pointer");
  *out = nullptr;
  int ndev = 0;
  hipError_t e = hipGetDeviceCount(&ndev);
  if (e != hipSuccess) return fail(nullptr, LTXW_ERR_HIP, "hipGetDeviceCount: %s", hipGetErrorString(e));
  if (device < 0 || device >= ndev)
    return fail(nullptr, LTXW_ERR_INVALID_ARG, "device %d not in [0, %d)", device, ndev);
  if (staging_bytes == 0) staging_bytes = 64u << 20;
  if (n_staging <= 0) n_staging = 16;
  if (staging_bytes % 4096 != 0)
    return fail(nullptr, LTXW_ERR_INVALID_ARG, "staging_bytes %zu is not a multiple of 4096", staging_bytes);
  ltxw_ctx* c = new (std::nothrow) ltxw_ctx();
  if (!c) return fail(nullptr, LTXW_ERR_OOM, "context allocation");
  c->device = device;
  c->stage_bytes = staging_bytes;
  c->n_stage = n_staging;
  c->host_threads = (int)std::max(1u, std::min(8u, std::thread::hardware_concurrency()));
  auto bail = [&](int code, const char* what, hipError_t he) {
    g_create_err = std::string(what) + ": " + hipGetErrorString(he);
    ltxw_ctx_destroy(c);
    return code;
  };
  if ((e = hipSetDevice(device)) != hipSuccess) return bail(LTXW_ERR_HIP, "hipSetDevice", e);
  if ((e = hipDeviceGetAttribute(&c->cu_count, hipDeviceAttributeMultiprocessorCount, device)) != hipSuccess)
    return bail(LTXW_ERR_HIP, "device attribute", e);
  if ((e = hipStreamCreateWithFlags(&c->compute, hipStreamNonBlocking)) != hipSuccess)
    return bail(LTXW_ERR_HIP, "compute stream", e);
  if ((e = hipStreamCreateWithFlags(&c->copy, hipStreamNonBlocking)) != hipSuccess)
    return bail(LTXW_ERR_HIP, "copy stream", e);
  if ((e = hipEventCreateWithFlags(&c->compute_mark, hipEventDisableTiming)) != hipSuccess)
    return bail(LTXW_ERR_HIP, "event", e);
  if ((e = ltxw::scratch_address(&c->scratch)) != hipSuccess) return bail(LTXW_ERR_HIP, "scratch address", e);
  c->tables.resize(2 * kTableGroup);
  for (auto& t : c->tables)
    if ((e = hipEventCreateWithFlags(&t.copied, hipEventDisableTiming)) != hipSuccess)
      return bail(LTXW_ERR_HIP, "event", e);
  *out = c;
  return LTXW_OK;
}

void ltxw_ctx_destroy(ltxw_ctx* ctx) {
  if (!ctx) return;
  (void)hipSetDevice(ctx->device);
  if (ctx->compute) (void)hipStreamSynchronize(ctx->compute);
  if (ctx->copy) (void)hipStreamSynchronize(ctx->copy);
  if (ctx->stage_block) (void)hipHostFree(ctx->stage_block);
  for (hipEvent_t ev : ctx->stage_done) (void)hipEventDestroy(ev);
  for (void* p : ctx->ring) (void)hipFree(p);
  if (ctx->tmp) (void)hipFree(ctx->tmp);
  for (hipEvent_t ev : ctx->ring_free) (void)hipEventDestroy(ev);
  for (hipEvent_t ev : ctx->ring_ready) (void)hipEventDestroy(ev);
  for (auto& t : ctx->tables) {
    if (t.host) (void)hipHostFree(t.host);
    if (t.dev) (void)hipFree(t.dev);
    if (t.copied) (void)hipEventDestroy(t.copied);
  }
  if (ctx->compute_mark) (void)hipEventDestroy(ctx->compute_mark);
  if (ctx->compute) (void)hipStreamDestroy(ctx->compute);
  if (ctx->copy) (void)hipStreamDestroy(ctx->copy);
  delete ctx;
}

const char* ltxw_last_error(const ltxw_ctx* ctx) {
  return ctx ? ctx->err.c_str() : g_create_err.c_str();
}

void* ltxw_ctx_stream(ltxw_ctx* ctx) { return ctx ? (void*)ctx->compute : nullptr; }

int ltxw_ctx_set_host_threads(ltxw_ctx* ctx, int n) {
  if (!ctx) return fail(ctx, LTXW_ERR_INVALID_ARG, "null context");
  if (n < 1 || n > 256) return fail(ctx, LTXW_ERR_INVALID_ARG, "host thread count %d outside [1, 256]", n);
  ctx->host_threads = n;
  return LTXW_OK;
}

int ltxw_alloc(ltxw_ctx* ctx, size_t bytes, void** dptr) {
  if (!ctx || !dptr) return fail(ctx, LTXW_ERR_INVALID_ARG, "null context or output pointer");
  *dptr = nullptr;
  if (bytes == 0) return LTXW_OK;
  HIP_TRY(ctx, hipSetDevice(ctx->device), "hipSetDevice");
  hipError_t e = hipMalloc(dptr, bytes);
  if (e != hipSuccess) {
    *dptr = nullptr;
    (void)hipGetLastError();
    return fail(ctx, LTXW_ERR_OOM, "device allocation of %zu bytes: %s", bytes, hipGetErrorString(e));
  }
  return LTXW_OK;
}

int ltxw_free(ltxw_ctx* ctx, void* dptr) {
  if (!ctx) return fail(ctx, LTXW_ERR_INVALID_ARG, "null context");
  if (!dptr) return LTXW_OK;
  // Work already queued may still read the buffer.
  HIP_TRY(ctx, hipStreamSynchronize(ctx->compute), "synchronize before free");
  HIP_TRY(ctx, hipFree(dptr), "hipFree");
  return LTXW_OK;
}

int ltxw_memset(ltxw_ctx* ctx, void* dptr, int value, size_t bytes) {
  if (!ctx || (!dptr && bytes)) return fail(ctx, LTXW_ERR_INVALID_ARG, "null context or pointer");
  if (bytes == 0) return LTXW_OK;
  if (int rc = check_extent(ctx, dptr, bytes, "memset destination")) return rc;
  HIP_TRY(ctx, hipMemsetAsync(dptr, value, bytes, ctx->compute), "hipMemsetAsync");
  return LTXW_OK;
}

int ltxw_upload(ltxw_ctx* ctx, const void* host_src, size_t bytes, void* dst) {
  if (!ctx) return fail(ctx, LTXW_ERR_INVALID_ARG, "null context");
  if (bytes == 0) return LTXW_OK;
  if (!host_src || !dst) return fail(ctx, LTXW_ERR_INVALID_ARG, "null source or destination");
  if (int rc = check_extent(ctx, dst, bytes, "upload destination")) return rc;
  HIP_TRY(ctx, hipSetDevice(ctx->device), "hipSetDevice");
  if (int rc = ltxw::ensure_staging(ctx)) return rc;
  // Call order: the copy must not overtake kernels or memsets already queued
  // on the compute stream that read or write `dst` (a buffer reused for the
  // next tensor while the previous one's kernel is still queued).
  HIP_TRY(ctx, hipEventRecord(ctx->compute_mark, ctx->compute), "upload ordering event");
  HIP_TRY(ctx, hipStreamWaitEvent(ctx->copy, ctx->compute_mark, 0), "copy waits for queued work");
  const char* src = (const char*)host_src;
  size_t done = 0;
  while (done < bytes) {
    size_t k = ctx->next_stage;
    ctx->next_stage = (k + 1) % ctx->stage.size();
    size_t len = std::min(ctx->stage_bytes, bytes - done);
    // The slot's previous copy must have left the buffer before it is refilled.
    HIP_TRY(ctx, hipEventSynchronize(ctx->stage_done[k]), "staging wait");
    memcpy(ctx->stage[k], src + done, len);
    HIP_TRY(ctx, hipMemcpyAsync((char*)dst + done, ctx->stage[k], len, hipMemcpyHostToDevice, ctx->copy),
            "hipMemcpyAsync H2D");
    HIP_TRY(ctx, hipEventRecord(ctx->stage_done[k], ctx->copy), "staging event");
    done += len;
  }
  // Later compute-stream work sees the data.
  size_t last = (ctx->next_stage + ctx->stage.size() - 1) % ctx->stage.size();
  HIP_TRY(ctx, hipStreamWaitEvent(ctx->compute, ctx->stage_done[last], 0), "compute waits for upload");
  return LTXW_OK;
}

int ltxw_download(ltxw_ctx* ctx, const void* src, size_t bytes, void* host_dst) {
  if (!ctx) return fail(ctx, LTXW_ERR_INVALID_ARG, "null context");
  if (bytes == 0) return LTXW_OK;
  if (!src || !host_dst) return fail(ctx, LTXW_ERR_INVALID_ARG, "null source or destination");
  if (int rc = check_extent(ctx, src, bytes, "download source")) return rc;
  HIP_TRY(ctx, hipSetDevice(ctx->device), "hipSetDevice");
  HIP_TRY(ctx, hipStreamSynchronize(ctx->compute), "synchronize before download");
  HIP_TRY(ctx, hipMemcpy(host_dst, src, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
  return LTXW_OK;
}

int ltxw_synchronize(ltxw_ctx* ctx) {
  if (!ctx) return fail(ctx, LTXW_ERR_INVALID_ARG, "null context");
  HIP_TRY(ctx, hipStreamSynchronize(ctx->copy), "copy stream synchronize");
  HIP_TRY(ctx, hipStreamSynchronize(ctx->compute), "compute stream synchronize");
  return LTXW_OK;
}

int ltxw_dequant(ltxw_ctx* ctx, const uint8_t* w, int64_t rows, int64_t cols, int fmt,
                 int scale_mode, const float* scales, void* out, int out_dtype) {
  return ltxw_dequant_lora(ctx, w, rows, cols, fmt, scale_mode, scales, nullptr, 0, out, out_dtype);
}

int ltxw_dequant_lora(ltxw_ctx* ctx, const uint8_t* w, int64_t rows, int64_t cols, int fmt,
                      int scale_mode, const float* scales, const ltxw_lora* loras,
                      int n_loras, void* out, int out_dtype) {
  if (!ctx) return fail(ctx, LTXW_ERR_INVALID_ARG, "null context");
  if (n_loras < 0 || n_loras > LTXW_MAX_LORAS)
    return fail(ctx, LTXW_ERR_INVALID_ARG, "n_loras %d outside [0, %d]", n_loras, LTXW_MAX_LORAS);
  if (n_loras > 0 && !loras) return fail(ctx, LTXW_ERR_INVALID_ARG, "null LoRA array");
  ltxw_tensor_desc d{};
  d.w = w;
  d.out = out;
  d.scales = scales;
  d.rows = rows;
  d.cols = cols;
  d.fmt = fmt;
  d.scale_mode = scale_mode;
  d.out_dtype = out_dtype;
  d.n_loras = n_loras;
  for (int l = 0; l < n_loras; ++l) d.loras[l] = loras[l];
  return ltxw::run_descs(ctx, &d, 1);
}

int ltxw_dequant_lora_grouped(ltxw_ctx* ctx, const ltxw_tensor_desc* descs, int n) {
  if (!ctx) return fail(ctx, LTXW_ERR_INVALID_ARG, "null context");
  if (n < 0 || (n > 0 && !descs)) return fail(ctx, LTXW_ERR_INVALID_ARG, "invalid descriptor array");
  return ltxw::run_descs(ctx, descs, n);
}

int ltxw_dequant_lora_grouped_noalloc(ltxw_ctx* ctx, const ltxw_tensor_desc* descs, int n) {
  if (!ctx) return fail(ctx, LTXW_ERR_INVALID_ARG, "null context");
  if (n < 0 || (n > 0 && !descs)) return fail(ctx, LTXW_ERR_INVALID_ARG, "invalid descriptor array");
  if (n > LTXW_NOALLOC_MAX_DESCS)
    return fail(ctx, LTXW_ERR_INVALID_ARG, "%d descriptors exceed the allocation-free call's limit of %d", n,
                LTXW_NOALLOC_MAX_DESCS);
  return ltxw::run_descs(ctx, descs, n, nullptr, true);
}

}  // extern "C"
