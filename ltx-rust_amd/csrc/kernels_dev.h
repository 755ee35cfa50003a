// Device code shared by the kernel translation units (kernels.hip,
// kernels_multi.hip): element helpers and the pieces of the fused pair
// schedule. Everything has internal linkage in each unit. CDNA4 (gfx950, wave64).
//
// Numerics (match ltx-rust's read path, crates/ltx-weights/src/store.rs:479-521):
//   deq  = fma(scale, decode(byte), 0)   store.rs:498-508 (the "+0" turns -0 into +0)
//   out  = deq + sum_l coeff_l * (B_l @ A_l)  store.rs:767-793 (order differs: MFMA)
//   bf16 = round-to-nearest-even, NaN quiet with sign kept (v_cvt_pk_bf16_f32)
// The hardware FP8 converts equal the closed form of fp8.rs:90-158 on every
// finite and infinite code; for NaN codes they return 0xFFC00000 where the
// reference returns f32::NAN (0x7FC00000), so NaN results are canonicalised.
#pragma once

#include "kernels.h"

namespace ltxw {
namespace {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr uint32_t kCanonNaN = 0x7FC00000u;

__device__ __forceinline__ float canon_nan(float x) {
  return __builtin_isnan(x) ? __builtin_bit_cast(float, kCanonNaN) : x;
}

// Accumulates x * 0 into t: t becomes NaN once any x is NaN (or infinite,
// whose product with 0 is NaN too; for those the canonicalisation below is a
// no-op, so the false alarm costs only time).
__device__ __forceinline__ float nan_probe(float t, float x) { return __builtin_fmaf(x, 0.0f, t); }

// True when any lane's probe accumulators hold a NaN: one wave-wide compare.
// (A ballot per value kept one 64-bit mask per value live in SGPRs; the fused
// epilogue's 64 of them spilled some 350 SGPRs into VGPR lanes.)
__device__ __forceinline__ bool any_nan_wave(float t0, float t1, float t2, float t3) {
  return __builtin_amdgcn_ballot_w64(__builtin_isnan((t0 + t1) + (t2 + t3))) != 0;
}

// Canonicalise the NaNs among n values, paying only an FMA per value when the
// whole wave holds none (the usual case); the selects run only if it does.
template <int N>
__device__ __forceinline__ void canon_nan_wave(float* v) {
  float t[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int j = 0; j < N; ++j) t[j & 3] = nan_probe(t[j & 3], v[j]);
  if (any_nan_wave(t[0], t[1], t[2], t[3])) {
#pragma unroll
    for (int j = 0; j < N; ++j) v[j] = canon_nan(v[j]);
  }
}

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  bf16x2 r = __builtin_convertvector((f32x2){a, b}, bf16x2);
  return __builtin_bit_cast(uint32_t, r);
}

// Four FP8 bytes of `word` (little-endian) -> four f32.
__device__ __forceinline__ void decode4(uint32_t word, int fmt, float* v) {
  f32x2 lo, hi;
  if (fmt == 0) {
    lo = __builtin_amdgcn_cvt_pk_f32_fp8(word, false);
    hi = __builtin_amdgcn_cvt_pk_f32_fp8(word, true);
  } else {
    lo = __builtin_amdgcn_cvt_pk_f32_bf8(word, false);
    hi = __builtin_amdgcn_cvt_pk_f32_bf8(word, true);
  }
  v[0] = lo[0];
  v[1] = lo[1];
  v[2] = hi[0];
  v[3] = hi[1];
}

__device__ __forceinline__ float decode1(uint32_t byte, int fmt) {
  float v[4];
  decode4(byte, fmt, v);
  return v[0];
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __builtin_bit_cast(float, (uint32_t)h << 16);
}

// IEEE binary16 -> f32, exact; a NaN keeps sign and payload and gets the
// quiet bit (as `half`'s f16::to_f32, store.rs:690-705).
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  if ((h & 0x7C00u) == 0x7C00u && (h & 0x3FFu))
    return __builtin_bit_cast(float, ((uint32_t)(h & 0x8000u) << 16) | 0x7FC00000u | ((uint32_t)(h & 0x3FFu) << 13));
  return (float)__builtin_bit_cast(_Float16, h);
}

// f32 -> bf16, round to nearest even; a NaN keeps sign and the top payload
// bits and gets the quiet bit (half's bf16::from_f32).
__device__ __forceinline__ uint16_t bf16_rne(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
  return (uint16_t)(pack_bf16(v, 0.0f) & 0xFFFFu);
}

// Element e of a LoRA factor of element type dt (0 bf16, 1 f32, 2 f16,
// 3 e4m3fn, 4 e5m2), widened exactly as lora.rs:176-209 does.
__device__ __forceinline__ float load_factor(const void* p, int dt, uint64_t e) {
  switch (dt) {
    case 0: return bf16_to_f32(reinterpret_cast<const uint16_t*>(p)[e]);
    case 1: return reinterpret_cast<const float*>(p)[e];
    case 2: return f16_to_f32(reinterpret_cast<const uint16_t*>(p)[e]);
    default: return canon_nan(decode1(reinterpret_cast<const uint8_t*>(p)[e], dt - 3));
  }
}

// Element e of a base tensor in any of the accepted formats
// (0 e4m3fn, 1 e5m2, 2 bf16, 3 f16, 4 f32; store.rs:672-729).
__device__ __forceinline__ float load_base(const JobDev& J, uint64_t e) {
  switch (J.fmt) {
    case 0:
    case 1: return canon_nan(decode1(J.w[e], J.fmt));
    case 2: return bf16_to_f32(reinterpret_cast<const uint16_t*>(J.w)[e]);
    case 3: return f16_to_f32(reinterpret_cast<const uint16_t*>(J.w)[e]);
    default: return reinterpret_cast<const float*>(J.w)[e];
  }
}

// Pointers read out of job descriptors are generic; marking them global makes
// the compiler emit global_load/global_store (not flat_*, which also count
// against the LDS counter and skip the global addressing modes).
template <typename T>
__device__ __forceinline__ __attribute__((address_space(1))) T* G(T* p) {
  return (__attribute__((address_space(1))) T*)(p);
}

// Workgroups are dispatched round-robin over the 8 XCDs; map them so that each
// XCD takes a contiguous range of logical tiles (tiles of one row band share
// their LoRA B rows in that XCD's L2). A bijection on [0, n). Launches of up
// to kRemapMinGrid workgroups (a few layers, resident at once or nearly)
// keep the dispatch order: measured 2-5% faster there (one 4096 x 4096 layer
// 12.5 -> 11.9 us), while the remap wins from about a DiT block up
// (kRemapMinGrid, kernels.h).
// Launches of at least this many workgroups use the B-fragment pair swap
// (BSW, below): measured 2% faster on two 4096 x 4096 layers (1024
// workgroups), 1.5-2% on four layers or an FFN matrix (2048), 1-3% per DiT
// block at rank 64 and 5-7% at rank 128, against 0.1-1 us slower on one
// layer (512 workgroups, all resident at once).
constexpr int64_t kSwapMinGrid = 1024;
// Single-LoRA launches of at most this many workgroups (two per CU: every
// workgroup starts at once) request the first unit's FP8 bytes before the
// factors: one 4096 x 4096 layer 11.8-12.2 -> 11.7-11.8 us; from four layers
// up the factors-first order is 1-3% faster.
constexpr int64_t kWFirstMaxGrid = 512;
// `main`: the workgroups of the launch's pair jobs. Workgroups from `main` on
// (the single-unit jobs at the launch's end) keep their order, so the last
// workgroups each XCD starts are narrow ones.
__device__ __forceinline__ uint32_t xcd_remap(uint32_t bid, uint32_t n, uint32_t main) {
  if (n <= kRemapMinGrid || bid >= main) return bid;
  constexpr uint32_t kXcd = 8;
  uint32_t per = main / kXcd, rem = main % kXcd;
  uint32_t x = bid % kXcd, k = bid / kXcd;
  return x < rem ? x * (per + 1) + k : rem * (per + 1) + (x - rem) * per + k;
}

// ---------------------------------------------------------------------------
// (b) Fused dequant + LoRA merge.
//
// Work unit: one band of 128 output columns [i0, i0+128) by 128 rows; each of
// a workgroup's 4 waves owns a strip of 32 rows, [r0, r0+32).
//
// LoRA product on v_mfma_f32_16x16x32_bf16 with M = output row o, N = output
// column i, K = rank r, and the N index permuted as i = i0 + 8*n + nb for
// N-block nb (0..7) and MFMA column n (0..15). With the C layout (lane l holds
// column n = l%16 and rows m = 4*(l/16) + v), lane l then owns, for each of
// its 8 rows, the 8 contiguous columns i0 + 8*(l%16) .. +7 across the 8
// N-blocks: the FP8 input (8 bytes per lane) and the bf16 output (16 bytes per
// lane) go straight between registers and HBM, 16 lanes covering 128
// contiguous columns of a row, with no LDS relayout.
//   A operand (o x r): LoRA B rows, 16-byte loads (r contiguous), from L2.
//   B operand (r x i): LoRA A transposed, staged per work unit in LDS as
//                      AT[slot][k] with slot = nb*16 + n (consecutive lanes
//                      read consecutive slots: conflict-free 128-bit reads).
// Several LoRAs are staged side by side along k (each padded to 32).
//
// Issue order is latency order: the L2-resident factor loads (A for the LDS
// stage, then every B fragment) go out first, the FP8 bytes and scales from
// HBM last. Loads retire in order, so staging, the barrier and the MFMAs run
// while the HBM data is still in flight. (Single-LoRA launches of at most
// kWFirstMaxGrid workgroups request the first unit's FP8 bytes first.)
// ---------------------------------------------------------------------------
// Job records are read with scalar loads through constant-address-space
// pointers, from the kernel's argument segment (records inline in the
// JobTable argument) or from the device table. Both are read-only for the
// launch's lifetime.
using CByte = const __attribute__((address_space(4))) unsigned char;
template <typename T>
__device__ __forceinline__ T kload(CByte* p) {
  static_assert(sizeof(T) % 4 == 0, "whole dwords");
  struct Raw {
    uint32_t w[sizeof(T) / 4];
  } r;
#pragma unroll
  for (int k = 0; k < (int)(sizeof(T) / 4); ++k)
    r.w[k] = *reinterpret_cast<const __attribute__((address_space(4))) uint32_t*>(p + 4 * k);
  return __builtin_bit_cast(T, r);
}

// The record of the job that owns workgroup `wg`: the last one whose
// unit_begin is <= wg (records in ascending unit_begin). Inline tables of up
// to kInlineBegins jobs: a count over JobTable::begins (one load, no
// dependent search); device tables: a binary search over the records.
template <int KS>
__device__ __forceinline__ CByte* job_record(const JobTable& t, uint32_t wg) {
  constexpr uint32_t S = sizeof(FusedJob) + KS * sizeof(StepDev);
  CByte* karg = (CByte*)__builtin_amdgcn_kernarg_segment_ptr();
  if (!t.table && t.n_jobs <= kInlineBegins) {
    uint32_t idx = 0;
#pragma unroll
    for (int j = 1; j < kInlineBegins; ++j) idx += t.begins[j] <= wg ? 1u : 0u;
    return karg + offsetof(JobTable, inl) + idx * S;
  }
  CByte* base = t.table ? (CByte*)(uint64_t)t.table : karg + offsetof(JobTable, inl);
  uint32_t lo = 0, hi = (uint32_t)t.n_jobs - 1;
  while (lo < hi) {
    const uint32_t mid = (lo + hi + 1) >> 1;
    if (kload<uint32_t>(base + mid * S + offsetof(FusedJob, unit_begin)) <= wg) lo = mid;
    else hi = mid - 1;
  }
  return base + lo * S;
}

__device__ __forceinline__ StepDev job_step(CByte* rec, int s) {
  return kload<StepDev>(rec + sizeof(FusedJob) + s * sizeof(StepDev));
}

// Loads and stores at a 32-bit byte offset from a wave-uniform base pointer,
// so the compiler can use the SGPR-base + VGPR-offset addressing mode (one
// VGPR of address per lane, no 64-bit address arithmetic). The host routes
// tensors whose byte extents do not fit 32 bits to the generic kernel.
template <typename T>
__device__ __forceinline__ T ld_at(const void* base, uint32_t off) {
  return *reinterpret_cast<const __attribute__((address_space(1))) T*>(
      (const __attribute__((address_space(1))) char*)base + off);
}
template <typename T>
__device__ __forceinline__ T ld_nt_at(const void* base, uint32_t off) {
  return __builtin_nontemporal_load(reinterpret_cast<const __attribute__((address_space(1))) T*>(
      (const __attribute__((address_space(1))) char*)base + off));
}
template <typename T>
__device__ __forceinline__ void st_nt_at(void* base, uint32_t off, T v) {
  __builtin_nontemporal_store(v, reinterpret_cast<__attribute__((address_space(1))) T*>(
                                     (__attribute__((address_space(1))) char*)base + off));
}

// ---------------------------------------------------------------------------
// (b') Workgroup schedule: two vertically adjacent work units of one band per
// workgroup, in straight-line code. A^T is staged once for both; the second
// unit's FP8 bytes are requested with the first unit's, and its L2-resident
// factor loads go out while the first unit's epilogue runs, so the second
// unit's HBM latency hides behind the first unit's LoRA chain.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t uni(uint32_t x) { return __builtin_amdgcn_readfirstlane(x); }
template <typename T>
__device__ __forceinline__ T* uni_ptr(T* p) {
  const uint64_t v = (uint64_t)p;
  return (T*)(((uint64_t)uni((uint32_t)(v >> 32)) << 32) | uni((uint32_t)v));
}

// The fields of one single-LoRA job the pipelined kernel uses, wave-uniform.
struct PJ {
  const uint8_t* w;
  void* out;
  const float* scales;
  const uint16_t* a;
  const uint16_t* b;
  uint32_t rows, cols, rank, bands_n, scale_mode, fmt;
  float coeff;
  uint32_t cmul;  // coeff applies (coeff != 1)
  uint32_t unit_begin;
  float tscale;   // the per-tensor scale (scale_mode 1), else 1
  uint32_t single;  // one unit per workgroup
};

template <int KS>
__device__ __forceinline__ PJ pj_load(const JobTable& t, uint32_t wg) {
  PJ p;
  if (t.n_jobs == 1) {
    // One-job launches read their JobDev, which sits at a fixed place in
    // the kernel arguments (its loads go out with the launch header's).
    const JobDev& J = t.one;
    p.w = uni_ptr(J.w);
    p.out = uni_ptr(J.out);
    p.scales = uni_ptr(J.scales);
    p.a = uni_ptr(J.lora[0].a);
    p.b = uni_ptr(J.lora[0].b);
    p.rows = uni((uint32_t)J.rows);
    p.cols = uni((uint32_t)J.cols);
    p.rank = uni((uint32_t)J.lora[0].rank);
    p.bands_n = uni((uint32_t)J.bands_n);
    p.scale_mode = uni((uint32_t)J.scale_mode);
    p.fmt = uni((uint32_t)J.fmt);
    p.coeff = __builtin_bit_cast(float, uni(__builtin_bit_cast(uint32_t, J.coeff_out)));
    p.cmul = uni(J.cmul);
    p.unit_begin = uni((uint32_t)J.unit_begin);
    p.single = 0;  // a split launch has several jobs
  } else {
    CByte* rec = job_record<KS>(t, wg);
    const FusedJob J = kload<FusedJob>(rec);
    const StepDev s0 = job_step(rec, 0);  // step 0 starts at the LoRA's B and A
    p.w = J.w;
    p.out = J.out;
    p.scales = J.scales;
    p.a = reinterpret_cast<const uint16_t*>(s0.a);
    p.b = reinterpret_cast<const uint16_t*>(s0.b);
    p.rows = J.rows;
    p.cols = J.cols;
    p.rank = s0.rank;
    p.bands_n = J.bands_n;
    p.scale_mode = J.scale_mode;
    p.fmt = J.fmt;
    p.coeff = J.coeff_out;
    p.cmul = J.cmul;
    p.unit_begin = J.unit_begin;
    p.single = J.single;
  }
  // One uniform load at the start: no per-lane load in the scale branch of
  // the factor issue (a vector load on one path only costs waits on both).
  p.tscale = p.scale_mode == 1 ? *G(uni_ptr(p.scales)) : 1.0f;
  return p;
}

template <int KS>
struct Frag {
  using Wv = u32x2;
  bf16x8 bf[KS][2];
  Wv wv[8];
  float sc[8];
};
template <int KS>
struct Stage {
  u32x4 lo[KS], hi[KS];
};

// A^T staging: for K-step t, thread tid loads ranks 32 t + 2 (tid % 16) and
// +1 of A for the 8 columns i0 + 8 g .. +7 of column group g and stores them
// into AT[slot][32 t + ..] with slot = (i % 8) * 16 + i / 8 for local column i.
// A wave's load covers 16 A rows x 64 bytes; A's row stride is a multiple of
// 128 bytes, so with g = tid / 16 all 16 pieces would sit at one offset of
// their 128-byte lines (the pattern the B-fragment pair swap avoids). Odd
// rank pairs take the partner wave's column groups instead (g = tid / 16 ^ 4,
// a bijection), so each load alternates between the two halves of the lines:
// one 4096 x 4096 layer 11.5 -> 11.2 us, a DiT block -0.8%.
__device__ __forceinline__ uint32_t a_group(int tid, uint32_t half_flip) {
  return (uint32_t)(tid >> 4) ^ ((uint32_t)(tid & 1) * half_flip);
}

template <int KS>
__device__ __forceinline__ void pp_issue_a(const PJ& J, uint32_t i0, int tid, Stage<KS>& st) {
  const int sq = tid & 15;
  const uint32_t scol = i0 + 8 * a_group(tid, 4);
  const bool scol_ok = scol < J.cols;
#pragma unroll
  for (int t = 0; t < KS; ++t) {
    const uint32_t k = 32 * t + 2 * sq;
    st.lo[t] = (u32x4){0u, 0u, 0u, 0u};
    st.hi[t] = st.lo[t];
    if (scol_ok && k < J.rank) st.lo[t] = ld_at<u32x4>(J.a, 2 * (k * J.cols + scol));
    if (scol_ok && k + 1 < J.rank) st.hi[t] = ld_at<u32x4>(J.a, 2 * ((k + 1) * J.cols + scol));
  }
}

// B-fragment pair swap (BSW). One B-fragment load covers 16 rows x 64 bytes
// (a K-step of 32 bf16 ranks). When the row stride (rank x 2 bytes) is a
// multiple of 128, those 16 pieces sit at the same offset in their 128-byte
// lines, and such loads measured 7% slower per DiT block at rank 128 than
// with a padded stride. With the swap, the two loads of a step pair (t, t ^ 1)
// fetch step t ^ 1's piece on odd rows instead, so each load alternates
// between the two halves of the lines; the MFMA takes each odd row's operand
// from its partner's register. Same data, same arithmetic: the output is
// bit-identical. It costs a little in a launch that runs as one round of
// workgroups, so it is used from kSwapMinGrid workgroups up.
template <int KS, bool BSW>
__device__ __forceinline__ bool pp_swap_lane(const PJ& J, int ln) {
  if constexpr (BSW && KS % 2 == 0) return (J.rank % 64 == 0) && (ln & 1);
  else return false;
}

template <int KS, bool FULL, bool BSW = false>
__device__ __forceinline__ void pp_issue_f(const PJ& J, uint32_t i0, uint32_t g0, int tid, Frag<KS>& f) {
  const int lane = tid & 63, wave = tid >> 6, ln = lane & 15, lg = lane >> 4;
  const uint32_t rows = J.rows;
  const uint32_t r0 = g0 + kStripRows * wave;
  const bool swl = pp_swap_lane<KS, BSW>(J, ln);
#pragma unroll
  for (int t = 0; t < KS; ++t) {
    const uint32_t kk = 32 * (swl ? (t ^ 1) : t) + 8 * lg;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const uint32_t ob = r0 + 16 * mb + ln;
      f.bf[t][mb] = (bf16x8){};
      if (kk < J.rank && (FULL || ob < rows)) f.bf[t][mb] = ld_at<bf16x8>(J.b, 2 * (ob * J.rank + kk));
    }
  }
  const uint32_t rl = r0 + 4 * lg;
  if (J.scale_mode == 2) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const uint32_t rb = rl + 16 * mb;
      if (FULL || rb + 3 < rows) {
        const f32x4 q = ld_at<f32x4>(J.scales, 4 * rb);
#pragma unroll
        for (int v = 0; v < 4; ++v) f.sc[4 * mb + v] = q[v];
      } else {
#pragma unroll
        for (int v = 0; v < 4; ++v) f.sc[4 * mb + v] = rb + v < rows ? ld_at<float>(J.scales, 4 * (rb + v)) : 1.0f;
      }
    }
  } else {
#pragma unroll
    for (int g = 0; g < 8; ++g) f.sc[g] = J.tscale;
  }
}

// (FragT: any fragment set with the wv[8] / sc[8] members.)
// The base bytes of 8 elements: u32x2 for FP8, u32x4 for 16-bit formats (the
// type of FragT::wv's elements says which).
template <int KS, bool FULL, class FragT>
__device__ __forceinline__ void pp_issue_w(const PJ& J, uint32_t i0, uint32_t g0, int tid, FragT& f) {
  using W = typename FragT::Wv;
  constexpr uint32_t esz = sizeof(W) / 8;  // bytes per element
  const int lane = tid & 63, wave = tid >> 6, ln = lane & 15, lg = lane >> 4;
  const uint32_t rows = J.rows, cols = J.cols;
  const uint32_t r0 = g0 + kStripRows * wave;
  const uint32_t rl = r0 + 4 * lg;
  const uint32_t ecol = i0 + 8 * ln;
  const bool col_ok = FULL || ecol < cols;
  const uint32_t e0 = rl * cols + ecol;
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    const uint32_t dr = 16 * (g >> 2) + (g & 3);
    f.wv[g] = W{};
    if (col_ok && (FULL || rl + dr < rows)) f.wv[g] = ld_nt_at<W>(J.w, esz * (e0 + dr * cols));
  }
}

// 8 base elements -> f32: FP8 through the hardware converts (FMT 0 e4m3fn,
// 1 e5m2), bf16 (2) by a shift, f16 (3) by the hardware convert; all exact.
template <int FMT, class W>
__device__ __forceinline__ void decode8(const W& w, float* x) {
  if constexpr (FMT <= 1) {
    decode4(w[0], FMT, x);
    decode4(w[1], FMT, x + 4);
  } else if constexpr (FMT == 2) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      x[2 * q] = __builtin_bit_cast(float, w[q] << 16);
      x[2 * q + 1] = __builtin_bit_cast(float, w[q] & 0xFFFF0000u);
    }
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      x[2 * q] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[q] & 0xFFFFu));
      x[2 * q + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[q] >> 16));
    }
  }
}

template <int KS>
__device__ __forceinline__ void pp_stage(const Stage<KS>& st, uint16_t* AT, int ld, int tid) {
  const int sq = tid & 15;
#pragma unroll
  for (int t = 0; t < KS; ++t)
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const uint32_t pair = __builtin_amdgcn_perm(st.hi[t][jj >> 1], st.lo[t][jj >> 1],
                                                  (jj & 1) ? 0x07060302u : 0x05040100u);
      *reinterpret_cast<uint32_t*>(&AT[(jj * 16 + a_group(tid, 4)) * ld + 32 * t + 2 * sq]) = pair;
    }
}

template <int KS>
struct Acc {
  f32x4 v[2][8];
};

// K-step T of the swapped MFMA chain (template recursion keeps every register
// index a compile-time constant; a computed index would put Frag in scratch).
template <int T, int KS>
__device__ __forceinline__ void pp_mfma_swapped(const Frag<KS>& f, const uint16_t* AT, int ld, int ln, int lg,
                                                bool swl, Acc<KS>& a) {
  if constexpr (T < KS) {
    constexpr int TP = T ^ 1;  // KS is even
    const bf16x8 b0 = swl ? f.bf[TP][0] : f.bf[T][0];
    const bf16x8 b1 = swl ? f.bf[TP][1] : f.bf[T][1];
    const int kk = 32 * T + 8 * lg;
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
      const bf16x8 at = *reinterpret_cast<const bf16x8*>(&AT[(nb * 16 + ln) * ld + kk]);
      a.v[0][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(b0, at, a.v[0][nb], 0, 0, 0);
      a.v[1][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(b1, at, a.v[1][nb], 0, 0, 0);
    }
    pp_mfma_swapped<T + 1, KS>(f, AT, ld, ln, lg, swl, a);
  }
}

template <int KS, bool BSW = false>
__device__ __forceinline__ void pp_mfma(const PJ& J, const Frag<KS>& f, const uint16_t* AT, int ld, int tid,
                                        Acc<KS>& a) {
  const int lane = tid & 63, ln = lane & 15, lg = lane >> 4;
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) a.v[mb][nb] = (f32x4){0.f, 0.f, 0.f, 0.f};
  if constexpr (BSW && KS % 2 == 0) {
    pp_mfma_swapped<0, KS>(f, AT, ld, ln, lg, pp_swap_lane<KS, BSW>(J, ln), a);
  } else {
#pragma unroll
    for (int t = 0; t < KS; ++t) {
      const int kk = 32 * t + 8 * lg;
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) {
        const bf16x8 at = *reinterpret_cast<const bf16x8*>(&AT[(nb * 16 + ln) * ld + kk]);
        a.v[0][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f.bf[t][0], at, a.v[0][nb], 0, 0, 0);
        a.v[1][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f.bf[t][1], at, a.v[1][nb], 0, 0, 0);
      }
    }
  }
}

// PROBE: the epilogue's NaN test as FMA probes and one wave-wide compare
// (launches of more than one round of workgroups: DiT block 152.7 -> 150.3 us,
// mixed block 266 -> 260 us, against one 64-bit ballot mask per value, which
// the compiler kept live in SGPRs and spilled to VGPR lanes). One-round
// launches keep the per-value ballots: with the probe one 4096 x 4096 layer
// took 12.9 us instead of 11.7, and with an integer-max test (no SGPR spills
// either) 13.2 us (alternating runs on one machine; the compiler lays that
// schedule's epilogue and second unit out differently, and which part of the
// new layout costs the time was not isolated).
template <bool F32OUT, int KS, bool FULL, int FMT, bool PROBE, class FragT>
__device__ __forceinline__ void pp_epilogue(const PJ& J, const FragT& f, Acc<KS>& a, uint32_t i0, uint32_t g0,
                                            int tid) {
  const int lane = tid & 63, wave = tid >> 6, ln = lane & 15, lg = lane >> 4;
  const uint32_t rows = J.rows, cols = J.cols;
  const uint32_t r0 = g0 + kStripRows * wave;
  const float c = J.coeff;
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) {
    // A flag from the job, not a test of c: the compiler would turn
    // `if (c != 1) v *= c` into an unconditional multiply.
    if (J.cmul) {
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) a.v[mb][nb] *= c;
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int g = 4 * mb + v;
      float x[8];
      decode8<FMT>(f.wv[g], x);
#pragma unroll
      for (int j = 0; j < 8; ++j) a.v[mb][j][v] = __builtin_fmaf(f.sc[g], x[j], a.v[mb][j][v]);
    }
  }
  // FP8 NaN codes decode to the reference's one NaN (f32::NAN); 16-bit bases
  // keep what the arithmetic makes of theirs.
  if constexpr (FMT <= 1) {
    bool any;
    if constexpr (PROBE) {
      float t[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int nb = 0; nb < 8; ++nb)
#pragma unroll
          for (int v = 0; v < 4; ++v) t[v] = nan_probe(t[v], a.v[mb][nb][v]);
      any = any_nan_wave(t[0], t[1], t[2], t[3]);
    } else {
      uint64_t m = 0;
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int nb = 0; nb < 8; ++nb)
#pragma unroll
          for (int v = 0; v < 4; ++v) m |= __builtin_amdgcn_ballot_w64(__builtin_isnan(a.v[mb][nb][v]));
      any = m != 0;
    }
    if (any) {
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int nb = 0; nb < 8; ++nb)
#pragma unroll
          for (int v = 0; v < 4; ++v) a.v[mb][nb][v] = canon_nan(a.v[mb][nb][v]);
    }
  }
  const uint32_t rl = r0 + 4 * lg;
  const uint32_t ecol = i0 + 8 * ln;
  const bool col_ok = FULL || ecol < cols;
  const uint32_t e0 = rl * cols + ecol;
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    const int mb = g >> 2, v = g & 3;
    const uint32_t dr = 16 * mb + v;
    if (col_ok && (FULL || rl + dr < rows)) {
      const uint32_t e = e0 + dr * cols;
      float x[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) x[j] = a.v[mb][j][v];
      if (F32OUT) {
        st_nt_at<f32x4>(J.out, 4 * e, (f32x4){x[0], x[1], x[2], x[3]});
        st_nt_at<f32x4>(J.out, 4 * e + 16, (f32x4){x[4], x[5], x[6], x[7]});
      } else {
        const u32x4 o = {pack_bf16(x[0], x[1]), pack_bf16(x[2], x[3]), pack_bf16(x[4], x[5]), pack_bf16(x[6], x[7])};
        st_nt_at<u32x4>(J.out, 2 * e, o);
      }
    }
  }
}


}  // namespace
}  // namespace ltxw
