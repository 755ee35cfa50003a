// HIP kernels for FP8 dequantisation and the fused dequant + LoRA merge, for
// CDNA4 (gfx950, wave64).
//
// Numerics (match ltx-rust's read path, crates/ltx-weights/src/store.rs:479-521):
//   deq  = fma(scale, decode(byte), 0)   store.rs:498-508 (the "+0" turns -0 into +0)
//   out  = deq + sum_l coeff_l * (B_l @ A_l)  store.rs:767-793 (order differs: MFMA)
//   bf16 = round-to-nearest-even, NaN quiet with sign kept (v_cvt_pk_bf16_f32)
// The hardware FP8 converts equal the closed form of fp8.rs:90-158 on every
// finite and infinite code; for NaN codes they return 0xFFC00000 where the
// reference returns f32::NAN (0x7FC00000), so NaN results are canonicalised.
#include <cstring>

#include "kernels_dev.h"

namespace ltxw {
namespace {

// ---------------------------------------------------------------------------
// (a) Streaming dequant, for tensors above kTileMaxElems elements and the
// unaligned or narrow ones. Each thread handles kChunksPerThread chunks of 16
// FP8 bytes: one 128-bit load, two 128-bit bf16 stores (four for f32).
// Loads are non-temporal (read once); stores are ordinary, which measured
// faster than non-temporal stores for this kernel on MI355X. One chunk per
// thread measured fastest on the large tensors this kernel takes
// (65536 x 4096: 138 us against 145 with two and 149 with four).
// ---------------------------------------------------------------------------
constexpr int kChunksPerThread = 1;

template <int FMT, int SMODE, bool F32OUT>
__global__ __launch_bounds__(256) void k_dequant(DequantArgs a) {
  const uint64_t base = (uint64_t)blockIdx.x * (kChunksPerThread * 256) + threadIdx.x;
  const u32x4* src = reinterpret_cast<const u32x4*>(a.w);
  u32x4 raw[kChunksPerThread];
#pragma unroll
  for (int c = 0; c < kChunksPerThread; ++c) {
    uint64_t idx = base + (uint64_t)c * 256;
    if (idx < a.n_chunks) raw[c] = __builtin_nontemporal_load(src + idx);
  }
  float st = 1.0f;
  if (SMODE == 1) st = a.scales[0];
#pragma unroll
  for (int c = 0; c < kChunksPerThread; ++c) {
    uint64_t idx = base + (uint64_t)c * 256;
    if (idx >= a.n_chunks) break;
    float v[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) decode4(raw[c][q], FMT, v + 4 * q);
    if (SMODE == 1) {
#pragma unroll
      for (int j = 0; j < 16; ++j) v[j] = __builtin_fmaf(st, v[j], 0.0f);
    } else if (SMODE == 2) {
      // Row of the chunk's first element; with cols >= 16 a chunk spans at
      // most one row boundary, after element `edge`.
      uint64_t e0 = idx * 16;
      uint64_t row0 = a.n <= 0xFFFFFFFFull ? (uint64_t)((uint32_t)e0 / (uint32_t)a.cols) : e0 / a.cols;
      uint64_t edge = (row0 + 1) * a.cols - e0;
      float s0 = a.scales[row0];
      float s1 = edge < 16 ? a.scales[row0 + 1] : s0;
#pragma unroll
      for (int j = 0; j < 16; ++j) v[j] = __builtin_fmaf((uint64_t)j < edge ? s0 : s1, v[j], 0.0f);
    }
    canon_nan_wave<16>(v);
    if (F32OUT) {
      f32x4* dst = reinterpret_cast<f32x4*>(a.out) + idx * 4;
#pragma unroll
      for (int q = 0; q < 4; ++q) G(dst)[q] = (f32x4){v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
    } else {
      u32x4* dst = reinterpret_cast<u32x4*>(a.out) + idx * 2;
      u32x4 lo = {pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]), pack_bf16(v[4], v[5]), pack_bf16(v[6], v[7])};
      u32x4 hi = {pack_bf16(v[8], v[9]), pack_bf16(v[10], v[11]), pack_bf16(v[12], v[13]), pack_bf16(v[14], v[15])};
      G(dst)[0] = lo;
      G(dst)[1] = hi;
    }
  }
}

// ---------------------------------------------------------------------------
// Generic path: one thread per element, in the reference's exact order
// (decode, fma(s, v, 0), then per LoRA and rank c = coeff*B[o,r];
// w = fma(c, A[r,i], w)), so it is bit-identical to the reference's f32.
// Used for shapes or alignments the vector kernels do not take.
// ---------------------------------------------------------------------------
template <bool F32OUT>
__global__ __launch_bounds__(256) void k_generic(GenericArgs g) {
  uint64_t k = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (k >= g.elem_count) return;
  const JobDev& J = g.job;
  uint64_t e = g.elem_begin + k;
  uint64_t cols = (uint64_t)J.cols;
  uint64_t o = e / cols, i = e % cols;
  float v = load_base(J, e);
  if (J.scale_mode != 0) {
    const float s = J.scales[J.scale_mode == 2 ? o : 0];
    v = g.plain_scale ? s * v : __builtin_fmaf(s, v, 0.0f);
  }
  if (g.has_post) v = v * g.post_mul;
#pragma unroll
  for (int l = 0; l < kMaxLoras; ++l) {
    if (l >= J.n_loras) break;
    const LoraDev L = J.lora[l];
    const uint64_t brow = o * (uint64_t)L.rank;
    for (int r = 0; r < L.rank; ++r) {
      float c = L.coeff * load_factor(L.b, L.dtype, brow + r);
      v = __builtin_fmaf(c, load_factor(L.a, L.dtype, (uint64_t)r * cols + i), v);
    }
  }
  // FP8 sources: a NaN can only come from a NaN code (decoded canonical) or
  // the arithmetic, and the reference's is canonical too.
  if (J.fmt <= 1) v = canon_nan(v);
  if (F32OUT)
    reinterpret_cast<float*>(J.out)[e] = v;
  else
    reinterpret_cast<uint16_t*>(J.out)[e] = bf16_rne(v);
}

// ---------------------------------------------------------------------------
// Tiled reference-order kernel: the arithmetic of k_generic (bit-identical to
// the reference's f32), with the LoRA factors staged through LDS.
// Workgroup: 128 columns x 64 rows; thread (cg = tid % 16, rs = tid / 16)
// owns columns i0 + 8*cg .. +7 of rows g0 + rs + 16*k, k < 4. Per LoRA, the
// ranks go in chunks of 32: A[r][band] and B[rows][r] widened to f32 into
// LDS, then every thread runs w = fma(coeff * B[o][r], A[r][i], w) in r order.
// VALU-bound (r FMAs per element); for f32 or mixed-type factors, non-FP8
// bases, odd shapes, coefficients the MFMA path does not take, and bit-exact
// requests.
// ---------------------------------------------------------------------------
constexpr int kExactR = 32;

// Factor element e widened to f32, element type fixed at compile time
// (FDT = kMixedFactors: the LoRA's own, read at run time).
constexpr int kMixedFactors = 5;
template <int FDT>
__device__ __forceinline__ float factor_at(const void* p, int dt, uint64_t e) {
  if constexpr (FDT == kMixedFactors) return load_factor(p, dt, e);
  else if constexpr (FDT == 0) return bf16_to_f32(reinterpret_cast<const uint16_t*>(p)[e]);
  else if constexpr (FDT == 1) return reinterpret_cast<const float*>(p)[e];
  else if constexpr (FDT == 2) return f16_to_f32(reinterpret_cast<const uint16_t*>(p)[e]);
  else return canon_nan(decode1(reinterpret_cast<const uint8_t*>(p)[e], FDT - 3));
}

// LDS slot of band column c in a staged A row: column 8q + 4h + j (q < 16,
// h < 2, j < 4) sits at 64h + 4q + j. Thread cg's columns 8cg .. 8cg + 7 are
// then the two 16-byte pieces at 4cg and 64 + 4cg, and the 16 lanes of one
// piece read 256 contiguous bytes: no bank conflicts (with 8 contiguous
// columns per lane, lanes cg and cg + 4 met in the same banks; rocprof's
// SQ_LDS_BANK_CONFLICT fell 11x, the layer's LDS waits 5x).
__device__ __forceinline__ int exact_slot(int c) {
  return ((c >> 2) & 1) * (kExactCols / 2) + ((c >> 3) << 2) + (c & 3);
}

// Five waves per SIMD (95 VGPRs, no spill) rather than the four the default
// register allocation leaves: one 4096 x 4096 layer at rank 64 51.5 -> 48.5 us,
// a DiT block 660 -> 600 us, both bit-identical.
template <bool F32OUT, int FDT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(5))) void k_exact(ExactArgs g) {
  __shared__ __attribute__((aligned(16))) float As[kExactR][kExactCols];
  __shared__ float Bs[kExactRows][kExactR + 1];
  const JobDev& J = g.job;
  const int tid = threadIdx.x, cg = tid & 15, rs = tid >> 4;
  const uint64_t rows = (uint64_t)J.rows, cols = (uint64_t)J.cols;
  const uint64_t band = blockIdx.x % g.bands_n, grp = blockIdx.x / g.bands_n;
  const uint64_t i0 = band * kExactCols, g0 = grp * kExactRows;
  const uint64_t c0 = i0 + 8 * cg;
  // FP8 rows of 8 whole, aligned elements load as one 8-byte word.
  const bool vec8 = J.fmt <= 1 && c0 + 8 <= cols && (cols & 7) == 0 && (((uintptr_t)J.w) & 7) == 0;
  float acc[4][8];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint64_t o = g0 + rs + 16 * k;
    if (o < rows && vec8) {
      const u32x2 wv = *reinterpret_cast<const u32x2*>(J.w + o * cols + c0);
      decode4(wv[0], J.fmt, acc[k]);
      decode4(wv[1], J.fmt, acc[k] + 4);
      canon_nan_wave<8>(acc[k]);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint64_t i = c0 + j;
        acc[k][j] = (o < rows && i < cols) ? load_base(J, o * cols + i) : 0.0f;
      }
    }
    // Uniform branches around whole loops (not selects per element).
    if (o < rows && J.scale_mode != 0) {
      const float s = J.scales[J.scale_mode == 2 ? o : 0];
      if (g.plain_scale) {
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[k][j] = s * acc[k][j];
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[k][j] = __builtin_fmaf(s, acc[k][j], 0.0f);
      }
    }
    if (o < rows && g.has_post) {
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[k][j] = acc[k][j] * g.post_mul;
    }
  }
  for (int l = 0; l < J.n_loras && l < kMaxLoras; ++l) {
    const LoraDev L = J.lora[l];
    const uint64_t rank = (uint64_t)L.rank;
    for (uint64_t r0 = 0; r0 < rank; r0 += kExactR) {
      __syncthreads();  // the previous chunk has been consumed
      {
        const uint64_t rr = r0 + (tid >> 3);
        const int cc = (tid & 7) * 16;
        // 16 consecutive A elements: two (bf16) or four (f32) 16-byte loads
        // when whole and aligned.
        const bool a_vec = (FDT == 0 || FDT == 1) && rr < rank && i0 + cc + 16 <= cols && (cols & 7) == 0 &&
                           (((uintptr_t)L.a) & 15) == 0;
        if (a_vec) {
          if constexpr (FDT == 0) {
            const u32x4* src = reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(L.a) + rr * cols + i0 + cc);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const u32x4 v = src[h];
#pragma unroll
              for (int hf = 0; hf < 2; ++hf)
                *reinterpret_cast<f32x4*>(&As[tid >> 3][exact_slot(cc + 8 * h + 4 * hf)]) =
                    (f32x4){__builtin_bit_cast(float, v[2 * hf] << 16), __builtin_bit_cast(float, v[2 * hf] & 0xFFFF0000u),
                            __builtin_bit_cast(float, v[2 * hf + 1] << 16),
                            __builtin_bit_cast(float, v[2 * hf + 1] & 0xFFFF0000u)};
            }
          } else if constexpr (FDT == 1) {
            const f32x4* src = reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(L.a) + rr * cols + i0 + cc);
#pragma unroll
            for (int h = 0; h < 4; ++h) *reinterpret_cast<f32x4*>(&As[tid >> 3][exact_slot(cc + 4 * h)]) = src[h];
          }
        } else {
#pragma unroll
          for (int q = 0; q < 16; ++q) {
            const uint64_t ii = i0 + cc + q;
            As[tid >> 3][exact_slot(cc + q)] = (rr < rank && ii < cols) ? factor_at<FDT>(L.a, L.dtype, rr * cols + ii) : 0.0f;
          }
        }
        // Bs holds c = coeff * B[o][r], rounded to f32 once here, exactly
        // as the reference forms it before each row's FMA pass.
        const uint64_t oo = g0 + (tid >> 2);
        const int q0 = (tid & 3) * 8;
        // 8 consecutive B elements: one (bf16) or two (f32) 16-byte loads when
        // whole and aligned.
        const bool b_vec = (FDT == 0 || FDT == 1) && oo < rows && r0 + q0 + 8 <= rank && (rank & 7) == 0 &&
                           (((uintptr_t)L.b) & 15) == 0;
        if (b_vec) {
          float bv[8];
          if constexpr (FDT == 0) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(L.b) + oo * rank + r0 + q0);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              bv[2 * q] = __builtin_bit_cast(float, v[q] << 16);
              bv[2 * q + 1] = __builtin_bit_cast(float, v[q] & 0xFFFF0000u);
            }
          } else if constexpr (FDT == 1) {
            const f32x4* src = reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(L.b) + oo * rank + r0 + q0);
            const f32x4 v0 = src[0], v1 = src[1];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              bv[q] = v0[q];
              bv[4 + q] = v1[q];
            }
          }
#pragma unroll
          for (int q = 0; q < 8; ++q) Bs[tid >> 2][q0 + q] = L.coeff * bv[q];
        } else {
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            const uint64_t rq = r0 + q0 + q;
            Bs[tid >> 2][q0 + q] =
                (oo < rows && rq < rank) ? L.coeff * factor_at<FDT>(L.b, L.dtype, oo * rank + rq) : 0.0f;
          }
        }
      }
      __syncthreads();
      const int nr = (int)(rank - r0 < (uint64_t)kExactR ? rank - r0 : (uint64_t)kExactR);
      // Zero-padded ranks beyond nr add fma(c, 0, w) = w + 0, which is not
      // the identity on -0; so the loop stops at nr exactly.
#pragma unroll 1
      for (int r = 0; r < nr; ++r) {
        const f32x4 a0 = *reinterpret_cast<const f32x4*>(&As[r][4 * cg]);
        const f32x4 a1 = *reinterpret_cast<const f32x4*>(&As[r][kExactCols / 2 + 4 * cg]);
        const float a[8] = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float c = Bs[rs + 16 * k][r];
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[k][j] = __builtin_fmaf(c, a[j], acc[k][j]);
        }
      }
    }
  }
  // Whole, aligned groups of 8 columns go out as 16-byte stores.
  const bool o_vec = c0 + 8 <= cols && (cols & 7) == 0 && (((uintptr_t)J.out) & 15) == 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint64_t o = g0 + rs + 16 * k;
    if (o >= rows) continue;
    if (J.fmt <= 1 || g.canon_nan) canon_nan_wave<8>(acc[k]);
    if (o_vec) {
      if (F32OUT) {
        f32x4* dst = reinterpret_cast<f32x4*>(reinterpret_cast<float*>(J.out) + o * cols + c0);
        dst[0] = (f32x4){acc[k][0], acc[k][1], acc[k][2], acc[k][3]};
        dst[1] = (f32x4){acc[k][4], acc[k][5], acc[k][6], acc[k][7]};
      } else {
        // The hardware pack is RNE; half's NaN rule (top payload bits, quiet
        // bit set) is applied only when the wave holds a NaN.
        u32x4 v;
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = pack_bf16(acc[k][2 * q], acc[k][2 * q + 1]);
        float t[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < 8; ++j) t[j & 3] = nan_probe(t[j & 3], acc[k][j]);
        if (any_nan_wave(t[0], t[1], t[2], t[3])) {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            v[q] = (uint32_t)bf16_rne(acc[k][2 * q]) | ((uint32_t)bf16_rne(acc[k][2 * q + 1]) << 16);
        }
        *reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(J.out) + o * cols + c0) = v;
      }
      continue;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint64_t i = c0 + j;
      if (i >= cols) continue;
      if (F32OUT) reinterpret_cast<float*>(J.out)[o * cols + i] = acc[k][j];
      else reinterpret_cast<uint16_t*>(J.out)[o * cols + i] = bf16_rne(acc[k][j]);
    }
  }
}

// Two vertically adjacent units of one band (rows [gA, gA + 256)).
// WFIRST (launches of at most kWFirstMaxGrid workgroups): the first unit's
// FP8 bytes are requested before the factors, and the second unit's factor
// fragments go out during the first unit's epilogue. Larger launches of 2
// K-steps and more request both units' factors before any FP8 bytes (loads
// complete in issue order, so the second unit's LoRA product then never
// waits for FP8 bytes); the registers this takes leave two waves per SIMD
// (DiT block 153.0 -> 150.2 us, rank-128 mixed-format block -2%; with one
// K-step the third wave per SIMD is worth more, +1.4%).
template <bool F32OUT, int KS, int FMT, bool FULL, bool BSW, bool WFIRST>
__device__ __forceinline__ void pair_units(const PJ& J, uint16_t* AT, uint32_t i0, uint32_t gA, uint32_t gB,
                                           bool hasB, int tid) {
  constexpr int LD = 32 * KS + 8;
  Stage<KS> st;
  Frag<KS> fa, fb;
  // Raised wave priority while the FP8 bytes are requested: where a wave of
  // another workgroup is in its epilogue on the same SIMD, these loads go
  // out first, so more memory requests are in flight. Alternating runs on
  // one machine: DiT block 149.2 -> 146.9 us with the priority over the whole
  // issue phase, 147.1 -> 146.2 us more with it on the FP8 loads only; one
  // layer (FP8 first) 11.58 -> 11.48 us over the whole issue phase,
  // 11.49 -> 11.37 us more on the FP8 loads only.
  if constexpr (WFIRST) {
    __builtin_amdgcn_s_setprio(2);
    pp_issue_w<KS, FULL>(J, i0, gA, tid, fa);
    __builtin_amdgcn_s_setprio(0);
    pp_issue_a<KS>(J, i0, tid, st);
    pp_issue_f<KS, FULL, BSW>(J, i0, gA, tid, fa);
    __builtin_amdgcn_s_setprio(2);
  } else {
    pp_issue_a<KS>(J, i0, tid, st);
    pp_issue_f<KS, FULL, BSW>(J, i0, gA, tid, fa);
    if constexpr (KS >= 2) pp_issue_f<KS, FULL, BSW>(J, i0, hasB ? gB : gA, tid, fb);
    __builtin_amdgcn_s_setprio(2);
    pp_issue_w<KS, FULL>(J, i0, gA, tid, fa);
  }
  pp_issue_w<KS, FULL>(J, i0, hasB ? gB : gA, tid, fb);
  __builtin_amdgcn_s_setprio(0);
  pp_stage<KS>(st, AT, LD, tid);
  __syncthreads();
  {
    Acc<KS> acc;
    pp_mfma<KS, BSW>(J, fa, AT, LD, tid, acc);
    if constexpr (WFIRST || KS == 1) pp_issue_f<KS, FULL, BSW>(J, i0, hasB ? gB : gA, tid, fb);
    pp_epilogue<F32OUT, KS, FULL, FMT, !WFIRST>(J, fa, acc, i0, gA, tid);
  }
  // Re-read the A^T fragments for the second unit rather than keeping them
  // live (64 VGPRs) across the first unit's epilogue.
  asm volatile("" ::: "memory");
  if (hasB) {
    Acc<KS> acc;
    pp_mfma<KS, BSW>(J, fb, AT, LD, tid, acc);
    pp_epilogue<F32OUT, KS, FULL, FMT, !WFIRST>(J, fb, acc, i0, gB, tid);
  }
}

// One unit per workgroup (the single-unit jobs at a large launch's end):
// the factors-first order of pair_units without the second unit.
template <bool F32OUT, int KS, int FMT, bool FULL, bool BSW>
__device__ __forceinline__ void one_unit(const PJ& J, uint16_t* AT, uint32_t i0, uint32_t g0, int tid) {
  constexpr int LD = 32 * KS + 8;
  Stage<KS> st;
  Frag<KS> f;
  pp_issue_a<KS>(J, i0, tid, st);
  pp_issue_f<KS, FULL, BSW>(J, i0, g0, tid, f);
  __builtin_amdgcn_s_setprio(2);
  pp_issue_w<KS, FULL>(J, i0, g0, tid, f);
  __builtin_amdgcn_s_setprio(0);
  pp_stage<KS>(st, AT, LD, tid);
  __syncthreads();
  Acc<KS> acc;
  pp_mfma<KS, BSW>(J, f, AT, LD, tid, acc);
  pp_epilogue<F32OUT, KS, FULL, FMT, true>(J, f, acc, i0, g0, tid);
}

// One workgroup per unit pair (per unit in a `single` job); the jobs'
// unit_begin count workgroups. BSW: the
// B-fragment pair swap (launches of kSwapMinGrid workgroups and more);
// WFIRST: FP8 bytes before factors (launches of at most kWFirstMaxGrid).
template <bool F32OUT, int KS, bool BSW, bool WFIRST>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(KS == 1 || (KS == 2 && WFIRST) ? 3 : 2))) void k_fused_pair(JobTable tab) {
  extern __shared__ __attribute__((aligned(16))) uint16_t AT[];
  const int tid = threadIdx.x;
  const uint32_t pair = xcd_remap(blockIdx.x, gridDim.x, tab.main_groups);
  const PJ J = pj_load<KS>(tab, pair);
  const uint32_t p = pair - J.unit_begin;
  const uint32_t i0 = (p % J.bands_n) * kBandCols;
  if constexpr (!WFIRST) {
    if (J.single) {
      const uint32_t g0 = (p / J.bands_n) * kUnitRows;
      const bool full1 = g0 + kUnitRows <= J.rows && i0 + kBandCols <= J.cols;
      if (J.fmt == 0) {
        if (full1) one_unit<F32OUT, KS, 0, true, BSW>(J, AT, i0, g0, tid);
        else one_unit<F32OUT, KS, 0, false, BSW>(J, AT, i0, g0, tid);
      } else {
        if (full1) one_unit<F32OUT, KS, 1, true, BSW>(J, AT, i0, g0, tid);
        else one_unit<F32OUT, KS, 1, false, BSW>(J, AT, i0, g0, tid);
      }
      return;
    }
  }
  const uint32_t gA = (p / J.bands_n) * (2 * kWavesPerGroup * kStripRows);
  const uint32_t gB = gA + kWavesPerGroup * kStripRows;
  const bool hasB = gB < J.rows;
  const bool full = gB + kWavesPerGroup * kStripRows <= J.rows && i0 + kBandCols <= J.cols;
  if (J.fmt == 0) {
    if (full) pair_units<F32OUT, KS, 0, true, BSW, WFIRST>(J, AT, i0, gA, gB, hasB, tid);
    else pair_units<F32OUT, KS, 0, false, BSW, WFIRST>(J, AT, i0, gA, gB, hasB, tid);
  } else {
    if (full) pair_units<F32OUT, KS, 1, true, BSW, WFIRST>(J, AT, i0, gA, gB, hasB, tid);
    else pair_units<F32OUT, KS, 1, false, BSW, WFIRST>(J, AT, i0, gA, gB, hasB, tid);
  }
}

// ---------------------------------------------------------------------------
// (a') Tiled dequant: the fused kernels' lane layout without the LoRA. A
// workgroup takes 64 rows x 128 columns of a column band; lane l of wave w
// handles the 8 columns i0 + 8 (l % 16) .. +7 of rows g0 + 16 w + 4 (l / 16)
// + {0..3}. The wave requests its FP8 bytes at raised priority
// (s_setprio 2), so that where several workgroups share a CU a wave's loads
// go out ahead of other waves' conversions and stores. Alternating runs on
// one machine, 200 launches behind the bench's pre-heat (4096 x 4096; FFN
// 16384 x 4096 / 4096 x 16384; 8192 x 8192, us): 128-row tiles, four per
// workgroup, no priority 9.65; 37.0 / 37.0; 38.2. 128-row tiles with the
// priority, one per workgroup 8.9-9.0; 34.9-35.2 / 34.1-34.4; 35.0-35.2,
// two 9.1, four 9.8. 64-row tiles with the priority 8.65-8.68; 35.1 /
// 34.5-34.7; 34.8-34.9. 32-row tiles 10.1; 34.8 / 34.4; 34.7.
// ---------------------------------------------------------------------------
template <int SMODE, bool FULL>
__device__ __forceinline__ void dqt_load(const DequantTileArgs& a, uint32_t i0, uint32_t g0, int tid, u32x2 (&wv)[4],
                                         float (&sc)[4], float tscale) {
  const int lane = tid & 63, wave = tid >> 6, ln = lane & 15, lg = lane >> 4;
  const uint32_t rl = g0 + 16 * wave + 4 * lg;
  const uint32_t ecol = i0 + 8 * ln;
  const bool col_ok = FULL || ecol < a.cols;
  const uint32_t e0 = rl * a.cols + ecol;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    wv[g] = (u32x2){0u, 0u};
    if (col_ok && (FULL || rl + g < a.rows)) wv[g] = ld_nt_at<u32x2>(a.w, e0 + g * a.cols);
  }
  if (SMODE == 2) {
    if (FULL || rl + 3 < a.rows) {
      const f32x4 q = ld_at<f32x4>(a.scales, 4 * rl);
#pragma unroll
      for (int v = 0; v < 4; ++v) sc[v] = q[v];
    } else {
#pragma unroll
      for (int v = 0; v < 4; ++v) sc[v] = rl + v < a.rows ? ld_at<float>(a.scales, 4 * (rl + v)) : 1.0f;
    }
  } else {
#pragma unroll
    for (int g = 0; g < 4; ++g) sc[g] = tscale;
  }
}

template <int FMT, int SMODE, bool F32OUT, bool FULL>
__device__ __forceinline__ void dqt_store(const DequantTileArgs& a, uint32_t i0, uint32_t g0, int tid,
                                          const u32x2 (&wv)[4], const float (&sc)[4]) {
  const int lane = tid & 63, wave = tid >> 6, ln = lane & 15, lg = lane >> 4;
  const uint32_t rl = g0 + 16 * wave + 4 * lg;
  const uint32_t ecol = i0 + 8 * ln;
  const bool col_ok = FULL || ecol < a.cols;
  const uint32_t e0 = rl * a.cols + ecol;
  float x[4][8];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    decode4(wv[g][0], FMT, x[g]);
    decode4(wv[g][1], FMT, x[g] + 4);
    if (SMODE != 0) {
#pragma unroll
      for (int j = 0; j < 8; ++j) x[g][j] = __builtin_fmaf(sc[g], x[g][j], 0.0f);
    }
  }
  canon_nan_wave<32>(&x[0][0]);
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    if (!(col_ok && (FULL || rl + g < a.rows))) continue;
    const uint32_t e = e0 + g * a.cols;
    if (F32OUT) {
      st_nt_at<f32x4>(a.out, 4 * e, (f32x4){x[g][0], x[g][1], x[g][2], x[g][3]});
      st_nt_at<f32x4>(a.out, 4 * e + 16, (f32x4){x[g][4], x[g][5], x[g][6], x[g][7]});
    } else {
      const u32x4 o = {pack_bf16(x[g][0], x[g][1]), pack_bf16(x[g][2], x[g][3]), pack_bf16(x[g][4], x[g][5]),
                       pack_bf16(x[g][6], x[g][7])};
      st_nt_at<u32x4>(a.out, 2 * e, o);
    }
  }
}

template <int FMT, int SMODE, bool F32OUT, bool FULL>
__device__ __forceinline__ void dqt_unit(const DequantTileArgs& a, uint32_t i0, uint32_t g0, int tid, float tscale) {
  u32x2 w[4];
  float sc[4];
  __builtin_amdgcn_s_setprio(2);
  dqt_load<SMODE, FULL>(a, i0, g0, tid, w, sc, tscale);
  __builtin_amdgcn_s_setprio(0);
  dqt_store<FMT, SMODE, F32OUT, FULL>(a, i0, g0, tid, w, sc);
}

template <int FMT, int SMODE, bool F32OUT>
__global__ __launch_bounds__(256) void k_dequant_tile(DequantTileArgs a) {
  const int tid = threadIdx.x;
  const uint32_t p = blockIdx.x;
  const uint32_t i0 = (p % a.bands_n) * kBandCols;
  const uint32_t g0 = (p / a.bands_n) * kTileRows;
  const bool full = g0 + kTileRows <= a.rows && i0 + kBandCols <= a.cols;
  const float tscale = SMODE == 1 ? *G(uni_ptr(a.scales)) : 1.0f;
  if (full) dqt_unit<FMT, SMODE, F32OUT, true>(a, i0, g0, tid, tscale);
  else dqt_unit<FMT, SMODE, F32OUT, false>(a, i0, g0, tid, tscale);
}

template <int FMT, int SMODE>
hipError_t dequant_tile_out(const DequantTileArgs& a, bool f32out, dim3 grid, hipStream_t s) {
  if (f32out)
    hipLaunchKernelGGL((k_dequant_tile<FMT, SMODE, true>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((k_dequant_tile<FMT, SMODE, false>), grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

template <int FMT>
hipError_t dequant_tile_scale(const DequantTileArgs& a, int smode, bool f32out, dim3 grid, hipStream_t s) {
  switch (smode) {
    case 0: return dequant_tile_out<FMT, 0>(a, f32out, grid, s);
    case 1: return dequant_tile_out<FMT, 1>(a, f32out, grid, s);
    default: return dequant_tile_out<FMT, 2>(a, f32out, grid, s);
  }
}

template <int FMT, int SMODE>
hipError_t dequant_dispatch_out(const DequantArgs& a, bool f32out, dim3 grid, hipStream_t s) {
  if (f32out)
    hipLaunchKernelGGL((k_dequant<FMT, SMODE, true>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((k_dequant<FMT, SMODE, false>), grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

template <int FMT>
hipError_t dequant_dispatch_scale(const DequantArgs& a, int smode, bool f32out, dim3 grid, hipStream_t s) {
  switch (smode) {
    case 0: return dequant_dispatch_out<FMT, 0>(a, f32out, grid, s);
    case 1: return dequant_dispatch_out<FMT, 1>(a, f32out, grid, s);
    default: return dequant_dispatch_out<FMT, 2>(a, f32out, grid, s);
  }
}

}  // namespace

hipError_t launch_dequant(const DequantArgs& a, int fmt, int scale_mode, bool f32out,
                          hipStream_t stream) {
  if (a.n_chunks == 0) return hipSuccess;
  uint64_t per_block = (uint64_t)kChunksPerThread * 256;
  dim3 grid((unsigned)((a.n_chunks + per_block - 1) / per_block));
  return fmt == 0 ? dequant_dispatch_scale<0>(a, scale_mode, f32out, grid, stream)
                  : dequant_dispatch_scale<1>(a, scale_mode, f32out, grid, stream);
}

hipError_t launch_dequant_tile(const DequantTileArgs& a, int fmt, int scale_mode, bool f32out,
                               hipStream_t stream) {
  const uint64_t groups = (uint64_t)a.bands_n * ((a.rows + kTileRows - 1) / kTileRows);
  if (groups == 0) return hipSuccess;
  dim3 grid((unsigned)groups);
  return fmt == 0 ? dequant_tile_scale<0>(a, scale_mode, f32out, grid, stream)
                  : dequant_tile_scale<1>(a, scale_mode, f32out, grid, stream);
}

template <int KS, bool BSW, bool WFIRST>
hipError_t launch_fused_sched(const JobTable& t, bool f32out, dim3 grid, size_t lds, hipStream_t stream) {
  if (f32out) hipLaunchKernelGGL((k_fused_pair<true, KS, BSW, WFIRST>), grid, dim3(256), lds, stream, t);
  else hipLaunchKernelGGL((k_fused_pair<false, KS, BSW, WFIRST>), grid, dim3(256), lds, stream, t);
  return hipGetLastError();
}

template <int KS>
hipError_t launch_fused_ks(const JobTable& t, bool f32out, dim3 grid, size_t lds, hipStream_t stream) {
  // The swap pairs the K-steps of one LoRA: an even number of them.
  if constexpr (KS % 2 == 0) {
    if (t.total_units >= kSwapMinGrid) return launch_fused_sched<KS, true, false>(t, f32out, grid, lds, stream);
  }
  if constexpr (KS <= 2) {
    if (t.total_units <= kWFirstMaxGrid) return launch_fused_sched<KS, false, true>(t, f32out, grid, lds, stream);
  }
  return launch_fused_sched<KS, false, false>(t, f32out, grid, lds, stream);
}

hipError_t launch_fused(const JobTable& t, bool f32out, bool multi, int fdt, bool base16, hipStream_t stream) {
  if (t.total_units == 0) return hipSuccess;
  dim3 grid((unsigned)t.total_units);
  const int ks = (t.lds_ld - 8) / 32;  // K-steps of the largest job
  if (multi) return launch_fused_multi(t, f32out, ks, fdt, base16, stream);
  size_t lds = (size_t)kBandCols * (size_t)t.lds_ld * sizeof(uint16_t);
  switch (ks) {
    case 1: return launch_fused_ks<1>(t, f32out, grid, lds, stream);
    case 2: return launch_fused_ks<2>(t, f32out, grid, lds, stream);
    case 3: return launch_fused_ks<3>(t, f32out, grid, lds, stream);
    case 4: return launch_fused_ks<4>(t, f32out, grid, lds, stream);
    case 5: return launch_fused_ks<5>(t, f32out, grid, lds, stream);
    case 6: return launch_fused_ks<6>(t, f32out, grid, lds, stream);
    case 7: return launch_fused_ks<7>(t, f32out, grid, lds, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_fused_multi(const JobTable& t, bool f32out, int ks, int fdt, bool base16, hipStream_t stream) {
  if (base16) return fdt == 0 ? launch_fused_multi_base16(t, f32out, ks, stream) : hipErrorInvalidValue;
  switch (fdt) {
    case 0: return launch_fused_multi_bf16(t, f32out, ks, stream);
    case 2: return launch_fused_multi_f16(t, f32out, ks, stream);
    case 3: return launch_fused_multi_e4m3fn(t, f32out, ks, stream);
    case 4: return launch_fused_multi_e5m2(t, f32out, ks, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_exact(const ExactArgs& a, bool f32out, hipStream_t stream) {
  const uint64_t rows = (uint64_t)a.job.rows;
  const uint64_t groups = (rows + kExactRows - 1) / kExactRows;
  const uint64_t blocks = groups * (uint64_t)a.bands_n;
  if (blocks == 0) return hipSuccess;
  if (blocks > 0x7FFFFFFFull) return hipErrorInvalidValue;
  dim3 grid((unsigned)blocks);
  // One compiled factor type when every LoRA of the tensor shares it.
  int fdt = a.job.n_loras > 0 ? a.job.lora[0].dtype : 0;
  for (int l = 1; l < a.job.n_loras && l < kMaxLoras; ++l)
    if (a.job.lora[l].dtype != fdt) fdt = kMixedFactors;
#define LTXW_EXACT_LAUNCH(F)                                                              \
  if (f32out) hipLaunchKernelGGL((k_exact<true, F>), grid, dim3(256), 0, stream, a);     \
  else hipLaunchKernelGGL((k_exact<false, F>), grid, dim3(256), 0, stream, a);
  switch (fdt) {
    case 0: LTXW_EXACT_LAUNCH(0) break;
    case 1: LTXW_EXACT_LAUNCH(1) break;
    case 2: LTXW_EXACT_LAUNCH(2) break;
    case 3: LTXW_EXACT_LAUNCH(3) break;
    case 4: LTXW_EXACT_LAUNCH(4) break;
    case kMixedFactors: LTXW_EXACT_LAUNCH(kMixedFactors) break;
    default: return hipErrorInvalidValue;
  }
#undef LTXW_EXACT_LAUNCH
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Scratch of the allocation-free grouped call and the kernel that fills it.

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

hipError_t scratch_address(void** ptr) { return hipGetSymbolAddress(ptr, HIP_SYMBOL(scratch)); }

namespace {

constexpr int kFillWords = 224;  // 16-byte words per launch: 3.5 KiB of kernel arguments

struct FillArgs {
  u32x4* dst;
  uint32_t n;  // words of this launch, <= kFillWords
  uint32_t pad[1];
  u32x4 words[kFillWords];
};
static_assert(sizeof(FillArgs) <= 4096, "kernel arguments of one fill launch");

__global__ __launch_bounds__(256) void k_fill_words(FillArgs a) {
  const uint32_t t = threadIdx.x;
  if (t < a.n) a.dst[t] = a.words[t];
}

}  // namespace

hipError_t launch_fill_words(void* dst, const void* src, size_t bytes, hipStream_t stream) {
  if (bytes % 16 != 0 || reinterpret_cast<uintptr_t>(dst) % 16 != 0) return hipErrorInvalidValue;
  const size_t words = bytes / 16;
  for (size_t w0 = 0; w0 < words; w0 += kFillWords) {
    FillArgs a;
    a.dst = reinterpret_cast<u32x4*>(dst) + w0;
    a.n = (uint32_t)std::min<size_t>(kFillWords, words - w0);
    a.pad[0] = 0;
    std::memcpy(static_cast<void*>(a.words), reinterpret_cast<const char*>(src) + 16 * w0, 16 * (size_t)a.n);
    hipLaunchKernelGGL(k_fill_words, dim3(1), dim3(256), 0, stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_generic(const GenericArgs& a, bool f32out, hipStream_t stream) {
  if (a.elem_count == 0) return hipSuccess;
  dim3 grid((unsigned)((a.elem_count + 255) / 256));
  if (f32out) hipLaunchKernelGGL((k_generic<true>), grid, dim3(256), 0, stream, a);
  else hipLaunchKernelGGL((k_generic<false>), grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace ltxw
