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

// Canonicalise the NaNs among n values, paying only a compare per value when
// the whole wave holds none (the usual case): the per-value NaN tests are
// combined into one wave-wide mask, and the selects run only if it is set.
template <int N>
__device__ __forceinline__ void canon_nan_wave(float* v) {
  uint64_t any = 0;
#pragma unroll
  for (int j = 0; j < N; ++j) any |= __builtin_amdgcn_ballot_w64(__builtin_isnan(v[j]));
  if (any) {
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
// 12.5 -> 11.9 us), while the remap wins from about a DiT block up.
constexpr uint32_t kRemapMinGrid = 2048;
__device__ __forceinline__ uint32_t xcd_remap(uint32_t bid, uint32_t n) {
  if (n <= kRemapMinGrid) return bid;
  constexpr uint32_t kXcd = 8;
  uint32_t per = n / kXcd, rem = n % kXcd;
  uint32_t x = bid % kXcd, k = bid / kXcd;
  return x < rem ? x * (per + 1) + k : rem * (per + 1) + (x - rem) * per + k;
}

// ---------------------------------------------------------------------------
// (a) Streaming dequant. Each thread handles kChunksPerThread chunks of 16
// FP8 bytes: one 128-bit load, two 128-bit bf16 stores (four for f32).
// Loads are non-temporal (read once); stores are ordinary, which measured
// faster than non-temporal stores for this kernel on MI355X.
// ---------------------------------------------------------------------------
constexpr int kChunksPerThread = 4;

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
// VALU-bound (r FMAs per element); for adapters whose factors are not bf16,
// non-FP8 bases, odd shapes, and bit-exact requests.
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

template <bool F32OUT, int FDT>
__global__ __launch_bounds__(256) void k_exact(ExactArgs g) {
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
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[k][j] = canon_nan(acc[k][j]);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint64_t i = c0 + j;
        acc[k][j] = (o < rows && i < cols) ? load_base(J, o * cols + i) : 0.0f;
      }
    }
    if (o < rows) {
      const float s = J.scale_mode == 0 ? 1.0f : J.scales[J.scale_mode == 2 ? o : 0];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float v = acc[k][j];
        if (J.scale_mode != 0) v = g.plain_scale ? s * v : __builtin_fmaf(s, v, 0.0f);
        if (g.has_post) v = v * g.post_mul;
        acc[k][j] = v;
      }
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
              for (int q = 0; q < 4; ++q) {
                As[tid >> 3][cc + 8 * h + 2 * q] = __builtin_bit_cast(float, v[q] << 16);
                As[tid >> 3][cc + 8 * h + 2 * q + 1] = __builtin_bit_cast(float, v[q] & 0xFFFF0000u);
              }
            }
          } else if constexpr (FDT == 1) {
            const f32x4* src = reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(L.a) + rr * cols + i0 + cc);
#pragma unroll
            for (int h = 0; h < 4; ++h) *reinterpret_cast<f32x4*>(&As[tid >> 3][cc + 4 * h]) = src[h];
          }
        } else {
#pragma unroll
          for (int q = 0; q < 16; ++q) {
            const uint64_t ii = i0 + cc + q;
            As[tid >> 3][cc + q] = (rr < rank && ii < cols) ? factor_at<FDT>(L.a, L.dtype, rr * cols + ii) : 0.0f;
          }
        }
        // Bs holds c = coeff * B[o][r], rounded to f32 once here, exactly
        // as the reference forms it before each row's FMA pass.
        const uint64_t oo = g0 + (tid >> 2);
        const int q0 = (tid & 3) * 8;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const uint64_t rq = r0 + q0 + q;
          Bs[tid >> 2][q0 + q] =
              (oo < rows && rq < rank) ? L.coeff * factor_at<FDT>(L.b, L.dtype, oo * rank + rq) : 0.0f;
        }
      }
      __syncthreads();
      const int nr = (int)(rank - r0 < (uint64_t)kExactR ? rank - r0 : (uint64_t)kExactR);
      // Zero-padded ranks beyond nr add fma(c, 0, w) = w + 0, which is not
      // the identity on -0; so the loop stops at nr exactly.
#pragma unroll 4
      for (int r = 0; r < nr; ++r) {
        const f32x4 a0 = *reinterpret_cast<const f32x4*>(&As[r][8 * cg]);
        const f32x4 a1 = *reinterpret_cast<const f32x4*>(&As[r][8 * cg + 4]);
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
    if (J.fmt <= 1) {
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[k][j] = canon_nan(acc[k][j]);
    }
    if (o_vec) {
      if (F32OUT) {
        f32x4* dst = reinterpret_cast<f32x4*>(reinterpret_cast<float*>(J.out) + o * cols + c0);
        dst[0] = (f32x4){acc[k][0], acc[k][1], acc[k][2], acc[k][3]};
        dst[1] = (f32x4){acc[k][4], acc[k][5], acc[k][6], acc[k][7]};
      } else {
        u32x4 v;
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = (uint32_t)bf16_rne(acc[k][2 * q]) | ((uint32_t)bf16_rne(acc[k][2 * q + 1]) << 16);
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
// while the HBM data is still in flight.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void load_job(const JobTable& t, uint64_t unit, JobDev& J) {
  if (t.n_jobs == 1) {
    J = t.one;
    return;
  }
  int lo = 0, hi = t.n_jobs - 1;  // last job with begins[j] <= unit
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if ((uint64_t)G(t.begins)[mid] <= unit) lo = mid; else hi = mid - 1;
  }
  // Copy the descriptor as 16-byte global loads (the table is 256-byte aligned).
  static_assert(sizeof(JobDev) % 16 == 0, "JobDev is copied in 16-byte pieces");
  u32x4 raw[sizeof(JobDev) / 16];
  const auto src = G(reinterpret_cast<const u32x4*>(t.jobs + lo));
#pragma unroll
  for (int k = 0; k < (int)(sizeof(JobDev) / 16); ++k) raw[k] = src[k];
  __builtin_memcpy(&J, raw, sizeof(JobDev));
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
};

__device__ __forceinline__ PJ pj_load(const JobTable& t, uint64_t unit) {
  JobDev J;
  load_job(t, unit, J);
  PJ p;
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
  // One uniform load at the start: no per-lane load in the scale branch of
  // the factor issue (a vector load on one path only costs waits on both).
  p.tscale = p.scale_mode == 1 ? *G(uni_ptr(J.scales)) : 1.0f;
  p.coeff = __builtin_bit_cast(float, uni(__builtin_bit_cast(uint32_t, J.coeff_out)));
  p.cmul = uni(J.cmul);
  p.unit_begin = uni((uint32_t)J.unit_begin);
  return p;
}

template <int KS>
struct Frag {
  bf16x8 bf[KS][2];
  u32x2 wv[8];
  float sc[8];
};
template <int KS>
struct Stage {
  u32x4 lo[KS], hi[KS];
};

// A^T staging: for K-step t, thread tid loads ranks 32 t + 2 (tid % 16) and
// +1 of A for the 8 columns i0 + 8 (tid / 16) .. +7 and stores them into
// AT[slot][32 t + ..] with slot = (i % 8) * 16 + i / 8 for local column i.
template <int KS>
__device__ __forceinline__ void pp_issue_a(const PJ& J, uint32_t i0, int tid, Stage<KS>& st) {
  const int sq = tid & 15;
  const uint32_t scol = i0 + 8 * (tid >> 4);
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

template <int KS, bool FULL>
__device__ __forceinline__ void pp_issue_f(const PJ& J, uint32_t i0, uint32_t g0, int tid, Frag<KS>& f) {
  const int lane = tid & 63, wave = tid >> 6, ln = lane & 15, lg = lane >> 4;
  const uint32_t rows = J.rows;
  const uint32_t r0 = g0 + kStripRows * wave;
#pragma unroll
  for (int t = 0; t < KS; ++t) {
    const uint32_t kk = 32 * t + 8 * lg;
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

template <int KS, bool FULL>
__device__ __forceinline__ void pp_issue_w(const PJ& J, uint32_t i0, uint32_t g0, int tid, Frag<KS>& f) {
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
    f.wv[g] = (u32x2){0u, 0u};
    if (col_ok && (FULL || rl + dr < rows)) f.wv[g] = ld_nt_at<u32x2>(J.w, e0 + dr * cols);
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
      *reinterpret_cast<uint32_t*>(&AT[(jj * 16 + (tid >> 4)) * ld + 32 * t + 2 * sq]) = pair;
    }
}

template <int KS>
struct Acc {
  f32x4 v[2][8];
};

template <int KS>
__device__ __forceinline__ void pp_mfma(const Frag<KS>& f, const uint16_t* AT, int ld, int tid, Acc<KS>& a) {
  const int lane = tid & 63, ln = lane & 15, lg = lane >> 4;
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) a.v[mb][nb] = (f32x4){0.f, 0.f, 0.f, 0.f};
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

template <bool F32OUT, int KS, bool FULL, int FMT>
__device__ __forceinline__ void pp_epilogue(const PJ& J, const Frag<KS>& f, Acc<KS>& a, uint32_t i0, uint32_t g0,
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
      decode4(f.wv[g][0], FMT, x);
      decode4(f.wv[g][1], FMT, x + 4);
#pragma unroll
      for (int j = 0; j < 8; ++j) a.v[mb][j][v] = __builtin_fmaf(f.sc[g], x[j], a.v[mb][j][v]);
    }
  }
  {
    uint64_t any = 0;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int nb = 0; nb < 8; ++nb)
#pragma unroll
        for (int v = 0; v < 4; ++v) any |= __builtin_amdgcn_ballot_w64(__builtin_isnan(a.v[mb][nb][v]));
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

template <bool F32OUT, int KS, int FMT>
__device__ __forceinline__ void pp_epilogue_any(const PJ& J, const Frag<KS>& f, Acc<KS>& a, uint32_t i0,
                                                uint32_t g0, int tid) {
  if (g0 + 128 <= J.rows && i0 + 128 <= J.cols) pp_epilogue<F32OUT, KS, true, FMT>(J, f, a, i0, g0, tid);
  else pp_epilogue<F32OUT, KS, false, FMT>(J, f, a, i0, g0, tid);
}

// Two vertically adjacent units of one band (rows [gA, gA + 256)).
template <bool F32OUT, int KS, int FMT, bool FULL>
__device__ __forceinline__ void pair_units(const PJ& J, uint16_t* AT, uint32_t i0, uint32_t gA, uint32_t gB,
                                           bool hasB, int tid) {
  constexpr int LD = 32 * KS + 8;
  Stage<KS> st;
  pp_issue_a<KS>(J, i0, tid, st);
  Frag<KS> fa, fb;
  pp_issue_f<KS, FULL>(J, i0, gA, tid, fa);
  pp_issue_w<KS, FULL>(J, i0, gA, tid, fa);
  pp_issue_w<KS, FULL>(J, i0, hasB ? gB : gA, tid, fb);
  pp_stage<KS>(st, AT, LD, tid);
  __syncthreads();
  {
    Acc<KS> acc;
    pp_mfma<KS>(fa, AT, LD, tid, acc);
    pp_issue_f<KS, FULL>(J, i0, hasB ? gB : gA, tid, fb);
    pp_epilogue<F32OUT, KS, FULL, FMT>(J, fa, acc, i0, gA, tid);
  }
  // Re-read the A^T fragments for the second unit rather than keeping them
  // live (64 VGPRs) across the first unit's epilogue.
  asm volatile("" ::: "memory");
  if (hasB) {
    Acc<KS> acc;
    pp_mfma<KS>(fb, AT, LD, tid, acc);
    pp_epilogue<F32OUT, KS, FULL, FMT>(J, fb, acc, i0, gB, tid);
  }
}

// One workgroup per unit pair; the jobs' unit_begin count pairs.
template <bool F32OUT, int KS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(KS <= 2 ? 3 : 2))) void k_fused_pair(JobTable tab) {
  extern __shared__ __attribute__((aligned(16))) uint16_t AT[];
  const int tid = threadIdx.x;
  const uint32_t pair = xcd_remap(blockIdx.x, gridDim.x);
  const PJ J = pj_load(tab, pair);
  const uint32_t p = pair - J.unit_begin;
  const uint32_t i0 = (p % J.bands_n) * kBandCols;
  const uint32_t gA = (p / J.bands_n) * (2 * kWavesPerGroup * kStripRows);
  const uint32_t gB = gA + kWavesPerGroup * kStripRows;
  const bool hasB = gB < J.rows;
  const bool full = gB + kWavesPerGroup * kStripRows <= J.rows && i0 + kBandCols <= J.cols;
  if (J.fmt == 0) {
    if (full) pair_units<F32OUT, KS, 0, true>(J, AT, i0, gA, gB, hasB, tid);
    else pair_units<F32OUT, KS, 0, false>(J, AT, i0, gA, gB, hasB, tid);
  } else {
    if (full) pair_units<F32OUT, KS, 1, true>(J, AT, i0, gA, gB, hasB, tid);
    else pair_units<F32OUT, KS, 1, false>(J, AT, i0, gA, gB, hasB, tid);
  }
}

// ---------------------------------------------------------------------------
// Several LoRAs per tensor, two units per workgroup. The LoRAs sit side by
// side along K (each padded to 32) and the host describes every K-step
// (StepDev: the step's A rows, B columns, rank and present ranks). One
// accumulator set carries the whole delta: at the last step of LoRA l, with
// LoRA l+1 following, the accumulator is multiplied by q = c_l / c_{l+1}, and
// the epilogue multiplies by the last coefficient:
//   delta = c_last (... ((B_0 A_0) q_0 + B_1 A_1) q_1 ...) = sum_l c_l B_l A_l
// up to a few f32 roundings (the host routes coefficients whose ratios could
// overflow or underflow to the reference-order kernel).
// ---------------------------------------------------------------------------
template <int KS>
struct PJM {
  PJ base;  // coeff / cmul: the last LoRA's coefficient
  const uint16_t* a[KS];
  const uint16_t* b[KS];
  uint32_t rank[KS];
  uint32_t klim[KS];
  float q[KS];
  uint32_t qmask;
};

template <int KS>
__device__ __forceinline__ PJM<KS> pjm_load(const JobTable& t, uint64_t unit) {
  JobDev J;
  load_job(t, unit, J);
  PJM<KS> m;
  m.base.w = uni_ptr(J.w);
  m.base.out = uni_ptr(J.out);
  m.base.scales = uni_ptr(J.scales);
  m.base.a = nullptr;
  m.base.b = nullptr;
  m.base.rows = uni((uint32_t)J.rows);
  m.base.cols = uni((uint32_t)J.cols);
  m.base.rank = 0;
  m.base.bands_n = uni((uint32_t)J.bands_n);
  m.base.scale_mode = uni((uint32_t)J.scale_mode);
  m.base.fmt = uni((uint32_t)J.fmt);
  m.base.tscale = m.base.scale_mode == 1 ? *G(uni_ptr(J.scales)) : 1.0f;
  m.base.coeff = __builtin_bit_cast(float, uni(__builtin_bit_cast(uint32_t, J.coeff_out)));
  m.base.cmul = uni(J.cmul);
  m.base.unit_begin = uni((uint32_t)J.unit_begin);
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    m.a[s] = uni_ptr(J.step[s].a);
    m.b[s] = uni_ptr(J.step[s].b);
    m.rank[s] = uni(J.step[s].rank);
    m.klim[s] = uni(J.step[s].klim);
    m.q[s] = __builtin_bit_cast(float, uni(__builtin_bit_cast(uint32_t, J.step[s].q)));
  }
  m.qmask = uni(J.qmask);
  return m;
}

template <int KS>
__device__ __forceinline__ void pm_issue_a(const PJM<KS>& M, uint32_t i0, int tid, Stage<KS>& st) {
  const int sq = tid & 15;
  const uint32_t cols = M.base.cols;
  const uint32_t scol = i0 + 8 * (tid >> 4);
  const bool scol_ok = scol < cols;
  const uint32_t k = 2 * sq;
#pragma unroll
  for (int t = 0; t < KS; ++t) {
    st.lo[t] = (u32x4){0u, 0u, 0u, 0u};
    st.hi[t] = st.lo[t];
    if (scol_ok && k < M.klim[t]) st.lo[t] = ld_at<u32x4>(M.a[t], 2 * (k * cols + scol));
    if (scol_ok && k + 1 < M.klim[t]) st.hi[t] = ld_at<u32x4>(M.a[t], 2 * ((k + 1) * cols + scol));
  }
}

template <int KS, bool FULL>
__device__ __forceinline__ void pm_issue_f(const PJM<KS>& M, uint32_t g0, int tid, Frag<KS>& f) {
  const int lane = tid & 63, wave = tid >> 6, ln = lane & 15, lg = lane >> 4;
  const uint32_t rows = M.base.rows;
  const uint32_t r0 = g0 + kStripRows * wave;
  const uint32_t kk = 8 * lg;
#pragma unroll
  for (int t = 0; t < KS; ++t) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const uint32_t ob = r0 + 16 * mb + ln;
      f.bf[t][mb] = (bf16x8){};
      if (kk < M.klim[t] && (FULL || ob < rows)) f.bf[t][mb] = ld_at<bf16x8>(M.b[t], 2 * (ob * M.rank[t] + kk));
    }
  }
  const uint32_t rl = r0 + 4 * lg;
  if (M.base.scale_mode == 2) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const uint32_t rb = rl + 16 * mb;
      if (FULL || rb + 3 < rows) {
        const f32x4 q = ld_at<f32x4>(M.base.scales, 4 * rb);
#pragma unroll
        for (int v = 0; v < 4; ++v) f.sc[4 * mb + v] = q[v];
      } else {
#pragma unroll
        for (int v = 0; v < 4; ++v)
          f.sc[4 * mb + v] = rb + v < rows ? ld_at<float>(M.base.scales, 4 * (rb + v)) : 1.0f;
      }
    }
  } else {
#pragma unroll
    for (int g = 0; g < 8; ++g) f.sc[g] = M.base.tscale;
  }
}

template <int KS>
__device__ __forceinline__ void pm_mfma(const PJM<KS>& M, const Frag<KS>& f, const uint16_t* AT, int ld, int tid,
                                        Acc<KS>& a) {
  const int lane = tid & 63, ln = lane & 15, lg = lane >> 4;
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) a.v[mb][nb] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < KS; ++t) {
    const int kk = 32 * t + 8 * lg;
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
      const bf16x8 at = *reinterpret_cast<const bf16x8*>(&AT[(nb * 16 + ln) * ld + kk]);
      a.v[0][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f.bf[t][0], at, a.v[0][nb], 0, 0, 0);
      a.v[1][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f.bf[t][1], at, a.v[1][nb], 0, 0, 0);
    }
    if (t + 1 < KS && (M.qmask & (1u << t))) {
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) a.v[mb][nb] *= M.q[t];
    }
  }
}

template <bool F32OUT, int KS, int FMT, bool FULL>
__device__ __forceinline__ void pair_units_multi(const PJM<KS>& M, uint16_t* AT, uint32_t i0, uint32_t gA,
                                                 uint32_t gB, bool hasB, int tid) {
  constexpr int LD = 32 * KS + 8;
  Stage<KS> st;
  pm_issue_a<KS>(M, i0, tid, st);
  Frag<KS> fa, fb;
  pm_issue_f<KS, FULL>(M, gA, tid, fa);
  pp_issue_w<KS, FULL>(M.base, i0, gA, tid, fa);
  pp_issue_w<KS, FULL>(M.base, i0, hasB ? gB : gA, tid, fb);
  pp_stage<KS>(st, AT, LD, tid);
  __syncthreads();
  {
    Acc<KS> acc;
    pm_mfma<KS>(M, fa, AT, LD, tid, acc);
    pm_issue_f<KS, FULL>(M, hasB ? gB : gA, tid, fb);
    pp_epilogue<F32OUT, KS, FULL, FMT>(M.base, fa, acc, i0, gA, tid);
  }
  asm volatile("" ::: "memory");
  if (hasB) {
    Acc<KS> acc;
    pm_mfma<KS>(M, fb, AT, LD, tid, acc);
    pp_epilogue<F32OUT, KS, FULL, FMT>(M.base, fb, acc, i0, gB, tid);
  }
}

template <bool F32OUT, int KS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void k_fused_pair_multi(JobTable tab) {
  extern __shared__ __attribute__((aligned(16))) uint16_t AT[];
  const int tid = threadIdx.x;
  const uint32_t pair = xcd_remap(blockIdx.x, gridDim.x);
  const PJM<KS> M = pjm_load<KS>(tab, pair);
  const uint32_t p = pair - M.base.unit_begin;
  const uint32_t i0 = (p % M.base.bands_n) * kBandCols;
  const uint32_t gA = (p / M.base.bands_n) * (2 * kWavesPerGroup * kStripRows);
  const uint32_t gB = gA + kWavesPerGroup * kStripRows;
  const bool hasB = gB < M.base.rows;
  const bool full = gB + kWavesPerGroup * kStripRows <= M.base.rows && i0 + kBandCols <= M.base.cols;
  if (M.base.fmt == 0) {
    if (full) pair_units_multi<F32OUT, KS, 0, true>(M, AT, i0, gA, gB, hasB, tid);
    else pair_units_multi<F32OUT, KS, 0, false>(M, AT, i0, gA, gB, hasB, tid);
  } else {
    if (full) pair_units_multi<F32OUT, KS, 1, true>(M, AT, i0, gA, gB, hasB, tid);
    else pair_units_multi<F32OUT, KS, 1, false>(M, AT, i0, gA, gB, hasB, tid);
  }
}

// ---------------------------------------------------------------------------
// (a') Tiled dequant: the fused kernels' tile walk and lane layout without
// the LoRA. A workgroup takes two vertically adjacent 128 x 128 units of a
// column band; lane l of wave w handles, in each unit, the 8 columns
// i0 + 8 (l % 16) .. +7 of rows r0 + 4 (l / 16) + {0..3, 16..19} with
// r0 = g0 + 32 w. Both units' bytes are requested before the first unit is
// converted. Faster than the streaming kernel on tensors of one layer's size
// (a launch that is resident at once); the streaming kernel wins on larger
// ones.
// ---------------------------------------------------------------------------
template <int SMODE, bool FULL>
__device__ __forceinline__ void dqt_load(const DequantTileArgs& a, uint32_t i0, uint32_t g0, int tid, u32x2 (&wv)[8],
                                         float (&sc)[8], float tscale) {
  const int lane = tid & 63, wave = tid >> 6, ln = lane & 15, lg = lane >> 4;
  const uint32_t rl = g0 + kStripRows * wave + 4 * lg;
  const uint32_t ecol = i0 + 8 * ln;
  const bool col_ok = FULL || ecol < a.cols;
  const uint32_t e0 = rl * a.cols + ecol;
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    const uint32_t dr = 16 * (g >> 2) + (g & 3);
    wv[g] = (u32x2){0u, 0u};
    if (col_ok && (FULL || rl + dr < a.rows)) wv[g] = ld_nt_at<u32x2>(a.w, e0 + dr * a.cols);
  }
  if (SMODE == 2) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const uint32_t rb = rl + 16 * mb;
      if (FULL || rb + 3 < a.rows) {
        const f32x4 q = ld_at<f32x4>(a.scales, 4 * rb);
#pragma unroll
        for (int v = 0; v < 4; ++v) sc[4 * mb + v] = q[v];
      } else {
#pragma unroll
        for (int v = 0; v < 4; ++v) sc[4 * mb + v] = rb + v < a.rows ? ld_at<float>(a.scales, 4 * (rb + v)) : 1.0f;
      }
    }
  } else {
#pragma unroll
    for (int g = 0; g < 8; ++g) sc[g] = tscale;
  }
}

template <int FMT, int SMODE, bool F32OUT, bool FULL>
__device__ __forceinline__ void dqt_store(const DequantTileArgs& a, uint32_t i0, uint32_t g0, int tid,
                                          const u32x2 (&wv)[8], const float (&sc)[8]) {
  const int lane = tid & 63, wave = tid >> 6, ln = lane & 15, lg = lane >> 4;
  const uint32_t rl = g0 + kStripRows * wave + 4 * lg;
  const uint32_t ecol = i0 + 8 * ln;
  const bool col_ok = FULL || ecol < a.cols;
  const uint32_t e0 = rl * a.cols + ecol;
  float x[8][8];
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    decode4(wv[g][0], FMT, x[g]);
    decode4(wv[g][1], FMT, x[g] + 4);
    if (SMODE != 0) {
#pragma unroll
      for (int j = 0; j < 8; ++j) x[g][j] = __builtin_fmaf(sc[g], x[g][j], 0.0f);
    }
  }
  canon_nan_wave<64>(&x[0][0]);
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    const uint32_t dr = 16 * (g >> 2) + (g & 3);
    if (!(col_ok && (FULL || rl + dr < a.rows))) continue;
    const uint32_t e = e0 + dr * a.cols;
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
__device__ __forceinline__ void dqt_pair(const DequantTileArgs& a, uint32_t i0, uint32_t gA, uint32_t gB, bool hasB,
                                         int tid, float tscale) {
  u32x2 wa[8], wb[8];
  float sa[8], sb[8];
  dqt_load<SMODE, FULL>(a, i0, gA, tid, wa, sa, tscale);
  if (hasB) dqt_load<SMODE, FULL>(a, i0, gB, tid, wb, sb, tscale);
  dqt_store<FMT, SMODE, F32OUT, FULL>(a, i0, gA, tid, wa, sa);
  if (hasB) dqt_store<FMT, SMODE, F32OUT, FULL>(a, i0, gB, tid, wb, sb);
}

template <int FMT, int SMODE, bool F32OUT>
__global__ __launch_bounds__(256) void k_dequant_tile(DequantTileArgs a) {
  const int tid = threadIdx.x;
  const uint32_t p = blockIdx.x;
  const uint32_t i0 = (p % a.bands_n) * kBandCols;
  const uint32_t gA = (p / a.bands_n) * kPairRows;
  const uint32_t gB = gA + kWavesPerGroup * kStripRows;
  const bool hasB = gB < a.rows;
  const bool full = gA + kPairRows <= a.rows && i0 + kBandCols <= a.cols;
  const float tscale = SMODE == 1 ? *G(uni_ptr(a.scales)) : 1.0f;
  if (full) dqt_pair<FMT, SMODE, F32OUT, true>(a, i0, gA, gB, hasB, tid, tscale);
  else dqt_pair<FMT, SMODE, F32OUT, false>(a, i0, gA, gB, hasB, tid, tscale);
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
  const uint64_t pairs = (uint64_t)a.bands_n * ((a.rows + kPairRows - 1) / kPairRows);
  if (pairs == 0) return hipSuccess;
  dim3 grid((unsigned)pairs);
  return fmt == 0 ? dequant_tile_scale<0>(a, scale_mode, f32out, grid, stream)
                  : dequant_tile_scale<1>(a, scale_mode, f32out, grid, stream);
}

template <int KS>
hipError_t launch_fused_ks(const JobTable& t, bool f32out, bool multi, dim3 grid, size_t lds, hipStream_t stream) {
  if (multi) {
    // Two or more LoRAs pad to at least two K-steps.
    if constexpr (KS >= 2) {
      if (f32out) hipLaunchKernelGGL((k_fused_pair_multi<true, KS>), grid, dim3(256), lds, stream, t);
      else hipLaunchKernelGGL((k_fused_pair_multi<false, KS>), grid, dim3(256), lds, stream, t);
    } else {
      return hipErrorInvalidValue;
    }
  } else {
    if (f32out) hipLaunchKernelGGL((k_fused_pair<true, KS>), grid, dim3(256), lds, stream, t);
    else hipLaunchKernelGGL((k_fused_pair<false, KS>), grid, dim3(256), lds, stream, t);
  }
  return hipGetLastError();
}

hipError_t launch_fused(const JobTable& t, bool f32out, bool multi, hipStream_t stream) {
  if (t.total_units == 0) return hipSuccess;
  dim3 grid((unsigned)t.total_units);
  size_t lds = (size_t)kBandCols * (size_t)t.lds_ld * sizeof(uint16_t);
  switch ((t.lds_ld - 8) / 32) {  // K-steps of the largest job
    case 1: return launch_fused_ks<1>(t, f32out, multi, grid, lds, stream);
    case 2: return launch_fused_ks<2>(t, f32out, multi, grid, lds, stream);
    case 3: return launch_fused_ks<3>(t, f32out, multi, grid, lds, stream);
    case 4: return launch_fused_ks<4>(t, f32out, multi, grid, lds, stream);
    case 5: return launch_fused_ks<5>(t, f32out, multi, grid, lds, stream);
    case 6: return launch_fused_ks<6>(t, f32out, multi, grid, lds, stream);
    case 7: return launch_fused_ks<7>(t, f32out, multi, grid, lds, stream);
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

hipError_t launch_generic(const GenericArgs& a, bool f32out, hipStream_t stream) {
  if (a.elem_count == 0) return hipSuccess;
  dim3 grid((unsigned)((a.elem_count + 255) / 256));
  if (f32out) hipLaunchKernelGGL((k_generic<true>), grid, dim3(256), 0, stream, a);
  else hipLaunchKernelGGL((k_generic<false>), grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace ltxw
