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

// Pointers read out of job descriptors are generic; marking them global makes
// the compiler emit global_load/global_store (not flat_*, which also count
// against the LDS counter and skip the global addressing modes).
template <typename T>
__device__ __forceinline__ __attribute__((address_space(1))) T* G(T* p) {
  return (__attribute__((address_space(1))) T*)(p);
}

// Workgroups are dispatched round-robin over the 8 XCDs; map them so that each
// XCD takes a contiguous range of logical tiles (tiles of one row band share
// their LoRA B rows in that XCD's L2). A bijection on [0, n).
__device__ __forceinline__ uint32_t xcd_remap(uint32_t bid, uint32_t n) {
  constexpr uint32_t kXcd = 8;
  uint32_t per = n / kXcd, rem = n % kXcd;
  uint32_t x = bid % kXcd, k = bid / kXcd;
  return x < rem ? x * (per + 1) + k : rem * (per + 1) + (x - rem) * per + k;
}

// ---------------------------------------------------------------------------
// (a) Streaming dequant. Each thread handles kChunksPerThread chunks of 16
// FP8 bytes: one 128-bit load, two 128-bit bf16 stores (four for f32).
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
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = canon_nan(v[j]);
    if (F32OUT) {
      f32x4* dst = reinterpret_cast<f32x4*>(a.out) + idx * 4;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        __builtin_nontemporal_store((f32x4){v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]}, dst + q);
    } else {
      u32x4* dst = reinterpret_cast<u32x4*>(a.out) + idx * 2;
      u32x4 lo = {pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]), pack_bf16(v[4], v[5]), pack_bf16(v[6], v[7])};
      u32x4 hi = {pack_bf16(v[8], v[9]), pack_bf16(v[10], v[11]), pack_bf16(v[12], v[13]), pack_bf16(v[14], v[15])};
      __builtin_nontemporal_store(lo, dst);
      __builtin_nontemporal_store(hi, dst + 1);
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
  float v = decode1(J.w[e], J.fmt);
  if (J.scale_mode == 1) v = __builtin_fmaf(J.scales[0], v, 0.0f);
  if (J.scale_mode == 2) v = __builtin_fmaf(J.scales[o], v, 0.0f);
#pragma unroll
  for (int l = 0; l < kMaxLoras; ++l) {
    if (l >= J.n_loras) break;
    const LoraDev L = J.lora[l];
    const uint16_t* brow = L.b + o * (uint64_t)L.rank;
    for (int r = 0; r < L.rank; ++r) {
      float c = L.coeff * bf16_to_f32(brow[r]);
      v = __builtin_fmaf(c, bf16_to_f32(L.a[(uint64_t)r * cols + i]), v);
    }
  }
  v = canon_nan(v);
  if (F32OUT)
    reinterpret_cast<float*>(J.out)[e] = v;
  else
    reinterpret_cast<uint16_t*>(J.out)[e] = (uint16_t)(pack_bf16(v, 0.0f) & 0xFFFFu);
}

// ---------------------------------------------------------------------------
// (b) Fused dequant + LoRA merge.
//
// Workgroup: 4 waves. Work unit: one band of 128 output columns [i0, i0+128)
// and 4*S strips of 32 rows; wave w walks strips w, w+4, ... of the unit.
//
// LoRA product on v_mfma_f32_16x16x32_bf16 with M = output row o, N = output
// column i, K = rank r, and the N index permuted as i = i0 + 8*n + nb for
// N-block nb (0..7) and MFMA column n (0..15). With the C layout (lane l holds
// column n = l%16 and rows m = 4*(l/16) + v), lane l then owns, for each of
// its 8 rows, the 8 contiguous columns i0 + 8*(l%16) .. +7 across the 8
// N-blocks: the FP8 input (8 bytes per lane) and the bf16 output (16 bytes per
// lane) are read and written straight from registers, 16 lanes covering 128
// contiguous columns of a row, with no LDS relayout.
//   A operand (o x r): LoRA B rows, 16-byte loads (r contiguous), from L2.
//   B operand (r x i): LoRA A transposed, staged once per work unit in LDS as
//                      AT[slot][k] with slot = nb*16 + n (consecutive lanes
//                      read consecutive slots: conflict-free 128-bit reads).
// Several LoRAs are staged side by side along k (each padded to 32).
// The FP8 bytes of the next strip are loaded while the current one computes.
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

struct StripIn {
  u32x2 w[8];   // FP8 bytes: group g = 4*mb + v -> row 16*mb + 4*(lane/16) + v
  float s[8];   // per-row scales of those rows
};

__device__ __forceinline__ void load_strip(const JobDev& J, int64_t r0, int64_t c, int lane, StripIn& x) {
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    const int64_t r = r0 + 16 * (g >> 2) + 4 * (lane >> 4) + (g & 3);
    x.w[g] = (u32x2){0u, 0u};
    x.s[g] = 1.0f;
    if (r < J.rows && c < J.cols) {
      x.w[g] = __builtin_nontemporal_load(G(reinterpret_cast<const u32x2*>(J.w + r * J.cols + c)));
      if (J.scale_mode == 2) x.s[g] = G(J.scales)[r];
    }
  }
}

// Stage rows [0, pad_rank(rank)) of LoRA A (zero past `rank`), columns
// [i0, i0 + 128) (zero past `cols`), transposed into AT[slot][koff + k] with
// slot = (i % 8) * 16 + i / 8 for local column i.
__device__ __forceinline__ void stage_at(uint16_t* AT, int ld, int koff, const LoraDev& L, int64_t i0,
                                         int64_t cols, int tid) {
  const int pairs = pad_rank(L.rank) / 2;
  const int items = pairs * 16;  // rank pairs x column chunks of 8
  for (int item = tid; item < items; item += 256) {
    const int q = item % pairs, cc = item / pairs;
    const int k = 2 * q;
    const int64_t col = i0 + 8 * cc;
    u32x4 lo = (u32x4){0u, 0u, 0u, 0u}, hi = lo;
    if (col < cols) {
      if (k < L.rank) lo = *G(reinterpret_cast<const u32x4*>(L.a + (int64_t)k * cols + col));
      if (k + 1 < L.rank) hi = *G(reinterpret_cast<const u32x4*>(L.a + (int64_t)(k + 1) * cols + col));
    }
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const uint32_t a0 = (lo[jj >> 1] >> (16 * (jj & 1))) & 0xFFFFu;
      const uint32_t a1 = (hi[jj >> 1] >> (16 * (jj & 1))) & 0xFFFFu;
      *reinterpret_cast<uint32_t*>(&AT[(jj * 16 + cc) * ld + koff + k]) = a0 | (a1 << 16);
    }
  }
}

// acc[mb][nb] += (B rows r0 + 16*mb + ..) x (AT slots of N-block nb) over the
// LoRA's K range; optionally starts the next strip's loads after the first
// B fragments are in flight.
__device__ __forceinline__ void lora_mfma(f32x4 (&acc)[2][8], const uint16_t* AT, int ld, int koff,
                                          const LoraDev& L, int64_t r0, int64_t rows, int ln, int lg) {
  const int64_t ob0 = r0 + ln, ob1 = r0 + 16 + ln;  // B rows feeding M-blocks 0 and 1
  for (int kb = 0; kb < L.rank; kb += 32) {
    const int kk = kb + 8 * lg;
    bf16x8 b0 = (bf16x8){}, b1 = (bf16x8){};
    if (kk < L.rank) {
      if (ob0 < rows) b0 = *G(reinterpret_cast<const bf16x8*>(L.b + ob0 * L.rank + kk));
      if (ob1 < rows) b1 = *G(reinterpret_cast<const bf16x8*>(L.b + ob1 * L.rank + kk));
    }
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
      const bf16x8 at = *reinterpret_cast<const bf16x8*>(&AT[(nb * 16 + ln) * ld + koff + kk]);
      acc[0][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(b0, at, acc[0][nb], 0, 0, 0);
      acc[1][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(b1, at, acc[1][nb], 0, 0, 0);
    }
  }
}

// MULTI = false: exactly one LoRA. MULTI = true: 2..kMaxLoras LoRAs.
template <bool F32OUT, bool MULTI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(MULTI ? 2 : 3))) void k_fused(JobTable tab) {
  extern __shared__ __attribute__((aligned(16))) uint16_t AT[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int ln = lane & 15;   // MFMA column n / output column group
  const int lg = lane >> 4;   // MFMA row group (rows 4*lg .. 4*lg+3 of an M-block)
  const uint64_t unit = xcd_remap(blockIdx.x, gridDim.x);

  JobDev J;
  load_job(tab, unit, J);
  const uint64_t u = unit - (uint64_t)J.unit_begin;
  const int S = tab.strips;
  const int64_t i0 = (int64_t)(u % (uint64_t)J.bands_n) * kBandCols;
  const int64_t row_base = (int64_t)(u / (uint64_t)J.bands_n) * (kWavesPerGroup * S * kStripRows);
  const int64_t rows = J.rows, cols = J.cols;
  const int64_t ecol = i0 + 8 * ln;
  const int ld = tab.lds_ld;
  const int nl = MULTI ? J.n_loras : 1;

  // Start the first strip's FP8 stream before anything else.
  StripIn cur, nxt;
  load_strip(J, row_base + wave * kStripRows, ecol, lane, cur);
  const float tscale = J.scale_mode == 1 ? G(J.scales)[0] : 1.0f;

  int koff[kMaxLoras];
  {
    int k0 = 0;
#pragma unroll
    for (int l = 0; l < kMaxLoras; ++l) {
      koff[l] = k0;
      if (l < nl) k0 += pad_rank(J.lora[l].rank);
    }
  }
#pragma unroll
  for (int l = 0; l < (MULTI ? kMaxLoras : 1); ++l) {
    if (l >= nl) break;
    stage_at(AT, ld, koff[l], J.lora[l], i0, cols, tid);
  }
  __syncthreads();

  for (int s = 0; s < S; ++s) {
    const int64_t r0 = row_base + (int64_t)(s * kWavesPerGroup + wave) * kStripRows;
    if (r0 >= rows) break;
    const int64_t r0n = r0 + kWavesPerGroup * kStripRows;
    const bool more = s + 1 < S && r0n < rows;

    f32x4 acc[2][8];
    float cfin;
    if (!MULTI) {
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) acc[mb][nb] = (f32x4){0.f, 0.f, 0.f, 0.f};
      if (more) load_strip(J, r0n, ecol, lane, nxt);
      lora_mfma(acc, AT, ld, koff[0], J.lora[0], r0, rows, ln, lg);
      cfin = J.lora[0].coeff;
    } else {
      f32x4 delta[2][8];
      if (more) load_strip(J, r0n, ecol, lane, nxt);
#pragma unroll
      for (int l = 0; l < kMaxLoras; ++l) {
        if (l >= nl) break;
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
          for (int nb = 0; nb < 8; ++nb) acc[mb][nb] = (f32x4){0.f, 0.f, 0.f, 0.f};
        lora_mfma(acc, AT, ld, koff[l], J.lora[l], r0, rows, ln, lg);
        const float c = J.lora[l].coeff;
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
          for (int nb = 0; nb < 8; ++nb)
#pragma unroll
            for (int v = 0; v < 4; ++v)
              delta[mb][nb][v] = l == 0 ? c * acc[mb][nb][v] : __builtin_fmaf(c, acc[mb][nb][v], delta[mb][nb][v]);
      }
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) acc[mb][nb] = delta[mb][nb];
      cfin = 1.0f;
    }

    // --- Epilogue straight from registers.
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      const int mb = g >> 2, v = g & 3;
      const int64_t r = r0 + 16 * mb + 4 * lg + v;
      if (r < rows && ecol < cols) {
        float x[8];
        decode4(cur.w[g][0], J.fmt, x);
        decode4(cur.w[g][1], J.fmt, x + 4);
        const float sc = J.scale_mode == 2 ? cur.s[g] : tscale;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if (J.scale_mode != 0) x[j] = __builtin_fmaf(sc, x[j], 0.0f);
          x[j] = canon_nan(__builtin_fmaf(cfin, acc[mb][j][v], x[j]));
        }
        if (F32OUT) {
          auto dst = G(reinterpret_cast<f32x4*>(reinterpret_cast<float*>(J.out) + r * cols + ecol));
          __builtin_nontemporal_store((f32x4){x[0], x[1], x[2], x[3]}, dst);
          __builtin_nontemporal_store((f32x4){x[4], x[5], x[6], x[7]}, dst + 1);
        } else {
          const u32x4 o = {pack_bf16(x[0], x[1]), pack_bf16(x[2], x[3]), pack_bf16(x[4], x[5]), pack_bf16(x[6], x[7])};
          __builtin_nontemporal_store(o, G(reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(J.out) + r * cols + ecol)));
        }
      }
    }
    cur = nxt;
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

hipError_t launch_fused(const JobTable& t, bool f32out, bool multi, hipStream_t stream) {
  if (t.total_units == 0) return hipSuccess;
  dim3 grid((unsigned)t.total_units);
  size_t lds = (size_t)kBandCols * (size_t)t.lds_ld * sizeof(uint16_t);
  if (f32out) {
    if (multi) hipLaunchKernelGGL((k_fused<true, true>), grid, dim3(256), lds, stream, t);
    else hipLaunchKernelGGL((k_fused<true, false>), grid, dim3(256), lds, stream, t);
  } else {
    if (multi) hipLaunchKernelGGL((k_fused<false, true>), grid, dim3(256), lds, stream, t);
    else hipLaunchKernelGGL((k_fused<false, false>), grid, dim3(256), lds, stream, t);
  }
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
