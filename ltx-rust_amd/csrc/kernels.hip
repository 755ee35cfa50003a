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
// Workgroup: 256 threads (4 waves), output tile kTileM x kTileN = 128 x 128.
// Wave w owns rows [32w, 32w+32) of the tile.
//
// LoRA product on MFMA v_mfma_f32_32x32x16_bf16 with M = output column i,
// N = output row o, K = rank r:
//   A operand (i x r) = A_lora^T, staged transposed in LDS (AT[i][r]) from
//                       coalesced row loads of A_lora, 64 ranks at a time;
//   B operand (r x o) = B_lora rows, 16-byte global loads (r is contiguous);
//   C (i x o) lane layout: lane l holds o = l%32 and, for accumulator v,
//                       i = 8*(v/4) + 4*(l/32) + v%4 within the 32-block.
// The f32 result is relaid through LDS (per wave, 16 rows at a time) into row
// order so that the FP8 input (read once, 8 bytes per lane, prefetched before
// the MFMA phase) and the bf16 output (16 bytes per lane) are coalesced:
// 16 lanes cover 128 contiguous columns of one row.
// ---------------------------------------------------------------------------
constexpr int kKC = 64;             // ranks staged per LDS pass
constexpr int kATLd = kKC + 8;      // AT row stride in bf16 (144 B: conflict-free b128 reads)
constexpr int kAccLd = kTileN + 4;  // relayout row stride in f32

__device__ __forceinline__ void load_job(const JobTable& t, uint64_t tile, JobDev& J) {
  if (t.n_jobs == 1) {
    J = t.one;
    return;
  }
  int lo = 0, hi = t.n_jobs - 1;  // last job with begins[j] <= tile
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if ((uint64_t)t.begins[mid] <= tile) lo = mid; else hi = mid - 1;
  }
  J = t.jobs[lo];
}

template <bool F32OUT, bool MULTI>
__global__ __launch_bounds__(256) void k_fused(JobTable tab) {
  __shared__ __attribute__((aligned(16))) uint16_t AT[kTileN * kATLd];
  __shared__ __attribute__((aligned(16))) float ACC[4][16 * kAccLd];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const uint64_t tile = xcd_remap(blockIdx.x, gridDim.x);

  JobDev J;
  load_job(tab, tile, J);
  const uint64_t t = tile - (uint64_t)J.tile_begin;
  const int64_t o0 = (int64_t)(t / (uint64_t)J.tiles_n) * kTileM;
  const int64_t i0 = (int64_t)(t % (uint64_t)J.tiles_n) * kTileN;
  const int64_t rows = J.rows, cols = J.cols;
  const int fmt = J.fmt;

  // --- Prefetch this lane's FP8 bytes for the epilogue (8 groups of 8).
  // Group (h, p): row 32*wave + 16*h + 4*p + lane/16, columns 8*(lane%16)..+7.
  const int ecol = 8 * (lane & 15);
  u32x2 raw[8];
  float rscale[8];
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    int64_t r = o0 + 32 * wave + 16 * (g >> 2) + 4 * (g & 3) + (lane >> 4);
    int64_t c = i0 + ecol;
    raw[g] = (u32x2){0u, 0u};
    rscale[g] = 1.0f;
    if (r < rows && c < cols) {
      raw[g] = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(J.w + r * cols + c));
      if (J.scale_mode == 2) rscale[g] = J.scales[r];
    }
  }
  const float tscale = J.scale_mode == 1 ? J.scales[0] : 1.0f;

  // --- LoRA products.
  f32x16 acc[4];
  f32x16 delta[MULTI ? 4 : 1];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) acc[mb] = (f32x16){};
  float cfin = 0.0f;

  const int64_t orow_b = o0 + 32 * wave + (lane & 31);  // B row this lane feeds
  const int khalf = 8 * (lane >> 5);

#pragma unroll
  for (int l = 0; l < kMaxLoras; ++l) {
    if (l >= J.n_loras) break;
    const LoraDev L = J.lora[l];
    for (int kc = 0; kc < L.rank; kc += kKC) {
      __syncthreads();  // previous AT contents fully consumed
      // Stage A_lora[kc..kc+64) x [i0..i0+128) into AT[i][k], zero outside.
#pragma unroll
      for (int it = 0; it < 2; ++it) {
        int item = tid + 256 * it;  // 32 rank pairs x 16 column chunks of 8
        int q = item & 31, cc = item >> 5;
        int k0 = kc + 2 * q;
        int64_t col = i0 + 8 * cc;
        u32x4 lo = (u32x4){0u, 0u, 0u, 0u}, hi = lo;
        if (col < cols) {
          if (k0 < L.rank) lo = *reinterpret_cast<const u32x4*>(L.a + (int64_t)k0 * cols + col);
          if (k0 + 1 < L.rank) hi = *reinterpret_cast<const u32x4*>(L.a + (int64_t)(k0 + 1) * cols + col);
        }
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
          uint32_t a0 = (lo[jj >> 1] >> (16 * (jj & 1))) & 0xFFFFu;
          uint32_t a1 = (hi[jj >> 1] >> (16 * (jj & 1))) & 0xFFFFu;
          *reinterpret_cast<uint32_t*>(&AT[(8 * cc + jj) * kATLd + 2 * q]) = a0 | (a1 << 16);
        }
      }
      __syncthreads();
      bf16x8 bfrag[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        int kk = kc + 16 * ks + khalf;
        bfrag[ks] = (bf16x8){};
        if (orow_b < rows && kk < L.rank)
          bfrag[ks] = *reinterpret_cast<const bf16x8*>(L.b + orow_b * L.rank + kk);
      }
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
          bf16x8 afrag = *reinterpret_cast<const bf16x8*>(&AT[(mb * 32 + (lane & 31)) * kATLd + 16 * ks + khalf]);
          acc[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(afrag, bfrag[ks], acc[mb], 0, 0, 0);
        }
      }
    }
    if (MULTI) {
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
        for (int v = 0; v < 16; ++v)
          delta[mb][v] = l == 0 ? L.coeff * acc[mb][v] : __builtin_fmaf(L.coeff, acc[mb][v], delta[mb][v]);
        acc[mb] = (f32x16){};
      }
    } else {
      cfin = L.coeff;
    }
  }
  if (MULTI) {
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) acc[mb] = delta[mb];
    cfin = 1.0f;
  }
  const bool has_lora = J.n_loras > 0;

  // --- Epilogue, 16 rows of each wave's 32 at a time.
  float* acc_lds = ACC[wave];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    __syncthreads();
    if (((lane & 31) >> 4) == h) {
      int orow = (lane & 31) - 16 * h;
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          int icol = mb * 32 + g4 * 8 + 4 * (lane >> 5);
          *reinterpret_cast<f32x4*>(&acc_lds[orow * kAccLd + icol]) =
              (f32x4){acc[mb][4 * g4], acc[mb][4 * g4 + 1], acc[mb][4 * g4 + 2], acc[mb][4 * g4 + 3]};
        }
    }
    __syncthreads();
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int g = 4 * h + p;
      const int orow = 4 * p + (lane >> 4);
      const int64_t r = o0 + 32 * wave + 16 * h + orow;
      const int64_t c = i0 + ecol;
      if (r < rows && c < cols) {
        f32x4 d0 = *reinterpret_cast<const f32x4*>(&acc_lds[orow * kAccLd + ecol]);
        f32x4 d1 = *reinterpret_cast<const f32x4*>(&acc_lds[orow * kAccLd + ecol + 4]);
        float v[8];
        decode4(raw[g][0], fmt, v);
        decode4(raw[g][1], fmt, v + 4);
        const float s = J.scale_mode == 2 ? rscale[g] : tscale;
        float d[8] = {d0[0], d0[1], d0[2], d0[3], d1[0], d1[1], d1[2], d1[3]};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if (J.scale_mode != 0) v[j] = __builtin_fmaf(s, v[j], 0.0f);
          if (has_lora) v[j] = __builtin_fmaf(cfin, d[j], v[j]);
          v[j] = canon_nan(v[j]);
        }
        if (F32OUT) {
          f32x4* dst = reinterpret_cast<f32x4*>(reinterpret_cast<float*>(J.out) + r * cols + c);
          __builtin_nontemporal_store((f32x4){v[0], v[1], v[2], v[3]}, dst);
          __builtin_nontemporal_store((f32x4){v[4], v[5], v[6], v[7]}, dst + 1);
        } else {
          u32x4 o = {pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]), pack_bf16(v[4], v[5]), pack_bf16(v[6], v[7])};
          __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(J.out) + r * cols + c));
        }
      }
    }
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
  if (t.total_tiles == 0) return hipSuccess;
  dim3 grid((unsigned)t.total_tiles);
  if (f32out) {
    if (multi) hipLaunchKernelGGL((k_fused<true, true>), grid, dim3(256), 0, stream, t);
    else hipLaunchKernelGGL((k_fused<true, false>), grid, dim3(256), 0, stream, t);
  } else {
    if (multi) hipLaunchKernelGGL((k_fused<false, true>), grid, dim3(256), 0, stream, t);
    else hipLaunchKernelGGL((k_fused<false, false>), grid, dim3(256), 0, stream, t);
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
