// The several-LoRA fused kernel (k_fused_pair_multi), templated on the factor
// element type; kernels_multi_*.hip instantiate it, one factor type per
// translation unit, so that they compile in parallel. CDNA4 (gfx950, wave64).
#pragma once

#include <type_traits>

#include "kernels_dev.h"

namespace ltxw {
namespace {

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
// Factor element types the kernel takes (ltxw_factor_dtype): bf16 (0) and
// f16 (2) feed the bf16 / f16 MFMA as stored; e4m3fn (3) and e5m2 (4) are
// widened to bf16 in registers, which is exact (every FP8 value, NaN and Inf
// included, is a bf16 value), so their products are the same as the
// reference's f32 ones. F32 factors take the reference-order kernel.
template <int FDT>
struct FactorRaw {
  using T = u32x4;  // 8 elements of 16 bits
  static constexpr uint32_t kBytes = 2;
};
template <>
struct FactorRaw<3> {
  using T = u32x2;  // 8 FP8 bytes
  static constexpr uint32_t kBytes = 1;
};
template <>
struct FactorRaw<4> : FactorRaw<3> {};

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// 8 raw elements -> 8 MFMA input elements, as 4 packed pairs.
template <int FDT>
__device__ __forceinline__ u32x4 to_pairs(const typename FactorRaw<FDT>::T& r) {
  if constexpr (FDT == 3 || FDT == 4) {
    float v[8];
    decode4(r[0], FDT - 3, v);
    decode4(r[1], FDT - 3, v + 4);
    return (u32x4){pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]), pack_bf16(v[4], v[5]), pack_bf16(v[6], v[7])};
  } else {
    return r;
  }
}

template <int FDT>
__device__ __forceinline__ f32x4 mfma_step(const u32x4& a, const u32x4& b, const f32x4& c) {
  if constexpr (FDT == 2)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

template <int KS>
struct PJM {
  PJ base;  // coeff / cmul: the last LoRA's coefficient
  const void* a[KS];
  const void* b[KS];
  uint32_t rank[KS];
  uint32_t klim[KS];
  float q[KS];
  uint32_t qmask;
  uint32_t pf;  // bit t: steps t and t + 1 swap their B pieces on odd rows (BSW launches)
};

template <int KS, bool BSW>
__device__ __forceinline__ PJM<KS> pjm_load(const JobTable& t, uint32_t wg) {
  CByte* rec = job_record<KS>(t, wg);
  const FusedJob J = kload<FusedJob>(rec);
  PJM<KS> m;
  m.base.w = J.w;
  m.base.out = J.out;
  m.base.scales = J.scales;
  m.base.a = nullptr;
  m.base.b = nullptr;
  m.base.rows = J.rows;
  m.base.cols = J.cols;
  m.base.rank = 0;
  m.base.bands_n = J.bands_n;
  m.base.scale_mode = J.scale_mode;
  m.base.fmt = J.fmt;
  m.base.tscale = m.base.scale_mode == 1 ? *G(J.scales) : 1.0f;
  m.base.coeff = J.coeff_out;
  m.base.cmul = J.cmul;
  m.base.unit_begin = J.unit_begin;
  m.base.single = J.single;
  m.pf = 0;
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const StepDev st = job_step(rec, s);
    m.a[s] = st.a;
    m.b[s] = st.b;
    m.rank[s] = st.rank;
    m.klim[s] = st.klim;
    m.q[s] = st.q;
    if constexpr (BSW) {
      if (s + 1 < KS) m.pf |= (st.pair & 1u) << s;
    }
  }
  m.qmask = J.qmask;
  return m;
}

template <int KS, int FDT>
struct StageM {
  typename FactorRaw<FDT>::T lo[KS], hi[KS];
};

// B16: the base is bf16 or f16 (16 bytes per 8 elements), else FP8.
template <int KS, int FDT, bool B16>
struct FragM {
  using Wv = typename std::conditional<B16, u32x4, u32x2>::type;
  typename FactorRaw<FDT>::T bf[KS][2];
  Wv wv[8];
  float sc[8];
};

template <int KS, int FDT>
__device__ __forceinline__ void pm_issue_a(const PJM<KS>& M, uint32_t i0, int tid, StageM<KS, FDT>& st) {
  using R = typename FactorRaw<FDT>::T;
  constexpr uint32_t E = FactorRaw<FDT>::kBytes;
  const int sq = tid & 15;
  const uint32_t cols = M.base.cols;
  // Column groups as in pp_issue_a; a group is 8 E bytes wide, so the partner
  // group in the other half of a 128-byte line is 64 / (8 E) groups away.
  const uint32_t scol = i0 + 8 * a_group(tid, 8 / E);
  const bool scol_ok = scol < cols;
  const uint32_t k = 2 * sq;
#pragma unroll
  for (int t = 0; t < KS; ++t) {
    st.lo[t] = R{};
    st.hi[t] = R{};
    if (scol_ok && k < M.klim[t]) st.lo[t] = ld_at<R>(M.a[t], E * (k * cols + scol));
    if (scol_ok && k + 1 < M.klim[t]) st.hi[t] = ld_at<R>(M.a[t], E * ((k + 1) * cols + scol));
  }
}

// As pp_stage, from raw factor elements.
template <int KS, int FDT>
__device__ __forceinline__ void pm_stage(const StageM<KS, FDT>& st, uint16_t* AT, int ld, int tid) {
  const int sq = tid & 15;
#pragma unroll
  for (int t = 0; t < KS; ++t) {
    const u32x4 lo = to_pairs<FDT>(st.lo[t]), hi = to_pairs<FDT>(st.hi[t]);
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const uint32_t pair = __builtin_amdgcn_perm(hi[jj >> 1], lo[jj >> 1], (jj & 1) ? 0x07060302u : 0x05040100u);
      *reinterpret_cast<uint32_t*>(&AT[(jj * 16 + a_group(tid, 8 / FactorRaw<FDT>::kBytes)) * ld + 32 * t + 2 * sq]) =
          pair;
    }
  }
}

template <int KS, bool FULL, int FDT, bool B16, bool BSW>
__device__ __forceinline__ void pm_issue_f(const PJM<KS>& M, uint32_t g0, int tid, FragM<KS, FDT, B16>& f) {
  using R = typename FactorRaw<FDT>::T;
  constexpr uint32_t E = FactorRaw<FDT>::kBytes;
  const int lane = tid & 63, wave = tid >> 6, ln = lane & 15, lg = lane >> 4;
  const uint32_t rows = M.base.rows;
  const uint32_t r0 = g0 + kStripRows * wave;
  const uint32_t kk = 8 * lg;
  if constexpr (BSW) {
    // The B-fragment pair swap of pp_issue_f (kernels_dev.h), with the pairs
    // from the host: for a pair (t, t + 1) of one LoRA (pf bit t), odd rows
    // fetch the other step's piece of their own row (both steps are whole,
    // so the piece exists); pm_mfma_at swaps the operands back.
    const bool odd = ln & 1;
#pragma unroll
    for (int t = 0; t < KS; ++t) {
      const bool first = t + 1 < KS && ((M.pf >> t) & 1u);
      const bool second = t >= 1 && ((M.pf >> (t - 1)) & 1u);
      const int64_t d = odd ? (first ? 32 * (int64_t)E : (second ? -32 * (int64_t)E : 0)) : 0;
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        const uint32_t ob = r0 + 16 * mb + ln;
        f.bf[t][mb] = R{};
        if (kk < M.klim[t] && (FULL || ob < rows))
          f.bf[t][mb] = *reinterpret_cast<const __attribute__((address_space(1))) R*>(
              (const __attribute__((address_space(1))) char*)M.b[t] + (int64_t)(E * (ob * M.rank[t] + kk)) + d);
      }
    }
  } else {
#pragma unroll
    for (int t = 0; t < KS; ++t) {
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        const uint32_t ob = r0 + 16 * mb + ln;
        f.bf[t][mb] = R{};
        if (kk < M.klim[t] && (FULL || ob < rows)) f.bf[t][mb] = ld_at<R>(M.b[t], E * (ob * M.rank[t] + kk));
      }
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

// K-step T of the swapped chain (template recursion: every register index is
// a compile-time constant, so FragM stays in registers).
template <int T, int KS, int FDT, bool B16>
__device__ __forceinline__ void pm_mfma_at(const PJM<KS>& M, const FragM<KS, FDT, B16>& f, const uint16_t* AT,
                                           int ld, int ln, int lg, Acc<KS>& a) {
  if constexpr (T < KS) {
    using R = typename FactorRaw<FDT>::T;
    const bool odd = ln & 1;
    R r0 = f.bf[T][0], r1 = f.bf[T][1];
    if constexpr (T + 1 < KS) {
      if ((M.pf >> T) & 1u) {
        r0 = odd ? f.bf[T + 1][0] : r0;
        r1 = odd ? f.bf[T + 1][1] : r1;
      }
    }
    if constexpr (T >= 1) {
      if ((M.pf >> (T - 1)) & 1u) {
        r0 = odd ? f.bf[T - 1][0] : r0;
        r1 = odd ? f.bf[T - 1][1] : r1;
      }
    }
    const int kk = 32 * T + 8 * lg;
    const u32x4 b0 = to_pairs<FDT>(r0), b1 = to_pairs<FDT>(r1);
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
      const u32x4 at = *reinterpret_cast<const u32x4*>(&AT[(nb * 16 + ln) * ld + kk]);
      a.v[0][nb] = mfma_step<FDT>(b0, at, a.v[0][nb]);
      a.v[1][nb] = mfma_step<FDT>(b1, at, a.v[1][nb]);
    }
    if (T + 1 < KS && (M.qmask & (1u << T))) {
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) a.v[mb][nb] *= M.q[T];
    }
    pm_mfma_at<T + 1, KS, FDT, B16>(M, f, AT, ld, ln, lg, a);
  }
}

template <int KS, int FDT, bool B16, bool BSW>
__device__ __forceinline__ void pm_mfma(const PJM<KS>& M, const FragM<KS, FDT, B16>& f, const uint16_t* AT, int ld,
                                        int tid, Acc<KS>& a) {
  const int lane = tid & 63, ln = lane & 15, lg = lane >> 4;
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) a.v[mb][nb] = (f32x4){0.f, 0.f, 0.f, 0.f};
  if constexpr (BSW) {
    pm_mfma_at<0, KS, FDT, B16>(M, f, AT, ld, ln, lg, a);
  } else {
#pragma unroll
    for (int t = 0; t < KS; ++t) {
      const int kk = 32 * t + 8 * lg;
      const u32x4 b0 = to_pairs<FDT>(f.bf[t][0]), b1 = to_pairs<FDT>(f.bf[t][1]);
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) {
        const u32x4 at = *reinterpret_cast<const u32x4*>(&AT[(nb * 16 + ln) * ld + kk]);
        a.v[0][nb] = mfma_step<FDT>(b0, at, a.v[0][nb]);
        a.v[1][nb] = mfma_step<FDT>(b1, at, a.v[1][nb]);
      }
      if (t + 1 < KS && (M.qmask & (1u << t))) {
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
          for (int nb = 0; nb < 8; ++nb) a.v[mb][nb] *= M.q[t];
      }
    }
  }
}

template <bool F32OUT, int KS, int FMT, bool FULL, int FDT, bool BSW, bool WFIRST>
__device__ __forceinline__ void pair_units_multi(const PJM<KS>& M, uint16_t* AT, uint32_t i0, uint32_t gA,
                                                 uint32_t gB, bool hasB, int tid) {
  constexpr int LD = 32 * KS + 8;
  constexpr bool B16 = FMT >= 2;
  StageM<KS, FDT> st;
  FragM<KS, FDT, B16> fa, fb;
  if constexpr (WFIRST) {  // as pair_units (kernels.hip): the first unit's base bytes first
    pp_issue_w<KS, FULL>(M.base, i0, gA, tid, fa);
    pm_issue_a<KS, FDT>(M, i0, tid, st);
    pm_issue_f<KS, FULL, FDT, B16, BSW>(M, gA, tid, fa);
  } else {
    pm_issue_a<KS, FDT>(M, i0, tid, st);
    pm_issue_f<KS, FULL, FDT, B16, BSW>(M, gA, tid, fa);
    // Raised wave priority while the FP8 bytes are requested, as in
    // pair_units: mixed block 257 -> 254.5 us (alternating runs on one machine;
    // over the whole issue phase it measured slower, 261 -> 265.5 us). The
    // one-round schedule above has none: on its FP8 loads it measured mixed
    // (one 4096 x 4096 layer with two rank-32 bf16 LoRAs 12.22 -> 12.35 us,
    // with one rank-64 f16 LoRA 12.70 -> 12.34 us).
    __builtin_amdgcn_s_setprio(2);
    pp_issue_w<KS, FULL>(M.base, i0, gA, tid, fa);
  }
  pp_issue_w<KS, FULL>(M.base, i0, hasB ? gB : gA, tid, fb);
  __builtin_amdgcn_s_setprio(0);
  pm_stage<KS, FDT>(st, AT, LD, tid);
  __syncthreads();
  {
    Acc<KS> acc;
    pm_mfma<KS, FDT, B16, BSW>(M, fa, AT, LD, tid, acc);
    pm_issue_f<KS, FULL, FDT, B16, BSW>(M, hasB ? gB : gA, tid, fb);
    pp_epilogue<F32OUT, KS, FULL, FMT, !WFIRST>(M.base, fa, acc, i0, gA, tid);
  }
  asm volatile("" ::: "memory");
  if (hasB) {
    Acc<KS> acc;
    pm_mfma<KS, FDT, B16, BSW>(M, fb, AT, LD, tid, acc);
    pp_epilogue<F32OUT, KS, FULL, FMT, !WFIRST>(M.base, fb, acc, i0, gB, tid);
  }
}

// One unit per workgroup (the single-unit jobs at a large launch's end), as
// one_unit (kernels.hip).
template <bool F32OUT, int KS, int FMT, bool FULL, int FDT, bool BSW>
__device__ __forceinline__ void one_unit_multi(const PJM<KS>& M, uint16_t* AT, uint32_t i0, uint32_t g0, int tid) {
  constexpr int LD = 32 * KS + 8;
  constexpr bool B16 = FMT >= 2;
  StageM<KS, FDT> st;
  FragM<KS, FDT, B16> f;
  pm_issue_a<KS, FDT>(M, i0, tid, st);
  pm_issue_f<KS, FULL, FDT, B16, BSW>(M, g0, tid, f);
  __builtin_amdgcn_s_setprio(2);
  pp_issue_w<KS, FULL>(M.base, i0, g0, tid, f);
  __builtin_amdgcn_s_setprio(0);
  pm_stage<KS, FDT>(st, AT, LD, tid);
  __syncthreads();
  Acc<KS> acc;
  pm_mfma<KS, FDT, B16, BSW>(M, f, AT, LD, tid, acc);
  pp_epilogue<F32OUT, KS, FULL, FMT, true>(M.base, f, acc, i0, g0, tid);
}

// BSW: the B-fragment pair swap (launches of kSwapMinGrid workgroups and
// more, 16-bit factors); WFIRST: base bytes before factors (launches of at
// most kWFirstMaxGrid workgroups, up to 2 K-steps).
template <bool F32OUT, int KS, int FDT, bool B16, bool BSW, bool WFIRST>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void k_fused_pair_multi(JobTable tab) {
  extern __shared__ __attribute__((aligned(16))) uint16_t AT[];
  const int tid = threadIdx.x;
  const uint32_t pair = xcd_remap(blockIdx.x, gridDim.x, tab.main_groups);
  const PJM<KS> M = pjm_load<KS, BSW>(tab, pair);
  const uint32_t p = pair - M.base.unit_begin;
  const uint32_t i0 = (p % M.base.bands_n) * kBandCols;
  // Base formats (ltxw_format): e4m3fn / e5m2, or with B16 bf16 / f16.
  constexpr int F0 = B16 ? 2 : 0, F1 = B16 ? 3 : 1;
  if constexpr (!WFIRST && KS <= 2) {
    if (M.base.single) {
      const uint32_t g0 = (p / M.base.bands_n) * kUnitRows;
      const bool full1 = g0 + kUnitRows <= M.base.rows && i0 + kBandCols <= M.base.cols;
      if (M.base.fmt == (uint32_t)F0) {
        if (full1) one_unit_multi<F32OUT, KS, F0, true, FDT, BSW>(M, AT, i0, g0, tid);
        else one_unit_multi<F32OUT, KS, F0, false, FDT, BSW>(M, AT, i0, g0, tid);
      } else {
        if (full1) one_unit_multi<F32OUT, KS, F1, true, FDT, BSW>(M, AT, i0, g0, tid);
        else one_unit_multi<F32OUT, KS, F1, false, FDT, BSW>(M, AT, i0, g0, tid);
      }
      return;
    }
  }
  const uint32_t gA = (p / M.base.bands_n) * (2 * kWavesPerGroup * kStripRows);
  const uint32_t gB = gA + kWavesPerGroup * kStripRows;
  const bool hasB = gB < M.base.rows;
  const bool full = gB + kWavesPerGroup * kStripRows <= M.base.rows && i0 + kBandCols <= M.base.cols;
  if (M.base.fmt == (uint32_t)F0) {
    if (full) pair_units_multi<F32OUT, KS, F0, true, FDT, BSW, WFIRST>(M, AT, i0, gA, gB, hasB, tid);
    else pair_units_multi<F32OUT, KS, F0, false, FDT, BSW, WFIRST>(M, AT, i0, gA, gB, hasB, tid);
  } else {
    if (full) pair_units_multi<F32OUT, KS, F1, true, FDT, BSW, WFIRST>(M, AT, i0, gA, gB, hasB, tid);
    else pair_units_multi<F32OUT, KS, F1, false, FDT, BSW, WFIRST>(M, AT, i0, gA, gB, hasB, tid);
  }
}

template <int KS, int FDT, bool B16, bool BSW, bool WFIRST>
hipError_t launch_multi_sched(const JobTable& t, bool f32out, dim3 grid, size_t lds, hipStream_t stream) {
  if (f32out) hipLaunchKernelGGL((k_fused_pair_multi<true, KS, FDT, B16, BSW, WFIRST>), grid, dim3(256), lds, stream, t);
  else hipLaunchKernelGGL((k_fused_pair_multi<false, KS, FDT, B16, BSW, WFIRST>), grid, dim3(256), lds, stream, t);
  return hipGetLastError();
}

template <int KS, int FDT, bool B16>
hipError_t launch_multi_ks(const JobTable& t, bool f32out, dim3 grid, size_t lds, hipStream_t stream) {
  // The swap pairs K-steps of 16-bit factors; the host marks the pairs.
  if constexpr (KS >= 2 && FactorRaw<FDT>::kBytes == 2) {
    if (t.total_units >= kSwapMinGrid) return launch_multi_sched<KS, FDT, B16, true, false>(t, f32out, grid, lds, stream);
  }
  // Base bytes first in one-round launches: one layer with rank-64 bf16 factors
  // 12.5 -> 12.1 us; with 5 K-steps (r32 + r128) it measured 1% slower.
  if constexpr (KS <= 2) {
    if (t.total_units <= kWFirstMaxGrid) return launch_multi_sched<KS, FDT, B16, false, true>(t, f32out, grid, lds, stream);
  }
  return launch_multi_sched<KS, FDT, B16, false, false>(t, f32out, grid, lds, stream);
}

template <int FDT, bool B16 = false>
hipError_t launch_multi_fdt(const JobTable& t, bool f32out, int ks, hipStream_t stream) {
  if (t.total_units == 0) return hipSuccess;
  dim3 grid((unsigned)t.total_units);
  size_t lds = (size_t)kBandCols * (size_t)t.lds_ld * sizeof(uint16_t);
  switch (ks) {
    case 1: return launch_multi_ks<1, FDT, B16>(t, f32out, grid, lds, stream);
    case 2: return launch_multi_ks<2, FDT, B16>(t, f32out, grid, lds, stream);
    case 3: return launch_multi_ks<3, FDT, B16>(t, f32out, grid, lds, stream);
    case 4: return launch_multi_ks<4, FDT, B16>(t, f32out, grid, lds, stream);
    case 5: return launch_multi_ks<5, FDT, B16>(t, f32out, grid, lds, stream);
    case 6: return launch_multi_ks<6, FDT, B16>(t, f32out, grid, lds, stream);
    case 7: return launch_multi_ks<7, FDT, B16>(t, f32out, grid, lds, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

}  // namespace ltxw
