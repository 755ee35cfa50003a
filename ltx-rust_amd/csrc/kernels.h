// Kernel launchers shared by the C ABI (api.cpp). Host-side declarations only.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace ltxw {

constexpr int kMaxLoras = 4;

// Work decomposition of the fused kernel. A workgroup (4 waves) owns one
// band of kBandCols output columns and 4 strips of kStripRows rows; wave w
// takes strip w.
constexpr int kBandCols = 128;
constexpr int kStripRows = 32;
constexpr int kWavesPerGroup = 4;
// Largest total LoRA rank (sum over a tensor's LoRAs, each padded to a
// multiple of 32) the fused kernel stages in LDS.
constexpr int kRankMax = 224;  // 128 slots x (224 + 8) bf16 = 59 KB of LDS

struct LoraDev {
  const uint16_t* b;  // [rows x rank], element type `dtype` (bf16 on the fused path)
  const uint16_t* a;  // [rank x cols]
  int32_t rank;
  float coeff;
  int32_t dtype;      // 0 bf16, 1 f32, 2 f16, 3 e4m3fn, 4 e5m2
  int32_t pad;
};

// One K-step (32 ranks) of the several-LoRA fused kernel, prepared on the
// host: the LoRAs of a tensor sit side by side along K, each padded to 32,
// and LoRA l owns the steps [kst_l, kst_l + pad_rank(rank_l) / 32).
struct StepDev {
  const void* a;      // A of the step's LoRA + 32 kt rows (row stride cols)
  const void* b;      // B of the step's LoRA + 32 kt columns (row stride rank)
  uint32_t rank;      // the LoRA's rank
  uint32_t klim;      // ranks of the step that exist: rank - 32 kt (>= 32: all)
  float q;            // factor applied to the accumulator after the step
  uint32_t pair;      // 1: this step and the next, both whole and of one LoRA with
                      // 16-bit factors and a row stride of a multiple of 128 bytes,
                      // may swap their B pieces on odd rows (kSwapMinGrid launches)
};
constexpr int kMaxSteps = kRankMax / 32;

// One tensor of a fused launch, as the kernel reads it.
struct JobDev {
  const uint8_t* w;
  void* out;
  const float* scales;
  int64_t rows;
  int64_t cols;
  int32_t fmt;
  int32_t scale_mode;
  int32_t n_loras;
  int32_t bands_n;     // column bands (ceil(cols / kBandCols))
  int64_t unit_begin;  // first flat work unit of this job in the launch
  LoraDev lora[kMaxLoras];
  // Fused kernels only (plan_fused). The accumulated product is multiplied by
  // coeff_out at the end when cmul is set. With several LoRAs, the step that
  // ends LoRA l (another one following) multiplies the accumulator by
  // q = c_l / c_{l+1}, so that it ends as (sum_l c_l B_l A_l) / c_last and one
  // register set holds the whole delta; qmask has bit t set for such steps.
  uint32_t qmask;
  uint32_t cmul;
  float coeff_out;
  uint32_t single;     // 1: one 128-row unit per workgroup (a launch's tail), else a pair
  StepDev step[kMaxSteps];
};

// One tensor of a fused launch as the fused kernels read it: this header,
// then one StepDev per K-step of the launch (record bytes
// sizeof(FusedJob) + KS * sizeof(StepDev), a multiple of 16). Built from a
// JobDev by the host (plan_fused fills the fields it copies).
struct FusedJob {
  const uint8_t* w;
  void* out;
  const float* scales;
  uint32_t rows, cols, bands_n;
  uint32_t unit_begin;  // first workgroup of this job in the launch
  uint32_t fmt, scale_mode, qmask, cmul;
  float coeff_out;
  uint32_t single;      // JobDev::single
};
static_assert(sizeof(FusedJob) == 64 && sizeof(StepDev) == 32, "record layout");

// Kernel arguments of a fused launch. The job records travel in the kernel
// arguments themselves (`inl`, read by the kernel from its argument segment)
// when they fit, so a grouped launch of a DiT block needs no table upload;
// larger launches read them from device memory (`table`).
constexpr int kInlineTableBytes = 2944;
constexpr int kInlineBegins = 16;
struct JobTable {
  JobDev one;            // the job of a one-job launch (n_jobs == 1)
  const void* table;     // device records; nullptr: the records are in `inl`
  int32_t n_jobs;
  int32_t lds_ld;        // AT row stride (bf16): 8 + the launch's largest total padded rank
  int64_t total_units;   // workgroups in the launch
  int32_t rec_bytes;     // bytes per job record: sizeof(FusedJob) + K-steps * sizeof(StepDev)
  uint32_t main_groups;  // workgroups of the pair jobs; the single-unit jobs follow them
  int32_t pad[2];
  // unit_begin of the inline records (n_jobs <= kInlineBegins; the rest
  // UINT32_MAX), so that a workgroup finds its record with one load.
  uint32_t begins[kInlineBegins];
  alignas(16) unsigned char inl[kInlineTableBytes];
};
static_assert(sizeof(JobTable) <= 4096, "kernel arguments of a fused launch");

struct DequantArgs {
  const uint8_t* w;
  void* out;
  const float* scales;
  uint64_t n;         // rows * cols elements
  uint64_t cols;
  uint64_t n_chunks;  // full 16-element chunks handled by the vector kernel
};

// Elementwise args for the generic (any shape / alignment) kernel.
struct GenericArgs {
  JobDev job;
  uint64_t elem_begin;  // first flat element handled
  uint64_t elem_count;
  // Open-time gate fold (store.rs:217-293): the scale as a plain multiply
  // (v * s, keeping -0) instead of fma(s, v, 0), then v * post_mul, both
  // before the LoRA deltas.
  int32_t plain_scale;
  int32_t has_post;
  float post_mul;
};

// Tiled reference-order kernel (any shape, alignment, base format and factor
// type): the generic kernel's arithmetic with the factors staged in LDS.
struct ExactArgs {
  JobDev job;
  int32_t plain_scale;  // as GenericArgs
  int32_t has_post;
  float post_mul;
  uint32_t bands_n;     // ceil(cols / kExactCols)
  int32_t canon_nan;    // canonicalise NaN results whatever the base format
};
constexpr int kExactCols = 128;
constexpr int kExactRows = 64;
hipError_t launch_exact(const ExactArgs& a, bool f32out, hipStream_t stream);

// Streaming dequant: n_chunks * 16 elements. Pointers 16-byte aligned.
hipError_t launch_dequant(const DequantArgs& a, int fmt, int scale_mode, bool f32out,
                          hipStream_t stream);

// Tiled dequant for tensors of up to kTileMaxElems elements (an FFN matrix
// of the DiT has 2^26): the fused kernels' lane layout (8 FP8 bytes per lane
// and row, 16 lanes per 128-column row segment) without the LoRA, kTileRows
// rows x 128 columns per workgroup. Requirements checked by the caller:
// cols % 8 == 0; w, out (and row scales) 16-byte aligned;
// rows * cols * 4 < 2^32.
struct DequantTileArgs {
  const uint8_t* w;
  void* out;
  const float* scales;
  uint32_t rows, cols, bands_n;
};
constexpr uint64_t kTileMaxElems = 1ull << 27;
constexpr int kTileRows = 64;
hipError_t launch_dequant_tile(const DequantTileArgs& a, int fmt, int scale_mode, bool f32out,
                               hipStream_t stream);

// Fused dequant + LoRA over every work unit of every job. Requirements checked
// by the caller: cols % 8 == 0, ranks % 8 == 0, all pointers 16-byte aligned,
// total padded rank <= kRankMax, the same K-steps for every job
// (lds_ld == 8 + 32 * K-steps). One workgroup per pair of vertically
// adjacent 128-row units (kPairRows rows); unit_begin and total_units count
// pairs. `multi`: the several-LoRA kernel (several LoRAs per tensor, or
// factors other than bf16), whose jobs all have factors of element type
// `fdt` and, with `base16`, bf16 / f16 bases. Every job's qmask, cmul,
// coeff_out and step[] are filled (plan_fused in api.cpp).
hipError_t launch_fused(const JobTable& t, bool f32out, bool multi, int fdt, bool base16, hipStream_t stream);

// The several-LoRA kernel alone (kernels_multi_dev.h); `ks` K-steps (1-7),
// every job's factors of element type `fdt` (ltxw_factor_dtype: 0 bf16,
// 2 f16, 3 e4m3fn, 4 e5m2), bases FP8 or, with `base16`, bf16 / f16 (bf16
// factors only). launch_fused calls it for `multi`.
hipError_t launch_fused_multi(const JobTable& t, bool f32out, int ks, int fdt, bool base16, hipStream_t stream);
// Its instantiations, one translation unit per factor type (kernels_multi_*.hip).
hipError_t launch_fused_multi_bf16(const JobTable& t, bool f32out, int ks, hipStream_t stream);
hipError_t launch_fused_multi_f16(const JobTable& t, bool f32out, int ks, hipStream_t stream);
hipError_t launch_fused_multi_e4m3fn(const JobTable& t, bool f32out, int ks, hipStream_t stream);
hipError_t launch_fused_multi_e5m2(const JobTable& t, bool f32out, int ks, hipStream_t stream);
// bf16 / f16 bases (no scale) with bf16 factors (kernels_multi_b16.hip).
hipError_t launch_fused_multi_base16(const JobTable& t, bool f32out, int ks, hipStream_t stream);

// Rows of one work unit (a band of kBandCols columns by kUnitRows rows). A
// workgroup of the fused kernels takes a pair of vertically adjacent units
// of one band (kPairRows rows): on one 4096 x 4096 layer with a rank-64
// LoRA, 4 units per workgroup measured no faster than 2. (The tiled dequant
// kernel takes kTileRows rows per workgroup.)
constexpr int kUnitRows = kWavesPerGroup * kStripRows;
constexpr int kPairRows = 2 * kUnitRows;
// Fused launches of more than this many workgroups map workgroups to XCDs
// in contiguous ranges; those of at most 2 K-steps, and every single-LoRA
// one, also end in single-unit workgroups (kTailPairs).
constexpr uint32_t kRemapMinGrid = 2048;
// Pair workgroups' worth of rows at a large launch's end that run as single
// units instead.
constexpr int64_t kTailPairs = 512;

// Padded K extent of one LoRA in the fused kernel's LDS stage.
__host__ __device__ inline int pad_rank(int rank) { return (rank + 31) / 32 * 32; }

// One thread per element, reference operation order. Any shape, alignment.
hipError_t launch_generic(const GenericArgs& a, bool f32out, hipStream_t stream);

// Device scratch of the allocation-free grouped call
// (ltxw_dequant_lora_grouped_noalloc): the job tables of its launches, in a
// file-scope device array of kScratchBytes per device, held until the
// process ends. Launches queued one after another on one stream reuse it
// from offset 0 (each table is written just before the launch that reads
// it); work from two streams on one device would race.
constexpr size_t kScratchBytes = 64 * 1024;
// Address of the calling thread's current device's copy of the scratch
// array (hipGetSymbolAddress).
hipError_t scratch_address(void** ptr);
// Writes `bytes` (a multiple of 16) of host data to device memory at `dst`
// (16-byte aligned) with kernel launches that carry the bytes as kernel
// arguments: no copy engine, no staging buffer, stream-ordered like any
// other launch.
hipError_t launch_fill_words(void* dst, const void* src, size_t bytes, hipStream_t stream);

}  // namespace ltxw
