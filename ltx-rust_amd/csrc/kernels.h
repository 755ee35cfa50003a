// Kernel launchers shared by the C ABI (api.cpp). Host-side declarations only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ltxw {

constexpr int kMaxLoras = 4;

// Tile of the fused kernel: TM output rows x TN output columns per workgroup.
constexpr int kTileM = 128;
constexpr int kTileN = 128;

struct LoraDev {
  const uint16_t* b;  // bf16 [rows x rank]
  const uint16_t* a;  // bf16 [rank x cols]
  int32_t rank;
  float coeff;
};

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
  int32_t tiles_n;     // tiles along cols
  int64_t tile_begin;  // first flat tile index of this job in the launch
  LoraDev lora[kMaxLoras];
};

struct JobTable {
  JobDev one;            // used when n_jobs == 1 (no device table needed)
  const JobDev* jobs;    // device array when n_jobs > 1
  const int64_t* begins; // device array of tile_begin, ascending
  int32_t n_jobs;
  int64_t total_tiles;
};

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
};

// Streaming dequant: n_chunks * 16 elements. Pointers 16-byte aligned.
hipError_t launch_dequant(const DequantArgs& a, int fmt, int scale_mode, bool f32out,
                          hipStream_t stream);

// Fused dequant + LoRA over every tile of every job. Requirements checked by
// the caller: cols % 8 == 0, ranks % 8 == 0, all pointers 16-byte aligned.
hipError_t launch_fused(const JobTable& t, bool f32out, bool multi, hipStream_t stream);

// One thread per element, reference operation order. Any shape, alignment.
hipError_t launch_generic(const GenericArgs& a, bool f32out, hipStream_t stream);

}  // namespace ltxw
