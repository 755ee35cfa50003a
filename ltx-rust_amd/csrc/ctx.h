// The context object behind the C ABI and the internal calls shared by the
// kernel entry points (api.cpp) and the weight store (store.cpp).
#pragma once

#include <hip/hip_runtime.h>

#include <string>
#include <vector>

#include "ltxw.h"

struct ltxw_ctx {
  int device = 0;
  int cu_count = 256;
  int host_threads = 8;
  hipStream_t compute = nullptr;
  hipStream_t copy = nullptr;
  // Recorded on the compute stream at each upload, which the copy stream
  // waits for: an upload lands after every operation queued before it.
  hipEvent_t compute_mark = nullptr;
  // Pinned staging ring for host -> device uploads (allocated on first use):
  // n_stage slots of stage_bytes, consecutive in one block. Slot k may be
  // refilled once stage_done[k] (recorded on the copy stream after the
  // slot's last copy) has completed.
  void* stage_block = nullptr;
  std::vector<void*> stage;
  std::vector<hipEvent_t> stage_done;
  size_t stage_bytes = 0;
  int n_stage = 0;
  size_t next_stage = 0;
  // Job tables of grouped launches: a ring of pinned host mirrors -> device
  // buffers, so that the host can queue several launches ahead of the GPU.
  struct TableSlot {
    void* host = nullptr;
    void* dev = nullptr;
    size_t cap = 0;
    hipEvent_t copied = nullptr;  // recorded after the slot's last upload (last slot of a group only)
  };
  std::vector<TableSlot> tables;
  size_t next_table = 0;
  // Device ring of the store's materialisation pipeline: FP8 bytes, scales
  // and factors of one batch of tensors per slot. `ring_free[k]` is recorded
  // on the compute stream after the last kernel that read slot k;
  // `ring_ready[k]` on the copy stream after the slot's last copy.
  std::vector<void*> ring;
  std::vector<hipEvent_t> ring_free, ring_ready;
  size_t ring_bytes = 0;
  // Device scratch of the store: the f32 accumulator of keys merged with
  // more LoRAs than one launch takes (grown on demand).
  void* tmp = nullptr;
  size_t tmp_bytes = 0;
  // This device's copy of the allocation-free call's scratch array
  // (hipGetSymbolAddress at context creation; shared by every context on
  // the device).
  void* scratch = nullptr;
  std::string err;
};

namespace ltxw {

// Records a formatted message on ctx (or the thread's create error) and returns code.
int fail(ltxw_ctx* ctx, int code, const char* fmt, ...) __attribute__((format(printf, 3, 4)));

// Allocates the pinned staging ring if it is not there yet.
int ensure_staging(ltxw_ctx* ctx);

// Per-descriptor extras of the store: the open-time gate fold (scale as a
// plain multiply, then a multiply by `post_mul`, before the LoRA deltas) and
// the NaN rule of chained passes. Descriptors with extras take the
// reference-order kernel.
struct DescEx {
  int32_t plain_scale = 0;
  int32_t has_post = 0;
  float post_mul = 1.0f;
  // Canonicalise NaN results as for an FP8 source (a later pass of a chain
  // whose first pass read FP8 bytes).
  int32_t canon_nan = 0;
};

// Validates and queues the descriptors on the compute stream (the body of
// ltxw_dequant_lora_grouped). `ex` (optional, n entries) routes descriptors
// with extras to the reference-order kernel. `noalloc`: job tables go to the
// device scratch array through fill launches instead of the pinned / device
// table ring (the body of ltxw_dequant_lora_grouped_noalloc; n <=
// LTXW_NOALLOC_MAX_DESCS, checked by the caller).
int run_descs(ltxw_ctx* ctx, const ltxw_tensor_desc* descs, int n, const DescEx* ex = nullptr,
              bool noalloc = false);

// Bytes per element of a base format (ltxw_format); 0 for an unknown one.
inline int format_bytes(int fmt) {
  switch (fmt) {
    case LTXW_FMT_E4M3FN:
    case LTXW_FMT_E5M2: return 1;
    case LTXW_FMT_BF16:
    case LTXW_FMT_F16: return 2;
    case LTXW_FMT_F32: return 4;
    default: return 0;
  }
}

}  // namespace ltxw
