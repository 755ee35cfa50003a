/*
 * ltxw — MI355X (gfx950) FP8 dequantisation + LoRA merge for ltx-rust's
 * `ltx-weights` read path. Plain C ABI: plain pointers and sizes, status
 * codes, no exceptions and no aborts across the boundary.
 *
 * Device pointers below are HBM addresses returned by ltxw_alloc (or any
 * hipMalloc'd memory on the context's device). Every operation runs on the
 * context's compute stream in call order; ltxw_synchronize waits for it.
 *
 * Reference interfaces these entry points replace (ltx-rust, crates/ltx-weights):
 *   - FP8 decode + scale in `WeightStore::read`      src/store.rs:479-508, src/fp8.rs:35-43,90-158
 *   - the LoRA expansion `LowRankDelta::add_to`     src/store.rs:767-793 (applied at :510-515)
 *   - the factor bookkeeping of `merge_lora`        src/store.rs:542-640 (coeff at :605-615)
 *   - `Entry::read_raw`'s host copy of mmap bytes   src/store.rs:45-78 (replaced by staged upload)
 *   - `WeightStore::open` / `LoraFile::open`        src/store.rs:124-208, src/lora.rs:60-85
 */
#ifndef LTXW_H
#define LTXW_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. Errors mirror the reference's `WeightError` variants where one
 * exists (src/error.rs:7-100); the message is available from ltxw_last_error. */
typedef enum {
  LTXW_OK = 0,
  LTXW_ERR_INVALID_ARG = 1,    /* null pointer, negative/overflowing size, bad enum */
  LTXW_ERR_UNSUPPORTED = 2,    /* WeightError::UnsupportedDtype */
  LTXW_ERR_OOM = 3,            /* device or pinned allocation failed */
  LTXW_ERR_HIP = 4,            /* HIP runtime error (message carries hipGetErrorString) */
  LTXW_ERR_IO = 5,             /* WeightError::Io */
  LTXW_ERR_FORMAT = 6,         /* WeightError::Safetensors / InvalidTensorData */
  LTXW_ERR_MISSING_KEY = 7,    /* WeightError::MissingKey */
  LTXW_ERR_DUPLICATE_KEY = 8,  /* WeightError::DuplicateKey */
  LTXW_ERR_LORA_SHAPE = 9,     /* WeightError::LoraShapeMismatch */
  LTXW_ERR_LORA_RANK = 10,     /* WeightError::LoraRankMismatch */
  LTXW_ERR_NO_LORA_MATCHES = 11, /* WeightError::NoLoraMatches */
  LTXW_ERR_QKV_SPLIT_DIM = 12,   /* WeightError::QkvSplitDim */
  LTXW_ERR_GATE_NOT_SCALAR = 13  /* WeightError::GateNotScalar */
} ltxw_status;

/* Base-weight storage formats: the FP8 formats of the hot path (safetensors
 * "F8_E4M3" / "F8_E5M2"; src/fp8.rs:3-7) and the other dtypes `read` widens
 * (src/store.rs:672-729: "BF16", "F16", "F32"). Scales apply to FP8 only
 * (src/store.rs:500); the non-FP8 formats take the one-element-per-thread path. */
typedef enum {
  LTXW_FMT_E4M3FN = 0,
  LTXW_FMT_E5M2 = 1,
  LTXW_FMT_BF16 = 2,
  LTXW_FMT_F16 = 3,
  LTXW_FMT_F32 = 4
} ltxw_format;

/* Scale convention. TENSOR is the reference's `{key}_scale` scalar
 * (src/store.rs:498-508: v = fma(scale, v, 0)). ROW (one f32 per output row,
 * out[o,i] = fma(scale[o], v, 0)) is an extension with no reference counterpart. */
typedef enum { LTXW_SCALE_NONE = 0, LTXW_SCALE_TENSOR = 1, LTXW_SCALE_ROW = 2 } ltxw_scale_mode;

/* Output element type: bf16 (round-to-nearest-even of the reference's f32)
 * or the reference's own f32 (`HostTensor.data`, src/host_tensor.rs:13-18). */
typedef enum { LTXW_OUT_BF16 = 0, LTXW_OUT_F32 = 1 } ltxw_out_dtype;

/* Maximum LoRAs merged into one tensor in a single launch. */
#define LTXW_MAX_LORAS 4

/* Element type of LoRA factors (src/lora.rs:176-209 widens all of them to
 * f32 exactly). BF16 (zero, the default) takes the MFMA path; the others take
 * the one-element-per-thread path in the reference's operation order. */
typedef enum {
  LTXW_FACTOR_BF16 = 0,
  LTXW_FACTOR_F32 = 1,
  LTXW_FACTOR_F16 = 2,
  LTXW_FACTOR_E4M3FN = 3,
  LTXW_FACTOR_E5M2 = 4
} ltxw_factor_dtype;

/* One low-rank delta coeff * (B @ A), the device form of the reference's
 * `LowRankDelta` (src/store.rs:751-763). B is [rows x rank] row-major
 * (`prefix.lora_B.weight`), A is [rank x cols] row-major
 * (`prefix.lora_A.weight`), both of element type `dtype`, aligned to it;
 * coeff = strength * alpha / rank (src/store.rs:615). */
typedef struct {
  const void* b;
  const void* a;
  int32_t rank;
  float coeff;
  int32_t dtype;     /* ltxw_factor_dtype */
  int32_t reserved;  /* 0 */
} ltxw_lora;

/* One tensor to materialise in a grouped launch. */
typedef struct {
  const uint8_t* w;        /* device [rows x cols] in `fmt` (element-aligned) */
  void* out;               /* device bf16 or f32 [rows x cols] */
  const float* scales;     /* device f32: 1 (TENSOR) or rows (ROW) values; NULL for NONE */
  int64_t rows;
  int64_t cols;
  int32_t fmt;             /* ltxw_format */
  int32_t scale_mode;      /* ltxw_scale_mode */
  int32_t out_dtype;       /* ltxw_out_dtype */
  int32_t n_loras;         /* 0..LTXW_MAX_LORAS, merged in array order */
  int32_t flags;           /* LTXW_DESC_* */
  ltxw_lora loras[LTXW_MAX_LORAS];
} ltxw_tensor_desc;

/* Bit-identical results with LoRA deltas: the reference's own operation
 * order (per element, per rank: w = fma(coeff * B[o,r], A[r,i], w)) instead
 * of the MFMA product. Slower (r FMAs per element on the vector units).
 * Tensors without deltas, and deltas the MFMA path does not take, are
 * bit-identical either way. */
#define LTXW_DESC_EXACT 1

typedef struct ltxw_ctx ltxw_ctx;

/* Create a context on HIP device `device` with a ring of `n_staging` pinned
 * host buffers of `staging_bytes` each (a multiple of 4096) for host->device
 * uploads (0 picks 64 MiB x 16; one pinned block, allocated on first use).
 * No reference counterpart: the reference has no device. */
int ltxw_ctx_create(int device, size_t staging_bytes, int n_staging, ltxw_ctx** out);
void ltxw_ctx_destroy(ltxw_ctx* ctx);

/* Host threads that copy mapped file bytes into the pinned ring during
 * ltxw_store_materialize (default min(8, hardware threads)). */
int ltxw_ctx_set_host_threads(ltxw_ctx* ctx, int n);

/* Message of the last failed call on this context ("" if none). With a NULL
 * context, the message of the last failed ltxw_ctx_create on this thread. */
const char* ltxw_last_error(const ltxw_ctx* ctx);

/* Device memory (replaces the reference's owned Vec<f32> result buffers). */
int ltxw_alloc(ltxw_ctx* ctx, size_t bytes, void** dptr);
int ltxw_free(ltxw_ctx* ctx, void* dptr);
int ltxw_memset(ltxw_ctx* ctx, void* dptr, int value, size_t bytes);

/* Host -> device copy staged through the pinned ring on the copy stream, in
 * call order: it starts after every operation queued on the context before
 * it (so a device buffer may be refilled while a kernel that reads it is
 * still queued), and the compute stream waits for it, so later operations
 * see the data. The host buffer may be reused as soon as the call returns
 * (it has been staged).
 * Replaces `Entry::read_raw`'s `to_vec` copy (src/store.rs:45-78). */
int ltxw_upload(ltxw_ctx* ctx, const void* host_src, size_t bytes, void* dst);

/* Device -> host copy after all prior work on the context (synchronous). */
int ltxw_download(ltxw_ctx* ctx, const void* src, size_t bytes, void* host_dst);

/* Wait until all work queued on the context has finished. */
int ltxw_synchronize(ltxw_ctx* ctx);

/* Dequantisation of one [rows x cols] tensor to out_dtype:
 * out = RNE(fma(scale, LUT[w], 0)) (or RNE(LUT[w]) for NONE); non-FP8
 * formats are widened exactly and take no scale.
 * Replaces the decode + scale of `WeightStore::read` (src/store.rs:488-508). */
int ltxw_dequant(ltxw_ctx* ctx, const uint8_t* w, int64_t rows, int64_t cols, int fmt,
                 int scale_mode, const float* scales, void* out, int out_dtype);

/* Fused dequant + LoRA merge of one tensor:
 * out = deq(w) + sum_l coeff_l * (B_l @ A_l), with B_l @ A_l on bf16 MFMA in f32.
 * Replaces `WeightStore::read` with merged deltas (src/store.rs:479-521,767-793).
 * `loras` is a host array of n_loras entries (device factor pointers). */
int ltxw_dequant_lora(ltxw_ctx* ctx, const uint8_t* w, int64_t rows, int64_t cols, int fmt,
                      int scale_mode, const float* scales, const ltxw_lora* loras,
                      int n_loras, void* out, int out_dtype);

/* Many tensors in one launch sequence (e.g. a whole DiT block), one kernel
 * per distinct path. `descs` is a host array. Replaces a loop of
 * `Scope::tensor` -> `read` over a block's linears (ltx-dit src/load.rs:149-170). */
int ltxw_dequant_lora_grouped(ltxw_ctx* ctx, const ltxw_tensor_desc* descs, int n);

/* ltxw_dequant_lora_grouped for callers that cannot allocate memory (code
 * under HIP graph capture, serving loops, harnesses that forbid it): the
 * same kernels and results (bit-identical), but no allocation of any kind
 * on the device or in pinned host memory. Job tables too large for a
 * launch's kernel arguments (more than about 20 tensors in one fused
 * launch) go to a static device array of 64 KiB per device (held until the
 * process ends), filled by small kernel launches that carry the table in
 * their arguments; calls with more than LTXW_NOALLOC_MAX_DESCS descriptors are
 * rejected (LTXW_ERR_INVALID_ARG) before anything is queued. Every context
 * on a device shares its array: calls queued on one context run in order,
 * but calls from two contexts on the same device that overlap in time race.
 * No counterpart in the reference (which has no device); added for callers
 * that cannot allocate. */
#define LTXW_NOALLOC_MAX_DESCS 128
int ltxw_dequant_lora_grouped_noalloc(ltxw_ctx* ctx, const ltxw_tensor_desc* descs, int n);

/* The context's compute stream (a hipStream_t), for callers that time or
 * order their own work against ltxw's. */
void* ltxw_ctx_stream(ltxw_ctx* ctx);

#ifdef __cplusplus
}
#endif
#endif
