/*
 * ltxw store — the host front end of ltx-rust's `ltx-weights` crate over the
 * ltxw device path: memory-mapped safetensors checkpoints, key renaming,
 * LoRA adapter files and their merge bookkeeping, and materialisation of
 * dequantised + merged tensors into HBM through a pinned staging pipeline.
 *
 * Reference interfaces (ltx-rust, crates/ltx-weights):
 *   - `WeightStore::open`                 src/store.rs:124-208 (KeyMap: src/key_map.rs:30-86, 237-268)
 *   - `keys` / `contains` / `shape` / `metadata`  src/store.rs:425-467
 *   - `WeightStore::read`                 src/store.rs:479-521
 *   - `WeightStore::merge_lora`           src/store.rs:542-640, `MergeReport` src/lora.rs:157-170
 *   - `LoraFile::{open, metadata, ic_layout, tensor_names, read_f32, tensor_info}`  src/lora.rs:43-152
 *
 * Error messages: every call that fails records a message for the calling
 * thread, read with ltxw_store_last_error(). Status codes are ltxw_status.
 * A store may be read from several threads at once (each with its own
 * context); ltxw_store_merge_lora and ltxw_store_close need exclusive access,
 * as `merge_lora(&mut self)` does.
 */
#ifndef LTXW_STORE_H
#define LTXW_STORE_H

#include "ltxw.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ltxw_store ltxw_store;
typedef struct ltxw_lora_file ltxw_lora_file;
typedef struct ltxw_merge_report ltxw_merge_report;

/* safetensors element types (the header's "dtype" strings). */
typedef enum {
  LTXW_DT_BOOL = 0, LTXW_DT_U8 = 1, LTXW_DT_I8 = 2, LTXW_DT_F8_E5M2 = 3, LTXW_DT_F8_E4M3 = 4,
  LTXW_DT_I16 = 5, LTXW_DT_U16 = 6, LTXW_DT_F16 = 7, LTXW_DT_BF16 = 8, LTXW_DT_I32 = 9,
  LTXW_DT_U32 = 10, LTXW_DT_F32 = 11, LTXW_DT_F64 = 12, LTXW_DT_I64 = 13, LTXW_DT_U64 = 14,
  LTXW_DT_F8_E8M0 = 15, LTXW_DT_F4 = 16, LTXW_DT_F6_E2M3 = 17, LTXW_DT_F6_E3M2 = 18, LTXW_DT_C64 = 19
} ltxw_dtype;

/* One rule of the reference's `KeyMap` (src/key_map.rs:30-86), applied in
 * order to every checkpoint key at open (`apply_key`, src/key_map.rs:237-268). */
typedef enum {
  LTXW_RULE_REQUIRE_ANY_PREFIX = 0, /* strs[0..n): drop keys starting with none of them (n == 0: keep all) */
  LTXW_RULE_REPLACE = 1,            /* n == 2: replace every occurrence of strs[0] by strs[1] */
  LTXW_RULE_DROP_PREFIX = 2,        /* n == 1: drop keys starting with strs[0] */
  LTXW_RULE_DROP_SUFFIX = 3,        /* n == 1: drop keys ending with strs[0] */
  LTXW_RULE_RENAME_EXACT = 4,       /* n == 2: a leading strs[0] becomes strs[1] */
  /* Open-time value transforms (n == 0), applied after renaming in this
   * order whatever their position in the list (src/store.rs:190-198):
   *   FOLD_GATES (src/store.rs:217-293): `.gate_msa/.gate_mlp/.gate_ctx`
   *     scalars (else LTXW_ERR_GATE_NOT_SCALAR) multiply their targets
   *     (`.attn.proj`, `.mlp.w_down`, `.context_proj` weight/bias) as
   *     (v [* scale]) * gate in f32, plain multiplies; gates and the targets'
   *     scale siblings disappear;
   *   SPLIT_QKV (src/store.rs:302-390): `P.qkv.{weight,bias}` with leading dim
   *     3d becomes `P.to_{q,k,v}.*` of leading dim d, FP8 scaled as `read`
   *     would (leading dim not a multiple of 3: LTXW_ERR_QKV_SPLIT_DIM);
   *   SYNTH_ZERO_TYPE_EMB (src/store.rs:398-419): a zero f32 `type_emb` of
   *     conv_in.weight's dim 1 when absent.
   * Transformed entries report dtype F32, as the reference's owned f32
   * copies do; their values are computed on the device when read. */
  LTXW_RULE_SPLIT_QKV = 5,
  LTXW_RULE_FOLD_GATES = 6,
  LTXW_RULE_SYNTH_ZERO_TYPE_EMB = 7
} ltxw_rule_kind;

typedef struct {
  int32_t kind;             /* ltxw_rule_kind */
  int32_t n;                /* number of strings */
  const char* const* strs;  /* UTF-8, NUL-terminated */
} ltxw_key_rule;

/* Message of the calling thread's last failed store / LoRA-file call. */
const char* ltxw_store_last_error(void);

/* Open and map one or more safetensors files (src/store.rs:124-208). Keys are
 * renamed by `rules`; a key defined twice after renaming is
 * LTXW_ERR_DUPLICATE_KEY; `__metadata__` merges with the first file winning.
 * `{key}_scale` siblings of FP8 tensors become internal (src/store.rs:174-187). */
int ltxw_store_open(const char* const* paths, int n_paths, const ltxw_key_rule* rules, int n_rules,
                    ltxw_store** out);
void ltxw_store_close(ltxw_store* s);

/* Visible keys (scale siblings excluded), in byte order of the key strings.
 * The string stays valid until the store is closed. */
int64_t ltxw_store_n_keys(const ltxw_store* s);
const char* ltxw_store_key(const ltxw_store* s, int64_t index);
/* 1 if `key` is present and visible, else 0 (src/store.rs:453-456). */
int ltxw_store_contains(const ltxw_store* s, const char* key);
/* dtype and shape of any entry, scale siblings included (src/store.rs:462-467).
 * Writes *ndim; shape[0..min(*ndim, max_dims)). */
int ltxw_store_tensor_info(const ltxw_store* s, const char* key, int32_t* dtype, int32_t* ndim,
                           int64_t* shape, int32_t max_dims);
/* Merged `__metadata__` value, or NULL when absent (src/store.rs:425-427). */
const char* ltxw_store_metadata(const ltxw_store* s, const char* key);

/* LoRA adapter file (src/lora.rs:60-85). */
int ltxw_lora_open(const char* path, ltxw_lora_file** out);
void ltxw_lora_close(ltxw_lora_file* f);
int64_t ltxw_lora_n_tensors(const ltxw_lora_file* f);
const char* ltxw_lora_tensor_name(const ltxw_lora_file* f, int64_t index);  /* byte order */
int ltxw_lora_tensor_info(const ltxw_lora_file* f, const char* name, int32_t* dtype, int32_t* ndim,
                          int64_t* shape, int32_t max_dims);
const char* ltxw_lora_metadata(const ltxw_lora_file* f, const char* key);
/* `reference_downscale_factor` / `reference_temporal_scale_factor`, 1 when
 * absent or not a u32; a stored 0 is LTXW_ERR_INVALID_ARG (src/lora.rs:105-110). */
int ltxw_lora_ic_layout(const ltxw_lora_file* f, uint32_t* downscale, uint32_t* temporal);
/* Host f32 copy of one tensor, n == its element count (src/lora.rs:124-146):
 * F32/F16/BF16/F8 widen exactly; a missing name is LTXW_ERR_MISSING_KEY. */
int ltxw_lora_read_f32(const ltxw_lora_file* f, const char* name, float* out, int64_t n);

/* Merge a LoRA file (src/store.rs:542-640): every `P.lora_A.weight` with a
 * base key `P.weight` in the store and a `P.lora_B.weight` gets a delta of
 * coefficient strength * alpha / rank (alpha from `P.alpha`, default rank).
 * Deltas stack across calls in call order. The file may be closed afterwards
 * (the store keeps it mapped). `report` (optional) receives a report to free
 * with ltxw_report_free. Errors leave the store unchanged. */
int ltxw_store_merge_lora(ltxw_store* s, const ltxw_lora_file* f, float strength, ltxw_merge_report** report);
/* Matched base keys / unmatched `lora_A` keys, each in byte order. */
int64_t ltxw_report_n_matched(const ltxw_merge_report* r);
const char* ltxw_report_matched(const ltxw_merge_report* r, int64_t index);
int64_t ltxw_report_n_unmatched(const ltxw_merge_report* r);
const char* ltxw_report_unmatched(const ltxw_merge_report* r, int64_t index);
void ltxw_report_free(ltxw_merge_report* r);
/* Merged deltas of a key, in application order: rank and coefficient. */
int ltxw_store_n_deltas(const ltxw_store* s, const char* key);
int ltxw_store_delta(const ltxw_store* s, const char* key, int index, int32_t* rank, float* coeff);

/* Options of ltxw_store_materialize and ltxw_store_read.
 * Scales: materialize scales row o by element o of a `{key}_scale` with
 *   exactly shape[0] elements (shape[0] > 1, two or more dims; an extension:
 *   per-output-channel FP8 scales) and by element 0 otherwise; read always by
 *   element 0 (src/store.rs:498-508, :732-735; empty: 1.0).
 *   LTXW_MAT_SCALE_FIRST selects the element-0 rule for materialize,
 *   LTXW_MAT_ROW_SCALES the per-row rule for read.
 * LoRA deltas: both run them in the reference's operation order by default
 *   (bit-identical to the reference's f32, then RNE for bf16). Materialize is
 *   bound by the host -> HBM copies, which hide these kernels (a 22B-parameter
 *   set with rank-64 deltas: 0.425 s either way). LTXW_MAT_MFMA selects the
 *   MFMA kernels where they take the tensor (within 1 bf16 ulp of the
 *   reference's result but for ill-conditioned elements); LTXW_MAT_EXACT
 *   states the default explicitly.
 * A rule and its opposite together are LTXW_ERR_INVALID_ARG. */
#define LTXW_MAT_SCALE_FIRST 1u
#define LTXW_MAT_EXACT 2u
#define LTXW_MAT_ROW_SCALES 4u
#define LTXW_MAT_MFMA 8u

/* Materialise tensors into caller-allocated device buffers: outs[k] holds
 * numel(keys[k]) elements of out_dtype (ltxw_out_dtype) in row-major order.
 * Per key: the base tensor widened (FP8: decoded and scaled), plus every
 * merged delta, as `read` (src/store.rs:479-521) computes it, rounded to
 * bf16 (RNE) or kept f32. Non-FP8 base tensors and >= 2-D shapes are
 * accepted; a key with deltas must be [out, in] (src/store.rs:767-779).
 * LoRA factors of every type `merge_lora` accepts are taken. A key merged with more
 * than LTXW_MAX_LORAS deltas runs all of them in the reference's order, in
 * passes of up to LTXW_MAX_LORAS deltas through an f32 accumulator (for bf16
 * output a device scratch buffer of 4 bytes per element, kept by the context).
 *
 * Bytes go mapped file -> pinned ring (ctx host threads) -> HBM on the copy
 * stream, batch by batch through a device ring, and each batch is
 * dequantised + merged on the compute stream while the next one copies.
 * Returns once every host read is done; the kernels complete in stream
 * order (ltxw_synchronize waits). New item with no reference counterpart;
 * it stands for `materialize_bf16` beside `read`. */
int ltxw_store_materialize(ltxw_store* s, ltxw_ctx* ctx, const char* const* keys, int64_t n_keys,
                           int32_t out_dtype, uint32_t flags, void* const* outs);

/* `WeightStore::read` (src/store.rs:479-521) on the device: the f32 tensor
 * into host memory (n == numel), bit-identical to the reference's (element-0
 * scale rule, every merged delta in merge order and in the reference's
 * operation order). `flags` (LTXW_MAT_ROW_SCALES, LTXW_MAT_MFMA) opt into the
 * extensions. Synchronous. */
int ltxw_store_read(ltxw_store* s, ltxw_ctx* ctx, const char* key, uint32_t flags, float* out, int64_t n);

#ifdef __cplusplus
}
#endif
#endif
