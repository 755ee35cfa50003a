/*
 * CPU oracle for the FP8 dequantisation + LoRA-merge read path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the oracle: tests/, the smoke
 * entry point and the bench's CPU-baseline leg may load it; the product
 * (libltxw) never links, loads or calls it.
 *
 * It restates, in plain C, the arithmetic of ltx-rust's `ltx-weights` read
 * path, in the reference's operation order:
 *
 *   decode (crates/ltx-weights/src/fp8.rs:90-158)
 *   -> scale  v = fma(scale, v, 0)         (crates/ltx-weights/src/store.rs:498-508)
 *   -> LoRA   for o, for r: c = coeff*B[o,r]; for i: w = fma(c, A[r,i], w)
 *                                          (crates/ltx-weights/src/store.rs:767-793)
 *   -> bf16   round-to-nearest-even, NaN quieted with sign kept
 *             (half 2.7.1 `bf16::from_f32`; the reference itself stops at f32)
 *
 * Extensions with no reference counterpart (parity unpinned against the
 * reference, pinned by closed form and brute force in tests/):
 *   - per-output-row scales: out[o,i] = fma(scale[o], v, 0).
 *
 * Everything here is single-pass scalar C; the multi-threaded entry splits
 * rows across threads, which does not change a single bit because every
 * output element's operation sequence is independent of every other's.
 */
#ifndef LTXW_ORACLE_H
#define LTXW_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_E4M3FN = 0, ORC_E5M2 = 1, ORC_BF16 = 2, ORC_F16 = 3, ORC_F32 = 4 };
enum { ORC_SCALE_NONE = 0, ORC_SCALE_TENSOR = 1, ORC_SCALE_ROW = 2 };

/* One low-rank delta, as the reference's `LowRankDelta` (store.rs:756-763):
 * b is [rows x rank], a is [rank x cols], both row-major, in `dtype`
 * (ORC_F32, ORC_BF16, ORC_F16, ORC_E4M3FN or ORC_E5M2; decoded exactly to
 * f32 first, as lora.rs:176-209 does); coeff = strength*alpha/rank. */
typedef struct {
  const void* b;
  const void* a;
  int32_t dtype;
  int32_t rank;
  float coeff;
} orc_lora;

float orc_e4m3fn_to_f32(uint8_t byte);
float orc_e5m2_to_f32(uint8_t byte);
uint16_t orc_bf16_from_f32(float x);
float orc_bf16_to_f32(uint16_t h);
float orc_f16_to_f32(uint16_t h);

/* Decode n raw elements of `dtype` to f32 (store.rs:672-729). */
void orc_decode_to_f32(const void* raw, int dtype, size_t n, float* out);

/* coeff = strength.mul_add(alpha / rank, 0) with alpha defaulting to rank
 * (store.rs:605-615). has_alpha = 0 means no `prefix.alpha` tensor. */
float orc_lora_coeff(float strength, int has_alpha, float alpha, int32_t rank);

/* Reference read path to host f32: decode `base` (rows x cols of
 * base_dtype), apply the FP8 scale (only when base_dtype is FP8 and
 * scale_mode != NONE), then add every LoRA in order. */
void orc_read_f32(const void* base, int base_dtype, int64_t rows, int64_t cols,
                  int scale_mode, const float* scales,
                  const orc_lora* loras, int n_loras, float* out);

/* Same, rows split over nthreads POSIX threads (bit-identical). */
void orc_read_f32_mt(const void* base, int base_dtype, int64_t rows, int64_t cols,
                     int scale_mode, const float* scales,
                     const orc_lora* loras, int n_loras, float* out, int nthreads);

/* orc_read_f32 followed by bf16 RNE of every element. */
void orc_read_bf16_mt(const void* base, int base_dtype, int64_t rows, int64_t cols,
                      int scale_mode, const float* scales,
                      const orc_lora* loras, int n_loras, uint16_t* out, int nthreads);

/* Exact-arithmetic reference in f64: scale*dec(w) + sum_l coeff_l*(B_l A_l),
 * with every product and sum carried in double. Rows [row0, row0+nrows). */
void orc_read_f64_rows(const void* base, int base_dtype, int64_t rows, int64_t cols,
                       int scale_mode, const float* scales,
                       const orc_lora* loras, int n_loras,
                       int64_t row0, int64_t nrows, double* out);

/* Conditioning bound per element for the LoRA sum: scale-free magnitude
 * |deq| + sum_l |coeff_l| * sum_r |B[o,r]|*|A[r,i]| (double). Rows as above. */
void orc_abs_bound_rows(const void* base, int base_dtype, int64_t rows, int64_t cols,
                        int scale_mode, const float* scales,
                        const orc_lora* loras, int n_loras,
                        int64_t row0, int64_t nrows, double* out);

/* Test hook: plant a deliberate mistake so tests can show that their
 * checks catch it. 0 = none (default). Values are listed in oracle.c. */
void orc_set_mutation(int m);

#ifdef __cplusplus
}
#endif
#endif
