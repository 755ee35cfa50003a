/*
 * CPU oracle for the FP8 dequantisation + LoRA-merge read path.
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, the smoke entry point and the
 * bench's CPU-baseline leg as the reference the HIP path is compared with;
 * never part of the product.
 *
 * Each function cites the reference file:line whose arithmetic it restates.
 * Compile without -ffast-math (signed zeros, NaN and fma must stay IEEE).
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* Planted-mistake switch for the tests that show the checks have teeth.
 *   1 e4m3fn subnormal step 2^-8 instead of 2^-9
 *   2 scale as plain s*v (keeps -0) instead of fma(s, v, 0)
 *   3 LoRA reads B transposed (B[r*rows + o])
 *   4 LoRA drops the coefficient (c = B[o,r])
 *   5 bf16 by truncation instead of round-to-nearest-even
 *   6 LoRA added before the scale (scale multiplies the delta too)
 *   7 per-row scale indexed by column
 *   8 alpha default 1 instead of rank
 *   9 e5m2 exponent bias 16 instead of 15
 *  10 f16 subnormal step 2^-25 instead of 2^-24
 *  11 f16 NaN without the quiet bit
 */
static int g_mutation = 0;
void orc_set_mutation(int m) { g_mutation = m; }

static inline float f_from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t bits_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* fp8.rs:90-120. S EEEE MMM, bias 7; 0x7F/0xFF NaN; no infinities.
 * Subnormal (E = 0): M * 2^-9, which is what the reference's per-mantissa
 * (exp, mant) table at fp8.rs:104-112 spells out bit by bit. */
float orc_e4m3fn_to_f32(uint8_t byte) {
  if (byte == 0x7F || byte == 0xFF) return f_from_bits(0x7FC00000u); /* f32::NAN */
  uint32_t sign = (byte & 0x80u) ? 0x80000000u : 0u;
  uint32_t e = (byte >> 3) & 0x0Fu, m = byte & 0x07u;
  if (e == 0) {
    if (m == 0) return f_from_bits(sign);
    float mag = (float)m * (g_mutation == 1 ? 0x1p-8f : 0x1p-9f);
    return f_from_bits(sign | bits_of(mag));
  }
  return f_from_bits(sign | ((e + 120u) << 23) | (m << 20));
}

/* fp8.rs:127-158. S EEEEE MM, bias 15; E = 31 is Inf (M = 0) or NaN. */
float orc_e5m2_to_f32(uint8_t byte) {
  uint32_t sign = (byte & 0x80u) ? 0x80000000u : 0u;
  uint32_t e = (byte >> 2) & 0x1Fu, m = byte & 0x03u;
  if (e == 31) return m == 0 ? f_from_bits(sign | 0x7F800000u) : f_from_bits(0x7FC00000u);
  if (e == 0) {
    if (m == 0) return f_from_bits(sign);
    return f_from_bits(sign | bits_of((float)m * 0x1p-16f));
  }
  uint32_t bias_adj = g_mutation == 9 ? 111u : 112u;
  return f_from_bits(sign | ((e + bias_adj) << 23) | (m << 21));
}

/* bf16 round-to-nearest-even with the NaN rule of half 2.7.1
 * (`bf16::from_f32`: NaN keeps sign and top mantissa bits, quiet bit set).
 * Adding 0x7FFF plus the kept LSB and truncating is the same rounding as
 * half's "round bit set and (sticky or LSB)" test. */
uint16_t orc_bf16_from_f32(float x) {
  uint32_t u = bits_of(x);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x0040u);
  if (g_mutation == 5) return (uint16_t)(u >> 16);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t h) { return f_from_bits((uint32_t)h << 16); }

/* IEEE binary16 -> f32, exact (half 2.7.1 `f16::to_f32`, used by
 * store.rs:690-705 and lora.rs:186-193). NaN: quiet bit set, payload kept. */
float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
  if (e == 31) {
    if (m == 0) return f_from_bits(sign | 0x7F800000u);
    return f_from_bits(sign | (g_mutation == 11 ? 0x7F800000u : 0x7FC00000u) | (m << 13));
  }
  if (e == 0) {
    float mag = (float)m * (g_mutation == 10 ? 0x1p-25f : 0x1p-24f);
    return f_from_bits(sign | bits_of(mag));
  }
  return f_from_bits(sign | ((e + 112u) << 23) | (m << 13));
}

/* store.rs:672-729: little-endian element decode per dtype. */
void orc_decode_to_f32(const void* raw, int dtype, size_t n, float* out) {
  const uint8_t* p = (const uint8_t*)raw;
  for (size_t k = 0; k < n; ++k) {
    switch (dtype) {
      case ORC_E4M3FN: out[k] = orc_e4m3fn_to_f32(p[k]); break;
      case ORC_E5M2: out[k] = orc_e5m2_to_f32(p[k]); break;
      case ORC_BF16: out[k] = orc_bf16_to_f32((uint16_t)(p[2 * k] | (p[2 * k + 1] << 8))); break;
      case ORC_F16: out[k] = orc_f16_to_f32((uint16_t)(p[2 * k] | (p[2 * k + 1] << 8))); break;
      default: {
        uint32_t u = (uint32_t)p[4 * k] | ((uint32_t)p[4 * k + 1] << 8) |
                     ((uint32_t)p[4 * k + 2] << 16) | ((uint32_t)p[4 * k + 3] << 24);
        out[k] = f_from_bits(u);
      }
    }
  }
}

/* store.rs:605-615: alpha defaults to rank; coeff = strength.mul_add(alpha/rank, 0). */
float orc_lora_coeff(float strength, int has_alpha, float alpha, int32_t rank) {
  float r = (float)rank;
  float a = has_alpha ? alpha : (g_mutation == 8 ? 1.0f : r);
  return fmaf(strength, a / r, 0.0f);
}

static int is_fp8(int dtype) { return dtype == ORC_E4M3FN || dtype == ORC_E5M2; }

typedef struct {
  float* b;
  float* a;
  int32_t rank;
  float coeff;
} dense_lora;

/* lora.rs:176-209 decodes factors to f32 once per merge; done here per call. */
static dense_lora* widen_loras(const orc_lora* loras, int n, int64_t rows, int64_t cols) {
  if (n <= 0) return NULL;
  dense_lora* d = (dense_lora*)calloc((size_t)n, sizeof(dense_lora));
  for (int l = 0; l < n; ++l) {
    size_t nb = (size_t)rows * (size_t)loras[l].rank, na = (size_t)loras[l].rank * (size_t)cols;
    d[l].b = (float*)malloc(nb * sizeof(float));
    d[l].a = (float*)malloc(na * sizeof(float));
    orc_decode_to_f32(loras[l].b, loras[l].dtype, nb, d[l].b);
    orc_decode_to_f32(loras[l].a, loras[l].dtype, na, d[l].a);
    d[l].rank = loras[l].rank;
    d[l].coeff = loras[l].coeff;
  }
  return d;
}

static void free_loras(dense_lora* d, int n) {
  if (!d) return;
  for (int l = 0; l < n; ++l) { free(d[l].b); free(d[l].a); }
  free(d);
}

static size_t elem_size(int dtype) {
  return is_fp8(dtype) ? 1 : (dtype == ORC_F32 ? 4 : 2);
}

/* store.rs:767-793 `LowRankDelta::add_to` on one row: for r in rank order,
 * c = scale * B[o,r] (rounded), then w[i] = fma(c, A[r,i], w[i]). */
static void lora_row(const dense_lora* L, int64_t rows, int64_t cols, int64_t o, float* w) {
  for (int32_t r = 0; r < L->rank; ++r) {
    float bval = g_mutation == 3 ? L->b[(size_t)r * (size_t)rows + (size_t)o]
                                 : L->b[(size_t)o * (size_t)L->rank + (size_t)r];
    float c = g_mutation == 4 ? bval : L->coeff * bval;
    const float* arow = L->a + (size_t)r * (size_t)cols;
    for (int64_t i = 0; i < cols; ++i) w[i] = fmaf(c, arow[i], w[i]);
  }
}

/* One output row of store.rs:479-521: decode, FP8 scale (498-508), LoRA (510-515). */
static void read_row(const uint8_t* base, int base_dtype, int64_t rows, int64_t cols,
                     int scale_mode, const float* scales, const dense_lora* d, int n_loras,
                     int64_t o, float* w) {
  size_t es = elem_size(base_dtype);
  orc_decode_to_f32(base + (size_t)o * (size_t)cols * es, base_dtype, (size_t)cols, w);
  if (g_mutation == 6)
    for (int l = 0; l < n_loras; ++l) lora_row(&d[l], rows, cols, o, w);
  if (is_fp8(base_dtype) && scale_mode != ORC_SCALE_NONE) {
    for (int64_t i = 0; i < cols; ++i) {
      float s = scale_mode == ORC_SCALE_TENSOR ? scales[0]
                : (g_mutation == 7 ? scales[i % rows] : scales[o]);
      w[i] = g_mutation == 2 ? s * w[i] : fmaf(s, w[i], 0.0f);
    }
  }
  if (g_mutation != 6)
    for (int l = 0; l < n_loras; ++l) lora_row(&d[l], rows, cols, o, w);
}

void orc_read_f32(const void* base, int base_dtype, int64_t rows, int64_t cols,
                  int scale_mode, const float* scales,
                  const orc_lora* loras, int n_loras, float* out) {
  orc_read_f32_mt(base, base_dtype, rows, cols, scale_mode, scales, loras, n_loras, out, 1);
}

typedef struct {
  const uint8_t* base;
  int base_dtype;
  int64_t rows, cols;
  int scale_mode;
  const float* scales;
  const dense_lora* d;
  int n_loras;
  int64_t r0, r1;
  float* out_f32;
  uint16_t* out_bf16;
} job_t;

static void* run_job(void* arg) {
  job_t* j = (job_t*)arg;
  float* tmp = j->out_f32 ? NULL : (float*)malloc((size_t)j->cols * sizeof(float));
  for (int64_t o = j->r0; o < j->r1; ++o) {
    float* w = j->out_f32 ? j->out_f32 + (size_t)o * (size_t)j->cols : tmp;
    read_row(j->base, j->base_dtype, j->rows, j->cols, j->scale_mode, j->scales, j->d,
             j->n_loras, o, w);
    if (j->out_bf16) {
      uint16_t* dst = j->out_bf16 + (size_t)o * (size_t)j->cols;
      for (int64_t i = 0; i < j->cols; ++i) dst[i] = orc_bf16_from_f32(w[i]);
    }
  }
  free(tmp);
  return NULL;
}

static void run_threads(const void* base, int base_dtype, int64_t rows, int64_t cols,
                        int scale_mode, const float* scales, const orc_lora* loras,
                        int n_loras, float* out_f32, uint16_t* out_bf16, int nthreads) {
  dense_lora* d = widen_loras(loras, n_loras, rows, cols);
  if (nthreads < 1) nthreads = 1;
  if (nthreads > rows) nthreads = rows > 0 ? (int)rows : 1;
  job_t* jobs = (job_t*)calloc((size_t)nthreads, sizeof(job_t));
  pthread_t* th = (pthread_t*)calloc((size_t)nthreads, sizeof(pthread_t));
  for (int t = 0; t < nthreads; ++t) {
    job_t* j = &jobs[t];
    j->base = (const uint8_t*)base; j->base_dtype = base_dtype; j->rows = rows; j->cols = cols;
    j->scale_mode = scale_mode; j->scales = scales; j->d = d; j->n_loras = n_loras;
    j->r0 = rows * t / nthreads; j->r1 = rows * (t + 1) / nthreads;
    j->out_f32 = out_f32; j->out_bf16 = out_bf16;
  }
  for (int t = 1; t < nthreads; ++t) pthread_create(&th[t], NULL, run_job, &jobs[t]);
  run_job(&jobs[0]);
  for (int t = 1; t < nthreads; ++t) pthread_join(th[t], NULL);
  free(th); free(jobs);
  free_loras(d, n_loras);
}

void orc_read_f32_mt(const void* base, int base_dtype, int64_t rows, int64_t cols,
                     int scale_mode, const float* scales,
                     const orc_lora* loras, int n_loras, float* out, int nthreads) {
  run_threads(base, base_dtype, rows, cols, scale_mode, scales, loras, n_loras, out, NULL, nthreads);
}

void orc_read_bf16_mt(const void* base, int base_dtype, int64_t rows, int64_t cols,
                      int scale_mode, const float* scales,
                      const orc_lora* loras, int n_loras, uint16_t* out, int nthreads) {
  run_threads(base, base_dtype, rows, cols, scale_mode, scales, loras, n_loras, NULL, out, nthreads);
}

/* Double-precision restatement of the same sum, for Frobenius checks. */
static void rows_f64(const void* base, int base_dtype, int64_t rows, int64_t cols,
                     int scale_mode, const float* scales, const orc_lora* loras,
                     int n_loras, int64_t row0, int64_t nrows, double* out, int absval) {
  dense_lora* d = widen_loras(loras, n_loras, rows, cols);
  float* dec = (float*)malloc((size_t)cols * sizeof(float));
  size_t es = elem_size(base_dtype);
  for (int64_t q = 0; q < nrows; ++q) {
    int64_t o = row0 + q;
    double* w = out + (size_t)q * (size_t)cols;
    orc_decode_to_f32((const uint8_t*)base + (size_t)o * (size_t)cols * es, base_dtype,
                      (size_t)cols, dec);
    double s = 1.0;
    if (is_fp8(base_dtype) && scale_mode == ORC_SCALE_TENSOR) s = scales[0];
    if (is_fp8(base_dtype) && scale_mode == ORC_SCALE_ROW) s = scales[o];
    for (int64_t i = 0; i < cols; ++i) {
      double v = s * (double)dec[i];
      w[i] = absval ? fabs(v) : v;
    }
    for (int l = 0; l < n_loras; ++l) {
      for (int32_t r = 0; r < d[l].rank; ++r) {
        double c = (double)d[l].coeff * (double)d[l].b[(size_t)o * (size_t)d[l].rank + (size_t)r];
        if (absval) c = fabs(c);
        const float* arow = d[l].a + (size_t)r * (size_t)cols;
        for (int64_t i = 0; i < cols; ++i) w[i] += c * (absval ? fabs((double)arow[i]) : (double)arow[i]);
      }
    }
  }
  free(dec);
  free_loras(d, n_loras);
}

void orc_read_f64_rows(const void* base, int base_dtype, int64_t rows, int64_t cols,
                       int scale_mode, const float* scales, const orc_lora* loras,
                       int n_loras, int64_t row0, int64_t nrows, double* out) {
  rows_f64(base, base_dtype, rows, cols, scale_mode, scales, loras, n_loras, row0, nrows, out, 0);
}

void orc_abs_bound_rows(const void* base, int base_dtype, int64_t rows, int64_t cols,
                        int scale_mode, const float* scales, const orc_lora* loras,
                        int n_loras, int64_t row0, int64_t nrows, double* out) {
  rows_f64(base, base_dtype, rows, cols, scale_mode, scales, loras, n_loras, row0, nrows, out, 1);
}
