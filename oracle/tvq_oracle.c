/*
 * tvq_oracle.c — CPU restatement of the reference's quantized-linear
 * arithmetic. TEST INFRASTRUCTURE ONLY: used by tests/, the smoke check and
 * bench.py's cpu_baseline leg as the checker; never linked into, or called
 * by, the product library.
 *
 * Functions and the reference code each restates:
 *   oracle_act_quant       nanovllm/quantization/utils.py:28-32
 *                          (quantize_int8_per_row_dynamic; same formula as
 *                          quantize_int8_per_channel, utils.py:21-25)
 *   oracle_gemm_i32        nanovllm/quantization/csrc/w8a8_gemm.cu:336-375
 *                          (int8 x int8 -> exact int32 accumulator)
 *   oracle_w8a8_epilogue   nanovllm/quantization/csrc/w8a8_gemm.cu:384-390
 *                          y = out((float(acc) * a_s[m]) * w_s[n] + bias[n]),
 *                          bias add fused (nvcc contracts mul+add to fma)
 *   oracle_w8a16_f64       nanovllm/quantization/cuda.py:293-300 with the
 *                          weight scale applied in exact arithmetic:
 *                          y = sum_k x[m,k]*q[n,k] * s[n] + b[n] in double
 *   oracle_quant_code_sweep utils.py:28-32 again: an exhaustive check that
 *                          the product's divide-free code equals rint(x / s)
 *
 * Pinned by: tests/test_oracle.py (closed-form special cases, numpy and
 * torch restatements, brute force on tiny inputs, invariants).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h >> 15) << 31;
  const uint32_t exp = (h >> 10) & 0x1f;
  const uint32_t man = h & 0x3ff;
  float f;
  if (exp == 0) {
    /* zero or subnormal: man * 2^-24 (exact in float) */
    f = ldexpf((float)man, -24);
    if (sign) f = -f;
    return f;
  }
  uint32_t u;
  if (exp == 31)
    u = sign | 0x7f800000u | (man << 13);
  else
    u = sign | ((exp + 112) << 23) | (man << 13);
  memcpy(&f, &u, 4);
  return f;
}

/* Round-to-nearest-even float -> bf16 (c10::BFloat16 semantics). */
static uint16_t f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40); /* quiet NaN */
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static float load16(const uint16_t* p, int64_t i, int is_bf16) {
  return is_bf16 ? bf16_to_f32(p[i]) : f16_to_f32(p[i]);
}

/* Per-row symmetric int8 quantization of a 16-bit [M,K] matrix. */
void oracle_act_quant(const uint16_t* x, int is_bf16, int64_t M, int64_t K, float eps, int8_t* q, float* s) {
  for (int64_t m = 0; m < M; ++m) {
    float amax = 0.0f;
    for (int64_t k = 0; k < K; ++k) {
      const float v = fabsf(load16(x, m * K + k, is_bf16));
      if (v > amax) amax = v;
    }
    float sc = amax / 127.0f;
    if (sc < eps) sc = eps;
    s[m] = sc;
    for (int64_t k = 0; k < K; ++k) {
      float t = rintf(load16(x, m * K + k, is_bf16) / sc);
      if (t > 127.0f) t = 127.0f;
      if (t < -127.0f) t = -127.0f;
      q[m * K + k] = (int8_t)t;
    }
  }
}

/* Same quantizer on an fp32 [M,K] matrix (weights are quantized from fp32). */
void oracle_quant_f32(const float* x, int64_t M, int64_t K, float eps, int8_t* q, float* s) {
  for (int64_t m = 0; m < M; ++m) {
    float amax = 0.0f;
    for (int64_t k = 0; k < K; ++k) {
      const float v = fabsf(x[m * K + k]);
      if (v > amax) amax = v;
    }
    float sc = amax / 127.0f;
    if (sc < eps) sc = eps;
    s[m] = sc;
    for (int64_t k = 0; k < K; ++k) {
      float t = rintf(x[m * K + k] / sc);
      if (t > 127.0f) t = 127.0f;
      if (t < -127.0f) t = -127.0f;
      q[m * K + k] = (int8_t)t;
    }
  }
}

/* acc[m,n] = sum_k xq[m,k] * w[n,k], exact (|acc| <= 127^2 * K < 2^31 for K <= 133144). */
void oracle_gemm_i32(const int8_t* xq, const int8_t* w, int64_t M, int64_t N, int64_t K, int32_t* acc) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      const int8_t* a = xq + m * K;
      const int8_t* b = w + n * K;
      int32_t sum = 0;
      for (int64_t k = 0; k < K; ++k) sum += (int32_t)a[k] * (int32_t)b[k];
      acc[m * N + n] = sum;
    }
  }
}

/* W8A8 epilogue to bf16 (out_bf16=1) or to fp32 values (out_bf16=0, y_f32). */
void oracle_w8a8_epilogue(const int32_t* acc, const float* a_s, const float* w_s, const float* bias_f32,
                          int64_t M, int64_t N, uint16_t* y_bf16, float* y_f32) {
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      const float p = (float)acc[m * N + n] * a_s[m];
      const float b = bias_f32 ? bias_f32[n] : 0.0f;
      const float v = fmaf(p, w_s[n], b);
      if (y_bf16) y_bf16[m * N + n] = f32_to_bf16(v);
      if (y_f32) y_f32[m * N + n] = v;
    }
  }
}

/* W8A16 product in double: y[m,n] = (sum_k x[m,k]*q[n,k]) * s[n] + b[n]. */
void oracle_w8a16_f64(const uint16_t* x, int is_bf16, const int8_t* q, const float* s, const float* bias_f32,
                      int64_t M, int64_t N, int64_t K, double* y) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      double sum = 0.0;
      for (int64_t k = 0; k < K; ++k) sum += (double)load16(x, m * K + k, is_bf16) * (double)q[n * K + k];
      y[m * N + n] = sum * (double)s[n] + (bias_f32 ? (double)bias_f32[n] : 0.0);
    }
  }
}

/* Round-to-nearest-even float -> IEEE half (subnormals, overflow to inf). */
static uint16_t f32_to_f16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7e00u;            /* NaN */
  if (a >= 0x477ff000u) return sign | 0x7c00u;           /* >= 65520 rounds to inf */
  if (a < 0x38800000u) {                                  /* below 2^-14: subnormal half */
    float mag;
    memcpy(&mag, &a, 4);
    return sign | (uint16_t)nearbyintf(mag * 16777216.0f);  /* mag / 2^-24, exact scaling */
  }
  const uint32_t mant = a & 0x7fffffu;
  uint32_t r = ((((a >> 23) - 127u + 15u) << 10) | (mant >> 13));
  const uint32_t rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r += 1u;
  return sign | (uint16_t)r;
}

/* The reference kernel's dequantized weight T(T(q) * T(s)) as T bits
 * (int8_weight_only_gemm.cu:401-411; cuda.py:293-300): T(q) exact, T(s) by
 * RNE, the product exact in float (<= 8 + 11 significant bits), one RNE. */
void oracle_w8a16_rounded_weights(const int8_t* q, const float* s, int is_bf16, int64_t N, int64_t K,
                                  uint16_t* wd) {
  for (int64_t n = 0; n < N; ++n) {
    const float sr = is_bf16 ? bf16_to_f32(f32_to_bf16(s[n])) : f16_to_f32(f32_to_f16(s[n]));
    for (int64_t k = 0; k < K; ++k) {
      const float p = (float)q[n * K + k] * sr;
      wd[n * K + k] = is_bf16 ? f32_to_bf16(p) : f32_to_f16(p);
    }
  }
}

/* float -> half RNE over an array (exposed so the tests can pin it). */
void oracle_f32_to_f16(const float* x, int64_t n, uint16_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = f32_to_f16(x[i]);
}

/* float -> bf16 RNE over an array (exposed so the tests can pin it). */
void oracle_f32_to_bf16(const float* x, int64_t n, uint16_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = f32_to_bf16(x[i]);
}

/* Exhaustive check of the product's divide-free per-token code against the
 * reference's rint(x / s) (utils.py:28-32; IEEE RN divide, ties-to-even).
 * The product (the act-quant and producer kernels) computes, with
 * rs = RN(1 / s),
 *   variant 0:  d = RN(x * rs);  q = fma(fma(-d, s, x), rs, d);  code = rint(q)
 *   variant 1:  code = rint(RN(x * rs))   (the plain form, known to differ)
 * and both are odd in x, so non-negative x covers every input. For every
 * finite non-negative 16-bit (bf16 or fp16) row maximum amax and every finite
 * non-negative 16-bit x <= amax, with s = max(RN(amax / 127), eps), count the
 * pairs whose code differs from clamp(rint(RN(x / s)), -127, 127).
 * Returns the mismatch count; *pairs gets the number of pairs checked. */
int64_t oracle_quant_code_sweep(int is_bf16, float eps, int variant, int64_t* pairs) {
  const uint16_t top = is_bf16 ? 0x7f80u : 0x7c00u; /* first non-finite pattern */
  int64_t bad = 0, n = 0;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : bad, n)
  for (int32_t a = 0; a < (int32_t)top; ++a) {
    const float amax = is_bf16 ? bf16_to_f32((uint16_t)a) : f16_to_f32((uint16_t)a);
    float s = amax / 127.0f;
    if (s < eps) s = eps;
    const float rs = 1.0f / s;
    for (int32_t b = 0; b <= a; ++b) {
      const float x = is_bf16 ? bf16_to_f32((uint16_t)b) : f16_to_f32((uint16_t)b);
      float want = rintf(x / s);
      if (want > 127.0f) want = 127.0f;
      float got;
      if (variant == 0) {
        const float d = x * rs;
        got = rintf(fmaf(fmaf(-d, s, x), rs, d));
      } else {
        got = rintf(x * rs);
      }
      if (got > 127.0f) got = 127.0f;
      bad += (got != want);
      n += 1;
    }
  }
  *pairs = n;
  return bad;
}
