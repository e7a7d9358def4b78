// Shared device helpers for the gfx950 quantized-linear kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tvq {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;

// Element-type tags. Activations / outputs are stored as raw 16-bit words.
struct BF16 {
  static constexpr bool kIsBF16 = true;
};
struct F16 {
  static constexpr bool kIsBF16 = false;
};

template <typename T>
__device__ __forceinline__ float to_float(uint16_t h);
template <>
__device__ __forceinline__ float to_float<BF16>(uint16_t h) {
  return __builtin_bit_cast(float, (uint32_t)h << 16);
}
template <>
__device__ __forceinline__ float to_float<F16>(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

// Round-to-nearest-even float -> 16-bit (matches c10::BFloat16 / c10::Half).
template <typename T>
__device__ __forceinline__ uint16_t from_float(float f);
template <>
__device__ __forceinline__ uint16_t from_float<BF16>(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}
template <>
__device__ __forceinline__ uint16_t from_float<F16>(float f) {
  // Pin the fp32 value first: otherwise the compiler may fuse the producing
  // multiply into a mixed-precision fma (v_fma_mix*) that rounds once,
  // straight to fp16, instead of rounding to fp32 and then to fp16 as the
  // reference does (static_cast<at::Half>(float)).
  asm("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// Four signed int8 packed in a dword -> four 16-bit floats (bf16 or fp16),
// packed two per dword. |q| <= 128 is exact in both formats. For bf16 the
// fp32 value has a zero low half, so taking the high half is exact; the
// int->float conversion compiles to one SDWA v_cvt_f32_i32 per byte.
template <typename T>
__device__ __forceinline__ u32x2 i8x4_to_16x4(uint32_t w);
template <>
__device__ __forceinline__ u32x2 i8x4_to_16x4<BF16>(uint32_t w) {
  const float f0 = (float)(int8_t)(w);
  const float f1 = (float)(int8_t)(w >> 8);
  const float f2 = (float)(int8_t)(w >> 16);
  const float f3 = (float)((int32_t)w >> 24);
  u32x2 r;
  // byte selector 0x07060302: high half of src0 (bytes 6,7) over high half of
  // src1 (bytes 2,3) -> {lo = bf16(f0), hi = bf16(f1)}.
  r.x = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, f1), __builtin_bit_cast(uint32_t, f0), 0x07060302u);
  r.y = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, f3), __builtin_bit_cast(uint32_t, f2), 0x07060302u);
  return r;
}
template <>
__device__ __forceinline__ u32x2 i8x4_to_16x4<F16>(uint32_t w) {
  const _Float16 h0 = (_Float16)(int8_t)(w);
  const _Float16 h1 = (_Float16)(int8_t)(w >> 8);
  const _Float16 h2 = (_Float16)(int8_t)(w >> 16);
  const _Float16 h3 = (_Float16)((int32_t)w >> 24);
  u32x2 r;
  r.x = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
  r.y = (uint32_t)__builtin_bit_cast(uint16_t, h2) | ((uint32_t)__builtin_bit_cast(uint16_t, h3) << 16);
  return r;
}

// Four signed int8 weights of one output channel, each multiplied by that
// channel's scale already rounded to T (sr), rounded once more to T: the
// element-wise T(T(q) * T(s)) of the reference's dequantization
// (int8_weight_only_gemm.cu:401-411; cuda.py:293-300). T(q) * T(s) has at most
// 8 + 11 significant bits, so the fp32 product is exact and the one RN
// conversion equals the reference's rounded multiply.
template <typename T>
__device__ __forceinline__ u32x2 i8x4_dq_to_16x4(uint32_t w, float sr) {
  const float f0 = (float)(int8_t)(w) * sr;
  const float f1 = (float)(int8_t)(w >> 8) * sr;
  const float f2 = (float)(int8_t)(w >> 16) * sr;
  const float f3 = (float)((int32_t)w >> 24) * sr;
  u32x2 r;
  r.x = (uint32_t)from_float<T>(f0) | ((uint32_t)from_float<T>(f1) << 16);
  r.y = (uint32_t)from_float<T>(f2) | ((uint32_t)from_float<T>(f3) << 16);
  return r;
}

// The channel scale rounded to the activation type, as a float.
template <typename T>
__device__ __forceinline__ float round_to(float s) {
  return to_float<T>(from_float<T>(s));
}

// One 16x16x32 MFMA on 16-bit operands held as four dwords (eight elements).
template <typename T>
__device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c);
template <>
__device__ __forceinline__ f32x4 mfma16x16x32<BF16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mfma16x16x32<F16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// One 32x32x16 MFMA on 16-bit operands (eight elements per lane).
template <typename T>
__device__ __forceinline__ f32x16 mfma32x32x16(u32x4 a, u32x4 b, f32x16 c);
template <>
__device__ __forceinline__ f32x16 mfma32x32x16<BF16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x16 mfma32x32x16<F16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// One 32x32x32 int8 MFMA with exact int32 accumulation.
__device__ __forceinline__ i32x16 mfma32x32x32_i8(u32x4 a, u32x4 b, i32x16 c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, a), __builtin_bit_cast(i32x4, b), c, 0, 0, 0);
}

// One 16x16x64 int8 MFMA with exact int32 accumulation.
__device__ __forceinline__ i32x4 mfma16x16x64_i8(u32x4 a, u32x4 b, i32x4 c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, a), __builtin_bit_cast(i32x4, b), c, 0, 0, 0);
}

__device__ __forceinline__ u32x4 ldg128(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

// Streaming (read-once) 128-bit load: non-temporal, for data each kernel
// reads exactly once (GEMV weights, producer and act-quant inputs), so it
// does not evict what other workgroups re-read.
__device__ __forceinline__ u32x4 ldg128_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// Kernel epilogues. Both apply the per-output-channel fp32 scale once per
// output element, after the dot product.
//   W8A16: y = acc * s[n] + bias[n]
//   W8A8 : y = (float(acc) * a_s[m]) * w_s[n] + bias[n]   (w8a8_gemm.cu:387-390
//          order; the bias add is fused as one fma, as nvcc contracts it)
__device__ __forceinline__ float epi_w8a16(float acc, float s, float b) { return __builtin_fmaf(acc, s, b); }
__device__ __forceinline__ float epi_w8a8(int32_t acc, float as, float ws, float b) {
  return __builtin_fmaf((float)acc * as, ws, b);
}
// The same with no bias tensor: b = +0 (an fma with +0, not a plain
// multiply, so that a -0 product still rounds to +0 exactly as above).
__device__ __forceinline__ float epi_w8a8_nb(int32_t acc, float as, float ws) {
  return __builtin_fmaf((float)acc * as, ws, 0.0f);
}
__device__ __forceinline__ float epi_w8a16_nb(float acc, float s) { return __builtin_fmaf(acc, s, 0.0f); }

// Per-token int8 code of x for scale s, bit-identical to
// clamp(rint(x / s), -127, 127) with an IEEE round-to-nearest divide
// (quantize_int8_per_row_dynamic, reference utils.py:28-32), given
// rs = RN(1/s), without a divide and without a branch:
//   d = RN(x * rs)            within about one ulp of x / s
//   r = fma(-d, s, x)         the remainder x - d*s, exact in fp32
//   q = fma(r, rs, d)         one correction step (Markstein)
// rint(q) equals rint(RN(x / s)) for every finite bf16 and fp16 pair x <= amax
// with s = max(RN(amax / 127), eps) (the code is odd in x): 5.3e8 bf16 and
// 5.0e8 fp16 pairs checked exhaustively on the CPU with a correctly rounded
// fmaf (oracle_quant_code_sweep, run by tests/test_oracle.py), with no
// mismatch, where rint(d) alone mismatches 3544 / 8365 times. |x / s| <= 127
// (1 + 2^-23) by the choice of s, so the clamp only guards non-finite rows.
__device__ __forceinline__ float quant_code(float x, float s, float rs) {
  const float d = x * rs;
  const float q = __builtin_fmaf(__builtin_fmaf(-d, s, x), rs, d);
  return fminf(fmaxf(rintf(q), -127.0f), 127.0f);
}

// Eight 16-bit inputs (a 16-byte vector) -> eight packed int8 codes.
template <typename T>
__device__ __forceinline__ u32x2 quant_codes8(const u32x4& v, float s, float rs) {
  uint32_t c[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t w = v[i >> 1];
    const float x = to_float<T>((uint16_t)((i & 1) ? (w >> 16) : (w & 0xffffu)));
    c[i] = (uint32_t)(int32_t)quant_code(x, s, rs) & 0xffu;
  }
  return u32x2{c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24), c[4] | (c[5] << 8) | (c[6] << 16) | (c[7] << 24)};
}

// SiLU(a) = a / (1 + exp(-a)) = a * rcp(1 + 2^(-a log2 e)), on the hardware
// exp2 and reciprocal (about 1 ulp each in fp32; the bf16/fp16 result is
// then rounded once, as the reference's fused elementwise kernel rounds).
__device__ __forceinline__ float silu_f(float a) {
  return a * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(a * -1.4426950408889634f));
}

}  // namespace tvq
