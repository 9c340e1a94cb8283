// Shared device helpers for the gfx950 Bigger Bird kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4_t;
typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2_t;

#define BB_DEV __device__ __forceinline__

namespace bb {

constexpr float kLog2e = 1.44269504088896340736f;

BB_DEV float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// Round-to-nearest-even float -> bf16 bits (NaN kept quiet).
BB_DEV uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;

// Two floats -> packed bf16x2 (RNE, one v_cvt_pk_bf16_f32), low half = a.
BB_DEV uint32_t pack_bf16x2(float a, float b) {
  const bf16x2_t v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}

BB_DEV bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

BB_DEV f32x16_t mfma32(bf16x8_t a, bf16x8_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// The 16-bit element type of a kernel instantiation: bf16, or fp16 when F16. Fragments travel as 16-byte bit
// patterns (bf16x8_t); the MFMA and the float -> 16-bit conversions (round to nearest even) follow the type.
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8_t;
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

template <bool F16>
BB_DEV f32x16_t mma32(bf16x8_t a, bf16x8_t b, f32x16_t c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

template <bool F16>
BB_DEV uint32_t pack2(float a, float b) {
  if constexpr (F16) {
    const f16x2_t v = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, v);
  } else {
    return pack_bf16x2(a, b);
  }
}

template <bool F16>
BB_DEV uint16_t to16(float f) {
  if constexpr (F16) return __builtin_bit_cast(uint16_t, (_Float16)f);
  else return f32_to_bf16(f);
}

// Value of the partner lane l ^ 32 combined with this lane's value.
BB_DEV float xhalf_max(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
BB_DEV float xhalf_sum(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

BB_DEV float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Deterministic exp2 for x <= 0 built only from correctly rounded operations (rint, fma, ldexp), so host and
// device produce identical bits: rint range reduction, degree-7 Taylor polynomial of 2^f on [-0.5, 0.5].
__host__ __device__ __forceinline__ float det_exp2(float x) {
  if (!(x > -100.0f)) return 0.0f;
  float n = rintf(x);
  float f = x - n;
  float p = 1.5252733804059840e-05f;
  p = fmaf(p, f, 1.5403530393381610e-04f);
  p = fmaf(p, f, 1.3333558146428443e-03f);
  p = fmaf(p, f, 9.6181291076284772e-03f);
  p = fmaf(p, f, 5.5504108664821580e-02f);
  p = fmaf(p, f, 2.4022650695910071e-01f);
  p = fmaf(p, f, 6.9314718055994531e-01f);
  p = fmaf(p, f, 1.0f);
  return ldexpf(p, (int)n);
}

// One round-to-nearest-even step from float64 to bf16 bits (no intermediate fp32 rounding).
BB_DEV uint16_t bf16_from_f64(double x) {
  if (x == 0.0 || !__builtin_isfinite(x)) return f32_to_bf16((float)x);
  double ax = fabs(x);
  double quantum;
  if (ax < 0x1p-126) {
    quantum = 0x1p-133;
  } else {
    int e;
    frexp(ax, &e);
    quantum = ldexp(1.0, e - 8);
  }
  double r = rint(x / quantum) * quantum;
  return (uint16_t)(__float_as_uint((float)r) >> 16);
}

// Order-preserving float <-> uint32 map, so that atomicMax on the key is a float max.
BB_DEV uint32_t float_to_ordered(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
BB_DEV float ordered_to_float(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

// 16-byte global load / store helpers (addresses must be 16-byte aligned).
BB_DEV u32x4_t ld16(const void* p) { return *reinterpret_cast<const u32x4_t*>(p); }
BB_DEV void st16(void* p, u32x4_t v) { *reinterpret_cast<u32x4_t*>(p) = v; }

}  // namespace bb
