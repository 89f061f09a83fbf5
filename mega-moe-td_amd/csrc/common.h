// Shared device/host helpers for libmegamoe (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/megamoe.h"

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------- errors
void mm_set_error(const char* fmt, ...);

#define MM_CHECK_ARG(cond, ...)       \
  do {                                \
    if (!(cond)) {                    \
      mm_set_error(__VA_ARGS__);      \
      return MM_E_ARG;                \
    }                                 \
  } while (0)

int mm_check_launch(const char* what);

static inline hipStream_t mm_hip_stream(mm_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

static inline size_t mm_align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// ---------------------------------------------------------------- streaming loads
// 16- / 8-byte loads of data read exactly once (gathered rows of the combine
// and of the gated-activation backward): the non-temporal hint keeps them
// from displacing reused lines in L2 (measured: combine 5.3 -> 5.8 TB/s).
typedef unsigned mm_u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned mm_u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 load_stream16(const void* p) {
  const mm_u32x4 t = __builtin_nontemporal_load(reinterpret_cast<const mm_u32x4*>(p));
  return make_uint4(t.x, t.y, t.z, t.w);
}
__device__ __forceinline__ uint2 load_stream8(const void* p) {
  const mm_u32x2 t = __builtin_nontemporal_load(reinterpret_cast<const mm_u32x2*>(p));
  return make_uint2(t.x, t.y);
}

// ---------------------------------------------------------------- bf16
// Round-to-nearest-even fp32 -> bf16 with gfx950's v_cvt_pk_bf16_f32: equal
// to torch's float->bfloat16 conversion for every non-NaN input (NaN stays a
// quiet NaN).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// Two fp32 -> packed fp16 (v_cvt_pk_f16_f32 / RNE).
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2_t));
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

__device__ __forceinline__ float round_bf16(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }

// ---------------------------------------------------------------- saved FC1 formats
// FP8 E4M3 ("fn": bias 7, no infinities, max 448, NaN = 0x7F/0xFF) with
// round-to-nearest-even and saturation to +-448, the conversion the
// reference's single-kernel save applies (kernels/fused_forward.py:893-942).
constexpr float kFp8Max = 448.0f;

__device__ __forceinline__ uint32_t f32_to_e4m3fn(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7fu;        // NaN
  if (a > 0x43e80000u) return sign | 0x7eu;        // beyond the 448/480 midpoint: saturate
  if (a < 0x3c800000u) {                           // below 2^-6: subnormal steps of 2^-9
    const float m = __builtin_rintf(__uint_as_float(a) * 512.0f);  // RNE, 0..8 (8 = smallest normal)
    return sign | static_cast<uint32_t>(m);
  }
  // normal: round the 23-bit mantissa to 3 bits (RNE, carries into the
  // exponent), then rebias the exponent from 127 to 7
  const uint32_t r = (a + 0x7ffffu + ((a >> 20) & 1u)) >> 20;
  return sign | (r - (120u << 3));
}

__device__ __forceinline__ float e4m3fn_to_f32(uint32_t b) {
  const uint32_t e = (b >> 3) & 0xfu, m = b & 7u;
  float v;
  if (e == 0)
    v = static_cast<float>(m) * (1.0f / 512.0f);
  else if (e == 15 && m == 7)
    v = __uint_as_float(0x7fc00000u);
  else
    v = __uint_as_float(((e + 120u) << 23) | (m << 20));
  return (b & 0x80u) ? -v : v;
}

// ---------------------------------------------------------------- activation
// Gated activation value act(gate) * v(up) in fp32, following the reference's
// _gated_activation (ops/_torch_forward.py:177-205).
// v_exp_f32 and v_rcp_f32 (about 1 ulp each; the results are rounded to
// bf16 afterwards).
__device__ __forceinline__ float mm_sigmoid(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

__device__ __forceinline__ float mm_tanh(float x) {
  // tanh(x) = 2*sigmoid(2x) - 1 (same rewrite the reference kernels use).
  return 2.0f * mm_sigmoid(2.0f * x) - 1.0f;
}

__device__ __forceinline__ float gated_act(int kind, float g, float u, float beta, float lbeta,
                                           float clamp_limit) {
  if (kind == MM_ACT_SWIGLU) {
    return (g * mm_sigmoid(g)) * u;
  } else if (kind == MM_ACT_CLAMP_SWIGLU) {
    float gc = fminf(g, clamp_limit);
    float uc = fminf(fmaxf(u, -clamp_limit), clamp_limit);
    return (gc * mm_sigmoid(gc)) * uc;
  } else {
    float a = beta * mm_tanh(g / beta) * mm_sigmoid(g);
    float v = lbeta > 0.0f ? lbeta * mm_tanh(u / lbeta) : u;
    return a * v;
  }
}
