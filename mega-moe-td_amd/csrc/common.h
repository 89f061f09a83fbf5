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

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

__device__ __forceinline__ float round_bf16(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }

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
