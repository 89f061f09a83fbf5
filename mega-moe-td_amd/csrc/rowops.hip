#include <stdlib.h>
// Row-wise bandwidth kernels: dispatch gather, top-k combine, routing-weight
// gradient gather, gated-activation backward. All are HBM-bound; each
// wavefront owns one row and moves it with 16-byte vector loads/stores.
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <type_traits>

#include "common.h"

// ---------------------------------------------------------------- errors
static thread_local char g_err[512] = "";

void mm_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int mm_check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    mm_set_error("%s: %s", what, hipGetErrorString(e));
    return MM_E_LAUNCH;
  }
  return MM_OK;
}

extern "C" const char* mm_last_error(void) { return g_err; }
extern "C" int mm_version(void) { return 1; }

namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerBlock = kThreads / 64;
constexpr int kMaxGrid = 8192;

struct alignas(16) Vec8 {
  uint16_t h[8];
};

__device__ __forceinline__ void vec8_to_f32(const uint4& v, float* f) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(w[i] << 16);
    f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ uint4 f32_to_vec8(const float* f) {
  return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                    pack_bf16x2(f[6], f[7]));
}

// out[i] = x[send_token[i]] for i < offsets[E].
__global__ __launch_bounds__(kThreads) void permute_kernel(const uint4* __restrict__ x, int64_t ldx_v,
                                                           const int32_t* __restrict__ send_token,
                                                           const int32_t* __restrict__ offsets, int E,
                                                           int64_t max_rows, int hidden_v,
                                                           uint4* __restrict__ out, int64_t ldo_v) {
  const int nvalid = static_cast<int>(min(static_cast<int64_t>(offsets[E]), max_rows));
  const int lane = threadIdx.x & 63;
  for (int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6); row < nvalid;
       row += gridDim.x * kRowsPerBlock) {
    const uint4* src = x + static_cast<int64_t>(send_token[row]) * ldx_v;
    uint4* dst = out + static_cast<int64_t>(row) * ldo_v;
    for (int v = lane; v < hidden_v; v += 64) dst[v] = src[v];
  }
}

// out[t] = bf16(sum_j fp32(y[route_to_send[t*k+j]])), slot order j = 0..k-1.
// Work is split into equal items: item i = (token i / nchunks, chunk
// i % nchunks of 64 * VPL vectors), one wavefront per item, so every item
// moves the same bytes (against up to 4 wavefronts per token interleaving
// 2 KiB passes, whose last pass per token was short: Kimi shape 181 -> 176
// us, Skew 213 -> 204 us). Each lane issues the loads of SLOTS slots for its
// VPL vectors before accumulating (SLOTS * VPL row reads in flight per lane;
// one round trip per 8 slots). Rows are read once: non-temporal loads.
template <int VPL, int SLOTS>
__global__ __launch_bounds__(kThreads) void combine_items_kernel(const uint4* __restrict__ y, int64_t ldy_v,
                                                                 const int32_t* __restrict__ route_to_send,
                                                                 int64_t T, int top_k, int hidden_v,
                                                                 uint4* __restrict__ out, int64_t ldo_v,
                                                                 int nchunks, const uint16_t* __restrict__ dscale,
                                                                 float* __restrict__ grad_rw) {
  const int lane = threadIdx.x & 63;
  const int64_t items = T * nchunks;
  for (int64_t w = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6); w < items;
       w += static_cast<int64_t>(gridDim.x) * kRowsPerBlock) {
    const int64_t t = w / nchunks;
    const int chunk = static_cast<int>(w % nchunks);
    const int v0 = chunk * 64 * VPL + lane;
    const int my_row = lane < top_k ? route_to_send[t * top_k + lane] : -1;
    // backward: the token's chunk-0 wavefront also gathers the routing-weight
    // gradient of its k slots (0 for dropped routes)
    if (grad_rw && chunk == 0 && lane < top_k)
      grad_rw[t * top_k + lane] = my_row >= 0 ? bf16_bits_to_f32(dscale[my_row]) : 0.0f;
    float acc[VPL][8];
#pragma unroll
    for (int u = 0; u < VPL; ++u)
#pragma unroll
      for (int q = 0; q < 8; ++q) acc[u][q] = 0.0f;
    for (int j0 = 0; j0 < top_k; j0 += SLOTS) {
      uint4 val[SLOTS][VPL];
      int rr[SLOTS];
#pragma unroll
      for (int jj = 0; jj < SLOTS; ++jj) {
        const int j = j0 + jj;
        rr[jj] = __shfl(my_row, j < top_k ? j : 0);
        if (j >= top_k) rr[jj] = -1;
#pragma unroll
        for (int u = 0; u < VPL; ++u) {
          const int v = v0 + u * 64;
          val[jj][u] = (rr[jj] >= 0 && v < hidden_v) ? load_stream16(y + static_cast<int64_t>(rr[jj]) * ldy_v + v)
                                                      : make_uint4(0, 0, 0, 0);
        }
      }
#pragma unroll
      for (int jj = 0; jj < SLOTS; ++jj) {
        if (rr[jj] < 0) continue;
#pragma unroll
        for (int u = 0; u < VPL; ++u) {
          float f[8];
          vec8_to_f32(val[jj][u], f);
#pragma unroll
          for (int q = 0; q < 8; ++q) acc[u][q] += f[q];
        }
      }
    }
    uint4* dst = out + t * ldo_v;
#pragma unroll
    for (int u = 0; u < VPL; ++u)
      if (v0 + u * 64 < hidden_v) dst[v0 + u * 64] = f32_to_vec8(acc[u]);
  }
}

__global__ __launch_bounds__(kThreads) void gather_route_grad_kernel(const uint16_t* __restrict__ dscale,
                                                                     const int32_t* __restrict__ r2s,
                                                                     int64_t R, float* __restrict__ g) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < R;
       i += static_cast<int64_t>(gridDim.x) * kThreads) {
    const int r = r2s[i];
    g[i] = r >= 0 ? bf16_bits_to_f32(dscale[r]) : 0.0f;
  }
}

// Gated activation derivative pair (value, d/dgate, v(up), d/dup), as in
// kernels/swiglu_bwd.py:52-83 of the reference.
__device__ __forceinline__ void act_pair(int kind, float a, float b, float beta, float lbeta, float L,
                                         float& act_a, float& dact_a, float& v, float& dv) {
  if (kind == MM_ACT_SWIGLU) {
    const float s = mm_sigmoid(a);
    act_a = a * s;
    dact_a = act_a * (1.0f - s) + s;
    v = b;
    dv = 1.0f;
  } else if (kind == MM_ACT_CLAMP_SWIGLU) {
    const float gc = fminf(a, L);
    const float uc = fminf(fmaxf(b, -L), L);
    const float s = mm_sigmoid(gc);
    act_a = gc * s;
    dact_a = (s + gc * s * (1.0f - s)) * (a <= L ? 1.0f : 0.0f);
    v = uc;
    dv = fabsf(b) <= L ? 1.0f : 0.0f;
  } else {
    const float t = mm_tanh(a / beta);
    const float s = mm_sigmoid(a);
    act_a = beta * t * s;
    dact_a = (1.0f - t * t) * s + beta * t * s * (1.0f - s);
    if (lbeta > 0.0f) {
      const float tu = mm_tanh(b / lbeta);
      v = lbeta * tu;
      dv = 1.0f - tu * tu;
    } else {
      v = b;
      dv = 1.0f;
    }
  }
}

// 8 consecutive saved FC1 values (bf16 / fp16 / fp8 e4m3) of one row -> fp32;
// v indexes 8-value vectors of the row, fp8 values are scaled by `sc`.
template <int FMT>
struct Fc1Row {
  static constexpr int BYTES = FMT == MM_FC1_FP8 ? 8 : 16;  // bytes per 8 values
  typedef typename std::conditional<FMT == MM_FC1_FP8, uint2, uint4>::type Vec;
  __device__ static Vec load(const uint8_t* row, int v) { return reinterpret_cast<const Vec*>(row)[v]; }
  __device__ static Vec load_stream(const uint8_t* row, int v) {
    if constexpr (FMT == MM_FC1_FP8)
      return load_stream8(row + static_cast<int64_t>(v) * BYTES);
    else
      return load_stream16(row + static_cast<int64_t>(v) * BYTES);
  }
  __device__ static Vec zero() {
    if constexpr (FMT == MM_FC1_FP8) return make_uint2(0, 0);
    else return make_uint4(0, 0, 0, 0);
  }
  __device__ static void to_f32(const Vec& x, float sc, float* f) {
    if constexpr (FMT == MM_FC1_BF16) {
      vec8_to_f32(x, f);
    } else if constexpr (FMT == MM_FC1_FP16) {
      typedef _Float16 h2 __attribute__((ext_vector_type(2)));
      const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const h2 h = __builtin_bit_cast(h2, w[i]);
        f[2 * i] = static_cast<float>(h[0]);
        f[2 * i + 1] = static_cast<float>(h[1]);
      }
    } else {
      const uint32_t w[2] = {x.x, x.y};
#pragma unroll
      for (int i = 0; i < 8; ++i) f[i] = e4m3fn_to_f32((w[i >> 2] >> ((i & 3) * 8)) & 0xffu) * sc;
    }
  }
};

template <int KIND, int FMT>
__global__ __launch_bounds__(kThreads) void swiglu_bwd_kernel(
    const uint4* __restrict__ ga, int64_t ld_ga_v, const uint8_t* __restrict__ fc1, int64_t ld_fc1,
    const float* __restrict__ fc1_scale, const float* __restrict__ scale, const int32_t* __restrict__ offsets,
    int E, int inter_v, float beta, float lbeta, float L, uint4* __restrict__ dab, uint16_t* __restrict__ dscale) {
  using F = Fc1Row<FMT>;
  constexpr int kind = KIND;
  const int nvalid = offsets[E];
  const int lane = threadIdx.x & 63;
  const int groups = inter_v * 8 / MM_FC1_SCALE_GROUP;  // FP8 scale groups per half row
  for (int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6); row < nvalid;
       row += gridDim.x * kRowsPerBlock) {
    const float s = round_bf16(scale[row]);
    const uint4* g_row = ga + static_cast<int64_t>(row) * ld_ga_v;
    const uint8_t* a_row = fc1 + static_cast<int64_t>(row) * ld_fc1 * (FMT == MM_FC1_FP8 ? 1 : 2);
    const uint8_t* b_row = a_row + static_cast<int64_t>(inter_v) * F::BYTES;
    const float* sc_row = FMT == MM_FC1_FP8 ? fc1_scale + static_cast<int64_t>(row) * 2 * groups : nullptr;
    uint4* d_row = dab + static_cast<int64_t>(row) * 2 * inter_v;
    float part = 0.0f;
    // two 8-value vectors per lane per pass: all six loads issue before the math
    for (int v0 = lane; v0 < inter_v; v0 += 128) {
      uint4 gv[2];
      typename F::Vec av[2], bv[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int v = v0 + 64 * u;
        const bool in = v < inter_v;
        gv[u] = in ? load_stream16(g_row + v) : make_uint4(0, 0, 0, 0);
        av[u] = in ? F::load_stream(a_row, v) : F::zero();
        bv[u] = in ? F::load_stream(b_row, v) : F::zero();
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int v = v0 + 64 * u;
        if (v >= inter_v) break;
        float sa = 1.0f, sb = 1.0f;
        if constexpr (FMT == MM_FC1_FP8) {
          const int grp = v * 8 / MM_FC1_SCALE_GROUP;
          sa = sc_row[grp];
          sb = sc_row[groups + grp];
        }
        float dc[8], a[8], b[8], da[8], db[8];
        vec8_to_f32(gv[u], dc);
        F::to_f32(av[u], sa, a);
        F::to_f32(bv[u], sb, b);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          float act_a, dact_a, vv, dv;
          act_pair(kind, a[q], b[q], beta, lbeta, L, act_a, dact_a, vv, dv);
          da[q] = dc[q] * dact_a * vv * s;
          db[q] = dc[q] * act_a * dv * s;
          part += act_a * vv * dc[q];
        }
        d_row[v] = f32_to_vec8(da);
        d_row[inter_v + v] = f32_to_vec8(db);
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) part += __shfl_xor(part, off);
    if (lane == 0) dscale[row] = f32_to_bf16_bits(part);
  }
}

// act[i] = bf16(act_fn(gate, up) * w[i]) from a saved FC1 row (any format):
// the FC1 epilogue's formula, bit-identical to the forward's act for a bf16
// save with the same fp32 weight.
template <int KIND, int FMT>
__global__ __launch_bounds__(kThreads) void gated_act_kernel(
    const uint8_t* __restrict__ fc1, int64_t ld_fc1, const float* __restrict__ fc1_scale,
    const float* __restrict__ w, const int32_t* __restrict__ offsets, int E, int inter_v, float beta, float lbeta,
    float L, uint4* __restrict__ act, int64_t ld_act_v) {
  using F = Fc1Row<FMT>;
  const int nvalid = offsets[E];
  const int lane = threadIdx.x & 63;
  const int groups = inter_v * 8 / MM_FC1_SCALE_GROUP;
  for (int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6); row < nvalid;
       row += gridDim.x * kRowsPerBlock) {
    const float wr = w[row];
    const uint8_t* a_row = fc1 + static_cast<int64_t>(row) * ld_fc1 * (FMT == MM_FC1_FP8 ? 1 : 2);
    const uint8_t* b_row = a_row + static_cast<int64_t>(inter_v) * F::BYTES;
    const float* sc_row = FMT == MM_FC1_FP8 ? fc1_scale + static_cast<int64_t>(row) * 2 * groups : nullptr;
    uint4* o_row = act + static_cast<int64_t>(row) * ld_act_v;
    for (int v = lane; v < inter_v; v += 64) {
      float sa = 1.0f, sb = 1.0f;
      if constexpr (FMT == MM_FC1_FP8) {
        const int grp = v * 8 / MM_FC1_SCALE_GROUP;
        sa = sc_row[grp];
        sb = sc_row[groups + grp];
      }
      float a[8], b[8], o[8];
      F::to_f32(F::load(a_row, v), sa, a);
      F::to_f32(F::load(b_row, v), sb, b);
#pragma unroll
      for (int q = 0; q < 8; ++q) o[q] = gated_act(KIND, a[q], b[q], beta, lbeta, L) * wr;
      o_row[v] = f32_to_vec8(o);
    }
  }
}

int grid_for_rows(int64_t rows) {
  int64_t g = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
  if (g < 1) g = 1;
  if (g > kMaxGrid) g = kMaxGrid;
  return static_cast<int>(g);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" int mm_permute(const uint16_t* x, int64_t ldx, const int32_t* send_token, const int32_t* offsets,
                          int32_t num_experts, int64_t max_rows, int32_t hidden, uint16_t* out, int64_t ldo,
                          mm_stream_t stream) {
  MM_CHECK_ARG(x && send_token && offsets && out, "mm_permute: null pointer");
  MM_CHECK_ARG(num_experts > 0 && hidden > 0 && max_rows >= 0, "mm_permute: bad sizes");
  MM_CHECK_ARG(hidden % 8 == 0 && ldx % 8 == 0 && ldo % 8 == 0 && aligned16(x) && aligned16(out),
               "mm_permute: rows must be 16-byte aligned (hidden, strides multiple of 8)");
  if (max_rows == 0) return MM_OK;
  permute_kernel<<<grid_for_rows(max_rows), kThreads, 0, mm_hip_stream(stream)>>>(
      reinterpret_cast<const uint4*>(x), ldx / 8, send_token, offsets, num_experts, max_rows, hidden / 8,
      reinterpret_cast<uint4*>(out), ldo / 8);
  return mm_check_launch("mm_permute");
}

namespace {

int launch_combine(const uint16_t* y, int64_t ldy, const int32_t* route_to_send, int64_t num_tokens,
                   int32_t top_k, int32_t hidden, uint16_t* out, int64_t ldo, const uint16_t* dscale,
                   float* grad_rw, mm_stream_t stream, const char* what) {
  MM_CHECK_ARG(num_tokens >= 0 && hidden > 0, "%s: bad sizes", what);
  MM_CHECK_ARG(top_k > 0 && top_k <= 64, "%s: top_k must be in [1, 64]", what);
  if (num_tokens == 0) return MM_OK;
  MM_CHECK_ARG(y && route_to_send && out, "%s: null pointer", what);
  MM_CHECK_ARG(hidden % 8 == 0 && ldy % 8 == 0 && ldo % 8 == 0 && aligned16(y) && aligned16(out),
               "%s: rows must be 16-byte aligned", what);
  const int nchunks = (hidden / 8 + 127) / 128;
  int64_t g = (num_tokens * nchunks + kRowsPerBlock - 1) / kRowsPerBlock;
  if (g > 65536) g = 65536;
  combine_items_kernel<2, 8><<<static_cast<int>(g), kThreads, 0, mm_hip_stream(stream)>>>(
      reinterpret_cast<const uint4*>(y), ldy / 8, route_to_send, num_tokens, top_k, hidden / 8,
      reinterpret_cast<uint4*>(out), ldo / 8, nchunks, dscale, grad_rw);
  return mm_check_launch(what);
}

}  // namespace

extern "C" int mm_combine(const uint16_t* y, int64_t ldy, const int32_t* route_to_send, int64_t num_tokens,
                          int32_t top_k, int32_t hidden, uint16_t* out, int64_t ldo, mm_stream_t stream) {
  return launch_combine(y, ldy, route_to_send, num_tokens, top_k, hidden, out, ldo, nullptr, nullptr, stream,
                        "mm_combine");
}

extern "C" int mm_combine_bwd(const uint16_t* dx, int64_t ldx, const int32_t* route_to_send, int64_t num_tokens,
                              int32_t top_k, int32_t hidden, uint16_t* grad_hidden, int64_t ldo,
                              const uint16_t* dscale, float* grad_rw, mm_stream_t stream) {
  MM_CHECK_ARG(num_tokens == 0 || (dscale && grad_rw), "mm_combine_bwd: null pointer");
  return launch_combine(dx, ldx, route_to_send, num_tokens, top_k, hidden, grad_hidden, ldo, dscale, grad_rw,
                        stream, "mm_combine_bwd");
}

extern "C" int mm_gather_route_grad(const uint16_t* dscale, const int32_t* route_to_send, int64_t num_routes,
                                    float* grad_rw, mm_stream_t stream) {
  MM_CHECK_ARG(num_routes >= 0, "mm_gather_route_grad: bad size");
  if (num_routes == 0) return MM_OK;
  MM_CHECK_ARG(dscale && route_to_send && grad_rw, "mm_gather_route_grad: null pointer");
  int64_t g = (num_routes + kThreads - 1) / kThreads;
  if (g > kMaxGrid) g = kMaxGrid;
  gather_route_grad_kernel<<<static_cast<int>(g), kThreads, 0, mm_hip_stream(stream)>>>(dscale, route_to_send,
                                                                                        num_routes, grad_rw);
  return mm_check_launch("mm_gather_route_grad");
}

extern "C" int mm_swiglu_bwd(const uint16_t* grad_act, int64_t ld_ga, const void* fc1_out, int64_t ld_fc1,
                             int32_t fc1_format, const float* fc1_scale, const float* scale,
                             const int32_t* offsets, int32_t num_experts, int64_t max_rows, int32_t inter,
                             int32_t act_kind, float situ_beta, float situ_linear_beta, float clamp_limit,
                             uint16_t* dab, uint16_t* dscale, mm_stream_t stream) {
  MM_CHECK_ARG(grad_act && fc1_out && scale && offsets && dab && dscale, "mm_swiglu_bwd: null pointer");
  MM_CHECK_ARG(num_experts > 0 && inter > 0 && max_rows >= 0, "mm_swiglu_bwd: bad sizes");
  MM_CHECK_ARG(fc1_format >= MM_FC1_BF16 && fc1_format <= MM_FC1_FP8, "mm_swiglu_bwd: bad fc1_format");
  MM_CHECK_ARG(fc1_format != MM_FC1_FP8 || (fc1_scale && inter % MM_FC1_SCALE_GROUP == 0),
               "mm_swiglu_bwd: FP8 fc1_out needs fc1_scale and inter %% %d == 0", MM_FC1_SCALE_GROUP);
  MM_CHECK_ARG(inter % 8 == 0 && ld_ga % 8 == 0 && ld_fc1 % 16 == 0 && ld_fc1 >= 2 * inter && ld_ga >= inter,
               "mm_swiglu_bwd: rows must be 16-byte aligned");
  MM_CHECK_ARG(aligned16(grad_act) && aligned16(fc1_out) && aligned16(dab), "mm_swiglu_bwd: misaligned");
  MM_CHECK_ARG(act_kind >= 0 && act_kind <= 2, "mm_swiglu_bwd: bad act_kind");
  if (max_rows == 0) return MM_OK;
  auto launch = [&](auto kernel) {
    kernel<<<grid_for_rows(max_rows), kThreads, 0, mm_hip_stream(stream)>>>(
        reinterpret_cast<const uint4*>(grad_act), ld_ga / 8, static_cast<const uint8_t*>(fc1_out), ld_fc1,
        fc1_scale, scale, offsets, num_experts, inter / 8, situ_beta, situ_linear_beta, clamp_limit,
        reinterpret_cast<uint4*>(dab), dscale);
  };
  auto by_format = [&](auto kind_tag) {
    constexpr int K = decltype(kind_tag)::value;
    if (fc1_format == MM_FC1_BF16)
      launch(swiglu_bwd_kernel<K, MM_FC1_BF16>);
    else if (fc1_format == MM_FC1_FP16)
      launch(swiglu_bwd_kernel<K, MM_FC1_FP16>);
    else
      launch(swiglu_bwd_kernel<K, MM_FC1_FP8>);
  };
  if (act_kind == MM_ACT_SWIGLU)
    by_format(std::integral_constant<int, MM_ACT_SWIGLU>());
  else if (act_kind == MM_ACT_CLAMP_SWIGLU)
    by_format(std::integral_constant<int, MM_ACT_CLAMP_SWIGLU>());
  else
    by_format(std::integral_constant<int, MM_ACT_SITUGLU>());
  return mm_check_launch("mm_swiglu_bwd");
}

extern "C" int mm_gated_act(const void* fc1_out, int64_t ld_fc1, int32_t fc1_format, const float* fc1_scale,
                            const float* weight_perm, const int32_t* offsets, int32_t num_experts, int64_t max_rows,
                            int32_t inter, int32_t act_kind, float situ_beta, float situ_linear_beta,
                            float clamp_limit, uint16_t* act, int64_t ld_act, mm_stream_t stream) {
  MM_CHECK_ARG(fc1_out && weight_perm && offsets && act, "mm_gated_act: null pointer");
  MM_CHECK_ARG(num_experts > 0 && inter > 0 && max_rows >= 0, "mm_gated_act: bad sizes");
  MM_CHECK_ARG(fc1_format >= MM_FC1_BF16 && fc1_format <= MM_FC1_FP8, "mm_gated_act: bad fc1_format");
  MM_CHECK_ARG(fc1_format != MM_FC1_FP8 || (fc1_scale && inter % MM_FC1_SCALE_GROUP == 0),
               "mm_gated_act: FP8 fc1_out needs fc1_scale and inter %% %d == 0", MM_FC1_SCALE_GROUP);
  MM_CHECK_ARG(inter % 8 == 0 && ld_fc1 % 16 == 0 && ld_fc1 >= 2 * inter && ld_act % 8 == 0 && ld_act >= inter,
               "mm_gated_act: rows must be 16-byte aligned");
  MM_CHECK_ARG(aligned16(fc1_out) && aligned16(act), "mm_gated_act: misaligned");
  MM_CHECK_ARG(act_kind >= 0 && act_kind <= 2, "mm_gated_act: bad act_kind");
  if (max_rows == 0) return MM_OK;
  auto launch = [&](auto kernel) {
    kernel<<<grid_for_rows(max_rows), kThreads, 0, mm_hip_stream(stream)>>>(
        static_cast<const uint8_t*>(fc1_out), ld_fc1, fc1_scale, weight_perm, offsets, num_experts, inter / 8,
        situ_beta, situ_linear_beta, clamp_limit, reinterpret_cast<uint4*>(act), ld_act / 8);
  };
  auto by_format = [&](auto kind_tag) {
    constexpr int K = decltype(kind_tag)::value;
    if (fc1_format == MM_FC1_BF16)
      launch(gated_act_kernel<K, MM_FC1_BF16>);
    else if (fc1_format == MM_FC1_FP16)
      launch(gated_act_kernel<K, MM_FC1_FP16>);
    else
      launch(gated_act_kernel<K, MM_FC1_FP8>);
  };
  if (act_kind == MM_ACT_SWIGLU)
    by_format(std::integral_constant<int, MM_ACT_SWIGLU>());
  else if (act_kind == MM_ACT_CLAMP_SWIGLU)
    by_format(std::integral_constant<int, MM_ACT_CLAMP_SWIGLU>());
  else
    by_format(std::integral_constant<int, MM_ACT_SITUGLU>());
  return mm_check_launch("mm_gated_act");
}
