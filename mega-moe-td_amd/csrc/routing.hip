// Stable expert-major routing on the device.
//
// Reference algorithm: runtime/routing.py:621-768 keeps routes whose expert
// id lies in [0, E), stable-argsorts them by expert id, and derives per-expert
// counts and exclusive offsets; kernels/fused_forward.py:158-480 builds the
// same order without a sort (private per-core histograms, an expert-major /
// core-minor prefix, then an order-preserving scatter) and
// kernels/fc2_combine.py:508-529 inverts it (route_to_send, -1 for drops).
//
// MI355X design: three small launches, no global atomics, no host sync.
// Up to 1024 experts the scatter runs four wavefronts per unit; above that
// (up to 32768, bounded by LDS) one wavefront per unit, whose ballot match
// masks alone give the stable rank (the reference's lower-bound path for
// large bin counts, runtime/routing.py:246-416, serves the same range).
//   1. route_count   one workgroup per chunk of ROUTE_CHUNK consecutive routes
//                    builds an LDS histogram -> unit_counts[unit][expert].
//   2. route_scan    one workgroup turns unit_counts into absolute start rows
//                    (expert-major, unit-minor), counts[] and offsets[E+1].
//   3. route_scatter each workgroup replays its chunk 256 routes at a time; a
//                    route's rank among equal experts inside a wavefront comes
//                    from ballot "match" masks, across the four wavefronts from
//                    tagged LDS counters, so the scatter is stable without a
//                    sort and writes every table exactly once.
#include <mutex>

#include "common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kIters = 8;                       // 256-route steps per unit
constexpr int kChunk = kThreads * kIters;       // routes per unit
constexpr int kMaxExperts4 = 1024;              // LDS bound of the 4-wave route_scatter (36 KiB)
constexpr int kMaxExperts = 32768;              // LDS bound of the 1-wave scatter (128 KiB) and the scan

__device__ __forceinline__ bool route_valid(int e, int E) { return e >= 0 && e < E; }

__global__ __launch_bounds__(kThreads) void route_count_kernel(const int32_t* __restrict__ sel,
                                                               int64_t R, int E, int nunits,
                                                               int32_t* __restrict__ unit_counts) {
  extern __shared__ int hist[];
  const int u = blockIdx.x;
  for (int e = threadIdx.x; e < E; e += kThreads) hist[e] = 0;
  __syncthreads();
  const int64_t start = static_cast<int64_t>(u) * kChunk;
  const int64_t end = min(R, start + kChunk);
  for (int64_t i = start + threadIdx.x; i < end; i += kThreads) {
    int e = sel[i];
    if (route_valid(e, E)) atomicAdd(&hist[e], 1);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += kThreads) unit_counts[static_cast<int64_t>(u) * E + e] = hist[e];
}

// Single workgroup: per-expert prefix over units, then an exclusive scan over
// experts. unit_counts[u][e] becomes the absolute first row of (u, e).
__global__ __launch_bounds__(1024) void route_scan_kernel(int32_t* __restrict__ unit_counts, int E,
                                                          int nunits, int32_t* __restrict__ counts,
                                                          int32_t* __restrict__ offsets) {
  extern __shared__ int tot[];  // E + 1024 scratch
  int* part = tot + E;
  const int tid = threadIdx.x;
  for (int e = tid; e < E; e += 1024) {
    int run = 0;
    int u = 0;
    for (; u + 8 <= nunits; u += 8) {
      int c[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) c[j] = unit_counts[static_cast<int64_t>(u + j) * E + e];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        unit_counts[static_cast<int64_t>(u + j) * E + e] = run;
        run += c[j];
      }
    }
    for (; u < nunits; ++u) {
      int c = unit_counts[static_cast<int64_t>(u) * E + e];
      unit_counts[static_cast<int64_t>(u) * E + e] = run;
      run += c;
    }
    tot[e] = run;
    counts[e] = run;
  }
  __syncthreads();
  // Exclusive scan of tot[0..E): each thread owns a contiguous slice.
  const int per = (E + 1023) / 1024;
  const int lo = min(E, tid * per), hi = min(E, lo + per);
  int s = 0;
  for (int e = lo; e < hi; ++e) s += tot[e];
  part[tid] = s;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {
    int v = tid >= off ? part[tid - off] : 0;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  int base = part[tid] - s;
  for (int e = lo; e < hi; ++e) {
    int c = tot[e];
    tot[e] = base;
    offsets[e] = base;
    base += c;
  }
  if (tid == 1023) offsets[E] = part[1023];
  __syncthreads();
  for (int e = tid; e < E; e += 1024) {
    const int b = tot[e];
    for (int u = 0; u < nunits; ++u) unit_counts[static_cast<int64_t>(u) * E + e] += b;
  }
}

__global__ __launch_bounds__(kThreads) void route_scatter_kernel(
    const int32_t* __restrict__ sel, int64_t R, int top_k, int E, int nbits,
    const int32_t* __restrict__ unit_base, const float* __restrict__ rw,
    int32_t* __restrict__ send_route, int32_t* __restrict__ send_token,
    int32_t* __restrict__ route_to_send, float* __restrict__ weight_perm) {
  extern __shared__ int lds[];
  int* run = lds;                 // [E]   next free row of each expert
  int* wcnt = run + E;            // [kWaves][E] routes of expert e in wave w (this step)
  int* wtag = wcnt + kWaves * E;  // [kWaves][E] step id that wrote wcnt
  const int u = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  for (int e = threadIdx.x; e < E; e += kThreads) {
    run[e] = unit_base[static_cast<int64_t>(u) * E + e];
#pragma unroll
    for (int w = 0; w < kWaves; ++w) wtag[w * E + e] = -1;
  }
  __syncthreads();
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int64_t start = static_cast<int64_t>(u) * kChunk;
  for (int it = 0; it < kIters; ++it) {
    const int64_t i = start + static_cast<int64_t>(it) * kThreads + threadIdx.x;
    const bool present = i < R;
    int e = present ? sel[i] : -1;
    const bool valid = present && route_valid(e, E);
    const int key = valid ? e : E;  // E = "not routed"
    // match mask: lanes of this wave holding the same key
    uint64_t mask = __ballot(1);
    for (int b = 0; b < nbits; ++b) {
      const bool bit = (key >> b) & 1;
      const uint64_t m = __ballot(bit);
      mask &= bit ? m : ~m;
    }
    const int rank_in_wave = __popcll(mask & lt_mask);
    const int cnt_in_wave = __popcll(mask);
    const bool leader = valid && rank_in_wave == 0;
    if (leader) {
      wcnt[wave * E + key] = cnt_in_wave;
      wtag[wave * E + key] = it;
    }
    __syncthreads();
    if (present) {
      if (valid) {
        int pos = run[key] + rank_in_wave;
        for (int w = 0; w < wave; ++w)
          if (wtag[w * E + key] == it) pos += wcnt[w * E + key];
        send_route[pos] = static_cast<int32_t>(i);
        send_token[pos] = static_cast<int32_t>(i / top_k);
        route_to_send[i] = pos;
        if (weight_perm != nullptr) weight_perm[pos] = rw[i];
      } else {
        route_to_send[i] = -1;
      }
    }
    __syncthreads();
    if (leader) atomicAdd(&run[key], cnt_in_wave);
    __syncthreads();
  }
}

// Scatter for large expert counts (E > kMaxExperts4): one wavefront per unit,
// so the stable rank of a route among equal experts comes from the ballot
// match mask alone and LDS holds only the E running row counters.
__global__ __launch_bounds__(64) void route_scatter_wave_kernel(
    const int32_t* __restrict__ sel, int64_t R, int top_k, int E, int nbits,
    const int32_t* __restrict__ unit_base, const float* __restrict__ rw,
    int32_t* __restrict__ send_route, int32_t* __restrict__ send_token,
    int32_t* __restrict__ route_to_send, float* __restrict__ weight_perm) {
  extern __shared__ int run[];  // [E] next free row of each expert
  const int u = blockIdx.x;
  const int lane = threadIdx.x;
  for (int e = lane; e < E; e += 64) run[e] = unit_base[static_cast<int64_t>(u) * E + e];
  __syncthreads();
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int64_t start = static_cast<int64_t>(u) * kChunk;
  for (int it = 0; it < kChunk / 64; ++it) {
    const int64_t i = start + static_cast<int64_t>(it) * 64 + lane;
    const bool present = i < R;
    const int e = present ? sel[i] : -1;
    const bool valid = present && route_valid(e, E);
    const int key = valid ? e : E;
    uint64_t mask = __ballot(1);
    for (int b = 0; b < nbits; ++b) {
      const bool bit = (key >> b) & 1;
      const uint64_t m = __ballot(bit);
      mask &= bit ? m : ~m;
    }
    const int rank = __popcll(mask & lt_mask);
    const int base = valid ? run[key] : 0;
    __syncthreads();  // every lane has read its expert's counter
    if (present) {
      if (valid) {
        const int pos = base + rank;
        send_route[pos] = static_cast<int32_t>(i);
        send_token[pos] = static_cast<int32_t>(i / top_k);
        route_to_send[i] = pos;
        if (weight_perm != nullptr) weight_perm[pos] = rw[i];
        if (rank == 0) run[key] = base + __popcll(mask);
      } else {
        route_to_send[i] = -1;
      }
    }
    __syncthreads();
  }
}

}  // namespace

extern "C" size_t mm_route_workspace_bytes(int64_t num_routes, int32_t num_experts) {
  const int64_t nunits = (num_routes + kChunk - 1) / kChunk;
  return mm_align_up(static_cast<size_t>(nunits) * static_cast<size_t>(num_experts) * 4 + 256, 256);
}

namespace {

int route_launch(const int32_t* selected, int64_t num_routes, int32_t top_k, int32_t num_experts,
                 const float* routing_weights, int32_t* counts, int32_t* offsets, int32_t* send_route,
                 int32_t* send_token, int32_t* route_to_send, float* weight_perm, int32_t* unit_counts,
                 hipStream_t s, const char* what) {
  const int E = num_experts;
  const int nunits = static_cast<int>((num_routes + kChunk - 1) / kChunk);
  if (E > kMaxExperts4) {
    // dynamic LDS above 64 KiB (up to 132 KiB at kMaxExperts); set once
    static std::once_flag once;
    std::call_once(once, [] {
      const int bytes = (kMaxExperts + 1024) * static_cast<int>(sizeof(int));
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(route_count_kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(route_scan_kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(route_scatter_wave_kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    });
  }
  if (nunits > 0) {
    route_count_kernel<<<nunits, kThreads, E * sizeof(int), s>>>(selected, num_routes, E, nunits,
                                                                 unit_counts);
  }
  route_scan_kernel<<<1, 1024, (E + 1024) * sizeof(int), s>>>(unit_counts, E, nunits, counts, offsets);
  if (nunits > 0) {
    const int nbits = 32 - __builtin_clz(static_cast<unsigned>(E));
    if (E <= kMaxExperts4) {
      const size_t lds = static_cast<size_t>(E) * (1 + 2 * kWaves) * sizeof(int);
      route_scatter_kernel<<<nunits, kThreads, lds, s>>>(selected, num_routes, top_k, E, nbits, unit_counts,
                                                         routing_weights, send_route, send_token,
                                                         route_to_send, weight_perm);
    } else {
      route_scatter_wave_kernel<<<nunits, 64, static_cast<size_t>(E) * sizeof(int), s>>>(
          selected, num_routes, top_k, E, nbits, unit_counts, routing_weights, send_route, send_token,
          route_to_send, weight_perm);
    }
  }
  return mm_check_launch(what);
}

}  // namespace

#define MM_ROUTE_CHECK_ARGS(what)                                                                          \
  MM_CHECK_ARG(num_routes >= 0 && num_routes < (int64_t(1) << 31), what ": num_routes out of range");     \
  MM_CHECK_ARG(top_k > 0, what ": top_k must be positive");                                                \
  MM_CHECK_ARG(num_experts > 0 && num_experts <= kMaxExperts, what ": num_experts must be in [1, %d]",     \
               kMaxExperts);                                                                               \
  MM_CHECK_ARG(counts && offsets, what ": counts/offsets must be non-null");                               \
  MM_CHECK_ARG(num_routes == 0 || (selected && send_route && send_token && route_to_send),                 \
               what ": route tables must be non-null");                                                    \
  MM_CHECK_ARG((weight_perm == nullptr) == (routing_weights == nullptr),                                   \
               what ": routing_weights and weight_perm must be given together")

extern "C" int mm_route(const int32_t* selected, int64_t num_routes, int32_t top_k, int32_t num_experts,
                        const float* routing_weights, int32_t* counts, int32_t* offsets,
                        int32_t* send_route, int32_t* send_token, int32_t* route_to_send,
                        float* weight_perm, void* workspace, size_t workspace_bytes,
                        mm_stream_t stream) {
  MM_ROUTE_CHECK_ARGS("mm_route");
  if (workspace_bytes < mm_route_workspace_bytes(num_routes, num_experts) || workspace == nullptr) {
    mm_set_error("mm_route: workspace too small");
    return MM_E_WS;
  }
  return route_launch(selected, num_routes, top_k, num_experts, routing_weights, counts, offsets, send_route,
                      send_token, route_to_send, weight_perm, static_cast<int32_t*>(workspace),
                      mm_hip_stream(stream), "mm_route");
}

// ---------------------------------------------------------------- no-allocation variant
//
// mm_route_noalloc keeps the per-unit count table (the only scratch mm_route
// uses) in a file-scope device array instead of a caller workspace. Every
// GPU the library runs on holds its own copy until the process ends; the
// host reaches it through the address hipGetSymbolAddress returns on that
// device (the array's name in host code is only a stand-in). The table is
// fully rewritten by route_count_kernel on every call, so nothing needs
// clearing; calls that overlap on one GPU (different streams) race on it.
namespace {

constexpr size_t kRouteScratchBytes = size_t(4) << 20;  // 4 MiB
static __device__ __align__(256) int32_t scratch[kRouteScratchBytes / sizeof(int32_t)];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
int32_t* g_scratch_ptr[kMaxDevices] = {nullptr};

int scratch_for_current_device(int32_t** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    mm_set_error("mm_route_noalloc: no usable current device (%s)", hipGetErrorString(e));
    return MM_E_LAUNCH;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      mm_set_error("mm_route_noalloc: hipGetSymbolAddress failed (%s)", hipGetErrorString(e));
      return MM_E_LAUNCH;
    }
    g_scratch_ptr[dev] = static_cast<int32_t*>(p);
  }
  *out = g_scratch_ptr[dev];
  return MM_OK;
}

}  // namespace

extern "C" size_t mm_route_noalloc_scratch_bytes(void) { return kRouteScratchBytes; }

extern "C" int mm_route_noalloc(const int32_t* selected, int64_t num_routes, int32_t top_k,
                                int32_t num_experts, const float* routing_weights, int32_t* counts,
                                int32_t* offsets, int32_t* send_route, int32_t* send_token,
                                int32_t* route_to_send, float* weight_perm, mm_stream_t stream) {
  MM_ROUTE_CHECK_ARGS("mm_route_noalloc");
  const size_t need = mm_route_workspace_bytes(num_routes, num_experts);
  if (need > kRouteScratchBytes) {
    mm_set_error("mm_route_noalloc: %lld routes x %d experts need %zu bytes of scratch, above the %zu-byte "
                 "maximum; use mm_route with a workspace",
                 static_cast<long long>(num_routes), num_experts, need, kRouteScratchBytes);
    return MM_E_ARG;
  }
  int32_t* ws = nullptr;
  if (int rc = scratch_for_current_device(&ws)) return rc;
  return route_launch(selected, num_routes, top_k, num_experts, routing_weights, counts, offsets, send_route,
                      send_token, route_to_send, weight_perm, ws, mm_hip_stream(stream), "mm_route_noalloc");
}
