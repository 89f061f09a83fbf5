// Grouped bf16 GEMMs over expert-major rows on CDNA4 MFMA.
//
// Reference: the FC1/FC2 cube GEMMs (kernels/dispatch_fc1.py:580-752,
// kernels/fc2_combine.py:139-213, kernels/fused_forward.py:551-1213), the
// backward dgrad GEMMs (kernels/dispatch_fc2_bwd.py:223-563,
// kernels/combine_fc1_bwd.py:114-247) and the grouped wgrad
// (kernels/transposed_grouped_gemm.py:24-100). They share one math: for each
// expert e, C_e = A_e * B_e over the rows [offsets[e], offsets[e+1]).
//
// MI355X design
//  * A workgroup of 8 wavefronts (2 per SIMD; 4 for the 128 x 128 tiles)
//    computes a BM x BN tile with v_mfma_f32_32x32x16_bf16, each wave owning
//    a (BM / WM) x (BN / WN) sub-tile. 256 x 256 tiles with K >= 1024 run 4
//    wavefronts of 128 x 128 (one per SIMD, accumulators in the AGPRs) with
//    register-staged operand copies interleaved with the MFMAs.
//  * Otherwise operands go global -> LDS with gfx950 LDS-DMA
//    (global_load_lds_dwordx4) through an NST-stage ring, one barrier per K
//    step. K-contiguous sources
//    sit in LDS as [rows][BK] with XOR-swizzled 16-byte slots and are read
//    with ds_read_b128; M/N-contiguous sources (gate_up_weight [E, H, 2I],
//    the natural down weight, both wgrad operands) keep their natural
//    [BK][cols] layout, swizzled per 4 K-rows, and are read with the
//    transposing ds_read_b64_tr_b16. No transposes in HBM or registers.
//  * Ragged experts: a one-workgroup kernel turns offsets[] into a list of
//    (expert, first row, end row) M-tiles on the device; the GEMM grid is an
//    upper bound and surplus workgroups exit at once. Workgroup ids are
//    remapped so that each XCD (ids congruent mod 8) receives a contiguous
//    range of tiles, grouped GROUP_M-deep along M so that A panels and B
//    tiles are reused from that XCD's L2. Waves whose rows lie past a
//    partial tile's end skip their MFMAs.
//  * FC1 epilogue: the B tile interleaves 32-column groups of gate and up;
//    the tile is staged in LDS as bf16 gate | up, and each thread turns one
//    8-column vector of a row into the weighted gated activation (plus the
//    saved raw FC1 output in bf16, fp16 or fp8 with per-row group scales).
//  * Weight gradients: deep-K experts use 256 x 256 tiles over the ragged K
//    (rows), with every expert's tiles spread evenly over the XCDs; small-K
//    experts use a persistent kernel that streams (tile, K step) stages
//    through an LDS ring and is bound by writing the gradient.
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <type_traits>

#include "common.h"

namespace {

constexpr int kThreads = 256;
constexpr int BK = 64;
constexpr int GROUP_M = 8;
constexpr int kXcds = 8;

struct TileList {
  int32_t count;  // number of M tiles
  int32_t pad[3];
  int4 tiles[1];  // (expert, first row, end row, 0) per M tile
};

__global__ __launch_bounds__(1024) void build_tiles_kernel(const int32_t* __restrict__ offsets, int E, int BM,
                                                           TileList* __restrict__ tl) {
  __shared__ int part[1024];
  const int tid = threadIdx.x;
  const int per = (E + 1023) / 1024;
  const int lo = min(E, tid * per), hi = min(E, lo + per);
  int s = 0;
  for (int e = lo; e < hi; ++e) s += (offsets[e + 1] - offsets[e] + BM - 1) / BM;
  part[tid] = s;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {
    int v = tid >= off ? part[tid - off] : 0;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  int t = part[tid] - s;
  for (int e = lo; e < hi; ++e) {
    const int r0 = offsets[e], r1 = offsets[e + 1];
    for (int r = r0; r < r1; r += BM) tl->tiles[t++] = make_int4(e, r, min(r + BM, r1), 0);
  }
  if (tid == 1023) tl->count = part[1023];
}

// Workgroup id -> logical tile id: XCD x (= pid % 8) receives the contiguous
// logical range [x * per, (x + 1) * per) of the `total` real tiles.
__device__ __forceinline__ int xcd_remap(int pid, int total) {
  const int padded = (total + kXcds - 1) / kXcds * kXcds;
  if (pid >= padded) return -1;
  const int per = padded / kXcds;
  const int l = (pid % kXcds) * per + pid / kXcds;
  return l < total ? l : -1;
}

// Grouped ordering of a (num_m x num_n) tile grid: GROUP_M M-tiles at a time
// sweep all N tiles, so an A panel and a B tile stay hot in L2.
__device__ __forceinline__ void grouped_mn(int l, int num_m, int num_n, int& m, int& n, int group_m = GROUP_M) {
  const int in_group = group_m * num_n;
  const int g = l / in_group;
  const int first = g * group_m;
  const int gs = min(num_m - first, group_m);
  const int r = l - g * in_group;
  m = first + r % gs;
  n = r / gs;
}

// ------------------------------------------------------------------ LDS tiles
//
// Both operand tiles are filled with gfx950 global_load_lds_dwordx4: lane l
// of a wave copies 16 bytes from its own global address to LDS base + 16*l,
// so each wave instruction fills one contiguous 1 KiB chunk and no staging
// registers are needed. Bank conflicts of the MFMA fragment reads are removed
// with XOR swizzles of the 16-byte vector slots, applied on the global side
// (which source vector a lane fetches) and undone on the LDS read side.
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef short v8i16 __attribute__((ext_vector_type(8)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void gbl_void;
typedef __attribute__((address_space(4))) const int32_t const_i32;

constexpr int kChunkElems = 512;  // 1 KiB of bf16 per wave instruction

// LDS-DMA copy issued from inline asm: the compiler does not track it, so it
// adds no conservative vmcnt(0) before later LDS reads (it would otherwise
// serialise every prefetch); completion is awaited explicitly with
// wait_vmcnt<N>() + a barrier. M0 (the LDS destination) is written only here.
// POL 1: non-temporal (streamed once; kept from displacing reused lines).
template <int POL = 0>
__device__ __forceinline__ void copy16_to_lds(const bf16* src, bf16* lds_chunk) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void*)(lds_chunk))));
  if constexpr (POL == 1)
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(src), "s"(m0) : "memory");
  else
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(m0) : "memory");
}

// s_waitcnt vmcnt(N) leaving expcnt / lgkmcnt unconstrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// wait until at most n * PER vector-memory ops of this wave are in flight
template <int PER, int MAXN>
__device__ __forceinline__ void wait_stages(int n) {
  if constexpr (MAXN >= 5) { if (n >= 5) { wait_vmcnt<5 * PER>(); return; } }
  if constexpr (MAXN >= 4) { if (n == 4) { wait_vmcnt<4 * PER>(); return; } }
  if constexpr (MAXN >= 3) { if (n == 3 || (MAXN == 3 && n > 3)) { wait_vmcnt<3 * PER>(); return; } }
  if constexpr (MAXN >= 2) { if (n == 2) { wait_vmcnt<2 * PER>(); return; } }
  if constexpr (MAXN >= 1) { if (n == 1) { wait_vmcnt<PER>(); return; } }
  wait_vmcnt<0>();
}

// Two consecutive int32 at a wave-uniform address, loaded through the scalar
// cache (completion tracked by lgkmcnt, not vmcnt).
__device__ __forceinline__ int2 scalar_load_i32x2(const int32_t* p) {
  uint64_t v;
  asm volatile("s_load_dwordx2 %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p) : "memory");
  return make_int2(static_cast<int>(static_cast<uint32_t>(v)), static_cast<int>(v >> 32));
}

// gfx950 transposing LDS read: within each 16-lane group, lane i receives
// element (i % 4) of the 8-byte chunk read by lane 4*j + i/4, for j = 0..3.
__device__ __forceinline__ v4i16 lds_read_tr16(const bf16* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(p));
}

// K-contiguous operand: LDS [ROWS][BK_] (BK_ = 64 or 32). Vector slot s of
// row r holds source K-vector s ^ swz(r). The LDS has 64 four-byte banks, so
// one pass of a 16-byte fragment read serves 16 lanes = 16 consecutive rows:
// for 128-byte rows, rows r and r + 1 sit in opposite bank halves and
// swz = (r >> 1) & 7 separates the 8 rows of each half; for 64-byte rows the
// row itself selects a quarter and swz = (r >> 2) & 3 separates the rest.
// (Measured: FC1 bank-conflict cycles 2.7e7 -> 8.7e5.) Rows outside the tile
// point at a valid row; their products are never stored.
template <int ROWS, int BK_, int NT = kThreads>
struct KcTile {
  static constexpr int ELEMS = ROWS * BK_;
  static constexpr int VPR = BK_ / 8;                      // vectors per row
  static constexpr int CHUNKS = ELEMS / kChunkElems;       // 1 KiB chunks per K step
  static constexpr int PER_WAVE = CHUNKS / (NT / 64);
  static_assert(PER_WAVE * (NT / 64) == CHUNKS, "chunks/waves mismatch");
  const bf16* ptr[PER_WAVE];

  __device__ static int swz(int r) { return VPR == 8 ? ((r >> 1) & 7) : ((r >> 2) & 3); }

  template <class RowPtr>
  __device__ void init(RowPtr row_ptr) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int v = 0; v < PER_WAVE; ++v) {
      const int q = (v * (NT / 64) + wave) * 64 + lane;
      const int r = q / VPR;
      ptr[v] = row_ptr(r) + ((q % VPR) ^ swz(r)) * 8;
    }
  }
  template <int POL = 0>
  __device__ void issue(bf16* lds, int64_t k0) const {
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int v = 0; v < PER_WAVE; ++v) copy16_to_lds<POL>(ptr[v] + k0, lds + (v * (NT / 64) + wave) * kChunkElems);
  }
  // Register-staged copy: the same vectors as issue(), loaded into VGPRs now
  // and written to the same LDS positions by put() later.
  template <int POL = 0>
  __device__ void load(u32x4_t (&r)[PER_WAVE], int64_t k0) const {
#pragma unroll
    for (int v = 0; v < PER_WAVE; ++v) {
      const u32x4_t* q = reinterpret_cast<const u32x4_t*>(ptr[v] + k0);
      if constexpr (POL == 1)
        r[v] = __builtin_nontemporal_load(q);
      else
        r[v] = *q;
    }
  }
  __device__ static void put(bf16* lds, const u32x4_t (&r)[PER_WAVE]) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int v = 0; v < PER_WAVE; ++v)
      *reinterpret_cast<u32x4_t*>(lds + (v * (NT / 64) + wave) * kChunkElems + lane * 8) = r[v];
  }
  // MFMA 32x32x16 operand: row r0 + lane%32, k = kk + 8*(lane/32) .. +8
  __device__ static bf16x8 frag(const bf16* lds, int r0, int kk, int lane) {
    const int r = r0 + (lane & 31);
    const int kv = (kk >> 3) + (lane >> 5);
    return *reinterpret_cast<const bf16x8*>(lds + r * BK_ + ((kv ^ swz(r)) << 3));
  }
};

// Swizzle of the N-contiguous tile: vector slot of (k, source vector cv) is
// cv ^ mn_swz(k). The pattern keeps the 4 K-rows x 32 bytes touched by a
// 16-lane transposing read in distinct banks for 128- and 256-byte passes.
__device__ __forceinline__ int mn_swz(int k) { return (0xEA40 >> ((k & 3) * 4)) & 0xF; }  // {0,4,10,14}

// M/N-contiguous operand: LDS [BK_][ROWS] in the source's natural layout
// (swizzled); MFMA fragments are read with the transposing LDS read.
template <int ROWS, int BK_, int NT = kThreads>
struct MnTile {
  static constexpr int ELEMS = BK_ * ROWS;
  static constexpr int VPR = ROWS / 8;                      // 16-byte vectors per K row
  static constexpr int CHUNKS = ELEMS / kChunkElems;
  static constexpr int PER_WAVE = CHUNKS / (NT / 64);
  static constexpr int KPC = 64 / VPR;                      // K rows per 1 KiB chunk
  static_assert(PER_WAVE * (NT / 64) == CHUNKS, "chunks/waves mismatch");
  static_assert(VPR >= 16, "swizzle needs >= 16 vectors per row");
  const bf16* ptr[PER_WAVE];

  // K row and source column (elements) this lane copies in instruction v.
  __device__ static int k_of(int v) {
    return ((v * (NT / 64) + (threadIdx.x >> 6)) * 64 + (threadIdx.x & 63)) / VPR;
  }
  __device__ static int col_of(int v) {
    const int q = (v * (NT / 64) + (threadIdx.x >> 6)) * 64 + (threadIdx.x & 63);
    return ((q % VPR) ^ mn_swz(q / VPR)) * 8;
  }
  // Fixed-stride source: element (k, c) at base + k*ld + col_off(c).
  template <class ColOff>
  __device__ void init_strided(const bf16* base, int64_t ld, ColOff col_off) {
#pragma unroll
    for (int v = 0; v < PER_WAVE; ++v) ptr[v] = base + static_cast<int64_t>(k_of(v)) * ld + col_off(col_of(v));
  }
  template <int POL = 0>
  __device__ void issue(bf16* lds, int64_t off) const {
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int v = 0; v < PER_WAVE; ++v) copy16_to_lds<POL>(ptr[v] + off, lds + (v * (NT / 64) + wave) * kChunkElems);
  }
  template <int POL = 0>
  __device__ void load(u32x4_t (&r)[PER_WAVE], int64_t off) const {
#pragma unroll
    for (int v = 0; v < PER_WAVE; ++v) {
      const u32x4_t* q = reinterpret_cast<const u32x4_t*>(ptr[v] + off);
      if constexpr (POL == 1)
        r[v] = __builtin_nontemporal_load(q);
      else
        r[v] = *q;
    }
  }
  __device__ static void put(bf16* lds, const u32x4_t (&r)[PER_WAVE]) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int v = 0; v < PER_WAVE; ++v)
      *reinterpret_cast<u32x4_t*>(lds + (v * (NT / 64) + wave) * kChunkElems + lane * 8) = r[v];
  }
  // Per-vector source (wgrad): src(v) -> row pointer (column 0 of the tile)
  // for the K row this lane copies in instruction v.
  template <class Src>
  __device__ static void issue_rows(bf16* lds, Src src) {
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int v = 0; v < PER_WAVE; ++v)
      copy16_to_lds(src(v) + col_of(v), lds + (v * (NT / 64) + wave) * kChunkElems);
  }
  __device__ static bf16x8 frag(const bf16* lds, int r0, int kk, int lane) {
    const int s = lane & 15, g = lane >> 4;
    const int k = kk + 8 * (g >> 1) + (s >> 2);
    const int col = r0 + 16 * (g & 1) + 4 * (s & 3);
    const bf16* q0 = lds + k * ROWS + ((((col >> 3) ^ mn_swz(k)) << 3) | (col & 7));
    const bf16* q1 = lds + (k + 4) * ROWS + ((((col >> 3) ^ mn_swz(k + 4)) << 3) | (col & 7));
    const v4i16 lo = lds_read_tr16(q0);
    const v4i16 hi = lds_read_tr16(q1);
    const v8i16 w = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(bf16x8, w);
  }
  // Zero K rows [k_valid, BK_) of a filled tile (ragged K tail).
  __device__ static void zero_tail(bf16* lds, int k_valid) {
    for (int i = threadIdx.x; i < (BK_ - k_valid) * VPR; i += NT)
      reinterpret_cast<uint4*>(lds + k_valid * ROWS)[i] = make_uint4(0, 0, 0, 0);
  }
};

// ------------------------------------------------------------------ MMA core
template <int BM, int BN, int WM, int WN>
struct MmaTile {
  static constexpr int TM = BM / WM, TN = BN / WN;
  static constexpr int MI = TM / 32, NI = TN / 32;
  f32x16 acc[MI][NI];

  __device__ void zero() {
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NI; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  }

  // One BK_-deep step; fragments of sub-step kk+16 are read while the MFMAs
  // of sub-step kk issue.
  // TRANS: the MFMA takes its operands swapped, so acc[i][j] holds the
  // transposed block and lane l has 4 consecutive output columns of row
  // l % 32 per group of 4 accumulator elements (see acc_col).
  template <class ATile, class BTile, int BK_, bool TRANS = false>
  __device__ void compute(const bf16* As, const bf16* Bs, int wm, int wn, int lane) {
    bf16x8 a[2][MI], b[2][NI];
#pragma unroll
    for (int i = 0; i < MI; ++i) a[0][i] = ATile::frag(As, wm * TM + i * 32, 0, lane);
#pragma unroll
    for (int j = 0; j < NI; ++j) b[0][j] = BTile::frag(Bs, wn * TN + j * 32, 0, lane);
#pragma unroll
    for (int s = 0; s < BK_ / 16; ++s) {
      const int cur = s & 1, nxt = cur ^ 1;
      if (s + 1 < BK_ / 16) {
#pragma unroll
        for (int i = 0; i < MI; ++i) a[nxt][i] = ATile::frag(As, wm * TM + i * 32, (s + 1) * 16, lane);
#pragma unroll
        for (int j = 0; j < NI; ++j) b[nxt][j] = BTile::frag(Bs, wn * TN + j * 32, (s + 1) * 16, lane);
      }
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j)
          acc[i][j] = TRANS ? __builtin_amdgcn_mfma_f32_32x32x16_bf16(b[cur][j], a[cur][i], acc[i][j], 0, 0, 0)
                            : __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[cur][i], b[cur][j], acc[i][j], 0, 0, 0);
      // schedule: each MFMA followed by (up to) two of the next step's LDS
      // fragment reads, instead of the reads clustered ahead of the MFMAs
      // (measured -3.5% FC1 time)
#pragma unroll
      for (int q = 0; q < MI * NI; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // LDS read
      }
    }
  }

  // Single 16-deep sub-step pieces for hand-scheduled loops (TRANS layout).
  template <class ATile, class BTile, int BK_>
  __device__ static void frags(bf16x8 (&a)[MI], bf16x8 (&b)[NI], const bf16* As, const bf16* Bs, int wm, int wn,
                               int kk, int lane) {
#pragma unroll
    for (int i = 0; i < MI; ++i) a[i] = ATile::frag(As, wm * TM + i * 32, kk, lane);
#pragma unroll
    for (int j = 0; j < NI; ++j) b[j] = BTile::frag(Bs, wn * TN + j * 32, kk, lane);
  }
  __device__ void mfmas_t(const bf16x8 (&a)[MI], const bf16x8 (&b)[NI]) {
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NI; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b[j], a[i], acc[i][j], 0, 0, 0);
  }

  // Tile row of accumulator element r (0..15) of a 32x32 block for `lane`;
  // the column is lane & 31.
  __device__ static int acc_row(int r, int lane) { return (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3); }
  // TRANS layout: elements 4g .. 4g + 3 of a block sit in row lane % 32 and
  // columns acc_col(g, lane) .. + 3.
  __device__ static int acc_col(int g, int lane) { return g * 8 + (lane >> 5) * 4; }
};

// Non-temporal 16- and 8-byte stores of GEMM outputs. Measured against plain
// stores: Kimi-scale weight-streaming GEMMs FC1 -2%, FC2 -8%, dgrads -1.5%;
// Qwen-like weight gradients -3 to -5%; the combine that reads FC2's output
// next is a few microseconds slower (the rows no longer wait in the
// memory-side cache).
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void store_out16(void* dst, uint4 v) {
  __builtin_nontemporal_store(u32x4_t{v.x, v.y, v.z, v.w}, reinterpret_cast<u32x4_t*>(dst));
}
__device__ __forceinline__ void store_out8(void* dst, uint2 v) {
  __builtin_nontemporal_store(u32x2_t{v.x, v.y}, reinterpret_cast<u32x2_t*>(dst));
}

// Epilogue staging: a BM x NC bf16 tile is written to LDS ([BM][NC+8], the
// padding keeps the two half-waves of a store on different banks), then
// copied out row by row with 16-byte global stores; rows >= rows are skipped.
template <int BM, int NC, int NT = kThreads>
struct StageOut {
  static constexpr int PITCH = NC + 8;
  static constexpr int ELEMS = BM * PITCH;
  __device__ static void put(bf16* lds, int r, int c, float v) {
    reinterpret_cast<uint16_t*>(lds)[r * PITCH + c] = f32_to_bf16_bits(v);
  }
  // four consecutive columns c .. c + 3 (c % 4 == 0) of row r: one 8-byte write
  __device__ static void put4(bf16* lds, int r, int c, float v0, float v1, float v2, float v3) {
    *reinterpret_cast<uint2*>(lds + r * PITCH + c) = make_uint2(pack_bf16x2(v0, v1), pack_bf16x2(v2, v3));
  }
  // out points at (row 0, column 0) of the tile; ld in elements.
  __device__ static void flush(const bf16* lds, int rows, bf16* out, int64_t ld) {
    __syncthreads();
    constexpr int VPR = NC / 8;
    for (int idx = threadIdx.x; idx < BM * VPR; idx += NT) {
      const int r = idx / VPR, cv = idx % VPR;
      if (r < rows)
        store_out16(out + static_cast<int64_t>(r) * ld + cv * 8, *reinterpret_cast<const uint4*>(lds + r * PITCH + cv * 8));
    }
  }
};

// ------------------------------------------------------------------ row GEMM
struct RowsArgs {
  const bf16* a;
  int64_t lda;
  const int32_t* a_rows;  // optional gather of A rows
  const bf16* b;
  int64_t b_se, b_sn, b_sk;
  int n, k;
  bf16* c;
  int64_t ldc;
  const TileList* tl;
  int group_m;  // M tiles per grouped sweep of the N tiles
  int xcd_mod;  // 1: M tile m runs on XCD m % 8 (its N tiles in order); 0: contiguous XCD shares
  // gated (FC1) epilogue
  const float* w;
  void* fc1_out;   // saved raw gate | up in fc1_fmt (MM_FC1_*), or null
  int fc1_fmt;
  float* fc1_scale;  // FP8 scale table [rows, 2I / MM_FC1_SCALE_GROUP]
  int inter;
  int act_kind;
  float beta, lbeta, clamp;
};

enum { EPI_STORE = 0, EPI_GATED = 1 };
enum { B_KCONTIG = 0, B_NCONTIG = 1 };

// NST-stage ring of LDS buffers: stage s is copied into buffer s % NST while
// the MFMAs consume stage s - NST + 1; one barrier per K step.
// Epilogue of a row-GEMM tile (LDS-staged, 16-byte stores); the caller
// has passed a barrier after the tile's last LDS reads.
// w_pre(it): routing weight of row threadIdx.x / (BN / 16) + it * NT / (BN / 16).
template <int BM, int BN, int NT, int EPI, int ACT, class Mma, class WFn>
__device__ __forceinline__ void rows_epilogue(const RowsArgs& p, bf16* smem, const Mma& mma, int row0, int rows,
                                              int nt, int wm, int wn, int lane, WFn w_pre) {
  using Out = StageOut<BM, BN, NT>;
  constexpr int EPI_VPR = BN / 16, EPI_IT = EPI == EPI_GATED ? BM * EPI_VPR / NT : 1;
  const int n0 = nt * BN;
  // The accumulators are
  // transposed (compute<..., true>): each lane stages 4 consecutive columns
  // of its row with one 8-byte write.
  const int trow = wm * Mma::TM + (lane & 31);
  if constexpr (EPI == EPI_STORE) {
#pragma unroll
    for (int i = 0; i < Mma::MI; ++i)
#pragma unroll
      for (int j = 0; j < Mma::NI; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          Out::put4(smem, trow + i * 32, wn * Mma::TN + j * 32 + Mma::acc_col(g, lane), mma.acc[i][j][4 * g],
                    mma.acc[i][j][4 * g + 1], mma.acc[i][j][4 * g + 2], mma.acc[i][j][4 * g + 3]);
    Out::flush(smem, rows, p.c + static_cast<int64_t>(row0) * p.ldc + n0, p.ldc);
  } else {
    // Stage bf16(gate) in LDS columns [0, BN/2) and bf16(up) in [BN/2, BN)
    // (tile column = output column - jbase), then each thread turns one
    // 8-column vector of a row into act = bf16(act_fn(gate, up) * w[row]).
    const int jbase = nt * (BN / 2);
#pragma unroll
    for (int i = 0; i < Mma::MI; ++i)
#pragma unroll
      for (int jj = 0; jj < Mma::NI; ++jj)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          Out::put4(smem, trow + i * 32,
                    (jj & 1) * (BN / 2) + wn * (Mma::TN / 2) + (jj >> 1) * 32 + Mma::acc_col(g, lane),
                    mma.acc[i][jj][4 * g], mma.acc[i][jj][4 * g + 1], mma.acc[i][jj][4 * g + 2],
                    mma.acc[i][jj][4 * g + 3]);
    __syncthreads();
    constexpr int VPR = BN / 16;  // 8-column vectors per output row
    const int64_t ldf = 2 * static_cast<int64_t>(p.inter);
    // every lane runs every pass (rows past the tile only skip their
    // stores) so that the 16 lanes of a row can reduce the FP8 group amax
    static_assert(VPR == EPI_VPR, "epilogue vector split");
#pragma unroll
    for (int it = 0; it < EPI_IT; ++it) {
      const int idx = threadIdx.x + it * NT;
      const int r = idx / VPR, cv = idx % VPR;
      const bool valid = r < rows;
      const uint4 gv = *reinterpret_cast<const uint4*>(smem + r * Out::PITCH + cv * 8);
      const uint4 uv = *reinterpret_cast<const uint4*>(smem + r * Out::PITCH + BN / 2 + cv * 8);
      const int64_t row = row0 + r;
      const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, uw[4] = {uv.x, uv.y, uv.z, uv.w};
      if (valid) {
        const float wr = w_pre(it);
        uint32_t ow[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float a0 = gated_act(ACT, __uint_as_float(gw[q] << 16), __uint_as_float(uw[q] << 16),
                                     p.beta, p.lbeta, p.clamp) * wr;
          const float a1 = gated_act(ACT, __uint_as_float(gw[q] & 0xffff0000u),
                                     __uint_as_float(uw[q] & 0xffff0000u), p.beta, p.lbeta, p.clamp) * wr;
          ow[q] = pack_bf16x2(a0, a1);
        }
        store_out16(p.c + row * p.ldc + jbase + cv * 8, make_uint4(ow[0], ow[1], ow[2], ow[3]));
      }
      if (!p.fc1_out) continue;
      if (p.fc1_fmt == MM_FC1_BF16) {
        if (valid) {
          uint16_t* fo = static_cast<uint16_t*>(p.fc1_out) + row * ldf + jbase + cv * 8;
          store_out16(fo, gv);
          store_out16(fo + p.inter, uv);
        }
      } else if (p.fc1_fmt == MM_FC1_FP16) {
        uint32_t gh[4], uh[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          gh[q] = pack_f16x2(__uint_as_float(gw[q] << 16), __uint_as_float(gw[q] & 0xffff0000u));
          uh[q] = pack_f16x2(__uint_as_float(uw[q] << 16), __uint_as_float(uw[q] & 0xffff0000u));
        }
        if (valid) {
          uint16_t* fo = static_cast<uint16_t*>(p.fc1_out) + row * ldf + jbase + cv * 8;
          store_out16(fo, make_uint4(gh[0], gh[1], gh[2], gh[3]));
          store_out16(fo + p.inter, make_uint4(uh[0], uh[1], uh[2], uh[3]));
        }
      } else if constexpr ((BN / 2) % MM_FC1_SCALE_GROUP == 0) {
        // FP8: one scale per row per MM_FC1_SCALE_GROUP columns of gate (and
        // of up); a tile row holds BN / 2 of them, i.e. one or two groups.
        // The group's 16 consecutive lanes reduce the amax of |bf16 value|
        // with xor shuffles. (Narrower tiles never see FP8: mm_fc1_swiglu
        // requires inter % MM_FC1_SCALE_GROUP == 0 for it, which selects
        // 256- or 512-wide tiles.)
        constexpr int GV = MM_FC1_SCALE_GROUP / 8;  // lanes per scale group
        static_assert(VPR % GV == 0, "scale groups tile the row");
        float ga = 0.0f, ua = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          ga = fmaxf(ga, fmaxf(fabsf(__uint_as_float(gw[q] << 16)), fabsf(__uint_as_float(gw[q] & 0xffff0000u))));
          ua = fmaxf(ua, fmaxf(fabsf(__uint_as_float(uw[q] << 16)), fabsf(__uint_as_float(uw[q] & 0xffff0000u))));
        }
#pragma unroll
        for (int off = 1; off < GV; off <<= 1) {
          ga = fmaxf(ga, __shfl_xor(ga, off));
          ua = fmaxf(ua, __shfl_xor(ua, off));
        }
        const float gs = ga > 0.0f ? ga : 1.0f, us = ua > 0.0f ? ua : 1.0f;
        const float gm = kFp8Max / gs, um = kFp8Max / us;
        uint32_t gq[2] = {0, 0}, uq[2] = {0, 0};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t g0 = f32_to_e4m3fn(__uint_as_float(gw[q] << 16) * gm);
          const uint32_t g1 = f32_to_e4m3fn(__uint_as_float(gw[q] & 0xffff0000u) * gm);
          const uint32_t u0 = f32_to_e4m3fn(__uint_as_float(uw[q] << 16) * um);
          const uint32_t u1 = f32_to_e4m3fn(__uint_as_float(uw[q] & 0xffff0000u) * um);
          gq[q >> 1] |= (g0 | (g1 << 8)) << ((q & 1) * 16);
          uq[q >> 1] |= (u0 | (u1 << 8)) << ((q & 1) * 16);
        }
        if (valid) {
          uint8_t* fo = static_cast<uint8_t*>(p.fc1_out) + row * ldf + jbase + cv * 8;
          store_out8(fo, make_uint2(gq[0], gq[1]));
          store_out8(fo + p.inter, make_uint2(uq[0], uq[1]));
          if (cv % GV == 0) {
            const int groups = p.inter / MM_FC1_SCALE_GROUP;
            float* sc = p.fc1_scale + row * (2 * groups) + (jbase + cv * 8) / MM_FC1_SCALE_GROUP;
            sc[0] = gs / kFp8Max;
            sc[groups] = us / kFp8Max;
          }
        }
      }
    }
  }
}

// REG: operands are loaded into VGPRs one stage ahead and written to a
// 2-deep LDS ring with ordinary LDS stores after each stage's MFMAs (one
// barrier per K step), instead of LDS-DMA copies.
template <int BM, int BN, int BK_, int NST, int BLAYOUT, int EPI, int NT = kThreads, int ACT = 0, bool REG = false,
          int BPOL = 0>
__global__ __launch_bounds__(NT) void grouped_rows_kernel(RowsArgs p) {
  constexpr int WN = 2, WM = NT / 64 / WN;  // 4 waves: 2x2, 8 waves: 4x2
  using Mma = MmaTile<BM, BN, WM, WN>;
  using ATile = KcTile<BM, BK_, NT>;
  using BTile = typename std::conditional<BLAYOUT == B_KCONTIG, KcTile<BN, BK_, NT>, MnTile<BN, BK_, NT>>::type;
  static_assert(EPI != EPI_GATED || (Mma::NI % 2 == 0 && BLAYOUT == B_NCONTIG), "gated epilogue layout");
  constexpr int STAGE = ATile::ELEMS + BTile::ELEMS;
  constexpr int LPS = ATile::PER_WAVE + BTile::PER_WAVE;  // copies per wave per stage
  using Out = StageOut<BM, BN, NT>;
  constexpr int SMEM = (NST * STAGE > Out::ELEMS) ? NST * STAGE : Out::ELEMS;
  __shared__ __attribute__((aligned(1024))) bf16 smem[SMEM];

  const int num_m = p.tl->count;
  const int num_n = p.n / BN;
  int mt, nt;
  if (p.xcd_mod) {
    const int j = blockIdx.x / kXcds;
    mt = (j / num_n) * kXcds + static_cast<int>(blockIdx.x % kXcds);
    nt = j % num_n;
    if (mt >= num_m) return;
  } else {
    const int l = xcd_remap(blockIdx.x, num_m * num_n);
    if (l < 0) return;
    grouped_mn(l, num_m, num_n, mt, nt, p.group_m);
  }
  const int4 tile = p.tl->tiles[mt];
  const int e = tile.x, row0 = tile.y, rows = tile.z - tile.y;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int n0 = nt * BN;
  const bf16* bexp = p.b + static_cast<int64_t>(e) * p.b_se;

  ATile la;
  la.init([&](int r) -> const bf16* {
    const int rr = row0 + min(r, rows - 1);  // rows past the tile re-read its last row
    const int64_t src = p.a_rows ? static_cast<int64_t>(p.a_rows[rr]) : static_cast<int64_t>(rr);
    return p.a + src * p.lda;
  });

  // B tile column c -> global column n. Gated: each wave's TN columns hold
  // 32-wide groups alternating gate / up of the same output columns.
  auto bcol = [&](int c) -> int64_t {
    if constexpr (EPI == EPI_GATED) {
      const int wnc = c / Mma::TN, ni = (c % Mma::TN) / 32, jj = c & 31;
      return static_cast<int64_t>(ni & 1) * p.inter + nt * (BN / 2) + wnc * (Mma::TN / 2) + (ni >> 1) * 32 + jj;
    } else {
      return n0 + c;
    }
  };

  BTile lb;
  int64_t b_step;  // element offset of one BK_ step along K
  if constexpr (BLAYOUT == B_KCONTIG) {
    lb.init([&](int c) -> const bf16* { return bexp + bcol(c) * p.b_sn; });
    b_step = BK_;
  } else {
    lb.init_strided(bexp, p.b_sk, bcol);
    b_step = static_cast<int64_t>(BK_) * p.b_sk;
  }
  auto issue = [&](int s) {
    bf16* buf = smem + (s % NST) * STAGE;
    la.issue(buf, static_cast<int64_t>(s) * BK_);
    lb.template issue<BPOL>(buf + ATile::ELEMS, s * b_step);
  };

  Mma mma;
  mma.zero();
  const int nk = p.k / BK_;
  // waves whose row slab lies entirely past the tile's valid rows (the
  // partial last tile of an expert) skip their MFMAs; their accumulators stay
  // zero and those rows are never stored
  const bool active = wm * Mma::TM < rows;
  // gated epilogue: each thread's routing weights (rows tid / VPR + i * NT / VPR
  // of the tile) are fetched now, their latency hidden by the main loop
  constexpr int EPI_VPR = BN / 16, EPI_IT = EPI == EPI_GATED ? BM * EPI_VPR / NT : 1;
  float w_pre[EPI_IT];
  if constexpr (EPI == EPI_GATED) {
    static_assert(NT % EPI_VPR == 0 && (BM * EPI_VPR) % NT == 0, "epilogue passes");
#pragma unroll
    for (int it = 0; it < EPI_IT; ++it) {
      const int r = threadIdx.x / EPI_VPR + it * (NT / EPI_VPR);
      w_pre[it] = r < rows ? p.w[row0 + r] : 0.0f;
    }
  }
  if constexpr (REG) {
    static_assert(NST == 2, "register staging uses a 2-deep LDS ring");
    u32x4_t ra[ATile::PER_WAVE], rb[BTile::PER_WAVE];
    auto gload = [&](int s) {
      la.load(ra, static_cast<int64_t>(s) * BK_);
      lb.template load<BPOL>(rb, s * b_step);
    };
    auto sput = [&](int s) {
      bf16* buf = smem + (s & 1) * STAGE;
      ATile::put(buf, ra);
      BTile::put(buf + ATile::ELEMS, rb);
    };
    static_assert(BK_ == 64, "four 16-deep sub-steps per stage");
    using Frag = bf16x8;
    Frag fa[2][Mma::MI], fb[2][Mma::NI];
    if (nk > 0) {
      gload(0);
      sput(0);
      if (nk > 1) gload(1);
    }
    __syncthreads();
    if (active) {
      Mma::template frags<ATile, BTile, BK_>(fa[0], fb[0], smem, smem + ATile::ELEMS, wm, wn, 0, lane);
      // Sub-step s issues its MFMAs from fragment set s & 1 while the next
      // sub-step's fragments load into the other set. Stage kt + 1's
      // registers go to LDS during sub-steps 0 (A) and 1 (B), into the slot
      // stage kt - 1 used (its last fragments were read before the previous
      // barrier), then stage kt + 2's loads are issued. The barrier after
      // sub-step 2 publishes stage kt + 1, whose first fragments are read
      // during sub-step 3.
      // Branch-free so that the scheduler can interleave the LDS writes and
      // global loads with the MFMAs: past the last stage the writes land in
      // a slot nobody reads again and the loads repeat the last stage.
      for (int kt = 0; kt < nk; ++kt) {
        const bf16* cur = smem + (kt & 1) * STAGE;
        bf16* nxt = smem + ((kt + 1) & 1) * STAGE;
#pragma unroll
        for (int ss = 0; ss < 4; ++ss) {
          const int c = ss & 1, n = c ^ 1;
          if (ss < 3)
            Mma::template frags<ATile, BTile, BK_>(fa[n], fb[n], cur, cur + ATile::ELEMS, wm, wn, (ss + 1) * 16, lane);
          else
            Mma::template frags<ATile, BTile, BK_>(fa[n], fb[n], nxt, nxt + ATile::ELEMS, wm, wn, 0, lane);
          mma.mfmas_t(fa[c], fb[c]);
          // each operand's next loads go out as soon as its registers are in
          // LDS: A (sub-step 0) one sub-step before B (sub-step 1), which
          // gives A's gathered rows the longer latency cover (E32 step -1%,
          // the Qwen-like dgrads -1 to -2%; issuing both at sub-step 0, with
          // both LDS writes there, measured +3-6%)
          if (ss == 0) {
            ATile::put(nxt, ra);
            la.load(ra, static_cast<int64_t>(min(kt + 2, nk - 1)) * BK_);
          }
          if (ss == 1) {
            BTile::put(nxt + ATile::ELEMS, rb);
            lb.template load<BPOL>(rb, min(kt + 2, nk - 1) * b_step);
          }
#pragma unroll
          for (int q = 0; q < Mma::MI * Mma::NI; ++q) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
            __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // LDS write
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // global load
          }
          if (ss == 2) __syncthreads();
        }
      }
    } else {
      for (int kt = 0; kt < nk; ++kt) {
        if (kt + 1 < nk) {
          sput(kt + 1);
          if (kt + 2 < nk) gload(kt + 2);
        }
        __syncthreads();
      }
    }
  } else {
#pragma unroll
  for (int s = 0; s < NST - 1; ++s)
    if (s < nk) issue(s);
  if (active) {
    for (int kt = 0; kt < nk; ++kt) {
      wait_stages<LPS, NST - 2>(min(nk - 1, kt + NST - 2) - kt);
      __syncthreads();
      if (kt + NST - 1 < nk) issue(kt + NST - 1);
      const bf16* cur = smem + (kt % NST) * STAGE;
      mma.template compute<ATile, BTile, BK_, true>(cur, cur + ATile::ELEMS, wm, wn, lane);
    }
  } else {  // same copies and barriers, no MFMAs
    for (int kt = 0; kt < nk; ++kt) {
      wait_stages<LPS, NST - 2>(min(nk - 1, kt + NST - 2) - kt);
      __syncthreads();
      if (kt + NST - 1 < nk) issue(kt + NST - 1);
    }
  }
  }
  __syncthreads();

  rows_epilogue<BM, BN, NT, EPI, ACT>(p, smem, mma, row0, rows, nt, wm, wn, lane, [&](int it) { return w_pre[it]; });
}

// ------------------------------------------------------------------ wgrad

struct WgradArgs {
  const bf16* p;
  int64_t ldp;
  const int32_t* p_rows;
  const bf16* q;
  int64_t ldq;
  const int32_t* q_rows;
  const int32_t* offsets;
  int n1, n2;
  bf16* c;
  int rows_cap;  // row capacity (max_rows): rows at or past it are never read
};

// Scheduling: the (t1, t2) tiles of every expert are split into 8 equal
// slices and slice x runs on XCD x (workgroup ids congruent to x mod 8), so
// hot and cold experts are spread evenly over the XCDs whatever the routing
// skew, while each XCD still sweeps a contiguous, L2-friendly block of one
// expert's tiles.
// DIRECT = true (small-K tiles): the output tile is staged in the stage
// buffers themselves (XOR-swizzled, unpadded) instead of a separate padded
// region, so LDS stays at 2 stages and several workgroups per CU overlap
// their 16-byte stores.
template <int BM, int BN, int BK_, int NST, bool DIRECT, int NT = kThreads>
__global__ __launch_bounds__(NT) void grouped_wgrad_kernel(WgradArgs a, int num_experts, int per_xcd) {
  constexpr int WN = 2, WM = NT / 64 / WN;
  using Mma = MmaTile<BM, BN, WM, WN>;
  using PTile = MnTile<BM, BK_, NT>;
  using QTile = MnTile<BN, BK_, NT>;
  constexpr int STAGE = PTile::ELEMS + QTile::ELEMS;
  using Out = StageOut<BM, BN, NT>;
  constexpr int SMEM = (DIRECT || NST * STAGE > Out::ELEMS) ? NST * STAGE : Out::ELEMS;
  __shared__ __attribute__((aligned(1024))) bf16 smem[SMEM];
  const int t1n = a.n1 / BM, t2n = a.n2 / BN;
  const int per_e = t1n * t2n;
  const int x = blockIdx.x % kXcds, j = blockIdx.x / kXcds;
  const int e = j / per_xcd;
  const int t = x * per_xcd + (j - e * per_xcd);
  if (e >= num_experts || t >= per_e) return;
  int t1, t2;
  grouped_mn(t, t1n, t2n, t1, t2);
  const int r0 = a.offsets[e], r1 = a.offsets[e + 1];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int64_t pc = static_cast<int64_t>(t1) * BM, qc = static_cast<int64_t>(t2) * BN;

  // Source rows of a stage are looked up one stage ahead (ordinary vector
  // loads); with the 2-stage ring their wait coincides with the stage wait.
  int prow[PTile::PER_WAVE], qrow[QTile::PER_WAVE];
  auto fetch_rows = [&](int s) {
    const int kbase = r0 + s * BK_;
#pragma unroll
    for (int v = 0; v < PTile::PER_WAVE; ++v) {
      const int r = min(kbase + PTile::k_of(v), r1 - 1);
      prow[v] = a.p_rows ? a.p_rows[r] : r;
    }
#pragma unroll
    for (int v = 0; v < QTile::PER_WAVE; ++v) {
      const int r = min(kbase + QTile::k_of(v), r1 - 1);
      qrow[v] = a.q_rows ? a.q_rows[r] : r;
    }
  };
  auto issue = [&](int s) {
    bf16* buf = smem + (s % NST) * STAGE;
    // one 32 x 32 -> 64-bit multiply-add per row address (strides < 2^32 are
    // checked on the host)
    PTile::issue_rows(buf, [&](int v) {
      return a.p + pc + static_cast<uint64_t>(static_cast<uint32_t>(prow[v])) * static_cast<uint32_t>(a.ldp);
    });
    QTile::issue_rows(buf + PTile::ELEMS, [&](int v) {
      return a.q + qc + static_cast<uint64_t>(static_cast<uint32_t>(qrow[v])) * static_cast<uint32_t>(a.ldq);
    });
  };

  Mma mma;
  mma.zero();
  const int nk = (r1 - r0 + BK_ - 1) / BK_;
  static_assert(NST == 2, "wgrad row-index prefetch assumes a 2-stage ring");
  if (nk > 0) {
    fetch_rows(0);
    issue(0);
    if (nk > 1) fetch_rows(1);
  }
  for (int kt = 0; kt < nk; ++kt) {
    wait_vmcnt<0>();
    __syncthreads();
    bf16* cur = smem + (kt % NST) * STAGE;
    const int kv = r1 - r0 - kt * BK_;
    if (kv < BK_) {  // ragged tail: zero the K rows past the expert's end
      PTile::zero_tail(cur, kv);
      QTile::zero_tail(cur + PTile::ELEMS, kv);
      __syncthreads();
    }
    if (kt + 1 < nk) {
      issue(kt + 1);
      if (kt + 2 < nk) fetch_rows(kt + 2);
    }
    mma.template compute<PTile, QTile, BK_, true>(cur, cur + PTile::ELEMS, wm, wn, lane);
  }
  bf16* out = a.c + static_cast<int64_t>(e) * a.n1 * a.n2 + static_cast<int64_t>(t1) * BM * a.n2 + t2 * BN;
  if constexpr (DIRECT) {
    // stage the tile unpadded in the (now idle) stage buffers, 16-byte
    // vector slot v of row r at v ^ (r & 7), then 16-byte stores
    static_assert(BM * BN <= NST * STAGE, "staging must fit the stage buffers");
    constexpr int VPR = BN / 8;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < Mma::MI; ++i)
#pragma unroll
      for (int jj = 0; jj < Mma::NI; ++jj)
#pragma unroll
        for (int g = 0; g < 4; ++g) {  // transposed accumulators: 4 consecutive columns per lane
          const int tr = wm * Mma::TM + i * 32 + (lane & 31);
          const int tc = wn * Mma::TN + jj * 32 + Mma::acc_col(g, lane);
          *reinterpret_cast<uint2*>(smem + tr * BN + ((((tc >> 3) ^ (tr & 7)) << 3) | (tc & 7))) =
              make_uint2(pack_bf16x2(mma.acc[i][jj][4 * g], mma.acc[i][jj][4 * g + 1]),
                         pack_bf16x2(mma.acc[i][jj][4 * g + 2], mma.acc[i][jj][4 * g + 3]));
        }
    __syncthreads();
    for (int idx = threadIdx.x; idx < BM * VPR; idx += NT) {
      const int r = idx / VPR, cv = idx % VPR;
      store_out16(out + static_cast<int64_t>(r) * a.n2 + cv * 8,
                  *reinterpret_cast<const uint4*>(smem + r * BN + ((cv ^ (r & 7)) << 3)));
    }
  } else {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < Mma::MI; ++i)
#pragma unroll
      for (int jj = 0; jj < Mma::NI; ++jj)
#pragma unroll
        for (int g = 0; g < 4; ++g)  // transposed accumulators: 4 consecutive columns per lane
          Out::put4(smem, wm * Mma::TM + i * 32 + (lane & 31), wn * Mma::TN + jj * 32 + Mma::acc_col(g, lane),
                    mma.acc[i][jj][4 * g], mma.acc[i][jj][4 * g + 1], mma.acc[i][jj][4 * g + 2],
                    mma.acc[i][jj][4 * g + 3]);
    Out::flush(smem, BM, out, a.n2);
  }
}


__device__ __attribute__((aligned(256))) bf16 g_wgrad_zero_row[256];  // never written: all zeros

// Deep-K weight gradient, register-staged (experts averaging more than
// kRegWgradRows rows): 4 waves of 128 x 128 (one per SIMD, accumulators in
// the AGPRs) over 256 x 256 output tiles, 64-row K steps, with the tile
// schedule of grouped_wgrad_kernel. Each stage's 16-byte vectors are loaded
// into VGPRs two stages ahead and written to a 2-deep LDS ring during the
// MFMAs of the stage before, as in the row GEMM's register-staged loop; all
// copies are ordinary loads, so the compiler's own wait counts cover them.
// Wave w copies the stage's K rows 16w .. 16w + 15 (two per 1 KiB chunk);
// the row ids of a gathered operand arrive one stage earlier, one load per
// wave (lanes 0..15), and are broadcast with readlane. P rows past the
// expert's end are read from a zero row (their products vanish), Q rows
// there from a clamped real row, so the loop body has no branch. The
// epilogue stages the tile in the (then idle) ring, XOR-swizzled, and stores
// 2 rows x 512 B per instruction.
template <int NT = 256>
__global__ __launch_bounds__(NT) void wgrad_reg_kernel(WgradArgs a, int num_experts, int per_xcd) {
  constexpr int BM = 256, BN = 256, BK_ = 64, WN = 2, WM = NT / 64 / WN;
  using Mma = MmaTile<BM, BN, WM, WN>;
  using PTile = MnTile<BM, BK_, NT>;
  using QTile = MnTile<BN, BK_, NT>;
  static_assert(NT == 256 && Mma::TM == 128 && Mma::TN == 128, "4 waves of 128 x 128");
  constexpr int STAGE = PTile::ELEMS + QTile::ELEMS;
  constexpr int PW = PTile::PER_WAVE;  // 1 KiB chunks per wave per operand per stage (8)
  constexpr int KPC = PTile::KPC;      // K rows per chunk (2)
  constexpr int RPW = PW * KPC;        // K rows per wave per stage (16)
  static_assert(PW == QTile::PER_WAVE && KPC == QTile::KPC && RPW * (NT / 64) == BK_, "copy split");
  __shared__ __attribute__((aligned(1024))) bf16 smem[2 * STAGE];
  static_assert(BM * BN <= 2 * STAGE, "epilogue staging fits the ring");

  const int t1n = a.n1 / BM, t2n = a.n2 / BN;
  const int per_e = t1n * t2n;
  const int x = blockIdx.x % kXcds, j = blockIdx.x / kXcds;
  const int e = j / per_xcd;
  const int t = x * per_xcd + (j - e * per_xcd);
  if (e >= num_experts || t >= per_e) return;
  int t1, t2;
  grouped_mn(t, t1n, t2n, t1, t2);
  const int r0 = min(a.offsets[e], a.rows_cap), r1 = min(a.offsets[e + 1], a.rows_cap);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int64_t pc = static_cast<int64_t>(t1) * BM, qc = static_cast<int64_t>(t2) * BN;
  const int nk = (r1 - r0 + BK_ - 1) / BK_;
  const int cap1 = a.rows_cap > 0 ? a.rows_cap - 1 : 0;
  const int half = lane >> 5;   // which row of its chunk the lane copies
  const int lcol = lane & 31;   // 16-byte slot of that row

  // row ids of this wave's RPW rows of stage s (lane l holds row l % RPW);
  // without a gather the load reads offsets[0] and its value is unused
  auto load_ids = [&](const int32_t* rows, int s) -> int {
    const int r = min(r0 + s * BK_ + wave * RPW + (lane & (RPW - 1)), cap1);
    return *(rows ? rows + r : a.offsets);
  };
  auto src = [&](const bf16* base, int64_t ld, const int32_t* rows, int ids, int s, int v, int64_t col0,
                 bool zero_tail) {
    const int kl = wave * RPW + v * KPC + half;  // K row within the stage
    const int kg = r0 + s * BK_ + kl;            // row of the expert-major order
    const int lo = __builtin_amdgcn_readlane(ids, v * KPC), hi = __builtin_amdgcn_readlane(ids, v * KPC + 1);
    const int row = rows ? (half ? hi : lo) : min(kg, cap1);
    const int c = (lcol ^ mn_swz(kl)) * 8;
    const uint64_t data = reinterpret_cast<uint64_t>(base + static_cast<int64_t>(row) * ld + col0 + c);
    const uint64_t zero = reinterpret_cast<uint64_t>(g_wgrad_zero_row + c);
    const uint64_t addr = (zero_tail && kg >= r1) ? zero : data;
    return *reinterpret_cast<const u32x4_t*>(addr);
  };
  u32x4_t ra[PW], rb[PW];
  int pid_cur = 0, qid_cur = 0, pid_nxt = 0, qid_nxt = 0;
  auto gload_p = [&](int s) {
#pragma unroll
    for (int v = 0; v < PW; ++v) ra[v] = src(a.p, a.ldp, a.p_rows, pid_cur, s, v, pc, true);
  };
  auto gload_q = [&](int s) {
#pragma unroll
    for (int v = 0; v < PW; ++v) rb[v] = src(a.q, a.ldq, a.q_rows, qid_cur, s, v, qc, false);
  };
  // chunk v of wave w sits at LDS chunk w * PW + v (rows 2 (w PW + v) + 0/1)
  auto put = [&](bf16* buf, const u32x4_t (&r)[PW]) {
#pragma unroll
    for (int v = 0; v < PW; ++v) *reinterpret_cast<u32x4_t*>(buf + (wave * PW + v) * kChunkElems + lane * 8) = r[v];
  };

  Mma mma;
  mma.zero();
  using Frag = bf16x8;
  Frag fa[2][Mma::MI], fb[2][Mma::NI];
  if (nk > 0) {
    pid_cur = load_ids(a.p_rows, 0);
    qid_cur = load_ids(a.q_rows, 0);
    gload_p(0);
    gload_q(0);
    put(smem, ra);
    put(smem + PTile::ELEMS, rb);
    if (nk > 1) {
      pid_cur = load_ids(a.p_rows, 1);
      qid_cur = load_ids(a.q_rows, 1);
      gload_p(1);
      gload_q(1);
      if (nk > 2) {
        pid_nxt = load_ids(a.p_rows, 2);
        qid_nxt = load_ids(a.q_rows, 2);
      }
    }
  }
  __syncthreads();
  if (nk > 0) {
    Mma::template frags<PTile, QTile, BK_>(fa[0], fb[0], smem, smem + PTile::ELEMS, wm, wn, 0, lane);
    // sub-step ss issues its MFMAs from fragment set ss & 1 while the next
    // sub-step's fragments load; stage kt + 1's registers go to LDS during
    // sub-steps 0 (P) and 1 (Q), then stage kt + 2's loads issue (its row
    // ids were loaded one stage before; stage kt + 3's go out with them);
    // the barrier after sub-step 2 publishes stage kt + 1. Past the last
    // stage the loads repeat it and the writes land in a slot nobody reads.
    for (int kt = 0; kt < nk; ++kt) {
      const bf16* cur = smem + (kt & 1) * STAGE;
      bf16* nxt = smem + ((kt + 1) & 1) * STAGE;
      const int s2 = min(kt + 2, nk - 1);
#pragma unroll
      for (int ss = 0; ss < 4; ++ss) {
        const int c = ss & 1, n = c ^ 1;
        if (ss < 3)
          Mma::template frags<PTile, QTile, BK_>(fa[n], fb[n], cur, cur + PTile::ELEMS, wm, wn, (ss + 1) * 16, lane);
        else
          Mma::template frags<PTile, QTile, BK_>(fa[n], fb[n], nxt, nxt + PTile::ELEMS, wm, wn, 0, lane);
        mma.mfmas_t(fa[c], fb[c]);
        if (ss == 0) {
          put(nxt, ra);
          pid_cur = pid_nxt;
          qid_cur = qid_nxt;
          gload_p(s2);
        }
        if (ss == 1) {
          put(nxt + PTile::ELEMS, rb);
          gload_q(s2);
          pid_nxt = load_ids(a.p_rows, min(kt + 3, nk - 1));
          qid_nxt = load_ids(a.q_rows, min(kt + 3, nk - 1));
        }
#pragma unroll
        for (int q = 0; q < Mma::MI * Mma::NI; ++q) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
          __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // LDS write
          __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // global load
        }
        if (ss == 2) __syncthreads();
      }
    }
  }
  __syncthreads();
  // epilogue: transposed accumulators (lane: row lane % 32 of block i, 4
  // consecutive columns); 16-byte slot v of tile row r at v ^ (r & 31)
  constexpr int VPR = BN / 8;
#pragma unroll
  for (int i = 0; i < Mma::MI; ++i)
#pragma unroll
    for (int jj = 0; jj < Mma::NI; ++jj)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int tr = wm * Mma::TM + i * 32 + (lane & 31);
        const int tc = wn * Mma::TN + jj * 32 + Mma::acc_col(g, lane);
        *reinterpret_cast<uint2*>(smem + tr * BN + ((((tc >> 3) ^ (tr & 31)) << 3) | (tc & 7))) =
            make_uint2(pack_bf16x2(mma.acc[i][jj][4 * g], mma.acc[i][jj][4 * g + 1]),
                       pack_bf16x2(mma.acc[i][jj][4 * g + 2], mma.acc[i][jj][4 * g + 3]));
      }
  __syncthreads();
  bf16* out = a.c + static_cast<int64_t>(e) * a.n1 * a.n2 + pc * a.n2 + qc;
#pragma unroll 4
  for (int idx = threadIdx.x; idx < BM * VPR; idx += NT) {
    const int r = idx / VPR, cv = idx % VPR;
    store_out16(out + static_cast<int64_t>(r) * a.n2 + cv * 8,
                *reinterpret_cast<const uint4*>(smem + r * BN + ((cv ^ (r & 31)) << 3)));
  }
}

// ------------------------------------------------------------------ small-K wgrad
//
// Weight gradient when experts hold few rows (K of the GEMM; e.g. 73 rows
// per expert at 4096 tokens, top-16 over 896 experts): the E x n1 x n2 bf16
// output write dominates.

// wait until at most n (rounded down to a multiple of STEP) vector-memory
// ops of this wave are outstanding; n is wave-uniform
template <int MAXN, int STEP>
__device__ __forceinline__ void wait_vmcnt_atmost(int n) {
  if constexpr (MAXN > 0) {
    if (n >= MAXN) {
      wait_vmcnt<MAXN>();
      return;
    }
    wait_vmcnt_atmost<MAXN - STEP, STEP>(n);
  } else {
    wait_vmcnt<0>();
  }
}

// Small-K weight gradient; gathered operands are read in place (the row ids
// of each stage come from scalar loads).
//  * Persistent: one 8-wave workgroup per CU walks a sequence of (expert,
//    256 x 256 output tile, 32-row K step) stages through an NST-deep LDS
//    ring, so the first stages of the next tile are in flight while the
//    current tile is staged and stored. Each XCD (workgroup ids congruent
//    mod 8) owns a fixed subset of the experts: every expert writes the same
//    n1 x n2 output whatever its row count, so this is balanced, and an
//    expert's rows are read into that XCD's L2 once. A team of the XCD's
//    workgroups takes every nc-th tile of its expert.
//  * The product is formed transposed, C^T = Q^T P, so each lane's
//    accumulator holds 4 consecutive output columns of one output row; every
//    wave stages its 64 x 128 sub-tile 64 columns at a time in a private LDS
//    slice with 8-byte writes and writes it back as full 128-byte row
//    segments with non-temporal 16-byte stores. The staging is separate from
//    the ring and wave-private, so tiles need no barrier of their own.
//  * Rows past the expert's end are copied from a zero row, so the K loop
//    has no tail fix-up; a stage holding <= 16 valid rows runs one 16-row
//    MFMA step instead of two.
//  * Every wave issues the same vector-memory ops (LPS copies per stage, SPT
//    stores per tile), and they complete in issue order, so each stage wait
//    counts exactly the ops issued after that stage.
struct TileCursor {
  int e, t, ks, nk, kr, r0;
  int estep;  // experts between this cursor's consecutive experts
  bool valid;
  // offsets[e], offsets[e + 1] come from one scalar load: the compiler emits
  // a vector load for them otherwise and follows it with vmcnt(0), which
  // drains every in-flight stage copy and tile store at each new expert
  __device__ void load_expert(const int32_t* offsets, int rows_cap) {
    const int2 o = scalar_load_i32x2(offsets + __builtin_amdgcn_readfirstlane(e));
    r0 = min(o.x, rows_cap);
    kr = min(o.y, rows_cap) - r0;
    nk = kr > 0 ? (kr + 31) / 32 : 1;  // an expert without rows still writes its zero tiles
  }
  __device__ void skip_empty(int c, int per_e, int E, const int32_t* offsets, int rows_cap) {
    while (valid && t >= per_e) {
      e += estep;
      t = c;
      valid = e < E;
    }
    if (valid) load_expert(offsets, rows_cap);
  }
  __device__ void init(int x, int step, int c, int per_e, int E, const int32_t* offsets, int rows_cap) {
    e = x;
    estep = step;
    t = c;
    ks = 0;
    valid = e < E;
    skip_empty(c, per_e, E, offsets, rows_cap);
  }
  __device__ void advance(int c, int nc, int per_e, int E, const int32_t* offsets, int rows_cap) {
    if (++ks < nk) return;
    ks = 0;
    t += nc;
    if (t >= per_e) skip_empty(c, per_e, E, offsets, rows_cap);
  }
};

template <int NST>
__global__ __launch_bounds__(512) void wgrad_persist_kernel(WgradArgs a, int num_experts) {
  constexpr int BM = 256, BN = 256, BKS = 32, WM = 2, WN = 4, NT = WM * WN * 64;
  using PTile = MnTile<BM, BKS, NT>;
  using QTile = MnTile<BN, BKS, NT>;
  using Mma = MmaTile<BN, BM, WM, WN>;  // transposed: MFMA rows = n2, columns = n1
  static_assert(Mma::TN == 64 && Mma::TM == 128, "wave sub-tile is 64 x 128");
  constexpr int HALVES = Mma::TM / 64;
  constexpr int STAGE = PTile::ELEMS + QTile::ELEMS;
  constexpr int LPS = PTile::PER_WAVE + QTile::PER_WAVE;  // copies per wave per stage
  constexpr int SUB = 64 * Mma::TN;                       // staging elements per wave
  constexpr int SPT = HALVES * SUB / 8 / 64;              // stores per lane per tile
  __shared__ __attribute__((aligned(1024))) bf16 smem[NST * STAGE + (NT / 64) * SUB];
  // Each XCD's workgroups form two teams (one if their count is odd), each
  // walking its own expert: team q of XCD x0 takes experts x0 + 8q,
  // x0 + 8q + 8 * teams, ... (16 workgroups per expert measured 2% faster
  // than 32 on the Kimi-scale gradients, and 4 teams no faster than 2).
  const int per_xcd = gridDim.x / kXcds;
  const int teams = per_xcd % 2 == 0 ? 2 : 1;
  const int team = (blockIdx.x / kXcds) % teams;
  const int x = blockIdx.x % kXcds + team * kXcds, c = blockIdx.x / kXcds / teams, nc = per_xcd / teams;
  const int t1n = a.n1 / BM, t2n = a.n2 / BN;
  const int per_e = t1n * t2n;
  // Tile t of an expert -> (t1, t2): the dimension with more tiles varies
  // fastest, so the workgroups of an XCD write tiles spread along it and
  // share the operand block of the other dimension. Measured on the
  // Kimi-scale gradients against the other order: dW1 (28 x 16 tiles)
  // 11.4 -> 10.3 ms, dW2 (28 x 8) 5.55 -> 5.3 ms; a transposed 8 x 28 shape
  // runs 4.8 ms in this order and 6.3 ms in the other.
  const bool t1_fast = t1n >= t2n;
  auto tile_of = [&](int t, int& t1, int& t2) {
    if (t1_fast) {
      t1 = t % t1n;
      t2 = t / t1n;
    } else {
      t1 = t / t2n;
      t2 = t % t2n;
    }
  };
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;
  bf16* stage_out = smem + NST * STAGE + wave * SUB;

  TileCursor cc, lc;  // consumer; copier (NST - 1 stages ahead)
  cc.init(x, kXcds * teams, c, per_e, num_experts, a.offsets, a.rows_cap);
  lc = cc;
  // Gathered operands: instruction v of this wave copies the stage's K rows
  // k0(v) .. k0(v) + KPC - 1 (k0 wave-uniform), so their row ids come from
  // scalar loads and each lane picks its own. The ids of a stage are loaded
  // as soon as the copier's cursor reaches it, one stage before its copies
  // are issued, so the loads are in flight meanwhile. Rows past the
  // expert's end are read from a zero row.
  constexpr int KPC = PTile::KPC;
  static_assert(PTile::KPC == QTile::KPC && PTile::PER_WAVE == QTile::PER_WAVE, "one K-row split for both operands");
  constexpr int PW = PTile::PER_WAVE;
  const int cap1 = a.rows_cap > 0 ? a.rows_cap - 1 : 0;
  int pid[PW][KPC] = {}, qid[PW][KPC] = {};
  auto load_ids = [&](const TileCursor& q) {
    const int rbase = q.r0 + q.ks * BKS;
    if (a.p_rows) {
#pragma unroll
      for (int v = 0; v < PW; ++v)
#pragma unroll
        for (int j = 0; j < KPC; ++j)
          pid[v][j] = *(const const_i32*)(a.p_rows + min(rbase + (v * (NT / 64) + wave) * KPC + j, cap1));
    }
    if (a.q_rows) {
#pragma unroll
      for (int v = 0; v < PW; ++v)
#pragma unroll
        for (int j = 0; j < KPC; ++j)
          qid[v][j] = *(const const_i32*)(a.q_rows + min(rbase + (v * (NT / 64) + wave) * KPC + j, cap1));
    }
  };
  // The zero row's address is read once (a load through the GOT would
  // otherwise be repeated, with its wait, at every stage), and each copy's
  // address is chosen with a bitwise select: with a conditional expression
  // the compiler branched around the address arithmetic of every copy.
  uint64_t zrow = reinterpret_cast<uint64_t>(g_wgrad_zero_row);
  asm volatile("" : "+s"(zrow));
  auto row_src = [&](const bf16* base, int64_t ld, bool gathered, const int (&id)[KPC], int rbase, int kv, int k0,
                     int k, int64_t col) -> const bf16* {
    int r = rbase + k;
    if (gathered) {
      int pick = id[0];
#pragma unroll
      for (int j = 1; j < KPC; ++j) pick = (k - k0 == j) ? id[j] : pick;
      r = pick;
    }
    // row offsets fit 32 x 32 bits (ld < 2^32 is checked on the host)
    const uint64_t d = reinterpret_cast<uint64_t>(base + col) +
                       2ull * (static_cast<uint64_t>(static_cast<uint32_t>(r)) * static_cast<uint32_t>(ld));
    const uint64_t m = 0ull - static_cast<uint64_t>(k >= kv);
    return reinterpret_cast<const bf16*>(d ^ ((d ^ zrow) & m));
  };
  auto issue = [&](const TileCursor& q, int buf) {
    bf16* dst = smem + buf * STAGE;
    int t1, t2;
    tile_of(q.t, t1, t2);
    const int kb = q.ks * BKS;
    const int rbase = q.r0 + kb;
    const int kv = q.kr - kb;
    PTile::issue_rows(dst, [&](int v) {
      return row_src(a.p, a.ldp, a.p_rows != nullptr, pid[v], rbase, kv, (v * (NT / 64) + wave) * KPC,
                     PTile::k_of(v), static_cast<int64_t>(t1) * BM);
    });
    QTile::issue_rows(dst + PTile::ELEMS, [&](int v) {
      return row_src(a.q, a.ldq, a.q_rows != nullptr, qid[v], rbase, kv, (v * (NT / 64) + wave) * KPC,
                     QTile::k_of(v), static_cast<int64_t>(t2) * BN);
    });
  };

  // vector-memory ops issued by this wave so far, and the count right after
  // each in-flight stage's copies (ring slot st % NST)
  int issued_ops = 0;
  int stage_mark[NST];
#pragma unroll
  for (int i = 0; i < NST; ++i) stage_mark[i] = 0;
  int nissued = 0;
  if (lc.valid) load_ids(lc);
  for (; nissued < NST - 1 && lc.valid; ++nissued) {
    issue(lc, nissued % NST);
    issued_ops += LPS;
#pragma unroll
    for (int i = 0; i < NST; ++i)
      if (i == nissued % NST) stage_mark[i] = issued_ops;
    lc.advance(c, nc, per_e, num_experts, a.offsets, a.rows_cap);
    if (lc.valid) load_ids(lc);
  }
  Mma mma;
  mma.zero();
  for (int st = 0; cc.valid; ++st) {
    int mark = 0;
#pragma unroll
    for (int i = 0; i < NST; ++i)
      if (i == st % NST) mark = stage_mark[i];
    wait_vmcnt_atmost<(NST - 2) * LPS + (NST - 1) * SPT, 4>(issued_ops - mark);
    __syncthreads();  // stage st landed; stage st - 1 consumed by every wave
    if (lc.valid) {
      issue(lc, nissued % NST);
      issued_ops += LPS;
#pragma unroll
      for (int i = 0; i < NST; ++i)
        if (i == nissued % NST) stage_mark[i] = issued_ops;
      lc.advance(c, nc, per_e, num_experts, a.offsets, a.rows_cap);
      if (lc.valid) load_ids(lc);
      ++nissued;
    }
    const bf16* pb = smem + (st % NST) * STAGE;
    const int kv = cc.kr - cc.ks * BKS;
    const int nsub = kv > 16 ? 2 : 1;  // a stage with <= 16 valid rows runs one 16-row step
    for (int ss = 0; ss < nsub; ++ss)
      mma.template compute<QTile, PTile, 16>(pb + PTile::ELEMS + ss * 16 * BN, pb + ss * 16 * BM, wm, wn, lane);
    if (cc.ks == cc.nk - 1) {
      int t1, t2;
      tile_of(cc.t, t1, t2);
      bf16* out = a.c + static_cast<int64_t>(cc.e) * a.n1 * a.n2 +
                  static_cast<int64_t>(t1 * BM + wn * Mma::TN) * a.n2 + t2 * BN + wm * Mma::TM;
#pragma unroll
      for (int h = 0; h < HALVES; ++h) {
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
#pragma unroll
          for (int j = 0; j < Mma::NI; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              const int i = 2 * h + ii;
              const int r = j * 32 + (lane & 31);
              const int v = ii * 4 + g;
              const uint32_t lo = pack_bf16x2(mma.acc[i][j][4 * g], mma.acc[i][j][4 * g + 1]);
              const uint32_t hi = pack_bf16x2(mma.acc[i][j][4 * g + 2], mma.acc[i][j][4 * g + 3]);
              *reinterpret_cast<uint2*>(stage_out + r * 64 + ((v ^ (r & 7)) << 3) + (lane >> 5) * 4) =
                  make_uint2(lo, hi);
            }
#pragma unroll
        for (int it = 0; it < SUB / 8 / 64; ++it) {
          const int r = it * 8 + (lane >> 3), cv = lane & 7;
          store_out16(out + static_cast<int64_t>(r) * a.n2 + h * 64 + cv * 8,
                      *reinterpret_cast<const uint4*>(stage_out + r * 64 + ((cv ^ (r & 7)) << 3)));
        }
      }
      issued_ops += SPT;
      mma.zero();
    }
    cc.advance(c, nc, per_e, num_experts, a.offsets, a.rows_cap);
  }
}

// ------------------------------------------------------------------ host side
constexpr int kMinBM = 128;  // smallest M tile: sizes the tile list

int64_t max_m_tiles(int64_t max_rows, int E, int BM) { return (max_rows + BM - 1) / BM + E; }

size_t tile_list_bytes(int64_t max_rows, int E) {
  return mm_align_up(sizeof(TileList) + sizeof(int4) * static_cast<size_t>(max_m_tiles(max_rows, E, kMinBM)), 256);
}

int launch_tiles(const int32_t* offsets, int E, int BM, void* ws, hipStream_t s) {
  build_tiles_kernel<<<1, 1024, 0, s>>>(offsets, E, BM, static_cast<TileList*>(ws));
  return mm_check_launch("build_tiles");
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Row-GEMM tile choice: 256x256 when experts average at least 96 rows,
// else a 128-row tile; 256-wide N tiles when N allows. With 129-255 rows per
// expert one 256-row tile covers an expert, so its weights stream once (two
// 128-row tiles read them twice: Kimi-scale layer at 8192 tokens, 146 rows
// per expert, 72.2 -> 63.0 ms per fwd+bwd step). From an average of 96 rows
// per expert on, softmax top-k routing puts about half the experts above 128
// rows, so the 256-row tile already pays (E=256 top-8 at 4096 tokens, 128
// rows per expert on average: 17.5 -> 16.4 ms per step); below that (Kimi at
// 4096 tokens, 73 rows) it loses to the 128-row tile (43 -> 48 ms at a
// threshold of 64).
struct RowsCfg {
  int bm, bn;
};

RowsCfg pick_rows_cfg(int64_t max_rows, int E, int n) {
  RowsCfg c;
  c.bn = (n % 256 == 0) ? 256 : 128;
  c.bm = (c.bn == 256 && max_rows >= 96 * static_cast<int64_t>(E)) ? 256 : 128;
  return c;
}

template <int BM, int BN, int BK_, int NST, int BLAYOUT, int EPI, int NT = kThreads, bool REG = false, int BPOL = 0>
void launch_rows_cfg(const RowsArgs& p, int64_t max_rows, int E, hipStream_t s) {
  const int64_t mm = max_m_tiles(max_rows, E, BM);
  const int64_t g = p.xcd_mod ? (mm + kXcds - 1) / kXcds * kXcds * (p.n / BN) : mm * (p.n / BN);
  const int grid = static_cast<int>((g + kXcds - 1) / kXcds * kXcds);
  if constexpr (EPI == EPI_GATED) {  // activation specialised at compile time
    if (p.act_kind == MM_ACT_SWIGLU)
      grouped_rows_kernel<BM, BN, BK_, NST, BLAYOUT, EPI, NT, MM_ACT_SWIGLU, REG><<<grid, NT, 0, s>>>(p);
    else if (p.act_kind == MM_ACT_CLAMP_SWIGLU)
      grouped_rows_kernel<BM, BN, BK_, NST, BLAYOUT, EPI, NT, MM_ACT_CLAMP_SWIGLU, REG><<<grid, NT, 0, s>>>(p);
    else
      grouped_rows_kernel<BM, BN, BK_, NST, BLAYOUT, EPI, NT, MM_ACT_SITUGLU, REG><<<grid, NT, 0, s>>>(p);
  } else {
    grouped_rows_kernel<BM, BN, BK_, NST, BLAYOUT, EPI, NT, 0, REG, BPOL><<<grid, NT, 0, s>>>(p);
  }
}

// 8 waves (2 per SIMD) per 128x256 workgroup by default: a second wave on
// each SIMD keeps the matrix core busy across the other's LDS waits and
// barriers (-7% time on the 128-row tiles of small experts against 4
// waves). MM_GEMM_WAVES=4 selects 4 waves.
int eight_waves() {
  const char* e = getenv("MM_GEMM_WAVES");  // read on every call
  return (e && strcmp(e, "4") == 0) ? 0 : 1;
}

// 256x256 row tiles with K >= 1024: 4 waves of 128x128 with register-staged
// operand copies (one wave per SIMD, 2/3 of the LDS fragment traffic of 8
// waves of 64x128; the next stage's LDS writes and the following stage's
// global loads interleaved with the MFMAs): E32 and Skew layer steps -3%,
// the K-contiguous dgrads -4 to -7%, against 8 waves with LDS-DMA copies,
// which run the shorter K loops (Qwen-like FC2, K = 768: 0.271 against
// 0.280 ms) and which MM_ROWS_DMA=1 selects everywhere.
bool rows_lds_dma() {
  const char* e = getenv("MM_ROWS_DMA");  // read on every call
  return e && strcmp(e, "1") == 0;
}

// Non-temporal weight copies in the 128-row row-GEMM tiles unless
// MM_WEIGHT_NT=0 (read on every call).
bool weight_nt() {
  const char* e = getenv("MM_WEIGHT_NT");
  return !(e && strcmp(e, "0") == 0);
}

enum { WG_WIDE = 0, WG_TILE = 1, WG_LARGE = 2 };

constexpr int kWideStages = 3;  // LDS: 3 x 32 KiB ring + 64 KiB staging = 160 KiB

// Compute units of the current device (cached per device).
int device_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

// The persistent small-K weight gradient is bound by writing the gradient
// while the K loop is short: kept up to 192 rows per expert on average
// (Kimi-scale 8192 tokens, 146 rows: FC1 wgrad 16.3 -> 15.7 ms against the
// deep-K kernel; 16384 tokens, 292 rows: deep-K 22.9 against 24.7 ms).
constexpr int64_t kSmallKRows = 192;

// Deep-K 256 x 256 weight gradient: the register-staged 4-wave kernel when
// experts average more than kRegWgradRows rows (Skew-like layer, 4096 rows
// per expert: dW1 3.47 -> 3.31 ms, dW2 1.99 -> 1.92 ms against 8 waves with
// LDS-DMA copies); below that the 8-wave kernel's second wave per SIMD
// hides the per-tile prologue and epilogue better (Qwen-like, 512 rows:
// dW1 0.585 against 0.62 ms). MM_WGRAD_REG=0 / 1 forces the choice.
constexpr int64_t kRegWgradRows = 2048;
bool wgrad_reg(int64_t max_rows, int E) {
  if (const char* e = getenv("MM_WGRAD_REG")) {
    if (strcmp(e, "0") == 0) return false;
    if (strcmp(e, "1") == 0) return true;
  }
  return max_rows > kRegWgradRows * static_cast<int64_t>(E);
}
bool wgrad_small_k(int64_t max_rows, int E) { return max_rows <= kSmallKRows * static_cast<int64_t>(E); }

template <int BLAYOUT, int EPI>
int run_rows(RowsArgs p, const int32_t* offsets, int64_t max_rows, int E, void* ws, hipStream_t s,
             const char* what) {
  const RowsCfg c = pick_rows_cfg(max_rows, E, p.n);
  // the largest grid any tile configuration launches (128-row M tiles padded
  // to a multiple of 8, 128-wide N tiles) must fit a 32-bit grid size
  if ((max_m_tiles(max_rows, E, 128) + kXcds - 1) / kXcds * kXcds * (p.n / 128) >= (int64_t(1) << 31)) {
    mm_set_error("%s: too many tiles for one launch", what);
    return MM_E_ARG;
  }
  if (int rc = launch_tiles(offsets, E, c.bm, ws, s)) return rc;
  p.tl = static_cast<const TileList*>(ws);
  // 128-row tiles (experts averaging < 256 rows, weight-streaming): one
  // expert's N tiles run together, so its gathered A panel stays in L2
  // (Kimi-scale: -5% layer time against 8-deep groups)
  p.group_m = c.bm == 128 ? 1 : GROUP_M;
  // 128-row tiles stream the weights: M tile m runs on XCD m % 8, so every
  // XCD reads experts spread over the whole weight tensor instead of one
  // contiguous eighth of it. Where the weights' placement made one part of
  // the tensor slower to read, the contiguous split left some XCDs finishing
  // late (per-workgroup clocks: XCDs 5-7 at 83-85 us per FC1-dgrad tile,
  // 0-4 at 91-92 us); Kimi-scale layer, five processes, one-process A/B:
  // -0.84, -0.34, -0.26, +0.03, +0.04 ms per step; alternating bench
  // processes on a sixth box: -0.32, -0.34, -0.18 ms. MM_XCD_MOD=0 restores
  // the contiguous split (read on every call).
  if (c.bm == 128) {
    const char* e = getenv("MM_XCD_MOD");
    p.xcd_mod = !(e && strcmp(e, "0") == 0);
  }
  if (c.bm == 256) {
    if (rows_lds_dma() || p.k < 1024)
      launch_rows_cfg<256, 256, 64, 2, BLAYOUT, EPI, 512>(p, max_rows, E, s);
    else
      launch_rows_cfg<256, 256, 64, 2, BLAYOUT, EPI, 256, true>(p, max_rows, E, s);
  } else if (c.bn == 256) {
    // Weight streaming with N-contiguous weights (FC1, FC2 of small
    // experts): 512-wide tiles halve the tile count and with it the per-tile
    // prologue / epilogue (Kimi-scale FC1 -6%, FC2 -10%; neutral to +2% for
    // the K-contiguous dgrads, which keep 256). BK 32 x 4 stages (4 x 40 KiB)
    // keeps three stages of weight in flight per CU instead of one 80 KiB
    // stage (Kimi-scale FC1 -4%, FC2 -6% against BK 64 x 2).
    // The K-contiguous weight tiles of the 128-row dgrads are read once, so
    // their LDS-DMA copies carry the non-temporal hint and do not displace
    // the activation panel that every N tile of an expert reuses from L2
    // (Kimi-scale layer, one process: FC2 dgrad 4.32 -> 4.13 ms, FC1 dgrad
    // 9.56 -> 8.96 ms; MM_WEIGHT_NT=0 drops it). For the N-contiguous FC1 /
    // FC2 weights it is neutral in isolation and 2.5% slower in the layer.
    const bool wnt = BLAYOUT == B_KCONTIG && weight_nt();
    bool wide = false;
    if constexpr (BLAYOUT == B_NCONTIG) {
      wide = p.n % 512 == 0;
      if (wide) launch_rows_cfg<128, 512, 32, 4, BLAYOUT, EPI, 512>(p, max_rows, E, s);
    }
    if (!wide) {
      // 8 waves: 32-row wave slabs, so rows past a small expert's count skip more MFMAs
      if (eight_waves()) {
        if (wnt)
          launch_rows_cfg<128, 256, 64, 3, BLAYOUT, EPI, 512, false, 1>(p, max_rows, E, s);
        else
          launch_rows_cfg<128, 256, 64, 3, BLAYOUT, EPI, 512>(p, max_rows, E, s);
      } else {
        launch_rows_cfg<128, 256, 64, 3, BLAYOUT, EPI>(p, max_rows, E, s);
      }
    }
  } else {
    launch_rows_cfg<128, 128, 64, 4, BLAYOUT, EPI>(p, max_rows, E, s);
  }
  return mm_check_launch(what);
}

}  // namespace

extern "C" size_t mm_gemm_workspace_bytes(int64_t max_rows, int32_t num_experts) {
  return tile_list_bytes(max_rows, num_experts);
}

extern "C" int mm_fc1_swiglu(const uint16_t* x, int64_t ldx, const int32_t* send_token, const uint16_t* w1,
                             const int32_t* offsets, const float* weight_perm, int32_t num_experts,
                             int64_t max_rows, int32_t hidden, int32_t inter, int32_t act_kind, float situ_beta,
                             float situ_linear_beta, float clamp_limit, uint16_t* act, void* fc1_out,
                             int32_t fc1_format, float* fc1_scale, void* workspace, size_t workspace_bytes,
                             mm_stream_t stream) {
  MM_CHECK_ARG(x && w1 && offsets && weight_perm && act, "mm_fc1_swiglu: null pointer");
  MM_CHECK_ARG(num_experts > 0 && max_rows >= 0 && max_rows < (int64_t(1) << 31), "mm_fc1_swiglu: bad sizes");
  MM_CHECK_ARG(hidden > 0 && hidden % BK == 0, "mm_fc1_swiglu: hidden must be a multiple of %d", BK);
  MM_CHECK_ARG(inter > 0 && inter % 64 == 0, "mm_fc1_swiglu: inter must be a multiple of 64");
  MM_CHECK_ARG(ldx % 8 == 0 && al16(x) && al16(w1), "mm_fc1_swiglu: 16-byte alignment required");
  MM_CHECK_ARG(act_kind >= 0 && act_kind <= 2, "mm_fc1_swiglu: bad act_kind");
  MM_CHECK_ARG(fc1_format >= MM_FC1_BF16 && fc1_format <= MM_FC1_FP8, "mm_fc1_swiglu: bad fc1_format");
  MM_CHECK_ARG(!fc1_out || fc1_format != MM_FC1_FP8 || (fc1_scale && inter % MM_FC1_SCALE_GROUP == 0),
               "mm_fc1_swiglu: FP8 fc1_out needs fc1_scale and inter %% %d == 0", MM_FC1_SCALE_GROUP);
  MM_CHECK_ARG(!fc1_out || (reinterpret_cast<uintptr_t>(fc1_out) & 7u) == 0, "mm_fc1_swiglu: fc1_out alignment");
  if (!workspace || workspace_bytes < tile_list_bytes(max_rows, num_experts)) {
    mm_set_error("mm_fc1_swiglu: workspace too small");
    return MM_E_WS;
  }
  if (max_rows == 0) return MM_OK;
  RowsArgs p{};
  p.a = reinterpret_cast<const bf16*>(x);
  p.lda = ldx;
  p.a_rows = send_token;
  p.b = reinterpret_cast<const bf16*>(w1);
  p.b_se = static_cast<int64_t>(hidden) * 2 * inter;
  p.b_sn = 1;
  p.b_sk = 2 * static_cast<int64_t>(inter);
  p.n = 2 * inter;
  p.k = hidden;
  p.c = reinterpret_cast<bf16*>(act);
  p.ldc = inter;
  p.w = weight_perm;
  p.fc1_out = fc1_out;
  p.fc1_fmt = fc1_format;
  p.fc1_scale = fc1_scale;
  p.inter = inter;
  p.act_kind = act_kind;
  p.beta = situ_beta;
  p.lbeta = situ_linear_beta;
  p.clamp = clamp_limit;
  return run_rows<B_NCONTIG, EPI_GATED>(p, offsets, max_rows, num_experts, workspace, mm_hip_stream(stream),
                                        "mm_fc1_swiglu");
}

extern "C" int mm_grouped_gemm(const uint16_t* a, int64_t lda, const int32_t* a_rows, const uint16_t* b,
                               int64_t b_se, int64_t b_sn, int64_t b_sk, const int32_t* offsets,
                               int32_t num_experts, int64_t max_rows, int32_t n, int32_t k, uint16_t* c,
                               int64_t ldc, void* workspace, size_t workspace_bytes, mm_stream_t stream) {
  MM_CHECK_ARG(a && b && offsets && c, "mm_grouped_gemm: null pointer");
  MM_CHECK_ARG(num_experts > 0 && max_rows >= 0 && max_rows < (int64_t(1) << 31), "mm_grouped_gemm: bad sizes");
  MM_CHECK_ARG(n > 0 && n % 128 == 0, "mm_grouped_gemm: n must be a multiple of 128");
  MM_CHECK_ARG(k > 0 && k % BK == 0, "mm_grouped_gemm: k must be a multiple of %d", BK);
  MM_CHECK_ARG(b_sn == 1 || b_sk == 1, "mm_grouped_gemm: B must be contiguous along N or K");
  MM_CHECK_ARG(lda % 8 == 0 && al16(a) && al16(b) && (b_sn == 1 ? b_sk % 8 == 0 : b_sn % 8 == 0) &&
                   b_se % 8 == 0,
               "mm_grouped_gemm: 16-byte alignment required");
  if (!workspace || workspace_bytes < tile_list_bytes(max_rows, num_experts)) {
    mm_set_error("mm_grouped_gemm: workspace too small");
    return MM_E_WS;
  }
  if (max_rows == 0) return MM_OK;
  RowsArgs p{};
  p.a = reinterpret_cast<const bf16*>(a);
  p.lda = lda;
  p.a_rows = a_rows;
  p.b = reinterpret_cast<const bf16*>(b);
  p.b_se = b_se;
  p.b_sn = b_sn;
  p.b_sk = b_sk;
  p.n = n;
  p.k = k;
  p.c = reinterpret_cast<bf16*>(c);
  p.ldc = ldc;
  hipStream_t s = mm_hip_stream(stream);
  if (b_sk == 1) return run_rows<B_KCONTIG, EPI_STORE>(p, offsets, max_rows, num_experts, workspace, s, "mm_grouped_gemm");
  return run_rows<B_NCONTIG, EPI_STORE>(p, offsets, max_rows, num_experts, workspace, s, "mm_grouped_gemm");
}

// Every weight-gradient kernel gathers its rows in place: no workspace.
extern "C" size_t mm_wgrad_workspace_bytes(int64_t max_rows, int32_t num_experts, int32_t n1, int32_t n2) {
  (void)max_rows;
  (void)num_experts;
  (void)n1;
  (void)n2;
  return 0;
}

extern "C" int mm_grouped_wgrad(const uint16_t* p, int64_t ldp, const int32_t* p_rows, const uint16_t* q,
                                int64_t ldq, const int32_t* q_rows, const int32_t* offsets, int32_t num_experts,
                                int64_t max_rows, int32_t n1, int32_t n2, uint16_t* c, void* workspace,
                                size_t workspace_bytes, mm_stream_t stream) {
  MM_CHECK_ARG(p && q && offsets && c, "mm_grouped_wgrad: null pointer");
  MM_CHECK_ARG(num_experts > 0, "mm_grouped_wgrad: bad num_experts");
  MM_CHECK_ARG(n1 > 0 && n1 % 128 == 0 && n2 > 0 && n2 % 128 == 0, "mm_grouped_wgrad: n1, n2 must be multiples of 128");
  MM_CHECK_ARG(ldp % 8 == 0 && ldq % 8 == 0 && al16(p) && al16(q), "mm_grouped_wgrad: 16-byte alignment required");
  MM_CHECK_ARG(max_rows >= 0 && max_rows < (int64_t(1) << 31), "mm_grouped_wgrad: bad max_rows");
  MM_CHECK_ARG(ldp >= 0 && ldp < (int64_t(1) << 32) && ldq >= 0 && ldq < (int64_t(1) << 32),
               "mm_grouped_wgrad: row strides must be below 2^32 elements");
  WgradArgs a{reinterpret_cast<const bf16*>(p), ldp, p_rows, reinterpret_cast<const bf16*>(q), ldq,
              q_rows, offsets, n1, n2, reinterpret_cast<bf16*>(c), static_cast<int>(max_rows)};
  hipStream_t s = mm_hip_stream(stream);
  // Experts averaging <= 192 rows (K of the wgrad GEMM): the output write
  // dominates -> the persistent 256 x 256-tile kernel when n1, n2 allow
  // (WG_WIDE), else 128 x 128 tiles (WG_TILE); both gather rows in place.
  // Otherwise 256-wide tiles with a deep K loop (WG_LARGE).
  // MM_WGRAD_KERNEL=wide|tile|large overrides the choice (wide falls back
  // to tile where it does not apply).
  int variant = wgrad_small_k(max_rows, num_experts) ? WG_WIDE : WG_LARGE;
  if (const char* ev = getenv("MM_WGRAD_KERNEL")) {
    if (strcmp(ev, "wide") == 0) variant = WG_WIDE;
    else if (strcmp(ev, "tile") == 0) variant = WG_TILE;
    else if (strcmp(ev, "large") == 0) variant = WG_LARGE;
  }
  if (variant == WG_WIDE) {
    if (n1 % 256 != 0 || n2 % 256 != 0) {
      variant = WG_TILE;
    } else {
      if (max_rows == 0) a.p_rows = a.q_rows = nullptr;  // no row is read: every tile is zero
      const int g = device_cus() / kXcds * kXcds;
      wgrad_persist_kernel<kWideStages><<<g > 0 ? g : kXcds, 512, 0, s>>>(a, num_experts);
      return mm_check_launch("mm_grouped_wgrad");
    }
  }
  const bool small = variant == WG_TILE;
  const int bm = (!small && n1 % 256 == 0) ? 256 : 128;
  const int bn = (!small && n2 % 256 == 0) ? 256 : 128;
  const int64_t per_e = static_cast<int64_t>(n1 / bm) * (n2 / bn);
  const int64_t per_xcd = (per_e + kXcds - 1) / kXcds;
  const int64_t grid64 = static_cast<int64_t>(num_experts) * per_xcd * kXcds;
  MM_CHECK_ARG(grid64 < (int64_t(1) << 31), "mm_grouped_wgrad: too many tiles");
  const int grid = static_cast<int>(grid64);
  const int px = static_cast<int>(per_xcd);
  if (small) {
    grouped_wgrad_kernel<128, 128, 32, 2, true><<<grid, kThreads, 0, s>>>(a, num_experts, px);
  } else if (bm == 256 && bn == 256) {
    if (wgrad_reg(max_rows, num_experts)) {
      wgrad_reg_kernel<><<<grid, 256, 0, s>>>(a, num_experts, px);
    } else {
      grouped_wgrad_kernel<256, 256, 64, 2, false, 512><<<grid, 512, 0, s>>>(a, num_experts, px);
    }
  } else if (bm == 256) {
    grouped_wgrad_kernel<256, 128, 64, 2, false><<<grid, kThreads, 0, s>>>(a, num_experts, px);
  } else if (bn == 256) {
    grouped_wgrad_kernel<128, 256, 64, 2, false><<<grid, kThreads, 0, s>>>(a, num_experts, px);
  } else {
    grouped_wgrad_kernel<128, 128, 64, 2, false><<<grid, kThreads, 0, s>>>(a, num_experts, px);
  }
  return mm_check_launch("mm_grouped_wgrad");
}
