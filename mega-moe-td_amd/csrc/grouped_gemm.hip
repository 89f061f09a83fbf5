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
//  * One workgroup = 4 wavefronts computing a BM x BN tile with
//    v_mfma_f32_32x32x16_bf16 (each wave owns a (BM/WM) x (BN/WN) sub-tile).
//  * Both operands are staged through LDS in a K-contiguous [row][BK+8]
//    layout (double-buffered, one barrier per K step). Sources whose K axis
//    is contiguous are copied with 16-byte vectors; sources whose M/N axis is
//    contiguous (e.g. gate_up_weight [E, H, 2I], or the rows of the wgrad
//    operands) are transposed on the way into LDS, 4 K-rows at a time.
//  * Ragged experts: a one-workgroup kernel turns offsets[] into a list of
//    (expert, first row) M-tiles on the device; the GEMM grid is an upper
//    bound and surplus workgroups exit at once. Workgroup ids are remapped so
//    that each XCD (ids congruent mod 8) receives a contiguous range of
//    tiles, and tiles are grouped GROUP_M-deep along M so that A panels and
//    B tiles are reused from that XCD's L2.
//  * FC1 epilogue: the B tile interleaves 32-column groups of gate and up so
//    every lane holds gate(i, j) and up(i, j) of the same (row, column) and
//    applies the weighted gated activation before a single bf16 store.
#include "common.h"

namespace {

constexpr int kThreads = 256;
constexpr int BK = 64;
constexpr int LDS_K = BK + 8;  // row pitch in bf16 elements (144 bytes)
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
__device__ __forceinline__ void grouped_mn(int l, int num_m, int num_n, int& m, int& n) {
  const int in_group = GROUP_M * num_n;
  const int g = l / in_group;
  const int first = g * GROUP_M;
  const int gs = min(num_m - first, GROUP_M);
  const int r = l - g * in_group;
  m = first + r % gs;
  n = r / gs;
}

// ------------------------------------------------------------------ loaders
// K-contiguous source: ROWS x BK tile; row r starts at row_ptr(r) (nullptr =
// zero row) and its BK columns k0 .. k0+BK are contiguous.
template <int ROWS>
struct KContigLoader {
  static constexpr int VPR = BK / 8;  // 16-byte vectors per row
  static constexpr int VPT = ROWS * VPR / kThreads;
  static_assert(VPT * kThreads == ROWS * VPR, "tile/threads mismatch");
  const bf16* ptr[VPT];
  uint4 reg[VPT];

  template <class RowPtr>
  __device__ void init(RowPtr row_ptr) {
#pragma unroll
    for (int v = 0; v < VPT; ++v) {
      const int idx = threadIdx.x + v * kThreads;
      const int r = idx / VPR, kv = idx % VPR;
      const bf16* q = row_ptr(r);
      ptr[v] = q ? q + kv * 8 : nullptr;
    }
  }
  __device__ void load(int k0) {
#pragma unroll
    for (int v = 0; v < VPT; ++v)
      reg[v] = ptr[v] ? *reinterpret_cast<const uint4*>(ptr[v] + k0) : make_uint4(0, 0, 0, 0);
  }
  __device__ void store(bf16* lds) const {
#pragma unroll
    for (int v = 0; v < VPT; ++v) {
      const int idx = threadIdx.x + v * kThreads;
      const int r = idx / VPR, kv = idx % VPR;
      *reinterpret_cast<uint4*>(lds + r * LDS_K + kv * 8) = reg[v];
    }
  }
};

// MN-contiguous source: element (k, c) of the tile lives at k_ptr(k)[col_off(c)]
// with 8 consecutive tile columns contiguous. Each thread loads 4 consecutive
// K rows of one 8-column vector and writes them transposed (eight 8-byte LDS
// stores) into the K-contiguous LDS tile.
template <int ROWS>
struct MNContigLoader {
  static constexpr int NV = ROWS / 8;                   // column vectors
  static constexpr int QPT = NV * (BK / 4) / kThreads;  // quads per thread
  static_assert(QPT * kThreads == NV * (BK / 4), "tile/threads mismatch");
  uint4 reg[QPT][4];

  template <class KPtr, class ColOff>
  __device__ void load(KPtr k_ptr, ColOff col_off) {
#pragma unroll
    for (int q = 0; q < QPT; ++q) {
      const int idx = threadIdx.x + q * kThreads;
      const int nv = idx % NV, kq = idx / NV;
      const int64_t co = col_off(nv * 8);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bf16* src = k_ptr(kq * 4 + i);
        reg[q][i] = src ? *reinterpret_cast<const uint4*>(src + co) : make_uint4(0, 0, 0, 0);
      }
    }
  }
  __device__ void store(bf16* lds) const {
#pragma unroll
    for (int q = 0; q < QPT; ++q) {
      const int idx = threadIdx.x + q * kThreads;
      const int nv = idx % NV, kq = idx / NV;
      const uint32_t w0[4] = {reg[q][0].x, reg[q][0].y, reg[q][0].z, reg[q][0].w};
      const uint32_t w1[4] = {reg[q][1].x, reg[q][1].y, reg[q][1].z, reg[q][1].w};
      const uint32_t w2[4] = {reg[q][2].x, reg[q][2].y, reg[q][2].z, reg[q][2].w};
      const uint32_t w3[4] = {reg[q][3].x, reg[q][3].y, reg[q][3].z, reg[q][3].w};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int sh = (j & 1) * 16;
        const uint32_t e0 = (w0[j >> 1] >> sh) & 0xffffu;
        const uint32_t e1 = (w1[j >> 1] >> sh) & 0xffffu;
        const uint32_t e2 = (w2[j >> 1] >> sh) & 0xffffu;
        const uint32_t e3 = (w3[j >> 1] >> sh) & 0xffffu;
        *reinterpret_cast<uint2*>(lds + (nv * 8 + j) * LDS_K + kq * 4) =
            make_uint2(e0 | (e1 << 16), e2 | (e3 << 16));
      }
    }
  }
};

// ------------------------------------------------------------------ MMA core
template <int BM, int BN, int WM, int WN>
struct MmaTile {
  static constexpr int TM = BM / WM, TN = BN / WN;
  static constexpr int MI = TM / 32, NI = TN / 32;
  static_assert(WM * WN == kThreads / 64, "4 waves per workgroup");
  f32x16 acc[MI][NI];

  __device__ void zero() {
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NI; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  }

  __device__ void compute(const bf16* As, const bf16* Bs, int wm, int wn, int lane) {
    const int lr = lane & 31, lk = (lane >> 5) * 8;
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      bf16x8 a[MI], b[NI];
#pragma unroll
      for (int i = 0; i < MI; ++i)
        a[i] = *reinterpret_cast<const bf16x8*>(As + (wm * TM + i * 32 + lr) * LDS_K + kk + lk);
#pragma unroll
      for (int j = 0; j < NI; ++j)
        b[j] = *reinterpret_cast<const bf16x8*>(Bs + (wn * TN + j * 32 + lr) * LDS_K + kk + lk);
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  }

  // Tile row of accumulator element r (0..15) of a 32x32 block for `lane`;
  // the column is lane & 31.
  __device__ static int acc_row(int r, int lane) { return (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3); }
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
  // gated (FC1) epilogue
  const float* w;
  bf16* fc1_out;
  int inter;
  int act_kind;
  float beta, lbeta, clamp;
};

enum { EPI_STORE = 0, EPI_GATED = 1 };
enum { B_KCONTIG = 0, B_NCONTIG = 1 };

template <int BM, int BN, int WM, int WN, int BLAYOUT, int EPI>
__global__ __launch_bounds__(kThreads) void grouped_rows_kernel(RowsArgs p) {
  using Mma = MmaTile<BM, BN, WM, WN>;
  static_assert(EPI != EPI_GATED || (Mma::NI == 2 && BLAYOUT == B_NCONTIG), "gated epilogue layout");
  __shared__ __attribute__((aligned(16))) bf16 smem[2][(BM + BN) * LDS_K];

  const int num_m = p.tl->count;
  const int num_n = p.n / BN;
  const int l = xcd_remap(blockIdx.x, num_m * num_n);
  if (l < 0) return;
  int mt, nt;
  grouped_mn(l, num_m, num_n, mt, nt);
  const int4 tile = p.tl->tiles[mt];
  const int e = tile.x, row0 = tile.y, rows = tile.z - tile.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int n0 = nt * BN;
  const bf16* bexp = p.b + static_cast<int64_t>(e) * p.b_se;

  KContigLoader<BM> la;
  la.init([&](int r) -> const bf16* {
    if (r >= rows) return nullptr;
    const int64_t src = p.a_rows ? static_cast<int64_t>(p.a_rows[row0 + r]) : static_cast<int64_t>(row0 + r);
    return p.a + src * p.lda;
  });

  // B tile column c -> global column n (gated: 32-wide gate/up interleave).
  auto bcol = [&](int c) -> int64_t {
    if constexpr (EPI == EPI_GATED) {
      const int wnc = c / 64, sub = (c / 32) & 1, jj = c & 31;
      return static_cast<int64_t>(sub) * p.inter + nt * (BN / 2) + wnc * 32 + jj;
    } else {
      return n0 + c;
    }
  };

  KContigLoader<BN> lbk;
  MNContigLoader<BN> lbn;
  if constexpr (BLAYOUT == B_KCONTIG) {
    lbk.init([&](int c) -> const bf16* { return bexp + bcol(c) * p.b_sn; });
  }
  auto load_b = [&](int k0) {
    if constexpr (BLAYOUT == B_KCONTIG) {
      lbk.load(k0);
    } else {
      lbn.load([&](int kk) -> const bf16* { return bexp + static_cast<int64_t>(k0 + kk) * p.b_sk; }, bcol);
    }
  };
  auto store_b = [&](bf16* lds) {
    if constexpr (BLAYOUT == B_KCONTIG) lbk.store(lds); else lbn.store(lds);
  };

  Mma mma;
  mma.zero();
  const int nk = p.k / BK;
  la.load(0);
  load_b(0);
  la.store(smem[0]);
  store_b(smem[0] + BM * LDS_K);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) {
      la.load((kt + 1) * BK);
      load_b((kt + 1) * BK);
    }
    mma.compute(smem[cur], smem[cur] + BM * LDS_K, wm, wn, lane);
    if (kt + 1 < nk) {
      la.store(smem[cur ^ 1]);
      store_b(smem[cur ^ 1] + BM * LDS_K);
    }
    __syncthreads();
  }

  // ---- epilogue
  const int col = lane & 31;
  if constexpr (EPI == EPI_STORE) {
#pragma unroll
    for (int i = 0; i < Mma::MI; ++i)
#pragma unroll
      for (int j = 0; j < Mma::NI; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int tr = wm * Mma::TM + i * 32 + Mma::acc_row(r, lane);
          if (tr < rows) {
            const int tc = wn * Mma::TN + j * 32 + col;
            reinterpret_cast<uint16_t*>(p.c)[static_cast<int64_t>(row0 + tr) * p.ldc + n0 + tc] =
                f32_to_bf16_bits(mma.acc[i][j][r]);
          }
        }
  } else {
    const int jcol = nt * (BN / 2) + wn * 32 + col;  // gate/up column index in [0, I)
#pragma unroll
    for (int i = 0; i < Mma::MI; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int tr = wm * Mma::TM + i * 32 + Mma::acc_row(r, lane);
        if (tr < rows) {
          const int64_t row = row0 + tr;
          const uint16_t gb = f32_to_bf16_bits(mma.acc[i][0][r]);
          const uint16_t ub = f32_to_bf16_bits(mma.acc[i][1][r]);
          if (p.fc1_out) {
            uint16_t* fo = reinterpret_cast<uint16_t*>(p.fc1_out) + row * (2 * static_cast<int64_t>(p.inter));
            fo[jcol] = gb;
            fo[p.inter + jcol] = ub;
          }
          const float v = gated_act(p.act_kind, bf16_bits_to_f32(gb), bf16_bits_to_f32(ub), p.beta, p.lbeta,
                                    p.clamp) * p.w[row];
          reinterpret_cast<uint16_t*>(p.c)[row * p.ldc + jcol] = f32_to_bf16_bits(v);
        }
      }
  }
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
};

template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(kThreads) void grouped_wgrad_kernel(WgradArgs a, int num_experts) {
  using Mma = MmaTile<BM, BN, WM, WN>;
  __shared__ __attribute__((aligned(16))) bf16 smem[2][(BM + BN) * LDS_K];
  const int t1n = a.n1 / BM, t2n = a.n2 / BN;
  const int per_e = t1n * t2n;
  const int l = xcd_remap(blockIdx.x, num_experts * per_e);
  if (l < 0) return;
  const int e = l / per_e;
  int t1, t2;
  grouped_mn(l - e * per_e, t1n, t2n, t1, t2);
  const int r0 = a.offsets[e], r1 = a.offsets[e + 1];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;

  MNContigLoader<BM> lp;
  MNContigLoader<BN> lq;
  auto load = [&](int k0) {
    lp.load(
        [&](int kk) -> const bf16* {
          const int r = r0 + k0 + kk;
          if (r >= r1) return nullptr;
          const int64_t src = a.p_rows ? static_cast<int64_t>(a.p_rows[r]) : static_cast<int64_t>(r);
          return a.p + src * a.ldp;
        },
        [&](int c) -> int64_t { return static_cast<int64_t>(t1) * BM + c; });
    lq.load(
        [&](int kk) -> const bf16* {
          const int r = r0 + k0 + kk;
          if (r >= r1) return nullptr;
          const int64_t src = a.q_rows ? static_cast<int64_t>(a.q_rows[r]) : static_cast<int64_t>(r);
          return a.q + src * a.ldq;
        },
        [&](int c) -> int64_t { return static_cast<int64_t>(t2) * BN + c; });
  };

  Mma mma;
  mma.zero();
  const int nk = (r1 - r0 + BK - 1) / BK;
  if (nk > 0) {
    load(0);
    lp.store(smem[0]);
    lq.store(smem[0] + BM * LDS_K);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const int cur = kt & 1;
      if (kt + 1 < nk) load((kt + 1) * BK);
      mma.compute(smem[cur], smem[cur] + BM * LDS_K, wm, wn, lane);
      if (kt + 1 < nk) {
        lp.store(smem[cur ^ 1]);
        lq.store(smem[cur ^ 1] + BM * LDS_K);
      }
      __syncthreads();
    }
  }
  uint16_t* out = reinterpret_cast<uint16_t*>(a.c) + static_cast<int64_t>(e) * a.n1 * a.n2;
  const int col = lane & 31;
#pragma unroll
  for (int i = 0; i < Mma::MI; ++i)
#pragma unroll
    for (int j = 0; j < Mma::NI; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = static_cast<int64_t>(t1) * BM + wm * Mma::TM + i * 32 + Mma::acc_row(r, lane);
        const int64_t cc = static_cast<int64_t>(t2) * BN + wn * Mma::TN + j * 32 + col;
        out[row * a.n2 + cc] = f32_to_bf16_bits(mma.acc[i][j][r]);
      }
}

// ------------------------------------------------------------------ host side
constexpr int kBM = 128, kBN = 128, kWM = 2, kWN = 2;

int64_t max_m_tiles(int64_t max_rows, int E, int BM) { return (max_rows + BM - 1) / BM + E; }

size_t tile_list_bytes(int64_t max_rows, int E) {
  return mm_align_up(sizeof(TileList) + sizeof(int4) * static_cast<size_t>(max_m_tiles(max_rows, E, kBM)), 256);
}

int launch_tiles(const int32_t* offsets, int E, void* ws, hipStream_t s) {
  build_tiles_kernel<<<1, 1024, 0, s>>>(offsets, E, kBM, static_cast<TileList*>(ws));
  return mm_check_launch("build_tiles");
}

int rows_grid(int64_t max_rows, int E, int n, int BN) {
  const int64_t g = max_m_tiles(max_rows, E, kBM) * (n / BN);
  return static_cast<int>((g + kXcds - 1) / kXcds * kXcds);
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" size_t mm_gemm_workspace_bytes(int64_t max_rows, int32_t num_experts) {
  return tile_list_bytes(max_rows, num_experts);
}

extern "C" int mm_fc1_swiglu(const uint16_t* x, int64_t ldx, const int32_t* send_token, const uint16_t* w1,
                             const int32_t* offsets, const float* weight_perm, int32_t num_experts,
                             int64_t max_rows, int32_t hidden, int32_t inter, int32_t act_kind, float situ_beta,
                             float situ_linear_beta, float clamp_limit, uint16_t* act, uint16_t* fc1_out,
                             void* workspace, size_t workspace_bytes, mm_stream_t stream) {
  MM_CHECK_ARG(x && w1 && offsets && weight_perm && act, "mm_fc1_swiglu: null pointer");
  MM_CHECK_ARG(num_experts > 0 && max_rows >= 0 && max_rows < (int64_t(1) << 31), "mm_fc1_swiglu: bad sizes");
  MM_CHECK_ARG(hidden > 0 && hidden % BK == 0, "mm_fc1_swiglu: hidden must be a multiple of %d", BK);
  MM_CHECK_ARG(inter > 0 && inter % (kBN / 2) == 0, "mm_fc1_swiglu: inter must be a multiple of %d", kBN / 2);
  MM_CHECK_ARG(ldx % 8 == 0 && al16(x) && al16(w1), "mm_fc1_swiglu: 16-byte alignment required");
  MM_CHECK_ARG(act_kind >= 0 && act_kind <= 2, "mm_fc1_swiglu: bad act_kind");
  if (!workspace || workspace_bytes < tile_list_bytes(max_rows, num_experts)) {
    mm_set_error("mm_fc1_swiglu: workspace too small");
    return MM_E_WS;
  }
  if (max_rows == 0) return MM_OK;
  hipStream_t s = mm_hip_stream(stream);
  if (int rc = launch_tiles(offsets, num_experts, workspace, s)) return rc;
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
  p.tl = static_cast<const TileList*>(workspace);
  p.w = weight_perm;
  p.fc1_out = reinterpret_cast<bf16*>(fc1_out);
  p.inter = inter;
  p.act_kind = act_kind;
  p.beta = situ_beta;
  p.lbeta = situ_linear_beta;
  p.clamp = clamp_limit;
  grouped_rows_kernel<kBM, kBN, kWM, kWN, B_NCONTIG, EPI_GATED>
      <<<rows_grid(max_rows, num_experts, p.n, kBN), kThreads, 0, s>>>(p);
  return mm_check_launch("mm_fc1_swiglu");
}

extern "C" int mm_grouped_gemm(const uint16_t* a, int64_t lda, const int32_t* a_rows, const uint16_t* b,
                               int64_t b_se, int64_t b_sn, int64_t b_sk, const int32_t* offsets,
                               int32_t num_experts, int64_t max_rows, int32_t n, int32_t k, uint16_t* c,
                               int64_t ldc, void* workspace, size_t workspace_bytes, mm_stream_t stream) {
  MM_CHECK_ARG(a && b && offsets && c, "mm_grouped_gemm: null pointer");
  MM_CHECK_ARG(num_experts > 0 && max_rows >= 0 && max_rows < (int64_t(1) << 31), "mm_grouped_gemm: bad sizes");
  MM_CHECK_ARG(n > 0 && n % kBN == 0, "mm_grouped_gemm: n must be a multiple of %d", kBN);
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
  hipStream_t s = mm_hip_stream(stream);
  if (int rc = launch_tiles(offsets, num_experts, workspace, s)) return rc;
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
  p.tl = static_cast<const TileList*>(workspace);
  const int grid = rows_grid(max_rows, num_experts, n, kBN);
  if (b_sk == 1)
    grouped_rows_kernel<kBM, kBN, kWM, kWN, B_KCONTIG, EPI_STORE><<<grid, kThreads, 0, s>>>(p);
  else
    grouped_rows_kernel<kBM, kBN, kWM, kWN, B_NCONTIG, EPI_STORE><<<grid, kThreads, 0, s>>>(p);
  return mm_check_launch("mm_grouped_gemm");
}

extern "C" int mm_grouped_wgrad(const uint16_t* p, int64_t ldp, const int32_t* p_rows, const uint16_t* q,
                                int64_t ldq, const int32_t* q_rows, const int32_t* offsets, int32_t num_experts,
                                int32_t n1, int32_t n2, uint16_t* c, void* workspace, size_t workspace_bytes,
                                mm_stream_t stream) {
  (void)workspace;
  (void)workspace_bytes;
  MM_CHECK_ARG(p && q && offsets && c, "mm_grouped_wgrad: null pointer");
  MM_CHECK_ARG(num_experts > 0, "mm_grouped_wgrad: bad num_experts");
  MM_CHECK_ARG(n1 > 0 && n1 % kBM == 0 && n2 > 0 && n2 % kBN == 0,
               "mm_grouped_wgrad: n1, n2 must be multiples of %d", kBM);
  MM_CHECK_ARG(ldp % 8 == 0 && ldq % 8 == 0 && al16(p) && al16(q), "mm_grouped_wgrad: 16-byte alignment required");
  WgradArgs a{p ? reinterpret_cast<const bf16*>(p) : nullptr, ldp, p_rows, reinterpret_cast<const bf16*>(q), ldq,
              q_rows, offsets, n1, n2, reinterpret_cast<bf16*>(c)};
  const int64_t tiles = static_cast<int64_t>(num_experts) * (n1 / kBM) * (n2 / kBN);
  MM_CHECK_ARG(tiles < (int64_t(1) << 31) - 8, "mm_grouped_wgrad: too many tiles");
  const int grid = static_cast<int>((tiles + kXcds - 1) / kXcds * kXcds);
  grouped_wgrad_kernel<kBM, kBN, kWM, kWN><<<grid, kThreads, 0, mm_hip_stream(stream)>>>(a, num_experts);
  return mm_check_launch("mm_grouped_wgrad");
}
