// fp32 MFMA GEMM core for gfx950 (CDNA4), shared by the plain GEMM entry point and
// the per-time-step recurrent kernels (which plug in their own epilogues).
//
//   C[M,N] = op(A)[M,K] . op(B)[K,N]
//
// One workgroup = 256 threads = 4 wave64s arranged WM x WN x WK.  A workgroup tile
// is BM x BN; each wave owns a (BM/WM) x (BN/WN) sub-tile made of 32x32 fragments
// computed with v_mfma_f32_32x32x2_f32, and the WK waves that share a sub-tile
// split every BK-slice of K between them (their partial tiles are summed in the
// epilogue).  A and B tiles are staged in LDS as [row][k] with k contiguous, so a
// lane reads its k-run with 128-bit LDS loads.
//
// k-ordering inside a wave's KS = BK/WK slice: for MFMA step i the lower half of the
// wave (lanes 0-31) supplies k = i and the upper half k = KS/2 + i.  A and B use the
// same permutation, so the sum over k is unchanged.
//
// Fragment layouts of v_mfma_f32_32x32x2_f32 (verified on gfx950):
//   A: lane l holds A[row = l%32][k = l/32]
//   B: lane l holds B[k = l/32][col = l%32]
//   D: lane l, reg r holds D[row = 8*(r/4) + 4*(l/32) + r%4][col = l%32]
#pragma once

#include "hsl_internal.h"

namespace hsl {

template <int BM_, int BN_, int BK_, int WM_, int WN_, int WK_>
struct GemmCfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_, WK = WK_;
  static constexpr int kThreads = 256;
  static_assert(WM * WN * WK == 4, "four waves per workgroup");
  static constexpr int TM = BM / WM, TN = BN / WN;
  static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile must be made of 32x32 fragments");
  static constexpr int FM = TM / 32, FN = TN / 32;
  static constexpr int KS = BK / WK;
  static constexpr int KH = KS / 2;
  static_assert(KH % 4 == 0, "each lane half reads k in runs of 4");
  static constexpr int LDK = BK + 4;  // LDS row stride in floats (keeps 16-byte alignment)
  static_assert((BM * BK / 4) % kThreads == 0 && (BN * BK / 4) % kThreads == 0,
                "tile loads must divide evenly over 256 threads");
  static constexpr int A_CHUNKS = BM * BK / 4 / kThreads;
  static constexpr int B_CHUNKS = BN * BK / 4 / kThreads;
  static constexpr int LDC = BN + 1;  // epilogue tile row stride
  static constexpr int LDS_AB = (BM + BN) * LDK;
  static constexpr int LDS_C = WK * BM * LDC;
  static constexpr int LDS_FLOATS = LDS_AB > LDS_C ? LDS_AB : LDS_C;
  static constexpr size_t LDS_BYTES = sizeof(float) * LDS_FLOATS;
};

struct GemmArgs {
  const float* A;
  const float* B;
  int M, N, K, lda, ldb;
  int k_per_split;  // multiple of BK; blockIdx.z selects the split
  int vec_a, vec_b; // 1 when 128-bit global loads are legal (alignment of base and ld)
  int tiles_n, tiles_m;
};

// Sum of the WK partial tiles at (m, n) of the staged epilogue tile.
template <class Cfg>
__device__ __forceinline__ float tile_value(const float* Cs, int m, int n) {
  float v = Cs[m * Cfg::LDC + n];
#pragma unroll
  for (int w = 1; w < Cfg::WK; ++w) v += Cs[w * Cfg::BM * Cfg::LDC + m * Cfg::LDC + n];
  return v;
}

template <class Cfg, bool TA>
__device__ __forceinline__ void load_a(const GemmArgs& g, int m0, int k0, int kend, f4 (&ra)[Cfg::A_CHUNKS]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int j = 0; j < Cfg::A_CHUNKS; ++j) {
    const int c = t + Cfg::kThreads * j;
    f4 v = {0.f, 0.f, 0.f, 0.f};
    if (!TA) {
      const int row = c / (Cfg::BK / 4), kq = c % (Cfg::BK / 4);
      const int m = m0 + row, k = k0 + kq * 4;
      if (m < g.M) {
        const float* p = g.A + (size_t)m * g.lda + k;
        if (g.vec_a && k + 3 < kend) {
          v = *reinterpret_cast<const f4*>(p);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) if (k + e < kend) v[e] = p[e];
        }
      }
    } else {
      const int krow = c / (Cfg::BM / 4), mq = c % (Cfg::BM / 4);
      const int k = k0 + krow, m = m0 + mq * 4;
      if (k < kend) {
        const float* p = g.A + (size_t)k * g.lda + m;
        if (g.vec_a && m + 3 < g.M) {
          v = *reinterpret_cast<const f4*>(p);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) if (m + e < g.M) v[e] = p[e];
        }
      }
    }
    ra[j] = v;
  }
}

template <class Cfg, bool TB>
__device__ __forceinline__ void load_b(const GemmArgs& g, int n0, int k0, int kend, f4 (&rb)[Cfg::B_CHUNKS]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int j = 0; j < Cfg::B_CHUNKS; ++j) {
    const int c = t + Cfg::kThreads * j;
    f4 v = {0.f, 0.f, 0.f, 0.f};
    if (TB) {  // B stored [N][K]
      const int row = c / (Cfg::BK / 4), kq = c % (Cfg::BK / 4);
      const int n = n0 + row, k = k0 + kq * 4;
      if (n < g.N) {
        const float* p = g.B + (size_t)n * g.ldb + k;
        if (g.vec_b && k + 3 < kend) {
          v = *reinterpret_cast<const f4*>(p);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) if (k + e < kend) v[e] = p[e];
        }
      }
    } else {   // B stored [K][N]
      const int krow = c / (Cfg::BN / 4), nq = c % (Cfg::BN / 4);
      const int k = k0 + krow, n = n0 + nq * 4;
      if (k < kend) {
        const float* p = g.B + (size_t)k * g.ldb + n;
        if (g.vec_b && n + 3 < g.N) {
          v = *reinterpret_cast<const f4*>(p);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) if (n + e < g.N) v[e] = p[e];
        }
      }
    }
    rb[j] = v;
  }
}

// Unmasked loads of one slice for a tile that lies inside both operands with 16-byte
// aligned rows and a whole slice of k (the condition is uniform over the workgroup; see
// gemm_tile): straight-line code, where the masked loads above carry a bounds and
// alignment branch per 16-byte chunk.
template <class Cfg, bool TA, bool TB>
__device__ __forceinline__ void load_ab_full(const GemmArgs& g, int m0, int n0, int k0, f4 (&ra)[Cfg::A_CHUNKS],
                                             f4 (&rb)[Cfg::B_CHUNKS]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int j = 0; j < Cfg::A_CHUNKS; ++j) {
    const int c = t + Cfg::kThreads * j;
    const float* p;
    if (!TA) {
      const int row = c / (Cfg::BK / 4), kq = c % (Cfg::BK / 4);
      p = g.A + (size_t)(m0 + row) * g.lda + k0 + kq * 4;
    } else {
      const int krow = c / (Cfg::BM / 4), mq = c % (Cfg::BM / 4);
      p = g.A + (size_t)(k0 + krow) * g.lda + m0 + mq * 4;
    }
    ra[j] = *reinterpret_cast<const f4*>(p);
  }
#pragma unroll
  for (int j = 0; j < Cfg::B_CHUNKS; ++j) {
    const int c = t + Cfg::kThreads * j;
    const float* p;
    if (TB) {
      const int row = c / (Cfg::BK / 4), kq = c % (Cfg::BK / 4);
      p = g.B + (size_t)(n0 + row) * g.ldb + k0 + kq * 4;
    } else {
      const int krow = c / (Cfg::BN / 4), nq = c % (Cfg::BN / 4);
      p = g.B + (size_t)(k0 + krow) * g.ldb + n0 + nq * 4;
    }
    rb[j] = *reinterpret_cast<const f4*>(p);
  }
}

template <class Cfg, bool TA, bool TB>
__device__ __forceinline__ void store_ab(float* As, float* Bs, const f4 (&ra)[Cfg::A_CHUNKS],
                                         const f4 (&rb)[Cfg::B_CHUNKS]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int j = 0; j < Cfg::A_CHUNKS; ++j) {
    const int c = t + Cfg::kThreads * j;
    if (!TA) {
      const int row = c / (Cfg::BK / 4), kq = c % (Cfg::BK / 4);
      *reinterpret_cast<f4*>(As + row * Cfg::LDK + kq * 4) = ra[j];
    } else {
      const int krow = c / (Cfg::BM / 4), mq = c % (Cfg::BM / 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) As[(mq * 4 + e) * Cfg::LDK + krow] = ra[j][e];
    }
  }
#pragma unroll
  for (int j = 0; j < Cfg::B_CHUNKS; ++j) {
    const int c = t + Cfg::kThreads * j;
    if (TB) {
      const int row = c / (Cfg::BK / 4), kq = c % (Cfg::BK / 4);
      *reinterpret_cast<f4*>(Bs + row * Cfg::LDK + kq * 4) = rb[j];
    } else {
      const int krow = c / (Cfg::BN / 4), nq = c % (Cfg::BN / 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) Bs[(nq * 4 + e) * Cfg::LDK + krow] = rb[j][e];
    }
  }
}

// Main loop: accumulates the workgroup tile (m0, n0) over k in [kbeg, kend) and
// leaves the WK partial tiles in LDS (Cs = smem) for the epilogue.  With ACC64 the
// MFMA accumulators restart from zero on every BK-slice and each slice's partial is
// added into fp64 registers, so a long K is summed as K/BK fp64 additions of
// BK-term fp32 partials (used for the weight gradients, K = T*B).
template <class Cfg, bool TA, bool TB, bool ACC64 = false>
__device__ __forceinline__ void gemm_tile(const GemmArgs& g, int m0, int n0, int kbeg, int kend, float* smem) {
  float* As = smem;
  float* Bs = smem + Cfg::BM * Cfg::LDK;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wk = wave % Cfg::WK;
  const int wn = (wave / Cfg::WK) % Cfg::WN;
  const int wm = wave / (Cfg::WK * Cfg::WN);
  const int half = lane >> 5, r32 = lane & 31;

  f16v acc[Cfg::FM][Cfg::FN];
#pragma unroll
  for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
    for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  double acc64[ACC64 ? Cfg::FM : 1][ACC64 ? Cfg::FN : 1][ACC64 ? 16 : 1];
  if (ACC64) {
#pragma unroll
    for (int i = 0; i < (ACC64 ? Cfg::FM : 1); ++i)
#pragma unroll
      for (int j = 0; j < (ACC64 ? Cfg::FN : 1); ++j)
#pragma unroll
        for (int r = 0; r < (ACC64 ? 16 : 1); ++r) acc64[i][j][r] = 0.0;
  }

  // full: the tile lies inside both operands, rows are 16-byte aligned and k splits
  // into whole slices, so every slice takes the unmasked loads (uniform branch)
  const bool full = g.vec_a && g.vec_b && (kend - kbeg) % Cfg::BK == 0 &&
                    (TA ? m0 + Cfg::BM <= g.M && g.M % 4 == 0 : m0 + Cfg::BM <= g.M) &&
                    (TB ? n0 + Cfg::BN <= g.N : n0 + Cfg::BN <= g.N && g.N % 4 == 0);
  f4 ra[Cfg::A_CHUNKS], rb[Cfg::B_CHUNKS];
  if (kbeg < kend) {
    if (full) {
      load_ab_full<Cfg, TA, TB>(g, m0, n0, kbeg, ra, rb);
    } else {
      load_a<Cfg, TA>(g, m0, kbeg, kend, ra);
      load_b<Cfg, TB>(g, n0, kbeg, kend, rb);
    }
  }
  for (int k0 = kbeg; k0 < kend; k0 += Cfg::BK) {
    __syncthreads();  // previous stage fully consumed
    store_ab<Cfg, TA, TB>(As, Bs, ra, rb);
    __syncthreads();
    if (k0 + Cfg::BK < kend) {  // prefetch the next stage into registers
      if (full) {
        load_ab_full<Cfg, TA, TB>(g, m0, n0, k0 + Cfg::BK, ra, rb);
      } else {
        load_a<Cfg, TA>(g, m0, k0 + Cfg::BK, kend, ra);
        load_b<Cfg, TB>(g, n0, k0 + Cfg::BK, kend, rb);
      }
    }
    const int kb = wk * Cfg::KS + half * Cfg::KH;
#pragma unroll
    for (int kk = 0; kk < Cfg::KH; kk += 4) {
      f4 av[Cfg::FM], bv[Cfg::FN];
#pragma unroll
      for (int i = 0; i < Cfg::FM; ++i)
        av[i] = *reinterpret_cast<const f4*>(As + (wm * Cfg::TM + i * 32 + r32) * Cfg::LDK + kb + kk);
#pragma unroll
      for (int j = 0; j < Cfg::FN; ++j)
        bv[j] = *reinterpret_cast<const f4*>(Bs + (wn * Cfg::TN + j * 32 + r32) * Cfg::LDK + kb + kk);
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
          for (int j = 0; j < Cfg::FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][e], bv[j][e], acc[i][j], 0, 0, 0);
    }
    if (ACC64) {
#pragma unroll
      for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
        for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            acc64[ACC64 ? i : 0][ACC64 ? j : 0][ACC64 ? r : 0] += (double)acc[i][j][r];
            acc[i][j][r] = 0.f;
          }
    }
  }
  if (ACC64) {
#pragma unroll
    for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
      for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = (float)acc64[ACC64 ? i : 0][ACC64 ? j : 0][ACC64 ? r : 0];
  }
  __syncthreads();  // A/B stage dead; reuse LDS for the epilogue tile
  float* Cs = smem + wk * Cfg::BM * Cfg::LDC;
#pragma unroll
  for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
    for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = wm * Cfg::TM + i * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
        const int n = wn * Cfg::TN + j * 32 + r32;
        Cs[m * Cfg::LDC + n] = acc[i][j][r];
      }
  __syncthreads();
}

// gemm_tile for a full tile (see load_ab_full) with DEPTH register stages: slices s+1 ..
// s+DEPTH-1 are loading while slice s is multiplied, and the barriers order LDS only
// (lds_barrier), so none of them waits for the loads in flight.  The k-steps alternate
// between two accumulators (even / odd k pairs), so back-to-back MFMAs do not depend on
// each other; the two are added before the epilogue.
template <class Cfg, bool TA, bool TB, int DEPTH>
__device__ __forceinline__ void gemm_tile_full_deep(const GemmArgs& g, int m0, int n0, int kbeg, int kend,
                                                    float* smem) {
  float* As = smem;
  float* Bs = smem + Cfg::BM * Cfg::LDK;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wk = wave % Cfg::WK;
  const int wn = (wave / Cfg::WK) % Cfg::WN;
  const int wm = wave / (Cfg::WK * Cfg::WN);
  const int half = lane >> 5, r32 = lane & 31;
  f16v acc[Cfg::FM][Cfg::FN], acc2[Cfg::FM][Cfg::FN];
#pragma unroll
  for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
    for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = acc2[i][j][r] = 0.f;
  f4 ra[DEPTH][Cfg::A_CHUNKS], rb[DEPTH][Cfg::B_CHUNKS];
#pragma unroll
  for (int d = 0; d < DEPTH - 1; ++d)
    if (kbeg + d * Cfg::BK < kend) load_ab_full<Cfg, TA, TB>(g, m0, n0, kbeg + d * Cfg::BK, ra[d], rb[d]);
  for (int k0 = kbeg; k0 < kend; k0 += DEPTH * Cfg::BK) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      const int ks = k0 + d * Cfg::BK;
      if (ks >= kend) break;
      lds_barrier();  // previous slice fully consumed
      store_ab<Cfg, TA, TB>(As, Bs, ra[d], rb[d]);
      lds_barrier();
      const int kn = ks + (DEPTH - 1) * Cfg::BK;  // into the stage of the slice before
      if (kn < kend) load_ab_full<Cfg, TA, TB>(g, m0, n0, kn, ra[(d + DEPTH - 1) % DEPTH], rb[(d + DEPTH - 1) % DEPTH]);
      const int kb = wk * Cfg::KS + half * Cfg::KH;
#pragma unroll
      for (int kk = 0; kk < Cfg::KH; kk += 4) {
        f4 av[Cfg::FM], bv[Cfg::FN];
#pragma unroll
        for (int i = 0; i < Cfg::FM; ++i)
          av[i] = *reinterpret_cast<const f4*>(As + (wm * Cfg::TM + i * 32 + r32) * Cfg::LDK + kb + kk);
#pragma unroll
        for (int j = 0; j < Cfg::FN; ++j)
          bv[j] = *reinterpret_cast<const f4*>(Bs + (wn * Cfg::TN + j * 32 + r32) * Cfg::LDK + kb + kk);
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
            for (int j = 0; j < Cfg::FN; ++j) {
              if (e & 1)
                acc2[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][e], bv[j][e], acc2[i][j], 0, 0, 0);
              else
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][e], bv[j][e], acc[i][j], 0, 0, 0);
            }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
    for (int j = 0; j < Cfg::FN; ++j) acc[i][j] += acc2[i][j];
  lds_barrier();  // A/B stage dead; reuse LDS for the epilogue tile
  float* Cs = smem + wk * Cfg::BM * Cfg::LDC;
#pragma unroll
  for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
    for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = wm * Cfg::TM + i * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
        const int n = wn * Cfg::TN + j * 32 + r32;
        Cs[m * Cfg::LDC + n] = acc[i][j][r];
      }
  __syncthreads();
}

// Maps blockIdx.x to a tile (tm, tn).  Workgroup i runs on XCD i % 8, so each XCD gets
// a contiguous range of the tile sequence (when the tile count divides by 8), and the
// sequence visits tiles in groups of 8 row panels: consecutive tiles walk down 8 rows
// of one column before moving to the next column.  The workgroups in flight on one XCD
// (two per CU) then share 8 A panels and 8 B panels, which stay in that XCD's L2,
// instead of sweeping every column of B for each row panel.
__device__ __forceinline__ void gemm_tile_order(int tiles_m, int tiles_n, int* tm, int* tn) {
  const int total = tiles_m * tiles_n;
  int id = blockIdx.x;
  if (total % 8 == 0) id = (id % 8) * (total / 8) + id / 8;
  constexpr int GM = 8;
  const int group = id / (GM * tiles_n);
  const int first = group * GM;
  const int rows = min(GM, tiles_m - first);
  const int in = id - group * GM * tiles_n;
  *tm = first + in % rows;
  *tn = in / rows;
}

__device__ __forceinline__ void tile_coords(const GemmArgs& g, int* tm, int* tn) {
  gemm_tile_order(g.tiles_m, g.tiles_n, tm, tn);
}

template <class Cfg, bool TA, bool TB, class Epi, bool ACC64 = false, int DEPTH = 1>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs g, Epi epi) {
  static_assert(DEPTH == 1 || !ACC64, "the deep pipeline has no fp64 fold");
  extern __shared__ float smem[];
  int tm, tn;
  tile_coords(g, &tm, &tn);
  const int m0 = tm * Cfg::BM, n0 = tn * Cfg::BN;
  const int kbeg = blockIdx.z * g.k_per_split;
  const int kend = min(g.K, kbeg + g.k_per_split);
  bool deep = false;
  if constexpr (DEPTH > 1)
    deep = g.vec_a && g.vec_b && (kend - kbeg) % Cfg::BK == 0 && m0 + Cfg::BM <= g.M && n0 + Cfg::BN <= g.N &&
           (!TA || g.M % 4 == 0) && (TB || g.N % 4 == 0);
  if (deep)
    gemm_tile_full_deep<Cfg, TA, TB, (DEPTH > 1 ? DEPTH : 2)>(g, m0, n0, kbeg, kend, smem);
  else
    gemm_tile<Cfg, TA, TB, ACC64>(g, m0, n0, kbeg, kend, smem);
  epi.template run<Cfg>(smem, m0, n0, blockIdx.z);
}

// ---- epilogues ------------------------------------------------------------------
// C = tile (+ bias[n]); row-major with ldc.
struct EpiStore {
  float* C;
  const float* bias;
  int M, N, ldc;
  template <class Cfg>
  __device__ __forceinline__ void run(const float* Cs, int m0, int n0, int) const {
    for (int e = threadIdx.x; e < Cfg::BM * Cfg::BN; e += Cfg::kThreads) {
      const int m = e / Cfg::BN, n = e % Cfg::BN;
      if (m0 + m < M && n0 + n < N) {
        float v = tile_value<Cfg>(Cs, m, n);
        if (bias) v += bias[n0 + n];
        C[(size_t)(m0 + m) * ldc + n0 + n] = v;
      }
    }
  }
};

// Split-K partial: P[split][M][N].
struct EpiPartial {
  float* P;
  int M, N;
  template <class Cfg>
  __device__ __forceinline__ void run(const float* Cs, int m0, int n0, int split) const {
    float* base = P + (size_t)split * M * N;
    for (int e = threadIdx.x; e < Cfg::BM * Cfg::BN; e += Cfg::kThreads) {
      const int m = e / Cfg::BN, n = e % Cfg::BN;
      if (m0 + m < M && n0 + n < N) base[(size_t)(m0 + m) * N + n0 + n] = tile_value<Cfg>(Cs, m, n);
    }
  }
};

// Splits actually used for a requested split count (k per split rounded up to BK).
template <class Cfg>
inline int split_layout(int K, int splits, int* k_per_split) {
  if (splits < 1) splits = 1;
  int kps = (K + splits - 1) / splits;
  kps = (kps + Cfg::BK - 1) / Cfg::BK * Cfg::BK;
  if (kps < Cfg::BK) kps = Cfg::BK;
  *k_per_split = kps;
  int n = (K + kps - 1) / kps;
  return n < 1 ? 1 : n;
}

template <class Cfg, bool TA, bool TB, class Epi, bool ACC64 = false, int DEPTH = 1>
inline int launch_gemm(const GemmArgs& g0, int splits, const Epi& epi, hipStream_t s) {
  GemmArgs g = g0;
  g.tiles_m = (g.M + Cfg::BM - 1) / Cfg::BM;
  g.tiles_n = (g.N + Cfg::BN - 1) / Cfg::BN;
  splits = split_layout<Cfg>(g.K, splits, &g.k_per_split);
  dim3 grid(g.tiles_m * g.tiles_n, 1, splits);
  hipLaunchKernelGGL((gemm_kernel<Cfg, TA, TB, Epi, ACC64, DEPTH>), grid, dim3(256), Cfg::LDS_BYTES, s, g, epi);
  HSL_HIP(hipGetLastError());
  return HSL_OK;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace hsl
