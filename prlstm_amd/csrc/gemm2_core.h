// Second-generation fp32 MFMA GEMM core for gfx950: double-buffered LDS (one barrier
// per BK-slice) and operand layouts chosen per transpose so that every global->LDS
// copy is a straight 128-bit store.
//
//   C[M,N] = op(A)[M,K] . op(B)[K,N]      (row-major, 32x32x2 fp32 MFMA fragments)
//
// * An operand whose k index is contiguous in memory (A not transposed, B transposed)
//   is staged as [row][k] and read by the MFMA lanes as 128-bit k-runs, with the same
//   half-wave k permutation as gemm_core.h (lanes 0-31 take k = i, lanes 32-63
//   k = KH + i; A and B agree, so the sum is unchanged).
// * An operand whose row index is contiguous (A transposed, B not transposed) is
//   staged as [k][row]; lanes read it with 32-bit loads of consecutive rows, which hit
//   consecutive banks, so neither the copy nor the reads have bank conflicts.
// * The store / split-K epilogues write straight from the accumulators: a fragment
//   register holds 32 consecutive columns of one row across lanes 0-31 (and another
//   row across lanes 32-63), i.e. 128-byte row segments.
// * ACC64 restarts the MFMA accumulators every BK-slice and adds each slice into fp64
//   registers (long K reductions, e.g. the weight gradients with K = T*B).
#pragma once

#include "gemm_core.h"

namespace hsl {

template <int BM_, int BN_, int BK_, bool ACC64_>
struct Gemm2Cfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_;
  static constexpr bool ACC64 = ACC64_;
  static constexpr int kThreads = 256;        // 2 x 2 waves
  static constexpr int TM = BM / 2, TN = BN / 2;
  static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile must be made of 32x32 fragments");
  static constexpr int FM = TM / 32, FN = TN / 32;
  static constexpr int KH = BK / 2;
  static_assert(KH % 4 == 0, "k-runs of 4");
  static constexpr int A_CHUNKS = BM * BK / 4 / kThreads;
  static constexpr int B_CHUNKS = BN * BK / 4 / kThreads;
  static_assert(A_CHUNKS * 4 * kThreads == BM * BK && B_CHUNKS * 4 * kThreads == BN * BK, "even split");
};

// LDS geometry of one operand: row-major [rows][k] (KMAJ=false) or [k][rows] (KMAJ=true).
template <int ROWS, int BK, bool KMAJ>
struct OperandLds {
  static constexpr int LD = KMAJ ? ROWS + 4 : BK + 4;   // floats per LDS row (16-byte aligned)
  static constexpr int FLOATS = (KMAJ ? BK : ROWS) * LD;
};

// Loads one BK-slice of an operand with ROWS rows (m or n) into registers.
// ROWMAJ_K = true: memory is [row][k] (k contiguous); false: memory is [k][row].
template <int ROWS, int BK, int CH, bool ROWMAJ_K>
__device__ __forceinline__ void g2_load(const float* base, int ld, int r0, int nrows, int k0, int kend, bool vec,
                                        f4 (&reg)[CH]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const int c = t + 256 * j;
    f4 v = {0.f, 0.f, 0.f, 0.f};
    if (ROWMAJ_K) {
      const int row = c / (BK / 4), kq = c % (BK / 4);
      const int r = r0 + row, k = k0 + kq * 4;
      if (r < nrows) {
        const float* p = base + (size_t)r * ld + k;
        if (vec && k + 3 < kend) {
          v = *reinterpret_cast<const f4*>(p);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) if (k + e < kend) v[e] = p[e];
        }
      }
    } else {
      const int krow = c / (ROWS / 4), rq = c % (ROWS / 4);
      const int k = k0 + krow, r = r0 + rq * 4;
      if (k < kend) {
        const float* p = base + (size_t)k * ld + r;
        if (vec && r + 3 < nrows) {
          v = *reinterpret_cast<const f4*>(p);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) if (r + e < nrows) v[e] = p[e];
        }
      }
    }
    reg[j] = v;
  }
}

// Copies the registers of g2_load into LDS in the operand's staging layout (both
// layouts receive the 4-vector unchanged: [row][k..k+3] or [k][row..row+3]).
template <int ROWS, int BK, int CH, bool ROWMAJ_K>
__device__ __forceinline__ void g2_store(float* lds, const f4 (&reg)[CH]) {
  using L = OperandLds<ROWS, BK, !ROWMAJ_K>;
  const int t = threadIdx.x;
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const int c = t + 256 * j;
    if (ROWMAJ_K) {
      const int row = c / (BK / 4), kq = c % (BK / 4);
      *reinterpret_cast<f4*>(lds + row * L::LD + kq * 4) = reg[j];
    } else {
      const int krow = c / (ROWS / 4), rq = c % (ROWS / 4);
      *reinterpret_cast<f4*>(lds + krow * L::LD + rq * 4) = reg[j];
    }
  }
}

// Reads the 4 k-values kb+kk..kb+kk+3 of operand row `row` for this lane.
template <int ROWS, int BK, bool KMAJ>
__device__ __forceinline__ f4 g2_read(const float* lds, int row, int k) {
  using L = OperandLds<ROWS, BK, KMAJ>;
  if (!KMAJ) return *reinterpret_cast<const f4*>(lds + row * L::LD + k);
  f4 v;
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = lds[(k + e) * L::LD + row];
  return v;
}

struct Gemm2Args {
  const float* A;
  const float* B;
  float* out;         // C (ldc) or split-K partials [split][M][N]
  const float* bias;  // [N] or null (store epilogue only)
  int M, N, K, lda, ldb, ldc;
  int k_per_split;
  int vec_a, vec_b;
  int tiles_m, tiles_n;
  int partial;        // 1: write partials (plane per blockIdx.z), no bias
};

template <class Cfg, bool TA, bool TB>
__global__ __launch_bounds__(256) void gemm2_kernel(Gemm2Args g) {
  constexpr bool AK = TA;    // A staged k-major when A is stored [K][M]
  constexpr bool BKM = !TB;  // B staged k-major when B is stored [K][N]
  using LA = OperandLds<Cfg::BM, Cfg::BK, AK>;
  using LB = OperandLds<Cfg::BN, Cfg::BK, BKM>;
  extern __shared__ float smem[];
  float* const as0 = smem;
  float* const as1 = smem + LA::FLOATS;
  float* const bs0 = smem + 2 * LA::FLOATS;
  float* const bs1 = smem + 2 * LA::FLOATS + LB::FLOATS;

  int tm, tn;
  {
    const int total = g.tiles_m * g.tiles_n;
    int id = blockIdx.x;
    if (total % 8 == 0) id = (id % 8) * (total / 8) + id / 8;  // contiguous tiles per XCD
    tm = id / g.tiles_n;
    tn = id % g.tiles_n;
  }
  const int m0 = tm * Cfg::BM, n0 = tn * Cfg::BN;
  const int kbeg = blockIdx.z * g.k_per_split;
  const int kend = min(g.K, kbeg + g.k_per_split);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int half = lane >> 5, r32 = lane & 31;

  f16v acc[Cfg::FM][Cfg::FN];
  double acc64[Cfg::ACC64 ? Cfg::FM : 1][Cfg::ACC64 ? Cfg::FN : 1][Cfg::ACC64 ? 16 : 1];
#pragma unroll
  for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
    for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        acc[i][j][r] = 0.f;
        if (Cfg::ACC64) acc64[Cfg::ACC64 ? i : 0][Cfg::ACC64 ? j : 0][Cfg::ACC64 ? r : 0] = 0.0;
      }

  f4 ra[Cfg::A_CHUNKS], rb[Cfg::B_CHUNKS];
  const int nk = (kend - kbeg + Cfg::BK - 1) / Cfg::BK;
  if (nk > 0) {
    g2_load<Cfg::BM, Cfg::BK, Cfg::A_CHUNKS, !TA>(g.A, g.lda, m0, g.M, kbeg, kend, g.vec_a, ra);
    g2_load<Cfg::BN, Cfg::BK, Cfg::B_CHUNKS, TB>(g.B, g.ldb, n0, g.N, kbeg, kend, g.vec_b, rb);
    g2_store<Cfg::BM, Cfg::BK, Cfg::A_CHUNKS, !TA>(as0, ra);
    g2_store<Cfg::BN, Cfg::BK, Cfg::B_CHUNKS, TB>(bs0, rb);
  }
  __syncthreads();
  for (int it = 0; it < nk; ++it) {
    const int cur = it & 1;
    const bool more = it + 1 < nk;
    if (more) {  // next slice into registers while this one is multiplied
      const int k1 = kbeg + (it + 1) * Cfg::BK;
      g2_load<Cfg::BM, Cfg::BK, Cfg::A_CHUNKS, !TA>(g.A, g.lda, m0, g.M, k1, kend, g.vec_a, ra);
      g2_load<Cfg::BN, Cfg::BK, Cfg::B_CHUNKS, TB>(g.B, g.ldb, n0, g.N, k1, kend, g.vec_b, rb);
    }
    const float* as = cur ? as1 : as0;
    const float* bs = cur ? bs1 : bs0;
    const int kb = half * Cfg::KH;
#pragma unroll
    for (int kk = 0; kk < Cfg::KH; kk += 4) {
      f4 av[Cfg::FM], bv[Cfg::FN];
#pragma unroll
      for (int i = 0; i < Cfg::FM; ++i) av[i] = g2_read<Cfg::BM, Cfg::BK, AK>(as, wm * Cfg::TM + i * 32 + r32, kb + kk);
#pragma unroll
      for (int j = 0; j < Cfg::FN; ++j) bv[j] = g2_read<Cfg::BN, Cfg::BK, BKM>(bs, wn * Cfg::TN + j * 32 + r32, kb + kk);
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
          for (int j = 0; j < Cfg::FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][e], bv[j][e], acc[i][j], 0, 0, 0);
    }
    if (Cfg::ACC64) {
#pragma unroll
      for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
        for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            acc64[Cfg::ACC64 ? i : 0][Cfg::ACC64 ? j : 0][Cfg::ACC64 ? r : 0] += (double)acc[i][j][r];
            acc[i][j][r] = 0.f;
          }
    }
    if (more) {  // the other buffer was last read in the previous slice, before the barrier below
      g2_store<Cfg::BM, Cfg::BK, Cfg::A_CHUNKS, !TA>(cur ? as0 : as1, ra);
      g2_store<Cfg::BN, Cfg::BK, Cfg::B_CHUNKS, TB>(cur ? bs0 : bs1, rb);
    }
    __syncthreads();
  }

  // epilogue straight from the fragments
  float* outp = g.partial ? g.out + (size_t)blockIdx.z * g.M * g.N : g.out;
  const int ldo = g.partial ? g.N : g.ldc;
#pragma unroll
  for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
    for (int j = 0; j < Cfg::FN; ++j) {
      const int n = n0 + wn * Cfg::TN + j * 32 + r32;
      if (n >= g.N) continue;
      const float bval = (!g.partial && g.bias) ? g.bias[n] : 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * Cfg::TM + i * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
        if (m < g.M) {
          const float v = Cfg::ACC64 ? (float)acc64[Cfg::ACC64 ? i : 0][Cfg::ACC64 ? j : 0][Cfg::ACC64 ? r : 0]
                                     : acc[i][j][r];
          outp[(size_t)m * ldo + n] = v + bval;
        }
      }
    }
}

template <class Cfg, bool TA, bool TB>
constexpr size_t gemm2_lds_bytes() {
  return sizeof(float) * 2 * (OperandLds<Cfg::BM, Cfg::BK, TA>::FLOATS + OperandLds<Cfg::BN, Cfg::BK, !TB>::FLOATS);
}

template <class Cfg>
inline int gemm2_split_layout(int K, int splits, int* kps_out) {
  if (splits < 1) splits = 1;
  int kps = (K + splits - 1) / splits;
  kps = (kps + Cfg::BK - 1) / Cfg::BK * Cfg::BK;
  if (kps < Cfg::BK) kps = Cfg::BK;
  *kps_out = kps;
  const int n = (K + kps - 1) / kps;
  return n < 1 ? 1 : n;
}

// Launches C = op(A) op(B) (+bias) directly (splits == 1) or the split-K partials
// (partial != nullptr, planes [splits][M][N]); returns the splits used in *used.
template <class Cfg, bool TA, bool TB>
inline int launch_gemm2(const float* A, const float* B, const float* bias, float* C, float* partial, int M, int N,
                        int K, int lda, int ldb, int ldc, int splits, int vec_a, int vec_b, hipStream_t s,
                        int* used) {
  Gemm2Args g{};
  g.A = A;
  g.B = B;
  g.bias = bias;
  g.M = M;
  g.N = N;
  g.K = K;
  g.lda = lda;
  g.ldb = ldb;
  g.ldc = ldc;
  g.vec_a = vec_a;
  g.vec_b = vec_b;
  g.tiles_m = (M + Cfg::BM - 1) / Cfg::BM;
  g.tiles_n = (N + Cfg::BN - 1) / Cfg::BN;
  const int n = gemm2_split_layout<Cfg>(K, partial ? splits : 1, &g.k_per_split);
  g.partial = partial ? 1 : 0;
  g.out = partial ? partial : C;
  if (used) *used = n;
  dim3 grid(g.tiles_m * g.tiles_n, 1, n);
  const size_t lds = gemm2_lds_bytes<Cfg, TA, TB>();
  hipLaunchKernelGGL((gemm2_kernel<Cfg, TA, TB>), grid, dim3(256), lds, s, g);
  HSL_HIP(hipGetLastError());
  return HSL_OK;
}

}  // namespace hsl
