// Third fp32 MFMA GEMM core for gfx950: the large products (input projection, weight
// gradients, dx) at full MFMA issue rate.
//
//   C[M,N] = op(A)[M,K] . op(B)[K,N]     (row-major, v_mfma_f32_32x32x2_f32 fragments)
//
// Workgroup = 4 waves (2 x 2), tile BM x BN, each wave a (BM/2) x (BN/2) block of 32x32
// fragments; LDS is double-buffered with one barrier per BK-slice.  The schedule of one
// slice is fixed with scheduling fences:
//
//   group 0     : the next slice's global loads are issued between the first MFMAs
//   groups 0..G : the LDS fragments of group g+1 are read while group g multiplies
//   group G/2   : the next slice's registers are written to the other LDS buffer,
//                 half a slice after they were requested
//   end         : one barrier
//
// so the MFMA pipe never waits on a global load or on the LDS copy.  Tiles that lie
// entirely inside the matrices (and 16-byte aligned operands) use unmasked 128-bit
// loads; edge tiles take the masked path of the same schedule.
//
// Operand staging: an operand whose k index is contiguous in memory is
// staged [row][k] and read as 128-bit k-runs with the half-wave k permutation (lanes
// 0-31 take k = kk + e, lanes 32-63 k = BK/2 + kk + e; A and B agree, so the sum is
// unchanged); an operand whose row index is contiguous is staged [k][row] and read with
// 32-bit loads of consecutive rows (conflict-free banks).  The epilogue writes straight
// from the accumulators: a fragment register holds 32 consecutive columns of one row
// across lanes 0-31 (and another row across lanes 32-63), i.e. 128-byte row segments.
//
// ACC64: the MFMA accumulators restart every FOLD slices and each restart adds them
// into fp64 registers (weight gradients: K = T*B summed as fp64 additions of
// FOLD*BK-term fp32 partials).
#pragma once

#include "gemm_core.h"

namespace hsl {

template <int BM_, int BN_, int BK_, bool ACC64_, int FOLD_ = 4>
struct Gemm3Cfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, FOLD = FOLD_;
  static constexpr bool ACC64 = ACC64_;
  static constexpr int kThreads = 256;
  static constexpr int TM = BM / 2, TN = BN / 2;
  static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile must be made of 32x32 fragments");
  static constexpr int FM = TM / 32, FN = TN / 32;
  static constexpr int KH = BK / 2;
  static constexpr int G = KH / 4;  // k-groups of 4 per half-wave per slice
  static_assert(KH % 4 == 0 && G >= 2, "at least two k-groups per slice");
  static constexpr int A_CHUNKS = BM * BK / 4 / kThreads;
  static constexpr int B_CHUNKS = BN * BK / 4 / kThreads;
  static_assert(A_CHUNKS * 4 * kThreads == BM * BK && B_CHUNKS * 4 * kThreads == BN * BK, "even split");
};

template <int ROWS, int BK, bool KCONT>
struct G3Lds {  // KCONT: staged [row][k]; else [k][row]
  static constexpr int LD = KCONT ? BK + 4 : ROWS + 4;
  static constexpr int FLOATS = (KCONT ? ROWS : BK) * LD;
};

struct Gemm3Args {
  const float* A;
  const float* B;
  float* out;         // C (ldc) or split-K partials [split][M][N]
  const float* bias;  // [N] or null
  int M, N, K, lda, ldb, ldc;
  int k_per_split;
  int vec;            // 1 when both operands allow 16-byte loads
  int tiles_m, tiles_n;
  int partial;
};

// One operand's per-thread global view: CH 16-byte chunks of a ROWS x BK slice.
template <int ROWS, int BK, int CH, bool KCONT>
struct G3Operand {
  const float* p[CH];  // chunk addresses at the current slice
  int row[CH];         // tile-relative row (KCONT) or k (row-contiguous) of the chunk
  int col[CH];         // tile-relative k (KCONT) or row of the chunk's first element
  __device__ __forceinline__ void init(const float* base, int ld, int r0, int k0) {
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int c = threadIdx.x + 256 * j;
      if (KCONT) {
        row[j] = c / (BK / 4);
        col[j] = (c % (BK / 4)) * 4;
        p[j] = base + (size_t)(r0 + row[j]) * ld + k0 + col[j];
      } else {
        row[j] = c / (ROWS / 4);
        col[j] = (c % (ROWS / 4)) * 4;
        p[j] = base + (size_t)(k0 + row[j]) * ld + r0 + col[j];
      }
    }
  }
  __device__ __forceinline__ void advance(int ld) {
#pragma unroll
    for (int j = 0; j < CH; ++j) p[j] += KCONT ? BK : (size_t)BK * ld;
  }
  // FULL: unmasked 16-byte loads.  Otherwise rows >= nrows and k >= kend read as 0
  // (r0, k0: the tile's first row and the slice's first k).
  template <bool FULL>
  __device__ __forceinline__ void load(f4 (&reg)[CH], int r0, int nrows, int k0, int kend, bool vec) const {
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      if (FULL) {
        reg[j] = *reinterpret_cast<const f4*>(p[j]);
      } else {
        f4 v = {0.f, 0.f, 0.f, 0.f};
        const int r = r0 + (KCONT ? row[j] : col[j]);
        const int k = k0 + (KCONT ? col[j] : row[j]);
        if (KCONT) {
          if (r < nrows) {
            if (vec && k + 3 < kend) {
              v = *reinterpret_cast<const f4*>(p[j]);
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e) if (k + e < kend) v[e] = p[j][e];
            }
          }
        } else {
          if (k < kend) {
            if (vec && r + 3 < nrows) {
              v = *reinterpret_cast<const f4*>(p[j]);
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e) if (r + e < nrows) v[e] = p[j][e];
            }
          }
        }
        reg[j] = v;
      }
    }
  }
  __device__ __forceinline__ void store(float* lds, const f4 (&reg)[CH]) const {
    using L = G3Lds<ROWS, BK, KCONT>;
#pragma unroll
    for (int j = 0; j < CH; ++j) *reinterpret_cast<f4*>(lds + row[j] * L::LD + col[j]) = reg[j];
  }
};

// The 4 k-values (k .. k+3 of this lane's half) of operand row `r` from LDS.
template <int ROWS, int BK, bool KCONT>
__device__ __forceinline__ f4 g3_read(const float* lds, int r, int k) {
  using L = G3Lds<ROWS, BK, KCONT>;
  if (KCONT) return *reinterpret_cast<const f4*>(lds + r * L::LD + k);
  f4 v;
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = lds[(k + e) * L::LD + r];
  return v;
}

template <class Cfg, bool TA, bool TB, bool FULL>
__device__ __forceinline__ void gemm3_tile(const Gemm3Args& g, int m0, int n0, int kbeg, int kend, float* smem) {
  constexpr bool AK = !TA;  // A k-contiguous ([M][K])
  constexpr bool BKc = TB;  // B k-contiguous ([N][K])
  using LA = G3Lds<Cfg::BM, Cfg::BK, AK>;
  using LB = G3Lds<Cfg::BN, Cfg::BK, BKc>;
  // buffers as integer offsets from smem: an indexed array of pointers would turn the
  // LDS accesses into flat ones
  constexpr int kBufA = LA::FLOATS, kB0 = 2 * LA::FLOATS, kBufB = LB::FLOATS;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int half = lane >> 5, r32 = lane & 31;
  const int arow = wm * Cfg::TM + r32, brow = wn * Cfg::TN + r32;
  const int kh = half * Cfg::KH;

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

  G3Operand<Cfg::BM, Cfg::BK, Cfg::A_CHUNKS, AK> oa;
  G3Operand<Cfg::BN, Cfg::BK, Cfg::B_CHUNKS, BKc> ob;
  oa.init(g.A, g.lda, m0, kbeg);
  ob.init(g.B, g.ldb, n0, kbeg);
  f4 ra[Cfg::A_CHUNKS], rb[Cfg::B_CHUNKS];
  const int nk = (kend - kbeg + Cfg::BK - 1) / Cfg::BK;
  if (nk > 0) {
    oa.template load<FULL>(ra, m0, g.M, kbeg, kend, g.vec);
    ob.template load<FULL>(rb, n0, g.N, kbeg, kend, g.vec);
    oa.store(smem, ra);
    ob.store(smem + kB0, rb);
  }
  __syncthreads();

  for (int it = 0; it < nk; ++it) {
    const int cur = it & 1;
    const bool more = it + 1 < nk;
    const float* la = smem + cur * kBufA;
    const float* lb = smem + kB0 + cur * kBufB;
    f4 av[2][Cfg::FM], bv[2][Cfg::FN];
#pragma unroll
    for (int i = 0; i < Cfg::FM; ++i) av[0][i] = g3_read<Cfg::BM, Cfg::BK, AK>(la, arow + 32 * i, kh);
#pragma unroll
    for (int j = 0; j < Cfg::FN; ++j) bv[0][j] = g3_read<Cfg::BN, Cfg::BK, BKc>(lb, brow + 32 * j, kh);
#pragma unroll
    for (int gi = 0; gi < Cfg::G; ++gi) {
      const int fb = gi & 1;
      if (gi + 1 < Cfg::G) {
#pragma unroll
        for (int i = 0; i < Cfg::FM; ++i)
          av[fb ^ 1][i] = g3_read<Cfg::BM, Cfg::BK, AK>(la, arow + 32 * i, kh + 4 * (gi + 1));
#pragma unroll
        for (int j = 0; j < Cfg::FN; ++j)
          bv[fb ^ 1][j] = g3_read<Cfg::BN, Cfg::BK, BKc>(lb, brow + 32 * j, kh + 4 * (gi + 1));
      }
      if (gi == 0 && more) {
        oa.advance(g.lda);
        ob.advance(g.ldb);
        const int k1 = kbeg + (it + 1) * Cfg::BK;
        oa.template load<FULL>(ra, m0, g.M, k1, kend, g.vec);
        ob.template load<FULL>(rb, n0, g.N, k1, kend, g.vec);
      }
      if (gi == Cfg::G / 2 && more) {
        oa.store(smem + (cur ^ 1) * kBufA, ra);
        ob.store(smem + kB0 + (cur ^ 1) * kBufB, rb);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
          for (int j = 0; j < Cfg::FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[fb][i][e], bv[fb][j][e], acc[i][j], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (Cfg::ACC64 && ((it + 1) % Cfg::FOLD == 0 || !more)) {
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
    __syncthreads();
  }

  float* outp = g.partial ? g.out + (size_t)blockIdx.z * g.M * g.N : g.out;
  const int ldo = g.partial ? g.N : g.ldc;
#pragma unroll
  for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
    for (int j = 0; j < Cfg::FN; ++j) {
      const int n = n0 + wn * Cfg::TN + j * 32 + r32;
      if (!FULL && n >= g.N) continue;
      const float bval = (!g.partial && g.bias) ? g.bias[n] : 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * Cfg::TM + i * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
        if (FULL || m < g.M) {
          const float v = Cfg::ACC64 ? (float)acc64[Cfg::ACC64 ? i : 0][Cfg::ACC64 ? j : 0][Cfg::ACC64 ? r : 0]
                                     : acc[i][j][r];
          outp[(size_t)m * ldo + n] = v + bval;
        }
      }
    }
}

template <class Cfg, bool TA, bool TB>
__global__ __launch_bounds__(256) void gemm3_kernel(Gemm3Args g) {
  extern __shared__ float smem[];
  int tm, tn;
  gemm_tile_order(g.tiles_m, g.tiles_n, &tm, &tn);
  const int m0 = tm * Cfg::BM, n0 = tn * Cfg::BN;
  const int kbeg = blockIdx.z * g.k_per_split;
  const int kend = min(g.K, kbeg + g.k_per_split);
  const bool full = g.vec && m0 + Cfg::BM <= g.M && n0 + Cfg::BN <= g.N && (kend - kbeg) % Cfg::BK == 0;
  if (full)
    gemm3_tile<Cfg, TA, TB, true>(g, m0, n0, kbeg, kend, smem);
  else
    gemm3_tile<Cfg, TA, TB, false>(g, m0, n0, kbeg, kend, smem);
}

template <class Cfg, bool TA, bool TB>
constexpr size_t gemm3_lds_bytes() {
  return sizeof(float) * 2 * (G3Lds<Cfg::BM, Cfg::BK, !TA>::FLOATS + G3Lds<Cfg::BN, Cfg::BK, TB>::FLOATS);
}

template <class Cfg>
inline int gemm3_split_layout(int K, int splits, int* kps_out) {
  if (splits < 1) splits = 1;
  int kps = (K + splits - 1) / splits;
  kps = (kps + Cfg::BK - 1) / Cfg::BK * Cfg::BK;
  if (kps < Cfg::BK) kps = Cfg::BK;
  *kps_out = kps;
  const int n = (K + kps - 1) / kps;
  return n < 1 ? 1 : n;
}

// C = op(A) op(B) (+bias) directly (partial == nullptr) or split-K partial planes
// [splits][M][N] (no bias); *used receives the planes written.
template <class Cfg, bool TA, bool TB>
inline int launch_gemm3(const float* A, const float* B, const float* bias, float* C, float* partial, int M, int N,
                        int K, int lda, int ldb, int ldc, int splits, int vec, hipStream_t s, int* used) {
  Gemm3Args g{};
  g.A = A;
  g.B = B;
  g.bias = bias;
  g.M = M;
  g.N = N;
  g.K = K;
  g.lda = lda;
  g.ldb = ldb;
  g.ldc = ldc;
  g.vec = vec;
  g.tiles_m = (M + Cfg::BM - 1) / Cfg::BM;
  g.tiles_n = (N + Cfg::BN - 1) / Cfg::BN;
  const int n = gemm3_split_layout<Cfg>(K, partial ? splits : 1, &g.k_per_split);
  g.partial = partial ? 1 : 0;
  g.out = partial ? partial : C;
  if (used) *used = n;
  dim3 grid(g.tiles_m * g.tiles_n, 1, n);
  hipLaunchKernelGGL((gemm3_kernel<Cfg, TA, TB>), grid, dim3(256), (gemm3_lds_bytes<Cfg, TA, TB>()), s, g);
  HSL_HIP(hipGetLastError());
  return HSL_OK;
}

}  // namespace hsl
