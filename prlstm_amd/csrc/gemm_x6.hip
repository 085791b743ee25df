// Large fp32 products on the 16-bit matrix cores, in two layouts:
//  * C[M,N] = A[M,K] . B[N,K]^T (+ bias[N]): the input projection x W_ih^T + b_ih
//    (_torch.py:96, _parallel.py:56) of parallel mode and of the per-step path;
//  * C[M,N] = A[K,M]^T . B[K,N]: the weight gradients dgates^T h and dgates^T x over
//    K = T*B (_torch.py:157-162, and autograd's in parallel mode), and C[M,N] = A[M,K] .
//    B[K,N]: dx = dgates W_ih (K = 4H); both summed as fp32 runs of 64 k folded into a
//    second fp32 accumulator, split along K into planes of at most kSplitLongKRun (2048) k each that are
//    added in fp64 (splitk_reduce, or the caller's own fp64 finalisation) -- the accuracy
//    that the fp32 kernel gets from folding its accumulators into fp64 registers, which the
//    8-wave tile has no room for.
//
// Products run on the exact three-way bf16 split of split_bf16.h (the six largest piece
// products, fp32 accumulation).  Every instruction adds 16 exact products to the
// accumulator, so a 16-deep k-step takes 6 accumulator roundings where
// v_mfma_f32_32x32x2_f32 takes 8, and the error against fp64 is that of the fp32 MFMA
// product (checked side by side in the GPU tests).  One 32x32x16 bf16 instruction issues
// every 16 ns per SIMD against 30 ns for 32x32x2 f32 (measured), so the six products of a
// k-step take 2.5x less matrix-core time than fp32.
//
// Non-finite operands: a piece product of an infinite piece with a zero or opposite-signed
// piece of the other operand is NaN, so IEEE infinities cannot survive the split.  The
// rule is therefore simple: a non-finite element of A makes its row of C NaN, one of B
// its column (v - v0 is NaN or infinite, and so are the later pieces); a finite value
// beyond the bf16 range (|v| > 3.3895e38) rounds to v0 = +-inf and counts as non-finite.
// hsl_set_split_products(0) gives the IEEE results of the fp32 instruction instead.
//
// Workgroup = 8 waves.  The projection uses 256 x 256 tiles (2 x 4 waves of 128 x 64, i.e.
// 4 x 2 fragments of 32 x 32); the long-K products use 256 x 128 tiles (4 x 2 waves of
// 64 x 64), which leave registers for the second accumulator.  One k-slice is 16 deep.  The
// fp32 operands of slice s+2 are requested while slice s multiplies; the registers of slice
// s+1 are split into the three bf16 pieces and written to the other LDS buffer
// ([piece][row][k], 48-byte rows, conflict-free 128-bit fragment reads) in between this
// slice's products (scheduling groups), then one barrier.  The loop body has no branches:
// the last slices store and request a repeat of the last slice, so the compiler can
// interleave the split with the products.  The output is written with non-temporal stores
// (it is read back only by later kernels), which keeps the operand panels in L2.
// Shapes with partial tiles (or operands without 16-byte alignment) launch a second
// instance that reads element-wise from clamped addresses and zeroes what lies outside.
// A row-contiguous operand ([k][row]) is loaded as k-rows of four rows per thread and
// written transposed, each row's k-pair as one 32-bit word per piece.  A bf16 B operand
// (a half-precision module's x or W_ih) is its own single piece: only it is staged and
// three products per k-step are issued (X6OperandB16).
#include <type_traits>

#include "gemm_core.h"
#include "split_bf16.h"

namespace hsl {
namespace {


constexpr int kBK = 16;                    // k per slice
constexpr int kThreads = 512;              // 8 waves
constexpr int kLDK = kBK + 8;              // LDS row stride in bf16 elements (48 bytes)

// Tile shape: BM x BN with WM x WN waves; FOLD > 0 adds the MFMA accumulators into a
// second fp32 accumulator every FOLD slices (so no accumulator rounding happens at the
// magnitude of a long running sum more than once per FOLD slices).
template <int BM_, int BN_, int WM_, int WN_, int FOLD_>
struct X6Shape {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, FOLD = FOLD_;
  static constexpr int TM = BM / WM, TN = BN / WN, FM = TM / 32, FN = TN / 32;
  static constexpr int PA = BM * kLDK, PB = BN * kLDK;  // one piece of A / of B
  static constexpr int BUF = 3 * (PA + PB);             // pieces 0-2 of A, then of B
  static constexpr size_t LDS = 2 * BUF * sizeof(unsigned short);
  static_assert(WM * WN * 64 == kThreads && TM % 32 == 0 && TN % 32 == 0, "wave layout");
  static_assert(LDS <= 160 * 1024, "LDS");
};
// x W^T: 256 x 256 tiles, 8 waves of 128 x 64
using ShapeProj = X6Shape<256, 256, 2, 4, 0>;
// A^T B: 256 x 128 tiles, 8 waves of 64 x 64, folded every 4 slices (64 k)
using ShapeWgrad = X6Shape<256, 128, 4, 2, 4>;

struct X6Args {
  const float* A;
  const float* B;
  const float* bias;  // [N] or null (direct output only)
  float* out;         // C (ldc) or split-K partial planes [split][M][N]
  int M, N, K, lda, ldb, ldc;
  int kps;            // k per split (a multiple of kBK)
  int partial;
  int tiles_m, tiles_n;
  int out_vec;  // output base and row stride 16-byte aligned (and the bias, if any)
  // Weight-gradient finalisation in the epilogue (direct output, staged path only): with
  // dotw != null, every row of C is scaled by rs[row / rs_rows] (a tile's rows share one
  // group) and each wave adds up dotw . C (unscaled, fp64) over its part of the tile into
  // dotp[(tile_m * tiles_n + tile_n) * 8 + wave].
  const float* rs;
  int rs_rows;
  const float* dotw;
  double* dotp;
};


// The value of the neighbouring lane (lane ^ 1), by DPP quad permutation [1, 0, 3, 2].
__device__ __forceinline__ float swap_pair_lane(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));
}


// One operand's share of a ROWS x 16-k slice: L = ROWS / 128 16-byte loads per thread.
//  KC (k contiguous, [row][k]): load j of thread t is row c / 4, k-quad c % 4 of the
//      slice (c = t + 512 j); the split writes 8 bytes per piece.
//  !KC (row contiguous, [k][row]), ROWS = 256: thread t loads rows 4 (t / 8) .. +3 at
//      k-rows 2 (t % 8) and +1 and pairs the two k of each row (4 bytes per piece and row).
//  !KC, ROWS = 128: thread t loads rows 4 (t / 16) .. +3 at k-row t % 16; lanes t and t^1
//      swap half their values, so the even lane writes rows 0-1 and the odd lane rows 2-3,
//      each as (k even, k odd) pairs.
// `kend` bounds k (the end of this workgroup's split): masked loads zero k >= kend and
// rows >= rows, reading clamped addresses.  NSET register sets hold loaded slices (N sets
// let a slice be requested N iterations before it is stored).
template <bool FULL, bool KC, int ROWS, int NSET = 1>
struct X6Operand {
  static constexpr int L = ROWS * kBK / 4 / kThreads;
  static_assert(L == 1 || L == 2, "128 or 256 rows");
  static constexpr int kWrites = KC ? 3 * L : (L == 2 ? 12 : 6);  // LDS writes per store
  static constexpr int kLoads = L;
  const float* base;
  int ld, rows, kend;
  int r[L], k[L];  // KC: row and k of load j; !KC: r[0] = first row, k[0] = first k
  int so[L];       // LDS element offsets within one piece
  f4 vv[NSET][2];
  __device__ __forceinline__ void init(const float* b, int ld_, int r0, int rows_, int kbeg, int kend_) {
    base = b;
    ld = ld_;
    rows = rows_;
    kend = kend_;
    const int t = threadIdx.x;
    if constexpr (KC) {
#pragma unroll
      for (int j = 0; j < L; ++j) {
        const int c = t + kThreads * j;
        r[j] = r0 + c / (kBK / 4);
        k[j] = kbeg + (c % (kBK / 4)) * 4;
        so[j] = (c / (kBK / 4)) * kLDK + (c % (kBK / 4)) * 4;
      }
    } else if constexpr (L == 2) {
      r[0] = r0 + 4 * (t / 8);
      k[0] = kbeg + 2 * (t % 8);
      so[0] = 4 * (t / 8) * kLDK + 2 * (t % 8);
    } else {
      const int odd = t & 1;
      r[0] = r0 + 4 * (t / 16);
      k[0] = kbeg + t % 16;
      so[0] = (4 * (t / 16) + 2 * odd) * kLDK + (t % 16) - odd;
    }
  }
  __device__ __forceinline__ f4 load_rows(int kk) const {  // !KC: 4 rows at k-row kk
    if constexpr (FULL) {
      return *reinterpret_cast<const f4*>(base + (size_t)kk * ld + r[0]);
    } else {
      f4 x;
      const bool kok = kk < kend;
      const float* kp = base + (size_t)(kok ? kk : kend - 1) * ld;  // a k-row that exists
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rr = r[0] + i;
        const float e = kp[rr < rows ? rr : rows - 1];
        x[i] = (kok && rr < rows) ? e : 0.f;
      }
      return x;
    }
  }
  template <int SET>
  __device__ __forceinline__ void load(int slice) {
    f4 (&v)[2] = vv[SET];
    const int ks = slice * kBK;
    if constexpr (KC) {
#pragma unroll
      for (int j = 0; j < L; ++j) {
        const int kk0 = k[j] + ks;
        if constexpr (FULL) {
          v[j] = *reinterpret_cast<const f4*>(base + (size_t)r[j] * ld + kk0);
        } else {
          const bool rok = r[j] < rows;
          const float* rp = base + (size_t)(rok ? r[j] : rows - 1) * ld;  // a row that exists
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int kk = kk0 + e;
            const float x = rp[kk < kend ? kk : kend - 1];
            v[j][e] = (rok && kk < kend) ? x : 0.f;
          }
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < L; ++e) v[e] = load_rows(k[0] + ks + e);
    }
  }
  // the three pieces into LDS: piece q of this operand starts at p0 + q * ROWS * kLDK
  template <int SET>
  __device__ __forceinline__ void store(unsigned short* p0) const {
    const f4 (&v)[2] = vv[SET];
    constexpr int P = ROWS * kLDK;
    if constexpr (KC) {
#pragma unroll
      for (int j = 0; j < L; ++j) {
        unsigned lo[3], hi[3];
        split2(v[j][0], v[j][1], lo);
        split2(v[j][2], v[j][3], hi);
#pragma unroll
        for (int q = 0; q < 3; ++q) *reinterpret_cast<u32x2*>(p0 + q * P + so[j]) = u32x2{lo[q], hi[q]};
      }
    } else if constexpr (L == 2) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        unsigned pc[3];
        split2(v[0][i], v[1][i], pc);
#pragma unroll
        for (int q = 0; q < 3; ++q) *reinterpret_cast<unsigned*>(p0 + q * P + so[0] + i * kLDK) = pc[q];
      }
    } else {
      const bool odd = threadIdx.x & 1;
      // even lane (k even) keeps rows 0-1 and receives the odd lane's rows 0-1; the odd
      // lane keeps rows 2-3 and receives the even lane's rows 2-3
      const float x0 = swap_pair_lane(odd ? v[0][0] : v[0][2]);
      const float x1 = swap_pair_lane(odd ? v[0][1] : v[0][3]);
      const float a0 = odd ? x0 : v[0][0], b0 = odd ? v[0][2] : x0;
      const float a1 = odd ? x1 : v[0][1], b1 = odd ? v[0][3] : x1;
      unsigned p0c[3], p1c[3];
      split2(a0, b0, p0c);
      split2(a1, b1, p1c);
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        *reinterpret_cast<unsigned*>(p0 + q * P + so[0]) = p0c[q];
        *reinterpret_cast<unsigned*>(p0 + q * P + so[0] + kLDK) = p1c[q];
      }
    }
  }
};

// A bf16 B operand ([k][row], 128 rows; a half-precision module's x or W_ih): a bf16
// value is its own single piece, so only piece 0 is staged and the products with B's
// pieces 1 and 2 (zero for such values) are not issued.  Thread t loads rows
// 4 (t / 16) .. +3 at k-row t % 16 (8 bytes); lanes t and t^1 swap two of those rows, so
// the even lane writes rows 0-1 and the odd lane rows 2-3, each as a (k even, k odd) pair.
template <bool FULL, int NSET = 1>
struct X6OperandB16 {
  static constexpr int kWrites = 2, kLoads = 1;
  const unsigned short* base;
  int ld, rows, kend;
  int r0q, k0;  // first row of the thread's quad, its k-row offset
  int so;
  u32x2 vv[NSET];  // rows 0-1 and rows 2-3 of the quad, two bf16 each
  __device__ __forceinline__ void init(const float* b, int ld_, int r0, int rows_, int kbeg, int kend_) {
    base = reinterpret_cast<const unsigned short*>(b);
    ld = ld_;
    rows = rows_;
    kend = kend_;
    const int t = threadIdx.x, odd = t & 1;
    r0q = r0 + 4 * (t / 16);
    k0 = kbeg + t % 16;
    so = (4 * (t / 16) + 2 * odd) * kLDK + (t % 16) - odd;
  }
  template <int SET>
  __device__ __forceinline__ void load(int slice) {
    u32x2& v = vv[SET];
    const int kk = k0 + slice * kBK;
    if constexpr (FULL) {
      v = *reinterpret_cast<const u32x2*>(base + (size_t)kk * ld + r0q);
    } else {
      const bool kok = kk < kend;
      const unsigned short* kp = base + (size_t)(kok ? kk : kend - 1) * ld;  // a k-row that exists
      unsigned e[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rr = r0q + i;
        const unsigned x = kp[rr < rows ? rr : rows - 1];
        e[i] = (kok && rr < rows) ? x : 0u;
      }
      v = u32x2{e[0] | (e[1] << 16), e[2] | (e[3] << 16)};
    }
  }
  template <int SET>
  __device__ __forceinline__ void store(unsigned short* p0) const {  // piece 0 only
    const u32x2& v = vv[SET];
    const bool odd = threadIdx.x & 1;
    const unsigned recv =
        static_cast<unsigned>(__builtin_amdgcn_mov_dpp(static_cast<int>(odd ? v[0] : v[1]), 0xB1, 0xF, 0xF, false));
    const unsigned ke = odd ? recv : v[0];  // the two rows at the even k
    const unsigned ko = odd ? v[1] : recv;  // the same two rows at the odd k
    *reinterpret_cast<unsigned*>(p0 + so) = (ke & 0xFFFFu) | (ko << 16);
    *reinterpret_cast<unsigned*>(p0 + so + kLDK) = (ke >> 16) | (ko & 0xFFFF0000u);
  }
};

template <class S, bool FULL, bool AKC, bool BKC, int BP>
__device__ __forceinline__ void x6_tile(const X6Args& g, int m0, int n0, unsigned short* sm) {
  static_assert(BP == 3 || (BP == 1 && !BKC && S::BN == 128), "bf16 B: row-contiguous, 128 rows");
  // The long-K shape (FOLD) keeps three slices in registers: a slice is requested three
  // iterations before it is stored, since one iteration's products (24 per wave) are much
  // shorter than a load's latency under load (one set: configs[4] dW_ih at 38% MFMA busy,
  // waves waiting 54% of their cycles; two sets took configs[4] from 2.54 to 2.42 ms per
  // step, three to 2.42-2.43).  The projection shape has no registers to spare.
  constexpr int NSET = S::FOLD ? 3 : 1;
  using OpA = X6Operand<FULL, AKC, S::BM, NSET>;
  using OpB = std::conditional_t<BP == 1, X6OperandB16<FULL, NSET>, X6Operand<FULL, BKC, S::BN, NSET>>;
  constexpr int NPP = BP == 1 ? 3 : 6;  // piece products per k-step
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / S::WN, wn = wave % S::WN;
  const int half = lane >> 5, r32 = lane & 31;
  const int kbeg = blockIdx.z * g.kps;
  const int kend = min(g.K, kbeg + g.kps);
  OpA oa;
  OpB ob;
  oa.init(g.A, g.lda, m0, g.M, kbeg, kend);
  ob.init(g.B, g.ldb, n0, g.N, kbeg, kend);
  f16v acc[S::FM][S::FN];
  f16v tot[S::FOLD ? S::FM : 1][S::FOLD ? S::FN : 1];
#pragma unroll
  for (int i = 0; i < S::FM; ++i)
#pragma unroll
    for (int j = 0; j < S::FN; ++j) {
      acc[i][j] = f16v{};
      if constexpr (S::FOLD) tot[i][j] = f16v{};
    }

  const int nk = (kend - kbeg + kBK - 1) / kBK;
  // slice s lives in register set s % NSET from its load to its store
  oa.template load<0>(0);
  ob.template load<0>(0);
  oa.template store<0>(sm);
  ob.template store<0>(sm + 3 * S::PA);
  oa.template load<1 % NSET>(min(1, nk - 1));
  ob.template load<1 % NSET>(min(1, nk - 1));
  if constexpr (NSET >= 2) {
    oa.template load<2 % NSET>(min(2, nk - 1));
    ob.template load<2 % NSET>(min(2, nk - 1));
  }
  if constexpr (NSET >= 3) {
    oa.template load<0>(min(3, nk - 1));
    ob.template load<0>(min(3, nk - 1));
  }
  __syncthreads();
  const int arow = (wm * S::TM + r32) * kLDK + 8 * half, brow = (wn * S::TN + r32) * kLDK + 8 * half;
  // iteration it: products of slice it (LDS buffer it&1), slice it+1 from register set SET
  // into the other buffer, slice it+NSET+1 requested into SET
  auto iteration = [&](int it, auto setc) __attribute__((always_inline)) {
    constexpr int SET = decltype(setc)::value;
    const unsigned short* base = sm + (it & 1) * S::BUF;
    u32x4 fa[3][S::FM], fb[3][S::FN];
#pragma unroll
    for (int q = 0; q < 3; ++q) {
#pragma unroll
      for (int i = 0; i < S::FM; ++i)
        fa[q][i] = *reinterpret_cast<const u32x4*>(base + q * S::PA + arow + 32 * i * kLDK);
      if (q < BP) {
#pragma unroll
        for (int j = 0; j < S::FN; ++j)
          fb[q][j] = *reinterpret_cast<const u32x4*>(base + 3 * S::PA + q * S::PB + brow + 32 * j * kLDK);
      }
    }
    // slice it+1 into the other buffer (its last reads were before the previous barrier)
    {
      unsigned short* const dstb = sm + ((it & 1) ^ 1) * S::BUF;
      oa.template store<SET>(dstb);
      ob.template store<SET>(dstb + 3 * S::PA);
    }
    const int nxt = min(it + NSET + 1, nk - 1);
    oa.template load<SET>(nxt);
    ob.template load<SET>(nxt);
#pragma unroll
    for (int pp = 0; pp < NPP; ++pp) {
      // one-piece B: (a0, b), (a1, b), (a2, b) -- the non-zero terms of the six-product
      // order, in that order, so the sums equal the split path's bit for bit
      const int qa = BP == 1 ? pp : kPa[pp], qb = BP == 1 ? 0 : kPb[pp];
#pragma unroll
      for (int i = 0; i < S::FM; ++i)
#pragma unroll
        for (int j = 0; j < S::FN; ++j) acc[i][j] = mfma_bf16(fa[qa][i], fb[qb][j], acc[i][j]);
    }
    if constexpr (FULL) {
      // fragment reads first; then A's split and LDS writes, with one product each (the
      // fragments are still arriving), and A's next loads as soon as those writes have
      // freed its registers, a whole iteration before their use (A streams from memory);
      // then B's writes with the other products between them, B's loads (B is mostly a
      // cache-resident weight), the rest of the products
      constexpr int kMfma = NPP * S::FM * S::FN;
      constexpr int kWA = OpA::kWrites, kWB = OpB::kWrites;
      constexpr int kValuA = 28 * OpA::kLoads, kValuB = 28 * OpB::kLoads;
      constexpr int kMfmaB = (kMfma - kWA + kWB - 1) / kWB;
      __builtin_amdgcn_sched_group_barrier(0x100, 3 * (S::FM + S::FN), 0);
#pragma unroll
      for (int w = 0; w < kWA; ++w) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, (kValuA + kWA - 1) / kWA, 0);
        __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x020, OpA::kLoads, 0);
#pragma unroll
      for (int w = 0; w < kWB; ++w) {
        __builtin_amdgcn_sched_group_barrier(0x008, kMfmaB, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, (kValuB + kWB - 1) / kWB, 0);
        __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x020, OpB::kLoads, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, kMfma, 0);
    }
    __syncthreads();
    if constexpr (S::FOLD) {
      if ((it + 1) % S::FOLD == 0 || it + 1 == nk) {
#pragma unroll
        for (int i = 0; i < S::FM; ++i)
#pragma unroll
          for (int j = 0; j < S::FN; ++j) {
            tot[i][j] += acc[i][j];
            acc[i][j] = f16v{};
          }
      }
    }
  };
  if constexpr (NSET == 1) {
    for (int it = 0; it < nk; ++it) iteration(it, std::integral_constant<int, 0>{});
  } else if constexpr (NSET == 2) {
    for (int it = 0; it < nk; it += 2) {
      iteration(it, std::integral_constant<int, 1>{});
      if (it + 1 < nk) iteration(it + 1, std::integral_constant<int, 0>{});
    }
  } else {
    // whole trips of three in the loop, the rest after it: an iteration skipped inside the
    // loop would leave a path on which fewer loads were issued, and the compiler's wait
    // before the first store of a trip then counts for that path (waiting for the loads
    // of the previous iteration instead of those of three iterations back)
    int it = 0;
    for (; it + 3 <= nk; it += 3) {
      iteration(it, std::integral_constant<int, 1>{});
      iteration(it + 1, std::integral_constant<int, 2>{});
      iteration(it + 2, std::integral_constant<int, 0>{});
    }
    if (it < nk) iteration(it, std::integral_constant<int, 1>{});
    if (it + 1 < nk) iteration(it + 1, std::integral_constant<int, 2>{});
  }

  float* outp = g.partial ? g.out + (size_t)blockIdx.z * g.M * g.N : g.out;
  const int ldo = g.partial ? g.N : g.ldc;
  if constexpr (FULL) {
    if (g.out_vec) {
      // Rows through LDS, written as 16-byte stores: a lane of the product layout holds
      // one column of 16 rows, so direct stores are 4 bytes each (128 per lane for a
      // 256x256 tile) and a wave cannot have more than 63 in flight; it then waits for
      // stores before it can issue the next.  Each wave stages its 32-row slab of each
      // 32-row block (32 x TN floats) in its own LDS region (the operand buffers, free
      // after the last slice's barrier) and reads it back as rows: 16 lanes per 256-byte
      // row segment, 4 rows per instruction, TN/16 instructions per slab.
      static_assert(S::TN == 64, "16 lanes x 4 columns per slab row");
      constexpr int kLds = S::TN + 4;  // padded slab row (floats)
      static_assert(8 * 32 * kLds * sizeof(float) <= S::LDS, "slabs fit the operand buffers");
      float* const slab = reinterpret_cast<float*>(sm) + wave * 32 * kLds;
      const int rl = lane >> 4, cl = 4 * (lane & 15);
      const int nb = n0 + wn * S::TN + cl;
      const f4 bv = (!g.partial && g.bias) ? *reinterpret_cast<const f4*>(g.bias + nb) : f4{0.f, 0.f, 0.f, 0.f};
      const bool fin = g.dotw != nullptr;  // uniform
      const float sc = fin ? g.rs[m0 / g.rs_rows] : 1.f;
      double dacc = 0.0;
#pragma unroll
      for (int i = 0; i < S::FM; ++i) {
        // the dot operand's rows of this slab, requested before the slab goes through LDS
        f4 wv[8];
        if (fin) {
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            const int m = m0 + wm * S::TM + i * 32 + 4 * q + rl;
            wv[q] = *reinterpret_cast<const f4*>(g.dotw + (size_t)m * ldo + nb);
          }
        }
#pragma unroll
        for (int j = 0; j < S::FN; ++j) {
          const f16v& res = S::FOLD ? tot[S::FOLD ? i : 0][S::FOLD ? j : 0] : acc[i][j];
#pragma unroll
          for (int r = 0; r < 16; ++r) slab[(8 * (r >> 2) + 4 * half + (r & 3)) * kLds + 32 * j + r32] = res[r];
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const int row = 4 * q + rl;
          f4 v = *reinterpret_cast<const f4*>(&slab[row * kLds + cl]) + bv;
          if (fin) {
#pragma unroll
            for (int e = 0; e < 4; ++e) dacc += (double)wv[q][e] * (double)v[e];
            v = v * sc;
          }
          const int m = m0 + wm * S::TM + i * 32 + row;
          __builtin_nontemporal_store(v, reinterpret_cast<f4*>(outp + (size_t)m * ldo + nb));
        }
      }
      if (fin) {
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) dacc += __shfl_xor(dacc, off);
        if (lane == 0) g.dotp[((size_t)(m0 / S::BM) * g.tiles_n + n0 / S::BN) * 8 + wave] = dacc;
      }
      return;
    }
  }
#pragma unroll
  for (int i = 0; i < S::FM; ++i)
#pragma unroll
    for (int j = 0; j < S::FN; ++j) {
      const int n = n0 + wn * S::TN + j * 32 + r32;
      if (!FULL && n >= g.N) continue;
      const float bval = (!g.partial && g.bias) ? g.bias[n] : 0.f;
      const f16v& res = S::FOLD ? tot[S::FOLD ? i : 0][S::FOLD ? j : 0] : acc[i][j];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * S::TM + i * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
        if (FULL || m < g.M) __builtin_nontemporal_store(res[r] + bval, outp + (size_t)m * ldo + n);
      }
    }
}

// FULL: every tile lies inside the matrices and every split is a whole number of slices
// (M, N multiples of the tile, K and the split length of 16, aligned operands); chosen
// per launch, so the unmasked kernel carries no edge code.  AKC / BKC: operand k-contiguous.
template <class S, bool FULL, bool AKC, bool BKC, int BP>
__global__ __launch_bounds__(kThreads) void gemm_x6_kernel(X6Args g) {
  extern __shared__ unsigned short x6_smem[];
  int tm, tn;
  if constexpr (S::FOLD) {
    // long-K products: each XCD (workgroup i runs on XCD i % 8) takes a contiguous range of
    // the tiles in row-major order, so the column tiles that share a panel of the long
    // operand A run side by side on one XCD and read it from its L2 once
    const int total = g.tiles_m * g.tiles_n;
    int id = blockIdx.x;
    if (total % 8 == 0) id = (id % 8) * (total / 8) + id / 8;
    tm = id / g.tiles_n;
    tn = id % g.tiles_n;
  } else {
    gemm_tile_order(g.tiles_m, g.tiles_n, &tm, &tn);
  }
  x6_tile<S, FULL, AKC, BKC, BP>(g, tm * S::BM, tn * S::BN, x6_smem);
}

template <class S, bool AKC, bool BKC, int BP = 3>
void x6_launch(X6Args g, bool vec, int splits, hipStream_t s) {
  g.tiles_m = (g.M + S::BM - 1) / S::BM;
  g.tiles_n = (g.N + S::BN - 1) / S::BN;
  const bool full = vec && g.M % S::BM == 0 && g.N % S::BN == 0 && g.K % kBK == 0 && g.kps % kBK == 0;
  const dim3 grid(g.tiles_m * g.tiles_n, 1, splits);
  if (full)
    hipLaunchKernelGGL((gemm_x6_kernel<S, true, AKC, BKC, BP>), grid, dim3(kThreads), S::LDS, s, g);
  else
    hipLaunchKernelGGL((gemm_x6_kernel<S, false, AKC, BKC, BP>), grid, dim3(kThreads), S::LDS, s, g);
}

}  // namespace

namespace {
// tiles of C = A B^T in a shape's tiling
template <class S>
long x6_tiles(int M, int N) {
  return (long)((M + S::BM - 1) / S::BM) * ((N + S::BN - 1) / S::BN);
}
}  // namespace

bool gemm_x6_applies(int M, int N, int K) {
  // one tile per CU at least (256 x 256, or else 256 x 128), and enough k to amortise the
  // tile's setup
  return (x6_tiles<ShapeProj>(M, N) >= 256 || x6_tiles<ShapeWgrad>(M, N) >= 256) && K >= 32;
}

int gemm_x6_longk_splits(int M, int N, int K) {
  // C = A^T B (weight gradients, K = T*B) or C = A B (dx = dgates W_ih, K = 4H): at least
  // one tile each way and >= 8 GFLOP.
  // Splits fill the chip (one workgroup per CU) and keep every split to at most kSplitLongKRun k,
  // summed inside the kernel as fp32 runs of 64 k (FOLD); the planes are added in fp64.
  using S = ShapeWgrad;
  if (M < S::BM || N < S::BN || K < 2 * kBK || 2.0 * M * N * K < 8e9) return 0;
  const long tiles = (long)((M + S::BM - 1) / S::BM) * ((N + S::BN - 1) / S::BN);
  long s = (256 + tiles - 1) / tiles;
  const long by_run = (K + kSplitLongKRun - 1) / kSplitLongKRun;
  if (by_run > s) s = by_run;
  if (s > K / kBK) s = K / kBK;
  if (s > 64) s = 64;
  return s < 1 ? 1 : (int)s;
}

int gemm_x6_wgrad_fin(const float* A, const float* B, float* C, const float* a_group, int group_rows,
                      const float* W, double* dotp, size_t dotp_cap, int M, int N, int K, int lda, int ldb, int ldc,
                      hipStream_t s, int* parts) {
  // A^T B on one split of whole 256 x 128 tiles, aligned rows, tiles within one row group
  using S = ShapeWgrad;
  *parts = 0;
  if (!split_products_mode() || gemm_x6_longk_splits(M, N, K) != 1) return HSL_OK;
  if (M % S::BM || N % S::BN || K % kBK || group_rows <= 0 || group_rows % S::BM) return HSL_OK;
  if (!aligned16(A) || !aligned16(B) || !aligned16(C) || !aligned16(W) || lda % 4 || ldb % 4 || ldc % 4) return HSL_OK;
  const size_t n = (size_t)(M / S::BM) * (N / S::BN) * 8;
  if (!dotp || n > dotp_cap) return HSL_OK;
  X6Args g{};
  g.A = A;
  g.B = B;
  g.out = C;
  g.M = M;
  g.N = N;
  g.K = K;
  g.lda = lda;
  g.ldb = ldb;
  g.ldc = ldc;
  g.kps = K;
  g.out_vec = 1;
  g.rs = a_group;
  g.rs_rows = group_rows;
  g.dotw = W;
  g.dotp = dotp;
  x6_launch<S, false, false>(g, true, 1, s);
  HSL_HIP(hipGetLastError());
  *parts = (int)(n / (M / group_rows));
  return HSL_OK;
}

int gemm_x6_run(const float* A, const void* B, const float* bias, float* C, float* partial, int M, int N, int K,
                int lda, int ldb, int ldc, int trans_a, int trans_b, int splits, hipStream_t s, int* used, int b_bf16) {
  if (M <= 0 || N <= 0 || K <= 0) return fail(HSL_ERR_ARG, "gemm_x6: empty product");
  if (trans_a && trans_b) return fail(HSL_ERR_ARG, "gemm_x6: layout not supported");
  if (b_bf16 && trans_b) return fail(HSL_ERR_ARG, "gemm_x6: a bf16 B must be [K][N] (trans_b = 0)");
  if (splits < 1 || (splits > 1 && !partial)) splits = 1;
  X6Args g{};
  g.A = A;
  g.B = static_cast<const float*>(B);  // bf16 data when b_bf16 (read as such by X6OperandB16)
  g.bias = partial ? nullptr : bias;
  g.out = partial ? partial : C;
  g.partial = partial ? 1 : 0;
  g.M = M;
  g.N = N;
  g.K = K;
  g.lda = lda;
  g.ldb = ldb;
  g.ldc = ldc;
  int kps = (K + splits - 1) / splits;
  kps = (kps + kBK - 1) / kBK * kBK;
  g.kps = kps;
  const int n = (K + kps - 1) / kps;
  if (used) *used = n;
  const bool vec = aligned16(A) && aligned16(B) && lda % 4 == 0 && ldb % 4 == 0;
  g.out_vec = aligned16(g.out) && (partial ? N % 4 == 0 : ldc % 4 == 0) && (g.bias == nullptr || aligned16(g.bias));
  if (b_bf16 && trans_a)
    x6_launch<ShapeWgrad, false, false, 1>(g, vec, n, s);  // dgates^T x with a bf16 x
  else if (b_bf16)
    x6_launch<ShapeWgrad, true, false, 1>(g, vec, n, s);  // dgates W_ih with a bf16 W_ih
  else if (!trans_a && trans_b && x6_tiles<ShapeProj>(M, N) >= 256)
    x6_launch<ShapeProj, true, true>(g, vec, n, s);  // x W^T: both operands k-contiguous
  else if (!trans_a && trans_b)
    x6_launch<ShapeWgrad, true, true>(g, vec, n, s);  // the same on 256 x 128 tiles (fewer than 256 of 256 x 256)
  else if (trans_a)
    x6_launch<ShapeWgrad, false, false>(g, vec, n, s);  // A^T B: both row-contiguous
  else
    x6_launch<ShapeWgrad, true, false>(g, vec, n, s);  // A B (dx = dgates W_ih): B row-contiguous
  HSL_HIP(hipGetLastError());
  return HSL_OK;
}

}  // namespace hsl
