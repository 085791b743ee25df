// Large fp32 products C[M,N] = A[M,K] . B[N,K]^T (+ bias[N]) on the 16-bit matrix cores:
// the input projection x W_ih^T + b_ih (_torch.py:96, _parallel.py:56) of parallel mode and
// of the per-step path, and hsl_gemm_f32 calls of that layout.
//
// Exact three-way split.  Each fp32 value v is written as v = v0 + v1 + v2 with bf16
// pieces v0 = bf16(v) (round to nearest even), v1 = bf16(v - v0), v2 = v - v0 - v1.  The
// residuals are exact in fp32: v - v0 has at most 16 significant bits, so v2 has at most
// 8 and is itself a bf16 value; the split loses nothing.  A product a b is then the sum
// of the nine piece products a_i b_j, each exact in fp32 (8-bit by 8-bit significands).
// |a1|, |b1| <= 2^-8 and |a2|, |b2| <= 2^-16 of |a|, |b|, so the three smallest (a1 b2,
// a2 b1, a2 b2) add up to less than 2^-23 |a b| and are dropped; the other six run on
// v_mfma_f32_32x32x16_bf16 with fp32 accumulation.  This is the "bf16x6" product of
// Henry, Tang and Heinecke ("Leveraging the bfloat16 Artificial Intelligence Datatype
// For Higher-Precision Computations", ARITH 2019).  Every instruction adds 16 exact
// products to the accumulator, so a 16-deep k-step takes 6 accumulator roundings where
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
// Workgroup = 8 waves (2 x 4) on a 256 x 256 tile, each wave 128 x 64 (4 x 2 fragments
// of 32 x 32).  One k-slice is 16 deep.  The fp32 operands of slice s+2 are requested
// while slice s multiplies; the registers of slice s+1 are split into the three bf16
// pieces and written to the other LDS buffer ([piece][row][k], 48-byte rows, conflict-free
// 128-bit fragment reads) in between this slice's 48 products (scheduling groups), then
// one barrier.  The loop body has no branches: the last slices store and request a
// repeat of the last slice, so the compiler can interleave the split with the products.
// Shapes with partial tiles (or operands without 16-byte alignment) launch a second
// instance that reads element-wise from clamped addresses and zeroes what lies outside.
#include "gemm_core.h"

namespace hsl {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

constexpr int kBT = 256;                   // tile rows and columns
constexpr int kBK = 16;                    // k per slice
constexpr int kThreads = 512;              // 8 waves, 2 (rows) x 4 (columns)
constexpr int kWN = 4, kTM = 128, kTN = 64, kFM = kTM / 32, kFN = kTN / 32;
constexpr int kLDK = kBK + 8;              // LDS row stride in bf16 elements (48 bytes)
constexpr int kPiece = kBT * kLDK;         // one piece of one operand
constexpr int kBuf = 6 * kPiece;           // pieces 0-2 of A, then pieces 0-2 of B
constexpr int kCh = kBT * kBK / 4 / kThreads;  // 16-byte chunks per thread and operand
constexpr size_t kLdsBytes = 2 * kBuf * sizeof(unsigned short);
static_assert(kCh * 4 * kThreads == kBT * kBK, "even split of a slice");
static_assert(kLdsBytes <= 160 * 1024, "LDS");

struct X6Args {
  const float* A;
  const float* B;
  const float* bias;
  float* C;
  int M, N, K, lda, ldb, ldc;
  int vec;  // 16-byte loads legal (aligned bases, lda % 4 == 0, ldb % 4 == 0)
  int tiles_m, tiles_n;
};

__device__ __forceinline__ unsigned bf16_pair(float a, float b) {  // round to nearest even
  const bf16x2 h = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(unsigned, h);
}
__device__ __forceinline__ float low_half(unsigned u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float high_half(unsigned u) { return __uint_as_float(u & 0xFFFF0000u); }

// The three bf16 pieces of four consecutive values (two packed pairs each).
__device__ __forceinline__ void split4(f4 v, u32x2 (&p)[3]) {
  const unsigned h0 = bf16_pair(v[0], v[1]), h1 = bf16_pair(v[2], v[3]);
  const float r0 = v[0] - low_half(h0), r1 = v[1] - high_half(h0), r2 = v[2] - low_half(h1), r3 = v[3] - high_half(h1);
  const unsigned m0 = bf16_pair(r0, r1), m1 = bf16_pair(r2, r3);
  const float s0 = r0 - low_half(m0), s1 = r1 - high_half(m0), s2 = r2 - low_half(m1), s3 = r3 - high_half(m1);
  p[0] = u32x2{h0, h1};
  p[1] = u32x2{m0, m1};
  p[2] = u32x2{bf16_pair(s0, s1), bf16_pair(s2, s3)};
}

__device__ __forceinline__ f16v mfma_bf16(u32x4 a, u32x4 b, f16v c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                 0, 0);
}

// Pieces (of A, of B) of the six products.
constexpr int kPa[6] = {0, 0, 1, 0, 1, 2};
constexpr int kPb[6] = {0, 1, 0, 2, 1, 0};

// One operand's chunks: chunk j of this thread is row c / 4, k-quad c % 4 of the slice
// (c = tid + 512 j).
template <bool FULL>
struct X6Operand {
  const float* base;
  int ld, rows, K;
  int r[kCh], kq[kCh];
  __device__ __forceinline__ void init(const float* b, int ld_, int r0, int rows_, int K_) {
    base = b;
    ld = ld_;
    rows = rows_;
    K = K_;
#pragma unroll
    for (int j = 0; j < kCh; ++j) {
      const int c = threadIdx.x + kThreads * j;
      r[j] = r0 + c / (kBK / 4);
      kq[j] = (c % (kBK / 4)) * 4;
    }
  }
  __device__ __forceinline__ void load(f4 (&v)[kCh], int slice) const {
#pragma unroll
    for (int j = 0; j < kCh; ++j) {
      const int k = slice * kBK + kq[j];
      if constexpr (FULL) {
        v[j] = *reinterpret_cast<const f4*>(base + (size_t)r[j] * ld + k);
      } else {
        const bool rok = r[j] < rows;
        const float* rp = base + (size_t)(rok ? r[j] : rows - 1) * ld;  // a row that exists
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int kk = k + e;
          const float x = rp[kk < K ? kk : K - 1];
          v[j][e] = (rok && kk < K) ? x : 0.f;
        }
      }
    }
  }
};

template <bool FULL>
__device__ __forceinline__ void x6_tile(const X6Args& g, int m0, int n0, unsigned short* sm) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / kWN, wn = wave % kWN;
  const int half = lane >> 5, r32 = lane & 31;
  X6Operand<FULL> oa, ob;
  oa.init(g.A, g.lda, m0, g.M, g.K);
  ob.init(g.B, g.ldb, n0, g.N, g.K);
  int so[kCh];  // LDS element offset of chunk j within one piece
#pragma unroll
  for (int j = 0; j < kCh; ++j) {
    const int c = threadIdx.x + kThreads * j;
    so[j] = (c / (kBK / 4)) * kLDK + (c % (kBK / 4)) * 4;
  }
  f4 ga[kCh], gb[kCh];
  auto store = [&](int buf) __attribute__((always_inline)) {
    unsigned short* base = sm + buf * kBuf;
#pragma unroll
    for (int j = 0; j < kCh; ++j) {
      u32x2 pa[3], pb[3];
      split4(ga[j], pa);
      split4(gb[j], pb);
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        *reinterpret_cast<u32x2*>(base + q * kPiece + so[j]) = pa[q];
        *reinterpret_cast<u32x2*>(base + (3 + q) * kPiece + so[j]) = pb[q];
      }
    }
  };
  f16v acc[kFM][kFN];
#pragma unroll
  for (int i = 0; i < kFM; ++i)
#pragma unroll
    for (int j = 0; j < kFN; ++j) acc[i][j] = f16v{};

  const int nk = (g.K + kBK - 1) / kBK;
  oa.load(ga, 0);
  ob.load(gb, 0);
  store(0);
  oa.load(ga, min(1, nk - 1));
  ob.load(gb, min(1, nk - 1));
  __syncthreads();
  const int arow = (wm * kTM + r32) * kLDK + 8 * half, brow = (wn * kTN + r32) * kLDK + 8 * half;
  for (int it = 0; it < nk; ++it) {
    const unsigned short* base = sm + (it & 1) * kBuf;
    u32x4 fa[3][kFM], fb[3][kFN];
#pragma unroll
    for (int q = 0; q < 3; ++q) {
#pragma unroll
      for (int i = 0; i < kFM; ++i)
        fa[q][i] = *reinterpret_cast<const u32x4*>(base + q * kPiece + arow + 32 * i * kLDK);
#pragma unroll
      for (int j = 0; j < kFN; ++j)
        fb[q][j] = *reinterpret_cast<const u32x4*>(base + (3 + q) * kPiece + brow + 32 * j * kLDK);
    }
    // slice it+1 into the other buffer (its last reads were before the previous barrier)
    store((it & 1) ^ 1);
    const int nxt = min(it + 2, nk - 1);
    oa.load(ga, nxt);
    ob.load(gb, nxt);
#pragma unroll
    for (int pp = 0; pp < 6; ++pp)
#pragma unroll
      for (int i = 0; i < kFM; ++i)
#pragma unroll
        for (int j = 0; j < kFN; ++j) acc[i][j] = mfma_bf16(fa[kPa[pp]][i], fb[kPb[pp]][j], acc[i][j]);
    if constexpr (FULL) {
      // fragment reads first, then the 48 products with the split and the LDS writes
      // spread between them, then the next slice's loads
      constexpr int kMfma = 6 * kFM * kFN, kWrites = 6 * kCh, kValu = 2 * 28 * kCh;
      __builtin_amdgcn_sched_group_barrier(0x100, 3 * (kFM + kFN), 0);
#pragma unroll
      for (int w = 0; w < kWrites; ++w) {
        __builtin_amdgcn_sched_group_barrier(0x008, kMfma / kWrites, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, kValu / kWrites, 0);
        __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x020, 2 * kCh, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, kMfma, 0);
    }
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < kFM; ++i)
#pragma unroll
    for (int j = 0; j < kFN; ++j) {
      const int n = n0 + wn * kTN + j * 32 + r32;
      if (!FULL && n >= g.N) continue;
      const float bval = g.bias ? g.bias[n] : 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * kTM + i * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
        if (FULL || m < g.M) g.C[(size_t)m * g.ldc + n] = acc[i][j][r] + bval;
      }
    }
}

// FULL: every tile lies inside the matrices (M, N multiples of 256, K of 16, aligned
// operands); chosen per launch, so the unmasked kernel carries no edge code.
template <bool FULL>
__global__ __launch_bounds__(kThreads) void gemm_x6_kernel(X6Args g) {
  extern __shared__ unsigned short x6_smem[];
  int tm, tn;
  gemm_tile_order(g.tiles_m, g.tiles_n, &tm, &tn);
  x6_tile<FULL>(g, tm * kBT, tn * kBT, x6_smem);
}

}  // namespace

bool gemm_x6_applies(int M, int N, int K) {
  // one 256 x 256 tile per CU at least, and enough k to amortise the tile's setup
  const long tiles = (long)((M + kBT - 1) / kBT) * ((N + kBT - 1) / kBT);
  return tiles >= 256 && K >= 32;
}

int gemm_x6_run(const float* A, const float* B, const float* bias, float* C, int M, int N, int K, int lda, int ldb,
                int ldc, hipStream_t s) {
  if (M <= 0 || N <= 0 || K <= 0) return fail(HSL_ERR_ARG, "gemm_x6: empty product");
  X6Args g{};
  g.A = A;
  g.B = B;
  g.bias = bias;
  g.C = C;
  g.M = M;
  g.N = N;
  g.K = K;
  g.lda = lda;
  g.ldb = ldb;
  g.ldc = ldc;
  g.vec = aligned16(A) && aligned16(B) && lda % 4 == 0 && ldb % 4 == 0;
  g.tiles_m = (M + kBT - 1) / kBT;
  g.tiles_n = (N + kBT - 1) / kBT;
  const bool full = g.vec && M % kBT == 0 && N % kBT == 0 && K % kBK == 0;
  if (full)
    hipLaunchKernelGGL(gemm_x6_kernel<true>, dim3(g.tiles_m * g.tiles_n), dim3(kThreads), kLdsBytes, s, g);
  else
    hipLaunchKernelGGL(gemm_x6_kernel<false>, dim3(g.tiles_m * g.tiles_n), dim3(kThreads), kLdsBytes, s, g);
  HSL_HIP(hipGetLastError());
  return HSL_OK;
}

}  // namespace hsl
