// 16-bit-input GEMM for half-precision modules: C[M,N] = A[M,K] . B[N,K]^T (+ bias[N]),
// A and B bf16 or fp16, C and the accumulation fp32 (hsl_gemm_b16, hsl_par_fwd_b16).
//
// The products of two 16-bit values are exact in fp32, so with fp32 accumulation this
// computes the same sum as the fp32 product of the widened operands; only the order in
// which the terms are added differs.  It runs on v_mfma_f32_32x32x16_{bf16,f16}, whose
// rate is 16x that of the fp32 instruction.
//
// Workgroup = 4 waves (2 x 2), tile 128 x 128, each wave 64 x 64 (2 x 2 fragments);
// BK = 64 k-values per slice, LDS double-buffered with one barrier per slice; the
// next slice's global loads are issued before the current slice's products.
// Fragment layout (gfx950): lane l supplies row (A) or column (B) l % 32 and eight
// consecutive k-values 8*(l/32) .. 8*(l/32)+7 of the 16 the instruction consumes (A and B
// use the same k assignment, so the sum is the full dot product); the accumulator layout
// is that of v_mfma_f32_32x32x2_f32: lane l, register r -> row 8(r/4) + 4(l/32) + r%4,
// column l%32.
#include "gemm_core.h"

namespace hsl {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));  // 8 16-bit values

constexpr int kBM = 128, kBN = 128, kBK = 64;
constexpr int kLD = kBK + 8;                       // LDS row stride in 16-bit elements (144 B)
constexpr int kTileElems = kBM * kLD;              // one operand, one buffer
constexpr int kChunks = kBM * kBK / 8 / 256;       // 16-byte chunks per thread per operand
static_assert(kChunks == 4, "tile split");

struct B16Args {
  const unsigned short* A;
  const unsigned short* B;
  const float* bias;
  float* C;
  int M, N, K, lda, ldb, ldc;
  int vec;  // 16-byte loads legal (aligned bases, lda/ldb % 8 == 0)
  int tiles_m, tiles_n;
};

template <bool FP16>
__device__ __forceinline__ f16v mfma16(u32x4 a, u32x4 b, f16v c) {
  if constexpr (FP16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

// chunk j of this thread: row c / 8, k-octet c % 8 of the slice (c = tid + 256 j)
template <bool FULL>
__device__ __forceinline__ void load_op(const unsigned short* base, int ld, int r0, int nrows, int k0, int K,
                                        bool vec, u32x4 (&reg)[kChunks]) {
#pragma unroll
  for (int j = 0; j < kChunks; ++j) {
    const int c = threadIdx.x + 256 * j;
    const int r = r0 + (c >> 3), k = k0 + (c & 7) * 8;
    const unsigned short* p = base + (size_t)r * ld + k;
    if (FULL) {
      reg[j] = *reinterpret_cast<const u32x4*>(p);
    } else {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (r < nrows) {
        if (vec && k + 7 < K) {
          v = *reinterpret_cast<const u32x4*>(p);
        } else {
          unsigned short e[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) e[i] = k + i < K ? p[i] : (unsigned short)0;
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] = (unsigned)e[2 * i] | ((unsigned)e[2 * i + 1] << 16);
        }
      }
      reg[j] = v;
    }
  }
}

__device__ __forceinline__ void store_op(unsigned short* lds, const u32x4 (&reg)[kChunks]) {
#pragma unroll
  for (int j = 0; j < kChunks; ++j) {
    const int c = threadIdx.x + 256 * j;
    *reinterpret_cast<u32x4*>(lds + (c >> 3) * kLD + (c & 7) * 8) = reg[j];
  }
}

template <bool FP16, bool FULL>
__device__ __forceinline__ void b16_tile(const B16Args& g, int m0, int n0, unsigned short* smem) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int half = lane >> 5, r32 = lane & 31;
  f16v acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f16v{};

  u32x4 ra[kChunks], rb[kChunks];
  const int nk = (g.K + kBK - 1) / kBK;
  if (nk > 0) {
    load_op<FULL>(g.A, g.lda, m0, g.M, 0, g.K, g.vec, ra);
    load_op<FULL>(g.B, g.ldb, n0, g.N, 0, g.K, g.vec, rb);
    store_op(smem, ra);
    store_op(smem + 2 * kTileElems, rb);
  }
  __syncthreads();
  for (int it = 0; it < nk; ++it) {
    const int cur = it & 1;
    const bool more = it + 1 < nk;
    if (more) {
      load_op<FULL>(g.A, g.lda, m0, g.M, (it + 1) * kBK, g.K, g.vec, ra);
      load_op<FULL>(g.B, g.ldb, n0, g.N, (it + 1) * kBK, g.K, g.vec, rb);
    }
    const unsigned short* la = smem + cur * kTileElems;
    const unsigned short* lb = smem + 2 * kTileElems + cur * kTileElems;
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      u32x4 av[2], bv[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        av[i] = *reinterpret_cast<const u32x4*>(la + (wm * 64 + i * 32 + r32) * kLD + ks * 16 + half * 8);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bv[j] = *reinterpret_cast<const u32x4*>(lb + (wn * 64 + j * 32 + r32) * kLD + ks * 16 + half * 8);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma16<FP16>(av[i], bv[j], acc[i][j]);
    }
    if (more) {  // the other buffer was last read in the previous slice, before the barrier below
      store_op(smem + (cur ^ 1) * kTileElems, ra);
      store_op(smem + 2 * kTileElems + (cur ^ 1) * kTileElems, rb);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + wn * 64 + j * 32 + r32;
      if (!FULL && n >= g.N) continue;
      const float bval = g.bias ? g.bias[n] : 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
        if (FULL || m < g.M) g.C[(size_t)m * g.ldc + n] = acc[i][j][r] + bval;
      }
    }
}

template <bool FP16>
__global__ __launch_bounds__(256) void gemm_b16_kernel(B16Args g) {
  extern __shared__ unsigned short smem16[];
  int tm, tn;
  gemm_tile_order(g.tiles_m, g.tiles_n, &tm, &tn);
  const int m0 = tm * kBM, n0 = tn * kBN;
  const bool full = g.vec && m0 + kBM <= g.M && n0 + kBN <= g.N && g.K % kBK == 0;
  if (full)
    b16_tile<FP16, true>(g, m0, n0, smem16);
  else
    b16_tile<FP16, false>(g, m0, n0, smem16);
}

constexpr size_t kB16Lds = sizeof(unsigned short) * 4 * kTileElems;

}  // namespace

int gemm_b16_run(const void* A, const void* B, const float* bias, float* C, int M, int N, int K, int lda, int ldb,
                 int ldc, int fmt, hipStream_t s) {
  if (M < 0 || N < 0 || K < 0) return fail(HSL_ERR_ARG, "gemm_b16: negative size");
  if (fmt != 0 && fmt != 1) return fail(HSL_ERR_ARG, "gemm_b16: format must be 0 (bf16) or 1 (fp16)");
  if (lda < (K > 0 ? K : 1) || ldb < (K > 0 ? K : 1) || ldc < (N > 0 ? N : 1))
    return fail(HSL_ERR_ARG, "gemm_b16: leading dimension smaller than the row length");
  if (M == 0 || N == 0) return HSL_OK;
  if (!C || (K > 0 && (!A || !B))) return fail(HSL_ERR_ARG, "gemm_b16: null pointer");
  B16Args g{};
  g.A = static_cast<const unsigned short*>(A);
  g.B = static_cast<const unsigned short*>(B);
  g.bias = bias;
  g.C = C;
  g.M = M;
  g.N = N;
  g.K = K;
  g.lda = lda;
  g.ldb = ldb;
  g.ldc = ldc;
  g.vec = aligned16(A) && aligned16(B) && lda % 8 == 0 && ldb % 8 == 0;
  g.tiles_m = (M + kBM - 1) / kBM;
  g.tiles_n = (N + kBN - 1) / kBN;
  const dim3 grid(g.tiles_m * g.tiles_n);
  if (fmt == 1)
    hipLaunchKernelGGL(gemm_b16_kernel<true>, grid, dim3(256), kB16Lds, s, g);
  else
    hipLaunchKernelGGL(gemm_b16_kernel<false>, grid, dim3(256), kB16Lds, s, g);
  HSL_HIP(hipGetLastError());
  return HSL_OK;
}

}  // namespace hsl

extern "C" int hsl_gemm_b16(const void* A, const void* B, const float* bias, float* C, int M, int N, int K, int lda,
                            int ldb, int ldc, int fmt, void* stream) {
  return hsl::gemm_b16_run(A, B, bias, C, M, N, K, lda, ldb, ldc, fmt, static_cast<hipStream_t>(stream));
}
