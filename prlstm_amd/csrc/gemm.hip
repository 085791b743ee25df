// hsl_gemm_f32: fp32 MFMA GEMM entry point with optional split-K.
//
// Large C = A B^T products (at least 256 tiles of 256 x 256, no fp64 folding) and large
// C = A^T B / A B products (weight gradients and dx, >= 8 GFLOP, split into fp32 runs of
// <= 2048 k added in fp64)
// run on the split-bf16 kernel of gemm_x6.hip (fp32 accuracy, 2.5x the matrix-core rate)
// unless hsl_set_split_products(0) selects the fp32 instruction for everything.
// Products with M, N >= 64 run on the third core (gemm3_core.h): 128x256, 128x128 or
// 128x64 tiles, whichever is the largest that still gives two workgroups per CU, and
// 128x64 tiles with fp64 folding for the long weight-gradient reductions.  Thinner
// products (one side below 64, e.g. the [B,H] carries) use the first core's 32x32 tile.
//
// Split-K writes fp32 partial tiles [splits][M][N] and a second kernel adds them in
// fp64 (plus the bias), so long reductions (K = T*B up to 65536 for the weight
// gradients) lose less accuracy than one fp32 running sum.
#include <algorithm>

#include "gemm3_core.h"

namespace hsl {

using CfgSmall = GemmCfg<32, 32, 32, 1, 1, 4>;
using Cfg3Wide = Gemm3Cfg<128, 256, 32, false>;
using Cfg3Sq = Gemm3Cfg<128, 128, 32, false>;
using Cfg3Narrow = Gemm3Cfg<128, 64, 32, false>;
// fp64-accumulating products: fp32 MFMA partials of 4 slices (128 k) folded into fp64
using Cfg3Acc = Gemm3Cfg<128, 64, 32, true, 4>;

namespace {

__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ P, int splits,
                                                            const float* __restrict__ bias, float* __restrict__ C,
                                                            int M, int N, int ldc) {
  const size_t total = (size_t)M * N;
  for (size_t e = blockIdx.x * (size_t)blockDim.x + threadIdx.x; e < total; e += (size_t)gridDim.x * blockDim.x) {
    double acc = 0.0;
    for (int z = 0; z < splits; ++z) acc += (double)P[(size_t)z * total + e];
    const int m = (int)(e / N), n = (int)(e % N);
    float v = (float)acc;
    if (bias) v += bias[n];
    C[(size_t)m * ldc + n] = v;
  }
}

// The same sums four elements per thread (N % 4 == 0, 16-byte aligned planes, C and bias):
// 16-byte loads of eight planes in flight per batch, added in plane order from 0.0 as above
// (bit for bit the same result).
__global__ __launch_bounds__(256) void splitk_reduce4_kernel(const float4* __restrict__ P, int splits,
                                                             const float* __restrict__ bias, float* __restrict__ C,
                                                             int M, int N, int ldc) {
  constexpr int kBatch = 8;
  const size_t total4 = (size_t)M * N / 4;
  for (size_t e = blockIdx.x * (size_t)blockDim.x + threadIdx.x; e < total4; e += (size_t)gridDim.x * blockDim.x) {
    double acc[4] = {0.0, 0.0, 0.0, 0.0};
    for (int z0 = 0; z0 < splits; z0 += kBatch) {
      float4 q[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i)
        q[i] = z0 + i < splits ? P[(size_t)(z0 + i) * total4 + e] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {  // adding +0.0 past the last plane is exact
        acc[0] += (double)q[i].x;
        acc[1] += (double)q[i].y;
        acc[2] += (double)q[i].z;
        acc[3] += (double)q[i].w;
      }
    }
    const size_t el = 4 * e;
    const int m = (int)(el / N), n = (int)(el % N);
    float4 v = make_float4((float)acc[0], (float)acc[1], (float)acc[2], (float)acc[3]);
    if (bias) {
      const float4 b = *reinterpret_cast<const float4*>(bias + n);
      v = make_float4(v.x + b.x, v.y + b.y, v.z + b.z, v.w + b.w);
    }
    *reinterpret_cast<float4*>(C + (size_t)m * ldc + n) = v;
  }
}

enum class Tile { Wide, Sq, Narrow, Acc, Small };

// Workgroups the chip runs at once with two per CU.
constexpr long kFill = 512;

long tiles_of(int M, int N, int bm, int bn) { return (long)((M + bm - 1) / bm) * ((N + bn - 1) / bn); }

Tile pick_tile(int M, int N, int acc64) {
  if (M < 64 || N < 64) return Tile::Small;
  if (acc64) return Tile::Acc;
  if (tiles_of(M, N, 128, 256) >= kFill) return Tile::Wide;
  if (tiles_of(M, N, 128, 128) >= kFill) return Tile::Sq;
  return Tile::Narrow;
}

long tile_count(Tile t, int M, int N) {
  switch (t) {
    case Tile::Wide: return tiles_of(M, N, 128, 256);
    case Tile::Sq: return tiles_of(M, N, 128, 128);
    case Tile::Narrow:
    case Tile::Acc: return tiles_of(M, N, 128, 64);
    default: return tiles_of(M, N, 32, 32);
  }
}

template <class Cfg>
int run3(const GemmDesc& d, float* partial, int splits, hipStream_t s, int* used) {
  const int vec = aligned16(d.A) && aligned16(d.B) && d.lda % 4 == 0 && d.ldb % 4 == 0;
  const float* bias = partial ? nullptr : d.bias;
  if (!d.trans_a && !d.trans_b)
    return launch_gemm3<Cfg, false, false>(d.A, d.B, bias, d.C, partial, d.M, d.N, d.K, d.lda, d.ldb, d.ldc, splits,
                                           vec, s, used);
  if (!d.trans_a && d.trans_b)
    return launch_gemm3<Cfg, false, true>(d.A, d.B, bias, d.C, partial, d.M, d.N, d.K, d.lda, d.ldb, d.ldc, splits,
                                          vec, s, used);
  if (d.trans_a && !d.trans_b)
    return launch_gemm3<Cfg, true, false>(d.A, d.B, bias, d.C, partial, d.M, d.N, d.K, d.lda, d.ldb, d.ldc, splits,
                                          vec, s, used);
  return launch_gemm3<Cfg, true, true>(d.A, d.B, bias, d.C, partial, d.M, d.N, d.K, d.lda, d.ldb, d.ldc, splits, vec,
                                       s, used);
}

template <class Epi>
int run_small(const GemmArgs& g, int ta, int tb, int splits, const Epi& epi, hipStream_t s, int acc64) {
  if (acc64) {
    if (!ta && !tb) return launch_gemm<CfgSmall, false, false, Epi, true>(g, splits, epi, s);
    if (!ta && tb) return launch_gemm<CfgSmall, false, true, Epi, true>(g, splits, epi, s);
    if (ta && !tb) return launch_gemm<CfgSmall, true, false, Epi, true>(g, splits, epi, s);
    return launch_gemm<CfgSmall, true, true, Epi, true>(g, splits, epi, s);
  }
  if (!ta && !tb) return launch_gemm<CfgSmall, false, false, Epi, false>(g, splits, epi, s);
  if (!ta && tb) return launch_gemm<CfgSmall, false, true, Epi, false>(g, splits, epi, s);
  if (ta && !tb) return launch_gemm<CfgSmall, true, false, Epi, false>(g, splits, epi, s);
  return launch_gemm<CfgSmall, true, true, Epi, false>(g, splits, epi, s);
}

// Number of k-slices the chosen kernel really launches for a requested split count.
int actual_splits(Tile t, int K, int splits) {
  int kps;
  switch (t) {
    case Tile::Wide: return gemm3_split_layout<Cfg3Wide>(K, splits, &kps);
    case Tile::Sq: return gemm3_split_layout<Cfg3Sq>(K, splits, &kps);
    case Tile::Narrow: return gemm3_split_layout<Cfg3Narrow>(K, splits, &kps);
    case Tile::Acc: return gemm3_split_layout<Cfg3Acc>(K, splits, &kps);
    default: return split_layout<CfgSmall>(K, splits, &kps);
  }
}

GemmArgs make_args(const GemmDesc& d) {
  GemmArgs g{};
  g.A = d.A;
  g.B = d.B;
  g.M = d.M;
  g.N = d.N;
  g.K = d.K;
  g.lda = d.lda;
  g.ldb = d.ldb;
  g.vec_a = aligned16(d.A) && d.lda % 4 == 0;
  g.vec_b = aligned16(d.B) && d.ldb % 4 == 0;
  return g;
}

// The product into C (partial == nullptr) or into split-K planes.
int dispatch(Tile t, const GemmDesc& d, float* partial, int splits, hipStream_t s, int* used) {
  switch (t) {
    case Tile::Wide: return run3<Cfg3Wide>(d, partial, splits, s, used);
    case Tile::Sq: return run3<Cfg3Sq>(d, partial, splits, s, used);
    case Tile::Narrow: return run3<Cfg3Narrow>(d, partial, splits, s, used);
    case Tile::Acc: return run3<Cfg3Acc>(d, partial, splits, s, used);
    default: break;
  }
  *used = actual_splits(t, d.K, partial ? splits : 1);
  if (partial) {
    EpiPartial epi{partial, d.M, d.N};
    return run_small(make_args(d), d.trans_a, d.trans_b, *used, epi, s, d.acc64);
  }
  EpiStore epi{d.C, d.bias, d.M, d.N, d.ldc};
  return run_small(make_args(d), d.trans_a, d.trans_b, 1, epi, s, d.acc64);
}

int check_desc(const GemmDesc& d) {
  if (d.M < 0 || d.N < 0 || d.K < 0) return fail(HSL_ERR_ARG, "gemm: negative size");
  const int a_cols = d.trans_a ? d.M : d.K, b_cols = d.trans_b ? d.K : d.N;
  if (d.lda < (a_cols > 0 ? a_cols : 1) || d.ldb < (b_cols > 0 ? b_cols : 1) || d.ldc < (d.N > 0 ? d.N : 1))
    return fail(HSL_ERR_ARG, "gemm: leading dimension smaller than the row length");
  if (d.M > 0 && d.N > 0 && (!d.C || (d.K > 0 && (!d.A || !d.B))))
    return fail(HSL_ERR_ARG, "gemm: null pointer");
  return HSL_OK;
}

}  // namespace

int gemm_pick_splits(int M, int N, int K, int acc64) {
  const long tiles = tile_count(pick_tile(M, N, acc64), M, N);
  if (tiles >= kFill || K < 1024) return 1;
  int s = (int)((2 * kFill + tiles - 1) / tiles);  // aim for ~1024 workgroups
  const int max_by_k = K / 512;                    // keep >= 512 k per split
  if (s > max_by_k) s = max_by_k;
  if (s > 64) s = 64;
  return s < 1 ? 1 : s;
}

size_t gemm_ws_bytes(int M, int N, int K, int acc64) {
  const int s = gemm_pick_splits(M, N, K, acc64);
  return s > 1 ? sizeof(float) * (size_t)s * M * N : 0;
}

namespace {
// Split count of the split-bf16 A^T B / A B kernel for this product when it is taken with at
// most `max_planes` partial planes (0: not taken, because split products are off, the
// product is small, or the planes would leave splits longer than kSplitLongKRun).
int x6_longk_take(const GemmDesc& d, long max_planes) {
  if (d.trans_b || !split_products_mode()) return 0;  // A^T B or A B
  int s = gemm_x6_longk_splits(d.M, d.N, d.K);
  if (s <= 0) return 0;
  if (s > max_planes) s = (int)max_planes;
  if (s < 1 || (long)s * kSplitLongKRun < d.K) return 0;
  return s;
}
}  // namespace

size_t gemm_ws_bytes_layout(int M, int N, int K, int acc64, int trans_a, int trans_b) {
  size_t need = gemm_ws_bytes(M, N, K, acc64);
  if (!trans_b && split_products_mode()) {
    const int s = gemm_x6_longk_splits(M, N, K);
    if (s > 1) need = std::max(need, sizeof(float) * (size_t)s * M * N);
  }
  return need;
}

int gemm_tn_planes(int M, int N, int K) {
  int s = gemm_pick_splits(M, N, K, 1);
  if (split_products_mode()) s = std::max(s, gemm_x6_longk_splits(M, N, K));
  return s;
}

int gemm_partials(const GemmDesc& d, float* partials, int splits, hipStream_t s, int* used) {
  HSL_CHECK(check_desc(d));
  if (const int sx = x6_longk_take(d, splits))
    return gemm_x6_run(d.A, d.B, nullptr, nullptr, partials, d.M, d.N, d.K, d.lda, d.ldb, d.N, d.trans_a, 0, sx, s,
                       used);
  return dispatch(pick_tile(d.M, d.N, d.acc64), d, partials, std::min(splits, gemm_pick_splits(d.M, d.N, d.K, d.acc64)), s,
                  used);
}

int gemm_run(const GemmDesc& d, void* ws, size_t ws_bytes, hipStream_t s) {
  HSL_CHECK(check_desc(d));
  if (d.M == 0 || d.N == 0) return HSL_OK;
  if (!d.trans_a && d.trans_b && !d.acc64 && split_products_mode() && gemm_x6_applies(d.M, d.N, d.K))
    return gemm_x6_run(d.A, d.B, d.bias, d.C, nullptr, d.M, d.N, d.K, d.lda, d.ldb, d.ldc, 0, 1, 1, s, nullptr);
  // planes the workspace holds (one split needs none: it writes C directly)
  const long planes = ws ? (long)(ws_bytes / (sizeof(float) * (size_t)d.M * d.N)) : 0;
  if (const int sx = x6_longk_take(d, planes > 1 ? planes : 1)) {
    if (sx == 1)
      return gemm_x6_run(d.A, d.B, d.bias, d.C, nullptr, d.M, d.N, d.K, d.lda, d.ldb, d.ldc, d.trans_a, 0, 1, s,
                         nullptr);
    float* P = static_cast<float*>(ws);
    int used = 1;
    HSL_CHECK(gemm_x6_run(d.A, d.B, nullptr, nullptr, P, d.M, d.N, d.K, d.lda, d.ldb, d.N, d.trans_a, 0, sx, s, &used));
    return splitk_reduce(P, used, d.bias, d.C, d.M, d.N, d.ldc, s);
  }
  const Tile t = pick_tile(d.M, d.N, d.acc64);
  int splits = gemm_pick_splits(d.M, d.N, d.K, d.acc64);
  if (splits > 1) splits = actual_splits(t, d.K, splits);
  const size_t need = sizeof(float) * (size_t)splits * d.M * d.N;
  if (splits > 1 && (ws == nullptr || ws_bytes < need)) splits = 1;
  float* P = static_cast<float*>(ws);
  int used = 1;
  if (splits == 1) return dispatch(t, d, nullptr, 1, s, &used);
  HSL_CHECK(dispatch(t, d, P, splits, s, &used));
  return splitk_reduce(P, used, d.bias, d.C, d.M, d.N, d.ldc, s);
}

namespace {
__global__ __launch_bounds__(256) void widen16_kernel(const unsigned short* __restrict__ src, float* __restrict__ dst,
                                                      size_t n, int fmt) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const unsigned short v = src[i];
    dst[i] = fmt == 0 ? __uint_as_float((unsigned)v << 16) : (float)__builtin_bit_cast(_Float16, v);
  }
}
}  // namespace

int widen16(const void* src, float* dst, size_t n, int fmt, hipStream_t s) {
  if (n == 0) return HSL_OK;
  int blocks = (int)std::min<size_t>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(widen16_kernel, dim3(blocks), dim3(256), 0, s, static_cast<const unsigned short*>(src), dst, n,
                     fmt);
  HSL_HIP(hipGetLastError());
  return HSL_OK;
}

int gemm_run_b16(const GemmDesc& d, int fmt, float* widen, void* ws, size_t ws_bytes, hipStream_t s) {
  HSL_CHECK(check_desc(d));
  if (d.trans_b) return fail(HSL_ERR_ARG, "gemm_run_b16: B must be [K][N]");
  if (d.M == 0 || d.N == 0) return HSL_OK;
  if (fmt == 0) {  // a bf16 value is one bf16 piece: the split kernel reads it as it is
    const long planes = ws ? (long)(ws_bytes / (sizeof(float) * (size_t)d.M * d.N)) : 0;
    if (const int sx = x6_longk_take(d, planes > 1 ? planes : 1)) {
      if (sx == 1)
        return gemm_x6_run(d.A, d.B, d.bias, d.C, nullptr, d.M, d.N, d.K, d.lda, d.ldb, d.ldc, d.trans_a, 0, 1, s,
                           nullptr, 1);
      float* P = static_cast<float*>(ws);
      int used = 1;
      HSL_CHECK(gemm_x6_run(d.A, d.B, nullptr, nullptr, P, d.M, d.N, d.K, d.lda, d.ldb, d.N, d.trans_a, 0, sx, s,
                            &used, 1));
      return splitk_reduce(P, used, d.bias, d.C, d.M, d.N, d.ldc, s);
    }
  }
  // otherwise the fp32 product of the widened B (same leading dimension)
  HSL_CHECK(widen16(d.B, widen, (size_t)d.K * d.ldb, fmt, s));
  GemmDesc w = d;
  w.B = widen;
  return gemm_run(w, ws, ws_bytes, s);
}

int splitk_reduce(const float* P, int splits, const float* bias, float* C, int M, int N, int ldc, hipStream_t s) {
  const size_t total = (size_t)M * N;
  if (total == 0) return HSL_OK;
  const bool vec = N % 4 == 0 && ldc % 4 == 0 && aligned16(P) && aligned16(C) && (!bias || aligned16(bias));
  if (vec) {
    int blocks = (int)((total / 4 + 255) / 256);
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(splitk_reduce4_kernel, dim3(blocks), dim3(256), 0, s, reinterpret_cast<const float4*>(P),
                       splits, bias, C, M, N, ldc);
    HSL_HIP(hipGetLastError());
    return HSL_OK;
  }
  int blocks = (int)((total + 255) / 256);
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3(blocks), dim3(256), 0, s, P, splits, bias, C, M, N, ldc);
  HSL_HIP(hipGetLastError());
  return HSL_OK;
}

}  // namespace hsl

extern "C" {

size_t hsl_gemm_ws_bytes(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  // enough for every layout: the split A^T B kernel may want more planes than the others
  return hsl::gemm_ws_bytes_layout(M, N, K, 0, 1, 0);
}

int hsl_gemm_f32(const float* A, const float* Bm, const float* bias, float* C, int M, int N, int K, int lda,
                 int ldb, int ldc, int trans_a, int trans_b, void* ws, size_t ws_bytes, void* stream) {
  hsl::GemmDesc d{A, Bm, bias, C, M, N, K, lda, ldb, ldc, trans_a ? 1 : 0, trans_b ? 1 : 0, 0};
  return hsl::gemm_run(d, ws, ws_bytes, static_cast<hipStream_t>(stream));
}

}  // extern "C"
