// hsl_gemm_f32: fp32 MFMA GEMM entry point with optional split-K.
//
// Split-K writes fp32 partial tiles [splits][M][N] and a second kernel adds them in
// fp64 (plus the bias), so long reductions (K = T*B up to 65536 for the weight
// gradients) lose less accuracy than one fp32 running sum.
#include "gemm2_core.h"

namespace hsl {

using CfgBig = GemmCfg<128, 128, 32, 2, 2, 1>;
using CfgMid = GemmCfg<64, 64, 32, 2, 2, 1>;
using CfgSmall = GemmCfg<32, 32, 32, 1, 1, 4>;
// fp64-accumulating products with both sides >= 64 use the double-buffered core.
using Cfg2Acc = Gemm2Cfg<64, 64, 32, true>;

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

enum class Tile { Big, Mid, Small };

Tile pick_tile(int M, int N, int acc64 = 0) {
  const long big_tiles = (long)((M + 127) / 128) * ((N + 127) / 128);
  if (!acc64 && M >= 128 && N >= 128 && big_tiles >= 128) return Tile::Big;
  const long mid_tiles = (long)((M + 63) / 64) * ((N + 63) / 64);
  if (M >= 64 && N >= 64 && mid_tiles >= 32) return Tile::Mid;
  return Tile::Small;
}

int tile_count(Tile t, int M, int N) {
  const int b = t == Tile::Big ? 128 : t == Tile::Mid ? 64 : 32;
  return ((M + b - 1) / b) * ((N + b - 1) / b);
}

template <class Cfg, class Epi, bool ACC64>
int dispatch_trans(const GemmArgs& g, int ta, int tb, int splits, const Epi& epi, hipStream_t s) {
  if (!ta && !tb) return launch_gemm<Cfg, false, false, Epi, ACC64>(g, splits, epi, s);
  if (!ta && tb) return launch_gemm<Cfg, false, true, Epi, ACC64>(g, splits, epi, s);
  if (ta && !tb) return launch_gemm<Cfg, true, false, Epi, ACC64>(g, splits, epi, s);
  return launch_gemm<Cfg, true, true, Epi, ACC64>(g, splits, epi, s);
}

// fp64-accumulating products use the 64x64 (or 32x32) tiles: the fp64 registers of
// the 128x128 tile would not fit next to its fp32 accumulators.
template <class Epi>
int dispatch(Tile t, const GemmArgs& g, int ta, int tb, int splits, const Epi& epi, hipStream_t s, int acc64) {
  if (acc64) {
    if (t == Tile::Small) return dispatch_trans<CfgSmall, Epi, true>(g, ta, tb, splits, epi, s);
    return dispatch_trans<CfgMid, Epi, true>(g, ta, tb, splits, epi, s);
  }
  switch (t) {
    case Tile::Big: return dispatch_trans<CfgBig, Epi, false>(g, ta, tb, splits, epi, s);
    case Tile::Mid: return dispatch_trans<CfgMid, Epi, false>(g, ta, tb, splits, epi, s);
    default: return dispatch_trans<CfgSmall, Epi, false>(g, ta, tb, splits, epi, s);
  }
}

bool use_v2(const GemmDesc& d) { return d.acc64 && d.M >= 64 && d.N >= 64; }

int dispatch_v2(const GemmDesc& d, float* partial, int splits, hipStream_t s, int* used) {
  const int vec_a = aligned16(d.A) && d.lda % 4 == 0, vec_b = aligned16(d.B) && d.ldb % 4 == 0;
  if (!d.trans_a && !d.trans_b)
    return launch_gemm2<Cfg2Acc, false, false>(d.A, d.B, d.bias, d.C, partial, d.M, d.N, d.K, d.lda, d.ldb, d.ldc,
                                               splits, vec_a, vec_b, s, used);
  if (!d.trans_a && d.trans_b)
    return launch_gemm2<Cfg2Acc, false, true>(d.A, d.B, d.bias, d.C, partial, d.M, d.N, d.K, d.lda, d.ldb, d.ldc,
                                              splits, vec_a, vec_b, s, used);
  if (d.trans_a && !d.trans_b)
    return launch_gemm2<Cfg2Acc, true, false>(d.A, d.B, d.bias, d.C, partial, d.M, d.N, d.K, d.lda, d.ldb, d.ldc,
                                              splits, vec_a, vec_b, s, used);
  return launch_gemm2<Cfg2Acc, true, true>(d.A, d.B, d.bias, d.C, partial, d.M, d.N, d.K, d.lda, d.ldb, d.ldc,
                                           splits, vec_a, vec_b, s, used);
}

// Number of k-slices the chosen kernel really launches for a requested split count.
int actual_splits(const GemmDesc& d, Tile t, int splits) {
  int kps;
  const int K = d.K;
  if (use_v2(d)) return gemm2_split_layout<Cfg2Acc>(K, splits, &kps);
  switch (t) {
    case Tile::Big: return split_layout<CfgBig>(K, splits, &kps);
    case Tile::Mid: return split_layout<CfgMid>(K, splits, &kps);
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
  const Tile t = pick_tile(M, N, acc64);
  const int tiles = tile_count(t, M, N);
  if (tiles >= 512 || K < 1024) return 1;
  int s = (1024 + tiles - 1) / tiles;     // aim for ~1024 workgroups
  const int max_by_k = K / 512;           // keep >= 512 k per split
  if (s > max_by_k) s = max_by_k;
  if (s > 64) s = 64;
  return s < 1 ? 1 : s;
}

size_t gemm_ws_bytes(int M, int N, int K, int acc64) {
  const int s = gemm_pick_splits(M, N, K, acc64);
  return s > 1 ? sizeof(float) * (size_t)s * M * N : 0;
}

int gemm_partials(const GemmDesc& d, float* partials, int splits, hipStream_t s, int* used) {
  HSL_CHECK(check_desc(d));
  if (use_v2(d)) return dispatch_v2(d, partials, splits, s, used);
  const Tile t = pick_tile(d.M, d.N, d.acc64);
  *used = actual_splits(d, t, splits);
  EpiPartial epi{partials, d.M, d.N};
  return dispatch(t, make_args(d), d.trans_a, d.trans_b, *used, epi, s, d.acc64);
}

int gemm_run(const GemmDesc& d, void* ws, size_t ws_bytes, hipStream_t s) {
  HSL_CHECK(check_desc(d));
  if (d.M == 0 || d.N == 0) return HSL_OK;
  const Tile t = pick_tile(d.M, d.N, d.acc64);
  int splits = gemm_pick_splits(d.M, d.N, d.K, d.acc64);
  if (splits > 1) splits = actual_splits(d, t, splits);
  const size_t need = sizeof(float) * (size_t)splits * d.M * d.N;
  if (splits > 1 && (ws == nullptr || ws_bytes < need)) splits = 1;
  float* P = static_cast<float*>(ws);
  if (use_v2(d)) {
    int used = 1;
    HSL_CHECK(dispatch_v2(d, splits > 1 ? P : nullptr, splits, s, &used));
    if (splits == 1) return HSL_OK;
    splits = used;
  } else if (splits == 1) {
    EpiStore epi{d.C, d.bias, d.M, d.N, d.ldc};
    return dispatch(t, make_args(d), d.trans_a, d.trans_b, 1, epi, s, d.acc64);
  } else {
    EpiPartial epi{P, d.M, d.N};
    HSL_CHECK(dispatch(t, make_args(d), d.trans_a, d.trans_b, splits, epi, s, d.acc64));
  }
  return splitk_reduce(P, splits, d.bias, d.C, d.M, d.N, d.ldc, s);
}

int splitk_reduce(const float* P, int splits, const float* bias, float* C, int M, int N, int ldc, hipStream_t s) {
  const size_t total = (size_t)M * N;
  if (total == 0) return HSL_OK;
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
  return hsl::gemm_ws_bytes(M, N, K, 0);
}

int hsl_gemm_f32(const float* A, const float* Bm, const float* bias, float* C, int M, int N, int K, int lda,
                 int ldb, int ldc, int trans_a, int trans_b, void* ws, size_t ws_bytes, void* stream) {
  hsl::GemmDesc d{A, Bm, bias, C, M, N, K, lda, ldb, ldc, trans_a ? 1 : 0, trans_b ? 1 : 0, 0};
  return hsl::gemm_run(d, ws, ws_bytes, static_cast<hipStream_t>(stream));
}

}  // extern "C"
