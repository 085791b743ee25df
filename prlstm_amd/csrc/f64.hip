// fp64 modules: both modes of the training step in double precision.
//
// The reference runs fp64 modules through its torch backend (test_cpp.py:150-165) and
// its parallel functional is dtype-generic (_parallel.py:38-74).  This path computes
// every value in fp64 with the same data layouts and C-ABI shapes as the fp32 entry
// points (include/hsl.h), so the autograd functions only change the entry names.  It
// is written for exactness first (gradient checks, fp64 training): an fp64 GEMM on the
// fp64 matrix instruction for every product (the per-step h W_s^T and dg W_s included),
// per-step cell kernels with one thread per (batch row, unit) and one thread per channel
// for the scans; every sum runs in a fixed order, so results are deterministic.
//
//   recurrent (_torch.py:86-170): W_s = a (x) W_hh, b_s = a (x) b_hh; gih = x W_ih^T + b_ih;
//     per step z = gih_t + b_s + h_{t-1} W_s^T, then the cell (_torch.py:27-36);
//     backward per step dh = dout_t + dg_{t+1} W_s (dh_n at T-1), the cell backward
//     (_torch.py:39-53), then dW_hh_s = dg^T h_prev, dW_ih = dg^T x, dx = dg W_ih,
//     db = colsum(dg), dW_hh = a dW_hh_s, db_hh = a db, da_g = sum_g(W_hh.dW_hh_s + b_hh db).
//   parallel (_parallel.py:21-74): gates = x W_ih^T + b_ih; the recurrence
//     c_t = max(f,eps) c_{t-1} + max(i g, eps), c_{-1} = max(c0, eps), out = o tanh(c),
//     with the checkpoint rows of the fp32 scan; its exact reverse-mode derivative.
#include <cmath>

#include "hsl_internal.h"

namespace hsl {
namespace {

constexpr int kCk = 8;  // steps per checkpoint row of c (as the fp32 scan)

__device__ __forceinline__ double sig64(double z) { return 1.0 / (1.0 + exp(-z)); }

// C[m][n] = (bias ? bias[n] : 0) + sum_k A(m,k) B(k,n), A(m,k) = A[m*sam + k*sak],
// B(k,n) = B[k*sbk + n*sbn], C row-major with ldc.  64x64 output tiles on 4 waves (a 32x32
// quarter each, 2x2 blocks of the fp64 matrix instruction 16x16x4), 16-deep k-slices
// through LDS (loaded along whichever index is contiguous in memory, the next slice into
// registers while the current one is multiplied); every output takes its k terms in
// increasing groups of four, one instruction per group.
// Split K: workgroup z covers k in [z*kc, min(K, (z+1)*kc)) and writes C + z*pst, so
// each split leaves a partial product that a fixed-order sum adds afterwards.
struct G64 {
  const double* A;
  const double* Bm;
  const double* bias;
  double* C;
  long long M, N, K, sam, sak, sbk, sbn, ldc;
  long long kc = 0;   // k per split (a multiple of 16); 0 = all of K
  long long pst = 0;  // distance between the splits' outputs
};

typedef double d4_t __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void gemm_f64_kernel(G64 g) {
  __shared__ double As[16][65];  // [k][m]
  __shared__ double Bs[16][65];  // [k][n]
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wm = (wv >> 1) * 32, wn = (wv & 1) * 32;  // this wave's 32x32 quarter of the tile
  const long long m0 = (long long)blockIdx.y * 64, n0 = (long long)blockIdx.x * 64;
  const long long kb0 = g.kc ? (long long)blockIdx.z * g.kc : 0;
  const long long kend = g.kc ? min(g.K, kb0 + g.kc) : g.K;
  double* C = g.C + (long long)blockIdx.z * g.pst;
  const bool a_kc = g.sak == 1, b_nc = g.sbn == 1;  // which index is contiguous
  d4_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = d4_t{0.0, 0.0, 0.0, 0.0};
  // this thread's 4 + 4 operand elements of a slice: LDS places and global offsets
  int am[4], ak[4], bn[4], bk[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int e = tid + 256 * r;
    am[r] = a_kc ? e >> 4 : e & 63;
    ak[r] = a_kc ? e & 15 : e >> 6;
    bn[r] = b_nc ? e & 63 : e >> 4;
    bk[r] = b_nc ? e >> 6 : e & 15;
  }
  double ra[4], rb[4];  // the next slice, loaded while the current one is multiplied
  auto load_slice = [&](long long k0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const long long m = m0 + am[r], ka = k0 + ak[r];
      ra[r] = (m < g.M && ka < kend) ? g.A[m * g.sam + ka * g.sak] : 0.0;
      const long long n = n0 + bn[r], kb = k0 + bk[r];
      rb[r] = (kb < kend && n < g.N) ? g.Bm[kb * g.sbk + n * g.sbn] : 0.0;
    }
  };
  if (kb0 < kend) load_slice(kb0);
  for (long long k0 = kb0; k0 < kend; k0 += 16) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      As[ak[r]][am[r]] = ra[r];
      Bs[bk[r]][bn[r]] = rb[r];
    }
    __syncthreads();
    if (k0 + 16 < kend) load_slice(k0 + 16);
    // v_mfma_f64_16x16x4: lane l holds A[l%16][l/16] and B[l/16][l%16] of a 16x16x4 step
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int kr = 4 * kk + (lane >> 4), c = lane & 15;
      const double a0 = As[kr][wm + c], a1 = As[kr][wm + 16 + c];
      const double b0 = Bs[kr][wn + c], b1 = Bs[kr][wn + 16 + c];
      acc[0][0] = __builtin_amdgcn_mfma_f64_16x16x4f64(a0, b0, acc[0][0], 0, 0, 0);
      acc[0][1] = __builtin_amdgcn_mfma_f64_16x16x4f64(a0, b1, acc[0][1], 0, 0, 0);
      acc[1][0] = __builtin_amdgcn_mfma_f64_16x16x4f64(a1, b0, acc[1][0], 0, 0, 0);
      acc[1][1] = __builtin_amdgcn_mfma_f64_16x16x4f64(a1, b1, acc[1][1], 0, 0, 0);
    }
    __syncthreads();
  }
  // result element i of a lane: row l/16 + 4i, column l%16 of the 16x16 block
#pragma unroll
  for (int bi = 0; bi < 2; ++bi)
#pragma unroll
    for (int bj = 0; bj < 2; ++bj)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const long long m = m0 + wm + 16 * bi + (lane >> 4) + 4 * i, n = n0 + wn + 16 * bj + (lane & 15);
        if (m < g.M && n < g.N) C[m * g.ldc + n] = (g.bias ? g.bias[n] : 0.0) + acc[bi][bj][i];
      }
}

// C[m][n] = (bias ? bias[n] : 0) + sum over s < S of part[s][m][n], in increasing s
__global__ void sum_splits_f64(const double* part, const double* bias, double* C, long long M, long long N,
                               long long ldc, int S) {
  const long long MN = M * N;
  for (long long e = blockIdx.x * 256ll + threadIdx.x; e < MN; e += (long long)gridDim.x * 256) {
    const long long m = e / N, n = e % N;
    double acc = 0.0;
    for (int z = 0; z < S; ++z) acc += part[z * MN + e];
    C[m * ldc + n] = (bias ? bias[n] : 0.0) + acc;
  }
}

constexpr long long kFillBlocks = 1024;  // workgroups that keep every CU busy (4 per CU)
constexpr long long kMinSplitK = 64;     // k per split at the least

// Splits of K for an M x N x K product: enough workgroups to fill the chip when the
// output alone has too few tiles, each split at least kMinSplitK deep.
inline int split_of(long long M, long long N, long long K) {
  const long long tiles = ((M + 63) / 64) * ((N + 63) / 64);
  if (tiles <= 0 || tiles >= kFillBlocks || K <= kMinSplitK) return 1;
  long long S = (kFillBlocks + tiles - 1) / tiles;
  S = min(S, (K + kMinSplitK - 1) / kMinSplitK);
  const long long kc = ((K + S - 1) / S + 15) / 16 * 16;
  return (int)((K + kc - 1) / kc);
}

inline long long kc_of(long long K, int S) { return S > 1 ? ((K + S - 1) / S + 15) / 16 * 16 : 0; }

// Doubles of partial products for gemm64 with S = split_of(M, N, K) (0 when unsplit).
inline size_t part_elems(long long M, long long N, long long K) {
  const int S = split_of(M, N, K);
  return S > 1 ? (size_t)S * M * N : 0;
}

int launch_gemm(const G64& g, int S, hipStream_t s) {
  const long long gy = (g.M + 63) / 64, gx = (g.N + 63) / 64;
  if (gy > 65535 || gx > (1ll << 31) - 1) return fail(HSL_ERR_UNSUPPORTED, "fp64 GEMM: %lld rows", g.M);
  hipLaunchKernelGGL(gemm_f64_kernel, dim3((unsigned)gx, (unsigned)gy, (unsigned)S), dim3(256), 0, s, g);
  HSL_HIP(hipGetLastError());
  return HSL_OK;
}

int gemm64(const G64& g, hipStream_t s) {
  if (g.M <= 0 || g.N <= 0) return HSL_OK;
  G64 u = g;
  u.kc = 0;
  u.pst = 0;
  return launch_gemm(u, 1, s);
}

// The S = split_of(M, N, K) partial products into part[S][M][N] (nothing is summed);
// returns S through *S_out.  S == 1 writes g.C directly (with g.bias).
int gemm64_parts(const G64& g, double* part, int* S_out, hipStream_t s) {
  const int S = split_of(g.M, g.N, g.K);
  *S_out = S;
  if (g.M <= 0 || g.N <= 0) return HSL_OK;
  if (S == 1) return gemm64(g, s);
  G64 p = g;
  p.bias = nullptr;
  p.C = part;
  p.ldc = g.N;
  p.kc = kc_of(g.K, S);
  p.pst = g.M * g.N;
  return launch_gemm(p, S, s);
}

// gemm64 with K split over part (part_elems(M, N, K) doubles) and the fixed-order sum.
int gemm64_split(const G64& g, double* part, hipStream_t s) {
  int S = 1;
  HSL_CHECK(gemm64_parts(g, part, &S, s));
  if (S == 1 || g.M <= 0 || g.N <= 0) return HSL_OK;
  const long long MN = g.M * g.N;
  const long long nb = min((MN + 255) / 256, 4096ll);
  hipLaunchKernelGGL(sum_splits_f64, dim3((unsigned)nb), dim3(256), 0, s, part, g.bias, g.C, g.M, g.N, g.ldc, S);
  HSL_HIP(hipGetLastError());
  return HSL_OK;
}

inline unsigned blocks_for(long long n) { return (unsigned)((n + 255) / 256); }

// dst[i] = src ? src[i] : 0 (a kernel rather than a memset or copy node, so that a caller
// may capture the call in a graph)
__global__ void copy_f64_kernel(double* dst, const double* src, long long n) {
  for (long long i = blockIdx.x * 256ll + threadIdx.x; i < n; i += (long long)gridDim.x * 256)
    dst[i] = src ? src[i] : 0.0;
}

int copy64(double* dst, const double* src, long long n, hipStream_t s) {
  if (n <= 0) return HSL_OK;
  const unsigned g = blocks_for(n) < 4096 ? blocks_for(n) : 4096;
  hipLaunchKernelGGL(copy_f64_kernel, dim3(g), dim3(256), 0, s, dst, src, n);
  HSL_HIP(hipGetLastError());
  return HSL_OK;
}

// W_s[n][k] = a[n/H] W_hh[n][k], b_s[n] = a[n/H] b_hh[n]
__global__ void scale_f64_kernel(const double* w_hh, const double* b_hh, const double* a, double* ws, double* bs,
                                 int H) {
  const long long total = 4ll * H * H;
  for (long long e = blockIdx.x * 256ll + threadIdx.x; e < total; e += (long long)gridDim.x * 256) {
    const long long nrow = e / H;
    ws[e] = a[nrow / H] * w_hh[e];
    if (e % H == 0) bs[nrow] = b_hh ? a[nrow / H] * b_hh[nrow] : 0.0;
  }
}

// One forward step t, after the S split-K partials zb[S][B][4H] of h_{t-1} W_s^T
// (gemm64_parts): thread (b, u) sums them in order, forms the four gates
// (gih_t + h W_s^T) + b_s and runs the cell.  c_{t-1} = c_save[t].
__global__ void rec_step_fwd_f64(const double* gih, const double* zb, int S, const double* bs, double* h_save,
                                 double* c_save, double* gact, double* tanh_c, int t, int B, int H) {
  const long long e = blockIdx.x * 256ll + threadIdx.x;
  if (e >= (long long)B * H) return;
  const int b = (int)(e / H), u = (int)(e % H);
  const long long plane = (long long)B * H;
  double z[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const long long n = (long long)g * H + u;
    const double* zp = zb + (long long)b * 4 * H + n;
    const long long zs = (long long)B * 4 * H;
    double hw = 0.0;
    int z0 = 0;
    for (; z0 + 8 <= S; z0 += 8) {  // loads issued together, added in order
      double v[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) v[q] = zp[(z0 + q) * zs];
#pragma unroll
      for (int q = 0; q < 8; ++q) hw += v[q];
    }
    for (; z0 < S; ++z0) hw += zp[z0 * zs];
    z[g] = (gih[((long long)t * B + b) * 4 * H + n] + hw) + bs[n];
  }
  const double i = sig64(z[0]), f = sig64(z[1]), gg = sig64(z[2]), o = sig64(z[3]);
  const double c = f * c_save[t * plane + e] + i * gg;
  const double tc = tanh(c);
  h_save[(t + 1) * plane + e] = o * tc;
  c_save[(t + 1) * plane + e] = c;
  double* ga = gact + ((long long)t * plane + e) * 4;
  ga[0] = i;
  ga[1] = f;
  ga[2] = gg;
  ga[3] = o;
  tanh_c[t * plane + e] = tc;
}

// One backward step t (T-1 down to 0): thread (b, u).  dh = (dh_n at T-1, else the
// in-order sum of the S split-K partials dhb[S][B][H] of dg_{t+1} W_s) + dout_t; the
// cell backward with dc carried in dcb; writes dg_t.
__global__ void rec_step_bwd_f64(const double* dout, const double* dh_n, const double* dc_n, const double* c_save,
                                 const double* gact, const double* tanh_c, const double* dhb, int S, double* dg,
                                 double* dcb, int t, int T, int B, int H) {
  const long long e = blockIdx.x * 256ll + threadIdx.x;
  if (e >= (long long)B * H) return;
  const int b = (int)(e / H), u = (int)(e % H);
  const long long plane = (long long)B * H, row4 = 4ll * H;
  double dh;
  double dc;
  if (t == T - 1) {
    dh = dh_n ? dh_n[e] : 0.0;
    dc = dc_n ? dc_n[e] : 0.0;
  } else {
    dh = 0.0;
    int z0 = 0;
    for (; z0 + 8 <= S; z0 += 8) {  // loads issued together, added in order
      double v[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) v[q] = dhb[(z0 + q) * plane + e];
#pragma unroll
      for (int q = 0; q < 8; ++q) dh += v[q];
    }
    for (; z0 < S; ++z0) dh += dhb[z0 * plane + e];
    dc = dcb[e];
  }
  dh = dh + dout[t * plane + e];
  const double* ga = gact + ((long long)t * plane + e) * 4;
  const double i = ga[0], f = ga[1], gg = ga[2], o = ga[3], tc = tanh_c[t * plane + e];
  const double cp = c_save[t * plane + e];
  const double d_o = dh * tc;
  const double dct = dc + dh * o * (1.0 - tc * tc);
  const double d_f = dct * cp;
  const double d_i = dct * gg;
  const double d_g = dct * i;
  double* d = dg + ((long long)t * B + b) * row4;
  d[u] = d_i * i * (1.0 - i);
  d[H + u] = d_f * f * (1.0 - f);
  d[2 * H + u] = d_g * gg * (1.0 - gg);
  d[3 * H + u] = d_o * o * (1.0 - o);
  dcb[e] = dct * f;
}

// Column sums db[n] = sum over rows r < R of dg[r][n], in two fixed-order levels:
// colsum_part_f64 sums chunk z (rows [z*rc, min(R, (z+1)*rc)), increasing r) into
// part[z][n], colsum_fin_f64 adds the chunks in increasing z.
constexpr long long kColChunk = 256;

inline int col_chunks(long long R) { return (int)max(1ll, (R + kColChunk - 1) / kColChunk); }

__global__ void colsum_part_f64(const double* dg, double* part, long long R, int N) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= N) return;
  const long long r0 = (long long)blockIdx.y * kColChunk, r1 = min(R, r0 + kColChunk);
  double acc = 0.0;
  for (long long r = r0; r < r1; ++r) acc += dg[r * N + n];
  part[(long long)blockIdx.y * N + n] = acc;
}

__global__ void colsum_fin_f64(const double* part, double* db, int Z, int N) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= N) return;
  double acc = 0.0;
  for (int z = 0; z < Z; ++z) acc += part[(long long)z * N + n];
  db[n] = acc;
}

int colsum64(const double* dg, double* part, double* db, long long R, int N, hipStream_t s) {
  const int Z = col_chunks(R);
  if (Z > 65535) return fail(HSL_ERR_UNSUPPORTED, "fp64 column sum: %lld rows", R);
  hipLaunchKernelGGL(colsum_part_f64, dim3(blocks_for(N), (unsigned)Z), dim3(256), 0, s, dg, part, R, N);
  HSL_HIP(hipGetLastError());
  hipLaunchKernelGGL(colsum_fin_f64, dim3(blocks_for(N)), dim3(256), 0, s, part, db, Z, N);
  HSL_HIP(hipGetLastError());
  return HSL_OK;
}

// dW_hh = a dW_hh_s, db_ih = db, db_hh = a db; rowdot[n] = W_hh[n].dW_hh_s[n] + b_hh[n] db[n].
// One wave per row n: lane l adds k = l, l+64, ... in order, then the 64 lane sums are
// added by a fixed butterfly (deterministic).
__global__ __launch_bounds__(64) void rec_final_rows_f64(const double* w_hh, const double* b_hh, const double* a,
                                                         const double* dws, const double* db, double* dw_hh,
                                                         double* db_ih, double* db_hh, double* rowdot, int H) {
  const int n = blockIdx.x, l = threadIdx.x;
  const double ag = a[n / H];
  double acc = 0.0;
  for (int k = l; k < H; k += 64) {
    const long long e = (long long)n * H + k;
    dw_hh[e] = ag * dws[e];
    acc = fma(w_hh[e], dws[e], acc);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (l == 0) {
    rowdot[n] = acc + (b_hh ? b_hh[n] * db[n] : 0.0);
    db_ih[n] = db[n];
    db_hh[n] = ag * db[n];
  }
}

// da[g] = sum of rowdot over the gate's H rows: one wave per gate, lane l adds rows
// u = l, l+64, ... in order, then a fixed butterfly adds the 64 lane sums.
__global__ __launch_bounds__(64) void rec_da_f64(const double* rowdot, double* da, int H) {
  const int g = blockIdx.x, l = threadIdx.x;
  double acc = 0.0;
  for (int u = l; u < H; u += 64) acc += rowdot[(long long)g * H + u];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (l == 0) da[g] = acc;
}

// Parallel-mode scans, one thread per (channel, time chunk).  T is cut into P chunks of L
// steps (L a multiple of the 8-step checkpoint group), so that channels x chunks fill the
// chip; 64-thread workgroups spread them over every CU.  Each chunk's 8-step groups issue
// their loads together before the serial chain.  The recurrences are affine, so a chunk
// composes to one affine map: pass 1 composes every chunk, pass 2 carries the state across
// the chunks of a channel, pass 3 reruns each chunk from its carried state and writes.
constexpr int kScanThreads = 64;
constexpr long long kScanLanes = 262144;  // channels x chunks that fill the chip

// Chunk length L (steps) of T: P = ceil(T / L) chunks.
inline int scan_chunk_len(int T, long long C) {
  const long long want = max(1ll, (kScanLanes + C - 1) / C);
  return (int)max(8ll, ((T + want - 1) / want + 7) / 8 * 8);
}

inline int scan_chunks(int T, int L) { return T > 0 ? (T + L - 1) / L : 0; }

// The forward of steps [t0, t1) of channel ch from state c: c_t = max(f,eps) c + max(i g,eps).
// kWrite: out = o tanh(c), the checkpoint row at every group start (and the last row at
// T-1); else only the composed map c_out = A c_in + Bc (A, Bc accumulated in place).
template <bool kWrite>
__device__ __forceinline__ void fwd_chunk(const double* gates, double eps, double* out, double* cck, int t0, int t1,
                                          int T, int B, int H, long long ch, double& c, double& A) {
  const long long C = (long long)B * H, b = ch / H, j = ch % H, row4 = 4ll * H;
  for (int g0 = t0; g0 < t1; g0 += kCk) {
    if (kWrite) cck[(long long)(g0 / kCk) * C + ch] = c;
    const int n = min(kCk, t1 - g0);
    double zi[kCk], zf[kCk], zg[kCk], zo[kCk];
#pragma unroll
    for (int k = 0; k < kCk; ++k) {
      if (k < n) {
        const double* z = gates + ((long long)(g0 + k) * B + b) * row4 + j;
        zi[k] = z[0];
        zf[k] = z[H];
        zg[k] = z[2 * H];
        if (kWrite) zo[k] = z[3 * H];
      }
    }
#pragma unroll
    for (int k = 0; k < kCk; ++k) {
      if (k < n) {
        const double f = fmax(sig64(zf[k]), eps), bb = fmax(sig64(zi[k]) * sig64(zg[k]), eps);
        c = fma(f, c, bb);
        if (kWrite) {
          out[(long long)(g0 + k) * C + ch] = sig64(zo[k]) * tanh(c);
        } else {
          A *= f;
        }
      }
    }
  }
  if (kWrite && t1 == T) cck[(long long)((T + kCk - 1) / kCk) * C + ch] = c;
}

// Pass 1: chunk p < P-1 of every channel composes to c_out = A c_in + Bc, kept in rows p
// (A) and P + p (Bc) of out, which pass 3 overwrites.
__global__ __launch_bounds__(kScanThreads) void scan_fwd_compose_f64(const double* gates, double eps, double* out,
                                                                     int T, int B, int H, int L, int P) {
  const long long ch = blockIdx.x * (long long)kScanThreads + threadIdx.x, C = (long long)B * H;
  const int p = blockIdx.y;
  if (ch >= C || p >= P - 1) return;
  double c = 0.0, A = 1.0;
  fwd_chunk<false>(gates, eps, nullptr, nullptr, p * L, min(T, (p + 1) * L), T, B, H, ch, c, A);
  out[(long long)p * C + ch] = A;
  out[(long long)(P + p) * C + ch] = c;
}

// Pass 2: c entering chunk p, written to the checkpoint row of step p*L.
__global__ __launch_bounds__(kScanThreads) void scan_fwd_carry_f64(const double* c0, double eps, const double* out,
                                                                   double* cck, int B, int H, int L, int P) {
  const long long ch = blockIdx.x * (long long)kScanThreads + threadIdx.x, C = (long long)B * H;
  if (ch >= C) return;
  double c = fmax(c0 ? c0[ch] : 0.0, eps);
  for (int p = 0; p + 1 < P; ++p) {
    c = fma(out[(long long)p * C + ch], c, out[(long long)(P + p) * C + ch]);
    cck[(long long)((p + 1) * L / kCk) * C + ch] = c;
  }
}

// Pass 3 (the whole scan when P = 1): out and the checkpoint rows of chunk p.  c_ck row m
// = the state carried into step 8m (row 0 = max(c0, eps)), the last row c_{T-1}.
__global__ __launch_bounds__(kScanThreads) void scan_fwd_f64(const double* gates, const double* c0, double eps,
                                                             double* out, double* cck, int T, int B, int H, int L) {
  const long long ch = blockIdx.x * (long long)kScanThreads + threadIdx.x, C = (long long)B * H;
  if (ch >= C) return;
  const int p = blockIdx.y;
  double c = p == 0 ? fmax(c0 ? c0[ch] : 0.0, eps) : cck[(long long)(p * L / kCk) * C + ch];
  double A = 1.0;
  fwd_chunk<true>(gates, eps, out, cck, p * L, min(T, (p + 1) * L), T, B, H, ch, c, A);
}

// The backward of steps [t0, t1) of channel ch, from the last step down.  The carried
// value is K = f~_{t+1} G_{t+1} (G_t = e_t + K), e_t = dout'_t o (1 - tanh^2 c_t)
// (+ dc_n at T-1) with dout' = dout (+ dh_n at T-1); c is recomputed per 8-step group
// from its checkpoint row.  kWrite: dgates from df~ = G c_{t-1}, db~ = G and the sigmoid
// / clamp chain (the clamps pass gradient where their input is >= eps); else only the
// composed map K_out = Fa K_in + K (Fa accumulated in place).  Ends with K = f~_{t0} G_{t0}
// and G = G_{t0}.
template <bool kWrite>
__device__ __forceinline__ void bwd_chunk(const double* gates, const double* cck, const double* dout,
                                          const double* dh_n, const double* dc_n, double eps, double* dgates, int t0,
                                          int t1, int T, int B, int H, long long ch, double& K, double& G,
                                          double& Fa) {
  const long long C = (long long)B * H, b = ch / H, j = ch % H, row4 = 4ll * H;
  for (int m = (t1 - 1) / kCk; m >= t0 / kCk; --m) {
    const int g0 = m * kCk, n = min(kCk, T - g0);
    double ig[kCk], fg[kCk], gg[kCk], og[kCk], dd[kCk];
#pragma unroll
    for (int k = 0; k < kCk; ++k) {
      if (k < n) {
        const double* z = gates + ((long long)(g0 + k) * B + b) * row4 + j;
        ig[k] = z[0];
        fg[k] = z[H];
        gg[k] = z[2 * H];
        og[k] = z[3 * H];
        dd[k] = dout[(long long)(g0 + k) * C + ch];
      }
    }
    double cs[kCk + 1];
    cs[0] = cck[(long long)m * C + ch];  // c_{g0-1} (max(c0, eps) for m = 0)
#pragma unroll
    for (int k = 0; k < kCk; ++k) {
      if (k < n) {
        ig[k] = sig64(ig[k]);
        fg[k] = sig64(fg[k]);
        gg[k] = sig64(gg[k]);
        og[k] = sig64(og[k]);
        cs[k + 1] = fma(fmax(fg[k], eps), cs[k], fmax(ig[k] * gg[k], eps));
      }
    }
#pragma unroll
    for (int k = kCk - 1; k >= 0; --k) {
      if (k < n) {
        const int t = g0 + k;
        const double c = cs[k + 1], cprev = cs[k], tc = tanh(c);
        double d = dd[k];
        if (t == T - 1 && dh_n) d += dh_n[ch];
        double e = d * og[k] * (1.0 - tc * tc);
        if (t == T - 1 && dc_n) e += dc_n[ch];
        G = e + K;
        const double ff = fmax(fg[k], eps);
        if (kWrite) {
          const double bb = ig[k] * gg[k];
          const double dbb = bb >= eps ? G : 0.0;
          const double dfp = fg[k] >= eps ? (G * cprev) * fg[k] * (1.0 - fg[k]) : 0.0;
          const double dbq = dbb * bb;
          double* dq = dgates + ((long long)t * B + b) * row4 + j;
          dq[0] = dbq * (1.0 - ig[k]);
          dq[H] = dfp;
          dq[2 * H] = dbq * (1.0 - gg[k]);
          dq[3 * H] = (d * tc) * og[k] * (1.0 - og[k]);
        } else {
          Fa *= ff;
        }
        K = ff * G;
      }
    }
  }
}

// Backward pass 1: chunk p >= 1 composes to K_out = Fa K_in + Kz, kept in ka[p], kb[p].
__global__ __launch_bounds__(kScanThreads) void scan_bwd_compose_f64(const double* gates, const double* cck,
                                                                     const double* dout, const double* dh_n,
                                                                     const double* dc_n, double eps, double* ka,
                                                                     double* kb, int T, int B, int H, int L,
                                                                     int P) {
  const long long ch = blockIdx.x * (long long)kScanThreads + threadIdx.x, C = (long long)B * H;
  const int p = blockIdx.y;
  if (ch >= C || p < 1 || p >= P) return;
  double K = 0.0, G = 0.0, Fa = 1.0;
  bwd_chunk<false>(gates, cck, dout, dh_n, dc_n, eps, nullptr, p * L, min(T, (p + 1) * L), T, B, H, ch, K, G, Fa);
  ka[(long long)p * C + ch] = Fa;
  kb[(long long)p * C + ch] = K;
}

// Backward pass 2: K entering chunk p from above (0 for the last chunk), in kin[p].
__global__ __launch_bounds__(kScanThreads) void scan_bwd_carry_f64(const double* ka, const double* kb, double* kin,
                                                                   int B, int H, int P) {
  const long long ch = blockIdx.x * (long long)kScanThreads + threadIdx.x, C = (long long)B * H;
  if (ch >= C) return;
  double K = 0.0;
  for (int p = P - 1; p >= 0; --p) {
    kin[(long long)p * C + ch] = K;
    if (p >= 1) K = fma(ka[(long long)p * C + ch], K, kb[(long long)p * C + ch]);
  }
}

// Backward pass 3 (the whole scan when P = 1, kin = nullptr): dgates of chunk p; chunk 0
// also gives dc0 = G_0 f~_0 [c0 >= eps].
__global__ __launch_bounds__(kScanThreads) void scan_bwd_f64(const double* gates, const double* c0,
                                                             const double* cck, const double* dout,
                                                             const double* dh_n, const double* dc_n, double eps,
                                                             const double* kin, double* dgates, double* dc0, int T,
                                                             int B, int H, int L) {
  const long long ch = blockIdx.x * (long long)kScanThreads + threadIdx.x, C = (long long)B * H;
  if (ch >= C) return;
  const int p = blockIdx.y;
  double K = kin ? kin[(long long)p * C + ch] : 0.0, G = 0.0, Fa = 1.0;
  bwd_chunk<true>(gates, cck, dout, dh_n, dc_n, eps, dgates, p * L, min(T, (p + 1) * L), T, B, H, ch, K, G, Fa);
  if (p == 0 && dc0) {
    const bool pass = (c0 ? c0[ch] : 0.0) >= eps;
    dc0[ch] = pass ? K : 0.0;  // K = f~_0 G_0
  }
}

struct RecF64Ws {
  double* ws;    // [4H][H] W_s
  double* bs;    // [4H]
  double* big;   // fwd: gih [T][B][4H]; bwd: dg [T][B][4H]
  double* sb;    // split-K partials: fwd [S][B][4H] of h_{t-1} W_s^T, bwd [S][B][H] of dg_{t+1} W_s
  double* part;  // split-K partials of the whole-sequence products, and the column sum's chunks
  double* dcb;   // [B][H]
  double* dws;   // [4H][H] dW_hh_s
  double* db;    // [4H]
  double* rowdot;  // [4H]
};

size_t carve_rec64(void* base, size_t cap, int T, int B, int D, int H, bool bwd, RecF64Ws* o) {
  Carver c(base, cap);
  const long long TB = (long long)T * B, N4 = 4ll * H;
  o->ws = c.take<double>((size_t)N4 * H);
  o->bs = c.take<double>((size_t)N4);
  o->big = c.take<double>((size_t)TB * N4);
  if (!bwd) {
    o->sb = c.take<double>(max(part_elems(B, N4, H), (size_t)B * N4));  // S == 1 writes [B][4H]
    o->part = c.take<double>(part_elems(TB, N4, D));
    return c.off;
  }
  o->sb = c.take<double>(max(part_elems(B, H, N4), (size_t)B * H));  // S == 1 writes [B][H]
  size_t np = max(part_elems(N4, H, TB), part_elems(N4, D, TB));
  np = max(np, part_elems(TB, D, N4));
  np = max(np, (size_t)col_chunks(TB) * N4);
  o->part = c.take<double>(np);
  o->dcb = c.take<double>((size_t)B * H);
  o->dws = c.take<double>((size_t)N4 * H);
  o->db = c.take<double>((size_t)N4);
  o->rowdot = c.take<double>((size_t)N4);
  return c.off;
}

struct ParF64Ws {
  double* dg;    // [T][B][4H]
  double* part;  // split-K partials and the column sum's chunks
  double* ka;    // [P][B*H] the scan chunks' composed maps and carries
  double* kb;
  double* kin;
};

size_t carve_par64(void* base, size_t cap, int T, int B, int D, int H, ParF64Ws* o) {
  Carver c(base, cap);
  const long long TB = (long long)T * B, N4 = 4ll * H;
  o->dg = c.take<double>((size_t)TB * N4);
  size_t np = max(part_elems(N4, D, TB), part_elems(TB, D, N4));
  np = max(np, (size_t)col_chunks(TB) * N4);
  o->part = c.take<double>(np);
  const long long C = (long long)B * H;
  const size_t pc = (size_t)scan_chunks(T, scan_chunk_len(T, C)) * C;
  o->ka = c.take<double>(pc);
  o->kb = c.take<double>(pc);
  o->kin = c.take<double>(pc);
  return c.off;
}

}  // namespace
}  // namespace hsl

using namespace hsl;

extern "C" {

size_t hsl_rec_fwd_f64_ws_bytes(int T, int B, int D, int H) {
  if (T < 0 || B < 0 || D < 0 || H < 0) return 0;
  RecF64Ws w;
  return carve_rec64(nullptr, 0, T, B, D, H, false, &w);
}

int hsl_rec_fwd_f64(const double* x, const double* h0, const double* c0, const double* w_ih, const double* w_hh,
                    const double* b_ih, const double* b_hh, const double* a, double* h_save, double* c_save,
                    double* gact, double* tanh_c, void* ws, size_t ws_bytes, int T, int B, int D, int H,
                    void* stream) {
  HSL_CHECK(check_shape("hsl_rec_fwd_f64", T, B, D, H));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (B == 0 || H == 0) return HSL_OK;
  if (!w_hh || !a || !h_save || !c_save || (T > 0 && (!x || !w_ih || !b_ih || !gact || !tanh_c)))
    return fail(HSL_ERR_ARG, "hsl_rec_fwd_f64: null pointer");
  RecF64Ws w;
  const size_t need = carve_rec64(ws, ws_bytes, T, B, D, H, false, &w);
  if (!ws || ws_bytes < need) return fail(HSL_ERR_ARG, "hsl_rec_fwd_f64: workspace %zu bytes, need %zu", ws_bytes, need);
  const size_t plane = (size_t)B * H;
  HSL_CHECK(copy64(h_save, h0, (long long)plane, s));
  HSL_CHECK(copy64(c_save, c0, (long long)plane, s));
  if (T == 0) return HSL_OK;
  hipLaunchKernelGGL(scale_f64_kernel, dim3(blocks_for(4ll * H * H) < 4096 ? blocks_for(4ll * H * H) : 4096),
                     dim3(256), 0, s, w_hh, b_hh, a, w.ws, w.bs, H);
  HSL_HIP(hipGetLastError());
  // gih = x W_ih^T + b_ih
  HSL_CHECK(gemm64_split(G64{x, w_ih, b_ih, w.big, (long long)T * B, 4ll * H, D, D, 1, 1, D, 4ll * H}, w.part, s));
  for (int t = 0; t < T; ++t) {
    // sb = the S split-K partials of h_{t-1} W_s^T  [S][B][4H]
    int S = 1;
    HSL_CHECK(gemm64_parts(G64{h_save + (size_t)t * plane, w.ws, nullptr, w.sb, B, 4ll * H, H, H, 1, 1, H, 4ll * H},
                           w.sb, &S, s));
    hipLaunchKernelGGL(rec_step_fwd_f64, dim3(blocks_for((long long)B * H)), dim3(256), 0, s, w.big, w.sb, S, w.bs,
                       h_save, c_save, gact, tanh_c, t, B, H);
    HSL_HIP(hipGetLastError());
  }
  return HSL_OK;
}

size_t hsl_rec_bwd_f64_ws_bytes(int T, int B, int D, int H) {
  if (T < 0 || B < 0 || D < 0 || H < 0) return 0;
  RecF64Ws w;
  return carve_rec64(nullptr, 0, T, B, D, H, true, &w);
}

int hsl_rec_bwd_f64(const double* dout, const double* dh_n, const double* dc_n, const double* x,
                    const double* h_save, const double* c_save, const double* gact, const double* tanh_c,
                    const double* w_ih, const double* w_hh, const double* b_hh, const double* a, double* dx,
                    double* dw_ih, double* dw_hh, double* db_ih, double* db_hh, double* da, double* dh0, double* dc0,
                    void* ws, size_t ws_bytes, int T, int B, int D, int H, void* stream) {
  HSL_CHECK(check_shape("hsl_rec_bwd_f64", T, B, D, H));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (H == 0) return HSL_OK;
  if (!dw_ih || !dw_hh || !db_ih || !db_hh || !da || !w_hh || !a || !w_ih)
    return fail(HSL_ERR_ARG, "hsl_rec_bwd_f64: null pointer");
  if (T > 0 && B > 0 && (!dout || !x || !h_save || !c_save || !gact || !tanh_c))
    return fail(HSL_ERR_ARG, "hsl_rec_bwd_f64: null pointer");
  RecF64Ws w;
  const size_t need = carve_rec64(ws, ws_bytes, T, B, D, H, true, &w);
  if (!ws || ws_bytes < need) return fail(HSL_ERR_ARG, "hsl_rec_bwd_f64: workspace %zu bytes, need %zu", ws_bytes, need);
  const size_t plane = (size_t)B * H;
  if (T == 0 || B == 0) {  // no steps: zero gradients, dh0 = dh_n and dc0 = dc_n
    HSL_CHECK(copy64(dw_ih, nullptr, 4ll * H * D, s));
    HSL_CHECK(copy64(dw_hh, nullptr, 4ll * H * H, s));
    HSL_CHECK(copy64(db_ih, nullptr, 4ll * H, s));
    HSL_CHECK(copy64(db_hh, nullptr, 4ll * H, s));
    HSL_CHECK(copy64(da, nullptr, 4, s));
    if (dh0) HSL_CHECK(copy64(dh0, dh_n, (long long)plane, s));
    if (dc0) HSL_CHECK(copy64(dc0, dc_n, (long long)plane, s));
    return HSL_OK;
  }
  hipLaunchKernelGGL(scale_f64_kernel, dim3(blocks_for(4ll * H * H) < 4096 ? blocks_for(4ll * H * H) : 4096),
                     dim3(256), 0, s, w_hh, b_hh, a, w.ws, w.bs, H);
  HSL_HIP(hipGetLastError());
  const long long TB = (long long)T * B, N4 = 4ll * H;
  for (int t = T - 1; t >= 0; --t) {
    // sb = the S split-K partials of dg_{t+1} W_s  [S][B][H]
    int S = 1;
    if (t < T - 1)
      HSL_CHECK(gemm64_parts(G64{w.big + (size_t)(t + 1) * B * N4, w.ws, nullptr, w.sb, B, H, N4, N4, 1, H, 1, H},
                             w.sb, &S, s));
    hipLaunchKernelGGL(rec_step_bwd_f64, dim3(blocks_for((long long)plane)), dim3(256), 0, s, dout, dh_n, dc_n,
                       c_save, gact, tanh_c, w.sb, S, w.big, w.dcb, t, T, B, H);
    HSL_HIP(hipGetLastError());
  }
  // dh0 = dg_0 W_s, dc0 = the carried dc
  if (dh0) HSL_CHECK(gemm64_split(G64{w.big, w.ws, nullptr, dh0, B, H, N4, N4, 1, H, 1, H}, w.sb, s));
  if (dc0) HSL_CHECK(copy64(dc0, w.dcb, (long long)plane, s));
  // dW_hh_s = dg^T h_prev (h_prev = h_save[0 .. T-1]), dW_ih = dg^T x, dx = dg W_ih
  HSL_CHECK(gemm64_split(G64{w.big, h_save, nullptr, w.dws, N4, H, TB, 1, N4, H, 1, H}, w.part, s));
  HSL_CHECK(gemm64_split(G64{w.big, x, nullptr, dw_ih, N4, D, TB, 1, N4, D, 1, D}, w.part, s));
  if (dx) HSL_CHECK(gemm64_split(G64{w.big, w_ih, nullptr, dx, TB, D, N4, N4, 1, D, 1, D}, w.part, s));
  HSL_CHECK(colsum64(w.big, w.part, w.db, TB, (int)N4, s));
  hipLaunchKernelGGL(rec_final_rows_f64, dim3((unsigned)N4), dim3(64), 0, s, w_hh, b_hh, a, w.dws, w.db, dw_hh,
                     db_ih, db_hh, w.rowdot, H);
  HSL_HIP(hipGetLastError());
  hipLaunchKernelGGL(rec_da_f64, dim3(4), dim3(64), 0, s, w.rowdot, da, H);
  HSL_HIP(hipGetLastError());
  return HSL_OK;
}

int hsl_par_fwd_f64(const double* x, const double* c0, const double* w_ih, const double* b_ih, double eps,
                    double* gates, double* out, double* c_ck, int T, int B, int D, int H, void* stream) {
  HSL_CHECK(check_shape("hsl_par_fwd_f64", T, B, D, H));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (T == 0 || B == 0 || H == 0) return HSL_OK;
  if (!x || !w_ih || !b_ih || !gates || !out || !c_ck) return fail(HSL_ERR_ARG, "hsl_par_fwd_f64: null pointer");
  HSL_CHECK(gemm64(G64{x, w_ih, b_ih, gates, (long long)T * B, 4ll * H, D, D, 1, 1, D, 4ll * H}, s));
  const long long C = (long long)B * H;
  const int L = scan_chunk_len(T, C), P = scan_chunks(T, L);
  if (P > 65535) return fail(HSL_ERR_UNSUPPORTED, "hsl_par_fwd_f64: %d scan chunks", P);
  const unsigned gx = (unsigned)((C + kScanThreads - 1) / kScanThreads);
  // rows [0, 2P-1) of out hold the chunk maps until the last pass (L >= 8 keeps 2P-1 <= T)
  if (P > 1 && 2ll * P - 1 > T) return fail(HSL_ERR_UNSUPPORTED, "hsl_par_fwd_f64: %d scan chunks", P);
  if (P > 1) {
    hipLaunchKernelGGL(scan_fwd_compose_f64, dim3(gx, (unsigned)(P - 1)), dim3(kScanThreads), 0, s, gates, eps, out, T,
                       B, H, L, P);
    HSL_HIP(hipGetLastError());
    hipLaunchKernelGGL(scan_fwd_carry_f64, dim3(gx), dim3(kScanThreads), 0, s, c0, eps, out, c_ck, B, H, L, P);
    HSL_HIP(hipGetLastError());
  }
  hipLaunchKernelGGL(scan_fwd_f64, dim3(gx, (unsigned)P), dim3(kScanThreads), 0, s, gates, c0, eps, out, c_ck, T, B, H,
                     L);
  HSL_HIP(hipGetLastError());
  return HSL_OK;
}

size_t hsl_par_bwd_f64_ws_bytes(int T, int B, int D, int H) {
  if (T < 0 || B < 0 || D < 0 || H < 0) return 0;
  ParF64Ws w;
  return carve_par64(nullptr, 0, T, B, D, H, &w);
}

int hsl_par_bwd_f64(const double* dout, const double* dh_n, const double* dc_n, const double* x, const double* c0,
                    const double* gates, const double* c_ck, const double* w_ih, double eps, double* dx,
                    double* dw_ih, double* db_ih, double* dc0, void* ws, size_t ws_bytes, int T, int B, int D, int H,
                    void* stream) {
  HSL_CHECK(check_shape("hsl_par_bwd_f64", T, B, D, H));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (H == 0) return HSL_OK;
  if (!dw_ih || !db_ih || !w_ih) return fail(HSL_ERR_ARG, "hsl_par_bwd_f64: null pointer");
  ParF64Ws w;
  const size_t need = carve_par64(ws, ws_bytes, T, B, D, H, &w);
  if (!ws || ws_bytes < need) return fail(HSL_ERR_ARG, "hsl_par_bwd_f64: workspace %zu bytes, need %zu", ws_bytes, need);
  double* dg = w.dg;
  if (T == 0 || B == 0) {
    HSL_CHECK(copy64(dw_ih, nullptr, 4ll * H * D, s));
    HSL_CHECK(copy64(db_ih, nullptr, 4ll * H, s));
    if (dc0) HSL_CHECK(copy64(dc0, nullptr, (long long)B * H, s));
    return HSL_OK;
  }
  if (!dout || !x || !gates || !c_ck) return fail(HSL_ERR_ARG, "hsl_par_bwd_f64: null pointer");
  const long long C = (long long)B * H;
  const int L = scan_chunk_len(T, C), P = scan_chunks(T, L);
  if (P > 65535) return fail(HSL_ERR_UNSUPPORTED, "hsl_par_bwd_f64: %d scan chunks", P);
  const unsigned gx = (unsigned)((C + kScanThreads - 1) / kScanThreads);
  if (P > 1) {
    hipLaunchKernelGGL(scan_bwd_compose_f64, dim3(gx, (unsigned)P), dim3(kScanThreads), 0, s, gates, c_ck, dout, dh_n,
                       dc_n, eps, w.ka, w.kb, T, B, H, L, P);
    HSL_HIP(hipGetLastError());
    hipLaunchKernelGGL(scan_bwd_carry_f64, dim3(gx), dim3(kScanThreads), 0, s, w.ka, w.kb, w.kin, B, H, P);
    HSL_HIP(hipGetLastError());
  }
  hipLaunchKernelGGL(scan_bwd_f64, dim3(gx, (unsigned)P), dim3(kScanThreads), 0, s, gates, c0, c_ck, dout, dh_n, dc_n,
                     eps, P > 1 ? w.kin : nullptr, dg, dc0, T, B, H, L);
  HSL_HIP(hipGetLastError());
  const long long TB = (long long)T * B, N4 = 4ll * H;
  HSL_CHECK(gemm64_split(G64{dg, x, nullptr, dw_ih, N4, D, TB, 1, N4, D, 1, D}, w.part, s));
  if (dx) HSL_CHECK(gemm64_split(G64{dg, w_ih, nullptr, dx, TB, D, N4, N4, 1, D, 1, D}, w.part, s));
  HSL_CHECK(colsum64(dg, w.part, db_ih, TB, (int)N4, s));
  return HSL_OK;
}

}  // extern "C"
