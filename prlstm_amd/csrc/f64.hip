// fp64 modules: both modes of the training step in double precision.
//
// The reference runs fp64 modules through its torch backend (test_cpp.py:150-165) and
// its parallel functional is dtype-generic (_parallel.py:38-74).  This path computes
// every value in fp64 with the same data layouts and C-ABI shapes as the fp32 entry
// points (include/hsl.h), so the autograd functions only change the entry names.  It
// is written for exactness, not speed (gradient checks, fp64 training): per-step
// kernels with one thread per (batch row, unit), a tiled fp64 GEMM and one thread per
// channel for the scans; every sum runs in a fixed order, so results are deterministic.
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
// B(k,n) = B[k*sbk + n*sbn], C row-major with ldc.  16x16 output tiles through LDS, k in
// increasing order (one fma per k).
struct G64 {
  const double* A;
  const double* Bm;
  const double* bias;
  double* C;
  long long M, N, K, sam, sak, sbk, sbn, ldc;
};

__global__ __launch_bounds__(256) void gemm_f64_kernel(G64 g) {
  __shared__ double As[16][17];
  __shared__ double Bs[16][17];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const long long m = (long long)blockIdx.y * 16 + ty, n = (long long)blockIdx.x * 16 + tx;
  double acc = 0.0;
  for (long long k0 = 0; k0 < g.K; k0 += 16) {
    const long long ka = k0 + tx, kb = k0 + ty;
    As[ty][tx] = (m < g.M && ka < g.K) ? g.A[m * g.sam + ka * g.sak] : 0.0;
    Bs[ty][tx] = (kb < g.K && n < g.N) ? g.Bm[kb * g.sbk + n * g.sbn] : 0.0;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; ++k) acc = fma(As[ty][k], Bs[k][tx], acc);
    __syncthreads();
  }
  if (m < g.M && n < g.N) g.C[m * g.ldc + n] = (g.bias ? g.bias[n] : 0.0) + acc;
}

int gemm64(const G64& g, hipStream_t s) {
  if (g.M <= 0 || g.N <= 0) return HSL_OK;
  const long long gy = (g.M + 15) / 16, gx = (g.N + 15) / 16;
  if (gy > 65535 || gx > (1ll << 31) - 1) return fail(HSL_ERR_UNSUPPORTED, "fp64 GEMM: %lld rows", g.M);
  hipLaunchKernelGGL(gemm_f64_kernel, dim3((unsigned)gx, (unsigned)gy), dim3(256), 0, s, g);
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

// One forward step t: thread (b, u).  h_{t-1} = h_save[t], c_{t-1} = c_save[t].
__global__ void rec_step_fwd_f64(const double* gih, const double* ws, const double* bs, double* h_save,
                                 double* c_save, double* gact, double* tanh_c, int t, int B, int H) {
  const long long e = blockIdx.x * 256ll + threadIdx.x;
  if (e >= (long long)B * H) return;
  const int b = (int)(e / H), u = (int)(e % H);
  const long long plane = (long long)B * H;
  const double* hp = h_save + t * plane + (long long)b * H;
  double z[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const long long n = (long long)g * H + u;
    double acc = 0.0;
    const double* wr = ws + n * H;
    for (int k = 0; k < H; ++k) acc = fma(hp[k], wr[k], acc);
    z[g] = (gih[((long long)t * B + b) * 4 * H + n] + acc) + bs[n];
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

// dh[b][u] = sum_n dg[b][n] W_s[n][u] over n < 4H, in increasing n
__device__ __forceinline__ double dh_from_dg(const double* dg_bt, const double* ws, int u, int H) {
  double acc = 0.0;
  for (int n = 0; n < 4 * H; ++n) acc = fma(dg_bt[n], ws[(long long)n * H + u], acc);
  return acc;
}

// One backward step t (T-1 down to 0): thread (b, u).  dh = (dh_n or dg_{t+1} W_s) +
// dout_t; the cell backward with dc carried in dcb; writes dg_t.
__global__ void rec_step_bwd_f64(const double* dout, const double* dh_n, const double* dc_n, const double* c_save,
                                 const double* gact, const double* tanh_c, const double* ws, double* dg, double* dcb,
                                 int t, int T, int B, int H) {
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
    dh = dh_from_dg(dg + ((long long)(t + 1) * B + b) * row4, ws, u, H);
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

// dh0 = dg_0 W_s, dc0 = the carried dc
__global__ void rec_h0_grads_f64(const double* dg, const double* ws, const double* dcb, double* dh0, double* dc0,
                                 int B, int H) {
  const long long e = blockIdx.x * 256ll + threadIdx.x;
  if (e >= (long long)B * H) return;
  const int b = (int)(e / H), u = (int)(e % H);
  if (dh0) dh0[e] = dh_from_dg(dg + (long long)b * 4 * H, ws, u, H);
  if (dc0) dc0[e] = dcb[e];
}

// db[n] = sum over rows r < R of dg[r][n], in increasing r
__global__ void colsum_f64(const double* dg, double* db, long long R, int N) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= N) return;
  double acc = 0.0;
  for (long long r = 0; r < R; ++r) acc += dg[r * N + n];
  db[n] = acc;
}

// dW_hh = a dW_hh_s, db_ih = db, db_hh = a db; rowdot[n] = W_hh[n].dW_hh_s[n] + b_hh[n] db[n]
__global__ void rec_final_rows_f64(const double* w_hh, const double* b_hh, const double* a, const double* dws,
                                   const double* db, double* dw_hh, double* db_ih, double* db_hh, double* rowdot,
                                   int H) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= 4 * H) return;
  const double ag = a[n / H];
  double acc = 0.0;
  for (int k = 0; k < H; ++k) {
    const long long e = (long long)n * H + k;
    dw_hh[e] = ag * dws[e];
    acc = fma(w_hh[e], dws[e], acc);
  }
  rowdot[n] = acc + (b_hh ? b_hh[n] * db[n] : 0.0);
  db_ih[n] = db[n];
  db_hh[n] = ag * db[n];
}

// da[g] = sum of rowdot over the gate's H rows, in increasing row (one thread per gate)
__global__ void rec_da_f64(const double* rowdot, double* da, int H) {
  const int g = threadIdx.x;
  if (g >= 4) return;
  double acc = 0.0;
  for (int u = 0; u < H; ++u) acc += rowdot[(long long)g * H + u];
  da[g] = acc;
}

// Parallel forward scan, one thread per channel (b, j): c_t = max(f,eps) c + max(i g,eps),
// out = o tanh(c); c_ck row m = the state carried into step 8m (row 0 = max(c0, eps)),
// the last row c_{T-1}.
__global__ void scan_fwd_f64(const double* gates, const double* c0, double eps, double* out, double* cck, int T,
                             int B, int H) {
  const long long ch = blockIdx.x * 256ll + threadIdx.x, C = (long long)B * H;
  if (ch >= C) return;
  const long long b = ch / H, j = ch % H, row4 = 4ll * H;
  double c = fmax(c0 ? c0[ch] : 0.0, eps);
  for (int t = 0; t < T; ++t) {
    if (t % kCk == 0) cck[(long long)(t / kCk) * C + ch] = c;
    const double* z = gates + ((long long)t * B + b) * row4 + j;
    const double f = fmax(sig64(z[H]), eps), bb = fmax(sig64(z[0]) * sig64(z[2 * H]), eps);
    c = fma(f, c, bb);
    out[(long long)t * C + ch] = sig64(z[3 * H]) * tanh(c);
  }
  cck[(long long)((T + kCk - 1) / kCk) * C + ch] = c;
}

// Parallel backward scan, one thread per channel: for each 8-step group from the last,
// c is recomputed from the group's checkpoint row, then the group's steps run in
// reverse: G_t = e_t + f~_{t+1} G_{t+1}, e_t = dout'_t o (1 - tanh^2 c_t) (+ dc_n at T-1),
// df~ = G c_{t-1}, db~ = G, and the sigmoid / clamp chain gives dgates (the clamps pass
// gradient where their input is >= eps); dc0 = G_0 f~_0 [c0 >= eps].
__global__ void scan_bwd_f64(const double* gates, const double* c0, const double* cck, const double* dout,
                             const double* dh_n, const double* dc_n, double eps, double* dgates, double* dc0, int T,
                             int B, int H) {
  const long long ch = blockIdx.x * 256ll + threadIdx.x, C = (long long)B * H;
  if (ch >= C) return;
  const long long b = ch / H, j = ch % H, row4 = 4ll * H;
  double G = 0.0, fnext = 0.0;  // G_{t+1} and f~_{t+1} (0 past T-1)
  double first_f = 0.0;
  const int ngroups = (T + kCk - 1) / kCk;
  for (int m = ngroups - 1; m >= 0; --m) {
    const int t0 = m * kCk, t1 = min(T, t0 + kCk);
    double cs[kCk + 1];
    cs[0] = cck[(long long)m * C + ch];  // c_{t0-1} (max(c0, eps) for m = 0)
    for (int t = t0; t < t1; ++t) {
      const double* z = gates + ((long long)t * B + b) * row4 + j;
      const double f = fmax(sig64(z[H]), eps), bb = fmax(sig64(z[0]) * sig64(z[2 * H]), eps);
      cs[t - t0 + 1] = fma(f, cs[t - t0], bb);
    }
    for (int t = t1 - 1; t >= t0; --t) {
      const double* z = gates + ((long long)t * B + b) * row4 + j;
      const double ig = sig64(z[0]), fg = sig64(z[H]), gg = sig64(z[2 * H]), og = sig64(z[3 * H]);
      const double c = cs[t - t0 + 1], cprev = cs[t - t0], tc = tanh(c);
      double d = dout[(long long)t * C + ch];
      if (t == T - 1 && dh_n) d += dh_n[ch];
      double e = d * og * (1.0 - tc * tc);
      if (t == T - 1 && dc_n) e += dc_n[ch];
      G = e + fnext * G;
      const double bb = ig * gg;
      const double dbb = bb >= eps ? G : 0.0;
      const double dfp = fg >= eps ? (G * cprev) * fg * (1.0 - fg) : 0.0;
      const double dbq = dbb * bb;
      double* dq = dgates + ((long long)t * B + b) * row4 + j;
      dq[0] = dbq * (1.0 - ig);
      dq[H] = dfp;
      dq[2 * H] = dbq * (1.0 - gg);
      dq[3 * H] = (d * tc) * og * (1.0 - og);
      fnext = fmax(fg, eps);
      first_f = fnext;
    }
  }
  if (dc0) {
    const bool pass = (c0 ? c0[ch] : 0.0) >= eps;
    dc0[ch] = (pass && T > 0) ? G * first_f : 0.0;
  }
}

struct RecF64Ws {
  double* ws;    // [4H][H] W_s
  double* bs;    // [4H]
  double* big;   // fwd: gih [T][B][4H]; bwd: dg [T][B][4H]
  double* dcb;   // [B][H]
  double* dws;   // [4H][H] dW_hh_s
  double* db;    // [4H]
  double* rowdot;  // [4H]
};

size_t carve_rec64(void* base, size_t cap, int T, int B, int H, bool bwd, RecF64Ws* o) {
  Carver c(base, cap);
  o->ws = c.take<double>((size_t)4 * H * H);
  o->bs = c.take<double>((size_t)4 * H);
  o->big = c.take<double>((size_t)T * B * 4 * H);
  if (bwd) {
    o->dcb = c.take<double>((size_t)B * H);
    o->dws = c.take<double>((size_t)4 * H * H);
    o->db = c.take<double>((size_t)4 * H);
    o->rowdot = c.take<double>((size_t)4 * H);
  }
  return c.off;
}

}  // namespace
}  // namespace hsl

using namespace hsl;

extern "C" {

size_t hsl_rec_fwd_f64_ws_bytes(int T, int B, int D, int H) {
  if (T < 0 || B < 0 || D < 0 || H < 0) return 0;
  RecF64Ws w;
  return carve_rec64(nullptr, 0, T, B, H, false, &w);
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
  const size_t need = carve_rec64(ws, ws_bytes, T, B, H, false, &w);
  if (!ws || ws_bytes < need) return fail(HSL_ERR_ARG, "hsl_rec_fwd_f64: workspace %zu bytes, need %zu", ws_bytes, need);
  const size_t plane = (size_t)B * H;
  HSL_CHECK(copy64(h_save, h0, (long long)plane, s));
  HSL_CHECK(copy64(c_save, c0, (long long)plane, s));
  if (T == 0) return HSL_OK;
  hipLaunchKernelGGL(scale_f64_kernel, dim3(blocks_for(4ll * H * H) < 4096 ? blocks_for(4ll * H * H) : 4096),
                     dim3(256), 0, s, w_hh, b_hh, a, w.ws, w.bs, H);
  HSL_HIP(hipGetLastError());
  // gih = x W_ih^T + b_ih
  HSL_CHECK(gemm64(G64{x, w_ih, b_ih, w.big, (long long)T * B, 4ll * H, D, D, 1, 1, D, 4ll * H}, s));
  for (int t = 0; t < T; ++t) {
    hipLaunchKernelGGL(rec_step_fwd_f64, dim3(blocks_for((long long)B * H)), dim3(256), 0, s, w.big, w.ws, w.bs,
                       h_save, c_save, gact, tanh_c, t, B, H);
    HSL_HIP(hipGetLastError());
  }
  return HSL_OK;
}

size_t hsl_rec_bwd_f64_ws_bytes(int T, int B, int D, int H) {
  if (T < 0 || B < 0 || D < 0 || H < 0) return 0;
  RecF64Ws w;
  return carve_rec64(nullptr, 0, T, B, H, true, &w);
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
  const size_t need = carve_rec64(ws, ws_bytes, T, B, H, true, &w);
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
  for (int t = T - 1; t >= 0; --t) {
    hipLaunchKernelGGL(rec_step_bwd_f64, dim3(blocks_for((long long)plane)), dim3(256), 0, s, dout, dh_n, dc_n,
                       c_save, gact, tanh_c, w.ws, w.big, w.dcb, t, T, B, H);
    HSL_HIP(hipGetLastError());
  }
  if (dh0 || dc0) {
    hipLaunchKernelGGL(rec_h0_grads_f64, dim3(blocks_for((long long)plane)), dim3(256), 0, s, w.big, w.ws, w.dcb,
                       dh0, dc0, B, H);
    HSL_HIP(hipGetLastError());
  }
  const long long TB = (long long)T * B, N4 = 4ll * H;
  // dW_hh_s = dg^T h_prev (h_prev = h_save[0 .. T-1]), dW_ih = dg^T x, dx = dg W_ih
  HSL_CHECK(gemm64(G64{w.big, h_save, nullptr, w.dws, N4, H, TB, 1, N4, H, 1, H}, s));
  HSL_CHECK(gemm64(G64{w.big, x, nullptr, dw_ih, N4, D, TB, 1, N4, D, 1, D}, s));
  if (dx) HSL_CHECK(gemm64(G64{w.big, w_ih, nullptr, dx, TB, D, N4, N4, 1, D, 1, D}, s));
  hipLaunchKernelGGL(colsum_f64, dim3(blocks_for(N4)), dim3(256), 0, s, w.big, w.db, TB, (int)N4);
  HSL_HIP(hipGetLastError());
  hipLaunchKernelGGL(rec_final_rows_f64, dim3(blocks_for(N4)), dim3(256), 0, s, w_hh, b_hh, a, w.dws, w.db, dw_hh,
                     db_ih, db_hh, w.rowdot, H);
  HSL_HIP(hipGetLastError());
  hipLaunchKernelGGL(rec_da_f64, dim3(1), dim3(64), 0, s, w.rowdot, da, H);
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
  hipLaunchKernelGGL(scan_fwd_f64, dim3(blocks_for((long long)B * H)), dim3(256), 0, s, gates, c0, eps, out, c_ck, T,
                     B, H);
  HSL_HIP(hipGetLastError());
  return HSL_OK;
}

size_t hsl_par_bwd_f64_ws_bytes(int T, int B, int D, int H) {
  if (T < 0 || B < 0 || D < 0 || H < 0) return 0;
  Carver c(nullptr, 0);
  c.take<double>((size_t)T * B * 4 * H);
  return c.off;
}

int hsl_par_bwd_f64(const double* dout, const double* dh_n, const double* dc_n, const double* x, const double* c0,
                    const double* gates, const double* c_ck, const double* w_ih, double eps, double* dx,
                    double* dw_ih, double* db_ih, double* dc0, void* ws, size_t ws_bytes, int T, int B, int D, int H,
                    void* stream) {
  HSL_CHECK(check_shape("hsl_par_bwd_f64", T, B, D, H));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (H == 0) return HSL_OK;
  if (!dw_ih || !db_ih || !w_ih) return fail(HSL_ERR_ARG, "hsl_par_bwd_f64: null pointer");
  Carver cv(ws, ws_bytes);
  double* dg = cv.take<double>((size_t)T * B * 4 * H);
  if (!ws || ws_bytes < cv.off) return fail(HSL_ERR_ARG, "hsl_par_bwd_f64: workspace %zu bytes, need %zu", ws_bytes, cv.off);
  if (T == 0 || B == 0) {
    HSL_CHECK(copy64(dw_ih, nullptr, 4ll * H * D, s));
    HSL_CHECK(copy64(db_ih, nullptr, 4ll * H, s));
    if (dc0) HSL_CHECK(copy64(dc0, nullptr, (long long)B * H, s));
    return HSL_OK;
  }
  if (!dout || !x || !gates || !c_ck) return fail(HSL_ERR_ARG, "hsl_par_bwd_f64: null pointer");
  hipLaunchKernelGGL(scan_bwd_f64, dim3(blocks_for((long long)B * H)), dim3(256), 0, s, gates, c0, c_ck, dout, dh_n,
                     dc_n, eps, dg, dc0, T, B, H);
  HSL_HIP(hipGetLastError());
  const long long TB = (long long)T * B, N4 = 4ll * H;
  HSL_CHECK(gemm64(G64{dg, x, nullptr, dw_ih, N4, D, TB, 1, N4, D, 1, D}, s));
  if (dx) HSL_CHECK(gemm64(G64{dg, w_ih, nullptr, dx, TB, D, N4, N4, 1, D, 1, D}, s));
  hipLaunchKernelGGL(colsum_f64, dim3(blocks_for(N4)), dim3(256), 0, s, dg, db_ih, TB, (int)N4);
  HSL_HIP(hipGetLastError());
  return HSL_OK;
}

}  // extern "C"
