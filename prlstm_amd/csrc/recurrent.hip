// Recurrent mode of HeadStartLSTM: forward time loop, BPTT and parameter gradients.
//
// Reference behaviour: HeadStartLSTMTorchFn (src/headstartlstm/_torch.py:86-170):
//   W_hh_s = a_rep (.) W_hh, b_hh_s = a_rep (.) b_hh           (_torch.py:91-94)
//   gih    = x W_ih^T + b_ih                                    (_torch.py:96)
//   z_t    = gih[t] + h_{t-1} W_hh_s^T + b_hh_s; cell          (_torch.py:111-120, :27-36)
//   reverse loop dh += dout[t]; cell bwd; dh = dg W_hh_s        (_torch.py:143-150, :39-53)
//   dW_hh_s = dg^T h_prev, dW_ih = dg^T x, db = sum dg, dx = dg W_ih, a-unscale (:153-168)
//
// Two implementations of the time loops:
//  * persistent (H <= 512, groups fit on the chip): one launch runs all T steps.  The
//    batch is split into groups of <= 4 rows; group g is served by workgroups
//    blockIdx % NG == g, which for NG = 8 are exactly the 32 workgroups of XCD g.
//    Each workgroup owns 16 hidden units (64 gate rows) and keeps its a-scaled
//    W_hh slice in VGPRs for the whole launch.  The per-step product runs on
//    v_mfma_f32_4x4x1_16b_f32 with the A operand (4 batch rows) broadcast to all 16
//    blocks (cbsz=4), so one instruction covers 4 batch rows x 64 gate rows.
//    Workgroups of a group hand h_t (forward) and partial dh (backward) to each other
//    through 4-byte words in rotating slots, with bounded waits.
//  * per-step (any shape): one fused GEMM+cell kernel per time step.
//
// v_mfma_f32_4x4x1_16b_f32 layout (verified on gfx950): A from lane 4b+i is
// A_b[i][0], B from lane 4b+j is B_b[0][j], result lane 4b+j, reg i holds D_b[i][j].
// With cbsz=4, abid=0 every block uses block 0's A (lanes 0-3).
#include <algorithm>
#include <mutex>
#include <cstdlib>
#include <type_traits>

#include "gemm_core.h"
#include "split_bf16.h"

namespace hsl {

// Per-step products: 32x32 tiles, four waves splitting each 128-deep k-slice.
using CfgStep = GemmCfg<32, 32, 128, 1, 1, 4>;
// Two register stages: the loads of slice s+1 are in flight while slice s multiplies.
constexpr int kStepDepth = 2;

namespace {

constexpr int kUnits = 16;       // hidden units per persistent workgroup
constexpr int kPadLdsBytes = 96 * 1024;  // dynamic LDS that keeps one persistent workgroup per CU

// ---------------------------------------------------------------------------------
// small helper kernels
// ---------------------------------------------------------------------------------
__global__ void fill_u64_kernel(unsigned long long* p, size_t n, unsigned long long v) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    p[i] = v;
}

// Fills three word ranges in one launch (error flag, hand-off slots, placement words);
// the slots, the bulk, with 16-byte stores when they are 16-byte aligned.
__global__ void fill3_u64_kernel(unsigned long long* a, size_t na, unsigned long long va, unsigned long long* b,
                                 size_t nb, unsigned long long vb, unsigned long long* c, size_t nc,
                                 unsigned long long vc) {
  const size_t tid = blockIdx.x * (size_t)blockDim.x + threadIdx.x, nth = (size_t)gridDim.x * blockDim.x;
  const size_t n16 = reinterpret_cast<uintptr_t>(b) % 16 == 0 ? nb / 2 : 0;
  ulonglong2* const b2 = reinterpret_cast<ulonglong2*>(b);
  for (size_t i = tid; i < n16; i += nth) b2[i] = make_ulonglong2(vb, vb);
  for (size_t i = 2 * n16 + tid; i < nb; i += nth) b[i] = vb;
  for (size_t i = tid; i < na; i += nth) a[i] = va;
  for (size_t i = tid; i < nc; i += nth) c[i] = vc;
}

__global__ void copy_f32_kernel(float* dst, const float* src, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    dst[i] = src ? src[i] : 0.f;
}

// W_s[n][k] = a[n/H] * W_hh[n][k] (reference layout) and, when w_perm is set, the
// unit-interleaved copy w_perm[4u+g][k] = W_s[g*H+u][k] used by the per-step forward.
// bs[n] = a[n/H] * b_hh[n].
__global__ void scale_whh_kernel(const float* __restrict__ w_hh, const float* __restrict__ b_hh,
                                 const float* __restrict__ a, float* __restrict__ w_s, float* __restrict__ w_perm,
                                 float* __restrict__ bs, int H) {
  const size_t total = (size_t)4 * H * H;
  for (size_t e = blockIdx.x * (size_t)blockDim.x + threadIdx.x; e < total; e += (size_t)gridDim.x * blockDim.x) {
    const int n = (int)(e / H), k = (int)(e % H);
    const int g = n / H, u = n % H;
    const float v = a[g] * w_hh[e];
    if (w_s) w_s[e] = v;
    if (w_perm) w_perm[(size_t)(4 * u + g) * H + k] = v;
  }
  if (bs) {
    for (int n = blockIdx.x * blockDim.x + threadIdx.x; n < 4 * H; n += gridDim.x * blockDim.x) bs[n] = a[n / H] * b_hh[n];
  }
}

// db_part[b][n] = sum_t dg[t][b][n] in fp64.
__global__ void colsum_time_kernel(const float* __restrict__ dg, double* __restrict__ db_part, int T, int BN4) {
  for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < BN4; e += gridDim.x * blockDim.x) {
    double acc = 0.0;
    for (int t = 0; t < T; ++t) acc += (double)dg[(size_t)t * BN4 + e];
    db_part[e] = acc;
  }
}

// dW_hh_s = sum of split-K partials (fp64); dW_hh = a * dW_hh_s; rowdot[n] = sum_k W_hh[n][k] dW_hh_s[n][k].
// Blocks past the 4H rows (when X is non-null) add the dW_ih planes X[xplanes][xn] in fp64
// of the fused backward into dw_ih, in the same launch.
__global__ __launch_bounds__(256) void whh_grad_finalize_kernel(const float* __restrict__ P, int splits,
                                                                const float* __restrict__ w_hh,
                                                                const float* __restrict__ a, float* __restrict__ dw_hh,
                                                                double* __restrict__ rowdot, int H,
                                                                const float* __restrict__ X, int xplanes,
                                                                float* __restrict__ dw_ih, size_t xn) {
  __shared__ double red[256];
  const int n = blockIdx.x;
  if (n >= 4 * H) {
    const size_t nb = gridDim.x - 4 * H;
    for (size_t e = (size_t)(n - 4 * H) * blockDim.x + threadIdx.x; e < xn; e += nb * blockDim.x) {
      double v = 0.0;
#pragma unroll 4
      for (int z = 0; z < xplanes; ++z) v += (double)X[(size_t)z * xn + e];
      dw_ih[e] = (float)v;
    }
    return;
  }
  const size_t plane = (size_t)4 * H * H;
  const float ag = a[n / H];
  double acc = 0.0;
  for (int k = threadIdx.x; k < H; k += blockDim.x) {
    const size_t e = (size_t)n * H + k;
    double v = 0.0;
#pragma unroll 4
    for (int z = 0; z < splits; ++z) v += (double)P[(size_t)z * plane + e];
    const float s = (float)v;
    dw_hh[e] = ag * s;
    acc += (double)w_hh[e] * (double)s;
  }
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) rowdot[n] = red[0];
}

// whh_grad_finalize_kernel on 16-byte groups (H % 4 == 0, every pointer 16-byte aligned):
// one wave per row n of dW_hh, each lane's planes requested in batches of 8 before they
// are added, and the row's da term reduced across the wave without LDS or barriers.
// Each element's planes are added in plane order from 0.0 in fp64, as in the kernel
// above, so dW_hh and dW_ih come out bit for bit the same; only the order of rowdot's
// fp64 sum differs.  Blocks past the 4H/4 row blocks sum the dW_ih planes.
__global__ __launch_bounds__(256) void whh_grad_finalize4_kernel(const float4* __restrict__ P, int splits,
                                                                 const float4* __restrict__ w_hh,
                                                                 const float* __restrict__ a,
                                                                 float4* __restrict__ dw_hh,
                                                                 double* __restrict__ rowdot, int H,
                                                                 const float4* __restrict__ X, int xplanes,
                                                                 float4* __restrict__ dw_ih, size_t xn4) {
  constexpr int kBatch = 8;
  const int rblocks = H;  // 4H rows, four per block
  auto add4 = [](double (&v)[4], const float4 q) {
    v[0] += (double)q.x;
    v[1] += (double)q.y;
    v[2] += (double)q.z;
    v[3] += (double)q.w;
  };
  auto sum_planes = [&](const float4* base, size_t stride, int nplanes, double (&v)[4]) {
    for (int z0 = 0; z0 < nplanes; z0 += kBatch) {
      float4 q[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i)
        q[i] = z0 + i < nplanes ? base[(size_t)(z0 + i) * stride] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int i = 0; i < kBatch; ++i) add4(v, q[i]);  // adding +0.0 past the last plane is exact
    }
  };
  if ((int)blockIdx.x >= rblocks) {
    const size_t nb = gridDim.x - rblocks;
    for (size_t e = (size_t)(blockIdx.x - rblocks) * blockDim.x + threadIdx.x; e < xn4; e += nb * blockDim.x) {
      double v[4] = {0.0, 0.0, 0.0, 0.0};
      sum_planes(X + e, xn4, xplanes, v);
      dw_ih[e] = make_float4((float)v[0], (float)v[1], (float)v[2], (float)v[3]);
    }
    return;
  }
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);  // < 4H: rblocks * 4 rows
  const int H4 = H / 4;
  const size_t plane4 = (size_t)H * H;  // 4H * H floats
  const float ag = a[n / H];
  double acc = 0.0;
  for (int k = lane; k < H4; k += 64) {
    const size_t e = (size_t)n * H4 + k;
    double v[4] = {0.0, 0.0, 0.0, 0.0};
    sum_planes(P + e, plane4, splits, v);
    const float4 s = make_float4((float)v[0], (float)v[1], (float)v[2], (float)v[3]);
    dw_hh[e] = make_float4(ag * s.x, ag * s.y, ag * s.z, ag * s.w);
    const float4 w = w_hh[e];
    acc += (double)w.x * (double)s.x;
    acc += (double)w.y * (double)s.y;
    acc += (double)w.z * (double)s.z;
    acc += (double)w.w * (double)s.w;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
  if (lane == 0) rowdot[n] = acc;
}

// Adds column entries p[b * stride] for b = b0, b0 + 1, ... in chunks of C into ps[b % 8]
// (b0 a multiple of 8); a chunk's C loads are all issued before the first addition.
template <int C>
__device__ __forceinline__ void add_parts(const double* __restrict__ p, size_t stride, int& b, int B, double (&ps)[8]) {
  for (; b + C <= B; b += C) {
    double v[C];
#pragma unroll
    for (int i = 0; i < C; ++i) v[i] = p[(size_t)(b + i) * stride];
#pragma unroll
    for (int i = 0; i < C; ++i) ps[i & 7] += v[i];
  }
}

// db_ih = db_hh_s = sum_b db_part[b][n]; db_hh = a * db; da[g] = sum_{n in g} rowdot[n] + b_hh[n] db[n].
// One workgroup per gate, one unit per thread while H <= 1024: the kernel is a handful of
// memory round trips, so every thread keeps all of its unit's partial loads in flight.
__global__ __launch_bounds__(1024) void bias_da_finalize_kernel(const double* __restrict__ db_part, int B,
                                                                const double* __restrict__ rowdot,
                                                                const float* __restrict__ b_hh,
                                                                const float* __restrict__ a, float* __restrict__ db_ih,
                                                                float* __restrict__ db_hh, float* __restrict__ da, int H,
                                                                const double* __restrict__ dotp, int dot_parts) {
  __shared__ double red[1024];
  const int g = blockIdx.x;
  const float ag = a ? a[g] : 1.0f;
  double acc = 0.0;
  for (int u = threadIdx.x; u < H; u += blockDim.x) {
    const int n = g * H + u;
    // eight independent partial sums, b % 8 each, in increasing b (fixed order: deterministic)
    double ps[8] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
    int b = 0;
    add_parts<32>(db_part + n, (size_t)4 * H, b, B, ps);
    add_parts<16>(db_part + n, (size_t)4 * H, b, B, ps);
    add_parts<8>(db_part + n, (size_t)4 * H, b, B, ps);
    for (; b < B; ++b) ps[0] += db_part[(size_t)b * 4 * H + n];
    const double s = ((ps[0] + ps[1]) + (ps[2] + ps[3])) + ((ps[4] + ps[5]) + (ps[6] + ps[7]));
    const float db = (float)s;
    if (db_ih) db_ih[n] = db;
    if (db_hh) db_hh[n] = ag * db;
    acc += (rowdot ? rowdot[n] : 0.0) + (b_hh ? (double)b_hh[n] * (double)db : 0.0);
  }
  if (dotp)
    for (int i = threadIdx.x; i < dot_parts; i += blockDim.x) acc += dotp[(size_t)g * dot_parts + i];
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int w = blockDim.x / 2; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0 && da) da[g] = (float)red[0];
}

// ---------------------------------------------------------------------------------
// per-step path: fused epilogues of the step GEMMs
// ---------------------------------------------------------------------------------
// Forward step t: tile columns are unit-interleaved (4u+g), so one tile holds all four
// gates of BN/4 units.  z = (gih + h W_s^T) + b_s (reference order), then the cell.
struct EpiCellFwd {
  const float* gih;     // [B,4H] at t
  const float* bs;      // [4H]
  const float* c_prev;  // [B,H]
  float* h_out;         // [B,H]
  float* c_out;         // [B,H]
  float* gact;          // [B,H,4] at t
  float* tanh_c;        // [B,H] at t
  int B, H;
  template <class Cfg>
  __device__ __forceinline__ void run(const float* Cs, int m0, int n0, int) const {
    constexpr int units = Cfg::BN / 4;
    for (int e = threadIdx.x; e < Cfg::BM * units; e += Cfg::kThreads) {
      const int m = e / units, uu = e % units;
      const int b = m0 + m, u = n0 / 4 + uu;
      if (b >= B || u >= H) continue;
      float act[4];
#pragma unroll
      for (int gt = 0; gt < 4; ++gt) {
        const int n = gt * H + u;
        const float z = (gih[(size_t)b * 4 * H + n] + tile_value<Cfg>(Cs, m, 4 * uu + gt)) + bs[n];
        act[gt] = sigmoid_f(z);
      }
      *reinterpret_cast<f4*>(gact + ((size_t)b * H + u) * 4) = f4{act[0], act[1], act[2], act[3]};
      const float c = act[1] * c_prev[(size_t)b * H + u] + act[0] * act[2];
      const float tc = tanh_f(c);
      h_out[(size_t)b * H + u] = act[3] * tc;
      c_out[(size_t)b * H + u] = c;
      tanh_c[(size_t)b * H + u] = tc;
    }
  }
};

// Cell backward (_torch.py:39-53) for one (b, u); returns the four pre-activation grads.
__device__ __forceinline__ void cell_bwd(float dh, float& dc, float cp, float i, float f, float g, float o, float tc,
                                         float dg[4]) {
  const float d_o = dh * tc;
  const float dct = dc + dh * o * (1.0f - tc * tc);
  const float d_f = dct * cp;
  dc = dct * f;
  const float d_i = dct * g;
  const float d_g = dct * i;
  dg[0] = d_i * i * (1.0f - i);
  dg[1] = d_f * f * (1.0f - f);
  dg[2] = d_g * g * (1.0f - g);
  dg[3] = d_o * o * (1.0f - o);
}

// Backward step t: tile = dg[t+1] W_s (columns = units).  dh = (tile + dh_n) + dout[t].
struct EpiCellBwd {
  const float* dout;     // [B,H] at t
  const float* dh_extra; // dh_n at t == T-1, else null
  const float* c_prev;   // c_save[t]
  const float* gact;     // [B,H,4] at t
  const float* tanh_c;   // [B,H] at t
  float* dc;             // [B,H] carry, updated in place
  float* dg;             // [B,4H] at t
  int B, H;
  template <class Cfg>
  __device__ __forceinline__ void run(const float* Cs, int m0, int n0, int) const {
    for (int e = threadIdx.x; e < Cfg::BM * Cfg::BN; e += Cfg::kThreads) {
      const int m = e / Cfg::BN, nn = e % Cfg::BN;
      const int b = m0 + m, u = n0 + nn;
      if (b >= B || u >= H) continue;
      const size_t bu = (size_t)b * H + u;
      float dh = tile_value<Cfg>(Cs, m, nn);
      if (dh_extra) dh = dh + dh_extra[bu];
      dh = dh + dout[bu];
      const f4 ga = *reinterpret_cast<const f4*>(gact + ((size_t)b * H + u) * 4);
      float dcv = dc[bu];
      float d[4];
      cell_bwd(dh, dcv, c_prev[bu], ga[0], ga[1], ga[2], ga[3], tanh_c[bu], d);
      dc[bu] = dcv;
#pragma unroll
      for (int gt = 0; gt < 4; ++gt) dg[(size_t)b * 4 * H + gt * H + u] = d[gt];
    }
  }
};

// Split-K form of the per-step cells: the step GEMM writes S fp32 partial planes
// P[S][B][N] (EpiPartial) and one thread per (b, u) adds them in plane order and runs
// the cell.  Used when the output has too few 32x32 tiles to fill the chip (the
// backward product dg W_s has only B x H outputs for a 4H-long reduction).
__global__ __launch_bounds__(256) void step_cell_fwd_kernel(const float* __restrict__ P, int S,
                                                           const float* __restrict__ gih, const float* __restrict__ bs,
                                                           const float* __restrict__ c_prev, float* __restrict__ h_out,
                                                           float* __restrict__ c_out, float* __restrict__ gact,
                                                           float* __restrict__ tanh_c, int B, int H) {
  const size_t n = (size_t)B * H, plane = (size_t)B * 4 * H;
  for (size_t e = blockIdx.x * (size_t)blockDim.x + threadIdx.x; e < n; e += (size_t)gridDim.x * blockDim.x) {
    const int b = (int)(e / H), u = (int)(e % H);
    const size_t col = (size_t)b * 4 * H + 4 * u;  // unit-interleaved columns 4u+g
    f4 z = *reinterpret_cast<const f4*>(P + col);
    for (int sp = 1; sp < S; ++sp) z += *reinterpret_cast<const f4*>(P + sp * plane + col);
    float act[4];
#pragma unroll
    for (int gt = 0; gt < 4; ++gt) {
      const int nn = gt * H + u;
      act[gt] = sigmoid_f((gih[(size_t)b * 4 * H + nn] + z[gt]) + bs[nn]);
    }
    *reinterpret_cast<f4*>(gact + e * 4) = f4{act[0], act[1], act[2], act[3]};
    const float c = act[1] * c_prev[e] + act[0] * act[2];
    const float tc = tanh_f(c);
    h_out[e] = act[3] * tc;
    c_out[e] = c;
    tanh_c[e] = tc;
  }
}

__global__ __launch_bounds__(256) void step_cell_bwd_kernel(const float* __restrict__ P, int S,
                                                           const float* __restrict__ dh_extra,
                                                           const float* __restrict__ dout,
                                                           const float* __restrict__ c_prev,
                                                           const float* __restrict__ gact,
                                                           const float* __restrict__ tanh_c, float* __restrict__ dc,
                                                           float* __restrict__ dg, int B, int H) {
  const size_t n = (size_t)B * H;
  for (size_t e = blockIdx.x * (size_t)blockDim.x + threadIdx.x; e < n; e += (size_t)gridDim.x * blockDim.x) {
    const int b = (int)(e / H), u = (int)(e % H);
    float dh = 0.f;
    for (int sp = 0; sp < S; ++sp) dh += P[sp * n + e];
    if (dh_extra) dh = dh + dh_extra[e];
    dh = dh + dout[e];
    const f4 ga = *reinterpret_cast<const f4*>(gact + e * 4);
    float dcv = dc[e];
    float d[4];
    cell_bwd(dh, dcv, c_prev[e], ga[0], ga[1], ga[2], ga[3], tanh_c[e], d);
    dc[e] = dcv;
#pragma unroll
    for (int gt = 0; gt < 4; ++gt) dg[(size_t)b * 4 * H + gt * H + u] = d[gt];
  }
}

// ---------------------------------------------------------------------------------
// persistent path
// ---------------------------------------------------------------------------------
// Hand-off between the workgroups of a batch group.  Values travel as 4-byte words in
// rotating slots that start out holding kEmpty, a signalling-NaN pattern: arithmetic
// never produces one (NaN results are quiet, i.e. have bit 22 set), and every published
// value is an arithmetic result, so a word is ready as soon as it differs from kEmpty.
// A word is set back to kEmpty by the lane that owns it once every reader is known to
// be done with it, and written again only slots later; see the two kernels for the
// exact schedule.
//
// Readers poll with relaxed device-scope loads (sc1), which are served by the reader's
// L2.  When every member of the group runs on the same XCD (checked at launch start,
// see agree_placement), writers use workgroup-scope stores, which land in that shared
// L2; a store's completion, which every later poll of the writing wave waits for, then
// means it is visible to the whole group.  Otherwise writers use device-scope stores
// and each step adds a device-scope release before its publish and an acquire after
// its receive (write-back and invalidation of the XCD's L2).
constexpr unsigned kEmpty = 0xFFFFFFFFu;
constexpr unsigned long long kEmpty2 = ~0ull;

}  // namespace

// Device errors of this library since they were last read (one word per device, sticky):
// bit 0 = a persistent kernel gave up a wait between workgroups.  Read and cleared by
// hsl_device_errors.
__device__ unsigned g_device_errors;

namespace {

// A wait gave up: the workgroup's LDS abort flag, the call's workspace flag and the
// sticky device word are raised (vector atomics to global memory).
__device__ __forceinline__ void raise_abort(int* abort_flag, int* err) {
  *abort_flag = 1;
  atomicOr(err, 1);
  atomicOr(&g_device_errors, 1u);
}
__device__ __forceinline__ float canon_nan(float v) { return v == v ? v : __uint_as_float(0x7FC00000u); }

// base + a byte offset held in 32 bits.  With a wave-uniform base this is the form
// global memory instructions take directly (scalar base + 32-bit vector offset), so
// no 64-bit address arithmetic runs per lane.
template <class T>
__device__ __forceinline__ T* byte_at(T* base, unsigned off) {
  using C = std::conditional_t<std::is_const_v<T>, const char, char>;
  return reinterpret_cast<T*>(reinterpret_cast<C*>(base) + off);
}

// All hand-off accesses address a uniform base plus a 32-bit lane offset (in words).
template <bool FAST>
__device__ __forceinline__ void word_put(float* base, unsigned off, float v) {
  unsigned* u = byte_at(reinterpret_cast<unsigned*>(base), 4u * off);
  if constexpr (FAST)
    __hip_atomic_store(u, __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  else
    __hip_atomic_store(u, __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A lane's N (1, 2, 4 or 8) words inside a block of 64 lanes: with N == 1 word 0 of
// lane l is at l; otherwise word j is at 128*(j/2) + 2*l + j%2, so a lane's words pair
// up into 8-byte loads and stores and the 64 lanes of a pair are contiguous.
template <int N>
__device__ __forceinline__ unsigned lane_word(unsigned l, unsigned j) {
  if constexpr (N == 1)
    return l;
  else
    return 128u * (j >> 1) + 2u * l + (j & 1u);
}

// off = block offset + lane_word<N>(lane, 0).
template <int N, bool FAST>
__device__ __forceinline__ void words_clear(float* base, unsigned off) {
  if constexpr (N == 1) {
    word_put<FAST>(base, off, __uint_as_float(kEmpty));
  } else {
    const unsigned long long e = kEmpty2;
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      unsigned long long* u = byte_at(reinterpret_cast<unsigned long long*>(base), 4u * (off + 128u * i));
      if constexpr (FAST)
        __hip_atomic_store(u, e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      else
        __hip_atomic_store(u, e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// Loads the lane's words whose flag in `need` is set (pairs are loaded together).
template <int N>
__device__ __forceinline__ void words_load(const float* base, unsigned off, const bool (&need)[N],
                                           unsigned (&v)[N]) {
  if constexpr (N == 1) {
    if (need[0])
      v[0] = __hip_atomic_load(byte_at(reinterpret_cast<unsigned*>(const_cast<float*>(base)), 4u * off),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      if (need[2 * i] || need[2 * i + 1]) {
        const unsigned long long w =
            __hip_atomic_load(byte_at(reinterpret_cast<unsigned long long*>(const_cast<float*>(base)),
                                      4u * (off + 128u * i)),
                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        v[2 * i] = static_cast<unsigned>(w);
        v[2 * i + 1] = static_cast<unsigned>(w >> 32);
      }
    }
  }
}

// Polls the lane's words until every word flagged in `expect` differs from kEmpty.
// Returns false (after setting the error flags) when the spin limit runs out.
template <int N>
__device__ __forceinline__ bool words_wait(const float* base, unsigned off, const bool (&expect)[N],
                                           unsigned (&v)[N], long long spin, int* abort_flag, int* err) {
  bool need[N];
#pragma unroll
  for (int j = 0; j < N; ++j) {
    need[j] = expect[j];
    v[j] = 0u;
  }
  words_load<N>(base, off, need, v);
  const long long t0 = wall_clock64();
  while (true) {
    bool ok = true;
#pragma unroll
    for (int j = 0; j < N; ++j) {
      need[j] = expect[j] && v[j] == kEmpty;
      ok = ok && !need[j];
    }
    if (__all(ok)) return true;
    if (wall_clock64() - t0 > spin) {
      raise_abort(abort_flag, err);
      return false;
    }
    words_load<N>(base, off, need, v);
  }
}

// x[l] + x[l ^ 16] and x[l] + x[l ^ 32] with gfx950's row and half swaps: with both
// operands x, the two results of a swap hold x[l] and x[partner] in every lane.
__device__ __forceinline__ float add_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float add_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ unsigned xcc_id() {
  unsigned x;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
  return x;
}


// Every workgroup of the group publishes its XCD id (device-scope) and reads all of
// the group's; returns true when they are all equal.  All members see the same words,
// so they all choose the same store mode.  Returns false and sets *abort on timeout.
__device__ bool agree_placement(unsigned long long* hello, int wg, int nw, long long spin, int* abort_flag,
                                int* err) {
  __shared__ int differs;
  const int tid = threadIdx.x;
  if (tid == 0) {
    differs = 0;
    tag_store(hello + wg, __uint_as_float(xcc_id()), 1u);
  }
  __syncthreads();
  if (tid < nw) {
    const long long t0 = wall_clock64();
    unsigned long long w;
    while (true) {
      w = tag_load(hello + tid);
      if (tag_of(w) == 1u) break;
      if (wall_clock64() - t0 > spin) {
        raise_abort(abort_flag, err);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (__float_as_uint(val_of(w)) != xcc_id()) differs = 1;
  }
  __syncthreads();
  return differs == 0;
}

// v_mfma_f32_4x4x1_16b_f32 with the A operand of block `kk` (lanes 4kk..4kk+3)
// broadcast to all 16 blocks.  kk is a compile-time constant at every call site after
// unrolling, so the switch folds to one instruction.
__device__ __forceinline__ f4 mfma4_bcast(float a, float b, f4 c, int kk) {
  switch (kk) {
    case 0: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 0, 0);
    case 1: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 1, 0);
    case 2: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 2, 0);
    case 3: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 3, 0);
    case 4: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 4, 0);
    case 5: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 5, 0);
    case 6: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 6, 0);
    case 7: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 7, 0);
    case 8: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 8, 0);
    case 9: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 9, 0);
    case 10: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 10, 0);
    case 11: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 11, 0);
    case 12: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 12, 0);
    case 13: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 13, 0);
    case 14: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 14, 0);
    default: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 15, 0);
  }
}

struct PFwdArgs {
  const float* gih;
  const float* w_hh;
  const float* b_hh;
  const float* a;
  const float* h0;
  const float* c0;
  float* h_save;
  float* c_save;
  float* gact;
  float* tanh_c;
  float* xbuf;                // [4 slots][NG][4 quarters][64 lanes x KQ/16 words] h words
  unsigned long long* hello;  // [NG][NWMAX]
  int* err;
  int T, B, H, Hp, NG, NGX, Bg, NW;
  int device_scope;  // 1: never use the XCD-local stores
  long long spin;
  // input-projection waves (launches with 512 threads; gih is then unused)
  const float* x;     // [T][B][D]
  const float* w_ih;  // [4H][D]
  const float* b_ih;  // [4H]
  int D;
};

// Per-wave step flags between the recurrent waves and the extra waves of a persistent
// workgroup (forward: h published; backward: products issued).  Accessed through an
// explicit LDS (address space 3) volatile pointer, so that the accesses are LDS
// instructions: as generic volatile accesses they become flat ones, after which the
// compiler waits for every outstanding global access of the wave.
__shared__ int s_step_flag[4];
typedef __attribute__((address_space(3))) volatile int lds_vint;
__device__ __forceinline__ lds_vint* step_flags() { return (lds_vint*)(s_step_flag); }

// Input projection inside the forward: xin[block parity][w][WG row][t%8 * 4 + batch slot]
// holds projection wave w's partial sum (over the w-th quarter of D) of x_t[b] . W_ih[row]
// for the 8 steps of a block.  Rows are padded to 36 floats.
constexpr int kXinSteps = 8;
// true: the projection products of a step wait for the recurrent waves' publish (an LDS
// flag).  With the products on 16-bit instructions, starting them at the step's barrier
// is faster (configs[2] forward 430-436 -> 412-415 us).
constexpr bool kXprojAfterPublish = false;
#ifndef HSL_XPROJ_SPLIT
#define HSL_XPROJ_SPLIT 1
#endif
constexpr bool kXprojSplit = HSL_XPROJ_SPLIT;  // split bf16 projection products when enabled
typedef float XinBuf[2][4][64][kXinSteps * 4 + 4];
// With the projection waves present, recurrent wave q's cell lanes do not store the
// step's saved activations themselves: they leave them in LDS and projection wave q
// stores them a step later, so that the recurrent wave's single completion counter
// covers only its hand-off stores and loads.  [step parity][wave][unit][h, c, tanh c, -,
// i, f, g, o]; it follows xin in the padding LDS.
typedef float SaveBuf[2][4][kUnits][8];
__device__ __forceinline__ SaveBuf* save_buf(XinBuf* xin) {
  return reinterpret_cast<SaveBuf*>(reinterpret_cast<char*>(xin) + sizeof(XinBuf));
}
// The recurrent waves' staging blocks for loading the W_hh slice (used before the first
// step only), after xin and the saves; the forward's dynamic LDS holds all three.
constexpr size_t kFwdWStageBytes = 4 * 64 * (64 + 4) * sizeof(float);
constexpr size_t kFwdLdsBytes = sizeof(XinBuf) + sizeof(SaveBuf) + kFwdWStageBytes;
static_assert(kFwdLdsBytes >= (size_t)kPadLdsBytes && kFwdLdsBytes <= 150 * 1024, "one workgroup per CU, LDS left for the rest");
__device__ __forceinline__ float* fwd_wstage(XinBuf* xin) {
  return reinterpret_cast<float*>(reinterpret_cast<char*>(xin) + sizeof(XinBuf) + sizeof(SaveBuf));
}

// Projection wave w stores the activations of step ts that recurrent wave w staged
// (batch slot w, the workgroup's 16 units; lanes 0-15).
__device__ __forceinline__ void store_saves(const PFwdArgs& p, int grp, int wg, const SaveBuf* sv, int w,
                                            int ts) {
  const int lane = threadIdx.x & 63, cb = grp * p.Bg + w, cu = wg * kUnits + (lane & 15);
  if (lane >= kUnits || w >= p.Bg || cb >= p.B || cu >= p.H) return;
  const f4 hc = *reinterpret_cast<const f4*>(&(*sv)[ts & 1][w][lane][0]);
  const f4 g = *reinterpret_cast<const f4*>(&(*sv)[ts & 1][w][lane][4]);
  const size_t plane = (size_t)p.B * p.H, e = (size_t)cb * p.H + cu;
  __builtin_nontemporal_store(hc[0], p.h_save + (size_t)(ts + 1) * plane + e);
  __builtin_nontemporal_store(hc[1], p.c_save + (size_t)(ts + 1) * plane + e);
  __builtin_nontemporal_store(hc[2], p.tanh_c + (size_t)ts * plane + e);
  __builtin_nontemporal_store(g, reinterpret_cast<f4*>(p.gact + ((size_t)ts * plane + e) * 4));
}

// Forward.  Wave q multiplies the q-th quarter of k (KQ values).  h_{t-1} of a quarter
// comes from NS = KQ/16 source workgroups (16 units each).  Lane l of wave q needs
// h[batch slot l%4][unit q*KQ + 16j + l/4] for j < NS; these NS words form the lane's
// part of a 64-lane block (lane_word), so the receive is NS/2 8-byte loads per lane.
// The 16 MFMAs of source j then read their A operand straight from the received
// registers: with cbsz=4, abid=kk broadcasts lanes 4kk..4kk+3, i.e. h[0..3][unit kk],
// to all 16 blocks.  One workgroup barrier per step joins the four k-quarters; wave q
// then runs the cell for batch slot q (lanes 0-15 = units).
//
// Slots: h_t goes to slot t%4.  After its publish in step t, the owner of a word clears
// it in slot (t+2)%4 (h_{t-2}).  By then the four waves together have received h_{t-1}
// from every workgroup of the group, each of which published it after reading h_{t-2}
// (a single wave has heard only from the sources of its quarter, which is why the
// clear comes after the barrier).  The clear completes before the owner's next receive
// does, hence before it publishes h_{t+1}; a reader of h_{t+2} has seen h_{t+1} first,
// so it sees the clear or h_{t+2}, never h_{t-2}.
//
// One wave per SIMD leaves no other wave to hide latency behind, so the step is written
// for a short dependent chain: uniform bases with 32-bit lane offsets for every access,
// the hand-off scope fixed at compile time (FAST: XCD-local), and 4 accumulator chains.
template <int KQ, bool FAST, bool XP>
__device__ __forceinline__ void rec_fwd_body(const PFwdArgs& p, int grp, int wg, f4 (&red)[2][4][64],
                                             XinBuf* xin, int& abort_flag) {
  constexpr int HP = 4 * KQ;
  constexpr int NS = KQ / kUnits;
  constexpr int GW = 4 * HP;  // words per group and slot
  const int T = p.T, B = p.B, H = p.H, NG = p.NG, Bg = p.Bg;
  const int lane = threadIdx.x & 63;
  const int q = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  // a-scaled W_hh slice: lane = gate row (gate lane/16, unit lane%16), registers = k quarter
  const int rgate = lane >> 4, ru = wg * kUnits + (lane & 15);
  const bool row_ok = ru < H;
  float wreg[KQ];
  {
    const float ag = p.a[rgate];
    const float* wrow = p.w_hh + (size_t)(row_ok ? rgate * H + ru : 0) * H;
    if (H % 4 == 0 && reinterpret_cast<uintptr_t>(p.w_hh) % 16 == 0) {
      // A lane holds KQ consecutive k of its own row, so loading its registers directly
      // touches 64 rows per instruction.  Instead the wave loads whole row segments (LPR
      // lanes x 16 bytes per row, RPI rows per instruction) into its own LDS staging
      // block and each lane reads its row back: an eighth of the cache-line requests.
      // At configs[2] the slice is in registers 9.3-9.7 us after launch instead of 11.2
      // (the rest is the 32 MiB that the eight XCDs' copies of W_hh read).
      constexpr int KC = KQ < 64 ? KQ : 64;  // k per staging pass
      constexpr int LPR = KC / 4, RPI = 64 / LPR, PITCH = KC + 4;
      float* const stg = fwd_wstage(xin) + q * 64 * PITCH;
      static_assert(4 * 64 * PITCH * sizeof(float) <= kFwdWStageBytes, "staging fits");
#pragma unroll
      for (int r0 = 0; r0 < KQ; r0 += KC) {
        f4 v[64 / RPI];
#pragma unroll
        for (int i = 0; i < 64 / RPI; ++i) {
          const int sr = RPI * i + lane / LPR;  // staged row = the lane that owns it
          const int su = wg * kUnits + (sr & 15);
          const int k = q * KQ + r0 + 4 * (lane % LPR);  // a multiple of 4: k < H implies k + 3 < H
          const float* const src = p.w_hh + (size_t)(su < H ? (sr >> 4) * H + su : 0) * H;
          v[i] = *reinterpret_cast<const f4*>(src + (k < H ? k : H - 4));
        }
#pragma unroll
        for (int i = 0; i < 64 / RPI; ++i)
          *reinterpret_cast<f4*>(stg + (RPI * i + lane / LPR) * PITCH + 4 * (lane % LPR)) = v[i];
#pragma unroll
        for (int m = 0; m < KC / 4; ++m) {
          const f4 w4 = *reinterpret_cast<const f4*>(stg + lane * PITCH + 4 * m);
          const int k = q * KQ + r0 + 4 * m;
#pragma unroll
          for (int e = 0; e < 4; ++e) wreg[r0 + 4 * m + e] = (row_ok && k < H) ? ag * w4[e] : 0.f;
        }
      }
    } else {
#pragma unroll
      for (int kk = 0; kk < KQ; ++kk) {
        const int k = q * KQ + kk;
        const float v = wrow[k < H ? k : H - 1];
        wreg[kk] = (row_ok && k < H) ? ag * v : 0.f;
      }
    }
  }

  // cell lanes: wave q, lane < 16 -> (batch slot q, unit cu); cb is wave-uniform.  The
  // gate pre-activations are formed and activated one gate per lane (gate lane/16, unit
  // lane%16) by all 64 lanes, and lanes 0-15 gather their unit's other three gates.
  const int cb = grp * Bg + q;
  const unsigned cu = wg * kUnits + (lane & 15);
  const int lgate = lane >> 4;
  const bool u_ok = q < Bg && cb < B && (int)cu < H;
  const bool c_ok = lane < kUnits && u_ok;
  const int cbc = cb < B ? cb : 0;  // clamped for the uniform bases below
  const unsigned cuc = (int)cu < H ? cu : H - 1;
  float bl = 0.f;  // the lane's gate bias: a_g b_hh (+ b_ih when the projection is fused)
  float c_reg = 0.f;
  if (u_ok) {
    bl = p.a[lgate] * p.b_hh[lgate * H + cu];
    if constexpr (XP) bl = p.b_ih[lgate * H + cu] + bl;  // the projection's bias joins here
  }
  if (c_ok) {
    const size_t b0 = (size_t)cb * H + cu;
    c_reg = p.c0 ? p.c0[b0] : 0.f;
    p.h_save[b0] = p.h0 ? p.h0[b0] : 0.f;
    p.c_save[b0] = c_reg;
  }

  // receive: word j of lane l, wave q at block xbuf[slot][grp][q], lane_word(l, j)
  const int wi = lane & 3, wkk = lane >> 2, wb = grp * Bg + wi;
  bool wv[NS];
#pragma unroll
  for (int j = 0; j < NS; ++j) wv[j] = wi < Bg && wb < B && (q * NS + j) * kUnits + wkk < H;
  const size_t slot_words = (size_t)NG * GW;
  float* const xg = p.xbuf + (size_t)grp * GW;
  const unsigned roff = q * 64 * NS + lane_word<NS>(lane, 0);
  // publish: the word of (batch slot q, unit cu) is read by lane 4*(cu%16) + q of wave
  // cu/KQ, as its word (cu%KQ)/16
  const unsigned woff = (cu / KQ) * 64 * NS + lane_word<NS>(4 * (cu & 15) + q, (cu % KQ) / kUnits);
  const size_t plane = (size_t)B * H, plane4 = 4 * plane;
  // per-step rows of the streamed arrays: uniform base + cu (+ g*H)
  const float* gih_row = p.gih + (size_t)cbc * 4 * H;
  float* hs_row = p.h_save + (size_t)cbc * H;
  float* cs_row = p.c_save + (size_t)cbc * H;
  float* tc_row = p.tanh_c + (size_t)cbc * H;
  float* ga_row = p.gact + (size_t)cbc * H * 4;  // [T][B][H][4]

  // Memory traffic of a step is placed so that no wait for it lands between the
  // receive and the publish: the input-projection row of step t+1 is requested right
  // after step t's receive (two register sets alternate, so no copy waits for it) and
  // is forced into registers right after step t+1's receive, by when it has long arrived
  // (forcing it earlier would also wait for the stores of step t, before the first
  // poll); the saved activations (staged in LDS for the projection waves when they are
  // present) and the slot clear are stored after the publish.  All of these stores have
  // completed once the next receive has (one in-order completion counter).
  // The streamed activations use non-temporal accesses so that they do not push the
  // hand-off slots out of L2.
  // (the lane's gate of) the input projection of a step; clamped address, so that the
  // load needs no condition
  const unsigned goff = 4u * (lgate * H + cuc);
  float giA = 0.f, giB = 0.f;
  if constexpr (!XP) giA = *byte_at(gih_row, goff);

  // One step; gi holds this step's projection value, gn receives the next one.  Returns
  // false when the group aborted.
  auto step = [&](int t, float& gi, float& gn) __attribute__((always_inline)) -> bool {
    // XP: projection wave q's partials of this step (lane = gate row, element = batch
    // slot) seed the accumulator of wave q, so the workgroup sum below includes x_t W_ih^T
    f4 xp = f4{0.f, 0.f, 0.f, 0.f};
    if constexpr (XP)
      xp = *reinterpret_cast<const f4*>(&(*xin)[(t / kXinSteps) & 1][q][lane][(t % kXinSteps) * 4]);
    float hv[NS];
    if (t == 0) {
#pragma unroll
      for (int j = 0; j < NS; ++j) {
        const int k = (q * NS + j) * kUnits + wkk;
        hv[j] = (wv[j] && p.h0) ? p.h0[(size_t)wb * H + k] : 0.f;
        asm volatile("" : "+v"(hv[j]));  // wait here, not after the loads below
      }
    } else {
      unsigned v[NS];
      words_wait<NS>(xg + (size_t)((t - 1) & 3) * slot_words, roff, wv, v, p.spin, &abort_flag, p.err);
      if constexpr (!FAST) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
#pragma unroll
      for (int j = 0; j < NS; ++j) {
        hv[j] = wv[j] ? __uint_as_float(v[j]) : 0.f;
        asm volatile("" : "+v"(hv[j]));  // settled before the loads below are issued
      }
    }
    asm volatile("" : "+v"(gi));
    if (!XP && t + 1 < T) gn = __builtin_nontemporal_load(byte_at(gih_row + (size_t)(t + 1) * plane4, goff));
    f4 acc[4];
    acc[0] = xp;
#pragma unroll
    for (int c = 1; c < 4; ++c) acc[c] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NS; ++j)
#pragma unroll
      for (int kk = 0; kk < kUnits; ++kk)
        acc[kk & 3] = mfma4_bcast(hv[j], wreg[j * kUnits + kk], acc[kk & 3], kk);
    const f4 zs = (acc[0] + acc[1]) + (acc[2] + acc[3]);
#pragma unroll
    for (int i = 0; i < 4; ++i) reinterpret_cast<float*>(&red[t & 1][i][lane])[q] = zs[i];
    lds_barrier();
    if (abort_flag) return false;

    // every lane: its gate of its unit (the four k-quarter sums of the row), then lanes
    // 0-15 take f, g and o of their unit from lanes +16, +32 and +48 (gfx950 row and half
    // swaps; the second result of a swap holds lane l+16 or l+32 in rows 0 and 2)
    float act[4];
    {
      const f4 pr = red[t & 1][q][lane];
      const float mm = (pr[0] + pr[1]) + (pr[2] + pr[3]);
      act[0] = sigmoid_f((XP ? mm : gi + mm) + bl);
      const auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(act[0]), __float_as_uint(act[0]), false, false);
      const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(act[0]), __float_as_uint(act[0]), false, false);
      const auto s48 = __builtin_amdgcn_permlane32_swap(s16[1], s16[1], false, false);
      act[1] = __uint_as_float(s16[1]);
      act[2] = __uint_as_float(s32[1]);
      act[3] = __uint_as_float(s48[1]);
    }
    if (c_ok) {
      const float c = act[1] * c_reg + act[0] * act[2];
      const float tc = tanh_f(c);
      const float h = act[3] * tc;
      c_reg = c;
      if constexpr (!FAST) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
      word_put<FAST>(xg + (size_t)(t & 3) * slot_words, woff, canon_nan(h));
      if constexpr (XP) {  // projection wave q stores them (store_saves)
        float* const sv = &(*save_buf(xin))[t & 1][q][lane & 15][0];
        *reinterpret_cast<f4*>(sv) = f4{h, c, tc, 0.f};
        *reinterpret_cast<f4*>(sv + 4) = f4{act[0], act[1], act[2], act[3]};
      } else {
        __builtin_nontemporal_store(h, byte_at(hs_row + (size_t)(t + 1) * plane, 4u * cu));
        __builtin_nontemporal_store(c, byte_at(cs_row + (size_t)(t + 1) * plane, 4u * cu));
        __builtin_nontemporal_store(tc, byte_at(tc_row + (size_t)t * plane, 4u * cu));
        __builtin_nontemporal_store(f4{act[0], act[1], act[2], act[3]},
                                    reinterpret_cast<f4*>(byte_at(ga_row + (size_t)t * plane4, 16u * cu)));
      }
      word_put<FAST>(xg + (size_t)((t + 2) & 3) * slot_words, woff, __uint_as_float(kEmpty));
    }
    if constexpr (XP && kXprojAfterPublish) {  // the projection waves' products may start now
      __builtin_amdgcn_sched_barrier(0);
      step_flags()[q] = t + 1;  // every lane writes the same value
      __builtin_amdgcn_sched_barrier(0);
    }
    return true;
  };

  if constexpr (XP) lds_barrier();  // block 0 of xin is written
  for (int t = 0; t < T; t += 2) {
    if (!step(t, giA, giB)) return;
    if (t + 1 < T && !step(t + 1, giB, giA)) return;
  }
}

// Input-projection waves (waves 4-7 of a 512-thread forward workgroup): they compute
// x_t W_ih^T for this workgroup's 64 gate rows and the group's four batch slots
// (_torch.py:96, there one GEMM before the loop) while the recurrent waves run, so the
// [T,B,4H] projection never goes through HBM.  Wave w takes the quarter k in
// [64w, 64w+64) of D (D <= 256); the 8 steps of a block form the 32 columns of one
// v_mfma_f32_32x32x2_f32 tile (column = t%8 * 4 + batch slot), rows = the 64 gate rows
// (two tiles), W_ih's rows held in registers for the whole launch.  The two half-waves
// take the two 32-wide halves of the quarter (A and B use the same k order).  Block m+1
// is computed during the first 6 steps of block m (the 64 products spread over them) and
// written to xin in step 8m+6, before the barrier of step 8m+7 (parity m+1; recurrent wave w reads its
// plane at the start of each step of block m+1, before that step's barrier, and the
// last reads of block m-1, which the write replaces, came before the barrier of step
// 8m-1).  Its x operands are loaded two blocks ahead.  Block 0 is computed and written
// before one extra barrier ahead of the first step.  The waves take part in every
// workgroup barrier of the recurrent waves and leave when the group aborts, as they do.
template <int KQ, bool XS>
__device__ __forceinline__ void rec_fwd_xproj(const PFwdArgs& p, int grp, int wg, XinBuf* xin, int& abort_flag) {
  const int T = p.T, B = p.B, H = p.H, D = p.D, Bg = p.Bg;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane((threadIdx.x >> 6) - 4);
  const int half = lane >> 5, l32 = lane & 31;
  const int kb = 64 * w + 32 * half;
  float wa[2][32];
  const bool wvec = reinterpret_cast<uintptr_t>(p.w_ih) % 16 == 0;  // D % 4 == 0 here
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const int r = rt * 32 + l32, u = wg * kUnits + (r & 15);
    const bool ok = u < H;
    const float* wrow = p.w_ih + (size_t)((r >> 4) * H + (ok ? u : 0)) * D;
    if (wvec) {  // 16-byte loads at clamped addresses (k is a multiple of 4)
#pragma unroll
      for (int i4 = 0; i4 < 8; ++i4) {
        const int k = kb + 4 * i4;
        const f4 v = *reinterpret_cast<const f4*>(wrow + (k < D ? k : D - 4));
#pragma unroll
        for (int e = 0; e < 4; ++e) wa[rt][4 * i4 + e] = (ok && k < D) ? v[e] : 0.f;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        const int k = kb + i;
        wa[rt][i] = (ok && k < D) ? wrow[k] : 0.f;
      }
    }
  }
  // XS: W_ih's rows as their three bf16 pieces for the four 16-deep k-steps (the fp32
  // rows are not kept)
  u32x4 wp[XS ? 2 : 1][XS ? 4 : 1][3];
  if constexpr (XS) {
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int i = 0; i < 4; ++i) split8(&wa[rt][8 * i], wp[rt][i]);
    __builtin_amdgcn_sched_barrier(0);  // the fp32 rows die before the x rows arrive
  }
  // column l32 = t%8 * 4 + batch slot; absent slots read batch 0 (their column is unused)
  const int bsl = l32 & 3, tl = l32 >> 2, cb = grp * Bg + bsl;
  const int cbr = (bsl < Bg && cb < B) ? cb : 0;
  // Loads are unconditional at clamped addresses (columns past D read the row's last
  // four values, finite, and meet zero W_ih registers): a conditional load would need a
  // select on its result, and the compiler would then wait for the HBM load right here,
  // two blocks before the values are used (1800 clocks at every block boundary).
  auto load_blk = [&](int m, float (&xo)[32]) {
    const int t = m * kXinSteps + tl;
    const float* row = p.x + ((size_t)(t < T ? t : T - 1) * B + cbr) * D;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int k4 = min(kb + 4 * j, D - 4);
      const f4 v = *reinterpret_cast<const f4*>(row + k4);
#pragma unroll
      for (int e = 0; e < 4; ++e) xo[4 * j + e] = v[e];
    }
  };
  f16v acc[2] = {f16v{}, f16v{}};
  // part `sub` of `of` parts of a block's products
  auto products = [&](const float (&xo)[32], int sub, int of) {
    if constexpr (XS) {
      // 16-deep k-steps on the exact bf16 split (split_bf16.h): k-step i multiplies the
      // lane's values 8i .. 8i+7 (A: W_ih row l%32, B: column l%32 of x; lanes 0-31 hold k
      // kb0 + 8i .., lanes 32-63 kb0 + 32 + 8i ..), six piece products each.  16-bit
      // products leave the recurrent wave on the same SIMD its issue slots, where the
      // fp32 instruction holds them off.
#pragma unroll
      for (int i = 4 * sub / of; i < 4 * (sub + 1) / of; ++i) {
        float xv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          xv[e] = xo[8 * i + e];
          asm volatile("" : "+v"(xv[e]));  // split here, next to the products
        }
        u32x4 pb[3];
        split8(xv, pb);
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
          for (int pp = 0; pp < 6; ++pp) acc[rt] = mfma_bf16(wp[rt][i][kPa[pp]], pb[kPb[pp]], acc[rt]);
      }
    } else {
#pragma unroll
      for (int i = 32 * sub / of; i < 32 * (sub + 1) / of; ++i)
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
          acc[rt] = __builtin_amdgcn_mfma_f32_32x32x2f32(wa[rt][i], xo[i], acc[rt], 0, 0, 0);
    }
  };
  auto write_blk = [&](int m) {  // D layout: lane l, register r -> row 8(r/4) + 4(l/32) + r%4, column l%32
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = rt * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
        (*xin)[m & 1][w][row][l32] = acc[rt][r];
      }
      acc[rt] = f16v{};
    }
  };

  // x operands of even / odd blocks, loaded two blocks ahead; XS: one set, loaded one
  // block ahead (its products start in the second step of a block, three steps after the
  // load, and the registers go to W_ih's pieces)
  constexpr int LA = XS ? 2 : 3;
  float xa[32], xb[XS ? 1 : 32];
  load_blk(0, xa);
  if constexpr (!XS) load_blk(1, xb);
  products(xa, 0, 1);
  write_blk(0);
  if constexpr (XS)
    load_blk(1, xa);
  else
    load_blk(2, xa);
  lds_barrier();  // the recurrent waves' barrier ahead of their first step
  // window j: the 8 steps of block j, computing block j+1 from its operand set in steps
  // 0-5 (k-steps 32 sub / 6 .. 32 (sub+1) / 6 in step sub) and writing it in step 6, when
  // those products have long finished (writing right after the last products made the
  // barrier of step 8m+7 wait for them)
  auto window = [&](int j, float (&xu)[32]) __attribute__((always_inline)) -> bool {
    const bool next = (j + 1) * kXinSteps < T;
#pragma unroll
    for (int sub = 0; sub < 8; ++sub) {
      const int t = j * kXinSteps + sub;
      if (t >= T) return false;
      lds_barrier();  // the recurrent waves' barrier of this step
      if (abort_flag) return false;
      if (t > 0) store_saves(p, grp, wg, save_buf(xin), w, t - 1);  // staged before this barrier
      if (next && sub == 6) {  // block j+1, whose products ended a step ago, to xin
        write_blk(j + 1);
        load_blk(j + LA, xu);
      } else if (next && sub < 6) {
        if constexpr (kXprojAfterPublish) {  // after the recurrent waves' publish of h_t
          const long long t0 = wall_clock64();
          while (true) {
            lds_vint* const f = step_flags();
            const int m0 = f[0], m1 = f[1], m2 = f[2], m3 = f[3];
            if (min(min(m0, m1), min(m2, m3)) > t) break;
            if (abort_flag) return false;
            if (wall_clock64() - t0 > p.spin) {
              raise_abort(&abort_flag, p.err);
              return false;
            }
            __builtin_amdgcn_s_sleep(1);
          }
        }
        products(xu, sub, 6);
      }
    }
    return true;
  };
  if constexpr (XS) {
    for (int j = 0;; ++j)
      if (!window(j, xa)) break;
  } else {
    for (int j = 0;; j += 2) {
      if (!window(j, xb)) break;
      if (!window(j + 1, xa)) break;
    }
  }
}

// After an abort every output the workgroup owns is NaN: the h_save/c_save rows 0..T and
// the gact/tanh_c rows of its units for the batch slot of the calling recurrent wave (the
// elements that wave's cell lanes write), so a loss or gradient computed from a call that
// gave up is NaN instead of silently wrong.
__device__ void poison_fwd(const PFwdArgs& p, int grp, int wg) {
  const int lane = threadIdx.x & 63, q = threadIdx.x >> 6;
  const int cb = grp * p.Bg + q, cu = wg * kUnits + (lane & 15);
  if (lane >= kUnits || q >= p.Bg || cb >= p.B || cu >= p.H) return;
  const float nan = __uint_as_float(0x7FC00000u);
  const size_t plane = (size_t)p.B * p.H, e = (size_t)cb * p.H + cu;
  for (int t = 0; t <= p.T; ++t) {
    p.h_save[t * plane + e] = nan;
    p.c_save[t * plane + e] = nan;
    if (t < p.T) {
      p.tanh_c[t * plane + e] = nan;
      *reinterpret_cast<f4*>(p.gact + (t * plane + e) * 4) = f4{nan, nan, nan, nan};
    }
  }
}

// XP: 512 threads; waves 4-7 compute the input projection (rec_fwd_xproj), which then
// is not read from gih, and store the saved activations.  Every wave ends with one more workgroup barrier: a wave that
// gave up a wait has set abort_flag before it (waves that left early have terminated
// and are not waited for), so all waves agree on whether to poison their outputs.
// XP: 0 = no projection waves, 1 = projection products on the fp32 instruction, 2 = on
// split bf16 pieces (hsl_set_split_products).
template <int KQ, int XP>
__global__ __launch_bounds__(XP ? 512 : 256, 1) void rec_fwd_persistent(PFwdArgs p) {
  constexpr int HP = 4 * KQ;
  __shared__ f4 red[2][4][64];  // [step parity][batch slot][gate row] -> 4 wave partials
  __shared__ int abort_flag;
  extern __shared__ char dyn_lds[];  // keeps one workgroup per CU; xin (XP), the saves, the W_hh staging
  XinBuf* const xin = reinterpret_cast<XinBuf*>(dyn_lds);
  const int grp = blockIdx.x % p.NGX, wg = blockIdx.x / p.NGX;
  if (grp >= p.NG) return;  // unused XCD slot (groups are padded to a multiple of 8)
  if (threadIdx.x == 0) abort_flag = 0;
  if (threadIdx.x < 4) step_flags()[threadIdx.x] = 0;  // steps whose h wave q has published
  const bool fast = agree_placement(p.hello + (size_t)grp * (HP / kUnits), wg, p.NW, p.spin, &abort_flag, p.err) &&
                    !p.device_scope;
  if (!abort_flag) {
    bool proj = false;
    if constexpr (XP) {
      if (threadIdx.x >= 256) {
        rec_fwd_xproj<KQ, XP == 2>(p, grp, wg, xin, abort_flag);
        proj = true;
      }
    }
    if (!proj) {
      if (fast)
        rec_fwd_body<KQ, true, (XP > 0)>(p, grp, wg, red, xin, abort_flag);
      else
        rec_fwd_body<KQ, false, (XP > 0)>(p, grp, wg, red, xin, abort_flag);
    }
  }
  // The projection waves' save stores complete before the barrier (workgroup-scope
  // release), so that the poison stores after it are the last writes.  The last step's
  // activations, staged before it, are stored after it.
  if (XP && threadIdx.x >= 256) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  lds_barrier();
  if constexpr (XP) {
    if (threadIdx.x >= 256 && !abort_flag && p.T > 0)
      store_saves(p, grp, wg, save_buf(xin), (threadIdx.x >> 6) - 4, p.T - 1);
  }
  if (abort_flag && threadIdx.x < 256) {
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    poison_fwd(p, grp, wg);
  }
}

// Per-step inputs of the persistent backward, loaded one step ahead: dout[t], c_{t-1}
// and the four gate activations of one (batch, unit).
struct StepIn {
  float dout, cp;
  f4 g;
};

struct PBwdArgs {
  const float* dout;
  const float* dh_n;
  const float* dc_n;
  const float* c_save;
  const float* gact;
  const float* tanh_c;
  const float* w_hh;
  const float* a;
  float* dgates;
  double* db_part;  // [B][4H]
  float* dh0;
  float* dc0;
  float* pbuf;                // [3 slots][NG][NWMAX readers][4 batch slots][64 lanes x PER words] partials
  unsigned long long* hello;  // [NG][NWMAX]
  int* err;
  int T, B, H, Hp, NG, NGX, Bg, NW;
  int device_scope;
  long long spin;
  // weight-gradient waves (launches with 512 threads): fp32 partial sums of
  // dW_hh_s = dg^T h_prev and dW_ih = dg^T x, one plane per (chunk of TS steps, group)
  const float* h_save;  // [T+1][B][H]
  const float* x;       // [T][B][D]
  float* wph;           // [chunks*NG][4H][H] fp32
  float* wpx;           // [NG][4H][D] (when dW_ih is fused): each group's fp64 sums rounded once
  int D, TS;
  int store_dg;  // 0: dgates are not needed after the kernel (not written)
};

// Backward.  Wave q owns batch slot q for the dh receive and the cell, and the q-th
// quarter of the columns for the partial product.  A lane of wave q gathers the
// partials of sources m, m+4, m+8, ... (m = lane/16) for unit lane%16, adds them in
// that order, and two cross-lane shuffles finish the fixed-order sum, so the
// receive needs no LDS and no barrier.  A lane's PER partials form its part of a
// 64-lane block (lane_word).  One workgroup barrier per step publishes the step's
// dgates (double-buffered in LDS) to the four column quarters.
//
// Slots: the partials published in step s go to slot s%3 and have exactly one reader,
// which clears them right after its receive in step s+1.  They are written again in
// step s+3, by a writer that has by then received the reader's step-s+2 partials; the
// reader publishes those only after its step-s+2 receive, which waits for the clear.
//
// As in the forward, every access uses a uniform base plus a 32-bit lane offset and the
// hand-off scope is a compile-time choice, keeping the per-step dependent chain short.
template <int KQ, bool FAST, bool GW>
__device__ __forceinline__ void rec_bwd_body(const PBwdArgs& p, int grp, int wg, float (&dgl)[2][4][68],
                                             int& abort_flag) {
  constexpr int HP = 4 * KQ;
  constexpr int CG = (KQ + 63) / 64;     // 64-column groups per wave
  constexpr int NWMAX = HP / kUnits;     // workgroups per group at most
  constexpr int PER = (NWMAX + 3) / 4;   // partials gathered per lane
  constexpr int RW = 4 * 64 * PER;       // words per reader workgroup and slot
  const int T = p.T, B = p.B, H = p.H, NG = p.NG, Bg = p.Bg, NW = p.NW;
  const int lane = threadIdx.x & 63;
  const int q = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  // W_s columns owned by this lane: col = q*KQ + cg*64 + lane; registers over the 64 rows.
  float wreg[CG][64];
  int col[CG];
  bool col_ok[CG];
  float av[4];
#pragma unroll
  for (int gt = 0; gt < 4; ++gt) av[gt] = p.a[gt];
#pragma unroll
  for (int cg = 0; cg < CG; ++cg) {
    const int cl = cg * 64 + lane;
    col[cg] = q * KQ + cl;
    col_ok[cg] = cl < KQ && col[cg] < H;
    const int cc = col_ok[cg] ? col[cg] : 0;  // clamped: every load is issued unconditionally
#pragma unroll
    for (int r = 0; r < 64; ++r) {
      const int u = wg * kUnits + (r & 15);
      wreg[cg][r] = p.w_hh[(size_t)((r >> 4) * H + (u < H ? u : H - 1)) * H + cc];
    }
#pragma unroll
    for (int r = 0; r < 64; ++r) {
      const int gt = r >> 4, u = wg * kUnits + (r & 15);
      asm volatile("" : "+v"(wreg[cg][r]));  // keeps the loads above out of the conditional
      wreg[cg][r] = (col_ok[cg] && u < H) ? av[gt] * wreg[cg][r] : 0.f;
    }
  }

  // cell thread: wave q, lane < 16 -> (batch slot q, unit cu); cb is wave-uniform
  const int uu = lane & 15, cb = grp * Bg + q;
  const unsigned cu = wg * kUnits + uu;
  const bool c_ok = lane < kUnits && q < Bg && cb < B && (int)cu < H;
  const int cbc = cb < B ? cb : 0;
  float dc = 0.f;
  double dbacc[4] = {0.0, 0.0, 0.0, 0.0};
  if (c_ok && p.dc_n) dc = p.dc_n[(size_t)cb * H + cu];

  // receive words: partial j of lane l (source l/16 + 4j, batch slot q, column cu) at
  // block pbuf[slot][grp][wg][q], lane_word(l, j)
  const int m = lane >> 4;
  const bool r_ok = q < Bg && cb < B && (int)cu < H;
  bool wv[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) wv[j] = r_ok && m + 4 * j < NW;
  const size_t slot_words = (size_t)NG * NWMAX * RW;
  float* const pg = p.pbuf + (size_t)grp * NWMAX * RW;
  const unsigned roff = wg * RW + q * 64 * PER + lane_word<PER>(lane, 0);
  // publish: the partial of column c for batch slot i goes to reader workgroup c/16,
  // wave i, lane 16*(wg%4) + c%16, word wg/4
  const unsigned poff0 = lane_word<PER>(16 * (wg & 3), wg >> 2);
  const size_t plane = (size_t)B * H, plane4 = 4 * plane;
  const bool full_group = Bg == 4 && grp * 4 + 3 < B;  // all four batch slots in use
  const float* dout_row = p.dout + (size_t)cbc * H;
  const float* cs_row = p.c_save + (size_t)cbc * H;
  const float* tc_row = p.tanh_c + (size_t)cbc * H;
  const float* ga_row = p.gact + (size_t)cbc * H * 4;  // [T][B][H][4]
  float* dg_row = p.dgates + (size_t)cbc * 4 * H;

  // Memory traffic of a step is placed so that no wait for it lands between the
  // receive and the publish: the saved activations of step t-1 are requested right
  // after step t's receive (two register sets alternate, so no copy waits for them)
  // and forced into registers right after the next step's receive, by when they have
  // long arrived; dgates and the slot clear are stored after the cell.  All of them have
  // completed once the next receive has (one in-order completion counter).  The
  // streamed activations use non-temporal accesses so that they do not push the
  // hand-off slots out of L2.
  // tanh(c_t) is not loaded: c_t is the previous (later-in-time) step's c_{t-1}, and
  // tanh_f of it equals the forward's saved value bit for bit (same function, same
  // input).
  auto load_step = [&](int ts, StepIn& nx) {
    nx.dout = __builtin_nontemporal_load(byte_at(dout_row + (size_t)ts * plane, 4u * cu));
    nx.cp = __builtin_nontemporal_load(byte_at(cs_row + (size_t)ts * plane, 4u * cu));
    nx.g = __builtin_nontemporal_load(reinterpret_cast<const f4*>(byte_at(ga_row + (size_t)ts * plane4, 16u * cu)));
  };
  StepIn nxA{0.f, 0.f, f4{0.f, 0.f, 0.f, 0.f}}, nxB{0.f, 0.f, f4{0.f, 0.f, 0.f, 0.f}};
  float tc_next = 0.f;  // tanh(c_t) of the next step to run
  if (c_ok && T > 0) {
    load_step(T - 1, nxA);
    tc_next = __builtin_nontemporal_load(byte_at(tc_row + (size_t)(T - 1) * plane, 4u * cu));
  }

  // Step s (time t = T-1-s) with its activations in cur; the next step's go to nxt.
  // Returns false when done (s == T) or when the group aborted.
  auto step = [&](int s, StepIn& cur, StepIn& nxt) __attribute__((always_inline)) -> bool {
    const int t = T - 1 - s;

    // ---- dh: dh_n, or the fixed-order sum of last step's partials ------------------
    float dh = 0.f;
    const float* src = nullptr;
    if (s == 0) {
      if (c_ok && p.dh_n) dh = p.dh_n[(size_t)cb * H + cu];
      asm volatile("" : "+v"(dh));
    } else {
      src = pg + (size_t)((s - 1) % 3) * slot_words;
      unsigned v[PER];
      words_wait<PER>(src, roff, wv, v, p.spin, &abort_flag, p.err);
      if constexpr (!FAST) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      float part = 0.f;
#pragma unroll
      for (int j = 0; j < PER; ++j) part += wv[j] ? __uint_as_float(v[j]) : 0.f;
      part = add_xor16(part);
      part = add_xor32(part);
      dh = part;
      asm volatile("" : "+v"(dh));  // settled before the loads below are issued
    }
    if (s == T) {  // dh is now the gradient w.r.t. h0
      if (c_ok) {
        const size_t bu = (size_t)cb * H + cu;
        if (p.dh0) p.dh0[bu] = dh;
        if (p.dc0) p.dc0[bu] = dc;
#pragma unroll
        for (int gt = 0; gt < 4; ++gt) p.db_part[(size_t)cb * 4 * H + gt * H + cu] = dbacc[gt];
      }
      return false;
    }
    asm volatile("" : "+v"(cur.dout), "+v"(cur.cp), "+v"(cur.g), "+v"(tc_next));
    if (c_ok && s + 1 < T) load_step(t - 1, nxt);
    const float tc = tc_next;
    tc_next = tanh_f(cur.cp);

    // ---- cell backward (wave q: batch slot q) ----------------------------------------
    float d[4] = {0.f, 0.f, 0.f, 0.f};
    if (c_ok) {
      dh = dh + cur.dout;
      cell_bwd(dh, dc, cur.cp, cur.g[0], cur.g[1], cur.g[2], cur.g[3], tc, d);
#pragma unroll
      for (int gt = 0; gt < 4; ++gt) dbacc[gt] += (double)d[gt];
    }
    if (lane < kUnits) {
#pragma unroll
      for (int gt = 0; gt < 4; ++gt) dgl[s & 1][q][gt * kUnits + uu] = d[gt];
    }
    if (src) words_clear<PER, FAST>(const_cast<float*>(src), roff);
    if (c_ok && p.store_dg) {
      float* dgp = dg_row + (size_t)t * plane4;
#pragma unroll
      for (int gt = 0; gt < 4; ++gt) __builtin_nontemporal_store(d[gt], byte_at(dgp, 4u * (gt * H + cu)));
    }
    lds_barrier();
    if (abort_flag) return false;

    // ---- partial dh_{t-1}[batch][col] over this workgroup's 64 rows ------------------
    // lane l holds dgates of batch slot l%4 for rows 4(l/4)..4(l/4)+3; the MFMA for row
    // r = 4kk+c broadcasts register c of lanes 4kk..4kk+3 (abid = kk).
    const f4 dv = *reinterpret_cast<const f4*>(&dgl[s & 1][lane & 3][4 * (lane >> 2)]);
    if constexpr (!FAST) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    float* const dst_slot = pg + (size_t)(s % 3) * slot_words;
#pragma unroll
    for (int cg = 0; cg < CG; ++cg) {
      f4 acc[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[c] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 16; ++kk) {
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[c] = mfma4_bcast(dv[c], wreg[cg][4 * kk + c], acc[c], kk);
      }
      if (GW && cg == CG - 1) {
        // the matrix pipe is free from here until the next step's products: tell the
        // weight-gradient wave on this SIMD (every lane writes the same value)
        __builtin_amdgcn_sched_barrier(0);
        step_flags()[q] = s + 1;
        __builtin_amdgcn_sched_barrier(0);
      }
      const f4 part = (acc[0] + acc[1]) + (acc[2] + acc[3]);
      if (col_ok[cg]) {
        const unsigned c = col[cg];
        const unsigned off = (c >> 4) * RW + poff0 + (PER == 1 ? 1u : 2u) * (c & 15u);
        if (full_group) {
#pragma unroll
          for (int i = 0; i < 4; ++i) word_put<FAST>(dst_slot + i * 64 * PER, off, canon_nan(part[i]));
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (i < Bg && grp * Bg + i < B) word_put<FAST>(dst_slot + i * 64 * PER, off, canon_nan(part[i]));
        }
      }
    }
    return true;
  };

  for (int s = 0; s <= T; s += 2) {
    if (!step(s, nxA, nxB)) return;
    if (!step(s + 1, nxB, nxA)) return;
  }
}

// Weight-gradient waves (waves 4-7 of a 512-thread backward workgroup).  The recurrent
// waves leave the matrix pipes idle for most of a step (waiting for partials, running
// the cell), so a second wave per SIMD accumulates this workgroup's 64 rows of
//   dW_hh_s[n][k] += sum_b dg_t[b][n] h_{t-1}[b][k],   dW_ih[n][d] += sum_b dg_t[b][n] x_t[b][d]
// in registers while they wait.  Per step, the dgates of the four batch slots are read
// from the LDS copy the recurrent waves already make (dgl, valid between the step's
// barrier and the next), h_{t-1} and x_t rows are loaded one step ahead, and the
// batch is the reduction index of the products.  The products start only after the
// recurrent waves have issued theirs (s_step_flag), so they fill the idle part of the step.
//
// Accuracy: no fp32 running sum spans more than a few hundred products.  dW_hh_s is
// written as an fp32 partial plane every TS steps (its gradient dW_hh = a dW_hh_s is
// a-scaled); dW_ih goes into an fp64 accumulator in LDS (64 rows x D, written once per
// group as a plane, rounded to fp32 once): at the start of each step one of the wave's 4*XT
// accumulator sets (two 16x16 tiles) is added to it with ds_add_f64 (no returned value)
// and restarted, so an fp32 run covers 4*XT steps.  The planes are summed in fp64
// afterwards.
//
// The wave takes part in every workgroup barrier of the recurrent waves (one per step)
// and leaves when the group aborts, as they do.
constexpr int kXaccLdsBytes = 64 * 256 * 8;  // fp64 dW_ih accumulator for D <= 256

// The products are v_mfma_f32_16x16x4_f32, one instruction per 16x16 tile and step (k =
// the four batch slots): the matrix-core time of two 32x32x2 per 32x32 tile in
// half-length instructions.  A second wave streaming 32x32x2 f32 products holds off the
// recurrent wave on its SIMD about twice as long as one streaming 16x16x4 (a same-XCD
// hand-off measured 1.52 against 0.89 us beside them, 0.42 us alone).  Wave w owns the
// 32-column groups w, w+4, ... of h and of x, each two 16-column tiles, and the four
// 16-row tiles.  rec_bwd_wgrad_win below does the same sums on 16-bit products.
template <int KQ, int XT>
__device__ __forceinline__ void rec_bwd_wgrad(const PBwdArgs& p, int grp, int wg, float (&dgl)[2][4][68],
                                                double* xacc, int& abort_flag) {
  constexpr int HT = KQ >= 32 ? KQ / 32 : 1;  // h column groups of 32 per wave (4*KQ >= H)
  constexpr int XA = XT > 0 ? XT : 1;
  const int T = p.T, B = p.B, H = p.H, D = p.D, Bg = p.Bg, NG = p.NG, TS = p.TS;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane((threadIdx.x >> 6) - 4);
  const int kb = lane >> 4, l16 = lane & 15;  // k index of the products = batch slot kb
  const int cb = grp * Bg + kb;
  const bool bok = kb < Bg && cb < B;
  const int brow = bok ? cb : 0;
  const int nth = (H + 31) / 32, ntx = (D + 31) / 32;
  // operand column of group g, half sub: clamped in range (a column past H or D only feeds
  // an output column that is never written)
  auto hcol = [&](int g, int sub) { return min((w + 4 * g) * 32 + 16 * sub + l16, H - 1); };
  auto xcol = [&](int g, int sub) { return min((w + 4 * g) * 32 + 16 * sub + l16, D - 1); };
  f4 acch[HT][2][4], accx[XA][2][4];  // [column group][half][row tile]
  auto zero_h = [&]() {
#pragma unroll
    for (int g = 0; g < HT; ++g)
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) acch[g][sub][rt] = f4{0.f, 0.f, 0.f, 0.f};
  };
  auto zero_x = [&]() {
#pragma unroll
    for (int g = 0; g < XA; ++g)
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) accx[g][sub][rt] = f4{0.f, 0.f, 0.f, 0.f};
  };
  zero_h();
  zero_x();
  // D-layout of a 16x16 tile: lane l, register r -> row 4(l/16) + r, column l%16
  auto tile_row = [&](int rt, int r) { return rt * 16 + 4 * kb + r; };
  if constexpr (XT > 0) {
#pragma unroll
    for (int g = 0; g < XT; ++g) {
      if (w + 4 * g >= ntx) continue;
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int rt = 0; rt < 4; ++rt)
#pragma unroll
          for (int r = 0; r < 4; ++r) xacc[tile_row(rt, r) * 256 + (w + 4 * g) * 32 + 16 * sub + l16] = 0.0;
    }
  }

  // operand rows of step s (time t = T-1-s): h_{t-1} = h_save[t], x_t
  struct Ops {
    float h[HT][2];
    float x[XA][2];
  };
  auto load_ops = [&](int t, Ops& o) {
    const float* hr = p.h_save + ((size_t)t * B + brow) * H;
#pragma unroll
    for (int g = 0; g < HT; ++g)
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) o.h[g][sub] = hr[hcol(g, sub)];
    if constexpr (XT > 0) {
      const float* xr = p.x + ((size_t)t * B + brow) * D;
#pragma unroll
      for (int g = 0; g < XT; ++g)
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) o.x[g][sub] = xr[xcol(g, sub)];
    }
  };
  // Row r64 = rt*16 + 4*kb + r of a tile is gate rt, unit wg*16 + 4*kb + r.
  const int ulane = wg * kUnits + 4 * kb;
  auto dump_h = [&](int chunk) {
    float* const plane = p.wph + ((size_t)chunk * NG + grp) * 4 * H * H;
#pragma unroll
    for (int g = 0; g < HT; ++g) {
      if (w + 4 * g >= nth) continue;
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        const int c = (w + 4 * g) * 32 + 16 * sub + l16;
        const unsigned lo = 4u * ((unsigned)ulane * H + c);
#pragma unroll
        for (int rt = 0; rt < 4; ++rt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float* const rb = plane + (size_t)(rt * H + r) * H;
            if (ulane + r < H && c < H) *byte_at(rb, lo) = acch[g][sub][rt][r];
          }
      }
    }
    zero_h();
  };
  // adds accumulator tile sel = 2*(g*2 + sub) ... of every wave's x groups to the fp64
  // copy: selection f in [0, 4 XT) picks (g, sub, row-tile pair)
  auto fold_x = [&](int sel) {
#pragma unroll
    for (int g = 0; g < XT; ++g) {
      if (w + 4 * g >= ntx) continue;
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int rp = 0; rp < 2; ++rp) {
          if (sel >= 0 && sel != 4 * g + 2 * sub + rp) continue;
#pragma unroll
          for (int rt = 2 * rp; rt < 2 * rp + 2; ++rt) {
#pragma unroll
            for (int r = 0; r < 4; ++r)
              __hip_atomic_fetch_add(&xacc[tile_row(rt, r) * 256 + (w + 4 * g) * 32 + 16 * sub + l16],
                                     (double)accx[g][sub][rt][r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            accx[g][sub][rt] = f4{0.f, 0.f, 0.f, 0.f};
          }
        }
    }
  };

  auto step = [&](int s, Ops& cur) __attribute__((always_inline)) -> bool {
    lds_barrier();  // the recurrent waves' barrier of step s: dgl[s&1] is complete
    if (abort_flag) return false;
    float a[4];  // [row tile]
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) a[rt] = dgl[s & 1][kb][rt * 16 + l16];
    if (!bok) {  // operand rows of absent batch slots are zero (their dgates are zero too)
#pragma unroll
      for (int g = 0; g < HT; ++g) cur.h[g][0] = cur.h[g][1] = 0.f;
#pragma unroll
      for (int g = 0; g < XA; ++g) cur.x[g][0] = cur.x[g][1] = 0.f;
    }
    // one accumulator set goes to the fp64 copy while the recurrent waves still issue
    // their products (its last products were issued a step ago); an fp32 run covers 4 XT
    // steps
    if constexpr (XT > 0)
      if (s > 0) fold_x((s - 1) % (4 * XT));
    const long long t0 = wall_clock64();
    while (true) {
      lds_vint* const f = step_flags();
      const int m0 = f[0], m1 = f[1], m2 = f[2], m3 = f[3];
      if (min(min(m0, m1), min(m2, m3)) > s) break;
      if (abort_flag) return false;
      if (wall_clock64() - t0 > p.spin) {
        raise_abort(&abort_flag, p.err);
        return false;
      }
      __builtin_amdgcn_s_sleep(1);
    }
#pragma unroll
    for (int g = 0; g < HT; ++g) {
      if (w + 4 * g >= nth) continue;
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int rt = 0; rt < 4; ++rt)
          acch[g][sub][rt] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[rt], cur.h[g][sub], acch[g][sub][rt], 0, 0, 0);
    }
#pragma unroll
    for (int g = 0; g < XT; ++g) {
      if (w + 4 * g >= ntx) continue;
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int rt = 0; rt < 4; ++rt)
          accx[g][sub][rt] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[rt], cur.x[g][sub], accx[g][sub][rt], 0, 0, 0);
    }
    if (s + 1 < T) load_ops(T - 2 - s, cur);
    if (s % TS == TS - 1 || s == T - 1) dump_h(s / TS);
    return true;
  };

  Ops op;
  if (T > 0) load_ops(T - 1, op);
  for (int s = 0; s < T; ++s)
    if (!step(s, op)) return;

  if constexpr (XT > 0) {  // this group's dW_ih rows (fp64 sums, rounded once) as a plane
    fold_x(-1);
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");  // the wave's own LDS adds
    float* const plane = p.wpx + (size_t)grp * 4 * H * D;
#pragma unroll
    for (int g = 0; g < XT; ++g) {
      if (w + 4 * g >= ntx) continue;
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        const int c = (w + 4 * g) * 32 + 16 * sub + l16;
#pragma unroll
        for (int rt = 0; rt < 4; ++rt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int r64 = tile_row(rt, r), u = wg * kUnits + (r64 & 15);
            if (u < H && c < D) plane[((size_t)(r64 >> 4) * H + u) * D + c] = (float)xacc[r64 * 256 + c];
          }
      }
    }
  }
}

// Weight gradients on split bf16 products over windows of eight steps (the default;
// hsl_set_split_products(0) selects rec_bwd_wgrad).  v_mfma_f32_16x16x32_bf16 needs
// a 32-deep k, here the 8 steps x 4 batch slots of a window: lane l holds k = 8 (l/16) + i
// of its row (A) or column (B), i.e. batch slot l/16 and step i of the window, in both
// operands.
//  - A (dgates, 64 rows = four 16-row tiles): after the barrier of each step, wave w
//    splits row tile w of the step's dgates (the recurrent waves' LDS copy) into three
//    bf16 pieces and writes them into element i of the lanes' 16-byte operands in LDS
//    (two window buffers, 24 KB).  Each wave reads a window's pieces into registers once,
//    at the first slot that uses them.
//  - B (h_{t-1} and x_t columns): read from memory a slot before the products that use
//    them, eight values per lane and tile, split in registers (split8).
//  - The products of window m run during the eight steps of window m+1 (slots), column
//    tile c at slot c % 8 (one or two tiles per slot), from the step's barrier on, beside
//    the recurrent waves' own products.  The last window (and what a short last window
//    leaves of the one before) runs in slots after the final barrier.
//  - dW_hh_s accumulates in registers and goes out as an fp32 plane per chunk of TS
//    steps (TS a multiple of 8); each dW_ih tile accumulates one window in registers and
//    is then added to the fp64 LDS copy (ds_add_f64).
// Six piece products per tile and window (split_bf16.h), smallest first.  Against the
// fp32 16x16x4 stage the recurrent waves lose less time to the products (a 16-bit stream
// holds off the other wave on the SIMD less than an fp32 one).  Returns true when the
// wave has taken part in the workgroup's final barrier (always, except after an abort
// inside the loop).
constexpr int kWin = 8;
constexpr unsigned kApieceBytes = 2u * 4u * 3u * 64u * 16u;  // [window parity][row tile][piece][lane]
constexpr int kBwdXLdsBytes = kXaccLdsBytes + (int)kApieceBytes;
// dynamic LDS of a backward with weight-gradient waves (XT >= 0), products on split bf16
// pieces (WS) or on the fp32 instruction
constexpr int bwd_lds_bytes(int xt, bool ws) {
  return xt > 0 ? (ws ? kBwdXLdsBytes : kXaccLdsBytes) : kPadLdsBytes;
}
static_assert(kApieceBytes <= (unsigned)kPadLdsBytes, "the A operands fit the padding LDS without dW_ih");

__device__ __forceinline__ f4 mfma16_bf16(u32x4 a, u32x4 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                 0, 0);
}

template <int J, int N, class F>
__device__ __forceinline__ bool for_steps(F&& f) {
  if constexpr (J == N) {
    return true;
  } else {
    if (!f(std::integral_constant<int, J>{})) return false;
    return for_steps<J + 1, N>(f);
  }
}

template <int KQ, int XT>
__device__ __forceinline__ bool rec_bwd_wgrad_win(const PBwdArgs& p, int grp, int wg, float (&dgl)[2][4][68],
                                                  char* lds, int& abort_flag) {
  constexpr int HT = KQ >= 32 ? KQ / 32 : 1;  // h column groups of 32 per wave (4*KQ >= H)
  constexpr int NH = 2 * HT;                   // h column tiles per wave
  constexpr int NX = XT > 0 ? 2 * XT : 0;      // x column tiles per wave
  constexpr int C = NH + NX;
  const int T = p.T, B = p.B, H = p.H, D = p.D, Bg = p.Bg, NG = p.NG, TS = p.TS;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane((threadIdx.x >> 6) - 4);
  const int kb = lane >> 4, l16 = lane & 15;  // batch slot of the lane's k values
  const int cb = grp * Bg + kb;
  const bool bok = kb < Bg && cb < B;
  const int nth = (H + 31) / 32, ntx = (D + 31) / 32;
  double* const xacc = reinterpret_cast<double*>(lds);
  const unsigned abase = XT > 0 ? (unsigned)kXaccLdsBytes : 0u;
  // the fields used inside the loop, as locals (the lambdas below capture these, not p)
  const float* const h_save = p.h_save;
  const float* const xrows = p.x;
  float* const wph = p.wph;

  // The lane's index as a value the compiler cannot see through: addresses derived from
  // it inside the loop are recomputed where they are used instead of being kept in
  // registers for the whole loop (which the 128 dW_hh accumulators do not leave room for).
  auto opaque_lane = [&]() {
    int l = lane;
    asm volatile("" : "+v"(l));
    return l;
  };
  // column tile c: h tiles (group c/2, half c%2) then x tiles
  auto tile_g = [](int c) { return c < NH ? c / 2 : (c - NH) / 2; };
  auto tile_sub = [](int c) { return c < NH ? c % 2 : (c - NH) % 2; };
  auto tile_on = [&](int c) { return w + 4 * tile_g(c) < (c < NH ? nth : ntx); };  // wave-uniform
  auto tile_col = [&](int c) { return (w + 4 * tile_g(c)) * 32 + 16 * tile_sub(c) + l16; };

  f4 acch[HT][2][4];  // [column group][half][row tile]
  auto zero_h = [&]() {
#pragma unroll
    for (int g = 0; g < HT; ++g)
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) acch[g][sub][rt] = f4{0.f, 0.f, 0.f, 0.f};
  };
  zero_h();
  // D-layout of a 16x16 tile: lane l, register r -> row 4(l/16) + r, column l%16
  auto tile_row = [&](int rt, int r) { return rt * 16 + 4 * kb + r; };
  if constexpr (XT > 0) {
#pragma unroll
    for (int c = NH; c < C; ++c) {
      if (!tile_on(c)) continue;
#pragma unroll
      for (int rt = 0; rt < 4; ++rt)
#pragma unroll
        for (int r = 0; r < 4; ++r) xacc[tile_row(rt, r) * 256 + tile_col(c)] = 0.0;
    }
  }

  // B of tile c for the eight steps of window win (clamped rows past T; zeroed at use).
  // No branch around the loads (a tile that is off loads clamped addresses it never
  // uses): the waits before the products count outstanding loads exactly only when every
  // path issues the same loads.
  auto load_b = [&](int c, int win, float (&v)[kWin]) {
    const int ol = opaque_lane();
    const int cl = (w + 4 * tile_g(c)) * 32 + 16 * tile_sub(c) + (ol & 15);
    const int col = c < NH ? min(cl, H - 1) : min(cl, D - 1);
    const int okb = ol >> 4;
    const int orow = okb < Bg && grp * Bg + okb < B ? grp * Bg + okb : 0;
#pragma unroll
    for (int i = 0; i < kWin; ++i) {
      const int s = kWin * win + i;
      const int t = s < T ? T - 1 - s : 0;
      if (c < NH)
        v[i] = *byte_at(h_save + (size_t)t * B * H, 4u * (unsigned)(orow * H + col));
      else
        v[i] = *byte_at(xrows + (size_t)t * B * D, 4u * (unsigned)(orow * D + col));
    }
  };
  // the A pieces of window win's four row tiles
  auto read_a = [&](int win, u32x4 (&a)[4][3]) {
    const char* const ab = lds + abase + (unsigned)(win & 1) * (4u * 3u * 1024u) + 16u * opaque_lane();
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int pc = 0; pc < 3; ++pc) a[rt][pc] = *reinterpret_cast<const u32x4*>(ab + (rt * 3 + pc) * 1024);
  };
  // the products of tile c for window win; steps i >= nvalid of the window do not exist
  auto products = [&](int c, int win, const float (&v)[kWin], int nvalid, const u32x4 (&a)[4][3]) {
    if (!tile_on(c)) return;
    float vv[kWin];
#pragma unroll
    for (int i = 0; i < kWin; ++i) vv[i] = (bok && i < nvalid) ? v[i] : 0.f;
    u32x4 bp[3];
    split8(vv, bp);
    const int ol = opaque_lane();
    const int g = tile_g(c), sub = tile_sub(c);
    f4 xa[4] = {f4{0.f, 0.f, 0.f, 0.f}, f4{0.f, 0.f, 0.f, 0.f}, f4{0.f, 0.f, 0.f, 0.f}, f4{0.f, 0.f, 0.f, 0.f}};
    // piece product i of the four row tiles in turn: four independent accumulators
    // between dependent products
#pragma unroll
    for (int i = 5; i >= 0; --i)
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        if (c < NH)
          acch[g][sub][rt] = mfma16_bf16(a[rt][kPa[i]], bp[kPb[i]], acch[g][sub][rt]);
        else
          xa[rt] = mfma16_bf16(a[rt][kPa[i]], bp[kPb[i]], xa[rt]);
      }
    if (c >= NH) {  // the window's dW_ih tile into the fp64 copy
      double* const xl = xacc + (4 * (ol >> 4)) * 256 + (w + 4 * g) * 32 + 16 * sub + (ol & 15);
#pragma unroll
      for (int rt = 0; rt < 4; ++rt)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          __hip_atomic_fetch_add(xl + (rt * 16 + r) * 256, (double)xa[rt][r], __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  };
  // Row r64 = rt*16 + 4*kb + r of a tile is gate rt, unit wg*16 + 4*kb + r.
  // (addresses from opaque_lane: the several call sites share no address registers)
  auto dump_h = [&](int chunk) {
    __builtin_amdgcn_sched_barrier(0);
    float* const plane = wph + ((size_t)chunk * NG + grp) * 4 * H * H;
    const int ol = opaque_lane();
    const int ul = wg * kUnits + 4 * (ol >> 4);
#pragma unroll
    for (int g = 0; g < HT; ++g) {
      if (w + 4 * g >= nth) continue;
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        const int c = (w + 4 * g) * 32 + 16 * sub + (ol & 15);
        const unsigned lo = 4u * ((unsigned)ul * H + c);
#pragma unroll
        for (int rt = 0; rt < 4; ++rt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float* const rb = plane + (size_t)(rt * H + r) * H;
            if (ul + r < H && c < H) *byte_at(rb, lo) = acch[g][sub][rt][r];
          }
      }
    }
    zero_h();
    __builtin_amdgcn_sched_barrier(0);
  };
  // element j of the lanes' A operands of row tile w in window buffer m&1: the three pieces
  // of v
  auto put_pieces = [&](int m, int j, float v) {
    const __bf16 p0 = (__bf16)v;
    const float r1 = v - (float)p0;
    const __bf16 p1 = (__bf16)r1;
    const __bf16 p2 = (__bf16)(r1 - (float)p1);
    char* const dst =
        lds + abase + (unsigned)(m & 1) * (4u * 3u * 1024u) + (unsigned)w * 3072u + 16u * opaque_lane() + 2u * j;
    *reinterpret_cast<__bf16*>(dst) = p0;
    *reinterpret_cast<__bf16*>(dst + 1024) = p1;
    *reinterpret_cast<__bf16*>(dst + 2048) = p2;
  };

  // Slot (m, j), m = 0..M (M windows): step s = 8m + j when s < T, and runs tile j of
  // window m-1 and, in the odd slots, one of the tiles past the eighth (xtile: the dW_ih
  // tiles when the workgroup has 12).  Slot 0 also reads the window's A pieces, so the
  // extra tiles go to the odd slots: put in slots 0-3 (tiles j and j+8) they made the
  // weight-gradient waves reach the recurrent waves' barrier 1.2 us late after slot 0 and
  // 0.24 us late after slots 1-3 (barrier-arrival stamps), and the configs[2] step took
  // 0.968-0.972 ms instead of 0.948-0.953.  Slots with s >= T come after the loop's last
  // step: the first of them (s == T) zeroes the A elements of the missing steps of the
  // last window and takes part in the final barrier, and they run the rest of the products
  // without waiting for anything.
  const int M = (T + kWin - 1) / kWin;
  const int last = M - 1, nvalid = T - kWin * last;  // steps of the last window
  static_assert(C - kWin <= kWin / 2, "one extra tile per odd slot");
  auto xtile = [](int j) constexpr { return (j % 2 == 1 && kWin + j / 2 < C) ? kWin + j / 2 : -1; };
  float nb[2][kWin];  // B of the next slot's tiles (j and xtile(j))
  u32x4 apc[4][3];    // A pieces of the window whose products the slots run
  bool final_done = false;
  auto slot = [&](int m, auto jc) __attribute__((always_inline)) -> bool {
    constexpr int j = decltype(jc)::value;
    const int s = kWin * m + j;
    __builtin_amdgcn_sched_barrier(0);  // nothing of another slot moves into this one
    if (s < T) {
      lds_barrier();  // the recurrent waves' barrier of step s: dgl[s&1] is complete
      if (abort_flag) return false;
      {
        const int ol = opaque_lane();
        put_pieces(m, j, dgl[s & 1][ol >> 4][w * 16 + (ol & 15)]);
      }
      // the window's A pieces, once per window (they serve its eight slots)
      if constexpr (j == 0) read_a(max(m - 1, 0), apc);
      // The products start at once, beside the recurrent waves' own: a slot that waited
      // for those (an LDS flag) reached the next barrier after the recurrent waves in
      // most steps (launch-phase stamps), and the step took its length.
    } else {
      if (s == T) {
        for (int jj = nvalid; jj < kWin; ++jj) put_pieces(last, jj, 0.f);
        lds_barrier();  // the workgroup's final barrier (the recurrent waves' last one)
        final_done = true;
        if (abort_flag) return false;
      }
      if (j == 0 || s == T) read_a(max(m - 1, 0), apc);
    }
    if (m > 0) {  // window m-1's tiles j and xtile(j)
      const int nv = m - 1 == last ? nvalid : kWin;
      if constexpr (j < C) products(j, m - 1, nb[0], nv, apc);
      if constexpr (xtile(j) >= 0) products(xtile(j), m - 1, nb[1], nv, apc);
      if constexpr (j == kWin - 1)
        if (m == M || (kWin * m) % TS == 0) dump_h(kWin * (m - 1) / TS);
    }
    {  // B of the next slot's tiles: window m-1, or window m after j = 7 (clamped: a
       // slot without products loads window 0 or M-1 and does not use it)
      constexpr int jn = (j + 1) % kWin;
      const int wn = min(max(j + 1 < kWin ? m - 1 : m, 0), M - 1);
      if constexpr (jn < C) load_b(jn, wn, nb[0]);
      if constexpr (xtile(jn) >= 0) load_b(xtile(jn), wn, nb[1]);
      // the loads stay here, a slot ahead of their use: without this the compiler sinks
      // them past the next barrier to the products, and each slot waits for memory twice
      asm volatile("" ::: "memory");
    }
    __builtin_amdgcn_sched_barrier(0);
    return true;
  };
  for (int m = 0; m <= M; ++m)
    if (!for_steps<0, kWin>([&](auto jc) { return slot(m, jc); })) return final_done;

  if constexpr (XT > 0) {  // this group's dW_ih rows (fp64 sums, rounded once) as a plane
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");  // the wave's own LDS adds
    float* const plane = p.wpx + (size_t)grp * 4 * H * D;
#pragma unroll
    for (int c = NH; c < C; ++c) {
      if (!tile_on(c)) continue;
      const int col = tile_col(c);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int rt = 0; rt < 4; ++rt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int r64 = tile_row(rt, r), u = wg * kUnits + (r64 & 15);
          if (u < H && col < D) plane[((size_t)(r64 >> 4) * H + u) * D + col] = (float)xacc[r64 * 256 + col];
        }
    }
  }
  return true;
}

// After an abort, a recurrent wave sets what its cell lanes own to NaN: dh0/dc0, the
// bias partials and (when they are stored) the dgates of its batch slot and the
// workgroup's units.
__device__ void poison_bwd(const PBwdArgs& p, int grp, int wg) {
  const int lane = threadIdx.x & 63, q = threadIdx.x >> 6;
  const int cb = grp * p.Bg + q, cu = wg * kUnits + (lane & 15);
  if (lane >= kUnits || q >= p.Bg || cb >= p.B || cu >= p.H) return;
  const float nan = __uint_as_float(0x7FC00000u);
  const int H = p.H;
  const size_t e = (size_t)cb * H + cu;
  if (p.dh0) p.dh0[e] = nan;
  if (p.dc0) p.dc0[e] = nan;
  for (int gt = 0; gt < 4; ++gt) p.db_part[(size_t)cb * 4 * H + gt * H + cu] = (double)nan;
  if (p.store_dg)
    for (int t = 0; t < p.T; ++t)
      for (int gt = 0; gt < 4; ++gt) p.dgates[((size_t)t * p.B + cb) * 4 * H + gt * H + cu] = nan;
}

// ... and a weight-gradient wave sets every element of the planes it writes to NaN: its
// 32-column tiles of the workgroup's 64 rows in the group's dW_hh_s plane of every chunk
// and, with XT > 0, in the group's dW_ih plane.
template <int KQ, int XT>
__device__ void poison_wgrad(const PBwdArgs& p, int grp, int wg) {
  constexpr int HT = KQ >= 32 ? KQ / 32 : 1;
  const int lane = threadIdx.x & 63, w = (threadIdx.x >> 6) - 4;
  const int H = p.H, D = p.D;
  const float nan = __uint_as_float(0x7FC00000u);
  const int chunks = (p.T + p.TS - 1) / p.TS;
  for (int r = lane >> 5; r < 64; r += 2) {
    const int u = wg * kUnits + (r & 15);
    if (u >= H) continue;
    const size_t row = (size_t)(r >> 4) * H + u;
    for (int i = 0; i < HT; ++i) {
      const int c = (w + 4 * i) * 32 + (lane & 31);
      if (c >= H) continue;
      for (int ch = 0; ch < chunks; ++ch) p.wph[(((size_t)ch * p.NG + grp) * 4 * H + row) * H + c] = nan;
    }
    if constexpr (XT > 0) {
      for (int i = 0; i < XT; ++i) {
        const int c = (w + 4 * i) * 32 + (lane & 31);
        if (c < D) p.wpx[((size_t)grp * 4 * H + row) * D + c] = nan;
      }
    }
  }
}

// XT < 0: 256 threads, recurrent waves only (weight gradients by separate GEMMs).
// XT >= 0: 512 threads; waves 4-7 accumulate dW_hh_s and, when XT > 0, dW_ih, on split
// bf16 products (WS, rec_bwd_wgrad_win) or on the fp32 instruction (rec_bwd_wgrad), as
// hsl_set_split_products selects.
// As in the forward, every wave ends with one more workgroup barrier and then poisons
// its outputs if any wave of the workgroup gave up a wait.
template <int KQ, int XT, bool WS>
__global__ __launch_bounds__(XT >= 0 ? 512 : 256, 1) void rec_bwd_persistent(PBwdArgs p) {
  constexpr int NWMAX = 4 * KQ / kUnits;
  constexpr bool GW = XT >= 0;
  __shared__ float dgl[2][4][64 + 4];  // [step parity][batch slot][gate row]
  __shared__ int abort_flag;
  const int grp = blockIdx.x % p.NGX, wg = blockIdx.x / p.NGX;
  if (grp >= p.NG) return;
  if (threadIdx.x == 0) abort_flag = 0;
  if (threadIdx.x < 4) step_flags()[threadIdx.x] = 0;  // steps whose products wave q has issued
  const bool fast = agree_placement(p.hello + (size_t)grp * NWMAX, wg, p.NW, p.spin, &abort_flag, p.err) &&
                    !p.device_scope;
  const bool wgrad_wave = GW && threadIdx.x >= 256;
  bool passed_final = false;  // the wave has taken part in the final barrier below
  if (!abort_flag) {
    if constexpr (GW) {
      if (wgrad_wave) {
        // [64][256] fp64 dW_ih accumulator (XT > 0), then the bf16 A operands of two
        // windows (dynamic LDS)
        extern __shared__ double xacc[];
        if constexpr (WS)
          passed_final =
              rec_bwd_wgrad_win<KQ, (XT > 0 ? XT : 0)>(p, grp, wg, dgl, reinterpret_cast<char*>(xacc), abort_flag);
        else
          rec_bwd_wgrad<KQ, (XT > 0 ? XT : 0)>(p, grp, wg, dgl, xacc, abort_flag);
      } else {
        __builtin_amdgcn_s_setprio(2);  // the recurrent chain first when both waves can issue
      }
    }
    if (!wgrad_wave) {
      if (fast)
        rec_bwd_body<KQ, true, GW>(p, grp, wg, dgl, abort_flag);
      else
        rec_bwd_body<KQ, false, GW>(p, grp, wg, dgl, abort_flag);
    }
  }
  if (!passed_final) lds_barrier();
  if (abort_flag) {
    if constexpr (GW) {
      if (wgrad_wave) {
        poison_wgrad<KQ, (XT > 0 ? XT : 0)>(p, grp, wg);
        return;
      }
    }
    poison_bwd(p, grp, wg);
  }
}

#include "rec_wide.h"
#include "rec_wide_fwd.h"
#include "rec_wide_bwd32.h"

// ---------------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------------
struct PersistentPlan {
  bool ok = false;
  int KQ = 0, Hp = 0, NG = 0, NGX = 0, Bg = 0, NW = 0, grid = 0;
  int XT = -1;  // backward: -1 no weight-gradient waves, 0 dW_hh only, 2 dW_hh and dW_ih
  bool XP = false;  // forward: input projection inside the kernel (512 threads)
  bool XS = false;  // with XP: its products on split bf16 pieces
  bool WS = true;   // backward with XT >= 0: weight-gradient products on split bf16 pieces
};

int pick_kq(int H) {
  if (H <= 64) return 16;
  if (H <= 128) return 32;
  if (H <= 256) return 64;
  if (H <= 512) return 128;
  return 0;
}

template <class K>
int max_resident(K kernel, int threads, int* out) {
  int occ = 0;
  HSL_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kernel, threads, kFwdLdsBytes));
  *out = occ;
  return HSL_OK;
}

// Weight-gradient waves in the persistent backward: on unless HSL_FUSED_WGRAD=0.
// Input projection inside the persistent forward: on unless HSL_FUSED_XPROJ=0.
bool fused_xproj_enabled() {
  static const bool on = [] {
    const char* e = getenv("HSL_FUSED_XPROJ");
    return !(e && e[0] == '0');
  }();
  return on;
}

bool fused_wgrad_enabled() {
  static const bool on = [] {
    const char* e = getenv("HSL_FUSED_WGRAD");
    return !(e && e[0] == '0');
  }();
  return on;
}

template <int KQ>
int fwd_resident(int xp, int* occ) {
  switch (xp) {
    case 0: return max_resident(rec_fwd_persistent<KQ, 0>, 256, occ);
    case 1: return max_resident(rec_fwd_persistent<KQ, 1>, 512, occ);
    default: return max_resident(rec_fwd_persistent<KQ, 2>, 512, occ);
  }
}

template <int KQ, bool WS>
int bwd_resident_ws(int xt, int* occ) {
  int o = 0;
  switch (xt) {
    case -1:
      HSL_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, rec_bwd_persistent<KQ, -1, true>, 256,
                                                           bwd_lds_bytes(-1, true)));
      break;
    case 0:
      HSL_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, rec_bwd_persistent<KQ, 0, WS>, 512,
                                                           bwd_lds_bytes(0, WS)));
      break;
    default:
      HSL_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, rec_bwd_persistent<KQ, 2, WS>, 512,
                                                           bwd_lds_bytes(2, WS)));
      break;
  }
  *occ = o;
  return HSL_OK;
}
template <int KQ>
int bwd_resident(int xt, bool ws, int* occ) {
  return ws ? bwd_resident_ws<KQ, true>(xt, occ) : bwd_resident_ws<KQ, false>(xt, occ);
}

int plan_persistent(int B, int H, int D, bool bwd, PersistentPlan* pl) {
  *pl = PersistentPlan{};
  const int mode = recurrent_path_mode();
  if (mode == 1) return HSL_OK;
  const int kq = pick_kq(H);
  if (kq == 0 || B < 1) return HSL_OK;
  DeviceInfo di;
  HSL_CHECK(device_info(&di));
  PersistentPlan p;
  p.KQ = kq;
  p.Hp = 4 * kq;
  p.NG = (B + 3) / 4;
  p.Bg = (B + p.NG - 1) / p.NG;
  // group g is served by workgroups blockIdx % NGX == g; NGX is a multiple of the XCD
  // count so that every group sits on one XCD (workgroup i runs on XCD i % 8)
  p.NGX = (p.NG + di.num_xcds - 1) / di.num_xcds * di.num_xcds;
  p.NW = (H + kUnits - 1) / kUnits;
  p.grid = p.NGX * p.NW;
  // dW_ih joins the weight-gradient waves when its 32-column tiles fit two per wave
  if (bwd && fused_wgrad_enabled()) p.XT = (D > 0 && D <= 256) ? 2 : 0;
  // the forward's projection waves hold W_ih rows for a quarter of D <= 256 each and read
  // x rows with 16-byte loads
  if (!bwd && fused_xproj_enabled()) p.XP = D > 0 && D <= 256 && D % 4 == 0;
  p.XS = kXprojSplit && split_products_mode();
  p.WS = split_products_mode() != 0;
  int occ = 0;
  for (;;) {
    if (bwd) {
      switch (kq) {
        case 16: HSL_CHECK(bwd_resident<16>(p.XT, p.WS, &occ)); break;
        case 32: HSL_CHECK(bwd_resident<32>(p.XT, p.WS, &occ)); break;
        case 64: HSL_CHECK(bwd_resident<64>(p.XT, p.WS, &occ)); break;
        default: HSL_CHECK(bwd_resident<128>(p.XT, p.WS, &occ)); break;
      }
    } else {
      const int xp = p.XP ? (p.XS ? 2 : 1) : 0;
      switch (kq) {
        case 16: HSL_CHECK(fwd_resident<16>(xp, &occ)); break;
        case 32: HSL_CHECK(fwd_resident<32>(xp, &occ)); break;
        case 64: HSL_CHECK(fwd_resident<64>(xp, &occ)); break;
        default: HSL_CHECK(fwd_resident<128>(xp, &occ)); break;
      }
    }
    // every workgroup must be resident at once: the waits are between workgroups
    p.ok = occ >= 1 && (long)occ * di.num_cus >= p.grid;
    if (p.ok || (p.XT < 0 && !p.XP)) break;
    p.XT = -1;  // retry without the weight-gradient / projection waves
    p.XP = false;
  }
  *pl = p;
  return HSL_OK;
}

// The W_hh-resident kernels for large H (rec_wide.h, rec_wide_fwd.h, rec_wide_bwd32.h): H = 32 U
// with U = 64 (2048) or 32 (1024), B <= 32, eight XCDs and all 256 workgroups resident at
// once (one per CU).
struct WidePlan {
  bool ok = false;
  int U = 0;
};

// dynamic LDS of the wide kernels, padded so that one workgroup fits per CU: the forward's
// h buffer of each chain, the backward's wave partials and gathered dg group
template <int U>
constexpr size_t wide_fwd_lds() {
  return WideFShape<U>::LDS_BYTES > (size_t)kPadLdsBytes ? WideFShape<U>::LDS_BYTES : (size_t)kPadLdsBytes;
}
template <int U>
constexpr size_t wide_bwd_lds() {  // rec_bwd_wide<64> or rec_bwd_wide1<32>
  constexpr size_t b = U == 32 ? (size_t)WideB1Shape<32>::LDS_BYTES : (size_t)WideBShape<U>::LDS_BYTES;
  return b > (size_t)kPadLdsBytes ? b : (size_t)kPadLdsBytes;
}

// exchange words of the wide kernels: forward h blocks then partial inboxes; backward dg
// broadcasts then partial inboxes (floats)
size_t wide_fwd_hfloats(int U) { return (size_t)kWideHSlots * 2 * (kWideXcds * kWideRowSubs) * 16 * U; }
size_t wide_fwd_floats(int U) {
  return wide_fwd_hfloats(U) + (size_t)kWidePSlots * 2 * kWideWgs * kWideKBlocks * (U / 8) * 16 * 4;
}
size_t wide_bwd_bfloats(int U) { return (size_t)kWideHSlots * kWideXcds * (16 * U) * 32; }
size_t wide_bwd_floats(int U) { return wide_bwd_bfloats(U) + (size_t)kWidePSlots * kWideWgs * (8 * 32 * (U / 8)); }

template <int U>
int wide_occupancy(bool bwd, int* occ) {
  if (bwd)
    HSL_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(
        occ, U == 32 ? (const void*)rec_bwd_wide1<32> : (const void*)rec_bwd_wide<64>, 256, wide_bwd_lds<U>()));
  else
    HSL_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(occ, rec_fwd_wide<U>, 256, wide_fwd_lds<U>()));
  return HSL_OK;
}

int plan_wide(int B, int H, bool bwd, WidePlan* pl) {
  *pl = WidePlan{};
  if (recurrent_path_mode() == 1 || B < 1 || B > 32 || (H != 2048 && H != 1024)) return HSL_OK;
  DeviceInfo di;
  HSL_CHECK(device_info(&di));
  if (di.num_xcds != kWideXcds || di.num_cus < kWideWgs) return HSL_OK;
  const int U = H / 32;
  int occ = 0;
  if (U == 64)
    HSL_CHECK(wide_occupancy<64>(bwd, &occ));
  else
    HSL_CHECK(wide_occupancy<32>(bwd, &occ));
  pl->ok = occ >= 1 && (long)occ * di.num_cus >= kWideWgs;
  pl->U = U;
  return HSL_OK;
}

// Chunks of the fused weight gradients' fp32 partial planes, at most 8 per group (the
// workspace holds 8).  Up to T = 2048 (window products) or T = 1024 (fp32 products) a
// chunk spans at most 256 or 128 steps: each running sum then takes at most 32 windows of
// six 32-term products, or 512 single products.  Longer sequences share the 8 chunks, so
// a chunk spans ceil(T / 8) steps (at T = 2048 with the fp32 products: 1024 single
// products per running sum, which the long-sequence test checks against the parity bar).
int wgrad_chunks(int T, bool ws) {
  const int span = ws ? 256 : 128;
  const int c = (T + span - 1) / span;
  return c < 1 ? 1 : (c > 8 ? 8 : c);
}

inline int grid_for(size_t n) {
  size_t b = (n + 255) / 256;
  if (b < 1) b = 1;
  if (b > 2048) b = 2048;
  return (int)b;
}

// k-splits of a per-step product with an M x N output (32x32 tiles) and depth K: enough
// workgroups to cover the chip twice, at least two 128-deep slices per split.  Returns
// the number of planes the launch really writes (1 = fused epilogue, no partials).
int step_splits(int M, int N, int K, int* k_per_split) {
  const int tiles = ((M + 31) / 32) * ((N + 31) / 32);
  int s = 1;
  if (tiles < 256 && K >= 512) {
    s = (512 + tiles - 1) / tiles;
    const int max_by_k = K / 256;
    if (s > max_by_k) s = max_by_k;
    if (s > 16) s = 16;
    if (s < 1) s = 1;
  }
  return split_layout<CfgStep>(K, s, k_per_split);
}

int fill_words(unsigned long long* p, size_t n, unsigned long long v, hipStream_t s) {
  if (n == 0) return HSL_OK;
  hipLaunchKernelGGL(fill_u64_kernel, dim3(grid_for(n)), dim3(256), 0, s, p, n, v);
  HSL_HIP(hipGetLastError());
  return HSL_OK;
}

// Before a persistent launch: error flag cleared, hand-off slots empty (every 4-byte
// word kEmpty), placement words cleared, in one launch.
int prepare_persistent(int* err, float* slots, size_t slot_floats, unsigned long long* hello, size_t hwords,
                       hipStream_t s) {
  const size_t n1 = 32, n2 = (slot_floats + 1) / 2;
  hipLaunchKernelGGL(fill3_u64_kernel, dim3(grid_for(n1 + (n2 + 1) / 2 + hwords)), dim3(256), 0, s,
                     reinterpret_cast<unsigned long long*>(err), n1, 0ull,
                     reinterpret_cast<unsigned long long*>(slots), n2, kEmpty2, hello, hwords, 0ull);
  HSL_HIP(hipGetLastError());
  return HSL_OK;
}

int copy_f32_impl(float* dst, const float* src, size_t n, hipStream_t s) {
  if (n == 0) return HSL_OK;
  hipLaunchKernelGGL(copy_f32_kernel, dim3(grid_for(n)), dim3(256), 0, s, dst, src, n);
  HSL_HIP(hipGetLastError());
  return HSL_OK;
}

// Workspace layouts.  The int error flag sits at offset 0 of both.
struct FwdWs {
  int* err;
  float* xbuf;                // [4*NG*4*Hp] (persistent)
  size_t xfloats;
  unsigned long long* hello;  // [NG*Hp/16]  (persistent)
  size_t hwords;
  float* gih;                 // [T*B*4H]    (input projection not fused)
  float* wbuf;                // h blocks, then partial inboxes (wide persistent)
  size_t wfloats, whfloats;   // all of wbuf; its h blocks
  unsigned long long* whello; // [256]       (wide persistent)
  float* w_perm;              // [4H*H]      (per-step)
  float* bs;                  // [4H]        (per-step)
  float* part;                // [S*B*4H]    (per-step split-K planes)
};

// Which parts of the forward workspace a call uses: the persistent exchange buffers, the
// [T,B,4H] input-gate buffer (not when the projection is fused into the persistent
// kernel) and the per-step buffers.  All three when the path is not known (no device).
struct FwdNeeds {
  bool xch = true, gih = true, step = true, wide = true;
};

size_t carve_fwd(void* ws, size_t cap, int T, int B, int H, FwdNeeds nd, FwdWs* o) {
  Carver c(ws, cap);
  *o = FwdWs{};
  o->err = c.take<int>(64);
  const int kq = pick_kq(H);
  if (nd.xch && kq) {
    const size_t ng = (size_t)(B + 3) / 4;
    o->hwords = ng * (size_t)(4 * kq / kUnits);
    o->xfloats = 4 * ng * 4 * (size_t)(4 * kq);
    o->xbuf = c.take<float>(o->xfloats);
    o->hello = c.take<unsigned long long>(o->hwords);
  }
  if (nd.gih) o->gih = c.take<float>((size_t)T * B * 4 * H);
  if (nd.wide && (H == 2048 || H == 1024)) {
    o->whfloats = wide_fwd_hfloats(H / 32);
    o->wfloats = wide_fwd_floats(H / 32);
    o->wbuf = c.take<float>(o->wfloats);
    o->whello = c.take<unsigned long long>(kWideWgs);
  }
  if (nd.step) {
    o->w_perm = c.take<float>((size_t)4 * H * H);
    o->bs = c.take<float>((size_t)4 * H);
    int kps;
    const int sp = step_splits(B, 4 * H, H, &kps);
    o->part = c.take<float>(sp > 1 ? (size_t)sp * B * 4 * H : 0);
  }
  return c.off;
}

// The workspace parts of a forward call with this plan; the fused projection needs a
// 16-byte aligned x.
FwdNeeds fwd_needs(const PersistentPlan& pl, const WidePlan& wp, bool x_aligned) {
  FwdNeeds nd;
  nd.xch = pl.ok;
  nd.gih = !(pl.ok && pl.XP && x_aligned);
  nd.wide = !pl.ok && wp.ok;
  nd.step = !pl.ok && !wp.ok;
  return nd;
}

struct BwdWs {
  int* err;
  double* db_part;           // [B*4H]
  double* rowdot;            // [4H]
  float* dc;                 // [B*H]   (per-step)
  float* w_s;                // [4H*H]  (per-step)
  float* part;               // [S*B*H] (per-step split-K planes)
  float* pbuf;                // [3*NG*NWMAX*4*64*PER] (persistent)
  size_t pfloats;
  unsigned long long* hello;  // [NG*NWMAX]           (persistent)
  size_t hwords;
  float* gemm;               // shared by the weight-gradient GEMMs
  size_t gemm_bytes;
  float* dgates;             // [T*B*4H] (when they feed a product)
  float* wbuf;               // dg broadcast slots, then partial inboxes (wide persistent)
  size_t wfloats;
  unsigned long long* whello; // [256] (wide persistent)
};

size_t gemm_region_bytes(int T, int B, int D, int H) {
  const int TB = T * B;
  const int s4 = gemm_tn_planes(4 * H, H, TB);
  size_t need = sizeof(float) * (size_t)s4 * 4 * H * H;  // dW_hh partials (always staged)
  const size_t g5 = gemm_ws_bytes_layout(4 * H, D, TB, 1, 1, 0);
  const size_t g6 = gemm_ws_bytes_layout(TB, D, 4 * H, 1, 0, 0);
  if (g5 > need) need = g5;
  if (g6 > need) need = g6;
  const size_t g7 = gemm_ws_bytes(B, H, 4 * H, 1);
  if (g7 > need) need = g7;
  if (pick_kq(H) && fused_wgrad_enabled()) {  // planes of the fused weight gradients
    const size_t ng = (B + 3) / 4;
    // sized for the fp32 products' shorter chunks, whatever the mode is now
    const size_t wg = sizeof(float) * wgrad_chunks(T, false) * ng * 4 * H * H +
                      (D <= 256 ? sizeof(float) * ng * 4 * H * D : 0);
    if (wg > need) need = wg;
  }
  return need;
}

// Which parts of the backward workspace a call uses: the persistent exchange buffers,
// the per-step buffers and the [T,B,4H] dgates (only when a product reads them: dx, or
// dW_ih when the persistent kernel does not accumulate it).  All when the path is not
// known (no device).
struct BwdNeeds {
  bool xch = true, step = true, dgates = true, wide = true;
};

BwdNeeds bwd_needs(const PersistentPlan& pl, const WidePlan& wp, bool with_dx) {
  BwdNeeds nd;
  nd.xch = pl.ok;
  nd.wide = !pl.ok && wp.ok;
  nd.step = !pl.ok && !wp.ok;
  nd.dgates = !(pl.ok && pl.XT > 0) || with_dx;
  return nd;
}

size_t carve_bwd(void* ws, size_t cap, int T, int B, int D, int H, BwdNeeds nd, BwdWs* o) {
  Carver c(ws, cap);
  *o = BwdWs{};
  o->err = c.take<int>(64);
  o->db_part = c.take<double>((size_t)B * 4 * H);
  o->rowdot = c.take<double>((size_t)4 * H);
  if (nd.step) {
    o->dc = c.take<float>((size_t)B * H);
    o->w_s = c.take<float>((size_t)4 * H * H);
    int kps;
    const int sp = step_splits(B, H, 4 * H, &kps);
    o->part = c.take<float>(sp > 1 ? (size_t)sp * B * H : 0);
  }
  const int kq = pick_kq(H);
  if (nd.xch && kq) {
    const size_t ng = (size_t)(B + 3) / 4;
    const size_t nwmax = (size_t)(4 * kq / kUnits);
    const size_t per = (nwmax + 3) / 4;
    o->hwords = ng * nwmax;
    o->pfloats = 3 * ng * nwmax * 4 * 64 * per;
    o->pbuf = c.take<float>(o->pfloats);
    o->hello = c.take<unsigned long long>(o->hwords);
  }
  if (nd.wide && (H == 2048 || H == 1024)) {
    o->wfloats = wide_bwd_floats(H / 32);
    o->wbuf = c.take<float>(o->wfloats);
    o->whello = c.take<unsigned long long>(kWideWgs);
  }
  o->gemm_bytes = gemm_region_bytes(T, B, D, H);
  o->gemm = c.take<float>(o->gemm_bytes / sizeof(float) + 1);
  if (nd.dgates) o->dgates = c.take<float>((size_t)T * B * 4 * H);
  return c.off;
}

int check_dims(int T, int B, int D, int H) { return check_shape("recurrent mode", T, B, D, H); }

template <int KQ>
void launch_fwd_persistent(const PFwdArgs& a, int grid, int xp, hipStream_t s) {
  switch (xp) {
    case 0: hipLaunchKernelGGL((rec_fwd_persistent<KQ, 0>), dim3(grid), dim3(256), kFwdLdsBytes, s, a); break;
    case 1: hipLaunchKernelGGL((rec_fwd_persistent<KQ, 1>), dim3(grid), dim3(512), kFwdLdsBytes, s, a); break;
    default: hipLaunchKernelGGL((rec_fwd_persistent<KQ, 2>), dim3(grid), dim3(512), kFwdLdsBytes, s, a); break;
  }
}
template <int KQ, bool WS>
void launch_bwd_persistent_ws(const PBwdArgs& a, int grid, int xt, hipStream_t s) {
  switch (xt) {
    case -1:
      hipLaunchKernelGGL((rec_bwd_persistent<KQ, -1, true>), dim3(grid), dim3(256), bwd_lds_bytes(-1, true), s, a);
      break;
    case 0:
      hipLaunchKernelGGL((rec_bwd_persistent<KQ, 0, WS>), dim3(grid), dim3(512), bwd_lds_bytes(0, WS), s, a);
      break;
    default:
      hipLaunchKernelGGL((rec_bwd_persistent<KQ, 2, WS>), dim3(grid), dim3(512), bwd_lds_bytes(2, WS), s, a);
      break;
  }
}
template <int KQ>
void launch_bwd_persistent(const PBwdArgs& a, int grid, int xt, bool ws, hipStream_t s) {
  if (ws)
    launch_bwd_persistent_ws<KQ, true>(a, grid, xt, s);
  else
    launch_bwd_persistent_ws<KQ, false>(a, grid, xt, s);
}

}  // namespace

int zero_words(unsigned long long* p, size_t n, hipStream_t s) { return fill_words(p, n, 0ull, s); }
int copy_f32(float* dst, const float* src, size_t n, hipStream_t s) { return copy_f32_impl(dst, src, n, s); }

int bias_grads_from_parts(const double* db_part, int B, const double* rowdot, const float* b_hh, const float* a,
                          float* db_ih, float* db_hh, float* da, int H, hipStream_t s, const double* dotp,
                          int dot_parts) {
  if (H == 0) return HSL_OK;
  hipLaunchKernelGGL(bias_da_finalize_kernel, dim3(4), dim3(1024), 0, s, db_part, B, rowdot, b_hh, a, db_ih, db_hh,
                     da, H, dotp, dot_parts);
  HSL_HIP(hipGetLastError());
  return HSL_OK;
}

}  // namespace hsl

namespace hsl {
namespace {
__global__ void clear_device_errors_kernel() { g_device_errors = 0u; }

// ---- the allocation-free forward (hsl_rec_fwd_noalloc) ----------------------------
// Its workspace is `scratch`, a static device array: each device that loads the library
// holds its own copy until the process ends.  In host code the array's name is only a
// stand-in; the device address comes from hipGetSymbolAddress, once per device with that
// device current, and is what the kernels are given.
constexpr size_t kNoAllocScratchBytes = (size_t)4 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_addr[64] = {};

int scratch_address(void** out) {
  int dev = 0;
  HSL_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) return fail(HSL_ERR_UNSUPPORTED, "device index %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_addr[dev]) {
    void* p = nullptr;
    HSL_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return fail(HSL_ERR_HIP, "hipGetSymbolAddress(scratch) gave a null address");
    g_scratch_addr[dev] = p;
  }
  *out = g_scratch_addr[dev];
  return HSL_OK;
}
}  // namespace
}  // namespace hsl

using namespace hsl;

extern "C" {

int hsl_device_errors(int* flags, int clear, void* stream) {
  if (!flags) return fail(HSL_ERR_ARG, "hsl_device_errors: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  unsigned v = 0;
  HSL_HIP(hipMemcpyFromSymbolAsync(&v, HIP_SYMBOL(g_device_errors), sizeof(v), 0, hipMemcpyDeviceToHost, s));
  HSL_HIP(hipStreamSynchronize(s));
  if (clear && v) {
    hipLaunchKernelGGL(clear_device_errors_kernel, dim3(1), dim3(1), 0, s);
    HSL_HIP(hipGetLastError());
    HSL_HIP(hipStreamSynchronize(s));
  }
  *flags = static_cast<int>(v);
  return HSL_OK;
}

size_t hsl_rec_fwd_ws_bytes(int T, int B, int D, int H) {
  if (T < 0 || B < 0 || D < 0 || H < 0) return 0;
  FwdWs w;
  FwdNeeds nd;  // every part when the path cannot be planned (no device)
  PersistentPlan pl;
  WidePlan wp;
  if (B > 0 && H > 0 && plan_persistent(B, H, D, false, &pl) == HSL_OK && plan_wide(B, H, false, &wp) == HSL_OK)
    nd = fwd_needs(pl, wp, true);
  return carve_fwd(nullptr, 0, T, B, H, nd, &w);
}

int hsl_rec_fwd(const float* x, const float* h0, const float* c0, const float* w_ih, const float* w_hh,
                const float* b_ih, const float* b_hh, const float* a, float* h_save, float* c_save, float* gact,
                float* tanh_c, void* ws, size_t ws_bytes, int T, int B, int D, int H, void* stream) {
  HSL_CHECK(check_dims(T, B, D, H));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (B == 0 || H == 0) return HSL_OK;
  if (!w_hh || !b_hh || !a || !h_save || !c_save || (T > 0 && (!x || !w_ih || !b_ih || !gact || !tanh_c)))
    return fail(HSL_ERR_ARG, "hsl_rec_fwd: null pointer");
  PersistentPlan pl;
  HSL_CHECK(plan_persistent(B, H, D, false, &pl));
  WidePlan wp;
  if (!pl.ok) HSL_CHECK(plan_wide(B, H, false, &wp));
  if (recurrent_path_mode() == 2 && !pl.ok && !wp.ok)
    return fail(HSL_ERR_UNSUPPORTED, "persistent path does not fit (B=%d H=%d)", B, H);
  const bool x_aligned = reinterpret_cast<uintptr_t>(x) % 16 == 0;
  if (pl.XP && !x_aligned) pl.XP = false;  // the fused projection loads x in 16-byte pieces
  FwdWs w;
  const size_t need = carve_fwd(ws, ws_bytes, T, B, H, fwd_needs(pl, wp, x_aligned), &w);
  if (!ws || ws_bytes < need)
    return fail(HSL_ERR_ARG, "hsl_rec_fwd: workspace %zu bytes, need %zu%s", ws_bytes, need,
                pl.ok && !x_aligned ? " (x is not 16-byte aligned, so the input-gate buffer is needed)" : "");

  if (pl.ok && T > 0)
    HSL_CHECK(prepare_persistent(w.err, w.xbuf, w.xfloats, w.hello, w.hwords, s));
  else if (wp.ok && T > 0)
    HSL_CHECK(prepare_persistent(w.err, w.wbuf, w.wfloats, w.whello, kWideWgs, s));
  else
    HSL_CHECK(zero_words(reinterpret_cast<unsigned long long*>(w.err), 32, s));
  if (T == 0) {
    HSL_CHECK(copy_f32(h_save, h0, (size_t)B * H, s));
    HSL_CHECK(copy_f32(c_save, c0, (size_t)B * H, s));
    return HSL_OK;
  }
  if (!(pl.ok && pl.XP)) {
    // input projection for all T at once (_torch.py:96)
    GemmDesc g1{x, w_ih, b_ih, w.gih, T * B, 4 * H, D, D, D, 4 * H, 0, 1, 0};
    const int tslot = timing_begin(kTimeInputProj, s);
    HSL_CHECK(gemm_run(g1, nullptr, 0, s));
    timing_end(tslot, s);
  }

  if (pl.ok) {
    PFwdArgs pa{w.gih, w_hh, b_hh, a, h0, c0, h_save, c_save, gact, tanh_c, w.xbuf, w.hello, w.err,
                T, B, H, pl.Hp, pl.NG, pl.NGX, pl.Bg, pl.NW, exchange_scope_mode(), spin_timeout_ticks(),
                x, w_ih, b_ih, D};
    const int xp = pl.XP ? (pl.XS ? 2 : 1) : 0;
    const int slot = timing_begin(kTimeRecFwd, s);
    switch (pl.KQ) {
      case 16: launch_fwd_persistent<16>(pa, pl.grid, xp, s); break;
      case 32: launch_fwd_persistent<32>(pa, pl.grid, xp, s); break;
      case 64: launch_fwd_persistent<64>(pa, pl.grid, xp, s); break;
      default: launch_fwd_persistent<128>(pa, pl.grid, xp, s); break;
    }
    HSL_HIP(hipGetLastError());
    timing_end(slot, s);
    note_recurrent_path(2);
    return HSL_OK;
  }
  if (wp.ok) {
    WFwdArgs wa{w.gih, w_hh, b_hh, a, h0, c0, h_save, c_save, gact, tanh_c, w.wbuf, w.wbuf + w.whfloats, w.whello,
                w.err, T, B, H, exchange_scope_mode(), spin_timeout_ticks()};
    const int slot = timing_begin(kTimeRecFwd, s);
    if (wp.U == 64)
      hipLaunchKernelGGL(rec_fwd_wide<64>, dim3(kWideWgs), dim3(256), wide_fwd_lds<64>(), s, wa);
    else
      hipLaunchKernelGGL(rec_fwd_wide<32>, dim3(kWideWgs), dim3(256), wide_fwd_lds<32>(), s, wa);
    HSL_HIP(hipGetLastError());
    timing_end(slot, s);
    note_recurrent_path(3);
    return HSL_OK;
  }

  // per-step path
  hipLaunchKernelGGL(scale_whh_kernel, dim3(grid_for((size_t)4 * H * H)), dim3(256), 0, s, w_hh, b_hh, a,
                     (float*)nullptr, w.w_perm, w.bs, H);
  HSL_HIP(hipGetLastError());
  HSL_CHECK(copy_f32(h_save, h0, (size_t)B * H, s));
  HSL_CHECK(copy_f32(c_save, c0, (size_t)B * H, s));
  const size_t plane = (size_t)B * H, plane4 = (size_t)B * 4 * H;
  int kps;
  const int nsp = step_splits(B, 4 * H, H, &kps);
  const int slot = timing_begin(kTimeStepFwd, s);
  for (int t = 0; t < T; ++t) {
    GemmArgs ga{};
    ga.A = h_save + t * plane;
    ga.B = w.w_perm;
    ga.M = B;
    ga.N = 4 * H;
    ga.K = H;
    ga.lda = H;
    ga.ldb = H;
    ga.vec_a = aligned16(ga.A) && H % 4 == 0;
    ga.vec_b = aligned16(ga.B) && H % 4 == 0;
    if (nsp == 1) {
      EpiCellFwd epi{w.gih + t * plane4, w.bs, c_save + t * plane, h_save + (t + 1) * plane,
                     c_save + (t + 1) * plane, gact + t * plane4, tanh_c + t * plane, B, H};
      HSL_CHECK((launch_gemm<CfgStep, false, true, EpiCellFwd, false, kStepDepth>(ga, 1, epi, s)));
    } else {
      EpiPartial epi{w.part, B, 4 * H};
      HSL_CHECK((launch_gemm<CfgStep, false, true, EpiPartial, false, kStepDepth>(ga, nsp, epi, s)));
      hipLaunchKernelGGL(step_cell_fwd_kernel, dim3(grid_for(plane)), dim3(256), 0, s, w.part, nsp,
                         w.gih + t * plane4, w.bs, c_save + t * plane, h_save + (t + 1) * plane,
                         c_save + (t + 1) * plane, gact + t * plane4, tanh_c + t * plane, B, H);
      HSL_HIP(hipGetLastError());
    }
  }
  timing_end(slot, s);
  note_recurrent_path(1);
  return HSL_OK;
}

int hsl_rec_fwd_noalloc(const float* x, const float* h0, const float* c0, const float* w_ih, const float* w_hh,
                        const float* b_ih, const float* b_hh, const float* a, float* h_save, float* c_save,
                        float* gact, float* tanh_c, int T, int B, int D, int H, void* stream) {
  HSL_CHECK(check_dims(T, B, D, H));
  if (B == 0 || H == 0) return HSL_OK;
  PersistentPlan pl;
  HSL_CHECK(plan_persistent(B, H, D, false, &pl));
  WidePlan wp;
  if (!pl.ok) HSL_CHECK(plan_wide(B, H, false, &wp));
  const bool x_aligned = reinterpret_cast<uintptr_t>(x) % 16 == 0;
  if (pl.XP && !x_aligned) pl.XP = false;
  FwdWs w;
  const size_t need = carve_fwd(nullptr, 0, T, B, H, fwd_needs(pl, wp, x_aligned), &w);
  if (need > kNoAllocScratchBytes)
    return fail(HSL_ERR_UNSUPPORTED,
                "hsl_rec_fwd_noalloc: T=%d B=%d D=%d H=%d needs %zu bytes of scratch, more than the %zu bytes of "
                "its static scratch buffer (the persistent path with the input projection fused -- H <= 512, "
                "D <= 256, D %% 4 == 0, 16-byte aligned x -- needs well under 1 MiB); call hsl_rec_fwd with a "
                "workspace instead",
                T, B, D, H, need, kNoAllocScratchBytes);
  void* ws = nullptr;
  HSL_CHECK(scratch_address(&ws));
  TimingSuppress no_events;
  return hsl_rec_fwd(x, h0, c0, w_ih, w_hh, b_ih, b_hh, a, h_save, c_save, gact, tanh_c, ws, kNoAllocScratchBytes, T,
                     B, D, H, stream);
}

size_t hsl_rec_bwd_ws_bytes_for(int T, int B, int D, int H, int with_dx) {
  if (T < 0 || B < 0 || D < 0 || H < 0) return 0;
  BwdWs w;
  BwdNeeds nd;  // every part when the path cannot be planned (no device)
  PersistentPlan pl;
  WidePlan wp;
  if (B > 0 && H > 0 && plan_persistent(B, H, D, true, &pl) == HSL_OK && plan_wide(B, H, true, &wp) == HSL_OK)
    nd = bwd_needs(pl, wp, with_dx != 0);
  return carve_bwd(nullptr, 0, T, B, D, H, nd, &w);
}

size_t hsl_rec_bwd_ws_bytes(int T, int B, int D, int H) { return hsl_rec_bwd_ws_bytes_for(T, B, D, H, 1); }

int hsl_rec_bwd(const float* dout, const float* dh_n, const float* dc_n, const float* x, const float* h_save,
                const float* c_save, const float* gact, const float* tanh_c, const float* w_ih, const float* w_hh,
                const float* b_hh, const float* a, float* dx, float* dw_ih, float* dw_hh, float* db_ih, float* db_hh,
                float* da, float* dh0, float* dc0, void* ws, size_t ws_bytes, int T, int B, int D, int H,
                void* stream) {
  HSL_CHECK(check_dims(T, B, D, H));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (!dw_ih || !dw_hh || !db_ih || !db_hh || !da || !w_ih || !w_hh || !b_hh || !a)
    return fail(HSL_ERR_ARG, "hsl_rec_bwd: null pointer");
  if (T > 0 && B > 0 && H > 0 && (!dout || !x || !h_save || !c_save || !gact || !tanh_c))
    return fail(HSL_ERR_ARG, "hsl_rec_bwd: null pointer");
  PersistentPlan pl;
  WidePlan wp;
  if (T > 0 && B > 0 && H > 0) HSL_CHECK(plan_persistent(B, H, D, true, &pl));
  if (T > 0 && B > 0 && H > 0 && !pl.ok) HSL_CHECK(plan_wide(B, H, true, &wp));
  if (T > 0 && B > 0 && H > 0 && recurrent_path_mode() == 2 && !pl.ok && !wp.ok)
    return fail(HSL_ERR_UNSUPPORTED, "persistent path does not fit (B=%d H=%d)", B, H);
  BwdWs w;
  const size_t need = carve_bwd(ws, ws_bytes, T, B, D, H, bwd_needs(pl, wp, dx != nullptr), &w);
  if (!ws || ws_bytes < need) return fail(HSL_ERR_ARG, "hsl_rec_bwd: workspace %zu bytes, need %zu", ws_bytes, need);
  const int TB = T * B;
  const size_t plane = (size_t)B * H, plane4 = (size_t)B * 4 * H;
  if (T == 0 || B == 0 || H == 0) {  // no time steps: all gradients are zero except the carries
    HSL_CHECK(zero_words(reinterpret_cast<unsigned long long*>(w.err), 32, s));
    HSL_CHECK(copy_f32(dw_ih, nullptr, (size_t)4 * H * D, s));
    HSL_CHECK(copy_f32(dw_hh, nullptr, (size_t)4 * H * H, s));
    HSL_CHECK(copy_f32(db_ih, nullptr, (size_t)4 * H, s));
    HSL_CHECK(copy_f32(db_hh, nullptr, (size_t)4 * H, s));
    HSL_CHECK(copy_f32(da, nullptr, 4, s));
    if (dh0) HSL_CHECK(copy_f32(dh0, dh_n, plane, s));
    if (dc0) HSL_CHECK(copy_f32(dc0, dc_n, plane, s));
    return HSL_OK;
  }

  // fused weight gradients: fp32 partial planes [nsplit][4H][H] and [nsplit][4H][D]
  // (the GEMM region, which the GEMMs below only use after these planes are reduced)
  const bool fused = pl.ok && pl.XT >= 0;
  const bool fused_ih = fused && pl.XT > 0;
  int wts = T, nsplit = 0;
  float* const wph = w.gemm;
  float* wpx = nullptr;
  if (fused) {
    const int nch = wgrad_chunks(T, pl.WS);
    wts = ((T + nch - 1) / nch + 7) / 8 * 8;  // whole 8-step windows per plane
    nsplit = (T + wts - 1) / wts * pl.NG;
    wpx = wph + (size_t)nsplit * 4 * H * H;
  }
  if (pl.ok)
    HSL_CHECK(prepare_persistent(w.err, w.pbuf, w.pfloats, w.hello, w.hwords, s));
  else if (wp.ok)
    HSL_CHECK(prepare_persistent(w.err, w.wbuf, w.wfloats, w.whello, kWideWgs, s));
  else
    HSL_CHECK(zero_words(reinterpret_cast<unsigned long long*>(w.err), 32, s));
  if (pl.ok) {
    PBwdArgs pa{dout, dh_n, dc_n, c_save, gact, tanh_c, w_hh, a, w.dgates, w.db_part, dh0, dc0, w.pbuf, w.hello,
                w.err, T, B, H, pl.Hp, pl.NG, pl.NGX, pl.Bg, pl.NW, exchange_scope_mode(), spin_timeout_ticks(),
                h_save, x, wph, fused_ih ? wpx : nullptr, D, wts,
                // dgates feed the GEMMs for whatever the kernel does not produce itself
                (!fused_ih || dx != nullptr) ? 1 : 0};
    const int slot = timing_begin(kTimeRecBwd, s);
    switch (pl.KQ) {
      case 16: launch_bwd_persistent<16>(pa, pl.grid, pl.XT, pl.WS, s); break;
      case 32: launch_bwd_persistent<32>(pa, pl.grid, pl.XT, pl.WS, s); break;
      case 64: launch_bwd_persistent<64>(pa, pl.grid, pl.XT, pl.WS, s); break;
      default: launch_bwd_persistent<128>(pa, pl.grid, pl.XT, pl.WS, s); break;
    }
    HSL_HIP(hipGetLastError());
    timing_end(slot, s);
    note_recurrent_path(2);
    note_backward_fused(fused_ih ? 2 : fused ? 1 : 0);
  } else if (wp.ok) {
    note_backward_fused(0);
    WBwdArgs wa{dout, dh_n, dc_n, c_save, gact, tanh_c, w_hh, a, w.dgates, w.db_part, dh0, dc0, w.wbuf,
                w.wbuf + wide_bwd_bfloats(wp.U), w.whello, w.err, T, B, H,
                exchange_scope_mode(), spin_timeout_ticks()};
    const int slot = timing_begin(kTimeRecBwd, s);
    if (wp.U == 64)
      hipLaunchKernelGGL(rec_bwd_wide<64>, dim3(kWideWgs), dim3(256), wide_bwd_lds<64>(), s, wa);
    else
      hipLaunchKernelGGL(rec_bwd_wide1<32>, dim3(kWideWgs), dim3(256), wide_bwd_lds<32>(), s, wa);
    HSL_HIP(hipGetLastError());
    timing_end(slot, s);
    note_recurrent_path(3);
  } else {
    note_backward_fused(0);
    hipLaunchKernelGGL(scale_whh_kernel, dim3(grid_for((size_t)4 * H * H)), dim3(256), 0, s, w_hh, b_hh, a, w.w_s,
                       (float*)nullptr, (float*)nullptr, H);
    HSL_HIP(hipGetLastError());
    HSL_CHECK(copy_f32(w.dc, dc_n, plane, s));
    int kps;
    const int nsp = step_splits(B, H, 4 * H, &kps);
    const int slot = timing_begin(kTimeStepBwd, s);
    for (int t = T - 1; t >= 0; --t) {
      GemmArgs ga{};
      ga.A = w.dgates + (size_t)(t + 1) * plane4;
      ga.B = w.w_s;
      ga.M = B;
      ga.N = H;
      ga.K = (t == T - 1) ? 0 : 4 * H;
      ga.lda = 4 * H;
      ga.ldb = H;
      ga.vec_a = aligned16(ga.A);
      ga.vec_b = aligned16(ga.B) && H % 4 == 0;
      if (nsp == 1) {
        EpiCellBwd epi{dout + t * plane, t == T - 1 ? dh_n : nullptr, c_save + t * plane, gact + t * plane4,
                       tanh_c + t * plane, w.dc, w.dgates + t * plane4, B, H};
        HSL_CHECK((launch_gemm<CfgStep, false, false, EpiCellBwd, false, kStepDepth>(ga, 1, epi, s)));
      } else {
        // the last step has no dgates_{t+1}: no product, zero planes summed
        if (ga.K > 0) {
          EpiPartial epi{w.part, B, H};
          HSL_CHECK((launch_gemm<CfgStep, false, false, EpiPartial, false, kStepDepth>(ga, nsp, epi, s)));
        }
        hipLaunchKernelGGL(step_cell_bwd_kernel, dim3(grid_for(plane)), dim3(256), 0, s, w.part,
                           ga.K > 0 ? nsp : 0, t == T - 1 ? dh_n : nullptr, dout + t * plane, c_save + t * plane,
                           gact + t * plane4, tanh_c + t * plane, w.dc, w.dgates + t * plane4, B, H);
        HSL_HIP(hipGetLastError());
      }
    }
    timing_end(slot, s);
    if (dh0) {
      GemmDesc gd{w.dgates, w.w_s, nullptr, dh0, B, H, 4 * H, 4 * H, H, H, 0, 0, 1};
      HSL_CHECK(gemm_run(gd, w.gemm, w.gemm_bytes, s));
    }
    if (dc0) HSL_CHECK(copy_f32(dc0, w.dc, plane, s));
    hipLaunchKernelGGL(colsum_time_kernel, dim3(grid_for(plane4)), dim3(256), 0, s, w.dgates, w.db_part, T,
                       (int)plane4);
    HSL_HIP(hipGetLastError());
    note_recurrent_path(1);
  }

  // dW_hh_s = dg^T h_prev (staged partials), then dW_hh = a dW_hh_s and the da row sums.
  // A one-split product does the second part in its own epilogue (dot_parts > 0).
  int splits = nsplit, dot_parts = 0;
  if (!fused)
    HSL_CHECK(gemm_x6_wgrad_fin(w.dgates, h_save, dw_hh, a, H, w_hh, w.rowdot, (size_t)4 * H, 4 * H, H, TB, 4 * H, H,
                                H, s, &dot_parts));
  if (!fused && !dot_parts) {
    GemmDesc g4{w.dgates, h_save, nullptr, w.gemm, 4 * H, H, TB, 4 * H, H, H, 1, 0, 1};
    // as many planes as asked for and as the region holds (the mode may have changed
    // since the workspace was sized)
    const int fit = (int)std::min<size_t>(w.gemm_bytes / (sizeof(float) * (size_t)4 * H * H), 1 << 20);
    HSL_CHECK(gemm_partials(g4, w.gemm, std::max(1, std::min(gemm_tn_planes(4 * H, H, TB), fit)), s, &splits));
  }
  if (!dot_parts) {  // dW_hh (and the fused dW_ih planes in extra blocks of the same launch)
    const size_t xn = fused_ih ? (size_t)4 * H * D : 0;
    auto al16 = [](const void* ptr) { return reinterpret_cast<uintptr_t>(ptr) % 16 == 0; };
    const bool vec = H % 4 == 0 && al16(wph) && al16(w_hh) && al16(dw_hh) &&
                     (!fused_ih || (al16(wpx) && al16(dw_ih)));
    if (vec) {
      const int xblocks = fused_ih ? grid_for(xn / 4) : 0;
      hipLaunchKernelGGL(whh_grad_finalize4_kernel, dim3(H + xblocks), dim3(256), 0, s,
                         reinterpret_cast<const float4*>(wph), splits, reinterpret_cast<const float4*>(w_hh), a,
                         reinterpret_cast<float4*>(dw_hh), w.rowdot, H, reinterpret_cast<const float4*>(wpx), pl.NG,
                         reinterpret_cast<float4*>(dw_ih), xn / 4);
    } else {
      const int xblocks = fused_ih ? grid_for(xn) : 0;
      hipLaunchKernelGGL(whh_grad_finalize_kernel, dim3(4 * H + xblocks), dim3(256), 0, s, wph, splits, w_hh, a,
                         dw_hh, w.rowdot, H, (const float*)wpx, pl.NG, dw_ih, xn);
    }
    HSL_HIP(hipGetLastError());
  }
  HSL_CHECK(bias_grads_from_parts(w.db_part, B, dot_parts ? nullptr : w.rowdot, b_hh, a, db_ih, db_hh, da, H, s,
                                  dot_parts ? w.rowdot : nullptr, dot_parts));
  // dW_ih = dg^T x ; dx = dg W_ih
  if (D > 0) {
    if (!fused_ih) {
      GemmDesc g5{w.dgates, x, nullptr, dw_ih, 4 * H, D, TB, 4 * H, D, D, 1, 0, 1};
      HSL_CHECK(gemm_run(g5, w.gemm, w.gemm_bytes, s));
    }
    if (dx) {
      GemmDesc g6{w.dgates, w_ih, nullptr, dx, TB, D, 4 * H, 4 * H, D, D, 0, 0, 1};
      HSL_CHECK(gemm_run(g6, w.gemm, w.gemm_bytes, s));
    }
  }
  return HSL_OK;
}

}  // extern "C"
