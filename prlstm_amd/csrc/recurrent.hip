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
//    through tagged 64-bit words (hsl_internal.h), with bounded waits.
//  * per-step (any shape): one fused GEMM+cell kernel per time step.
//
// v_mfma_f32_4x4x1_16b_f32 layout (verified on gfx950): A from lane 4b+i is
// A_b[i][0], B from lane 4b+j is B_b[0][j], result lane 4b+j, reg i holds D_b[i][j].
// With cbsz=4, abid=0 every block uses block 0's A (lanes 0-3).
#include "gemm_core.h"

namespace hsl {

using CfgStep = GemmCfg<32, 32, 32, 1, 1, 4>;

namespace {

constexpr int kUnits = 16;       // hidden units per persistent workgroup
constexpr int kPadLdsBytes = 96 * 1024;  // dynamic LDS that keeps one persistent workgroup per CU

// ---------------------------------------------------------------------------------
// small helper kernels
// ---------------------------------------------------------------------------------
__global__ void zero_u64_kernel(unsigned long long* p, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    p[i] = 0ull;
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
__global__ __launch_bounds__(256) void whh_grad_finalize_kernel(const float* __restrict__ P, int splits,
                                                                const float* __restrict__ w_hh,
                                                                const float* __restrict__ a, float* __restrict__ dw_hh,
                                                                double* __restrict__ rowdot, int H) {
  __shared__ double red[256];
  const int n = blockIdx.x;
  const size_t plane = (size_t)4 * H * H;
  const float ag = a[n / H];
  double acc = 0.0;
  for (int k = threadIdx.x; k < H; k += blockDim.x) {
    const size_t e = (size_t)n * H + k;
    double v = 0.0;
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

// db_ih = db_hh_s = sum_b db_part[b][n]; db_hh = a * db; da[g] = sum_{n in g} rowdot[n] + b_hh[n] db[n].
// One workgroup per gate.
__global__ __launch_bounds__(256) void bias_da_finalize_kernel(const double* __restrict__ db_part, int B,
                                                               const double* __restrict__ rowdot,
                                                               const float* __restrict__ b_hh,
                                                               const float* __restrict__ a, float* __restrict__ db_ih,
                                                               float* __restrict__ db_hh, float* __restrict__ da, int H) {
  __shared__ double red[256];
  const int g = blockIdx.x;
  const float ag = a ? a[g] : 1.0f;
  double acc = 0.0;
  for (int u = threadIdx.x; u < H; u += blockDim.x) {
    const int n = g * H + u;
    double s = 0.0;
    for (int b = 0; b < B; ++b) s += db_part[(size_t)b * 4 * H + n];
    const float db = (float)s;
    if (db_ih) db_ih[n] = db;
    if (db_hh) db_hh[n] = ag * db;
    acc += (rowdot ? rowdot[n] : 0.0) + (b_hh ? (double)b_hh[n] * (double)db : 0.0);
  }
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
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
  float* gact;          // [B,4H] at t
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
        gact[(size_t)b * 4 * H + n] = act[gt];
      }
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
  const float* gact;     // [B,4H] at t
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
      const float* ga = gact + (size_t)b * 4 * H + u;
      float dcv = dc[bu];
      float d[4];
      cell_bwd(dh, dcv, c_prev[bu], ga[0], ga[H], ga[2 * H], ga[3 * H], tanh_c[bu], d);
      dc[bu] = dcv;
#pragma unroll
      for (int gt = 0; gt < 4; ++gt) dg[(size_t)b * 4 * H + gt * H + u] = d[gt];
    }
  }
};

// ---------------------------------------------------------------------------------
// persistent path
// ---------------------------------------------------------------------------------
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
  unsigned long long* xbuf;  // [2][NG][4][Hp]
  int* err;
  int T, B, H, Hp, NG, Bg;
  long long spin;
};

// Waits until every word p[j] (valid[j]) carries `tag`; returns false on timeout.
template <int PER>
__device__ __forceinline__ bool wait_words(const unsigned long long* const (&p)[PER], const bool (&valid)[PER],
                                           unsigned tag, float (&out)[PER], long long spin) {
  bool ok[PER];
  unsigned long long w[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    ok[j] = !valid[j];
    w[j] = 0ull;
  }
  const long long t0 = wall_clock64();
  while (true) {
#pragma unroll
    for (int j = 0; j < PER; ++j)
      if (!ok[j]) w[j] = tag_load(p[j]);
    bool all = true;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      ok[j] = ok[j] || tag_of(w[j]) == tag;
      all = all && ok[j];
    }
    if (all) break;
    if (wall_clock64() - t0 > spin) return false;
    __builtin_amdgcn_s_sleep(1);
  }
#pragma unroll
  for (int j = 0; j < PER; ++j) out[j] = valid[j] ? val_of(w[j]) : 0.f;
  return true;
}

template <int KQ>
__global__ __launch_bounds__(256, 1) void rec_fwd_persistent(PFwdArgs p) {
  constexpr int HP = 4 * KQ;         // padded hidden size
  constexpr int PER = HP / 64;       // exchange words per thread (4*HP / 256)
  __shared__ float hl[4][HP + 4];    // h_{t-1} of the group's batch rows
  __shared__ float red[4][4][64];    // [wave][batch][row] partial products
  __shared__ float act[4][64];       // [batch][row] gate activations
  __shared__ int abort_flag;

  const int T = p.T, B = p.B, H = p.H, NG = p.NG, Bg = p.Bg;
  const int grp = blockIdx.x % NG, wg = blockIdx.x / NG;
  const int tid = threadIdx.x, lane = tid & 63, q = tid >> 6;
  const int gate = lane >> 4, uu = lane & 15, u = wg * kUnits + uu;
  const bool row_ok = u < H;
  const int n = gate * H + u;  // this lane's gate row (same mapping in every phase)

  if (tid == 0) abort_flag = 0;

  // a-scaled W_hh slice: lane = gate row, registers = this wave's quarter of k.
  const float ag = p.a[gate];
  float wreg[KQ];
#pragma unroll
  for (int kk = 0; kk < KQ; ++kk) {
    const int k = q * KQ + kk;
    wreg[kk] = (row_ok && k < H) ? ag * p.w_hh[(size_t)n * H + k] : 0.f;
  }
  const float bs = row_ok ? ag * p.b_hh[n] : 0.f;

  // phase-D thread -> (batch slot q, row lane); cell thread (tid < 64) -> (batch slot, unit)
  const int bd = grp * Bg + q;
  const bool d_ok = row_ok && q < Bg && bd < B;
  const int ci = tid >> 4, cu = wg * kUnits + (tid & 15), cb = grp * Bg + ci;
  const bool c_ok = tid < 64 && ci < Bg && cb < B && cu < H;
  float c_reg = 0.f;
  if (c_ok) {
    const size_t bu = (size_t)cb * H + cu;
    c_reg = p.c0[bu];
    p.h_save[bu] = p.h0[bu];
    p.c_save[bu] = c_reg;
  }

  // exchange words this thread gathers each step: (batch slot, k)
  const unsigned long long* wp[PER];
  bool wv[PER];
  int wi[PER], wk[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int idx = tid + 256 * j;
    wi[j] = idx / HP;
    wk[j] = idx % HP;
    const int b = grp * Bg + wi[j];
    wv[j] = wi[j] < Bg && b < B && wk[j] < H;
    wp[j] = nullptr;
  }
  __syncthreads();

  for (int t = 0; t < T; ++t) {
    // this step's input-gate value for phase D (independent of h: issue early)
    const float gi = d_ok ? p.gih[((size_t)t * B + bd) * 4 * H + n] : 0.f;

    // ---- gather h_{t-1} -------------------------------------------------------------
    if (t == 0) {
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        const int b = grp * Bg + wi[j];
        hl[wi[j]][wk[j]] = wv[j] ? p.h0[(size_t)b * H + wk[j]] : 0.f;
      }
    } else {
      const int slot = (t - 1) & 1;
#pragma unroll
      for (int j = 0; j < PER; ++j)
        wp[j] = p.xbuf + (((size_t)slot * NG + grp) * 4 + wi[j]) * HP + wk[j];
      float v[PER];
      if (!wait_words<PER>(wp, wv, (unsigned)t, v, p.spin)) {
        abort_flag = 1;
        atomicOr(p.err, 1);
      }
#pragma unroll
      for (int j = 0; j < PER; ++j) hl[wi[j]][wk[j]] = v[j];
    }
    __syncthreads();
    if (abort_flag) return;

    // ---- z-partials: 4 batch rows x 64 gate rows over this wave's k quarter ------------
    f4 acc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = f4{0.f, 0.f, 0.f, 0.f};
    const float* hrow = &hl[lane & 3][q * KQ];
#pragma unroll
    for (int kk = 0; kk < KQ; kk += 4) {
      const f4 hv = *reinterpret_cast<const f4*>(hrow + kk);
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[c] = __builtin_amdgcn_mfma_f32_4x4x1f32(hv[c], wreg[kk + c], acc[c], 4, 0, 0);
    }
    const f4 zs = (acc[0] + acc[1]) + (acc[2] + acc[3]);
#pragma unroll
    for (int i = 0; i < 4; ++i) red[q][i][lane] = zs[i];
    __syncthreads();

    // ---- activations: thread (batch slot q, row lane) ------------------------------
    {
      const float mm = (red[0][q][lane] + red[1][q][lane]) + (red[2][q][lane] + red[3][q][lane]);
      const float z = (gi + mm) + bs;
      const float s = sigmoid_f(z);
      act[q][lane] = s;
      if (d_ok) p.gact[((size_t)t * B + bd) * 4 * H + n] = s;
    }
    __syncthreads();

    // ---- cell update + publish h_t --------------------------------------------------
    if (c_ok) {
      const int cuu = tid & 15;
      const float ig = act[ci][cuu], fg = act[ci][16 + cuu], gg = act[ci][32 + cuu], og = act[ci][48 + cuu];
      const float c = fg * c_reg + ig * gg;
      const float tc = tanh_f(c);
      const float h = og * tc;
      c_reg = c;
      tag_store(p.xbuf + (((size_t)(t & 1) * NG + grp) * 4 + ci) * HP + cu, h, (unsigned)(t + 1));
      const size_t bu = (size_t)cb * H + cu;
      const size_t plane = (size_t)B * H;
      p.h_save[(size_t)(t + 1) * plane + bu] = h;
      p.c_save[(size_t)(t + 1) * plane + bu] = c;
      p.tanh_c[(size_t)t * plane + bu] = tc;
    }
  }
}

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
  unsigned long long* pbuf;  // [2][NG][NW][4][Hp]
  int* err;
  int T, B, H, Hp, NG, Bg, NW;
  long long spin;
};

template <int KQ>
__global__ __launch_bounds__(256, 1) void rec_bwd_persistent(PBwdArgs p) {
  constexpr int HP = 4 * KQ;
  constexpr int CG = (KQ + 63) / 64;     // 64-column groups per wave
  constexpr int NWMAX = HP / kUnits;     // workgroups per group at most
  constexpr int PER = NWMAX * 64 / 256;  // exchange words per thread
  static_assert(PER >= 1, "at least one word per thread");
  __shared__ float dgl[4][64 + 4];       // this step's dgates of the 64 rows, per batch slot
  __shared__ float prl[NWMAX][4][kUnits];
  __shared__ int abort_flag;

  const int T = p.T, B = p.B, H = p.H, NG = p.NG, Bg = p.Bg, NW = p.NW;
  const int grp = blockIdx.x % NG, wg = blockIdx.x / NG;
  const int tid = threadIdx.x, lane = tid & 63, q = tid >> 6;
  if (tid == 0) abort_flag = 0;

  // W_s columns owned by this lane: col = q*KQ + cg*64 + lane; registers over the 64 rows.
  float wreg[CG][64];
  int col[CG];
  bool col_ok[CG];
#pragma unroll
  for (int cg = 0; cg < CG; ++cg) {
    const int cl = cg * 64 + lane;
    col[cg] = q * KQ + cl;
    col_ok[cg] = cl < KQ && col[cg] < H;
#pragma unroll
    for (int r = 0; r < 64; ++r) {
      const int gt = r >> 4, u = wg * kUnits + (r & 15);
      wreg[cg][r] = (col_ok[cg] && u < H) ? p.a[gt] * p.w_hh[(size_t)(gt * H + u) * H + col[cg]] : 0.f;
    }
  }

  // cell thread (tid < 64) -> (batch slot ci, unit cu)
  const int ci = tid >> 4, cuu = tid & 15, cu = wg * kUnits + cuu, cb = grp * Bg + ci;
  const bool c_ok = tid < 64 && ci < Bg && cb < B && cu < H;
  float dc = 0.f;
  double dbacc[4] = {0.0, 0.0, 0.0, 0.0};
  if (c_ok) dc = p.dc_n[(size_t)cb * H + cu];

  // exchange words gathered each step: (source workgroup, batch slot, unit)
  const unsigned long long* wp[PER];
  bool wv[PER];
  int ws_[PER], wi[PER], wu[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int idx = tid + 256 * j;
    ws_[j] = idx / 64;
    wi[j] = (idx / kUnits) % 4;
    wu[j] = idx % kUnits;
    const int b = grp * Bg + wi[j], u = wg * kUnits + wu[j];
    wv[j] = ws_[j] < NW && wi[j] < Bg && b < B && u < H;
    wp[j] = nullptr;
  }
  __syncthreads();

  const size_t plane = (size_t)B * H;
  for (int s = 0; s <= T; ++s) {
    const int t = T - 1 - s;
    // prefetch this step's saved values (cell threads)
    float dout_v = 0.f, cp = 0.f, ig = 0.f, fg = 0.f, gg = 0.f, og = 0.f, tc = 0.f;
    if (c_ok && s < T) {
      const size_t bu = (size_t)cb * H + cu;
      dout_v = p.dout[(size_t)t * plane + bu];
      cp = p.c_save[(size_t)t * plane + bu];
      tc = p.tanh_c[(size_t)t * plane + bu];
      const float* ga = p.gact + ((size_t)t * B + cb) * 4 * H + cu;
      ig = ga[0];
      fg = ga[H];
      gg = ga[2 * H];
      og = ga[3 * H];
    }

    // ---- dh for this step: dh_n, or the sum of the partials published last step ------
    float dh = 0.f;
    if (s == 0) {
      if (c_ok) dh = p.dh_n[(size_t)cb * H + cu];
    } else {
      const int slot = (s - 1) & 1;
#pragma unroll
      for (int j = 0; j < PER; ++j)
        wp[j] = p.pbuf + ((((size_t)slot * NG + grp) * NWMAX + ws_[j]) * 4 + wi[j]) * HP + wg * kUnits + wu[j];
      float v[PER];
      if (!wait_words<PER>(wp, wv, (unsigned)s, v, p.spin)) {
        abort_flag = 1;
        atomicOr(p.err, 1);
      }
#pragma unroll
      for (int j = 0; j < PER; ++j)
        if (ws_[j] < NWMAX) prl[ws_[j]][wi[j]][wu[j]] = v[j];
      __syncthreads();
      if (abort_flag) return;
      if (c_ok) {
        for (int w = 0; w < NW; ++w) dh += prl[w][ci][cuu];
      }
    }
    if (s == T) {  // dh is now the gradient w.r.t. h0
      if (c_ok) {
        const size_t bu = (size_t)cb * H + cu;
        if (p.dh0) p.dh0[bu] = dh;
        if (p.dc0) p.dc0[bu] = dc;
#pragma unroll
        for (int gt = 0; gt < 4; ++gt) p.db_part[(size_t)cb * 4 * H + gt * H + cu] = dbacc[gt];
      }
      return;
    }

    // ---- cell backward -----------------------------------------------------------
    if (tid < 64) {
      float d[4] = {0.f, 0.f, 0.f, 0.f};
      if (c_ok) {
        dh = dh + dout_v;
        cell_bwd(dh, dc, cp, ig, fg, gg, og, tc, d);
        float* dgp = p.dgates + ((size_t)t * B + cb) * 4 * H + cu;
#pragma unroll
        for (int gt = 0; gt < 4; ++gt) {
          dgp[gt * H] = d[gt];
          dbacc[gt] += (double)d[gt];
        }
      }
#pragma unroll
      for (int gt = 0; gt < 4; ++gt) dgl[ci][gt * 16 + cuu] = d[gt];
    }
    __syncthreads();

    // ---- partial dh_{t-1}[batch][col] = sum over this workgroup's 64 rows -----------
    const float* drow = &dgl[lane & 3][0];
#pragma unroll
    for (int cg = 0; cg < CG; ++cg) {
      f4 acc[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[c] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int r = 0; r < 64; r += 4) {
        const f4 dv = *reinterpret_cast<const f4*>(drow + r);
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[c] = __builtin_amdgcn_mfma_f32_4x4x1f32(dv[c], wreg[cg][r + c], acc[c], 4, 0, 0);
      }
      const f4 part = (acc[0] + acc[1]) + (acc[2] + acc[3]);
      if (col_ok[cg]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (i < Bg && grp * Bg + i < B)
            tag_store(p.pbuf + ((((size_t)(s & 1) * NG + grp) * NWMAX + wg) * 4 + i) * HP + col[cg], part[i],
                      (unsigned)(s + 1));
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------------
struct PersistentPlan {
  bool ok = false;
  int KQ = 0, Hp = 0, NG = 0, Bg = 0, NW = 0, grid = 0;
};

int pick_kq(int H) {
  if (H <= 64) return 16;
  if (H <= 128) return 32;
  if (H <= 256) return 64;
  if (H <= 512) return 128;
  return 0;
}

template <class K>
int max_resident(K kernel, int* out) {
  int occ = 0;
  HSL_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kernel, 256, kPadLdsBytes));
  *out = occ;
  return HSL_OK;
}

int plan_persistent(int B, int H, bool bwd, PersistentPlan* pl) {
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
  p.NW = (H + kUnits - 1) / kUnits;
  p.grid = p.NG * p.NW;
  int occ = 0;
  switch (kq) {
    case 16: HSL_CHECK(bwd ? max_resident(rec_bwd_persistent<16>, &occ) : max_resident(rec_fwd_persistent<16>, &occ)); break;
    case 32: HSL_CHECK(bwd ? max_resident(rec_bwd_persistent<32>, &occ) : max_resident(rec_fwd_persistent<32>, &occ)); break;
    case 64: HSL_CHECK(bwd ? max_resident(rec_bwd_persistent<64>, &occ) : max_resident(rec_fwd_persistent<64>, &occ)); break;
    default: HSL_CHECK(bwd ? max_resident(rec_bwd_persistent<128>, &occ) : max_resident(rec_fwd_persistent<128>, &occ)); break;
  }
  // every workgroup must be resident at once: the waits are between workgroups
  p.ok = occ >= 1 && (long)occ * di.num_cus >= p.grid;
  *pl = p;
  return HSL_OK;
}

inline int grid_for(size_t n) {
  size_t b = (n + 255) / 256;
  if (b < 1) b = 1;
  if (b > 2048) b = 2048;
  return (int)b;
}

int zero_words_impl(unsigned long long* p, size_t n, hipStream_t s) {
  if (n == 0) return HSL_OK;
  hipLaunchKernelGGL(zero_u64_kernel, dim3(grid_for(n)), dim3(256), 0, s, p, n);
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
  float* gih;                // [T*B*4H]
  unsigned long long* xbuf;  // [2*NG*4*Hp] (persistent)
  float* w_perm;             // [4H*H]      (per-step)
  float* bs;                 // [4H]        (per-step)
  size_t words;
};

size_t carve_fwd(void* ws, size_t cap, int T, int B, int H, FwdWs* o) {
  Carver c(ws, cap);
  o->err = c.take<int>(64);
  o->gih = c.take<float>((size_t)T * B * 4 * H);
  const int kq = pick_kq(H);
  const size_t ng = (size_t)(B + 3) / 4;
  o->words = kq ? 2 * ng * 4 * (size_t)(4 * kq) : 0;
  o->xbuf = c.take<unsigned long long>(o->words);
  o->w_perm = c.take<float>((size_t)4 * H * H);
  o->bs = c.take<float>((size_t)4 * H);
  return c.off;
}

struct BwdWs {
  int* err;
  float* dgates;             // [T*B*4H]
  double* db_part;           // [B*4H]
  double* rowdot;            // [4H]
  float* dc;                 // [B*H]   (per-step)
  float* w_s;                // [4H*H]  (per-step)
  unsigned long long* pbuf;  // [2*NG*NWMAX*4*Hp] (persistent)
  size_t words;
  float* gemm;               // shared by the weight-gradient GEMMs
  size_t gemm_bytes;
};

size_t gemm_region_bytes(int T, int B, int D, int H) {
  const int TB = T * B;
  const int s4 = gemm_pick_splits(4 * H, H, TB, 1);
  size_t need = sizeof(float) * (size_t)s4 * 4 * H * H;  // dW_hh partials (always staged)
  const size_t g5 = gemm_ws_bytes(4 * H, D, TB, 1);
  const size_t g6 = gemm_ws_bytes(TB, D, 4 * H, 1);
  if (g5 > need) need = g5;
  if (g6 > need) need = g6;
  const size_t g7 = gemm_ws_bytes(B, H, 4 * H, 1);
  if (g7 > need) need = g7;
  return need;
}

size_t carve_bwd(void* ws, size_t cap, int T, int B, int D, int H, BwdWs* o) {
  Carver c(ws, cap);
  o->err = c.take<int>(64);
  o->dgates = c.take<float>((size_t)T * B * 4 * H);
  o->db_part = c.take<double>((size_t)B * 4 * H);
  o->rowdot = c.take<double>((size_t)4 * H);
  o->dc = c.take<float>((size_t)B * H);
  o->w_s = c.take<float>((size_t)4 * H * H);
  const int kq = pick_kq(H);
  const size_t ng = (size_t)(B + 3) / 4;
  o->words = kq ? 2 * ng * (size_t)(4 * kq / kUnits) * 4 * (size_t)(4 * kq) : 0;
  o->pbuf = c.take<unsigned long long>(o->words);
  o->gemm_bytes = gemm_region_bytes(T, B, D, H);
  o->gemm = c.take<float>(o->gemm_bytes / sizeof(float) + 1);
  return c.off;
}

int check_dims(int T, int B, int D, int H) {
  if (T < 0 || B < 0 || D < 0 || H < 0) return fail(HSL_ERR_ARG, "negative dimension (T=%d B=%d D=%d H=%d)", T, B, D, H);
  if ((long long)T * B * 4 * H > (1ll << 40)) return fail(HSL_ERR_UNSUPPORTED, "problem too large");
  if (T >= (1 << 30)) return fail(HSL_ERR_UNSUPPORTED, "T too large");
  return HSL_OK;
}

template <int KQ>
void launch_fwd_persistent(const PFwdArgs& a, int grid, hipStream_t s) {
  hipLaunchKernelGGL(rec_fwd_persistent<KQ>, dim3(grid), dim3(256), kPadLdsBytes, s, a);
}
template <int KQ>
void launch_bwd_persistent(const PBwdArgs& a, int grid, hipStream_t s) {
  hipLaunchKernelGGL(rec_bwd_persistent<KQ>, dim3(grid), dim3(256), kPadLdsBytes, s, a);
}

}  // namespace

int zero_words(unsigned long long* p, size_t n, hipStream_t s) { return zero_words_impl(p, n, s); }
int copy_f32(float* dst, const float* src, size_t n, hipStream_t s) { return copy_f32_impl(dst, src, n, s); }

int bias_grads_from_parts(const double* db_part, int B, const double* rowdot, const float* b_hh, const float* a,
                          float* db_ih, float* db_hh, float* da, int H, hipStream_t s) {
  if (H == 0) return HSL_OK;
  hipLaunchKernelGGL(bias_da_finalize_kernel, dim3(4), dim3(256), 0, s, db_part, B, rowdot, b_hh, a, db_ih, db_hh,
                     da, H);
  HSL_HIP(hipGetLastError());
  return HSL_OK;
}

}  // namespace hsl

using namespace hsl;

extern "C" {

size_t hsl_rec_fwd_ws_bytes(int T, int B, int D, int H) {
  (void)D;
  if (T < 0 || B < 0 || H < 0) return 0;
  FwdWs w;
  return carve_fwd(nullptr, 0, T, B, H, &w);
}

int hsl_rec_fwd(const float* x, const float* h0, const float* c0, const float* w_ih, const float* w_hh,
                const float* b_ih, const float* b_hh, const float* a, float* h_save, float* c_save, float* gact,
                float* tanh_c, void* ws, size_t ws_bytes, int T, int B, int D, int H, void* stream) {
  HSL_CHECK(check_dims(T, B, D, H));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (B == 0 || H == 0) return HSL_OK;
  if (!h0 || !c0 || !w_hh || !b_hh || !a || !h_save || !c_save || (T > 0 && (!x || !w_ih || !b_ih || !gact || !tanh_c)))
    return fail(HSL_ERR_ARG, "hsl_rec_fwd: null pointer");
  FwdWs w;
  const size_t need = carve_fwd(ws, ws_bytes, T, B, H, &w);
  if (!ws || ws_bytes < need) return fail(HSL_ERR_ARG, "hsl_rec_fwd: workspace %zu bytes, need %zu", ws_bytes, need);

  PersistentPlan pl;
  HSL_CHECK(plan_persistent(B, H, false, &pl));
  if (recurrent_path_mode() == 2 && !pl.ok)
    return fail(HSL_ERR_UNSUPPORTED, "persistent path does not fit (B=%d H=%d)", B, H);

  HSL_CHECK(zero_words(reinterpret_cast<unsigned long long*>(w.err), 32, s));
  if (T == 0) {
    HSL_CHECK(copy_f32(h_save, h0, (size_t)B * H, s));
    HSL_CHECK(copy_f32(c_save, c0, (size_t)B * H, s));
    return HSL_OK;
  }
  // input projection for all T at once (_torch.py:96)
  GemmDesc g1{x, w_ih, b_ih, w.gih, T * B, 4 * H, D, D, D, 4 * H, 0, 1};
  const int tslot = timing_begin(kTimeInputProj, s);
  HSL_CHECK(gemm_run(g1, nullptr, 0, s));
  timing_end(tslot, s);

  if (pl.ok) {
    HSL_CHECK(zero_words(w.xbuf, w.words, s));
    PFwdArgs pa{w.gih, w_hh, b_hh, a, h0, c0, h_save, c_save, gact, tanh_c, w.xbuf, w.err,
                T, B, H, pl.Hp, pl.NG, pl.Bg, spin_timeout_ticks()};
    const int slot = timing_begin(kTimeRecFwd, s);
    switch (pl.KQ) {
      case 16: launch_fwd_persistent<16>(pa, pl.grid, s); break;
      case 32: launch_fwd_persistent<32>(pa, pl.grid, s); break;
      case 64: launch_fwd_persistent<64>(pa, pl.grid, s); break;
      default: launch_fwd_persistent<128>(pa, pl.grid, s); break;
    }
    HSL_HIP(hipGetLastError());
    timing_end(slot, s);
    note_recurrent_path(2);
    return HSL_OK;
  }

  // per-step path
  hipLaunchKernelGGL(scale_whh_kernel, dim3(grid_for((size_t)4 * H * H)), dim3(256), 0, s, w_hh, b_hh, a,
                     (float*)nullptr, w.w_perm, w.bs, H);
  HSL_HIP(hipGetLastError());
  HSL_CHECK(copy_f32(h_save, h0, (size_t)B * H, s));
  HSL_CHECK(copy_f32(c_save, c0, (size_t)B * H, s));
  const size_t plane = (size_t)B * H, plane4 = (size_t)B * 4 * H;
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
    EpiCellFwd epi{w.gih + t * plane4, w.bs, c_save + t * plane, h_save + (t + 1) * plane, c_save + (t + 1) * plane,
                   gact + t * plane4, tanh_c + t * plane, B, H};
    HSL_CHECK((launch_gemm<CfgStep, false, true>(ga, 1, epi, s)));
  }
  timing_end(slot, s);
  note_recurrent_path(1);
  return HSL_OK;
}

size_t hsl_rec_bwd_ws_bytes(int T, int B, int D, int H) {
  if (T < 0 || B < 0 || D < 0 || H < 0) return 0;
  BwdWs w;
  return carve_bwd(nullptr, 0, T, B, D, H, &w);
}

int hsl_rec_bwd(const float* dout, const float* dh_n, const float* dc_n, const float* x, const float* h_save,
                const float* c_save, const float* gact, const float* tanh_c, const float* w_ih, const float* w_hh,
                const float* b_hh, const float* a, float* dx, float* dw_ih, float* dw_hh, float* db_ih, float* db_hh,
                float* da, float* dh0, float* dc0, void* ws, size_t ws_bytes, int T, int B, int D, int H,
                void* stream) {
  HSL_CHECK(check_dims(T, B, D, H));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (!dw_ih || !dw_hh || !db_ih || !db_hh || !da || !w_ih || !w_hh || !b_hh || !a)
    return fail(HSL_ERR_ARG, "hsl_rec_bwd: null pointer");
  if (T > 0 && B > 0 && H > 0 && (!dout || !dh_n || !dc_n || !x || !h_save || !c_save || !gact || !tanh_c))
    return fail(HSL_ERR_ARG, "hsl_rec_bwd: null pointer");
  BwdWs w;
  const size_t need = carve_bwd(ws, ws_bytes, T, B, D, H, &w);
  if (!ws || ws_bytes < need) return fail(HSL_ERR_ARG, "hsl_rec_bwd: workspace %zu bytes, need %zu", ws_bytes, need);
  HSL_CHECK(zero_words(reinterpret_cast<unsigned long long*>(w.err), 32, s));

  const int TB = T * B;
  const size_t plane = (size_t)B * H, plane4 = (size_t)B * 4 * H;
  if (T == 0 || B == 0 || H == 0) {  // no time steps: all gradients are zero except the carries
    HSL_CHECK(copy_f32(dw_ih, nullptr, (size_t)4 * H * D, s));
    HSL_CHECK(copy_f32(dw_hh, nullptr, (size_t)4 * H * H, s));
    HSL_CHECK(copy_f32(db_ih, nullptr, (size_t)4 * H, s));
    HSL_CHECK(copy_f32(db_hh, nullptr, (size_t)4 * H, s));
    HSL_CHECK(copy_f32(da, nullptr, 4, s));
    if (dh0) HSL_CHECK(copy_f32(dh0, dh_n, plane, s));
    if (dc0) HSL_CHECK(copy_f32(dc0, dc_n, plane, s));
    return HSL_OK;
  }

  PersistentPlan pl;
  HSL_CHECK(plan_persistent(B, H, true, &pl));
  if (recurrent_path_mode() == 2 && !pl.ok)
    return fail(HSL_ERR_UNSUPPORTED, "persistent path does not fit (B=%d H=%d)", B, H);

  if (pl.ok) {
    HSL_CHECK(zero_words(w.pbuf, w.words, s));
    PBwdArgs pa{dout, dh_n, dc_n, c_save, gact, tanh_c, w_hh, a, w.dgates, w.db_part, dh0, dc0, w.pbuf, w.err,
                T, B, H, pl.Hp, pl.NG, pl.Bg, pl.NW, spin_timeout_ticks()};
    const int slot = timing_begin(kTimeRecBwd, s);
    switch (pl.KQ) {
      case 16: launch_bwd_persistent<16>(pa, pl.grid, s); break;
      case 32: launch_bwd_persistent<32>(pa, pl.grid, s); break;
      case 64: launch_bwd_persistent<64>(pa, pl.grid, s); break;
      default: launch_bwd_persistent<128>(pa, pl.grid, s); break;
    }
    HSL_HIP(hipGetLastError());
    timing_end(slot, s);
    note_recurrent_path(2);
  } else {
    hipLaunchKernelGGL(scale_whh_kernel, dim3(grid_for((size_t)4 * H * H)), dim3(256), 0, s, w_hh, b_hh, a, w.w_s,
                       (float*)nullptr, (float*)nullptr, H);
    HSL_HIP(hipGetLastError());
    HSL_CHECK(copy_f32(w.dc, dc_n, plane, s));
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
      EpiCellBwd epi{dout + t * plane, t == T - 1 ? dh_n : nullptr, c_save + t * plane, gact + t * plane4,
                     tanh_c + t * plane, w.dc, w.dgates + t * plane4, B, H};
      HSL_CHECK((launch_gemm<CfgStep, false, false>(ga, 1, epi, s)));
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

  // dW_hh_s = dg^T h_prev (staged partials), then dW_hh = a dW_hh_s and the da row sums
  int splits = 1;
  {
    GemmDesc g4{w.dgates, h_save, nullptr, w.gemm, 4 * H, H, TB, 4 * H, H, H, 1, 0, 1};
    HSL_CHECK(gemm_partials(g4, w.gemm, gemm_pick_splits(4 * H, H, TB, 1), s, &splits));
  }
  hipLaunchKernelGGL(whh_grad_finalize_kernel, dim3(4 * H), dim3(256), 0, s, w.gemm, splits, w_hh, a, dw_hh,
                     w.rowdot, H);
  HSL_HIP(hipGetLastError());
  HSL_CHECK(bias_grads_from_parts(w.db_part, B, w.rowdot, b_hh, a, db_ih, db_hh, da, H, s));
  // dW_ih = dg^T x ; dx = dg W_ih
  if (D > 0) {
    GemmDesc g5{w.dgates, x, nullptr, dw_ih, 4 * H, D, TB, 4 * H, D, D, 1, 0, 1};
    HSL_CHECK(gemm_run(g5, w.gemm, w.gemm_bytes, s));
    if (dx) {
      GemmDesc g6{w.dgates, w_ih, nullptr, dx, TB, D, 4 * H, 4 * H, D, D, 0, 0, 1};
      HSL_CHECK(gemm_run(g6, w.gemm, w.gemm_bytes, s));
    }
  }
  return HSL_OK;
}

}  // extern "C"
