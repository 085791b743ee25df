// Parallel (scan) mode of HeadStartLSTM: forward scan, hand-written backward scan and
// the parallel-mode entry points.
//
// Reference behaviour (src/headstartlstm/_parallel.py:21-74):
//   gates = x W_ih^T + b_ih;  i,f,g,o = sigmoid(gates);  b = i*g
//   c_t = exp(a*_t + logcumsumexp([log max(c0,eps), log max(b,eps) - a*])_t),
//   a*_t = cumsum(log max(f,eps))
//   out = o * tanh(c);  h_n = out[T-1];  c_n = c[T-1]
// The log-domain expression is the closed form of the first-order linear recurrence
//   c_t = f~_t c_{t-1} + b~_t,   f~ = max(f,eps), b~ = max(i g, eps), c_{-1} = max(c0,eps)
// (all coefficients positive).  Here it is evaluated as a scan of the affine maps
// c -> f~ c + b~ in the linear domain: f~, b~ lie in [eps, 1), so nothing overflows,
// a running product that underflows is the exact fp32 limit, and every term is
// positive, so composing maps never cancels.  The backward is the mirror reverse
// scan G_t = e_t + f~_{t+1} G_{t+1} of the total gradient G_t = dL/dc_t; the clamps
// pass gradient where their input is >= eps (torch's clamp_min rule).
//
// Layout: gates [T,B,4H] (the GEMM output, never transposed), out [T,B,H].  One
// workgroup owns 64 consecutive channels (b,j) = one wave-width, so every load and
// store is a 256-byte row segment, and walks all of T in chunks of NW*L steps: each
// of the NW waves takes L consecutive steps, composes them into one map, the maps
// are combined through LDS, and each wave re-runs its steps from its carry-in.  The
// next chunk's loads are issued before the current chunk is processed.  Every [T,...]
// stream is read or written once, with non-temporal accesses (the streams bypass the
// caches' retention; measured 9% faster forward on MI355X).
//
// The cell state is not stored per step.  The forward writes c_ck [ceil(T/8)+1, B, H]:
// row m is the state carried into step 8m (row 0 = max(c0, eps)), i.e. the carry-in from
// which the wave holding steps 8m .. 8m+7 runs them, and the last row is c_{T-1} = c_n.
// The backward's waves hold the same 8-step groups and re-run c_t from the row with the
// forward's own operations, so its c_t equal the forward's bit for bit, and the scans move
// 20.5 + 36.5 bytes per element instead of 24 + 40.
//
// The streams are raw buffer accesses with a uniform base per time step (no 64-bit
// address arithmetic per lane; the kernels then run at the HBM rate this access pattern
// sustains, about 5.3 TB/s, with their arithmetic off the critical path): rows past T are
// given size 0 and lanes past the last channel an out-of-range offset, which reads 0 and
// drops stores, so no lane computes a 64-bit address or branches around an access.
// Chunks alternate between two register sets, and only the chunk that holds step T-1
// carries the end-of-sequence conditions.
#include <algorithm>
#include <type_traits>

#include "hsl_internal.h"

namespace hsl {
namespace {

// Element formats of the out / dout streams: fp32, or the 16-bit format of a half module's
// output (bf16, fp16), converted with round-to-nearest-even as torch's .to() does.
enum StreamFmt { kF32 = 0, kBf16 = 1, kF16 = 2 };
template <int F>
constexpr unsigned fmt_bytes() {
  return F == kF32 ? 4u : 2u;
}
template <int F>
__device__ __forceinline__ void out_store(float v, __amdgpu_buffer_rsrc_t r, unsigned voff) {
  if constexpr (F == kF32) {
    row_store_nt(v, r, voff, 0);
  } else {
    // v is first rounded to fp32 (kept from fusing into a mixed-precision multiply that
    // would round the product to 16 bits once), so the result is the fp32 value's
    // conversion, as torch's .to() of the fp32 output gives
    asm volatile("" : "+v"(v));
    unsigned short u;
    if constexpr (F == kBf16)
      u = __builtin_bit_cast(unsigned short, (__bf16)v);
    else
      u = __builtin_bit_cast(unsigned short, (_Float16)v);
    __builtin_amdgcn_raw_buffer_store_b16(u, r, (int)voff, 0, kCpolNt);
  }
}
template <int F>
__device__ __forceinline__ float in_load(__amdgpu_buffer_rsrc_t r, unsigned voff, int soff) {
  if constexpr (F == kF32) {
    return row_load(r, voff, soff);
  } else {
    const unsigned short u = __builtin_amdgcn_raw_buffer_load_b16(r, (int)voff, soff, kCpolNt);
    if constexpr (F == kBf16)
      return __uint_as_float((unsigned)u << 16);
    else
      return (float)__builtin_bit_cast(_Float16, u);
  }
}

constexpr int kFwdWaves = 16, kFwdSteps = 8;
constexpr int kBwdWaves = 8, kBwdSteps = 8;
constexpr int kCkSteps = 8;  // steps per checkpoint row of c (one wave's group in both scans)

template <int NW, int L, int OF>
__global__ __launch_bounds__(NW * 64) void scan_fwd_kernel(const float* __restrict__ gates, const float* __restrict__ c0,
                                                          float eps, void* __restrict__ out, float* __restrict__ cck,
                                                          int T, int B, int H) {
  static_assert(L == kCkSteps, "checkpoint rows are one per L-step group");
  __shared__ float2 sAV[NW][64];  // each wave's composed map (A, V) of the chunk
  __shared__ float sC[64];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int C = B * H;
  const int ch = blockIdx.x * 64 + lane;
  const bool ok = ch < C;
  const int b = ok ? ch / H : 0, j = ok ? ch % H : 0;
  const size_t gstride = (size_t)B * 4 * H, ostride = (size_t)C;  // per time step
  const unsigned grow = (unsigned)(gstride * 4), orow = (unsigned)(ostride * 4);
  const unsigned gv = ok ? (unsigned)(b * 4 * H + j) * 4u : kOffNone;  // lane offsets in a row
  const unsigned ov = ok ? (unsigned)ch * 4u : kOffNone;
  // out rows in their own element format
  constexpr unsigned OB = fmt_bytes<OF>();
  const unsigned orow_o = (unsigned)ostride * OB, ov_o = ok ? (unsigned)ch * OB : kOffNone;
  char* const outb = static_cast<char*>(out);
  const int hb = 4 * H;  // bytes between gate planes
  if (w == 0) sC[lane] = ok ? fmaxf(c0 ? c0[ch] : 0.f, eps) : 0.f;

  constexpr int CH = NW * L;
  const int nchunks = (T + CH - 1) / CH, nfull = T / CH;
  const int nck = (T + L - 1) / L;  // the c_n row
  // the step loads: rows past T have size 0 (they read 0)
  auto load = [&](int chunk, float(&r)[4][L]) {
#pragma unroll
    for (int s = 0; s < L; ++s) {
      const int t = chunk * CH + w * L + s;
      const auto rs = row_rsrc(gates + (size_t)t * gstride, t < T ? grow : 0u);
#pragma unroll
      for (int g = 0; g < 4; ++g) r[g][s] = row_load(rs, gv, g * hb);
    }
  };
  // one chunk from the registers cur, with the next chunk's loads issued into nxt first;
  // TAIL: steps past T are identity maps (only the last chunk has any)
  auto chunk = [&](auto tail, int k, float(&cur)[4][L], float(&nxt)[4][L]) {
    constexpr bool TAIL = decltype(tail)::value;
    if (k + 1 < nchunks) load(k + 1, nxt);
    float fv[L], bv[L], ogv[L];
    float A = 1.f, V = 0.f;
#pragma unroll
    for (int s = 0; s < L; ++s) {
      float f = fmaxf(sigmoid_f(cur[1][s]), eps);
      float bb = fmaxf(sigmoid_prod_f(cur[0][s], cur[2][s]), eps);
      if (TAIL && k * CH + w * L + s >= T) {
        f = 1.f;
        bb = 0.f;
      }
      fv[s] = f;
      bv[s] = bb;
      ogv[s] = sigmoid_f(cur[3][s]);
      A = f * A;
      V = f * V + bb;
    }
    sAV[w][lane] = float2{A, V};
    lds_barrier();
    // carry-in: the chunk's carry through the maps of waves 0 .. w-1, applied in order;
    // the maps are read four at a time (one LDS latency per four, where a serial loop
    // would wait for each read; an unrolled loop over all of them spilled registers)
    float c = sC[lane];
#pragma unroll 1
    for (int u0 = 0; u0 < w; u0 += 4) {
      float2 m[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) m[i] = sAV[min(u0 + i, NW - 1)][lane];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (u0 + i < w) c = m[i].x * c + m[i].y;
    }
    // the carry-in is this group's checkpoint row (groups past T store nothing)
    const int t0 = k * CH + w * L;
    row_store_nt(c, row_rsrc(cck + (size_t)(k * NW + w) * ostride, t0 < T ? orow : 0u), ov, 0);
#pragma unroll
    for (int s = 0; s < L; ++s) {
      const int t = t0 + s;
      const unsigned obytes = (!TAIL || t < T) ? orow_o : 0u;
      c = __builtin_fmaf(fv[s], c, bv[s]);  // the backward repeats exactly this from the carry-in
      // c >= eps > 0 (a positive combination of positive terms)
      out_store<OF>(ogv[s] * tanh_pos_f(c),
                    row_rsrc(reinterpret_cast<const float*>(outb + (size_t)t * orow_o), obytes), ov_o);
    }
    // the group holding step T-1 writes c_{T-1} (steps past T are identity maps)
    row_store_nt(c, row_rsrc(cck + (size_t)nck * ostride, (t0 < T && T <= t0 + L) ? orow : 0u), ov, 0);
    lds_barrier();
    if (w == NW - 1) sC[lane] = c;
  };
  // chunks alternate between two register sets, so no copies between them
  float ra[4][L], rb[4][L];
  if (nchunks > 0) load(0, ra);
  int k = 0;
  for (; k + 1 < nfull; k += 2) {
    chunk(std::false_type{}, k, ra, rb);
    chunk(std::false_type{}, k + 1, rb, ra);
  }
  if (k < nchunks) chunk(std::true_type{}, k++, ra, rb);
  if (k < nchunks) chunk(std::true_type{}, k, rb, ra);
}

// Reverse scan.  For wave steps [ws, we] and G_in = G_{we+1}:
//   G_t = e_t + f~_{t+1} G_{t+1},  e_t = dout'_t o_t (1 - tanh^2 c_t) (+ dc_n at T-1),
//   dout'_t = dout_t (+ dh_n at T-1),  f~_T = 0.
// Then df~_t = G_t c_{t-1}, db~_t = G_t and the sigmoid/clamp chain gives dgates.
template <int NW, int L, int DF>
__global__ __launch_bounds__(NW * 64) void scan_bwd_kernel(
    const float* __restrict__ gates, const float* __restrict__ c0, const float* __restrict__ cck,
    const void* __restrict__ dout, const float* __restrict__ dh_n, const float* __restrict__ dc_n, float eps,
    float* __restrict__ dgates, double* __restrict__ db_part, float* __restrict__ dc0, int T, int B, int H) {
  static_assert(L == kCkSteps, "a wave's steps are one checkpoint group");
  __shared__ float2 sAV[NW][64];  // each wave's composed reverse map (A, V) of the chunk
  __shared__ float sG[64];
  __shared__ double sdb[NW][4][64];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int C = B * H;
  const int ch = blockIdx.x * 64 + lane;
  const bool ok = ch < C;
  const int b = ok ? ch / H : 0, j = ok ? ch % H : 0;
  const size_t gstride = (size_t)B * 4 * H, ostride = (size_t)C;
  const unsigned grow = (unsigned)(gstride * 4), orow = (unsigned)(ostride * 4);
  const unsigned gv = ok ? (unsigned)(b * 4 * H + j) * 4u : kOffNone;
  const unsigned ov = ok ? (unsigned)ch * 4u : kOffNone;
  // dout rows in their own element format
  constexpr unsigned DB = fmt_bytes<DF>();
  const unsigned drow = (unsigned)ostride * DB, dv = ok ? (unsigned)ch * DB : kOffNone;
  const char* const doutb = static_cast<const char*>(dout);
  const int hb = 4 * H;
  const float c0v = (ok && c0) ? c0[ch] : 0.f;
  const bool c0_pass = ok && c0v >= eps;
  const float dhn = (ok && dh_n) ? dh_n[ch] : 0.f, dcn = (ok && dc_n) ? dc_n[ch] : 0.f;
  if (w == 0) sG[lane] = 0.f;

  constexpr int CH = NW * L;
  const int nchunks = (T + CH - 1) / CH;
  // per step: zi zf zg zo dout; plus zf at we+1 (fnext) and the group's checkpoint row, the
  // c carried into its first step (cin); rows past T read 0
  auto load = [&](int chunk, float(&r)[5][L], float& fnext, float& cin) {
    const int ws = chunk * CH + w * L;
    // a 16-bit dout: the wave's L rows as one buffer (fewer scalar registers than a buffer
    // per row, which made that instance spill them; the fp32 one keeps a buffer per row)
    const int nd = min(T - ws, L);
    const auto rd = row_rsrc(reinterpret_cast<const float*>(doutb + (size_t)ws * drow), nd > 0 ? (unsigned)nd * drow : 0u);
#pragma unroll
    for (int s = 0; s < L; ++s) {
      const int t = ws + s;
      const auto rg = row_rsrc(gates + (size_t)t * gstride, t < T ? grow : 0u);
#pragma unroll
      for (int g = 0; g < 4; ++g) r[g][s] = row_load(rg, gv, g * hb);
      if constexpr (DF == kF32)
        r[4][s] = in_load<DF>(row_rsrc(reinterpret_cast<const float*>(doutb + (size_t)t * drow), t < T ? drow : 0u),
                              dv, 0);
      else
        r[4][s] = in_load<DF>(rd, dv, s * (int)drow);
    }
    const int tn = ws + L;
    fnext = row_load<0>(row_rsrc(gates + (size_t)tn * gstride, tn < T ? grow : 0u), gv, hb);
    cin = row_load(row_rsrc(cck + (size_t)(chunk * NW + w) * ostride, ws < T ? orow : 0u), ov, 0);
  };
  double dbacc[4] = {0.0, 0.0, 0.0, 0.0};
  float g_first = 0.f, f_first = 0.f;  // G and f~ at this wave's first step (for dc0)
  // one chunk (reverse); LAST: the chunk holding step T-1, the only one with steps at or
  // past T-1 (dh_n, dc_n, f~_T = 0, identity maps past T)
  auto chunk = [&](auto last, int k, float(&cur)[5][L], float cur_fn, float cur_cin, float(&nxt)[5][L],
                   float& nxt_fn, float& nxt_cin) {
    constexpr bool LAST = decltype(last)::value;
    if (k > 0) load(k - 1, nxt, nxt_fn, nxt_cin);
    const int ws = k * CH + w * L;
    // sigma(z_f), sigma(z_o), c and tanh(c) of each step, computed once and used by both
    // passes; c_t is recomputed from the carry-in by the forward's own operations, so it
    // equals the forward's bit for bit; f~_{t+1} (0 beyond T) is step s+1's sigma(z_f), e_t
    float fgv[L], ogv[L], cv[L], tcv[L], fn[L], ev[L];
    float c = cur_cin;
#pragma unroll
    for (int s = 0; s < L; ++s) {
      fgv[s] = sigmoid_f(cur[1][s]);
      ogv[s] = sigmoid_f(cur[3][s]);
      c = __builtin_fmaf(fmaxf(fgv[s], eps), c, fmaxf(sigmoid_prod_f(cur[0][s], cur[2][s]), eps));
      cv[s] = c;
      tcv[s] = tanh_pos_f(c);  // c >= eps > 0
    }
    const float fg_after = sigmoid_f(cur_fn);
#pragma unroll
    for (int s = 0; s < L; ++s) {
      const int t = ws + s;
      fn[s] = (!LAST || t + 1 < T) ? fmaxf(s + 1 < L ? fgv[s + 1] : fg_after, eps) : 0.f;
      float d = cur[4][s];
      if (LAST && t == T - 1) d = d + dhn;
      float e = d * ogv[s] * (1.0f - tcv[s] * tcv[s]);
      if (LAST && t == T - 1) e = e + dcn;
      ev[s] = (!LAST || t < T) ? e : 0.f;
    }
    float A = 1.f, V = 0.f;
#pragma unroll
    for (int s = L - 1; s >= 0; --s) {
      if (!LAST || ws + s < T) {
        V = ev[s] + fn[s] * V;
        A = fn[s] * A;
      }
    }
    sAV[w][lane] = float2{A, V};
    lds_barrier();
    // carry-in from the later waves NW-1 .. w+1, applied in order; the maps are read four
    // at a time (one LDS latency per four)
    float G = sG[lane];
#pragma unroll 1
    for (int u0 = NW - 1; u0 > w; u0 -= 4) {
      float2 m[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) m[i] = sAV[max(u0 - i, 0)][lane];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (u0 - i > w) G = m[i].x * G + m[i].y;
    }
    float dsum[4] = {0.f, 0.f, 0.f, 0.f};  // the chunk's dgates sums, added into fp64 below
#pragma unroll
    for (int s = L - 1; s >= 0; --s) {
      const int t = ws + s;
      if (!LAST || t < T) {
        G = ev[s] + fn[s] * G;
        const float ig = sigmoid_f(cur[0][s]), gg = sigmoid_f(cur[2][s]);
        const float fg = fgv[s], og = ogv[s], tc = tcv[s];
        const float cprev = s > 0 ? cv[s - 1] : cur_cin;
        float d = cur[4][s];
        if (LAST && t == T - 1) d = d + dhn;
        const float bb = ig * gg;
        const float dbb = bb >= eps ? G : 0.f;
        const float dfp = fg >= eps ? (G * cprev) * fg * (1.0f - fg) : 0.f;
        const float dbq = dbb * bb;
        const float dip = dbq * (1.0f - ig);
        const float dgp = dbq * (1.0f - gg);
        const float dop = (d * tc) * og * (1.0f - og);
        const auto rq = row_rsrc(dgates + (size_t)t * gstride, grow);
        row_store_nt(dip, rq, gv, 0);
        row_store_nt(dfp, rq, gv, hb);
        row_store_nt(dgp, rq, gv, 2 * hb);
        row_store_nt(dop, rq, gv, 3 * hb);
        dsum[0] += dip;
        dsum[1] += dfp;
        dsum[2] += dgp;
        dsum[3] += dop;
        if (s == 0) {
          g_first = G;
          f_first = fmaxf(fg, eps);
        }
      }
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) dbacc[g] += (double)dsum[g];
    lds_barrier();
    if (w == 0) sG[lane] = G;
  };
  // chunks alternate between two register sets, so no copies between them
  float ra[5][L], rb[5][L];
  float fa = 0.f, pa = 0.f, fb = 0.f, pb = 0.f;
  if (nchunks > 0) {
    load(nchunks - 1, ra, fa, pa);
    chunk(std::true_type{}, nchunks - 1, ra, fa, pa, rb, fb, pb);
  }
  int k = nchunks - 2;
  for (; k >= 1; k -= 2) {
    chunk(std::false_type{}, k, rb, fb, pb, ra, fa, pa);
    chunk(std::false_type{}, k - 1, ra, fa, pa, rb, fb, pb);
  }
  if (k == 0) chunk(std::false_type{}, 0, rb, fb, pb, ra, fa, pa);
  // dc0 = G_0 f~_0 where the clamp of c0 passes gradient
  if (w == 0 && ok && dc0) dc0[ch] = (c0_pass && T > 0) ? g_first * f_first : 0.f;
  if (db_part) {
#pragma unroll
    for (int g = 0; g < 4; ++g) sdb[w][g][lane] = dbacc[g];
    __syncthreads();
    if (w == 0 && ok) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        double s = 0.0;
        for (int u = 0; u < NW; ++u) s += sdb[u][g][lane];
        db_part[(size_t)b * 4 * H + g * H + j] = s;
      }
    }
  }
}

// one time step of gates (16 B H bytes) is addressed as a buffer of < 2^31 bytes
int check_scan_dims(int T, int B, int H, int D = 0) { return check_shape("parallel mode", T, B, D, H); }

// out (forward) and dout (backward) in format sf (StreamFmt); everything else fp32.
int scan_fwd(const float* gates, const float* c0, float eps, void* out, float* cck, int T, int B, int H,
             hipStream_t s, int sf = kF32) {
  const int C = B * H;
  if (C == 0 || T == 0) return HSL_OK;
  const int slot = timing_begin(kTimeScanFwd, s);
  const dim3 grid((C + 63) / 64), block(kFwdWaves * 64);
  if (sf == kBf16)
    hipLaunchKernelGGL((scan_fwd_kernel<kFwdWaves, kFwdSteps, kBf16>), grid, block, 0, s, gates, c0, eps, out, cck,
                       T, B, H);
  else if (sf == kF16)
    hipLaunchKernelGGL((scan_fwd_kernel<kFwdWaves, kFwdSteps, kF16>), grid, block, 0, s, gates, c0, eps, out, cck,
                       T, B, H);
  else
    hipLaunchKernelGGL((scan_fwd_kernel<kFwdWaves, kFwdSteps, kF32>), grid, block, 0, s, gates, c0, eps, out, cck,
                       T, B, H);
  HSL_HIP(hipGetLastError());
  timing_end(slot, s);
  return HSL_OK;
}

int scan_bwd(const float* gates, const float* c0, const float* cck, const void* dout, const float* dh_n,
             const float* dc_n, float eps, float* dgates, double* db_part, float* dc0, int T, int B, int H,
             hipStream_t s, int sf = kF32) {
  const int C = B * H;
  if (C == 0) return HSL_OK;
  if (T == 0) {  // no steps: dc0 = dc_n through the clamp is not reached; all zero
    if (dc0) HSL_CHECK(copy_f32(dc0, nullptr, (size_t)C, s));
    if (db_part) HSL_CHECK(zero_words(reinterpret_cast<unsigned long long*>(db_part), (size_t)4 * C, s));
    return HSL_OK;
  }
  const int slot = timing_begin(kTimeScanBwd, s);
  const dim3 grid((C + 63) / 64), block(kBwdWaves * 64);
  if (sf == kBf16)
    hipLaunchKernelGGL((scan_bwd_kernel<kBwdWaves, kBwdSteps, kBf16>), grid, block, 0, s, gates, c0, cck, dout, dh_n,
                       dc_n, eps, dgates, db_part, dc0, T, B, H);
  else if (sf == kF16)
    hipLaunchKernelGGL((scan_bwd_kernel<kBwdWaves, kBwdSteps, kF16>), grid, block, 0, s, gates, c0, cck, dout, dh_n,
                       dc_n, eps, dgates, db_part, dc0, T, B, H);
  else
    hipLaunchKernelGGL((scan_bwd_kernel<kBwdWaves, kBwdSteps, kF32>), grid, block, 0, s, gates, c0, cck, dout, dh_n,
                       dc_n, eps, dgates, db_part, dc0, T, B, H);
  HSL_HIP(hipGetLastError());
  timing_end(slot, s);
  return HSL_OK;
}

struct ParWs {
  float* dgates;    // [T*B*4H]
  double* db_part;  // [B*4H]
  float* gemm;
  size_t gemm_bytes;
};

size_t carve_par(void* ws, size_t cap, int T, int B, int D, int H, ParWs* o) {
  Carver c(ws, cap);
  o->dgates = c.take<float>((size_t)T * B * 4 * H);
  o->db_part = c.take<double>((size_t)B * 4 * H);
  size_t g = gemm_ws_bytes_layout(4 * H, D, T * B, 1, 1, 0);
  const size_t g6 = gemm_ws_bytes_layout(T * B, D, 4 * H, 1, 0, 0);
  if (g6 > g) g = g6;
  o->gemm_bytes = g;
  o->gemm = c.take<float>(g / sizeof(float) + 1);
  return c.off;
}

// The parallel backward with an fp32 (fmt < 0) or 16-bit (fmt 0 bf16, 1 fp16) x and W_ih.
// The 16-bit workspace adds one region that holds a widened x or W_ih when a product has
// to run on the fp32 kernels.
size_t carve_par_b16(void* ws, size_t cap, int T, int B, int D, int H, ParWs* o, float** widen) {
  const size_t off = carve_par(ws, cap, T, B, D, H, o);
  Carver c(ws, cap);
  c.off = off;
  const size_t n = std::max((size_t)T * B * D, (size_t)4 * H * D);
  float* w = c.take<float>(n + 1);
  if (widen) *widen = w;
  return c.off;
}

int par_bwd_impl(const void* dout, const float* dh_n, const float* dc_n, const void* x, const float* c0,
                 const float* gates, const float* c_ck, const void* w_ih, float eps, float* dx, float* dw_ih,
                 float* db_ih, float* dc0, void* ws, size_t ws_bytes, int T, int B, int D, int H, int fmt,
                 hipStream_t s) {
  const char* fn = fmt < 0 ? "hsl_par_bwd" : "hsl_par_bwd_b16";
  HSL_CHECK(check_scan_dims(T, B, H, D));
  if (H == 0) return HSL_OK;
  if (!dw_ih || !db_ih || !w_ih) return fail(HSL_ERR_ARG, "%s: null pointer", fn);
  ParWs w;
  float* widen = nullptr;
  const size_t need =
      fmt < 0 ? carve_par(ws, ws_bytes, T, B, D, H, &w) : carve_par_b16(ws, ws_bytes, T, B, D, H, &w, &widen);
  if (!ws || ws_bytes < need) return fail(HSL_ERR_ARG, "%s: workspace %zu bytes, need %zu", fn, ws_bytes, need);
  if (T == 0 || B == 0) {
    HSL_CHECK(copy_f32(dw_ih, nullptr, (size_t)4 * H * D, s));
    HSL_CHECK(copy_f32(db_ih, nullptr, (size_t)4 * H, s));
    if (dc0) HSL_CHECK(copy_f32(dc0, nullptr, (size_t)B * H, s));
    return HSL_OK;
  }
  if (!dout || !x || !gates || !c_ck) return fail(HSL_ERR_ARG, "%s: null pointer", fn);
  HSL_CHECK(scan_bwd(gates, c0, c_ck, dout, dh_n, dc_n, eps, w.dgates, w.db_part, dc0, T, B, H, s,
                     fmt < 0 ? kF32 : (fmt == 0 ? kBf16 : kF16)));
  HSL_CHECK(bias_grads_from_parts(w.db_part, B, nullptr, nullptr, nullptr, db_ih, nullptr, nullptr, H, s));
  const int TB = T * B;
  if (D > 0) {
    // dW_ih = dgates^T x, dx = dgates W_ih (B operands [K][N]; 16-bit ones pass as such)
    GemmDesc g5{w.dgates, static_cast<const float*>(x), nullptr, dw_ih, 4 * H, D, TB, 4 * H, D, D, 1, 0, 1};
    if (fmt < 0)
      HSL_CHECK(gemm_run(g5, w.gemm, w.gemm_bytes, s));
    else
      HSL_CHECK(gemm_run_b16(g5, fmt, widen, w.gemm, w.gemm_bytes, s));
    if (dx) {
      GemmDesc g6{w.dgates, static_cast<const float*>(w_ih), nullptr, dx, TB, D, 4 * H, 4 * H, D, D, 0, 0, 1};
      if (fmt < 0)
        HSL_CHECK(gemm_run(g6, w.gemm, w.gemm_bytes, s));
      else
        HSL_CHECK(gemm_run_b16(g6, fmt, widen, w.gemm, w.gemm_bytes, s));
    }
  }
  return HSL_OK;
}

}  // namespace
}  // namespace hsl

using namespace hsl;

extern "C" {

int hsl_scan_ck_rows(int T) { return T < 0 ? 0 : (T + kCkSteps - 1) / kCkSteps + 1; }

int hsl_scan_fwd(const float* gates, const float* c0, float eps, float* out, float* c_ck, int T, int B, int H,
                 void* stream) {
  HSL_CHECK(check_scan_dims(T, B, H));
  if (T > 0 && B > 0 && H > 0 && (!gates || !out || !c_ck)) return fail(HSL_ERR_ARG, "hsl_scan_fwd: null pointer");
  return scan_fwd(gates, c0, eps, out, c_ck, T, B, H, static_cast<hipStream_t>(stream));
}

int hsl_scan_bwd(const float* gates, const float* c0, const float* c_ck, const float* dout, const float* dh_n,
                 const float* dc_n, float eps, float* dgates, double* db_part, float* dc0, int T, int B, int H,
                 void* stream) {
  HSL_CHECK(check_scan_dims(T, B, H));
  if (B > 0 && H > 0 && T > 0 && (!gates || !c_ck || !dout || !dgates))
    return fail(HSL_ERR_ARG, "hsl_scan_bwd: null pointer");
  return scan_bwd(gates, c0, c_ck, dout, dh_n, dc_n, eps, dgates, db_part, dc0, T, B, H,
                  static_cast<hipStream_t>(stream));
}

int hsl_par_fwd(const float* x, const float* c0, const float* w_ih, const float* b_ih, float eps, float* gates,
                float* out, float* c_ck, int T, int B, int D, int H, void* stream) {
  HSL_CHECK(check_scan_dims(T, B, H, D));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (T == 0 || B == 0 || H == 0) return HSL_OK;
  if (!x || !w_ih || !b_ih || !gates || !out || !c_ck) return fail(HSL_ERR_ARG, "hsl_par_fwd: null pointer");
  GemmDesc g1{x, w_ih, b_ih, gates, T * B, 4 * H, D, D, D, 4 * H, 0, 1, 0};
  const int slot = timing_begin(kTimeInputProj, s);
  HSL_CHECK(gemm_run(g1, nullptr, 0, s));
  timing_end(slot, s);
  return scan_fwd(gates, c0, eps, out, c_ck, T, B, H, s);
}

int hsl_par_fwd_b16(const void* x, const float* c0, const void* w_ih, const float* b_ih, float eps, float* gates,
                    void* out, float* c_ck, int T, int B, int D, int H, int fmt, void* stream) {
  if (fmt != 0 && fmt != 1) return fail(HSL_ERR_ARG, "hsl_par_fwd_b16: format must be 0 (bf16) or 1 (fp16)");
  HSL_CHECK(check_scan_dims(T, B, H, D));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (T == 0 || B == 0 || H == 0) return HSL_OK;
  if (!x || !w_ih || !b_ih || !gates || !out || !c_ck) return fail(HSL_ERR_ARG, "hsl_par_fwd_b16: null pointer");
  const int slot = timing_begin(kTimeInputProj, s);
  HSL_CHECK(gemm_b16_run(x, w_ih, b_ih, gates, T * B, 4 * H, D, D, D, 4 * H, fmt, s));
  timing_end(slot, s);
  return scan_fwd(gates, c0, eps, out, c_ck, T, B, H, s, fmt == 0 ? kBf16 : kF16);
}

size_t hsl_par_bwd_ws_bytes(int T, int B, int D, int H) {
  if (T < 0 || B < 0 || D < 0 || H < 0) return 0;
  ParWs w;
  return carve_par(nullptr, 0, T, B, D, H, &w);
}

size_t hsl_par_bwd_b16_ws_bytes(int T, int B, int D, int H) {
  if (T < 0 || B < 0 || D < 0 || H < 0) return 0;
  ParWs w;
  return carve_par_b16(nullptr, 0, T, B, D, H, &w, nullptr);
}

int hsl_par_bwd(const float* dout, const float* dh_n, const float* dc_n, const float* x, const float* c0,
                const float* gates, const float* c_ck, const float* w_ih, float eps, float* dx, float* dw_ih,
                float* db_ih, float* dc0, void* ws, size_t ws_bytes, int T, int B, int D, int H, void* stream) {
  return par_bwd_impl(dout, dh_n, dc_n, x, c0, gates, c_ck, w_ih, eps, dx, dw_ih, db_ih, dc0, ws, ws_bytes, T, B, D,
                      H, -1, static_cast<hipStream_t>(stream));
}

int hsl_par_bwd_b16(const void* dout, const float* dh_n, const float* dc_n, const void* x, const float* c0,
                    const float* gates, const float* c_ck, const void* w_ih, float eps, float* dx, float* dw_ih,
                    float* db_ih, float* dc0, void* ws, size_t ws_bytes, int T, int B, int D, int H, int fmt,
                    void* stream) {
  if (fmt != 0 && fmt != 1) return fail(HSL_ERR_ARG, "hsl_par_bwd_b16: format must be 0 (bf16) or 1 (fp16)");
  return par_bwd_impl(dout, dh_n, dc_n, x, c0, gates, c_ck, w_ih, eps, dx, dw_ih, db_ih, dc0, ws, ws_bytes, T, B, D,
                      H, fmt, static_cast<hipStream_t>(stream));
}

}  // extern "C"
