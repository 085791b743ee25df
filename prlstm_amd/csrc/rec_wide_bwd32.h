// Single-chain persistent recurrent backward for H = 1024 (U = 32), B <= 32.  Included by
// recurrent.hip after rec_wide.h, whose grid, hand-off helpers, slot rotation and argument
// block it uses; it reads the same buffers as the two-chain backward there, laid out for one
// chain of 32 batch rows.  At H = 1024 a step's products are a quarter of those at H = 2048
// (1.7 us of the chip's fp32 matrix time per step), too short to hide a second chain's
// hand-offs, and the two-chain form measured slower there (published T64 B32 D512 H1024
// shape: 1.062 -> 1.077 ms per training step), so this form runs instead.
//
// Workgroup (x, c) holds W_hh's 16U gate rows of XCD x for the columns [U c, +U) as in the
// two-chain backward; wave w takes rows [4U w, +4U), one column tile of 32 x 2U k-steps in
// the accumulator registers.  Per iteration:
//   1. products: wave w reads a_g dg_{t+1} of its 4U rows and all 32 batch rows from the
//      XCD's broadcast buffer, 8 groups at a time (the next 8 are requested before the
//      current ones multiply), on v_mfma_f32_32x32x2_f32 (M = 32 columns, N = 32 batch);
//   2. the four waves' partials [U columns x 32 batch] are summed in LDS and sent to the
//      reducing workgroups (c / 4, 8 (c % 4) + sl) as in the two-chain form;
//   3. reducer lane (unit su of slice c, batch b) sums the 8 row XCDs' partials in XCD
//      order, adds dout_t (and dh_n at t = T-1), runs the cell backward, stores dgates_t,
//      adds it to the lane's fp64 bias sums and publishes a_g dg_t: its U/8 units x 4 gates
//      x 32 batch are one contiguous group of 16U words of the broadcast buffer.
// One more product after t = 0 gives dh0.  Slots: broadcast of iteration k in slot k%4, its
// owner clears slot (k+2)%4 after publishing; partials of iteration k in slot (k-1)%3,
// cleared by their one reader.
// Buffers: dgbuf [4 slots][8 XCDs][16U rows x 32 batch]; inbox [3 slots][256][8 x 32 x U/8].

__device__ __forceinline__ void wide_ksteps4_32(f16v (&acc)[4], const float (&w)[4][1], f4 h) {
  asm volatile(
      "s_nop 1\n\t"
      "v_mfma_f32_32x32x2_f32 %0, %4, %8, %0\n\t"
      "v_mfma_f32_32x32x2_f32 %1, %5, %9, %1\n\t"
      "v_mfma_f32_32x32x2_f32 %2, %6, %10, %2\n\t"
      "v_mfma_f32_32x32x2_f32 %3, %7, %11, %3"
      : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3])
      : "a"(w[0][0]), "a"(w[1][0]), "a"(w[2][0]), "a"(w[3][0]), "v"(h[0]), "v"(h[1]), "v"(h[2]), "v"(h[3]));
}

// The wave's partial of 4 consecutive columns, register group q, from the accumulators
// (k-step e % 4 in acc[e % 4]).
__device__ __forceinline__ f4 wide_partial1(const f16v (&acc)[4], int q) {
  f4 v;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int r = 4 * q + e;
    v[e] = (acc[0][r] + acc[1][r]) + (acc[2][r] + acc[3][r]);
  }
  return v;
}

// Wait states after the last products of a step, before any instruction reads their
// accumulators (an XDL result read by VALU, LDS or memory instructions needs up to 18 on
// the 16-pass 32x32x2; the compiler cannot see inside the asm above, so it adds none).
__device__ __forceinline__ void wide_ksteps_drain32(f16v (&acc)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(acc[i]));
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
  for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(acc[i]));
}

template <int U>
struct WideB1Shape {
  static_assert(U == 32, "the single-chain backward serves H = 1024");
  static constexpr int CT = U / 32;           // column tiles of 32 per wave
  static constexpr int SU = U / 8;            // units per reducer slice
  static constexpr int ROWS = 16 * U;         // gate rows held per XCD
  static constexpr int WROWS = 4 * U;         // gate rows per wave
  static constexpr int NQ = U / 2;            // 16-byte groups of a wave's dg operands (2U k-steps)
  static constexpr int INBOX = 8 * 32 * SU;   // inbox words of a reducer per slot: [src x][batch][unit]
  static constexpr int GROUP = 16 * U;        // words of a reducer's published dg group
  static constexpr int RED = 32 * U;          // floats of one wave's partials [U columns][32 batch]
  static constexpr int LDS_BYTES = 4 * (4 * RED + GROUP);  // wave partials + the gathered dg group
  static constexpr int REDUCERS = 32 * SU;    // reducer lanes (unit, batch) of a workgroup
  // the same exchange buffers as the two-chain backward
  static_assert(kWideHSlots * kWideXcds * ROWS * 32 == kWideHSlots * 2 * kWideXcds * WideBShape<U>::XBUF &&
                    INBOX == 2 * WideBShape<U>::INBOX,
                "buffer sizes");
};

// word of (local row rho, batch b) in an XCD's broadcast buffer: wave w = rho / 4U reads
// group j (k-steps 4j .. 4j+3 of its rows) at 128U w + 256 j + 4 l
template <int U>
__device__ __forceinline__ unsigned wideb1_pos(int rho, int b) {
  const int w = rho / (4 * U), rl = rho % (4 * U), i = rl >> 1, l = b + 32 * (rl & 1);
  return 128u * U * w + 256u * (i >> 2) + 4u * l + (i & 3);
}

template <int U, bool FAST>
__device__ __forceinline__ void rec_bwd_wide1_body(const WBwdArgs& p, int x, int c, float* red, float* gst,
                                                  int& abort_flag) {
  using S = WideB1Shape<U>;
  constexpr int CT = S::CT, SU = S::SU;
  const int T = p.T, B = p.B, H = p.H;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hb = lane >> 5, l32 = lane & 31;
  const int ubase = 4 * U * x;  // first unit of the XCD's rows

  // W_hh^T block of this wave: column tile ct, k-step 4 i4 + e -> column m = l%32 of the
  // tile (unit U c + 32 ct + m), row rho = 4U w + 2 (4 i4 + e) + l/32 (unit ubase + rho/4,
  // gate rho % 4); unscaled, a multiplies the dg operand instead
  float wreg[S::NQ][4][CT];
#pragma unroll
  for (int i8 = 0; i8 < S::NQ; i8 += 4) {
#pragma unroll
    for (int i4 = i8; i4 < i8 + 4; ++i4)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int rho = S::WROWS * w + 2 * (4 * i4 + e) + hb;
        const float* row = p.w_hh + ((size_t)(rho & 3) * H + ubase + (rho >> 2)) * H + U * c + l32;
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) wreg[i4][e][ct] = row[32 * ct];
      }
#pragma unroll
    for (int i4 = i8; i4 < i8 + 4; ++i4)
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) asm volatile("" : "+a"(wreg[i4][e][ct]));  // held in the accumulator file
  }

  // reducer lane (tid < REDUCERS): unit su of this workgroup's slice (slice c of XCD x:
  // units ubase + SU c + su), batch cb
  const int su = tid >> 5, cb = tid & 31;
  const bool reducer = tid < S::REDUCERS;
  const bool c_ok = reducer && cb < B;
  const int unit = ubase + SU * c + su;
  float ag[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) ag[g] = p.a[g];
  float dc = 0.f;
  double dbacc[4] = {0.0, 0.0, 0.0, 0.0};
  if (c_ok && p.dc_n) dc = p.dc_n[(size_t)cb * H + unit];
  const size_t plane = (size_t)B * H, plane4 = 4 * plane;
  const bool h_ok = l32 < B;
  // broadcast buffer of this XCD; this workgroup's group in it
  const size_t bslot = (size_t)kWideXcds * S::ROWS * 32;
  float* const bx = p.dgbuf + (size_t)x * S::ROWS * 32;
  // send: lane (c4 = tid / 32, batch sb = tid % 32) sends columns SU c4 .. +SU (slice c4)
  // to reducer (c / 4, 8 (c % 4) + c4), inbox [src x][sb][SU units]
  const int c4 = tid >> 5, sb = tid & 31;
  const int dst = (c >> 2) + kWideXcds * (8 * (c & 3) + c4);
  const size_t islot = (size_t)kWideWgs * S::INBOX;
  for (int k = 0; k <= T; ++k) {
    const int t = T - 1 - k;  // the cell's step (-1 after the last product: dh0)
    // the cell's inputs of step t, requested before the products so that their latency runs
    // under them (lanes without a cell read clamped addresses)
    float in_do = 0.f, in_c = 0.f, in_tc = 0.f, in_dhn = 0.f;
    f4 in_ga = f4{0.f, 0.f, 0.f, 0.f};
    if (reducer && k < T) {
      const size_t ec = c_ok ? (size_t)cb * H + unit : 0, tp = (size_t)t * plane + ec;
      in_do = p.dout[tp];
      in_ga = *reinterpret_cast<const f4*>(p.gact + tp * 4);
      in_c = p.c_save[tp];
      in_tc = p.tanh_c[tp];
      if (k == 0 && p.dh_n) in_dhn = p.dh_n[ec];
    }
    float dsum = 0.f;
    if (k > 0) {
      // ---- 1. products with a_g dg_{t+1} of the wave's rows ---------------------------
      const __amdgpu_buffer_rsrc_t src =
          wide_rsrc(bx + (size_t)((k - 1) % kWideHSlots) * bslot + 128u * U * w, 128 * U);
      f16v acc[4] = {f16v{}, f16v{}, f16v{}, f16v{}};
      u4v qa[8], qb[8];
      auto issue = [&](u4v (&q)[8], int jb) {
#pragma unroll
        for (int j = 0; j < 8; ++j) q[j] = h_ok ? quad_load(src, 256u * (jb + j) + 4u * lane) : u4v{0u, 0u, 0u, 0u};
      };
      // waits for groups jb .. jb+7 (all eight reloaded while any word is kEmpty: the loop
      // then keeps no state beyond the values)
      auto settle = [&](u4v (&q)[8], int jb) -> bool {
        const long long t0 = wall_clock64();
        while (true) {
          unsigned m = 0u;
#pragma unroll
          for (int j = 0; j < 8; ++j) m = max(m, max(max(q[j][0], q[j][1]), max(q[j][2], q[j][3])));
          if (__all(m != kEmpty)) return true;
          if (wall_clock64() - t0 > p.spin) {
            raise_abort(&abort_flag, p.err);
            return false;
          }
          issue(q, jb);
        }
      };
      auto mult = [&](const u4v (&q)[8], int jb) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          wide_ksteps4_32(acc, wreg[jb + j],
                       f4{__uint_as_float(q[j][0]), __uint_as_float(q[j][1]), __uint_as_float(q[j][2]),
                          __uint_as_float(q[j][3])});
      };
      static_assert(S::NQ == 16, "two batches of eight groups");
      issue(qa, 0);
      if (!settle(qa, 0)) return;
      issue(qb, 8);
      mult(qa, 0);
      if (!settle(qb, 8)) return;
      mult(qb, 8);
      wide_ksteps_drain32(acc);
      // ---- 2. the four waves' partials summed in LDS, sent to the reducers ------------
      // D layout: lane l, register 4 q + e -> column 8 q + 4 (l/32) + e of tile ct, batch
      // l%32; red[w][column quad][batch] holds 4 columns
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<f4*>(&red[((w * (U / 4) + 8 * ct + 2 * q + hb) * 32 + l32) * 4]) =
              wide_partial1(acc, q);
      lds_barrier();
      if (abort_flag) return;
      if (sb < B) {
        const __amdgpu_buffer_rsrc_t d =
            wide_rsrc(p.inbox + (size_t)((k - 1) % kWidePSlots) * islot, (size_t)kWideWgs * S::INBOX);
#pragma unroll
        for (int qq = 0; qq < SU / 4; ++qq) {
          f4 sum = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ww = 0; ww < 4; ++ww)
            sum = sum + *reinterpret_cast<const f4*>(&red[((ww * (U / 4) + (SU / 4) * c4 + qq) * 32 + sb) * 4]);
          quad_put<false>(d, (unsigned)(dst * S::INBOX + x * 32 * SU + sb * SU + 4 * qq), sum);
        }
      }
      // ---- 3a. the reducer's sum of the 8 row XCDs' partials --------------------------
      if (c_ok) {
        const __amdgpu_buffer_rsrc_t ib =
            wide_rsrc(p.inbox + (size_t)((k - 1) % kWidePSlots) * islot + (size_t)blockIdx.x * S::INBOX, S::INBOX);
        unsigned v[8];
        const long long t0 = wall_clock64();
        while (true) {
          unsigned m = 0u;
#pragma unroll
          for (int sx = 0; sx < 8; ++sx) {
            v[sx] = __builtin_amdgcn_raw_buffer_load_b32(ib, (int)(4u * (sx * 32 * SU + cb * SU + su)), 0, kCpolSc1);
            m = max(m, v[sx]);
          }
          if (__all(m != kEmpty)) break;
          if (wall_clock64() - t0 > p.spin) {
            raise_abort(&abort_flag, p.err);
            return;
          }
        }
#pragma unroll
        for (int sx = 0; sx < 8; ++sx)
          __builtin_amdgcn_raw_buffer_store_b32(kEmpty, ib, (int)(4u * (sx * 32 * SU + cb * SU + su)), 0, kCpolSc1);
        dsum = __uint_as_float(v[0]);
#pragma unroll
        for (int sx = 1; sx < 8; ++sx) dsum += __uint_as_float(v[sx]);
      }
    }
    if (k == T) {  // dh of h0, the carry into c0, the bias partials
      if (c_ok) {
        if (p.dh0) p.dh0[(size_t)cb * H + unit] = dsum;
        if (p.dc0) p.dc0[(size_t)cb * H + unit] = dc;
#pragma unroll
        for (int g = 0; g < 4; ++g) p.db_part[(size_t)cb * 4 * H + g * H + unit] = dbacc[g];
      }
      break;
    }
    // ---- 3b. cell backward of step t, dgates_t, the broadcast of a_g dg_t ---------------
    float d[4] = {0.f, 0.f, 0.f, 0.f};
    if (c_ok) {
      const float dh = (k > 0 ? dsum : in_dhn) + in_do;
      cell_bwd(dh, dc, in_c, in_ga[0], in_ga[1], in_ga[2], in_ga[3], in_tc, d);
      float* const dg = p.dgates + (size_t)t * plane4 + (size_t)cb * 4 * H + unit;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        __builtin_nontemporal_store(d[g], dg + (size_t)g * H);
        dbacc[g] += (double)d[g];
      }
    }
    // gather: rows 4 (SU c + su) + g of this XCD are word GROUP c + (wideb1_pos - GROUP c) of
    // the buffer; absent batch rows publish 0
    if (reducer) {
#pragma unroll
      for (int g = 0; g < 4; ++g)
        gst[wideb1_pos<U>(4 * (SU * c + su) + g, cb) - (unsigned)S::GROUP * c] = c_ok ? canon_nan(ag[g] * d[g]) : 0.f;
    }
    lds_barrier();
    if (abort_flag) return;
    if (tid < S::GROUP / 4) {
      const f4 qv = *reinterpret_cast<const f4*>(&gst[4 * tid]);
      const __amdgpu_buffer_rsrc_t bp =
          wide_rsrc(bx + (size_t)(k % kWideHSlots) * bslot + (size_t)S::GROUP * c, S::GROUP);
      quad_store<FAST>(bp, 4u * tid, u4v{__float_as_uint(qv[0]), __float_as_uint(qv[1]), __float_as_uint(qv[2]),
                                         __float_as_uint(qv[3])});
      const __amdgpu_buffer_rsrc_t bc =
          wide_rsrc(bx + (size_t)((k + 2) % kWideHSlots) * bslot + (size_t)S::GROUP * c, S::GROUP);
      quad_store<FAST>(bc, 4u * tid, u4v{kEmpty, kEmpty, kEmpty, kEmpty});
    }
  }
}

// After an abort the reducer lanes set what they own to NaN: dgates of their unit and batch
// row at every step, the bias partials, and dh0 / dc0.
template <int U>
__device__ void poison_wide_bwd1(const WBwdArgs& p, int x, int c) {
  using S = WideB1Shape<U>;
  const int tid = threadIdx.x, su = tid >> 5, cb = tid & 31;
  if (tid >= S::REDUCERS || cb >= p.B) return;
  const int unit = 4 * U * x + S::SU * c + su, H = p.H;
  const float nan = __uint_as_float(0x7FC00000u);
  const size_t e = (size_t)cb * H + unit;
  if (p.dh0) p.dh0[e] = nan;
  if (p.dc0) p.dc0[e] = nan;
  for (int g = 0; g < 4; ++g) p.db_part[(size_t)cb * 4 * H + g * H + unit] = (double)nan;
  for (int t = 0; t < p.T; ++t)
    for (int g = 0; g < 4; ++g) p.dgates[((size_t)t * p.B + cb) * 4 * H + g * H + unit] = nan;
}

template <int U>
__global__ __launch_bounds__(256, 1) void rec_bwd_wide1(WBwdArgs p) {
  using S = WideB1Shape<U>;
  extern __shared__ float wide_lds[];  // wave partials, then the gathered dg group (padded: one workgroup per CU)
  __shared__ int abort_flag;
  const int x = blockIdx.x % kWideXcds, c = blockIdx.x / kWideXcds;
  if (threadIdx.x == 0) abort_flag = 0;
  const bool fast = agree_placement(p.hello + (size_t)x * (kWideRowSubs * kWideKBlocks), c,
                                    kWideRowSubs * kWideKBlocks, p.spin, &abort_flag, p.err) &&
                    !p.device_scope;
  if (!abort_flag) {
    if (fast)
      rec_bwd_wide1_body<U, true>(p, x, c, wide_lds, wide_lds + 4 * S::RED, abort_flag);
    else
      rec_bwd_wide1_body<U, false>(p, x, c, wide_lds, wide_lds + 4 * S::RED, abort_flag);
  }
  lds_barrier();
  if (abort_flag) poison_wide_bwd1<U>(p, x, c);
}

