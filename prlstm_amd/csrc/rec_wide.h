// Persistent recurrent kernels for a large hidden size, H = 32 U with U = 64 (H = 2048,
// configs[3]) or U = 32 (H = 1024, the reference's published T64 B32 D512 H1024 shape),
// B <= 32.  Included by recurrent.hip: they share that file's hand-off helpers and its
// device error word.  This file holds what the wide forward (rec_wide_fwd.h) and backward
// share -- the grid, the hand-off buffers and their access helpers, the slot rotation --
// and the backward.
//
// W_hh stays in registers for the whole launch: 4H x H floats over 256 workgroups is
// 256 KB per CU at H = 2048 and 64 KB at H = 1024, where the per-step path streams it
// from the Infinity Cache every step (_torch.py:111-120 runs one h W_hh^T product per
// step).  All 256 workgroups are resident at once, one per CU, 32 on each of the 8 XCDs
// (blockIdx % 8 = XCD); each step's values cross the XCDs once.
//
// Hand-off words are 4-byte values that start out kEmpty, as in the other persistent
// kernels.  Values that cross XCDs use device-scope stores and loads; values that stay on
// an XCD use workgroup-scope stores (sc0) when every member of the group runs on the
// group's XCD.
//
// Slots (forward; the backward uses the same rotation for its dg broadcasts and partials).
// h_t goes to slot t%4 of its block; after publishing h_t the owner clears its word in slot
// (t+2)%4.  Every workgroup's step-t products need h_{t-1} of all H units (the 8 workgroups
// of a row group cover all k), and every unit's h_{t-1} needed the partials of its row
// group at t-1, which read h_{t-2} of all units: so when the owner publishes h_t, every
// reader has read h_{t-2}.  A reader of h_{t+2} read the owner's h_{t+1} first, which the
// owner published after its clear completed (its next receive waits for it), so it sees
// the clear or h_{t+2}.  Partials of step t go to slot t%3 and have one reader, which clears
// them after reading; the writer uses that slot again at step t+3, after receiving h_{t+2},
// which needed the reader's h_{t+1}, published after the clear completed.

constexpr int kWideXcds = 8, kWideRowSubs = 4, kWideKBlocks = 8;
constexpr int kWideWgs = kWideXcds * kWideRowSubs * kWideKBlocks;  // 256
constexpr int kWideHSlots = 4, kWidePSlots = 3;

// Hand-off buffers addressed as raw buffers, so that a lane moves 16 bytes in one access
// with the coherence bits of the relaxed atomics it replaces: loads sc1 (served by the
// device's coherent level, as an agent-scope atomic load), stores sc0 (XCD L2, workgroup
// scope) or sc1 (agent scope).  Each 4-byte word is written whole, and readers accept a
// word only when it is not kEmpty, so 16-byte accesses need no further ordering.
typedef unsigned u4v __attribute__((ext_vector_type(4)));
constexpr int kCpolSc0 = 1, kCpolSc1 = 16;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t wide_rsrc(const float* base, size_t words) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, (int)(4 * words), 0x00020000);
}
__device__ __forceinline__ u4v quad_load(__amdgpu_buffer_rsrc_t r, unsigned word) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)(4u * word), 0, kCpolSc1);
}
template <bool FAST>
__device__ __forceinline__ void quad_store(__amdgpu_buffer_rsrc_t r, unsigned word, u4v v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, (int)(4u * word), 0, FAST ? kCpolSc0 : kCpolSc1);
}
typedef unsigned u2v __attribute__((ext_vector_type(2)));
template <bool FAST>
__device__ __forceinline__ void pair_store(__amdgpu_buffer_rsrc_t r, unsigned word, u2v v) {
  __builtin_amdgcn_raw_buffer_store_b64(v, r, (int)(4u * word), 0, FAST ? kCpolSc0 : kCpolSc1);
}

template <bool FAST>
__device__ __forceinline__ void quad_put(__amdgpu_buffer_rsrc_t r, unsigned word, f4 v) {
  quad_store<FAST>(r, word, u4v{__float_as_uint(canon_nan(v[0])), __float_as_uint(canon_nan(v[1])),
                                __float_as_uint(canon_nan(v[2])), __float_as_uint(canon_nan(v[3]))});
}

// Four k-steps of the wide backward's products for the wave's two column tiles:
// acc[rt + 2 (k % 2)] += W[k][rt] dg[k], on v_mfma_f32_32x32x2_f32 with the W operand read
// from the accumulator register file (the compiler does not keep a 256-register operand
// block there by itself).
// Even and odd k-steps go to separate accumulators, so a product depends on the one two
// instructions back.  The leading nops separate VALU writes of the operands from the
// products' reads.
__device__ __forceinline__ void wide_ksteps4(f16v (&acc)[4], const float (&w)[4][2], f4 h) {
  asm volatile(
      "s_nop 1\n\t"
      "v_mfma_f32_32x32x2_f32 %0, %4, %12, %0\n\t"
      "v_mfma_f32_32x32x2_f32 %1, %5, %12, %1\n\t"
      "v_mfma_f32_32x32x2_f32 %2, %6, %13, %2\n\t"
      "v_mfma_f32_32x32x2_f32 %3, %7, %13, %3\n\t"
      "v_mfma_f32_32x32x2_f32 %0, %8, %14, %0\n\t"
      "v_mfma_f32_32x32x2_f32 %1, %9, %14, %1\n\t"
      "v_mfma_f32_32x32x2_f32 %2, %10, %15, %2\n\t"
      "v_mfma_f32_32x32x2_f32 %3, %11, %15, %3"
      : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3])
      : "a"(w[0][0]), "a"(w[0][1]), "a"(w[1][0]), "a"(w[1][1]), "a"(w[2][0]), "a"(w[2][1]), "a"(w[3][0]),
        "a"(w[3][1]), "v"(h[0]), "v"(h[1]), "v"(h[2]), "v"(h[3]));
}

// The same for one column tile (U = 32): k-step e of the four goes to accumulator e, so a
// product depends on the one four instructions back.
__device__ __forceinline__ void wide_ksteps4(f16v (&acc)[4], const float (&w)[4][1], f4 h) {
  asm volatile(
      "s_nop 1\n\t"
      "v_mfma_f32_32x32x2_f32 %0, %4, %8, %0\n\t"
      "v_mfma_f32_32x32x2_f32 %1, %5, %9, %1\n\t"
      "v_mfma_f32_32x32x2_f32 %2, %6, %10, %2\n\t"
      "v_mfma_f32_32x32x2_f32 %3, %7, %11, %3"
      : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3])
      : "a"(w[0][0]), "a"(w[1][0]), "a"(w[2][0]), "a"(w[3][0]), "v"(h[0]), "v"(h[1]), "v"(h[2]), "v"(h[3]));
}

// The wave's partial of 4 consecutive columns of column tile rt, register group q, from the
// accumulators: two tiles keep tile rt in acc[rt] (even k-steps) and acc[rt + 2] (odd), one
// tile keeps k-step e % 4 in acc[e % 4].
template <int RT>
__device__ __forceinline__ f4 wide_partial(const f16v (&acc)[4], int rt, int q) {
  f4 v;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int r = 4 * q + e;
    v[e] = RT == 2 ? acc[rt][r] + acc[rt + 2][r] : (acc[0][r] + acc[1][r]) + (acc[2][r] + acc[3][r]);
  }
  return v;
}

// Wait states after the last products of a step, before any instruction reads their
// accumulators (an XDL result read by VALU, LDS or memory instructions needs up to 18 on
// the 16-pass 32x32x2; the compiler cannot see inside the asm above, so it adds none).
__device__ __forceinline__ void wide_ksteps_drain(f16v (&acc)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(acc[i]));
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
  for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(acc[i]));
}

// ---------------------------------------------------------------------------------
// Persistent recurrent backward for H = 32 U (U = 64: H = 2048, configs[3]; U = 32:
// H = 1024), B <= 32: the mirror of the wide forward in rec_wide_fwd.h (_torch.py:133-150: dh_t = dout_t +
// dg_{t+1} W_s, then the cell backward).  Workgroup (x, c), blockIdx = x + 8 c, sits on XCD
// x and holds W_hh's 16U gate rows of units [4U x, +4U) (unit-interleaved) for the output
// columns (units) [U c, +U); wave w takes rows [4U w, +4U) (units [4U x + U w, +U)), U/32
// column tiles x 2U k-steps in the accumulator registers.  The rows of XCD x are the gate
// rows of the units whose cells run on XCD x, so the broadcast of a dg (4H values per batch
// row, four times h) stays inside the XCD; the partial sums of dh (H per batch row) cross
// XCDs instead.  Per iteration:
//   1. products: wave w reads a dg_{t+1} of its 4U rows from the XCD's broadcast buffer,
//      8 groups at a time (the next 8 are requested before the current ones multiply);
//   2. the four waves' partials [U columns x 32 batch] are summed in LDS and sent to the
//      reducing workgroups of the columns' XCD (c / 4): slice sl of U/8 units goes to
//      workgroup (c / 4, 8 (c % 4) + sl), whose inbox holds the 8 row XCDs' partials;
//   3. reducer lane (unit su of slice s, batch b) sums them in XCD order, adds dout_t (and
//      dh_n at t = T-1), runs the cell backward with the dc carry in a register, stores
//      dgates_t, adds it to the lane's fp64 sums over t (the bias gradients' partials,
//      _torch.py:163, written at the end) and publishes a_g dg_t (the a-scaling of W_s
//      moved to the operand) to the
//      XCD's broadcast buffer: its U/8 units x 4 gates x 32 batch are one contiguous group
//      of 16U words, gathered in LDS and written in full cache lines.
// One more product after t = 0 gives dh0.  Slots as in the forward: broadcast of iteration
// k in slot k%4, its owner clears slot (k+2)%4 after publishing; partials of iteration k in
// slot k%3, cleared by their one reader.
template <int U>
struct WideBShape {
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
};

struct WBwdArgs {
  const float* dout;    // [T][B][H]
  const float* dh_n;    // [B][H] or null
  const float* dc_n;    // [B][H] or null
  const float* c_save;  // [T+1][B][H]
  const float* gact;    // [T][B][H][4]
  const float* tanh_c;  // [T][B][H]
  const float* w_hh;
  const float* a;
  float* dgates;        // [T][B][4H]
  double* db_part;      // [B][4H]: sum over t of dgates, in fp64
  float* dh0;           // [B][H] or null
  float* dc0;           // [B][H] or null
  float* dgbuf;         // [4 slots][8 XCDs][16U rows x 32 batch]
  float* inbox;         // [3 slots][256 workgroups][INBOX]
  unsigned long long* hello;  // [8][32]
  int* err;
  int T, B, H;
  int device_scope;
  long long spin;
};

// word of (local row rho, batch b) in an XCD's broadcast buffer: wave w = rho / 4U reads
// group j (k-steps 4j .. 4j+3 of its rows) at 128U w + 256 j + 4 l
template <int U>
__device__ __forceinline__ unsigned wideb_pos(int rho, int b) {
  const int w = rho / (4 * U), rl = rho % (4 * U), i = rl >> 1, l = b + 32 * (rl & 1);
  return 128u * U * w + 256u * (i >> 2) + 4u * l + (i & 3);
}

template <int U, bool FAST>
__device__ __forceinline__ void rec_bwd_wide_body(const WBwdArgs& p, int x, int c, float* red, float* gst,
                                                  int& abort_flag) {
  using S = WideBShape<U>;
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
          wide_ksteps4(acc, wreg[jb + j],
                       f4{__uint_as_float(q[j][0]), __uint_as_float(q[j][1]), __uint_as_float(q[j][2]),
                          __uint_as_float(q[j][3])});
      };
      static_assert(S::NQ == 16 || S::NQ == 32, "two or four batches of eight groups");
      issue(qa, 0);
      if (!settle(qa, 0)) return;
      issue(qb, 8);
      mult(qa, 0);
      if (!settle(qb, 8)) return;
      if constexpr (S::NQ == 32) {
        issue(qa, 16);
        mult(qb, 8);
        if (!settle(qa, 16)) return;
        issue(qb, 24);
        mult(qa, 16);
        if (!settle(qb, 24)) return;
        mult(qb, 24);
      } else {
        mult(qb, 8);
      }
      wide_ksteps_drain(acc);
      // ---- 2. the four waves' partials summed in LDS, sent to the reducers ------------
      // D layout: lane l, register 4 q + e -> column 8 q + 4 (l/32) + e of tile ct, batch
      // l%32; red[w][column quad][batch] holds 4 columns
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<f4*>(&red[((w * (U / 4) + 8 * ct + 2 * q + hb) * 32 + l32) * 4]) =
              wide_partial<CT>(acc, ct, q);
      lds_barrier();
      if (abort_flag) return;
      if (sb < B) {
        const __amdgpu_buffer_rsrc_t d =
            wide_rsrc(p.inbox + (size_t)((k - 1) % kWidePSlots) * islot + (size_t)dst * S::INBOX, S::INBOX);
#pragma unroll
        for (int qq = 0; qq < SU / 4; ++qq) {
          f4 sum = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ww = 0; ww < 4; ++ww)
            sum = sum + *reinterpret_cast<const f4*>(&red[((ww * (U / 4) + (SU / 4) * c4 + qq) * 32 + sb) * 4]);
          quad_put<false>(d, (unsigned)(x * 32 * SU + sb * SU + 4 * qq), sum);
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
      const size_t e = (size_t)cb * H + unit;
      float dh = (k > 0 ? dsum : (p.dh_n ? p.dh_n[e] : 0.f)) + p.dout[(size_t)t * plane + e];
      const f4 ga = *reinterpret_cast<const f4*>(p.gact + ((size_t)t * plane + e) * 4);
      cell_bwd(dh, dc, p.c_save[(size_t)t * plane + e], ga[0], ga[1], ga[2], ga[3], p.tanh_c[(size_t)t * plane + e], d);
      float* const dg = p.dgates + (size_t)t * plane4 + (size_t)cb * 4 * H + unit;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        __builtin_nontemporal_store(d[g], dg + (size_t)g * H);
        dbacc[g] += (double)d[g];
      }
    }
    // gather: rows 4 (SU c + su) + g of this XCD are word GROUP c + (wideb_pos - GROUP c) of
    // the buffer; absent batch rows publish 0
    if (reducer) {
#pragma unroll
      for (int g = 0; g < 4; ++g)
        gst[wideb_pos<U>(4 * (SU * c + su) + g, cb) - (unsigned)S::GROUP * c] = c_ok ? canon_nan(ag[g] * d[g]) : 0.f;
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
__device__ void poison_wide_bwd(const WBwdArgs& p, int x, int c) {
  using S = WideBShape<U>;
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
__global__ __launch_bounds__(256, 1) void rec_bwd_wide(WBwdArgs p) {
  using S = WideBShape<U>;
  extern __shared__ float wide_lds[];  // wave partials, then the gathered dg group (padded: one workgroup per CU)
  __shared__ int abort_flag;
  const int x = blockIdx.x % kWideXcds, c = blockIdx.x / kWideXcds;
  if (threadIdx.x == 0) abort_flag = 0;
  const bool fast = agree_placement(p.hello + (size_t)x * (kWideRowSubs * kWideKBlocks), c,
                                    kWideRowSubs * kWideKBlocks, p.spin, &abort_flag, p.err) &&
                    !p.device_scope;
  if (!abort_flag) {
    if (fast)
      rec_bwd_wide_body<U, true>(p, x, c, wide_lds, wide_lds + 4 * S::RED, abort_flag);
    else
      rec_bwd_wide_body<U, false>(p, x, c, wide_lds, wide_lds + 4 * S::RED, abort_flag);
  }
  lds_barrier();
  if (abort_flag) poison_wide_bwd<U>(p, x, c);
}
