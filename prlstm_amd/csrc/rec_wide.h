// Persistent recurrent kernels for a large hidden size, H = 32 U with U = 64 (H = 2048,
// configs[3]) or U = 32 (H = 1024, the reference's published T64 B32 D512 H1024 shape),
// B <= 32.  Included by recurrent.hip: they share that file's hand-off helpers and its
// device error word.  This file holds what the wide forward (rec_wide_fwd.h) and the
// backwards share -- the grid, the hand-off buffers and their access helpers, the slot
// rotation, the 16x16x4 product helper -- and the two-chain backward run at H = 2048 (the
// H = 1024 backward is the single-chain form of rec_wide_bwd32.h).
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
template <bool FAST>
__device__ __forceinline__ void quad_put(__amdgpu_buffer_rsrc_t r, unsigned word, f4 v) {
  quad_store<FAST>(r, word, u4v{__float_as_uint(canon_nan(v[0])), __float_as_uint(canon_nan(v[1])),
                                __float_as_uint(canon_nan(v[2])), __float_as_uint(canon_nan(v[3]))});
}

// Four k-steps of one quad of the wide products: acc[rt][e % 2] += W[e][rt] v[e] on
// v_mfma_f32_16x16x4_f32 (M = 16 rows of tile rt, N = 16 batch rows, K = 4), W read from the
// accumulator registers (the compiler does not keep a 256-register operand block there by
// itself), v the lane's operand values of the four k-steps.  A product depends on the one
// 2 RT instructions back.  The leading nop separates VALU writes of the operand from the
// products' reads.  Forward: rows are gate rows, v = h; backward: rows are W columns
// (units), v = a_g dg.
__device__ __forceinline__ void wide_quad16(f4 (&acc)[4][2], const float (&w)[4][4], f4 h) {
  asm volatile(
      "s_nop 1\n\t"
      "v_mfma_f32_16x16x4_f32 %0, %8, %24, %0\n\t"
      "v_mfma_f32_16x16x4_f32 %2, %9, %24, %2\n\t"
      "v_mfma_f32_16x16x4_f32 %4, %10, %24, %4\n\t"
      "v_mfma_f32_16x16x4_f32 %6, %11, %24, %6\n\t"
      "v_mfma_f32_16x16x4_f32 %1, %12, %25, %1\n\t"
      "v_mfma_f32_16x16x4_f32 %3, %13, %25, %3\n\t"
      "v_mfma_f32_16x16x4_f32 %5, %14, %25, %5\n\t"
      "v_mfma_f32_16x16x4_f32 %7, %15, %25, %7\n\t"
      "v_mfma_f32_16x16x4_f32 %0, %16, %26, %0\n\t"
      "v_mfma_f32_16x16x4_f32 %2, %17, %26, %2\n\t"
      "v_mfma_f32_16x16x4_f32 %4, %18, %26, %4\n\t"
      "v_mfma_f32_16x16x4_f32 %6, %19, %26, %6\n\t"
      "v_mfma_f32_16x16x4_f32 %1, %20, %27, %1\n\t"
      "v_mfma_f32_16x16x4_f32 %3, %21, %27, %3\n\t"
      "v_mfma_f32_16x16x4_f32 %5, %22, %27, %5\n\t"
      "v_mfma_f32_16x16x4_f32 %7, %23, %27, %7"
      : "+v"(acc[0][0]), "+v"(acc[0][1]), "+v"(acc[1][0]), "+v"(acc[1][1]), "+v"(acc[2][0]), "+v"(acc[2][1]),
        "+v"(acc[3][0]), "+v"(acc[3][1])
      : "a"(w[0][0]), "a"(w[0][1]), "a"(w[0][2]), "a"(w[0][3]), "a"(w[1][0]), "a"(w[1][1]), "a"(w[1][2]),
        "a"(w[1][3]), "a"(w[2][0]), "a"(w[2][1]), "a"(w[2][2]), "a"(w[2][3]), "a"(w[3][0]), "a"(w[3][1]),
        "a"(w[3][2]), "a"(w[3][3]), "v"(h[0]), "v"(h[1]), "v"(h[2]), "v"(h[3]));
}
__device__ __forceinline__ void wide_quad16(f4 (&acc)[2][2], const float (&w)[4][2], f4 h) {
  asm volatile(
      "s_nop 1\n\t"
      "v_mfma_f32_16x16x4_f32 %0, %4, %12, %0\n\t"
      "v_mfma_f32_16x16x4_f32 %2, %5, %12, %2\n\t"
      "v_mfma_f32_16x16x4_f32 %1, %6, %13, %1\n\t"
      "v_mfma_f32_16x16x4_f32 %3, %7, %13, %3\n\t"
      "v_mfma_f32_16x16x4_f32 %0, %8, %14, %0\n\t"
      "v_mfma_f32_16x16x4_f32 %2, %9, %14, %2\n\t"
      "v_mfma_f32_16x16x4_f32 %1, %10, %15, %1\n\t"
      "v_mfma_f32_16x16x4_f32 %3, %11, %15, %3"
      : "+v"(acc[0][0]), "+v"(acc[0][1]), "+v"(acc[1][0]), "+v"(acc[1][1])
      : "a"(w[0][0]), "a"(w[0][1]), "a"(w[1][0]), "a"(w[1][1]), "a"(w[2][0]), "a"(w[2][1]), "a"(w[3][0]),
        "a"(w[3][1]), "v"(h[0]), "v"(h[1]), "v"(h[2]), "v"(h[3]));
}

// Wait states after the last products of a phase, before any instruction reads their
// accumulators (the compiler cannot see inside the asm above, so it adds none).
template <int RT>
__device__ __forceinline__ void wide_drain16(f4 (&acc)[RT][2]) {
#pragma unroll
  for (int i = 0; i < RT; ++i) asm volatile("" : "+v"(acc[i][0]), "+v"(acc[i][1]));
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
  for (int i = 0; i < RT; ++i) asm volatile("" : "+v"(acc[i][0]), "+v"(acc[i][1]));
}

// ---------------------------------------------------------------------------------
// Persistent recurrent backward for H = 32 U, B <= 32, run for U = 64 (H = 2048, configs[3];
// H = 1024 runs the single-chain form of rec_wide_bwd32.h): the mirror of the wide forward
// in rec_wide_fwd.h (_torch.py:133-150:
// dh_t = dout_t + dg_{t+1} W_s, then the cell backward).  Workgroup (x, c), blockIdx =
// x + 8 c, sits on XCD x and holds W_hh's 16U gate rows of units [4U x, +4U) (unit-
// interleaved) for the output columns (units) [U c, +U); wave w takes rows [4U w, +4U)
// (units [4U x + U w, +U)).  The rows of XCD x are the gate rows of the units whose cells
// run on XCD x, so the broadcast of a dg stays inside the XCD; the partial sums of dh cross
// XCDs instead.
//
// As in the forward, the batch is split into two chains of 16 rows that never meet, run
// half an iteration apart, so that one chain's hand-offs cross the chip while the other's
// products run.  Per chain and iteration k (k = 0 .. T; the cell of step t = T-1-k):
//   P. products: wave w reads a_g dg_{t+1} of its 4U rows and the chain's 16 batch rows
//      from the XCD's broadcast buffer of the chain (U/4 16-byte groups per lane) and runs
//      them in two halves; v_mfma_f32_16x16x4_f32 with M = 16 columns, N = 16 batch rows,
//      K = 4 rows;
//   S. the four waves' partials [U columns x 16 batch] are summed in LDS and sent to the
//      reducing workgroups of the columns' XCD (c / 4): slice sl of U/8 units goes to
//      workgroup (c / 4, 8 (c % 4) + sl), whose inbox holds the 8 row XCDs' partials;
//   R. reducer lane (unit su of slice c, batch row) sums them in XCD order, adds dout_t (and
//      dh_n at k = 0), runs the cell backward with the dc carry in a register, stores
//      dgates_t, adds it to the lane's fp64 sums over t (the bias gradients' partials,
//      _torch.py:163, written at the end) and publishes a_g dg_t (the a-scaling of W_s
//      moved to the operand): the slice's U/8 units x 4 gates x 16 batch rows are one
//      contiguous group of 64 U/8 words of the chain's buffer, gathered in LDS and written
//      in full cache lines.
// Every wave runs one fixed sequence per iteration k, chain 1 half an iteration behind:
//   1. first half of chain 0's products;   2. chain 1's R of iteration k-1;
//   3. second half of chain 0's products, its S;   4. first half of chain 1's products;
//   5. chain 0's R of iteration k;   6. second half of chain 1's products, its S.
// At k = 0 only step 5 runs; chain 1's R of iteration T follows the loop.  R of iteration
// T writes dh0 (the last products' sum), dc0 and the bias partials instead of a cell.  The
// cell inputs of an R (dout, c, tanh c, the gate activations) are requested after the
// operand of the products before it has arrived, so their HBM latency runs under those
// products and not under R's poll (requested just before the poll, the wait for the poll
// included them: configs[3] +55 us; a phase ahead: -26 us).
// Slots per chain as in the forward: the broadcast of iteration k in slot k%4, its owner
// clears slot (k+2)%4 after publishing; partials of iteration k in slot (k-1)%3, cleared
// by their one reader.
//
// Layouts per chain.  Operand of wave w, k-step i (rows 4U w + 4i .. +3), lane l: row
// 4U w + 4i + l/16, batch row l%16; group j holds k-steps 4j .. 4j+3 of each lane, the XCD
// buffer word 64U w + 256 j + 4 l + i%4.  The reducer group of slice c (units SU c .. +SU
// of the XCD's 4U, SU = U/8) starts at word 64 SU c; unit su, gate g, batch row b is word
// 256 (su / 4) + 4 (16 g + b) + su % 4 of it.
template <int U>
struct WideBShape {
  static constexpr int CT = U / 16;            // column tiles of 16 per wave
  static constexpr int SU = U / 8;             // units per reducer slice
  static constexpr int NQ = U / 4;             // operand groups of a wave per chain (U k-steps of 4)
  static constexpr int QS = SU / 4;            // 16-byte quads of one (slice, batch row) partial
  static constexpr int XBUF = 256 * U;         // words of an XCD's broadcast buffer per chain (16U rows x 16)
  static constexpr int INBOX = 8 * 16 * SU;    // inbox words of a reducer per slot and chain: [src x][batch][unit]
  static constexpr int GROUP = 64 * SU;        // words of a reducer's published group per chain
  static constexpr int RED = 16 * U;           // floats of one wave's partials per chain [U columns][16 batch]
  static constexpr int REDUCERS = 16 * SU;     // reducer lanes per chain (threads 128 c .. +REDUCERS)
  static constexpr int SENDERS = 8 * 16 * QS;  // sender lanes per chain
  static constexpr int LDS_BYTES = 4 * (2 * 4 * RED + 2 * GROUP);  // per chain: wave partials, dg group
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
  float* dgbuf;         // [4 slots][2 chains][8 XCDs][XBUF]
  float* inbox;         // [3 slots][2 chains][256 workgroups][INBOX]
  unsigned long long* hello;  // [8][32]
  int* err;
  int T, B, H;
  int device_scope;
  long long spin;
};

template <int U, bool FAST>
__device__ __forceinline__ void rec_bwd_wide_body(const WBwdArgs& p, int x, int c, float* red, float* gst,
                                                  int& abort_flag) {
  using S = WideBShape<U>;
  constexpr int CT = S::CT, SU = S::SU, NQ = S::NQ, NH = NQ / 2;
  const int T = p.T, B = p.B, H = p.H;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lq = lane >> 4;
  const int ubase = 4 * U * x;  // first unit of the XCD's rows
  const int nch = B > 16 ? 2 : 1;

  // W_hh^T block of this wave: group j, k-step e, column tile ct -> row 4U w + 4 (4j + e) +
  // l/16 (unit ubase + U w + 4j + e, gate l/16), column U c + 16 ct + l%16; unscaled, a
  // multiplies the dg operand instead
  float wreg[NQ][4][CT];
  {
    const float* const wb = p.w_hh + ((size_t)lq * H + ubase + U * w) * H + U * c + l16;
#pragma unroll
    for (int j8 = 0; j8 < NQ; j8 += 4) {
#pragma unroll
      for (int j = j8; j < j8 + 4; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int ct = 0; ct < CT; ++ct) wreg[j][e][ct] = wb[(size_t)(4 * j + e) * H + 16 * ct];
#pragma unroll
      for (int j = j8; j < j8 + 4; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int ct = 0; ct < CT; ++ct) asm volatile("" : "+a"(wreg[j][e][ct]));  // held in the accumulator file
    }
  }

  // reducer role: threads 128 rc .. +REDUCERS serve chain rc; index ri -> unit su of this
  // workgroup's slice (slice c of XCD x: units ubase + SU c + su), batch row 16 rc + cb
  const int rc = tid >> 7, ri = tid & 127;
  const bool reducer = ri < S::REDUCERS;
  const int su = ri >> 4, cb = ri & 15, brow = 16 * rc + cb;
  const bool c_ok = reducer && brow < B;
  const int unit = ubase + SU * c + su;
  float ag[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) ag[g] = p.a[g];
  float dc = 0.f;
  double dbacc[4] = {0.0, 0.0, 0.0, 0.0};
  if (c_ok && p.dc_n) dc = p.dc_n[(size_t)brow * H + unit];
  const size_t plane = (size_t)B * H, plane4 = 4 * plane;
  // sender role: thread -> slice c4 of the workgroup's columns, batch row sb of the chain,
  // quad qq of the slice's SU units; the slice goes to reducer (c / 4, 8 (c % 4) + c4)
  const bool sender = tid < S::SENDERS;
  const int c4 = tid / (16 * S::QS), sb = (tid % (16 * S::QS)) / S::QS, qq = tid % S::QS;
  const int dst = (c >> 2) + kWideXcds * (8 * (c & 3) + c4);
  auto xbuf = [&](int k, int ch) { return p.dgbuf + ((size_t)((k % kWideHSlots) * 2 + ch) * kWideXcds + x) * S::XBUF; };
  auto inbox = [&](int k, int ch, int wg) {
    return p.inbox + ((size_t)((k % kWidePSlots) * 2 + ch) * kWideWgs + wg) * S::INBOX;
  };

  // P: chain ch's operand of iteration k (a_g dg of iteration k-1), all NQ groups of the
  // wave, received with the first half of the products (the second half then waits for no
  // memory)
  auto fetch_issue = [&](int ch, int k, u4v (&q)[NQ]) {
    const __amdgpu_buffer_rsrc_t src = wide_rsrc(xbuf(k - 1, ch) + 64 * U * w, 64 * U);
#pragma unroll
    for (int j = 0; j < NQ; ++j) q[j] = quad_load(src, 256u * j + 4u * lane);
  };
  auto fetch_settle = [&](int ch, int k, u4v (&q)[NQ]) -> bool {
    const __amdgpu_buffer_rsrc_t src = wide_rsrc(xbuf(k - 1, ch) + 64 * U * w, 64 * U);
    const long long t0 = wall_clock64();
    while (true) {  // all of the lane's groups reloaded while any word is kEmpty
      unsigned m = 0u;
#pragma unroll
      for (int j = 0; j < NQ; ++j) m = max(m, max(max(q[j][0], q[j][1]), max(q[j][2], q[j][3])));
      if (__all(m != kEmpty)) return true;
      if (wall_clock64() - t0 > p.spin) {
        raise_abort(&abort_flag, p.err);
        return false;
      }
#pragma unroll
      for (int j = 0; j < NQ; ++j) q[j] = quad_load(src, 256u * j + 4u * lane);
    }
  };
  // half HF of the products
  auto mult = [&](const u4v (&q)[NQ], auto hfc, f4 (&acc)[CT][2]) {
    constexpr int J0 = decltype(hfc)::value * NH;
#pragma unroll
    for (int j = J0; j < J0 + NH; ++j)
      wide_quad16(acc, wreg[j],
                  f4{__uint_as_float(q[j][0]), __uint_as_float(q[j][1]), __uint_as_float(q[j][2]),
                     __uint_as_float(q[j][3])});
  };
  auto zero_acc = [&](f4 (&acc)[CT][2]) {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) acc[ct][0] = acc[ct][1] = f4{0.f, 0.f, 0.f, 0.f};
  };
  // S: chain ch's partials of iteration k summed over the waves, sent to the reducers.  D of
  // tile ct: lane l, register i -> column 16 ct + 4 (l/16) + i, batch row l%16; the chain's
  // red[w][column quad][batch row] holds 4 columns
  auto fetch = [&](int ch, int k, u4v (&q)[NQ]) -> bool {
    fetch_issue(ch, k, q);
    return fetch_settle(ch, k, q);
  };
  auto send = [&](int ch, int k, f4 (&acc)[CT][2]) -> bool {
    wide_drain16<CT>(acc);
    float* const rb = red + ch * 4 * S::RED;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
      *reinterpret_cast<f4*>(&rb[((w * (U / 4) + 4 * ct + lq) * 16 + l16) * 4]) = acc[ct][0] + acc[ct][1];
    lds_barrier();
    if (abort_flag) return false;
    {
      // one descriptor over every workgroup's inbox of the slot (the same for all lanes: a
      // descriptor that differs between lanes makes the compiler loop over its values);
      // every lane stores, lanes without a partial past the descriptor's end (dropped), so
      // that the store's count in the completion counter does not depend on the lane
      const __amdgpu_buffer_rsrc_t d = wide_rsrc(inbox(k - 1, ch, 0), (size_t)kWideWgs * S::INBOX);
      const bool mine = sender && 16 * ch + sb < B;
      const int cq = S::QS * c4 + qq;
      f4 sum = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ww = 0; ww < 4; ++ww) sum = sum + *reinterpret_cast<const f4*>(&rb[((ww * (U / 4) + (mine ? cq : 0)) * 16 + (mine ? sb : 0)) * 4]);
      quad_put<false>(d, mine ? (unsigned)(dst * S::INBOX + x * 16 * SU + sb * SU + 4 * qq) : (unsigned)(kWideWgs * S::INBOX), sum);
    }
    return true;
  };
  // R: chain ch's reducers of iteration k
  struct CellIn {
    float dout, c, tc, dhn;
    f4 ga;
  };
  // the cell's inputs of chain ch's step t = T-1-k, requested a product phase before the
  // reducer uses them (lanes without a cell read clamped addresses)
  auto cell_in = [&](int ch, int k, CellIn& in) {
    in = CellIn{0.f, 0.f, 0.f, 0.f, f4{0.f, 0.f, 0.f, 0.f}};
    if (rc == ch && k < T) {
      const size_t ec = c_ok ? (size_t)brow * H + unit : 0, tp = (size_t)(T - 1 - k) * plane + ec;
      in.dout = p.dout[tp];
      in.ga = *reinterpret_cast<const f4*>(p.gact + tp * 4);
      in.c = p.c_save[tp];
      in.tc = p.tanh_c[tp];
      if (k == 0 && p.dh_n) in.dhn = p.dh_n[ec];
    }
    __builtin_amdgcn_sched_barrier(0);  // requested here, not sunk to their use
  };
  auto reduce = [&](int ch, int k, const CellIn& in) -> bool {
    const bool mine = rc == ch;  // wave-uniform
    float dsum = 0.f;
    if (k > 0 && mine && c_ok) {
      const __amdgpu_buffer_rsrc_t ib = wide_rsrc(inbox(k - 1, ch, blockIdx.x), S::INBOX);
      unsigned v[8];
      const long long t0 = wall_clock64();
      while (true) {
        unsigned m = 0u;
#pragma unroll
        for (int sx = 0; sx < 8; ++sx) {
          v[sx] = __builtin_amdgcn_raw_buffer_load_b32(ib, (int)(4u * (sx * 16 * SU + cb * SU + su)), 0, kCpolSc1);
          m = max(m, v[sx]);
        }
        if (__all(m != kEmpty)) break;
        if (wall_clock64() - t0 > p.spin) {
          raise_abort(&abort_flag, p.err);
          return false;
        }
      }
#pragma unroll
      for (int sx = 0; sx < 8; ++sx)
        __builtin_amdgcn_raw_buffer_store_b32(kEmpty, ib, (int)(4u * (sx * 16 * SU + cb * SU + su)), 0, kCpolSc1);
      dsum = __uint_as_float(v[0]);
#pragma unroll
      for (int sx = 1; sx < 8; ++sx) dsum += __uint_as_float(v[sx]);
    }
    if (k == T) {  // dh of h0, the carry into c0, the bias partials
      if (mine && c_ok) {
        const size_t e = (size_t)brow * H + unit;
        if (p.dh0) p.dh0[e] = dsum;
        if (p.dc0) p.dc0[e] = dc;
#pragma unroll
        for (int g = 0; g < 4; ++g) p.db_part[(size_t)brow * 4 * H + g * H + unit] = dbacc[g];
      }
      return true;
    }
    const int t = T - 1 - k;
    float d[4] = {0.f, 0.f, 0.f, 0.f};
    if (mine && c_ok) {
      const float dh = (k > 0 ? dsum : in.dhn) + in.dout;
      cell_bwd(dh, dc, in.c, in.ga[0], in.ga[1], in.ga[2], in.ga[3], in.tc, d);
      float* const dg = p.dgates + (size_t)t * plane4 + (size_t)brow * 4 * H + unit;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        __builtin_nontemporal_store(d[g], dg + (size_t)g * H);
        dbacc[g] += (double)d[g];
      }
    }
    // gather the group; absent batch rows publish 0
    float* const gs = gst + ch * S::GROUP;
    if (mine && reducer) {
#pragma unroll
      for (int g = 0; g < 4; ++g) gs[256 * (su >> 2) + 4 * (16 * g + cb) + (su & 3)] = c_ok ? canon_nan(ag[g] * d[g]) : 0.f;
    }
    lds_barrier();
    if (abort_flag) return false;
    if (tid < S::GROUP / 4) {  // publish, then clear the slot of two iterations ago
      const f4 qv = *reinterpret_cast<const f4*>(&gs[4 * tid]);
      const __amdgpu_buffer_rsrc_t bp = wide_rsrc(xbuf(k, ch) + (size_t)S::GROUP * c, S::GROUP);
      quad_store<FAST>(bp, 4u * tid, u4v{__float_as_uint(qv[0]), __float_as_uint(qv[1]), __float_as_uint(qv[2]),
                                         __float_as_uint(qv[3])});
      const __amdgpu_buffer_rsrc_t bc = wide_rsrc(xbuf(k + 2, ch) + (size_t)S::GROUP * c, S::GROUP);
      quad_store<FAST>(bc, 4u * tid, u4v{kEmpty, kEmpty, kEmpty, kEmpty});
    }
    return true;
  };

  using IC0 = std::integral_constant<int, 0>;
  using IC1 = std::integral_constant<int, 1>;
  // one iteration k >= 1 with NCH chains (instantiated per NCH: no branches between phases)
  auto step = [&](int k, auto nchc) __attribute__((always_inline)) -> bool {
    constexpr int NCH = decltype(nchc)::value;
    f4 acc[CT][2];
    u4v q[NQ];
    CellIn in;
    zero_acc(acc);
    if (!fetch(0, k, q)) return false;  // 1
    if constexpr (NCH > 1) cell_in(1, k - 1, in);
    mult(q, IC0{}, acc);
    if constexpr (NCH > 1) {
      if (!reduce(1, k - 1, in)) return false;  // 2
    }
    mult(q, IC1{}, acc);  // 3
    if constexpr (NCH > 1) {
      // chain 1's operand requested before chain 0's send, whose first instructions wait
      // for the last products' results (q's last readers were issued 24 wait states before)
      wide_drain16<CT>(acc);
      fetch_issue(1, k, q);
    }
    if (!send(0, k, acc)) return false;
    if constexpr (NCH > 1) {
      zero_acc(acc);
      if (!fetch_settle(1, k, q)) return false;  // 4
      cell_in(0, k, in);
      mult(q, IC0{}, acc);
    } else {
      cell_in(0, k, in);
    }
    if (!reduce(0, k, in)) return false;  // 5
    if constexpr (NCH > 1) {
      mult(q, IC1{}, acc);  // 6
      if (!send(1, k, acc)) return false;
    }
    return true;
  };
  {
    CellIn in0;
    cell_in(0, 0, in0);
    if (!reduce(0, 0, in0)) return;
  }
  if (nch > 1) {
    for (int k = 1; k <= T; ++k)
      if (!step(k, std::integral_constant<int, 2>{})) return;
    CellIn inT;
    cell_in(1, T, inT);
    reduce(1, T, inT);
  } else {
    for (int k = 1; k <= T; ++k)
      if (!step(k, std::integral_constant<int, 1>{})) return;
  }
}

// After an abort the reducer lanes set what they own to NaN: dgates of their unit and batch
// row at every step, the bias partials, and dh0 / dc0.
template <int U>
__device__ void poison_wide_bwd(const WBwdArgs& p, int x, int c) {
  using S = WideBShape<U>;
  const int tid = threadIdx.x, ri = tid & 127, su = ri >> 4, brow = 16 * (tid >> 7) + (ri & 15);
  if (ri >= S::REDUCERS || brow >= p.B) return;
  const int unit = 4 * U * x + S::SU * c + su, H = p.H;
  const float nan = __uint_as_float(0x7FC00000u);
  const size_t e = (size_t)brow * H + unit;
  if (p.dh0) p.dh0[e] = nan;
  if (p.dc0) p.dc0[e] = nan;
  for (int g = 0; g < 4; ++g) p.db_part[(size_t)brow * 4 * H + g * H + unit] = (double)nan;
  for (int t = 0; t < p.T; ++t)
    for (int g = 0; g < 4; ++g) p.dgates[((size_t)t * p.B + brow) * 4 * H + g * H + unit] = nan;
}

template <int U>
__global__ __launch_bounds__(256, 1) void rec_bwd_wide(WBwdArgs p) {
  using S = WideBShape<U>;
  extern __shared__ float wide_lds[];  // per chain: wave partials; then per chain the dg group (padded: one workgroup per CU)
  __shared__ int abort_flag;
  const int x = blockIdx.x % kWideXcds, c = blockIdx.x / kWideXcds;
  if (threadIdx.x == 0) abort_flag = 0;
  const bool fast = agree_placement(p.hello + (size_t)x * (kWideRowSubs * kWideKBlocks), c,
                                    kWideRowSubs * kWideKBlocks, p.spin, &abort_flag, p.err) &&
                    !p.device_scope;
  if (!abort_flag) {
    if (fast)
      rec_bwd_wide_body<U, true>(p, x, c, wide_lds, wide_lds + 2 * 4 * S::RED, abort_flag);
    else
      rec_bwd_wide_body<U, false>(p, x, c, wide_lds, wide_lds + 2 * 4 * S::RED, abort_flag);
  }
  lds_barrier();
  if (abort_flag) poison_wide_bwd<U>(p, x, c);
}
