// Persistent recurrent forward for H = 32 U (U = 64: H = 2048, configs[3]; U = 32:
// H = 1024), B <= 32, with W_hh resident in the accumulator registers.  Included by
// recurrent.hip after rec_wide.h, whose grid, hand-off helpers and slot rotation it uses.
//
// Workgroup (x, r, kb), blockIdx = x + 8 (8 r + kb), sits on XCD x:
//   rows: the four gates of units [4U x + U r, +U) (4U gate rows, unit-interleaved); wave w
//         takes units [U w / 4, +U/4) of them;
//   k:    units [4U kb, +4U), all of them for every wave.
// The 8 workgroups (x, r, 0..7) are a row group: together they hold all H k units of the
// row group's 4U gate rows, each one's products are a partial over its k block, and each
// runs the cells of one slice of U/8 of the group's units, summing the 8 partials of its
// slice in source order.  Partials stay on the XCD; h blocks (one row group's units) cross
// XCDs: every workgroup reads the 4 blocks of its k units.
//
// The batch is split into two chains of 16 rows (chain c: batch rows 16c .. 16c+15).  The
// rows of the two chains never meet, so while the h hand-off of one chain crosses the
// XCDs, the other chain's products keep the matrix cores busy.  Products run on
// v_mfma_f32_16x16x4_f32 (M = 16 gate rows, N = the chain's 16 batch rows, K = 4), which
// has the same rate as 32x32x2 and wastes nothing on a 16-row chain.  Every wave runs one
// fixed sequence per step t, with chain 1 half a step behind chain 0:
//   1. first half of chain 0's products with h0_{t-1} (LDS);
//   2. chain 1's cells of step t-1: the 8 partials of each (unit, batch row), sent in step 7
//      of the previous iteration (their hand-off ran under steps 8 and 1), the cell,
//      h1_{t-1} gathered and published;
//   3. second half of chain 0's products; its partials sent to the cell workgroups;
//   4. h1_{t-1} of the wave's block received into LDS (its hand-off ran under step 3);
//   5. first half of chain 1's products;
//   6. chain 0's cells of step t (partials sent in step 3), h0_t published;
//   7. second half of chain 1's products, partials sent;
//   8. h0_t received into LDS (its hand-off ran under step 7).
// Chain 1's cells of the last step follow the loop.  At H = 2048 the words of the receives
// in steps 4 and 8 are requested before the sends of steps 3 and 7.
//
// Wave w holds the rows of units [U w / 4, +U/4) (U/16 row tiles of 16) for all 4U k of the
// workgroup (U k-steps of 4): U^2/16 values per lane in the accumulator registers.  Inside
// each quad j of four k-steps (16 k), lane l's k-step e takes k = 16 j + 4 (l/16) + e, so a
// lane's four values of a quad are four consecutive k (one 16-byte load of W per row tile).
//   A operand (W): lane l of k-step 4j + e, tile rt: row 16 rt + l%16 of the wave (unit
//     4 rt + (l%16)/4, gate l%4), k = 4U kb + 16 j + 4 (l/16) + e.
//   B operand (h): lane l of k-step 4j + e: h[batch 16c + l%16][k = 4U kb + 16 j + 4 (l/16) + e].
//   D: lane l, register g: gate g of unit 4 rt + l/16, batch row l%16 of the chain.
// LDS holds one buffer per chain: quad j of lane l at [j][l].  An h block (16 batch rows x U
// units of a row group, one chain) has the same layout: unit u (of the block) of batch row n
// is word 256 (u/16) + 4 l + u%4 with l = 16 ((u%16)/4) + n; wave w receives block (kb, w),
// LDS quads [w U/16, +U/16).  Row-group member kb publishes its slice of U/8 units
// (u0 = U kb / 8 onwards) as whole quads: lanes l < U/2 write words 256 (u0/16) +
// 64 ((u0%16)/4) + 4 l .. +3.
// Slots per chain: h_t in slot t%4, the owner clears (t+2)%4 after publishing; partials of
// step t in slot t%3, cleared by their one reader.  The cell lanes' h values are gathered in
// LDS and published by one wave in whole cache lines (scattered 4-byte device-scope stores
// from 256 lanes took about 1 us longer to reach the readers on the other XCDs).
template <int U>
struct WideFShape {
  static_assert(U == 32 || U == 64, "H = 1024 or H = 2048");
  static constexpr int RT = U / 16;        // row tiles of 16 per wave
  static constexpr int NQ = U / 4;         // quads of 4 k-steps per lane and chain (U k-steps)
  static constexpr int BQ = U / 16;        // quads per lane of one h block
  static constexpr int SU = U / 8;         // units per slice
  static constexpr int CELLS = SU * 16;    // cells per chain and workgroup
  static constexpr int CPW = CELLS / 4;    // cells per wave (lanes 0 .. CPW-1)
  static constexpr int HB = 256 * BQ;      // words of one h block
  static constexpr int PS = SU * 16 * 4;   // words of one source's partial slice
  static constexpr int IW = 8 * PS;        // inbox words per chain and workgroup
  static constexpr int LDS_BYTES = 2 * NQ * 64 * 16;  // one h buffer per chain
};

struct WFwdArgs {
  const float* gih;   // [T][B][4H]: x W_ih^T + b_ih
  const float* w_hh;  // [4H][H]
  const float* b_hh;
  const float* a;
  const float* h0;
  const float* c0;
  float* h_save;
  float* c_save;
  float* gact;
  float* tanh_c;
  float* hbuf;    // [4 slots][2 chains][32 row groups][HB] h blocks
  float* inbox;   // [3 slots][2 chains][256 workgroups][IW] partial slices
  unsigned long long* hello;  // [8][32] placement words
  int* err;
  int T, B, H;
  int device_scope;  // 1: partials with device-scope stores too
  long long spin;
};

template <int U, bool FAST>
__device__ __forceinline__ void rec_fwd_wide_body(const WFwdArgs& p, int x, int r, int kb, f4* hs,
                                                   int& abort_flag) {
  using S = WideFShape<U>;
  constexpr int RT = S::RT, NQ = S::NQ, BQ = S::BQ, SU = S::SU;
  const int T = p.T, B = p.B, H = p.H;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lq = lane >> 4;
  const int nch = B > 16 ? 2 : 1;  // chains with at least one batch row

  const int ubase = 4 * U * x + U * r;  // first unit of the workgroup's rows
  const int kbase = 4 * U * kb;         // first k (unit) of the workgroup's k block
  // W block: quad j, k-step e, tile rt -> row (gate l%4, unit ubase + U w/4 + 4 rt + (l%16)/4),
  // k = kbase + 16 j + 4 (l/16) + e; unscaled (a scales the summed product in the cell).  A
  // lane's quad is 16 consecutive bytes of its row: one load of four rows' 64-byte segments
  // per 16 lanes (4-byte loads of k-steps 4 apart touched 16 rows per instruction and took
  // the first step 31 us after launch at configs[3], against 10 us for the backward's slice)
  float wreg[NQ][4][RT];
  {
    const float* rows[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int u = ubase + U / 4 * w + 4 * rt + (l16 >> 2);
      rows[rt] = p.w_hh + ((size_t)(l16 & 3) * H + u) * H + kbase + 4 * lq;
    }
    const bool w16 = reinterpret_cast<uintptr_t>(p.w_hh) % 16 == 0;  // uniform
#pragma unroll
    for (int j8 = 0; j8 < NQ; j8 += 4) {
#pragma unroll
      for (int j = j8; j < j8 + 4; ++j)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          f4 v;
          if (w16) {
            v = *reinterpret_cast<const f4*>(rows[rt] + 16 * j);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = rows[rt][16 * j + e];
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) wreg[j][e][rt] = v[e];
        }
#pragma unroll
      for (int j = j8; j < j8 + 4; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) asm volatile("" : "+a"(wreg[j][e][rt]));  // held in the accumulator file
    }
  }

  // cell lane: lanes < CPW of wave w -> cell ci = CPW w + lane: unit su = ci / 16 of slice kb,
  // batch row n = ci % 16 of each chain
  const bool cell = lane < S::CPW;
  const int ci = S::CPW * w + lane, su = ci >> 4, cn = ci & 15;
  const int unit = ubase + SU * kb + su;  // < H
  float ag[4] = {0.f, 0.f, 0.f, 0.f}, bs[4] = {0.f, 0.f, 0.f, 0.f}, c_reg[2] = {0.f, 0.f};
  bool c_ok[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) c_ok[c] = cell && 16 * c + cn < B;
  if (cell) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      ag[g] = p.a[g];
      bs[g] = ag[g] * p.b_hh[g * H + unit];
    }
  }
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    if (c_ok[c]) {
      const size_t e = (size_t)(16 * c + cn) * H + unit;
      c_reg[c] = p.c0 ? p.c0[e] : 0.f;
      p.h_save[e] = p.h0 ? p.h0[e] : 0.f;
      p.c_save[e] = c_reg[c];
    }
  }
  const size_t plane = (size_t)B * H, plane4 = 4 * plane;
  const int me = blockIdx.x;
  // h buffers: [4 slots][2 chains][32 row groups][HB]; inboxes: [3 slots][2 chains][256][IW]
  auto hblock = [&](int slot, int c, int g) { return p.hbuf + ((size_t)(slot * 2 + c) * 32 + g) * S::HB; };
  auto inbox = [&](int slot, int c, int wg) { return p.inbox + ((size_t)(slot * 2 + c) * kWideWgs + wg) * S::IW; };
  // each chain's published h values, in the order of the group; entries of absent batch
  // rows are never written and publish 0
  __shared__ __attribute__((aligned(16))) float hst[2][128];
  if (tid < 128) hst[0][tid] = hst[1][tid] = 0.f;
  // the published quads of this workgroup's slice inside block (x, r)
  const unsigned pub_u0 = SU * kb, pub_off = 256u * (pub_u0 / 16) + 64u * ((pub_u0 % 16) / 4);

  // h of chain c for the step after `tin` (its values h_tin) into the chain's LDS buffer:
  // wave w takes block (kb, w) and polls until none of its words is kEmpty.  recv_h0 takes
  // h0 instead (tin = -1).
  auto recv_h0 = [&](int c) {
    f4* const buf = hs + (size_t)c * NQ * 64;
    const bool h_ok = 16 * c + l16 < B;
#pragma unroll
    for (int j = 0; j < BQ; ++j) {
      f4 v = f4{0.f, 0.f, 0.f, 0.f};
      if (h_ok && p.h0) {
        const float* row = p.h0 + (size_t)(16 * c + l16) * H + kbase + U * w + 4 * lq;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = row[16 * j + e];
      }
      buf[(w * BQ + j) * 64 + lane] = v;
    }
  };
  auto recv_src = [&](int c, int tin) {
    return wide_rsrc(hblock(tin % kWideHSlots, c, kb * kWideRowSubs + w), S::HB);
  };
  // Poll loads are issued by every lane, unconditionally: a lane without a value reads
  // from past the end of the buffer (0, never kEmpty).
  auto recv_off = [&](int c, int j) { return 16 * c + l16 < B ? 256u * j + 4u * lane : (unsigned)S::HB; };
  // recv_issue requests the words (at H = 2048 right after the last products of a phase,
  // so that their latency overlaps the wait of the following send for those products'
  // results), recv_settle polls until none is kEmpty and writes them to LDS
  auto recv_issue = [&](int c, int tin, u4v (&q4)[BQ]) {
    const __amdgpu_buffer_rsrc_t src = recv_src(c, tin);
#pragma unroll
    for (int j = 0; j < BQ; ++j) q4[j] = quad_load(src, recv_off(c, j));
  };
  auto recv_settle = [&](int c, int tin, u4v (&q4)[BQ]) -> bool {
    f4* const buf = hs + (size_t)c * NQ * 64;
    const __amdgpu_buffer_rsrc_t src = recv_src(c, tin);
    const bool h_ok = 16 * c + l16 < B;
    const long long t0 = wall_clock64();
    while (true) {  // all of the lane's groups reloaded while any word is kEmpty
      unsigned m = 0u;
#pragma unroll
      for (int j = 0; j < BQ; ++j) m = max(m, max(max(q4[j][0], q4[j][1]), max(q4[j][2], q4[j][3])));
      if (__all(m != kEmpty)) break;
      if (wall_clock64() - t0 > p.spin) {
        raise_abort(&abort_flag, p.err);
        return false;
      }
#pragma unroll
      for (int j = 0; j < BQ; ++j) q4[j] = quad_load(src, recv_off(c, j));
    }
#pragma unroll
    for (int j = 0; j < BQ; ++j)
      buf[(w * BQ + j) * 64 + lane] =
          h_ok ? f4{__uint_as_float(q4[j][0]), __uint_as_float(q4[j][1]), __uint_as_float(q4[j][2]),
                    __uint_as_float(q4[j][3])}
               : f4{0.f, 0.f, 0.f, 0.f};
    return true;
  };

  // the input projection of chain c's cells at step t (requested before the products, used
  // by the cells after them)
  auto load_gin = [&](int c, int t, float (&gin)[4]) {
#pragma unroll
    for (int gt = 0; gt < 4; ++gt) gin[gt] = 0.f;
    if (c_ok[c]) {
      const float* g = p.gih + (size_t)t * plane4 + (size_t)(16 * c + cn) * 4 * H + unit;
#pragma unroll
      for (int gt = 0; gt < 4; ++gt) gin[gt] = __builtin_nontemporal_load(g + (size_t)gt * H);
    }
  };
  // quads [J0, J1) of chain c's products into acc
  typedef __attribute__((address_space(3))) const volatile f4 lds_vf4;
  auto products = [&](int c, auto j0c, auto j1c, f4 (&acc)[RT][2]) {
    constexpr int J0 = decltype(j0c)::value, J1 = decltype(j1c)::value;
    lds_vf4* const hv = (lds_vf4*)(hs + (size_t)c * NQ * 64);
    f4 hcur = hv[J0 * 64 + lane];
#pragma unroll
    for (int j = J0; j < J1; ++j) {
      const f4 hnext = j + 1 < J1 ? hv[(j + 1) * 64 + lane] : hcur;
      wide_quad16(acc, wreg[j], hcur);
      hcur = hnext;
    }
  };
  auto zero_acc = [&](f4 (&acc)[RT][2]) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[rt][0] = acc[rt][1] = f4{0.f, 0.f, 0.f, 0.f};
  };
  // chain c's partials of step t to the cell workgroups
  // (every lane stores: a lane of an absent batch row past the descriptor's end, where the
  // store is dropped, so that the stores' count in the completion counter does not depend
  // on the lane)
  auto send = [&](int c, int t, f4 (&acc)[RT][2]) {
    wide_drain16<RT>(acc);
    const bool mine = 16 * c + l16 < B;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int ur = U / 4 * w + 4 * rt + lq;  // unit of the row group
      const int dst = x + kWideXcds * (r * kWideKBlocks + ur / SU);
      // one descriptor over every workgroup's inbox of the slot (the same for all lanes: a
      // descriptor that differs between lanes makes the compiler loop over its values)
      const __amdgpu_buffer_rsrc_t d = wide_rsrc(inbox(t % kWidePSlots, c, 0), (size_t)kWideWgs * S::IW);
      quad_put<FAST>(d, mine ? (unsigned)(dst * S::IW + kb * S::PS) + 4u * ((ur % SU) * 16 + l16) : (unsigned)(kWideWgs * S::IW),
                     acc[rt][0] + acc[rt][1]);
    }
  };

  // chain c's cells of step t: polls until none of the cells' 8 partials is kEmpty, clears
  // the partials' slot, runs the cells and publishes h_t
  auto cell_off = [&](int s) { return (unsigned)s * S::PS + 4u * (su * 16 + cn); };
  auto cell_poll = [&](int c, int s) { return c_ok[c] ? cell_off(s) : (unsigned)S::IW; };
  auto cells = [&](int c, int t, const float (&gin)[4]) -> bool {
    if (cell) {
      const __amdgpu_buffer_rsrc_t ib = wide_rsrc(inbox(t % kWidePSlots, c, me), S::IW);
      u4v v[kWideKBlocks];
#pragma unroll
      for (int s = 0; s < kWideKBlocks; ++s) v[s] = quad_load(ib, cell_poll(c, s));
      const long long t0 = wall_clock64();
      while (true) {  // all eight reloaded while any word is kEmpty
        unsigned m = 0u;
#pragma unroll
        for (int s = 0; s < kWideKBlocks; ++s) m = max(m, max(max(v[s][0], v[s][1]), max(v[s][2], v[s][3])));
        if (__all(m != kEmpty)) break;
        if (wall_clock64() - t0 > p.spin) {
          raise_abort(&abort_flag, p.err);
          return false;
        }
#pragma unroll
        for (int s = 0; s < kWideKBlocks; ++s) v[s] = quad_load(ib, cell_poll(c, s));
      }
      if (c_ok[c]) {
#pragma unroll
        for (int s = 0; s < kWideKBlocks; ++s) quad_store<FAST>(ib, cell_off(s), u4v{kEmpty, kEmpty, kEmpty, kEmpty});
        auto as_f4 = [](u4v q) {
          return f4{__uint_as_float(q[0]), __uint_as_float(q[1]), __uint_as_float(q[2]), __uint_as_float(q[3])};
        };
        f4 z = as_f4(v[0]);
#pragma unroll
        for (int s = 1; s < kWideKBlocks; ++s) z = z + as_f4(v[s]);
        float act[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) act[g] = sigmoid_f((gin[g] + ag[g] * z[g]) + bs[g]);
        const float cc = act[1] * c_reg[c] + act[0] * act[2];
        const float tc = tanh_f(cc);
        const float h = act[3] * tc;
        c_reg[c] = cc;
        hst[c][4 * (16 * (su >> 2) + cn) + (su & 3)] = canon_nan(h);
        const size_t e = (size_t)(16 * c + cn) * H + unit;
        __builtin_nontemporal_store(h, p.h_save + (size_t)(t + 1) * plane + e);
        __builtin_nontemporal_store(cc, p.c_save + (size_t)(t + 1) * plane + e);
        __builtin_nontemporal_store(tc, p.tanh_c + (size_t)t * plane + e);
        __builtin_nontemporal_store(f4{act[0], act[1], act[2], act[3]},
                                    reinterpret_cast<f4*>(p.gact + ((size_t)t * plane + e) * 4));
      }
    }
    lds_barrier();  // the chain's h values are gathered
    if (abort_flag) return false;
    if (w == 0) {  // publish them, then clear the slot of two steps ago
      float* const own = hblock(0, c, x * kWideRowSubs + r) + pub_off;
      const size_t hslot = (size_t)2 * 32 * S::HB;  // words between slots
      const __amdgpu_buffer_rsrc_t hp = wide_rsrc(own + (size_t)(t % kWideHSlots) * hslot, 256);
      const __amdgpu_buffer_rsrc_t hc = wide_rsrc(own + (size_t)((t + 2) % kWideHSlots) * hslot, 256);
      // U/2 lanes, one quad each; the other lanes store past the descriptors' end (dropped),
      // so that no store depends on a lane condition
      const unsigned lw = lane < 4 * SU ? 4u * lane : 256u;
      const f4 hv = *reinterpret_cast<const f4*>(&hst[c][4 * min(lane, 4 * SU - 1)]);
      quad_store<false>(hp, lw, u4v{__float_as_uint(hv[0]), __float_as_uint(hv[1]), __float_as_uint(hv[2]),
                                    __float_as_uint(hv[3])});
      quad_store<false>(hc, lw, u4v{kEmpty, kEmpty, kEmpty, kEmpty});
    }
    return true;
  };

  using IC0 = std::integral_constant<int, 0>;
  using ICH = std::integral_constant<int, NQ / 2>;
  using ICN = std::integral_constant<int, NQ>;
  // both chains' h0 into LDS
  recv_h0(0);
  if (nch > 1) recv_h0(1);
  lds_barrier();
  float gin0[4], gin1[4];
  // One step; NCH chains, FIRST: t == 0 (chain 1 has no step t-1).  h0_t is received at the
  // last step too (every workgroup publishes it).
  auto step = [&](int t, auto nchc, auto firstc) __attribute__((always_inline)) -> bool {
    constexpr int NCH = decltype(nchc)::value;
    constexpr bool FIRST = decltype(firstc)::value;
    f4 acc[RT][2];
    load_gin(0, t, gin0);
    zero_acc(acc);
    products(0, IC0{}, ICH{}, acc);                                     // 1
    if constexpr (NCH > 1 && !FIRST) {                                  // 2
      if (!cells(1, t - 1, gin1)) return false;
    }
    products(0, ICH{}, ICN{}, acc);                                     // 3
    // At H = 2048 a receive's words are requested before the preceding send (configs[3]
    // 2.43 -> 2.40 ms per step); at H = 1024 that measured slower (1.048 -> 1.067 ms) and
    // the words are requested after it.
    constexpr bool kAhead = U == 64;
    u4v hq[BQ];
    if constexpr (NCH > 1 && !FIRST && kAhead) {
      wide_drain16<RT>(acc);  // the products' last operand reads are done
      recv_issue(1, t - 1, hq);
    }
    send(0, t, acc);
    if constexpr (NCH > 1) {
      if constexpr (!FIRST) {                                           // 4
        if constexpr (!kAhead) recv_issue(1, t - 1, hq);
        if (!recv_settle(1, t - 1, hq)) return false;
        lds_barrier();
        if (abort_flag) return false;
      }
      load_gin(1, t, gin1);
      zero_acc(acc);
      products(1, IC0{}, ICH{}, acc);                                   // 5
    }
    if (!cells(0, t, gin0)) return false;                               // 6
    if constexpr (NCH > 1) {
      products(1, ICH{}, ICN{}, acc);                                   // 7
      if constexpr (kAhead) {
        wide_drain16<RT>(acc);
        recv_issue(0, t, hq);
      }
      send(1, t, acc);
      if constexpr (!kAhead) recv_issue(0, t, hq);
    } else {
      recv_issue(0, t, hq);
    }
    if (!recv_settle(0, t, hq)) return false;                           // 8
    lds_barrier();
    return !abort_flag;
  };
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using BT = std::true_type;
  using BF = std::false_type;
  if (T > 0) {
    if (nch > 1) {
      if (!step(0, I2{}, BT{})) return;
      for (int t = 1; t < T; ++t)
        if (!step(t, I2{}, BF{})) return;
      if (!cells(1, T - 1, gin1)) return;
    } else {
      for (int t = 0; t < T; ++t)
        if (!step(t, I1{}, BF{})) return;
    }
  }
}

// After an abort the cell lanes set their outputs (rows 0..T of h_save / c_save, the
// activations of every step) to NaN: lane (unit su, batch row cb) of the workgroup's slice.
template <int U>
__device__ void poison_wide_fwd(const WFwdArgs& p, int x, int r, int kb) {
  constexpr int SU = WideFShape<U>::SU;
  const int tid = threadIdx.x, su = tid >> 5, cb = tid & 31;
  if (tid >= 32 * SU || cb >= p.B) return;
  const int unit = 4 * U * x + U * r + SU * kb + su;
  const float nan = __uint_as_float(0x7FC00000u);
  const size_t plane = (size_t)p.B * p.H, e = (size_t)cb * p.H + unit;
  for (int t = 0; t <= p.T; ++t) {
    p.h_save[t * plane + e] = nan;
    p.c_save[t * plane + e] = nan;
    if (t < p.T) {
      p.tanh_c[t * plane + e] = nan;
      *reinterpret_cast<f4*>(p.gact + (t * plane + e) * 4) = f4{nan, nan, nan, nan};
    }
  }
}

template <int U>
__global__ __launch_bounds__(256, 1) void rec_fwd_wide(WFwdArgs p) {
  extern __shared__ f4 wide_hs[];  // one h buffer per chain (sized to keep one workgroup per CU)
  __shared__ int abort_flag;
  const int x = blockIdx.x % kWideXcds, loc = blockIdx.x / kWideXcds;
  const int r = loc / kWideKBlocks, kb = loc % kWideKBlocks;
  if (threadIdx.x == 0) abort_flag = 0;
  const bool fast = agree_placement(p.hello + (size_t)x * (kWideRowSubs * kWideKBlocks), loc,
                                    kWideRowSubs * kWideKBlocks, p.spin, &abort_flag, p.err) &&
                    !p.device_scope;
  if (!abort_flag) {
    if (fast)
      rec_fwd_wide_body<U, true>(p, x, r, kb, wide_hs, abort_flag);
    else
      rec_fwd_wide_body<U, false>(p, x, r, kb, wide_hs, abort_flag);
  }
  lds_barrier();
  if (abort_flag) poison_wide_fwd<U>(p, x, r, kb);
}
