// Persistent recurrent forward for a large hidden size (H = 32 U with U = 64, i.e. H = 2048,
// configs[3]), B <= 32.  Included by recurrent.hip: it shares that file's hand-off
// helpers and its device error word.
//
// W_hh (a-scaled) stays in registers for the whole launch: 64 MiB at H = 2048 is 256 KB per
// CU over 256 workgroups, where the per-step path streams it from the Infinity Cache every
// step (_torch.py:111-120 runs one h W_hh^T product per step).  Workgroup (x, r, kb),
// blockIdx = x + 8 (8 r + kb), sits on XCD x:
//   rows: the four gates of units [4U x + U r, +U) (4U gate rows, unit-interleaved);
//   k:    units [4U kb, +4U); wave w takes [4U kb + U w, +U).
// Wave w holds its 4U x U block of W in registers (U^2 / 16 per lane: 256 at U = 64) and
// multiplies it with h_{t-1}[32 batch][its U units] on v_mfma_f32_32x32x2_f32 (M = gate
// rows, N = batch, 4U/32 row tiles x U/2 k-steps).  Per step:
//   1. receive: wave w reads h block (kb, w) (the 32 x U values that row group (kb, w)
//      publishes) -- from another XCD for 7 of 8 workgroups;
//   2. products; the four waves' partials go to LDS and are summed there;
//   3. the workgroup's partial for the 8 slices of U/8 units goes to the 8 workgroups
//      (x, r, j) of its row group, one slice each (XCD-local);
//   4. lane (unit su of slice kb, batch b) sums the 8 partials of its slice in source
//      order, runs the cell and publishes h_t[b][unit] in h block (x, r).
// Hand-off words are 4-byte values that start out kEmpty, as in the other persistent
// kernels.  h blocks cross XCDs: device-scope stores and loads.  Partials stay on the XCD:
// workgroup-scope stores (sc0) when every member of the row group runs on the group's XCD.
//
// Slots.  h_t goes to slot t%4 of its block; after publishing h_t the owner clears its word
// in slot (t+2)%4.  Every workgroup's step-t products need h_{t-1} of all H units (the 8
// workgroups of a row group cover all k), and every unit's h_{t-1} needed the partials of
// its row group at t-1, which read h_{t-2} of all units: so when the owner publishes h_t,
// every reader has read h_{t-2}.  A reader of h_{t+2} read the owner's h_{t+1} first, which
// the owner published after its clear completed (its next receive waits for it), so it sees
// the clear or h_{t+2}.  Partials of step t go to slot t%3 and have one reader, which clears
// them after reading; the writer uses that slot again at step t+3, after receiving h_{t+2},
// which needed the reader's h_{t+1}, published after the clear completed.

constexpr int kWideXcds = 8, kWideRowSubs = 4, kWideKBlocks = 8;
constexpr int kWideWgs = kWideXcds * kWideRowSubs * kWideKBlocks;  // 256
constexpr int kWideHSlots = 4, kWidePSlots = 3;

template <int U>
struct WideShape {
  static constexpr int KS = U / 2;          // k-steps of 2 per wave
  static constexpr int RT = 4 * U / 32;     // row tiles of 32 gate rows
  static constexpr int SU = U / 8;          // units per slice
  static constexpr int CELLS = SU * 32;     // cell lanes (slice units x 32 batch)
  static constexpr int HW = 32 * U;         // words of an h block
  static constexpr int PW = SU * 32 * 4;    // words of one partial slice (one source)
  static constexpr int IW = kWideKBlocks * PW;  // inbox words of a workgroup (8 sources)
  static constexpr int RED_BYTES = 4 * U * 32 * 16;  // LDS: [wave][unit][batch] f4
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
  float* hbuf;    // [4 slots][8 x][4 r][HW] h blocks
  float* inbox;   // [3 slots][256 workgroups][8 sources][PW] partial slices
  unsigned long long* hello;  // [8][32] placement words
  int* err;
  int T, B, H;
  int device_scope;  // 1: partials with device-scope stores too
  long long spin;
};

// Word of (batch b, unit kk of the block) in an h block: lane l = b + 32 (kk % 2) of a reader
// wave loads the 8-byte pairs (kk/2 = 2j, 2j + 1) at 128 j + 2 l.
__device__ __forceinline__ unsigned wide_hpos(int b, int kk) {
  const int i = kk >> 1, l = b + 32 * (kk & 1);
  return 128u * (i >> 1) + 2u * l + (i & 1);
}

// Polls the lane's N 16-byte groups until no word is kEmpty (groups with expect false are
// skipped).  Returns false after raising the error flags when the spin limit runs out.
template <int N>
__device__ __forceinline__ bool quads_wait(const float* base, const unsigned (&off)[N], bool expect, f4 (&v)[N],
                                           long long spin, int* abort_flag, int* err) {
  auto load = [&](int i) {
    const unsigned long long* p = byte_at(reinterpret_cast<const unsigned long long*>(base), 4u * off[i]);
    const unsigned long long lo = __hip_atomic_load(const_cast<unsigned long long*>(p), __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT);
    const unsigned long long hi = __hip_atomic_load(const_cast<unsigned long long*>(p + 1), __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT);
    v[i] = f4{__uint_as_float((unsigned)lo), __uint_as_float((unsigned)(lo >> 32)), __uint_as_float((unsigned)hi),
              __uint_as_float((unsigned)(hi >> 32))};
  };
  auto full = [&](int i) {
    return __float_as_uint(v[i][0]) != kEmpty && __float_as_uint(v[i][1]) != kEmpty &&
           __float_as_uint(v[i][2]) != kEmpty && __float_as_uint(v[i][3]) != kEmpty;
  };
  bool need[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    need[i] = expect;
    v[i] = f4{0.f, 0.f, 0.f, 0.f};
    if (need[i]) load(i);
  }
  const long long t0 = wall_clock64();
  while (true) {
    bool ok = true;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      need[i] = need[i] && !full(i);
      ok = ok && !need[i];
    }
    if (__all(ok)) return true;
    if (wall_clock64() - t0 > spin) {
      raise_abort(abort_flag, err);
      return false;
    }
#pragma unroll
    for (int i = 0; i < N; ++i)
      if (need[i]) load(i);
  }
}

template <bool FAST>
__device__ __forceinline__ void quad_put(float* base, unsigned off, f4 v) {
  unsigned long long* p = byte_at(reinterpret_cast<unsigned long long*>(base), 4u * off);
  const unsigned long long lo = (unsigned long long)__float_as_uint(canon_nan(v[0])) |
                                ((unsigned long long)__float_as_uint(canon_nan(v[1])) << 32);
  const unsigned long long hi = (unsigned long long)__float_as_uint(canon_nan(v[2])) |
                                ((unsigned long long)__float_as_uint(canon_nan(v[3])) << 32);
  if constexpr (FAST) {
    __hip_atomic_store(p, lo, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    __hip_atomic_store(p + 1, hi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  } else {
    __hip_atomic_store(p, lo, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(p + 1, hi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

template <bool FAST>
__device__ __forceinline__ void quad_clear(float* base, unsigned off) {
  unsigned long long* p = byte_at(reinterpret_cast<unsigned long long*>(base), 4u * off);
  if constexpr (FAST) {
    __hip_atomic_store(p, kEmpty2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    __hip_atomic_store(p + 1, kEmpty2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  } else {
    __hip_atomic_store(p, kEmpty2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(p + 1, kEmpty2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// One k-step of the wide products: acc[rt] += W[rt] h for the RT row tiles, on
// v_mfma_f32_32x32x2_f32 with the W operand read from the accumulator register file (the
// compiler does not keep a 256-register operand block there by itself).  The leading nops
// separate the VALU writes of h and of the zeroed accumulators from the products' reads; the
// RT accumulators are independent, so a tile's next product is RT products behind.
template <int RT>
__device__ __forceinline__ void wide_kstep(f16v (&acc)[RT], const float (&w)[RT], float h) {
  static_assert(RT == 8, "eight row tiles (U = 64)");
  asm volatile(
      "s_nop 1\n\t"
      "v_mfma_f32_32x32x2_f32 %0, %8, %16, %0\n\t"
      "v_mfma_f32_32x32x2_f32 %1, %9, %16, %1\n\t"
      "v_mfma_f32_32x32x2_f32 %2, %10, %16, %2\n\t"
      "v_mfma_f32_32x32x2_f32 %3, %11, %16, %3\n\t"
      "v_mfma_f32_32x32x2_f32 %4, %12, %16, %4\n\t"
      "v_mfma_f32_32x32x2_f32 %5, %13, %16, %5\n\t"
      "v_mfma_f32_32x32x2_f32 %6, %14, %16, %6\n\t"
      "v_mfma_f32_32x32x2_f32 %7, %15, %16, %7"
      : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]), "+v"(acc[4]), "+v"(acc[5]), "+v"(acc[6]),
        "+v"(acc[7])
      : "a"(w[0]), "a"(w[1]), "a"(w[2]), "a"(w[3]), "a"(w[4]), "a"(w[5]), "a"(w[6]), "a"(w[7]), "v"(h));
}

// Wait states after the last products of a step, before any instruction reads their
// accumulators (an XDL result read by VALU, LDS or memory instructions needs up to 18 on
// the 16-pass 32x32x2; the compiler cannot see inside the asm above, so it adds none).
template <int RT>
__device__ __forceinline__ void wide_kstep_drain(f16v (&acc)[RT]) {
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) asm volatile("" : "+v"(acc[rt]));
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) asm volatile("" : "+v"(acc[rt]));
}

template <int U, bool FAST>
__device__ __forceinline__ void rec_fwd_wide_body(const WFwdArgs& p, int x, int r, int kb, f4* red,
                                                  int& abort_flag) {
  using S = WideShape<U>;
  const int T = p.T, B = p.B, H = p.H;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hb = lane >> 5, l32 = lane & 31;

  // W_hh block of this wave: row tile rt, k-step i -> row m = l%32 of the tile (unit offset
  // (32 rt + m) / 4, gate m % 4), k = kbase + 2 i + l/32.  It is held unscaled (a register
  // that only feeds the products can live in the accumulator file); the gate's a scales the
  // summed product in the cell.
  const int ubase = 4 * U * x + U * r;  // first unit of the workgroup's rows
  const int kbase = 4 * U * kb + U * w;  // first k (unit) of the wave's block
  float wreg[S::KS][S::RT];
#pragma unroll
  for (int rt = 0; rt < S::RT; ++rt) {
    const int rho = 32 * rt + l32, g = rho & 3, u = ubase + (rho >> 2);
    const float* row = p.w_hh + ((size_t)g * H + u) * H + kbase + hb;
#pragma unroll
    for (int i = 0; i < S::KS; ++i) wreg[i][rt] = row[2 * i];
  }
#pragma unroll
  for (int i = 0; i < S::KS; ++i)
#pragma unroll
    for (int rt = 0; rt < S::RT; ++rt) asm volatile("" : "+a"(wreg[i][rt]));  // held in the accumulator file

  // cell lane: tid < CELLS -> unit su of this workgroup's slice kb, batch cb
  const int su = tid >> 5, cb = tid & 31;
  const bool cell = tid < S::CELLS;
  const bool c_ok = cell && cb < B;
  const int unit = ubase + S::SU * kb + su;  // < H
  float c_reg = 0.f, bs[4] = {0.f, 0.f, 0.f, 0.f}, ag[4] = {0.f, 0.f, 0.f, 0.f};
  if (c_ok) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      ag[g] = p.a[g];
      bs[g] = ag[g] * p.b_hh[g * H + unit];
    }
    const size_t e = (size_t)cb * H + unit;
    c_reg = p.c0 ? p.c0[e] : 0.f;
    p.h_save[e] = p.h0 ? p.h0[e] : 0.f;
    p.c_save[e] = c_reg;
  }
  const size_t plane = (size_t)B * H, plane4 = 4 * plane;
  const int me = blockIdx.x;
  // partial slice j of this workgroup -> inbox of workgroup (x, r, j), source kb
  const unsigned pofs = (unsigned)kb * S::PW + 4u * (su * 32 + cb);
  const size_t inbox_slot = (size_t)kWideWgs * S::IW;
  // own h word in block (x, r) and the words this wave reads in block (kb, w)
  const size_t hblock = S::HW, hslot = (size_t)kWideXcds * kWideRowSubs * S::HW;
  float* const hown = p.hbuf + (size_t)(x * kWideRowSubs + r) * hblock;
  const float* const hsrc = p.hbuf + (size_t)(kb * kWideRowSubs + w) * hblock;
  const unsigned hpos = wide_hpos(cb, S::SU * kb + su);
  const bool h_ok = l32 < B;  // batch column of this lane in the products

  float gin[4] = {0.f, 0.f, 0.f, 0.f};
  for (int t = 0; t < T; ++t) {
    // ---- 1. h_{t-1} of the wave's k block: hreg[i] = h[l%32][kbase + 2i + l/32] ----
    float hreg[S::KS];
    if (t == 0) {
#pragma unroll
      for (int i = 0; i < S::KS; ++i) {
        hreg[i] = (h_ok && p.h0) ? p.h0[(size_t)l32 * H + kbase + 2 * i + hb] : 0.f;
        asm volatile("" : "+v"(hreg[i]));
      }
    } else {
      constexpr int NW = S::KS;  // words per lane (pairs loaded together)
      const float* src = hsrc + (size_t)((t - 1) % kWideHSlots) * hslot;
      bool need[NW / 2];
      unsigned long long v2[NW / 2];
#pragma unroll
      for (int j = 0; j < NW / 2; ++j) {
        need[j] = h_ok;
        v2[j] = 0ull;
        if (need[j])
          v2[j] = __hip_atomic_load(
              const_cast<unsigned long long*>(byte_at(reinterpret_cast<const unsigned long long*>(src), 4u * (128u * j + 2u * lane))),
              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      const long long t0 = wall_clock64();
      while (true) {
        bool ok = true;
#pragma unroll
        for (int j = 0; j < NW / 2; ++j) {
          need[j] = need[j] && ((unsigned)v2[j] == kEmpty || (unsigned)(v2[j] >> 32) == kEmpty);
          ok = ok && !need[j];
        }
        if (__all(ok)) break;
        if (wall_clock64() - t0 > p.spin) {
          raise_abort(&abort_flag, p.err);
          return;
        }
#pragma unroll
        for (int j = 0; j < NW / 2; ++j)
          if (need[j])
            v2[j] = __hip_atomic_load(
                const_cast<unsigned long long*>(byte_at(reinterpret_cast<const unsigned long long*>(src), 4u * (128u * j + 2u * lane))),
                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
#pragma unroll
      for (int j = 0; j < NW / 2; ++j) {
        hreg[2 * j] = h_ok ? __uint_as_float((unsigned)v2[j]) : 0.f;
        hreg[2 * j + 1] = h_ok ? __uint_as_float((unsigned)(v2[j] >> 32)) : 0.f;
        asm volatile("" : "+v"(hreg[2 * j]), "+v"(hreg[2 * j + 1]));
      }
    }
    // this step's input projection for the cell lanes (used after the products)
    if (c_ok) {
      const float* g = p.gih + (size_t)t * plane4 + (size_t)cb * 4 * H + unit;
#pragma unroll
      for (int gt = 0; gt < 4; ++gt) gin[gt] = __builtin_nontemporal_load(g + (size_t)gt * H);
    }

    // ---- 2. products, the four waves' partials summed through LDS ------------------
    f16v acc[S::RT];
#pragma unroll
    for (int rt = 0; rt < S::RT; ++rt) acc[rt] = f16v{};
#pragma unroll
    for (int i = 0; i < S::KS; ++i) wide_kstep<S::RT>(acc, wreg[i], hreg[i]);
    wide_kstep_drain<S::RT>(acc);
    // D layout: lane l, register 4 q + g -> gate row 8 q + 4 (l/32) + g of the tile, batch l%32;
    // with unit-interleaved rows that is gate g of unit offset 8 rt + 2 q + l/32
#pragma unroll
    for (int rt = 0; rt < S::RT; ++rt)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        red[(w * U + 8 * rt + 2 * q + hb) * 32 + l32] =
            f4{acc[rt][4 * q], acc[rt][4 * q + 1], acc[rt][4 * q + 2], acc[rt][4 * q + 3]};
    lds_barrier();
    if (abort_flag) return;

    // ---- 3. the workgroup's partial of slice j -> workgroup (x, r, j) ---------------
    if (cell) {
      float* const ib = p.inbox + (size_t)(t % kWidePSlots) * inbox_slot;
#pragma unroll 2
      for (int j = 0; j < kWideKBlocks; ++j) {
        const int uo = S::SU * j + su;
        const f4 s = ((red[(0 * U + uo) * 32 + cb] + red[(1 * U + uo) * 32 + cb]) +
                      red[(2 * U + uo) * 32 + cb]) + red[(3 * U + uo) * 32 + cb];
        const int dst = x + kWideXcds * (r * kWideKBlocks + j);
        if (cb < B) quad_put<FAST>(ib + (size_t)dst * S::IW, pofs, s);
      }
    }
    lds_barrier();  // red is read; the next step may overwrite it

    // ---- 4. the cell of slice kb: sum the 8 sources, activate, publish h_t ---------
    if (cell) {
      float* const ib = p.inbox + (size_t)(t % kWidePSlots) * inbox_slot + (size_t)me * S::IW;
      unsigned offs[kWideKBlocks];
#pragma unroll
      for (int sidx = 0; sidx < kWideKBlocks; ++sidx) offs[sidx] = (unsigned)sidx * S::PW + 4u * (su * 32 + cb);
      f4 v[kWideKBlocks];
      if (!quads_wait<kWideKBlocks>(ib, offs, c_ok, v, p.spin, &abort_flag, p.err)) return;
      if (c_ok) {
#pragma unroll
        for (int sidx = 0; sidx < kWideKBlocks; ++sidx) quad_clear<FAST>(ib, offs[sidx]);
        f4 z = v[0];
#pragma unroll
        for (int sidx = 1; sidx < kWideKBlocks; ++sidx) z = z + v[sidx];
        float act[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) act[g] = sigmoid_f((gin[g] + ag[g] * z[g]) + bs[g]);
        const float c = act[1] * c_reg + act[0] * act[2];
        const float tc = tanh_f(c);
        const float h = act[3] * tc;
        c_reg = c;
        word_put<false>(hown + (size_t)(t % kWideHSlots) * hslot, hpos, canon_nan(h));
        const size_t e = (size_t)cb * H + unit;
        __builtin_nontemporal_store(h, p.h_save + (size_t)(t + 1) * plane + e);
        __builtin_nontemporal_store(c, p.c_save + (size_t)(t + 1) * plane + e);
        __builtin_nontemporal_store(tc, p.tanh_c + (size_t)t * plane + e);
        __builtin_nontemporal_store(f4{act[0], act[1], act[2], act[3]},
                                    reinterpret_cast<f4*>(p.gact + ((size_t)t * plane + e) * 4));
        word_put<false>(hown + (size_t)((t + 2) % kWideHSlots) * hslot, hpos, __uint_as_float(kEmpty));
      }
    }
  }
}

// After an abort the cell lanes set their outputs (rows 0..T of h_save / c_save, the
// activations of every step) to NaN.
template <int U>
__device__ void poison_wide_fwd(const WFwdArgs& p, int x, int r, int kb) {
  using S = WideShape<U>;
  const int tid = threadIdx.x, su = tid >> 5, cb = tid & 31;
  if (tid >= S::CELLS || cb >= p.B) return;
  const int unit = 4 * U * x + U * r + S::SU * kb + su;
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
  extern __shared__ f4 wide_red[];  // [4 waves][U units][32 batch] (keeps one workgroup per CU)
  __shared__ int abort_flag;
  const int x = blockIdx.x % kWideXcds, loc = blockIdx.x / kWideXcds;
  const int r = loc / kWideKBlocks, kb = loc % kWideKBlocks;
  if (threadIdx.x == 0) abort_flag = 0;
  const bool fast = agree_placement(p.hello + (size_t)x * (kWideRowSubs * kWideKBlocks), loc,
                                    kWideRowSubs * kWideKBlocks, p.spin, &abort_flag, p.err) &&
                    !p.device_scope;
  if (!abort_flag) {
    if (fast)
      rec_fwd_wide_body<U, true>(p, x, r, kb, wide_red, abort_flag);
    else
      rec_fwd_wide_body<U, false>(p, x, r, kb, wide_red, abort_flag);
  }
  lds_barrier();
  if (abort_flag) poison_wide_fwd<U>(p, x, r, kb);
}
