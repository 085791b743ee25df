// Internal helpers shared by the HeadStartLSTM HIP kernels (gfx950 / CDNA4).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "../../include/hsl.h"

namespace hsl {

// ---- host-side error reporting ------------------------------------------------
int fail(int code, const char* fmt, ...);        // records text, returns code
int hip_fail(hipError_t e, const char* what);    // HSL_ERR_HIP with the HIP text
#define HSL_HIP(call)                                         \
  do {                                                        \
    hipError_t hsl_e_ = (call);                               \
    if (hsl_e_ != hipSuccess) return ::hsl::hip_fail(hsl_e_, #call); \
  } while (0)
#define HSL_CHECK(call)                    \
  do {                                     \
    int hsl_rc_ = (call);                  \
    if (hsl_rc_ != HSL_OK) return hsl_rc_; \
  } while (0)

// Shape check shared by every entry point that takes (T, B, D, H) (D = 0 where there is
// none): negative sizes are HSL_ERR_ARG, shapes beyond the 32-bit index math of the
// kernels and GEMMs are HSL_ERR_UNSUPPORTED.  `who` names the entry point in the text.
int check_shape(const char* who, int T, int B, int D, int H);

// Per-device facts queried once.
struct DeviceInfo {
  int device = -1;
  int num_cus = 0;
  int num_xcds = 8;
};
int device_info(DeviceInfo* out);

// Process-wide options (see hsl_set_recurrent_path / hsl_set_spin_timeout_us).
int recurrent_path_mode();
int exchange_scope_mode();  // 1: persistent kernels always use device-scope stores
int split_products_mode();  // 1: large A B^T products on split bf16 pieces (gemm_x6.hip)
// Timing hooks (active only after hsl_set_timing(1)): events around one launch.
enum TimingKind { kTimeRecFwd = 1, kTimeRecBwd = 2, kTimeScanFwd = 3, kTimeScanBwd = 4,
                  kTimeInputProj = 5, kTimeStepFwd = 6, kTimeStepBwd = 7 };
int timing_begin(int kind, hipStream_t s);
void timing_end(int slot, hipStream_t s);
// While one is alive, timing_begin records nothing on this thread (it creates HIP events,
// which the allocation-free entry points must not do).
struct TimingSuppress {
  TimingSuppress();
  ~TimingSuppress();
  TimingSuppress(const TimingSuppress&) = delete;
  TimingSuppress& operator=(const TimingSuppress&) = delete;
};
long long spin_timeout_ticks();   // in wall_clock64 ticks (100 MHz)
void note_recurrent_path(int path);
void note_backward_fused(int fused);  // 0, 1 (dW_hh) or 2 (dW_hh and dW_ih)

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Carves a caller-provided workspace into aligned pieces.
struct Carver {
  char* base;
  size_t cap;
  size_t off = 0;
  Carver(void* b, size_t c) : base(static_cast<char*>(b)), cap(c) {}
  template <class T>
  T* take(size_t count) {
    off = align_up(off, 256);
    T* p = reinterpret_cast<T*>(base ? base + off : nullptr);
    off += count * sizeof(T);
    return p;
  }
  bool fits() const { return off <= cap; }
};

// ---- GEMM (gemm.hip) ------------------------------------------------------------
struct GemmDesc {
  const float* A;
  const float* B;
  const float* bias;  // [N] or null
  float* C;
  int M, N, K, lda, ldb, ldc;
  int trans_a, trans_b;
  int acc64;  // 1: fp64 accumulation across BK-slices (long K reductions)
};
size_t gemm_ws_bytes_layout(int M, int N, int K, int acc64, int trans_a, int trans_b);
size_t gemm_ws_bytes(int M, int N, int K, int acc64);
// Full product with optional split-K through ws (ws may be null when ws_bytes==0).
int gemm_run(const GemmDesc& d, void* ws, size_t ws_bytes, hipStream_t s);
// C = op(A) B with a 16-bit B ([K][ldb] row-major, d.B; fmt 0 = bf16, 1 = fp16): a bf16 B
// goes straight to the split kernel where that applies; otherwise B is widened into
// `widen` (K * ldb floats) and the fp32 product runs.
int gemm_run_b16(const GemmDesc& d, int fmt, float* widen, void* ws, size_t ws_bytes, hipStream_t s);
int widen16(const void* src, float* dst, size_t n, int fmt, hipStream_t s);
// Split-K partial sums kept as fp32 [used][M][N] in `partials` (room for `splits`
// planes); *used receives the number of planes written (<= splits).  Used by the
// fused epilogues of the weight gradients.
int gemm_partials(const GemmDesc& d, float* partials, int splits, hipStream_t s, int* used);
// Partial planes to provide for an A^T B product given to gemm_partials (fp32 or split-bf16).
int gemm_tn_planes(int M, int N, int K);
// C[M][N] (row stride ldc) = sum over the `splits` fp32 planes P[z][M][N], added in fp64
// (+ bias[N] when non-null).
int splitk_reduce(const float* P, int splits, const float* bias, float* C, int M, int N, int ldc, hipStream_t s);
int gemm_pick_splits(int M, int N, int K, int acc64);
// C[M][N] = A[M][K] . B[N][K]^T (+ bias[N]) with 16-bit A and B (fmt 0 bf16, 1 fp16),
// fp32 accumulation and output (gemm_b16.hip).
// Longest k-range of one split of a split-bf16 A^T B / A B product (its fp32 running sum
// is folded every 64 k; the splits are added in fp64).  4096 put configs[4] dW_ih at 1.48x
// the parity tolerance against fp64 (the CPU's own fp32 product: 1.12x); 2048 gives 1.08x.
constexpr int kSplitLongKRun = 2048;
bool gemm_x6_applies(int M, int N, int K);  // C = A B^T products (input projection)
int gemm_x6_longk_splits(int M, int N, int K);  // C = A^T B or A B: split count, 0 = not taken
// Split-bf16 product (gemm_x6.hip): any layout but trans_a = trans_b = 1;
// with partial != nullptr the k-splits go to planes [used][M][N] (no bias).
// b_bf16: B holds bf16 values (one piece each; trans_b = 0 only), three products per step.
int gemm_x6_run(const float* A, const void* B, const float* bias, float* C, float* partial, int M, int N, int K,
                int lda, int ldb, int ldc, int trans_a, int trans_b, int splits, hipStream_t s, int* used,
                int b_bf16 = 0);
// dW = A^T B written with its finalisation (one split of the split-bf16 kernel): row r of
// C = a_group[r / group_rows] * (A^T B)[r], and per group the fp64 sum of W . (A^T B) in
// parts[group][*parts] of dotp.  *parts = 0: the shape does not qualify and nothing ran.
int gemm_x6_wgrad_fin(const float* A, const float* B, float* C, const float* a_group, int group_rows,
                      const float* W, double* dotp, size_t dotp_cap, int M, int N, int K, int lda, int ldb, int ldc,
                      hipStream_t s, int* parts);
int gemm_b16_run(const void* A, const void* B, const float* bias, float* C, int M, int N, int K, int lda, int ldb,
                 int ldc, int fmt, hipStream_t s);

// ---- shared finalisation (recurrent.hip) ------------------------------------------
// db = sum_b db_part[b][:] ; db_ih = db ; db_hh = a_g db ; da[g] = sum_{n in g} rowdot[n] + b_hh[n] db[n].
// Any of rowdot, b_hh, a, db_hh, da may be null (parallel mode only wants db_ih).
// rowdot [4H] (or dotp [4][dot_parts], from gemm_x6_wgrad_fin): the fp64 sums of W_hh . dW_hh_s
int bias_grads_from_parts(const double* db_part, int B, const double* rowdot, const float* b_hh, const float* a,
                          float* db_ih, float* db_hh, float* da, int H, hipStream_t s, const double* dotp = nullptr,
                          int dot_parts = 0);
int zero_words(unsigned long long* p, size_t n, hipStream_t s);
int copy_f32(float* dst, const float* src, size_t n, hipStream_t s);

// ---- device math ----------------------------------------------------------------
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));

// exp(x) = 2^t (1 + dl) with t = x*L (L = fp32 log2 e) on v_exp_f32.  t is rounded, and
// at |x| ~ 80 that rounding alone is ~64 ulp of the result, so the reduced argument
// dl = x - t ln 2 is formed in two fmas (Cody and Waite's split ln 2 = C1 + C2, C1 with
// 16 significant bits; the first fma cancels almost exactly and is computed with one
// rounding) and put back as fma(2^t, dl, 2^t), so the correction is not rounded against 1.
// |dl| < 0.35 whenever |t| < 2^24.  For |t| >= 128 the result is 0 or inf (or NaN for NaN
// x) and is returned as v_exp_f32 gives it (there dl can be infinite or NaN).  Six VALU
// operations and one transcendental.  exp_scaled_f<K>(x) = exp_f(K x) bit for bit for
// K = +-1, +-2 (x L K is x L scaled by a power of two).
template <int K>
__device__ __forceinline__ float exp_scaled_f(float x) {
  constexpr float L = 1.44269502162933349609375f * K, C1 = 0.693145751953125f, C2 = 1.428606765330187e-06f;
  const float t = x * L;
  const float dl = __builtin_fmaf(-t, C2, __builtin_fmaf(-t, C1, K * x));
  const float r = __builtin_amdgcn_exp2f(t);
  return __builtin_fabsf(t) < 128.0f ? __builtin_fmaf(r, dl, r) : r;
}
__device__ __forceinline__ float exp_f(float x) { return exp_scaled_f<1>(x); }
// sigmoid from its definition with v_rcp_f32; exp overflow gives inf and rcp(inf) = 0, so
// sigmoid(-large) -> 0 and sigmoid(+large) -> 1 without NaN.  Error: exp's, the rounding
// of 1 + e and v_rcp_f32's (about 1 ulp each).
__device__ __forceinline__ float sigmoid_f(float x) { return __builtin_amdgcn_rcpf(1.0f + exp_scaled_f<-1>(x)); }
// sigmoid(x) sigmoid(y) = 1 / ((1 + e^-x)(1 + e^-y)) with one v_rcp_f32 for both.  The
// denominators are >= 1 (or NaN), so their product is never 0 * inf; one that overflows
// gives 0.  Error: the two exps', three roundings and the rcp's.
__device__ __forceinline__ float sigmoid_prod_f(float x, float y) {
  return __builtin_amdgcn_rcpf((1.0f + exp_scaled_f<-1>(x)) * (1.0f + exp_scaled_f<-1>(y)));
}
// tanh: for |x| < 1 the odd polynomial x + x^3 P(x^2), P of degree 6 fitted to
// (tanh(x)/x - 1)/x^2 on [0, 1] by iteratively reweighted least squares in fp64 (relative
// error of the model 4.6e-9); there 1 - 2/(1 + e^{2x}) would cancel (1.7e-4 relative error
// at x = 1e-4).  For |x| >= 1, 1 - 2/(1 + e^{2|x|}) with the sign restored; it saturates to
// +-1 for large |x| (rcp(inf) = 0).  Its exp needs no argument correction: an error e in
// e^{2|x|} moves the result by 2E/(1+E)^2 e (E = e^{2|x|}), at most 0.21 e for |x| >= 1,
// and e grows only with |x| while that factor falls as 2/E.  Both sides are computed and
// one is selected, so the dependent chain is the longer of the two, not their sum.
// tanh_pos_f: the same for x >= 0 (or NaN), without the sign handling.
template <bool POS>
__device__ __forceinline__ float tanh_impl(float x) {
  constexpr float P0 = -0.33333295583724976f, P1 = 0.13332344591617584f, P2 = -0.05387980490922928f,
                  P3 = 0.021486664190888405f, P4 = -0.007946118712425232f, P5 = 0.0023013753816485405f,
                  P6 = -0.00035845543607138097f;
  constexpr float L2 = 2.8853900432586669921875f;  // fp32 2 log2 e
  const float ax = POS ? x : __builtin_fabsf(x);
  const float s = x * x;
  float p = __builtin_fmaf(s, P6, P5);
  p = __builtin_fmaf(s, p, P4);
  p = __builtin_fmaf(s, p, P3);
  p = __builtin_fmaf(s, p, P2);
  p = __builtin_fmaf(s, p, P1);
  p = __builtin_fmaf(s, p, P0);
  const float small = __builtin_fmaf(x * s, p, x);
  const float big = __builtin_fmaf(-2.0f, __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(ax * L2)), 1.0f);
  return ax < 1.0f ? small : (POS ? big : __builtin_copysignf(big, x));
}
__device__ __forceinline__ float tanh_f(float x) { return tanh_impl<false>(x); }
__device__ __forceinline__ float tanh_pos_f(float x) { return tanh_impl<true>(x); }

// Rows of floats addressed as a raw buffer: a uniform base and size in bytes, per-lane
// byte offsets and a uniform byte offset.  A lane whose offset is at or beyond the size
// reads 0 and its store is dropped, so lanes past the end (offset kOffNone) and rows
// past the last step (size 0) need no branch and touch no memory.  Sizes < 2^31.
constexpr unsigned kOffNone = 0x80000000u;
constexpr int kCpolNt = 2;  // non-temporal: the stream is touched once
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const float* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, (int)bytes, 0x00020000);
}
template <int CPOL = kCpolNt>
__device__ __forceinline__ float row_load(__amdgpu_buffer_rsrc_t r, unsigned voff, int soff) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, soff, CPOL));
}
__device__ __forceinline__ void row_store_nt(float v, __amdgpu_buffer_rsrc_t r, unsigned voff, int soff) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, (int)voff, soff, kCpolNt);
}

// Workgroup barrier that orders LDS accesses only.  __syncthreads() also waits for
// the wave's outstanding global loads and stores; the persistent kernels and the scans
// keep those in flight across the barrier on purpose.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// 64-bit {tag:hi32, value:lo32} words used to hand values between workgroups of a
// persistent kernel.  Stores and loads are relaxed device-scope atomics (each word
// is read or written whole); a reader accepts a word only when its tag matches the
// step it waits for, so no separate barrier or fence is needed.
__device__ __forceinline__ void tag_store(unsigned long long* p, float v, unsigned tag) {
  unsigned long long w = (static_cast<unsigned long long>(tag) << 32) | __float_as_uint(v);
  __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long tag_load(const unsigned long long* p) {
  return __hip_atomic_load(const_cast<unsigned long long*>(p), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned tag_of(unsigned long long w) { return static_cast<unsigned>(w >> 32); }
__device__ __forceinline__ float val_of(unsigned long long w) { return __uint_as_float(static_cast<unsigned>(w)); }

}  // namespace hsl
