// Library-wide state of libhsl: error text, per-device facts, options.
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <vector>

#include "hsl_internal.h"

namespace hsl {

namespace {
thread_local char g_err[512] = "";
// process-wide, not per thread: autograd runs the backward on its own worker thread
std::atomic<int> g_last_path{0};
std::atomic<int> g_last_fused{0};
std::atomic<int> g_path_mode{0};
std::atomic<int> g_exchange_scope{0};
std::atomic<int> g_split_products{1};
std::atomic<long long> g_spin_us{2000000};
std::mutex g_dev_mu;
DeviceInfo g_devs[64];
}  // namespace

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

// The kernels and GEMMs hold these in 32-bit integers: the GEMM rows and reduction
// length T*B, the elements of a [4H, max(D, H)] weight, and the bytes of one time step of
// a [B, 4H] or [B, D] row block (addressed as a raw buffer of < 2^31 bytes).  Whole
// [T, B, max(4H, D)] buffers are sized in size_t, bounded at 2^40 elements.
int check_shape(const char* who, int T, int B, int D, int H) {
  if (T < 0 || B < 0 || D < 0 || H < 0)
    return fail(HSL_ERR_ARG, "%s: negative dimension (T=%d B=%d D=%d H=%d)", who, T, B, D, H);
  const long long t = T, b = B, d = D, g = 4ll * H, lim = 1ll << 31;
  const long long row = g > d ? g : d;      // widest per-(t, b) row in floats
  const long long wcols = d > H ? d : H;    // columns of the widest weight
  if (t * b >= lim || g * wcols >= lim || 4 * b * row >= lim || t >= (1ll << 30) || t * b * row > (1ll << 40))
    return fail(HSL_ERR_UNSUPPORTED,
                "%s: T=%d B=%d D=%d H=%d is beyond the library's 32-bit index range (needs T*B < 2^31, "
                "4H*max(D,H) < 2^31 and a time step's [B, max(4H,D)] row block < 2^31 bytes)",
                who, T, B, D, H);
  return HSL_OK;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(HSL_ERR_HIP, "%s failed: %s", what, hipGetErrorString(e));
}

int device_info(DeviceInfo* out) {
  int dev = 0;
  HSL_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) return fail(HSL_ERR_UNSUPPORTED, "device index %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_dev_mu);
  DeviceInfo& d = g_devs[dev];
  if (d.device != dev) {
    int cus = 0;
    HSL_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    d.num_cus = cus;
    d.num_xcds = 8;  // MI355X: 8 XCDs; workgroup i is dispatched to XCD i % 8
    d.device = dev;
  }
  *out = d;
  return HSL_OK;
}

// ---- optional per-kernel timing (hsl_set_timing) ---------------------------------
namespace {
struct TimingRec {
  hipEvent_t start, stop;
  int kind;
};
std::mutex g_tmu;
std::vector<TimingRec> g_trecs;
std::atomic<int> g_timing{0};
}  // namespace

namespace {
thread_local int g_timing_off = 0;  // > 0 inside a TimingSuppress scope on this thread
}  // namespace

TimingSuppress::TimingSuppress() { ++g_timing_off; }
TimingSuppress::~TimingSuppress() { --g_timing_off; }

int timing_begin(int kind, hipStream_t s) {
  if (!g_timing.load() || g_timing_off > 0) return -1;
  TimingRec r{nullptr, nullptr, kind};
  if (hipEventCreate(&r.start) != hipSuccess || hipEventCreate(&r.stop) != hipSuccess) return -1;
  if (hipEventRecord(r.start, s) != hipSuccess) return -1;
  std::lock_guard<std::mutex> lk(g_tmu);
  g_trecs.push_back(r);
  return (int)g_trecs.size() - 1;
}

void timing_end(int slot, hipStream_t s) {
  if (slot < 0) return;
  std::lock_guard<std::mutex> lk(g_tmu);
  if (slot < (int)g_trecs.size()) (void)hipEventRecord(g_trecs[slot].stop, s);
}

int recurrent_path_mode() { return g_path_mode.load(); }
int exchange_scope_mode() { return g_exchange_scope.load(); }
int split_products_mode() { return g_split_products.load(); }
long long spin_timeout_ticks() { return g_spin_us.load() * 100; }  // 100 MHz clock
void note_recurrent_path(int path) { g_last_path.store(path); }
void note_backward_fused(int fused) { g_last_fused.store(fused); }

namespace {
// y[i] = f(x[i]) for the device math of the kernels (fn 0 exp_f, 1 sigmoid_f, 2 tanh_f).
__global__ void eval_math_kernel(int fn, const float* __restrict__ x, float* __restrict__ y, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const float v = x[i];
    y[i] = fn == 0 ? exp_f(v) : fn == 1 ? sigmoid_f(v) : fn == 2 ? tanh_f(v) : sigmoid_prod_f(v, x[n - 1 - i]);
  }
}
}  // namespace

}  // namespace hsl

extern "C" {

int hsl_abi_version(void) { return HSL_ABI_VERSION; }

const char* hsl_last_error(void) { return hsl::g_err; }

int hsl_set_recurrent_path(int mode) {
  if (mode < 0 || mode > 2) mode = 0;
  return hsl::g_path_mode.exchange(mode);
}

long long hsl_set_spin_timeout_us(long long us) {
  if (us < 1) us = 1;
  return hsl::g_spin_us.exchange(us);
}

int hsl_last_recurrent_path(void) { return hsl::g_last_path.load(); }
int hsl_last_backward_fused(void) { return hsl::g_last_fused.load(); }

int hsl_set_exchange_scope(int mode) { return hsl::g_exchange_scope.exchange(mode == 1 ? 1 : 0); }

int hsl_set_split_products(int on) { return hsl::g_split_products.exchange(on ? 1 : 0); }

int hsl_set_timing(int on) { return hsl::g_timing.exchange(on ? 1 : 0); }

int hsl_timing_collect(int kind, double* total_ms, int* count) {
  if (!total_ms || !count) return hsl::fail(HSL_ERR_ARG, "hsl_timing_collect: null pointer");
  std::lock_guard<std::mutex> lk(hsl::g_tmu);
  double sum = 0.0;
  int n = 0;
  std::vector<hsl::TimingRec> keep;
  for (auto& r : hsl::g_trecs) {
    if (r.kind != kind) {
      keep.push_back(r);
      continue;
    }
    float ms = 0.f;
    HSL_HIP(hipEventSynchronize(r.stop));
    HSL_HIP(hipEventElapsedTime(&ms, r.start, r.stop));
    sum += ms;
    ++n;
    (void)hipEventDestroy(r.start);
    (void)hipEventDestroy(r.stop);
  }
  hsl::g_trecs.swap(keep);
  *total_ms = sum;
  *count = n;
  return HSL_OK;
}

int hsl_eval_math(int fn, const float* x, float* y, size_t n, void* stream) {
  if (fn < 0 || fn > 3)
    return hsl::fail(HSL_ERR_ARG, "hsl_eval_math: fn %d is not 0 (exp), 1 (sigmoid), 2 (tanh) or 3 (sigmoid product)",
                     fn);
  if (n == 0) return HSL_OK;
  if (!x || !y) return hsl::fail(HSL_ERR_ARG, "hsl_eval_math: null pointer");
  size_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(hsl::eval_math_kernel, dim3((unsigned)blocks), dim3(256), 0, static_cast<hipStream_t>(stream), fn,
                     x, y, n);
  HSL_HIP(hipGetLastError());
  return HSL_OK;
}

int hsl_poll_error(const void* ws, int* flag, void* stream) {
  if (!ws || !flag) return hsl::fail(HSL_ERR_ARG, "hsl_poll_error: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  HSL_HIP(hipMemcpyAsync(flag, ws, sizeof(int), hipMemcpyDeviceToHost, s));
  HSL_HIP(hipStreamSynchronize(s));
  return HSL_OK;
}

}  // extern "C"
