/*
 * hsl.h -- C ABI of the HeadStartLSTM training hot path on MI355X (gfx950).
 *
 * HeadStartLSTM is a one-layer LSTM with sigmoid g-gate and a learnable
 * per-gate scale a[4] on the recurrent term:
 *   z_t = x_t W_ih^T + b_ih + a (.) (h_{t-1} W_hh^T + b_hh)      gate order [i,f,g,o]
 *   i,f,g,o = sigmoid(z_t);  c_t = f c_{t-1} + i g;  h_t = o tanh(c_t)
 * Parallel mode drops the a-term and solves c_t = f c_{t-1} + i g as a scan.
 *
 * Conventions for every entry point:
 *  - all tensor pointers are device memory, fp32, contiguous row-major, caller
 *    allocated; shapes are given by T (time), B (batch), D (input), H (hidden);
 *  - the last argument is the HIP stream (hipStream_t passed as void*; NULL is
 *    the null stream); work is only enqueued, nothing is synchronised, and no
 *    device memory is allocated, so every call can be captured in a hipGraph;
 *  - the initial states h0/c0 and the incoming gradients dh_n/dc_n may be
 *    NULL, which every entry point reads as all-zero [B,H] (the reference's
 *    hx=None, __init__.py:174-176, and an unused h_n/c_n), so no zero buffers
 *    need to be filled;
 *  - the return value is HSL_OK (0) or an HSL_ERR_* code; hsl_last_error()
 *    then returns a message (per host thread);
 *  - scratch memory is passed in as (ws, ws_bytes); the needed size is given by
 *    the matching *_ws_bytes() query.  Calls that share one workspace on
 *    different streams at the same time race.
 *
 * Each entry point names the reference code it replaces
 * (m-j-tilley/prLSTM, src/headstartlstm/...).
 */
#ifndef HSL_H
#define HSL_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HSL_ABI_VERSION 3

enum hsl_status {
  HSL_OK = 0,
  HSL_ERR_ARG = 1,          /* bad shape / null pointer / workspace too small */
  HSL_ERR_UNSUPPORTED = 2,  /* shape outside what the kernels handle          */
  HSL_ERR_HIP = 3,          /* a HIP runtime call failed                       */
  HSL_ERR_DEVICE = 4        /* a kernel reported an error (see hsl_poll_error) */
};

/* Library identity and error text.  (No reference counterpart.) */
int hsl_abi_version(void);
const char* hsl_last_error(void);

/* Recurrent-path selection: 0 = automatic (persistent kernels where the shape
 * fits on chip, else one launch per time step), 1 = always per-step,
 * 2 = persistent only (HSL_ERR_UNSUPPORTED if it does not fit).  Returns the
 * previous value.  Process-wide. */
int hsl_set_recurrent_path(int mode);
/* Bound, in microseconds, on any wait a persistent kernel does for another
 * workgroup (default 2,000,000).  On expiry the kernel stops and raises the
 * device error flag instead of waiting forever.  Returns the previous value. */
long long hsl_set_spin_timeout_us(long long us);
/* Hand-off between the workgroups of a persistent kernel: 0 = automatic (stores
 * that stay in the XCD's L2 when the launch verifies that every workgroup of a
 * batch group runs on one XCD, device-scope stores otherwise), 1 = always
 * device-scope stores.  Returns the previous value.  Process-wide. */
int hsl_set_exchange_scope(int mode);
/* Large products run by default (on = 1) on the bf16 matrix instructions with
 * every fp32 operand split exactly into three bf16 pieces and the six largest piece
 * products accumulated in fp32 (error that of the fp32 MFMA product):
 *  - C = A B^T (+bias) with at least 256 output tiles of 256 x 256: the input
 *    projection x W_ih^T + b_ih (_torch.py:96, _parallel.py:56);
 *  - C = A^T B and C = A B of at least 8 GFLOP with M >= 256, N >= 128: the weight
 *    gradients and dx (_torch.py:157-162), as fp32 runs of 64 k folded into a second
 *    fp32 sum, split along K into planes of at most 2048 k added in fp64 (workspace
 *    permitting; otherwise the fp32 kernel runs);
 *  - the products the persistent recurrent kernels fuse (H <= 512): the forward's input
 *    projection and the backward's weight gradients (k = 8 steps x 4 batch rows).
 * on = 0 uses the fp32 MFMA instruction for every product.  With
 * on = 1 a non-finite element of A (or one beyond the bf16 range, 3.3895e38) makes
 * its row of C NaN and one of B its column, where the fp32 instruction would give
 * IEEE infinities.  Returns
 * the previous value.  Process-wide.  No counterpart in the reference (its torch
 * backend calls torch.nn.functional.linear). */
int hsl_set_split_products(int on);
/* Which path the last hsl_rec_fwd / hsl_rec_bwd in this process (on any host
 * thread; autograd runs the backward on its own thread) used: 1 = per-step,
 * 2 = persistent, 3 = the persistent kernels that hold W_hh in the registers of
 * 256 workgroups (H = 1024 or 2048, B <= 32). */
int hsl_last_recurrent_path(void);
/* Whether the last hsl_rec_bwd (in this process, on any thread) accumulated the
 * weight gradients inside the persistent kernel: 0 = no (separate GEMMs), 1 = dW_hh,
 * 2 = dW_hh and dW_ih (D <= 256).  (No reference counterpart.) */
int hsl_last_backward_fused(void);
/* Measurement hook (no reference counterpart): with timing on, the library
 * records a pair of HIP events on the launch stream around each launch of the
 * persistent recurrent kernels (kind 1 forward, 2 backward), the scan kernels
 * (3 forward, 4 backward), the input projection (5) and the per-step loops
 * (6 forward, 7 backward).  hsl_timing_collect waits for and sums the recorded
 * pairs of one kind (milliseconds) and forgets them.  Not for graph capture. */
int hsl_set_timing(int on);
int hsl_timing_collect(int kind, double* total_ms, int* count);
/* Copy the device error flag kept at the start of a recurrent workspace into
 * *flag (synchronises `stream`); nonzero means a persistent wait timed out. */
int hsl_poll_error(const void* ws, int* flag, void* stream);
/* Device errors raised by this library's kernels on the current device since
 * they were last cleared: one sticky word per device, whatever workspace or
 * stream the failing call used.  Bit 0: a persistent kernel gave up a wait
 * between workgroups (hsl_set_spin_timeout_us).  Waits for `stream`, stores the
 * word in *flags and, when clear != 0, resets it.  Such an abort is never
 * silent: the aborting workgroups also fill every output they own with NaN
 * (forward: their rows of h_save, c_save, gact, tanh_c; backward: their dW
 * planes, bias partials, dgates and dh0/dc0), so the results of the call are NaN.
 * Counterpart of the reference's loud failures (TORCH_CHECK at
 * _csrc/lstm_cell.cpp:38-43, RuntimeError at _metal.py:85-87). */
int hsl_device_errors(int* flags, int clear, void* stream);
/* Test hook (no reference counterpart): y[i] = f(x[i]) for n fp32 values with
 * the device math of the kernels, fn 0 = exp, 1 = sigmoid, 2 = tanh, and
 * fn 3 = sigmoid(x[i]) sigmoid(x[n-1-i]) as the scans form i*g (the reference
 * computes them with torch.sigmoid / torch.tanh, _torch.py:29-34,
 * _parallel.py:58-63). */
int hsl_eval_math(int fn, const float* x, float* y, size_t n, void* stream);

/* ---------------------------------------------------------------------------
 * Recurrent mode: replaces HeadStartLSTMTorchFn (_torch.py:86-170).
 * ------------------------------------------------------------------------- */

/* Workspace for hsl_rec_fwd on the current device: the exchange buffers of the
 * persistent kernel, plus the input-gate buffer [T,B,4H] when the input projection
 * is not fused into it, or the per-step path's buffers when that path runs.  The
 * size assumes a 16-byte aligned x (the fused projection reads x in 16-byte pieces;
 * with an unaligned x the call needs the input-gate buffer too and reports the
 * size).  Without a usable device, the size that covers every path. */
size_t hsl_rec_fwd_ws_bytes(int T, int B, int D, int H);

/* Forward: _torch.py:86-131 (a-prescale :91-94, input GEMM :96, time loop
 * :111-120).  Writes
 *   h_save [T+1,B,H]   h_save[0] = h0, h_save[t+1] = h_t  (output = h_save[1:])
 *   c_save [T+1,B,H]   c_save[0] = c0, c_save[t+1] = c_t
 *   gact   [T,B,H,4]   sigmoid gate activations (i, f, g, o) of each unit
 *   tanh_c [T,B,H]     tanh(c_t)
 * gact and tanh_c are what hsl_rec_bwd reads back. */
int hsl_rec_fwd(const float* x, const float* h0, const float* c0,
                const float* w_ih, const float* w_hh, const float* b_ih,
                const float* b_hh, const float* a,
                float* h_save, float* c_save, float* gact, float* tanh_c,
                void* ws, size_t ws_bytes, int T, int B, int D, int H, void* stream);

/* hsl_rec_fwd without a workspace argument, for callers that cannot allocate
 * device memory (code under hipGraph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  No counterpart in the reference.  Its workspace is a static
 * scratch array of 4 MiB inside the library, one per device, held until the
 * process ends; the call allocates nothing (no hipMalloc, no events) and clears
 * the parts that must start empty with a fill kernel.  Shapes whose workspace
 * exceeds 4 MiB are rejected with HSL_ERR_UNSUPPORTED; the persistent path with
 * the input projection fused (H <= 512, D <= 256, D % 4 == 0, 16-byte aligned x,
 * a batch that fits the chip) needs well under 1 MiB.  Every call on one device
 * shares that device's scratch: calls that overlap on one device (two streams,
 * two threads) race.  Results equal hsl_rec_fwd's bit for bit. */
int hsl_rec_fwd_noalloc(const float* x, const float* h0, const float* c0,
                        const float* w_ih, const float* w_hh, const float* b_ih,
                        const float* b_hh, const float* a,
                        float* h_save, float* c_save, float* gact, float* tanh_c,
                        int T, int B, int D, int H, void* stream);

/* Workspace for hsl_rec_bwd on the current device: fp64 reduction buffers, the
 * exchange buffers or the per-step buffers of the path that runs, the weight-
 * gradient planes / GEMM split-K partials, and dgates [T,B,4H] when a product reads
 * them (dx requested, or dW_ih not accumulated inside the persistent kernel).
 * hsl_rec_bwd_ws_bytes is enough for any call (dx requested); _for gives the size for
 * a call with (with_dx != 0) == (dx != NULL).  Without a usable device, the size
 * that covers every path. */
size_t hsl_rec_bwd_ws_bytes(int T, int B, int D, int H);
size_t hsl_rec_bwd_ws_bytes_for(int T, int B, int D, int H, int with_dx);

/* Backward: _torch.py:133-170 (reverse loop :143-150, batched GEMMs :153-162,
 * a-unscale :165-168).  dout [T,B,H], dh_n/dc_n [B,H].  Writes dx [T,B,D] (skipped
 * when dx is NULL),
 * dw_ih [4H,D], dw_hh [4H,H], db_ih [4H], db_hh [4H], da [4].  dh0/dc0 [B,H]
 * receive the gradients w.r.t. h0/c0 when non-NULL (the reference torch
 * backend returns None for them, _torch.py:170; its Metal backend returns
 * them, _metal.py:154-174). */
int hsl_rec_bwd(const float* dout, const float* dh_n, const float* dc_n,
                const float* x, const float* h_save, const float* c_save,
                const float* gact, const float* tanh_c,
                const float* w_ih, const float* w_hh, const float* b_hh, const float* a,
                float* dx, float* dw_ih, float* dw_hh, float* db_ih, float* db_hh,
                float* da, float* dh0, float* dc0,
                void* ws, size_t ws_bytes, int T, int B, int D, int H, void* stream);

/* ---------------------------------------------------------------------------
 * Parallel (scan) mode: replaces headstartlstm_parallel (_parallel.py:38-74)
 * and the autograd backward torch derives for it.
 * ------------------------------------------------------------------------- */

/* Forward: gates = x W_ih^T + b_ih ([T,B,4H], kept for the backward), then the
 * scan c_t = max(f_t,eps) c_{t-1} + max(i_t g_t, eps), c_{-1} = max(c0,eps)
 * (the recurrence _parallel.py:21-35 evaluates in the log domain), and
 * out_t = o_t tanh(c_t).  Writes gates, out [T,B,H] and c_ck
 * [hsl_scan_ck_rows(T), B, H]: the cell state at every 8th step, kept for the
 * backward (row m < R-1 is the state carried into step 8m, row 0 = max(c0,eps)),
 * and c_n in its last row R-1.
 * h_n = out[T-1], c_n = c_ck[R-1] (_parallel.py:74). */
int hsl_scan_ck_rows(int T); /* R = ceil(T/8) + 1 */
int hsl_par_fwd(const float* x, const float* c0, const float* w_ih, const float* b_ih,
                float eps, float* gates, float* out, float* c_ck,
                int T, int B, int D, int H, void* stream);

/* hsl_par_fwd for a half-precision module: x [T,B,D] and w_ih [4H,D] are bf16
 * (fmt 0) or fp16 (fmt 1); b_ih, c0, gates and c_ck are fp32, and out [T,B,H] is in
 * the module's format (x's): the fp32 scan output rounded to nearest even when it is
 * stored, as the module's output conversion rounds it.  The input projection runs on
 * 16-bit MFMA with fp32 accumulation: each product of two 16-bit values is exact in
 * fp32, so gates equal the fp32 projection of the widened operands up to the order of
 * the fp32 additions.  Replaces the same call sites as hsl_par_fwd (_parallel.py:38-74)
 * for modules moved to bf16/fp16 (the way test_parallel.py:22-38 runs bf16). */
int hsl_par_fwd_b16(const void* x, const float* c0, const void* w_ih, const float* b_ih,
                    float eps, float* gates, void* out, float* c_ck,
                    int T, int B, int D, int H, int fmt, void* stream);

size_t hsl_par_bwd_ws_bytes(int T, int B, int D, int H);

/* Backward of hsl_par_fwd w.r.t. x, W_ih, b_ih and c0 (W_hh, b_hh, a and h0
 * are unused in parallel mode, so they get no gradient, _parallel.py:41-43).
 * dout [T,B,H], dh_n/dc_n [B,H] are the gradients of out, h_n, c_n.
 * dx and dc0 may be NULL (then they are not computed). */
int hsl_par_bwd(const float* dout, const float* dh_n, const float* dc_n,
                const float* x, const float* c0, const float* gates, const float* c_ck,
                const float* w_ih, float eps,
                float* dx, float* dw_ih, float* db_ih, float* dc0,
                void* ws, size_t ws_bytes, int T, int B, int D, int H, void* stream);

/* hsl_par_bwd for a bf16 (fmt 0) or fp16 (fmt 1) module: x, w_ih and dout (the
 * gradient of hsl_par_fwd_b16's out) are 16-bit, everything else as in hsl_par_bwd
 * (fp32 gradients).  The results equal hsl_par_bwd's on the widened x, w_ih and dout
 * bit for bit.  A bf16 x / w_ih is read by
 * the split-product kernel as it is (one bf16 piece, three products per k-step
 * instead of six); otherwise (fp16, or products too small for that kernel) it is
 * widened into the workspace first.  Backward of the reference's parallel path for
 * a module moved to bf16/fp16 (_parallel.py:38-74, run that way by
 * test_parallel.py:22-38). */
size_t hsl_par_bwd_b16_ws_bytes(int T, int B, int D, int H);
int hsl_par_bwd_b16(const void* dout, const float* dh_n, const float* dc_n,
                    const void* x, const float* c0, const float* gates, const float* c_ck,
                    const void* w_ih, float eps,
                    float* dx, float* dw_ih, float* db_ih, float* dc0,
                    void* ws, size_t ws_bytes, int T, int B, int D, int H, int fmt, void* stream);

/* fp64 modules (the reference runs them through its torch backend, test_cpp.py:150-165,
 * and its parallel functional is dtype-generic, _parallel.py:38-74).  Every argument,
 * layout and output is that of the fp32 entry point of the same name without "_f64"
 * (hsl_rec_fwd, hsl_rec_bwd, hsl_par_fwd, hsl_par_bwd), with double for float; all
 * arithmetic is fp64.  Products run on the fp64 matrix instruction (split along K into
 * partials summed in a fixed order when the output is small), recurrent mode launches a
 * product and a cell kernel per time step, and the parallel scans run time-chunked in
 * three passes; every sum runs in a fixed order (deterministic results).  The recurrent
 * backward's workspace always holds the [T,B,4H] dgates. */
size_t hsl_rec_fwd_f64_ws_bytes(int T, int B, int D, int H);
int hsl_rec_fwd_f64(const double* x, const double* h0, const double* c0,
                    const double* w_ih, const double* w_hh, const double* b_ih,
                    const double* b_hh, const double* a,
                    double* h_save, double* c_save, double* gact, double* tanh_c,
                    void* ws, size_t ws_bytes, int T, int B, int D, int H, void* stream);
size_t hsl_rec_bwd_f64_ws_bytes(int T, int B, int D, int H);
int hsl_rec_bwd_f64(const double* dout, const double* dh_n, const double* dc_n,
                    const double* x, const double* h_save, const double* c_save,
                    const double* gact, const double* tanh_c,
                    const double* w_ih, const double* w_hh, const double* b_hh, const double* a,
                    double* dx, double* dw_ih, double* dw_hh, double* db_ih, double* db_hh,
                    double* da, double* dh0, double* dc0,
                    void* ws, size_t ws_bytes, int T, int B, int D, int H, void* stream);
int hsl_par_fwd_f64(const double* x, const double* c0, const double* w_ih, const double* b_ih,
                    double eps, double* gates, double* out, double* c_ck,
                    int T, int B, int D, int H, void* stream);
size_t hsl_par_bwd_f64_ws_bytes(int T, int B, int D, int H);
int hsl_par_bwd_f64(const double* dout, const double* dh_n, const double* dc_n,
                    const double* x, const double* c0, const double* gates, const double* c_ck,
                    const double* w_ih, double eps,
                    double* dx, double* dw_ih, double* db_ih, double* dc0,
                    void* ws, size_t ws_bytes, int T, int B, int D, int H, void* stream);

/* The scan kernels on their own (used by hsl_par_fwd / hsl_par_bwd).
 * hsl_scan_fwd: gates [T,B,4H] pre-activations -> out [T,B,H], c_ck (as in
 * hsl_par_fwd).
 * hsl_scan_bwd: -> dgates [T,B,4H] (pre-activation gradients) and, when
 * db_part is non-NULL, per-batch column sums of dgates as doubles [B,4H];
 * dc0 may be NULL. */
int hsl_scan_fwd(const float* gates, const float* c0, float eps,
                 float* out, float* c_ck, int T, int B, int H, void* stream);
int hsl_scan_bwd(const float* gates, const float* c0, const float* c_ck,
                 const float* dout, const float* dh_n, const float* dc_n, float eps,
                 float* dgates, double* db_part, float* dc0,
                 int T, int B, int H, void* stream);

/* ---------------------------------------------------------------------------
 * fp32 MFMA GEMM used by both modes (torch.nn.functional.linear at
 * _torch.py:96 / _parallel.py:56 and the `@` products at _torch.py:157-162).
 *   C[M,N] = op(A)[M,K] . op(B)[K,N] (+ bias[N] when bias != NULL)
 *   trans_a = 0: A is [M,lda] row-major; 1: A is [K,lda] and op(A) = A^T
 *   trans_b = 0: B is [K,ldb] row-major; 1: B is [N,ldb] and op(B) = B^T
 * Split-K (for K much larger than M*N) goes through ws; with ws_bytes = 0 the
 * product is computed without splitting.  hsl_gemm_ws_bytes is enough for every
 * layout (the split-bf16 A^T B kernel may use more planes than the others).
 * ------------------------------------------------------------------------- */
size_t hsl_gemm_ws_bytes(int M, int N, int K);
int hsl_gemm_f32(const float* A, const float* Bm, const float* bias, float* C,
                 int M, int N, int K, int lda, int ldb, int ldc,
                 int trans_a, int trans_b, void* ws, size_t ws_bytes, void* stream);

/* C[M,N] = A[M,K] . B[N,K]^T (+ bias[N]) with A, B bf16 (fmt 0) or fp16 (fmt 1),
 * fp32 accumulation, C and bias fp32 (row-major, leading dimensions in elements).
 * The 16-bit counterpart of hsl_gemm_f32's trans_b product (F.linear,
 * _parallel.py:56) used by hsl_par_fwd_b16. */
int hsl_gemm_b16(const void* A, const void* B, const float* bias, float* C,
                 int M, int N, int K, int lda, int ldb, int ldc, int fmt, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HSL_H */
