/*
 * defmuon_hip.h -- C ABI of the MI355X (gfx950) polar-factor library
 *                  (libdefmuon_hip.so, built from spectral-deflation_amd/csrc).
 *
 * Drop-in boundary for the polar-factor path of deflated Muon in
 * ComputationalRobotics/Spectral-Deflation.  Each entry point names the reference
 * function it replaces (paths relative to that tree).
 *
 * Conventions
 *   - All pointers are device pointers; nothing here allocates.  Outputs and the
 *     workspace are caller-owned; size the workspace with the *_workspace_size
 *     call for the same shape.
 *   - Work is enqueued on `stream` (a hipStream_t); no entry point synchronises.
 *   - Matrices are row-major.  "Tall" batches are (batch, n, m) with n >= m.
 *   - Return value: 0 on success; 1 bad argument/shape; 2 workspace too small;
 *     3 HIP launch failure.  dmh_last_error() describes the last failure of the
 *     calling thread.
 *   - The sketch width r of the front-end entries is at most 64.
 */
#ifndef DEFMUON_HIP_H
#define DEFMUON_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* dmh_stream_t; /* hipStream_t */

/* Text of the calling thread's last error. */
const char* dmh_last_error(void);

/* ---- bf16 Newton-Schulz / Polar Express chain --------------------------------
 * Replaces the bf16 GEMM chains of
 *   zeropower_via_newtonschulz5   defmuon/optim/muon.py:16-44
 *   PolarExpress                  defmuon/optim/polar_express.py:21-34
 *   _horner_iterate               defmuon/optim/deflation_batched.py:196-204
 * for `batch` same-shape matrices in one grouped launch per GEMM phase.
 *
 *   x            (batch, rows, cols), element strides (x_bstride, x_rstride,
 *                x_cstride); x_dtype 0 = fp32, 1 = bf16
 *   out          (batch, rows, cols) bf16, contiguous
 *   orient_tall  1: x is the tall operand T (step G = T^T T, T <- aT + T(bG + cG^2),
 *                the deflated arms' convention); 0: x is the wide operand W
 *                (A = W W^T, W <- aW + (bA + cA^2) W, muon.py / polar_express.py)
 *   entry_mode   0: x used as is; 1: x / (||x||_F + 1e-7); 2: x / (1.01 ||x||_F + 1e-7)
 *                (norm per matrix over the un-rounded input)
 *   coeffs       steps x 3 doubles (a, b, c) per step
 * Limit: the padded iterate (rows and cols rounded up to multiples of 256, bf16) must
 * stay below 2^31 bytes (32-bit operand addressing); larger shapes return 1.  The
 * same limit applies to the chain of dmh_deflated_polar*.
 */
int dmh_ns_workspace_size(int batch, int rows, int cols, int orient_tall, size_t* bytes);
int dmh_ns_chain(dmh_stream_t stream, const void* x, int x_dtype, int batch, int rows, int cols,
                 long long x_bstride, long long x_rstride, long long x_cstride, void* out,
                 int orient_tall, int entry_mode, const double* coeffs, int steps, void* ws,
                 size_t ws_bytes);

/* Allocation-free variant of dmh_ns_chain.  It has no counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same arguments
 * without the workspace, which is a static device array of DMH_NS_SCRATCH_BYTES
 * (64 MiB) per GPU.  The array belongs to the library's code object, which the HIP
 * runtime loads on a GPU when any of the library's kernels first runs there: every
 * process that uses the library holds 64 MiB of HBM on each GPU it runs on until it
 * ends, whether or not it calls this entry.
 * A shape whose workspace (dmh_ns_workspace_size) exceeds it returns 2.  Every call
 * on one GPU uses the same array: calls that overlap on one GPU race. */
#define DMH_NS_SCRATCH_BYTES (64u << 20)
int dmh_ns_chain_noalloc(dmh_stream_t stream, const void* x, int x_dtype, int batch, int rows,
                         int cols, long long x_bstride, long long x_rstride,
                         long long x_cstride, void* out, int orient_tall, int entry_mode,
                         const double* coeffs, int steps);

/* ---- fp32 tall-convention chain ---------------------------------------------
 * The dtype-preserving path of _horner_iterate (defmuon/optim/deflation_batched.py:
 * 196-204) for fp32 input: per (a, b, c) in coeffs, G = X^T X, B = b G + (c G) G,
 * X <- a X + X B, in fp32.  x, out: (batch, n, m) fp32, contiguous, distinct.
 */
int dmh_horner_f32_workspace_size(int batch, int n, int m, size_t* bytes);
int dmh_horner_f32(dmh_stream_t stream, const float* x, int batch, int n, int m, float* out,
                   const double* coeffs, int steps, void* ws, size_t ws_bytes);

/* ---- randomized-SVD deflation front-end (fp32, fp64 Gram) --------------------
 * One workspace size serves dmh_orth (call it with n = rows, m = r), dmh_project,
 * dmh_rsvd and dmh_rmfro_clip.  Shapes: n >= m >= r, 1 <= r <= 64, n < 2^23 rows
 * (status 1 and "unsupported shape" otherwise).
 */
int dmh_rsvd_workspace_size(int batch, int n, int m, int r, size_t* bytes);
int dmh_rmfro_workspace_size(int batch, int n, int m, int r, size_t* bytes);

/* Batched CholeskyQR, `passes` passes: Q = X L^-T with L = chol(X^T X) (fp64).
 * Replaces _orth_b, defmuon/optim/deflation_batched.py:117-128.
 * X, Q: (batch, rows, r) fp32.  A non-positive pivot gives Q = 0 for that matrix
 * (the reference leaves it undefined: cholesky_ex info is ignored). */
int dmh_orth(dmh_stream_t stream, const float* X, int batch, int rows, int r, int passes,
             float* Q, void* ws, size_t ws_bytes);

/* Rayleigh-Ritz: thin SVD of Q^T A.  Replaces _project_b,
 * defmuon/optim/deflation_batched.py:131-139.
 * Q (batch, n, r), A (batch, n, m) fp32 -> U (batch, n, r), s (batch, r)
 * descending, V (batch, m, r). */
int dmh_project(dmh_stream_t stream, const float* Q, const float* A, int batch, int n, int m,
                int r, float* U, float* s, float* V, void* ws, size_t ws_bytes);

/* Subspace iteration (niter power steps, qr_passes CholeskyQR passes) and
 * Rayleigh-Ritz on A (batch, n, m) with the caller's sketch Omega (batch, m, r).
 * Replaces _rsvd_b, defmuon/optim/deflation_batched.py:142-148. */
int dmh_rsvd(dmh_stream_t stream, const float* A, const float* Omega, int batch, int n, int m,
             int r, int niter, int qr_passes, float* U, float* s, float* V, void* ws,
             size_t ws_bytes);

/* The deflation front-end.  Replaces batched_rmfro_clip,
 * defmuon/optim/deflation_batched.py:155-189 (with Omega injected; the caller
 * draws it with torch.randn exactly as :172-174 does).
 *   gate:  kr = #(s > thresh s0); fired = s[kw-1] < ratio s0 && 1 <= kr < r;
 *          k = fired ? clamp(kr, 1, r-1) : 0                       (k: int64)
 *   X0 = (A - U_k S_k V_k^T) / d + U_k (1/pad) V_k^T,  d = ||A - U_k S_k V_k^T||_F + 1e-7
 *   X0: (batch, n, m), bf16 if out_bf16 else fp32; d: (batch,) fp32. */
int dmh_rmfro_clip(dmh_stream_t stream, const float* A, const float* Omega, int batch, int n,
                   int m, int r, int kw, float ratio, float thresh, float pad, int niter,
                   int qr_passes, void* X0, int out_bf16, long long* k, float* d, void* ws,
                   size_t ws_bytes);

/* Fused deflated polar factor: the front-end above followed by the bf16 chain
 * (tall convention, no entry scaling) over `steps` (a, b, c) triples, i.e. what
 * muon.py:298 BATCHED_CLIP(out_dtype=bf16) followed by muon.py:310-312 _iterate
 * computes for one shape group.  X0 is written straight into the chain's packed
 * operands instead of a separate tensor.  out: (batch, n, m) bf16; k, d as for
 * dmh_rmfro_clip.  Workspace: dmh_deflated_polar_workspace_size.
 * chain_event: optional hipEvent_t recorded on `stream` between the front-end and
 * the chain (phase timing); NULL for none. */
int dmh_deflated_polar_workspace_size(int batch, int n, int m, int r, size_t* bytes);
int dmh_deflated_polar(dmh_stream_t stream, const float* A, const float* Omega, int batch, int n,
                       int m, int r, int kw, float ratio, float thresh, float pad, int niter,
                       int qr_passes, const double* coeffs, int steps, void* out, long long* k,
                       float* d, void* ws, size_t ws_bytes, void* chain_event);

/* The two halves of dmh_deflated_polar, on one workspace of
 * dmh_deflated_polar_workspace_size, so that the front-ends of several shape
 * groups can run on separate streams before their chains (muon.py:283-312 runs the
 * groups one after the other; each group's result is the same either way).
 *   _front: BATCHED_CLIP (deflation_batched.py:155-189) with X0 left, bf16, in the
 *           chain's packed operand inside ws; writes k and d.
 *   _chain: the bf16 iteration (deflation_batched.py:196-211 via muon.py:310-312)
 *           from that operand, same batch/n/m, to out (batch, n, m) bf16.
 * ws must stay untouched between the two calls (stream-ordered); the chain works in
 * place on the entry, so each _front is followed by one chain call. */
int dmh_deflated_polar_front(dmh_stream_t stream, const float* A, const float* Omega, int batch,
                             int n, int m, int r, int kw, float ratio, float thresh, float pad,
                             int niter, int qr_passes, long long* k, float* d, void* ws,
                             size_t ws_bytes);
int dmh_deflated_polar_chain(dmh_stream_t stream, int batch, int n, int m, const double* coeffs,
                             int steps, void* out, void* ws, size_t ws_bytes);

/* ---- optimizer glue either side of the polar path (one launch per group) --------
 * One descriptor per Muon parameter of a tall-shape group.  The group's stack is
 * (B, n, m), B = the sum of `blocks`; a parameter's block k (rows k*rows/blocks ..)
 * is the tall matrix (n, m) = transpose ? (cols, rows/blocks) : (rows/blocks, cols),
 * stored at stack + offset + k*n*m.  All tensors fp32 and contiguous.
 *
 * dmh_momentum_stack replaces muon.py:266-289 (per parameter: buf.mul_(mu).add_(g);
 * g' = g.add(buf, alpha=mu) if nesterov else buf; _qkv_split; .float(); .mT for wide;
 * torch.cat): momentum buffers are updated in place and g' written into `stack`.
 * dmh_apply_update replaces muon.py:316-332 for rms scaling: p.mul_(decay) then
 * p.add_(u, alpha) with u the bf16 polar factor read from `ustack` (same layout as
 * the stack) and put back into the parameter's layout; alpha = -lr*sqrt(fan_out/fan_in),
 * decay = 1 - lr*wd per parameter. */
typedef struct {
  const float* grad;   /* (rows, cols) */
  float* momentum;     /* (rows, cols), updated in place */
  float* param;        /* (rows, cols), updated in place by dmh_apply_update */
  int rows, cols;
  int blocks;          /* 3 for a W_QKV parameter, else 1 */
  int transpose;       /* 1: rows/blocks < cols, the block is stored transposed */
  long long offset;    /* elements */
  float alpha, decay;  /* dmh_apply_update only */
} dmh_glue_param;
int dmh_momentum_stack(dmh_stream_t stream, const dmh_glue_param* params, int count,
                       float momentum, int nesterov, float* stack);
int dmh_apply_update(dmh_stream_t stream, const dmh_glue_param* params, int count,
                     const void* ustack);

/* ---- AdamW backup for the non-Muon parameters (one launch per group) ------------
 * Replaces the per-parameter loop of muon.py:408-436 (buf1.lerp_(g, 1 - beta1);
 * buf2.lerp_(g.square(), 1 - beta2); g = buf1 / (eps + buf2.sqrt());
 * p.mul_(1 - lr*wd); p.add_(g, alpha=-lr/scale)) with the same fp32 operations in
 * the same order.  `table` (device memory, `count` entries) lists the group's
 * parameters; `chunk_start` (device memory, count + 1 ints) gives each parameter's
 * first chunk of dmh_adamw_chunks-sized work, chunk_start[count] = nchunks.  The
 * caller keeps both arrays while the tensors stay at the same addresses, so such a
 * step allocates and copies nothing.  w1 = 1 - beta1, w2 = 1 - beta2, decay = 1 - lr*wd,
 * alpha = -lr/scale with scale the bias correction of the (common) step count. */
typedef struct {
  float* param;        /* updated in place */
  const float* grad;
  float* moment1;      /* updated in place */
  float* moment2;      /* updated in place */
  long long numel;
} dmh_adamw_param;
int dmh_adamw_chunks(long long numel);
int dmh_adamw_step(dmh_stream_t stream, const dmh_adamw_param* table, int count,
                   const int* chunk_start, int nchunks, float w1, float w2, float eps,
                   float decay, float alpha);

#ifdef __cplusplus
}
#endif

#endif /* DEFMUON_HIP_H */
