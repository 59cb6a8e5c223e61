// Batched randomized-SVD deflation front-end (fp32 / fp64) on CDNA4.
//
// Replaces, for a batch of same-shape tall matrices A (B, n, m), n >= m:
//   _orth_b             defmuon/optim/deflation_batched.py:117-128  (CholeskyQR, fp64 Gram)
//   _project_b          defmuon/optim/deflation_batched.py:131-139  (Rayleigh-Ritz thin SVD)
//   _rsvd_b             defmuon/optim/deflation_batched.py:142-148  (subspace iteration)
//   batched_rmfro_clip  defmuon/optim/deflation_batched.py:155-189  (gate, remove, restore)
//
// Sketch width r <= RP = 64 columns are carried zero-padded to RP everywhere.
// Kernels:
//   skinny_gemm<ROWS>   C = A X       (n x RP)   fp32 MFMA 32x32x2, A streamed by rows
//   skinny_gemm<COLS>   C = A^T Y     (m x RP)   fp32 MFMA 32x32x2, A streamed by columns
//   gram_partials       partial fp64 Gram Y^T Y over row chunks
//   chol_inv            sum partials, Cholesky in LDS (fp64), M = L^-T  (one workgroup)
//   right_mult          C = Y M       (rows x RP) x (RP x RP)
//   eig_gate            Jacobi eigen-decomposition of Bp Bp^T in LDS (fp64) -> s, Ub;
//                       the deflation gate and the per-column deflate/restore weights
//   deflate_norm        partial ||A - U diag(s h) V^T||_F^2 (fp64)
//   finish_norm         d = ||W||_F + 1e-7
//   deflate_restore     X0 = W / d + U diag(h / pad) V^T  -> bf16 or fp32
#include "common.h"

#include <math.h>

namespace dmh {

constexpr int RP = 64;           // padded sketch width
constexpr int SG_ROWS = 128;     // output rows per skinny-GEMM workgroup
constexpr int SG_K = 32;         // K chunk
constexpr int GRAM_CHUNKS = 8;   // row chunks of the Gram reduction
constexpr int DT = 64;           // deflate tile (rows and columns)

// ---------------------------------------------------------------------------
// skinny GEMMs on fp32 MFMA.  v_mfma_f32_32x32x2f32: lane l supplies
// srcA[row = l%32][k = l/32] and srcB[k = l/32][col = l%32]; the result
// D[row][col] sits in lane col + 32 * ((row >> 2) & 1), register
// 4 * (row >> 3) + (row & 3).
// ---------------------------------------------------------------------------
enum { SG_ROWSTREAM = 0, SG_COLSTREAM = 1 };

// MODE ROWSTREAM: C[i][c] = sum_j A[i][j] X[j][c],  i < n, j < m, X (m x xcols, ld_x)
// MODE COLSTREAM: C[j][c] = sum_i A[i][j] X[i][c],  j < m, i < n, X (n x xcols, ld_x)
// C is (rows x RP) with ld RP; columns >= xcols come out zero.
template <int MODE>
__global__ __launch_bounds__(256) void skinny_gemm(const float* __restrict__ A, int n, int m,
                                                   long long a_bs, const float* __restrict__ X,
                                                   int ld_x, int xcols, long long x_bs,
                                                   float* __restrict__ C, long long c_bs) {
  constexpr int APITCH = MODE == SG_ROWSTREAM ? SG_K + 1 : SG_ROWS;
  constexpr int AROWS = MODE == SG_ROWSTREAM ? SG_ROWS : SG_K;
  __shared__ float As[AROWS * APITCH];
  __shared__ float Xs[SG_K * RP];

  const int b = blockIdx.y;
  const int r0 = blockIdx.x * SG_ROWS;        // first output row (i or j)
  const int outrows = MODE == SG_ROWSTREAM ? n : m;
  const int K = MODE == SG_ROWSTREAM ? m : n;
  A += (long long)b * a_bs;
  X += (long long)b * x_bs;
  C += (long long)b * c_bs;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  f32x16 acc0, acc1;
#pragma unroll
  for (int e = 0; e < 16; ++e) { acc0[e] = 0.f; acc1[e] = 0.f; }

  // per-thread staging: A tile 4096 floats (16 / thread), X tile 2048 (8 / thread)
  float ra[16], rx[8];
#define DMH_SG_LOAD(k0)                                                          \
  do {                                                                           \
    _Pragma("unroll") for (int u = 0; u < 16; ++u) {                             \
      const int e = tid + 256 * u;                                               \
      float v = 0.f;                                                             \
      if (MODE == SG_ROWSTREAM) {                                                \
        const int row = e >> 5, col = e & 31;                                    \
        const int gi = r0 + row, gk = (k0) + col;                                \
        if (gi < n && gk < m) v = A[(long long)gi * m + gk];                     \
      } else {                                                                   \
        const int row = e >> 7, col = e & 127;                                   \
        const int gk = (k0) + row, gj = r0 + col;                                \
        if (gk < n && gj < m) v = A[(long long)gk * m + gj];                     \
      }                                                                          \
      ra[u] = v;                                                                 \
    }                                                                            \
    _Pragma("unroll") for (int u = 0; u < 8; ++u) {                              \
      const int e = tid + 256 * u;                                               \
      const int row = e >> 6, col = e & 63;                                      \
      const int gk = (k0) + row;                                                 \
      float v = 0.f;                                                             \
      if (gk < K && col < xcols) v = X[(long long)gk * ld_x + col];              \
      rx[u] = v;                                                                 \
    }                                                                            \
  } while (0)

  const int nchunks = (K + SG_K - 1) / SG_K;
  DMH_SG_LOAD(0);
  const int l32 = lane & 31, lh = lane >> 5;
  const int wrow = wave * 32;   // this wave's 32 output rows within the tile
  for (int ch = 0; ch < nchunks; ++ch) {
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int e = tid + 256 * u;
      if (MODE == SG_ROWSTREAM) As[(e >> 5) * APITCH + (e & 31)] = ra[u];
      else As[(e >> 7) * APITCH + (e & 127)] = ra[u];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) Xs[tid + 256 * u] = rx[u];
    __syncthreads();
    if (ch + 1 < nchunks) DMH_SG_LOAD((ch + 1) * SG_K);
#pragma unroll
    for (int p = 0; p < SG_K / 2; ++p) {
      const int kk = 2 * p + lh;
      float av;
      if (MODE == SG_ROWSTREAM) av = As[(wrow + l32) * APITCH + kk];
      else av = As[kk * APITCH + wrow + l32];
      const float b0 = Xs[kk * RP + l32];
      const float b1 = Xs[kk * RP + 32 + l32];
      acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(av, b0, acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(av, b1, acc1, 0, 0, 0);
    }
  }
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int row = r0 + wrow + 8 * (e >> 2) + 4 * lh + (e & 3);
    if (row < outrows) {
      C[(long long)row * RP + l32] = acc0[e];
      C[(long long)row * RP + 32 + l32] = acc1[e];
    }
  }
#undef DMH_SG_LOAD
}

// ---------------------------------------------------------------------------
// fp64 Gram of a (rows x RP) fp32 matrix, partial over GRAM_CHUNKS row chunks
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void gram_partials(const float* __restrict__ Y, int rows,
                                                     long long y_bs, double* __restrict__ part) {
  __shared__ float Ys[64 * RP];
  const int b = blockIdx.y, chunk = blockIdx.x;
  const int per = (rows + GRAM_CHUNKS - 1) / GRAM_CHUNKS;
  const int lo = chunk * per, hi = min(rows, lo + per);
  Y += (long long)b * y_bs;
  const int tid = threadIdx.x;
  const int bi = tid >> 4, bj = tid & 15;   // this thread's 4x4 block of the Gram
  double g[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int c = 0; c < 4; ++c) g[a][c] = 0.0;
  for (int base = lo; base < hi; base += 64) {
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int e = tid + 256 * u;
      const int row = base + (e >> 6);
      Ys[e] = row < hi ? Y[(long long)row * RP + (e & 63)] : 0.f;
    }
    __syncthreads();
    const int nr = min(64, hi - base);
    for (int rr = 0; rr < nr; ++rr) {
      const float4 x = *(const float4*)&Ys[rr * RP + 4 * bi];
      const float4 y = *(const float4*)&Ys[rr * RP + 4 * bj];
      const double xv[4] = {x.x, x.y, x.z, x.w};
      const double yv[4] = {y.x, y.y, y.z, y.w};
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int c = 0; c < 4; ++c) g[a][c] = fma(xv[a], yv[c], g[a][c]);
    }
  }
  double* out = part + ((long long)b * GRAM_CHUNKS + chunk) * RP * RP;
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int c = 0; c < 4; ++c) out[(4 * bi + a) * RP + 4 * bj + c] = g[a][c];
}

__device__ void sum_gram_partials(const double* part, int b, int r, double (*G)[RP + 1]) {
  const double* p = part + (long long)b * GRAM_CHUNKS * RP * RP;
  for (int e = threadIdx.x; e < RP * RP; e += blockDim.x) {
    const int i = e / RP, j = e % RP;
    double s = 0.0;
    for (int c = 0; c < GRAM_CHUNKS; ++c) s += p[(long long)c * RP * RP + e];
    G[i][j] = (i < r && j < r) ? s : 0.0;
  }
}

// ---------------------------------------------------------------------------
// Cholesky of the r x r Gram (lower, in place) and M = L^-T, one workgroup per
// matrix.  A non-positive or non-finite pivot marks the matrix degenerate: M is
// then zero, so everything downstream of it is zero and the gate declines.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void chol_inv(const double* __restrict__ part, int r,
                                                float* __restrict__ M, int* __restrict__ degen) {
  __shared__ double G[RP][RP + 1];
  __shared__ double Li[RP][RP + 1];
  __shared__ int fail;
  const int b = blockIdx.x, tid = threadIdx.x;
  sum_gram_partials(part, b, r, G);
  if (tid == 0) fail = 0;
  __syncthreads();
  for (int k = 0; k < r; ++k) {
    if (tid == 0) {
      const double d = G[k][k];
      if (!(d > 0.0) || !isfinite(d)) fail = 1;
      G[k][k] = sqrt(d > 0.0 ? d : 1.0);
    }
    __syncthreads();
    const double lkk = G[k][k];
    for (int i = k + 1 + tid; i < r; i += blockDim.x) G[i][k] /= lkk;
    __syncthreads();
    const int w = r - k - 1;
    for (int e = tid; e < w * w; e += blockDim.x) {
      const int i = k + 1 + e / w, j = k + 1 + e % w;
      if (j <= i) G[i][j] -= G[i][k] * G[j][k];
    }
    __syncthreads();
  }
  // Li = L^-1 (lower): column j by forward substitution
  if (tid < r) {
    const int j = tid;
    for (int i = 0; i < r; ++i) {
      double s = (i == j) ? 1.0 : 0.0;
      for (int t = j; t < i; ++t) s -= G[i][t] * Li[t][j];
      Li[i][j] = i < j ? 0.0 : s / G[i][i];
    }
  }
  __syncthreads();
  // M = L^-T: M[a][c] = Li[c][a]
  float* Mb = M + (long long)b * RP * RP;
  for (int e = tid; e < RP * RP; e += blockDim.x) {
    const int a = e / RP, c = e % RP;
    Mb[e] = (!fail && a < r && c < r) ? (float)Li[c][a] : 0.f;
  }
  if (tid == 0 && degen) degen[b] |= fail;
}

// C (rows x RP) = Y (rows x RP) * M (RP x RP), per matrix
__global__ __launch_bounds__(256) void right_mult(const float* __restrict__ Y, int rows,
                                                  long long y_bs, const float* __restrict__ M,
                                                  float* __restrict__ C, long long c_bs) {
  __shared__ float Ms[RP * RP];
  __shared__ float Ys[64][RP + 1];
  const int b = blockIdx.y, r0 = blockIdx.x * 64, tid = threadIdx.x;
  const float* Mb = M + (long long)b * RP * RP;
  for (int e = tid; e < RP * RP; e += 256) Ms[e] = Mb[e];
  for (int e = tid; e < 64 * RP; e += 256) {
    const int row = r0 + e / RP;
    Ys[e / RP][e % RP] = row < rows ? Y[(long long)b * y_bs + (long long)row * RP + e % RP] : 0.f;
  }
  __syncthreads();
  const int col = tid & 63, rq = tid >> 6;
  for (int rr = rq; rr < 64; rr += 4) {
    float s = 0.f;
#pragma unroll 16
    for (int a = 0; a < RP; ++a) s = fmaf(Ys[rr][a], Ms[a * RP + col], s);
    const int row = r0 + rr;
    if (row < rows) C[(long long)b * c_bs + (long long)row * RP + col] = s;
  }
}

// ---------------------------------------------------------------------------
// Eigen-decomposition of H = Bp Bp^T (r x r, fp64) by cyclic Jacobi with the
// round-robin ordering (r/2 disjoint rotations per round), then the gate.
// Outputs per matrix: s (descending, fp32), Ub (RP x RP: column t = eigenvector
// of s_t), UbS = Ub diag(1/s) (for V = Bp^T Ub / s), the deflation width k and
// the deflate / restore weights cw[t] = s_t h_t, cr[t] = h_t / pad.
// ---------------------------------------------------------------------------
struct GateParams {
  int r, kw;
  float ratio, thresh, pad;
};

__global__ __launch_bounds__(256) void eig_gate(const double* __restrict__ part, GateParams gp,
                                                const int* __restrict__ degen,
                                                float* __restrict__ s_out, int s_ld,
                                                float* __restrict__ Ub, float* __restrict__ UbS,
                                                long long* __restrict__ k_out,
                                                int* __restrict__ k_int,
                                                float* __restrict__ cw, float* __restrict__ cr) {
  __shared__ double H[RP][RP + 1];
  __shared__ double V[RP][RP + 1];
  __shared__ double cs_c[RP / 2], cs_s[RP / 2];
  __shared__ int pp[RP / 2], qq[RP / 2];
  __shared__ double red[256];
  __shared__ int order[RP];
  __shared__ float sv[RP];
  const int b = blockIdx.x, tid = threadIdx.x;
  const int r = gp.r;
  sum_gram_partials(part, b, r, H);
  for (int e = tid; e < RP * RP; e += 256) V[e / RP][e % RP] = (e / RP == e % RP) ? 1.0 : 0.0;
  __syncthreads();

  const int rn = (r + 1) & ~1;   // even count for the round-robin (index r is a dummy)
  const int npairs = rn / 2;
  for (int sweep = 0; sweep < 30; ++sweep) {
    // convergence: off-diagonal mass against the diagonal
    double off = 0.0, dia = 0.0;
    for (int e = tid; e < r * r; e += 256) {
      const int i = e / r, j = e % r;
      const double h = H[i][j];
      if (i == j) dia += h * h; else off += h * h;
    }
    red[tid] = off;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) { if (tid < w) red[tid] += red[tid + w]; __syncthreads(); }
    const double offs = red[0];
    __syncthreads();
    red[tid] = dia;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) { if (tid < w) red[tid] += red[tid + w]; __syncthreads(); }
    const double dias = red[0];
    __syncthreads();
    if (offs <= 1e-30 * dias || offs == 0.0) break;

    for (int round = 0; round < rn - 1; ++round) {
      if (tid < npairs) {
        // round-robin: position 0 fixed, the others rotate
        auto slot = [&](int x) { return x == 0 ? 0 : 1 + (x - 1 + round) % (rn - 1); };
        int p = slot(tid), q = slot(rn - 1 - tid);
        if (p > q) { const int t = p; p = q; q = t; }
        double c = 1.0, s = 0.0;
        if (q < r) {
          const double hpq = H[p][q];
          if (fabs(hpq) > 1e-300) {
            const double theta = (H[q][q] - H[p][p]) / (2.0 * hpq);
            const double t = (theta >= 0 ? 1.0 : -1.0) / (fabs(theta) + sqrt(1.0 + theta * theta));
            c = 1.0 / sqrt(1.0 + t * t);
            s = t * c;
          }
        }
        pp[tid] = p; qq[tid] = q; cs_c[tid] = c; cs_s[tid] = s;
      }
      __syncthreads();
      // rows: H <- J^T H
      for (int e = tid; e < npairs * r; e += 256) {
        const int pr = e / r, col = e % r;
        const int p = pp[pr], q = qq[pr];
        if (q >= r) continue;
        const double c = cs_c[pr], s = cs_s[pr];
        const double hp = H[p][col], hq = H[q][col];
        H[p][col] = c * hp - s * hq;
        H[q][col] = s * hp + c * hq;
      }
      __syncthreads();
      // columns: H <- H J, V <- V J
      for (int e = tid; e < npairs * r; e += 256) {
        const int pr = e / r, row = e % r;
        const int p = pp[pr], q = qq[pr];
        if (q >= r) continue;
        const double c = cs_c[pr], s = cs_s[pr];
        const double hp = H[row][p], hq = H[row][q];
        H[row][p] = c * hp - s * hq;
        H[row][q] = s * hp + c * hq;
        const double vp = V[row][p], vq = V[row][q];
        V[row][p] = c * vp - s * vq;
        V[row][q] = s * vp + c * vq;
      }
      __syncthreads();
    }
  }
  // sort eigenvalues descending (stable rank; NaN ranks last)
  if (tid < RP) order[tid] = tid;
  __syncthreads();
  if (tid < r) {
    const double li = isnan(H[tid][tid]) ? -INFINITY : H[tid][tid];
    int rank = 0;
    for (int j = 0; j < r; ++j) {
      const double lj = isnan(H[j][j]) ? -INFINITY : H[j][j];
      rank += (lj > li) || (lj == li && j < tid);
    }
    order[rank] = tid;
  }
  __syncthreads();
  const bool bad = degen && degen[b];
  if (tid < RP) {
    float sval = 0.f;
    if (tid < r && !bad) {
      const double l = H[order[tid]][order[tid]];
      sval = (float)sqrt(l > 0.0 ? l : 0.0);
    }
    sv[tid] = sval;
  }
  __syncthreads();
  // gate, fp32 comparisons as torch does them (deflation_batched.py:177-180)
  __shared__ int s_kk, s_fired;
  if (tid == 0) {
    const float s0 = sv[0];
    const float thr = gp.thresh * s0;
    int kr = 0;
    for (int i = 0; i < r; ++i) kr += sv[i] > thr;
    const bool fired = (sv[gp.kw - 1] < gp.ratio * s0) && kr >= 1 && kr < r;
    int kk = kr < 1 ? 1 : (kr > r - 1 ? r - 1 : kr);
    s_kk = kk;
    s_fired = fired ? 1 : 0;
    k_out[b] = fired ? (long long)kk : 0LL;
    k_int[b] = fired ? kk : 0;
  }
  __syncthreads();
  const int kk = s_kk, fired = s_fired;
  if (tid < RP) {
    if (tid < r) s_out[(long long)b * s_ld + tid] = sv[tid];
    const float h = (fired && tid < kk) ? 1.f : 0.f;
    cw[(long long)b * RP + tid] = sv[tid] * h;
    cr[(long long)b * RP + tid] = h * (1.0f / gp.pad);
  }
  float* Ubb = Ub + (long long)b * RP * RP;
  float* UbSb = UbS + (long long)b * RP * RP;
  for (int e = tid; e < RP * RP; e += 256) {
    const int a = e / RP, t = e % RP;   // row a of Ub, column t (sorted)
    float u = 0.f;
    if (a < r && t < r && !bad) u = (float)V[a][order[t]];
    Ubb[e] = u;
    UbSb[e] = sv[t] > 0.f ? u / sv[t] : 0.f;
  }
}

// ---------------------------------------------------------------------------
// Deflate / restore.  Per 64 x 64 tile of A: W = A - sum_{t<k} U[i][t] cw[t] V[j][t]
// ---------------------------------------------------------------------------
template <bool RESTORE>
__global__ __launch_bounds__(256) void deflate_tile(
    const float* __restrict__ A, int n, int m, const float* __restrict__ U,
    const float* __restrict__ V, const int* __restrict__ kvec, const float* __restrict__ cw,
    const float* __restrict__ cr, double* __restrict__ npart, const float* __restrict__ dvec,
    void* __restrict__ X0, int out_bf16) {
  __shared__ float Us[DT][RP + 1];    // U[i][t] (row i of the tile)
  __shared__ float Vt[RP][DT + 4];    // V[j][t] transposed: Vt[t][j]
  __shared__ float cws[RP], crs[RP];
  __shared__ double red[256];
  const int b = blockIdx.z;
  const int i0 = blockIdx.y * DT, j0 = blockIdx.x * DT;
  const int tid = threadIdx.x;
  const int k = kvec[b];
  const float* Ab = A + (long long)b * n * m;
  for (int e = tid; e < DT * RP; e += 256) {
    const int rr = e / RP, t = e % RP;
    const int gi = i0 + rr, gj = j0 + rr;
    Us[rr][t] = (t < k && gi < n) ? U[((long long)b * n + gi) * RP + t] : 0.f;
    Vt[t][rr] = (t < k && gj < m) ? V[((long long)b * m + gj) * RP + t] : 0.f;
  }
  if (tid < RP) { cws[tid] = cw[b * RP + tid]; crs[tid] = cr[b * RP + tid]; }
  __syncthreads();
  const int c4 = (tid & 15) * 4;         // 4 consecutive columns
  const int rb = tid >> 4;               // rows rb, rb + 16, rb + 32, rb + 48
  float w[4][4], h[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const int gi = i0 + rb + 16 * a;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int gj = j0 + c4 + c;
      w[a][c] = (gi < n && gj < m) ? Ab[(long long)gi * m + gj] : 0.f;
      h[a][c] = 0.f;
    }
  }
  for (int t = 0; t < k; ++t) {
    const float4 v = *(const float4*)&Vt[t][c4];
    const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const float u = Us[rb + 16 * a][t];
      const float uw = u * cws[t];
      const float ur = u * crs[t];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        w[a][c] = fmaf(-uw, vv[c], w[a][c]);
        if (RESTORE) h[a][c] = fmaf(ur, vv[c], h[a][c]);
      }
    }
  }
  if (!RESTORE) {
    double s = 0.0;
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int c = 0; c < 4; ++c) s += (double)w[a][c] * (double)w[a][c];
    red[tid] = s;
    __syncthreads();
    for (int wdt = 128; wdt > 0; wdt >>= 1) {
      if (tid < wdt) red[tid] += red[tid + wdt];
      __syncthreads();
    }
    if (tid == 0) {
      const long long tiles = (long long)gridDim.x * gridDim.y;
      npart[(long long)b * tiles + blockIdx.y * gridDim.x + blockIdx.x] = red[0];
    }
  } else {
    const float d = dvec[b];
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int gi = i0 + rb + 16 * a;
      if (gi >= n) continue;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int gj = j0 + c4 + c;
        if (gj >= m) continue;
        const float x = w[a][c] / d + h[a][c];
        const long long off = (long long)b * n * m + (long long)gi * m + gj;
        if (out_bf16) ((bf16*)X0)[off] = f2bf(x);
        else ((float*)X0)[off] = x;
      }
    }
  }
}

__global__ __launch_bounds__(256) void finish_norm(const double* __restrict__ npart, int tiles,
                                                   float* __restrict__ d) {
  __shared__ double red[256];
  const int b = blockIdx.x, tid = threadIdx.x;
  double s = 0.0;
  for (int t = tid; t < tiles; t += 256) s += npart[(long long)b * tiles + t];
  red[tid] = s;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (tid < w) red[tid] += red[tid + w];
    __syncthreads();
  }
  if (tid == 0) d[b] = (float)sqrt(red[0]) + 1e-7f;
}

// strided copy of the first r of RP columns: dst (B, rows, r) contiguous
__global__ __launch_bounds__(256) void copy_cols(const float* __restrict__ src, int rows, int r,
                                                 float* __restrict__ dst) {
  const int b = blockIdx.y;
  const long long total = (long long)rows * r;
  for (long long e = blockIdx.x * 256LL + threadIdx.x; e < total; e += 256LL * gridDim.x) {
    const int row = (int)(e / r), c = (int)(e - (long long)row * r);
    dst[(long long)b * total + e] = src[((long long)b * rows + row) * RP + c];
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
struct RsvdWs {
  float *Y, *Q, *Z, *Zq, *Bt, *U, *V, *M, *Ub, *UbS, *cw, *cr, *s;
  double *gram, *npart;
  int *kint, *degen;
  float* d;
  size_t bytes;
};

static size_t align_up(size_t x) { return (x + 255) & ~(size_t)255; }

static RsvdWs rsvd_layout(void* base, int B, int n, int m) {
  RsvdWs w{};
  char* p = (char*)base;
  size_t off = 0;
  auto take = [&](size_t bytes) { char* q = p ? p + off : nullptr; off += align_up(bytes); return q; };
  const size_t nR = (size_t)B * n * RP * sizeof(float), mR = (size_t)B * m * RP * sizeof(float);
  const size_t RR = (size_t)B * RP * RP * sizeof(float);
  w.Y = (float*)take(nR);
  w.Q = (float*)take(nR);
  w.U = (float*)take(nR);
  w.Z = (float*)take(mR);
  w.Zq = (float*)take(mR);
  w.Bt = (float*)take(mR);
  w.V = (float*)take(mR);
  w.M = (float*)take(RR);
  w.Ub = (float*)take(RR);
  w.UbS = (float*)take(RR);
  w.cw = (float*)take((size_t)B * RP * sizeof(float));
  w.cr = (float*)take((size_t)B * RP * sizeof(float));
  w.s = (float*)take((size_t)B * RP * sizeof(float));
  w.d = (float*)take((size_t)B * sizeof(float));
  w.gram = (double*)take((size_t)B * GRAM_CHUNKS * RP * RP * sizeof(double));
  const size_t tiles = (size_t)ceil_div(n, DT) * ceil_div(m, DT);
  w.npart = (double*)take((size_t)B * tiles * sizeof(double));
  w.kint = (int*)take((size_t)B * sizeof(int));
  w.degen = (int*)take((size_t)B * sizeof(int));
  w.bytes = off;
  return w;
}

static int check_dims(const char* what, int B, int n, int m, int r) {
  if (B < 0 || n <= 0 || m <= 0 || r <= 0 || r > RP || r > m || n < m) {
    set_error("%s: unsupported shape (B=%d n=%d m=%d r=%d; need n >= m >= r, 1 <= r <= %d)",
              what, B, n, m, r, RP);
    return DMH_EINVAL;
  }
  return DMH_OK;
}

// Y = A X (rows n) or Y = A^T X (rows m)
static int sg(hipStream_t st, int mode, const float* A, int B, int n, int m, const float* X,
              int ld_x, int xcols, long long x_bs, float* C, long long c_bs) {
  const int outrows = mode == SG_ROWSTREAM ? n : m;
  dim3 grid(ceil_div(outrows, SG_ROWS), B);
  if (mode == SG_ROWSTREAM)
    hipLaunchKernelGGL(skinny_gemm<SG_ROWSTREAM>, grid, dim3(256), 0, st, A, n, m,
                       (long long)n * m, X, ld_x, xcols, x_bs, C, c_bs);
  else
    hipLaunchKernelGGL(skinny_gemm<SG_COLSTREAM>, grid, dim3(256), 0, st, A, n, m,
                       (long long)n * m, X, ld_x, xcols, x_bs, C, c_bs);
  DMH_CHECK_LAUNCH("skinny_gemm");
  return DMH_OK;
}

// Q = orth(Y) by CholeskyQR (Y, Q: rows x RP), `passes` times; Q may alias nothing.
static int orth(hipStream_t st, const float* Y, float* Q, float* tmp, int B, int rows, int r,
                int passes, const RsvdWs& w) {
  const float* src = Y;
  for (int p = 0; p < passes; ++p) {
    float* dst = (p == passes - 1) ? Q : (p % 2 == 0 ? tmp : Q);
    hipLaunchKernelGGL(gram_partials, dim3(GRAM_CHUNKS, B), dim3(256), 0, st, src, rows,
                       (long long)rows * RP, w.gram);
    DMH_CHECK_LAUNCH("gram_partials");
    hipLaunchKernelGGL(chol_inv, dim3(B), dim3(256), 0, st, w.gram, r, w.M, w.degen);
    DMH_CHECK_LAUNCH("chol_inv");
    hipLaunchKernelGGL(right_mult, dim3(ceil_div(rows, 64), B), dim3(256), 0, st, src, rows,
                       (long long)rows * RP, w.M, dst, (long long)rows * RP);
    DMH_CHECK_LAUNCH("right_mult");
    src = dst;
  }
  if (passes == 0) {
    hipMemcpyAsync(Q, Y, (size_t)B * rows * RP * sizeof(float), hipMemcpyDeviceToDevice, st);
    DMH_CHECK_LAUNCH("orth copy");
  }
  return DMH_OK;
}

// The subspace iteration and Rayleigh-Ritz: leaves U (n x RP), V (m x RP), the
// gate outputs and s in the workspace.
static int rsvd_core(hipStream_t st, const float* A, const float* Omega, int B, int n, int m,
                     int r, int niter, int passes, const GateParams& gp, long long* k_out,
                     const RsvdWs& w) {
  int rc;
  hipMemsetAsync(w.degen, 0, (size_t)B * sizeof(int), st);
  // Y = A Omega ; Q = orth(Y)
  if ((rc = sg(st, SG_ROWSTREAM, A, B, n, m, Omega, r, r, (long long)m * r, w.Y,
               (long long)n * RP)))
    return rc;
  if ((rc = orth(st, w.Y, w.Q, w.U, B, n, r, passes, w))) return rc;
  for (int it = 0; it < niter; ++it) {
    // Z = orth(A^T Q) ; Q = orth(A Z)
    if ((rc = sg(st, SG_COLSTREAM, A, B, n, m, w.Q, RP, RP, (long long)n * RP, w.Z,
                 (long long)m * RP)))
      return rc;
    if ((rc = orth(st, w.Z, w.Zq, w.V, B, m, r, passes, w))) return rc;
    if ((rc = sg(st, SG_ROWSTREAM, A, B, n, m, w.Zq, RP, RP, (long long)m * RP, w.Y,
                 (long long)n * RP)))
      return rc;
    if ((rc = orth(st, w.Y, w.Q, w.U, B, n, r, passes, w))) return rc;
  }
  // Bp^T = A^T Q (m x RP); H = Bp Bp^T = Gram of Bp^T
  if ((rc = sg(st, SG_COLSTREAM, A, B, n, m, w.Q, RP, RP, (long long)n * RP, w.Bt,
               (long long)m * RP)))
    return rc;
  hipLaunchKernelGGL(gram_partials, dim3(GRAM_CHUNKS, B), dim3(256), 0, st, w.Bt, m,
                     (long long)m * RP, w.gram);
  DMH_CHECK_LAUNCH("gram_partials (Bp)");
  hipLaunchKernelGGL(eig_gate, dim3(B), dim3(256), 0, st, w.gram, gp, w.degen, w.s, RP, w.Ub,
                     w.UbS, k_out, w.kint, w.cw, w.cr);
  DMH_CHECK_LAUNCH("eig_gate");
  // U = Q Ub ; V = Bp^T Ub diag(1/s)
  hipLaunchKernelGGL(right_mult, dim3(ceil_div(n, 64), B), dim3(256), 0, st, w.Q, n,
                     (long long)n * RP, w.Ub, w.U, (long long)n * RP);
  DMH_CHECK_LAUNCH("right_mult (U)");
  hipLaunchKernelGGL(right_mult, dim3(ceil_div(m, 64), B), dim3(256), 0, st, w.Bt, m,
                     (long long)m * RP, w.UbS, w.V, (long long)m * RP);
  DMH_CHECK_LAUNCH("right_mult (V)");
  return DMH_OK;
}

}  // namespace dmh

using namespace dmh;

extern "C" {

int dmh_rsvd_workspace_size(int batch, int n, int m, int r, size_t* bytes) {
  if (!bytes) {
    set_error("dmh_rsvd_workspace_size: null output");
    return DMH_EINVAL;
  }
  if (check_dims("dmh_rsvd_workspace_size", batch, n, m, r)) return DMH_EINVAL;
  *bytes = rsvd_layout(nullptr, batch, n, m).bytes;
  return DMH_OK;
}

int dmh_rmfro_workspace_size(int batch, int n, int m, int r, size_t* bytes) {
  return dmh_rsvd_workspace_size(batch, n, m, r, bytes);
}

int dmh_orth(hipStream_t stream, const float* X, int batch, int rows, int r, int passes,
             float* Q, void* ws, size_t ws_bytes) {
  if (batch == 0) return DMH_OK;
  if (!X || !Q || passes < 0) {
    set_error("dmh_orth: bad arguments (passes=%d)", passes);
    return DMH_EINVAL;
  }
  if (check_dims("dmh_orth", batch, rows, r, r)) return DMH_EINVAL;
  RsvdWs w = rsvd_layout(ws, batch, rows, r);
  if (!ws || ws_bytes < w.bytes) {
    set_error("dmh_orth: workspace %zu < %zu bytes", ws_bytes, w.bytes);
    return DMH_EWORKSPACE;
  }
  // pad X (rows x r) into Y (rows x RP), orthonormalise, copy out r columns
  hipMemsetAsync(w.degen, 0, (size_t)batch * sizeof(int), stream);
  hipMemsetAsync(w.Y, 0, (size_t)batch * rows * RP * sizeof(float), stream);
  hipMemcpy2DAsync(w.Y, RP * sizeof(float), X, r * sizeof(float), r * sizeof(float),
                   (size_t)batch * rows, hipMemcpyDeviceToDevice, stream);
  DMH_CHECK_LAUNCH("dmh_orth pack");
  int rc = orth(stream, w.Y, w.Q, w.U, batch, rows, r, passes, w);
  if (rc) return rc;
  hipLaunchKernelGGL(copy_cols, dim3(ceil_div((long long)rows * r, 256) > 4096 ? 4096 : ceil_div((long long)rows * r, 256), batch),
                     dim3(256), 0, stream, w.Q, rows, r, Q);
  DMH_CHECK_LAUNCH("copy_cols");
  return DMH_OK;
}

int dmh_rsvd(hipStream_t stream, const float* A, const float* Omega, int batch, int n, int m,
             int r, int niter, int qr_passes, float* U, float* s, float* V, void* ws,
             size_t ws_bytes) {
  if (batch == 0) return DMH_OK;
  if (!A || !Omega || !U || !s || !V || niter < 0 || qr_passes < 0) {
    set_error("dmh_rsvd: bad arguments (niter=%d qr_passes=%d)", niter, qr_passes);
    return DMH_EINVAL;
  }
  if (check_dims("dmh_rsvd", batch, n, m, r)) return DMH_EINVAL;
  RsvdWs w = rsvd_layout(ws, batch, n, m);
  if (!ws || ws_bytes < w.bytes) {
    set_error("dmh_rsvd: workspace %zu < %zu bytes", ws_bytes, w.bytes);
    return DMH_EWORKSPACE;
  }
  GateParams gp{r, 1, 0.f, 0.f, 1.f};
  long long* kdummy = (long long*)w.npart;   // gate outputs unused here
  int rc = rsvd_core(stream, A, Omega, batch, n, m, r, niter, qr_passes, gp, kdummy, w);
  if (rc) return rc;
  const int gb = ceil_div((long long)n * r, 256) > 4096 ? 4096 : ceil_div((long long)n * r, 256);
  hipLaunchKernelGGL(copy_cols, dim3(gb, batch), dim3(256), 0, stream, w.U, n, r, U);
  const int gm = ceil_div((long long)m * r, 256) > 4096 ? 4096 : ceil_div((long long)m * r, 256);
  hipLaunchKernelGGL(copy_cols, dim3(gm, batch), dim3(256), 0, stream, w.V, m, r, V);
  hipMemcpy2DAsync(s, r * sizeof(float), w.s, RP * sizeof(float), r * sizeof(float), batch,
                   hipMemcpyDeviceToDevice, stream);
  DMH_CHECK_LAUNCH("dmh_rsvd outputs");
  return DMH_OK;
}

int dmh_rmfro_clip(hipStream_t stream, const float* A, const float* Omega, int batch, int n,
                   int m, int r, int kw, float ratio, float thresh, float pad, int niter,
                   int qr_passes, void* X0, int out_bf16, long long* k, float* d, void* ws,
                   size_t ws_bytes) {
  if (batch == 0) return DMH_OK;
  if (!A || !Omega || !X0 || !k || !d || kw < 1 || kw > r || niter < 0 || qr_passes < 0 ||
      !(pad > 0.f)) {
    set_error("dmh_rmfro_clip: bad arguments (kw=%d r=%d niter=%d qr_passes=%d pad=%g)", kw, r,
              niter, qr_passes, (double)pad);
    return DMH_EINVAL;
  }
  if (check_dims("dmh_rmfro_clip", batch, n, m, r)) return DMH_EINVAL;
  RsvdWs w = rsvd_layout(ws, batch, n, m);
  if (!ws || ws_bytes < w.bytes) {
    set_error("dmh_rmfro_clip: workspace %zu < %zu bytes", ws_bytes, w.bytes);
    return DMH_EWORKSPACE;
  }
  GateParams gp{r, kw, ratio, thresh, pad};
  int rc = rsvd_core(stream, A, Omega, batch, n, m, r, niter, qr_passes, gp, k, w);
  if (rc) return rc;
  dim3 grid(ceil_div(m, DT), ceil_div(n, DT), batch);
  const int tiles = grid.x * grid.y;
  hipLaunchKernelGGL(deflate_tile<false>, grid, dim3(256), 0, stream, A, n, m, w.U, w.V, w.kint,
                     w.cw, w.cr, w.npart, nullptr, nullptr, 0);
  DMH_CHECK_LAUNCH("deflate_tile (norm)");
  hipLaunchKernelGGL(finish_norm, dim3(batch), dim3(256), 0, stream, w.npart, tiles, d);
  DMH_CHECK_LAUNCH("finish_norm");
  hipLaunchKernelGGL(deflate_tile<true>, grid, dim3(256), 0, stream, A, n, m, w.U, w.V, w.kint,
                     w.cw, w.cr, nullptr, d, X0, out_bf16);
  DMH_CHECK_LAUNCH("deflate_tile (restore)");
  return DMH_OK;
}

int dmh_project(hipStream_t stream, const float* Q, const float* A, int batch, int n, int m,
                int r, float* U, float* s, float* V, void* ws, size_t ws_bytes) {
  if (batch == 0) return DMH_OK;
  if (!Q || !A || !U || !s || !V) {
    set_error("dmh_project: null pointer argument");
    return DMH_EINVAL;
  }
  if (check_dims("dmh_project", batch, n, m, r)) return DMH_EINVAL;
  RsvdWs w = rsvd_layout(ws, batch, n, m);
  if (!ws || ws_bytes < w.bytes) {
    set_error("dmh_project: workspace %zu < %zu bytes", ws_bytes, w.bytes);
    return DMH_EWORKSPACE;
  }
  hipMemsetAsync(w.degen, 0, (size_t)batch * sizeof(int), stream);
  hipMemsetAsync(w.Q, 0, (size_t)batch * n * RP * sizeof(float), stream);
  hipMemcpy2DAsync(w.Q, RP * sizeof(float), Q, r * sizeof(float), r * sizeof(float),
                   (size_t)batch * n, hipMemcpyDeviceToDevice, stream);
  DMH_CHECK_LAUNCH("dmh_project pack");
  int rc = sg(stream, SG_COLSTREAM, A, batch, n, m, w.Q, RP, RP, (long long)n * RP, w.Bt,
              (long long)m * RP);
  if (rc) return rc;
  hipLaunchKernelGGL(gram_partials, dim3(GRAM_CHUNKS, batch), dim3(256), 0, stream, w.Bt, m,
                     (long long)m * RP, w.gram);
  DMH_CHECK_LAUNCH("gram_partials (Bp)");
  GateParams gp{r, 1, 0.f, 0.f, 1.f};
  hipLaunchKernelGGL(eig_gate, dim3(batch), dim3(256), 0, stream, w.gram, gp, w.degen, w.s, RP,
                     w.Ub, w.UbS, (long long*)w.npart, w.kint, w.cw, w.cr);
  DMH_CHECK_LAUNCH("eig_gate");
  hipLaunchKernelGGL(right_mult, dim3(ceil_div(n, 64), batch), dim3(256), 0, stream, w.Q, n,
                     (long long)n * RP, w.Ub, w.U, (long long)n * RP);
  hipLaunchKernelGGL(right_mult, dim3(ceil_div(m, 64), batch), dim3(256), 0, stream, w.Bt, m,
                     (long long)m * RP, w.UbS, w.V, (long long)m * RP);
  DMH_CHECK_LAUNCH("right_mult (U, V)");
  const int gb = ceil_div((long long)n * r, 256) > 4096 ? 4096 : ceil_div((long long)n * r, 256);
  hipLaunchKernelGGL(copy_cols, dim3(gb, batch), dim3(256), 0, stream, w.U, n, r, U);
  const int gm = ceil_div((long long)m * r, 256) > 4096 ? 4096 : ceil_div((long long)m * r, 256);
  hipLaunchKernelGGL(copy_cols, dim3(gm, batch), dim3(256), 0, stream, w.V, m, r, V);
  hipMemcpy2DAsync(s, r * sizeof(float), w.s, RP * sizeof(float), r * sizeof(float), batch,
                   hipMemcpyDeviceToDevice, stream);
  DMH_CHECK_LAUNCH("dmh_project outputs");
  return DMH_OK;
}

}  // extern "C"
