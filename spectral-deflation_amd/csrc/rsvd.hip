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
//                       (both for the shapes sk_fast() leaves out: n or m not a
//                       multiple of 8, or a matrix of 2 GiB or more)
//   sk_rows             C = A X       (n x RP)   split-bf16 MFMA 16x16x32, X staged in LDS
//   sk_cols, sk_reduce  C = A^T Y     (m x RP)   split-bf16 MFMA 32x32x16, row-split partials
//   gram_partials       partial fp64 Gram Y^T Y over row chunks (gram_partials_pair: two)
//   chol_inv            sum partials, Cholesky in LDS (fp64, blocked by 8-column
//                       panels over 8 waves), M = L^-T by blocked forward
//                       substitution  (one workgroup)
//   right_mult          C = Y M       (rows x RP) x (RP x RP)
//   eig_gate            Jacobi eigen-decomposition of Bp Bp^T in LDS (fp64) -> s, Ub;
//                       the deflation gate and the per-column deflate/restore weights
//                       and d = ||A - U diag(s h) V^T||_F + 1e-7 from r x r quantities
//   eig_head_gate       the same outputs for the clip / fused paths from the deflated
//                       eigenpairs only: Householder tridiagonalisation, multisection
//                       for the top kw eigenvalues, inverse iteration on the head
//   deflate_restore     X0 = W / d + U diag(h / pad) V^T  -> bf16 / fp32, or straight
//                       into the NS chain's packed operands (fused deflated polar)
#include "common.h"
#include "ns_chain.h"

#include <math.h>

namespace dmh {

constexpr int RP = 64;           // padded sketch width
constexpr int SG_ROWS = 128;     // output rows per skinny-GEMM workgroup
constexpr int SG_K = 32;         // K chunk
constexpr int GRAM_CHUNKS = 8;   // row chunks of the Gram reduction

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
                                                   float* __restrict__ C, long long c_bs,
                                                   double* __restrict__ asq) {
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
  double sq = 0.0;   // sum of squares of this thread's A elements (asq != nullptr)
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
    if (MODE == SG_ROWSTREAM && asq) {
      float f = 0.f;
#pragma unroll
      for (int u = 0; u < 16; ++u) f = fmaf(ra[u], ra[u], f);
      sq += (double)f;
    }
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
  if (MODE == SG_ROWSTREAM && asq) {
    __syncthreads();
    double* red = (double*)As;   // 256 doubles fit in the A tile
    red[tid] = sq;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
      if (tid < w) red[tid] += red[tid + w];
      __syncthreads();
    }
    if (tid == 0) asq[(long long)b * gridDim.x + blockIdx.x] = red[0];
  }
#undef DMH_SG_LOAD
}

// ---------------------------------------------------------------------------
// Cholesky of the r x r Gram (lower, in place) and M = L^-T, one workgroup per
// matrix.  A non-positive or non-finite pivot marks the matrix degenerate: M is
// then zero, so everything downstream of it is zero and the gate declines.
// ---------------------------------------------------------------------------
__device__ __forceinline__ double lane_val(double v, int lane) {
  const long long bits = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_readlane((int)(bits & 0xffffffffLL), lane);
  const int hi = __builtin_amdgcn_readlane((int)(bits >> 32), lane);
  return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

// 1/sqrt(x) and 1/x in fp64 from the hardware estimates plus Newton steps
// (relative error ~1e-16 for the positive normal arguments used here)
__device__ __forceinline__ double rsqrt_nr(double x) {
  double y = __builtin_amdgcn_rsq(x);
  y = y * (1.5 - 0.5 * x * y * y);
  y = y * (1.5 - 0.5 * x * y * y);
  return y;
}
__device__ __forceinline__ double rcp_nr(double x) {
  double y = __builtin_amdgcn_rcp(x);
  y = y * (2.0 - x * y);
  y = y * (2.0 - x * y);
  return y;
}

// One workgroup per matrix.  Lane l of every wave keeps row l of the (identity-padded)
// Gram, each wave a block of its columns, in registers; the factorization and the
// inversion are fully unrolled over the 64 x 64 problem.  Step k of the right-looking
// Cholesky: the wave owning column k broadcasts the pivot by readlane and publishes the
// new column L[k.., k] through LDS; every wave then updates its columns with broadcast
// LDS reads.  Entries right of the diagonal of a lane's row are updated too (their
// values are never read), which keeps the update free of per-lane predication.  Then
// L goes to LDS by rows and lane l of wave 0 computes column l of L^-1 by forward
// substitution.
constexpr int CHOL_THREADS = 512;   // all sum the Gram partials and factor; wave 0 inverts

__global__ __launch_bounds__(CHOL_THREADS) void chol_inv(const double* __restrict__ part, int r,
                                                         float* __restrict__ M,
                                                         int* __restrict__ degen) {
  constexpr int LP = RP + 2;   // row pitch (doubles): 16-byte aligned rows, 4-way at most
  constexpr int PER = RP * RP / CHOL_THREADS;
  const int b = blockIdx.x, tid = threadIdx.x, l = tid & 63;
  __shared__ __attribute__((aligned(16))) double Ls[RP * LP];   // Gram, then L by rows
  __shared__ __attribute__((aligned(16))) double Lc[RP * RP];   // row k: column k of L
  __shared__ double Ld[RP];                                     // 1 / L[k][k]
  {
    // every load of the partials issued up front (summed in chunk order)
    const double* pb = part + (long long)b * GRAM_CHUNKS * RP * RP;
    double acc[PER];
#pragma unroll
    for (int u = 0; u < PER; ++u) acc[u] = 0.0;
#pragma unroll
    for (int c = 0; c < GRAM_CHUNKS; ++c)
#pragma unroll
      for (int u = 0; u < PER; ++u) acc[u] += pb[(long long)c * RP * RP + tid + CHOL_THREADS * u];
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int e = tid + CHOL_THREADS * u;
      const int i = e / RP, j = e % RP;
      Ls[i * LP + j] = (i < r && j < r) ? acc[u] : (i == j ? 1.0 : 0.0);
    }
  }
  __syncthreads();
  // right-looking Cholesky with the columns split over the 8 waves: lane l holds row l,
  // wave w columns CW w .. CW w + CW - 1 (g[c] = G[l][CW w + c]).  Blocked by the waves'
  // column panels: the owner of panel p factors its CW columns alone (pivot k: one
  // reciprocal square root, L[.][k] formed and applied to the panel's later columns, the
  // multipliers by readlane) and publishes them in rows CW p .. of Lc; after one barrier
  // the waves of later panels apply the CW new columns to theirs.  Every element sees
  // the same operations in the same order as in a one-wave loop over k (one barrier per
  // panel instead of one per pivot: 25 -> 11 us per workgroup).
  constexpr int CW = RP / (CHOL_THREADS / 64);   // columns per wave
  static_assert(RP % (CHOL_THREADS / 64) == 0, "the waves share the columns evenly");
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  double g[CW];
#pragma unroll
  for (int c = 0; c < CW; ++c) g[c] = Ls[l * LP + CW * wave + c];
  bool fail = false;
  for (int pnl = 0; pnl < CHOL_THREADS / 64; ++pnl) {
    if (wave == pnl) {
#pragma unroll
      for (int kc = 0; kc < CW; ++kc) {
        const int k = CW * pnl + kc;
        const double dk = lane_val(g[kc], k);
        fail |= !(dk > 0.0) || !isfinite(dk);
        const double dkp = dk > 0.0 ? dk : 1.0;
        const double rs = rsqrt_nr(dkp);
        const double lik = (l > k) ? g[kc] * rs : (l == k ? dkp * rs : 0.0);
        g[kc] = lik;
        Lc[k * RP + l] = lik;
        if (l == 0) Ld[k] = rs;
#pragma unroll
        for (int c = kc + 1; c < CW; ++c) g[c] = fma(-lik, lane_val(lik, CW * pnl + c), g[c]);
      }
    }
    __syncthreads();
    if (wave > pnl) {
#pragma unroll
      for (int kc = 0; kc < CW; ++kc) {
        const int k = CW * pnl + kc;
        const double lik = Lc[k * RP + l];
#pragma unroll
        for (int c = 0; c < CW; ++c) g[c] = fma(-lik, Lc[k * RP + CW * wave + c], g[c]);
      }
    }
  }
  // L by rows into LDS (each wave its columns); a failed pivot anywhere declines
  __shared__ int s_fail;
  if (tid == 0) s_fail = 0;
  __syncthreads();
#pragma unroll
  for (int c = 0; c < CW; ++c) Ls[l * LP + CW * wave + c] = g[c];
  if (fail) s_fail = 1;
  __syncthreads();
  fail = s_fail != 0;
  // x = column l of L^-1 (lane l) by forward substitution,
  // L[i][i] x_i = delta_il - sum_{t<i} L[i][t] x_t, x_i = 0 for i < l, blocked by the
  // waves' rows: wave w holds rows CW w .. CW w + CW - 1 of every column.  Block J: wave J
  // solves its rows (the terms of its own block) and publishes them in LDS; after one
  // barrier the later waves subtract the block's terms from their rows' sums.  Each sum
  // takes its terms in the same order as a one-lane loop over t (even t in s0, odd t in
  // s1), so the inverse is bit-identical to it (16 -> 6 us per workgroup).
  double* const Xs = Lc;   // (Lc is free once L is in Ls by rows)
  double s0[CW], s1[CW], xr[CW];
#pragma unroll
  for (int q = 0; q < CW; ++q) {
    s0[q] = (CW * wave + q == l) ? 1.0 : 0.0;
    s1[q] = 0.0;
    xr[q] = 0.0;
  }
  for (int J = 0; J < CHOL_THREADS / 64; ++J) {
    if (wave == J) {
#pragma unroll
      for (int q = 0; q < CW; ++q) {
        const int i = CW * J + q;
#pragma unroll
        for (int t2 = 0; t2 < q; ++t2) {
          const double lit = Ls[i * LP + CW * J + t2];
          if (t2 & 1) s1[q] = fma(-lit, xr[t2], s1[q]);
          else s0[q] = fma(-lit, xr[t2], s0[q]);
        }
        xr[q] = (i < l) ? 0.0 : (s0[q] + s1[q]) * Ld[i];
        Xs[i * RP + l] = xr[q];
      }
    }
    __syncthreads();
    if (wave > J) {
#pragma unroll
      for (int t2 = 0; t2 < CW; ++t2) {
        const int t = CW * J + t2;
        const double xt = Xs[t * RP + l];
#pragma unroll
        for (int q = 0; q < CW; ++q) {
          const double lit = Ls[(CW * wave + q) * LP + t];
          if (t2 & 1) s1[q] = fma(-lit, xt, s1[q]);
          else s0[q] = fma(-lit, xt, s0[q]);
        }
      }
    }
  }
  static_assert(CW % 4 == 0, "the rows of a wave go out as whole float4s");
  // M = L^-T: M[a][c] = (L^-1)[c][a], so row l of M is x; wave w writes its CW entries
  float* Mb = M + (long long)b * RP * RP + (long long)l * RP + CW * wave;
#pragma unroll
  for (int q = 0; q < CW; q += 4) {
    const int c = CW * wave + q;
    float4 v;
    v.x = (!fail && l < r && c < r) ? (float)xr[q] : 0.f;
    v.y = (!fail && l < r && c + 1 < r) ? (float)xr[q + 1] : 0.f;
    v.z = (!fail && l < r && c + 2 < r) ? (float)xr[q + 2] : 0.f;
    v.w = (!fail && l < r && c + 3 < r) ? (float)xr[q + 3] : 0.f;
    *(float4*)&Mb[q] = v;
  }
  if (tid == 0 && degen && fail) degen[b] = 1;
}

// C (rows x RP) = Y (rows x RP) * M (RP x RP), per matrix; 64 rows per workgroup,
// a 4 x 4 output block per thread.  CT (optional): the same product transposed,
// RP x ldct per matrix (the layout the skinny GEMMs read their small operand in).
struct RightMult {
  const float* Y; int rows; long long y_bs;
  const float* M;
  float* C; long long c_bs;
  float* CT; int ldct;
};

// rows r0 .. r0 + 63 of matrix b
__device__ __forceinline__ void right_mult_tile(const RightMult& p, int b, int r0) {
  const float* __restrict__ Y = p.Y;
  const float* __restrict__ M = p.M;
  float* __restrict__ C = p.C;
  float* __restrict__ CT = p.CT;
  const int rows = p.rows, ldct = p.ldct;
  const long long y_bs = p.y_bs, c_bs = p.c_bs;
  __shared__ __attribute__((aligned(16))) float Ms[RP * RP];
  __shared__ __attribute__((aligned(16))) float Ys[64][RP + 4];
  const int tid = threadIdx.x;
  const float* Mb = M + (long long)b * RP * RP;
  const float* Yb = Y + (long long)b * y_bs;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int e = tid + 256 * u;              // float4 index
    *(float4*)&Ms[4 * e] = *(const float4*)&Mb[4 * e];
    const int rr = e >> 4, c4 = (e & 15) * 4;
    const int row = r0 + rr;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (row < rows) v = *(const float4*)&Yb[(long long)row * RP + c4];
    *(float4*)&Ys[rr][c4] = v;
  }
  __syncthreads();
  const int ty = tid >> 4, tx = tid & 15;
  float acc[4][4] = {};
#pragma unroll 8
  for (int a2 = 0; a2 < RP; ++a2) {
    const float4 m = *(const float4*)&Ms[a2 * RP + 4 * tx];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float y = Ys[4 * ty + i][a2];
      acc[i][0] = fmaf(y, m.x, acc[i][0]);
      acc[i][1] = fmaf(y, m.y, acc[i][1]);
      acc[i][2] = fmaf(y, m.z, acc[i][2]);
      acc[i][3] = fmaf(y, m.w, acc[i][3]);
    }
  }
  if (C) {   // (null when only the transposed product is read downstream)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = r0 + 4 * ty + i;
      if (row < rows)
        *(float4*)&C[(long long)b * c_bs + (long long)row * RP + 4 * tx] =
            make_float4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]);
    }
  }
  if (!CT) return;
  float* CTb = CT + (long long)b * RP * ldct;
  const int row0 = r0 + 4 * ty;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float* dst = CTb + (long long)(4 * tx + k) * ldct + row0;
    if (row0 + 3 < rows && (ldct & 3) == 0) {
      *(float4*)dst = make_float4(acc[0][k], acc[1][k], acc[2][k], acc[3][k]);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (row0 + i < rows) dst[i] = acc[i][k];
    }
  }
}

// grid (ceil(rows / 64), batch)
__global__ __launch_bounds__(256) void right_mult(RightMult p) {
  right_mult_tile(p, blockIdx.y, blockIdx.x * 64);
}

// two independent products in one launch (U = Q Ub and V = Bp^T Ub diag(1/s) of the
// Rayleigh-Ritz step): grid (ceil(p.rows / 64) + ceil(q.rows / 64), batch)
__global__ __launch_bounds__(256) void right_mult_pair(RightMult p, RightMult q) {
  const int np = (p.rows + 63) / 64;
  if ((int)blockIdx.x < np) right_mult_tile(p, blockIdx.y, blockIdx.x * 64);
  else right_mult_tile(q, blockIdx.y, (blockIdx.x - np) * 64);
}

// dst (RP x ldd per matrix) = src^T for src (rows x cols, leading dim lds), zero
// for the columns cols..RP-1: the transposed layout of the skinny GEMMs' small operand.
__global__ __launch_bounds__(256) void transpose_rp(const float* __restrict__ src, int rows,
                                                    int cols, int lds, long long s_bs,
                                                    float* __restrict__ dst, int ldd) {
  __shared__ float t[64][RP + 1];
  const int b = blockIdx.y, r0 = blockIdx.x * 64, tid = threadIdx.x;
  for (int e = tid; e < 64 * RP; e += 256) {
    const int rr = e / RP, c = e % RP;
    const int row = r0 + rr;
    t[rr][c] = (row < rows && c < cols) ? src[(long long)b * s_bs + (long long)row * lds + c] : 0.f;
  }
  __syncthreads();
  for (int e = tid; e < 64 * RP; e += 256) {
    const int c = e / 64, rr = e % 64;
    const int row = r0 + rr;
    if (row < rows) dst[(long long)b * RP * ldd + (long long)c * ldd + row] = t[rr][c];
  }
}

// ---------------------------------------------------------------------------
// Skinny GEMMs on bf16 MFMA with split operands.  A stays fp32 in HBM; every fp32
// value x is split on the fly into bf16 terms x = x_h + x_m + x_l (SPLITS = 3) or
// x_h + x_l (SPLITS = 2) and the product is summed over the term pairs that matter
// (6 of 9, resp. 3 of 4) in fp32 accumulators: SPLITS = 3 is accurate to fp32
// rounding (all four products of the front-end use it: the Frobenius divisor is
// formed from the Ritz values as ||A||^2 - sum lambda (2 - G), which amplifies
// their error by the head-to-remainder energy ratio), SPLITS = 2 to ~2^-16 per
// product.  No LDS: the A
// operand goes from HBM straight into MFMA operand registers, so the kernels run
// at the HBM roofline (4 B per element of A) instead of the fp32 MFMA rate.
//
// v_mfma_f32_32x32x16_bf16: lane l supplies row l%32, k = 8(l/32)..+7 of the first
// operand and column l%32 of the second; the result D[8g + 4(l/32) + q][l%32] is
// acc[4g + q].
// ---------------------------------------------------------------------------
template <int SPLITS>
__device__ __forceinline__ void split_bf16(const float (&x)[8], bf16x8 (&t)[SPLITS]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float r = x[e];
#pragma unroll
    for (int s = 0; s < SPLITS; ++s) {
      const bf16 h = f2bf(r);
      t[s][e] = h;
      r -= bf2f(h);
    }
  }
}

template <int SPLITS>
__device__ __forceinline__ f32x16 mfma_split(const bf16x8 (&a)[SPLITS], const bf16x8 (&b)[SPLITS],
                                             f32x16 acc) {
  // smallest terms first
  if (SPLITS == 3) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[1], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[2], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[2], b[0], acc, 0, 0, 0);
  }
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[0], acc, 0, 0, 0);
  return acc;
}

constexpr int SKR_ROWS = 256;   // rows of A per sk_rows workgroup (4 waves x 64)
constexpr int SKC_COLS = 256;   // columns of A per sk_cols workgroup (4 waves x 64)
// sk_cols workgroups to aim for (row splits).  Fewer splits than a full second round
// of workgroups measured faster: GPT-2-large tall group (360 column blocks) 377 us at 2
// splits vs 412 at 3; square group (720) 200 us at 1 split vs 217 at 2.
constexpr int SKC_TARGET = 720;
constexpr int SK_MAXS = 16;     // maximum row splits of sk_cols

// The small operand S of a skinny product (RP x lds fp32, row c = its column c) is the
// first MFMA operand: lane l supplies row 32 cb + l % 32 and 8 contraction indices.  A
// workgroup stages chunks of SK_KC contraction indices of S in LDS, already split into
// bf16 terms, so each chunk is read from L2 and split once per workgroup rather than
// once per wave; the waves then read their fragments from LDS.  Rows are padded to
// SK_PITCH bf16 (144 B), which makes the 16-byte fragment reads of 16 consecutive lanes
// cover the 64 banks once.  Two chunk buffers: the next chunk is written while the
// current one is read, one barrier per chunk.
constexpr int SK_KC = 64;
constexpr int SK_PITCH = SK_KC + 8;
constexpr int SK_TERM = RP * SK_PITCH;       // bf16 per split term
constexpr int SK_BUF = 3 * SK_TERM;          // bf16 per chunk buffer (up to 3 terms)

// Loads of the skinny products go through buffer descriptors: a load whose byte offset
// is at or beyond the descriptor's size returns zeros without touching memory.  Offsets
// outside a matrix (rows beyond n, indices beyond m, steps past the end) are set to
// SK_OOB, so every load is unconditional: no branches, and the compiler can count the
// loads in flight across steps.  The host keeps every operand below 2^31 bytes.
constexpr unsigned SK_OOB = 0xF0000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t sk_rsrc(const float* p, long long elems) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, (int)(elems * 4), 0x00020000);
}
__device__ __forceinline__ float4 sk_ld4(__amdgpu_buffer_rsrc_t r, unsigned off) {
  return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}
__device__ __forceinline__ float2 sk_ld2(__amdgpu_buffer_rsrc_t r, unsigned off) {
  return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0));
}
// ---------------------------------------------------------------------------
// fp64 Gram of a (rows x RP) fp32 matrix, partial over GRAM_CHUNKS row chunks: one
// wave per chunk on the fp64 MFMA (v_mfma_f64_16x16x4_f64, D[i][j] += sum_k A[i][k]
// B[k][j] over 4 rows k); a second wave per chunk, adding up through LDS, was slower.  Lane l loads row r + l/16, columns 4(l%16) .. +3 (a wave
// covers 4 whole rows, 1 KB contiguous) and supplies element c of its quad as A[l%16]
// [l/16] and B[l/16][l%16] of column class c: the product of classes c and c' is the
// 16 x 16 block G[4i + c][4j + c'].  The ten blocks c <= c' hold every entry of the
// symmetric Gram once; the store mirrors the off-diagonal classes.  Output element e of
// lane l is block entry (i, j) = (l/16 + 4e, l%16) (lane layout checked on the device).
// Products of fp32 values are exact in fp64; only the order of the fp64 sums differs
// from a row-by-row loop.  Two register sets of GRAM_G 4-row groups alternate, so one
// set's loads are in flight while the other's MFMAs run (rows at or past the chunk's
// end load zeros through the buffer descriptor).
// ---------------------------------------------------------------------------
constexpr int GRAM_G = 4;   // 4-row groups per register set

__device__ __forceinline__ void gram_mfma(const float4 (&v)[GRAM_G], f64x4 (&acc)[10]) {
#pragma unroll
  for (int u = 0; u < GRAM_G; ++u) {
    const double a[4] = {(double)v[u].x, (double)v[u].y, (double)v[u].z, (double)v[u].w};
    int t = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int c2 = c; c2 < 4; ++c2, ++t)
        acc[t] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[c], a[c2], acc[t], 0, 0, 0);
  }
}

// STAGE: the partial leaves through LDS (for short chunks: GRAM_STAGE_ROWS rows or less)
template <bool STAGE>
__device__ __forceinline__ void gram_chunk(const float* __restrict__ Y, int rows, long long y_bs,
                                           double* __restrict__ part, int b, int chunk, int l) {
  const int per = (rows + GRAM_CHUNKS - 1) / GRAM_CHUNKS;
  const int lo = chunk * per, hi = min(rows, lo + per);
  const __amdgpu_buffer_rsrc_t yr = sk_rsrc(Y + (long long)b * y_bs, (long long)rows * RP);
  const int kr = l >> 4, cq = 4 * (l & 15);
  auto load = [&](int r0, float4 (&v)[GRAM_G]) {
#pragma unroll
    for (int u = 0; u < GRAM_G; ++u) {
      const int row = r0 + 4 * u + kr;
      v[u] = sk_ld4(yr, row < hi ? (unsigned)(row * RP + cq) * 4u : SK_OOB);
    }
  };
  f64x4 acc[10];
#pragma unroll
  for (int t = 0; t < 10; ++t) acc[t] = f64x4{0.0, 0.0, 0.0, 0.0};
  constexpr int SET = 4 * GRAM_G;   // rows per register set
  float4 va[GRAM_G], vb[GRAM_G];
  load(lo, va);
  // (the empty asm statements keep each set's loads where they are: hoisted, they would
  // wait for the other set's loads still in flight)
  for (int r = lo; r < hi; r += 2 * SET) {
    load(r + SET, vb);
    asm volatile("" ::: "memory");
    gram_mfma(va, acc);
    asm volatile("" ::: "memory");
    load(r + 2 * SET, va);
    asm volatile("" ::: "memory");
    gram_mfma(vb, acc);
    asm volatile("" ::: "memory");
  }
  double* out = part + ((long long)b * GRAM_CHUNKS + chunk) * RP * RP;
  if constexpr (!STAGE) {   // long chunks: the stores are a small part, straight from registers
    int t = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int c2 = c; c2 < 4; ++c2, ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int p = 4 * (kr + 4 * e) + c, q = cq + c2;
          out[p * RP + q] = acc[t][e];
          if (c != c2) out[q * RP + p] = acc[t][e];
        }
  } else {
    // Short chunks: the partial leaves through LDS, 32 rows at a time, as whole 512-byte
    // rows (from the accumulators, the mirrored entries are 8-byte stores scattered over
    // 16 rows per instruction: a fifth of the kernel's time at 160-row chunks; at 640
    // rows the LDS kernel is 4% slower, so long chunks keep the stores from registers).
    __shared__ __attribute__((aligned(16))) double S[32][RP + 2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      int t = 0;
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int c2 = c; c2 < 4; ++c2, ++t)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int p = 4 * (kr + 4 * e) + c, q = cq + c2;
            if ((p >> 5) == h) S[p & 31][q] = acc[t][e];
            if (c != c2 && (q >> 5) == h) S[q & 31][p] = acc[t][e];
          }
      __syncthreads();
      // lane l: doubles 2 (l % 32), +1 of rows 2 i + l / 32 of this half
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = 2 * i + (l >> 5), col = 2 * (l & 31);
        *(double2*)&out[(32 * h + row) * RP + col] = *(const double2*)&S[row][col];
      }
      __syncthreads();
    }
  }
}

constexpr int GRAM_STAGE_ROWS = 256;
__host__ __device__ constexpr bool gram_stage(int rows) {
  return (rows + GRAM_CHUNKS - 1) / GRAM_CHUNKS <= GRAM_STAGE_ROWS;
}

// grid (GRAM_CHUNKS, batch); STAGE = gram_stage(rows)
template <bool STAGE>
__global__ __launch_bounds__(64) void gram_partials(const float* __restrict__ Y, int rows,
                                                    long long y_bs, double* __restrict__ part) {
  gram_chunk<STAGE>(Y, rows, y_bs, part, blockIdx.y, blockIdx.x, threadIdx.x);
}

// two independent Gram partials in one launch (Bp Bp^T and Q^T Q before the gate):
// grid (2 GRAM_CHUNKS, batch); S1, S2 = gram_stage(rows1), gram_stage(rows2)
template <bool S1, bool S2>
__global__ __launch_bounds__(64) void gram_partials_pair(const float* __restrict__ Y1, int rows1,
                                                         double* __restrict__ part1,
                                                         const float* __restrict__ Y2, int rows2,
                                                         double* __restrict__ part2) {
  if ((int)blockIdx.x < GRAM_CHUNKS)
    gram_chunk<S1>(Y1, rows1, (long long)rows1 * RP, part1, blockIdx.y, blockIdx.x, threadIdx.x);
  else
    gram_chunk<S2>(Y2, rows2, (long long)rows2 * RP, part2, blockIdx.y,
                   blockIdx.x - GRAM_CHUNKS, threadIdx.x);
}

// A copy the compiler cannot fold away: a prefetch slot is copied out before its next
// load is issued into the same registers, so the loop carries the slot in place and no
// register move of in-flight data (which would wait for the load) is needed at the
// loop's back edge.
__device__ __forceinline__ float sk_mov(float x) {
  float y;
  asm volatile("v_mov_b32 %0, %1" : "=v"(y) : "v"(x));
  return y;
}
__device__ __forceinline__ float4 sk_mov(float4 x) {
  return make_float4(sk_mov(x.x), sk_mov(x.y), sk_mov(x.z), sk_mov(x.w));
}
__device__ __forceinline__ float2 sk_mov(float2 x) { return make_float2(sk_mov(x.x), sk_mov(x.y)); }

// A chunk is 512 units: unit u is row c = u / 8, contraction indices k0 + 8 (u % 8) ..
// +7 (zero at and beyond kend; 8-index groups are whole).  With Q units per thread
// (2 for a 256-thread workgroup, 1 for 512), thread t stages the units t + (512 / Q) q.
template <int Q = 2>
struct SkStageQ {
  float4 v[Q][2];
};
typedef SkStageQ<2> SkStage;

template <int Q = 2>
__device__ __forceinline__ void sk_stage_load(SkStageQ<Q>& st, __amdgpu_buffer_rsrc_t sr, int lds,
                                              int k0, int kend, int tid) {
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const int u = tid + (512 / Q) * q;
    const int c = u >> 3, k = k0 + 8 * (u & 7);
    const unsigned off = k < kend ? (unsigned)(c * lds + k) * 4u : SK_OOB;
    st.v[q][0] = sk_ld4(sr, off);
    st.v[q][1] = sk_ld4(sr, off + 16u);
  }
}

// Keeps the split of a staged chunk at the point of this call: without it the compiler
// hoists the split to the top of the loop, where it waits for the staging loads just
// issued and with them for every prefetched load of A.
template <int Q = 2>
__device__ __forceinline__ void sk_pin(SkStageQ<Q>& st) {
#pragma unroll
  for (int q = 0; q < Q; ++q)
#pragma unroll
    for (int h = 0; h < 2; ++h)
      asm volatile("" : "+v"(st.v[q][h].x), "+v"(st.v[q][h].y), "+v"(st.v[q][h].z),
                   "+v"(st.v[q][h].w));
}

// PERM = false: index k of the chunk at position k of its row.  PERM = true: the
// order of sk_rows' 16x16 fragments -- within each 32-index step, the 4-index group
// a = 0..7 at position 8a (a < 4) or 8(a - 4) + 4 (a >= 4), so positions 8g .. 8g + 7
// hold the indices 4g .. 4g + 3 and 16 + 4g .. 16 + 4g + 3.
template <int SPLITS, bool PERM = false, int Q = 2>
__device__ __forceinline__ void sk_stage_store(const SkStageQ<Q>& st, bf16* buf, int tid) {
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const int u = tid + (512 / Q) * q;
    const int c = u >> 3, kk = 8 * (u & 7);
    const float x[8] = {st.v[q][0].x, st.v[q][0].y, st.v[q][0].z, st.v[q][0].w,
                        st.v[q][1].x, st.v[q][1].y, st.v[q][1].z, st.v[q][1].w};
    bf16x8 t[SPLITS];
    split_bf16<SPLITS>(x, t);
    if (PERM) {
      // the 8 indices are the 4-index groups a0 and a0 + 1 (a0 even) of step kk / 32
      const int a0 = (kk & 31) >> 2, step = kk & ~31;
      const int p0 = step + (a0 < 4 ? 8 * a0 : 8 * (a0 - 4) + 4), p1 = p0 + 8;
#pragma unroll
      for (int s = 0; s < SPLITS; ++s) {
        bf16* row = buf + s * SK_TERM + c * SK_PITCH;
        *(bf16x4*)(row + p0) = __builtin_shufflevector(t[s], t[s], 0, 1, 2, 3);
        *(bf16x4*)(row + p1) = __builtin_shufflevector(t[s], t[s], 4, 5, 6, 7);
      }
    } else {
#pragma unroll
      for (int s = 0; s < SPLITS; ++s) *(bf16x8*)(buf + s * SK_TERM + c * SK_PITCH + kk) = t[s];
    }
  }
}

// Fragments of the staged chunk for contraction offset koff (within the chunk) of
// this lane: rows 32 cb + l32, indices koff .. koff + 7.
template <int SPLITS>
__device__ __forceinline__ void sk_frags(const bf16* buf, int koff, int l32,
                                         bf16x8 (&xs)[2][SPLITS]) {
#pragma unroll
  for (int cb = 0; cb < 2; ++cb)
#pragma unroll
    for (int s = 0; s < SPLITS; ++s)
      xs[cb][s] = *(const bf16x8*)(buf + s * SK_TERM + (32 * cb + l32) * SK_PITCH + koff);
}

// Workgroup barrier for the chunk buffers: the LDS writes and reads issued before it
// have completed (lgkmcnt), global loads in flight stay in flight.  The empty asm
// statements keep the compiler from moving LDS accesses across it.
__device__ __forceinline__ void sk_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// The six term products of a split pair on the 16x16x32 MFMA (smallest terms first,
// as mfma_split)
template <int SPLITS>
__device__ __forceinline__ void mfma_split16(const bf16x8 (&a)[SPLITS], const bf16x8 (&b)[SPLITS],
                                             f32x4& acc) {
  if (SPLITS == 3) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[1], b[1], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b[2], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[2], b[0], acc, 0, 0, 0);
  }
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[1], b[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b[0], acc, 0, 0, 0);
}
template <int SPLITS>
__device__ __forceinline__ void mfma_split16(const bf16x8 (&a)[SPLITS], const bf16x8 (&b)[SPLITS],
                                             f32x4 (&acc)[4], int rb) {
  mfma_split16<SPLITS>(a, b, acc[rb]);
}

// C (n x RP, per matrix) = A (n x m) X, with X given transposed: XT (RP x ldxt),
// XT[c][k] = X[k][c].  Needs m % 8 == 0.  asq: per-workgroup sums of squares of A.
// v_mfma_f32_16x16x32_bf16: lane l supplies row l%16 and 8 contraction indices of
// each operand; the result D[4(l/16) + q][l%16] is acc[q].  The first operand is X
// (D's rows are C's columns c), the second A (D's columns are rows i of A).
// Wave w owns rows r0 .. r0 + 63 (four 16-row blocks rb) and all RP columns (four
// 16-column blocks cb).  A is read 32 contraction indices (128 bytes of each row) per
// step: lane (l16, g) loads the floats 4g .. 4g + 3 and 16 + 4g .. 16 + 4g + 3 of row
// 16 rb + l16, so each load instruction covers 64 contiguous bytes of 16 rows (four
// lanes per row).  The memory system serves that faster than the 32x32 MFMA's
// layout, two lanes per row and 32 rows per instruction: a loads-only probe of the two
// patterns over GPT-2-large's 72 x (5120 x 1280) fp32 ran 327 vs 400 us.  The lane's 8
// indices per step are not consecutive; the staged X chunk is stored in the same order
// (sk_stage_store<., true>), so the fragment of lane (l16, g) is 16 contiguous bytes.
template <int SPLITS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void sk_rows(const float* __restrict__ A, int n, int m,
                                               const float* __restrict__ XT, int ldxt,
                                               float* __restrict__ C, double* __restrict__ asq) {
  __shared__ __attribute__((aligned(16))) bf16 xl[2 * SK_BUF];
  const int b = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, g = lane >> 4;
  const int r0 = blockIdx.x * SKR_ROWS + wave * 64;
  A += (long long)b * n * m;
  XT += (long long)b * RP * ldxt;
  C += (long long)b * n * RP;
  const __amdgpu_buffer_rsrc_t ar = sk_rsrc(A, (long long)n * m);
  const __amdgpu_buffer_rsrc_t xr = sk_rsrc(XT, (long long)RP * ldxt);
  unsigned abase[4];   // byte offset of the lane's first float, SK_OOB for rows >= n
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    const int i = r0 + 16 * rb + l16;
    abase[rb] = i < n ? (unsigned)(i * m + 4 * g) * 4u : SK_OOB;
  }
  f32x4 acc[4][4];   // [cb][rb]
#pragma unroll
  for (int cb = 0; cb < 4; ++cb)
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[cb][rb][e] = 0.f;
  double sq = 0.0;
  const int nch = (m + SK_KC - 1) / SK_KC;  // staged chunks
  // the lane's floats of step ks: a[rb][h] = row 16 rb + l16, indices 32 ks + 16 h +
  // 4 g .. + 3 (a group at or past m loads zeros; m % 4 == 0 keeps groups whole)
  auto load = [&](int ks, float4 (&a)[4][2]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int k = 32 * ks + 16 * h;
      const bool kin = k + 4 * g < m;
#pragma unroll
      for (int rb = 0; rb < 4; ++rb)
        a[rb][h] = sk_ld4(ar, kin ? abase[rb] + (unsigned)k * 4u : SK_OOB);
    }
  };
  SkStage stg;
  sk_stage_load(stg, xr, ldxt, 0, m, tid);
  sk_stage_store<SPLITS, true>(stg, xl, tid);
  sk_stage_load(stg, xr, ldxt, SK_KC, m, tid);
  // A two steps ahead: slot p holds step 2 ch + p (SK_KC / 32 == 2 steps per chunk)
  static_assert(SK_KC == 64, "two A slots per staged chunk");
  float4 ab[2][4][2];
  load(0, ab[0]);
  load(1, ab[1]);
  sk_barrier();
  for (int ch = 0; ch < nch; ++ch) {
    const bf16* buf = xl + (ch & 1) * SK_BUF;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      // a step past the end of a partial last chunk multiplies zeros
      const int ks = 2 * ch + p;
      float4 ac[4][2];
#pragma unroll
      for (int rb = 0; rb < 4; ++rb)
#pragma unroll
        for (int h = 0; h < 2; ++h) ac[rb][h] = sk_mov(ab[p][rb][h]);
      load(ks + 2, ab[p]);
      // two row blocks at a time (the split terms of all four would cost occupancy)
#pragma unroll
      for (int rp = 0; rp < 4; rp += 2) {
        bf16x8 as[2][SPLITS];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const float4 lo = ac[rp + u][0], hi = ac[rp + u][1];
          const float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
          if (asq) {
            float f = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) f = fmaf(v[e], v[e], f);
            sq += (double)f;
          }
          split_bf16<SPLITS>(v, as[u]);
        }
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
          bf16x8 xs[SPLITS];
#pragma unroll
          for (int s = 0; s < SPLITS; ++s)
            xs[s] = *(const bf16x8*)(buf + s * SK_TERM + (16 * cb + l16) * SK_PITCH + 32 * p + 8 * g);
#pragma unroll
          for (int u = 0; u < 2; ++u) mfma_split16<SPLITS>(xs, as[u], acc[cb], rp + u);
        }
      }
    }
    // (after the last chunk this stages zeros nobody reads: no branch in the loop, so
    // the compiler keeps the prefetched loads in flight across iterations)
    sk_pin(stg);
    sk_stage_store<SPLITS, true>(stg, xl + ((ch + 1) & 1) * SK_BUF, tid);
    sk_barrier();
    sk_stage_load(stg, xr, ldxt, (ch + 2) * SK_KC, m, tid);
  }
  // D[c][i] = C[i][c]: lane holds columns c = 16 cb + 4 g + q of row i = 16 rb + l16
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    const int i = r0 + 16 * rb + l16;
    if (i >= n) continue;
#pragma unroll
    for (int cb = 0; cb < 4; ++cb)
      *(float4*)&C[(long long)i * RP + 16 * cb + 4 * g] =
          make_float4(acc[cb][rb][0], acc[cb][rb][1], acc[cb][rb][2], acc[cb][rb][3]);
  }
  if (asq) {
    __shared__ double red[256];
    red[tid] = sq;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
      if (tid < w) red[tid] += red[tid + w];
      __syncthreads();
    }
    if (tid == 0) asq[(long long)b * gridDim.x + blockIdx.x] = red[0];
  }
}

// sk_rows with A streamed global -> LDS by the gfx950 direct-to-LDS load
// (buffer_load_dwordx4 ... lds) instead of into registers.  Same products, same
// operands, same order per accumulator, so C is bit-identical to sk_rows'.  Loads that
// land in registers compete with the MFMAs that read registers: a read-only stream over
// GPT-2-large's 72 x (5120 x 1280) fp32 that also issues 96 16x16x32 MFMAs per 8 KB per
// wave ran at 4.1 TB/s with register loads, 5.7 TB/s with the same bytes landing in LDS.
// WV waves of 256 / WV rows each (8 waves of 32 rows, two per SIMD, one workgroup
// per compute unit: 457 vs 542 us for 4 waves of 64 rows, one per SIMD, on the tall
// group; sk_rows 508 us); each wave streams its own rows in stages
// of 32 contraction indices (128 bytes of each row) through a ring of SKD_NST stages
// of its own, so the ring needs no workgroup barrier; the small operand is staged and
// split per 64-index chunk as in sk_rows (one barrier per chunk).  Stage row r holds
// the row's 16-byte chunk c in slot c ^ ((r >> 1) & 7): the fragment reads (16
// consecutive rows, one chunk) then cover the 64 banks once.  The per-workgroup sums
// of squares add the same values in another order (8 waves) than sk_rows.  Needs
// m % 64 == 0.
constexpr int SKD_NST = 3;   // A stages in flight per wave

typedef __attribute__((address_space(3))) void* sk_lds_ptr;

__device__ __forceinline__ void sk_load_lds16(__amdgpu_buffer_rsrc_t r, char* lds, int voff,
                                              int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (sk_lds_ptr)lds, 16, voff, soff, 0, 0);
}

__device__ __forceinline__ int skd_slot(int r, int c) { return c ^ ((r >> 1) & 7); }

// vmcnt(n) with expcnt and lgkmcnt left at their maxima
__device__ __forceinline__ void skd_wait_vm(int n) {
  switch (n) {
    case 10: __builtin_amdgcn_s_waitcnt(0x0F7A); break;
    case 20: __builtin_amdgcn_s_waitcnt(0x4F74); break;
    default: __builtin_amdgcn_s_waitcnt(0x0F70); break;
  }
}

template <int SPLITS, int WV>
__global__ __launch_bounds__(64 * WV) __attribute__((amdgpu_waves_per_eu(1, 1))) void sk_rows_dtl(
    const float* __restrict__ A, int n, int m, const float* __restrict__ XT, int ldxt,
    float* __restrict__ C, double* __restrict__ asq) {
  constexpr int NT = 64 * WV, RPW = SKR_ROWS / WV, NRB = RPW / 16;
  constexpr int WSTAGE = RPW * 128;       // bytes of one wave's stage
  constexpr int LPS = WSTAGE / 1024;      // direct-to-LDS loads per wave and stage
  constexpr int Q = 512 / NT;             // staging units per thread
  // Vector memory instructions in issue order: stage s's LPS loads, then s+1's, the
  // next chunk's 2 Q staging loads, s+2's; so when stage s is read, VM_AFTER issued
  // after it may still be in flight (the same count at both steps of a chunk).  Stages
  // past the end are loaded too (into slots nobody reads; rows past the matrix load
  // zeros), so that count holds to the last step.
  constexpr int VM_AFTER = 2 * LPS + 2 * Q;
  static_assert(VM_AFTER == 10 || VM_AFTER == 20, "skd_wait_vm");
  static_assert(NRB % 2 == 0, "row blocks go in pairs");
  // One LDS array for the A ring, the staged small operand and the final reduction:
  // with separate arrays the compiler tags their accesses with alias scopes and then
  // makes every read of the ring wait for all direct-to-LDS loads in flight
  // (vmcnt(0)), which would leave no stage in flight; the waits here are explicit.
  __shared__ __attribute__((aligned(1024))) char smem[SKD_NST * WV * WSTAGE + 2 * SK_BUF * 2];
  char* const aring = smem;
  bf16* const xl = (bf16*)(smem + SKD_NST * WV * WSTAGE);
  const int b = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, g = lane >> 4;
  const int r0 = blockIdx.x * SKR_ROWS + wave * RPW;
  A += (long long)b * n * m;
  XT += (long long)b * RP * ldxt;
  C += (long long)b * n * RP;
  // the wave's rows only: rows at or past n load zeros
  const int rh = n - r0;
  const int rows_here = __builtin_amdgcn_readfirstlane(rh < 0 ? 0 : (rh > RPW ? RPW : rh));
  const __amdgpu_buffer_rsrc_t ar =
      sk_rsrc(A + (long long)(rh > 0 ? r0 : 0) * m, (long long)rows_here * m);
  const __amdgpu_buffer_rsrc_t xr = sk_rsrc(XT, (long long)RP * ldxt);
  // load q of a stage: rows 8 q + lane / 8, the row's chunk (lane % 8) ^ swizzle into
  // LDS slot lane % 8 (the stage's k offset goes in the scalar offset)
  int voff[LPS];
#pragma unroll
  for (int q = 0; q < LPS; ++q) {
    const int r = 8 * q + lane / 8;
    voff[q] = r * m * 4 + skd_slot(r, lane % 8) * 16;
  }
  char* const wring = aring + wave * WSTAGE;   // slot j at wring + j * WV * WSTAGE
#define SKD_ISSUE(s_)                                                                  \
  do {                                                                                 \
    char* dst_ = wring + ((s_) % SKD_NST) * WV * WSTAGE;                               \
    _Pragma("unroll") for (int q = 0; q < LPS; ++q)                                    \
      sk_load_lds16(ar, dst_ + q * 1024, voff[q], (s_) * 128);                         \
  } while (0)
  // the lane's fragment offsets within a stage: row 16 rb + l16, chunks g and 4 + g
  int foff[NRB][2];
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int r = 16 * rb + l16;
      foff[rb][h] = r * 128 + skd_slot(r, 4 * h + g) * 16;
    }
  f32x4 acc[4][NRB];   // [cb][rb]
#pragma unroll
  for (int cb = 0; cb < 4; ++cb)
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[cb][rb][e] = 0.f;
  double sq = 0.0;
  const int nch = m / SK_KC;
  // (the next chunk's staging loads are issued and consumed within one iteration:
  // carried across the loop's back edge, their registers were copied at the loop head,
  // which waited for them)
  {
    SkStageQ<Q> stg;
    sk_stage_load<Q>(stg, xr, ldxt, 0, m, tid);
    sk_stage_store<SPLITS, true, Q>(stg, xl, tid);
  }
  SKD_ISSUE(0);
  SKD_ISSUE(1);
  sk_barrier();
  for (int ch = 0; ch < nch; ++ch) {
    const bf16* buf = xl + (ch & 1) * SK_BUF;
    SkStageQ<Q> stg;
    sk_stage_load<Q>(stg, xr, ldxt, (ch + 1) * SK_KC, m, tid);
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int ks = 2 * ch + p;
      SKD_ISSUE(ks + 2);
      skd_wait_vm(VM_AFTER);   // stage ks has landed
      const char* st = wring + (ks % SKD_NST) * WV * WSTAGE;
#pragma unroll
      for (int rp = 0; rp < NRB; rp += 2) {
        bf16x8 as[2][SPLITS];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const f32x4 lo = *(const f32x4*)(st + foff[rp + u][0]);
          const f32x4 hi = *(const f32x4*)(st + foff[rp + u][1]);
          const float v[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          if (asq) {
            float f = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) f = fmaf(v[e], v[e], f);
            sq += (double)f;
          }
          split_bf16<SPLITS>(v, as[u]);
        }
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
          bf16x8 xs[SPLITS];
#pragma unroll
          for (int s = 0; s < SPLITS; ++s)
            xs[s] = *(const bf16x8*)(buf + s * SK_TERM + (16 * cb + l16) * SK_PITCH + 32 * p + 8 * g);
#pragma unroll
          for (int u = 0; u < 2; ++u) mfma_split16<SPLITS>(xs, as[u], acc[cb][rp + u]);
        }
      }
    }
    sk_pin<Q>(stg);
    sk_stage_store<SPLITS, true, Q>(stg, xl + ((ch + 1) & 1) * SK_BUF, tid);
    sk_barrier();
  }
#undef SKD_ISSUE
  // every load issued has landed before the wave ends (the last ones fill unread slots)
  skd_wait_vm(0);
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb) {
    const int i = r0 + 16 * rb + l16;
    if (i >= n) continue;
#pragma unroll
    for (int cb = 0; cb < 4; ++cb)
      *(float4*)&C[(long long)i * RP + 16 * cb + 4 * g] =
          make_float4(acc[cb][rb][0], acc[cb][rb][1], acc[cb][rb][2], acc[cb][rb][3]);
  }
  if (asq) {
    double* red = (double*)smem;   // the ring is no longer read
    __syncthreads();
    red[tid] = sq;
    __syncthreads();
    for (int w = NT / 2; w > 0; w >>= 1) {
      if (tid < w) red[tid] += red[tid + w];
      __syncthreads();
    }
    if (tid == 0) asq[(long long)b * gridDim.x + blockIdx.x] = red[0];
  }
}

// Partial C = A^T Y over the rows [s * rps, (s+1) * rps) of split s = blockIdx.y:
// part[s][b] (m x RP) = sum_i A[i][j] Y[i][c], with Y given transposed: YT (RP x
// ldyt), YT[c][i] = Y[i][c] (staged in LDS like sk_rows' X).  Wave w owns 64 columns
// of A; lane l reads the columns j0 + 2 l32 + {0, 1} of 8 consecutive rows, i.e. two
// 32-column MFMA blocks (block e holds the columns j0 + 2 l32 + e).  Needs m % 2 == 0,
// n % 8 == 0 and rps % 16 == 0.
template <int SPLITS>
__global__ __launch_bounds__(256) void sk_cols(const float* __restrict__ A, int n, int m,
                                               const float* __restrict__ YT, int ldyt, int rps,
                                               float* __restrict__ part) {
  __shared__ __attribute__((aligned(16))) bf16 yl[2 * SK_BUF];
  const int b = blockIdx.z, s = blockIdx.y, tid = threadIdx.x, lane = tid & 63,
            wave = tid >> 6;
  const int l32 = lane & 31, hk = lane >> 5;
  const int nb = gridDim.z;
  const int j0 = blockIdx.x * SKC_COLS + 64 * wave;
  const int jl = j0 + 2 * l32;           // this lane's two columns
  const bool jin = jl < m;
  A += (long long)b * n * m;
  YT += (long long)b * RP * ldyt;
  const int ib = s * rps, ie = min(n, ib + rps);
  f32x16 acc[2][2];   // [e][cb]
#pragma unroll
  for (int e = 0; e < 2; ++e)
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[e][cb][v] = 0.f;
  const int nch = (ie - ib + SK_KC - 1) / SK_KC;
  const __amdgpu_buffer_rsrc_t ar = sk_rsrc(A, (long long)n * m);
  const __amdgpu_buffer_rsrc_t yr = sk_rsrc(YT, (long long)RP * ldyt);
  // rows ib + 16 ks + 8 hk .. +7 of the lane's two columns (a step at or past nk, or a
  // column beyond m, loads zeros)
  const unsigned cbase = jin ? (unsigned)jl * 4u : SK_OOB;
  auto load = [&](int ks, float2 (&a)[8]) {
    const int i0 = ib + 16 * ks + 8 * hk;
    const bool iin = i0 < ie;            // 8-row groups are whole
#pragma unroll
    for (int t = 0; t < 8; ++t)
      a[t] = sk_ld2(ar, iin ? cbase + (unsigned)((i0 + t) * m) * 4u : SK_OOB);
  };
  SkStage stg;
  sk_stage_load(stg, yr, ldyt, ib, ie, tid);
  sk_stage_store<SPLITS>(stg, yl, tid);
  sk_stage_load(stg, yr, ldyt, ib + SK_KC, ie, tid);
  // A two substeps ahead: slot p & 1 holds substep ks (SK_KC / 16 == 4 per chunk)
  static_assert(SK_KC % 32 == 0, "an even number of A substeps per staged chunk");
  float2 ab[2][8];
  load(0, ab[0]);
  load(1, ab[1]);
  sk_barrier();
  for (int ch = 0; ch < nch; ++ch) {
    const bf16* buf = yl + (ch & 1) * SK_BUF;
#pragma unroll
    for (int p = 0; p < SK_KC / 16; ++p) {
      // a substep past nk (the end of a partial last chunk) multiplies zeros
      const int ks = ch * (SK_KC / 16) + p;
      float2 ac[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) ac[t] = sk_mov(ab[p & 1][t]);
      load(ks + 2, ab[p & 1]);
      bf16x8 as[2][SPLITS], ys[2][SPLITS];
      {
        const float v0[8] = {ac[0].x, ac[1].x, ac[2].x, ac[3].x, ac[4].x, ac[5].x, ac[6].x, ac[7].x};
        const float v1[8] = {ac[0].y, ac[1].y, ac[2].y, ac[3].y, ac[4].y, ac[5].y, ac[6].y, ac[7].y};
        split_bf16<SPLITS>(v0, as[0]);
        split_bf16<SPLITS>(v1, as[1]);
      }
      sk_frags<SPLITS>(buf, 16 * p + 8 * hk, l32, ys);
#pragma unroll
      for (int e = 0; e < 2; ++e)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) acc[e][cb] = mfma_split<SPLITS>(ys[cb], as[e], acc[e][cb]);
    }
    // (after the last chunk this stages zeros nobody reads: no branch in the loop)
    sk_pin(stg);
    sk_stage_store<SPLITS>(stg, yl + ((ch + 1) & 1) * SK_BUF, tid);
    sk_barrier();
    sk_stage_load(stg, yr, ldyt, ib + (ch + 2) * SK_KC, ie, tid);
  }
  // D[c][col] = C[j][c], col = l32 -> j = j0 + 2 l32 + e
  float* pb = part + ((long long)s * nb + b) * m * RP;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int j = jl + e;
    if (!jin) continue;
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *(float4*)&pb[(long long)j * RP + 32 * cb + 8 * g + 4 * hk] =
            make_float4(acc[e][cb][4 * g], acc[e][cb][4 * g + 1], acc[e][cb][4 * g + 2],
                        acc[e][cb][4 * g + 3]);
  }
}

// C[b] = sum_s part[s][b] in split order (deterministic), float4 per thread
__global__ __launch_bounds__(256) void sk_reduce(const float* __restrict__ part, int nsplit,
                                                 long long per_split, float* __restrict__ C) {
  const long long e4 = (long long)blockIdx.x * 256 + threadIdx.x;
  if (e4 * 4 >= per_split) return;
  float4 acc = *(const float4*)&part[e4 * 4];
  for (int s = 1; s < nsplit; ++s) {
    const float4 v = *(const float4*)&part[(long long)s * per_split + e4 * 4];
    acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
  }
  *(float4*)&C[e4 * 4] = acc;
}

// ---------------------------------------------------------------------------
// Eigen-decomposition of H = Bp Bp^T (r x r, fp64) by parallel cyclic Jacobi
// (round-robin ordering: RP/2 disjoint rotations per round, all pairs once per
// sweep of RP-1 rounds), one 256-thread workgroup per matrix.
//
// Storage order.  H and V are kept permuted so that every round rotates the
// fixed pairs (2t, 2t+1): with the tournament schedule "position 0 stays, the
// others move one seat", the positions of round rd+1 are those of round rd
// taken through a fixed permutation sigma, applied while the rotated matrix is
// written to the other buffer:  H <- Pi^T (J^T H J) Pi,  V <- V J Pi.  The
// invariant H = V^T H0 V holds throughout, so at the end diag(H) are the
// eigenvalues and the columns of V (original coordinates) their eigenvectors;
// perm[] tracks the original index of each position (rows/columns >= r are
// zero padding and never rotate).  All addresses are then fixed per thread.
//
// One round, one barrier: every wave computes all 32 angles itself from the
// current buffer (identical results), then the workgroup writes the next
// buffer: the 2x2 blocks (t, u), t <= u, as R_t^T X R_u (diagonal blocks by the
// Golub-Van Loan update h_pp -= tan h_pq, h_qq += tan h_pq, h_pq = 0), and V's
// column pairs.  Every round moves the seats, rotating or not, so that each
// sweep visits every pair.  A pair is not rotated when h_pq^2 <= 1e-24 |h_pp h_qq|
// or |h_pq| <= 1e-15 trace(H); after each sweep the whole of H is checked
// against the same test, and the iteration ends when no pair passes it.  Then
// the gate.
// Outputs per matrix: s (descending, fp32), Ub (RP x RP: column t = eigenvector
// of s_t), UbS = Ub diag(1/s) (for V = Bp^T Ub / s), the deflation width k and
// the deflate / restore weights cw[t] = s_t h_t, cr[t] = h_t / pad.
// ---------------------------------------------------------------------------
struct GateParams {
  int r, kw;
  float ratio, thresh, pad;
};

constexpr int JP = RP + 2;   // H row pitch (doubles): rows 16-byte aligned
constexpr int NPAIR = RP / 2;
constexpr int EG_THREADS = 512;
constexpr int EG_WAVES = EG_THREADS / 64;
constexpr int EG_OFF = NPAIR * (NPAIR - 1) / 2;   // off-diagonal 2x2 blocks (t < u)
constexpr int VR = RP / EG_WAVES;                 // rows of V per wave
static_assert(EG_OFF <= EG_THREADS && EG_OFF > EG_THREADS - 64,
              "one off-diagonal block per thread, the last wave partly idle");
static_assert(VR * EG_WAVES == RP, "V rows split evenly over the waves");

// next-round position of the element at position x (inverse of the seat move)
__device__ __forceinline__ int jac_next(int x) {
  if (x == 0) return 0;
  if (x == 2) return 1;
  if (x == RP - 1) return RP - 2;
  return (x & 1) ? x + 2 : x - 2;
}


__global__ __launch_bounds__(EG_THREADS) void eig_gate(const double* __restrict__ part,
                                                       GateParams gp,
                                                       const int* __restrict__ degen,
                                                       float* __restrict__ s_out, int s_ld,
                                                       float* __restrict__ Ub,
                                                       float* __restrict__ UbS,
                                                       long long* __restrict__ k_out,
                                                       int* __restrict__ k_int,
                                                       float* __restrict__ cw,
                                                       float* __restrict__ cr,
                                                       const double* __restrict__ qpart,
                                                       const double* __restrict__ asq, int asq_n,
                                                       float* __restrict__ d_out,
                                                       int* __restrict__ wflag) {
  __shared__ __attribute__((aligned(16))) double Hs[2][RP * JP];   // upper triangle in use
  // per wave: c, s, tan of pair t in slot t (slots 32.. take the duplicates of lanes 32..)
  __shared__ __attribute__((aligned(16))) double ang[EG_WAVES][64][4];
  __shared__ float Vf[RP * (RP + 1)];     // eigenvectors at the end, column = original index
  __shared__ int perm[3][RP];             // original index of each position (3 rounds)
  __shared__ double s_tr;
  __shared__ int order[RP];
  __shared__ float sv[RP];
  const int b = blockIdx.x, tid = threadIdx.x, l = tid & 63, wave = tid >> 6;
  const int r = gp.r;
  {
    const double* pb = part + (long long)b * GRAM_CHUNKS * RP * RP;
#pragma unroll
    for (int e = tid; e < RP * RP; e += EG_THREADS) {
      const int i = e / RP, j = e % RP;
      double acc = 0.0;
#pragma unroll
      for (int c = 0; c < GRAM_CHUNKS; ++c) acc += pb[(long long)c * RP * RP + e];
      Hs[0][i * JP + j] = (i < r && j < r) ? acc : 0.0;
    }
    if (tid < RP) perm[0][tid] = tid;
  }
  __syncthreads();
  // absolute floor for |h_pq| (trace H = sum of the eigenvalues, invariant): off-
  // diagonals at rounding level relative to the largest eigenvalue stop rotating,
  // which guarantees the sweeps end
  if (wave == 0) {
    double tr = (l < r) ? fabs(Hs[0][l * JP + l]) : 0.0;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) tr += __shfl_xor(tr, o);
    if (l == 0) s_tr = tr;
  }
  __syncthreads();
  const double floor_pq = 1e-15 * s_tr;

  // H: only the upper triangle (row <= column) is read and written after the load.
  // Thread T < EG_OFF rotates the off-diagonal block (t, u), t < u, with u running
  // fastest over consecutive threads (contiguous LDS rows); lanes 0..31 of the last
  // wave also write the diagonal blocks, from their angle computation.  Read offsets
  // (current buffer) and write offsets (next buffer, through the seat move, folded
  // into the upper triangle) are fixed per thread.
  auto up = [](int i, int j) { return i <= j ? i * JP + j : j * JP + i; };
  int bt = 0, bu = 0, rp = 0, rq = 0, wr[4] = {0, 0, 0, 0}, dw[3];
  if (tid < EG_OFF) {
    int t = 0, rem = tid;
    while (rem >= NPAIR - 1 - t) { rem -= NPAIR - 1 - t; ++t; }
    bt = t;
    bu = t + 1 + rem;
    const int p = 2 * bt, q = p + 1, p2 = 2 * bu, q2 = p2 + 1;
    rp = p * JP + p2;   // (p, p2), (p, q2)
    rq = q * JP + p2;   // (q, p2), (q, q2)
    const int np_ = jac_next(p), nq = jac_next(q), np2 = jac_next(p2), nq2 = jac_next(q2);
    wr[0] = up(np_, np2); wr[1] = up(np_, nq2); wr[2] = up(nq, np2); wr[3] = up(nq, nq2);
  }
  {
    const int t = l & (NPAIR - 1), p = 2 * t, q = p + 1;
    dw[0] = up(jac_next(p), jac_next(p));
    dw[1] = up(jac_next(p), jac_next(q));
    dw[2] = up(jac_next(q), jac_next(q));
  }
  const bool diag_writer = wave == EG_WAVES - 1 && l < NPAIR;
  // V (the accumulated rotations) in registers: lane l holds column l (the original
  // index l, which never moves) for rows VR wave .. VR wave + VR - 1.  A round rotates
  // the columns of the position pairs (2t, 2t + 1): lane l finds its position and its
  // partner's original index in perm and takes the partner's values by a lane shuffle,
  // so V costs no LDS traffic.  V's update for a round runs at the start of the next
  // one, beside that round's angle computation (the two are independent, and both
  // are latency chains); perm is kept for three rounds for it.
  float v[VR];
#pragma unroll
  for (int i = 0; i < VR; ++i) v[i] = (VR * wave + i == l) ? 1.f : 0.f;
  int pos = l, pb = 0;
  // the previous round: position, angles (lanes 0..31), perm buffer; the first
  // update is the identity (c = 1, s = 0)
  int ppos = l, ppb = 0;
  float pcf = 1.f, psf = 0.f;
  auto vstep = [&]() {
    const int pc = perm[ppb][ppos ^ 1];   // the partner's original index (= its lane)
    const float c = __shfl(pcf, ppos >> 1), s = __shfl(psf, ppos >> 1);
    const bool isp = (ppos & 1) == 0;
#pragma unroll
    for (int i = 0; i < VR; ++i) {
      const float o = __shfl(v[i], pc);
      v[i] = isp ? c * v[i] - s * o : s * o + c * v[i];
    }
  };

  int cur = 0;
  for (int sweep = 0; sweep < 40; ++sweep) {
    for (int rd = 0; rd < RP - 1; ++rd) {
      const double* Hc = Hs[cur];
      double* Hn = Hs[cur ^ 1];
      vstep();
      // angles of the round, every lane without branches (lane l: pair l % 32)
      float cf, sf;
      {
        const int t = l & (NPAIR - 1);
        const double2 pq = *(const double2*)&Hc[(2 * t) * JP + 2 * t];   // h_pp, h_pq
        const double hpp = pq.x, hpq = pq.y;
        const double hqq = Hc[(2 * t + 1) * JP + 2 * t + 1];
        const bool rot = hpq * hpq > 1e-24 * fabs(hpp * hqq) && fabs(hpq) > floor_pq;
        const double theta = (hqq - hpp) * (0.5 * rcp_nr(rot ? hpq : 1.0));
        const double th2 = theta * theta;
        // |theta| + sqrt(1 + theta^2)
        const double den = fabs(theta) + (1.0 + th2) * rsqrt_nr(1.0 + th2);
        const double tr_ = (theta >= 0 ? 1.0 : -1.0) * rcp_nr(den);
        const double cr_ = rsqrt_nr(1.0 + tr_ * tr_);
        const double c = rot ? cr_ : 1.0, sn = rot ? tr_ * cr_ : 0.0, tn = rot ? tr_ : 0.0;
        *(double2*)&ang[wave][l][0] = make_double2(c, sn);
        ang[wave][l][2] = tn;
        cf = (float)c;
        sf = (float)sn;
        if (diag_writer) {   // the diagonal block of pair t (Golub-Van Loan update)
          Hn[dw[0]] = hpp - tn * hpq;
          Hn[dw[1]] = tn == 0.0 ? hpq : 0.0;   // unrotated pairs keep h_pq
          Hn[dw[2]] = hqq + tn * hpq;
        }
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // this wave's angles are in LDS
      if (tid < EG_OFF) {
        const double2 xp = *(const double2*)&Hc[rp], xq = *(const double2*)&Hc[rq];
        const double2 a1 = *(const double2*)&ang[wave][bt][0];
        const double2 a2 = *(const double2*)&ang[wave][bu][0];
        const double c1 = a1.x, s1 = a1.y, c2 = a2.x, s2 = a2.y;
        // rows: R_t^T X, then columns: (R_t^T X) R_u
        const double y00 = c1 * xp.x - s1 * xq.x, y01 = c1 * xp.y - s1 * xq.y;
        const double y10 = s1 * xp.x + c1 * xq.x, y11 = s1 * xp.y + c1 * xq.y;
        Hn[wr[0]] = c2 * y00 - s2 * y01;
        Hn[wr[1]] = s2 * y00 + c2 * y01;
        Hn[wr[2]] = c2 * y10 - s2 * y11;
        Hn[wr[3]] = s2 * y10 + c2 * y11;
      }
      const int nb = pb == 2 ? 0 : pb + 1;
      if (l < RP / EG_WAVES) {
        const int x = (RP / EG_WAVES) * wave + l;
        perm[nb][jac_next(x)] = perm[pb][x];
      }
      ppos = pos; ppb = pb; pcf = cf; psf = sf;
      pos = jac_next(pos);
      pb = nb;
      __syncthreads();
      cur ^= 1;
    }
    // converged when no off-diagonal entry would still rotate
    const double* Hc = Hs[cur];
    int live = 0;
    for (int e = tid; e < RP * RP; e += EG_THREADS) {
      const int i = e / RP, j = e % RP;
      if (i < j) {
        const double h = Hc[i * JP + j];
        live |= h * h > 1e-24 * fabs(Hc[i * JP + i] * Hc[j * JP + j]) && fabs(h) > floor_pq;
      }
    }
    if (!__syncthreads_or(live)) break;
  }
  vstep();   // the last round's V update
#pragma unroll
  for (int i = 0; i < VR; ++i) Vf[(VR * wave + i) * (RP + 1) + l] = v[i];
  const double* H = Hs[cur];
  const int* pm = perm[pb];
  __syncthreads();
  // sort eigenvalues descending over the real positions (original index < r;
  // stable rank; NaN ranks last)
  if (tid < RP) {
    const bool real = pm[tid] < r;
    const double li = isnan(H[tid * JP + tid]) ? -INFINITY : H[tid * JP + tid];
    int rank = 0;
    for (int j = 0; j < RP; ++j) {
      if (pm[j] >= r) continue;
      const double lj = isnan(H[j * JP + j]) ? -INFINITY : H[j * JP + j];
      rank += (lj > li) || (lj == li && j < tid);
    }
    if (real) order[rank] = tid;
  }
  __syncthreads();
  const bool bad = degen && degen[b];
  if (tid < RP) {
    float sval = 0.f;
    if (tid < r && !bad) {
      const double ev = H[order[tid] * JP + order[tid]];
      sval = (float)sqrt(ev > 0.0 ? ev : 0.0);
    }
    sv[tid] = sval;
  }
  __syncthreads();
  // gate, fp32 comparisons as torch does them (deflation_batched.py:177-180)
  const float s0 = sv[0];
  const float thr = gp.thresh * s0;
  int kr = 0;
  for (int j = 0; j < r; ++j) kr += sv[j] > thr;
  const bool fired = (sv[gp.kw - 1] < gp.ratio * s0) && kr >= 1 && kr < r;
  const int kk = kr < 1 ? 1 : (kr > r - 1 ? r - 1 : kr);
  if (tid == 0) {
    k_out[b] = fired ? (long long)kk : 0LL;
    k_int[b] = fired ? kk : 0;
  }
  if (tid < RP) {
    if (tid < r) s_out[(long long)b * s_ld + tid] = sv[tid];
    const float h = (fired && tid < kk) ? 1.f : 0.f;
    cw[(long long)b * RP + tid] = sv[tid] * h;
    cr[(long long)b * RP + tid] = h * (1.0f / gp.pad);
  }
  float* Ubb = Ub + (long long)b * RP * RP;
  float* UbSb = UbS + (long long)b * RP * RP;
  for (int e = tid; e < RP * RP; e += EG_THREADS) {
    const int a = e / RP, t = e % RP;   // row a of Ub, column t (sorted)
    float u = 0.f;
    if (a < r && t < r && !bad) u = Vf[a * (RP + 1) + pm[order[t]]];
    Ubb[e] = u;
    UbSb[e] = sv[t] > 0.f ? u / sv[t] : 0.f;
  }
  if (!d_out || wave != 0) return;
  // ||W||_F^2 for W = A - sum_{t<k} s_t U_t V_t^T with U_t = Q Ub_t, V_t = Bp^T Ub_t / s_t:
  //   <A, U_t V_t^T> = Ub_t^T (Q^T A)(A^T Q) Ub_t / s_t = lambda_t / s_t,
  //   V_t^T V_t' = delta_tt' lambda_t / s_t^2,  U_t^T U_t = Ub_t^T (Q^T Q) Ub_t = G_t,
  // so ||W||^2 = ||A||^2 - sum_{t<k} lambda_t (2 - G_t).  Q^T Q is kept (not assumed
  // to be I): single-pass CholeskyQR in fp32 leaves it ~kappa*eps off the identity,
  // and the reference's explicit W sees the same Q.  (Wave 0 only; the spare H
  // buffer is no longer read by the other waves, which have left.)
  double asum = 0.0;
  for (int i = l; i < asq_n; i += 64) asum += asq[(long long)b * asq_n + i];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) asum += __shfl_xor(asum, o);
  double w2 = asum;
  if (fired) {
    const double lam_l = (l < r) ? H[order[l] * JP + order[l]] : 0.0;   // lambda of rank l
    __builtin_amdgcn_wave_barrier();
    // Q^T Q into the free buffer
    double* G = Hs[cur ^ 1];
    const double* qb = qpart + (long long)b * GRAM_CHUNKS * RP * RP;
    for (int e = l; e < RP * RP; e += 64) {
      const int i = e / RP, j = e % RP;
      double acc = 0.0;
#pragma unroll
      for (int c = 0; c < GRAM_CHUNKS; ++c) acc += qb[(long long)c * RP * RP + e];
      G[i * JP + j] = (i < r && j < r) ? acc : 0.0;
    }
    __builtin_amdgcn_wave_barrier();
    double head = 0.0;
    for (int t = 0; t < kk; ++t) {
      const int ct = pm[order[t]];   // column of V (original index) of rank t
      double y = 0.0;                       // (Q^T Q Ub_t)_l
      if (l < r)
        for (int c = 0; c < r; ++c) y = fma(G[l * JP + c], (double)Vf[c * (RP + 1) + ct], y);
      double gt = (l < r) ? (double)Vf[l * (RP + 1) + ct] * y : 0.0;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) gt += __shfl_xor(gt, o);
      const double lam = __shfl(lam_l, t);
      head += lam * (2.0 - gt);
    }
    w2 = asum - head;
  }
  if (l == 0) d_out[b] = (float)sqrt(w2 > 0.0 ? w2 : 0.0) + 1e-7f;
  // When the removed head holds nearly all of A's energy the difference above loses
  // its digits (its error grows as ||A||^2 / ||W||^2, while an explicit ||W||_F's
  // grows as ||A|| / ||W||): below 1% of ||A||^2 the matrix is flagged and d is
  // recomputed from W itself (w_norm_partials, then deflate_restore).
  if (l == 0 && wflag) wflag[b] = fired && w2 < 1e-2 * asum ? 1 : 0;
}

// ---------------------------------------------------------------------------
// Gate eigen-decomposition for the clip and fused paths, where only the head
// eigenpairs (the deflated directions) and the eigenvalues the gate compares are
// needed; one 512-thread workgroup per matrix.
//  1. Householder reduction of H = Bp Bp^T (r x r, fp64) to tridiagonal form
//     T = Q^T H Q (LAPACK's convention: reflector k = I - tau_k v_k v_k^T acts on
//     rows k+1.., v_k[k+1] = 1, T[k+1][k] = ||H[k+1:, k]||), by one wave: lane l owns
//     column l of the trailing block, kept whole (both triangles) in LDS, so every
//     access is a row read or write across the lanes.
//  2. Every eigenvalue of T by multisection: lane j of each of the 8 waves evaluates
//     the Sturm count (the number of eigenvalues below x, from the pivots of
//     T - x I) at one of 8 interior points of the j-th smallest eigenvalue's bracket,
//     so each pass shrinks every bracket 9x (EH_PASSES passes from the Gershgorin
//     interval).
//  3. The top nv = min(kw, r) eigenpairs -- every value the gate compares at the
//     default thresholds -- by inverse iteration on T (partial-pivoting elimination of
//     T - sigma I, one lane per eigenpair, start vectors fixed per index, Rayleigh-
//     quotient shifts), vectors whose eigenvalues lie within 1e-3 ||T|| of the previous
//     one re-orthogonalised in order after every step; further deflated directions
//     the gate asks for (thresholds set apart) the same way afterwards.  Then each
//     vector is back-transformed, Q y.
//  4. The gate, the deflate / restore weights and d exactly as eig_gate computes them.
// Degenerate matrices (flagged by the Cholesky) skip 1-3 and come out declined, as
// in eig_gate.
// ---------------------------------------------------------------------------
constexpr int EH_THREADS = 512;
constexpr int EH_WAVES = EH_THREADS / 64;
constexpr int EH_ITERS = 3;     // inverse-iteration steps per eigenpair, at most
constexpr int EH_VL = 32;       // eigenpairs per inverse-iteration batch (lanes)
constexpr int ZP = RP + 2;      // row pitch (doubles) of the eigenvector rows

union EhScratch {
  struct {
    double H[RP * JP];                                 // H, reduced in place
    double pw[EH_WAVES][RP];                           // the waves' partial products
  } red;                                               // (step 1)
  struct {
    double u0[RP][EH_VL], u1[RP][EH_VL], u2[RP][EH_VL];   // band U of T - sigma I, per lane
    double y[RP][EH_VL];                                  // the lane's vector
  } lu;                                                // (step 4)
  double G[RP * JP];                                   // Q^T Q (step 5)
};

// Wave-wide reductions of a double: within each row of 16 lanes by DPP moves (lanes
// l ^ 1, l ^ 2, then the mirrored half-row and row), then the four row results read
// from lanes 0, 16, 32, 48 -- every lane gets the same value.  All 64 lanes active.
__device__ __forceinline__ double dpp_d(double v, int ctrl_sel) {
  const long long bits = __double_as_longlong(v);
  int lo = (int)(bits & 0xffffffffLL), hi = (int)(bits >> 32);
  switch (ctrl_sel) {
    case 0: lo = __builtin_amdgcn_mov_dpp(lo, 0xB1, 0xF, 0xF, false);
            hi = __builtin_amdgcn_mov_dpp(hi, 0xB1, 0xF, 0xF, false); break;   // quad [1,0,3,2]
    case 1: lo = __builtin_amdgcn_mov_dpp(lo, 0x4E, 0xF, 0xF, false);
            hi = __builtin_amdgcn_mov_dpp(hi, 0x4E, 0xF, 0xF, false); break;   // quad [2,3,0,1]
    case 2: lo = __builtin_amdgcn_mov_dpp(lo, 0x141, 0xF, 0xF, false);
            hi = __builtin_amdgcn_mov_dpp(hi, 0x141, 0xF, 0xF, false); break;  // row_half_mirror
    default: lo = __builtin_amdgcn_mov_dpp(lo, 0x140, 0xF, 0xF, false);
             hi = __builtin_amdgcn_mov_dpp(hi, 0x140, 0xF, 0xF, false); break; // row_mirror
  }
  return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}
__device__ __forceinline__ double wave_sum_d(double v) {
  v += dpp_d(v, 0);
  v += dpp_d(v, 1);
  v += dpp_d(v, 2);
  v += dpp_d(v, 3);
  return (lane_val(v, 0) + lane_val(v, 16)) + (lane_val(v, 32) + lane_val(v, 48));
}
__device__ __forceinline__ double wave_min_d(double v) {
  v = fmin(v, dpp_d(v, 0));
  v = fmin(v, dpp_d(v, 1));
  v = fmin(v, dpp_d(v, 2));
  v = fmin(v, dpp_d(v, 3));
  return fmin(fmin(lane_val(v, 0), lane_val(v, 16)), fmin(lane_val(v, 32), lane_val(v, 48)));
}
__device__ __forceinline__ double wave_max_d(double v) {
  v = fmax(v, dpp_d(v, 0));
  v = fmax(v, dpp_d(v, 1));
  v = fmax(v, dpp_d(v, 2));
  v = fmax(v, dpp_d(v, 3));
  return fmax(fmax(lane_val(v, 0), lane_val(v, 16)), fmax(lane_val(v, 32), lane_val(v, 48)));
}
// 1/x from the hardware estimate and one Newton step
__device__ __forceinline__ double rcp_nr1(double x) {
  double y = __builtin_amdgcn_rcp(x);
  return fma(y, fma(-x, y, 1.0), y);
}
// the compiler keeps LDS accesses on either side in order; a wave's LDS accesses
// complete in order, so reads after it see every lane's earlier writes
__device__ __forceinline__ void wave_lds_order() {
  __builtin_amdgcn_wave_barrier();
  asm volatile("" ::: "memory");
}

// Start vector of inverse iteration for eigenpair t: fixed pseudo-random entries in
// (-1, 1) (a hash of (t, i)), zero past r.
__device__ __forceinline__ double eh_start(int t, int i, int r) {
  if (i >= r) return 0.0;
  unsigned h = (unsigned)(t * RP + i) * 2654435761u;
  h ^= h >> 15; h *= 2246822519u; h ^= h >> 13;
  return ((double)(h >> 8) + 0.5) * (2.0 / 16777216.0) - 1.0;
}

// Inverse iteration for eigenpairs t0 .. t1-1 (t1 - t0 <= EH_VL) on wave 0: lane
// t - t0 refines lamd[t] (a bracket midpoint on entry, the Rayleigh quotient on exit)
// and leaves the eigenvector y_t of T in row t of Z (eh_back_transform makes it
// Q y_t).  Each lane's vector and band factors live in LDS columns (sc.lu.y[i][lane],
// ...), walked by plain loops.
__device__ __forceinline__ void eh_inverse_iteration(int t0, int t1, int r, double tn,
                                                     const double* dd, const double* ee,
                                                     const double* taus, const double* Vr,
                                                     double* lamd, double* Z, EhScratch& sc,
                                                     int l) {
  const int t = t0 + l;
  const bool lane = l < EH_VL;            // lanes that own a column of the scratch
  const bool act = lane && t < t1;
  const int cl = lane ? l : 0;
  const double eps_tn = 2.220446049250313e-16 * (tn > 0.0 ? tn : 1.0);
  double sigma = act ? lamd[t] : 0.0;
  if (lane) {
    double n0 = 0.0;
    for (int i = 0; i < RP; ++i) {
      const double v = act ? eh_start(t, i, r) : 0.0;
      n0 = fma(v, v, n0);
      sc.lu.y[i][cl] = v;
    }
    const double s0n = n0 > 0.0 ? rsqrt_nr(n0) : 0.0;
    for (int i = 0; i < RP; ++i) sc.lu.y[i][cl] *= s0n;
  }
  // a step has converged when the solve amplified the unit start vector by 1e8 / ||T||
  // (the shift then lies within ~1e-8 ||T|| |c| of the eigenvalue, c the start vector's
  // component along it); at most EH_ITERS steps
  bool conv = !act;
  for (int it = 0; it < EH_ITERS; ++it) {
    if (lane && !conv) {
      // (T - sigma I) x = y: forward elimination with row interchanges
      double cur0 = dd[0] - sigma, cur1 = ee[0];
      double yc = sc.lu.y[0][cl];
#pragma unroll 4
      for (int i = 0; i + 1 < RP; ++i) {
        const double sub = ee[i], nd = dd[i + 1] - sigma, ns = (i + 2 < RP) ? ee[i + 1] : 0.0;
        const double yn = sc.lu.y[i + 1][cl];
        const bool sw = fabs(cur0) < fabs(sub);
        const double piv = sw ? sub : (cur0 != 0.0 ? cur0 : eps_tn);
        const double mlt = (sw ? cur0 : sub) * rcp_nr(piv);
        sc.lu.u0[i][cl] = piv;
        sc.lu.u1[i][cl] = sw ? nd : cur1;
        sc.lu.u2[i][cl] = sw ? ns : 0.0;
        sc.lu.y[i][cl] = sw ? yn : yc;
        yc = sw ? fma(-mlt, yn, yc) : fma(-mlt, yc, yn);
        const double c0 = sw ? fma(-mlt, nd, cur1) : fma(-mlt, cur1, nd);
        cur1 = sw ? -mlt * ns : ns;
        cur0 = c0;
      }
      sc.lu.u0[RP - 1][cl] = cur0 != 0.0 ? cur0 : eps_tn;
      // back substitution, then |x| and the Rayleigh quotient
      double x1 = 0.0, x2 = 0.0, nrm = 0.0;
#pragma unroll 4
      for (int i = RP - 1; i >= 0; --i) {
        const double yi = i == RP - 1 ? yc : sc.lu.y[i][cl];
        double s = fma(-sc.lu.u1[i][cl], x1, yi);
        s = fma(-sc.lu.u2[i][cl], x2, s);
        const double x = s * rcp_nr(sc.lu.u0[i][cl]);
        sc.lu.y[i][cl] = x;
        nrm = fma(x, x, nrm);
        x2 = x1;
        x1 = x;
      }
      const double inv = act && nrm > 0.0 ? rsqrt_nr(nrm) : 0.0;
      conv = nrm * tn * tn >= 1e16;
      double rq = 0.0, rq2 = 0.0, yp = 0.0;
#pragma unroll 8
      for (int i = 0; i < RP; ++i) {
        const double yi = sc.lu.y[i][cl] * inv;
        sc.lu.y[i][cl] = yi;
        rq = fma(dd[i] * yi, yi, rq);
        if (i > 0) rq2 = fma(ee[i - 1] * yp, yi, rq2);
        yp = yi;
      }
      if (act) sigma = fma(2.0, rq2, rq);
    }
    const bool done = __all(conv);
    // eigenvalues within 1e-3 ||T|| of their predecessor: Gram-Schmidt in order
    const double sprev = __shfl_up(sigma, 1);
    const bool clus = act && t > t0 && fabs(sigma - sprev) <= 1e-3 * tn;
    if (__any(clus)) {
      wave_lds_order();
      const unsigned long long cmask = __ballot(clus);
      for (int u = t0 + 1; u < t1; ++u) {
        if (!((cmask >> (u - t0)) & 1ull)) continue;
        int s0 = u - 1;
        while (s0 > t0 && ((cmask >> (s0 - t0)) & 1ull)) --s0;   // first member of u's cluster
        // lane l: entry l of the vectors (columns u - t0 and q - t0 of the scratch)
        double zu = sc.lu.y[l][u - t0];
        for (int q = s0; q < u; ++q) {
          const double zq = sc.lu.y[l][q - t0];
          const double dot = wave_sum_d(zq * zu);
          zu = fma(-dot, zq, zu);
        }
        const double nn = wave_sum_d(zu * zu);
        zu *= nn > 0.0 ? rsqrt_nr(nn) : 0.0;
        sc.lu.y[l][u - t0] = zu;
        wave_lds_order();
      }
    }
    wave_lds_order();
    if (done) break;
  }
  // the eigenvalue of the final vector (a cluster's Gram-Schmidt may have moved it)
  if (act) {
    double rq = 0.0, rq2 = 0.0, yp = 0.0;
#pragma unroll 8
    for (int i = 0; i < RP; ++i) {
      const double yi = sc.lu.y[i][cl];
      rq = fma(dd[i] * yi, yi, rq);
      if (i > 0) rq2 = fma(ee[i - 1] * yp, yi, rq2);
      yp = yi;
    }
    sigma = fma(2.0, rq2, rq);
  }
  if (act) {
    lamd[t] = sigma;
    for (int i = 0; i < RP; ++i) Z[t * ZP + i] = sc.lu.y[i][cl];   // before the back-transform
  }
  wave_lds_order();
}

// Z[t] <- Q Z[t] = H_0 H_1 ... H_{r-3} Z[t] for t < nvec, the last reflector first.
// Eight lanes per vector, eight entries each (lane l: vector 8 wave + l / 8, entries
// 8 (l % 8) .. +7), so a wave carries 8 vectors and each reflector's dot product is 8
// fmas and a reduction over 8 lanes in 3 DPP steps.  (One vector per wave, one entry
// per lane and a 64-lane reduction per reflector took ~30 us for 8 vectors.)
__device__ __forceinline__ void eh_back_transform(int nvec, int r, const double* taus,
                                                  const double* Vr, double* Z, int wave, int l) {
  if (8 * wave >= nvec) return;   // uniform over the wave
  const int t = 8 * wave + (l >> 3), e0 = 8 * (l & 7);
  const bool live = t < nvec;
  double z[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) z[c] = live ? Z[t * ZP + e0 + c] : 0.0;
  for (int k = r - 3; k >= 0; --k) {
    const double tk = taus[k];
    if (tk == 0.0) continue;
    double v[8];   // reflector k: zero for entries <= k and past r
#pragma unroll
    for (int c = 0; c < 8; ++c) v[c] = Vr[k * RP + e0 + c];
    double s0 = v[0] * z[0], s1 = v[1] * z[1];
#pragma unroll
    for (int c = 2; c < 8; c += 2) {
      s0 = fma(v[c], z[c], s0);
      s1 = fma(v[c + 1], z[c + 1], s1);
    }
    double sq = s0 + s1;
    sq += dpp_d(sq, 0);   // pairs
    sq += dpp_d(sq, 1);   // quads
    sq += dpp_d(sq, 2);   // the 8 lanes of the vector (half-row mirror)
    sq *= tk;
#pragma unroll
    for (int c = 0; c < 8; ++c) z[c] = fma(-sq, v[c], z[c]);
  }
  if (live) {
#pragma unroll
    for (int c = 0; c < 8; ++c) Z[t * ZP + e0 + c] = z[c];
  }
}

__global__ __launch_bounds__(EH_THREADS) void eig_head_gate(
    const double* __restrict__ part, GateParams gp, const int* __restrict__ degen,
    float* __restrict__ s_out, int s_ld, float* __restrict__ Ub, float* __restrict__ UbS,
    long long* __restrict__ k_out, int* __restrict__ k_int, float* __restrict__ cw,
    float* __restrict__ cr, const double* __restrict__ qpart, const double* __restrict__ asq,
    int asq_n, float* __restrict__ d_out, int* __restrict__ wflag) {
  __shared__ __attribute__((aligned(16))) EhScratch sc;
  __shared__ __attribute__((aligned(16))) double Vr[RP * RP];   // reflector k in row k
  __shared__ __attribute__((aligned(16))) double Z[RP * ZP];    // eigenvector t in row t
  __shared__ double dd[RP], ee[RP], e2s[RP], taus[RP], lamd[RP];
  __shared__ int cnt[2][EH_THREADS];
  __shared__ float sv[RP];
  __shared__ double s_lo, s_hi, s_tn;
  const int b = blockIdx.x, tid = threadIdx.x, l = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = gp.r;
  const bool bad = degen && degen[b];
  {
    const double* pb = part + (long long)b * GRAM_CHUNKS * RP * RP;
    for (int e = tid; e < RP * RP; e += EH_THREADS) {
      const int i = e / RP, j = e % RP;
      double acc = 0.0;
#pragma unroll
      for (int c = 0; c < GRAM_CHUNKS; ++c) acc += pb[(long long)c * RP * RP + e];
      sc.red.H[i * JP + j] = (i < r && j < r) ? acc : 0.0;
    }
  }
  __syncthreads();
  // ---- 1. tridiagonal reduction: every wave forms each reflector itself (the same
  // values: same inputs, same order), so that only the matrix-vector product and the
  // rank-2 update, whose rows (every 8th) the waves share, need workgroup barriers
  if (!bad) {
    double* H = sc.red.H;
    for (int k = 0; k + 2 < r; ++k) {
      const double xi = (l > k && l < r) ? H[k * JP + l] : 0.0;   // H[l][k] = H[k][l]
      const double x0 = lane_val(xi, k + 1);
      const double sg = wave_sum_d(l > k + 1 ? xi * xi : 0.0);
      double vl = 0.0, tk = 0.0, ek = x0;   // sg == 0: already reduced, no reflection
      if (sg != 0.0) {
        const double mu = sqrt(x0 * x0 + sg);
        const double v0 = x0 <= 0.0 ? x0 - mu : -sg / (x0 + mu);
        const double v02 = v0 * v0;
        tk = 2.0 * v02 / (sg + v02);
        const double iv0 = 1.0 / v0;
        vl = l == k + 1 ? 1.0 : ((l > k + 1 && l < r) ? xi * iv0 : 0.0);
        ek = mu;
      }
      if (wave == 0) {
        Vr[k * RP + l] = vl;
        if (l == 0) { dd[k] = H[k * JP + k]; ee[k] = ek; taus[k] = tk; }
      }
      if (tk != 0.0) {   // uniform over the workgroup
        // p = tau H22 v: wave w sums rows k+1+w, k+1+w+8, ... (lane l: column l)
        double a0 = 0.0, a1 = 0.0;
        int j = k + 1 + wave;
        for (; j + EH_WAVES < r; j += 2 * EH_WAVES) {
          a0 = fma(H[j * JP + l], lane_val(vl, j), a0);
          a1 = fma(H[(j + EH_WAVES) * JP + l], lane_val(vl, j + EH_WAVES), a1);
        }
        if (j < r) a0 = fma(H[j * JP + l], lane_val(vl, j), a0);
        sc.red.pw[wave][l] = a0 + a1;
        __syncthreads();
        double pl = 0.0;
#pragma unroll
        for (int w = 0; w < EH_WAVES; ++w) pl += sc.red.pw[w][l];   // same order in every wave
        pl = (l > k && l < r) ? tk * pl : 0.0;
        const double K = wave_sum_d(pl * vl);
        const double wl = pl - (0.5 * tk * K) * vl;
        // H22 -= v w^T + w v^T, rows k+1+w, k+1+w+8, ... by wave w
        for (int jj = k + 1 + wave; jj < r; jj += EH_WAVES) {
          const double vj = lane_val(vl, jj), wj = lane_val(wl, jj);
          if (l > k && l < r) {
            double h = H[jj * JP + l];
            h = fma(-vj, wl, h);
            h = fma(-wj, vl, h);
            H[jj * JP + l] = h;
          }
        }
      }
      __syncthreads();
    }
    if (wave == 0) {
      // the trailing 2 x 2 (or 1 x 1) block; padding past r: a diagonal far above the
      // spectrum, decoupled (zero off-diagonal), so it never counts and never mixes in
      if (l == 0) {
        if (r >= 2) {
          dd[r - 2] = H[(r - 2) * JP + r - 2];
          dd[r - 1] = H[(r - 1) * JP + r - 1];
          ee[r - 2] = H[(r - 1) * JP + r - 2];
          taus[r - 2] = 0.0;
        } else {
          dd[0] = H[0];
        }
      }
      wave_lds_order();
      double gl = INFINITY, gh = -INFINITY;
      if (l < r) {
        const double em = l > 0 ? fabs(ee[l - 1]) : 0.0, ep = l + 1 < r ? fabs(ee[l]) : 0.0;
        gl = dd[l] - em - ep;
        gh = dd[l] + em + ep;
      }
      const double lo = wave_min_d(gl), hi = wave_max_d(gh);
      const double tn = fmax(fabs(lo), fabs(hi));
      if (l >= r) dd[l] = 2.0 * tn + 1.0;
      if (l + 1 >= r) ee[l] = 0.0;
      if (l + 2 >= r && l < r) taus[l] = 0.0;
      wave_lds_order();
      e2s[l] = ee[l] * ee[l];
      if (l == 0) {   // brackets widened by rounding-level margins
        const double mg = 4.0 * 2.220446049250313e-16 * (tn * RP) + 1e-300;
        s_lo = lo - mg;
        s_hi = hi + mg;
        s_tn = tn;
      }
    }
  }
  __syncthreads();
  // ---- 2. the top nE = min(kw, r) eigenvalues (every value the gate compares) by
  // multisection: nE <= 32: 16 threads per eigenvalue, each evaluating the Sturm count
  // at one of 16 interior points of its bracket (17 sub-intervals per pass); nE > 32:
  // 8 threads (9 sub-intervals)
  const int nE = min(gp.kw, r);
  const int npt = nE <= 32 ? 16 : 8;           // points per bracket
  const int slot = tid / npt, pt = tid % npt;  // eigenvalue slot (descending), point
  if (!bad) {
    double e2max = 0.0;
    for (int i = 0; i + 1 < r; ++i) e2max = fmax(e2max, e2s[i]);
    const double pivmin = 2.2250738585072014e-308 * fmax(1.0, e2max);
    const int npass = npt == 16 ? 9 : 12;      // brackets ~2 ||T|| / 17^9 or / 9^12
    const double inv_sect = 1.0 / (double)(npt + 1);
    double L = s_lo, U = s_hi;
    const int j = r - 1 - slot;                // ascending index of the eigenvalue
    const bool live = slot < nE;
    for (int p = 0; p < npass; ++p) {
      // (the same expression as the readers' below, so all threads agree on the points)
      const double x = fma(U - L, (double)(pt + 1) * inv_sect, L);
      int c = 0;
      if (live) {
        asm volatile("" ::: "memory");   // T's rows are read in batches, not all up front
        double q = dd[0] - x;
        if (fabs(q) < pivmin) q = -pivmin;
        c = q < 0.0;
#pragma unroll
        for (int i = 1; i < RP; ++i) {
          if ((i & 7) == 0) asm volatile("" ::: "memory");
          q = (dd[i] - x) - e2s[i - 1] * rcp_nr1(q);
          if (fabs(q) < pivmin) q = -pivmin;
          c += q < 0.0;
        }
      }
      cnt[p & 1][tid] = c;
      __syncthreads();
      double nL = L, nU = U;
      bool found = false;
      for (int w = 0; w < npt; ++w) {
        const double xw = fma(U - L, (double)(w + 1) * inv_sect, L);
        if (!found) {
          if (cnt[p & 1][slot * npt + w] > j) { nU = xw; found = true; }
          else nL = xw;
        }
      }
      L = nL;
      U = nU;
    }
    if (pt == 0 && live) lamd[slot] = 0.5 * (L + U);   // descending
  }
  __syncthreads();
  // ---- 3. gate, fp32 comparisons as torch does them (deflation_batched.py:177-180),
  // on the bracket midpoints (brackets ~1e-11 ||T||: every comparison is decided unless
  // a value lies within ~1e-8 relative of its threshold)
  if (tid < RP) {
    float sval = 0.f;
    if (tid < nE && !bad) {
      const double ev = lamd[tid];
      sval = (float)sqrt(ev > 0.0 ? ev : 0.0);
    }
    sv[tid] = sval;
  }
  __syncthreads();
  const float s0 = sv[0];
  const float thr = gp.thresh * s0;
  int kr = 0;
  for (int j = 0; j < nE; ++j) kr += sv[j] > thr;
  // (thresh >= ratio: whenever the gate fires, every value past the top nE lies below
  // sv[kw-1] < ratio s0 <= thr, so the top nE hold the whole count)
  const bool could_fire = (sv[gp.kw - 1] < gp.ratio * s0) && kr >= 1;
  const bool fired = could_fire && kr < r;
  const int kk = kr < 1 ? 1 : (kr > r - 1 ? r - 1 : kr);
  // ---- 4. the deflated eigenpairs (wave 0): inverse iteration, Rayleigh-quotient
  // eigenvalues, back-transform; their singular values replace the bracket values
  if (fired) {
    if (!bad && wave == 0)
      for (int t0 = 0; t0 < kk; t0 += EH_VL)
        eh_inverse_iteration(t0, min(t0 + EH_VL, kk), r, s_tn, dd, ee, taus, Vr, lamd, Z, sc, l);
    __syncthreads();
    if (!bad) eh_back_transform(kk, r, taus, Vr, Z, wave, l);
    __syncthreads();
    if (tid < kk) {
      const double ev = lamd[tid];
      sv[tid] = (float)sqrt(ev > 0.0 ? ev : 0.0);
    }
    __syncthreads();
  }
  if (tid == 0) {
    k_out[b] = fired ? (long long)kk : 0LL;
    k_int[b] = fired ? kk : 0;
  }
  const int nh = fired ? kk : 0;   // columns of Ub filled
  if (tid < RP) {
    if (tid < r) s_out[(long long)b * s_ld + tid] = sv[tid];
    const float h = (fired && tid < kk) ? 1.f : 0.f;
    cw[(long long)b * RP + tid] = sv[tid] * h;
    cr[(long long)b * RP + tid] = h * (1.0f / gp.pad);
  }
  float* Ubb = Ub + (long long)b * RP * RP;
  float* UbSb = UbS + (long long)b * RP * RP;
  for (int e = tid; e < RP * RP; e += EH_THREADS) {
    const int a = e / RP, t = e % RP;   // row a of Ub, column t
    float u = 0.f;
    if (a < r && t < nh && !bad) u = (float)Z[t * ZP + a];
    Ubb[e] = u;
    UbSb[e] = sv[t] > 0.f ? u / sv[t] : 0.f;
  }
  if (d_out && fired) {   // Q^T Q, summed by every thread
    const double* qb = qpart + (long long)b * GRAM_CHUNKS * RP * RP;
    for (int e = tid; e < RP * RP; e += EH_THREADS) {
      const int i = e / RP, j = e % RP;
      double acc = 0.0;
#pragma unroll
      for (int c = 0; c < GRAM_CHUNKS; ++c) acc += qb[(long long)c * RP * RP + e];
      sc.G[i * JP + j] = (i < r && j < r) ? acc : 0.0;
    }
    __syncthreads();
  }
  if (!d_out || wave != 0) return;
  // ||W||_F^2 = ||A||^2 - sum_{t<k} lambda_t (2 - G_t), G_t = Ub_t^T (Q^T Q) Ub_t (see
  // eig_gate)
  double asum = 0.0;
  for (int i = l; i < asq_n; i += 64) asum += asq[(long long)b * asq_n + i];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) asum += __shfl_xor(asum, o);
  double w2 = asum;
  if (fired) {
    const double* G = sc.G;
    double head = 0.0;
    for (int t = 0; t < kk; ++t) {
      double y = 0.0;   // (Q^T Q Ub_t)_l, with Ub_t rounded to fp32 as stored
      if (l < r)
        for (int c = 0; c < r; ++c) y = fma(G[l * JP + c], (double)(float)Z[t * ZP + c], y);
      double gt = (l < r) ? (double)(float)Z[t * ZP + l] * y : 0.0;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) gt += __shfl_xor(gt, o);
      head += lamd[t] * (2.0 - gt);
    }
    w2 = asum - head;
  }
  if (l == 0) d_out[b] = (float)sqrt(w2 > 0.0 ? w2 : 0.0) + 1e-7f;
  if (l == 0 && wflag) wflag[b] = fired && w2 < 1e-2 * asum ? 1 : 0;
}

// ---------------------------------------------------------------------------
// Restore pass (deflation_batched.py:184-188):
//   X0 = (A - U diag(s h) V^T) / d + U diag(h / pad) V^T
//      = A / d - sum_{t<k} U[i][t] (cw_t / d - cr_t) V[j][t]
// per 64 x 64 tile, rank-k update on VALU (k <= 63), fp32.  Outputs, any subset:
//   X0   (B, n, m) bf16 or fp32, the API tensor
//   T, W the NS chain's packed bf16 operands (T: np x mp in the chain's 64 x 64
//        block layout, W: its transpose, row-major; zero outside n x m), so the
//        chain can start without its entry pass
// ---------------------------------------------------------------------------
constexpr int DR_ROWS = 64, DR_COLS = 128;
constexpr int DR_KC = 16;   // head columns staged per chunk

// restore tiles per matrix
__host__ __device__ inline int wn_tiles(int n, int m) {
  return ((m + DR_COLS - 1) / DR_COLS) * ((n + DR_ROWS - 1) / DR_ROWS);
}

// w_norm_partials' workgroups (and partial sums) per matrix
constexpr int WN_PARTS = 32;
__host__ __device__ inline int wn_parts(int n, int m) {
  const int t = wn_tiles(n, m);
  return t < WN_PARTS ? t : WN_PARTS;
}

// LDS of one restore tile: the head chunk (U rows of the tile, V rows of the tile
// transposed) while the rank-k update runs, then the bf16 tile of W = T^T.
union RestoreLds {
  struct {
    float Us[DR_ROWS][DR_KC + 1];        // U[i][t0 + t]
    float Vt[DR_KC][DR_COLS + 4];        // V[j][t0 + t] as Vt[t][j]
  } head;
  bf16 tw[DR_COLS][DR_ROWS + 8];         // tile of W = T^T
};

// Pieces shared by the restore pass and the explicit ||W||_F pass.  Thread tid
// holds rows rw + 8 a (a = 0..7, rw = tid / 32) and columns c4 .. c4 + 3 (c4 =
// 4 (tid % 32)) of a 64 x 128 tile; zeros outside n x m.
__device__ __forceinline__ void dr_load_tile(const float* __restrict__ Ab, int n, int m, int i0,
                                             int j0, int rw, int c4, bool vec,
                                             float (&x)[8][4]) {
#pragma unroll
  for (int a = 0; a < 8; ++a) {
    const int gi = i0 + rw + 8 * a, gj = j0 + c4;
    if (gi < n && vec && gj + 3 < m) {
      const float4 v = *(const float4*)&Ab[(long long)gi * m + gj];
      x[a][0] = v.x; x[a][1] = v.y; x[a][2] = v.z; x[a][3] = v.w;
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c)
        x[a][c] = (gi < n && gj + c < m) ? Ab[(long long)gi * m + gj + c] : 0.f;
    }
  }
}

// Head columns t0 .. t0 + kc - 1 of the tile's U rows (64) and V rows (128), zero
// past kc or the matrix: thread tid loads U[i0 + tid/16 + 16 q][t0 + tid%16], q < 4,
// and V[j0 + tid/16 + 16 q][t0 + tid%16], q < 8, so each row's 16 floats are one
// 64-byte piece.
static_assert(DR_ROWS * DR_KC == 4 * 256 && DR_COLS * DR_KC == 8 * 256, "head chunk per thread");
__device__ __forceinline__ void dr_load_head(const float* __restrict__ Ub,
                                             const float* __restrict__ Vb, int n, int m, int i0,
                                             int j0, int t0, int kc, int tid, float (&ur)[4],
                                             float (&vr)[8]) {
  const int t = tid % DR_KC, r0 = tid / DR_KC;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int gi = i0 + r0 + 16 * q;
    ur[q] = (t < kc && gi < n) ? Ub[(long long)gi * RP + t0 + t] : 0.f;
  }
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int gj = j0 + r0 + 16 * q;
    vr[q] = (t < kc && gj < m) ? Vb[(long long)gj * RP + t0 + t] : 0.f;
  }
}

__device__ __forceinline__ void dr_stage_head(RestoreLds& sm, const float (&ur)[4],
                                              const float (&vr)[8], int tid) {
  const int t = tid % DR_KC, r0 = tid / DR_KC;
#pragma unroll
  for (int q = 0; q < 4; ++q) sm.head.Us[r0 + 16 * q][t] = ur[q];
#pragma unroll
  for (int q = 0; q < 8; ++q) sm.head.Vt[t][r0 + 16 * q] = vr[q];
}

// x -= sum_{t < kc} U[i][t0 + t] coef[t0 + t] V[j][t0 + t], t in order
__device__ __forceinline__ void dr_apply_head(const RestoreLds& sm, const float* coef, int t0,
                                              int kc, int rw, int c4, float (&x)[8][4]) {
  for (int t = 0; t < kc; ++t) {
    const float4 v = *(const float4*)&sm.head.Vt[t][c4];
    const float ct = coef[t0 + t];
#pragma unroll
    for (int a = 0; a < 8; ++a) {
      const float u = sm.head.Us[rw + 8 * a][t] * ct;
      x[a][0] = fmaf(-u, v.x, x[a][0]);
      x[a][1] = fmaf(-u, v.y, x[a][1]);
      x[a][2] = fmaf(-u, v.z, x[a][2]);
      x[a][3] = fmaf(-u, v.w, x[a][3]);
    }
  }
}

__global__ __launch_bounds__(256) void deflate_restore(
    const float* __restrict__ A, int n, int m, const float* __restrict__ U,
    const float* __restrict__ V, const int* __restrict__ kvec, const float* __restrict__ cw,
    const float* __restrict__ cr, float* __restrict__ dvec, const int* __restrict__ wflag,
    const double* __restrict__ wpart, void* __restrict__ X0,
    int x0_mode /*0 none, 1 bf16, 2 fp32*/, bf16* __restrict__ T, bf16* __restrict__ W, int np,
    int mp) {
  __shared__ __attribute__((aligned(16))) RestoreLds sm;
  __shared__ float coef[RP];
  const int b = blockIdx.z;
  const int i0 = blockIdx.y * DR_ROWS, j0 = blockIdx.x * DR_COLS;
  const int tid = threadIdx.x;
  const int k = kvec[b];
  const int c4 = (tid & 31) * 4;      // 4 consecutive columns of the tile
  const int rw = tid >> 5;            // rows rw + 8a, a = 0..7
  const bool vec = (m & 3) == 0;
  // Every global read of the tile goes out before the first wait: A (the bulk of the
  // traffic), the first head chunk, and the norm partials of a flagged matrix
  float x[8][4], ur[4], vr[8];
  dr_load_tile(A + (long long)b * n * m, n, m, i0, j0, rw, c4, vec, x);
  const float* Ub = U + (long long)b * n * RP;
  const float* Vb = V + (long long)b * m * RP;
  if (k > 0) dr_load_head(Ub, Vb, n, m, i0, j0, 0, min(DR_KC, k), tid, ur, vr);
  float d = dvec[b];
  if (wflag && wflag[b]) {
    // d from W itself: every workgroup sums the same partials in the same order
    // (so all agree on d bit for bit); the first stores it as the API's d
    const int nt = wn_parts(n, m);
    __shared__ double wsum[256];
    double acc = 0.0;
    for (int t = tid; t < nt; t += 256) acc += wpart[(long long)b * nt + t];
    wsum[tid] = acc;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
      if (tid < w) wsum[tid] += wsum[tid + w];
      __syncthreads();
    }
    d = (float)sqrt(wsum[0]) + 1e-7f;
    if (blockIdx.x == 0 && blockIdx.y == 0 && tid == 0) dvec[b] = d;
  }
  if (tid < RP) coef[tid] = cw[b * RP + tid] / d - cr[b * RP + tid];
#pragma unroll
  for (int a = 0; a < 8; ++a)
#pragma unroll
    for (int c = 0; c < 4; ++c) x[a][c] = x[a][c] / d;
  for (int t0 = 0; t0 < k; t0 += DR_KC) {
    const int kc = min(DR_KC, k - t0);
    if (t0 > 0) dr_load_head(Ub, Vb, n, m, i0, j0, t0, kc, tid, ur, vr);
    __syncthreads();   // coef visible; the previous chunk consumed
    dr_stage_head(sm, ur, vr, tid);
    __syncthreads();
    dr_apply_head(sm, coef, t0, kc, rw, c4, x);
  }
  if (W) __syncthreads();   // the head chunk is consumed before tw overwrites it
#pragma unroll
  for (int a = 0; a < 8; ++a) {
    const int il = rw + 8 * a;
    const int gi = i0 + il, gj = j0 + c4;
    bf16x4 o;
#pragma unroll
    for (int c = 0; c < 4; ++c) o[c] = f2bf((gi < n && gj + c < m) ? x[a][c] : 0.f);
    if (x0_mode && gi < n) {
      const long long off = (long long)b * n * m + (long long)gi * m + gj;
      if (x0_mode == 1 && vec && gj + 3 < m) {
        *(bf16x4*)((bf16*)X0 + off) = o;
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          if (gj + c >= m) continue;
          if (x0_mode == 1) ((bf16*)X0)[off + c] = o[c];
          else ((float*)X0)[off + c] = x[a][c];
        }
      }
    }
    if (T && gi < np && gj < mp)   // the chain's block layout (blk_off)
      *(bf16x4*)(T + (long long)b * np * mp + blk_off(gi, gj, np)) = o;
    if (W) {
#pragma unroll
      for (int c = 0; c < 4; ++c) sm.tw[c4 + c][il] = o[c];
    }
  }
  if (W) {
    __syncthreads();
    // row jj of W's tile: DR_ROWS bf16 = 8 chunks of 16 bytes
    for (int e = tid; e < DR_COLS * 8; e += 256) {
      const int jj = e >> 3, ch = (e & 7) * 8;
      const int gj = j0 + jj, gi = i0 + ch;
      if (gj < mp && gi < np)
        *(uint4*)(W + (long long)b * mp * np + (long long)gj * np + gi) = *(const uint4*)&sm.tw[jj][ch];
    }
  }
}

// Explicit ||W||_F^2 for the matrices eig_gate flagged (head energy above 99% of
// ||A||^2): W = A - U diag(cw) V^T over the restore's 64 x 128 tiles, per-thread
// squares summed in fp64.  wn_parts() workgroups per matrix stride over its tiles,
// one partial each (wpart[b][part]); other matrices' workgroups return at once, so
// the common case costs B * WN_PARTS empty workgroups.  deflate_restore turns the
// partials into d.
__global__ __launch_bounds__(256) void w_norm_partials(
    const float* __restrict__ A, int n, int m, const float* __restrict__ U,
    const float* __restrict__ V, const int* __restrict__ kvec, const float* __restrict__ cw,
    const int* __restrict__ wflag, double* __restrict__ wpart) {
  const int b = blockIdx.z;
  if (!wflag[b]) return;   // uniform over the workgroup
  __shared__ __attribute__((aligned(16))) RestoreLds sm;
  __shared__ float coef[RP];
  __shared__ double red[256];
  const int tid = threadIdx.x;
  const int k = kvec[b];
  const float* Ab = A + (long long)b * n * m;
  const float* Ub = U + (long long)b * n * RP;
  const float* Vb = V + (long long)b * m * RP;
  const int c4 = (tid & 31) * 4, rw = tid >> 5;
  const bool vec = (m & 3) == 0;
  const int tiles_x = (m + DR_COLS - 1) / DR_COLS, ntiles = wn_tiles(n, m);
  if (tid < RP) coef[tid] = cw[b * RP + tid];
  double sq = 0.0;
  // the next tile's A and first head chunk are requested before this tile's work
  float x[8][4], ur[4], vr[8];
  int tile = blockIdx.x;
  if (tile < ntiles) {
    const int i0 = (tile / tiles_x) * DR_ROWS, j0 = (tile % tiles_x) * DR_COLS;
    dr_load_tile(Ab, n, m, i0, j0, rw, c4, vec, x);
    if (k > 0) dr_load_head(Ub, Vb, n, m, i0, j0, 0, min(DR_KC, k), tid, ur, vr);
  }
  while (tile < ntiles) {
    const int i0 = (tile / tiles_x) * DR_ROWS, j0 = (tile % tiles_x) * DR_COLS;
    const int nt = tile + gridDim.x;
    float xn[8][4], un[4], vn[8];
    if (nt < ntiles) {
      const int ni0 = (nt / tiles_x) * DR_ROWS, nj0 = (nt % tiles_x) * DR_COLS;
      dr_load_tile(Ab, n, m, ni0, nj0, rw, c4, vec, xn);
      if (k > 0) dr_load_head(Ub, Vb, n, m, ni0, nj0, 0, min(DR_KC, k), tid, un, vn);
    }
    for (int t0 = 0; t0 < k; t0 += DR_KC) {
      const int kc = min(DR_KC, k - t0);
      if (t0 > 0) dr_load_head(Ub, Vb, n, m, i0, j0, t0, kc, tid, ur, vr);
      __syncthreads();   // coef written; the previous chunk's readers done
      dr_stage_head(sm, ur, vr, tid);
      __syncthreads();
      dr_apply_head(sm, coef, t0, kc, rw, c4, x);
    }
#pragma unroll
    for (int a = 0; a < 8; ++a)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int gi = i0 + rw + 8 * a, gj = j0 + c4 + c;
        if (gi < n && gj < m) sq += (double)x[a][c] * (double)x[a][c];
      }
    tile = nt;
#pragma unroll
    for (int a = 0; a < 8; ++a)
#pragma unroll
      for (int c = 0; c < 4; ++c) x[a][c] = xn[a][c];
#pragma unroll
    for (int q = 0; q < 4; ++q) ur[q] = un[q];
#pragma unroll
    for (int q = 0; q < 8; ++q) vr[q] = vn[q];
  }
  red[tid] = sq;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (tid < w) red[tid] += red[tid + w];
    __syncthreads();
  }
  if (tid == 0) wpart[(long long)b * wn_parts(n, m) + blockIdx.x] = red[0];
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

// dst (rows x RP per matrix) = src (rows x cols, contiguous per matrix) with zero
// columns cols..RP-1; cols = RP copies, cols = 0 zero-fills
__global__ __launch_bounds__(256) void pad_cols(const float* __restrict__ src, int rows, int cols,
                                                float* __restrict__ dst) {
  const int b = blockIdx.y;
  const long long total = (long long)rows * RP;
  for (long long e = blockIdx.x * 256LL + threadIdx.x; e < total; e += 256LL * gridDim.x) {
    const int row = (int)(e / RP), c = (int)(e - (long long)row * RP);
    dst[(long long)b * total + e] =
        c < cols ? src[((long long)b * rows + row) * cols + c] : 0.f;
  }
}

__global__ __launch_bounds__(256) void fill_zero_i32(int* __restrict__ p, int count) {
  for (int e = blockIdx.x * 256 + threadIdx.x; e < count; e += 256 * gridDim.x) p[e] = 0;
}

// ---------------------------------------------------------------------------
// host side (no hipMemset/hipMemcpy: every clear and copy is a kernel, so the
// whole sequence stays plain kernel nodes if a caller captures it in a graph)
// ---------------------------------------------------------------------------
struct RsvdWs {
  float *Y, *Q, *Z, *Zq, *Bt, *U, *V, *M, *Ub, *UbS, *cw, *cr, *s;
  float *XT, *QT, *part;   // split-bf16 skinny GEMMs: transposed small operands, row-split partials
  double *gram, *gramq, *asq, *wpart;   // wpart: per-tile sums of W^2 (flagged matrices)
  long long* k64;
  int *kint, *degen, *wflag;
  size_t bytes;
};

static size_t align_up(size_t x) { return (x + 255) & ~(size_t)255; }

// The split-bf16 skinny GEMMs need m and n to be multiples of 8; other shapes run the
// fp32-MFMA kernels.
// The split-bf16 skinny products: shapes they cover (their buffer-descriptor offsets
// are 32-bit, below SK_OOB).
static bool sk_fast(int n, int m) {
  return n % 8 == 0 && m % 8 == 0 && (long long)n * m * 4 < (1LL << 31) &&
         (long long)RP * n * 4 < (1LL << 31);
}

static int zero_ints(hipStream_t st, int* p, int count) {
  if (count <= 0) return DMH_OK;
  const int blocks = ceil_div(count, 256) > 1024 ? 1024 : ceil_div(count, 256);
  hipLaunchKernelGGL(fill_zero_i32, dim3(blocks), dim3(256), 0, st, p, count);
  DMH_CHECK_LAUNCH("fill_zero_i32");
  return DMH_OK;
}

// dst (B, rows, RP) = src (B, rows, cols) zero-padded to RP columns
static int pad_to_rp(hipStream_t st, const float* src, int B, int rows, int cols, float* dst) {
  const long long total = (long long)rows * RP;
  const int gb = ceil_div(total, 256) > 4096 ? 4096 : ceil_div(total, 256);
  hipLaunchKernelGGL(pad_cols, dim3(gb, B), dim3(256), 0, st, src, rows, cols, dst);
  DMH_CHECK_LAUNCH("pad_cols");
  return DMH_OK;
}

// Row splits of sk_cols: about SKC_TARGET workgroups in all, at least 256 rows each.
static void sk_splits(int B, int n, int m, int* S, int* rps) {
  const long long wgs = (long long)ceil_div(m, SKC_COLS) * (B > 0 ? B : 1);
  int s = (int)((SKC_TARGET + wgs - 1) / wgs);
  s = s < 1 ? 1 : (s > SK_MAXS ? SK_MAXS : s);
  while (s > 1 && n / s < 256) --s;
  int r = ceil_div(n, s);
  r = (r + 15) / 16 * 16;
  *S = ceil_div(n, r);
  *rps = r;
}

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
  w.gram = (double*)take((size_t)B * GRAM_CHUNKS * RP * RP * sizeof(double));
  w.gramq = (double*)take((size_t)B * GRAM_CHUNKS * RP * RP * sizeof(double));
  w.asq = (double*)take((size_t)B * ceil_div(n, SG_ROWS) * sizeof(double));
  w.k64 = (long long*)take((size_t)B * sizeof(long long));
  w.kint = (int*)take((size_t)B * sizeof(int));
  w.degen = (int*)take((size_t)B * sizeof(int));
  w.wflag = (int*)take((size_t)B * sizeof(int));
  w.wpart = (double*)take((size_t)B * WN_PARTS * sizeof(double));
  if (sk_fast(n, m)) {
    int S, rps;
    sk_splits(B, n, m, &S, &rps);
    w.XT = (float*)take((size_t)B * RP * m * sizeof(float));
    w.QT = (float*)take((size_t)B * RP * n * sizeof(float));
    w.part = (float*)take((size_t)S * B * m * RP * sizeof(float));
  }
  w.bytes = off;
  return w;
}

static int check_dims(const char* what, int B, int n, int m, int r) {
  // (the Gram kernel addresses a sketch-width panel, n x RP fp32, with 32-bit offsets)
  if (B < 0 || n <= 0 || m <= 0 || r <= 0 || r > RP || r > m || n < m ||
      (long long)n * RP * 4 >= (1LL << 31)) {
    set_error("%s: unsupported shape (B=%d n=%d m=%d r=%d; need n >= m >= r, 1 <= r <= %d, "
              "n < 2^23)", what, B, n, m, r, RP);
    return DMH_EINVAL;
  }
  return DMH_OK;
}

// Y = A X (rows n) or Y = A^T X (rows m); asq: per-workgroup sums of squares of A
static int sg(hipStream_t st, int mode, const float* A, int B, int n, int m, const float* X,
              int ld_x, int xcols, long long x_bs, float* C, long long c_bs,
              double* asq = nullptr) {
  const int outrows = mode == SG_ROWSTREAM ? n : m;
  dim3 grid(ceil_div(outrows, SG_ROWS), B);
  if (mode == SG_ROWSTREAM)
    hipLaunchKernelGGL(skinny_gemm<SG_ROWSTREAM>, grid, dim3(256), 0, st, A, n, m,
                       (long long)n * m, X, ld_x, xcols, x_bs, C, c_bs, asq);
  else
    hipLaunchKernelGGL(skinny_gemm<SG_COLSTREAM>, grid, dim3(256), 0, st, A, n, m,
                       (long long)n * m, X, ld_x, xcols, x_bs, C, c_bs, (double*)nullptr);
  DMH_CHECK_LAUNCH("skinny_gemm");
  return DMH_OK;
}

static int gram(hipStream_t st, const float* Y, int B, int rows, double* part) {
  if (gram_stage(rows))
    hipLaunchKernelGGL(gram_partials<true>, dim3(GRAM_CHUNKS, B), dim3(64), 0, st, Y, rows,
                       (long long)rows * RP, part);
  else
    hipLaunchKernelGGL(gram_partials<false>, dim3(GRAM_CHUNKS, B), dim3(64), 0, st, Y, rows,
                       (long long)rows * RP, part);
  DMH_CHECK_LAUNCH("gram_partials");
  return DMH_OK;
}

// Q = orth(Y) by CholeskyQR (Y, Q: rows x RP), `passes` times; QT (optional, RP x rows):
// Q transposed, for the split-bf16 skinny GEMMs.
// need_q = false (with QT given): Q itself is not read afterwards, only QT -- the last
// pass writes QT alone
static int orth(hipStream_t st, const float* Y, float* Q, float* tmp, int B, int rows, int r,
                int passes, const RsvdWs& w, float* QT = nullptr, bool need_q = true) {
  const float* src = Y;
  int rc;
  for (int p = 0; p < passes; ++p) {
    const bool last = p == passes - 1;
    float* dst = last ? Q : (p % 2 == 0 ? tmp : Q);
    if ((rc = gram(st, src, B, rows, w.gram))) return rc;
    hipLaunchKernelGGL(chol_inv, dim3(B), dim3(CHOL_THREADS), 0, st, w.gram, r, w.M, w.degen);
    DMH_CHECK_LAUNCH("chol_inv");
    const RightMult rm{src, rows, (long long)rows * RP, w.M,
                       last && QT && !need_q ? (float*)nullptr : dst, (long long)rows * RP,
                       last ? QT : (float*)nullptr, rows};
    hipLaunchKernelGGL(right_mult, dim3(ceil_div(rows, 64), B), dim3(256), 0, st, rm);
    DMH_CHECK_LAUNCH("right_mult");
    src = dst;
  }
  if (passes == 0) {
    if ((rc = pad_to_rp(st, Y, B, rows, RP, Q))) return rc;
    if (QT) {
      hipLaunchKernelGGL(transpose_rp, dim3(ceil_div(rows, 64), B), dim3(256), 0, st, Y, rows, RP,
                         RP, (long long)rows * RP, QT, rows);
      DMH_CHECK_LAUNCH("orth transpose");
    }
  }
  return DMH_OK;
}

// Y (n x RP) = A XT^T with the split-bf16 kernel (XT: RP x m); asq optional
static int skr(hipStream_t st, const float* A, int B, int n, int m, const float* XT, float* Y,
               double* asq) {
  dim3 grid(ceil_div(n, SKR_ROWS), B);
  // the direct-to-LDS variant needs whole 64-index chunks; DMH_SKR_DTL=0 selects the
  // register-load kernel (same results) for comparisons
  const char* e = getenv("DMH_SKR_DTL");
  if (m % SK_KC == 0 && !(e && e[0] == '0'))
    hipLaunchKernelGGL((sk_rows_dtl<3, 8>), grid, dim3(512), 0, st, A, n, m, XT, m, Y, asq);
  else
    hipLaunchKernelGGL(sk_rows<3>, grid, dim3(256), 0, st, A, n, m, XT, m, Y, asq);
  DMH_CHECK_LAUNCH("sk_rows");
  return DMH_OK;
}

// C (m x RP) = A^T YT^T with the split-bf16 kernel (YT: RP x n), row splits reduced
// in order
static int skc(hipStream_t st, const float* A, int B, int n, int m, const float* YT, float* C,
               const RsvdWs& w) {
  int S, rps;
  sk_splits(B, n, m, &S, &rps);
  dim3 grid(ceil_div(m, SKC_COLS), S, B);
  // one split: the kernel writes C itself
  hipLaunchKernelGGL(sk_cols<3>, grid, dim3(256), 0, st, A, n, m, YT, n, rps, S == 1 ? C : w.part);
  DMH_CHECK_LAUNCH("sk_cols");
  if (S == 1) return DMH_OK;
  const long long per = (long long)B * m * RP;
  hipLaunchKernelGGL(sk_reduce, dim3((unsigned)ceil_div(per / 4, 256)), dim3(256), 0, st, w.part,
                     S, per, C);
  DMH_CHECK_LAUNCH("sk_reduce");
  return DMH_OK;
}

// U = Q Ub and V = Bp^T Ub diag(1/s), one launch
static int launch_uv(hipStream_t st, const RsvdWs& w, int B, int n, int m) {
  const RightMult pu{w.Q, n, (long long)n * RP, w.Ub, w.U, (long long)n * RP, nullptr, 0};
  const RightMult pv{w.Bt, m, (long long)m * RP, w.UbS, w.V, (long long)m * RP, nullptr, 0};
  hipLaunchKernelGGL(right_mult_pair, dim3(ceil_div(n, 64) + ceil_div(m, 64), B), dim3(256), 0,
                     st, pu, pv);
  DMH_CHECK_LAUNCH("right_mult (U, V)");
  return DMH_OK;
}

// The subspace iteration and Rayleigh-Ritz: leaves U (n x RP), V (m x RP), the
// gate outputs and s in the workspace; with d != nullptr also d = ||W||_F + 1e-7.
static int rsvd_core(hipStream_t st, const float* A, const float* Omega, int B, int n, int m,
                     int r, int niter, int passes, const GateParams& gp, long long* k_out,
                     float* d, const RsvdWs& w) {
  int rc;
  if ((rc = zero_ints(st, w.degen, B))) return rc;
  const bool fast = sk_fast(n, m);
  if (fast) {
    // split-bf16 path, 3 terms (fp32-accurate) for every product
    hipLaunchKernelGGL(transpose_rp, dim3(ceil_div(m, 64), B), dim3(256), 0, st, Omega, m, r, r,
                       (long long)m * r, w.XT, m);
    DMH_CHECK_LAUNCH("transpose Omega");
    if ((rc = skr(st, A, B, n, m, w.XT, w.Y, d ? w.asq : nullptr))) return rc;
    // (Q is read only after the last power iteration: the earlier orthonormalisations,
    // and every one of Z, feed the next skinny product through their transposes alone)
    if ((rc = orth(st, w.Y, w.Q, w.U, B, n, r, passes, w, w.QT, niter == 0))) return rc;
    for (int it = 0; it < niter; ++it) {
      if ((rc = skc(st, A, B, n, m, w.QT, w.Z, w))) return rc;
      if ((rc = orth(st, w.Z, w.Zq, w.V, B, m, r, passes, w, w.XT, false))) return rc;
      if ((rc = skr(st, A, B, n, m, w.XT, w.Y, nullptr))) return rc;
      if ((rc = orth(st, w.Y, w.Q, w.U, B, n, r, passes, w, w.QT, it == niter - 1))) return rc;
    }
    if ((rc = skc(st, A, B, n, m, w.QT, w.Bt, w))) return rc;
  } else {
    // Y = A Omega (and ||A||^2 partials) ; Q = orth(Y)
    if ((rc = sg(st, SG_ROWSTREAM, A, B, n, m, Omega, r, r, (long long)m * r, w.Y,
                 (long long)n * RP, d ? w.asq : nullptr)))
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
    // Bp^T = A^T Q (m x RP)
    if ((rc = sg(st, SG_COLSTREAM, A, B, n, m, w.Q, RP, RP, (long long)n * RP, w.Bt,
                 (long long)m * RP)))
      return rc;
  }
  // H = Bp Bp^T = Gram of Bp^T (and Q^T Q for d, in the same launch)
  if (d) {
    const dim3 gg(2 * GRAM_CHUNKS, B);
    if (gram_stage(m) && gram_stage(n))
      hipLaunchKernelGGL((gram_partials_pair<true, true>), gg, dim3(64), 0, st, w.Bt, m, w.gram,
                         w.Q, n, w.gramq);
    else if (gram_stage(m))
      hipLaunchKernelGGL((gram_partials_pair<true, false>), gg, dim3(64), 0, st, w.Bt, m, w.gram,
                         w.Q, n, w.gramq);
    else
      hipLaunchKernelGGL((gram_partials_pair<false, false>), gg, dim3(64), 0, st, w.Bt, m,
                         w.gram, w.Q, n, w.gramq);
    DMH_CHECK_LAUNCH("gram_partials (Bp, Q)");
  } else if ((rc = gram(st, w.Bt, B, m, w.gram))) {
    return rc;
  }
  if (d && gp.thresh >= gp.ratio) {
    // clip / fused paths: the head eigenpairs only (with the clip threshold at or above
    // the gate ratio, every deflated direction lies within the gate window)
    hipLaunchKernelGGL(eig_head_gate, dim3(B), dim3(EH_THREADS), 0, st, w.gram, gp, w.degen, w.s,
                       RP, w.Ub, w.UbS, k_out, w.kint, w.cw, w.cr, w.gramq, w.asq,
                       ceil_div(n, fast ? SKR_ROWS : SG_ROWS), d, w.wflag);
    DMH_CHECK_LAUNCH("eig_head_gate");
  } else {
    hipLaunchKernelGGL(eig_gate, dim3(B), dim3(EG_THREADS), 0, st, w.gram, gp, w.degen, w.s, RP,
                       w.Ub, w.UbS, k_out, w.kint, w.cw, w.cr, d ? w.gramq : nullptr,
                       d ? w.asq : nullptr, ceil_div(n, fast ? SKR_ROWS : SG_ROWS), d,
                       d ? w.wflag : nullptr);
    DMH_CHECK_LAUNCH("eig_gate");
  }
  // U = Q Ub ; V = Bp^T Ub diag(1/s)
  return launch_uv(st, w, B, n, m);
}

static int launch_restore(hipStream_t st, const float* A, int B, int n, int m, const RsvdWs& w,
                          float* d, void* X0, int x0_mode, bf16* T, bf16* W, int np,
                          int mp) {
  const int rows = T ? np : n, cols = T ? mp : m;
  hipLaunchKernelGGL(w_norm_partials, dim3(wn_parts(n, m), 1, B),
                     dim3(256), 0, st, A, n, m, w.U, w.V, w.kint, w.cw, w.wflag, w.wpart);
  DMH_CHECK_LAUNCH("w_norm_partials");
  dim3 grid(ceil_div(cols, DR_COLS), ceil_div(rows, DR_ROWS), B);
  hipLaunchKernelGGL(deflate_restore, grid, dim3(256), 0, st, A, n, m, w.U, w.V, w.kint, w.cw,
                     w.cr, d, w.wflag, w.wpart, X0, x0_mode, T, W, np, mp);
  DMH_CHECK_LAUNCH("deflate_restore");
  return DMH_OK;
}

static size_t fused_bytes(int B, int n, int m, size_t* chain_off) {
  const size_t rs = rsvd_layout(nullptr, B, n, m).bytes;
  const size_t cb = chain_ws(nullptr, B, chain_dims(n, m, 1)).bytes;
  if (chain_off) *chain_off = align_up(rs);
  return align_up(rs) + cb;
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

int dmh_deflated_polar_workspace_size(int batch, int n, int m, int r, size_t* bytes) {
  if (!bytes) {
    set_error("dmh_deflated_polar_workspace_size: null output");
    return DMH_EINVAL;
  }
  if (check_dims("dmh_deflated_polar_workspace_size", batch, n, m, r) ||
      chain_check("dmh_deflated_polar_workspace_size", chain_dims(n, m, 1)))
    return DMH_EINVAL;
  *bytes = fused_bytes(batch, n, m, nullptr);
  return DMH_OK;
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
  int rc = zero_ints(stream, w.degen, batch);
  if (!rc) rc = pad_to_rp(stream, X, batch, rows, r, w.Y);
  if (!rc) rc = orth(stream, w.Y, w.Q, w.U, batch, rows, r, passes, w);
  if (rc) return rc;
  const int gb = ceil_div((long long)rows * r, 256) > 4096 ? 4096 : ceil_div((long long)rows * r, 256);
  hipLaunchKernelGGL(copy_cols, dim3(gb, batch), dim3(256), 0, stream, w.Q, rows, r, Q);
  DMH_CHECK_LAUNCH("copy_cols");
  return DMH_OK;
}

static int copy_usv(hipStream_t stream, const RsvdWs& w, int batch, int n, int m, int r,
                    float* U, float* s, float* V) {
  const int gb = ceil_div((long long)n * r, 256) > 4096 ? 4096 : ceil_div((long long)n * r, 256);
  hipLaunchKernelGGL(copy_cols, dim3(gb, batch), dim3(256), 0, stream, w.U, n, r, U);
  const int gm = ceil_div((long long)m * r, 256) > 4096 ? 4096 : ceil_div((long long)m * r, 256);
  hipLaunchKernelGGL(copy_cols, dim3(gm, batch), dim3(256), 0, stream, w.V, m, r, V);
  hipLaunchKernelGGL(copy_cols, dim3(1, batch), dim3(256), 0, stream, w.s, 1, r, s);
  DMH_CHECK_LAUNCH("U, s, V outputs");
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
  int rc = zero_ints(stream, w.degen, batch);
  if (!rc) rc = pad_to_rp(stream, Q, batch, n, r, w.Q);
  if (rc) return rc;
  rc = sg(stream, SG_COLSTREAM, A, batch, n, m, w.Q, RP, RP, (long long)n * RP, w.Bt,
              (long long)m * RP);
  if (rc) return rc;
  if ((rc = gram(stream, w.Bt, batch, m, w.gram))) return rc;
  GateParams gp{r, 1, 0.f, 0.f, 1.f};
  hipLaunchKernelGGL(eig_gate, dim3(batch), dim3(EG_THREADS), 0, stream, w.gram, gp, w.degen, w.s, RP,
                     w.Ub, w.UbS, w.k64, w.kint, w.cw, w.cr, (const double*)nullptr,
                     (const double*)nullptr, 0, (float*)nullptr, (int*)nullptr);
  DMH_CHECK_LAUNCH("eig_gate");
  if ((rc = launch_uv(stream, w, batch, n, m))) return rc;
  return copy_usv(stream, w, batch, n, m, r, U, s, V);
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
  int rc = rsvd_core(stream, A, Omega, batch, n, m, r, niter, qr_passes, gp, w.k64, nullptr, w);
  if (rc) return rc;
  return copy_usv(stream, w, batch, n, m, r, U, s, V);
}

static int clip_args(const char* what, const float* A, const float* Omega, const void* X0,
                     const long long* k, const float* d, int batch, int n, int m, int r, int kw,
                     int niter, int qr_passes, float pad) {
  if (!A || !Omega || !X0 || !k || !d || kw < 1 || kw > r || niter < 0 || qr_passes < 0 ||
      !(pad > 0.f)) {
    set_error("%s: bad arguments (kw=%d r=%d niter=%d qr_passes=%d pad=%g)", what, kw, r, niter,
              qr_passes, (double)pad);
    return DMH_EINVAL;
  }
  return check_dims(what, batch, n, m, r);
}

int dmh_rmfro_clip(hipStream_t stream, const float* A, const float* Omega, int batch, int n,
                   int m, int r, int kw, float ratio, float thresh, float pad, int niter,
                   int qr_passes, void* X0, int out_bf16, long long* k, float* d, void* ws,
                   size_t ws_bytes) {
  if (batch == 0) return DMH_OK;
  if (clip_args("dmh_rmfro_clip", A, Omega, X0, k, d, batch, n, m, r, kw, niter, qr_passes, pad))
    return DMH_EINVAL;
  RsvdWs w = rsvd_layout(ws, batch, n, m);
  if (!ws || ws_bytes < w.bytes) {
    set_error("dmh_rmfro_clip: workspace %zu < %zu bytes", ws_bytes, w.bytes);
    return DMH_EWORKSPACE;
  }
  GateParams gp{r, kw, ratio, thresh, pad};
  int rc = rsvd_core(stream, A, Omega, batch, n, m, r, niter, qr_passes, gp, k, d, w);
  if (rc) return rc;
  return launch_restore(stream, A, batch, n, m, w, d, X0, out_bf16 ? 1 : 2, nullptr, nullptr, 0,
                        0);
}

// Front-end half of dmh_deflated_polar: rSVD, gate and d, and the deflated entry
// X0 written (bf16) straight into the chain's packed operand inside ws.
int dmh_deflated_polar_front(hipStream_t stream, const float* A, const float* Omega, int batch,
                             int n, int m, int r, int kw, float ratio, float thresh, float pad,
                             int niter, int qr_passes, long long* k, float* d, void* ws,
                             size_t ws_bytes) {
  if (batch == 0) return DMH_OK;
  // ws stands in for the output pointer: the entry goes into the workspace
  if (clip_args("dmh_deflated_polar_front", A, Omega, ws, k, d, batch, n, m, r, kw, niter,
                qr_passes, pad) ||
      chain_check("dmh_deflated_polar_front", chain_dims(n, m, 1)))
    return DMH_EINVAL;
  size_t chain_off = 0;
  const size_t need = fused_bytes(batch, n, m, &chain_off);
  if (!ws || ws_bytes < need) {
    set_error("dmh_deflated_polar_front: workspace %zu < %zu bytes", ws_bytes, need);
    return DMH_EWORKSPACE;
  }
  RsvdWs w = rsvd_layout(ws, batch, n, m);
  const ChainDims cd = chain_dims(n, m, 1);
  const ChainWs cw = chain_ws((char*)ws + chain_off, batch, cd);
  GateParams gp{r, kw, ratio, thresh, pad};
  int rc = rsvd_core(stream, A, Omega, batch, n, m, r, niter, qr_passes, gp, k, d, w);
  if (rc) return rc;
  return launch_restore(stream, A, batch, n, m, w, d, nullptr, 0, cw.T0, nullptr, cd.np, cd.mp);
}

// Chain half of dmh_deflated_polar: `steps` iterations from the entry that
// dmh_deflated_polar_front left in ws (same batch, n, m), polar factors to out
// (batch, n, m) bf16.
int dmh_deflated_polar_chain(hipStream_t stream, int batch, int n, int m, const double* coeffs,
                             int steps, void* out, void* ws, size_t ws_bytes) {
  if (batch == 0) return DMH_OK;
  if (batch < 0 || n < m || m <= 0 || !out || steps < 0 || (steps > 0 && !coeffs)) {
    set_error("dmh_deflated_polar_chain: bad arguments (batch=%d n=%d m=%d steps=%d)", batch, n,
              m, steps);
    return DMH_EINVAL;
  }
  if (chain_check("dmh_deflated_polar_chain", chain_dims(n, m, 1))) return DMH_EINVAL;
  size_t chain_off = 0;
  const size_t need = fused_bytes(batch, n, m, &chain_off);
  if (!ws || ws_bytes < need) {
    set_error("dmh_deflated_polar_chain: workspace %zu < %zu bytes", ws_bytes, need);
    return DMH_EWORKSPACE;
  }
  const ChainDims cd = chain_dims(n, m, 1);
  const ChainWs cw = chain_ws((char*)ws + chain_off, batch, cd);
  return chain_run_packed(stream, cw, batch, cd, 1, coeffs, steps, (bf16*)out);
}

int dmh_deflated_polar(hipStream_t stream, const float* A, const float* Omega, int batch, int n,
                       int m, int r, int kw, float ratio, float thresh, float pad, int niter,
                       int qr_passes, const double* coeffs, int steps, void* out, long long* k,
                       float* d, void* ws, size_t ws_bytes, void* chain_event) {
  if (batch == 0) return DMH_OK;
  if (clip_args("dmh_deflated_polar", A, Omega, out, k, d, batch, n, m, r, kw, niter, qr_passes,
                pad))
    return DMH_EINVAL;
  if (steps < 0 || (steps > 0 && !coeffs)) {
    set_error("dmh_deflated_polar: bad steps/coeffs (steps=%d)", steps);
    return DMH_EINVAL;
  }
  int rc = dmh_deflated_polar_front(stream, A, Omega, batch, n, m, r, kw, ratio, thresh, pad,
                                    niter, qr_passes, k, d, ws, ws_bytes);
  if (rc) return rc;
  if (chain_event && hipEventRecord((hipEvent_t)chain_event, stream) != hipSuccess) {
    set_error("dmh_deflated_polar: hipEventRecord failed");
    return DMH_ELAUNCH;
  }
  return dmh_deflated_polar_chain(stream, batch, n, m, coeffs, steps, out, ws, ws_bytes);
}

}  // extern "C"
