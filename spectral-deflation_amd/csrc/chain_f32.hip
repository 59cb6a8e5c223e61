// fp32 tall-convention polynomial chain (the dtype-preserving path of
//   _horner_iterate   defmuon/optim/deflation_batched.py:196-204
// for fp32 input: G = X^T X;  B = b G + (c G) G;  X <- a X + X B, all in fp32, with the
// reference's rounding points: c G and b G rounded on their own, each sum of two
// rounded terms rounded once; only the products' summation order differs).
//
// The bf16 chain (ns_chain.hip) is the training path; this one serves callers that
// hand the iteration fp32 matrices (the reference's own convergence study runs it in
// fp32), one launch per GEMM phase over the batch.  Each phase is
//   C[i][j] = fl(fl(beta * R[i][j]) + fl(sum_k fl(s * P(i, k)) Q(j, k)))
// (the R term only where beta != 0, the scale s of P applied as its K slices are
// staged) with P and Q read through element strides, so T^T T, (c G) G and X B need
// no transposed copies.  64 x 64 output tiles, 16-deep K slices staged in LDS, 4 x 4
// outputs per thread accumulated in k order with fp32 FMAs.  (MI355X's fp32 matrix
// cores have the same 157.3 TFLOP/s peak as its fp32 vector units, so this path
// stays on the VALU.)
#include "common.h"

namespace dmh {

constexpr int F_TILE = 64;
constexpr int F_BK = 16;

struct F32Gemm {
  const float* P; long long p_bs; int p_si, p_sk;   // P(i, k) = P[b*p_bs + i*p_si + k*p_sk]
  float p_scale;                                     // staged as fl(p_scale * P(i, k))
  const float* Q; long long q_bs; int q_sj, q_sk;   // Q(j, k)
  const float* R; long long r_bs; int r_ld;         // R[i][j] (beta != 0 only)
  float* C; long long c_bs; int c_ld;               // C[i][j]
  int I, J, K;
  float beta;
};

// one K slice of a 64-row operand panel into LDS, S[k][row] = fl(scale * operand);
// coalesced along the operand's unit-stride index
__device__ __forceinline__ void f32_stage(float (*S)[F_TILE + 4], const float* base, int si,
                                          int sk, int r0, int rows, int k0, int K,
                                          float scale) {
  const int t = threadIdx.x;
  if (si == 1) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int r = t & 63, k = (t >> 6) + 4 * u;
      const int gr = r0 + r, gk = k0 + k;
      S[k][r] = (gr < rows && gk < K) ? __fmul_rn(scale, base[(long long)gr * si + (long long)gk * sk]) : 0.f;
    }
  } else {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int k = t & 15, r = (t >> 4) + 16 * u;
      const int gr = r0 + r, gk = k0 + k;
      S[k][r] = (gr < rows && gk < K) ? __fmul_rn(scale, base[(long long)gr * si + (long long)gk * sk]) : 0.f;
    }
  }
}

__global__ __launch_bounds__(256) void gemm_f32(F32Gemm g) {
  __shared__ float Ps[F_BK][F_TILE + 4];
  __shared__ float Qs[F_BK][F_TILE + 4];
  const int b = blockIdx.z;
  const int i0 = blockIdx.y * F_TILE, j0 = blockIdx.x * F_TILE;
  const float* P = g.P + (long long)b * g.p_bs;
  const float* Q = g.Q + (long long)b * g.q_bs;
  const int ti = threadIdx.x >> 4, tj = threadIdx.x & 15;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < g.K; k0 += F_BK) {
    f32_stage(Ps, P, g.p_si, g.p_sk, i0, g.I, k0, g.K, g.p_scale);
    f32_stage(Qs, Q, g.q_sj, g.q_sk, j0, g.J, k0, g.K, 1.f);
    __syncthreads();
#pragma unroll
    for (int k = 0; k < F_BK; ++k) {
      const float4 pv = *(const float4*)&Ps[k][4 * ti];
      const float4 qv = *(const float4*)&Qs[k][4 * tj];
      const float p[4] = {pv.x, pv.y, pv.z, pv.w}, q[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
      for (int x = 0; x < 4; ++x)
#pragma unroll
        for (int y = 0; y < 4; ++y) acc[x][y] = fmaf(p[x], q[y], acc[x][y]);
    }
    __syncthreads();
  }
  float* C = g.C + (long long)b * g.c_bs;
  const float* R = g.beta != 0.f ? g.R + (long long)b * g.r_bs : nullptr;
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    const int i = i0 + 4 * ti + x;
    if (i >= g.I) continue;
#pragma unroll
    for (int y = 0; y < 4; ++y) {
      const int j = j0 + 4 * tj + y;
      if (j >= g.J) continue;
      float v = acc[x][y];
      if (R) v = __fadd_rn(__fmul_rn(g.beta, R[(long long)i * g.r_ld + j]), v);
      C[(long long)i * g.c_ld + j] = v;
    }
  }
}

__global__ __launch_bounds__(256) void copy_f32(const float* __restrict__ src, float* __restrict__ dst,
                                                long long count) {
  for (long long e = blockIdx.x * 256LL + threadIdx.x; e < count; e += 256LL * gridDim.x)
    dst[e] = src[e];
}

static int launch_f32(const F32Gemm& g, int batch, hipStream_t stream, const char* what) {
  const dim3 grid(ceil_div(g.J, F_TILE), ceil_div(g.I, F_TILE), batch);
  hipLaunchKernelGGL(gemm_f32, grid, dim3(256), 0, stream, g);
  DMH_CHECK_LAUNCH(what);
  return DMH_OK;
}

static size_t horner_f32_ws(int batch, int n, int m) {
  return (size_t)batch * (2 * (size_t)m * m + (size_t)n * m) * sizeof(float);
}

}  // namespace dmh

using namespace dmh;

extern "C" {

int dmh_horner_f32_workspace_size(int batch, int n, int m, size_t* bytes) {
  if (batch < 0 || n <= 0 || m <= 0 || !bytes) {
    set_error("dmh_horner_f32_workspace_size: bad arguments");
    return DMH_EINVAL;
  }
  *bytes = horner_f32_ws(batch, n, m);
  return DMH_OK;
}

int dmh_horner_f32(hipStream_t stream, const float* x, int batch, int n, int m, float* out,
                   const double* coeffs, int steps, void* ws, size_t ws_bytes) {
  if (batch == 0) return DMH_OK;
  if (!x || !out || batch < 0 || n <= 0 || m <= 0 || steps < 0 || (steps > 0 && !coeffs)) {
    set_error("dmh_horner_f32: bad arguments (batch=%d n=%d m=%d steps=%d)", batch, n, m, steps);
    return DMH_EINVAL;
  }
  const size_t need = horner_f32_ws(batch, n, m);
  if (!ws || ws_bytes < need) {
    set_error("dmh_horner_f32: workspace %zu < %zu bytes", ws_bytes, need);
    return DMH_EWORKSPACE;
  }
  const long long tsz = (long long)n * m, gsz = (long long)m * m;
  if (steps == 0) {
    const long long count = tsz * batch;
    const int blocks = (int)std::min<long long>((count + 255) / 256, 8192);
    hipLaunchKernelGGL(copy_f32, dim3(blocks), dim3(256), 0, stream, x, out, count);
    DMH_CHECK_LAUNCH("dmh_horner_f32 copy");
    return DMH_OK;
  }
  float* G = (float*)ws;
  float* Bm = G + gsz * batch;
  float* tmp = Bm + gsz * batch;
  const float* src = x;
  for (int it = 0; it < steps; ++it) {
    const float a = (float)coeffs[3 * it], b = (float)coeffs[3 * it + 1],
                c = (float)coeffs[3 * it + 2];
    float* dst = ((steps - 1 - it) % 2 == 0) ? out : tmp;   // the last step lands in out
    int rc;
    // G = X^T X: P(i, k) = Q(i, k) = X[k][i]
    F32Gemm g1{src, tsz, 1, m, 1.f, src, tsz, 1, m, nullptr, 0, 0, G, gsz, m, m, m, n, 0.f};
    if ((rc = launch_f32(g1, batch, stream, "dmh_horner_f32 G"))) return rc;
    // B = b G + (c G) G: P(i, k) = c G[i][k], Q(j, k) = G[k][j]
    F32Gemm g2{G, gsz, m, 1, c, G, gsz, 1, m, G, gsz, m, Bm, gsz, m, m, m, m, b};
    if ((rc = launch_f32(g2, batch, stream, "dmh_horner_f32 B"))) return rc;
    // X' = a X + X B: P(i, k) = X[i][k], Q(j, k) = B[k][j]
    F32Gemm g3{src, tsz, m, 1, 1.f, Bm, gsz, 1, m, src, tsz, m, dst, tsz, m, n, m, m, a};
    if ((rc = launch_f32(g3, batch, stream, "dmh_horner_f32 X"))) return rc;
    src = dst;
  }
  return DMH_OK;
}

}  // extern "C"
