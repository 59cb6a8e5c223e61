// fp32 tall-convention polynomial chain (the dtype-preserving path of
//   _horner_iterate   defmuon/optim/deflation_batched.py:196-204
// for fp32 input: G = X^T X;  B = b G + (c G) G;  X <- a X + X B, all in fp32, with the
// reference's rounding points: c G and b G rounded on their own, each sum of two
// rounded terms rounded once; only the products' summation differs).
//
// The bf16 chain (ns_chain.hip) is the training path; this one serves callers that
// hand the iteration fp32 matrices (the reference's own convergence study runs it in
// fp32), one launch per GEMM phase over the batch.  Each phase is
//   C[i][j] = fl(fl(beta * R[i][j]) + fl(sum_k fl(s * P(i, k)) Q(j, k)))
// (the R term only where beta != 0, the scale s of P applied as its K slices are
// staged) with P and Q read through element strides, so T^T T, (c G) G and X B need
// no transposed copies.  The products run on the fp32 matrix cores
// (v_mfma_f32_32x32x2_f32, fp32 products and accumulation): 128 x 128 output tiles,
// 4 waves of 64 x 64 (2 x 2 blocks of 32 x 32), 16-deep K slices double-buffered in
// LDS as [k][row] (one barrier per slice), the next slice loaded into registers while
// the current one is multiplied.  Without packed fp32 (which this build leaves off)
// the vector units peak at half the matrix cores' 157.3 TFLOP/s.
#include "common.h"

namespace dmh {

constexpr int F_TILE = 128;
constexpr int F_BK = 16;
constexpr int F_LD = F_TILE + 4;   // LDS row stride (floats): 16-byte aligned rows

struct F32Gemm {
  const float* P; long long p_bs; int p_si, p_sk;   // P(i, k) = P[b*p_bs + i*p_si + k*p_sk]
  float p_scale;                                     // staged as fl(p_scale * P(i, k))
  const float* Q; long long q_bs; int q_sj, q_sk;   // Q(j, k)
  const float* R; long long r_bs; int r_ld;         // R[i][j] (beta != 0 only)
  float* C; long long c_bs; int c_ld;               // C[i][j]
  int I, J, K;
  float beta;
};

// One operand's K slice: 8 values per thread, held in registers between the global
// loads and the LDS stores.  KMAJ: the operand's rows are contiguous (element (r, k)
// at r + k * sk): thread t takes rows 4 (t % 32) .. +3 of slice rows k = t / 32 and
// t / 32 + 8.  Otherwise (k contiguous, (r, k) at r * sr + k): rows t / 4 and
// t / 4 + 64, k = 4 (t % 4) .. +3.  VEC: 16-byte loads (every bound and stride a
// multiple of 4 and the base 16-byte aligned, so a float4 is wholly in or out).
template <bool KMAJ, bool VEC>
struct F32Slice {
  float4 v[2];
  __device__ __forceinline__ void load(const float* base, int sr, int sk, int r0, int rows,
                                       int k0, int K, float scale) {
    const int t = threadIdx.x;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int r = KMAJ ? r0 + 4 * (t & 31) : r0 + (t >> 2) + 64 * u;
      const int k = KMAJ ? k0 + (t >> 5) + 8 * u : k0 + 4 * (t & 3);
      float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
      if (VEC) {
        if (r < rows && k < K) x = *(const float4*)(base + (long long)r * sr + (long long)k * sk);
      } else {
        float e[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int rq = KMAJ ? r + q : r, kq = KMAJ ? k : k + q;
          e[q] = (rq < rows && kq < K) ? base[(long long)rq * sr + (long long)kq * sk] : 0.f;
        }
        x = make_float4(e[0], e[1], e[2], e[3]);
      }
      if (scale != 1.f)
        x = make_float4(__fmul_rn(scale, x.x), __fmul_rn(scale, x.y), __fmul_rn(scale, x.z),
                        __fmul_rn(scale, x.w));
      v[u] = x;
    }
  }
  // S[k][r]: slice row k holds the operand's values for contraction index k0 + k
  __device__ __forceinline__ void store(float (*S)[F_LD]) const {
    const int t = threadIdx.x;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      if (KMAJ) {
        *(float4*)&S[(t >> 5) + 8 * u][4 * (t & 31)] = v[u];
      } else {
        const int r = (t >> 2) + 64 * u, k = 4 * (t & 3);
        S[k][r] = v[u].x;
        S[k + 1][r] = v[u].y;
        S[k + 2][r] = v[u].z;
        S[k + 3][r] = v[u].w;
      }
    }
  }
};

__device__ __forceinline__ f32x16 mfma_f32_32x32x2(float a, float b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// P K-major (PK: its rows contiguous) or k-contiguous; Q always K-major.  At most 128
// VGPRs, so that four workgroups share a CU (4% faster than the compiler's 140).
// grid (ceil(J / 128), ceil(I / 128), batch)
template <bool PK, bool VEC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4)))
void gemm_f32(F32Gemm g) {
  __shared__ __attribute__((aligned(16))) float Ps[2][F_BK][F_LD];
  __shared__ __attribute__((aligned(16))) float Qs[2][F_BK][F_LD];
  const int b = blockIdx.z;
  const int i0 = blockIdx.y * F_TILE, j0 = blockIdx.x * F_TILE;
  const float* P = g.P + (long long)b * g.p_bs;
  const float* Q = g.Q + (long long)b * g.q_bs;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wi = 64 * (wave >> 1), wj = 64 * (wave & 1);   // the wave's 64 x 64 block
  const int r32 = lane & 31, kh = lane >> 5;
  F32Slice<PK, VEC> sp;
  F32Slice<true, VEC> sq;
  const int p_sr = PK ? 1 : g.p_si, p_sk = PK ? g.p_sk : 1;
  f32x16 acc[2][2];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[x][y][e] = 0.f;
  const int nk = (g.K + F_BK - 1) / F_BK;
  sp.load(P, p_sr, p_sk, i0, g.I, 0, g.K, g.p_scale);
  sq.load(Q, 1, g.q_sk, j0, g.J, 0, g.K, 1.f);
  sp.store(Ps[0]);
  sq.store(Qs[0]);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) {   // next slice into registers under this slice's products
      sp.load(P, p_sr, p_sk, i0, g.I, (kt + 1) * F_BK, g.K, g.p_scale);
      sq.load(Q, 1, g.q_sk, j0, g.J, (kt + 1) * F_BK, g.K, 1.f);
    }
#pragma unroll
    for (int kk = 0; kk < F_BK; kk += 2) {
      // lanes 0-31 hold contraction index kk, lanes 32-63 kk + 1
      const float a0 = Ps[cur][kk + kh][wi + r32], a1 = Ps[cur][kk + kh][wi + 32 + r32];
      const float b0 = Qs[cur][kk + kh][wj + r32], b1 = Qs[cur][kk + kh][wj + 32 + r32];
      acc[0][0] = mfma_f32_32x32x2(a0, b0, acc[0][0]);
      acc[0][1] = mfma_f32_32x32x2(a0, b1, acc[0][1]);
      acc[1][0] = mfma_f32_32x32x2(a1, b0, acc[1][0]);
      acc[1][1] = mfma_f32_32x32x2(a1, b1, acc[1][1]);
    }
    if (kt + 1 < nk) {
      // the other buffer was last read in slice kt - 1, before the previous barrier
      sp.store(Ps[cur ^ 1]);
      sq.store(Qs[cur ^ 1]);
    }
    __syncthreads();
  }
  // acc[x][y][e] holds C[wi + 32 x + 8 (e / 4) + 4 kh + e % 4][wj + 32 y + r32]
  float* C = g.C + (long long)b * g.c_bs;
  const float* R = g.beta != 0.f ? g.R + (long long)b * g.r_bs : nullptr;
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y) {
      const int j = j0 + wj + 32 * y + r32;
      if (j >= g.J) continue;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int i = i0 + wi + 32 * x + 8 * (e >> 2) + 4 * kh + (e & 3);
        if (i >= g.I) continue;
        float v = acc[x][y][e];
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

static bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

static int launch_f32(const F32Gemm& g, int batch, hipStream_t stream, const char* what) {
  const bool pk = g.p_si == 1;
  if (g.q_sj != 1 || (!pk && g.p_sk != 1)) {
    set_error("%s: operand layout not supported (P strides %d,%d, Q strides %d,%d)", what,
              g.p_si, g.p_sk, g.q_sj, g.q_sk);
    return DMH_EINVAL;
  }
  // 16-byte staging loads when every float4 lies wholly inside or outside the operand
  const bool vec = al16(g.P) && al16(g.Q) && g.p_bs % 4 == 0 && g.q_bs % 4 == 0 &&
                   g.q_sk % 4 == 0 && g.J % 4 == 0 &&
                   (pk ? (g.p_sk % 4 == 0 && g.I % 4 == 0) : (g.p_si % 4 == 0 && g.K % 4 == 0));
  const dim3 grid(ceil_div(g.J, F_TILE), ceil_div(g.I, F_TILE), batch);
  if (pk && vec) hipLaunchKernelGGL((gemm_f32<true, true>), grid, dim3(256), 0, stream, g);
  else if (pk) hipLaunchKernelGGL((gemm_f32<true, false>), grid, dim3(256), 0, stream, g);
  else if (vec) hipLaunchKernelGGL((gemm_f32<false, true>), grid, dim3(256), 0, stream, g);
  else hipLaunchKernelGGL((gemm_f32<false, false>), grid, dim3(256), 0, stream, g);
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
