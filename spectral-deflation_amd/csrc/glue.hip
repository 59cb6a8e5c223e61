// The optimizer glue on either side of the polar path, fused per shape group.
//
// Input side (defmuon/optim/muon.py:266-289): for every parameter of a tall-shape
// group, the Nesterov momentum update
//     buf <- buf * mu + g ;   g' = g + mu * buf   (or g' = buf without Nesterov)
// then the W_QKV split (muon.py:160-165), the fp32 cast, the wide -> tall
// transpose and the torch.cat into the (B, n, m) stack that the deflation
// front-end reads -- one launch for the whole group instead of about eight
// elementwise passes and a copy per parameter.
//
// Output side (muon.py:316-332): u (the bf16 polar factor, tall) back into the
// parameter's layout and
//     p <- p * (1 - lr wd) ;   p <- p + (-lr_p) * u
// again one launch per group.
//
// Rounding follows the reference's separate torch ops: each op rounds to fp32,
// so products and sums are kept apart (the functions below switch off the
// compiler's multiply-add contraction, which otherwise fuses them); the ops that
// torch runs as one elementwise kernel with an alpha (add(b, alpha)) are one fused
// multiply-add, as torch's own kernel evaluates a + alpha * b.
//
// Parameters travel by value in the kernel arguments (GLUE_MAX per launch, more in
// several launches), so the library allocates nothing and copies nothing to the
// device for them.
#include "common.h"

namespace dmh {

constexpr int GLUE_MAX = 32;   // parameters per launch
constexpr int GT = 64;         // tile edge

struct GlueParam {
  const float* grad;   // (rows, cols), contiguous
  float* buf;          // momentum buffer, same shape, updated in place
  float* param;        // the parameter, same shape
  int rows, cols;      // the parameter's shape
  int blocks;          // matrices along the rows (3 for W_QKV)
  int transpose;       // 1: each block is stored transposed in the stack
  long long offset;    // element offset of the first block in the stack
  float alpha;         // update: -lr * sqrt(fan_out / fan_in)
  float decay;         // update: 1 - lr * wd
};

struct GlueArgs {
  GlueParam p[GLUE_MAX];
  int count;
  float mu;
  int nesterov;
  float* stack;          // momentum side: (B, n, m) fp32
  const bf16* ustack;    // update side: (B, n, m) bf16
};

// tall block shape of a parameter and its tile counts
struct BlockGeom {
  int rb, n, m, tn, tm, tiles;
};
__device__ __forceinline__ BlockGeom geom(const GlueParam& d) {
  BlockGeom g;
  g.rb = d.rows / d.blocks;
  g.n = d.transpose ? d.cols : g.rb;
  g.m = d.transpose ? g.rb : d.cols;
  g.tn = (g.n + GT - 1) / GT;
  g.tm = (g.m + GT - 1) / GT;
  g.tiles = d.blocks * g.tn * g.tm;
  return g;
}

__device__ __forceinline__ float nesterov_step(float grad, float& buf, float mu, int nesterov) {
#pragma clang fp contract(off)
  const float t = buf * mu;                     // buf.mul_(mu)
  buf = t + grad;                               // .add_(grad)
  return nesterov ? fmaf(mu, buf, grad) : buf;  // grad.add(buf, alpha=mu)
}

__device__ __forceinline__ float decayed(float p, float decay) {
#pragma clang fp contract(off)
  return p * decay;                             // p.mul_(1 - lr wd)
}

// 16-byte access is possible for a parameter when its rows, its tall block's rows
// and every base address are 4-element aligned (then a whole 64 x 64 tile is read and
// written 4 elements per lane)
__device__ __forceinline__ bool glue_vec(const GlueParam& d, const BlockGeom& g, const void* other) {
  return (d.cols & 3) == 0 && (g.m & 3) == 0 && (g.n & 3) == 0 && (d.offset & 3) == 0 &&
         ((((uintptr_t)d.grad) | ((uintptr_t)d.buf) | ((uintptr_t)d.param) |
           ((uintptr_t)other)) & 15) == 0;
}

// One workgroup per 64 x 64 tile of a tall block (grid-stride over the tiles of
// parameter blockIdx.y).  Without transpose both sides are row-contiguous; with it
// the tile goes through LDS so that the parameter side is read along its rows and
// the stack side written along its rows.  Whole tiles of aligned parameters move 4
// elements per lane (16 lanes per 64-element row); edge tiles go element by element.
__global__ __launch_bounds__(256) void momentum_stack(GlueArgs a) {
  __shared__ float t[GT][GT + 1];
  const GlueParam& d = a.p[blockIdx.y];
  const BlockGeom g = geom(d);
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int c4 = (threadIdx.x & 15) * 4, r16 = threadIdx.x >> 4;   // vector lanes
  const bool vec = glue_vec(d, g, a.stack);
  for (int tile = blockIdx.x; tile < g.tiles; tile += gridDim.x) {
    const int k = tile / (g.tn * g.tm);
    const int rem = tile - k * g.tn * g.tm;
    const int i0 = (rem / g.tm) * GT, j0 = (rem % g.tm) * GT;   // in the tall block
    float* dst = a.stack + d.offset + (long long)k * g.n * g.m;
    const bool whole = vec && i0 + GT <= g.n && j0 + GT <= g.m;
    if (!d.transpose) {
      if (whole) {
#pragma unroll
        for (int q = 0; q < GT / 16; ++q) {
          const int i = i0 + r16 + 16 * q, j = j0 + c4;
          const long long src = (long long)(k * g.rb + i) * d.cols + j;
          float4 b = *(const float4*)(d.buf + src);
          const float4 gr = *(const float4*)(d.grad + src);
          float4 v;
          v.x = nesterov_step(gr.x, b.x, a.mu, a.nesterov);
          v.y = nesterov_step(gr.y, b.y, a.mu, a.nesterov);
          v.z = nesterov_step(gr.z, b.z, a.mu, a.nesterov);
          v.w = nesterov_step(gr.w, b.w, a.mu, a.nesterov);
          *(float4*)(d.buf + src) = b;
          *(float4*)(dst + (long long)i * g.m + j) = v;
        }
        continue;
      }
      for (int ii = ty; ii < GT; ii += 4) {
        const int i = i0 + ii, j = j0 + tx;
        if (i >= g.n || j >= g.m) continue;
        const long long src = (long long)(k * g.rb + i) * d.cols + j;
        float b = d.buf[src];
        const float v = nesterov_step(d.grad[src], b, a.mu, a.nesterov);
        d.buf[src] = b;
        dst[(long long)i * g.m + j] = v;
      }
    } else {
      // tall (i, j) = parameter (k rb + j, i): parameter rows j0.., columns i0..
      __syncthreads();
      if (whole) {
#pragma unroll
        for (int q = 0; q < GT / 16; ++q) {
          const int rr = r16 + 16 * q;
          const long long src = (long long)(k * g.rb + j0 + rr) * d.cols + i0 + c4;
          float4 b = *(const float4*)(d.buf + src);
          const float4 gr = *(const float4*)(d.grad + src);
          t[rr][c4 + 0] = nesterov_step(gr.x, b.x, a.mu, a.nesterov);
          t[rr][c4 + 1] = nesterov_step(gr.y, b.y, a.mu, a.nesterov);
          t[rr][c4 + 2] = nesterov_step(gr.z, b.z, a.mu, a.nesterov);
          t[rr][c4 + 3] = nesterov_step(gr.w, b.w, a.mu, a.nesterov);
          *(float4*)(d.buf + src) = b;
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < GT / 16; ++q) {
          const int ii = r16 + 16 * q;
          *(float4*)(dst + (long long)(i0 + ii) * g.m + j0 + c4) =
              make_float4(t[c4][ii], t[c4 + 1][ii], t[c4 + 2][ii], t[c4 + 3][ii]);
        }
        continue;
      }
      for (int rr = ty; rr < GT; rr += 4) {
        const int pr = j0 + rr, pc = i0 + tx;
        if (pr < g.m && pc < g.n) {
          const long long src = (long long)(k * g.rb + pr) * d.cols + pc;
          float b = d.buf[src];
          t[rr][tx] = nesterov_step(d.grad[src], b, a.mu, a.nesterov);
          d.buf[src] = b;
        }
      }
      __syncthreads();
      for (int ii = ty; ii < GT; ii += 4) {
        const int i = i0 + ii, j = j0 + tx;
        if (i < g.n && j < g.m) dst[(long long)i * g.m + j] = t[tx][ii];
      }
    }
  }
}

__global__ __launch_bounds__(256) void apply_update(GlueArgs a) {
  __shared__ float t[GT][GT + 1];
  const GlueParam& d = a.p[blockIdx.y];
  const BlockGeom g = geom(d);
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int c4 = (threadIdx.x & 15) * 4, r16 = threadIdx.x >> 4;   // vector lanes
  // (bf16 updates: 4 elements are 8 bytes)
  const bool vec = glue_vec(d, g, nullptr) && (((uintptr_t)a.ustack) & 7) == 0;
  for (int tile = blockIdx.x; tile < g.tiles; tile += gridDim.x) {
    const int k = tile / (g.tn * g.tm);
    const int rem = tile - k * g.tn * g.tm;
    const int i0 = (rem / g.tm) * GT, j0 = (rem % g.tm) * GT;
    const bf16* src = a.ustack + d.offset + (long long)k * g.n * g.m;
    const bool whole = vec && i0 + GT <= g.n && j0 + GT <= g.m;
    if (!d.transpose) {
      if (whole) {
#pragma unroll
        for (int q = 0; q < GT / 16; ++q) {
          const int i = i0 + r16 + 16 * q, j = j0 + c4;
          const long long pi = (long long)(k * g.rb + i) * d.cols + j;
          float4 pv = *(const float4*)(d.param + pi);
          const bf16x4 u = *(const bf16x4*)(src + (long long)i * g.m + j);
          pv.x = fmaf(d.alpha, bf2f(u[0]), decayed(pv.x, d.decay));
          pv.y = fmaf(d.alpha, bf2f(u[1]), decayed(pv.y, d.decay));
          pv.z = fmaf(d.alpha, bf2f(u[2]), decayed(pv.z, d.decay));
          pv.w = fmaf(d.alpha, bf2f(u[3]), decayed(pv.w, d.decay));
          *(float4*)(d.param + pi) = pv;
        }
        continue;
      }
      for (int ii = ty; ii < GT; ii += 4) {
        const int i = i0 + ii, j = j0 + tx;
        if (i >= g.n || j >= g.m) continue;
        const long long pi = (long long)(k * g.rb + i) * d.cols + j;
        const float pd = decayed(d.param[pi], d.decay);
        d.param[pi] = fmaf(d.alpha, bf2f(src[(long long)i * g.m + j]), pd);   // p.add_(u, alpha)
      }
    } else {
      __syncthreads();
      if (whole) {
#pragma unroll
        for (int q = 0; q < GT / 16; ++q) {
          const int ii = r16 + 16 * q;
          const bf16x4 u = *(const bf16x4*)(src + (long long)(i0 + ii) * g.m + j0 + c4);
          t[ii][c4 + 0] = bf2f(u[0]);
          t[ii][c4 + 1] = bf2f(u[1]);
          t[ii][c4 + 2] = bf2f(u[2]);
          t[ii][c4 + 3] = bf2f(u[3]);
        }
        __syncthreads();
        // parameter (k rb + j, i) = tall (i, j): parameter rows j0.., columns i0..
#pragma unroll
        for (int q = 0; q < GT / 16; ++q) {
          const int rr = r16 + 16 * q;
          const long long pi = (long long)(k * g.rb + j0 + rr) * d.cols + i0 + c4;
          float4 pv = *(const float4*)(d.param + pi);
          pv.x = fmaf(d.alpha, t[c4 + 0][rr], decayed(pv.x, d.decay));
          pv.y = fmaf(d.alpha, t[c4 + 1][rr], decayed(pv.y, d.decay));
          pv.z = fmaf(d.alpha, t[c4 + 2][rr], decayed(pv.z, d.decay));
          pv.w = fmaf(d.alpha, t[c4 + 3][rr], decayed(pv.w, d.decay));
          *(float4*)(d.param + pi) = pv;
        }
        continue;
      }
      for (int ii = ty; ii < GT; ii += 4) {
        const int i = i0 + ii, j = j0 + tx;
        t[ii][tx] = (i < g.n && j < g.m) ? bf2f(src[(long long)i * g.m + j]) : 0.f;
      }
      __syncthreads();
      // parameter (k rb + j, i) = tall (i, j): parameter rows j0.., columns i0..
      for (int rr = ty; rr < GT; rr += 4) {
        const int pr = j0 + rr, pc = i0 + tx;
        if (pr >= g.m || pc >= g.n) continue;
        const long long pi = (long long)(k * g.rb + pr) * d.cols + pc;
        const float pd = decayed(d.param[pi], d.decay);
        d.param[pi] = fmaf(d.alpha, t[tx][rr], pd);
      }
    }
  }
}

static int glue_launch(hipStream_t stream, const GlueParam* ps, int count, float mu,
                       int nesterov, float* stack, const bf16* ustack, int update,
                       const char* what) {
  for (int c0 = 0; c0 < count; c0 += GLUE_MAX) {
    GlueArgs a{};
    a.count = count - c0 < GLUE_MAX ? count - c0 : GLUE_MAX;
    a.mu = mu;
    a.nesterov = nesterov;
    a.stack = stack;
    a.ustack = ustack;
    int tiles = 1;
    for (int i = 0; i < a.count; ++i) {
      const GlueParam& d = ps[c0 + i];
      const int rb = d.rows / d.blocks;
      const int n = d.transpose ? d.cols : rb, m = d.transpose ? rb : d.cols;
      const int t = d.blocks * ceil_div(n, GT) * ceil_div(m, GT);
      if (t > tiles) tiles = t;
      a.p[i] = d;
    }
    const int gx = tiles < 2048 ? tiles : 2048;
    if (update)
      hipLaunchKernelGGL(apply_update, dim3(gx, a.count), dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL(momentum_stack, dim3(gx, a.count), dim3(256), 0, stream, a);
    DMH_CHECK_LAUNCH(what);
  }
  return DMH_OK;
}

static int check_params(const char* what, const GlueParam* ps, int count, int update) {
  if (count < 0 || (count > 0 && !ps)) {
    set_error("%s: bad parameter list (count=%d)", what, count);
    return DMH_EINVAL;
  }
  for (int i = 0; i < count; ++i) {
    const GlueParam& d = ps[i];
    const bool ptrs = update ? d.param != nullptr : (d.grad && d.buf);
    if (!ptrs || d.rows <= 0 || d.cols <= 0 || d.blocks <= 0 || d.rows % d.blocks != 0 ||
        d.offset < 0 || (d.transpose != 0 && d.transpose != 1)) {
      set_error("%s: bad parameter %d (rows=%d cols=%d blocks=%d transpose=%d)", what, i, d.rows,
                d.cols, d.blocks, d.transpose);
      return DMH_EINVAL;
    }
  }
  return DMH_OK;
}

// ---------------------------------------------------------------------------
// AdamW backup of the Muon optimizer (muon.py:408-436) for every non-Muon parameter
// of a group in one launch.  Per element, the reference's torch ops in order, each
// rounded to fp32:
//     m1 <- lerp(m1, g, w1)           m1.lerp_(g, 1 - beta1)
//     m2 <- lerp(m2, g * g, w2)       m2.lerp_(g.square(), 1 - beta2)
//     u  <- m1 / (sqrt(m2) + eps)     buf1 / (eps + buf2.sqrt())
//     p  <- p * decay                 p.mul_(1 - lr wd)
//     p  <- p + alpha * u             p.add_(u, alpha=-lr / scale)
// torch's lerp takes self + w (end - self) for |w| < 0.5, else end - (end - self)(1 - w),
// each as one elementwise expression (a fused multiply-add); the division and the
// square root are correctly rounded, as torch's are.
// The parameter table and the chunk boundaries are device arrays the caller keeps
// (the same tensors every step), so a launch copies and allocates nothing.
// ---------------------------------------------------------------------------
struct AdamwParam {
  float* param;
  const float* grad;
  float* m1;
  float* m2;
  long long numel;
};
constexpr int ADAMW_CHUNK = 4096;   // elements per workgroup

__device__ __forceinline__ float torch_lerp(float self, float end, float w) {
  return fabsf(w) < 0.5f ? fmaf(w, end - self, self) : fmaf(-(end - self), 1.0f - w, end);
}

__device__ __forceinline__ void adamw_elem(float& p, float g, float& m1, float& m2, float w1,
                                           float w2, float eps, float decay, float alpha) {
#pragma clang fp contract(off)
  m1 = torch_lerp(m1, g, w1);
  const float g2 = g * g;
  m2 = torch_lerp(m2, g2, w2);
  const float u = m1 / (sqrtf(m2) + eps);
  const float pd = p * decay;
  p = fmaf(alpha, u, pd);
}

// chunk c of the group: parameter i with chunk_start[i] <= c < chunk_start[i + 1]
__global__ __launch_bounds__(256) void adamw_step(const AdamwParam* __restrict__ tab, int count,
                                                  const int* __restrict__ chunk_start, float w1,
                                                  float w2, float eps, float decay, float alpha) {
  const int c = blockIdx.x;
  int lo = 0, hi = count;   // chunk_start[lo] <= c < chunk_start[hi]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (chunk_start[mid] <= c) lo = mid; else hi = mid;
  }
  const AdamwParam d = tab[lo];
  const long long e0 = (long long)(c - chunk_start[lo]) * ADAMW_CHUNK;
  const long long e1 = e0 + ADAMW_CHUNK < d.numel ? e0 + ADAMW_CHUNK : d.numel;
  const bool vec = ((((uintptr_t)d.param) | ((uintptr_t)d.grad) | ((uintptr_t)d.m1) |
                     ((uintptr_t)d.m2)) & 15) == 0;
  const long long ev = vec ? e0 + ((e1 - e0) & ~3LL) : e0;   // end of the 16-byte part
  for (long long e = e0 + 4 * threadIdx.x; e < ev; e += 4 * 256) {
    float4 p = *(const float4*)(d.param + e);
    const float4 g = *(const float4*)(d.grad + e);
    float4 a = *(const float4*)(d.m1 + e);
    float4 v = *(const float4*)(d.m2 + e);
    adamw_elem(p.x, g.x, a.x, v.x, w1, w2, eps, decay, alpha);
    adamw_elem(p.y, g.y, a.y, v.y, w1, w2, eps, decay, alpha);
    adamw_elem(p.z, g.z, a.z, v.z, w1, w2, eps, decay, alpha);
    adamw_elem(p.w, g.w, a.w, v.w, w1, w2, eps, decay, alpha);
    *(float4*)(d.param + e) = p;
    *(float4*)(d.m1 + e) = a;
    *(float4*)(d.m2 + e) = v;
  }
  for (long long e = ev + threadIdx.x; e < e1; e += 256) {
    float p = d.param[e], a = d.m1[e], v = d.m2[e];
    adamw_elem(p, d.grad[e], a, v, w1, w2, eps, decay, alpha);
    d.param[e] = p;
    d.m1[e] = a;
    d.m2[e] = v;
  }
}

}  // namespace dmh

using namespace dmh;

extern "C" {

static_assert(sizeof(AdamwParam) == 40, "dmh_adamw_param layout");

int dmh_adamw_chunks(long long numel) {
  return numel <= 0 ? 0 : (int)((numel + ADAMW_CHUNK - 1) / ADAMW_CHUNK);
}

int dmh_adamw_step(hipStream_t stream, const void* table, int count, const int* chunk_start,
                   int nchunks, float w1, float w2, float eps, float decay, float alpha) {
  if (count == 0 || nchunks == 0) return DMH_OK;
  if (count < 0 || nchunks < 0 || !table || !chunk_start) {
    set_error("dmh_adamw_step: bad arguments (count=%d nchunks=%d)", count, nchunks);
    return DMH_EINVAL;
  }
  hipLaunchKernelGGL(adamw_step, dim3(nchunks), dim3(256), 0, stream, (const AdamwParam*)table,
                     count, chunk_start, w1, w2, eps, decay, alpha);
  DMH_CHECK_LAUNCH("adamw_step");
  return DMH_OK;
}

// layout of the descriptor the C header declares (dmh_glue_param)
static_assert(sizeof(GlueParam) == 56, "dmh_glue_param layout");

int dmh_momentum_stack(hipStream_t stream, const void* params, int count, float momentum,
                       int nesterov, float* stack) {
  const GlueParam* ps = (const GlueParam*)params;
  if (int rc = check_params("dmh_momentum_stack", ps, count, 0)) return rc;
  if (count == 0) return DMH_OK;
  if (!stack) {
    set_error("dmh_momentum_stack: null stack");
    return DMH_EINVAL;
  }
  return glue_launch(stream, ps, count, momentum, nesterov != 0, stack, nullptr, 0,
                     "momentum_stack");
}

int dmh_apply_update(hipStream_t stream, const void* params, int count, const void* ustack) {
  const GlueParam* ps = (const GlueParam*)params;
  if (int rc = check_params("dmh_apply_update", ps, count, 1)) return rc;
  if (count == 0) return DMH_OK;
  if (!ustack) {
    set_error("dmh_apply_update: null update stack");
    return DMH_EINVAL;
  }
  return glue_launch(stream, ps, count, 0.f, 0, nullptr, (const bf16*)ustack, 1,
                     "apply_update");
}

}  // extern "C"
