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

// One workgroup per 64 x 64 tile of a tall block (grid-stride over the tiles of
// parameter blockIdx.y).  Without transpose both sides are row-contiguous; with it
// the tile goes through LDS so that the parameter side is read along its rows and
// the stack side written along its rows.
__global__ __launch_bounds__(256) void momentum_stack(GlueArgs a) {
  __shared__ float t[GT][GT + 1];
  const GlueParam& d = a.p[blockIdx.y];
  const BlockGeom g = geom(d);
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int tile = blockIdx.x; tile < g.tiles; tile += gridDim.x) {
    const int k = tile / (g.tn * g.tm);
    const int rem = tile - k * g.tn * g.tm;
    const int i0 = (rem / g.tm) * GT, j0 = (rem % g.tm) * GT;   // in the tall block
    float* dst = a.stack + d.offset + (long long)k * g.n * g.m;
    if (!d.transpose) {
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
  for (int tile = blockIdx.x; tile < g.tiles; tile += gridDim.x) {
    const int k = tile / (g.tn * g.tm);
    const int rem = tile - k * g.tn * g.tm;
    const int i0 = (rem / g.tm) * GT, j0 = (rem % g.tm) * GT;
    const bf16* src = a.ustack + d.offset + (long long)k * g.n * g.m;
    if (!d.transpose) {
      for (int ii = ty; ii < GT; ii += 4) {
        const int i = i0 + ii, j = j0 + tx;
        if (i >= g.n || j >= g.m) continue;
        const long long pi = (long long)(k * g.rb + i) * d.cols + j;
        const float pd = decayed(d.param[pi], d.decay);
        d.param[pi] = fmaf(d.alpha, bf2f(src[(long long)i * g.m + j]), pd);   // p.add_(u, alpha)
      }
    } else {
      __syncthreads();
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

}  // namespace dmh

using namespace dmh;

extern "C" {

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
