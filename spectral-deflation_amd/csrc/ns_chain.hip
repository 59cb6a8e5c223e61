// Grouped bf16 Newton-Schulz / Polar Express chain on CDNA4 MFMA.
//
// Replaces the torch.compile'd GEMM chains of
//   zeropower_via_newtonschulz5   defmuon/optim/muon.py:16-44
//   PolarExpress                  defmuon/optim/polar_express.py:21-34
//   _horner_iterate               defmuon/optim/deflation_batched.py:196-211
// for a batch of same-shape matrices in one launch per GEMM phase.
//
// Layout.  Every matrix of the batch is held twice in a zero-padded workspace,
// as W (m x n, the wide convention, m <= n) and as T = W^T (n x m), both bf16
// row-major with m, n rounded up to the 256 tile.  One iteration (a, b, c) is
//
//   K1  A  = W W^T                  (m x m, K = n)  symmetric: upper tiles only
//   K2  B' = b A + c A A + a I      (m x m, K = m)  symmetric: upper tiles only
//   K3  T' = T B' ; W' = T'^T       (n x m, K = m)
//
// so every product is an "NT" GEMM C[i][j] = sum_k P[i][k] Q[j][k] whose two
// operands are both K-contiguous, which is the layout the MFMA operand
// registers want (A and B' symmetric make A A and T B' NT products).  Zero
// padding is a fixed point of every phase (a I is added on the m true diagonal
// entries only), so no kernel needs bounds checks on its loads.
//
// Rounding.  A is stored bf16; B' = bf16(b*A + bf16(c*AA) + a*I); T' = bf16(T B')
// with fp32 accumulation.  The reference's compiled graph rounds c*A to bf16
// before the product and forms bf16(a*T + bf16(T B)); this kernel scales the fp32
// accumulator by c instead (keeps A*A symmetric, so K2 skips half its tiles) and
// folds a*T into the product through the diagonal of B' (a T + T B = T (B + a I)),
// which removes K3's read of T and the rounding of T B, a term several times
// larger than T' itself.
#include "common.h"
#include "ns_chain.h"

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

namespace dmh {

static thread_local char g_err[512];

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

// ---------------------------------------------------------------------------
// MFMA GEMM tile: 256 x 256 output per workgroup, 8 waves (two per SIMD) of
// 128 x 64, K stages of 64 in a 2-slot LDS ring (one stage of loads in flight
// while the other is consumed), one workgroup barrier per stage.
//
// Operand tiles go global -> LDS with the gfx950 direct-to-LDS load
// (buffer_load_dwordx4 ... lds: lane L of a wave writes 16 bytes at base + 16 L,
// no VGPR round trip).  An LDS row is 64 bf16 = 128 B = 8 chunks of 16 B; chunk c
// of row r sits in slot c ^ swz(r), so the 16-byte fragment reads hit distinct
// banks.  The swizzle is applied by choosing, for each lane, which global chunk it
// fetches into its fixed LDS slot.
// ---------------------------------------------------------------------------
constexpr int TILE = CHAIN_TILE;
constexpr int TK = 64;
constexpr int NSTAGE = 2;
constexpr int KSUB = TK / 16;                // k16 MFMA substeps per stage
constexpr int CHUNKS = TK / 8;               // 16-byte chunks per LDS row
constexpr int ROWB = TK * 2;                 // bytes per LDS row
constexpr int OPB = TILE * ROWB;             // bytes per operand tile (32 KB)
constexpr int STAGEB = 2 * OPB;              // P + Q
static_assert(KSUB == 4 && CHUNKS == 8, "the main loop is written for 64-wide K stages");
// 8 waves, two per SIMD (so one wave's MFMAs fill the other's waits), as a
// 2 x 4 grid of 128 x 64 wave tiles: 4 x 2 MFMA blocks of 32 x 32 per wave.
constexpr int GEMM_WAVES = 8;
constexpr int GEMM_THREADS = 64 * GEMM_WAVES;
constexpr int WAVES_N = 4;                      // waves along the Q rows (output columns)
constexpr int WT_M = TILE / (GEMM_WAVES / WAVES_N), WT_N = TILE / WAVES_N;
constexpr int BM = WT_M / 32, BN = WT_N / 32;   // MFMA blocks per wave
constexpr int LROWS = 64 / CHUNKS;                // tile rows per load instruction
constexpr int LQ = TILE / GEMM_WAVES / LROWS;   // loads per operand per stage per lane
constexpr int RING_BYTES = NSTAGE * STAGEB > 128 * 1024 ? NSTAGE * STAGEB : 128 * 1024;
static_assert(RING_BYTES <= 160 * 1024, "LDS ring and epilogue tile must fit the 160 KB of a CU");
// loads of the stages younger than the one waited for (8 per stage per wave)
constexpr int RING_VMCNT = 2 * LQ * (NSTAGE - 2);

enum { EPI_STORE = 0, EPI_POLY = 1 };

struct GemmArgs {
  const bf16* P; long long p_bs; int p_ld;      // rows i of C
  const bf16* Q; long long q_bs; int q_ld;      // rows j of C
  int K;                                         // multiple of TK
  int tiles_m, tiles_n;                          // tiles per matrix
  int sym;                                       // upper-triangular tiles, mirrored stores
  float alpha, beta;                             // POLY: (b, c)
  float diag_add; int diag_lim;                  // POLY: + diag_add on C[i][i], i < diag_lim
  const bf16* aux; long long aux_bs; int aux_ld; // POLY: A (indexed [i][j])
  bf16* out; long long out_bs; int out_ld;       // C[i][j]   (may be null)
  bf16* outT; long long outT_bs; int outT_ld;    // C[j][i]   (may be null)
  int valid_i, valid_j;                          // stores limited to i < valid_i, j < valid_j
};

__device__ __forceinline__ void decode_tile(const GemmArgs& g, int lid, int& b, int& ti, int& tj) {
  if (g.sym) {
    const int T = g.tiles_m;
    const int per = T * (T + 1) / 2;
    b = lid / per;
    int rem = lid - b * per;
    ti = 0;
    while (rem >= T - ti) { rem -= T - ti; ++ti; }
    tj = ti + rem;
  } else {
    const int per = g.tiles_m * g.tiles_n;
    b = lid / per;
    const int t = lid - b * per;
    ti = t / g.tiles_n;
    tj = t - ti * g.tiles_n;
  }
}

// 16-byte slot of chunk c in LDS row r is c ^ lds_swz(r): the fragment reads of 8
// consecutive rows (and of 16, on two 128-byte halves) hit distinct banks.
__device__ __forceinline__ int lds_swz(int r) { return (r ^ (r >> 3)) & (CHUNKS - 1); }

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Workgroup barrier for the LDS ring.  Every wave has already waited (vmcnt) for
// its own direct-to-LDS loads of the stage about to be read, and its fragment
// reads of the stage about to be refilled have been consumed by its MFMAs, so the
// barrier needs no memory fence: __syncthreads() would make the compiler drain
// all outstanding loads (vmcnt(0)), i.e. the whole prefetch ring, at every step.
// The empty asm statements keep the compiler from moving LDS accesses across it.
__device__ __forceinline__ void ring_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <int EPI>
__global__ __attribute__((amdgpu_flat_work_group_size(GEMM_THREADS, GEMM_THREADS),
                          amdgpu_waves_per_eu(GEMM_WAVES / 4, GEMM_WAVES / 4)))
void gemm_nt_bf16(GemmArgs g) {
  __shared__ __attribute__((aligned(1024))) char smem[RING_BYTES];

  const int lid = xcd_remap(blockIdx.x, gridDim.x);
  int b, ti, tj;
  decode_tile(g, lid, b, ti, tj);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform (SGPR)
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;

  const bf16* P = g.P + (long long)b * g.p_bs + (long long)(ti * TILE) * g.p_ld;
  const bf16* Q = g.Q + (long long)b * g.q_bs + (long long)(tj * TILE) * g.q_ld;

  // Loader: buffer loads straight into LDS (buffer_load_dwordx4 ... lds).  Wave w,
  // instruction q covers tile rows (TILE/GEMM_WAVES) w + LROWS q .. +LROWS-1; lane L
  // fills slot L % CHUNKS of row (TILE/GEMM_WAVES) w + LROWS q + L / CHUNKS with the
  // global chunk slot ^ swz(row).  The per-lane byte
  // offsets are fixed for the whole K loop, the K step goes into the scalar offset
  // and the LDS destination (M0) is wave-uniform, so a load costs no VALU work.
  const __amdgpu_buffer_rsrc_t rP =
      __builtin_amdgcn_make_buffer_rsrc((void*)P, (short)0, TILE * g.p_ld * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t rQ =
      __builtin_amdgcn_make_buffer_rsrc((void*)Q, (short)0, TILE * g.q_ld * 2, 0x00020000);
  const int lrow0 = (TILE / GEMM_WAVES) * wave + lane / CHUNKS;
  const int lslot = lane % CHUNKS;
  int boffP[LQ], boffQ[LQ];   // byte offsets within the tile
#pragma unroll
  for (int q = 0; q < LQ; ++q) {
    const int r = lrow0 + LROWS * q;
    const int c = lslot ^ lds_swz(r);
    boffP[q] = (r * g.p_ld + c * 8) * 2;
    boffQ[q] = (r * g.q_ld + c * 8) * 2;
  }
  char* const lds_wave = smem + wave * (TILE / GEMM_WAVES) * ROWB;   // this wave's first row

#define DMH_GLOAD(k0, st)                                                              \
  do {                                                                                 \
    char* dP = lds_wave + (st) * STAGEB;                                               \
    char* dQ = dP + OPB;                                                               \
    const int so = (k0) * 2;                                                           \
    _Pragma("unroll") for (int q = 0; q < LQ; ++q) {                                   \
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rP, (lds_ptr_t)(dP + q * LROWS * ROWB), 16, \
                                               boffP[q], so, 0, 0);                    \
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rQ, (lds_ptr_t)(dQ + q * LROWS * ROWB), 16, \
                                               boffQ[q], so, 0, 0);                    \
    }                                                                                  \
  } while (0)

  f32x16 acc[BM][BN];
#pragma unroll
  for (int i = 0; i < BM; ++i)
#pragma unroll
    for (int j = 0; j < BN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  const int r32 = lane & 31;
  const int hi = lane >> 5;
  // byte offsets of this lane's fragments: row 32 i + r32 of the wave's P rows (and
  // 32 j + r32 of its Q rows), 16-byte chunk 2 s + hi for k16 substep s
  int offP[BM][KSUB], offQ[BN][KSUB];
#pragma unroll
  for (int i = 0; i < BM; ++i) {
    const int row = WT_M * wm + 32 * i + r32;
#pragma unroll
    for (int st = 0; st < KSUB; ++st) offP[i][st] = row * ROWB + ((2 * st + hi) ^ lds_swz(row)) * 16;
  }
#pragma unroll
  for (int j = 0; j < BN; ++j) {
    const int row = WT_N * wn + 32 * j + r32;
#pragma unroll
    for (int st = 0; st < KSUB; ++st)
      offQ[j][st] = OPB + row * ROWB + ((2 * st + hi) ^ lds_swz(row)) * 16;
  }

  // Main loop, software-pipelined at two levels:
  //  * LDS ring: stages kt+1..kt+NSTAGE-1 are in flight while stage kt is consumed.
  //    The prefetch is unconditional: past the last stage it re-fetches the last
  //    stage into the free slot (never read), so every step waits on the same
  //    vmcnt and the loop body has no branches.
  //  * fragments: substep s+1 is read from LDS under the MFMAs of substep s, and
  //    substep 0 of stage kt+1 under the last substep of stage kt, so the MFMA pipe
  //    never waits on LDS; the one barrier per stage sits before the last substep.
  // The slot refilled at step kt (stage kt+NSTAGE-1) held stage kt-1, whose last
  // fragment reads completed (lgkmcnt(0)) before the barrier of step kt-1.
  const int nk = g.K / TK;
#pragma unroll
  for (int p = 0; p < NSTAGE - 1; ++p) DMH_GLOAD(min(p, nk - 1) * TK, p);
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(RING_VMCNT) : "memory");   // stage 0 landed (own loads)
  ring_barrier();                                       // ... and everyone's

#define DMH_RD(F, base, st)                                                            \
  do {                                                                                 \
    _Pragma("unroll") for (int i = 0; i < BM; ++i)                                     \
      F##p[i] = *(const bf16x8*)((base) + offP[i][st]);                                \
    _Pragma("unroll") for (int j = 0; j < BN; ++j)                                     \
      F##q[j] = *(const bf16x8*)((base) + offQ[j][st]);                                \
  } while (0)
#define DMH_MM(F)                                                                      \
  do {                                                                                 \
    _Pragma("unroll") for (int i = 0; i < BM; ++i)                                     \
      _Pragma("unroll") for (int j = 0; j < BN; ++j)                                   \
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(F##q[j], F##p[i], acc[i][j], 0, 0, 0); \
  } while (0)
  // MFMAs of one substep with the next substep's fragment reads among them
#define DMH_SCHED_SUB()                                                                \
  do {                                                                                 \
    _Pragma("unroll") for (int x = 0; x < BM + BN; ++x) {                              \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                               \
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                               \
    }                                                                                  \
    __builtin_amdgcn_sched_group_barrier(0x008, BM * BN - (BM + BN), 0);               \
  } while (0)

  bf16x8 f0p[BM], f0q[BN], f1p[BM], f1q[BN];
  DMH_RD(f0, smem, 0);
  int s_cur = 0;   // ring slot of stage kt
  for (int kt = 0; kt < nk; ++kt) {
    const int s_nxt = s_cur + 1 == NSTAGE ? 0 : s_cur + 1;
    const int s_pre = s_cur == 0 ? NSTAGE - 1 : s_cur - 1;   // slot of stage kt + NSTAGE - 1
    const char* cur = smem + s_cur * STAGEB;
    const char* nxt = smem + s_nxt * STAGEB;
    DMH_GLOAD(min(kt + NSTAGE - 1, nk - 1) * TK, s_pre);
    DMH_RD(f1, cur, 1);
    DMH_MM(f0);
    DMH_RD(f0, cur, 2);
    DMH_MM(f1);
    DMH_RD(f1, cur, 3);
    DMH_MM(f0);
    // prefetch loads first, then substeps 0..2 with the reads of 1..3 among them
    __builtin_amdgcn_sched_group_barrier(0x020, 2 * LQ, 0);   // VMEM (direct-to-LDS)
    DMH_SCHED_SUB();
    DMH_SCHED_SUB();
    DMH_SCHED_SUB();
    // stage kt+1 landed: the younger loads in flight are those of stages
    // kt+2 .. kt+NSTAGE-1, and loads retire in issue order
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(RING_VMCNT) : "memory");
    ring_barrier();
    DMH_RD(f0, nxt, 0);
    DMH_MM(f1);
    DMH_SCHED_SUB();
    s_cur = s_nxt;
  }
#undef DMH_RD
#undef DMH_MM
#undef DMH_SCHED_SUB
#undef DMH_GLOAD
  // the re-fetches past the last stage may still be landing in LDS
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // ---- epilogue -------------------------------------------------------------
  // The 256x256 output tile is staged through LDS as bf16 (the whole 128 KB),
  // so both output layouts leave in 16-byte coalesced stores.
  //   phase 1  acc -> LDS: v = bf16(acc) (bf16(c * acc) for POLY)
  //   phase 2  row-major pass: POLY epilogue (aux read in 16 B), store C[i][j]
  //   phase 3  transposed pass: 8 rows x 4 columns per step, transposed in
  //            registers, store C^T[j][i]
  // LDS element (i, j) of the tile sits at byte i*512 + 16*((j>>3) ^ swz(i)) + 2*(j&7);
  // swz(i) = ((i>>3)&3) | ((((i&7) ^ (i>>5)) & 7) << 2) keeps 32 consecutive rows (phase
  // 1) and rows 8 apart (phase 3) on distinct 16-byte slots.
  // acc[i][j][4g+q] holds C[i0 + (lane&31)][j0 + 8g + 4(lane>>5) + q].
  // The barriers below only order LDS (lgkmcnt), so the aux tile, fetched in one
  // batch up front, stays in flight while the accumulators drain.
  const int gi0 = ti * TILE, gj0 = tj * TILE;
  constexpr int NU = TILE * TILE / 8 / GEMM_THREADS;   // 16-byte chunks per thread
  bf16x8 av[NU];
  if (EPI == EPI_POLY) {
    const bf16* auxb = g.aux + (long long)b * g.aux_bs + (long long)gi0 * g.aux_ld + gj0;
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int e = tid + GEMM_THREADS * u;
      av[u] = *(const bf16x8*)(auxb + (long long)(e >> 5) * g.aux_ld + (e & 31) * 8);
    }
  }
  ring_barrier();
  char* const cs = smem;
  auto cswz = [](int i) { return ((i >> 3) & 3) | ((((i & 7) ^ (i >> 5)) & 7) << 2); };
  auto caddr = [&](int i, int j) { return i * 512 + 16 * ((j >> 3) ^ cswz(i)) + 2 * (j & 7); };
#pragma unroll
  for (int bi = 0; bi < BM; ++bi) {
    const int il = WT_M * wm + 32 * bi + r32;
#pragma unroll
    for (int bj = 0; bj < BN; ++bj) {
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const int jl = WT_N * wn + 32 * bj + 8 * gq + 4 * (lane >> 5);
        bf16x4 o;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float v = acc[bi][bj][4 * gq + q];
          o[q] = f2bf(EPI == EPI_POLY ? g.beta * v : v);
        }
        *(bf16x4*)(cs + caddr(il, jl)) = o;
      }
    }
  }
  ring_barrier();
  const bool diag = g.sym && ti == tj;
  if (diag) {
    // exact symmetry: the lower triangle of a diagonal tile takes the upper one's
    // values.  8x8 blocks (I, J), I >= J: block (J, I) is read as 8 rows of 16 B,
    // transposed in registers and written over block (I, J); on the diagonal
    // blocks only the strictly lower elements are replaced.  Reads and writes of
    // one thread touch blocks no other thread writes.
    for (int blk = tid; blk < 32 * 33 / 2; blk += GEMM_THREADS) {
      int I = (int)((sqrtf(8.f * blk + 1.f) - 1.f) * 0.5f);
      while ((I + 1) * (I + 2) / 2 <= blk) ++I;
      while (I * (I + 1) / 2 > blk) --I;
      const int J = blk - I * (I + 1) / 2;
      bf16x8 src[8];
#pragma unroll
      for (int r = 0; r < 8; ++r) src[r] = *(const bf16x8*)(cs + caddr(8 * J + r, 8 * I));
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        bf16x8 d;
#pragma unroll
        for (int r = 0; r < 8; ++r) d[r] = src[r][c];
        if (I == J) {
#pragma unroll
          for (int r = 0; r < 8; ++r)
            if (r >= c) d[r] = src[c][r];
        }
        *(bf16x8*)(cs + caddr(8 * I + c, 8 * J)) = d;
      }
    }
    ring_barrier();
  }
  const bool need_t = g.outT && (!g.sym || !diag);
  bf16* outb = g.out ? g.out + (long long)b * g.out_bs : nullptr;
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int e = tid + GEMM_THREADS * u;
    const int il = e >> 5, jc = (e & 31) * 8;
    char* lp = cs + il * 512 + 16 * ((jc >> 3) ^ cswz(il));
    bf16x8 v = *(const bf16x8*)lp;
    const int gi = gi0 + il, gj = gj0 + jc;
    if (EPI == EPI_POLY) {
      const int qd = diag && gi < g.diag_lim ? il - jc : -1;   // the diagonal's slot, if here
#pragma unroll
      for (int q = 0; q < 8; ++q)
        v[q] = f2bf(g.alpha * bf2f(av[u][q]) + bf2f(v[q]) + (q == qd ? g.diag_add : 0.f));
      if (need_t) *(bf16x8*)lp = v;
    }
    if (outb && gi < g.valid_i) {
      bf16* op = outb + (long long)gi * g.out_ld + gj;
      if (gj + 7 < g.valid_j && (g.out_ld & 7) == 0) {
        *(bf16x8*)op = v;
      } else {
#pragma unroll
        for (int q = 0; q < 8; ++q)
          if (gj + q < g.valid_j) op[q] = v[q];
      }
    }
  }
  if (!need_t) return;
  ring_barrier();
  bf16* outtb = g.outT + (long long)b * g.outT_bs;
  for (int u = 0; u < TILE * TILE / 32 / GEMM_THREADS; ++u) {
    const int e = tid + GEMM_THREADS * u;
    const int ic = (e & 31) * 8, jg = (e >> 5) * 4;   // rows ic..ic+7, columns jg..jg+3
    uint2 r[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) r[q] = *(const uint2*)(cs + caddr(ic + q, jg));
    const int gi = gi0 + ic;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int gj = gj0 + jg + c;
      // column c of the 8x4 block: halves (c&1) of words (c>>1)
      uint32_t w[4];
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const uint32_t x0 = (c >> 1) ? r[2 * h].y : r[2 * h].x;
        const uint32_t x1 = (c >> 1) ? r[2 * h + 1].y : r[2 * h + 1].x;
        const uint32_t lo = (c & 1) ? (x0 >> 16) : (x0 & 0xffffu);
        const uint32_t hi = (c & 1) ? (x1 & 0xffff0000u) : (x1 << 16);
        w[h] = lo | hi;
      }
      if (gj >= g.valid_j) continue;
      bf16* tp = outtb + (long long)gj * g.outT_ld + gi;
      if (gi + 7 < g.valid_i && (g.outT_ld & 7) == 0) {
        *(uint4*)tp = make_uint4(w[0], w[1], w[2], w[3]);
      } else {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          if (gi + q < g.valid_i) {
            const uint16_t bits = (uint16_t)((w[q >> 1] >> (16 * (q & 1))) & 0xffffu);
            tp[q] = __builtin_bit_cast(bf16, bits);
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// entry: Frobenius norm partials, then scale + cast + pack into padded T and W
// ---------------------------------------------------------------------------
constexpr int NORM_CHUNKS = 64;

struct InView {
  const void* x; int dtype;            // 0 fp32, 1 bf16
  long long bs, rs, cs;                // element strides
  int rows, cols;
};

__device__ __forceinline__ float load_in(const InView& v, int b, int r, int c) {
  const long long off = (long long)b * v.bs + (long long)r * v.rs + (long long)c * v.cs;
  if (v.dtype == 0) return ((const float*)v.x)[off];
  return bf2f(((const bf16*)v.x)[off]);
}

__global__ __launch_bounds__(256) void entry_norm_partials(InView v, double* partials) {
  const int b = blockIdx.y, chunk = blockIdx.x;
  const long long total = (long long)v.rows * v.cols;
  const long long per = (total + NORM_CHUNKS - 1) / NORM_CHUNKS;
  const long long lo = chunk * per;
  const long long hi = lo + per < total ? lo + per : total;
  double s = 0.0;
  for (long long e = lo + threadIdx.x; e < hi; e += blockDim.x) {
    const int r = (int)(e / v.cols), c = (int)(e - (long long)r * v.cols);
    const float x = load_in(v, b, r, c);
    s += (double)x * (double)x;
  }
  __shared__ double red[256];
  red[threadIdx.x] = s;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) partials[b * NORM_CHUNKS + chunk] = red[0];
}

// Pack 64x64 tiles of T-space (i < np rows, j < mp cols).  in_tall: the input is
// T (rows = n); otherwise it is W (rows = m) and is transposed on the way.
// scale_mode: 0 none, 1: 1/(||x||+1e-7), 2: 1/(1.01||x||+1e-7).
__global__ __launch_bounds__(256) void entry_pack(InView v, int in_tall, int scale_mode,
                                                  const double* partials, int n, int m,
                                                  int np, int mp, bf16* T, bf16* W) {
  __shared__ float tile[64][65];
  const int b = blockIdx.z;
  const int i0 = blockIdx.y * 64, j0 = blockIdx.x * 64;
  float scale = 1.f;
  if (scale_mode) {
    __shared__ float s_scale;
    if (threadIdx.x == 0) {
      double s = 0.0;
      for (int c = 0; c < NORM_CHUNKS; ++c) s += partials[b * NORM_CHUNKS + c];
      const float nrm = (float)sqrt(s);
      const float den = scale_mode == 2 ? nrm * 1.01f + 1e-7f : nrm + 1e-7f;
      s_scale = den;
    }
    __syncthreads();
    scale = s_scale;
  }
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  // load in the input's natural orientation (coalesced along its columns)
  for (int rr = ty; rr < 64; rr += 4) {
    float x = 0.f;
    if (in_tall) {
      const int i = i0 + rr, j = j0 + tx;
      if (i < n && j < m) x = load_in(v, b, i, j);
      tile[rr][tx] = x;
    } else {
      const int j = j0 + rr, i = i0 + tx;   // W[j][i]
      if (i < n && j < m) x = load_in(v, b, j, i);
      tile[tx][rr] = x;
    }
  }
  __syncthreads();
  bf16* Tb = T + (long long)b * np * mp;
  bf16* Wb = W + (long long)b * mp * np;
  for (int rr = ty; rr < 64; rr += 4) {
    const float xt = scale_mode ? tile[rr][tx] / scale : tile[rr][tx];
    Tb[(long long)(i0 + rr) * mp + j0 + tx] = f2bf(xt);
    const float xw = scale_mode ? tile[tx][rr] / scale : tile[tx][rr];
    Wb[(long long)(j0 + rr) * np + i0 + tx] = f2bf(xw);
  }
}

// steps == 0: copy the packed entry out in the input's orientation
__global__ __launch_bounds__(256) void copy_out(const bf16* T, int np, int mp, int n, int m,
                                                int out_tall, bf16* out) {
  const int b = blockIdx.y;
  const long long total = (long long)n * m;
  for (long long e = blockIdx.x * 256LL + threadIdx.x; e < total; e += 256LL * gridDim.x) {
    int i, j;
    if (out_tall) { i = (int)(e / m); j = (int)(e - (long long)i * m); }
    else { j = (int)(e / n); i = (int)(e - (long long)j * n); }
    out[(long long)b * total + e] = T[(long long)b * np * mp + (long long)i * mp + j];
  }
}

ChainDims chain_dims(int rows, int cols, int orient_tall) {
  ChainDims d;
  d.n = orient_tall ? rows : cols;
  d.m = orient_tall ? cols : rows;
  d.np = ceil_div(d.n, TILE) * TILE;
  d.mp = ceil_div(d.m, TILE) * TILE;
  return d;
}

ChainWs chain_ws(void* ws, int batch, const ChainDims& d) {
  ChainWs w{};
  const size_t tw = (size_t)batch * d.np * d.mp;
  const size_t sq = (size_t)batch * d.mp * d.mp;
  const size_t part = (size_t)batch * NORM_CHUNKS * sizeof(double);
  w.bytes = (4 * tw + 2 * sq) * sizeof(bf16) + ((part + 255) / 256) * 256;
  if (!ws) return w;
  w.T0 = (bf16*)ws;
  w.W0 = w.T0 + tw;
  w.T1 = w.W0 + tw;
  w.W1 = w.T1 + tw;
  w.A = w.W1 + tw;
  w.B = w.A + sq;
  w.partials = (double*)(w.B + sq);
  return w;
}

template <int EPI>
static int launch_gemm(const GemmArgs& g, int batch, hipStream_t stream, const char* what) {
  const int per = g.sym ? g.tiles_m * (g.tiles_m + 1) / 2 : g.tiles_m * g.tiles_n;
  const long long blocks = (long long)per * batch;
  if (blocks <= 0 || blocks > 0x7fffffffLL) {
    set_error("%s: bad grid (%lld blocks)", what, blocks);
    return DMH_EINVAL;
  }
  hipLaunchKernelGGL(gemm_nt_bf16<EPI>, dim3((unsigned)blocks), dim3(GEMM_THREADS), 0, stream, g);
  DMH_CHECK_LAUNCH(what);
  return DMH_OK;
}

int chain_run_packed(hipStream_t stream, const ChainWs& w, int batch, const ChainDims& d,
                     int orient_tall, const double* coeffs, int steps, bf16* outp) {
  if (steps == 0) {
    const long long total = (long long)d.n * d.m;
    const int blocks = (int)std::min<long long>((total + 255) / 256, 4096);
    hipLaunchKernelGGL(copy_out, dim3(blocks, batch), dim3(256), 0, stream, w.T0, d.np, d.mp,
                       d.n, d.m, orient_tall, outp);
    DMH_CHECK_LAUNCH("copy_out");
    return DMH_OK;
  }
  const int tm = d.mp / TILE, tn = d.np / TILE;
  bf16 *Tc = w.T0, *Wc = w.W0, *Tn = w.T1, *Wn = w.W1;
  bf16 *Am = w.A, *Bm = w.B;
  for (int it = 0; it < steps; ++it) {
    const float a = (float)coeffs[3 * it + 0];
    const float bcoef = (float)coeffs[3 * it + 1];
    const float c = (float)coeffs[3 * it + 2];
    const bool last = it + 1 == steps;
    int rc;
    // K1: A = W W^T
    GemmArgs g1{};
    g1.P = Wc; g1.p_bs = (long long)d.mp * d.np; g1.p_ld = d.np;
    g1.Q = Wc; g1.q_bs = g1.p_bs; g1.q_ld = d.np;
    g1.K = d.np; g1.tiles_m = tm; g1.tiles_n = tm; g1.sym = 1;
    g1.out = Am; g1.out_bs = (long long)d.mp * d.mp; g1.out_ld = d.mp;
    g1.outT = Am; g1.outT_bs = g1.out_bs; g1.outT_ld = d.mp;
    g1.valid_i = d.mp; g1.valid_j = d.mp;
    if ((rc = launch_gemm<EPI_STORE>(g1, batch, stream, "ns K1 (W W^T)"))) return rc;
    // K2: B = b A + c A A
    GemmArgs g2 = g1;
    g2.P = Am; g2.p_bs = (long long)d.mp * d.mp; g2.p_ld = d.mp;
    g2.Q = Am; g2.q_bs = g2.p_bs; g2.q_ld = d.mp;
    g2.K = d.mp;
    g2.alpha = bcoef; g2.beta = c; g2.diag_add = a; g2.diag_lim = d.m;
    g2.aux = Am; g2.aux_bs = g2.p_bs; g2.aux_ld = d.mp;
    g2.out = Bm; g2.outT = Bm;
    if ((rc = launch_gemm<EPI_POLY>(g2, batch, stream, "ns K2 (bA + cA^2 + aI)"))) return rc;
    // K3: T' = T B'  (and W' = T'^T)
    GemmArgs g3{};
    g3.P = Tc; g3.p_bs = (long long)d.np * d.mp; g3.p_ld = d.mp;
    g3.Q = Bm; g3.q_bs = (long long)d.mp * d.mp; g3.q_ld = d.mp;
    g3.K = d.mp; g3.tiles_m = tn; g3.tiles_n = tm; g3.sym = 0;
    if (!last) {
      g3.out = Tn; g3.out_bs = g3.p_bs; g3.out_ld = d.mp;
      g3.outT = Wn; g3.outT_bs = (long long)d.mp * d.np; g3.outT_ld = d.np;
      g3.valid_i = d.np; g3.valid_j = d.mp;
    } else if (orient_tall) {
      g3.out = outp; g3.out_bs = (long long)d.n * d.m; g3.out_ld = d.m;
      g3.valid_i = d.n; g3.valid_j = d.m;
    } else {
      g3.outT = outp; g3.outT_bs = (long long)d.n * d.m; g3.outT_ld = d.n;
      g3.valid_i = d.n; g3.valid_j = d.m;
    }
    if ((rc = launch_gemm<EPI_STORE>(g3, batch, stream, "ns K3 (T B')"))) return rc;
    bf16* t = Tc; Tc = Tn; Tn = t;
    t = Wc; Wc = Wn; Wn = t;
  }
  return DMH_OK;
}

}  // namespace dmh

using namespace dmh;

extern "C" {

const char* dmh_last_error(void) { return g_err; }

int dmh_ns_workspace_size(int batch, int rows, int cols, int orient_tall, size_t* bytes) {
  if (batch < 0 || rows <= 0 || cols <= 0 || !bytes) {
    set_error("dmh_ns_workspace_size: bad arguments");
    return DMH_EINVAL;
  }
  *bytes = chain_ws(nullptr, batch, chain_dims(rows, cols, orient_tall)).bytes;
  return DMH_OK;
}

int dmh_ns_chain(hipStream_t stream, const void* x, int x_dtype, int batch, int rows, int cols,
                 long long x_bstride, long long x_rstride, long long x_cstride, void* out,
                 int orient_tall, int entry_mode, const double* coeffs, int steps, void* ws,
                 size_t ws_bytes) {
  if (batch == 0) return DMH_OK;
  if (!x || !out || batch < 0 || rows <= 0 || cols <= 0 || steps < 0 ||
      (steps > 0 && !coeffs) || (x_dtype != 0 && x_dtype != 1) || entry_mode < 0 ||
      entry_mode > 2) {
    set_error("dmh_ns_chain: bad arguments (batch=%d rows=%d cols=%d steps=%d dtype=%d mode=%d)",
              batch, rows, cols, steps, x_dtype, entry_mode);
    return DMH_EINVAL;
  }
  const ChainDims d = chain_dims(rows, cols, orient_tall);
  const ChainWs w = chain_ws(ws, batch, d);
  if (!ws || ws_bytes < w.bytes) {
    set_error("dmh_ns_chain: workspace %zu < %zu bytes", ws_bytes, w.bytes);
    return DMH_EWORKSPACE;
  }
  InView v{x, x_dtype, x_bstride, x_rstride, x_cstride, rows, cols};
  if (entry_mode) {
    hipLaunchKernelGGL(entry_norm_partials, dim3(NORM_CHUNKS, batch), dim3(256), 0, stream, v,
                       w.partials);
    DMH_CHECK_LAUNCH("entry_norm_partials");
  }
  hipLaunchKernelGGL(entry_pack, dim3(d.mp / 64, d.np / 64, batch), dim3(256), 0, stream, v,
                     orient_tall, entry_mode, w.partials, d.n, d.m, d.np, d.mp, w.T0, w.W0);
  DMH_CHECK_LAUNCH("entry_pack");
  return chain_run_packed(stream, w, batch, d, orient_tall, coeffs, steps, (bf16*)out);
}

}  // extern "C"
