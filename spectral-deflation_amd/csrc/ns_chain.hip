// Grouped bf16 Newton-Schulz / Polar Express chain on CDNA4 MFMA.
//
// Replaces the torch.compile'd GEMM chains of
//   zeropower_via_newtonschulz5   defmuon/optim/muon.py:16-44
//   PolarExpress                  defmuon/optim/polar_express.py:21-34
//   _horner_iterate               defmuon/optim/deflation_batched.py:196-211
// for a batch of same-shape matrices in one launch per GEMM phase.
//
// Layout.  Every matrix of the batch is held as the tall iterate T (n x m, n >= m;
// W = T^T is the wide convention), bf16 in a zero-padded workspace with m, n
// rounded up to the 256 tile, stored in 64 x 64 blocks (blk_off in ns_chain.h) so
// that every K stage of the GEMMs reads contiguous memory.  One iteration (a, b, c) is
//
//   K1  A  = T^T T                  (m x m, K = n)  symmetric: upper tiles only
//   K2  B' = b A + c A A + a I      (m x m, K = m)  symmetric: upper tiles only
//   K3  T' = T B'                   (n x m, K = m)
//
// K2 and K3 are "NT" GEMMs C[i][j] = sum_k P[i][k] Q[j][k] whose two operands are
// K-contiguous rows (A and B' are symmetric), the layout the MFMA operand
// registers want.  K1 contracts over the rows of T: its operand tiles are loaded
// K-major and turned into MFMA fragments by the transposing LDS read of gfx950,
// so the iterate is never stored transposed.  Zero padding is a fixed point of
// every phase (a I is added on the m true diagonal entries only), so no kernel
// needs bounds checks on its loads.
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

#include <mutex>
#include <stdlib.h>
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
// MFMA GEMM: persistent workgroups (one per CU) over 256 x 256 output tiles, 8
// waves (two per SIMD) of 128 x 64, K stages of 64 in a 2-slot LDS ring (one
// stage of loads in flight while the other is consumed), one workgroup barrier
// per stage.
//
// Each workgroup walks a list of tiles.  While the MFMAs of a tile's last K stage
// run, the first stage of the workgroup's next tile is already loading into the
// free ring slot, and the epilogue goes through a small per-wave staging area
// outside the ring, so it needs no workgroup barrier and overlaps those loads;
// workgroup start-up and the first-stage load latency are paid once per CU, not
// once per tile.
//
// Operand tiles go global -> LDS with the gfx950 direct-to-LDS load
// (buffer_load_dwordx4 ... lds: lane L of a wave writes 16 bytes at base + 16 L,
// no VGPR round trip).  An LDS row is 64 bf16 = 128 B = 8 chunks of 16 B; chunk c
// of row r sits in slot c ^ swz(r), so the 16-byte fragment reads hit distinct
// banks.  The swizzle is applied by choosing, for each lane, which global chunk it
// fetches into its fixed LDS slot.
// ---------------------------------------------------------------------------
constexpr int TK = 64;
constexpr int NSTAGE = 2;
constexpr int KSUB = TK / 16;                // k16 MFMA substeps per stage
constexpr int CHUNKS = TK / 8;               // 16-byte chunks per LDS row
constexpr int ROWB = TK * 2;                 // bytes per LDS row
constexpr int LROWS = 64 / CHUNKS;           // tile rows per load instruction
static_assert(KSUB == 4 && CHUNKS == 8, "the main loop is written for 64-wide K stages");
static_assert(NSTAGE == 2, "the ring waits are written for two slots (vmcnt(0))");

// Output tile shapes.  TL = 256: 8 waves (two per SIMD, so one wave's MFMAs fill the
// other's waits) as a 2 x 4 grid of 128 x 64 wave tiles (4 x 2 MFMA blocks of 32 x 32
// per wave), one workgroup per CU.  TL = 128, for matrices too small to give every
// CU several 256 x 256 tiles: 4 waves as a 2 x 2 grid of 64 x 64 wave tiles (2 x 2
// blocks), 80 KB of LDS, two workgroups (again two waves per SIMD) per CU.
template <int TL>
struct GemmCfg {
  static constexpr int TILE = TL;
  static constexpr int WAVES = TL == 256 ? 8 : 4;
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int WAVES_N = TL == 256 ? 4 : 2;   // waves along the Q rows (output columns)
  static constexpr int WT_M = TILE / (WAVES / WAVES_N), WT_N = TILE / WAVES_N;
  static constexpr int BM = WT_M / 32, BN = WT_N / 32;   // MFMA blocks per wave
  static constexpr int OPB = TILE * ROWB;               // bytes per operand tile
  static constexpr int STAGEB = 2 * OPB;                // P + Q
  static constexpr int LQ = TILE / WAVES / LROWS;       // loads per operand per stage per lane
  static constexpr int KROWB = TILE * 2;                // bytes per K-major LDS row
  static constexpr int KCH = TILE / 8;                  // 16-byte chunks per K-major row
  static constexpr int RING_BYTES = NSTAGE * STAGEB;
  // epilogue staging: one 32 x 64 bf16 block row of the wave's output at a time
  static constexpr int EPI_WAVE_BYTES = 32 * WT_N * 2;
  static constexpr int SMEM_BYTES = RING_BYTES + WAVES * EPI_WAVE_BYTES;
  static constexpr int WG_PER_CU = (160 * 1024) / SMEM_BYTES;
  // vector memory instructions a wave's epilogue issues for a whole, aligned wave tile
  static constexpr int ROW_STORES = 4 * BM, T_STORES = 2 * BM * BN, AUX_LOADS = 4 * BM;
  static_assert(WT_N == 64, "the epilogue staging is written for 64-column wave tiles");
  static_assert(BM % 2 == 0, "the transposed epilogue pass takes block rows in pairs");
  static_assert(LQ == 4 && TK / WAVES * KROWB == LQ * 1024, "loader layout");
  static_assert(SMEM_BYTES <= 160 * 1024, "LDS ring and epilogue staging must fit 160 KB");
  static_assert(WAVES * WG_PER_CU == 8, "two waves per SIMD");
};

enum { EPI_STORE = 0, EPI_POLY = 1 };

// P, Q and aux are block-layout matrices (blk_off) of p_rows, q_rows, aux_rows rows;
// out / outT are block-layout when out_rows / outT_rows > 0, else row-major with
// their leading dimension (the caller's output).
struct GemmArgs {
  const bf16* P; long long p_bs; int p_rows;    // rows i of C
  const bf16* Q; long long q_bs; int q_rows;    // rows j of C
  int K;                                         // multiple of TK
  int tiles_m, tiles_n;                          // tiles per matrix
  int sym;                                       // upper-triangular tiles, mirrored stores
  int total_tiles;                               // over the batch
  int batch, rev;                                // rev: walk the batch from its last matrix
  int kspread;                                   // K walk starts at stage kspread (ti + tj) mod nk
  float alpha, beta;                             // POLY: (b, c)
  float diag_add; int diag_lim;                  // POLY: + diag_add on C[i][i], i < diag_lim
  const bf16* aux; long long aux_bs; int aux_rows; // POLY: A (indexed [i][j])
  bf16* out; long long out_bs; int out_ld, out_rows;      // C[i][j]   (may be null)
  bf16* outT; long long outT_bs; int outT_ld, outT_rows;  // C[j][i]   (may be null)
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
  if (g.rev) b = g.batch - 1 - b;
}

// Tiles of this workgroup: first, first + step, ... < end.  The dispatcher deals
// workgroups round-robin over the 8 XCDs, so workgroup w runs on XCD w % 8; the
// tile list is cut into 8 contiguous ranges, one per XCD, sized by the XCD's
// number of workgroups, and the workgroups of an XCD take its range round-robin.
// At any moment the CUs of one XCD work on consecutive tiles, whose operands
// share that XCD's L2.
__device__ __forceinline__ void tile_range(int total, int& first, int& step, int& end) {
  constexpr int NXCD = 8;
  const int G = gridDim.x, bid = blockIdx.x;
  const int x = bid % NXCD, s = bid / NXCD;
  const int q = G / NXCD, r = G % NXCD;
  const int cnt = q + (x < r ? 1 : 0);
  const int pre = x * q + (x < r ? x : r);
  first = (int)((long long)total * pre / G) + s;
  step = cnt;
  end = (int)((long long)total * (pre + cnt) / G);
}

// 16-byte slot of chunk c in LDS row r is c ^ lds_swz(r): the fragment reads of 8
// consecutive rows (and of 16, on two 128-byte halves) hit distinct banks.
__device__ __forceinline__ int lds_swz(int r) { return (r ^ (r >> 3)) & (CHUNKS - 1); }

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Workgroup barrier for the LDS ring.  Every wave has already waited (vmcnt) for
// its own direct-to-LDS loads of the stage about to be read, and its fragment
// reads of the stage about to be refilled have been consumed by its MFMAs, so the
// barrier needs no memory fence: __syncthreads() would make the compiler drain
// all outstanding loads (vmcnt(0)) at every step.
// The empty asm statements keep the compiler from moving LDS accesses across it.
__device__ __forceinline__ void ring_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Buffer descriptor of one operand tile of a block-layout matrix with R rows.
// Row-operand layout (TNL = 0): rows t*TILE..+TILE-1 of a K-contiguous matrix; the
// descriptor starts at their first K stage (4 consecutive blocks, 32 KB) and
// covers the later stages, R * 128 bytes apart.  K-major layout (TNL = 1): columns
// t*TILE..+TILE-1 of a matrix whose row k holds the operand's values for
// contraction index k (R = K rows): 4 whole block columns, R * 128 bytes each.
template <int TNL, int TILE>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const bf16* base, long long bs,
                                                           int R, int K, int b, int t) {
  if (TNL) {
    const bf16* p = base + (long long)b * bs + (long long)(t * TILE) * R;
    return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, TILE * R * 2, 0x00020000);
  }
  const bf16* p = base + (long long)b * bs + (long long)(t * TILE / CHAIN_BLK) * CHAIN_BLK * CHAIN_BLK;
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, (K / TK - 1) * R * ROWB + TILE * ROWB,
                                           0x00020000);
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4* lds_s16x4_t;

// MFMA operand fragment (8 consecutive k of one column) from a K-major LDS tile,
// with the gfx950 transposing LDS read (ds_read_b64_tr_b16): within each group of
// 16 lanes, result lane j, element e is element j % 4 of the 8-byte chunk addressed
// by lane 4 e + j / 4.  Lane 16 g + 4 e + q addresses row k0 + e, columns c0 + 4 q
// .. +3, so lane 16 g + j receives column c0 + j at rows k0 .. k0+3; the second read
// (rows k0+4 .. k0+7) is 4 rows (of krowb bytes) further.
__device__ __forceinline__ bf16x8 lds_tr_frag(const char* p, int krowb) {
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t)(p));
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t)(p + 4 * krowb));
  const bf16x4 l4 = __builtin_bit_cast(bf16x4, lo), h4 = __builtin_bit_cast(bf16x4, hi);
  return __builtin_shufflevector(l4, h4, 0, 1, 2, 3, 4, 5, 6, 7);
}

// The GEMM's builtins behind plain device functions: inside the kernel template their
// arguments have types that depend on the tile size, and the host pass of the
// compiler rejects a target builtin whose call it has to resolve at instantiation.
__device__ __forceinline__ void load_lds16(__amdgpu_buffer_rsrc_t r, char* lds, int voff,
                                           int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds, 16, voff, soff, 0, 0);
}
__device__ __forceinline__ f32x16 mfma_32x32x16(const bf16x8& a, const bf16x8& b,
                                                 const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Store 8 consecutive bf16 at dst (elements q with mask bit q set); a full, aligned
// chunk leaves as one 16-byte non-temporal store: the products are read back only by
// the next launch, so they should not evict the operand panels this launch's other
// tiles still read from L2.
__device__ __forceinline__ void store8(bf16* dst, const bf16x8& v, unsigned mask, bool aligned) {
  if (mask == 0xffu && aligned) {
    __builtin_nontemporal_store(v, (bf16x8*)dst);
  } else {
#pragma unroll
    for (int q = 0; q < 8; ++q)
      if (mask & (1u << q)) dst[q] = v[q];
  }
}

// TNL = 0: C[i][j] = sum_k P[i][k] Q[j][k] (both operands K-contiguous rows).
// TNL = 1: C[i][j] = sum_k P[k][i] Q[k][j] (both operands K-major: their row k holds
//          the values of every output index for contraction index k).
template <int EPI, int TNL, int TL>
__global__ __attribute__((amdgpu_flat_work_group_size(GemmCfg<TL>::THREADS, GemmCfg<TL>::THREADS),
                          amdgpu_waves_per_eu(2, 2)))
void gemm_nt_bf16(GemmArgs g) {
  using C = GemmCfg<TL>;
  constexpr int TILE = C::TILE, GEMM_WAVES = C::WAVES, WAVES_N = C::WAVES_N;
  constexpr int WT_M = C::WT_M, WT_N = C::WT_N, BM = C::BM, BN = C::BN;
  constexpr int OPB = C::OPB, STAGEB = C::STAGEB, LQ = C::LQ, KROWB = C::KROWB, KCH = C::KCH;
  constexpr int RING_BYTES = C::RING_BYTES, EPI_WAVE_BYTES = C::EPI_WAVE_BYTES;
  __shared__ __attribute__((aligned(1024))) char smem[C::SMEM_BYTES];

  int lid, lstep, lend;
  tile_range(g.total_tiles, lid, lstep, lend);
  if (lid >= lend) return;   // uniform over the workgroup

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform (SGPR)
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;

  // Loader: buffer loads straight into LDS (buffer_load_dwordx4 ... lds).  Wave w,
  // instruction q covers tile rows (TILE/GEMM_WAVES) w + LROWS q .. +LROWS-1; lane L
  // fills slot L % CHUNKS of row (TILE/GEMM_WAVES) w + LROWS q + L / CHUNKS with the
  // global chunk slot ^ swz(row).  The per-lane byte offsets are the same for every
  // tile and K step (the tile base is in the buffer descriptor, the K step in the
  // scalar offset) and the LDS destination (M0) is wave-uniform, so a load costs no
  // VALU work.
  //
  // K-major tiles (TNL) are 64 rows (k) of KROWB = 2 TILE bytes (KCH chunks of 16 B,
  // the TILE output indices); chunk c of row r sits in slot c ^ 4 (r & 3), which
  // spreads the transposing fragment reads (4 rows x 4 chunks per 16 lanes) over the
  // banks.  Instruction q of wave w fills the 1024 / KROWB rows starting at
  // (64 / GEMM_WAVES) w + (1024 / KROWB) q (1 KB), so the LDS destinations are the
  // same as for the row-operand tiles.
  // In global memory (block layout): a row-operand stage is 256 rows of 128 B, one
  // after the other, and the next stage is R * 128 bytes further; a K-major stage is
  // 64 rows of four 128-byte pieces, one per block column (R * 128 bytes apart), and
  // the next stage is the next 8 KB block of each column.
  int boffP[LQ], boffQ[LQ];   // byte offsets within the tile
  if (TNL) {
    constexpr int RPI = 1024 / KROWB;   // K-major rows per load instruction
#pragma unroll
    for (int q = 0; q < LQ; ++q) {
      const int r = (TK / GEMM_WAVES) * wave + RPI * q + lane / KCH;
      const int c = (lane % KCH) ^ (4 * (r & 3));
      boffP[q] = (c >> 3) * g.p_rows * ROWB + r * ROWB + (c & 7) * 16;
      boffQ[q] = (c >> 3) * g.q_rows * ROWB + r * ROWB + (c & 7) * 16;
    }
  } else {
    const int lrow0 = (TILE / GEMM_WAVES) * wave + lane / CHUNKS;
    const int lslot = lane % CHUNKS;
#pragma unroll
    for (int q = 0; q < LQ; ++q) {
      const int r = lrow0 + LROWS * q;
      const int c = lslot ^ lds_swz(r);
      boffP[q] = r * ROWB + c * 16;
      boffQ[q] = r * ROWB + c * 16;
    }
  }
  // scalar byte offset of K stage k0 (a multiple of 64): k0 / 64 block columns
  // further (row operands), or k0 rows down each block column (K-major)
  const int kstepP = TNL ? ROWB : g.p_rows * 2, kstepQ = TNL ? ROWB : g.q_rows * 2;
  char* const lds_wave = smem + wave * (TILE / GEMM_WAVES) * ROWB;   // this wave's first row

#define DMH_GLOAD(rp, rq, k0, st)                                                      \
  do {                                                                                 \
    char* dP = lds_wave + (st) * STAGEB;                                               \
    char* dQ = dP + OPB;                                                               \
    const int soP = (k0) * kstepP, soQ = (k0) * kstepQ;                                \
    _Pragma("unroll") for (int q = 0; q < LQ; ++q) {                                   \
      load_lds16(rp, dP + q * LROWS * ROWB, boffP[q], soP);                            \
      load_lds16(rq, dQ + q * LROWS * ROWB, boffQ[q], soQ);                            \
    }                                                                                  \
  } while (0)

  const int r32 = lane & 31;
  const int hi = lane >> 5;
  // byte offsets of this lane's fragments: row 32 i + r32 of the wave's P rows (and
  // 32 j + r32 of its Q rows), 16-byte chunk 2 s + hi for k16 substep s
  // (K-major tiles: first of the two transposing reads of column block c0, rows
  // 16 st + 8 (g >> 1) + e, with g = lane / 16, e = (lane / 4) % 4, q = lane % 4)
  int offP[BM][KSUB], offQ[BN][KSUB];
  auto frag_off = [&](int c0, int st) {
    if (TNL) {
      const int gq = lane >> 4, e = (lane >> 2) & 3, q = lane & 3;
      const int k = 16 * st + 8 * (gq >> 1) + e;
      const int c = c0 + 16 * (gq & 1) + 4 * q;
      return k * KROWB + (((c >> 3) ^ (4 * (k & 3))) * 16) + (c & 7) * 2;
    }
    const int row = c0 + r32;
    return row * ROWB + ((2 * st + hi) ^ lds_swz(row)) * 16;
  };
#pragma unroll
  for (int i = 0; i < BM; ++i)
#pragma unroll
    for (int st = 0; st < KSUB; ++st) offP[i][st] = frag_off(WT_M * wm + 32 * i, st);
#pragma unroll
  for (int j = 0; j < BN; ++j)
#pragma unroll
    for (int st = 0; st < KSUB; ++st) offQ[j][st] = OPB + frag_off(WT_N * wn + 32 * j, st);

#define DMH_RD(F, base, st)                                                            \
  do {                                                                                 \
    _Pragma("unroll") for (int i = 0; i < BM; ++i)                                     \
      F##p[i] = TNL ? lds_tr_frag((base) + offP[i][st], KROWB)                         \
                    : *(const bf16x8*)((base) + offP[i][st]);                          \
    _Pragma("unroll") for (int j = 0; j < BN; ++j)                                     \
      F##q[j] = TNL ? lds_tr_frag((base) + offQ[j][st], KROWB)                         \
                    : *(const bf16x8*)((base) + offQ[j][st]);                          \
  } while (0)
#define DMH_MM(F)                                                                      \
  do {                                                                                 \
    _Pragma("unroll") for (int i = 0; i < BM; ++i)                                     \
      _Pragma("unroll") for (int j = 0; j < BN; ++j)                                   \
        acc[i][j] = mfma_32x32x16(F##q[j], F##p[i], acc[i][j]);                       \
  } while (0)
  // MFMAs of one substep with the next substep's fragment reads among them
#define DMH_SCHED_SUB()                                                                \
  do {                                                                                 \
    _Pragma("unroll") for (int x = 0; x < BM + BN; ++x) {                              \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                               \
      __builtin_amdgcn_sched_group_barrier(0x100, TNL ? 2 : 1, 0);                     \
    }                                                                                  \
    if constexpr (BM * BN > BM + BN)                                                   \
      __builtin_amdgcn_sched_group_barrier(0x008, BM * BN - (BM + BN), 0);             \
  } while (0)

  const int nk = g.K / TK;
  int b, ti, tj;
  decode_tile(g, lid, b, ti, tj);
  __amdgpu_buffer_rsrc_t rP = tile_rsrc<TNL, TILE>(g.P, g.p_bs, g.p_rows, g.K, b, ti);
  __amdgpu_buffer_rsrc_t rQ = tile_rsrc<TNL, TILE>(g.Q, g.q_bs, g.q_rows, g.K, b, tj);
  // Each tile walks its K stages starting at stage kspread (ti + tj) % nk and
  // wrapping around: the tiles that share an operand panel (same ti, or same tj) are
  // then at different K stages at any moment, so each line of a shared panel is
  // fetched from memory by the first of them and found in L2 by the others a few
  // stages later, instead of all of them waiting on the same miss.  The best spread
  // differs by product (measured over 0..6: K1 1, K2 0, K3 2).  The offset depends
  // on the tile alone, so a matrix gets the same result whatever batch it is in.
  int kofs = (g.kspread * (ti + tj)) % nk;
  DMH_GLOAD(rP, rQ, kofs * TK, 0);

  char* const stg = smem + RING_BYTES + wave * EPI_WAVE_BYTES;   // this wave's staging
  f32x16 acc[BM][BN];
  bf16x8 f0p[BM], f0q[BN], f1p[BM], f1q[BN];
  int s_cur = 0;   // ring slot of the stage being consumed
  int vm_after = 0; // vector memory instructions issued after the prefetch of stage 0
  for (;;) {
    // the workgroup's next tile, if any (its first stages are loaded and prefetched
    // during this tile's last steps)
    const int nlid = lid + lstep;
    const bool more = nlid < lend;
    int nb = b, nti = ti, ntj = tj;
    if (more) decode_tile(g, nlid, nb, nti, ntj);
    const __amdgpu_buffer_rsrc_t rPn = tile_rsrc<TNL, TILE>(g.P, g.p_bs, g.p_rows, g.K, nb, nti);
    const __amdgpu_buffer_rsrc_t rQn = tile_rsrc<TNL, TILE>(g.Q, g.q_bs, g.q_rows, g.K, nb, ntj);

    // Main loop of one tile, software-pipelined at two levels:
    //  * LDS ring: stage kt+1 is in flight while stage kt is consumed;
    //  * fragments: substep s+1 is read from LDS under the MFMAs of substep s, and
    //    substep 0 of stage kt+1 under the last substep of stage kt, so the MFMA pipe
    //    never waits on LDS; the one barrier per stage sits before the last substep.
    // The slot refilled at step kt (stage kt+1) held stage kt-1, whose last fragment
    // reads completed (lgkmcnt(0)) before the barrier of step kt-1.
    // Stage 0 was requested before the previous tile's epilogue, whose vm_after
    // vector memory instructions (aux loads, stores) followed it.  Vector memory
    // instructions of a wave complete in order (the compiler's own waits in the
    // epilogue count on it too), so waiting until at most vm_after are outstanding
    // lands stage 0 and leaves the stores draining under this tile's first stage.
    // (the builtin, not inline asm, so that the compiler's own wait tracking sees it;
    // encoding: vmcnt in bits 3:0 and 15:14, expcnt and lgkmcnt left at their maxima)
    switch (vm_after) {
      case 8: __builtin_amdgcn_s_waitcnt(0x0F78); break;
      case 16: __builtin_amdgcn_s_waitcnt(0x4F70); break;
      case 24: __builtin_amdgcn_s_waitcnt(0x4F78); break;
      case 32: __builtin_amdgcn_s_waitcnt(0x8F70); break;
      case 48: __builtin_amdgcn_s_waitcnt(0xCF70); break;
      default: __builtin_amdgcn_s_waitcnt(0x0F70); break;
    }
    ring_barrier();
#pragma unroll
    for (int i = 0; i < BM; ++i)
#pragma unroll
      for (int j = 0; j < BN; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
    DMH_RD(f0, smem + s_cur * STAGEB, 0);
    for (int kt = 0; kt + 1 < nk; ++kt) {
      const int s_nxt = s_cur ^ 1;
      const char* cur = smem + s_cur * STAGEB;
      const char* nxt = smem + s_nxt * STAGEB;
      const int ks = kt + 1 + kofs;
      DMH_GLOAD(rP, rQ, (ks < nk ? ks : ks - nk) * TK, s_nxt);
      // MFMA sections run at wave priority 1 and the load issue, the wait and the
      // barrier at 0, so a SIMD's arbiter favours the wave that has MFMAs to issue
      // (-0.2 to -0.8% of the chain time)
      __builtin_amdgcn_s_setprio(1);
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
      __builtin_amdgcn_s_setprio(0);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");        // stage kt+1 landed (own loads)
      ring_barrier();                                          // ... and everyone's
      __builtin_amdgcn_s_setprio(1);
      DMH_RD(f0, nxt, 0);
      DMH_MM(f1);
      DMH_SCHED_SUB();
      __builtin_amdgcn_s_setprio(0);
      s_cur = s_nxt;
    }
    // Last stage: the next tile's first stage goes into the free slot (it held stage
    // nk-2, or the previous tile's last stage, both consumed before a barrier) and
    // stays in flight under the epilogue.
    const int nkofs = (g.kspread * (nti + ntj)) % nk;
    if (more) DMH_GLOAD(rPn, rQn, nkofs * TK, s_cur ^ 1);
    // Nothing may be scheduled across this point: the next tile's first wait counts
    // on exactly vm_after vector memory instructions (the epilogue's aux loads and
    // stores) following these loads in program order.
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(1);
    {
      const char* cur = smem + s_cur * STAGEB;
      DMH_RD(f1, cur, 1);
      DMH_MM(f0);
      DMH_RD(f0, cur, 2);
      DMH_MM(f1);
      DMH_RD(f1, cur, 3);
      DMH_MM(f0);
      DMH_MM(f1);
      DMH_SCHED_SUB();
      DMH_SCHED_SUB();
      DMH_SCHED_SUB();
      __builtin_amdgcn_sched_group_barrier(0x008, BM * BN, 0);
    }
    __builtin_amdgcn_s_setprio(0);

    // ---- epilogue (per wave, no workgroup barrier) ----------------------------
    // The wave's 128 x 64 output goes out through its 4 KB staging area:
    //   row pass, one 32 x 64 block row at a time:
    //     phase 1  acc -> staging: v = bf16(acc) (bf16(c * acc) for POLY)
    //     phase 2  16-byte chunks: POLY epilogue (aux read in 16 B), store C[i][j];
    //              with a transposed store to come, POLY's values go back into acc
    //              (phase 2b, through the staging area)
    //   transposed pass (outT), one 64 x 32 block at a time: acc -> staging, then
    //     each lane reads 8 rows x 4 columns, transposes them in registers and
    //     stores C^T[j][i] in 16-byte chunks; the 64 lanes of a store cover 8 whole
    //     128-byte lines (8 rows j x 64 i).  (Half-line stores of a transposed
    //     32-row block made the next launch's reads of those lines slow: the chain
    //     ran 10% longer.)
    // Row-pass staging element (r, c) sits at byte rpos(r, c>>3) + 2*(c&7), the 16-byte
    // chunks of a row XOR-swizzled by r&7 and r>>4; transposed-pass element (i, j) at
    // tpos(i, j>>2) + 2*(j&3), the 64-byte rows permuted by i ^ (i>>3 & 3) and the 8-byte
    // units swizzled by i&7 and bits 4-5 of i.  With 32 or with 64 four-byte LDS banks the
    // transposed pass's 8-byte writes and reads are then conflict free (an unswizzled
    // read of 8 rows i = 8a + q by 8 consecutive lanes hit one bank 8 times) and the
    // row pass's 8-byte writes at most 2-way (4-way with the r&7 swizzle alone).
    // acc[i][j][4g+q] holds C[32 i + (lane&31)][32 j + 8g + 4(lane>>5) + q] of the
    // wave tile.
    // Diagonal tiles of a symmetric product are stored whole, row-major: the MFMAs
    // compute C[i][j] and C[j][i] from the same products in the same order.
    {
      const int wi0 = ti * TILE + WT_M * wm, wj0 = tj * TILE + WT_N * wn;
      const bool diag = g.sym && ti == tj;
      auto rpos = [](int r, int ch) { return r * 128 + 16 * (ch ^ (r & 7) ^ ((r >> 4) & 1)); };
      auto tpos = [](int i, int u) {
        return (i ^ ((i >> 3) & 3)) * 64 + 8 * (u ^ (i & 7) ^ ((i >> 2) & 4) ^ (((i >> 5) & 1) * 6));
      };
      bf16* outb = g.out ? g.out + (long long)b * g.out_bs : nullptr;
      bf16* outtb = g.outT && !diag ? g.outT + (long long)b * g.outT_bs : nullptr;
      const bool al_out = g.out_rows > 0 || (g.out_ld & 7) == 0;
      const bool al_outT = g.outT_rows > 0 || (g.outT_ld & 7) == 0;
      // element offsets of C[i][j..j+7] and C^T[j][i..i+7] (8 consecutive bf16 either way:
      // blocks are 64 wide and the chunks 8-aligned)
      auto out_off = [&](int i, int j) {
        return g.out_rows > 0 ? blk_off(i, j, g.out_rows) : (long long)i * g.out_ld + j;
      };
      auto outT_off = [&](int j, int i) {
        return g.outT_rows > 0 ? blk_off(j, i, g.outT_rows) : (long long)j * g.outT_ld + i;
      };
      const bf16* auxb = EPI == EPI_POLY ? g.aux + (long long)b * g.aux_bs : nullptr;
      // one store per 16-byte chunk when the wave's 128 x 64 block is whole and
      // aligned: the epilogue then issues a known number of memory instructions
      const bool whole = wi0 + WT_M <= g.valid_i && wj0 + WT_N <= g.valid_j &&
                         (!outb || al_out) && (!outtb || al_outT);
      vm_after = whole ? (outb ? C::ROW_STORES : 0) + (outtb ? C::T_STORES : 0) +
                             (EPI == EPI_POLY ? C::AUX_LOADS : 0)
                       : -1;
      // POLY: the aux of block row 0 is requested up front and that of row bi+1 once
      // row bi's accumulators are staged, so the reads run one block row ahead of
      // their use (latency hidden under the staging, registers bounded)
      constexpr int AUX_AHEAD = 1;
      bf16x8 av[EPI == EPI_POLY ? BM : 1][4];
      auto load_aux = [&](int bi) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int u = lane + 64 * v;
          const int gi = wi0 + 32 * bi + (u >> 3), gj = wj0 + 8 * (u & 7);
          av[bi][v] = *(const bf16x8*)(auxb + blk_off(gi, gj, g.aux_rows));
        }
      };
      if (EPI == EPI_POLY) {
#pragma unroll
        for (int bi = 0; bi < AUX_AHEAD; ++bi) load_aux(bi);
      }
#pragma unroll
      for (int bi = 0; bi < BM; ++bi) {
        const int i0 = wi0 + 32 * bi;   // global row of staging row 0
        // phase 1
#pragma unroll
        for (int bj = 0; bj < BN; ++bj) {
#pragma unroll
          for (int gq = 0; gq < 4; ++gq) {
            bf16x4 o;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const float v = acc[bi][bj][4 * gq + q];
              o[q] = f2bf(EPI == EPI_POLY ? g.beta * v : v);
            }
            const int ch = 4 * bj + gq;
            *(bf16x4*)(stg + rpos(r32, ch) + 8 * hi) = o;
          }
        }
        if (EPI == EPI_POLY && bi + AUX_AHEAD < BM) load_aux(bi + AUX_AHEAD);
        // phase 2: plain stores read a lane's chunks two at a time, so two LDS reads
        // share one wait (not a read-wait-store chain per chunk; four at a time spill
        // registers in K3, and POLY, shorter still, reads each chunk where it uses
        // it); whole wave tiles store without masks or branches
        bf16x8 val[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int u = lane + 64 * v;
          const int r = u >> 3, ch = u & 7;
          if (EPI == EPI_POLY) val[v] = *(const bf16x8*)(stg + rpos(r, ch));
          else if ((v & 1) == 0) {
            val[v] = *(const bf16x8*)(stg + rpos(r, ch));
            val[v + 1] = *(const bf16x8*)(stg + rpos((u + 64) >> 3, (u + 64) & 7));
          }
          const int gi = i0 + r, gj = wj0 + 8 * ch;
          if (EPI == EPI_POLY) {
            const int qd = diag && gi < g.diag_lim ? gi - gj : -1;   // the diagonal's slot, if here
#pragma unroll
            for (int q = 0; q < 8; ++q)
              val[v][q] = f2bf(g.alpha * bf2f(av[EPI == EPI_POLY ? bi : 0][v][q]) + bf2f(val[v][q]) +
                               (q == qd ? g.diag_add : 0.f));
            if (outtb) *(bf16x8*)(stg + rpos(r, ch)) = val[v];
          }
          if (outb) {
            if (whole) {
              __builtin_nontemporal_store(val[v], (bf16x8*)(outb + out_off(gi, gj)));
            } else if (gi < g.valid_i) {
              unsigned mask = 0xffu;
              if (gj + 8 > g.valid_j) mask = gj >= g.valid_j ? 0u : (1u << (g.valid_j - gj)) - 1u;
              if (mask) store8(outb + out_off(gi, gj), val[v], mask, al_out);
            }
          }
        }
        // phase 2b: POLY's stored values back into acc (the inverse of phase 1)
        if (EPI == EPI_POLY && outtb) {
#pragma unroll
          for (int bj = 0; bj < BN; ++bj) {
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
              const int ch = 4 * bj + gq;
              const bf16x4 o = *(const bf16x4*)(stg + rpos(r32, ch) + 8 * hi);
#pragma unroll
              for (int q = 0; q < 4; ++q) acc[bi][bj][4 * gq + q] = bf2f(o[q]);
            }
          }
        }
      }
      // transposed pass
      if (outtb) {
        const int a = lane & 7, c = lane >> 3;   // rows 8a..8a+7, columns 4c..4c+3 of a block
#pragma unroll
        for (int bp = 0; bp < BM / 2; ++bp) {
#pragma unroll
          for (int bj = 0; bj < BN; ++bj) {
            // acc -> staging: block rows 2 bp, 2 bp + 1 (i < 64), column block bj (j < 32)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
              for (int gq = 0; gq < 4; ++gq) {
                bf16x4 o;
#pragma unroll
                for (int q = 0; q < 4; ++q) o[q] = f2bf(acc[2 * bp + h][bj][4 * gq + q]);
                const int i = 32 * h + r32, unit = 2 * gq + hi;
                *(bf16x4*)(stg + tpos(i, unit)) = o;
              }
            }
            uint2 rr[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
              const int i = 8 * a + q;
              rr[q] = *(const uint2*)(stg + tpos(i, c));
            }
            const int gi = wi0 + 64 * bp + 8 * a;
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) {
              const int gj = wj0 + 32 * bj + 4 * c + cc;
              // column cc of the 8x4 block: halves (cc&1) of words (cc>>1)
              uint32_t w[4];
#pragma unroll
              for (int h = 0; h < 4; ++h) {
                const uint32_t x0 = (cc >> 1) ? rr[2 * h].y : rr[2 * h].x;
                const uint32_t x1 = (cc >> 1) ? rr[2 * h + 1].y : rr[2 * h + 1].x;
                const uint32_t lo = (cc & 1) ? (x0 >> 16) : (x0 & 0xffffu);
                const uint32_t hw = (cc & 1) ? (x1 & 0xffff0000u) : (x1 << 16);
                w[h] = lo | hw;
              }
              const uint4 wv = make_uint4(w[0], w[1], w[2], w[3]);
              if (whole) {
                __builtin_nontemporal_store(__builtin_bit_cast(bf16x8, wv),
                                            (bf16x8*)(outtb + outT_off(gj, gi)));
                continue;
              }
              if (gj >= g.valid_j) continue;
              unsigned mask = 0xffu;
              if (gi + 8 > g.valid_i) mask = gi >= g.valid_i ? 0u : (1u << (g.valid_i - gi)) - 1u;
              if (mask) store8(outtb + outT_off(gj, gi), __builtin_bit_cast(bf16x8, wv), mask, al_outT);
            }
          }
        }
      }
    }
    if (!more) break;
    lid = nlid; b = nb; ti = nti; tj = ntj;
    rP = rPn; rQ = rQn;
    kofs = nkofs;
    s_cur ^= 1;
  }
#undef DMH_RD
#undef DMH_MM
#undef DMH_SCHED_SUB
#undef DMH_GLOAD
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

// Sum of squares of one matrix of the input, NORM_CHUNKS partials per matrix (fp64,
// per element), one workgroup per partial.  When the matrix's rows are contiguous
// and back to back (column stride 1, row stride = cols) the matrix is one run of
// rows * cols elements, read in 16-byte loads from its first 16-byte boundary on;
// otherwise each workgroup takes a range of rows and reads them element by element.
__global__ __launch_bounds__(256) void entry_norm_partials(InView v, double* partials) {
  const int b = blockIdx.y, chunk = blockIdx.x, tid = threadIdx.x;
  double s = 0.0;
  if (v.cs == 1 && v.rs == v.cols) {
    const long long total = (long long)v.rows * v.cols;
    const long long per = (total + NORM_CHUNKS - 1) / NORM_CHUNKS;
    const long long lo = (long long)chunk * per;
    const long long hi = lo + per < total ? lo + per : total;
    const int vec = v.dtype == 0 ? 4 : 8;   // elements per 16 bytes
    const char* base = (const char*)v.x + ((long long)b * v.bs) * (v.dtype == 0 ? 4 : 2);
    const int esz = v.dtype == 0 ? 4 : 2;
    // first element of [lo, hi) on a 16-byte boundary
    long long a = lo + (long long)((16 - (((uintptr_t)(base + lo * esz)) & 15)) & 15) / esz;
    if (a > hi) a = hi;
    const long long nvec = (hi - a) / vec;
    const long long tail = a + nvec * vec;
    for (long long e = lo + tid; e < a; e += 256) {
      const float x = v.dtype == 0 ? ((const float*)base)[e] : bf2f(((const bf16*)base)[e]);
      s += (double)x * (double)x;
    }
    if (v.dtype == 0) {
      const float4* p4 = (const float4*)(base + a * 4);
      for (long long q = tid; q < nvec; q += 256) {
        const float4 x = p4[q];
        s += (double)x.x * (double)x.x + (double)x.y * (double)x.y +
             (double)x.z * (double)x.z + (double)x.w * (double)x.w;
      }
    } else {
      const bf16x8* p8 = (const bf16x8*)(base + a * 2);
      for (long long q = tid; q < nvec; q += 256) {
        const bf16x8 x = p8[q];
#pragma unroll
        for (int k = 0; k < 8; ++k) s += (double)bf2f(x[k]) * (double)bf2f(x[k]);
      }
    }
    for (long long e = tail + tid; e < hi; e += 256) {
      const float x = v.dtype == 0 ? ((const float*)base)[e] : bf2f(((const bf16*)base)[e]);
      s += (double)x * (double)x;
    }
  } else {
    const int rpc = (v.rows + NORM_CHUNKS - 1) / NORM_CHUNKS;
    const int r0 = chunk * rpc, r1 = r0 + rpc < v.rows ? r0 + rpc : v.rows;
    for (int r = r0; r < r1; ++r)
      for (int c = tid; c < v.cols; c += 256) {
        const float x = load_in(v, b, r, c);
        s += (double)x * (double)x;
      }
  }
  __shared__ double red[256];
  red[tid] = s;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (tid < w) red[tid] += red[tid + w];
    __syncthreads();
  }
  if (tid == 0) partials[b * NORM_CHUNKS + chunk] = red[0];
}

// Pack 64x64 tiles of T (i < np rows, j < mp cols) into the chain's block layout.
// in_tall: the input is T (rows = n); otherwise it is W = T^T (rows = m) and is
// transposed on the way through LDS.  scale_mode: 0 none, 1: x / (||x|| + 1e-7),
// 2: x / (1.01 ||x|| + 1e-7), one fp32 division and one bf16 rounding per element.
// fp32 input whose rows are contiguous and 16-byte aligned is read 4 elements at a
// time (16 lanes per 64-column row); anything else element by element.
__global__ __launch_bounds__(256) void entry_pack(InView v, int in_tall, int scale_mode,
                                                  const double* partials, int n, int m,
                                                  int np, int mp, bf16* T) {
  __shared__ float tile[64][65];
  const int b = blockIdx.z, tid = threadIdx.x;
  const int i0 = blockIdx.y * 64, j0 = blockIdx.x * 64;
  float den = 1.f;
  if (scale_mode) {
    __shared__ float s_den;
    if (tid == 0) {
      double s = 0.0;
      for (int c = 0; c < NORM_CHUNKS; ++c) s += partials[b * NORM_CHUNKS + c];
      const float nrm = (float)sqrt(s);
      s_den = scale_mode == 2 ? nrm * 1.01f + 1e-7f : nrm + 1e-7f;
    }
    __syncthreads();
    den = s_den;
  }
  bf16* Tb = T + (long long)b * np * mp;
  const float* xf = (const float*)v.x;
  const bool vec = v.dtype == 0 && v.cs == 1 && (v.rs & 3) == 0 && (v.bs & 3) == 0 &&
                   (((uintptr_t)v.x) & 15) == 0;
  // 4 consecutive elements of row r, columns c..c+3 of the input (zero outside
  // rows x cols)
  auto load4 = [&](int r, int c, int rows, int cols) {
    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
    if (r >= rows) return x;
    if (vec && c + 3 < cols) {
      x = *(const float4*)(xf + (long long)b * v.bs + (long long)r * v.rs + c);
    } else {
      if (c + 0 < cols) x.x = load_in(v, b, r, c + 0);
      if (c + 1 < cols) x.y = load_in(v, b, r, c + 1);
      if (c + 2 < cols) x.z = load_in(v, b, r, c + 2);
      if (c + 3 < cols) x.w = load_in(v, b, r, c + 3);
    }
    return x;
  };
  const int cq = (tid & 15) * 4;   // 4 columns of the tile
  const int rr0 = tid >> 4;        // rows rr0 + 16 k
  if (in_tall) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int i = i0 + rr0 + 16 * k;
      float4 x = load4(i, j0 + cq, n, m);
      if (scale_mode) { x.x = x.x / den; x.y = x.y / den; x.z = x.z / den; x.w = x.w / den; }
      bf16x4 o;
      o[0] = f2bf(x.x); o[1] = f2bf(x.y); o[2] = f2bf(x.z); o[3] = f2bf(x.w);
      *(bf16x4*)(Tb + blk_off(i, j0 + cq, np)) = o;
    }
  } else {
    // input rows j0.. (columns of T), columns i0.. (rows of T): W[j][i] -> tile[j][i]
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int jj = rr0 + 16 * k;
      const float4 x = load4(j0 + jj, i0 + cq, m, n);
      tile[jj][cq + 0] = x.x; tile[jj][cq + 1] = x.y; tile[jj][cq + 2] = x.z; tile[jj][cq + 3] = x.w;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int ii = rr0 + 16 * k;
      float y[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        y[q] = tile[cq + q][ii];
        if (scale_mode) y[q] = y[q] / den;
      }
      bf16x4 o;
      o[0] = f2bf(y[0]); o[1] = f2bf(y[1]); o[2] = f2bf(y[2]); o[3] = f2bf(y[3]);
      *(bf16x4*)(Tb + blk_off(i0 + ii, j0 + cq, np)) = o;
    }
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
    out[(long long)b * total + e] = T[(long long)b * np * mp + blk_off(i, j, np)];
  }
}

ChainDims chain_dims(int rows, int cols, int orient_tall) {
  ChainDims d;
  d.n = orient_tall ? rows : cols;
  d.m = orient_tall ? cols : rows;
  d.np = ceil_div(d.n, CHAIN_TILE) * CHAIN_TILE;
  d.mp = ceil_div(d.m, CHAIN_TILE) * CHAIN_TILE;
  return d;
}

int chain_check(const char* what, const ChainDims& d) {
  // the largest operand is the padded iterate T (np x mp bf16, np >= mp); its buffer
  // descriptor's record count and the loaders' byte offsets are 32-bit
  if ((long long)d.np * d.mp * (long long)sizeof(bf16) >= (1LL << 31)) {
    set_error("%s: a %d x %d matrix pads to %d x %d bf16 = %lld bytes, beyond the chain's "
              "32-bit operand addressing (< 2^31 bytes)", what, d.n, d.m, d.np, d.mp,
              (long long)d.np * d.mp * (long long)sizeof(bf16));
    return DMH_EINVAL;
  }
  return DMH_OK;
}

ChainWs chain_ws(void* ws, int batch, const ChainDims& d) {
  ChainWs w{};
  const size_t tw = (size_t)batch * d.np * d.mp;
  const size_t sq = (size_t)batch * d.mp * d.mp;
  const size_t part = (size_t)batch * NORM_CHUNKS * sizeof(double);
  w.bytes = (2 * tw + 2 * sq) * sizeof(bf16) + ((part + 255) / 256) * 256;
  if (!ws) return w;
  w.T0 = (bf16*)ws;
  w.T1 = w.T0 + tw;
  w.A = w.T1 + tw;
  w.B = w.A + sq;
  w.partials = (double*)(w.B + sq);
  return w;
}

// compute units of the current device (one persistent GEMM workgroup each)
static int device_cus() {
  constexpr int MAXDEV = 64;
  static int cus[MAXDEV];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAXDEV) return 0;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cus[dev] = n;
  }
  return cus[dev];
}

// One persistent launch of a GEMM phase with TILE x TILE output tiles over rows x cols
// outputs per matrix (multiples of 256); one workgroup per free workgroup slot
// (GemmCfg::WG_PER_CU per compute unit), or fewer when there are fewer tiles.
template <int EPI, int TNL, int TL>
static int launch_gemm_tl(GemmArgs g, int rows, int cols, int batch, hipStream_t stream,
                          const char* what) {
  using Cf = GemmCfg<TL>;
  g.tiles_m = rows / TL;
  g.tiles_n = cols / TL;
  const long long per = g.sym ? (long long)g.tiles_m * (g.tiles_m + 1) / 2
                              : (long long)g.tiles_m * g.tiles_n;
  const long long tiles = per * batch;
  const long long slots = (long long)device_cus() * Cf::WG_PER_CU;
  if (tiles <= 0 || tiles > 0x7fffffffLL || slots <= 0) {
    set_error("%s: bad grid (%lld tiles, %lld workgroup slots)", what, tiles, slots);
    return DMH_EINVAL;
  }
  g.total_tiles = (int)tiles;
  g.batch = batch;
  const int grid = (int)(tiles < slots ? tiles : slots);
  hipLaunchKernelGGL((gemm_nt_bf16<EPI, TNL, TL>), dim3(grid), dim3(Cf::THREADS), 0, stream, g);
  DMH_CHECK_LAUNCH(what);
  return DMH_OK;
}

template <int EPI, int TNL>
static int launch_gemm(const GemmArgs& g, int tile, int rows, int cols, int batch,
                       hipStream_t stream, const char* what) {
  return tile == 128 ? launch_gemm_tl<EPI, TNL, 128>(g, rows, cols, batch, stream, what)
                     : launch_gemm_tl<EPI, TNL, 256>(g, rows, cols, batch, stream, what);
}

// Output tile size of the three phases (K1, K2, K3) for a shape.  Chosen from the
// shape alone, never from the batch, so a matrix's result does not depend on the
// batch it is computed in (the tile fixes each output's K-walk order).  The m x m
// products of a matrix with m <= 768 have at most 6 upper 256 x 256 tiles, too few to
// keep the CUs busy: they run on 128 x 128 tiles (GPT-2 small, m = 768: the chain
// 1.91 -> 1.59 ms per deflated polar step); the tall product T B' keeps 256 x 256
// tiles there (128 x 128: 1.66 ms), as do K1 and K2 from m = 1024 on (GPT-2 medium
// 6.10 ms with 256 x 256 tiles everywhere, 6.31 with 128 x 128 for K1).
static void phase_tiles(const ChainDims& d, int tile[3]) {
  const int small = d.mp <= 768 ? 128 : 256;
  tile[0] = small;
  tile[1] = small;
  tile[2] = 256;
  const char* env = getenv("DMH_CHAIN_TILES");   // tuning override "k1,k2,k3"
  int t[3];
  if (env && sscanf(env, "%d,%d,%d", &t[0], &t[1], &t[2]) == 3)
    for (int i = 0; i < 3; ++i) tile[i] = t[i] == 128 ? 128 : 256;
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
  int tl[3];
  phase_tiles(d, tl);
  // Consecutive launches walk the batch in opposite directions, so each one starts
  // on the matrices the previous one wrote last, which are still in the memory-side
  // cache (the group's operands are several times its size).  The entry pack wrote
  // the batch in increasing order, so K1 of the first iteration runs reversed.
  int rev = 1;
  bf16 *Tc = w.T0, *Tn = w.T1;
  bf16 *Am = w.A, *Bm = w.B;
  for (int it = 0; it < steps; ++it) {
    const float a = (float)coeffs[3 * it + 0];
    const float bcoef = (float)coeffs[3 * it + 1];
    const float c = (float)coeffs[3 * it + 2];
    const bool last = it + 1 == steps;
    int rc;
    // K1: A = W W^T = T^T T, with both operands read K-major from T (row k of T
    // holds column k of W)
    GemmArgs g1{};
    g1.P = Tc; g1.p_bs = (long long)d.np * d.mp; g1.p_rows = d.np;
    g1.Q = Tc; g1.q_bs = g1.p_bs; g1.q_rows = d.np;
    g1.K = d.np; g1.sym = 1;
    g1.out = Am; g1.out_bs = (long long)d.mp * d.mp; g1.out_rows = d.mp;
    g1.outT = Am; g1.outT_bs = g1.out_bs; g1.outT_rows = d.mp;
    g1.valid_i = d.mp; g1.valid_j = d.mp;
    g1.rev = rev; rev ^= 1;
    g1.kspread = 1;
    if ((rc = launch_gemm<EPI_STORE, 1>(g1, tl[0], d.mp, d.mp, batch, stream, "ns K1 (T^T T)")))
      return rc;
    // K2: B = b A + c A A
    GemmArgs g2 = g1;
    g2.P = Am; g2.p_bs = (long long)d.mp * d.mp; g2.p_rows = d.mp;
    g2.Q = Am; g2.q_bs = g2.p_bs; g2.q_rows = d.mp;
    g2.K = d.mp;
    g2.alpha = bcoef; g2.beta = c; g2.diag_add = a; g2.diag_lim = d.m;
    g2.aux = Am; g2.aux_bs = g2.p_bs; g2.aux_rows = d.mp;
    g2.out = Bm; g2.outT = Bm;
    g2.rev = rev; rev ^= 1;
    g2.kspread = 0;
    if ((rc = launch_gemm<EPI_POLY, 0>(g2, tl[1], d.mp, d.mp, batch, stream,
                                      "ns K2 (bA + cA^2 + aI)")))
      return rc;
    // K3: T' = T B' (the final iterate in the caller's orientation)
    GemmArgs g3{};
    g3.P = Tc; g3.p_bs = (long long)d.np * d.mp; g3.p_rows = d.np;
    g3.Q = Bm; g3.q_bs = (long long)d.mp * d.mp; g3.q_rows = d.mp;
    g3.K = d.mp; g3.sym = 0;
    if (!last) {
      g3.out = Tn; g3.out_bs = g3.p_bs; g3.out_rows = d.np;
      g3.valid_i = d.np; g3.valid_j = d.mp;
    } else if (orient_tall) {
      g3.out = outp; g3.out_bs = (long long)d.n * d.m; g3.out_ld = d.m;
      g3.valid_i = d.n; g3.valid_j = d.m;
    } else {
      g3.outT = outp; g3.outT_bs = (long long)d.n * d.m; g3.outT_ld = d.n;
      g3.valid_i = d.n; g3.valid_j = d.m;
    }
    g3.rev = rev; rev ^= 1;
    g3.kspread = 2;
    if ((rc = launch_gemm<EPI_STORE, 0>(g3, tl[2], d.np, d.mp, batch, stream, "ns K3 (T B')")))
      return rc;
    bf16* t = Tc; Tc = Tn; Tn = t;
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
  const ChainDims d = chain_dims(rows, cols, orient_tall);
  if (chain_check("dmh_ns_workspace_size", d)) return DMH_EINVAL;
  *bytes = chain_ws(nullptr, batch, d).bytes;
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
  if (chain_check("dmh_ns_chain", d)) return DMH_EINVAL;
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
                     orient_tall, entry_mode, w.partials, d.n, d.m, d.np, d.mp, w.T0);
  DMH_CHECK_LAUNCH("entry_pack");
  return chain_run_packed(stream, w, batch, d, orient_tall, coeffs, steps, (bf16*)out);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// dmh_ns_chain_noalloc: dmh_ns_chain with its workspace in a static device array
// (for callers that cannot allocate: code under HIP graph capture, serving loops,
// harnesses that forbid hipMalloc).  Each GPU holds its own copy of the array from
// the moment the library's code object is loaded there (the first launch of any of
// its kernels on that GPU) until the process ends, whether or not this entry is used.  The array's host-side name is not a
// device address: its address on the current device comes from hipGetSymbolAddress,
// once per device, and only that pointer is handed to kernels.  Every call on a GPU
// uses the same array, so calls that overlap on one GPU (other streams, other
// threads) race; the chain writes every byte of its workspace it reads, so nothing
// needs clearing between calls.
// ---------------------------------------------------------------------------
namespace dmh {

static __device__ __align__(256) unsigned char scratch[DMH_NS_SCRATCH_BYTES];

static int scratch_address(void** out) {
  constexpr int MAXDEV = 64;
  static void* addr[MAXDEV];
  static std::mutex mu;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAXDEV) {
    set_error("dmh_ns_chain_noalloc: no usable current device (%d)", dev);
    return DMH_ELAUNCH;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      set_error("dmh_ns_chain_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                hipGetErrorString(e));
      return DMH_ELAUNCH;
    }
    addr[dev] = p;
  }
  *out = addr[dev];
  return DMH_OK;
}

}  // namespace dmh

extern "C" int dmh_ns_chain_noalloc(hipStream_t stream, const void* x, int x_dtype, int batch,
                                    int rows, int cols, long long x_bstride, long long x_rstride,
                                    long long x_cstride, void* out, int orient_tall,
                                    int entry_mode, const double* coeffs, int steps) {
  if (batch == 0) return DMH_OK;
  if (batch < 0 || rows <= 0 || cols <= 0) {
    set_error("dmh_ns_chain_noalloc: bad arguments (batch=%d rows=%d cols=%d)", batch, rows, cols);
    return DMH_EINVAL;
  }
  const ChainDims d = chain_dims(rows, cols, orient_tall);
  if (chain_check("dmh_ns_chain_noalloc", d)) return DMH_EINVAL;
  const size_t need = chain_ws(nullptr, batch, d).bytes;
  if (need > (size_t)DMH_NS_SCRATCH_BYTES) {
    set_error("dmh_ns_chain_noalloc: batch=%d of %dx%d needs %zu bytes of workspace, more than "
              "the %zu-byte static scratch; use dmh_ns_chain with a caller workspace",
              batch, rows, cols, need, (size_t)DMH_NS_SCRATCH_BYTES);
    return DMH_EWORKSPACE;
  }
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc) return rc;
  return dmh_ns_chain(stream, x, x_dtype, batch, rows, cols, x_bstride, x_rstride, x_cstride, out,
                      orient_tall, entry_mode, coeffs, steps, ws, (size_t)DMH_NS_SCRATCH_BYTES);
}
