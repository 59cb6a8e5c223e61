// Internal interface of the bf16 NS chain (ns_chain.hip) used by the fused
// deflated-polar entry (rsvd.hip).
#pragma once

#include "common.h"

namespace dmh {

constexpr int CHAIN_TILE = 256;

// size of the static workspace of dmh_ns_chain_noalloc (the same value as
// DMH_NS_SCRATCH_BYTES in include/defmuon_hip.h)
#define DMH_NS_SCRATCH_BYTES (64u << 20)

struct ChainDims {
  int n, m, np, mp;   // tall operand T is n x m; padded to multiples of CHAIN_TILE
};

// Block layout of the chain's bf16 operands in its workspace (T: np x mp, A and
// B': mp x mp): 64 x 64 blocks of 8 KB, row-major inside a block, the blocks of
// one block column consecutive.  Element (i, j) of a matrix with R rows sits at
// blk_off(i, j, R).  The 64-column slice of a 256-row panel that one GEMM K stage
// reads is then one contiguous 32 KB run, and the 64 k-rows of a 256-column panel
// (the transposed operand of T^T T) are four contiguous 8 KB runs, instead of 256
// (or 64) rows scattered at the matrix's row stride.
constexpr int CHAIN_BLK = 64;
__host__ __device__ __forceinline__ long long blk_off(int i, int j, int R) {
  return ((long long)(j >> 6) * (R >> 6) + (i >> 6)) * (CHAIN_BLK * CHAIN_BLK) + (i & 63) * CHAIN_BLK +
         (j & 63);
}

// Workspace of one chain call: the tall iterate T double-buffered, A = T^T T and
// B = bA + cA^2 + aI, and the entry's norm partials.
struct ChainWs {
  bf16 *T0, *T1, *A, *B;
  double* partials;
  size_t bytes;
};

ChainDims chain_dims(int rows, int cols, int orient_tall);
// DMH_OK, or DMH_EINVAL (with the error text) when a padded operand reaches 2^31
// bytes: the GEMMs address their operands through 32-bit buffer descriptors and offsets
int chain_check(const char* what, const ChainDims& d);
ChainWs chain_ws(void* ws, int batch, const ChainDims& d);   // ws == nullptr: sizes only

// Run `steps` iterations from T0 already packed in the workspace; the result
// goes to `out` (batch, rows, cols) bf16 in the orientation given.
int chain_run_packed(hipStream_t stream, const ChainWs& w, int batch, const ChainDims& d,
                     int orient_tall, const double* coeffs, int steps, bf16* out);

}  // namespace dmh
