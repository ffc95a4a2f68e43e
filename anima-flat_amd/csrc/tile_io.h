// Tile formats and HBM -> LDS staging shared by the attention kernels.
//
// Every streamed operand is a tile of 64 rows x 128 bf16 (16 KB), held in LDS
// in one of two layouts that make the 16-byte MFMA operand reads of a wave
// free of bank conflicts on the 64 banks of 4 bytes:
//
// Row tile (rows = keys or queries, 128 head-dim values each):
//   element (r, d) at (r >> 4) * 2048 + (d >> 3) * 128 + (r & 15) * 8 + (d & 7),
//   i.e. 256-byte slices of (16-row group, 16-byte chunk). An A-operand read
//   of row 32 t + li, chunk 2 kk + hh (lane li = lane % 32, hh = lane / 32) is
//   at row_rd(lane) + 4096 t + 256 kk: 16 lanes cover 16 consecutive slots.
//
// Transposed tile (rows = head-dim values, 64 keys or queries each), the
//   exact LDS image the transposed operand reads want, with the 64 columns
//   taken in 16-column chunks c4 and, inside a chunk, in the order of the
//   32x32 MFMA accumulator rows (so an accumulator tile converted to bf16
//   feeds the next MFMA as its B operand unchanged):
//   element (d, col) at (d >> 4) * 1024 + c' * 128 + (d & 15) * 8 + e, where
//   c' = 2 c4 + h holds columns tt_col(c', e) = 16 c4 + 8 (e >> 2) + 4 h + (e & 3).
//   The A-operand read of rows 32 dt + li, chunk c4 is at
//   tt_rd(lane) + 2048 dt + 256 c4. These tiles are written to HBM by a
//   packing pass (pack_transposed_tile) and copied into LDS linearly.
//
// Staging: global_load_lds_dwordx4 (DMA straight into LDS, no registers).
//   One instruction moves 64 lanes x 16 B = 1 KB, written contiguously at
//   M0 + 16 * lane, so a tile is 16 blocks of 1 KB. For a row tile, block blk
//   holds rows 16 (blk >> 2) + (lane & 15), chunks 4 (blk & 3) + (lane >> 4).
#pragma once

#include "aa_common.h"

namespace aa {

constexpr int kTileRows = 64;
constexpr int kTileElems = kTileRows * 128;  // 16 KB of bf16
constexpr int kTileBlocks = 16;              // 1 KB DMA blocks per tile

// Column of a transposed tile stored at chunk slot c' = 2 c4 + h, element e.
__device__ __forceinline__ int tt_col(int cp, int e) {
  return 16 * (cp >> 1) + 8 * ((e >> 2) & 1) + 4 * (cp & 1) + (e & 3);
}

// Per-lane read bases (elements) of the two layouts.
__device__ __forceinline__ int row_rd(int lane) {
  const int li = lane & 31, hh = lane >> 5;
  return (li >> 4) * 2048 + (li & 15) * 8 + hh * 128;
}
__device__ __forceinline__ int tt_rd(int lane) {
  const int li = lane & 31, hh = lane >> 5;
  return (li >> 4) * 1024 + hh * 128 + (li & 15) * 8;
}

// Workgroup-wide (256 threads): rows [row0, row0 + 64) of a [rows x 128]
// matrix (row stride rs elements, 16-byte aligned rows; rows >= nrows read as
// zero) into the transposed tile format at dst. `stage` is 64 x 136 bf16 of
// LDS. Begins and ends with a barrier, so `stage` may be reused right after.
constexpr int kPackRow = 128 + 8;  // padded LDS row of the staging copy
__device__ __forceinline__ void pack_transposed_tile(const bf16* __restrict__ src, int64_t rs,
                                                     int row0, int nrows, bf16* __restrict__ dst,
                                                     bf16* stage) {
  const int tid = threadIdx.x;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int id = tid + 256 * i;
    const int row = id >> 4, dc = id & 15;
    u32x4 w = {0u, 0u, 0u, 0u};
    if (row0 + row < nrows) w = ld16(src + (int64_t)(row0 + row) * rs + 8 * dc);
    st16(stage + row * kPackRow + 8 * dc, w);
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int oi = tid + 256 * i;  // 16-byte output chunk, in output order
    const int d = 16 * (oi >> 7) + (oi & 15);
    const int cp = (oi >> 4) & 7;
    bf16x8 w;
#pragma unroll
    for (int e = 0; e < 8; ++e) w[e] = stage[tt_col(cp, e) * kPackRow + d];
    *reinterpret_cast<bf16x8*>(dst + 8 * oi) = w;
  }
  __syncthreads();
}

typedef __attribute__((address_space(3))) void lds_void;

// 16 bytes per lane from global memory straight into LDS at
// lds_base + 16 * lane (global_load_lds_dwordx4; M0 holds the LDS base).
// Issued as inline asm so the compiler does not treat every later LDS read as
// possibly depending on this write: completion is tracked by wait_dma() and
// the workgroup barrier that follows it.
__device__ __forceinline__ void dma16(const void* src, const void* lds_base) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void*)lds_base);
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(m0)
               : "memory", "m0");
}

__device__ __forceinline__ void wait_dma() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// DMA blocks [b0, b0 + N) of a row tile whose row 0 is at `base` (row stride
// rs elements); rows at or past `nrows` (>= 1) re-read row nrows - 1, finite
// data the caller masks.
template <int N>
__device__ __forceinline__ void dma_row_tile(const bf16* base, int64_t rs, int nrows,
                                             const bf16* lds_tile, int b0, int lane) {
  const int l15 = lane & 15, lq = lane >> 4;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int blk = b0 + i;
    const int row = min(16 * (blk >> 2) + l15, nrows - 1);
    const int chunk = 4 * (blk & 3) + lq;
    dma16(base + (int64_t)row * rs + 8 * chunk, lds_tile + blk * 512);
  }
}

// One DMA block (blk in 0..15) of a row tile, as dma_row_tile.
__device__ __forceinline__ void dma_row_block(const bf16* base, int64_t rs, int nrows,
                                              const bf16* lds_tile, int blk, int lane) {
  const int row = min(16 * (blk >> 2) + (lane & 15), nrows - 1);
  const int chunk = 4 * (blk & 3) + (lane >> 4);
  dma16(base + (int64_t)row * rs + 8 * chunk, lds_tile + blk * 512);
}

// Swizzled row tile (dK/dV kernel): element (r, d) at
//   (r >> 4) * 2048 + (d >> 3) * 128 + (((r & 15) ^ (4 * ((d >> 3) & 3))) * 8) + (d & 7),
// i.e. the row tile with the row slot inside each 256-byte slice XORed with
// 4 * (chunk % 4). Row-operand reads (16 rows of one chunk per 16 lanes) stay
// conflict free, and so do transposed reads with ds_read_b64_tr_b16 (4 rows x
// 4 chunks per 32 lanes land in 16 distinct slots). One DMA block blk holds
// rows 16 (blk >> 2) + ((lane & 15) ^ (4 (lane >> 4))), chunk 4 (blk & 3) + (lane >> 4).
__device__ __forceinline__ void dma_row_block_swz(const bf16* base, int64_t rs, int nrows,
                                                  const bf16* lds_tile, int blk, int lane) {
  const int row = min(16 * (blk >> 2) + ((lane & 15) ^ (4 * (lane >> 4))), nrows - 1);
  const int chunk = 4 * (blk & 3) + (lane >> 4);
  dma16(base + (int64_t)row * rs + 8 * chunk, lds_tile + blk * 512);
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// ds_read_b64_tr_b16: in each group of 16 lanes, lanes 4 j .. 4 j + 3 give
// the addresses of the four 8-byte pieces of row j (16 consecutive bf16) and
// lane i receives element i of rows 0..3.
__device__ __forceinline__ s16x4 ds_read_tr(const bf16* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(lds_void*)p);
}

// DMA blocks [b0, b0 + N) of a tile stored contiguously (16 KB) at `src`.
template <int N>
__device__ __forceinline__ void dma_linear_tile(const bf16* src, const bf16* lds_tile, int b0,
                                                int lane) {
#pragma unroll
  for (int i = 0; i < N; ++i) dma16(src + (b0 + i) * 512 + lane * 8, lds_tile + (b0 + i) * 512);
}

// Workgroups are dispatched round-robin over the 8 XCDs (block i on XCD
// i % 8). Remap so each XCD gets a contiguous range of logical blocks, whose
// shared K/V (or Q/dO) rows then stay in that XCD's L2.
__device__ __forceinline__ int xcd_remap(int bid, int total) {
  if ((total & 7) != 0) return bid;
  return (bid & 7) * (total >> 3) + (bid >> 3);
}

}  // namespace aa
