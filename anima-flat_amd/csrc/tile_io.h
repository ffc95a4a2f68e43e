// LDS tile formats and HBM -> LDS staging shared by the attention kernels.
//
// Every streamed operand is a tile of 64 rows x 128 bf16 (16 KB): 64 keys or
// queries, each with its 128 head-dim values. LDS has 64 banks of 4 bytes;
// every format below keeps its operand reads free of bank conflicts. The
// row tiles serve the head_dim-384 forward (32-row sub-tiles); the line tiles
// further down serve the head_dim-128 forward and the backward.
//
// Row tile: element (r, d) at (r >> 4) * 2048 + (d >> 3) * 128 + (r & 15) * 8 + (d & 7),
//   i.e. 256-byte slices of (16-row group, 16-byte chunk). An A-operand read
//   of row 32 t + li, chunk 2 kk + hh (lane li = lane % 32, hh = lane / 32) is
//   at row_rd(lane) + 4096 t + 256 kk: 16 lanes cover 16 consecutive slots.
//
// Swizzled row tile: the same with the row slot inside each slice XORed with
//   4 * (chunk % 4): element (r, d) at
//   (r >> 4) * 2048 + (d >> 3) * 128 + (((r & 15) ^ (4 * ((d >> 3) & 3))) * 8) + (d & 7).
//   It can be read transposed with ds_read_b64_tr_b16 (swz_tr_rd): the 32
//   lanes of one read touch 4 rows x 4 chunks, which land in 16 distinct
//   slots.
//
// Transposed operand: the A operand of v_mfma_f32_32x32x16_bf16 with the
//   tile's rows as the k index, A[m][k] = tile(row k, column 32 dt + m) for
//   the 16 rows of chunk c4. The rows of a chunk are taken in the order in
//   which a 32x32 accumulator holds its rows (lane half h = lane / 32 holds
//   rows 8 (e / 4) + 4 h + (e % 4), e = 0..7), so that accumulator tiles
//   rounded to bf16 are the matching B operands as they are.
//
// Staging: global_load_lds_dwordx4 (DMA straight into LDS, no registers).
//   One instruction moves 64 lanes x 16 B = 1 KB, written contiguously at
//   M0 + 16 * lane, so a tile is 16 blocks of 1 KB; the global address of
//   each lane picks the (row, chunk) that lands in its slot.
#pragma once

#include "aa_common.h"

namespace aa {

constexpr int kTileRows = 64;
constexpr int kTileElems = kTileRows * 128;  // 16 KB of bf16

// Per-lane read offset (elements) of a row-operand read of a row tile.
__device__ __forceinline__ int row_rd(int lane) {
  const int li = lane & 31, hh = lane >> 5;
  return (li >> 4) * 2048 + (li & 15) * 8 + hh * 128;
}

// Per-lane offsets of the two ds_read_b64_tr_b16 reads (r2 = 0, 1) of a
// transposed operand of a swizzled row tile. In a group of 16 lanes
// (G = lane / 16), lanes 4 j .. 4 j + 3 (c = lane % 4) address the four
// 8-byte pieces of row 16 c4 + 4 (G >> 1) + j + 8 r2, columns
// 32 dt + 16 (G & 1) + 4 c .. + 3, and lane 16 G + i receives column
// 32 dt + 16 (G & 1) + i of those four rows: A[m][k] with m = lane % 32 and
// k = 8 (G >> 1) + 4 r2 + j, the accumulator row order.
__device__ __forceinline__ int swz_tr_rd(int lane, int r2) {
  const int G = lane >> 4, j = (lane >> 2) & 3, c = lane & 3;
  const int slot = (((4 * (G >> 1) + j) ^ (4 * (c >> 1))) & 7) + 8 * (r2 ^ (G & 1));
  return 256 * (G & 1) + 128 * (c >> 1) + 4 * (c & 1) + 8 * slot;
}

// Workgroup-wide DMA helpers ------------------------------------------------

typedef __attribute__((address_space(3))) void lds_void;

// 16 bytes per lane from global memory straight into LDS at
// lds_base + 16 * lane (global_load_lds_dwordx4; M0 holds the LDS base).
// Issued as inline asm so the compiler does not treat every later LDS read as
// possibly depending on this write: completion is tracked by wait_dma() (or
// an explicit vmcnt) and the workgroup barrier that follows it.
__device__ __forceinline__ void dma16(const void* src, const void* lds_base) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void*)lds_base);
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(m0)
               : "memory", "m0");
}

// The same with a compile-time byte offset on the global address
// (global_load_lds_dwordx4's immediate offset, 0 <= kOff < 4096): DMAs from
// one base at fixed strides share one address computation. The instruction
// adds its offset to the LDS address as well (M0 + offset + 16 * lane), so M0
// is set kOff bytes below the destination.
template <int kOff>
__device__ __forceinline__ void dma16_off(const void* src, const void* lds_base) {
  static_assert(kOff >= 0 && kOff < 4096, "immediate offset range");
  const uint32_t m0 =
      __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void*)lds_base) - (uint32_t)kOff;
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off offset:%2" ::"v"(src), "s"(m0),
               "n"(kOff)
               : "memory", "m0");
}

__device__ __forceinline__ void wait_dma() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Transposed operand reads ---------------------------------------------------

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// ds_read_b64_tr_b16: in each group of 16 lanes, lanes 4 j .. 4 j + 3 give
// the addresses of the four 8-byte pieces of row j (16 consecutive bf16) and
// lane i receives element i of rows 0..3.
__device__ __forceinline__ s16x4 ds_read_tr(const bf16* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(lds_void*)p);
}

// 32-bit LDS byte address of a pointer into __shared__ memory.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(lds_void*)p;
}

typedef __attribute__((address_space(3))) bf16x8 lds_bf16x8;

// 16-byte read at an LDS byte address (ds_read_b128; constant parts of the
// address fold into the instruction's offset field).
__device__ __forceinline__ bf16x8 lds_ld16(uint32_t addr) {
  return *(const lds_bf16x8*)(uintptr_t)addr;
}

// ds_read_b64_tr_b16 at an LDS byte address.
__device__ __forceinline__ s16x4 lds_ld8_tr(uint32_t addr) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(uintptr_t)addr);
}

// Line tile (the forward's K and V) -------------------------------------------
//
// 64 rows x 128 d as 16 blocks of 8 rows x 64 d (1 KB): block 8 (d >> 6)
// + (r >> 3), row r & 7 of it at 64 elements, the row's 16-byte chunk
// ch = (d >> 3) & 7 in slot ch ^ f(r). One DMA instruction fills one block
// from 8 rows x 128 bytes, i.e. whole cache lines; the row-tile DMA (16 rows
// x 64 bytes, half lines) streams at well under half that rate.
//   K, read as row operands: fk(r) = (r & 7) ^ ((r >> 3) & 1). The 16 rows of
//     an operand read's lane group hold its chunk in 16 distinct (row parity,
//     slot) pairs: 16 distinct bank groups.
//   V, read transposed: fv(r) = 4 ((r >> 1) & 1). The 32 lanes of one
//     ds_read_b64_tr_b16 read 4 rows x 4 chunks; the XOR sends rows 2 and 3
//     of a block to the other half of the row's 8 slots, so the 32 8-byte
//     pieces cover all 64 banks.

// DMA of 16 bytes per lane from sbase + voff (sbase wave-uniform, held in
// SGPRs: the per-lane address is one 32-bit byte offset) to LDS at byte
// address lds_byte + 16 lane.
__device__ __forceinline__ void dma16_sva(const void* sbase, uint32_t voff, uint32_t lds_byte) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_byte);
  // readfirstlane returns int: widen each half through uint32_t (a signed
  // int would sign-extend the low half into the high one).
  const uint64_t sb = (uint64_t)(uintptr_t)sbase;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)sb);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(sb >> 32));
  const uint64_t sbu = ((uint64_t)hi << 32) | (uint64_t)lo;
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbu), "s"(m0)
               : "memory", "m0");
}
// The same with the LDS destination as a pointer into __shared__ memory.
__device__ __forceinline__ void dma16_sv(const void* sbase, uint32_t voff, const void* lds_dst) {
  dma16_sva(sbase, voff, (uint32_t)(uintptr_t)(lds_void*)lds_dst);
}

// Chunk (0..7, within the block's 64 d) that DMA lane `lane` moves into its
// slot: row (lane >> 3) of the block, slot lane & 7. blk_odd = block parity.
__device__ __forceinline__ int line_k_chunk(int lane, int blk_odd) {
  return (lane & 7) ^ (lane >> 3) ^ blk_odd;
}
__device__ __forceinline__ int line_v_chunk(int lane) {
  return (lane & 7) ^ (4 * ((lane >> 4) & 1));
}

// Row-operand read of a K line tile: row 32 kt + li, chunk 2 kk + hh
// (kk = 0..7) is at line_k_rd(lane, kk & 3) + 4096 (kk >> 2) + 2048 kt.
__device__ __forceinline__ int line_k_rd(int lane, int j) {
  const int li = lane & 31, hh = lane >> 5;
  const int fk = (li & 7) ^ ((li >> 3) & 1);
  return ((li >> 3) * 512 + (li & 7) * 64 + (hh ^ fk) * 8) ^ (16 * j);
}

// Transposed-read offsets of a V line tile (the pieces swz_tr_rd describes:
// in a group of 16 lanes G = lane / 16, lanes 4 j + c address piece c of row
// 16 c4 + 4 (G >> 1) + j + 8 r2, columns 32 dt + 16 (G & 1) + 4 c .. + 3):
// the piece is at line_v_tr(lane, dt & 1) + 4096 (dt >> 1) + 1024 c4 + 512 r2.
__device__ __forceinline__ int line_v_tr(int lane, int dt_odd) {
  const int G = lane >> 4, j = (lane >> 2) & 3, c = lane & 3;
  const int ri = 4 * (G >> 1) + j;
  return ri * 64 + 16 * (G & 1) + 8 * (c >> 1) + 4 * (c & 1) + 32 * (dt_odd ^ ((j >> 1) & 1));
}

// Transposed operand (dt, c4) of a V line tile; tr = line_v_tr(lane, dt & 1).
__device__ __forceinline__ bf16x8 read_tr_line(const bf16* tile, int c4, int dt, int tr) {
  const bf16* base = tile + 4096 * (dt >> 1) + 1024 * c4 + tr;
  const s16x4 lo = ds_read_tr(base);
  const s16x4 hi = ds_read_tr(base + 512);
  return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// Dual line tile (the backward's tiles, read both as rows and transposed):
// the line tile's blocks with f(r) = T[r & 7] ^ 2 ((r >> 3) & 1),
// T = 0 2 4 6 1 3 5 7. Row-operand reads: the 16 rows of a lane group hold a
// chunk in 16 distinct (row parity, slot) pairs; transposed reads: rows 2 and
// 3 of every 4 land in the other half of the row's slots (T differs in bit 2),
// so the 32 lanes of a ds_read_b64_tr_b16 cover all banks.
__device__ __forceinline__ int dual_t(int ri) {
  return ((ri & 1) << 1) | (((ri >> 1) & 1) << 2) | ((ri >> 2) & 1);
}

// Chunk that DMA lane `lane` moves into its slot (row lane >> 3 of the block).
__device__ __forceinline__ int dual_chunk(int lane, int blk_odd) {
  return (lane & 7) ^ dual_t(lane >> 3) ^ (2 * blk_odd);
}

// Row operand (t, kk): row 32 t + li, chunk 2 kk + hh (kk = 0..7) at
// dual_row_rd(lane, kk & 3) + 4096 (kk >> 2) + 2048 t.
__device__ __forceinline__ int dual_row_rd(int lane, int j) {
  const int li = lane & 31, hh = lane >> 5;
  const int f = dual_t(li & 7) ^ (2 * ((li >> 3) & 1));
  return ((li >> 3) * 512 + (li & 7) * 64 + (hh ^ f) * 8) ^ (16 * j);
}

// Transposed-read offsets (the pieces swz_tr_rd describes, rows 16 c4 +
// 4 (G >> 1) + j + 8 r2, columns 32 dt + 16 (G & 1) + 4 c .. + 3): the piece
// is at dual_tr_rd(lane, dt & 1, r2) + 4096 (dt >> 1) + 1024 c4 + 512 r2.
__device__ __forceinline__ int dual_tr_rd(int lane, int dt_odd, int r2) {
  const int G = lane >> 4, j = (lane >> 2) & 3, c = lane & 3;
  const int ri = 4 * (G >> 1) + j;
  const int chunk = 4 * dt_odd + 2 * (G & 1) + (c >> 1);
  return ri * 64 + 8 * (chunk ^ dual_t(ri) ^ (2 * r2)) + 4 * (c & 1);
}

// Transposed operand (dt, c4) of a dual line tile; tr[2 p + r2] =
// dual_tr_rd(lane, p, r2).
__device__ __forceinline__ bf16x8 read_tr_dual(const bf16* tile, int c4, int dt, const int* tr) {
  const bf16* base = tile + 4096 * (dt >> 1) + 1024 * c4;
  const s16x4 lo = ds_read_tr(base + tr[2 * (dt & 1)]);
  const s16x4 hi = ds_read_tr(base + 512 + tr[2 * (dt & 1) + 1]);
  return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// DMA of one wave's quarter of a dual line tile: blocks 4 g .. 4 g + 3 =
// d-half g >> 1, rows 32 (g & 1) + 8 i + (lane >> 3), i = 0..3. Whole tiles
// take a scalar row base per instruction and a 32-bit per-lane byte offset;
// a partial tile (nrows < 64, nrows >= 1) re-reads row nrows - 1 for the rows
// past it.
struct DualDma {
  int g;
  uint32_t off0, off1;  // lane_off(g, lane, rs, 0 / 1)

  __device__ __forceinline__ static int col(int g, int lane, int odd) {
    return 64 * (g >> 1) + 8 * dual_chunk(lane, odd);
  }
  // Per-lane byte offset from a block's first row: row lane >> 3, the chunk
  // of an even (odd = 0) or odd block.
  __device__ __forceinline__ static uint32_t lane_off(int g, int lane, int64_t rs, int odd) {
    return (uint32_t)((lane >> 3) * rs + col(g, lane, odd)) * 2u;
  }
  __device__ __forceinline__ void setup(int g_, int lane, int64_t rs) {
    g = g_;
    off0 = lane_off(g, lane, rs, 0);
    off1 = lane_off(g, lane, rs, 1);
  }
  __device__ __forceinline__ void issue(const bf16* base, int64_t rs, int nrows, bf16* tile,
                                        int lane) const {
    issue_quad(g, base, rs, nrows, tile, lane, off0, off1);
  }
  // The DMA itself, with the offsets given (kernels short of registers pass
  // lane_off(...) computed at the call instead of holding them).
  __device__ __forceinline__ static void issue_quad(int g, const bf16* base, int64_t rs, int nrows,
                                                    bf16* tile, int lane, uint32_t o0, uint32_t o1) {
    const int rw = 32 * (g & 1);
    if (nrows >= kTileRows) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        dma16_sv(base + (int64_t)(rw + 8 * i) * rs, (i & 1) ? o1 : o0, tile + (4 * g + i) * 512);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = min(rw + 8 * i + (lane >> 3), nrows - 1);
        dma16(base + (int64_t)r * rs + col(g, lane, i & 1), tile + (4 * g + i) * 512);
      }
    }
  }
};

// Wave-private row staging -----------------------------------------------------
//
// 32 rows x 128 bf16 (8 KB) per wave, 16-byte chunk c of row r at element
// r * 128 + ((c ^ (r & 15)) * 8). Rows move between HBM and the staging area
// 4 whole 256-byte rows per instruction (DMA in, 16-byte stores out), and
// lanes read or write them in the MFMA register layouts (lane li = lane % 32
// is row li) without bank conflicts: 16 lanes on one chunk of 16 rows hit 16
// distinct slots. Loading or storing the register layouts straight from HBM
// touches 32 rows x 16-32 B per instruction instead.

__device__ __forceinline__ int stage_at(int r, int c) { return r * 128 + ((c ^ (r & 15)) * 8); }

// DMA of rows row0 .. row0 + 31 (row stride rs) into the staging area; rows
// at or past nrows (>= 1) re-read row nrows - 1.
__device__ __forceinline__ void stage_rows_in(const bf16* base, int64_t rs, int row0, int nrows,
                                              int lane, const bf16* stage) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = 4 * i + (lane >> 4);
    const int row = min(row0 + r, nrows - 1);
    const int c = (lane & 15) ^ (r & 15);
    dma16(base + (int64_t)row * rs + 8 * c, stage + 512 * i);
  }
}

// Row operand kk of staged row li: elements 16 kk + 8 hh .. + 7.
__device__ __forceinline__ bf16x8 staged_operand(const bf16* stage, int lane, int kk) {
  const int li = lane & 31, hh = lane >> 5;
  return *reinterpret_cast<const bf16x8*>(stage + stage_at(li, 2 * kk + hh));
}

// Four 32x32 accumulators acc[dt] holding [d = 32 dt + 8 (r / 4) + 4 hh + r % 4]
// [row li] (register r), times scale, as bf16 rows into the staging area.
__device__ __forceinline__ void stage_acc_rows(const f32x16 (&acc)[4], float scale, int lane,
                                               bf16* stage) {
  const int li = lane & 31, hh = lane >> 5;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      const u32x2 w = {pack_bf16(acc[dt][4 * rq] * scale, acc[dt][4 * rq + 1] * scale),
                       pack_bf16(acc[dt][4 * rq + 2] * scale, acc[dt][4 * rq + 3] * scale)};
      *reinterpret_cast<u32x2*>(stage + stage_at(li, 4 * dt + rq) + 4 * hh) = w;
    }
}

// Staged rows r with row0 + r < nrows to base + (row0 + r) * rs.
__device__ __forceinline__ void stage_rows_out(bf16* base, int64_t rs, int row0, int nrows,
                                               int lane, const bf16* stage) {
  const int c = lane & 15;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = (lane >> 4) + 4 * i;
    const u32x4 v = *reinterpret_cast<const u32x4*>(stage + stage_at(r, c));
    if (row0 + r < nrows) st16_nt(base + (int64_t)(row0 + r) * rs + 8 * c, v);
  }
}

// Workgroups are dispatched round-robin over the 8 XCDs (block i on XCD
// i % 8). Remap so each XCD gets a contiguous range of logical blocks, whose
// shared K/V (or Q/dO) rows then stay in that XCD's L2.
__device__ __forceinline__ int xcd_remap(int bid, int total) {
  if ((total & 7) != 0) return bid;
  return (bid & 7) * (total >> 3) + (bid >> 3);
}

}  // namespace aa
