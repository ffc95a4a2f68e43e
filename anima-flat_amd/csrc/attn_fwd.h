// Shared by the two head_dim-128 forward kernels (attn_fwd.hip: one wave per
// SIMD, 64 queries per wave; attn_fwd_pp.hip: two phase-shifted waves per
// SIMD, 32 queries per wave): the launch parameters, the work item of 256
// queries of one (batch, head) and its decoding, and the split-partial layout
// that attn_fwd_combine_kernel merges for both.
#pragma once

#include "tile_io.h"

namespace aa {

constexpr int kD = 128;
constexpr int kBN = 64;                    // keys per tile
constexpr float kRescaleThreshold = 8.0f;  // log2 units
constexpr int kQPerWg = 256;               // queries per work item

struct FwdParams {
  const bf16* q;
  const bf16* k;
  const bf16* v;
  bf16* o;
  float* lse;
  const int32_t* seqused;
  const float* ln_pad;
  int64_t qs0, qs1, qs2;
  int64_t ks0, ks1, ks2;
  int64_t vs0, vs1, vs2;
  int64_t os0, os1, os2;
  int H, Sq, Sk, nqblk, total_blocks;
  float c;  // softmax_scale * log2(e)
  // Key split of the last work items (see split_plan): blocks past full_blocks
  // each take one of nsplit key ranges of work item full_blocks + j / nsplit
  // and write normalised partials (part_o [j][split][256][128] bf16,
  // part_lse [j][split][256] fp32) that attn_fwd_combine_kernel merges.
  int full_blocks, split_items, nsplit;
  // Workgroups resident at once (one per CU): the unsplit blocks are mapped
  // to work items round by round (see attn_fwd_kernel).
  int round_blocks;
  bf16* part_o;
  float* part_lse;
};

// (batch, head, query block) of one work item; klen keys attended.
struct Item {
  int b, h, qblk, klen, ntiles;
};

__device__ __forceinline__ Item decode_item(const FwdParams& p, int it) {
  Item r;
  r.qblk = it % p.nqblk;
  const int bh = it / p.nqblk;
  r.b = bh / p.H;
  r.h = bh - r.b * p.H;
  r.klen = p.seqused ? min((int)p.seqused[r.b], p.Sk) : p.Sk;
  r.ntiles = r.klen > 0 ? (r.klen + kBN - 1) / kBN : 0;
  return r;
}

// Block -> (work item, key range): blocks start in index order, so block
// r R + j (R = round_blocks) runs in round r and takes an item of that
// round's range [r R, r R + R), XCD-aware within the round (the query blocks
// of one head share an XCD and its L2). Mapping over the whole grid instead
// would mix items of every batch into each round, and with per-batch key
// lengths (seqused) every round would then last as long as its longest item.
// Blocks past full_blocks take key range `split` of a split item.
__device__ __forceinline__ void block_item(const FwdParams& p, int blk, int& item_idx, int& split) {
  split = -1;
  if (blk < p.full_blocks) {
    const int r = blk / p.round_blocks;
    const int j = blk - r * p.round_blocks;
    const int in_round = min(p.round_blocks, p.full_blocks - r * p.round_blocks);
    item_idx = r * p.round_blocks + xcd_remap(j, in_round);
  } else {
    const int j = blk - p.full_blocks;
    item_idx = p.full_blocks + j / p.nsplit;
    split = j - (j / p.nsplit) * p.nsplit;
  }
}

__device__ __forceinline__ void block_item(const FwdParams& p, int& item_idx, int& split) {
  block_item(p, (int)blockIdx.x, item_idx, split);
}

// Launches the two-group kernel of attn_fwd_pp.hip over `blocks` workgroups.
void launch_attn_fwd_pp(const FwdParams& p, unsigned blocks, hipStream_t stream);

}  // namespace aa
