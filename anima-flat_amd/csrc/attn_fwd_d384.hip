// Flash-attention forward at head_dim 384, non-causal, bf16 in / fp32
// accumulate, for gfx950: the VAE decoder's mid-block attention (one head,
// S = (H/8)(W/8) tokens, 16384 at 1024x1024; src/vae.py:230-241, where it
// goes through ffpa_attn_func or SDPA).
//
// Work decomposition
//   One workgroup = 4 waves, one per SIMD, = 128 queries of one (batch,
//   head) over one key range. A wave owns 32 queries: their Q^T operands
//   (24 x 16 head-dim values, 96 VGPRs) and O^T accumulators (12 blocks of
//   32 d x 32 queries, 192 registers) stay in registers for the whole range,
//   which takes the whole register file of a SIMD, hence one wave per SIMD.
//   With B * H * S / 128 work items short of the CU count (128 items at
//   16384 tokens), the keys are split into ranges whose normalised partials
//   (bf16 O, fp32 LSE) attn_fwd_d384_combine_kernel merges.
//
// Per 32-key tile and wave: S^T = K Q^T is one 32x32 accumulator, 24
//   v_mfma_f32_32x32x16_bf16 over the head dimension (A = 16-byte reads of
//   the K rows in LDS, B = Q^T registers); O^T += V^T P^T is 12 d-blocks x 2
//   key chunks = 24 MFMAs (A = transposed ds_read_b64_tr_b16 reads of the V
//   rows, B = P^T from the S^T accumulator as it is, tile_io.h). The softmax
//   is 16 scores per lane per tile, a third of the d=128 kernel's VALU work
//   per MFMA, so a single wave can keep the matrix pipe busy if its VALU work
//   runs between its MFMAs: each tile is two phases of 24 slots, each slot one
//   MFMA plus a fixed slice of VALU work, held in place by sched_barrier and
//   by empty asm statements that anchor each slot's results (without them
//   the compiler sinks the softmax into phase 2, next to its MFMA users):
//     phase 1: S^T of tile t+1 (QK MFMAs) | P of tile t (fma, exp2, bf16,
//              row sums)
//     phase 2: O^T += V^T P^T of tile t   | row max of tile t+1
//   followed by the (rare) lazy rescale of O and l when tile t+1 raised a
//   row max by more than 8 in log2 units (as in the d=128 kernel).
//
// K/V staging: a 3-stage LDS ring of 48 KB stages (K and V of 32 keys as
//   three 32-row x 128 sub-tiles each: K in the row-tile format, V in the
//   swizzled one, tile_io.h), filled by DMA (global_load_lds_dwordx4). K of
//   tile t+3 and V of tile t+2 are issued during tile t, one DMA instruction
//   every four slots of both phases, so each half has two tiles of lead time;
//   waves 0-1 move K, waves 2-3 move V. A DMA instruction holds its wave
//   while the CU's load path is busy: with all 12 of a tile issued in
//   consecutive slots of phase 1 (the four waves at once), phase 1 took
//   ~2460 cycles for its 24 MFMAs against ~1150 for phase 2's; spread over
//   both phases, 434 -> 403 us at 16384 tokens (staggering the four waves'
//   slots instead was slower, 505 us).
#include <algorithm>
#include <cmath>
#include <string>
#include <type_traits>

#include "aa_common.h"
#include "attn_fwd_d384.h"
#include "tile_io.h"

namespace aa {
namespace d384 {

constexpr int kD = 384;
constexpr int kChunks = 3;                 // 128-wide head-dim chunks
constexpr int kBN = 32;                    // keys per tile
constexpr int kWaves = 4;                  // one per SIMD
constexpr int kQPerWg = kWaves * 32;       // 128 queries per work item
constexpr int kStages = 3;
constexpr int kSub = 4096;                 // 32 rows x 128 bf16 = 8 KB
constexpr int kStageElems = 2 * kChunks * kSub;  // K0 K1 K2 V0 V1 V2 = 48 KB
constexpr int kDmaPerTile = 12;            // DMA instructions per wave per K or V tile
constexpr int kMaxSplit = 8;
constexpr float kRescaleThreshold = 8.0f;  // log2 units
constexpr int kPf = 6;                     // operands read ahead of their MFMA
constexpr int kQA = 16;                    // Q^T operands kept in AGPRs (the rest in VGPRs)

struct Params {
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
  int H, Sq, Sk, nqblk, items, nsplit;
  float c;  // softmax_scale * log2(e)
  bf16* part_o;     // [items * nsplit][128][384] normalised partials, bf16
  float* part_lse;  // [items * nsplit][128]
};

// DMA blocks 4 g .. 4 g + 3 of a row tile (not swizzled) whose row 0 is at
// `base`: rows 16 g + (lane & 15), chunk 4 i + lq (lq = lane >> 4) for block
// 4 g + i, at element 2048 g + 512 i + 8 lane of the tile. Rows at or past
// nrows (>= 1) re-read row nrows - 1, finite data whose scores are masked.
__device__ __forceinline__ void dma_row_quad(const bf16* base, int64_t rs, int nrows,
                                             const bf16* lds_tile, int g, int lane) {
  const int row = min(16 * g + (lane & 15), nrows - 1);
  const bf16* src = base + (int64_t)row * rs + 8 * (lane >> 4);
  const bf16* dst = lds_tile + 4 * g * 512;
  dma16_off<0>(src, dst);
  dma16_off<64>(src, dst + 512);
  dma16_off<128>(src, dst + 1024);
  dma16_off<192>(src, dst + 1536);
}

// Every MFMA is the compiler's builtin, so that the compiler pads the hazards
// between an MFMA and the VALU code around it (a VALU write to an MFMA's
// source registers right after its issue corrupts its operands; the
// softmax work interleaved with the QK MFMAs sits exactly there). Register
// files are steered instead: O^T stays in AGPRs because its zeros, rescales
// and last reads are pinned there (Wave::setup, update_max, fence_o).
__device__ __forceinline__ void mfma_o(f32x16& acc, bf16x8 a, bf16x8 b) {
  acc = mfma32(a, b, acc);
}

// One tile's DMA work of one wave: three quads of 4 DMA instructions (16
// rows x 4 chunks of 8 columns each), issued one instruction per MFMA slot of
// phase 1. A wave with no tile left to move issues the same 12 instructions
// into a dummy LDS area instead, so that every wave issues exactly 12 per
// tile and one vmcnt(12) is the wait everywhere.
struct DmaJob {
  const bf16* src[3];  // this lane's global address of quad q (offsets 64 i bytes follow)
  const bf16* dst[3];  // LDS destination of quad q (blocks at + 512 i elements)

  template <int i>
  __device__ __forceinline__ void issue() const {
    dma16_off<64 * (i & 3)>(src[i >> 2], dst[i >> 2] + 512 * (i & 3));
  }
};

struct Item {
  int b, h, qblk, klen;
};

__device__ __forceinline__ Item decode_item(const Params& p, int it) {
  Item r;
  r.qblk = it % p.nqblk;
  const int bh = it / p.nqblk;
  r.b = bh / p.H;
  r.h = bh - r.b * p.H;
  r.klen = p.seqused ? max(0, min((int)p.seqused[r.b], p.Sk)) : p.Sk;
  return r;
}

struct Wave {
  bf16x8 qreg[24];  // Q^T: lane holds Q[query li][16 kk + 8 hh + 0..7]; kk < kQA in AGPRs
  f32x16 o[12];     // O^T block db: d = 32 db + 8 (r / 4) + 4 hh + r % 4
  f32x16 s;         // S^T of the current tile: key 8 (r / 4) + 4 hh + r % 4
  f32x16 sn;        // S^T of the next tile
  bf16x8 pb[2];     // P^T of the current tile, keys 0-15 and 16-31
  float m_raw;      // running row max in raw score units
  float mt;         // row max of the next tile (raw)
  f32x4 lsum;       // row sum of query li (all four elements), by MFMA
  bf16x8 sel;       // 0/1 selector: the A operand of the row-sum MFMA
  float c, thr_raw;
  int li, hh, k_rd, v_tr0, v_tr1;

  __device__ __forceinline__ void setup(int lane, float c_) {
    li = lane & 31;
    hh = lane >> 5;
    k_rd = row_rd(lane);
    v_tr0 = swz_tr_rd(lane, 0);
    v_tr1 = swz_tr_rd(lane, 1);
    c = c_;
    thr_raw = kRescaleThreshold / c;
    // Zeros pinned into AGPRs, the file every later MFMA keeps O in.
#pragma unroll
    for (int db = 0; db < 12; ++db) {
      o[db] = f32x16{};
      asm volatile("" : "+a"(o[db]));
    }
    m_raw = -INFINITY;
    lsum = f32x4{};
    // Row sums by v_mfma_f32_16x16x32_bf16 with the P^T operand as B: in that
    // shape lane l's 8 values are B[k = 8 (l / 16) + i][n = l % 16], i.e.
    // query n (+16 for odd l / 16) over one half of the chunk's keys. With
    // A[m][k] = 1 where bit 2 of m equals bit 3 of k, D[m][n] sums query n
    // for m % 8 < 4 and query n + 16 otherwise, which puts the row sum of
    // query li in all four D values of the lane. (v_dot2c_f32_bf16 over the
    // bf16 pairs would stall the matrix pipe for about half an MFMA each.)
    const bf16 one = (bf16)(((lane & 15) >> 2 & 1) == ((lane >> 4) & 1) ? 1.0f : 0.0f);
#pragma unroll
    for (int i = 0; i < 8; ++i) sel[i] = one;
  }

  // Operand reads address LDS as one pinned 32-bit byte base per tile (two
  // for the transposed V^T reads) plus compile-time offsets, which fold into
  // the instructions' immediate field; computed per operand, the addresses
  // would take a VGPR each and push the Q^T operands out to scratch.
  //
  // K operand kk (head-dim 16 kk .. 16 kk + 15) of the tile whose K starts at
  // byte address kb: sub-tile kk / 8, chunk pair kk % 8.
  template <int kk>
  __device__ __forceinline__ bf16x8 k_op(uint32_t kb) const {
    return lds_ld16(kb + 2 * ((kk >> 3) * kSub + 256 * (kk & 7)));
  }
  __device__ __forceinline__ uint32_t k_base(const bf16* kst) const {
    uint32_t b = lds_addr(kst + k_rd);
    asm volatile("" : "+v"(b));
    return b;
  }
  // V^T operand of PV op i (d-block db = i % 12, key chunk c4 = i / 12) of the
  // tile whose V starts at vst: bases vb0 / vb1 of the two transposed reads.
  template <int i>
  __device__ __forceinline__ bf16x8 v_op(uint32_t vb0, uint32_t vb1) const {
    constexpr int db = i % 12, c4 = i / 12;
    constexpr uint32_t off = 2 * ((db >> 2) * kSub + 2048 * c4 + 512 * (db & 3));
    const s16x4 lo = lds_ld8_tr(vb0 + off);
    const s16x4 hi = lds_ld8_tr(vb1 + off);
    return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  }
  __device__ __forceinline__ void v_bases(const bf16* vst, uint32_t& vb0, uint32_t& vb1) const {
    vb0 = lds_addr(vst + v_tr0);
    vb1 = lds_addr(vst + v_tr1);
    asm volatile("" : "+v"(vb0), "+v"(vb1));
  }

  // S^T of a tile without interleaved work (the first tile of a range).
  __device__ __forceinline__ void qk_plain(const bf16* kst, f32x16& acc) {
    bf16x8 q[kPf];
    const uint32_t kb = k_base(kst);
    static_for<0, 24 + kPf>([&](auto I) {
      constexpr int i = decltype(I)::value;
      if constexpr (i >= kPf) {
        constexpr int op = i - kPf;
        acc = mfma32(q[op % kPf], qreg[op], op == 0 ? f32x16{} : acc);
      }
      if constexpr (i < 24) q[i % kPf] = this->template k_op<i>(kb);
      __builtin_amdgcn_sched_barrier(0);
    });
  }

  // Keeps O in AGPRs up to this point and orders the VALU code that follows
  // after every MFMA that wrote it.
  __device__ __forceinline__ void fence_o() {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3"
                 : "+a"(o[0]), "+a"(o[1]), "+a"(o[2]), "+a"(o[3]), "+a"(o[4]), "+a"(o[5]),
                   "+a"(o[6]), "+a"(o[7]), "+a"(o[8]), "+a"(o[9]), "+a"(o[10]), "+a"(o[11]));
  }

  // Scores of keys at or past klen (tile at key offset kb) to -inf.
  __device__ __forceinline__ void mask(f32x16& acc, int kb, int klen) const {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = kb + 8 * (r >> 2) + 4 * hh + (r & 3);
      if (key >= klen) acc[r] = -INFINITY;
    }
  }

  __device__ __forceinline__ float row_max(const f32x16& a) const {
    float ma = max3f(a[0], a[1], a[2]);
    float mb = max3f(a[3], a[4], a[5]);
    ma = max3f(ma, a[6], a[7]);
    mb = max3f(mb, a[8], a[9]);
    ma = max3f(ma, a[10], a[11]);
    mb = max3f(mb, a[12], a[13]);
    return pair_max(max3f(ma, mb, max2f(a[14], a[15])));
  }

  // Phase 1: S^T of the next tile (kst, skipped when QK is false) with P of
  // the current tile s -> pb and the row sums in the same slots.
  template <bool QK>
  __device__ __forceinline__ void phase1(const bf16* kst, const DmaJob& job) {
    const float mc = m_raw * c;
    bf16x8 q[kPf];
    float pf = 0.f;
    const uint32_t kb = QK ? k_base(kst) : 0u;
    static_for<0, 24 + kPf>([&](auto I) {
      constexpr int i = decltype(I)::value;
      if constexpr (QK && i >= kPf) {
        constexpr int op = i - kPf;
        sn = mfma32(q[op % kPf], qreg[op], op == 0 ? f32x16{} : sn);
      }
      if constexpr (QK && i < 24) q[i % kPf] = this->template k_op<i>(kb);
      if constexpr (QK && i % 4 == 2 && i / 4 < kDmaPerTile / 2) job.template issue<i / 4>();
      // P: one score per slot for slots 0-15, packed and summed in pairs.
      if constexpr (i < 16) {
        const float e = fast_exp2(fmaf(s[i], c, -mc));
        if constexpr ((i & 1) == 0) {
          pf = e;
        } else {
          pb[i >> 3][(i & 7) - 1] = (bf16)pf;
          pb[i >> 3][i & 7] = (bf16)e;
          // Anchored in this slot: left alone, the compiler sinks the whole
          // P computation into phase 2, next to its MFMA users, where it
          // stalls them instead of overlapping phase 1's.
          asm volatile("" : "+v"(pb[i >> 3]));
        }
      }
      // The row sums of a finished P^T operand (16 keys), on the matrix pipe.
      if constexpr (i == 8 || i == 16) {
        lsum = __builtin_amdgcn_mfma_f32_16x16x32_bf16(sel, pb[(i >> 3) - 1], lsum, 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    });
  }

  // Phase 2: O^T += V^T P^T of the current tile (vst) with the row max of the
  // next tile sn (when MAX) in the first slots.
  template <bool MAX>
  __device__ __forceinline__ void phase2(const bf16* vst, const DmaJob& job) {
    bf16x8 q[kPf];
    float ma = 0.f, mb = 0.f;
    uint32_t vb0, vb1;
    v_bases(vst, vb0, vb1);
    static_for<0, 24 + kPf>([&](auto I) {
      constexpr int i = decltype(I)::value;
      if constexpr (i >= kPf) {
        constexpr int op = i - kPf;
        constexpr int db = op % 12, c4 = op / 12;
        mfma_o(o[db], q[op % kPf], pb[c4]);
      }
      if constexpr (i < 24) q[i % kPf] = this->template v_op<i>(vb0, vb1);
      if constexpr (i % 4 == 2 && i / 4 < kDmaPerTile / 2) job.template issue<kDmaPerTile / 2 + i / 4>();
      if constexpr (MAX) {
        if constexpr (i == kPf) {
          ma = max3f(sn[0], sn[1], sn[2]);
          mb = max3f(sn[3], sn[4], sn[5]);
        } else if constexpr (i == kPf + 2) {
          ma = max3f(ma, sn[6], sn[7]);
          mb = max3f(mb, sn[8], sn[9]);
        } else if constexpr (i == kPf + 4) {
          ma = max3f(ma, sn[10], sn[11]);
          mb = max3f(mb, sn[12], sn[13]);
        } else if constexpr (i == kPf + 6) {
          mt = pair_max(max3f(ma, mb, max2f(sn[14], sn[15])));
        }
        asm volatile("" : "+v"(ma), "+v"(mb));
      }
      __builtin_amdgcn_sched_barrier(0);
    });
  }

  // Lazy rescale for the next tile's max mt (after its PV-free phase 2).
  __device__ __forceinline__ void update_max() {
    const bool need = mt > m_raw + thr_raw;
    if (__builtin_amdgcn_ballot_w64(need)) {
      const float mn = need ? mt : m_raw;
      const float alpha = fast_exp2((m_raw - mn) * c);
      fence_o();
      // One accumulator block at a time, pinned back into AGPRs: otherwise the
      // compiler reads all 192 values into VGPRs first and spills.
#pragma unroll
      for (int db = 0; db < 12; ++db) {
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
        asm volatile("" : "+a"(o[db]));
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) lsum[r] *= alpha;
      m_raw = mn;
    }
  }

  __device__ __forceinline__ float row_sum() const { return lsum[0]; }
};

// Block -> (item, split): logical index L = xcd_remap(block) runs split-major,
// so the workgroups of one XCD take consecutive query blocks of one key range
// and share its K/V tiles in that XCD's L2.
__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(1, 1)))
void attn_fwd_d384_kernel(Params p) {
  // The ring, then 4 KB that DMAs with nothing to move write into.
  __shared__ __attribute__((aligned(1024))) bf16 lds[kStages * kStageElems + 2048];
  const bf16* dummy = lds + kStages * kStageElems;

  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int split = L / p.items;
  const int item = L - split * p.items;
  const Item it = decode_item(p, item);
  const int ntiles_all = (it.klen + kBN - 1) / kBN;
  const int per = (ntiles_all + p.nsplit - 1) / p.nsplit;
  const int t0 = min(split * per, ntiles_all);
  const int n = min(per, ntiles_all - t0);

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int qrow0 = it.qblk * kQPerWg + wave * 32;

  Wave w;
  w.setup(lane, p.c);

  const bf16* kp = p.k + it.b * p.ks0 + it.h * p.ks2;
  const bf16* vp = p.v + it.b * p.vs0 + it.h * p.vs2;
  auto stage = [&](int t) -> bf16* { return lds + (t % kStages) * kStageElems; };
  const bool k_mover = wave < 2;
  // DMA job of tile t: K (waves 0-1, row tile) or V (waves 2-3, swizzled row
  // tile), 3 quads per wave: quad x = 0..5 of the tensor covers chunk x / 2,
  // row group x % 2. Rows past the tile's keys re-read its last key (their
  // scores are masked). t >= n gives the dummy job.
  auto job_of = [&](int t) -> DmaJob {
    DmaJob j;
    const int lq = lane >> 4;
#pragma unroll
    for (int qd = 0; qd < 3; ++qd) {
      if (t >= n) {
        j.src[qd] = kp + 8 * lq;
        j.dst[qd] = dummy;
        continue;
      }
      const int kb = (t0 + t) * kBN;
      const int nrows = it.klen - kb;
      const int x = 3 * (k_mover ? wave : wave - 2) + qd;
      const int g = x & 1;
      const int r = k_mover ? (lane & 15) : ((lane & 15) ^ (4 * lq));
      const int row = min(16 * g + r, nrows - 1);
      const bf16* base = k_mover ? kp + (int64_t)kb * p.ks1 : vp + (int64_t)kb * p.vs1;
      const int64_t rs = k_mover ? p.ks1 : p.vs1;
      j.src[qd] = base + (int64_t)row * rs + 128 * (x >> 1) + 8 * lq;
      j.dst[qd] = stage(t) + ((k_mover ? 0 : kChunks) + (x >> 1)) * kSub + 4 * g * 512;
    }
    return j;
  };
  auto issue_now = [&](int t) {
    const DmaJob j = job_of(t);
    static_for<0, 12>([&](auto I) { j.template issue<decltype(I)::value>(); });
  };

  // Q rows of this wave, three 128-wide chunks, staged in ring stages 1-2
  // (free until tile 1's DMA, issued after the barrier that follows every
  // wave's read); tile 0 into stage 0.
  bf16* qst = lds + kStageElems + wave * (kChunks * 4096);
  const bf16* qbase = p.q + it.b * p.qs0 + it.h * p.qs2;
#pragma unroll
  for (int j = 0; j < kChunks; ++j)
    stage_rows_in(qbase + 128 * j, p.qs1, qrow0, p.Sq, lane, qst + j * 4096);
  if (n > 0) issue_now(0);
  wait_dma();
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kChunks; ++j)
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      w.qreg[8 * j + kk] = staged_operand(qst + j * 4096, lane, kk);
      if (8 * j + kk < kQA) asm volatile("" : "+a"(w.qreg[8 * j + kk]));
    }
  __syncthreads();

  if (n > 0) {
    // Lead: K of tiles 1, 2 and V of tile 1 (or dummy jobs).
    issue_now(1);
    if (k_mover) issue_now(2);
    w.qk_plain(stage(0), w.s);
    const int kb0 = t0 * kBN;
    if (kb0 + kBN > it.klen) w.mask(w.s, kb0, it.klen);
    w.m_raw = w.row_max(w.s);

    // Tile t needs K of tile t+1 (QK) and V of tile t (PV). Every wave issues
    // one job of 12 DMAs per tile, K movers three tiles ahead and V movers
    // two, so at the top of tile t exactly one job (the last) may still be
    // in flight; the barrier then publishes every wave's. The job issued in
    // tile t, K of t+3 / V of t+2, reuses the K half of tile t's stage (its
    // QK ran in tile t-1) / the V half of tile t-1's (its PV ran in tile t-1).
    // The last tile runs the same body (one code path through the loop keeps
    // the accumulators in place): its QK of a tile n reads stale LDS and is
    // discarded, and neither the mask nor the max update runs for it.
    for (int t = 0; t < n; ++t) {
      asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
      __syncthreads();
      const DmaJob job = job_of(k_mover ? t + 3 : t + 2);
      w.phase1<true>(stage(t + 1), job);
      const bool more = t + 1 < n;
      const int kbn = (t0 + t + 1) * kBN;
      if (more && kbn + kBN > it.klen) w.mask(w.sn, kbn, it.klen);
      w.phase2<true>(stage(t) + kChunks * kSub, job);
      if (more) w.update_max();
      w.s = w.sn;
    }
  }
  wait_dma();  // no DMA may land in LDS after the workgroup ends

  // Output: O / l (and the padding correction), or the range's partial.
  w.fence_o();
  const float l_tot = w.row_sum();
  const bool any = l_tot > 0.f;
  const float lse = any ? (w.m_raw * w.c + __log2f(l_tot)) * kLn2 : -INFINITY;
  float scale = any ? 1.0f / l_tot : 0.f;
  // O rows (or the range's partial O, normalised like O and rounded to bf16,
  // with its LSE in fp32) leave through LDS row staging, 4 whole 256-byte rows
  // per store.
  const bool partial = p.nsplit > 1;
  const int64_t rec = (int64_t)item * p.nsplit + split;
  if (!partial && p.ln_pad) scale *= 1.0f / (1.0f + expf(p.ln_pad[it.b] - lse));
  __syncthreads();  // every wave is done with the ring
  bf16* st = lds + wave * 4096;
  bf16* obase = partial ? p.part_o + rec * kQPerWg * kD : p.o + it.b * p.os0 + it.h * p.os2;
  const int64_t ors = partial ? (int64_t)kD : p.os1;
  const int orow0 = partial ? wave * 32 : qrow0;
  const int onrows = partial ? kQPerWg : p.Sq;
#pragma unroll
  for (int j = 0; j < kChunks; ++j) {
    const f32x16 oj[4] = {w.o[4 * j], w.o[4 * j + 1], w.o[4 * j + 2], w.o[4 * j + 3]};
    stage_acc_rows(oj, scale, lane, st);
    stage_rows_out(obase + 128 * j, ors, orow0, onrows, lane, st);
  }
  if (partial) {
    if (w.hh == 0) p.part_lse[rec * kQPerWg + wave * 32 + w.li] = lse;
  } else {
    const int qrow = qrow0 + w.li;
    if (p.lse && w.hh == 0 && qrow < p.Sq) p.lse[((int64_t)it.b * p.H + it.h) * p.Sq + qrow] = lse;
  }
}

// Merges the key-range partials: 4 queries per workgroup, 48 lanes per query
// with 8 head-dim values (16 bytes) each. O = sum_s exp(lse_s - lse) O_s with
// lse = log sum_s exp(lse_s), then the optional padding correction.
constexpr int kCombineQ = 4;  // queries per combine workgroup
__global__ __launch_bounds__(192) void attn_fwd_d384_combine_kernel(Params p) {
  const int gq = blockIdx.x * kCombineQ + (int)threadIdx.x / 48;  // item * 128 + local query
  const int item = gq / kQPerWg, qloc = gq - item * kQPerWg;
  if (item >= p.items) return;
  const Item it = decode_item(p, item);
  const int qrow = it.qblk * kQPerWg + qloc;
  if (qrow >= p.Sq) return;
  const int d0 = 8 * ((int)threadIdx.x % 48);
  const int64_t rec0 = (int64_t)item * p.nsplit;
  // Every load goes out before any is used (one memory round trip).
  u32x4 raw[kMaxSplit];
#pragma unroll
  for (int s = 0; s < kMaxSplit; ++s)
    if (s < p.nsplit) raw[s] = ld16(p.part_o + ((rec0 + s) * kQPerWg + qloc) * kD + d0);
  float ls[kMaxSplit];
  float mx = -INFINITY;
#pragma unroll
  for (int s = 0; s < kMaxSplit; ++s) {
    ls[s] = s < p.nsplit ? p.part_lse[(rec0 + s) * kQPerWg + qloc] : -INFINITY;
    mx = fmaxf(mx, ls[s]);
  }
  float lse = -INFINITY;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (mx > -INFINITY) {
    float sum = 0.f;
#pragma unroll
    for (int s = 0; s < kMaxSplit; ++s) sum += expf(ls[s] - mx);
    lse = mx + logf(sum);
#pragma unroll
    for (int s = 0; s < kMaxSplit; ++s)
      if (s < p.nsplit && ls[s] > -INFINITY) {
        const float wgt = expf(ls[s] - lse);
        float v[8];
        unpack8(raw[s], v);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = fmaf(wgt, v[i], acc[i]);
      }
  }
  float scale = 1.f;
  if (p.ln_pad) scale = 1.0f / (1.0f + expf(p.ln_pad[it.b] - lse));
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] *= scale;
  bf16* op = p.o + it.b * p.os0 + (int64_t)qrow * p.os1 + it.h * p.os2 + d0;
  st16_nt(op, pack8(acc));
  if (p.lse && d0 == 0) p.lse[((int64_t)it.b * p.H + it.h) * p.Sq + qrow] = lse;
}

// Key split: ranges per work item so that items x ranges fills the CUs
// without exceeding them (one round), at most 8, each of at least 4 tiles.
// items x ranges <= ncu bounds the partials at ncu x 128 x (384 bf16 + 1 float).
static int plan_split(int64_t items, int64_t Sk, int ncu) {
  if (items <= 0 || ncu <= 0 || 2 * items > ncu) return 1;
  const int64_t tiles = (Sk + kBN - 1) / kBN;
  int64_t ns = ncu / items;
  ns = std::min<int64_t>(ns, kMaxSplit);
  ns = std::min<int64_t>(ns, std::max<int64_t>(tiles / 4, 1));
  return (int)std::max<int64_t>(ns, 1);
}

static int64_t items_of(int64_t B, int64_t Sq, int64_t H) {
  return B * H * ((Sq + kQPerWg - 1) / kQPerWg);
}

static size_t partial_bytes(int64_t items, int nsplit) {
  if (nsplit <= 1) return 0;
  return (size_t)items * nsplit * kQPerWg * (kD * sizeof(bf16) + sizeof(float));  // bf16 O, fp32 LSE
}

}  // namespace d384

size_t attn_fwd_d384_workspace(int64_t B, int64_t Sq, int64_t Sk, int64_t H, int ncu) {
  if (B <= 0 || Sq <= 0 || Sk <= 0 || H <= 0) return 0;
  const int64_t items = d384::items_of(B, Sq, H);
  return d384::partial_bytes(items, d384::plan_split(items, Sk, ncu));
}

static bool strides_ok(const int64_t* s) { return s[0] % 8 == 0 && s[1] % 8 == 0 && s[2] % 8 == 0; }

int attn_fwd_d384(const aa_attn_fwd_args* a, int ncu, hipStream_t stream) {
  using namespace d384;
  if (a->B < 0 || a->Sq < 0 || a->Sk < 0 || a->H <= 0) return fail(AA_EINVAL, "attn_fwd: negative size");
  if (a->B == 0 || a->Sq == 0) return AA_OK;
  // Sk == 0 is accepted as at head_dim 128: every work item has an empty key
  // range, reads no K/V and writes O = 0, LSE = -inf.
  if (!a->q || !a->out || (a->Sk > 0 && (!a->k || !a->v)))
    return fail(AA_EINVAL, "attn_fwd: null tensor");
  if (a->ln_pad && !a->seqused_k) return fail(AA_EINVAL, "attn_fwd: ln_pad needs seqused_k");
  if (!(a->softmax_scale > 0.f) || !std::isfinite(a->softmax_scale))
    return fail(AA_EINVAL, "attn_fwd: softmax_scale must be positive and finite");
  if (!aligned16(a->q) || !aligned16(a->k) || !aligned16(a->v) || !aligned16(a->out))
    return fail(AA_EINVAL, "attn_fwd: tensors must be 16-byte aligned");
  if (!strides_ok(a->q_stride) || !strides_ok(a->k_stride) || !strides_ok(a->v_stride) ||
      !strides_ok(a->out_stride))
    return fail(AA_EINVAL, "attn_fwd: batch/seq/head strides must be multiples of 8 elements");
  if (a->Sq > (1 << 30) || a->Sk > (1 << 30) || a->H > 65535 || a->B > 65535)
    return fail(AA_EUNSUPPORTED, "attn_fwd: size out of range");
  const int64_t items = items_of(a->B, a->Sq, a->H);
  const int nsplit = plan_split(items, a->Sk, ncu);
  if (items * nsplit > (int64_t)1 << 31) return fail(AA_EUNSUPPORTED, "attn_fwd: too many work items");
  const size_t need = partial_bytes(items, nsplit);
  if (need > 0 && (!a->workspace || a->workspace_bytes < need))
    return fail(AA_EINVAL, "attn_fwd: workspace too small (aa_attn_fwd_workspace)");
  if (need > 0 && !aligned16(a->workspace))
    return fail(AA_EINVAL, "attn_fwd: workspace must be 16-byte aligned");

  Params p;
  p.q = (const bf16*)a->q;
  p.k = (const bf16*)a->k;
  p.v = (const bf16*)a->v;
  p.o = (bf16*)a->out;
  p.lse = a->lse;
  p.seqused = a->seqused_k;
  p.ln_pad = a->ln_pad;
  p.qs0 = a->q_stride[0]; p.qs1 = a->q_stride[1]; p.qs2 = a->q_stride[2];
  p.ks0 = a->k_stride[0]; p.ks1 = a->k_stride[1]; p.ks2 = a->k_stride[2];
  p.vs0 = a->v_stride[0]; p.vs1 = a->v_stride[1]; p.vs2 = a->v_stride[2];
  p.os0 = a->out_stride[0]; p.os1 = a->out_stride[1]; p.os2 = a->out_stride[2];
  p.H = (int)a->H;
  p.Sq = (int)a->Sq;
  p.Sk = (int)a->Sk;
  p.nqblk = (int)((a->Sq + kQPerWg - 1) / kQPerWg);
  p.items = (int)items;
  p.nsplit = nsplit;
  p.c = a->softmax_scale * kLog2e;
  p.part_o = need > 0 ? (bf16*)a->workspace : nullptr;
  p.part_lse = need > 0 ? (float*)(p.part_o + (size_t)items * nsplit * kQPerWg * kD) : nullptr;

  attn_fwd_d384_kernel<<<dim3((unsigned)(items * nsplit)), kWaves * 64, 0, stream>>>(p);
  if (int rc = check_launch("attn_fwd d384")) return rc;
  if (nsplit > 1) {
    attn_fwd_d384_combine_kernel<<<dim3((unsigned)(items * kQPerWg / kCombineQ)), 192, 0, stream>>>(p);
    return check_launch("attn_fwd d384 combine");
  }
  return AA_OK;
}

}  // namespace aa
