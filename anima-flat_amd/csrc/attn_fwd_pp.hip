// Flash-attention forward, non-causal, head_dim 128, bf16 in / fp32 accumulate,
// for gfx950 (CDNA4): v_mfma_f32_32x32x16_bf16 for both products. The kernel
// for short key ranges (aa_attn_fwd takes it when Sk is at most
// kPingPongMaxSk, attn_fwd.hip): its two phase-shifted wave groups hide more
// of a work item's fixed costs (Q in, first tiles, O out) than the one-wave-
// per-SIMD kernel of attn_fwd.hip, which is faster on long key ranges.
//
// Work decomposition
//   One workgroup = 8 waves = 256 queries of one (batch, head). Each wave
//   owns 32 queries for the whole kernel; K/V tiles of 64 keys are streamed
//   into a 4-stage LDS ring and shared by the 8 waves. The waves run in two
//   phase-shifted groups so that MFMA and softmax work overlap on every SIMD
//   (schedule at the kernel).
//
// Transposed formulation (per wave, per 64-key tile)
//   S^T = K Q^T   : A = K rows from the LDS line tile (32 keys x 16 d per
//                   MFMA), B = Q^T from registers (loaded once).
//   O^T += V^T P^T: A = V^T (32 d x 16 keys), read transposed from the LDS
//                   V rows, B = P^T from the S^T accumulators.
//   The 32x32 accumulator layout puts column j = lane%32 in every lane, with
//   rows 8*(r/4) + 4*(lane/32) + r%4 in register r. With queries as columns,
//   every lane holds one query: the softmax row max/sum are in-lane
//   reductions plus one v_permlane32_swap with the partner lane, and the
//   output rescale is a per-lane scalar multiply.
//
// K/V staging (tile_io.h): K and V rows are copied HBM -> LDS by DMA
//   (global_load_lds_dwordx4) into line tiles, blocks of 8 rows x 64 d that
//   one DMA instruction fills from 8 whole 128-byte lines; the 16-byte chunk
//   XOR differs: K's suits its 16-byte ds_read_b128 operand reads, V's its
//   V^T operands, pairs of ds_read_b64_tr_b16 transposed reads. Both are free
//   of bank conflicts.
//
// Q and O staging: each wave's 32 Q rows come in by DMA (4 rows x 256 B per
//   instruction) into ring stages that the first tiles do not use, and are
//   read into the Q^T registers from there; O leaves the same way, written to
//   free ring stages and stored 4 whole rows per instruction. (Loading and
//   storing straight from the accumulator layout touches 32 rows x 16-32 B
//   per instruction; staging cut the fixed cost of a round of work items by
//   about 5 us.)
//
// Key order of P^T
//   The B operand of the MFMA wants, in lane l, 8 consecutive k-indices
//   8*(l/32)+i of a 16-key chunk. The S^T accumulators hold, for that lane,
//   keys {4h..4h+3, 8+4h..8+4h+3} (h = l/32) of the chunk. Since PV sums over
//   keys, the V^T operand only has to list its keys in the same order, which
//   the transposed reads do by addressing those rows.
//
// Online softmax with lazy rescaling
//   The running max m is tracked on raw scores s = q.k; probabilities are
//   p = exp2(s*c - m*c) with c = scale * log2(e), one FMA and one v_exp_f32
//   per score. m is only raised when a tile's max exceeds it by more than
//   8/c (8 in log2 units), so p <= 256 and the O/l rescale (a pass over the
//   64 accumulator registers) runs only a few times per row. The row sums add
//   the fp32 probabilities: v_dot2c_f32_bf16 over the bf16 pairs stalls the
//   partner wave's MFMAs for about half an MFMA each.
#include <cmath>
#include <type_traits>

#include "attn_fwd.h"
#include "tile_io.h"

namespace aa {
namespace pp {

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// All but the newest n tiles of this wave's DMA complete (8 instructions per
// tile for a group-A wave: 4 K + 4 V). n is wave-uniform, 0..3.
__device__ __forceinline__ void wait_dma_tiles_in_flight(int n) {
  switch (n) {
    case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    case 1: asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
    case 2: asm volatile("s_waitcnt vmcnt(16)" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(24)" ::: "memory"); break;
  }
}

constexpr int kWaves = 8;    // two groups of 4, one wave of each group per SIMD
constexpr int kDmaWaves = 4; // group A issues every DMA
constexpr int kStages = 4;   // K/V ring depth (4 x 32 KB)
constexpr int kAhead = kStages - 2;  // tiles of DMA in flight beyond the next one
static_assert(kWaves * 32 == kQPerWg, "work item size");
constexpr int kDmaPerWave = 16 / kDmaWaves;  // 1 KB DMA blocks per group-A wave per tile, K and V each
static_assert(2 * kDmaPerWave == 8, "the DMA waits count 8 instructions per tile");

// K/V tile DMA of one group-A wave into K and V line tiles (tile_io.h). A DMA
// instruction fills one 1 KB block = 8 rows x 64 d from 8 whole 128-byte
// lines; wave w fills blocks 4 w .. 4 w + 3: d-half w >> 1, rows
// 32 (w & 1) + 8 i + (lane >> 3) for i = 0..3. Full tiles use a scalar row
// base per instruction and a 32-bit per-lane offset. Rows past klen (last
// tile only) re-read row klen-1: finite data whose scores are masked to
// -inf, so their P is 0.
struct KVDma {
  int b0, rw, rbase, kcol0, kcol1, vcol;  // rw: the wave's first row (uniform)
  uint32_t koff0, koff1, voff;

  __device__ __forceinline__ void setup(const FwdParams& p, int wave, int lane) {
    b0 = wave * kDmaPerWave;
    rw = 32 * (wave & 1);
    rbase = rw + (lane >> 3);
    const int h64 = 64 * (wave >> 1);
    kcol0 = h64 + 8 * line_k_chunk(lane, 0);
    kcol1 = h64 + 8 * line_k_chunk(lane, 1);
    vcol = h64 + 8 * line_v_chunk(lane);
    const int r = lane >> 3;
    koff0 = (uint32_t)(r * p.ks1 + kcol0) * 2u;
    koff1 = (uint32_t)(r * p.ks1 + kcol1) * 2u;
    voff = (uint32_t)(r * p.vs1 + vcol) * 2u;
  }

  // Tile t (keys 64 t ..) of the (batch, head) at kp / vp into kd / vd.
  __device__ __forceinline__ void issue(const FwdParams& p, const bf16* kp, const bf16* vp, int klen,
                                        int t, bf16* kd, bf16* vd) const {
    const int kb = t * kBN;
    static_assert(kDmaPerWave == 4, "four DMA blocks per wave per tile");
    if (kb + kBN <= klen) {
#pragma unroll
      for (int i = 0; i < kDmaPerWave; ++i) {
        const int row0 = kb + rw + 8 * i;
        dma16_sv(vp + (int64_t)row0 * p.vs1, voff, vd + (b0 + i) * 512);
      }
#pragma unroll
      for (int i = 0; i < kDmaPerWave; ++i) {
        const int row0 = kb + rw + 8 * i;
        dma16_sv(kp + (int64_t)row0 * p.ks1, (i & 1) ? koff1 : koff0, kd + (b0 + i) * 512);
      }
    } else {
#pragma unroll
      for (int i = 0; i < kDmaPerWave; ++i) {
        const int r = min(kb + rbase + 8 * i, klen - 1);
        dma16(vp + (int64_t)r * p.vs1 + vcol, vd + (b0 + i) * 512);
      }
#pragma unroll
      for (int i = 0; i < kDmaPerWave; ++i) {
        const int r = min(kb + rbase + 8 * i, klen - 1);
        dma16(kp + (int64_t)r * p.ks1 + ((i & 1) ? kcol1 : kcol0), kd + (b0 + i) * 512);
      }
    }
  }
};

// Per-wave state and work of the forward: 32 queries, their Q^T operands,
// O^T accumulators and running softmax statistics.
struct FwdWave {
  bf16x8 qreg[8];  // Q^T operand: lane holds Q[query li][16 kk + 8 hh + 0..7]
  f32x16 o[4];     // O^T, d = 32 dt + rows
  // Running max in raw score units (before the scale); l partial sums in
  // four independent chains.
  float m_raw;
  float l4[4];
  f32x16 s0, s1;  // S^T of the tile between its M and X blocks
  bf16x8 pb[4];   // P^T of the tile between its X block and the next M block
  int hh, li;
  int k_rd[4];  // line_k_rd(lane, j)
  int v_tr[2];  // line_v_tr(lane, dt & 1)
  float c, thr_raw;

  __device__ __forceinline__ void setup(int lane, float c_) {
    li = lane & 31;
    hh = lane >> 5;
    // K operand (kt, kk): row 32 kt + li, chunk 2 kk + hh of the K line tile
    // -> k_rd[kk & 3] + 4096 (kk >> 2) + 2048 kt. V^T operand (dt, c4): the
    // transposed read of the V line tile (tile_io.h), keys in the order of
    // the P^T B operands.
#pragma unroll
    for (int j = 0; j < 4; ++j) k_rd[j] = line_k_rd(lane, j);
    v_tr[0] = line_v_tr(lane, 0);
    v_tr[1] = line_v_tr(lane, 1);
    c = c_;
    thr_raw = kRescaleThreshold / c;
  }

  __device__ __forceinline__ void reset() {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[dt][r] = 0.f;
    m_raw = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) l4[i] = 0.f;
  }

  // Q rows of this wave's 32 queries (qrow0 ..) into its 8 KB of LDS
  // (tile_io.h row staging); rows past Sq re-read row Sq - 1 (their results
  // are never stored).
  __device__ __forceinline__ void dma_q(const FwdParams& p, const Item& it, int qrow0, int lane,
                                        const bf16* stage) const {
    stage_rows_in(p.q + it.b * p.qs0 + it.h * p.qs2, p.qs1, qrow0, p.Sq, lane, stage);
  }
  // Q^T operands from the staged rows: qreg[kk] = row li, chunk 2 kk + hh.
  __device__ __forceinline__ void read_q(const bf16* stage, int lane) {
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) qreg[kk] = staged_operand(stage, lane, kk);
  }

  // M block: up to 32 MFMAs in one unrolled stream, fed by a queue of LDS
  // operands read kPrefetch MFMAs ahead (sched_barrier fences pin the order):
  //   ops 0-15 : O^T += V^T P^T of the V tile vs, op = 4 c4 + dt (A operand:
  //              the transposed read of the V rows)
  //   ops 16-31: S^T = K Q^T of the K tile ks, op = 16 + 2 kk + kt (A operand:
  //              one 16-byte read of the K tile; two accumulator chains s0, s1)
  // PV / QK select which half runs (the first tile has no PV, the tail no QK).
  // A queue of 6 measured about 1% faster than 8, 10 or 12 at every shape
  // tried (4096x4096, 9216x9216, 4096x512, 1024x1024) and needs fewer VGPRs.
  template <bool PV, bool QK, int kPrefetch = 6>
  __device__ __forceinline__ void mblock(const bf16* vs, const bf16* ks) {
    constexpr int first = PV ? 0 : 16;
    constexpr int last = QK ? 32 : 16;
    if constexpr (QK) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s0[r] = 0.f;
        s1[r] = 0.f;
      }
    }
    bf16x8 q_ops[kPrefetch];
    auto load_op = [&](int op) -> bf16x8 {
      if (op < 16) return read_tr_line(vs, op >> 2, op & 3, v_tr[op & 1]);
      const int kk = (op - 16) >> 1, kt = (op - 16) & 1;
      return *reinterpret_cast<const bf16x8*>(ks + k_rd[kk & 3] + 4096 * (kk >> 2) + 2048 * kt);
    };
    auto run_op = [&](int op, bf16x8 a) {
      if (op < 16) {
        const int c4 = op >> 2, dt = op & 3;
        o[dt] = mfma32(a, pb[c4], o[dt]);
      } else {
        const int kk = (op - 16) >> 1, kt = (op - 16) & 1;
        if (kt == 0) s0 = mfma32(a, qreg[kk], s0);
        else s1 = mfma32(a, qreg[kk], s1);
      }
    };
#pragma unroll
    for (int i = first; i < last + kPrefetch; ++i) {
      // Consume slot (i - first) % kPrefetch before refilling it.
      if (i - kPrefetch >= first) run_op(i - kPrefetch, q_ops[(i - kPrefetch - first) % kPrefetch]);
      if (i < last) q_ops[(i - first) % kPrefetch] = load_op(i);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // Softmax of the tile at key offset kb: mask (last tile only), row max,
  // lazy rescale, P, sums.
  __device__ __forceinline__ void softmax(int kb, int klen) {
    if (kb + kBN > klen) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kb + 8 * (r >> 2) + 4 * hh + (r & 3);
        if (key >= klen) s0[r] = -INFINITY;
        if (key + 32 >= klen) s1[r] = -INFINITY;
      }
    }
    // Row max of the raw scores (two v_max3 chains), then over the lane pair.
    float ma = max3f(s0[0], s1[0], s0[1]);
    float mb = max3f(s1[1], s0[2], s1[2]);
#pragma unroll
    for (int r = 3; r < 15; r += 2) {
      ma = max3f(ma, s0[r], s1[r]);
      mb = max3f(mb, s0[r + 1], s1[r + 1]);
    }
    float mt = max3f(ma, mb, max2f(s0[15], s1[15]));
    mt = pair_max(mt);

    const bool need = mt > m_raw + thr_raw;
    if (__builtin_amdgcn_ballot_w64(need)) {
      const float mn = need ? mt : m_raw;
      const float alpha = fast_exp2((m_raw - mn) * c);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
#pragma unroll
      for (int i = 0; i < 4; ++i) l4[i] *= alpha;
      m_raw = mn;
    }

    // P^T = exp2(s c - m c) in bf16 as four 16-key B operands.
    const float mc = m_raw * c;
    float ef[4][8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      ef[0][i] = fast_exp2(fmaf(s0[i], c, -mc));
      ef[1][i] = fast_exp2(fmaf(s0[8 + i], c, -mc));
      ef[2][i] = fast_exp2(fmaf(s1[i], c, -mc));
      ef[3][i] = fast_exp2(fmaf(s1[8 + i], c, -mc));
#pragma unroll
      for (int c4 = 0; c4 < 4; ++c4) pb[c4][i] = (bf16)ef[c4][i];
    }
    // Row sums of the fp32 probabilities (one chain per 16-key chunk).
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) {
#pragma unroll
      for (int j = 0; j < 8; ++j) l4[c4] += ef[c4][j];
    }
  }

  // Partial result of one key range: O / l rounded to bf16 and the range's
  // LSE (fp32), for the combine pass (no padding correction here). `row` is
  // the (item, split) record; the wave holds queries qloc0 .. qloc0 + 31. The
  // rows leave like O in the epilogue (row staging, 4 whole 256-byte rows per
  // store). In fp32 the partials doubled the bytes a short forward writes and
  // its combine pass reads (config 1: 33.8 MB).
  __device__ __forceinline__ void store_partial(const FwdParams& p, int64_t row, int qloc0,
                                                int lane, bf16* stage) const {
    const float l_tot = pair_sum((l4[0] + l4[1]) + (l4[2] + l4[3]));
    const bool any = l_tot > 0.f;
    const float lse = any ? (m_raw * c + __log2f(l_tot)) * kLn2 : -INFINITY;
    const float scale = any ? 1.0f / l_tot : 0.f;
    stage_acc_rows(o, scale, lane, stage);
    stage_rows_out(p.part_o + row * kQPerWg * kD, kD, qloc0, kQPerWg, lane, stage);
    if (hh == 0) p.part_lse[row * kQPerWg + qloc0 + li] = lse;
  }

  // Normalise, optional padding correction, store O and LSE of queries
  // qrow0 .. qrow0 + 31. O goes out through this wave's 8 KB of LDS (tile_io.h
  // row staging), 4 whole 256-byte rows per store.
  __device__ __forceinline__ void epilogue(const FwdParams& p, const Item& it, int qrow0, int lane,
                                           bf16* stage) const {
    const int qrow = qrow0 + li;
    const float m_run = m_raw * c;
    const float l_run = (l4[0] + l4[1]) + (l4[2] + l4[3]);
    const float l_tot = pair_sum(l_run);
    const bool any = l_tot > 0.f;
    const float lse = any ? (m_run + __log2f(l_tot)) * kLn2 : -INFINITY;
    float scale = any ? 1.0f / l_tot : 0.f;
    if (p.ln_pad) scale *= 1.0f / (1.0f + expf(p.ln_pad[it.b] - lse));
    stage_acc_rows(o, scale, lane, stage);
    if (p.lse && hh == 0 && qrow < p.Sq) p.lse[((int64_t)it.b * p.H + it.h) * p.Sq + qrow] = lse;
    stage_rows_out(p.o + it.b * p.os0 + it.h * p.os2, p.os1, qrow0, p.Sq, lane, stage);
  }
};

// Phase-shifted ("ping-pong") schedule. Waves 0-3 (group A) and 4-7 (group B)
// run the same per-tile work, one phase apart:
//   M(j): O^T += V_{j-1}^T P_{j-1}^T (16 MFMA) and S_j^T = K_j Q^T (16 MFMA)
//   X(j): softmax of S_j -> P_j (exp, max, sums, rare rescale)
//   phase 2j  : A runs M(j), B runs X(j-1)
//   phase 2j+1: A runs X(j), B runs M(j)
// with a workgroup barrier between phases. Waves w and w+4 share a SIMD, so
// on every SIMD one wave is in an MFMA block while its partner is in a VALU
// block and the matrix and vector pipes overlap. Tile j sits in stage
// j % kStages; its DMA is issued at phase 2(j-kAhead)+1 and complete (wait +
// barrier) by the end of phase 2j-1; its K is read in phases 2j, 2j+1 and
// its V in 2j+2, 2j+3. Both groups run the same instruction stream,
// M(m) | barrier | X(m) | barrier; group B executes one extra barrier first
// (group A one extra at the end), which shifts B by exactly one phase. Only
// group A issues and waits for the DMA: tile m+kAhead at the start of its
// X(m), off the MFMA stream (the stage it overwrites held tile m-2, whose V
// group B last read in phase 2m-1), and tile m+1 is complete before the
// barrier that ends its X(m); the barriers order it for group B.
//
// One workgroup per work item (256 queries of one (batch, head)), or per
// key range of one of the last work items when they are split.
__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_fwd_pp_kernel(FwdParams p) {
  __shared__ __attribute__((aligned(1024))) bf16 kv_lds[kStages][2][kTileElems];

  int item_idx, split;
  block_item(p, item_idx, split);
  const Item it = decode_item(p, item_idx);
  // Key tiles [t0, t0 + ntiles) of the item.
  int t0 = 0, ntiles = it.ntiles;
  if (split >= 0) {
    const int per = (it.ntiles + p.nsplit - 1) / p.nsplit;
    t0 = min(split * per, it.ntiles);
    ntiles = min(per, it.ntiles - t0);
  }
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool group_a = wave < 4;
  const int lane = tid & 63;
  const int qloc = wave * 32 + (lane & 31);
  const int qrow = it.qblk * kQPerWg + qloc;

  FwdWave w;
  w.setup(lane, p.c);
  // Q rows staged in ring stages 2 and 3 (free until tile 2's DMA, which
  // group A issues after the first barrier that follows every wave's read).
  bf16* qstage = &kv_lds[2 + (wave >> 2)][0][0] + (wave & 3) * 4096;
  w.dma_q(p, it, qrow - (lane & 31), lane, qstage);
  w.reset();
  KVDma dma;
  dma.setup(p, wave, lane);
  const bf16* kp = p.k + it.b * p.ks0 + it.h * p.ks2;
  const bf16* vp = p.v + it.b * p.vs0 + it.h * p.vs2;
  auto issue_tile = [&](int t) {
    dma.issue(p, kp, vp, it.klen, t0 + t, kv_lds[t % kStages][0], kv_lds[t % kStages][1]);
  };

  static_assert(kAhead >= 1 && kAhead <= 4, "lookahead");
  auto wait_for_next = [&](int m) {  // tile m+1 complete; later issued tiles may be in flight
    const int last_issued = min(m + kAhead, ntiles - 1);
    wait_dma_tiles_in_flight(max(last_issued - (m + 1), 0));
  };
  if (group_a && ntiles > 0) {
    for (int t = 0; t < kAhead && t < ntiles; ++t) issue_tile(t);
    wait_for_next(-1);  // also the Q rows, issued before
  } else {
    wait_dma();
  }
  w.read_q(qstage, lane);
  __syncthreads();
  if (!group_a) __syncthreads();
  if (ntiles > 0) {
    w.mblock<false, true>(kv_lds[0][1], kv_lds[0][0]);
    __syncthreads();
    if (group_a && kAhead < ntiles) issue_tile(kAhead);
    w.softmax(t0 * kBN, it.klen);
    if (group_a) wait_for_next(0);
    __syncthreads();
    for (int m = 1; m < ntiles; ++m) {
      w.mblock<true, true>(kv_lds[(m - 1) % kStages][1], kv_lds[m % kStages][0]);
      __syncthreads();
      if (group_a && m + kAhead < ntiles) issue_tile(m + kAhead);
      w.softmax((t0 + m) * kBN, it.klen);
      if (group_a) wait_for_next(m);
      __syncthreads();
    }
    w.mblock<true, false>(kv_lds[(ntiles - 1) % kStages][1], kv_lds[0][0]);
  }
  if (group_a) __syncthreads();
  // Output staging: the two stages after the last tile's are free (group B
  // may still be reading the last tile's V in its final M block; nothing else
  // is read or in flight).
  bf16* stage = &kv_lds[(ntiles + (wave >> 2)) % kStages][0][0] + (wave & 3) * 4096;
  if (split < 0) w.epilogue(p, it, qrow - (lane & 31), lane, stage);
  else w.store_partial(p, (int64_t)(item_idx - p.full_blocks) * p.nsplit + split, wave * 32, lane, stage);
}

}  // namespace pp

void launch_attn_fwd_pp(const FwdParams& p, unsigned blocks, hipStream_t stream) {
  pp::attn_fwd_pp_kernel<<<dim3(blocks), pp::kWaves * 64, 0, stream>>>(p);
}

}  // namespace aa
