// Flash-attention backward, non-causal, head_dim 128, bf16 in / fp32 accumulate,
// for gfx950 (v_mfma_f32_32x32x16_bf16). Deterministic: no atomics, every
// reduction in a fixed order.
//
//   z = scale * q k^T, P = softmax(z) (recomputed from the forward LSE),
//   dV = P^T dO, dP = dO V^T, dZ = P o (dP - D) with D = rowsum(dO o O),
//   dK = scale * dZ^T Q, dQ = scale * dZ K.
//
// Two kernels, launched in this order:
// 1. dq_kernel: 8 waves x 32 queries per workgroup, two groups one phase
//    apart; streams 64-key tiles (K rows, V rows: 32 KB) and reads K^T from
//    the K rows with transposed LDS reads (dQ leaves through LDS row
//    staging). Queries are the columns:
//      S^T = K Q^T, dP^T = V dO^T, dQ^T += K^T dZ^T.
//    Each query's lse * log2(e) and -D (D = rowsum(dO o O), from the dO^T
//    operands it holds and one read of O) it computes itself and writes to a
//    1 KB stats record per 64 queries for the second kernel.
// 2. a dK/dV kernel: by default dkdv1w_kernel (attn_bwd_dkdv.hip: one wave
//    per SIMD doing both roles below for its 32 keys, slot-pinned), or with
//    AA_DKDV_KERNEL=2role this file's dkdv_kernel, described here:
//    8 waves, 128 keys per workgroup (32 per wave pair, split
//    by role, the roles one phase apart, at the kernel); streams 64-query
//    tiles (Q rows, dO rows, stats: 33 KB) into LDS by DMA and reads Q^T and
//    dO^T from the same rows with transposed LDS reads. Keys are the
//    accumulator columns (lane % 32), K and V sit in registers (read once
//    from rows staged in LDS; dK and dV leave through LDS the same way):
//      S  = Q K^T        A = Q rows (LDS),  B = K^T (registers)
//      dP = dO V^T       A = dO rows (LDS), B = V^T (registers)
//      dV^T += dO^T P    A = dO^T (LDS),    B = P from the S accumulators
//      dK^T += Q^T dZ    A = Q^T (LDS),     B = dZ from the accumulators
// The transposed reads list the keys / queries of each 16-column chunk in the
// accumulator row order, so the bf16-rounded accumulators are the B operands
// as they are.
#include <algorithm>
#include <cstdlib>
#include <string>

#include "attn_bwd.h"
#include "tile_io.h"

namespace aa {

namespace bwd {

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// ------------------------------------------------------------ dK, dV --

// 8 waves; pair w (waves w and w + 4, which share SIMD w) owns keys
// 32 w .. 32 w + 31 of the workgroup's 128 and splits the work by role:
// A (wave w) holds K and accumulates dV^T, B (wave w + 4) holds V and
// accumulates dK^T. Per 64-query tile t each role runs one MFMA block and one
// VALU block:
//   A: M_A(t) = dV^T += dO^T_{t-1} P_{t-1} (16) and S_t = Q_t K^T (16)
//      X_A(t) = P_t = exp2(S_t c - lse2_t) -> bf16 B operands, copied to the
//               pair's LDS slot for B
//   B: M_B(t) = dK^T += Q^T_{t-1} dZ_{t-1} (16) and dP_t - D_t = dO_t V^T (16,
//               accumulators start at -D_t)
//      X_B(t) = dZ_t = P_t o (dP_t - D_t) (P_t from the slot)
// The two roles run the same instruction stream one phase apart (B executes
// one extra barrier first, A one at the end), with a workgroup barrier
// between phases:
//   phase 2t   : A runs M_A(t), B runs X_B(t-1)
//   phase 2t+1 : A runs X_A(t), B runs M_B(t)
// so on every SIMD one wave's MFMAs overlap the other wave's VALU work.
// Only the Q and dO rows of each query tile come into LDS (dual line tiles,
// tile_io.h) with its stats record, in a 4-stage ring: the S / dP A
// operands are 16-byte row reads, the dV / dK A operands (dO^T, Q^T of the
// previous tile) are pairs of ds_read_b64_tr_b16 transposed reads of the same
// tiles. The B waves DMA tile t+2 at the start of X_B(t-1) (phase 2t); it is
// complete at the end of phase 2t+3.
constexpr int kDkWaves = 8;
static_assert(kDkWaves == kDkParts, "one partial record per wave");
constexpr int kDkQueue = 8;   // A operands in flight per wave
constexpr int kDkStages = 4;  // query tiles in the LDS ring

__global__ __launch_bounds__(kDkWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void dkdv_kernel(Params p, int nkblk, int total_blocks) {
  __shared__ __attribute__((aligned(1024))) bf16 rows[kDkStages][2][kTileElems];  // [stage][Q, dO]
  __shared__ __attribute__((aligned(1024))) float stat[kDkStages][kStat];
  __shared__ __attribute__((aligned(1024))) bf16x8 pslot[4][4][64];  // [pair][c4][lane]

  const int logical = xcd_remap(blockIdx.x, total_blocks);
  const int per_split = total_blocks / p.nsplit;
  const int split = logical / per_split;
  const int rest = logical - split * per_split;
  const int kblk = rest % nkblk;
  const int bh = rest / nkblk;
  const int b = bh / p.H, h = bh - (bh / p.H) * p.H;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int pair = wave & 3;
  const bool role_a = wave < 4;
  const int lane = tid & 63;
  const int li = lane & 31, hh = lane >> 5;

  // B operand of the role's S / dP product: lane holds K (A) or V (B)
  // [key][16 kk + 8 hh + 0..7], read from the wave's rows staged in LDS
  // (tile_io.h) in ring stages 2 and 3, which the first query tiles' DMA
  // leaves alone until after the first barrier. Keys past Sk re-read key
  // Sk - 1: their accumulators are never stored.
  const int key0 = kblk * kKeysPerWg + pair * 32;
  bf16x8 kv[8];
  const bf16* kvstage = &rows[2 + (wave >> 2)][0][0] + (wave & 3) * 4096;
  if (role_a) stage_rows_in(p.k + b * p.s_k[0] + h * p.s_k[2], p.s_k[1], key0, p.Sk, lane, kvstage);
  else stage_rows_in(p.v + b * p.s_v[0] + h * p.s_v[2], p.s_v[1], key0, p.Sk, lane, kvstage);

  const bf16* qbase = p.q + b * p.s_q[0] + h * p.s_q[2];
  const bf16* dobase = p.dout + b * p.s_do[0] + h * p.s_do[2];
  // Query tiles tq0 .. tq0 + ntiles - 1 (all of them without a split).
  const int tper = (p.ntq + p.nsplit - 1) / p.nsplit;
  const int tq0 = min(split * tper, p.ntq);
  const int ntiles = min(tper, p.ntq - tq0);
  const float* statb = p.stats + ((int64_t)bh * p.ntq + tq0) * kStat;

  // DMA by the B waves, g = wave - 4: blocks 4 g .. 4 g + 3 of the Q and dO
  // dual line tiles (8 rows x 128 bytes per instruction); wave 4 also copies
  // the stats record (9 DMA instructions per tile for wave 4, 8 for the other
  // B waves).
  const int g = wave & 3;
  DualDma qdma, dodma;
  qdma.setup(g, lane, p.s_q[1]);
  dodma.setup(g, lane, p.s_do[1]);
  auto issue_tile = [&](int t) {
    const int st = t % kDkStages, q0 = (tq0 + t) * kT, nr = min(kT, p.Sq - q0);
    qdma.issue(qbase + (int64_t)q0 * p.s_q[1], p.s_q[1], nr, rows[st][0], lane);
    dodma.issue(dobase + (int64_t)q0 * p.s_do[1], p.s_do[1], nr, rows[st][1], lane);
    if (wave == 4) dma16(statb + (int64_t)t * kStat + 4 * lane, stat[st]);
  };

  // Per-lane read offsets in the dual line tiles (tile_io.h): row operand
  // (hq, kk) at rrd[kk & 3] + 4096 (kk >> 2) + 2048 hq; transposed operand
  // (c4, dt), queries in the order of the P / dZ B operands, via trd.
  int rrd[4], trd[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    rrd[j] = dual_row_rd(lane, j);
    trd[j] = dual_tr_rd(lane, j >> 1, j & 1);
  }
  const float c = p.c;

  f32x16 acc[4];  // dV^T (A) or dK^T (B)
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;
  f32x16 x[2];    // S_t (A) or dP_t - D_t (B); register r of half hq is query
                  // 32 hq + 8 (r >> 2) + 4 hh + (r & 3)
  bf16x8 bop[4];  // P_{t-1} (A) or dZ_{t-1} (B), B operands of the next M block

  // M block of tile t: ops 0-15 (PV) acc[dt] += T_{t-1}(dt, c4) bop[c4] with
  // c4 = op / 4, dt = op % 4; ops 16-31 (QK) x[hq] += R_t(hq, kk) kv[kk] with
  // hq = (op - 16) / 8, kk = op % 8. T = dO^T (A) or Q^T (B), read transposed
  // from the previous tile's dO / Q rows; R = Q rows (A) or dO rows (B). x
  // starts at 0 (A: the zero pad of the stats record) or -D_t (B). One
  // unrolled stream fed by a kDkQueue-deep operand queue.
  auto mblock = [&](int t, auto pv_tag, auto qk_tag) {
    constexpr bool PV = decltype(pv_tag)::value;
    constexpr bool QK = decltype(qk_tag)::value;
    constexpr int first = PV ? 0 : 16;
    constexpr int last = QK ? 32 : 16;
    const bf16* tt = rows[(t + kDkStages - 1) % kDkStages][role_a ? 1 : 0];
    const bf16* rr = rows[t % kDkStages][role_a ? 0 : 1];
    if constexpr (QK) {
      const float* init = stat[t % kDkStages] + (role_a ? 2 * kT : kT);
#pragma unroll
      for (int hq = 0; hq < 2; ++hq)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const f32x4 v4 = *reinterpret_cast<const f32x4*>(init + 32 * hq + 8 * rq + 4 * hh);
#pragma unroll
          for (int i = 0; i < 4; ++i) x[hq][4 * rq + i] = v4[i];
        }
    }
    auto load_op = [&](int op) -> bf16x8 {
      if (op < 16) return read_tr_dual(tt, op >> 2, op & 3, trd);
      const int w = op - 16, kk = w & 7;
      return *reinterpret_cast<const bf16x8*>(rr + rrd[kk & 3] + 4096 * (kk >> 2) + 2048 * (w >> 3));
    };
    auto run_op = [&](int op, bf16x8 a) {
      if (op < 16) {
        acc[op & 3] = mfma32(a, bop[op >> 2], acc[op & 3]);
      } else {
        const int w = op - 16;
        x[w >> 3] = mfma32(a, kv[w & 7], x[w >> 3]);
      }
    };
    bf16x8 queue[kDkQueue];
#pragma unroll
    for (int i = first; i < last + kDkQueue; ++i) {
      if (i - kDkQueue >= first) run_op(i - kDkQueue, queue[(i - kDkQueue - first) % kDkQueue]);
      if (i < last) queue[(i - first) % kDkQueue] = load_op(i);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // X block of tile t (B first copies tile t + 3).
  auto xblock = [&](int t) {
    if (role_a) {
      const float* l2p = stat[t % kDkStages];
#pragma unroll
      for (int hq = 0; hq < 2; ++hq)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const f32x4 l2 = *reinterpret_cast<const f32x4*>(l2p + 32 * hq + 8 * rq + 4 * hh);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = 4 * rq + i;
            bop[2 * hq + (r >> 3)][r & 7] = (bf16)fast_exp2(fmaf(x[hq][r], c, -l2[i]));
          }
        }
#pragma unroll
      for (int c4 = 0; c4 < 4; ++c4) pslot[pair][c4][lane] = bop[c4];
    } else {
      if (t + 3 < ntiles) issue_tile(t + 3);
#pragma unroll
      for (int c4 = 0; c4 < 4; ++c4) bop[c4] = pslot[pair][c4][lane];
#pragma unroll
      for (int hq = 0; hq < 2; ++hq)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int c4 = 2 * hq + (r >> 3);
          bop[c4][r & 7] = (bf16)((float)bop[c4][r & 7] * x[hq][r]);
        }
    }
  };

  // Stages: tile t in t % 4, written at phase 2t-4 (the stage of tile t-4,
  // whose last reads were in phase 2t-5), read in phases 2t .. 2t+3. At the
  // end of M_B(t) (phase 2t+1) a B wave waits for tile t+1; tile t+2 may be in
  // flight.
  const int tile_dma = wave == 4 ? 9 : 8;  // DMA instructions per tile (B waves)
  auto wait_tile_next = [&](int t) {
    if (t + 2 < ntiles) {
      if (tile_dma == 9) asm volatile("s_waitcnt vmcnt(9)" ::: "memory");
      else asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    } else {
      wait_dma();
    }
  };
  if (ntiles > 0 && !role_a) issue_tile(0);
  wait_dma();  // the staged K / V rows (and tile 0)
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) kv[kk] = staged_operand(kvstage, lane, kk);
  __syncthreads();
  if (ntiles > 0) {
    if (!role_a) {  // the DMA of X_B(-2) and X_B(-1), then the phase shift
      if (1 < ntiles) issue_tile(1);
      if (2 < ntiles) issue_tile(2);
      __syncthreads();
    }
    mblock(0, std::false_type{}, std::true_type{});
    if (!role_a) wait_tile_next(0);
    __syncthreads();
    xblock(0);
    __syncthreads();
    for (int t = 1; t < ntiles; ++t) {
      mblock(t, std::true_type{}, std::true_type{});
      if (!role_a) wait_tile_next(t);
      __syncthreads();
      xblock(t);
      __syncthreads();
    }
    mblock(ntiles, std::true_type{}, std::false_type{});
    if (role_a) __syncthreads();
  }

  // dV (A) / dK (B) rows out through LDS staging: the stages of tiles
  // ntiles-4 and ntiles-3 are free (B may still be reading tile ntiles-1 in
  // its final M block; no DMA is in flight).
  if (p.nsplit > 1) {
    // Partial accumulators, 16 coalesced 1 KB stores per wave: float4 j of
    // lane l at ((logical * 8 + wave) * 16 + j) * 64 + l.
    f32x4* dst = reinterpret_cast<f32x4*>(p.part) + ((int64_t)logical * kDkWaves + wave) * 16 * 64 + lane;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const f32x4 v4 = {acc[j >> 2][4 * (j & 3)], acc[j >> 2][4 * (j & 3) + 1], acc[j >> 2][4 * (j & 3) + 2],
                        acc[j >> 2][4 * (j & 3) + 3]};
      __builtin_nontemporal_store(v4, dst + j * 64);
    }
    return;
  }
  bf16* ostage = &rows[(ntiles + (wave >> 2)) % kDkStages][0][0] + (wave & 3) * 4096;
  stage_acc_rows(acc, role_a ? 1.0f : p.scale, lane, ostage);
  if (role_a) stage_rows_out(p.dv + b * p.s_dv[0] + h * p.s_dv[2], p.s_dv[1], key0, p.Sk, lane, ostage);
  else stage_rows_out(p.dk + b * p.s_dk[0] + h * p.s_dk[2], p.s_dk[1], key0, p.Sk, lane, ostage);
}

// Sums the query-split partials of either dK/dV kernel in split order and
// writes dV and dK (times the softmax scale) as bf16. A workgroup's partial
// holds, per record w, float4 j of lane l at ((w * 16 + j) * 64 + l):
// accumulator block dt = j / 4, registers 4 (j % 4) .. + 3, i.e. key
// 32 (w % 4) + l % 32 of the key block and head-dim 32 dt + 8 (j % 4) +
// 4 (l / 32) .. + 3; records 0-3 hold dV^T, 4-7 dK^T (the waves of
// dkdv_kernel; both accumulators of each wave of the one-wave kernel). One
// thread per (key, 8 consecutive head-dims): the
// float4s of lanes l and l + 32 of every split, all loaded before the sums,
// and one 16-byte store (8-byte stores of one lane's half took 11.7 us for
// B=2, 512 keys, 16 heads, 2 splits).
constexpr int kMaxDkSplit = 4;
__global__ __launch_bounds__(256) void dkdv_combine_kernel(Params p, int nkblk, int per_split) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;  // (rest, wave, j, li)
  const int li = (int)(gid & 31);
  const int j = (int)((gid >> 5) & 15);
  const int wave = (int)((gid >> 9) & 7);
  const int rest = (int)(gid >> 12);
  if (rest >= per_split) return;
  const int kblk = rest % nkblk, bh = rest / nkblk;
  const int b = bh / p.H, h = bh - b * p.H;
  const int key = kblk * kKeysPerWg + (wave & 3) * 32 + li;
  if (key >= p.Sk) return;
  const f32x4* src = reinterpret_cast<const f32x4*>(p.part) + (((int64_t)rest * kDkParts + wave) * 16 + j) * 64 + li;
  const int64_t split_stride = (int64_t)per_split * kDkParts * 16 * 64;
  f32x4 v[kMaxDkSplit][2];
#pragma unroll
  for (int s = 0; s < kMaxDkSplit; ++s) {
    if (s < p.nsplit) {
      v[s][0] = src[s * split_stride];
      v[s][1] = src[s * split_stride + 32];
    }
  }
  f32x4 sum0 = v[0][0], sum1 = v[0][1];
#pragma unroll
  for (int s = 1; s < kMaxDkSplit; ++s) {
    if (s < p.nsplit) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sum0[i] += v[s][0][i];
        sum1[i] += v[s][1][i];
      }
    }
  }
  const bool is_dv = wave < 4;
  const float sc = is_dv ? 1.0f : p.scale;
  const int d0 = 32 * (j >> 2) + 8 * (j & 3);
  bf16* out = is_dv ? p.dv + b * p.s_dv[0] + (int64_t)key * p.s_dv[1] + h * p.s_dv[2]
                    : p.dk + b * p.s_dk[0] + (int64_t)key * p.s_dk[1] + h * p.s_dk[2];
  const u32x4 w = {pack_bf16(sum0[0] * sc, sum0[1] * sc), pack_bf16(sum0[2] * sc, sum0[3] * sc),
                   pack_bf16(sum1[0] * sc, sum1[1] * sc), pack_bf16(sum1[2] * sc, sum1[3] * sc)};
  *reinterpret_cast<u32x4*>(out + d0) = w;
}

// ------------------------------------------------------------------ dQ --

// 8 waves x 32 queries (256 per workgroup), Q^T and dO^T in registers; keys
// are the accumulator rows. Per 64-key tile t a wave runs
//   M(t): dQ^T += K^T_{t-1} dZ^T_{t-1} (16 MFMA; K^T read transposed from the
//         K rows of tile t-1), S^T_t = K_t Q^T (16), dP^T_t - D = V_t dO^T
//         (16, accumulators start at -D)
//   X(t): dZ^T_t = exp2(S^T_t c - lse2) o (dP^T_t - D) as bf16 B operands.
// Waves 0-3 (group A) and 4-7 (group B) run the same stream one phase apart
// (B executes one extra barrier first, A one at the end):
//   phase 2t: A runs M(t), B runs X(t-1);  phase 2t+1: A runs X(t), B runs M(t)
// K and V rows stream into a 4-stage ring of dual line tiles (tile_io.h):
// group A DMAs tile t+2 at the start of X(t) (phase 2t+1) into the stage of
// tile t-2 (last read in phase 2t-1) and waits for tile t+1 at its end.
constexpr int kDqWaves = 8;                  // two per SIMD
constexpr int kDqQueue = 6;                  // operand queue depth (register-bound at 2 waves/SIMD)
constexpr int kDqStages = 4;
constexpr int kQueriesPerWg = kDqWaves * 32;

__global__ __launch_bounds__(kDqWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void dq_kernel(Params p, int nqblk, int total_blocks) {
  __shared__ __attribute__((aligned(1024))) bf16 tiles[kDqStages][2][kTileElems];  // [stage][K, V]

  const int logical = xcd_remap(blockIdx.x, total_blocks);
  const int qblk = logical % nqblk;
  const int bh = logical / nqblk;
  const int b = bh / p.H, h = bh - (bh / p.H) * p.H;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool group_a = wave < 4;
  const int lane = tid & 63;
  const int li = lane & 31, hh = lane >> 5;

  // Q^T / dO^T operands: lane holds Q[query][16 kk + 8 hh + 0..7].
  const int qrow = qblk * kQueriesPerWg + wave * 32 + li;
  const bool q_ok = qrow < p.Sq;
  bf16x8 qreg[8], doreg[8];
  {
    const bf16* qp = p.q + b * p.s_q[0] + h * p.s_q[2] + (int64_t)qrow * p.s_q[1] + 8 * hh;
    const bf16* dp = p.dout + b * p.s_do[0] + h * p.s_do[2] + (int64_t)qrow * p.s_do[1] + 8 * hh;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      u32x4 a = {0u, 0u, 0u, 0u}, e = {0u, 0u, 0u, 0u};
      if (q_ok) {
        a = ld16(qp + 16 * kk);
        e = ld16(dp + 16 * kk);
      }
      qreg[kk] = as_bf16x8(a);
      doreg[kk] = as_bf16x8(e);
    }
  }
  // The query's stats: lse2 = lse * log2(e) and -D, D = rowsum(dO o O) (this
  // lane's 64 values against its dO^T operands, then the partner lane's
  // half). They also go to the query's stats record, which dkdv_kernel reads
  // (it runs after this kernel): rows past Sq get lse2 = +inf (P = 0) and
  // D = 0, and every record's second half is the zero pad dkdv uses to start
  // its S accumulators.
  float lse2 = INFINITY, ndlt = 0.f;  // -D
  if (q_ok) {
    lse2 = p.lse[(int64_t)bh * p.Sq + qrow] * kLog2e;
    const bf16* op = p.o + b * p.s_o[0] + h * p.s_o[2] + (int64_t)qrow * p.s_o[1] + 8 * hh;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      float x[8], y[8];
      unpack8(ld16(op + 16 * kk), x);
      unpack8(__builtin_bit_cast(u32x4, doreg[kk]), y);
#pragma unroll
      for (int i = 0; i < 8; ++i) ndlt = fmaf(y[i], x[i], ndlt);
    }
  }
  ndlt = -pair_sum(ndlt);
  if (hh == 0 && qrow < p.ntq * kT) {
    float* st = p.stats + ((int64_t)bh * p.ntq + qrow / kT) * kStat + (qrow % kT);
    st[0] = lse2;
    st[kT] = ndlt;
    st[2 * kT] = 0.f;
    st[3 * kT] = 0.f;
  }

  const bf16* kbase = p.k + b * p.s_k[0] + h * p.s_k[2];
  const bf16* vbase = p.v + b * p.s_v[0] + h * p.s_v[2];
  const int ntiles = p.ntk;

  // DMA by group A, g = wave: blocks 4 g .. 4 g + 3 of the K and V dual line
  // tiles (8 rows x 128 bytes per instruction). The lane offsets are computed
  // at each issue: held in registers they would push this kernel past 256.
  const int g = wave & 3;
  auto issue_tile = [&](int t) {
    const int st = t % kDqStages, k0 = t * kT, nr = min(kT, p.Sk - k0);
    // An opaque copy of the lane index keeps the compiler from hoisting the
    // offsets out of the tile loop (where they would hold registers again).
    int ln = lane;
    asm volatile("" : "+v"(ln));
    DualDma::issue_quad(g, kbase + (int64_t)k0 * p.s_k[1], p.s_k[1], nr, tiles[st][0], ln,
                        DualDma::lane_off(g, ln, p.s_k[1], 0), DualDma::lane_off(g, ln, p.s_k[1], 1));
    DualDma::issue_quad(g, vbase + (int64_t)k0 * p.s_v[1], p.s_v[1], nr, tiles[st][1], ln,
                        DualDma::lane_off(g, ln, p.s_v[1], 0), DualDma::lane_off(g, ln, p.s_v[1], 1));
  };

  // Read offsets in the dual line tiles (tile_io.h): row operands (row
  // 32 hk + li, chunk 2 kk + hh) at rrd[kk & 3] + 4096 (kk >> 2) + 2048 hk;
  // transposed operands (c4, dt), keys in the order of the dZ^T B operands,
  // via trd.
  int rrd[4], trd[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    rrd[j] = dual_row_rd(lane, j);
    trd[j] = dual_tr_rd(lane, j >> 1, j & 1);
  }
  const float c = p.c;

  f32x16 dq[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[i][r] = 0.f;
  // S^T and dP^T - D of the tile between its M and X blocks; register r of
  // half hk is key 32 hk + 8 (r >> 2) + 4 hh + (r & 3) of the tile.
  f32x16 s[2], dp[2];
  bf16x8 zb[4];  // dZ^T of the previous tile, B operands of the next M block

  // M block of tile t, one unrolled stream of up to 48 MFMAs fed by a
  // kDqQueue-deep operand queue:
  //   ops 0-15 : c4 = op / 4, dt = op % 4: dQ^T[dt] += K^T_{t-1}(dt, c4) zb[c4]
  //   ops 16-47: w = op - 16, kk = w / 4, hk = (w / 2) % 2;
  //              even w: S^T[hk] += K_t rows x Q^T, odd w: dP^T[hk] += V_t rows x dO^T
  auto mblock = [&](int t, auto pv_tag, auto qk_tag) {
    constexpr bool PV = decltype(pv_tag)::value;
    constexpr bool QK = decltype(qk_tag)::value;
    constexpr int first = PV ? 0 : 16;
    constexpr int last = QK ? 48 : 16;
    const bf16* kprev = tiles[(t + kDqStages - 1) % kDqStages][0];
    const bf16* kr = tiles[t % kDqStages][0];
    const bf16* vr = tiles[t % kDqStages][1];
    if constexpr (QK) {
#pragma unroll
      for (int hk = 0; hk < 2; ++hk)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          s[hk][r] = 0.f;
          dp[hk][r] = ndlt;
        }
    }
    auto load_op = [&](int op) -> bf16x8 {
      if (op < 16) return read_tr_dual(kprev, op >> 2, op & 3, trd);
      const int w = op - 16, kk = w >> 2, hk = (w >> 1) & 1;
      return *reinterpret_cast<const bf16x8*>(((w & 1) ? vr : kr) + rrd[kk & 3] + 4096 * (kk >> 2) +
                                               2048 * hk);
    };
    auto run_op = [&](int op, bf16x8 a) {
      if (op < 16) {
        dq[op & 3] = mfma32(a, zb[op >> 2], dq[op & 3]);
      } else {
        const int w = op - 16, kk = w >> 2, hk = (w >> 1) & 1;
        if (w & 1) dp[hk] = mfma32(a, doreg[kk], dp[hk]);
        else s[hk] = mfma32(a, qreg[kk], s[hk]);
      }
    };
    bf16x8 queue[kDqQueue];
#pragma unroll
    for (int i = first; i < last + kDqQueue; ++i) {
      if (i - kDqQueue >= first) run_op(i - kDqQueue, queue[(i - kDqQueue - first) % kDqQueue]);
      if (i < last) queue[(i - first) % kDqQueue] = load_op(i);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // X block of tile t; group A first copies tile t + 2 and at the end waits
  // for tile t + 1 (tile t + 2 may stay in flight: 8 DMA per wave per tile).
  auto xblock = [&](int t) {
    if (group_a && t + 2 < ntiles) issue_tile(t + 2);
    const int kb = t * kT;
    // Keys past Sk (last tile only, a wave-uniform branch) get S = -inf, so
    // P = 0. Masking per element on every tile, as a select after the exp,
    // put ~96 VALU instructions into every softmax phase.
    if (kb + kT > p.Sk) {
#pragma unroll
      for (int hk = 0; hk < 2; ++hk)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (kb + 32 * hk + 8 * (r >> 2) + 4 * hh + (r & 3) >= p.Sk) s[hk][r] = -INFINITY;
    }
#pragma unroll
    for (int hk = 0; hk < 2; ++hk)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        zb[2 * hk + (r >> 3)][r & 7] = (bf16)(fast_exp2(fmaf(s[hk][r], c, -lse2)) * dp[hk][r]);
    // The wait takes the dZ operands as inputs so that it stays after the
    // VALU work above (a plain asm statement may be hoisted over it).
    if (group_a) {
      if (t + 2 < ntiles)
        asm volatile("s_waitcnt vmcnt(8)" ::"v"(zb[0]), "v"(zb[1]), "v"(zb[2]), "v"(zb[3]) : "memory");
      else
        asm volatile("s_waitcnt vmcnt(0)" ::"v"(zb[0]), "v"(zb[1]), "v"(zb[2]), "v"(zb[3]) : "memory");
    }
  };

  if (ntiles > 0 && group_a) {
    issue_tile(0);
    if (1 < ntiles) {
      issue_tile(1);
      asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    } else {
      wait_dma();
    }
  }
  __syncthreads();
  if (!group_a) __syncthreads();  // the phase shift
  if (ntiles > 0) {
    mblock(0, std::false_type{}, std::true_type{});
    __syncthreads();
    xblock(0);
    __syncthreads();
    for (int t = 1; t < ntiles; ++t) {
      mblock(t, std::true_type{}, std::true_type{});
      __syncthreads();
      xblock(t);
      __syncthreads();
    }
    mblock(ntiles, std::true_type{}, std::false_type{});
  }
  if (group_a) __syncthreads();

  // dQ rows out through LDS staging in the stages of tiles ntiles-4 and
  // ntiles-3 (free: group B may still be reading tile ntiles-1 in its final
  // M block; no DMA is in flight).
  bf16* ostage = &tiles[(ntiles + (wave >> 2)) % kDqStages][0][0] + (wave & 3) * 4096;
  stage_acc_rows(dq, p.scale, lane, ostage);
  stage_rows_out(p.dq + b * p.s_dq[0] + h * p.s_dq[2], p.s_dq[1], qblk * kQueriesPerWg + wave * 32,
                 p.Sq, lane, ostage);
}

static bool stride_ok(const int64_t* s) {
  return (s[0] % 8) == 0 && (s[1] % 8) == 0 && (s[2] % 8) == 0 && s[0] < (1ll << 40) &&
         s[1] < (1ll << 40) && s[2] < (1ll << 40);
}

// Query splits of dkdv_kernel: when its workgroups (one per 128 keys of each
// (batch, head)) fill at most half of the CUs, as for the 512-key text
// context at B = 2 and 16 heads (128 workgroups), each key block's query
// tiles are split over up to 4 workgroups, each covering at least 4 tiles.
static int dkdv_split(int64_t B, int64_t Sq, int64_t Sk, int64_t H, int ncu) {
  const int64_t blocks = B * H * ((Sk + kKeysPerWg - 1) / kKeysPerWg);
  const int64_t ntq = (Sq + kT - 1) / kT;
  if (ncu <= 0 || blocks <= 0 || 2 * blocks > ncu) return 1;
  int64_t ns = std::min<int64_t>(kMaxDkSplit, ncu / blocks);
  ns = std::min<int64_t>(ns, ntq / 4);
  return (int)std::max<int64_t>(ns, 1);
}

struct WsLayout {
  size_t stats, part, total;
  int nsplit;
};

static WsLayout ws_layout(int64_t B, int64_t Sq, int64_t Sk, int64_t H) {
  const int64_t ntq = (Sq + kT - 1) / kT;
  WsLayout w;
  w.nsplit = dkdv_split(B, Sq, Sk, H, device_cu_count());
  w.stats = 0;
  w.part = w.stats + (size_t)(B * H * ntq) * kStat * sizeof(float);
  const int64_t blocks = B * H * ((Sk + kKeysPerWg - 1) / kKeysPerWg);
  const size_t part_bytes =
      w.nsplit > 1 ? (size_t)w.nsplit * blocks * kDkParts * 64 * 64 * sizeof(float) : 0;
  w.total = w.part + part_bytes;
  return w;
}

// Which dK/dV kernel runs: the one-wave-per-SIMD kernel of attn_bwd_dkdv.hip
// (1, the default) or the two-role kernel above (0). AA_DKDV_KERNEL=1w|2role
// forces one (the GPU tests run both on every shape); -1 for another value.
static int dkdv_kernel_choice() {
  const char* e = std::getenv("AA_DKDV_KERNEL");
  if (e && *e) {
    const std::string v = e;
    if (v == "2role") return 0;
    if (v == "1w") return 1;
    return -1;
  }
  return 1;
}

}  // namespace bwd
}  // namespace aa

using namespace aa;

extern "C" size_t aa_attn_bwd_workspace(int64_t B, int64_t Sq, int64_t Sk, int64_t H, int64_t hd) {
  (void)hd;
  if (B <= 0 || Sq <= 0 || H <= 0 || Sk < 0) return 0;
  return bwd::ws_layout(B, Sq, Sk, H).total;
}

extern "C" int aa_attn_bwd(const aa_attn_bwd_args* a, void* workspace, size_t workspace_bytes,
                           void* stream) {
  clear_error();
  if (!a) return fail(AA_EINVAL, "attn_bwd: null args");
  if (a->dtype != AA_DTYPE_BF16) return fail(AA_EUNSUPPORTED, "only bf16 attention is implemented");
  if (a->hd != bwd::kD) return fail(AA_EUNSUPPORTED, "head_dim must be 128");
  if (a->B < 0 || a->Sq < 0 || a->Sk < 0 || a->H <= 0)
    return fail(AA_EINVAL, "attn_bwd: negative size");
  if (a->Sq > (1 << 30) || a->Sk > (1 << 30) || a->H > 65535 || a->B > 65535)
    return fail(AA_EUNSUPPORTED, "attn_bwd: size out of range");
  if (a->B == 0) return AA_OK;
  const void* ptrs[] = {a->dout, a->q, a->k, a->v, a->out, a->dq, a->dk, a->dv};
  for (const void* ptr : ptrs) {
    if (!ptr) return fail(AA_EINVAL, "attn_bwd: null tensor");
    if (!aligned16(ptr)) return fail(AA_EINVAL, "attn_bwd: tensors must be 16-byte aligned");
  }
  if (!a->lse) return fail(AA_EINVAL, "attn_bwd: null lse");
  const int64_t* strides[] = {a->dout_stride, a->q_stride,  a->k_stride,  a->v_stride,
                              a->out_stride,  a->dq_stride, a->dk_stride, a->dv_stride};
  for (const int64_t* s : strides)
    if (!bwd::stride_ok(s)) return fail(AA_EINVAL, "attn_bwd: strides must be multiples of 8");
  // The tile DMA addresses rows by a 32-bit unsigned per-lane byte offset (up
  // to 7 rows past a scalar row base).
  for (const int64_t* s : {a->q_stride, a->dout_stride, a->k_stride, a->v_stride})
    if (s[1] < 0 || s[1] >= (1 << 24))
      return fail(AA_EUNSUPPORTED, "attn_bwd: q / dout / k / v sequence strides must be in [0, 2^24) elements");
  if (!(a->softmax_scale > 0.f)) return fail(AA_EINVAL, "attn_bwd: softmax_scale must be > 0");
  const int dkdv_which = bwd::dkdv_kernel_choice();
  if (dkdv_which < 0) return fail(AA_EINVAL, "AA_DKDV_KERNEL must be 1w or 2role");
  const bwd::WsLayout wl = bwd::ws_layout(a->B, a->Sq, a->Sk, a->H);
  const size_t need = aa_attn_bwd_workspace(a->B, a->Sq, a->Sk, a->H, a->hd);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return fail(AA_EINVAL, "attn_bwd: workspace too small");
  if (need > 0 && !aligned16(workspace))
    return fail(AA_EINVAL, "attn_bwd: workspace must be 16-byte aligned");

  bwd::Params p;
  p.dout = (const bf16*)a->dout;
  p.q = (const bf16*)a->q;
  p.k = (const bf16*)a->k;
  p.v = (const bf16*)a->v;
  p.o = (const bf16*)a->out;
  p.lse = a->lse;
  p.dq = (bf16*)a->dq;
  p.dk = (bf16*)a->dk;
  p.dv = (bf16*)a->dv;
  for (int i = 0; i < 3; ++i) {
    p.s_do[i] = a->dout_stride[i];
    p.s_q[i] = a->q_stride[i];
    p.s_k[i] = a->k_stride[i];
    p.s_v[i] = a->v_stride[i];
    p.s_o[i] = a->out_stride[i];
    p.s_dq[i] = a->dq_stride[i];
    p.s_dk[i] = a->dk_stride[i];
    p.s_dv[i] = a->dv_stride[i];
  }
  char* ws = (char*)workspace;
  p.stats = (float*)(ws + wl.stats);
  p.part = (float*)(ws + wl.part);
  p.nsplit = wl.nsplit;
  p.H = (int)a->H;
  p.Sq = (int)a->Sq;
  p.Sk = (int)a->Sk;
  p.ntq = (int)((a->Sq + bwd::kT - 1) / bwd::kT);
  p.ntk = (int)((a->Sk + bwd::kT - 1) / bwd::kT);
  p.scale = a->softmax_scale;
  p.c = a->softmax_scale * kLog2e;
  hipStream_t st = (hipStream_t)stream;

  const int64_t BH = a->B * a->H;
  // dq_kernel first: it writes the stats records that dkdv_kernel reads.
  // Nothing reads the workspace when Sq == 0 (dK = dV = 0 and no dQ rows).
  if (a->Sq > 0) {
    const int nqblk = (int)((a->Sq + bwd::kQueriesPerWg - 1) / bwd::kQueriesPerWg);
    const int total = (int)(BH * nqblk);
    bwd::dq_kernel<<<dim3((unsigned)total), bwd::kDqWaves * 64, 0, st>>>(p, nqblk, total);
    if (int rc = check_launch("attn_bwd dq")) return rc;
  }
  if (a->Sk > 0) {
    const int nkblk = (int)((a->Sk + bwd::kKeysPerWg - 1) / bwd::kKeysPerWg);
    const int per_split = (int)(BH * nkblk);
    const int total = per_split * p.nsplit;
    if (dkdv_which == 1) bwd::launch_dkdv1w(p, nkblk, total, st);
    else bwd::dkdv_kernel<<<dim3((unsigned)total), bwd::kDkWaves * 64, 0, st>>>(p, nkblk, total);
    if (int rc = check_launch("attn_bwd dkdv")) return rc;
    if (p.nsplit > 1) {
      const int64_t threads = (int64_t)per_split * bwd::kDkParts * 16 * 32;
      bwd::dkdv_combine_kernel<<<dim3((unsigned)(threads / 256)), 256, 0, st>>>(p, nkblk, per_split);
      if (int rc = check_launch("attn_bwd dkdv combine")) return rc;
    }
  }
  return AA_OK;
}
