// dK / dV of the flash-attention backward with one wave per SIMD, for gfx950
// (v_mfma_f32_32x32x16_bf16). Deterministic: every sum in a fixed order.
//
// One workgroup = 4 waves = 128 keys of one (batch, head), over the whole
// query range or one part of it (the query split, attn_bwd.hip). Wave w owns
// keys 32 w .. 32 w + 31 and does, per 64-query tile, what the two-role
// kernel (dkdv_kernel, attn_bwd.hip) deals to two waves:
//   S      = Q K^T       A = Q rows (LDS),        B = K^T (AGPRs, read once)
//   dP - D = dO V^T      A = dO rows (LDS),       B = V^T (AGPRs), started at -D
//   P = exp2(S c - lse2),  dZ = P o (dP - D)      (fp32; P and dZ rounded to bf16)
//   dV^T  += dO^T P      A = dO^T (transposed LDS reads), B = P
//   dK^T  += Q^T dZ      A = Q^T (transposed LDS reads),  B = dZ
// Keys are the accumulator columns (lane % 32), queries the rows: register r
// of query half hq is query 32 hq + 8 (r >> 2) + 4 hh + (r & 3). The
// transposed reads list each 16-query chunk in that order, so the rounded P
// and dZ registers are the B operands as they are (tile_io.h).
//
// Why one wave per SIMD: in the two-role kernel one wave's 32-MFMA block runs
// beside its partner's VALU block, with a workgroup barrier between phases.
// The phases differ in length (the exp work beside one block is heavier than
// the dZ products beside the other) and the slowest of 8 waves ends each
// phase; measured with the shader clock, the barriers took about a third of
// every tile. Here a tile is 64 slots of one MFMA each, the VALU work is
// dealt to fixed slots beside the MFMAs (the forward's technique,
// attn_fwd.hip), and the 4 waves meet at one barrier per tile:
//   slots  0-15: S of tile t+1        | P and dZ of tile t, one unit of two
//   slots 16-31: dP - D of tile t+1   |   scores every three slots from slot 7
//   slots 32-63: dV^T and dK^T of tile t, alternating, chunk by chunk
// S and dP - D are double-buffered (computed one tile before their use). The
// DMA of tile t+3 (Q rows, dO rows, the stats record) goes out one
// instruction per slot.
//
// Registers (512 per lane): dV^T, dK^T and the K^T, V^T operands in AGPRs
// (192); S, dP - D (2 x 64), P, dZ (32), the operand queues and the stats in
// VGPRs. The file is built with -mllvm -amdgpu-mfma-vgpr-form=1 (build.py):
// the S and dP MFMAs are builtins whose accumulators the VALU reads, the dV
// and dK MFMAs inline asm on AGPR accumulators.
#include <type_traits>

#include "attn_bwd.h"
#include "tile_io.h"

namespace aa {
namespace bwd {
namespace w1 {

constexpr int kWaves = 4;  // one per SIMD
static_assert(kWaves * 32 == kKeysPerWg, "32 keys per wave");
constexpr int kStages = 4;                       // query tiles in the LDS ring
constexpr int kLead = kStages - 1;               // tile t + kLead is fetched during tile t
constexpr uint32_t kTileBytes = kTileElems * 2;  // one 64 x 128 bf16 tile
constexpr uint32_t kStageBytes = 2 * kTileBytes; // Q tile, then dO tile
constexpr uint32_t kDoOff = kTileBytes;
constexpr uint32_t kStatBytes = kStat * 4;
constexpr uint32_t kNegDOff = kT * 4;            // -D in a stats record (bytes)

// Operand reads ahead of their MFMA: row operands (S, dP) kRPf slots ahead,
// transposed ones (dV, dK) kTPf slots ahead, into queues one entry longer
// than that needs (two for the transposed ones: an inline-asm MFMA's operand
// stays allocated for one slot after it).
constexpr int kRPf = 3, kRQ = kRPf + 1;
constexpr int kTPf = 3, kTQ = kTPf + 2;
constexpr int rread_slot(int j) { return j < kRPf ? 0 : j - kRPf; }
constexpr int tread_slot(int j) { return 32 + j - kTPf; }
// Unit u: scores 2 jp, 2 jp + 1 of the P / dZ operand c4 (u = 4 c4 + jp).
// FMA in slot unit_slot(u), exp one slot later, the P pack and the dZ
// products two slots later, the dZ pack three slots later: the last unit of
// chunk c4 packs P in slot 12 c4 + 18 and dZ in 12 c4 + 19, before the
// chunk's first dV (slot 32 + 8 c4) and dK (33 + 8 c4) MFMAs.
constexpr int unit_slot(int u) { return 3 * u + 7; }
// DMA instruction i of the tile's job: slot 4 i + 3; the stats record
// (wave 0 only) in slot 34.
constexpr int dma_slot(int i) { return 4 * i + 3; }
constexpr int kStatSlot = 34;

// DMA of one wave's quarter of the Q and dO dual line tiles of a query tile
// (tile_io.h): blocks 4 g .. 4 g + 3 (g = wave) = d-half g >> 1, rows
// 32 (g & 1) + 8 i + (lane >> 3). A job takes one scalar base per tensor (the
// tile's first row) and per-lane 32-bit byte offsets holding each lane's row
// and column. Rows at or past Sq re-read row Sq - 1 (their stats give P = 0
// and dZ = 0). Wave 0 also moves the tile's stats record (1 KB).
struct QdoDma {
  uint32_t qo[4], oo[4];  // per-lane offsets of blocks 0-3 (rows inside Sq unless `clamped`)
  bool clamped;
  const bf16* qb;
  const bf16* ob;
  const float* sb;  // the stats record
  uint32_t dst;     // LDS byte address of this wave's first Q block
  uint32_t sdst;    // LDS byte address of the stats record

  __device__ __forceinline__ static int row_of(int g, int i, int lane) {
    return 32 * (g & 1) + 8 * i + (lane >> 3);
  }
  __device__ __forceinline__ static int col(int g, int i, int lane) {
    return 64 * (g >> 1) + 8 * dual_chunk(lane, i & 1);
  }
  __device__ __forceinline__ void fixed(const Params& p, int g, int lane) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = row_of(g, i, lane);
      qo[i] = (uint32_t)(r * p.s_q[1] + col(g, i, lane)) * 2u;
      oo[i] = (uint32_t)(r * p.s_do[1] + col(g, i, lane)) * 2u;
    }
    clamped = false;
  }
  // The job of the tile whose first query row is q0 (< Sq), into the ring
  // stage at byte address `stage`, stats record srec into LDS at sdst_.
  __device__ __forceinline__ void prepare(const Params& p, int q0, uint32_t stage, uint32_t sdst_,
                                          const float* srec, int g, const bf16* qbase,
                                          const bf16* obase, int lane) {
    dst = stage + (uint32_t)(4 * g) * 1024u;
    sdst = sdst_;
    sb = srec;
    if (q0 + kT <= p.Sq) {
      qb = qbase + (int64_t)q0 * p.s_q[1];
      ob = obase + (int64_t)q0 * p.s_do[1];
      if (clamped) fixed(p, g, lane);
    } else {
      const int last = p.Sq - 1;
      qb = qbase + (int64_t)q0 * p.s_q[1];
      ob = obase + (int64_t)q0 * p.s_do[1];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = min(q0 + row_of(g, i, lane), last) - q0;
        qo[i] = (uint32_t)(r * p.s_q[1] + col(g, i, lane)) * 2u;
        oo[i] = (uint32_t)(r * p.s_do[1] + col(g, i, lane)) * 2u;
      }
      clamped = true;
    }
  }
  // DMA instruction i of the job: 0-3 the Q blocks, 4-7 the dO blocks.
  template <int i>
  __device__ __forceinline__ void issue() const {
    constexpr uint32_t off = (i < 4 ? 0u : kDoOff) + (uint32_t)(i & 3) * 1024u;
    if constexpr (i < 4) dma16_sva(qb, qo[i & 3], dst + off);
    else dma16_sva(ob, oo[i & 3], dst + off);
  }
  __device__ __forceinline__ void issue_stats(int lane) const {
    dma16_sva(sb, 16u * (uint32_t)lane, sdst);
  }
};

// dV^T / dK^T += A B on AGPR accumulators (inline asm: the builtin would
// follow the function-wide VGPR accumulator form). The accumulators are only
// read by VALU code behind fence_acc(); the A / B operands are read when the
// MFMA issues.
__device__ __forceinline__ void mfma_acc(f32x16& acc, bf16x8 a, bf16x8 b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
__device__ __forceinline__ void keep_alive(bf16x8 v) { asm volatile("" ::"v"(v)); }

__device__ __forceinline__ f32x4 lds_ld16f(uint32_t addr) {
  return __builtin_bit_cast(f32x4, lds_ld16(addr));
}

struct DkWave {
  bf16x8 kop[8], vop[8];  // K^T / V^T (kk): lane holds K / V[key li][16 kk + 8 hh + 0..7]; AGPRs
  f32x16 av[4], ak[4];    // dV^T, dK^T (dt): d = 32 dt + rows, key li; AGPRs
  f32x16 xs[2][2];        // S (buffer, hq)
  f32x16 xp[2][2];        // dP - D (buffer, hq)
  bf16x8 bp[4], bz[4];    // P, dZ of the tile (c4): queries of chunk c4 in accumulator order, key li
  float c;
  int li, hh;
  uint32_t rrd[4];  // LDS byte address of the row-operand reads of the next tile (Q tile;
                    // dual_row_rd(lane, j)); advanced one stage per tile
  uint32_t trd[4];  // ... of the transposed reads of this tile (dual_tr_rd(lane, p, r2) at
                    // 2 p + r2)
  uint32_t sthis, snext;  // LDS byte address of this lane's stats in this / the next tile's record

  __device__ __forceinline__ void setup(int lane, float c_, uint32_t ring) {
    li = lane & 31;
    hh = lane >> 5;
#pragma unroll
    for (int j = 0; j < 4; ++j) rrd[j] = ring + 2u * (uint32_t)dual_row_rd(lane, j);
#pragma unroll
    for (int q = 0; q < 4; ++q) trd[q] = ring + 2u * (uint32_t)dual_tr_rd(lane, q >> 1, q & 1);
    c = c_;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      av[dt] = f32x16{};
      ak[dt] = f32x16{};
      asm volatile("" : "+a"(av[dt]), "+a"(ak[dt]));
    }
  }

  // K^T and V^T operands from this wave's staged rows (32 K rows, then 32 V
  // rows), kept in AGPRs.
  __device__ __forceinline__ void read_kv(const bf16* kst, const bf16* vst, int lane) {
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      kop[kk] = staged_operand(kst, lane, kk);
      vop[kk] = staged_operand(vst, lane, kk);
      asm volatile("" : "+a"(kop[kk]), "+a"(vop[kk]));
    }
  }

  // Row operand j of the next tile: j < 16: Q rows (hq = j & 1, kk = j >> 1)
  // for S; j >= 16: dO rows (hq = j & 1, kk = (j - 16) >> 1) for dP.
  template <int j>
  __device__ __forceinline__ bf16x8 row_op() const {
    constexpr int hq = j & 1, kk = (j & 15) >> 1;
    constexpr uint32_t off = (j < 16 ? 0u : kDoOff) + 8192u * (kk >> 2) + 4096u * hq;
    return lds_ld16(rrd[kk & 3] + off);
  }
  // Transposed operand j of this tile (slot 32 + j): even j: dO^T (dt, c4)
  // for dV; odd j: Q^T (dt, c4) for dK; c4 = j >> 3, dt = (j >> 1) & 3.
  template <int j>
  __device__ __forceinline__ bf16x8 tr_op() const {
    constexpr int c4 = j >> 3, dt = (j >> 1) & 3;
    constexpr uint32_t off = ((j & 1) ? 0u : kDoOff) + 8192u * (dt >> 1) + 2048u * c4;
    const s16x4 lo = lds_ld8_tr(trd[2 * (dt & 1)] + off);
    const s16x4 hi = lds_ld8_tr(trd[2 * (dt & 1) + 1] + off + 1024u);
    return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  }

  // -D of the next tile's queries into the dP - D accumulators of buffer B
  // (step k = 4 hq + rq: registers 4 rq .. 4 rq + 3 of half hq).
  template <int B, int k>
  __device__ __forceinline__ void load_negd() {
    constexpr int hq = k >> 2, rq = k & 3;
    const f32x4 v = lds_ld16f(snext + kNegDOff + 128u * hq + 32u * rq);
#pragma unroll
    for (int i = 0; i < 4; ++i) xp[B][hq][4 * rq + i] = v[i];
  }

  // S (j < 16) or dP - D (j >= 16) MFMA j of the next tile into buffer B.
  template <int B, int j>
  __device__ __forceinline__ void next_mfma(bf16x8 a) {
    constexpr int hq = j & 1, kk = (j & 15) >> 1;
    if constexpr (j < 16) xs[B][hq] = mfma32(a, kop[kk], kk == 0 ? f32x16{} : xs[B][hq]);
    else xp[B][hq] = mfma32(a, vop[kk], xp[B][hq]);
  }

  // Unit u of buffer B, in four stages (see unit_slot). l2: the lse2 values
  // of the unit's pair (queries 32 hq + 8 rq + 4 hh .. + 3).
  template <int B, int u>
  __device__ __forceinline__ void u_fma(const f32x4& l2, float (&fa)[2][2]) const {
    constexpr int c4 = u >> 2, jp = u & 3, hq = c4 >> 1, r = 8 * (c4 & 1) + 2 * jp, e = 2 * (jp & 1);
    fa[u & 1][0] = fmaf(xs[B][hq][r], c, -l2[e]);
    fa[u & 1][1] = fmaf(xs[B][hq][r + 1], c, -l2[e + 1]);
    asm volatile("" : "+v"(fa[u & 1][0]), "+v"(fa[u & 1][1]));
  }
  template <int u>
  __device__ __forceinline__ void u_exp(const float (&fa)[2][2], float (&fe)[2][2]) const {
    fe[u & 1][0] = fast_exp2(fa[u & 1][0]);
    fe[u & 1][1] = fast_exp2(fa[u & 1][1]);
    asm volatile("" : "+v"(fe[u & 1][0]), "+v"(fe[u & 1][1]));
  }
  template <int B, int u>
  __device__ __forceinline__ void u_pack_p(const float (&fe)[2][2], float (&fz)[2][2]) {
    constexpr int c4 = u >> 2, jp = u & 3, hq = c4 >> 1, r = 8 * (c4 & 1) + 2 * jp;
    bp[c4][2 * jp] = (bf16)fe[u & 1][0];
    bp[c4][2 * jp + 1] = (bf16)fe[u & 1][1];
    fz[u & 1][0] = fe[u & 1][0] * xp[B][hq][r];
    fz[u & 1][1] = fe[u & 1][1] * xp[B][hq][r + 1];
    asm volatile("" : "+v"(bp[c4]), "+v"(fz[u & 1][0]), "+v"(fz[u & 1][1]));
  }
  template <int u>
  __device__ __forceinline__ void u_pack_z(const float (&fz)[2][2]) {
    constexpr int c4 = u >> 2, jp = u & 3;
    bz[c4][2 * jp] = (bf16)fz[u & 1][0];
    bz[c4][2 * jp + 1] = (bf16)fz[u & 1][1];
    asm volatile("" : "+v"(bz[c4]));
  }

  // Moves the row-operand / transposed read bases on by `delta` bytes.
  __device__ __forceinline__ void advance_rows(uint32_t delta) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      rrd[j] += delta;
      asm volatile("" : "+v"(rrd[j]));
    }
  }
  __device__ __forceinline__ void advance_tr(uint32_t delta) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      trd[j] += delta;
      asm volatile("" : "+v"(trd[j]));
    }
  }

  // S and dP - D of the range's first tile into buffer B (no other work).
  template <int B>
  __device__ __forceinline__ void first() {
    bf16x8 rq[kRQ];
    static_for<0, 32>([&](auto G) {
      constexpr int g = decltype(G)::value;
      if constexpr (g < 8) this->template load_negd<B, g>();
      static_for<0, 32>([&](auto J) {
        constexpr int j = decltype(J)::value;
        if constexpr (rread_slot(j) == g) rq[j % kRQ] = this->template row_op<j>();
      });
      this->template next_mfma<B, g>(rq[g % kRQ]);
      __builtin_amdgcn_sched_barrier(0);
    });
  }

  // One tile t of the slot schedule: P, dZ, dV^T, dK^T of tile t (its S and
  // dP - D in buffer SB); with NEXT, S and dP - D of tile t+1 (its rows one
  // ring stage, dstage bytes, past tile t's) into buffer 1 - SB. The DMA job
  // is issued in its slots (and the stats record by wave 0).
  template <int SB, bool NEXT>
  __device__ __forceinline__ void tile(uint32_t dstage, uint32_t dstat, const QdoDma& dma,
                                       bool stats_dma, int lane) {
    constexpr int NB = 1 - SB;
    if constexpr (NEXT) {
      advance_rows(dstage);
      snext = sthis + dstat;
    }
    bf16x8 rq[kRQ], tq[kTQ];
    f32x4 l2[2];
    float fa[2][2], fe[2][2], fz[2][2];
    static_for<0, 64>([&](auto G) {
      constexpr int g = decltype(G)::value;
      if constexpr (NEXT && g < 8) this->template load_negd<NB, g>();
      // Operand reads.
      if constexpr (NEXT) {
        static_for<0, 32>([&](auto J) {
          constexpr int j = decltype(J)::value;
          if constexpr (rread_slot(j) == g) rq[j % kRQ] = this->template row_op<j>();
        });
      }
      static_for<0, 32>([&](auto J) {
        constexpr int j = decltype(J)::value;
        if constexpr (tread_slot(j) == g) tq[j % kTQ] = this->template tr_op<j>();
      });
      // lse2 of each unit pair, two slots before its first unit.
      static_for<0, 16>([&](auto U) {
        constexpr int u = decltype(U)::value;
        if constexpr ((u & 1) == 0 && unit_slot(u) - 2 == g) {
          constexpr int c4 = u >> 2, jp = u & 3, hq = c4 >> 1, rq4 = 2 * (c4 & 1) + (jp >> 1);
          l2[(u >> 1) & 1] = lds_ld16f(sthis + 128u * hq + 32u * rq4);
        }
      });
      // The slot's MFMA.
      if constexpr (g < 32) {
        if constexpr (NEXT) this->template next_mfma<NB, g>(rq[g % kRQ]);
      } else {
        constexpr int j = g - 32, c4 = j >> 3, dt = (j >> 1) & 3;
        if constexpr ((j & 1) == 0) mfma_acc(av[dt], tq[j % kTQ], bp[c4]);
        else mfma_acc(ak[dt], tq[j % kTQ], bz[c4]);
      }
      // P / dZ units of tile t.
      static_for<0, 16>([&](auto U) {
        constexpr int u = decltype(U)::value;
        if constexpr (unit_slot(u) == g) this->template u_fma<SB, u>(l2[(u >> 1) & 1], fa);
        if constexpr (unit_slot(u) + 1 == g) this->template u_exp<u>(fa, fe);
        if constexpr (unit_slot(u) + 2 == g) this->template u_pack_p<SB, u>(fe, fz);
        if constexpr (unit_slot(u) + 3 == g) this->template u_pack_z<u>(fz);
      });
      // DMA.
      static_for<0, 8>([&](auto I) {
        constexpr int i = decltype(I)::value;
        if constexpr (dma_slot(i) == g) dma.template issue<i>();
      });
      if constexpr (g == kStatSlot) {
        if (stats_dma) dma.issue_stats(lane);
      }
      // The operands of the previous slot's inline-asm MFMA stay allocated to
      // the end of this slot: the compiler does not see that MFMA still
      // reading them.
      if constexpr (g > 32) {
        constexpr int j = g - 33, c4 = j >> 3;
        keep_alive(tq[j % kTQ]);
        if constexpr ((j & 1) == 0) keep_alive(bp[c4]);
        else keep_alive(bz[c4]);
      }
      __builtin_amdgcn_sched_barrier(0);
    });
    keep_alive(tq[31 % kTQ]);
    keep_alive(bz[3]);
    advance_tr(dstage);
    if constexpr (NEXT) sthis = snext;
  }

  // Keeps the accumulators in AGPRs up to this point and orders the VALU code
  // that follows after every MFMA that wrote them.
  __device__ __forceinline__ void fence_acc() {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3"
                 : "+a"(av[0]), "+a"(av[1]), "+a"(av[2]), "+a"(av[3]), "+a"(ak[0]), "+a"(ak[1]),
                   "+a"(ak[2]), "+a"(ak[3]));
  }
};

__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(1, 1)))
void dkdv1w_kernel(Params p, int nkblk, int total_blocks) {
  __shared__ __attribute__((aligned(1024))) bf16 ring[kStages * 2 * kTileElems];
  __shared__ __attribute__((aligned(1024))) float stat[kStages * kStat];

  const int logical = xcd_remap(blockIdx.x, total_blocks);
  const int per_split = total_blocks / p.nsplit;
  const int split = logical / per_split;
  const int rest = logical - split * per_split;
  const int kblk = rest % nkblk;
  const int bh = rest / nkblk;
  const int b = bh / p.H, h = bh - (bh / p.H) * p.H;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int key0 = kblk * kKeysPerWg + wave * 32;

  // Query tiles tq0 .. tq0 + ntiles - 1 (all of them without a split).
  const int tper = (p.ntq + p.nsplit - 1) / p.nsplit;
  const int tq0 = min(split * tper, p.ntq);
  const int ntiles = min(tper, p.ntq - tq0);
  const float* statb = p.stats + ((int64_t)bh * p.ntq + tq0) * kStat;

  const uint32_t ring0 = lds_addr(ring);
  const uint32_t stat0 = lds_addr(stat);
  auto stage_addr = [&](int t) -> uint32_t { return ring0 + (uint32_t)(t % kStages) * kStageBytes; };
  auto stat_addr = [&](int t) -> uint32_t { return stat0 + (uint32_t)(t % kStages) * kStatBytes; };

  DkWave w;
  w.setup(lane, p.c, ring0);
  w.sthis = stat0 + 16u * (uint32_t)w.hh;
  // The wave's K and V rows staged in ring stages 2 and 3 (16 KB per wave),
  // free until tile 2's DMA, which goes out after the barrier that follows
  // every wave's read. Keys past Sk re-read key Sk - 1 (never stored).
  bf16* kst = ring + 2 * (2 * kTileElems) + wave * 8192;
  stage_rows_in(p.k + b * p.s_k[0] + h * p.s_k[2], p.s_k[1], key0, p.Sk, lane, kst);
  stage_rows_in(p.v + b * p.s_v[0] + h * p.s_v[2], p.s_v[1], key0, p.Sk, lane, kst + 4096);

  const bf16* qbase = p.q + b * p.s_q[0] + h * p.s_q[2];
  const bf16* obase = p.dout + b * p.s_do[0] + h * p.s_do[2];
  QdoDma dma;
  dma.fixed(p, wave, lane);
  const bool stats_dma = wave == 0;
  // The job of tile t; past the range, a dummy job that re-reads the range's
  // first tile into the stage, which nothing reads again: every tile then
  // issues the same number of DMA instructions and one vmcnt serves every
  // wait.
  auto prepare_job = [&](int t) {
    const int tt = t < ntiles ? t : 0;
    dma.prepare(p, (tq0 + tt) * kT, stage_addr(t), stat_addr(t), statb + (int64_t)tt * kStat, wave,
                qbase, obase, lane);
  };
  auto issue_job = [&](int t) {  // the whole job of tile t at once
    prepare_job(t);
    static_for<0, 8>([&](auto I) { dma.template issue<decltype(I)::value>(); });
    if (stats_dma) dma.issue_stats(lane);
  };
  if (ntiles > 0) {
    issue_job(0);
    issue_job(1);
    // The K / V rows and tile 0 (tile 1's job, issued last, may still be in
    // flight: the first tile's top waits for it).
    if (stats_dma) asm volatile("s_waitcnt vmcnt(9)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  } else {
    wait_dma();
  }
  __syncthreads();  // tile 0 and every wave's K / V rows
  w.read_kv(kst, kst + 4096, lane);
  __syncthreads();  // every wave has read its K / V rows
  if (ntiles > 0) {
    issue_job(2);
    // S of tile t lives in buffer (b0 + t) & 1, with b0 chosen so that the
    // last tile, the one without a next tile, always uses buffer 0.
    const int b0 = (ntiles - 1) & 1;
    w.snext = w.sthis;  // tile 0's record
    if (b0) w.first<1>();
    else w.first<0>();

    // Tile t: at its top, tile t+1 (issued two tiles earlier) is complete in
    // this wave (the job of tile t+2 may be in flight) and the barrier
    // publishes every wave's part. The job issued during tile t, tile t+3,
    // reuses the stage of tile t-1, whose rows and stats were last read in
    // tile t-1, before that barrier.
    auto top = [&](int t) {
      if (stats_dma) asm volatile("s_waitcnt vmcnt(9)" ::: "memory");
      else asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
      __syncthreads();
      prepare_job(t + kLead);
    };
    auto run = [&](auto sb, auto next, int t) {
      constexpr int SB = decltype(sb)::value;
      constexpr bool NEXT = decltype(next)::value;
      top(t);
      w.tile<SB, NEXT>(stage_addr(t + 1) - stage_addr(t), stat_addr(t + 1) - stat_addr(t), dma,
                       stats_dma, lane);
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    int t = 0;
    if (b0) {
      run(I1{}, std::true_type{}, 0);
      t = 1;
    }
    for (; t + 1 < ntiles; t += 2) {
      run(I0{}, std::true_type{}, t);
      run(I1{}, std::true_type{}, t + 1);
    }
    run(I0{}, std::false_type{}, t);  // t == ntiles - 1
  }
  wait_dma();
  __syncthreads();  // every wave is done with the ring; no DMA in flight

  w.fence_acc();
  if (p.nsplit > 1) {
    // Partial accumulators: record wave (dV^T) and 4 + wave (dK^T), 16
    // coalesced 1 KB stores each.
    f32x4* dst = reinterpret_cast<f32x4*>(p.part) + ((int64_t)logical * kDkParts + wave) * 16 * 64 + lane;
    f32x4* dstk = dst + (int64_t)kWaves * 16 * 64;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const f32x16& v = w.av[j >> 2];
      const f32x16& k = w.ak[j >> 2];
      const int e = 4 * (j & 3);
      __builtin_nontemporal_store(f32x4{v[e], v[e + 1], v[e + 2], v[e + 3]}, dst + j * 64);
      __builtin_nontemporal_store(f32x4{k[e], k[e + 1], k[e + 2], k[e + 3]}, dstk + j * 64);
    }
    return;
  }
  // dV and dK rows out through the ring: 16 KB per wave.
  bf16* ostage = ring + wave * 8192;
  const f32x16 va[4] = {w.av[0], w.av[1], w.av[2], w.av[3]};
  stage_acc_rows(va, 1.0f, lane, ostage);
  stage_rows_out(p.dv + b * p.s_dv[0] + h * p.s_dv[2], p.s_dv[1], key0, p.Sk, lane, ostage);
  const f32x16 ka[4] = {w.ak[0], w.ak[1], w.ak[2], w.ak[3]};
  stage_acc_rows(ka, p.scale, lane, ostage + 4096);
  stage_rows_out(p.dk + b * p.s_dk[0] + h * p.s_dk[2], p.s_dk[1], key0, p.Sk, lane, ostage + 4096);
}

}  // namespace w1

void launch_dkdv1w(const Params& p, int nkblk, int total, hipStream_t stream) {
  w1::dkdv1w_kernel<<<dim3((unsigned)total), w1::kWaves * 64, 0, stream>>>(p, nkblk, total);
}

}  // namespace bwd
}  // namespace aa
