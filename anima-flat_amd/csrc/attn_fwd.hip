// Flash-attention forward, non-causal, head_dim 128, bf16 in / fp32 accumulate,
// for gfx950 (CDNA4): v_mfma_f32_32x32x16_bf16 for both products.
//
// Work decomposition
//   One workgroup = 4 waves, one per SIMD, = 256 queries of one (batch,
//   head). Each wave owns 64 queries (two blocks of 32) for the whole key
//   range; K/V tiles of 64 keys stream through a 4-stage LDS ring that the 4
//   waves share. Every K or V^T operand a wave reads from LDS feeds two MFMAs
//   (one per query block): 0.5 KB of LDS reads per MFMA.
//
// Why one wave per SIMD with 64 queries: a 32x32x16 MFMA holds up the
//   SIMD's issue of other vector work for about 20 of the 32 cycles it keeps
//   the matrix pipe busy, so a tile costs the SIMD roughly the sum of its MFMA,
//   softmax VALU and LDS-read issue time, whichever wave issues them. With 32
//   queries per wave (two waves per SIMD) every MFMA needed its own 1 KB
//   operand, two LDS reads; with 64 queries the same operand serves two
//   MFMAs, which removes a quarter of the per-tile issue time.
//
// Transposed formulation (per wave, per 64-key tile, per query block qb)
//   S^T = K Q^T   : A = K rows from the LDS line tile (32 keys x 16 d per
//                   MFMA), B = Q^T from registers (loaded once).
//   O^T += V^T P^T: A = V^T (32 d x 16 keys), read transposed from the LDS
//                   V rows, B = P^T from the S^T accumulators.
//   The 32x32 accumulator layout puts column j = lane%32 in every lane, with
//   rows 8*(r/4) + 4*(lane/32) + r%4 in register r. With queries as columns,
//   every lane holds one query of each block: the softmax row max/sum are
//   in-lane reductions plus one v_permlane32_swap with the partner lane, and
//   the output rescale is a per-lane scalar multiply.
//
// Slot schedule: a tile is 64 slots of one MFMA each; the other work of the
//   tile is dealt to fixed slots and held there by sched_barrier:
//     slots  0-31: S^T of tile t+1 (QK)     | P of tile t (fma, exp, bf16, sums)
//     slots 32-63: O^T += V^T P^T of tile t | the rest of P (in the fix-up
//                                             form: then the row max of tile
//                                             t+1, and the rare lazy rescale)
//   The K/V DMA of tile t+3 is issued one instruction per 4 slots.
//
// K/V staging (tile_io.h): K and V rows are copied HBM -> LDS by DMA
//   (global_load_lds_dwordx4) into line tiles, blocks of 8 rows x 64 d that
//   one DMA instruction fills from 8 whole 128-byte lines; the 16-byte chunk
//   XOR differs: K's suits its 16-byte ds_read_b128 operand reads, V's its
//   V^T operands, pairs of ds_read_b64_tr_b16 transposed reads. Both are free
//   of bank conflicts.
//
// Q and O staging: each wave's 64 Q rows come in by DMA (4 rows x 256 B per
//   instruction) into ring stages that the first tiles do not use, and are
//   read into the Q^T registers from there; O leaves the same way through the
//   ring after the last tile, 4 whole rows per store.
//
// Key order of P^T
//   The B operand of the MFMA wants, in lane l, 8 consecutive k-indices
//   8*(l/32)+i of a 16-key chunk. The S^T accumulators hold, for that lane,
//   keys {4h..4h+3, 8+4h..8+4h+3} (h = l/32) of the chunk. Since PV sums over
//   keys, the V^T operand only has to list its keys in the same order, which
//   the transposed reads do by addressing those rows.
//
// Softmax: first-tile max, fix-up with a running max
//   Probabilities are p = exp2(s*c - m*c) on raw scores s = q.k with
//   c = scale * log2(e), one FMA and one v_exp_f32 per score. m is the row
//   max of the range's first tile, kept for the whole range (see
//   attn_fwd_fixup_kernel for the rows where that leaves the exponent range).
//   The fix-up form tracks the running max with lazy rescaling: m is only
//   raised when a tile's max exceeds it by more than 8/c (8 in log2 units),
//   so p <= 256 and the O/l rescale (a pass over the 128 accumulator
//   registers) runs only a few times per row. The row sum is
//   taken over the bf16-rounded P that feeds the MFMA, on the matrix pipe: a
//   v_mfma_f32_16x16x32_bf16 of each P operand against a 0/1 selector (see
//   FwdWave::setup), 8 small MFMAs per tile in place of 32 v_dot2c_f32_bf16,
//   each of which held the matrix pipe for about half an MFMA.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <mutex>
#include <string>
#include <type_traits>

#include "attn_fwd.h"
#include "attn_fwd_d384.h"
#include "tile_io.h"

namespace aa {

constexpr int kWaves = 4;                    // one per SIMD
constexpr int kQPerWave = 64;                // two blocks of 32 queries
static_assert(kWaves * kQPerWave == kQPerWg, "work item size");
constexpr int kStages = 4;                   // K/V ring depth (4 x 32 KB)
constexpr int kLead = kStages - 1;           // tile t + kLead is fetched during tile t
constexpr uint32_t kStageBytes = 2u * kTileElems * sizeof(bf16);  // K tile, then V tile
constexpr uint32_t kVOff = kTileElems * sizeof(bf16);             // V tile in a stage

// K/V tile DMA of one wave into the K and V line tiles of a ring stage
// (tile_io.h). A DMA instruction fills one 1 KB block = 8 rows x 64 d from 8
// whole 128-byte lines; wave w fills blocks 4 w .. 4 w + 3 of the K tile and
// of the V tile: d-half w >> 1, rows 32 (w & 1) + 8 i + (lane >> 3),
// i = 0..3. A job (one tile) takes one scalar base per tensor (the tile's
// first row) and per-lane 32-bit byte offsets that hold each lane's row and
// column, so its instructions need no address arithmetic. Rows at or past Sk
// re-read row Sk - 1: finite data, and rows at or past the key length have
// their scores masked to -inf (P = 0).
struct KVDma {
  uint32_t ko[4], vo[4];      // per-lane offsets of blocks 0-3 (those of a tile inside Sk
                              // unless `clamped`)
  bool clamped;
  const bf16* kbase;          // this job's scalar bases
  const bf16* vbase;
  uint32_t dst;               // LDS byte address of this job's first K block

  __device__ __forceinline__ static int row_of(int wave, int i, int lane) {
    return 32 * (wave & 1) + 8 * i + (lane >> 3);
  }
  __device__ __forceinline__ static int kcol(int wave, int i, int lane) {
    return 64 * (wave >> 1) + 8 * line_k_chunk(lane, i & 1);
  }
  __device__ __forceinline__ static int vcol(int wave, int lane) {
    return 64 * (wave >> 1) + 8 * line_v_chunk(lane);
  }

  __device__ __forceinline__ void fixed(const FwdParams& p, int wave, int lane) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = row_of(wave, i, lane);
      ko[i] = (uint32_t)(r * p.ks1 + kcol(wave, i, lane)) * 2u;
      vo[i] = (uint32_t)(r * p.vs1 + vcol(wave, lane)) * 2u;
    }
    clamped = false;
  }
  __device__ __forceinline__ void setup(const FwdParams& p, int wave, int lane) {
    fixed(p, wave, lane);
  }

  // The job of the tile whose first key row is kbrow (when real), else a
  // dummy job that moves rows from 0 into the same stage, which nothing reads
  // again: every tile then issues the same number of DMA instructions and one
  // vmcnt serves every wait. Only a tile that reaches past Sk (or a dummy job
  // with Sk < 64) needs clamped offsets.
  __device__ __forceinline__ void prepare(const FwdParams& p, bool real, int kbrow, uint32_t stage,
                                          int wave, const bf16* kp, const bf16* vp, int lane) {
    const int row0 = real ? kbrow : 0;
    dst = stage + (uint32_t)(4 * wave) * 1024u;
    if (row0 + kBN <= p.Sk) {
      kbase = kp + (int64_t)row0 * p.ks1;
      vbase = vp + (int64_t)row0 * p.vs1;
      if (clamped) fixed(p, wave, lane);
    } else {
      const int last = p.Sk - 1;
      const int rs = min(row0, last);
      kbase = kp + (int64_t)rs * p.ks1;
      vbase = vp + (int64_t)rs * p.vs1;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = min(row0 + row_of(wave, i, lane), last) - rs;
        ko[i] = (uint32_t)(r * p.ks1 + kcol(wave, i, lane)) * 2u;
        vo[i] = (uint32_t)(r * p.vs1 + vcol(wave, lane)) * 2u;
      }
      clamped = true;
    }
  }

  // DMA instruction i of the job: 0-3 the K blocks, 4-7 the V blocks.
  template <int i>
  __device__ __forceinline__ void issue() const {
    constexpr uint32_t off = (i < 4 ? 0u : kVOff) + (uint32_t)(i & 3) * 1024u;
    if constexpr (i < 4) dma16_sva(kbase, ko[i & 3], dst + off);
    else dma16_sva(vbase, vo[i & 3], dst + off);
  }
};

// Operand reads ahead of their MFMA: K operands (each feeds the two MFMAs of
// a pair of slots) are read kKPf pairs ahead, V^T operands kVPf pairs ahead
// into a queue one entry longer than that needs (a V^T operand stays
// allocated for one slot after its last MFMA).
constexpr int kKPf = 2, kKQ = kKPf + 1;
constexpr int kVPf = 2, kVQ = kVPf + 2;
constexpr int kread_slot(int j) { return j < kKPf ? 0 : 2 * (j - kKPf); }
constexpr int vread_slot(int pp) { return 32 + 2 * (pp - kVPf); }
// P unit u (2 scores of query block (u >> 2) & 1, key chunk u >> 3) starts in
// slot 3u / 2 and ends two slots later (slots 0-48); the P operand of chunk c4
// is first used in slot 32 + 8 c4, after its last unit. Max steps of the next
// tile: slots 48-63.
constexpr int exp_slot(int u) { return (3 * u) / 2; }
constexpr int kMaxSlot0 = 48;
// DMA instruction i of the tile's job: slot 4 i + 3.
constexpr int dma_slot(int i) { return 4 * i + 3; }

// O^T += V^T P^T with O in AGPRs, as inline asm: the builtin would follow the
// function-wide choice of one register file for every MFMA accumulator, and S
// must stay in VGPRs for the softmax. O is only read or written by VALU code
// behind fence_o(), and the A/B operands are read when the MFMA issues.
__device__ __forceinline__ void mfma_pv(f32x16& acc, bf16x8 a, bf16x8 b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
__device__ __forceinline__ void keep_alive(bf16x8 v) { asm volatile("" ::"v"(v)); }
// Row sums (the accumulator and the 0/1 selector in AGPRs, as for O).
__device__ __forceinline__ void mfma_rowsum(f32x4& acc, bf16x8 sel, bf16x8 p) {
  asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "a"(sel), "v"(p));
}

// Per-wave state and work: 64 queries (blocks qb = 0, 1 of 32), their Q^T
// operands, O^T accumulators and running softmax statistics.
struct FwdWave {
  bf16x8 qreg[2][8];  // Q^T (qb, kk): lane holds Q[32 qb + li][16 kk + 8 hh + 0..7]; AGPRs
  f32x16 o[4][2];     // O^T (dt, qb): d = 32 dt + rows, query 32 qb + li; AGPRs
  f32x16 s[2][2][2];  // S^T (buffer, kb, qb): keys 32 kb + rows of the tile, query 32 qb + li
  bf16x8 pb[4][2];    // P^T (c4, qb): keys 16 c4 + .. of the tile, in accumulator order
  float m_raw[2];     // running max of query 32 qb + li, raw score units
  float mt[2];        // row max of the next tile (raw)
  f32x4 lsum[2];      // row sum of query 32 qb + li (all four elements), by MFMA
  bf16x8 sel;         // 0/1 selector: the A operand of the row-sum MFMA
  float c, thr_raw;
  int li, hh;
  uint32_t kb4[4];  // LDS byte address of this lane's K operand reads in the next tile's K
                    // (line_k_rd(lane, j)); advanced one stage per tile
  uint32_t vb2[2];  // ... of its V^T operand reads in this tile's V (line_v_tr(lane, p))

  // LDS read bases start at ring stage 0 (tile 0).
  __device__ __forceinline__ void setup(int lane, float c_, uint32_t ring) {
    li = lane & 31;
    hh = lane >> 5;
#pragma unroll
    for (int j = 0; j < 4; ++j) kb4[j] = ring + 2u * (uint32_t)line_k_rd(lane, j);
    vb2[0] = ring + kVOff + 2u * (uint32_t)line_v_tr(lane, 0);
    vb2[1] = ring + kVOff + 2u * (uint32_t)line_v_tr(lane, 1);
    c = c_;
    thr_raw = kRescaleThreshold / c;
    // Zeros pinned into AGPRs, the file every later MFMA keeps O in.
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        o[dt][qb] = f32x16{};
        asm volatile("" : "+a"(o[dt][qb]));
      }
    m_raw[0] = m_raw[1] = -INFINITY;
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      lsum[qb] = f32x4{};
      asm volatile("" : "+a"(lsum[qb]));
    }
    // Row sums by v_mfma_f32_16x16x32_bf16 with the P^T operand as B: in that
    // shape lane l's 8 values are B[k = 8 (l / 16) + i][n = l % 16], i.e.
    // query n (+16 for odd l / 16) over one half of the chunk's keys. With
    // A[m][k] = 1 where bit 2 of m equals bit 3 of k, D[m][n] sums query n
    // for m % 8 < 4 and query n + 16 otherwise, which puts the row sum of
    // query li = lane % 32 in all four D values of lane `lane`.
    {
      const bf16 one = (bf16)(((lane & 15) >> 2 & 1) == ((lane >> 4) & 1) ? 1.0f : 0.0f);
#pragma unroll
      for (int i = 0; i < 8; ++i) sel[i] = one;
      asm volatile("" : "+a"(sel));
    }
  }

  // Q^T operands from this wave's 64 staged rows (two 32-row staging areas),
  // kept in AGPRs (the MFMA reads its B operand from either file).
  __device__ __forceinline__ void read_q(const bf16* stage, int lane) {
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        qreg[qb][kk] = staged_operand(stage + qb * 4096, lane, kk);
        asm volatile("" : "+a"(qreg[qb][kk]));
      }
  }

  // K operand pair j = 8 kb + kk (keys 32 kb .., head-dim 16 kk ..) of the K
  // tile at kb4.
  template <int j>
  __device__ __forceinline__ bf16x8 k_op() const {
    constexpr int kb = j >> 3, kk = j & 7;
    return lds_ld16(kb4[kk & 3] + 8192u * (kk >> 2) + 4096u * kb);
  }
  // V^T operand pair pp = 4 c4 + dt (d 32 dt .., keys of chunk c4).
  template <int pp>
  __device__ __forceinline__ bf16x8 v_op() const {
    constexpr int c4 = pp >> 2, dt = pp & 3;
    constexpr uint32_t off = 8192u * (dt >> 1) + 2048u * c4;
    const s16x4 lo = lds_ld8_tr(vb2[dt & 1] + off);
    const s16x4 hi = lds_ld8_tr(vb2[dt & 1] + off + 1024u);
    return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  }
  // Moves the K / V^T read bases on by `delta` bytes (the next ring stage).
  __device__ __forceinline__ void advance_k(uint32_t delta) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      kb4[j] += delta;
      asm volatile("" : "+v"(kb4[j]));
    }
  }
  __device__ __forceinline__ void advance_v(uint32_t delta) {
    vb2[0] += delta;
    vb2[1] += delta;
    asm volatile("" : "+v"(vb2[0]), "+v"(vb2[1]));
  }

  // Scores of keys at or past klen (tile at key offset kb) to -inf.
  template <int B>
  __device__ __forceinline__ void mask(int kb, int klen) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kb + 32 * kt + 8 * (r >> 2) + 4 * hh + (r & 3);
          if (key >= klen) s[B][kt][qb][r] = -INFINITY;
        }
  }

  // Max step k (0..15) of S^T buffer B: block kb = k >> 3, query block
  // qb = k & 1, registers 4 ((k >> 1) & 3) .. + 3, into mx[qb].
  template <int B, int k>
  __device__ __forceinline__ void max_step(float (&mx)[2]) const {
    constexpr int kb = k >> 3, qb = k & 1, r0 = 4 * ((k >> 1) & 3);
    const f32x16& a = s[B][kb][qb];
    if constexpr (k < 2) {
      mx[qb] = max2f(max3f(a[r0], a[r0 + 1], a[r0 + 2]), a[r0 + 3]);
    } else {
      mx[qb] = max3f(mx[qb], a[r0], a[r0 + 1]);
      mx[qb] = max3f(mx[qb], a[r0 + 2], a[r0 + 3]);
    }
  }

  // P unit u of S^T buffer B: scores 2 jp, 2 jp + 1 of the P operand (c4, qb),
  // c4 = u >> 3, qb = (u >> 2) & 1, jp = u & 3, and their sum, in three
  // stages one slot apart (fma, exp, pack + sum): the stages of consecutive
  // units share a slot, so no VALU instruction waits on the one before it.
  // fa / fe carry two units' values between the stages.
  template <int B, int u>
  __device__ __forceinline__ void p_fma(const float (&mc)[2], float (&fa)[2][2]) const {
    constexpr int c4 = u >> 3, qb = (u >> 2) & 1, jp = u & 3;
    constexpr int kb = c4 >> 1, r = 8 * (c4 & 1) + 2 * jp;
    fa[u & 1][0] = fmaf(s[B][kb][qb][r], c, -mc[qb]);
    fa[u & 1][1] = fmaf(s[B][kb][qb][r + 1], c, -mc[qb]);
    asm volatile("" : "+v"(fa[u & 1][0]), "+v"(fa[u & 1][1]));
  }
  template <int u>
  __device__ __forceinline__ void p_exp(const float (&fa)[2][2], float (&fe)[2][2]) const {
    fe[u & 1][0] = fast_exp2(fa[u & 1][0]);
    fe[u & 1][1] = fast_exp2(fa[u & 1][1]);
    asm volatile("" : "+v"(fe[u & 1][0]), "+v"(fe[u & 1][1]));
  }
  template <int u>
  __device__ __forceinline__ void p_pack(const float (&fe)[2][2]) {
    constexpr int c4 = u >> 3, qb = (u >> 2) & 1, jp = u & 3;
    pb[c4][qb][2 * jp] = (bf16)fe[u & 1][0];
    pb[c4][qb][2 * jp + 1] = (bf16)fe[u & 1][1];
    // Anchored in its slot: left alone, the compiler sinks the P work next to
    // its MFMA users.
    asm volatile("" : "+v"(pb[c4][qb]));
  }
  // Row sums of the P operand (c4, qb) on the matrix pipe (see setup): the
  // VALU alternatives cost the SIMD's vector issue (fp32 adds) or stall the
  // matrix pipe for half an MFMA each (v_dot2c_f32_bf16).
  template <int c4, int qb>
  __device__ __forceinline__ void p_sum() {
    mfma_rowsum(lsum[qb], sel, pb[c4][qb]);
  }

  // S^T of the first tile of the range (no other work to interleave).
  template <int B>
  __device__ __forceinline__ void qk_first() {
    bf16x8 kq[kKQ];
    static_for<0, 32 + 2 * kKPf>([&](auto G) {
      constexpr int g = decltype(G)::value;
      static_for<0, 16>([&](auto J) {
        constexpr int j = decltype(J)::value;
        if constexpr (kread_slot(j) == g) kq[j % kKQ] = this->template k_op<j>();
      });
      if constexpr (g < 32) {
        constexpr int j = g >> 1, kb = j >> 3, kk = j & 7, qb = g & 1;
        s[B][kb][qb] = mfma32(kq[j % kKQ], qreg[qb][kk], kk == 0 ? f32x16{} : s[B][kb][qb]);
      }
      __builtin_amdgcn_sched_barrier(0);
    });
  }

  // Row max of S^T buffer B into mt (no other work).
  template <int B>
  __device__ __forceinline__ void max_plain() {
    float mx[2];
    static_for<0, 16>([&](auto K) { this->template max_step<B, decltype(K)::value>(mx); });
    mt[0] = pair_max(mx[0]);
    mt[1] = pair_max(mx[1]);
  }

  // One tile t of the slot schedule. S^T of tile t is in buffer SB; with
  // NEXT, S^T of tile t+1 (its K one ring stage, dstage bytes, past tile t's)
  // goes to buffer 1 - SB (masked first when its keys end inside it:
  // mask_next) and, with TRACK, its row max to mt. The DMA job is issued in
  // its slots.
  template <int SB, bool NEXT, bool TRACK>
  __device__ __forceinline__ void tile(uint32_t dstage, bool mask_next, int kb_next, int klen,
                                       const KVDma& dma) {
    constexpr int NB = 1 - SB;
    const float mc[2] = {m_raw[0] * c, m_raw[1] * c};
    if constexpr (NEXT) advance_k(dstage);
    bf16x8 kq[kKQ], vq[kVQ];
    float mx[2];
    float fa[2][2], fe[2][2];
    static_for<0, 64>([&](auto G) {
      constexpr int g = decltype(G)::value;
      if constexpr (NEXT && g == kMaxSlot0) {
        if (mask_next) mask<NB>(kb_next, klen);
      }
      // Operand reads.
      if constexpr (NEXT) {
        static_for<0, 16>([&](auto J) {
          constexpr int j = decltype(J)::value;
          if constexpr (kread_slot(j) == g) kq[j % kKQ] = this->template k_op<j>();
        });
      }
      static_for<0, 16>([&](auto P) {
        constexpr int pp = decltype(P)::value;
        if constexpr (vread_slot(pp) == g) vq[pp % kVQ] = this->template v_op<pp>();
      });
      // The slot's MFMA.
      if constexpr (g < 32) {
        if constexpr (NEXT) {
          constexpr int j = g >> 1, kb = j >> 3, kk = j & 7, qb = g & 1;
          s[NB][kb][qb] = mfma32(kq[j % kKQ], qreg[qb][kk], kk == 0 ? f32x16{} : s[NB][kb][qb]);
        }
      } else {
        constexpr int op = g - 32, pp = op >> 1, c4 = pp >> 2, dt = pp & 3, qb = op & 1;
        mfma_pv(o[dt][qb], vq[pp % kVQ], pb[c4][qb]);
        if constexpr (dt == 2) this->template p_sum<c4, qb>();
      }

      // P units of tile t, three stages per unit.
      static_for<0, 32>([&](auto U) {
        constexpr int u = decltype(U)::value;
        if constexpr (exp_slot(u) == g) this->template p_fma<SB, u>(mc, fa);
        if constexpr (exp_slot(u) + 1 == g) this->template p_exp<u>(fa, fe);
        if constexpr (exp_slot(u) + 2 == g) this->template p_pack<u>(fe);
      });
      // Row max of tile t+1.
      if constexpr (NEXT && TRACK && g >= kMaxSlot0) {
        this->template max_step<NB, g - kMaxSlot0>(mx);
        asm volatile("" : "+v"(mx[0]), "+v"(mx[1]));
      }
      // DMA.
      static_for<0, 8>([&](auto I) {
        constexpr int i = decltype(I)::value;
        if constexpr (dma_slot(i) == g) dma.template issue<i>();
      });
      // The operands of the previous slot's inline-asm MFMA stay allocated to
      // the end of this slot: the compiler does not see that MFMA still
      // reading them and would hand their registers to this slot's VALU
      // results, whose writes would then wait for it.
      if constexpr (g > 32) {
        constexpr int op = g - 33, pp = op >> 1, c4 = pp >> 2, dt = pp & 3, qb = op & 1;
        keep_alive(vq[pp % kVQ]);
        if constexpr (dt == 3) keep_alive(pb[c4][qb]);
      }
      __builtin_amdgcn_sched_barrier(0);
    });
    keep_alive(vq[15 % kVQ]);
    keep_alive(pb[3][1]);
    advance_v(dstage);
    if constexpr (NEXT && TRACK) {
      mt[0] = pair_max(mx[0]);
      mt[1] = pair_max(mx[1]);
    }
  }

  // Keeps O in AGPRs up to this point and orders the VALU code that follows
  // after every MFMA that wrote it.
  __device__ __forceinline__ void fence_o() {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3"
                 : "+a"(o[0][0]), "+a"(o[1][0]), "+a"(o[2][0]), "+a"(o[3][0]), "+a"(o[0][1]),
                   "+a"(o[1][1]), "+a"(o[2][1]), "+a"(o[3][1]), "+a"(lsum[0]), "+a"(lsum[1]));
  }

  // Lazy rescale for the next tile's max mt: m is raised (and O and l scaled
  // down) only where mt exceeds it by more than thr_raw.
  __device__ __forceinline__ void update_max() {
    const bool n0 = mt[0] > m_raw[0] + thr_raw;
    const bool n1 = mt[1] > m_raw[1] + thr_raw;
    if (__builtin_amdgcn_ballot_w64(n0 || n1)) {
      const float mn0 = n0 ? mt[0] : m_raw[0];
      const float mn1 = n1 ? mt[1] : m_raw[1];
      const float a0 = fast_exp2((m_raw[0] - mn0) * c);
      const float a1 = fast_exp2((m_raw[1] - mn1) * c);
      fence_o();
      // One accumulator block at a time, pinned back into AGPRs: otherwise the
      // compiler reads all 128 values into VGPRs first.
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][0][r] *= a0;
        asm volatile("" : "+a"(o[dt][0]));
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][1][r] *= a1;
        asm volatile("" : "+a"(o[dt][1]));
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        lsum[0][r] *= a0;
        lsum[1][r] *= a1;
      }
      asm volatile("" : "+a"(lsum[0]), "+a"(lsum[1]));
      m_raw[0] = mn0;
      m_raw[1] = mn1;
    }
  }

  // After a pass that kept every row's first-tile max as m (no per-tile max,
  // no rescale): whether every row sum is at most 2^64 (so every p was
  // finite and 1/l is a normal number) and every O^T accumulator finite.
  // Then the result is the one a running max gives, up to fp32 rounding: m
  // only sets the exponent range. Reads O, so after fence_o().
  __device__ __forceinline__ bool sums_in_range() const {
    float mo = 0.f;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int r = 0; r < 16; r += 2) mo = max3abs(mo, o[dt][qb][r], o[dt][qb][r + 1]);
    return lsum[0][0] <= 0x1p64f && lsum[1][0] <= 0x1p64f && mo <= 0x1.fffffep127f;
  }

  // O (or the range's partial O) of query block qb: O / l, optional padding
  // correction, bf16, out through the 8 KB staging area `stage` (tile_io.h
  // row staging, 4 whole 256-byte rows per store); LSE in fp32.
  template <int qb>
  __device__ __forceinline__ float finish(float pad_ln, bool pad, bf16* obase, int64_t ors,
                                          int orow0, int onrows, int lane, bf16* stage) const {
    const float l_tot = lsum[qb][0];
    const bool any = l_tot > 0.f;
    const float lse = any ? (m_raw[qb] * c + __log2f(l_tot)) * kLn2 : -INFINITY;
    float scale = any ? 1.0f / l_tot : 0.f;
    if (pad) scale *= 1.0f / (1.0f + expf(pad_ln - lse));
    const f32x16 ob[4] = {o[0][qb], o[1][qb], o[2][qb], o[3][qb]};
    stage_acc_rows(ob, scale, lane, stage);
    stage_rows_out(obase, ors, orow0, onrows, lane, stage);
    return lse;
  }
};

// Exponent range. attn_fwd_kernel keeps every row's max at its first key
// tile's for the whole range (no per-tile max and no rescale: ~34 VALU
// instructions fewer per tile and wave), so p = exp2((s - m) c) only stays
// finite while no later score exceeds that max by ~64 in log2 units. m only
// sets the exponent range: the result is the one a running max gives, up to
// fp32 rounding, as long as every p, every row sum and O stay finite, which
// FwdWave::sums_in_range() checks after the pass. A workgroup with a row that
// failed it writes kRerunMark in place of its output, and
// attn_fwd_fixup_kernel, launched right after on the same stream, reads every
// block's mark place and runs the marked ones again with the running max and
// the lazy rescale (fwd_block<true>, the form attn_fwd_kernel<true> runs alone
// where one launch is cheaper).
//
// The mark: a NaN with a payload (the default quiet NaN converts to bf16
// 0x7fc0), in the first element of the block's output, the O row of its
// first query or its key range's partial O record. The first launch writes
// every block's output or its mark, so the mark place never holds a stale
// value; an output that holds the mark's bits anyway (a NaN input can carry
// that payload through) only costs an exact second run of its block.
constexpr uint16_t kRerunMark = 0x7fc1;

__device__ __forceinline__ int64_t part_record(const FwdParams& p, int item_idx, int split) {
  return (int64_t)(item_idx - p.full_blocks) * p.nsplit + split;
}

__device__ __forceinline__ uint16_t* mark_ptr(const FwdParams& p, int item_idx, int split) {
  const int qblk = item_idx % p.nqblk, bh = item_idx / p.nqblk;
  const int b = bh / p.H, h = bh - b * p.H;
  return reinterpret_cast<uint16_t*>(
      split < 0 ? p.o + b * p.os0 + (int64_t)qblk * kQPerWg * p.os1 + h * p.os2
                : p.part_o + part_record(p, item_idx, split) * kQPerWg * kD);
}

// One workgroup's work: block blk's work item (256 queries of one (batch,
// head)), or one key range of one of the last work items when they are split.
// TRACK: the running max with the lazy rescale, else the first tile's max
// (and the mark when a row leaves the range).
template <bool TRACK>
__device__ __forceinline__ void fwd_block(const FwdParams& p, int blk, bf16* kv_lds) {
  int item_idx, split;
  block_item(p, blk, item_idx, split);
  const int64_t part_row = part_record(p, item_idx, split);
  uint16_t* mark = mark_ptr(p, item_idx, split);
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
  const int lane = tid & 63;
  const int qrow0 = it.qblk * kQPerWg + wave * kQPerWave;  // the wave's first query

  const uint32_t ring = lds_addr(kv_lds);
  auto stage_addr = [&](int t) -> uint32_t { return ring + (uint32_t)(t % kStages) * kStageBytes; };

  FwdWave w;
  w.setup(lane, p.c, ring);
  // Q rows staged in ring stages 2 and 3 (16 KB per wave), free until tile
  // 2's DMA, which is issued after the barrier that follows every wave's read.
  bf16* qstage = kv_lds + 2 * (2 * kTileElems) + wave * 8192;
  {
    const bf16* qb = p.q + it.b * p.qs0 + it.h * p.qs2;
    stage_rows_in(qb, p.qs1, qrow0, p.Sq, lane, qstage);
    stage_rows_in(qb, p.qs1, qrow0 + 32, p.Sq, lane, qstage + 4096);
  }
  KVDma dma;
  dma.setup(p, wave, lane);
  const bf16* kp = p.k + it.b * p.ks0 + it.h * p.ks2;
  const bf16* vp = p.v + it.b * p.vs0 + it.h * p.vs2;
  auto issue_job = [&](int t) {  // the whole job of tile t at once
    dma.prepare(p, t < ntiles, (t0 + t) * kBN, stage_addr(t), wave, kp, vp, lane);
    static_for<0, 8>([&](auto I) { dma.template issue<decltype(I)::value>(); });
  };
  if (ntiles > 0) {
    issue_job(0);
    issue_job(1);
    // The Q rows and tile 0 (tile 1's 8 instructions may still be in
    // flight: the first tile's top waits for them).
    asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  } else {
    wait_dma();
  }
  __syncthreads();  // Q rows and tile 0 from every wave
  w.read_q(qstage, lane);
  __syncthreads();  // every wave has read its Q rows
  if (ntiles > 0) {
    issue_job(2);
    // S^T of tile t lives in buffer (b0 + t) & 1, with b0 chosen so that the
    // last tile, the one without a next tile, always uses buffer 0.
    const int b0 = (ntiles - 1) & 1;
    const int kb0 = t0 * kBN;
    if (b0) {
      w.qk_first<1>();
      if (kb0 + kBN > it.klen) w.mask<1>(kb0, it.klen);
      w.max_plain<1>();
    } else {
      w.qk_first<0>();
      if (kb0 + kBN > it.klen) w.mask<0>(kb0, it.klen);
      w.max_plain<0>();
    }
    w.m_raw[0] = w.mt[0];
    w.m_raw[1] = w.mt[1];

    // Tile t: at its top, tile t+1 (issued two tiles earlier) is complete in
    // this wave (at most the job of tile t+2 is in flight) and the barrier
    // publishes every wave's part. The job issued during tile t, tile t+3,
    // reuses the stage of tile t-1, whose K was read in tile t-2 and V in
    // tile t-1, before that barrier.
    auto top = [&](int t) {
      asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
      __syncthreads();
      const int tn = t + kLead;
      dma.prepare(p, tn < ntiles, (t0 + tn) * kBN, stage_addr(tn), wave, kp, vp, lane);
    };
    auto run = [&](auto sb, auto next, int t) {
      constexpr int SB = decltype(sb)::value;
      constexpr bool NEXT = decltype(next)::value;
      top(t);
      const int kbn = (t0 + t + 1) * kBN;
      w.tile<SB, NEXT, TRACK>(stage_addr(t + 1) - stage_addr(t), kbn + kBN > it.klen, kbn, it.klen,
                              dma);
      if constexpr (NEXT && TRACK) w.update_max();
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

  w.fence_o();
  if constexpr (!TRACK) {
    if (ntiles > 0) {
      // Every wave's verdict through LDS (ring stage 3; the output staging
      // uses stages 0-1).
      int* flags = reinterpret_cast<int*>(kv_lds + 3 * 2 * kTileElems);
      const bool out_of_range = !w.sums_in_range();
      if (lane == 0) flags[wave] = __builtin_amdgcn_ballot_w64(out_of_range) != 0;
      __syncthreads();
      if (__builtin_amdgcn_readfirstlane(flags[0] | flags[1] | flags[2] | flags[3])) {
        if (tid == 0) *mark = kRerunMark;
        return;
      }
    }
  }

  // Output through the ring: 16 KB per wave.
  bf16* stage = kv_lds + wave * 8192;
  if (split < 0) {
    const bool pad = p.ln_pad != nullptr;
    const float pad_ln = pad ? p.ln_pad[it.b] : 0.f;
    bf16* obase = p.o + it.b * p.os0 + it.h * p.os2;
    const float lse0 = w.finish<0>(pad_ln, pad, obase, p.os1, qrow0, p.Sq, lane, stage);
    const float lse1 = w.finish<1>(pad_ln, pad, obase, p.os1, qrow0 + 32, p.Sq, lane, stage + 4096);
    if (p.lse && w.hh == 0) {
      float* lp = p.lse + ((int64_t)it.b * p.H + it.h) * p.Sq;
      if (qrow0 + w.li < p.Sq) lp[qrow0 + w.li] = lse0;
      if (qrow0 + 32 + w.li < p.Sq) lp[qrow0 + 32 + w.li] = lse1;
    }
  } else {
    const int64_t row = part_row;
    bf16* obase = p.part_o + row * kQPerWg * kD;
    const int q0 = wave * kQPerWave;
    const float lse0 = w.finish<0>(0.f, false, obase, kD, q0, kQPerWg, lane, stage);
    const float lse1 = w.finish<1>(0.f, false, obase, kD, q0 + 32, kQPerWg, lane, stage + 4096);
    if (w.hh == 0) {
      p.part_lse[row * kQPerWg + q0 + w.li] = lse0;
      p.part_lse[row * kQPerWg + q0 + 32 + w.li] = lse1;
    }
  }
}

// One block per workgroup: TRACK false is the first-tile-max form, which
// attn_fwd_fixup_kernel must follow; TRACK true the running max (one launch).
template <bool TRACK>
__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(1, 1)))
void attn_fwd_kernel(FwdParams p) {
  __shared__ __attribute__((aligned(1024))) bf16 kv_lds[kStages * 2 * kTileElems];
  fwd_block<TRACK>(p, blockIdx.x, kv_lds);
}

// The fix-up launch: at most one workgroup per CU (one round), workgroup g
// taking blocks g, g + G, g + 2 G, ... (G = gridDim.x), 64 at a time: wave 0
// loads their mark places (one lane each) and the workgroup runs the marked
// blocks one after another. Without marks every workgroup exits after one
// load per lane; with every block marked the work is one more pass over the
// grid.
__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(1, 1)))
void attn_fwd_fixup_kernel(FwdParams p, int nblocks) {
  __shared__ __attribute__((aligned(1024))) bf16 kv_lds[kStages * 2 * kTileElems];
  __shared__ uint64_t marked;
  for (int base = blockIdx.x; base < nblocks; base += 64 * gridDim.x) {
    if (threadIdx.x < 64) {
      const int blk = base + (int)threadIdx.x * (int)gridDim.x;
      bool m = false;
      if (blk < nblocks) {
        int item_idx, split;
        block_item(p, blk, item_idx, split);
        m = *mark_ptr(p, item_idx, split) == kRerunMark;
      }
      const uint64_t bal = __builtin_amdgcn_ballot_w64(m);
      if (threadIdx.x == 0) marked = bal;
    }
    __syncthreads();
    uint64_t todo = marked;
    __syncthreads();  // every wave has read `marked` before the next chunk
    while (todo) {
      const int i = __builtin_ctzll(todo);
      todo &= todo - 1;
      fwd_block<true>(p, base + i * (int)gridDim.x, kv_lds);
      __syncthreads();  // the ring is free for the next block
    }
  }
}

// Merges the key-range partials of the split work items: 16 queries per
// workgroup, 16 lanes per query with 8 head-dim values (16 bytes) each.
// O = sum_s exp(lse_s - lse) O_s with lse = log sum_s exp(lse_s), then the
// optional padding correction, bf16 O and LSE. (With 4 values per lane the
// pass ran at ~2.6 TB/s: too few bytes in flight per lane.)
constexpr int kCombineQ = 16;  // queries per combine workgroup
__global__ __launch_bounds__(256) void attn_fwd_combine_kernel(FwdParams p) {
  const int gq = blockIdx.x * kCombineQ + (threadIdx.x >> 4);  // split-item query index
  const int j = gq / kQPerWg, qloc = gq - j * kQPerWg;
  if (j >= p.split_items) return;
  const Item it = decode_item(p, p.full_blocks + j);
  const int qrow = it.qblk * kQPerWg + qloc;
  if (qrow >= p.Sq) return;
  const int d0 = 8 * (threadIdx.x & 15);
  const int64_t row0 = (int64_t)j * p.nsplit;
  // Every load (the splits' O rows and LSEs) goes out before any is used:
  // one memory round trip instead of one per split.
  u32x4 raw[8];
#pragma unroll
  for (int s = 0; s < 8; ++s)
    if (s < p.nsplit) raw[s] = ld16(p.part_o + ((row0 + s) * kQPerWg + qloc) * kD + d0);
  float ls[8];
  float mx = -INFINITY;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    ls[s] = s < p.nsplit ? p.part_lse[(row0 + s) * kQPerWg + qloc] : -INFINITY;
    mx = fmaxf(mx, ls[s]);
  }
  float lse = -INFINITY;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (mx > -INFINITY) {
    float sum = 0.f;
#pragma unroll
    for (int s = 0; s < 8; ++s) sum += expf(ls[s] - mx);
    lse = mx + logf(sum);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      // A range with no keys left its partial unwritten: skipped, not
      // weighted by 0 (its bytes may hold NaN).
      if (s < p.nsplit && ls[s] > -INFINITY) {
        const float wgt = expf(ls[s] - lse);
        float v[8];
        unpack8(raw[s], v);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = fmaf(wgt, v[i], acc[i]);
      }
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

static bool stride_ok(const int64_t* s) {
  return (s[0] % 8) == 0 && (s[1] % 8) == 0 && (s[2] % 8) == 0;
}

}  // namespace aa

using namespace aa;

// Key split of the work items of a partial last round. With T work items
// on ncu CUs, the last T % ncu items would run alone on under half the chip;
// when that is so, each of them is split into nsplit key ranges (up to 8, at
// most one per key tile) so that they fill the CUs of that round.
struct SplitPlan {
  int full_blocks, split_items, nsplit;
};

static SplitPlan split_plan(int64_t T, int64_t Sk, int ncu) {
  SplitPlan s{(int)T, 0, 1};
  if (ncu <= 0 || T <= 0) return s;
  const int64_t rem = T % ncu;
  if (rem == 0 || 2 * rem > ncu) return s;
  const int64_t ntk = (Sk + kBN - 1) / kBN;
  const int ns = (int)std::min<int64_t>(std::min<int64_t>(8, ncu / rem), ntk);
  if (ns < 2) return s;
  s.full_blocks = (int)(T - rem);
  s.split_items = (int)rem;
  s.nsplit = ns;
  return s;
}

static size_t split_workspace_bytes(const SplitPlan& s) {
  // bf16 O rows and one fp32 LSE per query.
  return (size_t)s.split_items * s.nsplit * kQPerWg * (kD * sizeof(bf16) + sizeof(float));
}

static int64_t work_items(int64_t B, int64_t Sq, int64_t H) {
  return B * H * ((Sq + kQPerWg - 1) / kQPerWg);
}

extern "C" size_t aa_attn_fwd_workspace(int64_t B, int64_t Sq, int64_t Sk, int64_t H, int64_t hd) {
  if (hd == 384) return attn_fwd_d384_workspace(B, Sq, Sk, H, device_cu_count());
  if (B <= 0 || Sq <= 0 || Sk <= 0 || H <= 0) return 0;
  return split_workspace_bytes(split_plan(work_items(B, Sq, H), Sk, device_cu_count()));
}

// Validates args and fills the kernel parameters (no launch).
static int prepare(const aa_attn_fwd_args* a, FwdParams& p) {
  if (!a) return fail(AA_EINVAL, "attn_fwd: null args");
  if (a->dtype != AA_DTYPE_BF16) return fail(AA_EUNSUPPORTED, "only bf16 attention is implemented");
  if (a->hd != kD) return fail(AA_EUNSUPPORTED, "head_dim must be 128 or 384");
  if (a->B < 0 || a->Sq < 0 || a->Sk < 0 || a->H <= 0)
    return fail(AA_EINVAL, "attn_fwd: negative size");
  if (a->Sq > (1 << 30) || a->Sk > (1 << 30) || a->H > 65535 || a->B > 65535)
    return fail(AA_EUNSUPPORTED, "attn_fwd: size out of range");
  if (a->B == 0 || a->Sq == 0) return AA_OK;
  // K and V may be null when there are no keys (nothing reads them).
  if (!a->q || !a->out || (a->Sk > 0 && (!a->k || !a->v)))
    return fail(AA_EINVAL, "attn_fwd: null tensor");
  if (!aligned16(a->q) || !aligned16(a->k) || !aligned16(a->v) || !aligned16(a->out))
    return fail(AA_EINVAL, "attn_fwd: tensors must be 16-byte aligned");
  if (!stride_ok(a->q_stride) || !stride_ok(a->k_stride) || !stride_ok(a->v_stride) ||
      !stride_ok(a->out_stride))
    return fail(AA_EINVAL, "attn_fwd: strides must be multiples of 8 elements");
  if (a->ln_pad && !a->seqused_k) return fail(AA_EINVAL, "attn_fwd: ln_pad needs seqused_k");
  if (!(a->softmax_scale > 0.f) || !std::isfinite(a->softmax_scale))
    return fail(AA_EINVAL, "attn_fwd: softmax_scale must be positive and finite");
  // The K/V tile DMA addresses rows by a 32-bit unsigned per-lane byte
  // offset (up to 7 rows past a scalar row base): the stride must be
  // non-negative and small enough.
  if (a->k_stride[1] < 0 || a->v_stride[1] < 0 || a->k_stride[1] >= (1 << 24) ||
      a->v_stride[1] >= (1 << 24))
    return fail(AA_EUNSUPPORTED, "attn_fwd: key/value sequence stride must be in [0, 2^24) elements");

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
  const int64_t total = work_items(a->B, a->Sq, a->H);
  if (total > 0x7fffffff / 8) return fail(AA_EUNSUPPORTED, "attn_fwd: grid too large");
  p.total_blocks = (int)total;
  p.c = a->softmax_scale * kLog2e;
  const SplitPlan sp = split_plan(total, a->Sk, device_cu_count());
  const size_t ws_need = split_workspace_bytes(sp);
  if (ws_need > 0 && (!a->workspace || a->workspace_bytes < ws_need))
    return fail(AA_EINVAL, "attn_fwd: workspace too small (aa_attn_fwd_workspace)");
  if (ws_need > 0 && !aligned16(a->workspace))
    return fail(AA_EINVAL, "attn_fwd: workspace must be 16-byte aligned");
  p.full_blocks = sp.full_blocks;
  const int ncu = device_cu_count();
  p.round_blocks = ncu > 0 ? std::min(ncu, std::max(sp.full_blocks, 1)) : std::max(sp.full_blocks, 1);
  p.split_items = sp.split_items;
  p.nsplit = sp.nsplit;
  p.part_o = (bf16*)a->workspace;
  p.part_lse = (float*)(p.part_o + (size_t)sp.split_items * sp.nsplit * kQPerWg * kD);
  return AA_OK;
}

// Split partials of aa_attn_fwd_noalloc. split_plan splits at most ncu / 2
// items into at most ncu / items key ranges, so the partials never exceed
// ncu * kQPerWg records of kD bf16 + one float (17,039,360 bytes at 256 CUs); the
// head-dim-384 forward's never exceed kD384MaxPartialBytes (25,296,896). The
// array holds the larger, resident on every device the library runs on.
constexpr size_t kFwdScratchBytes =
    std::max((size_t)256 * kQPerWg * (kD * sizeof(bf16) + sizeof(float)), kD384MaxPartialBytes);
static __device__ __align__(256) uint8_t scratch[kFwdScratchBytes];

// Device address of `scratch` on the current device, looked up once per
// device. In host code `scratch` names a host-side stand-in, so only this
// address may be passed to kernels.
static int fwd_scratch(void** out) {
  constexpr int kMaxDevices = 64;
  static std::atomic<void*> addr[kMaxDevices];
  static std::mutex lock;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(AA_EHIP, "attn_fwd_noalloc: no current device");
  void* p = addr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> g(lock);
    p = addr[dev].load(std::memory_order_relaxed);
    if (!p) {
      const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p)
        return fail(AA_EHIP, std::string("attn_fwd_noalloc: hipGetSymbolAddress: ") +
                                 hipGetErrorString(e));
      addr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return AA_OK;
}

// Which head_dim-128 kernel runs: the two-group kernel of attn_fwd_pp.hip (0)
// up to kPingPongMaxSk keys, where a work item's fixed costs weigh most, and
// this file's one-wave-per-SIMD kernel (1) beyond. Measured on MI355X at
// B = 1-2, 4096 queries: the two-group kernel is 5-8% faster at 512 and 1024
// keys, the two tie at 2048, the one-wave kernel is ~3% faster at 4096.
// AA_FWD_KERNEL=pp|1w forces one (tests run both on every shape); -1 for
// another value.
constexpr int64_t kPingPongMaxSk = 2048;
static int fwd_kernel_choice(int64_t Sk) {
  const char* e = std::getenv("AA_FWD_KERNEL");
  if (e && *e) {
    const std::string v = e;
    if (v == "pp") return 0;
    if (v == "1w") return 1;
    return -1;
  }
  return Sk <= kPingPongMaxSk ? 0 : 1;
}

// Which form of the one-wave kernel runs: the first-tile max (true) saves
// ~3% of the tile loop but needs the fix-up launch after it, which costs
// ~4.7 us even when it finds nothing to do (MI355X, kernel trace), so it pays
// from about one round of 64-tile work items on: more rounds of blocks than
// CUs, or longer key ranges. Measured (median, one process): B=1 4096 tokens
// (one round of 64 tiles) at par; B=2 233.8 -> 229.0 us, B=16 1883 -> 1826
// us, 9216 tokens 617 -> 580 us. AA_FWD_FIRST_TILE_MAX=0|1 forces one.
static bool fwd_first_tile_max(const FwdParams& p, int blocks) {
  const char* e = std::getenv("AA_FWD_FIRST_TILE_MAX");
  if (e && *e) return e[0] != '0';
  const int ncu = std::max(device_cu_count(), 1);
  const int64_t rounds = (blocks + ncu - 1) / ncu;
  const int64_t tiles = ((int64_t)p.Sk + kBN - 1) / kBN;
  return rounds * tiles > 64;
}

extern "C" int aa_attn_fwd(const aa_attn_fwd_args* a, void* stream);

extern "C" int aa_attn_fwd_noalloc(const aa_attn_fwd_args* a, void* stream) {
  clear_error();
  if (!a) return fail(AA_EINVAL, "attn_fwd_noalloc: null args");
  aa_attn_fwd_args b = *a;
  b.workspace = nullptr;
  b.workspace_bytes = 0;
  if (a->B > 0 && a->Sq > 0 && a->Sk > 0 && a->H > 0) {
    const size_t need = aa_attn_fwd_workspace(a->B, a->Sq, a->Sk, a->H, a->hd);
    if (need > kFwdScratchBytes)
      return fail(AA_EUNSUPPORTED, "attn_fwd_noalloc: split partials of " + std::to_string(need) +
                                       " bytes exceed the fixed scratch of " +
                                       std::to_string(kFwdScratchBytes) + " bytes");
    if (need > 0) {
      if (int rc = fwd_scratch(&b.workspace)) return rc;
      b.workspace_bytes = kFwdScratchBytes;
    }
  }
  return aa_attn_fwd(&b, stream);
}

extern "C" int aa_attn_fwd(const aa_attn_fwd_args* a, void* stream) {
  clear_error();
  if (a && a->hd == 384) {
    if (a->dtype != AA_DTYPE_BF16) return fail(AA_EUNSUPPORTED, "only bf16 attention is implemented");
    return attn_fwd_d384(a, device_cu_count(), (hipStream_t)stream);
  }
  FwdParams p;
  if (int rc = prepare(a, p)) return rc;
  if (a->B == 0 || a->Sq == 0) return AA_OK;
  hipStream_t st = (hipStream_t)stream;
  const int blocks = p.full_blocks + p.split_items * p.nsplit;
  const int which = fwd_kernel_choice(p.Sk);
  if (which < 0) return fail(AA_EINVAL, "AA_FWD_KERNEL must be pp or 1w");
  if (which == 0) launch_attn_fwd_pp(p, (unsigned)blocks, st);
  else if (fwd_first_tile_max(p, blocks)) {
    attn_fwd_kernel<false><<<dim3((unsigned)blocks), kWaves * 64, 0, st>>>(p);
    if (int rc = check_launch("attn_fwd")) return rc;
    // Re-runs the blocks whose rows left the first tile's exponent range.
    const int fix_groups = std::min(blocks, std::max(device_cu_count(), 1));
    attn_fwd_fixup_kernel<<<dim3((unsigned)fix_groups), kWaves * 64, 0, st>>>(p, blocks);
  } else {
    attn_fwd_kernel<true><<<dim3((unsigned)blocks), kWaves * 64, 0, st>>>(p);
  }
  if (int rc = check_launch("attn_fwd")) return rc;
  if (p.split_items > 0) {
    const int groups = (p.split_items * kQPerWg + kCombineQ - 1) / kCombineQ;
    attn_fwd_combine_kernel<<<dim3((unsigned)groups), 256, 0, st>>>(p);
    return check_launch("attn_fwd combine");
  }
  return AA_OK;
}
