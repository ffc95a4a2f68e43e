// Flash-attention forward, non-causal, head_dim 128, bf16 in / fp32 accumulate,
// for gfx950 (CDNA4): v_mfma_f32_32x32x16_bf16 for both products.
//
// Work decomposition
//   One workgroup = NW waves = NW*32 queries of one (batch, head). Each wave
//   owns 32 queries for the whole kernel; K/V tiles of 64 keys are streamed
//   into LDS and shared by the NW waves. Two LDS stages: the DMA of tile t+1
//   runs while tile t is consumed.
//
// Transposed formulation (per wave, per 64-key tile)
//   S^T = K Q^T   : A = K rows from LDS (32 keys x 16 d per MFMA),
//                   B = Q^T from registers (loaded once).
//   O^T += V^T P^T: A = V^T (32 d x 16 keys) read from the row-major V tile
//                   with ds_read_b64_tr_b16, B = P^T from the S^T accumulators.
//   The 32x32 accumulator layout puts column j = lane%32 in every lane, with
//   rows 8*(r/4) + 4*(lane/32) + r%4 in register r. With queries as columns,
//   every lane holds one query: the softmax row max/sum are in-lane
//   reductions plus one v_permlane32_swap with the partner lane, and the
//   output rescale is a per-lane scalar multiply.
//
// K/V staging: global_load_lds_dwordx4 (DMA, no registers). A DMA instruction
//   writes 64 lanes x 16 B contiguously, i.e. 4 rows of 256 B, so rows are not
//   padded; bank conflicts (64 banks of 4 B) are avoided by XOR-swizzling the
//   16-byte chunks of each row instead: chunk c of row r is stored at
//   c ^ (r & 15) for K (the MFMA A reads hit 16 different rows per 16 lanes)
//   and at c ^ 4*(r & 3) for V (a transposed read covers 4 rows x 64 B per
//   32 lanes). The lane picks which global chunk it fetches so that the LDS
//   side stays contiguous.
//
// Transposed read (ds_read_b64_tr_b16): within each group of 16 lanes, lane i
//   receives element (i & 3) of the 4 b16 values addressed by lanes
//   4j + (i >> 2), j = 0..3. With source lane s pointing at
//   V[k0 + (s >> 2)][d0 + 4 (s & 3)], lane i gets V[k0 + j][d0 + i], j = 0..3:
//   4 keys of one d column, i.e. a row of V^T.
//
// Key permutation for P^T
//   The B operand of the MFMA wants, in lane l, 8 consecutive k-indices
//   8*(l/32)+i of a 16-key chunk. The S^T accumulators hold, for that lane,
//   keys {4h..4h+3, 8+4h..8+4h+3} (h = l/32) of the chunk. Since PV sums over
//   keys, the A operand is read in the same order: its elements 0-3 are keys
//   4h..4h+3 and 4-7 are keys 8+4h..8+4h+3 (two transposed reads).
//
// Online softmax with lazy rescaling
//   The running max m is tracked on raw scores s = q.k; probabilities are
//   p = exp2(s*c - m*c) with c = scale * log2(e), one FMA and one v_exp_f32
//   per score. m is only raised when a tile's max exceeds it by more than
//   8/c (8 in log2 units), so p <= 256 and the O/l rescale (a pass over the
//   64 accumulator registers) runs only a few times per row. The row sum is
//   taken over the bf16-rounded P that feeds the MFMA, with v_dot2c_f32_bf16.
#include <cmath>
#include <type_traits>

#include "aa_common.h"

namespace aa {

constexpr int kD = 128;
constexpr int kBN = 64;                     // keys per tile
constexpr int kTileElems = kBN * kD;        // one K or V tile (16 KB)
constexpr float kRescaleThreshold = 8.0f;   // log2 units

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
};

typedef __attribute__((address_space(3))) void lds_void;
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// Address-space casts keep the pointer's provenance (the __shared__ array it
// points into), so the compiler can tell a DMA into one stage from reads of
// the other and does not insert waits for the in-flight DMA before them.
__device__ __forceinline__ lds_void* to_lds(const void* p) { return (lds_void*)p; }

// Transposed LDS read: 4 bf16 per lane (lane mapping in the header).
__device__ __forceinline__ s16x4 lds_read_tr(const bf16* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p);
}

__device__ __forceinline__ void wait_dma() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

template <int NW>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_fwd_kernel(FwdParams p) {
  static_assert(NW == 4 || NW == 8, "4 or 8 waves per workgroup");
  constexpr int kDmaPerWave = 16 / NW;  // 1 KB DMA instructions per wave per tile (K and V each)
  __shared__ __attribute__((aligned(1024))) bf16 k_lds0[kTileElems];
  __shared__ __attribute__((aligned(1024))) bf16 k_lds1[kTileElems];
  __shared__ __attribute__((aligned(1024))) bf16 v_lds0[kTileElems];
  __shared__ __attribute__((aligned(1024))) bf16 v_lds1[kTileElems];

  // Block -> (batch, head, query block). Workgroups are dispatched round-robin
  // over the 8 XCDs; remap so each XCD gets a contiguous range of logical
  // blocks, i.e. the same few heads, whose K/V then stay in that XCD's L2.
  int logical = blockIdx.x;
  if ((p.total_blocks & 7) == 0) {
    logical = (blockIdx.x & 7) * (p.total_blocks >> 3) + (blockIdx.x >> 3);
  }
  const int qblk = logical % p.nqblk;
  const int bh = logical / p.nqblk;
  const int b = bh / p.H;
  const int h = bh - b * p.H;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int li = lane & 31;
  const int hh = lane >> 5;

  const int klen = p.seqused ? min((int)p.seqused[b], p.Sk) : p.Sk;
  const int ntiles = klen > 0 ? (klen + kBN - 1) / kBN : 0;

  // Q^T operand: lane holds Q[query li][16*kk + 8*hh + 0..7] for kk = 0..7.
  const int qrow = qblk * (NW * 32) + wave * 32 + li;
  bf16x8 qreg[8];
  {
    const bf16* qp = p.q + b * p.qs0 + h * p.qs2 + (int64_t)qrow * p.qs1 + 8 * hh;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      u32x4 w = {0u, 0u, 0u, 0u};
      if (qrow < p.Sq) w = ld16(qp + 16 * kk);
      qreg[kk] = as_bf16x8(w);
    }
  }

  const bf16* kp = p.k + b * p.ks0 + h * p.ks2;
  const bf16* vp = p.v + b * p.vs0 + h * p.vs2;

  // DMA of tile t into (kd, vd): this wave fills 1 KB blocks wave*kDmaPerWave + i
  // (rows 4*blk .. 4*blk+3). Rows past klen re-read row klen-1 (finite data;
  // their scores are masked).
  auto issue_tile = [&](int t, bf16* kd, bf16* vd) {
    const int kb = t * kBN;
    const int slot = lane & 15;
#pragma unroll
    for (int i = 0; i < kDmaPerWave; ++i) {
      const int blk = wave * kDmaPerWave + i;
      const int row = 4 * blk + (lane >> 4);
      const int src = min(kb + row, klen - 1);
      const bf16* gk = kp + (int64_t)src * p.ks1 + 8 * (slot ^ (row & 15));
      const bf16* gv = vp + (int64_t)src * p.vs1 + 8 * (slot ^ (4 * (row & 3)));
      __builtin_amdgcn_global_load_lds(gk, to_lds(kd + blk * 512), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(gv, to_lds(vd + blk * 512), 16, 0, 0);
    }
  };

  // Per-lane LDS read offsets (elements). K operand (kt, kk): row 32kt + li,
  // logical chunk 2kk + hh stored at (2kk + hh) ^ (li & 15).
  int k_off[8];
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) k_off[kk] = li * kD + 8 * ((2 * kk + hh) ^ (li & 15));
  // V^T operand (dt, c4, half): source lane s = lane & 15 of group g = lane >> 4
  // reads 4 d at row 16*c4 + 4*(g>>1) + 8*half + (s>>2), d = 32dt + 16(g&1) + 4(s&3).
  const int g = lane >> 4, s = lane & 15;
  const int vrow = 4 * (g >> 1) + (s >> 2);
  int v_off[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    const int dcol = 32 * dt + 16 * (g & 1) + 4 * (s & 3);
    const int chunk = (dcol >> 3) ^ (4 * (vrow & 3));
    v_off[dt] = vrow * kD + 8 * chunk + (dcol & 7);
  }

  f32x16 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[dt][r] = 0.f;
  // Running max in raw score units (before the scale); l partial sums in
  // four independent chains.
  float m_raw = -INFINITY;
  float l4[4] = {0.f, 0.f, 0.f, 0.f};
  const float c = p.c;
  const float thr_raw = kRescaleThreshold / c;
  const bf16x2 ones = {(bf16)1.0f, (bf16)1.0f};

  // One 64-key tile: S^T, softmax, O^T += V^T P^T. MASK excludes keys >= klen
  // (only the last tile of a row can need it).
  auto process = [&](const bf16* ks, const bf16* vs, int kb, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    // S^T = K Q^T: two independent 32-key accumulator chains.
    f32x16 s0, s1;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s0[r] = 0.f;
      s1[r] = 0.f;
    }
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      const bf16x8 x0 = *reinterpret_cast<const bf16x8*>(ks + k_off[kk]);
      const bf16x8 x1 = *reinterpret_cast<const bf16x8*>(ks + 32 * kD + k_off[kk]);
      s0 = mfma32(x0, qreg[kk], s0);
      s1 = mfma32(x1, qreg[kk], s1);
    }
    if constexpr (MASK) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kb + 8 * (r >> 2) + 4 * hh + (r & 3);
        if (key >= klen) s0[r] = -INFINITY;
        if (key + 32 >= klen) s1[r] = -INFINITY;
      }
    }
    // Row max of the raw scores, then over the lane pair.
    float mt = fmaxf(s0[0], s1[0]);
#pragma unroll
    for (int r = 1; r < 16; ++r) mt = fmaxf(mt, fmaxf(s0[r], s1[r]));
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
    bf16x8 pb[4];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      pb[0][i] = (bf16)fast_exp2(fmaf(s0[i], c, -mc));
      pb[1][i] = (bf16)fast_exp2(fmaf(s0[8 + i], c, -mc));
      pb[2][i] = (bf16)fast_exp2(fmaf(s1[i], c, -mc));
      pb[3][i] = (bf16)fast_exp2(fmaf(s1[8 + i], c, -mc));
    }
    // Row sum of the bf16 P that feeds the MFMA (v_dot2 with ones).
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bf16x2 pair = {pb[c4][2 * j], pb[c4][2 * j + 1]};
        l4[c4] = __builtin_amdgcn_fdot2_f32_bf16(pair, ones, l4[c4], false);
      }
    }

    // O^T += V^T P^T: A operand from two transposed reads (keys 4h.. and 8+4h..).
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const bf16* base = vs + 16 * c4 * kD + v_off[dt];
        const s16x4 lo = lds_read_tr(base);
        const s16x4 hi = lds_read_tr(base + 8 * kD);
        const s16x8 both = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        o[dt] = mfma32(__builtin_bit_cast(bf16x8, both), pb[c4], o[dt]);
      }
    }
  };

  // Main loop over full tiles, unrolled by two so that each half reads one
  // statically known LDS stage while the DMA fills the other.
  const int nfull = klen / kBN;  // tiles whose 64 keys are all valid
  if (ntiles > 0) {
    issue_tile(0, k_lds0, v_lds0);
    wait_dma();
  }
  __syncthreads();
  int t = 0;
  for (; t + 1 < nfull; t += 2) {
    issue_tile(t + 1, k_lds1, v_lds1);
    process(k_lds0, v_lds0, t * kBN, std::false_type{});
    wait_dma();
    __syncthreads();
    if (t + 2 < ntiles) issue_tile(t + 2, k_lds0, v_lds0);
    process(k_lds1, v_lds1, (t + 1) * kBN, std::false_type{});
    wait_dma();
    __syncthreads();
  }
  // At most two tiles remain: one full tile (odd nfull) and/or the partial
  // tail; tile t sits in stage t & 1.
  for (; t < ntiles; ++t) {
    bf16* kc = (t & 1) ? k_lds1 : k_lds0;
    bf16* vc = (t & 1) ? v_lds1 : v_lds0;
    if (t + 1 < ntiles) issue_tile(t + 1, (t & 1) ? k_lds0 : k_lds1, (t & 1) ? v_lds0 : v_lds1);
    if (t < nfull) {
      process(kc, vc, t * kBN, std::false_type{});
    } else {
      process(kc, vc, t * kBN, std::true_type{});
    }
    wait_dma();
    __syncthreads();
  }

  const float m_run = m_raw * c;
  const float l_run = (l4[0] + l4[1]) + (l4[2] + l4[3]);

  // Epilogue: normalise, optional padding correction, store O and LSE.
  const float l_tot = pair_sum(l_run);
  const bool any = l_tot > 0.f;
  const float lse = any ? (m_run + __log2f(l_tot)) * kLn2 : -INFINITY;
  float scale = any ? 1.0f / l_tot : 0.f;
  if (p.ln_pad) scale *= 1.0f / (1.0f + expf(p.ln_pad[b] - lse));
  if (qrow < p.Sq) {
    bf16* op = p.o + b * p.os0 + (int64_t)qrow * p.os1 + h * p.os2 + 4 * hh;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        u32x2 w = {pack_bf16(o[dt][4 * rq] * scale, o[dt][4 * rq + 1] * scale),
                   pack_bf16(o[dt][4 * rq + 2] * scale, o[dt][4 * rq + 3] * scale)};
        *reinterpret_cast<u32x2*>(op + 32 * dt + 8 * rq) = w;
      }
    }
    if (p.lse && hh == 0) p.lse[((int64_t)b * p.H + h) * p.Sq + qrow] = lse;
  }
}

static bool stride_ok(const int64_t* s) {
  return (s[0] % 8) == 0 && (s[1] % 8) == 0 && (s[2] % 8) == 0;
}

}  // namespace aa

using namespace aa;

extern "C" int aa_attn_fwd(const aa_attn_fwd_args* a, void* stream) {
  clear_error();
  if (!a) return fail(AA_EINVAL, "attn_fwd: null args");
  if (a->dtype != AA_DTYPE_BF16) return fail(AA_EUNSUPPORTED, "only bf16 attention is implemented");
  if (a->hd != kD) return fail(AA_EUNSUPPORTED, "head_dim must be 128");
  if (a->B < 0 || a->Sq < 0 || a->Sk < 0 || a->H <= 0)
    return fail(AA_EINVAL, "attn_fwd: negative size");
  if (a->Sq > (1 << 30) || a->Sk > (1 << 30) || a->H > 65535 || a->B > 65535)
    return fail(AA_EUNSUPPORTED, "attn_fwd: size out of range");
  if (a->B == 0 || a->Sq == 0) return AA_OK;
  if (!a->q || !a->k || !a->v || !a->out) return fail(AA_EINVAL, "attn_fwd: null tensor");
  if (!aligned16(a->q) || !aligned16(a->k) || !aligned16(a->v) || !aligned16(a->out))
    return fail(AA_EINVAL, "attn_fwd: tensors must be 16-byte aligned");
  if (!stride_ok(a->q_stride) || !stride_ok(a->k_stride) || !stride_ok(a->v_stride) ||
      !stride_ok(a->out_stride))
    return fail(AA_EINVAL, "attn_fwd: strides must be multiples of 8 elements");
  if (a->ln_pad && !a->seqused_k) return fail(AA_EINVAL, "attn_fwd: ln_pad needs seqused_k");
  if (!(a->softmax_scale > 0.f) || !std::isfinite(a->softmax_scale))
    return fail(AA_EINVAL, "attn_fwd: softmax_scale must be positive and finite");

  constexpr int NW = 4;
  FwdParams p;
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
  p.nqblk = (int)((a->Sq + NW * 32 - 1) / (NW * 32));
  const int64_t total = a->B * a->H * p.nqblk;
  if (total > 0x7fffffff) return fail(AA_EUNSUPPORTED, "attn_fwd: grid too large");
  p.total_blocks = (int)total;
  p.c = a->softmax_scale * kLog2e;
  attn_fwd_kernel<NW><<<dim3((unsigned)total), NW * 64, 0, (hipStream_t)stream>>>(p);
  return check_launch("attn_fwd");
}
