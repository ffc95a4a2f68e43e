// Flash-attention forward, non-causal, head_dim 128, bf16 in / fp32 accumulate,
// for gfx950 (CDNA4): v_mfma_f32_32x32x16_bf16 for both products.
//
// Work decomposition
//   One workgroup = NW waves = NW*32 queries of one (batch, head). Each wave
//   owns 32 queries for the whole kernel; K/V tiles of 64 keys are streamed
//   through LDS (double-buffered) and shared by the NW waves.
//
// Transposed formulation (per wave, per 64-key tile)
//   S^T = K Q^T   : A = K rows from LDS (32 keys x 16 d per MFMA),
//                   B = Q^T from registers (loaded once).
//   O^T += V^T P^T: A = V^T rows from LDS (32 d x 16 keys),
//                   B = P^T straight from the S^T accumulators.
//   The 32x32 accumulator layout puts column j = lane%32 in every lane, with
//   rows 8*(r/4) + 4*(lane/32) + r%4 in register r. With queries as columns,
//   every lane holds one query: the softmax row max/sum are in-lane
//   reductions plus one v_permlane32_swap with the partner lane, and the
//   output rescale is a per-lane scalar multiply.
//
// Key permutation for P^T
//   The B operand of the MFMA wants, in lane l, 8 consecutive k-indices
//   8*(l/32)+i of a 16-key chunk. The S^T accumulators hold, for that lane,
//   keys {4h..4h+3, 8+4h..8+4h+3} (h = l/32) of the chunk. Since PV sums over
//   keys, the chunk is processed in the permuted order
//   position 8h + 4g + i  <->  key 8g + 4h + i,
//   and V^T is written to LDS in that same order. Groups of 4 keys stay
//   contiguous, so each thread transposes a 4-key x 8-d block in registers
//   and writes eight 8-byte rows of V^T.
//
// Online softmax with lazy rescaling
//   Scores are kept in log2 units (t = s * scale * log2 e). The running max
//   m is only raised when a tile's max exceeds it by more than 8, so
//   p = exp2(t - m) <= 256 and the O/l rescale (a full pass over the 64
//   accumulator registers) runs only a handful of times per row.
#include "aa_common.h"

namespace aa {

constexpr int kD = 128;
constexpr int kBN = 64;                  // keys per tile
constexpr int kKStride = kD + 8;         // K tile row stride (elements), 272 B
constexpr int kVStride = kBN + 8;        // V^T tile row stride (elements), 144 B
constexpr int kKTile = kBN * kKStride;   // elements
constexpr int kVTile = kD * kVStride;    // elements
constexpr int kStage = kKTile + kVTile;  // one K + V^T buffer
constexpr float kRescaleThreshold = 8.0f;

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

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

template <int NW>
__global__ __launch_bounds__(NW * 64) void attn_fwd_kernel(FwdParams p) {
  static_assert(NW == 4, "the V^T staging assigns one 4-key x 8-d block per thread");
  constexpr int NT = NW * 64;
  constexpr int kKChunks = kBN * kD / 8 / NT;  // 16-byte K chunks per thread per tile
  __shared__ __attribute__((aligned(16))) bf16 smem[2 * kStage];

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
  const int wave = tid >> 6;
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

  // Tile staging registers.
  u32x4 kr[kKChunks];
  u32x4 vr[4];
  const int vq = tid & 15;  // 4-key group of the tile this thread transposes
  const int vd = tid >> 4;  // 8-wide d chunk
  // Position of key group vq in the permuted key order (see header).
  const int vpos = 16 * (vq >> 2) + 8 * (vq & 1) + 4 * ((vq >> 1) & 1);

  auto load_tile = [&](int t) {
    const int kb = t * kBN;
#pragma unroll
    for (int i = 0; i < kKChunks; ++i) {
      const int id = tid + NT * i;
      const int key = id >> 4, dc = id & 15;
      u32x4 w = {0u, 0u, 0u, 0u};
      if (kb + key < klen) w = ld16(kp + (int64_t)(kb + key) * p.ks1 + 8 * dc);
      kr[i] = w;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = 4 * vq + i;
      u32x4 w = {0u, 0u, 0u, 0u};
      if (kb + key < klen) w = ld16(vp + (int64_t)(kb + key) * p.vs1 + 8 * vd);
      vr[i] = w;
    }
  };

  auto store_tile = [&](bf16* stage) {
    bf16* ks = stage;
    bf16* vt = stage + kKTile;
#pragma unroll
    for (int i = 0; i < kKChunks; ++i) {
      const int id = tid + NT * i;
      const int key = id >> 4, dc = id & 15;
      st16(ks + key * kKStride + 8 * dc, kr[i]);
    }
    // Transpose the 4 keys x 8 d block: row d of V^T gets the 4 keys' values.
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const uint32_t a0 = vr[0][m], a1 = vr[1][m], a2 = vr[2][m], a3 = vr[3][m];
      u32x2 lo = {(a0 & 0xffffu) | (a1 << 16), (a2 & 0xffffu) | (a3 << 16)};
      u32x2 hi = {(a0 >> 16) | (a1 & 0xffff0000u), (a2 >> 16) | (a3 & 0xffff0000u)};
      *reinterpret_cast<u32x2*>(vt + (8 * vd + 2 * m) * kVStride + vpos) = lo;
      *reinterpret_cast<u32x2*>(vt + (8 * vd + 2 * m + 1) * kVStride + vpos) = hi;
    }
  };

  f32x16 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[dt][r] = 0.f;
  float m_run = -INFINITY;
  float l_run = 0.f;

  if (ntiles > 0) {
    load_tile(0);
    store_tile(smem);
  }
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const bf16* ks = smem + (t & 1) * kStage;
    const bf16* vt = ks + kKTile;
    if (t + 1 < ntiles) load_tile(t + 1);

    // S^T = K Q^T for two 32-key halves of the tile.
    f32x16 s[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kt][r] = 0.f;
      const bf16* arow = ks + (32 * kt + li) * kKStride + 8 * hh;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(arow + 16 * kk);
        s[kt] = mfma32(a, qreg[kk], s[kt]);
      }
    }

    // Scale to log2 units, mask keys past klen, row max.
    const int kb = t * kBN;
    const bool partial = kb + kBN > klen;
    float mt = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float x = s[kt][r] * p.c;
        if (partial) {
          const int key = kb + 32 * kt + 8 * (r >> 2) + 4 * hh + (r & 3);
          if (key >= klen) x = -INFINITY;
        }
        s[kt][r] = x;
        mt = fmaxf(mt, x);
      }
    }
    mt = pair_max(mt);

    const bool need = mt > m_run + kRescaleThreshold;
    if (__builtin_amdgcn_ballot_w64(need)) {
      const float mn = need ? mt : m_run;
      const float alpha = fast_exp2(m_run - mn);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
      l_run *= alpha;
      m_run = mn;
    }

    // P^T in bf16 as four 16-key B operands; row sum in fp32.
    bf16x8 pb[4];
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float pv = fast_exp2(s[c4 >> 1][(c4 & 1) * 8 + i] - m_run);
        l_run += pv;
        pb[c4][i] = (bf16)pv;
      }
    }

    // O^T += V^T P^T.
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const bf16* arow = vt + (32 * dt + li) * kVStride + 8 * hh;
#pragma unroll
      for (int c4 = 0; c4 < 4; ++c4) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(arow + 16 * c4);
        o[dt] = mfma32(a, pb[c4], o[dt]);
      }
    }

    if (t + 1 < ntiles) store_tile(smem + ((t + 1) & 1) * kStage);
    __syncthreads();
  }

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
