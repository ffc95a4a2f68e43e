// Flash-attention backward, non-causal, head_dim 128, bf16 in / fp32 accumulate,
// for gfx950 (v_mfma_f32_32x32x16_bf16). Deterministic: three kernels, no
// atomics, every reduction in a fixed order.
//
//   z = scale * q k^T, P = softmax(z) (recomputed from the forward LSE),
//   dV = P^T dO, dP = dO V^T, dZ = P o (dP - D) with D = rowsum(dO o O),
//   dK = scale * dZ^T Q, dQ = scale * dZ K.
//
// 1. rowdot_kernel: D[b,h,q] = sum_d dO*O in fp32.
// 2. dkdv_kernel: one workgroup per 128 keys (4 waves x 32 keys); loops over
//    64-query tiles staged in LDS (row-major and transposed copies of Q and
//    dO). Per wave and tile, with keys as accumulator columns (lane%32):
//      S  = Q K^T      (A = Q rows from LDS,  B = K^T from registers)
//      dP = dO V^T     (A = dO rows from LDS, B = V^T from registers)
//      dV^T += dO^T P  (A = dO^T from LDS,    B = P from the S accumulators)
//      dK^T += Q^T dZ  (A = Q^T from LDS,     B = dZ from the accumulators)
// 3. dq_kernel: one workgroup per 128 queries (4 waves x 32 queries); loops
//    over 64-key tiles (K row-major and transposed, V row-major). With
//    queries as columns:
//      S^T = K Q^T, dP^T = V dO^T, dQ^T += K^T dZ^T.
// Transposed LDS copies use the same permuted row order inside each group of
// 16 rows as the forward kernel's V^T (position 8h+4g+i <-> row 8g+4h+i), so
// the accumulator registers feed the next MFMA as B operands unchanged.
#include "aa_common.h"

namespace aa {

namespace bwd {

constexpr int kD = 128;
constexpr int kT = 64;               // rows (queries or keys) per streamed tile
constexpr int kRStride = kD + 8;     // row-major tile stride (elements)
constexpr int kTStride = kT + 8;     // transposed tile stride (elements)
constexpr int kRTile = kT * kRStride;
constexpr int kTTile = kD * kTStride;

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// Thread unit of a 64 x 128 tile: rows 4*g4 .. 4*g4+3, d columns 8*dc .. 8*dc+7
// (g4 = tid & 15, dc = tid >> 4; 256 threads cover the tile).
struct Unit {
  u32x4 r[4];
};

__device__ __forceinline__ void load_unit(Unit& u, const bf16* base, int64_t rstride, int row0,
                                          int nvalid, int g4, int dc) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = row0 + 4 * g4 + i;
    u32x4 w = {0u, 0u, 0u, 0u};
    if (row < nvalid) w = ld16(base + (int64_t)row * rstride + 8 * dc);
    u.r[i] = w;
  }
}

__device__ __forceinline__ void store_rows(const Unit& u, bf16* tile, int g4, int dc) {
#pragma unroll
  for (int i = 0; i < 4; ++i) st16(tile + (4 * g4 + i) * kRStride + 8 * dc, u.r[i]);
}

__device__ __forceinline__ int perm_pos(int g4) {
  return 16 * (g4 >> 2) + 8 * (g4 & 1) + 4 * ((g4 >> 1) & 1);
}

__device__ __forceinline__ void store_transposed(const Unit& u, bf16* tile, int g4, int dc) {
  const int pos = perm_pos(g4);
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const uint32_t a0 = u.r[0][m], a1 = u.r[1][m], a2 = u.r[2][m], a3 = u.r[3][m];
    u32x2 lo = {(a0 & 0xffffu) | (a1 << 16), (a2 & 0xffffu) | (a3 << 16)};
    u32x2 hi = {(a0 >> 16) | (a1 & 0xffff0000u), (a2 >> 16) | (a3 & 0xffff0000u)};
    *reinterpret_cast<u32x2*>(tile + (8 * dc + 2 * m) * kTStride + pos) = lo;
    *reinterpret_cast<u32x2*>(tile + (8 * dc + 2 * m + 1) * kTStride + pos) = hi;
  }
}

// Row index held by accumulator register r of a 32x32 MFMA tile, lane half hh.
__device__ __forceinline__ int acc_row(int r, int hh) { return 8 * (r >> 2) + 4 * hh + (r & 3); }

struct Params {
  const bf16* dout;
  const bf16* q;
  const bf16* k;
  const bf16* v;
  const bf16* o;
  const float* lse;
  float* delta;  // [B, H, Sq]
  bf16* dq;
  bf16* dk;
  bf16* dv;
  int64_t s_do[3], s_q[3], s_k[3], s_v[3], s_o[3], s_dq[3], s_dk[3], s_dv[3];
  int H, Sq, Sk;
  float c;      // scale * log2(e)
  float scale;  // softmax scale
};

// D = rowsum(dO * O): 16 lanes per (b, q, h) row of 128.
__global__ __launch_bounds__(256) void rowdot_kernel(Params p, int64_t nrow) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row = gid >> 4;
  if (row >= nrow) return;
  const int lane = (int)(gid & 15);
  // row = ((b * Sq) + q) * H + h
  const int h = (int)(row % p.H);
  const int64_t bq = row / p.H;
  const int q = (int)(bq % p.Sq);
  const int b = (int)(bq / p.Sq);
  float x[8], y[8];
  unpack8(ld16(p.dout + b * p.s_do[0] + (int64_t)q * p.s_do[1] + h * p.s_do[2] + 8 * lane), x);
  unpack8(ld16(p.o + b * p.s_o[0] + (int64_t)q * p.s_o[1] + h * p.s_o[2] + 8 * lane), y);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) s += x[i] * y[i];
  s = group_sum<16>(s);
  if (lane == 0) p.delta[((int64_t)b * p.H + h) * p.Sq + q] = s;
}

// ------------------------------------------------------------------ dK, dV --

constexpr int kKeysPerWg = 128;  // 4 waves x 32 keys

__global__ __launch_bounds__(256) void dkdv_kernel(Params p, int nkblk) {
  // Two stages x {Q rows, Q^T, dO rows, dO^T} + per-query lse2 and D.
  constexpr int kStage = 2 * kRTile + 2 * kTTile;
  __shared__ __attribute__((aligned(16))) bf16 smem[2 * kStage];
  __shared__ __attribute__((aligned(16))) float rowstat[2][2][kT];  // [stage][lse2 | D][query]

  const int kblk = blockIdx.x % nkblk;
  const int bh = blockIdx.x / nkblk;
  const int b = bh / p.H, h = bh - (bh / p.H) * p.H;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int li = lane & 31, hh = lane >> 5;
  const int g4 = tid & 15, dc = tid >> 4;

  const int key = kblk * kKeysPerWg + wave * 32 + li;
  const bool key_ok = key < p.Sk;
  bf16x8 kreg[8], vreg[8];
  {
    const bf16* kp = p.k + b * p.s_k[0] + h * p.s_k[2] + (int64_t)key * p.s_k[1] + 8 * hh;
    const bf16* vp = p.v + b * p.s_v[0] + h * p.s_v[2] + (int64_t)key * p.s_v[1] + 8 * hh;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      u32x4 a = {0u, 0u, 0u, 0u}, c = {0u, 0u, 0u, 0u};
      if (key_ok) {
        a = ld16(kp + 16 * kk);
        c = ld16(vp + 16 * kk);
      }
      kreg[kk] = as_bf16x8(a);
      vreg[kk] = as_bf16x8(c);
    }
  }

  const bf16* qbase = p.q + b * p.s_q[0] + h * p.s_q[2];
  const bf16* dobase = p.dout + b * p.s_do[0] + h * p.s_do[2];
  const float* lse = p.lse + ((int64_t)b * p.H + h) * p.Sq;
  const float* delta = p.delta + ((int64_t)b * p.H + h) * p.Sq;
  const int ntiles = (p.Sq + kT - 1) / kT;

  Unit uq, udo;
  float stat = 0.f;
  auto load_tile = [&](int t) {
    load_unit(uq, qbase, p.s_q[1], t * kT, p.Sq, g4, dc);
    load_unit(udo, dobase, p.s_do[1], t * kT, p.Sq, g4, dc);
    if (tid < 2 * kT) {
      const int qq = t * kT + (tid & (kT - 1));
      if (tid < kT) stat = qq < p.Sq ? lse[qq] * kLog2e : INFINITY;
      else stat = qq < p.Sq ? delta[qq] : 0.f;
    }
  };
  auto store_tile = [&](int st) {
    bf16* base = smem + st * kStage;
    store_rows(uq, base, g4, dc);
    store_transposed(uq, base + kRTile, g4, dc);
    store_rows(udo, base + kRTile + kTTile, g4, dc);
    store_transposed(udo, base + 2 * kRTile + kTTile, g4, dc);
    if (tid < 2 * kT) rowstat[st][tid >> 6][tid & (kT - 1)] = stat;
  };

  f32x16 dk[4], dv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      dk[i][r] = 0.f;
      dv[i][r] = 0.f;
    }

  if (ntiles > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int st = t & 1;
    const bf16* qrows = smem + st * kStage;
    const bf16* qT = qrows + kRTile;
    const bf16* dorows = qT + kTTile;
    const bf16* doT = dorows + kRTile;
    if (t + 1 < ntiles) load_tile(t + 1);

    // S = Q K^T and dP = dO V^T for two 32-query halves.
    f32x16 s[2], dp[2];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[qt][r] = 0.f;
        dp[qt][r] = 0.f;
      }
      const bf16* qa = qrows + (32 * qt + li) * kRStride + 8 * hh;
      const bf16* da = dorows + (32 * qt + li) * kRStride + 8 * hh;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        s[qt] = mfma32(*reinterpret_cast<const bf16x8*>(qa + 16 * kk), kreg[kk], s[qt]);
        dp[qt] = mfma32(*reinterpret_cast<const bf16x8*>(da + 16 * kk), vreg[kk], dp[qt]);
      }
    }

    // P = exp2(S c - lse2[q]); dZ = P (dP - D[q]). Rows are queries.
    bf16x8 pb[4], zb[4];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int q0 = 32 * qt + 8 * rq + 4 * hh;
        const f32x4 l2 = *reinterpret_cast<const f32x4*>(&rowstat[st][0][q0]);
        const f32x4 dd = *reinterpret_cast<const f32x4*>(&rowstat[st][1][q0]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 4 * rq + i;
          const float pv = fast_exp2(s[qt][r] * p.c - l2[i]);
          const float zv = pv * (dp[qt][r] - dd[i]);
          const int c4 = 2 * qt + (r >> 3);
          pb[c4][r & 7] = (bf16)pv;
          zb[c4][r & 7] = (bf16)zv;
        }
      }
    }

    // dV^T += dO^T P, dK^T += Q^T dZ.
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const bf16* doa = doT + (32 * dt + li) * kTStride + 8 * hh;
      const bf16* qa = qT + (32 * dt + li) * kTStride + 8 * hh;
#pragma unroll
      for (int c4 = 0; c4 < 4; ++c4) {
        dv[dt] = mfma32(*reinterpret_cast<const bf16x8*>(doa + 16 * c4), pb[c4], dv[dt]);
        dk[dt] = mfma32(*reinterpret_cast<const bf16x8*>(qa + 16 * c4), zb[c4], dk[dt]);
      }
    }

    if (t + 1 < ntiles) store_tile(st ^ 1);
    __syncthreads();
  }

  if (key_ok) {
    bf16* dkp = p.dk + b * p.s_dk[0] + (int64_t)key * p.s_dk[1] + h * p.s_dk[2] + 4 * hh;
    bf16* dvp = p.dv + b * p.s_dv[0] + (int64_t)key * p.s_dv[1] + h * p.s_dv[2] + 4 * hh;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const f32x16& a = dk[dt];
        const f32x16& c = dv[dt];
        u32x2 wk = {pack_bf16(a[4 * rq] * p.scale, a[4 * rq + 1] * p.scale),
                    pack_bf16(a[4 * rq + 2] * p.scale, a[4 * rq + 3] * p.scale)};
        u32x2 wv = {pack_bf16(c[4 * rq], c[4 * rq + 1]), pack_bf16(c[4 * rq + 2], c[4 * rq + 3])};
        *reinterpret_cast<u32x2*>(dkp + 32 * dt + 8 * rq) = wk;
        *reinterpret_cast<u32x2*>(dvp + 32 * dt + 8 * rq) = wv;
      }
    }
  }
}

// ---------------------------------------------------------------------- dQ --

constexpr int kQueriesPerWg = 128;  // 4 waves x 32 queries

__global__ __launch_bounds__(256) void dq_kernel(Params p, int nqblk) {
  constexpr int kStage = 2 * kRTile + kTTile;  // K rows, K^T, V rows
  __shared__ __attribute__((aligned(16))) bf16 smem[2 * kStage];

  const int qblk = blockIdx.x % nqblk;
  const int bh = blockIdx.x / nqblk;
  const int b = bh / p.H, h = bh - (bh / p.H) * p.H;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int li = lane & 31, hh = lane >> 5;
  const int g4 = tid & 15, dc = tid >> 4;

  const int qrow = qblk * kQueriesPerWg + wave * 32 + li;
  const bool q_ok = qrow < p.Sq;
  bf16x8 qreg[8], doreg[8];
  {
    const bf16* qp = p.q + b * p.s_q[0] + h * p.s_q[2] + (int64_t)qrow * p.s_q[1] + 8 * hh;
    const bf16* dp = p.dout + b * p.s_do[0] + h * p.s_do[2] + (int64_t)qrow * p.s_do[1] + 8 * hh;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      u32x4 a = {0u, 0u, 0u, 0u}, c = {0u, 0u, 0u, 0u};
      if (q_ok) {
        a = ld16(qp + 16 * kk);
        c = ld16(dp + 16 * kk);
      }
      qreg[kk] = as_bf16x8(a);
      doreg[kk] = as_bf16x8(c);
    }
  }
  const int64_t srow = ((int64_t)b * p.H + h) * p.Sq + qrow;
  const float lse2 = q_ok ? p.lse[srow] * kLog2e : INFINITY;
  const float dlt = q_ok ? p.delta[srow] : 0.f;

  const bf16* kbase = p.k + b * p.s_k[0] + h * p.s_k[2];
  const bf16* vbase = p.v + b * p.s_v[0] + h * p.s_v[2];
  const int ntiles = (p.Sk + kT - 1) / kT;

  Unit uk, uv;
  auto load_tile = [&](int t) {
    load_unit(uk, kbase, p.s_k[1], t * kT, p.Sk, g4, dc);
    load_unit(uv, vbase, p.s_v[1], t * kT, p.Sk, g4, dc);
  };
  auto store_tile = [&](int st) {
    bf16* base = smem + st * kStage;
    store_rows(uk, base, g4, dc);
    store_transposed(uk, base + kRTile, g4, dc);
    store_rows(uv, base + kRTile + kTTile, g4, dc);
  };

  f32x16 dq[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[i][r] = 0.f;

  if (ntiles > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int st = t & 1;
    const bf16* krows = smem + st * kStage;
    const bf16* kT_ = krows + kRTile;
    const bf16* vrows = kT_ + kTTile;
    if (t + 1 < ntiles) load_tile(t + 1);

    f32x16 s[2], dp[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[kt][r] = 0.f;
        dp[kt][r] = 0.f;
      }
      const bf16* ka = krows + (32 * kt + li) * kRStride + 8 * hh;
      const bf16* va = vrows + (32 * kt + li) * kRStride + 8 * hh;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        s[kt] = mfma32(*reinterpret_cast<const bf16x8*>(ka + 16 * kk), qreg[kk], s[kt]);
        dp[kt] = mfma32(*reinterpret_cast<const bf16x8*>(va + 16 * kk), doreg[kk], dp[kt]);
      }
    }

    const int kb = t * kT;
    const bool partial = kb + kT > p.Sk;
    bf16x8 zb[4];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float pv = fast_exp2(s[kt][r] * p.c - lse2);
        if (partial && kb + 32 * kt + acc_row(r, hh) >= p.Sk) pv = 0.f;
        const float zv = pv * (dp[kt][r] - dlt);
        zb[2 * kt + (r >> 3)][r & 7] = (bf16)zv;
      }
    }

#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const bf16* ka = kT_ + (32 * dt + li) * kTStride + 8 * hh;
#pragma unroll
      for (int c4 = 0; c4 < 4; ++c4) {
        dq[dt] = mfma32(*reinterpret_cast<const bf16x8*>(ka + 16 * c4), zb[c4], dq[dt]);
      }
    }

    if (t + 1 < ntiles) store_tile(st ^ 1);
    __syncthreads();
  }

  if (q_ok) {
    bf16* dqp = p.dq + b * p.s_dq[0] + (int64_t)qrow * p.s_dq[1] + h * p.s_dq[2] + 4 * hh;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const f32x16& a = dq[dt];
        u32x2 w = {pack_bf16(a[4 * rq] * p.scale, a[4 * rq + 1] * p.scale),
                   pack_bf16(a[4 * rq + 2] * p.scale, a[4 * rq + 3] * p.scale)};
        *reinterpret_cast<u32x2*>(dqp + 32 * dt + 8 * rq) = w;
      }
    }
  }
}

static bool stride_ok(const int64_t* s) {
  return (s[0] % 8) == 0 && (s[1] % 8) == 0 && (s[2] % 8) == 0;
}

}  // namespace bwd
}  // namespace aa

using namespace aa;

extern "C" size_t aa_attn_bwd_workspace(int64_t B, int64_t Sq, int64_t Sk, int64_t H, int64_t hd) {
  (void)Sk;
  (void)hd;
  if (B <= 0 || Sq <= 0 || H <= 0) return 0;
  return (size_t)(B * H * Sq) * sizeof(float);
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
  const size_t need = aa_attn_bwd_workspace(a->B, a->Sq, a->Sk, a->H, a->hd);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return fail(AA_EINVAL, "attn_bwd: workspace too small");

  bwd::Params p;
  p.dout = (const bf16*)a->dout;
  p.q = (const bf16*)a->q;
  p.k = (const bf16*)a->k;
  p.v = (const bf16*)a->v;
  p.o = (const bf16*)a->out;
  p.lse = a->lse;
  p.delta = (float*)workspace;
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
  p.H = (int)a->H;
  p.Sq = (int)a->Sq;
  p.Sk = (int)a->Sk;
  p.scale = a->softmax_scale;
  p.c = a->softmax_scale * kLog2e;
  hipStream_t st = (hipStream_t)stream;

  const int64_t BH = a->B * a->H;
  if (a->Sq > 0) {
    const int64_t nrow = a->B * a->Sq * a->H;
    bwd::rowdot_kernel<<<dim3((unsigned)((nrow * 16 + 255) / 256)), 256, 0, st>>>(p, nrow);
    if (int rc = check_launch("attn_bwd rowdot")) return rc;
  }
  if (a->Sk > 0) {
    const int nkblk = (int)((a->Sk + bwd::kKeysPerWg - 1) / bwd::kKeysPerWg);
    bwd::dkdv_kernel<<<dim3((unsigned)(BH * nkblk)), 256, 0, st>>>(p, nkblk);
    if (int rc = check_launch("attn_bwd dkdv")) return rc;
  }
  if (a->Sq > 0) {
    const int nqblk = (int)((a->Sq + bwd::kQueriesPerWg - 1) / bwd::kQueriesPerWg);
    bwd::dq_kernel<<<dim3((unsigned)(BH * nqblk)), 256, 0, st>>>(p, nqblk);
    if (int rc = check_launch("attn_bwd dq")) return rc;
  }
  return AA_OK;
}
