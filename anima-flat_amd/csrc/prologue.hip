// QK-RMSNorm + rotate-half RoPE prologue and per-head RMSNorm, forward and
// backward, for head_dim 128 (two halves of 64).
//
// Work unit: one "section" = one (token, head) slice of 128 bf16 = 256 bytes,
// handled by a group of 8 lanes. Lane j of the group holds elements
// [8j, 8j+8) of the first half and [64+8j, 64+8j+8) of the second half, so
// every rotate-half pair (x[i], x[i+64]) sits in one lane and each lane moves
// two 16-byte chunks. The RMS sum is reduced over the 8 lanes of the group.
// The forward kernels give each group more than one section (see each).
//
// These kernels are HBM-bound: per section they read 256 B and write 256 B;
// cos/sin rows (2 x 256 B per token) and the weights stay in L2/L1.
#include "aa_common.h"
#include "norm_rope.h"

namespace aa {

// Section counts are below kMaxSections (the host checks): 2^31 sections of
// 256 bytes would be 512 GiB, more than one GPU holds, so 32-bit section
// indices cover every real tensor.
constexpr uint32_t kMaxSections = 0x7fffff00u;

// qkv [ntok, 3*H*128] -> q, k [ntok, H, 128] (+ v copy). A token's qkv row
// holds its q heads, then its k heads, then its v heads. Each 8-lane group
// takes one (token, head) pair: the q and k sections of that head (and the v
// section when copying V), which share the RoPE row of the token's position.
// All of the group's section loads are issued first, so a lane has four
// 16-byte loads in flight (six with V). A wave covers 8 consecutive pairs.
template <bool WITH_V>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(8, 8))) void
qkv_norm_rope_fwd_kernel(
    const bf16* __restrict__ qkv, bf16* __restrict__ q, bf16* __restrict__ k,
    bf16* __restrict__ v, const float* __restrict__ qw, const float* __restrict__ kw,
    const float* __restrict__ cos, const float* __restrict__ sin, uint32_t npair, uint32_t S,
    uint32_t H, float eps) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int j = (int)(gid & 7);
  // The last wave's surplus groups compute the last pair and store nothing.
  const bool valid = (gid >> 3) < (int64_t)npair;
  const uint32_t pair = valid ? (uint32_t)(gid >> 3) : npair - 1;
  const uint32_t token = pair / H;
  const uint32_t head = pair - token * H;
  const int64_t width = (int64_t)H * kHd;
  const bf16* row = qkv + (int64_t)token * 3 * width + head * kHd;
  RawSection xq, xk, xv;
  load_raw(row, j, xq);
  load_raw(row + width, j, xk);
  if constexpr (WITH_V) load_raw(row + 2 * width, j, xv);
  float c[8], s[8];
  load_rot(cos, sin, token % S, j, c, s);
  // Keeps all loads ahead of the first section's arithmetic.
  __builtin_amdgcn_sched_barrier(0);
  const int64_t dst_off = (int64_t)token * width + head * kHd;
  if constexpr (WITH_V) {
    if (valid) {
      st16_nt(v + dst_off + 8 * j, xv.a);
      st16_nt(v + dst_off + kHalf + 8 * j, xv.b);
    }
  }
  float oa[8], ob[8];
  norm_scale(unpack_section(xq), qw, j, eps, oa, ob);
  rotate_half(oa, ob, c, s);
  if (valid) {
    st16_nt(q + dst_off + 8 * j, pack8(oa));
    st16_nt(q + dst_off + kHalf + 8 * j, pack8(ob));
  }
  norm_scale(unpack_section(xk), kw, j, eps, oa, ob);
  rotate_half(oa, ob, c, s);
  if (valid) {
    st16_nt(k + dst_off + 8 * j, pack8(oa));
    st16_nt(k + dst_off + kHalf + 8 * j, pack8(ob));
  }
}

// Sections per 8-lane group in head_norm_fwd_kernel: a lane then has
// 2 kHnSecs 16-byte loads in flight before its first use. A wave takes
// 8 kHnSecs consecutive sections, its group r sections r, r + 8, ..., so
// each pair of load instructions reads 2 KiB of consecutive bytes.
constexpr int kHnSecs = 2;

// Section index of round i for lane gid.
__device__ __forceinline__ uint32_t hn_section(int64_t gid, int i) {
  return (uint32_t)(gid >> 6) * (8 * kHnSecs) + 8 * i + ((uint32_t)(gid >> 3) & 7);
}

// x [ntok, H*128] -> y [ntok, H, 128].
__global__ __launch_bounds__(256) void head_norm_fwd_kernel(const bf16* __restrict__ x,
                                                            bf16* __restrict__ y,
                                                            const float* __restrict__ w,
                                                            uint32_t nsec, float eps) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int j = (int)(gid & 7);
  RawSection xs[kHnSecs];
#pragma unroll
  for (int i = 0; i < kHnSecs; ++i)
    load_raw(x + (int64_t)min(hn_section(gid, i), nsec - 1) * kHd, j, xs[i]);
  __builtin_amdgcn_sched_barrier(0);  // all rounds' loads first
#pragma unroll
  for (int i = 0; i < kHnSecs; ++i) {
    const uint32_t sec = hn_section(gid, i);
    float oa[8], ob[8];
    norm_scale(unpack_section(xs[i]), w, j, eps, oa, ob);
    if (sec < nsec) {  // out-of-range rounds computed the clamped last section
      bf16* dst = y + (int64_t)sec * kHd;
      st16_nt(dst + 8 * j, pack8(oa));
      st16_nt(dst + kHalf + 8 * j, pack8(ob));
    }
  }
}

// ------------------------------------------------------------- backward --

// Threads per block of the head_norm and the QKV backward. For the QKV
// backward 256 threads measured 28.3 us at config 5 against 26.2 us (twice
// the partial records for the reduction to read).
constexpr int kBwdThreads = 512;
constexpr int kBwdGroups = kBwdThreads / 8;  // 8-lane groups per block
constexpr int kQkvThreads = 512;
constexpr int kQkvGroups = kQkvThreads / 8;
// (token, head) items per block: one per group in the QKV backward, two in
// the head_norm backward.
constexpr int kQkvBwdItems = kQkvGroups;
constexpr int kHnBwdItems = 2 * kBwdGroups;

// Backward of one section (src/kernels/rope.py:244-274): rotate dy back,
// then dx = rstd * (u - xhat * mean(u * xhat)) with u = dy' * w; g receives
// this lane's 16 weight-gradient terms dy' * xhat (a half, then b half).
template <bool ROTATE>
__device__ __forceinline__ void norm_section_bwd(Section x, Section d, const float* w,
                                                 const float* c, const float* sn, int j,
                                                 float eps, float* oa, float* ob, float* g) {
  if constexpr (ROTATE) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float da = d.a[i], db = d.b[i];
      d.a[i] = da * c[i] + db * sn[i];
      d.b[i] = db * c[i] - da * sn[i];
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss += x.a[i] * x.a[i] + x.b[i] * x.b[i];
  ss = group_sum<8>(ss);
  const float rstd = rsqrtf(ss / (float)kHd + eps);
  float wa[8], wb[8];
  load_w(w, j, wa, wb);
  float dot = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    x.a[i] *= rstd;  // xhat
    x.b[i] *= rstd;
    dot += (d.a[i] * wa[i]) * x.a[i] + (d.b[i] * wb[i]) * x.b[i];
  }
  const float cm = group_sum<8>(dot) / (float)kHd;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    oa[i] = rstd * (d.a[i] * wa[i] - x.a[i] * cm);
    ob[i] = rstd * (d.b[i] * wb[i] - x.b[i] * cm);
    g[i] = d.a[i] * x.a[i];
    g[8 + i] = d.b[i] * x.b[i];
  }
}

// Arguments of both backward kernels (head_norm: x, dy0, dx, w0 only).
struct NormBwdParams {
  const bf16* x;    // [ntok, xrow]: q sections at row offset head * 128, k at (H + head) * 128
  const bf16* dy0;  // [ntok, H * 128] gradient of the first normalised set (q)
  const bf16* dy1;  // [ntok, H * 128] gradient of the second (k); QKV only
  const bf16* dv;   // [ntok, H * 128] copied into dx at row offset (2 H + head) * 128; QKV only
  bf16* dx;         // [ntok, xrow]
  const float* w0;
  const float* w1;
  const float* cos;
  const float* sin;
  float* partial;  // [nblock][2 * 128] (head_norm [nblock][128]) weight-gradient sums
  uint32_t nitem, S, H;
  uint32_t xrow;  // elements per x / dx row
  float eps;
};

// QKV backward: one (token, head) item per 8-lane group, 64 per block, no
// loop. The item is a head's q and k sections, their gradients and its dV
// section (passed through into dqkv): all ten 16-byte loads per lane, and
// the RoPE row of the token, are issued before any arithmetic. Each group
// writes its weight-gradient terms to its own LDS row; the block adds the 64
// rows in order into partial[block].
__device__ __forceinline__ void qkv_norm_bwd_block(const NormBwdParams& p) {
  constexpr int kRow = 2 * kHd + 4;  // q terms, k terms; padded against LDS bank conflicts
  __shared__ __align__(16) float red[kQkvGroups * kRow];
  const int tid = threadIdx.x;
  const int j = tid & 7;
  const int g = tid >> 3;
  const uint32_t item = blockIdx.x * kQkvGroups + g;
  const bool valid = item < p.nitem;
  const uint32_t it = valid ? item : p.nitem - 1;  // surplus groups redo the last item
  const uint32_t token = it / p.H;
  const uint32_t head = it - token * p.H;
  const int64_t width = (int64_t)p.H * kHd;
  const bf16* xrow = p.x + (int64_t)token * p.xrow + head * kHd;
  const int64_t doff = (int64_t)token * width + head * kHd;

  RawSection xq, dq, xk, dk, vv;
  float c[8], sn[8];
  load_raw(xrow, j, xq);
  load_raw(p.dy0 + doff, j, dq);
  load_raw(xrow + width, j, xk);
  load_raw(p.dy1 + doff, j, dk);
  load_raw(p.dv + doff, j, vv);
  load_rot(p.cos, p.sin, token % p.S, j, c, sn);
  __builtin_amdgcn_sched_barrier(0);  // all loads first

  bf16* dxrow = p.dx + (int64_t)token * p.xrow + head * kHd;
  if (valid) {
    st16_nt(dxrow + 2 * width + 8 * j, vv.a);
    st16_nt(dxrow + 2 * width + kHalf + 8 * j, vv.b);
  }
  float oa[8], ob[8], gr[16];
  float* row = red + g * kRow;
  norm_section_bwd<true>(unpack_section(xq), unpack_section(dq), p.w0, c, sn, j, p.eps, oa, ob,
                         gr);
  if (valid) {
    st16_nt(dxrow + 8 * j, pack8(oa));
    st16_nt(dxrow + kHalf + 8 * j, pack8(ob));
  }
#pragma unroll
  for (int i = 0; i < 8; i += 4) {  // invalid items add zeros
    const float m = valid ? 1.f : 0.f;
    *reinterpret_cast<f32x4*>(row + 8 * j + i) =
        f32x4{m * gr[i], m * gr[i + 1], m * gr[i + 2], m * gr[i + 3]};
    *reinterpret_cast<f32x4*>(row + kHalf + 8 * j + i) =
        f32x4{m * gr[8 + i], m * gr[9 + i], m * gr[10 + i], m * gr[11 + i]};
  }
  norm_section_bwd<true>(unpack_section(xk), unpack_section(dk), p.w1, c, sn, j, p.eps, oa, ob,
                         gr);
  if (valid) {
    st16_nt(dxrow + width + 8 * j, pack8(oa));
    st16_nt(dxrow + width + kHalf + 8 * j, pack8(ob));
  }
#pragma unroll
  for (int i = 0; i < 8; i += 4) {
    const float m = valid ? 1.f : 0.f;
    *reinterpret_cast<f32x4*>(row + kHd + 8 * j + i) =
        f32x4{m * gr[i], m * gr[i + 1], m * gr[i + 2], m * gr[i + 3]};
    *reinterpret_cast<f32x4*>(row + kHd + kHalf + 8 * j + i) =
        f32x4{m * gr[8 + i], m * gr[9 + i], m * gr[10 + i], m * gr[11 + i]};
  }
  __syncthreads();
  if (tid < 2 * kHd) {
    float sum = 0.f;
    for (int gg = 0; gg < kQkvGroups; ++gg) sum += red[gg * kRow + tid];
    p.partial[(int64_t)blockIdx.x * 2 * kHd + tid] = sum;
  }
}

// head_norm backward: each 8-lane group takes items g and 64 + g of the
// block's 128 (sections in [token, head] order), all four 16-byte loads per
// lane issued first, and adds both sections' weight-gradient terms before
// they go to its LDS row.
__device__ __forceinline__ void head_norm_bwd_block(const NormBwdParams& p) {
  constexpr int kRow = kHd + 4;
  __shared__ __align__(16) float red[kBwdGroups * kRow];
  const int tid = threadIdx.x;
  const int j = tid & 7;
  const int g = tid >> 3;
  RawSection x[2], d[2];
  uint32_t sec[2];
  bool valid[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint32_t idx = blockIdx.x * kHnBwdItems + i * kBwdGroups + g;
    valid[i] = idx < p.nitem;
    sec[i] = valid[i] ? idx : p.nitem - 1;
    load_raw(p.x + (int64_t)sec[i] * kHd, j, x[i]);
    load_raw(p.dy0 + (int64_t)sec[i] * kHd, j, d[i]);
  }
  __builtin_amdgcn_sched_barrier(0);  // all loads first
  float acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.f;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    float oa[8], ob[8], gr[16];
    norm_section_bwd<false>(unpack_section(x[i]), unpack_section(d[i]), p.w0, nullptr, nullptr,
                            j, p.eps, oa, ob, gr);
    if (valid[i]) {
      bf16* out = p.dx + (int64_t)sec[i] * kHd;
      st16_nt(out + 8 * j, pack8(oa));
      st16_nt(out + kHalf + 8 * j, pack8(ob));
    }
    const float m = valid[i] ? 1.f : 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = fmaf(m, gr[e], acc[e]);
  }
  float* row = red + g * kRow;
#pragma unroll
  for (int i = 0; i < 8; i += 4) {
    *reinterpret_cast<f32x4*>(row + 8 * j + i) = f32x4{acc[i], acc[i + 1], acc[i + 2], acc[i + 3]};
    *reinterpret_cast<f32x4*>(row + kHalf + 8 * j + i) =
        f32x4{acc[8 + i], acc[9 + i], acc[10 + i], acc[11 + i]};
  }
  __syncthreads();
  if (tid < kHd) {
    float sum = 0.f;
    for (int gg = 0; gg < kBwdGroups; ++gg) sum += red[gg * kRow + tid];
    p.partial[(int64_t)blockIdx.x * kHd + tid] = sum;
  }
}

__global__ __launch_bounds__(kQkvThreads) void qkv_norm_bwd_kernel(NormBwdParams p) {
  qkv_norm_bwd_block(p);
}
__global__ __launch_bounds__(kBwdThreads) void head_norm_bwd_kernel(NormBwdParams p) {
  head_norm_bwd_block(p);
}

// Weight-gradient reduction of partial[nrow][n] (n = 128 or 256 outputs) in
// one launch, in a fixed order. Block b owns outputs 32 b .. 32 b + 31, one
// 128-byte line of every partial row: 8 lanes read a row's line as 16-byte
// loads (so the launch fetches each partial byte once), 128 row groups take
// rows r, r + 128, ... (a batch's loads issued together, then added in
// order), and the 128 group sums meet in a fixed pairwise tree through LDS.
// The launch is bound by latency, not bytes: ~4.1-4.7 us for the 1 MB of
// config 5's partials, the same with 64 blocks reading 16-byte columns
// (which fetch each line 8 times). (Folding this into the norm kernel's
// tail, the last block of each group of chunks adding behind a device-scope
// atomic counter, measured 105 us instead of ~30 for the whole backward: on
// the 8-XCD MI355X a device-scope release fence writes back the XCD's L2,
// once per block.)
constexpr int kRedThreads = 1024;
constexpr int kRedRowGroups = kRedThreads / 8;
constexpr int kRedCols = 32;
__global__ __launch_bounds__(kRedThreads) void reduce_partials_kernel(
    const float* __restrict__ partial, uint32_t nrow, int n, float* __restrict__ out0,
    float* __restrict__ out1) {
  constexpr int kBatch = 8;
  __shared__ f32x4 red[kRedRowGroups][8];
  const int l8 = threadIdx.x & 7;
  const int rg = threadIdx.x >> 3;
  const int col = blockIdx.x * kRedCols + 4 * l8;
  f32x4 s = {0.f, 0.f, 0.f, 0.f};
  uint32_t r = rg;
  for (; r + (uint32_t)kRedRowGroups * (kBatch - 1) < nrow; r += kRedRowGroups * kBatch) {
    f32x4 t[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i)
      t[i] = ldf4(partial + (int64_t)(r + kRedRowGroups * i) * n + col);
#pragma unroll
    for (int i = 0; i < kBatch; ++i) s += t[i];
  }
  for (; r < nrow; r += kRedRowGroups) s += ldf4(partial + (int64_t)r * n + col);
  red[rg][l8] = s;
  __syncthreads();
#pragma unroll
  for (int w = kRedRowGroups / 2; w > 0; w >>= 1) {
    if (rg < w) red[rg][l8] += red[rg + w][l8];
    __syncthreads();
  }
  if (threadIdx.x < kRedCols) {
    const int c = threadIdx.x;
    const int o = blockIdx.x * kRedCols + c;
    const float t = red[0][c / 4][c % 4];
    if (o < kHd) out0[o] = t;
    else out1[o - kHd] = t;
  }
}

__global__ void zero_f32_kernel(float* __restrict__ a, float* __restrict__ b, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    a[i] = 0.f;
    b[i] = 0.f;
  }
}

// Blocks of a backward over nitem (token, head) items, per_block each.
static int64_t bwd_blocks(int64_t nitem, int per_block) {
  return (nitem + per_block - 1) / per_block;
}
// Weight-gradient workspace: the blocks' partials.
static size_t wgrad_workspace(int64_t nitem, int64_t n, int per_block) {
  return (size_t)bwd_blocks(nitem, per_block) * (size_t)n * sizeof(float);
}

// The norm launch, then the fixed-order weight-gradient reduction into out0
// (first weight) and out1 (second).
template <bool QKV>
static int launch_norm_bwd(NormBwdParams p, int64_t nitem, float* out0, float* out1,
                           hipStream_t st, const char* what) {
  p.nitem = (uint32_t)nitem;
  const dim3 grid((unsigned)bwd_blocks(nitem, QKV ? kQkvBwdItems : kHnBwdItems));
  if constexpr (QKV) qkv_norm_bwd_kernel<<<grid, kQkvThreads, 0, st>>>(p);
  else head_norm_bwd_kernel<<<grid, kBwdThreads, 0, st>>>(p);
  if (int rc = check_launch(what)) return rc;
  const int n = (QKV ? 2 : 1) * kHd;
  reduce_partials_kernel<<<dim3(n / kRedCols), kRedThreads, 0, st>>>(p.partial, grid.x, n, out0,
                                                                     out1);
  return check_launch(what);
}

static int check_common(int64_t B, int64_t S, int64_t H, int64_t hd, int dtype) {
  if (dtype != AA_DTYPE_BF16) return fail(AA_EUNSUPPORTED, "only bf16 activations are implemented");
  if (hd != kHd) return fail(AA_EUNSUPPORTED, "head_dim must be 128");
  if (B < 0 || S < 0 || H <= 0 || H > 4096) return fail(AA_EINVAL, "bad B/S/H");
  return AA_OK;
}

}  // namespace aa

using namespace aa;

extern "C" int aa_qkv_norm_rope_fwd(const void* qkv, void* q, void* k, void* v,
                                    const float* q_weight, const float* k_weight,
                                    const float* cos, const float* sin, int64_t B, int64_t S,
                                    int64_t H, int64_t hd, float eps, int dtype, void* stream) {
  clear_error();
  if (int rc = check_common(B, S, H, hd, dtype)) return rc;
  if (B * S == 0) return AA_OK;
  if (!qkv || !q || !k || !q_weight || !k_weight || !cos || !sin)
    return fail(AA_EINVAL, "qkv_norm_rope_fwd: null pointer");
  if (!aligned16(qkv) || !aligned16(q) || !aligned16(k) || (v && !aligned16(v)) ||
      !aligned16(q_weight) || !aligned16(k_weight) || !aligned16(cos) || !aligned16(sin))
    return fail(AA_EINVAL, "qkv_norm_rope_fwd: pointers must be 16-byte aligned");
  const int64_t npair = B * S * H;
  if (3 * npair > (int64_t)kMaxSections)
    return fail(AA_EINVAL, "qkv_norm_rope_fwd: tensor too large");
  const dim3 grid((unsigned)((npair * 8 + 255) / 256));
  hipStream_t st = (hipStream_t)stream;
  if (v) {
    qkv_norm_rope_fwd_kernel<true><<<grid, 256, 0, st>>>(
        (const bf16*)qkv, (bf16*)q, (bf16*)k, (bf16*)v, q_weight, k_weight, cos, sin,
        (uint32_t)npair, (uint32_t)S, (uint32_t)H, eps);
  } else {
    qkv_norm_rope_fwd_kernel<false><<<grid, 256, 0, st>>>(
        (const bf16*)qkv, (bf16*)q, (bf16*)k, nullptr, q_weight, k_weight, cos, sin,
        (uint32_t)npair, (uint32_t)S, (uint32_t)H, eps);
  }
  return check_launch("qkv_norm_rope_fwd");
}

extern "C" int aa_head_norm_fwd(const void* x, void* y, const float* weight, int64_t B, int64_t S,
                                int64_t H, int64_t hd, float eps, int dtype, void* stream) {
  clear_error();
  if (int rc = check_common(B, S, H, hd, dtype)) return rc;
  if (B * S == 0) return AA_OK;
  if (!x || !y || !weight) return fail(AA_EINVAL, "head_norm_fwd: null pointer");
  if (!aligned16(x) || !aligned16(y) || !aligned16(weight))
    return fail(AA_EINVAL, "head_norm_fwd: pointers must be 16-byte aligned");
  const int64_t nsec = B * S * H;
  if (nsec > (int64_t)kMaxSections) return fail(AA_EINVAL, "head_norm_fwd: tensor too large");
  const dim3 grid((unsigned)(((nsec + kHnSecs - 1) / kHnSecs * 8 + 255) / 256));
  head_norm_fwd_kernel<<<grid, 256, 0, (hipStream_t)stream>>>((const bf16*)x, (bf16*)y, weight,
                                                              (uint32_t)nsec, eps);
  return check_launch("head_norm_fwd");
}

extern "C" size_t aa_qkv_norm_rope_bwd_workspace(int64_t B, int64_t S, int64_t H, int64_t hd) {
  if (B <= 0 || S <= 0 || H <= 0) return 0;
  return wgrad_workspace(B * S * H, 2 * hd, kQkvBwdItems);
}

extern "C" size_t aa_head_norm_bwd_workspace(int64_t B, int64_t S, int64_t H, int64_t hd) {
  if (B <= 0 || S <= 0 || H <= 0) return 0;
  return wgrad_workspace(B * S * H, hd, kHnBwdItems);
}

extern "C" int aa_qkv_norm_rope_bwd(const void* qkv, const void* dq, const void* dk,
                                    const void* dv, void* dqkv, const float* q_weight,
                                    const float* k_weight, const float* cos, const float* sin,
                                    float* dq_weight, float* dk_weight, void* workspace,
                                    size_t workspace_bytes, int64_t B, int64_t S, int64_t H,
                                    int64_t hd, float eps, int dtype, void* stream) {
  clear_error();
  if (int rc = check_common(B, S, H, hd, dtype)) return rc;
  if (!qkv || !dq || !dk || !dv || !dqkv || !q_weight || !k_weight || !cos || !sin ||
      !dq_weight || !dk_weight)
    return fail(AA_EINVAL, "qkv_norm_rope_bwd: null pointer");
  if (!aligned16(qkv) || !aligned16(dq) || !aligned16(dk) || !aligned16(dv) ||
      !aligned16(dqkv) || !aligned16(q_weight) || !aligned16(k_weight) || !aligned16(cos) ||
      !aligned16(sin))
    return fail(AA_EINVAL, "qkv_norm_rope_bwd: pointers must be 16-byte aligned");
  const int64_t ntok = B * S;
  if (3 * ntok * H > (int64_t)kMaxSections)
    return fail(AA_EINVAL, "qkv_norm_rope_bwd: tensor too large");
  if (ntok > 0 && (!workspace || workspace_bytes < aa_qkv_norm_rope_bwd_workspace(B, S, H, hd)))
    return fail(AA_EINVAL, "qkv_norm_rope_bwd: workspace too small");
  hipStream_t st = (hipStream_t)stream;
  if (ntok == 0) {  // no tokens: weight gradients are zero
    zero_f32_kernel<<<1, kHd, 0, st>>>(dq_weight, dk_weight, kHd);
    return check_launch("qkv_norm_rope_bwd zero");
  }
  NormBwdParams p{};
  p.x = (const bf16*)qkv;
  p.dy0 = (const bf16*)dq;
  p.dy1 = (const bf16*)dk;
  p.dv = (const bf16*)dv;
  p.dx = (bf16*)dqkv;
  p.w0 = q_weight;
  p.w1 = k_weight;
  p.cos = cos;
  p.sin = sin;
  p.partial = (float*)workspace;
  p.S = (uint32_t)S;
  p.H = (uint32_t)H;
  p.xrow = (uint32_t)(3 * H * kHd);
  p.eps = eps;
  return launch_norm_bwd<true>(p, ntok * H, dq_weight, dk_weight, st, "qkv_norm_rope_bwd");
}

extern "C" int aa_head_norm_bwd(const void* x, const void* dy, void* dx, const float* weight,
                                float* dweight, void* workspace, size_t workspace_bytes, int64_t B,
                                int64_t S, int64_t H, int64_t hd, float eps, int dtype,
                                void* stream) {
  clear_error();
  if (int rc = check_common(B, S, H, hd, dtype)) return rc;
  if (!x || !dy || !dx || !weight || !dweight) return fail(AA_EINVAL, "head_norm_bwd: null pointer");
  if (!aligned16(x) || !aligned16(dy) || !aligned16(dx) || !aligned16(weight))
    return fail(AA_EINVAL, "head_norm_bwd: pointers must be 16-byte aligned");
  const int64_t ntok = B * S;
  if (ntok * H > (int64_t)kMaxSections) return fail(AA_EINVAL, "head_norm_bwd: tensor too large");
  if (ntok > 0 && (!workspace || workspace_bytes < aa_head_norm_bwd_workspace(B, S, H, hd)))
    return fail(AA_EINVAL, "head_norm_bwd: workspace too small");
  hipStream_t st = (hipStream_t)stream;
  if (ntok == 0) {
    zero_f32_kernel<<<1, kHd, 0, st>>>(dweight, dweight, kHd);
    return check_launch("head_norm_bwd zero");
  }
  NormBwdParams p{};
  p.x = (const bf16*)x;
  p.dy0 = (const bf16*)dy;
  p.dy1 = (const bf16*)dy;
  p.dx = (bf16*)dx;
  p.w0 = weight;
  p.w1 = weight;
  p.partial = (float*)workspace;
  p.S = (uint32_t)S;
  p.H = (uint32_t)H;
  p.xrow = (uint32_t)(H * kHd);
  p.eps = eps;
  return launch_norm_bwd<false>(p, ntok * H, dweight, dweight, st, "head_norm_bwd");
}
