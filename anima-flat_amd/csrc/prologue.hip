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

// Backward of one section (src/kernels/rope.py:244-274): rotate dy back,
// then dx = rstd * (u - xhat * mean(u * xhat)) with u = dy' * w; returns the
// per-dimension weight-gradient terms dy' * xhat through ga/gb.
template <bool ROTATE>
__device__ __forceinline__ void norm_section_bwd(const bf16* src, const bf16* dy, bf16* dx,
                                                 const float* w, const float* cos,
                                                 const float* sin, int64_t pos, int j, float eps,
                                                 float* ga, float* gb) {
  Section x, d;
  load_section(src, j, x);
  load_section(dy, j, d);
  if constexpr (ROTATE) {
    float c[8], s[8];
    load_rot(cos, sin, pos, j, c, s);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float da = d.a[i], db = d.b[i];
      d.a[i] = da * c[i] + db * s[i];
      d.b[i] = db * c[i] - da * s[i];
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss += x.a[i] * x.a[i] + x.b[i] * x.b[i];
  ss = group_sum<8>(ss);
  const float rstd = rsqrtf(ss / (float)kHd + eps);
  float wa[8], wb[8];
  load_w(w, j, wa, wb);
  float xa[8], xb[8], ua[8], ub[8];
  float dot = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    xa[i] = x.a[i] * rstd;
    xb[i] = x.b[i] * rstd;
    ua[i] = d.a[i] * wa[i];
    ub[i] = d.b[i] * wb[i];
    dot += ua[i] * xa[i] + ub[i] * xb[i];
  }
  const float c = group_sum<8>(dot) / (float)kHd;
  float oa[8], ob[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    oa[i] = rstd * (ua[i] - xa[i] * c);
    ob[i] = rstd * (ub[i] - xb[i] * c);
    ga[i] += d.a[i] * xa[i];
    gb[i] += d.b[i] * xb[i];
  }
  st16_nt(dx + 8 * j, pack8(oa));
  st16_nt(dx + kHalf + 8 * j, pack8(ob));
}

constexpr int kBwdThreads = 256;
constexpr int kBwdGroups = kBwdThreads / 8;  // 32 sections in flight per block

// One block per chunk of `rows` consecutive tokens. Normalised sections per
// token: NWHICH*H (q then k for the QKV prologue, one set for head_norm).
// Group g handles items g, g+32, ... of the chunk's (token, section) pairs
// and keeps per-lane weight-gradient sums for each of the NWHICH weights; the
// block then reduces them over groups in a fixed order into
// partial[chunk][which][128].
template <bool ROTATE, int NWHICH>
__global__ __launch_bounds__(kBwdThreads) void norm_bwd_kernel(
    const bf16* __restrict__ x, const bf16* __restrict__ dy0, const bf16* __restrict__ dy1,
    const bf16* __restrict__ dv, bf16* __restrict__ dx, const float* __restrict__ w0,
    const float* __restrict__ w1, const float* __restrict__ cos, const float* __restrict__ sin,
    float* __restrict__ partial, int64_t ntok, int64_t S, int H, int rows, float eps) {
  __shared__ float red[kBwdGroups][NWHICH][kHd];
  const int tid = threadIdx.x;
  const int j = tid & 7;
  const int g = tid >> 3;
  const int64_t width = (int64_t)H * kHd;
  // x and dx rows hold NWHICH (+1 with dv) sections of width H*128 each.
  const int64_t xrow = dv ? 3 * width : NWHICH * width;
  float acc[NWHICH][16];
#pragma unroll
  for (int wi = 0; wi < NWHICH; ++wi)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[wi][i] = 0.f;

  const int64_t first = (int64_t)blockIdx.x * rows;
  const int nrows = (int)(ntok - first < rows ? ntok - first : rows);
  // The chunk's (token, section) pairs in token-major order, dealt to the
  // groups round-robin, so every group works whatever H is (head_norm has
  // 16 sections per token for 32 groups).
  const int per_tok = NWHICH * H;
  int r = g / per_tok;
  int sec = g - r * per_tok;
  while (r < nrows) {
    const int64_t token = first + r;
    const int which = sec / H;
    const int head = sec - which * H;
    const bf16* src = x + token * xrow + which * width + head * kHd;
    const bf16* dy = (which == 0 ? dy0 : dy1) + token * width + head * kHd;
    bf16* out = dx + token * xrow + which * width + head * kHd;
    const float* w = which == 0 ? w0 : w1;
    const int64_t pos = token % S;
    if (NWHICH == 1 || which == 0) {
      norm_section_bwd<ROTATE>(src, dy, out, w, cos, sin, pos, j, eps, acc[0], acc[0] + 8);
    } else {
      norm_section_bwd<ROTATE>(src, dy, out, w, cos, sin, pos, j, eps, acc[NWHICH - 1],
                               acc[NWHICH - 1] + 8);
    }
    sec += kBwdGroups;
    while (sec >= per_tok) {
      sec -= per_tok;
      ++r;
    }
  }
  if (dv) {  // dV passes through the prologue unchanged: copy it into dqkv.
    for (int rr = 0; rr < nrows; ++rr) {
      const int64_t token = first + rr;
      for (int c = tid; c < (int)(width / 8); c += kBwdThreads) {
        st16_nt(dx + token * xrow + 2 * width + 8 * c, ld16(dv + token * width + 8 * c));
      }
    }
  }
#pragma unroll
  for (int wi = 0; wi < NWHICH; ++wi) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      red[g][wi][8 * j + i] = acc[wi][i];
      red[g][wi][kHalf + 8 * j + i] = acc[wi][8 + i];
    }
  }
  __syncthreads();
  for (int o = tid; o < NWHICH * kHd; o += kBwdThreads) {
    const int wi = o / kHd, dim = o % kHd;
    float s = 0.f;
    for (int gg = 0; gg < kBwdGroups; ++gg) s += red[gg][wi][dim];
    partial[((int64_t)blockIdx.x * NWHICH + wi) * kHd + dim] = s;
  }
}

// Weight-gradient reduction of partial[nchunk][n] (n <= 256 outputs) in one
// launch, in a fixed order: block b owns outputs 8 b .. 8 b + 7; its 32 lane
// groups r sum chunks r, r + 32, r + 64, ... in order (the loads of a batch
// issued together, then added in sequence), and the 32 group sums are added
// in order through LDS. (Folding this into norm_bwd_kernel's tail, the last
// block of each group of chunks adding behind a device-scope atomic counter,
// measured 105 us instead of ~30 for the whole backward: on the 8-XCD MI355X a
// device-scope release fence writes back the XCD's L2, once per block.)
constexpr int kRedOut = 8;     // outputs per block
constexpr int kRedLanes = 32;  // lane groups per output
__global__ __launch_bounds__(kRedOut * kRedLanes) void reduce_partials_kernel(
    const float* __restrict__ partial, int64_t nchunk, int n, float* __restrict__ out0,
    float* __restrict__ out1) {
  constexpr int kBatch = 8;
  __shared__ float red[kRedLanes][kRedOut];
  const int oo = threadIdx.x % kRedOut;
  const int r = threadIdx.x / kRedOut;
  const int o = blockIdx.x * kRedOut + oo;
  float s = 0.f;
  if (o < n) {
    int64_t c = r;
    for (; c + (int64_t)kRedLanes * (kBatch - 1) < nchunk; c += (int64_t)kRedLanes * kBatch) {
      float t[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) t[i] = partial[(c + (int64_t)kRedLanes * i) * n + o];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) s += t[i];
    }
    for (; c < nchunk; c += kRedLanes) s += partial[c * n + o];
  }
  red[r][oo] = s;
  __syncthreads();
  if (r == 0 && o < n) {
    float t = 0.f;
    for (int rr = 0; rr < kRedLanes; ++rr) t += red[rr][oo];
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

constexpr int kBwdRows = 8;  // tokens per block: enough blocks to keep the CUs' loads in flight

static int64_t bwd_chunks(int64_t B, int64_t S) { return (B * S + kBwdRows - 1) / kBwdRows; }
// Weight-gradient workspace: the per-chunk partials.
static size_t wgrad_workspace(int64_t B, int64_t S, int64_t n) {
  return (size_t)bwd_chunks(B, S) * (size_t)n * sizeof(float);
}

// Fixed-order sum of partial[nchunk][n] into out0 / out1 (outputs 0..127 /
// 128..255).
static void reduce_wgrad(float* partial, int64_t nchunk, int n, float* out0, float* out1,
                         hipStream_t st) {
  reduce_partials_kernel<<<dim3((unsigned)((n + kRedOut - 1) / kRedOut)), kRedOut * kRedLanes, 0,
                           st>>>(partial, nchunk, n, out0, out1);
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
  (void)H;
  return wgrad_workspace(B, S, 2 * hd);
}

extern "C" size_t aa_head_norm_bwd_workspace(int64_t B, int64_t S, int64_t H, int64_t hd) {
  (void)H;
  return wgrad_workspace(B, S, hd);
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
  const int64_t nchunk = bwd_chunks(B, S);
  if (nchunk > 0 && (!workspace || workspace_bytes < aa_qkv_norm_rope_bwd_workspace(B, S, H, hd)))
    return fail(AA_EINVAL, "qkv_norm_rope_bwd: workspace too small");
  hipStream_t st = (hipStream_t)stream;
  if (nchunk == 0) {  // no tokens: weight gradients are zero
    zero_f32_kernel<<<1, kHd, 0, st>>>(dq_weight, dk_weight, kHd);
    return check_launch("qkv_norm_rope_bwd zero");
  }
  float* partial = (float*)workspace;
  norm_bwd_kernel<true, 2><<<dim3((unsigned)nchunk), kBwdThreads, 0, st>>>(
      (const bf16*)qkv, (const bf16*)dq, (const bf16*)dk, (const bf16*)dv, (bf16*)dqkv,
      q_weight, k_weight, cos, sin, partial, B * S, S, (int)H, kBwdRows, eps);
  if (int rc = check_launch("qkv_norm_rope_bwd")) return rc;
  reduce_wgrad(partial, nchunk, 2 * kHd, dq_weight, dk_weight, st);
  return check_launch("qkv_norm_rope_bwd reduce");
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
  const int64_t nchunk = bwd_chunks(B, S);
  if (nchunk > 0 && (!workspace || workspace_bytes < aa_head_norm_bwd_workspace(B, S, H, hd)))
    return fail(AA_EINVAL, "head_norm_bwd: workspace too small");
  hipStream_t st = (hipStream_t)stream;
  if (nchunk == 0) {
    zero_f32_kernel<<<1, kHd, 0, st>>>(dweight, dweight, kHd);
    return check_launch("head_norm_bwd zero");
  }
  float* partial = (float*)workspace;
  norm_bwd_kernel<false, 1><<<dim3((unsigned)nchunk), kBwdThreads, 0, st>>>(
      (const bf16*)x, (const bf16*)dy, nullptr, nullptr, (bf16*)dx, weight, weight, nullptr,
      nullptr, partial, B * S, S, (int)H, kBwdRows, eps);
  if (int rc = check_launch("head_norm_bwd")) return rc;
  reduce_wgrad(partial, nchunk, kHd, dweight, dweight, st);
  return check_launch("head_norm_bwd reduce");
}
