// Padding correction of trimmed cross-attention, forward and backward.
//
// Attention over only the first len keys of a zero-padded context of S_full
// keys differs from attention over all of them: the padded keys have logit 0
// and value 0, so they only add (S_full - len) to the softmax denominator.
// With lse the log-sum-exp over the kept keys and ln_pad = log(S_full - len),
// the full result is out * g with g = 1/(1 + exp(ln_pad - lse)).
//
// Layout: out, y, dy, dout [B, S, H, 128] contiguous; lse, dlse [B, H, S];
// ln_pad [B]. 16 lanes per (token, head) row of 128 values, 8 values a lane.
#include "aa_common.h"

namespace aa {

constexpr int kCsHd = 128;

__device__ __forceinline__ float pad_gain(float ln_pad, float lse) {
  return 1.0f / (1.0f + expf(ln_pad - lse));
}

__global__ __launch_bounds__(256) void ctx_scale_fwd_kernel(const bf16* __restrict__ out,
                                                            const float* __restrict__ lse,
                                                            const float* __restrict__ ln_pad,
                                                            bf16* __restrict__ y, int64_t nrow,
                                                            int64_t S, int H) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row = gid >> 4;  // (token, head)
  if (row >= nrow) return;
  const int lane = (int)(gid & 15);
  const int64_t token = row / H;
  const int head = (int)(row - token * H);
  const int64_t b = token / S, s = token - b * S;
  const float g = pad_gain(ln_pad[b], lse[(b * H + head) * S + s]);
  float x[8];
  unpack8(ld16(out + row * kCsHd + 8 * lane), x);
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] *= g;
  st16(y + row * kCsHd + 8 * lane, pack8(x));
}

__global__ __launch_bounds__(256) void ctx_scale_bwd_kernel(
    const bf16* __restrict__ out, const float* __restrict__ lse, const float* __restrict__ ln_pad,
    const bf16* __restrict__ dy, bf16* __restrict__ dout, float* __restrict__ dlse, int64_t nrow,
    int64_t S, int H) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row = gid >> 4;
  if (row >= nrow) return;
  const int lane = (int)(gid & 15);
  const int64_t token = row / H;
  const int head = (int)(row - token * H);
  const int64_t b = token / S, s = token - b * S;
  const int64_t li = (b * H + head) * S + s;
  const float g = pad_gain(ln_pad[b], lse[li]);
  float x[8], d[8];
  unpack8(ld16(out + row * kCsHd + 8 * lane), x);
  unpack8(ld16(dy + row * kCsHd + 8 * lane), d);
  float dot = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    dot += d[i] * x[i];
    d[i] *= g;
  }
  st16(dout + row * kCsHd + 8 * lane, pack8(d));
  dot = group_sum<16>(dot);
  if (lane == 0) dlse[li] = dot * g * (1.0f - g);
}

}  // namespace aa

using namespace aa;

static int ctx_check(const void* out, const float* lse, const float* ln_pad, const void* y,
                     int64_t B, int64_t S, int64_t H, int64_t hd, int dtype) {
  if (dtype != AA_DTYPE_BF16) return fail(AA_EUNSUPPORTED, "only bf16 activations are implemented");
  if (hd != kCsHd) return fail(AA_EUNSUPPORTED, "head_dim must be 128");
  if (B < 0 || S < 0 || H <= 0) return fail(AA_EINVAL, "bad B/S/H");
  if (B * S == 0) return AA_OK;
  if (!out || !lse || !ln_pad || !y) return fail(AA_EINVAL, "ctx_scale: null pointer");
  if (!aligned16(out) || !aligned16(y)) return fail(AA_EINVAL, "ctx_scale: misaligned pointer");
  return AA_OK;
}

extern "C" int aa_ctx_scale_fwd(const void* out, const float* lse, const float* ln_pad, void* y,
                                int64_t B, int64_t S, int64_t H, int64_t hd, int dtype,
                                void* stream) {
  clear_error();
  if (int rc = ctx_check(out, lse, ln_pad, y, B, S, H, hd, dtype)) return rc;
  const int64_t nrow = B * S * H;
  if (nrow == 0) return AA_OK;
  ctx_scale_fwd_kernel<<<dim3((unsigned)((nrow * 16 + 255) / 256)), 256, 0,
                         (hipStream_t)stream>>>((const bf16*)out, lse, ln_pad, (bf16*)y, nrow, S,
                                                (int)H);
  return check_launch("ctx_scale_fwd");
}

extern "C" int aa_ctx_scale_bwd(const void* out, const float* lse, const float* ln_pad,
                                const void* dy, void* dout, float* dlse, int64_t B, int64_t S,
                                int64_t H, int64_t hd, int dtype, void* stream) {
  clear_error();
  if (int rc = ctx_check(out, lse, ln_pad, dout, B, S, H, hd, dtype)) return rc;
  const int64_t nrow = B * S * H;
  if (nrow == 0) return AA_OK;
  if (!dy || !dlse) return fail(AA_EINVAL, "ctx_scale_bwd: null pointer");
  if (!aligned16(dy)) return fail(AA_EINVAL, "ctx_scale_bwd: misaligned pointer");
  ctx_scale_bwd_kernel<<<dim3((unsigned)((nrow * 16 + 255) / 256)), 256, 0,
                         (hipStream_t)stream>>>((const bf16*)out, lse, ln_pad, (const bf16*)dy,
                                                (bf16*)dout, dlse, nrow, S, (int)H);
  return check_launch("ctx_scale_bwd");
}
