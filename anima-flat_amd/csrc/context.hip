// On-device length bookkeeping of a zero-padded text context.
//
// For ctx [B, S, C] the length of item b is the 1-based index of its last row
// with any non-zero element (at least 1); seqused[b] = length (int32) and
// ln_pad[b] = log(S - length) (-inf when nothing is padded). Zero means +0 or
// -0; NaN counts as non-zero. The test is on the bits, so it serves 2-byte
// (bf16, fp16) and 4-byte (fp32) elements alike: magnitude bits 0x7fff or
// 0x7fffffff.
//
// Two launches, no atomics and no host read: ctx_rows_kernel writes, per
// (item, 32-row chunk), the largest 1-based index of a non-zero row (0 if
// none) into the workspace; ctx_len_finalize_kernel takes the maximum over an
// item's chunks. Each wave checks 8 rows, a row at a time with all 64 lanes
// reading 16 bytes each (1 KB per load instruction).
#include <cmath>

#include "aa_common.h"

namespace aa {

constexpr int kCtxRowsPerBlock = 32;  // 4 waves x 8 rows

__global__ __launch_bounds__(256) void ctx_rows_kernel(const uint8_t* __restrict__ ctx,
                                                       int64_t S, int64_t row_bytes,
                                                       int64_t stride_b, int64_t stride_s,
                                                       int elem_bytes, int nchunk,
                                                       int32_t* __restrict__ ws) {
  __shared__ int best[4];
  const int chunk = blockIdx.x, b = blockIdx.y;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint32_t mask = elem_bytes == 2 ? 0x7fff7fffu : 0x7fffffffu;
  int last = 0;
  for (int i = 0; i < 8; ++i) {
    const int64_t s = (int64_t)chunk * kCtxRowsPerBlock + wave * 8 + i;
    if (s >= S) break;
    const uint8_t* row = ctx + b * stride_b + s * stride_s;
    uint32_t any = 0;
    for (int64_t off = 16 * lane; off < row_bytes; off += 1024) {
      const u32x4 w = ld16(row + off);
      any |= (w[0] & mask) | (w[1] & mask) | (w[2] & mask) | (w[3] & mask);
    }
    if (__builtin_amdgcn_ballot_w64(any != 0)) last = (int)(s + 1);
  }
  if (lane == 0) best[wave] = last;
  __syncthreads();
  if (threadIdx.x == 0)
    ws[(int64_t)b * nchunk + chunk] = max(max(best[0], best[1]), max(best[2], best[3]));
}

__global__ __launch_bounds__(256) void ctx_len_finalize_kernel(const int32_t* __restrict__ ws,
                                                               int nchunk, int64_t B, int64_t S,
                                                               int32_t* __restrict__ seqused,
                                                               float* __restrict__ ln_pad) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  int len = 1;
  for (int c = 0; c < nchunk; ++c) len = max(len, (int)ws[b * nchunk + c]);
  seqused[b] = len;
  ln_pad[b] = logf((float)(S - len));
}

}  // namespace aa

using namespace aa;

static int ctx_chunks(int64_t S) { return (int)((S + kCtxRowsPerBlock - 1) / kCtxRowsPerBlock); }

extern "C" size_t aa_context_lengths_workspace(int64_t B, int64_t S) {
  if (B <= 0 || S <= 0) return 0;
  return (size_t)B * ctx_chunks(S) * sizeof(int32_t);
}

extern "C" int aa_context_lengths(const void* ctx, int64_t B, int64_t S, int64_t C,
                                  int64_t stride_b, int64_t stride_s, int elem_bytes,
                                  int32_t* seqused, float* ln_pad, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  clear_error();
  if (B < 0 || S <= 0 || C <= 0) return fail(AA_EINVAL, "context_lengths: bad B/S/C");
  if (B == 0) return AA_OK;
  if (B > 65535 || S > (1 << 30)) return fail(AA_EUNSUPPORTED, "context_lengths: size out of range");
  if (elem_bytes != 2 && elem_bytes != 4)
    return fail(AA_EUNSUPPORTED, "context_lengths: elements must be 2 or 4 bytes");
  if (!ctx || !seqused || !ln_pad) return fail(AA_EINVAL, "context_lengths: null pointer");
  const int64_t row_bytes = C * elem_bytes;
  if (!aligned16(ctx) || row_bytes % 16 != 0 || (stride_b * elem_bytes) % 16 != 0 ||
      (stride_s * elem_bytes) % 16 != 0)
    return fail(AA_EINVAL,
                "context_lengths: rows must be 16-byte aligned and a multiple of 16 bytes long");
  if (stride_b < 0 || stride_s < 0) return fail(AA_EINVAL, "context_lengths: negative stride");
  if (!workspace || workspace_bytes < aa_context_lengths_workspace(B, S))
    return fail(AA_EINVAL, "context_lengths: workspace too small (aa_context_lengths_workspace)");
  hipStream_t st = (hipStream_t)stream;
  const int nchunk = ctx_chunks(S);
  ctx_rows_kernel<<<dim3((unsigned)nchunk, (unsigned)B), 256, 0, st>>>(
      (const uint8_t*)ctx, S, row_bytes, stride_b * elem_bytes, stride_s * elem_bytes, elem_bytes,
      nchunk, (int32_t*)workspace);
  if (int rc = check_launch("context_lengths")) return rc;
  ctx_len_finalize_kernel<<<dim3((unsigned)((B + 255) / 256)), 256, 0, st>>>(
      (const int32_t*)workspace, nchunk, B, S, seqused, ln_pad);
  return check_launch("context_lengths finalize");
}
