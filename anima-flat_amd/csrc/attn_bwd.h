// Shared by the backward's kernels (attn_bwd.hip: dq_kernel, the two-role
// dkdv_kernel and the query-split combine pass; attn_bwd_dkdv.hip: the
// one-wave-per-SIMD dK/dV kernel): the launch parameters, the stats record
// that dq_kernel writes for the dK/dV kernels, and the layout of the dK/dV
// query-split partials that dkdv_combine_kernel sums.
#pragma once

#include "tile_io.h"

namespace aa {
namespace bwd {

constexpr int kD = 128;
constexpr int kT = kTileRows;  // rows (queries or keys) per streamed tile
constexpr int kStat = 256;     // floats per 64-query stats record: lse2[64], -D[64], zero pad
constexpr int kKeysPerWg = 128;  // keys per dK/dV workgroup (both kernels)
// Partial records per dK/dV workgroup in query-split mode: record w < 4 holds
// dV^T and record 4 + w holds dK^T of keys 32 w .. 32 w + 31 of the block;
// float4 j (0..15) of lane l of record r is at ((r * 16 + j) * 64 + l).
constexpr int kDkParts = 8;

struct Params {
  const bf16* dout;
  const bf16* q;
  const bf16* k;
  const bf16* v;
  const bf16* o;
  const float* lse;
  bf16* dq;
  bf16* dk;
  bf16* dv;
  int64_t s_do[3], s_q[3], s_k[3], s_v[3], s_o[3], s_dq[3], s_dk[3], s_dv[3];
  float* stats;  // [B][H][ntq][kStat]
  // Query split of the dK/dV kernels (see dkdv_split): with nsplit > 1,
  // workgroup (split, b, h, key block) covers query tiles split * ceil(ntq /
  // nsplit) .. and writes its fp32 dV^T / dK^T accumulators to part (layout
  // above), which the combine pass sums in a fixed order.
  float* part;
  int nsplit;
  int H, Sq, Sk, ntq, ntk;
  float c;      // scale * log2(e)
  float scale;  // softmax scale
};

// Launches the one-wave-per-SIMD dK/dV kernel of attn_bwd_dkdv.hip over
// `total` workgroups (nkblk key blocks per (batch, head), times nsplit).
void launch_dkdv1w(const Params& p, int nkblk, int total, hipStream_t stream);

}  // namespace bwd
}  // namespace aa
