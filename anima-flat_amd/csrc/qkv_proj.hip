// Fused QKV projection + QK-RMSNorm + rotate-half RoPE: q, k, v straight
// from the hidden states and the projection weight, one launch.
//
// The reference computes qkv = hid @ W^T (nn.Linear without bias, bf16 out,
// src/model.py:134,308-316) and then qkv_norm_rope on it (rope.py:616-645),
// a 3 * H * 128 * 2-byte round trip per token through HBM between the two.
// Here the projection's output tile never leaves the chip:
//
//   out tile = 256 tokens x 128 columns = one (q | k | v, head) section of 256
//   tokens; acc = X[256 x K] . W[128 x K]^T in fp32 on v_mfma_f32_32x32x16_bf16,
//   rounded to bf16 (the value the reference's GEMM writes), staged in LDS,
//   then per token RMSNorm + rotation (norm_rotate, the prologue's math) for
//   q and k, a copy for v, and 256-byte row stores into q, k, v [ntok, H, 128].
//
// Main loop: 8 waves, each a 64-token x 64-column block (2 x 2 accumulators),
// over K in stages of 64: the stage's X rows (256 x 128 B) and W rows
// (128 x 128 B) move HBM -> LDS by DMA (global_load_lds_dwordx4, no
// registers) into a 3-stage ring, two stages ahead, one barrier per stage.
// Tiles in LDS use the row-tile format of the attention kernels with 64-wide
// rows: element (r, k) at (r >> 4) * 1024 + (k >> 3) * 128 + (r & 15) * 8
// + (k & 7), so an operand read (16 lanes on one 16-byte chunk of 16
// consecutive rows) covers 256 contiguous bytes.
//
// Work order: workgroups go to XCDs in contiguous ranges (xcd_remap), and
// within the range in groups of 4 token tiles x all column tiles, so the 32
// workgroups an XCD runs at once share 4 X tiles and 8 W tiles in its L2.
#include "aa_common.h"
#include "norm_rope.h"
#include "tile_io.h"

namespace aa {

constexpr int kPM = 256;                        // tokens per workgroup
constexpr int kPN = 128;                        // output columns per workgroup (one section)
constexpr int kPK = 64;                         // K per stage
constexpr int kPStages = 3;
constexpr int kPThreads = 512;
constexpr int kPXElems = kPM * kPK;             // 32 KiB
constexpr int kPStageElems = kPXElems + kPN * kPK;  // + 16 KiB of W
constexpr int kPGroupM = 4;                     // token tiles per work-order group

struct ProjParams {
  const bf16* x;  // hidden states, row r at x + r * xs
  int64_t xs;
  const bf16* w;  // [3 H 128, K]
  bf16* q;        // [ntok, H, 128] each
  bf16* k;
  bf16* v;
  const float* qw;
  const float* kw;
  const float* cos;
  const float* sin;
  int64_t ntok;
  int64_t S;
  int H;
  int K;
  int mtiles;
  float eps;
};

// DMA of row group g (16 rows x 64 k) of a tile whose row 0 is at `base`
// (row stride rs elements, already offset to the stage's k): two 1 KiB
// blocks, chunks 0-3 and 4-7 of the same rows. Rows at or past `nrows` re-read
// row nrows - 1 (their results are not stored).
__device__ __forceinline__ void dma_proj_group(const bf16* base, int64_t rs, int nrows,
                                               bf16* tile, int g, int lane) {
  const int row = min(16 * g + (lane & 15), nrows - 1);
  const bf16* src = base + (int64_t)row * rs + 8 * (lane >> 4);
  bf16* dst = tile + g * 1024;
  dma16_off<0>(src, dst);
  dma16_off<64>(src, dst + 512);
}

__global__ __launch_bounds__(kPThreads) void qkv_proj_kernel(ProjParams p) {
  __shared__ __attribute__((aligned(16))) bf16 lds[kPStages * kPStageElems];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  // Tile of this workgroup.
  const int ntn = 3 * p.H;
  const int total = p.mtiles * ntn;
  const int L = xcd_remap(blockIdx.x, total);
  const int group = L / (kPGroupM * ntn);
  const int within = L - group * kPGroupM * ntn;
  const int gm = min(kPGroupM, p.mtiles - group * kPGroupM);
  const int mt = group * kPGroupM + within % gm;
  const int nt = within / gm;

  const int64_t row0 = (int64_t)mt * kPM;
  const int nrows = (int)min<int64_t>(kPM, p.ntok - row0);
  const bf16* xbase = p.x + row0 * p.xs;
  const bf16* wbase = p.w + (int64_t)nt * kPN * p.K;

  // Stage s -> ring slot s % 3; wave w moves X row groups 2w, 2w + 1 and W row group w.
  auto issue = [&](int s) {
    bf16* st = lds + (s % kPStages) * kPStageElems;
    const int k0 = s * kPK;
    dma_proj_group(xbase + k0, p.xs, nrows, st, 2 * wave, lane);
    dma_proj_group(xbase + k0, p.xs, nrows, st, 2 * wave + 1, lane);
    dma_proj_group(wbase + k0, p.K, kPN, st + kPXElems, wave, lane);
  };

  const int nk = p.K / kPK;
  issue(0);
  if (nk > 1) issue(1);

  const int wm = wave & 3;   // tokens 64 wm .. 64 wm + 63
  const int wn = wave >> 2;  // columns 64 wn .. 64 wn + 63
  const int li = lane & 31;
  const int hh = lane >> 5;
  // Row 32 t + li of a 64-row block, chunk 2 kk + hh: rd + 2048 t + 256 kk.
  const int rd = (li >> 4) * 1024 + (li & 15) * 8 + hh * 128;

  f32x16 acc[2][2];
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[c][t][e] = 0.f;

  for (int s = 0; s < nk; ++s) {
    // This wave's DMAs of stage s are done once at most the 6 of stage s + 1
    // are outstanding; the barrier then publishes every wave's and retires
    // all reads of stage s - 1, whose slot the DMA of stage s + 2 reuses.
    if (s + 1 < nk) {
      asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();
    if (s + 2 < nk) issue(s + 2);
    const bf16* xs = lds + (s % kPStages) * kPStageElems + wm * 4096 + rd;
    const bf16* ws = lds + (s % kPStages) * kPStageElems + kPXElems + wn * 4096 + rd;
#pragma unroll
    for (int kk = 0; kk < kPK / 16; ++kk) {
      const bf16x8 a0 = *reinterpret_cast<const bf16x8*>(ws + 256 * kk);
      const bf16x8 a1 = *reinterpret_cast<const bf16x8*>(ws + 2048 + 256 * kk);
      const bf16x8 b0 = *reinterpret_cast<const bf16x8*>(xs + 256 * kk);
      const bf16x8 b1 = *reinterpret_cast<const bf16x8*>(xs + 2048 + 256 * kk);
      acc[0][0] = mfma32(a0, b0, acc[0][0]);
      acc[0][1] = mfma32(a0, b1, acc[0][1]);
      acc[1][0] = mfma32(a1, b0, acc[1][0]);
      acc[1][1] = mfma32(a1, b1, acc[1][1]);
    }
  }
  __syncthreads();  // every wave is done with the ring: reuse it as the output tile

  // acc[c][t] holds out^T: lane li is token 64 wm + 32 t + li, element e is
  // column 64 wn + 32 c + 8 (e / 4) + 4 hh + (e % 4). Staged as bf16 rows of
  // 128 columns, 16-byte chunk ch of row r at r * 128 + ((ch ^ (r & 15)) * 8).
  bf16* tile = lds;
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int r = 64 * wm + 32 * t + li;
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const int ch = 8 * wn + 4 * c + e4;
        u32x2 w2;
        w2[0] = pack_bf16(acc[c][t][4 * e4], acc[c][t][4 * e4 + 1]);
        w2[1] = pack_bf16(acc[c][t][4 * e4 + 2], acc[c][t][4 * e4 + 3]);
        *reinterpret_cast<u32x2*>(tile + r * 128 + ((ch ^ (r & 15)) * 8) + 4 * hh) = w2;
      }
    }
  __syncthreads();

  // Per token: the section's RMSNorm + rotation (q, k) or a copy (v), 8 lanes
  // per token, two 16-byte chunks per lane, 256-byte rows out.
  const int j = tid & 7;
  const int grp = tid >> 3;
  const int seg = nt / p.H;
  const int head = nt - seg * p.H;
  bf16* out = seg == 0 ? p.q : (seg == 1 ? p.k : p.v);
  const float* nw = seg == 0 ? p.qw : p.kw;
  for (int r = grp; r < nrows; r += kPThreads / 8) {
    const u32x4 ra = *reinterpret_cast<const u32x4*>(tile + r * 128 + ((j ^ (r & 15)) * 8));
    const u32x4 rb =
        *reinterpret_cast<const u32x4*>(tile + r * 128 + (((8 + j) ^ (r & 15)) * 8));
    const int64_t token = row0 + r;
    bf16* dst = out + (token * p.H + head) * kHd;
    if (seg == 2) {
      st16(dst + 8 * j, ra);
      st16(dst + kHalf + 8 * j, rb);
    } else {
      Section x;
      unpack8(ra, x.a);
      unpack8(rb, x.b);
      float oa[8], ob[8];
      norm_rotate<true>(x, nw, p.cos, p.sin, token % p.S, j, p.eps, oa, ob);
      st16(dst + 8 * j, pack8(oa));
      st16(dst + kHalf + 8 * j, pack8(ob));
    }
  }
}

}  // namespace aa

using namespace aa;

extern "C" int aa_qkv_proj_norm_rope(const void* hid, int64_t hid_row_stride, const void* weight,
                                     void* q, void* k, void* v, const float* q_weight,
                                     const float* k_weight, const float* cos, const float* sin,
                                     int64_t B, int64_t S, int64_t H, int64_t hd, float eps,
                                     int dtype, void* stream) {
  clear_error();
  if (dtype != AA_DTYPE_BF16) return fail(AA_EUNSUPPORTED, "only bf16 activations are implemented");
  if (hd != kHd) return fail(AA_EUNSUPPORTED, "head_dim must be 128");
  if (B < 0 || S < 0 || H <= 0 || H > 64) return fail(AA_EINVAL, "qkv_proj: bad B/S/H (H <= 64)");
  const int64_t K = H * kHd;
  if (B * S == 0) return AA_OK;
  if (!hid || !weight || !q || !k || !v || !q_weight || !k_weight || !cos || !sin)
    return fail(AA_EINVAL, "qkv_proj: null pointer");
  if (hid_row_stride < K || hid_row_stride % 8 != 0)
    return fail(AA_EINVAL, "qkv_proj: hidden row stride must be >= H*128 and a multiple of 8");
  if (!aligned16(hid) || !aligned16(weight) || !aligned16(q) || !aligned16(k) || !aligned16(v) ||
      !aligned16(q_weight) || !aligned16(k_weight) || !aligned16(cos) || !aligned16(sin))
    return fail(AA_EINVAL, "qkv_proj: pointers must be 16-byte aligned");
  const int64_t ntok = B * S;
  const int64_t mtiles = (ntok + kPM - 1) / kPM;
  const int64_t total = mtiles * 3 * H;
  if (total > 0x7fffffff) return fail(AA_EUNSUPPORTED, "qkv_proj: too many tokens");
  ProjParams p;
  p.x = (const bf16*)hid;
  p.xs = hid_row_stride;
  p.w = (const bf16*)weight;
  p.q = (bf16*)q;
  p.k = (bf16*)k;
  p.v = (bf16*)v;
  p.qw = q_weight;
  p.kw = k_weight;
  p.cos = cos;
  p.sin = sin;
  p.ntok = ntok;
  p.S = S;
  p.H = (int)H;
  p.K = (int)K;
  p.mtiles = (int)mtiles;
  p.eps = eps;
  qkv_proj_kernel<<<dim3((unsigned)total), kPThreads, 0, (hipStream_t)stream>>>(p);
  return check_launch("qkv_proj_norm_rope");
}
