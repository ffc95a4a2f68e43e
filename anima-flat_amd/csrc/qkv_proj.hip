// Fused QKV projection + QK-RMSNorm + rotate-half RoPE: q, k, v straight
// from the hidden states and the projection weight, one launch.
//
// The reference computes qkv = hid @ W^T (nn.Linear without bias, bf16 out,
// src/model.py:134,308-316) and then qkv_norm_rope on it (rope.py:616-645),
// a 3 * H * 128 * 2-byte round trip per token through HBM between the two.
// Here the projection's output tile never leaves the chip:
//
//   out tile = 256 tokens x 256 columns = two (q | k | v, head) sections of
//   256 tokens; acc = X[256 x K] . W[256 x K]^T in fp32 on
//   v_mfma_f32_32x32x16_bf16, rounded to bf16 (the value the reference's GEMM
//   writes), staged in LDS, then per token RMSNorm + rotation (norm_rotate,
//   the prologue's math) for q and k, a copy for v, and 256-byte row stores
//   into q, k, v [ntok, H, 128].
//
// Main loop: 8 waves, each 64 tokens x one 128-column section (2 x 4
// accumulators: 6 operand reads per 8 MFMAs), over K in stages of 32: the
// stage's X and W rows (2 x 256 x 64 B) move HBM -> LDS by DMA
// (global_load_lds_dwordx4, no registers) into a 4-stage ring, three stages
// ahead, one barrier per stage. Tiles in LDS use the row-tile format of the
// attention kernels with 32-wide rows: element (r, k) at (r >> 4) * 512
// + (k >> 3) * 128 + (r & 15) * 8 + (k & 7), so an operand read (16 lanes on
// one 16-byte chunk of 16 consecutive rows) covers 256 contiguous bytes and
// one DMA instruction fills one 16-row group.
//
// Work order: workgroups go to XCDs in contiguous ranges (xcd_remap), and
// within the range in groups of 4 token tiles x all column tiles, so the 32
// workgroups an XCD runs at once share 4 X tiles and 8 W tiles in its L2.
// With an odd number of sections (3 H) the last column tile holds one.
#include <string>

#include "aa_common.h"
#include "norm_rope.h"
#include "tile_io.h"

namespace aa {

constexpr int kPM = 256;                            // tokens per workgroup
constexpr int kPN = 256;                            // output columns: two sections
constexpr int kPK = 32;                             // K per stage
constexpr int kPStages = 4;
constexpr int kPThreads = 512;
constexpr int kPXElems = kPM * kPK;                 // 16 KiB
constexpr int kPStageElems = kPXElems + kPN * kPK;  // + 16 KiB of W
constexpr int kPGroupM = 4;                         // token tiles per work-order group

// The projection's output columns are nseg segments of H sections of 128:
// segment g goes to out[g] ([ntok, H, 128]), RMS-normalised with weight nw[g]
// (then rotated when rope[g]) or copied when nw[g] is null.
//   qkv + prologue (model.py:308-316): q (norm, rope), k (norm, rope), v (copy)
//   xq + head_norm (model.py:324):     q (norm)
//   xkv + k-norm (model.py:256-258):   k (norm), v (copy)
struct ProjParams {
  const bf16* x;  // input rows, row r at x + r * xs
  int64_t xs;
  const bf16* w;  // [nseg H 128, K]
  bf16* out[3];
  const float* nw[3];
  int rope[3];
  int nseg;
  const float* cos;
  const float* sin;
  int64_t ntok;
  int64_t S;
  int H;
  int K;
  int mtiles;
  float eps;
};

// DMA of row group g (16 rows x 32 k, 1 KiB) of a tile whose row 0 is at
// `base` (row stride rs elements, already offset to the stage's k): lane
// moves chunk lane >> 4 of row 16 g + (lane & 15). Rows at or past `nrows`
// re-read row nrows - 1 (their results are not stored).
__device__ __forceinline__ void dma_proj_group(const bf16* base, int64_t rs, int nrows,
                                               bf16* tile, int g, int lane) {
  const int row = min(16 * g + (lane & 15), nrows - 1);
  dma16_off<0>(base + (int64_t)row * rs + 8 * (lane >> 4), tile + g * 512);
}

__global__ __launch_bounds__(kPThreads) void qkv_proj_kernel(ProjParams p) {
  __shared__ __attribute__((aligned(16))) bf16 lds[kPStages * kPStageElems];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  // Tile of this workgroup: token tile mt, sections 2 nt and 2 nt + 1.
  const int nsec = p.nseg * p.H;
  const int ntn = (nsec + 1) / 2;
  const int total = p.mtiles * ntn;
  const int L = xcd_remap(blockIdx.x, total);
  const int group = L / (kPGroupM * ntn);
  const int within = L - group * kPGroupM * ntn;
  const int gm = min(kPGroupM, p.mtiles - group * kPGroupM);
  const int mt = group * kPGroupM + within % gm;
  const int nt = within / gm;

  const int64_t row0 = (int64_t)mt * kPM;
  const int nrows = (int)min<int64_t>(kPM, p.ntok - row0);
  const int ncols = min(kPN, (nsec - 2 * nt) * kHd);
  const bf16* xbase = p.x + row0 * p.xs;
  const bf16* wbase = p.w + (int64_t)nt * kPN * p.K;

  // Stage s -> ring slot s % 4; wave w moves X and W row groups 2w, 2w + 1.
  auto issue = [&](int s) {
    bf16* st = lds + (s % kPStages) * kPStageElems;
    const int k0 = s * kPK;
    dma_proj_group(xbase + k0, p.xs, nrows, st, 2 * wave, lane);
    dma_proj_group(xbase + k0, p.xs, nrows, st, 2 * wave + 1, lane);
    dma_proj_group(wbase + k0, p.K, ncols, st + kPXElems, 2 * wave, lane);
    dma_proj_group(wbase + k0, p.K, ncols, st + kPXElems, 2 * wave + 1, lane);
  };

  const int nk = p.K / kPK;
  issue(0);
  if (nk > 1) issue(1);
  if (nk > 2) issue(2);

  const int wm = wave & 3;   // tokens 64 wm .. 64 wm + 63
  const int wn = wave >> 2;  // section 2 nt + wn: columns 128 wn .. 128 wn + 127
  const int li = lane & 31;
  const int hh = lane >> 5;
  // Row 32 t + li of a row block, chunk 2 kk + hh: rd + 1024 t + 256 kk.
  const int rd = (li >> 4) * 512 + (li & 15) * 8 + hh * 128;

  f32x16 acc[4][2];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[c][t][e] = 0.f;

  for (int s = 0; s < nk; ++s) {
    // This wave's DMAs of stage s are done once at most those of the stages
    // after it (4 each) are outstanding; the barrier then publishes every
    // wave's and retires all reads of stage s - 1, whose slot the DMA of
    // stage s + 3 reuses.
    if (s + 2 < nk) {
      asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    } else if (s + 1 < nk) {
      asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();
    if (s + 3 < nk) issue(s + 3);
    const bf16* xs = lds + (s % kPStages) * kPStageElems + wm * 2048 + rd;
    const bf16* ws = lds + (s % kPStages) * kPStageElems + kPXElems + wn * 4096 + rd;
#pragma unroll
    for (int kk = 0; kk < kPK / 16; ++kk) {
      bf16x8 a[4], b[2];
#pragma unroll
      for (int c = 0; c < 4; ++c) a[c] = *reinterpret_cast<const bf16x8*>(ws + 1024 * c + 256 * kk);
#pragma unroll
      for (int t = 0; t < 2; ++t) b[t] = *reinterpret_cast<const bf16x8*>(xs + 1024 * t + 256 * kk);
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int t = 0; t < 2; ++t) acc[c][t] = mfma32(a[c], b[t], acc[c][t]);
    }
  }
  __syncthreads();  // every wave is done with the ring: reuse it as the output tiles

  // acc[c][t] holds out^T: lane li is token 64 wm + 32 t + li, element e is
  // column 32 c + 8 (e / 4) + 4 hh + (e % 4) of section wn. Staged as bf16
  // rows of 128 columns per section, 16-byte chunk ch of row r at
  // r * 128 + ((ch ^ (r & 15)) * 8).
  bf16* mine = lds + wn * (kPM * kHd);
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int r = 64 * wm + 32 * t + li;
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const int ch = 4 * c + e4;
        u32x2 w2;
        w2[0] = pack_bf16(acc[c][t][4 * e4], acc[c][t][4 * e4 + 1]);
        w2[1] = pack_bf16(acc[c][t][4 * e4 + 2], acc[c][t][4 * e4 + 3]);
        *reinterpret_cast<u32x2*>(mine + r * 128 + ((ch ^ (r & 15)) * 8) + 4 * hh) = w2;
      }
    }
  __syncthreads();

  // Per (token, section): RMSNorm + rotation (q, k) or a copy (v), 8 lanes
  // per item, two 16-byte chunks per lane, 256-byte rows out.
  const int j = tid & 7;
  const int grp = tid >> 3;
  const int nmine = ncols / kHd;
  for (int sc = 0; sc < nmine; ++sc) {
    const int gsec = 2 * nt + sc;
    const int seg = gsec / p.H;
    const int head = gsec - seg * p.H;
    bf16* out = p.out[seg];
    const float* nw = p.nw[seg];
    const bool rope = p.rope[seg] != 0;
    const bf16* tile = lds + sc * (kPM * kHd);
    for (int r = grp; r < nrows; r += kPThreads / 8) {
      const u32x4 ra = *reinterpret_cast<const u32x4*>(tile + r * 128 + ((j ^ (r & 15)) * 8));
      const u32x4 rb =
          *reinterpret_cast<const u32x4*>(tile + r * 128 + (((8 + j) ^ (r & 15)) * 8));
      const int64_t token = row0 + r;
      bf16* dst = out + (token * p.H + head) * kHd;
      if (!nw) {
        st16_nt(dst + 8 * j, ra);
        st16_nt(dst + kHalf + 8 * j, rb);
      } else {
        Section x;
        unpack8(ra, x.a);
        unpack8(rb, x.b);
        float oa[8], ob[8];
        if (rope) norm_rotate<true>(x, nw, p.cos, p.sin, token % p.S, j, p.eps, oa, ob);
        else norm_rotate<false>(x, nw, nullptr, nullptr, 0, j, p.eps, oa, ob);
        st16_nt(dst + 8 * j, pack8(oa));
        st16_nt(dst + kHalf + 8 * j, pack8(ob));
      }
    }
  }
}

}  // namespace aa

using namespace aa;

// Validates and launches one fused projection (nseg segments of H sections).
// What the epilogue does with one output segment.
enum SegMode { kCopy = 0, kNorm = 1, kNormRope = 2 };

static int launch_proj(const char* what, const void* hid, int64_t hid_row_stride, const void* weight,
                       int64_t K, int nseg, void* const* outs, const float* const* nws,
                       const int* modes, const float* cos, const float* sin, int64_t B, int64_t S,
                       int64_t H, int64_t hd, float eps, int dtype, hipStream_t st) {
  const std::string w = what;
  if (hd != kHd) return fail(AA_EUNSUPPORTED, "head_dim must be 128");
  if (dtype != AA_DTYPE_BF16) return fail(AA_EUNSUPPORTED, "only bf16 activations are implemented");
  if (B < 0 || S < 0 || H <= 0 || H > 64) return fail(AA_EINVAL, w + ": bad B/S/H (H <= 64)");
  if (K <= 0 || K % kPK != 0 || K > (1 << 20))
    return fail(AA_EUNSUPPORTED, w + ": the input width must be a positive multiple of 32");
  if (B * S == 0) return AA_OK;
  if (!hid || !weight) return fail(AA_EINVAL, w + ": null pointer");
  bool any_rope = false;
  for (int g = 0; g < nseg; ++g) {
    if (!outs[g] || (modes[g] != kCopy && !nws[g])) return fail(AA_EINVAL, w + ": null pointer");
    if (!aligned16(outs[g]) || (modes[g] != kCopy && !aligned16(nws[g])))
      return fail(AA_EINVAL, w + ": pointers must be 16-byte aligned");
    any_rope = any_rope || modes[g] == kNormRope;
  }
  if (any_rope && (!cos || !sin)) return fail(AA_EINVAL, w + ": null pointer");
  if (any_rope && (!aligned16(cos) || !aligned16(sin)))
    return fail(AA_EINVAL, w + ": pointers must be 16-byte aligned");
  if (hid_row_stride < K || hid_row_stride % 8 != 0)
    return fail(AA_EINVAL, w + ": input row stride must be >= the input width and a multiple of 8");
  if (!aligned16(hid) || !aligned16(weight))
    return fail(AA_EINVAL, w + ": pointers must be 16-byte aligned");
  const int64_t ntok = B * S;
  const int64_t mtiles = (ntok + kPM - 1) / kPM;
  const int64_t total = mtiles * ((nseg * H + 1) / 2);
  if (total > 0x7fffffff) return fail(AA_EUNSUPPORTED, w + ": too many tokens");
  ProjParams p;
  p.x = (const bf16*)hid;
  p.xs = hid_row_stride;
  p.w = (const bf16*)weight;
  for (int g = 0; g < 3; ++g) {
    p.out[g] = g < nseg ? (bf16*)outs[g] : nullptr;
    p.nw[g] = g < nseg && modes[g] != kCopy ? nws[g] : nullptr;
    p.rope[g] = g < nseg && modes[g] == kNormRope;
  }
  p.nseg = nseg;
  p.cos = cos;
  p.sin = sin;
  p.ntok = ntok;
  p.S = S;
  p.H = (int)H;
  p.K = (int)K;
  p.mtiles = (int)mtiles;
  p.eps = eps;
  qkv_proj_kernel<<<dim3((unsigned)total), kPThreads, 0, st>>>(p);
  return check_launch(what);
}

extern "C" int aa_qkv_proj_norm_rope(const void* hid, int64_t hid_row_stride, const void* weight,
                                     void* q, void* k, void* v, const float* q_weight,
                                     const float* k_weight, const float* cos, const float* sin,
                                     int64_t B, int64_t S, int64_t H, int64_t hd, float eps,
                                     int dtype, void* stream) {
  clear_error();
  void* outs[3] = {q, k, v};
  const float* nws[3] = {q_weight, k_weight, nullptr};
  const int modes[3] = {kNormRope, kNormRope, kCopy};
  return launch_proj("qkv_proj", hid, hid_row_stride, weight, H * hd, 3, outs, nws, modes, cos,
                     sin, B, S, H, hd, eps, dtype, (hipStream_t)stream);
}

extern "C" int aa_proj_head_norm(const void* x, int64_t x_row_stride, const void* weight,
                                 int64_t K, void* y, const float* norm_weight, int64_t B,
                                 int64_t S, int64_t H, int64_t hd, float eps, int dtype,
                                 void* stream) {
  clear_error();
  void* outs[1] = {y};
  const float* nws[1] = {norm_weight};
  const int modes[1] = {kNorm};
  return launch_proj("proj_head_norm", x, x_row_stride, weight, K, 1, outs, nws, modes, nullptr,
                     nullptr, B, S, H, hd, eps, dtype, (hipStream_t)stream);
}

extern "C" int aa_kv_proj_norm(const void* ctx, int64_t ctx_row_stride, const void* weight,
                               int64_t K, void* k, void* v, const float* k_weight, int64_t B,
                               int64_t S, int64_t H, int64_t hd, float eps, int dtype,
                               void* stream) {
  clear_error();
  void* outs[2] = {k, v};
  const float* nws[2] = {k_weight, nullptr};
  const int modes[2] = {kNorm, kCopy};
  return launch_proj("kv_proj_norm", ctx, ctx_row_stride, weight, K, 2, outs, nws, modes, nullptr,
                     nullptr, B, S, H, hd, eps, dtype, (hipStream_t)stream);
}
