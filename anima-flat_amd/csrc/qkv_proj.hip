// Fused input projections of the attention block: a bf16 GEMM whose output
// tile is normalised (and rotated) on chip before it is stored.
//
// The reference computes the projection with nn.Linear (no bias, bf16 out)
// and then normalises it in a second kernel, a round trip of the projection
// output through HBM:
//   qkv = b.qkv(hid); q, k, v = qkv_norm_rope(qkv, ...)   (src/model.py:308-316)
//   q = head_norm(b.xq(hid), ...)                          (src/model.py:324)
//   k, v = b.xkv(ctx).unbind(...); k = F.rms_norm(k, ...)  (src/model.py:256-258)
// Here acc = X[MT x K] . W[NS 128 x K]^T in fp32 on v_mfma_f32_32x32x16_bf16,
// rounded to bf16 (the value the reference's GEMM writes), staged in LDS, then
// per token and 128-column section: RMSNorm (+ rotate-half RoPE) with the
// prologue's math (norm_rotate) or a copy, and 256-byte row stores.
//
// Main loop: waves of 64 tokens x WN columns (2 x WN/32 accumulators), over K
// in stages of 64: the stage's X and W rows move L2 -> LDS by DMA
// (global_load_lds_dwordx4, no registers) into a ring of two stages, one
// ahead (each wave's share issued over the first k-steps of the stage before),
// one barrier per stage. Each DMA instruction moves 8 rows x 128 bytes,
// whole cache lines: with 16 rows x 64 bytes (half lines) per instruction the
// same loads stream at well under half the rate, which bounded this kernel.
// A stage in LDS is blocks of 8 rows x 64 k (1 KiB, one DMA instruction);
// element (r, k) at (r >> 3) * 512 + (r & 7) * 64 + ((k >> 3) ^ f(r)) * 8
// + (k & 7) with f(r) = (r & 7) ^ ((r >> 3) & 1). The XOR places the 16-byte
// chunk an operand read takes from 16 consecutive rows in 16 distinct
// (row parity, slot) pairs, i.e. 16 distinct bank groups: conflict-free.
//
// Tile shapes (ProjTile): 256 x 2 sections (8 waves of 64 x 128), 256 x 3
// sections (8 waves of 64 x 192: 8 operand reads per 12 MFMAs) and 128 x 1
// section (4 waves of 64 x 64, two workgroups per CU, for small token
// counts). The host picks the shape with the least work on the busiest CU
// (whole rounds of workgroups over the chip), so a projection fills the chip
// in whole rounds where it can. Every shape accumulates each output in the
// same order (16 k per MFMA, in increasing k), so all give identical bits.
//
// Work order: workgroups go to XCDs in contiguous ranges (xcd_remap), and
// within the range in groups of 4 token tiles x all column tiles, so the
// workgroups an XCD runs at once share a few X and W tiles in its L2. The
// last column tile may hold fewer sections.
#include <algorithm>
#include <cstdlib>
#include <string>
#include <type_traits>

#include "aa_common.h"
#include "norm_rope.h"
#include "tile_io.h"

namespace aa {

constexpr int kPK = 64;       // K per stage
constexpr int kPKMin = 32;    // K granularity: a last stage may hold 32
constexpr int kPGroupM = 4;   // token tiles per work-order group

template <int MT, int NS, int WN, int PS>
struct ProjTile {
  static constexpr int kMT = MT;                       // tokens per workgroup
  static constexpr int kNS = NS;                       // sections per workgroup
  static constexpr int kN = NS * kHd;                  // columns per workgroup
  static constexpr int kWN = WN;                       // columns per wave
  static constexpr int kWaves = (MT / 64) * (kN / WN);
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kXElems = MT * kPK;
  static constexpr int kStageElems = (MT + kN) * kPK;
  static constexpr int kBlocks = (MT + kN) / 8;        // 8-row DMA blocks per stage
  static constexpr int kBPW = kBlocks / kWaves;        // ... per wave
  static constexpr int kCB = WN / 32;                  // 32-column blocks per wave
  static constexpr int kRingElems = 2 * kStageElems;
  // The next stage's DMA of a wave goes out in this many parts, one per
  // k-step from the first: the load path takes one instruction per ~11
  // cycles, so 8 waves issuing 8-10 each at once hold most of them back from
  // their MFMAs for up to ~900 cycles. Two parts: QKV B=1 99.6 -> 95.5 us
  // (tile B), xq 64.7 -> 62.2 us (tile A); four parts were slower, and so was
  // splitting at all with four waves (tile C, whose two workgroups per CU
  // already overlap one's loads with the other's MFMAs).
  static constexpr int kDmaParts = kWaves == 8 ? 2 : 1;
  // Sections staged per epilogue pass (the ring holds the staged bf16 tiles).
  static constexpr int kPassSecs = PS;
  static_assert(MT % 64 == 0 && kN % WN == 0 && WN % 32 == 0, "wave tiling");
  static_assert(kBlocks % kWaves == 0 && kBPW % 2 == 0, "DMA blocks split evenly, in pairs");
  static_assert(PS >= 1 && PS <= NS && PS * MT * kHd <= kRingElems, "staging");
  static_assert(kRingElems * 2 <= 160 * 1024, "LDS");
};

// The last argument is the sections staged per epilogue pass. TileB stages
// one at a time: with two, a wave whose columns straddle the passes keeps
// 128 accumulators live through the first pass's normalisation and spills.
using TileA = ProjTile<256, 2, 128, 2>;  // 128 KiB ring
using TileB = ProjTile<256, 3, 192, 1>;  // 160 KiB ring
using TileC = ProjTile<128, 1, 64, 1>;   // 64 KiB ring, two workgroups per CU

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

template <class T>
__global__ __launch_bounds__(T::kThreads) void qkv_proj_kernel(ProjParams p) {
  __shared__ __attribute__((aligned(16))) bf16 lds[T::kRingElems];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // Tile of this workgroup: token tile mt, sections NS nt .. NS nt + NS - 1.
  const int nsec = p.nseg * p.H;
  const int ntn = (nsec + T::kNS - 1) / T::kNS;
  const int total = p.mtiles * ntn;
  const int L = xcd_remap(blockIdx.x, total);
  const int group = L / (kPGroupM * ntn);
  const int within = L - group * kPGroupM * ntn;
  const int gm = min(kPGroupM, p.mtiles - group * kPGroupM);
  const int mt = group * kPGroupM + within % gm;
  const int nt = within / gm;

  const int64_t row0 = (int64_t)mt * T::kMT;
  const int nrows = (int)min<int64_t>(T::kMT, p.ntok - row0);
  const int ncols = min(T::kN, (nsec - T::kNS * nt) * kHd);
  const bf16* xbase = p.x + row0 * p.xs;
  const bf16* wbase = p.w + (int64_t)nt * T::kN * p.K;

  // DMA lane roles: row (lane >> 3) of an 8-row block, LDS slot lane & 7,
  // which holds chunk slot ^ f(row); f's second term is the block's parity,
  // and a wave's blocks come in (even, odd) pairs.
  const int drow = lane >> 3;
  const int dchunk0 = (lane & 7) ^ drow;  // even blocks
  const int dchunk1 = dchunk0 ^ 1;        // odd blocks

  // Stage s -> ring slot s & 1: MT / 8 X blocks then kN / 8 W blocks,
  // contiguous (block b at b * 512); wave w moves blocks w G .. w G + G - 1.
  // A last stage of 32 k (K % 64 == 32) loads chunks 4..7 from chunks 0..3
  // (in bounds; those products are not computed).
  // Blocks lo .. hi - 1 of the wave's share of stage s.
  auto issue = [&](int s, int lo, int hi) {
    bf16* st = lds + (s & 1) * T::kStageElems;
    const int k0 = s * kPK;
    const int cmask = p.K - k0 >= kPK ? 7 : 3;
#pragma unroll
    for (int i = 0; i < T::kBPW; ++i) {
      if (i < lo || i >= hi) continue;
      // Wave-uniform: block b, its first row b0 (clamped), the source matrix.
      const int b = wave * T::kBPW + i;
      const bool is_x = b < T::kMT / 8;
      const int last = (is_x ? nrows : ncols) - 1;
      const int b0 = min(8 * (is_x ? b : b - T::kMT / 8), last);
      const int64_t rs = is_x ? p.xs : (int64_t)p.K;
      const bf16* sbase = (is_x ? xbase : wbase) + b0 * rs + k0;
      const uint32_t voff = (uint32_t)(min(drow, last - b0) * rs +
                                       8 * (((i & 1) ? dchunk1 : dchunk0) & cmask)) * 2;
      dma16_sv(sbase, voff, st + b * 512);
    }
  };

  const int nk = (p.K + kPK - 1) / kPK;
  const int nfull = p.K / kPK;  // stages of 64 k; a last one of 32 when K % 64 == 32
  issue(0, 0, T::kBPW);

  constexpr int kWavesM = T::kMT / 64;
  const int wm = wave % kWavesM;  // tokens 64 wm .. 64 wm + 63
  const int wn = wave / kWavesM;  // columns WN wn .. WN wn + WN - 1
  const int li = lane & 31;
  const int hh = lane >> 5;
  // Operand read of rows R + li (R a multiple of 32), k-step kk (16 k):
  // chunk 2 kk + hh of row li, at (R >> 3) * 512 + (kbase ^ 16 kk) with
  // kbase = (li >> 3) * 512 + (li & 7) * 64 + (hh ^ f(li)) * 8.
  const int kbase = (li >> 3) * 512 + (li & 7) * 64 + (hh ^ (li & 7) ^ ((li >> 3) & 1)) * 8;

  f32x16 acc[T::kCB][2];
#pragma unroll
  for (int c = 0; c < T::kCB; ++c)
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[c][t][e] = 0.f;

  // One stage of NSTEPS k-steps. Operands of kPre k-steps are read ahead of
  // their MFMAs: those of the first kPre steps before the next stage's DMA
  // starts going out (its asm is a compiler memory barrier, so they cannot
  // sink to their MFMAs), the rest kPre steps ahead. The DMA goes out in
  // kDmaParts parts, one at the start of each of the first k-steps. With 192
  // accumulator registers (kCB = 6) only one k-step's operands fit beside
  // them at two waves per SIMD.
  constexpr int kPre = T::kCB <= 4 ? 2 : 1;
  auto stage = [&](int s, auto nsteps) {
    constexpr int NSTEPS = decltype(nsteps)::value;
    // This wave's DMAs of stage s are done; the barrier publishes every
    // wave's and retires all reads of stage s - 1, whose slot stage s + 1
    // reuses.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    const bf16* stg = lds + (s & 1) * T::kStageElems;
    const bf16* xs = stg + wm * 4096;
    const bf16* ws = stg + T::kXElems + wn * (T::kWN / 8) * 512;
    bf16x8 a[NSTEPS][T::kCB], b[NSTEPS][2];
    auto read = [&](int kk) {
      const int ko = kbase ^ (16 * kk);
#pragma unroll
      for (int c = 0; c < T::kCB; ++c) a[kk][c] = *reinterpret_cast<const bf16x8*>(ws + 2048 * c + ko);
#pragma unroll
      for (int t = 0; t < 2; ++t) b[kk][t] = *reinterpret_cast<const bf16x8*>(xs + 2048 * t + ko);
    };
#pragma unroll
    for (int kk = 0; kk < kPre && kk < NSTEPS; ++kk) read(kk);
    constexpr int kParts = T::kDmaParts < NSTEPS ? T::kDmaParts : NSTEPS;
    auto part = [&](int j) {
      if (s + 1 < nk) issue(s + 1, j * T::kBPW / kParts, (j + 1) * T::kBPW / kParts);
    };
    part(0);
#pragma unroll
    for (int kk = 0; kk < NSTEPS; ++kk) {
      if (kk >= 1 && kk < kParts) part(kk);
      if constexpr (kPre > 1) {
        if (kk + kPre < NSTEPS) read(kk + kPre);
      }
#pragma unroll
      for (int c = 0; c < T::kCB; ++c)
#pragma unroll
        for (int t = 0; t < 2; ++t) acc[c][t] = mfma32(a[kk][c], b[kk][t], acc[c][t]);
      if constexpr (kPre == 1) {
        __builtin_amdgcn_sched_barrier(0);
        if (kk + 1 < NSTEPS) read(kk + 1);
      }
    }
  };
  for (int s = 0; s < nfull; ++s) stage(s, std::integral_constant<int, kPK / 16>{});
  if (nk > nfull) stage(nfull, std::integral_constant<int, kPKMin / 16>{});

  // acc[c][t] holds out^T: lane li is token 64 wm + 32 t + li, element e is
  // tile column WN wn + 32 c + 8 (e / 4) + 4 hh + (e % 4). Staged per pass of
  // kPassSecs sections as bf16 rows of 128 columns per section, 16-byte chunk
  // ch of row r at r * 128 + ((ch ^ (r & 15)) * 8).
  const int j = tid & 7;
  const int grp = tid >> 3;
  const int nmine = ncols / kHd;
#pragma unroll
  for (int p0 = 0; p0 < T::kNS; p0 += T::kPassSecs) {
    __syncthreads();  // the ring (or the previous pass's tiles) is free
#pragma unroll
    for (int c = 0; c < T::kCB; ++c) {
      const int col = T::kWN * wn + 32 * c;
      const int sec = col >> 7;
      if (sec < p0 || sec >= p0 + T::kPassSecs) continue;
      bf16* mine = lds + (sec - p0) * (T::kMT * kHd);
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int r = 64 * wm + 32 * t + li;
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
          const int ch = ((col & 127) >> 3) + e4;
          u32x2 w2;
          w2[0] = pack_bf16(acc[c][t][4 * e4], acc[c][t][4 * e4 + 1]);
          w2[1] = pack_bf16(acc[c][t][4 * e4 + 2], acc[c][t][4 * e4 + 3]);
          *reinterpret_cast<u32x2*>(mine + r * 128 + ((ch ^ (r & 15)) * 8) + 4 * hh) = w2;
        }
      }
    }
    __syncthreads();

    // Per (token, section): RMSNorm (+ rotation) or a copy, 8 lanes per item,
    // two 16-byte chunks per lane, 256-byte rows out.
    const int send = min(p0 + T::kPassSecs, nmine);
    for (int sc = p0; sc < send; ++sc) {
      const int gsec = T::kNS * nt + sc;
      const int seg = gsec / p.H;
      const int head = gsec - seg * p.H;
      bf16* out = p.out[seg];
      const float* nw = p.nw[seg];
      const bool rope = p.rope[seg] != 0;
      const bf16* tile = lds + (sc - p0) * (T::kMT * kHd);
      for (int r = grp; r < nrows; r += T::kThreads / 8) {
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
}

}  // namespace aa

using namespace aa;

// Validates and launches one fused projection (nseg segments of H sections).
// What the epilogue does with one output segment.
enum SegMode { kCopy = 0, kNorm = 1, kNormRope = 2 };

// Tile shape for ntok tokens x nsec sections: 0 = TileA, 1 = TileB, 2 =
// TileC, the one with the least time on the busiest CU: whole rounds of
// workgroups over the chip (TileC runs two per CU) times the time of one
// round. Round times measured on MI355X at K = 2048 (graph-timed): A 62-66 us,
// B 87-97 us, C 40 us (two workgroups) -> weights 1.93, 2.85, 2 x 0.62. With
// them the QKV projection at B = 2 takes two rounds of B (193.5 us) rather
// than three of A (198.3 us, A/B on one box). Ties go to the lower index. The environment variable AA_PROJ_TILE = a, b or c
// forces a shape (all give identical results); any other value is an error
// (-1).
static int pick_tile(int64_t ntok, int64_t nsec) {
  if (const char* e = std::getenv("AA_PROJ_TILE")) {
    if (e[0] && !e[1] && e[0] >= 'a' && e[0] <= 'c') return e[0] - 'a';
    return -1;
  }
  const int64_t cus = std::max(1, device_cu_count());
  struct Shape {
    int64_t mt, ns, per_cu;
    double weight;  // time of one round, per workgroup on a CU
  } shapes[3] = {{TileA::kMT, TileA::kNS, 1, 1.93},
                 {TileB::kMT, TileB::kNS, 1, 2.85},
                 {TileC::kMT, TileC::kNS, 2, 0.62}};
  int best = 0;
  double best_cost = 0;
  for (int i = 0; i < 3; ++i) {
    const Shape& sh = shapes[i];
    const int64_t wgs = (ntok + sh.mt - 1) / sh.mt * ((nsec + sh.ns - 1) / sh.ns);
    const int64_t slots = cus * sh.per_cu;
    const double cost = (double)((wgs + slots - 1) / slots) * sh.per_cu * sh.weight;
    if (i == 0 || cost < best_cost) {
      best = i;
      best_cost = cost;
    }
  }
  return best;
}

static int launch_proj(const char* what, const void* hid, int64_t hid_row_stride, const void* weight,
                       int64_t K, int nseg, void* const* outs, const float* const* nws,
                       const int* modes, const float* cos, const float* sin, int64_t B, int64_t S,
                       int64_t H, int64_t hd, float eps, int dtype, hipStream_t st) {
  const std::string w = what;
  if (hd != kHd) return fail(AA_EUNSUPPORTED, "head_dim must be 128");
  if (dtype != AA_DTYPE_BF16) return fail(AA_EUNSUPPORTED, "only bf16 activations are implemented");
  if (B < 0 || S < 0 || H <= 0 || H > 64) return fail(AA_EINVAL, w + ": bad B/S/H (H <= 64)");
  if (K <= 0 || K % kPKMin != 0 || K > (1 << 20))
    return fail(AA_EUNSUPPORTED, w + ": the input width must be a positive multiple of 32");
  if (B * S == 0) return AA_OK;
  // The DMA's per-lane byte offsets within an 8-row block are 32-bit:
  // 7 rows x stride x 2 bytes must stay below 2^32.
  if (hid_row_stride > (int64_t(1) << 27))
    return fail(AA_EUNSUPPORTED, w + ": input row stride must be at most 2^27 elements");
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
  const int tile = pick_tile(ntok, nseg * H);
  if (tile < 0) return fail(AA_EINVAL, "AA_PROJ_TILE must be a, b or c");
  const int64_t mt = tile == 2 ? TileC::kMT : TileA::kMT;
  const int ns = tile == 0 ? TileA::kNS : tile == 1 ? TileB::kNS : TileC::kNS;
  const int64_t mtiles = (ntok + mt - 1) / mt;
  const int64_t total = mtiles * ((nseg * H + ns - 1) / ns);
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
  if (tile == 0) qkv_proj_kernel<TileA><<<dim3((unsigned)total), TileA::kThreads, 0, st>>>(p);
  else if (tile == 1) qkv_proj_kernel<TileB><<<dim3((unsigned)total), TileB::kThreads, 0, st>>>(p);
  else qkv_proj_kernel<TileC><<<dim3((unsigned)total), TileC::kThreads, 0, st>>>(p);
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
