// Per-token FP8 quantisation of activations (the consumer of the attention
// output in the FP8 model path), optionally after GELU.
//
// For each row x of K values: y = x (or GELU(x)), scale = max(max|y|, 1e-12)
// / 448, q = e4m3fn(clamp(y / scale, -448, 448)) with round-to-nearest-even,
// and the fp32 scale per row. One wave per row, four rows per workgroup, the
// row cut into units of 16 values (8 when K % 16 != 0) spread over the 64
// lanes, K <= 8192: one HBM read of the row and one write of its bytes. The
// row max is a wave reduction, so no LDS and no barrier stand between a row's
// loads and its stores, and every lane keeps all its units' loads in flight
// at once. At 2 x 4096 x 2048: a workgroup of 256 lanes per row, with the max
// exchanged through LDS, ran 12.4 us (4.1 TB/s); one wave per row 9.9 us;
// with nontemporal code stores 7.6 us; with GELU a template parameter instead
// of a uniform branch per value 7.46 us; with 16-value units (one 16-byte
// store each instead of two 8-byte ones) 7.06 us, 7.1 TB/s.
//
// e4m3fn (OCP FP8 E4M3, "fn": no infinities, NaN = S.1111.111): exponent bias
// 7, 3 mantissa bits, largest finite 448 = 1.75 * 2^8, normal down to 2^-6,
// subnormals m * 2^-9. gfx950's v_cvt_pk_fp8_f32 converts to this format with
// round-to-nearest-even: it agreed with an integer re-implementation of that
// rounding on every fp32 value of magnitude 2^-30 .. 448 (both signs), and the
// GPU tests check every e4m3 tie point and its fp32 neighbours through this
// kernel. The clamp keeps the input finite and in range. (Replacing the
// integer encoding by the instruction took the kernel from 18.8 to 12.8 us at
// 2 x 4096 x 2048, the reciprocal-based quotients in rq_store to 11.8 us.)
//
// GELU uses the erf approximation 7.1.26 of Abramowitz and Stegun (Handbook
// of Mathematical Functions, 1964; |error| <= 1.5e-7), the form the
// reference's kernel uses: erf(z) ~ 1 - t (a1 + t (a2 + t (a3 + t (a4 + t a5))))
// exp(-z^2), t = 1 / (1 + p |z|).
#include <cmath>

#include "aa_common.h"

namespace aa {

constexpr int kRqThreads = 256;
constexpr int kRqRowsPerBlock = kRqThreads / 64;  // one wave per row
constexpr int kRqMaxK = 8192;

__device__ __forceinline__ float gelu_as(float x) {
  const float z = x * 0.7071067811865476f;
  const float az = fabsf(z);
  const float t = 1.0f / (1.0f + 0.3275911f * az);
  const float poly =
      ((((1.061405429f * t - 1.453152027f) * t + 1.421413741f) * t - 0.284496736f) * t +
       0.254829592f) *
      t;
  const float y = 1.0f - poly * expf(-az * az);
  return 0.5f * x * (1.0f + (z < 0.f ? -y : y));
}

// Quantise this lane's units of the row (unit lane + 64 p, U values each):
// y / scale (correctly rounded), clamp, e4m3fn, U bytes stored at once. With
// kMarkstein the quotient comes from the correctly rounded reciprocal rcp of
// the scale (Markstein): q0 = RN(y * rcp) is within an ulp of the quotient,
// e = y - q0 * scale is exact (FMA), and RN(q0 + e * rcp) is the correctly
// rounded quotient unless something underflows. The caller takes this path
// when the row's amax is at least 2^-60: a quotient whose remainder could
// underflow is then below 2^-60 itself and encodes to zero either way. Other
// rows divide.
template <int NU, int U, bool kMarkstein>
__device__ __forceinline__ void rq_store(const float (&v)[NU][U], float scale, float rcp,
                                         int nunit, int lane, uint8_t* qr) {
#pragma unroll
  for (int p = 0; p < NU; ++p) {
    const int u = lane + 64 * p;
    if (u < nunit) {
      float y[U];
#pragma unroll
      for (int i = 0; i < U; ++i) {
        float t;
        if constexpr (kMarkstein) {
          // The sign is the input's (scale > 0); the FMAs alone would turn
          // -0.0 into +0.0 (-0 + +0 rounds to +0), which the division keeps.
          const float q0 = v[p][i] * rcp;
          t = copysignf(fmaf(fmaf(-q0, scale, v[p][i]), rcp, q0), v[p][i]);
        } else {
          t = v[p][i] / scale;
        }
        y[i] = fminf(fmaxf(t, -448.0f), 448.0f);
      }
      uint32_t w[U / 4];
#pragma unroll
      for (int h = 0; h < U / 4; ++h) {
        int word = __builtin_amdgcn_cvt_pk_fp8_f32(y[4 * h], y[4 * h + 1], 0, false);
        word = __builtin_amdgcn_cvt_pk_fp8_f32(y[4 * h + 2], y[4 * h + 3], word, true);
        w[h] = (uint32_t)word;
      }
      if constexpr (U == 16) {
        st16_nt(qr + 16 * u, u32x4{w[0], w[1], w[2], w[3]});
      } else {
        __builtin_nontemporal_store(u32x2{w[0], w[1]}, reinterpret_cast<u32x2*>(qr + 8 * u));
      }
    }
  }
}

// One wave per row; each lane takes units lane + 64 p (p < NU) of U
// consecutive values (U = 16 when K % 16 == 0: two 16-byte loads and one
// 16-byte store per unit; else U = 8). K <= 64 NU U.
template <int NU, int U, bool GELU>
__global__ __launch_bounds__(kRqThreads) void rowquant_kernel(const bf16* __restrict__ x,
                                                              uint8_t* __restrict__ q,
                                                              float* __restrict__ s, int64_t rows,
                                                              int K) {
  constexpr int W = U / 8;  // 16-byte loads per unit
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRqRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole waves; the kernel has no barrier
  const int nunit = K / U;
  const bf16* xr = x + row * K;
  u32x4 raw[NU][W];
#pragma unroll
  for (int p = 0; p < NU; ++p) {
    const int u = lane + 64 * p;
    if (u < nunit) {
#pragma unroll
      for (int w = 0; w < W; ++w) raw[p][w] = ld16(xr + U * u + 8 * w);
    }
  }
  float v[NU][U];
  float amax = 0.f;
#pragma unroll
  for (int p = 0; p < NU; ++p) {
    const int u = lane + 64 * p;
    if (u < nunit) {
#pragma unroll
      for (int w = 0; w < W; ++w) unpack8(raw[p][w], &v[p][8 * w]);
#pragma unroll
      for (int i = 0; i < U; ++i) {
        if constexpr (GELU) v[p][i] = gelu_as(v[p][i]);
        amax = fmaxf(amax, fabsf(v[p][i]));
      }
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  const float scale = fmaxf(amax, 1e-12f) / 448.0f;
  uint8_t* qr = q + row * K;
  if (amax >= 0x1p-60f) {
    rq_store<NU, U, true>(v, scale, 1.0f / scale, nunit, lane, qr);
  } else {
    rq_store<NU, U, false>(v, scale, 0.f, nunit, lane, qr);
  }
  if (lane == 0) s[row] = scale;
}

template <int NU, int U>
static void launch_rowquant(dim3 grid, hipStream_t st, const bf16* x, uint8_t* q, float* s,
                            int64_t rows, int K, bool gelu) {
  if (gelu) rowquant_kernel<NU, U, true><<<grid, kRqThreads, 0, st>>>(x, q, s, rows, K);
  else rowquant_kernel<NU, U, false><<<grid, kRqThreads, 0, st>>>(x, q, s, rows, K);
}

}  // namespace aa

using namespace aa;

extern "C" int aa_rowquant(const void* x, int64_t rows, int64_t K, int gelu, void* q, float* s,
                           int dtype, void* stream) {
  clear_error();
  if (dtype != AA_DTYPE_BF16)
    return fail(AA_EUNSUPPORTED, "rowquant: only bf16 input is implemented");
  if (rows < 0 || K <= 0) return fail(AA_EINVAL, "rowquant: bad rows/K");
  if (K % 8 != 0 || K > kRqMaxK)
    return fail(AA_EUNSUPPORTED, "rowquant: K must be a multiple of 8 and at most 8192");
  if (rows > 0x7fffffff) return fail(AA_EUNSUPPORTED, "rowquant: too many rows");
  if (rows == 0) return AA_OK;
  if (!x || !q || !s) return fail(AA_EINVAL, "rowquant: null pointer");
  if (!aligned16(x) || ((uintptr_t)q & 7u) != 0)
    return fail(AA_EINVAL, "rowquant: x must be 16-byte and q 8-byte aligned");
  const dim3 grid((unsigned)((rows + kRqRowsPerBlock - 1) / kRqRowsPerBlock));
  hipStream_t st = (hipStream_t)stream;
  const bf16* xb = (const bf16*)x;
  uint8_t* qb = (uint8_t*)q;
  const int k = (int)K;
  const bool g = gelu != 0;
  if (K % 16 == 0 && ((uintptr_t)q & 15u) == 0) {  // 16 values (16 code bytes) per unit
    if (K <= 2048) launch_rowquant<2, 16>(grid, st, xb, qb, s, rows, k, g);
    else if (K <= 4096) launch_rowquant<4, 16>(grid, st, xb, qb, s, rows, k, g);
    else launch_rowquant<8, 16>(grid, st, xb, qb, s, rows, k, g);
  } else {
    if (K <= 2048) launch_rowquant<4, 8>(grid, st, xb, qb, s, rows, k, g);
    else if (K <= 4096) launch_rowquant<8, 8>(grid, st, xb, qb, s, rows, k, g);
    else launch_rowquant<16, 8>(grid, st, xb, qb, s, rows, k, g);
  }
  return check_launch("rowquant");
}
