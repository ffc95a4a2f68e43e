// RMSNorm and rotate-half RoPE of one head section (head_dim 128), shared by
// the QKV prologue and the fused projection.
//
// A section is one (token, head) slice of 128 values handled by a group of 8
// lanes: lane j holds elements [8j, 8j+8) of the first half and
// [64+8j, 64+8j+8) of the second, so every rotate-half pair (x[i], x[i+64])
// sits in one lane; the RMS sum is reduced over the 8 lanes of the group.
#pragma once

#include "aa_common.h"

namespace aa {

constexpr int kHd = 128;
constexpr int kHalf = 64;

struct Section {
  float a[8];
  float b[8];
};

__device__ __forceinline__ void load_section(const bf16* src, int j, Section& s) {
  unpack8(ld16(src + 8 * j), s.a);
  unpack8(ld16(src + kHalf + 8 * j), s.b);
}

// A section's two 16-byte chunks as loaded, before unpacking.
struct RawSection {
  u32x4 a;
  u32x4 b;
};

__device__ __forceinline__ void load_raw(const bf16* src, int j, RawSection& r) {
  r.a = ld16(src + 8 * j);
  r.b = ld16(src + kHalf + 8 * j);
}

__device__ __forceinline__ Section unpack_section(const RawSection& r) {
  Section s;
  unpack8(r.a, s.a);
  unpack8(r.b, s.b);
  return s;
}

__device__ __forceinline__ void load_w(const float* w, int j, float* wa, float* wb) {
  f32x4 w0 = ldf4(w + 8 * j), w1 = ldf4(w + 8 * j + 4);
  f32x4 w2 = ldf4(w + kHalf + 8 * j), w3 = ldf4(w + kHalf + 8 * j + 4);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    wa[i] = w0[i];
    wa[i + 4] = w1[i];
    wb[i] = w2[i];
    wb[i + 4] = w3[i];
  }
}

__device__ __forceinline__ void load_rot(const float* cos, const float* sin, int64_t pos, int j,
                                         float* c, float* s) {
  const float* cp = cos + pos * kHalf + 8 * j;
  const float* sp = sin + pos * kHalf + 8 * j;
  f32x4 c0 = ldf4(cp), c1 = ldf4(cp + 4), s0 = ldf4(sp), s1 = ldf4(sp + 4);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    c[i] = c0[i];
    c[i + 4] = c1[i];
    s[i] = s0[i];
    s[i + 4] = s1[i];
  }
}

// rstd over the section's 128 values, y = bf16(x * rstd * w).
__device__ __forceinline__ void norm_scale(const Section& x, const float* w, int j, float eps,
                                           float* oa, float* ob) {
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss += x.a[i] * x.a[i] + x.b[i] * x.b[i];
  ss = group_sum<8>(ss);
  const float rstd = rsqrtf(ss / (float)kHd + eps);
  float wa[8], wb[8];
  load_w(w, j, wa, wb);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    oa[i] = round_bf16(x.a[i] * rstd * wa[i]);
    ob[i] = round_bf16(x.b[i] * rstd * wb[i]);
  }
}

// out_a = y_a cos - y_b sin, out_b = y_b cos + y_a sin (the order of
// src/kernels/rope.py:39-58), in place, with this lane's 8 cos / sin values.
__device__ __forceinline__ void rotate_half(float* a, float* b, const float* c, const float* s) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float ya = a[i], yb = b[i];
    a[i] = ya * c[i] - yb * s[i];
    b[i] = yb * c[i] + ya * s[i];
  }
}

// norm_scale, then with ROTATE rotate_half by the RoPE row of position pos.
template <bool ROTATE>
__device__ __forceinline__ void norm_rotate(const Section& x, const float* w, const float* cos,
                                            const float* sin, int64_t pos, int j, float eps,
                                            float* oa, float* ob) {
  norm_scale(x, w, j, eps, oa, ob);
  if constexpr (ROTATE) {
    float c[8], s[8];
    load_rot(cos, sin, pos, j, c, s);
    rotate_half(oa, ob, c, s);
  }
}

}  // namespace aa
