// Calibration for the measurement, not part of the attention path: the rate at
// which this GPU sustains v_mfma_f32_32x32x16_bf16 when nothing else runs
// (operands in registers, no memory traffic in the timed loop, one workgroup
// of one wave per SIMD on every CU), for operands of a given distribution.
// Under a full matrix-pipe load the clock falls below the one the published
// dense peak assumes, the more so the more the operand bits toggle; this rate
// is the ceiling that MFMA-bound kernels on such data approach. bench.py
// reports it beside the roofline (libanima_calib.so, built by build.py).
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kThreads = 256;  // one wave per SIMD
constexpr int kChains = 8;     // independent accumulators per wave

// Operand value of (lane, slot, element) for distribution dist: 0 = sum of
// four uniforms on [-1, 1) scaled to unit variance (close to N(0,1)),
// 1 = uniform on [0, 1), 2 = zero. A 32-bit integer hash (Wang's mix) gives
// the uniforms.
__device__ uint32_t mix(uint32_t x) {
  x = (x ^ 61u) ^ (x >> 16);
  x *= 9u;
  x ^= x >> 4;
  x *= 0x27d4eb2du;
  return x ^ (x >> 15);
}
__device__ float uni(uint32_t key) { return (float)(mix(key) >> 8) * (1.0f / 16777216.0f); }
__device__ float value(int dist, uint32_t key) {
  if (dist == 2) return 0.f;
  if (dist == 1) return uni(key);
  float s = 0.f;
  for (int i = 0; i < 4; ++i) s += 2.f * uni(key * 4u + (uint32_t)i) - 1.f;
  return s * 0.8660254f;  // sqrt(3 / 4): unit variance
}

__global__ __launch_bounds__(kThreads) void calib_mfma_kernel(int dist, int iters, float* out) {
  __shared__ float pad[96 * 256];  // 96 KiB: one workgroup per CU
  pad[threadIdx.x] = 1.f;
  __syncthreads();
  bf16x8 op[8];  // four A and four B operands, rotated between iterations
  const uint32_t base = (blockIdx.x * kThreads + threadIdx.x) * 64u;
#pragma unroll
  for (int s = 0; s < 8; ++s)
#pragma unroll
    for (int e = 0; e < 8; ++e) op[s][e] = (__bf16)value(dist, base + 8u * s + e);
  f32x16 acc[kChains];
#pragma unroll
  for (int j = 0; j < kChains; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.f;
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int j = 0; j < kChains; ++j)
      acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op[j & 3], op[4 + ((j + 1) & 3)], acc[j], 0, 0, 0);
    const bf16x8 t = op[0];
    op[0] = op[1];
    op[1] = op[2];
    op[2] = op[3];
    op[3] = t;
    asm volatile("" : "+v"(op[0]), "+v"(op[1]), "+v"(op[2]), "+v"(op[3]));
  }
  float s = pad[(threadIdx.x + 1) % kThreads];
#pragma unroll
  for (int j = 0; j < kChains; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) s += acc[j][r];
  out[blockIdx.x * kThreads + threadIdx.x] = s;
}

}  // namespace

// Sustained MFMA rate (TFLOP/s, into *tflops) for operand distribution dist
// (0: ~N(0,1), 1: U[0,1), 2: zero): one warm-up launch, then the best of
// `reps` timed launches of `iters` iterations (8 MFMAs per wave each) on
// every CU of the current device, on `stream`. Returns 0, or -1 on a bad
// argument or a HIP error.
extern "C" int aa_calib_mfma(int dist, int iters, int reps, float* tflops, void* stream) {
  if (dist < 0 || dist > 2 || iters <= 0 || reps <= 0 || !tflops) return -1;
  int dev = 0, ncu = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || ncu <= 0)
    return -1;
  hipStream_t st = (hipStream_t)stream;
  float* out = nullptr;
  if (hipMalloc(&out, (size_t)ncu * kThreads * sizeof(float)) != hipSuccess) return -1;
  hipEvent_t e0, e1;
  int rc = 0;
  if (hipEventCreate(&e0) != hipSuccess) rc = -1;
  if (rc == 0 && hipEventCreate(&e1) != hipSuccess) {
    (void)hipEventDestroy(e0);
    rc = -1;
  }
  if (rc == 0) {
    float best_ms = 0.f;
    calib_mfma_kernel<<<dim3(ncu), kThreads, 0, st>>>(dist, iters, out);
    for (int r = 0; r < reps && rc == 0; ++r) {
      (void)hipEventRecord(e0, st);
      calib_mfma_kernel<<<dim3(ncu), kThreads, 0, st>>>(dist, iters, out);
      (void)hipEventRecord(e1, st);
      float ms = 0.f;
      if (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess) rc = -1;
      if (rc == 0 && (r == 0 || ms < best_ms)) best_ms = ms;
    }
    if (rc == 0 && hipGetLastError() != hipSuccess) rc = -1;
    if (rc == 0) {
      const double flops = (double)ncu * (kThreads / 64) * iters * kChains * 32.0 * 32.0 * 16.0 * 2.0;
      *tflops = (float)(flops / (best_ms * 1e-3) / 1e12);
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
  }
  (void)hipFree(out);
  return rc;
}
