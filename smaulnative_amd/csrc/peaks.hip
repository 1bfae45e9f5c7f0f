// peaks.hip -- measured ceilings of MI355X (gfx950) for the roofline of this
// library's kernels: the dense bf16 MFMA rate of the instruction the prefill
// GEMM issues (v_mfma_f32_32x32x16_bf16) and the HBM read rate of a stream of
// 16-byte loads.  Measurement only (bench.py --peaks); no reference
// counterpart and nothing on the MoE path calls them.
#include "smaul_common.h"

using smaul::check_launch;
using smaul::fail;

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int PEAK_CHAINS = 8;  // independent accumulators per wave (hides the MFMA latency)

// Every wave issues `iters` rounds of PEAK_CHAINS independent 32x32x16 bf16
// MFMAs; the operands are formed from the lane id so the compiler cannot fold
// them, and one value per wave is stored so the chains stay live.
__global__ void __launch_bounds__(256) peak_mfma_kernel(float* out, int iters) {
  const int lane = threadIdx.x & 63;
  bf16x8_t a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = (__bf16)(0.001f * (float)(lane + i));
    b[i] = (__bf16)(0.002f * (float)(lane - i));
  }
  f32x16_t acc[PEAK_CHAINS];
#pragma unroll
  for (int c = 0; c < PEAK_CHAINS; ++c)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[c][r] = 0.0f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int c = 0; c < PEAK_CHAINS; ++c) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[c], 0, 0, 0);
  }
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < PEAK_CHAINS; ++c) s += acc[c][lane & 15];
  if (lane == 0) out[blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)] = s;
}

// Grid-stride read of n 16-byte vectors; each thread folds what it read into
// one word so the loads stay live (stored only if it matches an impossible
// pattern, so the writes cost nothing).
__global__ void __launch_bounds__(256) peak_stream_kernel(const uint4* __restrict__ src, int64_t n, uint32_t* out) {
  uint32_t x = 0;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const uint4 v = src[i];
    x ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (x == 0x9e3779b9u) out[0] = x;
}

}  // namespace

extern "C" {

int smaul_peak_mfma(float* out, int workgroups, int iters, hipStream_t stream) {
  if (!out || workgroups < 1 || iters < 1) return fail(SMAUL_ERR_INVALID, "peak_mfma: bad arguments");
  hipLaunchKernelGGL(peak_mfma_kernel, dim3((unsigned)workgroups), dim3(256), 0, stream, out, iters);
  return check_launch("peak_mfma_kernel");
}

int smaul_peak_stream(const void* src, int64_t bytes, uint32_t* out, int workgroups, hipStream_t stream) {
  if (!src || !out || bytes < 16 || bytes % 16 != 0 || workgroups < 1)
    return fail(SMAUL_ERR_INVALID, "peak_stream: bad arguments");
  hipLaunchKernelGGL(peak_stream_kernel, dim3((unsigned)workgroups), dim3(256), 0, stream, (const uint4*)src,
                     bytes / 16, out);
  return check_launch("peak_stream_kernel");
}

}  // extern "C"
