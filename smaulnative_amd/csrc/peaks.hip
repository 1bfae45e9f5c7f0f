// peaks.hip -- measured ceilings of MI355X (gfx950) for the roofline of this
// library's kernels: the dense bf16 MFMA rate of the instruction the prefill
// GEMM issues (v_mfma_f32_32x32x16_bf16), the HBM read rate of a stream of
// 16-byte loads, and the rate at which the GEMM's LDS-DMA loads
// (global_load_lds_dwordx4) fill LDS from L2-resident data.  Measurement only
// (bench.py --peaks); no reference counterpart and nothing on the MoE path
// calls them.
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

// LDS DMA, as the prefill GEMM issues it: each lane copies 16 bytes from
// base + off to LDS address lds + 16 * lane (M0 = lds).
typedef __attribute__((address_space(3))) void* lds_vptr_t;
__device__ __forceinline__ uint32_t lds_offset(const void* p) { return (uint32_t)(uintptr_t)(lds_vptr_t)p; }
__device__ __forceinline__ const void* uniform_ptr(const void* p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const void*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ void dma16(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               :: "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(off), "s"(uniform_ptr(base)) : "memory");
}

constexpr int PEAK_DMA_REGION = 64;  // 1 KB chunks read by one workgroup (64 KB, L2-resident after a pass)
constexpr int PEAK_DMA_SLOTS = 8;    // 1 KB LDS slots per wave

// Every wave copies `iters` rounds of 8 chunks of 1 KB from its workgroup's
// 64 KB region into its LDS slots, two rounds in flight; one word of LDS is
// stored at the end so the copies are not dead.
__global__ void __launch_bounds__(256) peak_lds_dma_kernel(const char* __restrict__ src, int iters, uint32_t* out) {
  __shared__ __attribute__((aligned(1024))) char smem[4 * PEAK_DMA_SLOTS * 1024];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const char* base = src + (size_t)blockIdx.x * PEAK_DMA_REGION * 1024;
  const uint32_t lds0 = lds_offset(&smem[0]);
  static_assert((PEAK_DMA_REGION & (PEAK_DMA_REGION - 1)) == 0, "chunk index taken modulo a power of two");
  for (int it = 0; it < iters; ++it) {
    const int r = it & (PEAK_DMA_REGION - 1);  // the chunk pattern repeats every 64 rounds; no overflow
#pragma unroll
    for (int s = 0; s < PEAK_DMA_SLOTS; ++s)
      dma16(base + (size_t)(((r * PEAK_DMA_SLOTS + s) * 7 + wave) & (PEAK_DMA_REGION - 1)) * 1024, lane * 16,
            lds0 + (wave * PEAK_DMA_SLOTS + s) * 1024);
    asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) out[blockIdx.x] = *(const uint32_t*)&smem[0];
}

}  // namespace

extern "C" {

int smaul_peak_mfma(float* out, int workgroups, int iters, hipStream_t stream) {
  if (!out || workgroups < 1 || iters < 1) return fail(SMAUL_ERR_INVALID, "peak_mfma: bad arguments");
  hipLaunchKernelGGL(peak_mfma_kernel, dim3((unsigned)workgroups), dim3(256), 0, stream, out, iters);
  return check_launch("peak_mfma_kernel");
}

int smaul_peak_lds_dma(const void* src, int64_t bytes, uint32_t* out, int workgroups, int iters,
                       hipStream_t stream) {
  if (!src || !out || workgroups < 1 || iters < 1 || bytes < (int64_t)workgroups * PEAK_DMA_REGION * 1024)
    return fail(SMAUL_ERR_INVALID, "peak_lds_dma: bad arguments (src needs 64 KB per workgroup)");
  hipLaunchKernelGGL(peak_lds_dma_kernel, dim3((unsigned)workgroups), dim3(256), 0, stream, (const char*)src, iters,
                     out);
  return check_launch("peak_lds_dma_kernel");
}

int smaul_peak_stream(const void* src, int64_t bytes, uint32_t* out, int workgroups, hipStream_t stream) {
  if (!src || !out || bytes < 16 || bytes % 16 != 0 || workgroups < 1)
    return fail(SMAUL_ERR_INVALID, "peak_stream: bad arguments");
  hipLaunchKernelGGL(peak_stream_kernel, dim3((unsigned)workgroups), dim3(256), 0, stream, (const uint4*)src,
                     bytes / 16, out);
  return check_launch("peak_stream_kernel");
}

}  // extern "C"
