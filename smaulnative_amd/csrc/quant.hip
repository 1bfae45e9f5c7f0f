// quant.hip -- the tiled E4M3 quantizer on MI355X (gfx950).
//
// Replaces the reference's native quantizer kernel/quant_cpu.cpp:64-137
// (fp8_quantize_tiles, reached through CpuBackend.fp8_quantize_tiles,
// kernel/compute.py:246-263) and gives the same codes and scales as its torch
// path (kernel/fp8_tile.py:100-113), bit for bit:
//   amax_t = max |w| over the finite entries of the tile, at least 1e-12
//   sc_t   = max(amax_t / 448, 1e-12)
//   n      = clamp(nan_to_num(w / sc_t, nan=0), -448, 448)
//   code   = order[first i with bounds[i] >= n]       (0 where n == 0)
// `order` / `bounds` are the sorted-codebook permutation and its 255
// midpoints, passed in by the caller from the same tables the reference
// uses: the codebook has duplicate values (0x7E/0x7F = 448, 0xFE/0xFF =
// -448), so which duplicate a saturated weight gets is the tables' tie order.
//
// Layout: w fp32 [out_f, in_f] row-major; codes uint8 [out_f, ldc] with
// ldc >= nt * tile (the padding of the last tile is written as code 0, as the
// reference returns it); scales fp32 [out_f, nt].  An HBM-bound pass: 4 bytes
// read and 1 written per weight, every tile read once.
#include "smaul_common.h"

using smaul::check_launch;
using smaul::fail;

namespace {

constexpr int QUANT_THREADS = 256;

__global__ void quant_clear_kernel(unsigned long long* counter) { *counter = 0ull; }

// first i in [0, 255] with bounds[i] >= n (std::lower_bound / torch.bucketize)
__device__ __forceinline__ uint8_t quant_encode(float n, const float* sb, const uint8_t* so) {
  if (n == 0.0f) return 0;
  int lo = 0, hi = 255;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (sb[mid] < n) lo = mid + 1;
    else hi = mid;
  }
  return so[lo];
}

// SEG: tile is a power of two <= 64; a wave covers 64 / tile consecutive
// tiles of one row, lanes in aligned segments of `tile`.  Otherwise a wave
// covers one tile, lane l holding elements l, l + 64, ... of it.
template <bool SEG>
__global__ void __launch_bounds__(QUANT_THREADS)
quant_tiles_kernel(const float* __restrict__ w, int64_t out_f, int64_t in_f, int tile, int64_t nt, int64_t ldc,
                   const uint8_t* __restrict__ order, const float* __restrict__ bounds, uint8_t* __restrict__ codes,
                   float* __restrict__ scales, unsigned long long* __restrict__ nonfinite, int64_t units) {
  __shared__ float sb[256];
  __shared__ uint8_t so[256];
  if (threadIdx.x < 255) sb[threadIdx.x] = bounds[threadIdx.x];
  if (threadIdx.x < 256) so[threadIdx.x] = order[threadIdx.x];
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int64_t unit = ((int64_t)blockIdx.x * QUANT_THREADS + threadIdx.x) >> 6;
  if (unit >= units) return;  // whole waves: the shuffles below stay uniform
  const int per_wave = SEG ? 64 / tile : 1;            // tiles per wave
  const int64_t waves_per_row = (nt + per_wave - 1) / per_wave;
  const int64_t row = unit / waves_per_row;
  const int64_t t = (unit % waves_per_row) * per_wave + (SEG ? lane / tile : 0);
  const float* wr = w + row * in_f;
  int bad = 0;
  float amax = 0.0f;
  if constexpr (SEG) {
    const int64_t k = t * tile + lane % tile;
    float v = 0.0f;
    if (t < nt && k < in_f) v = wr[k];
    if (!__builtin_isfinite(v)) ++bad;
    amax = __builtin_isfinite(v) ? fabsf(v) : 0.0f;
    for (int o = 1; o < tile; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    const float am = amax < 1e-12f ? 1e-12f : amax;
    const float sc = fmaxf(am / 448.0f, 1e-12f);
    if (t < nt) {
      float n = v / sc;
      if (n != n) n = 0.0f;
      n = fminf(fmaxf(n, -448.0f), 448.0f);
      codes[row * ldc + k] = quant_encode(n, sb, so);
      if (lane % tile == 0) scales[row * nt + t] = sc;
    }
  } else {
    const int64_t k0 = t * tile;
    for (int j = lane; j < tile; j += 64) {
      const int64_t k = k0 + j;
      const float v = k < in_f ? wr[k] : 0.0f;
      if (!__builtin_isfinite(v)) ++bad;
      if (__builtin_isfinite(v)) amax = fmaxf(amax, fabsf(v));
    }
    for (int o = 1; o < 64; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    const float am = amax < 1e-12f ? 1e-12f : amax;
    const float sc = fmaxf(am / 448.0f, 1e-12f);
    for (int j = lane; j < tile; j += 64) {
      const int64_t k = k0 + j;
      float n = (k < in_f ? wr[k] : 0.0f) / sc;
      if (n != n) n = 0.0f;
      n = fminf(fmaxf(n, -448.0f), 448.0f);
      codes[row * ldc + k] = quant_encode(n, sb, so);
    }
    if (lane == 0) scales[row * nt + t] = sc;
  }
  // the wave's non-finite count, one atomic per wave that saw any
  for (int o = 32; o >= 1; o >>= 1) bad += __shfl_xor(bad, o, 64);
  if (lane == 0 && bad) atomicAdd(nonfinite, (unsigned long long)bad);
}

}  // namespace

extern "C" {

int smaul_fp8_quantize_tiles(const float* w, int64_t out_f, int64_t in_f, int64_t tile, const uint8_t* order,
                             const float* bounds, uint8_t* codes, int64_t ldc, float* scales,
                             unsigned long long* nonfinite, hipStream_t stream) {
  if (tile <= 0) return fail(SMAUL_ERR_INVALID, "quantize_tiles: tile must be > 0, got %lld", (long long)tile);
  if (out_f <= 0 || in_f <= 0)
    return fail(SMAUL_ERR_INVALID, "quantize_tiles: out_f/in_f must be positive, got %lld/%lld", (long long)out_f,
                (long long)in_f);
  const int64_t nt = (in_f + tile - 1) / tile;
  if (ldc < nt * tile) return fail(SMAUL_ERR_INVALID, "quantize_tiles: ldc %lld < nt*tile %lld", (long long)ldc,
                                   (long long)(nt * tile));
  if (tile > (1 << 20)) return fail(SMAUL_ERR_UNSUPPORTED, "quantize_tiles: tile too large");
  if (!w || !order || !bounds || !codes || !scales || !nonfinite)
    return fail(SMAUL_ERR_INVALID, "quantize_tiles: null pointer");
  hipLaunchKernelGGL(quant_clear_kernel, dim3(1), dim3(1), 0, stream, nonfinite);
  int rc = check_launch("quant_clear_kernel");
  if (rc) return rc;
  const bool seg = tile <= 64 && (tile & (tile - 1)) == 0;
  const int64_t per_wave = seg ? 64 / tile : 1;
  const int64_t units = out_f * ((nt + per_wave - 1) / per_wave);
  const int64_t blocks = (units * 64 + QUANT_THREADS - 1) / QUANT_THREADS;
  if (blocks > 2147483647LL) return fail(SMAUL_ERR_UNSUPPORTED, "quantize_tiles: matrix too large");
  if (seg)
    hipLaunchKernelGGL((quant_tiles_kernel<true>), dim3((unsigned)blocks), dim3(QUANT_THREADS), 0, stream, w, out_f,
                       in_f, (int)tile, nt, ldc, order, bounds, codes, scales, nonfinite, units);
  else
    hipLaunchKernelGGL((quant_tiles_kernel<false>), dim3((unsigned)blocks), dim3(QUANT_THREADS), 0, stream, w, out_f,
                       in_f, (int)tile, nt, ldc, order, bounds, codes, scales, nonfinite, units);
  return check_launch("quant_tiles_kernel");
}

}  // extern "C"
