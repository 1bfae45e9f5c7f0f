// backward.hip -- the input gradient of the tiled-FP8 linear on MI355X (gfx950).
//
// dx[r, i] = sum_o g[r, o] * W[o, i] with W[o, i] = lut[w[o, i]] * s[o, i / tile]:
// the backend entry fp8_backward_input (kernel/compute.py:145-153), replacing
// the reference's native kernel kernel/fp8_cpu.cpp:167-259.  Training only;
// not on the forward path.
//
// A workgroup owns a 64 x 64 tile of dx and walks the output dimension o in
// chunks of 32: the chunk of g (transposed) and the chunk of W decoded to
// fp32 (lut * s rounded once, as the reference's fast path forms it) are
// staged in LDS, and each thread accumulates a 4 x 4 block with fused
// multiply-adds.  The sum over o runs in another order than the reference's
// eight-way split, so results agree to fp32 rounding (relative 1e-6), not
// bitwise.  It is a VALU kernel: the backward is not timed here, and an fp32
// gradient would need three bf16 terms per value to go through MFMA exactly.
#include "smaul_common.h"

using smaul::check_launch;
using smaul::fail;

namespace {

constexpr float e4m3_value(int c) {
  const int e = (c >> 3) & 15, m = c & 7;
  float mag = 0.0f;
  if (e == 15 && m == 7) {
    mag = 448.0f;
  } else if (e == 0) {
    mag = (float)m / 512.0f;
  } else {
    float p = 1.0f;
    for (int i = 7; i < e; ++i) p *= 2.0f;
    for (int i = e; i < 7; ++i) p *= 0.5f;
    mag = (1.0f + (float)m / 8.0f) * p;
  }
  return (c & 128) ? -mag : mag;
}

struct Lut {
  float v[256];
  constexpr Lut() : v() {
    for (int c = 0; c < 256; ++c) v[c] = e4m3_value(c);
  }
};
__constant__ Lut kLut = Lut();

constexpr int BW_T = 64;   // dx tile: rows and input columns
constexpr int BW_K = 32;   // output dimension per LDS chunk

__global__ void __launch_bounds__(256)
fp8_backward_input_kernel(const float* __restrict__ g, const uint8_t* __restrict__ w, const float* __restrict__ s,
                          float* __restrict__ dx, int64_t rows, int64_t in_f, int64_t out_f, int64_t tile,
                          int64_t nt) {
  __shared__ float sg[BW_K][BW_T + 4];  // g chunk, [o][row]
  __shared__ float sw[BW_K][BW_T + 4];  // decoded W chunk, [o][col]
  const int tid = threadIdx.x;
  const int tx = tid & 15, ty = tid >> 4;
  const int64_t r0 = (int64_t)blockIdx.y * BW_T, c0 = (int64_t)blockIdx.x * BW_T;
  float acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = 0.0f;
  for (int64_t o0 = 0; o0 < out_f; o0 += BW_K) {
    // 32 x 64 of each: 8 loads per thread per operand, coalesced along o for g
    // and along i for w
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int idx = tid + q * 256;
      {
        const int ko = idx & (BW_K - 1), rr = idx >> 5;
        const int64_t r = r0 + rr, o = o0 + ko;
        sg[ko][rr] = (r < rows && o < out_f) ? g[r * out_f + o] : 0.0f;
      }
      {
        const int cc = idx & (BW_T - 1), ko = idx >> 6;
        const int64_t i = c0 + cc, o = o0 + ko;
        float v = 0.0f;
        if (i < in_f && o < out_f) v = kLut.v[w[o * in_f + i]] * s[o * nt + i / tile];
        sw[ko][cc] = v;
      }
    }
    __syncthreads();
#pragma unroll 8
    for (int k = 0; k < BW_K; ++k) {
      float gv[4], wv[4];
#pragma unroll
      for (int a = 0; a < 4; ++a) gv[a] = sg[k][ty * 4 + a];
#pragma unroll
      for (int b = 0; b < 4; ++b) wv[b] = sw[k][tx * 4 + b];
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = __builtin_fmaf(gv[a], wv[b], acc[a][b]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const int64_t r = r0 + ty * 4 + a;
    if (r >= rows) continue;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int64_t i = c0 + tx * 4 + b;
      if (i < in_f) dx[r * in_f + i] = acc[a][b];
    }
  }
}

}  // namespace

extern "C" {

int smaul_fp8_backward_input(const float* g, const uint8_t* w, const float* s, float* dx, int64_t rows,
                             int64_t in_f, int64_t out_f, int64_t tile, hipStream_t stream) {
  // in_f / out_f may be 0, as in the reference (fp8_cpu.cpp:227-228): no
  // columns, or an empty sum (dx all zeros, g / w / s not read)
  if (tile <= 0 || in_f < 0 || out_f < 0 || rows < 0)
    return fail(SMAUL_ERR_INVALID, "fp8_backward_input: need tile > 0 and in_f, out_f, rows >= 0, got %lld/%lld/%lld",
                (long long)tile, (long long)in_f, (long long)out_f);
  if (rows == 0 || in_f == 0) return SMAUL_OK;
  if (!dx || (out_f > 0 && (!g || !w || !s))) return fail(SMAUL_ERR_INVALID, "fp8_backward_input: null pointer");
  const int64_t gx = (in_f + BW_T - 1) / BW_T, gy = (rows + BW_T - 1) / BW_T;
  if (gx > 2147483647LL || gy > 65535) return fail(SMAUL_ERR_UNSUPPORTED, "fp8_backward_input: grid too large");
  hipLaunchKernelGGL(fp8_backward_input_kernel, dim3((unsigned)gx, (unsigned)gy), dim3(256), 0, stream, g, w, s, dx,
                     rows, in_f, out_f, tile, (in_f + tile - 1) / tile);
  return check_launch("fp8_backward_input_kernel");
}

}  // extern "C"
