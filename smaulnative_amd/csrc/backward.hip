// backward.hip -- the input gradient of the tiled-FP8 linear on MI355X (gfx950).
//
// dx[r, i] = sum_o g[r, o] * W[o, i] with W[o, i] = lut[w[o, i]] * s[o, i / tile]:
// the backend entry fp8_backward_input (kernel/compute.py:145-153), replacing
// the reference's native kernel kernel/fp8_cpu.cpp:167-259.  Training only;
// not on the forward path.
//
// Two kernels, each a workgroup per 64 x 64 tile of dx walking the output
// dimension o in chunks of 32, whose sums over o run in another order than
// the reference's eight-way split: results agree to fp32 rounding (relative
// 1e-6), not bitwise.
//  - fp8_backward_input_mfma_kernel (tile a multiple of 64, so the tile's 64
//    input columns share one scale column kb): dx[r, i] = sum_o (g[r, o] *
//    s[o, kb]) * lut[w[o, i]].  The products g * s are formed in fp32 and
//    split exactly into three bf16 terms, the codes decode exactly to bf16,
//    so every matrix-core product is exact and the sums are fp32.  (The
//    reference rounds lut * s instead of g * s: the same to fp32 rounding.)
//  - fp8_backward_input_kernel (any tile): the chunk of W decoded to fp32
//    (lut * s rounded once, as the reference's fast path forms it) and of g
//    staged in LDS, each thread a 4 x 4 block of fused multiply-adds.
#include "e4m3.h"
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

typedef float f32x16_t __attribute__((ext_vector_type(16)));

// Four waves, each 32 rows x 32 columns of the tile (v_mfma_f32_32x32x16_bf16:
// lane l holds row / column l % 32 of the operands at k = 8 (l / 32) + 0..7,
// and column l % 32, rows (r / 4) 8 + (l / 32) 4 + r % 4 of the sums).  Per
// chunk of BWM_K = 64 o: every thread turns 16 values of g * s (one row, 16
// consecutive o) into their three bf16 terms and writes them to LDS, and
// transposes a 4 x 4 block of codes (4 o x 4 columns, v_perm) into four
// column words of 4 o; the loads of the next chunk are issued before the
// chunk's MFMAs.  VEC: g rows and code rows are
// 16-byte aligned and whole chunks are in range (out_f % 64 == 0, in_f % 64
// == 0), so they load as 16-byte vectors.
constexpr int BWM_K = 64;

template <bool CANON, bool VEC>
__global__ void __launch_bounds__(256)
fp8_backward_input_mfma_kernel(const float* __restrict__ g, const uint8_t* __restrict__ w,
                               const float* __restrict__ s, float* __restrict__ dx, int64_t rows, int64_t in_f,
                               int64_t out_f, int64_t tile, int64_t nt) {
  __shared__ __attribute__((aligned(16))) uint16_t sa[3][BW_T][BWM_K + 8];  // terms of g * s, [row][o]
  // codes, [column][o]; rows of 72 bytes: the word writes of a wave meet at
  // most two to a bank, the 8-byte fragment reads none
  __shared__ __attribute__((aligned(16))) uint8_t sw[BW_T][BWM_K + 8];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  // Workgroup b runs on XCD b % 8: each XCD takes a contiguous band of the
  // tiles in row order, so the column tiles that read the same g rows share
  // one L2 (in launch order they went to eight L2s, with a 38 % hit rate at
  // config 2's gate shape)
  int64_t r0, c0;
  {
    const int64_t nc = gridDim.x, total = nc * gridDim.y, full = (total / 8) * 8;
    int64_t lin = (int64_t)blockIdx.y * nc + blockIdx.x;
    if (lin < full) lin = (lin % 8) * (full / 8) + lin / 8;
    r0 = (lin / nc) * BW_T;
    c0 = (lin % nc) * BW_T;
  }
  const int64_t kb = c0 / tile;
  // this thread's staging: g row ar, 16 o from ao; codes of o wo..wo+3 x columns wc..wc+3
  const int ar = tid >> 2, ao = (tid & 3) * 16;
  const int wo = (tid >> 4) * 4, wc = (tid & 15) * 4;
  const int64_t gr = r0 + ar;
  float gv[16], sv[16];
  uint32_t cw[4];  // row wo + r, columns wc..wc+3 (byte c = column wc + c)
  auto load = [&](int64_t o0) {
    if constexpr (VEC) {
      const float4* gp = (const float4*)(g + (gr < rows ? gr : rows - 1) * out_f + o0 + ao);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 v = gp[q];
        gv[4 * q] = v.x;
        gv[4 * q + 1] = v.y;
        gv[4 * q + 2] = v.z;
        gv[4 * q + 3] = v.w;
      }
      // the wave's lanes hold the chunk's 64 scales, lane l that of o = (l & 3) * 16 + (l >> 2),
      // and each lane gathers its 16 (ao = (l & 3) * 16) with cross-lane reads
      const float sl = s[(o0 + (lane & 3) * 16 + (lane >> 2)) * nt + kb];
#pragma unroll
      for (int j = 0; j < 16; ++j) sv[j] = __shfl(sl, (j << 2) | (lane & 3), 64);
#pragma unroll
      for (int r = 0; r < 4; ++r) cw[r] = *(const uint32_t*)(w + (o0 + wo + r) * in_f + c0 + wc);
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int64_t o = o0 + ao + j;
        gv[j] = (gr < rows && o < out_f) ? g[gr * out_f + o] : 0.0f;
        sv[j] = o < out_f ? s[o * nt + kb] : 0.0f;
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t o = o0 + wo + r;
        uint32_t v = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int64_t i = c0 + wc + c;
          v |= ((o < out_f && i < in_f) ? (uint32_t)w[o * in_f + i] : 0u) << (8 * c);  // code 0 decodes to +0
        }
        cw[r] = v;
      }
    }
  };
  f32x16_t acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
  load(0);
  for (int64_t o0 = 0; o0 < out_f; o0 += BWM_K) {
    {
      uint32_t t[3][8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        float a = gv[2 * q] * sv[2 * q], b = gv[2 * q + 1] * sv[2 * q + 1];
#pragma unroll
        for (int p = 0; p < 3; ++p) {  // term p: the bf16 rounding of what terms < p leave (exact differences)
          t[p][q] = pack_bf16(a, b);
          a = a - bf2f(t[p][q] & 0xffffu);
          b = b - bf2f(t[p][q] >> 16);
        }
      }
#pragma unroll
      for (int p = 0; p < 3; ++p) {
        *(uint4*)&sa[p][ar][ao] = make_uint4(t[p][0], t[p][1], t[p][2], t[p][3]);
        *(uint4*)&sa[p][ar][ao + 8] = make_uint4(t[p][4], t[p][5], t[p][6], t[p][7]);
      }
      // 4 x 4 byte transpose: column word c = (row 0 byte c, ..., row 3 byte c)
      // (v_perm: selector bytes 0-3 pick from the second operand, 4-7 from the first)
      const uint32_t lo01 = __builtin_amdgcn_perm(cw[1], cw[0], 0x05010400u);
      const uint32_t hi01 = __builtin_amdgcn_perm(cw[1], cw[0], 0x07030602u);
      const uint32_t lo23 = __builtin_amdgcn_perm(cw[3], cw[2], 0x05010400u);
      const uint32_t hi23 = __builtin_amdgcn_perm(cw[3], cw[2], 0x07030602u);
      *(uint32_t*)&sw[wc + 0][wo] = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);
      *(uint32_t*)&sw[wc + 1][wo] = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u);
      *(uint32_t*)&sw[wc + 2][wo] = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u);
      *(uint32_t*)&sw[wc + 3][wo] = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u);
    }
    __syncthreads();
    if (o0 + BWM_K < out_f) load(o0 + BWM_K);
#pragma unroll
    for (int ks = 0; ks < BWM_K / 16; ++ks) {
      const int ob = ks * 16 + (lane >> 5) * 8;
      const int fr = wm * 32 + (lane & 31), fc = wn * 32 + (lane & 31);
      const uint2 c = *(const uint2*)&sw[fc][ob];
      uint32_t d[4];
      decode4<CANON>(c.x, d[0], d[1]);
      decode4<CANON>(c.y, d[2], d[3]);
      const bf16x8_t bf = __builtin_bit_cast(bf16x8_t, make_uint4(d[0], d[1], d[2], d[3]));
#pragma unroll
      for (int p = 0; p < 3; ++p)
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(*(const bf16x8_t*)&sa[p][fr][ob], bf, acc, 0, 0, 0);
    }
    __syncthreads();
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int64_t row = r0 + wm * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
    const int64_t col = c0 + wn * 32 + (lane & 31);
    if (row < rows && col < in_f) dx[row * in_f + col] = acc[r];
  }
}

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
  const int64_t nt = (in_f + tile - 1) / tile;
  if (tile % BW_T == 0) {  // a dx tile's columns share one scale column
    const bool vec = out_f % BWM_K == 0 && in_f % BW_T == 0 && ((uintptr_t)g & 15) == 0 && ((uintptr_t)w & 15) == 0;
    if (vec)
      hipLaunchKernelGGL((fp8_backward_input_mfma_kernel<false, true>), dim3((unsigned)gx, (unsigned)gy), dim3(256), 0,
                         stream, g, w, s, dx, rows, in_f, out_f, tile, nt);
    else
      hipLaunchKernelGGL((fp8_backward_input_mfma_kernel<false, false>), dim3((unsigned)gx, (unsigned)gy), dim3(256),
                         0, stream, g, w, s, dx, rows, in_f, out_f, tile, nt);
    return check_launch("fp8_backward_input_mfma_kernel");
  }
  hipLaunchKernelGGL(fp8_backward_input_kernel, dim3((unsigned)gx, (unsigned)gy), dim3(256), 0, stream, g, w, s, dx,
                     rows, in_f, out_f, tile, nt);
  return check_launch("fp8_backward_input_kernel");
}

}  // extern "C"
