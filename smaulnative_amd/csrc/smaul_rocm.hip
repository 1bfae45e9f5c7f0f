// libsmaul_rocm.so -- tiled-FP8 MoE forward for MI355X (gfx950 / CDNA4).
//
// Kernels:
//   fp8_gemm_dma_kernel  prefill grouped GEMM (bf16 activations, tile 64):
//                     128x256 tiles, A rows / E4M3 codes / scales copied to LDS
//                     by DMA, codes decoded to bf16 in registers
//                     (v_cvt_scalef32_pk_bf16_fp8), v_mfma_f32_32x32x16_bf16,
//                     scale * partial added per 64-wide K tile
//                     (sum_k x[k] * lut[w[k]] * s[k / tile], fp8_cpu.cpp:49-98),
//                     optional SwiGLU epilogue.
//   fp8_gemm_kernel   the register-staged grouped / dense GEMM for everything
//                     else (fp32 activations, tiles 32 and 128*m, short segments).
//   decode_stream_kernel  T <= 64: units of (segment, 16 columns) streamed
//                     through a register ring, K split across the waves; the
//                     gate/up instance dispatches for itself.
//   decode_gemm_kernel    split-K decode GEMM for shapes the ring cannot take.
//   router_mfma_kernel    bf16 router logits on the matrix cores (exact three-
//                     term weight split) + softmax + top-k + renormalisation;
//   router_kernel     the fp32 router for the other shapes.
//   dispatch kernels  deterministic per-expert token order (ballot ranks);
//                     for E <= 16 the scan runs inside the scatter's blocks.
//   combine_kernel    weighted un-permute in ascending expert order;
//   combine_norm_kernel  the same followed by RMSNorm of each row;
//   combine_norm_route_kernel  and then the next layer's router on the
//                     normed rows (a chain of layers).
//   rms_norm_kernel   RMSNorm over rows.
//
// Host-side entry points are the extern "C" functions declared in
// include/smaul_rocm.h.  Nothing here allocates device memory or synchronises.
#include <hip/hip_runtime.h>
#include <stdarg.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <cmath>
#include <stdlib.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "e4m3.h"
#include "smaul_common.h"
#include "smaul_rocm.h"
#include "topk_select.h"

#define SMAUL_VERSION 100

namespace {

typedef float f32x4_t __attribute__((ext_vector_type(4)));

using smaul::check_launch;
using smaul::fail;

// ---------------------------------------------------------------------------
// scalar helpers
// ---------------------------------------------------------------------------
// fp32 -> bf16 bits, round to nearest even; NaN -> 0x7FC0 (torch's
// c10::BFloat16 conversion, the `.to(torch.bfloat16)` of the reference).
__device__ __forceinline__ uint32_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// Split an fp32 value into two bf16 terms: x ~= hi + lo (error <= 2^-18 |x|).
__device__ __forceinline__ void split_bf16(float x, uint32_t& hi, uint32_t& lo) {
  hi = f2bf(x);
  lo = f2bf(x - bf2f(hi));
}


// Loads through explicit global-address-space pointers.  Pointers read from
// memory (per-expert weight tables, gathered rows) are otherwise generic, and
// a generic (flat) load counts against both the vector-memory and the LDS
// wait counters, so the compiler drains every outstanding load before the
// next LDS access.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(1))) u32x4_t* g_u4p;
typedef const __attribute__((address_space(1))) float* g_fp;
__device__ __forceinline__ uint4 ldg16(const void* p) {
  const u32x4_t v = *(g_u4p)p;
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float ldgf(const float* p) { return *(g_fp)p; }

// Device-coherent reads of data that other workgroups of the same launch wrote
// (with agent-scope atomic stores): a raw buffer load with the
// device-scope cache policy (sc1) is served past this XCD's L2, which may hold
// a stale copy of the line.  The descriptor covers `bytes` bytes from p
// (word 3 is the gfx9 raw-buffer format).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t coh_rsrc(const void* p, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 coh_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16 /* sc1 */);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// silu(v) = v / (1 + e^-v) with the hardware exp2 and reciprocal (about two
// ulp in fp32).  Every caller rounds the result to the activation dtype or
// compares it at a tolerance far above that.
__device__ __forceinline__ float silu_f(float v) {
  const float e = __builtin_amdgcn_exp2f(-v * 1.4426950408889634f);
  return v * __builtin_amdgcn_rcpf(1.0f + e);
}

// ---------------------------------------------------------------------------
// grouped / dense FP8 GEMM
// ---------------------------------------------------------------------------
struct GemmArgs {
  const void* x;               // activations: bf16 or fp32, row stride ldx elements
  const int32_t* row_idx;      // logical row -> x row (nullptr: identity)
  int64_t ldx;
  // Per-expert weights.  If wp != nullptr the e-th expert's codes are wp[e],
  // otherwise w + e * w_estride (same for scales and the SwiGLU "up" set).
  const uint8_t* const* wp;
  const float* const* sp;
  const uint8_t* const* wp2;
  const float* const* sp2;
  const uint8_t* w;
  const float* s;
  const uint8_t* w2;
  const float* s2;
  int64_t w_estride, s_estride;
  void* y;                     // output rows in logical order, row stride ldy
  int64_t ldy;
  int64_t K, N, nt, tile;
  const int32_t* seg_off;      // [E+1] (nullptr: dense, R rows, one expert)
  const int32_t* tile_off;     // [E+1]
  int64_t R;
  int E;
  int tiled;                   // codes/scales in the tiled layout (SMAUL_FLAG_TILED_LAYOUT)
  // Weight K blocks when the activations carry two K planes (the LDS-DMA
  // GEMM of fp32 x split into bf16 hi and lo halves, K = 2 * kw): stage kt
  // reads activation block kt and weight / scale block kt mod (kw / 64).
  // 0: the weights span K.
  int64_t kw;
  // SwiGLU with fp32 output only: when > 0 the products are stored as their
  // bf16 hi / lo split (split_bf16), hi at y[row * ldy + col] and lo at
  // y[row * ldy + y_lo + col] (bf16 elements): the two planes the next GEMM
  // of fp32 activations reads.
  int64_t y_lo;
};

// Where an expert's codes and scales for column n and 64-wide K block kb
// live: codes at n * wc + kb * wk (+ k within the block), scales at
// n * sc + kb * sk.  The reference layout ([N][K] codes, [N][nt] scales:
// FP8Linear's w8 / sc) or the tiled one ([K/64][N][64] codes, [K/64][N]
// scales), in which the 64-wide K block of consecutive columns is
// contiguous: a K stage of a column tile is then whole cache lines.
struct WLayout {
  int64_t wc, wk, sc, sk;
};
__device__ __forceinline__ WLayout wlayout(const GemmArgs& p) {
  return p.tiled ? WLayout{64, p.N * 64, 1, p.N} : WLayout{p.kw ? p.kw : p.K, 64, p.nt, 1};
}

// The expert segment of m-tile mt of a grouped GEMM, with all of its loads
// in one round trip: lane j reads tile_off[j], tile_off[j + 1], seg_off[j],
// seg_off[j + 1] and expert j's pointers, and the expert is the number of
// lanes whose tiles end at or before mt (tile_off is non-decreasing).
// Dense calls (no segment table) have one expert covering rows [0, R).
// Returns false when mt is past the last tile (uniform).
struct TileSeg {
  int e, row0, rows;
  const uint8_t* w1;
  const float* s1;
  const uint8_t* w2;
  const float* s2;
};

template <int BM>
__device__ __forceinline__ bool tile_lookup(const GemmArgs& p, int mt, int lane, TileSeg& t) {
  if (!p.seg_off) {
    t.e = 0;
    t.row0 = mt * BM;
    t.rows = (int)min<int64_t>(BM, p.R - t.row0);
    t.w1 = p.wp ? p.wp[0] : p.w;
    t.s1 = p.sp ? p.sp[0] : p.s;
    t.w2 = p.wp2 ? p.wp2[0] : p.w2;
    t.s2 = p.sp2 ? p.sp2[0] : p.s2;
    return t.rows > 0;
  }
  const bool live = lane < p.E;
  const int to0 = live ? p.tile_off[lane] : 0;
  const int to1 = live ? p.tile_off[lane + 1] : 0x7fffffff;
  const int so0 = live ? p.seg_off[lane] : 0;
  const int so1 = live ? p.seg_off[lane + 1] : 0;
  uint64_t w1 = 0, s1 = 0, w2 = 0, s2 = 0;
  if (live) {
    w1 = (uint64_t)(uintptr_t)(p.wp ? p.wp[lane] : p.w + lane * p.w_estride);
    s1 = (uint64_t)(uintptr_t)(p.sp ? p.sp[lane] : p.s + lane * p.s_estride);
    if (p.wp2 || p.w2) {
      w2 = (uint64_t)(uintptr_t)(p.wp2 ? p.wp2[lane] : p.w2 + lane * p.w_estride);
      s2 = (uint64_t)(uintptr_t)(p.sp2 ? p.sp2[lane] : p.s2 + lane * p.s_estride);
    }
  }
  const int total = __builtin_amdgcn_readlane(to1, p.E - 1);
  if (mt >= total) return false;
  const int e = (int)__popcll(__ballot(to1 <= mt));
  t.e = e;
  t.row0 = __builtin_amdgcn_readlane(so0, e) + (mt - __builtin_amdgcn_readlane(to0, e)) * BM;
  t.rows = min(BM, __builtin_amdgcn_readlane(so1, e) - t.row0);
  auto lane_ptr = [&](uint64_t v) -> uint64_t {
    const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, e);
    const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(v >> 32), e);
    return ((uint64_t)hi << 32) | lo;
  };
  t.w1 = (const uint8_t*)(uintptr_t)lane_ptr(w1);
  t.s1 = (const float*)(uintptr_t)lane_ptr(s1);
  t.w2 = (const uint8_t*)(uintptr_t)lane_ptr(w2);
  t.s2 = (const float*)(uintptr_t)lane_ptr(s2);
  return t.rows > 0;
}

// KMODE: how scale tiles line up with the 64-wide K stages.
//   0: tile == 32   (two scale tiles per stage, one MFMA each)
//   1: tile == 64   (one scale tile per stage)
//   2: tile == 64*m (a scale tile spans m stages; the partial carries over)
template <int BM, int BNB, int WM, int WN, bool SWIGLU, int NSPLIT>
struct GemmCfg {
  static constexpr int NT = WM * WN * 64;
  static constexpr int BNO = SWIGLU ? BNB / 2 : BNB;   // output columns per workgroup
  static constexpr int TM = BM / WM;                   // rows per wave
  static constexpr int TNB = BNB / WN;                 // staged weight rows per wave
  static constexpr int TNO = SWIGLU ? TNB / 2 : TNB;   // output columns per wave
  static constexpr int FM = TM / 16;
  static constexpr int NJ = TNB / 16;                  // 16-wide weight tiles per wave
  static constexpr int FN = TNO / 16;                  // 16-wide output tiles per wave
  static constexpr int LDK = 64 + 8;                   // padded LDS row (bf16 elements)
  static constexpr int A_PER_ROW = NSPLIT == 1 ? 8 : 16;   // 16-byte chunks per 64-K row
  static constexpr int A_CH = BM * A_PER_ROW / NT;
  static constexpr int B_CH = BNB * 4 / NT;
  static_assert(TM % 16 == 0 && TNO % 16 == 0, "wave tile must be a multiple of 16");
  static_assert(A_CH >= 1 && (BM * A_PER_ROW) % NT == 0, "A staging split");
  static_assert(B_CH >= 1 && (BNB * 4) % NT == 0, "B staging split");
};

constexpr int GROUP_M = 8;

template <int BM, int BNB, int WM, int WN, int MT, bool REMAP, bool SWIGLU, int NSPLIT, bool OUT_BF16,
          int KMODE, bool CANON, bool VEC>
__global__ void __launch_bounds__(WM * WN * 64)
fp8_gemm_kernel(GemmArgs p) {
  using C = GemmCfg<BM, BNB, WM, WN, SWIGLU, NSPLIT>;
  static_assert(MT == 16 || MT == 32, "MFMA tile is 16x16x32 or 32x32x16");
  static_assert(C::TM % MT == 0 && C::TNO % MT == 0, "wave tile must be a multiple of the MFMA tile");
  constexpr int NT = C::NT, BNO = C::BNO, TM = C::TM, TNO = C::TNO, FM = C::FM, NJ = C::NJ,
                FN = C::FN, LDK = C::LDK, A_PER_ROW = C::A_PER_ROW, A_CH = C::A_CH,
                B_CH = C::B_CH;
  constexpr int SPS = KMODE == 0 ? 2 : 1;   // scale rows per stage
  constexpr int A_ELEMS = 64 / A_PER_ROW;

  __shared__ __attribute__((aligned(16))) uint16_t sA[2][NSPLIT][BM][LDK];
  __shared__ __attribute__((aligned(16))) uint16_t sB[2][BNB][LDK];
  __shared__ float sS[2][SPS][BNB];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  // ---- which tile does this workgroup own ----------------------------------
  // Workgroups are dispatched round-robin over the 8 XCDs (each with its own
  // L2).  Remap the linear id so each XCD walks a contiguous band of tiles,
  // then order that band in groups of GROUP_M row tiles x all column tiles,
  // column-major inside a group: the concurrently running workgroups of an
  // XCD share a few A row tiles and a few weight column tiles.
  int mt, nt_idx;
  {
    const int n_tiles = gridDim.x, m_tiles = gridDim.y;
    const int total = n_tiles * m_tiles;
    int lin = blockIdx.y * n_tiles + blockIdx.x;
    if constexpr (REMAP) {
      constexpr int NXCD = 8;
      const int full = (total / NXCD) * NXCD;
      if (lin < full) lin = (lin % NXCD) * (full / NXCD) + lin / NXCD;
      const int group = GROUP_M * n_tiles;
      const int g = lin / group, within = lin % group;
      const int m_first = g * GROUP_M;
      const int gm = min(GROUP_M, m_tiles - m_first);
      mt = m_first + within % gm;
      nt_idx = within / gm;
    } else {
      mt = lin / n_tiles;
      nt_idx = lin % n_tiles;
    }
  }
  TileSeg ts;
  if (!tile_lookup<BM>(p, mt, lane, ts)) return;  // uniform per workgroup
  const int row0 = ts.row0, rows_here = ts.rows;
  const int n0 = nt_idx * BNO;
  const int64_t K = p.K, N = p.N, nt = p.nt;
  const WLayout L = wlayout(p);

  const uint8_t* W1 = ts.w1;
  const float* S1 = ts.s1;
  const uint8_t* W2 = W1;
  const float* S2 = S1;
  if constexpr (SWIGLU) {
    W2 = ts.w2;
    S2 = ts.s2;
  }

  // ---- per-thread staging assignments --------------------------------------
  const char* arow[A_CH];
  int akoff[A_CH], arl[A_CH];
#pragma unroll
  for (int i = 0; i < A_CH; ++i) {
    const int c = tid + i * NT;
    const int r = c / A_PER_ROW;
    arl[i] = r;
    akoff[i] = (c % A_PER_ROW) * A_ELEMS;
    // Rows past the segment end load a valid row of the segment instead: MFMA
    // output rows depend only on their own A row, and those rows are never
    // stored, so the staging loop needs no branch.
    const int64_t lr = row0 + (r < rows_here ? r : rows_here - 1);
    const int64_t xr = p.row_idx ? (int64_t)p.row_idx[lr] : lr;
    arow[i] = (const char*)p.x + xr * p.ldx * (NSPLIT == 1 ? 2 : 4);
  }
  const uint8_t* brow[B_CH];
  int bkoff[B_CH], brl[B_CH];
#pragma unroll
  for (int i = 0; i < B_CH; ++i) {
    const int c = tid + i * NT;
    const int r = c >> 2;
    brl[i] = r;
    bkoff[i] = (c & 3) * 16;
    const bool up = SWIGLU && r >= BNO;
    int64_t col = n0 + (up ? r - BNO : r);
    if (col >= N) col = N - 1;  // columns past N are computed but never stored
    brow[i] = (up ? W2 : W1) + col * L.wc;
  }
  // scale staging: slot q = tid + i*NT < SPS * BNB owns (sub, column)
  constexpr int S_CH = (SPS * BNB + NT - 1) / NT;
  const float* srow[S_CH];
  int s_sub[S_CH], s_col[S_CH];
  bool s_own[S_CH];
#pragma unroll
  for (int i = 0; i < S_CH; ++i) {
    const int q = tid + i * NT;
    s_own[i] = q < SPS * BNB;
    s_sub[i] = (q / BNB) % SPS;
    s_col[i] = q % BNB;
    const bool up = SWIGLU && s_col[i] >= BNO;
    int64_t col = n0 + (up ? s_col[i] - BNO : s_col[i]);
    if (col >= N) col = N - 1;
    srow[i] = (up ? S2 : S1) + col * L.sc;
  }
  // K % 64 == 0: every stage is full and the loads need no K guard
  const bool full_k = (K & 63) == 0;

  uint4 ra[A_CH];
  uint4 rb[B_CH];
  float rs[S_CH];

  auto load_stage = [&](int64_t kt) {
    const int64_t k0 = kt * 64;
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int64_t kk = k0 + akoff[i];
      if constexpr (VEC) {
        ra[i] = (full_k || kk < K) ? ldg16(arow[i] + kk * (NSPLIT == 1 ? 2 : 4)) : make_uint4(0, 0, 0, 0);
      } else {
        uint32_t v[4] = {0, 0, 0, 0};
        {
          if constexpr (NSPLIT == 1) {
            const uint16_t* src = (const uint16_t*)arow[i];
#pragma unroll
            for (int q = 0; q < 8; ++q)
              if (kk + q < K) v[q >> 1] |= (uint32_t)src[kk + q] << ((q & 1) * 16);
          } else {
            const uint32_t* src = (const uint32_t*)arow[i];
#pragma unroll
            for (int q = 0; q < 4; ++q)
              if (kk + q < K) v[q] = src[kk + q];
          }
        }
        ra[i] = make_uint4(v[0], v[1], v[2], v[3]);
      }
    }
#pragma unroll
    for (int i = 0; i < B_CH; ++i) {
      const int64_t kk = k0 + bkoff[i];
      if constexpr (VEC) {
        // (the tiled layout needs K % 64 == 0: kk < K always)
        rb[i] = (full_k || kk < K) ? ldg16(brow[i] + kt * L.wk + bkoff[i]) : make_uint4(0, 0, 0, 0);
      } else {
        uint32_t v[4] = {0, 0, 0, 0};
        {
#pragma unroll
          for (int q = 0; q < 16; ++q)
            if (kk + q < K) v[q >> 2] |= (uint32_t)brow[i][kk + q] << ((q & 3) * 8);
        }
        rb[i] = make_uint4(v[0], v[1], v[2], v[3]);
      }
    }
#pragma unroll
    for (int i = 0; i < S_CH; ++i) {
      int64_t kb;
      if constexpr (KMODE == 0) kb = kt * 2 + s_sub[i];
      else if constexpr (KMODE == 1) kb = kt;
      else kb = k0 / p.tile;
      rs[i] = ldgf(srow[i] + (kb < nt ? kb : nt - 1) * L.sk);  // kb == nt only past K (zero data)
    }
  };

  auto store_stage = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      if constexpr (NSPLIT == 1) {
        *(uint4*)&sA[buf][0][arl[i]][akoff[i]] = ra[i];
      } else {
        const float f[4] = {__uint_as_float(ra[i].x), __uint_as_float(ra[i].y),
                            __uint_as_float(ra[i].z), __uint_as_float(ra[i].w)};
        uint32_t h[4], l[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) split_bf16(f[q], h[q], l[q]);
        *(uint2*)&sA[buf][0][arl[i]][akoff[i]] = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
        *(uint2*)&sA[buf][NSPLIT - 1][arl[i]][akoff[i]] =
            make_uint2(l[0] | (l[1] << 16), l[2] | (l[3] << 16));
      }
    }
#pragma unroll
    for (int i = 0; i < B_CH; ++i) {
      uint32_t d[8];
      decode4<CANON>(rb[i].x, d[0], d[1]);
      decode4<CANON>(rb[i].y, d[2], d[3]);
      decode4<CANON>(rb[i].z, d[4], d[5]);
      decode4<CANON>(rb[i].w, d[6], d[7]);
      uint4* dst = (uint4*)&sB[buf][brl[i]][bkoff[i]];
      dst[0] = make_uint4(d[0], d[1], d[2], d[3]);
      dst[1] = make_uint4(d[4], d[5], d[6], d[7]);
    }
#pragma unroll
    for (int i = 0; i < S_CH; ++i)
      if (s_own[i]) sS[buf][s_sub[i]][s_col[i]] = rs[i];
  };

  // ---- accumulators --------------------------------------------------------
  // MT x MT output tiles: FMT row tiles x NJT weight tiles per wave; an MT=16
  // tile holds 4 fp32 per lane, an MT=32 tile 16.
  constexpr int FMT = TM / MT, NJT = (C::TNB) / MT, FNT = TNO / MT, NACC = MT * MT / 64;
  typedef float accv_t __attribute__((ext_vector_type(NACC)));
  accv_t acc[FMT][NJT];
#pragma unroll
  for (int i = 0; i < FMT; ++i)
#pragma unroll
    for (int j = 0; j < NJT; ++j)
#pragma unroll
      for (int r = 0; r < NACC; ++r) acc[i][j][r] = 0.0f;
  [[maybe_unused]] accv_t part[KMODE == 2 ? FMT : 1][KMODE == 2 ? NJT : 1];
  if constexpr (KMODE == 2) {
#pragma unroll
    for (int i = 0; i < FMT; ++i)
#pragma unroll
      for (int j = 0; j < NJT; ++j)
#pragma unroll
        for (int r = 0; r < NACC; ++r) part[i][j][r] = 0.0f;
  }

  // LDS row (inside sB) of weight tile j for this lane
  int bl_row[NJT];
#pragma unroll
  for (int j = 0; j < NJT; ++j) {
    const bool up = SWIGLU && j >= FNT;
    const int jj = up ? j - FNT : j;
    bl_row[j] = (up ? BNO : 0) + wn * TNO + jj * MT + (lane & (MT - 1));
  }
  const int a_row_base = wm * TM + (lane & (MT - 1));
  // k offset of this lane inside one MFMA k-step (8 bf16 per lane)
  const int k_lane = MT == 16 ? (lane >> 4) * 8 : (lane >> 5) * 8;
  constexpr int KSTEP = MT == 16 ? 32 : 16;     // K per MFMA
  constexpr int NKS = 64 / KSTEP;               // MFMA k-steps per stage
  constexpr int KS_PER_TILE32 = 32 / KSTEP;     // k-steps per 32-wide scale tile (KMODE 0)
  accv_t zacc;
#pragma unroll
  for (int r = 0; r < NACC; ++r) zacc[r] = 0.0f;

  auto mfma = [&](const bf16x8_t& a, const bf16x8_t& b, const accv_t& c) -> accv_t {
    if constexpr (MT == 16) return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    else return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  };

  const int64_t nk = (K + 63) / 64;

  auto compute_stage = [&](int64_t kt) {
    const int cur = (int)(kt & 1);
    bf16x8_t af[NKS][NSPLIT][FMT];
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
      for (int sp = 0; sp < NSPLIT; ++sp)
#pragma unroll
        for (int i = 0; i < FMT; ++i)
          af[ks][sp][i] = *(const bf16x8_t*)&sA[cur][sp][a_row_base + i * MT][ks * KSTEP + k_lane];
    bool tile_start = true, tile_end = true;
    if constexpr (KMODE == 2) {
      tile_start = ((kt * 64) % p.tile) == 0;
      tile_end = (((kt + 1) * 64) % p.tile) == 0 || kt == nk - 1;
    }
#pragma unroll
    for (int j = 0; j < NJT; ++j) {
      bf16x8_t bf[NKS];
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) bf[ks] = *(const bf16x8_t*)&sB[cur][bl_row[j]][ks * KSTEP + k_lane];
      const float sc0 = sS[cur][0][bl_row[j]];
      const float sc1 = sS[cur][SPS - 1][bl_row[j]];
#pragma unroll
      for (int i = 0; i < FMT; ++i) {
        if constexpr (KMODE == 0) {
#pragma unroll
          for (int half = 0; half < 2; ++half) {
            accv_t q = zacc;
#pragma unroll
            for (int ks = half * KS_PER_TILE32; ks < (half + 1) * KS_PER_TILE32; ++ks)
#pragma unroll
              for (int sp = 0; sp < NSPLIT; ++sp) q = mfma(af[ks][sp][i], bf[ks], q);
            const float sc = half ? sc1 : sc0;
#pragma unroll
            for (int r = 0; r < NACC; ++r) acc[i][j][r] = __builtin_fmaf(sc, q[r], acc[i][j][r]);
          }
        } else {
          accv_t q = zacc;
          if constexpr (KMODE == 2) q = tile_start ? zacc : part[i][j];
#pragma unroll
          for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
            for (int sp = 0; sp < NSPLIT; ++sp) q = mfma(af[ks][sp][i], bf[ks], q);
          if constexpr (KMODE == 1) {
#pragma unroll
            for (int r = 0; r < NACC; ++r) acc[i][j][r] = __builtin_fmaf(sc0, q[r], acc[i][j][r]);
          } else {
            if (tile_end) {
#pragma unroll
              for (int r = 0; r < NACC; ++r) acc[i][j][r] = __builtin_fmaf(sc0, q[r], acc[i][j][r]);
            }
            part[i][j] = q;
          }
        }
      }
    }
  };

  // Two LDS buffers: stage kt+1 is fetched into registers while stage kt is
  // computed, then decoded into the other buffer.  The last stage is peeled so
  // the loop body has no conditional load/store.
  load_stage(0);
  store_stage(0);
  __syncthreads();
  for (int64_t kt = 0; kt + 1 < nk; ++kt) {
    load_stage(kt + 1);
    // Scheduling fences: keep the next stage's global loads ahead of this
    // stage's MFMAs and its LDS stores (which wait for those loads) after
    // them, so the load latency overlaps a whole stage of compute.
    __builtin_amdgcn_sched_barrier(0);
    compute_stage(kt);
    __builtin_amdgcn_sched_barrier(0);
    store_stage((int)((kt + 1) & 1));
    __syncthreads();
  }
  compute_stage(nk - 1);

  // ---- epilogue ------------------------------------------------------------
  // MFMA output layout: lane holds column (lane % MT) of its tile; for MT=16
  // rows (lane/16)*4 + r, for MT=32 rows (r/4)*8 + (lane/32)*4 + r%4.
#pragma unroll
  for (int i = 0; i < FMT; ++i) {
#pragma unroll
    for (int r = 0; r < NACC; ++r) {
      const int rin = MT == 16 ? (lane >> 4) * 4 + r : (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
      const int lr = wm * TM + i * MT + rin;
      if (lr >= rows_here) continue;
      const int64_t orow = row0 + lr;
#pragma unroll
      for (int j = 0; j < FNT; ++j) {
        const int64_t col = n0 + wn * TNO + j * MT + (lane & (MT - 1));
        if (col >= N) continue;
        float v;
        if constexpr (SWIGLU) {
          float g = acc[i][j][r], u = acc[i][j + FNT][r];
          if constexpr (OUT_BF16) {
            g = bf2f(f2bf(g));
            u = bf2f(f2bf(u));
          }
          v = silu_f(g) * u;
        } else {
          v = acc[i][j][r];
        }
        if constexpr (OUT_BF16) {
          ((uint16_t*)p.y)[orow * p.ldy + col] = (uint16_t)f2bf(v);
        } else {
          ((float*)p.y)[orow * p.ldy + col] = v;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// grouped GEMM for bf16 activations and 64-wide scale tiles: LDS-DMA staging,
// per-wave decode, NSTAGE-deep pipeline
// ---------------------------------------------------------------------------
// Per 64-wide K stage a workgroup stages BM activation rows (bf16, 128 B per
// row), BN weight columns (raw E4M3 codes, 64 B per column) and the BN fp32
// scales of that K tile straight from global memory into LDS with
// global_load_lds_dwordx4 / _dword: no staging registers and no VALU work.
// Each wave then reads its A fragments and its raw codes from LDS, decodes the
// codes to bf16 in registers (v_cvt_scalef32_pk_bf16_fp8) and runs
// v_mfma_f32_32x32x16_bf16.  Codes (1 B) instead of decoded bf16 (2 B) in LDS
// halve the weight side of the LDS traffic and footprint.  NSTAGE stages are
// in flight: the loads of stage kt + NSTAGE - 1 are issued while stage kt is
// computed, so the load latency is covered by NSTAGE - 1 stages of MFMA work.
//
// K order inside a stage: lane group g = lane / 32 feeds the MFMA k-slots
// 8g..8g+7 of k-step ks with the actual k = (4g + ks) * 8 + 0..7, for A and
// for B alike.  The four k-steps of a stage therefore cover the 64 k of one
// scale tile exactly once; the partial sum of the stage is the same set of
// exact bf16 x bf16 products, and each lane's A bytes (64) and code bytes (32)
// of a stage are contiguous.
//
// LDS rows keep their 16-byte chunks XOR-swizzled by row index, so the 32
// consecutive rows that one fragment read touches fall in distinct banks both
// for 32 banks read 8 lanes at a time and for 64 banks read 16 at a time.
__device__ __forceinline__ int swz_a(int r) { return (r & 6) | ((r ^ (r >> 3)) & 1); }        // 8 chunks
__device__ __forceinline__ int swz_b(int r) { return ((r >> 1) & 2) | (((r >> 1) ^ (r >> 3)) & 1); }  // 4

typedef __attribute__((address_space(3))) void* lds_vptr_t;

__device__ __forceinline__ uint32_t lds_offset(const void* p) { return (uint32_t)(uintptr_t)(lds_vptr_t)p; }

// LDS DMA: each lane copies 16 (or 4) bytes from base + off to LDS address
// lds + 16 (or 4) * lane.  Issued as inline asm so the compiler's wait-count
// pass does not treat every later LDS read as dependent on it (it cannot tell
// the stage buffers apart); the kernels wait for it explicitly (vmcnt) before
// the barrier that publishes a buffer.  M0 holds the LDS address (all 32 bits
// are used: addresses above 64 KB land where they should on gfx950); nothing
// else in these kernels uses M0.
// The base address is wave-uniform by construction; readfirstlane makes that
// explicit so it always lands in scalar registers.
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
__device__ __forceinline__ void dma4(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2"
               :: "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(off), "s"(uniform_ptr(base)) : "memory");
}
// wait until at most N of this wave's vector-memory loads are outstanding
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}

typedef float f32x16_t __attribute__((ext_vector_type(16)));


template <int BM, int BN, int WM, int WN, int NSTAGE, bool SWIGLU, bool X32 = false>
struct DmaGemmCfg {
  static constexpr int NW = WM * WN;
  static constexpr int BNO = SWIGLU ? BN / 2 : BN;       // output columns per workgroup
  static constexpr int TM = BM / WM;                     // rows per wave
  static constexpr int TN = BN / WN;                     // staged weight columns per wave
  static constexpr int TNO = SWIGLU ? TN / 2 : TN;       // output columns per wave
  static constexpr int FM = TM / 32, FN = TN / 32, FNO = TNO / 32;
  // X32: the activation rows arrive as fp32 (256 B per 64-wide K block) and
  // are split in place into a bf16 hi plane and a lo plane of 128 B rows
  static constexpr int A_BYTES = BM * 128 * (X32 ? 2 : 1), B_BYTES = BN * 64, S_BYTES = BN * 4;
  static constexpr int STAGE = A_BYTES + B_BYTES + S_BYTES;
  static constexpr int A_INS = A_BYTES / 1024 / NW;      // 1 KB DMA instructions per wave per stage
  static constexpr int B_INS = B_BYTES / 1024 / NW;
  static constexpr int S_INS = BN / 64;                  // 256 B scale DMAs per stage, waves 0..S_INS-1
  static constexpr int DMA_MIN = A_INS + B_INS;          // DMAs per stage issued by every wave
  // Row tiles per L2 group of the tile order (the remap below): gate/up walks
  // 4 row tiles x all column tiles, down 8 (measured best for each at the
  // C5 shape, d = 2048 / h = 5120, and no different at C3).
  static constexpr int GM = SWIGLU ? 4 : GROUP_M;
  static constexpr int OUT_LD = BNO + 8;                 // plain epilogue LDS row (bf16 elements)
  static constexpr int LDS = (SWIGLU || NSTAGE * STAGE > BM * OUT_LD * 2) ? NSTAGE * STAGE : BM * OUT_LD * 2;
  static_assert(TM % 32 == 0 && TNO % 32 == 0, "wave tile must be a multiple of 32");
  static_assert(A_INS >= 1 && A_BYTES % (1024 * NW) == 0, "A staging split");
  static_assert(B_INS >= 1 && B_BYTES % (1024 * NW) == 0, "B staging split");
  static_assert(S_INS <= NW && BN % 64 == 0, "scale staging split");
  static_assert(!SWIGLU || BNO % 64 == 0, "gate/up halves must not share a DMA instruction");
  static_assert(NSTAGE >= 2 && DMA_MIN * (NSTAGE - 2) < 64, "pipeline depth");
  static_assert(LDS <= 160 * 1024, "LDS budget");
};

// OUT_F32: the fp32 sums are stored as they are (the dense fp8_forward
// contract), straight from the MFMA layout; with SWIGLU, silu(gate) * up in
// fp32 (SwiFFN with fp32 activations, whose products the reference keeps in
// fp32).  Otherwise the sums are rounded to bf16 and stored through LDS
// (plain) or, with the SwiGLU epilogue, as 8-byte row pieces after an
// exchange inside each quad of lanes.
//
// X32 (OUT_F32 only): fp32 activations.  The stage's rows are staged as fp32
// and, after its barrier, split in place by all threads into x = hi + lo
// (split_bf16, |x - hi - lo| <= 2^-18 |x|) in two bf16 planes of the usual
// layout; each k-step then runs hi and lo MFMAs into the same partial, so the
// scale multiplies s * (hi . w + lo . w) per 64-wide K block.
template <int BM, int BN, int WM, int WN, int NSTAGE, bool SWIGLU, bool CANON, bool REMAP, bool OUT_F32 = false,
          bool X32 = false>
// Tiles of at most 128 x 128 staged columns fit three workgroups per CU.
__global__ void __launch_bounds__(WM * WN * 64, (BM * BN <= 128 * 128 ? 3 : 2))
fp8_gemm_dma_kernel(GemmArgs p) {
  static_assert(!X32 || (OUT_F32 && !SWIGLU), "fp32 activations split in LDS are the fp8_forward path");
  using C = DmaGemmCfg<BM, BN, WM, WN, NSTAGE, SWIGLU, X32>;
  constexpr int NW = C::NW, BNO = C::BNO, TM = C::TM, TN = C::TN, TNO = C::TNO, FM = C::FM, FN = C::FN,
                FNO = C::FNO, A_BYTES = C::A_BYTES, B_BYTES = C::B_BYTES, STAGE = C::STAGE,
                A_INS = C::A_INS, B_INS = C::B_INS, S_INS = C::S_INS;

  __shared__ __attribute__((aligned(1024))) char smem[C::LDS];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: DMA bases are scalar
  const int wm = wave / WN, wn = wave % WN;

  int mt, nt_idx;
  {
    const int n_tiles = gridDim.x, m_tiles = gridDim.y;
    const int total = n_tiles * m_tiles;
    int lin = blockIdx.y * n_tiles + blockIdx.x;
    if constexpr (REMAP) {
      constexpr int NXCD = 8;
      const int full = (total / NXCD) * NXCD;
      if (lin < full) lin = (lin % NXCD) * (full / NXCD) + lin / NXCD;
      const int group = C::GM * n_tiles;
      const int g = lin / group, within = lin % group;
      const int m_first = g * C::GM;
      const int gm = min(C::GM, m_tiles - m_first);
      mt = m_first + within % gm;
      nt_idx = within / gm;
    } else {
      mt = lin / n_tiles;
      nt_idx = lin % n_tiles;
    }
  }
  TileSeg ts;
  if (!tile_lookup<BM>(p, mt, lane, ts)) return;  // uniform per workgroup
  const int row0 = ts.row0, rows_here = ts.rows;
  const int n0 = nt_idx * BNO;
  const int64_t K = p.K;
  const WLayout L = wlayout(p);

  const uint8_t* W1 = ts.w1;
  const float* S1 = ts.s1;
  const uint8_t* W2 = W1;
  const float* S2 = S1;
  if constexpr (SWIGLU) {
    W2 = ts.w2;
    S2 = ts.s2;
  }

  // ---- DMA source offsets of this lane (32-bit; the host checks the range) --
  // A instruction q stages rows 8q..8q+7: lane -> row 8q + lane/8, LDS chunk
  // lane%8, which holds logical chunk (lane%8) ^ swz_a(row).  Rows past the
  // segment end load the segment's last row: MFMA output rows depend only on
  // their own A row and those rows are never stored.
  // X32: instruction q stages fp32 rows 4q..4q+3 unswizzled (lane -> row
  // 4q + lane/16, 16-byte chunk lane%16); the split writes the swizzled planes.
  uint32_t a_off[A_INS];
#pragma unroll
  for (int a = 0; a < A_INS; ++a) {
    if constexpr (X32) {
      const int r = (wave * A_INS + a) * 4 + (lane >> 4);
      const int64_t lr = row0 + (r < rows_here ? r : rows_here - 1);
      const int64_t xr = p.row_idx ? (int64_t)p.row_idx[lr] : lr;
      a_off[a] = (uint32_t)(xr * p.ldx * 4 + (lane & 15) * 16);
    } else {
      const int r = (wave * A_INS + a) * 8 + (lane >> 3);
      const int c = (lane & 7) ^ swz_a(r);
      const int64_t lr = row0 + (r < rows_here ? r : rows_here - 1);
      const int64_t xr = p.row_idx ? (int64_t)p.row_idx[lr] : lr;
      a_off[a] = (uint32_t)(xr * p.ldx * 2 + c * 16);
    }
  }
  // B instruction q stages weight columns 16q..16q+15 (64 B each).  The host
  // guarantees N % BNO == 0, so every staged column exists, the gate and up
  // halves of a SwiGLU tile never share an instruction, and the lane's source
  // offset is the same for all of its instructions (the swizzle depends only
  // on row bits 1..3): the instruction's column block goes into the scalar
  // base.
  uint32_t b_off;
  {
    const int r = lane >> 2;
    b_off = (uint32_t)(r * L.wc + (((lane & 3) ^ swz_b(r)) << 4));
  }
  auto b_src = [&](int b) -> const uint8_t* {
    const int q = wave * B_INS + b;
    const bool up = SWIGLU && q * 16 >= BNO;
    const int64_t col0 = n0 + (up ? q * 16 - BNO : q * 16);
    return (up ? W2 : W1) + col0 * L.wc;
  };
  // scale instruction `wave` (waves < S_INS) stages columns 64*wave + lane
  const float* s_src = S1;
  if (wave < S_INS) {
    const bool up = SWIGLU && wave * 64 >= BNO;
    s_src = (up ? S2 : S1) + (n0 + (up ? wave * 64 - BNO : wave * 64)) * L.sc;
  }
  const uint32_t s_off = (uint32_t)(lane * L.sc * 4);

  // The K advance of a stage goes into the (scalar) base addresses; the
  // per-lane offsets stay fixed.  Every wave issues DMA_MIN = A_INS + B_INS
  // loads per stage, waves < S_INS one more (the scales, issued first).
  const uint32_t lds0 = lds_offset(&smem[0]);
  const int kwb = (int)(p.kw >> 6);  // weight K blocks of a two-plane activation (0: none)
  auto dma_stage = [&](int kt, int buf) {
    const uint32_t lbase = lds0 + (uint32_t)(buf * STAGE);
    const int kb = kt >= kwb && kwb > 0 ? kt - kwb : kt;  // the weight block of activation block kt
    if (S_INS == NW || wave < S_INS) dma4(s_src + kb * L.sk, s_off, lbase + A_BYTES + B_BYTES + wave * 256);
    const char* xa = (const char*)p.x + kt * (X32 ? 256 : 128);
#pragma unroll
    for (int a = 0; a < A_INS; ++a) dma16(xa, a_off[a], lbase + (wave * A_INS + a) * 1024);
#pragma unroll
    for (int b = 0; b < B_INS; ++b) dma16(b_src(b) + kb * L.wk, b_off, lbase + A_BYTES + (wave * B_INS + b) * 1024);
  };

  // ---- fragment addresses (fixed over K) -----------------------------------
  // Row tiles are 32 rows apart and the swizzles depend only on row bits 0..3,
  // so tile i / j adds a constant to the addresses of tile 0.
  const int g = lane >> 5, l32 = lane & 31;
  int a_addr[4];
  {
    const int r = wm * TM + l32;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) a_addr[ks] = r * 128 + (((g * 4 + ks) ^ swz_a(r)) << 4);
  }
  auto b_row = [&](int j) -> int {  // staged weight row of tile j (lane 0)
    if constexpr (SWIGLU) return j < FNO ? wn * TNO + j * 32 : BNO + wn * TNO + (j - FNO) * 32;
    else return wn * TN + j * 32;
  };
  int b_addr[2];
  const int s_addr = A_BYTES + B_BYTES + (b_row(0) + l32) * 4;
  {
    const int r = b_row(0) + l32;
    b_addr[0] = A_BYTES + r * 64 + (((g * 2) ^ swz_b(r)) << 4);
    b_addr[1] = A_BYTES + r * 64 + (((g * 2 + 1) ^ swz_b(r)) << 4);
  }

  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  f32x16_t zacc;
#pragma unroll
  for (int r = 0; r < 16; ++r) zacc[r] = 0.0f;

  // One stage: both column tiles' codes decoded first (B fragments for all
  // FN tiles), then the FM x FN 32x32 tiles in order t = i * FN + j.  The
  // MFMA chain of tile t is issued before the scale FMAs of tile t - 1, which
  // by then have their partial: the matrix core works on tile t while the
  // VALU applies the previous tile's scales (a wave issues in order, so the
  // reverse order would leave one unit idle while the other works).  A
  // fragments are held for two row tiles at a time, the next one read from
  // LDS while the current one is used.
  auto compute_stage = [&](int buf) {
    const char* base = smem + buf * STAGE;
    bf16x8_t bfr[FN][4];
    float sc[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int dj = b_row(j) - b_row(0);
      const uint4 c0 = *(const uint4*)(base + b_addr[0] + dj * 64);
      const uint4 c1 = *(const uint4*)(base + b_addr[1] + dj * 64);
      sc[j] = *(const float*)(base + s_addr + dj * 4);
      uint32_t d[16];
      decode4<CANON>(c0.x, d[0], d[1]);
      decode4<CANON>(c0.y, d[2], d[3]);
      decode4<CANON>(c0.z, d[4], d[5]);
      decode4<CANON>(c0.w, d[6], d[7]);
      decode4<CANON>(c1.x, d[8], d[9]);
      decode4<CANON>(c1.y, d[10], d[11]);
      decode4<CANON>(c1.z, d[12], d[13]);
      decode4<CANON>(c1.w, d[14], d[15]);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        bfr[j][ks] = __builtin_bit_cast(bf16x8_t, make_uint4(d[4 * ks], d[4 * ks + 1], d[4 * ks + 2], d[4 * ks + 3]));
    }
    bf16x8_t af[2][4];
    bf16x8_t afl[X32 ? 2 : 1][4];  // X32: the lo plane, BM * 128 bytes after the hi plane
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      af[0][ks] = *(const bf16x8_t*)(base + a_addr[ks]);
      if constexpr (X32) afl[0][ks] = *(const bf16x8_t*)(base + BM * 128 + a_addr[ks]);
    }
    f32x16_t qp;
#pragma unroll
    for (int t = 0; t < FM * FN; ++t) {
      const int i = t / FN, j = t % FN;
      if (j == 0 && i + 1 < FM) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          af[(i + 1) & 1][ks] = *(const bf16x8_t*)(base + a_addr[ks] + (i + 1) * 32 * 128);
          if constexpr (X32)
            afl[(i + 1) & 1][ks] = *(const bf16x8_t*)(base + BM * 128 + a_addr[ks] + (i + 1) * 32 * 128);
        }
      }
      // one MFMA of tile t, then four of tile t - 1's FMAs, four times over;
      // the scheduling fences keep that order
      f32x16_t q = zacc;
      const int pi = (t - 1) / FN, pj = (t - 1) % FN;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        q = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i & 1][ks], bfr[j][ks], q, 0, 0, 0);
        if constexpr (X32) q = __builtin_amdgcn_mfma_f32_32x32x16_bf16(afl[i & 1][ks], bfr[j][ks], q, 0, 0, 0);
        if (t > 0) {
#pragma unroll
          for (int r = ks * 4; r < ks * 4 + 4; ++r) acc[pi][pj][r] = __builtin_fmaf(sc[pj], qp[r], acc[pi][pj][r]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      qp = q;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[FM - 1][FN - 1][r] = __builtin_fmaf(sc[FN - 1], qp[r], acc[FM - 1][FN - 1][r]);
  };

  // X32: the split of stage buffer b's fp32 rows into the hi and lo planes, in
  // place (every thread reads its EPT consecutive values of one row, a
  // barrier, then writes their two bf16 halves to the swizzled planes, and a
  // barrier publishes them).
  auto split_stage = [&](int b) {
    if constexpr (X32) {
      constexpr int EPT = BM * 64 / (NW * 64), TPR = 64 / EPT;
      static_assert(EPT % 8 == 0 && EPT * TPR == 64, "whole 16-byte chunks per thread");
      char* base = smem + b * STAGE;
      const int r = tid / TPR, k0 = (tid % TPR) * EPT;
      float v[EPT];
#pragma unroll
      for (int q = 0; q < EPT / 4; ++q) {
        const float4 f = *(const float4*)(base + r * 256 + (k0 + 4 * q) * 4);
        v[4 * q] = f.x;
        v[4 * q + 1] = f.y;
        v[4 * q + 2] = f.z;
        v[4 * q + 3] = f.w;
      }
      __syncthreads();
#pragma unroll
      for (int c = 0; c < EPT / 8; ++c) {
        uint32_t h[8], l[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) split_bf16(v[8 * c + e], h[e], l[e]);
        const int pc = ((k0 / 8 + c) ^ swz_a(r)) << 4;
        *(uint4*)(base + r * 128 + pc) =
            make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
        *(uint4*)(base + BM * 128 + r * 128 + pc) =
            make_uint4(l[0] | (l[1] << 16), l[2] | (l[3] << 16), l[4] | (l[5] << 16), l[6] | (l[7] << 16));
      }
      __syncthreads();
    }
  };

  // ---- the pipeline ----------------------------------------------------------
  // At the top of iteration kt this wave has the loads of stages
  // kt .. kt+NSTAGE-2 in flight; waiting until at most (NSTAGE-2)*DMA_MIN are
  // outstanding completes stage kt (a wave with the extra scale load may also
  // wait for the oldest load of the next stage, which is only conservative).
  // The barrier then publishes stage kt and tells every wave that buffer
  // (kt-1) % NSTAGE, computed in the previous iteration, may be refilled.
  // Stages past the end re-load the last stage into a buffer nobody reads
  // again, so the loop body has no branch around its loads (a branch costs
  // registers and spills).
  const int nk = (int)(K >> 6);
#pragma unroll
  for (int s = 0; s + 1 < NSTAGE; ++s) dma_stage(s < nk ? s : nk - 1, s);
  int buf = 0, nbuf = NSTAGE - 1;
  for (int kt = 0; kt < nk; ++kt) {
    wait_vm<C::DMA_MIN * (NSTAGE - 2)>();
    __syncthreads();
    const int ks = kt + NSTAGE - 1;
    dma_stage(ks < nk ? ks : nk - 1, nbuf);
    split_stage(buf);
    compute_stage(buf);
    buf = buf + 1 == NSTAGE ? 0 : buf + 1;
    nbuf = nbuf + 1 == NSTAGE ? 0 : nbuf + 1;
  }
  wait_vm<0>();
  if constexpr (OUT_F32) {
    // A lane holds column l32 of each 32x32 tile, rows (r/4)*8 + g*4 + r%4:
    // each store instruction writes 128 contiguous bytes of two rows.  SwiGLU:
    // tile j (gate) and tile j + FNO (up) hold the same output columns; split
    // into planes (y_lo > 0), the register epilogue below stores them.
    if (!SWIGLU || p.y_lo == 0) {  // uniform
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FNO; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int lr = wm * TM + i * 32 + (r >> 2) * 8 + g * 4 + (r & 3);
            float v = acc[i][j][r];
            if constexpr (SWIGLU) v = silu_f(v) * acc[i][j + FNO][r];
            if (lr < rows_here) ((float*)p.y)[(int64_t)(row0 + lr) * p.ldy + n0 + wn * TNO + j * 32 + l32] = v;
          }
      return;
    }
  }

  if constexpr (!SWIGLU) {
    // ---- plain epilogue: through LDS, then 16-byte row stores ---------------
    // (measured faster than the register exchange below for 256 outputs per
    // workgroup: half as many store instructions, whole 512-byte rows)
    // A lane holds column l32 of each 32x32 tile, rows (r/4)*8 + g*4 + r%4;
    // the tile is rounded to bf16, written to LDS as [row][col] and stored
    // row by row.
    __syncthreads();  // every wave is done with the stage buffers
    constexpr int OUT_LD = C::OUT_LD;
    uint16_t* so = (uint16_t*)smem;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int j = 0; j < FNO; ++j) {
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
          const uint32_t o = pack_bf16(acc[i][j][r], acc[i][j][r + 1]);
          const int lr = wm * TM + i * 32 + (r >> 2) * 8 + g * 4 + (r & 3);  // r even: rows lr, lr+1
          const int lc = wn * TNO + j * 32 + l32;
          so[lr * OUT_LD + lc] = (uint16_t)(o & 0xffffu);
          so[(lr + 1) * OUT_LD + lc] = (uint16_t)(o >> 16);
        }
      }
    }
    __syncthreads();
    constexpr int CPR = BNO / 8;  // 16-byte chunks per output row
    for (int c = tid; c < BM * CPR; c += NW * 64) {
      const int row = c / CPR, ch = c - row * CPR;
      if (row < rows_here)
        *(uint4*)((uint16_t*)p.y + (int64_t)(row0 + row) * p.ldy + n0 + ch * 8) =
            *(const uint4*)(so + row * OUT_LD + ch * 8);
    }
    return;
  }

  // ---- SwiGLU epilogue: bf16 rows stored from registers ---------------------
  // A lane holds column l32 of each 32x32 tile, rows (r/4)*8 + g*4 + r%4.
  // Gate and up are rounded to bf16 first, as the reference's FP8Linear
  // outputs are, then silu(gate)*up is rounded again (OUT_F32, the planes of
  // fp32 activations: silu(gate)*up in fp32, stored as its bf16 hi and lo
  // terms, split_bf16).  Two exchanges inside each quad of lanes (DPP quad
  // permutes, no LDS, no barrier) turn a lane's four rows x one column into
  // one row x four columns: lane 4m+s ends with row (r/4)*8 + g*4 + s,
  // columns 4m..4m+3, so the 8 lanes of a row store 64 contiguous bytes and
  // the WN waves complete the row.
  const int qs = lane & 3;
  const bool hi2 = (lane & 2) != 0;
  // v_perm selectors for the lane ^ 1 step (src0 = partner, src1 = own):
  // even lanes take own bytes 0-1 then partner bytes 0-1, odd lanes partner
  // bytes 2-3 then own bytes 2-3
  const uint32_t psel = (lane & 1) ? 0x03020706u : 0x05040100u;
  // d0 = rows +0 (low half), +1 (high half) of column l32, d1 = rows +2, +3
  // -> this lane's row piece (columns 4m..4m+3 of row +s)
  auto exchange = [&](uint32_t d0, uint32_t d1) -> uint2 {
    // lane ^ 1: even lanes take rows +0 / +2 of columns (c, c+1), odd
    // lanes rows +1 / +3 of columns (c-1, c)
    const uint32_t e0 =
        __builtin_amdgcn_perm((uint32_t)__builtin_amdgcn_mov_dpp((int)d0, 0xB1, 0xF, 0xF, false), d0, psel);
    const uint32_t e1 =
        __builtin_amdgcn_perm((uint32_t)__builtin_amdgcn_mov_dpp((int)d1, 0xB1, 0xF, 0xF, false), d1, psel);
    // lane ^ 2: lanes s < 2 keep row +s (e0) and take columns 4m+2..4m+3
    // of it; lanes s >= 2 keep row +s (e1) and take columns 4m..4m+1
    const uint32_t rv = (uint32_t)__builtin_amdgcn_mov_dpp((int)(hi2 ? e0 : e1), 0x4E, 0xF, 0xF, false);
    return make_uint2(hi2 ? rv : e0, hi2 ? e1 : rv);
  };
#pragma unroll
  for (int i = 0; i < FM; ++i) {
#pragma unroll
    for (int j = 0; j < FNO; ++j) {
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int r = a * 4 + q;
          if constexpr (OUT_F32) {
            v[q] = silu_f(acc[i][j][r]) * acc[i][j + FNO][r];
          } else {
            const uint32_t gu = pack_bf16(acc[i][j][r], acc[i][j + FNO][r]);  // gate, up rounded to bf16
            const float gr = __builtin_bit_cast(float, gu << 16);
            const float ur = __builtin_bit_cast(float, gu & 0xffff0000u);
            v[q] = silu_f(gr) * ur;
          }
        }
        const int lr = wm * TM + i * 32 + a * 8 + g * 4 + qs;
        uint16_t* dst = (uint16_t*)p.y + (int64_t)(row0 + lr) * p.ldy + n0 + wn * TNO + j * 32 + (l32 & ~3);
        if constexpr (OUT_F32) {
          uint32_t h[4], l[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) split_bf16(v[q], h[q], l[q]);
          const uint2 oh = exchange(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
          const uint2 ol = exchange(l[0] | (l[1] << 16), l[2] | (l[3] << 16));
          if (lr < rows_here) {
            *(uint2*)dst = oh;
            *(uint2*)(dst + p.y_lo) = ol;
          }
        } else {
          const uint2 o = exchange(pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]));
          if (lr < rows_here) *(uint2*)dst = o;
        }
      }
    }
  }
}

// Launch configurations: (rows, staged weight rows, wave grid) per workgroup.
struct CfgBig {
  static constexpr int BM = 128, BNB = 128, WM = 2, WN = 2, MT = 32;
  static constexpr bool REMAP = true;
};
// fp32 activations stage two bf16 planes of A, so they keep a 128-row tile
struct CfgBigF32 {
  static constexpr int BM = 128, BNB = 128, WM = 2, WN = 2, MT = 16;
  static constexpr bool REMAP = true;
};
struct CfgSmall {
  static constexpr int BM = 32, BNB = 128, WM = 1, WN = 4, MT = 16;
  static constexpr bool REMAP = false;
};

int kmode_of(int64_t tile) {
  if (tile == 32) return 0;
  if (tile == 64) return 1;
  if (tile > 64 && tile % 64 == 0) return 2;
  return -1;
}

template <class CF, bool SWIGLU, int NSPLIT, bool OUT_BF16, int KMODE, bool CANON, bool VEC>
int launch_gemm_k(const GemmArgs& a, int64_t m_tiles, hipStream_t stream) {
  constexpr int BNO = SWIGLU ? CF::BNB / 2 : CF::BNB;
  const int64_t n_tiles = (a.N + BNO - 1) / BNO;
  if (m_tiles <= 0 || n_tiles <= 0) return SMAUL_OK;
  if (m_tiles > 65535 || n_tiles > 65535) return fail(SMAUL_ERR_UNSUPPORTED, "gemm grid too large");
  dim3 grid((unsigned)n_tiles, (unsigned)m_tiles);
  hipLaunchKernelGGL(
      (fp8_gemm_kernel<CF::BM, CF::BNB, CF::WM, CF::WN, CF::MT, CF::REMAP, SWIGLU, NSPLIT, OUT_BF16, KMODE,
                       CANON, VEC>),
      grid, dim3(CF::WM * CF::WN * 64), 0, stream, a);
  return check_launch("fp8_gemm_kernel");
}

template <class CF, bool SWIGLU, int NSPLIT, bool OUT_BF16, bool CANON, bool VEC>
int launch_gemm(const GemmArgs& a, int64_t m_tiles, hipStream_t stream) {
  switch (kmode_of(a.tile)) {
    case 0: return launch_gemm_k<CF, SWIGLU, NSPLIT, OUT_BF16, 0, CANON, VEC>(a, m_tiles, stream);
    case 1: return launch_gemm_k<CF, SWIGLU, NSPLIT, OUT_BF16, 1, CANON, VEC>(a, m_tiles, stream);
    case 2: return launch_gemm_k<CF, SWIGLU, NSPLIT, OUT_BF16, 2, CANON, VEC>(a, m_tiles, stream);
    default: return fail(SMAUL_ERR_UNSUPPORTED, "tile %lld: need 32 or a multiple of 64", (long long)a.tile);
  }
}

// ---------------------------------------------------------------------------
// decode-regime grouped GEMM (at most 64 rows per expert), split over K
// ---------------------------------------------------------------------------
// A workgroup owns one expert and one 16-wide output column tile (for SwiGLU
// the gate and the up tile of the same columns) for all of the expert's rows
// (1..4 row tiles of 16).  Its KS waves split the 64-wide K blocks evenly, so
// a layer runs E * column tiles * KS waves and every wave can keep all (or a
// large part) of its weight codes in flight at once: the decode GEMMs are
// bound by how many bytes are outstanding, not by math.  Weight codes stream
// from HBM straight into registers: lane l reads 16 consecutive codes of
// column (l & 15) at k = (l >> 4) * 16 inside each 64-wide K block, DB blocks
// ahead of use, and the A fragments are read with the same k mapping, so
// every MFMA still sums exactly the products of one 64-wide scale tile.  The
// waves' fp32 partials are summed through LDS in wave order (deterministic),
// then wave 0 applies the epilogue.
// At most 8 K-split waves per workgroup; a one-row-tile wave keeps a ring of
// 4 K blocks in flight.
template <bool SWIGLU>
struct DecodeKS {
  static constexpr int MAX = 8;
};

// Entry e of a per-expert pointer table, read through the constant address
// space: the table is written by the host before the launch and never by a
// kernel, so the (wave-uniform) read is a scalar load.
template <class T>
__device__ __forceinline__ T* table_entry(T* const* table, int e) {
  typedef __attribute__((address_space(4))) const uint64_t* ctab_t;
  return (T*)(uintptr_t)((ctab_t)(uintptr_t)table)[e];
}

// One wave: rows row0..row0+nrows-1 of one expert against CT tiles of 16
// weight columns (tile t: codes W1 + t*16*K, scales S1 + t*16*nt, the lane's
// column already folded in; with SWIGLU also the up columns W2, S2) over K
// blocks kb0..kb0+nblk-1.  The CT tiles share the wave's A fragments, so per
// byte of weight codes streamed from HBM the wave loads 1/CT of the
// activation bytes.  SWIGLU (gate/up) rows are token indices read through
// p.row_idx; down reads its rows in place.
template <bool SWIGLU, bool CANON, int NRT, int DB, int CT>
__device__ __forceinline__ void decode_wave(const GemmArgs& p, const uint8_t* W1, const float* S1,
                                            const uint8_t* W2, const float* S2, int row0, int nrows,
                                            int64_t kb0, int64_t nblk, int lane, f32x4_t (*acc1)[4],
                                            f32x4_t (*acc2)[4]) {
  constexpr int NH = SWIGLU ? 2 : 1;
  const int kq = (lane >> 4) * 16;
  const WLayout L = wlayout(p);
  const int64_t tstride_w = 16 * L.wc, tstride_s = 16 * L.sc;
  // Row indices first; rows past the segment are computed, never stored.
  int64_t xr[NRT];
#pragma unroll
  for (int rt = 0; rt < NRT; ++rt) {
    const int64_t lr = row0 + min(rt * 16 + (lane & 15), nrows - 1);
    if constexpr (SWIGLU) xr[rt] = p.row_idx[lr];
    else xr[rt] = lr;
  }
  const uint16_t* arow[NRT];
  const f32x4_t z4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < CT; ++t)
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt) acc1[t][rt] = acc2[t][rt] = z4;
  // Prefetch ring of DB 64-wide K blocks: weight codes, scales and the A
  // fragments all travel in it, in the order they are consumed, so each
  // block's wait (vmcnt retires in order) never waits for a later block.
  uint4 bw[DB][NH][CT], a0[DB][NRT], a1[DB][NRT];
  float sw[DB][NH][CT];
  auto fetch_w = [&](int slot, int64_t kb) {
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
      for (int t = 0; t < CT; ++t) {
        bw[slot][h][t] = ldg16((h ? W2 : W1) + t * tstride_w + kb * L.wk + kq);
        sw[slot][h][t] = ldgf((h ? S2 : S1) + t * tstride_s + kb * L.sk);
      }
  };
  auto fetch_a = [&](int slot, int64_t kb) {
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt) {
      a0[slot][rt] = ldg16(arow[rt] + kb * 64 + kq);
      a1[slot][rt] = ldg16(arow[rt] + kb * 64 + kq + 8);
    }
  };
  // consume slot i; optionally refill it with block `next`
  auto step = [&](int i, bool refill, int64_t next) {
    bf16x8_t g0[NH][CT], g1[NH][CT];
    float sg[NH][CT];
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
      for (int t = 0; t < CT; ++t) {
        uint32_t d[8];
        decode4<CANON>(bw[i][h][t].x, d[0], d[1]);
        decode4<CANON>(bw[i][h][t].y, d[2], d[3]);
        decode4<CANON>(bw[i][h][t].z, d[4], d[5]);
        decode4<CANON>(bw[i][h][t].w, d[6], d[7]);
        g0[h][t] = __builtin_bit_cast(bf16x8_t, make_uint4(d[0], d[1], d[2], d[3]));
        g1[h][t] = __builtin_bit_cast(bf16x8_t, make_uint4(d[4], d[5], d[6], d[7]));
        sg[h][t] = sw[i][h][t];
      }
    bf16x8_t x0[NRT], x1[NRT];
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt) {
      x0[rt] = __builtin_bit_cast(bf16x8_t, a0[i][rt]);
      x1[rt] = __builtin_bit_cast(bf16x8_t, a1[i][rt]);
    }
    if (refill) {
      fetch_w(i, next);
      fetch_a(i, next);
    }
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
      for (int h = 0; h < NH; ++h)
#pragma unroll
        for (int t = 0; t < CT; ++t) {
          f32x4_t q = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x0[rt], g0[h][t], z4, 0, 0, 0);
          q = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x1[rt], g1[h][t], q, 0, 0, 0);
          f32x4_t& acc = h ? acc2[t][rt] : acc1[t][rt];
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[r] = __builtin_fmaf(sg[h][t], q[r], acc[r]);
        }
  };
  // nblk is a multiple of DB (the launcher picks DB): full rounds with
  // refills, then a last round without, so no step is conditional.  The
  // first round issues every weight load before the activation loads, which
  // wait for the row indices: the HBM stream starts one round trip earlier.
#pragma unroll
  for (int i = 0; i < DB; ++i) fetch_w(i, kb0 + i);
#pragma unroll
  for (int rt = 0; rt < NRT; ++rt) arow[rt] = (const uint16_t*)p.x + xr[rt] * p.ldx;
#pragma unroll
  for (int i = 0; i < DB; ++i) fetch_a(i, kb0 + i);
  const int64_t rounds = nblk / DB;
  for (int64_t r = 0; r + 1 < rounds; ++r) {
#pragma unroll
    for (int i = 0; i < DB; ++i) step(i, true, kb0 + (r + 1) * DB + i);
  }
#pragma unroll
  for (int i = 0; i < DB; ++i) step(i, false, 0);
}

// A workgroup owns one expert and DecodeCT output column tiles of 16 (for
// SwiGLU the gate and the up tiles of the same columns: one tile, two weight
// streams; for down two tiles of one stream); its KS waves split the K
// blocks evenly.
template <bool SWIGLU>
constexpr int DecodeCT = SWIGLU ? 1 : 2;

template <bool SWIGLU, bool CANON, int DB>
__global__ void __launch_bounds__(DecodeKS<SWIGLU>::MAX * 64)
decode_gemm_kernel(GemmArgs p, int col_groups, int ks_count) {
  constexpr int NH = SWIGLU ? 2 : 1;  // weight streams (gate, up)
  constexpr int CT = DecodeCT<SWIGLU>;
  // every wave's partials: [K split][stream][tile][row tile][r][lane] -- element
  // (row rt*16 + (lane>>4)*4 + r, column t*16 + (lane & 15)) of the group
  __shared__ float red[DecodeKS<SWIGLU>::MAX][NH][CT][4][4][64];
  const int lane = threadIdx.x & 63;
  const int ks = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // uniform: the expert's pointer-table entries and segment bounds are scalar loads
  const int e = __builtin_amdgcn_readfirstlane((int)blockIdx.x / col_groups);
  const int cg = (int)blockIdx.x - e * col_groups;
  if (e >= p.E) return;  // uniform per workgroup
  const int seg0 = p.seg_off[e];
  const int seg_rows = p.seg_off[e + 1] - seg0;
  const int64_t n0 = (int64_t)cg * CT * 16;
  // the lane's column of tile 0 (the launcher guarantees N % (16 * CT) == 0,
  // so every tile of every group lies inside the matrix)
  const int64_t col = n0 + (lane & 15);
  const WLayout L = wlayout(p);
  const uint8_t* W1 = table_entry(p.wp, e) + col * L.wc;
  const float* S1 = table_entry(p.sp, e) + col * L.sc;
  const uint8_t* W2 = SWIGLU ? table_entry(p.wp2, e) + col * L.wc : W1;
  const float* S2 = SWIGLU ? table_entry(p.sp2, e) + col * L.sc : S1;
  const int64_t nblk = (p.K >> 6) / ks_count;
  const int64_t kb0 = ks * nblk;
  const int nthr = ks_count * 64;
  // up to 64 rows per pass (the decode regime has at most 64); more rows
  // re-stream the weights once per 64
  for (int rb = 0; rb < seg_rows; rb += 64) {
    const int row0 = seg0 + rb;
    const int nrows = min(64, seg_rows - rb);
    const int nrt = (nrows + 15) >> 4;
    f32x4_t acc1[CT][4], acc2[CT][4];
    // prefetch depth shrinks as the A fragments per block grow (the launcher
    // guarantees nblk % DB == 0 with DB a power of two)
    switch (nrt) {
      case 1: decode_wave<SWIGLU, CANON, 1, DB, CT>(p, W1, S1, W2, S2, row0, nrows, kb0, nblk, lane, acc1, acc2); break;
      case 2: decode_wave<SWIGLU, CANON, 2, (DB >= 2 ? DB / 2 : 1), CT>(p, W1, S1, W2, S2, row0, nrows, kb0, nblk, lane, acc1, acc2); break;
      case 3: decode_wave<SWIGLU, CANON, 3, (DB >= 4 ? DB / 4 : 1), CT>(p, W1, S1, W2, S2, row0, nrows, kb0, nblk, lane, acc1, acc2); break;
      default: decode_wave<SWIGLU, CANON, 4, (DB >= 4 ? DB / 4 : 1), CT>(p, W1, S1, W2, S2, row0, nrows, kb0, nblk, lane, acc1, acc2); break;
    }
#pragma unroll
    for (int t = 0; t < CT; ++t)
#pragma unroll
      for (int rt = 0; rt < 4; ++rt)
        if (rt < nrt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            red[ks][0][t][rt][r][lane] = acc1[t][rt][r];
            if constexpr (SWIGLU) red[ks][NH - 1][t][rt][r][lane] = acc2[t][rt][r];
          }
    __syncthreads();
    // The workgroup's threads share the sums (in K-split order,
    // deterministic) and the epilogue: one output element each.
    for (int q = threadIdx.x; q < CT * nrt * 256; q += nthr) {
      const int t = q / (nrt * 256), qq = q - t * nrt * 256;
      const int rt = qq >> 8, r = (qq >> 6) & 3, ln = qq & 63;
      const int lr = rt * 16 + (ln >> 4) * 4 + r;
      const int64_t oc = n0 + t * 16 + (ln & 15);
      float g = red[0][0][t][rt][r][ln];
      for (int k2 = 1; k2 < ks_count; ++k2) g += red[k2][0][t][rt][r][ln];
      float v = g;
      if constexpr (SWIGLU) {
        float u = red[0][NH - 1][t][rt][r][ln];
        for (int k2 = 1; k2 < ks_count; ++k2) u += red[k2][NH - 1][t][rt][r][ln];
        v = silu_f(bf2f(f2bf(g))) * bf2f(f2bf(u));
      }
      if (lr < nrows && oc < p.N) ((uint16_t*)p.y)[(int64_t)(row0 + lr) * p.ldy + oc] = (uint16_t)f2bf(v);
    }
    __syncthreads();  // red[] is reused by the next 64-row pass
  }
}

// SWIGLU (gate/up) gathers its rows through a.row_idx; down reads its rows
// in place (a.row_idx is null): the decode kernel relies on exactly that.
template <bool SWIGLU, bool CANON, int DB>
int launch_decode_db(const GemmArgs& a, int ks_count, hipStream_t stream) {
  if (SWIGLU != (a.row_idx != nullptr)) return fail(SMAUL_ERR_INVALID, "decode gemm: row gather mismatch");
  constexpr int CT = DecodeCT<SWIGLU>;
  if (a.N % (16 * CT) != 0) return fail(SMAUL_ERR_INVALID, "decode gemm: N must be a multiple of %d", 16 * CT);
  const int col_groups = (int)(a.N / (16 * CT));
  const int64_t blocks = (int64_t)a.E * col_groups;
  hipLaunchKernelGGL((decode_gemm_kernel<SWIGLU, CANON, DB>), dim3((unsigned)blocks), dim3(ks_count * 64), 0,
                     stream, a, col_groups, ks_count);
  return check_launch("decode_gemm_kernel");
}

// ---------------------------------------------------------------------------
// routing results shared by the router and the dispatch kernels
// ---------------------------------------------------------------------------
constexpr int ROUTE_THREADS = 256;
constexpr int ROUTE_WAVES = ROUTE_THREADS / 64;
constexpr int MAX_E = 64;
constexpr int ROUTE_WFLOATS = 8192;  // router-weight chunk staged in LDS (32 KB)

struct RouteOut {
  float* prob;
  int64_t* topi;
  float* topw;
  int32_t* blockcnt;   // [nb][E], or nullptr
  // fused dispatch (single block only); nullptr otherwise
  int32_t* counts;
  int32_t* seg_off;
  int32_t* tile_off;
  int32_t* perm_row;
  float* perm_w;
  int32_t* inv;
  int block_m;
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// a slot is dispatched when its weight is positive (model.py:576); ids out of
// range and repeats of an expert already in the row are not (the router
// never produces either)
__device__ __forceinline__ uint64_t selection_of(const int* ti, const float* tw, int E, int k) {
  uint64_t sel = 0;
  for (int j = 0; j < k; ++j) {
    const int ee = ti[j];
    if (tw[j] > 0.0f && ee >= 0 && ee < E && !((sel >> ee) & 1ull)) sel |= 1ull << ee;
  }
  return sel;
}

// Token t's top-k ids (outside [0, E) as -1) and weights, as the dispatch
// reads them (t invalid: -1 / 0); every load is issued before the first is
// used, so the k reads take one round trip.
__device__ __forceinline__ void load_topk(const int64_t* topi, const float* topw, int64_t t, int k, bool valid,
                                          int E, int (&ti)[8], float (&tw)[8]) {
  int64_t v[8];
  float w[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    v[j] = -1;
    w[j] = 0.0f;
  }
  if (valid) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (j < k) {
        v[j] = topi[t * k + j];
        w[j] = topw[t * k + j];
      }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    ti[j] = (j < k && v[j] >= 0 && v[j] < E) ? (int)v[j] : -1;
    tw[j] = j < k ? w[j] : 0.0f;
  }
}

// Deterministic dispatch of up to 64 tokens by one wave: lane t holds token
// t's top-k ids and weights (load_topk); each expert's rows are the tokens
// that selected it, ranked by ballot in ascending token order
// (model.py:574-581).  A token's live slots are the first slot of each
// expert with a positive weight (selection_of); the others get inv -1.  The
// expert loop only ranks; every store follows it (E <= 64).
__device__ __forceinline__ void dispatch_one_wave(const int* ti, const float* tw, bool valid, int lane,
                                                  const RouteOut& o, int E, int k) {
  const int64_t t = lane;
  bool live[8];
  uint64_t sel = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int ee = ti[j];
    live[j] = valid && j < k && tw[j] > 0.0f && ee >= 0 && ee < E && !((sel >> ee) & 1ull);
    if (live[j]) sel |= 1ull << ee;
  }
  const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  int pos[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) pos[j] = -1;
  int off = 0, toff = 0, my_n = 0, my_off = 0, my_toff = 0;
  for (int e = 0; e < E; ++e) {
    const uint64_t b = __ballot((sel >> e) & 1ull);
    const int n = __popcll(b);
    if (lane == e) {
      my_n = n;
      my_off = off;
      my_toff = toff;
    }
    const int p = off + __popcll(b & lt);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (live[j] && ti[j] == e) pos[j] = p;
    off += n;
    toff += (n + o.block_m - 1) / o.block_m;
  }
  if (lane < E) {
    o.counts[lane] = my_n;
    o.seg_off[lane] = my_off;
    o.tile_off[lane] = my_toff;
  }
  if (lane == 0) {
    o.seg_off[E] = off;
    o.tile_off[E] = toff;
  }
  if (valid) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (j < k) {
        if (live[j]) {
          o.perm_row[pos[j]] = (int32_t)t;
          o.perm_w[pos[j]] = tw[j];
        }
        o.inv[t * k + j] = live[j] ? pos[j] : -1;
      }
  }
}

// ---- router building blocks (router_kernel; route_select also backs the
// tie fallback of the MFMA router) -------------------------------------------

// Router columns per LDS chunk and the lane's 8-column groups per chunk.
template <int EMAX>
struct RouteShape {
  static constexpr int DC = ROUTE_WFLOATS / EMAX;   // columns per chunk
  static constexpr int XG = (DC / 8 + 63) / 64;     // 8-column groups per lane
};

// Activations of TB tokens (rows tw0.., rows past T clamped to T-1: computed,
// never written) for the lane's column groups of chunk [c0, c0 + cw).
template <bool XBF16, int TB, int EMAX>
__device__ __forceinline__ void route_load_x(const void* x, int64_t T, int64_t tw0, int c0, int cw, int d,
                                             int lane, uint4 (&xr)[RouteShape<EMAX>::XG][TB][XBF16 ? 1 : 2]) {
  constexpr int XG = RouteShape<EMAX>::XG;
  constexpr int XW = XBF16 ? 1 : 2;
#pragma unroll
  for (int q = 0; q < XG; ++q) {
    const int g = lane + 64 * q;
    if (g < (cw >> 3)) {
#pragma unroll
      for (int a = 0; a < TB; ++a) {
        const int64_t t = tw0 + a < T ? tw0 + a : T - 1;
        if constexpr (XBF16) {
          xr[q][a][0] = ldg16((const uint16_t*)x + t * d + c0 + g * 8);
        } else {
          xr[q][a][0] = ldg16((const float*)x + t * d + c0 + g * 8);
          xr[q][a][XW - 1] = ldg16((const float*)x + t * d + c0 + g * 8 + 4);
        }
      }
    }
  }
}

// acc[a * EMAX + e] += the lane's column groups of chunk (width cw) of token a
// times router row e, staged in sW[e * cw + c]; per lane the groups are summed
// in ascending order, 8 columns at a time in column order (fmaf).
template <bool XBF16, int TB, int EMAX>
__device__ __forceinline__ void route_fma(const uint4 (&xr)[RouteShape<EMAX>::XG][TB][XBF16 ? 1 : 2],
                                          const float* sW, int cw, int lane, float (&acc)[TB * EMAX]) {
  constexpr int XG = RouteShape<EMAX>::XG;
  constexpr int XW = XBF16 ? 1 : 2;
#pragma unroll
  for (int q = 0; q < XG; ++q) {
    const int g = lane + 64 * q;
    if (g < (cw >> 3)) {
      float xv[TB][8];
#pragma unroll
      for (int a = 0; a < TB; ++a) {
        if constexpr (XBF16) {
          const uint4 v = xr[q][a][0];
          xv[a][0] = bf2f(v.x & 0xffff); xv[a][1] = bf2f(v.x >> 16);
          xv[a][2] = bf2f(v.y & 0xffff); xv[a][3] = bf2f(v.y >> 16);
          xv[a][4] = bf2f(v.z & 0xffff); xv[a][5] = bf2f(v.z >> 16);
          xv[a][6] = bf2f(v.w & 0xffff); xv[a][7] = bf2f(v.w >> 16);
        } else {
          const uint4 v0 = xr[q][a][0], v1 = xr[q][a][XW - 1];
          xv[a][0] = __uint_as_float(v0.x); xv[a][1] = __uint_as_float(v0.y);
          xv[a][2] = __uint_as_float(v0.z); xv[a][3] = __uint_as_float(v0.w);
          xv[a][4] = __uint_as_float(v1.x); xv[a][5] = __uint_as_float(v1.y);
          xv[a][6] = __uint_as_float(v1.z); xv[a][7] = __uint_as_float(v1.w);
        }
      }
#pragma unroll
      for (int e = 0; e < EMAX; ++e) {
        const float4 w0 = *(const float4*)&sW[e * cw + g * 8];
        const float4 w1 = *(const float4*)&sW[e * cw + g * 8 + 4];
        const float wv8[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
        for (int a = 0; a < TB; ++a)
#pragma unroll
          for (int qq = 0; qq < 8; ++qq)
            acc[a * EMAX + e] = __builtin_fmaf(xv[a][qq], wv8[qq], acc[a * EMAX + e]);
      }
    }
  }
}

// Halving butterfly over the 64 lanes: at each step a lane keeps half of its
// values and adds the partner's copy of them, so the TB*EMAX sums need
// TB*EMAX-1 exchanges in all (instead of 6 per value) and the exchanges of a
// step are independent.  Every value is summed over the same xor tree of
// lanes whatever TB is.  Afterwards acc[0] of lane l is the full sum of value
// index vidx (returned); with 32 values the even lanes hold them.
template <int TB, int EMAX>
__device__ __forceinline__ int route_butterfly(float (&acc)[TB * EMAX], int lane) {
  constexpr int N = TB * EMAX;
  static_assert(N == 32 || N == 64, "router reduction expects 32 or 64 partial sums per lane");
  int vidx = 0;
#pragma unroll
  for (int step = 0; step < 6; ++step) {
    const int m = 32 >> step;
    const int n = N >> step;
    const bool up = (lane & m) != 0;
    const uint32_t upmask = up ? 0xffffffffu : 0u;
    if (n >= 2) {
      const int half = n >> 1;
#pragma unroll
      for (int i = 0; i < N / 2; ++i) {
        if (i < half) {
          // select with a bit mask, not `up ? acc[i] : acc[i + half]`: the
          // compiler turns that into a dynamically indexed array read (a
          // compare/select over every element of acc)
          const uint32_t lo = __float_as_uint(acc[i]), hi = __float_as_uint(acc[i + half]);
          const uint32_t give = (lo & upmask) | (hi & ~upmask);
          const uint32_t keep = (hi & upmask) | (lo & ~upmask);
          acc[i] = __uint_as_float(keep) + __shfl_xor(__uint_as_float(give), m, 64);
        }
      }
      if (up) vidx += half;
    } else {
      acc[0] += __shfl_xor(acc[0], m, 64);
    }
  }
  return vidx;
}

// One token (model.py:558-570): softmax of its logits lg[0..E) (torch's
// exp(v - max) / sum form), top-k (torch's CPU order; q is scratch for the
// tie path), the < 1e-6 guarded renormalisation.  Writes prob/topi/topw of
// token t when `write`; returns the ids and weights in ti/tv.
template <int EMAX>
__device__ __forceinline__ void route_select(const float* lg, smaul_topk::Pair* q, int E, int k, int64_t t,
                                             const RouteOut& o, bool write, int (&ti)[8], float (&tv)[8]) {
  float v[EMAX];
#pragma unroll
  for (int e = 0; e < EMAX; ++e) v[e] = e < E ? lg[e] : 0.0f;
  float mx = v[0];  // NaN propagates, as in torch's max reduction
#pragma unroll
  for (int e = 1; e < EMAX; ++e)
    if (e < E) mx = (v[e] > mx || v[e] != v[e]) ? v[e] : mx;
  float sum = 0.0f;
#pragma unroll
  for (int e = 0; e < EMAX; ++e)
    if (e < E) {
      v[e] = expf(v[e] - mx);
      sum = sum + v[e];
    }
  const float rs = 1.0f / sum;
  bool ties = false;
#pragma unroll
  for (int e = 0; e < EMAX; ++e)
    if (e < E) {
      v[e] = v[e] * rs;
      if (write) o.prob[t * E + e] = v[e];
      ties |= v[e] != v[e];
    }
  // Top-k.  With all-distinct values the selection is unique: the k largest
  // in descending order, found in registers.  Equal values (or NaN) go
  // through the exact restatement of torch's selection steps.
  if constexpr (EMAX <= 16) {
#pragma unroll
    for (int a = 0; a < EMAX; ++a)
#pragma unroll
      for (int b = a + 1; b < EMAX; ++b)
        if (b < E) ties |= v[a] == v[b];
  } else {
    ties = true;
  }
  if (!ties) {
    uint64_t used = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (j < k) {
        int bi = -1;
        float bv = 0.0f;
#pragma unroll
        for (int e = 0; e < EMAX; ++e)
          if (e < E && !((used >> e) & 1ull) && (bi < 0 || v[e] > bv)) {
            bi = e;
            bv = v[e];
          }
        used |= 1ull << bi;
        ti[j] = bi;
        tv[j] = bv;
      }
    }
  } else {
#pragma unroll
    for (int e = 0; e < EMAX; ++e)
      if (e < E) q[e] = smaul_topk::Pair{v[e], e};
    smaul_topk::topk_small(q, E, k);  // k <= 8
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (j < k) {
        ti[j] = q[j].i;
        tv[j] = q[j].v;
      }
  }
  float denom = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j)
    if (j < k) denom = denom + tv[j];
  const bool tiny = denom < 1e-6f;
  const float dcl = fmaxf(denom, 1e-9f);
#pragma unroll
  for (int j = 0; j < 8; ++j)
    if (j < k) {
      tv[j] = tiny ? 1.0f / (float)k : tv[j] / dcl;
      if (write) {
        o.topi[t * k + j] = ti[j];
        o.topw[t * k + j] = tv[j];
      }
    }
}

// ---- router logits on the matrix cores (bf16 activations) ------------------
// The fp32 router weight is split exactly into three bf16 terms,
// w = w0 + w1 + w2 (w0 = bf16(w), w1 = bf16(w - w0), w2 = w - w0 - w1, which
// has at most 8 significant bits), so every product x * wi of a bf16
// activation is exact in fp32 and v_mfma_f32_16x16x32_bf16 sums them in fp32:
// the logits carry fp32 accumulation error only, as a scalar fmaf chain does.
// A pass covers 64 tokens (four MFMA N-tiles of 16; one tile, 16 tokens, in
// the decode step's blocks) and up to 16 experts (the M rows; rows past E are
// zero).  K is cut into RK_SLICES fixed slices of KSW 32-wide k-steps; a wave
// computes whole slices (each with all of the block's token tiles, the three
// weight terms in separate accumulators) and leaves one partial per (slice,
// token, expert) in LDS; the logit is the sum of the slices in slice order
// plus the bias.  Nothing depends on the number of waves or on the tokens
// per block, so every launch shape produces the same bits for a token.  The weight terms are made in registers from the lane's own fp32
// weights (no LDS staging).
constexpr int RK_SLICES = 8;
constexpr int RK_TOK = 64;
constexpr int RK_PART_FLOATS = RK_SLICES * RK_TOK * 16;

// fp32 -> bf16 bits, round to nearest even (v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t bf16_rne(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}

// One K slice of the logits: load() issues every activation and weight load
// of the slice, compute() waits for them, runs the MFMAs and writes the
// partials part[(slice * TOK + token) * 16 + expert].  Split so that a caller
// can issue other loads in between that compute() does not wait for.
// d <= RK_SLICES * 32 * KSW columns.
template <int KSW, int NTT = 4>
struct RouteSlice {
  static constexpr int TOK = NTT * 16;  // tokens of the block
  uint4 xr[NTT][KSW];
  float4 wr[KSW][2];
  bf16x8_t wa[KSW][3];  // the weights as three bf16 terms (split())
  int slice;

  // Every load is issued unconditionally from an in-bounds address (column
  // 0, expert 0 or token T-1 where the true one is out of range) and masked
  // in compute(), so all of them are in flight together.
  __device__ __forceinline__ void load(const uint16_t* x, const float* gw, int E, int64_t T, int64_t t0, int d,
                                       int sl, int lane) {
    slice = sl;
    const int n = lane & 15, g = lane >> 4;
#pragma unroll
    for (int i = 0; i < KSW; ++i) {
      const int c = (slice * KSW + i) * 32 + 8 * g;
      const int cc = c < d ? c : 0;  // d % 8 == 0: a group is all in or all out
#pragma unroll
      for (int tt = 0; tt < NTT; ++tt) {
        const int64_t t = t0 + tt * 16 + n < T ? t0 + tt * 16 + n : T - 1;  // computed, never written
        xr[tt][i] = ldg16(x + t * d + cc);
      }
      const int64_t wrow = n < E ? n : 0;
      wr[i][0] = *(const float4*)(gw + wrow * d + cc);
      wr[i][1] = *(const float4*)(gw + wrow * d + cc + 4);
    }
  }

  // load() in two parts: the weights alone, and the activations from a
  // [tokens][d] bf16 copy in LDS (rows at and past nvalid read row nvalid-1,
  // as load() does past T)
  __device__ __forceinline__ void load_w(const float* gw, int E, int d, int sl, int lane) {
    slice = sl;
    const int n = lane & 15, g = lane >> 4;
#pragma unroll
    for (int i = 0; i < KSW; ++i) {
      const int c = (slice * KSW + i) * 32 + 8 * g;
      const int cc = c < d ? c : 0;
      const int64_t wrow = n < E ? n : 0;
      wr[i][0] = *(const float4*)(gw + wrow * d + cc);
      wr[i][1] = *(const float4*)(gw + wrow * d + cc + 4);
    }
  }
  __device__ __forceinline__ void load_x_lds(const uint16_t* sx, int d, int nvalid, int lane) {
    const int n = lane & 15, g = lane >> 4;
#pragma unroll
    for (int i = 0; i < KSW; ++i) {
      const int c = (slice * KSW + i) * 32 + 8 * g;
      const int cc = c < d ? c : 0;
#pragma unroll
      for (int tt = 0; tt < NTT; ++tt) {
        const int t = tt * 16 + n < nvalid ? tt * 16 + n : nvalid - 1;
        xr[tt][i] = *(const uint4*)(sx + t * d + cc);
      }
    }
  }

  // block i of the weights as three bf16 terms: w = hi + mid + lo, each term
  // the bf16 rounding of what the terms before it leave
  __device__ __forceinline__ void terms(int i, bf16x8_t (&a)[3]) const {
    const float w8[8] = {wr[i][0].x, wr[i][0].y, wr[i][0].z, wr[i][0].w,
                         wr[i][1].x, wr[i][1].y, wr[i][1].z, wr[i][1].w};
    uint32_t q0[8], q1[8], q2[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      q0[j] = bf16_rne(w8[j]);
      const float r1 = w8[j] - bf2f(q0[j]);
      q1[j] = bf16_rne(r1);
      q2[j] = bf16_rne(r1 - bf2f(q1[j]));
    }
    a[0] = __builtin_bit_cast(bf16x8_t, make_uint4(q0[0] | (q0[1] << 16), q0[2] | (q0[3] << 16),
                                                   q0[4] | (q0[5] << 16), q0[6] | (q0[7] << 16)));
    a[1] = __builtin_bit_cast(bf16x8_t, make_uint4(q1[0] | (q1[1] << 16), q1[2] | (q1[3] << 16),
                                                   q1[4] | (q1[5] << 16), q1[6] | (q1[7] << 16)));
    a[2] = __builtin_bit_cast(bf16x8_t, make_uint4(q2[0] | (q2[1] << 16), q2[2] | (q2[3] << 16),
                                                   q2[4] | (q2[5] << 16), q2[6] | (q2[7] << 16)));
  }
  // the weights out of range (column >= d, expert >= E) to zero
  __device__ __forceinline__ void mask_w(int E, int d, int lane) {
    const int n = lane & 15, g = lane >> 4;
#pragma unroll
    for (int i = 0; i < KSW; ++i) {
      const int c = (slice * KSW + i) * 32 + 8 * g;
      if (c >= d || n >= E) wr[i][0] = wr[i][1] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }

  // Waits for the loads, runs the MFMAs and writes the partials; PRE: the
  // weights' terms were made by split() (which holds them all at once: for a
  // caller with time and registers to spare before the activations arrive),
  // else each block's terms are made as it is used.
  template <bool PRE = false>
  __device__ __forceinline__ void compute(int E, int d, int lane, float* part) {
    const int n = lane & 15, g = lane >> 4;
#pragma unroll
    for (int i = 0; i < KSW; ++i) {
      const int c = (slice * KSW + i) * 32 + 8 * g;
      if (c >= d) {
#pragma unroll
        for (int tt = 0; tt < NTT; ++tt) xr[tt][i] = make_uint4(0u, 0u, 0u, 0u);
      }
    }
    if constexpr (!PRE) mask_w(E, d, lane);
    f32x4_t acc[NTT][3];
#pragma unroll
    for (int tt = 0; tt < NTT; ++tt)
#pragma unroll
      for (int term = 0; term < 3; ++term) acc[tt][term] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < KSW; ++i) {
      bf16x8_t a[3];
      if constexpr (PRE) {
        a[0] = wa[i][0];
        a[1] = wa[i][1];
        a[2] = wa[i][2];
      } else {
        terms(i, a);
      }
#pragma unroll
      for (int tt = 0; tt < NTT; ++tt)
#pragma unroll
        for (int term = 0; term < 3; ++term)
          acc[tt][term] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[term], __builtin_bit_cast(bf16x8_t, xr[tt][i]),
                                                                  acc[tt][term], 0, 0, 0);
    }
    // lane holds experts 4g + r of token tt*16 + n
#pragma unroll
    for (int tt = 0; tt < NTT; ++tt)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        part[(slice * TOK + tt * 16 + n) * 16 + 4 * g + r] = (acc[tt][0][r] + acc[tt][1][r]) + acc[tt][2][r];
  }
  // every block's terms ahead of compute<true>() (waits for the weight loads)
  __device__ __forceinline__ void split(int E, int d, int lane) {
    mask_w(E, d, lane);
#pragma unroll
    for (int i = 0; i < KSW; ++i) terms(i, wa[i]);
  }
};

// The sum over slices, in slice order, plus the bias: slog[token][e] for
// e < E, tokens t0.. below T.  Follows the barrier after the partials; ends
// with a barrier.
template <int EMAX, int TOK = RK_TOK>
__device__ __forceinline__ void route_reduce(const float* gb, int E, int64_t T, int64_t t0, int nw,
                                             const float* part, float (*slog)[EMAX]) {
  for (int q = threadIdx.x; q < TOK * EMAX; q += nw * 64) {
    const int tok = q / EMAX, e = q - tok * EMAX;
    if (e < E && t0 + tok < T) {
      float v = part[tok * 16 + e];
#pragma unroll
      for (int sl = 1; sl < RK_SLICES; ++sl) v += part[(sl * TOK + tok) * 16 + e];
      slog[tok][e] = gb ? v + gb[e] : v;
    }
  }
  __syncthreads();
}

// Logits of tokens t0 .. t0+63 (rows past T: not written) into slog[token][e]
// for e < E <= EMAX <= 16, by nw waves of this workgroup (all must call it).
// part: RK_PART_FLOATS of LDS.  Ends with a barrier.
template <int KSW, int EMAX, int NTT>
__device__ __forceinline__ void route_logits(const uint16_t* x, const float* gw, const float* gb, int E, int64_t T,
                                             int64_t t0, int d, int nw, float* part, float (*slog)[EMAX]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int sl = wave; sl < RK_SLICES; sl += nw) {
    RouteSlice<KSW, NTT> rs;
    rs.load(x, gw, E, T, t0, d, sl, lane);
    rs.compute(E, d, lane, part);
  }
  __syncthreads();
  route_reduce<EMAX, NTT * 16>(gb, E, T, t0, nw, part, slog);
}

// the k-steps per slice for model width d (0: too wide for the MFMA router)
inline int route_ksw(int64_t d) {
  if (d % 8 != 0) return 0;
  if (d <= RK_SLICES * 32 * 4) return 4;
  if (d <= RK_SLICES * 32 * 8) return 8;
  return 0;
}

// Softmax / top-k / renormalisation of one token by a group of EMAX lanes
// (lane j of the group: expert j), the arithmetic of route_select: the same
// max, expf, sequential sum (the group's values gathered in expert order),
// 1/sum scaling and rank-order renormalisation, so the bits match it.  With
// equal probabilities or NaN in the group its first lane runs route_select
// itself (torch's tie order).  Writes prob/topi/topw when `write`, and the
// top-k to s_ti/s_tw (rows of EMAX... 8 slots) and the selection counts to
// s_cnt (if not null).  Every lane of the wave must call it.
template <int EMAX>
__device__ __forceinline__ void route_select_group(const float* lg, smaul_topk::Pair* q, int E, int k, int64_t t,
                                                   bool tvalid, const RouteOut& o, bool write, int* s_ti_row,
                                                   float* s_tw_row, int* s_cnt) {
  constexpr int G = EMAX;
  static_assert(G == 4 || G == 8 || G == 16, "group width");
  const int lane = threadIdx.x & 63;
  const int j = lane & (G - 1);
  const int gbase = lane & ~(G - 1);
  const uint64_t gmask = ((G == 64 ? 0ull : (1ull << G)) - 1ull) << gbase;
  const bool ev = j < E;
  const float v = (tvalid && ev) ? lg[j] : 0.0f;
  float mx = ev ? v : -__builtin_inff();
#pragma unroll
  for (int m = 1; m < G; m <<= 1) mx = fmaxf(mx, __shfl_xor(mx, m, 64));
  const float ex = ev ? expf(v - mx) : 0.0f;
  float sum = 0.0f;
#pragma unroll
  for (int e = 0; e < G; ++e) {
    const float xe = __shfl(ex, gbase + e, 64);
    if (e < E) sum = sum + xe;
  }
  const float rs = 1.0f / sum;
  const float p = ex * rs;
  int rank = 0;
  bool tie = p != p;
#pragma unroll
  for (int e = 0; e < G; ++e) {
    const float pe = __shfl(p, gbase + e, 64);
    if (e < E && e != j) {
      rank += pe > p ? 1 : 0;
      tie |= (pe == p) || (pe != pe);
    }
  }
  const bool gtie = (__ballot(tie && ev && tvalid) & gmask) != 0ull;
  // renormalisation denominator: the selected probabilities in rank order
  const uint64_t lt_mask = gmask;
  float denom = 0.0f;
#pragma unroll
  for (int r = 0; r < 8; ++r)
    if (r < k) {
      const uint64_t m = __ballot(ev && rank == r) & lt_mask;
      const int src = m ? (int)__builtin_ctzll(m) : gbase;
      const float pr = __shfl(p, src, 64);
      denom = denom + pr;
    }
  if (!tvalid) return;
  if (!gtie) {
    if (ev) {
      if (write) o.prob[t * E + j] = p;
      if (rank < k) {
        const bool tiny = denom < 1e-6f;
        const float dcl = fmaxf(denom, 1e-9f);
        const float tv = tiny ? 1.0f / (float)k : p / dcl;
        if (write) {
          o.topi[t * k + rank] = j;
          o.topw[t * k + rank] = tv;
        }
        s_ti_row[rank] = j;
        s_tw_row[rank] = tv;
        if (s_cnt && tv > 0.0f) atomicAdd(&s_cnt[j], 1);
      }
    }
  } else if (j == 0) {
    int ti[8];
    float tv[8];
    route_select<EMAX>(lg, q, E, k, t, o, write, ti, tv);
#pragma unroll
    for (int jj = 0; jj < 8; ++jj)
      if (jj < k) {
        s_ti_row[jj] = ti[jj];
        s_tw_row[jj] = tv[jj];
      }
    if (s_cnt) {
      const uint64_t sel = selection_of(ti, tv, E, k);
      for (int e = 0; e < E; ++e)
        if ((sel >> e) & 1ull) atomicAdd(&s_cnt[e], 1);
    }
  }
}

// ---------------------------------------------------------------------------
// decode, streaming form (decode_stream_kernel)
// ---------------------------------------------------------------------------
// The grid is one workgroup per CU.  The work is a list of units, one per
// (segment, 16-column tile), where a segment is up to DS_ROWS rows of one
// expert; workgroup g walks the contiguous unit range [g*U/G, (g+1)*U/G).
// Its waves split K: wave ks owns KBW consecutive 64-wide blocks and keeps
// that slice of the segment's activation rows in registers for as long as the
// segment lasts, so per unit it streams only weight codes and scales, and it
// keeps DS_D units of them in flight (a register ring that runs across unit
// boundaries; the refill of a block is issued as soon as the block is
// decoded).  Per unit the waves' fp32 partials meet in LDS (two buffers, one
// barrier per unit) and are summed in K-split order: deterministic.
constexpr int DS_ROWS = 32;
constexpr int DS_WMAX = 8;
constexpr int DS_D = 2;

// Segments of the executed experts, one lane per expert (E <= 64).  The lane
// also holds its expert's weight and scale pointers, loaded beside the
// segment bounds, so no pointer-table read waits in the unit loop.
struct DsSegs {
  int incl;    // inclusive prefix of segment counts up to this lane's expert
  int nseg;    // segments of this lane's expert
  int lo;      // its first row
  int rows;    // its rows
  int total;   // segments over all experts (uniform)
  uint64_t w1, s1, w2, s2;  // its codes and scales (w2/s2: the up projection)
};

// pointer held by lane e (uniform e) -> scalar
template <class T>
__device__ __forceinline__ T* ds_ptr(uint64_t v, int e) {
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, e);
  const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(v >> 32), e);
  return (T*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

// lane e < E: its expert's weight and scale pointers
__device__ __forceinline__ void ds_pointers(const GemmArgs& p, int lane, DsSegs& s) {
  s.w1 = s.s1 = s.w2 = s.s2 = 0;
  if (lane < p.E) {
    s.w1 = (uint64_t)(uintptr_t)p.wp[lane];
    s.s1 = (uint64_t)(uintptr_t)p.sp[lane];
    if (p.wp2) {
      s.w2 = (uint64_t)(uintptr_t)p.wp2[lane];
      s.s2 = (uint64_t)(uintptr_t)p.sp2[lane];
    }
  }
}

// lane e < E: its expert's rows [lo, hi); segment counts and their prefix
__device__ __forceinline__ void ds_finish(int lo, int hi, int lane, DsSegs& s) {
  s.lo = lo;
  s.rows = hi - lo;
  s.nseg = (s.rows + DS_ROWS - 1) / DS_ROWS;
  int inc = s.nseg;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_up(inc, o, 64);
    if (lane >= o) inc += u;
  }
  s.incl = inc;
  s.total = __builtin_amdgcn_readlane(inc, 63);
}

__device__ __forceinline__ DsSegs ds_segments(const GemmArgs& p, int lane) {
  DsSegs s;
  int lo = 0, hi = 0;
  if (lane < p.E) {
    lo = p.seg_off[lane];
    hi = p.seg_off[lane + 1];
  }
  ds_pointers(p, lane, s);
  ds_finish(lo, hi, lane, s);
  return s;
}

// segment j (uniform, < total) -> expert, first row, rows (all uniform)
__device__ __forceinline__ void ds_locate(const DsSegs& s, int j, int& e, int& row0, int& nrows) {
  e = (int)__popcll(__ballot(s.incl <= j));
  const int pass = j - __builtin_amdgcn_readlane(s.incl - s.nseg, e);
  row0 = __builtin_amdgcn_readlane(s.lo, e) + pass * DS_ROWS;
  nrows = min(DS_ROWS, __builtin_amdgcn_readlane(s.rows, e) - pass * DS_ROWS);
}

// The register ring of weight codes and scales: DS_D units of this wave's K
// slice (blocks kb0 .. kb0+KBW-1 of 16 columns), unit u of segment j = u / ctn
// at column tile u % ctn.
template <bool SWIGLU, int KBW>
struct DsRing {
  static constexpr int NH = SWIGLU ? 2 : 1;
  uint4 bw[DS_D][KBW][NH];
  float sw[DS_D][KBW][NH];

  // the wave's codes and scales of unit u: block b of stream h at
  // wsrc[h] + b*64 and ssrc[h] + b
  __device__ __forceinline__ static void unit_src(const GemmArgs& p, const DsSegs& sg, int ctn, int64_t kb0, int kq,
                                                  int lane, int u, const uint8_t* (&wsrc)[NH],
                                                  const float* (&ssrc)[NH]) {
    const int j = u / ctn;
    const int ct = u - j * ctn;
    int e, r0, nr;
    ds_locate(sg, j, e, r0, nr);
    const int64_t col = (int64_t)ct * 16 + (lane & 15);
    const WLayout L = wlayout(p);
    wsrc[0] = ds_ptr<const uint8_t>(sg.w1, e) + col * L.wc + kb0 * L.wk + kq;
    ssrc[0] = ds_ptr<const float>(sg.s1, e) + col * L.sc + kb0 * L.sk;
    if constexpr (SWIGLU) {
      wsrc[NH - 1] = ds_ptr<const uint8_t>(sg.w2, e) + col * L.wc + kb0 * L.wk + kq;
      ssrc[NH - 1] = ds_ptr<const float>(sg.s2, e) + col * L.sc + kb0 * L.sk;
    }
  }
  __device__ __forceinline__ void fetch(const GemmArgs& p, const DsSegs& sg, int ctn, int64_t kb0, int kq, int lane,
                                        int slot, int u) {
    const uint8_t* ws[NH];
    const float* ss[NH];
    unit_src(p, sg, ctn, kb0, kq, lane, u, ws, ss);
    const WLayout L = wlayout(p);
#pragma unroll
    for (int b = 0; b < KBW; ++b)
#pragma unroll
      for (int h = 0; h < NH; ++h) {
        bw[slot][b][h] = ldg16(ws[h] + b * L.wk);
        sw[slot][b][h] = ldgf(ss[h] + b * L.sk);
      }
  }
};

// ridx: logical row -> activation row (SwiGLU only; down reads its rows in
// place).
// COH: the outputs are stored with device scope, for workgroups of the same
// launch that read them (the fused combine of decode_stream_kernel).
template <bool SWIGLU, bool CANON, int KBW, int NRT, bool COH = false>
__device__ __forceinline__ void ds_body(const GemmArgs& p, const DsSegs& sg, const int32_t* ridx, int u0,
                                        int u1, int ctn, float* red, int nw) {
  constexpr int NH = SWIGLU ? 2 : 1;
  const int lane = threadIdx.x & 63;
  const int ks = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kq = (lane >> 4) * 16;
  const int64_t kb0 = (int64_t)ks * KBW;
  const f32x4_t z4 = {0.f, 0.f, 0.f, 0.f};
  const int last = u1 - 1;
  DsRing<SWIGLU, KBW> ring;
  const WLayout L = wlayout(p);

  // the segment's activation rows, this wave's K slice
  uint4 a0[NRT][KBW], a1[NRT][KBW];
  // this wave's 2 KB tile for turning whole-line row loads into the MFMA
  // operand layout: 16 rows x 8 16-byte slots, slot c of row r at c ^ (r >> 1)
  // (conflict-free for the writes, 8 lanes per row, and for the reads, one
  // row per lane of each 16)
  __shared__ uint4 s_rows[DS_WMAX][16 * 8];
  auto load_a = [&](int j) {
    int e, r0, nr;
    ds_locate(sg, j, e, r0, nr);
    if (nr > 0) {  // uniform (always true unless a caller asks for empty segments)
      // Whole 128-byte lines: a0 holds row rt*16 + (lane >> 3), a1 row
      // rt*16 + 8 + (lane >> 3), 16-byte chunk lane & 7 of each K block (the
      // MFMA layout, row lane & 15 and chunks 2g / 2g+1, reads each line in
      // halves: twice the requests).
      const int wr = lane >> 3, wc = lane & 7;
#pragma unroll
      for (int rt = 0; rt < NRT; ++rt) {
        const int64_t lr0 = r0 + min(rt * 16 + wr, nr - 1);
        const int64_t lr1 = r0 + min(rt * 16 + 8 + wr, nr - 1);
        const int64_t xr0 = SWIGLU ? (int64_t)ridx[lr0] : lr0;
        const int64_t xr1 = SWIGLU ? (int64_t)ridx[lr1] : lr1;
        const uint16_t* ar0 = (const uint16_t*)p.x + xr0 * p.ldx + kb0 * 64 + wc * 8;
        const uint16_t* ar1 = (const uint16_t*)p.x + xr1 * p.ldx + kb0 * 64 + wc * 8;
#pragma unroll
        for (int b = 0; b < KBW; ++b) {
          a0[rt][b] = ldg16(ar0 + b * 64);
          a1[rt][b] = ldg16(ar1 + b * 64);
        }
      }
      // to the MFMA layout through the tile (one wave's LDS operations run in
      // order, so each read sees the writes before it)
      uint4* tile = s_rows[ks];
      const int rr = lane & 15, g = lane >> 4;
#pragma unroll
      for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
        for (int b = 0; b < KBW; ++b) {
          tile[wr * 8 + (wc ^ (wr >> 1))] = a0[rt][b];
          tile[(8 + wr) * 8 + (wc ^ ((8 + wr) >> 1))] = a1[rt][b];
          a0[rt][b] = tile[rr * 8 + ((2 * g) ^ (rr >> 1))];
          a1[rt][b] = tile[rr * 8 + ((2 * g + 1) ^ (rr >> 1))];
        }
    } else {
#pragma unroll
      for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
        for (int b = 0; b < KBW; ++b) a0[rt][b] = a1[rt][b] = make_uint4(0u, 0u, 0u, 0u);
    }
    // Wait for the rows here: on the path that reloads them they are the
    // newest loads, and a wait placed after the branch would have to assume
    // that path, draining the whole ring on every unit.
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
      for (int b = 0; b < KBW; ++b)
        asm volatile("" ::"v"(__builtin_bit_cast(u32x4_t, a0[rt][b])), "v"(__builtin_bit_cast(u32x4_t, a1[rt][b])));
  };

  // the first unit's codes go out first, then its rows, then the rest of the ring
  ring.fetch(p, sg, ctn, kb0, kq, lane, 0, u0);
  int cur_j = u0 / ctn;
  load_a(cur_j);
#pragma unroll
  for (int i = 1; i < DS_D; ++i) ring.fetch(p, sg, ctn, kb0, kq, lane, i, min(u0 + i, last));

  const int nthr = nw * 64;
  const int per_buf = nw * NH * NRT * 256;
  int buf = 0;
  // Unit u in ring slot i: its segment's rows, the MFMAs and scale FMAs of the
  // wave's K slice, the refill of slot i with unit `next` (when refill), the
  // partials to LDS, one barrier, and the workgroup's epilogue.
  auto unit = [&](int i, int u, bool refill, int next) {
    const int j = u / ctn;
    if (j != cur_j) {  // uniform: a new segment's rows
      load_a(j);
      cur_j = j;
    }
    const uint8_t* nws[NH];
    const float* nss[NH];
    if (refill) DsRing<SWIGLU, KBW>::unit_src(p, sg, ctn, kb0, kq, lane, next, nws, nss);
    f32x4_t acc[NH][NRT];
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
      for (int rt = 0; rt < NRT; ++rt) acc[h][rt] = z4;
#pragma unroll
    for (int b = 0; b < KBW; ++b) {
      bf16x8_t g0[NH], g1[NH];
      float sc[NH];
#pragma unroll
      for (int h = 0; h < NH; ++h) {
        uint32_t d[8];
        decode4<CANON>(ring.bw[i][b][h].x, d[0], d[1]);
        decode4<CANON>(ring.bw[i][b][h].y, d[2], d[3]);
        decode4<CANON>(ring.bw[i][b][h].z, d[4], d[5]);
        decode4<CANON>(ring.bw[i][b][h].w, d[6], d[7]);
        g0[h] = __builtin_bit_cast(bf16x8_t, make_uint4(d[0], d[1], d[2], d[3]));
        g1[h] = __builtin_bit_cast(bf16x8_t, make_uint4(d[4], d[5], d[6], d[7]));
        sc[h] = ring.sw[i][b][h];
        if (refill) {
          ring.bw[i][b][h] = ldg16(nws[h] + b * L.wk);
          ring.sw[i][b][h] = ldgf(nss[h] + b * L.sk);
        }
      }
#pragma unroll
      for (int rt = 0; rt < NRT; ++rt) {
#pragma unroll
        for (int h = 0; h < NH; ++h) {
          f32x4_t q = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a0[rt][b]), g0[h], z4, 0,
                                                              0, 0);
          q = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a1[rt][b]), g1[h], q, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[h][rt][r] = __builtin_fmaf(sc[h], q[r], acc[h][rt][r]);
        }
      }
    }
    // partials: red[buf][ks][h][rt][lane][r], one 16-byte write per (h, rt)
    float* rb = red + buf * per_buf;
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
      for (int rt = 0; rt < NRT; ++rt)
        *(f32x4_t*)&rb[((ks * NH + h) * NRT + rt) * 256 + lane * 4] = acc[h][rt];
    __syncthreads();
    int e, r0, nr;
    ds_locate(sg, j, e, r0, nr);
    const int ct = u - j * ctn;
    for (int q = threadIdx.x; q < NRT * 256; q += nthr) {
      const int rt = q >> 8, ln = (q >> 2) & 63, r = q & 3;
      const int lr = rt * 16 + (ln >> 4) * 4 + r;
      // all partials are read before the first add (independent LDS reads in
      // flight together), then summed in K-split order
      float pg[DS_WMAX], pu[DS_WMAX];
#pragma unroll
      for (int k2 = 0; k2 < DS_WMAX; ++k2)
        if (k2 < nw) {
          pg[k2] = rb[(k2 * NH) * NRT * 256 + q];
          if constexpr (SWIGLU) pu[k2] = rb[(k2 * NH + 1) * NRT * 256 + q];
        }
      float g = pg[0];
#pragma unroll
      for (int k2 = 1; k2 < DS_WMAX; ++k2)
        if (k2 < nw) g += pg[k2];
      float v = g;
      if constexpr (SWIGLU) {
        float uu = pu[0];
#pragma unroll
        for (int k2 = 1; k2 < DS_WMAX; ++k2)
          if (k2 < nw) uu += pu[k2];
        v = silu_f(bf2f(f2bf(g))) * bf2f(f2bf(uu));
      }
      if (lr < nr) {
        uint16_t* dst = (uint16_t*)p.y + (int64_t)(r0 + lr) * p.ldy + (int64_t)ct * 16 + (ln & 15);
        if constexpr (COH) __hip_atomic_store(dst, (uint16_t)f2bf(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else *dst = (uint16_t)f2bf(v);
      }
    }
    buf ^= 1;
  };
  // Whole rounds of DS_D units with every refill issued (past the range they
  // re-load the last unit, which is never consumed), then a last partial
  // round without refills: no unit is computed twice and no load sits behind
  // a branch inside the rounds.
  const int n = u1 - u0;
  int it = 0;
  for (; it + DS_D < n; it += DS_D) {
#pragma unroll
    for (int i = 0; i < DS_D; ++i) unit(i, u0 + it + i, true, min(u0 + it + i + DS_D, last));
  }
#pragma unroll
  for (int i = 0; i < DS_D; ++i)
    if (it + i < n) unit(i, u0 + it + i, false, 0);  // uniform
}

// Inputs of the dispatch that the gate/up kernel performs itself (FUSED):
// the router's top-k ids and weights of T <= 64 tokens, and where workgroup 0
// writes the dispatch for the later stages.
struct DsDispatch {
  const int64_t* topi;
  const float* topw;
  RouteOut o;
  int T, k;
  int32_t* sync;  // non-null: workgroup 0 clears the fused combine's sync words for the down kernel
};

// The combine + norm + next router fused into the tail of the decode down
// kernel (CNR): the inputs of combine_norm_route_kernel, and the arrival
// count (sync[0]), cleared by the gate/up kernel of the same layer.
struct CnrArgs {
  const int64_t* topi;
  const float* topw;
  const int32_t* inv;
  void* out;
  const float* weight;
  float eps;
  void* norm_out;
  int64_t T;
  int d, k;
  const float* ngw;
  const float* ngb;
  RouteOut no;
  int nE, nk;
  int32_t* sync;
  int64_t ybytes;
  // the arrival count the combining workgroups wait for is gridDim.x +
  // wait_extra (0 in use; smaul_debug_tail_wait raises it so that a test can
  // make the wait give up), polled at most spin_limit times
  int wait_extra;
  int spin_limit;
};
constexpr int CNR_TAIL_TOK = 8;         // tokens per combining workgroup (one per wave)
template <int NCH, int EMAX, bool EXACT, int KSW, int TOK, bool COH>
struct CnrBlock;
constexpr int CNR_SPIN_LIMIT = 1 << 20;  // polls of the arrival count before giving up

// Bounded waits that gave up, per device since the library was loaded (or the
// last reset by smaul_wait_timeouts).  Incremented only on a give-up, so the
// normal path never touches it.
__device__ int32_t g_wait_timeouts = 0;

// The dispatch of the fused gate/up kernel (FUSED below): wave 0 ranks the
// T <= 64 tokens per expert into s_perm / s_off (LDS), workgroup 0 also
// writes the dispatch for the later stages and clears dd.sync; returns the
// segments, with p's pointers.  All threads call it (it ends with a barrier).
__device__ __forceinline__ void ds_fused_dispatch(const GemmArgs& p, const DsDispatch& dd, int lane, DsSegs& sg,
                                                  int32_t* s_perm, int32_t* s_off) {
  ds_pointers(p, lane, sg);
  if (threadIdx.x < 64) {
    const bool valid = lane < dd.T;
    int ti[8];
    float tw[8];
    load_topk(dd.topi, dd.topw, lane, dd.k, valid, p.E, ti, tw);
    const uint64_t sel = valid ? selection_of(ti, tw, p.E, dd.k) : 0ull;
    const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    int off = 0;
    for (int e = 0; e < p.E; ++e) {
      const uint64_t b = __ballot((sel >> e) & 1ull);
      if (lane == 0) s_off[e] = off;
      if ((sel >> e) & 1ull) s_perm[off + __popcll(b & lt)] = lane;
      off += __popcll(b);
    }
    if (lane == 0) s_off[p.E] = off;
    if (blockIdx.x == 0) dispatch_one_wave(ti, tw, valid, lane, dd.o, p.E, dd.k);
    if (blockIdx.x == 0 && lane == 0 && dd.sync) dd.sync[0] = 0;
  }
  __syncthreads();
  ds_finish(lane < p.E ? s_off[lane] : 0, lane < p.E ? s_off[lane + 1] : 0, lane, sg);
}

// Bounded wait of the workgroup until *ctr reaches target (device scope),
// polled by thread 0 at most `limit` times.  Returns true when the target was
// reached; false when the wait gave up, which is counted in g_wait_timeouts.
// Ends with a workgroup barrier.
__device__ __forceinline__ bool ds_wait_all(const int32_t* ctr, int target, int limit) {
  __shared__ int s_reached;
  if (threadIdx.x == 0) {
    int spins = 0, reached = 1;
    while (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
      if (++spins > limit) {
        __hip_atomic_fetch_add(&g_wait_timeouts, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        reached = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    s_reached = reached;
  }
  __syncthreads();
  return s_reached != 0;
}

// A combining workgroup whose wait gave up must not combine rows that other
// workgroups may not have written: wave w instead writes NaN over token t0 +
// w's out and norm_out rows (bf16, d <= 1024) and, for a next router, NaN
// prob / topw and topi -1 (an id that no dispatch takes).
__device__ __forceinline__ void cnr_poison(const CnrArgs& cr, int64_t t0, bool route) {
  const int lane = threadIdx.x & 63;
  const int64_t t = t0 + (threadIdx.x >> 6);
  if (t >= cr.T) return;
  const uint32_t nan2 = 0x7fc07fc0u;  // two bf16 NaNs
  const uint4 nan8 = make_uint4(nan2, nan2, nan2, nan2);
  const int nch = cr.d / 16;
  for (int c = lane; c < nch; c += 64) {
    uint4* o = (uint4*)((char*)cr.out + (t * cr.d + c * 16) * 2);
    o[0] = nan8;
    o[1] = nan8;
    if (cr.norm_out) {
      uint4* n = (uint4*)((char*)cr.norm_out + (t * cr.d + c * 16) * 2);
      n[0] = nan8;
      n[1] = nan8;
    }
  }
  if (route) {
    const float qnan = __uint_as_float(0x7fc00000u);
    if (lane < cr.nE) cr.no.prob[t * cr.nE + lane] = qnan;
    if (lane < cr.nk) {
      cr.no.topi[t * cr.nk + lane] = -1;
      cr.no.topw[t * cr.nk + lane] = qnan;
    }
  }
}

// The combine tail (CNR below) after this workgroup's down units: wait for
// its own device-scope output stores, count itself in *arr; the first
// ceil(T / 8) to arrive prefetch what the combine needs besides y, wait for
// all gridDim.x arrivals and run the combine + norm + next router of 8
// tokens each (or, when the wait gives up, poison those tokens).  Every
// workgroup returns from it.
template <int CEMAX, bool CEXACT>
__device__ __forceinline__ void cnr_tail(const CnrArgs& cr, const void* y, int32_t* arr) {
  __shared__ int s_arrival;
  __builtin_amdgcn_s_waitcnt(0);  // this wave's output stores have completed
  __syncthreads();
  if (threadIdx.x == 0) s_arrival = (int)__hip_atomic_fetch_add(arr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  const int ncw = (int)((cr.T + CNR_TAIL_TOK - 1) / CNR_TAIL_TOK);
  const int a = s_arrival;
  if (a >= ncw) return;  // uniform: the first ncw to arrive combine (they wait longest)
  const int64_t t0 = (int64_t)a * CNR_TAIL_TOK;
  CnrBlock<1, CEMAX, CEXACT, 4, CNR_TAIL_TOK, true> b;
  b.prefetch_slots(cr.topi, cr.topw, cr.inv, cr.weight, cr.T, cr.d, cr.k, t0);
  b.prefetch_router(cr.ngw, cr.ngb, cr.nE, cr.d);
  b.prepare_router(cr.nE, cr.d);
  if (!ds_wait_all(arr, (int)gridDim.x + cr.wait_extra, cr.spin_limit)) {  // uniform
    cnr_poison(cr, t0, true);
    return;
  }
  b.finish(y, cr.ybytes, cr.out, cr.weight, cr.eps, cr.norm_out, cr.T, cr.d, cr.ngw, cr.ngb, cr.no, cr.nE, cr.nk, t0);
}

// The same tail without a next router (defined after CombineNormRow)
template <bool NORM>
__device__ void cn_tail(const CnrArgs& cr, const void* y, int32_t* arr);

// FUSED (gate/up only): every workgroup ranks the T <= 64 tokens per expert
// itself into LDS (one wave, ballot ranks in token order, the same rule as
// dispatch_one_wave) instead of reading a dispatch written by an earlier
// kernel; workgroup 0 also writes that dispatch (counts, seg_off, tile_off,
// perm_row, perm_w, inv) for the down projection and the combine.  The
// top-k is read from dd.topi/dd.topw (the router kernel's output).
//
// TAIL (down only, 8 waves): after its units every workgroup waits for its
// own device-scope output stores, then counts itself in sync[0]; the first
// ceil(T / 8) workgroups to arrive load what the combine needs besides the
// outputs (slots, router weights), wait (a bounded poll: the others are
// already running; a wait that gives up poisons its tokens, cnr_poison, and
// counts itself in g_wait_timeouts) until all have arrived, and each then
// combines 8 tokens,
// reading the outputs device-coherently: TAIL_CNR also normalises them and
// runs the next layer's router (replacing the combine_norm_route_kernel
// launch, with the same arithmetic: CnrBlock), TAIL_CN normalises
// (combine_norm_kernel's arithmetic), TAIL_C only combines (combine_kernel's).
constexpr int TAIL_NONE = 0, TAIL_C = 1, TAIL_CN = 2, TAIL_CNR = 3;
template <bool SWIGLU, bool CANON, int KBW, bool FUSED, int TAIL = TAIL_NONE, int CEMAX = 8, bool CEXACT = false>
__global__ void __launch_bounds__(DS_WMAX * 64)
decode_stream_kernel(GemmArgs p, int nw, DsDispatch dd, CnrArgs cr) {
  constexpr int NH = SWIGLU ? 2 : 1;
  static_assert(!FUSED || SWIGLU, "the fused dispatch feeds the gate/up projection");
  // the partial sums of the GEMM
  constexpr int RED_FLOATS = 2 * DS_WMAX * NH * (DS_ROWS / 16) * 256;
  __shared__ __attribute__((aligned(16))) float red[RED_FLOATS];
  __shared__ int32_t s_perm[FUSED ? 64 * 8 : 1];
  __shared__ int32_t s_off[FUSED ? MAX_E + 1 : 1];
  const int lane = threadIdx.x & 63;
  const int ctn = (int)(p.N >> 4);
  DsSegs sg;
  if constexpr (FUSED) {
    ds_fused_dispatch(p, dd, lane, sg, s_perm, s_off);
  } else {
    sg = ds_segments(p, lane);
  }
  const int32_t* ridx = FUSED ? (const int32_t*)s_perm : p.row_idx;
  const int64_t U = (int64_t)sg.total * ctn;
  // Workgroup b runs on XCD b % 8: the 8 XCDs take contiguous eighths of the
  // unit list, so a segment's activation rows are read into one or two L2s
  // rather than all eight.
  const int G = (int)gridDim.x;
  const int gx = G % 8 == 0 ? (int)(blockIdx.x % 8) * (G / 8) + (int)(blockIdx.x / 8) : (int)blockIdx.x;
  const int u0 = (int)((int64_t)gx * U / G);
  const int u1 = (int)((int64_t)(gx + 1) * U / G);
  constexpr bool COH = TAIL != TAIL_NONE;
  static_assert(!COH || !SWIGLU, "the combine follows the down projection");
  if constexpr (!COH) {
    if (u0 >= u1) return;  // uniform per workgroup
  }
  if (u0 < u1) {
    // two row tiles when any segment has more than 16 rows
    if (__ballot(sg.rows > 16) != 0) ds_body<SWIGLU, CANON, KBW, 2, COH>(p, sg, ridx, u0, u1, ctn, red, nw);
    else ds_body<SWIGLU, CANON, KBW, 1, COH>(p, sg, ridx, u0, u1, ctn, red, nw);
  }
  if constexpr (TAIL == TAIL_CNR) cnr_tail<CEMAX, CEXACT>(cr, p.y, cr.sync);
  if constexpr (TAIL == TAIL_CN || TAIL == TAIL_C) cn_tail<TAIL == TAIL_CN>(cr, p.y, cr.sync);
}

// K blocks per wave of the streaming decode kernel for K/64 = nkb blocks
// (at most DS_WMAX waves), or 0 when no instance fits
int ds_kbw(int64_t nkb, bool swiglu) {
  // gate/up beyond 2 blocks per wave, and 4 blocks per wave for down, spill
  // registers with rows held for up to 64 tokens; those shapes run
  // decode_gemm_kernel
  const int cand[2] = {2, 5};
  for (int kb : cand) {
    if (swiglu && kb != 2) continue;
    if (nkb % kb == 0 && nkb / kb <= DS_WMAX) return kb;
  }
  return 0;
}

// compute units of the current device (cached per device)
int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// Returns 1 when the shape has no streaming instance (the caller then runs
// decode_gemm_kernel), else the launch status.  dd != nullptr: the gate/up
// kernel performs the dispatch itself (FUSED).
template <bool SWIGLU, bool CANON>
int launch_decode_stream(const GemmArgs& a, const DsDispatch* dd, hipStream_t stream) {
  const int64_t nkb = a.K / 64;
  if (a.N % 16 != 0 || a.E > 64) return 1;
  const int kbw = ds_kbw(nkb, SWIGLU);
  if (kbw == 0) return 1;
  const int nw = (int)(nkb / kbw);
  const int64_t ctn = a.N / 16;
  // units: at most E * ctn * (64 / DS_ROWS) in the decode regime; a grid of
  // one workgroup per CU, never more workgroups than that
  const int64_t g = std::min<int64_t>(cu_count(), std::max<int64_t>(1, a.E * ctn * (64 / DS_ROWS)));
  const DsDispatch none{};
  const dim3 grid((unsigned)g), block(nw * 64);
  if constexpr (SWIGLU) {
    if (dd) {
      hipLaunchKernelGGL((decode_stream_kernel<true, CANON, 2, true>), grid, block, 0, stream, a, nw, *dd, CnrArgs{});
      return check_launch("decode_stream_kernel");
    }
  }
  if (kbw == 2) {
    hipLaunchKernelGGL((decode_stream_kernel<SWIGLU, CANON, 2, false>), grid, block, 0, stream, a, nw, none, CnrArgs{});
  } else {
    if constexpr (!SWIGLU)
      hipLaunchKernelGGL((decode_stream_kernel<false, CANON, 5, false>), grid, block, 0, stream, a, nw, none, CnrArgs{});
  }
  return check_launch("decode_stream_kernel");
}

// The decode down projection with the combine + norm + next router in its
// tail (CNR).  Returns 1 when the shape has no such instance: canonical codes,
// 8 K-split waves (one per combined token of a workgroup), a router of 4 < E
// <= 16 experts on d <= 1024, and at least ceil(T / 8) workgroups.
template <int EMAX, bool EXACT>
int launch_down_cnr_e(const GemmArgs& a, int kbw, int64_t g, const CnrArgs& cr, hipStream_t stream) {
  const DsDispatch none{};
  const dim3 grid((unsigned)g), block(8 * 64);
  if (kbw == 2)
    hipLaunchKernelGGL((decode_stream_kernel<false, true, 2, false, TAIL_CNR, EMAX, EXACT>), grid, block, 0, stream,
                       a, 8, none, cr);
  else
    hipLaunchKernelGGL((decode_stream_kernel<false, true, 5, false, TAIL_CNR, EMAX, EXACT>), grid, block, 0, stream,
                       a, 8, none, cr);
  return check_launch("decode_stream_kernel");
}

int launch_down_cnr(const GemmArgs& a, bool canon, const CnrArgs& cr, hipStream_t stream) {
  if (!canon || a.N % 16 != 0 || a.E > 64 || cr.d > 1024 || cr.nE <= 4 || cr.nE > 16) return 1;
  const int64_t nkb = a.K / 64;
  const int kbw = ds_kbw(nkb, false);
  if (kbw == 0 || nkb / kbw != 8) return 1;
  const int64_t ctn = a.N / 16;
  const int64_t g = std::min<int64_t>(cu_count(), std::max<int64_t>(1, a.E * ctn * (64 / DS_ROWS)));
  if (g < (cr.T + CNR_TAIL_TOK - 1) / CNR_TAIL_TOK) return 1;
  if (cr.nE == 16) return launch_down_cnr_e<16, true>(a, kbw, g, cr, stream);
  if (cr.nE > 8) return launch_down_cnr_e<16, false>(a, kbw, g, cr, stream);
  if (cr.nE == 8) return launch_down_cnr_e<8, true>(a, kbw, g, cr, stream);
  return launch_down_cnr_e<8, false>(a, kbw, g, cr, stream);
}

// The decode down projection with the combine (norm: and the output RMSNorm)
// in its tail, for layers without a next router.  Returns 1 when the shape
// has no such instance: canonical codes, 8 K-split waves, d <= 1024 and at
// least ceil(T / 8) workgroups.
int launch_down_cn(const GemmArgs& a, bool canon, const CnrArgs& cr, bool norm, hipStream_t stream) {
  if (!canon || a.N % 16 != 0 || a.E > 64 || cr.d > 1024) return 1;
  const int64_t nkb = a.K / 64;
  const int kbw = ds_kbw(nkb, false);
  if (kbw == 0 || nkb / kbw != 8) return 1;
  const int64_t ctn = a.N / 16;
  const int64_t g = std::min<int64_t>(cu_count(), std::max<int64_t>(1, a.E * ctn * (64 / DS_ROWS)));
  if (g < (cr.T + CNR_TAIL_TOK - 1) / CNR_TAIL_TOK) return 1;
  const DsDispatch none{};
  const dim3 grid((unsigned)g), block(8 * 64);
#define SMAUL_CN(KB, TL) \
  hipLaunchKernelGGL((decode_stream_kernel<false, true, KB, false, TL>), grid, block, 0, stream, a, 8, none, cr)
  if (kbw == 2) {
    if (norm) SMAUL_CN(2, TAIL_CN);
    else SMAUL_CN(2, TAIL_C);
  } else {
    if (norm) SMAUL_CN(5, TAIL_CN);
    else SMAUL_CN(5, TAIL_C);
  }
#undef SMAUL_CN
  return check_launch("decode_stream_kernel");
}

template <bool SWIGLU, bool CANON>
int launch_decode(const GemmArgs& a, hipStream_t stream) {
  if (SWIGLU != (a.row_idx != nullptr)) return fail(SMAUL_ERR_INVALID, "decode gemm: row gather mismatch");
  {
    const int rc = launch_decode_stream<SWIGLU, CANON>(a, nullptr, stream);
    if (rc != 1) return rc;
  }
  const int64_t nkb = a.K / 64;
  for (int db = 4; db >= 2; db /= 2)
    for (int ks = DecodeKS<SWIGLU>::MAX; ks >= 1; --ks) {
      if (nkb % ks != 0 || (nkb / ks) % db != 0) continue;
      if (db == 4) return launch_decode_db<SWIGLU, CANON, 4>(a, ks, stream);
      return launch_decode_db<SWIGLU, CANON, 2>(a, ks, stream);
    }
  return fail(SMAUL_ERR_INVALID, "decode gemm: K/64 must be even");
}

// ---------------------------------------------------------------------------
// router: logits, softmax, top-k (torch CPU order), renormalisation
// ---------------------------------------------------------------------------
// A workgroup of 4 waves owns a block of TB*4 tokens (32 when E <= 4, 16
// when E <= 16, else 4), so a CU holds several blocks whose phases overlap and
// a 64-token decode step spreads over several CUs.  The router weight is staged in LDS (in column
// chunks of at most 32 KB); inside a wave the 64 lanes split the model
// dimension into 8-wide groups (coalesced 16-byte loads of x), each lane keeps
// TB tokens x EMAX experts of partial dot products, and a butterfly over the
// lanes completes them.  One thread per token then runs softmax, the top-k
// selection and the renormalisation, and the block's per-expert dispatch
// counts are written for the dispatch scan.  With a single block (T <= TB*4)
// the same workgroup also performs the dispatch.
template <bool XBF16, int TB, int EMAX, bool EXACT>
__global__ void __launch_bounds__(ROUTE_THREADS)
router_kernel(const void* __restrict__ x, const float* __restrict__ gw, const float* __restrict__ gb,
              RouteOut o, int64_t T, int d, int E_arg, int k) {
  // EXACT: E == EMAX, so every expert guard below is decided at compile time
  const int E = EXACT ? EMAX : E_arg;
  constexpr int TPB = TB * ROUTE_WAVES;
  __shared__ __attribute__((aligned(16))) float sW[ROUTE_WFLOATS];
  __shared__ float slog[TPB][EMAX];
  __shared__ smaul_topk::Pair spair[TPB][EMAX];
  __shared__ int s_ti[TPB][8];
  __shared__ float s_tw[TPB][8];
  __shared__ int s_cnt[EMAX];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t t0 = (int64_t)blockIdx.x * TPB;
  if (tid < EMAX) s_cnt[tid] = 0;

  // ---- logits: this wave's TB tokens ---------------------------------------
  // Weight rows e >= E are staged as zeros, so the loops below carry no
  // expert guard and unroll fully.
  const int64_t tw0 = t0 + wave * TB;
  float acc[TB * EMAX];
#pragma unroll
  for (int i = 0; i < TB * EMAX; ++i) acc[i] = 0.0f;
  // Model columns are processed in chunks of DC (the router-weight chunk that
  // fits the 32 KB LDS stage).  Per chunk the activations are loaded first:
  // they do not depend on the staged weights, so their latency overlaps the
  // weight staging, and every load of a chunk is in flight before any is
  // used.  The fp32 summation order (per lane: column groups in ascending
  // order, then the butterfly) does not depend on this load order.
  constexpr int DC = RouteShape<EMAX>::DC;
  constexpr int XG = RouteShape<EMAX>::XG;
  constexpr int WI = (EMAX * DC / 4 + ROUTE_THREADS - 1) / ROUTE_THREADS;  // weight float4s per thread
  constexpr int XW = XBF16 ? 1 : 2;                                         // 16-byte loads per group
  for (int c0 = 0; c0 < d; c0 += DC) {
    const int cw = min(DC, d - c0);  // d % 8 == 0
    uint4 xr[XG][TB][XW];
    route_load_x<XBF16, TB, EMAX>(x, T, tw0, c0, cw, d, lane, xr);
    __syncthreads();  // the previous chunk's readers are done with sW
    const int nw = EMAX * (cw >> 2);
    float4 wv[WI];
#pragma unroll
    for (int i = 0; i < WI; ++i) {
      const int idx = tid + i * ROUTE_THREADS;
      const int e = idx / (cw >> 2), qq = idx % (cw >> 2);
      wv[i] = (idx < nw && e < E) ? *(const float4*)(gw + (int64_t)e * d + c0 + qq * 4) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int i = 0; i < WI; ++i) {
      const int idx = tid + i * ROUTE_THREADS;
      if (idx < nw) *(float4*)&sW[(idx / (cw >> 2)) * cw + (idx % (cw >> 2)) * 4] = wv[i];
    }
    __syncthreads();
    route_fma<XBF16, TB, EMAX>(xr, sW, cw, lane, acc);
  }
  {
    const int vidx = route_butterfly<TB, EMAX>(acc, lane);
    const int a = vidx / EMAX, e = vidx % EMAX;
    const bool writer = TB * EMAX == 64 || (lane & 1) == 0;
    if (writer && e < E) slog[wave * TB + a][e] = gb ? acc[0] + gb[e] : acc[0];
  }
  __syncthreads();

  // ---- per token: softmax, top-k, renormalisation (model.py:558-570) --------
  if (tid < TPB) {
    const int64_t t = t0 + tid;
    if (t < T) {
      int ti[8];
      float tv[8];
      route_select<EMAX>(slog[tid], spair[tid], E, k, t, o, true, ti, tv);
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (j < k) {
          s_ti[tid][j] = ti[j];
          s_tw[tid][j] = tv[j];
        }
      const uint64_t sel = selection_of(ti, tv, E, k);
      for (int e = 0; e < E; ++e)
        if ((sel >> e) & 1ull) atomicAdd(&s_cnt[e], 1);
    }
  }
  __syncthreads();
  if (o.blockcnt && tid < E) o.blockcnt[(int64_t)blockIdx.x * E + tid] = s_cnt[tid];

  // ---- fused dispatch for a single block (T <= TPB) ---------------------------
  if (o.counts && gridDim.x == 1 && wave == 0) {
    const bool valid = lane < T && lane < TPB;
    dispatch_one_wave(s_ti[valid ? lane : 0], s_tw[valid ? lane : 0], valid, lane, o, E, k);
  }
}

// bf16 activations, E <= 16: the logits on the matrix cores (route_logits,
// 64 tokens per workgroup of 8 waves), then the per-token softmax / top-k /
// renormalisation by groups of EMAX lanes, block counts and the single-block
// dispatch, as router_kernel.
constexpr int ROUTE_MFMA_TPB = RK_TOK;
constexpr int ROUTE_MFMA_THREADS = 512;

// NTT token tiles of 16 per block: 4 (ROUTE_MFMA_TPB tokens) in general, 1
// for the decode step, where a block per 16 tokens shortens each block's
// loads; the arithmetic per token is the same either way.
template <int EMAX, bool EXACT, int KSW, int NTT>
__global__ void __launch_bounds__(ROUTE_MFMA_THREADS)
router_mfma_kernel(const uint16_t* __restrict__ x, const float* __restrict__ gw, const float* __restrict__ gb,
                   RouteOut o, int64_t T, int d, int E_arg, int k) {
  static_assert(EMAX <= 16, "the MFMA router covers up to 16 experts");
  const int E = EXACT ? EMAX : E_arg;
  constexpr int TPB = NTT * 16;
  constexpr int NWAVES = ROUTE_MFMA_THREADS / 64;
  __shared__ __attribute__((aligned(16))) float part[RK_SLICES * TPB * 16];
  __shared__ float slog[TPB][EMAX];
  __shared__ smaul_topk::Pair spair[TPB][EMAX];
  __shared__ int s_ti[TPB][8];
  __shared__ float s_tw[TPB][8];
  __shared__ int s_cnt[EMAX];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t t0 = (int64_t)blockIdx.x * TPB;
  if (tid < EMAX) s_cnt[tid] = 0;
  route_logits<KSW, EMAX, NTT>(x, gw, gb, E, T, t0, d, NWAVES, part, slog);

  {
    // EMAX lanes per token
    constexpr int TPW = 64 / EMAX;
    for (int tl = wave * TPW + (lane / EMAX); tl < TPB; tl += NWAVES * TPW) {
      const int64_t t = t0 + tl;
      route_select_group<EMAX>(slog[tl], spair[tl], E, k, t, t < T, o, true, s_ti[tl], s_tw[tl], s_cnt);
    }
  }
  __syncthreads();
  if (o.blockcnt && tid < E) o.blockcnt[(int64_t)blockIdx.x * E + tid] = s_cnt[tid];
  if (o.counts && gridDim.x == 1 && wave == 0) {
    const bool valid = lane < T && lane < TPB;
    dispatch_one_wave(s_ti[valid ? lane : 0], s_tw[valid ? lane : 0], valid, lane, o, E, k);
  }
}

// ---------------------------------------------------------------------------
// dispatch for many blocks: counts per block, scan over blocks, ranked scatter
// ---------------------------------------------------------------------------
// Per-expert order is ascending token index (the boolean-mask gather order of
// model.py:574-581): blocks are consecutive token ranges, a block's tokens are
// ranked by ballot in token order, and each block starts at the exclusive
// scan of the earlier blocks' counts.
constexpr int DISPATCH_TPB = 64;

__device__ __forceinline__ uint64_t token_selection(const int64_t* topi, const float* topw, int64_t t,
                                                    int E, int k) {
  int ti[8];
  float tw[8];
  for (int j = 0; j < k; ++j) {
    const int64_t v = topi[t * k + j];
    ti[j] = (v >= 0 && v < E) ? (int)v : -1;
    tw[j] = topw[t * k + j];
  }
  return selection_of(ti, tw, E, k);
}

__global__ void __launch_bounds__(64)
block_count_kernel(const int64_t* __restrict__ topi, const float* __restrict__ topw,
                   int32_t* __restrict__ blockcnt, int64_t T, int E, int k, int tpb) {
  const int lane = threadIdx.x;
  const int64_t t = (int64_t)blockIdx.x * tpb + lane;
  const uint64_t sel = (lane < tpb && t < T) ? token_selection(topi, topw, t, E, k) : 0ull;
  for (int e = 0; e < E; ++e) {
    const int n = __popcll(__ballot((sel >> e) & 1ull));
    if (lane == 0) blockcnt[(int64_t)blockIdx.x * E + e] = n;
  }
}

// One wave per expert: a running exclusive scan of the per-block counts in
// chunks of 64 blocks (shuffle prefix sums), then one thread turns the totals
// into segment and tile offsets.  blockoff is relative to the segment start.
constexpr int SCAN_THREADS = 1024;

__global__ void __launch_bounds__(SCAN_THREADS)
dispatch_scan_kernel(const int32_t* __restrict__ blockcnt, int32_t* __restrict__ blockoff,
                     int32_t* __restrict__ counts, int32_t* __restrict__ seg_off,
                     int32_t* __restrict__ tile_off, int64_t nb, int E, int block_m) {
  __shared__ int s_tot[MAX_E];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int e = wave; e < E; e += SCAN_THREADS / 64) {
    int running = 0;
    for (int64_t b0 = 0; b0 < nb; b0 += 64) {
      const int64_t b = b0 + lane;
      const int v = b < nb ? blockcnt[b * E + e] : 0;
      int inc = v;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(inc, o, 64);
        if (lane >= o) inc += u;
      }
      if (b < nb) blockoff[b * E + e] = running + inc - v;
      running += __shfl(inc, 63, 64);
    }
    if (lane == 0) s_tot[e] = running;
  }
  __syncthreads();
  if (tid == 0) {
    int base = 0, tbase = 0;
    for (int e = 0; e < E; ++e) {
      counts[e] = s_tot[e];
      seg_off[e] = base;
      tile_off[e] = tbase;
      base += s_tot[e];
      tbase += (s_tot[e] + block_m - 1) / block_m;
    }
    seg_off[E] = base;
    tile_off[E] = tbase;
  }
}

__global__ void __launch_bounds__(64)
dispatch_scatter_kernel(const int64_t* __restrict__ topi, const float* __restrict__ topw,
                        const int32_t* __restrict__ blockoff, const int32_t* __restrict__ seg_off,
                        int32_t* __restrict__ perm_row, float* __restrict__ perm_w, int32_t* __restrict__ inv,
                        int64_t T, int E, int k, int tpb) {
  const int lane = threadIdx.x;
  const int64_t t = (int64_t)blockIdx.x * tpb + lane;
  const bool valid = lane < tpb && t < T;
  int ti[8];
  float tw[8];
  uint64_t sel = 0;
  if (valid) {
    for (int j = 0; j < k; ++j) {
      const int64_t v = topi[t * k + j];
      ti[j] = (v >= 0 && v < E) ? (int)v : -1;
      tw[j] = topw[t * k + j];
    }
    sel = selection_of(ti, tw, E, k);
  }
  const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  const int32_t* off = blockoff + (int64_t)blockIdx.x * E;
  for (int e = 0; e < E; ++e) {
    const uint64_t b = __ballot((sel >> e) & 1ull);
    if ((sel >> e) & 1ull) {
      const int pos = seg_off[e] + off[e] + __popcll(b & lt);
      perm_row[pos] = (int32_t)t;
      for (int j = 0; j < k; ++j)
        if (ti[j] == e && tw[j] > 0.0f) {
          perm_w[pos] = tw[j];
          inv[t * k + j] = pos;
          break;
        }
    }
  }
  if (valid) {
    uint64_t seen = 0;
    for (int j = 0; j < k; ++j) {
      const int ee = ti[j];
      const bool ok = tw[j] > 0.0f && ee >= 0 && ee < E && !((seen >> ee) & 1ull);
      if (ok) seen |= 1ull << ee;
      else inv[t * k + j] = -1;
    }
  }
}

// Scan and scatter in one launch (E <= EMAX <= 16): every block sums the
// per-block expert counts of all blocks itself, its own prefix and the totals
// (integer sums: the offsets of dispatch_scan_kernel), block 0 writes counts,
// seg_off and tile_off, and the scatter follows as in dispatch_scatter_kernel.
// The count reads are issued with the token's top-k reads, so the scan costs
// no round trip of its own.  Launched only for nb <= SCAN_FUSED_CHUNKS * 64
// blocks (the unrolled count reads cover every block).
constexpr int SCAN_FUSED_CHUNKS = 4;  // count reads unrolled for up to 4 * 64 blocks
template <int EMAX>
__global__ void __launch_bounds__(64)
dispatch_scan_scatter_kernel(const int64_t* __restrict__ topi, const float* __restrict__ topw,
                             const int32_t* __restrict__ blockcnt, int32_t* __restrict__ counts,
                             int32_t* __restrict__ seg_off_out, int32_t* __restrict__ tile_off,
                             int32_t* __restrict__ perm_row, float* __restrict__ perm_w, int32_t* __restrict__ inv,
                             int64_t T, int E, int k, int tpb, int64_t nb, int block_m) {
  const int lane = threadIdx.x;
  const int64_t t = (int64_t)blockIdx.x * tpb + lane;
  const bool valid = lane < tpb && t < T;
  int ti[8];
  float tw[8];
  load_topk(topi, topw, t, k, valid, E, ti, tw);
  int before[EMAX], total[EMAX];
#pragma unroll
  for (int e = 0; e < EMAX; ++e) before[e] = total[e] = 0;
  auto add_block = [&](int64_t b, int v, int e) {
    total[e] += v;
    if (b < (int64_t)blockIdx.x) before[e] += v;
  };
  int cv[SCAN_FUSED_CHUNKS][EMAX];
#pragma unroll
  for (int c = 0; c < SCAN_FUSED_CHUNKS; ++c) {
    const int64_t b = c * 64 + lane;
#pragma unroll
    for (int e = 0; e < EMAX; ++e) cv[c][e] = (e < E && b < nb) ? blockcnt[b * E + e] : 0;
  }
#pragma unroll
  for (int c = 0; c < SCAN_FUSED_CHUNKS; ++c)
#pragma unroll
    for (int e = 0; e < EMAX; ++e) add_block(c * 64 + lane, cv[c][e], e);
#pragma unroll
  for (int e = 0; e < EMAX; ++e)
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      before[e] += __shfl_xor(before[e], o, 64);
      total[e] += __shfl_xor(total[e], o, 64);
    }
  int segoff[EMAX];
  int base = 0, tbase = 0;
#pragma unroll
  for (int e = 0; e < EMAX; ++e)
    if (e < E) {
      segoff[e] = base;
      if (blockIdx.x == 0 && lane == 0) {
        counts[e] = total[e];
        seg_off_out[e] = base;
        tile_off[e] = tbase;
      }
      base += total[e];
      tbase += (total[e] + block_m - 1) / block_m;
    }
  if (blockIdx.x == 0 && lane == 0) {
    seg_off_out[E] = base;
    tile_off[E] = tbase;
  }
  const uint64_t sel = valid ? selection_of(ti, tw, E, k) : 0ull;
  const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
  for (int e = 0; e < EMAX; ++e) {
    if (e < E) {  // uniform: every lane takes part in the ballot
      const uint64_t b = __ballot((sel >> e) & 1ull);
      if ((sel >> e) & 1ull) {
        const int pos = segoff[e] + before[e] + __popcll(b & lt);
        perm_row[pos] = (int32_t)t;
        for (int j = 0; j < k; ++j)
          if (ti[j] == e && tw[j] > 0.0f) {
            perm_w[pos] = tw[j];
            inv[t * k + j] = pos;
            break;
          }
      }
    }
  }
  if (valid) {
    uint64_t seen = 0;
    for (int j = 0; j < k; ++j) {
      const int ee = ti[j];
      const bool ok = tw[j] > 0.0f && ee >= 0 && ee < E && !((seen >> ee) & 1ull);
      if (ok) seen |= 1ull << ee;
      else inv[t * k + j] = -1;
    }
  }
}

// Dispatch of at most 64 tokens in one wave, straight from the router outputs
// (the decode regime: one launch instead of block counts, scan and scatter).
__global__ void __launch_bounds__(64)
dispatch_small_kernel(const int64_t* __restrict__ topi, const float* __restrict__ topw, RouteOut o, int64_t T,
                      int E, int k) {
  const int lane = threadIdx.x;
  const bool valid = lane < T;
  int ti[8];
  float tw[8];
  load_topk(topi, topw, lane, k, valid, E, ti, tw);
  dispatch_one_wave(ti, tw, valid, lane, o, E, k);
}

// ---------------------------------------------------------------------------
// combine: out[t] = cast(sum over ascending expert id of y * w), fp32, no FMA
// ---------------------------------------------------------------------------
// The dispatched slots of token t (inv >= 0) as (yperm row, weight) in
// ascending expert id, the summation order of the combine; returns their
// count.  Every inv/topi/topw read of the token is issued before the first is
// used, and the slots are ordered by an odd-even transposition sort over
// fixed register indices (dispatched experts of a token are distinct).
__device__ __forceinline__ int combine_slots(const int64_t* topi, const float* topw, const int32_t* inv, int64_t t,
                                             int k, int (&rw)[8], float (&wt)[8]) {
  int pos[8], key[8];
  int64_t ti[8];
#pragma unroll
  for (int j = 0; j < 8; ++j)
    if (j < k) {
      pos[j] = inv[t * k + j];
      ti[j] = topi[t * k + j];
      wt[j] = topw[t * k + j];
    }
  int n = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const bool live = j < k && pos[j] >= 0;
    key[j] = live ? (int)ti[j] : 0x7fffffff;
    rw[j] = live ? pos[j] : 0;
    n += live ? 1 : 0;
  }
#pragma unroll
  for (int pass = 0; pass < 8; ++pass) {
    if (pass >= k) break;  // k passes sort k keys
#pragma unroll
    for (int i = pass & 1; i + 1 < 8; i += 2) {
      if (i + 1 >= k) break;
      if (key[i] > key[i + 1]) {
        const int tk = key[i], tr = rw[i];
        const float tw = wt[i];
        key[i] = key[i + 1];
        rw[i] = rw[i + 1];
        wt[i] = wt[i + 1];
        key[i + 1] = tk;
        rw[i + 1] = tr;
        wt[i + 1] = tw;
      }
    }
  }
  return n;
}

template <bool BF16, int CW, int KM>
__global__ void __launch_bounds__(256)
combine_kernel(const void* __restrict__ yperm, const int64_t* __restrict__ topi,
               const float* __restrict__ topw, const int32_t* __restrict__ inv,
               void* __restrict__ out, int64_t T, int d, int k) {
  // a thread handles CW columns of one token (the widest of 32, 16, 8 that
  // divides d; 32 for bf16 only) as NV 16-byte chunks: chunk v of the
  // token's thread j is chunk v * cpt + j of the row, so the threads of a
  // token read (and write) consecutive chunks with each instruction, whole
  // cache lines.  Every row load of its k <= KM slots is issued before the
  // first product, and registers are held for KM slots only.
  static_assert(CW == 8 || CW == 16 || (CW == 32 && BF16), "columns per thread");
  static_assert(KM == 2 || KM == 4 || KM == 8, "slots per token");
  constexpr int EPC = BF16 ? 8 : 4;            // elements per 16-byte chunk
  constexpr int NV = CW / EPC;                 // chunks per thread
  const int cpt = d / CW;                      // threads per token (d % CW == 0)
  const int64_t gidx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t t = gidx / cpt;
  if (t >= T) return;
  const int j = (int)(gidx % cpt);
  int rw[8];
  float wt[8];
  const int n = combine_slots(topi, topw, inv, t, k, rw, wt);
  uint4 yv[KM][NV];
#pragma unroll
  for (int s = 0; s < KM; ++s)
    if (s < n) {
      const char* src = (const char*)yperm + (int64_t)rw[s] * d * (BF16 ? 2 : 4);
#pragma unroll
      for (int v = 0; v < NV; ++v) yv[s][v] = ldg16(src + (int64_t)(v * cpt + j) * 16);
    }
  float acc[CW];
#pragma unroll
  for (int q = 0; q < CW; ++q) acc[q] = 0.0f;
#pragma unroll
  for (int s = 0; s < KM; ++s)
    if (s < n) {
      float y[CW];
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        if constexpr (BF16) {
          const uint4 w = yv[s][v];
          y[v * 8 + 0] = bf2f(w.x & 0xffff); y[v * 8 + 1] = bf2f(w.x >> 16);
          y[v * 8 + 2] = bf2f(w.y & 0xffff); y[v * 8 + 3] = bf2f(w.y >> 16);
          y[v * 8 + 4] = bf2f(w.z & 0xffff); y[v * 8 + 5] = bf2f(w.z >> 16);
          y[v * 8 + 6] = bf2f(w.w & 0xffff); y[v * 8 + 7] = bf2f(w.w >> 16);
        } else {
          const uint4 w = yv[s][v];
          y[v * 4 + 0] = __uint_as_float(w.x); y[v * 4 + 1] = __uint_as_float(w.y);
          y[v * 4 + 2] = __uint_as_float(w.z); y[v * 4 + 3] = __uint_as_float(w.w);
        }
      }
#pragma unroll
      for (int q = 0; q < CW; ++q) {
        const float pr = y[q] * wt[s];  // rounded product (library built with -ffp-contract=off)
        acc[q] = acc[q] + pr;
      }
    }
  if constexpr (BF16) {
    uint4* dst = (uint4*)((uint16_t*)out + t * d);
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      uint4 o;
      o.x = f2bf(acc[v * 8 + 0]) | (f2bf(acc[v * 8 + 1]) << 16);
      o.y = f2bf(acc[v * 8 + 2]) | (f2bf(acc[v * 8 + 3]) << 16);
      o.z = f2bf(acc[v * 8 + 4]) | (f2bf(acc[v * 8 + 5]) << 16);
      o.w = f2bf(acc[v * 8 + 6]) | (f2bf(acc[v * 8 + 7]) << 16);
      dst[v * cpt + j] = o;
    }
  } else {
    float4* dst = (float4*)((float*)out + t * d);
#pragma unroll
    for (int v = 0; v < NV; ++v)
      dst[v * cpt + j] = make_float4(acc[v * 4], acc[v * 4 + 1], acc[v * 4 + 2], acc[v * 4 + 3]);
  }
}

// ---------------------------------------------------------------------------
// RMSNorm over rows: out = cast((x * rsqrt(mean(x^2) + eps)) * weight), fp32
// ---------------------------------------------------------------------------
// One wave per row, four rows per workgroup.  VEC (d a multiple of 16,
// 16-byte aligned rows): lane l owns the 16-column chunks l, l+64, ...; the row
// sum of squares adds each chunk left to right, the chunks in order, then the
// lanes by butterfly (rms_chunk_sumsq, wave_sum).  combine_norm_kernel sums in
// exactly this order, so the fused MoE output norm and this kernel agree
// bitwise.  The first RMS_KEEP chunks of a lane stay in registers between the
// reduction and the scaling pass; chunks past them are read again.
constexpr int RMS_KEEP = 4;

__device__ __forceinline__ float rms_chunk_sumsq(float ss, const float (&f)[16]) {
#pragma unroll
  for (int q = 0; q < 16; ++q) ss = ss + f[q] * f[q];
  return ss;
}

// 16 values (bf16 or fp32) from VPC 16-byte vectors
template <bool BF16>
__device__ __forceinline__ void rms_unpack(const uint4* v, float (&f)[16]) {
  if constexpr (BF16) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      f[j * 8 + 0] = bf2f(v[j].x & 0xffff); f[j * 8 + 1] = bf2f(v[j].x >> 16);
      f[j * 8 + 2] = bf2f(v[j].y & 0xffff); f[j * 8 + 3] = bf2f(v[j].y >> 16);
      f[j * 8 + 4] = bf2f(v[j].z & 0xffff); f[j * 8 + 5] = bf2f(v[j].z >> 16);
      f[j * 8 + 6] = bf2f(v[j].w & 0xffff); f[j * 8 + 7] = bf2f(v[j].w >> 16);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f[j * 4 + 0] = __uint_as_float(v[j].x); f[j * 4 + 1] = __uint_as_float(v[j].y);
      f[j * 4 + 2] = __uint_as_float(v[j].z); f[j * 4 + 3] = __uint_as_float(v[j].w);
    }
  }
}

// (f * r) * weight for 16 columns from c0, cast and stored at dst and/or
// lds_dst (either may be null)
template <bool BF16>
__device__ __forceinline__ void rms_scale_store_w(const float (&f)[16], float r, const float (&wv)[16], bool hasw,
                                                  char* dst, char* lds_dst = nullptr) {
  float o[16];
#pragma unroll
  for (int q = 0; q < 16; ++q) o[q] = f[q] * r;
  if (hasw) {
#pragma unroll
    for (int q = 0; q < 16; ++q) o[q] = o[q] * wv[q];
  }
  if constexpr (BF16) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      uint4 w;
      w.x = f2bf(o[j * 8 + 0]) | (f2bf(o[j * 8 + 1]) << 16);
      w.y = f2bf(o[j * 8 + 2]) | (f2bf(o[j * 8 + 3]) << 16);
      w.z = f2bf(o[j * 8 + 4]) | (f2bf(o[j * 8 + 5]) << 16);
      w.w = f2bf(o[j * 8 + 6]) | (f2bf(o[j * 8 + 7]) << 16);
      if (dst) ((uint4*)dst)[j] = w;
      if (lds_dst) ((uint4*)lds_dst)[j] = w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float4 w = make_float4(o[j * 4], o[j * 4 + 1], o[j * 4 + 2], o[j * 4 + 3]);
      if (dst) ((float4*)dst)[j] = w;
      if (lds_dst) ((float4*)lds_dst)[j] = w;
    }
  }
}

// the same with the norm weight read here (all 16 loads in flight before the first product)
template <bool BF16>
__device__ __forceinline__ void rms_scale_store(const float (&f)[16], float r, const float* weight, int c0,
                                                char* dst, char* lds_dst = nullptr) {
  float wv[16];
  if (weight) {
#pragma unroll
    for (int q = 0; q < 16; ++q) wv[q] = ldgf(weight + c0 + q);
  }
  rms_scale_store_w<BF16>(f, r, wv, weight != nullptr, dst, lds_dst);
}

template <bool BF16, bool VEC>
__global__ void __launch_bounds__(256)
rms_norm_kernel(const void* __restrict__ x, const float* __restrict__ weight,
                void* __restrict__ out, int64_t T, int d, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  constexpr int ES = BF16 ? 2 : 4;   // bytes per element
  const char* row = (const char*)x + t * (int64_t)d * ES;
  char* orow = (char*)out + t * (int64_t)d * ES;
  float ss = 0.0f;
  if constexpr (VEC) {
    constexpr int VPC = BF16 ? 2 : 4;  // 16-byte vectors per 16-column chunk
    const int nch = d / 16;
    uint4 keep[RMS_KEEP][VPC];
#pragma unroll
    for (int i = 0; i < RMS_KEEP; ++i) {
      const int c = lane + i * 64;
#pragma unroll
      for (int v = 0; v < VPC; ++v) keep[i][v] = c < nch ? ldg16(row + c * 16 * ES + v * 16) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < RMS_KEEP; ++i) {
      float f[16];
      rms_unpack<BF16>(keep[i], f);
      ss = rms_chunk_sumsq(ss, f);
    }
    for (int c = lane + RMS_KEEP * 64; c < nch; c += 64) {
      uint4 v[VPC];
#pragma unroll
      for (int j = 0; j < VPC; ++j) v[j] = ldg16(row + c * 16 * ES + j * 16);
      float f[16];
      rms_unpack<BF16>(v, f);
      ss = rms_chunk_sumsq(ss, f);
    }
    ss = wave_sum(ss);
    const float r = 1.0f / __fsqrt_rn(ss / (float)d + eps);
#pragma unroll
    for (int i = 0; i < RMS_KEEP; ++i) {
      const int c = lane + i * 64;
      if (c < nch) {
        float f[16];
        rms_unpack<BF16>(keep[i], f);
        rms_scale_store<BF16>(f, r, weight, c * 16, orow + c * 16 * ES);
      }
    }
    for (int c = lane + RMS_KEEP * 64; c < nch; c += 64) {
      uint4 v[VPC];
#pragma unroll
      for (int j = 0; j < VPC; ++j) v[j] = ldg16(row + c * 16 * ES + j * 16);
      float f[16];
      rms_unpack<BF16>(v, f);
      rms_scale_store<BF16>(f, r, weight, c * 16, orow + c * 16 * ES);
    }
  } else {
    for (int c = lane; c < d; c += 64) {
      const float f = BF16 ? bf2f(((const uint16_t*)row)[c]) : ((const float*)row)[c];
      ss = ss + f * f;
    }
    ss = wave_sum(ss);
    const float r = 1.0f / __fsqrt_rn(ss / (float)d + eps);
    for (int c = lane; c < d; c += 64) {
      float f = BF16 ? bf2f(((const uint16_t*)row)[c]) : ((const float*)row)[c];
      f = f * r;
      if (weight) f = f * weight[c];
      if constexpr (BF16) ((uint16_t*)orow)[c] = (uint16_t)f2bf(f);
      else ((float*)orow)[c] = f;
    }
  }
}

// Combine followed by RMSNorm of each output row (Block's norm of the MoE
// output, model.py:636, 124-139), one wave per token: lane l owns the
// 16-column chunks l, l+64, ... (NCH of them, d <= NCH*1024).  Each chunk is
// combined exactly as combine_kernel does (ascending expert order, fp32 sum
// from +0 of rounded products), written to out, and its rounded values enter
// the row sum of squares in rms_norm_kernel's order; then norm_out = cast((v *
// r) * weight).  Chunks are combined one after another, every slot row load of
// a chunk in flight together.
template <bool BF16, int NCH>
struct CombineNormRow {
  static_assert(NCH >= 1 && NCH <= RMS_KEEP, "chunks per lane");
  static constexpr int ES = BF16 ? 2 : 4;
  static constexpr int VPC = BF16 ? 2 : 4;
  float v[NCH][16];  // the combined row as stored in out (rounded to the dtype)
  float r;           // 1 / rms
  int rw[8];         // the token's yperm rows (combine_slots order) and weights
  float wt[8];
  int n;
  float wv[NCH][16];  // the norm weight of the lane's columns (load_weight)
  bool hasw;
  // PACK (bf16, one chunk per lane): the lane's out and norm_out values, two
  // per word (combine() and norm()), so that to_lds() and store() only move
  // them.  Wider rows convert in to_lds() / store() (held packed beside the
  // row and the weight, they would not fit the registers of 16 waves).
  static constexpr bool PACK = BF16 && NCH == 1;
  uint32_t po[PACK ? NCH : 1][8], pn[PACK ? NCH : 1][8];

  // the norm weight of the lane's columns into registers (read once, before
  // to_lds / store; weight may be null)
  __device__ __forceinline__ void load_weight(const float* weight, int d, int lane) {
    hasw = weight != nullptr;
    if (!hasw) return;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = lane + i * 64;
      if (c < d / 16) {
#pragma unroll
        for (int q = 0; q < 16; ++q) wv[i][q] = ldgf(weight + c * 16 + q);
      }
    }
  }

  // the combine of the chunks and the row's 1/rms; no store.  COH: yperm
  // (ybytes long) was written by other workgroups of the running launch and
  // is read device-coherently.
  template <bool COH = false>
  __device__ __forceinline__ void compute(const void* yperm, const int64_t* topi, const float* topw,
                                          const int32_t* inv, float eps, int64_t t, int d, int k, int lane,
                                          int64_t ybytes = 0) {
    slots(topi, topw, inv, t, k);
    combine<COH>(yperm, eps, d, lane, ybytes);
  }
  // the slot loads alone (they do not depend on yperm)
  __device__ __forceinline__ void slots(const int64_t* topi, const float* topw, const int32_t* inv, int64_t t,
                                        int k) {
    n = combine_slots(topi, topw, inv, t, k, rw, wt);
  }
  // the combine of the slots loaded by slots(), and (SS) the row's 1/rms
  template <bool COH = false, bool SS = true>
  __device__ __forceinline__ void combine(const void* yperm, float eps, int d, int lane, int64_t ybytes = 0) {
    const int nch = d / 16;
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = lane + i * 64;
#pragma unroll
      for (int q = 0; q < 16; ++q) v[i][q] = 0.0f;
      if (c < nch) {
        uint4 yv[8][VPC];
#pragma unroll
        for (int s = 0; s < 8; ++s)
          if (s < n) {
            const int64_t off = ((int64_t)rw[s] * d + c * 16) * ES;
            if constexpr (COH) {
              const __amdgpu_buffer_rsrc_t yr = coh_rsrc(yperm, ybytes);
#pragma unroll
              for (int j = 0; j < VPC; ++j) yv[s][j] = coh_load16(yr, (uint32_t)(off + j * 16));
            } else {
              const char* src = (const char*)yperm + off;
#pragma unroll
              for (int j = 0; j < VPC; ++j) yv[s][j] = ldg16(src + j * 16);
            }
          }
#pragma unroll
        for (int s = 0; s < 8; ++s)
          if (s < n) {
            float y[16];
            rms_unpack<BF16>(yv[s], y);
#pragma unroll
            for (int q = 0; q < 16; ++q) {
              const float pr = y[q] * wt[s];  // rounded product (library built with -ffp-contract=off)
              v[i][q] = v[i][q] + pr;
            }
          }
        if constexpr (PACK) {
#pragma unroll
          for (int q = 0; q < 16; q += 2) {
            const uint32_t b0 = f2bf(v[i][q]), b1 = f2bf(v[i][q + 1]);
            po[i][q / 2] = b0 | (b1 << 16);
            v[i][q] = bf2f(b0);
            v[i][q + 1] = bf2f(b1);
          }
        } else if constexpr (BF16) {
#pragma unroll
          for (int q = 0; q < 16; ++q) v[i][q] = bf2f(f2bf(v[i][q]));
        }
      }
      if constexpr (SS) ss = rms_chunk_sumsq(ss, v[i]);
    }
    if constexpr (SS) {
      // rms_norm_kernel also adds RMS_KEEP - NCH all-zero chunks here: +0 changes nothing
      ss = wave_sum(ss);
      r = 1.0f / __fsqrt_rn(ss / (float)d + eps);
    }
  }

  // PACK: the normalised row, (v * r) * weight rounded to bf16, into pn;
  // after combine() and load_weight() (else a no-op)
  __device__ __forceinline__ void norm(int d, int lane) {
    if constexpr (!PACK) return;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = lane + i * 64;
      if (c < d / 16) {
        float o[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) o[q] = v[i][q] * r;
        if (hasw) {
#pragma unroll
          for (int q = 0; q < 16; ++q) o[q] = o[q] * wv[i][q];
        }
#pragma unroll
        for (int q = 0; q < 16; q += 2) pn[i][q / 2] = f2bf(o[q]) | (f2bf(o[q + 1]) << 16);
      }
    }
  }

  // the normalised row to LDS only (lds_row: d values of the dtype); after
  // norm()
  __device__ __forceinline__ void to_lds(int d, int lane, char* lds_row) const {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = lane + i * 64;
      if (c < d / 16) {
        if constexpr (PACK) {
          uint4* dst = (uint4*)(lds_row + c * 16 * ES);
          dst[0] = make_uint4(pn[i][0], pn[i][1], pn[i][2], pn[i][3]);
          dst[1] = make_uint4(pn[i][4], pn[i][5], pn[i][6], pn[i][7]);
        } else {
          rms_scale_store_w<BF16>(v[i], r, wv[i], hasw, nullptr, lds_row + c * 16 * ES);
        }
      }
    }
  }

  // out of token t alone (PACK); after combine()
  __device__ __forceinline__ void store_out(void* out, int64_t t, int d, int lane) const {
    static_assert(PACK, "bf16 rows of one chunk per lane");
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = lane + i * 64;
      if (c < d / 16) {
        uint4* dst = (uint4*)((char*)out + (t * d + c * 16) * ES);
        dst[0] = make_uint4(po[i][0], po[i][1], po[i][2], po[i][3]);
        dst[1] = make_uint4(po[i][4], po[i][5], po[i][6], po[i][7]);
      }
    }
  }

  // out and norm_out of token t; after norm()
  __device__ __forceinline__ void store(void* out, void* norm_out, int64_t t, int d, int lane) const {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = lane + i * 64;
      if (c < d / 16) {
        char* dst = (char*)out + (t * d + c * 16) * ES;
        if constexpr (PACK) {
          uint4* no = (uint4*)((char*)norm_out + (t * d + c * 16) * ES);
          no[0] = make_uint4(pn[i][0], pn[i][1], pn[i][2], pn[i][3]);
          no[1] = make_uint4(pn[i][4], pn[i][5], pn[i][6], pn[i][7]);
          ((uint4*)dst)[0] = make_uint4(po[i][0], po[i][1], po[i][2], po[i][3]);
          ((uint4*)dst)[1] = make_uint4(po[i][4], po[i][5], po[i][6], po[i][7]);
        } else if constexpr (BF16) {
          rms_scale_store_w<BF16>(v[i], r, wv[i], hasw, (char*)norm_out + (t * d + c * 16) * ES);
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            uint4 w;
            w.x = f2bf(v[i][j * 8 + 0]) | (f2bf(v[i][j * 8 + 1]) << 16);
            w.y = f2bf(v[i][j * 8 + 2]) | (f2bf(v[i][j * 8 + 3]) << 16);
            w.z = f2bf(v[i][j * 8 + 4]) | (f2bf(v[i][j * 8 + 5]) << 16);
            w.w = f2bf(v[i][j * 8 + 6]) | (f2bf(v[i][j * 8 + 7]) << 16);
            ((uint4*)dst)[j] = w;
          }
        } else {
          rms_scale_store_w<BF16>(v[i], r, wv[i], hasw, (char*)norm_out + (t * d + c * 16) * ES);
#pragma unroll
          for (int j = 0; j < 4; ++j)
            ((float4*)dst)[j] = make_float4(v[i][j * 4], v[i][j * 4 + 1], v[i][j * 4 + 2], v[i][j * 4 + 3]);
        }
      }
    }
  }
};

// The same tail without a next router (a layer whose caller routes its output
// itself): the first ceil(T / 8) workgroups to arrive combine 8 tokens each,
// one wave per token, with CombineNormRow (the arithmetic of combine_kernel,
// and with NORM of combine_norm_kernel), reading y device-coherently.
template <bool NORM>
__device__ void cn_tail(const CnrArgs& cr, const void* y, int32_t* arr) {
  __shared__ int s_arrival;
  __builtin_amdgcn_s_waitcnt(0);  // this wave's output stores have completed
  __syncthreads();
  if (threadIdx.x == 0) s_arrival = (int)__hip_atomic_fetch_add(arr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  const int ncw = (int)((cr.T + CNR_TAIL_TOK - 1) / CNR_TAIL_TOK);
  const int a = s_arrival;
  if (a >= ncw) return;  // uniform: the first ncw to arrive combine
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)a * CNR_TAIL_TOK + (threadIdx.x >> 6);
  const bool mine = t < cr.T;  // uniform per wave
  CombineNormRow<true, 1> cn;
  if (mine) {
    cn.slots(cr.topi, cr.topw, cr.inv, t, cr.k);
    if (NORM) cn.load_weight(cr.weight, cr.d, lane);
  }
  if (!ds_wait_all(arr, (int)gridDim.x + cr.wait_extra, cr.spin_limit)) {  // uniform
    cnr_poison(cr, (int64_t)a * CNR_TAIL_TOK, false);
    return;
  }
  if (mine) {
    cn.template combine<true, NORM>(y, cr.eps, cr.d, lane, cr.ybytes);
    if constexpr (NORM) {
      cn.norm(cr.d, lane);
      cn.store(cr.out, cr.norm_out, t, cr.d, lane);
    } else {
      cn.store_out(cr.out, t, cr.d, lane);
    }
  }
}

template <bool BF16, int NCH>
__global__ void __launch_bounds__(256)
combine_norm_kernel(const void* __restrict__ yperm, const int64_t* __restrict__ topi,
                    const float* __restrict__ topw, const int32_t* __restrict__ inv,
                    void* __restrict__ out, const float* __restrict__ weight, float eps,
                    void* __restrict__ norm_out, int64_t T, int d, int k) {
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  CombineNormRow<BF16, NCH> cn;
  cn.compute(yperm, topi, topw, inv, eps, t, d, k, threadIdx.x & 63);
  cn.load_weight(weight, d, threadIdx.x & 63);
  cn.norm(d, threadIdx.x & 63);
  cn.store(out, norm_out, t, d, threadIdx.x & 63);
}

// The combine and output norm of 16 tokens (one wave each, combine_norm_row)
// followed by the next layer's router on the normed rows: the logits, softmax
// and top-k of router_mfma_kernel for these 16 tokens (RouteSlice over the
// same K slices, route_reduce, route_select_group), so the per-token
// arithmetic, and the bits, are those of routing norm_out in a kernel of its
// own.  The normed rows reach the router through LDS (a copy beside the
// norm_out stores) and the bias stays in a register.  Writes the next layer's
// prob/topi/topw (no counts: the next gate/up kernel or dispatch builds its
// dispatch from the top-k).
constexpr int CNR_TOK = 16;
constexpr int CNR_DMAX = 2048;  // the MFMA router's widest d

// Workgroup barrier for LDS data only: waits for this wave's LDS accesses,
// not for its global stores (__syncthreads waits for those too).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
// The combine + norm + next router of the TOK tokens from t0, by the calling
// workgroup's TOK waves (wave w: token t0 + w; waves < RK_SLICES also run the
// router's K slices), in three phases: prefetch_slots (the top-k, weights and
// yperm rows of each token, and the norm weight), prefetch_router (the router
// weights and bias of the K-slice waves) and finish (the rest).  The loads of
// the first two do not depend on yperm, so a caller that waits for yperm can
// issue them before it waits, and also split the router weights into their
// bf16 terms meanwhile (prepare_router).  COH: yperm (ybytes long) was written by other workgroups of the
// running launch and is read device-coherently.
template <int NCH, int EMAX, bool EXACT, int KSW, int TOK, bool COH>
struct CnrBlock {
  static_assert(EMAX <= 16, "the MFMA router covers up to 16 experts");
  static constexpr int NWAVES = TOK;
  // RouteSlice's partial logits: one 16-token MFMA tile per K slice, whatever
  // TOK (<= 16) is
  static constexpr int RT = RouteSlice<KSW, 1>::TOK;
  static_assert(TOK <= RT, "one MFMA token tile");
  static_assert(NWAVES >= RK_SLICES, "one K slice per router wave");
  static_assert(TOK * EMAX <= RK_SLICES * 64, "the bias-adding threads are router-wave threads");
  // (At KSW = 8 the row held through the routing would spill: stored first.)
  static constexpr bool LATE_STORE = KSW == 4;

  CombineNormRow<true, NCH> cn;
  RouteSlice<KSW, 1> rs;
  float bias = 0.0f;
  bool routed = false;  // router weights and bias loaded
  bool split = false;   // router weights split into bf16 terms

  __device__ __forceinline__ static int nvalid_of(int64_t T, int64_t t0) { return (int)min<int64_t>(TOK, T - t0); }

  __device__ __forceinline__ void prefetch_slots(const int64_t* topi, const float* topw, const int32_t* inv,
                                                 const float* weight, int64_t T, int d, int k, int64_t t0) {
    const int wave = threadIdx.x >> 6;
    if (wave < nvalid_of(T, t0)) {  // uniform per wave
      cn.slots(topi, topw, inv, t0 + wave, k);
      // the norm weight too where the row is held through the routing (with
      // it live from here, the wider rows of KSW = 8 would spill)
      if (LATE_STORE) cn.load_weight(weight, d, threadIdx.x & 63);
    }
  }
  __device__ __forceinline__ void prefetch_router(const float* ngw, const float* ngb, int nE, int d) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int E = EXACT ? EMAX : nE;
    const int re = (int)(threadIdx.x % EMAX);
    if (wave < RK_SLICES) {  // uniform per wave
      rs.load_w(ngw, E, d, wave, lane);
      if (threadIdx.x < (unsigned)(TOK * EMAX) && re < E && ngb) bias = ngb[re];
    }
    routed = true;
  }
  // the split of the router weights into bf16 terms (waits for their loads),
  // for a caller that has time to spare before the combine
  __device__ __forceinline__ void prepare_router(int nE, int d) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (wave < RK_SLICES) rs.split(EXACT ? EMAX : nE, d, lane);  // uniform per wave
    split = true;
  }

  __device__ __forceinline__ void finish(const void* __restrict__ yperm, int64_t ybytes, void* __restrict__ out,
                                         const float* __restrict__ weight, float eps, void* norm_out, int64_t T,
                                         int d, const float* __restrict__ ngw, const float* __restrict__ ngb,
                                         RouteOut no, int nE, int nk, int64_t t0) {
    __shared__ __attribute__((aligned(16))) float part[RK_SLICES * RT * 16];
    __shared__ float slog[TOK][EMAX];
    __shared__ smaul_topk::Pair spair[TOK][EMAX];
    __shared__ int s_ti[TOK][8];
    __shared__ float s_tw[TOK][8];
    __shared__ __attribute__((aligned(16))) uint16_t sx[TOK * CNR_DMAX];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int E = EXACT ? EMAX : nE;
    const int nvalid = nvalid_of(T, t0);
    // The combine and norm first, the normed row to LDS only.  Unless
    // prefetched, the router weights and bias are loaded after the barrier: a
    // CU returns reads in issue order, so cold weights issued before the
    // combine's slot reads would hold those up.  The global stores of out /
    // norm_out go out after the routing MFMAs, so that the wait for the
    // weights does not also wait for them.
    const bool mine = wave < nvalid;  // uniform per wave
    if (mine) {
      cn.template combine<COH>(yperm, eps, d, lane, ybytes);
      if (!LATE_STORE) cn.load_weight(weight, d, lane);
      cn.norm(d, lane);
      cn.to_lds(d, lane, (char*)(sx + wave * d));
      if (!LATE_STORE) cn.store(out, norm_out, t0 + wave, d, lane);
    }
    lds_barrier();
    // route_reduce's thread q = tok * EMAX + e adds bias[e]
    const int re = (int)(threadIdx.x % EMAX);
    if (!routed) prefetch_router(ngw, ngb, nE, d);
    if (wave < RK_SLICES) {  // uniform per wave
      rs.load_x_lds(sx, d, nvalid, lane);
      if (split) rs.template compute<true>(E, d, lane, part);
      else rs.compute(E, d, lane, part);
    }
    if (LATE_STORE && mine) cn.store(out, norm_out, t0 + wave, d, lane);
    lds_barrier();
    // route_reduce with the bias from a register (the same sums, in slice order)
    if (threadIdx.x < (unsigned)(TOK * EMAX)) {
      const int tok = (int)threadIdx.x / EMAX;
      if (re < E && t0 + tok < T) {
        float v = part[tok * 16 + re];
#pragma unroll
        for (int sl = 1; sl < RK_SLICES; ++sl) v += part[(sl * RT + tok) * 16 + re];
        slog[tok][re] = ngb ? v + bias : v;
      }
    }
    lds_barrier();
    constexpr int TPW = 64 / EMAX;
    for (int tl = wave * TPW + (lane / EMAX); tl < TOK; tl += NWAVES * TPW) {
      const int64_t t = t0 + tl;
      route_select_group<EMAX>(slog[tl], spair[tl], E, nk, t, t < T, no, true, s_ti[tl], s_tw[tl], nullptr);
    }
  }
};

template <int NCH, int EMAX, bool EXACT, int KSW>
__global__ void __launch_bounds__(CNR_TOK * 64)
combine_norm_route_kernel(const void* __restrict__ yperm, const int64_t* __restrict__ topi,
                          const float* __restrict__ topw, const int32_t* __restrict__ inv, void* __restrict__ out,
                          const float* __restrict__ weight, float eps, void* norm_out, int64_t T, int d, int k,
                          const float* __restrict__ ngw, const float* __restrict__ ngb, RouteOut no, int nE,
                          int nk) {
  const int64_t t0 = (int64_t)blockIdx.x * CNR_TOK;
  CnrBlock<NCH, EMAX, EXACT, KSW, CNR_TOK, false> b;
  b.prefetch_slots(topi, topw, inv, weight, T, d, k, t0);
  b.finish(yperm, 0, out, weight, eps, norm_out, T, d, ngw, ngb, no, nE, nk, t0);
}

// ---------------------------------------------------------------------------
// code canonicalisation (device repack cache): 0x7F -> 0x7E, 0xFF -> 0xFE
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
canonicalize_kernel(const uint8_t* __restrict__ in, uint8_t* __restrict__ out, int64_t n) {
  const int64_t nv = n / 16;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nv; i += stride) {
    uint4 v = ((const uint4*)in)[i];
    v.x = canon4(v.x);
    v.y = canon4(v.y);
    v.z = canon4(v.z);
    v.w = canon4(v.w);
    ((uint4*)out)[i] = v;
  }
  if (blockIdx.x == 0 && threadIdx.x < (n & 15)) {
    const int64_t j = nv * 16 + threadIdx.x;
    const uint8_t c = in[j];
    out[j] = ((c & 0x7f) == 0x7f) ? (uint8_t)(c - 1) : c;
  }
}

// The tiled layout (WLayout): canonical codes out[(kb * N + n) * 64 + j] =
// in[n * K + kb * 64 + j], one thread per 16 bytes of out, and fp32 scales
// sout[kb * N + n] = sin[n * nb + kb], nb = K / 64.
__global__ void __launch_bounds__(256)
tile_codes_kernel(const uint8_t* __restrict__ in, uint8_t* __restrict__ out, int64_t N, int64_t K) {
  const int64_t nv = N * K / 16;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nv; i += stride) {
    const int64_t o = i * 16;
    const int64_t kb = o / (N * 64);
    const int64_t n = (o / 64) % N;
    const int64_t j = o % 64;
    uint4 v = *(const uint4*)(in + n * K + kb * 64 + j);
    v.x = canon4(v.x);
    v.y = canon4(v.y);
    v.z = canon4(v.z);
    v.w = canon4(v.w);
    *(uint4*)(out + o) = v;
  }
}

__global__ void __launch_bounds__(256)
tile_scales_kernel(const float* __restrict__ in, float* __restrict__ out, int64_t N, int64_t nb) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < N * nb; i += stride) {
    const int64_t kb = i / N, n = i - kb * N;
    out[i] = in[n * nb + kb];
  }
}

// ---------------------------------------------------------------------------
// host helpers
// ---------------------------------------------------------------------------
bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
bool dtype_ok(int dt) { return dt == SMAUL_DTYPE_F32 || dt == SMAUL_DTYPE_BF16; }

// block_m 16 selects the decode-regime kernels (at most 64 rows per expert:
// every token appears at most once per expert, so T <= 64 guarantees it).
constexpr int DECODE_BM = 16;
// block_m 64: the LDS-DMA kernels on 64-row tiles, for a layer whose 128-row
// gate/up grid is under four workgroups per CU (chosen inside
// smaul_moe_forward only, where the code-alignment flag is known; every
// output is the same sum in the same order as on 128-row tiles).  Measured
// (d 1024, h 2560, E 8, top-2): T 768 80.4 -> 67.7 us, T 2048 122.1 -> 110.5
// us; at 1440 and 5280 workgroups (T 4096, 16384) 64-row tiles lose 1-6 %.
constexpr int DMA_SMALL_BM = 64;

bool decode_shape_ok(int64_t d, int64_t h, int64_t tile) { return tile == 64 && d % 128 == 0 && h % 128 == 0; }


int pick_block_m(int64_t T, int64_t d, int64_t h, int64_t E, int64_t k, int64_t tile, int act_dtype) {
  if (T <= 64 && act_dtype == SMAUL_DTYPE_BF16 && decode_shape_ok(d, h, tile)) return DECODE_BM;
  // rows per expert on average; small segments use the 32-row tile
  const int64_t avg = (T * k + E - 1) / (E > 0 ? E : 1);
  if (avg < 96) return CfgSmall::BM;
  // 128-row tiles: the LDS-DMA kernels where they apply (moe_gemm decides),
  // else the register-staged ones
  return act_dtype == SMAUL_DTYPE_BF16 ? CfgBig::BM : CfgBigF32::BM;
}

template <class CF, class CF32, bool CANON>
int gemm_dispatch_moe_c(const GemmArgs& a, bool swiglu, int act_dtype, int64_t m_tiles, hipStream_t s) {
  if (swiglu) {
    if (act_dtype == SMAUL_DTYPE_BF16) return launch_gemm<CF, true, 1, true, CANON, true>(a, m_tiles, s);
    return launch_gemm<CF32, true, 2, false, CANON, true>(a, m_tiles, s);
  }
  if (act_dtype == SMAUL_DTYPE_BF16) return launch_gemm<CF, false, 1, true, CANON, true>(a, m_tiles, s);
  return launch_gemm<CF32, false, 2, false, CANON, true>(a, m_tiles, s);
}

template <class CF, class CF32>
int gemm_dispatch_moe(const GemmArgs& a, bool swiglu, int act_dtype, int64_t m_tiles, bool canon,
                      hipStream_t s) {
  return canon ? gemm_dispatch_moe_c<CF, CF32, true>(a, swiglu, act_dtype, m_tiles, s)
               : gemm_dispatch_moe_c<CF, CF32, false>(a, swiglu, act_dtype, m_tiles, s);
}

template <class CF, int NSPLIT>
int gemm_dispatch_dense(const GemmArgs& a, bool vec, bool canon, int64_t m_tiles, hipStream_t s) {
  if (!vec) return launch_gemm<CF, false, NSPLIT, false, false, false>(a, m_tiles, s);
  return canon ? launch_gemm<CF, false, NSPLIT, false, true, true>(a, m_tiles, s)
               : launch_gemm<CF, false, NSPLIT, false, false, true>(a, m_tiles, s);
}

int64_t align256(int64_t v) { return (v + 255) & ~int64_t(255); }

// LDS-DMA grouped GEMM shapes: (BM rows, BN staged weight columns, wave
// grid, pipeline depth).  8 waves (2 per SIMD) and a 3-deep pipeline use
// 147 KB of LDS: one workgroup per CU.
// 128-row tiles of 4 waves (each 128 rows x 64 staged columns) with two
// stage buffers: 68 KB of LDS, so two workgroups share a CU and one's
// prologue and epilogue overlap the other's main loop.
struct CfgDmaGU {  // gate+up with the SwiGLU epilogue: 128 rows x 128 outputs
  static constexpr int BM = 128, BN = 256, WM = 1, WN = 4, NSTAGE = 2;
};
struct CfgDmaDown {  // down projection: 128 rows x 256 outputs
  static constexpr int BM = 128, BN = 256, WM = 1, WN = 4, NSTAGE = 2;
};
// Down projection with few tiles (under four rounds of two per CU): 128 rows
// x 128 outputs, 49 KB of LDS, three workgroups per CU, so the last partial
// round is of smaller tiles and each CU hides one workgroup's DMA waits with
// two others.  Measured: C3 down 189.5 vs 197.1 us; at C5 (sixteen rounds)
// the wide tile stays faster (2.47 vs 2.58 ms).
struct CfgDmaDownN {
  static constexpr int BM = 128, BN = 128, WM = 1, WN = 4, NSTAGE = 2;
};
// Smaller tiles for dense GEMMs whose 128x256 grid would leave most of the
// 512 workgroup slots (two per CU) empty: every workgroup of such a grid runs
// in the first round, so the launch takes one tile's whole latency, and a
// smaller tile shortens it.  Deeper pipelines cover the DMA latency that the
// second workgroup of a CU no longer hides.
struct CfgDmaGU64 {  // 64 rows x 128 outputs (gate+up), 4 waves of 64 rows x 32 outputs
  static constexpr int BM = 64, BN = 256, WM = 1, WN = 4, NSTAGE = 2;
};
struct CfgDma64x128 {  // 64 rows x 128 outputs
  static constexpr int BM = 64, BN = 128, WM = 1, WN = 4, NSTAGE = 3;
};
struct CfgDma32x128 {  // 32 rows x 128 outputs
  static constexpr int BM = 32, BN = 128, WM = 1, WN = 4, NSTAGE = 4;
};

template <class CF, bool SWIGLU, bool CANON, bool OUT_F32 = false, bool X32 = false>
int launch_gemm_dma(const GemmArgs& a, int64_t m_tiles, hipStream_t stream) {
  constexpr int BNO = SWIGLU ? CF::BN / 2 : CF::BN;
  const int64_t n_tiles = (a.N + BNO - 1) / BNO;
  if (m_tiles <= 0 || n_tiles <= 0) return SMAUL_OK;
  if (m_tiles > 65535 || n_tiles > 65535) return fail(SMAUL_ERR_UNSUPPORTED, "gemm grid too large");
  hipLaunchKernelGGL(
      (fp8_gemm_dma_kernel<CF::BM, CF::BN, CF::WM, CF::WN, CF::NSTAGE, SWIGLU, CANON, true, OUT_F32, X32>),
      dim3((unsigned)n_tiles, (unsigned)m_tiles), dim3(CF::WM * CF::WN * 64), 0, stream, a);
  return check_launch("fp8_gemm_dma_kernel");
}

// The dense (one-segment) LDS-DMA GEMM with its tile chosen by grid size:
// the 128-row tile where its grid fills the workgroup slots (two per CU),
// else 64 x 128 (gate+up: 64 rows x 128 outputs, two stages, three
// workgroups per CU), or 32 x 128 where even that leaves CUs without a
// workgroup; -1 when N is not a multiple of 128.  Measured at config 2
// (kernel trace, 4096 rows): gate+up 22.0 -> 18.3 us, down (K 1280, N 512)
// 24.2 -> 11.7 us; 32 x 128 tiles there: 11.4 us; the gate+up tile of 64
// outputs on a 2 x 2 wave grid (three stages) 0.9 us slower than 128 outputs.
enum DenseTile { DT_128x256 = 0, DT_64x256_GU = 1, DT_64x128 = 2, DT_32x128 = 3 };
int pick_dense_tile(bool swiglu, int64_t rows, int64_t N) {
  if (N % 128 != 0) return -1;
  const int64_t cus = cu_count();
  auto tiles = [&](int64_t bm, int64_t bno) { return ((rows + bm - 1) / bm) * (N / bno); };
  if (swiglu) return tiles(128, 128) >= 2 * cus ? DT_128x256 : DT_64x256_GU;
  if (N % 256 == 0 && tiles(128, 256) >= 2 * cus) return DT_128x256;
  return tiles(64, 128) >= cus ? DT_64x128 : DT_32x128;
}

template <bool SWIGLU, bool CANON, bool OUT_F32, bool X32 = false>
int launch_dense_dma(const GemmArgs& a, int tile, hipStream_t stream) {
  const int64_t rows = a.R;
  switch (tile) {
    case DT_128x256:
      return launch_gemm_dma<CfgDmaGU, SWIGLU, CANON, OUT_F32, X32>(a, (rows + 127) / 128, stream);
    case DT_64x256_GU:
      if constexpr (SWIGLU) return launch_gemm_dma<CfgDmaGU64, SWIGLU, CANON, OUT_F32>(a, (rows + 63) / 64, stream);
      break;
    case DT_64x128:
      if constexpr (!SWIGLU)
        return launch_gemm_dma<CfgDma64x128, SWIGLU, CANON, OUT_F32, X32>(a, (rows + 63) / 64, stream);
      break;
    case DT_32x128:
      if constexpr (!SWIGLU)
        return launch_gemm_dma<CfgDma32x128, SWIGLU, CANON, OUT_F32, X32>(a, (rows + 31) / 32, stream);
      break;
    default:
      break;
  }
  return fail(SMAUL_ERR_INVALID, "dense gemm: no tile for this shape");
}

// The LDS-DMA kernel needs bf16 activations, 64-wide scale tiles, K a
// multiple of 64, N a multiple of the workgroup's output columns, 16-byte
// aligned code rows and activation rows, 8-byte aligned output row pieces (its
// epilogue stores four bf16 columns at a time), and byte offsets that fit its
// 32-bit per-lane offsets.
// The fp32-activation form (X32): the same shapes, fp32 rows 16-byte aligned,
// byte offsets of 4-byte elements within 32 bits.
bool x32_gemm_ok(const GemmArgs& a, int64_t x_rows) {
  if (a.tile != 64 || (a.K & 63) != 0 || a.N % 128 != 0 || !aligned16(a.x) || (a.ldx & 3) != 0) return false;
  if (((uintptr_t)a.y & 7u) != 0 || (a.ldy & 3) != 0) return false;
  const int64_t lim = (int64_t)1 << 31;
  return x_rows * a.ldx * 4 < lim && a.N * a.K < lim && a.N * a.nt < lim;
}

bool dma_gemm_ok(const GemmArgs& a, int act_dtype, int flags, int64_t x_rows, int64_t bno) {
  if (act_dtype != SMAUL_DTYPE_BF16 || a.tile != 64 || (a.K & 63) != 0 || a.N % bno != 0) return false;
  if (!(flags & SMAUL_FLAG_ALIGNED_CODES) || !aligned16(a.x) || (a.ldx & 7) != 0) return false;
  if (((uintptr_t)a.y & 7u) != 0 || (a.ldy & 3) != 0) return false;
  const int64_t lim = (int64_t)1 << 31;
  return x_rows * a.ldx * 2 < lim && a.N * a.K < lim && a.N * a.nt < lim;
}

}  // namespace

// ---------------------------------------------------------------------------
// Static scratch for smaul_moe_forward_noalloc: a fixed device array per GPU,
// held from the library's first call on that GPU until the process ends.  In
// host code `scratch` names a host-side stand-in, never the device memory:
// the device address comes from hipGetSymbolAddress, once per device, with
// that device current, and only that address is handed to kernels.
// ---------------------------------------------------------------------------
static __device__ __align__(256) char scratch[SMAUL_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's scratch address (looked up on the first call per device).
int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(SMAUL_ERR_HIP, "noalloc: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(SMAUL_ERR_UNSUPPORTED, "noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(SMAUL_ERR_HIP, "noalloc: hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SMAUL_OK;
}
}  // namespace

// ===========================================================================
// C ABI
// ===========================================================================
extern "C" {

int smaul_version(void) { return SMAUL_VERSION; }

const char* smaul_last_error(void) { return smaul::g_err; }

int smaul_fp8_linear(const void* x, int x_dtype, const uint8_t* w, const float* s, void* y,
                     int y_dtype, int64_t rows, int64_t in_f, int64_t out_f, int64_t tile, int flags,
                     hipStream_t stream) {
  if (tile <= 0 || in_f <= 0 || out_f <= 0 || rows < 0)
    return fail(SMAUL_ERR_INVALID, "tile/in_f/out_f must be positive, got %lld/%lld/%lld",
                (long long)tile, (long long)in_f, (long long)out_f);
  if (!dtype_ok(x_dtype) || y_dtype != SMAUL_DTYPE_F32)
    return fail(SMAUL_ERR_INVALID, "x dtype must be f32|bf16 and y dtype f32");
  if (flags & SMAUL_FLAG_TILED_LAYOUT)
    return fail(SMAUL_ERR_INVALID, "fp8_linear: codes and scales must be in the reference layout");
  if (kmode_of(tile) < 0)
    return fail(SMAUL_ERR_UNSUPPORTED, "tile %lld: need 32 or a multiple of 64", (long long)tile);
  if (rows == 0) return SMAUL_OK;
  if (!x || !w || !s || !y) return fail(SMAUL_ERR_INVALID, "null pointer");
  GemmArgs a{};
  a.x = x;
  a.row_idx = nullptr;
  a.ldx = in_f;
  a.w = w;
  a.s = s;
  a.w_estride = 0;
  a.s_estride = 0;
  a.y = y;
  a.ldy = out_f;
  a.K = in_f;
  a.N = out_f;
  a.nt = (in_f + tile - 1) / tile;
  a.tile = tile;
  a.seg_off = nullptr;
  a.tile_off = nullptr;
  a.R = rows;
  a.E = 1;
  const bool vec = (in_f % 16 == 0) && aligned16(x) && aligned16(w);
  const bool canon = (flags & SMAUL_FLAG_CANONICAL_CODES) != 0;
  const bool small = rows <= 64;
  // bf16 x, 64-wide tiles and 16-byte aligned code rows: the LDS-DMA kernel
  // with its tile sized to the grid, fp32 sums stored as they are
  const int dt = small ? -1 : pick_dense_tile(false, rows, out_f);
  if (dt >= 0 && vec && dma_gemm_ok(a, x_dtype, flags | SMAUL_FLAG_ALIGNED_CODES, rows, 128))
    return canon ? launch_dense_dma<false, true, true>(a, dt, stream) : launch_dense_dma<false, false, true>(a, dt, stream);
  // fp32 x, 64-wide tiles: the same kernel staging fp32 rows and splitting
  // them into bf16 hi / lo planes in LDS (X32)
  if (dt >= 0 && vec && x_dtype == SMAUL_DTYPE_F32 && x32_gemm_ok(a, rows))
    return canon ? launch_dense_dma<false, true, true, true>(a, dt, stream)
                 : launch_dense_dma<false, false, true, true>(a, dt, stream);
  if (x_dtype == SMAUL_DTYPE_BF16) {
    const int64_t bm = small ? CfgSmall::BM : CfgBig::BM;
    const int64_t mt = (rows + bm - 1) / bm;
    return small ? gemm_dispatch_dense<CfgSmall, 1>(a, vec, canon, mt, stream)
                 : gemm_dispatch_dense<CfgBig, 1>(a, vec, canon, mt, stream);
  }
  const int64_t bm = small ? CfgSmall::BM : CfgBigF32::BM;
  const int64_t mt = (rows + bm - 1) / bm;
  return small ? gemm_dispatch_dense<CfgSmall, 2>(a, vec, canon, mt, stream)
               : gemm_dispatch_dense<CfgBigF32, 2>(a, vec, canon, mt, stream);
}

namespace {

// fp32 activations -> two bf16 planes side by side (split_bf16): out row r
// holds hi(x[r, :]) in columns [0, K) and lo(x[r, :]) in [K, 2K).  One thread
// per 8 consecutive values: two 16-byte loads, one 16-byte store per plane.
__global__ void __launch_bounds__(256) split_planes_kernel(const float* __restrict__ x, uint16_t* __restrict__ out,
                                                           int64_t rows, int64_t K) {
  const int64_t per_row = K >> 3;
  const int64_t n = rows * per_row;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / per_row, c = (i - r * per_row) * 8;
    const float4 v0 = *(const float4*)(x + r * K + c);
    const float4 v1 = *(const float4*)(x + r * K + c + 4);
    const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    uint32_t h[8], l[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) split_bf16(v[q], h[q], l[q]);
    uint16_t* o = out + r * 2 * K + c;
    *(uint4*)o = make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
    *(uint4*)(o + K) = make_uint4(l[0] | (l[1] << 16), l[2] | (l[3] << 16), l[4] | (l[5] << 16), l[6] | (l[7] << 16));
  }
}

// x [rows, K] fp32 (K % 8 == 0, 16-byte aligned) -> planes [rows, 2K] bf16
int launch_split_planes(const float* x, uint16_t* planes, int64_t rows, int64_t K, hipStream_t stream) {
  const int64_t n8 = rows * (K / 8);
  const int64_t blocks = std::min<int64_t>((n8 + 255) / 256, 4096);
  hipLaunchKernelGGL(split_planes_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, x, planes, rows, K);
  return check_launch("split_planes_kernel");
}

// The two-plane LDS-DMA path of smaul_fp8_linear_ws applies (fp32 x, tile
// 64, shapes the DMA GEMM takes): the dense tile, else -1.
int planes_tile(int x_dtype, const void* x, const uint8_t* w, int64_t rows, int64_t in_f, int64_t out_f,
                int64_t tile, int flags) {
  if (x_dtype != SMAUL_DTYPE_F32 || tile != 64 || rows <= 64 || in_f % 64 != 0) return -1;
  if ((flags & SMAUL_FLAG_TILED_LAYOUT) || !aligned16(x) || !aligned16(w) || in_f % 16 != 0) return -1;
  return pick_dense_tile(false, rows, out_f);
}

}  // namespace

// Up to this many rows, fp32 x takes smaul_fp8_linear's in-LDS split (X32)
// rather than the planes pass: a separate launch costs more than it saves on
// short calls (C-ABI timings: 512 x 512 -> 1536 12.6 vs 16.4 us, 300 x 256 ->
// 384 8.5 vs 12.5 us; 4096 x 512 -> 1280 35.6 vs 32.7 us, 16384 x 1024 ->
// 2560 316 vs 259 us).
constexpr int64_t PLANES_MIN_ROWS = 1025;

int64_t smaul_fp8_linear_workspace_size(int64_t rows, int64_t in_f, int x_dtype) {
  if (rows < 0 || in_f < 0) return -1;
  return (x_dtype == SMAUL_DTYPE_F32 && rows >= PLANES_MIN_ROWS) ? rows * in_f * 4 : 0;
}

int smaul_fp8_linear_ws(const void* x, int x_dtype, const uint8_t* w, const float* s, void* y, int y_dtype,
                        int64_t rows, int64_t in_f, int64_t out_f, int64_t tile, int flags, void* workspace,
                        int64_t workspace_bytes, hipStream_t stream) {
  const int dt = (rows >= PLANES_MIN_ROWS && y && s && y_dtype == SMAUL_DTYPE_F32 && kmode_of(tile) >= 0)
                     ? planes_tile(x_dtype, x, w, rows, in_f, out_f, tile, flags)
                     : -1;
  if (dt < 0 || !workspace || !aligned16(workspace) ||
      workspace_bytes < smaul_fp8_linear_workspace_size(rows, in_f, x_dtype))
    return smaul_fp8_linear(x, x_dtype, w, s, y, y_dtype, rows, in_f, out_f, tile, flags, stream);
  GemmArgs a{};
  a.x = workspace;  // [rows][2 * in_f] bf16: hi plane, then lo plane
  a.row_idx = nullptr;
  a.ldx = 2 * in_f;
  a.w = w;
  a.s = s;
  a.y = y;
  a.ldy = out_f;
  a.K = 2 * in_f;
  a.kw = in_f;
  a.N = out_f;
  a.nt = in_f / 64;
  a.tile = 64;
  a.R = rows;
  a.E = 1;
  if (!dma_gemm_ok(a, SMAUL_DTYPE_BF16, flags | SMAUL_FLAG_ALIGNED_CODES, rows, 128))
    return smaul_fp8_linear(x, x_dtype, w, s, y, y_dtype, rows, in_f, out_f, tile, flags, stream);
  const int rc = launch_split_planes((const float*)x, (uint16_t*)workspace, rows, in_f, stream);
  if (rc != SMAUL_OK) return rc;
  const bool canon = (flags & SMAUL_FLAG_CANONICAL_CODES) != 0;
  return canon ? launch_dense_dma<false, true, true>(a, dt, stream) : launch_dense_dma<false, false, true>(a, dt, stream);
}

// router launch shape for E experts: (tokens per wave, expert register width)
// router tokens per wave for E experts (E <= 4, 8, 16, 64): TB * EMAX partial
// sums per lane
static constexpr int route_tb(int64_t E) { return E <= 4 ? 8 : E <= 16 ? 4 : 1; }
// tokens per router workgroup: bf16 activations run router_mfma_kernel
static bool route_mfma_ok(int64_t E, int64_t d, int x_dtype) {
  return x_dtype == SMAUL_DTYPE_BF16 && E <= 16 && route_ksw(d) != 0;
}
// Up to ROUTE_SMALL_T tokens the MFMA router takes 16 tokens per workgroup
// (more workgroups for a short call; the arithmetic per token is the same).
constexpr int64_t ROUTE_SMALL_T = 2048;
static int route_tpb(int64_t T, int64_t E, int64_t d, int x_dtype) {
  if (route_mfma_ok(E, d, x_dtype)) return T <= ROUTE_SMALL_T ? 16 : ROUTE_MFMA_TPB;
  return route_tb(E) * ROUTE_WAVES;
}

// The decode router (T <= 64, bf16, the MFMA router's shapes): one block per
// 16 tokens, top-k only (no dispatch).
static int launch_router_small(const void* x, const float* gate_w, const float* gate_b, const RouteOut& o,
                               int64_t T, int64_t d, int64_t E, int64_t k, hipStream_t stream) {
  const uint16_t* xb = (const uint16_t*)x;
  const dim3 grid((unsigned)((T + 15) / 16)), block(ROUTE_MFMA_THREADS);
  const int ksw = route_ksw(d);
#define SMAUL_ROUTE_S2(EMAX, EXACT)                                                                            \
  if (ksw == 4)                                                                                                \
    hipLaunchKernelGGL((router_mfma_kernel<EMAX, EXACT, 4, 1>), grid, block, 0, stream, xb, gate_w, gate_b, o, T, \
                       (int)d, (int)E, (int)k);                                                                \
  else                                                                                                         \
    hipLaunchKernelGGL((router_mfma_kernel<EMAX, EXACT, 8, 1>), grid, block, 0, stream, xb, gate_w, gate_b, o, T, \
                       (int)d, (int)E, (int)k);
#define SMAUL_ROUTE_S(EMAX)     \
  if (E == EMAX) {              \
    SMAUL_ROUTE_S2(EMAX, true)  \
  } else {                      \
    SMAUL_ROUTE_S2(EMAX, false) \
  }
  if (E <= 4) {
    SMAUL_ROUTE_S(4)
  } else if (E <= 8) {
    SMAUL_ROUTE_S(8)
  } else {
    SMAUL_ROUTE_S(16)
  }
#undef SMAUL_ROUTE_S
#undef SMAUL_ROUTE_S2
  return check_launch("router_mfma_kernel");
}

static int launch_router(const void* x, int x_dtype, const float* gate_w, const float* gate_b,
                         const RouteOut& o, int64_t T, int64_t d, int64_t E, int64_t k,
                         hipStream_t stream) {
  const int64_t tpb = route_tpb(T, E, d, x_dtype);
  const int64_t nb = (T + tpb - 1) / tpb;
  if (nb > 2147483647LL) return fail(SMAUL_ERR_UNSUPPORTED, "router: too many tokens");
  if (route_mfma_ok(E, d, x_dtype) && tpb == 16) return launch_router_small(x, gate_w, gate_b, o, T, d, E, k, stream);
  const bool bf = x_dtype == SMAUL_DTYPE_BF16;
  if (route_mfma_ok(E, d, x_dtype)) {
    const uint16_t* xb = (const uint16_t*)x;
    const dim3 grid((unsigned)nb), block(ROUTE_MFMA_THREADS);
    const int ksw = route_ksw(d);
#define SMAUL_ROUTE_M2(EMAX, EXACT)                                                                          \
  if (ksw == 4)                                                                                              \
    hipLaunchKernelGGL((router_mfma_kernel<EMAX, EXACT, 4, 4>), grid, block, 0, stream, xb, gate_w, gate_b, o, T, \
                       (int)d, (int)E, (int)k);                                                              \
  else                                                                                                       \
    hipLaunchKernelGGL((router_mfma_kernel<EMAX, EXACT, 8, 4>), grid, block, 0, stream, xb, gate_w, gate_b, o, T, \
                       (int)d, (int)E, (int)k);
#define SMAUL_ROUTE_M(EMAX)     \
  if (E == EMAX) {              \
    SMAUL_ROUTE_M2(EMAX, true)  \
  } else {                      \
    SMAUL_ROUTE_M2(EMAX, false) \
  }
    if (E <= 4) {
      SMAUL_ROUTE_M(4)
    } else if (E <= 8) {
      SMAUL_ROUTE_M(8)
    } else {
      SMAUL_ROUTE_M(16)
    }
#undef SMAUL_ROUTE_M
#undef SMAUL_ROUTE_M2
    return check_launch("router_mfma_kernel");
  }
  const dim3 grid((unsigned)nb), block(ROUTE_THREADS);
#define SMAUL_ROUTE1(TB, EMAX, EXACT)                                                                     \
  if (bf)                                                                                                 \
    hipLaunchKernelGGL((router_kernel<true, TB, EMAX, EXACT>), grid, block, 0, stream, x, gate_w, gate_b, o, \
                       T, (int)d, (int)E, (int)k);                                                        \
  else                                                                                                    \
    hipLaunchKernelGGL((router_kernel<false, TB, EMAX, EXACT>), grid, block, 0, stream, x, gate_w, gate_b, \
                       o, T, (int)d, (int)E, (int)k);
#define SMAUL_ROUTE(TB, EMAX)    \
  if (E == EMAX) {               \
    SMAUL_ROUTE1(TB, EMAX, true)  \
  } else {                       \
    SMAUL_ROUTE1(TB, EMAX, false) \
  }
  static_assert(route_tb(4) * 4 == 32 && route_tb(8) * 8 == 32 && route_tb(16) * 16 == 64 && route_tb(64) * 64 == 64,
                "router butterfly expects 32 or 64 partial sums per lane");
  if (E <= 4) {
    SMAUL_ROUTE(route_tb(4), 4)
  } else if (E <= 8) {
    SMAUL_ROUTE(route_tb(8), 8)
  } else if (E <= 16) {
    SMAUL_ROUTE(route_tb(16), 16)
  } else {
    SMAUL_ROUTE(route_tb(64), 64)
  }
#undef SMAUL_ROUTE1
#undef SMAUL_ROUTE
  return check_launch("router_kernel");
}

static int check_router_args(const void* x, int x_dtype, const float* gate_w, int64_t T, int64_t d,
                             int64_t E, int64_t k) {
  if (T < 0 || d <= 0 || E < 1 || E > MAX_E || k < 1 || k > E || k > 8)
    return fail(SMAUL_ERR_INVALID, "router: need T>=0, d>0, 1<=k<=min(E,8), E<=64 (T=%lld d=%lld E=%lld k=%lld)",
                (long long)T, (long long)d, (long long)E, (long long)k);
  if (!dtype_ok(x_dtype)) return fail(SMAUL_ERR_INVALID, "router: bad x dtype");
  if (d % 8 != 0) return fail(SMAUL_ERR_UNSUPPORTED, "router: d must be a multiple of 8");
  if (T > 0 && (!x || !gate_w)) return fail(SMAUL_ERR_INVALID, "router: null pointer");
  if (T > 0 && (!aligned16(x) || !aligned16(gate_w)))
    return fail(SMAUL_ERR_INVALID, "router: x and gate_w must be 16-byte aligned");
  return SMAUL_OK;
}

int smaul_moe_router(const void* x, int x_dtype, const float* gate_w, const float* gate_b,
                     float* prob, int64_t* topi, float* topw, int64_t T, int64_t d, int64_t E,
                     int64_t k, hipStream_t stream) {
  int rc = check_router_args(x, x_dtype, gate_w, T, d, E, k);
  if (rc) return rc;
  if (T == 0) return SMAUL_OK;
  if (!prob || !topi || !topw) return fail(SMAUL_ERR_INVALID, "router: null output pointer");
  RouteOut o{};
  o.prob = prob;
  o.topi = topi;
  o.topw = topw;
  return launch_router(x, x_dtype, gate_w, gate_b, o, T, d, E, k, stream);
}

int64_t smaul_moe_dispatch_workspace_size(int64_t T, int64_t E) {
  if (T < 0 || E < 1) return -1;
  const int64_t nb = (T + DISPATCH_TPB - 1) / DISPATCH_TPB;
  return align256(nb * E * 4) * 2;
}

static int launch_scan_scatter(const int64_t* topi, const float* topw, int32_t* blockcnt,
                               int32_t* blockoff, int32_t* counts, int32_t* seg_off, int32_t* tile_off,
                               int32_t* perm_row, float* perm_w, int32_t* inv, int64_t T, int64_t E,
                               int64_t k, int64_t block_m, int64_t tpb, hipStream_t stream) {
  const int64_t nb = (T + tpb - 1) / tpb;
  // One launch while every block can sum all block counts from its unrolled
  // reads (nb <= 256); past that each block would re-read nb * E counts, a
  // cost growing with nb^2, so the scan runs once in its own kernel.
  if (E <= 16 && nb <= SCAN_FUSED_CHUNKS * 64) {
#define SMAUL_SCS(EMAX)                                                                                         \
  hipLaunchKernelGGL((dispatch_scan_scatter_kernel<EMAX>), dim3((unsigned)nb), dim3(64), 0, stream, topi, topw, \
                     blockcnt, counts, seg_off, tile_off, perm_row, perm_w, inv, T, (int)E, (int)k, (int)tpb, nb, \
                     (int)block_m)
    if (E <= 8) SMAUL_SCS(8);
    else SMAUL_SCS(16);
#undef SMAUL_SCS
    return check_launch("dispatch_scan_scatter_kernel");
  }
  hipLaunchKernelGGL(dispatch_scan_kernel, dim3(1), dim3(SCAN_THREADS), 0, stream, blockcnt, blockoff, counts,
                     seg_off, tile_off, nb, (int)E, (int)block_m);
  int rc = check_launch("dispatch_scan_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(dispatch_scatter_kernel, dim3((unsigned)nb), dim3(64), 0, stream, topi, topw, blockoff,
                     seg_off, perm_row, perm_w, inv, T, (int)E, (int)k, (int)tpb);
  return check_launch("dispatch_scatter_kernel");
}

int smaul_moe_dispatch(const int64_t* topi, const float* topw, int32_t* counts, int32_t* seg_off,
                       int32_t* tile_off, int32_t* perm_row, float* perm_w, int32_t* inv, int64_t T,
                       int64_t E, int64_t k, int64_t block_m, void* workspace, int64_t workspace_bytes,
                       hipStream_t stream) {
  if (T < 0 || E < 1 || E > MAX_E || k < 1 || k > E || k > 8)
    return fail(SMAUL_ERR_INVALID, "dispatch: need T>=0, 1<=k<=min(E,8), E<=64");
  if (T * k > 2147483647LL) return fail(SMAUL_ERR_UNSUPPORTED, "dispatch: T*k exceeds int32");
  if (!(block_m == 16 || block_m == 32 || block_m == 64 || block_m == 128 || block_m == 256))
    return fail(SMAUL_ERR_INVALID, "dispatch: block_m must be 16..256 (power of two)");
  if (!topi || !topw || !counts || !seg_off || !tile_off || !perm_row || !perm_w || !inv)
    return fail(SMAUL_ERR_INVALID, "dispatch: null pointer");
  const int64_t need = smaul_moe_dispatch_workspace_size(T, E);
  if (workspace_bytes < need || (need > 0 && !workspace))
    return fail(SMAUL_ERR_INVALID, "dispatch: workspace %lld < %lld bytes", (long long)workspace_bytes,
                (long long)need);
  const int64_t nb = (T + DISPATCH_TPB - 1) / DISPATCH_TPB;
  int32_t* blockcnt = (int32_t*)workspace;
  int32_t* blockoff = (int32_t*)((char*)workspace + align256(nb * E * 4));
  if (nb > 0) {
    hipLaunchKernelGGL(block_count_kernel, dim3((unsigned)nb), dim3(64), 0, stream, topi, topw, blockcnt, T,
                       (int)E, (int)k, DISPATCH_TPB);
    int rc = check_launch("block_count_kernel");
    if (rc) return rc;
  }
  return launch_scan_scatter(topi, topw, blockcnt, blockoff, counts, seg_off, tile_off, perm_row, perm_w, inv,
                             T, E, k, block_m, DISPATCH_TPB, stream);
}

int smaul_moe_block_m(int64_t T, int64_t d, int64_t h, int64_t E, int64_t k, int64_t tile,
                      int act_dtype) {
  return pick_block_m(T, d, h, E, k, tile, act_dtype);
}

static int moe_gemm(bool swiglu, const void* act, int act_dtype, const int32_t* perm_row,
                    const uint8_t* const* w1, const float* const* s1, const uint8_t* const* w2,
                    const float* const* s2, void* out, const int32_t* seg_off,
                    const int32_t* tile_off, int64_t max_tiles, int64_t E, int64_t K, int64_t N,
                    int64_t tile, int64_t block_m, int flags, hipStream_t stream) {
  if (!dtype_ok(act_dtype)) return fail(SMAUL_ERR_INVALID, "moe gemm: bad dtype");
  if (E < 1 || E > MAX_E || K <= 0 || N <= 0 || tile <= 0 || max_tiles < 0)
    return fail(SMAUL_ERR_INVALID, "moe gemm: bad sizes");
  if (kmode_of(tile) < 0) return fail(SMAUL_ERR_UNSUPPORTED, "moe gemm: tile must be 32 or a multiple of 64");
  if (K % 16 != 0 || !aligned16(act))
    return fail(SMAUL_ERR_UNSUPPORTED, "moe gemm: K must be a multiple of 16 and activations 16-byte aligned");
  const int64_t big_bm = act_dtype == SMAUL_DTYPE_BF16 ? CfgBig::BM : CfgBigF32::BM;
  if (!(block_m == big_bm || block_m == CfgSmall::BM ||
        ((block_m == DECODE_BM || block_m == DMA_SMALL_BM) && act_dtype == SMAUL_DTYPE_BF16)))
    return fail(SMAUL_ERR_INVALID, "moe gemm: block_m must come from smaul_moe_block_m");
  if (!act || !w1 || !s1 || !out || !seg_off || !tile_off || (swiglu && (!w2 || !s2)))
    return fail(SMAUL_ERR_INVALID, "moe gemm: null pointer");
  if ((flags & SMAUL_FLAG_TILED_LAYOUT) && (tile != 64 || K % 64 != 0))
    return fail(SMAUL_ERR_INVALID, "moe gemm: the tiled layout needs tile 64 and K a multiple of 64");
  if (max_tiles == 0) return SMAUL_OK;
  GemmArgs a{};
  a.x = act;
  a.row_idx = perm_row;
  a.ldx = K;
  a.wp = w1;
  a.sp = s1;
  a.wp2 = w2;
  a.sp2 = s2;
  a.y = out;
  a.ldy = N;
  a.K = K;
  a.N = N;
  a.nt = (K + tile - 1) / tile;
  a.tile = tile;
  a.seg_off = seg_off;
  a.tile_off = tile_off;
  a.E = (int)E;
  a.tiled = (flags & SMAUL_FLAG_TILED_LAYOUT) != 0;
  const bool canon = (flags & SMAUL_FLAG_CANONICAL_CODES) != 0;
  if (block_m == DECODE_BM) {
    // decode kernels: K in whole 64-wide blocks, one scale per block, rows per
    // expert <= 64 (the dispatch rows of T <= 64 tokens)
    if (tile != 64 || K % 128 != 0)
      return fail(SMAUL_ERR_INVALID, "moe gemm: block_m %d needs tile 64 and K a multiple of 128", DECODE_BM);
    if (swiglu) return canon ? launch_decode<true, true>(a, stream) : launch_decode<true, false>(a, stream);
    return canon ? launch_decode<false, true>(a, stream) : launch_decode<false, false>(a, stream);
  }
  // 128-row tiles: the LDS-DMA kernels when the activations are bf16, the
  // codes promised 16-byte aligned and the shapes fit them (row indices of
  // x and of hdn are both below max_tiles * block_m); the register-staged
  // kernels otherwise, on the same tile table
  static_assert(CfgDmaGU::BM == CfgBig::BM && CfgDmaDown::BM == CfgBig::BM && CfgDmaDownN::BM == CfgBig::BM,
                "one tile table for both kernels");
  if (block_m == big_bm &&
      dma_gemm_ok(a, act_dtype, flags, max_tiles * block_m, swiglu ? CfgDmaGU::BN / 2 : CfgDmaDown::BN)) {
    if (swiglu)
      return canon ? launch_gemm_dma<CfgDmaGU, true, true>(a, max_tiles, stream)
                   : launch_gemm_dma<CfgDmaGU, true, false>(a, max_tiles, stream);
    if (max_tiles * (N / CfgDmaDown::BN) < 8 * (int64_t)cu_count())
      return canon ? launch_gemm_dma<CfgDmaDownN, false, true>(a, max_tiles, stream)
                   : launch_gemm_dma<CfgDmaDownN, false, false>(a, max_tiles, stream);
    return canon ? launch_gemm_dma<CfgDmaDown, false, true>(a, max_tiles, stream)
                 : launch_gemm_dma<CfgDmaDown, false, false>(a, max_tiles, stream);
  }
  if (block_m == DMA_SMALL_BM) {  // no other kernel runs this tile table
    static_assert(CfgDmaGU64::BM == DMA_SMALL_BM && CfgDma64x128::BM == DMA_SMALL_BM, "64-row tile table");
    if (!dma_gemm_ok(a, act_dtype, flags, max_tiles * block_m, 128))
      return fail(SMAUL_ERR_UNSUPPORTED, "moe gemm: block_m 64 needs the LDS-DMA kernels' shapes and aligned codes");
    if (swiglu)
      return canon ? launch_gemm_dma<CfgDmaGU64, true, true>(a, max_tiles, stream)
                   : launch_gemm_dma<CfgDmaGU64, true, false>(a, max_tiles, stream);
    return canon ? launch_gemm_dma<CfgDma64x128, false, true>(a, max_tiles, stream)
                 : launch_gemm_dma<CfgDma64x128, false, false>(a, max_tiles, stream);
  }
  if (block_m == big_bm)
    return gemm_dispatch_moe<CfgBig, CfgBigF32>(a, swiglu, act_dtype, max_tiles, canon, stream);
  return gemm_dispatch_moe<CfgSmall, CfgSmall>(a, swiglu, act_dtype, max_tiles, canon, stream);
}

int smaul_moe_gate_up(const void* x, int act_dtype, const int32_t* perm_row,
                      const uint8_t* const* gate_w, const float* const* gate_s,
                      const uint8_t* const* up_w, const float* const* up_s, void* hdn,
                      const int32_t* seg_off, const int32_t* tile_off, int64_t max_tiles, int64_t E,
                      int64_t d, int64_t h, int64_t tile, int64_t block_m, int flags,
                      hipStream_t stream) {
  if (!perm_row) return fail(SMAUL_ERR_INVALID, "gate_up: null perm_row");
  return moe_gemm(true, x, act_dtype, perm_row, gate_w, gate_s, up_w, up_s, hdn, seg_off, tile_off,
                  max_tiles, E, d, h, tile, block_m, flags, stream);
}

int smaul_moe_down(const void* hdn, int act_dtype, const uint8_t* const* down_w,
                   const float* const* down_s, void* yperm, const int32_t* seg_off,
                   const int32_t* tile_off, int64_t max_tiles, int64_t E, int64_t d, int64_t h,
                   int64_t tile, int64_t block_m, int flags, hipStream_t stream) {
  return moe_gemm(false, hdn, act_dtype, nullptr, down_w, down_s, nullptr, nullptr, yperm, seg_off,
                  tile_off, max_tiles, E, h, d, tile, block_m, flags, stream);
}

// Dense SwiGLU FFN (one expert, every row): the grouped kernels in their
// dense form (no segment table, no row gather).  gate and up run as one
// launch with the SwiGLU epilogue into hdn (the workspace), then down writes
// out directly.
// bf16: hdn [rows, h].  fp32: two parts of align256(rows * h * 4) bytes; the
// register-staged kernels keep hdn in fp32 in the first, the LDS-DMA path
// (swiffn_f32_planes) puts the bf16 hi / lo planes of x in the first and those
// of hdn in the second.  A workspace of only the first part runs the
// register-staged kernels.
int64_t smaul_swiffn_workspace_size(int64_t rows, int64_t h, int act_dtype) {
  if (rows < 0 || h <= 0 || !dtype_ok(act_dtype)) return -1;
  return act_dtype == SMAUL_DTYPE_BF16 ? align256(rows * h * 2) : align256(rows * h * 4) + align256(rows * h * 4);
}

static int dense_gemm(bool swiglu, const void* act, int act_dtype, const uint8_t* w1, const float* s1,
                      const uint8_t* w2, const float* s2, void* out, int64_t rows, int64_t K, int64_t N,
                      int64_t tile, int flags, hipStream_t stream) {
  GemmArgs a{};
  a.x = act;
  a.row_idx = nullptr;
  a.ldx = K;
  a.w = w1;
  a.s = s1;
  a.w2 = w2;
  a.s2 = s2;
  a.y = out;
  a.ldy = N;
  a.K = K;
  a.N = N;
  a.nt = (K + tile - 1) / tile;
  a.tile = tile;
  a.seg_off = nullptr;
  a.tile_off = nullptr;
  a.R = rows;
  a.E = 1;
  a.tiled = (flags & SMAUL_FLAG_TILED_LAYOUT) != 0;
  const bool canon = (flags & SMAUL_FLAG_CANONICAL_CODES) != 0;
  const int dt = pick_dense_tile(swiglu, rows, N);
  if (dt >= 0 && dma_gemm_ok(a, act_dtype, flags | SMAUL_FLAG_ALIGNED_CODES, rows, 128)) {
    if (swiglu)
      return canon ? launch_dense_dma<true, true, false>(a, dt, stream)
                   : launch_dense_dma<true, false, false>(a, dt, stream);
    return canon ? launch_dense_dma<false, true, false>(a, dt, stream)
                 : launch_dense_dma<false, false, false>(a, dt, stream);
  }
  const bool small = rows <= 64;
  if (act_dtype == SMAUL_DTYPE_BF16) {
    const int64_t mt = (rows + (small ? CfgSmall::BM : CfgBig::BM) - 1) / (small ? CfgSmall::BM : CfgBig::BM);
    return small ? gemm_dispatch_moe<CfgSmall, CfgSmall>(a, swiglu, act_dtype, mt, canon, stream)
                 : gemm_dispatch_moe<CfgBig, CfgBigF32>(a, swiglu, act_dtype, mt, canon, stream);
  }
  const int64_t mt = (rows + (small ? CfgSmall::BM : CfgBigF32::BM) - 1) / (small ? CfgSmall::BM : CfgBigF32::BM);
  return small ? gemm_dispatch_moe<CfgSmall, CfgSmall>(a, swiglu, act_dtype, mt, canon, stream)
               : gemm_dispatch_moe<CfgBig, CfgBigF32>(a, swiglu, act_dtype, mt, canon, stream);
}

// SwiFFN with fp32 activations on the LDS-DMA kernels: x is split into bf16
// hi / lo planes, gate+up runs over both (K doubled, each weight block read
// for its hi and its lo half) and its SwiGLU epilogue, in fp32, stores the
// products already split into the two planes of hdn, over which the down
// projection runs with fp32 output: every value the reference forms in fp32
// stays within 2^-18 relative of it.  The planes of x go into the workspace's
// first part (rows * 2d bf16 <= rows * h fp32), those of hdn into the second.
// Returns -1 (nothing launched) when the shape does not fit: tile 64, d and h
// multiples of 128, d <= h, more than 64 rows, and the kernels' offset limits;
// otherwise a status.
static int swiffn_f32_planes(const float* x, const uint8_t* gw, const float* gs, const uint8_t* uw, const float* us,
                             const uint8_t* dw, const float* ds, float* out, char* ws, int64_t hdn_bytes,
                             int64_t rows, int64_t d, int64_t h, int64_t tile, int flags, hipStream_t stream) {
  if (tile != 64 || d % 128 != 0 || h % 128 != 0 || d > h || rows <= 64) return -1;
  uint16_t* xplanes = (uint16_t*)ws;
  uint16_t* hplanes = (uint16_t*)(ws + hdn_bytes);
  GemmArgs a{};
  a.x = xplanes;
  a.ldx = 2 * d;
  a.w = gw;
  a.s = gs;
  a.w2 = uw;
  a.s2 = us;
  a.y = hplanes;
  a.ldy = 2 * h;
  a.y_lo = h;
  a.K = 2 * d;
  a.kw = d;
  a.N = h;
  a.nt = d / 64;
  a.tile = 64;
  a.R = rows;
  a.E = 1;
  a.tiled = (flags & SMAUL_FLAG_TILED_LAYOUT) != 0;
  GemmArgs b = a;
  b.y_lo = 0;
  b.x = hplanes;
  b.ldx = 2 * h;
  b.w = dw;
  b.s = ds;
  b.w2 = nullptr;
  b.s2 = nullptr;
  b.y = out;
  b.ldy = d;
  b.K = 2 * h;
  b.kw = h;
  b.N = d;
  b.nt = h / 64;
  const int fl = flags | SMAUL_FLAG_ALIGNED_CODES;  // swiffn requires 16-byte aligned codes
  const int dtg = pick_dense_tile(true, rows, h), dtd = pick_dense_tile(false, rows, d);
  if (dtg < 0 || dtd < 0 || !dma_gemm_ok(a, SMAUL_DTYPE_BF16, fl, rows, 128) ||
      !dma_gemm_ok(b, SMAUL_DTYPE_BF16, fl, rows, 128))
    return -1;
  const bool canon = (flags & SMAUL_FLAG_CANONICAL_CODES) != 0;
  int rc = launch_split_planes(x, xplanes, rows, d, stream);
  if (rc != SMAUL_OK) return rc;
  rc = canon ? launch_dense_dma<true, true, true>(a, dtg, stream) : launch_dense_dma<true, false, true>(a, dtg, stream);
  if (rc != SMAUL_OK) return rc;
  return canon ? launch_dense_dma<false, true, true>(b, dtd, stream) : launch_dense_dma<false, false, true>(b, dtd, stream);
}

int smaul_swiffn_forward(const void* x, int act_dtype, const uint8_t* gate_w8, const float* gate_s,
                         const uint8_t* up_w8, const float* up_s, const uint8_t* down_w8, const float* down_s,
                         void* out, void* workspace, int64_t workspace_bytes, int64_t rows, int64_t d, int64_t h,
                         int64_t tile, int flags, hipStream_t stream) {
  if (!dtype_ok(act_dtype)) return fail(SMAUL_ERR_INVALID, "swiffn: activation dtype must be f32|bf16");
  if (rows < 0 || d <= 0 || h <= 0 || tile <= 0)
    return fail(SMAUL_ERR_INVALID, "swiffn: need rows >= 0 and positive d, h, tile");
  if (kmode_of(tile) < 0) return fail(SMAUL_ERR_UNSUPPORTED, "swiffn: tile must be 32 or a multiple of 64");
  if (d % 16 != 0 || h % 16 != 0) return fail(SMAUL_ERR_UNSUPPORTED, "swiffn: d and h must be multiples of 16");
  if ((flags & SMAUL_FLAG_TILED_LAYOUT) && (tile != 64 || d % 64 != 0 || h % 64 != 0))
    return fail(SMAUL_ERR_INVALID, "swiffn: the tiled layout needs tile 64 and d, h multiples of 64");
  // fp32: the hdn part is required, the planes part optional (see the size query)
  const int64_t hdn_bytes = align256(rows * h * (act_dtype == SMAUL_DTYPE_BF16 ? 2 : 4));
  if (workspace_bytes < hdn_bytes) return fail(SMAUL_ERR_INVALID, "swiffn: workspace %lld < %lld bytes",
                                                (long long)workspace_bytes, (long long)hdn_bytes);
  if (rows == 0) return SMAUL_OK;
  if (!x || !gate_w8 || !gate_s || !up_w8 || !up_s || !down_w8 || !down_s || !out || !workspace)
    return fail(SMAUL_ERR_INVALID, "swiffn: null pointer");
  if (!aligned16(x) || !aligned16(out) || !aligned16(workspace) || !aligned16(gate_w8) || !aligned16(up_w8) ||
      !aligned16(down_w8))
    return fail(SMAUL_ERR_UNSUPPORTED, "swiffn: x, codes, out and workspace must be 16-byte aligned");
  if (rows * (h > d ? h : d) > 2147483647LL) return fail(SMAUL_ERR_UNSUPPORTED, "swiffn: rows * width exceeds int32");
  if (act_dtype == SMAUL_DTYPE_F32 && workspace_bytes >= smaul_swiffn_workspace_size(rows, h, act_dtype)) {
    const int rc = swiffn_f32_planes((const float*)x, gate_w8, gate_s, up_w8, up_s, down_w8, down_s, (float*)out,
                                     (char*)workspace, hdn_bytes, rows, d, h, tile, flags, stream);
    if (rc != -1) return rc;  // -1: the shape does not fit the LDS-DMA kernels
  }
  int rc = dense_gemm(true, x, act_dtype, gate_w8, gate_s, up_w8, up_s, workspace, rows, d, h, tile, flags, stream);
  if (rc) return rc;
  return dense_gemm(false, workspace, act_dtype, down_w8, down_s, nullptr, nullptr, out, rows, h, d, tile, flags,
                    stream);
}

int smaul_moe_combine(const void* yperm, int act_dtype, const int64_t* topi, const float* topw,
                      const int32_t* inv, void* out, int64_t T, int64_t d, int64_t k,
                      hipStream_t stream) {
  if (!dtype_ok(act_dtype) || T < 0 || d <= 0 || k < 1 || k > 8)
    return fail(SMAUL_ERR_INVALID, "combine: bad arguments");
  if (d % 8 != 0) return fail(SMAUL_ERR_UNSUPPORTED, "combine: d must be a multiple of 8");
  if (T == 0) return SMAUL_OK;
  if (!yperm || !topi || !topw || !inv || !out) return fail(SMAUL_ERR_INVALID, "combine: null pointer");
  if (!aligned16(yperm) || !aligned16(out)) return fail(SMAUL_ERR_INVALID, "combine: unaligned buffers");
  const bool bf16 = act_dtype == SMAUL_DTYPE_BF16;
  const int cw = (bf16 && d % 32 == 0) ? 32 : d % 16 == 0 ? 16 : 8;
  const int km = k <= 2 ? 2 : k <= 4 ? 4 : 8;
  const int64_t total = T * (d / cw);
  const dim3 grid((unsigned)((total + 255) / 256)), block(256);
#define SMAUL_COMB(B, CW, KM)                                                                                  \
  hipLaunchKernelGGL((combine_kernel<B, CW, KM>), grid, block, 0, stream, yperm, topi, topw, inv, out, T, (int)d, \
                     (int)k)
#define SMAUL_COMB_K(B, CW)       \
  if (km == 2) SMAUL_COMB(B, CW, 2); \
  else if (km == 4) SMAUL_COMB(B, CW, 4); \
  else SMAUL_COMB(B, CW, 8)
  if (bf16) {
    if (cw == 32) { SMAUL_COMB_K(true, 32); }
    else if (cw == 16) { SMAUL_COMB_K(true, 16); }
    else { SMAUL_COMB_K(true, 8); }
  } else {
    if (cw == 16) { SMAUL_COMB_K(false, 16); }
    else { SMAUL_COMB_K(false, 8); }
  }
#undef SMAUL_COMB_K
#undef SMAUL_COMB
  return check_launch("combine_kernel");
}

int smaul_rms_norm(const void* x, int act_dtype, const float* weight, void* out, int64_t T,
                   int64_t d, float eps, hipStream_t stream) {
  if (!dtype_ok(act_dtype) || T < 0 || d <= 0 || d > INT32_MAX)
    return fail(SMAUL_ERR_INVALID, "rms_norm: bad arguments");
  if (!(eps > 0.0f) || !std::isfinite(eps)) return fail(SMAUL_ERR_INVALID, "rms_norm: eps must be positive finite");
  if (T == 0) return SMAUL_OK;
  if (!x || !out) return fail(SMAUL_ERR_INVALID, "rms_norm: null pointer");
  const bool bf = act_dtype == SMAUL_DTYPE_BF16;
  const bool vec = aligned16(x) && aligned16(out) && d % 16 == 0;
  const dim3 grid((unsigned)((T + 3) / 4)), block(256);
  if (bf) {
    if (vec) hipLaunchKernelGGL((rms_norm_kernel<true, true>), grid, block, 0, stream, x, weight, out, T, (int)d, eps);
    else hipLaunchKernelGGL((rms_norm_kernel<true, false>), grid, block, 0, stream, x, weight, out, T, (int)d, eps);
  } else {
    if (vec) hipLaunchKernelGGL((rms_norm_kernel<false, true>), grid, block, 0, stream, x, weight, out, T, (int)d, eps);
    else hipLaunchKernelGGL((rms_norm_kernel<false, false>), grid, block, 0, stream, x, weight, out, T, (int)d, eps);
  }
  return check_launch("rms_norm_kernel");
}

// Workspace layout (each piece 256-byte aligned):
//   seg_off[E+1] tile_off[E+1] perm_row[T*k] perm_w[T*k] inv[T*k]
//   blockcnt[nb*E] blockoff[nb*E]  (nb = router token blocks)
//   hdn[T*k, h] (act dtype)  yperm[T*k, d] (act dtype)
static int64_t route_blocks(int64_t T, int64_t E, int64_t d, int x_dtype) {
  const int64_t tpb = route_tpb(T, E, d, x_dtype);
  return (T + tpb - 1) / tpb;
}

int64_t smaul_moe_workspace_size(int64_t T, int64_t d, int64_t h, int64_t E, int64_t k,
                                 int act_dtype) {
  if (T < 0 || d <= 0 || h <= 0 || E < 1 || k < 1 || !dtype_ok(act_dtype)) return -1;
  const int64_t el = act_dtype == SMAUL_DTYPE_BF16 ? 2 : 4;
  const int64_t R = T * k;
  int64_t n = 0;
  n += align256((E + 1) * 4) * 2;
  n += align256(R * 4) * 3;
  n += align256(route_blocks(T, E, d, act_dtype) * E * 4) * 2;
  n += align256(R * h * el);
  n += align256(R * d * el);
  n += 256;  // sync words of the decode path's fused combine
  // fp32 x: its bf16 hi / lo planes for the LDS-DMA GEMMs (moe_f32_planes)
  if (act_dtype == SMAUL_DTYPE_F32) n += align256(T * d * 4);
  return n;
}

// The RMSNorm that follows the MoE output (smaul_moe_forward_norm)
struct OutNorm {
  const float* weight;
  float eps;
  void* out;
};

// The next layer's router, run on the normed output (smaul_moe_forward_chain)
struct NextRoute {
  const float* gate_w;
  const float* gate_b;
  int64_t E, k;
  float* prob;
  int64_t* topi;
  float* topw;
};

// combine + norm + the next layer's MFMA router in one kernel (bf16, d <= 2048)
static int launch_combine_norm_route(const void* yperm, const int64_t* topi, const float* topw, const int32_t* inv,
                                     void* out, const OutNorm& nrm, const NextRoute& nr, int64_t T, int64_t d,
                                     int64_t k, hipStream_t stream) {
  RouteOut no{};
  no.prob = nr.prob;
  no.topi = nr.topi;
  no.topw = nr.topw;
  const dim3 grid((unsigned)((T + CNR_TOK - 1) / CNR_TOK)), block(CNR_TOK * 64);
  const int E = (int)nr.E;
#define SMAUL_CNR2(NCH, KSW, EMAX, EXACT)                                                                         \
  hipLaunchKernelGGL((combine_norm_route_kernel<NCH, EMAX, EXACT, KSW>), grid, block, 0, stream, yperm, topi, topw, \
                     inv, out, nrm.weight, nrm.eps, nrm.out, T, (int)d, (int)k, nr.gate_w, nr.gate_b, no, E,       \
                     (int)nr.k)
#define SMAUL_CNR1(NCH, KSW)                                                 \
  if (E <= 4) {                                                              \
    if (E == 4) SMAUL_CNR2(NCH, KSW, 4, true); else SMAUL_CNR2(NCH, KSW, 4, false);   \
  } else if (E <= 8) {                                                       \
    if (E == 8) SMAUL_CNR2(NCH, KSW, 8, true); else SMAUL_CNR2(NCH, KSW, 8, false);   \
  } else {                                                                   \
    if (E == 16) SMAUL_CNR2(NCH, KSW, 16, true); else SMAUL_CNR2(NCH, KSW, 16, false); \
  }
  if (route_ksw(d) == 4) {
    SMAUL_CNR1(1, 4)
  } else {
    SMAUL_CNR1(2, 8)
  }
#undef SMAUL_CNR1
#undef SMAUL_CNR2
  return check_launch("combine_norm_route_kernel");
}

// The last stage of the layer: the combine, or the combine and the output
// norm (fused when d % 16 == 0 and d <= 4096, else the two kernels), and the
// next layer's router on the normed rows when nr is given (fused into the
// same kernel for bf16 activations and the MFMA router's shapes, else
// smaul_moe_router on norm_out).
static int finish_combine(const void* yperm, int act_dtype, const int64_t* topi, const float* topw,
                          const int32_t* inv, void* out, int64_t T, int64_t d, int64_t k, const OutNorm* nrm,
                          const NextRoute* nr, hipStream_t stream) {
  if (!nrm) return smaul_moe_combine(yperm, act_dtype, topi, topw, inv, out, T, d, k, stream);
  const bool fuse_norm =
      d % 16 == 0 && d <= 64 * 16 * RMS_KEEP && aligned16(yperm) && aligned16(out) && aligned16(nrm->out);
  if (nr) {
    if (fuse_norm && route_mfma_ok(nr->E, d, act_dtype) && aligned16(nr->gate_w))
      return launch_combine_norm_route(yperm, topi, topw, inv, out, *nrm, *nr, T, d, k, stream);
    const int rc = finish_combine(yperm, act_dtype, topi, topw, inv, out, T, d, k, nrm, nullptr, stream);
    if (rc) return rc;
    return smaul_moe_router(nrm->out, act_dtype, nr->gate_w, nr->gate_b, nr->prob, nr->topi, nr->topw, T, d, nr->E,
                            nr->k, stream);
  }
  if (fuse_norm) {
    const int nch = (int)((d + 1023) / 1024);
    const dim3 grid((unsigned)((T + 3) / 4)), block(256);
    const bool bf = act_dtype == SMAUL_DTYPE_BF16;
#define SMAUL_CN(BF, N) hipLaunchKernelGGL((combine_norm_kernel<BF, N>), grid, block, 0, stream, yperm, topi, topw, \
                                           inv, out, nrm->weight, nrm->eps, nrm->out, T, (int)d, (int)k)
    if (nch == 1) { if (bf) SMAUL_CN(true, 1); else SMAUL_CN(false, 1); }
    else if (nch == 2) { if (bf) SMAUL_CN(true, 2); else SMAUL_CN(false, 2); }
    else { if (bf) SMAUL_CN(true, 4); else SMAUL_CN(false, 4); }
#undef SMAUL_CN
    return check_launch("combine_norm_kernel");
  }
  const int rc = smaul_moe_combine(yperm, act_dtype, topi, topw, inv, out, T, d, k, stream);
  if (rc) return rc;
  return smaul_rms_norm(out, act_dtype, nrm->weight, nrm->out, T, d, nrm->eps, stream);
}

// The fused decode tail's wait: arrivals beyond the grid and the poll limit
// (smaul_debug_tail_wait; 0 and CNR_SPIN_LIMIT in use)
static std::atomic<int> g_tail_wait_extra{0};
static std::atomic<int> g_tail_spin_limit{CNR_SPIN_LIMIT};
static void tail_wait_settings(int& extra, int& limit) {
  extra = g_tail_wait_extra.load(std::memory_order_relaxed);
  limit = g_tail_spin_limit.load(std::memory_order_relaxed);
}

__global__ void wait_timeouts_kernel(int32_t* out, int reset) {
  const int32_t v = __hip_atomic_load(&g_wait_timeouts, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  *out = v;
  if (reset) __hip_atomic_fetch_sub(&g_wait_timeouts, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// fp32 activations through the LDS-DMA grouped GEMMs: the tile rows (128,
// or 64 where a 128-row gate+up grid is under four workgroups per CU, as for
// bf16) when the shapes fit (tile 64, d and h multiples of 128, codes
// promised 16-byte aligned, the kernels' 32-bit offsets for the planes of x
// and of hdn), else 0.
static int64_t f32_planes_block_m(int64_t T, int64_t d, int64_t h, int64_t E, int64_t k, int64_t tile, int flags,
                                  int64_t R, int cus) {
  if (tile != 64 || d % 128 != 0 || h % 128 != 0 || !(flags & SMAUL_FLAG_ALIGNED_CODES)) return 0;
  const int64_t lim = (int64_t)1 << 31;
  const int64_t hrows = ((R + CfgBig::BM - 1) / CfgBig::BM + E) * CfgBig::BM;  // >= the rows either tiling indexes
  if (T * d * 4 >= lim || hrows * h * 4 >= lim || 2 * h * d >= lim) return 0;
  return ((R + CfgBig::BM - 1) / CfgBig::BM + E) * (h / 128) < 4 * (int64_t)cus ? DMA_SMALL_BM : CfgBig::BM;
}

// The grouped gate+up and down of fp32 x (after the dispatch, on the tile
// table of block_m rows): x split into bf16 hi / lo planes ([T][2d]); gate+up
// over both planes of the gathered rows (K doubled, weight blocks wrapped)
// with the SwiGLU product kept in fp32 and stored as the planes of hdn
// ([R][2h], the fp32 hdn's bytes); down over those planes with fp32 output
// into yperm.  Every value the reference forms in fp32 stays within 2^-18
// relative of it.
static int moe_f32_planes(const float* x, uint16_t* xplanes, const int32_t* perm_row, const uint8_t* const* gw,
                          const float* const* gs, const uint8_t* const* uw, const float* const* us,
                          const uint8_t* const* dw, const float* const* ds, uint16_t* hplanes, float* yperm,
                          const int32_t* seg_off, const int32_t* tile_off, int64_t max_tiles, int64_t T, int64_t d,
                          int64_t h, int64_t E, int64_t bm, int flags, hipStream_t stream) {
  GemmArgs g{};
  g.x = xplanes;
  g.row_idx = perm_row;
  g.ldx = 2 * d;
  g.wp = gw;
  g.sp = gs;
  g.wp2 = uw;
  g.sp2 = us;
  g.y = hplanes;
  g.ldy = 2 * h;
  g.y_lo = h;
  g.K = 2 * d;
  g.kw = d;
  g.N = h;
  g.nt = d / 64;
  g.tile = 64;
  g.seg_off = seg_off;
  g.tile_off = tile_off;
  g.E = (int)E;
  g.tiled = (flags & SMAUL_FLAG_TILED_LAYOUT) != 0;
  GemmArgs dn = g;
  dn.x = hplanes;
  dn.row_idx = nullptr;
  dn.ldx = 2 * h;
  dn.wp = dw;
  dn.sp = ds;
  dn.wp2 = nullptr;
  dn.sp2 = nullptr;
  dn.y = yperm;
  dn.ldy = d;
  dn.y_lo = 0;
  dn.K = 2 * h;
  dn.kw = h;
  dn.N = d;
  dn.nt = h / 64;
  if (!dma_gemm_ok(g, SMAUL_DTYPE_BF16, flags, T, 128) || !dma_gemm_ok(dn, SMAUL_DTYPE_BF16, flags, max_tiles * bm, 128))
    return fail(SMAUL_ERR_UNSUPPORTED, "moe_forward: fp32 planes shapes outside the LDS-DMA kernels");
  const bool canon = (flags & SMAUL_FLAG_CANONICAL_CODES) != 0;
  int rc = launch_split_planes(x, xplanes, T, d, stream);
  if (rc != SMAUL_OK) return rc;
  if (bm == DMA_SMALL_BM) {
    rc = canon ? launch_gemm_dma<CfgDmaGU64, true, true, true>(g, max_tiles, stream)
               : launch_gemm_dma<CfgDmaGU64, true, false, true>(g, max_tiles, stream);
    if (rc != SMAUL_OK) return rc;
    return canon ? launch_gemm_dma<CfgDma64x128, false, true, true>(dn, max_tiles, stream)
                 : launch_gemm_dma<CfgDma64x128, false, false, true>(dn, max_tiles, stream);
  }
  rc = canon ? launch_gemm_dma<CfgDmaGU, true, true, true>(g, max_tiles, stream)
             : launch_gemm_dma<CfgDmaGU, true, false, true>(g, max_tiles, stream);
  if (rc != SMAUL_OK) return rc;
  if (d % CfgDmaDown::BN != 0 || max_tiles * (d / CfgDmaDown::BN) < 8 * (int64_t)cu_count())
    return canon ? launch_gemm_dma<CfgDmaDownN, false, true, true>(dn, max_tiles, stream)
                 : launch_gemm_dma<CfgDmaDownN, false, false, true>(dn, max_tiles, stream);
  return canon ? launch_gemm_dma<CfgDmaDown, false, true, true>(dn, max_tiles, stream)
               : launch_gemm_dma<CfgDmaDown, false, false, true>(dn, max_tiles, stream);
}

static int moe_forward_impl(const void* x, int act_dtype, const float* gate_w, const float* gate_b,
                            const uint8_t* const* gate_w8, const float* const* gate_s,
                            const uint8_t* const* up_w8, const float* const* up_s,
                            const uint8_t* const* down_w8, const float* const* down_s, void* out,
                            float* prob, int64_t* topi, float* topw, int32_t* counts, void* workspace,
                            int64_t workspace_bytes, int64_t T, int64_t d, int64_t h, int64_t E, int64_t k,
                            int64_t tile, int flags, const OutNorm* nrm, bool routed, const NextRoute* nr,
                            hipStream_t stream) {
  const int64_t need = smaul_moe_workspace_size(T, d, h, E, k, act_dtype);
  if (need < 0) return fail(SMAUL_ERR_INVALID, "moe_forward: bad sizes");
  if (workspace_bytes < need)
    return fail(SMAUL_ERR_INVALID, "moe_forward: workspace %lld < %lld bytes", (long long)workspace_bytes,
                (long long)need);
  int rc = check_router_args(x, act_dtype, gate_w, T, d, E, k);
  if (rc) return rc;
  if (T == 0) return SMAUL_OK;
  if (T * k > 2147483647LL) return fail(SMAUL_ERR_UNSUPPORTED, "moe_forward: T*k exceeds int32");
  if (((uintptr_t)workspace & 255u) != 0) return fail(SMAUL_ERR_INVALID, "moe_forward: workspace not 256-byte aligned");
  if ((flags & SMAUL_FLAG_TILED_LAYOUT) && (tile != 64 || d % 64 != 0 || h % 64 != 0))
    return fail(SMAUL_ERR_INVALID, "moe_forward: the tiled layout needs tile 64 and d, h multiples of 64");
  const int64_t el = act_dtype == SMAUL_DTYPE_BF16 ? 2 : 4;
  const int64_t R = T * k;
  const int64_t nb = route_blocks(T, E, d, act_dtype);
  char* ws = (char*)workspace;
  int32_t* seg_off = (int32_t*)ws;
  ws += align256((E + 1) * 4);
  int32_t* tile_off = (int32_t*)ws;
  ws += align256((E + 1) * 4);
  int32_t* perm_row = (int32_t*)ws;
  ws += align256(R * 4);
  float* perm_w = (float*)ws;
  ws += align256(R * 4);
  int32_t* inv = (int32_t*)ws;
  ws += align256(R * 4);
  int32_t* blockcnt = (int32_t*)ws;
  ws += align256(nb * E * 4);
  int32_t* blockoff = (int32_t*)ws;
  ws += align256(nb * E * 4);
  void* hdn = ws;
  ws += align256(R * h * el);
  void* yperm = ws;
  ws += align256(R * d * el);
  int32_t* sync = (int32_t*)ws;
  ws += 256;
  uint16_t* xplanes = act_dtype == SMAUL_DTYPE_F32 ? (uint16_t*)ws : nullptr;

  int64_t bm = pick_block_m(T, d, h, E, k, tile, act_dtype);
  // fp32 x on the LDS-DMA kernels over bf16 hi / lo planes (128- or 64-row
  // tiles, by the same grid rule as bf16), else the register-staged kernels
  const int64_t f32p_bm = act_dtype == SMAUL_DTYPE_F32
                              ? f32_planes_block_m(T, d, h, E, k, tile, flags, R, cu_count())
                              : 0;
  if (f32p_bm) bm = f32p_bm;
  if (bm == CfgBig::BM && act_dtype == SMAUL_DTYPE_BF16 &&
      ((R + CfgBig::BM - 1) / CfgBig::BM + E) * (h / 128) < 4 * (int64_t)cu_count()) {
    // a 128-row gate/up grid under four workgroups per CU: 64-row tiles
    // (DMA_SMALL_BM) where both projections fit the LDS-DMA kernels
    const int64_t mt = (R + DMA_SMALL_BM - 1) / DMA_SMALL_BM + E;
    GemmArgs g{};
    g.x = x;
    g.ldx = d;
    g.y = hdn;
    g.ldy = h;
    g.K = d;
    g.N = h;
    g.nt = d / 64;
    g.tile = tile;
    GemmArgs dn = g;
    dn.x = hdn;
    dn.ldx = h;
    dn.y = yperm;
    dn.ldy = d;
    dn.K = h;
    dn.N = d;
    dn.nt = h / 64;
    if (dma_gemm_ok(g, act_dtype, flags, T, 128) && dma_gemm_ok(dn, act_dtype, flags, mt * DMA_SMALL_BM, 128))
      bm = DMA_SMALL_BM;
  }
  // decode regime: the gate/up kernel dispatches for itself
  const bool fused = bm == DECODE_BM && aligned16(x) && h % 16 == 0 &&
                     ds_kbw(d / 64, true) != 0;
  RouteOut o{};
  o.prob = prob;
  o.topi = topi;
  o.topw = topw;
  o.blockcnt = blockcnt;
  o.block_m = (int)bm;
  RouteOut od = o;
  od.counts = counts;
  od.seg_off = seg_off;
  od.tile_off = tile_off;
  od.perm_row = perm_row;
  od.perm_w = perm_w;
  od.inv = inv;
  if (nb == 1 && !fused) o = od;  // one router block: it dispatches too
  if (routed) {
    // prob/topi/topw came with the call (the previous layer's fused router)
  } else if (fused && route_mfma_ok(E, d, act_dtype)) {
    // decode: top-k only, one block per 16 tokens; the gate/up kernel dispatches
    RouteOut ot = o;
    ot.blockcnt = nullptr;
    rc = launch_router_small(x, gate_w, gate_b, ot, T, d, E, k, stream);
  } else {
    rc = launch_router(x, act_dtype, gate_w, gate_b, o, T, d, E, k, stream);
  }
  if (rc) return rc;
  const int64_t max_tiles = (R + bm - 1) / bm + E;
  if (fused) {
    GemmArgs a{};
    a.x = x;
    a.ldx = d;
    a.wp = gate_w8;
    a.sp = gate_s;
    a.wp2 = up_w8;
    a.sp2 = up_s;
    a.y = hdn;
    a.ldy = h;
    a.K = d;
    a.N = h;
    a.nt = d / 64;
    a.tile = 64;
    a.seg_off = seg_off;
    a.tile_off = tile_off;
    a.E = (int)E;
    a.tiled = (flags & SMAUL_FLAG_TILED_LAYOUT) != 0;
    // the combine + norm + next router in the down kernel's tail, when the
    // shapes allow it (the same conditions as combine_norm_route_kernel, and
    // launch_down_cnr's)
    const bool canon = (flags & SMAUL_FLAG_CANONICAL_CODES) != 0;
    const bool cnr = nrm && nr && act_dtype == SMAUL_DTYPE_BF16 && d % 16 == 0 && aligned16(yperm) &&
                     aligned16(out) && aligned16(nrm->out) && route_mfma_ok(nr->E, d, act_dtype) &&
                     aligned16(nr->gate_w) && route_ksw(d) == 4 && T <= 64;
    // without a next router: the combine (and the norm) alone in that tail
    const bool cn = !nr && act_dtype == SMAUL_DTYPE_BF16 && d % 16 == 0 && aligned16(yperm) && aligned16(out) &&
                    (!nrm || aligned16(nrm->out)) && T <= 64;
    GemmArgs b{};
    b.x = hdn;
    b.ldx = h;
    b.wp = down_w8;
    b.sp = down_s;
    b.y = yperm;
    b.ldy = d;
    b.K = h;
    b.N = d;
    b.nt = h / 64;
    b.tile = 64;
    b.seg_off = seg_off;
    b.tile_off = tile_off;
    b.E = (int)E;
    b.tiled = a.tiled;
    CnrArgs cr{};
    if (cnr) {
      RouteOut no{};
      no.prob = nr->prob;
      no.topi = nr->topi;
      no.topw = nr->topw;
      cr = CnrArgs{topi, topw, inv, out, nrm->weight, nrm->eps, nrm->out, T, (int)d, (int)k, nr->gate_w,
                   nr->gate_b, no, (int)nr->E, (int)nr->k, sync, R * d * el};
    }
    if (cn) {
      cr = CnrArgs{topi, topw, inv, out, nrm ? nrm->weight : nullptr, nrm ? nrm->eps : 0.0f,
                   nrm ? nrm->out : nullptr, T, (int)d, (int)k, nullptr, nullptr, RouteOut{}, 0, 0, sync,
                   R * d * el};
    }
    tail_wait_settings(cr.wait_extra, cr.spin_limit);
    DsDispatch dd{topi, topw, od, (int)T, (int)k, (cnr || cn) ? sync : nullptr};
    rc = canon ? launch_decode_stream<true, true>(a, &dd, stream) : launch_decode_stream<true, false>(a, &dd, stream);
    if (rc) return rc;
    if (cnr || cn) {
      rc = cnr ? launch_down_cnr(b, canon, cr, stream) : launch_down_cn(b, canon, cr, nrm != nullptr, stream);
      if (rc != 1) return rc;  // else: no fused instance for this shape
    }
    rc = smaul_moe_down(hdn, act_dtype, down_w8, down_s, yperm, seg_off, tile_off, max_tiles, E, d, h, tile,
                        bm, flags, stream);
    if (rc) return rc;
    return finish_combine(yperm, act_dtype, topi, topw, inv, out, T, d, k, nrm, nr, stream);
  }
  if (routed && T > 64) {  // the dispatch from the given top-k, as smaul_moe_dispatch
    const int64_t nbd = (T + DISPATCH_TPB - 1) / DISPATCH_TPB;  // <= nb: blockcnt/blockoff fit
    hipLaunchKernelGGL(block_count_kernel, dim3((unsigned)nbd), dim3(64), 0, stream, topi, topw, blockcnt, T,
                       (int)E, (int)k, DISPATCH_TPB);
    rc = check_launch("block_count_kernel");
    if (rc) return rc;
    rc = launch_scan_scatter(topi, topw, blockcnt, blockoff, counts, seg_off, tile_off, perm_row, perm_w, inv,
                             T, E, k, bm, DISPATCH_TPB, stream);
    if (rc) return rc;
  } else if ((nb > 1 || routed) && T <= 64) {  // one wave dispatches straight from topi/topw
    hipLaunchKernelGGL(dispatch_small_kernel, dim3(1), dim3(64), 0, stream, topi, topw, od, T, (int)E, (int)k);
    rc = check_launch("dispatch_small_kernel");
    if (rc) return rc;
  } else if (nb > 1) {
    rc = launch_scan_scatter(topi, topw, blockcnt, blockoff, counts, seg_off, tile_off, perm_row, perm_w, inv,
                             T, E, k, bm, route_tpb(T, E, d, act_dtype), stream);
    if (rc) return rc;
  }
  if (f32p_bm) {
    rc = moe_f32_planes((const float*)x, xplanes, perm_row, gate_w8, gate_s, up_w8, up_s, down_w8, down_s,
                        (uint16_t*)hdn, (float*)yperm, seg_off, tile_off, max_tiles, T, d, h, E, bm, flags, stream);
  } else {
    rc = smaul_moe_gate_up(x, act_dtype, perm_row, gate_w8, gate_s, up_w8, up_s, hdn, seg_off, tile_off,
                           max_tiles, E, d, h, tile, bm, flags, stream);
    if (rc) return rc;
    rc = smaul_moe_down(hdn, act_dtype, down_w8, down_s, yperm, seg_off, tile_off, max_tiles, E, d, h, tile,
                        bm, flags, stream);
  }
  if (rc) return rc;
  return finish_combine(yperm, act_dtype, topi, topw, inv, out, T, d, k, nrm, nr, stream);
}

int smaul_moe_forward(const void* x, int act_dtype, const float* gate_w, const float* gate_b,
                      const uint8_t* const* gate_w8, const float* const* gate_s,
                      const uint8_t* const* up_w8, const float* const* up_s,
                      const uint8_t* const* down_w8, const float* const* down_s, void* out,
                      float* prob, int64_t* topi, float* topw, int32_t* counts, void* workspace,
                      int64_t workspace_bytes, int64_t T, int64_t d, int64_t h, int64_t E, int64_t k,
                      int64_t tile, int flags, hipStream_t stream) {
  return moe_forward_impl(x, act_dtype, gate_w, gate_b, gate_w8, gate_s, up_w8, up_s, down_w8, down_s, out, prob,
                          topi, topw, counts, workspace, workspace_bytes, T, d, h, E, k, tile, flags, nullptr,
                          false, nullptr, stream);
}

int smaul_moe_forward_noalloc(const void* x, int act_dtype, const float* gate_w, const float* gate_b,
                              const uint8_t* const* gate_w8, const float* const* gate_s,
                              const uint8_t* const* up_w8, const float* const* up_s,
                              const uint8_t* const* down_w8, const float* const* down_s, void* out,
                              float* prob, int64_t* topi, float* topw, int32_t* counts, int64_t T, int64_t d,
                              int64_t h, int64_t E, int64_t k, int64_t tile, int flags, hipStream_t stream) {
  const int64_t need = smaul_moe_workspace_size(T, d, h, E, k, act_dtype);
  if (need < 0) return fail(SMAUL_ERR_INVALID, "moe_forward_noalloc: bad sizes");
  if (need > (int64_t)SMAUL_NOALLOC_SCRATCH_BYTES)
    return fail(SMAUL_ERR_UNSUPPORTED,
                "moe_forward_noalloc: the layer needs %lld bytes of workspace, more than the %lld-byte static "
                "scratch; use smaul_moe_forward with a workspace",
                (long long)need, (long long)SMAUL_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc) return rc;
  // Nothing in the workspace has to start at zero: every stage writes what
  // the next one reads (counts, offsets, tables, hdn, yperm) in this call.
  return moe_forward_impl(x, act_dtype, gate_w, gate_b, gate_w8, gate_s, up_w8, up_s, down_w8, down_s, out, prob,
                          topi, topw, counts, ws, (int64_t)SMAUL_NOALLOC_SCRATCH_BYTES, T, d, h, E, k, tile, flags,
                          nullptr, false, nullptr, stream);
}

int smaul_moe_forward_norm(const void* x, int act_dtype, const float* gate_w, const float* gate_b,
                           const uint8_t* const* gate_w8, const float* const* gate_s,
                           const uint8_t* const* up_w8, const float* const* up_s,
                           const uint8_t* const* down_w8, const float* const* down_s, void* out,
                           float* prob, int64_t* topi, float* topw, int32_t* counts, void* workspace,
                           int64_t workspace_bytes, int64_t T, int64_t d, int64_t h, int64_t E, int64_t k,
                           int64_t tile, int flags, const float* norm_w, float eps, void* norm_out,
                           hipStream_t stream) {
  if (!(eps > 0.0f) || !std::isfinite(eps)) return fail(SMAUL_ERR_INVALID, "moe_forward_norm: eps must be positive finite");
  if (T > 0 && !norm_out) return fail(SMAUL_ERR_INVALID, "moe_forward_norm: null norm_out");
  const OutNorm nrm{norm_w, eps, norm_out};
  return moe_forward_impl(x, act_dtype, gate_w, gate_b, gate_w8, gate_s, up_w8, up_s, down_w8, down_s, out, prob,
                          topi, topw, counts, workspace, workspace_bytes, T, d, h, E, k, tile, flags, &nrm, false,
                          nullptr, stream);
}

int smaul_moe_forward_chain(const void* x, int act_dtype, const float* gate_w, const float* gate_b,
                            const uint8_t* const* gate_w8, const float* const* gate_s,
                            const uint8_t* const* up_w8, const float* const* up_s,
                            const uint8_t* const* down_w8, const float* const* down_s, void* out,
                            float* prob, int64_t* topi, float* topw, int32_t* counts, void* workspace,
                            int64_t workspace_bytes, int64_t T, int64_t d, int64_t h, int64_t E, int64_t k,
                            int64_t tile, int flags, const float* norm_w, float eps, void* norm_out, int routed,
                            const float* next_gate_w, const float* next_gate_b, int64_t next_E, int64_t next_k,
                            float* next_prob, int64_t* next_topi, float* next_topw, hipStream_t stream) {
  if (!(eps > 0.0f) || !std::isfinite(eps)) return fail(SMAUL_ERR_INVALID, "moe_forward_chain: eps must be positive finite");
  if (T > 0 && !norm_out) return fail(SMAUL_ERR_INVALID, "moe_forward_chain: null norm_out");
  if (T > 0 && routed && (!prob || !topi || !topw))
    return fail(SMAUL_ERR_INVALID, "moe_forward_chain: routed needs prob, topi and topw");
  NextRoute nr{next_gate_w, next_gate_b, next_E, next_k, next_prob, next_topi, next_topw};
  if (next_gate_w) {
    // the next router reads norm_out: same rows, width and dtype as x
    int rc = check_router_args(norm_out, act_dtype, next_gate_w, T, d, next_E, next_k);
    if (rc) return rc;
    if (T > 0 && (!next_prob || !next_topi || !next_topw))
      return fail(SMAUL_ERR_INVALID, "moe_forward_chain: null next-router output");
  }
  const OutNorm nrm{norm_w, eps, norm_out};
  return moe_forward_impl(x, act_dtype, gate_w, gate_b, gate_w8, gate_s, up_w8, up_s, down_w8, down_s, out, prob,
                          topi, topw, counts, workspace, workspace_bytes, T, d, h, E, k, tile, flags, &nrm,
                          routed != 0, next_gate_w ? &nr : nullptr, stream);
}

int smaul_wait_timeouts(int32_t* out, int reset, hipStream_t stream) {
  if (!out) return fail(SMAUL_ERR_INVALID, "wait_timeouts: null out");
  hipLaunchKernelGGL(wait_timeouts_kernel, dim3(1), dim3(1), 0, stream, out, reset);
  return check_launch("wait_timeouts_kernel");
}

int smaul_debug_tail_wait(int extra_arrivals, int spin_limit) {
  if (extra_arrivals < 0 || spin_limit < 1) return fail(SMAUL_ERR_INVALID, "debug_tail_wait: need extra >= 0, limit >= 1");
  g_tail_wait_extra.store(extra_arrivals, std::memory_order_relaxed);
  g_tail_spin_limit.store(spin_limit, std::memory_order_relaxed);
  return SMAUL_OK;
}

int smaul_fp8_canonicalize(const uint8_t* codes, uint8_t* out, int64_t n, hipStream_t stream) {
  if (n < 0) return fail(SMAUL_ERR_INVALID, "canonicalize: n < 0");
  if (n == 0) return SMAUL_OK;
  if (!codes || !out) return fail(SMAUL_ERR_INVALID, "canonicalize: null pointer");
  if (!aligned16(codes) || !aligned16(out)) return fail(SMAUL_ERR_INVALID, "canonicalize: buffers must be 16-byte aligned");
  const int64_t nv = n / 16;
  int64_t blocks = (nv + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(canonicalize_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, codes, out, n);
  return check_launch("canonicalize_kernel");
}

int smaul_fp8_tile_layout(const uint8_t* codes, const float* scales, uint8_t* codes_out, float* scales_out,
                          int64_t N, int64_t K, hipStream_t stream) {
  if (N < 0 || K < 0 || K % 64 != 0) return fail(SMAUL_ERR_INVALID, "tile_layout: need N >= 0 and K a multiple of 64");
  if (N == 0 || K == 0) return SMAUL_OK;
  if (!codes || !scales || !codes_out || !scales_out) return fail(SMAUL_ERR_INVALID, "tile_layout: null pointer");
  if (!aligned16(codes) || !aligned16(codes_out))
    return fail(SMAUL_ERR_INVALID, "tile_layout: code buffers must be 16-byte aligned");
  const int64_t nv = N * K / 16, ns = N * (K / 64);
  // the copy reads other columns than it writes: overlapping buffers would race
  auto overlap = [](const void* a, const void* b, int64_t bytes) {
    const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
    return x < y + (uintptr_t)bytes && y < x + (uintptr_t)bytes;
  };
  if (overlap(codes, codes_out, N * K) || overlap(scales, scales_out, ns * 4))
    return fail(SMAUL_ERR_INVALID, "tile_layout: the output buffers must not overlap the inputs");
  const unsigned bc = (unsigned)std::min<int64_t>(8192, std::max<int64_t>(1, (nv + 255) / 256));
  const unsigned bs = (unsigned)std::min<int64_t>(8192, std::max<int64_t>(1, (ns + 255) / 256));
  hipLaunchKernelGGL(tile_codes_kernel, dim3(bc), dim3(256), 0, stream, codes, codes_out, N, K);
  int rc = check_launch("tile_codes_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(tile_scales_kernel, dim3(bs), dim3(256), 0, stream, scales, scales_out, N, K / 64);
  return check_launch("tile_scales_kernel");
}

int smaul_selftest_topk(const float* vals, int64_t n, int64_t k, int64_t* out_idx) {
  if (!vals || !out_idx || n < 1 || n > MAX_E || k < 1 || k > n)
    return fail(SMAUL_ERR_INVALID, "selftest_topk: need 1<=k<=n<=64");
  smaul_topk::Pair q[MAX_E];
  for (int i = 0; i < n; ++i) q[i] = smaul_topk::Pair{vals[i], i};
  if (k <= 17) smaul_topk::topk_small(q, (int)n, (int)k);  // the router's path
  else smaul_topk::topk(q, (int)n, (int)k);
  for (int i = 0; i < k; ++i) out_idx[i] = q[i].i;
  return SMAUL_OK;
}

}  // extern "C"
