/*
 * CPU oracle: restatement of the reference tiled-E4M3 forward GEMM.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the HIP kernels are
 * compared against; it is never part of the shipped product path.  Only
 * tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg load it.
 *
 * Follows /root/reference/kernel/fp8_cpu.cpp:
 *   - codebook            fp8_cpu.cpp:16-26  (0x7F/0xFF decode to +-448)
 *   - task grid           fp8_cpu.cpp:130-139 (MR=32 rows x OB=64 outputs)
 *   - per-task loop       fp8_cpu.cpp:49-98
 * The reference has two arithmetic orders inside one task, and both are
 * reproduced here because they round differently:
 *   - the "fast" K-block (task is exactly 32 rows x 64 outputs and the K block
 *     is a whole 64): weight = lut*s rounded to fp32 first, then
 *     acc = acc + x*weight                                   (fp8_cpu.cpp:66,77)
 *   - every other K block: acc = acc + (x*lut)*s              (fp8_cpu.cpp:90)
 * Accumulation is sequential in k with no fused multiply-add; this file must be
 * compiled with -ffp-contract=off (oracle/Makefile), exactly like the reference
 * (kernel/compute.py:40-46).  Neither gcc's auto-vectorisation nor the
 * threading below changes any result: every output is owned by one task and
 * summed in the same order.
 */
#include <stdint.h>
#include <string.h>
#include <math.h>

static float g_lut[256];
static int g_lut_ready = 0;

/* fp8_cpu.cpp:16-26 / fp8_tile.py:39-48: e=(c>>3)&15, m=c&7. */
static void build_lut(void) {
  for (int c = 0; c < 256; ++c) {
    int e = (c >> 3) & 15, m = c & 7;
    float s = (c & 128) ? -1.0f : 1.0f;
    float v;
    if (e == 15 && m == 7) v = s * 448.0f;
    else if (e == 0) v = s * ldexpf((float)m, -9);
    else v = s * (1.0f + (float)m / 8.0f) * ldexpf(1.0f, e - 7);
    g_lut[c] = v;
  }
  g_lut_ready = 1;
}

void oracle_e4m3_lut(float* out256) {
  if (!g_lut_ready) build_lut();
  memcpy(out256, g_lut, sizeof(g_lut));
}

/* One reference task: rows [r0, r0+MR), outputs [ob0, ob0+OBR). */
static void forward_task(const float* xp, const uint8_t* wp, const float* sp, float* yp,
                         int64_t in_f, int64_t out_f, int64_t nt, int64_t tile,
                         int64_t r0, int64_t MR, int64_t ob0, int64_t OBR) {
  float acc[32][64];
  float wt[64][64];
  for (int64_t r = 0; r < MR; ++r)
    for (int64_t o = 0; o < OBR; ++o) acc[r][o] = 0.0f;
  for (int64_t kt = 0; kt < in_f; kt += 64) {
    const int64_t Kr = (in_f - kt) < 64 ? (in_f - kt) : 64;
    if (MR == 32 && OBR == 64 && Kr == 64) {
      for (int64_t k2 = 0; k2 < 64; ++k2) {
        const int64_t st = (kt + k2) / tile;
        for (int64_t o2 = 0; o2 < 64; ++o2) {
          const int64_t o = ob0 + o2;
          wt[k2][o2] = g_lut[wp[o * in_f + kt + k2]] * sp[o * nt + st];
        }
      }
      for (int64_t r = 0; r < 32; ++r) {
        const float* xr = xp + (r0 + r) * in_f + kt;
        for (int64_t k2 = 0; k2 < 64; ++k2) {
          const float xv = xr[k2];
          for (int64_t o2 = 0; o2 < 64; ++o2) {
            const float p = xv * wt[k2][o2];
            acc[r][o2] = acc[r][o2] + p;
          }
        }
      }
    } else {
      for (int64_t r = 0; r < MR; ++r) {
        const float* xr = xp + (r0 + r) * in_f + kt;
        for (int64_t k2 = 0; k2 < Kr; ++k2) {
          const float xv = xr[k2];
          const int64_t st = (kt + k2) / tile;
          for (int64_t o2 = 0; o2 < OBR; ++o2) {
            const int64_t o = ob0 + o2;
            const float p = (xv * g_lut[wp[o * in_f + kt + k2]]) * sp[o * nt + st];
            acc[r][o2] = acc[r][o2] + p;
          }
        }
      }
    }
  }
  for (int64_t r = 0; r < MR; ++r)
    for (int64_t o = 0; o < OBR; ++o) yp[(r0 + r) * out_f + ob0 + o] = acc[r][o];
}

/* fp8_cpu.cpp:100-141: y[rows, out_f] = x[rows, in_f] . decode(w, s)^T.
 * Returns 0, or -1 on a non-positive tile / negative size. */
int oracle_fp8_forward(const float* x, const uint8_t* w, const float* s, float* y,
                       int64_t rows, int64_t in_f, int64_t out_f, int64_t tile,
                       int nthreads) {
  if (tile <= 0 || in_f < 0 || out_f < 0 || rows < 0) return -1;
  if (!g_lut_ready) build_lut();
  const int64_t nt = (in_f + tile - 1) / tile;
  const int64_t MR = 32, OB = 64;
  const int64_t nmb = (rows + MR - 1) / MR, nob = (out_f + OB - 1) / OB;
  const int64_t ntask = nmb * nob;
  (void)nthreads;
#pragma omp parallel for schedule(dynamic, 4) num_threads(nthreads > 0 ? nthreads : 1)
  for (int64_t task = 0; task < ntask; ++task) {
    const int64_t mb = task / nob, ob = task % nob;
    const int64_t mr = (rows - mb * MR) < MR ? (rows - mb * MR) : MR;
    const int64_t obr = (out_f - ob * OB) < OB ? (out_f - ob * OB) : OB;
    forward_task(x, w, s, y, in_f, out_f, nt, tile, mb * MR, mr, ob * OB, obr);
  }
  return 0;
}

/*
 * Backward-input, fp8_cpu.cpp:167-259: dx[r, i] = sum_o g[r, o] * W[o, i].
 * Tasks of RB=16 rows x IB=8 input columns; the output dimension runs in
 * blocks of 64.  A block takes the "fast" order (fp8_cpu.cpp:182-206) when the
 * task is exactly 16 x 8 and the block a whole 64: w = lut*s rounded first,
 * eight accumulators a0..a7 (a0 continuing the running total, the others from
 * zero), a_j += g[o]*w[o] for o = j (mod 8), then ((a0+a1)+(a2+a3)) +
 * ((a4+a5)+(a6+a7)).  Every other block (fp8_cpu.cpp:208-214) adds
 * (g*lut)*s to the running total in o order.
 */
static void backward_task(const float* gp, const uint8_t* wp, const float* sp, float* dxp, int64_t in_f,
                          int64_t out_f, int64_t nt, int64_t tile, int64_t r0, int64_t RB, int64_t ib0,
                          int64_t IBR) {
  float acc[16][8];
  float wsub[64][8];
  for (int64_t r = 0; r < RB; ++r)
    for (int64_t k = 0; k < IBR; ++k) acc[r][k] = 0.0f;
  for (int64_t ob = 0; ob < out_f; ob += 64) {
    const int64_t OBR = (out_f - ob) < 64 ? (out_f - ob) : 64;
    if (RB == 16 && IBR == 8 && OBR == 64) {
      for (int64_t o2 = 0; o2 < 64; ++o2)
        for (int64_t k2 = 0; k2 < 8; ++k2) {
          const int64_t o = ob + o2, i = ib0 + k2;
          wsub[o2][k2] = g_lut[wp[o * in_f + i]] * sp[o * nt + i / tile];
        }
      for (int64_t r = 0; r < 16; ++r) {
        const float* gr = gp + (r0 + r) * out_f + ob;
        for (int64_t k2 = 0; k2 < 8; ++k2) {
          float a[8];
          a[0] = acc[r][k2];
          for (int j = 1; j < 8; ++j) a[j] = 0.0f;
          for (int64_t o2 = 0; o2 < 64; o2 += 8)
            for (int j = 0; j < 8; ++j) a[j] = a[j] + gr[o2 + j] * wsub[o2 + j][k2];
          acc[r][k2] = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
        }
      }
    } else {
      for (int64_t o2 = 0; o2 < OBR; ++o2) {
        const int64_t o = ob + o2;
        for (int64_t r = 0; r < RB; ++r) {
          const float gv = gp[(r0 + r) * out_f + o];
          for (int64_t k2 = 0; k2 < IBR; ++k2) {
            const int64_t i = ib0 + k2;
            acc[r][k2] = acc[r][k2] + gv * g_lut[wp[o * in_f + i]] * sp[o * nt + i / tile];
          }
        }
      }
    }
  }
  for (int64_t r = 0; r < RB; ++r)
    for (int64_t k = 0; k < IBR; ++k) dxp[(r0 + r) * in_f + ib0 + k] = acc[r][k];
}

int oracle_fp8_backward_input(const float* g, const uint8_t* w, const float* s, float* dx, int64_t rows,
                              int64_t in_f, int64_t out_f, int64_t tile, int threads) {
  if (tile <= 0 || in_f < 0 || out_f < 0 || rows < 0) return 1;
  if (!g_lut_ready) build_lut();
  const int64_t nt = (in_f + tile - 1) / tile;
  const int64_t nrb = (rows + 15) / 16, nib = (in_f + 7) / 8;
#pragma omp parallel for schedule(dynamic, 4) num_threads(threads > 0 ? threads : 1)
  for (int64_t task = 0; task < nrb * nib; ++task) {
    const int64_t rb = task / nib, ib = task % nib;
    const int64_t RB = (rows - rb * 16) < 16 ? (rows - rb * 16) : 16;
    const int64_t IBR = (in_f - ib * 8) < 8 ? (in_f - ib * 8) : 8;
    backward_task(g, w, s, dx, in_f, out_f, nt, tile, rb * 16, RB, ib * 8, IBR);
  }
  return 0;
}
