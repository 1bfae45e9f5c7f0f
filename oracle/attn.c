/*
 * CPU oracle: restatement of the reference linear-attention recurrence.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the HIP kernels are
 * compared against; it is never part of the shipped product path.
 *
 * Follows /root/reference/kernel/attn_cpu.cpp:
 *   - recurrence          attn_cpu.cpp:16-24
 *       kn_t = k_t / max(||k_t||, 1e-6)        (norm accumulated in double)
 *       S_t = S_{t-1} + kn_t (x) v_t,  z_t = z_{t-1} + kn_t
 *       num_t = q_t @ S_t,  den_t = max(q_t . z_t, eps),  y_t = num_t / den_t
 *   - normalize_key       attn_cpu.cpp:40-51
 *   - forward task        attn_cpu.cpp:53-98 (and the state variant :103-142)
 *   - decode step         attn_cpu.cpp:421-492
 *   - backward            attn_cpu.cpp:227-368 (pass A forward in time for dQ,
 *                         pass B reverse in time for dK/dV, then the
 *                         key-normalisation backward)
 * Layouts: Q/K/V/Y [B,T,H,D], DEN [B,T,H], S [B,H,D,D] (row i = key index),
 * z [B,H,D].  Every sum is sequential in i with separate multiply and add
 * (this file is built with -ffp-contract=off, like the reference), so the
 * reference's AVX lanes and scalar remainder give the same bits as this loop:
 * each element is a plain mul then add in the same order.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static int64_t qkv_off(int64_t b, int64_t t, int64_t h, int64_t T, int64_t H, int64_t D) {
  return ((b * T + t) * H + h) * D;
}

/* attn_cpu.cpp:40-51: norm in double, clamp, one fp32 reciprocal. */
static void normalize_key(const float* k, float* kn, int64_t D) {
  double n2 = 0.0;
  for (int64_t i = 0; i < D; ++i) n2 += (double)k[i] * (double)k[i];
  const float n = (float)sqrt(n2);
  const float nc = (!isfinite(n) || n < 1e-6f) ? 1e-6f : n;
  const float inv = 1.0f / nc;
  for (int64_t i = 0; i < D; ++i) kn[i] = k[i] * inv;
}

/* One recurrence step on state (S, z); writes y[D], returns den. */
static float step(float* S, float* z, const float* q, const float* k, const float* v, float* y, float* kn,
                  float* num, int64_t D, float eps) {
  normalize_key(k, kn, D);
  for (int64_t i = 0; i < D; ++i) {
    const float ki = kn[i];
    z[i] += ki;
    float* Sr = S + i * D;
    for (int64_t j = 0; j < D; ++j) Sr[j] = Sr[j] + ki * v[j];
  }
  float den = 0.0f;
  for (int64_t j = 0; j < D; ++j) num[j] = 0.0f;
  for (int64_t i = 0; i < D; ++i) {
    const float qi = q[i];
    const float* Sr = S + i * D;
    for (int64_t j = 0; j < D; ++j) num[j] = num[j] + qi * Sr[j];
    den += qi * z[i];
  }
  const float denc = den < eps ? eps : den;
  for (int64_t j = 0; j < D; ++j) y[j] = num[j] / denc;
  return denc;
}

/* attn_forward (attn_cpu.cpp:144-212): DEN, S_out, z_out may be NULL. */
int oracle_attn_forward(const float* Q, const float* K, const float* V, float* Y, float* DEN, float* S_out,
                        float* z_out, int64_t B, int64_t T, int64_t H, int64_t D, float eps) {
  if (B < 0 || T < 0 || H < 0 || D <= 0) return 1;
  float* S = (float*)malloc(sizeof(float) * (size_t)(D * D + 3 * D));
  if (!S) return 2;
  float* z = S + D * D;
  float* kn = z + D;
  float* num = kn + D;
  for (int64_t b = 0; b < B; ++b)
    for (int64_t h = 0; h < H; ++h) {
      memset(S, 0, sizeof(float) * (size_t)(D * D + D));
      for (int64_t t = 0; t < T; ++t) {
        const int64_t o = qkv_off(b, t, h, T, H, D);
        const float denc = step(S, z, Q + o, K + o, V + o, Y + o, kn, num, D, eps);
        if (DEN) DEN[(b * T + t) * H + h] = denc;
      }
      if (S_out) memcpy(S_out + (b * H + h) * D * D, S, sizeof(float) * (size_t)(D * D));
      if (z_out) memcpy(z_out + (b * H + h) * D, z, sizeof(float) * (size_t)D);
    }
  free(S);
  return 0;
}

/* attn_step (attn_cpu.cpp:421-492): S [B,H,D,D] and z [B,H,D] advanced in place. */
int oracle_attn_step(float* S, float* z, const float* q, const float* k, const float* v, float* y, int64_t B,
                     int64_t H, int64_t D, float eps) {
  if (B < 0 || H < 0 || D <= 0) return 1;
  float* kn = (float*)malloc(sizeof(float) * (size_t)(2 * D));
  if (!kn) return 2;
  float* num = kn + D;
  for (int64_t task = 0; task < B * H; ++task)
    step(S + task * D * D, z + task * D, q + task * D, k + task * D, v + task * D, y + task * D, kn, num, D, eps);
  free(kn);
  return 0;
}

/* The reference's 8-lane dot product (attn_cpu.cpp:31-35 hsum8 and the AVX
 * loops that feed it): lane l sums a[j] * b[j] over j = l, l + 8, ... below
 * the last multiple of 8, from +0, one rounded product then one add each; the
 * lanes are added left to right; the scalar remainder follows in order. */
static float dot8(const float* a, const float* b, int64_t D) {
  float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  int64_t j = 0;
  for (; j + 8 <= D; j += 8)
    for (int l = 0; l < 8; ++l) acc[l] = acc[l] + a[j + l] * b[j + l];
  float s = acc[0] + acc[1] + acc[2] + acc[3] + acc[4] + acc[5] + acc[6] + acc[7];
  for (; j < D; ++j) s += a[j] * b[j];
  return s;
}

/* attn_backward (attn_cpu.cpp:227-368): dQ, dK, dV [B,T,H,D] from dY, Q, K
 * (raw), V, the forward's Y and DEN. */
int oracle_attn_backward(const float* dY, const float* Q, const float* K, const float* V, const float* Y,
                         const float* DEN, float* dQ, float* dK, float* dV, int64_t B, int64_t T, int64_t H,
                         int64_t D, float eps) {
  if (B < 0 || T < 0 || H < 0 || D <= 0) return 1;
  float* S = (float*)malloc(sizeof(float) * (size_t)(D * D + 5 * D));
  if (!S) return 2;
  float* z = S + D * D;
  float* kn = z + D;
  float* num = kn + D;
  float* dnum = num + D;
  float* col = dnum + D;
  for (int64_t b = 0; b < B; ++b)
    for (int64_t h = 0; h < H; ++h) {
      /* pass A (:227-292): the forward again, and dq = S dnum + dden z */
      memset(S, 0, sizeof(float) * (size_t)(D * D + D));
      for (int64_t t = 0; t < T; ++t) {
        const int64_t o = qkv_off(b, t, h, T, H, D);
        const float *qt = Q + o, *vt = V + o, *dyt = dY + o;
        normalize_key(K + o, kn, D);
        for (int64_t i = 0; i < D; ++i) {
          z[i] += kn[i];
          float* Sr = S + i * D;
          for (int64_t j = 0; j < D; ++j) Sr[j] = Sr[j] + kn[i] * vt[j];
        }
        float den = 0.0f;
        for (int64_t j = 0; j < D; ++j) num[j] = 0.0f;
        for (int64_t i = 0; i < D; ++i) {
          const float* Sr = S + i * D;
          for (int64_t j = 0; j < D; ++j) num[j] = num[j] + qt[i] * Sr[j];
          den += qt[i] * z[i];
        }
        const float denc = den < eps ? eps : den;
        const float inv = 1.0f / denc;
        float yd = 0.0f;
        for (int64_t j = 0; j < D; ++j) {
          const float yj = num[j] / denc;
          dnum[j] = dyt[j] * inv;
          yd += dyt[j] * yj;
        }
        const float dden = -yd * inv;
        for (int64_t i = 0; i < D; ++i) dQ[o + i] = dot8(S + i * D, dnum, D) + dden * z[i];
      }
      /* pass B (:294-368), reverse in time: Dm, dz are the adjoints of S, z */
      float* Dm = S;
      float* dz = z;
      memset(Dm, 0, sizeof(float) * (size_t)(D * D + D));
      for (int64_t t = T - 1; t >= 0; --t) {
        const int64_t o = qkv_off(b, t, h, T, H, D);
        const float *qt = Q + o, *kt = K + o, *vt = V + o, *dyt = dY + o, *yt = Y + o;
        float *dkt = dK + o, *dvt = dV + o;
        normalize_key(kt, kn, D);
        const float inv = 1.0f / DEN[(b * T + t) * H + h];
        float yd = 0.0f;
        for (int64_t j = 0; j < D; ++j) {
          dnum[j] = dyt[j] * inv;
          yd += dyt[j] * yt[j];
        }
        const float dden = -yd * inv;
        for (int64_t i = 0; i < D; ++i) {
          float* Dr = Dm + i * D;
          for (int64_t j = 0; j < D; ++j) Dr[j] = Dr[j] + dnum[j] * qt[i];
          dz[i] += dden * qt[i];
        }
        for (int64_t j = 0; j < D; ++j) col[j] = 0.0f;
        for (int64_t i = 0; i < D; ++i) {
          const float* Dr = Dm + i * D;
          for (int64_t j = 0; j < D; ++j) col[j] = col[j] + Dr[j] * kn[i];
          dkt[i] = dz[i] + dot8(Dr, vt, D);
        }
        for (int64_t j = 0; j < D; ++j) dvt[j] = col[j];
        /* k / max(||k||, 1e-6) backward (:355-367), sums in double */
        double n2 = 0.0, kd = 0.0;
        for (int64_t i = 0; i < D; ++i) {
          n2 += (double)kt[i] * (double)kt[i];
          kd += (double)kt[i] * (double)dkt[i];
        }
        const float n = (float)sqrt(n2);
        const float nc = (!isfinite(n) || n < 1e-6f) ? 1e-6f : n;
        float sc = (float)(kd / ((double)nc * nc * nc));
        if (!isfinite(sc)) sc = 0.0f;
        const float invn = 1.0f / nc;
        for (int64_t i = 0; i < D; ++i) dkt[i] = dkt[i] * invn - kt[i] * sc;
      }
    }
  free(S);
  return 0;
}
