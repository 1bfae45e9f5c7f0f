// attn.hip -- the linear-attention recurrence of SmaulLinear on MI355X (gfx950).
//
// Replaces the reference's native CPU kernels kernel/attn_cpu.cpp
// (attn_forward :144-212, attn_step :421-492, attn_backward :227-368) behind
// the backend entries attn_forward / attn_step / attn_backward
// (kernel/compute.py:265-322).  Per (batch, head):
//   kn_t = k_t / max(||k_t||, 1e-6)          ||k_t|| accumulated in double
//   S_t = S_{t-1} + kn_t (x) v_t,  z_t = z_{t-1} + kn_t
//   num_t = q_t @ S_t,  den_t = max(q_t . z_t, eps),  y_t = num_t / den_t
// Layouts: Q/K/V/Y [B,T,H,D] fp32, DEN [B,T,H], S [B,H,D,D] (row i is the key
// index), z [B,H,D].
//
// The results are bit-identical to the reference kernel: every (b, h) runs
// its T steps in order, each sum runs sequentially over i with a separate
// multiply and add (the library is built with -ffp-contract=off), the key
// norm is a sequential double sum, and the division and square root are
// correctly rounded.  Element (i, j) of S and entry j of num are owned by one
// thread (column j), so the reference's per-element order holds exactly.
//
// Parallelism is over (b, h) tasks, one workgroup each; within a task over
// the D columns of S.  For D <= 128 (every preset of the reference:
// model.py:1020-1085) the task's S lives in registers, one column per
// thread, and a chunk of CH time steps of q/k/v is staged through LDS with
// coalesced loads, the chunk's key norms computed by CH threads in parallel.
// Larger D (the reference accepts D <= 2048) keeps S in global memory: the
// caller's S_out, or a workspace when the state is not wanted.
#include "smaul_common.h"

using smaul::check_launch;
using smaul::fail;

namespace {

// 1 / max(||k||, 1e-6) of one key (attn_cpu.cpp:40-51): the norm summed in
// double in index order, rounded to fp32, clamped, one fp32 reciprocal.
__device__ __forceinline__ float attn_inv_norm(const float* k, int D) {
  double n2 = 0.0;
  for (int i = 0; i < D; ++i) {
    const double ki = (double)k[i];
    n2 = n2 + ki * ki;
  }
  const float n = (float)__builtin_sqrt(n2);
  const float nc = (!__builtin_isfinite(n) || n < 1e-6f) ? 1e-6f : n;
  return 1.0f / nc;
}

constexpr int ATTN_CH = 16;  // time steps staged per chunk (register kernel)

// S in registers: thread j owns column j (S[0..D-1][j]) and z[j].
template <int DMAX>
__global__ void __launch_bounds__(DMAX)
attn_fwd_reg_kernel(const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
                    float* __restrict__ Y, float* __restrict__ DEN, float* __restrict__ S_out,
                    float* __restrict__ z_out, int64_t T, int H, int D, float eps) {
  __shared__ __attribute__((aligned(16))) float s_q[ATTN_CH][DMAX];
  __shared__ __attribute__((aligned(16))) float s_k[ATTN_CH][DMAX];
  __shared__ __attribute__((aligned(16))) float s_v[ATTN_CH][DMAX];
  __shared__ __attribute__((aligned(16))) float s_kn[DMAX];
  __shared__ __attribute__((aligned(16))) float s_z[DMAX];
  __shared__ float s_inv[ATTN_CH];
  const int64_t task = blockIdx.x;
  const int64_t b = task / H, h = task % H;
  const int j = threadIdx.x;
  const bool col = j < D;
  float S[DMAX];
#pragma unroll
  for (int i = 0; i < DMAX; ++i) S[i] = 0.0f;
  float zj = 0.0f;
  const int64_t rs = (int64_t)H * D;          // stride between time steps
  const int64_t base = (b * T * H + h) * D;   // (b, t = 0, h)
  for (int64_t t0 = 0; t0 < T; t0 += ATTN_CH) {
    const int nt = (int)(T - t0 < ATTN_CH ? T - t0 : ATTN_CH);
    // stage the chunk: every thread loads its column of each step
    if (col) {
#pragma unroll
      for (int tt = 0; tt < ATTN_CH; ++tt)
        if (tt < nt) {
          const int64_t o = base + (t0 + tt) * rs + j;
          s_q[tt][j] = Q[o];
          s_k[tt][j] = K[o];
          s_v[tt][j] = V[o];
        }
    }
    __syncthreads();
    if (j < nt) s_inv[j] = attn_inv_norm(s_k[j], D);
    __syncthreads();
    for (int tt = 0; tt < nt; ++tt) {
      float vj = 0.0f;
      if (col) {
        const float knj = s_k[tt][j] * s_inv[tt];
        zj = zj + knj;
        s_kn[j] = knj;
        s_z[j] = zj;
        vj = s_v[tt][j];
      }
      __syncthreads();
      float num = 0.0f, den = 0.0f;
#pragma unroll
      for (int i = 0; i < DMAX; ++i) {
        if (i < D) {
          const float qi = s_q[tt][i];
          S[i] = S[i] + s_kn[i] * vj;
          num = num + qi * S[i];
          den = den + qi * s_z[i];
        }
      }
      const float denc = den < eps ? eps : den;
      const int64_t t = t0 + tt;
      if (col) Y[base + t * rs + j] = num / denc;
      if (DEN && j == 0) DEN[(b * T + t) * H + h] = denc;
      __syncthreads();  // s_kn / s_z are rewritten by the next step
    }
  }
  if (col) {
    if (S_out) {
      float* so = S_out + task * D * D + j;
#pragma unroll
      for (int i = 0; i < DMAX; ++i)
        if (i < D) so[(int64_t)i * D] = S[i];
    }
    if (z_out) z_out[task * D + j] = zj;
  }
}

constexpr int ATTN_GTHREADS = 256;
constexpr int ATTN_DMAX = 2048;  // attn_cpu.cpp:173-174

// One step of a task with S in global memory (Sg = the task's [D][D]) and z
// in LDS: thread j updates the columns it owns (j, j + 256, ...).  q/k/v are
// the step's rows; returns nothing, writes y and (thread 0) den.
__device__ void attn_step_global(float* Sg, float* s_z, float* s_q, float* s_k, float* s_v, float* s_kn,
                                 float* s_inv, const float* q, const float* k, const float* v, float* y,
                                 float* den_out, int D, float eps, float* z_global) {
  const int tid = threadIdx.x;
  for (int i = tid; i < D; i += ATTN_GTHREADS) {
    s_q[i] = q[i];
    s_k[i] = k[i];
    s_v[i] = v[i];
  }
  __syncthreads();
  if (tid == 0) *s_inv = attn_inv_norm(s_k, D);
  __syncthreads();
  const float inv = *s_inv;
  for (int i = tid; i < D; i += ATTN_GTHREADS) {
    const float kn = s_k[i] * inv;
    s_kn[i] = kn;
    const float zi = s_z[i] + kn;
    s_z[i] = zi;
    if (z_global) z_global[i] = zi;
  }
  __syncthreads();
  for (int jj = tid; jj < D; jj += ATTN_GTHREADS) {
    const float vj = s_v[jj];
    float num = 0.0f, den = 0.0f;
    float* col = Sg + jj;
    for (int i = 0; i < D; ++i) {
      const float qi = s_q[i];
      const float sv = col[(int64_t)i * D] + s_kn[i] * vj;
      col[(int64_t)i * D] = sv;
      num = num + qi * sv;
      den = den + qi * s_z[i];
    }
    const float denc = den < eps ? eps : den;
    y[jj] = num / denc;
    if (jj == 0 && den_out) *den_out = denc;
  }
  __syncthreads();  // the LDS rows are rewritten by the next step
}

__global__ void __launch_bounds__(ATTN_GTHREADS)
attn_fwd_global_kernel(const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
                       float* __restrict__ Y, float* __restrict__ DEN, float* __restrict__ S_state,
                       float* __restrict__ z_out, int64_t T, int H, int D, float eps) {
  __shared__ float s_q[ATTN_DMAX], s_k[ATTN_DMAX], s_v[ATTN_DMAX], s_kn[ATTN_DMAX], s_z[ATTN_DMAX];
  __shared__ float s_inv;
  const int64_t task = blockIdx.x;
  const int64_t b = task / H, h = task % H;
  const int tid = threadIdx.x;
  float* Sg = S_state + task * D * D;
  // each thread clears the columns it owns; z starts at zero
  for (int jj = tid; jj < D; jj += ATTN_GTHREADS)
    for (int i = 0; i < D; ++i) Sg[(int64_t)i * D + jj] = 0.0f;
  for (int i = tid; i < D; i += ATTN_GTHREADS) s_z[i] = 0.0f;
  __syncthreads();
  const int64_t rs = (int64_t)H * D;
  const int64_t base = (b * T * H + h) * D;
  for (int64_t t = 0; t < T; ++t) {
    const int64_t o = base + t * rs;
    attn_step_global(Sg, s_z, s_q, s_k, s_v, s_kn, &s_inv, Q + o, K + o, V + o, Y + o,
                     DEN ? DEN + (b * T + t) * H + h : nullptr, D, eps, nullptr);
  }
  if (z_out)
    for (int i = tid; i < D; i += ATTN_GTHREADS) z_out[task * D + i] = s_z[i];
}

__global__ void __launch_bounds__(ATTN_GTHREADS)
attn_step_kernel(float* __restrict__ S, float* __restrict__ z, const float* __restrict__ q,
                 const float* __restrict__ k, const float* __restrict__ v, float* __restrict__ y, int D,
                 float eps) {
  __shared__ float s_q[ATTN_DMAX], s_k[ATTN_DMAX], s_v[ATTN_DMAX], s_kn[ATTN_DMAX], s_z[ATTN_DMAX];
  __shared__ float s_inv;
  const int64_t task = blockIdx.x;
  const int64_t o = task * D;
  for (int i = threadIdx.x; i < D; i += ATTN_GTHREADS) s_z[i] = z[o + i];
  __syncthreads();
  attn_step_global(S + task * D * D, s_z, s_q, s_k, s_v, s_kn, &s_inv, q + o, k + o, v + o, y + o, nullptr, D,
                   eps, z + o);
}

// ---------------------------------------------------------------------------
// backward (attn_cpu.cpp:227-368)
// ---------------------------------------------------------------------------
// Per (b, h) task, two passes over time:
//   A (forward): the recurrence again, then dnum = dy / den, dden = -(dy . y)
//     / den and dq = S dnum + dden z;
//   B (reverse): the adjoints Dm of S and dz of z, Dm += dnum (x) q, dz += dden
//     q, dv = Dm^T kn, dk~ = Dm v + dz, then the key-normalisation backward
//     dk = dk~ / nc - k (k . dk~) / nc^3 (sums in double).
// Bit-identical to the reference kernel: every sum runs in its order.  The
// column sums (num, dv) belong to the thread owning column j and run over i;
// den, (dy . y) and the double sums are sequential, computed by every thread
// that needs them (or thread 0); the row sums (dq, dk~) belong to the thread
// owning row i and run over j the way the reference's 8-lane AVX loop does
// (dot8_lanes).  The state S / Dm is in LDS for D <= 128 (rows padded to D +
// 1 floats, so the row walks of consecutive threads fall in different banks),
// else in the workspace; q/k/v/dy/y are staged CH steps at a time.

// The reference's dot of a row with a vector (attn_cpu.cpp:31-35 and the AVX
// loops feeding hsum8): lane l sums a[j] * b[j] over j = l, l + 8, ... below
// the last multiple of 8, from +0; the lanes are added left to right; the
// remainder follows in order.
__device__ __forceinline__ float dot8_lanes(const float* a, const float* b, int D) {
  float acc[8];
#pragma unroll
  for (int l = 0; l < 8; ++l) acc[l] = 0.0f;
  int j = 0;
  for (; j + 8 <= D; j += 8) {
#pragma unroll
    for (int l = 0; l < 8; ++l) acc[l] = acc[l] + a[j + l] * b[j + l];
  }
  float s = acc[0];
#pragma unroll
  for (int l = 1; l < 8; ++l) s = s + acc[l];
  for (; j < D; ++j) s = s + a[j] * b[j];
  return s;
}

template <int DMAX, int CH, int NT, bool LDS_STATE>
__global__ void __launch_bounds__(NT)
attn_bwd_kernel(const float* __restrict__ dY, const float* __restrict__ Q, const float* __restrict__ K,
                const float* __restrict__ V, const float* __restrict__ Y, const float* __restrict__ DEN,
                float* __restrict__ dQ, float* __restrict__ dK, float* __restrict__ dV, float* __restrict__ state_g,
                int64_t T, int H, int D, float eps) {
  __shared__ float s_state[LDS_STATE ? DMAX * (DMAX + 1) : 1];
  __shared__ float s_q[CH][DMAX], s_k[CH][DMAX], s_v[CH][DMAX], s_dy[CH][DMAX], s_y[CH][DMAX];
  __shared__ float s_kn[DMAX], s_z[DMAX], s_dnum[DMAX], s_t[DMAX];
  __shared__ float s_inv[CH], s_den[CH], s_sc[2];
  const int64_t task = blockIdx.x;
  const int64_t b = task / H, h = task % H;
  const int tid = threadIdx.x;
  float* st = LDS_STATE ? s_state : state_g + task * (int64_t)D * D;
  const int64_t LD = LDS_STATE ? D + 1 : D;
  const int64_t rs = (int64_t)H * D;         // stride between time steps
  const int64_t base = (b * T * H + h) * D;  // (b, t = 0, h)
  auto clear_state = [&]() {
    for (int64_t e = tid; e < (int64_t)D * LD; e += NT) st[e] = 0.0f;
    for (int i = tid; i < D; i += NT) s_z[i] = 0.0f;
  };
  // steps [t0, t0 + nt) of q/k/v/dy (and y, with_y) into the staging rows,
  // their key norms' reciprocals (and DEN) alongside
  auto stage = [&](int64_t t0, int nt, bool with_y) {
    for (int e = tid; e < nt * D; e += NT) {
      const int tt = e / D, j = e - tt * D;
      const int64_t o = base + (t0 + tt) * rs + j;
      s_q[tt][j] = Q[o];
      s_k[tt][j] = K[o];
      s_v[tt][j] = V[o];
      s_dy[tt][j] = dY[o];
      if (with_y) s_y[tt][j] = Y[o];
    }
    __syncthreads();
    for (int tt = tid; tt < nt; tt += NT) {
      s_inv[tt] = attn_inv_norm(s_k[tt], D);
      if (with_y) s_den[tt] = DEN[(b * T + t0 + tt) * H + h];
    }
    __syncthreads();
  };

  // ---- pass A: dQ ----------------------------------------------------------
  clear_state();
  __syncthreads();
  for (int64_t t0 = 0; t0 < T; t0 += CH) {
    const int nt = (int)(T - t0 < CH ? T - t0 : CH);
    stage(t0, nt, false);
    for (int tt = 0; tt < nt; ++tt) {
      const int64_t o = base + (t0 + tt) * rs;
      for (int i = tid; i < D; i += NT) {
        const float kn = s_k[tt][i] * s_inv[tt];
        s_kn[i] = kn;
        s_z[i] = s_z[i] + kn;
      }
      __syncthreads();
      for (int j = tid; j < D; j += NT) {  // column j: S update, num, den
        const float vj = s_v[tt][j];
        float num = 0.0f, den = 0.0f;
        for (int i = 0; i < D; ++i) {
          const float qi = s_q[tt][i];
          const float sv = st[i * LD + j] + s_kn[i] * vj;
          st[i * LD + j] = sv;
          num = num + qi * sv;
          den = den + qi * s_z[i];
        }
        const float denc = den < eps ? eps : den;
        s_t[j] = num / denc;                       // y_j
        s_dnum[j] = s_dy[tt][j] * (1.0f / denc);
        if (j == 0) s_sc[0] = denc;
      }
      __syncthreads();
      const float inv = 1.0f / s_sc[0];
      float yd = 0.0f;
      for (int j = 0; j < D; ++j) yd = yd + s_dy[tt][j] * s_t[j];
      const float dden = -yd * inv;
      for (int i = tid; i < D; i += NT)  // row i: dq
        dQ[o + i] = dot8_lanes(st + i * LD, s_dnum, D) + dden * s_z[i];
      __syncthreads();
    }
  }

  // ---- pass B, reverse in time: dK, dV -----------------------------------
  clear_state();  // Dm and dz
  __syncthreads();
  for (int64_t t1 = T; t1 > 0; t1 -= CH) {
    const int64_t t0 = t1 - CH > 0 ? t1 - CH : 0;
    const int nt = (int)(t1 - t0);
    stage(t0, nt, true);
    for (int tt = nt - 1; tt >= 0; --tt) {
      const int64_t o = base + (t0 + tt) * rs;
      const float invd = 1.0f / s_den[tt];
      for (int i = tid; i < D; i += NT) {
        s_kn[i] = s_k[tt][i] * s_inv[tt];
        s_dnum[i] = s_dy[tt][i] * invd;
      }
      __syncthreads();
      float yd = 0.0f;
      for (int j = 0; j < D; ++j) yd = yd + s_dy[tt][j] * s_y[tt][j];
      const float dden = -yd * invd;
      for (int j = tid; j < D; j += NT) {  // column j: Dm update, dv
        const float dn = s_dnum[j];
        float col = 0.0f;
        for (int i = 0; i < D; ++i) {
          const float dm = st[i * LD + j] + dn * s_q[tt][i];
          st[i * LD + j] = dm;
          col = col + dm * s_kn[i];
        }
        dV[o + j] = col;
      }
      for (int i = tid; i < D; i += NT) s_z[i] = s_z[i] + dden * s_q[tt][i];  // dz
      __syncthreads();
      for (int i = tid; i < D; i += NT) s_t[i] = s_z[i] + dot8_lanes(st + i * LD, s_v[tt], D);  // dk~
      __syncthreads();
      if (tid == 0) {
        double n2 = 0.0, kd = 0.0;
        for (int i = 0; i < D; ++i) {
          const double ki = (double)s_k[tt][i];
          n2 = n2 + ki * ki;
          kd = kd + ki * (double)s_t[i];
        }
        const float n = (float)__builtin_sqrt(n2);
        const float nc = (!__builtin_isfinite(n) || n < 1e-6f) ? 1e-6f : n;
        float sc = (float)(kd / ((double)nc * nc * nc));
        if (!__builtin_isfinite(sc)) sc = 0.0f;
        s_sc[0] = sc;
        s_sc[1] = 1.0f / nc;
      }
      __syncthreads();
      for (int i = tid; i < D; i += NT) dK[o + i] = s_t[i] * s_sc[1] - s_k[tt][i] * s_sc[0];
      __syncthreads();
    }
  }
}

int check_attn_shape(int64_t B, int64_t T, int64_t H, int64_t D, float eps, const char* what) {
  if (B < 0 || T < 0 || H < 0 || D <= 0)
    return fail(SMAUL_ERR_INVALID, "%s: bad shape [%lld,%lld,%lld,%lld]", what, (long long)B, (long long)T,
                (long long)H, (long long)D);
  if (D > ATTN_DMAX)
    return fail(SMAUL_ERR_INVALID, "%s: D=%lld out of the supported range (0, %d]", what, (long long)D, ATTN_DMAX);
  if (!(eps > 0.0f) || !__builtin_isfinite(eps))
    return fail(SMAUL_ERR_INVALID, "%s: eps must be positive finite, got %g", what, (double)eps);
  if (B * H > 2147483647LL) return fail(SMAUL_ERR_UNSUPPORTED, "%s: B*H exceeds the grid", what);
  if (H > 2147483647LL) return fail(SMAUL_ERR_UNSUPPORTED, "%s: H too large", what);
  return SMAUL_OK;
}

}  // namespace

extern "C" {

int64_t smaul_attn_workspace_size(int64_t B, int64_t H, int64_t D, int need_state) {
  if (B < 0 || H < 0 || D <= 0) return -1;
  if (D <= 128 || need_state) return 0;
  return B * H * D * D * (int64_t)sizeof(float);
}

int smaul_attn_forward(const float* Q, const float* K, const float* V, float* Y, float* DEN, float* S_out,
                       float* z_out, int64_t B, int64_t T, int64_t H, int64_t D, float eps, void* workspace,
                       int64_t workspace_bytes, hipStream_t stream) {
  int rc = check_attn_shape(B, T, H, D, eps, "attn_forward");
  if (rc) return rc;
  if ((S_out == nullptr) != (z_out == nullptr))
    return fail(SMAUL_ERR_INVALID, "attn_forward: S_out and z_out go together");
  if (B == 0 || H == 0) return SMAUL_OK;
  if (T > 0 && (!Q || !K || !V || !Y)) return fail(SMAUL_ERR_INVALID, "attn_forward: null pointer");
  const dim3 grid((unsigned)(B * H));
  if (D <= 128) {
    if (T == 0 && !S_out) return SMAUL_OK;  // T == 0 with a state: the kernel writes zeros
    if (D <= 64)
      hipLaunchKernelGGL((attn_fwd_reg_kernel<64>), grid, dim3(64), 0, stream, Q, K, V, Y, DEN, S_out, z_out, T,
                         (int)H, (int)D, eps);
    else
      hipLaunchKernelGGL((attn_fwd_reg_kernel<128>), grid, dim3(128), 0, stream, Q, K, V, Y, DEN, S_out, z_out, T,
                         (int)H, (int)D, eps);
    return check_launch("attn_fwd_reg_kernel");
  }
  float* state = S_out;
  if (!state) {
    const int64_t need = smaul_attn_workspace_size(B, H, D, 0);
    if (workspace_bytes < need || !workspace)
      return fail(SMAUL_ERR_INVALID, "attn_forward: workspace %lld < %lld bytes", (long long)workspace_bytes,
                  (long long)need);
    state = (float*)workspace;
  }
  if (T == 0 && !S_out) return SMAUL_OK;
  hipLaunchKernelGGL(attn_fwd_global_kernel, grid, dim3(ATTN_GTHREADS), 0, stream, Q, K, V, Y, DEN, state, z_out, T,
                     (int)H, (int)D, eps);
  return check_launch("attn_fwd_global_kernel");
}

int smaul_attn_step(float* S, float* z, const float* q, const float* k, const float* v, float* y, int64_t B,
                    int64_t H, int64_t D, float eps, hipStream_t stream) {
  int rc = check_attn_shape(B, 1, H, D, eps, "attn_step");
  if (rc) return rc;
  if (B == 0 || H == 0) return SMAUL_OK;
  if (!S || !z || !q || !k || !v || !y) return fail(SMAUL_ERR_INVALID, "attn_step: null pointer");
  hipLaunchKernelGGL(attn_step_kernel, dim3((unsigned)(B * H)), dim3(ATTN_GTHREADS), 0, stream, S, z, q, k, v, y,
                     (int)D, eps);
  return check_launch("attn_step_kernel");
}

int smaul_attn_backward(const float* dY, const float* Q, const float* K, const float* V, const float* Y,
                        const float* DEN, float* dQ, float* dK, float* dV, int64_t B, int64_t T, int64_t H, int64_t D,
                        float eps, void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  int rc = check_attn_shape(B, T, H, D, eps, "attn_backward");
  if (rc) return rc;
  if (B == 0 || H == 0 || T == 0) return SMAUL_OK;
  if (!dY || !Q || !K || !V || !Y || !DEN || !dQ || !dK || !dV)
    return fail(SMAUL_ERR_INVALID, "attn_backward: null pointer");
  const dim3 grid((unsigned)(B * H));
  if (D <= 64) {
    hipLaunchKernelGGL((attn_bwd_kernel<64, 16, 64, true>), grid, dim3(64), 0, stream, dY, Q, K, V, Y, DEN, dQ, dK,
                       dV, nullptr, T, (int)H, (int)D, eps);
    return check_launch("attn_bwd_kernel");
  }
  if (D <= 128) {
    hipLaunchKernelGGL((attn_bwd_kernel<128, 16, 128, true>), grid, dim3(128), 0, stream, dY, Q, K, V, Y, DEN, dQ,
                       dK, dV, nullptr, T, (int)H, (int)D, eps);
    return check_launch("attn_bwd_kernel");
  }
  const int64_t need = smaul_attn_workspace_size(B, H, D, 0);
  if (workspace_bytes < need || !workspace)
    return fail(SMAUL_ERR_INVALID, "attn_backward: workspace %lld < %lld bytes", (long long)workspace_bytes,
                (long long)need);
  hipLaunchKernelGGL((attn_bwd_kernel<ATTN_DMAX, 1, ATTN_GTHREADS, false>), grid, dim3(ATTN_GTHREADS), 0, stream, dY,
                     Q, K, V, Y, DEN, dQ, dK, dV, (float*)workspace, T, (int)H, (int)D, eps);
  return check_launch("attn_bwd_kernel");
}

}  // extern "C"
