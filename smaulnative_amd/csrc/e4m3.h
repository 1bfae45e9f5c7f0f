// e4m3.h -- bf16 vector types and the exact E4M3 -> bf16 decode shared by the
// kernels of libsmaul_rocm.so (gfx950).
#ifndef SMAUL_E4M3_H
#define SMAUL_E4M3_H

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf2f(uint32_t b) { return __uint_as_float(b << 16); }

// two fp32 -> two bf16 (low half a), v_cvt_pk_bf16_f32: round to nearest even
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  const bf16x2_t v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}

// The reference codebook decodes 0x7F/0xFF to +-448 where OCP E4M3FN has NaN;
// every other code is identical.  Rewrite those two codes to 0x7E/0xFE (also
// +-448) so the hardware OCP conversion is exact for all 256 codes.
__device__ __forceinline__ uint32_t canon4(uint32_t w) {
  const uint32_t t = w & 0x7f7f7f7fu;
  const uint32_t m = (t + 0x01010101u) & 0x80808080u;  // bit 7 set where t == 0x7f
  return w - (m >> 7);
}

// 4 E4M3 codes (bytes 0..3 of w) -> 4 bf16 packed in two dwords, exact.
// CANON: the codes are already canonical (no 0x7F/0xFF bytes).
template <bool CANON>
__device__ __forceinline__ void decode4(uint32_t w, uint32_t& lo, uint32_t& hi) {
  if constexpr (!CANON) w = canon4(w);
  bf16x2_t a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false);
  bf16x2_t b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true);
  lo = __builtin_bit_cast(uint32_t, a);
  hi = __builtin_bit_cast(uint32_t, b);
}

}  // namespace

#endif  // SMAUL_E4M3_H
