// Block-quantization helpers shared by the rowwise and dual-layout
// BF16 -> MXFP4 kernels. The rule they implement is the reference's
// (code/kernel/per_token_quant_mxfp4.cu:151-254); see quant.hip for the
// derivation of the fast path.
#pragma once
#include <cstring>
#include "omo_device.cuh"

namespace omo_hip {

// Reference scale rule from an fp32 amax (already max'ed with eps).
// Returns the E8M0 byte; *inv receives 1/y_s.
__device__ __forceinline__ uint32_t ref_scale(float amax, float fp4_max, float* inv) {
  float z = fmaxf(amax / fp4_max, 1e-10f);
  if (z == __builtin_inff()) { *inv = 0.0f; return 126u; }
  int c = ceil_log2_normal(z);
  if (c >= 128) { *inv = 0.0f; return 126u; }  // exp2f(128) overflows: y_s = inf
  // 1/2^c is exact; c == 127 gives the binary32 subnormal 2^-127.
  *inv = (c <= 126) ? exp2i(-c) : __uint_as_float(0x00400000u);
  return (uint32_t)(c + 127) & 0xFFu;
}

// fmaxf(m, |x|) for the bf16 pattern x, skipping every NaN pattern. The
// reference's CUDA fmaxf drops NaN operands, signalling ones included; the
// hardware max in IEEE mode returns a quiet NaN for a signalling operand,
// which would restart a running maximum after an sNaN input.
__device__ __forceinline__ float fmax_abs_bf16(float m, uint32_t x) {
  const uint32_t a = x & 0x7FFFu;
  return a <= 0x7F80u ? fmaxf(m, bf16_to_f32(a)) : m;
}

// Emulation of the reference for one chunk of a quad. All four lanes of the
// quad must call it together (DPP reduction).
__device__ __forceinline__ void quant_chunk_ref(const u32x4& d, float eps, float fp4_min, float fp4_max,
                                                uint32_t* codes, uint32_t* byte) {
  const uint32_t w[4] = {d[0], d[1], d[2], d[3]};
  float amax = eps;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    amax = fmax_abs_bf16(amax, w[k]);
    amax = fmax_abs_bf16(amax, w[k] >> 16);
  }
  amax = quad_fmax(amax);
  float inv;
  *byte = ref_scale(amax, fp4_max, &inv);
  uint32_t out = 0;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    float qx = fminf(fmaxf(bf16_to_f32(w[k] & 0xFFFFu) * inv, fp4_min), fp4_max);
    float qy = fminf(fmaxf(bf16_to_f32(w[k] >> 16) * inv, fp4_min), fp4_max);
    out |= (e2m1_from_f32_ref(qx) | (e2m1_from_f32_ref(qy) << 4)) << (8 * k);
  }
  *codes = out;
}

// Scale of a block whose max |x| bf16 pattern is amax_bits (< 0x7F80):
// returns y_s = 2^c and sets *byte = c + 127. For amax = (1 + f/128) 2^E,
// ceil(log2(amax / 6)) = E - 2 + (f > 64) = ((amax_bits + 63) >> 7) - 129, f > 64
// being the carry of f + 63 into the exponent field. The reference takes the
// scale of fmaxf(eps, amax) and the scale is monotone in its argument, so c
// is max(that, c_eps), where c_eps >= -33 already holds the 1e-10 floor:
// c + 127 = max(((amax_bits + 63) >> 7) - 2, c_eps + 127), and the subtraction
// inside the shift ((amax_bits - 193) >> 7, arithmetic) only differs below
// amax_bits = 193, where the maximum takes c_eps + 127 either way.
__device__ __forceinline__ float fast_block_scale(uint32_t amax_bits, int c_eps, uint32_t* byte) {
  const int b = max((int)(amax_bits - 193u) >> 7, c_eps + 127);
  *byte = (uint32_t)b;
  return __uint_as_float((uint32_t)b << 23);
}

// Fast path for one chunk: returns the 4 code bytes; *byte gets the scale.
// amax_bits is the quad-wide max of |x| bit patterns, < 0x7F80. The four
// conversions write the four bytes of r, so its initial value is unused.
__device__ __forceinline__ uint32_t quant_chunk_fast(const u32x4& d, uint32_t amax_bits, int c_eps, uint32_t* byte) {
  const float y_s = fast_block_scale(amax_bits, c_eps, byte);
  uint32_t r = d[0];
  r = cvt_pk_fp4<0>(r, d[0], y_s);
  r = cvt_pk_fp4<1>(r, d[1], y_s);
  r = cvt_pk_fp4<2>(r, d[2], y_s);
  r = cvt_pk_fp4<3>(r, d[3], y_s);
  return r;
}

__device__ __forceinline__ uint32_t chunk_absmax_bits(const u32x4& d) {
  uint32_t m = pk_max_u16(pk_max_u16(d[0] & 0x7FFF7FFFu, d[1] & 0x7FFF7FFFu),
                          pk_max_u16(d[2] & 0x7FFF7FFFu, d[3] & 0x7FFF7FFFu));
  return max(m & 0xFFFFu, m >> 16);
}

// Host-side scale exponent for amax == eps (exact
// ceil(log2(max(fl(eps/fp4_max), 1e-10f)))).
static inline int host_c_eps(float eps, float fp4_max) {
  float y = eps / fp4_max;
  float z = y > 1e-10f ? y : 1e-10f;
  uint32_t b;
  memcpy(&b, &z, 4);
  return (int)((b >> 23) & 0xFFu) - 127 + ((b & 0x7FFFFFu) != 0u);
}

}  // namespace omo_hip
