// Device-side helpers shared by the MXFP4 kernels (gfx950 / CDNA4 only).
//
// Bit-level conventions used throughout:
//   * bf16 values travel as their 16-bit patterns; two of them share a dword,
//     element 2j in the low half, element 2j+1 in the high half.
//   * an MXFP4 code byte holds element 2j in its low nibble and 2j+1 in its
//     high nibble (code/kernel/per_token_quant_mxfp4.cu:256-262).
//   * an E8M0 scale byte s stands for 2^(s-127).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace omo_hip {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// gfx950 scaled FP4 converts, written as (non-volatile) inline asm.
// ROCm 7.2's lowering of __builtin_amdgcn_cvt_scalef32_pk_fp4_bf16 feeds
// element 0 of a u32x4 to the converts that name elements 1..3, and the
// bf16x2 results of __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4 get their
// halves mis-assigned; the asm form is opaque to that lowering and still
// schedules freely. op_sel selects the byte of the 32-bit destination
// (pk_fp4_bf16) or of the source (pk_bf16_fp4).
//
// cvt_pk_fp4<B>(old, src, scale): byte B of `old` = the two E2M1 nibbles of
// the bf16 pair `src` (element 0 in the low nibble) divided by `scale`,
// round-to-nearest-even, saturating at +-6.
template <int B>
__device__ __forceinline__ uint32_t cvt_pk_fp4(uint32_t old, uint32_t src, float scale) {
  if constexpr (B == 0) asm("v_cvt_scalef32_pk_fp4_bf16 %0, %1, %2" : "+v"(old) : "v"(src), "v"(scale));
  else if constexpr (B == 1) asm("v_cvt_scalef32_pk_fp4_bf16 %0, %1, %2 op_sel:[0,0,1,0]" : "+v"(old) : "v"(src), "v"(scale));
  else if constexpr (B == 2) asm("v_cvt_scalef32_pk_fp4_bf16 %0, %1, %2 op_sel:[0,0,0,1]" : "+v"(old) : "v"(src), "v"(scale));
  else asm("v_cvt_scalef32_pk_fp4_bf16 %0, %1, %2 op_sel:[0,0,1,1]" : "+v"(old) : "v"(src), "v"(scale));
  return old;
}

// cvt_pk_bf16_fp4<B>(src, scale): the two E2M1 nibbles of byte B of `src`
// times `scale`, as a bf16 pair (low nibble in the low half).
template <int B>
__device__ __forceinline__ uint32_t cvt_pk_bf16_fp4(uint32_t src, float scale) {
  uint32_t r;
  if constexpr (B == 0) asm("v_cvt_scalef32_pk_bf16_fp4 %0, %1, %2" : "=v"(r) : "v"(src), "v"(scale));
  else if constexpr (B == 1) asm("v_cvt_scalef32_pk_bf16_fp4 %0, %1, %2 op_sel:[1,0,0]" : "=v"(r) : "v"(src), "v"(scale));
  else if constexpr (B == 2) asm("v_cvt_scalef32_pk_bf16_fp4 %0, %1, %2 op_sel:[0,1,0]" : "=v"(r) : "v"(src), "v"(scale));
  else asm("v_cvt_scalef32_pk_bf16_fp4 %0, %1, %2 op_sel:[1,1,0]" : "=v"(r) : "v"(src), "v"(scale));
  return r;
}

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// Packed unsigned 16-bit max of both halves (v_pk_max_u16).
__device__ __forceinline__ uint32_t pk_max_u16(uint32_t a, uint32_t b) {
  u16x2_t r = __builtin_elementwise_max(__builtin_bit_cast(u16x2_t, a), __builtin_bit_cast(u16x2_t, b));
  return __builtin_bit_cast(uint32_t, r);
}

// DPP quad permutations: every lane reads the value of lane (quad base + sel[i]).
// quad_perm encodings: [1,0,3,2] = 0xB1, [2,3,0,1] = 0x4E.
__device__ __forceinline__ uint32_t dpp_quad_xor1(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);
}
__device__ __forceinline__ uint32_t dpp_quad_xor2(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);
}

// Maximum over the 4 lanes of a quad (all 4 lanes must be active). With every
// source lane active, bound_ctrl changes nothing; set, it lets each step fold
// into one v_max_u32 with a DPP operand.
__device__ __forceinline__ uint32_t quad_max_u32(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, true));
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, true));
  return v;
}
__device__ __forceinline__ float quad_fmax(float v) {
  v = fmaxf(v, __uint_as_float(dpp_quad_xor1(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(dpp_quad_xor2(__float_as_uint(v))));
  return v;
}

// E2M1 nibble -> bf16 bits, the reference decode
// (code/kernel/per_token_Mxfp4ToBf16_dequant.cu:137-150): em<<6 | sign<<15,
// +126<<7 when the exponent bits are non-zero, code 1 -> 0.5 (0x3F00).
__device__ __forceinline__ uint32_t e2m1_to_bf16_bits(uint32_t nib) {
  uint32_t em = nib & 7u;
  uint32_t x = (em << 6) | ((nib & 8u) << 12);
  x += (em & 6u) ? (126u << 7) : 0u;
  x = (em == 1u) ? (16128u | (x & 0x8000u)) : x;
  return x;
}

// float -> E2M1 nibble by the reference's integer round-to-nearest-even path
// (code/kernel/per_token_quant_mxfp4.cu:103-112, 213-254). The shift in the
// denormal adjustment reaches >= 32 for exponents <= 94; the reference runs
// on PTX where such shifts yield 0, so the shift is clamped explicitly here
// (v_lshrrev_b32 would otherwise use only the low 5 bits of the amount).
__device__ __forceinline__ uint32_t e2m1_from_f32_ref(float q) {
  const uint32_t lo = 126u;
  uint32_t bits = __float_as_uint(q);
  uint32_t sign = bits & 0x80000000u;
  uint32_t e = (bits >> 23) & 0xFFu;
  uint32_t m = bits & 0x7FFFFFu;
  uint32_t shift = 127u - (e + 1u);
  uint32_t dm = shift >= 32u ? 0u : ((0x400000u | (m >> 1)) >> shift);
  m = (e < 127u) ? dm : m;
  e = (e > lo ? e : lo) - lo;
  uint32_t m2 = m >> 21;
  uint32_t inc = (m2 & 1u) & (((m & 0x1FFFFFu) != 0u) | ((m2 >> 1) & 1u));
  uint32_t r = (((e << 2) | m2) + inc) >> 1;
  r = r > 7u ? 7u : r;
  return ((sign >> 28) | r) & 0xFu;
}

// cvt_pk_f32_fp4<B>(src, scale, &lo, &hi): the two E2M1 nibbles of byte B
// of `src` (low nibble -> lo) times `scale`, as two fp32 values (exact for
// scale 2^k). Byte 0 is written as the bare instruction; bytes 1..3 use the
// compiler builtin, which encodes the byte in op_sel.
template <int B>
__device__ __forceinline__ void cvt_pk_f32_fp4(uint32_t src, float scale, float* lo, float* hi) {
  static_assert(B >= 0 && B < 4, "byte select 0..3");
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  f32x2_t r;
  if constexpr (B == 0) {
    asm("v_cvt_scalef32_pk_f32_fp4 %0, %1, %2" : "=v"(r) : "v"(src), "v"(scale));
  } else {
    r = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(src, scale, B);
  }
  *lo = r[0];
  *hi = r[1];
}

// IEEE binary32 -> bf16 bits, round to nearest even; NaN -> 0x7FFF.
// Stands for __floats2bfloat162_rn (per_token_Mxfp4ToBf16_dequant.cu:153).
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FFFu;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// Two floats in [-448, 448] (never NaN) -> two OCP E4M3 bytes, RNE, packed in
// the low 16 bits (a in bits 0..7). v_cvt_pk_fp8_f32 on gfx950 is OCP E4M3FN
// round-to-nearest-even; in this range it equals the __nv_fp8_e4m3(float)
// constructor (RNE, satfinite) that the reference uses.
__device__ __forceinline__ uint32_t fp8x2_from_f32(float a, float b) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xFFFFu;
}

// Four such floats -> four E4M3 bytes (a in bits 0..7). The first
// conversion's passed-through upper half is overwritten by the second, so its
// old operand is a's own bits rather than a register zeroed for it.
__device__ __forceinline__ uint32_t fp8x4_from_f32(float a, float b, float c, float d) {
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, __float_as_int(a), false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);
}

// Workgroup b of a 1-D grid is dispatched to XCD b % 8, and each XCD has its
// own L2. This renumbers the grid so that XCD x takes one contiguous run of
// logical indices (a bijection on [0, n)); workgroups adjacent in logical
// order then share an L2, e.g. tiles that read the same scale lines.
__device__ __forceinline__ uint32_t xcd_contiguous(uint32_t b, uint32_t n) {
  const uint32_t x = b & 7u, j = b >> 3, q = n >> 3, r = n & 7u;
  return x * q + (x < r ? x : r) + j;
}

// threadIdx.x through an empty asm statement: address arithmetic built on it
// is recomputed where it is used instead of being hoisted out of the loop and
// held in registers for the whole kernel.
__device__ __forceinline__ int opaque_tid() {
  int t = (int)threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

// Exact ceil(log2(z)) for a finite normal float z > 0.
__device__ __forceinline__ int ceil_log2_normal(float z) {
  uint32_t b = __float_as_uint(z);
  return (int)((b >> 23) & 0xFFu) - 127 + ((b & 0x7FFFFFu) != 0u);
}

// 2^k as a float for k in [-126, 127].
__device__ __forceinline__ float exp2i(int k) { return __uint_as_float((uint32_t)(k + 127) << 23); }

}  // namespace omo_hip
