// MXFP4 -> BF16 dequant over the flat code tensor.
//
// Semantics follow omo_per_token_Mxfp4ToBf16_dequant_kernel
// (code/kernel/per_token_Mxfp4ToBf16_dequant.cu:70-160): element i takes
// scale byte i/32 (the kernel indexes the scales flat, :129), the E2M1 code
// decodes to bf16 bits (:137-150), the E8M0 byte decodes as bf16 bits s<<7
// (so s=0 -> 0.0 and s=255 -> +inf, :22-29), the product is formed in fp32
// and rounded to bf16 (RNE, :152-156).
//
// Layout in HBM: each lane reads one dword of codes (8 elements, 4 B) and
// writes 16 B of bf16, so a wave reads 256 contiguous code bytes and writes
// 1 KiB of contiguous output per instruction; 4 lanes share a scale byte.
//
// Fast path: for a scale byte s in [2, 252] every product code*2^(s-127) is a
// normal bf16 value, so the result is the code's bf16 pattern with s-127
// added to its exponent field (zero codes stay +-0). The four code-magnitude
// patterns per exponent are looked up with v_perm_b32 from per-lane byte
// tables that already include the exponent offset. Other scale bytes take
// the fp32 restatement.
#include "omo_device.cuh"
#include "omo_internal.h"

namespace omo_hip {

// Reference restatement for one code dword (8 elements) under scale byte sb.
__device__ __forceinline__ u32x4 dequant_dword_ref(uint32_t c, uint32_t sb) {
  const float sc = bf16_to_f32((sb & 0xFFu) << 7);
  u32x4 o;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    uint32_t byte = (c >> (8 * k)) & 0xFFu;
    uint32_t lo = f32_to_bf16_rne(bf16_to_f32(e2m1_to_bf16_bits(byte & 0xFu)) * sc);
    uint32_t hi = f32_to_bf16_rne(bf16_to_f32(e2m1_to_bf16_bits(byte >> 4)) * sc);
    o[k] = lo | (hi << 16);
  }
  return o;
}

// Fast path, valid for 2 <= sb <= 252.
//   mag  m = code & 7, bf16(m) = {0, 0x3F00, 0x3F80, 0x3FC0, 0x4000, 0x4040, 0x4080, 0x40C0}
//   out  = m ? bf16(m) + (sb-127)*128 : 0, then | sign<<15.
// Byte tables tl (low bytes) / th (high bytes) of the 8 offset patterns are
// built once per lane; each output dword (2 elements) is two v_perm lookups.
__device__ __forceinline__ u32x4 dequant_dword_fast(uint32_t c, uint32_t sb) {
  const uint32_t off = ((sb - 127u) << 7) & 0xFFFFu;
  const uint32_t off2 = off | (off << 16);
  // Patterns for magnitudes (1,0), (3,2), (5,4), (7,6) as packed u16 pairs.
  u16x2_t p10 = __builtin_bit_cast(u16x2_t, 0x3F000000u) + __builtin_bit_cast(u16x2_t, off2 & 0xFFFF0000u);
  u16x2_t p32 = __builtin_bit_cast(u16x2_t, 0x3FC03F80u) + __builtin_bit_cast(u16x2_t, off2);
  u16x2_t p54 = __builtin_bit_cast(u16x2_t, 0x40404000u) + __builtin_bit_cast(u16x2_t, off2);
  u16x2_t p76 = __builtin_bit_cast(u16x2_t, 0x40C04080u) + __builtin_bit_cast(u16x2_t, off2);
  const uint32_t w10 = __builtin_bit_cast(uint32_t, p10), w32 = __builtin_bit_cast(uint32_t, p32);
  const uint32_t w54 = __builtin_bit_cast(uint32_t, p54), w76 = __builtin_bit_cast(uint32_t, p76);
  // tl bytes [m0..m3] / [m4..m7]: low bytes of the patterns; th: high bytes.
  const uint32_t tl_lo = __builtin_amdgcn_perm(w32, w10, 0x06040200u);
  const uint32_t tl_hi = __builtin_amdgcn_perm(w76, w54, 0x06040200u);
  const uint32_t th_lo = __builtin_amdgcn_perm(w32, w10, 0x07050301u);
  const uint32_t th_hi = __builtin_amdgcn_perm(w76, w54, 0x07050301u);
  u32x4 o;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    // n = [byte_k & 0xF (half 0), byte_k >> 4 (half 1)]
    uint32_t bb = __builtin_amdgcn_perm(0u, c, 0x0C000C00u | (uint32_t)(k | (k << 16)));
    uint32_t n = (bb & 0x0000000Fu) | ((bb >> 4) & 0x000F0000u);
    uint32_t mag = n & 0x00070007u;
    uint32_t selL = mag | 0x0C000C00u;         // [m0, 0, m1, 0]
    uint32_t selH = (mag << 8) | 0x000C000Cu;  // [0, m0, 0, m1]
    uint32_t lo = __builtin_amdgcn_perm(tl_hi, tl_lo, selL);
    uint32_t hi = __builtin_amdgcn_perm(th_hi, th_lo, selH);
    uint32_t sign = (n & 0x00080008u) << 12;
    o[k] = lo | hi | sign;
  }
  return o;
}

template <int UNROLL>
__global__ __launch_bounds__(256) void dequant_bf16_kernel(const uint32_t* __restrict__ q, const uint8_t* __restrict__ s,
                                                           u32x4* __restrict__ out, int64_t ndw) {
  const int64_t base = (int64_t)blockIdx.x * (256 * UNROLL) + threadIdx.x;
  uint32_t c[UNROLL], sb[UNROLL];
#pragma unroll
  for (int u = 0; u < UNROLL; u++) {
    const int64_t i = base + (int64_t)u * 256;
    if (i < ndw) {
      c[u] = __builtin_nontemporal_load(q + i);
      sb[u] = s[i >> 2];
    }
  }
#pragma unroll
  for (int u = 0; u < UNROLL; u++) {
    const int64_t i = base + (int64_t)u * 256;
    if (i >= ndw) continue;
    u32x4 o;
    if (sb[u] - 2u <= 250u) {
      o = dequant_dword_fast(c[u], sb[u]);
    } else {
      o = dequant_dword_ref(c[u], sb[u]);
    }
    __builtin_nontemporal_store(o, out + i);
  }
}

hipError_t launch_dequant_bf16(const void* q, const void* s, void* out, int64_t nbytes, hipStream_t stream) {
  const int64_t ndw = nbytes / 4;
  if (ndw == 0) return hipSuccess;
  constexpr int U = 4;
  const int64_t blocks = (ndw + 256 * U - 1) / (256 * U);
  hipLaunchKernelGGL((dequant_bf16_kernel<U>), dim3((unsigned)blocks), dim3(256), 0, stream,
                     static_cast<const uint32_t*>(q), static_cast<const uint8_t*>(s), static_cast<u32x4*>(out), ndw);
  return hipGetLastError();
}

}  // namespace omo_hip
