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
// Fast path: for scale bytes 1..254, v_cvt_scalef32_pk_bf16_fp4 (two
// elements per instruction, scale operand 2^(s-127)) returns exactly the
// reference's rounded products, including subnormal results at s = 1 and
// overflow to inf near s = 254; it is checked against the reference rule for
// every code byte under every scale byte. Scale byte 0 (which the hardware
// reads as 2^-127, the reference as 0.0) and 255 (hardware NaN, reference
// inf) take the fp32 restatement.
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

// Fast path, valid for 1 <= sb <= 254.
__device__ __forceinline__ u32x4 dequant_dword_fast(uint32_t c, uint32_t sb) {
  const float sc = __uint_as_float(sb << 23);
  u32x4 o;
  o[0] = cvt_pk_bf16_fp4<0>(c, sc);
  o[1] = cvt_pk_bf16_fp4<1>(c, sc);
  o[2] = cvt_pk_bf16_fp4<2>(c, sc);
  o[3] = cvt_pk_bf16_fp4<3>(c, sc);
  return o;
}

// Workgroup b covers code dwords [b * 256 * UNROLL, +256 * UNROLL): a
// workgroup-uniform base pointer per tensor and 32-bit lane offsets, so each
// load and store takes one address operation. NT_CODES: code dwords are
// loaded non-temporally (scale bytes, each read by four lanes, never).
template <int UNROLL, bool NT_CODES>
__global__ __launch_bounds__(256) void dequant_bf16_kernel(const uint32_t* __restrict__ q, const uint8_t* __restrict__ s,
                                                           u32x4* __restrict__ out, int64_t ndw) {
  constexpr uint32_t kSpan = 256 * UNROLL;
  const int64_t b0 = (int64_t)blockIdx.x * kSpan;
  const uint32_t* qb = q + b0;
  const uint8_t* sb0 = s + (b0 >> 2);
  u32x4* ob = out + b0;
  const uint32_t lim = ndw - b0 < (int64_t)kSpan ? (uint32_t)(ndw - b0) : kSpan;  // dwords of this workgroup
  uint32_t c[UNROLL], sb[UNROLL];
  // Loads at clamped indices, all issued before the first wait: loads under
  // a per-lane bounds branch made the compiler wait for the first scale byte
  // at the branch's join before issuing the rest.
#pragma unroll
  for (int u = 0; u < UNROLL; u++) {
    const uint32_t i = min(u * 256 + threadIdx.x, lim - 1);
    c[u] = NT_CODES ? __builtin_nontemporal_load(qb + i) : qb[i];
    sb[u] = sb0[i >> 2];
  }
  // All outputs are formed before the first store: a store ahead of the
  // next dword's conversion made the wait for that dword's loads wait for
  // the store as well (loads and stores share one counter).
  u32x4 o[UNROLL];
#pragma unroll
  for (int u = 0; u < UNROLL; u++) {
    if (sb[u] - 1u <= 253u) {
      o[u] = dequant_dword_fast(c[u], sb[u]);
    } else {
      o[u] = dequant_dword_ref(c[u], sb[u]);
    }
  }
#pragma unroll
  for (int u = 0; u < UNROLL; u++) {
    const uint32_t i = u * 256 + threadIdx.x;
    if (i < lim) __builtin_nontemporal_store(o[u], ob + i);
  }
}

// Row-strided variant: row r's codes at q + r * q_stride, its scale bytes at
// s + r * s_stride (bytes), output [rows, K] bf16 contiguous. Reads the
// expert-parallel payload row [codes | scales] in place instead of the two
// .contiguous() copies of its unpacking (code/megatron-0.15.0rc7.diff:101-122).
// Workgroup b covers segment b % bpr of row b / bpr. Four dwords per lane
// at any launch size: at 4096 x 7168 (896 dwords per row) two per lane,
// with half the second segment idle, took 12.4 against 11.5 us.
template <int UNROLL>
__global__ __launch_bounds__(256) void dequant_rows_kernel(const uint8_t* __restrict__ q, int64_t q_stride,
                                                           const uint8_t* __restrict__ s, int64_t s_stride,
                                                           u32x4* __restrict__ out, int64_t K, int bpr) {
  const int64_t row = blockIdx.x / (uint32_t)bpr;
  const int seg = (int)(blockIdx.x - row * bpr);
  const int dpr = (int)(K / 8);  // code dwords per row
  const uint32_t* qr = reinterpret_cast<const uint32_t*>(q + row * q_stride);
  const uint8_t* sr = s + row * s_stride;
  u32x4* orow = out + row * dpr;
  const uint32_t base = seg * (256 * UNROLL) + threadIdx.x;
  uint32_t c[UNROLL], sb[UNROLL];
#pragma unroll
  for (int u = 0; u < UNROLL; u++) {  // clamped, as in dequant_bf16_kernel; unsigned offsets
    const uint32_t i = min(base + u * 256, (uint32_t)dpr - 1);
    c[u] = qr[i];
    sb[u] = sr[i >> 2];
  }
  u32x4 o[UNROLL];  // all outputs before the first store, as in dequant_bf16_kernel
#pragma unroll
  for (int u = 0; u < UNROLL; u++)
    o[u] = (sb[u] - 1u <= 253u) ? dequant_dword_fast(c[u], sb[u]) : dequant_dword_ref(c[u], sb[u]);
#pragma unroll
  for (int u = 0; u < UNROLL; u++) {
    const uint32_t i = base + u * 256;
    if (i < (uint32_t)dpr) __builtin_nontemporal_store(o[u], orow + i);
  }
}

hipError_t launch_dequant_rows(const void* q, int64_t q_stride, const void* s, int64_t s_stride, void* out,
                               int64_t rows, int64_t K, hipStream_t stream) {
  if (rows == 0 || K == 0) return hipSuccess;
  constexpr int U = 4;
  const int bpr = (int)((K / 8 + 256 * U - 1) / (256 * U));
  return launch((dequant_rows_kernel<U>), dim3((unsigned)(rows * bpr)), dim3(256), 0, stream,
                     static_cast<const uint8_t*>(q), q_stride, static_cast<const uint8_t*>(s), s_stride,
                     static_cast<u32x4*>(out), K, bpr);
}

hipError_t launch_dequant_bf16(const void* q, const void* s, void* out, int64_t nbytes, hipStream_t stream) {
  const int64_t ndw = nbytes / 4;
  if (ndw == 0) return hipSuccess;
  // Four dwords per lane when the launch is one round of resident
  // workgroups (8 per CU): every load is then issued at once (cfg1's 4096 x
  // 4096 takes 1.4 us longer as two rounds of two-dword workgroups). Larger
  // tensors take two dwords per lane, more rounds with less tail each:
  // 8192 x 7168 21.6 against 22.0 us, 4096 x 7168 11.5 against 11.6 us.
  // Code loads are non-temporal in the one-round launch only: 4096 x 4096
  // 7.14 against 7.20 us from cold buffers and the quantize + dequantize
  // round trip 15.14 against 15.66 us, while 8192 x 7168 in rounds took
  // 24.7 against 21.6 us that way.
  const int64_t b4 = (ndw + 1023) / 1024;
  if (b4 <= 8 * (int64_t)current_device_caps().cus)
    return launch((dequant_bf16_kernel<4, true>), dim3((unsigned)b4), dim3(256), 0, stream,
                  static_cast<const uint32_t*>(q), static_cast<const uint8_t*>(s), static_cast<u32x4*>(out), ndw);
  const int64_t b2 = (ndw + 511) / 512;
  return launch((dequant_bf16_kernel<2, false>), dim3((unsigned)b2), dim3(256), 0, stream,
                static_cast<const uint32_t*>(q), static_cast<const uint8_t*>(s), static_cast<u32x4*>(out), ndw);
}

}  // namespace omo_hip
