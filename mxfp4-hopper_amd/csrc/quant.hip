// BF16 -> MXFP4 rowwise quantize (1x32 blocks over the flat tensor).
//
// Semantics follow per_token_group_quant_4bit_kernel_coalescing
// (code/kernel/per_token_quant_mxfp4.cu:121-266):
//   amax  = fmaxf(eps, |x_j|) over the 32 elements (NaN ignored)     :151,170-178
//   y_s   = 2^ceil(log2(max(amax / fp4_max, 1e-10f)))               :185-187
//   scale = (uint8)((int)log2(y_s) + 127)                            :192
//   q_j   = clamp(x_j * (1/y_s), fp4_min, fp4_max) -> E2M1 RNE nibble :200-254
//
// Layout in HBM: the input is read as 16-byte chunks of 8 bf16; four
// consecutive chunks form one 32-element block. Chunk i is handled by one
// lane, so a block is a DPP quad (lanes 4k..4k+3) and the block amax is two
// quad_perm max steps. A wave touches 1 KiB of contiguous input per load,
// 256 B of contiguous codes per store and 16 contiguous scale bytes.
//
// Fast path (fp4_min == -6, fp4_max == 6, block free of inf/NaN):
//   * amax via packed u16 max of |x| bit patterns (monotone for non-NaN),
//   * the scale exponent in closed form: for a bf16 amax = (1+f/128)*2^E,
//     ceil(log2(amax/6)) = E - 2 + (f > 64); amax/6 is either an exact power
//     of two (f == 64) or at least 0.5% away from one, so rounding of the
//     quotient never moves the ceiling; the 1e-10 floor is exponent -33;
//   * q = x / 2^c is exact and |q| <= 6, so v_cvt_scalef32_pk_fp4_bf16
//     (round-to-nearest-even, verified bit-exact against the reference rule
//     over every bf16 value and every reachable c in [-33, 126]) yields the
//     reference nibbles, 2 elements per instruction.
// Blocks holding inf or NaN, and non-default clamp constants, take the
// emulation path, which restates the reference operations in fp32.
#include "omo_internal.h"
#include "omo_quant.cuh"

namespace omo_hip {

struct QuantArgs {
  const u32x4* __restrict__ x;  // bf16, 8 per chunk
  uint32_t* __restrict__ q;     // 8 nibbles per chunk
  uint8_t* __restrict__ s;      // one E8M0 byte per 4 chunks
  int64_t nchunks;              // numel / 8, multiple of 4
  float eps, fp4_min, fp4_max;
  int c_eps;                    // scale exponent when amax == eps (fast path)
};

template <int UNROLL, bool STANDARD>
__global__ __launch_bounds__(256) void quant_rowwise_kernel(QuantArgs a) {
  const int64_t base = (int64_t)blockIdx.x * (256 * UNROLL) + threadIdx.x;
  u32x4 d[UNROLL];
#pragma unroll
  for (int u = 0; u < UNROLL; u++) {
    const int64_t ch = base + (int64_t)u * 256;
    if (ch < a.nchunks) d[u] = __builtin_nontemporal_load(a.x + ch);
  }
  const bool quad_leader = (threadIdx.x & 3u) == 0u;
#pragma unroll
  for (int u = 0; u < UNROLL; u++) {
    const int64_t ch = base + (int64_t)u * 256;
    // nchunks is a multiple of 4 and quads are 4-aligned, so a quad is
    // either fully inside or fully outside the tensor.
    if (ch >= a.nchunks) continue;
    uint32_t codes, byte;
    if (STANDARD) {
      uint32_t am = quad_max_u32(chunk_absmax_bits(d[u]));
      if (__builtin_expect(am < 0x7F80u, 1)) {
        codes = quant_chunk_fast(d[u], am, a.eps, a.c_eps, &byte);
      } else {
        quant_chunk_ref(d[u], a.eps, a.fp4_min, a.fp4_max, &codes, &byte);
      }
    } else {
      quant_chunk_ref(d[u], a.eps, a.fp4_min, a.fp4_max, &codes, &byte);
    }
    // Codes are streamed out non-temporally (each wave store is 256
    // contiguous bytes); the one-byte scale stores stay temporal, which
    // measured faster for them.
    __builtin_nontemporal_store(codes, a.q + ch);
    if (quad_leader) a.s[ch >> 2] = (uint8_t)byte;
  }
}

// Row-strided variant: row r of the codes starts at q + r * q_stride and its
// scales at s + r * s_stride (bytes), so the outputs can be interleaved, e.g.
// the expert-parallel payload row [codes (K/2 B) | scales (K/32 B)] that
// Megatron builds with torch.cat (code/megatron-0.15.0rc7.diff:93-99,
// 163-170). Workgroup b covers segment b % bpr of row b / bpr; a quad (one
// block) never straddles rows because K % 32 == 0 and segments start at
// multiples of 256 chunks. Reference rule with fp4_min = -6, fp4_max = 6.
struct QuantRowsArgs {
  const uint16_t* __restrict__ x;  // [rows, K] bf16
  uint8_t* __restrict__ q;
  uint8_t* __restrict__ s;
  int64_t K, q_stride, s_stride;
  int bpr;                         // workgroups per row
  float eps;
  int c_eps;
};

template <int UNROLL>
__global__ __launch_bounds__(256) void quant_rows_kernel(QuantRowsArgs a) {
  const int64_t row = blockIdx.x / (uint32_t)a.bpr;
  const int seg = (int)(blockIdx.x - row * a.bpr);
  const int cpr = (int)(a.K / 8);  // 16 B chunks per row
  const u32x4* xr = reinterpret_cast<const u32x4*>(a.x + row * a.K);
  uint32_t* qr = reinterpret_cast<uint32_t*>(a.q + row * a.q_stride);
  uint8_t* sr = a.s + row * a.s_stride;
  const int base = seg * (256 * UNROLL) + (int)threadIdx.x;
  u32x4 d[UNROLL];
#pragma unroll
  for (int u = 0; u < UNROLL; u++) {
    const int c = base + u * 256;
    if (c < cpr) d[u] = __builtin_nontemporal_load(xr + c);
  }
  const bool quad_leader = (threadIdx.x & 3u) == 0u;
#pragma unroll
  for (int u = 0; u < UNROLL; u++) {
    const int c = base + u * 256;
    if (c >= cpr) continue;  // whole quads
    uint32_t codes, byte;
    const uint32_t am = quad_max_u32(chunk_absmax_bits(d[u]));
    if (__builtin_expect(am < 0x7F80u, 1)) {
      codes = quant_chunk_fast(d[u], am, a.eps, a.c_eps, &byte);
    } else {
      quant_chunk_ref(d[u], a.eps, -6.0f, 6.0f, &codes, &byte);
    }
    __builtin_nontemporal_store(codes, qr + c);
    if (quad_leader) sr[c >> 2] = (uint8_t)byte;
  }
}

hipError_t launch_quant_rows(const void* x, void* q, int64_t q_stride, void* s, int64_t s_stride, int64_t rows,
                             int64_t K, float eps, hipStream_t stream) {
  if (rows == 0 || K == 0) return hipSuccess;
  constexpr int U = 2;
  QuantRowsArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.q = static_cast<uint8_t*>(q);
  a.s = static_cast<uint8_t*>(s);
  a.K = K;
  a.q_stride = q_stride;
  a.s_stride = s_stride;
  a.bpr = (int)((K / 8 + 256 * U - 1) / (256 * U));
  a.eps = eps;
  a.c_eps = host_c_eps(eps, 6.0f);
  hipLaunchKernelGGL((quant_rows_kernel<U>), dim3((unsigned)(rows * a.bpr)), dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_quant_rowwise(const void* x, void* q, void* s, int64_t numel, float eps, float fp4_min,
                                float fp4_max, hipStream_t stream) {
  QuantArgs a;
  a.x = static_cast<const u32x4*>(x);
  a.q = static_cast<uint32_t*>(q);
  a.s = static_cast<uint8_t*>(s);
  a.nchunks = numel / 8;
  a.eps = eps;
  a.fp4_min = fp4_min;
  a.fp4_max = fp4_max;
  a.c_eps = host_c_eps(eps, fp4_max);
  if (a.nchunks == 0) return hipSuccess;
  constexpr int U = 2;
  const int64_t blocks = (a.nchunks + 256 * U - 1) / (256 * U);
  const bool standard = (fp4_max == 6.0f && fp4_min == -6.0f);
  if (standard) {
    hipLaunchKernelGGL((quant_rowwise_kernel<U, true>), dim3((unsigned)blocks), dim3(256), 0, stream, a);
  } else {
    hipLaunchKernelGGL((quant_rowwise_kernel<U, false>), dim3((unsigned)blocks), dim3(256), 0, stream, a);
  }
  return hipGetLastError();
}

}  // namespace omo_hip
