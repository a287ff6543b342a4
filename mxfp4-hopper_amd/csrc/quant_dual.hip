// Fused dual-layout BF16 -> MXFP4 quantize: rowwise 1x32 blocks along K and
// columnwise 32x1 blocks along M from one read of the input.
//
// The columnwise output is defined by the TE integration as
// quant_rowwise(X.T.contiguous()) (code/transformer_engine-2.8.diff:1463-1466):
// codes [K, M/2] and scales [K, M/32]. The reference pays a full transpose
// copy plus a second quantize pass for it; here each 32x256 input tile is
// read once, quantized rowwise from registers (same DPP-quad scheme as the
// rowwise kernel) and staged in LDS, from where each thread reads one
// 32-element column and quantizes it along M. Both layouts use the
// reference block rule (code/kernel/per_token_quant_mxfp4.cu:151-254) with
// fp4_min = -6, fp4_max = 6, the constants of the quantize wrapper
// (code/kernel/api/mxfp4.py:11-12, 152-154).
#include "omo_internal.h"
#include "omo_quant.cuh"

namespace omo_hip {

constexpr int kDualRows = 32;
constexpr int kDualCols = 256;
constexpr int kDualPitch = kDualCols * 2 + 16;  // bytes per LDS row

__global__ __launch_bounds__(256) void quant_dual_kernel(const uint16_t* __restrict__ x, uint32_t* __restrict__ row_q,
                                                         uint8_t* __restrict__ row_s, uint8_t* __restrict__ col_q,
                                                         uint8_t* __restrict__ col_s, int64_t M, int64_t K, float eps,
                                                         int c_eps) {
  __shared__ __attribute__((aligned(16))) uint8_t tile[kDualRows * kDualPitch];
  const int t = threadIdx.x;
  const int64_t k0 = (int64_t)blockIdx.x * kDualCols, m0 = (int64_t)blockIdx.y * kDualRows;
  // 32 rows x 32 chunks of 8 bf16; thread t owns chunks t + 256 k.
  u32x4 d[4];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int cid = t + 256 * k, r = cid >> 5, cc = cid & 31;
    const int64_t col = k0 + cc * 8;
    if (col < K) d[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(x + (m0 + r) * K + col));
  }
  const bool quad_leader = (t & 3) == 0;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int cid = t + 256 * k, r = cid >> 5, cc = cid & 31;
    const int64_t col = k0 + cc * 8;
    if (col >= K) continue;  // K % 32 == 0: a quad is entirely in or out
    *reinterpret_cast<u32x4*>(tile + r * kDualPitch + cc * 16) = d[k];
    uint32_t codes, byte;
    const uint32_t am = quad_max_u32(chunk_absmax_bits(d[k]));
    if (am < 0x7F80u) {
      codes = quant_chunk_fast(d[k], am, eps, c_eps, &byte);
    } else {
      quant_chunk_ref(d[k], eps, -6.0f, 6.0f, &codes, &byte);
    }
    const int64_t grow = m0 + r;
    __builtin_nontemporal_store(codes, row_q + (grow * K + col) / 8);
    if (quad_leader) row_s[grow * (K / 32) + col / 32] = (uint8_t)byte;
  }
  __syncthreads();
  const int64_t kc = k0 + t;
  if (kc >= K) return;
  uint32_t p[16];
  uint32_t amax_bits = 0;
#pragma unroll
  for (int j = 0; j < 16; j++) {
    const uint32_t lo = *reinterpret_cast<const uint16_t*>(tile + (2 * j) * kDualPitch + 2 * t);
    const uint32_t hi = *reinterpret_cast<const uint16_t*>(tile + (2 * j + 1) * kDualPitch + 2 * t);
    p[j] = lo | (hi << 16);
    amax_bits = max(amax_bits, max(lo & 0x7FFFu, hi & 0x7FFFu));
  }
  uint32_t byte;
  u32x4 codes;
  if (amax_bits < 0x7F80u) {
    codes = quant_block32_fast(p, amax_bits, eps, c_eps, &byte);
  } else {
    codes = quant_block32_ref(p, eps, -6.0f, 6.0f, &byte);
  }
  __builtin_nontemporal_store(codes, reinterpret_cast<u32x4*>(col_q + kc * (M / 2) + m0 / 2));
  col_s[kc * (M / 32) + m0 / 32] = (uint8_t)byte;
}

hipError_t launch_quant_dual(const void* x, void* row_q, void* row_s, void* col_q, void* col_s, int64_t M, int64_t K,
                             float eps, hipStream_t stream) {
  if (M == 0 || K == 0) return hipSuccess;
  dim3 grid((unsigned)((K + kDualCols - 1) / kDualCols), (unsigned)(M / kDualRows));
  hipLaunchKernelGGL(quant_dual_kernel, grid, dim3(256), 0, stream, static_cast<const uint16_t*>(x),
                     static_cast<uint32_t*>(row_q), static_cast<uint8_t*>(row_s), static_cast<uint8_t*>(col_q),
                     static_cast<uint8_t*>(col_s), M, K, eps, host_c_eps(eps, 6.0f));
  return hipGetLastError();
}

}  // namespace omo_hip
