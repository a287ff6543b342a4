// Row gather of MXFP4 tensors: the data movement of TE's moe_permute for
// MXFP4 inputs (code/transformer_engine-2.8.diff:256-261, 338-354), which
// permutes the code rows [T, H/2] and the scale rows [T, H/32] of the tokens
// into expert-major order with TE's own row permutation kernel.
//
// Output row r of both tensors is input row src[r]; an index outside
// [0, n_src) writes a zero row (the padding rows of a permutation with more
// output rows than routed tokens). Inputs may be strided (bytes between rows),
// so the expert-parallel payload rows [codes | scales] are read in place.
//
// One wave per output row, 4 rows per 256-thread workgroup; each lane moves
// V-sized pieces (16 B when every row start and row length allows it), four
// loads in flight before their stores. Source rows are read with ordinary
// loads: a token routed to k experts is read k times, and the repeats then
// come from cache. Code rows are stored non-temporally where each is whole
// 128 B lines (H % 256 == 0 and a 128 B aligned output), else with ordinary
// stores; scale rows (H/32 bytes, sharing lines with the next output row)
// always with ordinary stores, so their lines are completed in L2.
#include "omo_device.cuh"
#include "omo_internal.h"

namespace omo_hip {

template <typename V, bool NT_OUT>
__device__ __forceinline__ void copy_row(const uint8_t* __restrict__ in, bool ok, uint8_t* __restrict__ out,
                                         int64_t bytes, int lane) {
  constexpr int U = 4;
  const int64_t n = bytes / (int64_t)sizeof(V);
  const V* src = reinterpret_cast<const V*>(in);
  V* dst = reinterpret_cast<V*>(out);
  V zero;
  memset(&zero, 0, sizeof(V));
  for (int64_t i0 = lane; i0 < n; i0 += 64 * U) {
    V v[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int64_t i = i0 + 64 * u;
      v[u] = zero;
      if (ok && i < n) v[u] = src[i];
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int64_t i = i0 + 64 * u;
      if (i < n) {
        if (NT_OUT) __builtin_nontemporal_store(v[u], dst + i);
        else dst[i] = v[u];
      }
    }
  }
}

template <typename V, bool NT_A>
__global__ __launch_bounds__(256) void gather_rows_kernel(const uint8_t* __restrict__ a, int64_t a_stride,
                                                          int64_t a_bytes, const uint8_t* __restrict__ b,
                                                          int64_t b_stride, int64_t b_bytes,
                                                          const int32_t* __restrict__ src, int64_t n_src,
                                                          int64_t n_out, uint8_t* __restrict__ out_a,
                                                          uint8_t* __restrict__ out_b) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= n_out) return;
  const int lane = (int)(threadIdx.x & 63);
  const int64_t sr = src[r];
  const bool ok = sr >= 0 && sr < n_src;
  const int64_t rr = ok ? sr : 0;
  copy_row<V, NT_A>(a + rr * a_stride, ok, out_a + r * a_bytes, a_bytes, lane);
  copy_row<V, false>(b + rr * b_stride, ok, out_b + r * b_bytes, b_bytes, lane);
}

template <typename V>
hipError_t launch_gather(bool nt_a, dim3 grid, hipStream_t stream, const uint8_t* a, int64_t a_stride,
                         int64_t a_bytes, const uint8_t* b, int64_t b_stride, int64_t b_bytes, const int32_t* src,
                         int64_t n_src, int64_t n_out, uint8_t* out_a, uint8_t* out_b) {
  auto kernel = nt_a ? gather_rows_kernel<V, true> : gather_rows_kernel<V, false>;
  return launch(kernel, grid, dim3(256), 0, stream, a, a_stride, a_bytes, b, b_stride, b_bytes, src, n_src, n_out,
                out_a, out_b);
}

hipError_t launch_gather_rows(const void* a, int64_t a_stride, int64_t a_bytes, const void* b, int64_t b_stride,
                              int64_t b_bytes, const int32_t* src, int64_t n_src, int64_t n_out, void* out_a,
                              void* out_b, hipStream_t stream) {
  if (n_out == 0) return hipSuccess;
  // widest piece dividing every row start and row length
  const uint64_t bits = (uint64_t)a_stride | (uint64_t)a_bytes | (uint64_t)b_stride | (uint64_t)b_bytes |
                        reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
                        reinterpret_cast<uintptr_t>(out_a) | reinterpret_cast<uintptr_t>(out_b);
  // Non-temporal code-row stores only where every output row is whole 128 B
  // lines; otherwise neighbouring rows share lines, which L2 must merge.
  const bool nt_a = a_bytes % 128 == 0 && (reinterpret_cast<uintptr_t>(out_a) & 127) == 0;
  const dim3 grid((unsigned)((n_out + 3) / 4));
  const uint8_t *pa = static_cast<const uint8_t*>(a), *pb = static_cast<const uint8_t*>(b);
  uint8_t *qa = static_cast<uint8_t*>(out_a), *qb = static_cast<uint8_t*>(out_b);
  if ((bits & 15) == 0)
    return launch_gather<u32x4>(nt_a, grid, stream, pa, a_stride, a_bytes, pb, b_stride, b_bytes, src, n_src, n_out,
                                qa, qb);
  if ((bits & 3) == 0)
    return launch_gather<uint32_t>(nt_a, grid, stream, pa, a_stride, a_bytes, pb, b_stride, b_bytes, src, n_src,
                                   n_out, qa, qb);
  return launch_gather<uint8_t>(nt_a, grid, stream, pa, a_stride, a_bytes, pb, b_stride, b_bytes, src, n_src, n_out,
                                qa, qb);
}

}  // namespace omo_hip
