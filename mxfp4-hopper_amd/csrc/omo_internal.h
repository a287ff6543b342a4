// Internal host-side launcher declarations of the MXFP4 HIP library. Each
// launcher assumes its arguments were validated by the C-ABI layer
// (omo_abi.hip) and only enqueues work on `stream`.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <cstring>
#include <tuple>
#include <type_traits>
#include <utility>

namespace omo_hip {

// Enqueues `kernel` with its arguments converted to the kernel's parameter
// types and returns the status of this launch alone (hipLaunchKernel's return
// value), so an error left earlier on the calling thread by other code is
// neither reported as this launch's failure nor cleared.
template <typename... P, typename... A>
hipError_t launch(void (*kernel)(P...), dim3 grid, dim3 block, size_t lds, hipStream_t stream, A&&... args) {
  static_assert(sizeof...(P) == sizeof...(A), "kernel argument count");
  std::tuple<std::decay_t<P>...> vals(static_cast<std::decay_t<P>>(std::forward<A>(args))...);
  return std::apply(
      [&](auto&... v) {
        void* ptrs[] = {static_cast<void*>(&v)...};
        return hipLaunchKernel(reinterpret_cast<const void*>(kernel), grid, block, ptrs, lds, stream);
      },
      vals);
}

hipError_t launch_quant_rowwise(const void* x, void* q, void* s, int64_t numel, float eps, float fp4_min,
                                float fp4_max, hipStream_t stream);

hipError_t launch_dequant_bf16(const void* q, const void* s, void* out, int64_t nbytes, hipStream_t stream);

hipError_t launch_mxfp4_to_fp8(const void* q, const void* s, void* out, float* out_s, int64_t M, int64_t Kb,
                               hipStream_t stream);

hipError_t launch_mxfp4_to_fp8_col(const void* q, const void* s, void* out, float* out_s, int64_t M, int64_t Kb,
                                   float eps, hipStream_t stream);

hipError_t launch_row_to_fp8_col(const void* q, const void* s, void* out, float* out_s, int64_t M, int64_t N,
                                 float eps, hipStream_t stream);

hipError_t launch_row_to_fp8_col_msplit(const void* q, const void* s, void* out, float* out_s, int64_t total_rows,
                                        int64_t N, const int32_t* lens, const int32_t* offs, const int32_t* soffs,
                                        int64_t nsplits, int64_t max_split_len, int64_t out_capacity,
                                        int64_t out_s_rows, float eps, hipStream_t stream);

// Row-strided variants (bytes between consecutive rows of codes / scales).
hipError_t launch_quant_rows(const void* x, void* q, int64_t q_stride, void* s, int64_t s_stride, int64_t rows,
                             int64_t K, float eps, hipStream_t stream);

hipError_t launch_dequant_rows(const void* q, int64_t q_stride, const void* s, int64_t s_stride, void* out,
                               int64_t rows, int64_t K, hipStream_t stream);

// src: optional int32 source row per output row (indices outside [0, n_src)
// read zeros); M output rows.
hipError_t launch_mxfp4_to_fp8_rows(const void* q, int64_t q_stride, const void* s, int64_t s_stride,
                                    const int32_t* src, int64_t n_src, void* out, float* out_s, int64_t M, int64_t Kb,
                                    hipStream_t stream);

// Gather rows of two byte tensors (codes and scales of MXFP4 rows) into
// contiguous outputs: out row r = input row src[r]; zeros for indices
// outside [0, n_src).
hipError_t launch_gather_rows(const void* a, int64_t a_stride, int64_t a_bytes, const void* b, int64_t b_stride,
                              int64_t b_bytes, const int32_t* src, int64_t n_src, int64_t n_out, void* out_a,
                              void* out_b, hipStream_t stream);

hipError_t launch_quant_dual(const void* x, void* row_q, void* row_s, void* col_q, void* col_s, int64_t M, int64_t K,
                             float eps, hipStream_t stream);

// One tensor of a grouped dual-layout quantize (validated by the ABI layer).
struct DualSpec {
  const void* x;
  void *row_q, *row_s, *col_q, *col_s;
  int64_t M, K;
};

hipError_t launch_quant_dual_grouped(const DualSpec* items, int count, float eps, hipStream_t stream);

// Properties of the current device, queried once per device and cached:
// compute units, and the largest LDS allocation of one workgroup in bytes.
struct DeviceCaps {
  int cus;
  int lds_per_workgroup;
};
DeviceCaps current_device_caps();

}  // namespace omo_hip
