// extern "C" boundary of libomo_mxfp4.so: argument validation, then launch.
// Declarations and the reference interface each entry point replaces are in
// include/omo_mxfp4.h. No function here allocates device memory or
// synchronizes; every check runs on the host before any HIP call.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <vector>

#include "../../include/omo_mxfp4.h"
#include "omo_internal.h"

namespace {

thread_local char g_err[512] = "";

int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return status;
}

int ok() {
  g_err[0] = '\0';
  return OMO_OK;
}

int from_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return ok();
  return fail(OMO_ERR_HIP, "%s: HIP launch failed: %s", what, hipGetErrorString(e));
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// Products of caller-supplied sizes go through size_mul: a * b for a, b >= 0,
// or -1 when it passes 2^60 (beyond any device's memory, and far enough below
// 2^63 that the small multiples taken of it afterwards stay exact).
constexpr int64_t kMaxSize = (int64_t)1 << 60;

int64_t size_mul(int64_t a, int64_t b) {
  int64_t r;
  if (a < 0 || b < 0 || __builtin_mul_overflow(a, b, &r) || r > kMaxSize) return -1;
  return r;
}

#define REQUIRE(cond, ...)                                  \
  do {                                                      \
    if (!(cond)) return fail(OMO_ERR_INVALID_ARGUMENT, __VA_ARGS__); \
  } while (0)

// A buffer that must hold `need` units: non-null when need > 0, large enough.
#define REQUIRE_BUF(name, ptr, have, need)                                                            \
  do {                                                                                                \
    REQUIRE((have) >= 0 && (need) >= 0, "%s: negative size", name);                                   \
    REQUIRE((need) == 0 || (ptr) != nullptr, "%s: null pointer", name);                               \
    REQUIRE((have) >= (need), "%s: buffer holds %lld, needs %lld", name, (long long)(have), (long long)(need)); \
  } while (0)

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

// Shared checks of the three requant entry points taking (rows, row_bytes).
int check_requant_common(const char* fn, const void* input, int64_t rows, int64_t row_bytes, int scale_ue8m0) {
  REQUIRE(rows >= 0 && row_bytes >= 0, "%s: negative shape", fn);
  if (scale_ue8m0) return fail(OMO_ERR_UNSUPPORTED, "%s: scale_ue8m0 is not supported (the reference asserts it off)", fn);
  REQUIRE(size_mul(rows, row_bytes) >= 0, "%s: shape too large", fn);
  REQUIRE(rows * row_bytes % 128 == 0, "%s: input.numel() %% 128 != 0 (input.numel()=%lld)", fn,
          (long long)(rows * row_bytes));
  (void)input;
  return OMO_OK;
}

int requant_rowwise(const char* fn, const void* input, int64_t rows, int64_t row_bytes, const void* input_s,
                    int64_t input_s_bytes, void* output_q, int64_t output_q_bytes, void* output_s,
                    int64_t output_s_elems, int scale_ue8m0, void* stream) {
  int rc = check_requant_common(fn, input, rows, row_bytes, scale_ue8m0);
  if (rc != OMO_OK) return rc;
  REQUIRE(row_bytes % 64 == 0, "%s: row bytes must be a multiple of 64 (got %lld); pad as the wrapper does", fn,
          (long long)row_bytes);
  const int64_t n = rows * row_bytes;
  REQUIRE_BUF("input", input, n, n);
  REQUIRE_BUF("input_s", input_s, input_s_bytes, n / 16);
  REQUIRE_BUF("output_q", output_q, output_q_bytes, 2 * n);
  REQUIRE_BUF("output_s", output_s, output_s_elems, n / 64);
  REQUIRE(n / 64 < (int64_t)1 << 31, "%s: too many 128-element groups", fn);
  REQUIRE(aligned(input, 8) && aligned(input_s, 4) && aligned(output_q, 16) && aligned(output_s, 4),
          "%s: misaligned buffer (input needs 8 B, input_s 4 B, output_q 16 B)", fn);
  if (n == 0) return ok();
  return from_hip(omo_hip::launch_mxfp4_to_fp8(input, input_s, output_q, static_cast<float*>(output_s), rows,
                                               row_bytes, as_stream(stream)),
                  fn);
}

// Payload rows [codes (cols/2 B) | scales (cols/32 B)], stride 17 cols / 32 bytes.
int check_packed(const char* fn, int64_t rows, int64_t cols) {
  REQUIRE(rows >= 0 && cols >= 0, "%s: negative shape", fn);
  REQUIRE(cols % 128 == 0, "%s: cols must be a multiple of 128 (got %lld)", fn, (long long)cols);
  REQUIRE(rows < ((int64_t)1 << 31) / (cols / 8 / 256 + 1), "%s: too many rows", fn);
  return OMO_OK;
}

// Shared checks of the permutation entry points: strided input rows of codes
// and scales, num_out int32 source indices.
int check_permute(const char* fn, const void* codes, int64_t codes_bytes, int64_t code_stride, const void* scales,
                  int64_t scales_bytes, int64_t scale_stride, int64_t num_tokens, int64_t cols,
                  const int32_t* src_rows, int64_t num_out) {
  REQUIRE(num_tokens >= 0 && cols >= 0 && num_out >= 0, "%s: negative shape", fn);
  REQUIRE(cols % 32 == 0, "%s: cols must be a multiple of 32 (got %lld)", fn, (long long)cols);
  REQUIRE(num_tokens < ((int64_t)1 << 31) && num_out < ((int64_t)1 << 31), "%s: too many rows", fn);
  REQUIRE(cols <= kMaxSize && code_stride <= kMaxSize && scale_stride <= kMaxSize, "%s: shape too large", fn);
  REQUIRE(code_stride >= cols / 2 && scale_stride >= cols / 32, "%s: row stride shorter than the row", fn);
  const int64_t code_span = num_tokens == 0 ? 0 : size_mul(num_tokens - 1, code_stride);
  const int64_t scale_span = num_tokens == 0 ? 0 : size_mul(num_tokens - 1, scale_stride);
  REQUIRE(code_span >= 0 && scale_span >= 0 && size_mul(num_out, cols) >= 0, "%s: shape too large", fn);
  const int64_t code_need = num_tokens == 0 ? 0 : code_span + cols / 2;
  const int64_t scale_need = num_tokens == 0 ? 0 : scale_span + cols / 32;
  REQUIRE_BUF("codes", codes, codes_bytes, code_need);
  REQUIRE_BUF("scales", scales, scales_bytes, scale_need);
  REQUIRE(num_out == 0 || src_rows != nullptr, "%s: src_rows: null pointer", fn);
  REQUIRE(aligned(src_rows, 4), "%s: src_rows must be 4-byte aligned", fn);
  return OMO_OK;
}

// Checks of one dual-layout quantize (single or grouped).
int check_dual(const char* fn, const void* input, int64_t rows, int64_t cols, const void* row_q, int64_t row_q_bytes,
               const void* row_s, int64_t row_s_bytes, const void* col_q, int64_t col_q_bytes, const void* col_s,
               int64_t col_s_bytes) {
  REQUIRE(rows >= 0 && cols >= 0, "%s: negative shape", fn);
  REQUIRE(rows % 32 == 0 && cols % 32 == 0, "%s: rows and cols must be multiples of 32 (got %lld x %lld)", fn,
          (long long)rows, (long long)cols);
  const int64_t tiles = size_mul(rows / 32 + 1, cols / 256 + 1);
  REQUIRE(tiles >= 0 && tiles < ((int64_t)1 << 30), "%s: too many tiles", fn);
  const int64_t n = rows * cols;
  REQUIRE_BUF("input", input, n, n);
  REQUIRE_BUF("row_q", row_q, row_q_bytes, n / 2);
  REQUIRE_BUF("row_s", row_s, row_s_bytes, n / 32);
  REQUIRE_BUF("col_q", col_q, col_q_bytes, n / 2);
  REQUIRE_BUF("col_s", col_s, col_s_bytes, n / 32);
  REQUIRE(aligned(input, 16) && aligned(col_q, 16) && aligned(row_q, 4), "%s: misaligned buffer", fn);
  return OMO_OK;
}

}  // namespace

extern "C" {

int omo_hip_abi_version(void) { return OMO_ABI_VERSION; }

const char* omo_hip_status_string(int status) {
  switch (status) {
    case OMO_OK: return "ok";
    case OMO_ERR_INVALID_ARGUMENT: return "invalid argument";
    case OMO_ERR_UNSUPPORTED: return "unsupported";
    case OMO_ERR_HIP: return "HIP error";
    default: return "unknown status";
  }
}

const char* omo_hip_last_error(void) { return g_err; }

int omo_hip_per_token_group_quant_fp4(const void* input, int64_t numel, void* output_q, int64_t output_q_bytes,
                                      void* output_s, int64_t output_s_bytes, int group_size, float eps,
                                      float fp4_min, float fp4_max, int scale_ue8m0, void* stream) {
  const char* fn = "omo_per_token_group_quant_fp4";
  REQUIRE(group_size > 0, "%s: group_size must be positive", fn);
  REQUIRE(numel >= 0 && numel % group_size == 0, "%s: input.numel() %% group_size != 0", fn);
  if (scale_ue8m0)
    return fail(OMO_ERR_UNSUPPORTED, "%s: scale_ue8m0 (column-major int32 scales) is not supported", fn);
  if (group_size != 32)
    return fail(OMO_ERR_UNSUPPORTED, "%s: group_size must be 32 (MXFP4 blocks), got %d", fn, group_size);
  REQUIRE(std::isfinite(eps) && std::isfinite(fp4_min) && std::isfinite(fp4_max) && fp4_max > 0.0f,
          "%s: eps, fp4_min, fp4_max must be finite and fp4_max > 0", fn);
  REQUIRE_BUF("input", input, numel, numel);
  REQUIRE_BUF("output_q", output_q, output_q_bytes, numel / 2);
  REQUIRE_BUF("output_s", output_s, output_s_bytes, numel / 32);
  REQUIRE(aligned(input, 16) && aligned(output_q, 4), "%s: input must be 16-byte and output_q 4-byte aligned", fn);
  if (numel == 0) return ok();
  return from_hip(omo_hip::launch_quant_rowwise(input, output_q, output_s, numel, eps, fp4_min, fp4_max,
                                                as_stream(stream)),
                  fn);
}

int omo_hip_per_token_Mxfp4ToBf16_dequant(const void* input, int64_t input_bytes, const void* input_s,
                                          int64_t input_s_bytes, void* output_q, int64_t output_q_elems,
                                          void* output_s, int64_t output_s_bytes, int group_size, float eps,
                                          float fp4_min, float fp4_max, int scale_ue8m0, void* stream) {
  const char* fn = "omo_per_token_Mxfp4ToBf16_dequant";
  (void)output_s; (void)output_s_bytes; (void)group_size; (void)eps; (void)fp4_min; (void)fp4_max;
  if (scale_ue8m0) return fail(OMO_ERR_UNSUPPORTED, "%s: scale_ue8m0 is not supported (the reference asserts it off)", fn);
  REQUIRE(input_bytes >= 0 && input_bytes % 128 == 0, "%s: input.numel() %% 128 != 0", fn);
  REQUIRE(input_bytes <= kMaxSize, "%s: shape too large", fn);
  REQUIRE_BUF("input", input, input_bytes, input_bytes);
  REQUIRE_BUF("input_s", input_s, input_s_bytes, input_bytes / 16);
  REQUIRE_BUF("output_q", output_q, output_q_elems, 2 * input_bytes);
  REQUIRE(aligned(input, 4) && aligned(output_q, 16), "%s: input must be 4-byte and output_q 16-byte aligned", fn);
  if (input_bytes == 0) return ok();
  return from_hip(omo_hip::launch_dequant_bf16(input, input_s, output_q, input_bytes, as_stream(stream)), fn);
}

int omo_hip_per_token_Mxfp4ToFp8(const void* input, int64_t rows, int64_t row_bytes, const void* input_s,
                                 int64_t input_s_bytes, void* output_q, int64_t output_q_bytes, void* output_s,
                                 int64_t output_s_elems, int group_size, float eps, float fp4_min, float fp4_max,
                                 int scale_ue8m0, void* stream) {
  (void)group_size; (void)eps; (void)fp4_min; (void)fp4_max;
  return requant_rowwise("omo_per_token_Mxfp4ToFp8", input, rows, row_bytes, input_s, input_s_bytes, output_q,
                         output_q_bytes, output_s, output_s_elems, scale_ue8m0, stream);
}

int omo_hip_per_token_Mxfp4ToBf16ToFp8(const void* input, int64_t rows, int64_t row_bytes, const void* input_s,
                                       int64_t input_s_bytes, void* output_q, int64_t output_q_bytes, void* output_s,
                                       int64_t output_s_elems, int group_size, float eps, float fp4_min,
                                       float fp4_max, int scale_ue8m0, void* stream) {
  (void)group_size; (void)eps; (void)fp4_min; (void)fp4_max;
  return requant_rowwise("omo_per_token_Mxfp4ToBf16ToFp8", input, rows, row_bytes, input_s, input_s_bytes, output_q,
                         output_q_bytes, output_s, output_s_elems, scale_ue8m0, stream);
}

int omo_hip_per_token_Mxfp4ToFp8_col(const void* input, int64_t rows, int64_t row_bytes, const void* input_s,
                                     int64_t input_s_bytes, void* output_q, int64_t output_q_bytes, void* output_s,
                                     int64_t output_s_elems, int group_size, float eps, float fp4_min, float fp4_max,
                                     int scale_ue8m0, void* stream) {
  const char* fn = "omo_per_token_Mxfp4ToFp8_col";
  (void)group_size; (void)fp4_min; (void)fp4_max;
  int rc = check_requant_common(fn, input, rows, row_bytes, scale_ue8m0);
  if (rc != OMO_OK) return rc;
  REQUIRE(rows % 128 == 0 && row_bytes % 128 == 0,
          "%s: rows and row bytes must be multiples of 128 (got %lld x %lld); the reference reads whole "
          "128x128-byte tiles without bounds checks", fn, (long long)rows, (long long)row_bytes);
  REQUIRE(!std::isnan(eps), "%s: eps is NaN", fn);
  const int64_t n = rows * row_bytes;
  REQUIRE_BUF("input", input, n, n);
  REQUIRE_BUF("input_s", input_s, input_s_bytes, n / 16);
  REQUIRE_BUF("output_q", output_q, output_q_bytes, 2 * n);
  REQUIRE_BUF("output_s", output_s, output_s_elems, (rows / 128) * 2 * row_bytes);
  REQUIRE(aligned(input, 16) && aligned(input_s, 8) && aligned(output_q, 16) && aligned(output_s, 4),
          "%s: input/output_q need 16-byte, input_s 8-byte alignment", fn);
  if (n == 0) return ok();
  return from_hip(omo_hip::launch_mxfp4_to_fp8_col(input, input_s, output_q, static_cast<float*>(output_s), rows,
                                                   row_bytes, eps, as_stream(stream)),
                  fn);
}

int omo_hip_per_token_Mxfp4RowToBf16ToFp8Col(const void* input, int64_t rows, int64_t row_bytes, const void* input_s,
                                             int64_t input_s_rows, int64_t input_s_cols, void* output_q,
                                             int64_t output_q_rows, int64_t output_q_cols, void* output_s,
                                             int64_t output_s_rows, int64_t output_s_cols, float eps, void* stream) {
  const char* fn = "omo_per_token_Mxfp4RowToBf16ToFp8Col";
  REQUIRE(rows >= 0 && row_bytes >= 0, "%s: negative shape", fn);
  REQUIRE(row_bytes <= kMaxSize / 2 && size_mul(rows, 2 * row_bytes) >= 0, "%s: shape too large", fn);
  const int64_t M = rows, N = row_bytes * 2;
  // the shape checks of per_token_Mxfp4RowToBf16ToFp8Col.cu:219-224
  REQUIRE(input_s_rows == M, "%s: input_s.size(0) != M", fn);
  REQUIRE(input_s_cols == (N + 31) / 32, "%s: input_s.size(1) != ceil(N/32)", fn);
  REQUIRE(output_q_rows == N && output_q_cols == M, "%s: output_q must be [N, M]", fn);
  REQUIRE(output_s_rows == (M + 127) / 128 && output_s_cols == N, "%s: output_s must be [ceil(M/128), N]", fn);
  REQUIRE(!std::isnan(eps), "%s: eps is NaN", fn);
  REQUIRE_BUF("input", input, M * row_bytes, M * row_bytes);
  REQUIRE_BUF("input_s", input_s, input_s_rows * input_s_cols, M * ((N + 31) / 32));
  REQUIRE_BUF("output_q", output_q, output_q_rows * output_q_cols, N * M);
  REQUIRE_BUF("output_s", output_s, output_s_rows * output_s_cols, ((M + 127) / 128) * N);
  REQUIRE(aligned(output_s, 4), "%s: output_s must be 4-byte aligned", fn);
  if (M == 0 || N == 0) return ok();
  return from_hip(omo_hip::launch_row_to_fp8_col(input, input_s, output_q, static_cast<float*>(output_s), M, N, eps,
                                                 as_stream(stream)),
                  fn);
}

int omo_hip_per_token_Mxfp4RowToBf16ToFp8Col_msplit(const void* input, int64_t rows, int64_t row_bytes,
                                                    const void* input_s, int64_t input_s_bytes, void* output_q,
                                                    int64_t output_q_bytes, void* output_s, int64_t output_s_elems,
                                                    const int32_t* m_splits, const int32_t* split_offsets,
                                                    const int32_t* scale_offsets, int64_t num_splits,
                                                    int64_t max_split_len, float eps, void* stream) {
  const char* fn = "omo_per_token_Mxfp4RowToBf16ToFp8Col_msplit";
  REQUIRE(rows >= 0 && row_bytes >= 0 && num_splits >= 0 && max_split_len >= 0, "%s: negative shape", fn);
  REQUIRE(num_splits <= 65535, "%s: at most 65535 splits", fn);
  REQUIRE(!std::isnan(eps), "%s: eps is NaN", fn);
  REQUIRE(row_bytes <= kMaxSize / 2 && size_mul(rows, 2 * row_bytes) >= 0, "%s: shape too large", fn);
  const int64_t M = rows, N = row_bytes * 2;
  // Every split the kernel converts lies inside the M rows, so a longer
  // max_split_len only adds workgroups that exit at once.
  if (max_split_len > M) max_split_len = M;
  REQUIRE_BUF("input", input, M * row_bytes, M * row_bytes);
  // the kernel reads scale byte row*(N/32) + col/32 for rows < M, cols < N
  const int64_t s_need = M == 0 || N == 0 ? 0 : (M - 1) * (N / 32) + (N - 1) / 32 + 1;
  REQUIRE_BUF("input_s", input_s, input_s_bytes, s_need);
  REQUIRE_BUF("output_q", output_q, output_q_bytes, M * N);
  REQUIRE(output_s_elems >= 0 && (output_s_elems == 0 || output_s != nullptr), "%s: output_s", fn);
  REQUIRE(num_splits == 0 || (m_splits && split_offsets && scale_offsets), "%s: null split metadata", fn);
  REQUIRE(aligned(output_s, 4) && aligned(m_splits, 4) && aligned(split_offsets, 4) && aligned(scale_offsets, 4),
          "%s: misaligned buffer", fn);
  if (num_splits == 0 || N == 0) return ok();
  const int64_t out_s_rows = output_s_elems / N;
  return from_hip(omo_hip::launch_row_to_fp8_col_msplit(input, input_s, output_q, static_cast<float*>(output_s), M, N,
                                                        m_splits, split_offsets, scale_offsets, num_splits,
                                                        max_split_len, output_q_bytes, out_s_rows, eps,
                                                        as_stream(stream)),
                  fn);
}

int omo_hip_quant_mxfp4_dual(const void* input, int64_t rows, int64_t cols, void* row_q, int64_t row_q_bytes,
                             void* row_s, int64_t row_s_bytes, void* col_q, int64_t col_q_bytes, void* col_s,
                             int64_t col_s_bytes, float eps, void* stream) {
  const char* fn = "omo_quant_mxfp4_dual";
  REQUIRE(std::isfinite(eps), "%s: eps must be finite", fn);
  int rc = check_dual(fn, input, rows, cols, row_q, row_q_bytes, row_s, row_s_bytes, col_q, col_q_bytes, col_s,
                      col_s_bytes);
  if (rc != OMO_OK) return rc;
  if (rows == 0 || cols == 0) return ok();
  return from_hip(omo_hip::launch_quant_dual(input, row_q, row_s, col_q, col_s, rows, cols, eps, as_stream(stream)),
                  fn);
}

int omo_hip_quant_mxfp4_dual_grouped(const omo_dual_item* items, int64_t count, float eps, void* stream) {
  const char* fn = "omo_quant_mxfp4_dual_grouped";
  REQUIRE(count >= 0 && count <= ((int64_t)1 << 20), "%s: bad item count %lld", fn, (long long)count);
  REQUIRE(count == 0 || items != nullptr, "%s: items: null pointer", fn);
  REQUIRE(std::isfinite(eps), "%s: eps must be finite", fn);
  std::vector<omo_hip::DualSpec> specs;
  specs.reserve((size_t)count);
  int64_t tiles = 0;
  for (int64_t i = 0; i < count; i++) {
    const omo_dual_item& it = items[i];
    int rc = check_dual(fn, it.input, it.rows, it.cols, it.row_q, it.row_q_bytes, it.row_s, it.row_s_bytes, it.col_q,
                        it.col_q_bytes, it.col_s, it.col_s_bytes);
    if (rc != OMO_OK) {
      char item_msg[64];
      snprintf(item_msg, sizeof(item_msg), " (item %lld)", (long long)i);
      strncat(g_err, item_msg, sizeof(g_err) - strlen(g_err) - 1);
      return rc;
    }
    specs.push_back({it.input, it.row_q, it.row_s, it.col_q, it.col_s, it.rows, it.cols});
    tiles += (it.rows / 32 + 1) * (it.cols / 256 + 1);
  }
  REQUIRE(tiles < ((int64_t)1 << 30), "%s: too many tiles", fn);
  if (count == 0) return ok();
  return from_hip(omo_hip::launch_quant_dual_grouped(specs.data(), (int)count, eps, as_stream(stream)), fn);
}

int omo_hip_quant_mxfp4_packed(const void* input, int64_t rows, int64_t cols, void* output, int64_t output_bytes,
                               float eps, void* stream) {
  const char* fn = "omo_quant_mxfp4_packed";
  int rc = check_packed(fn, rows, cols);
  if (rc != OMO_OK) return rc;
  REQUIRE(std::isfinite(eps), "%s: eps must be finite", fn);
  const int64_t stride = cols / 32 * 17;
  REQUIRE_BUF("input", input, rows * cols, rows * cols);
  REQUIRE_BUF("output", output, output_bytes, rows * stride);
  REQUIRE(aligned(input, 16) && aligned(output, 4), "%s: input must be 16-byte and output 4-byte aligned", fn);
  if (rows == 0 || cols == 0) return ok();
  uint8_t* out = static_cast<uint8_t*>(output);
  return from_hip(omo_hip::launch_quant_rows(input, out, stride, out + cols / 2, stride, rows, cols, eps,
                                             as_stream(stream)),
                  fn);
}

int omo_hip_packed_Mxfp4ToBf16_dequant(const void* input, int64_t rows, int64_t cols, void* output,
                                       int64_t output_elems, void* stream) {
  const char* fn = "omo_packed_Mxfp4ToBf16_dequant";
  int rc = check_packed(fn, rows, cols);
  if (rc != OMO_OK) return rc;
  const int64_t stride = cols / 32 * 17;
  REQUIRE_BUF("input", input, rows * stride, rows * stride);
  REQUIRE_BUF("output", output, output_elems, rows * cols);
  REQUIRE(aligned(input, 4) && aligned(output, 16), "%s: input must be 4-byte and output 16-byte aligned", fn);
  if (rows == 0 || cols == 0) return ok();
  const uint8_t* in = static_cast<const uint8_t*>(input);
  return from_hip(omo_hip::launch_dequant_rows(in, stride, in + cols / 2, stride, output, rows, cols,
                                               as_stream(stream)),
                  fn);
}

int omo_hip_packed_Mxfp4ToFp8(const void* input, int64_t rows, int64_t cols, void* output_q, int64_t output_q_bytes,
                              void* output_s, int64_t output_s_elems, void* stream) {
  const char* fn = "omo_packed_Mxfp4ToFp8";
  int rc = check_packed(fn, rows, cols);
  if (rc != OMO_OK) return rc;
  REQUIRE(rows < ((int64_t)1 << 32) && cols / 128 * rows < ((int64_t)1 << 31), "%s: too many groups", fn);
  const int64_t stride = cols / 32 * 17;
  REQUIRE_BUF("input", input, rows * stride, rows * stride);
  REQUIRE_BUF("output_q", output_q, output_q_bytes, rows * cols);
  REQUIRE_BUF("output_s", output_s, output_s_elems, rows * (cols / 128));
  REQUIRE(aligned(input, 4) && aligned(output_q, 16) && aligned(output_s, 4),
          "%s: input needs 4-byte, output_q 16-byte, output_s 4-byte alignment", fn);
  if (rows == 0 || cols == 0) return ok();
  const uint8_t* in = static_cast<const uint8_t*>(input);
  return from_hip(omo_hip::launch_mxfp4_to_fp8_rows(in, stride, in + cols / 2, stride, nullptr, rows, output_q,
                                                    static_cast<float*>(output_s), rows, cols / 2,
                                                    as_stream(stream)),
                  fn);
}

int omo_hip_mxfp4_permute_rows(const void* codes, int64_t codes_bytes, int64_t code_stride, const void* scales,
                               int64_t scales_bytes, int64_t scale_stride, int64_t num_tokens, int64_t cols,
                               const int32_t* src_rows, int64_t num_out, void* out_codes, int64_t out_codes_bytes,
                               void* out_scales, int64_t out_scales_bytes, void* stream) {
  const char* fn = "omo_mxfp4_permute_rows";
  int rc = check_permute(fn, codes, codes_bytes, code_stride, scales, scales_bytes, scale_stride, num_tokens, cols,
                         src_rows, num_out);
  if (rc != OMO_OK) return rc;
  REQUIRE_BUF("out_codes", out_codes, out_codes_bytes, num_out * (cols / 2));
  REQUIRE_BUF("out_scales", out_scales, out_scales_bytes, num_out * (cols / 32));
  if (num_out == 0 || cols == 0) return ok();
  return from_hip(omo_hip::launch_gather_rows(codes, code_stride, cols / 2, scales, scale_stride, cols / 32,
                                              src_rows, num_tokens, num_out, out_codes, out_scales,
                                              as_stream(stream)),
                  fn);
}

int omo_hip_permute_Mxfp4ToFp8(const void* codes, int64_t codes_bytes, int64_t code_stride, const void* scales,
                               int64_t scales_bytes, int64_t scale_stride, int64_t num_tokens, int64_t cols,
                               const int32_t* src_rows, int64_t num_out, void* output_q, int64_t output_q_bytes,
                               void* output_s, int64_t output_s_elems, void* stream) {
  const char* fn = "omo_permute_Mxfp4ToFp8";
  int rc = check_permute(fn, codes, codes_bytes, code_stride, scales, scales_bytes, scale_stride, num_tokens, cols,
                         src_rows, num_out);
  if (rc != OMO_OK) return rc;
  REQUIRE(cols % 128 == 0, "%s: cols must be a multiple of 128 (got %lld)", fn, (long long)cols);
  REQUIRE(code_stride % 4 == 0 && scale_stride % 4 == 0 && aligned(codes, 4) && aligned(scales, 4),
          "%s: code and scale rows must be 4-byte aligned", fn);
  REQUIRE(cols / 128 * num_out < ((int64_t)1 << 31), "%s: too many groups", fn);
  REQUIRE_BUF("output_q", output_q, output_q_bytes, num_out * cols);
  REQUIRE_BUF("output_s", output_s, output_s_elems, num_out * (cols / 128));
  REQUIRE(aligned(output_q, 16) && aligned(output_s, 4), "%s: output_q needs 16-byte, output_s 4-byte alignment",
          fn);
  if (num_out == 0 || cols == 0) return ok();
  return from_hip(omo_hip::launch_mxfp4_to_fp8_rows(codes, code_stride, scales, scale_stride, src_rows, num_tokens,
                                                    output_q, static_cast<float*>(output_s), num_out, cols / 2,
                                                    as_stream(stream)),
                  fn);
}

}  // extern "C"
