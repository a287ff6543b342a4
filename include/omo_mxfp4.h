/*
 * omo_mxfp4.h -- C ABI of the MI355X (gfx950) MXFP4 quantize / dequantize /
 * requantize library (libomo_mxfp4.so).
 *
 * Every entry point replaces one host function of the reference's `omo`
 * torch extension (paths relative to the reference repository root) and
 * keeps its argument order; tensors become (pointer, size) pairs. All
 * buffers are device memory allocated by the caller; the library never
 * allocates and never synchronizes. Work is enqueued on `stream` (a
 * hipStream_t, NULL = the default stream) and is asynchronous, like the
 * reference's launches on the current CUDA stream.
 *
 * Every function validates its arguments before touching the GPU and
 * returns OMO_OK or a negative status; omo_hip_last_error() then describes
 * the failure (thread-local). Sizes are element counts unless named
 * *_bytes; products of sizes are formed without wrapping, and a shape whose
 * byte count passes 2^60 is refused. Data layouts (bit patterns) are those of the reference:
 *   bf16      : 16-bit patterns, row-major
 *   codes     : uint8, two E2M1 nibbles per byte, element 2j in the low nibble
 *   scales    : uint8 E8M0, byte s means 2^(s-127), one per 32 elements
 *   fp8       : uint8 OCP E4M3 (torch.float8_e4m3fn)
 *   fp32      : IEEE binary32
 */
#ifndef OMO_MXFP4_H
#define OMO_MXFP4_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OMO_OK 0
#define OMO_ERR_INVALID_ARGUMENT (-1) /* shape, size, alignment or value check failed */
#define OMO_ERR_UNSUPPORTED (-2)      /* a mode the reference kernels do not implement */
#define OMO_ERR_HIP (-3)              /* the HIP runtime reported an error at launch */

#define OMO_ABI_VERSION 1

#if defined(__GNUC__)
#define OMO_API __attribute__((visibility("default")))
#else
#define OMO_API
#endif

OMO_API int omo_hip_abi_version(void);
OMO_API const char* omo_hip_status_string(int status);
OMO_API const char* omo_hip_last_error(void);

/* BF16 -> MXFP4 rowwise quantize of a flat tensor in 1x32 blocks.
 * Replaces omo::omo_per_token_group_quant_fp4
 * (code/kernel/per_token_quant_mxfp4.cu:387-487; binding code/kernel/ops.cu:28-29).
 * input: numel bf16 (16-byte aligned); output_q: numel/2 bytes (4-byte aligned);
 * output_s: numel/32 bytes in flat block order. group_size must be 32 and
 * scale_ue8m0 0 (the reference's row-major launch path, :429-473). */
OMO_API int omo_hip_per_token_group_quant_fp4(const void* input, int64_t numel, void* output_q, int64_t output_q_bytes,
                                      void* output_s, int64_t output_s_bytes, int group_size, float eps,
                                      float fp4_min, float fp4_max, int scale_ue8m0, void* stream);

/* MXFP4 -> BF16 dequant of a flat code tensor.
 * Replaces omo::omo_per_token_Mxfp4ToBf16_dequant
 * (code/kernel/per_token_Mxfp4ToBf16_dequant.cu:164-238; binding code/kernel/ops.cu:30-31).
 * input: input_bytes codes (multiple of 128, 4-byte aligned); input_s:
 * input_bytes/16 scale bytes; output_q: 2*input_bytes bf16 (16-byte aligned).
 * output_s is accepted and left untouched, as in the reference; group_size,
 * eps, fp4_min, fp4_max are ignored (the reference forces group 128, :179). */
OMO_API int omo_hip_per_token_Mxfp4ToBf16_dequant(const void* input, int64_t input_bytes, const void* input_s,
                                          int64_t input_s_bytes, void* output_q, int64_t output_q_elems,
                                          void* output_s, int64_t output_s_bytes, int group_size, float eps,
                                          float fp4_min, float fp4_max, int scale_ue8m0, void* stream);

/* MXFP4 -> FP8 E4M3 rowwise requant with 1x128 power-of-two fp32 scales
 * stored transposed [row_bytes/64, rows].
 * Replaces omo::omo_per_token_Mxfp4ToFp8 (code/kernel/per_token_Mxfp4ToFp8.cu:238-309,
 * declared code/kernel/per_token_Mxfp4ToFp8.h:6; imported by
 * code/kernel/api/mxfp4_dequant.py:1).
 * input: [rows, row_bytes] codes, row_bytes % 64 == 0 (8-byte aligned); input_s:
 * rows*row_bytes/16 bytes; output_q: [rows, 2*row_bytes] fp8 (16-byte aligned);
 * output_s: rows*row_bytes/64 floats. */
OMO_API int omo_hip_per_token_Mxfp4ToFp8(const void* input, int64_t rows, int64_t row_bytes, const void* input_s,
                                 int64_t input_s_bytes, void* output_q, int64_t output_q_bytes, void* output_s,
                                 int64_t output_s_elems, int group_size, float eps, float fp4_min, float fp4_max,
                                 int scale_ue8m0, void* stream);

/* Bound as omo_per_token_Mxfp4ToBf16ToFp8 (code/kernel/ops.cu:32-33) and
 * called by code/kernel/api/mxfp4_dequant.py:116 with the same signature as
 * omo_per_token_Mxfp4ToFp8; the reference ships no source for it. Same
 * computation as omo_hip_per_token_Mxfp4ToFp8. */
OMO_API int omo_hip_per_token_Mxfp4ToBf16ToFp8(const void* input, int64_t rows, int64_t row_bytes, const void* input_s,
                                       int64_t input_s_bytes, void* output_q, int64_t output_q_bytes, void* output_s,
                                       int64_t output_s_elems, int group_size, float eps, float fp4_min,
                                       float fp4_max, int scale_ue8m0, void* stream);

/* MXFP4 rowwise -> FP8 transposed [2*row_bytes, rows] with 128-row
 * power-of-two scales [rows/128, 2*row_bytes] (sign dropped, as the reference).
 * Replaces omo::omo_per_token_Mxfp4ToFp8_col
 * (code/kernel/per_token_Mxfp4ToFp8_col.cu:305-384; binding code/kernel/ops.cu:40-41).
 * rows % 128 == 0 and row_bytes % 128 == 0 (the reference kernel has no
 * bounds checks); input and output_q 16-byte aligned, input_s 8-byte aligned. */
OMO_API int omo_hip_per_token_Mxfp4ToFp8_col(const void* input, int64_t rows, int64_t row_bytes, const void* input_s,
                                     int64_t input_s_bytes, void* output_q, int64_t output_q_bytes, void* output_s,
                                     int64_t output_s_elems, int group_size, float eps, float fp4_min, float fp4_max,
                                     int scale_ue8m0, void* stream);

/* MXFP4 rowwise -> fp32 -> FP8 columnwise [N, M] with per-(128 rows, column)
 * scale_inv = amax/448 [ceil(M/128), N] (TE GEMM_READY columnwise).
 * Replaces omo::omo_per_token_Mxfp4RowToBf16ToFp8Col
 * (code/kernel/per_token_Mxfp4RowToBf16ToFp8Col.cu:204-246; binding code/kernel/ops.cu:36-37).
 * input [rows=M, row_bytes=N/2]; input_s [M, ceil(N/32)]; output_q [N, M];
 * output_s [ceil(M/128), N]; the shape checks are those of :211-224. */
OMO_API int omo_hip_per_token_Mxfp4RowToBf16ToFp8Col(const void* input, int64_t rows, int64_t row_bytes, const void* input_s,
                                             int64_t input_s_rows, int64_t input_s_cols, void* output_q,
                                             int64_t output_q_rows, int64_t output_q_cols, void* output_s,
                                             int64_t output_s_rows, int64_t output_s_cols, float eps, void* stream);

/* Grouped (per-expert) variant with power-of-two scales. m_splits,
 * split_offsets and scale_offsets are int32 device arrays of num_splits
 * entries; split i's output is a contiguous [N, m_splits[i]] block at
 * split_offsets[i]*N. The metadata stays on the device, so the host cannot
 * check it: tiles whose metadata points outside the buffers (split_offsets[i]
 * + m_splits[i] > rows, or scale_offsets[i] + ceil(m_splits[i]/128) >
 * output_s rows) are skipped on the device, that split's output is then left
 * partly or wholly unwritten, and the call still returns OMO_OK. Callers
 * building the arrays on the host check those two bounds first (the Python
 * wrapper derives them from m_splits, where they hold by construction).
 * Replaces omo::omo_per_token_Mxfp4RowToBf16ToFp8Col_msplit
 * (code/kernel/per_token_Mxfp4RowToBf16ToFp8Col_msplit.cu:232-283; binding code/kernel/ops.cu:38-39). */
OMO_API int omo_hip_per_token_Mxfp4RowToBf16ToFp8Col_msplit(const void* input, int64_t rows, int64_t row_bytes,
                                                    const void* input_s, int64_t input_s_bytes, void* output_q,
                                                    int64_t output_q_bytes, void* output_s, int64_t output_s_elems,
                                                    const int32_t* m_splits, const int32_t* split_offsets,
                                                    const int32_t* scale_offsets, int64_t num_splits,
                                                    int64_t max_split_len, float eps, void* stream);

/* Fused dual-layout BF16 -> MXFP4 quantize: rowwise codes [rows, cols/2] +
 * scales [rows, cols/32] and columnwise codes [cols, rows/2] + scales
 * [cols, rows/32], the latter equal to the rowwise quantize of the transpose.
 * Replaces the two-pass columnwise path of TE's _QuantizeFunc.forward
 * (code/transformer_engine-2.8.diff:1463-1466: mxfp4_quant(tensor) and
 * mxfp4_quant(tensor.T.contiguous())). rows % 32 == 0, cols % 32 == 0; input
 * and col_q 16-byte aligned, row_q 4-byte aligned; fp4 range fixed to +-6. */
OMO_API int omo_hip_quant_mxfp4_dual(const void* input, int64_t rows, int64_t cols, void* row_q, int64_t row_q_bytes,
                             void* row_s, int64_t row_s_bytes, void* col_q, int64_t col_q_bytes, void* col_s,
                             int64_t col_s_bytes, float eps, void* stream);

/* One tensor of a grouped dual-layout quantize (host struct; pointers are
 * device memory; sizes as in omo_hip_quant_mxfp4_dual). */
typedef struct omo_dual_item {
  const void* input;
  int64_t rows, cols;
  void* row_q;
  int64_t row_q_bytes;
  void* row_s;
  int64_t row_s_bytes;
  void* col_q;
  int64_t col_q_bytes;
  void* col_s;
  int64_t col_s_bytes;
} omo_dual_item;

/* omo_hip_quant_mxfp4_dual over `count` tensors in one launch (per 32
 * tensors), e.g. the gate/up/down weights of all local experts, which TE
 * quantizes one GEMM at a time (code/transformer_engine-2.8.diff:1463-1466
 * per tensor). Each item is validated like the single-tensor call; outputs
 * are identical to `count` separate calls. `items` is host memory. */
OMO_API int omo_hip_quant_mxfp4_dual_grouped(const omo_dual_item* items, int64_t count, float eps, void* stream);

/* Expert-parallel payload rows (code/megatron-0.15.0rc7.diff:32-63): row t
 * of a [rows, 17*cols/32] uint8 tensor holds the row's MXFP4 codes (cols/2
 * bytes) followed by its E8M0 scales (cols/32 bytes), the layout Megatron
 * builds with torch.cat before the DeepEP dispatch and splits again with two
 * .contiguous() copies after it. The three functions below write or read
 * that layout in place. cols % 128 == 0 (dword-aligned rows).
 *
 * Quantize straight into payload rows. Replaces MXFP4Quantizer's quantize
 * (omo_per_token_group_quant_fp4, code/kernel/ops.cu:28-29) followed by
 * _pack_rowwise_components (code/megatron-0.15.0rc7.diff:93-99, called at
 * :163-170). input [rows, cols] bf16 (16-byte aligned); output
 * rows*17*cols/32 bytes (4-byte aligned); fp4 range fixed to +-6. */
OMO_API int omo_hip_quant_mxfp4_packed(const void* input, int64_t rows, int64_t cols, void* output,
                                       int64_t output_bytes, float eps, void* stream);

/* MXFP4 -> BF16 dequant of payload rows into [rows, cols] bf16 (16-byte
 * aligned). Replaces _unpack_rowwise_components (code/megatron-0.15.0rc7.diff:101-122)
 * followed by omo_per_token_Mxfp4ToBf16_dequant (code/kernel/ops.cu:30-31).
 * input 4-byte aligned. */
OMO_API int omo_hip_packed_Mxfp4ToBf16_dequant(const void* input, int64_t rows, int64_t cols, void* output,
                                               int64_t output_elems, void* stream);

/* MXFP4 -> FP8 E4M3 rowwise requant of payload rows: output_q [rows, cols]
 * fp8 (16-byte aligned) and output_s [cols/128, rows] fp32, the outputs of
 * omo_per_token_Mxfp4ToFp8 (code/kernel/per_token_Mxfp4ToFp8.cu:86-309) on the
 * unpacked tensors. Replaces _unpack_rowwise_components
 * (code/megatron-0.15.0rc7.diff:101-122) followed by that requant. input
 * 4-byte aligned. */
OMO_API int omo_hip_packed_Mxfp4ToFp8(const void* input, int64_t rows, int64_t cols, void* output_q,
                                      int64_t output_q_bytes, void* output_s, int64_t output_s_elems, void* stream);

/* MXFP4 row permutation: the data movement of TE's moe_permute for MXFP4
 * inputs (code/transformer_engine-2.8.diff:256-261, 338-354), which permutes
 * the code rows [T, cols/2] and scale rows [T, cols/32] into expert-major
 * order. Output row r of out_codes [num_out, cols/2] and out_scales
 * [num_out, cols/32] is input row src_rows[r] (int32 device array, num_out
 * entries); an index outside [0, num_tokens) gives a zero row. Input rows
 * are code_stride / scale_stride bytes apart (payload rows can be read in
 * place); codes_bytes / scales_bytes bound the input buffers. cols % 32 == 0. */
OMO_API int omo_hip_mxfp4_permute_rows(const void* codes, int64_t codes_bytes, int64_t code_stride,
                                       const void* scales, int64_t scales_bytes, int64_t scale_stride,
                                       int64_t num_tokens, int64_t cols, const int32_t* src_rows, int64_t num_out,
                                       void* out_codes, int64_t out_codes_bytes, void* out_scales,
                                       int64_t out_scales_bytes, void* stream);

/* The permutation fused with the FP8 E4M3 rowwise requant: output_q
 * [num_out, cols] fp8 (16-byte aligned) and output_s [cols/128, num_out]
 * fp32 equal omo_per_token_Mxfp4ToFp8 (code/kernel/per_token_Mxfp4ToFp8.cu:86-309)
 * applied to the permuted rows, zero rows included. cols % 128 == 0; code and
 * scale rows 4-byte aligned. */
OMO_API int omo_hip_permute_Mxfp4ToFp8(const void* codes, int64_t codes_bytes, int64_t code_stride,
                                       const void* scales, int64_t scales_bytes, int64_t scale_stride,
                                       int64_t num_tokens, int64_t cols, const int32_t* src_rows, int64_t num_out,
                                       void* output_q, int64_t output_q_bytes, void* output_s,
                                       int64_t output_s_elems, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* OMO_MXFP4_H */
