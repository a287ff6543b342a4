// MXFP4 rowwise -> fp32 -> FP8 E4M3 columnwise (TE "GEMM_READY" layout).
//
// Dense semantics follow omo_per_token_Mxfp4RowToBf16ToFp8Col_kernel
// (code/kernel/per_token_Mxfp4RowToBf16ToFp8Col.cu:39-197) on 128x128 tiles:
//   v[r][c]  = bf16(code) * bf16(s << 7), fp32, 0 outside the tensor  :98-127
//   amax[c]  = fmaxf(eps, |v[r][c]|) over the tile's 128 rows          :131-138
//   out_s    = amax / 448 at [tile_m * N + c]                          :142
//   q        = v * (amax > 1e-9 ? 448 / amax : 0), clamped, E4M3 RNE  :159-178
//   out      = [c * M + r]                                             :181-195
// The reference has no barrier between the LDS writes of the dequantized
// tile and the amax reads of other threads (:126 -> :131); the intended,
// barriered semantics are implemented (every value is seen by the amax).
//
// Grouped semantics follow omo_per_token_Mxfp4RowToBf16ToFp8Col_split_kernel
// (code/kernel/per_token_Mxfp4RowToBf16ToFp8Col_msplit.cu:48-224): per split
// i the rows [off_i, off_i + len_i) form their own tiles, the amax is seeded
// with 0, the scale is the power of two of compute_te_pow2_scale (:23-43),
// out_s = 1/scale at [(soff_i + tile) * N + c], q = v * scale, and the
// split's output block [N, len_i] starts at off_i * N.
//
// Both kernels stage the tile's code bytes (8 KiB) and scale bytes in LDS
// and recompute v from them; each thread owns one output column segment of
// 64 rows so the FP8 stores are 16 B vectors along M.
#include "omo_device.cuh"
#include "omo_internal.h"

namespace omo_hip {

constexpr int kTile = 128;
constexpr int kCodePitch = 64 + 4;  // code bytes per tile row (+pad)

struct TileSmem {
  uint8_t codes[kTile * kCodePitch];
  uint8_t scales[kTile][4];
  float part[2][kTile];
  float mult[kTile];
};

// Stage the codes/scales of tile rows [row0, row0 + rows_valid) and element
// columns [col0, col0 + 128) into LDS; out-of-range bytes become 0.
__device__ __forceinline__ void stage_tile(TileSmem& sm, const uint8_t* __restrict__ q, const uint8_t* __restrict__ s,
                                           int64_t N, int64_t row0, int rows_valid, int64_t col0, bool vec_ok) {
  const int t = threadIdx.x;
  const int64_t half = N / 2, sstride = N / 32;
#pragma unroll
  for (int k = 0; k < 2; k++) {
    const int cidx = t + 256 * k;  // 512 chunks of 16 code bytes
    const int r = cidx >> 2, c16 = cidx & 3;
    const int64_t gcol = col0 + c16 * 32;  // first element of the chunk
    uint32_t w[4] = {0u, 0u, 0u, 0u};
    if (r < rows_valid && gcol < N) {
      const uint8_t* src = q + (row0 + r) * half + gcol / 2;
      if (vec_ok && gcol + 32 <= N) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(src);
        w[0] = v[0]; w[1] = v[1]; w[2] = v[2]; w[3] = v[3];
      } else {
        const int nb = (int)((N - gcol) / 2 < 16 ? (N - gcol) / 2 : 16);
        for (int j = 0; j < nb; j++) w[j >> 2] |= (uint32_t)src[j] << (8 * (j & 3));
      }
    }
    uint32_t* dst = reinterpret_cast<uint32_t*>(sm.codes + r * kCodePitch + c16 * 16);
    dst[0] = w[0]; dst[1] = w[1]; dst[2] = w[2]; dst[3] = w[3];
  }
  if (t < kTile) {
    uint32_t sv = 0;
    if (t < rows_valid) {
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int64_t gcol = col0 + 32 * j;
        // the reference indexes scales with row stride N/32 (floor)
        if (gcol < N) sv |= (uint32_t)s[(row0 + t) * sstride + gcol / 32] << (8 * j);
      }
    }
    *reinterpret_cast<uint32_t*>(&sm.scales[t][0]) = sv;
  }
}

// Dequantized value of tile element (r, c), 0 outside the tensor.
__device__ __forceinline__ float tile_value(const TileSmem& sm, int r, int c, bool valid) {
  const uint32_t byte = sm.codes[r * kCodePitch + (c >> 1)];
  const uint32_t nib = (c & 1) ? (byte >> 4) : (byte & 0xFu);
  const float sc = bf16_to_f32((uint32_t)sm.scales[r][c >> 5] << 7);
  const float v = bf16_to_f32(e2m1_to_bf16_bits(nib)) * sc;
  return valid ? v : 0.0f;
}

// amax over the tile column c (seeded with `seed`), combined over 2 halves.
__device__ __forceinline__ float tile_column_amax(TileSmem& sm, int rows_valid, bool col_valid, float seed) {
  const int t = threadIdx.x, c = t & (kTile - 1), h = t >> 7;
  float m = seed;
  for (int r = h * 64; r < h * 64 + 64; r++) m = fmaxf(m, fabsf(tile_value(sm, r, c, col_valid && r < rows_valid)));
  sm.part[h][c] = m;
  __syncthreads();
  return fmaxf(sm.part[0][c], sm.part[1][c]);
}

// Quantize the tile column owned by this thread (rows h*64 .. h*64+63) with
// multiplier `mult` and write it to dst[0 .. rows) (dst = column base).
__device__ __forceinline__ void tile_column_store(const TileSmem& sm, int c, int h, int rows_valid, bool col_valid,
                                                  float mult, uint8_t* __restrict__ dst, bool vec_ok) {
#pragma unroll
  for (int r16 = 0; r16 < 64; r16 += 16) {
    const int rb = h * 64 + r16;
    uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < 16; j += 2) {
      const float v0 = tile_value(sm, rb + j, c, col_valid && rb + j < rows_valid) * mult;
      const float v1 = tile_value(sm, rb + j + 1, c, col_valid && rb + j + 1 < rows_valid) * mult;
      const float q0 = fminf(fmaxf(v0, -448.0f), 448.0f);
      const float q1 = fminf(fmaxf(v1, -448.0f), 448.0f);
      w[j >> 2] |= fp8x2_from_f32(q0, q1) << (8 * (j & 3));
    }
    if (rb >= rows_valid) break;
    if (vec_ok && rb + 16 <= rows_valid) {
      u32x4 o;
      o[0] = w[0]; o[1] = w[1]; o[2] = w[2]; o[3] = w[3];
      __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(dst + rb));
    } else {
      for (int j = 0; j < 16 && rb + j < rows_valid; j++) dst[rb + j] = (uint8_t)(w[j >> 2] >> (8 * (j & 3)));
    }
  }
}

__global__ __launch_bounds__(256) void row_to_fp8_col_kernel(const uint8_t* __restrict__ q, const uint8_t* __restrict__ s,
                                                             uint8_t* __restrict__ out, float* __restrict__ out_s,
                                                             int64_t M, int64_t N, float eps, bool vin, bool vout) {
  __shared__ TileSmem sm;
  const int64_t bm = blockIdx.x, bn = blockIdx.y;
  const int64_t row0 = bm * kTile, col0 = bn * kTile;
  const int rows_valid = (int)(M - row0 < kTile ? M - row0 : kTile);
  stage_tile(sm, q, s, N, row0, rows_valid, col0, vin);
  __syncthreads();
  const int t = threadIdx.x, c = t & (kTile - 1);
  const bool col_valid = col0 + c < N;
  const float amax = tile_column_amax(sm, rows_valid, col_valid, eps);
  if (t < kTile && col_valid) {
    out_s[bm * N + col0 + c] = amax / 448.0f;
    sm.mult[c] = (amax > 1e-9f) ? (448.0f / amax) : 0.0f;
  } else if (t < kTile) {
    sm.mult[c] = 0.0f;
  }
  __syncthreads();
  const int oc = t >> 1, oh = t & 1;
  if (col0 + oc < N) tile_column_store(sm, oc, oh, rows_valid, true, sm.mult[oc], out + (col0 + oc) * M + row0, vout);
}

// compute_te_pow2_scale with FP8_E4M3_MAX = 448: the multiplier 1/2^k and the
// stored 1/multiplier, both exact powers of two (or 0 / inf).
__device__ __forceinline__ void te_pow2(float amax, float eps, float* mult, float* inv) {
  if (amax <= eps) { *mult = 1.0f; *inv = 1.0f; return; }
  const uint32_t b = __float_as_uint(amax / 448.0f);
  uint32_t e = (b >> 23) & 0xFFu;
  if (b & 0x7FFFFFu) e += 1u;
  const float div = __uint_as_float(e << 23);  // 2^(e-127), 0 for e == 0, inf for e == 255
  *inv = div;                                   // 1.0f / (1.0 / div) == div for these values
  if (e == 0u) *mult = __builtin_inff();
  else if (e >= 255u) *mult = 0.0f;
  else if (e == 254u) *mult = __uint_as_float(0x00400000u);  // 2^-127, subnormal
  else *mult = exp2i(127 - (int)e);
}

__global__ __launch_bounds__(256) void row_to_fp8_col_msplit_kernel(
    const uint8_t* __restrict__ q, const uint8_t* __restrict__ s, uint8_t* __restrict__ out, float* __restrict__ out_s,
    const int32_t* __restrict__ lens, const int32_t* __restrict__ offs, const int32_t* __restrict__ soffs,
    int64_t total_rows, int64_t N, int64_t out_s_rows, float eps, bool vin) {
  __shared__ TileSmem sm;
  const int64_t split = blockIdx.x, bm = blockIdx.y, bn = blockIdx.z;
  const int64_t len = lens[split];
  if (bm * kTile >= len) return;
  const int64_t start = offs[split], sstart = soffs[split];
  // Metadata arrives on the device; tiles whose rows or scale rows fall
  // outside the buffers are skipped rather than written out of bounds.
  if (start < 0 || start + len > total_rows || sstart < 0 || sstart + bm >= out_s_rows) return;
  const int64_t row0 = start + bm * kTile, col0 = bn * kTile;
  const int rows_valid = (int)(len - bm * kTile < kTile ? len - bm * kTile : kTile);
  stage_tile(sm, q, s, N, row0, rows_valid, col0, vin);
  __syncthreads();
  const int t = threadIdx.x, c = t & (kTile - 1);
  const bool col_valid = col0 + c < N;
  const float amax = tile_column_amax(sm, rows_valid, col_valid, 0.0f);
  if (t < kTile) {
    float mult = 0.0f, inv = 0.0f;
    te_pow2(amax, eps, &mult, &inv);
    sm.mult[c] = mult;
    if (col_valid) out_s[(sstart + bm) * N + col0 + c] = inv;
  }
  __syncthreads();
  const int oc = t >> 1, oh = t & 1;
  if (col0 + oc < N) {
    uint8_t* dst = out + start * N + (col0 + oc) * len + bm * kTile;
    const bool vout = ((start * N + (col0 + oc) * len + bm * kTile) & 15) == 0 &&
                      ((reinterpret_cast<uintptr_t>(out) & 15) == 0);
    tile_column_store(sm, oc, oh, rows_valid, true, sm.mult[oc], dst, vout);
  }
}

hipError_t launch_row_to_fp8_col(const void* q, const void* s, void* out, float* out_s, int64_t M, int64_t N, float eps,
                                 hipStream_t stream) {
  if (M == 0 || N == 0) return hipSuccess;
  const bool vin = (N % 32 == 0) && ((reinterpret_cast<uintptr_t>(q) & 15) == 0);
  const bool vout = (M % 16 == 0) && ((reinterpret_cast<uintptr_t>(out) & 15) == 0);
  dim3 grid((unsigned)((M + kTile - 1) / kTile), (unsigned)((N + kTile - 1) / kTile));
  hipLaunchKernelGGL(row_to_fp8_col_kernel, grid, dim3(256), 0, stream, static_cast<const uint8_t*>(q),
                     static_cast<const uint8_t*>(s), static_cast<uint8_t*>(out), out_s, M, N, eps, vin, vout);
  return hipGetLastError();
}

hipError_t launch_row_to_fp8_col_msplit(const void* q, const void* s, void* out, float* out_s, int64_t total_rows,
                                        int64_t N, const int32_t* lens, const int32_t* offs, const int32_t* soffs,
                                        int64_t nsplits, int64_t max_split_len, int64_t out_capacity,
                                        int64_t out_s_rows, float eps, hipStream_t stream) {
  (void)out_capacity;  // the ABI layer checks out_capacity >= total_rows * N
  if (nsplits == 0 || max_split_len <= 0 || N == 0) return hipSuccess;
  const bool vin = (N % 32 == 0) && ((reinterpret_cast<uintptr_t>(q) & 15) == 0);
  dim3 grid((unsigned)nsplits, (unsigned)((max_split_len + kTile - 1) / kTile), (unsigned)((N + kTile - 1) / kTile));
  hipLaunchKernelGGL(row_to_fp8_col_msplit_kernel, grid, dim3(256), 0, stream, static_cast<const uint8_t*>(q),
                     static_cast<const uint8_t*>(s), static_cast<uint8_t*>(out), out_s, lens, offs, soffs, total_rows, N,
                     out_s_rows, eps, vin);
  return hipGetLastError();
}

}  // namespace omo_hip
