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
// Two tile shapes. Where N % 32 == 0 and the codes are 16 B aligned, tiles
// are 128 rows x 256 element columns (the last band partial when N % 256 !=
// 0), one 256-thread workgroup each, a lane per code dword (wide_tile,
// below), for any M. Other inputs (codes not 16 B aligned, N % 32 != 0)
// take 128 x 128 tiles, one 512-thread block per tile, described here.
// The tile's code bytes (128 rows x 64 B) and
// scale bytes are staged in LDS. Lane t owns code-byte column p = t/8 (two
// element columns) and the 16 rows of eighth q = t%8, so 8 adjacent lanes
// hold a full tile column: the column amax is two quad_perm steps and one
// row_half_mirror step of DPP, and the eight lanes write the column's 128
// output rows as eight contiguous 16 B pieces.
// Code loads are ordinary (temporal) loads: a tile reads one 64 B half of
// each 128 B code line and the next column tile the other half, which then
// usually hits in L2; with non-temporal loads the dense kernel took 16.6 us
// instead of 12.7 us at 4096 x 7168.
// When all 16 scale bytes of a lane lie in [1, 252] no product can be inf
// or NaN, and v_cvt_scalef32_pk_f32_fp4 gives both columns' exact fp32
// values of a row in one instruction; otherwise the lane restates the
// reference per element.
#include <algorithm>

#include "omo_device.cuh"
#include "omo_internal.h"

namespace omo_hip {

constexpr int kTile = 128;
constexpr int kCodePitch = 64 + 16;  // LDS bytes per code row (16 B aligned rows)

constexpr int kRcThreads = 512;

// LDS row of tile row r: the 8 lanes of a column read rows 16q + j at the
// same time; storing row 16q + j at 8j + q puts those rows at consecutive LDS
// rows (distinct banks) instead of 16 rows apart (the same bank).
__device__ __forceinline__ int lds_row(int r) { return ((r & 15) << 3) | (r >> 4); }

// Maximum over the 8 lanes 8k..8k+7 (all active).
__device__ __forceinline__ float oct_fmax(float v) {
  v = quad_fmax(v);
  // row_half_mirror (0x141): lane i of each 8-lane half-row reads lane 7 - i
  const float o = __uint_as_float((uint32_t)__builtin_amdgcn_mov_dpp((int)__float_as_uint(v), 0x141, 0xF, 0xF, false));
  return fmaxf(v, o);
}

// oct_fmax for values that are all >= 0 (not NaN): such floats are ordered as
// their bit patterns are as signed integers, so the maximum is an integer
// maximum, which needs none of the NaN quieting that fmaxf costs (two more
// instructions per step) and folds into DPP forms.
__device__ __forceinline__ float oct_max_nonneg(float v) {
  int x = __float_as_int(v);
  x = max(x, __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, true));   // quad_perm [1,0,3,2]
  x = max(x, __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, true));   // quad_perm [2,3,0,1]
  x = max(x, __builtin_amdgcn_mov_dpp(x, 0x141, 0xF, 0xF, true));  // row_half_mirror
  return __int_as_float(x);
}

// Column maxima of n values per lane reduced over 8-lane groups: the integer
// form when every lane of the wave holds values >= 0 (the usual case: the
// maxima start from 0 or eps and take |v|), else fmaxf.
template <int n>
__device__ __forceinline__ void oct_max_all(float (&a)[n]) {
  bool nonneg = true;
#pragma unroll
  for (int e = 0; e < n; e++) nonneg = nonneg && a[e] >= 0.0f;  // false for NaN
  if (__builtin_amdgcn_ballot_w64(!nonneg) == 0) {
#pragma unroll
    for (int e = 0; e < n; e++) a[e] = oct_max_nonneg(a[e]);
  } else {
#pragma unroll
    for (int e = 0; e < n; e++) a[e] = oct_fmax(a[e]);
  }
}

struct RowColSmem {
  uint8_t codes[kTile * kCodePitch];
  uint32_t fscales[4][kTile];  // s << 23: the fp32 pattern of 2^(s-127), [MX block of the tile][row]
  uint8_t scales[4][kTile];    // the scale bytes themselves
};

// A lane's share of one tile's staging data: one 16 B chunk of codes and,
// for lanes 0..127, the four scale bytes of one row.
struct StageRegs {
  u32x4 codes;
  uint32_t scales;
};

// Load the staging data of tile rows [row0, row0 + rows_valid), element
// columns [col0, col0 + 128). Missing codes become 0; missing scales 127
// (1.0), so out-of-tensor elements dequantize to exactly 0 on the fast path.
// vin: 16 B vector code loads are allowed (N % 32 == 0, aligned base);
// vs: a scale row's four bytes of the tile are one aligned dword
// (N % 128 == 0, 4 B aligned base). The byte fallbacks keep exact bounds.
__device__ __forceinline__ StageRegs rc_load(const uint8_t* __restrict__ q, const uint8_t* __restrict__ s, int64_t N,
                                             int64_t row0, int rows_valid, int64_t col0, bool vin, bool vs) {
  const int t = threadIdx.x;
  const int64_t half = N / 2, sstride = N / 32;
  StageRegs g;
  {
    const int r = t >> 2, c16 = t & 3;  // 512 chunks of 16 code bytes, one per lane
    const int64_t gcol = col0 + c16 * 32;
    u32x4 w = {0u, 0u, 0u, 0u};
    if (r < rows_valid && gcol < N) {
      const uint8_t* src = q + (row0 + r) * half + gcol / 2;
      if (vin && gcol + 32 <= N) {
        w = *reinterpret_cast<const u32x4*>(src);
      } else {
        const int nb = (int)((N - gcol) / 2 < 16 ? (N - gcol) / 2 : 16);
        for (int j = 0; j < nb; j++) w[j >> 2] |= (uint32_t)src[j] << (8 * (j & 3));
      }
    }
    g.codes = w;
  }
  g.scales = 0x7F7F7F7Fu;
  if (t < kTile && t < rows_valid) {
    // the reference indexes scales with row stride N/32 (floor)
    const uint8_t* srow = s + (row0 + t) * sstride + col0 / 32;
    if (vs) {
      g.scales = *reinterpret_cast<const uint32_t*>(srow);
    } else {
#pragma unroll
      for (int j = 0; j < 4; j++) {
        if (col0 + 32 * j < N) g.scales = (g.scales & ~(0xFFu << (8 * j))) | ((uint32_t)srow[j] << (8 * j));
      }
    }
  }
  return g;
}

// Staging loads of an interior tile when every tile is whole and aligned
// (M % 128 == 0, N % 128 == 0, 16 B aligned codes, 4 B aligned scales):
// unconditional vector loads only, so the compiler can count the waits for
// them separately from the stores still in flight. Lanes 128..511 load a
// copy of the scale dword of row t % 128, which they do not use.
__device__ __forceinline__ StageRegs rc_load_full(const uint8_t* __restrict__ q, const uint8_t* __restrict__ s,
                                                  int64_t N, int64_t row0, int64_t col0) {
  const int t = threadIdx.x;
  StageRegs g;
  g.codes = *reinterpret_cast<const u32x4*>(q + (row0 + (t >> 2)) * (N / 2) + col0 / 2 + (t & 3) * 16);
  g.scales = *reinterpret_cast<const uint32_t*>(s + (row0 + (t & (kTile - 1))) * (N / 32) + col0 / 32);
  return g;
}

__device__ __forceinline__ void rc_put(RowColSmem& sm, const StageRegs& g) {
  const int t = threadIdx.x;
  *reinterpret_cast<u32x4*>(sm.codes + lds_row(t >> 2) * kCodePitch + (t & 3) * 16) = g.codes;
  if (t < kTile) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t b = (g.scales >> (8 * j)) & 0xFFu;
      sm.scales[j][t] = (uint8_t)b;
      sm.fscales[j][t] = b << 23;
    }
  }
}

// Output of one lane: the fp8 bytes of its 16 rows for both element columns.
struct LaneCols {
  u32x4 e0, e1;
};

// scale bytes 1..252 in every byte of w (no zero byte, no byte >= 253)
__device__ __forceinline__ bool bytes_in_1_252(uint32_t w) {
  const uint32_t zero = (w - 0x01010101u) & ~w & 0x80808080u;
  const uint32_t big = ((w & 0x7F7F7F7Fu) + 0x03030303u) & w & 0x80808080u;
  return (zero | big) == 0u;
}

// Value of lane `src` of the calling lane's wave.
__device__ __forceinline__ float lane_value(float v, int src) {
  return __int_as_float(__builtin_amdgcn_ds_bpermute(src << 2, __float_as_int(v)));
}

// compute_te_pow2_scale (per_token_Mxfp4RowToBf16ToFp8Col_msplit.cu:23-43)
// with FP8_E4M3_MAX = 448: multiplier 1/2^k and stored scale 2^k, 2^k the
// smallest power of two at or above fl(amax / 448); 1 and 1 for amax <= eps.
__device__ __forceinline__ void te_pow2_scale(float a, float eps, float* mult, float* inv) {
  if (a <= eps) {
    *mult = 1.0f;
    *inv = 1.0f;
    return;
  }
  const uint32_t b = __float_as_uint(a / 448.0f);
  uint32_t e = (b >> 23) & 0xFFu;
  if (b & 0x7FFFFFu) e += 1u;
  *inv = __uint_as_float(e << 23);  // 2^(e-127); 0 for e == 0, inf for e == 255
  if (e == 0u) *mult = __builtin_inff();
  else if (e >= 255u) *mult = 0.0f;
  else if (e == 254u) *mult = __uint_as_float(0x00400000u);  // 2^-127, subnormal
  else *mult = exp2i(127 - (int)e);
}

// Column scale factors from the column amax. Every lane of an 8-lane column
// group holds a0, a1 (the amax of columns 2p, 2p+1); lanes q = 0..3 of the
// group each compute one of the four results and the group reads them back,
// so each lane runs one division instead of four.
template <bool MSPLIT>
__device__ __forceinline__ void rc_factors(float a0, float a1, float eps, float* m0, float* m1, float* inv0,
                                           float* inv1) {
  const int lane = (int)(threadIdx.x & 63), qq = lane & 7, base = lane & ~7;
  const float a = (qq & 1) ? a1 : a0;
  float mult, inv;
  if (MSPLIT) {
    te_pow2_scale(a, eps, &mult, &inv);
    *m0 = lane_value(mult, base);
    *m1 = lane_value(mult, base + 1);
    *inv0 = lane_value(inv, base);
    *inv1 = lane_value(inv, base + 1);
  } else {
    // lanes q&2 == 0: 448 / amax (0 when amax <= 1e-9); q&2 != 0: amax / 448
    const bool is_inv = (qq & 2) != 0;
    float r = (is_inv ? a : 448.0f) / (is_inv ? 448.0f : a);
    if (!is_inv && !(a > 1e-9f)) r = 0.0f;
    *m0 = lane_value(r, base);
    *m1 = lane_value(r, base + 1);
    *inv0 = lane_value(r, base + 2);
    *inv1 = lane_value(r, base + 3);
  }
}

template <bool MSPLIT>
__device__ __forceinline__ void rc_tile(RowColSmem& sm, int rows_valid, int64_t N, int64_t col0, float seed, float eps,
                                        float* __restrict__ out_s_row, LaneCols& res) {
  const int t = threadIdx.x, p = t >> 3, qq = t & 7;
  const int blk = p >> 4;
  const bool col_valid = col0 + 2 * p < N;  // N is even: both columns or neither
  uint32_t sw[4], cb[16];
  float sc[16];
#pragma unroll
  for (int j4 = 0; j4 < 4; j4++) {
    sw[j4] = *reinterpret_cast<const uint32_t*>(&sm.scales[blk][16 * qq + 4 * j4]);
    const u32x4 f = *reinterpret_cast<const u32x4*>(&sm.fscales[blk][16 * qq + 4 * j4]);
#pragma unroll
    for (int k = 0; k < 4; k++) sc[4 * j4 + k] = __uint_as_float(f[k]);
  }
#pragma unroll
  for (int j = 0; j < 16; j++) cb[j] = sm.codes[lds_row(16 * qq + j) * kCodePitch + p];
  const bool fast = bytes_in_1_252(sw[0]) && bytes_in_1_252(sw[1]) && bytes_in_1_252(sw[2]) && bytes_in_1_252(sw[3]);
  float a0 = seed, a1 = seed;
  if (fast) {
#pragma unroll
    for (int j = 0; j < 16; j++) {
      float v0, v1;
      cvt_pk_f32_fp4<0>(cb[j], sc[j], &v0, &v1);
      a0 = fmaxf(a0, fabsf(v0));
      a1 = fmaxf(a1, fabsf(v1));
    }
  } else {
#pragma unroll
    for (int j = 0; j < 16; j++) {
      const bool ok = col_valid && (16 * qq + j) < rows_valid;
      const float s16 = bf16_to_f32(((sw[j >> 2] >> (8 * (j & 3))) & 0xFFu) << 7);
      const float v0 = ok ? bf16_to_f32(e2m1_to_bf16_bits(cb[j] & 0xFu)) * s16 : 0.0f;
      const float v1 = ok ? bf16_to_f32(e2m1_to_bf16_bits(cb[j] >> 4)) * s16 : 0.0f;
      a0 = fmaxf(a0, fabsf(v0));
      a1 = fmaxf(a1, fabsf(v1));
    }
  }
  {
    float am[2] = {a0, a1};
    oct_max_all(am);
    a0 = am[0];
    a1 = am[1];
  }
  float m0, m1, inv0, inv1;
  rc_factors<MSPLIT>(a0, a1, eps, &m0, &m1, &inv0, &inv1);
  if (qq == 0 && col_valid) {
    out_s_row[2 * p] = inv0;
    out_s_row[2 * p + 1] = inv1;
  }
  uint32_t w0[4] = {0u, 0u, 0u, 0u}, w1[4] = {0u, 0u, 0u, 0u};
  // The reference clamps v * m to +-448 before the E4M3 conversion. Where
  // |v * m| <= 448 (1 + 2^-23), which E4M3 RNE rounds to at most 448 (only
  // |x| > 464 overflows), the clamp changes no byte and is left out:
  //  * dense: |v| <= amax and m = fl(448 / amax);
  //  * grouped, amax > eps: m = 2^-k with 2^k the smallest power of two at
  //    or above fl(amax / 448); amax = c * 2^j for an E2M1 magnitude c, so
  //    amax / 448 = (c / 7) 2^(j - 6) is never within rounding distance of a
  //    power of two, 2^k >= amax / 448 exactly and |v * m| <= 448;
  //  * grouped, amax <= eps: m = 1, so the bound needs amax <= 448.
  // Otherwise (grouped with amax in (448, eps]) the clamp stays; a grouped
  // tile also needs finite multipliers to be NaN-free here.
  const bool finite_m = !MSPLIT || (m0 < __builtin_inff() && m1 < __builtin_inff());
  const bool no_clamp = !MSPLIT || ((a0 > eps || a0 <= 448.0f) && (a1 > eps || a1 <= 448.0f));
  if (fast && finite_m) {
    if (no_clamp) {
#pragma unroll
      for (int j4 = 0; j4 < 4; j4++) {
        float x[4], y[4];  // rows 4 j4 + k of columns 2p (x), 2p + 1 (y)
#pragma unroll
        for (int k = 0; k < 4; k++) {
          float v0, v1;
          cvt_pk_f32_fp4<0>(cb[4 * j4 + k], sc[4 * j4 + k], &v0, &v1);
          x[k] = v0 * m0;
          y[k] = v1 * m1;
        }
        // bytes 0, 1 from the low-word convert, bytes 2, 3 from the high-word one
        w0[j4] = fp8x4_from_f32(x[0], x[1], x[2], x[3]);
        w1[j4] = fp8x4_from_f32(y[0], y[1], y[2], y[3]);
      }
    } else {
#pragma unroll
      for (int j4 = 0; j4 < 4; j4++) {
        float x[4], y[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
          float v0, v1;
          cvt_pk_f32_fp4<0>(cb[4 * j4 + k], sc[4 * j4 + k], &v0, &v1);
          x[k] = __builtin_amdgcn_fmed3f(v0 * m0, -448.0f, 448.0f);
          y[k] = __builtin_amdgcn_fmed3f(v1 * m1, -448.0f, 448.0f);
        }
        w0[j4] = fp8x4_from_f32(x[0], x[1], x[2], x[3]);
        w1[j4] = fp8x4_from_f32(y[0], y[1], y[2], y[3]);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 16; j += 2) {
      float v[2][2];
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const bool ok = col_valid && (16 * qq + j + h) < rows_valid;
        const float s16 = bf16_to_f32(((sw[(j + h) >> 2] >> (8 * ((j + h) & 3))) & 0xFFu) << 7);
        v[h][0] = ok ? bf16_to_f32(e2m1_to_bf16_bits(cb[j + h] & 0xFu)) * s16 : 0.0f;
        v[h][1] = ok ? bf16_to_f32(e2m1_to_bf16_bits(cb[j + h] >> 4)) * s16 : 0.0f;
      }
      const float x0 = fminf(fmaxf(v[0][0] * m0, -448.0f), 448.0f);
      const float x1 = fminf(fmaxf(v[1][0] * m0, -448.0f), 448.0f);
      const float y0 = fminf(fmaxf(v[0][1] * m1, -448.0f), 448.0f);
      const float y1 = fminf(fmaxf(v[1][1] * m1, -448.0f), 448.0f);
      w0[j >> 2] |= fp8x2_from_f32(x0, x1) << (8 * (j & 3));
      w1[j >> 2] |= fp8x2_from_f32(y0, y1) << (8 * (j & 3));
    }
  }
  res.e0 = u32x4{w0[0], w0[1], w0[2], w0[3]};
  res.e1 = u32x4{w1[0], w1[1], w1[2], w1[3]};
}

// Write a lane's 16 bytes of one output column (rows 16q .. 16q+15 of the
// tile) to dst[0 .. 16), stopping at rows_valid. dst may have any byte
// alignment: the 16 B store is emitted as one global_store_dwordx4, which
// the hardware splits when it is unaligned (checked at every offset 0..15).
// A partial piece of n = 1..15 bytes is written as at most four stores of 8,
// 4, 2 and 1 bytes (the bits of n, largest first), so each one's source
// bytes start at a multiple of its size within the 16 (a loop of single
// byte stores cost 4 us over cfg5's ragged splits).
__device__ __forceinline__ void rc_store(uint8_t* __restrict__ dst, const u32x4& w, int r_base, int rows_valid) {
  if (r_base + 16 <= rows_valid) {
    __builtin_memcpy(dst, &w, 16);
  } else if (r_base < rows_valid) {
    const int n = rows_valid - r_base;
    int pos = 0;
    if (n & 8) {
      const u32x2 h = {w[0], w[1]};
      __builtin_memcpy(dst, &h, 8);
      pos = 8;
    }
    const uint32_t wd = pos ? w[2] : w[0];  // dword holding byte pos
    const uint32_t wn = pos ? w[3] : w[1];  // the next one
    if (n & 4) {
      __builtin_memcpy(dst + pos, &wd, 4);
      pos += 4;
    }
    const uint32_t v = (n & 4) ? wn : wd;   // dword holding byte pos now
    if (n & 2) {
      const uint16_t h = (uint16_t)v;
      __builtin_memcpy(dst + pos, &h, 2);
      pos += 2;
    }
    if (n & 1) dst[pos] = (uint8_t)((n & 2) ? v >> 16 : v);
  }
}

// Persistent over tiles (tile = blockIdx.x + k * gridDim.x, tile_m fastest):
// the next tile's codes and scales are loaded into registers while the
// current tile is converted, so reads and writes overlap. FULL: every tile
// is whole and aligned, and all loads and stores are unconditional vector
// operations.
template <bool FULL>
__global__ __launch_bounds__(kRcThreads) void row_to_fp8_col_kernel(const uint8_t* __restrict__ q,
                                                                    const uint8_t* __restrict__ s,
                                                                    uint8_t* __restrict__ out, float* __restrict__ out_s,
                                                                    int64_t M, int64_t N, int tiles_m, int tiles,
                                                                    float eps, bool vin, bool vs) {
  __shared__ RowColSmem sm;
  int tile = blockIdx.x;
  if (tile >= tiles) return;
  auto rows_of = [&](int tl) {
    if (FULL) return kTile;
    const int64_t r0 = (int64_t)(tl % tiles_m) * kTile;
    return (int)(M - r0 < kTile ? M - r0 : kTile);
  };
  auto load = [&](int tl) {
    const int64_t r0 = (int64_t)(tl % tiles_m) * kTile, c0 = (int64_t)(tl / tiles_m) * kTile;
    return FULL ? rc_load_full(q, s, N, r0, c0) : rc_load(q, s, N, r0, rows_of(tl), c0, vin, vs);
  };
  const int t = threadIdx.x, p = t >> 3, qq = t & 7;
  rc_put(sm, load(tile));
  __syncthreads();
  for (;;) {
    const int64_t bm = tile % tiles_m, bn = tile / tiles_m;
    const int64_t row0 = bm * kTile, col0 = bn * kTile;
    const int rows_valid = rows_of(tile);
    // Load the next tile (the last iteration reloads its own tile, unused)
    // before this tile's stores: the wait for the load before the LDS put
    // below then leaves this tile's stores in flight.
    const int nxt = tile + (int)gridDim.x;
    const StageRegs g = load(nxt < tiles ? nxt : tile);
    LaneCols res;
    rc_tile<false>(sm, rows_valid, N, col0, eps, eps, out_s + bm * N + col0, res);
    const int64_t c = col0 + 2 * p;
    if (FULL) {
      __builtin_nontemporal_store(res.e0, reinterpret_cast<u32x4*>(out + c * M + row0 + 16 * qq));
      __builtin_nontemporal_store(res.e1, reinterpret_cast<u32x4*>(out + (c + 1) * M + row0 + 16 * qq));
    } else if (c < N) {
      rc_store(out + c * M + row0 + 16 * qq, res.e0, 16 * qq, rows_valid);
      rc_store(out + (c + 1) * M + row0 + 16 * qq, res.e1, 16 * qq, rows_valid);
    }
    if (nxt >= tiles) break;
    tile = nxt;
    __syncthreads();  // this tile's LDS reads are done
    rc_put(sm, g);
    __syncthreads();
  }
}

// Tiles of 128 rows x 256 element columns (16 B aligned codes, N % 32 == 0;
// the last band partial when N % 256 != 0), one 256-thread workgroup per tile. Lane t owns code
// bytes 4c .. 4c+3 (element columns 8c .. 8c+7, one MX column), c = t / 8,
// and rows 16q .. 16q+15, q = t % 8: per row it reads one code dword from
// LDS (instead of one byte per two element columns), the 8 lanes of a code
// dword reduce its 8 column maxima with DPP, lane q computes column 8c + q's
// factors only (its scale-row entry and multiplier; the group reads the
// multipliers back with ds_bpermute), and the 8 lanes write each of the 8
// columns' 128 rows as eight 16 B pieces. The arithmetic per element and the
// fast-path conditions are those of rc_tile. Used by the dense kernel on
// whole aligned tensors (every workgroup resident at once on the benchmark
// shapes: 896 tiles at 4096 x 7168) and by the per-split kernel.
constexpr int kWideCols = 256;
constexpr int64_t kMaxGridYZ = 65535;  // below the y and z grid limits (65536)
constexpr int kWidePitch = 128 + 32;  // 16 B aligned LDS rows; 40 dwords keep a wave's row reads on distinct banks

struct WideSmem {
  uint8_t codes[kTile * kWidePitch];
  uint32_t fscales[8][kTile];  // s << 23, [MX column of the tile][row]
  uint8_t scales[8][kTile];
  uint32_t odd_scales[2];      // per staging wave: a scale byte of its rows outside [1, 252]
};

// The output pass converts with volatile asm, so the compiler neither keeps
// the column-maximum pass's 128 values per lane alive for it (it converts
// again) nor hoists its conversions above the clamp branch, and spills none
// of them. The column-maximum pass uses the builtin, which the compiler
// schedules around the conversion's latency.
template <int B>
__device__ __forceinline__ void cvt_pk_f32_fp4_once(uint32_t src, float scale, float* lo, float* hi) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  f32x2_t r;
  if constexpr (B == 0) asm volatile("v_cvt_scalef32_pk_f32_fp4 %0, %1, %2" : "=v"(r) : "v"(src), "v"(scale));
  if constexpr (B == 1) asm volatile("v_cvt_scalef32_pk_f32_fp4 %0, %1, %2 op_sel:[1,0,0]" : "=v"(r) : "v"(src), "v"(scale));
  if constexpr (B == 2) asm volatile("v_cvt_scalef32_pk_f32_fp4 %0, %1, %2 op_sel:[0,1,0]" : "=v"(r) : "v"(src), "v"(scale));
  if constexpr (B == 3) asm volatile("v_cvt_scalef32_pk_f32_fp4 %0, %1, %2 op_sel:[1,1,0]" : "=v"(r) : "v"(src), "v"(scale));
  *lo = r[0];
  *hi = r[1];
}

// Column maxima of the lane's 16 rows in fp32, two values per conversion.
// Measured and not kept: sign bits cleared and v_cvt_scalef32_pk_bf16_fp4
// into packed 16-bit maxima (two columns per v_pk_max_u16, exact for scale
// bytes 1..252, a quarter fewer instructions): 9.17 against 8.86 us at
// 4096 x 7168.
template <int B>
__device__ __forceinline__ void wide_amax_fast(const uint32_t (&cw)[16], const float (&sc)[16], float (&a)[8]) {
#pragma unroll
  for (int j = 0; j < 16; j++) {
    float v0, v1;
    cvt_pk_f32_fp4<B>(cw[j], sc[j], &v0, &v1);
    a[2 * B] = fmaxf(a[2 * B], fabsf(v0));
    a[2 * B + 1] = fmaxf(a[2 * B + 1], fabsf(v1));
  }
}

// Columns 2b, 2b+1 of the lane (the nibbles of code byte b) for its 16 rows.
template <int B, bool CLAMP>
__device__ __forceinline__ void wide_pair_fast(const uint32_t (&cw)[16], const float (&sc)[16], float m0, float m1,
                                               u32x4& w0, u32x4& w1) {
#pragma unroll
  for (int j4 = 0; j4 < 4; j4++) {
    float x[4], y[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      float v0, v1;
      cvt_pk_f32_fp4_once<B>(cw[4 * j4 + k], sc[4 * j4 + k], &v0, &v1);
      x[k] = CLAMP ? __builtin_amdgcn_fmed3f(v0 * m0, -448.0f, 448.0f) : v0 * m0;
      y[k] = CLAMP ? __builtin_amdgcn_fmed3f(v1 * m1, -448.0f, 448.0f) : v1 * m1;
    }
    w0[j4] = fp8x4_from_f32(x[0], x[1], x[2], x[3]);
    w1[j4] = fp8x4_from_f32(y[0], y[1], y[2], y[3]);
  }
}

// Per split, no clamp: the multiplier of a column is 1 / inv with inv = 2^k,
// and v_cvt_scalef32_pk_fp8_f32 (x, y, inv) gives the bytes of
// v_cvt_pk_fp8_f32 (x / inv, y / inv) = v_cvt_pk_fp8_f32 (x * m, y * m)
// (checked equal on the GPU for every finite 2^k, k = -126 .. 127, over all
// E2M1 magnitudes times 2^e and random inputs), one instruction per two
// values instead of three.
template <int B>
__device__ __forceinline__ void wide_pair_scaled(const uint32_t (&cw)[16], const float (&sc)[16], float inv0,
                                                 float inv1, u32x4& w0, u32x4& w1) {
  typedef short s16x2 __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int j4 = 0; j4 < 4; j4++) {
    float x[4], y[4];
#pragma unroll
    for (int k = 0; k < 4; k++) cvt_pk_f32_fp4_once<B>(cw[4 * j4 + k], sc[4 * j4 + k], &x[k], &y[k]);
    // the first conversion's passed-through upper half is overwritten by the second
    const s16x2 a = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(
        __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(__builtin_bit_cast(s16x2, x[0]), x[0], x[1], inv0, false), x[2], x[3],
        inv0, true);
    const s16x2 b = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(
        __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(__builtin_bit_cast(s16x2, y[0]), y[0], y[1], inv1, false), y[2], y[3],
        inv1, true);
    w0[j4] = (uint32_t)(uint16_t)a[0] | ((uint32_t)(uint16_t)a[1] << 16);
    w1[j4] = (uint32_t)(uint16_t)b[0] | ((uint32_t)(uint16_t)b[1] << 16);
  }
}

// Conversion of one staged wide tile: lane (cg, qq) converts element columns
// 8cg .. 8cg+7 of tile rows 16qq .. 16qq+15 and hands column e's 16 bytes
// (rows in order) to put(e, w). codes: the tile's first LDS code row (rows
// permuted by lds_row, pitch bytes apart); scl / fscl: the 128 scale bytes
// and 2^(s-127) patterns of the lane's MX column; fast: every scale byte of
// the tile is in [1, 252] (else the restatement). The scale-row entry of
// column 8cg + qq goes to out_s_lane when store_s. The 8 lanes of a code
// dword must be 8 adjacent lanes of a wave.
template <bool MSPLIT, typename Put>
__device__ __forceinline__ void wide_convert(const uint8_t* codes, int pitch, const uint8_t* scl, const uint32_t* fscl,
                                             int cg, int qq, float eps, bool fast, bool store_s,
                                             float* __restrict__ out_s_lane, Put&& put) {
  uint32_t cw[16];
  float sc[16];
#pragma unroll
  for (int j4 = 0; j4 < 4; j4++) {
    const u32x4 f = *reinterpret_cast<const u32x4*>(fscl + 16 * qq + 4 * j4);
#pragma unroll
    for (int k = 0; k < 4; k++) sc[4 * j4 + k] = __uint_as_float(f[k]);
  }
#pragma unroll
  for (int j = 0; j < 16; j++) cw[j] = *reinterpret_cast<const uint32_t*>(codes + lds_row(16 * qq + j) * pitch + 4 * cg);
  float a[8];
#pragma unroll
  for (int e = 0; e < 8; e++) a[e] = MSPLIT ? 0.0f : eps;
  if (fast) {
    wide_amax_fast<0>(cw, sc, a);
    wide_amax_fast<1>(cw, sc, a);
    wide_amax_fast<2>(cw, sc, a);
    wide_amax_fast<3>(cw, sc, a);
  } else {
    const u32x4 sw = *reinterpret_cast<const u32x4*>(scl + 16 * qq);
#pragma unroll
    for (int j = 0; j < 16; j++) {
      const float s16 = bf16_to_f32(((sw[j >> 2] >> (8 * (j & 3))) & 0xFFu) << 7);
#pragma unroll
      for (int e = 0; e < 8; e++) a[e] = fmaxf(a[e], fabsf(bf16_to_f32(e2m1_to_bf16_bits((cw[j] >> (4 * e)) & 0xFu)) * s16));
    }
  }
  oct_max_all(a);
  float ae = a[0];
#pragma unroll
  for (int e = 1; e < 8; e++) ae = qq == e ? a[e] : ae;
  float mown, iown;
  if (MSPLIT) {
    te_pow2_scale(ae, eps, &mown, &iown);
  } else {
    // 448 / amax (0 when amax <= 1e-9) and amax / 448
    mown = 448.0f / ae;
    if (!(ae > 1e-9f)) mown = 0.0f;
    iown = ae / 448.0f;
  }
  if (store_s) __builtin_nontemporal_store(iown, out_s_lane);
  const int base = (int)(threadIdx.x & 63) & ~7;
  float m[8], iv[8];
#pragma unroll
  for (int e = 0; e < 8; e++) m[e] = lane_value(mown, base + e);
  if (MSPLIT) {
#pragma unroll
    for (int e = 0; e < 8; e++) iv[e] = lane_value(iown, base + e);
  }
  // The clamp to +-448 is left out where it changes no byte, as in rc_tile:
  // always for the dense kernel; per split where every column has amax > eps
  // or amax <= 448 (and finite multipliers).
  bool finite_m = true, no_clamp = true;
  if (MSPLIT) {
#pragma unroll
    for (int e = 0; e < 8; e++) {
      // multiplier and scale finite (the scaled conversion divides by inv)
      finite_m = finite_m && m[e] < __builtin_inff() && iv[e] < __builtin_inff();
      no_clamp = no_clamp && (a[e] > eps || a[e] <= 448.0f);
    }
  }
  if (fast && finite_m) {
    u32x4 w0, w1;
    if (MSPLIT && no_clamp) {
      wide_pair_scaled<0>(cw, sc, iv[0], iv[1], w0, w1);
      put(0, w0);
      put(1, w1);
      wide_pair_scaled<1>(cw, sc, iv[2], iv[3], w0, w1);
      put(2, w0);
      put(3, w1);
      wide_pair_scaled<2>(cw, sc, iv[4], iv[5], w0, w1);
      put(4, w0);
      put(5, w1);
      wide_pair_scaled<3>(cw, sc, iv[6], iv[7], w0, w1);
      put(6, w0);
      put(7, w1);
    } else if (no_clamp) {
      wide_pair_fast<0, false>(cw, sc, m[0], m[1], w0, w1);
      put(0, w0);
      put(1, w1);
      wide_pair_fast<1, false>(cw, sc, m[2], m[3], w0, w1);
      put(2, w0);
      put(3, w1);
      wide_pair_fast<2, false>(cw, sc, m[4], m[5], w0, w1);
      put(4, w0);
      put(5, w1);
      wide_pair_fast<3, false>(cw, sc, m[6], m[7], w0, w1);
      put(6, w0);
      put(7, w1);
    } else {
      wide_pair_fast<0, true>(cw, sc, m[0], m[1], w0, w1);
      put(0, w0);
      put(1, w1);
      wide_pair_fast<1, true>(cw, sc, m[2], m[3], w0, w1);
      put(2, w0);
      put(3, w1);
      wide_pair_fast<2, true>(cw, sc, m[4], m[5], w0, w1);
      put(4, w0);
      put(5, w1);
      wide_pair_fast<3, true>(cw, sc, m[6], m[7], w0, w1);
      put(6, w0);
      put(7, w1);
    }
  } else {
    const u32x4 sw = *reinterpret_cast<const u32x4*>(scl + 16 * qq);
#pragma unroll 1
    for (int e = 0; e < 8; e++) {
      uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int j = 0; j < 16; j += 2) {
        float x[2];
#pragma unroll
        for (int h = 0; h < 2; h++) {
          const float s16 = bf16_to_f32(((sw[(j + h) >> 2] >> (8 * ((j + h) & 3))) & 0xFFu) << 7);
          const float v = bf16_to_f32(e2m1_to_bf16_bits((cw[j + h] >> (4 * e)) & 0xFu)) * s16;
          x[h] = fminf(fmaxf(v * m[e], -448.0f), 448.0f);
        }
        w[j >> 2] |= fp8x2_from_f32(x[0], x[1]) << (8 * (j & 3));
      }
      put(e, u32x4{w[0], w[1], w[2], w[3]});
    }
  }
}

// One tile: code rows row0 .. row0 + rows_valid - 1 (the others read as
// codes 0 with scale 127, i.e. exact zeros), element columns col0 .. col0 +
// 255. Element column col0 + e, tile row r is written at obase + e * cstride
// + r; the scale-row entry of column col0 + e at out_s_row[e]. Dense
// (MSPLIT false): amax seeded with eps, factors 448 / amax and amax / 448.
// Per split: amax seeded with 0, te_pow2_scale factors. RAGGED: rows_valid
// may be below 128 and the output pieces may have any alignment; stores are
// then ordinary stores at the exact place, whose partial lines (shared with
// the neighbouring tiles of the column) are completed in L2, unless line_nt
// says every column piece of the tile is one whole 128 B line. Not RAGGED:
// rows_valid == 128 and 16 B aligned non-temporal stores.
// SBYTE: the 8 scale bytes of a tile row are read one by one (rows of N / 32
// scale bytes that are not 8 B aligned, N % 256 != 0). PARTIAL: only element
// columns col0 .. col0 + cols_valid - 1 exist (the last band when N % 256 !=
// 0; cols_valid a multiple of 32): the missing 16 B code chunks of a row read
// its last chunk and are zeroed, their scale bytes read as 127, and the lanes
// of the missing columns store nothing.
template <bool MSPLIT, bool RAGGED, bool PARTIAL = false, bool SBYTE = false>
__device__ __forceinline__ void wide_tile(WideSmem& sm, const uint8_t* __restrict__ q, const uint8_t* __restrict__ s,
                                          int64_t N, int64_t row0, int rows_valid, int64_t col0, float eps,
                                          float* __restrict__ out_s_row, uint8_t* __restrict__ obase, int64_t cstride,
                                          bool line_nt, int cols_valid = kWideCols) {
  const int t = threadIdx.x;
  const int nch = PARTIAL ? cols_valid / 32 : 8;  // code chunks (and MX columns) per tile row
  // ---- stage codes (1024 chunks of 16 B, 8 rows x 128 B per wave load) and scales.
  // RAGGED: a row past rows_valid loads the tile's last row (in bounds, lines
  // the tile reads anyway) and is replaced by codes 0 / scale 127 afterwards,
  // so that the four loads issue back to back: loads under a branch each
  // waited for completion before the next was issued (dense 4000 x 7168:
  // 10.6 against 11.4 us).
  // Lane t loads chunk t & 7 of rows (t >> 3) + 32k: one 64-bit row product
  // per lane, the rest workgroup-uniform steps of 32 rows. Per split the code
  // loads are non-temporal (cfg5's 8 splits 50.3 against 49.0 us); the
  // dense kernel, one round of resident workgroups, keeps ordinary ones
  // (4096 x 7168 8.9 against 9.5 us non-temporal).
  u32x4 cv[4];
  const uint8_t* qt = q + row0 * (N / 2) + col0 / 2 + 16 * (PARTIAL ? min(t & 7, nch - 1) : (t & 7));
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int r = (t >> 3) + 32 * k;
    const int64_t rr = RAGGED ? min(r, rows_valid - 1) : (t >> 3);
    const u32x4* src = reinterpret_cast<const u32x4*>(qt + rr * (N / 2) + (RAGGED ? 0 : 32 * k * (N / 2)));
    cv[k] = MSPLIT ? __builtin_nontemporal_load(src) : *src;
  }
  u32x2 sv = {0x7F7F7F7Fu, 0x7F7F7F7Fu};
  if (t < kTile) {
    const uint8_t* srow = s + (row0 + (RAGGED ? min(t, rows_valid - 1) : t)) * (N / 32) + col0 / 32;
    if (SBYTE) {
      uint32_t w[2] = {0u, 0u};
#pragma unroll
      for (int c = 0; c < 8; c++) w[c >> 2] |= (c < nch ? (uint32_t)srow[c] : 0x7Fu) << (8 * (c & 3));
      sv = u32x2{w[0], w[1]};
    } else {
      sv = *reinterpret_cast<const u32x2*>(srow);
    }
  }
  if (RAGGED || PARTIAL) {
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int r = (t + 256 * k) >> 3, c16 = (t + 256 * k) & 7;
      if ((RAGGED && r >= rows_valid) || (PARTIAL && c16 >= nch)) cv[k] = u32x4{0u, 0u, 0u, 0u};
    }
    if (RAGGED && t >= rows_valid) sv = u32x2{0x7F7F7F7Fu, 0x7F7F7F7Fu};
  }
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int id = t + 256 * k, r = id >> 3, c16 = id & 7;
    *reinterpret_cast<u32x4*>(sm.codes + lds_row(r) * kWidePitch + c16 * 16) = cv[k];
  }
  if (t < kTile) {
#pragma unroll
    for (int c = 0; c < 8; c++) {
      const uint32_t b = (sv[c >> 2] >> (8 * (c & 3))) & 0xFFu;
      sm.scales[c][t] = (uint8_t)b;
      sm.fscales[c][t] = b << 23;
    }
    // the fast path's test, once per tile: every scale byte in [1, 252]
    // (padding rows and missing columns hold 127); the two staging waves
    // each record whether any of their rows fails it
    const int odd = __any(!(bytes_in_1_252(sv[0]) && bytes_in_1_252(sv[1])));
    if ((t & 63) == 0) sm.odd_scales[t >> 6] = (uint32_t)odd;
  }
  __syncthreads();
  const bool fast = (sm.odd_scales[0] | sm.odd_scales[1]) == 0u;
  const int qq = t & 7, cg = t >> 3, mx = cg >> 2;
  const bool col_ok = !PARTIAL || mx < nch;  // this lane's 8 element columns exist
  uint8_t* o = obase + 8 * cg * cstride + 16 * qq;
  wide_convert<MSPLIT>(sm.codes, kWidePitch, sm.scales[mx], sm.fscales[mx], cg, qq, eps, fast, col_ok,
                       out_s_row + 8 * cg + qq, [&](int e, const u32x4& w) {
                         if (PARTIAL && !col_ok) return;
                         if (RAGGED && !line_nt) rc_store(o + e * cstride, w, 16 * qq, rows_valid);
                         else __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(o + e * cstride));
                       });
}

// A tile of band col0 / 256: the whole band, or (NARROWN, N % 256 != 0)
// the last band's N - col0 columns.
template <bool MSPLIT, bool RAGGED, bool NARROWN>
__device__ __forceinline__ void wide_tile_any(WideSmem& sm, const uint8_t* __restrict__ q,
                                              const uint8_t* __restrict__ s, int64_t N, int64_t row0, int rows_valid,
                                              int64_t col0, float eps, float* __restrict__ out_s_row,
                                              uint8_t* __restrict__ obase, int64_t cstride, bool line_nt) {
  if (!NARROWN || col0 + kWideCols <= N) {
    wide_tile<MSPLIT, RAGGED, false, NARROWN>(sm, q, s, N, row0, rows_valid, col0, eps, out_s_row, obase, cstride,
                                              line_nt);
  } else {
    wide_tile<MSPLIT, RAGGED, true, NARROWN>(sm, q, s, N, row0, rows_valid, col0, eps, out_s_row, obase, cstride,
                                             line_nt, (int)(N - col0));
  }
}

// Dense, tile (bm, bn) = blockIdx renumbered per XCD, bn fastest. Not
// RAGGED: whole aligned tiles (M % 128 == 0, 16 B aligned output). RAGGED:
// any M, any output alignment (the last row tile partial). NARROWN: N % 32
// == 0 but not a multiple of 256, or scale rows not 8 B aligned (the last
// band partial, scale bytes read one by one).
template <bool RAGGED, bool NARROWN>
__global__ __launch_bounds__(256, 4) void row_to_fp8_col_wide_kernel(const uint8_t* __restrict__ q,
                                                                     const uint8_t* __restrict__ s,
                                                                     uint8_t* __restrict__ out,
                                                                     float* __restrict__ out_s, int64_t M, int64_t N,
                                                                     float eps) {
  __shared__ WideSmem sm;
  // bands fastest within each XCD's contiguous range (each XCD a run of row
  // tiles, every band): 4096 x 7168 8.9 us against 9.3 with row tiles
  // fastest and 9.2-9.4 with each XCD a 2-D block of tiles
  const uint32_t L = xcd_contiguous(blockIdx.x, gridDim.x), gx = (uint32_t)((N + kWideCols - 1) / kWideCols);
  const int64_t bn = L % gx, bm = L / gx;
  const int64_t row0 = bm * kTile, col0 = bn * kWideCols;
  const int rows_valid = RAGGED ? (int)(M - row0 < kTile ? M - row0 : kTile) : kTile;
  wide_tile_any<false, RAGGED, NARROWN>(sm, q, s, N, row0, rows_valid, col0, eps, out_s + bm * N + col0,
                                        out + col0 * M + row0, M, false);
}

// Per split on the 256-column tiles: workgroup (split, bm, bn) as in
// row_to_fp8_col_msplit_kernel. A split whose length and block start
// start * N are multiples of 128 (the start always is when N % 128 == 0) has
// every column piece on one whole 128 B line when the output base is 128 B
// aligned (out_line): those tiles store non-temporally (30.9 us against 43.0
// us with ordinary stores over 8 such splits of 7168 columns); the others
// keep ordinary stores, since non-temporal partial lines are not merged in L2
// (ragged splits took 81.4 us that way against 58.2 us).
// Row tile bm, column band bn of a split with rows [start, start + len) and
// scale rows from sstart. Metadata arrives on the device; tiles whose rows
// or scale rows fall outside the buffers are skipped rather than written out
// of bounds. Uniform over the workgroup.
template <bool NARROWN>
__device__ __forceinline__ void msplit_wide_tile(WideSmem& sm, const uint8_t* __restrict__ q,
                                                 const uint8_t* __restrict__ s, uint8_t* __restrict__ out,
                                                 float* __restrict__ out_s, int64_t len, int64_t start, int64_t sstart,
                                                 int64_t bm, int64_t bn, int64_t total_rows, int64_t N,
                                                 int64_t out_s_rows, float eps, bool out_line) {
  if (bm * kTile >= len) return;
  if (start < 0 || start + len > total_rows || sstart < 0 || sstart + bm >= out_s_rows) return;
  const int64_t row0 = start + bm * kTile, col0 = bn * kWideCols;
  const int rows_valid = (int)(len - bm * kTile < kTile ? len - bm * kTile : kTile);
  wide_tile_any<true, true, NARROWN>(sm, q, s, N, row0, rows_valid, col0, eps, out_s + (sstart + bm) * N + col0,
                                     out + start * N + col0 * len + bm * kTile, len,
                                     out_line && len % kTile == 0 && (start * N) % kTile == 0);
}

template <bool NARROWN>
__global__ __launch_bounds__(256, 4) void row_to_fp8_col_msplit_wide_kernel(
    const uint8_t* __restrict__ q, const uint8_t* __restrict__ s, uint8_t* __restrict__ out, float* __restrict__ out_s,
    const int32_t* __restrict__ lens, const int32_t* __restrict__ offs, const int32_t* __restrict__ soffs,
    int64_t total_rows, int64_t N, int64_t out_s_rows, float eps, bool out_line, int64_t bm0, int64_t bn0) {
  __shared__ WideSmem sm;
  const int64_t split = blockIdx.x, bm = bm0 + blockIdx.y, bn = bn0 + blockIdx.z;
  const int64_t len = lens[split];
  if (bm * kTile >= len) return;
  msplit_wide_tile<NARROWN>(sm, q, s, out, out_s, len, offs[split], soffs[split], bm, bn, total_rows, N, out_s_rows, eps,
                   out_line);
}

// Inclusive sum over the 64 lanes of a wave: DPP shifts within each 16-lane
// row (a lane without a source adds 0), then row 0's total into row 1 and
// row 2's into row 3 (row_bcast:15), then rows 0-1's total into rows 2-3
// (row_bcast:31).
__device__ __forceinline__ int wave_inclusive_sum(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, true);   // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, true);   // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true);   // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, true);   // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15 into rows 1, 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31 into rows 2, 3
  return v;
}

// Per split on a flat grid, for at most 128 splits. The tiles that hold rows
// (ceil(len_i / 128) row tiles of split i, at most the grid's tm, times the
// column bands) are numbered split by split, band by band, row tile fastest,
// and handed to the XCDs in one of two orders. Each wave finds its
// workgroup's tile itself: lane l reads the metadata of splits l + 64k, wave
// sums number the tiles, a ballot finds the split. Workgroups past the last
// tile (of their XCD) exit.
//  * Ranges: the whole numbering is cut into eight contiguous ranges, one per
//    XCD, so every XCD gets the same number of tiles, and the two row tiles
//    that share a column's 128 B output lines run next to each other on one
//    XCD, where their partial lines merge in L2. An XCD then holds about one
//    split when there are eight.
//  * Band walk: split after split, the split's tiles are cut into eight
//    contiguous ranges of ceil(tiles_i / 8), one per XCD, so that each XCD
//    owns a group of bands (parts of bands at its range's ends), and each XCD
//    walks its range row tile by row tile (all its bands of row tile m, then
//    those of m + 1). The XCDs read each split's rows in a shared sweep, and
//    the row tiles sharing an output line still run a few workgroups apart
//    on the XCD that owns the column.
// On 16431 routed rows x 7168 (wide tiles), band walk against ranges: 49.5
// against 55.4 us for 8 splits (1801..2279 rows), 49.5/54.9 for 4 uneven,
// 51.0/53.9 for 16, 51.2/52.7 for 32; past 64 splits the ranges win (53.9
// against 54.3 us at 65, 56.1/57.3 at 100, 60.1/61.7 at 128). On rows of
// few bands the ranges win (the same rows, 8 splits: N = 2048, 14.3 against
// 15.9 us; 2880, 19.1 against 22.0; 3072, 19.1 against 20.8; 4096, 29.1
// against 29.9), on more the band walk (5120, 36.7 against 38.3; 6144, 41.9
// against 46.9). The wide kernel walks bands up to 64 splits on rows of more
// than 16 bands, also with a partial last band (N = 7040: 50.5-52.7 us for 4
// to 32 splits, 51.1 for 8 nearly equal ones). The 128-column tiles (codes
// not 16 B aligned) keep the ranges, which won there at every count (N =
// 7040: 70.0 against 79.4 us at 8 splits, 82.0/91.0 at 16).
// On the 3-D grid (split, row tile, band) a split's tiles all land on one
// XCD when the split count is a multiple of 8 (the XCD holding the longest
// splits then finishes last) and are scattered otherwise. On 16431 routed
// rows x 7168 with the same tile code, the ranges took 52.2-56.1 us for 4 to
// 65 splits of any balance and 57.6 and 62.0 us for 100 and 128 splits; the
// 3-D grid 54.7 us for cfg5's 8 nearly equal splits, 72-174 us for 4 to 32
// uneven ones and 70-74 us for 65 to 128. Past 128 splits the 3-D grid is
// kept: hundreds of short splits balance by their number, and four metadata
// chunks per lane lost there (77.7 against 76.1 us at 200 splits, 82.1
// against 77.4 at 256).
constexpr int kFlatMaxSplits = 128;  // lane l of each wave holds splits l and l + 64

// Workgroups of the flat grid, enough for either order: every XCD gets at
// most ceil(tm * bands / 8) tiles of each split.
__host__ __device__ constexpr int64_t flat_grid_blocks(int64_t nsplits, int64_t tm, int64_t bands) {
  return 8 * nsplits * ((tm * bands + 7) / 8);
}

// Band walk: tile (S row tiles x B bands, T = S * B, numbered band by band
// with the row tile fastest) of position j in XCD xcd's walk over its
// contiguous range of per_xcd tiles, row tile by row tile. False past the
// range.
__device__ __forceinline__ bool band_walk_tile(int xcd, int j, int S, int T, int per_xcd, int* bm, int* bn) {
  const int lo = xcd * per_xcd, hi = min(T, lo + per_xcd);
  if (j >= hi - lo) return false;
  const int bn0 = lo / S, m0 = lo - bn0 * S;  // first tile of the range
  const int bn1 = hi / S, m1 = hi - bn1 * S;  // one past the last
  // tiles of the range in row tiles below m: band bn0 holds [m0, S) (or
  // [m0, m1) when bn0 == bn1), bands bn0 + 1 .. bn1 - 1 all, band bn1 [0, m1)
  auto below = [&](int m) {
    if (bn0 == bn1) return max(0, min(m, m1) - m0);
    return m * (bn1 - bn0 - 1) + max(0, m - m0) + min(m, m1);
  };
  int a = 0, b = S;  // below(a) <= j < below(b) = hi - lo
  while (b - a > 1) {
    const int mid = (a + b) >> 1;
    if (below(mid) <= j) a = mid;
    else b = mid;
  }
  *bm = a;
  *bn = bn0 + (a >= m0 ? 0 : 1) + (j - below(a));
  return true;
}

// The tile of this workgroup on the flat grid: split, row tile bm and band
// bn, or false past the last tile (uniform over the workgroup).
template <int CHUNKS,  // splits per lane: 1 (up to 64 splits) or 2 (up to 128)
          bool WALK>   // band walk, else ranges
__device__ __forceinline__ bool flat_split_tile(const int32_t* __restrict__ lens, const int32_t* __restrict__ offs,
                                                const int32_t* __restrict__ soffs, int nsplits, int tm, int bands,
                                                int64_t* len, int64_t* start, int64_t* sstart, int64_t* bm,
                                                int64_t* bn) {
  const int lane = (int)(threadIdx.x & 63);
  const int xcd = (int)(blockIdx.x & 7u);
  int len_l[CHUNKS], start_l[CHUNKS], sstart_l[CHUNKS];
#pragma unroll
  for (int k = 0; k < CHUNKS; k++) {
    const int i = lane + 64 * k;
    len_l[k] = start_l[k] = sstart_l[k] = 0;
    if (i < nsplits) {
      len_l[k] = lens[i];
      start_l[k] = offs[i];
      sstart_l[k] = soffs[i];
    }
  }
  // Each split's share of the numbering, in split order (chunk k's splits
  // follow those of chunks 0 .. k-1): ranges count whole splits' row tiles
  // (times bands below), band walk this XCD's tiles of each split.
  int rows_l[CHUNKS], per_l[CHUNKS], lo_l[CHUNKS], hi_l[CHUNKS];
  int before = 0;
#pragma unroll
  for (int k = 0; k < CHUNKS; k++) {
    rows_l[k] = len_l[k] > 0 ? (int)min(((int64_t)len_l[k] + kTile - 1) / kTile, (int64_t)tm) : 0;
    per_l[k] = (rows_l[k] * bands + 7) / 8;
    const int n = WALK ? min(max(rows_l[k] * bands - xcd * per_l[k], 0), per_l[k]) : rows_l[k];
    const int incl = wave_inclusive_sum(n);
    lo_l[k] = before + incl - n;
    hi_l[k] = before + incl;
    before += __builtin_amdgcn_readlane(incl, 63);
  }
  // the position to find: j in this XCD's walk, or L in the whole numbering
  // (at most nsplits * tm * bands, below the grid size, itself below 2^31)
  int j;
  if (WALK) {
    j = (int)(blockIdx.x >> 3);
    if (j >= before) return false;
  } else {
    const uint32_t n_real = (uint32_t)before * (uint32_t)bands;
    if (blockIdx.x >= n_real) return false;
    j = (int)xcd_contiguous(blockIdx.x, n_real);
  }
  const int unit = WALK ? 1 : bands;  // numbering units per share unit
  // exactly one split's range [unit * lo, unit * hi) holds j
  int S = 1, per = 1, r = 0;
  *len = *start = *sstart = 0;
#pragma unroll
  for (int k = 0; k < CHUNKS; k++) {
    const uint64_t hit = __ballot(j >= unit * lo_l[k] && j < unit * hi_l[k]);
    if (hit) {
      const int i = (int)__builtin_ctzll(hit);
      S = __builtin_amdgcn_readlane(rows_l[k], i);
      per = __builtin_amdgcn_readlane(per_l[k], i);
      r = j - unit * __builtin_amdgcn_readlane(lo_l[k], i);
      *len = __builtin_amdgcn_readlane(len_l[k], i);
      *start = __builtin_amdgcn_readlane(start_l[k], i);
      *sstart = __builtin_amdgcn_readlane(sstart_l[k], i);
    }
  }
  if (WALK) {
    int tbm, tbn;
    if (!band_walk_tile(xcd, r, S, S * bands, per, &tbm, &tbn)) return false;
    *bm = tbm;
    *bn = tbn;
  } else {
    *bm = r % S;
    *bn = r / S;
  }
  return true;
}

template <int CHUNKS, bool WALK, bool NARROWN>
__global__ __launch_bounds__(256, 4) void row_to_fp8_col_msplit_flat_kernel(
    const uint8_t* __restrict__ q, const uint8_t* __restrict__ s, uint8_t* __restrict__ out, float* __restrict__ out_s,
    const int32_t* __restrict__ lens, const int32_t* __restrict__ offs, const int32_t* __restrict__ soffs,
    int64_t total_rows, int64_t N, int64_t out_s_rows, float eps, bool out_line, int nsplits, int tm, int bands) {
  __shared__ WideSmem sm;
  int64_t len, start, sstart, bm, bn;
  if (!flat_split_tile<CHUNKS, WALK>(lens, offs, soffs, nsplits, tm, bands, &len, &start, &sstart, &bm, &bn)) return;
  msplit_wide_tile<NARROWN>(sm, q, s, out, out_s, len, start, sstart, bm, bn, total_rows, N, out_s_rows, eps, out_line);
}

// A split's output column c is a run of len bytes at off*N + c*len, so a
// tile's 128-row piece of a column starts at an arbitrary byte alignment.
// Each lane stores its 16 bytes of a column at their exact place: one 16 B
// store whatever the alignment (a previous version staged the pieces in LDS
// and wrote aligned 16 B blocks plus partial edge blocks; ragged cfg5 splits
// took 86.7 us that way against 60.8 us now, the same as 16-aligned splits).
// Row tile bm, 128-column band bn of a split (rows [start, start + len),
// scale rows from sstart), with the metadata checks of the wide form.
__device__ __forceinline__ void msplit_narrow_tile(RowColSmem& sm, const uint8_t* __restrict__ q,
                                                   const uint8_t* __restrict__ s, uint8_t* __restrict__ out,
                                                   float* __restrict__ out_s, int64_t len, int64_t start,
                                                   int64_t sstart, int64_t bm, int64_t bn, int64_t total_rows,
                                                   int64_t N, int64_t out_s_rows, float eps, bool vin, bool vs) {
  if (bm * kTile >= len) return;
  // Metadata arrives on the device; tiles whose rows or scale rows fall
  // outside the buffers are skipped rather than written out of bounds.
  if (start < 0 || start + len > total_rows || sstart < 0 || sstart + bm >= out_s_rows) return;
  const int64_t row0 = start + bm * kTile, col0 = bn * kTile;
  const int rows_valid = (int)(len - bm * kTile < kTile ? len - bm * kTile : kTile);
  rc_put(sm, rc_load(q, s, N, row0, rows_valid, col0, vin, vs));
  __syncthreads();
  LaneCols res;
  rc_tile<true>(sm, rows_valid, N, col0, 0.0f, eps, out_s + (sstart + bm) * N + col0, res);
  const int t = threadIdx.x, p = t >> 3, qq = t & 7;
  const int64_t c = col0 + 2 * p;
  if (c < N) {  // N is even: both columns or neither
    const int64_t o0 = start * N + c * len + bm * kTile + 16 * qq;
    rc_store(out + o0, res.e0, 16 * qq, rows_valid);
    rc_store(out + o0 + len, res.e1, 16 * qq, rows_valid);
  }
}

__global__ __launch_bounds__(kRcThreads) void row_to_fp8_col_msplit_kernel(
    const uint8_t* __restrict__ q, const uint8_t* __restrict__ s, uint8_t* __restrict__ out, float* __restrict__ out_s,
    const int32_t* __restrict__ lens, const int32_t* __restrict__ offs, const int32_t* __restrict__ soffs,
    int64_t total_rows, int64_t N, int64_t out_s_rows, float eps, bool vin, bool vs, int64_t bm0, int64_t bn0) {
  __shared__ RowColSmem sm;
  const int64_t split = blockIdx.x, bm = bm0 + blockIdx.y, bn = bn0 + blockIdx.z;
  const int64_t len = lens[split];
  if (bm * kTile >= len) return;
  msplit_narrow_tile(sm, q, s, out, out_s, len, offs[split], soffs[split], bm, bn, total_rows, N, out_s_rows, eps, vin,
                     vs);
}

// The 128-column tiles on the flat grid (at most 128 splits), as the wide
// form, for codes that are not 16 B aligned. On 16431 routed rows x 7040
// columns: 4, 16 and 32 uneven splits 71.4, 96.2 and 85.8 us against 94.1,
// 313.3 and 177.7 us on the 3-D grid; cfg5's 8 nearly equal splits 71.3
// against 65.8 us (the tile search of twice as many 512-thread workgroups
// costs more than the 3-D grid's one split per XCD, which any imbalance
// above about 8% undoes).
template <int CHUNKS>
__global__ __launch_bounds__(kRcThreads) void row_to_fp8_col_msplit_narrow_flat_kernel(
    const uint8_t* __restrict__ q, const uint8_t* __restrict__ s, uint8_t* __restrict__ out, float* __restrict__ out_s,
    const int32_t* __restrict__ lens, const int32_t* __restrict__ offs, const int32_t* __restrict__ soffs,
    int64_t total_rows, int64_t N, int64_t out_s_rows, float eps, bool vin, bool vs, int nsplits, int tm, int bands) {
  __shared__ RowColSmem sm;
  int64_t len, start, sstart, bm, bn;
  if (!flat_split_tile<CHUNKS, false>(lens, offs, soffs, nsplits, tm, bands, &len, &start, &sstart, &bm, &bn)) return;
  msplit_narrow_tile(sm, q, s, out, out_s, len, start, sstart, bm, bn, total_rows, N, out_s_rows, eps, vin, vs);
}

hipError_t launch_row_to_fp8_col(const void* q, const void* s, void* out, float* out_s, int64_t M, int64_t N, float eps,
                                 hipStream_t stream) {
  if (M == 0 || N == 0) return hipSuccess;
  const bool vin = (N % 32 == 0) && ((reinterpret_cast<uintptr_t>(q) & 15) == 0);
  const bool vs = (N % 128 == 0) && ((reinterpret_cast<uintptr_t>(s) & 3) == 0);
  const bool vout = (M % 16 == 0) && ((reinterpret_cast<uintptr_t>(out) & 15) == 0);
  const bool full = vin && vs && vout && (M % kTile == 0);
  if (vin) {
    // the 256-column tiles; their scale rows are read 8 bytes at a time when
    // 8 B aligned (N % 256 == 0), else byte by byte with the last band
    // partial. 4096 x 7040: 9.5 us against 12.6 us on the 128-column tiles;
    // 16384 x 7040: 29.2 against 56.0; 4096 x 2880: 5.6 against 8.4.
    const bool narrow_n = N % kWideCols != 0 || (reinterpret_cast<uintptr_t>(s) & 7) != 0;
    const bool whole = vout && M % kTile == 0;
    const dim3 grid((unsigned)(((M + kTile - 1) / kTile) * ((N + kWideCols - 1) / kWideCols)));
    auto kernel = narrow_n ? (whole ? row_to_fp8_col_wide_kernel<false, true> : row_to_fp8_col_wide_kernel<true, true>)
                           : (whole ? row_to_fp8_col_wide_kernel<false, false> : row_to_fp8_col_wide_kernel<true, false>);
    return launch(kernel, grid, dim3(256), 0, stream, static_cast<const uint8_t*>(q), static_cast<const uint8_t*>(s),
                  static_cast<uint8_t*>(out), out_s, M, N, eps);
  }
  const int64_t tiles_m = (M + kTile - 1) / kTile, tiles = tiles_m * ((N + kTile - 1) / kTile);
  // one wave of resident blocks: two 512-thread blocks per CU at this
  // kernel's register use (4 waves per SIMD)
  const int64_t grid_cap = 2 * (int64_t)current_device_caps().cus;
  const int64_t grid = tiles < grid_cap ? tiles : grid_cap;
  auto kernel = full ? row_to_fp8_col_kernel<true> : row_to_fp8_col_kernel<false>;
  return launch(kernel, dim3((unsigned)grid), dim3(kRcThreads), 0, stream, static_cast<const uint8_t*>(q),
                     static_cast<const uint8_t*>(s), static_cast<uint8_t*>(out), out_s, M, N, (int)tiles_m, (int)tiles,
                     eps, vin, vs);
}

hipError_t launch_row_to_fp8_col_msplit(const void* q, const void* s, void* out, float* out_s, int64_t total_rows,
                                        int64_t N, const int32_t* lens, const int32_t* offs, const int32_t* soffs,
                                        int64_t nsplits, int64_t max_split_len, int64_t out_capacity,
                                        int64_t out_s_rows, float eps, hipStream_t stream) {
  (void)out_capacity;  // the ABI layer checks out_capacity >= total_rows * N
  if (nsplits == 0 || max_split_len <= 0 || N == 0) return hipSuccess;
  const bool vin = (N % 32 == 0) && ((reinterpret_cast<uintptr_t>(q) & 15) == 0);
  const bool vs = (N % 128 == 0) && ((reinterpret_cast<uintptr_t>(s) & 3) == 0);
  const bool wide = vin;  // 256-column tiles (the last band partial where N % 256 != 0)
  const bool narrow_n = N % kWideCols != 0 || (reinterpret_cast<uintptr_t>(s) & 7) != 0;
  const int64_t tiles_m = (max_split_len + kTile - 1) / kTile;
  const int64_t bands = wide ? (N + kWideCols - 1) / kWideCols : (N + kTile - 1) / kTile;
  // Unused dynamic LDS caps the wide kernel's residency at 4 workgroups per
  // CU (6 by its own LDS and registers): fewer tiles' partial output lines
  // wait in L2 at once. Ragged cfg5 splits: 49.6 us against 51.0, and 59.8
  // against 62.8 right after a 512 MB fill (dirty caches, as in a layer step).
  const int per_wg = current_device_caps().lds_per_workgroup / 4 - 2560;
  const size_t reserve = per_wg > (int)sizeof(WideSmem) ? (size_t)(per_wg - (int)sizeof(WideSmem)) : 0;
  const bool out_line = (reinterpret_cast<uintptr_t>(out) & 127) == 0;
  // A launch holds at most 2^32 - 1 work-items along x (gridDim.x times the
  // workgroup size), so the flat grid's limit depends on the kernel's width.
  const int64_t flat_threads = wide ? 256 : kRcThreads;
  if (nsplits <= kFlatMaxSplits && tiles_m * bands + 7 <= (int64_t)UINT32_MAX / flat_threads / nsplits) {
    const dim3 grid((unsigned)flat_grid_blocks(nsplits, tiles_m, bands));
    if (wide) {
      // band walk up to 64 splits on rows of more than 16 bands, else contiguous ranges
      const bool walk = nsplits <= 64 && bands > 16;
      auto kernel = narrow_n ? (nsplits > 64 ? row_to_fp8_col_msplit_flat_kernel<2, false, true>
                                : walk     ? row_to_fp8_col_msplit_flat_kernel<1, true, true>
                                           : row_to_fp8_col_msplit_flat_kernel<1, false, true>)
                             : (nsplits > 64 ? row_to_fp8_col_msplit_flat_kernel<2, false, false>
                                : walk     ? row_to_fp8_col_msplit_flat_kernel<1, true, false>
                                           : row_to_fp8_col_msplit_flat_kernel<1, false, false>);
      return launch(kernel, grid, dim3(256), reserve, stream, static_cast<const uint8_t*>(q),
                    static_cast<const uint8_t*>(s), static_cast<uint8_t*>(out), out_s, lens, offs, soffs, total_rows, N,
                    out_s_rows, eps, out_line, (int)nsplits, (int)tiles_m, (int)bands);
    }
    auto kernel = nsplits <= 64 ? row_to_fp8_col_msplit_narrow_flat_kernel<1> : row_to_fp8_col_msplit_narrow_flat_kernel<2>;
    return launch(kernel, grid, dim3(kRcThreads), 0, stream, static_cast<const uint8_t*>(q),
                  static_cast<const uint8_t*>(s), static_cast<uint8_t*>(out), out_s, lens, offs, soffs, total_rows, N,
                  out_s_rows, eps, vin, vs, (int)nsplits, (int)tiles_m, (int)bands);
  }
  // Grid y (row tiles) and z (column bands) hold at most 65536 each: longer
  // splits or wider rows take several launches over offset ranges.
  for (int64_t bm0 = 0; bm0 < tiles_m; bm0 += kMaxGridYZ) {
    for (int64_t bn0 = 0; bn0 < bands; bn0 += kMaxGridYZ) {
      const dim3 grid((unsigned)nsplits, (unsigned)std::min<int64_t>(tiles_m - bm0, kMaxGridYZ),
                      (unsigned)std::min<int64_t>(bands - bn0, kMaxGridYZ));
      const hipError_t e =
          wide ? launch(narrow_n ? row_to_fp8_col_msplit_wide_kernel<true> : row_to_fp8_col_msplit_wide_kernel<false>,
                        grid, dim3(256), reserve, stream,
                        static_cast<const uint8_t*>(q), static_cast<const uint8_t*>(s), static_cast<uint8_t*>(out),
                        out_s, lens, offs, soffs, total_rows, N, out_s_rows, eps, out_line, bm0, bn0)
               : launch(row_to_fp8_col_msplit_kernel, grid, dim3(kRcThreads), 0, stream,
                        static_cast<const uint8_t*>(q), static_cast<const uint8_t*>(s), static_cast<uint8_t*>(out),
                        out_s, lens, offs, soffs, total_rows, N, out_s_rows, eps, vin, vs, bm0, bn0);
      if (e != hipSuccess) return e;
    }
  }
  return hipSuccess;
}

}  // namespace omo_hip
