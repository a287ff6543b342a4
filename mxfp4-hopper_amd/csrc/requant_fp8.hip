// MXFP4 -> FP8 E4M3 requant, rowwise (1x128 power-of-two scales stored
// transposed) and the transposed-output variant.
//
// Rowwise semantics follow omo_per_token_Mxfp4ToFp8_kernel
// (code/kernel/per_token_Mxfp4ToFp8.cu:92-235). Per 128-element group G
// (64 code bytes, 4 E8M0 bytes s[4G..4G+3]):
//   g   = (uint16)(max(s) - 6)                                 :162-165
//   y_s = fp32 with bits ((uint8)g) << 23, stored at [col*M + row] :172-180
//   per element: bf16(code) - ((uint16)(g - s_i) << 7) (mod 2^16), as fp32,
//   clamped by fmaxf(-448, fminf(448, .)), then E4M3 RNE.       :192-229
// The modular subtraction is kept exactly, including its wrap for zero
// codes (-448 when s_i <= max(s) - 7) and for max(s) < 6.
//
// Transposed semantics follow omo_per_token_Mxfp4ToFp8_col_kernel
// (code/kernel/per_token_Mxfp4ToFp8_col.cu:110-301) on 128-row x 128-byte
// tiles: per MX column c of the tile g_c = (uint8)(max(eps8, max_rows s) - 6),
// y_s(g_c) replicated over the column's 32 outputs of scale row by (:183-212),
// element value (bf16(code) - ((uint8)(g_c - s) << 7)) & 0x7FFF (sign
// dropped, :244-274), clamped by fminf(fmaxf(., -448), 448), E4M3 RNE, and
// written to [element_column * M + row] (:282-290).
#include "omo_device.cuh"
#include "omo_internal.h"

namespace omo_hip {

// ---------------------------------------------------------------- rowwise
// A code dword (8 elements) becomes 8 FP8 bytes; a lane converts two of them.
//
// The reference subtracts off = 128 * (adjust mod 512) from the bf16 pattern
// of each code, adjust = (uint16)(g - s_i). Write d for the signed value of
// adjust mod 512. Subtracting a multiple of 128 never touches the low 7 bits
// and flips bit 15 exactly when the code is negative, so the result for a
// negative code is the result for its magnitude with the sign flipped; after
// the symmetric clamp and E4M3 rounding that is a flip of bit 7, except
// where the pattern is a NaN (both signs clamp to +448).
//
// Fast path, d in [-6, 5]: code * 2^-d is a normal E4M3 value for every
// nonzero magnitude (0.5 * 2^-5 = 2^-6 at the bottom, 6 * 2^6 = 384 at the
// top), so its byte is the E4M3 pattern of the code with -d added to the
// exponent field: {0x30, 0x38, 0x3C, 0x40, 0x44, 0x48, 0x4C} - 8d. A zero
// code gives 0 for d <= 0 and the wrapped -inf -> -448 (0xFE) for d >= 1.
// No NaN pattern arises in this range. The eight bytes form a per-lane
// table; v_perm_b32 looks up four elements per instruction.
__device__ __forceinline__ u32x2 to_fp8_dword_fast(uint32_t c, int d) {
  const uint32_t sh = (uint32_t)(-8 * d);
  // every byte stays in [0x08, 0x7C], so whole-dword arithmetic is per-byte
  const uint32_t t_lo = (0x3C383000u + sh * 0x01010100u) | (d >= 1 ? 0xFEu : 0u);
  const uint32_t t_hi = 0x4C484440u + sh * 0x01010101u;
  const uint32_t lo = c & 0x0F0F0F0Fu, hi = (c >> 4) & 0x0F0F0F0Fu;
  const uint32_t a = __builtin_amdgcn_perm(hi, lo, 0x05010400u);  // nibbles of elements 0..3
  const uint32_t b = __builtin_amdgcn_perm(hi, lo, 0x07030602u);  // elements 4..7
  u32x2 o;
  o[0] = __builtin_amdgcn_perm(t_hi, t_lo, a & 0x07070707u) ^ ((a << 4) & 0x80808080u);
  o[1] = __builtin_amdgcn_perm(t_hi, t_lo, b & 0x07070707u) ^ ((b << 4) & 0x80808080u);
  return o;
}

// Reference restatement for one code dword under the 16-bit offset `offset`.
__device__ __forceinline__ u32x2 to_fp8_dword_ref(uint32_t c, uint32_t offset) {
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const uint32_t byte = (c >> (8 * k)) & 0xFFu;
    const uint32_t a0 = (e2m1_to_bf16_bits(byte & 0xFu) - offset) & 0xFFFFu;
    const uint32_t a1 = (e2m1_to_bf16_bits(byte >> 4) - offset) & 0xFFFFu;
    const float f0 = fmaxf(-448.0f, fminf(448.0f, bf16_to_f32(a0)));
    const float f1 = fmaxf(-448.0f, fminf(448.0f, bf16_to_f32(a1)));
    const uint32_t pr = fp8x2_from_f32(f0, f1);
    if (k < 2) lo |= pr << (16 * k); else hi |= pr << (16 * (k - 2));
  }
  u32x2 o;
  o[0] = lo;
  o[1] = hi;
  return o;
}

// Block tile: kRqRows rows x kRqGroups groups of 128 elements (256 code
// bytes per row, 8 KiB per block). Lane e of the tile (e = u * 256 + t)
// converts code pair c = e % (8 kRqGroups) of tile row e / (8 kRqGroups):
// 16 B stores, contiguous over 16-lane row pieces. The fp32 scales of a tile
// land in kRqGroups runs of kRqRows consecutive floats of the transposed
// scale tensor [K/128, M], each written whole by one block, so no 128 B line
// of it is assembled from partial writes of several workgroups on different
// XCDs. Codes are read and FP8 bytes written non-temporally (streamed once).
constexpr int kRqGroups = 4;
constexpr int kRqRows = 32;
template <int UNROLL>
__global__ __launch_bounds__(256) void mxfp4_to_fp8_kernel(const u32x2* __restrict__ q,
                                                           const uint32_t* __restrict__ s4,
                                                           u32x4* __restrict__ out, float* __restrict__ out_s,
                                                           uint32_t M, uint32_t gpr, uint32_t gx) {
  constexpr int PPR = 8 * kRqGroups;  // pairs per tile row
  const uint32_t bx = blockIdx.x % gx, by = blockIdx.x / gx;
  const int64_t ppr_all = 8 * (int64_t)gpr;
  u32x2 c[UNROLL];
  uint32_t sd[UNROLL];
#pragma unroll
  for (int u = 0; u < UNROLL; u++) {
    const int e = u * 256 + threadIdx.x;
    const uint32_t r = by * kRqRows + e / PPR, cp = bx * PPR + e % PPR;
    if (r < M && cp < 8 * gpr) {
      const int64_t i = (int64_t)r * ppr_all + cp;
      c[u] = __builtin_nontemporal_load(q + i);
      sd[u] = s4[i >> 3];
    }
  }
#pragma unroll
  for (int u = 0; u < UNROLL; u++) {
    const int e = u * 256 + threadIdx.x;
    const uint32_t r = by * kRqRows + e / PPR, cp = bx * PPR + e % PPR;
    if (r >= M || cp >= 8 * gpr) continue;
    const int64_t i = (int64_t)r * ppr_all + cp;
    const uint32_t s = sd[u];
    const uint32_t smax = max(max(s & 0xFFu, (s >> 8) & 0xFFu), max((s >> 16) & 0xFFu, s >> 24));
    const uint32_t g16 = (smax - 6u) & 0xFFFFu;
    const uint32_t s_i = (s >> (8 * ((uint32_t)(i & 7) >> 1))) & 0xFFu;
    const uint32_t adj = (g16 - s_i) & 0xFFFFu;
    const int d = (int)(adj & 511u) - ((adj & 256u) ? 512 : 0);
    u32x2 o0, o1;
    if ((unsigned)(d + 6) <= 11u) {
      o0 = to_fp8_dword_fast(c[u][0], d);
      o1 = to_fp8_dword_fast(c[u][1], d);
    } else {
      const uint32_t offset = (adj << 7) & 0xFFFFu;
      o0 = to_fp8_dword_ref(c[u][0], offset);
      o1 = to_fp8_dword_ref(c[u][1], offset);
    }
    u32x4 o;
    o[0] = o0[0];
    o[1] = o0[1];
    o[2] = o1[0];
    o[3] = o1[1];
    __builtin_nontemporal_store(o, out + i);
    if ((cp & 7) == 0) out_s[(int64_t)(cp >> 3) * M + r] = __uint_as_float((g16 & 0xFFu) << 23);
  }
}

hipError_t launch_mxfp4_to_fp8(const void* q, const void* s, void* out, float* out_s, int64_t M, int64_t Kb,
                               hipStream_t stream) {
  if (M == 0 || Kb == 0) return hipSuccess;
  constexpr int U = kRqRows * 8 * kRqGroups / 256;
  const int64_t gpr = Kb / 64;
  const int64_t gx = (gpr + kRqGroups - 1) / kRqGroups, gy = (M + kRqRows - 1) / kRqRows;
  hipLaunchKernelGGL((mxfp4_to_fp8_kernel<U>), dim3((unsigned)(gx * gy)), dim3(256), 0, stream,
                     static_cast<const u32x2*>(q), static_cast<const uint32_t*>(s), static_cast<u32x4*>(out), out_s,
                     (uint32_t)M, (uint32_t)gpr, (uint32_t)gx);
  return hipGetLastError();
}

// ------------------------------------------------------------ transposed
// One 256-thread block per 128-row x 128-byte tile. The code tile and its
// 128x8 scale bytes are staged in LDS; each thread then produces one output
// row segment (one element column of the tile, 128 contiguous FP8 bytes =
// a full 128 B line).
constexpr int kColTile = 128;
constexpr int kColPitch = kColTile + 4;

__global__ __launch_bounds__(256) void mxfp4_to_fp8_col_kernel(const uint8_t* __restrict__ q,
                                                               const uint8_t* __restrict__ s,
                                                               uint8_t* __restrict__ out, float* __restrict__ out_s,
                                                               int64_t M, int64_t Kb, uint32_t eps8) {
  __shared__ uint8_t tile[kColTile * kColPitch];
  __shared__ uint8_t stile[kColTile][8];
  __shared__ uint32_t gpart[4][8];
  __shared__ uint32_t gcol[8];
  const int t = threadIdx.x;
  const int64_t bx = blockIdx.x, by = blockIdx.y;
  const int64_t row0 = by * kColTile;
  const int64_t sstride = Kb / 16;
  // codes: 128 rows x 128 B = 1024 chunks of 16 B
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int cidx = t + 256 * k;
    const int r = cidx >> 3, c16 = cidx & 7;
    const u32x4 v = *reinterpret_cast<const u32x4*>(q + (row0 + r) * Kb + bx * kColTile + c16 * 16);
    uint32_t* dst = reinterpret_cast<uint32_t*>(tile + r * kColPitch + c16 * 16);
    dst[0] = v[0];
    dst[1] = v[1];
    dst[2] = v[2];
    dst[3] = v[3];
  }
  if (t < kColTile) {
    const u32x2 sv = *reinterpret_cast<const u32x2*>(s + (row0 + t) * sstride + bx * 8);
    *reinterpret_cast<u32x2*>(&stile[t][0]) = sv;
  }
  __syncthreads();
  // per MX column: max over 128 rows (seeded with (uint8)eps)
  {
    const int c = t & 7, rq = t >> 3;  // rows 4rq..4rq+3
    uint32_t m = eps8;
#pragma unroll
    for (int j = 0; j < 4; j++) m = max(m, (uint32_t)stile[rq * 4 + j][c]);
    m = max(m, (uint32_t)__shfl_xor((int)m, 8));
    m = max(m, (uint32_t)__shfl_xor((int)m, 16));
    m = max(m, (uint32_t)__shfl_xor((int)m, 32));
    if ((t & 63) < 8) gpart[t >> 6][c] = m;
  }
  __syncthreads();
  if (t < 8) {
    const uint32_t m = max(max(gpart[0][t], gpart[1][t]), max(gpart[2][t], gpart[3][t]));
    gcol[t] = (m - 6u) & 0xFFu;
  }
  __syncthreads();
  // scale row by: 256 floats, entry j holds column j/32
  out_s[by * (Kb * 2) + bx * 256 + t] = __uint_as_float(gcol[t >> 5] << 23);
  // outputs: thread t -> element column e = t of the tile (byte t/2, nibble t&1)
  const int b = t >> 1, h = t & 1, cblk = b >> 4;
  const uint32_t g = gcol[cblk];
  uint8_t* orow = out + (bx * 256 + t) * M + row0;
#pragma unroll
  for (int m16 = 0; m16 < kColTile; m16 += 16) {
    uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < 16; j++) {
      const int r = m16 + j;
      const uint32_t val = tile[r * kColPitch + b];
      const uint32_t nib = h ? (val >> 4) : (val & 0xFu);
      const uint32_t adj = (g - (uint32_t)stile[r][cblk]) & 0xFFu;
      const uint32_t a = ((e2m1_to_bf16_bits(nib) - (adj << 7)) & 0xFFFFu) & 0x7FFFu;
      const float f = fminf(fmaxf(bf16_to_f32(a), -448.0f), 448.0f);
      const uint32_t byte = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(f, f, 0, false) & 0xFFu;
      w[j >> 2] |= byte << (8 * (j & 3));
    }
    u32x4 o;
    o[0] = w[0];
    o[1] = w[1];
    o[2] = w[2];
    o[3] = w[3];
    __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(orow + m16));
  }
}

hipError_t launch_mxfp4_to_fp8_col(const void* q, const void* s, void* out, float* out_s, int64_t M, int64_t Kb,
                                   float eps, hipStream_t stream) {
  if (M == 0 || Kb == 0) return hipSuccess;
  uint32_t eps8 = 0;
  if (eps > 0.0f) eps8 = eps >= 255.0f ? 255u : (uint32_t)eps;  // (uint8_t)eps, truncating
  dim3 grid((unsigned)(Kb / kColTile), (unsigned)(M / kColTile));
  hipLaunchKernelGGL(mxfp4_to_fp8_col_kernel, grid, dim3(256), 0, stream, static_cast<const uint8_t*>(q),
                     static_cast<const uint8_t*>(s), static_cast<uint8_t*>(out), out_s, M, Kb, eps8);
  return hipGetLastError();
}

}  // namespace omo_hip
