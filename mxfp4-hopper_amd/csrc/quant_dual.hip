// Fused dual-layout BF16 -> MXFP4 quantize: rowwise 1x32 blocks along K and
// columnwise 32x1 blocks along M from one read of the input.
//
// The columnwise output is defined by the TE integration as
// quant_rowwise(X.T.contiguous()) (code/transformer_engine-2.8.diff:1463-1466):
// codes [K, M/2] and scales [K, M/32]. The reference pays a full transpose
// copy plus a second quantize pass for it. Both layouts here use the
// reference block rule (code/kernel/per_token_quant_mxfp4.cu:151-254) with
// fp4_min = -6, fp4_max = 6, the constants of the quantize wrapper
// (code/kernel/api/mxfp4.py:11-12, 152-154).
//
// Tiles are 64 rows x 256 columns (32 KiB of bf16), 512 threads. Each lane
// loads 4 chunks of 16 B (rows r0 + 16k of one 16 B column chunk); the
// rowwise blocks are quantized from registers exactly as in the rowwise
// kernel (a block is a DPP quad) and their codes leave as full 128 B lines
// (non-temporal stores). The tile is staged in LDS without padding: the 16 B
// chunks of each 16-row band are XOR-swizzled so the column pass reads four
// bands from four different 64 B bank ranges. In the column pass, lanes
// 4i..4i+3 own column pair i, one 16-row half of a 32-row block each: a lane
// reads one dword (two adjacent columns) from 16 rows, repacks the columns
// into bf16 pairs with v_perm_b32, combines the block amax with its partner
// lane (DPP), and converts its half block to 8 code bytes per column. The
// four lanes' 8 B stores then write each column's 32 B piece of the
// transposed codes as one contiguous run. (With the two 16 B halves of a
// piece stored by different waves, each store instruction touched 64
// different lines; pairing them cut the 7168 x 18432 kernel from 93 to 83 us.)
//
#include "omo_internal.h"
#include "omo_quant.cuh"

namespace omo_hip {

constexpr int kDualRows = 64;
constexpr int kDualCols = 256;
constexpr int kDualPitch = kDualCols * 2;  // bytes per LDS row (no padding: swizzled)
constexpr int kXcds = 8;
constexpr int kDualGroupMax = 32;
constexpr int kDualThreads = 512;

// Half of a 32-element column block: 8 packed bf16 pairs (rows 2j low, 2j+1
// high); amax_bits is the whole block's max |x| bit pattern (< 0x7F80).
// Returns the 8 code bytes.
__device__ __forceinline__ uint2 quant_half16_fast(const uint32_t (&p)[8], uint32_t amax_bits, int c_eps,
                                                   uint32_t* byte) {
  const float y_s = fast_block_scale(amax_bits, c_eps, byte);
  uint2 out;
  uint32_t r = p[0];  // all four bytes are written
  r = cvt_pk_fp4<0>(r, p[0], y_s);
  r = cvt_pk_fp4<1>(r, p[1], y_s);
  r = cvt_pk_fp4<2>(r, p[2], y_s);
  r = cvt_pk_fp4<3>(r, p[3], y_s);
  out.x = r;
  r = p[4];
  r = cvt_pk_fp4<0>(r, p[4], y_s);
  r = cvt_pk_fp4<1>(r, p[5], y_s);
  r = cvt_pk_fp4<2>(r, p[6], y_s);
  r = cvt_pk_fp4<3>(r, p[7], y_s);
  out.y = r;
  return out;
}

// Reference emulation for a half block; the two lanes holding a block's
// halves (lanes 2i, 2i+1) call it together.
__device__ __forceinline__ uint2 quant_half16_ref(const uint32_t (&p)[8], float eps, uint32_t* byte) {
  float amax = eps;
#pragma unroll
  for (int k = 0; k < 8; k++) {
    amax = fmax_abs_bf16(amax, p[k]);
    amax = fmax_abs_bf16(amax, p[k] >> 16);
  }
  amax = fmaxf(amax, __uint_as_float(dpp_quad_xor1(__float_as_uint(amax))));
  float inv;
  *byte = ref_scale(amax, 6.0f, &inv);
  uint32_t o[2];
#pragma unroll
  for (int w = 0; w < 2; w++) {
    uint32_t v = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint32_t pk = p[4 * w + k];
      const float qx = fminf(fmaxf(bf16_to_f32(pk & 0xFFFFu) * inv, -6.0f), 6.0f);
      const float qy = fminf(fmaxf(bf16_to_f32(pk >> 16) * inv, -6.0f), 6.0f);
      v |= (e2m1_from_f32_ref(qx) | (e2m1_from_f32_ref(qy) << 4)) << (8 * k);
    }
    o[w] = v;
  }
  return make_uint2(o[0], o[1]);
}

// One 64 x 256 tile (index `logical`, M-fastest) of the [M, K] tensor x,
// 512 threads.
__device__ __forceinline__ void dual_tile(const uint16_t* __restrict__ x, uint32_t* __restrict__ row_q,
                                          uint8_t* __restrict__ row_s, uint8_t* __restrict__ col_q,
                                          uint8_t* __restrict__ col_s, int64_t M, int64_t K, int tiles_m,
                                          int logical, float eps, int c_eps, uint8_t* tile, uint8_t* rs_tile) {
  const int t = threadIdx.x;
  const int64_t mt = logical % tiles_m, kt = logical / tiles_m;
  const int64_t m0 = mt * kDualRows, k0 = kt * kDualCols;
  const int rows_valid = (int)(M - m0 < kDualRows ? M - m0 : kDualRows);  // 32 or 64
  // lane t owns 16 B column chunk cc of rows r0 + 16k (k = 0..3)
  const int r0 = t >> 5, cc = t & 31;
  const int64_t col = k0 + cc * 8;
  const int64_t cl = col < K ? col : K - 8;
  u32x4 d[4];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int r = r0 + 16 * k;
    const int rr = r < rows_valid ? r : rows_valid - 1;
    d[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(x + (m0 + rr) * K + cl));
  }
  const bool quad_leader = (t & 3) == 0;
  uint32_t* rq = row_q + (m0 + r0) * (K / 8) + col / 8;
  uint32_t codes[4];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    // row r0 + 16k is in 16-row band k: its chunks are stored XORed by 4k,
    // so the four bands sit in four different 64 B bank ranges
    *reinterpret_cast<u32x4*>(tile + (r0 + 16 * k) * kDualPitch + ((cc ^ (k << 2)) * 16)) = d[k];
    uint32_t byte;
    const uint32_t am = quad_max_u32(chunk_absmax_bits(d[k]));
    if (__builtin_expect(am < 0x7F80u, 1)) {
      codes[k] = quant_chunk_fast(d[k], am, c_eps, &byte);
    } else {
      quant_chunk_ref(d[k], eps, -6.0f, 6.0f, &codes[k], &byte);
    }
    // the 8 scale bytes of a tile row are gathered in LDS and leave as one store
    if (quad_leader) rs_tile[(r0 + 16 * k) * 8 + (cc >> 2)] = (uint8_t)byte;
  }
  // The code stores follow all four conversions: a store under the bounds
  // test ahead of the next chunk made the wait for that chunk's load wait
  // for the store as well (loads and stores share one counter).
#pragma unroll
  for (int k = 0; k < 4; k++)
    if (r0 + 16 * k < rows_valid && col < K) __builtin_nontemporal_store(codes[k], rq + k * 2 * K);  // 16 rows down
  __syncthreads();
  if (t < rows_valid) {
    uint8_t* rs = row_s + (m0 + t) * (K / 32) + k0 / 32;
    const int nsc = (int)((K - k0) / 32 < 8 ? (K - k0) / 32 : 8);
    if (nsc == 8 && (reinterpret_cast<uintptr_t>(rs) & 7) == 0) {
      *reinterpret_cast<uint2*>(rs) = *reinterpret_cast<const uint2*>(rs_tile + t * 8);
    } else {
      for (int j = 0; j < nsc; j++) rs[j] = rs_tile[t * 8 + j];
    }
  }
  // ---- columnwise: lanes 4i..4i+3 own column pair i; lane 4i + 2g + h holds
  // rows 32g + 16h .. +15 (half h of row block g), so the four lanes' 8 B
  // code stores form the column's 32 B piece
  const int h = t & 1, g = (t >> 1) & 1, p = t >> 2;
  const int64_t kc = k0 + 2 * p;
  // every lane runs the column pass (rows and columns past the tensor read
  // the tile's clamped copies) so that the scale exchange below sees all
  // lanes; only valid results are stored
  const bool active = 32 * g < rows_valid && kc < K;
  const int band = 2 * g + h;
  const int pp = 4 * (p ^ (band << 4));
  uint32_t ca[8], cb[8];
  uint32_t amax_a = 0, amax_b = 0;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const uint32_t w0 = *reinterpret_cast<const uint32_t*>(tile + (16 * band + 2 * j) * kDualPitch + pp);
    const uint32_t w1 = *reinterpret_cast<const uint32_t*>(tile + (16 * band + 2 * j + 1) * kDualPitch + pp);
    ca[j] = __builtin_amdgcn_perm(w1, w0, 0x05040100u);  // column 2p: rows 2j (low), 2j+1 (high)
    cb[j] = __builtin_amdgcn_perm(w1, w0, 0x07060302u);  // column 2p+1
    amax_a = pk_max_u16(amax_a, ca[j] & 0x7FFF7FFFu);
    amax_b = pk_max_u16(amax_b, cb[j] & 0x7FFF7FFFu);
  }
  amax_a = max(amax_a & 0xFFFFu, amax_a >> 16);
  amax_b = max(amax_b & 0xFFFFu, amax_b >> 16);
  amax_a = max(amax_a, dpp_quad_xor1(amax_a));  // the other half of the block
  amax_b = max(amax_b, dpp_quad_xor1(amax_b));
  uint32_t byte_a, byte_b;
  uint2 qa, qb;
  if (__builtin_expect(amax_a < 0x7F80u, 1)) qa = quant_half16_fast(ca, amax_a, c_eps, &byte_a);
  else qa = quant_half16_ref(ca, eps, &byte_a);
  if (__builtin_expect(amax_b < 0x7F80u, 1)) qb = quant_half16_fast(cb, amax_b, c_eps, &byte_b);
  else qb = quant_half16_ref(cb, eps, &byte_b);
  const int64_t mo = (m0 + 16 * band) / 2;
  if (active) {
    *reinterpret_cast<uint2*>(col_q + kc * (M / 2) + mo) = qa;
    *reinterpret_cast<uint2*>(col_q + (kc + 1) * (M / 2) + mo) = qb;
  }
  // A column's two scale bytes of this tile (row blocks g = 0, 1) sit in
  // lanes 4p + 2g; swapping them (quad lane ^ 2) lets lane 4p write column
  // kc's pair and lane 4p + 2 column kc + 1's as one 2-byte store each.
  const uint32_t oa = dpp_quad_xor2(byte_a), ob = dpp_quad_xor2(byte_b);
  if (h == 0 && kc < K) {
    const int64_t so = m0 / 32;  // even: m0 is a multiple of 64
    uint8_t* const cs = col_s + (kc + g) * (M / 32) + so;
    if (rows_valid == kDualRows && (M / 32) % 2 == 0 && (reinterpret_cast<uintptr_t>(col_s) & 1) == 0) {
      const uint32_t pair = g == 0 ? (byte_a | (oa << 8)) : (ob | (byte_b << 8));
      *reinterpret_cast<uint16_t*>(cs) = (uint16_t)pair;
    } else if (active) {
      col_s[kc * (M / 32) + so + g] = (uint8_t)byte_a;
      col_s[(kc + 1) * (M / 32) + so + g] = (uint8_t)byte_b;
    }
  }
}

// ---- four tiles per workgroup, for M % 64 == 0 and K % 256 == 0
//
// A workgroup quantizes the (up to) four vertically adjacent 64 x 256 tiles
// of a 256-row super-tile one after the other, as dual_tile does, and keeps
// each lane's transposed-code pieces (8 B per column and tile) and column
// scale pairs in registers. After the last tile the pieces are staged in LDS
// (the tile buffer, now free) and leave as whole 128 B column lines, eight
// lanes per line in one store instruction, and each column's 8 scale bytes
// as one 8-byte store. A tile's rowwise codes and scale bytes are staged in
// LDS too and stored one tile later, after that tile's loads were consumed:
// loads and stores share one vector-memory counter, so a store issued just
// ahead of a load makes the wait for that load wait for the store as well.
// Memory-only copies of this schedule (the same loads and stores, no
// arithmetic) run within 1-2 us of the kernel: its time is set by the mix of
// the strided 512 B row reads with the 128 B code lines and the 8-byte scale
// pieces, whose lines other workgroups complete. Rowwise codes leave
// non-temporally and the column lines through L2: temporal row codes ran
// the same, non-temporal column lines 79 against 75-78 us (and, in the
// band-group order, 76.5 against 71.7 us).
constexpr int kSuperSteps = 4;
constexpr int kSuperRows = kDualRows * kSuperSteps;  // 256

struct DualSuperSmem {
  // the staged 64 x 256 input tile; after a super-tile's last tile, its
  // transposed codes [256 columns][128 B] (16 B pieces XOR-swizzled by column)
  __attribute__((aligned(16))) uint8_t tile[kDualRows * kDualPitch];
  __attribute__((aligned(16))) uint32_t row_codes[2][kDualRows * kDualCols / 8];  // by tile parity
  __attribute__((aligned(8))) uint8_t row_scales[2][kDualRows * 8];
};

// Byte offset of transposed-code byte `b` (0..127) of column c in the staging area.
__device__ __forceinline__ int col_stage_off(int c, int b) { return c * 128 + ((((b >> 4) ^ c) & 7) << 4) + (b & 15); }

// Rowwise codes and scale bytes of one tile (64 rows from m0), staged in
// buffer `buf`: each lane stores 16 code bytes (8 lanes per 128 B line of a
// row) and lanes 0..63 one row's 8 scale bytes.
__device__ __forceinline__ void dual_row_flush(const DualSuperSmem& sm, int buf, uint32_t* __restrict__ row_q,
                                               uint8_t* __restrict__ row_s, int64_t m0, int64_t k0, int64_t K,
                                               bool rs_vec) {
  const int t = threadIdx.x;
  const int row = t >> 3, piece = t & 7;
  const u32x4 c = *reinterpret_cast<const u32x4*>(&sm.row_codes[buf][row * (kDualCols / 8) + 4 * piece]);
  __builtin_nontemporal_store(c, reinterpret_cast<u32x4*>(row_q + (m0 + row) * (K / 8) + k0 / 8 + 4 * piece));
  if (t < kDualRows) {
    uint8_t* rs = row_s + (m0 + t) * (K / 32) + k0 / 32;
    const uint2 v = *reinterpret_cast<const uint2*>(&sm.row_scales[buf][t * 8]);
    if (rs_vec) {
      *reinterpret_cast<uint2*>(rs) = v;
    } else {
      for (int j = 0; j < 8; j++) rs[j] = (uint8_t)((j < 4 ? v.x : v.y) >> (8 * (j & 3)));
    }
  }
}

__device__ __forceinline__ void dual_super4(const uint16_t* __restrict__ x, uint32_t* __restrict__ row_q,
                                            uint8_t* __restrict__ row_s, uint8_t* __restrict__ col_q,
                                            uint8_t* __restrict__ col_s, int64_t M, int64_t K, int ms, int kb,
                                            float eps, int c_eps, DualSuperSmem& sm) {
  const int t = threadIdx.x;
  const int64_t m0s = (int64_t)ms * kSuperRows, k0 = (int64_t)kb * kDualCols;
  const int steps = (int)((M - m0s) / kDualRows < kSuperSteps ? (M - m0s) / kDualRows : kSuperSteps);
  const int r0 = t >> 5, cc = t & 31;
  const bool quad_leader = (t & 3) == 0;
  const int h = t & 1, g = (t >> 1) & 1, p = t >> 2;
  const int band = 2 * g + h;
  const int pp = 4 * (p ^ (band << 4));
  const int64_t kc = k0 + 2 * p;
  const bool rs_vec = (reinterpret_cast<uintptr_t>(row_s) & 7) == 0;
  uint2 acc_a[4], acc_b[4];  // [tile] -> this lane's 8 B of columns kc, kc + 1
#pragma unroll
  for (int s = 0; s < 4; s++) acc_a[s] = acc_b[s] = make_uint2(0u, 0u);
  uint32_t sc_lo = 0, sc_hi = 0;  // scale pairs of column kc + g, tile s at bytes 2s, 2s + 1
  for (int st = 0; st < steps; st++) {
    const int64_t m0 = m0s + st * kDualRows;
    const int buf = st & 1;
    const uint16_t* src = x + (m0 + r0) * K + k0 + cc * 8;
    u32x4 d[4];
#pragma unroll
    for (int k = 0; k < 4; k++) d[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + 16 * k * K));
#pragma unroll
    for (int k = 0; k < 4; k++) {
      *reinterpret_cast<u32x4*>(sm.tile + (r0 + 16 * k) * kDualPitch + ((cc ^ (k << 2)) * 16)) = d[k];
      uint32_t codes, byte;
      const uint32_t am = quad_max_u32(chunk_absmax_bits(d[k]));
      if (__builtin_expect(am < 0x7F80u, 1)) {
        codes = quant_chunk_fast(d[k], am, c_eps, &byte);
      } else {
        quant_chunk_ref(d[k], eps, -6.0f, 6.0f, &codes, &byte);
      }
      sm.row_codes[buf][(r0 + 16 * k) * (kDualCols / 8) + cc] = codes;
      if (quad_leader) sm.row_scales[buf][(r0 + 16 * k) * 8 + (cc >> 2)] = (uint8_t)byte;
    }
    if (st > 0) dual_row_flush(sm, buf ^ 1, row_q, row_s, m0 - kDualRows, k0, K, rs_vec);
    __syncthreads();
    uint32_t ca[8], cb[8];
    uint32_t amax_a = 0, amax_b = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const uint32_t w0 = *reinterpret_cast<const uint32_t*>(sm.tile + (16 * band + 2 * j) * kDualPitch + pp);
      const uint32_t w1 = *reinterpret_cast<const uint32_t*>(sm.tile + (16 * band + 2 * j + 1) * kDualPitch + pp);
      ca[j] = __builtin_amdgcn_perm(w1, w0, 0x05040100u);
      cb[j] = __builtin_amdgcn_perm(w1, w0, 0x07060302u);
      amax_a = pk_max_u16(amax_a, ca[j] & 0x7FFF7FFFu);
      amax_b = pk_max_u16(amax_b, cb[j] & 0x7FFF7FFFu);
    }
    amax_a = max(amax_a & 0xFFFFu, amax_a >> 16);
    amax_b = max(amax_b & 0xFFFFu, amax_b >> 16);
    amax_a = max(amax_a, dpp_quad_xor1(amax_a));
    amax_b = max(amax_b, dpp_quad_xor1(amax_b));
    uint32_t byte_a, byte_b;
    uint2 qa, qb;
    if (__builtin_expect(amax_a < 0x7F80u, 1)) qa = quant_half16_fast(ca, amax_a, c_eps, &byte_a);
    else qa = quant_half16_ref(ca, eps, &byte_a);
    if (__builtin_expect(amax_b < 0x7F80u, 1)) qb = quant_half16_fast(cb, amax_b, c_eps, &byte_b);
    else qb = quant_half16_ref(cb, eps, &byte_b);
#pragma unroll
    for (int s = 0; s < 4; s++) {
      if (s == st) {
        acc_a[s] = qa;
        acc_b[s] = qb;
      }
    }
    const uint32_t oa = dpp_quad_xor2(byte_a), ob = dpp_quad_xor2(byte_b);
    const uint32_t pair = g == 0 ? (byte_a | (oa << 8)) : (ob | (byte_b << 8));
    if (st < 2) sc_lo |= pair << (16 * st);
    else sc_hi |= pair << (16 * (st - 2));
    __syncthreads();  // this tile's LDS reads are done before the next tile's writes
  }
  dual_row_flush(sm, (steps - 1) & 1, row_q, row_s, m0s + (int64_t)(steps - 1) * kDualRows, k0, K, rs_vec);
  {
    const int tt = opaque_tid(), pl = tt >> 2, bl = tt & 3;
#pragma unroll
    for (int s = 0; s < 4; s++) {
      if (s < steps) {
        *reinterpret_cast<uint2*>(sm.tile + col_stage_off(2 * pl, 32 * s + 8 * bl)) = acc_a[s];
        *reinterpret_cast<uint2*>(sm.tile + col_stage_off(2 * pl + 1, 32 * s + 8 * bl)) = acc_b[s];
      }
    }
  }
  __syncthreads();
  {
    const int tc = opaque_tid();
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int c = (tc >> 3) + 64 * j, piece = tc & 7;
      if (piece < 2 * steps) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(sm.tile + col_stage_off(c, 16 * piece));
        *reinterpret_cast<u32x4*>(col_q + (k0 + c) * (M / 2) + m0s / 2 + 16 * piece) = v;
      }
    }
  }
  if (h == 0) {  // lane g: column kc + g's scale bytes of the super-tile
    uint8_t* cs = col_s + (kc + g) * (M / 32) + m0s / 32;
    if (steps == kSuperSteps && (reinterpret_cast<uintptr_t>(cs) & 7) == 0) {
      *reinterpret_cast<uint2*>(cs) = make_uint2(sc_lo, sc_hi);
    } else {
      for (int j = 0; j < 2 * steps; j++) cs[j] = (uint8_t)((j < 4 ? sc_lo : sc_hi) >> (8 * (j & 3)));
    }
  }
}

// Super-tile order of the four-tile kernels. The S x B super-tiles of a
// tensor (S super-rows, B bands of 256 columns), numbered M-fastest
// (L = band * S + super-row), are cut into eight contiguous ranges of
// per_xcd = ceil(S * B / 8), one per XCD, so each XCD owns a group of whole
// bands (the ends of its range may be parts of bands). Each XCD walks its
// range super-row by super-row: all of its bands of super-row m, then those of
// m + 1. The eight XCDs thus sweep the tensor's rows together: at any moment
// the chip reads a few whole 256-row stripes of the input, each row's codes
// are written by all XCDs at about the same time, and each XCD's column codes
// fill its own contiguous region. Memory-only copies of the schedule at 7168 x
// 18432 (heavy-tailed weights, rotating buffers): 68.0 us against 73.3 us for
// M-fastest ranges (each XCD finishing one band before the next) and 73.4 us
// for K-fastest ones (the XCDs on different stripes), which also write 10 MB
// more (scale lines leaving L2 partly filled); the kernel 71.6 us against
// 76.6 us in M-fastest ranges. Returns false past the XCD's range.
__device__ __forceinline__ bool band_group_tile(int xcd, int j, int S, int T, int per_xcd, int* ms, int* kb) {
  const int lo = xcd * per_xcd, hi = min(T, lo + per_xcd);
  if (j >= hi - lo) return false;
  const int kb0 = lo / S, ms0 = lo - kb0 * S;  // first tile of the range
  const int kb1 = hi / S, ms1 = hi - kb1 * S;  // one past the last
  // tiles of the range in super-rows below m: band kb0 holds super-rows
  // [ms0, S) (or [ms0, ms1) when kb0 == kb1), bands kb0 + 1 .. kb1 - 1 all,
  // band kb1 [0, ms1)
  auto below = [&](int m) {
    if (kb0 == kb1) return max(0, min(m, ms1) - ms0);
    return m * (kb1 - kb0 - 1) + max(0, m - ms0) + min(m, ms1);
  };
  int a = 0, b = S;  // below(a) <= j < below(b) = hi - lo
  while (b - a > 1) {
    const int mid = (a + b) >> 1;
    if (below(mid) <= j) a = mid;
    else b = mid;
  }
  *ms = a;
  *kb = kb0 + (a >= ms0 ? 0 : 1) + (j - below(a));
  return true;
}

// At most 80 VGPRs (six waves per SIMD): three 512-thread workgroups per CU,
// which the LDS (52 KB each) also allows; at 86 the compiler's own choice,
// two fit and the kernel ran 8% slower. Loading the next tile into the
// registers the row pass has consumed, before the column pass, needs 95
// (two workgroups per CU: 72.75 against 72.0 us at cfg3); within 80 even a
// one-chunk prefetch spills.
__global__ __launch_bounds__(kDualThreads) __attribute__((amdgpu_waves_per_eu(6))) void quant_dual_super_kernel(
    const uint16_t* __restrict__ x, uint32_t* __restrict__ row_q, uint8_t* __restrict__ row_s,
    uint8_t* __restrict__ col_q, uint8_t* __restrict__ col_s, int64_t M, int64_t K, int tiles_ms, int tiles,
    int per_xcd, float eps, int c_eps) {
  __shared__ DualSuperSmem sm;
  const int b = blockIdx.x;
  int ms, kb;
  if (!band_group_tile(b % kXcds, b / kXcds, tiles_ms, tiles, per_xcd, &ms, &kb)) return;
  dual_super4(x, row_q, row_s, col_q, col_s, M, K, ms, kb, eps, c_eps, sm);
}

// band_group: the 64-row tiles in band-group order (band_group_tile over
// tiles instead of super-tiles), else each XCD takes a contiguous M-fastest
// range. Measured (graph replays): 8192 x 7168 37.1 us against 38.3, 4096 x
// 7168 20.7 against 21.1; with fewer than six tiles per CU the ranges are
// ahead (7168 x 2048 11.7 against 12.0, 2048 x 2048 5.5 against 5.9).
__global__ __launch_bounds__(kDualThreads) void quant_dual_kernel(const uint16_t* __restrict__ x, uint32_t* __restrict__ row_q,
                                                         uint8_t* __restrict__ row_s, uint8_t* __restrict__ col_q,
                                                         uint8_t* __restrict__ col_s, int64_t M, int64_t K,
                                                         int tiles_m, int tiles, int per_xcd, bool band_group, float eps,
                                                         int c_eps) {
  __shared__ __attribute__((aligned(16))) uint8_t tile[kDualRows * kDualPitch];
  __shared__ __attribute__((aligned(8))) uint8_t rs_tile[kDualRows * 8];
  const int b = blockIdx.x;
  int logical;
  if (band_group) {
    int ms, kb;
    if (!band_group_tile(b % kXcds, b / kXcds, tiles_m, tiles, per_xcd, &ms, &kb)) return;
    logical = kb * tiles_m + ms;
  } else {
    logical = (b % kXcds) * per_xcd + b / kXcds;
    if (logical >= tiles) return;
  }
  dual_tile(x, row_q, row_s, col_q, col_s, M, K, tiles_m, logical, eps, c_eps, tile, rs_tile);
}

// Grouped form: one launch over up to kDualGroupMax tensors (e.g. the weights
// of all local experts). Every XCD takes its band-group share of each item,
// item after item, so the XCDs sweep the items one after another together.
// The descriptor table travels by value in the kernel arguments.
struct DualItem {
  const uint16_t* x;
  uint32_t* row_q;
  uint8_t* row_s;
  uint8_t* col_q;
  uint8_t* col_s;
  int64_t M, K;
  int tiles_m;         // the item's tile rows (64 or 256 rows each, by kernel)
  int tiles, per_xcd;  // its tiles and their per-XCD share
};

struct DualGroup {
  DualItem item[kDualGroupMax];
  int count, tiles, per_xcd, c_eps;
  float eps;
};

// Each XCD takes its band-group share of each item, item after item, over
// the items' 64-row tiles. cfg5's 24 expert weights (16 of 7168 x 2048, 8 of
// 2048 x 7168, 224 super-tiles each): 208.8 us against 212.3 us for the
// four-tile kernel over contiguous ranges of all items' super-tiles, 214.4 us
// with contiguous ranges of all items' 64-row tiles and 223-226 us with whole
// items per XCD. Smaller items as well: 8 of 2048 x 2048 24.1 against 25.3 us
// with the contiguous ranges, 16 of 1024 x 4096 43 against 45, 32 of 2048 x
// 768 35.5-38.4 against 39.6-41.2. Each XCD a run of row tiles of each item
// (all its bands, so the items of 8 bands write whole row-scale halves from
// one XCD) took 215-218 us for those items and 224-226 us for all items,
// against 206-211 us. The four-tile kernel in this per-item band-group order
// (quant_dual_grouped_super_kernel) made the cfg5 layer step 3.5 us slower.
__global__ __launch_bounds__(kDualThreads) void quant_dual_grouped_kernel(const DualGroup g) {
  __shared__ __attribute__((aligned(16))) uint8_t tile[kDualRows * kDualPitch];
  __shared__ __attribute__((aligned(8))) uint8_t rs_tile[kDualRows * 8];
  const int b = blockIdx.x, xcd = b % kXcds;
  int j = b / kXcds, i = 0;
  for (; i < g.count; i++) {
    const int n = min(max(g.item[i].tiles - xcd * g.item[i].per_xcd, 0), g.item[i].per_xcd);
    if (j < n) break;
    j -= n;
  }
  if (i == g.count) return;
  const DualItem& it = g.item[i];
  int ms, kb;
  if (!band_group_tile(xcd, j, it.tiles_m, it.tiles, it.per_xcd, &ms, &kb)) return;
  dual_tile(it.x, it.row_q, it.row_s, it.col_q, it.col_s, it.M, it.K, it.tiles_m, kb * it.tiles_m + ms, g.eps, g.c_eps,
            tile, rs_tile);
}

// Grouped form of quant_dual_super_kernel: every item has M % 64 == 0,
// K % 256 == 0 and aligned buffers; tiles_m counts super-rows.
__global__ __launch_bounds__(kDualThreads) __attribute__((amdgpu_waves_per_eu(6))) void quant_dual_grouped_super_kernel(
    const DualGroup g) {
  __shared__ DualSuperSmem sm;
  const int b = blockIdx.x, xcd = b % kXcds;
  // the XCD's share of each item, item after item
  int j = b / kXcds, i = 0;
  for (; i < g.count; i++) {
    const int n = min(max(g.item[i].tiles - xcd * g.item[i].per_xcd, 0), g.item[i].per_xcd);
    if (j < n) break;
    j -= n;
  }
  if (i == g.count) return;
  const DualItem& it = g.item[i];
  int ms, kb;
  if (!band_group_tile(xcd, j, it.tiles_m, it.tiles, it.per_xcd, &ms, &kb)) return;
  dual_super4(it.x, it.row_q, it.row_s, it.col_q, it.col_s, it.M, it.K, ms, kb, g.eps, g.c_eps, sm);
}

// Shapes and buffers the four-tile kernels take: whole 64 x 256 tiles, 16 B
// aligned input, rowwise codes and transposed codes.
static bool dual_super_ok(const void* x, const void* row_q, const void* col_q, int64_t M, int64_t K) {
  return M % kDualRows == 0 && K % kDualCols == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
         (reinterpret_cast<uintptr_t>(row_q) & 15) == 0 && (reinterpret_cast<uintptr_t>(col_q) & 15) == 0;
}

hipError_t launch_quant_dual(const void* x, void* row_q, void* row_s, void* col_q, void* col_s, int64_t M, int64_t K,
                             float eps, hipStream_t stream) {
  if (M == 0 || K == 0) return hipSuccess;
  const int64_t tiles_m = (M + kDualRows - 1) / kDualRows;
  const int64_t tiles_k = (K + kDualCols - 1) / kDualCols;
  const int64_t tiles = tiles_m * tiles_k;
  const int64_t sm = (M + kSuperRows - 1) / kSuperRows, st = sm * tiles_k;
  // The four-tile kernel needs its super-tiles to fill the CUs several times
  // over; below four per CU the one-tile kernel's four times as many
  // workgroups finish sooner (7168 x 2048: 11.8 us against 16.1; 8192 x 7168:
  // 39.9 against 41.4; 16384 x 7168, 1792 super-tiles: 70.8 against 69.0).
  if (dual_super_ok(x, row_q, col_q, M, K) && st >= 4 * (int64_t)current_device_caps().cus) {
    const int64_t spx = (st + kXcds - 1) / kXcds;
    return launch(quant_dual_super_kernel, dim3((unsigned)(spx * kXcds)), dim3(kDualThreads), 0, stream,
                       static_cast<const uint16_t*>(x), static_cast<uint32_t*>(row_q), static_cast<uint8_t*>(row_s),
                       static_cast<uint8_t*>(col_q), static_cast<uint8_t*>(col_s), M, K, (int)sm, (int)st, (int)spx,
                       eps, host_c_eps(eps, 6.0f));
  }
  const int64_t per_xcd = (tiles + kXcds - 1) / kXcds;
  const bool band_group = tiles >= 6 * (int64_t)current_device_caps().cus;
  return launch(quant_dual_kernel, dim3((unsigned)(per_xcd * kXcds)), dim3(kDualThreads), 0, stream,
                     static_cast<const uint16_t*>(x), static_cast<uint32_t*>(row_q), static_cast<uint8_t*>(row_s),
                     static_cast<uint8_t*>(col_q), static_cast<uint8_t*>(col_s), M, K, (int)tiles_m, (int)tiles,
                     (int)per_xcd, band_group, eps, host_c_eps(eps, 6.0f));
}

hipError_t launch_quant_dual_grouped(const DualSpec* items, int count, float eps, hipStream_t stream) {
  for (int base = 0; base < count; base += kDualGroupMax) {
    DualGroup g;
    memset(&g, 0, sizeof(g));
    g.count = count - base < kDualGroupMax ? count - base : kDualGroupMax;
    // the four-tile kernel where every item would take it alone
    bool super = true;
    for (int j = 0; j < g.count; j++) {
      const DualSpec& d = items[base + j];
      const int64_t st = ((d.M + kSuperRows - 1) / kSuperRows) * ((d.K + kDualCols - 1) / kDualCols);
      super = super && (d.M == 0 || d.K == 0 ||
                        (dual_super_ok(d.x, d.row_q, d.col_q, d.M, d.K) && st >= 4 * (int64_t)current_device_caps().cus));
    }
    const int unit_rows = super ? kSuperRows : kDualRows;
    int tiles = 0, super_slots = 0;
    for (int j = 0; j < g.count; j++) {
      const DualSpec& d = items[base + j];
      DualItem& it = g.item[j];
      it.x = static_cast<const uint16_t*>(d.x);
      it.row_q = static_cast<uint32_t*>(d.row_q);
      it.row_s = static_cast<uint8_t*>(d.row_s);
      it.col_q = static_cast<uint8_t*>(d.col_q);
      it.col_s = static_cast<uint8_t*>(d.col_s);
      it.M = d.M;
      it.K = d.K;
      it.tiles_m = (int)((d.M + unit_rows - 1) / unit_rows);
      it.tiles = (d.M == 0 || d.K == 0) ? 0 : it.tiles_m * (int)((d.K + kDualCols - 1) / kDualCols);
      it.per_xcd = (it.tiles + kXcds - 1) / kXcds;
      tiles += it.tiles;
      super_slots += it.per_xcd;  // XCD 0 has the largest share of every item: the grid's slots per XCD
    }
    if (tiles == 0) continue;
    g.tiles = tiles;
    g.per_xcd = super_slots;
    g.eps = eps;
    g.c_eps = host_c_eps(eps, 6.0f);
    auto kernel = super ? quant_dual_grouped_super_kernel : quant_dual_grouped_kernel;
    const hipError_t e = launch(kernel, dim3((unsigned)(g.per_xcd * kXcds)), dim3(kDualThreads), 0, stream, g);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace omo_hip
