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
__device__ __forceinline__ uint2 quant_half16_fast(const uint32_t (&p)[8], uint32_t amax_bits, float eps, int c_eps,
                                                   uint32_t* byte) {
  const float xmax = bf16_to_f32(amax_bits);
  int c = (int)(amax_bits >> 7) - 129 + ((amax_bits & 0x7Fu) > 64u ? 1 : 0);
  c = c < -33 ? -33 : c;
  c = (xmax > eps) ? c : c_eps;
  *byte = (uint32_t)(c + 127);
  const float y_s = exp2i(c);
  uint2 out;
  uint32_t r = 0;
  r = cvt_pk_fp4<0>(r, p[0], y_s);
  r = cvt_pk_fp4<1>(r, p[1], y_s);
  r = cvt_pk_fp4<2>(r, p[2], y_s);
  r = cvt_pk_fp4<3>(r, p[3], y_s);
  out.x = r;
  r = 0;
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
#pragma unroll
  for (int k = 0; k < 4; k++) {
    // row r0 + 16k is in 16-row band k: its chunks are stored XORed by 4k,
    // so the four bands sit in four different 64 B bank ranges
    *reinterpret_cast<u32x4*>(tile + (r0 + 16 * k) * kDualPitch + ((cc ^ (k << 2)) * 16)) = d[k];
    uint32_t codes, byte;
    const uint32_t am = quad_max_u32(chunk_absmax_bits(d[k]));
    if (__builtin_expect(am < 0x7F80u, 1)) {
      codes = quant_chunk_fast(d[k], am, eps, c_eps, &byte);
    } else {
      quant_chunk_ref(d[k], eps, -6.0f, 6.0f, &codes, &byte);
    }
    if (r0 + 16 * k < rows_valid && col < K) __builtin_nontemporal_store(codes, rq + k * 2 * K);  // 16 rows down
    // the 8 scale bytes of a tile row are gathered in LDS and leave as one store
    if (quad_leader) rs_tile[(r0 + 16 * k) * 8 + (cc >> 2)] = (uint8_t)byte;
  }
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
  if (__builtin_expect(amax_a < 0x7F80u, 1)) qa = quant_half16_fast(ca, amax_a, eps, c_eps, &byte_a);
  else qa = quant_half16_ref(ca, eps, &byte_a);
  if (__builtin_expect(amax_b < 0x7F80u, 1)) qb = quant_half16_fast(cb, amax_b, eps, c_eps, &byte_b);
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

__global__ __launch_bounds__(kDualThreads) void quant_dual_kernel(const uint16_t* __restrict__ x, uint32_t* __restrict__ row_q,
                                                         uint8_t* __restrict__ row_s, uint8_t* __restrict__ col_q,
                                                         uint8_t* __restrict__ col_s, int64_t M, int64_t K,
                                                         int tiles_m, int tiles, int per_xcd, float eps, int c_eps) {
  __shared__ __attribute__((aligned(16))) uint8_t tile[kDualRows * kDualPitch];
  __shared__ __attribute__((aligned(8))) uint8_t rs_tile[kDualRows * 8];
  const int b = blockIdx.x;
  const int logical = (b % kXcds) * per_xcd + b / kXcds;
  if (logical >= tiles) return;
  dual_tile(x, row_q, row_s, col_q, col_s, M, K, tiles_m, logical, eps, c_eps, tile, rs_tile);
}

// Grouped form: one launch over up to kDualGroupMax tensors (e.g. the weights
// of all local experts), whose tiles are numbered item after item and then
// spread over the XCDs like the tiles of one tensor. The descriptor table
// travels by value in the kernel arguments.
struct DualItem {
  const uint16_t* x;
  uint32_t* row_q;
  uint8_t* row_s;
  uint8_t* col_q;
  uint8_t* col_s;
  int64_t M, K;
  int tiles_m, tile_begin;  // first logical tile of this item
};

struct DualGroup {
  DualItem item[kDualGroupMax];
  int count, tiles, per_xcd, c_eps;
  float eps;
};

__global__ __launch_bounds__(kDualThreads) void quant_dual_grouped_kernel(const DualGroup g) {
  __shared__ __attribute__((aligned(16))) uint8_t tile[kDualRows * kDualPitch];
  __shared__ __attribute__((aligned(8))) uint8_t rs_tile[kDualRows * 8];
  const int b = blockIdx.x;
  const int logical = (b % kXcds) * g.per_xcd + b / kXcds;
  if (logical >= g.tiles) return;
  int i = 0;
  while (i + 1 < g.count && logical >= g.item[i + 1].tile_begin) i++;
  const DualItem& it = g.item[i];
  dual_tile(it.x, it.row_q, it.row_s, it.col_q, it.col_s, it.M, it.K, it.tiles_m, logical - it.tile_begin, g.eps,
            g.c_eps, tile, rs_tile);
}

hipError_t launch_quant_dual(const void* x, void* row_q, void* row_s, void* col_q, void* col_s, int64_t M, int64_t K,
                             float eps, hipStream_t stream) {
  if (M == 0 || K == 0) return hipSuccess;
  const int64_t tiles_m = (M + kDualRows - 1) / kDualRows;
  const int64_t tiles_k = (K + kDualCols - 1) / kDualCols;
  const int64_t tiles = tiles_m * tiles_k;
  const int64_t per_xcd = (tiles + kXcds - 1) / kXcds;
  hipLaunchKernelGGL(quant_dual_kernel, dim3((unsigned)(per_xcd * kXcds)), dim3(kDualThreads), 0, stream,
                     static_cast<const uint16_t*>(x), static_cast<uint32_t*>(row_q), static_cast<uint8_t*>(row_s),
                     static_cast<uint8_t*>(col_q), static_cast<uint8_t*>(col_s), M, K, (int)tiles_m, (int)tiles,
                     (int)per_xcd, eps, host_c_eps(eps, 6.0f));
  return hipGetLastError();
}

hipError_t launch_quant_dual_grouped(const DualSpec* items, int count, float eps, hipStream_t stream) {
  for (int base = 0; base < count; base += kDualGroupMax) {
    DualGroup g;
    memset(&g, 0, sizeof(g));
    g.count = count - base < kDualGroupMax ? count - base : kDualGroupMax;
    int tiles = 0;
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
      it.tiles_m = (int)((d.M + kDualRows - 1) / kDualRows);
      it.tile_begin = tiles;
      tiles += (d.M == 0 || d.K == 0) ? 0 : it.tiles_m * (int)((d.K + kDualCols - 1) / kDualCols);
    }
    if (tiles == 0) continue;
    g.tiles = tiles;
    g.per_xcd = (tiles + kXcds - 1) / kXcds;
    g.eps = eps;
    g.c_eps = host_c_eps(eps, 6.0f);
    hipLaunchKernelGGL(quant_dual_grouped_kernel, dim3((unsigned)(g.per_xcd * kXcds)), dim3(kDualThreads), 0, stream, g);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace omo_hip
