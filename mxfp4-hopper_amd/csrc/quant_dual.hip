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
// Tiles are 64 rows x 256 columns (32 KiB of bf16). Each lane loads 8 chunks
// of 16 B (two rows of 512 B per wave and load); the rowwise blocks are
// quantized from registers exactly as in the rowwise kernel (a block is a
// DPP quad) and their codes leave as full 128 B lines (non-temporal
// stores). The tile is staged in LDS; each lane then reads one dword (two
// adjacent columns) from 32 consecutive rows, repacks the two columns into
// bf16 pairs with v_perm_b32 and quantizes both 32-element column blocks
// (16 B of codes each).
//
// Tile order is XCD-aware: workgroup b runs on XCD b % 8, so the tiles are
// numbered so that each XCD takes a contiguous run of tiles that walks down
// M first. The four vertically adjacent tiles that fill one 128 B line of
// columnwise codes then run at the same time behind the same L2.
#include "omo_internal.h"
#include "omo_quant.cuh"

namespace omo_hip {

constexpr int kDualRows = 64;
constexpr int kDualCols = 256;
constexpr int kDualPitch = kDualCols * 2 + 16;  // bytes per LDS row
constexpr int kXcds = 8;
constexpr int kDualGroupMax = 32;

// One 64 x 256 tile (index `logical`, M-fastest) of the [M, K] tensor x.
__device__ __forceinline__ void dual_tile(const uint16_t* __restrict__ x, uint32_t* __restrict__ row_q,
                                          uint8_t* __restrict__ row_s, uint8_t* __restrict__ col_q,
                                          uint8_t* __restrict__ col_s, int64_t M, int64_t K, int tiles_m,
                                          int logical, float eps, int c_eps, uint8_t* tile) {
  const int t = threadIdx.x;
  const int64_t mt = logical % tiles_m, kt = logical / tiles_m;
  const int64_t m0 = mt * kDualRows, k0 = kt * kDualCols;
  const int rows_valid = (int)(M - m0 < kDualRows ? M - m0 : kDualRows);  // 32 or 64
  // ---- load: 64 rows x 32 chunks of 8 bf16; lane owns chunks t + 256 k.
  // Chunks outside the tensor load from a clamped in-bounds address (and are
  // ignored below), so every load is unconditional.
  u32x4 d[8];
#pragma unroll
  for (int k = 0; k < 8; k++) {
    const int cid = t + 256 * k, r = cid >> 5, cc = cid & 31;
    const int64_t col = k0 + cc * 8;
    const int rr = r < rows_valid ? r : rows_valid - 1;
    const int64_t cl = col < K ? col : K - 8;
    d[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(x + (m0 + rr) * K + cl));
  }
  // ---- rowwise blocks from registers; stage the tile in LDS
  // Lane t holds rows r0 + 8k (k = 0..7) of one 16 B column chunk cc, so its
  // code, scale and LDS addresses advance by a fixed stride per k.
  const bool quad_leader = (t & 3) == 0;
  const int r0 = t >> 5, cc = t & 31;
  const int64_t col = k0 + cc * 8;
  uint32_t* rq = row_q + (m0 + r0) * (K / 8) + col / 8;
  uint8_t* rs = row_s + (m0 + r0) * (K / 32) + col / 32;
  uint8_t* lt = tile + r0 * kDualPitch + cc * 16;
#pragma unroll
  for (int k = 0; k < 8; k++) {
    // K % 32 == 0 and rows_valid is uniform per row: a quad is entirely in or out
    if (r0 + 8 * k >= rows_valid || col >= K) continue;
    *reinterpret_cast<u32x4*>(lt + 8 * k * kDualPitch) = d[k];
    uint32_t codes, byte;
    const uint32_t am = quad_max_u32(chunk_absmax_bits(d[k]));
    if (am < 0x7F80u) {
      codes = quant_chunk_fast(d[k], am, eps, c_eps, &byte);
    } else {
      quant_chunk_ref(d[k], eps, -6.0f, 6.0f, &codes, &byte);
    }
    __builtin_nontemporal_store(codes, rq + k * K);  // 8 rows down; streamed out
    if (quad_leader) rs[k * (K / 4)] = (uint8_t)byte;
  }
  __syncthreads();
  // ---- columnwise: lane owns columns 2p, 2p+1 of row block g (32 rows)
  const int p = t & 127, g = t >> 7;
  const int64_t kc = k0 + 2 * p;
  if (32 * g >= rows_valid || kc >= K) return;
  uint32_t ca[16], cb[16];
  uint32_t amax_a = 0, amax_b = 0;
#pragma unroll
  for (int j = 0; j < 16; j++) {
    const uint32_t w0 = *reinterpret_cast<const uint32_t*>(tile + (32 * g + 2 * j) * kDualPitch + 4 * p);
    const uint32_t w1 = *reinterpret_cast<const uint32_t*>(tile + (32 * g + 2 * j + 1) * kDualPitch + 4 * p);
    ca[j] = __builtin_amdgcn_perm(w1, w0, 0x05040100u);  // column 2p: rows 2j (low), 2j+1 (high)
    cb[j] = __builtin_amdgcn_perm(w1, w0, 0x07060302u);  // column 2p+1
    amax_a = pk_max_u16(amax_a, ca[j] & 0x7FFF7FFFu);
    amax_b = pk_max_u16(amax_b, cb[j] & 0x7FFF7FFFu);
  }
  amax_a = max(amax_a & 0xFFFFu, amax_a >> 16);
  amax_b = max(amax_b & 0xFFFFu, amax_b >> 16);
  uint32_t byte_a, byte_b;
  u32x4 qa, qb;
  if (amax_a < 0x7F80u) qa = quant_block32_fast(ca, amax_a, eps, c_eps, &byte_a);
  else qa = quant_block32_ref(ca, eps, -6.0f, 6.0f, &byte_a);
  if (amax_b < 0x7F80u) qb = quant_block32_fast(cb, amax_b, eps, c_eps, &byte_b);
  else qb = quant_block32_ref(cb, eps, -6.0f, 6.0f, &byte_b);
  const int64_t mo = (m0 + 32 * g) / 2;
  *reinterpret_cast<u32x4*>(col_q + kc * (M / 2) + mo) = qa;
  *reinterpret_cast<u32x4*>(col_q + (kc + 1) * (M / 2) + mo) = qb;
  const int64_t so = (m0 + 32 * g) / 32;
  col_s[kc * (M / 32) + so] = (uint8_t)byte_a;
  col_s[(kc + 1) * (M / 32) + so] = (uint8_t)byte_b;
}

__global__ __launch_bounds__(256) void quant_dual_kernel(const uint16_t* __restrict__ x, uint32_t* __restrict__ row_q,
                                                         uint8_t* __restrict__ row_s, uint8_t* __restrict__ col_q,
                                                         uint8_t* __restrict__ col_s, int64_t M, int64_t K,
                                                         int tiles_m, int tiles, int per_xcd, float eps, int c_eps) {
  __shared__ __attribute__((aligned(16))) uint8_t tile[kDualRows * kDualPitch];
  const int b = blockIdx.x;
  const int logical = (b % kXcds) * per_xcd + b / kXcds;
  if (logical >= tiles) return;
  dual_tile(x, row_q, row_s, col_q, col_s, M, K, tiles_m, logical, eps, c_eps, tile);
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

__global__ __launch_bounds__(256) void quant_dual_grouped_kernel(const DualGroup g) {
  __shared__ __attribute__((aligned(16))) uint8_t tile[kDualRows * kDualPitch];
  const int b = blockIdx.x;
  const int logical = (b % kXcds) * g.per_xcd + b / kXcds;
  if (logical >= g.tiles) return;
  int i = 0;
  while (i + 1 < g.count && logical >= g.item[i + 1].tile_begin) i++;
  const DualItem& it = g.item[i];
  dual_tile(it.x, it.row_q, it.row_s, it.col_q, it.col_s, it.M, it.K, it.tiles_m, logical - it.tile_begin, g.eps,
            g.c_eps, tile);
}

hipError_t launch_quant_dual(const void* x, void* row_q, void* row_s, void* col_q, void* col_s, int64_t M, int64_t K,
                             float eps, hipStream_t stream) {
  if (M == 0 || K == 0) return hipSuccess;
  const int64_t tiles_m = (M + kDualRows - 1) / kDualRows;
  const int64_t tiles_k = (K + kDualCols - 1) / kDualCols;
  const int64_t tiles = tiles_m * tiles_k;
  const int64_t per_xcd = (tiles + kXcds - 1) / kXcds;
  hipLaunchKernelGGL(quant_dual_kernel, dim3((unsigned)(per_xcd * kXcds)), dim3(256), 0, stream,
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
    hipLaunchKernelGGL(quant_dual_grouped_kernel, dim3((unsigned)(g.per_xcd * kXcds)), dim3(256), 0, stream, g);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace omo_hip
