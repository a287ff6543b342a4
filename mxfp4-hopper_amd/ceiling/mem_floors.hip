// Memory-only copies of the codec kernels whose time is set by their loads
// and stores. Each kernel issues the global loads and stores of the product
// kernel it is named after - the same addresses, widths, cache policies,
// workgroup shape, workgroup order and LDS footprint (so the same residency)
// - with the arithmetic replaced by XORs of the loaded data. The time of one
// of these is the floor of its product kernel's access pattern on this HBM.
// Built into libomo_ceiling.so for bench.py's floors leg; nothing in the
// product calls them.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <stdint.h>
#include <string.h>

typedef uint32_t fu32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t fu32x2 __attribute__((ext_vector_type(2)));

namespace {

// The product's XCD-contiguous workgroup order (csrc/omo_device.cuh).
__device__ __forceinline__ uint32_t xcd_order(uint32_t b, uint32_t n) {
  const uint32_t x = b & 7u, j = b >> 3, q = n >> 3, r = n & 7u;
  return x * q + (x < r ? x : r) + j;
}

// ---- dual-layout quantize, four 64 x 256 tiles per workgroup (quant_dual_super_kernel)
struct DualFloorSmem {
  __attribute__((aligned(16))) uint8_t tile[64 * 512];
  __attribute__((aligned(16))) uint32_t row_codes[2][64 * 32];
  __attribute__((aligned(8))) uint8_t row_scales[2][64 * 8];
};

__device__ __forceinline__ void dual_floor_flush(const DualFloorSmem& sm, int buf, uint32_t* __restrict__ row_q,
                                                 uint8_t* __restrict__ row_s, int64_t m0, int64_t k0, int64_t K) {
  const int t = threadIdx.x, row = t >> 3, piece = t & 7;
  const fu32x4 c = *reinterpret_cast<const fu32x4*>(&sm.row_codes[buf][row * 32 + 4 * piece]);
  __builtin_nontemporal_store(c, reinterpret_cast<fu32x4*>(row_q + (m0 + row) * (K / 8) + k0 / 8 + 4 * piece));
  if (row_s != nullptr && t < 64) {
    *reinterpret_cast<fu32x2*>(row_s + (m0 + t) * (K / 32) + k0 / 32) =
        *reinterpret_cast<const fu32x2*>(&sm.row_scales[buf][t * 8]);
  }
}

// The product's band-group order (quant_dual_super_kernel): super-tiles
// numbered M-fastest (L = band * S + super-row) are cut into eight
// contiguous ranges of per_xcd, one per XCD, and each XCD walks its range
// super-row by super-row. False past the XCD's range.
__device__ __forceinline__ bool floor_band_group(int xcd, int j, int S, int T, int per_xcd, int* ms, int* kb) {
  const int lo = xcd * per_xcd, hi = min(T, lo + per_xcd);
  if (j >= hi - lo) return false;
  const int kb0 = lo / S, ms0 = lo - kb0 * S, kb1 = hi / S, ms1 = hi - kb1 * S;
  auto below = [&](int m) {  // tiles of the range in super-rows below m
    if (kb0 == kb1) return max(0, min(m, ms1) - ms0);
    return m * (kb1 - kb0 - 1) + max(0, m - ms0) + min(m, ms1);
  };
  int a = 0, b = S;
  while (b - a > 1) {
    const int mid = (a + b) >> 1;
    if (below(mid) <= j) a = mid;
    else b = mid;
  }
  *ms = a;
  *kb = kb0 + (a >= ms0 ? 0 : 1) + (j - below(a));
  return true;
}

// Aligned groups (bands % 8 == 0): bands in groups of 8, i.e. one 64 B half of
// every row-scale line, so no half is written by two XCDs. With G = bands / 8
// groups, XCD x takes the whole groups x, x + 8, ... (the first 8 (G / 8)),
// walked super-row by super-row, then its eighth of the last G % 8 groups,
// numbered super-row by super-row. False past the XCD's share.
__device__ __forceinline__ bool floor_aligned_groups(int xcd, int j, int S, int bands, int* ms, int* kb) {
  const int G = bands / 8, q = G / 8, r = G % 8;
  if (j < 8 * q * S) {
    const int w = j % (8 * q);
    *ms = j / (8 * q);
    *kb = 8 * (xcd + 8 * (w / 8)) + w % 8;
    return true;
  }
  if (j >= 8 * q * S + r * S) return false;
  const int i = xcd * r * S + (j - 8 * q * S);
  *ms = i / (8 * r);
  *kb = 64 * q + i % (8 * r);
  return true;
}

// M % 256 == 0, K % 256 == 0, 16 B aligned buffers (the shapes the bench uses).
// SCM 0: the product's scale stores (8 B per row per tile, 8 B per column per
// super-tile, ordinary stores); SCM 1: no scale stores (the bound the code
// traffic alone sets); SCM 2: the same scale bytes written as whole lines,
// each workgroup's 2 KB of row scales and 2 KB of column scales contiguous at
// its tile number * 2048 with non-temporal 16 B stores - not the output
// layout, the bound a layout-free scale store would set. ORDER 0: the
// product's band-group order; 1: contiguous ranges of the M-fastest
// numbering per XCD (each XCD finishing one band before the next); 2:
// contiguous ranges of the K-fastest numbering; 3: aligned groups
// (floor_aligned_groups).
template <int SCM, int ORDER>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(6))) void dual_floor(
    const uint16_t* __restrict__ x, uint32_t* __restrict__ row_q, uint8_t* __restrict__ row_s,
    uint8_t* __restrict__ col_q, uint8_t* __restrict__ col_s, int64_t M, int64_t K, int tiles_ms, int tiles,
    int per_xcd) {
  __shared__ DualFloorSmem sm;
  const int b = blockIdx.x;
  const int t = threadIdx.x, r0 = t >> 5, cc = t & 31;
  const int tiles_k = (int)(K / 256);
  int ms, kb, logical;
  if (ORDER == 0) {
    if (!floor_band_group(b % 8, b / 8, tiles_ms, tiles, per_xcd, &ms, &kb)) return;
    logical = kb * tiles_ms + ms;
  } else if (ORDER == 3) {
    if (!floor_aligned_groups(b % 8, b / 8, tiles_ms, tiles_k, &ms, &kb)) return;
    logical = kb * tiles_ms + ms;
  } else {
    logical = (b % 8) * per_xcd + b / 8;
    if (logical >= tiles) return;
    ms = ORDER == 2 ? logical / tiles_k : logical % tiles_ms;
    kb = ORDER == 2 ? logical % tiles_k : logical / tiles_ms;
  }
  const int64_t m0s = (int64_t)ms * 256, k0 = (int64_t)kb * 256;
  uint32_t acc = 0;
  for (int st = 0; st < 4; st++) {
    const int64_t m0 = m0s + 64 * st;
    const int buf = st & 1;
    const uint16_t* src = x + (m0 + r0) * K + k0 + cc * 8;
    fu32x4 d[4];
#pragma unroll
    for (int k = 0; k < 4; k++) d[k] = __builtin_nontemporal_load(reinterpret_cast<const fu32x4*>(src + 16 * k * K));
#pragma unroll
    for (int k = 0; k < 4; k++) {
      *reinterpret_cast<fu32x4*>(sm.tile + (r0 + 16 * k) * 512 + ((cc ^ (k << 2)) * 16)) = d[k];
      sm.row_codes[buf][(r0 + 16 * k) * 32 + cc] = d[k].x ^ d[k].y;
      if ((t & 3) == 0) sm.row_scales[buf][(r0 + 16 * k) * 8 + (cc >> 2)] = (uint8_t)d[k].z;
    }
    if (st > 0) dual_floor_flush(sm, buf ^ 1, row_q, SCM == 0 ? row_s : nullptr, m0 - 64, k0, K);
    __syncthreads();
    acc ^= *reinterpret_cast<const uint32_t*>(sm.tile + ((t * 68) & 32764));
    __syncthreads();
  }
  dual_floor_flush(sm, 1, row_q, SCM == 0 ? row_s : nullptr, m0s + 192, k0, K);
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int c = (t >> 3) + 64 * j, piece = t & 7;
    fu32x4 v = *reinterpret_cast<const fu32x4*>(sm.tile + c * 128 + 16 * piece);
    v.x ^= acc;
    *reinterpret_cast<fu32x4*>(col_q + (k0 + c) * (M / 2) + m0s / 2 + 16 * piece) = v;
  }
  if (SCM == 0 && (t & 1) == 0) {
    const int c = 2 * (t >> 2) + ((t >> 1) & 1);
    *reinterpret_cast<fu32x2*>(col_s + (k0 + c) * (M / 32) + m0s / 32) = fu32x2{acc, (uint32_t)c};
  }
  if (SCM == 2 && t < 128) {
    const fu32x4 w = {acc, (uint32_t)t, (uint32_t)logical, 1u};
    __builtin_nontemporal_store(w, reinterpret_cast<fu32x4*>(row_s + (int64_t)logical * 2048 + 16 * t));
    __builtin_nontemporal_store(w, reinterpret_cast<fu32x4*>(col_s + (int64_t)logical * 2048 + 16 * t));
  }
  if (SCM == 1 && acc == 0x9E3779B9u) row_s[t] = 1;  // keeps the LDS reads
}

// ---- grouped dual-layout quantize, one 64 x 256 tile per workgroup (quant_dual_grouped_kernel)
constexpr int kFloorGroupMax = 32;

// Forms every value of v here, in code every lane runs, so that the waits
// for their loads come before the stores that follow (a value formed inside
// a store's bounds test left the compiler a wait at the test's join that
// covered the earlier stores too), as the product kernels' conversions do.
template <int N>
__device__ __forceinline__ void floor_materialize(fu32x4 (&v)[N]) {
#pragma unroll
  for (int u = 0; u < N; u++) asm volatile("" : "+v"(v[u]));
}

struct FloorItem {
  const uint16_t* x;
  uint32_t* row_q;
  uint8_t* row_s;
  uint8_t* col_q;
  uint8_t* col_s;
  int64_t M, K;
  int tiles_m, tiles, per_xcd;
};

struct FloorGroup {
  FloorItem item[kFloorGroupMax];
  int count;
};

// One tile's loads and stores as the product's one-tile kernel issues them
// (M % 64 == 0, K % 256 == 0): four 16 B non-temporal loads per lane, then
// four 4 B non-temporal row-code stores, 64 rows' 8 scale bytes gathered in
// LDS and stored after the barrier, then per column pair two 8 B code stores
// and a 2-byte scale store (SCM 1: no scale stores).
template <int SCM>
__device__ __forceinline__ void dual_tile_floor(const FloorItem& it, int64_t m0, int64_t k0, uint8_t* tile,
                                                uint8_t* rs_tile) {
  const int64_t M = it.M, K = it.K;
  const int t = threadIdx.x, r0 = t >> 5, cc = t & 31;
  const int64_t col = k0 + cc * 8;
  fu32x4 d[4];
#pragma unroll
  for (int k = 0; k < 4; k++)
    d[k] = __builtin_nontemporal_load(reinterpret_cast<const fu32x4*>(it.x + (m0 + r0 + 16 * k) * K + col));
  uint32_t* rq = it.row_q + (m0 + r0) * (K / 8) + col / 8;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    *reinterpret_cast<fu32x4*>(tile + (r0 + 16 * k) * 512 + ((cc ^ (k << 2)) * 16)) = d[k];
    if ((t & 3) == 0) rs_tile[(r0 + 16 * k) * 8 + (cc >> 2)] = (uint8_t)d[k].z;
  }
  floor_materialize(d);
#pragma unroll
  for (int k = 0; k < 4; k++) __builtin_nontemporal_store(d[k].x ^ d[k].y, rq + k * 2 * K);
  __syncthreads();
  if (SCM == 0 && t < 64)
    *reinterpret_cast<fu32x2*>(it.row_s + (m0 + t) * (K / 32) + k0 / 32) = *reinterpret_cast<const fu32x2*>(rs_tile + t * 8);
  const int h = t & 1, g = (t >> 1) & 1, p = t >> 2, band = 2 * g + h;
  const int64_t kc = k0 + 2 * p;
  const int pp = 4 * (p ^ (band << 4));
  uint32_t a0 = 0, a1 = 0;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const uint32_t w0 = *reinterpret_cast<const uint32_t*>(tile + (16 * band + 2 * j) * 512 + pp);
    const uint32_t w1 = *reinterpret_cast<const uint32_t*>(tile + (16 * band + 2 * j + 1) * 512 + pp);
    if (j < 4) a0 ^= w0 ^ (w1 << 1);
    else a1 ^= w0 ^ (w1 << 1);
  }
  const int64_t mo = (m0 + 16 * band) / 2;
  *reinterpret_cast<fu32x2*>(it.col_q + kc * (M / 2) + mo) = fu32x2{a0, a1};
  *reinterpret_cast<fu32x2*>(it.col_q + (kc + 1) * (M / 2) + mo) = fu32x2{a1, a0};
  if (SCM == 0 && h == 0) *reinterpret_cast<uint16_t*>(it.col_s + (kc + g) * (M / 32) + m0 / 32) = (uint16_t)(a0 ^ a1);
  if (SCM == 1 && a0 == 0x9E3779B9u) it.row_s[t] = 1;  // keeps the LDS reads
}

// The product's grouped order: each XCD takes its band-group share of each
// item, item after item.
template <int SCM>
__global__ __launch_bounds__(512) void dual_grouped_floor(const FloorGroup g) {
  __shared__ __attribute__((aligned(16))) uint8_t tile[64 * 512];
  __shared__ __attribute__((aligned(8))) uint8_t rs_tile[64 * 8];
  const int b = blockIdx.x, xcd = b % 8;
  int j = b / 8, i = 0;
  for (; i < g.count; i++) {
    const int n = min(max(g.item[i].tiles - xcd * g.item[i].per_xcd, 0), g.item[i].per_xcd);
    if (j < n) break;
    j -= n;
  }
  if (i == g.count) return;
  const FloorItem& it = g.item[i];
  int ms, kb;
  if (!floor_band_group(xcd, j, it.tiles_m, it.tiles, it.per_xcd, &ms, &kb)) return;
  dual_tile_floor<SCM>(it, (int64_t)ms * 64, (int64_t)kb * 256, tile, rs_tile);
}

// ---- row -> col FP8, 128 x 256 tiles (row_to_fp8_col_wide_kernel, row_to_fp8_col_msplit_wide_kernel)
constexpr int kWideSmemBytes = 128 * 160 + 8 * 128 * 4 + 8 * 128;  // the product's WideSmem

// A lane's 16 bytes of one column at dst, stopping at rows_valid: the
// product's store of a column piece (one 16 B store, or 8/4/2/1-byte pieces
// at the end of a split).
__device__ __forceinline__ void floor_piece(uint8_t* __restrict__ dst, const fu32x4& w, int r_base, int rows_valid) {
  if (r_base + 16 <= rows_valid) {
    memcpy(dst, &w, 16);
  } else if (r_base < rows_valid) {
    const int n = rows_valid - r_base;
    int pos = 0;
    if (n & 8) {
      const fu32x2 h = {w[0], w[1]};
      memcpy(dst, &h, 8);
      pos = 8;
    }
    if (n & 4) {
      const uint32_t v = w[2];
      memcpy(dst + pos, &v, 4);
      pos += 4;
    }
    if (n & 2) {
      const uint16_t v = (uint16_t)w[3];
      memcpy(dst + pos, &v, 2);
      pos += 2;
    }
    if (n & 1) dst[pos] = (uint8_t)(w[3] >> 16);
  }
}

// One tile: loads of code rows row0 .. row0 + rows_valid - 1 and their scale
// bytes (rows past rows_valid reload the last row, as the product does), the
// LDS staging, then eight 16 B column pieces and one scale-row float per lane.
template <bool RAGGED>
__device__ __forceinline__ void wide_floor_tile(uint8_t* sm, const uint8_t* __restrict__ q, const uint8_t* __restrict__ s,
                                                int64_t N, int64_t row0, int rows_valid, int64_t col0,
                                                float* __restrict__ out_s_row, uint8_t* __restrict__ obase,
                                                int64_t cstride, bool line_nt) {
  const int t = threadIdx.x;
  fu32x4 cv[4];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int id = t + 256 * k, r = id >> 3, c16 = id & 7;
    const int rr = RAGGED ? min(r, rows_valid - 1) : r;
    const fu32x4* src = reinterpret_cast<const fu32x4*>(q + (row0 + rr) * (N / 2) + col0 / 2 + c16 * 16);
    cv[k] = RAGGED ? __builtin_nontemporal_load(src) : *src;  // per split non-temporal, as the product
  }
  fu32x2 sv = {0x7F7F7F7Fu, 0x7F7F7F7Fu};
  if (t < 128) sv = *reinterpret_cast<const fu32x2*>(s + (row0 + (RAGGED ? min(t, rows_valid - 1) : t)) * (N / 32) + col0 / 32);
  if (RAGGED) {
#pragma unroll
    for (int k = 0; k < 4; k++)
      if (((t + 256 * k) >> 3) >= rows_valid) cv[k] = fu32x4{0u, 0u, 0u, 0u};
    if (t >= rows_valid) sv = fu32x2{0x7F7F7F7Fu, 0x7F7F7F7Fu};
  }
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int id = t + 256 * k;
    *reinterpret_cast<fu32x4*>(sm + (id >> 3) * 160 + (id & 7) * 16) = cv[k];
  }
  if (t < 128) *reinterpret_cast<fu32x2*>(sm + 128 * 160 + t * 8) = sv;
  __syncthreads();
  const int qq = t & 7, cg = t >> 3;
  fu32x4 w = *reinterpret_cast<const fu32x4*>(sm + (qq * 16 + cg) * 160 + 16 * (cg & 7));
  w.y ^= *reinterpret_cast<const uint32_t*>(sm + 128 * 160 + 8 * (t & 127));
  __builtin_nontemporal_store(__uint_as_float(w.x & 0x3FFFFFFFu), out_s_row + 8 * cg + qq);
  uint8_t* o = obase + 8 * cg * cstride + 16 * qq;
#pragma unroll
  for (int e = 0; e < 8; e++) {
    const fu32x4 we = w ^ fu32x4{(uint32_t)e, 0u, 0u, 0u};
    if (RAGGED && !line_nt) floor_piece(o + e * cstride, we, 16 * qq, rows_valid);
    else __builtin_nontemporal_store(we, reinterpret_cast<fu32x4*>(o + e * cstride));
  }
}

// Dense, M % 128 == 0, N % 256 == 0, 16 B aligned output.
__global__ __launch_bounds__(256, 4) void rowcol_floor(const uint8_t* __restrict__ q, const uint8_t* __restrict__ s,
                                                       uint8_t* __restrict__ out, float* __restrict__ out_s, int64_t M,
                                                       int64_t N) {
  __shared__ __attribute__((aligned(16))) uint8_t sm[kWideSmemBytes];
  const uint32_t L = xcd_order(blockIdx.x, gridDim.x), gx = (uint32_t)(N / 256);
  const int64_t bn = L % gx, bm = L / gx;
  wide_floor_tile<false>(sm, q, s, N, bm * 128, 128, bn * 256, out_s + bm * N + bn * 256, out + bn * 256 * M + bm * 128,
                         M, false);
}

// Per split, N % 256 == 0 (grid: split, row tile, column band).
__global__ __launch_bounds__(256, 4) void msplit_floor(const uint8_t* __restrict__ q, const uint8_t* __restrict__ s,
                                                       uint8_t* __restrict__ out, float* __restrict__ out_s,
                                                       const int32_t* __restrict__ lens, const int32_t* __restrict__ offs,
                                                       const int32_t* __restrict__ soffs, int64_t total_rows, int64_t N,
                                                       int64_t out_s_rows, bool out_line) {
  __shared__ __attribute__((aligned(16))) uint8_t sm[kWideSmemBytes];
  const int64_t split = blockIdx.x, bm = blockIdx.y, bn = blockIdx.z;
  const int64_t len = lens[split];
  if (bm * 128 >= len) return;
  const int64_t start = offs[split], sstart = soffs[split];
  if (start < 0 || start + len > total_rows || sstart < 0 || sstart + bm >= out_s_rows) return;
  const int rows_valid = (int)(len - bm * 128 < 128 ? len - bm * 128 : 128);
  wide_floor_tile<true>(sm, q, s, N, start + bm * 128, rows_valid, bn * 256, out_s + (sstart + bm) * N + bn * 256,
                        out + start * N + bn * 256 * len + bm * 128, len, out_line && len % 128 == 0);
}

// Per split on the product's flat grid (at most 64 splits): real tiles
// numbered split by split, band by band, row tile fastest, spread over the
// XCDs in contiguous ranges; workgroups past the last real tile exit.
__device__ __forceinline__ int wave_prefix(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);
  return v;
}

template <bool WALK>  // the product's band walk (rows of more than 16 bands), else its contiguous ranges
__global__ __launch_bounds__(256, 4) void msplit_flat_floor(const uint8_t* __restrict__ q, const uint8_t* __restrict__ s,
                                                            uint8_t* __restrict__ out, float* __restrict__ out_s,
                                                            const int32_t* __restrict__ lens,
                                                            const int32_t* __restrict__ offs,
                                                            const int32_t* __restrict__ soffs, int64_t total_rows,
                                                            int64_t N, int64_t out_s_rows, bool out_line, int nsplits,
                                                            int tm, int bands) {
  __shared__ __attribute__((aligned(16))) uint8_t sm[kWideSmemBytes];
  const int lane = (int)(threadIdx.x & 63);
  int len_l = 0, start_l = 0, sstart_l = 0;
  if (lane < nsplits) {
    len_l = lens[lane];
    start_l = offs[lane];
    sstart_l = soffs[lane];
  }
  // band walk: split after split, each XCD takes a contiguous range of
  // ceil(tiles_i / 8) of the split's band-major tiles and walks it row tile
  // by row tile. Ranges: the whole band-major numbering of all splits' tiles
  // in eight contiguous ranges, one per XCD.
  const int xcd = (int)(blockIdx.x & 7u);
  const int rows_l = len_l > 0 ? (int)min(((int64_t)len_l + 127) / 128, (int64_t)tm) : 0;
  const int per_l = (rows_l * bands + 7) / 8;
  const int n_l = WALK ? min(max(rows_l * bands - xcd * per_l, 0), per_l) : rows_l;
  const int incl = wave_prefix(n_l), excl = incl - n_l;
  int j;
  if (WALK) {
    j = (int)(blockIdx.x >> 3);
    if (j >= __builtin_amdgcn_readlane(incl, 63)) return;
  } else {
    const uint32_t n_real = (uint32_t)__builtin_amdgcn_readlane(incl, 63) * (uint32_t)bands;
    if (blockIdx.x >= n_real) return;
    j = (int)xcd_order(blockIdx.x, n_real);
  }
  const int unit = WALK ? 1 : bands;
  const uint64_t hit = __ballot(j >= unit * excl && j < unit * incl);
  const int i = (int)__builtin_ctzll(hit);
  const int S = __builtin_amdgcn_readlane(rows_l, i), per = __builtin_amdgcn_readlane(per_l, i);
  const int r = j - unit * __builtin_amdgcn_readlane(excl, i);
  int tbm, tbn;
  if (WALK) {
    if (!floor_band_group(xcd, r, S, S * bands, per, &tbm, &tbn)) return;
  } else {
    tbm = r % S;
    tbn = r / S;
  }
  const int64_t bm = tbm, bn = tbn;
  const int64_t len = __builtin_amdgcn_readlane(len_l, i), start = __builtin_amdgcn_readlane(start_l, i),
                sstart = __builtin_amdgcn_readlane(sstart_l, i);
  if (bm * 128 >= len) return;
  if (start < 0 || start + len > total_rows || sstart < 0 || sstart + bm >= out_s_rows) return;
  const int rows_valid = (int)(len - bm * 128 < 128 ? len - bm * 128 : 128);
  wide_floor_tile<true>(sm, q, s, N, start + bm * 128, rows_valid, bn * 256, out_s + (sstart + bm) * N + bn * 256,
                        out + start * N + bn * 256 * len + bm * 128, len, out_line && len % 128 == 0);
}

// ---- per-split row -> col FP8, band schedule (a schedule the product does not use)
// One workgroup per (split, 64-column band): it loads the band's 32 code
// bytes and 2 scale bytes of every row of the split into LDS (four 16 B
// loads in flight per lane), then writes the band's whole output region,
// the contiguous [64 columns x len] block at off * N + c0 * len, in address
// order as aligned non-temporal 16 B stores (each lane's chunk gathered from
// LDS as the conversion would: column o / len, row o % len), its two partial
// end chunks as bytes, and its scale-row entries. Splits of at most
// kBandMaxRows rows (the LDS holds the split's band).
constexpr int kBandMaxRows = 4352;

__global__ __launch_bounds__(256) void msplit_band_floor(const uint8_t* __restrict__ q, const uint8_t* __restrict__ s,
                                                         uint8_t* __restrict__ out, float* __restrict__ out_s,
                                                         const int32_t* __restrict__ lens,
                                                         const int32_t* __restrict__ offs,
                                                         const int32_t* __restrict__ soffs, int64_t N, int bands,
                                                         int total, int per_xcd) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int b = blockIdx.x;
  const int logical = (int)xcd_order((uint32_t)b, (uint32_t)(per_xcd * 8));
  if (logical >= total) return;
  const int i = logical / bands, band = logical % bands;
  const int len = lens[i];
  if (len <= 0) return;
  const int64_t row0 = offs[i], c0 = (int64_t)band * 64;
  const int t = threadIdx.x;
  const int nr = (len + 127) / 128;  // rounds of 128 rows (two 16 B chunks per row)
  for (int k0 = 0; k0 < nr; k0 += 4) {
    fu32x4 v[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int r = (k0 + u) * 128 + (t >> 1);
      const int rr = r < len ? r : len - 1;
      v[u] = *reinterpret_cast<const fu32x4*>(q + (row0 + rr) * (N / 2) + c0 / 2 + 16 * (t & 1));
    }
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int r = (k0 + u) * 128 + (t >> 1);
      if (k0 + u < nr && r < len) *reinterpret_cast<fu32x4*>(lds + r * 32 + 16 * (t & 1)) = v[u];
    }
  }
  uint8_t* lsc = lds + len * 32;
  for (int r = t; r < len; r += 256)
    *reinterpret_cast<uint16_t*>(lsc + 2 * r) = *reinterpret_cast<const uint16_t*>(s + (row0 + r) * (N / 32) + c0 / 32);
  __syncthreads();
  uint8_t* base = out + row0 * N + c0 * len;
  const int64_t size = 64LL * len;
  const uintptr_t a0 = reinterpret_cast<uintptr_t>(base), a1 = a0 + size;
  const uintptr_t f0 = (a0 + 15) & ~(uintptr_t)15, f1 = a1 & ~(uintptr_t)15;
  const int nch = f1 > f0 ? (int)((f1 - f0) / 16) : 0;
  const int ldsz = len * 32;
  int o = (int)(f0 - a0) + 16 * t;
  int c = o / len, r = o - c * len;
  for (int j = t; j < nch; j += 256) {
    const uint32_t idx = ((uint32_t)(r * 32 + (c >> 1)) & ~7u) % (uint32_t)(ldsz - 8);
    const fu32x2 w = *reinterpret_cast<const fu32x2*>(lds + idx);
    const fu32x4 val = {w.x ^ lsc[2 * r], w.y, w.x + (uint32_t)c, w.y ^ (uint32_t)r};
    __builtin_nontemporal_store(val, reinterpret_cast<fu32x4*>(f0 + 16 * (int64_t)j));
    r += 4096;
    while (r >= len) {
      r -= len;
      c++;
    }
  }
  if (f1 >= f0) {
    const int head = (int)(f0 - a0), tail = (int)(a1 - f1);
    if (t < head) base[t] = lds[t];
    if (t >= 64 && t - 64 < tail) reinterpret_cast<uint8_t*>(f1)[t - 64] = lds[t];
  } else if (t < size) {
    base[t] = lds[t];
  }
  const int tiles = (len + 127) / 128;
  for (int k = t; k < tiles * 64; k += 256) {
    const int tr = k >> 6, cc = k & 63;
    out_s[(int64_t)(soffs[i] + tr) * N + c0 + cc] = (float)lds[(tr * 4096 + cc) % ldsz];
  }
}

// ---- rowwise FP8 requant, 16 rows x 4 groups of 128 elements (mxfp4_to_fp8_kernel<16, true, false>)
__global__ __launch_bounds__(256) void requant_floor(const uint8_t* __restrict__ q, const uint8_t* __restrict__ s,
                                                     fu32x4* __restrict__ out, float* __restrict__ out_s, uint32_t M,
                                                     uint32_t gpr, uint32_t gx) {
  const uint32_t L = xcd_order(blockIdx.x, gridDim.x), bx = L % gx, by = L / gx;
  const int64_t kb = 64 * (int64_t)gpr, ppr = 8 * (int64_t)gpr;
  fu32x2 c[2];
  uint32_t sd[2];
#pragma unroll
  for (int u = 0; u < 2; u++) {  // unconditional loads at clamped indices: the pattern's best case
    const int e = u * 256 + threadIdx.x;
    const uint32_t r = by * 16 + e / 32, cp = bx * 32 + e % 32;
    const uint32_t rr = r < M ? r : M - 1, cpc = cp < 8 * gpr ? cp : 8 * gpr - 1;
    c[u] = *reinterpret_cast<const fu32x2*>(q + rr * kb + 8 * (int64_t)cpc);
    sd[u] = *reinterpret_cast<const uint32_t*>(s + rr * (kb / 16) + 4 * (cpc >> 3));
  }
  // every store after both pairs' loads, as the product orders them
  fu32x4 v[2];
#pragma unroll
  for (int u = 0; u < 2; u++) v[u] = fu32x4{c[u][0], c[u][1], sd[u], c[u][0] ^ sd[u]};
  floor_materialize(v);
#pragma unroll
  for (int u = 0; u < 2; u++) {
    const int e = u * 256 + threadIdx.x;
    const uint32_t r = by * 16 + e / 32, cp = bx * 32 + e % 32;
    if (r >= M || cp >= 8 * gpr) continue;
    __builtin_nontemporal_store(v[u], out + (int64_t)r * ppr + cp);
    if ((cp & 7) == 0) out_s[(int64_t)(cp >> 3) * M + r] = __uint_as_float(v[u][2] & 0x3FFFFFFFu);
  }
}

// ---- dequant to bf16, U code dwords per lane (dequant_bf16_kernel<U, U == 4>, the product's choice of U)
template <int U>
__global__ __launch_bounds__(256) void dequant_floor(const uint32_t* __restrict__ q, const uint8_t* __restrict__ s,
                                                     fu32x4* __restrict__ out, int64_t ndw) {
  // the product's addressing: a workgroup base and clamped 32-bit lane offsets
  const int64_t b0 = (int64_t)blockIdx.x * (256 * U);
  const uint32_t* qb = q + b0;
  const uint8_t* sb0 = s + (b0 >> 2);
  fu32x4* ob = out + b0;
  const uint32_t lim = ndw - b0 < 256 * U ? (uint32_t)(ndw - b0) : 256u * U;
  uint32_t c[U], sb[U];
#pragma unroll
  for (int u = 0; u < U; u++) {
    const uint32_t i = min(u * 256 + threadIdx.x, lim - 1);
    c[u] = U == 4 ? __builtin_nontemporal_load(qb + i) : qb[i];  // the product's load policy
    sb[u] = sb0[i >> 2];
  }
  fu32x4 v[U];  // every store after all loads, as the product orders them
#pragma unroll
  for (int u = 0; u < U; u++) v[u] = fu32x4{c[u], sb[u], c[u] ^ sb[u], c[u] + sb[u]};
  floor_materialize(v);
#pragma unroll
  for (int u = 0; u < U; u++) {
    const uint32_t i = u * 256 + threadIdx.x;
    if (i < lim) __builtin_nontemporal_store(v[u], ob + i);
  }
}

int device_lds() {
  int dev = 0, lds = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
    return 0;
  return lds;
}

}  // namespace

extern "C" {

// Dual-layout floor for x [M, K] bf16 (M % 256 == 0, K % 256 == 0): outputs as
// the product's (row codes M*K/2, row scales M*K/32, column codes, column scales).
__attribute__((visibility("default"))) int omo_floor_dual(const void* x, void* row_q, void* row_s, void* col_q,
                                                          void* col_s, int64_t M, int64_t K, hipStream_t stream) {
  if (M <= 0 || K <= 0 || M % 256 || K % 256) return -1;
  const int tiles_ms = (int)(M / 256), tiles = (int)(tiles_ms * (K / 256)), per_xcd = (tiles + 7) / 8;
  hipLaunchKernelGGL((dual_floor<0, 0>), dim3((unsigned)(per_xcd * 8)), dim3(512), 0, stream,
                     static_cast<const uint16_t*>(x), static_cast<uint32_t*>(row_q), static_cast<uint8_t*>(row_s),
                     static_cast<uint8_t*>(col_q), static_cast<uint8_t*>(col_s), M, K, tiles_ms, tiles, per_xcd);
  return (int)hipGetLastError();
}

// Other schedules of the dual-layout traffic on the same buffers: kind 1 =
// no scale stores, 2 = scales as whole non-temporal lines (layout-free
// bound), 3 = the product's stores in contiguous K-fastest ranges per XCD,
// 4 = in contiguous M-fastest ranges per XCD, 5 = in aligned groups (K % 2048 == 0).
__attribute__((visibility("default"))) int omo_floor_dual_variant(int kind, const void* x, void* row_q, void* row_s,
                                                                  void* col_q, void* col_s, int64_t M, int64_t K,
                                                                  hipStream_t stream) {
  if (M <= 0 || K <= 0 || M % 256 || K % 256 || kind < 1 || kind > 5) return -1;
  if (kind == 5 && K % 2048) return -1;
  const int tiles_ms = (int)(M / 256), tiles = (int)(tiles_ms * (K / 256)), per_xcd = (tiles + 7) / 8;
  auto kern = kind == 1 ? dual_floor<1, 0>
              : kind == 2 ? dual_floor<2, 0>
              : kind == 3 ? dual_floor<0, 2>
              : kind == 4 ? dual_floor<0, 1>
                          : dual_floor<0, 3>;
  hipLaunchKernelGGL(kern, dim3((unsigned)(per_xcd * 8)), dim3(512), 0, stream, static_cast<const uint16_t*>(x),
                     static_cast<uint32_t*>(row_q), static_cast<uint8_t*>(row_s), static_cast<uint8_t*>(col_q),
                     static_cast<uint8_t*>(col_s), M, K, tiles_ms, tiles, per_xcd);
  return (int)hipGetLastError();
}

// Dense row -> col floor: codes [M, N/2], scales [M, N/32] -> [N, M] bytes and
// [M/128, N] floats (M % 128 == 0, N % 256 == 0).
__attribute__((visibility("default"))) int omo_floor_rowcol(const void* q, const void* s, void* out, float* out_s,
                                                            int64_t M, int64_t N, hipStream_t stream) {
  if (M <= 0 || N <= 0 || M % 128 || N % 256) return -1;
  hipLaunchKernelGGL(rowcol_floor, dim3((unsigned)((M / 128) * (N / 256))), dim3(256), 0, stream,
                     static_cast<const uint8_t*>(q), static_cast<const uint8_t*>(s), static_cast<uint8_t*>(out), out_s, M,
                     N);
  return (int)hipGetLastError();
}

// Per-split row -> col floor with the product launcher's LDS reserve
// (residency capped at four workgroups per CU); N % 256 == 0, metadata as the
// product's (int32 device arrays). Its flat grid reads one split per lane, so
// it takes at most 64 splits (split x row tile x band beyond): it matches the
// product's grid only up to 64 splits (the product's flat grid takes 128),
// with the product's order (band walk on rows of more than 16 bands, else
// contiguous ranges).
__attribute__((visibility("default"))) int omo_floor_msplit(const void* q, const void* s, void* out, float* out_s,
                                                            int64_t total_rows, int64_t N, const int32_t* lens,
                                                            const int32_t* offs, const int32_t* soffs, int64_t nsplits,
                                                            int64_t max_split_len, int64_t out_s_rows,
                                                            hipStream_t stream) {
  if (N <= 0 || N % 256 || nsplits <= 0 || nsplits > 65535 || max_split_len <= 0 || max_split_len > total_rows ||
      (max_split_len + 127) / 128 > 65535 || N / 256 > 65535)
    return -1;
  const int per_wg = device_lds() / 4 - 2560;
  const size_t reserve = per_wg > kWideSmemBytes ? (size_t)(per_wg - kWideSmemBytes) : 0;
  const int64_t tm = (max_split_len + 127) / 128, bands = N / 256;
  if (nsplits <= 64 && tm * bands + 7 <= (int64_t)UINT32_MAX / 256 / nsplits) {
    hipLaunchKernelGGL(bands > 16 ? msplit_flat_floor<true> : msplit_flat_floor<false>,
                       dim3((unsigned)(8 * nsplits * ((tm * bands + 7) / 8))), dim3(256), reserve, stream,
                       static_cast<const uint8_t*>(q), static_cast<const uint8_t*>(s), static_cast<uint8_t*>(out), out_s,
                       lens, offs, soffs, total_rows, N, out_s_rows, (reinterpret_cast<uintptr_t>(out) & 127) == 0,
                       (int)nsplits, (int)tm, (int)bands);
    return (int)hipGetLastError();
  }
  const dim3 grid((unsigned)nsplits, (unsigned)tm, (unsigned)bands);
  hipLaunchKernelGGL(msplit_floor, grid, dim3(256), reserve, stream, static_cast<const uint8_t*>(q),
                     static_cast<const uint8_t*>(s), static_cast<uint8_t*>(out), out_s, lens, offs, soffs, total_rows, N,
                     out_s_rows, (reinterpret_cast<uintptr_t>(out) & 127) == 0);
  return (int)hipGetLastError();
}

// Per-split band-schedule floor (msplit_band_floor): N % 64 == 0, every split
// at most kBandMaxRows rows (max_split_len bounds them; the split table is
// the product's int32 device arrays).
__attribute__((visibility("default"))) int omo_floor_msplit_band(const void* q, const void* s, void* out, float* out_s,
                                                                 int64_t N, const int32_t* lens, const int32_t* offs,
                                                                 const int32_t* soffs, int64_t nsplits,
                                                                 int64_t max_split_len, hipStream_t stream) {
  if (N <= 0 || N % 64 || nsplits <= 0 || max_split_len <= 0 || max_split_len > kBandMaxRows ||
      nsplits * (N / 64) > 0x7FFFFFFF / 8)
    return -1;
  const int bands = (int)(N / 64), total = (int)(nsplits * bands), per_xcd = (total + 7) / 8;
  // at least 256 B: the partial end chunks copy LDS bytes 0..79
  const size_t lds = std::max<size_t>((size_t)max_split_len * 34 + 16, 256);
  static bool attr = false;
  if (!attr) {
    if (hipFuncSetAttribute((const void*)msplit_band_floor, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)(kBandMaxRows * 34 + 16)) != hipSuccess)
      return -2;
    attr = true;
  }
  hipLaunchKernelGGL(msplit_band_floor, dim3((unsigned)(per_xcd * 8)), dim3(256), lds, stream,
                     static_cast<const uint8_t*>(q), static_cast<const uint8_t*>(s), static_cast<uint8_t*>(out), out_s,
                     lens, offs, soffs, N, bands, total, per_xcd);
  return (int)hipGetLastError();
}

// Rowwise FP8 requant floor: codes [M, Kb], scales [M, Kb/16] -> [M, 2 Kb]
// bytes and [Kb/64, M] floats (Kb % 64 == 0, 8 B aligned codes).
__attribute__((visibility("default"))) int omo_floor_requant(const void* q, const void* s, void* out, float* out_s,
                                                             int64_t M, int64_t Kb, hipStream_t stream) {
  if (M <= 0 || Kb <= 0 || Kb % 64 || M > 0x7FFFFFFF) return -1;
  const int64_t gpr = Kb / 64, gx = (gpr + 3) / 4, gy = (M + 15) / 16;
  hipLaunchKernelGGL(requant_floor, dim3((unsigned)(gx * gy)), dim3(256), 0, stream, static_cast<const uint8_t*>(q),
                     static_cast<const uint8_t*>(s), static_cast<fu32x4*>(out), out_s, (uint32_t)M, (uint32_t)gpr,
                     (uint32_t)gx);
  return (int)hipGetLastError();
}

// Dequant floor: ndw code dwords (+ ndw/4 scale bytes) -> ndw x 16 B.
__attribute__((visibility("default"))) int omo_floor_dequant(const void* q, const void* s, void* out, int64_t ndw,
                                                             hipStream_t stream) {
  if (ndw <= 0) return -1;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return -1;
  if ((ndw + 1023) / 1024 <= 8 * (int64_t)cus)  // the product's rule
    hipLaunchKernelGGL(dequant_floor<4>, dim3((unsigned)((ndw + 1023) / 1024)), dim3(256), 0, stream,
                       static_cast<const uint32_t*>(q), static_cast<const uint8_t*>(s), static_cast<fu32x4*>(out), ndw);
  else
    hipLaunchKernelGGL(dequant_floor<2>, dim3((unsigned)((ndw + 511) / 512)), dim3(256), 0, stream,
                       static_cast<const uint32_t*>(q), static_cast<const uint8_t*>(s), static_cast<fu32x4*>(out), ndw);
  return (int)hipGetLastError();
}


// Grouped dual-layout floor over `count` items (at most 32; each M % 64 == 0,
// K % 256 == 0, 16 B aligned buffers): x[i] [M[i], K[i]] bf16 with the
// product's four outputs. scm 0 = the product's stores, 1 = no scale stores.
__attribute__((visibility("default"))) int omo_floor_dual_grouped(int scm, const void* const* x, void* const* row_q,
                                                                  void* const* row_s, void* const* col_q,
                                                                  void* const* col_s, const int64_t* M,
                                                                  const int64_t* K, int count, hipStream_t stream) {
  if (scm < 0 || scm > 1 || count <= 0 || count > kFloorGroupMax) return -1;
  FloorGroup g;
  memset(&g, 0, sizeof(g));
  g.count = count;
  int64_t slots = 0;
  for (int i = 0; i < count; i++) {
    if (M[i] <= 0 || K[i] <= 0 || M[i] % 64 || K[i] % 256 || (M[i] / 64) * (K[i] / 256) > 0x7FFFFFFF / 8) return -1;
    FloorItem& it = g.item[i];
    it.x = static_cast<const uint16_t*>(x[i]);
    it.row_q = static_cast<uint32_t*>(row_q[i]);
    it.row_s = static_cast<uint8_t*>(row_s[i]);
    it.col_q = static_cast<uint8_t*>(col_q[i]);
    it.col_s = static_cast<uint8_t*>(col_s[i]);
    it.M = M[i];
    it.K = K[i];
    it.tiles_m = (int)(M[i] / 64);
    it.tiles = it.tiles_m * (int)(K[i] / 256);
    it.per_xcd = (it.tiles + 7) / 8;
    slots += it.per_xcd;
  }
  if (slots > 0x7FFFFFFF / 8) return -1;
  hipLaunchKernelGGL(scm ? dual_grouped_floor<1> : dual_grouped_floor<0>, dim3((unsigned)(slots * 8)), dim3(512), 0,
                     stream, g);
  return (int)hipGetLastError();
}

}  // extern "C"
