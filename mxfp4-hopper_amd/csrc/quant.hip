// BF16 -> MXFP4 rowwise quantize (1x32 blocks over the flat tensor).
//
// Semantics follow per_token_group_quant_4bit_kernel_coalescing
// (code/kernel/per_token_quant_mxfp4.cu:121-266):
//   amax  = fmaxf(eps, |x_j|) over the 32 elements (NaN ignored)     :151,170-178
//   y_s   = 2^ceil(log2(max(amax / fp4_max, 1e-10f)))               :185-187
//   scale = (uint8)((int)log2(y_s) + 127)                            :192
//   q_j   = clamp(x_j * (1/y_s), fp4_min, fp4_max) -> E2M1 RNE nibble :200-254
//
// Layout in HBM: the input is read as 16-byte chunks of 8 bf16; four
// consecutive chunks form one 32-element block. Chunk i is handled by one
// lane, so a block is a DPP quad (lanes 4k..4k+3) and the block amax is two
// quad_perm max steps. A wave touches 1 KiB of contiguous input per load,
// 256 B of contiguous codes per store and 16 contiguous scale bytes.
//
// Fast path (fp4_min == -6, fp4_max == 6, block free of inf/NaN):
//   * amax via packed u16 max of |x| bit patterns (monotone for non-NaN),
//   * the scale exponent in closed form: for a bf16 amax = (1+f/128)*2^E,
//     ceil(log2(amax/6)) = E - 2 + (f > 64); amax/6 is either an exact power
//     of two (f == 64) or at least 0.5% away from one, so rounding of the
//     quotient never moves the ceiling; the scale of fmaxf(eps, amax) is
//     the larger of the two scales, so eps and the 1e-10 floor (exponent
//     -33) enter as max(c, c_eps);
//   * q = x / 2^c is exact and |q| <= 6, so v_cvt_scalef32_pk_fp4_bf16
//     (round-to-nearest-even, verified bit-exact against the reference rule
//     over every bf16 value and every reachable c in [-33, 126]) yields the
//     reference nibbles, 2 elements per instruction.
// Blocks holding inf or NaN, and non-default clamp constants, take the
// emulation path, which restates the reference operations in fp32.
//
// Tensors whose per-CU share fits one LDS round and divides well into the
// kernel's steps (e.g. 4096 x 7168, 8192 x 7168) take quant_phased_kernel,
// which reads and converts a workgroup's share into LDS before writing it;
// the others take quant_rowwise_kernel. Both produce the same bytes.
#include "omo_internal.h"
#include "omo_quant.cuh"

namespace omo_hip {

struct QuantArgs {
  const u32x4* __restrict__ x;  // bf16, 8 per chunk
  uint32_t* __restrict__ q;     // 8 nibbles per chunk
  uint8_t* __restrict__ s;      // one E8M0 byte per 4 chunks
  int64_t nchunks;              // numel / 8, multiple of 4
  float eps, fp4_min, fp4_max;
  int c_eps;                    // scale exponent when amax == eps (fast path)
};

// EAGER: every chunk of the lane is loaded (at a clamped index), converted
// and only then stored, so no wait separates one chunk's stores from the
// next chunk's conversion. Otherwise each chunk is loaded under a bounds
// test and stored before the next one converts; the wait for its loads
// before the second chunk then also covers the first chunk's stores (loads
// and stores share one counter), which slows each wave down. That pacing
// pays on tensors too large for one LDS round per CU (16431 x 7168: 46.6
// against 47.4 us eager) and costs elsewhere (16431 x 2048 15.45 against
// 15.03 us, 2048 x 2048 3.53 against 3.37, 1000 x 7168 4.72 against 4.48;
// 16431 x 4096 27.8 either way).
template <int UNROLL, bool STANDARD, bool EAGER>
__global__ __launch_bounds__(256) void quant_rowwise_kernel(QuantArgs a) {
  const int64_t base = (int64_t)blockIdx.x * (256 * UNROLL) + threadIdx.x;
  const bool quad_leader = (threadIdx.x & 3u) == 0u;
  u32x4 d[UNROLL];
#pragma unroll
  for (int u = 0; u < UNROLL; u++) {
    const int64_t ch = base + (int64_t)u * 256;
    if (EAGER) d[u] = __builtin_nontemporal_load(a.x + (ch < a.nchunks ? ch : a.nchunks - 1));
    else if (ch < a.nchunks) d[u] = __builtin_nontemporal_load(a.x + ch);
  }
  uint32_t codes[UNROLL], byte[UNROLL];
#pragma unroll
  for (int u = 0; u < UNROLL; u++) {
    const int64_t ch = base + (int64_t)u * 256;
    // nchunks is a multiple of 4 and quads are 4-aligned, so a quad is
    // either fully inside or fully outside the tensor (EAGER: an outside
    // quad converts four copies of the last chunk and stores nothing).
    if (!EAGER && ch >= a.nchunks) continue;
    if (STANDARD) {
      uint32_t am = quad_max_u32(chunk_absmax_bits(d[u]));
      if (__builtin_expect(am < 0x7F80u, 1)) {
        codes[u] = quant_chunk_fast(d[u], am, a.c_eps, &byte[u]);
      } else {
        quant_chunk_ref(d[u], a.eps, a.fp4_min, a.fp4_max, &codes[u], &byte[u]);
      }
    } else {
      quant_chunk_ref(d[u], a.eps, a.fp4_min, a.fp4_max, &codes[u], &byte[u]);
    }
    if (EAGER) continue;
    // Codes are streamed out non-temporally (each wave store is 256
    // contiguous bytes); the one-byte scale stores stay temporal, which
    // measured faster for them.
    __builtin_nontemporal_store(codes[u], a.q + ch);
    if (quad_leader) a.s[ch >> 2] = (uint8_t)byte[u];
  }
  if (EAGER) {
#pragma unroll
    for (int u = 0; u < UNROLL; u++) {
      const int64_t ch = base + (int64_t)u * 256;
      if (ch >= a.nchunks) continue;
      __builtin_nontemporal_store(codes[u], a.q + ch);
      if (quad_leader) a.s[ch >> 2] = (uint8_t)byte[u];
    }
  }
}


// Two-phase form for large tensors (default clamp constants, 16 B aligned
// outputs): one 1024-thread workgroup per CU takes a contiguous share of the
// chunks and, in rounds that fit its LDS, first reads and quantizes the
// round (codes and scale bytes kept in LDS), then writes the round out as
// 16 B stores. Every workgroup follows the same schedule, so HBM sees long
// read phases and short write phases instead of reads and writes
// interleaved: at 8192 x 7168 this takes 23.0 us against 24.6 us for
// quant_rowwise_kernel. The loads of the next step are issued before the
// current step is converted (without that, the conversion delays the loads
// and the kernel took 27.9 us). Measured and not kept (8192 x 7168, same box
// each): loads two steps ahead 24.4 against 23.2 us; steps of 1024 or 4096
// chunks 25.9 / 24.0; writing the first half of the round while the second
// is read 27.0 against 23.7; step i of every workgroup in one contiguous
// region (workgroups interleaved) 23.7 against 23.0; temporal code stores in
// the write phase 24.1 against 23.6 (and no faster 4096 x 4096 round trip).
constexpr int kPhThreads = 1024;
constexpr int kPhUnroll = 2;
constexpr int kWaitVmcnt0 = 0x0F70;  // s_waitcnt vmcnt(0) expcnt(7) lgkmcnt(15), gfx9 field layout

// Quantizes the step of chunks [i0, i0 + kPhThreads * kPhUnroll) held in d
// (lane t: chunks i0 + u * kPhThreads + t) into lds_q / lds_s, writing only
// chunks below n. Every lane converts every loaded chunk (past n: a reload
// of chunk 0), so each load is consumed on every path: a load skipped under
// a per-lane bounds test left the compiler a wait for it at the register's
// next write, in the write phase, where that wait also covered every code
// store issued so far.
__device__ __forceinline__ void ph_convert_step(const QuantArgs& a, const u32x4 (&d)[kPhUnroll], int i0, int n,
                                                uint32_t* lds_q, uint8_t* lds_s) {
  const int t = threadIdx.x;
  const bool quad_leader = (t & 3) == 0;
#pragma unroll
  for (int u = 0; u < kPhUnroll; u++) {
    const int i = i0 + u * kPhThreads + t;
    uint32_t codes, byte;
    const uint32_t am = quad_max_u32(chunk_absmax_bits(d[u]));
    if (__builtin_expect(am < 0x7F80u, 1)) {
      codes = quant_chunk_fast(d[u], am, a.c_eps, &byte);
    } else {
      quant_chunk_ref(d[u], a.eps, -6.0f, 6.0f, &codes, &byte);
    }
    if (i < n) {
      lds_q[i] = codes;
      if (quad_leader) lds_s[i >> 2] = (uint8_t)byte;
    }
  }
}

// Read phase of the two-phase kernels: loads chunks [c0, c0 + n) of a.x (n a
// multiple of 4, so quads are whole), quantizes them and leaves the code
// dwords in lds_q[0, n) and the scale bytes in lds_s[0, n / 4). The caller
// synchronizes before reading them. Each step's loads are issued before the
// previous step is converted; the last step is peeled off so that it issues
// no loads past the share (a reload of chunk 0 per lane there, unused, cost
// 23.43 against 23.12 us at 8192 x 7168 and 16.15 against 15.90 us for the
// 4096 x 4096 quantize + dequantize round trip).
__device__ __forceinline__ void ph_read_phase(const QuantArgs& a, int64_t c0, int n, uint32_t* lds_q, uint8_t* lds_s) {
  const int t = threadIdx.x;
  constexpr int kStep = kPhThreads * kPhUnroll;
  u32x4 nx[kPhUnroll];
#pragma unroll
  for (int u = 0; u < kPhUnroll; u++) {
    const int i = u * kPhThreads + t;
    nx[u] = __builtin_nontemporal_load(a.x + c0 + (i < n ? i : 0));
  }
  int i0 = 0;
  for (; i0 + kStep < n; i0 += kStep) {
    u32x4 d[kPhUnroll];
#pragma unroll
    for (int u = 0; u < kPhUnroll; u++) d[u] = nx[u];
#pragma unroll
    for (int u = 0; u < kPhUnroll; u++) {
      const int i = i0 + kStep + u * kPhThreads + t;
      nx[u] = __builtin_nontemporal_load(a.x + c0 + (i < n ? i : 0));
    }
    ph_convert_step(a, d, i0, n, lds_q, lds_s);
  }
  ph_convert_step(a, nx, i0, n, lds_q, lds_s);
  // Every load is consumed and no store is outstanding yet, so this wait
  // costs nothing; without it the compiler, unsure whether registers reused
  // in the write phase still await a load, waited between the code stores
  // and the scale stores for every code store (23.01 against 22.84 us at
  // 8192 x 7168). The same loop with two register sets, so that the next
  // step's loads go out before the wait for the current one, took 23.58.
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
}

__global__ __launch_bounds__(kPhThreads) void quant_phased_kernel(QuantArgs a, int64_t share, int round) {
  extern __shared__ __attribute__((aligned(16))) uint32_t ph_lds[];  // round code dwords, then round/4 scale bytes
  uint8_t* lsc = reinterpret_cast<uint8_t*>(ph_lds + round);
  const int t = threadIdx.x;
  const int64_t wg_begin = (int64_t)blockIdx.x * share;
  const int64_t wg_end = wg_begin + share < a.nchunks ? wg_begin + share : a.nchunks;
  for (int64_t r0 = wg_begin; r0 < wg_end; r0 += round) {
    // chunks of this round: a multiple of 4, so quads are whole
    const int n = (int)(wg_end - r0 < round ? wg_end - r0 : round);
    if (r0 != wg_begin) __syncthreads();  // the previous round's LDS reads are done
    ph_read_phase(a, r0, n, ph_lds, lsc);
    __syncthreads();
    for (int i = 4 * t; i < n; i += 4 * kPhThreads)
      __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(&ph_lds[i]), reinterpret_cast<u32x4*>(a.q + r0 + i));
    // Scale bytes leave non-temporally too: as ordinary stores they stayed
    // in L2 to be written back at the kernel's end (8192 x 7168: 23.04
    // against 22.65 us; the 4096 x 4096 round trip 15.85 against 15.73).
    const int nsb = n / 4;  // scale bytes of the round
    uint8_t* sdst = a.s + r0 / 4;
    for (int i = 16 * t; i < nsb; i += 16 * kPhThreads) {
      if (i + 16 <= nsb) {
        __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(lsc + i), reinterpret_cast<u32x4*>(sdst + i));
      } else {
        for (int j = i; j < nsb; j++) sdst[j] = lsc[j];
      }
    }
  }
}

// Row-strided variant: row r of the codes starts at q + r * q_stride and its
// scales at s + r * s_stride (bytes), so the outputs can be interleaved, e.g.
// the expert-parallel payload row [codes (K/2 B) | scales (K/32 B)] that
// Megatron builds with torch.cat (code/megatron-0.15.0rc7.diff:93-99,
// 163-170). Workgroup b covers segment b % bpr of row b / bpr; a quad (one
// block) never straddles rows because K % 32 == 0 and segments start at
// multiples of 256 chunks. Reference rule with fp4_min = -6, fp4_max = 6.
struct QuantRowsArgs {
  const uint16_t* __restrict__ x;  // [rows, K] bf16
  uint8_t* __restrict__ q;
  uint8_t* __restrict__ s;
  int64_t K, q_stride, s_stride;
  int bpr;                         // workgroups per row
  float eps;
  int c_eps;
};

template <int UNROLL>
__global__ __launch_bounds__(256) void quant_rows_kernel(QuantRowsArgs a) {
  const int64_t row = blockIdx.x / (uint32_t)a.bpr;
  const int seg = (int)(blockIdx.x - row * a.bpr);
  const int cpr = (int)(a.K / 8);  // 16 B chunks per row
  const u32x4* xr = reinterpret_cast<const u32x4*>(a.x + row * a.K);
  uint32_t* qr = reinterpret_cast<uint32_t*>(a.q + row * a.q_stride);
  uint8_t* sr = a.s + row * a.s_stride;
  const int base = seg * (256 * UNROLL) + (int)threadIdx.x;
  // loads at clamped indices and stores after every conversion, as in the
  // EAGER form of quant_rowwise_kernel (quads past the row convert copies
  // of its last chunk and store nothing)
  u32x4 d[UNROLL];
#pragma unroll
  for (int u = 0; u < UNROLL; u++) {
    const int c = base + u * 256;
    d[u] = __builtin_nontemporal_load(xr + (c < cpr ? c : cpr - 1));
  }
  const bool quad_leader = (threadIdx.x & 3u) == 0u;
  uint32_t codes[UNROLL], byte[UNROLL];
#pragma unroll
  for (int u = 0; u < UNROLL; u++) {
    const uint32_t am = quad_max_u32(chunk_absmax_bits(d[u]));
    if (__builtin_expect(am < 0x7F80u, 1)) {
      codes[u] = quant_chunk_fast(d[u], am, a.c_eps, &byte[u]);
    } else {
      quant_chunk_ref(d[u], a.eps, -6.0f, 6.0f, &codes[u], &byte[u]);
    }
  }
#pragma unroll
  for (int u = 0; u < UNROLL; u++) {
    const int c = base + u * 256;
    if (c >= cpr) continue;  // whole quads
    __builtin_nontemporal_store(codes[u], qr + c);
    if (quad_leader) sr[c >> 2] = (uint8_t)byte[u];
  }
}

// Two-phase form of the payload rows [codes (K/2 B) | scales (K/32 B)],
// stride 17K/32 B, for K % 512 == 0 (whole 16 B pieces per row) and 16 B
// aligned buffers: workgroup b takes rows [b * rpw, b * rpw + rpw), whose
// chunks are contiguous in the input and whose payload rows are contiguous
// in the output. The read phase converts them into LDS as in
// quant_phased_kernel; the write phase then covers the output region with
// 16 B stores, piece j of a row coming from the row's code dwords for
// j < K/32 and from its scale bytes after that.
__global__ __launch_bounds__(kPhThreads) void quant_phased_rows_kernel(QuantArgs a, uint8_t* __restrict__ out,
                                                                       int64_t rows, int rpw, int cpr) {
  extern __shared__ __attribute__((aligned(16))) uint32_t ph_lds[];  // rpw * cpr code dwords, then scale bytes
  uint8_t* lsc = reinterpret_cast<uint8_t*>(ph_lds + (int64_t)rpw * cpr);
  const int64_t row0 = (int64_t)blockIdx.x * rpw;
  const int nrows = (int)(rows - row0 < rpw ? rows - row0 : rpw);
  ph_read_phase(a, row0 * cpr, nrows * cpr, ph_lds, lsc);
  __syncthreads();
  const int cq = cpr / 4;          // 16 B pieces of codes per row
  const int ppr = cq + cpr / 64;   // 16 B pieces per payload row
  u32x4* dst = reinterpret_cast<u32x4*>(out + row0 * (int64_t)ppr * 16);
  for (int i = threadIdx.x; i < nrows * ppr; i += kPhThreads) {
    const int r = i / ppr;
    const int j = i - r * ppr;
    const u32x4* src = j < cq ? reinterpret_cast<const u32x4*>(ph_lds + r * cpr) + j
                              : reinterpret_cast<const u32x4*>(lsc + r * (cpr / 4)) + (j - cq);
    __builtin_nontemporal_store(*src, dst + i);
  }
}

hipError_t launch_quant_rows(const void* x, void* q, int64_t q_stride, void* s, int64_t s_stride, int64_t rows,
                             int64_t K, float eps, hipStream_t stream) {
  if (rows == 0 || K == 0) return hipSuccess;
  constexpr int U = 2;
  QuantRowsArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.q = static_cast<uint8_t*>(q);
  a.s = static_cast<uint8_t*>(s);
  a.K = K;
  a.q_stride = q_stride;
  a.s_stride = s_stride;
  a.bpr = (int)((K / 8 + 256 * U - 1) / (256 * U));
  a.eps = eps;
  a.c_eps = host_c_eps(eps, 6.0f);
  // Payload rows (scales right after the codes, one stride) take the
  // two-phase kernel when rpw whole rows per workgroup give every CU a share
  // of at least 6144 chunks that fits its LDS and fills the 2048-chunk steps
  // to at least 95% or takes at most four of them, the conditions under
  // which quant_phased_kernel wins (2048 x 7168, 3.5 steps: 7.7 us against
  // 9.3 one-pass).
  const int64_t stride = K / 32 * 17;
  const bool packed = q_stride == stride && s_stride == stride && static_cast<uint8_t*>(s) == a.q + K / 2;
  const bool aligned16 = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(q)) & 15) == 0;
  if (packed && aligned16 && K % 512 == 0) {
    const DeviceCaps dc = current_device_caps();
    const int64_t cpr = K / 8;
    const int64_t rpw = (rows + dc.cus - 1) / dc.cus;
    const int64_t grid = (rows + rpw - 1) / rpw;
    const int64_t share = rpw * cpr;
    const int64_t steps = (share + kPhThreads * kPhUnroll - 1) / (kPhThreads * kPhUnroll);
    const double fill = (double)(rows * cpr) / ((double)grid * kPhThreads * kPhUnroll * (double)steps);
    const int64_t lds = share * 4 + share / 4;
    if (share >= 6144 && lds <= dc.lds_per_workgroup && (fill >= 0.95 || steps <= 4) && grid >= dc.cus / 2) {
      QuantArgs p;
      p.x = static_cast<const u32x4*>(x);
      p.q = nullptr;
      p.s = nullptr;
      p.nchunks = rows * cpr;
      p.eps = eps;
      p.fp4_min = -6.0f;
      p.fp4_max = 6.0f;
      p.c_eps = a.c_eps;
      return launch(quant_phased_rows_kernel, dim3((unsigned)grid), dim3(kPhThreads), (size_t)lds, stream, p,
                         a.q, rows, (int)rpw, (int)cpr);
    }
  }
  return launch((quant_rows_kernel<U>), dim3((unsigned)(rows * a.bpr)), dim3(256), 0, stream, a);
}

hipError_t launch_quant_rowwise(const void* x, void* q, void* s, int64_t numel, float eps, float fp4_min,
                                float fp4_max, hipStream_t stream) {
  QuantArgs a;
  a.x = static_cast<const u32x4*>(x);
  a.q = static_cast<uint32_t*>(q);
  a.s = static_cast<uint8_t*>(s);
  a.nchunks = numel / 8;
  a.eps = eps;
  a.fp4_min = fp4_min;
  a.fp4_max = fp4_max;
  a.c_eps = host_c_eps(eps, fp4_max);
  if (a.nchunks == 0) return hipSuccess;
  constexpr int U = 2;
  const int64_t blocks = (a.nchunks + 256 * U - 1) / (256 * U);
  const bool standard = (fp4_max == 6.0f && fp4_min == -6.0f);
  const DeviceCaps dc = current_device_caps();
  const bool aligned16 = ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(s)) & 15) == 0;
  // Two-phase kernel when each workgroup's share (a multiple of 64 chunks,
  // 16 B of scale bytes) is at least 6144 chunks (at 4096, 2048 x 4096 ran
  // 5.48 us two-phase against 5.06 us one-pass; at 6144, 3072 x 4096 6.59
  // against 7.15; 4096 x 4096, a share of 8192, 8.15 against 8.79), fits its
  // LDS in one round (4 B of codes + 1/4 B of scale per chunk), and either
  // fills its steps of 2048 chunks to at least 95% or takes at most four of
  // them (2048 x 7168, 3.5 steps: 7.49 against 8.22). Measured where neither
  // holds: 16431 x 2048 (8.03 steps per CU) and 16431 x 4096 (16.06) ran
  // 6-8% slower two-phase than quant_rowwise_kernel, both in 9 / 17 steps and
  // with the surplus chunks loaded alongside the first step (8 / 16 steps);
  // several rounds per workgroup (alternating read and write phases) measured
  // 6-12% slower, and 4096 x 4096 as one round of one-pass workgroups (four
  // chunks per lane) 0.8 us slower per quantize + dequantize round trip.
  const int64_t share = ((a.nchunks + dc.cus - 1) / dc.cus + 63) / 64 * 64;
  const int64_t cap = (int64_t)dc.lds_per_workgroup * 4 / 17 / 64 * 64;
  const int64_t steps = (share + kPhThreads * kPhUnroll - 1) / (kPhThreads * kPhUnroll);
  const double fill = (double)a.nchunks / ((double)dc.cus * kPhThreads * kPhUnroll * (double)steps);
  if (standard && aligned16 && share >= 6144 && share <= cap && (fill >= 0.95 || steps <= 4)) {
    const int round = (int)share;
    return launch(quant_phased_kernel, dim3((unsigned)dc.cus), dim3(kPhThreads), (size_t)round * 4 + round / 4,
                       stream, a, share, round);
  }
  // per-chunk stores where the share exceeds one LDS round (see quant_rowwise_kernel)
  const bool eager = share <= cap;
  auto kernel = standard ? (eager ? quant_rowwise_kernel<U, true, true> : quant_rowwise_kernel<U, true, false>)
                         : (eager ? quant_rowwise_kernel<U, false, true> : quant_rowwise_kernel<U, false, false>);
  return launch(kernel, dim3((unsigned)blocks), dim3(256), 0, stream, a);
}

}  // namespace omo_hip
