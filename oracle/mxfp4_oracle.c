/*
 * mxfp4_oracle.c -- CPU restatement of the reference MXFP4 kernels.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the parity checker for the HIP
 * library and the timed CPU baseline in bench.py. Only tests/, the smoke()
 * entry point and bench.py's cpu_baseline leg may load it. The product path
 * (the HIP library and the omo / omo_python_api packages) never calls it.
 *
 * Every function follows the reference CUDA kernel operation by operation,
 * including its quirks, so that a mismatch against the GPU means a GPU bug.
 * All paths are relative to the reference repository root.
 *
 * Pins (see tests/test_oracle_*.py): each function below is checked against
 * an independent statement of the same mathematics -- textbook E2M1
 * round-to-nearest-even, an exact closed form of the E8M0 scale rule,
 * exact products + torch's bfloat16 / float8_e4m3fn casts, brute-force index
 * maps, and hand-derived known answers for the quirks.
 *
 * Build: gcc -O2 -ffp-contract=off -fno-fast-math -fPIC -shared -pthread
 *        (see oracle/Makefile). No FMA contraction: every float op is a
 *        separately rounded IEEE-754 binary32 operation, as in the reference
 *        (built without --use_fast_math, code/kernel/setup.py:46-56).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORACLE_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------------ */
/* bit helpers                                                               */
/* ------------------------------------------------------------------------ */
static inline float u32_as_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_as_u32(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bf16_to_f32(uint16_t b) { return u32_as_f32((uint32_t)b << 16); }

/* PTX shr.u32 clamps shift amounts >= 32 to 32 (result 0). The reference
 * relies on this in adjust_denormal_opt2 (per_token_quant_mxfp4.cu:103-112),
 * where the shift is 126-e and reaches >= 32 for e <= 94. */
static inline uint32_t ptx_shr_u32(uint32_t x, uint32_t s) { return s >= 32u ? 0u : (x >> s); }

/* cvt.rzi.s32.f32: truncation toward zero, saturating to [INT_MIN, INT_MAX],
 * NaN -> 0 (PTX ISA float-to-integer conversion semantics). The reference
 * reaches the saturating case through (int)log2f(inf) for a block holding an
 * infinity (per_token_quant_mxfp4.cu:192). */
static inline int32_t cvt_rzi_s32(float f) {
  if (isnan(f)) return 0;
  if (f >= 2147483648.0f) return INT32_MAX;
  if (f <= -2147483648.0f) return INT32_MIN;
  return (int32_t)f;
}

/* float -> uint8 conversion (cvt.rzi.u8.f32 semantics: truncate, clamp to
 * [0,255], NaN -> 0). Used for `uint8_t local_absmax = eps`
 * (per_token_Mxfp4ToFp8_col.cu:141). */
static inline uint8_t cvt_rzi_u8(float f) {
  if (!(f > 0.0f)) return 0;
  if (f >= 255.0f) return 255;
  return (uint8_t)f;
}

/* IEEE binary32 -> bfloat16, round to nearest even; NaN -> 0x7FFF.
 * Stands for __floats2bfloat162_rn (per_token_Mxfp4ToBf16_dequant.cu:153).
 * The NaN payload is not pinned by anything in the reference. */
static inline uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = f32_as_u32(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FFFu;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* IEEE binary32 -> OCP FP8 E4M3 (e4m3fn), round to nearest even, saturate
 * finite overflow to +-448, NaN -> 0x7F. Stands for the __nv_fp8_e4m3(float)
 * constructor (RNE, satfinite), used at per_token_Mxfp4ToFp8.cu:228-229,
 * per_token_Mxfp4ToFp8_col.cu:289-290, per_token_Mxfp4RowToBf16ToFp8Col.cu:177,
 * per_token_Mxfp4RowToBf16ToFp8Col_msplit.cu:196. Written from the OCP
 * format definition: bias 7, 3 mantissa bits, subnormal step 2^-9, max 448. */
static inline uint8_t f32_to_e4m3_rne_sat(float f) {
  uint32_t u = f32_as_u32(f);
  uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7F;
  float a = fabsf(f);
  if (a >= 464.0f) return sign | 0x7E; /* >= midpoint(448, 512): saturate */
  if (a < 0.015625f) {                 /* below 2^-6: subnormal grid of 2^-9 */
    float k = nearbyintf(a * 512.0f);  /* exact scaling, RNE to integer */
    return sign | (uint8_t)k;          /* k == 8 encodes 2^-6 (exp 1, mant 0) */
  }
  int e;
  float m = frexpf(a, &e); /* a = m * 2^e, m in [0.5, 1) */
  int exp = e - 1;         /* a = (2m) * 2^exp, 2m in [1, 2) */
  float k = nearbyintf((2.0f * m - 1.0f) * 8.0f);
  int ki = (int)k;
  if (ki == 8) { ki = 0; exp += 1; }
  int be = exp + 7;
  if (be > 15 || (be == 15 && ki == 7)) return sign | 0x7E;
  return sign | (uint8_t)((be << 3) | ki);
}

/* E2M1 nibble -> bfloat16 bits, the decode used by every reference
 * dequant/requant kernel (per_token_Mxfp4ToBf16_dequant.cu:137-150,
 * per_token_Mxfp4ToFp8.cu:192-214, per_token_Mxfp4RowToBf16ToFp8Col.cu:108-121).
 * nib is the 4-bit code in the low bits. */
static inline uint16_t e2m1_to_bf16_bits(uint8_t nib) {
  uint8_t em = nib & 0x07;
  uint16_t x = (uint16_t)((uint16_t)em << 6) | (uint16_t)((nib & 0x08) << 12);
  if ((em & 0x06) != 0) x = (uint16_t)(x + (uint16_t)(126u << 7));
  if (em == 0x01) x = (uint16_t)(16128u | (x & 0x8000u));
  return x;
}

/* ------------------------------------------------------------------------ */
/* threading                                                                 */
/* ------------------------------------------------------------------------ */
typedef void (*range_fn)(void* ctx, int64_t begin, int64_t end);
typedef struct { range_fn fn; void* ctx; int64_t b, e; } job_t;
static void* job_main(void* p) { job_t* j = (job_t*)p; j->fn(j->ctx, j->b, j->e); return NULL; }

static void parallel_for(int64_t n, int nthreads, range_fn fn, void* ctx) {
  if (n <= 0) return;
  if (nthreads < 1) nthreads = 1;
  if (nthreads > 256) nthreads = 256;
  if ((int64_t)nthreads > n) nthreads = (int)n;
  if (nthreads == 1) { fn(ctx, 0, n); return; }
  pthread_t th[256];
  job_t jobs[256];
  int64_t chunk = (n + nthreads - 1) / nthreads;
  int started = 0;
  for (int t = 0; t < nthreads; t++) {
    int64_t b = (int64_t)t * chunk, e = b + chunk;
    if (b >= n) break;
    if (e > n) e = n;
    jobs[t].fn = fn; jobs[t].ctx = ctx; jobs[t].b = b; jobs[t].e = e;
    if (pthread_create(&th[t], NULL, job_main, &jobs[t]) != 0) { fn(ctx, b, e); jobs[t].fn = NULL; }
    started = t + 1;
  }
  for (int t = 0; t < started; t++)
    if (jobs[t].fn) pthread_join(th[t], NULL);
}

/* ======================================================================== */
/* A. BF16 -> MXFP4 quantize, rowwise 1x32 groups over the flat tensor.      */
/*    per_token_group_quant_4bit_kernel_coalescing,                          */
/*    code/kernel/per_token_quant_mxfp4.cu:121-266                           */
/* ======================================================================== */

/* One float -> E2M1 nibble by the reference's integer RNE path
 * (per_token_quant_mxfp4.cu:213-254). */
ORACLE_API uint8_t oracle_e2m1_from_f32(float q) {
  const uint32_t E8_BIAS = 127, E2_BIAS = 1, lo = E8_BIAS - E2_BIAS;
  uint32_t bits = f32_as_u32(q);
  uint32_t sign = bits & 0x80000000u;
  uint32_t exponent = (bits >> 23) & 0xFFu;
  uint32_t mant = bits & 0x7FFFFFu;
  /* adjust_denormal_opt2 (:103-112) */
  uint32_t shift = E8_BIAS - (exponent + 1u);
  uint32_t denormal_mant = ptx_shr_u32(0x400000u | (mant >> 1), shift);
  uint32_t mask = (uint32_t)(-(int32_t)(exponent < E8_BIAS));
  mant = (denormal_mant & mask) | (mant & ~mask);
  /* exponent rebias (:229-230) */
  exponent = (exponent > lo ? exponent : lo) - lo;
  /* guard / sticky / lsb (:232-241) */
  uint32_t m2 = mant >> 21;
  uint32_t lsb_keep = (m2 >> 1) & 1u;
  uint32_t guard = m2 & 1u;
  uint32_t sticky = (mant & 0x1FFFFFu) != 0u;
  uint32_t round_inc = guard & (sticky | lsb_keep);
  /* COMPUTE_E2M1_DATA + saturate (:30-31, :244-245) */
  uint32_t result = (((exponent << 2) | m2) + round_inc) >> 1;
  uint32_t data = result > 7u ? 7u : result;
  return (uint8_t)(((sign >> 28) | data) & 0x0Fu);
}

/* The scale rule of one group (per_token_quant_mxfp4.cu:185-192), from the
 * group's amax (already max'ed with eps). Returns the E8M0 byte and the
 * float y_s. */
static inline uint8_t scale_rule(float amax, float fp4_max, float* y_s_out) {
  float y_s = amax / fp4_max;
  y_s = exp2f(ceilf(log2f(fmaxf(y_s, 1e-10f))));
  uint32_t q = (uint32_t)cvt_rzi_s32(log2f(y_s)) + 127u; /* add.s32 wraps */
  *y_s_out = y_s;
  return (uint8_t)(q & 0xFFu);
}

ORACLE_API uint8_t oracle_e8m0_scale_from_amax(float amax, float fp4_max) {
  float y;
  return scale_rule(amax, fp4_max, &y);
}

typedef struct {
  const uint16_t* x; uint8_t* q; uint8_t* s;
  float eps, fmin, fmax;
} quant_ctx;

static void quant_range(void* p, int64_t g0, int64_t g1) {
  const quant_ctx* c = (const quant_ctx*)p;
  for (int64_t g = g0; g < g1; g++) {
    const uint16_t* in = c->x + g * 32;
    /* amax over the 32 elements, seeded with eps; the reference's fmaxf drops
       every NaN, signalling ones included (:151,170-178). glibc's fmaxf returns
       a quiet NaN when an operand is signalling, which would restart the
       maximum after an sNaN, so the NaN test is a comparison here. */
    float amax = c->eps;
    for (int j = 0; j < 32; j++) {
      const float a = fabsf(bf16_to_f32(in[j]));
      if (a > amax) amax = a;
    }
    float y_s;
    c->s[g] = scale_rule(amax, c->fmax, &y_s);
    const float inv_y_s = 1.0f / y_s; /* :200 */
    for (int j = 0; j < 32; j += 2) {
      float qx = fminf(fmaxf(bf16_to_f32(in[j]) * inv_y_s, c->fmin), c->fmax);
      float qy = fminf(fmaxf(bf16_to_f32(in[j + 1]) * inv_y_s, c->fmin), c->fmax);
      uint8_t lo = oracle_e2m1_from_f32(qx), hi = oracle_e2m1_from_f32(qy);
      c->q[g * 16 + j / 2] = (uint8_t)((lo & 0x0F) | ((hi & 0x0F) << 4)); /* :256-262 */
    }
  }
}

/* x: numel bf16 values (numel % 32 == 0); codes: numel/2 bytes;
 * scales: numel/32 bytes, flat group order (per_token_quant_mxfp4.cu:161). */
ORACLE_API int oracle_quant_mxfp4(const uint16_t* x, int64_t numel, float eps, float fp4_min,
                                  float fp4_max, uint8_t* codes, uint8_t* scales, int nthreads) {
  if (numel < 0 || numel % 32 != 0) return -1;
  quant_ctx c = {x, codes, scales, eps, fp4_min, fp4_max};
  parallel_for(numel / 32, nthreads, quant_range, &c);
  return 0;
}

/* ======================================================================== */
/* B. MXFP4 -> BF16 dequant, flat.                                           */
/*    omo_per_token_Mxfp4ToBf16_dequant_kernel,                              */
/*    code/kernel/per_token_Mxfp4ToBf16_dequant.cu:70-160                    */
/* ======================================================================== */
typedef struct { const uint8_t* q; const uint8_t* s; uint16_t* out; } deq_ctx;

static void deq_range(void* p, int64_t b0, int64_t b1) {
  const deq_ctx* c = (const deq_ctx*)p;
  for (int64_t b = b0; b < b1; b++) {
    /* thread T covers bytes [8T, 8T+8) and reads scale T/2 == byte/16 (:128-129) */
    uint8_t sb = c->s[b / 16];
    float scale_val = bf16_to_f32((uint16_t)((uint16_t)sb << 7)); /* :22-29, :131-132 */
    uint8_t v = c->q[b];
    float f0 = bf16_to_f32(e2m1_to_bf16_bits(v & 0x0F)) * scale_val;
    float f1 = bf16_to_f32(e2m1_to_bf16_bits(v >> 4)) * scale_val;
    c->out[2 * b] = f32_to_bf16_rne(f0); /* :152-156 */
    c->out[2 * b + 1] = f32_to_bf16_rne(f1);
  }
}

/* codes: nbytes bytes (the host requires nbytes % 128 == 0, :179-182);
 * scales: nbytes/16 bytes; out: 2*nbytes bf16. */
ORACLE_API int oracle_dequant_bf16(const uint8_t* codes, const uint8_t* scales, int64_t nbytes,
                                   uint16_t* out, int nthreads) {
  if (nbytes < 0 || nbytes % 128 != 0) return -1;
  deq_ctx c = {codes, scales, out};
  parallel_for(nbytes, nthreads, deq_range, &c);
  return 0;
}

/* ======================================================================== */
/* C. MXFP4 -> FP8 E4M3 rowwise requant, 1x128 power-of-two scales stored   */
/*    transposed [K/64, M].                                                  */
/*    omo_per_token_Mxfp4ToFp8_kernel, code/kernel/per_token_Mxfp4ToFp8.cu:92-235 */
/* ======================================================================== */
typedef struct { const uint8_t* q; const uint8_t* s; uint8_t* out; float* outs; int64_t M, Kb; } r8_ctx;

static void r8_range(void* p, int64_t g0, int64_t g1) {
  const r8_ctx* c = (const r8_ctx*)p;
  const int64_t gpr = c->Kb / 64; /* 128-element groups per row */
  for (int64_t G = g0; G < g1; G++) {
    /* uint8 max of the group's 4 block scales (:159-165) */
    uint8_t smax = 0;
    for (int k = 0; k < 4; k++) { uint8_t v = c->s[4 * G + k]; if (v > smax) smax = v; }
    uint16_t g16 = (uint16_t)((int)smax - 6);
    float y_s = u32_as_f32((uint32_t)(uint8_t)g16 << 23); /* scale_to_float(uint8) :78-83,172 */
    int64_t row = G / gpr, col = G % gpr;
    c->outs[col * c->M + row] = y_s; /* :175-180 */
    for (int t = 0; t < 8; t++) {        /* 8 threads per group */
      uint8_t s_i = c->s[4 * G + t / 2]; /* scale_in[threadIdx.x/2] */
      uint16_t scale_adjust = (uint16_t)((int)g16 - (int)s_i);     /* :166 */
      uint16_t offset = (uint16_t)((int)scale_adjust << 7);       /* :217 */
      for (int j = 0; j < 8; j++) {
        int64_t byte = G * 64 + t * 8 + j;
        uint8_t v = c->q[byte];
        uint16_t x0 = e2m1_to_bf16_bits(v & 0x0F), x1 = e2m1_to_bf16_bits(v >> 4);
        uint16_t a0 = (uint16_t)((int)x0 - (int)offset), a1 = (uint16_t)((int)x1 - (int)offset);
        float q0 = fmaxf(-448.0f, fminf(448.0f, bf16_to_f32(a0))); /* :223-224 */
        float q1 = fmaxf(-448.0f, fminf(448.0f, bf16_to_f32(a1)));
        c->out[2 * byte] = f32_to_e4m3_rne_sat(q0);
        c->out[2 * byte + 1] = f32_to_e4m3_rne_sat(q1);
      }
    }
  }
}

/* codes [M, Kb] (Kb % 64 == 0), scales [M, Kb/16]; out fp8 [M, 2Kb];
 * outs fp32 [Kb/64, M]. */
ORACLE_API int oracle_mxfp4_to_fp8(const uint8_t* codes, const uint8_t* scales, int64_t M, int64_t Kb,
                                   uint8_t* out, float* outs, int nthreads) {
  if (M < 0 || Kb <= 0 || Kb % 64 != 0) return -1;
  r8_ctx c = {codes, scales, out, outs, M, Kb};
  parallel_for(M * Kb / 64, nthreads, r8_range, &c);
  return 0;
}

/* ======================================================================== */
/* D. MXFP4 rowwise -> FP8 transposed [2Kb, M], scales [M/128, 2Kb] with the */
/*    sign dropped. omo_per_token_Mxfp4ToFp8_col_kernel,                     */
/*    code/kernel/per_token_Mxfp4ToFp8_col.cu:110-301                        */
/* ======================================================================== */
typedef struct { const uint8_t* q; const uint8_t* s; uint8_t* out; float* outs; int64_t M, Kb; uint8_t eps8; } c8_ctx;

static void c8_range(void* p, int64_t t0, int64_t t1) {
  const c8_ctx* c = (const c8_ctx*)p;
  const int64_t tx = c->Kb / 128, M = c->M, Kb = c->Kb, sstride = Kb * 2 / 32;
  uint8_t g[8], adj[128][8];
  for (int64_t t = t0; t < t1; t++) {
    int64_t by = t / tx, bx = t % tx;
    for (int cc = 0; cc < 8; cc++) {
      uint8_t mx = c->eps8; /* `uint8_t local_absmax = eps` (:141) */
      for (int r = 0; r < 128; r++) {
        uint8_t v = c->s[(by * 128 + r) * sstride + bx * 8 + cc]; /* :176-177 */
        if (v > mx) mx = v;
      }
      g[cc] = (uint8_t)(mx - 6); /* :195 */
      float y_s = u32_as_f32((uint32_t)g[cc] << 23);
      for (int lane = 0; lane < 32; lane++)
        c->outs[by * (Kb * 2) + bx * 256 + lane + cc * 32] = y_s; /* :210-212 */
      for (int r = 0; r < 128; r++)
        adj[r][cc] = (uint8_t)(g[cc] - c->s[(by * 128 + r) * sstride + bx * 8 + cc]); /* :218 */
    }
    for (int r = 0; r < 128; r++) {
      for (int bc = 0; bc < 128; bc++) {
        uint8_t v = c->q[(by * 128 + r) * Kb + bx * 128 + bc];
        uint8_t sc = adj[r][bc / 16]; /* :241 */
        uint16_t x0 = e2m1_to_bf16_bits(v & 0x0F), x1 = e2m1_to_bf16_bits(v >> 4);
        uint16_t a0 = (uint16_t)((int)x0 - ((int)sc << 7)); /* :270-271 */
        uint16_t a1 = (uint16_t)((int)x1 - ((int)sc << 7));
        a0 &= 0x7FFF; a1 &= 0x7FFF; /* sign dropped (:273-274) */
        float q0 = fminf(fmaxf(bf16_to_f32(a0), -448.0f), 448.0f); /* :279-280 */
        float q1 = fminf(fmaxf(bf16_to_f32(a1), -448.0f), 448.0f);
        int64_t col = by * 128 + r, rowb = bx * 256 + bc * 2; /* :282-287 */
        c->out[rowb * M + col] = f32_to_e4m3_rne_sat(q0);
        c->out[(rowb + 1) * M + col] = f32_to_e4m3_rne_sat(q1);
      }
    }
  }
}

/* codes [M, Kb] with M % 128 == 0 and Kb % 128 == 0 (the reference kernel
 * has no bounds checks, :166); scales [M, Kb/16]; out [2Kb, M]; outs [M/128, 2Kb]. */
ORACLE_API int oracle_mxfp4_to_fp8_col(const uint8_t* codes, const uint8_t* scales, int64_t M, int64_t Kb,
                                       float eps, uint8_t* out, float* outs, int nthreads) {
  if (M < 0 || M % 128 != 0 || Kb <= 0 || Kb % 128 != 0) return -1;
  c8_ctx c = {codes, scales, out, outs, M, Kb, cvt_rzi_u8(eps)};
  parallel_for((M / 128) * (Kb / 128), nthreads, c8_range, &c);
  return 0;
}

/* ======================================================================== */
/* E/F. MXFP4 rowwise -> fp32 -> FP8 columnwise (TE GEMM_READY), dense and   */
/*      per-split. The dense kernel's missing barrier                         */
/*      (per_token_Mxfp4RowToBf16ToFp8Col.cu:126 -> :131) is restated with   */
/*      the barrier, i.e. the amax sees every dequantized value of the tile. */
/* ======================================================================== */

/* Fill the 128x128 fp32 tile v[col][row] as the load phase of both kernels
 * does (dense :70-128, msplit :95-147). rows_valid counts tile rows that
 * exist; row0 is the first global row. */
static void load_tile(const uint8_t* codes, const uint8_t* scales, int64_t N, int64_t row0,
                      int rows_valid, int64_t col0, float v[128][129]) {
  for (int t = 0; t < 1024; t++) {
    int local_row = t * 16 / 128, lc0 = (t * 16) % 128;
    int64_t grow = row0 + local_row, gcol = col0 + lc0;
    int in_bounds = (local_row < rows_valid) && (gcol < N);
    float dscale = 1.0f;
    int64_t byte_off = 0;
    if (in_bounds) {
      byte_off = grow * (N / 2) + gcol / 2;
      uint8_t su = scales[grow * (N / 32) + gcol / 32]; /* dense :91-93, msplit :115-117 */
      dscale = bf16_to_f32((uint16_t)((uint16_t)su << 7));
    }
    for (int i = 0; i < 16; i++) {
      int lc = lc0 + i;
      if (!in_bounds || gcol + i >= N) { v[lc][local_row] = 0.0f; continue; }
      uint8_t packed = codes[byte_off + i / 2];
      uint8_t nib = (i % 2 == 0) ? (packed & 0x0F) : (packed >> 4);
      v[lc][local_row] = bf16_to_f32(e2m1_to_bf16_bits(nib)) * dscale;
    }
  }
}

typedef struct { const uint8_t* q; const uint8_t* s; uint8_t* out; float* outs; int64_t M, N; float eps; } rc_ctx;

static void rc_range(void* p, int64_t t0, int64_t t1) {
  const rc_ctx* c = (const rc_ctx*)p;
  const int64_t tn = (c->N + 127) / 128, M = c->M, N = c->N;
  float(*v)[129] = (float(*)[129])malloc(sizeof(float) * 128 * 129);
  for (int64_t t = t0; t < t1; t++) {
    int64_t bm = t / tn, bn = t % tn;
    int64_t row0 = bm * 128, col0 = bn * 128;
    int rows_valid = (int)((M - row0) < 128 ? (M - row0) : 128);
    load_tile(c->q, c->s, N, row0, rows_valid, col0, v);
    for (int lc = 0; lc < 128; lc++) {
      float amax = c->eps; /* :132-137 */
      for (int r = 0; r < 128; r++) amax = fmaxf(amax, fabsf(v[lc][r]));
      int64_t gcol = col0 + lc;
      if (gcol >= N) continue;
      c->outs[bm * N + gcol] = amax / 448.0f; /* :142 */
      float qs = (amax > 1e-9f) ? (448.0f / amax) : 0.0f; /* :161 */
      for (int r = 0; r < rows_valid; r++) {
        float qv = v[lc][r] * qs;
        qv = fminf(fmaxf(qv, -448.0f), 448.0f); /* :173-174 */
        c->out[gcol * M + row0 + r] = f32_to_e4m3_rne_sat(qv); /* :181-195 */
      }
    }
  }
  free(v);
}

/* codes [M, N/2], scales with row stride N/32 (as the kernel indexes,
 * :91-92); out fp8 [N, M]; outs fp32 [ceil(M/128), N]. */
ORACLE_API int oracle_row_to_fp8_col(const uint8_t* codes, const uint8_t* scales, int64_t M, int64_t N,
                                     float eps, uint8_t* out, float* outs, int nthreads) {
  if (M < 0 || N < 0 || N % 2 != 0) return -1;
  rc_ctx c = {codes, scales, out, outs, M, N, eps};
  parallel_for(((M + 127) / 128) * ((N + 127) / 128), nthreads, rc_range, &c);
  return 0;
}

/* compute_te_pow2_scale (per_token_Mxfp4RowToBf16ToFp8Col_msplit.cu:23-43),
 * with FP8_E4M3_MAX = 448 (the constant comes from a header the reference
 * does not ship). Returns the quantization multiplier 1/2^k. */
ORACLE_API float oracle_te_pow2_scale(float amax, float eps) {
  if (amax <= eps) return 1.0f;
  float raw = amax / 448.0f;
  uint32_t sb = f32_as_u32(raw);
  uint32_t e = (sb >> 23) & 0xFFu;
  if ((sb & 0x7FFFFFu) != 0) e += 1;
  float div = u32_as_f32(e << 23);
  return (float)(1.0 / (double)div); /* `1.0 / aligned_divisor` is a double division */
}

typedef struct {
  const uint8_t* q; const uint8_t* s; uint8_t* out; float* outs; int64_t N;
  const int32_t* lens; const int32_t* offs; const int32_t* soffs; int64_t ybl, tn; float eps;
} ms_ctx;

static void ms_range(void* p, int64_t t0, int64_t t1) {
  const ms_ctx* c = (const ms_ctx*)p;
  const int64_t N = c->N;
  float(*v)[129] = (float(*)[129])malloc(sizeof(float) * 128 * 129);
  for (int64_t t = t0; t < t1; t++) {
    int64_t split = t / (c->ybl * c->tn), rem = t % (c->ybl * c->tn);
    int64_t bm = rem / c->tn, bn = rem % c->tn;
    int64_t len = c->lens[split];
    if (bm * 128 >= len) continue; /* early exit :76-77 */
    int64_t start = c->offs[split], sstart = c->soffs[split];
    int64_t row0 = start + bm * 128, col0 = bn * 128;
    int rows_valid = (int)((len - bm * 128) < 128 ? (len - bm * 128) : 128);
    load_tile(c->q, c->s, N, row0, rows_valid, col0, v);
    for (int lc = 0; lc < 128; lc++) {
      float amax = 0.0f; /* :152-158 */
      for (int r = 0; r < 128; r++) amax = fmaxf(amax, fabsf(v[lc][r]));
      float sc = oracle_te_pow2_scale(amax, c->eps);
      int64_t gcol = col0 + lc;
      if (gcol >= N) continue;
      c->outs[(sstart + bm) * N + gcol] = 1.0f / sc; /* :165-169 */
      for (int r = 0; r < rows_valid; r++) {
        float qv = v[lc][r] * sc;
        qv = fminf(fmaxf(qv, -448.0f), 448.0f); /* :191-194 */
        c->out[start * N + gcol * len + bm * 128 + r] = f32_to_e4m3_rne_sat(qv); /* :199-221 */
      }
    }
  }
  free(v);
}

/* codes [total_M, N/2]; scales row stride N/32; per split i: rows
 * [offs[i], offs[i]+lens[i]) -> out block [N, lens[i]] at offs[i]*N, scales
 * rows soffs[i] .. + ceil(lens[i]/128). The grid covers ceil(max_split_len/128)
 * row tiles per split (:256). */
ORACLE_API int oracle_row_to_fp8_col_msplit(const uint8_t* codes, const uint8_t* scales, int64_t N,
                                            const int32_t* lens, const int32_t* offs, const int32_t* soffs,
                                            int64_t nsplits, int64_t max_split_len, float eps,
                                            uint8_t* out, float* outs, int nthreads) {
  if (N < 0 || N % 2 != 0 || nsplits < 0 || max_split_len < 0) return -1;
  int64_t ybl = (max_split_len + 127) / 128, tn = (N + 127) / 128;
  ms_ctx c = {codes, scales, out, outs, N, lens, offs, soffs, ybl, tn, eps};
  parallel_for(nsplits * ybl * tn, nthreads, ms_range, &c);
  return 0;
}

/* Scalar helpers exported for the pinning tests. */
ORACLE_API uint8_t oracle_f32_to_e4m3(float f) { return f32_to_e4m3_rne_sat(f); }
ORACLE_API uint16_t oracle_f32_to_bf16(float f) { return f32_to_bf16_rne(f); }
ORACLE_API uint16_t oracle_e2m1_to_bf16_bits(uint8_t nib) { return e2m1_to_bf16_bits(nib); }
