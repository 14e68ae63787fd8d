/*
 * CPU oracle for the dynamic block-scaled FP8 linear path.  TEST INFRASTRUCTURE ONLY:
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this file's
 * library, as the checker or as the timed CPU baseline; the product path never does.
 *
 * This is a plain-C restatement of the arithmetic that the reference engine runs in its
 * Triton kernels (reference: engine/kernels/sm89_fp8.py).  Each function cites the lines
 * it follows.  Compiled with -ffp-contract=off and without fast-math, so every float
 * operation below is one IEEE-754 binary32 operation with round-to-nearest-even.
 *
 * Pins (tests/test_oracle.py):
 *   f32 -> e4m3fn encode: against torch's float8_e4m3fn cast over ~8.4M fp32 bit patterns
 *     covering every exponent, every rounding midpoint and the subnormal range, plus the
 *     256-code decode table against the OCP definition.
 *   act quant: the reference tests' invariants (zero row -> +0 scales, tiny row -> scale
 *     < 1e-12, -0 row -> code 0x80, +-448 row -> 0x7E/0xFE with scale 1.0, row
 *     independence) and closed-form checks (the group amax element encodes to +-448,
 *     |dequant - x| <= half an e4m3 ulp).
 *   block GEMM: an fp64 dense reference with a rounding-error bound, exact power-of-two
 *     scaling laws on a_s rows and w_s blocks (catch index/transpose mistakes), and a
 *     brute-force pure-Python evaluation on tiny tail shapes.
 */
#include <math.h>
#include <stdlib.h>
#include <stdint.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_GROUP 128

/* ---- number formats ------------------------------------------------------------- */

static inline float bits_to_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* bf16 -> f32 is a 16-bit shift (exact). */
float orc_bf16_to_f32(uint16_t h) { return bits_to_f32((uint32_t)h << 16); }

/* IEEE binary16 -> f32, exact. */
float orc_f16_to_f32(uint16_t h) {
  int s = h >> 15, e = (h >> 10) & 31, m = h & 1023;
  double v;
  if (e == 31) return bits_to_f32((s ? 0x80000000u : 0) | 0x7f800000u | (m ? 0x400000u : 0));
  if (e == 0) v = ldexp((double)m, -24);
  else v = ldexp((double)(1024 + m), e - 25);
  return (float)(s ? -v : v);
}

/* f32 -> bf16, round to nearest even (torch's .to(bfloat16) / Triton's cast). */
uint16_t orc_f32_to_bf16(float f) {
  uint32_t u = f32_to_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40); /* quiet NaN */
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* f32 -> binary16, round to nearest even, overflow to +-inf. */
uint16_t orc_f32_to_f16(float f) {
  uint32_t u = f32_to_bits(f);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  double a = fabs((double)f);
  if (f != f) return 0x7e00;
  if (a == 0.0) return sign;
  if (a < ldexp(1.0, -14)) {                       /* subnormal grid: spacing 2^-24 */
    double q = nearbyint(ldexp(a, 24));            /* exact scaling, RNE */
    return (uint16_t)(sign | (uint16_t)q);          /* q == 1024 is the smallest normal */
  }
  int e;
  double m = frexp(a, &e);                          /* a = m * 2^e, m in [0.5, 1) */
  double q = nearbyint(m * 2048.0);                 /* 11 significant bits, RNE */
  if (q == 2048.0) { q = 1024.0; e += 1; }
  int biased = e - 1 + 15;
  if (biased >= 31) return (uint16_t)(sign | 0x7c00);
  return (uint16_t)(sign | (uint16_t)(biased << 10) | (uint16_t)((int)q - 1024));
}

/* OCP e4m3fn decode: bias 7, 3 mantissa bits, no infinities, 0x7F/0xFF are NaN. */
float orc_e4m3_to_f32(uint8_t c) {
  int s = c >> 7, e = (c >> 3) & 15, m = c & 7;
  double v;
  if (e == 15 && m == 7) return bits_to_f32(0x7fc00000u);
  if (e == 0) v = ldexp((double)m, -9);
  else v = ldexp((double)(8 + m), e - 10);
  return (float)(s ? -v : v);
}

/* f32 -> OCP e4m3fn with round-to-nearest-even and saturation to +-448 (the
 * cvt.rn.satfinite behaviour of the reference's `.to(tl.float8e4nv)`,
 * engine/kernels/sm89_fp8.py:324).  On the quantizer's path |v| <= 448*(1+2^-23),
 * which rounds to 448 without reaching the saturation branch. */
uint8_t orc_f32_to_e4m3(float f) {
  uint32_t u = f32_to_bits(f);
  uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  double a = fabs((double)f);
  if (f != f) return (uint8_t)(sign | 0x7f);
  if (a == 0.0) return sign;
  if (a < ldexp(1.0, -6)) {                         /* subnormal grid: spacing 2^-9 */
    double q = nearbyint(ldexp(a, 9));              /* q == 8 is the smallest normal */
    return (uint8_t)(sign | (uint8_t)q);
  }
  int e;
  double m = frexp(a, &e);
  double q = nearbyint(m * 16.0);                   /* 4 significant bits, RNE */
  if (q == 16.0) { q = 8.0; e += 1; }
  int biased = e - 1 + 7;
  int code = (biased << 3) | ((int)q - 8);
  if (biased > 15 || code > 0x7e) code = 0x7e;      /* satfinite */
  return (uint8_t)(sign | (uint8_t)code);
}

void orc_f32_to_e4m3_array(const float* x, uint8_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_f32_to_e4m3(x[i]);
}

/* ---- a1: per-token 1x128 activation quantizer ------------------------------------ */

/* Follows _quantize_activation_kernel, engine/kernels/sm89_fp8.py:304-332, and the
 * wrapper quantize_sm89_fp8_activation, :401-424:
 *   t = x[m, 128g : 128g+128] as fp32, with the K tail read as 0.0     (:315-317)
 *   s = max(|t|) / 448.0, stored raw (0 for an all-zero group)          (:320)
 *   q = (t / max(s, 1e-12)).to(e4m3fn)                                  (:321-323)
 * x: M x K elements of bf16 (is_fp16 = 0) or fp16 (is_fp16 = 1), element strides
 * (sxm, sxk).  q: M x K bytes, row stride K (:326).  s: M x ceil(K/128) fp32 (:330). */
void orc_act_quant(const uint16_t* x, int is_fp16, int64_t M, int64_t K, int64_t sxm,
                   int64_t sxk, uint8_t* q, float* s) {
  const int64_t G = (K + ORC_GROUP - 1) / ORC_GROUP;
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t g = 0; g < G; ++g) {
      float t[ORC_GROUP];
      float amax = 0.0f;
      for (int j = 0; j < ORC_GROUP; ++j) {
        int64_t k = g * ORC_GROUP + j;
        float v = 0.0f;
        if (k < K) {
          uint16_t h = x[m * sxm + k * sxk];
          v = is_fp16 ? orc_f16_to_f32(h) : orc_bf16_to_f32(h);
        }
        t[j] = v;
        float av = fabsf(v);
        if (av > amax) amax = av;
      }
      float scale = amax / 448.0f;
      float den = scale > 1e-12f ? scale : 1e-12f;
      s[m * G + g] = scale;
      for (int j = 0; j < ORC_GROUP; ++j) {
        int64_t k = g * ORC_GROUP + j;
        if (k < K) q[m * K + k] = orc_f32_to_e4m3(t[j] / den);
      }
    }
  }
}

/* ---- a2: block-scaled FP8 GEMM ------------------------------------------------------ */

/* Follows _fp8_split_gemm_kernel, engine/kernels/sm89_fp8.py:344-398:
 *   acc = 0 (fp32)                                                        (:365)
 *   for kb in increasing order:                                           (:371)
 *     acc += (dot(q[m, kb], W[n, kb]) * a_s[m, kb]) * w_s[n / 128, kb]     (:387-391)
 *   out = acc.to(out dtype)                                               (:394-397)
 * The 128-long dot of e4m3 values is formed exactly in binary64 (each product has at
 * most 8 significant bits and the sum spans < 2^-18 .. 2^25, so no rounding occurs)
 * and rounded once to fp32: the correctly rounded value of the MMA's fp32 result.
 * q: M x K codes, row stride ldq; a_s: element (m, kb) at as[m*as_sm + kb*as_sk];
 * w: N x K codes (K contiguous, the "NT" layout), row stride ldw;
 * w_s: element (nb, kb) at ws[nb*ws_sn + kb*ws_sk];  out: M x N, row stride ldo. */
void orc_block_gemm(const uint8_t* q, int64_t ldq, const float* as, int64_t as_sm,
                    int64_t as_sk, const uint8_t* w, int64_t ldw, const float* ws,
                    int64_t ws_sn, int64_t ws_sk, uint16_t* out, int out_fp16, int64_t ldo,
                    int64_t M, int64_t N, int64_t K, int nthreads) {
  const int64_t G = (K + ORC_GROUP - 1) / ORC_GROUP;
  static float lut[256];
  static int lut_ready = 0;
  if (!lut_ready) {
    for (int c = 0; c < 256; ++c) lut[c] = orc_e4m3_to_f32((uint8_t)c);
    lut_ready = 1;
  }
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(dynamic, 1) collapse(2)
#endif
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n0 = 0; n0 < N; n0 += 64) {
      const int64_t n1 = n0 + 64 < N ? n0 + 64 : N;
      for (int64_t n = n0; n < n1; ++n) {
        float acc = 0.0f;
        for (int64_t g = 0; g < G; ++g) {
          const int64_t k0 = g * ORC_GROUP;
          const int64_t k1 = k0 + ORC_GROUP < K ? k0 + ORC_GROUP : K;
          const uint8_t* qa = q + m * ldq;
          const uint8_t* wb = w + n * ldw;
          double dot = 0.0;
          for (int64_t k = k0; k < k1; ++k) dot += (double)lut[qa[k]] * (double)lut[wb[k]];
          float d = (float)dot;
          float t = d * as[m * as_sm + g * as_sk];
          t = t * ws[(n / ORC_GROUP) * ws_sn + g * ws_sk];
          acc = acc + t;
        }
        out[m * ldo + n] = out_fp16 ? orc_f32_to_f16(acc) : orc_f32_to_bf16(acc);
      }
    }
  }
}

/* a4 (sm89_fp8_linear's split path, engine/kernels/sm89_fp8.py:501-505): quantize the
 * activation, then the block GEMM.  Scratch q (M x K) and s (M x ceil(K/128)) are
 * caller-provided. */
void orc_linear(const uint16_t* x, int is_fp16, int64_t M, int64_t K, int64_t sxm,
                int64_t sxk, const uint8_t* w, const float* ws, int64_t N, uint16_t* out,
                int out_fp16, uint8_t* q_scratch, float* s_scratch, int nthreads) {
  const int64_t G = (K + ORC_GROUP - 1) / ORC_GROUP;
  orc_act_quant(x, is_fp16, M, K, sxm, sxk, q_scratch, s_scratch);
  orc_block_gemm(q_scratch, K, s_scratch, G, 1, w, K, ws, G, 1, out, out_fp16, N, M, N, K,
                 nthreads);
}

/* SiLU(gate) * up in bf16, following the reference's _silu_mul_kernel
 * (engine/kernels/fused.py:127-137): silu = bf16(g / (1 + exp(-g))) in fp32 with an IEEE
 * division, then bf16(silu * u).  exp(-g) is evaluated in binary64 and rounded once to
 * binary32 (the correctly rounded fp32 exp in all but double-rounding corner cases); a GPU's
 * faithfully rounded expf may differ in the last place, so callers compare h within one
 * bf16 ulp and quantize the GPU's own h for the bit-exact code check. */
void orc_silu_mul(const uint16_t* gate, const uint16_t* up, int64_t n, uint16_t* h) {
  for (int64_t i = 0; i < n; ++i) {
    float g = orc_bf16_to_f32(gate[i]);
    float u = orc_bf16_to_f32(up[i]);
    float e = (float)exp(-(double)g);
    float den = 1.0f + e;
    float silu = orc_bf16_to_f32(orc_f32_to_bf16(g / den));
    h[i] = orc_f32_to_bf16(silu * u);
  }
}

/* Threads PyTorch's CUDA reduction assigns to one row of a last-dim fp32 mean over 4-wide
 * vectors (setReduceConfig), as the reference reproduces it in _torch_reduce_block_width
 * (engine/kernels/fused.py:205-214). */
static int64_t orc_last_pow2(int64_t n) {
  int64_t p = 1;
  while (p * 2 <= n) p *= 2;
  return p;
}
int64_t orc_rmsnorm_block_width(int64_t rows, int64_t n_cols) {
  const int64_t max_threads = 512, warp = 32;
  int64_t dim0 = n_cols / 4;
  int64_t dim0_pow2 = dim0 < max_threads ? orc_last_pow2(dim0) : max_threads;
  int64_t dim1_pow2 = rows < max_threads ? orc_last_pow2(rows > 0 ? rows : 1) : max_threads;
  int64_t lim = max_threads / (dim0_pow2 < warp ? dim0_pow2 : warp);
  int64_t height = dim1_pow2 < lim ? dim1_pow2 : lim;
  int64_t cap = max_threads / height;
  return dim0_pow2 < cap ? dim0_pow2 : cap;
}

/* Qwen3 RMSNorm as the reference's _rms_norm_kernel computes it (engine/kernels/fused.py:
 * 89-124, 165-199) for `rows` rows of width n_cols (a multiple of 4):
 *   x   = bf16(x + residual)               with a residual (summed[] receives it)
 *   ss  = rounded squares summed in PyTorch's order: bw = orc_rmsnorm_block_width(rows, K)
 *         threads; thread t runs four accumulators over vectors v = k*bw + t (element 4v+q
 *         into accumulator q), combines ((a0 + a1) + a2) + a3; threads fold s[t] += s[t+h]
 *         for h = bw/2 .. 1
 *   var = ss * fl(1 / K);  inv = 1 / sqrt(var + eps)  (double, rounded once to fp32 -- the
 *         reference uses libdevice's approximate rsqrt here)
 *   y   = bf16(w * bf16(x * inv))
 * x and residual rows are `ld` elements apart; y and summed are dense. */
/* The row's sum of squares in the reference's order (fused.py:95-115, the tree of
 * fused.py:61-75): part[] holds bw floats of scratch. */
static float orc_rms_sumsq(const float* xs, int64_t n_cols, int64_t bw, float* part) {
  const int64_t nvec = n_cols / 4;
  for (int64_t t = 0; t < bw; ++t) {
    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int64_t v = t; v < nvec; v += bw)
      for (int q = 0; q < 4; ++q) {
        float sq = xs[4 * v + q] * xs[4 * v + q];
        a[q] = a[q] + sq;
      }
    part[t] = ((a[0] + a[1]) + a[2]) + a[3];
  }
  for (int64_t h = bw / 2; h >= 1; h /= 2)
    for (int64_t t = 0; t < h; ++t) part[t] = part[t] + part[t + h];
  return part[0];
}

/* Row r's x (bf16(x + residual) with a residual, whose bits go to summed when non-null). */
static void orc_rms_row(const uint16_t* x, const uint16_t* residual, int64_t ld, int64_t r, int64_t n_cols,
                        float* xs, uint16_t* summed) {
  for (int64_t c = 0; c < n_cols; ++c) {
    float v = orc_bf16_to_f32(x[r * ld + c]);
    if (residual) {
      uint16_t sb = orc_f32_to_bf16(v + orc_bf16_to_f32(residual[r * ld + c]));
      if (summed) summed[r * n_cols + c] = sb;
      v = orc_bf16_to_f32(sb);
    }
    xs[c] = v;
  }
}

/* The sums of squares orc_rmsnorm forms, one per row (exposed so that tests can pin the
 * summation order itself). */
void orc_rmsnorm_sumsq(const uint16_t* x, const uint16_t* residual, int64_t ld, int64_t rows, int64_t n_cols,
                       float* out) {
  const int64_t bw = orc_rmsnorm_block_width(rows, n_cols);
  float* part = (float*)malloc((size_t)bw * sizeof(float));
  float* xs = (float*)malloc((size_t)n_cols * sizeof(float));
  for (int64_t r = 0; r < rows; ++r) {
    orc_rms_row(x, residual, ld, r, n_cols, xs, NULL);
    out[r] = orc_rms_sumsq(xs, n_cols, bw, part);
  }
  free(part);
  free(xs);
}

void orc_rmsnorm(const uint16_t* x, const uint16_t* residual, int64_t ld, const uint16_t* w, int64_t rows,
                 int64_t n_cols, float eps, uint16_t* y, uint16_t* summed) {
  const int64_t bw = orc_rmsnorm_block_width(rows, n_cols);
  const float inv_k = 1.0f / (float)n_cols;
  float* part = (float*)malloc((size_t)bw * sizeof(float));
  float* xs = (float*)malloc((size_t)n_cols * sizeof(float));
  for (int64_t r = 0; r < rows; ++r) {
    orc_rms_row(x, residual, ld, r, n_cols, xs, summed);
    float var = orc_rms_sumsq(xs, n_cols, bw, part) * inv_k;
    float inv = (float)(1.0 / sqrt((double)(var + eps)));
    for (int64_t c = 0; c < n_cols; ++c) {
      float normed = orc_bf16_to_f32(orc_f32_to_bf16(xs[c] * inv));
      y[r * n_cols + c] = orc_f32_to_bf16(orc_bf16_to_f32(w[c]) * normed);
    }
  }
  free(part);
  free(xs);
}

int orc_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
