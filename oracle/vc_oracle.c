/*
 * CPU restatement of the sageattn_vc numerical contract.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker for the HIP kernels in
 * cake-opt-vc_attention_amd/csrc. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it; the product never does.
 *
 * Every function cites the reference file:line whose arithmetic it restates
 * (paths relative to the reference repository root; "sal/" abbreviates
 * third_party/sageattention_local/). Where the reference's own arithmetic is
 * order-dependent or not IEEE (fast-math division, warp-tree float sums,
 * Triton's lowered division), this file fixes one deterministic definition
 * that the HIP kernels implement identically:
 *   - every division is IEEE binary32 RN;
 *   - every sum that feeds a payload byte is an fp64 sum in a fixed order
 *     ("tile tree" below, or sequential where stated);
 *   - every FMA is a single-rounding fmaf/fma.
 * Build with -ffp-contract=off so the compiler cannot fuse a*b+c by itself.
 */
#include <math.h>
#include <quadmath.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define VCO_EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------ */
/* Scalar formats                                                     */
/* ------------------------------------------------------------------ */

static inline float u32_as_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_as_u32(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

VCO_EXPORT float vco_bf16_to_f32(uint16_t x) { return u32_as_f32((uint32_t)x << 16); }

/* IEEE RN-even float -> bfloat16 (NaN kept quiet). */
VCO_EXPORT uint16_t vco_f32_to_bf16(float f) {
  uint32_t u = f32_as_u32(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  uint32_t r = u + 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(r >> 16);
}

VCO_EXPORT float vco_f16_to_f32(uint16_t h) {
  uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0) {
    /* zero or subnormal: m * 2^-24, exact in float */
    float v = (float)m * 5.9604644775390625e-08f;
    return s ? -v : v;
  }
  if (e == 31) return u32_as_f32(s | 0x7f800000u | (m << 13));
  return u32_as_f32(s | ((e + 112u) << 23) | (m << 13));
}

/* IEEE RN-even float -> binary16 with overflow to inf. */
VCO_EXPORT uint16_t vco_f32_to_f16(float f) {
  uint32_t u = f32_as_u32(f);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  float a = fabsf(f);
  if (a != a) return (uint16_t)(sign | 0x7e00u);
  if (a >= 65520.0f) return (uint16_t)(sign | 0x7c00u); /* rounds to inf */
  if (a < 6.103515625e-05f) {
    /* subnormal range: quantum 2^-24; a*2^24 is exact, rint is RN-even */
    float q = rintf(a * 16777216.0f);
    return (uint16_t)(sign | (uint16_t)q);
  }
  int e;
  (void)frexpf(a, &e);            /* a in [2^(e-1), 2^e) */
  int E = e - 1;                  /* unbiased exponent */
  float q = rintf(ldexpf(a, 10 - E)); /* mantissa with hidden bit in [1024, 2048] */
  uint32_t mq = (uint32_t)q;
  if (mq == 2048u) { mq = 1024u; E += 1; }
  return (uint16_t)(sign | (uint16_t)((uint32_t)(E + 15) << 10) | (uint16_t)(mq - 1024u));
}

/* OCP E4M3 (float8_e4m3fn) decode. */
VCO_EXPORT float vco_e4m3_decode(uint8_t c) {
  float sign = (c & 0x80u) ? -1.0f : 1.0f;
  uint32_t e = (c >> 3) & 15u, m = c & 7u;
  if ((c & 0x7fu) == 0x7fu) return u32_as_f32(0x7fc00000u);
  if (e == 0) return sign * (float)m * 0.001953125f;       /* m * 2^-9 */
  return sign * ldexpf((float)(8u + m), (int)e - 10);      /* (1+m/8) * 2^(e-7) */
}

/* OCP E4M3 encode: round to nearest even, saturate finite (|x| > 448 -> 448).
 * Sign is preserved, including for results that round to zero.
 * Reference behaviour: cvt.rn.satfinite.e4m3x2.f32 (sal/csrc/numeric_conversion.cuh:53-54)
 * and __nv_cvt_float_to_fp8(..., __NV_SATFINITE, __NV_E4M3) (sal/csrc/vc/preprocess.cu:55).
 * The encoding itself follows the OCP 8-bit floating point specification. */
VCO_EXPORT uint8_t vco_e4m3_encode(float x) {
  uint8_t sign = (f32_as_u32(x) >> 24) & 0x80u;
  float a = fabsf(x);
  if (a != a) return (uint8_t)(sign | 0x7fu);
  if (a >= 448.0f) return (uint8_t)(sign | 0x7eu);
  if (a < 0.015625f) {                      /* below 2^-6: subnormal quantum 2^-9 */
    float q = rintf(a * 512.0f);            /* exact scaling, RN-even */
    return (uint8_t)(sign | (uint8_t)q);    /* q == 8 is the smallest normal, code 8 */
  }
  int e;
  (void)frexpf(a, &e);
  int E = e - 1;                            /* a in [2^E, 2^(E+1)) */
  float q = rintf(ldexpf(a, 3 - E));        /* in [8, 16] */
  uint32_t mq = (uint32_t)q;
  if (mq == 16u) { mq = 8u; E += 1; }
  uint32_t code = ((uint32_t)(E + 7) << 3) | (mq - 8u);
  if (code > 0x7eu) code = 0x7eu;
  return (uint8_t)(sign | code);
}

/* ExpCast byte: clamp(RNE(fmaf(shifted, 8*log2(e), 119.65)), 0, 120).
 * Reference: vc_expcast_code, sal/csrc/vc/expcast.cuh:6-9; oracle form
 * sal/sageattention_local/vc_reference.py:9-11 and src/vc_attention/core.py:68-76.
 * The constants are the exact fp32 values written in the reference. */
static const float kExpA = 11.541560173034668f;
static const float kExpB = 119.6500015258789f;

VCO_EXPORT uint8_t vco_expcast_code(float shifted) {
  float u = fmaf(shifted, kExpA, kExpB);
  u = fmaxf(0.0f, u);                 /* fmaxf(0, NaN) == 0, as in the reference */
  u = fminf(120.0f, u);
  return (uint8_t)rintf(u);
}

VCO_EXPORT void vco_expcast_codes(const float* x, uint8_t* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = vco_expcast_code(x[i]);
}

VCO_EXPORT void vco_e4m3_encode_array(const float* x, uint8_t* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = vco_e4m3_encode(x[i]);
}

VCO_EXPORT void vco_e4m3_decode_array(const uint8_t* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = vco_e4m3_decode(x[i]);
}

/* Correctly rounded binary32 exp2(x) (round to nearest, ties to even). The binary64 libm
 * value (glibc's exp2 is within 0.51 ulp of binary64, i.e. 2^-52 relative) decides the
 * binary32 rounding unless it lies within 2^-44 (relative) of a binary32 rounding boundary;
 * then exp2 is evaluated again in binary128 (libquadmath, 113-bit significand) and rounded
 * once to binary32. This defines the Sage FP8 control path's probability, whose reference
 * (sal/sageattention_local/vc_reference.py:68-75: torch.exp2 of the binary32 shifted logit,
 * then float8_e4m3fn) names no rounding for exp2. */
VCO_EXPORT float vco_exp2_rn(float x) {
  if (x != x) return x;
  const double y = exp2((double)x);
  const float f = (float)y;
  if (f == INFINITY) return f;
  const double up = 0.5 * ((double)f + (double)nextafterf(f, INFINITY));
  const double dn = 0.5 * ((double)f + (double)nextafterf(f, -INFINITY));
  const double tol = ldexp(y, -44);
  if (fabs(y - up) <= tol || fabs(y - dn) <= tol) return (float)exp2q((__float128)x);
  return f;
}

/* E4M3 byte of the control path's probability p = exp2(x): OCP E4M3 (RN-even, satfinite) of
 * vco_exp2_rn(x) (sal/csrc/qattn/attn_utils.cuh:355-455 with exp_offset; the byte of
 * vc_reference.py:75). */
VCO_EXPORT uint8_t vco_fp8_exp2_code(float x) { return vco_e4m3_encode(vco_exp2_rn(x)); }

VCO_EXPORT void vco_fp8_exp2_codes(const float* x, uint8_t* y, int64_t n) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) y[i] = vco_fp8_exp2_code(x[i]);
}

/* y[i] = vco_fp8_exp2_code(x) for x with the binary32 bits first + i (an exhaustive sweep of
 * a bit range without materializing the inputs). */
VCO_EXPORT void vco_fp8_exp2_sweep(uint32_t first, int64_t n, uint8_t* y) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) y[i] = vco_fp8_exp2_code(u32_as_f32(first + (uint32_t)i));
}

/* Round-to-nearest-even to an unsigned byte with saturation to [0, 255];
 * this is the documented behaviour of the gfx950 instruction the fused kernel
 * uses to produce ExpCast codes (v_cvt_pk_u8_f32). NaN maps to 0. */
VCO_EXPORT void vco_cvt_u8_array(const float* x, uint8_t* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    float u = x[i];
    if (u != u) { y[i] = 0; continue; }
    u = fmaxf(0.0f, fminf(255.0f, u));
    y[i] = (uint8_t)rintf(u);
  }
}

/* ------------------------------------------------------------------ */
/* Input helpers                                                      */
/* ------------------------------------------------------------------ */

/* dtype: 0 = float16, 1 = bfloat16 (the two input dtypes sageattn_vc accepts,
 * sal/sageattention_local/vc.py:132-133). */
static inline float load_in(const uint16_t* p, int dtype) {
  return dtype == 1 ? vco_bf16_to_f32(*p) : vco_f16_to_f32(*p);
}
static inline uint16_t store_in(float f, int dtype) {
  return dtype == 1 ? vco_f32_to_bf16(f) : vco_f32_to_f16(f);
}
/* Round a float to the input dtype and back (exact widening). */
static inline float round_in(float f, int dtype) {
  uint16_t b = store_in(f, dtype);
  return load_in(&b, dtype);
}

/* Fixed fp64 reduction of one 128-token tile of one channel.
 * x[key] for key in 0..127 (missing keys are +0.0). The order is the one the
 * HIP tile kernels use: thread kk (0..15) adds keys kk + 16*i for i = 0..7
 * sequentially from +0.0; then partners kk^1, then kk^2; then the four
 * wave results as (w0 + w1) + (w2 + w3). */
VCO_EXPORT double vco_tile_tree_sum(const double* x) {
  double a[16], b[16], c[16];
  for (int kk = 0; kk < 16; ++kk) {
    double s = 0.0;
    for (int i = 0; i < 8; ++i) s += x[kk + 16 * i];
    a[kk] = s;
  }
  for (int kk = 0; kk < 16; ++kk) b[kk] = a[kk] + a[kk ^ 1];
  for (int kk = 0; kk < 16; ++kk) c[kk] = b[kk] + b[kk ^ 2];
  return (c[0] + c[4]) + (c[8] + c[12]);
}

/* ------------------------------------------------------------------ */
/* Grouping (V cluster reorder)                                       */
/* ------------------------------------------------------------------ */

/* torch.linspace(0, n-1, count) in fp32, truncated to int64, with torch's
 * symmetric formula: first half start + step*i, second half end - step*(count-1-i).
 * Reference: at::linspace(0, n-1, count, fp32).to(kLong), sal/csrc/vc/clustering.cu:150-152. */
VCO_EXPORT void vco_linspace_ids(int64_t n, int count, int64_t* ids) {
  if (count == 1) { ids[0] = 0; return; }
  float start = 0.0f, end = (float)(n - 1);
  float step = (end - start) / (float)(count - 1);
  int half = count / 2;
  for (int i = 0; i < count; ++i) {
    float v;
    if (i < half) { float t = step * (float)i; v = start + t; }
    else { float t = step * (float)(count - 1 - i); v = end - t; }
    ids[i] = (int64_t)v;
  }
}

/* Deterministic Lloyd grouping, per head.
 * Reference policy: sal/csrc/vc/clustering.cu:21-137 and pybind.cpp:6-44
 * (count = min(clusters, n); centers initialised to V[linspace ids]; each
 * iteration assigns every token to the nearest center with ties to the lowest
 * id; all but the last iteration recompute non-empty centers as the mean of
 * their tokens; empty centers keep their value; the result is the stable
 * argsort of the final labels). Distances here are the direct fp64
 * sum_d fma(x_d - c_d, x_d - c_d, acc), sequential over d (the reference uses
 * fp32 |x|^2 + |c|^2 - 2x.c; see the FP64 oracle in
 * tests/test_sage_vc_grouping_cuda.py:8-23). Center sums are fp64: per
 * 128-token tile sequentially over tokens, then sequentially over tiles.
 * Warm start (src/vc_attention/core.py:153-171, the grouping a LayoutCache refresh
 * reruns with its cached centers): centers_in (nullable, [BH][count][D]) replaces the
 * linspace initialisation; centers_next (nullable) receives the same center update
 * applied once more to the final labels, i.e. the centers core.py returns.
 * v: [BH][n][D]; perm [BH][n]; labels [BH][n]; centers [BH][count][D] (the final
 * assignment's centers). */
static void update_centers(const uint16_t* vh, int dtype, int64_t n, int D, int count, const int32_t* lab,
                           float* centers, double* tile_sum, double* total, int64_t* cnt) {
  int64_t tiles = (n + 127) / 128;
  for (int i = 0; i < count * D; ++i) total[i] = 0.0;
  for (int c = 0; c < count; ++c) cnt[c] = 0;
  for (int64_t tile = 0; tile < tiles; ++tile) {
    for (int i = 0; i < count * D; ++i) tile_sum[i] = 0.0;
    int64_t end = (tile + 1) * 128 < n ? (tile + 1) * 128 : n;
    for (int64_t t = tile * 128; t < end; ++t) {
      int c = lab[t];
      cnt[c] += 1;
      for (int d = 0; d < D; ++d) tile_sum[c * D + d] += (double)load_in(vh + t * D + d, dtype);
    }
    for (int i = 0; i < count * D; ++i) total[i] += tile_sum[i];
  }
  for (int c = 0; c < count; ++c)
    if (cnt[c] > 0)
      for (int d = 0; d < D; ++d) centers[c * D + d] = (float)(total[c * D + d] / (double)cnt[c]);
}

VCO_EXPORT int vco_group_values_ex(const uint16_t* v, int dtype, int64_t BH, int64_t n, int D,
                                   int clusters, int iterations, const float* centers_in, int64_t* perm,
                                   int32_t* labels, float* centers_out, float* centers_next) {
  int count = clusters < n ? clusters : (int)n;
  if (count < 1 || count > 256 || iterations < 1) return 1;
  int64_t ids[256];
  vco_linspace_ids(n, count, ids);
  /* heads are independent: one head per OpenMP iteration, buffers per thread */
#pragma omp parallel for schedule(dynamic)
  for (int64_t h = 0; h < BH; ++h) {
    float* centers = (float*)malloc(sizeof(float) * count * D);
    double* tile_sum = (double*)malloc(sizeof(double) * count * D);
    double* total = (double*)malloc(sizeof(double) * count * D);
    int64_t* cnt = (int64_t*)malloc(sizeof(int64_t) * count);
    const uint16_t* vh = v + h * n * D;
    int32_t* lab = labels + h * n;
    for (int c = 0; c < count; ++c)
      for (int d = 0; d < D; ++d)
        centers[c * D + d] = centers_in ? centers_in[(h * count + c) * D + d] : load_in(vh + ids[c] * D + d, dtype);
    for (int it = 0; it < iterations; ++it) {
      for (int64_t t = 0; t < n; ++t) {
        double best = INFINITY;
        int bestc = 0;
        for (int c = 0; c < count; ++c) {
          double acc = 0.0;
          for (int d = 0; d < D; ++d) {
            double diff = (double)load_in(vh + t * D + d, dtype) - (double)centers[c * D + d];
            acc = fma(diff, diff, acc);
          }
          if (acc < best) { best = acc; bestc = c; }
        }
        lab[t] = bestc;
      }
      if (it + 1 < iterations) update_centers(vh, dtype, n, D, count, lab, centers, tile_sum, total, cnt);
    }
    if (centers_out) memcpy(centers_out + h * count * D, centers, sizeof(float) * count * D);
    if (centers_next) {
      update_centers(vh, dtype, n, D, count, lab, centers, tile_sum, total, cnt);
      memcpy(centers_next + h * count * D, centers, sizeof(float) * count * D);
    }
    /* stable counting sort by label */
    int64_t pos = 0;
    for (int c = 0; c < count; ++c)
      for (int64_t t = 0; t < n; ++t)
        if (lab[t] == c) perm[h * n + pos++] = t;
    free(centers); free(tile_sum); free(total); free(cnt);
  }
  return 0;
}

VCO_EXPORT int vco_group_values(const uint16_t* v, int dtype, int64_t BH, int64_t n, int D,
                                int clusters, int iterations, int64_t* perm, int32_t* labels,
                                float* centers_out) {
  return vco_group_values_ex(v, dtype, BH, n, D, clusters, iterations, NULL, perm, labels, centers_out, NULL);
}

/* ------------------------------------------------------------------ */
/* K channel mean (K smoothing)                                       */
/* ------------------------------------------------------------------ */

/* km_d = RN_in(RN_f32(S_d / n)) with S_d the fp64 sum of the (permuted) keys:
 * tile tree per 128-key tile, tiles added sequentially from +0.0.
 * Reference: km = k.mean(dim=2, keepdim=True), sal/sageattention_local/vc.py:158
 * (torch's fp32-accumulated mean; order differs, see header).
 * k: [BH][n][D]; perm (nullable) [BH][n]; km: [BH][D] in the input dtype. */
VCO_EXPORT void vco_k_mean(const uint16_t* k, int dtype, int64_t BH, int64_t n, int D,
                           const int64_t* perm, uint16_t* km) {
  int64_t tiles = (n + 127) / 128;
  /* every (head, channel) mean is independent: threads split them, results unchanged */
#pragma omp parallel for schedule(static) collapse(2)
  for (int64_t h = 0; h < BH; ++h) {
    for (int d = 0; d < D; ++d) {
      double x[128];
      double s = 0.0;
      for (int64_t t = 0; t < tiles; ++t) {
        for (int i = 0; i < 128; ++i) {
          int64_t key = t * 128 + i;
          if (key < n) {
            int64_t src = perm ? perm[h * n + key] : key;
            x[i] = (double)load_in(k + (h * n + src) * D + d, dtype);
          } else {
            x[i] = 0.0;
          }
        }
        s += vco_tile_tree_sum(x);
      }
      km[h * D + d] = store_in((float)(s / (double)n), dtype);
    }
  }
}

/* ------------------------------------------------------------------ */
/* Normalized Sylvester-Hadamard rotation of Q/K rows                 */
/* ------------------------------------------------------------------ */

/* In place on one row of W = 2^p binary32 values: for stride s = 1, 2, 4, ..., W/2 every
 * pair (i, i + s) with bit s of i clear becomes (x_i + x_{i+s}, x_i - x_{i+s}), each RN;
 * then every value is multiplied by norm = RN_f32(1 / sqrt(W)) (computed in binary64).
 * Reference: hadamard, src/vc_attention/core.py:79-92 (stride order, (left+right,
 * left-right)); transform_qk_kernel, csrc/kernels.cu:104-123 and its normalization :402. */
static void hadamard_row(float* x, int W) {
  for (int s = 1; s < W; s <<= 1)
    for (int i = 0; i < W; ++i)
      if (!(i & s)) {
        const float a = x[i], b = x[i + s];
        x[i] = a + b;
        x[i + s] = a - b;
      }
  const float norm = (float)(1.0 / sqrt((double)W));
  for (int i = 0; i < W; ++i) x[i] = x[i] * norm;
}

static int pow2_at_least(int D) {
  int W = 1;
  while (W < D) W <<= 1;
  return W;
}

/* rows x D binary32 values -> rows x W (W the power of two >= D; zero padded). */
VCO_EXPORT void vco_hadamard(const float* x, int64_t rows, int D, float* out) {
  const int W = pow2_at_least(D);
  for (int64_t r = 0; r < rows; ++r) {
    float* y = out + r * W;
    for (int i = 0; i < W; ++i) y[i] = i < D ? x[r * D + i] : 0.0f;
    hadamard_row(y, W);
  }
}

/* Reference preprocess_qk (csrc/bindings.cpp:87-116; core.py:96-107): inputs widened to
 * binary32; k_smooth subtracts the binary32 channel mean of K, km = RN_f32(S/n) with S the
 * binary64 sum over keys, taken per 128-key tile in key order and then over tiles in
 * order; hadamard rotates Q and (centred) K rows (width W = pow2 >= D, else D).
 * dtype: 0 fp16, 1 bf16, 2 fp32 (element type of q and k, contiguous [BH][n][D]).
 * qo [BH][nq][Wq], ko [BH][nk][W]; Q is copied unchanged when hadamard = 0. */
static float load_any(const void* p, int64_t i, int dtype) {
  if (dtype == 2) return ((const float*)p)[i];
  return load_in((const uint16_t*)p + i, dtype);
}

VCO_EXPORT void vco_preprocess_qk(const void* q, const void* k, int dtype, int64_t BH, int64_t nq,
                                  int64_t nk, int D, int k_smooth, int hadamard, float* qo, float* ko) {
  const int W = hadamard ? pow2_at_least(D) : D;
  const int64_t tiles = (nk + 127) / 128;
  float* mean = (float*)calloc((size_t)D, sizeof(float));
  for (int64_t h = 0; h < BH; ++h) {
    if (k_smooth) {
      for (int d = 0; d < D; ++d) {
        double total = 0.0;
        for (int64_t t = 0; t < tiles; ++t) {
          double part = 0.0;
          for (int64_t key = t * 128; key < nk && key < t * 128 + 128; ++key)
            part += (double)load_any(k, (h * nk + key) * D + d, dtype);
          total += part;
        }
        mean[d] = (float)(total / (double)nk);
      }
    }
    for (int64_t r = 0; r < nq; ++r) {
      float* y = qo + (h * nq + r) * W;
      for (int i = 0; i < W; ++i) y[i] = i < D ? load_any(q, (h * nq + r) * D + i, dtype) : 0.0f;
      if (hadamard) hadamard_row(y, W);
    }
    for (int64_t r = 0; r < nk; ++r) {
      float* y = ko + (h * nk + r) * W;
      for (int i = 0; i < W; ++i) {
        float x = i < D ? load_any(k, (h * nk + r) * D + i, dtype) : 0.0f;
        if (k_smooth && i < D) x = x - mean[i];
        y[i] = x;
      }
      if (hadamard) hadamard_row(y, W);
    }
  }
  free(mean);
}

/* ------------------------------------------------------------------ */
/* Sage per-thread INT8 quantizer                                     */
/* ------------------------------------------------------------------ */

/* One quantization group: s = RN(RN(amax/127) + 1e-7f); y = RN(x/s);
 * y = RN(y + (y >= 0 ? 0.5 : -0.5)); q = trunc(y).
 * Reference: sal/sageattention_local/triton/quant_per_thread.py:39-46 (Q)
 * and :85-98 (K); the Triton division is restated as IEEE division. */
static inline float int8_scale(float amax) {
  float s = amax / 127.0f;
  return s + 1e-7f;
}
static inline int8_t int8_code(float x, float s) {
  float y = x / s;
  y = y + (y >= 0.0f ? 0.5f : -0.5f);
  return (int8_t)(int)truncf(y);
}

/* Q: rows {16g+t, 16g+t+8} of each 16-row group share a scale; scale index
 * (row/16)*8 + row%8; qs has ceil(n/64)*32 entries per head (rows past n
 * contribute 0 and groups made only of such rows get scale 1e-7f).
 * Reference: quant_per_thread.py:21-46, launch :180-193 (BLKQ=64, WARPQ=16
 * from sal/sageattention_local/vc.py:159). q: [BH][n][D]; q8 [BH][n][D]. */
static void quant_q_rows(const uint16_t* q, int dtype, int64_t BH, int64_t n, int D, int rotate,
                         int8_t* q8, float* qs) {
  int64_t groups16 = (n + 63) / 64 * 4;
  /* groups are independent: threads split (head, group); each thread has its own rows */
#pragma omp parallel
  {
  float* rows = (float*)malloc(sizeof(float) * 2 * D);
#pragma omp for schedule(static) collapse(2)
  for (int64_t h = 0; h < BH; ++h) {
    for (int64_t g = 0; g < groups16; ++g) {
      for (int t = 0; t < 8; ++t) {
        int64_t r0 = g * 16 + t;
        float amax = 0.0f;
        for (int e = 0; e < 2; ++e) {
          const int64_t r = r0 + 8 * e;
          for (int d = 0; d < D; ++d) rows[e * D + d] = r < n ? load_in(q + (h * n + r) * D + d, dtype) : 0.0f;
          if (rotate) hadamard_row(rows + e * D, D);
          for (int d = 0; d < D; ++d) amax = fmaxf(amax, fabsf(rows[e * D + d]));
        }
        float s = int8_scale(amax);
        qs[h * groups16 * 8 + g * 8 + t] = s;
        for (int e = 0; e < 2; ++e) {
          const int64_t r = r0 + 8 * e;
          if (r < n)
            for (int d = 0; d < D; ++d) q8[(h * n + r) * D + d] = int8_code(rows[e * D + d], s);
        }
      }
    }
  }
  free(rows);
  }
}

VCO_EXPORT void vco_quant_q(const uint16_t* q, int dtype, int64_t BH, int64_t n, int D,
                            int8_t* q8, float* qs) {
  quant_q_rows(q, dtype, BH, n, D, 0, q8, qs);
}

/* The same quantizer on Hadamard-rotated rows: q' = hadamard_row(float(q)) in binary32, not
 * rounded back to the input dtype. No counterpart in the reference's sageattn_vc (the
 * rotation is the gap its H200_INT8.md:99-104 names); the rotation is core.py:79-92's. */
VCO_EXPORT void vco_quant_q_rot(const uint16_t* q, int dtype, int64_t BH, int64_t n, int D,
                                int8_t* q8, float* qs) {
  quant_q_rows(q, dtype, BH, n, D, 1, q8, qs);
}

/* K: after centring k'' = RN_in(RN_f32(k - km)) (vc.py:158 and
 * quant_per_thread.py:158-159), each 128-key tile j has four groups
 * t = (key%8)/2, i.e. keys 128j + 8i + 2t + e; scale index j*4 + t.
 * Reference: quant_per_thread.py:48-98, launch :181,195-202 (BLKK=128, WARPK=128).
 * perm (nullable) gathers keys first (vc.py:155). km (nullable) disables centring. */
static void quant_k_rows(const uint16_t* k, int dtype, int64_t BH, int64_t n, int D,
                         const int64_t* perm, const uint16_t* km, int rotate, int8_t* k8, float* ks) {
  int64_t tiles = (n + 127) / 128;
  /* tiles are independent: threads split (head, tile); each thread has its own buffer */
#pragma omp parallel
  {
  float* buf = (float*)malloc(sizeof(float) * 32 * D);
#pragma omp for schedule(static) collapse(2)
  for (int64_t h = 0; h < BH; ++h) {
    for (int64_t j = 0; j < tiles; ++j) {
      for (int t = 0; t < 4; ++t) {
        float amax = 0.0f;
        for (int i = 0; i < 16; ++i)
          for (int e = 0; e < 2; ++e) {
            int64_t key = 128 * j + 8 * i + 2 * t + e;
            float* row = buf + (i * 2 + e) * D;
            for (int d = 0; d < D; ++d) {
              float x = 0.0f;
              if (key < n) {
                int64_t src = perm ? perm[h * n + key] : key;
                x = load_in(k + (h * n + src) * D + d, dtype);
                if (km) x = round_in(x - load_in(km + h * D + d, dtype), dtype);
              }
              row[d] = x;
            }
            if (rotate) hadamard_row(row, D);
            for (int d = 0; d < D; ++d) amax = fmaxf(amax, fabsf(row[d]));
          }
        float s = int8_scale(amax);
        ks[h * tiles * 4 + j * 4 + t] = s;
        for (int i = 0; i < 16; ++i)
          for (int e = 0; e < 2; ++e) {
            int64_t key = 128 * j + 8 * i + 2 * t + e;
            if (key >= n) continue;
            for (int d = 0; d < D; ++d) k8[(h * n + key) * D + d] = int8_code(buf[(i * 2 + e) * D + d], s);
          }
      }
    }
  }
  free(buf);
  }
}

VCO_EXPORT void vco_quant_k(const uint16_t* k, int dtype, int64_t BH, int64_t n, int D,
                            const int64_t* perm, const uint16_t* km, int8_t* k8, float* ks) {
  quant_k_rows(k, dtype, BH, n, D, perm, km, 0, k8, ks);
}

/* Rotated K: k'' = RN_in(RN_f32(k - km)) as above, then hadamard_row in binary32. */
VCO_EXPORT void vco_quant_k_rot(const uint16_t* k, int dtype, int64_t BH, int64_t n, int D,
                                const int64_t* perm, const uint16_t* km, int8_t* k8, float* ks) {
  quant_k_rows(k, dtype, BH, n, D, perm, km, 1, k8, ks);
}

/* ------------------------------------------------------------------ */
/* FP8 block-scaled Q/K (vc27)                                        */
/* ------------------------------------------------------------------ */

/* K channel mean kept in binary32: km = RN_f32(S / n) with S the fp64 sum of the
 * channel over all keys in the tile-tree order of vco_k_mean. The reference sums in
 * fp32 per 128-key block and then over blocks (sal/csrc/vc/qk_fp8.cu:10-35); its
 * validation accepts any mean within rtol 2e-5 of the fp64 mean
 * (scripts/validate_fp8_qk.py:42), and this definition is that mean rounded once. */
VCO_EXPORT void vco_k_mean_f32(const uint16_t* k, int dtype, int64_t BH, int64_t n, int D,
                               float* km) {
  int64_t tiles = (n + 127) / 128;
#pragma omp parallel for schedule(static) collapse(2)
  for (int64_t h = 0; h < BH; ++h) {
    for (int d = 0; d < D; ++d) {
      double x[128];
      double s = 0.0;
      for (int64_t t = 0; t < tiles; ++t) {
        for (int i = 0; i < 128; ++i) {
          int64_t key = t * 128 + i;
          x[i] = key < n ? (double)load_in(k + (h * n + key) * D + d, dtype) : 0.0;
        }
        s += vco_tile_tree_sum(x);
      }
      km[h * D + d] = (float)(s / (double)n);
    }
  }
}

/* One E4M3 block of `rows` rows x D channels: x' = mean ? RN_f32(x - mean_d) : x;
 * s = max(RN(amax / 448), 1e-12f); code = e4m3_satfinite(RN(x' / s)) with IEEE division.
 * Rows past n are not part of the block. scales [BH][ceil(n/rows)].
 * Reference: quantize_qk_fp8, sal/csrc/vc/qk_fp8.cu:38-74 (Q: rows 64, K: rows 128 and
 * centred); restated by scripts/validate_fp8_qk.py:8-20. */
VCO_EXPORT void vco_quant_fp8_block(const uint16_t* x, int dtype, int64_t BH, int64_t n, int D,
                                    int rows, const float* mean, uint8_t* codes, float* scales) {
  const int64_t blocks = (n + rows - 1) / rows;
#pragma omp parallel for schedule(static) collapse(2)
  for (int64_t h = 0; h < BH; ++h) {
    for (int64_t b = 0; b < blocks; ++b) {
      float amax = 0.0f;
      const int64_t r1 = (b + 1) * rows < n ? (b + 1) * rows : n;
      for (int64_t r = b * rows; r < r1; ++r)
        for (int d = 0; d < D; ++d) {
          float v = load_in(x + (h * n + r) * D + d, dtype);
          if (mean) v = v - mean[h * D + d];
          amax = fmaxf(amax, fabsf(v));
        }
      float s = amax / 448.0f;
      s = fmaxf(s, 1e-12f);
      scales[h * blocks + b] = s;
      for (int64_t r = b * rows; r < r1; ++r)
        for (int d = 0; d < D; ++d) {
          float v = load_in(x + (h * n + r) * D + d, dtype);
          if (mean) v = v - mean[h * D + d];
          codes[(h * n + r) * D + d] = vco_e4m3_encode(v / s);
        }
    }
  }
}

/* ------------------------------------------------------------------ */
/* V quantization                                                     */
/* ------------------------------------------------------------------ */

/* Smoothing off: per channel amax over all tokens; vs = RN(amax/448);
 * r = RN(448/amax); payload = e4m3_sat(RN(x*r)); a zero channel gives vs = 0
 * and zero bytes. Reference: sal/sageattention_local/vc.py:163-166,
 * quant.py:224-293, MeanScaleKernel<64,false> sal/csrc/fused/fused.cu:316-427
 * (restated with IEEE division; zero channels per the zero-safe fix checked in
 * tests/test_fp8_zero_values.py:12-28).
 * Output v8 is LOGICAL: [BH][D][tiles*128], token order, padding zero bytes. */
VCO_EXPORT void vco_quant_v_channel(const uint16_t* v, int dtype, int64_t BH, int64_t n, int D,
                                    const int64_t* perm, uint8_t* v8, float* vs) {
  int64_t npad = (n + 127) / 128 * 128;
#pragma omp parallel for schedule(static) collapse(2)
  for (int64_t h = 0; h < BH; ++h) {
    for (int d = 0; d < D; ++d) {
      float amax = 0.0f;
      for (int64_t t = 0; t < n; ++t) {
        int64_t src = perm ? perm[h * n + t] : t;
        amax = fmaxf(amax, fabsf(load_in(v + (h * n + src) * D + d, dtype)));
      }
      uint8_t* out = v8 + (h * D + d) * npad;
      if (amax == 0.0f) {
        vs[h * D + d] = 0.0f;
        memset(out, 0, (size_t)npad);
        continue;
      }
      vs[h * D + d] = amax / 448.0f;
      float r = 448.0f / amax;
      for (int64_t t = 0; t < npad; ++t) {
        if (t < n) {
          int64_t src = perm ? perm[h * n + t] : t;
          out[t] = vco_e4m3_encode(load_in(v + (h * n + src) * D + d, dtype) * r);
        } else {
          out[t] = 0;
        }
      }
    }
  }
}

/* Smoothing on: per (tile, channel) mean_t = RN_f32(S/count) with S the tile
 * tree fp64 sum; residual r = RN(x - mean_t); peak_t = max |r|.
 * channel_scale=1: vs_d = max(P > 0 ? RN(P/448) : 1, RN(M/65504)) with
 *   P = max_t peak_t, M = max_t |mean_t|; vs [BH][D].
 * channel_scale=0: per (tile, channel) scale_t = max(peak_t > 0 ? RN(peak_t/448) : 1,
 *   RN(|mean_t|/65504)); vs [BH][tiles][D].
 * means[t][d] = RN_f16(RN(mean_t / scale)); payload = e4m3_sat(RN(r / scale));
 * padded tokens get zero bytes.
 * Reference: value_stats / value_channel_scales / value_channel_quantize,
 * sal/csrc/vc/preprocess.cu:67-135 (channel) and value_blocks :24-57 (block).
 * Output v8 is LOGICAL [BH][D][tiles*128]; means [BH][tiles][D] binary16 bits. */
VCO_EXPORT void vco_quant_v_smooth(const uint16_t* v, int dtype, int64_t BH, int64_t n, int D,
                                   const int64_t* perm, int channel_scale, uint8_t* v8, float* vs,
                                   uint16_t* means) {
  int64_t tiles = (n + 127) / 128, npad = tiles * 128;
  /* (head, channel) pairs are independent: threads split them with private buffers */
#pragma omp parallel
  {
  float* mean = (float*)malloc(sizeof(float) * tiles);
  float* peak = (float*)malloc(sizeof(float) * tiles);
  float* xs = (float*)malloc(sizeof(float) * npad);
  double x[128];
#pragma omp for schedule(static) collapse(2)
  for (int64_t h = 0; h < BH; ++h) {
    for (int d = 0; d < D; ++d) {
      for (int64_t t = 0; t < npad; ++t) {
        if (t < n) {
          int64_t src = perm ? perm[h * n + t] : t;
          xs[t] = load_in(v + (h * n + src) * D + d, dtype);
        } else {
          xs[t] = 0.0f;
        }
      }
      float P = 0.0f, M = 0.0f;
      for (int64_t j = 0; j < tiles; ++j) {
        int64_t cnt = n - j * 128 < 128 ? n - j * 128 : 128;
        for (int i = 0; i < 128; ++i) x[i] = (double)xs[j * 128 + i];
        float mu = (float)(vco_tile_tree_sum(x) / (double)cnt);
        float pk = 0.0f;
        for (int64_t i = 0; i < cnt; ++i) pk = fmaxf(pk, fabsf(xs[j * 128 + i] - mu));
        mean[j] = mu;
        peak[j] = pk;
        P = fmaxf(P, pk);
        M = fmaxf(M, fabsf(mu));
      }
      float chan = 0.0f;
      if (channel_scale) {
        chan = P > 0.0f ? P / 448.0f : 1.0f;
        chan = fmaxf(chan, M / 65504.0f);
        vs[h * D + d] = chan;
      }
      for (int64_t j = 0; j < tiles; ++j) {
        float s = chan;
        if (!channel_scale) {
          s = peak[j] > 0.0f ? peak[j] / 448.0f : 1.0f;
          s = fmaxf(s, fabsf(mean[j]) / 65504.0f);
          vs[(h * tiles + j) * D + d] = s;
        }
        means[(h * tiles + j) * D + d] = vco_f32_to_f16(mean[j] / s);
        int64_t cnt = n - j * 128 < 128 ? n - j * 128 : 128;
        uint8_t* out = v8 + (h * D + d) * npad + j * 128;
        for (int64_t i = 0; i < 128; ++i)
          out[i] = i < cnt ? vco_e4m3_encode((xs[j * 128 + i] - mean[j]) / s) : 0;
      }
    }
  }
  free(mean); free(peak); free(xs);
  }
}

/* ------------------------------------------------------------------ */
/* Attention: P bytes (exact) and decoded-payload output (fp64 accumulate) */
/* ------------------------------------------------------------------ */

/* RN-even to an unsigned byte with saturation to [0, 255] (NaN -> 0): the byte
 * conversion of the folded ExpCast encode (sal/csrc/vc/expcast.cuh:37-48,58-66). */
static inline uint8_t cvt_u8_rne(float u) {
  if (u != u) return 0;
  u = fmaxf(0.0f, fminf(255.0f, u));
  return (uint8_t)rintf(u);
}

/* How a (row, key) pair's raw QK score and scales come out of a payload.
 * INT8 (sageattn_vc): exact int32 dot product, qs index (row/16)*8 + row%8 over
 *   ceil(nq/64)*32 entries, ks index tile*4 + (key%8)/2 (sal/csrc/vc/vc_sm90.cu:288-289).
 * FP8 block (vc27, sal/sageattention_local/vc_fp8.py; vc_reference.py:23-24,37-40): the
 *   binary32 rounding of the exact sum of decoded E4M3 products, qs index row/64 over
 *   ceil(nq/64) entries, ks index tile. Rows past nq score 0 (zero Q rows). */
typedef struct {
  const int8_t* q8;
  const int8_t* k8;
  const float* qs;
  const float* ks;
  const float* dec; /* E4M3 decode table (FP8 block) */
  int64_t nq, nk, tiles, qsn;
  int D, fp8;
} qk_view;

static inline qk_view make_qk_view(const int8_t* q8, const int8_t* k8, const float* qs, const float* ks,
                                   int64_t nq, int64_t nk, int D, int fp8, const float* dec) {
  qk_view v = {q8, k8, qs, ks, dec, nq, nk, (nk + 127) / 128, fp8 ? (nq + 63) / 64 : (nq + 63) / 64 * 32, D, fp8};
  return v;
}

static inline float qk_raw(const qk_view* v, int64_t h, int64_t r, int64_t key) {
  if (r >= v->nq) return 0.0f;
  const int8_t* qrow = v->q8 + (h * v->nq + r) * v->D;
  const int8_t* krow = v->k8 + (h * v->nk + key) * v->D;
  if (v->fp8) {
    double acc = 0.0;  /* every product of two E4M3 values and their sum are exact in fp64 */
    for (int d = 0; d < v->D; ++d) acc += (double)v->dec[(uint8_t)qrow[d]] * (double)v->dec[(uint8_t)krow[d]];
    return (float)acc;
  }
  int32_t acc = 0;
  for (int d = 0; d < v->D; ++d) acc += (int32_t)qrow[d] * (int32_t)krow[d];
  return (float)acc;
}

static inline float qk_qscale(const qk_view* v, int64_t h, int64_t r) {
  return v->fp8 ? v->qs[h * v->qsn + r / 64] : v->qs[h * v->qsn + (r / 16) * 8 + r % 8];
}

static inline float qk_kscale(const qk_view* v, int64_t h, int64_t t, int i) {
  return v->fp8 ? v->ks[h * v->tiles + t] : v->ks[h * v->tiles * 4 + t * 4 + (i % 8) / 2];
}

/* Folded ExpCast encode of the reference's default kernel modes (vc12..vc15, "optimized")
 * without block values: sal/csrc/vc/vc_math.cuh:16-111, vc_probability_prepare with
 * FoldAffine. Per 16-row group and tile (one Hopper warp: 16 rows x 4 key groups),
 *   safe = every thread's scale >= FLT_MIN, gain = RN(scale * 8 log2 e) finite and
 *          |m'| <= 128 for every row of the group (m' after this tile's update);
 * a safe group encodes code = sat_u8(RNE(fmaf(base, gain, fmaf(-m', A, B)))), an unsafe
 * one falls back to the unfused code of every row. Rows past nq (zero Q rows in the
 * reference's tile) take part with acc = 0. Returns safe[BH][ceil(nq/16)][tiles] for the
 * groups that hold a requested row (others are left 0). */
static uint8_t* affine_safe_flags(const qk_view* v, int64_t BH, float sm, const int64_t* rows,
                                  int64_t nrows) {
  const int64_t nq = v->nq, nk = v->nk, tiles = v->tiles, groups = (nq + 15) / 16;
  uint8_t* flags = (uint8_t*)calloc((size_t)(BH * groups * tiles), 1);
  uint8_t* wanted = (uint8_t*)calloc((size_t)groups, 1);
  for (int64_t i = 0; i < nrows; ++i) wanted[rows[i] / 16] = 1;
#pragma omp parallel for schedule(dynamic) collapse(2)
  for (int64_t h = 0; h < BH; ++h) {
    for (int64_t g = 0; g < groups; ++g) {
      if (!wanted[g]) continue;
      float m[16];
      for (int r = 0; r < 16; ++r) m[r] = -5000000.0f;
      for (int64_t t = 0; t < tiles; ++t) {
        const int last = t == tiles - 1;
        int ok = 1;
        for (int rr = 0; rr < 16; ++rr) {
          const int64_t r = g * 16 + rr;
          const float qscale = qk_qscale(v, h, r);
          float tmax = -INFINITY;
          for (int gk = 0; gk < 4; ++gk) {
            const float scale = last ? sm : sm * (qscale * qk_kscale(v, h, t, 2 * gk));
            const float gain = scale * kExpA;
            if (!(scale >= 1.1754943508222875e-38f) || !isfinite(gain)) ok = 0;
          }
          for (int i = 0; i < 128; ++i) {
            const int64_t key = t * 128 + i;
            if (key >= nk) continue;
            const float dq = qscale * qk_kscale(v, h, t, i);
            const float f = qk_raw(v, h, r, key);
            const float lg = last ? (f * dq) * sm : f * (sm * dq);
            tmax = fmaxf(tmax, lg);
          }
          m[rr] = fmaxf(m[rr], tmax);
          if (!(fabsf(m[rr]) <= 128.0f)) ok = 0;
        }
        flags[(h * groups + g) * tiles + t] = (uint8_t)ok;
      }
    }
  }
  free(wanted);
  return flags;
}

/* For each selected query row, stream the 128-key tiles in order:
 *   dq = RN(qs_row * ks_group)
 *   tiles before the last: logit = RN(float(acc) * RN(sm * dq))
 *   last tile:             logit = RN(RN(float(acc) * dq) * sm), keys >= nk -> -inf
 *   m' = max(m, max logit) with m0 = -5e6; alpha = expf(m - m')
 *   code = expcast(RN(logit - m')); p = e4m3 decode(code)
 *   mass = sum p; out = out*alpha + p.V (+ mass*mean) ; den = den*alpha + mass
 *   final out/den (* channel V scale).
 * Reference: body sal/csrc/vc/vc_sm90.cu:284-412 (tiles before the last),
 * :414-549 (last tile, masking), :551-612 (epilogue); probability contract
 * sal/csrc/vc/vc_math.cuh:268-384; mean restore :410-474; decoded-payload
 * oracle sal/sageattention_local/vc_reference.py:20-91.
 *
 * expcast = 0 is the upstream Sage FP8 control path instead
 * (sal/sageattention_local/vc_reference.py:31-32,58-66; sal/csrc/vc/vc_sm90.cu:177,284-296;
 * sal/csrc/qattn/attn_utils.cuh:30, update_mdo :355-455 with exp_offset; sal/csrc/vc/vc_math.cuh:358-362):
 *   s2 = RN(sm * RN(log2 e)); base/factor as above with s2 in place of sm
 *   (tiles before the last: base = float(acc), factor = RN(s2 * dq); last tile:
 *   base = RN(float(acc) * dq), factor = s2);
 *   m' = max(m, max_k fmaf(base, factor, -8.807f)); alpha = exp2(m - m')
 *   p = exp2(fmaf(base, factor, -m')) (binary32, correctly rounded: vco_exp2_rn);
 *   P byte = E4M3(p), RN-even;
 *   mass = sum p (unrounded, also in the mean restore); PV uses the decoded P byte.
 * q8 [BH][nq][D]; k8 [BH][nk][D]; v8 LOGICAL [BH][D][tiles*128];
 * qs [BH][ceil(nq/64)*32]; ks [BH][tiles*4];
 * vs: NULL (no scale), [BH][D] (channel) or [BH][tiles][D] (block_scale=1);
 * means: NULL or [BH][tiles][D] binary16 bits;
 * rows [nrows] query indices; out [BH][nrows][D] float;
 * pcodes (nullable) [BH][nrows][tiles*128]. */
static void attention_rows(const int8_t* q8, const int8_t* k8, const uint8_t* v8,
                           const float* qs, const float* ks, const float* vs,
                           const uint16_t* means, int block_scale, int64_t BH, int64_t nq,
                           int64_t nk, int D, float sm, const int64_t* rows, int64_t nrows,
                           float* out, uint8_t* pcodes, int mode, int qk_fp8) {
  const int expcast = mode != 0, affine = mode == 2;
  int64_t tiles = (nk + 127) / 128, npad = tiles * 128;
  float* vdec = (float*)malloc(sizeof(float) * 256);  /* decode table */
  for (int c = 0; c < 256; ++c) vdec[c] = vco_e4m3_decode((uint8_t)c);
  const qk_view view = make_qk_view(q8, k8, qs, ks, nq, nk, D, qk_fp8, vdec);
  const float s = expcast ? sm : sm * 1.4426950408889634f;
  uint8_t* safe = affine ? affine_safe_flags(&view, BH, sm, rows, nrows) : NULL;
#pragma omp parallel for schedule(dynamic) collapse(2)
  for (int64_t h = 0; h < BH; ++h) {
    for (int64_t ri = 0; ri < nrows; ++ri) {
      int64_t r = rows[ri];
      const float qscale = qk_qscale(&view, h, r);
      float m = -5000000.0f;
      double den = 0.0;
      double o[128];
      float logit[128], factor[128], abase[128];
      uint8_t code[128];
      for (int d = 0; d < D; ++d) o[d] = 0.0;
      for (int64_t t = 0; t < tiles; ++t) {
        int last = t == tiles - 1;
        float tmax = -INFINITY;
        for (int i = 0; i < 128; ++i) {
          int64_t key = t * 128 + i;
          if (key >= nk) { logit[i] = -INFINITY; abase[i] = -INFINITY; factor[i] = 1.0f; continue; }
          float dq = qscale * qk_kscale(&view, h, t, i);
          float f = qk_raw(&view, h, r, key);
          float base, fac;
          if (!last) { base = f; fac = s * dq; }
          else { base = f * dq; fac = s; }
          if (expcast) {
            float lg = base * fac;
            logit[i] = lg;
            abase[i] = base;
            factor[i] = fac;
            tmax = fmaxf(tmax, lg);
          } else {
            logit[i] = base;  /* the control path keeps base and factor apart */
            factor[i] = fac;
            tmax = fmaxf(tmax, fmaf(base, fac, -8.807f));
          }
        }
        float mnew = fmaxf(m, tmax);
        float alpha = expcast ? expf(m - mnew) : exp2f(m - mnew);
        m = mnew;
        double mass = 0.0;
        double prod[128];
        for (int d = 0; d < D; ++d) prod[d] = 0.0;
        for (int i = 0; i < 128; ++i) {
          double p;
          if (expcast) {
            if (affine && safe[(h * ((nq + 15) / 16) + r / 16) * tiles + t]) {
              const float gain = factor[i] * kExpA;
              const float bias = fmaf(-mnew, kExpA, kExpB);
              code[i] = cvt_u8_rne(fmaf(abase[i], gain, bias));
            } else {
              float shifted = logit[i] - mnew;
              code[i] = vco_expcast_code(shifted);
            }
            p = (double)vdec[code[i]];
            mass += p;
          } else {
            float e = vco_exp2_rn(fmaf(logit[i], factor[i], -mnew));
            code[i] = vco_e4m3_encode(e);
            p = (double)vdec[code[i]];
            mass += (double)e;
          }
          if (p != 0.0)
            for (int d = 0; d < D; ++d)
              prod[d] += p * (double)vdec[v8[(h * D + d) * npad + t * 128 + i]];
        }
        if (pcodes) memcpy(pcodes + (h * nrows + ri) * npad + t * 128, code, 128);
        for (int d = 0; d < D; ++d) {
          double c = prod[d];
          if (means) {
            c += mass * (double)vco_f16_to_f32(means[(h * tiles + t) * D + d]);
            if (block_scale) c *= (double)vs[(h * tiles + t) * D + d];
          }
          o[d] = o[d] * (double)alpha + c;
        }
        den = den * (double)alpha + mass;
      }
      for (int d = 0; d < D; ++d) {
        double y = o[d] / den;
        if (vs && !block_scale) y *= (double)vs[h * D + d];
        out[(h * nrows + ri) * D + d] = (float)y;
      }
    }
  }
  free(vdec);
  free(safe);
}

VCO_EXPORT void vco_attention(const int8_t* q8, const int8_t* k8, const uint8_t* v8,
                              const float* qs, const float* ks, const float* vs,
                              const uint16_t* means, int block_scale, int64_t BH, int64_t nq,
                              int64_t nk, int D, float sm, const int64_t* rows, int64_t nrows,
                              float* out, uint8_t* pcodes) {
  attention_rows(q8, k8, v8, qs, ks, vs, means, block_scale, BH, nq, nk, D, sm, rows, nrows,
                 out, pcodes, 1, 0);
}

/* The folded ExpCast encode of the reference's default modes without block values. */
VCO_EXPORT void vco_attention_affine(const int8_t* q8, const int8_t* k8, const uint8_t* v8,
                                     const float* qs, const float* ks, const float* vs,
                                     const uint16_t* means, int block_scale, int64_t BH,
                                     int64_t nq, int64_t nk, int D, float sm,
                                     const int64_t* rows, int64_t nrows, float* out,
                                     uint8_t* pcodes) {
  attention_rows(q8, k8, v8, qs, ks, vs, means, block_scale, BH, nq, nk, D, sm, rows, nrows,
                 out, pcodes, 2, 0);
}

/* The Sage FP8 control path (expcast=False); pcodes receives the E4M3 bytes of P. */
VCO_EXPORT void vco_attention_control(const int8_t* q8, const int8_t* k8, const uint8_t* v8,
                                      const float* qs, const float* ks, const float* vs,
                                      const uint16_t* means, int block_scale, int64_t BH,
                                      int64_t nq, int64_t nk, int D, float sm,
                                      const int64_t* rows, int64_t nrows, float* out,
                                      uint8_t* pcodes) {
  attention_rows(q8, k8, v8, qs, ks, vs, means, block_scale, BH, nq, nk, D, sm, rows, nrows,
                 out, pcodes, 0, 0);
}

/* The FP8 block-scaled QK variant (vc27: sal/sageattention_local/vc_fp8.py:12-60,
 * sal/csrc/vc/fp8_dispatch.cuh): q8/k8 hold E4M3 bytes, qs [BH][ceil(nq/64)],
 * ks [BH][tiles]; mode 0 control, 1 unfused ExpCast, 2 folded ExpCast (the reference's
 * FP8 kernel folds the ExpCast encode, fp8_dispatch.cuh:4-9). No block values. */
VCO_EXPORT void vco_attention_fp8(const uint8_t* q8, const uint8_t* k8, const uint8_t* v8,
                                  const float* qs, const float* ks, const float* vs, int64_t BH,
                                  int64_t nq, int64_t nk, int D, float sm, const int64_t* rows,
                                  int64_t nrows, float* out, uint8_t* pcodes, int mode) {
  attention_rows((const int8_t*)q8, (const int8_t*)k8, v8, qs, ks, vs, NULL, 0, BH, nq, nk, D, sm,
                 rows, nrows, out, pcodes, mode, 1);
}
