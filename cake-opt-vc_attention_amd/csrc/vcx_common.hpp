// Shared host/device helpers for the gfx950 sageattn_vc kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>

#include "../../include/vcx.h"

namespace vcx {

// ------------------------------------------------------------------ errors

// Per-thread message behind vcx_last_error().
std::string& last_error();
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Record the pending launch error of the last kernel (if any).
int check_launch(const char* what);

#define VCX_REQUIRE(cond, ...)                              \
  do {                                                      \
    if (!(cond)) return ::vcx::fail(VCX_EINVAL, __VA_ARGS__); \
  } while (0)

#define VCX_LAUNCHED(what)                      \
  do {                                          \
    int vcx_rc_ = ::vcx::check_launch(what);    \
    if (vcx_rc_) return vcx_rc_;                \
  } while (0)

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }
inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ------------------------------------------------------------------ layout

constexpr int kTile = 128;  // keys per tile (the reference's CTA_K and V block size)

// Storage position p (0..127) inside a V tile -> token offset. Lane group G = p/32
// of the fused kernel owns byte b = p%32 of its FP8 MFMA operand, which the QK
// accumulator layout fills with key 16*(b/4) + 8*((b/2)%2) + 2*G + b%2.
__host__ __device__ inline int value_token(int p) {
  int G = p >> 5, b = p & 31;
  return 16 * (b >> 2) + 8 * ((b >> 1) & 1) + 2 * G + (b & 1);
}
// Inverse of value_token.
__host__ __device__ inline int value_position(int key) {
  return 32 * ((key & 7) >> 1) + 4 * (key >> 4) + 2 * ((key >> 3) & 1) + (key & 1);
}

// ------------------------------------------------------------------ device formats

__device__ inline float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

__device__ inline float f16_bits_to_f32(uint32_t b) {
  _Float16 h;
  uint16_t s = static_cast<uint16_t>(b);
  __builtin_memcpy(&h, &s, 2);
  return static_cast<float>(h);
}

// IEEE RN-even float -> bfloat16 bits (NaN kept quiet).
__device__ inline uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return ((u >> 16) | 0x40u) & 0xffffu;
  return ((u + 0x7fffu + ((u >> 16) & 1u)) >> 16) & 0xffffu;
}

// IEEE RN-even float -> binary16 bits (v_cvt_f16_f32 under the default RNE mode).
__device__ inline uint32_t f32_to_f16_bits(float f) {
  _Float16 h = static_cast<_Float16>(f);
  uint16_t s;
  __builtin_memcpy(&s, &h, 2);
  return s;
}

template <int DT>
__device__ inline float in_to_f32(uint32_t bits) {
  if constexpr (DT == VCX_BFLOAT16) return bf16_bits_to_f32(bits);
  else return f16_bits_to_f32(bits);
}
template <int DT>
__device__ inline uint32_t f32_to_in(float f) {
  if constexpr (DT == VCX_BFLOAT16) return f32_to_bf16_bits(f);
  else return f32_to_f16_bits(f);
}
template <int DT>
__device__ inline float round_in(float f) { return in_to_f32<DT>(f32_to_in<DT>(f)); }

// OCP E4M3 with saturation: clamp to +-448 then the gfx950 conversion, which
// rounds to nearest even (checked exhaustively on the E4M3 boundaries against
// the CPU oracle by the convert probe).
__device__ inline uint32_t e4m3_sat(float x) {
  float y = fminf(448.0f, fmaxf(-448.0f, x));
  return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(y, 0.0f, 0, false)) & 0xffu;
}

// E4M3 bytes (packed, element 0 in the low byte) of four Sage FP8 control-path probabilities
// p = exp2(x), equal to E4M3_RNE(RN_f32(exp2(x))) with a correctly rounded binary32 exp2.
// On entry p holds the hardware exp2 (v_exp_f32, within one ulp of exp2 on every binary32
// input). The bytes of p - 2 ulps and p + 2 ulps agree unless an E4M3 rounding midpoint lies
// within two ulps of p; only then does the lane recompute exp2 in binary64 and round it once
// to binary32 (p is updated to that value). The upper neighbours of two probabilities come
// from one 64-bit add (v_lshl_add_u64). SAT = true (what the fused kernel uses) forms the
// lower neighbours with a saturating subtraction per probability. SAT = false uses one 64-bit
// subtraction per pair, half the instructions, but a borrow out of a low half below 2 ulps (p
// = 0 or the smallest subnormal, i.e. x below about -149) then yields a NaN byte and a
// needless recheck: bytes stay right, but rows whose scores lie more than about 103 nats
// below the row maximum recheck on most tiles. Same-box A/B of the control path: SAT costs
// 5.8 % (D128) and 11 % (D64) on N(0,1) scores and is 4-5 times faster with Q scaled by 25.
// Reference: the probability byte of sal/sageattention_local/vc_reference.py:68-75 and
// sal/csrc/qattn/attn_utils.cuh:355-455.
// fp8_exp2_bounds gives the bytes of both neighbour sets (lo, hi); fp8_exp2_word resolves a
// disagreement. Binary64 exp2 rounded once to binary32: one out-of-line copy for the rare
// recheck.
__device__ __noinline__ inline float exp2_via_f64(float x) { return static_cast<float>(exp2(static_cast<double>(x))); }

template <bool SAT = false, bool REUSE = false>
__device__ inline void fp8_exp2_bounds(const float (&p)[4], uint32_t& lo, uint32_t& hi) {
  constexpr uint64_t kTwoUlps = 0x0000000200000002ull;
  float dn[4], up[4];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint64_t pr = (static_cast<uint64_t>(__float_as_uint(p[2 * h + 1])) << 32) | __float_as_uint(p[2 * h]);
    const uint64_t u = pr + kTwoUlps;
    up[2 * h] = __uint_as_float(static_cast<uint32_t>(u));
    up[2 * h + 1] = __uint_as_float(static_cast<uint32_t>(u >> 32));
    if constexpr (SAT) {
#pragma unroll
      for (int r = 2 * h; r < 2 * h + 2; ++r)
        dn[r] = __uint_as_float(__builtin_elementwise_sub_sat(__float_as_uint(p[r]), 2u));  // p >= 0: stops at +0
    } else {
      const uint64_t d = pr - kTwoUlps;
      dn[2 * h] = __uint_as_float(static_cast<uint32_t>(d));
      dn[2 * h + 1] = __uint_as_float(static_cast<uint32_t>(d >> 32));
    }
  }
  // REUSE: the first conversion of each word writes its low half over an input that dies
  // there (the high half is written next) instead of a zeroed register; one move less per
  // word, at the price of a longer-lived input where registers are short
  lo = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(dn[0], dn[1], REUSE ? __float_as_int(dn[0]) : 0, false));
  lo = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(dn[2], dn[3], static_cast<int>(lo), true));
  hi = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(up[0], up[1], REUSE ? __float_as_int(up[0]) : 0, false));
  hi = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(up[2], up[3], static_cast<int>(hi), true));
}

// The four bytes themselves: the lower neighbours' bytes when both neighbours agree, else the
// binary64 recheck.
template <bool SAT = false>
__device__ inline uint32_t fp8_exp2_word(const float (&x)[4], float (&p)[4]) {
  uint32_t lo, hi;
  fp8_exp2_bounds<SAT>(p, lo, hi);
  if (__builtin_expect(lo != hi, 0)) {
#pragma unroll
    for (int r = 0; r < 4; ++r) p[r] = exp2_via_f64(x[r]);
    lo = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(p[0], p[1], 0, false));
    lo = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(p[2], p[3], static_cast<int>(lo), true));
  }
  return lo;
}

// ExpCast constants (exact fp32 values of the reference, expcast.cuh:7).
constexpr float kExpA = 11.541560173034668f;
constexpr float kExpB = 119.6500015258789f;

// Sage INT8 scale and code for one group (quant_per_thread.py:41-44, IEEE division).
__device__ inline float int8_scale(float amax) { return __fadd_rn(__fdiv_rn(amax, 127.0f), 1e-7f); }
__device__ inline int int8_code(float x, float s) {
  float y = __fdiv_rn(x, s);
  y = __fadd_rn(y, y >= 0.0f ? 0.5f : -0.5f);
  return static_cast<int>(truncf(y));
}
// int8_code(x, s) with the quotient from r = RN(1/s) (one IEEE division per group):
// q0 = RN(x*r), e = x - q0*s (one FMA, exact unless it underflows), y = RN(q0 + e*r).
// This is the correctly rounded x/s whenever the residual does not underflow (Markstein's
// correction theorem, "IA-64 and Elementary Functions", 2000), i.e. for |x| >= 2^-102.
// Below that, |x/s| < 2^-102 / 1e-7 < 0.25 (every group scale is >= 1e-7), and both
// quotients give code 0. A GPU comparison against __fdiv_rn over every bf16 and fp16 x
// and 18k scales, plus 1.9e10 random binary32 x, found no differing code.
__device__ inline float recip_rn(float s) { return __fdiv_rn(1.0f, s); }
__device__ inline int int8_code_r(float x, float s, float r) {
  const float q0 = __fmul_rn(x, r);
  float y = __builtin_fmaf(__builtin_fmaf(-q0, s, x), r, q0);
  y = __fadd_rn(y, y >= 0.0f ? 0.5f : -0.5f);
  return static_cast<int>(truncf(y));
}

// ------------------------------------------------------------------ wave helpers

// Cross-lane reductions without the LDS pipe. dpp_move<CTRL> reads another lane of the same
// row of 16 through a DPP operand: quad_perm xor 1 (0xB1) and xor 2 (0x4E), row_half_mirror
// (0x141: i <-> 7-i), row_mirror (0x140: i <-> 15-i). The gfx950 permlane swaps return
// {x[l], x[l ^ 16]} (or ^ 32) in some order, so max and + over the pair are exact.
template <int CTRL>
__device__ inline float dpp_move(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ inline float max_xor16(float v) {
  const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}
__device__ inline float max_xor32(float v) {
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}
// x + x[l ^ 16] and x + x[l ^ 32] in binary64 (the pair's sum: addition commutes).
__device__ inline double add_xor16(double v) {
  const uint64_t b = static_cast<uint64_t>(__double_as_longlong(v));
  const auto lo = __builtin_amdgcn_permlane16_swap(static_cast<uint32_t>(b), static_cast<uint32_t>(b), false, false);
  const auto hi = __builtin_amdgcn_permlane16_swap(static_cast<uint32_t>(b >> 32), static_cast<uint32_t>(b >> 32), false, false);
  return __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hi[0]) << 32) | lo[0])) +
         __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hi[1]) << 32) | lo[1]));
}
__device__ inline double add_xor32(double v) {
  const uint64_t b = static_cast<uint64_t>(__double_as_longlong(v));
  const auto lo = __builtin_amdgcn_permlane32_swap(static_cast<uint32_t>(b), static_cast<uint32_t>(b), false, false);
  const auto hi = __builtin_amdgcn_permlane32_swap(static_cast<uint32_t>(b >> 32), static_cast<uint32_t>(b >> 32), false, false);
  return __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hi[0]) << 32) | lo[0])) +
         __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hi[1]) << 32) | lo[1]));
}
// Maximum over each 32-lane half of the wave (exact in any pairing order): quad exchanges,
// the 8- and 16-lane mirrors, then lane l ^ 16.
__device__ inline float half_wave_max(float v) {
  v = fmaxf(v, dpp_move<0xB1>(v));
  v = fmaxf(v, dpp_move<0x4E>(v));
  v = fmaxf(v, dpp_move<0x141>(v));
  v = fmaxf(v, dpp_move<0x140>(v));
  return max_xor16(v);
}

// Normalized Sylvester-Hadamard rotation of one row of W = CPT * L values held by L
// consecutive lanes (lane c of the group holds entries c*CPT .. c*CPT + CPT - 1). Strides
// 1, 2, 4, ... in order: the in-lane strides first, then lane xor 1, 2, ...; each pair
// (a, b) with a the lower entry becomes (RN(a + b), RN(a - b)); then every entry is
// multiplied by norm = RN_f32(1/sqrt(W)). Every lane of the group must take part.
// Reference: hadamard, src/vc_attention/core.py:79-92; transform_qk_kernel, csrc/kernels.cu:104-123.
template <int CPT, int L>
__device__ inline void hadamard_row(float (&x)[CPT], int c, float norm) {
#pragma unroll
  for (int s = 1; s < CPT; s <<= 1)
#pragma unroll
    for (int j = 0; j < CPT; ++j)
      if (!(j & s)) {
        const float a = x[j], b = x[j + s];
        x[j] = __fadd_rn(a, b);
        x[j + s] = __fsub_rn(a, b);
      }
  // Lane xor 1 and 2 stay inside a quad of lanes: a DPP quad_perm move reads the partner
  // ([1,0,3,2] = 0xB1, [2,3,0,1] = 0x4E) without the LDS-pipe permute of __shfl_xor.
#pragma unroll
  for (int m = 1; m < L; m <<= 1)
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      const float other = m == 1 ? dpp_move<0xB1>(x[j]) : m == 2 ? dpp_move<0x4E>(x[j]) : __shfl_xor(x[j], m, 64);
      x[j] = (c & m) ? __fsub_rn(other, x[j]) : __fadd_rn(x[j], other);
    }
#pragma unroll
  for (int j = 0; j < CPT; ++j) x[j] = __fmul_rn(x[j], norm);
}

}  // namespace vcx
