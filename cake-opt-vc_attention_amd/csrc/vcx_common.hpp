// Shared host/device helpers for the gfx950 sageattn_vc kernels.
#pragma once

#include <hip/hip_runtime.h>

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

__device__ inline float wave_xor_max(float v, int mask) { return fmaxf(v, __shfl_xor(v, mask, 64)); }

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
      float other;
      if (m == 1)
        other = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x[j]), 0xB1, 0xF, 0xF, false));
      else if (m == 2)
        other = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x[j]), 0x4E, 0xF, 0xF, false));
      else
        other = __shfl_xor(x[j], m, 64);
      x[j] = (c & m) ? __fsub_rn(other, x[j]) : __fadd_rn(x[j], other);
    }
#pragma unroll
  for (int j = 0; j < CPT; ++j) x[j] = __fmul_rn(x[j], norm);
}

}  // namespace vcx
