// Fused sageattn_vc forward for gfx950 (MI355X).
//
// One workgroup = 4 waves = 128 query rows; each wave owns 32 rows as two
// 16-row groups. Per 128-key tile:
//   S^T = K Q^T       v_mfma_i32_16x16x64_i8   (A = K rows from LDS, B = Q^T in VGPRs)
//   logits, online max, ExpCast codes         VALU, one query row per lane
//   O^T += V^T P^T    v_mfma_f32_16x16x128_f8f6f4 (A = V^T from LDS, B = codes in VGPRs)
//   row mass          the same MFMA with an all-ones A operand
// The 16x16 accumulator layout (lane l holds rows 4*(l/16)+r, column l%16)
// puts the 32 scores of one query row of a 16-key block in the 4 lanes
// l%16 + 16*G; the codes of block j, rows r=0..3 form byte 4j+r of the lane's
// PV B operand, so P never leaves the registers. K rows are loaded into the
// A operand in the order key(j, 4G+r) = 16j + 8(r/2) + 2G + r%2, which gives
// every lane group G exactly the keys of Sage K-scale group (key%8)/2 == G;
// the V payload is stored in the matching order (vcx_value_token).
//
// K and V^T tiles stream through LDS with gfx950 direct-to-LDS loads
// (global_load_lds_dwordx4), double buffered, placed so that the operand reads
// run at the conflict-free ds_read_b128 rate (key_row / chunk_xor below).
//
// Numerical contract (reference sal/csrc/vc/vc_sm90.cu:284-612, vc_math.cuh:268-474):
//   tiles before the last: logit = RN(float(acc) * RN(sm * RN(qs*ks)))
//   last tile:             logit = RN(RN(float(acc) * RN(qs*ks)) * sm), keys >= Nk -> -inf
//   m' = max(m, rowmax), code = sat_u8(RNE(fmaf(RN(logit-m'), A, B)))
//   alpha = exp2((m - m') * log2(e)) (hardware exp2; alpha == 1 exactly when m' == m)
//   O = alpha*O + PV (+ mass*mean), den = alpha*den + mass, out = O/den * vs.
// The P bytes follow the contract exactly; alpha, O and den only feed the
// bf16/fp16 output, whose tolerance covers the exp2 approximation. With per-channel
// V scales (VM 1) the mass*mean term is deferred: every 16 tiles one f16 MFMA per
// channel block adds sum_t mean_t (x) w_t, w_t the tile mass rescaled with O.
//
// PM = 2 (expcast = 2, no block values) is the folded encode of the reference's default
// kernel modes (vc_math.cuh:16-111): code = sat_u8(RNE(fmaf(base, RN(scale*A), fmaf(-m', A, B))))
// with scale = RN(sm*RN(qs*ks)) (last tile: base = RN(float(acc)*dq), scale = sm), and the
// unfused code above for a whole 16-row group in a tile where some |m'| > 128, a scale
// underflows or a gain overflows (the reference's warp-wide fallback).
//
// QF = 1 is the block-scaled FP8 QK format (the reference's experimental vc27,
// sal/sageattention_local/vc_fp8.py, fp8_dispatch.cuh): E4M3 Q/K with one scale per
// 64 query rows and one per 128-key tile, scores from v_mfma_f32_16x16x128_f8f6f4 (the
// same K/Q fragment loads, two 16-byte halves per lane; D64 pads the second half with
// zeros), V per-channel E4M3 with no block values, and the PM 0/1/2 probability paths.
//
// PM = 0 is the Sage FP8 control path (expcast=False; vc_sm90.cu:177,
// attn_utils.cuh:355-455): a.sm = RN(sm * RN(log2 e)), base/factor as above,
// m' = max(m, max fmaf(base, factor, -8.807)), P = E4M3(exp2(fmaf(base, factor, -m'))) with
// the correctly rounded binary32 exp2 (fp8_exp2_word: v_exp_f32, rechecked in binary64 next
// to an E4M3 rounding midpoint); den and the mean restore use the unrounded sum of P.
#include "vcx_common.hpp"

#include <functional>
#include <map>
#include <mutex>
#include <type_traits>
#include <utility>
#include <vector>

namespace vcx {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kThreadsPerBlock = 256;
constexpr int kRowsPerBlock = 128;

struct AttnArgs {
  const int8_t* q8;
  const int8_t* k8;
  const uint8_t* v8;
  const float* qs;
  const float* ks;
  const float* vs;
  const uint16_t* means;
  void* out;
  int64_t osb, osh, osn;
  int64_t H, Nq, Nk, tiles, qblocks, qs_len;
  float sm;
  uint8_t* pdump;
  int64_t prow0, prow1;
  // Block list: nfull 128-row blocks, dealt to the 8 XCDs as contiguous ranges; the last kconv
  // blocks of every XCD's range run as two 64-row blocks each, after all its 128-row blocks.
  int64_t nfull, kconv;
};

// LDS placement of the K and V^T tiles. Both operands are read as lane (G = l/16,
// li = l%16) -> LDS row 16b + li, physical 16-byte chunk X ^ x(li), where X is what the
// lane group needs (QK: 4ds + G; PV: 4h + G) and x(li) = li & 7 for 128-byte rows,
// (li >> 1) & 3 for the 64-byte K rows of D64. On gfx950 this read pattern runs at the
// conflict-free ds_read_b128 rate (4.55 clocks per wave instruction per CU, measured);
// XORs keyed on the key row instead of the reading lane ran 2-way conflicted (8.2).
//  K:   LDS row p holds key 16(p/16) + kr(p%16) (kr: the MFMA row order, whose lane
//       group G gets Sage K-scale group (key%8)/2 == G); chunk q holds channel chunk
//       q ^ x(p).
//  V^T: LDS row = channel; physical chunk q holds token chunk 2(q' & 3) + q'/4 with
//       q' = q ^ (channel & 7), so lane group G finds its chunks 2G, 2G + 1 at 4h + G.
__device__ inline int key_row(int p) {
  const int r = p & 15;
  return (p & ~15) + 8 * ((r & 3) >> 1) + 2 * (r >> 2) + (r & 1);
}
template <int D>
__device__ inline int chunk_xor(int p) { return D == 128 ? (p & 7) : ((p >> 1) & 3); }

typedef __attribute__((address_space(3))) void lds_void;
typedef const __attribute__((address_space(1))) void global_void;

// Direct-to-LDS loads of one key tile. Each of the 4 waves issues D/32
// instructions for K and D/32 for V^T; instruction n of wave w fills the 64
// consecutive 16-byte slots (w*(D/32) + n)*64 + lane. Slot s is LDS row s/(D/16) (K)
// or s/8 (V^T) at physical chunk s%(D/16) or s%8; the source row and chunk follow the
// placement above.
// Lane-constant parts of the addresses are precomputed once per kernel.
// Raw buffer resource over [base, base + bytes): out-of-range lanes read zeros.
__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}

// Value modes: VM 0 = no smoothing (per-channel V scale in the epilogue),
// 1 = block-mean smoothing with per-channel scales, 2 = block-mean smoothing
// with per-block scales (applied to every tile's contribution).
// VM 1 and 2 defer the block-mean restore: the fp16 means of tile t land in slot t % NR of
// an LDS ring, and every kChunk tiles one f16 MFMA per channel block adds
// sum_t mean_t (x) w_t to O (w_t: the row's tile mass, rescaled like O). VM 2 also rings
// the tile's fp32 V scales and feeds RN_f16(vs_t * mean_t) to that MFMA instead.
constexpr int kChunk = 16, kRing = 32;

template <int D, int VM, int QF = 0>
struct TileLoader {
  static constexpr bool SMOOTH = VM >= 1, BSCALE = VM == 2, RING = VM >= 1;
  // Ring slots: the DMA of tile t+1 is in flight while a flush reads tiles t-15..t, so a
  // ring needs kChunk + 1 slots; VM 1 keeps 32 (power of two), VM 2 (which also rings
  // 4*D bytes of V scales per tile) the minimum, to stay within two blocks' LDS per CU.
  static constexpr int NR = BSCALE ? kChunk + 1 : kRing;
  // Slot strides of the rings, padded by 16 bytes: a flush reads slots 4 apart in the four
  // lane groups, and 4 x (2D + 16) = 64 mod 256 puts those reads in four different 64-byte
  // bank windows (unpadded, 4 x 2D is a multiple of 256: four-way bank conflicts).
  static constexpr int RS = 2 * D + 16, VS = 4 * D + 16;
  // Meta region of a buffer: the tile's K scales (INT8: 4 Sage key-group scales, 16 bytes;
  // FP8 block: one scale, 4 bytes), loaded by wave 0 with the means; V scales by wave 1.
  static constexpr int MR = SMOOTH ? (2 * D) / 16 : 0;  // lanes that load the tile's means
  static constexpr int VL = BSCALE ? (4 * D) / 16 : 0;  // lanes that load the tile's V scales
  static constexpr int KS_OFF = 0;
  static constexpr int META_BYTES = 16;
  static constexpr int N = D / 32;  // instructions per wave per operand
  uint32_t koff[N];                 // lane byte offset inside the K tile (row*D + chunk*16)
  uint32_t voff[N];                 // lane byte offset inside the V^T tile columns
  uint32_t moff;                    // lane byte offset of the meta load (wave 0)
  __amdgpu_buffer_rsrc_t rk, rv, rm, rs, rb;
  uint8_t* ring;                    // RING: LDS ring of NR tiles x D fp16 means
  uint8_t* vsring;                  // BSCALE: LDS ring of NR tiles x D fp32 V scales
  int wave;

  __device__ inline void init(const AttnArgs& a, int64_t bh) {
    wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int64_t npad = a.tiles * kTile;
#pragma unroll
    for (int n = 0; n < N; ++n) {
      const int s = (wave * N + n) * 64 + lane;
      const int p = s / (D / 16), phys = s % (D / 16);
      koff[n] = static_cast<uint32_t>(key_row(p) * D + ((phys ^ chunk_xor<D>(p)) * 16));
      const int ch = s >> 3, q = (s & 7) ^ (ch & 7);
      voff[n] = static_cast<uint32_t>(ch * static_cast<int>(npad) + (2 * (q & 3) + (q >> 2)) * 16);
    }
    // Per-head resources. K rows past Nk read zeros (their logits are masked anyway).
    rk = make_rsrc(a.k8 + bh * a.Nk * D, static_cast<uint32_t>(a.Nk * D));
    rv = make_rsrc(a.v8 + bh * D * npad, static_cast<uint32_t>(D * npad));
    if constexpr (QF == 1) rs = make_rsrc(a.ks + bh * a.tiles, static_cast<uint32_t>(a.tiles * 4));
    else rs = make_rsrc(a.ks + bh * a.tiles * 4, static_cast<uint32_t>(a.tiles * 16));
    if constexpr (SMOOTH) rm = make_rsrc(a.means + bh * a.tiles * D, static_cast<uint32_t>(a.tiles * D * 2));
    if constexpr (BSCALE) rb = make_rsrc(a.vs + bh * a.tiles * D, static_cast<uint32_t>(a.tiles * D * 4));
    moff = static_cast<uint32_t>(lane * 16);
  }

  // All addresses are a wave-uniform soffset (the tile) plus lane-constant
  // voffsets: no per-lane address arithmetic in the loop.
  __device__ inline void issue(int64_t t, uint8_t* lk, uint8_t* lv, uint8_t* lm) const {
    const int lane = threadIdx.x & 63;
    if (wave == 0) {
      if constexpr (SMOOTH) {
        uint8_t* dst = ring + (t % NR) * RS;
        if (lane < MR)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rm, (lds_void*)dst, 16, moff, static_cast<int>(t * D * 2), 0, 0);
      }
      if (lane == 0) {
        if constexpr (QF == 1)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(lm + KS_OFF), 4, 0, static_cast<int>(t * 4), 0, 0);
        else
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(lm + KS_OFF), 16, 0, static_cast<int>(t * 16), 0, 0);
      }
    }
    if constexpr (BSCALE) {
      if (wave == 1 && lane < VL)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void*)(vsring + (t % NR) * VS), 16, moff,
                                                 static_cast<int>(t * D * 4), 0, 0);
    }
    const int kso = static_cast<int>(t * kTile * D);
#pragma unroll
    for (int n = 0; n < N; ++n)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void*)(lk + (wave * N + n) * 1024), 16, koff[n], kso, 0, 0);
    const int vso = static_cast<int>(t * kTile);
#pragma unroll
    for (int n = 0; n < N; ++n)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_void*)(lv + (wave * N + n) * 1024), 16, voff[n], vso, 0, 0);
  }
};

__device__ inline v4f mfma_fp8(const v8i& a, const v8i& b, const v4f& c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}
// Row mass: A = 16 x 128 ones in FP4 E2M1 (0x2 = 1.0; 16 bytes per lane, so the compiler
// keeps four registers instead of eight), B = the E4M3 probabilities. Same 8-pass timing as
// the E4M3 x E4M3 product (measured) and the same sums: every product is exactly P.
__device__ inline v4f mfma_mass(const v4i& ones4, const v8i& b, const v4f& c) {
  const v8i a = {ones4[0], ones4[1], ones4[2], ones4[3], 0, 0, 0, 0};  // upper half unread
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 4, 0, 0, 0, 0, 0);
}

// v_max_f32 / v_max3_f32 as single instructions: fmaxf lowers to maxnum, around which the
// compiler inserts NaN-quieting copies of values coming out of the permlane swaps. The
// operands here are finite or -inf.
__device__ inline float vmax(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ inline float vmax3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// Row reductions over the four lane groups that hold one query row: gfx950
// permlane swaps give each lane the values of lanes l^16 and l^32 without an LDS
// round trip. Every lane of the row ends with the same value (the adds commute).
// running_max returns max(m, row maximum of x).
__device__ inline float running_max(float m, float x) {
  const auto x16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = vmax(__uint_as_float(x16[0]), __uint_as_float(x16[1]));
  const auto x32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return vmax3(m, __uint_as_float(x32[0]), __uint_as_float(x32[1]));
}

// running_max2 gives mn[g] = max(m[g], row maximum of x[g]) for both row groups of a wave
// in one reduction. With the wave's 16-lane rows R0..R3 (lane group G = row RG): the 16-lane
// swap of x[0] against x[1] and a maximum leave (x0 of R0|R1, x1 of R0|R1, x0 of R2|R3,
// x1 of R2|R3) in R0..R3; the 32-lane swap and a maximum complete each group's maximum
// (R0, R2: group 0; R1, R3: group 1); a last 16-lane swap hands every lane both.
__device__ inline void running_max2(const float (&m)[2], const float (&x)[2], float (&mn)[2]) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x[0]), __float_as_uint(x[1]), false, false);
  const float c = vmax(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(c), __float_as_uint(c), false, false);
  const float d = vmax(__uint_as_float(b[0]), __uint_as_float(b[1]));
  const auto e = __builtin_amdgcn_permlane16_swap(__float_as_uint(d), __float_as_uint(d), false, false);
  mn[0] = vmax(m[0], __uint_as_float(e[0]));
  mn[1] = vmax(m[1], __uint_as_float(e[1]));
}

// Whether `pred` holds on some active lane (a scalar test of the lane mask).
__device__ inline bool wave_any(bool pred) { return __builtin_amdgcn_ballot_w64(pred) != 0; }

__device__ inline float row_sum(float x) {
  const auto x16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(x16[0]) + __uint_as_float(x16[1]);
  const auto x32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(x32[0]) + __uint_as_float(x32[1]);
}

// Sage's FP8 offset: the control path's row maximum is lowered by 8.807 so that the
// largest probability is 2^8.807 ~ 448, the E4M3 maximum (sal/csrc/qattn/attn_utils.cuh:30).
constexpr float kFp8Offset = 8.807f;
// The folded path starts its QK accumulators at the bits of 1.5 * 2^23: with |acc| < 2^22
// they read as the float 12582912 + acc, so float(acc) is one exact subtraction.
constexpr int kBias = 0x4B400000;
constexpr float kBiasF = 12582912.0f;

// Mask of the active lanes whose x is a positive normal number: one v_cmp_class_f32 into an
// SGPR pair (the ballot of __builtin_amdgcn_classf adds a select and a compare).
__device__ inline uint64_t pos_normal_lanes(float x) {
  uint64_t r;
  asm("v_cmp_class_f32_e64 %0, %1, %2" : "=s"(r) : "v"(x), "s"(1 << 8));
  return r;
}

// Score of accumulator element r: FP8 scores are floats already; the folded path's
// INT8 accumulators carry the kBias offset.
__device__ inline float acc_value(const v4f& acc, int r) { return acc[r]; }
__device__ inline float acc_value(const v4i& acc, int r) { return __int_as_float(acc[r]) - kBiasF; }

// NQG: 16-row groups per wave (2: a 128-row block of 4 waves; 1: a 64-row block, the
// finer work pieces that end each XCD's list of blocks).
template <int D, int VM, bool DUMP, int PM, int QF = 0, int NQG = 2>
struct Wave {
  static constexpr bool EC = PM != 0;  // ExpCast bytes (1 unfused, 2 folded) or the control path (0)
  // Biased INT8 accumulators (float(acc) = one v_sub_f32): the folded path, the unfused
  // path at D128 with channel-scale smoothing (same-box: smoothing 11.13 -> 11.06 ms, long
  // 43.24 -> 43.00 ms) and the control path at D128 (but its per-block-scale diagnostic
  // variant). D64 (168 VGPRs at three waves per SIMD) and the unfused path with per-block V
  // scales keep v_cvt_f32_i32: the bias register costs them spills.
  static constexpr bool IB = QF == 0 && (PM == 2 || (PM == 1 && D == 128 && VM == 1) ||
                                         (PM == 0 && D == 128 && !(VM == 2 && DUMP)));
  static constexpr int kD = D;
  static constexpr int DS = D / 64;  // 64-deep QK steps
  static constexpr int CB = D / 16;  // 16-channel output blocks
  static constexpr bool SMOOTH = VM >= 1, BSCALE = VM == 2;
  typedef TileLoader<D, VM, QF> LD;
  typedef std::conditional_t<QF == 1, v4f, v4i> Acc;  // 16x16 score accumulator

  // The exact float value of one INT8 score accumulator element.
  __device__ static inline float acc_float(int x) {
    if constexpr (IB) return __int_as_float(x) - kBiasF;
    else return static_cast<float>(x);
  }

  // DACC: the row mass accumulates in the C operand of the all-ones MFMA (element 0 is the
  // row's denominator; the history rescale scales only that element, the other three are
  // never read) instead of a zero-started MFMA and one addition per tile: ExpCast without
  // block values at D128 (D64's three waves per SIMD have no registers for it).
  static constexpr bool DACC = EC && VM == 0 && D == 128;
  v4i qf[NQG][DS];
  float qsv[NQG];
  int64_t row[NQG];
  float m[NQG], den[NQG];
  v4f dacc[NQG];
  // Folded encode: fmaf(-m, A, B) of the running maximum, refreshed only when m moves
  float fbias[NQG];
  v4f O[NQG][CB];
  float wts[NQG][4];  // VM 1, 2: pending mean weights of chunk tiles 4G..4G+3 (row li)
  int koff[DS], voff[2];
  v4i ones;  // all-ones FP4 (E2M1) A operand of the row-mass MFMA
  v4i bacc;  // kBias in every element: the initial QK accumulator of the biased paths
  // Folded encode (INT8 QK): the per-tile fold conditions are known to hold on every tile
  // but the last (set once per wave by fold_precheck; wave-uniform)
  int fold_ok;
  int G, li;
  int64_t bh_;

  // The folded encode's conditions on a tile before the last (scale = RN(sm * RN(qs * ks))
  // and gain = RN(scale * A) positive normal, |m'| <= 128) hold on every such tile when
  //  - RN(sm * RN(qs * ks)) is a positive normal at the head's smallest and largest K scale
  //    and RN(scale * A) is one at the largest (RN and multiplication by positive factors
  //    are monotone, so every tile's scale and gain lie between these; the K scales are
  //    compared as bit patterns, which orders positive floats and sends zero, negative,
  //    NaN and infinite scales to an end that fails), and
  //  - |logit| <= RN(128 * sum|q8| * scale_hi) <= 128 for the lane's row: every score's
  //    |acc| <= 128 * sum|q8|, so every logit, each tile's maximum and from the first tile on
  //    the running maximum stay within it.
  // fold_ok is the AND over the wave; when it fails the tiles test the conditions.
  __device__ inline void fold_precheck(const AttnArgs& a, int lane) {
    const uint32_t* kb = reinterpret_cast<const uint32_t*>(a.ks) + bh_ * a.tiles * 4;
    uint32_t kmin = 0xffffffffu, kmax = 0u;
    // 16 loads per lane in flight before any is used (one round trip per 1024 scales)
    constexpr int kBatch = 16;
    const int64_t n = a.tiles * 4;
    for (int64_t i0 = lane; i0 < n; i0 += 64 * kBatch) {
      uint32_t u[kBatch];
#pragma unroll
      for (int b = 0; b < kBatch; ++b) u[b] = i0 + 64 * b < n ? kb[i0 + 64 * b] : kb[i0];
      __builtin_amdgcn_sched_barrier(0);  // all loads issued before the first use
#pragma unroll
      for (int b = 0; b < kBatch; ++b) {
        kmin = u[b] < kmin ? u[b] : kmin;
        kmax = u[b] > kmax ? u[b] : kmax;
      }
    }
#pragma unroll
    for (int sh = 32; sh >= 1; sh >>= 1) {
      const uint32_t lo = __shfl_xor(kmin, sh), hi = __shfl_xor(kmax, sh);
      kmin = lo < kmin ? lo : kmin;
      kmax = hi > kmax ? hi : kmax;
    }
    uint64_t ok = __builtin_amdgcn_read_exec();
#pragma unroll
    for (int qg = 0; qg < NQG; ++qg) {
      int asum = 0;
#pragma unroll
      for (int ds = 0; ds < DS; ++ds)
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int by = 0; by < 4; ++by) {
            const int x = static_cast<int8_t>((static_cast<uint32_t>(qf[qg][ds][e]) >> (8 * by)) & 0xffu);
            asum += x < 0 ? -x : x;
          }
      asum += __shfl_xor(asum, 16);
      asum += __shfl_xor(asum, 32);
      const float s_lo = a.sm * (qsv[qg] * __uint_as_float(kmin));
      const float s_hi = a.sm * (qsv[qg] * __uint_as_float(kmax));
      const float bound = static_cast<float>(128 * asum) * s_hi;
      ok &= pos_normal_lanes(s_lo) & pos_normal_lanes(s_hi) & pos_normal_lanes(s_hi * kExpA) &
            __builtin_amdgcn_ballot_w64(bound <= 128.0f);
    }
    fold_ok = __builtin_amdgcn_readfirstlane(ok == __builtin_amdgcn_read_exec() ? 1 : 0);
  }

  __device__ inline v8i load_v(const uint8_t* lv, int cb) const {
    const v4i lo = *reinterpret_cast<const v4i*>(lv + cb * 16 * kTile + voff[0]);
    const v4i hi = *reinterpret_cast<const v4i*>(lv + cb * 16 * kTile + voff[1]);
    return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }

  // Phase 1 of a tile for row group qg: the values the encode reads (PM 2 and 0: float(acc),
  // on the last tile float(acc) * dq or -inf past Nk; PM 1: the logits), the logit scale
  // (PM 2) or log2-domain factor (PM 0), and the maximum over this lane's keys.
  template <bool LAST>
  __device__ __forceinline__ float logits(const AttnArgs& a, int64_t t, int qg, const Acc (&Sq)[8], float ksv,
                                          float (&bs)[8][4], float& scl) const {
    float tmo;
    const float dq = qsv[qg] * ksv;
    if constexpr (PM == 2) {
      const float scale = LAST ? a.sm : a.sm * dq;
      scl = scale;
      if constexpr (!LAST && QF == 1) {
        // scale > 0, so RN(max(base) * scale) is the maximum of the rounded logits
        float bm = -INFINITY;
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            bs[j][r] = Sq[j][r];
            bm = fmaxf(bm, bs[j][r]);
          }
        tmo = bm * scale;
      } else if constexpr (!LAST) {
        // float(acc) is exact and monotone: the row maximum is taken on the integers
        int im = Sq[0][0];
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            im = im > Sq[j][r] ? im : Sq[j][r];
            bs[j][r] = __int_as_float(Sq[j][r]) - kBiasF;
          }
        // the biased bits read as 12582912 + max: one exact subtraction gives float(max)
        tmo = (__int_as_float(im) - kBiasF) * scale;
      } else {
        float bm = -INFINITY;
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int64_t key = t * kTile + 16 * j + 8 * (r >> 1) + 2 * G + (r & 1);
            const float f = acc_value(Sq[j], r);
            bs[j][r] = key < a.Nk ? f * dq : -INFINITY;
            bm = fmaxf(bm, bs[j][r]);
          }
        tmo = bm * scale;
      }
    } else if constexpr (PM == 1) {
      float tm = -INFINITY;
      if constexpr (!LAST) {
        const float c = a.sm * dq;
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            bs[j][r] = acc_float(Sq[j][r]) * c;
            tm = fmaxf(tm, bs[j][r]);
          }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int64_t key = t * kTile + 16 * j + 8 * (r >> 1) + 2 * G + (r & 1);
            float x = (acc_float(Sq[j][r]) * dq) * a.sm;
            bs[j][r] = key < a.Nk ? x : -INFINITY;
            tm = fmaxf(tm, bs[j][r]);
          }
      }
      tmo = tm;
    } else {
      // Sage FP8 control path: log2-domain logits (a.sm carries RN(sm * RN(log2 e))),
      // running maximum with the upstream 8.807 offset, P = E4M3(exp2(.)) and an
      // unrounded mass.
      const float f = LAST ? a.sm : a.sm * dq;
      scl = f;
      float tm;
      if constexpr (!LAST) {
        // f > 0, so fmaf(b, f, -offset) is monotone in b: the maximum is taken on the
        // scores (on the integers for INT8 accumulators), then shifted once
        if constexpr (QF == 0) {
          int im = Sq[0][0];
#pragma unroll
          for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              im = im > Sq[j][r] ? im : Sq[j][r];
              bs[j][r] = acc_float(Sq[j][r]);
            }
          tm = __builtin_fmaf(acc_float(im), f, -kFp8Offset);
        } else {
          float bm = -INFINITY;
#pragma unroll
          for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              bs[j][r] = Sq[j][r];
              bm = vmax(bm, bs[j][r]);
            }
          tm = __builtin_fmaf(bm, f, -kFp8Offset);
        }
        // f = +inf (an extreme sm_scale) with a zero maximum gives NaN where the maximum of
        // the shifted terms (each -inf or NaN) is -inf
        if (tm != tm) tm = -INFINITY;
      } else {
        tm = -INFINITY;
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float b;
            if constexpr (QF == 1) b = Sq[j][r];
            else b = acc_float(Sq[j][r]);
            const int64_t key = t * kTile + 16 * j + 8 * (r >> 1) + 2 * G + (r & 1);
            b = key < a.Nk ? b * dq : -INFINITY;
            bs[j][r] = b;
            tm = fmaxf(tm, __builtin_fmaf(b, f, -kFp8Offset));
          }
      }
      tmo = tm;
    }
    return tmo;
  }

  // Rescale the history of row group qg, in which some maximum moved (dm = m - m' on each
  // lane): alpha = exp(dm) (exp2 of the log2-domain difference on the control path) is
  // exactly 1 on the other lanes, and O, den (and the pending mean weights) are scaled before
  // the tile's PV adds in.
  __device__ __forceinline__ void rescale(int qg, float dm) {
    const float alpha = EC ? __builtin_amdgcn_exp2f(dm * 1.44269504088896341f) : __builtin_amdgcn_exp2f(dm);
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) O[qg][cb] *= alpha;
    if constexpr (DACC) dacc[qg][0] *= alpha;
    else den[qg] *= alpha;
    if constexpr (SMOOTH) {
#pragma unroll
      for (int j = 0; j < 4; ++j) wts[qg][j] *= alpha;
    }
  }

  // Phase 3 of a tile for row group qg: the P bytes against the running maximum mx (and on
  // the control path the row's unrounded mass tmq).
  template <bool LAST, bool PRE>
  __device__ __forceinline__ void bytes(const AttnArgs& a, const float (&bs)[8][4], float scl, float mx, float fb,
                                        v8i& Pq, float& tmq) const {
    if constexpr (PM == 2) {
      // Folded ExpCast encode (the reference's default kernel modes without block
      // values, sal/csrc/vc/vc_math.cuh:16-111): code = RNE(fmaf(base, gain, bias)) with
      // gain = RN(scale * A) and bias = fmaf(-m', A, B), unless some row of this 16-row
      // group has |m'| > 128 or a lane's scale underflows or its gain overflows; then the
      // whole group takes the unfused code RNE(fmaf(RN(RN(base * scale) - m'), A, B)).
      const float scale = scl;
      const float gain = scale * kExpA;
      // every lane admits the fold: scale a positive normal (so gain is a positive normal
      // or +inf) and gain a positive normal (finite), |m'| <= 128; lane masks combined on
      // the scalar unit
      bool fold = true;
      if constexpr (!PRE) {
        const uint64_t safe = pos_normal_lanes(scale) & pos_normal_lanes(gain) &
                              __builtin_amdgcn_ballot_w64(fabsf(mx) <= 128.0f);
        fold = safe == __builtin_amdgcn_read_exec();
      }
      if (fold) {
        const float bias = fb;  // fmaf(-mx, A, B), kept with the running maximum
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          uint32_t w = 0;
#pragma unroll
          for (int r = 0; r < 4; ++r) w = __builtin_amdgcn_cvt_pk_u8_f32(__builtin_fmaf(bs[j][r], gain, bias), r, w);
          Pq[j] = static_cast<int>(w);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          uint32_t w = 0;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float lgt = bs[j][r] * scale;
            w = __builtin_amdgcn_cvt_pk_u8_f32(__builtin_fmaf(lgt - mx, kExpA, kExpB), r, w);
          }
          Pq[j] = static_cast<int>(w);
        }
      }
    } else if constexpr (PM == 1) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        uint32_t w = 0;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float u = __builtin_fmaf(bs[j][r] - mx, kExpA, kExpB);
          w = __builtin_amdgcn_cvt_pk_u8_f32(u, r, w);
        }
        Pq[j] = static_cast<int>(w);
      }
    } else {
      const float f = scl;
      // Bytes of the +-2 ulp neighbours of every probability (the lower ones by a saturating
      // subtraction on every tile, so that p = 0, i.e. a score more than about 103 nats
      // below the row maximum, never forces a recheck); an E4M3 midpoint within two ulps
      // (the neighbours disagree, a few lanes per million) takes the binary64 recheck.
      // At D128 the recheck is one branch per tile (a lane that missed redoes its tile from
      // the scores, which stay live), so the loop stays one block that the MFMAs
      // interleave with; D64's three waves per SIMD have no registers for that and branch
      // per four probabilities.
      float ls = -0.0f;  // -0 + p = p: the first addition folds away
      if constexpr (D == 128) {
        uint32_t miss = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          float pr[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) pr[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(bs[j][r], f, -mx));
          uint32_t lo, hi;
          fp8_exp2_bounds<true, true>(pr, lo, hi);
          Pq[j] = static_cast<int>(lo);
          miss |= lo ^ hi;
#pragma unroll
          for (int r = 0; r < 4; ++r) ls += pr[r];
        }
        if (__builtin_expect(miss != 0, 0)) {
          ls = -0.0f;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            float xs[4], pr[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              float b = bs[j][r];
              asm volatile("" : "+v"(b));  // recomputed here, not kept live from the loop above
              xs[r] = __builtin_fmaf(b, f, -mx);
              pr[r] = __builtin_amdgcn_exp2f(xs[r]);
            }
            Pq[j] = static_cast<int>(fp8_exp2_word<true>(xs, pr));
#pragma unroll
            for (int r = 0; r < 4; ++r) ls += pr[r];
          }
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          float xs[4], pr[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            xs[r] = __builtin_fmaf(bs[j][r], f, -mx);
            pr[r] = __builtin_amdgcn_exp2f(xs[r]);
          }
          Pq[j] = static_cast<int>(fp8_exp2_word<true>(xs, pr));
#pragma unroll
          for (int r = 0; r < 4; ++r) ls += pr[r];
        }
      }
      tmq = row_sum(ls);
    }
  }

  // DUMP: the P bytes of rows prow0..prow1 to pdump in logical key order.
  __device__ __forceinline__ void dump_p(const AttnArgs& a, int64_t t, int qg, const v8i& Pq) const {
    if constexpr (DUMP) {
      if (row[qg] >= a.prow0 && row[qg] < a.prow1 && row[qg] < a.Nq) {
        const int64_t npad = a.tiles * kTile;
        uint8_t* dst = a.pdump + (bh_ * (a.prow1 - a.prow0) + (row[qg] - a.prow0)) * npad + t * kTile;
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            dst[16 * j + 8 * (r >> 1) + 2 * G + (r & 1)] = static_cast<uint8_t>((static_cast<uint32_t>(Pq[j]) >> (8 * r)) & 0xffu);
      }
    }
  }

  // PRE: the fold conditions hold on this tile (fold_precheck), so it does not test them
  template <bool LAST, bool PRE = false>
  __device__ inline void tile(const AttnArgs& a, int64_t t, const uint8_t* lk, const uint8_t* lv, const uint8_t* lm) {
    const float ksv = *reinterpret_cast<const float*>(lm + LD::KS_OFF + (QF == 1 ? 0 : 4 * G));

    // ---- S^T = K Q^T
    Acc S[NQG][8];
    v4i kf[8][DS];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) kf[j][ds] = *reinterpret_cast<const v4i*>(lk + j * 16 * D + koff[ds]);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (j + 2 < 8) {
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) kf[j + 2][ds] = *reinterpret_cast<const v4i*>(lk + (j + 2) * 16 * D + koff[ds]);
      }
#pragma unroll
      for (int qg = 0; qg < NQG; ++qg) {
        if constexpr (QF == 1) {
          // E4M3 x E4M3 over all D channels in one 128-deep step; lane group G holds the
          // channel sets {16G..16G+15} and {64+16G..64+16G+15} for both operands.
          const v8i ka = DS == 2 ? v8i{kf[j][0][0], kf[j][0][1], kf[j][0][2], kf[j][0][3],
                                       kf[j][DS - 1][0], kf[j][DS - 1][1], kf[j][DS - 1][2], kf[j][DS - 1][3]}
                                 : v8i{kf[j][0][0], kf[j][0][1], kf[j][0][2], kf[j][0][3], 0, 0, 0, 0};
          const v8i qb = DS == 2 ? v8i{qf[qg][0][0], qf[qg][0][1], qf[qg][0][2], qf[qg][0][3],
                                       qf[qg][DS - 1][0], qf[qg][DS - 1][1], qf[qg][DS - 1][2], qf[qg][DS - 1][3]}
                                 : v8i{qf[qg][0][0], qf[qg][0][1], qf[qg][0][2], qf[qg][0][3], 0, 0, 0, 0};
          S[qg][j] = mfma_fp8(ka, qb, v4f{0.0f, 0.0f, 0.0f, 0.0f});
        } else {
          v4i acc = IB ? bacc : v4i{0, 0, 0, 0};
#pragma unroll
          for (int ds = 0; ds < DS; ++ds) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(kf[j][ds], qf[qg][ds], acc, 0, 0, 0);
          S[qg][j] = acc;
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }

    // ---- logits, online max, P bytes (ExpCast codes, or E4M3 probabilities on the control path)
    v8i P[NQG];
    float tmass[NQG], bs[NQG][8][4], tmax[NQG], scl[NQG];
    // The history of a row group in which some maximum moved is rescaled before this tile's
    // PV adds in. At D64 the scaling sits inside the branches where a maximum can move, so
    // the common tile carries no rescale state (two instructions per tile; same-box D64 with
    // smoothing 0.4-0.7 % faster); at D128 that placement costs the main kernel 0.3 % (its
    // register allocation moves), so there the flags resc / dm carry it to one place after
    // the bytes.
    constexpr bool kEarly = D == 64;
    bool resc[NQG];
    float dm[NQG];
#pragma unroll
    for (int qg = 0; qg < NQG; ++qg) resc[qg] = false;
    auto moved = [&](int qg, float mn) {
      if constexpr (kEarly) {
        if (wave_any(m[qg] != mn)) rescale(qg, m[qg] - mn);
      } else {
        resc[qg] = wave_any(m[qg] != mn);
        dm[qg] = m[qg] - mn;
      }
    };
    if constexpr (PM == 0) {
      // Control path, one row group at a time (D64's three waves per SIMD have no registers
      // for both groups' probabilities at once).
#pragma unroll
      for (int qg = 0; qg < NQG; ++qg) {
        tmax[qg] = logits<LAST>(a, t, qg, S[qg], ksv, bs[qg], scl[qg]);
        const float mn = running_max(m[qg], tmax[qg]);
        moved(qg, mn);
        m[qg] = mn;
        bytes<LAST, PRE>(a, bs[qg], scl[qg], m[qg], 0.0f, P[qg], tmass[qg]);
        if constexpr (DUMP) dump_p(a, t, qg, P[qg]);
      }
    } else {
#pragma unroll
      for (int qg = 0; qg < NQG; ++qg) tmax[qg] = logits<LAST>(a, t, qg, S[qg], ksv, bs[qg], scl[qg]);
      // Both row groups' running maxima in one cross-lane reduction, skipped when no lane's
      // maximum exceeds its row's running maximum (then no row maximum moves).
      uint64_t up = __builtin_amdgcn_ballot_w64(tmax[0] > m[0]);
      if constexpr (NQG == 2) up |= __builtin_amdgcn_ballot_w64(tmax[1] > m[1]);
      if (up != 0) {
        float mn[NQG];
        if constexpr (NQG == 2) running_max2(m, tmax, mn);
        else mn[0] = running_max(m[0], tmax[0]);
#pragma unroll
        for (int qg = 0; qg < NQG; ++qg) {
          moved(qg, mn[qg]);
          m[qg] = mn[qg];
          if constexpr (PM == 2) fbias[qg] = __builtin_fmaf(-mn[qg], kExpA, kExpB);
        }
      }
#pragma unroll
      for (int qg = 0; qg < NQG; ++qg) {
        bytes<LAST, PRE>(a, bs[qg], scl[qg], m[qg], fbias[qg], P[qg], tmass[qg]);
        if constexpr (DUMP) dump_p(a, t, qg, P[qg]);
      }
    }

    if constexpr (!kEarly) {
#pragma unroll
      for (int qg = 0; qg < NQG; ++qg)
        if (resc[qg]) rescale(qg, dm[qg]);
    }

    // ---- O^T += V^T P^T, mass = 1^T P^T
    const v4f zero = {0.0f, 0.0f, 0.0f, 0.0f};
    float mass[NQG];
    if constexpr (BSCALE) {
      // Per-block V scales: O += vs_t * PV_t per channel, one FMA per element on the PV
      // temporary of each channel block; the mean term vs_t * mean_t * mass joins the
      // deferred restore below.
#pragma unroll
      for (int qg = 0; qg < NQG; ++qg) {
        if constexpr (EC) mass[qg] = mfma_mass(ones, P[qg], zero)[0];
        else mass[qg] = tmass[qg];
        den[qg] += mass[qg];
      }
      const uint8_t* vsl = vsring + (t % LD::NR) * LD::VS;
      v8i vc = load_v(lv, 0), vn;
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        if (cb + 1 < CB) vn = load_v(lv, cb + 1);
        const float4 vsb = *reinterpret_cast<const float4*>(vsl + 4 * (16 * cb + 4 * G));
        const float sc[4] = {vsb.x, vsb.y, vsb.z, vsb.w};
#pragma unroll
        for (int qg = 0; qg < NQG; ++qg) {
          const v4f pv = mfma_fp8(vc, P[qg], zero);
#pragma unroll
          for (int r = 0; r < 4; ++r) O[qg][cb][r] = __builtin_fmaf(pv[r], sc[r], O[qg][cb][r]);
        }
        vc = vn;
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      v8i vf[CB];
      vf[0] = load_v(lv, 0);
      if (CB > 1) vf[1] = load_v(lv, 1);
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        if (cb + 2 < CB) vf[cb + 2] = load_v(lv, cb + 2);
#pragma unroll
        for (int qg = 0; qg < NQG; ++qg) O[qg][cb] = mfma_fp8(vf[cb], P[qg], O[qg][cb]);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int qg = 0; qg < NQG; ++qg) {
        if constexpr (DACC) {
          dacc[qg] = mfma_mass(ones, P[qg], dacc[qg]);
        } else {
          if constexpr (EC) mass[qg] = mfma_mass(ones, P[qg], zero)[0];
          else mass[qg] = tmass[qg];
          den[qg] += mass[qg];
        }
      }
    }
    if constexpr (SMOOTH) {
      // Deferred block-mean restore: tile t is position c of its chunk; lane group
      // G = c / 4 keeps the row's mass in slot c % 4 (the MFMA's k = c). At the chunk's
      // end (or the last tile) O^T[ch][row] += sum_k mean_k[ch] * w_k[row] over the
      // chunk, as v_mfma_f32_16x16x16f16 (A: means from the ring, exact in fp16, or with
      // per-block scales RN_f16(vs_k[ch] * mean_k[ch]); B: the weights as fp16 hi and lo
      // parts).
      // Slots of tiles past the last hold w = 0.
      const int c = static_cast<int>(t & (kChunk - 1));
      // one select per row group: the slot c & 3 is wave-uniform (a scalar branch), only the
      // lane-group test G == c / 4 is per lane
      const bool mine = G == (c >> 2);
      switch (c & 3) {
        case 0: set_weight<0>(mine, mass); break;
        case 1: set_weight<1>(mine, mass); break;
        case 2: set_weight<2>(mine, mass); break;
        default: set_weight<3>(mine, mass); break;
      }
      if (LAST || c == kChunk - 1) flush_means(ring, t - c);
    }
  }

  template <int J>
  __device__ __forceinline__ void set_weight(bool mine, const float (&mass)[NQG]) {
#pragma unroll
    for (int qg = 0; qg < NQG; ++qg) wts[qg][J] = mine ? mass[qg] : wts[qg][J];
  }

  // O += means (x) weights over the chunk that starts at tile `base` (VM 1, 2). Each weight
  // goes in as two fp16 parts, hi = RN_f16(w) and lo = RN_f16(w - hi) (w - hi is exact in
  // binary32), so the mean term carries about 22 bits of the weight instead of 11.
  __device__ inline void flush_means(const uint8_t* ring, int64_t base) {
    typedef _Float16 v4h __attribute__((ext_vector_type(4)));
    v4h b[NQG], bl[NQG];
#pragma unroll
    for (int qg = 0; qg < NQG; ++qg) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        b[qg][j] = static_cast<_Float16>(wts[qg][j]);
        bl[qg][j] = static_cast<_Float16>(wts[qg][j] - static_cast<float>(b[qg][j]));
        wts[qg][j] = 0.0f;
      }
    }
    const uint8_t* col = ring + 2 * li;
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      v4h av;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t slot = (static_cast<uint32_t>(base) + 4 * G + j) % LD::NR;
        const _Float16 mh = *reinterpret_cast<const _Float16*>(col + slot * LD::RS + 32 * cb);
        if constexpr (BSCALE) {
          const float vsv = *reinterpret_cast<const float*>(vsring + slot * LD::VS + 4 * (16 * cb + li));
          av[j] = static_cast<_Float16>(static_cast<float>(mh) * vsv);
        } else {
          av[j] = mh;
        }
      }
#pragma unroll
      for (int qg = 0; qg < NQG; ++qg) {
        O[qg][cb] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, bl[qg], O[qg][cb], 0, 0, 0);
        O[qg][cb] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, b[qg], O[qg][cb], 0, 0, 0);
      }
    }
  }
  const uint8_t* ring = nullptr;
  const uint8_t* vsring = nullptr;
};

// D64 without per-block V scales runs three workgroups per CU (at most 168 VGPRs; its
// 37 KB of LDS allows four): the VALU-bound D64 loop gains from the third wave per SIMD
// (same-box: smoothing D64 8.15 -> 7.75 ms). D128 is held to two by its 64-74 KB of LDS.
template <int D, int VM>
constexpr int kBlocksPerCU = (D == 64 && VM < 2) ? 3 : 2;


// Tiles 0 .. tiles-2, two per iteration so each buffer is a fixed LDS object; on return t is
// the last tile, whose K/V the DMA has been issued for (buffer t & 1).
template <bool PRE, class W, class LD, class TI>
__device__ __forceinline__ void body_tiles(W& w, const LD& ld, const AttnArgs& a, TI& t, uint8_t* lds0,
                                           uint8_t* lds1, uint8_t* meta0, uint8_t* meta1) {
  constexpr int KB = kTile * W::kD;
  const TI body = static_cast<TI>(a.tiles) - 1;
  for (; t + 2 <= body; t += 2) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    ld.issue(t + 1, lds1, lds1 + KB, meta1);
    w.template tile<false, PRE>(a, t, lds0, lds0 + KB, meta0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    ld.issue(t + 2, lds0, lds0 + KB, meta0);
    w.template tile<false, PRE>(a, t + 1, lds1, lds1 + KB, meta1);
  }
  if (t < body) {  // odd count of body tiles: one more from buffer 0, last tile lands in buffer 1
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    ld.issue(t + 1, lds1, lds1 + KB, meta1);
    w.template tile<false, PRE>(a, t, lds0, lds0 + KB, meta0);
    ++t;
  }
}

// One block's rows [row0, row0 + 64 * NQG) of head bh: 4 waves of 16 * NQG rows.
template <int D, int VM, bool DUMP, int OUT, int PM, int QF, int NQG>
__device__ __forceinline__ void attn_block(const AttnArgs& a, int64_t bh, int64_t row0, uint8_t* lds0, uint8_t* lds1,
                                           uint8_t* meta0, uint8_t* meta1, uint8_t* ring, uint8_t* vsring) {
  typedef TileLoader<D, VM, QF> LD;
  typedef Wave<D, VM, DUMP, PM, QF, NQG> W;
  constexpr int KB = kTile * D;
  constexpr int RING_BYTES = LD::RING ? LD::NR * LD::RS : 16;
  constexpr int VSRING_BYTES = LD::BSCALE ? LD::NR * LD::VS : 16;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  W w;
  w.G = lane >> 4;
  w.li = lane & 15;
  w.bh_ = bh;
  // Lane-constant LDS offsets.
#pragma unroll
  for (int ds = 0; ds < W::DS; ++ds) w.koff[ds] = w.li * D + ((((D == 128) ? 4 * ds : 0) + w.G) ^ chunk_xor<D>(w.li)) * 16;
#pragma unroll
  for (int h = 0; h < 2; ++h) w.voff[h] = w.li * kTile + (((4 * h + w.G) ^ (w.li & 7)) * 16);

  // Q fragments (B operand) and per-row scales.
#pragma unroll
  for (int qg = 0; qg < NQG; ++qg) {
    const int64_t r = row0 + wave * (16 * NQG) + qg * 16 + w.li;
    w.row[qg] = r;
    // Q scale: Sage per-thread INT8 index (row/16)*8 + row%8, or the FP8 row block row/64
    const int64_t si = QF == 1 ? r / 64 : (r / 16) * 8 + r % 8;
    w.qsv[qg] = si < a.qs_len ? a.qs[bh * a.qs_len + si] : 1.0f;
#pragma unroll
    for (int ds = 0; ds < W::DS; ++ds) {
      if (r < a.Nq) w.qf[qg][ds] = *reinterpret_cast<const v4i*>(a.q8 + (bh * a.Nq + r) * D + ds * 64 + w.G * 16);
      else w.qf[qg][ds] = v4i{0, 0, 0, 0};
    }
    w.m[qg] = -5000000.0f;
    w.den[qg] = 0.0f;
    w.dacc[qg] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    w.fbias[qg] = __builtin_fmaf(5000000.0f, kExpA, kExpB);
#pragma unroll
    for (int j = 0; j < 4; ++j) w.wts[qg][j] = 0.0f;
#pragma unroll
    for (int cb = 0; cb < W::CB; ++cb) w.O[qg][cb] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  }

  // Without block values the opaque copy keeps the compiler from rebuilding the constant
  // operand every tile; the smoothing variants have no registers to spare for it.
  w.ones = v4i{0x22222222, 0x22222222, 0x22222222, 0x22222222};
  if constexpr (VM == 0 && (D == 128 || PM == 2)) asm volatile("" : "+v"(w.ones));
  w.bacc = v4i{kBias, kBias, kBias, kBias};
  if constexpr (W::IB && VM == 0 && D == 128) asm volatile("" : "+v"(w.bacc));
  w.fold_ok = 0;
  if constexpr (PM == 2 && QF == 0) w.fold_precheck(a, lane);

  LD ld;
  ld.init(a, bh);
  if constexpr (LD::RING) {
    // The last chunk's flush reads ring slots of tiles past the last one (weight 0):
    // they must hold finite values, so the rings start zeroed.
    for (int i = threadIdx.x; i < RING_BYTES / 16; i += kThreadsPerBlock)
      reinterpret_cast<uint4*>(ring)[i] = make_uint4(0, 0, 0, 0);
    if constexpr (LD::BSCALE) {
      for (int i = threadIdx.x; i < VSRING_BYTES / 16; i += kThreadsPerBlock)
        reinterpret_cast<uint4*>(vsring)[i] = make_uint4(0, 0, 0, 0);
    }
    __syncthreads();
    ld.ring = ring;
    w.ring = ring;
    ld.vsring = vsring;
    w.vsring = vsring;
  }
  ld.issue(0, lds0, lds0 + KB, meta0);
  // Tiles before the last; a wave whose fold conditions were prechecked runs the copy of
  // the loop without the tests.
  // 32-bit tile index (tiles < 2^23), so the loop test stays on the scalar unit; the
  // per-block-scale variants keep 64 bits (with 32 their register allocation spills)
  typedef std::conditional_t<VM == 2, int64_t, int> TI;
  TI t = 0;
  if constexpr (PM == 2 && QF == 0) {
    if (w.fold_ok) body_tiles<true>(w, ld, a, t, lds0, lds1, meta0, meta1);
    else body_tiles<false>(w, ld, a, t, lds0, lds1, meta0, meta1);
  } else {
    body_tiles<false>(w, ld, a, t, lds0, lds1, meta0, meta1);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (t & 1) w.template tile<true>(a, t, lds1, lds1 + KB, meta1);
  else w.template tile<true>(a, t, lds0, lds0 + KB, meta0);

  // ---- epilogue: normalise, per-channel V scale, store 4 channels per lane and block
  const int64_t b = bh / a.H, h = bh % a.H;
#pragma unroll
  for (int qg = 0; qg < NQG; ++qg) {
    if (w.row[qg] >= a.Nq) continue;
    const float inv = 1.0f / (W::DACC ? w.dacc[qg][0] : w.den[qg]);
    uint16_t* out = static_cast<uint16_t*>(a.out) + b * a.osb + h * a.osh + w.row[qg] * a.osn;
#pragma unroll
    for (int cb = 0; cb < W::CB; ++cb) {
      const int ch = 16 * cb + 4 * w.G;
      // per-channel V scale (per-block scales were applied tile by tile)
      const float4 sc = W::BSCALE ? make_float4(1.0f, 1.0f, 1.0f, 1.0f)
                                                  : *reinterpret_cast<const float4*>(a.vs + bh * D + ch);
      const float y0 = w.O[qg][cb][0] * inv * sc.x, y1 = w.O[qg][cb][1] * inv * sc.y;
      const float y2 = w.O[qg][cb][2] * inv * sc.z, y3 = w.O[qg][cb][3] * inv * sc.w;
      uint2 packed;
      if constexpr (OUT == VCX_BFLOAT16) {
        packed.x = f32_to_bf16_bits(y0) | (f32_to_bf16_bits(y1) << 16);
        packed.y = f32_to_bf16_bits(y2) | (f32_to_bf16_bits(y3) << 16);
      } else {
        packed.x = f32_to_f16_bits(y0) | (f32_to_f16_bits(y1) << 16);
        packed.y = f32_to_f16_bits(y2) | (f32_to_f16_bits(y3) << 16);
      }
      *reinterpret_cast<uint2*>(out + ch) = packed;
    }
  }
}

template <int D, int VM, bool DUMP, int OUT, int PM, int QF = 0>
__global__ __launch_bounds__(kThreadsPerBlock, (kBlocksPerCU<D, VM>)) void attn_kernel(AttnArgs a) {
#if defined(__HIP_DEVICE_COMPILE__)  // device code; the host pass only emits the launch stub
  typedef TileLoader<D, VM, QF> LD;
  constexpr int KB = kTile * D, VB = D * kTile;
  __shared__ __attribute__((aligned(16))) uint8_t lds0[KB + VB];
  __shared__ __attribute__((aligned(16))) uint8_t lds1[KB + VB];
  __shared__ __attribute__((aligned(16))) uint8_t meta0[LD::META_BYTES];
  __shared__ __attribute__((aligned(16))) uint8_t meta1[LD::META_BYTES];
  constexpr int RING_BYTES = LD::RING ? LD::NR * LD::RS : 16;
  __shared__ __attribute__((aligned(16))) uint8_t ring[RING_BYTES];
  constexpr int VSRING_BYTES = LD::BSCALE ? LD::NR * LD::VS : 16;
  __shared__ __attribute__((aligned(16))) uint8_t vsring[VSRING_BYTES];

  // XCD-aware order: the hardware deals blocks round-robin over 8 XCDs; give each XCD a
  // contiguous range of (head, query block) so its L2 serves one head. The j-th block of XCD
  // x is the j-th entry of its list: the range's first n_x - kconv 128-row blocks, then each
  // of its last kconv blocks as two 64-row halves, so that the XCD's last round is made of
  // half-length pieces (the grid has nfull + 8 * kconv blocks; kconv <= nfull / 8).
  const int64_t p = blockIdx.x;
  const int64_t per = a.nfull / 8, rem = a.nfull % 8, xcd = p % 8, j = p / 8;
  const int64_t start = xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per;
  const int64_t nfx = per + (xcd < rem ? 1 : 0) - a.kconv;
  if (j < nfx) {
    const int64_t logical = start + j;
    const int64_t bh = logical / a.qblocks, qb = logical % a.qblocks;
    attn_block<D, VM, DUMP, OUT, PM, QF, 2>(a, bh, qb * kRowsPerBlock, lds0, lds1, meta0, meta1, ring, vsring);
  } else {
    const int64_t hj = j - nfx, logical = start + nfx + hj / 2;
    const int64_t bh = logical / a.qblocks, qb = logical % a.qblocks;
    attn_block<D, VM, DUMP, OUT, PM, QF, 1>(a, bh, qb * kRowsPerBlock + (hj & 1) * (kRowsPerBlock / 2), lds0, lds1,
                                           meta0, meta1, ring, vsring);
  }
#else
  (void)a;
#endif
}

// Explicit instantiation of every launch variant: hipcc's host pass otherwise
// emitted the kernel handle of only the first variant named in each ternary.
template __global__ void attn_kernel<64, 0, false, 0, 2>(AttnArgs);
template __global__ void attn_kernel<64, 0, false, 1, 2>(AttnArgs);
template __global__ void attn_kernel<64, 0, true, 0, 2>(AttnArgs);
template __global__ void attn_kernel<64, 0, true, 1, 2>(AttnArgs);
template __global__ void attn_kernel<128, 0, false, 0, 2>(AttnArgs);
template __global__ void attn_kernel<128, 0, false, 1, 2>(AttnArgs);
template __global__ void attn_kernel<128, 0, true, 0, 2>(AttnArgs);
template __global__ void attn_kernel<128, 0, true, 1, 2>(AttnArgs);
template __global__ void attn_kernel<64, 0, false, 0, 1>(AttnArgs);
template __global__ void attn_kernel<64, 0, false, 1, 1>(AttnArgs);
template __global__ void attn_kernel<64, 0, true, 0, 1>(AttnArgs);
template __global__ void attn_kernel<64, 0, true, 1, 1>(AttnArgs);
template __global__ void attn_kernel<64, 1, false, 0, 1>(AttnArgs);
template __global__ void attn_kernel<64, 1, false, 1, 1>(AttnArgs);
template __global__ void attn_kernel<64, 1, true, 0, 1>(AttnArgs);
template __global__ void attn_kernel<64, 1, true, 1, 1>(AttnArgs);
template __global__ void attn_kernel<64, 2, false, 0, 1>(AttnArgs);
template __global__ void attn_kernel<64, 2, false, 1, 1>(AttnArgs);
template __global__ void attn_kernel<64, 2, true, 0, 1>(AttnArgs);
template __global__ void attn_kernel<64, 2, true, 1, 1>(AttnArgs);
template __global__ void attn_kernel<128, 0, false, 0, 1>(AttnArgs);
template __global__ void attn_kernel<128, 0, false, 1, 1>(AttnArgs);
template __global__ void attn_kernel<128, 0, true, 0, 1>(AttnArgs);
template __global__ void attn_kernel<128, 0, true, 1, 1>(AttnArgs);
template __global__ void attn_kernel<128, 1, false, 0, 1>(AttnArgs);
template __global__ void attn_kernel<128, 1, false, 1, 1>(AttnArgs);
template __global__ void attn_kernel<128, 1, true, 0, 1>(AttnArgs);
template __global__ void attn_kernel<128, 1, true, 1, 1>(AttnArgs);
template __global__ void attn_kernel<128, 2, false, 0, 1>(AttnArgs);
template __global__ void attn_kernel<128, 2, false, 1, 1>(AttnArgs);
template __global__ void attn_kernel<128, 2, true, 0, 1>(AttnArgs);
template __global__ void attn_kernel<128, 2, true, 1, 1>(AttnArgs);
template __global__ void attn_kernel<64, 0, false, 0, 0>(AttnArgs);
template __global__ void attn_kernel<64, 0, false, 1, 0>(AttnArgs);
template __global__ void attn_kernel<64, 0, true, 0, 0>(AttnArgs);
template __global__ void attn_kernel<64, 0, true, 1, 0>(AttnArgs);
template __global__ void attn_kernel<64, 1, false, 0, 0>(AttnArgs);
template __global__ void attn_kernel<64, 1, false, 1, 0>(AttnArgs);
template __global__ void attn_kernel<64, 1, true, 0, 0>(AttnArgs);
template __global__ void attn_kernel<64, 1, true, 1, 0>(AttnArgs);
template __global__ void attn_kernel<64, 2, false, 0, 0>(AttnArgs);
template __global__ void attn_kernel<64, 2, false, 1, 0>(AttnArgs);
template __global__ void attn_kernel<64, 2, true, 0, 0>(AttnArgs);
template __global__ void attn_kernel<64, 2, true, 1, 0>(AttnArgs);
template __global__ void attn_kernel<128, 0, false, 0, 0>(AttnArgs);
template __global__ void attn_kernel<128, 0, false, 1, 0>(AttnArgs);
template __global__ void attn_kernel<128, 0, true, 0, 0>(AttnArgs);
template __global__ void attn_kernel<128, 0, true, 1, 0>(AttnArgs);
template __global__ void attn_kernel<128, 1, false, 0, 0>(AttnArgs);
template __global__ void attn_kernel<128, 1, false, 1, 0>(AttnArgs);
template __global__ void attn_kernel<128, 1, true, 0, 0>(AttnArgs);
template __global__ void attn_kernel<128, 1, true, 1, 0>(AttnArgs);
template __global__ void attn_kernel<128, 2, false, 0, 0>(AttnArgs);
template __global__ void attn_kernel<128, 2, false, 1, 0>(AttnArgs);
template __global__ void attn_kernel<128, 2, true, 0, 0>(AttnArgs);
template __global__ void attn_kernel<128, 2, true, 1, 0>(AttnArgs);

template __global__ void attn_kernel<64, 0, false, 0, 2, 1>(AttnArgs);
template __global__ void attn_kernel<64, 0, false, 1, 2, 1>(AttnArgs);
template __global__ void attn_kernel<64, 0, true, 0, 2, 1>(AttnArgs);
template __global__ void attn_kernel<64, 0, true, 1, 2, 1>(AttnArgs);
template __global__ void attn_kernel<128, 0, false, 0, 2, 1>(AttnArgs);
template __global__ void attn_kernel<128, 0, false, 1, 2, 1>(AttnArgs);
template __global__ void attn_kernel<128, 0, true, 0, 2, 1>(AttnArgs);
template __global__ void attn_kernel<128, 0, true, 1, 2, 1>(AttnArgs);
template __global__ void attn_kernel<64, 0, false, 0, 1, 1>(AttnArgs);
template __global__ void attn_kernel<64, 0, false, 1, 1, 1>(AttnArgs);
template __global__ void attn_kernel<64, 0, true, 0, 1, 1>(AttnArgs);
template __global__ void attn_kernel<64, 0, true, 1, 1, 1>(AttnArgs);
template __global__ void attn_kernel<128, 0, false, 0, 1, 1>(AttnArgs);
template __global__ void attn_kernel<128, 0, false, 1, 1, 1>(AttnArgs);
template __global__ void attn_kernel<128, 0, true, 0, 1, 1>(AttnArgs);
template __global__ void attn_kernel<128, 0, true, 1, 1, 1>(AttnArgs);
template __global__ void attn_kernel<64, 0, false, 0, 0, 1>(AttnArgs);
template __global__ void attn_kernel<64, 0, false, 1, 0, 1>(AttnArgs);
template __global__ void attn_kernel<64, 0, true, 0, 0, 1>(AttnArgs);
template __global__ void attn_kernel<64, 0, true, 1, 0, 1>(AttnArgs);
template __global__ void attn_kernel<128, 0, false, 0, 0, 1>(AttnArgs);
template __global__ void attn_kernel<128, 0, false, 1, 0, 1>(AttnArgs);
template __global__ void attn_kernel<128, 0, true, 0, 0, 1>(AttnArgs);
template __global__ void attn_kernel<128, 0, true, 1, 0, 1>(AttnArgs);

// Makespan, in units of one 128-row block's time, of one XCD's block list on S slots served
// in list order, each block to the slot that frees first: n - k full blocks, then 2k halves
// of relative length h.
double list_makespan(int64_t n, int64_t k, int S, double h) {
  std::vector<double> slot(static_cast<size_t>(S), 0.0);
  const int64_t nf = n - k, r = nf / S, f = nf % S;
  for (int i = 0; i < S; ++i) slot[static_cast<size_t>(i)] = static_cast<double>(r + (i < f ? 1 : 0));
  std::make_heap(slot.begin(), slot.end(), std::greater<double>());
  for (int64_t i = 0; i < 2 * k; ++i) {
    std::pop_heap(slot.begin(), slot.end(), std::greater<double>());
    slot.back() += h;
    std::push_heap(slot.begin(), slot.end(), std::greater<double>());
  }
  return *std::max_element(slot.begin(), slot.end());
}

// Relative length of a 64-row block: half the MFMA and encode work, the same K/V streaming.
constexpr double kHalfBlockTime = 0.6;

// How many of each XCD's last 128-row blocks run as two 64-row blocks: the k in [0, min(nfull/8,
// 2 S)] with the smallest modelled makespan of the fullest XCD (the smallest such k), S = the
// XCD's block slots (CUs / 8 x blocks per CU). Cached per (nfull, S).
int64_t tail_split(int64_t nfull, int blocks_per_cu) {
  static std::mutex mu;
  static std::map<std::pair<int64_t, int>, int64_t> cache;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus < 8)
    return 0;
  const int S = cus / 8 * blocks_per_cu;
  std::lock_guard<std::mutex> lock(mu);
  const auto key = std::make_pair(nfull, S);
  const auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  const int64_t per = nfull / 8, n = per + (nfull % 8 ? 1 : 0);
  int64_t best = 0;
  double best_t = list_makespan(n, 0, S, kHalfBlockTime);
  for (int64_t k = 1; k <= std::min<int64_t>(per, 2 * S); ++k) {
    const double t = list_makespan(n, k, S, kHalfBlockTime);
    if (t < best_t - 1e-9) { best_t = t; best = k; }
  }
  if (cache.size() >= 4096) cache.clear();  // a serving process sees a bounded set of shapes; stay small
  cache.emplace(key, best);
  return best;
}

template <int D, int VM, bool DUMP, int OUT, int PM, int QF>
int launch(const AttnArgs& a, hipStream_t st) {
  AttnArgs b = a;
  b.kconv = tail_split(a.nfull, kBlocksPerCU<D, VM>);
  const int64_t grid = b.nfull + 8 * b.kconv;
  attn_kernel<D, VM, DUMP, OUT, PM, QF><<<dim3(static_cast<unsigned>(grid)), kThreadsPerBlock, 0, st>>>(b);
  return check_launch("attn_kernel");
}

template <int D, int VM, int PM, int QF>
int launch_out(const AttnArgs& a, bool dump, int out_dtype, hipStream_t st) {
  if (dump) {
    return out_dtype == VCX_BFLOAT16 ? launch<D, VM, true, VCX_BFLOAT16, PM, QF>(a, st)
                                     : launch<D, VM, true, VCX_FLOAT16, PM, QF>(a, st);
  }
  return out_dtype == VCX_BFLOAT16 ? launch<D, VM, false, VCX_BFLOAT16, PM, QF>(a, st)
                                   : launch<D, VM, false, VCX_FLOAT16, PM, QF>(a, st);
}

template <int D, int VM, int QF = 0>
int launch_mode(const AttnArgs& a, bool dump, int out_dtype, int mode, hipStream_t st) {
  if constexpr (VM == 0) {
    if (mode == 2) return launch_out<D, VM, 2, QF>(a, dump, out_dtype, st);
  }
  return mode == 1 ? launch_out<D, VM, 1, QF>(a, dump, out_dtype, st)
                   : launch_out<D, VM, 0, QF>(a, dump, out_dtype, st);
}

// Argument checks shared by the INT8 and FP8 block entry points.
int check_common(int64_t B, int64_t H, int64_t Nq, int64_t Nk, int64_t D, int expcast, int out_dtype,
                 float sm_scale, void* out, int64_t o_sb, int64_t o_sh, int64_t o_sn, const uint8_t* p_dump,
                 int64_t p_row_begin, int64_t p_row_end) {
  VCX_REQUIRE(B >= 1 && H >= 1 && Nq >= 1 && Nk >= 1, "B, H, Nq, Nk must be positive");
  VCX_REQUIRE(D == 64 || D == 128, "D must be 64 or 128");
  VCX_REQUIRE(B * H <= 65535, "B*H exceeds 65535");
  VCX_REQUIRE(Nq < (int64_t(1) << 30) && Nk < (int64_t(1) << 30), "sequence too long");
  VCX_REQUIRE(cdiv(Nk, kTile) * kTile * D < (int64_t(1) << 31), "K/V payload of one head must be below 2 GiB");
  VCX_REQUIRE(expcast >= 0 && expcast <= 2, "expcast must be 0, 1 or 2");
  VCX_REQUIRE(out_dtype == VCX_FLOAT16 || out_dtype == VCX_BFLOAT16, "out_dtype must be float16 or bfloat16");
  VCX_REQUIRE(std::isfinite(sm_scale) && sm_scale > 0.0f, "sm_scale must be positive and finite FP32");
  VCX_REQUIRE(aligned(out, 8) && o_sb % 4 == 0 && o_sh % 4 == 0 && o_sn % 4 == 0 && o_sn >= D && o_sb >= 0 &&
                  o_sh >= 0,
              "out must be 8-byte aligned with strides that are multiples of 4 elements and sn >= D");
  if (p_dump) {
    VCX_REQUIRE(p_row_begin >= 0 && p_row_begin < p_row_end && p_row_end <= Nq, "invalid P dump row range");
  }
  return VCX_OK;
}

}  // namespace
}  // namespace vcx

using namespace vcx;

extern "C" int vcx_attention_fwd(const int8_t* q8, const int8_t* k8, const uint8_t* v8, const float* qs,
                                 const float* ks, const float* vs, const uint16_t* means, int64_t B,
                                 int64_t H, int64_t Nq, int64_t Nk, int64_t D, int expcast,
                                 int block_values, int channel_scale, float sm_scale, int out_dtype,
                                 void* out, int64_t o_sb, int64_t o_sh, int64_t o_sn, uint8_t* p_dump,
                                 int64_t p_row_begin, int64_t p_row_end, void* stream) {
  if (int rc = check_common(B, H, Nq, Nk, D, expcast, out_dtype, sm_scale, out, o_sb, o_sh, o_sn, p_dump,
                            p_row_begin, p_row_end))
    return rc;
  VCX_REQUIRE(expcast != 2 || !block_values, "the folded ExpCast encode (expcast = 2) is defined without block values");
  VCX_REQUIRE(block_values || channel_scale, "per-block V scales require block values (smoothing)");
  VCX_REQUIRE(q8 && k8 && v8 && qs && ks && vs && out, "null tensor pointer");
  VCX_REQUIRE(!block_values || means, "means must be non-null with block values");
  VCX_REQUIRE(aligned(q8, 16) && aligned(k8, 16) && aligned(v8, 16), "q8/k8/v8 must be 16-byte aligned");
  VCX_REQUIRE(aligned(qs, 4) && aligned(ks, 4) && aligned(vs, 16), "scale pointer alignment (vs needs 16 bytes)");
  VCX_REQUIRE(!block_values || aligned(means, 8), "means must be 8-byte aligned");
  AttnArgs a{};
  a.q8 = q8; a.k8 = k8; a.v8 = v8; a.qs = qs; a.ks = ks; a.vs = vs; a.means = means; a.out = out;
  a.osb = o_sb; a.osh = o_sh; a.osn = o_sn;
  a.H = H; a.Nq = Nq; a.Nk = Nk; a.tiles = cdiv(Nk, kTile); a.qblocks = cdiv(Nq, kRowsPerBlock);
  a.qs_len = cdiv(Nq, 64) * 32;
  // The control path works in the log2 domain: RN(sm * RN(log2 e)) (sal/csrc/vc/vc_sm90.cu:177).
  a.sm = expcast != 0 ? sm_scale : sm_scale * 1.4426950408889634f;
  a.pdump = p_dump; a.prow0 = p_row_begin; a.prow1 = p_row_end;
  const int64_t nblocks = B * H * a.qblocks;
  VCX_REQUIRE(nblocks < (int64_t(1) << 30), "too many blocks");
  a.nfull = nblocks;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool dump = p_dump != nullptr;
  if (D == 128) {
    if (!block_values) return launch_mode<128, 0>(a, dump, out_dtype, expcast, st);
    return channel_scale ? launch_mode<128, 1>(a, dump, out_dtype, expcast, st)
                         : launch_mode<128, 2>(a, dump, out_dtype, expcast, st);
  }
  if (!block_values) return launch_mode<64, 0>(a, dump, out_dtype, expcast, st);
  return channel_scale ? launch_mode<64, 1>(a, dump, out_dtype, expcast, st)
                       : launch_mode<64, 2>(a, dump, out_dtype, expcast, st);
}

extern "C" int vcx_attention_fwd_fp8(const uint8_t* q8, const uint8_t* k8, const uint8_t* v8, const float* qs,
                                     const float* ks, const float* vs, int64_t B, int64_t H, int64_t Nq,
                                     int64_t Nk, int64_t D, int expcast, float sm_scale, int out_dtype, void* out,
                                     int64_t o_sb, int64_t o_sh, int64_t o_sn, uint8_t* p_dump,
                                     int64_t p_row_begin, int64_t p_row_end, void* stream) {
  if (int rc = check_common(B, H, Nq, Nk, D, expcast, out_dtype, sm_scale, out, o_sb, o_sh, o_sn, p_dump,
                            p_row_begin, p_row_end))
    return rc;
  VCX_REQUIRE(q8 && k8 && v8 && qs && ks && vs && out, "null tensor pointer");
  VCX_REQUIRE(aligned(q8, 16) && aligned(k8, 16) && aligned(v8, 16), "q8/k8/v8 must be 16-byte aligned");
  VCX_REQUIRE(aligned(qs, 4) && aligned(ks, 4) && aligned(vs, 16), "scale pointer alignment (vs needs 16 bytes)");
  AttnArgs a{};
  a.q8 = reinterpret_cast<const int8_t*>(q8); a.k8 = reinterpret_cast<const int8_t*>(k8); a.v8 = v8;
  a.qs = qs; a.ks = ks; a.vs = vs; a.means = nullptr; a.out = out;
  a.osb = o_sb; a.osh = o_sh; a.osn = o_sn;
  a.H = H; a.Nq = Nq; a.Nk = Nk; a.tiles = cdiv(Nk, kTile); a.qblocks = cdiv(Nq, kRowsPerBlock);
  a.qs_len = cdiv(Nq, 64);
  a.sm = expcast != 0 ? sm_scale : sm_scale * 1.4426950408889634f;
  a.pdump = p_dump; a.prow0 = p_row_begin; a.prow1 = p_row_end;
  const int64_t nblocks = B * H * a.qblocks;
  VCX_REQUIRE(nblocks < (int64_t(1) << 30), "too many blocks");
  a.nfull = nblocks;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool dump = p_dump != nullptr;
  return D == 128 ? launch_mode<128, 0, 1>(a, dump, out_dtype, expcast, st)
                  : launch_mode<64, 0, 1>(a, dump, out_dtype, expcast, st);
}

namespace vcx {
namespace {
// One thread per four inputs: the control path's probability bytes via fp8_exp2_word
// (SAT: the saturating lower neighbours the fused kernel uses; else the 64-bit pair form).
template <bool SAT>
__global__ void fp8_exp2_probe_kernel(const float* x, uint8_t* y, int64_t n) {
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
  if (i >= n) return;
  float xs[4], pr[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    xs[r] = i + r < n ? x[i + r] : -INFINITY;
    pr[r] = __builtin_amdgcn_exp2f(xs[r]);
  }
  const uint32_t w = fp8_exp2_word<SAT>(xs, pr);
#pragma unroll
  for (int r = 0; r < 4; ++r)
    if (i + r < n) y[i + r] = static_cast<uint8_t>(w >> (8 * r));
}
}  // namespace
}  // namespace vcx

extern "C" int vcx_fp8_exp2_codes(const float* x, uint8_t* y, int64_t n, int form, void* stream) {
  VCX_REQUIRE(n >= 0 && (n == 0 || (x != nullptr && y != nullptr)), "invalid probe arguments");
  VCX_REQUIRE(form == 0 || form == 1, "form must be 0 or 1");
  VCX_REQUIRE(aligned(x, 4), "x must be 4-byte aligned");
  if (n == 0) return VCX_OK;
  const int64_t threads = cdiv(n, 4), blocks = cdiv(threads, 256);
  VCX_REQUIRE(blocks < (int64_t(1) << 31), "n too large");
  if (form) fp8_exp2_probe_kernel<true><<<dim3(static_cast<unsigned>(blocks)), 256, 0, static_cast<hipStream_t>(stream)>>>(x, y, n);
  else fp8_exp2_probe_kernel<false><<<dim3(static_cast<unsigned>(blocks)), 256, 0, static_cast<hipStream_t>(stream)>>>(x, y, n);
  return check_launch("fp8_exp2_probe_kernel");
}

namespace {
int resources_of(const void* fn, int64_t* out) {
  hipFuncAttributes attr{};
  hipError_t e = hipFuncGetAttributes(&attr, fn);
  if (e != hipSuccess) return fail(VCX_EHIP, "hipFuncGetAttributes: %s", hipGetErrorString(e));
  out[0] = attr.numRegs;
  out[1] = 0;
  out[2] = static_cast<int64_t>(attr.sharedSizeBytes);
  out[3] = 0;
  out[4] = attr.maxThreadsPerBlock;
  out[5] = static_cast<int64_t>(attr.localSizeBytes);
  return VCX_OK;
}
}  // namespace

extern "C" int vcx_kernel_resources(int64_t D, int block_values, int64_t* out) {
  VCX_REQUIRE(out != nullptr, "out is null");
  VCX_REQUIRE(D == 64 || D == 128, "D must be 64 or 128");
  const void* fn;
  if (D == 128) fn = block_values ? reinterpret_cast<const void*>(&attn_kernel<128, 1, false, VCX_BFLOAT16, 1>)
                                  : reinterpret_cast<const void*>(&attn_kernel<128, 0, false, VCX_BFLOAT16, 2>);
  else fn = block_values ? reinterpret_cast<const void*>(&attn_kernel<64, 1, false, VCX_BFLOAT16, 1>)
                         : reinterpret_cast<const void*>(&attn_kernel<64, 0, false, VCX_BFLOAT16, 2>);
  return resources_of(fn, out);
}

namespace {
template <int D, int VM, int PM, int OUT>
const void* kernel_of() { return reinterpret_cast<const void*>(&attn_kernel<D, VM, false, OUT, PM>); }

template <int D, int OUT>
const void* kernel_of(int vm, int pm) {
  if (vm == 0) return pm == 2 ? kernel_of<D, 0, 2, OUT>() : pm == 1 ? kernel_of<D, 0, 1, OUT>() : kernel_of<D, 0, 0, OUT>();
  if (vm == 1) return pm == 1 ? kernel_of<D, 1, 1, OUT>() : kernel_of<D, 1, 0, OUT>();
  return pm == 1 ? kernel_of<D, 2, 1, OUT>() : kernel_of<D, 2, 0, OUT>();
}
}  // namespace

extern "C" int vcx_kernel_resources_mode(int64_t D, int value_mode, int expcast, int out_dtype, int64_t* out) {
  VCX_REQUIRE(out != nullptr, "out is null");
  VCX_REQUIRE(D == 64 || D == 128, "D must be 64 or 128");
  VCX_REQUIRE(value_mode >= 0 && value_mode <= 2, "value_mode must be 0, 1 or 2");
  VCX_REQUIRE(expcast >= 0 && expcast <= 2, "expcast must be 0, 1 or 2");
  VCX_REQUIRE(expcast != 2 || value_mode == 0, "the folded ExpCast encode (expcast = 2) is defined without block values");
  VCX_REQUIRE(out_dtype == VCX_FLOAT16 || out_dtype == VCX_BFLOAT16, "out_dtype must be float16 or bfloat16");
  const void* fn = D == 128 ? (out_dtype == VCX_BFLOAT16 ? kernel_of<128, VCX_BFLOAT16>(value_mode, expcast)
                                                         : kernel_of<128, VCX_FLOAT16>(value_mode, expcast))
                            : (out_dtype == VCX_BFLOAT16 ? kernel_of<64, VCX_BFLOAT16>(value_mode, expcast)
                                                         : kernel_of<64, VCX_FLOAT16>(value_mode, expcast));
  if (int rc = resources_of(fn, out)) return rc;
  int blocks = 0;
  hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, fn, kThreadsPerBlock, 0);
  if (e != hipSuccess) return fail(VCX_EHIP, "hipOccupancyMaxActiveBlocksPerMultiprocessor: %s", hipGetErrorString(e));
  out[6] = blocks;
  return VCX_OK;
}

extern "C" int vcx_kernel_resources_fp8(int64_t D, int expcast, int64_t* out) {
  VCX_REQUIRE(out != nullptr, "out is null");
  VCX_REQUIRE(D == 64 || D == 128, "D must be 64 or 128");
  const void* fn;
  if (D == 128) fn = expcast ? reinterpret_cast<const void*>(&attn_kernel<128, 0, false, VCX_BFLOAT16, 2, 1>)
                             : reinterpret_cast<const void*>(&attn_kernel<128, 0, false, VCX_BFLOAT16, 0, 1>);
  else fn = expcast ? reinterpret_cast<const void*>(&attn_kernel<64, 0, false, VCX_BFLOAT16, 2, 1>)
                    : reinterpret_cast<const void*>(&attn_kernel<64, 0, false, VCX_BFLOAT16, 0, 1>);
  return resources_of(fn, out);
}
