// V grouping on gfx950: deterministic Lloyd clustering (1..256 centers per head) and a
// stable counting sort of the labels, as in the reference's grouping
// (third_party/sageattention_local/csrc/vc/clustering.cu:21-167 for at most 8 clusters,
// pybind.cpp:6-44 for the wider range and the legacy entry point).
//
// Contract (identical in oracle/vc_oracle.c vco_group_values_ex):
//   count = min(clusters, n); centers = centers_in, or V[ids] as fp32 with
//   ids = trunc(fp32 linspace(0, n-1, count));
//   distance = sum over d (sequential) of fma(x_d - c_d, x_d - c_d, acc) in fp64,
//   argmin with ties to the lowest id; every iteration but the last replaces every
//   non-empty center by RN_f32(fp64 sum / count), the sum taken sequentially over the
//   cluster's tokens inside each 128-token tile and then sequentially over tiles;
//   perm = stable sort of tokens by label; centers_next = that same update applied to
//   the final labels (the warm start of the next refresh).
//
// Two schedules, bit-identical where both apply:
//   fused   (count <= 8): the assignment kernel also forms per-(tile, cluster) fp64 sums
//           over ballot-built token lists; a second kernel adds them over tiles.
//   general (any count, and every count under mode 1): the assignment kernel counts
//           labels per tile in LDS; the labels are sorted, and the update walks each
//           cluster's sorted token list (tokens ascending), closing a partial sum at each
//           tile boundary. Tiles without the cluster contribute +0.0 to the fused sum,
//           which leaves it unchanged (partial sums start at +0.0 and are never -0.0), so
//           both schedules add the same values in the same order.
#include "vcx_common.hpp"

#include <type_traits>

namespace vcx {
namespace {

constexpr int kFusedClusters = 8;  // the fused schedule's center slots per head
constexpr int kMaxClusters = 256;
constexpr int kGroupThreads = 128;  // one thread per token of a 128-token tile

struct Ids {
  int32_t v[kMaxClusters];
};

// A workgroup barrier that orders LDS accesses only. __syncthreads() also waits for every
// outstanding global load of the wave, which would drain the next tile's loads at each
// barrier of the current tile. The assignment kernel shares data between its threads
// through LDS alone.
__device__ inline void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Whether an assignment block runs a run of tiles, loading the next tile during the
// current one (else one tile per block).
constexpr bool assign_prefetch(int dt, bool general, bool wide) { return !general && dt == VCX_BFLOAT16 && wide; }

typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

__device__ inline const uint16_t* head_ptr(const void* x, int64_t bh, int64_t H, int64_t sb, int64_t sh) {
  return reinterpret_cast<const uint16_t*>(x) + (bh / H) * sb + (bh % H) * sh;
}

// The fused schedule's centers also in the form its bf16 dot-product pre-pass reads: each
// fp32 value c as two bf16 parts, hi = RN_bf16(c) and lo = RN_bf16(c - hi) (the
// subtraction is exact; |c - hi| <= 2^-8 |c| and, unless c - hi is a power of two (then lo
// takes it exactly), c - hi lies below 2^(e-8) for 2^e <= |c|, so lo leaves at most half its
// ulp, 2^(e-17)): |c - hi - lo| <= 2^-17 |c|; parts [BH][8][2][D] (bf16 bits);
// and the norms |c|^2 [BH][8], RN_f32 of the fp64 sum of the D squares (each exact; the
// summation order is free: only its error bound, far below 2^-24 relative, enters the
// pre-pass).
struct CenterForms {
  uint16_t* parts;
  float* norms;
};

__device__ inline void store_center_parts(float x, int64_t slot, int d, int D, const CenterForms& f) {
  const uint32_t hi = f32_to_bf16_bits(x);
  f.parts[slot * 2 * D + d] = static_cast<uint16_t>(hi);
  f.parts[slot * 2 * D + D + d] = static_cast<uint16_t>(f32_to_bf16_bits(__fsub_rn(x, bf16_bits_to_f32(hi))));
}

// One wave's sum of x^2 (fp64, a butterfly: the order is free), left in every lane.
__device__ inline double wave_square_sum(float x) {
  double q = static_cast<double>(x) * static_cast<double>(x);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) q += __shfl_xor(q, o, 64);
  return q;
}

// Open tokens of the bf16 pre-pass, resolved by the whole wave. cl: the head's 8 binary32
// centers, channel-major ([D][8]).
//
// wave_row_b32: the 8 binary32 distances of one staged row; lane (c = lane / 8, s = lane % 8)
// forms the sum over channels [s D/8, (s + 1) D/8) of fma(x_d - c_d, x_d - c_d, acc), and
// three butterfly additions give every lane of cluster c the same total. Every term is
// non-negative, so in any order each distance lies within 2 * 130 * 2^-24 relative of the
// exact one (each term passes at most D/8 + 3 + 2 roundings), and a second smallest above
// kOrder times the smallest settles the argmin, as in the per-thread chains. Returns whether
// it is settled, with the argmin (ties to the lowest id) in lab.
template <int DT, int D>
__device__ bool wave_row_b32(const uint16_t* row, const float* cl, int count, int lane, int& lab) {
  constexpr int CH = D / 8;
  const int c = lane >> 3, s = lane & 7;
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < CH / 8; ++i) {
    const uint4 q = *reinterpret_cast<const uint4*>(row + s * CH + 8 * i);
    const uint32_t wq[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int d = s * CH + 8 * i + 2 * k;
      const float d0 = __fsub_rn(in_to_f32<DT>(wq[k] & 0xffffu), cl[d * kFusedClusters + c]);
      acc = __fmaf_rn(d0, d0, acc);
      const float d1 = __fsub_rn(in_to_f32<DT>(wq[k] >> 16), cl[(d + 1) * kFusedClusters + c]);
      acc = __fmaf_rn(d1, d1, acc);
    }
  }
  // a + b and b + a are the same value, so both lanes of each pair hold the same sum
  acc = __fadd_rn(acc, __shfl_xor(acc, 1, 64));
  acc = __fadd_rn(acc, __shfl_xor(acc, 2, 64));
  acc = __fadd_rn(acc, __shfl_xor(acc, 4, 64));
  float b32 = INFINITY, s32 = INFINITY;
  lab = 0;
  bool finite = true;  // a NaN distance fails every compare below
#pragma unroll
  for (int k = 0; k < kFusedClusters; ++k) {
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), 8 * k));
    if (k < count) {
      finite = finite && a >= 0.0f;
      if (a < b32) {  // ties keep the lowest id (and make the order unsure)
        s32 = b32;
        b32 = a;
        lab = k;
      } else if (a < s32) {
        s32 = a;
      }
    }
  }
  constexpr float kOrder = 1.0f + 4.0e-5f;  // > (1 + e) / (1 - e), e = 130 * 2^-24
  return finite && s32 > b32 * kOrder + 1.0e-37f;
}

// wave_rows_b64: the contract's fp64 chains for up to 8 open rows at once, taken from open
// in token order (and cleared there). Lane (j = lane / 8, c = lane % 8) runs row j's chain
// for cluster c: distance_c = sum over d (in order) of fma(x_d - c_d, x_d - c_d, acc), the
// centers the exact widenings of the binary32 ones. The label is the first strict minimum
// from +inf (NaN and infinite distances never win; no finite distance keeps label 0), i.e. the
// smallest (value, id) pair with every such distance and every slot past count read as +inf:
// a butterfly over the 8 lanes of a row, the same in each. Lane t of the wave takes the label
// of its own token.
template <int DT, int D, int kStride>
__device__ void wave_rows_b64(const uint16_t* xs, int row0, uint64_t& open, const float* cl, int count, int lane,
                              int& best) {
  int rows[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    rows[j] = open ? __builtin_ctzll(open) : -1;
    open &= open - 1;
  }
  const int j = lane >> 3, c = lane & 7;
  int t = -1;
#pragma unroll
  for (int k = 0; k < 8; ++k)
    if (j == k) t = rows[k];
  double a = INFINITY;
  if (t >= 0) {
    const uint16_t* row = xs + (row0 + t) * kStride;
    a = 0.0;
#pragma unroll 1
    for (int i = 0; i < D / 8; ++i) {
      const uint4 q = *reinterpret_cast<const uint4*>(row + 8 * i);
      const uint32_t wq[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int d = 8 * i + 2 * k;
        const double d0 = __dsub_rn(static_cast<double>(in_to_f32<DT>(wq[k] & 0xffffu)),
                                    static_cast<double>(cl[d * kFusedClusters + c]));
        a = __fma_rn(d0, d0, a);
        const double d1 = __dsub_rn(static_cast<double>(in_to_f32<DT>(wq[k] >> 16)),
                                    static_cast<double>(cl[(d + 1) * kFusedClusters + c]));
        a = __fma_rn(d1, d1, a);
      }
    }
  }
  double v = (c < count && a < INFINITY) ? a : INFINITY;
  int id = c;
#pragma unroll
  for (int m = 1; m < 8; m <<= 1) {
    const double ov = __shfl_xor(v, m, 64);
    const int oid = __shfl_xor(id, m, 64);
    if (ov < v || (ov == v && oid < id)) {
      v = ov;
      id = oid;
    }
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int lab = __builtin_amdgcn_readlane(id, 8 * k);
    if (lane == rows[k]) best = lab;
  }
}

// Centers are kept as fp32 (the contract's values) and as their exact fp64 widening,
// which the assignment reads with wave-uniform (scalar) loads. Slots are CS per head
// (CS = 8 for the fused schedule, count rounded up to 8 for the general one); slots at or
// past count hold zeros. Initial values: centers_in [BH][count][D], else V[ids].
template <int DT>
__global__ void grp_init_kernel(const void* v, int64_t H, int64_t sb, int64_t sh, int64_t sn, Ids ids,
                                int count, int CS, int D, const float* centers_in, float* centers,
                                double* centers64, CenterForms forms) {
  __shared__ double red[kFusedClusters][128];  // squares, for the norms (CS = 8 with forms)
  const int64_t bh = blockIdx.x;
  const uint16_t* base = head_ptr(v, bh, H, sb, sh);
  const int d = threadIdx.x;
  for (int c = 0; c < CS; ++c) {
    float x = 0.0f;
    if (c < count) x = centers_in ? centers_in[(bh * count + c) * D + d] : in_to_f32<DT>(base[ids.v[c] * sn + d]);
    centers[(bh * CS + c) * D + d] = x;
    centers64[(bh * CS + c) * D + d] = static_cast<double>(x);
    if (forms.parts) {
      store_center_parts(x, bh * CS + c, d, D, forms);
      red[c][d] = static_cast<double>(x) * static_cast<double>(x);
    }
  }
  if (forms.parts) {
    __syncthreads();
    if (d < CS) {  // thread c sums cluster c's squares (the order is free)
      double q = 0.0;
      for (int i = 0; i < D; ++i) q += red[d][i];
      forms.norms[bh * CS + d] = static_cast<float>(q);
    }
  }
}

// grid (tiles, B*H), 128 threads. Assign every token of the tile and write the tile's
// per-cluster counts (pcnt, CS slots per tile). Fused schedule (!GENERAL, count <= 8):
// with STATS also the tile's per-cluster fp64 channel sums. General schedule: counts from
// an LDS histogram.
// The tile is staged through LDS with coalesced loads. On bf16 rows the fused schedule
// first runs a dot-product pre-pass on the MFMA. Where that does not settle a token, each
// thread reads its token's row 16 bytes at a time and runs the distance chains of 8
// clusters side by side (d outermost), chunk after chunk of 8 centers, in binary32 and,
// where that does not settle the argmin either, in fp64. The fused schedule's binary32
// centers sit in LDS channel-major at D64 and behind the bf16 pre-pass, and come through
// broadcast reads (as scalar operands, 8 centers x 16 channels outgrew the SGPRs and
// spilled into VGPR lanes); the fp16 D128 fused schedule, the general schedule and their
// fp64 chains read them through scalar loads.
template <int DT, int D, bool STATS, bool WIDE, bool GENERAL>
__global__ __launch_bounds__(kGroupThreads) void grp_assign_kernel(
    const void* v, int64_t H, int64_t n, int64_t sb, int64_t sh, int64_t sn, int count, int CS,
    const float* __restrict__ centers32, const double* __restrict__ centers64, CenterForms forms,
    int32_t* labels, double* psum, int32_t* pcnt, int64_t tiles, int64_t items, int64_t per) {
  constexpr int kStride = D + 8;  // 16-bit elements per staged row (16-byte aligned rows)
  constexpr bool FS = STATS && !GENERAL;  // per-cluster sums: one more row, of zeros (padding)
  __shared__ __attribute__((aligned(16))) uint16_t xs[(kTile + (FS ? 1 : 0)) * kStride];
  const int tid = threadIdx.x;
  // bf16 rows, fused schedule: a dot-product pre-pass on the MFMA settles most tokens
  // (below); with 16-byte rows each block also runs several tiles with the next one's
  // loads in flight
  constexpr bool MF = !GENERAL && DT == VCX_BFLOAT16, PREFETCH = assign_prefetch(DT, GENERAL, WIDE);
  // items (head, tile) first .. last - 1, in order: consecutive tiles of a head (one item
  // per block without the prefetch)
  const int64_t first = blockIdx.x * (PREFETCH ? per : 1);
  const int64_t last = PREFETCH ? (first + per < items ? first + per : items) : first + 1;
  if (first >= items) return;
  if constexpr (FS) {
    if (tid < kStride / 8) *reinterpret_cast<uint4*>(&xs[kTile * kStride + 8 * tid]) = make_uint4(0, 0, 0, 0);
  }
  // Staging: coalesced loads of a tile into registers, then stored to LDS once every reader
  // of the previous tile is done. Behind the bf16 pre-pass (whose block runs several tiles)
  // the next tile's loads are issued before the current tile's work, so that their latency
  // overlaps it; elsewhere a block runs one tile and the registers stay free for the
  // chains. 16-byte pieces when every row is 16-byte aligned (WIDE), else 4-byte pieces; a
  // full tile (every tile but a partial last one) loads without per-row tests.
  using Piece = std::conditional_t<WIDE, uint4, uint32_t>;
  constexpr int kElems = WIDE ? 8 : 2, kPieces = D / kElems, kPer = kTile * kPieces / kGroupThreads;
  Piece val[kPer];
  auto load = [&](int64_t item) {
    const int64_t tile = item % tiles;
    const uint16_t* base = head_ptr(v, item / tiles, H, sb, sh);
    if ((tile + 1) * kTile <= n) {
      // a wave-uniform base per load plus one 32-bit lane offset (kGroupThreads is a
      // multiple of kPieces, so a thread keeps its piece and moves down whole rows)
      const char* tb = reinterpret_cast<const char*>(base + tile * kTile * sn);
      const uint32_t lane_off = static_cast<uint32_t>(((tid / kPieces) * sn + kElems * (tid % kPieces)) * 2);
#pragma unroll
      for (int k = 0; k < kPer; ++k)
        val[k] = *reinterpret_cast<const Piece*>(tb + k * (kGroupThreads / kPieces) * sn * 2 + lane_off);
    } else {
#pragma unroll
      for (int k = 0; k < kPer; ++k) {
        const int s = tid + k * kGroupThreads, row = s / kPieces, part = s % kPieces;
        const int64_t tok = tile * kTile + row;
        val[k] = tok < n ? *reinterpret_cast<const Piece*>(base + tok * sn + kElems * part) : Piece{};
      }
    }
  };
  __shared__ int hist[GENERAL ? kMaxClusters : 1];
  // Fused schedule at D64, and at D128 behind the bf16 pre-pass (where the chains are the
  // rare path): the head's 8 binary32 centers, channel-major ([d][8]), so that one
  // wave-uniform (broadcast) 16-byte LDS read gives four clusters' values of a channel.
  constexpr bool LDSC = !GENERAL && (D == 64 || DT == VCX_BFLOAT16);
  __shared__ __attribute__((aligned(16))) float cl[LDSC ? kFusedClusters * D : 4];
  // bf16 pre-pass state of the current head (fused schedule): the A operand (row r < 8
  // holds cluster r's hi part, row r >= 8 cluster r - 8's lo part; lane group G holds
  // channels 8G..8G+7 of each 32-channel step) and the norms of the four clusters whose
  // result rows this lane receives (clusters 4(G & 1)..+3).
  constexpr int KS = D / 32;
  const int lane = tid & 63, G = lane >> 4, r = lane & 15, w = tid >> 6;
  v8bf af[KS];
  float cn[4];
  if constexpr (PREFETCH) load(first);
  int64_t head = -1;
  for (int64_t item = first; item < last; ++item) {
    const int64_t tile = item % tiles, bh = item / tiles;
    if constexpr (!PREFETCH) load(item);
    lds_barrier();  // every reader of the previous tile is done
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int s = tid + k * kGroupThreads, row = s / kPieces, part = s % kPieces;
      *reinterpret_cast<Piece*>(&xs[row * kStride + kElems * part]) = val[k];
    }
    if constexpr (GENERAL) {
      for (int c = tid; c < count; c += kGroupThreads) hist[c] = 0;
    }
    if (bh != head) {
      head = bh;
      if constexpr (LDSC) {
        const float* src = centers32 + bh * kFusedClusters * D;
        for (int e = tid; e < kFusedClusters * D; e += kGroupThreads) cl[(e % D) * kFusedClusters + e / D] = src[e];
      }
      if constexpr (MF) {
        const int cr = r & 7;
        const uint16_t* part = forms.parts + ((bh * kFusedClusters + cr) * 2 + (r >> 3)) * D;
#pragma unroll
        for (int k = 0; k < KS; ++k) {
          uint4 a = make_uint4(0, 0, 0, 0);
          if (cr < count) a = *reinterpret_cast<const uint4*>(part + 32 * k + 8 * G);
          af[k] = __builtin_bit_cast(v8bf, a);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int c = 4 * (G & 1) + j;
          cn[j] = c < count ? forms.norms[bh * kFusedClusters + c] : 0.0f;
        }
        // wait for these loads here: a use of the values on this path keeps the compiler
        // from waiting for every load (the next tile's included) where the tile work uses
        // them
        asm volatile("" ::"v"(af[0]), "v"(cn[0]), "v"(cn[1]), "v"(cn[2]), "v"(cn[3]));
#pragma unroll
        for (int k = 1; k < KS; ++k) asm volatile("" ::"v"(af[k]));
      }
    }
    lds_barrier();
    if constexpr (PREFETCH) {
      if (item + 1 < last) load(item + 1);
    }
    const int64_t tok = tile * kTile + tid;
    int best = 0;
    // The label is the argmin of the fp64 distances. The same distances are first formed in
    // binary32 (x - c rounded, then a fused multiply-add chain): every term is non-negative,
    // so each binary32 distance lies within (D + 2) * 2^-24 relative (plus a subnormal-sized
    // absolute term) of the exact one. When the second smallest exceeds the smallest by more
    // than twice that bound, the exact and the fp64 distances order the same way and the
    // binary32 argmin is the label; otherwise (ties, near ties, overflow) the lane takes the
    // fp64 chains below.
    bool sure = false;
    // bf16 rows, fused schedule: the dot-product pre-pass. distance_c = X + C_c - 2 P_c with
    // u = 2^-24 and
    //   X = |x|^2: per lane a chain of D/8 bf16 dot2 steps over exact squares, then the sums
    //     of the four lane groups' partials; each of the D/8 + 2 steps may err by 2u of the
    //     running sum, so |X' - X| <= (D/4 + 4) u X;
    //   C_c = |c|^2, precomputed (one rounding of a sum far more accurate than u);
    //   P_c = x.c on the bf16 MFMA: x is exact in bf16 and c enters as its two bf16 parts
    //     (|c - hi - lo| <= 2^-17 |c|), so every product is exact in fp32. With A = sum
    //     |x_d c_d| <= (X + C) / 2, each of the D + D/32 accumulations (D products and the
    //     running sum at each 32-channel step) may err by 2u (whatever the MFMA's internal
    //     order, rounding or denormal flushing) of the part's sum of magnitudes: at most
    //     (1 + 2^-8) A for the hi part, 2^-8 (1 + 2^-8) A for the lo part; and the parts
    //     leave 2^-17 A out;
    //   plus one rounding each for S = X + C, hi + lo and S - 2P (|S - 2P| <= 2S).
    // Doubling the P terms (2A <= S) gives |D'_c - D_c| <= ((D/4 + 9 + 2.016 (D + D/32)) u +
    // 2^-17) S + 1e-30 (the absolute term covers flushed subnormal products); kKappa is that
    // factor with a 2 % margin. A token whose best center b (lowest id on equal values) has
    // D_b + E_b < D_c - E_c for every other center c has b as its exact argmin, with a gap
    // about 10^7 times the fp64 chains' own error, so b is the fp64 argmin too. Ties, near
    // ties and non-finite values go on to the binary32 and fp64 stages below.
    if constexpr (MF) {
      constexpr float kKappa = ((D / 4 + 9 + 2.016f * (D + KS)) * 5.9604645e-8f + 7.6293945e-6f) * 1.02f;
      __shared__ uint8_t pre[kTile];  // the pre-pass's label, bit 7 set when it is settled
#pragma unroll 1
      for (int nb = 0; nb < 4; ++nb) {
        const int t = 64 * w + 16 * nb + r;  // this lane's B column: token t of the tile
        v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
        float x2 = 0.0f;
#pragma unroll
        for (int k = 0; k < KS; ++k) {
          const uint4 q = *reinterpret_cast<const uint4*>(&xs[t * kStride + 32 * k + 8 * G]);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[k], __builtin_bit_cast(v8bf, q), acc, 0, 0, 0);
          const uint32_t wq[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
          for (int e = 0; e < 4; ++e)
            x2 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2bf, wq[e]), __builtin_bit_cast(v2bf, wq[e]), x2, false);
        }
        // Sums over lane pairs: a permlane swap returns {own, partner} on the lower lane
        // group of each pair and {partner, own} on the upper one, and both add the same two
        // values (addition is commutative), so every lane of a token holds the same X and P.
        {
          const auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x2), __float_as_uint(x2), false, false);
          x2 = __uint_as_float(s16[0]) + __uint_as_float(s16[1]);
          const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x2), __float_as_uint(x2), false, false);
          x2 = __uint_as_float(s32[0]) + __uint_as_float(s32[1]);
        }
        // D_c and E_c of this lane's four clusters; a non-finite D_c or E_c becomes NaN (it then
        // fails every comparison below), a slot past count +inf with E = 0 (never the best,
        // always separated)
        float dd[4], ee[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[j]), __float_as_uint(acc[j]), false, false);
          const float p = __fadd_rn(__uint_as_float(s[0]), __uint_as_float(s[1]));  // hi + lo
          const float S = __fadd_rn(x2, cn[j]);
          dd[j] = __fsub_rn(S, 2.0f * p);
          ee[j] = __fmaf_rn(kKappa, S, 1.0e-30f);
          if (!(__builtin_isfinite(dd[j]) && __builtin_isfinite(ee[j]))) dd[j] = __builtin_nanf("");
          if (4 * (G & 1) + j >= count) {
            dd[j] = INFINITY;
            ee[j] = 0.0f;
          }
        }
        // clusters 4..7 from lane group 1 to lane group 0 (the other groups compute the same
        // decision on other values and do not store it)
        float D8[8], E8[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const auto sd = __builtin_amdgcn_permlane16_swap(__float_as_uint(dd[j]), __float_as_uint(dd[j]), false, false);
          const auto se = __builtin_amdgcn_permlane16_swap(__float_as_uint(ee[j]), __float_as_uint(ee[j]), false, false);
          D8[j] = dd[j];
          E8[j] = ee[j];
          D8[4 + j] = __uint_as_float(sd[1]);
          E8[4 + j] = __uint_as_float(se[1]);
        }
        // b = the first strict minimum of D; settled when no other center's D_c - E_c fails to
        // exceed D_b + E_b (a NaN fails, so does everything when D_b + E_b is NaN; with one
        // cluster the label is 0 either way)
        float bv = D8[0], be = E8[0];
        int b = 0;
#pragma unroll
        for (int c = 1; c < 8; ++c)
          if (D8[c] < bv) {
            bv = D8[c];
            be = E8[c];
            b = c;
          }
        const float ub = __fadd_rn(bv, be);
        int open = 0;
#pragma unroll
        for (int c = 0; c < 8; ++c) open += !(__fsub_rn(D8[c], E8[c]) > ub);
        if (G == 0) pre[t] = static_cast<uint8_t>(b | (open == 1 ? 0x80 : 0));
      }
      lds_barrier();
      best = pre[tid] & 7;
      sure = (pre[tid] & 0x80) != 0;
    }
    // The wave's open tokens. A few go through the binary32 stage one at a time, by the whole
    // wave (each about 100 instructions), and what that leaves open through the fp64 chains 8
    // rows at a time; with more than kWaveRows every lane runs its own chains below (binary32,
    // then fp64 where needed: about 2300 and 3200 instructions for the wave, whatever the
    // count).
    constexpr int kWaveRows = 8;
    uint64_t open = 0;
    bool many = false;
    if constexpr (MF) {
      open = __ballot(tok < n && !sure);
      many = __popcll(open) > kWaveRows;
      if (!many) {
        uint64_t left = 0;
        for (uint64_t o = open; o; o &= o - 1) {
          const int t = __builtin_ctzll(o);
          int lab;
          if (!wave_row_b32<DT, D>(&xs[(64 * w + t) * kStride], cl, count, lane, lab)) left |= 1ull << t;
          if (lane == t) best = lab;
        }
        open = left;
        sure = true;
      } else {
        open = 0;
      }
    }
    if (tok < n && LDSC && !sure) {
      float b32 = INFINITY, s32 = INFINITY;
      float acc[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) acc[c] = 0.0f;
      const float4* cl4 = reinterpret_cast<const float4*>(cl);
#pragma unroll 2
      for (int i = 0; i < D / 8; ++i) {
        const uint4 q = *reinterpret_cast<const uint4*>(&xs[tid * kStride + 8 * i]);
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int d = 8 * i + 2 * k;
          const float x0 = in_to_f32<DT>(w[k] & 0xffffu), x1 = in_to_f32<DT>(w[k] >> 16);
          const float4 a0 = cl4[2 * d], a1 = cl4[2 * d + 1], b0 = cl4[2 * d + 2], b1 = cl4[2 * d + 3];
          const float c0v[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
          const float c1v[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
          for (int c = 0; c < 8; ++c) {
            const float d0 = __fsub_rn(x0, c0v[c]);
            acc[c] = __fmaf_rn(d0, d0, acc[c]);
            const float d1 = __fsub_rn(x1, c1v[c]);
            acc[c] = __fmaf_rn(d1, d1, acc[c]);
          }
        }
      }
      bool finite = true;  // a NaN distance (NaN in V or a center) fails every compare below
#pragma unroll
      for (int c = 0; c < 8; ++c)
        if (c < count) {
          finite = finite && acc[c] >= 0.0f;
          if (acc[c] < b32) {  // ties keep the lowest id (and make the order unsure)
            s32 = b32;
            b32 = acc[c];
            best = c;
          } else if (acc[c] < s32) {
            s32 = acc[c];
          }
        }
      constexpr float kOrder = 1.0f + 4.0e-5f;  // > (1 + e) / (1 - e), e = 130 * 2^-24
      // NaN distances never enter b32 / s32, so they are tested separately: with one the fp64
      // chains decide, as in the oracle; an infinite b32 also leaves the order unsure
      sure = finite && s32 > b32 * kOrder + 1.0e-37f;
    }
    if (tok < n && !LDSC && !sure) {
      float b32 = INFINITY, s32 = INFINITY;
      bool finite = true;  // a NaN distance (NaN in V or a center) fails every compare below
      for (int c0 = 0; c0 < count; c0 += 8) {
        const float* cen = centers32 + (bh * CS + c0) * D;  // wave-uniform: scalar loads
        float acc[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[c] = 0.0f;
#pragma unroll 2
        for (int i = 0; i < D / 8; ++i) {
          const uint4 q = *reinterpret_cast<const uint4*>(&xs[tid * kStride + 8 * i]);
          const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const int d = 8 * i + 2 * k;
            const float x0 = in_to_f32<DT>(w[k] & 0xffffu), x1 = in_to_f32<DT>(w[k] >> 16);
#pragma unroll
            for (int c = 0; c < 8; ++c) {
              const float d0 = __fsub_rn(x0, cen[c * D + d]);
              acc[c] = __fmaf_rn(d0, d0, acc[c]);
              const float d1 = __fsub_rn(x1, cen[c * D + d + 1]);
              acc[c] = __fmaf_rn(d1, d1, acc[c]);
            }
          }
        }
#pragma unroll
        for (int c = 0; c < 8; ++c)
          if (c0 + c < count) {
            finite = finite && acc[c] >= 0.0f;
            if (acc[c] < b32) {  // ties keep the lowest id (and make the order unsure)
              s32 = b32;
              b32 = acc[c];
              best = c0 + c;
            } else if (acc[c] < s32) {
              s32 = acc[c];
            }
          }
      }
      constexpr float kOrder = 1.0f + 4.0e-5f;  // > (1 + e) / (1 - e), e = 130 * 2^-24
      sure = finite && s32 > b32 * kOrder + 1.0e-37f;  // NaN distances: the fp64 chains decide
    }
    if constexpr (MF) {
      // what the wave-wide binary32 stage left open (at most kWaveRows tokens): the fp64
      // chains, 8 rows at a time
      while (open) wave_rows_b64<DT, D, kStride>(xs, 64 * w, open, cl, count, lane, best);
    }
    if (tok < n && !sure) {
      // first strict minimum from +inf: NaN and infinite distances never win, and a token with
      // no finite distance keeps label 0 (the oracle's rule)
      best = 0;
      double best_d = INFINITY;
      // kC clusters side by side (4 behind the D64 pre-pass, which keeps the registers of a
      // third wave per SIMD)
      constexpr int kC = (MF && D == 64) ? 4 : 8;
      for (int c0 = 0; c0 < count; c0 += kC) {
        const double* cen = centers64 + (bh * CS + c0) * D;  // wave-uniform: scalar loads
        // distance_c = sum over d (in order) of fma(x_d - c_d, x_d - c_d, acc) in fp64
        double acc[kC];
#pragma unroll
        for (int c = 0; c < kC; ++c) acc[c] = 0.0;
#pragma unroll 2
        for (int i = 0; i < D / 8; ++i) {
          const uint4 q = *reinterpret_cast<const uint4*>(&xs[tid * kStride + 8 * i]);
          const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const int d = 8 * i + 2 * k;
            const double x0 = static_cast<double>(in_to_f32<DT>(w[k] & 0xffffu));
            const double x1 = static_cast<double>(in_to_f32<DT>(w[k] >> 16));
            // fused schedule: the fp64 centers are the exact widenings of the LDS fp32 ones
            double c0v[kC], c1v[kC];
            if constexpr (LDSC) {
              const float* r0 = cl + d * kFusedClusters + c0;
#pragma unroll
              for (int c = 0; c < kC; c += 4) {
                const float4 a = *reinterpret_cast<const float4*>(r0 + c);
                const float4 b = *reinterpret_cast<const float4*>(r0 + kFusedClusters + c);
                c0v[c] = a.x, c0v[c + 1] = a.y, c0v[c + 2] = a.z, c0v[c + 3] = a.w;
                c1v[c] = b.x, c1v[c + 1] = b.y, c1v[c + 2] = b.z, c1v[c + 3] = b.w;
              }
            } else {
#pragma unroll
              for (int c = 0; c < kC; ++c) {
                c0v[c] = cen[c * D + d];
                c1v[c] = cen[c * D + d + 1];
              }
            }
#pragma unroll
            for (int c = 0; c < kC; ++c) {
              const double d0 = __dsub_rn(x0, c0v[c]);
              acc[c] = __fma_rn(d0, d0, acc[c]);
              const double d1 = __dsub_rn(x1, c1v[c]);
              acc[c] = __fma_rn(d1, d1, acc[c]);
            }
          }
        }
#pragma unroll
        for (int c = 0; c < kC; ++c)
          if (c0 + c < count && acc[c] < best_d) {  // ties keep the lowest id
            best_d = acc[c];
            best = c0 + c;
          }
      }
    }
    if (tok < n) labels[bh * n + tok] = best;
    const int64_t meta = (bh * tiles + tile) * CS;
    if constexpr (GENERAL) {
      if (tok < n) atomicAdd(&hist[best], 1);
      lds_barrier();
      for (int c = tid; c < count; c += kGroupThreads) pcnt[meta + c] = hist[c];
    } else {
      // Per-tile counts from wave ballots, which also give each token its rank among the
      // earlier tokens of its wave with the same label.
      __shared__ int wcount[2][kFusedClusters];
      const int L = tok < n ? best : -1;
      const int wv = tid >> 6;
      int rank = 0;
#pragma unroll
      for (int c = 0; c < kFusedClusters; ++c) {
        const uint64_t m = __ballot(L == c);
        if (L == c)
          rank = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32), __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0));
        if (lane == 0) wcount[wv][c] = __popcll(m);
      }
      lds_barrier();
      if (tid < count) pcnt[meta + tid] = wcount[0][tid] + wcount[1][tid];
      if constexpr (STATS) {
        // Per-cluster sums over the tile's tokens in token order. Each cluster's list holds
        // the LDS byte offsets of its tokens' staged rows, padded to a multiple of 8 entries
        // with the zero row: adding +0.0 leaves a partial sum unchanged (it starts at +0.0 and
        // is never -0.0). A step reads 8 offsets at once, then the 8 values, then adds them
        // in list order; each wave takes half of the clusters.
        constexpr int kB = 8;
        constexpr uint16_t kZeroRow = kTile * kStride * 2;
        __shared__ int start[kFusedClusters + 1];
        __shared__ __attribute__((aligned(16))) uint16_t order[kTile + kB * kFusedClusters];
        if (tid == 0) {
          int acc = 0;
          for (int c = 0; c < kFusedClusters; ++c) {
            start[c] = acc;
            acc += (wcount[0][c] + wcount[1][c] + kB - 1) & ~(kB - 1);
          }
          start[kFusedClusters] = acc;
        }
        lds_barrier();
        if (L >= 0) order[start[L] + (wv ? wcount[0][L] : 0) + rank] = static_cast<uint16_t>(tid * kStride * 2);
        if (tid < kB * kFusedClusters) {
          const int c = tid / kB, slot = start[c] + wcount[0][c] + wcount[1][c] + tid % kB;
          if (slot < start[c + 1]) order[slot] = kZeroRow;
        }
        lds_barrier();
        {
          // wave wv sums clusters 4 wv .. 4 wv + 3, each lane D/64 adjacent channels (one
          // 2- or 4-byte read per token, as many independent chains)
          constexpr int CPL = D / 64;
          using Word = std::conditional_t<CPL == 2, uint32_t, uint16_t>;
          const uint8_t* col = reinterpret_cast<const uint8_t*>(xs) + 2 * CPL * lane;
          const int c_end = 4 * wv + 4 < count ? 4 * wv + 4 : count;
          for (int c = 4 * wv; c < c_end; ++c) {
            double acc[CPL];
#pragma unroll
            for (int j = 0; j < CPL; ++j) acc[j] = 0.0;
            const int b = __builtin_amdgcn_readfirstlane(start[c]), e = __builtin_amdgcn_readfirstlane(start[c + 1]);
            for (int k = b; k < e; k += kB) {
              const uint4 o = *reinterpret_cast<const uint4*>(&order[k]);
              const uint32_t ow[4] = {o.x, o.y, o.z, o.w};
              uint32_t xw[kB];
#pragma unroll
              for (int i = 0; i < kB / 2; ++i) {
                xw[2 * i] = *reinterpret_cast<const Word*>(col + (ow[i] & 0xffffu));
                xw[2 * i + 1] = *reinterpret_cast<const Word*>(col + (ow[i] >> 16));
              }
#pragma unroll
              for (int i = 0; i < kB; ++i)
#pragma unroll
                for (int j = 0; j < CPL; ++j)
                  acc[j] = __dadd_rn(acc[j], static_cast<double>(in_to_f32<DT>((xw[i] >> (16 * j)) & 0xffffu)));
            }
            double* dst = &psum[(meta + c) * D + CPL * lane];
            if constexpr (CPL == 2) {
              double2 pr;
              pr.x = acc[0];
              pr.y = acc[1];
              *reinterpret_cast<double2*>(dst) = pr;
            } else {
              dst[0] = acc[0];
            }
          }
        }
      }
    }
  }
}

// Fused schedule. grid (B*H, count), D threads: new center = RN_f32(sum / n) for a
// non-empty cluster, the fp64 sum taken over tiles in order. The launch is small (one
// block per head and cluster), so its time is the chain of load round trips: each batch
// puts 80 tiles' partials in flight before adding them in order.
__global__ __launch_bounds__(128) void grp_update_kernel(float* centers, double* centers64, const double* psum,
                                                         const int32_t* pcnt, int64_t tiles, int D,
                                                         CenterForms forms) {
  __shared__ double red[2];
  const int64_t bh = blockIdx.x;
  const int c = blockIdx.y, d = threadIdx.x;
  // Token count of the cluster: an integer sum (exact in any order), spread over the lanes,
  // then a butterfly per wave and the waves' totals through LDS.
  __shared__ int64_t cnt_sh[2];
  int64_t part = 0;
  for (int64_t t = d; t < tiles; t += D) part += pcnt[(bh * tiles + t) * kFusedClusters + c];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) part += __shfl_xor(part, o, 64);
  if ((d & 63) == 0) cnt_sh[d >> 6] = part;
  __syncthreads();
  const int64_t total = D > 64 ? cnt_sh[0] + cnt_sh[1] : cnt_sh[0];
  // Batches of kBatch tiles by buffer loads from the batch's first tile: the lane's channel
  // in the vector offset, the tile (wave-uniform, kept below the tile count) in the scalar
  // one, so that a batch costs only its data registers (295 tiles: 4 round trips, 5 with
  // batches of 64 by flat loads).
  constexpr int kBatch = 80;
  const double* hb = psum + (bh * tiles * kFusedClusters + c) * D;
  const int stride = kFusedClusters * D;
  double s = 0.0;
  for (int64_t t = 0; t < tiles; t += kBatch) {
    const int last = static_cast<int>((tiles - t < kBatch ? tiles - t : kBatch) - 1);
    const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(const_cast<double*>(hb + t * stride), 0,
                                                                        (last * stride + D) * 8, 0x00020000);
    double v[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i)
      v[i] = __builtin_bit_cast(double, __builtin_amdgcn_raw_buffer_load_b64(rp, d * 8, (i < last ? i : last) * stride * 8, 0));
    __builtin_amdgcn_sched_barrier(0);  // every load of the batch issued before the first add
#pragma unroll
    for (int i = 0; i < kBatch; ++i)
      if (i <= last) s = __dadd_rn(s, v[i]);
  }
  if (total > 0) {  // the same on every thread of the block
    const float x = static_cast<float>(__ddiv_rn(s, static_cast<double>(total)));
    centers[(bh * kFusedClusters + c) * D + d] = x;
    centers64[(bh * kFusedClusters + c) * D + d] = static_cast<double>(x);
    if (forms.parts) {
      store_center_parts(x, bh * kFusedClusters + c, d, D, forms);
      const double q = wave_square_sum(x);
      if ((d & 63) == 0) red[d >> 6] = q;
      __syncthreads();
      if (d == 0) forms.norms[bh * kFusedClusters + c] = static_cast<float>(D > 64 ? red[0] + red[1] : red[0]);
    }
  }
}

// General schedule. grid (B*H, count), D threads: cluster c's tokens are
// perm[offsets[tile 0][c] .. + n_c) in ascending order; each thread sums its channel,
// closing the tile partial whenever the token's tile changes (loads batched, order kept).
template <int DT>
__global__ void grp_update_sorted_kernel(const void* v, int64_t H, int64_t n, int64_t sb, int64_t sh, int64_t sn,
                                         int count, int CS, const int64_t* perm, const int64_t* offsets,
                                         const int32_t* pcnt, int64_t tiles, int D, float* centers,
                                         double* centers64) {
  const int64_t bh = blockIdx.x;
  const int c = blockIdx.y, d = threadIdx.x;
  const uint16_t* base = head_ptr(v, bh, H, sb, sh);
  const int64_t begin = offsets[bh * tiles * CS + c];
  const int64_t end = offsets[(bh * tiles + tiles - 1) * CS + c] + pcnt[(bh * tiles + tiles - 1) * CS + c];
  const int64_t* p = perm + bh * n;
  constexpr int kBatch = 16;
  double s = 0.0, part = 0.0;
  int64_t cur = -1;
  for (int64_t i = begin; i < end; i += kBatch) {
    int64_t tk[kBatch];
    float x[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) tk[j] = i + j < end ? p[i + j] : -1;
#pragma unroll
    for (int j = 0; j < kBatch; ++j) x[j] = tk[j] >= 0 ? in_to_f32<DT>(base[tk[j] * sn + d]) : 0.0f;
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      if (tk[j] < 0) break;
      const int64_t tl = tk[j] >> 7;
      if (tl != cur) {
        s = __dadd_rn(s, part);
        part = 0.0;
        cur = tl;
      }
      part = __dadd_rn(part, static_cast<double>(x[j]));
    }
  }
  s = __dadd_rn(s, part);
  const int64_t total = end - begin;
  if (total > 0) {
    const float x = static_cast<float>(__ddiv_rn(s, static_cast<double>(total)));
    centers[(bh * CS + c) * D + d] = x;
    centers64[(bh * CS + c) * D + d] = static_cast<double>(x);
  }
}

// grid (B*H), 256 threads: start offset of each (tile, label) in the sorted order, labels
// in order and tiles in order within a label. Integer counts, so the sums may be formed in
// any order: 32 lanes per label each sum a contiguous segment of tiles (loads batched), a
// shuffle scan over the 32 segments gives each segment's start inside its label, and the
// labels' totals in LDS give each label's start. Labels are taken 8 at a time.
constexpr int kOffsetThreads = 256;
__global__ __launch_bounds__(kOffsetThreads) void grp_offsets_kernel(const int32_t* pcnt, int64_t tiles, int count,
                                                                     int CS, int64_t* offsets) {
  __shared__ int64_t total[kMaxClusters];
  const int64_t bh = blockIdx.x;
  const int tid = threadIdx.x, r = tid & 31, sub = tid >> 5;
  const int64_t per = (tiles + 31) / 32, t0 = r * per < tiles ? r * per : tiles;
  const int64_t t1 = t0 + per < tiles ? t0 + per : tiles;
  const int32_t* head = pcnt + bh * tiles * CS;
  constexpr int kBatch = 16;
  auto seg_sum = [&](int c) {
    int64_t s = 0;
    int64_t t = t0;
    for (; t + kBatch <= t1; t += kBatch) {
      int v[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) v[i] = head[(t + i) * CS + c];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) s += v[i];
    }
    if (t < t1) {  // the partial last batch, its loads issued together too
      int v[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) v[i] = head[(t + i < t1 ? t + i : t) * CS + c];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) s += t + i < t1 ? v[i] : 0;
    }
    return s;
  };
  // exclusive start of this lane's segment inside its label (all 32 lanes take part)
  auto seg_start = [&](int64_t s, int64_t& incl) {
    incl = s;
#pragma unroll
    for (int o = 1; o < 32; o <<= 1) {
      const int64_t y = __shfl_up(incl, o, 32);
      if (r >= o) incl += y;
    }
    return incl - s;
  };
  for (int c0 = 0; c0 < count; c0 += 8) {
    const int c = c0 + sub;
    int64_t incl;
    seg_start(c < count ? seg_sum(c) : 0, incl);
    if (r == 31 && c < count) total[c] = incl;
  }
  __syncthreads();
  for (int c0 = 0; c0 < count; c0 += 8) {
    const int c = c0 + sub;
    int64_t incl;
    int64_t off = seg_start(c < count ? seg_sum(c) : 0, incl);
    if (c < count) {
      for (int i = 0; i < c; ++i) off += total[i];
      int64_t* out = offsets + bh * tiles * CS + c;
      for (int64_t t = t0; t < t1; ++t) {
        out[t * CS] = off;
        off += head[t * CS + c];
      }
    }
  }
}

// grid (tiles, B*H), 128 threads (one per token): perm[offset(tile, L) + rank] = token, rank
// = tokens of the tile before this one with the same label. Each wave finds its lanes with
// the same label by ballots over the label's bits; the second wave adds the first wave's
// count of that label (from LDS).
__global__ __launch_bounds__(kGroupThreads) void grp_scatter_kernel(const int32_t* labels, int64_t n, int CS,
                                                                    const int64_t* offsets, int64_t* perm) {
  __shared__ int first[kMaxClusters];
  const int64_t tile = blockIdx.x, bh = blockIdx.y, tiles = gridDim.x;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t tok = tile * kTile + tid;
  const int L = tok < n ? labels[bh * n + tok] : -1;
  for (int i = tid; i < CS; i += kGroupThreads) first[i] = 0;
  // labels are below 256; -1 (past n) differs from every label in bit 8
  uint64_t same = ~0ull;
#pragma unroll
  for (int b = 0; b < 9; ++b) {
    const bool bit = ((L >> b) & 1) != 0;
    const uint64_t m = __builtin_amdgcn_ballot_w64(bit);
    same &= bit ? m : ~m;
  }
  const int before = __builtin_popcountll(same & ((1ull << lane) - 1ull));
  __syncthreads();
  // the highest lane of each label group in wave 0 records the group's size
  if (w == 0 && L >= 0 && (same >> lane) == 1ull) first[L] = before + 1;
  __syncthreads();
  if (tok >= n) return;
  const int rank = before + (w == 1 ? first[L] : 0);
  perm[bh * n + offsets[(bh * tiles + tile) * CS + L] + rank] = tok;
}

size_t align_up(size_t x) { return (x + 255) & ~size_t(255); }

struct GroupWs {
  float* centers;
  double* centers64;
  double* psum;
  int32_t* pcnt;
  int32_t* labels;
  int64_t* offsets;
  CenterForms forms;  // fused schedule only (the pre-pass runs on bf16 rows)
  size_t bytes;
};

// Slots per head: 8 for the fused schedule, count rounded up to 8 for the general one
// (the assignment reads centers in chunks of 8).
int center_slots(int count, bool general) { return general ? (count + 7) / 8 * 8 : kFusedClusters; }

GroupWs group_ws(void* base, int64_t BH, int64_t N, int64_t D, int CS, bool general) {
  const int64_t tiles = cdiv(N, kTile);
  GroupWs w{};
  size_t off = 0;
  auto take = [&](size_t bytes) { char* p = static_cast<char*>(base) + off; off += align_up(bytes); return p; };
  w.centers = reinterpret_cast<float*>(take(sizeof(float) * BH * CS * D));
  w.centers64 = reinterpret_cast<double*>(take(sizeof(double) * BH * CS * D));
  w.psum = general ? nullptr : reinterpret_cast<double*>(take(sizeof(double) * BH * tiles * CS * D));
  w.pcnt = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * BH * tiles * CS));
  w.labels = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * BH * N));
  w.offsets = reinterpret_cast<int64_t*>(take(sizeof(int64_t) * BH * tiles * CS));
  if (!general) {
    w.forms.parts = reinterpret_cast<uint16_t*>(take(sizeof(uint16_t) * BH * CS * 2 * D));
    w.forms.norms = reinterpret_cast<float*>(take(sizeof(float) * BH * CS));
  }
  w.bytes = off;
  return w;
}

// torch.linspace(0, n-1, count) in fp32 (symmetric two-half formula), truncated.
void linspace_ids(int64_t n, int count, Ids& ids) {
  if (count == 1) { ids.v[0] = 0; return; }
  const float start = 0.0f, end = static_cast<float>(n - 1);
  const float step = (end - start) / static_cast<float>(count - 1);
  const int half = count / 2;
  for (int i = 0; i < count; ++i) {
    float v;
    if (i < half) { const float t = step * static_cast<float>(i); v = start + t; }
    else { const float t = step * static_cast<float>(count - 1 - i); v = end - t; }
    ids.v[i] = static_cast<int32_t>(v);
  }
}

}  // namespace

// Workspace of one grouping call: the larger of the two schedules' needs for this count
// (count = min(clusters, N)); the caller has checked clusters in [1, 256].
size_t ws_group(int64_t BH, int64_t N, int64_t D, int clusters) {
  const int count = static_cast<int>(std::min<int64_t>(clusters, N));
  size_t bytes = group_ws(nullptr, BH, N, D, center_slots(count, true), true).bytes;
  if (count <= kFusedClusters) bytes = std::max(bytes, group_ws(nullptr, BH, N, D, kFusedClusters, false).bytes);
  return bytes;
}

}  // namespace vcx

using namespace vcx;

extern "C" int vcx_group_values(const void* v, int dtype, int64_t B, int64_t H, int64_t N, int64_t D,
                                int64_t v_sb, int64_t v_sh, int64_t v_sn, int clusters, int iterations, int mode,
                                const float* centers_in, int64_t* perm, int32_t* labels, float* centers,
                                float* centers_next, void* workspace, size_t workspace_bytes, void* stream) {
  VCX_REQUIRE(B >= 1 && H >= 1 && N >= 1, "B, H, N must be positive");
  VCX_REQUIRE(D == 64 || D == 128, "D must be 64 or 128");
  VCX_REQUIRE(B * H <= 65535 && N < (int64_t(1) << 30) && B * H * cdiv(N, kTile) < (int64_t(1) << 31),
              "shape exceeds launch bounds");
  VCX_REQUIRE(dtype == VCX_FLOAT16 || dtype == VCX_BFLOAT16, "dtype must be float16 or bfloat16");
  VCX_REQUIRE(clusters >= 1 && clusters <= kMaxClusters && iterations >= 1 && iterations <= 100,
              "clusters must be in [1, 256] and iterations in [1, 100]");
  VCX_REQUIRE(mode == VCX_GROUP_AUTO || mode == VCX_GROUP_GENERAL, "mode must be VCX_GROUP_AUTO or VCX_GROUP_GENERAL");
  const int count = static_cast<int>(clusters < N ? clusters : N);
  const bool general = mode == VCX_GROUP_GENERAL || count > kFusedClusters;
  VCX_REQUIRE(v != nullptr && aligned(v, 4), "v must be non-null and 4-byte aligned");
  VCX_REQUIRE(v_sb % 2 == 0 && v_sh % 2 == 0 && v_sn % 2 == 0 && v_sn >= D && v_sb >= 0 && v_sh >= 0,
              "v strides must be even, non-negative, with sn >= D");
  VCX_REQUIRE(perm != nullptr && aligned(perm, 8), "perm must be non-null and 8-byte aligned");
  VCX_REQUIRE(aligned(labels, 4) && aligned(centers, 4) && aligned(centers_in, 4) && aligned(centers_next, 4),
              "labels/centers misaligned");
  const int64_t BH = B * H, tiles = cdiv(N, kTile);
  const int CS = center_slots(count, general);
  VCX_REQUIRE(workspace != nullptr && aligned(workspace, 256), "workspace must be non-null and 256-byte aligned");
  GroupWs ws = group_ws(workspace, BH, N, D, CS, general);
  VCX_REQUIRE(workspace_bytes >= ws.bytes, "workspace too small: need %zu bytes", ws.bytes);
  int32_t* lab = labels ? labels : ws.labels;
  Ids ids{};
  linspace_ids(N, count, ids);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool wide = aligned(v, 16) && v_sb % 8 == 0 && v_sh % 8 == 0 && v_sn % 8 == 0;
  auto copy_centers = [&](float* dst) -> int {
    hipError_t e = hipMemcpy2DAsync(dst, sizeof(float) * count * D, ws.centers, sizeof(float) * CS * D,
                                    sizeof(float) * count * D, BH, hipMemcpyDeviceToDevice, st);
    if (e != hipSuccess) return fail(VCX_EHIP, "hipMemcpy2DAsync: %s", hipGetErrorString(e));
    return VCX_OK;
  };
  auto run = [&](auto dt, auto dd) -> int {
    constexpr int DT = decltype(dt)::value, DD = decltype(dd)::value;
    // Assignment items are the BH * tiles (head, tile) pairs. With the prefetch (bf16 rows,
    // fused schedule, 16-byte rows) a block takes a run of two consecutive items, loading
    // the second during the first; otherwise one item per block. Same-box A/B on the
    // [1,28,37741,128] smoothing workload, grouping call: runs of 2 290 us, one item per
    // block 309 us, runs of 4 306 us, one run per resident block (9 items) 328 us; the
    // longer runs lose the hardware's dynamic balancing of slow (fallback-heavy) tiles.
    auto assign = [&](auto stats, auto gen, double* psum) -> int {
      constexpr bool ST = decltype(stats)::value, GE = decltype(gen)::value;
      auto launch = [&](auto kernel, bool runs) -> int {
        const int64_t items = BH * tiles;
        int64_t per = 1;
        if (runs) {  // only where more items than resident blocks
          int dev = 0, cus = 0, occ = 0;
          if (hipGetDevice(&dev) != hipSuccess ||
              hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
              hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kernel, kGroupThreads, 0) != hipSuccess)
            return fail(VCX_EHIP, "grouping: device query failed");
          per = std::min<int64_t>(cdiv(items, static_cast<int64_t>(std::max(cus, 1)) * std::max(occ, 1)), 2);
        }
        const int64_t grid = cdiv(items, per);
        kernel<<<dim3(static_cast<unsigned>(grid)), kGroupThreads, 0, st>>>(
            v, H, N, v_sb, v_sh, v_sn, count, CS, ws.centers, ws.centers64, ws.forms, lab, psum, ws.pcnt, tiles,
            items, per);
        return VCX_OK;
      };
      if (wide) return launch(grp_assign_kernel<DT, DD, ST, true, GE>, assign_prefetch(DT, GE, true));
      return launch(grp_assign_kernel<DT, DD, ST, false, GE>, assign_prefetch(DT, GE, false));
    };
    auto sort = [&]() -> int {
      grp_offsets_kernel<<<dim3(BH), kOffsetThreads, 0, st>>>(ws.pcnt, tiles, count, CS, ws.offsets);
      VCX_LAUNCHED("grp_offsets_kernel");
      grp_scatter_kernel<<<dim3(tiles, BH), kGroupThreads, 0, st>>>(lab, N, CS, ws.offsets, perm);
      VCX_LAUNCHED("grp_scatter_kernel");
      return VCX_OK;
    };
    grp_init_kernel<DT><<<dim3(BH), DD, 0, st>>>(v, H, v_sb, v_sh, v_sn, ids, count, CS, DD, centers_in,
                                                  ws.centers, ws.centers64,
                                                  DT == VCX_BFLOAT16 ? ws.forms : CenterForms{});
    VCX_LAUNCHED("grp_init_kernel");
    for (int it = 0; it < iterations; ++it) {
      const bool last = it + 1 == iterations, update = !last || centers_next != nullptr;
      if (!general) {
        if (int rc = update ? assign(std::true_type(), std::false_type(), ws.psum)
                            : assign(std::false_type(), std::false_type(), nullptr))
          return rc;
        VCX_LAUNCHED("grp_assign_kernel");
        if (last) {
          if (int rc = sort()) return rc;
          if (centers)
            if (int rc = copy_centers(centers)) return rc;
        }
        if (update) {
          grp_update_kernel<<<dim3(BH, count), DD, 0, st>>>(ws.centers, ws.centers64, ws.psum, ws.pcnt, tiles, DD,
                                                           DT == VCX_BFLOAT16 ? ws.forms : CenterForms{});
          VCX_LAUNCHED("grp_update_kernel");
        }
      } else {
        if (int rc = assign(std::false_type(), std::true_type(), nullptr)) return rc;
        VCX_LAUNCHED("grp_assign_kernel<general>");
        if (int rc = sort()) return rc;
        if (last && centers)
          if (int rc = copy_centers(centers)) return rc;
        if (update) {
          grp_update_sorted_kernel<DT><<<dim3(BH, count), DD, 0, st>>>(v, H, N, v_sb, v_sh, v_sn, count, CS, perm,
                                                                       ws.offsets, ws.pcnt, tiles, DD, ws.centers,
                                                                       ws.centers64);
          VCX_LAUNCHED("grp_update_sorted_kernel");
        }
      }
    }
    if (centers_next)
      if (int rc = copy_centers(centers_next)) return rc;
    return VCX_OK;
  };
  if (dtype == VCX_BFLOAT16) {
    if (D == 128) return run(std::integral_constant<int, VCX_BFLOAT16>(), std::integral_constant<int, 128>());
    return run(std::integral_constant<int, VCX_BFLOAT16>(), std::integral_constant<int, 64>());
  }
  if (D == 128) return run(std::integral_constant<int, VCX_FLOAT16>(), std::integral_constant<int, 128>());
  return run(std::integral_constant<int, VCX_FLOAT16>(), std::integral_constant<int, 64>());
}
