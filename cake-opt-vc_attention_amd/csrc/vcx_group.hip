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

__device__ inline const uint16_t* head_ptr(const void* x, int64_t bh, int64_t H, int64_t sb, int64_t sh) {
  return reinterpret_cast<const uint16_t*>(x) + (bh / H) * sb + (bh % H) * sh;
}

// Centers are kept as fp32 (the contract's values) and as their exact fp64 widening,
// which the assignment reads with wave-uniform (scalar) loads. Slots are CS per head
// (CS = 8 for the fused schedule, count rounded up to 8 for the general one); slots at or
// past count hold zeros. Initial values: centers_in [BH][count][D], else V[ids].
template <int DT>
__global__ void grp_init_kernel(const void* v, int64_t H, int64_t sb, int64_t sh, int64_t sn, Ids ids,
                                int count, int CS, int D, const float* centers_in, float* centers,
                                double* centers64) {
  const int64_t bh = blockIdx.x;
  const uint16_t* base = head_ptr(v, bh, H, sb, sh);
  const int d = threadIdx.x;
  for (int c = 0; c < CS; ++c) {
    float x = 0.0f;
    if (c < count) x = centers_in ? centers_in[(bh * count + c) * D + d] : in_to_f32<DT>(base[ids.v[c] * sn + d]);
    centers[(bh * CS + c) * D + d] = x;
    centers64[(bh * CS + c) * D + d] = static_cast<double>(x);
  }
}

// grid (tiles, B*H), 128 threads. Assign every token of the tile and write the tile's
// per-cluster counts (pcnt, CS slots per tile). Fused schedule (!GENERAL, count <= 8):
// with STATS also the tile's per-cluster fp64 channel sums. General schedule: counts from
// an LDS histogram.
// The tile is staged through LDS with coalesced loads; each thread then reads its token's
// row 16 bytes at a time and runs the distance chains of 8 clusters side by side (d
// outermost), chunk after chunk of 8 centers, in binary32 and, where that does not settle
// the argmin, in fp64. The fused schedule's binary32 centers sit in LDS channel-major and
// come through broadcast reads (as scalar operands, 8 centers x 16 channels outgrew the
// SGPRs and spilled into VGPR lanes); the general schedule and the fp64 chains read them
// through scalar loads.
template <int DT, int D, bool STATS, bool WIDE, bool GENERAL>
__global__ __launch_bounds__(kGroupThreads) void grp_assign_kernel(
    const void* v, int64_t H, int64_t n, int64_t sb, int64_t sh, int64_t sn, int count, int CS,
    const float* __restrict__ centers32, const double* __restrict__ centers64, int32_t* labels, double* psum,
    int32_t* pcnt) {
  constexpr int kStride = D + 8;  // 16-bit elements per staged row (16-byte aligned rows)
  __shared__ __attribute__((aligned(16))) uint16_t xs[kTile * kStride];
  const int64_t tile = blockIdx.x, bh = blockIdx.y, tiles = gridDim.x;
  const int tid = threadIdx.x;
  const uint16_t* base = head_ptr(v, bh, H, sb, sh);
  // Stage the tile with coalesced loads, all of a thread's loads issued before
  // its LDS stores: 16-byte pieces when every row is 16-byte aligned (WIDE),
  // else 4-byte pieces.
  if constexpr (WIDE) {
    constexpr int kPieces = D / 8, kPer = kTile * kPieces / kGroupThreads;
    uint4 val[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int s = tid + k * kGroupThreads, row = s / kPieces, part = s % kPieces;
      const int64_t tok = tile * kTile + row;
      val[k] = tok < n ? *reinterpret_cast<const uint4*>(base + tok * sn + 8 * part) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int s = tid + k * kGroupThreads, row = s / kPieces, part = s % kPieces;
      *reinterpret_cast<uint4*>(&xs[row * kStride + 8 * part]) = val[k];
    }
  } else {
    constexpr int kPieces = D / 2, kPer = kTile * kPieces / kGroupThreads;
    uint32_t val[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int s = tid + k * kGroupThreads, row = s / kPieces, part = s % kPieces;
      const int64_t tok = tile * kTile + row;
      val[k] = tok < n ? *reinterpret_cast<const uint32_t*>(base + tok * sn + 2 * part) : 0u;
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int s = tid + k * kGroupThreads, row = s / kPieces, part = s % kPieces;
      *reinterpret_cast<uint32_t*>(&xs[row * kStride + 2 * part]) = val[k];
    }
  }
  __shared__ int hist[GENERAL ? kMaxClusters : 1];
  if constexpr (GENERAL) {
    for (int c = tid; c < count; c += kGroupThreads) hist[c] = 0;
  }
  // Fused schedule: the head's 8 binary32 centers, channel-major ([d][8]), so that one
  // wave-uniform (broadcast) 16-byte LDS read gives four clusters' values of a channel.
  constexpr bool LDSC = !GENERAL && D == 64;
  __shared__ __attribute__((aligned(16))) float cl[LDSC ? kFusedClusters * D : 4];
  if constexpr (LDSC) {
    const float* src = centers32 + bh * kFusedClusters * D;
    for (int e = tid; e < kFusedClusters * D; e += kGroupThreads) cl[(e % D) * kFusedClusters + e / D] = src[e];
  }
  __syncthreads();
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
  if (tok < n && LDSC) {
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
  if (tok < n && !LDSC) {
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
  if (tok < n && !sure) {
    // first strict minimum from +inf: NaN and infinite distances never win, and a token with
    // no finite distance keeps label 0 (the oracle's rule)
    best = 0;
    double best_d = INFINITY;
    for (int c0 = 0; c0 < count; c0 += 8) {
      const double* cen = centers64 + (bh * CS + c0) * D;  // wave-uniform: scalar loads
      // distance_c = sum over d (in order) of fma(x_d - c_d, x_d - c_d, acc) in fp64
      double acc[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) acc[c] = 0.0;
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
          double c0v[8], c1v[8];
          if constexpr (LDSC) {
            const float4* cl4 = reinterpret_cast<const float4*>(cl);
            const float4 a0 = cl4[2 * d], a1 = cl4[2 * d + 1], b0 = cl4[2 * d + 2], b1 = cl4[2 * d + 3];
            const float f0[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
            const float f1[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
            for (int c = 0; c < 8; ++c) {
              c0v[c] = static_cast<double>(f0[c]);
              c1v[c] = static_cast<double>(f1[c]);
            }
          } else {
#pragma unroll
            for (int c = 0; c < 8; ++c) {
              c0v[c] = cen[c * D + d];
              c1v[c] = cen[c * D + d + 1];
            }
          }
#pragma unroll
          for (int c = 0; c < 8; ++c) {
            const double d0 = __dsub_rn(x0, c0v[c]);
            acc[c] = __fma_rn(d0, d0, acc[c]);
            const double d1 = __dsub_rn(x1, c1v[c]);
            acc[c] = __fma_rn(d1, d1, acc[c]);
          }
        }
      }
#pragma unroll
      for (int c = 0; c < 8; ++c)
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
    __syncthreads();
    for (int c = tid; c < count; c += kGroupThreads) pcnt[meta + c] = hist[c];
    return;
  } else {
    // Stable order of the tile's tokens by label: wave ballots give each token its
    // rank among the earlier tokens with the same label.
    __shared__ int wcount[2][kFusedClusters];
    __shared__ int start[kFusedClusters + 1];
    __shared__ uint8_t order[kTile];
    const int L = tok < n ? best : -1;
    const int lane = tid & 63, wv = tid >> 6;
    int rank = 0;
#pragma unroll
    for (int c = 0; c < kFusedClusters; ++c) {
      const uint64_t m = __ballot(L == c);
      if (L == c)
        rank = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32), __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0));
      if (lane == 0) wcount[wv][c] = __popcll(m);
    }
    __syncthreads();
    if (tid == 0) {
      int acc = 0;
      for (int c = 0; c < kFusedClusters; ++c) {
        start[c] = acc;
        acc += wcount[0][c] + wcount[1][c];
      }
      start[kFusedClusters] = acc;
    }
    __syncthreads();
    if (L >= 0) order[start[L] + (wv ? wcount[0][L] : 0) + rank] = static_cast<uint8_t>(tid);
    if (tid < count) pcnt[meta + tid] = wcount[0][tid] + wcount[1][tid];
    if constexpr (STATS) {
      __syncthreads();
      if (tid < D) {
        // per-cluster sums over the tile's tokens in token order, 8 tokens a step: their
        // indices (the same on every lane) and then their values are all loaded before the
        // additions, which keep the list order
        constexpr int kB = 8;
        for (int c = 0; c < count; ++c) {
          double acc = 0.0;
          const int b = __builtin_amdgcn_readfirstlane(start[c]), e = __builtin_amdgcn_readfirstlane(start[c + 1]);
          for (int k = b; k < e; k += kB) {
            int ti[kB];
            float xv[kB];
#pragma unroll
            for (int i = 0; i < kB; ++i) ti[i] = __builtin_amdgcn_readfirstlane(order[k + i < e ? k + i : e - 1]);
#pragma unroll
            for (int i = 0; i < kB; ++i) xv[i] = in_to_f32<DT>(xs[ti[i] * kStride + tid]);
#pragma unroll
            for (int i = 0; i < kB; ++i)
              if (k + i < e) acc = __dadd_rn(acc, static_cast<double>(xv[i]));
          }
          psum[(meta + c) * D + tid] = acc;
        }
      }
    }
  }
}

// Fused schedule. grid (B*H, count), D threads: new center = RN_f32(sum / n) for a
// non-empty cluster, the fp64 sum taken over tiles in order. The launch is small (one
// block per head and cluster), so its time is the chain of load round trips: each batch
// puts 64 tiles' partials in flight before adding them in order (5 round trips for 295
// tiles instead of 19 with batches of 16).
__global__ __launch_bounds__(128) void grp_update_kernel(float* centers, double* centers64, const double* psum,
                                                         const int32_t* pcnt, int64_t tiles, int D) {
  const int64_t bh = blockIdx.x;
  const int c = blockIdx.y, d = threadIdx.x;
  // Token count of the cluster: an integer sum (exact in any order), spread over the lanes
  // and combined in LDS.
  __shared__ int64_t cnt_sh[128];
  int64_t part = 0;
  for (int64_t t = d; t < tiles; t += D) part += pcnt[(bh * tiles + t) * kFusedClusters + c];
  cnt_sh[d] = part;
  __syncthreads();
  int64_t total = 0;
  for (int i = 0; i < D; ++i) total += cnt_sh[i];
  constexpr int kBatch = 64;
  const double* col = psum + (bh * tiles * kFusedClusters + c) * D + d;
  const int64_t stride = static_cast<int64_t>(kFusedClusters) * D;
  double s = 0.0;
  int64_t t = 0;
  for (; t + kBatch <= tiles; t += kBatch) {
    double v[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) v[i] = col[(t + i) * stride];
    __builtin_amdgcn_sched_barrier(0);  // every load of the batch issued before the first add
#pragma unroll
    for (int i = 0; i < kBatch; ++i) s = __dadd_rn(s, v[i]);
  }
  for (; t < tiles; ++t) s = __dadd_rn(s, col[t * stride]);
  if (total > 0) {
    const float x = static_cast<float>(__ddiv_rn(s, static_cast<double>(total)));
    centers[(bh * kFusedClusters + c) * D + d] = x;
    centers64[(bh * kFusedClusters + c) * D + d] = static_cast<double>(x);
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
    for (; t < t1; ++t) s += head[t * CS + c];
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
  VCX_REQUIRE(B * H <= 65535 && N < (int64_t(1) << 30), "shape exceeds launch bounds");
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
    auto assign = [&](auto stats, auto gen, double* psum) {
      constexpr bool ST = decltype(stats)::value, GE = decltype(gen)::value;
      if (wide)
        grp_assign_kernel<DT, DD, ST, true, GE><<<dim3(tiles, BH), kGroupThreads, 0, st>>>(
            v, H, N, v_sb, v_sh, v_sn, count, CS, ws.centers, ws.centers64, lab, psum, ws.pcnt);
      else
        grp_assign_kernel<DT, DD, ST, false, GE><<<dim3(tiles, BH), kGroupThreads, 0, st>>>(
            v, H, N, v_sb, v_sh, v_sn, count, CS, ws.centers, ws.centers64, lab, psum, ws.pcnt);
    };
    auto sort = [&]() -> int {
      grp_offsets_kernel<<<dim3(BH), kOffsetThreads, 0, st>>>(ws.pcnt, tiles, count, CS, ws.offsets);
      VCX_LAUNCHED("grp_offsets_kernel");
      grp_scatter_kernel<<<dim3(tiles, BH), kGroupThreads, 0, st>>>(lab, N, CS, ws.offsets, perm);
      VCX_LAUNCHED("grp_scatter_kernel");
      return VCX_OK;
    };
    grp_init_kernel<DT><<<dim3(BH), DD, 0, st>>>(v, H, v_sb, v_sh, v_sn, ids, count, CS, DD, centers_in,
                                                  ws.centers, ws.centers64);
    VCX_LAUNCHED("grp_init_kernel");
    for (int it = 0; it < iterations; ++it) {
      const bool last = it + 1 == iterations, update = !last || centers_next != nullptr;
      if (!general) {
        if (update) assign(std::true_type(), std::false_type(), ws.psum);
        else assign(std::false_type(), std::false_type(), nullptr);
        VCX_LAUNCHED("grp_assign_kernel");
        if (last) {
          if (int rc = sort()) return rc;
          if (centers)
            if (int rc = copy_centers(centers)) return rc;
        }
        if (update) {
          grp_update_kernel<<<dim3(BH, count), DD, 0, st>>>(ws.centers, ws.centers64, ws.psum, ws.pcnt, tiles, DD);
          VCX_LAUNCHED("grp_update_kernel");
        }
      } else {
        assign(std::false_type(), std::true_type(), nullptr);
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
