// V grouping on gfx950: deterministic Lloyd clustering (<= 8 centers per head)
// and a stable counting sort of the labels, as in the reference's fused
// grouping (third_party/sageattention_local/csrc/vc/clustering.cu:21-167).
//
// Contract (identical in oracle/vc_oracle.c vco_group_values):
//   ids = trunc(fp32 linspace(0, n-1, count)), centers = V[ids] as fp32;
//   distance = sum over d (sequential) of fma(x_d - c_d, x_d - c_d, acc) in fp64,
//   argmin with ties to the lowest id; all but the last iteration replace every
//   non-empty center by RN_f32(fp64 sum / count), the sum taken sequentially
//   over tokens inside each 128-token tile and then sequentially over tiles;
//   perm = stable sort of tokens by label.
#include "vcx_common.hpp"

namespace vcx {
namespace {

constexpr int kMaxClusters = 8;
constexpr int kGroupThreads = 128;  // one thread per token of a 128-token tile

struct Ids {
  int64_t v[kMaxClusters];
};

__device__ inline const uint16_t* head_ptr(const void* x, int64_t bh, int64_t H, int64_t sb, int64_t sh) {
  return reinterpret_cast<const uint16_t*>(x) + (bh / H) * sb + (bh % H) * sh;
}

// Centers are kept as fp32 (the contract's values) and as their exact fp64
// widening, which the assignment reads with wave-uniform (scalar) loads; unused
// slots of the fp64 copy are zero.
template <int DT>
__global__ void grp_init_kernel(const void* v, int64_t H, int64_t sb, int64_t sh, int64_t sn, Ids ids,
                                int count, int D, float* centers, double* centers64) {
  const int64_t bh = blockIdx.x;
  const uint16_t* base = head_ptr(v, bh, H, sb, sh);
  const int d = threadIdx.x;
  for (int c = 0; c < kMaxClusters; ++c) {
    const float x = c < count ? in_to_f32<DT>(base[ids.v[c] * sn + d]) : 0.0f;
    if (c < count) centers[(bh * kMaxClusters + c) * D + d] = x;
    centers64[(bh * kMaxClusters + c) * D + d] = static_cast<double>(x);
  }
}

// grid (tiles, B*H), 128 threads. Assign every token of the tile; with STATS
// also write the tile's per-cluster fp64 channel sums; always write the tile's
// per-cluster counts (used by the center update and by the sort).
// The tile is staged through LDS with coalesced loads; each thread then reads
// its token's row 16 bytes at a time and runs the distance chains of all
// clusters side by side (d outermost); the fp64 centers are wave-uniform and
// come through scalar loads.
template <int DT, int D, bool STATS, bool WIDE>
__global__ __launch_bounds__(kGroupThreads) void grp_assign_kernel(
    const void* v, int64_t H, int64_t n, int64_t sb, int64_t sh, int64_t sn, int count,
    const double* __restrict__ centers64, int32_t* labels, double* psum, int32_t* pcnt) {
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
  const double* cen = centers64 + bh * kMaxClusters * D;  // wave-uniform: scalar loads
  __syncthreads();
  const int64_t tok = tile * kTile + tid;
  int best = 0;
  if (tok < n) {
    // distance_c = sum over d (in order) of fma(x_d - c_d, x_d - c_d, acc) in fp64
    double acc[kMaxClusters];
#pragma unroll
    for (int c = 0; c < kMaxClusters; ++c) acc[c] = 0.0;
#pragma unroll 2
    for (int i = 0; i < D / 8; ++i) {
      const uint4 q = *reinterpret_cast<const uint4*>(&xs[tid * kStride + 8 * i]);
      const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int d = 8 * i + 2 * k;
        const double x0 = static_cast<double>(in_to_f32<DT>(w[k] & 0xffffu));
        const double x1 = static_cast<double>(in_to_f32<DT>(w[k] >> 16));
#pragma unroll
        for (int c = 0; c < kMaxClusters; ++c) {
          const double d0 = __dsub_rn(x0, cen[c * D + d]);
          acc[c] = __fma_rn(d0, d0, acc[c]);
          const double d1 = __dsub_rn(x1, cen[c * D + d + 1]);
          acc[c] = __fma_rn(d1, d1, acc[c]);
        }
      }
    }
    double best_d = acc[0];
#pragma unroll
    for (int c = 1; c < kMaxClusters; ++c)
      if (c < count && acc[c] < best_d) {  // ties keep the lowest id
        best_d = acc[c];
        best = c;
      }
    labels[bh * n + tok] = best;
  }
  // Stable order of the tile's tokens by label: wave ballots give each token its
  // rank among the earlier tokens with the same label.
  __shared__ int wcount[2][kMaxClusters];
  __shared__ int start[kMaxClusters + 1];
  __shared__ uint8_t order[kTile];
  const int L = tok < n ? best : -1;
  const int lane = tid & 63, wv = tid >> 6;
  int rank = 0;
#pragma unroll
  for (int c = 0; c < kMaxClusters; ++c) {
    const uint64_t m = __ballot(L == c);
    if (L == c) rank = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32), __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0));
    if (lane == 0) wcount[wv][c] = __popcll(m);
  }
  __syncthreads();
  if (tid == 0) {
    int acc = 0;
    for (int c = 0; c < kMaxClusters; ++c) {
      start[c] = acc;
      acc += wcount[0][c] + wcount[1][c];
    }
    start[kMaxClusters] = acc;
  }
  __syncthreads();
  if (L >= 0) order[start[L] + (wv ? wcount[0][L] : 0) + rank] = static_cast<uint8_t>(tid);
  const int64_t meta = (bh * tiles + tile) * kMaxClusters;
  if (tid < count) pcnt[meta + tid] = wcount[0][tid] + wcount[1][tid];
  if constexpr (STATS) {
    __syncthreads();
    if (tid < D) {
      // per-cluster sums over the tile's tokens in token order
      for (int c = 0; c < count; ++c) {
        double acc = 0.0;
        const int e = start[c + 1];
        for (int k = start[c]; k < e; ++k) {
          const int t = order[k];
          acc = __dadd_rn(acc, static_cast<double>(in_to_f32<DT>(xs[t * kStride + tid])));
        }
        psum[(meta + c) * D + tid] = acc;
      }
    }
  }
}

// grid (B*H, count), D threads: new center = RN_f32(sum / n) for a non-empty
// cluster, the fp64 sum taken over tiles in order (loads batched).
__global__ void grp_update_kernel(float* centers, double* centers64, const double* psum, const int32_t* pcnt,
                                  int64_t tiles, int D) {
  const int64_t bh = blockIdx.x;
  const int c = blockIdx.y, d = threadIdx.x;
  constexpr int kBatch = 16;
  double s = 0.0;
  int64_t total = 0;
  int64_t t = 0;
  for (; t + kBatch <= tiles; t += kBatch) {
    double v[kBatch];
    int cnt[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int64_t meta = (bh * tiles + t + i) * kMaxClusters + c;
      v[i] = psum[meta * D + d];
      cnt[i] = pcnt[meta];
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      s = __dadd_rn(s, v[i]);
      total += cnt[i];
    }
  }
  for (; t < tiles; ++t) {
    const int64_t meta = (bh * tiles + t) * kMaxClusters + c;
    s = __dadd_rn(s, psum[meta * D + d]);
    total += pcnt[meta];
  }
  if (total > 0) {
    const float x = static_cast<float>(__ddiv_rn(s, static_cast<double>(total)));
    centers[(bh * kMaxClusters + c) * D + d] = x;
    centers64[(bh * kMaxClusters + c) * D + d] = static_cast<double>(x);
  }
}

// grid (B*H), 64 threads: start offset of each (tile, label) in the sorted order
// (integer counts, so the batched loads do not change the result).
__global__ void grp_offsets_kernel(const int32_t* pcnt, int64_t tiles, int count, int64_t* offsets) {
  __shared__ int64_t total[kMaxClusters];
  const int64_t bh = blockIdx.x;
  const int c = threadIdx.x;
  constexpr int kBatch = 16;
  const int32_t* col = pcnt + bh * tiles * kMaxClusters + c;
  if (c < count) {
    int64_t s = 0;
    int64_t t = 0;
    for (; t + kBatch <= tiles; t += kBatch) {
      int v[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) v[i] = col[(t + i) * kMaxClusters];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) s += v[i];
    }
    for (; t < tiles; ++t) s += col[t * kMaxClusters];
    total[c] = s;
  }
  __syncthreads();
  if (c < count) {
    int64_t off = 0;
    for (int i = 0; i < c; ++i) off += total[i];
    int64_t* out = offsets + bh * tiles * kMaxClusters + c;
    int64_t t = 0;
    for (; t + kBatch <= tiles; t += kBatch) {
      int v[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) v[i] = col[(t + i) * kMaxClusters];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        out[(t + i) * kMaxClusters] = off;
        off += v[i];
      }
    }
    for (; t < tiles; ++t) {
      out[t * kMaxClusters] = off;
      off += col[t * kMaxClusters];
    }
  }
}

// grid (tiles, B*H), 128 threads: stable scatter of token indices.
__global__ __launch_bounds__(kGroupThreads) void grp_scatter_kernel(const int32_t* labels, int64_t n,
                                                                    const int64_t* offsets, int64_t* perm) {
  __shared__ int lab[kTile];
  const int64_t tile = blockIdx.x, bh = blockIdx.y, tiles = gridDim.x;
  const int tid = threadIdx.x;
  const int64_t tok = tile * kTile + tid;
  const int L = tok < n ? labels[bh * n + tok] : -1;
  lab[tid] = L;
  __syncthreads();
  if (tok >= n) return;
  int rank = 0;
  for (int t = 0; t < tid; ++t) rank += lab[t] == L;
  perm[bh * n + offsets[(bh * tiles + tile) * kMaxClusters + L] + rank] = tok;
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

GroupWs group_ws(void* base, int64_t BH, int64_t N, int64_t D) {
  const int64_t tiles = cdiv(N, kTile);
  GroupWs w{};
  size_t off = 0;
  auto take = [&](size_t bytes) { char* p = static_cast<char*>(base) + off; off += align_up(bytes); return p; };
  w.centers = reinterpret_cast<float*>(take(sizeof(float) * BH * kMaxClusters * D));
  w.centers64 = reinterpret_cast<double*>(take(sizeof(double) * BH * kMaxClusters * D));
  w.psum = reinterpret_cast<double*>(take(sizeof(double) * BH * tiles * kMaxClusters * D));
  w.pcnt = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * BH * tiles * kMaxClusters));
  w.labels = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * BH * N));
  w.offsets = reinterpret_cast<int64_t*>(take(sizeof(int64_t) * BH * tiles * kMaxClusters));
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
    ids.v[i] = static_cast<int64_t>(v);
  }
}

}  // namespace

size_t ws_group(int64_t BH, int64_t N, int64_t D) { return group_ws(nullptr, BH, N, D).bytes; }

}  // namespace vcx

using namespace vcx;

extern "C" int vcx_group_values(const void* v, int dtype, int64_t B, int64_t H, int64_t N, int64_t D,
                                int64_t v_sb, int64_t v_sh, int64_t v_sn, int clusters, int iterations,
                                int64_t* perm, int32_t* labels, float* centers, void* workspace,
                                size_t workspace_bytes, void* stream) {
  VCX_REQUIRE(B >= 1 && H >= 1 && N >= 1, "B, H, N must be positive");
  VCX_REQUIRE(D == 64 || D == 128, "D must be 64 or 128");
  VCX_REQUIRE(B * H <= 65535 && N < (int64_t(1) << 30), "shape exceeds launch bounds");
  VCX_REQUIRE(dtype == VCX_FLOAT16 || dtype == VCX_BFLOAT16, "dtype must be float16 or bfloat16");
  VCX_REQUIRE(clusters >= 1 && clusters <= 256 && iterations >= 1 && iterations <= 100,
              "clusters must be in [1, 256] and iterations in [1, 100]");
  const int count = static_cast<int>(clusters < N ? clusters : N);
  if (count > kMaxClusters)
    return fail(VCX_EUNSUPPORTED, "grouping supports at most %d effective clusters (got %d)", kMaxClusters, count);
  VCX_REQUIRE(v != nullptr && aligned(v, 4), "v must be non-null and 4-byte aligned");
  VCX_REQUIRE(v_sb % 2 == 0 && v_sh % 2 == 0 && v_sn % 2 == 0 && v_sn >= D && v_sb >= 0 && v_sh >= 0,
              "v strides must be even, non-negative, with sn >= D");
  VCX_REQUIRE(perm != nullptr && aligned(perm, 8), "perm must be non-null and 8-byte aligned");
  VCX_REQUIRE(aligned(labels, 4) && aligned(centers, 4), "labels/centers misaligned");
  const int64_t BH = B * H, tiles = cdiv(N, kTile);
  VCX_REQUIRE(workspace != nullptr && aligned(workspace, 256), "workspace must be non-null and 256-byte aligned");
  GroupWs ws = group_ws(workspace, BH, N, D);
  VCX_REQUIRE(workspace_bytes >= ws.bytes, "workspace too small: need %zu bytes", ws.bytes);
  int32_t* lab = labels ? labels : ws.labels;
  Ids ids{};
  linspace_ids(N, count, ids);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool wide = aligned(v, 16) && v_sb % 8 == 0 && v_sh % 8 == 0 && v_sn % 8 == 0;
  auto run = [&](auto dt, auto dd) -> int {
    constexpr int DT = decltype(dt)::value, DD = decltype(dd)::value;
    auto assign = [&](auto stats, double* psum) {
      constexpr bool ST = decltype(stats)::value;
      if (wide)
        grp_assign_kernel<DT, DD, ST, true><<<dim3(tiles, BH), kGroupThreads, 0, st>>>(
            v, H, N, v_sb, v_sh, v_sn, count, ws.centers64, lab, psum, ws.pcnt);
      else
        grp_assign_kernel<DT, DD, ST, false><<<dim3(tiles, BH), kGroupThreads, 0, st>>>(
            v, H, N, v_sb, v_sh, v_sn, count, ws.centers64, lab, psum, ws.pcnt);
    };
    grp_init_kernel<DT><<<dim3(BH), DD, 0, st>>>(v, H, v_sb, v_sh, v_sn, ids, count, DD, ws.centers, ws.centers64);
    VCX_LAUNCHED("grp_init_kernel");
    for (int it = 0; it < iterations; ++it) {
      if (it + 1 < iterations) {
        assign(std::true_type(), ws.psum);
        VCX_LAUNCHED("grp_assign_kernel<stats>");
        grp_update_kernel<<<dim3(BH, count), DD, 0, st>>>(ws.centers, ws.centers64, ws.psum, ws.pcnt, tiles, DD);
        VCX_LAUNCHED("grp_update_kernel");
      } else {
        assign(std::false_type(), nullptr);
        VCX_LAUNCHED("grp_assign_kernel");
      }
    }
    grp_offsets_kernel<<<dim3(BH), 64, 0, st>>>(ws.pcnt, tiles, count, ws.offsets);
    VCX_LAUNCHED("grp_offsets_kernel");
    grp_scatter_kernel<<<dim3(tiles, BH), kGroupThreads, 0, st>>>(lab, N, ws.offsets, perm);
    VCX_LAUNCHED("grp_scatter_kernel");
    if (centers) {
      hipError_t e = hipMemcpy2DAsync(centers, sizeof(float) * count * DD, ws.centers,
                                      sizeof(float) * kMaxClusters * DD, sizeof(float) * count * DD, BH,
                                      hipMemcpyDeviceToDevice, st);
      if (e != hipSuccess) return fail(VCX_EHIP, "hipMemcpy2DAsync: %s", hipGetErrorString(e));
    }
    return VCX_OK;
  };
  if (dtype == VCX_BFLOAT16) {
    if (D == 128) return run(std::integral_constant<int, VCX_BFLOAT16>(), std::integral_constant<int, 128>());
    return run(std::integral_constant<int, VCX_BFLOAT16>(), std::integral_constant<int, 64>());
  }
  if (D == 128) return run(std::integral_constant<int, VCX_FLOAT16>(), std::integral_constant<int, 128>());
  return run(std::integral_constant<int, VCX_FLOAT16>(), std::integral_constant<int, 64>());
}
