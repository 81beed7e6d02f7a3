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

template <int DT>
__global__ void grp_init_kernel(const void* v, int64_t H, int64_t sb, int64_t sh, int64_t sn, Ids ids,
                                int count, int D, float* centers) {
  const int64_t bh = blockIdx.x;
  const uint16_t* base = head_ptr(v, bh, H, sb, sh);
  const int d = threadIdx.x;
  for (int c = 0; c < count; ++c)
    centers[(bh * kMaxClusters + c) * D + d] = in_to_f32<DT>(base[ids.v[c] * sn + d]);
}

// grid (tiles, B*H), 128 threads. Assign every token of the tile; with STATS
// also write the tile's per-cluster fp64 channel sums; always write the tile's
// per-cluster counts (used by the center update and by the sort).
template <int DT, int D, bool STATS>
__global__ __launch_bounds__(kGroupThreads) void grp_assign_kernel(
    const void* v, int64_t H, int64_t n, int64_t sb, int64_t sh, int64_t sn, int count,
    const float* centers, int32_t* labels, double* psum, int32_t* pcnt) {
  constexpr int kStride = D + 2;  // 16-bit elements; odd word stride avoids bank conflicts
  __shared__ uint16_t xs[kTile * kStride];
  __shared__ float cen[kMaxClusters * D];
  __shared__ int lab[kTile];
  const int64_t tile = blockIdx.x, bh = blockIdx.y, tiles = gridDim.x;
  const int tid = threadIdx.x;
  const uint16_t* base = head_ptr(v, bh, H, sb, sh);
  // Stage the tile: 4-byte pieces so every LDS row start stays word aligned.
  for (int s = tid; s < kTile * (D / 2); s += kGroupThreads) {
    const int row = s / (D / 2), part = s % (D / 2);
    const int64_t tok = tile * kTile + row;
    uint32_t val = 0;
    if (tok < n) val = *reinterpret_cast<const uint32_t*>(base + tok * sn + 2 * part);
    *reinterpret_cast<uint32_t*>(&xs[row * kStride + 2 * part]) = val;
  }
  for (int s = tid; s < count * D; s += kGroupThreads) cen[s] = centers[bh * kMaxClusters * D + s];
  __syncthreads();
  const int64_t tok = tile * kTile + tid;
  int best = 0;
  if (tok < n) {
    double best_d = INFINITY;
    for (int c = 0; c < count; ++c) {
      double acc = 0.0;
#pragma unroll 8
      for (int d = 0; d < D; ++d) {
        double diff = __dsub_rn(static_cast<double>(in_to_f32<DT>(xs[tid * kStride + d])),
                                static_cast<double>(cen[c * D + d]));
        acc = __fma_rn(diff, diff, acc);
      }
      if (acc < best_d) { best_d = acc; best = c; }
    }
    labels[bh * n + tok] = best;
  }
  lab[tid] = tok < n ? best : -1;
  __syncthreads();
  const int64_t meta = (bh * tiles + tile) * kMaxClusters;
  if (tid < count) {
    int cnt = 0;
    for (int t = 0; t < kTile; ++t) cnt += lab[t] == tid;
    pcnt[meta + tid] = cnt;
  }
  if constexpr (STATS) {
    if (tid < D) {
      double acc[kMaxClusters];
#pragma unroll
      for (int c = 0; c < kMaxClusters; ++c) acc[c] = 0.0;
      for (int t = 0; t < kTile; ++t) {
        const int L = lab[t];
        const double x = static_cast<double>(in_to_f32<DT>(xs[t * kStride + tid]));
#pragma unroll
        for (int c = 0; c < kMaxClusters; ++c)
          if (L == c) acc[c] = __dadd_rn(acc[c], x);
      }
      for (int c = 0; c < count; ++c) psum[(meta + c) * D + tid] = acc[c];
    }
  }
}

// grid (B*H), D threads: new center = RN_f32(sum / n) for non-empty clusters.
__global__ void grp_update_kernel(float* centers, const double* psum, const int32_t* pcnt, int64_t tiles,
                                  int count, int D) {
  const int64_t bh = blockIdx.x;
  const int d = threadIdx.x;
  for (int c = 0; c < count; ++c) {
    double s = 0.0;
    int64_t total = 0;
    for (int64_t t = 0; t < tiles; ++t) {
      const int64_t meta = (bh * tiles + t) * kMaxClusters + c;
      s = __dadd_rn(s, psum[meta * D + d]);
      total += pcnt[meta];
    }
    if (total > 0) centers[(bh * kMaxClusters + c) * D + d] = static_cast<float>(__ddiv_rn(s, static_cast<double>(total)));
  }
}

// grid (B*H), 64 threads: start offset of each (tile, label) in the sorted order.
__global__ void grp_offsets_kernel(const int32_t* pcnt, int64_t tiles, int count, int64_t* offsets) {
  __shared__ int64_t total[kMaxClusters];
  const int64_t bh = blockIdx.x;
  const int c = threadIdx.x;
  if (c < count) {
    int64_t s = 0;
    for (int64_t t = 0; t < tiles; ++t) s += pcnt[(bh * tiles + t) * kMaxClusters + c];
    total[c] = s;
  }
  __syncthreads();
  if (c < count) {
    int64_t off = 0;
    for (int i = 0; i < c; ++i) off += total[i];
    for (int64_t t = 0; t < tiles; ++t) {
      const int64_t meta = (bh * tiles + t) * kMaxClusters + c;
      offsets[meta] = off;
      off += pcnt[meta];
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
  auto run = [&](auto dt, auto dd) -> int {
    constexpr int DT = decltype(dt)::value, DD = decltype(dd)::value;
    grp_init_kernel<DT><<<dim3(BH), DD, 0, st>>>(v, H, v_sb, v_sh, v_sn, ids, count, DD, ws.centers);
    VCX_LAUNCHED("grp_init_kernel");
    for (int it = 0; it < iterations; ++it) {
      if (it + 1 < iterations) {
        grp_assign_kernel<DT, DD, true><<<dim3(tiles, BH), kGroupThreads, 0, st>>>(
            v, H, N, v_sb, v_sh, v_sn, count, ws.centers, lab, ws.psum, ws.pcnt);
        VCX_LAUNCHED("grp_assign_kernel<stats>");
        grp_update_kernel<<<dim3(BH), DD, 0, st>>>(ws.centers, ws.psum, ws.pcnt, tiles, count, DD);
        VCX_LAUNCHED("grp_update_kernel");
      } else {
        grp_assign_kernel<DT, DD, false><<<dim3(tiles, BH), kGroupThreads, 0, st>>>(
            v, H, N, v_sb, v_sh, v_sn, count, ws.centers, lab, nullptr, ws.pcnt);
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
