// C-ABI plumbing of libvcx: version, per-thread error text, workspace sizes.
#include "vcx_common.hpp"

namespace vcx {

size_t ws_prepare_qk(int64_t BH, int64_t N, int64_t D);
size_t ws_prepare_v(int64_t BH, int64_t N, int64_t D);
size_t ws_preprocess_qk(int64_t BH, int64_t N, int64_t D);
size_t ws_group(int64_t BH, int64_t N, int64_t D, int clusters);

std::string& last_error() {
  static thread_local std::string msg;
  return msg;
}

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  last_error() = buf;
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(VCX_EHIP, "%s launch failed: %s", what, hipGetErrorString(e));
  return VCX_OK;
}

// Each of the grid's one-wave blocks (8: the hardware deals consecutive blocks to the 8 XCDs
// in turn) reads the shader-clock counter (s_memtime, ticks at the current engine clock) and
// the constant-rate real-time counter (s_memrealtime) across a window of `ticks` real-time
// ticks. The window ends on the real-time counter alone, so the loop always terminates.
__global__ __launch_bounds__(64) void clock_probe_kernel(unsigned long long* out, unsigned long long ticks) {
  const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
  const unsigned long long c0 = __builtin_amdgcn_s_memtime();
  unsigned long long r = r0;
  while (r - r0 < ticks) {
    __builtin_amdgcn_s_sleep(2);
    r = __builtin_amdgcn_s_memrealtime();
  }
  const unsigned long long c1 = __builtin_amdgcn_s_memtime();
  if (threadIdx.x == 0) {
    out[2 * blockIdx.x] = c1 - c0;
    out[2 * blockIdx.x + 1] = r - r0;
  }
}

}  // namespace vcx

extern "C" int vcx_clock_probe(int64_t window_us, uint64_t* out, int* wall_khz, void* stream) {
  VCX_REQUIRE(out != nullptr && wall_khz != nullptr, "null pointer");
  VCX_REQUIRE(vcx::aligned(out, 8), "out must be 8-byte aligned");
  VCX_REQUIRE(window_us >= 1 && window_us <= 10000000, "window_us must be in [1, 10000000]");
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(wall_khz, hipDeviceAttributeWallClockRate, dev);
  if (e != hipSuccess) return vcx::fail(VCX_EHIP, "wall clock rate: %s", hipGetErrorString(e));
  VCX_REQUIRE(*wall_khz > 0, "device reports no wall clock rate");
  const unsigned long long ticks = static_cast<unsigned long long>(window_us) * static_cast<unsigned long long>(*wall_khz) / 1000ull;
  vcx::clock_probe_kernel<<<dim3(VCX_CLOCK_PROBE_BLOCKS), 64, 0, static_cast<hipStream_t>(stream)>>>(
      reinterpret_cast<unsigned long long*>(out), ticks > 0 ? ticks : 1);
  return vcx::check_launch("clock_probe_kernel");
}

extern "C" int vcx_abi_version(void) { return VCX_ABI_VERSION; }

extern "C" const char* vcx_last_error(void) { return vcx::last_error().c_str(); }

extern "C" int vcx_value_token(int p) {
  if (p < 0 || p >= vcx::kTile) return -1;
  return vcx::value_token(p);
}

extern "C" int vcx_workspace_bytes(int op, int64_t B, int64_t H, int64_t N, int64_t D, int smooth,
                                   int clusters, size_t* bytes) {
  (void)smooth;
  VCX_REQUIRE(bytes != nullptr, "bytes is null");
  VCX_REQUIRE(B >= 1 && H >= 1 && N >= 1 && D >= 1 && D <= 128, "invalid shape");
  VCX_REQUIRE(op == VCX_WS_PREPROCESS_QK || D == 64 || D == 128, "invalid shape");
  const int64_t BH = B * H;
  switch (op) {
    case VCX_WS_PREPROCESS_QK: *bytes = vcx::ws_preprocess_qk(BH, N, D); return VCX_OK;
    case VCX_WS_PREPARE_QK: *bytes = vcx::ws_prepare_qk(BH, N, D); return VCX_OK;
    case VCX_WS_PREPARE_V: *bytes = vcx::ws_prepare_v(BH, N, D); return VCX_OK;
    case VCX_WS_GROUP:
      VCX_REQUIRE(clusters >= 1 && clusters <= 256, "clusters must be in [1, 256]");
      *bytes = vcx::ws_group(BH, N, D, clusters);
      return VCX_OK;
    default: return vcx::fail(VCX_EINVAL, "unknown workspace op %d", op);
  }
}
