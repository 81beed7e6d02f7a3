// C-ABI plumbing of libvcx: version, per-thread error text, workspace sizes.
#include "vcx_common.hpp"

namespace vcx {

size_t ws_prepare_qk(int64_t BH, int64_t N, int64_t D);
size_t ws_prepare_v(int64_t BH, int64_t N, int64_t D);
size_t ws_preprocess_qk(int64_t BH, int64_t N, int64_t D);
size_t ws_group(int64_t BH, int64_t N, int64_t D);

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

}  // namespace vcx

extern "C" int vcx_abi_version(void) { return VCX_ABI_VERSION; }

extern "C" const char* vcx_last_error(void) { return vcx::last_error().c_str(); }

extern "C" int vcx_value_token(int p) {
  if (p < 0 || p >= vcx::kTile) return -1;
  return vcx::value_token(p);
}

extern "C" int vcx_workspace_bytes(int op, int64_t B, int64_t H, int64_t N, int64_t D, int smooth,
                                   int clusters, size_t* bytes) {
  (void)smooth;
  (void)clusters;
  VCX_REQUIRE(bytes != nullptr, "bytes is null");
  VCX_REQUIRE(B >= 1 && H >= 1 && N >= 1 && D >= 1 && D <= 128, "invalid shape");
  VCX_REQUIRE(op == VCX_WS_PREPROCESS_QK || D == 64 || D == 128, "invalid shape");
  const int64_t BH = B * H;
  switch (op) {
    case VCX_WS_PREPROCESS_QK: *bytes = vcx::ws_preprocess_qk(BH, N, D); return VCX_OK;
    case VCX_WS_PREPARE_QK: *bytes = vcx::ws_prepare_qk(BH, N, D); return VCX_OK;
    case VCX_WS_PREPARE_V: *bytes = vcx::ws_prepare_v(BH, N, D); return VCX_OK;
    case VCX_WS_GROUP: *bytes = vcx::ws_group(BH, N, D); return VCX_OK;
    default: return vcx::fail(VCX_EINVAL, "unknown workspace op %d", op);
  }
}
