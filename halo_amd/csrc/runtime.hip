// Error reporting and build metadata for the C-ABI.
#include "common.hpp"

namespace halo {
namespace {
thread_local std::string g_last_error;
}
void set_error(const std::string& msg) { g_last_error = msg; }
}  // namespace halo

extern "C" const char* halo_last_error(void) { return halo::g_last_error.c_str(); }

extern "C" const char* halo_build_info(void) {
  return "halo_amd HIP kernels for gfx950 (wave64); hipcc " __clang_version__;
}

// Device-visible address of pinned host memory (hipHostMalloc / a pinned
// tensor), so kernels can read cold-tier chunks in place over the host link.
extern "C" int halo_host_device_pointer(const void* host, void** dev) {
  if (host == nullptr || dev == nullptr) {
    halo::set_error("null pointer argument");
    return HALO_E_INVALID;
  }
  *dev = nullptr;
  hipPointerAttribute_t attr;
  if (hipPointerGetAttributes(&attr, host) != hipSuccess || attr.type != hipMemoryTypeHost) {
    (void)hipGetLastError();
    halo::set_error("not pinned host memory (hipHostMalloc / pin_memory)");
    return HALO_E_INVALID;
  }
  void* d = nullptr;
  if (hipHostGetDevicePointer(&d, const_cast<void*>(host), 0) != hipSuccess || d == nullptr) {
    (void)hipGetLastError();
    halo::set_error("hipHostGetDevicePointer failed");
    return HALO_E_HIP;
  }
  *dev = d;
  return HALO_OK;
}
