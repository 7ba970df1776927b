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
