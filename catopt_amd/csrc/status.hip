// ABI version, status strings and the per-thread HIP error slot.
#include "common.hpp"

namespace catopt {
static thread_local int32_t g_last_hip_error = 0;

int32_t set_hip_error(hipError_t e) {
  g_last_hip_error = static_cast<int32_t>(e);
  return CATOPT_E_HIP;
}
}  // namespace catopt

extern "C" int32_t catopt_hip_abi_version(void) { return CATOPT_HIP_ABI_VERSION; }

extern "C" const char* catopt_hip_strerror(int32_t status) {
  switch (status) {
    case CATOPT_OK: return "ok";
    case CATOPT_E_INVAL: return "invalid argument";
    case CATOPT_E_UNSUPPORTED: return "unsupported configuration";
    case CATOPT_E_HIP: return "HIP runtime error";
    case CATOPT_E_WORKSPACE: return "workspace too small";
    default: return "unknown status";
  }
}

extern "C" int32_t catopt_hip_last_hip_error(void) { return catopt::g_last_hip_error; }
