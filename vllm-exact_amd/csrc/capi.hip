// Library-level C ABI: version and status strings.
#include "common.h"

extern "C" const char* vxa_version(void) { return "vllm-exact-amd 0.1.0 (gfx950)"; }

extern "C" const char* vxa_status_string(int status) {
  switch (status) {
    case VXA_OK: return "ok";
    case VXA_ERR_ARG: return "invalid argument";
    case VXA_ERR_UNSUPPORTED: return "unsupported shape or config";
    case VXA_ERR_WORKSPACE: return "workspace missing or too small";
    case VXA_ERR_LAUNCH: return "kernel launch failed";
    case VXA_ERR_TOO_LARGE: return "problem larger than the fixed scratch of the no-allocation entry point";
    default: return "unknown status";
  }
}
