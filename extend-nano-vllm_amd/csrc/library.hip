// Library-level entry points: status names and version.
#include "common.h"

extern "C" const char* nva_status_string(int status) {
  switch (status) {
    case NVA_OK: return "ok";
    case NVA_ERR_ARG: return "invalid argument";
    case NVA_ERR_WORKSPACE: return "workspace missing or too small";
    case NVA_ERR_UNSUPPORTED: return "unsupported configuration";
    case NVA_ERR_LAUNCH: return "kernel launch failed";
    case NVA_ERR_CAPACITY: return "input exceeds the static scratch capacity";
    default: return "unknown status";
  }
}

extern "C" const char* nva_version(void) { return "nanovllm_amd 0.1.0 gfx950"; }
