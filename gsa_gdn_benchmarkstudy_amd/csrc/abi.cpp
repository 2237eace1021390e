// Version and status-string entry points of the C ABI.
#include "../../include/gsa_hip.h"

extern "C" int gsa_abi_version(void) { return GSA_ABI_VERSION; }

extern "C" const char* gsa_status_string(int status) {
  switch (status) {
    case GSA_OK: return "ok";
    case GSA_ERR_NULL: return "a required pointer is NULL";
    case GSA_ERR_SHAPE: return "unsupported or inconsistent sizes";
    case GSA_ERR_DTYPE: return "unknown dtype code";
    case GSA_ERR_ALIGN: return "pointer or stride breaks the 16-byte vector-load alignment";
    case GSA_ERR_K: return "k out of range";
    case GSA_ERR_FLAGS: return "unknown flag or order code";
    case GSA_ERR_SCRATCH: return "sizes exceed the static scratch of gsa_indexer_select_noalloc";
    default: break;
  }
  return status < 0 ? "HIP launch error (negated hipError_t)" : "unknown status";
}
