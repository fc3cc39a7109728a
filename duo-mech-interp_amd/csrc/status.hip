// Status strings and ABI version of the q35hip C library.
#include "q35hip.h"

extern "C" const char* q35_status_string(int status) {
  switch (status) {
    case Q35_OK: return "ok";
    case Q35_EINVAL: return "invalid argument (null pointer, non-positive or inconsistent size)";
    case Q35_EUNSUPPORTED: return "unsupported size or dtype for this build";
    case Q35_EWORKSPACE: return "workspace missing or too small";
    case Q35_ELAUNCH: return "kernel launch failed";
    case Q35_ESCRATCH: return "request exceeds the fixed scratch of an allocation-free entry point";
    default: return "unknown status";
  }
}

extern "C" int q35_abi_version(void) { return 14; }
