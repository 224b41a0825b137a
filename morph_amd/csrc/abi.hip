// Library-wide C entry points: ABI version and status strings.
#include "common.h"

extern "C" int morph_abi_version(void) { return MORPH_ABI_VERSION; }

extern "C" const char* morph_strerror(int status) {
  switch (status) {
    case MORPH_OK: return "ok";
    case MORPH_EINVAL: return "invalid argument (null pointer, negative size or bad count)";
    case MORPH_EDTYPE: return "unsupported dtype";
    case MORPH_ELAUNCH: return "HIP kernel launch failed";
    case MORPH_ERANGE: return "size exceeds what this entry point supports";
    case MORPH_EWORKSPACE: return "workspace missing or too small";
    default: return "unknown morph status";
  }
}
