// Error reporting and version entry points of the C ABI.
#include <string>

#include "sg_common.h"

namespace sg {

namespace {
thread_local std::string g_last_error;
}

int set_error(int code, const std::string& message) {
  g_last_error = message;
  return code;
}

void clear_error() { g_last_error.clear(); }

}  // namespace sg

extern "C" int sg_abi_version(void) { return SG_ABI_VERSION; }

extern "C" const char* sg_last_error(void) { return sg::g_last_error.c_str(); }

extern "C" int64_t sg_abi_struct_size(int32_t which) {
  switch (which) {
    case 0: return static_cast<int64_t>(sizeof(SgTreeAttnArgs));
    case 1: return static_cast<int64_t>(sizeof(SgKvCommitArgs));
    case 2: return static_cast<int64_t>(sizeof(SgTreeSampleArgs));
    case 3: return static_cast<int64_t>(sizeof(SgKvSplitArgs));
    case 4: return static_cast<int64_t>(sizeof(SgLmHeadArgs));
    case 5: return static_cast<int64_t>(sizeof(SgAddRmsNormArgs));
    case 6: return static_cast<int64_t>(sizeof(SgQkNormRopeArgs));
    default: return -1;
  }
}
