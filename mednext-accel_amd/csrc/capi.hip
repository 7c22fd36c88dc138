// C-ABI glue shared by all kernel families: the per-thread error message slot
// and the ABI revision.
#include "common.h"

namespace mednext {
namespace {
thread_local std::string g_last_error;
}  // namespace

void set_error(const std::string& msg) { g_last_error = msg; }

}  // namespace mednext

extern "C" const char* mednext_hip_last_error(void) { return mednext::g_last_error.c_str(); }

extern "C" int32_t mednext_hip_abi_version(void) { return 14; }
