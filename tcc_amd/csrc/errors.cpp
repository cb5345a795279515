// Thread-local text of the last host-side error of the C-ABI.
#include <string>

#include "../../include/tcc_swtcf.h"

namespace tcc {
namespace {
thread_local std::string g_last_error;
}
void set_last_error(const std::string& msg) { g_last_error = msg; }
void clear_last_error() { g_last_error.clear(); }
}  // namespace tcc

extern "C" const char* tcc_last_error(void) { return tcc::g_last_error.c_str(); }
