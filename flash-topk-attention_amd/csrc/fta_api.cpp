// Library-wide C ABI pieces: error reporting and version query.
#include <string>

#include "fta_host.h"

namespace {
thread_local std::string g_last_error;
}

namespace fta {
void set_error(const std::string& msg) { g_last_error = msg; }
}  // namespace fta

extern "C" {
const char* fta_last_error(void) { return g_last_error.c_str(); }
int fta_version(void) { return 1; }
}
