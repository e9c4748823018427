// Shared host-side helpers of the library.
#pragma once

#include <string>

namespace wc {

// Records `msg` as this thread's last error and returns `code`.
int fail(int code, const std::string& msg);
extern thread_local std::string g_last_error;

}  // namespace wc
