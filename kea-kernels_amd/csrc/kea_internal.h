// Internal helpers shared by the library's translation units: the thread-local error message.
#pragma once

#include <string>

#include "../../include/kea_lowbit.h"

namespace kea {

// Records `message` as the calling thread's last error and returns `code` (a KEA_E* value or a hipError_t).
int fail(int code, const std::string &message);

}  // namespace kea
