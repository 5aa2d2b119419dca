// Internal helpers shared by the library's translation units: the thread-local error message.
#pragma once

#include <string>

#include "../../include/kea_lowbit.h"

namespace kea {

// Records `message` as the calling thread's last error and returns `code` (a KEA_E* value or a hipError_t).
int fail(int code, const std::string &message);

// A dispatch packet holds each grid dimension as a 32-bit count of work-items: `blocks` workgroups of `threads`
// work-items along one dimension must stay within it, or the launch would be truncated and leave work undone.
inline bool fits_dispatch(long long blocks, long long threads) {
    return blocks >= 0 && blocks * threads <= 0xFFFFFFFFLL;
}

}  // namespace kea
