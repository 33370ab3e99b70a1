// internal.hpp -- helpers shared by the host-side translation units (not exported).
#pragma once

namespace ebh {
// Record this thread's error message (returned by ebh_last_error) and return code.
__attribute__((visibility("hidden"), format(printf, 2, 3))) int set_error(int code,
                                                                          const char* fmt, ...);
}  // namespace ebh
