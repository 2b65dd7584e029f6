// host_status.hpp — the library's error reporting, with no HIP dependency,
// so that the host-only parts (page policy, arena free list) also build as
// plain C++ (a sanitizer build of them includes only this header).
#pragma once

#include "../../include/nyion_hip.h"

namespace nyion {

// Records `fmt` as this thread's nyion_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

}  // namespace nyion
