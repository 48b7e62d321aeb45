// cpb_internal.h -- what the library's host translation units share.
#pragma once
#include "cpb_moe.h"

namespace cpb {
// Record the message of a failing call (returned by cpb_moe_last_error() on
// this thread) and return code.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
}  // namespace cpb
