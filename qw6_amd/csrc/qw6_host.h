// qw6_host.h -- host-side helpers shared by the library's translation units.
#pragma once

#include "qw6_hip.h"

namespace qw6 {

// Record an error message (qw6_hip_last_error, stderr); returns -1.
int qw6_fail(const char* fmt, ...);
// HIP device of a context.
int ctx_device(const qw6_hip_ctx_t* c);

}  // namespace qw6
