// rt_capi_util.hpp -- error-reporting helpers shared by the C ABI sources.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/rt_hip.h"

namespace rt {

// Record a printf-style message for rt_last_error() and return `code`.
rt_status set_error(rt_status code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// RT_OK for hipSuccess, otherwise RT_ENOMEM / RT_EHIP with the HIP message.
rt_status hip_error(hipError_t e, const char *what);
bool aligned16(const void *p);

}  // namespace rt
