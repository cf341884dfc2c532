// capi_internal.hpp -- host-side helpers shared by the C ABI's source files.
#pragma once

namespace mgpt {

// Records a printf-style description for mgpt_moe_last_error() on this host
// thread and returns `code`.
int fail(int code, const char* fmt, ...);

}  // namespace mgpt
