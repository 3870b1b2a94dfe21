// hcg_runtime.h -- host-side state shared by the library's source files.
#pragma once

#include <string>

#define HCG_INTERNAL __attribute__((visibility("hidden")))

namespace hcg {

// Text of the calling thread's last error, returned by hcg_last_error().
HCG_INTERNAL extern thread_local std::string t_last_error;

// Records a printf-style message as the thread's last error; returns code.
HCG_INTERNAL int set_error(int code, const char* fmt, ...);

}  // namespace hcg
