// status.hpp -- failure reporting shared by every translation unit (no HIP headers).
#pragma once
#include <string>

namespace kvc {
// Records a failure message for kvc_last_error() and returns `status`.
int set_error(int status, const std::string& msg);
}  // namespace kvc
