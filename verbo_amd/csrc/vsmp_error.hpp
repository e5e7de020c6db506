// Per-thread error text of the C ABI (read with vsmp_last_error).
#pragma once

#include <string>

namespace vsmp {

// Stores `msg` as the calling thread's last error and returns -1.
int set_error(const std::string& msg);
void clear_error();

}  // namespace vsmp
