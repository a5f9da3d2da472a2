// Host-side helpers shared by the C ABI translation units.
#pragma once

#include <string>

namespace gi {

// Records the calling thread's last error text and returns code.
int set_error(int code, const std::string &msg);
void clear_error();

} // namespace gi
