// Thread-local last-error text shared by every C entry point of the library.
#pragma once

#include <string>

namespace tge {
void set_last_error(const std::string& message);
}  // namespace tge
