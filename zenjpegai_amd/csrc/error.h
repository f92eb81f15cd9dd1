// Error carrying one of the ZJAI_E_* status codes across the C++ internals; the C-ABI catches
// it and returns the code (no exception crosses the ABI). Host-only, no HIP headers.
#pragma once

#include <stdexcept>
#include <string>

namespace zjai {

struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

}  // namespace zjai
