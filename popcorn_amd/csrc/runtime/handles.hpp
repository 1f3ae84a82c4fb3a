// Definitions of the opaque C-ABI handle types shared by the runtime's
// translation units.
#pragma once

#include <memory>

#include "popcorn.hpp"

struct popcorn_library_s {
    std::unique_ptr<popcorn::KernelLibrary> lib;
};
