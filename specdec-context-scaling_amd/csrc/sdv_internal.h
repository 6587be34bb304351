// Host+device shared internals of libsdv (not part of the public ABI).
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "sdv.h"
#include "sdv_device.h"

namespace sdv {

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

inline size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

}  // namespace sdv
