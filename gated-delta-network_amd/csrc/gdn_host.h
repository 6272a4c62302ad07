// Host-side helpers shared by the C-ABI entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "gdn_amd.h"

namespace gdn {

// Records a printf-style message as the calling thread's last error and
// returns `code` so call sites can write `return fail(GDN_ERR_INVALID, ...)`.
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

// Clears the calling thread's last error.
void clear_error();

// Checks the launch that was just enqueued; GDN_ERR_LAUNCH on failure.
int check_launch(const char *what);

inline bool aligned(const void *p, size_t a) {
  return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

// True when [a, a + na) and [b, b + nb) share at least one byte.
inline bool overlaps(const void *a, size_t na, const void *b, size_t nb) {
  if (!a || !b || na == 0 || nb == 0) return false;
  const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
  return x < y + nb && y < x + na;
}

}  // namespace gdn
