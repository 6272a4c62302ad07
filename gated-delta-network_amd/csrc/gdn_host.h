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

// Token-sequential recurrence (gdn_recurrent.hip) over num_seqs sequences:
// packed by cu (int32/int64 on the device) or, with cu == nullptr, of
// fixed_len tokens each.  With a non-null `enable`, the kernel does nothing
// unless *enable (on the device) is non-zero.  variant: row tiling index, -1 =
// built-in.  Error messages start with `what`.
int recurrent_launch(const uint16_t *q, const uint16_t *k, const uint16_t *v, const float *state,
                     const float *A_log, const uint16_t *a, const float *dt_bias,
                     const uint16_t *b, const void *cu, int cu64, int num_seqs, int T,
                     int fixed_len, const int *enable, float scale, uint16_t *out,
                     float *new_state, hipStream_t stream, int variant, const char *what);
int recurrent_num_variants();

}  // namespace gdn
