// Host-side helpers shared by the C-ABI entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>


#include "gdn_amd.h"
#include "gdn_args.h"
#include "gdn_device.h"

namespace gdn {

// Checks the launch that was just enqueued; GDN_ERR_LAUNCH on failure.
int check_launch(const char *what);

// Token-sequential recurrence (gdn_recurrent.hip) over num_seqs sequences:
// packed by cu (int32/int64 on the device) or, with cu == nullptr, of
// fixed_len tokens each.  With a non-null `enable`, the kernel does nothing
// unless *enable (on the device) is non-zero.  With a non-null `status` (and
// cu), status[s] receives the contract bits of sequence s (cu_status_bits).
// variant: row tiling index, -1 = built-in.  Error messages start with `what`.
int recurrent_launch(const uint16_t *q, const uint16_t *k, const uint16_t *v, const float *state,
                     const float *A_log, const uint16_t *a, const float *dt_bias,
                     const uint16_t *b, const void *cu, int cu64, int num_seqs, int T,
                     int fixed_len, const int *enable, int *status, const Heads &H,
                     float scale, uint16_t *out, float *new_state, hipStream_t stream,
                     int variant, const char *what);
int recurrent_num_variants();
// The variant of recurrent_launch that runs block_launch.
int recurrent_block_variant();

// The same cases in 16-token blocks of the chunked form (gdn_block.hip): one
// workgroup per (sequence, v-head), or two (64 state columns each) for
// batches of at most 128 such pairs.  Arguments as recurrent_launch's.
int block_launch(const uint16_t *q, const uint16_t *k, const uint16_t *v, const float *state,
                 const float *A_log, const uint16_t *a, const float *dt_bias, const uint16_t *b,
                 const void *cu, int cu64, int num_seqs, int T, int fixed_len, const int *enable,
                 int *status, const Heads &H, float scale, uint16_t *out, float *new_state,
                 hipStream_t stream, const char *what);

// One decode step (gdn_decode.hip) with head layout H; variant as in
// gdn_decode_fwd_variant.  Validates its arguments; messages start with `what`.
int decode_launch(const gdn_bf16 *q, const gdn_bf16 *k, const gdn_bf16 *v, const float *state,
                  const float *A_log, const gdn_bf16 *a, const float *dt_bias, const gdn_bf16 *b,
                  float scale, gdn_bf16 *output, float *new_state, int batch, void *stream,
                  int variant, const Heads &H, const char *what);

}  // namespace gdn
