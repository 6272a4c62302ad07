// Host-side helpers shared by the C-ABI entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>


#include "gdn_amd.h"
#include "gdn_device.h"

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

// Validates a head layout (q/k heads hqk >= 1, v-heads hv a multiple of hqk,
// at most kMaxHeads) into H; GDN_ERR_INVALID with a message otherwise.
constexpr int kMaxHeads = 1024;
inline int make_heads(int hqk, int hv, const char *what, Heads &H) {
  if (hqk < 1 || hv < 1 || hv > kMaxHeads || hv % hqk != 0)
    return fail(GDN_ERR_INVALID, "%s: heads %d q/k, %d v (need v a multiple of q/k, <= %d)", what,
                hqk, hv, kMaxHeads);
  H = Heads{hqk, hv, hv / hqk};
  return GDN_OK;
}

// Token-sequential recurrence (gdn_recurrent.hip) over num_seqs sequences:
// packed by cu (int32/int64 on the device) or, with cu == nullptr, of
// fixed_len tokens each.  With a non-null `enable`, the kernel does nothing
// unless *enable (on the device) is non-zero.  variant: row tiling index, -1 =
// built-in.  Error messages start with `what`.
int recurrent_launch(const uint16_t *q, const uint16_t *k, const uint16_t *v, const float *state,
                     const float *A_log, const uint16_t *a, const float *dt_bias,
                     const uint16_t *b, const void *cu, int cu64, int num_seqs, int T,
                     int fixed_len, const int *enable, const Heads &H, float scale,
                     uint16_t *out, float *new_state, hipStream_t stream, int variant,
                     const char *what);
int recurrent_num_variants();
// The variant of recurrent_launch that runs block_launch.
int recurrent_block_variant();

// The same cases in 16-token blocks of the chunked form (gdn_block.hip): one
// workgroup per (sequence, v-head), or two (64 state columns each) for
// batches of at most 128 such pairs.  Arguments as recurrent_launch's.
int block_launch(const uint16_t *q, const uint16_t *k, const uint16_t *v, const float *state,
                 const float *A_log, const uint16_t *a, const float *dt_bias, const uint16_t *b,
                 const void *cu, int cu64, int num_seqs, int T, int fixed_len, const int *enable,
                 const Heads &H, float scale, uint16_t *out, float *new_state,
                 hipStream_t stream, const char *what);

// Path cost models in microseconds, fitted to graph-replay sweeps of each
// path on MI355X (sequence count N = 1..256 of equal lengths L = 8..256,
// multi-token decode B = 1..128 with 4..16 tokens).  L = longest sequence,
// T = tokens, nt = chunks of 64, g = N * hv (sequence, v-head) groups.
// Token by token (recurrent kernel): the serial token chain plus VALU work
// per token and state traffic per group.
__host__ __device__ inline float cost_by_token(float L, float T, float hv, float g) {
  return 3.0f + 0.24f * L + 0.003f * T * hv + 0.021f * g;
}
// 16-token blocks (block kernel): two workgroups of 64 columns per group up
// to 128 groups (~2.8 us per block), then one of 128 columns per group, two
// resident per CU (512 on the chip): ~3.5 us per block alone on a CU, ~4.7 us
// two to a CU; plus the state's traffic per group.
__host__ __device__ inline float cost_by_block(float L, float g) {
  const float rounds = ceilf(g / 512.0f), blocks = ceilf(L / 16.0f);
  const float per_block = g <= 128.0f ? 2.8f : g <= 256.0f ? 3.5f : 4.7f;
  return 4.5f + 0.015f * g + 0.008f * fmaxf(g - 256.0f, 0.0f) + rounds * blocks * per_block;
}
// Chunks: fixed launches, per-sequence work up to ~40 sequences and the
// per-chunk throughput beyond, plus the serial chunk chain of the longest.
__host__ __device__ inline float cost_by_chunks(float L, float nt, float hv, float g) {
  const float per_seq = fminf(0.13f * g, 11.0f + 0.081f * g);
  return 20.0f + fmaxf(per_seq, 0.081f * nt * hv) + 0.5f * ceilf(L / 64.0f);
}

// One decode step (gdn_decode.hip) with head layout H; variant as in
// gdn_decode_fwd_variant.  Validates its arguments; messages start with `what`.
int decode_launch(const gdn_bf16 *q, const gdn_bf16 *k, const gdn_bf16 *v, const float *state,
                  const float *A_log, const gdn_bf16 *a, const float *dt_bias, const gdn_bf16 *b,
                  float scale, gdn_bf16 *output, float *new_state, int batch, void *stream,
                  int variant, const Heads &H, const char *what);

}  // namespace gdn
