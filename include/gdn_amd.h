/*
 * gdn_amd.h -- C ABI of the MI355X (gfx950) Gated DeltaNet operators.
 *
 * Shapes are fixed by the operator definitions gdn_decode_qk4_v8_d128_k_last
 * and gdn_prefill_qk4_v8_d128_k_last: 4 q/k heads, 8 v-heads (head hv reads
 * q/k head hv/2), head size 128, recurrent state in k-last layout
 * [*, 8, 128 (V), 128 (K)] float32.  All tensors are dense, row-major and
 * live in device memory of the current HIP device.  bf16 tensors are passed
 * as their 16-bit patterns (gdn_bf16).  Nothing here allocates device memory
 * or synchronises the host; every launch goes to the given HIP stream
 * (NULL = the legacy default stream).
 *
 * Return value: GDN_OK (0) or a negative GDN_ERR_* code; gdn_last_error()
 * then describes the failure (thread-local, valid until the next call from
 * the same thread).
 */
#ifndef GDN_AMD_H
#define GDN_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t gdn_bf16;

#define GDN_OK 0
#define GDN_ERR_INVALID (-1)   /* bad pointer, size, alignment or aliasing */
#define GDN_ERR_LAUNCH (-2)    /* the HIP runtime refused a launch */
#define GDN_ERR_WORKSPACE (-3) /* workspace missing or smaller than required */

/* ABI version of this header; bumped on any signature change. */
int gdn_abi_version(void);

/* Text of the last error raised on the calling thread ("" if none). */
const char *gdn_last_error(void);

/*
 * One decode step (T = 1) for a batch of B sequences.
 *
 * Replaces the launch behind the reference's decode entry point
 * kernel(q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state):
 *   solutions/gdn_decode_qk4_v8_d128_k_last/solution/triton/kernel.py:85-113
 *   and its CUDA twin gdn_decode_cuda(), solution/cuda/binding.py:127-168.
 * Semantics: reference/gdn_decode_ref.py:12-83.
 *
 *   q, k      [B, 1, 4, 128] bf16      v         [B, 1, 8, 128] bf16
 *   state     [B, 8, 128, 128] f32 or NULL (treated as zeros)
 *   A_log     [8] f32                  a, b      [B, 1, 8] bf16
 *   dt_bias   [8] f32                  scale     > 0, already resolved
 *   output    [B, 1, 8, 128] bf16      new_state [B, 8, 128, 128] f32
 *
 * new_state may be the same buffer as state (in-place update); any other
 * overlap between an output and an input is rejected.  state/new_state must
 * be 16-byte aligned, q/k 8-byte aligned.
 */
int gdn_decode_fwd(const gdn_bf16 *q, const gdn_bf16 *k, const gdn_bf16 *v, const float *state,
                   const float *A_log, const gdn_bf16 *a, const float *dt_bias,
                   const gdn_bf16 *b, float scale, gdn_bf16 *output, float *new_state,
                   int batch, void *stream);

/*
 * gdn_decode_fwd with an explicit tiling, the counterpart of the block_v
 * argument of the reference's gdn_decode_cuda (solutions/
 * gdn_decode_qk4_v8_d128_k_last/solution/cuda/binding.py:127-131,206-211).
 * variant = tiling index (0..9, rows per workgroup 128/64/32/16/32/32/16/8/64/64
 * with 256/256/256/256/128/64/64/64/128/64 threads) + 16 for non-temporal state
 * loads/stores; -1 = the built-in choice for the batch size (what
 * gdn_decode_fwd uses).  Results are identical for every variant.
 */
int gdn_decode_fwd_variant(const gdn_bf16 *q, const gdn_bf16 *k, const gdn_bf16 *v,
                           const float *state, const float *A_log, const gdn_bf16 *a,
                           const float *dt_bias, const gdn_bf16 *b, float scale,
                           gdn_bf16 *output, float *new_state, int batch, void *stream,
                           int variant);

/*
 * Decode of `tokens` >= 1 consecutive tokens per batch row (multi-token /
 * speculative decode): for each row, the T = 1 step of gdn_decode_fwd applied
 * token after token, the state read once, carried on chip between tokens and
 * written once at the end.  No counterpart in the reference, whose decode asserts
 * T == 1 (reference/gdn_decode_ref.py:32-36); it extends the same entry point
 * kernel(q, k, v, state, ...) of solutions/gdn_decode_qk4_v8_d128_k_last/
 * solution/triton/kernel.py:85 to T > 1, and equals gdn_prefill_fwd on `batch`
 * sequences of `tokens` tokens each (reference/gdn_prefill_ref.py:71-89).
 *
 *   q, k      [B, T, 4, 128] bf16      v         [B, T, 8, 128] bf16
 *   a, b      [B, T, 8] bf16           output    [B, T, 8, 128] bf16
 *   state, new_state, A_log, dt_bias, scale as for gdn_decode_fwd.
 *
 * variant: row tiling of the token-sequential kernel (0..9: 4, 8, 16, 8, 16,
 * 32, 16, 64, 32, 64 rows per workgroup with 64, 128, 256, 64, 128, 256, 64,
 * 256, 64, 64 threads; every tiling gives identical results), 10 = the block
 * kernel (one workgroup per row and v-head applies the tokens in blocks of 16
 * in the chunked form on MFMA; same function within the stated tolerances,
 * not bit for bit), -1 = built-in: tokens == 1 runs gdn_decode_fwd, more run
 * token by token or in blocks by a cost model fitted on MI355X (blocks from
 * about 4 tokens at 64 rows, 6 at 16 rows).
 */
int gdn_decode_multi_fwd(const gdn_bf16 *q, const gdn_bf16 *k, const gdn_bf16 *v,
                         const float *state, const float *A_log, const gdn_bf16 *a,
                         const float *dt_bias, const gdn_bf16 *b, float scale,
                         gdn_bf16 *output, float *new_state, int batch, int tokens, void *stream,
                         int variant);

/*
 * Decode for any head layout: num_qk_heads q/k heads and num_v_heads v-heads
 * (a multiple of num_qk_heads; v-head h reads q/k head h / (num_v_heads /
 * num_qk_heads)), head size 128, `tokens` >= 1 per row.  No counterpart in the
 * reference, whose definitions fix 4/8 heads (reference/gdn_decode_ref.py:32-36);
 * the contest behind it names other layouts such as 16/32 (FAQ.md:109-111).
 * Tensors are those of gdn_decode_multi_fwd with 4 -> num_qk_heads and
 * 8 -> num_v_heads.  variant: with tokens == 1 and -1 the decode kernel's
 * built-in tiling; otherwise the token-sequential kernel's tiling (as for
 * gdn_decode_multi_fwd).
 */
int gdn_decode_fwd_heads(const gdn_bf16 *q, const gdn_bf16 *k, const gdn_bf16 *v,
                         const float *state, const float *A_log, const gdn_bf16 *a,
                         const float *dt_bias, const gdn_bf16 *b, float scale,
                         gdn_bf16 *output, float *new_state, int batch, int tokens,
                         int num_qk_heads, int num_v_heads, void *stream, int variant);

/*
 * Bytes of device workspace gdn_prefill_fwd needs for a packed batch of
 * total_tokens tokens in num_seqs sequences.  The bound does not depend on the
 * individual lengths (they stay on the device), so a caller can size it once.
 * Replaces the module-level buffer cache of the reference prefill,
 * solutions/gdn_prefill_qk4_v8_d128_k_last/solution/triton/fla_kernels.py:950-957.
 */
size_t gdn_prefill_workspace_bytes(int total_tokens, int num_seqs);

/*
 * Where a prefill call leaves, in its workspace, whether cu_seqlens kept the
 * contract below: num_seqs int32 words from this byte offset, word s = bit 0
 * if cu_seqlens[s+1] < cu_seqlens[s], bit 1 if either is outside [0, T]; all
 * zero for a well-formed batch.  Every call with num_seqs >= 1 writes them on
 * the device, in the first kernel that reads the bounds, so the check needs
 * no host read or sync of cu_seqlens.  -1 for invalid arguments.  No
 * counterpart in the reference, which reads the bounds on the host and skips
 * a sequence whose length is not positive (reference/gdn_prefill_ref.py:55-61)
 * without reporting it.
 */
long long gdn_prefill_status_offset(int total_tokens, int num_seqs, int num_qk_heads,
                                    int num_v_heads);

/*
 * Reader of those words for tests and debugging (it synchronizes: not for
 * the hot path): waits for `stream`, then ORs the num_seqs words the last
 * prefill call on `workspace` with this (T, N, heads) left into *status (0:
 * well-formed).  workspace NULL reads the scratch of gdn_prefill_fwd_noalloc
 * on the current device.  No counterpart in the reference.
 */
int gdn_prefill_status(const void *workspace, int total_tokens, int num_seqs, int num_qk_heads,
                       int num_v_heads, void *stream, int *status);

/*
 * Chunked prefill over a packed batch of variable-length sequences.
 *
 * Replaces the six launches behind the reference's prefill entry point
 * kernel(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, output,
 * new_state): solutions/gdn_prefill_qk4_v8_d128_k_last/solution/triton/
 * fla_kernels.py:975-1053.  Semantics: reference/gdn_prefill_ref.py:12-91.
 *
 *   q, k       [T, 4, 128] bf16         v          [T, 8, 128] bf16
 *   state      [N, 8, 128, 128] f32 or NULL (treated as zeros)
 *   A_log      [8] f32                  a, b       [T, 8] bf16
 *   dt_bias    [8] f32                  cu_seqlens [N + 1] int32 or int64
 *   scale      > 0, already resolved    output     [T, 8, 128] bf16
 *   new_state  [N, 8, 128, 128] f32     workspace  >= gdn_prefill_workspace_bytes(T, N)
 *
 * cu_seqlens stays on the device and is never read by the host.  Sequence s
 * is the tokens [cu_seqlens[s], cu_seqlens[s+1]); the offsets must be
 * non-decreasing and within [0, T], but need not start at 0 or end at T: as
 * in the reference (gdn_prefill_ref.py:49-62), the output rows before
 * cu_seqlens[0] and from cu_seqlens[N] on are written as zeros, and a single
 * sequence's state covers exactly its own tokens (a batch outside this
 * contract leaves the outputs unspecified but never accesses memory out of
 * bounds, and says so in its status words: gdn_prefill_status_offset).  With
 * num_seqs = 0 the whole output is zeroed and the workspace may be NULL.  A
 * zero-length sequence gets an all-zero new_state, as the reference does.
 * new_state may alias state; output must be 16-byte aligned and must not
 * overlap any input.
 *
 * The batch takes one of three paths: every sequence token by token with the
 * state in registers (one launch), every sequence in 16-token blocks with the
 * state in MFMA tiles (one launch: the block kernel of gdn_decode_multi_fwd),
 * or all through the chunk-64 pipeline.  A batch of at most 96 tokens runs
 * sequentially (one sequence in blocks when a cost model favours them),
 * a longer single sequence through the chunks; for the others the
 * host picks the faster sequential kind at the mean length and, unless the
 * chunks win for any longest sequence, the device compares cost models of
 * it and of the chunks from the longest sequence, the chunk count, T and N
 * (fitted on MI355X: many short-to-medium sequences go in blocks, e.g. 64 x
 * 256 tokens 115 us vs 171 us through the chunks).  Results agree within the
 * stated tolerance either way (the reference measured the same crossover
 * between its sequential scan and chunked kernels,
 * OPTIMIZATION_LOG.md:79,170-184).
 */
int gdn_prefill_fwd(const gdn_bf16 *q, const gdn_bf16 *k, const gdn_bf16 *v,
                    const float *state, const float *A_log, const gdn_bf16 *a,
                    const float *dt_bias, const gdn_bf16 *b, const void *cu_seqlens,
                    int cu_seqlens_is_int64, int num_seqs, int total_tokens, float scale,
                    gdn_bf16 *output, float *new_state, void *workspace,
                    size_t workspace_bytes, void *stream);

/*
 * gdn_prefill_fwd with an explicit form of the per-chunk operands:
 * variant 0 = WY form (the intra kernel forms w = (I+A)^-1 beta e^G K and
 * u = (I+A)^-1 beta V; each serial state step is v_new = u - w S: the
 * shortest chain), 1 = T form (the intra kernel stores only (I+A)^-1; each
 * state step forms beta V - beta e^G K S from the inputs: less memory
 * traffic, one more exchange per step), -1 = the built-in choice (what
 * gdn_prefill_fwd uses, decided on the device: the T form for batches of at
 * least 144 chunks with more than three times the chunks of their longest
 * sequence, or of at least 384 with at least 1.5 times, and for batches of
 * at most 768 state units -- sequence x v-head x 16-column block -- whose
 * longest sequence has at most 12 chunks; the WY form otherwise and for one
 * sequence: t_form_wins in csrc/gdn_common.h), 2 = WY form with one
 * serial chain of state steps per sequence, 3 = WY form with the two-segment
 * scan for a single sequence of at least two chunks (the second half of the
 * chunks runs beside the first from a zero state and from the identity, and
 * one more launch applies the first half's final state: half the serial
 * chain; 0 and -1 take it from 9 chunks on when 24 x num_v_heads <= 256;
 * with 8 v-heads and at least 30 first-half chunks the state launch also
 * computes the first half's output as its chain goes, on the CUs the scan
 * leaves idle), 4 = as 3 with that early output stopped after one chunk per
 * workgroup (a test of the path that computes the rest afterwards; same
 * results as 3).
 * The counterpart of
 * the reference's autotuned launch parameters of
 * chunk_gated_delta_rule_fwd_kernel_h (solutions/
 * gdn_prefill_qk4_v8_d128_k_last/solution/triton/fla_kernels.py:407-426,
 * 1028-1035).  Both forms compute the same function within the stated
 * tolerances (not bit for bit); a batch that runs token by token does not
 * depend on the variant.
 */
int gdn_prefill_fwd_variant(const gdn_bf16 *q, const gdn_bf16 *k, const gdn_bf16 *v,
                            const float *state, const float *A_log, const gdn_bf16 *a,
                            const float *dt_bias, const gdn_bf16 *b, const void *cu_seqlens,
                            int cu_seqlens_is_int64, int num_seqs, int total_tokens, float scale,
                            gdn_bf16 *output, float *new_state, void *workspace,
                            size_t workspace_bytes, void *stream, int variant);

/*
 * gdn_prefill_fwd with every tuning choice explicit (for sweeps and tests):
 *   state_tiling       the form, as the variant of gdn_prefill_fwd_variant
 *                      (-1 built-in)
 *   recurrent_max_len  a batch whose longest sequence has at most this many
 *                      tokens runs through the sequential kernel; -1 =
 *                      built-in, -2 = never (always chunked)
 *   recurrent_tiling   the sequential kernel, as the variant of
 *                      gdn_decode_multi_fwd (10 = blocks; -1 built-in: token
 *                      by token, or under the built-in path choice the kind
 *                      it picks)
 */
int gdn_prefill_fwd_tuned(const gdn_bf16 *q, const gdn_bf16 *k, const gdn_bf16 *v,
                          const float *state, const float *A_log, const gdn_bf16 *a,
                          const float *dt_bias, const gdn_bf16 *b, const void *cu_seqlens,
                          int cu_seqlens_is_int64, int num_seqs, int total_tokens, float scale,
                          gdn_bf16 *output, float *new_state, void *workspace,
                          size_t workspace_bytes, void *stream, int state_tiling,
                          int recurrent_max_len, int recurrent_tiling);

/*
 * Prefill for any head layout (see gdn_decode_fwd_heads): the workspace size
 * and gdn_prefill_fwd_tuned with num_qk_heads / num_v_heads in place of 4 / 8
 * (q, k [T, num_qk_heads, 128]; v, output [T, num_v_heads, 128]; a, b
 * [T, num_v_heads]; A_log, dt_bias [num_v_heads]; state, new_state
 * [N, num_v_heads, 128, 128]).  No counterpart in the reference (4/8 heads
 * only, reference/gdn_prefill_ref.py:33-36).  The workspace size is 0 for an
 * invalid layout.
 */
size_t gdn_prefill_workspace_bytes_heads(int total_tokens, int num_seqs, int num_qk_heads,
                                         int num_v_heads);
int gdn_prefill_fwd_heads(const gdn_bf16 *q, const gdn_bf16 *k, const gdn_bf16 *v,
                          const float *state, const float *A_log, const gdn_bf16 *a,
                          const float *dt_bias, const gdn_bf16 *b, const void *cu_seqlens,
                          int cu_seqlens_is_int64, int num_seqs, int total_tokens,
                          int num_qk_heads, int num_v_heads, float scale, gdn_bf16 *output,
                          float *new_state, void *workspace, size_t workspace_bytes, void *stream,
                          int state_tiling, int recurrent_max_len, int recurrent_tiling);

/*
 * gdn_prefill_fwd without a workspace argument: an entry point that
 * allocates nothing, for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  Same arguments, semantics,
 * kernels and results as gdn_prefill_fwd; the workspace is a static device
 * array of GDN_PREFILL_SCRATCH_BYTES per GPU, held until the process ends, so
 * a batch needing more (gdn_prefill_workspace_bytes(T, N) above the maximum:
 * e.g. one sequence of more than ~3,700 tokens) is refused with
 * GDN_ERR_WORKSPACE.  `stream` must belong to the current device.  Calls that
 * overlap in time on one GPU share that array and race: order them (one
 * stream, or events).  The first call on a device looks up the array's
 * device address (no allocation).
 */
#define GDN_PREFILL_SCRATCH_BYTES (64u << 20)
int gdn_prefill_fwd_noalloc(const gdn_bf16 *q, const gdn_bf16 *k, const gdn_bf16 *v,
                            const float *state, const float *A_log, const gdn_bf16 *a,
                            const float *dt_bias, const gdn_bf16 *b, const void *cu_seqlens,
                            int cu_seqlens_is_int64, int num_seqs, int total_tokens, float scale,
                            gdn_bf16 *output, float *new_state, void *stream);

/*
 * Measurement support (no counterpart in the reference): copies `bytes`
 * bytes from src to dst in the decode kernel's access pattern (one wave per
 * 32 KiB, every load before the first store, non-temporal), i.e. the HBM
 * streaming ceiling of a kernel that reads and writes each byte of a state
 * once at that size, launch ramp included.  bytes must be a multiple of
 * 32768; src and dst 16-byte aligned and disjoint.  bench.py reports the
 * decode step against it.
 */
int gdn_stream_copy(const void *src, void *dst, size_t bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* GDN_AMD_H */
