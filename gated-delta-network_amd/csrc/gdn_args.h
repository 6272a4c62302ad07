// Host-side argument checks, workspace layout and path planning of the C-ABI
// entry points.  Everything here is plain host code (no HIP header, no device
// call), defined in gdn_args.cpp: the library calls it before any launch, and
// the CPU sanitizer build (tests/sanitize/) compiles the same file with
// -fsanitize=address,undefined and drives it with the C-ABI test cases.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "gdn_amd.h"
#include "gdn_common.h"

namespace gdn {

// Records a printf-style message as the calling thread's last error and
// returns `code` so call sites can write `return fail(GDN_ERR_INVALID, ...)`.
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the calling thread's last error.
void clear_error();
// The calling thread's last error message ("" if none).
const char *last_error_text();

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
int make_heads(int hqk, int hv, const char *what, Heads &H);

// Arguments of a decode step over `batch` rows of `tokens` tokens each
// (gdn_decode_fwd: tokens = 1; gdn_decode_multi_fwd): pointers, scale,
// alignment (state/new_state 16 bytes, q/k 8, v/a/b/output 2) and every
// forbidden overlap (new_state may be exactly state).  GDN_OK or an error.
int check_decode_args(const gdn_bf16 *q, const gdn_bf16 *k, const gdn_bf16 *v, const float *state,
                      const float *A_log, const gdn_bf16 *a, const float *dt_bias,
                      const gdn_bf16 *b, float scale, const gdn_bf16 *output,
                      const float *new_state, int batch, int tokens, const Heads &H,
                      const char *what);

// Kernel for `tokens` tokens per row of a checked multi-token decode batch
// (gdn_decode_multi_fwd): *kernel = kDecodeStep the plain decode step (one
// token, the built-in choice), -1 the token-by-token kernel with its built-in
// tiling, 0 .. kNumRecTilings - 1 a token-by-token tiling, kNumRecTilings the
// 16-token block kernel.  `variant` -1 is the built-in
// choice (token by token or blocks by the cost models, at B = 64: 4 tokens
// 18.8 vs 19.5 us, 8 tokens 26.3 vs 19.9 us, 16 tokens 41.2 vs 20.6 us);
// the block kernel reads q, k and v rows with 16-byte loads, so it is never
// chosen for, and refuses, rows that are not 16-byte aligned.
constexpr int kDecodeStep = -2;
int plan_multi(const void *q, const void *k, const void *v, int batch, int tokens, const Heads &H,
               int variant, const char *what, int *kernel);

// Prefill workspace: every region starts on a 256-byte boundary.
struct PrefillLayout {
  int nt_max;  // upper bound on the chunk count from (T, N) alone
  // The T form keeps T in the w region and (beta, beta e^G) in the u region.
  // status: the contract bits of each sequence's cu_seqlens bounds (int per
  // sequence; bit 0 decreasing, bit 1 outside [0, T]), written by every call.
  size_t chunks, offsets, status, G, dcy, eg, w, u, kt, ht, vnt;
  // Two-segment scan of one sequence (N == 1 only, else empty): the map's
  // linear part per chunk of the second segment, the first segment's final
  // state and the second segment's map (offset, linear part).
  size_t htm, send, cend, mend;
  // Early output of the two-segment scan (N == 1): a progress word per first-
  // segment state unit, then a done flag per (chunk, v-head) of the segment.
  size_t early, total;
};

// Upper bound on the chunks of N sequences totalling T tokens: each sequence
// adds at most one partial chunk, and no chunk is empty.
long long max_chunks(long long T, long long N);
PrefillLayout prefill_layout(int T, int N, const Heads &H);

// Arguments of a prefill call: counts, pointers, scale, alignment, the tuning
// choices (variant -1..3, rec_max >= -2, rec_variant -1..num_rec_variants-1),
// the workspace (none needed for N == 0) and every forbidden overlap.  Fills
// *L with the workspace layout.  GDN_OK or an error.
int check_prefill_args(const gdn_bf16 *q, const gdn_bf16 *k, const gdn_bf16 *v, const float *state,
                       const float *A_log, const gdn_bf16 *a, const float *dt_bias,
                       const gdn_bf16 *b, const void *cu_seqlens, int cu64, int N, int T,
                       float scale, const gdn_bf16 *output, const float *new_state,
                       const void *workspace, size_t ws_bytes, int variant, int rec_max,
                       int rec_variant, int num_rec_variants, const Heads &H,
                       const char *what, PrefillLayout *L);

// Path choice between a sequential kernel and the chunk pipeline, from
// sweeps of all three paths on MI355X.  A batch of at most kRecurrentMaxLen
// tokens runs sequentially: token by token, or one sequence in blocks when
// the cost models favour them (one sequence of 64 tokens: 16.1 us in blocks,
// 20.1 us token by token, 20.7 us chunked).  Otherwise the sequential
// candidate is the block kernel (gdn_block.hip) or the token-by-token kernel,
// whichever the cost models rate faster at the mean length, and the device
// compares its cost model with the chunks' at the batch's longest sequence
// and chunk count (index kernel) -- unless the host already knows the chunks
// win: at N equal sequences of the mean length, the candidate's best case,
// it does not beat the chunks by more than a device-side choice costs
// (kDeviceChoiceCost).
constexpr int kRecurrentMaxLen = 96;

// Two-segment scan of one sequence (state kernel, SplitScan): three groups of
// 8 workgroups per v-head, one per CU, so it needs 24 H.v <= 256; the built-in
// choice takes it from kSplitMinChunks chunks on (MI355X, graph replay, one
// chain vs two segments: 28.3 vs 28.4 us at 8 chunks, 30.3 vs 29.5 at 9, 39.3
// vs 35.3 at 16, 53.3 vs 43.9 at 32, 64.5 vs 53.1 at 40).  Variants: 0 / -1
// built in, 2 never (one chain), 3 always (one sequence of at least two
// chunks).
constexpr int kSplitMinChunks = 9;

// Compute units of the target (MI355X: 256).  The WY intra kernel runs each
// (chunk, v-head) as two workgroups (its w and u halves) while that leaves
// at most kIntraSplitPerCu workgroups per CU: a batch too small to fill the
// CUs then halves its per-chunk latency instead of idling CUs.
constexpr int kNumCus = 256;
constexpr int kIntraSplitPerCu = 2;
// Workgroups the state kernel keeps resident per CU (its VGPRs): when the
// device makes the path choice, its grid is capped at this many per CU and
// it loops over the rest of its units (a multiple of 8, so a unit keeps its
// XCD), so that a batch handed to a sequential kernel does not dispatch a
// full grid (N x 64 workgroups) of idle ones.
constexpr int kStatePerCu = 2;

// What a prefill call launches, decided from (T, N), the head layout and the
// tuning arguments alone (cu_seqlens is never read on the host).
struct PrefillPlan {
  bool sequential;  // the whole batch through one sequential kernel, no chunk launch
  int seq_variant;  // that kernel: a recurrent_launch tiling, block_variant, or -1 built in
  int choose;       // 0: chunks; 1 / 2 / 3: the index kernel picks sequential or chunks
                    // (by rec_max / token vs chunk costs / block vs chunk costs)
  bool single;      // one sequence without a chunk table (bounds read on the device)
  int form;         // per-chunk operands: 0 WY, 1 T, -1 the index kernel's rule
  int split_nt0;    // two-segment scan: first chunk of the second segment; 0 none
  bool intra_split; // WY intra kernel as two workgroups per (chunk, v-head)
  bool loop;        // the state kernel loops over its units in a capped grid
                    // (when the device makes the path choice, choose != 0)
  bool self_index;  // no index launch: the intra kernel builds the chunk table
                    // (2..kSelfIndexMax sequences, an intra grid of 1..
                    // kSelfIndexMaxGrid workgroups), launched first
  // launch grids (workgroups, capped at the resident ones; the kernels loop
  // over the remaining units); 0 = not launched
  long long intra_grid, state_grid, split_grid, out_grid;
  // workgroups added to the state launch for the first segment's early output
  // (two-segment scan with 8 v-heads); 0 none
  long long early_grid;
  // chunks each early workgroup computes before it stops (0: no limit;
  // variant 4 stops them after one, so that the output launch computes the
  // rest of the segment through its fallback)
  int early_limit;
};

// rec_max >= 0 (explicit): sequential iff the longest sequence has at most
//                          rec_max tokens;
// rec_max == -2:           always chunks;
// rec_max == -1 (built in): token by token if T <= kRecurrentMaxLen; chunks
//                          for one longer sequence; else the cost models.
// block_variant: the rec_variant value that names the block kernel.
// GDN_OK, or GDN_ERR_INVALID if a grid exceeds a launch's limits.
int plan_prefill(int T, int N, const Heads &H, const PrefillLayout &L, int variant, int rec_max,
                 int rec_variant, int block_variant, const char *what, PrefillPlan &P);

}  // namespace gdn
