// Definitions shared by the kernels and the host-side planning code.  This
// header includes no HIP header, so the host-side code (gdn_args.cpp) also
// builds with a plain host compiler -- the CPU sanitizer build does that,
// defining __host__ and __device__ empty on its command line.
#pragma once

#include <math.h>
#include <stddef.h>
#include <stdint.h>

namespace gdn {

constexpr int kHQK = 4;    // q/k heads of the reference definitions
constexpr int kHV = 8;     // their v heads; v-head h reads q/k head h / 2
constexpr int kDK = 128;   // key head size
constexpr int kDV = 128;   // value head size
constexpr int kChunk = 64; // prefill chunk length

// Head layout of a call: qk q/k heads, v v-heads, v a multiple of qk; v-head h
// reads q/k head h / ratio (GVA without copies).  Head size is always 128.
struct Heads {
  int qk, v, ratio;
};

// Path cost models in microseconds, fitted to graph-replay sweeps of each
// path on MI355X (sequence count N = 1..256 of equal lengths L = 8..16384,
// multi-token decode B = 1..128 with 4..16 tokens).  L = longest sequence,
// T = tokens, nt = chunks of 64, g = N * hv (sequence, v-head) groups.
// Token by token (recurrent kernel): the serial token chain plus VALU work
// per token and state traffic per group (refit after the kernel's state
// accesses went non-temporal and its tiling was re-swept: 86 shapes N =
// 1..256, L = 1..512, rms error 6 %, largest 21 % at 256 one-token sequences,
// where the state traffic binds).
__host__ __device__ inline float cost_by_token(float L, float T, float hv, float g) {
  return 3.56f + 0.216f * L + 0.00297f * T * hv + 0.0131f * g;
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
// Operand form of the chunks (WY or T) for a batch of nt chunks whose
// longest sequence has lc chunks and whose state recurrence has `units`
// (sequence, v-head, 16-column) workgroups, from graph-replay sweeps of both
// forms on MI355X (129 batches: N = 2..64 equal sequences of 64..16384
// tokens and ragged mixes; 0.25 % above the faster form on average, at most
// 7.8 %).  The T form (a quarter of the WY form's per-chunk workspace
// traffic, a longer serial step):
//  * for large batches -- from 144 chunks on when the batch holds more than
//    three times the longest sequence's chunks, or from 384 on with at least
//    1.5 times (the WY form's ~0.6 MB per chunk slot then no longer stays in
//    the memory-side cache);
//  * for small ones -- at most 768 units (three per CU) and chains of at
//    most 12 chunks, where the WY intra kernel's heavier outputs outweigh
//    T's longer steps (4 x 384 tokens: 35.8 vs 30.0 us, 8 x 192: 36.0 vs
//    30.4 us);
// else the WY form, and always for one sequence (nt == lc).  Both clauses
// only turn true as chunks grow or the longest sequence shrinks.
__host__ __device__ inline bool t_form_wins(float nt, float lc, float units) {
  const bool large = nt >= 144.0f && (nt > 3.0f * lc || (nt >= 384.0f && nt >= 1.5f * lc));
  const bool small = units <= 768.0f && lc <= 12.0f && nt > lc;
  return large || small;
}
// State units of the chunk recurrence: (sequence, v-head, 16-column V block).
__host__ __device__ inline float state_units(float N, float hv) { return N * hv * 8.0f; }
// Chunks in one form (t: T, else WY) for N > 1 sequences, fitted to the same
// sweeps where the sequential paths compete (at most 256 chunks; rms 8-9 %):
// fixed launches, the intra and output kernels' work per chunk and v-head,
// and the state recurrence -- the longest sequence's chain of lc steps, or
// the batch's nt * hv * 8 unit-steps over the 512 resident state workgroups,
// whichever is longer; a step takes longer once some CU holds two state
// workgroups (more than 256 units).
__host__ __device__ inline float cost_by_chunks_form(float L, float nt, float hv, float N, bool t) {
  const float lc = ceilf(L / 64.0f), units = state_units(N, hv);
  const float steps = fmaxf(lc, nt * hv / 64.0f);
  if (t) return 20.6f + 0.0457f * nt * hv + (units <= 256.0f ? 0.631f : 0.785f) * steps;
  return 19.8f + 0.0567f * nt * hv + (units <= 256.0f ? 0.373f : 0.454f) * steps;
}
// Chunks in the form t_form_wins picks.
__host__ __device__ inline float cost_by_chunks(float L, float nt, float hv, float N) {
  return cost_by_chunks_form(L, nt, hv, N,
                             t_form_wins(nt, ceilf(L / 64.0f), state_units(N, hv)));
}

// What a path choice made on the device costs (graph replay, MI355X): the
// index kernel and the chunk kernels returning at once when the sequential
// path wins (~9 us over the sequential kernel alone), the sequential kernel
// returning at once when the chunks win (~5 us).  The device prefers the
// sequential path only by more than the difference of the two; the host
// leaves the choice to the device only when the sequential path can win by
// more than the whole.
constexpr float kDeviceChoiceCost = 9.0f;
constexpr float kSeqChoiceMargin = 4.0f;

// Batches of at most kSelfIndexMax sequences whose intra launch is at most
// kSelfIndexMaxGrid workgroups (two rounds at five per CU) are indexed by
// the intra kernel itself (one sequence per thread of its 256), without the
// index launch (~4.7 us): each of its workgroups then scans cu_seqlens
// before its chunk, ~2 us per round of workgroups (8x2048, 2104 workgroups:
// 144.1 -> 139.5 us per call; 4x8192, 4128: intra 37.1 -> 44.9 us for 4.9 us
// of index kernel saved, so it keeps the index kernel).
constexpr int kSelfIndexMax = 256;
constexpr long long kSelfIndexMaxGrid = 2560;

// First chunk of the second segment of a two-segment scan over nt chunks.
__host__ __device__ inline int split_first(int nt) { return (nt + 1) / 2; }

// Workgroups of a per-(chunk, v-head) launch over nt chunk slots: the pairs
// (chunk, q/k head) rounded up to a multiple of the 8 XCDs, times the v-heads
// per q/k head (the mapping is chunk_head_of in gdn_prefill.hip).
__host__ __device__ inline long long chunk_head_grid(int nt, const Heads &H) {
  return (static_cast<long long>(nt) * H.qk + 7) / 8 * 8 * H.ratio;
}

// Row tilings of the token-by-token kernel (gdn_recurrent.hip); the
// sequential-kernel index kNumRecTilings names the 16-token block kernel.
constexpr int kNumRecTilings = 10;

// new_state tiles of a two-segment scan, per v-head (16 rows x 32 columns).
constexpr int kStateTiles = (kDV / 16) * (kDK / 32);

// Early output of a two-segment scan (8 v-heads: each head's 24 state
// workgroups on one XCD, 192 of the 256 CUs).  The state launch adds
// kEarlyGrid workgroups, kEarlyGrid / 8 per head on the head's XCD, that
// compute the first segment's output while its chain runs: chunk c as soon as
// the head's 8 first-segment units have stored its ht and v_new (they publish
// a progress word per unit, read through the XCD's L2).  The last kEarlyTail
// chunks of the segment, finished too close to the chain's end, are left to
// the output launch (kEarlyTail workgroups per head instead of one per
// chunk), which also computes any chunk not marked done.  Built in from
// 2 kEarlyTail first-segment chunks on (1x8192, graph replay: the state
// launch 53.1 -> 55.3 us, the output launch 29.4 -> 23.2 us; a tail of 7
// chunks left the early workgroups a backlog past the chain's end).
constexpr int kEarlyGrid = 64;
constexpr int kEarlyTail = 15;
__host__ __device__ inline long long early_words(int nt0, int hv) {
  return (static_cast<long long>(nt0) + kDV / 16) * hv;
}

}  // namespace gdn
