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
// Operand form of the chunks (WY or T) for a batch of nt chunks whose
// longest sequence has lc chunks, from graph-replay sweeps of both forms on
// MI355X (N = 1..64 equal sequences of 128..16384 tokens; 0.3 % above the
// faster form over the sweep): the T form from 192 chunks on when the batch
// holds more than three times the longest sequence's chunks, or from 384 on
// with at least twice (the WY form's workspace, ~1 MB per chunk, then no
// longer stays in the memory-side cache); else the WY form, and always for
// one sequence (nt == lc).
__host__ __device__ inline bool t_form_wins(float nt, float lc) {
  return nt >= 192.0f && (nt > 3.0f * lc || (nt >= 384.0f && nt >= 2.0f * lc));
}
// Chunks in one form (t: T, else WY) for N > 1 sequences, fitted to the same
// sweeps (rms 4-5 %): fixed launches, the intra and output kernels' work per
// chunk and v-head, and the state recurrence -- the longest sequence's chain
// of lc steps, or the batch's nt * hv * 8 unit-steps over the 512 resident
// state workgroups, whichever is longer; a step takes longer once some CU
// holds two state workgroups (more than 256 units of N * hv * 8).
__host__ __device__ inline float cost_by_chunks_form(float L, float nt, float hv, float N, bool t) {
  const float lc = ceilf(L / 64.0f), units = N * hv * 8.0f;
  const float steps = fmaxf(lc, nt * hv / 64.0f);
  if (t) return 10.6f + 0.039f * nt * hv + (units <= 256.0f ? 1.09f : 1.85f) * steps;
  return 24.6f + 0.033f * nt * hv + (units <= 256.0f ? 0.81f : 1.80f) * steps;
}
// Chunks in the form t_form_wins picks.
__host__ __device__ inline float cost_by_chunks(float L, float nt, float hv, float N) {
  return cost_by_chunks_form(L, nt, hv, N, t_form_wins(nt, ceilf(L / 64.0f)));
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

}  // namespace gdn
