// Gated DeltaNet chunked prefill over a packed batch of variable-length
// sequences (chunk = 64 tokens, WY representation), gfx950.
//
// Semantics: reference/gdn_prefill_ref.py:12-91.  Per sequence, v-head h and
// chunk of C <= 64 tokens (g_i = -exp(A_log) softplus(a_i + dt_bias) is the
// log decay, G = chunk-local inclusive cumsum of g, beta_i = sigmoid(b_i),
// S = the [K=128, V=128] state at the chunk start):
//   A_ij  = beta_i exp(G_i - G_j) <k_i, k_j>  for i > j, else 0
//   T     = (I + A)^-1                       (unit lower triangular)
//   u     = T (beta * V),   w = T (beta exp(G) * K)
//   v_new = u - w S
//   o_i   = scale (exp(G_i) q_i S + sum_{j<=i} exp(G_i - G_j) <q_i, k_j> v_new_j)
//   S    <- exp(G_last) S + K^T (exp(G_last - G) * v_new)
// the same chunked algebra as the reference's inlined FLA pipeline
// (solutions/gdn_prefill_qk4_v8_d128_k_last/solution/triton/fla_kernels.py:
// 858-905, 197-314, 334-383, 411-671, 714-796), re-planned for CDNA4:
//
//   1. index  : one workgroup turns cu_seqlens (on the device, never copied
//               to the host) into the chunk table and per-sequence chunk
//               offsets, and picks the per-chunk form below (for a batch of
//               few sequences and intra workgroups the intra kernel does this
//               itself, 1b).  A zero-length sequence gets no chunk (the
//               reference's seq-id rule, fla_kernels.py:63, would misnumber
//               every later sequence).  It also records whether cu_seqlens
//               kept its contract (status words).
//   2. intra  : per (chunk, v-head): gating, cumsum, K K^T on MFMA, the
//               64x64 triangular inverse in LDS (and, in the WY form, its
//               products with K and V).  No GVA copies: v-head h reads q/k
//               head h/2 directly.
//   3. state  : per (sequence, v-head, 16 columns of V): the serial
//               recurrence over chunks with the f32 state in MFMA
//               accumulators; stores the chunk-start state and v_new.
//   4. output : per (chunk, v-head): o from Q S, the masked Q K^T and v_new
//               (after a two-segment scan of one sequence, 3b: with the
//               second segment's output in the same launch).
//
// Two forms of the state-independent per-chunk operands, chosen per batch:
//   WY form: the intra kernel forms w and u (and K^T fragments); a state step
//            is v_new = u - w S, then the update: two LDS exchanges.  The
//            shortest serial chain -- best when one sequence's chain bounds
//            the call (one sequence, or one much longer than the rest).
//   T form:  the intra kernel stores only T = (I + A)^-1; a state step forms
//            the right-hand side from the inputs, v_new = T (beta V - beta
//            e^G K S): a third exchange per step, but a quarter of the
//            intra kernel's HBM traffic and fewer bytes per step -- best
//            when many sequences keep every CU and the memory system busy.
// Rule (index kernel, t_form_wins in gdn_common.h, from sweeps of both on
// MI355X): the T form from 144 chunks on when the batch holds more than three
// times the chunks of its longest sequence, or from 384 on with at least 1.5
// times; and for small batches of at most 768 state units (sequence x v-head
// x 16-column block) whose longest sequence has at most 12 chunks.  One
// sequence always takes the WY form.
//
// Precision.  The state recurrence must hold 1e-3 of max|S| after 128-512
// chunks.  Rounding any operand of w S or K^T v_new (or u, w themselves) to
// one bf16 leaves ~2-4e-3 of max|S|, so those products use split bf16: an f32
// operand x is carried as hi + lo (both bf16, x = hi + lo to ~2^-17) and a
// product of two such operands as hi*hi + hi*lo + lo*hi (three MFMAs), or two
// when the other operand is exact in bf16 (K, V).  u, w, T and the state stay
// f32.  The output path (Q S, Q K^T, P v_new) uses single bf16 operands: its
// error stays ~2^-9 relative, far inside the bf16 output tolerance.
#include <mutex>
#include <vector>

#include "gdn_device.h"
#include "gdn_host.h"

namespace gdn {

// LDS row strides (elements), padded by 16 bytes against bank conflicts.
constexpr int kStrideK = 136;  // bf16 [64][128] tiles
constexpr int kStrideT = 72;   // bf16 [*][64]   tiles
// LDS of one chunk's output (Q, P, G): the output kernel's, and the state
// kernel's early-output workgroups'
constexpr int kOutputLds = kChunk * kStrideK * 2 + kChunk * kStrideT * 2 + kChunk * 4;

constexpr int kTElems = kChunk * kChunk * 2;  // T of one (chunk, head): hi + lo bf16

// ---------------------------------------------------------------------------
// 1. chunk table: chunks[c] = {sequence, first token, tokens (1..64), chunk
// number within the sequence} for c < NT, {-1, 0, 0, 0} up to nt_max;
// offsets[s] = first chunk of sequence s, offsets[N] = NT.  Token bounds are
// clamped to [0, T] and the chunk count to nt_max, so a malformed cu_seqlens
// cannot send any later kernel out of bounds.
//
// Form choice: offsets[N + 2] = form (0 WY, 1 T) -- `form` when it is 0 or 1,
// else the rule in the file header from the chunk count and the longest
// sequence.
//
// Path choice (choose != 0): one sequential kernel (token by token or in
// 16-token blocks) takes the whole batch when choose == 1 and no sequence is
// longer than rec_max tokens, or when its cost model (cost_by_token for
// choose == 2, cost_by_block for 3; gdn_host.h) is at most the chunks'
// (cost_by_chunks) at the batch's longest sequence and chunk count.  Then
// every sequence gets zero chunks and the path flag offsets[N + 1] is 1
// (else 0).
// ---------------------------------------------------------------------------
// Maximum of x over the workgroup into *dst (LDS, initially <= every x): a
// butterfly within each wave, then one LDS atomic per wave (1024 atomics on
// one word serialize: ~2 us).
__device__ __forceinline__ void block_max_into(int x, int *dst) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const int y = __shfl_xor(x, off);
    x = y > x ? y : x;
  }
  if ((threadIdx.x & 63) == 0) atomicMax(dst, x);
}
// Sum of x over the workgroup into *dst (LDS, initially 0), the same way.
__device__ __forceinline__ void block_sum_into(int x, int *dst) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off);
  if ((threadIdx.x & 63) == 0) atomicAdd(dst, x);
}

// The path the device picks (choose != 0, set on the host): sequential (true)
// or chunks, from the batch's longest sequence and chunk count (the form the
// chunks would take: `form` 0 / 1 as set, else t_form_wins).
__device__ __forceinline__ bool device_picks_sequential(int choose, int rec_max, int longest,
                                                        int chunks, int N, int T, int hv,
                                                        int form) {
  if (choose == 1) return longest <= rec_max;
  if (choose < 2) return false;
  const float L = static_cast<float>(longest), fhv = static_cast<float>(hv);
  const float g = static_cast<float>(N) * fhv;
  const float by_seq = choose == 2 ? cost_by_token(L, static_cast<float>(T), fhv, g)
                                   : cost_by_block(L, g);
  const float fnt = static_cast<float>(chunks);
  const bool t = form == 1 ||
                 (form != 0 && t_form_wins(fnt, ceilf(L / kChunk), state_units(static_cast<float>(N), fhv)));
  return by_seq + kSeqChoiceMargin <= cost_by_chunks_form(L, fnt, fhv, static_cast<float>(N), t);
}

__global__ __launch_bounds__(1024) void prefill_index_kernel(const void *cu, int cu64, int N, int T,
                                                              int nt_max, int choose, int rec_max,
                                                              int hv, int form, int4 *chunks,
                                                              int *offsets, int *status) {
  __shared__ int s_incl[1024], s_bos[1024], s_eos[1024];
  __shared__ int s_wsum[16];
  __shared__ int s_longest, s_most_chunks, s_chunks;
  const int tid = threadIdx.x;
  if (tid == 0) s_longest = s_most_chunks = s_chunks = 0;
  __syncthreads();
  // Sequence s's bounds as given, their contract bits into status[s] (in the
  // first pass that reads them), and clamped into [0, T].
  auto bounds = [&](int s, bool write_status, int &bos, int &eos) {
    const long long lo = raw_cu(cu, cu64, s), hi = raw_cu(cu, cu64, s + 1);
    if (write_status) status[s] = cu_status_bits(lo, hi, T);
    bos = static_cast<int>(lo < 0 ? 0 : lo > T ? T : lo);
    eos = static_cast<int>(hi < 0 ? 0 : hi > T ? T : hi);
    eos = eos < bos ? bos : eos;
  };
  if (choose != 0) {
    int longest = 0, nch = 0;
    for (int s = tid; s < N; s += 1024) {
      int bos, eos;
      bounds(s, true, bos, eos);
      const int len = eos - bos;
      longest = len > longest ? len : longest;
      nch += (len + kChunk - 1) / kChunk;
    }
    block_max_into(longest, &s_longest);
    block_sum_into(nch, &s_chunks);
  }
  __syncthreads();
  const bool sequential =
      device_picks_sequential(choose, rec_max, s_longest, s_chunks, N, T, hv, form);
  if (tid == 0) offsets[N + 1] = sequential ? 1 : 0;
  long long carry = 0;
  int most_chunks = 0;
  for (int base = 0; base < N; base += 1024) {
    const int s = base + tid;
    int n = 0;
    if (s < N && !sequential) {
      int bos, eos;
      bounds(s, choose == 0, bos, eos);
      n = (eos - bos + kChunk - 1) / kChunk;
      s_bos[tid] = bos;
      s_eos[tid] = eos;
    }
    most_chunks = n > most_chunks ? n : most_chunks;
    // inclusive scan of n over the tile: within each wave by lane shifts,
    // then the totals of the earlier waves
    int incl = n;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(incl, off);
      if ((tid & 63) >= off) incl += y;
    }
    if ((tid & 63) == 63) s_wsum[tid >> 6] = incl;
    __syncthreads();
    for (int w = 0; w < (tid >> 6); ++w) incl += s_wsum[w];
    s_incl[tid] = incl;
    __syncthreads();
    const int tile_total = s_incl[1023];
    if (s < N) {
      const long long first = carry + s_incl[tid] - n;
      offsets[s] = static_cast<int>(first < nt_max ? first : nt_max);
    }
    const int count = N - base < 1024 ? N - base : 1024;
    const long long end = carry + tile_total < nt_max ? carry + tile_total : nt_max;
    for (long long c = carry + tid; c < end; c += 1024) {
      const int r = static_cast<int>(c - carry);
      int lo = 0, hi = count - 1;  // first idx with s_incl[idx] > r
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (s_incl[mid] > r) hi = mid; else lo = mid + 1;
      }
      const int excl = lo == 0 ? 0 : s_incl[lo - 1];
      const int sq = base + lo, local = r - excl;
      const int eos = s_eos[lo];
      const int start = s_bos[lo] + local * kChunk;
      const int len = eos - start < kChunk ? eos - start : kChunk;
      chunks[c] = make_int4(sq, start, len, local);
    }
    carry += tile_total;
    __syncthreads();
  }
  block_max_into(most_chunks, &s_most_chunks);
  __syncthreads();
  const int nt = static_cast<int>(carry < nt_max ? carry : nt_max);
  if (tid == 0) {
    offsets[N] = nt;
    offsets[N + 2] = (form == 0 || form == 1)
                         ? form
                         : (t_form_wins(static_cast<float>(nt), static_cast<float>(s_most_chunks),
                                        state_units(static_cast<float>(N), static_cast<float>(hv)))
                                ? 1
                                : 0);
  }
  for (int c = nt + tid; c < nt_max; c += 1024) chunks[c] = make_int4(-1, 0, 0, 0);
}

// Chunk c of the table; for a single sequence (one.cu != nullptr) there is no
// table and the entry is computed from the sequence's bounds.
__device__ __forceinline__ int4 chunk_info(const int4 *chunks, int c, const OneSeq &one) {
  if (one.cu != nullptr) {
    int bos, eos;
    one_seq_bounds(one, bos, eos);
    const int start = bos + c * kChunk, rest = eos - start;
    return rest > 0 ? make_int4(0, start, rest < kChunk ? rest : kChunk, c) : make_int4(-1, 0, 0, 0);
  }
  // the same entry in every lane: keep it in SGPRs (buffer descriptors built
  // from it are then uniform, with no per-lane loop around each load)
  const int4 e = chunks[c];
  return make_int4(__builtin_amdgcn_readfirstlane(e.x), __builtin_amdgcn_readfirstlane(e.y),
                   __builtin_amdgcn_readfirstlane(e.z), __builtin_amdgcn_readfirstlane(e.w));
}

// ---------------------------------------------------------------------------
// 1b. the chunk table built inside the intra kernel (several sequences, at
// most kSelfIndexMax, and an intra grid of at most kSelfIndexMaxGrid
// workgroups; gdn_common.h): each workgroup scans cu_seqlens itself -- one
// sequence per thread, a prefix sum of the chunk counts in LDS -- and finds
// its own chunk by binary search; workgroup 0 writes offsets, the chunk
// count and the flags, and the workgroup of v-head 0 of each chunk slot its
// chunk-table entry, for the state and output kernels.  A batch then needs no
// index launch (~4.7 us): the intra kernel is the first launch, the path the
// device picks included (the sequential kernel runs after it and reads the
// flag).  Same results as the index kernel, entry by entry.
// ---------------------------------------------------------------------------
struct SelfIndex {
  const void *cu;  // nullptr: the index kernel built the table
  int cu64, N, T, choose, rec_max, form;
  int4 *chunks;
  int *offsets;
  int *status;     // per-sequence contract bits (also for one sequence)
  int *early;      // one sequence: words of the two-segment scan's early output,
  int n_early;     // zeroed by the first workgroups (nullptr: none)
};
constexpr int kSelfIndexLds = 3 * kSelfIndexMax * 4 + 16 * 4;

struct SelfIndexed {
  int nt, form;
};

__device__ __forceinline__ SelfIndexed self_index(char *smem, const SelfIndex &si, int nt_max,
                                                  int hv) {
  int *const s_incl = reinterpret_cast<int *>(smem);
  int *const s_bos = s_incl + kSelfIndexMax;
  int *const s_eos = s_bos + kSelfIndexMax;
  int *const s_red = s_eos + kSelfIndexMax;  // longest, most chunks, wave totals [4..7]
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int N = si.N, T = si.T;
  int n = 0, len = 0;
  if (tid < 2) s_red[tid] = 0;
  if (tid < N) {
    const long long lo = raw_cu(si.cu, si.cu64, tid), hi = raw_cu(si.cu, si.cu64, tid + 1);
    if (blockIdx.x == 0) si.status[tid] = cu_status_bits(lo, hi, T);
    const int bos = static_cast<int>(lo < 0 ? 0 : lo > T ? T : lo);
    int eos = static_cast<int>(hi < 0 ? 0 : hi > T ? T : hi);
    eos = eos < bos ? bos : eos;
    len = eos - bos;
    n = (len + kChunk - 1) / kChunk;
    s_bos[tid] = bos;
    s_eos[tid] = eos;
  }
  int incl = n;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(incl, off);
    if (lane >= off) incl += y;
  }
  if (lane == 63) s_red[4 + wv] = incl;
  __syncthreads();
  for (int w = 0; w < wv; ++w) incl += s_red[4 + w];
  s_incl[tid] = incl;
  block_max_into(len, &s_red[0]);
  block_max_into(n, &s_red[1]);
  __syncthreads();
  const int total = s_incl[N - 1];
  const bool sequential = device_picks_sequential(si.choose, si.rec_max, s_red[0], total, N, T,
                                                  hv, si.form);
  const int nt = sequential ? 0 : (total < nt_max ? total : nt_max);
  const int form = (si.form == 0 || si.form == 1)
                       ? si.form
                       : (t_form_wins(static_cast<float>(nt), static_cast<float>(s_red[1]),
                                      state_units(static_cast<float>(N), static_cast<float>(hv)))
                              ? 1
                              : 0);
  if (blockIdx.x == 0) {
    if (tid < N) {
      const int first = sequential ? 0 : s_incl[tid] - n;
      si.offsets[tid] = first < nt_max ? first : nt_max;
    }
    if (tid == 0) {
      si.offsets[N] = nt;
      si.offsets[N + 1] = sequential ? 1 : 0;
      si.offsets[N + 2] = form;
    }
  }
  return SelfIndexed{nt, form};
}

// Entry c of the chunk table from the self index's LDS arrays.
__device__ __forceinline__ int4 self_chunk(const char *smem, int N, int c, int nt) {
  if (c >= nt) return make_int4(-1, 0, 0, 0);
  const int *const s_incl = reinterpret_cast<const int *>(smem);
  const int *const s_bos = s_incl + kSelfIndexMax;
  const int *const s_eos = s_bos + kSelfIndexMax;
  int lo = 0, hi = N - 1;  // first sequence with s_incl > c
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (s_incl[mid] > c) hi = mid; else lo = mid + 1;
  }
  const int local = c - (lo == 0 ? 0 : s_incl[lo - 1]);
  const int start = s_bos[lo] + local * kChunk;
  const int len = s_eos[lo] - start < kChunk ? s_eos[lo] - start : kChunk;
  return make_int4(lo, start, len, local);
}

// Workgroup id -> (chunk c, v-head h) for the per-(chunk, head) kernels, so
// that the `ratio` v-heads reading one q/k head of one chunk are dispatched
// back to back on the same XCD: ids are dealt round-robin over the 8 XCDs,
// so id = 8 s + x runs on XCD x, and consecutive s on one XCD take the
// v-heads of one (chunk, q/k head) pair -- the second and later ones find
// that chunk's q/k rows in the XCD's L2.  Pairs are numbered P = 8 p + x in
// chunk-major order.  False for ids past the last pair.
__device__ __forceinline__ bool chunk_head_of(int id, int nt, const Heads &H, int &c, int &h) {
  const int x = id & 7, sl = id >> 3;
  const int p = sl / H.ratio, r = sl - p * H.ratio;
  const long long P = 8LL * p + x;
  if (P >= static_cast<long long>(nt) * H.qk) return false;
  c = static_cast<int>(P / H.qk);
  h = static_cast<int>(P - static_cast<long long>(c) * H.qk) * H.ratio + r;
  return true;
}

// WY form of the intra kernel, per chunk c and v-head h (30 KB of LDS):
//   * wave 0: gating, chunk-local cumsum G, decay factors.
//   * K rows -> LDS row-major (V rows wait in registers).
//   * A = strictly-lower(beta_i exp(G_i - G_j) K K^T) on MFMA, stored as its
//     ten lower 16x16 blocks; K^T fragments for the state kernel.
//   * the four diagonal blocks of (I + A) inverted by forward substitution
//     (wave w, block w), in place of the diagonal blocks of A.
//   * w = (I + A)^-1 (beta exp(G) K) and then u = (I + A)^-1 (beta V) by
//     blocked forward substitution: wave w owns 32 right-hand-side columns
//     and walks the four 16-row block rows,
//       Y_i = D_i (X_i - sum_{j<i} A_ij Y_j),
//     on split-bf16 MFMAs with every Y_j kept in registers; the X_i operands
//     (4 consecutive tokens of one feature) come straight from the row-major
//     tile through gfx950's transposing LDS read, so no transposed copy of K
//     or V is kept.  w is turned into A-operand fragments through the K
//     tile's space once the w-solve is done; V then takes that space.
// PART: 0 = w then u in one workgroup; 1 = w only; 2 = u only (a chunk's two
// halves in two workgroups, for batches too small to fill the CUs).
// Outputs go to the workspace in the exact fragment order the state kernel
// reads: u as MFMA result tiles, w as hi/lo A-operand fragments, K^T as
// A-operand fragments.
constexpr int kABlk = 16 * 20;  // one 16x16 f32 block of A, rows padded to 20
// The w region of one (chunk, head) in the WY form (32 KB): the bf16 hi
// plane (16 KB), the fp8 lo plane (8 KB), then lo's inverse scale (a float).
constexpr uint32_t kWLoOff = kChunk * kDK * 2;
constexpr uint32_t kWScaleOff = kWLoOff + kChunk * kDK;
constexpr int kIntraWyLds = kChunk * kStrideK * 2 + 10 * kABlk * 4 + 3 * kChunk * 4 + 16;
// Block (ib, jb), jb <= ib, of the compact lower-triangular A.
__device__ __forceinline__ int ablk(int ib, int jb) { return (ib * (ib + 1) / 2 + jb) * kABlk; }

// The B operand of a 16x16x16 product contracting over tokens: rows
// r0..r0+3 (tokens) of column c0 + (lane & 15) of a row-major bf16 tile,
// gathered by one transposing read (16-lane group g passes its own r0, c0).
__device__ __forceinline__ u32x2 tile_col4(const uint16_t *tile, int r0, int c0, int r16) {
  return ds_read_tr16(&tile[(r0 + (r16 >> 2)) * kStrideK + c0 + 4 * (r16 & 3)]);
}

// A = strictly-lower(beta_i exp(G_i - G_j) K K^T) of one chunk from its K
// rows in LDS (row-major, stride kStrideK), as the ten lower 16x16 blocks of
// sA (ablk; rows padded to 20 floats).  Wave w computes blocks w, w + 4 and
// (waves 0, 1) w + 8, the three as independent MFMA chains side by side (one
// block at a time left each wave waiting on its LDS reads and a 4-deep MFMA
// chain per block).  G_i - G_j <= 0 for every kept entry (g <= 0); the clamp
// keeps the others finite; exp is the hardware exp2 of x log2(e) (a few
// 2^-24 relative, far below the split-bf16 products' 2^-17).
__device__ __forceinline__ void build_A(const uint16_t *sK, float *sA, const float *sG,
                                        const float *sBeta, int len, int wave, int lane) {
  const int r16 = lane & 15, g = lane >> 4, kg = 8 * g;
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  int mb[3], nb[3];
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    int t = wv + 4 * q;
    t = t < 10 ? t : 9;  // waves 2, 3 repeat block 9 as their third (not stored)
    // t = 0..9 -> (mb, nb) = (3,3) (3,2) (3,1) (3,0) (2,2) (2,1) (2,0) (1,1) (1,0) (0,0)
    mb[q] = t < 4 ? 3 : t < 7 ? 2 : t < 9 ? 1 : 0;
    nb[q] = t < 4 ? 3 - t : t < 7 ? 6 - t : t < 9 ? 8 - t : 0;
  }
  f32x4 acc[3];
#pragma unroll
  for (int q = 0; q < 3; ++q) acc[q] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kk = 0; kk < 4; ++kk)
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      const u32x4 af = *reinterpret_cast<const u32x4 *>(&sK[(16 * mb[q] + r16) * kStrideK + 32 * kk + kg]);
      const u32x4 bf = *reinterpret_cast<const u32x4 *>(&sK[(16 * nb[q] + r16) * kStrideK + 32 * kk + kg]);
      acc[q] = mfma_bf16(af, bf, acc[q]);
    }
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    if (q == 2 && wv >= 2) break;
    const float Gj = sG[16 * nb[q] + r16];
    const f32x4 Gi = *reinterpret_cast<const f32x4 *>(&sG[16 * mb[q] + 4 * g]);
    const f32x4 Bi = *reinterpret_cast<const f32x4 *>(&sBeta[16 * mb[q] + 4 * g]);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = 16 * mb[q] + 4 * g + r, j = 16 * nb[q] + r16;
      const float d = __builtin_amdgcn_exp2f(fminf(Gi[r] - Gj, 0.f) * 1.44269504088896341f);
      const float e = Bi[r] * d * acc[q][r];
      sA[ablk(mb[q], nb[q]) + (4 * g + r) * 20 + r16] = (i > j && i < len) ? e : 0.f;
    }
  }
}

// Diagonal blocks D_w = (I + A_ww)^-1 in place of A_ww: wave w, lane j < 16
// solves column j, column-oriented (each solved x_m is applied to all later
// rows at once, so the serial chain is one FMA per row).  Every read of A_ww
// precedes the writes in the wave's program order.
__device__ __forceinline__ void diag_inverse(float *sA, int wave, int lane) {
  if (lane < 16) {
    float *Aw = sA + ablk(wave, wave);
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = i == lane ? 1.f : 0.f;
#pragma unroll
    for (int m = 0; m < 15; ++m) {
      const float xm = x[m];
#pragma unroll
      for (int i = m + 1; i < 16; ++i) x[i] -= Aw[i * 20 + m] * xm;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) Aw[i * 20 + lane] = x[i];
  }
}

// Blocked forward substitution (I + A) Y = diag(scl) X for the 32 columns
// col0.. of this wave; X row-major in sX ([64][kStrideK] bf16), A in sA with
// the diagonal inverses D_i in place of A_ii.  16x16x16 MFMAs (a result
// tile's layout is the next product's B-operand layout), each row block
// waiting on the ones above it.
__device__ __forceinline__ void wy_solve(const uint16_t *sX, const float *scl, const float *sA,
                                         int col0, int g, int r16, f32x4 (&Y)[4][2]) {
  u32x2 Yh[4][2], Yl[4][2];  // hi/lo splits of Y (B operands)
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    // Z = X_i - sum_{j<i} A_ij Y_j
    const f32x4 s4 = *reinterpret_cast<const f32x4 *>(&scl[16 * i + 4 * g]);
    f32x4 Z[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const u32x2 x2 = tile_col4(sX, 16 * i + 4 * g, col0 + 16 * nt, r16);
      Z[nt] = f32x4{s4[0] * __uint_as_float(x2[0] << 16),
                    s4[1] * __uint_as_float(x2[0] & 0xffff0000u),
                    s4[2] * __uint_as_float(x2[1] << 16),
                    s4[3] * __uint_as_float(x2[1] & 0xffff0000u)};
    }
#pragma unroll
    for (int j = 0; j < i; ++j) {
      const f32x4 la = *reinterpret_cast<const f32x4 *>(&sA[ablk(i, j) + r16 * 20 + 4 * g]);
      u32x2 lh, ll;
      split4(-la, lh, ll);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) Z[nt] = mfma16_x3(lh, ll, Yh[j][nt], Yl[j][nt], Z[nt]);
    }
    // Y_i = D_i Z
    const f32x4 d4 = *reinterpret_cast<const f32x4 *>(&sA[ablk(i, i) + r16 * 20 + 4 * g]);
    u32x2 dh, dl;
    split4(d4, dh, dl);
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      u32x2 zh, zl;
      split4(Z[nt], zh, zl);
      Y[i][nt] = mfma16_x3(dh, dl, zh, zl, f32x4{0.f, 0.f, 0.f, 0.f});
      split4(Y[i][nt], Yh[i][nt], Yl[i][nt]);
    }
  }
}

// Block column j = wave of T = (I + A)^-1 from the ten lower blocks of sA
// (A, with the diagonal inverses D_i in place of A_ii): T_jj = D_j and, for
// i > j, T_ij = -D_i sum_{j<=m<i} A_im T_mj, on split-bf16 16x16x16 MFMAs (a
// result tile's layout is the next product's B-operand layout, so the column
// stays in registers).  Tc[i] = T_ij in MFMA result order (lane holds rows
// 4g..4g+3, column r16); zero above the diagonal.
__device__ __forceinline__ void t_column(const float *sA, int wave, int g, int r16,
                                         f32x4 (&Tc)[4]) {
  const int j = wave;
  u32x2 Th[4], Tl[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (i < j) {  // above the diagonal
      Tc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
      Th[i] = Tl[i] = u32x2{0u, 0u};
    } else if (i == j) {  // T_jj = D_j
      const float *d = &sA[ablk(i, i) + (4 * g) * 20 + r16];
      Tc[i] = f32x4{d[0], d[20], d[40], d[60]};
      split4(Tc[i], Th[i], Tl[i]);
    } else {
      // Z = -sum_{j<=m<i} A_im T_mj, then T_ij = D_i Z
      f32x4 Z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int m = 0; m < i; ++m) {
        if (m < j) continue;
        const f32x4 la = *reinterpret_cast<const f32x4 *>(&sA[ablk(i, m) + r16 * 20 + 4 * g]);
        u32x2 lh, ll;
        split4(-la, lh, ll);
        Z = mfma16_x3(lh, ll, Th[m], Tl[m], Z);
      }
      const f32x4 d4 = *reinterpret_cast<const f32x4 *>(&sA[ablk(i, i) + r16 * 20 + 4 * g]);
      u32x2 dh, dl, zh, zl;
      split4(d4, dh, dl);
      split4(Z, zh, zl);
      Tc[i] = mfma16_x3(dh, dl, zh, zl, f32x4{0.f, 0.f, 0.f, 0.f});
      split4(Tc[i], Th[i], Tl[i]);
    }
  }
}

// Y = T diag(scl) X for the 32 columns col0.. of this wave: X row-major in
// sX ([64][kStrideK] bf16, exact), T = (I + A)^-1 in the ten lower blocks of
// sA (f32, rows of 20), scl per token.  T diag(scl) is split into bf16 hi and
// lo A operands of 16x16x32 MFMAs (two products per k-step, X exact); the
// k-steps of T's zero blocks above the diagonal are skipped, a half-zero one
// reads zeros.  Result tiles Y[i][nt]: rows 16 i + 4 g .., column col0 +
// 16 nt + r16.
__device__ __forceinline__ void wy_gemm(const uint16_t *sX, const float *scl, const float *sA,
                                        int col0, int g, int r16, f32x4 (&Y)[4][2]) {
  const int kg = 8 * g;
  u32x4 xb[2][2];  // X: k-step kk (tokens 32 kk + 8 g ..), column tile nt
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const u32x2 y = tile_col4(sX, 32 * kk + kg + 4 * hh, col0 + 16 * nt, r16);
        xb[kk][nt][2 * hh] = y[0];
        xb[kk][nt][2 * hh + 1] = y[1];
      }
  f32x4 s0[2], s1[2];  // scl of the lane's 8 tokens per k-step
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    s0[kk] = *reinterpret_cast<const f32x4 *>(&scl[32 * kk + kg]);
    s1[kk] = *reinterpret_cast<const f32x4 *>(&scl[32 * kk + kg + 4]);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) Y[i][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      if (kk == 1 && i < 2) continue;  // block columns 2, 3 of row tiles 0, 1: zero
      // T[16 i + r16][32 kk + 8 g ..]: block (i, jb), columns 8 (g & 1) ..
      const int jb = 2 * kk + (g >> 1);
      const bool live = jb <= i;
      const float *row = &sA[ablk(i, live ? jb : i) + r16 * 20 + 8 * (g & 1)];
      const f32x4 t0 = *reinterpret_cast<const f32x4 *>(row);
      const f32x4 t1 = *reinterpret_cast<const f32x4 *>(row + 4);
      float x8[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x8[e] = live ? t0[e] * s0[kk][e] : 0.f;
        x8[4 + e] = live ? t1[e] * s1[kk][e] : 0.f;
      }
      u32x4 ah, al;
      split8(x8, ah, al);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        Y[i][nt] = mfma_bf16(ah, xb[kk][nt], Y[i][nt]);
        Y[i][nt] = mfma_bf16(al, xb[kk][nt], Y[i][nt]);
      }
    }
  }
}

// T of the chunk over A in sA (every wave calls it; LDS barriers inside):
// each wave's block column by t_column, then, once no wave reads A any
// more, written over the ten lower blocks of sA.
__device__ __forceinline__ void t_into_sA(float *sA, int wave, int g, int r16) {
  f32x4 Tc[4];
  t_column(sA, wave, g, r16, Tc);
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (i < wave) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) sA[ablk(i, wave) + (4 * g + r) * 20 + r16] = Tc[i][r];
  }
  __syncthreads();
}

// Batches of at least this many (chunk, v-head) units (three per CU of the
// 256) form w and u as T and two products (wy_gemm) instead of two solves.
constexpr int kIntraGemmMinUnits = 3 * 256;

template <int PART>
__device__ __forceinline__ void wy_intra(
    char *smem, int c, int h, int start, int len, const uint16_t *__restrict__ k,
    const uint16_t *__restrict__ v, const float *__restrict__ A_log, const uint16_t *__restrict__ a,
    const float *__restrict__ dt_bias, const uint16_t *__restrict__ b, const Heads &H,
    float *__restrict__ ws_G, float *__restrict__ ws_dcy, float *__restrict__ ws_eg,
    uint16_t *__restrict__ ws_w, float *__restrict__ ws_u, uint16_t *__restrict__ ws_kt,
    bool gemm) {
  constexpr bool kW = PART != 2, kU = PART != 1;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g = lane >> 4, kg = g * 8;
  const int hq = h / H.ratio;
  const size_t ch_head = static_cast<size_t>(c) * H.v + h;

  //   sX:  K row-major; after the w-solve f32 scratch for w's fragments; then
  //        V row-major for the u-solve.
  //   sA:  the ten lower 16x16 blocks of A; the diagonal ones become D_w.
  uint16_t *const sX = reinterpret_cast<uint16_t *>(smem);                   // [64][136]
  float *const sA = reinterpret_cast<float *>(sX + kChunk * kStrideK);        // 10 blocks
  float *const sBeta = sA + 10 * kABlk, *const sBG = sBeta + kChunk, *const sG = sBG + kChunk;
  float *const sWmax = sG + kChunk;                                           // max |w| per wave
  float *const scr = reinterpret_cast<float *>(sX);                           // [64][68]
  constexpr int kStrideS = 68;
  static_assert(kChunk * kStrideS * 4 <= kChunk * kStrideK * 2, "w scratch must fit the tile");

  // K rows -> LDS, then V rows into registers (rows past the chunk read
  // zero through the descriptors' range).  Thread t moves 16 bytes of rows
  // (t + 256 i) / 16.  The K loads go first, the gating of wave 0 runs while
  // they are in flight; V is loaded only once K is in LDS: every workgroup of
  // a launch loads at once, and K alone arrives sooner (V is first needed
  // after the w-solve, or after A for the u-only half).
  u32x4 vrows[4];
  {
    const uint32_t kstride = static_cast<uint32_t>(H.qk) * (kDK * 2);
    const auto rk = buf_rsrc(k + (static_cast<size_t>(start) * H.qk + hq) * kDK,
                             static_cast<uint32_t>(len) * kstride);
    u32x4 krows[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = tid + 256 * i;
      krows[i] = buf_load16(rk, static_cast<uint32_t>(idx >> 4) * kstride + (idx & 15) * 16);
    }
    // Gating and the chunk-local cumsum (wave 0, lane = token).  Padding
    // tokens get g = 0 and beta = 0, so G stays at G_last past the end of the
    // chunk.
    if (wave == 0) {
      float gl, be;
      chunk_gates(lane, start, len, h, H, A_log, a, dt_bias, b, gl, be);
      float G = gl;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float y = __shfl_up(G, off);
        if (lane >= off) G += y;
      }
      sG[lane] = G;
      sBeta[lane] = be;
      sBG[lane] = be * expf(G);
      if (kW) {  // (the u-only half leaves these to the w half)
        const float G_last = __shfl(G, 63);
        ws_G[ch_head * kChunk + lane] = G;
        ws_dcy[ch_head * kChunk + lane] = expf(G_last - G);
        if (lane == 0) ws_eg[ch_head] = expf(G_last);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = tid + 256 * i;
      *reinterpret_cast<u32x4 *>(&sX[(idx >> 4) * kStrideK + (idx & 15) * 8]) = krows[i];
    }
  }
  __syncthreads();
  if (kU) {
    const uint32_t vstride = static_cast<uint32_t>(H.v) * (kDV * 2);
    const auto rv = buf_rsrc(v + (static_cast<size_t>(start) * H.v + h) * kDV,
                             static_cast<uint32_t>(len) * vstride);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = tid + 256 * i;
      vrows[i] = buf_load16(rv, static_cast<uint32_t>(idx >> 4) * vstride + (idx & 15) * 16);
    }
  }

  build_A(sX, sA, sG, sBeta, len, wave, lane);
  // K^T as A-operand fragments of the state kernel (one v-head per q/k head
  // writes them): fragment (mt, kk), lane (g, r16) = the 8 tokens 32 kk +
  // 8 g .. of feature 16 mt + r16; wave w writes fragments 4 w .. 4 w + 3.
  if (kW && h % H.ratio == 0) {
    uint16_t *ktf = ws_kt + (static_cast<size_t>(c) * H.qk + hq) * (kDK * kChunk);
    const auto rkt = buf_rsrc(ktf, kDK * kChunk * 2);
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      const int fi = 4 * wave + f, mt = fi >> 1, kk = fi & 1;
      u32x4 x;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const u32x2 y = tile_col4(sX, 32 * kk + kg + 4 * hh, 16 * mt, r16);
        x[2 * hh] = y[0];
        x[2 * hh + 1] = y[1];
      }
      buf_store16_sc1(rkt, static_cast<uint32_t>(fi * 64 + lane) * 16u, x);
    }
  }
  __syncthreads();

  // Diagonal blocks D_w = (I + A_ww)^-1 in place of A_ww (diag_inverse).
  if (kU && !kW) {
    // the u-only half: K is dead once A is built, V takes its place
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = tid + 256 * i;
      *reinterpret_cast<u32x4 *>(&sX[(idx >> 4) * kStrideK + (idx & 15) * 8]) = vrows[i];
    }
  }
  diag_inverse(sA, wave, lane);
  __syncthreads();
  // w = T diag(beta e^G) K and u = T diag(beta) V: with `gemm`, T =
  // (I + A)^-1 first (over A) and two products (wy_gemm); else two blocked
  // forward substitutions (wy_solve).  T's serial column walk costs ~1.9 us
  // at 1x8192, and the products (16x16x32, no chain between row blocks) save
  // more once several workgroups share each CU (intra 21.7 -> 20.8 us at
  // 1x8192, 23.1 -> 21.9 us at 2x4096, 15.4 us either way at 1x4096 with two
  // per CU); with fewer, and for the split halves (one solve each), the
  // solves are faster (1x1024 11.7 vs 12.5 us, configs[3] 19.2 vs 20.0 us).
  // The choice depends on the batch's chunk count alone (not on the launch
  // grid, an upper bound), so a batch gets the same bits whichever way it
  // was indexed and whether its form was set or picked on the device.
  if (gemm) t_into_sA(sA, wave, g, r16);
  auto solve = [&](const float *scl, f32x4 (&Y)[4][2]) {
    if (gemm)
      wy_gemm(sX, scl, sA, 32 * wave, g, r16, Y);
    else
      wy_solve(sX, scl, sA, 32 * wave, g, r16, Y);
  };
  const int col0 = 32 * wave;
  if (kW) {
    f32x4 Y[4][2];
    solve(sBG, Y);
    {
      float m = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
          for (int r = 0; r < 4; ++r) m = fmaxf(m, fabsf(Y[i][nt][r]));
      m = wave_max(m);
      if (lane == 0) sWmax[wave] = m;
    }
    __syncthreads();  // K is dead: its space is the w scratch
    // w -> A-operand fragments (row 16 mb + r16, features 32 kk + 8 g ..):
    // hi = w rounded to bf16, [mb][kk][lane][8] (this plane alone serves the
    // second-segment output); lo = (w - hi) 2^s as OCP fp8, [mb][kk / 2]
    // [lane][kk % 2][8] at byte kWLoOff, 2^-s (one float) at kWScaleOff.  In
    // two passes of 64 features through the f32 scratch: waves 2p, 2p + 1
    // fill it, then wave w converts fragments (w, 2p) and (w, 2p + 1) and
    // stores their low parts as one 16-byte row.
    uint16_t *wf = ws_w + ch_head * (kChunk * kDK * 2);
    const auto rwf = buf_rsrc(wf, kChunk * kDK * 4);
    float lo_inv;
    const float lo_sc = fp8_lo_scale(fmaxf(fmaxf(sWmax[0], sWmax[1]), fmaxf(sWmax[2], sWmax[3])),
                                     &lo_inv);
    if (tid == 0) *reinterpret_cast<float *>(reinterpret_cast<char *>(wf) + kWScaleOff) = lo_inv;
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
      if ((wave >> 1) == pass) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              scr[(16 * i + 4 * g + r) * kStrideS + (col0 & 63) + 16 * nt + r16] = Y[i][nt][r];
      }
      __syncthreads();
      u32x4 lo8;
#pragma unroll
      for (int kk2 = 0; kk2 < 2; ++kk2) {
        const float *row = &scr[(16 * wave + r16) * kStrideS + 32 * kk2 + kg];
        const f32x4 x0 = *reinterpret_cast<const f32x4 *>(row);
        const f32x4 x1 = *reinterpret_cast<const f32x4 *>(row + 4);
        const float x8[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
        const u32x4 hi = pack8(x8);
        float hf[8];
        unpack8(hi, hf);
        float lo[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) lo[e] = (x8[e] - hf[e]) * lo_sc;
        lo8[2 * kk2] = pk4_fp8(lo[0], lo[1], lo[2], lo[3]);
        lo8[2 * kk2 + 1] = pk4_fp8(lo[4], lo[5], lo[6], lo[7]);
        buf_store16_sc1(rwf, static_cast<uint32_t>((wave * 4 + 2 * pass + kk2) * 64 + lane) * 16u, hi);
      }
      buf_store16_sc1(rwf, kWLoOff + static_cast<uint32_t>(wave * 2048 + pass * 1024 + lane * 16),
                      lo8);
      __syncthreads();
    }
    if (kU) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int idx = tid + 256 * i;
        *reinterpret_cast<u32x4 *>(&sX[(idx >> 4) * kStrideK + (idx & 15) * 8]) = vrows[i];
      }
      __syncthreads();
    }
  }
  if (kU) {
    f32x4 Y[4][2];
    solve(sBeta, Y);
    // u tiles in MFMA result order: [chunk][head][row tile][col tile][lane][4]
    const auto rut = buf_rsrc(ws_u + ch_head * (kChunk * kDV), kChunk * kDV * 4);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
        buf_store16_sc1(rut, static_cast<uint32_t>((i * 8 + 2 * wave + nt) * 64 + lane) * 16u,
                        __builtin_bit_cast(u32x4, Y[i][nt]));
  }
}


// T form of the intra kernel (per chunk c, v-head h; LDS from smem, 30 KB):
//   * wave 0: gating, chunk-local cumsum G, the per-token vectors.
//   * A = strictly-lower(beta_i exp(G_i - G_j) K K^T) on MFMA (K exact bf16).
//   * T = (I + A)^-1: the four 16x16 diagonal blocks D_i by forward
//     substitution (wave i), then wave j walks block column j (t_column),
//       T_jj = D_j,   T_ij = -D_i sum_{j<=m<i} A_im T_mj   (i > j),
//     on split-bf16 16x16x16 MFMAs (a result tile's layout is the next
//     product's B-operand layout, so the column stays in registers).
// T goes to the workspace (w region) as split A-operand fragments of the
// state kernel, which applies it to the state-dependent right-hand side
// itself; (beta, beta e^G) go to the u region.
constexpr int kIntraTLds = kChunk * kStrideK * 2 + 10 * kABlk * 4 + 2 * kChunk * 4;
__device__ __forceinline__ void t_intra(
    char *smem, int c, int h, int start, int len, const uint16_t *__restrict__ k,
    const float *__restrict__ A_log, const uint16_t *__restrict__ a,
    const float *__restrict__ dt_bias, const uint16_t *__restrict__ b, const Heads &H,
    float *__restrict__ ws_G, float *__restrict__ ws_dcy, float *__restrict__ ws_eg,
    uint16_t *__restrict__ ws_w, float *__restrict__ ws_u) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g = lane >> 4, kg = g * 8;
  const int hq = h / H.ratio;
  const size_t ch_head = static_cast<size_t>(c) * H.v + h;

  constexpr int kStrideA4 = 68;  // f32 stride of the T scratch (16-byte rows)
  //   sK: K row-major until A is built, then T (f32 [64][68]) for the
  //       fragment transposition.
  //   sA: the ten lower 16x16 blocks of A (as the WY kernel's); the
  //       diagonal ones become the inverses D_w.
  uint16_t *const sK = reinterpret_cast<uint16_t *>(smem);                   // [64][136]
  float *const sA = reinterpret_cast<float *>(sK + kChunk * kStrideK);        // 10 blocks
  float *const sBeta = sA + 10 * kABlk, *const sG = sBeta + kChunk;
  static_assert(kChunk * kStrideA4 * 4 <= kChunk * kStrideK * 2, "T must fit in the K tile");
  float *const sT = reinterpret_cast<float *>(sK);

  // K row-major into LDS (rows past the chunk read zero through the
  // descriptor's range); every load issued before the LDS stores, and the
  // gating of wave 0 runs while they are in flight.
  {
    const uint32_t rstride = static_cast<uint32_t>(H.qk) * (kDK * 2);
    const auto rs = buf_rsrc(k + (static_cast<size_t>(start) * H.qk + hq) * kDK,
                             static_cast<uint32_t>(len) * rstride);
    u32x4 kv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = tid + 256 * i;
      kv[i] = buf_load16(rs, static_cast<uint32_t>(idx >> 4) * rstride + (idx & 15) * 16);
    }
    // Gating and the chunk-local cumsum (wave 0, lane = token).  Padding
    // tokens get g = 0 and beta = 0, so G stays at G_last past the end of the
    // chunk.
    if (wave == 0) {
      float gl, be;
      chunk_gates(lane, start, len, h, H, A_log, a, dt_bias, b, gl, be);
      float G = gl;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float y = __shfl_up(G, off);
        if (lane >= off) G += y;
      }
      sG[lane] = G;
      sBeta[lane] = be;
      const float G_last = __shfl(G, 63);
      ws_G[ch_head * kChunk + lane] = G;
      ws_dcy[ch_head * kChunk + lane] = expf(G_last - G);
      float *bb = ws_u + ch_head * (kChunk * kDV);  // (beta, beta e^G) in the u region
      bb[lane] = be;
      bb[kChunk + lane] = be * expf(G);
      if (lane == 0) ws_eg[ch_head] = expf(G_last);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = tid + 256 * i;
      *reinterpret_cast<u32x4 *>(&sK[(idx >> 4) * kStrideK + (idx & 15) * 8]) = kv[i];
    }
  }
  __syncthreads();

  build_A(sK, sA, sG, sBeta, len, wave, lane);
  __syncthreads();

  diag_inverse(sA, wave, lane);  // D_w = (I + A_ww)^-1 in place of A_ww
  __syncthreads();

  // Block column j = wave of T (t_column), in MFMA result order.
  f32x4 Tc[4];
  t_column(sA, wave, g, r16, Tc);
  // sK (K) is dead since A was built: T (f32) goes there, upper blocks zero.
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      sT[(16 * i + 4 * g + r) * kStrideA4 + 16 * wave + r16] = Tc[i][r];
  __syncthreads();

  // T as A-operand fragments of the state kernel (row 16*rt + r16, 8
  // consecutive k), split hi/lo: [chunk][head][rt][kk][lane][hi 8 | lo 8].
  // (Plain stores: written through, as the WY form's outputs are, T made
  // the state kernel's T-form steps slower: 4x8192 252.7 -> 273.9 us.)
  uint16_t *tf = ws_w + ch_head * (kChunk * kDK * 2);  // T in the w region
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    const f32x4 x0 = *reinterpret_cast<const f32x4 *>(&sT[(16 * wave + r16) * kStrideA4 + 32 * kk + kg]);
    const f32x4 x1 = *reinterpret_cast<const f32x4 *>(&sT[(16 * wave + r16) * kStrideA4 + 32 * kk + kg + 4]);
    const float x8[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
    u32x4 hi, lo;
    split8(x8, hi, lo);
    uint16_t *dst = tf + ((wave * 2 + kk) * 64 + lane) * 16;
    *reinterpret_cast<u32x4 *>(dst) = hi;
    *reinterpret_cast<u32x4 *>(dst + 8) = lo;
  }
}


// ---------------------------------------------------------------------------
// 2. intra-chunk: per (chunk c, v-head h) = chunk_head_of(unit), one kernel
// instantiated per form with its own LDS size (WY 31 KB: four to five
// workgroups per CU; T 35 KB: four), and once for a form the device picks
// (FORM -1: the index kernel's flag chooses the path per launch; the union
// of both, 35 KB and 104 VGPRs, still fits four per CU), so a device-decided
// batch pays one intra launch, not two.
//
// One unit per workgroup: looping over units raised register pressure (the
// WY intra kernel would drop to three workgroups per CU, the output kernel
// would spill); only the state kernel loops (see there).
// ---------------------------------------------------------------------------
// SPLIT: two workgroups per (chunk, v-head), the w half and the u half;
// workgroup id 16 s + 8 p + x (x = XCD) is half p of the pair 8 s + x, so
// both halves of a chunk run on the same XCD and share its K rows in L2.
template <bool SPLIT>
__device__ __forceinline__ void intra_wy_unit(
    char *smem, int c, int h, int4 ch, int half, const uint16_t *__restrict__ k,
    const uint16_t *__restrict__ v, const float *__restrict__ A_log,
    const uint16_t *__restrict__ a, const float *__restrict__ dt_bias,
    const uint16_t *__restrict__ b, const Heads &H, float *__restrict__ ws_G,
    float *__restrict__ ws_dcy, float *__restrict__ ws_eg, uint16_t *__restrict__ ws_w,
    float *__restrict__ ws_u, uint16_t *__restrict__ ws_kt, bool gemm) {
  if (!SPLIT)
    wy_intra<0>(smem, c, h, ch.y, ch.z, k, v, A_log, a, dt_bias, b, H, ws_G, ws_dcy, ws_eg,
                    ws_w, ws_u, ws_kt, gemm);
  else if (half)
    wy_intra<2>(smem, c, h, ch.y, ch.z, k, v, A_log, a, dt_bias, b, H, ws_G, ws_dcy, ws_eg,
                    ws_w, ws_u, ws_kt, false);
  else
    wy_intra<1>(smem, c, h, ch.y, ch.z, k, v, A_log, a, dt_bias, b, H, ws_G, ws_dcy, ws_eg,
                    ws_w, ws_u, ws_kt, false);
}

template <int FORM, bool SPLIT>
__device__ __forceinline__ void intra_body(
    const uint16_t *__restrict__ k, const uint16_t *__restrict__ v,
    const float *__restrict__ A_log, const uint16_t *__restrict__ a,
    const float *__restrict__ dt_bias, const uint16_t *__restrict__ b,
    const int4 *__restrict__ chunks, OneSeq one, int nt_max, Heads H,
    const int *__restrict__ form_flag, const SelfIndex &si, float *__restrict__ ws_G,
    float *__restrict__ ws_dcy, float *__restrict__ ws_eg, uint16_t *__restrict__ ws_w,
    float *__restrict__ ws_u, uint16_t *__restrict__ ws_kt) {
  static_assert(!(SPLIT && FORM != 0), "only the WY form splits into halves");
  constexpr int kLds0 = FORM == 0 ? kIntraWyLds
                        : FORM == 1 ? kIntraTLds
                                    : (kIntraWyLds > kIntraTLds ? kIntraWyLds : kIntraTLds);
  constexpr int kLds = kLds0 > kSelfIndexLds ? kLds0 : kSelfIndexLds;
  __shared__ __align__(16) char smem[kLds];
  // This workgroup's (chunk, v-head) -- and, split, its half: workgroup id
  // 16 s + 8 p + x is half p of the pair 8 s + x (the same for both forms).
  const int id = blockIdx.x;
  const int pair = SPLIT ? (((id >> 4) << 3) | (id & 7)) : id;
  const int half = SPLIT ? (id >> 3) & 1 : 0;
  int c = 0, h = 0;
  const bool unit = chunk_head_of(pair, nt_max, H, c, h);
  int form = FORM;
  int4 ch;
  int nt;  // the batch's chunks
  if (si.cu != nullptr) {
    if (!unit && id != 0) return;
    const SelfIndexed x = self_index(smem, si, nt_max, H.v);
    if (FORM < 0) form = x.form;
    nt = x.nt;
    ch = self_chunk(smem, si.N, c, x.nt);
    if (unit && h == 0 && half == 0) si.chunks[c] = ch;
    __syncthreads();  // the LDS arrays are dead: the unit's tiles take their place
    if (!unit) return;
  } else {
    // one sequence: its contract bits (several: the index kernel's)
    if (one.cu != nullptr && id == 0 && threadIdx.x == 0)
      si.status[0] = cu_status_bits(raw_cu(one.cu, one.cu64, 0), raw_cu(one.cu, one.cu64, 1), one.T);
    // the early-output words start each call at zero (the state launch
    // after this one counts up from them): 256 per workgroup (the grid has
    // more than enough); only the WY form runs one sequence
    if constexpr (FORM == 0) {
      if (si.early != nullptr && id < (si.n_early + 255) / 256) {
        const int i = id * 256 + static_cast<int>(threadIdx.x);
        if (i < si.n_early) si.early[i] = 0;
      }
    }
    if (!unit) return;
    if (FORM < 0) form = *form_flag;
    if (one.cu != nullptr) {
      int bos, eos;
      one_seq_bounds(one, bos, eos);
      nt = (eos - bos + kChunk - 1) / kChunk;
    } else {
      nt = si.offsets[si.N];  // the index kernel's chunk count
    }
    ch = chunk_info(chunks, c, one);
  }
  if (ch.x < 0) return;
  if (form == 1)
    t_intra(smem, c, h, ch.y, ch.z, k, A_log, a, dt_bias, b, H, ws_G, ws_dcy, ws_eg, ws_w, ws_u);
  else
    intra_wy_unit<SPLIT>(smem, c, h, ch, half, k, v, A_log, a, dt_bias, b, H, ws_G, ws_dcy, ws_eg,
                         ws_w, ws_u, ws_kt, !SPLIT && nt * H.v >= kIntraGemmMinUnits);
}

template <int FORM, bool SPLIT>
__global__ __launch_bounds__(256) void prefill_intra_kernel(
    const uint16_t *__restrict__ k, const uint16_t *__restrict__ v,
    const float *__restrict__ A_log, const uint16_t *__restrict__ a,
    const float *__restrict__ dt_bias, const uint16_t *__restrict__ b,
    const int4 *__restrict__ chunks, OneSeq one, int nt_max, Heads H,
    const int *__restrict__ form_flag, SelfIndex si, float *__restrict__ ws_G,
    float *__restrict__ ws_dcy, float *__restrict__ ws_eg, uint16_t *__restrict__ ws_w,
    float *__restrict__ ws_u, uint16_t *__restrict__ ws_kt) {
  intra_body<FORM, SPLIT>(k, v, A_log, a, dt_bias, b, chunks, one, nt_max, H, form_flag, si, ws_G,
                          ws_dcy, ws_eg, ws_w, ws_u, ws_kt);
}
// the form left to the device: held to five workgroups per CU, as each form
// alone (the union of both paths needs a few more registers than either)
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(5)))
void prefill_intra_either_kernel(
    const uint16_t *__restrict__ k, const uint16_t *__restrict__ v,
    const float *__restrict__ A_log, const uint16_t *__restrict__ a,
    const float *__restrict__ dt_bias, const uint16_t *__restrict__ b,
    const int4 *__restrict__ chunks, OneSeq one, int nt_max, Heads H,
    const int *__restrict__ form_flag, SelfIndex si, float *__restrict__ ws_G,
    float *__restrict__ ws_dcy, float *__restrict__ ws_eg, uint16_t *__restrict__ ws_w,
    float *__restrict__ ws_u, uint16_t *__restrict__ ws_kt) {
  intra_body<-1, false>(k, v, A_log, a, dt_bias, b, chunks, one, nt_max, H, form_flag, si, ws_G,
                        ws_dcy, ws_eg, ws_w, ws_u, ws_kt);
}

// ---------------------------------------------------------------------------
// 3. state recurrence: the two forms of a step, then the kernel.
// ---------------------------------------------------------------------------
constexpr uint32_t kWBytes = kChunk * kDK * 4;    // w region of one (chunk, head)
constexpr uint32_t kKtBytes = kDK * kChunk * 2;   // K^T of one (chunk, q/k head)
constexpr uint32_t kUBytes = kChunk * kDV * 4;    // u of one (chunk, head), f32

struct WyFrag {
  u32x4 wh[4];         // w rows 16*wave + (lane & 15), k-steps 0..3 (bf16 hi)
  u32x4 wl8[2];        // the same rows' low parts, fp8, k-steps (0, 1) and (2, 3)
  float wls;           // the low parts' inverse scale
  u32x4 ka[2][2];      // K^T rows 16*(2*wave + mi) + (lane & 15), k-steps 0..1
  f32x4 u;             // u[16*rw + 4*(lane >> 4) + r][vw + (lane & 15)]
  f32x4 dcy;           // exp(G_last - G_i) of the lane's four v_new rows
  float eg;            // exp(G_last)
};

// The fragments of chunk c, in seven parts of at most two loads that the
// state step issues at seven points of the step before (so that no wave
// issues a burst of loads and waits for the texture unit): 0-1 K^T, 2-3 w hi,
// 4 w lo, 5 u and the decay factors, 6 exp(G_last) and w lo's scale.
template <int PART, bool LOAD_U>
__device__ __forceinline__ void load_wy_part(WyFrag &f, int c, int h, const Heads &H,
                                             int vw, int wave, int lane, const float *ws_dcy,
                                             const float *ws_eg, const uint16_t *ws_w,
                                             const float *ws_u, const uint16_t *ws_kt) {
  const size_t ch_head = static_cast<size_t>(c) * H.v + h;
  // w: hi [mb][kk][lane][8] and fp8 lo [mb][kk / 2][lane][kk % 2][8]
  // fragments of this wave's 16 rows, and lo's inverse scale
  const auto rw = buf_rsrc(ws_w + ch_head * (kWBytes / 2), kWBytes);
  const uint32_t wo = static_cast<uint32_t>(wave) * 4096u + static_cast<uint32_t>(lane) * 16u;
  const uint32_t lo = kWLoOff + static_cast<uint32_t>(wave) * 2048u + static_cast<uint32_t>(lane) * 16u;
  if constexpr (PART <= 1) {
    // K^T: [mt][kk][lane][8] fragments of this wave's two 16-row tiles
    const auto rk = buf_rsrc(ws_kt + (static_cast<size_t>(c) * H.qk + h / H.ratio) * (kKtBytes / 2), kKtBytes);
    const uint32_t ko = static_cast<uint32_t>(wave) * 4096u + static_cast<uint32_t>(lane) * 16u;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) f.ka[PART][kk] = buf_load16(rk, ko + PART * 2048 + kk * 1024);
  } else if constexpr (PART <= 3) {
#pragma unroll
    for (int kk = 2 * (PART - 2); kk < 2 * (PART - 1); ++kk) f.wh[kk] = buf_load16(rw, wo + kk * 1024);
  } else if constexpr (PART == 4) {
    f.wl8[0] = buf_load16(rw, lo);
    f.wl8[1] = buf_load16(rw, lo + 1024);
  } else if constexpr (PART == 5) {
    const int q4 = 4 * (lane >> 4);
    // u: [row tile][col tile][lane][4] result tiles
    if constexpr (LOAD_U) {
      const auto ru = buf_rsrc(ws_u + ch_head * (kUBytes / 4), kUBytes);
      f.u = __builtin_bit_cast(f32x4, buf_load16(ru, static_cast<uint32_t>((wave * 8 + (vw >> 4)) * 64 + lane) * 16u));
    } else {
      f.u = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const auto rd = buf_rsrc(ws_dcy + ch_head * kChunk, kChunk * 4);
    f.dcy = __builtin_bit_cast(f32x4, buf_load16(rd, static_cast<uint32_t>(16 * wave + q4) * 4u));
  } else {
    f.eg = buf_load_f32(ws_eg + ch_head);
    f.wls = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rw, kWScaleOff, 0, 0));
  }
}

// WY form of a state step (see the kernel comment): wave w owns K-rows
// 32w..32w+31 of the state tile and v_new rows (tokens) 16w..16w+15.
// Everything a chunk needs that does not depend on the state (w, K^T, u,
// decay factors) is prefetched into registers two chunks ahead, so the
// serial chain per chunk is two LDS exchanges, two barriers and the MFMAs.
//
// MAP: the linear part of the map over the chunks instead of the state --
// rows v0..v0+15 of the identity as the start, u = 0 (no u loads), no v_new
// stores; ht then receives M over the chunks before c (rows j = v0..v0+15 of
// [j][k]) at chunk index c - ht_c0.
// PROG: publish the unit's progress in *prog for the early output (every
// thread stores the same word: no divergent branch splits the loop body).
constexpr int kStateWyLds = 2 * 16 * kStrideK * 2 + 3 * 16 * kStrideT * 2;
template <bool MAP, bool PROG>
__device__ __forceinline__ void wy_state(
    char *smem, int c0, int nch, int npre, int h, int v0, int wave, int lane, size_t sbase,
    const float *state, float *new_state, const float *ws_dcy, const float *ws_eg,
    const uint16_t *ws_w, const float *ws_u, const uint16_t *ws_kt, uint16_t *ws_ht,
    uint16_t *ws_vnt, const Heads &H, int ht_c0, int *prog, int prog_tag) {
  const int ct = 0;  // one 16-column tile per workgroup
  const int r16 = lane & 15, kg = (lane >> 4) * 8, q4 = 4 * (lane >> 4);
  const int lc = 16 * ct;
  const int vw = v0 + lc;
  uint16_t *const sSh = reinterpret_cast<uint16_t *>(smem);
  uint16_t *const sSl = sSh + 16 * kStrideK;
  uint16_t *const sVh = sSl + 16 * kStrideK;
  uint16_t *const sVl = sVh + 16 * kStrideT;
  uint16_t *const sN = sVl + 16 * kStrideT;  // v_new, bf16 [v][token]

  f32x4 S[2];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) {
    const int kr = 16 * (2 * wave + mi) + q4, vc = vw + r16;
    if constexpr (MAP) {
#pragma unroll
      for (int r = 0; r < 4; ++r) S[mi][r] = vc == kr + r ? 1.f : 0.f;
    } else if (state != nullptr) {
      S[mi] = *reinterpret_cast<const f32x4 *>(state + sbase + vc * kDK + kr);
    } else {
      S[mi] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }

  // One chunk of the recurrence, from the prefetched fragments f, while the
  // fragments of chunk cn go into g (free since the step before) in seven
  // parts, each pinned between scheduling barriers where the wave would wait
  // anyway: at the start of (a) (for the update's results), before each
  // barrier, after (b)'s and (d)'s LDS reads, and among (b)'s and (d)'s MFMAs.
  auto chunk_at = [&](int i) { return c0 + (i < npre ? i : npre - 1); };
#define GDN_PART(P, G, I)                                                                     \
  __builtin_amdgcn_sched_barrier(0);                                                          \
  load_wy_part<P, !MAP>(G, chunk_at(I), h, H, vw, wave, lane, ws_dcy, ws_eg, ws_w, ws_u,    \
                        ws_kt);                                                               \
  __builtin_amdgcn_sched_barrier(0)
  auto step = [&](const WyFrag &f, int c, WyFrag &g, int cn) {
    const size_t ch_head = static_cast<size_t>(c) * H.v + h;
    uint16_t *ht = ws_ht + (static_cast<size_t>(c - ht_c0) * H.v + h) * (kDV * kDK);
    uint16_t *vnt = ws_vnt + ch_head * (kDV * kChunk);
    GDN_PART(0, g, cn);
    // (a) chunk-start state: split copy into LDS ([v][k]) for w S, whose hi
    //     half (rounded to nearest) is also the bf16 chunk-start state of the
    //     output kernel.
#pragma unroll
    for (int mi = 0; mi < 2; ++mi) {
      const int kr = 16 * (2 * wave + mi) + q4, vl = lc + r16;
      uint32_t h0, h1, l0, l1;
      split2_rne(S[mi][0], S[mi][1], h0, l0);
      split2_rne(S[mi][2], S[mi][3], h1, l1);
      *reinterpret_cast<u32x2 *>(&sSh[vl * kStrideK + kr]) = u32x2{h0, h1};
      *reinterpret_cast<u32x2 *>(&sSl[vl * kStrideK + kr]) = u32x2{l0, l1};
    }
    GDN_PART(1, g, cn);
    __syncthreads();
    // ht: the workgroup's 16 rows of the bf16 chunk-start state ([v][k], 4 KB
    // contiguous) from the LDS copy, one 16-byte store per thread
    {
      const int t = threadIdx.x, row = t >> 4, k0 = (t & 15) * 8;
      *reinterpret_cast<u32x4 *>(ht + (vw + row) * kDK + k0) =
          *reinterpret_cast<const u32x4 *>(&sSh[(lc + row) * kStrideK + k0]);
    }

    // (b) w S for rows 16*wave..+15; three independent accumulation chains
    //     (hi*hi, hi*lo, lo*hi) shorten the dependent MFMA sequence.  w's
    //     low part is widened from fp8 to bf16 here, at its use (exact), and
    //     its scale applied to the lo*hi chain in (c).
    f32x4 P0 = {0.f, 0.f, 0.f, 0.f}, P1 = P0, P2 = P0;
    u32x4 sh[4], sl[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      sh[kk] = *reinterpret_cast<const u32x4 *>(&sSh[(lc + r16) * kStrideK + 32 * kk + kg]);
      sl[kk] = *reinterpret_cast<const u32x4 *>(&sSl[(lc + r16) * kStrideK + 32 * kk + kg]);
    }
    GDN_PART(2, g, cn);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const u32x4 wl = fp8x8_to_bf16(f.wl8[kk >> 1][2 * (kk & 1)], f.wl8[kk >> 1][2 * (kk & 1) + 1]);
      P0 = mfma_bf16(f.wh[kk], sh[kk], P0);
      P1 = mfma_bf16(f.wh[kk], sl[kk], P1);
      P2 = mfma_bf16(wl, sh[kk], P2);
      if (kk == 1) {
        GDN_PART(3, g, cn);
      }
    }

    // (c) v_new = u - w S -> workspace (bf16, [v][token]) for the output
    //     kernel; exp(G_last - G_i) v_new -> LDS (split, [v][token]) for K^T v.
    {
      const int vl = lc + r16;
      float vn[4], vs[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        vn[r] = f.u[r] - ((P0[r] + P1[r]) + P2[r] * f.wls);
        vs[r] = f.dcy[r] * vn[r];
      }
      const u32x2 rn = {pk_bf16(vn[0], vn[1]), pk_bf16(vn[2], vn[3])};
      uint32_t h0, h1, l0, l1;
      split2(vs[0], vs[1], h0, l0);
      split2(vs[2], vs[3], h1, l1);
      const u32x2 hi = {h0, h1}, lo = {l0, l1};
      const int i0 = 16 * wave + q4;
      if constexpr (!MAP) *reinterpret_cast<u32x2 *>(&sN[vl * kStrideT + i0]) = rn;
      *reinterpret_cast<u32x2 *>(&sVh[vl * kStrideT + i0]) = hi;
      *reinterpret_cast<u32x2 *>(&sVl[vl * kStrideT + i0]) = lo;
    }
    GDN_PART(4, g, cn);
    __syncthreads();
    // Progress for the early output: each wave has used u of chunk c, loaded
    // in step c - 2 after its ht and v_new stores of chunk c - 2; vector
    // memory operations complete in order, so those stores have reached L2,
    // and chunks c0 .. c - 2 are out.  The word carries the unit's XCD
    // (prog_tag) above the chunk count.
    if constexpr (PROG)
      __hip_atomic_store(prog, prog_tag | (c - c0 >= 2 ? c - c0 - 1 : 0), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_WORKGROUP);
    // v_new: the workgroup's 16 rows of [v][token] bf16 (2 KB contiguous) from
    // the LDS copy, one 8-byte store per thread
    if constexpr (!MAP) {
      const int t = threadIdx.x, row = t >> 4, i0 = (t & 15) * 4;
      *reinterpret_cast<u32x2 *>(vnt + (vw + row) * kChunk + i0) =
          *reinterpret_cast<const u32x2 *>(&sN[(lc + row) * kStrideT + i0]);
    }

    // (d) S <- exp(G_last) S + K^T (exp(G_last - G) v_new); K is exact in bf16,
    //     so two MFMAs (hi, lo) per k-step, in two independent chains.
    u32x4 vh[2], vl[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      vh[kk] = *reinterpret_cast<const u32x4 *>(&sVh[(lc + r16) * kStrideT + 32 * kk + kg]);
      vl[kk] = *reinterpret_cast<const u32x4 *>(&sVl[(lc + r16) * kStrideT + 32 * kk + kg]);
    }
    GDN_PART(5, g, cn);
#pragma unroll
    for (int mi = 0; mi < 2; ++mi) {
      if (mi == 1) {
        GDN_PART(6, g, cn);
      }
      f32x4 acc = S[mi];
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] *= f.eg;
      f32x4 acc2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        acc = mfma_bf16(f.ka[mi][kk], vh[kk], acc);
        acc2 = mfma_bf16(f.ka[mi][kk], vl[kk], acc2);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) S[mi][r] = acc[r] + acc2[r];
    }
  };

  // Ring of three fragment sets: chunk i uses set i % 3 while the set of
  // chunk i + 1 is in flight and that of chunk i + 2 goes out during the step.
  // The loop body is three straight steps with one exit test, at the back
  // edge, so the loop head is reached with the same loads pending from both
  // of its predecessors and the compiler waits for exactly the set in use (an
  // exit after each step made it merge those paths and wait for nearly every
  // prefetch).  The last 0-2 chunks run after the loop.  Prefetches are
  // clamped to npre chunks, a bound known at launch (for one sequence, from
  // T), so the first ones go out before the chunk count arrives from memory;
  // past the last chunk they re-read a chunk slot of the workspace and are
  // never used.  (A fourth set measured slower: the extra registers push
  // accumulators into AGPRs.)
  if (npre > 0) {
    WyFrag fa, fb, fc;
    auto load_all = [&](WyFrag &g, int i) {
      GDN_PART(0, g, i);
      GDN_PART(1, g, i);
      GDN_PART(2, g, i);
      GDN_PART(3, g, i);
      GDN_PART(4, g, i);
      GDN_PART(5, g, i);
      GDN_PART(6, g, i);
    };
    load_all(fa, 0);
    load_all(fb, 1);
    int ci = 0;
    for (; ci + 3 <= nch; ci += 3) {
      step(fa, c0 + ci, fc, ci + 2);
      step(fb, c0 + ci + 1, fa, ci + 3);
      step(fc, c0 + ci + 2, fb, ci + 4);
    }
    if (ci < nch) step(fa, c0 + ci, fc, ci + 2);
    if (ci + 1 < nch) step(fb, c0 + ci + 1, fa, ci + 3);
  }
#undef GDN_PART

  // Final state (zeros for a zero-length sequence, as the reference).
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) {
    const int kr = 16 * (2 * wave + mi) + q4, vc = vw + r16;
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    *reinterpret_cast<f32x4 *>(new_state + sbase + vc * kDK + kr) = (MAP || nch > 0) ? S[mi] : z;
  }
}


struct TFrag {
  u32x4 kf[4];          // K rows 16*wave + (lane & 15), k-steps 0..3 (A operand of K S)
  u32x4 th[2], tl[2];   // T rows 16*wave + (lane & 15), k-steps 0..1 (hi / lo)
  f32x4 beta, bg, dcy;  // beta, beta e^G, exp(G_last - G) of rows 16*wave + 4*(lane >> 4) + r
  u32x2 vr;             // V[16*wave + (lane >> 2)][v0 + 4*(lane & 3) + 0..3], bf16 (through
                        // LDS to the rows 16*wave + 4*(lane >> 4) + r of column
                        // v0 + (lane & 15) that Y needs)
  float eg;             // exp(G_last)
};

// Per-lane byte offsets of the fragment loads: fixed for the whole kernel.
struct FragOffsets {
  uint32_t k, t, v, vec;
};
__device__ __forceinline__ u32x2 buf_load8(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, 0));
}

// Fragments of chunk c (tokens [start, start + len)) for v-head h, in six
// parts that the state step issues after the last use of the registers they
// refill (so that no wave issues all of a set's loads at once): 0 K rows
// 0..1, 1 K rows 2..3 and the per-token beta, beta e^G, 2 T, 3 V, 4 the decay
// factors, 5 exp(G_last).  V is one 8-byte load per lane (a row's 16
// columns in four lanes) instead of four 2-byte loads.  T is lower triangular: the rows of waves 0 and 1
// (0..31) are zero in columns 32..63, so those waves load (and multiply)
// only the first k-step.
template <int PART>
__device__ __forceinline__ void load_t_part(TFrag &f, int c, int start, int len, int h,
                                            const Heads &H, const FragOffsets &o,
                                            const uint16_t *k, const uint16_t *v,
                                            const float *ws_dcy, const float *ws_eg,
                                            const uint16_t *ws_w, const float *ws_u,
                                            bool t_upper) {
  const size_t ch_head = static_cast<size_t>(c) * H.v + h;
  const uint32_t nlen = static_cast<uint32_t>(len);
  if constexpr (PART <= 1) {
    const auto rk = buf_rsrc(k + (static_cast<size_t>(start) * H.qk + h / H.ratio) * kDK,
                             nlen * static_cast<uint32_t>(H.qk) * (kDK * 2));
#pragma unroll
    for (int kk = 2 * PART; kk < 2 * PART + 2; ++kk) f.kf[kk] = buf_load16(rk, o.k + kk * 64);
    if constexpr (PART == 1) {
      const auto rb = buf_rsrc(ws_u + ch_head * (kChunk * kDV), 2 * kChunk * 4);  // (beta, beta e^G)
      f.beta = __builtin_bit_cast(f32x4, buf_load16(rb, o.vec));
      f.bg = __builtin_bit_cast(f32x4, buf_load16(rb, o.vec + kChunk * 4));
    }
  } else if constexpr (PART == 2) {
    const auto rt = buf_rsrc(ws_w + ch_head * (kChunk * kDK * 2), kTElems * 2);  // T, w region
    f.th[0] = buf_load16(rt, o.t);
    f.tl[0] = buf_load16(rt, o.t + 16);
    if (t_upper) {
      f.th[1] = buf_load16(rt, o.t + 2048);
      f.tl[1] = buf_load16(rt, o.t + 2048 + 16);
    } else {
      f.th[1] = f.tl[1] = u32x4{0u, 0u, 0u, 0u};
    }
  } else if constexpr (PART == 3) {
    const auto rv = buf_rsrc(v + (static_cast<size_t>(start) * H.v + h) * kDV,
                             nlen * static_cast<uint32_t>(H.v) * (kDV * 2));
    f.vr = buf_load8(rv, o.v);
  } else if constexpr (PART == 4) {
    const auto rd = buf_rsrc(ws_dcy + ch_head * kChunk, kChunk * 4);
    f.dcy = __builtin_bit_cast(f32x4, buf_load16(rd, o.vec));
  } else {
    f.eg = buf_load_f32(ws_eg + ch_head);
  }
}

// T form of a state step (see the kernel comment): wave w owns K-rows
// 32w..32w+31 of the state tile and tokens 16w..16w+15 of the per-chunk
// products.  Per chunk:
//   X     = K S                              (K exact bf16, S split)
//   Y     = beta V - beta e^G X              (the state-dependent right-hand side)
//   v_new = T Y                              (= u - w S, without w or u)
//   S    <- e^G_last S + K^T (D v_new)       (D = exp(G_last - G))
// Three LDS exchanges (S, Y, D v_new) with a barrier each.  K and V come
// straight from the input tensors; everything that does not depend on the
// state (K, T, V, the per-token vectors) is prefetched into registers one
// chunk ahead through buffer descriptors.  K^T, the A operand of the update,
// is read transposed out of the LDS copy of the chunk's K rows.
constexpr int kStateTLds =
    2 * 16 * kStrideK * 2 + 5 * 16 * kStrideT * 2 + kChunk * kStrideK * 2 + kChunk * 16 * 2;
__device__ __forceinline__ void t_state(
    char *smem, int c0, int nch, int bos, int eos, int h, int v0, int wave, int lane,
    size_t sbase, const uint16_t *k, const uint16_t *v, const float *state, float *new_state,
    const float *ws_dcy, const float *ws_eg, const uint16_t *ws_w, const float *ws_u,
    uint16_t *ws_ht, uint16_t *ws_vnt, const Heads &H) {
  const int r16 = lane & 15, g = lane >> 4, kg = 8 * g, q4 = 4 * g;
  const int vc = v0 + r16;  // this lane's state column
  uint16_t *const sSh = reinterpret_cast<uint16_t *>(smem);  // S^T split, [v][k]
  uint16_t *const sSl = sSh + 16 * kStrideK;
  uint16_t *const sYh = sSl + 16 * kStrideK;                 // Y split, [v][token]
  uint16_t *const sYl = sYh + 16 * kStrideT;
  uint16_t *const sVh = sYl + 16 * kStrideT;                 // D v_new split, [v][token]
  uint16_t *const sVl = sVh + 16 * kStrideT;
  uint16_t *const sK = sVl + 16 * kStrideT;                  // the chunk's K rows, [token][k]
  uint16_t *const sN = sK + kChunk * kStrideK;               // v_new, bf16 [v][token]
  uint16_t *const sV = sN + 16 * kStrideT;                   // the chunk's V slice, [token][16]

  f32x4 S[2];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) {
    const int kr = 16 * (2 * wave + mi) + q4;
    if (state != nullptr && nch > 0)
      S[mi] = *reinterpret_cast<const f32x4 *>(state + sbase + vc * kDK + kr);
    else
      S[mi] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  FragOffsets fo;
  fo.k = (static_cast<uint32_t>(16 * wave + r16) * H.qk * kDK + kg) * 2;
  fo.t = static_cast<uint32_t>(wave) * 4096u + static_cast<uint32_t>(lane) * 32u;
  fo.v = (static_cast<uint32_t>(16 * wave + (lane >> 2)) * H.v * kDV + v0 + 4 * (lane & 3)) * 2;
  fo.vec = static_cast<uint32_t>(16 * wave + q4) * 4u;

  // Chunk i's fragments, part P (past the last chunk: the last chunk again,
  // so every step issues the same loads).
  auto load = [&](auto part, TFrag &f, int i) {
    i = i < nch ? i : nch - 1;
    const int start = bos + i * kChunk, rem = eos - start;
    __builtin_amdgcn_sched_barrier(0);
    load_t_part<decltype(part)::value>(f, c0 + i, start, rem < kChunk ? rem : kChunk, h, H, fo,
                                       k, v, ws_dcy, ws_eg, ws_w, ws_u, wave >= 2);
    __builtin_amdgcn_sched_barrier(0);
  };
  using TP0 = std::integral_constant<int, 0>;
  using TP1 = std::integral_constant<int, 1>;
  using TP2 = std::integral_constant<int, 2>;
  using TP3 = std::integral_constant<int, 3>;
  using TP4 = std::integral_constant<int, 4>;
  using TP5 = std::integral_constant<int, 5>;

  // One chunk of the recurrence, from the prefetched fragments f, which are
  // refilled with chunk cn's as the step finishes with each part: K rows and
  // the per-token vectors after (b), T after (c)'s products, V after Y, the
  // decay factors after (c), exp(G_last) after (d).
  auto step = [&](TFrag &f, int c, int cn) {
    const size_t ch_head = static_cast<size_t>(c) * H.v + h;
    uint16_t *ht = ws_ht + ch_head * (kDV * kDK);
    uint16_t *vnt = ws_vnt + ch_head * (kDV * kChunk);
    // (a) chunk-start state: split copy into LDS ([v][k]) for K S, whose hi
    //     half (rounded to nearest) is also the bf16 chunk-start state of the
    //     output kernel; the chunk's K rows and V slice into LDS.
#pragma unroll
    for (int mi = 0; mi < 2; ++mi) {
      const int kr = 16 * (2 * wave + mi) + q4;
      uint32_t h0, h1, l0, l1;
      split2_rne(S[mi][0], S[mi][1], h0, l0);
      split2_rne(S[mi][2], S[mi][3], h1, l1);
      *reinterpret_cast<u32x2 *>(&sSh[r16 * kStrideK + kr]) = u32x2{h0, h1};
      *reinterpret_cast<u32x2 *>(&sSl[r16 * kStrideK + kr]) = u32x2{l0, l1};
    }
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      *reinterpret_cast<u32x4 *>(&sK[(16 * wave + r16) * kStrideK + 32 * kk + kg]) = f.kf[kk];
    *reinterpret_cast<u32x2 *>(&sV[(16 * wave + (lane >> 2)) * 16 + 4 * (lane & 3)]) = f.vr;
    __syncthreads();
    // ht: the workgroup's 16 rows of the bf16 chunk-start state ([v][k], 4 KB
    // contiguous) from the LDS copy, one 16-byte store per thread (stores of
    // each lane's own 8 bytes, 32-byte pieces of 16 rows, cost ~20 us at
    // 4x8192), non-temporal: the T form runs batches whose ht and v_new
    // (48 KB per chunk and head) outgrow the caches, and streaming them past
    // L2 leaves it to the K, T and V lines the head's workgroups share
    // (4x8192 state 163 -> 156 us)
    {
      const int t = threadIdx.x, row = t >> 4, k0 = (t & 15) * 8;
      __builtin_nontemporal_store(*reinterpret_cast<const u32x4 *>(&sSh[row * kStrideK + k0]),
                                  reinterpret_cast<u32x4 *>(ht + (v0 + row) * kDK + k0));
    }

    // (b) X = K S for tokens 16*wave..+15 (two chains: S hi, S lo), then
    //     Y = beta V - beta e^G X -> LDS (split, [v][token]).  K^T fragments
    //     for (d): 8 tokens of one K column from the LDS copy of K.
    {
      f32x4 X0 = {0.f, 0.f, 0.f, 0.f}, X1 = X0;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const u32x4 sh = *reinterpret_cast<const u32x4 *>(&sSh[r16 * kStrideK + 32 * kk + kg]);
        const u32x4 sl = *reinterpret_cast<const u32x4 *>(&sSl[r16 * kStrideK + 32 * kk + kg]);
        X0 = mfma_bf16(f.kf[kk], sh, X0);
        X1 = mfma_bf16(f.kf[kk], sl, X1);
      }
      load(TP0{}, f, cn);
      // V[16 wave + 4 g + r][v0 + r16], r = 0..3, by one transposing read
      const u32x2 vt = ds_read_tr16(&sV[(16 * wave + q4 + (r16 >> 2)) * 16 + 4 * (r16 & 3)]);
      const float vf[4] = {__uint_as_float(vt[0] << 16), __uint_as_float(vt[0] & 0xffff0000u),
                           __uint_as_float(vt[1] << 16), __uint_as_float(vt[1] & 0xffff0000u)};
      float y[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) y[r] = f.beta[r] * vf[r] - f.bg[r] * (X0[r] + X1[r]);
      uint32_t h0, h1, l0, l1;
      split2(y[0], y[1], h0, l0);
      split2(y[2], y[3], h1, l1);
      const int i0 = 16 * wave + q4;
      *reinterpret_cast<u32x2 *>(&sYh[r16 * kStrideT + i0]) = u32x2{h0, h1};
      *reinterpret_cast<u32x2 *>(&sYl[r16 * kStrideT + i0]) = u32x2{l0, l1};
    }
    load(TP1{}, f, cn);
    load(TP3{}, f, cn);
    u32x4 ka[2][2];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const u32x2 x = ds_read_tr16(&sK[(32 * kk + kg + 4 * hh + (r16 >> 2)) * kStrideK +
                                           32 * wave + 16 * mi + 4 * (r16 & 3)]);
          ka[mi][kk][2 * hh] = x[0];
          ka[mi][kk][2 * hh + 1] = x[1];
        }
    __syncthreads();

    // (c) v_new = T Y for tokens 16*wave..+15 (T and Y split: three chains)
    //     -> workspace (bf16, [v][token]) for the output kernel;
    //     D v_new -> LDS (split, [v][token]) for K^T (D v_new).
    {
      f32x4 P0 = {0.f, 0.f, 0.f, 0.f}, P1 = P0, P2 = P0;
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        if (kk == 1 && wave < 2) break;  // T's rows 0..31 are zero in columns 32..63
        const u32x4 yh = *reinterpret_cast<const u32x4 *>(&sYh[r16 * kStrideT + 32 * kk + kg]);
        const u32x4 yl = *reinterpret_cast<const u32x4 *>(&sYl[r16 * kStrideT + 32 * kk + kg]);
        P0 = mfma_bf16(f.th[kk], yh, P0);
        P1 = mfma_bf16(f.th[kk], yl, P1);
        P2 = mfma_bf16(f.tl[kk], yh, P2);
      }
      load(TP2{}, f, cn);
      float vn[4], vs[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        vn[r] = (P0[r] + P1[r]) + P2[r];
        vs[r] = f.dcy[r] * vn[r];
      }
      const u32x2 rn = {pk_bf16(vn[0], vn[1]), pk_bf16(vn[2], vn[3])};
      uint32_t h0, h1, l0, l1;
      split2(vs[0], vs[1], h0, l0);
      split2(vs[2], vs[3], h1, l1);
      const int i0 = 16 * wave + q4;
      *reinterpret_cast<u32x2 *>(&sN[r16 * kStrideT + i0]) = rn;
      *reinterpret_cast<u32x2 *>(&sVh[r16 * kStrideT + i0]) = u32x2{h0, h1};
      *reinterpret_cast<u32x2 *>(&sVl[r16 * kStrideT + i0]) = u32x2{l0, l1};
    }
    load(TP4{}, f, cn);
    __syncthreads();
    // v_new: the workgroup's 16 rows of [v][token] bf16 (2 KB contiguous) from
    // the LDS copy, one 8-byte store per thread
    {
      const int t = threadIdx.x, row = t >> 4, i0 = (t & 15) * 4;
      __builtin_nontemporal_store(*reinterpret_cast<const u32x2 *>(&sN[row * kStrideT + i0]),
                                  reinterpret_cast<u32x2 *>(vnt + (v0 + row) * kChunk + i0));
    }

    // (d) S <- exp(G_last) S + K^T (D v_new); K is exact in bf16, so two MFMAs
    //     (hi, lo) per k-step, in two independent chains.
#pragma unroll
    for (int mi = 0; mi < 2; ++mi) {
      f32x4 acc = S[mi];
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] *= f.eg;
      f32x4 acc2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const u32x4 vh = *reinterpret_cast<const u32x4 *>(&sVh[r16 * kStrideT + 32 * kk + kg]);
        const u32x4 vl = *reinterpret_cast<const u32x4 *>(&sVl[r16 * kStrideT + 32 * kk + kg]);
        acc = mfma_bf16(ka[mi][kk], vh, acc);
        acc2 = mfma_bf16(ka[mi][kk], vl, acc2);
      }
      if (mi == 1) load(TP5{}, f, cn);
#pragma unroll
      for (int r = 0; r < 4; ++r) S[mi][r] = acc[r] + acc2[r];
    }
  };

  // Two fragment sets: chunk i uses set i % 2 while the set of chunk i + 1
  // is in flight and its own registers are refilled with chunk i + 2's as
  // the step finishes with them (a third set does not fit in the
  // registers).  The loop body is two straight steps with one exit test, at
  // the back edge, so the loop head is reached with the same loads pending
  // from both of its predecessors and the compiler waits for exactly the set
  // in use (an exit after each step made it merge those paths and wait for
  // nearly every prefetch).  A last odd chunk runs after the loop.  The
  // scheduling barriers around each part keep the compiler from moving a
  // load, or work on the other set's registers (with its load waits), across
  // the step.
  if (nch > 0) {
    TFrag fa, fb;
    auto load_all = [&](TFrag &f, int i) {
      load(TP0{}, f, i);
      load(TP1{}, f, i);
      load(TP2{}, f, i);
      load(TP3{}, f, i);
      load(TP4{}, f, i);
      load(TP5{}, f, i);
    };
    load_all(fa, 0);
    load_all(fb, 1);
    int ci = 0;
    for (; ci + 2 <= nch; ci += 2) {
      step(fa, c0 + ci, ci + 2);
      step(fb, c0 + ci + 1, ci + 3);
    }
    if (ci < nch) step(fa, c0 + ci, ci + 2);
  }

  // Final state (zeros for a zero-length sequence, as the reference).
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) {
    const int kr = 16 * (2 * wave + mi) + q4;
    *reinterpret_cast<f32x4 *>(new_state + sbase + vc * kDK + kr) = S[mi];
  }
}


// ---------------------------------------------------------------------------
// 3. state recurrence: per (sequence s, v-head h, 16 columns of V), unit
// h + H.v * (vb + 8 s): with 8 v-heads every unit of one head lands on the
// same XCD (workgroups are dealt round-robin over the 8 XCDs, and the grid is
// a multiple of 8), so the per-head operands stream through one L2.  The state tile
// S[:, v0:v0+16] ([K=128] x [16], f32) lives in MFMA accumulators.  The form
// is `form` (0 WY, 1 T) or, when form < 0, the index kernel's flag.
//
// What bounds a step (MI355X counters): the bytes each workgroup streams in
// per chunk (WY ~52 KB: w, K^T, u; T ~35 KB: K, T, V), from L2 at 400-750
// cycles latency with a bounded number of misses in flight per CU, and the
// serial chain of exchanges (two in the WY form, three in the T form).
//
// Two-segment scan (one sequence, WY form, sp.nt0 > 0).  Each chunk maps the
// state affinely, S -> S M_c + C_c, so the chunks [nt0, nt) need not wait for
// the state at nt0: beside the chain over [0, nt0) (from the initial state,
// ending in sp.send), the chunks [nt0, nt) run from a zero state (their ht
// and v_new are then the offsets; the end is sp.cend) and from the identity
// (MAP: the linear parts M into sp.htm; the end is sp.mend).  The three
// groups of 8 workgroups per head run side by side, s = 0, 1, 2 below, so the
// serial chain is half as long; prefill_output_split_kernel (the second
// segment's output, split_out_unit, and the new_state tiles) combines them.
// ---------------------------------------------------------------------------
struct SplitScan {
  int nt0;        // first chunk of the second segment; 0 = one chain
  uint16_t *htm;  // [nt - nt0][H.v][128 j][128 k] bf16
  float *send, *cend, *mend;  // [H.v][128][128] f32 each
  // early output of the first segment (8 v-heads; nullptr: none): [H.v][8]
  // progress words of the first segment's units, then [nt0][H.v] done flags
  int *early;
  int early_limit;  // chunks per early workgroup before it stops; 0 no limit
};

// One unit of the state kernel: sequence s, v-head h, V-block vb (unit =
// h + H.v (vb + 8 s)); `form` as settled for the batch (0 WY, 1 T).
__device__ __forceinline__ void state_unit(
    char *smem, int unit, const uint16_t *k, const uint16_t *v, const float *state,
    float *new_state, const int4 *chunks, const int *offsets, const float *ws_dcy,
    const float *ws_eg, const uint16_t *ws_w, const float *ws_u, const uint16_t *ws_kt,
    uint16_t *ws_ht, uint16_t *ws_vnt, int nt_max, const OneSeq &one, const Heads &H, int form,
    const SplitScan &sp) {
  constexpr int NVB = kDV / 16;
  const int h = unit % H.v;
  const int rest = unit / H.v;
  const int vb = rest % NVB, s = rest / NVB;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform, in SGPRs

  // This unit's chunks: c0 .. c0 + nch - 1 (prefetches clamped to npre
  // chunks, known at launch for one sequence); the tokens [bos, eos).
  int c0 = 0, nch = 0, npre = 0, bos = 0, eos = 0;
  int *prog = nullptr, prog_tag = 0;
  size_t sbase = (static_cast<size_t>(s) * H.v + h) * kDV * kDK;  // [V][K]
  if (one.cu != nullptr) {
    one_seq_bounds(one, bos, eos);
    nch = (eos - bos + kChunk - 1) / kChunk;
    npre = nt_max;
  } else {
    c0 = offsets[s];
    nch = offsets[s + 1] - c0 > 0 ? offsets[s + 1] - c0 : 0;
    npre = nch;
    if (form == 1 && nch > 0) {  // the T form's token range
      const int4 first = chunks[c0], last = chunks[c0 + nch - 1];
      bos = first.y;
      eos = last.y + last.z;
    }
  }
  if (sp.nt0 > 0) {  // two-segment scan of one sequence (WY form)
    sbase = static_cast<size_t>(h) * kDV * kDK;
    if (s == 2) {
      wy_state<true, false>(smem, sp.nt0, nch - sp.nt0, nt_max - sp.nt0, h, vb * 16, wave, lane, sbase,
                     nullptr, sp.mend, ws_dcy, ws_eg, ws_w, ws_u, ws_kt, sp.htm, ws_vnt, H, sp.nt0,
                     nullptr, 0);
      return;
    }
    if (s == 0) {
      nch = nch < sp.nt0 ? nch : sp.nt0;
      npre = sp.nt0;
      new_state = sp.send;
      if (sp.early != nullptr) {
        prog = sp.early + h * NVB + vb;
        prog_tag = early_tag();
      }
    } else {
      c0 = sp.nt0;
      nch -= sp.nt0;
      npre = nt_max - sp.nt0;
      state = nullptr;
      new_state = sp.cend;
    }
  }
  if (form == 1) {
    // the T form reads K and V itself: the sequence's tokens [bos, eos)
    t_state(smem, c0, nch, bos, eos, h, vb * 16, wave, lane, sbase, k, v, state, new_state, ws_dcy,
            ws_eg, ws_w, ws_u, ws_ht, ws_vnt, H);
  } else if (prog != nullptr) {
    wy_state<false, true>(smem, c0, nch, npre, h, vb * 16, wave, lane, sbase, state, new_state,
                          ws_dcy, ws_eg, ws_w, ws_u, ws_kt, ws_ht, ws_vnt, H, 0, prog, prog_tag);
  } else {
    wy_state<false, false>(smem, c0, nch, npre, h, vb * 16, wave, lane, sbase, state, new_state,
                           ws_dcy, ws_eg, ws_w, ws_u, ws_kt, ws_ht, ws_vnt, H, 0, nullptr, 0);
  }
}

__device__ __forceinline__ void early_output(char *smem, int e, int ne, const uint16_t *q,
                                             const uint16_t *k, const OneSeq &one, const Heads &H,
                                             const float *ws_G, const uint16_t *ws_ht,
                                             const uint16_t *ws_vnt, float scale, uint16_t *out,
                                             const SplitScan &sp);
constexpr int kStateLds0 = kStateWyLds > kStateTLds ? kStateWyLds : kStateTLds;
constexpr int kStateLds = kStateLds0 > kOutputLds + 16 ? kStateLds0 : kOutputLds + 16;

// The state launch of a two-segment scan with early output has kEarlyGrid
// more workgroups than units, after them (early_output).
template <bool LOOP>
__global__ __launch_bounds__(256) void prefill_state_kernel(
    const uint16_t *k, const uint16_t *v, const float *state, float *new_state,
    const int4 *chunks, const int *offsets, const float *ws_dcy, const float *ws_eg,
    const uint16_t *ws_w, const float *ws_u, const uint16_t *ws_kt, uint16_t *ws_ht,
    uint16_t *ws_vnt, int N, int nt_max, OneSeq one, Heads H, int form, SplitScan sp,
    const void *cu, int cu64, int T, uint16_t *out, const uint16_t *q, const float *ws_G,
    float scale) {
  __shared__ __align__(16) char smem[kStateLds];
  // (the bounds of the rows this batch covers are loaded now, used at the end)
  const CoveredRows rows = covered_rows(cu, cu64, N, T);
  if (one.cu == nullptr) {
    if (offsets[N + 1]) return;  // the sequential kernel owns the batch
    if (form < 0) form = offsets[N + 2];
  }
  const int units = (sp.nt0 > 0 ? 3 : N) * H.v * (kDV / 16);
  if (!LOOP) {
    if (static_cast<int>(blockIdx.x) < units)
      state_unit(smem, blockIdx.x, k, v, state, new_state, chunks, offsets, ws_dcy, ws_eg, ws_w,
                 ws_u, ws_kt, ws_ht, ws_vnt, nt_max, one, H, form, sp);
    else if (sp.early != nullptr)
      early_output(smem, blockIdx.x - units, gridDim.x - units, q, k, one, H, ws_G, ws_ht, ws_vnt,
                   scale, out, sp);
  } else {
    for (int unit = blockIdx.x; unit < units; unit += gridDim.x) {
      state_unit(smem, unit, k, v, state, new_state, chunks, offsets, ws_dcy, ws_eg, ws_w, ws_u,
                 ws_kt, ws_ht, ws_vnt, nt_max, one, H, form, sp);
      __syncthreads();  // the next unit reuses the LDS tiles
    }
  }
  // The chunk pipeline owns the batch: rows outside every sequence get zeros.
  zero_rows_outside(out, rows, T, H.v, blockIdx.x, gridDim.x);
}

// ---------------------------------------------------------------------------
// 3b. two-segment scan: the output of the second segment's chunks (units of
// prefill_output_split_kernel, after the state kernel).  With S0 = sp.send (the state at chunk nt0) and,
// for a chunk c >= nt0, M_c = sp.htm (the linear part of the map over chunks
// nt0..c-1, bf16 [j][k]) and C_c = ht (its offset, bf16 [v][k]), the
// chunk-start state is S_c = S0 M_c + C_c, and the second chain left
// v_off = u - w C_c^T in vnt.  The output
//   o = scale (E Q S_c^T + P v_new),  v_new = u - w S_c^T
// (E = diag exp(G_i), P = mask_{j<=i} exp(G_i - G_j) q_i . k_j) is linear in
// S_c, so it splits into the output of the offset chain and a correction
// that never forms S_c:
//   o = scale (E Q C_c^T + P v_off + R S0^T),  R = (E Q - P w) M_c^T
//                                                = E (Q M_c^T) - P (w M_c^T).
// Each workgroup produces the output of one chunk c >= nt0 and v-head h
// (c = nt0 + id / H.v, h = id % H.v, so a head's workgroups share an XCD and
// read S0 from its L2).  Wave w owns the output columns v and the columns j
// of R in 32 w .. 32 w + 31.  Operands in bf16 as in the output kernel (w and
// S0 rounded once); results in f32.  new_state = S0 M + C (M = sp.mend, C =
// sp.cend) is computed by extra workgroups of the output kernel's launch
// (split_state_tile), which runs beside this one's in the same round.
// ---------------------------------------------------------------------------
constexpr int kSplitOutLds = 2 * kChunk * kStrideK * 2 + kChunk * kDK * 2 + kChunk * kStrideT * 2 + kChunk * 4;
__device__ __forceinline__ void split_out_unit(
    uint16_t *smem, int id, const uint16_t *__restrict__ q, const uint16_t *__restrict__ k,
    const OneSeq &one, const Heads &H, const SplitScan &sp, const float *__restrict__ ws_G,
    const uint16_t *__restrict__ ws_w, const uint16_t *__restrict__ ws_ht,
    const uint16_t *__restrict__ ws_vnt, float scale, uint16_t *__restrict__ out) {
  constexpr size_t kElems = static_cast<size_t>(kDV) * kDK;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = sp.nt0 + id / H.v, h = id % H.v;
  int bos, eos;
  one_seq_bounds(one, bos, eos);
  const int start = bos + c * kChunk, rest = eos - start;
  if (rest <= 0) return;  // past the sequence's last chunk
  const int len = rest < kChunk ? rest : kChunk;
  const int hq = h / H.ratio;
  const size_t ch_head = static_cast<size_t>(c) * H.v + h;
  const int r16 = lane & 15, g = lane >> 4, kg = 8 * g, q4 = 4 * g;
  uint16_t *const sQ = smem;                    // [64][kStrideK]: Q, then R, then o
  uint16_t *const sK = sQ + kChunk * kStrideK;  // [64][kStrideK]
  uint16_t *const sW = sK + kChunk * kStrideK;  // w's hi fragments [jb][kk][lane][8]
  uint16_t *const sP = sW + kChunk * kDK;       // [64][kStrideT]
  float *const sG = reinterpret_cast<float *>(sP + kChunk * kStrideT);
  const float *const S0 = sp.send + static_cast<size_t>(h) * kElems;
  const uint16_t *const Mc = sp.htm + (static_cast<size_t>(c - sp.nt0) * H.v + h) * kElems;
  const uint16_t *const Cc = ws_ht + ch_head * kElems;
  const uint16_t *const Vo = ws_vnt + ch_head * (kDV * kChunk);
  const uint16_t *const wsrc = ws_w + ch_head * (kWBytes / 2);

  // --- Every global load is issued here, so that one memory latency covers
  // them all: Q and K rows (rows past the chunk read zero through the
  // descriptors' range), G and the hi plane of w's stored fragments
  // [hi | lo][jb][kk][lane][8] (A operands of w M^T, all 64 rows) -> LDS;
  // the S0 rows of this wave's columns n = 32 wave + 16 nt + r16 (B operands
  // of R S0^T) into registers.
  const uint32_t rstride = static_cast<uint32_t>(H.qk) * (kDK * 2);
  const size_t qk0 = (static_cast<size_t>(start) * H.qk + hq) * kDK;
  {
    const auto rq = buf_rsrc(q + qk0, static_cast<uint32_t>(len) * rstride);
    const auto rk = buf_rsrc(k + qk0, static_cast<uint32_t>(len) * rstride);
    u32x4 qv[4], kv[4], wv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = tid + 256 * i;
      const uint32_t off = static_cast<uint32_t>(idx >> 4) * rstride + (idx & 15) * 16;
      qv[i] = buf_load16(rq, off);
      kv[i] = buf_load16(rk, off);
      wv[i] = *reinterpret_cast<const u32x4 *>(wsrc + idx * 8);  // the hi plane
    }
    if (tid < kChunk) sG[tid] = ws_G[ch_head * kChunk + tid];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = tid + 256 * i;
      *reinterpret_cast<u32x4 *>(&sQ[(idx >> 4) * kStrideK + (idx & 15) * 8]) = qv[i];
      *reinterpret_cast<u32x4 *>(&sK[(idx >> 4) * kStrideK + (idx & 15) * 8]) = kv[i];
      *reinterpret_cast<u32x4 *>(&sW[idx * 8]) = wv[i];
    }
  }
  f32x4 s0r[2][4][2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int n = 32 * wave + 16 * nt + r16;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      s0r[nt][kk][0] = *reinterpret_cast<const f32x4 *>(S0 + n * kDK + 32 * kk + kg);
      s0r[nt][kk][1] = *reinterpret_cast<const f32x4 *>(S0 + n * kDK + 32 * kk + kg + 4);
    }
  }
  __syncthreads();

  // --- P rows 16 wave .. +15 -> LDS (as the output kernel).
  {
    const int mb = wave;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      if (nb <= mb) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const u32x4 af = *reinterpret_cast<const u32x4 *>(&sQ[(16 * mb + r16) * kStrideK + 32 * kk + kg]);
          const u32x4 bf = *reinterpret_cast<const u32x4 *>(&sK[(16 * nb + r16) * kStrideK + 32 * kk + kg]);
          acc = mfma_bf16(af, bf, acc);
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * mb + q4 + r, j = 16 * nb + r16;
        const float p = (j <= i && i < len) ? expf(sG[i] - sG[j]) * acc[r] : 0.f;
        sP[i * kStrideT + j] = f32_to_bf16(p);
      }
    }
  }
  // S0 as bf16 B operands; then the B operands of this wave's columns: C_c
  // rows (E Q C^T), M_c rows (Q M^T, w M^T) and v_off rows (P v_off), loaded
  // before the barrier so that their latency overlaps it.
  u32x4 sb[2][4];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt)
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const f32x4 x0 = s0r[nt][kk][0], x1 = s0r[nt][kk][1];
      sb[nt][kk] = u32x4{pk_bf16(x0[0], x0[1]), pk_bf16(x0[2], x0[3]), pk_bf16(x1[0], x1[1]),
                         pk_bf16(x1[2], x1[3])};
    }
  u32x4 cb[2][4], mb4[2][4], vb[2][2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int n = 32 * wave + 16 * nt + r16;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      cb[nt][kk] = *reinterpret_cast<const u32x4 *>(Cc + n * kDK + 32 * kk + kg);
      mb4[nt][kk] = *reinterpret_cast<const u32x4 *>(Mc + n * kDK + 32 * kk + kg);
    }
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) vb[nt][kk] = *reinterpret_cast<const u32x4 *>(Vo + n * kChunk + 32 * kk + kg);
  }
  __syncthreads();

  // --- O = E Q C^T + P v_off, then Y = E Q M^T (rows: all 64 tokens; two
  // passes over the Q tile keep fewer operands live).
  f32x4 O[4][2], Y[4][2];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) O[mb][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const u32x4 qa = *reinterpret_cast<const u32x4 *>(&sQ[(16 * mb + r16) * kStrideK + 32 * kk + kg]);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) O[mb][nt] = mfma_bf16(qa, cb[nt][kk], O[mb][nt]);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float e = expf(sG[16 * mb + q4 + r]);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) O[mb][nt][r] *= e;
    }
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const u32x4 pa = *reinterpret_cast<const u32x4 *>(&sP[(16 * mb + r16) * kStrideT + 32 * kk + kg]);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) O[mb][nt] = mfma_bf16(pa, vb[nt][kk], O[mb][nt]);
    }
  }
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) Y[mb][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const u32x4 qa = *reinterpret_cast<const u32x4 *>(&sQ[(16 * mb + r16) * kStrideK + 32 * kk + kg]);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) Y[mb][nt] = mfma_bf16(qa, mb4[nt][kk], Y[mb][nt]);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float e = expf(sG[16 * mb + q4 + r]);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) Y[mb][nt][r] *= e;
    }
  }

  // --- Z = w M^T (rows: all 64 tokens j; A = the hi halves of w's stored
  // fragments [jb][kk][lane][hi 8 | lo 8]), then R = Y - P Z: Z's 16x16
  // result tiles (4 consecutive j per lane) are the B operands of 16x16x16
  // MFMAs as they stand.
#pragma unroll
  for (int jb = 0; jb < 4; ++jb) {
    f32x4 Z[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const u32x4 wa = *reinterpret_cast<const u32x4 *>(&sW[((jb * 4 + kk) * 64 + lane) * 8]);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) Z[nt] = mfma_bf16(wa, mb4[nt][kk], Z[nt]);
    }
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const u32x2 zb = {pk_bf16(Z[nt][0], Z[nt][1]), pk_bf16(Z[nt][2], Z[nt][3])};
      // rows i of blocks mb >= jb see the columns j of block jb
#pragma unroll
      for (int mb = jb; mb < 4; ++mb) {
        const u32x2 pa = *reinterpret_cast<const u32x2 *>(&sP[(16 * mb + r16) * kStrideT + 16 * jb + q4]);
        f32x4 pz = mfma16_bf16(pa, zb, f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int r = 0; r < 4; ++r) Y[mb][nt][r] -= pz[r];
      }
    }
  }
  __syncthreads();  // every wave is done with the Q tile: R takes its place

  uint16_t *const sR = sQ;  // [64][kStrideK]: R[i][j]
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        sR[(16 * mb + q4 + r) * kStrideK + 32 * wave + 16 * nt + r16] = f32_to_bf16(Y[mb][nt][r]);
  __syncthreads();

  // --- O += R S0^T.
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const u32x4 ra = *reinterpret_cast<const u32x4 *>(&sR[(16 * mb + r16) * kStrideK + 32 * kk + kg]);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) O[mb][nt] = mfma_bf16(ra, sb[nt][kk], O[mb][nt]);
    }
  __syncthreads();  // every wave is done with R: o takes its place

  uint16_t *const sO = sQ;  // [64][kStrideK]
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        sO[(16 * mb + q4 + r) * kStrideK + 32 * wave + 16 * nt + r16] = f32_to_bf16(scale * O[mb][nt][r]);
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = tid + 256 * i, row = idx >> 4, c8 = (idx & 15) * 8;
    if (row < len)
      *reinterpret_cast<u32x4 *>(out + ((static_cast<size_t>(start) + row) * H.v + h) * kDV + c8) =
          *reinterpret_cast<const u32x4 *>(&sO[row * kStrideK + c8]);
  }
}

// new_state tile of a two-segment scan: rows 16 rb .. +15, columns 32 cb ..
// +31 of head h, new_state = S0 M + C in f32 FMAs, with S0's rows and M's
// columns staged in LDS (24 KB of the output kernel's 27 KB).  Thread t owns
// column 32 cb + (t & 31) of rows 16 rb + (t >> 5) and 16 rb + (t >> 5) + 8.
__device__ __forceinline__ void split_state_tile(char *smem, int f, const Heads &H,
                                                 const SplitScan &sp, float *new_state) {
  constexpr size_t kElems = static_cast<size_t>(kDV) * kDK;
  const int tid = threadIdx.x;
  const int h = f % H.v, t = f / H.v, rb = t / (kDK / 32), cb = t % (kDK / 32);
  float *sS0 = reinterpret_cast<float *>(smem);  // [16][128]
  float *sMc = sS0 + 16 * kDK;                   // [128][32]
  const float *S0 = sp.send + h * kElems + static_cast<size_t>(16 * rb) * kDK;
  const float *M = sp.mend + h * kElems + 32 * cb;
  f32x4 sv[2], mv[4];
#pragma unroll
  for (int i = 0; i < 2; ++i) sv[i] = reinterpret_cast<const f32x4 *>(S0)[tid + 256 * i];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = tid + 256 * i;
    mv[i] = *reinterpret_cast<const f32x4 *>(M + (idx >> 3) * kDK + 4 * (idx & 7));
  }
  const int col = tid & 31, r0 = tid >> 5;
  const size_t o0 = h * kElems + static_cast<size_t>(16 * rb + r0) * kDK + 32 * cb + col;
  float acc0 = sp.cend[o0], acc1 = sp.cend[o0 + 8 * kDK];
#pragma unroll
  for (int i = 0; i < 2; ++i) reinterpret_cast<f32x4 *>(sS0)[tid + 256 * i] = sv[i];
#pragma unroll
  for (int i = 0; i < 4; ++i) reinterpret_cast<f32x4 *>(sMc)[tid + 256 * i] = mv[i];
  __syncthreads();
#pragma unroll 4
  for (int j = 0; j < kDK; j += 4) {
    const f32x4 a = *reinterpret_cast<const f32x4 *>(&sS0[r0 * kDK + j]);
    const f32x4 b = *reinterpret_cast<const f32x4 *>(&sS0[(r0 + 8) * kDK + j]);
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const float m = sMc[(j + jj) * 32 + col];
      acc0 = fmaf(a[jj], m, acc0);
      acc1 = fmaf(b[jj], m, acc1);
    }
  }
  new_state[o0] = acc0;
  new_state[o0 + 8 * kDK] = acc1;
}

// ---------------------------------------------------------------------------
// 4. chunk output: per (chunk c, v-head h) = chunk_head_of(blockIdx.x).
//   P  = mask_{j<=i} exp(G_i - G_j) Q K^T      (waves split the rows)
//   O  = exp(G_i) Q S_c + P v_new              (waves split the columns)
// ---------------------------------------------------------------------------
// ready(): (early output) called by every thread once the inputs' part is
// done and before ht / v_new are read; false: stop without output.  Returns
// false only then.
struct AlwaysReady {
  __device__ bool operator()() const { return true; }
};
template <typename Ready = AlwaysReady>
__device__ __forceinline__ bool output_chunk(
    char *osmem, int c, int h, const uint16_t *__restrict__ q, const uint16_t *__restrict__ k,
    const int4 *__restrict__ chunks, const OneSeq &one, const Heads &H,
    const float *__restrict__ ws_G, const uint16_t *__restrict__ ws_ht, const uint16_t *__restrict__ ws_vnt, float scale,
    uint16_t *__restrict__ out, Ready ready = Ready{}) {
  uint16_t *const sQ = reinterpret_cast<uint16_t *>(osmem);  // [64][kStrideK]
  uint16_t *const sP = sQ + kChunk * kStrideK;                // [64][kStrideT]
  float *const sG = reinterpret_cast<float *>(sP + kChunk * kStrideT);
  const int4 ch = chunk_info(chunks, c, one);
  if (ch.x < 0) return true;
  const int start = ch.y, len = ch.z;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, kg = (lane >> 4) * 8, q4 = 4 * (lane >> 4);
  const int hq = h / H.ratio;
  const size_t ch_head = static_cast<size_t>(c) * H.v + h;

  // K rows as B operands of Q K^T straight from the input (16 contiguous
  // bytes per lane; rows past the chunk read zero through the descriptor's
  // range): wave w needs the rows of key blocks 0..w.
  const auto rk = buf_rsrc(k + (static_cast<size_t>(start) * H.qk + hq) * kDK,
                           static_cast<uint32_t>(len) * static_cast<uint32_t>(H.qk) * (kDK * 2));
  u32x4 kb[4][4];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      kb[nb][kk] = nb <= wave ? buf_load16(rk, (static_cast<uint32_t>(16 * nb + r16) * H.qk * kDK +
                                                32 * kk + kg) * 2)
                              : u32x4{0u, 0u, 0u, 0u};

  if (tid < kChunk) sG[tid] = ws_G[ch_head * kChunk + tid];
  {
    // Q rows (zero past the chunk through the descriptor's range), every load
    // issued before the LDS stores.
    const uint32_t rstride = static_cast<uint32_t>(H.qk) * (kDK * 2);
    const auto rq = buf_rsrc(q + (static_cast<size_t>(start) * H.qk + hq) * kDK,
                             static_cast<uint32_t>(len) * rstride);
    u32x4 qv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = tid + 256 * i;
      qv[i] = buf_load16(rq, static_cast<uint32_t>(idx >> 4) * rstride + (idx & 15) * 16);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = tid + 256 * i;
      *reinterpret_cast<u32x4 *>(&sQ[(idx >> 4) * kStrideK + (idx & 15) * 8]) = qv[i];
    }
  }
  __syncthreads();

  {
    const int mb = wave;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      if (nb <= mb) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const u32x4 af = *reinterpret_cast<const u32x4 *>(&sQ[(16 * mb + r16) * kStrideK + 32 * kk + kg]);
          acc = mfma_bf16(af, kb[nb][kk], acc);
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * mb + q4 + r, j = 16 * nb + r16;
        const float p = (j <= i && i < len) ? expf(sG[i] - sG[j]) * acc[r] : 0.f;
        sP[i * kStrideT + j] = f32_to_bf16(p);
      }
    }
  }
  if (!ready()) return false;
  // The chunk-start state and v_new fragments of this wave's columns, loaded
  // before the barrier (the K fragments are dead): their latency overlaps it.
  u32x4 hbf[2][4], vbf[2][2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int n = 16 * (2 * wave + nt) + r16;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      hbf[nt][kk] = *reinterpret_cast<const u32x4 *>(ws_ht + (ch_head * kDV + n) * kDK + 32 * kk + kg);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
      vbf[nt][kk] = *reinterpret_cast<const u32x4 *>(ws_vnt + (ch_head * kDV + n) * kChunk + 32 * kk + kg);
  }
  __syncthreads();

  f32x4 O[4][2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) O[mb][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const u32x4 qa = *reinterpret_cast<const u32x4 *>(&sQ[(16 * mb + r16) * kStrideK + 32 * kk + kg]);
        O[mb][nt] = mfma_bf16(qa, hbf[nt][kk], O[mb][nt]);
      }
    }
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r) O[mb][nt][r] *= expf(sG[16 * mb + q4 + r]);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const u32x4 pa = *reinterpret_cast<const u32x4 *>(&sP[(16 * mb + r16) * kStrideT + 32 * kk + kg]);
        O[mb][nt] = mfma_bf16(pa, vbf[nt][kk], O[mb][nt]);
      }
    }
  }
  // o = scale * O through LDS (the Q tile's space), so that every global
  // store is 16 contiguous bytes of one token row.
  __syncthreads();
  uint16_t *sO = sQ;  // [64][kStrideK]
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int n = 16 * (2 * wave + nt) + r16;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r) sO[(16 * mb + q4 + r) * kStrideK + n] = f32_to_bf16(scale * O[mb][nt][r]);
  }
  __syncthreads();
  for (int idx = tid; idx < kChunk * 16; idx += 256) {
    const int row = idx >> 4, c8 = (idx & 15) * 8;
    if (row < len)
      *reinterpret_cast<u32x4 *>(out + ((static_cast<size_t>(start) + row) * H.v + h) * kDV + c8) =
          *reinterpret_cast<const u32x4 *>(&sO[row * kStrideK + c8]);
  }
  return true;
}

// One workgroup of an output launch: a new_state tile of a two-segment scan
// (the first kStateTiles H.v ids), else (chunk, v-head) = chunk_head_of(id).
__device__ __forceinline__ void output_unit(
    char *osmem, int id, const uint16_t *__restrict__ q, const uint16_t *__restrict__ k,
    const int4 *__restrict__ chunks, const OneSeq &one, int nt_max, const Heads &H,
    const float *__restrict__ ws_G, const uint16_t *__restrict__ ws_ht, const uint16_t *__restrict__ ws_vnt, float scale,
    uint16_t *__restrict__ out, const SplitScan &sp, float *__restrict__ new_state) {
  static_assert(16 * kDK * 4 + kDK * 32 * 4 <= kOutputLds, "new_state tile must fit");
  const int nfix = sp.nt0 > 0 ? kStateTiles * H.v : 0;
  if (id < nfix) {
    split_state_tile(osmem, id, H, sp, new_state);
    return;
  }
  int c, h;
  if (!chunk_head_of(id - nfix, nt_max, H, c, h)) return;
  output_chunk(osmem, c, h, q, k, chunks, one, H, ws_G, ws_ht, ws_vnt, scale, out);
}

// Early output of a two-segment scan (SplitScan::early): workgroup e of the
// ne added to the state launch computes, for v-head h = e % 8, the output of
// the first segment's chunks c = e / 8, e / 8 + ne / 8, ... below the
// segment's last kEarlyTail chunks, each as soon as the head's 8 first-
// segment units have published it, and marks the chunk done for the output
// launch.  Workgroups are dealt round-robin over the 8 XCDs, so the head's
// state units (blockIdx.x = h + 8 (vb + 8 s)) and its early workgroups
// (blockIdx.x = 192 + e with e % 8 = h) share an XCD and its L2.  A progress
// word holds the publishing unit's XCD (early_tag) above its chunk count, and
// is read past L1 (an agent-scope load): a word of the reader's XCD comes
// from the shared L2, where the unit's ht and v_new stores already are; a
// word of another XCD, which could only arrive through a write-back ahead of
// its data, stops the workgroup.  So does a wait of kEarlyPatience ticks of
// the 100 MHz wall clock without progress.  The output launch computes every
// chunk not marked done.
constexpr long long kEarlyPatience = 5000;  // 50 us
struct EarlyWait {  // the early output's wait for chunk c (see early_output)
  const int *prog;
  int *s_go;
  int c, me;
  int *seen;
  long long *t_seen;
  __device__ bool operator()() const {
    constexpr int NVB = kDV / 16;
    constexpr int kCount = (1 << 24) - 1;
    if (threadIdx.x < 64) {
      const int lane = threadIdx.x;
      int go = 1;
      for (;;) {
        const int w = lane < NVB ? __hip_atomic_load(prog + lane, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT)
                                 : me | kCount;
        if (__ballot(w != 0 && (w & ~kCount) != me) != 0) {
          go = 0;  // published from another XCD
          break;
        }
        int m = w & kCount;  // 0 while unpublished
        m = min(m, __shfl_xor(m, 4));
        m = min(m, __shfl_xor(m, 2));
        m = min(m, __shfl_xor(m, 1));
        m = __shfl(m, 0);
        if (m > c) break;
        const long long t = wall_clock64();
        if (m > *seen) {
          *seen = m;
          *t_seen = t;
        } else if (t - *t_seen > kEarlyPatience) {
          go = 0;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
      if (threadIdx.x == 0) *s_go = go;
    }
    __syncthreads();
    return *s_go != 0;
  }
};
__device__ __forceinline__ void early_output(char *smem, int e, int ne, const uint16_t *q,
                                             const uint16_t *k, const OneSeq &one, const Heads &H,
                                             const float *ws_G, const uint16_t *ws_ht,
                                             const uint16_t *ws_vnt, float scale, uint16_t *out,
                                             const SplitScan &sp) {
  constexpr int NVB = kDV / 16;
  const int h = e % H.v, step = ne / H.v;
  int bos, eos;
  one_seq_bounds(one, bos, eos);
  const int nch = (eos - bos + kChunk - 1) / kChunk;
  const int n1 = nch < sp.nt0 ? nch : sp.nt0;
  int *const done = sp.early + H.v * NVB;
  int seen = 0;  // the head's least published count so far, and when it last grew
  long long t_seen = wall_clock64();
  for (int c = e / H.v, n = 0; c < n1 - kEarlyTail; c += step, ++n) {
    if (n == sp.early_limit && n > 0) return;
    // the chunk's q, k and gates are read, and P formed, before the wait:
    // only ht and v_new need the chain
    const EarlyWait ready{sp.early + h * NVB, reinterpret_cast<int *>(smem + kOutputLds), c,
                          early_tag(), &seen, &t_seen};
    if (!output_chunk(smem, c, h, q, k, nullptr, one, H, ws_G, ws_ht, ws_vnt, scale, out, ready))
      return;
    __syncthreads();  // the chunk's LDS reads are done before the next one's writes
    if (threadIdx.x == 0) done[c * H.v + h] = 1;
  }
}

// The first segment's chunks that the early output leaves to the output
// launch (SplitScan::early): workgroup (j, h) = (r / 8, r % 8) computes chunk
// n1 - kEarlyTail + j of v-head h (n1: the segment's chunks of this
// sequence), then every chunk c = j + kEarlyTail i below n1 - kEarlyTail
// whose done flag the state launch did not set (none, unless an early
// workgroup stopped).
__device__ __forceinline__ void early_rest(char *smem, int r, const uint16_t *q, const uint16_t *k,
                                           const OneSeq &one, const Heads &H, const float *ws_G,
                                           const uint16_t *ws_ht, const uint16_t *ws_vnt,
                                           float scale, uint16_t *out, const SplitScan &sp) {
  const int h = r % H.v, j = r / H.v;
  int bos, eos;
  one_seq_bounds(one, bos, eos);
  const int nch = (eos - bos + kChunk - 1) / kChunk;
  const int n1 = nch < sp.nt0 ? nch : sp.nt0, first = n1 - kEarlyTail;
  const int *const done = sp.early + H.v * (kDV / 16);
  unsigned *const s_todo = reinterpret_cast<unsigned *>(smem + kOutputLds);
  if (first + j >= 0)
    output_chunk(smem, first + j, h, q, k, nullptr, one, H, ws_G, ws_ht, ws_vnt, scale, out);
  for (int cb = j; cb < first; cb += 64 * kEarlyTail) {
    __syncthreads();  // the LDS of the chunk before is free
    if (threadIdx.x < 64) {
      const int c = cb + kEarlyTail * static_cast<int>(threadIdx.x);
      const unsigned long long m = __ballot(c < first && done[c * H.v + h] == 0);
      if (threadIdx.x == 0) {
        s_todo[0] = static_cast<unsigned>(m);
        s_todo[1] = static_cast<unsigned>(m >> 32);
      }
    }
    __syncthreads();
    unsigned long long m = (static_cast<unsigned long long>(s_todo[1]) << 32) | s_todo[0];
    while (m != 0) {
      const int i = __builtin_ctzll(m);
      m &= m - 1;
      __syncthreads();
      output_chunk(smem, cb + kEarlyTail * i, h, q, k, nullptr, one, H, ws_G, ws_ht, ws_vnt, scale,
                   out);
    }
  }
}

// 27 KB of LDS and at most 128 VGPRs: four workgroups per CU.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4)))
void prefill_output_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ k,
    const int4 *__restrict__ chunks, OneSeq one, int nt_max, Heads H,
    const float *__restrict__ ws_G, const uint16_t *__restrict__ ws_ht, const uint16_t *__restrict__ ws_vnt, float scale,
    uint16_t *__restrict__ out, SplitScan sp, float *__restrict__ new_state) {
  __shared__ __align__(16) char osmem[kOutputLds];
  output_unit(osmem, blockIdx.x, q, k, chunks, one, nt_max, H, ws_G, ws_ht, ws_vnt, scale, out, sp,
              new_state);
}

// After a two-segment scan: the first segment's output and the new_state
// tiles (ids below out_units, as prefill_output_kernel) and the second
// segment's (split_out_unit) in one launch, the short units first, so that
// the two run side by side instead of one after the other (1x8192: 30.0 us
// against 19.5 + 12.6 us as two launches).
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void prefill_output_split_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ k, OneSeq one, int out_chunks,
    Heads H, const float *__restrict__ ws_G, const uint16_t *__restrict__ ws_w,
    const uint16_t *__restrict__ ws_ht, const uint16_t *__restrict__ ws_vnt, float scale,
    uint16_t *__restrict__ out, SplitScan sp, float *__restrict__ new_state, int out_units) {
  static_assert(kOutputLds <= kSplitOutLds, "the output unit fits the split unit's LDS");
  __shared__ __align__(16) uint16_t smem[kSplitOutLds / 2];
  const int id = blockIdx.x, nfix = kStateTiles * H.v;
  if (sp.early != nullptr && id >= nfix && id < out_units)
    early_rest(reinterpret_cast<char *>(smem), id - nfix, q, k, one, H, ws_G, ws_ht, ws_vnt, scale,
               out, sp);
  else if (id < out_units)
    output_unit(reinterpret_cast<char *>(smem), id, q, k, nullptr, one, out_chunks, H, ws_G, ws_ht,
                ws_vnt, scale, out, sp, new_state);
  else
    split_out_unit(smem, id - out_units, q, k, one, H, sp, ws_G, ws_w, ws_ht, ws_vnt, scale, out);
}

// The output of a batch without sequences (N == 0): every row is zero.
__global__ __launch_bounds__(256) void prefill_zero_kernel(uint16_t *out, const void *cu, int cu64,
                                                           int T, int hv) {
  zero_uncovered_rows(out, cu, cu64, 0, T, hv, blockIdx.x, gridDim.x);
}

// The contract bits of one sequence whose call launches no intra kernel (no
// tokens: the intra kernel otherwise writes them).
__global__ __launch_bounds__(64) void prefill_status_kernel(const void *cu, int cu64, int T,
                                                          int *status) {
  if (threadIdx.x == 0) status[0] = cu_status_bits(raw_cu(cu, cu64, 0), raw_cu(cu, cu64, 1), T);
}

static int prefill_launch(const gdn_bf16 *q, const gdn_bf16 *k, const gdn_bf16 *v,
                          const float *state, const float *A_log, const gdn_bf16 *a,
                          const float *dt_bias, const gdn_bf16 *b, const void *cu_seqlens,
                          int cu64, int N, int T, float scale, gdn_bf16 *output, float *new_state,
                          void *workspace, size_t ws_bytes, void *stream_ptr, int variant,
                          int rec_max, int rec_variant, int hqk, int hv, const char *what) {
  clear_error();
  Heads H;
  if (int rc = make_heads(hqk, hv, what, H)) return rc;
  PrefillLayout L;
  if (int rc = check_prefill_args(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, cu64, N, T,
                                  scale, output, new_state, workspace, ws_bytes, variant, rec_max,
                                  rec_variant, recurrent_num_variants(), H, what, &L))
    return rc;
  if (N == 0 && T == 0) return GDN_OK;
  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  if (N == 0) {  // no sequence: every output row is zero
    const size_t units = static_cast<size_t>(T) * H.v * (kDV / 8);
    const unsigned grid = static_cast<unsigned>(units / 256 + 1 < 1024 ? units / 256 + 1 : 1024);
    hipLaunchKernelGGL(prefill_zero_kernel, dim3(grid), dim3(256), 0, stream, output, cu_seqlens,
                       cu64, T, H.v);
    return check_launch(what);
  }
  PrefillPlan P;
  if (int rc = plan_prefill(T, N, H, L, variant, rec_max, rec_variant, recurrent_block_variant(),
                            what, P))
    return rc;
  // The whole batch through one sequential kernel (token by token, or in
  // 16-token blocks), decided on the host.
  char *ws = static_cast<char *>(workspace);
  int *status = reinterpret_cast<int *>(ws + L.status);
  if (P.sequential)
    return recurrent_launch(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, cu64, N, T, 0,
                            nullptr, status, H, scale, output, new_state, stream, P.seq_variant,
                            what);

  int4 *chunks = reinterpret_cast<int4 *>(ws + L.chunks);
  int *offsets = reinterpret_cast<int *>(ws + L.offsets);
  float *wsG = reinterpret_cast<float *>(ws + L.G);
  float *wsD = reinterpret_cast<float *>(ws + L.dcy);
  float *wsE = reinterpret_cast<float *>(ws + L.eg);
  uint16_t *wsw = reinterpret_cast<uint16_t *>(ws + L.w);
  float *wsu = reinterpret_cast<float *>(ws + L.u);
  uint16_t *kt = reinterpret_cast<uint16_t *>(ws + L.kt);
  uint16_t *ht = reinterpret_cast<uint16_t *>(ws + L.ht);
  uint16_t *vnt = reinterpret_cast<uint16_t *>(ws + L.vnt);
  const OneSeq one{P.single ? cu_seqlens : nullptr, cu64, T};
  int rc = GDN_OK;
  // Several sequences: the index kernel builds the chunk table and, when the
  // plan leaves it to the device (P.choose != 0), sets the path flag read by
  // the sequential and state kernels (the chunk table is then empty) -- or,
  // for at most kSelfIndexMax sequences, the intra kernel does it itself
  // (P.self_index), launched first.
  if (!P.single && !P.self_index) {
    hipLaunchKernelGGL(prefill_index_kernel, dim3(1), dim3(1024), 0, stream, cu_seqlens, cu64, N, T,
                       L.nt_max, P.choose, rec_max, H.v, P.form, chunks, offsets, status);
    if ((rc = check_launch(what))) return rc;
  }
  auto sequential_kernel = [&]() {
    return recurrent_launch(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, cu64, N, T, 0,
                            offsets + N + 1, nullptr, H, scale, output, new_state, stream,
                            P.seq_variant, what);
  };
  if (P.choose != 0 && !P.self_index) {
    if ((rc = sequential_kernel())) return rc;
  }
  // two-segment scan with early output: its words, zeroed by the intra launch
  int *early = P.early_grid > 0 ? reinterpret_cast<int *>(ws + L.early) : nullptr;
  if (P.intra_grid > 0) {
    const int *flag = offsets + N + 2;  // read only when the device picks the form
    const SelfIndex si{P.self_index ? cu_seqlens : nullptr, cu64, N, T, P.choose, rec_max, P.form,
                       chunks, offsets, status, early,
                       static_cast<int>(early_words(P.split_nt0, H.v))};
    auto intra = P.intra_split ? prefill_intra_kernel<0, true>
                 : P.form == 0 ? prefill_intra_kernel<0, false>
                 : P.form == 1 ? prefill_intra_kernel<1, false>
                               : prefill_intra_either_kernel;
    hipLaunchKernelGGL(intra, dim3(static_cast<unsigned>(P.intra_grid)), dim3(256), 0, stream, k,
                       v, A_log, a, dt_bias, b, chunks, one, L.nt_max, H, flag, si, wsG, wsD, wsE,
                       wsw, wsu, kt);
    if ((rc = check_launch(what))) return rc;
  }
  if (P.choose != 0 && P.self_index) {
    if ((rc = sequential_kernel())) return rc;
  }
  if (P.single && P.intra_grid == 0) {
    hipLaunchKernelGGL(prefill_status_kernel, dim3(1), dim3(64), 0, stream, cu_seqlens, cu64, T,
                       status);
    if ((rc = check_launch(what))) return rc;
  }
  SplitScan sp{P.split_nt0, nullptr, nullptr, nullptr, nullptr, nullptr, P.early_limit};
  if (sp.nt0 > 0) {
    sp.htm = reinterpret_cast<uint16_t *>(ws + L.htm);
    sp.send = reinterpret_cast<float *>(ws + L.send);
    sp.cend = reinterpret_cast<float *>(ws + L.cend);
    sp.mend = reinterpret_cast<float *>(ws + L.mend);
    sp.early = early;
  }
  hipLaunchKernelGGL(P.loop ? prefill_state_kernel<true> : prefill_state_kernel<false>,
                     dim3(static_cast<unsigned>(P.state_grid + P.early_grid)), dim3(256), 0,
                     stream, k, v, state, new_state, chunks, offsets, wsD, wsE, wsw, wsu, kt, ht,
                     vnt, N, L.nt_max, one, H, P.form, sp, cu_seqlens, cu64, T, output, q, wsG,
                     scale);
  if ((rc = check_launch(what))) return rc;
  if (P.split_grid > 0) {
    // the first segment's output and new_state (the output kernel's units),
    // then the second segment's output, in one launch
    hipLaunchKernelGGL(prefill_output_split_kernel,
                       dim3(static_cast<unsigned>(P.out_grid + P.split_grid)), dim3(256), 0, stream,
                       q, k, one, sp.nt0, H, wsG, wsw, ht, vnt, scale, output, sp, new_state,
                       static_cast<int>(P.out_grid));
    return check_launch(what);
  }
  if (P.out_grid > 0) {
    // with the two-segment scan, the output kernel covers the first segment
    // and new_state (extra workgroups first in its grid)
    const int out_chunks = sp.nt0 > 0 ? sp.nt0 : L.nt_max;
    hipLaunchKernelGGL(prefill_output_kernel, dim3(static_cast<unsigned>(P.out_grid)), dim3(256), 0,
                       stream, q, k, chunks, one, out_chunks, H, wsG, ht, vnt, scale, output, sp,
                       new_state);
    if ((rc = check_launch(what))) return rc;
  }
  return GDN_OK;
}

}  // namespace gdn

extern "C" size_t gdn_prefill_workspace_bytes(int total_tokens, int num_seqs) {
  return gdn_prefill_workspace_bytes_heads(total_tokens, num_seqs, gdn::kHQK, gdn::kHV);
}

extern "C" size_t gdn_prefill_workspace_bytes_heads(int total_tokens, int num_seqs,
                                                    int num_qk_heads, int num_v_heads) {
  if (total_tokens < 0 || num_seqs < 0 || num_qk_heads < 1 || num_v_heads < 1 ||
      num_v_heads > gdn::kMaxHeads || num_v_heads % num_qk_heads != 0)
    return 0;
  const gdn::Heads H{num_qk_heads, num_v_heads, num_v_heads / num_qk_heads};
  return gdn::prefill_layout(total_tokens, num_seqs, H).total;
}

extern "C" int gdn_prefill_fwd(const gdn_bf16 *q, const gdn_bf16 *k, const gdn_bf16 *v,
                               const float *state, const float *A_log, const gdn_bf16 *a,
                               const float *dt_bias, const gdn_bf16 *b, const void *cu_seqlens,
                               int cu_seqlens_is_int64, int num_seqs, int total_tokens, float scale,
                               gdn_bf16 *output, float *new_state, void *workspace,
                               size_t workspace_bytes, void *stream) {
  return gdn::prefill_launch(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, cu_seqlens_is_int64,
                             num_seqs, total_tokens, scale, output, new_state, workspace,
                             workspace_bytes, stream, -1, -1, -1, gdn::kHQK, gdn::kHV,
                             "gdn_prefill_fwd");
}

extern "C" int gdn_prefill_fwd_variant(const gdn_bf16 *q, const gdn_bf16 *k, const gdn_bf16 *v,
                                       const float *state, const float *A_log, const gdn_bf16 *a,
                                       const float *dt_bias, const gdn_bf16 *b,
                                       const void *cu_seqlens, int cu_seqlens_is_int64,
                                       int num_seqs, int total_tokens, float scale,
                                       gdn_bf16 *output, float *new_state, void *workspace,
                                       size_t workspace_bytes, void *stream, int variant) {
  return gdn::prefill_launch(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, cu_seqlens_is_int64,
                             num_seqs, total_tokens, scale, output, new_state, workspace,
                             workspace_bytes, stream, variant, -1, -1, gdn::kHQK, gdn::kHV,
                             "gdn_prefill_fwd_variant");
}

extern "C" int gdn_prefill_fwd_tuned(const gdn_bf16 *q, const gdn_bf16 *k, const gdn_bf16 *v,
                                     const float *state, const float *A_log, const gdn_bf16 *a,
                                     const float *dt_bias, const gdn_bf16 *b,
                                     const void *cu_seqlens, int cu_seqlens_is_int64,
                                     int num_seqs, int total_tokens, float scale,
                                     gdn_bf16 *output, float *new_state, void *workspace,
                                     size_t workspace_bytes, void *stream, int state_tiling,
                                     int recurrent_max_len, int recurrent_tiling) {
  return gdn::prefill_launch(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, cu_seqlens_is_int64,
                             num_seqs, total_tokens, scale, output, new_state, workspace,
                             workspace_bytes, stream, state_tiling, recurrent_max_len,
                             recurrent_tiling, gdn::kHQK, gdn::kHV, "gdn_prefill_fwd_tuned");
}

extern "C" int gdn_prefill_fwd_heads(const gdn_bf16 *q, const gdn_bf16 *k, const gdn_bf16 *v,
                                     const float *state, const float *A_log, const gdn_bf16 *a,
                                     const float *dt_bias, const gdn_bf16 *b,
                                     const void *cu_seqlens, int cu_seqlens_is_int64,
                                     int num_seqs, int total_tokens, int num_qk_heads,
                                     int num_v_heads, float scale, gdn_bf16 *output,
                                     float *new_state, void *workspace, size_t workspace_bytes,
                                     void *stream, int state_tiling, int recurrent_max_len,
                                     int recurrent_tiling) {
  return gdn::prefill_launch(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, cu_seqlens_is_int64,
                             num_seqs, total_tokens, scale, output, new_state, workspace,
                             workspace_bytes, stream, state_tiling, recurrent_max_len,
                             recurrent_tiling, num_qk_heads, num_v_heads, "gdn_prefill_fwd_heads");
}

// ---------------------------------------------------------------------------
// Allocation-free prefill.  The workspace is `scratch`, a file-scope device
// array of GDN_PREFILL_SCRATCH_BYTES: every GPU the library runs on holds its
// own copy, at its own address, until the process ends.  That address is
// looked up once per device (hipGetSymbolAddress with the device current, on
// the entry point's first call there) and only the looked-up pointer is
// handed to the kernels: in host code the array's name is a stand-in, not a
// device address.  Nothing in the workspace needs to start at zero -- every
// region is written by an earlier kernel of the same call before it is read
// -- so the previous call's contents are harmless.  All calls on one GPU
// share its array: calls that overlap in time on one GPU (different streams
// or host threads without ordering) race on it.
// ---------------------------------------------------------------------------
namespace gdn {

static __device__ __align__(256) unsigned char scratch[GDN_PREFILL_SCRATCH_BYTES];

constexpr int kMaxScratchDevices = 64;
static std::mutex g_scratch_mutex;
static void *g_scratch_ptr[kMaxScratchDevices];

// The scratch array of the device `stream` runs on, which must be the current
// device (the lookup resolves the array of the current device).
static int device_scratch(void *stream, void **ptr, const char *what) {
  int cur = -1;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess || cur < 0 || cur >= kMaxScratchDevices)
    return fail(GDN_ERR_LAUNCH, "%s: no usable current device (%s)", what, hipGetErrorString(e));
  if (stream != nullptr) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev);
    if (e != hipSuccess) return fail(GDN_ERR_INVALID, "%s: bad stream (%s)", what, hipGetErrorString(e));
    if (sdev != cur)
      return fail(GDN_ERR_INVALID, "%s: the stream is on device %d, the current device is %d", what,
                  static_cast<int>(sdev), cur);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[cur] == nullptr) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(GDN_ERR_LAUNCH, "%s: hipGetSymbolAddress(scratch) on device %d failed: %s", what,
                  cur, hipGetErrorString(e));
    g_scratch_ptr[cur] = p;
  }
  *ptr = g_scratch_ptr[cur];
  return GDN_OK;
}

}  // namespace gdn

extern "C" int gdn_prefill_fwd_noalloc(const gdn_bf16 *q, const gdn_bf16 *k, const gdn_bf16 *v,
                                       const float *state, const float *A_log, const gdn_bf16 *a,
                                       const float *dt_bias, const gdn_bf16 *b,
                                       const void *cu_seqlens, int cu_seqlens_is_int64,
                                       int num_seqs, int total_tokens, float scale,
                                       gdn_bf16 *output, float *new_state, void *stream) {
  gdn::clear_error();
  if (total_tokens < 0 || num_seqs < 0)
    return gdn::fail(GDN_ERR_INVALID, "gdn_prefill_fwd_noalloc: num_seqs=%d, total_tokens=%d",
                     num_seqs, total_tokens);
  const size_t need = gdn_prefill_workspace_bytes(total_tokens, num_seqs);
  if (need > GDN_PREFILL_SCRATCH_BYTES)
    return gdn::fail(GDN_ERR_WORKSPACE, "gdn_prefill_fwd_noalloc: %d tokens in %d sequences need "
                     "%zu bytes of workspace, more than the %zu-byte static scratch (use "
                     "gdn_prefill_fwd with a workspace)", total_tokens, num_seqs, need,
                     static_cast<size_t>(GDN_PREFILL_SCRATCH_BYTES));
  void *ws = nullptr;
  if (int rc = gdn::device_scratch(stream, &ws, "gdn_prefill_fwd_noalloc")) return rc;
  return gdn::prefill_launch(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, cu_seqlens_is_int64,
                             num_seqs, total_tokens, scale, output, new_state, ws,
                             GDN_PREFILL_SCRATCH_BYTES, stream, -1, -1, -1, gdn::kHQK, gdn::kHV,
                             "gdn_prefill_fwd_noalloc");
}

extern "C" long long gdn_prefill_status_offset(int total_tokens, int num_seqs, int num_qk_heads,
                                               int num_v_heads) {
  if (total_tokens < 0 || num_seqs < 1 || num_qk_heads < 1 || num_v_heads < 1 ||
      num_v_heads > gdn::kMaxHeads || num_v_heads % num_qk_heads != 0)
    return -1;
  const gdn::Heads H{num_qk_heads, num_v_heads, num_v_heads / num_qk_heads};
  return static_cast<long long>(gdn::prefill_layout(total_tokens, num_seqs, H).status);
}

extern "C" int gdn_prefill_status(const void *workspace, int total_tokens, int num_seqs,
                                  int num_qk_heads, int num_v_heads, void *stream, int *status) {
  gdn::clear_error();
  const long long off = gdn_prefill_status_offset(total_tokens, num_seqs, num_qk_heads, num_v_heads);
  if (status == nullptr || off < 0)
    return gdn::fail(GDN_ERR_INVALID, "gdn_prefill_status: status=%p, T=%d, N=%d, heads %d/%d",
                     static_cast<void *>(status), total_tokens, num_seqs, num_qk_heads, num_v_heads);
  const char *ws = static_cast<const char *>(workspace);
  if (ws == nullptr) {
    const size_t need = gdn_prefill_workspace_bytes_heads(total_tokens, num_seqs, num_qk_heads,
                                                          num_v_heads);
    if (need > GDN_PREFILL_SCRATCH_BYTES)
      return gdn::fail(GDN_ERR_WORKSPACE, "gdn_prefill_status: %d tokens in %d sequences do not fit "
                       "the static scratch", total_tokens, num_seqs);
    void *p = nullptr;
    if (int rc = gdn::device_scratch(stream, &p, "gdn_prefill_status")) return rc;
    ws = static_cast<const char *>(p);
  }
  std::vector<int> words(static_cast<size_t>(num_seqs));
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e = hipMemcpyAsync(words.data(), ws + off, words.size() * sizeof(int),
                                hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  if (e != hipSuccess)
    return gdn::fail(GDN_ERR_LAUNCH, "gdn_prefill_status: reading the status words failed: %s",
                     hipGetErrorString(e));
  int bits = 0;
  for (int w : words) bits |= w;
  *status = bits;
  return GDN_OK;
}
