// Host-side argument checks, workspace layout and path planning (gdn_args.h).
// Plain host C++: built into the library by the host compiler and, unchanged,
// into the CPU sanitizer build of tests/sanitize/.
#include "gdn_args.h"

#include <stdarg.h>
#include <stdio.h>

namespace gdn {

static thread_local char g_last_error[512] = "";

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_last_error[0] = '\0'; }

const char *last_error_text() { return g_last_error; }

int make_heads(int hqk, int hv, const char *what, Heads &H) {
  if (hqk < 1 || hv < 1 || hv > kMaxHeads || hv % hqk != 0)
    return fail(GDN_ERR_INVALID, "%s: heads %d q/k, %d v (need v a multiple of q/k, <= %d)", what,
                hqk, hv, kMaxHeads);
  H = Heads{hqk, hv, hv / hqk};
  return GDN_OK;
}

static bool bad_scale(float scale) { return !(scale > 0.0f) || scale == __builtin_inff(); }

int check_decode_args(const gdn_bf16 *q, const gdn_bf16 *k, const gdn_bf16 *v, const float *state,
                      const float *A_log, const gdn_bf16 *a, const float *dt_bias,
                      const gdn_bf16 *b, float scale, const gdn_bf16 *output,
                      const float *new_state, int batch, int tokens, const Heads &H,
                      const char *what) {
  if (batch < 0 || tokens < 1) return fail(GDN_ERR_INVALID, "%s: batch=%d, tokens=%d", what, batch, tokens);
  if (!q || !k || !v || !A_log || !a || !dt_bias || !b || !output || !new_state)
    return fail(GDN_ERR_INVALID, "%s: null pointer argument", what);
  if (bad_scale(scale)) return fail(GDN_ERR_INVALID, "%s: scale must be finite and > 0", what);
  if (!aligned(new_state, 16) || (state && !aligned(state, 16)))
    return fail(GDN_ERR_INVALID, "%s: state/new_state must be 16-byte aligned", what);
  if (!aligned(q, 8) || !aligned(k, 8))
    return fail(GDN_ERR_INVALID, "%s: q/k must be 8-byte aligned", what);
  if (!aligned(v, 2) || !aligned(a, 2) || !aligned(b, 2) || !aligned(output, 2))
    return fail(GDN_ERR_INVALID, "%s: v/a/b/output must be 2-byte aligned", what);
  const long long total = static_cast<long long>(batch) * tokens;
  if (total > 0x7fffffffLL) return fail(GDN_ERR_INVALID, "%s: batch*tokens too large", what);
  const size_t nb = static_cast<size_t>(batch), nt = static_cast<size_t>(total);
  const size_t nV = static_cast<size_t>(H.v), nQK = static_cast<size_t>(H.qk);
  const size_t state_bytes = nb * nV * kDV * kDK * sizeof(float);
  const size_t out_bytes = nt * nV * kDV * sizeof(uint16_t);
  // new_state may be exactly state (in-place); no other overlap is allowed.
  if (state != new_state && overlaps(state, state_bytes, new_state, state_bytes))
    return fail(GDN_ERR_INVALID, "%s: new_state partially overlaps state", what);
  const void *ins[] = {q, k, v, a, b, A_log, dt_bias, state};
  const size_t in_bytes[] = {nt * nQK * kDK * 2, nt * nQK * kDK * 2, nt * nV * kDV * 2,
                             nt * nV * 2,        nt * nV * 2,        nV * 4,
                             nV * 4,             state ? state_bytes : 0};
  for (int i = 0; i < 8; ++i) {
    if (overlaps(output, out_bytes, ins[i], in_bytes[i]))
      return fail(GDN_ERR_INVALID, "%s: output overlaps an input", what);
    if (i < 7 && overlaps(new_state, state_bytes, ins[i], in_bytes[i]))
      return fail(GDN_ERR_INVALID, "%s: new_state overlaps an input", what);
  }
  if (overlaps(output, out_bytes, new_state, state_bytes))
    return fail(GDN_ERR_INVALID, "%s: output overlaps new_state", what);
  return GDN_OK;
}

int plan_multi(const void *q, const void *k, const void *v, int batch, int tokens, const Heads &H,
               int variant, const char *what, int *kernel) {
  *kernel = -1;
  if (variant < -1 || variant > kNumRecTilings)
    return fail(GDN_ERR_INVALID, "%s: unknown variant %d", what, variant);
  if (tokens == 1 && variant == -1) {
    *kernel = kDecodeStep;
    return GDN_OK;
  }
  const bool rows16 = aligned(q, 16) && aligned(k, 16) && aligned(v, 16);
  if (variant == kNumRecTilings && !rows16)
    return fail(GDN_ERR_INVALID, "%s: the block kernel needs 16-byte aligned q/k/v", what);
  if (variant == -1 && rows16) {
    const float L = static_cast<float>(tokens), fhv = static_cast<float>(H.v);
    const float g = static_cast<float>(batch) * fhv;
    const float total = static_cast<float>(static_cast<long long>(batch) * tokens);
    if (cost_by_block(L, g) < cost_by_token(L, total, fhv, g)) variant = kNumRecTilings;
  }
  *kernel = variant;
  return GDN_OK;
}

long long max_chunks(long long T, long long N) {
  if (T <= 0 || N <= 0) return 0;
  const long long bound = (T + N * (kChunk - 1)) / kChunk;
  return bound < T ? bound : T;
}

PrefillLayout prefill_layout(int T, int N, const Heads &H) {
  PrefillLayout L{};
  const long long nt = max_chunks(T, N);
  L.nt_max = static_cast<int>(nt);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off = (off + bytes + 255) & ~static_cast<size_t>(255);
    return o;
  };
  const size_t n = static_cast<size_t>(nt);
  const size_t nN = N > 0 ? static_cast<size_t>(N) : 0;
  L.chunks = take(n * 16);                // int4 per chunk
  L.offsets = take((nN + 3) * sizeof(int));  // + path and form flags
  L.status = take(nN * sizeof(int));         // contract bits per sequence
  const size_t hv = static_cast<size_t>(H.v), hqk = static_cast<size_t>(H.qk);
  L.G = take(n * hv * kChunk * 4);
  L.dcy = take(n * hv * kChunk * 4);
  L.eg = take(n * hv * 4);
  L.w = take(n * hv * kChunk * kDK * 4);  // hi and lo bf16
  L.u = take(n * hv * kChunk * kDV * 4);
  L.kt = take(n * hqk * kDK * kChunk * 2);
  L.ht = take(n * hv * kDV * kDK * 2);
  L.vnt = take(n * hv * kDV * kChunk * 2);
  const size_t n1 = N == 1 ? static_cast<size_t>(nt - split_first(static_cast<int>(nt))) : 0;
  const size_t one = N == 1 ? 1 : 0;
  L.htm = take(n1 * hv * kDV * kDK * 2);
  L.send = take(one * hv * kDV * kDK * 4);
  L.cend = take(one * hv * kDV * kDK * 4);
  L.mend = take(one * hv * kDV * kDK * 4);
  L.early = take(N == 1 ? static_cast<size_t>(early_words(split_first(static_cast<int>(nt)), H.v)) * 4 : 0);
  L.total = off;
  return L;
}

int check_prefill_args(const gdn_bf16 *q, const gdn_bf16 *k, const gdn_bf16 *v, const float *state,
                       const float *A_log, const gdn_bf16 *a, const float *dt_bias,
                       const gdn_bf16 *b, const void *cu_seqlens, int cu64, int N, int T,
                       float scale, const gdn_bf16 *output, const float *new_state,
                       const void *workspace, size_t ws_bytes, int variant, int rec_max,
                       int rec_variant, int num_rec_variants, const Heads &H,
                       const char *what, PrefillLayout *L) {
  *L = PrefillLayout{};
  if (N < 0 || T < 0) return fail(GDN_ERR_INVALID, "%s: num_seqs=%d, total_tokens=%d", what, N, T);
  if (!cu_seqlens) return fail(GDN_ERR_INVALID, "%s: null cu_seqlens", what);
  if (!A_log || !dt_bias) return fail(GDN_ERR_INVALID, "%s: null pointer argument", what);
  if (T > 0 && (!q || !k || !v || !a || !b || !output))
    return fail(GDN_ERR_INVALID, "%s: null pointer argument", what);
  if (N > 0 && !new_state) return fail(GDN_ERR_INVALID, "%s: null new_state", what);
  if (bad_scale(scale)) return fail(GDN_ERR_INVALID, "%s: scale must be finite and > 0", what);
  if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16))
    return fail(GDN_ERR_INVALID, "%s: q/k/v must be 16-byte aligned", what);
  if (!aligned(new_state, 16) || (state && !aligned(state, 16)))
    return fail(GDN_ERR_INVALID, "%s: state/new_state must be 16-byte aligned", what);
  if (!aligned(output, 16)) return fail(GDN_ERR_INVALID, "%s: output must be 16-byte aligned", what);
  if (!aligned(a, 2) || !aligned(b, 2)) return fail(GDN_ERR_INVALID, "%s: a/b must be 2-byte aligned", what);
  if (!aligned(cu_seqlens, cu64 ? 8 : 4)) return fail(GDN_ERR_INVALID, "%s: cu_seqlens misaligned", what);
  if (variant < -1 || variant > 4)
    return fail(GDN_ERR_INVALID, "%s: unknown variant %d (0 WY form, 1 T form, 2 WY one chain, 3 WY "
                "two segments, 4 as 3 with the early output cut short)", what, variant);
  if (rec_max < -2) return fail(GDN_ERR_INVALID, "%s: recurrent_max_len %d < -2", what, rec_max);
  if (rec_variant < -1 || rec_variant >= num_rec_variants)
    return fail(GDN_ERR_INVALID, "%s: unknown recurrent tiling %d", what, rec_variant);
  if (N == 0 && T == 0) return GDN_OK;

  // (a batch without sequences only zero-fills the output: no workspace needed)
  if (N > 0) {
    *L = prefill_layout(T, N, H);
    if (!workspace || ws_bytes < L->total)
      return fail(GDN_ERR_WORKSPACE, "%s: workspace of %zu bytes, %zu needed", what, ws_bytes, L->total);
    if (!aligned(workspace, 256)) return fail(GDN_ERR_INVALID, "%s: workspace must be 256-byte aligned", what);
  }
  const size_t ws_total = L->total;
  const void *ws = N > 0 ? workspace : nullptr;

  const size_t nT = static_cast<size_t>(T), nN = static_cast<size_t>(N);
  const size_t nV = static_cast<size_t>(H.v), nQK = static_cast<size_t>(H.qk);
  const size_t state_bytes = nN * nV * kDV * kDK * 4;
  const size_t out_bytes = nT * nV * kDV * 2;
  const void *ins[] = {q, k, v, a, b, A_log, dt_bias, cu_seqlens, state};
  const size_t in_bytes[] = {nT * nQK * kDK * 2, nT * nQK * kDK * 2, nT * nV * kDV * 2,
                             nT * nV * 2,        nT * nV * 2,        nV * 4,
                             nV * 4,             (nN + 1) * (cu64 ? 8 : 4),
                             state ? state_bytes : 0};
  for (int i = 0; i < 9; ++i) {
    if (overlaps(output, out_bytes, ins[i], in_bytes[i]))
      return fail(GDN_ERR_INVALID, "%s: output overlaps an input", what);
    if (i < 8 && overlaps(new_state, state_bytes, ins[i], in_bytes[i]))
      return fail(GDN_ERR_INVALID, "%s: new_state overlaps an input", what);
    if (overlaps(ws, ws_total, ins[i], in_bytes[i]))
      return fail(GDN_ERR_INVALID, "%s: workspace overlaps an input", what);
  }
  if (state != new_state && overlaps(state, state_bytes, new_state, state_bytes))
    return fail(GDN_ERR_INVALID, "%s: new_state partially overlaps state", what);
  if (overlaps(output, out_bytes, new_state, state_bytes) || overlaps(ws, ws_total, output, out_bytes) ||
      overlaps(ws, ws_total, new_state, state_bytes))
    return fail(GDN_ERR_INVALID, "%s: outputs/workspace overlap", what);
  return GDN_OK;
}

int plan_prefill(int T, int N, const Heads &H, const PrefillLayout &L, int variant, int rec_max,
                 int rec_variant, int block_variant, const char *what, PrefillPlan &P) {
  P = PrefillPlan{};
  P.seq_variant = rec_variant;
  const float fT = static_cast<float>(T), fhv = static_cast<float>(H.v);
  if (rec_max >= 0) {
    P.sequential = rec_max >= T;
    P.choose = N > 1 ? 1 : 0;
  } else if (rec_max == -1) {
    P.sequential = T <= kRecurrentMaxLen;
    if (P.sequential && N == 1 && P.seq_variant < 0) {
      // one short sequence: token by token or in blocks, by the cost models
      if (cost_by_block(fT, fhv) < cost_by_token(fT, fT, fhv, fhv)) P.seq_variant = block_variant;
    }
    if (!P.sequential && N > 1) {
      const float g = static_cast<float>(N) * fhv, mean = ceilf(fT / static_cast<float>(N));
      const float by_token = cost_by_token(mean, fT, fhv, g), by_block = cost_by_block(mean, g);
      if (P.seq_variant < 0 && by_block < by_token) P.seq_variant = block_variant;
      const bool blocks = P.seq_variant == block_variant;
      const float seq_lo = blocks ? by_block : by_token;
      // The sequential path's best case against the chunks is N equal
      // sequences of the mean length (its cost grows with the longest
      // sequence ~10x faster than the chunks'): the device gets the choice
      // only if the sequential path wins there by more than the choice costs.
      const float fN = static_cast<float>(N);
      const float chunks_eq = cost_by_chunks(mean, fN * ceilf(mean / kChunk), fhv, fN);
      if (seq_lo + kDeviceChoiceCost < chunks_eq) P.choose = blocks ? 3 : 2;
    }
  }
  if (P.sequential) return GDN_OK;

  // One sequence needs no chunk table: the kernels read its bounds
  // [cu[0], cu[1]) themselves and compute its chunks.
  P.single = N == 1 && P.choose == 0;
  // Form of the per-chunk operands: `variant` when 0 (WY) or 1 (T); else the
  // index kernel's rule (t_form_wins), settled here when (T, N) alone exclude
  // the T form -- the rule fails at the largest chunk count possible (nt_max)
  // and the chunks of the mean length, a lower bound on the longest
  // sequence's (the rule only turns true as chunks grow or the longest
  // shrinks) -- so that only one intra kernel is launched.
  P.form = variant >= 2 ? 0 : variant;
  if (P.form < 0) {
    const long long mean_chunks = ((static_cast<long long>(T) + N - 1) / N + kChunk - 1) / kChunk;
    const bool t_possible =
        !P.single && t_form_wins(static_cast<float>(L.nt_max), static_cast<float>(mean_chunks),
                                 state_units(static_cast<float>(N), static_cast<float>(H.v)));
    P.form = t_possible ? -1 : 0;
  }
  const long long grid = chunk_head_grid(L.nt_max, H);
  if (grid > 0x7fffffffLL) return fail(GDN_ERR_INVALID, "%s: too many tokens", what);
  P.intra_grid = L.nt_max > 0 ? grid : 0;
  P.intra_split = P.form == 0 && 2 * P.intra_grid <= static_cast<long long>(kNumCus) * kIntraSplitPerCu;
  if (P.intra_split) P.intra_grid *= 2;
  P.loop = P.choose != 0;
  P.self_index = !P.single && N <= kSelfIndexMax && P.intra_grid > 0 &&
                 P.intra_grid <= kSelfIndexMaxGrid;
  auto cap = [&P](long long units, int per_cu) {
    const long long most = static_cast<long long>(kNumCus) * per_cu;
    return P.loop && units > most ? most : units;
  };

  if (P.single && P.form == 0 && variant != 2 && L.nt_max >= 2 && 24 * H.v <= 256 &&
      (variant >= 3 || L.nt_max >= kSplitMinChunks))
    P.split_nt0 = split_first(L.nt_max);
  const bool split = P.split_nt0 > 0;
  const long long state_units = static_cast<long long>(split ? 3 : N) * H.v * (kDV / 16);
  if (state_units > 0x7fffffffLL) return fail(GDN_ERR_INVALID, "%s: too many sequences", what);
  P.state_grid = cap(state_units, kStatePerCu);
  P.split_grid = split ? static_cast<long long>(L.nt_max - P.split_nt0) * H.v : 0;
  P.early_grid = split && H.v == 8 && state_units + kEarlyGrid <= kNumCus &&
                         P.split_nt0 >= 2 * kEarlyTail
                     ? kEarlyGrid
                     : 0;
  P.early_limit = variant == 4 ? 1 : 0;
  // with the early output, kEarlyTail workgroups per head cover the first
  // segment (its last chunks, and any the early workgroups left)
  P.out_grid = L.nt_max > 0 ? (P.early_grid > 0 ? static_cast<long long>(kEarlyTail) * H.v
                                                 : chunk_head_grid(split ? P.split_nt0 : L.nt_max, H)) +
                                  (split ? kStateTiles * H.v : 0)
                            : 0;
  return GDN_OK;
}

}  // namespace gdn
