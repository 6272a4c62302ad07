// Gated DeltaNet token-sequential recurrence: the state of one (sequence,
// v-head, block of V-rows) lives in registers for the whole sequence and every
// token is one fused decode step on it.
//
// Semantics: the per-token loop of reference/gdn_prefill_ref.py:71-89 (and,
// for a single token, reference/gdn_decode_ref.py:60-81):
//   g = exp(-exp(A_log[h]) * softplus(a_t + dt_bias[h])),  beta = sigmoid(b_t)
//   for every V-row r:  pred = g <S[r,:], k_t>,  v_new = beta (v_t[r] - pred)
//                       S[r,:] = g S[r,:] + v_new k_t
//                       o_t[r] = scale <S[r,:], q_t> = scale (g <S_old[r],q_t> + v_new <k_t,q_t>)
// with q/k head h/2 (GVA without copies).  It serves
//   * prefill of batches of short sequences, where the chunked pipeline's
//     fixed cost (four dependent launches, a full chunk of work per sequence)
//     dominates: the sequential-scan / chunked crossover of
//     OPTIMIZATION_LOG.md:79,170-184, chosen on the device from the longest
//     sequence of the batch;
//   * decode of T > 1 tokens per batch row (multi-token / speculative decode),
//     a fixed-length batch [B, T, ...] that is exactly the packed layout.
//
// Work mapping (gfx950, wave64) as in the decode kernel: a state row of 128
// floats is held by an aligned group of 16 lanes, 8 floats per lane (columns
// 4c..4c+3 and 64+4c..64+4c+3), so the two row dot products per token are 8
// FMAs and 4 DPP adds.  A workgroup of WAVES waves owns 4*WAVES*PASSES rows.
// Per token each lane loads its 8 columns of k and q (two 8-byte loads each)
// and one bf16 of v per pass, 2-8 tokens ahead of use (a register ring); the
// gating of a ring turn's tokens is computed at once, one token per lane, and
// read back with readlane.
#include "gdn_device.h"
#include "gdn_host.h"

namespace gdn {

template <int PASSES>
struct TokenIn {
  u16x4 k0, k1, q0, q1;
  uint16_t v[PASSES];
};

template <int WAVES, int PASSES>
__global__ __launch_bounds__(64 * WAVES) void recurrent_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ k,
    const uint16_t *__restrict__ v, const float *state, const float *__restrict__ A_log,
    const uint16_t *__restrict__ a, const float *__restrict__ dt_bias,
    const uint16_t *__restrict__ b, const void *__restrict__ cu, int cu64, int N, int T,
    int fixed_len, const int *__restrict__ enable, int *__restrict__ status, Heads H,
    float scale, uint16_t *__restrict__ out, float *new_state) {
  constexpr int kRows = 4 * WAVES * PASSES;
  constexpr int kTiles = kDV / kRows;
  static_assert(kDV % kRows == 0, "row block must divide 128");

  const int h = blockIdx.x % H.v;  // consecutive workgroups: the v-heads
  const int rest = blockIdx.x / H.v;
  const int tile = rest % kTiles, s = rest / kTiles;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c4 = 4 * (lane & 15);
  const int row0 = tile * kRows + wave * 4 * PASSES + (lane >> 4);  // pass p: row0 + 4p

  // The path flag and the sequence's bounds, loaded together (one wait for
  // both), before the state loads, which do not depend on them.
  const int en = enable != nullptr ? *enable : 1;
  long long lo = 0, hi = 0;
  if (cu != nullptr) {
    lo = raw_cu(cu, cu64, s);
    hi = raw_cu(cu, cu64, s + 1);
  }
  if (en == 0) return;  // the batch went through the chunks
  int bos, len;
  if (cu != nullptr) {
    bos = static_cast<int>(lo < 0 ? 0 : lo > T ? T : lo);
    const int eos = static_cast<int>(hi < 0 ? 0 : hi > T ? T : hi);
    len = eos > bos ? eos - bos : 0;
    // the batch's contract bits, one entry per sequence (host-routed batches)
    if (status != nullptr && h == 0 && tile == 0 && threadIdx.x == 0)
      status[s] = cu_status_bits(lo, hi, T);
  } else {
    bos = s * fixed_len;
    len = fixed_len;
  }
  const int hq = h / H.ratio;
  // The state is read once and written once: non-temporal accesses through
  // a descriptor of the (sequence, head) state, as in the decode kernel (over
  // rotating state sets: B=64 T=2 decode 15.3 -> 12.5 us, 256x1 prefill 63.2
  // -> 58.5 us against plain accesses).  The loads do not wait for the
  // sequence's length: a zero-length sequence's state is read and dropped
  // at the final store (zeroing it here would wait for the loads before the
  // token loads go out).
  const size_t sbase = (static_cast<size_t>(s) * H.v + h) * kDV * kDK;
  constexpr uint32_t kHeadBytes = kDV * kDK * 4;
  f32x4 Sa[PASSES], Sb[PASSES];  // columns c4.. and 64 + c4..
  if (state != nullptr) {
    const auto rs = buf_rsrc(state + sbase, kHeadBytes);
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const uint32_t off = static_cast<uint32_t>((row0 + 4 * p) * kDK + c4) * 4u;
      Sa[p] = buf_load16_nt(rs, off);
      Sb[p] = buf_load16_nt(rs, off + 256u);
    }
  } else {
#pragma unroll
    for (int p = 0; p < PASSES; ++p) Sa[p] = Sb[p] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  if (len > 0) {
    const float rate = expf(A_log[h]);
    const float dtb = dt_bias[h];
    auto load_token = [&](int t, TokenIn<PASSES> &x) {
      const size_t tok = static_cast<size_t>(bos) + t;
      const uint16_t *kp = k + (tok * H.qk + hq) * kDK + c4;
      const uint16_t *qp = q + (tok * H.qk + hq) * kDK + c4;
      x.k0 = *reinterpret_cast<const u16x4 *>(kp);
      x.k1 = *reinterpret_cast<const u16x4 *>(kp + 64);
      x.q0 = *reinterpret_cast<const u16x4 *>(qp);
      x.q1 = *reinterpret_cast<const u16x4 *>(qp + 64);
      const uint16_t *vp = v + (tok * H.v + h) * kDV + row0;
#pragma unroll
      for (int p = 0; p < PASSES; ++p) x.v[p] = vp[4 * p];
    };

    // One token: x holds its k, q, v; (g, beta) its gating.  Every lane of a
    // row group holds the row's o, so all 16 store the same two bytes (one
    // coalesced write) and no lane needs a branch.
    auto step = [&](const TokenIn<PASSES> &x, int t, float g, float beta) {
      float kf[8], qf[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        kf[e] = bf16_to_f32(x.k0[e]);
        kf[4 + e] = bf16_to_f32(x.k1[e]);
        qf[e] = bf16_to_f32(x.q0[e]);
        qf[4 + e] = bf16_to_f32(x.q1[e]);
      }
      float pkq = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) pkq = fmaf(kf[e], qf[e], pkq);
      const float kq = row16_sum(pkq);
      uint16_t *op = out + ((static_cast<size_t>(bos) + t) * H.v + h) * kDV + row0;
#pragma unroll
      for (int p = 0; p < PASSES; ++p) {
        float sk0 = 0.f, sk1 = 0.f, sq0 = 0.f, sq1 = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sk0 = fmaf(Sa[p][e], kf[e], sk0);
          sk1 = fmaf(Sb[p][e], kf[4 + e], sk1);
          sq0 = fmaf(Sa[p][e], qf[e], sq0);
          sq1 = fmaf(Sb[p][e], qf[4 + e], sq1);
        }
        const float sk = row16_sum(sk0 + sk1);
        const float sq = row16_sum(sq0 + sq1);
        const float vn = beta * (bf16_to_f32(x.v[p]) - g * sk);
        const float o = scale * fmaf(g, sq, vn * kq);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          Sa[p][e] = fmaf(vn, kf[e], g * Sa[p][e]);
          Sb[p][e] = fmaf(vn, kf[4 + e], g * Sb[p][e]);
        }
        op[4 * p] = f32_to_bf16(o);
      }
    };

    // Everything is loaded ahead of use by unconditional loads (indices past
    // the end are clamped to the last token), so the compiler can wait for
    // exactly the data in use: token t sits in ring slot t % kDepth, refilled
    // with token t + kDepth right after use, and the raw gating inputs of a
    // ring turn arrive one turn ahead.  The main loop runs whole turns as
    // straight-line code (no branch, so the pending-load bookkeeping at its
    // header is exact); the last len % kDepth tokens follow it.
    constexpr int kDepth = PASSES <= 2 ? 8 : (PASSES <= 4 ? 4 : 2);
    const int last = len - 1;
    auto gate_idx = [&](int t0) {  // gating input of token t0 + lane (clamped)
      const int t = t0 + (lane & (kDepth - 1));
      return (static_cast<size_t>(bos) + (t < last ? t : last)) * H.v + h;
    };
    uint16_t a_raw = a[gate_idx(0)], b_raw = b[gate_idx(0)];
    TokenIn<PASSES> ring[kDepth];
#pragma unroll
    for (int r = 0; r < kDepth; ++r) load_token(r < last ? r : last, ring[r]);
    // Gating of the turn's tokens, token t0 + (lane % kDepth) in each lane.
    auto gate = [&](float &gl, float &bl) {
      gl = expf(-rate * softplus20(bf16_to_f32(a_raw) + dtb));
      bl = sigmoidf_(bf16_to_f32(b_raw));
    };
    const int full = len - len % kDepth;
    int t0 = 0;
    for (; t0 < full; t0 += kDepth) {
      float gl, bl;
      gate(gl, bl);
      a_raw = a[gate_idx(t0 + kDepth)];
      b_raw = b[gate_idx(t0 + kDepth)];
#pragma unroll
      for (int r = 0; r < kDepth; ++r) {
        const int t = t0 + r;
        const float g = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gl), r));
        const float beta = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bl), r));
        step(ring[r], t, g, beta);
        load_token(t + kDepth < last ? t + kDepth : last, ring[r]);
      }
    }
    if (t0 < len) {  // the remaining len - full tokens, already in slots 0..
      float gl, bl;
      gate(gl, bl);
#pragma unroll
      for (int r = 0; r < kDepth - 1; ++r) {
        if (t0 + r < len) {
          const float g = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gl), r));
          const float beta = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bl), r));
          step(ring[r], t0 + r, g, beta);
        }
      }
    }
  }

  // Final state; all zeros for a zero-length sequence (gdn_prefill_ref.py:61-62).
  const auto rd = buf_rsrc(new_state + sbase, kHeadBytes);
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const uint32_t off = static_cast<uint32_t>((row0 + 4 * p) * kDK + c4) * 4u;
    buf_store16_nt(rd, off, len > 0 ? Sa[p] : z);
    buf_store16_nt(rd, off + 256u, len > 0 ? Sb[p] : z);
  }
  // A packed batch: rows outside every sequence get zeros.
  if (cu != nullptr) zero_uncovered_rows(out, cu, cu64, N, T, H.v, blockIdx.x, gridDim.x);
}

namespace {

struct RecVariant {
  int waves, passes;
};
// rows per workgroup = 4 * waves * passes
constexpr RecVariant kRecVariants[] = {
    {1, 1}, {2, 1}, {4, 1}, {1, 2}, {2, 2}, {4, 2}, {1, 4}, {4, 4}, {1, 8}, {1, 16}};
constexpr int kNumRecVariants = sizeof(kRecVariants) / sizeof(kRecVariants[0]);
static_assert(kNumRecVariants == kNumRecTilings, "the tiling count is shared with the host code");

template <int W, int P>
void launch_rec(long long groups, hipStream_t stream, const uint16_t *q, const uint16_t *k,
                const uint16_t *v, const float *state, const float *A_log, const uint16_t *a,
                const float *dt_bias, const uint16_t *b, const void *cu, int cu64, int N, int T,
                int fixed_len, const int *enable, int *status, const Heads &H, float scale,
                uint16_t *out, float *new_state) {
  const long long blocks = groups * (kDV / (4 * W * P));
  hipLaunchKernelGGL((recurrent_kernel<W, P>), dim3(static_cast<unsigned>(blocks)), dim3(64 * W),
                     0, stream, q, k, v, state, A_log, a, dt_bias, b, cu, cu64, N, T, fixed_len,
                     enable, status, H, scale, out, new_state);
}

}  // namespace

// Variants 0 .. kNumRecVariants - 1: the row tilings above; kNumRecVariants:
// the 16-token block kernel (gdn_block.hip).
int recurrent_num_variants() { return kNumRecVariants + 1; }
int recurrent_block_variant() { return kNumRecVariants; }

// Built-in tiling from a sweep on MI355X (every tiling, B = 1..256 rows of
// T = 2, 4, 8 tokens, graph replay over rotating states): few (sequence,
// head) groups -> the smallest row blocks (the serial token loop is spread
// over the most waves); more -> one wave streaming 8..32 rows (within ~5 % of
// the best tiling everywhere; 64-row four-wave blocks, the earlier choice for
// more than 128 groups, were up to 14 % slower at B = 64..256).
int recurrent_default_variant(long long groups) {
  if (groups <= 32) return 0;     // 4 rows, 1 wave
  if (groups <= 64) return 3;     // 8 rows, 1 wave
  if (groups <= 256) return 6;    // 16 rows, 1 wave
  if (groups <= 1024) return 8;   // 32 rows, 1 wave
  return 6;                       // 16 rows, 1 wave
}

int recurrent_launch(const uint16_t *q, const uint16_t *k, const uint16_t *v, const float *state,
                     const float *A_log, const uint16_t *a, const float *dt_bias,
                     const uint16_t *b, const void *cu, int cu64, int num_seqs, int T,
                     int fixed_len, const int *enable, int *status, const Heads &H,
                     float scale, uint16_t *out, float *new_state, hipStream_t stream,
                     int variant, const char *what) {
  const long long groups = static_cast<long long>(num_seqs) * H.v;
  if (variant < 0) variant = recurrent_default_variant(groups);
  if (variant == kNumRecVariants)
    return block_launch(q, k, v, state, A_log, a, dt_bias, b, cu, cu64, num_seqs, T, fixed_len,
                        enable, status, H, scale, out, new_state, stream, what);
  if (variant > kNumRecVariants)
    return fail(GDN_ERR_INVALID, "%s: recurrent tiling %d out of range", what, variant);
  const RecVariant rv = kRecVariants[variant];
  if (groups * (kDV / (4 * rv.waves * rv.passes)) > 0x7fffffffLL)
    return fail(GDN_ERR_INVALID, "%s: too many sequences for one launch", what);
#define GDN_REC(W, P)                                                                          \
  if (rv.waves == W && rv.passes == P)                                                        \
    launch_rec<W, P>(groups, stream, q, k, v, state, A_log, a, dt_bias, b, cu, cu64, num_seqs, \
                     T, fixed_len, enable, status, H, scale, out, new_state);
  GDN_REC(1, 1)
  GDN_REC(2, 1)
  GDN_REC(4, 1)
  GDN_REC(1, 2)
  GDN_REC(2, 2)
  GDN_REC(4, 2)
  GDN_REC(1, 4)
  GDN_REC(4, 4)
  GDN_REC(1, 8)
  GDN_REC(1, 16)
#undef GDN_REC
  return check_launch(what);
}

}  // namespace gdn

namespace gdn {

// T >= 1 tokens per row for `batch` rows with head layout (hqk, hv).
static int multi_launch(const gdn_bf16 *q, const gdn_bf16 *k, const gdn_bf16 *v,
                        const float *state, const float *A_log, const gdn_bf16 *a,
                        const float *dt_bias, const gdn_bf16 *b, float scale, gdn_bf16 *output,
                        float *new_state, int batch, int tokens, int hqk, int hv, void *stream,
                        int variant, const char *what) {
  clear_error();
  Heads H;
  if (int rc = make_heads(hqk, hv, what, H)) return rc;
  if (int rc = check_decode_args(q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state,
                                 batch, tokens, H, what))
    return rc;
  int kernel;
  if (int rc = plan_multi(q, k, v, batch, tokens, H, variant, what, &kernel)) return rc;
  if (batch == 0) return GDN_OK;
  const long long total = static_cast<long long>(batch) * tokens;
  // one token per row: the plain decode step, whose kernel is tuned for it
  if (kernel == kDecodeStep)
    return decode_launch(q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state, batch,
                         stream, -1, H, what);
  return recurrent_launch(q, k, v, state, A_log, a, dt_bias, b, nullptr, 0, batch,
                          static_cast<int>(total), tokens, nullptr, nullptr, H, scale, output,
                          new_state, static_cast<hipStream_t>(stream), kernel, what);
}

}  // namespace gdn

extern "C" int gdn_decode_multi_fwd(const gdn_bf16 *q, const gdn_bf16 *k, const gdn_bf16 *v,
                                    const float *state, const float *A_log, const gdn_bf16 *a,
                                    const float *dt_bias, const gdn_bf16 *b, float scale,
                                    gdn_bf16 *output, float *new_state, int batch, int tokens,
                                    void *stream, int variant) {
  return gdn::multi_launch(q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state, batch,
                           tokens, gdn::kHQK, gdn::kHV, stream, variant, "gdn_decode_multi_fwd");
}

extern "C" int gdn_decode_fwd_heads(const gdn_bf16 *q, const gdn_bf16 *k, const gdn_bf16 *v,
                                    const float *state, const float *A_log, const gdn_bf16 *a,
                                    const float *dt_bias, const gdn_bf16 *b, float scale,
                                    gdn_bf16 *output, float *new_state, int batch, int tokens,
                                    int num_qk_heads, int num_v_heads, void *stream,
                                    int variant) {
  return gdn::multi_launch(q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state, batch,
                           tokens, num_qk_heads, num_v_heads, stream, variant,
                           "gdn_decode_fwd_heads");
}
