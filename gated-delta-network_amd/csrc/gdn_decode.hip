// Gated DeltaNet decode (T = 1): one fused, HBM-bound pass over the state.
//
// Semantics: reference/gdn_decode_ref.py:12-83.  Per (batch row n, v-head h):
//   decay = exp(-exp(A_log[h]) * softplus(a + dt_bias[h])),  beta = sigmoid(b)
//   for every V-row r of the k-last state S[n,h] ([V=128, K=128] f32):
//     pred  = decay * <S[r,:], k>          v_new = beta * (v[r] - pred)
//     S'[r] = decay * S[r,:] + v_new * k   o[r]  = scale * <S'[r,:], q>
// where q, k are q/k head h/2 (GVA without copies).  <S'[r], q> is evaluated
// as decay*<S[r],q> + v_new*<k,q>, so both row reductions run together.
//
// Work mapping (gfx950, wave64): a row of 128 floats is held by one aligned
// group of 16 lanes, 8 floats per lane as two 16-byte loads at columns 4c and
// 64+4c (c = lane % 16), so each wave-wide load instruction reads 4 x 256
// contiguous bytes.  The row sums use 4 DPP adds inside the 16-lane group.  A
// workgroup of WAVES waves covers 4*WAVES rows per pass and PASSES passes;
// every load -- the gating inputs, q/k, v, then every pass's state -- is
// issued before any arithmetic, so one workgroup keeps 4*WAVES*PASSES*512
// bytes of state in flight from its start (B=64: 12.0 -> 11.5 us per step
// in 20-step graphs against the gating computed first).  Each lane needs
// only its 8 columns of q and k, loaded once; v is one load per wave and o
// one store per wave.
#include "gdn_device.h"
#include "gdn_host.h"

namespace gdn {

template <int WAVES, int PASSES, bool HAS_STATE, bool NONTEMPORAL>
__global__ __launch_bounds__(64 * WAVES) void decode_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ k,
    const uint16_t *__restrict__ v, const float *state, const float *__restrict__ A_log,
    const uint16_t *__restrict__ a, const float *__restrict__ dt_bias,
    const uint16_t *__restrict__ b, float scale, uint16_t *__restrict__ out, float *new_state,
    Heads H) {
  constexpr int kRowsPerPass = 4 * WAVES;
  constexpr int kRows = kRowsPerPass * PASSES;
  constexpr int kTiles = kDV / kRows;
  static_assert(kDV % kRows == 0, "row tile must divide 128");

  const int tile = blockIdx.x % kTiles;
  const int nh = blockIdx.x / kTiles;  // n * H.v + h
  // The reference's head shape (8 v-heads over 4 q/k heads) by shifts: the
  // divisions by run-time head counts put ~45 scalar instructions ahead of
  // the first load (B=64: 11.30 -> 11.23 us per step in 20-step graphs).
  int h, n, hq;
  if (H.v == 8 && H.ratio == 2) {
    h = nh & 7;
    n = nh >> 3;
    hq = h >> 1;
  } else {
    h = nh % H.v;
    n = nh / H.v;
    hq = h / H.ratio;
  }
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c = lane & 15;
  const int row0 = tile * kRows + wave * 4 + (lane >> 4);

  // Every load is issued before any arithmetic, in the order the work needs
  // the data: the gating inputs, q/k and v (small, used first), then the
  // state rows.  The scheduling barrier keeps the gating arithmetic -- and
  // the wait for its inputs -- after the state loads, so each wave has its
  // whole share of the state in flight at once, as a streaming copy does
  // (with the gating first, every wave waited out one load latency before
  // its first state load).
  const uint16_t a_raw = a[nh], b_raw = b[nh];
  const float alog = A_log[h], dtb = dt_bias[h];
  // This lane's 8 columns of q and k (q/k head h/2).
  const int qk_off = (n * H.qk + hq) * kDK;
  const u16x4 qa = *reinterpret_cast<const u16x4 *>(q + qk_off + 4 * c);
  const u16x4 qb = *reinterpret_cast<const u16x4 *>(q + qk_off + 64 + 4 * c);
  const u16x4 ka = *reinterpret_cast<const u16x4 *>(k + qk_off + 4 * c);
  const u16x4 kb = *reinterpret_cast<const u16x4 *>(k + qk_off + 64 + 4 * c);
  // v: one 2-byte load per lane, lane j of row group g holding the row of
  // pass j (passes past the last load the last one's), broadcast to the group
  // in each pass (row_bcast16) -- instead of one load instruction per pass.
  static_assert(PASSES <= 16, "one lane of a 16-lane group per pass");
  const int jl = (lane & 15) < PASSES ? (lane & 15) : PASSES - 1;
  const uint16_t v_raw = v[nh * kDV + row0 + jl * kRowsPerPass];
  __builtin_amdgcn_sched_barrier(0);  // (the small loads stay ahead of the state's)

  // The state rows; non-temporal loads go through a descriptor of the head's
  // state (buf_load16_nt), non-temporal stores through flat addresses (B=64:
  // 11.56 -> 11.36 us per step in 20-step graphs against descriptor stores,
  // which a plain copy prefers).
  f32x4 s[PASSES][2];
  float vr[PASSES];
  const size_t head_base = static_cast<size_t>(nh) * kDV * kDK;
  constexpr uint32_t kHeadBytes = kDV * kDK * 4;
  const auto rs = buf_rsrc(HAS_STATE ? state + head_base : new_state + head_base, kHeadBytes);
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int row = row0 + p * kRowsPerPass;
    const size_t base = head_base + static_cast<size_t>(row) * kDK;
    const uint32_t off = static_cast<uint32_t>(row * kDK + 4 * c) * 4u;
    if constexpr (HAS_STATE) {
      const f32x4 *src0 = reinterpret_cast<const f32x4 *>(state + base + 4 * c);
      const f32x4 *src1 = reinterpret_cast<const f32x4 *>(state + base + 64 + 4 * c);
      if constexpr (NONTEMPORAL) {
        s[p][0] = buf_load16_nt(rs, off);
        s[p][1] = buf_load16_nt(rs, off + 256u);
      } else {
        s[p][0] = *src0;
        s[p][1] = *src1;
      }
    } else {
      s[p][0] = f32x4{0.f, 0.f, 0.f, 0.f};
      s[p][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // Gating (reference/gdn_decode_ref.py:42-44), in every lane: a few
  // transcendental ops, cheaper than a broadcast.
  const float decay = expf(gdn_log_decay(alog, bf16_to_f32(a_raw), dtb));
  const float beta = sigmoidf_(bf16_to_f32(b_raw));
  float qf[8], kf[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    qf[i] = bf16_to_f32(qa[i]);
    qf[4 + i] = bf16_to_f32(qb[i]);
    kf[i] = bf16_to_f32(ka[i]);
    kf[4 + i] = bf16_to_f32(kb[i]);
  }
  const float vl = bf16_to_f32(v_raw);
#pragma unroll
  for (int p = 0; p < PASSES; ++p) vr[p] = row_bcast16(vl, p);

  float kq = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) kq = fmaf(kf[i], qf[i], kq);
  kq = row16_sum(kq);
  float ov = 0.f;  // the output of this lane's pass (lane c of its group: pass c)

#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int row = row0 + p * kRowsPerPass;
    float sv[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sv[i] = s[p][0][i];
      sv[4 + i] = s[p][1][i];
    }
    float sk = 0.f, sq = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      sk = fmaf(sv[i], kf[i], sk);
      sq = fmaf(sv[i], qf[i], sq);
    }
    sk = row16_sum(sk);
    sq = row16_sum(sq);
    const float v_new = beta * (vr[p] - decay * sk);
    const float o = scale * fmaf(decay, sq, v_new * kq);
    f32x4 n0, n1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      n0[i] = fmaf(decay, sv[i], v_new * kf[i]);
      n1[i] = fmaf(decay, sv[4 + i], v_new * kf[4 + i]);
    }
    const size_t base = head_base + static_cast<size_t>(row) * kDK;
    f32x4 *dst0 = reinterpret_cast<f32x4 *>(new_state + base + 4 * c);
    f32x4 *dst1 = reinterpret_cast<f32x4 *>(new_state + base + 64 + 4 * c);
    if constexpr (NONTEMPORAL) {
      __builtin_nontemporal_store(n0, dst0);
      __builtin_nontemporal_store(n1, dst1);
    } else {
      *dst0 = n0;
      *dst1 = n1;
    }
    if (c == p) ov = o;  // every lane of the group holds the row's o
  }
  // o: lane j of row group g writes the row of pass j, one store instruction
  if (c < PASSES) out[nh * kDV + row0 + c * kRowsPerPass] = f32_to_bf16(ov);
}

namespace {

typedef void (*decode_fn)(const uint16_t *, const uint16_t *, const uint16_t *, const float *,
                          const float *, const uint16_t *, const float *, const uint16_t *,
                          float, uint16_t *, float *, Heads);

struct DecodeVariant {
  int waves, passes;
  decode_fn with_state[2];  // [nontemporal]
  decode_fn no_state[2];
};

#define GDN_DECODE_VARIANT(W, P)                                                     \
  {                                                                                  \
    W, P, {decode_kernel<W, P, true, false>, decode_kernel<W, P, true, true>}, {     \
      decode_kernel<W, P, false, false>, decode_kernel<W, P, false, true>            \
    }                                                                                \
  }

// Tilings: rows per workgroup = 4 * waves * passes.
const DecodeVariant kVariants[] = {
    GDN_DECODE_VARIANT(4, 8),  // 0: 128 rows, 256 threads
    GDN_DECODE_VARIANT(4, 4),  // 1:  64 rows, 256 threads
    GDN_DECODE_VARIANT(4, 2),  // 2:  32 rows, 256 threads
    GDN_DECODE_VARIANT(4, 1),  // 3:  16 rows, 256 threads
    GDN_DECODE_VARIANT(2, 4),  // 4:  32 rows, 128 threads
    GDN_DECODE_VARIANT(1, 8),  // 5:  32 rows,  64 threads
    GDN_DECODE_VARIANT(1, 4),  // 6:  16 rows,  64 threads
    GDN_DECODE_VARIANT(1, 2),  // 7:   8 rows,  64 threads
    GDN_DECODE_VARIANT(2, 8),  // 8:  64 rows, 128 threads
    GDN_DECODE_VARIANT(1, 16), // 9:  64 rows,  64 threads
};
constexpr int kNumVariants = sizeof(kVariants) / sizeof(kVariants[0]);
constexpr int kNontemporalFlag = 16;

// Built-in tiling per batch size, from the MI355X sweep of every tiling at
// B = 1..512 (HIP-graph replay timing in 20-step graphs, 8 rotating states;
// the close calls confirmed by interleaved repeats): small batches want many
// small workgroups, B = 17..128 one wave streaming 64 rows (32 KiB in
// flight per wave), and beyond that -- many waves resident per CU for the
// whole launch -- 32-row workgroups of four waves (B = 256: 43.8 us against
// 45.3 us with one-wave 8-row ones; B = 512: 85.1 against 87.7 us);
// non-temporal state accesses win at every size.
int default_variant(int batch) {
  if (batch <= 4) return 3 + kNontemporalFlag;    // 16 rows, 256 threads
  if (batch <= 8) return 4 + kNontemporalFlag;    // 32 rows, 128 threads
  if (batch <= 16) return 6 + kNontemporalFlag;   // 16 rows,  64 threads
  if (batch <= 128) return 9 + kNontemporalFlag;  // 64 rows,  64 threads
  return 2 + kNontemporalFlag;                    // 32 rows, 256 threads
}

}  // namespace

int decode_launch(const gdn_bf16 *q, const gdn_bf16 *k, const gdn_bf16 *v, const float *state,
                  const float *A_log, const gdn_bf16 *a, const float *dt_bias, const gdn_bf16 *b,
                  float scale, gdn_bf16 *output, float *new_state, int batch, void *stream,
                  int variant, const Heads &H, const char *what) {
  clear_error();
  if (int rc = check_decode_args(q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state,
                                 batch, 1, H, what))
    return rc;
  if (batch == 0) return GDN_OK;

  // The built-in tiling depends on the number of state rows, counted in
  // batch rows of the reference layout (8 v-heads).
  if (variant < 0) variant = default_variant(static_cast<int>((static_cast<long long>(batch) * H.v + kHV - 1) / kHV));
  const int nt = (variant & kNontemporalFlag) ? 1 : 0;
  const int vi = variant & (kNontemporalFlag - 1);
  if (vi >= kNumVariants) return fail(GDN_ERR_INVALID, "%s: unknown variant %d", what, variant);
  const DecodeVariant &cfg = kVariants[vi];
  const int rows = 4 * cfg.waves * cfg.passes;
  const long long blocks = static_cast<long long>(batch) * H.v * (kDV / rows);
  if (blocks > 0x7fffffffLL) return fail(GDN_ERR_INVALID, "%s: batch too large", what);
  decode_fn fn = state ? cfg.with_state[nt] : cfg.no_state[nt];
  hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(blocks)), dim3(64 * cfg.waves), 0,
                     static_cast<hipStream_t>(stream), q, k, v, state, A_log, a, dt_bias, b,
                     scale, output, new_state, H);
  return check_launch(what);
}

}  // namespace gdn

extern "C" int gdn_decode_fwd(const gdn_bf16 *q, const gdn_bf16 *k, const gdn_bf16 *v,
                              const float *state, const float *A_log, const gdn_bf16 *a,
                              const float *dt_bias, const gdn_bf16 *b, float scale,
                              gdn_bf16 *output, float *new_state, int batch, void *stream) {
  return gdn::decode_launch(q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state, batch,
                            stream, -1, gdn::Heads{gdn::kHQK, gdn::kHV, gdn::kHV / gdn::kHQK},
                            "gdn_decode_fwd");
}

extern "C" int gdn_decode_fwd_variant(const gdn_bf16 *q, const gdn_bf16 *k, const gdn_bf16 *v,
                                      const float *state, const float *A_log, const gdn_bf16 *a,
                                      const float *dt_bias, const gdn_bf16 *b, float scale,
                                      gdn_bf16 *output, float *new_state, int batch, void *stream,
                                      int variant) {
  return gdn::decode_launch(q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state, batch,
                            stream, variant, gdn::Heads{gdn::kHQK, gdn::kHV, gdn::kHV / gdn::kHQK},
                            "gdn_decode_fwd");
}
