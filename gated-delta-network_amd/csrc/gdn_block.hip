// Gated DeltaNet over short sequences in blocks of 16 tokens: one workgroup per
// (sequence, v-head) keeps the whole [V=128, K=128] f32 state in MFMA result
// tiles for the sequence and applies it block by block in the chunked (WY)
// form, the intra-block work included.
//
// Semantics: the per-token loop of reference/gdn_prefill_ref.py:71-89 (for
// one token, reference/gdn_decode_ref.py:60-81).  Per block of n <= 16
// tokens (g = log decay, G = its cumsum within the block, beta = sigmoid(b),
// S = the state at the block start, k-last: S[v][k]):
//   A     = strictly-lower(beta_i exp(G_i - G_j) k_i . k_j),  Ti = (I + A)^-1
//   W     = Ti diag(beta e^G) K,     U = Ti diag(beta) V
//   v_new = U - W S^T
//   o_i   = scale (exp(G_i) q_i S^T + sum_{j<=i} exp(G_i - G_j) (q_i . k_j) v_new_j)
//   S    <- exp(G_last) S + (diag(exp(G_last - G)) v_new)^T K
// the algebra of the chunk pipeline (gdn_prefill.hip) on 16-token blocks,
// fused into one launch.  It serves the token-sequential cases: decode of
// T > 1 tokens per row, and prefill of batches of short sequences.
//
// Work mapping (gfx950, wave64, 256 threads): wave w owns 32 state columns
// (or 16, when two workgroups share a (sequence, v-head): block_kernel<1>)
// for all 128 k, as result tiles of S^T (rows k, columns v: 4 consecutive k
// per lane), the B operand layout of an MFMA contracting over k (W S^T,
// q S^T; two k-tiles form one K=32 operand); v_new comes out of those
// products as tiles of 4 consecutive tokens per lane, the B operand of the
// update K^T v_new and of P v_new.  K^T and the token-major operands of W
// and U are read transposed out of the block's K and V rows in LDS
// (ds_read_b64_tr_b16).  Products whose error reaches the state use split
// bf16 (x = hi + lo), as in the chunk pipeline; P v_new uses single bf16
// operands, as the chunk pipeline's output (at large outputs, where only the
// relative 1e-2 bar applies, that costs up to ~0.4 %).
#include "gdn_device.h"
#include "gdn_host.h"

namespace gdn {

constexpr int kBlk = 16;        // tokens per block
constexpr int kBStride = 136;   // bf16 row stride of the q/k/v block tiles
constexpr int kBStrideA = 20;   // f32 row stride of the 16x16 A^T and Ti tiles
constexpr int kBStrideP = 24;   // bf16 row stride of P
// Pending decay factor below which step (7) folds the decay into the state
// tiles: 1, so every block's decay e^{G_last} < 1 is folded and the tiles
// hold the state itself, finite wherever the reference's f32 state is (a
// lazy S / c with c down to 2^-60 overflowed at |S| ~ 3e20: the all-0.5
// input of OPTIMIZATION_LOG.md:217-220 passes that at ~65 tokens).  c stays
// a run-time value, 1 or an unfolded exact-1 decay: with c a compile-time 1
// the compiler orders the block loop differently, measured 1.5 us slower at
// B=64 T=16 (16.4 -> 18.0 us).
constexpr float kFoldBelow = 1.f;
// Largest (sequence, v-head) count that runs as two 64-column workgroups.
constexpr long long kBlockHalfMaxPairs = 128;

// CV = 16-column state tiles per wave: 2 (the workgroup holds all 128
// columns) or 1 (two workgroups per (sequence, v-head), each 64 columns, for
// batches too small to fill the CUs: each repeats the intra-block work and
// owns half the state products).
template <int CV>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void block_kernel(const uint16_t *__restrict__ q, const uint16_t *__restrict__ k,
                  const uint16_t *__restrict__ v, const float *state,
                  const float *__restrict__ A_log, const uint16_t *__restrict__ a,
                  const float *__restrict__ dt_bias, const uint16_t *__restrict__ b,
                  const void *__restrict__ cu, int cu64, int N, int T, int fixed_len,
                  const int *__restrict__ enable, int *__restrict__ status, Heads H, float scale,
                  uint16_t *__restrict__ out, float *new_state) {
  __shared__ __align__(16) uint16_t sQ[kBlk * kBStride];
  __shared__ __align__(16) uint16_t sK[kBlk * kBStride];
  __shared__ __align__(16) uint16_t sV[kBlk * kBStride];
  __shared__ __align__(16) float sAt[kBlk * kBStrideA];
  __shared__ __align__(16) float sTi[kBlk * kBStrideA];
  __shared__ __align__(16) uint16_t sWh[kBlk * kBStride];  // W split: hi
  __shared__ __align__(16) uint16_t sWl[kBlk * kBStride];  //          lo
  __shared__ __align__(16) uint16_t sP[kBlk * kBStrideP];
  // by block parity: G, beta, e^G and e^(G_last - G) of each token
  __shared__ float sG[2][kBlk], sBeta[2][kBlk], sEG[2][kBlk], sED[2][kBlk];

  const int half = CV == 2 ? 0 : static_cast<int>(blockIdx.x & 1u);
  const int pair = CV == 2 ? static_cast<int>(blockIdx.x) : static_cast<int>(blockIdx.x >> 1);
  const int h = pair % H.v, s = pair / H.v;
  const int col0 = 64 * half + 16 * CV * __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g = lane >> 4, q4 = 4 * g, kg = 8 * g;
  const int hq = h / H.ratio;

  // The path flag and the sequence's bounds, loaded together (one wait).
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
    if (status != nullptr && h == 0 && half == 0 && threadIdx.x == 0)
      status[s] = cu_status_bits(lo, hi, T);
  } else {
    bos = s * fixed_len;
    len = fixed_len;
  }
  bos = __builtin_amdgcn_readfirstlane(bos);
  len = __builtin_amdgcn_readfirstlane(len);

  // The state as result tiles of S^T: St[kt][vi] holds S[v][k] at
  // k = 16 kt + q4 + r, v = 32 wave + 16 vi + r16.
  // The state is read once and written once: non-temporal accesses, as in
  // the decode kernel (B=64 T=8 decode 19.1 -> 16.3 us; 64x16 prefill over
  // rotating state sets 29.6 -> 24.5 us).
  const size_t sbase = (static_cast<size_t>(s) * H.v + h) * kDV * kDK;
  f32x4 St[8][CV];
  const uint32_t qk_stride = static_cast<uint32_t>(H.qk) * (kDK * 2);
  const uint32_t v_stride = static_cast<uint32_t>(H.v) * (kDV * 2);
  // The inputs of a block -- this thread's 16 bytes of its q, k and v rows
  // (row tid / 16; rows past the sequence read zero through the descriptors'
  // range) and, in wave 0, the raw gates of token `lane` -- are loaded one
  // block ahead of use.
  struct BlockIn {
    u32x4 q, k, v;
    uint16_t a, b;
  };
  const int row = tid >> 4, c16 = tid & 15;
  const float rate = expf(A_log[h]), dtb = dt_bias[h];
  auto load_block = [&](int t0, BlockIn &x) {
    const int n = len - t0 < kBlk ? len - t0 : kBlk;  // <= 0 past the end: all zero
    const uint32_t nn = n > 0 ? static_cast<uint32_t>(n) : 0u;
    const int start = bos + t0;
    const size_t qk0 = (static_cast<size_t>(start) * H.qk + hq) * kDK;
    const auto rq = buf_rsrc(q + qk0, nn * qk_stride);
    const auto rk = buf_rsrc(k + qk0, nn * qk_stride);
    const size_t v0 = (static_cast<size_t>(start) * H.v + h) * kDV;
    const auto rv = buf_rsrc(v + v0, nn * v_stride);
    x.q = buf_load16(rq, row * qk_stride + c16 * 16);
    x.k = buf_load16(rk, row * qk_stride + c16 * 16);
    x.v = buf_load16(rv, row * v_stride + c16 * 16);
    const size_t g0 = static_cast<size_t>(start) * H.v + h;
    const uint32_t gbytes = nn * static_cast<uint32_t>(H.v) * 2u;
    const uint32_t goff = static_cast<uint32_t>(lane) * static_cast<uint32_t>(H.v) * 2u;
    x.a = __builtin_amdgcn_raw_buffer_load_b16(buf_rsrc(a + g0, gbytes), goff, 0, 0);
    x.b = __builtin_amdgcn_raw_buffer_load_b16(buf_rsrc(b + g0, gbytes), goff, 0, 0);
  };
  // Gating of a block of n tokens (one wave, token `lane`): log decay,
  // in-block cumsum G, beta and the decay factors into the LDS buffer of the
  // block's parity.
  auto gate_block = [&](int n, uint16_t a_raw, uint16_t b_raw, int par) {
    const float gl = lane < n ? -rate * softplus20(bf16_to_f32(a_raw) + dtb) : 0.f;
    const float be = lane < n ? sigmoidf_(bf16_to_f32(b_raw)) : 0.f;
    float G = gl;
#pragma unroll
    for (int off = 1; off < kBlk; off <<= 1) {
      const float y = __shfl_up(G, off, kBlk);
      if (r16 >= off) G += y;
    }
    const float G_last = __shfl(G, kBlk - 1, kBlk);
    if (lane < kBlk) {
      sG[par][lane] = G;
      sBeta[par][lane] = be;
      sEG[par][lane] = expf(G);
      sED[par][lane] = expf(G_last - G);
    }
  };
  float c = 1.f;  // the state is c * St (step (7))
  // The first block's inputs are requested before the state: the loads
  // return in order, so steps (1)-(4), which do not read the state, need not
  // wait for all 64 KB of it.
  // No branch around these loads: the descriptors of an empty sequence, or
  // of a call without a state, have range 0 and their loads return zeros.
  // (With a branch, the compiler's load waits had to cover both paths, and
  // wave 0's gating of block 0 waited for the whole state.)
  BlockIn cur;
  load_block(0, cur);
  const auto rs = buf_rsrc(state != nullptr ? state + sbase : new_state + sbase,
                           state != nullptr && len > 0 ? kDV * kDK * 4u : 0u);
  // offset of S[col0 + 16 vi + r16][16 kt + q4]: per lane (r16, q4), per wave
  // (col0, vi) and constant (kt)
  const uint32_t lane_off = static_cast<uint32_t>(r16 * kDK + q4) * 4u;
#pragma unroll
  for (int kt = 0; kt < 8; ++kt)
#pragma unroll
    for (int vi = 0; vi < CV; ++vi)
      St[kt][vi] = buf_load16_nt(rs, lane_off + 64u * kt,
                                 static_cast<uint32_t>((col0 + 16 * vi) * kDK) * 4u);

  if (len > 0 && wave == 0) gate_block(len < kBlk ? len : kBlk, cur.a, cur.b, 0);
  for (int t0 = 0; t0 < len; t0 += kBlk) {
    const int n = len - t0 < kBlk ? len - t0 : kBlk;
    const int start = bos + t0;
    const int par = (t0 / kBlk) & 1;
    const float *bG = sG[par], *bBeta = sBeta[par], *bEG = sEG[par], *bED = sED[par];

    // (1) this block's q, k, v rows into LDS (its gates are there already);
    //     the next block's inputs requested.
    *reinterpret_cast<u32x4 *>(&sQ[row * kBStride + c16 * 8]) = cur.q;
    *reinterpret_cast<u32x4 *>(&sK[row * kBStride + c16 * 8]) = cur.k;
    *reinterpret_cast<u32x4 *>(&sV[row * kBStride + c16 * 8]) = cur.v;
    if (t0 + kBlk < len) load_block(t0 + kBlk, cur);
    __syncthreads();

    // (2) A = strictly-lower(beta_i e^{G_i - G_j} K K^T) (wave 0), stored
    //     transposed: sAt[j][i] = A_ij.
    //     G_i - G_j <= 0 wherever an entry is kept (g <= 0); the clamp keeps
    //     the discarded entries finite.
    auto masked_qk = [&](const uint16_t *sX, f32x4 &e) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const u32x4 af = *reinterpret_cast<const u32x4 *>(&sX[r16 * kBStride + 32 * kk + kg]);
        const u32x4 bf = *reinterpret_cast<const u32x4 *>(&sK[r16 * kBStride + 32 * kk + kg]);
        acc = mfma_bf16(af, bf, acc);
      }
      const float Gj = bG[r16];
#pragma unroll
      for (int r = 0; r < 4; ++r) e[r] = expf(fminf(bG[q4 + r] - Gj, 0.f)) * acc[r];
    };
    if (wave == 0) {
      f32x4 e;
      masked_qk(sK, e);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = q4 + r, j = r16;
        sAt[j * kBStrideA + i] = i > j ? bBeta[i] * e[r] : 0.f;
      }
    }
    __syncthreads();

    // (3) wave 0: Ti = (I + A)^-1 by column-oriented forward substitution,
    //     lane j < 16 solving column j (each solved x_m is applied to all
    //     later rows at once, so the serial chain is one FMA per row);
    //     wave 1: P = mask_{j<=i}(e^{G_i - G_j} Q K^T); wave 2: the next
    //     block's gates.  Then every wave splits its state for step (5).
    if (wave == 0) {
      if (lane < kBlk) {
        float x[kBlk];
#pragma unroll
        for (int i = 0; i < kBlk; ++i) x[i] = i == lane ? 1.f : 0.f;
#pragma unroll
        for (int m = 0; m < kBlk - 1; ++m) {
          const float xm = x[m];
#pragma unroll
          for (int i = m + 1; i < kBlk; ++i) x[i] -= sAt[m * kBStrideA + i] * xm;
        }
#pragma unroll
        for (int i = 0; i < kBlk; ++i) sTi[i * kBStrideA + lane] = x[i];
      }
    } else if (wave == 1) {
      f32x4 e;
      masked_qk(sQ, e);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = q4 + r, j = r16;
        sP[i * kBStrideP + j] = f32_to_bf16((j <= i && i < n) ? e[r] : 0.f);
      }
    } else if (wave == 2 && t0 + kBlk < len) {
      const int n1 = len - t0 - kBlk < kBlk ? len - t0 - kBlk : kBlk;
      gate_block(n1, cur.a, cur.b, par ^ 1);
    }
    // The state split for the K=32 products of step (5): slot 8 g + e of
    // k-block kk is k = 32 kk + 4 g + e (e < 4) or 32 kk + 16 + 4 g + e - 4
    // (the k of two state tiles), the same map for the A operands.
    u32x4 Sh[4][CV], Sl[4][CV];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
      for (int vi = 0; vi < CV; ++vi) {
        u32x2 h0, l0, h1, l1;
        split4(St[2 * kk][vi], h0, l0);
        split4(St[2 * kk + 1][vi], h1, l1);
        Sh[kk][vi] = u32x4{h0[0], h0[1], h1[0], h1[1]};
        Sl[kk][vi] = u32x4{l0[0], l0[1], l1[0], l1[1]};
      }
    __syncthreads();

    // (4) W = Ti diag(beta e^G) K for the features 32 wave .. +31 (-> LDS, split)
    //     and U = Ti diag(beta) V for this wave's columns (registers).  One
    //     K=32 product each: slots 8 g + e carry Ti's hi part (e < 4) and lo
    //     part (e >= 4) of token 4 g + e mod 4 against the same K (V) entry
    //     twice, a transposed read of the rows.
    f32x4 U[CV];
    {
      const f32x4 ti = *reinterpret_cast<const f32x4 *>(&sTi[r16 * kBStrideA + q4]);
      f32x4 tw, tu;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float be = bBeta[q4 + e];
        tu[e] = ti[e] * be;
        tw[e] = ti[e] * be * bEG[q4 + e];
      }
      u32x2 twh, twl, tuh, tul;
      split4(tw, twh, twl);
      split4(tu, tuh, tul);
      const u32x4 twa = {twh[0], twh[1], twl[0], twl[1]}, tua = {tuh[0], tuh[1], tul[0], tul[1]};
#pragma unroll
      for (int vi = 0; vi < CV; ++vi) {  // U for this wave's state columns
        const int u0 = col0 + 16 * vi;
        const u32x2 vb = ds_read_tr16(&sV[(q4 + (r16 >> 2)) * kBStride + u0 + 4 * (r16 & 3)]);
        U[vi] = mfma_bf16(tua, u32x4{vb[0], vb[1], vb[0], vb[1]}, f32x4{0.f, 0.f, 0.f, 0.f});
      }
#pragma unroll
      for (int ft = 0; ft < 2; ++ft) {  // W for the features 32 wave .. +31 (all 128 per block)
        const int c0 = 32 * wave + 16 * ft;
        const u32x2 kb = ds_read_tr16(&sK[(q4 + (r16 >> 2)) * kBStride + c0 + 4 * (r16 & 3)]);
        const f32x4 w = mfma_bf16(twa, u32x4{kb[0], kb[1], kb[0], kb[1]}, f32x4{0.f, 0.f, 0.f, 0.f});
        // W as bf16 hi/lo (the A operands of step (5), split once here)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint32_t wb = __float_as_uint(w[r]) & 0xffff0000u;
          sWh[(q4 + r) * kBStride + c0 + r16] = static_cast<uint16_t>(wb >> 16);
          sWl[(q4 + r) * kBStride + c0 + r16] = f32_to_bf16(w[r] - __uint_as_float(wb));
        }
      }
    }
    __syncthreads();

    // (5) v_new = U - W S^T for this wave's columns (W and S split: three
    //     K=32 products per 32 k).
    f32x4 vn[CV];
    {
      f32x4 P0[CV], P1[CV], P2[CV];
#pragma unroll
      for (int vi = 0; vi < CV; ++vi) P0[vi] = P1[vi] = P2[vi] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int wo = r16 * kBStride + 32 * kk + q4;
        const u32x2 h0 = *reinterpret_cast<const u32x2 *>(&sWh[wo]);
        const u32x2 h1 = *reinterpret_cast<const u32x2 *>(&sWh[wo + 16]);
        const u32x2 l0 = *reinterpret_cast<const u32x2 *>(&sWl[wo]);
        const u32x2 l1 = *reinterpret_cast<const u32x2 *>(&sWl[wo + 16]);
        const u32x4 wh = {h0[0], h0[1], h1[0], h1[1]}, wl = {l0[0], l0[1], l1[0], l1[1]};
#pragma unroll
        for (int vi = 0; vi < CV; ++vi) {
          P0[vi] = mfma_bf16(wh, Sh[kk][vi], P0[vi]);
          P1[vi] = mfma_bf16(wh, Sl[kk][vi], P1[vi]);
          P2[vi] = mfma_bf16(wl, Sh[kk][vi], P2[vi]);
        }
      }
#pragma unroll
      for (int vi = 0; vi < CV; ++vi)
#pragma unroll
        for (int r = 0; r < 4; ++r) vn[vi][r] = U[vi][r] - c * ((P0[vi][r] + P1[vi][r]) + P2[vi][r]);
    }

    // (6) o = scale (e^{G_i} q_i S^T + P v_new) for this wave's columns.
    {
      f32x4 O[CV];
#pragma unroll
      for (int vi = 0; vi < CV; ++vi) O[vi] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const uint16_t *qrow = &sQ[r16 * kBStride + 32 * kk + q4];
        const u32x2 q0 = *reinterpret_cast<const u32x2 *>(qrow);
        const u32x2 q1 = *reinterpret_cast<const u32x2 *>(qrow + 16);
        const u32x4 qa = {q0[0], q0[1], q1[0], q1[1]};
#pragma unroll
        for (int vi = 0; vi < CV; ++vi) {
          O[vi] = mfma_bf16(qa, Sh[kk][vi], O[vi]);
          O[vi] = mfma_bf16(qa, Sl[kk][vi], O[vi]);
        }
      }
      float eg[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) eg[r] = c * bEG[q4 + r];
      const u32x2 pa = *reinterpret_cast<const u32x2 *>(&sP[r16 * kBStrideP + q4]);
      // rows past the block's n tokens fall outside the descriptor: dropped
      const uint32_t ostride = static_cast<uint32_t>(H.v) * kDV * 2u;
      const auto ro = buf_rsrc(out + (static_cast<size_t>(start) * H.v + h) * kDV,
                               static_cast<uint32_t>(n) * ostride);
#pragma unroll
      for (int vi = 0; vi < CV; ++vi) {
        // P v_new in a tile of its own, added by VALU: no accumulation chain
        // mixes the 16x16x32 and 16x16x16 MFMA shapes.
        const u32x2 vb = {pk_bf16(vn[vi][0], vn[vi][1]), pk_bf16(vn[vi][2], vn[vi][3])};
        const f32x4 pv = mfma16_bf16(pa, vb, f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int r = 0; r < 4; ++r) O[vi][r] = fmaf(O[vi][r], eg[r], pv[r]);
        const uint32_t vc2 = static_cast<uint32_t>(col0 + 16 * vi + r16) * 2u;
#pragma unroll
        for (int r = 0; r < 4; ++r)
          __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16(scale * O[vi][r]), ro,
                                                static_cast<uint32_t>(q4 + r) * ostride + vc2, 0, 0);
      }
    }

    // (7) S <- e^{G_last} S + K^T (D v_new), D = e^{G_last - G}: A = K^T rows
    //     (a transposed read of the K rows), B = D v_new split.  The tiles
    //     hold S / c: a pending factor cn = c e^{G_last} below kFoldBelow
    //     (every decay below 1, or NaN) is folded in, the tiles take
    //     cn and c returns to 1; otherwise the update is added as
    //     K^T (D v_new) / cn.
    {
      float cn = c * bEG[kBlk - 1];
      const bool rescale = !(cn >= kFoldBelow);
      if (rescale) {
#pragma unroll
        for (int kt = 0; kt < 8; ++kt)
#pragma unroll
          for (int vi = 0; vi < CV; ++vi)
#pragma unroll
            for (int r = 0; r < 4; ++r) St[kt][vi][r] *= cn;
        cn = 1.f;
      }
      const float inv = 1.f / cn;
      u32x4 dvb[CV];
#pragma unroll
      for (int vi = 0; vi < CV; ++vi) {
        f32x4 dv;
#pragma unroll
        for (int r = 0; r < 4; ++r) dv[r] = bED[q4 + r] * inv * vn[vi][r];
        u32x2 dvh, dvl;
        split4(dv, dvh, dvl);
        // one K=32 product per tile: slots 8 g + e pair K^T's token
        // 4 g + e mod 4 with D v_new's hi part (e < 4) and lo part (e >= 4)
        dvb[vi] = u32x4{dvh[0], dvh[1], dvl[0], dvl[1]};
      }
#pragma unroll
      for (int kt = 0; kt < 8; ++kt) {
        const u32x2 ka = ds_read_tr16(&sK[(q4 + (r16 >> 2)) * kBStride + 16 * kt + 4 * (r16 & 3)]);
        const u32x4 kaa = {ka[0], ka[1], ka[0], ka[1]};
#pragma unroll
        for (int vi = 0; vi < CV; ++vi) St[kt][vi] = mfma_bf16(kaa, dvb[vi], St[kt][vi]);
      }
      c = cn;
    }
    __syncthreads();  // the block's LDS tiles are free for the next block
  }

  // Final state c St; all zeros for a zero-length sequence
  // (gdn_prefill_ref.py:61-62).  Flat non-temporal stores: through the
  // descriptor they cost ~0.5 us more per call (B=64 T=16 decode 15.8 ->
  // 16.5 us).
#pragma unroll
  for (int kt = 0; kt < 8; ++kt)
#pragma unroll
    for (int vi = 0; vi < CV; ++vi) {
      f32x4 x = St[kt][vi];
#pragma unroll
      for (int r = 0; r < 4; ++r) x[r] *= c;
      const int vc = col0 + 16 * vi + r16;
      __builtin_nontemporal_store(
          x, reinterpret_cast<f32x4 *>(new_state + sbase + vc * kDK + 16 * kt + q4));
    }
  // A packed batch: rows outside every sequence get zeros.
  if (cu != nullptr) zero_uncovered_rows(out, cu, cu64, N, T, H.v, blockIdx.x, gridDim.x);
}

int block_launch(const uint16_t *q, const uint16_t *k, const uint16_t *v, const float *state,
                 const float *A_log, const uint16_t *a, const float *dt_bias, const uint16_t *b,
                 const void *cu, int cu64, int num_seqs, int T, int fixed_len, const int *enable,
                 int *status, const Heads &H, float scale, uint16_t *out, float *new_state,
                 hipStream_t stream, const char *what) {
  const long long pairs = static_cast<long long>(num_seqs) * H.v;
  if (pairs > 0x3fffffffLL) return fail(GDN_ERR_INVALID, "%s: too many sequences for one launch", what);
  if (pairs == 0) return GDN_OK;
  // Two workgroups of 64 columns per (sequence, v-head) while that still
  // leaves every workgroup a CU of its own (kBlockHalfMaxPairs), one of 128
  // columns otherwise.
  if (pairs <= kBlockHalfMaxPairs)
    hipLaunchKernelGGL(block_kernel<1>, dim3(static_cast<unsigned>(2 * pairs)), dim3(256), 0, stream,
                       q, k, v, state, A_log, a, dt_bias, b, cu, cu64, num_seqs, T, fixed_len, enable, status, H,
                       scale, out, new_state);
  else
    hipLaunchKernelGGL(block_kernel<2>, dim3(static_cast<unsigned>(pairs)), dim3(256), 0, stream,
                       q, k, v, state, A_log, a, dt_bias, b, cu, cu64, num_seqs, T, fixed_len, enable, status, H,
                       scale, out, new_state);
  return check_launch(what);
}

}  // namespace gdn
