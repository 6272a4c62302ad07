// Device-side helpers shared by the GDN kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gdn_common.h"

namespace gdn {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// float -> bf16 bits, round to nearest even (gfx950 v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// Two floats -> packed bf16 pair (a in bits 0..15), one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  const f32x2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// Split of two floats into bf16 hi/lo pairs: hi keeps the top 16 bits of each
// (so x - hi is exact), lo is that remainder rounded to nearest even;
// x = hi + lo to ~2^-17 relative.
__device__ __forceinline__ void split2(float a, float b, uint32_t &hi, uint32_t &lo) {
  const uint32_t ua = __float_as_uint(a) & 0xffff0000u;
  const uint32_t ub = __float_as_uint(b) & 0xffff0000u;
  hi = (ua >> 16) | ub;
  lo = pk_bf16(a - __uint_as_float(ua), b - __uint_as_float(ub));
}

// The same split with hi rounded to nearest even (x - hi is still exact), so
// that hi is also x's bf16 value: one copy serves both the split products and
// a bf16 image of x.
__device__ __forceinline__ void split2_rne(float a, float b, uint32_t &hi, uint32_t &lo) {
  hi = pk_bf16(a, b);
  lo = pk_bf16(a - __uint_as_float(hi << 16), b - __uint_as_float(hi & 0xffff0000u));
}

// Data-parallel-primitive lane moves.  CTRL is a DPP control word:
//   0xB1 quad_perm[1,0,3,2] (lane ^ 1)   0x4E quad_perm[2,3,0,1] (lane ^ 2)
//   0x141 row_half_mirror (i <-> 7-i within 8 lanes)
//   0x140 row_mirror      (i <-> 15-i within 16 lanes)
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

// Lane j of each aligned group of 16 lanes (one DPP "row"), to every lane of
// the group: DPP row_newbcast:j (control 0x150 + j).  j must be a constant
// after unrolling.
__device__ __forceinline__ float row_bcast16(float x, int j) {
  switch (j) {
#define GDN_BCAST(J) \
  case J:            \
    return dpp<0x150 + J>(x);
    GDN_BCAST(0) GDN_BCAST(1) GDN_BCAST(2) GDN_BCAST(3) GDN_BCAST(4) GDN_BCAST(5) GDN_BCAST(6)
    GDN_BCAST(7) GDN_BCAST(8) GDN_BCAST(9) GDN_BCAST(10) GDN_BCAST(11) GDN_BCAST(12)
    GDN_BCAST(13) GDN_BCAST(14) GDN_BCAST(15)
#undef GDN_BCAST
    default:
      return x;
  }
}

// Sum over each aligned group of 16 lanes (one DPP "row"); every lane of the
// group receives the total.  Four DPP adds, no LDS traffic.
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp<0xB1>(x);
  x += dpp<0x4E>(x);
  x += dpp<0x141>(x);
  x += dpp<0x140>(x);
  return x;
}

// softplus with torch's threshold (x > 20 -> x), as F.softplus(beta=1, threshold=20).
__device__ __forceinline__ float softplus20(float x) {
  return x > 20.0f ? x : log1pf(expf(x));
}

// Log-space decay -exp(A_log) * softplus(a + dt_bias).
__device__ __forceinline__ float gdn_log_decay(float A_log, float a, float dt_bias) {
  return -expf(A_log) * softplus20(a + dt_bias);
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }

// cu_seqlens[i] (int32 or int64 on the device), clamped to [0, T] so that a
// malformed batch can never index outside the packed tensors.
__device__ __forceinline__ int load_cu(const void *cu, int is64, int i, int T) {
  long long x = is64 ? static_cast<const long long *>(cu)[i] : static_cast<const int *>(cu)[i];
  x = x < 0 ? 0 : x;
  return static_cast<int>(x > T ? T : x);
}

// cu_seqlens as given (no clamp), and the contract bits of sequence s from
// its bounds cu[s], cu[s+1]: bit 0 the bounds decrease, bit 1 one of them is
// outside [0, T].  Zero for a well-formed batch.
__device__ __forceinline__ long long raw_cu(const void *cu, int is64, int i) {
  return is64 ? static_cast<const long long *>(cu)[i] : static_cast<const int *>(cu)[i];
}
__device__ __forceinline__ int cu_status_bits(long long lo, long long hi, int T) {
  return (hi < lo ? 1 : 0) | ((lo < 0 || lo > T || hi < 0 || hi > T) ? 2 : 0);
}

// Token rows of a packed batch that no sequence covers -- [0, cu[0]) and
// [cu[N], T) -- get a zero output, as in the reference, which zero-fills its
// output and writes only the rows [cu[s], cu[s+1]) of each sequence
// (reference/gdn_prefill_ref.py:49-51,56-62).  Workgroup `wg` of `nwg` clears
// its share with 16-byte stores (out is 16-byte aligned; a token row is
// hv * 256 bytes).  A batch spanning [0, T), the usual case, costs two uniform
// loads and a compare.
// (covered_rows loads the bounds, zero_rows_outside fills: a kernel that
// must not wait for the loads at its end issues them at its start.)
struct CoveredRows {
  int lo, hi;
};
__device__ __forceinline__ CoveredRows covered_rows(const void *cu, int cu64, int N, int T) {
  const int lo = load_cu(cu, cu64, 0, T);
  const int hi = load_cu(cu, cu64, N, T);
  return CoveredRows{lo, hi < lo ? lo : hi};
}
__device__ __forceinline__ void zero_rows_outside(uint16_t *out, CoveredRows r, int T, int hv,
                                                  unsigned wg, unsigned nwg) {
  const int lo = r.lo, hi = r.hi;
  if (lo == 0 && hi == T) return;
  const size_t per_row = static_cast<size_t>(hv) * (kDV / 8);  // 16-byte units per token row
  const size_t head = static_cast<size_t>(lo) * per_row;
  const size_t total = head + static_cast<size_t>(T - hi) * per_row;
  const size_t step = static_cast<size_t>(nwg) * blockDim.x;
  for (size_t i = static_cast<size_t>(wg) * blockDim.x + threadIdx.x; i < total; i += step) {
    const size_t u = i < head ? i : i - head + static_cast<size_t>(hi) * per_row;
    *reinterpret_cast<uint4 *>(out + u * 8) = make_uint4(0u, 0u, 0u, 0u);
  }
}
__device__ __forceinline__ void zero_uncovered_rows(uint16_t *out, const void *cu, int cu64, int N,
                                                    int T, int hv, unsigned wg, unsigned nwg) {
  zero_rows_outside(out, covered_rows(cu, cu64, N, T), T, hv, wg, nwg);
}

// A batch of one sequence runs without a chunk table: its tokens are
// [cu[0], cu[1]) (clamped to [0, T]), read on the device by every kernel that
// needs them, so no host read of cu_seqlens is ever required.  cu == nullptr:
// the batch has a chunk table (more than one sequence).
struct OneSeq {
  const void *cu;
  int cu64, T;
};
__device__ __forceinline__ void one_seq_bounds(const OneSeq &o, int &bos, int &eos) {
  bos = load_cu(o.cu, o.cu64, 0, o.T);
  eos = load_cu(o.cu, o.cu64, 1, o.T);
  eos = eos < bos ? bos : eos;
}

// The XCD (accelerator complex die) the wave runs on: hardware register
// XCC_ID of gfx940 and later.  MI355X deals the workgroups of a launch
// round-robin over its 8 XCDs (workgroups i and i + 8 on one XCD; which XCD
// takes workgroup 0 varies from launch to launch), each with its own L2;
// stores of one XCD are seen by the other CUs of that XCD through its L2
// before any write-back.
__device__ __forceinline__ int xcc_id() {
  int x;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
  return x & 0xf;
}
// The XCD as the top byte of a progress word (never 0).
__device__ __forceinline__ int early_tag() { return (xcc_id() + 1) << 24; }

}  // namespace gdn

namespace gdn {

// ---------------------------------------------------------------------------
// MFMA (gfx950 v_mfma_f32_16x16x32_bf16) and the fragment conventions used by
// every prefill kernel.  For one 16x16 output tile D = A (16x32) * B (32x16):
//   A operand: lane l holds A[l & 15][8*(l >> 4) + e], e = 0..7 (8 bf16)
//   B operand: lane l holds B[8*(l >> 4) + e][l & 15]
//   D (4 f32): lane l holds D[4*(l >> 4) + r][l & 15], r = 0..3
// Only the pairing of A's and B's k-index matters for the sum, and both use
// the same (l >> 4, e) -> k map, so a fragment is always "8 consecutive k of
// one row of A" or "8 consecutive k of one column of B".
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x4 mfma_bf16(const u32x4 a, const u32x4 b, const f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Splits 8 floats into bf16 hi and lo parts with x = hi + lo + O(2^-17 |x|):
// hi keeps the top 16 bits (exact remainder x - hi), lo is the remainder
// rounded to nearest even.  Element e goes to bits [16e, 16e+16).
__device__ __forceinline__ void split8(const float *x, u32x4 &hi, u32x4 &lo) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t h, l;
    split2(x[2 * i], x[2 * i + 1], h, l);
    hi[i] = h;
    lo[i] = l;
  }
}

// Rounds 8 floats to bf16 (nearest even) and packs them.
__device__ __forceinline__ u32x4 pack8(const float *x) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = pk_bf16(x[2 * i], x[2 * i + 1]);
  return r;
}

// OCP fp8 (e4m3) through gfx950's scaled conversions (scale 1: the callers
// apply their own power-of-two scale).  pk4_fp8 packs four floats, element e
// in byte e (round to nearest even); fp8x8_to_bf16 widens eight such bytes
// (element e in byte e of d0:d1) to bf16, exactly: e4m3's 4 significant bits
// and exponent range fit bf16.
typedef short s16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pk4_fp8(float a, float b, float c, float d) {
  s16x2 o = {0, 0};
  o = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(o, a, b, 1.0f, false);
  o = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(o, c, d, 1.0f, true);
  return __builtin_bit_cast(uint32_t, o);
}
__device__ __forceinline__ u32x4 fp8x8_to_bf16(uint32_t d0, uint32_t d1) {
  u32x4 r;
  r[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d0, 1.0f, false));
  r[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d0, 1.0f, true));
  r[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d1, 1.0f, false));
  r[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d1, 1.0f, true));
  return r;
}

// Power-of-two scale for the fp8 low part of a bf16 split of values whose
// largest magnitude is m: with hi rounded to nearest, |x - hi| <= 2^-8 |x|
// < 2^(e-8) for m = f 2^e, f in [0.5, 1), so 2^s with s = 15 - e maps every
// low part below 2^7, inside e4m3's range (448), and keeps those within
// 2^-13 of the largest in its normal range.  Returns 2^s and sets *inv =
// 2^-s (s clamped to [-126, 126]: both normal floats; m = 0 gives 2^126).
__device__ __forceinline__ float fp8_lo_scale(float m, float *inv) {
  const int e = static_cast<int>((__float_as_uint(m) >> 23) & 0xffu) - 126;
  int s = 15 - e;
  s = s < -126 ? -126 : (s > 126 ? 126 : s);
  *inv = __uint_as_float(static_cast<uint32_t>(127 - s) << 23);
  return __uint_as_float(static_cast<uint32_t>(127 + s) << 23);
}

// Largest value over the wave (every lane receives it): DPP within each row
// of 16 lanes, then the four row results through readlane.
__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, dpp<0xB1>(x));
  x = fmaxf(x, dpp<0x4E>(x));
  x = fmaxf(x, dpp<0x141>(x));
  x = fmaxf(x, dpp<0x140>(x));
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Unpacks 8 bf16 (as produced by pack8 / loaded from memory) to floats.
__device__ __forceinline__ void unpack8(const u32x4 p, float *x) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = __uint_as_float(p[i] << 16);
    x[2 * i + 1] = __uint_as_float(p[i] & 0xffff0000u);
  }
}


// Buffer descriptor (gfx9 word 3 = 0x00020000: raw 32-bit records) over
// `bytes` bytes at a wave-uniform base.  Loads through it take the base in
// SGPRs and a 32-bit per-lane byte offset that never changes across chunks,
// so a prefetch loop needs no address registers: with 64-bit VGPR addresses
// the compiler recomputed them every chunk and, reusing registers of loads
// still in flight, had to wait for the newest prefetch set at the loop head.
// A load at or past `bytes` returns zero: the rows past the end of a chunk.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), static_cast<short>(0), bytes,
                                           0x00020000);
}
__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
}
// Streaming 16-byte accesses through a descriptor, cache policy nt (bit 1 of
// the instruction's cache-policy operand): for state read or written once
// (decode loads at B=64: ~1 % faster than flat non-temporal loads).
constexpr int kCachePolicyNt = 2;
__device__ __forceinline__ f32x4 buf_load16_nt(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0,
                                                                         kCachePolicyNt));
}
__device__ __forceinline__ void buf_store16_nt(__amdgpu_buffer_rsrc_t r, uint32_t byte_off,
                                               f32x4 x) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, x), r, byte_off, 0,
                                         kCachePolicyNt);
}
// 16-byte store through a descriptor with cache policy sc1 (bit 4: agent
// scope, written through past L2 as it goes): for the WY intra kernel's
// outputs, which the next kernel reads, so that the kernel does not end on
// an L2 write-back of them (1x8192 intra 20.9 -> 19.1 us; calls 1x1024 33.8
// -> 32.2 us, configs[3] 63.4 -> 62.2 us).
constexpr int kCachePolicySc1 = 16;
__device__ __forceinline__ void buf_store16_sc1(__amdgpu_buffer_rsrc_t r, uint32_t byte_off,
                                                u32x4 x) {
  __builtin_amdgcn_raw_buffer_store_b128(x, r, byte_off, 0, kCachePolicySc1);
}
// The same with a wave-uniform part of the offset in the instruction's
// scalar offset (one VGPR of per-lane offset serves many loads).
__device__ __forceinline__ f32x4 buf_load16_nt(__amdgpu_buffer_rsrc_t r, uint32_t lane_off,
                                               uint32_t uniform_off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, lane_off, uniform_off,
                                                                         kCachePolicyNt));
}
// One float at a wave-uniform address, as a vector load issued in program
// order with the fragments it belongs to.
__device__ __forceinline__ float buf_load_f32(const float *p) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(buf_rsrc(p, 4), 0u, 0, 0));
}

// Gating of token `lane` of a chunk of `len` tokens from `start` (v-head h):
// g = log decay, beta = sigmoid(b); both loads go through descriptors bounded
// at the chunk's end and are issued before any arithmetic; padding tokens
// (lane >= len) get g = beta = 0.
__device__ __forceinline__ void chunk_gates(int lane, int start, int len, int h, const Heads &H,
                                            const float *A_log, const uint16_t *a,
                                            const float *dt_bias, const uint16_t *b, float &gl,
                                            float &be) {
  const size_t base = static_cast<size_t>(start) * H.v + h;
  const uint32_t bytes = static_cast<uint32_t>(len) * static_cast<uint32_t>(H.v) * 2u;
  const uint32_t off = static_cast<uint32_t>(lane) * static_cast<uint32_t>(H.v) * 2u;
  const uint16_t ar = __builtin_amdgcn_raw_buffer_load_b16(buf_rsrc(a + base, bytes), off, 0, 0);
  const uint16_t br = __builtin_amdgcn_raw_buffer_load_b16(buf_rsrc(b + base, bytes), off, 0, 0);
  const float al = A_log[h], db = dt_bias[h];
  gl = lane < len ? gdn_log_decay(al, bf16_to_f32(ar), db) : 0.f;
  be = lane < len ? sigmoidf_(bf16_to_f32(br)) : 0.f;
}


typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// gfx950 ds_read_b64_tr_b16: within each group of 16 lanes, source lane s
// reads the four 16-bit values D[s][0..3] at its own LDS address and lane t
// receives D[4j + (t >> 2)][t & 3], j = 0..3 (pinned by an on-device probe
// of the instruction).  So with lane s of group g addressing row
// 8g + 4h + (s >> 2), column c0 + 4 (s & 3) of a row-major tile, lane t
// gets the tile's column c0 + t at rows 8g + 4h .. 8g + 4h + 3: half h of
// a transposed MFMA operand fragment.
__device__ __forceinline__ u32x2 ds_read_tr16(const uint16_t *p) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                       (lds_s16x4 *)(const_cast<uint16_t *>(p))));
}

// v_mfma_f32_16x16x16_bf16: A lane l holds A[l & 15][4*(l >> 4) + e], B lane l
// holds B[4*(l >> 4) + e][l & 15] (e = 0..3), D as for the 16x16x32 form.  D's
// rows 4*(l >> 4) + r are exactly B's k-rows, so a result tile feeds the next
// product as its B operand without leaving the lane.
__device__ __forceinline__ f32x4 mfma16_bf16(const u32x2 a, const u32x2 b, const f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                    __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
}

// Split of four floats into (hi, lo) bf16 pairs for the K=16 MFMA.
__device__ __forceinline__ void split4(const f32x4 x, u32x2 &hi, u32x2 &lo) {
  uint32_t h0, h1, l0, l1;
  split2(x[0], x[1], h0, l0);
  split2(x[2], x[3], h1, l1);
  hi = u32x2{h0, h1};
  lo = u32x2{l0, l1};
}

// acc += A * B with both operands split (hi*hi + hi*lo + lo*hi).
__device__ __forceinline__ f32x4 mfma16_x3(const u32x2 ah, const u32x2 al, const u32x2 bh,
                                           const u32x2 bl, f32x4 acc) {
  acc = mfma16_bf16(ah, bh, acc);
  acc = mfma16_bf16(ah, bl, acc);
  return mfma16_bf16(al, bh, acc);
}

}  // namespace gdn
