/*
 * Sequential Gated DeltaNet prefill recurrence in C -- TEST INFRASTRUCTURE ONLY.
 *
 * Restates the per-token loop of reference/gdn_prefill_ref.py:71-89 (same op
 * order: old = g*S; old_v = k @ old; new_v = beta*v + (1-beta)*old_v;
 * S = old - k (x) old_v + k (x) new_v; o = scale * q @ S) so that the oracle
 * reaches the full benchmark sizes (up to 4 x 8192 tokens) in seconds.  The
 * gating (g, beta) is computed by the numpy oracle and passed in, so this file
 * holds only the recurrence.  Every (sequence, v-head) pair is independent and
 * runs on its own OpenMP thread.
 *
 * Inputs are float32 arrays (bf16 tensors arrive as their exact float values);
 * HQK q/k heads and HV v-heads (4 and 8 for the reference definitions; v-head
 * h reads q/k head h / (HV / HQK)):
 *   q, k      [T, HQK, 128]      v        [T, HV, 128]
 *   g, beta   [T, HV]            (multiplicative decay and sigmoid(b))
 *   state     [N, HV, 128, 128]  k-last ([V, K]); may be NULL (zeros)
 *   cu        [N + 1] int64
 * Outputs:
 *   o         [T, HV, 128] float32, NOT rounded to bf16 (the caller rounds)
 *   new_state [N, HV, 128, 128] float32 (zeros for a zero-length sequence,
 *             reference/gdn_prefill_ref.py:61-62)
 * use_f64 != 0 evaluates the recurrence in double precision instead.
 */
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define DK 128
#define DV 128

static void run_head_f32(const float *q, const float *k, const float *v, const float *g,
                         const float *beta, const float *s0, int64_t bos, int64_t eos,
                         int h, int HQK, int NHV, float scale, float *o, float *s_out) {
  /* S is held as [K][V] (the reference's transposed view, gdn_prefill_ref.py:65). */
  float *S = (float *)malloc(sizeof(float) * DK * DV);
  float old_v[DV], new_v[DV];
  const int hq = h / (NHV / HQK);
  for (int kk = 0; kk < DK; ++kk)
    for (int vv = 0; vv < DV; ++vv) S[kk * DV + vv] = s0 ? s0[vv * DK + kk] : 0.0f;
  for (int64_t t = bos; t < eos; ++t) {
    const float *qt = q + (t * HQK + hq) * DK;
    const float *kt = k + (t * HQK + hq) * DK;
    const float *vt = v + (t * NHV + h) * DV;
    const float gt = g[t * NHV + h], bt = beta[t * NHV + h];
    for (int i = 0; i < DK * DV; ++i) S[i] = gt * S[i];
    for (int vv = 0; vv < DV; ++vv) old_v[vv] = 0.0f;
    for (int kk = 0; kk < DK; ++kk)
      for (int vv = 0; vv < DV; ++vv) old_v[vv] += kt[kk] * S[kk * DV + vv];
    for (int vv = 0; vv < DV; ++vv) new_v[vv] = bt * vt[vv] + (1.0f - bt) * old_v[vv];
    for (int kk = 0; kk < DK; ++kk)
      for (int vv = 0; vv < DV; ++vv)
        S[kk * DV + vv] = S[kk * DV + vv] - kt[kk] * old_v[vv] + kt[kk] * new_v[vv];
    float *ot = o + (t * NHV + h) * DV;
    for (int vv = 0; vv < DV; ++vv) ot[vv] = 0.0f;
    for (int kk = 0; kk < DK; ++kk)
      for (int vv = 0; vv < DV; ++vv) ot[vv] += qt[kk] * S[kk * DV + vv];
    for (int vv = 0; vv < DV; ++vv) ot[vv] *= scale;
  }
  for (int vv = 0; vv < DV; ++vv)
    for (int kk = 0; kk < DK; ++kk) s_out[vv * DK + kk] = S[kk * DV + vv];
  free(S);
}

static void run_head_f64(const float *q, const float *k, const float *v, const float *g,
                         const float *beta, const float *s0, int64_t bos, int64_t eos,
                         int h, int HQK, int NHV, float scale, float *o, float *s_out) {
  double *S = (double *)malloc(sizeof(double) * DK * DV);
  double old_v[DV], new_v[DV], acc[DV];
  const int hq = h / (NHV / HQK);
  for (int kk = 0; kk < DK; ++kk)
    for (int vv = 0; vv < DV; ++vv) S[kk * DV + vv] = s0 ? (double)s0[vv * DK + kk] : 0.0;
  for (int64_t t = bos; t < eos; ++t) {
    const float *qt = q + (t * HQK + hq) * DK;
    const float *kt = k + (t * HQK + hq) * DK;
    const float *vt = v + (t * NHV + h) * DV;
    const double gt = g[t * NHV + h], bt = beta[t * NHV + h];
    for (int i = 0; i < DK * DV; ++i) S[i] = gt * S[i];
    for (int vv = 0; vv < DV; ++vv) old_v[vv] = 0.0;
    for (int kk = 0; kk < DK; ++kk)
      for (int vv = 0; vv < DV; ++vv) old_v[vv] += (double)kt[kk] * S[kk * DV + vv];
    for (int vv = 0; vv < DV; ++vv) new_v[vv] = bt * vt[vv] + (1.0 - bt) * old_v[vv];
    for (int kk = 0; kk < DK; ++kk)
      for (int vv = 0; vv < DV; ++vv)
        S[kk * DV + vv] = S[kk * DV + vv] - kt[kk] * old_v[vv] + kt[kk] * new_v[vv];
    for (int vv = 0; vv < DV; ++vv) acc[vv] = 0.0;
    for (int kk = 0; kk < DK; ++kk)
      for (int vv = 0; vv < DV; ++vv) acc[vv] += (double)qt[kk] * S[kk * DV + vv];
    float *ot = o + (t * NHV + h) * DV;
    for (int vv = 0; vv < DV; ++vv) ot[vv] = (float)(scale * acc[vv]);
  }
  for (int vv = 0; vv < DV; ++vv)
    for (int kk = 0; kk < DK; ++kk) s_out[vv * DK + kk] = (float)S[kk * DV + vv];
  free(S);
}

/* Threads of the (sequence, v-head) loop below for later calls from this
 * thread; n <= 0 restores every processor.  Returns the count in effect. */
int gdn_oracle_set_threads(int n) {
  omp_set_num_threads(n > 0 ? n : omp_get_num_procs());
  return omp_get_max_threads();
}

int gdn_oracle_prefill_seq(const float *q, const float *k, const float *v, const float *g,
                           const float *beta, const float *state, const int64_t *cu, int N,
                           int HQK, int NHV, float scale, float *o, float *new_state,
                           int use_f64) {
  if (N < 0 || HQK < 1 || NHV < 1 || NHV % HQK != 0) return -1;
  for (int s = 0; s < N; ++s)
    if (cu[s + 1] < cu[s]) return -1;
  memset(new_state, 0, sizeof(float) * (size_t)N * NHV * DV * DK);
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
  for (int s = 0; s < N; ++s) {
    for (int h = 0; h < NHV; ++h) {
      const int64_t bos = cu[s], eos = cu[s + 1];
      if (eos - bos <= 0) continue;
      const float *s0 = state ? state + ((size_t)s * NHV + h) * DV * DK : NULL;
      float *so = new_state + ((size_t)s * NHV + h) * DV * DK;
      if (use_f64)
        run_head_f64(q, k, v, g, beta, s0, bos, eos, h, HQK, NHV, scale, o, so);
      else
        run_head_f32(q, k, v, g, beta, s0, bos, eos, h, HQK, NHV, scale, o, so);
    }
  }
  return 0;
}
