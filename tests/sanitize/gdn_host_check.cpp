// CPU driver of the library's host-side code (gated-delta-network_amd/csrc/
// gdn_args.cpp: argument checks, workspace layout, path planning) for the
// sanitizer build.  tests/test_host_sanitize.py compiles it together with
// gdn_args.cpp under -fsanitize=address,undefined and feeds it one call per
// line on stdin; it prints one result line per call.  No GPU, no HIP: the
// pointers are plain integers that are compared and never dereferenced.
//
//   decode  WHAT q k v state A_log a dt_bias b scale output new_state batch tokens hqk hv
//   multi   WHAT q k v state A_log a dt_bias b scale output new_state batch tokens hqk hv variant
//   prefill WHAT q k v state A_log a dt_bias b cu cu64 N T scale output new_state ws ws_bytes
//           variant rec_max rec_variant hqk hv
//   layout  T N hqk hv
//   plan    T N hqk hv variant rec_max rec_variant
//
// decode / multi / prefill print "rc<TAB>message" (the library's status and
// gdn_last_error text; multi adds the chosen kernel); layout prints
// "rc nt_max total"; plan prints "rc" and the PrefillPlan fields.
#include <stdio.h>
#include <string.h>

#include "gdn_args.h"

using namespace gdn;

template <class T>
static T *ptr(unsigned long long x) {
  return reinterpret_cast<T *>(static_cast<uintptr_t>(x));
}

static void print_status(int rc) { printf("%d\t%s\n", rc, last_error_text()); }

static void print_plan(int rc, const PrefillPlan &P) {
  printf("%d %d %d %d %d %d %d %lld %lld %lld %lld %d %d %d %lld\n", rc, P.sequential ? 1 : 0,
         P.seq_variant, P.choose, P.single ? 1 : 0, P.form, P.split_nt0, P.intra_grid, P.state_grid,
         P.split_grid, P.out_grid, P.intra_split ? 1 : 0, P.loop ? 1 : 0, P.self_index ? 1 : 0,
         P.early_grid);
}

int main() {
  static char line[8192];
  while (fgets(line, sizeof(line), stdin)) {
    char cmd[32], what[64];
    int n = 0;
    if (sscanf(line, "%31s%n", cmd, &n) != 1) continue;
    const char *rest = line + n;
    clear_error();
    if (!strcmp(cmd, "decode") || !strcmp(cmd, "multi")) {
      const bool multi = !strcmp(cmd, "multi");
      unsigned long long p[10];
      float scale;
      int batch, tokens, hqk, hv, variant = -1;
      const int got = sscanf(rest, "%63s %llu %llu %llu %llu %llu %llu %llu %llu %f %llu %llu %d %d %d %d %d",
                             what, &p[0], &p[1], &p[2], &p[3], &p[4], &p[5], &p[6], &p[7], &scale,
                             &p[8], &p[9], &batch, &tokens, &hqk, &hv, &variant);
      if (got != (multi ? 17 : 16)) {
        printf("parse error\n");
        return 2;
      }
      Heads H;
      int rc = make_heads(hqk, hv, what, H);
      if (rc == GDN_OK)
        rc = check_decode_args(ptr<const gdn_bf16>(p[0]), ptr<const gdn_bf16>(p[1]),
                               ptr<const gdn_bf16>(p[2]), ptr<const float>(p[3]),
                               ptr<const float>(p[4]), ptr<const gdn_bf16>(p[5]),
                               ptr<const float>(p[6]), ptr<const gdn_bf16>(p[7]), scale,
                               ptr<const gdn_bf16>(p[8]), ptr<const float>(p[9]), batch, tokens,
                               H, what);
      if (multi) {
        int kernel = -1;
        if (rc == GDN_OK)
          rc = plan_multi(ptr<const void>(p[0]), ptr<const void>(p[1]), ptr<const void>(p[2]), batch,
                          tokens, H, variant, what, &kernel);
        printf("%d\t%s\t%d\n", rc, last_error_text(), kernel);
      } else {
        print_status(rc);
      }
    } else if (!strcmp(cmd, "prefill")) {
      unsigned long long p[13], ws_bytes;
      float scale;
      int cu64, N, T, variant, rec_max, rec_variant, hqk, hv;
      if (sscanf(rest,
                 "%63s %llu %llu %llu %llu %llu %llu %llu %llu %llu %d %d %d %f %llu %llu %llu %llu "
                 "%d %d %d %d %d",
                 what, &p[0], &p[1], &p[2], &p[3], &p[4], &p[5], &p[6], &p[7], &p[8], &cu64, &N, &T,
                 &scale, &p[9], &p[10], &p[11], &ws_bytes, &variant, &rec_max, &rec_variant, &hqk,
                 &hv) != 23) {
        printf("parse error\n");
        return 2;
      }
      Heads H;
      PrefillLayout L;
      int rc = make_heads(hqk, hv, what, H);
      if (rc == GDN_OK)
        rc = check_prefill_args(ptr<const gdn_bf16>(p[0]), ptr<const gdn_bf16>(p[1]),
                                ptr<const gdn_bf16>(p[2]), ptr<const float>(p[3]),
                                ptr<const float>(p[4]), ptr<const gdn_bf16>(p[5]),
                                ptr<const float>(p[6]), ptr<const gdn_bf16>(p[7]),
                                ptr<const void>(p[8]), cu64, N, T, scale,
                                ptr<const gdn_bf16>(p[9]), ptr<const float>(p[10]),
                                ptr<const void>(p[11]), static_cast<size_t>(ws_bytes), variant,
                                rec_max, rec_variant, kNumRecTilings + 1, H, what, &L);
      if (rc == GDN_OK && N > 0) {
        PrefillPlan P;
        rc = plan_prefill(T, N, H, L, variant, rec_max, rec_variant, kNumRecTilings, what, P);
      }
      print_status(rc);
    } else if (!strcmp(cmd, "layout")) {
      int T, N, hqk, hv;
      if (sscanf(rest, "%d %d %d %d", &T, &N, &hqk, &hv) != 4) {
        printf("parse error\n");
        return 2;
      }
      Heads H;
      const int rc = make_heads(hqk, hv, "layout", H);
      if (rc != GDN_OK || T < 0 || N < 0) {
        printf("%d 0 0\n", rc != GDN_OK ? rc : GDN_ERR_INVALID);
      } else {
        const PrefillLayout L = prefill_layout(T, N, H);
        printf("0 %d %zu\n", L.nt_max, L.total);
      }
    } else if (!strcmp(cmd, "plan")) {
      int T, N, hqk, hv, variant, rec_max, rec_variant;
      if (sscanf(rest, "%d %d %d %d %d %d %d", &T, &N, &hqk, &hv, &variant, &rec_max,
                 &rec_variant) != 7) {
        printf("parse error\n");
        return 2;
      }
      Heads H;
      PrefillPlan P{};
      int rc = make_heads(hqk, hv, "plan", H);
      if (rc == GDN_OK) {
        const PrefillLayout L = prefill_layout(T, N, H);
        rc = plan_prefill(T, N, H, L, variant, rec_max, rec_variant, kNumRecTilings, "plan", P);
      }
      print_plan(rc, P);
    } else {
      printf("unknown command %s\n", cmd);
      return 2;
    }
    fflush(stdout);
  }
  return 0;
}
