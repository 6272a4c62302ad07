// Gated DeltaNet chunked prefill: C-ABI entry points (kernels to follow).
#include "gdn_device.h"
#include "gdn_host.h"

extern "C" size_t gdn_prefill_workspace_bytes(int total_tokens, int num_seqs) {
  (void)total_tokens;
  (void)num_seqs;
  return 0;
}

extern "C" int gdn_prefill_fwd(const gdn_bf16 *, const gdn_bf16 *, const gdn_bf16 *, const float *,
                               const float *, const gdn_bf16 *, const float *, const gdn_bf16 *,
                               const void *, int, int, int, float, gdn_bf16 *, float *, void *,
                               size_t, void *) {
  return gdn::fail(GDN_ERR_LAUNCH, "gdn_prefill_fwd: not available in this build");
}
