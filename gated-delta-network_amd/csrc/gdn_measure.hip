// Measurement support: an HBM streaming copy in the decode kernel's access
// pattern, the practical ceiling a kernel that reads and writes each byte of a
// state once can reach at a given size (launch ramp included).
#include "gdn_host.h"

namespace gdn {

typedef float f32x4v __attribute__((ext_vector_type(4)));

// One wave per workgroup, 32 KiB per workgroup: every load issued before the
// first store, non-temporal both ways (as decode_kernel<1, 16, *, true>).
constexpr int kCopyPerLane = 32;
constexpr size_t kCopyBlock = 64 * kCopyPerLane * sizeof(f32x4v);

__global__ __launch_bounds__(64) void stream_copy_kernel(const f32x4v *__restrict__ src,
                                                         f32x4v *__restrict__ dst) {
  const size_t base = static_cast<size_t>(blockIdx.x) * (64 * kCopyPerLane) + threadIdx.x;
  f32x4v r[kCopyPerLane];
#pragma unroll
  for (int i = 0; i < kCopyPerLane; ++i) r[i] = __builtin_nontemporal_load(src + base + 64 * i);
#pragma unroll
  for (int i = 0; i < kCopyPerLane; ++i) __builtin_nontemporal_store(r[i], dst + base + 64 * i);
}

}  // namespace gdn

extern "C" int gdn_stream_copy(const void *src, void *dst, size_t bytes, void *stream) {
  gdn::clear_error();
  if (!src || !dst) return gdn::fail(GDN_ERR_INVALID, "gdn_stream_copy: null pointer");
  if (!gdn::aligned(src, 16) || !gdn::aligned(dst, 16))
    return gdn::fail(GDN_ERR_INVALID, "gdn_stream_copy: buffers must be 16-byte aligned");
  if (bytes % gdn::kCopyBlock != 0)
    return gdn::fail(GDN_ERR_INVALID, "gdn_stream_copy: bytes=%zu is not a multiple of %zu", bytes,
                     gdn::kCopyBlock);
  if (gdn::overlaps(src, bytes, dst, bytes))
    return gdn::fail(GDN_ERR_INVALID, "gdn_stream_copy: buffers overlap");
  const size_t blocks = bytes / gdn::kCopyBlock;
  if (blocks == 0) return GDN_OK;
  if (blocks > 0x7fffffffu) return gdn::fail(GDN_ERR_INVALID, "gdn_stream_copy: too large");
  hipLaunchKernelGGL(gdn::stream_copy_kernel, dim3(static_cast<unsigned>(blocks)), dim3(64), 0,
                     static_cast<hipStream_t>(stream), static_cast<const gdn::f32x4v *>(src),
                     static_cast<gdn::f32x4v *>(dst));
  return gdn::check_launch("gdn_stream_copy");
}
