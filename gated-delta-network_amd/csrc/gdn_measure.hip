// Measurement support: an HBM streaming copy in the decode kernel's access
// pattern, the practical ceiling a kernel that reads and writes each byte of a
// state once can reach at a given size (launch ramp included).
#include "gdn_device.h"
#include "gdn_host.h"

namespace gdn {

// One wave per workgroup, 32 KiB per workgroup: every load issued before the
// first store, non-temporal buffer accesses both ways (as
// decode_kernel<1, 16, *, true>).  Of the copy shapes measured (flat or
// buffer accesses, 1-32 vectors per lane, 64 or 256 threads, each cache
// policy) this one is the fastest: 10.7 us per 2 x 32 MiB in 200-launch
// graphs, against 12.0 us for the same shape through flat pointers.
constexpr int kCopyPerLane = 32;
constexpr size_t kCopyBlock = 64 * kCopyPerLane * sizeof(f32x4);

__global__ __launch_bounds__(64) void stream_copy_kernel(const f32x4 *__restrict__ src,
                                                         f32x4 *__restrict__ dst) {
  const size_t base = static_cast<size_t>(blockIdx.x) * (64 * kCopyPerLane);
  const auto rs = buf_rsrc(src + base, static_cast<uint32_t>(kCopyBlock));
  const auto rd = buf_rsrc(dst + base, static_cast<uint32_t>(kCopyBlock));
  f32x4 r[kCopyPerLane];
#pragma unroll
  for (int i = 0; i < kCopyPerLane; ++i)
    r[i] = buf_load16_nt(rs, static_cast<uint32_t>(threadIdx.x + 64 * i) * 16u);
  // every load before the first store (left alone, the compiler keeps only
  // 14 loads in flight to save registers: 11.9 us instead of 10.7 us)
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < kCopyPerLane; ++i)
    buf_store16_nt(rd, static_cast<uint32_t>(threadIdx.x + 64 * i) * 16u, r[i]);
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
                     static_cast<hipStream_t>(stream), static_cast<const gdn::f32x4 *>(src),
                     static_cast<gdn::f32x4 *>(dst));
  return gdn::check_launch("gdn_stream_copy");
}
