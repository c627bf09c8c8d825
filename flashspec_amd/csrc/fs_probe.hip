// Measurement helpers: a plain streaming read of one device buffer, and a streaming 2:1 copy (read
// 2n bytes, write n).  Their rates on the same GPU are the practical HBM ceilings that the decode
// kernels' reads and the quantizers' fp16-in / int8-out traffic are compared against (the published
// 8 TB/s is a peak no access pattern reaches).  No counterpart in the reference.
#include "fs_paged.h"

namespace fs {

// Grid-stride non-temporal 16-byte loads, one per lane per step: the fastest plain read
// measured on MI355X (256 MiB, 2048 workgroups of 256 lanes: 7.08 TB/s against 6.4 TB/s with
// cached loads; 2 loads in flight per lane or 512/1024-lane workgroups were no faster).  The
// XOR of every word read reaches memory only when it equals `magic`, which keeps the loads from
// being dropped while writing nothing in practice (and, if it ever matches, one word of the
// caller's `sink`).
__global__ void __launch_bounds__(256) stream_read_kernel(const uint4* __restrict__ src, int64_t n16,
                                                          unsigned* sink, unsigned magic) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  unsigned acc = 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) {
    const uint4 v = stream_load(src + i);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == magic) sink[0] = acc;
}

// Reads 16 bytes per lane per step (non-temporal, as the quantizers read their fp16 source) and
// writes 8 of them (the low byte pair of each word) to dst: the traffic of an fp16 -> int8 pass
// with no arithmetic.
__global__ void __launch_bounds__(256) stream_copy_half_kernel(const uint4* __restrict__ src, int64_t n16,
                                                               uint2* __restrict__ dst) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) {
    const uint4 v = stream_load(src + i);
    dst[i] = make_uint2(__builtin_amdgcn_perm(v.y, v.x, 0x05040100u), __builtin_amdgcn_perm(v.w, v.z, 0x05040100u));
  }
}

}  // namespace fs

using namespace fs;

extern "C" int fs_stream_copy_half(const void* src, int64_t src_bytes, void* dst, int blocks, void* stream) {
  if (!src || !dst) return set_error(FS_ERR_INVALID, "null tensor pointer");
  if (src_bytes <= 0 || src_bytes % 16 != 0)
    return set_error(FS_ERR_INVALID, "src_bytes must be a positive multiple of 16");
  if ((uintptr_t)src % 16 != 0 || (uintptr_t)dst % 8 != 0)
    return set_error(FS_ERR_INVALID, "src must be 16-byte and dst 8-byte aligned");
  if (blocks <= 0 || blocks > 65536) return set_error(FS_ERR_INVALID, "blocks must be in [1, 65536]");
  hipLaunchKernelGGL(stream_copy_half_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (const uint4*)src,
                     src_bytes / 16, (uint2*)dst);
  return check_launch("stream_copy_half_kernel");
}

extern "C" int fs_stream_read(const void* src, int64_t bytes, unsigned* sink, int blocks, void* stream) {
  if (!src || !sink) return set_error(FS_ERR_INVALID, "null tensor pointer");
  if (bytes <= 0 || bytes % 16 != 0) return set_error(FS_ERR_INVALID, "bytes must be a positive multiple of 16");
  if ((uintptr_t)src % 16 != 0) return set_error(FS_ERR_INVALID, "src must be 16-byte aligned");
  if (blocks <= 0 || blocks > 65536) return set_error(FS_ERR_INVALID, "blocks must be in [1, 65536]");
  hipLaunchKernelGGL(stream_read_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (const uint4*)src,
                     bytes / 16, sink, 0x9e3779b9u);
  return check_launch("stream_read_kernel");
}
