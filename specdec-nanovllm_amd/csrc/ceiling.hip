// ceiling.hip — the box's streaming-read ceiling, measured by the bench beside
// every HBM-bound kernel of this library.
//
// The reference quotes its kernels against the bandwidth its own GPU reaches on
// a plain streaming copy rather than the data-sheet figure
// (nanovllm/kernels/README.md:27-35). The kernels here read far more than they
// write, so the matching ceiling on MI355X is a streaming read: a grid-stride
// pass of 16-byte nontemporal loads over `bytes` of device memory, each lane
// one load in flight per iteration, every loaded word folded into a register
// that guards a store which is practically never taken (so the loads cannot be
// dropped). Many waves with one load each measured best on the box: 6 - 8
// workgroups of 256 threads per CU reached 6.9 - 7.2 TB/s over 155 MB - 1 GiB,
// against 5.5 - 6.6 TB/s with 2 - 8 loads in flight per lane.
#include "sd_common.h"

namespace {

__global__ __launch_bounds__(256) void stream_read_kernel(const sd::u32x4* __restrict__ p,
                                                          int64_t n16, uint32_t* sink) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  sd::u32x4 fold = {0u, 0u, 0u, 0u};
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n16; i += stride) {
    const sd::u32x4 v = __builtin_nontemporal_load(p + i);
    fold.x ^= v.x;
    fold.y ^= v.y;
    fold.z ^= v.z;
    fold.w ^= v.w;
  }
  const uint32_t f = fold.x ^ fold.y ^ fold.z ^ fold.w;
  if (f == 0x9E3779B9u && threadIdx.x == 0) sink[0] = f;
}

}  // namespace

extern "C" int sd_stream_read(const void* src, int64_t bytes, void* sink, int32_t workgroups,
                              void* stream) {
  sd::clear_error();
  if (!src || !sink || bytes < 16 || bytes % 16 != 0 || !sd::aligned16(src) ||
      (reinterpret_cast<uintptr_t>(sink) & 3u) != 0) {
    sd::set_error("stream_read: needs a 16-byte aligned source of a positive multiple of 16 "
                  "bytes and a 4-byte aligned sink (bytes=%lld)", (long long)bytes);
    return SD_ERR_VALUE;
  }
  if (bytes > (int64_t{1} << 40)) {
    sd::set_error("stream_read: at most 2^40 bytes (got %lld)", (long long)bytes);
    return SD_ERR_UNSUPPORTED;
  }
  int wg = workgroups;
  if (wg <= 0) wg = sd::device_cus() * 6;
  if (wg > (1 << 20)) wg = 1 << 20;
  hipLaunchKernelGGL(stream_read_kernel, dim3(static_cast<unsigned>(wg)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const sd::u32x4*>(src),
                     bytes / 16, static_cast<uint32_t*>(sink));
  return sd::check_launch("stream_read");
}
