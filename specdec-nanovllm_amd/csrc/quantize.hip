// quantize.hip — symmetric int8 weight quantization for gfx950: the W8A16
// format's producer, `quantize_weight` (nanovllm/layers/quant.py:123-148) and
// `quantize_tensor` of the offline converter (scripts/quantize_int8.py:53-83).
//
// Per row n and group g (the whole row for per-channel, group_size columns
// for per-group), in fp32:
//   amax  = max |w|            scale = max(amax / 127, 1e-8)
//   q     = clamp(round_half_even(w / scale), -127, 127)   (int8)
// with the fp32 scale (the stored scale is then rounded to bf16, after q).
// One wave per (row, group): a pass for amax (wave max), a second pass over
// the same bytes (now in cache) for q. HBM-bound: N K elem_bytes read once
// from HBM, N K + 2 N G' written.
#include <math.h>

#include "sd_common.h"

namespace {

constexpr int kThreads = 256;

struct QuantParams {
  const void* w;
  int64_t ws;  // row stride (elements)
  int8_t* q;
  int64_t qs;
  uint16_t* scale;  // (N, groups) bf16, row-major
  int64_t N;
  int32_t K, G, groups;
};

// eight consecutive elements of a row as fp32
template <typename T> __device__ __forceinline__ void load8(const T* p, float v[8]);
template <> __device__ __forceinline__ void load8<float>(const float* p, float v[8]) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}
template <typename H>
__device__ __forceinline__ void load8_16(const uint16_t* p, float v[8]) {
  const sd::u32x4 a = sd::load16(p);
  const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = sd::from_bits<H>(static_cast<uint16_t>(w[e / 2] >> (16 * (e & 1))));
}
template <> __device__ __forceinline__ void load8<__bf16>(const __bf16* p, float v[8]) {
  load8_16<__bf16>(reinterpret_cast<const uint16_t*>(p), v);
}
template <> __device__ __forceinline__ void load8<_Float16>(const _Float16* p, float v[8]) {
  load8_16<_Float16>(reinterpret_cast<const uint16_t*>(p), v);
}

template <typename T>
__global__ __launch_bounds__(kThreads) void quantize_kernel(QuantParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6);
  if (item >= p.N * p.groups) return;
  const int64_t n = item / p.groups;
  const int g = static_cast<int>(item - n * p.groups);
  const T* row = static_cast<const T*>(p.w) + n * p.ws + static_cast<int64_t>(g) * p.G;
  float amax = 0.f;
  for (int e0 = lane * 8; e0 < p.G; e0 += 64 * 8) {
    float v[8];
    load8<T>(row + e0, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[e]));
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  const float scale = fmaxf(amax / 127.f, 1e-8f);
  int8_t* qrow = p.q + n * p.qs + static_cast<int64_t>(g) * p.G;
  for (int e0 = lane * 8; e0 < p.G; e0 += 64 * 8) {
    float v[8];
    load8<T>(row + e0, v);
    uint32_t w[2] = {0u, 0u};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float r = fminf(fmaxf(rintf(v[e] / scale), -127.f), 127.f);
      w[e / 4] |= (static_cast<uint32_t>(static_cast<int32_t>(r)) & 0xffu) << (8 * (e & 3));
    }
    *reinterpret_cast<uint2*>(qrow + e0) = make_uint2(w[0], w[1]);
  }
  if (lane == 0) p.scale[n * p.groups + g] = sd::to_bits<__bf16>(scale);
}

}  // namespace

extern "C" int sd_quantize_int8(const void* w, int64_t w_stride, int32_t dtype, int8_t* q,
                                int64_t q_stride, void* scale, int64_t N, int32_t K,
                                int32_t group_size, void* stream) {
  sd::clear_error();
  const int G = group_size > 0 ? group_size : K;
  if (N < 0 || K <= 0 || group_size < 0 || K % 8 || G % 8 || K % G ||
      (dtype != SD_BF16 && dtype != SD_F16 && dtype != SD_F32)) {
    sd::set_error("quantize_int8: need K and the group size multiples of 8, the group size "
                  "dividing K, dtype bf16/fp16/fp32 (N=%lld K=%d group=%d dtype=%d)",
                  (long long)N, K, group_size, dtype);
    return SD_ERR_UNSUPPORTED;
  }
  if (N == 0) return SD_OK;
  if (!w || !q || !scale) {
    sd::set_error("quantize_int8: null pointer argument");
    return SD_ERR_VALUE;
  }
  if (!sd::aligned16(w) || w_stride % 8 || (reinterpret_cast<uintptr_t>(q) & 7u) || q_stride % 8) {
    sd::set_error("quantize_int8: weight rows must be 16-byte aligned, int8 rows 8-byte aligned");
    return SD_ERR_UNSUPPORTED;
  }
  const int groups = K / G;
  const int64_t wgs = (N * groups + kThreads / 64 - 1) / (kThreads / 64);
  if (wgs > 0x7fffffff) {
    sd::set_error("quantize_int8: too many rows (%lld)", (long long)N);
    return SD_ERR_UNSUPPORTED;
  }
  QuantParams p{w, w_stride, q, q_stride, static_cast<uint16_t*>(scale), N, K, G, groups};
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(wgs));
  if (dtype == SD_BF16) hipLaunchKernelGGL(quantize_kernel<__bf16>, grid, dim3(kThreads), 0, st, p);
  else if (dtype == SD_F16) hipLaunchKernelGGL(quantize_kernel<_Float16>, grid, dim3(kThreads), 0, st, p);
  else hipLaunchKernelGGL(quantize_kernel<float>, grid, dim3(kThreads), 0, st, p);
  return sd::check_launch("quantize_int8");
}
