// sd_common.h — shared device/host helpers for the gfx950 kernels.
//
// Conventions used by every kernel in this directory:
//  * wave64: `lane` = threadIdx.x & 63, `wave` = threadIdx.x >> 6;
//  * 16-byte global loads/stores (`u32x4`), LDS rows padded so that the
//    column reads of the MFMA operand gathers are bank-conflict free;
//  * MFMA v_mfma_f32_16x16x32_{bf16,f16} operand layout (CDNA4):
//      A (16 x 32):  lane l holds A[l % 16][8 * (l / 16) + j], j = 0..7
//      B (32 x 16):  lane l holds B[8 * (l / 16) + j][l % 16], j = 0..7
//      D (16 x 16):  lane l holds D[4 * (l / 16) + i][l % 16], i = 0..3
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <initializer_list>

#include "specdec_amd.h"

namespace sd {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- dtypes
// Element traits: `T` is the 16-bit storage type (__bf16 or _Float16).
template <typename T> struct Elem;
template <> struct Elem<__bf16> {
  typedef bf16x8 vec8;
  static __device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};
template <> struct Elem<_Float16> {
  typedef f16x8 vec8;
  static __device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                 __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

// fp32 -> T, round to nearest even, of the fp32 value itself. The empty asm
// keeps the compiler from folding the multiply-add that produced x into the
// conversion (v_fma_mix*_f16 rounds the exact a * b + c straight to fp16, one
// rounding where the source says two): without it the bits of an fp16 output
// near a rounding midpoint depend on which form the compiler picked for that
// output, so two kernels computing the same fp32 value could disagree.
// bf16 has no such fused form on gfx950 (v_cvt_pk_bf16_f32 takes the fp32
// value), so only the fp16 conversion carries the fence.
template <typename T> __device__ __forceinline__ T round16(float x) {
  if constexpr (sizeof(T) == 2 && !__is_same(T, __bf16)) asm("" : "+v"(x));
  return static_cast<T>(x);
}
// fp32 -> 16-bit storage bits, round to nearest even.
template <typename T> __device__ __forceinline__ uint16_t to_bits(float x) {
  return __builtin_bit_cast(uint16_t, round16<T>(x));
}
// Pack two fp32 into one dword of two 16-bit values (lo in bits 0..15), each
// rounded to nearest even (bf16: one v_cvt_pk_bf16_f32 for the pair).
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
template <typename T> __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  if constexpr (__is_same(T, __bf16))
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
  else
    return static_cast<uint32_t>(to_bits<T>(lo)) | (static_cast<uint32_t>(to_bits<T>(hi)) << 16);
}
template <typename T> __device__ __forceinline__ float from_bits(uint16_t b) {
  return static_cast<float>(__builtin_bit_cast(T, b));
}
// acc + a.lo * b.lo + a.hi * b.hi over two packed 16-bit values (v_dot2c_f32_*:
// the products are exact in fp32).
template <typename T> __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
  if constexpr (__is_same(T, __bf16))
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b),
                                           acc, false);
  else
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), acc, false);
}
// Split two fp32 values into 16-bit hi parts and 16-bit parts of the remainder:
// a = float(hi_a) + float(lo_a) to ~2^-17 relative (hi and lo each RNE).
template <typename T>
__device__ __forceinline__ void split_pack(float a, float b, uint32_t& hi, uint32_t& lo) {
  if constexpr (__is_same(T, __bf16)) {
    // a bf16 is the top half of its fp32: the rounded values are the packed
    // word's halves moved into place
    hi = pack2<T>(a, b);
    lo = pack2<T>(a - __uint_as_float(hi << 16), b - __uint_as_float(hi & 0xffff0000u));
  } else {
    const T ha = round16<T>(a), hb = round16<T>(b);
    hi = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, ha)) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, hb)) << 16);
    lo = pack2<T>(a - static_cast<float>(ha), b - static_cast<float>(hb));
  }
}

__device__ __forceinline__ u32x4 load16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
// Scalar (SMEM) load of a wave-uniform address that nothing writes while the
// kernel runs (block tables, lengths). It completes on lgkmcnt, so using the
// value never waits for the vector loads in flight — which a vector load of the
// same address would (vmcnt counts in order).
__device__ __forceinline__ int32_t load_scalar_i32(const int32_t* p) {
  int32_t v;
  asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p));
  return v;
}

// 16-byte load of data read once (KV cache, weights): the nontemporal hint
// keeps the stream from displacing reusable lines in the caches.
__device__ __forceinline__ u32x4 load16_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void store16(void* p, u32x4 v) {
  *reinterpret_cast<u32x4*>(p) = v;
}

// `keep ? off : 0` for a load offset, formed without a branch. The compiler
// turns a select whose operand is an address computation into a branch around
// it, and the join after such a branch copies the loaded registers, which waits
// for every vector load in flight (s_waitcnt vmcnt(0)): the prefetch issued one
// step earlier then lands before the next one is issued. An opaque mask keeps
// the select an AND; the offset (not the pointer) is masked so that the load
// stays a global one (a pointer rebuilt from an integer loads through the flat
// path, which the compiler also waits for in full).
__device__ __forceinline__ int64_t keep_or_zero(bool keep, int64_t off) {
  uint32_t m = keep ? ~0u : 0u;
  asm("" : "+v"(m));
  return static_cast<int64_t>(static_cast<uint64_t>(off) & ((static_cast<uint64_t>(m) << 32) | m));
}

// keep_or_zero for a 32-bit offset.
__device__ __forceinline__ uint32_t keep_or_zero32(bool keep, uint32_t off) {
  uint32_t m = keep ? ~0u : 0u;
  asm("" : "+v"(m));
  return off & m;
}

// Orders LDS traffic between the lanes of one wave (a wave-private LDS tile
// written by some lanes and read by others): a compiler barrier plus the
// wavefront-scope fences of the AMDGPU memory model.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Butterfly max/sum over the four lane groups that share `l % 16`.
__device__ __forceinline__ float max_over_groups(float v) {
  v = fmaxf(v, __shfl_xor(v, 16));
  v = fmaxf(v, __shfl_xor(v, 32));
  return v;
}
// The same with the byte addresses of lanes l ^ 16 and l ^ 32 formed once by
// the caller (ds_bpermute operands), for loops that exchange every step.
struct XorAddr {
  int a16, a32;
};
__device__ __forceinline__ XorAddr xor_addr() {
  const int l = threadIdx.x & 63;
  return XorAddr{(l ^ 16) << 2, (l ^ 32) << 2};
}
__device__ __forceinline__ float max_over_groups(float v, const XorAddr& x) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_ds_bpermute(x.a16, __float_as_int(v))));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_ds_bpermute(x.a32, __float_as_int(v))));
  return v;
}
__device__ __forceinline__ float sum_over_groups(float v) {
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

// Inclusive prefix sum over the 64 lanes of a wave with DPP moves (VALU
// latency, no LDS round trips): Hillis-Steele shifts by 1, 2, 4 and 8 inside
// each row of 16 lanes (lanes whose source is outside the row add 0), then lane
// 15's total added to row 1 and row 3 (row_bcast:15), then lane 31's total to
// rows 2 and 3 (row_bcast:31). Every lane must be active.
__device__ __forceinline__ int wave_inclusive_sum(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15 -> rows 1, 3
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31 -> rows 2, 3
  return x;
}

// v plus lane (DPP control CTRL)'s v; lanes whose source lane is outside its
// row add 0.
template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                          0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over each 32-lane half of the wave, the same value in all 32 lanes of the
// half (every step adds two lanes' values, which commute): xor 1 and xor 2
// inside quads, the mirrors inside 8 and 16 lanes, then the two 16-lane rows
// of the half swapped (v_permlane16_swap) and added. A half whose lanes are all
// inactive does not disturb the other.
__device__ __forceinline__ float half_wave_sum(float v) {
  v = dpp_add<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v = dpp_add<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v = dpp_add<0x141>(v);  // row_half_mirror
  v = dpp_add<0x140>(v);  // row_mirror
  const auto z = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, v),
                                                  __builtin_bit_cast(uint32_t, v), false, false);
  return __builtin_bit_cast(float, static_cast<uint32_t>(z[0])) +
         __builtin_bit_cast(float, static_cast<uint32_t>(z[1]));
}

// The xor butterfly `for (off = TOP; off > 0; off >>= 1) v += __shfl_xor(v, off)`
// (TOP 32 or 16; the whole wave active) without LDS, bit for bit: each step
// adds, in every lane l, v[l] and v[l ^ off] (a + b and b + a are the same
// float). xor 32 and xor 16 are v_permlane32_swap / v_permlane16_swap of v
// with itself (the two outputs of a lane are its own and its partner's
// value), xor 8 rotates each 16-lane row by 8. A row then repeats with period
// 8, so its rotation by 4 brings lane l ^ 4's value to lane l; xor 2 and xor 1
// are quad permutations.
template <int TOP>
__device__ __forceinline__ float xor_sum_down(float v) {
  static_assert(TOP == 32 || TOP == 16, "xor butterfly from lane distance 32 or 16");
  if constexpr (TOP == 32) {
    const auto z = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v),
                                                    __builtin_bit_cast(uint32_t, v), false, false);
    v = __builtin_bit_cast(float, static_cast<uint32_t>(z[0])) +
        __builtin_bit_cast(float, static_cast<uint32_t>(z[1]));
  }
  const auto z = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, v),
                                                  __builtin_bit_cast(uint32_t, v), false, false);
  v = __builtin_bit_cast(float, static_cast<uint32_t>(z[0])) +
      __builtin_bit_cast(float, static_cast<uint32_t>(z[1]));
  v = dpp_add<0x128>(v);  // row_ror:8
  v = dpp_add<0x124>(v);  // row_ror:4
  v = dpp_add<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v = dpp_add<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  return v;
}

// v of lane l (a wave-uniform l), as a uniform value
__device__ __forceinline__ float lane_value(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

// 2^x on the transcendental unit (v_exp_f32) without denormal fix-ups:
// results below 2^-126 flush to 0, 2^-inf = 0. Softmax weights only.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Add + RMSNorm of one row by the first 256 threads of a workgroup (every
// thread calls it; it synchronises the workgroup; threads past 256 hold no
// elements, so a larger workgroup gives the same bits): h = x (+ res) in fp32,
// out = bf16(bf16(h * rsqrt(mean(h^2) + eps)) * w), res_out = bf16(h) (when
// res_out). Thread t holds the 8-element chunks t, t + 256, ... (H <= 8192,
// H % 8 == 0); the sum of squares runs per thread over its chunks, then over
// the wave (xor shuffles 32 .. 1), then over the 4 waves in order, so any two
// callers produce the same bits. `red` holds 4 floats of LDS; `out` may be a
// global or an LDS row.
template <typename T>
__device__ __forceinline__ void add_rmsnorm_row(const uint16_t* x, const uint16_t* res,
                                                const uint16_t* w, int H, float eps, float* red,
                                                uint16_t* out, uint16_t* res_out) {
#pragma clang fp contract(off)
  constexpr int kChunks = 4;
  float v[kChunks][8];
  float ss = 0.f;
  // the weight's chunks load with the row's (one round trip, not one after the sum)
  u32x4 wq[kChunks];
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int e0 = (c * 256 + static_cast<int>(threadIdx.x)) * 8;
    wq[c] = threadIdx.x < 256 && e0 < H ? load16(w + e0) : u32x4{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int e0 = (c * 256 + static_cast<int>(threadIdx.x)) * 8;
    if (threadIdx.x < 256 && e0 < H) {
      const u32x4 a = load16(x + e0);
      const uint32_t aw[4] = {a.x, a.y, a.z, a.w};
      u32x4 b = {0u, 0u, 0u, 0u};
      if (res) b = load16(res + e0);
      const uint32_t bw[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float f = from_bits<T>(static_cast<uint16_t>(aw[i / 2] >> (16 * (i & 1))));
        if (res) f = f + from_bits<T>(static_cast<uint16_t>(bw[i / 2] >> (16 * (i & 1))));
        v[c][i] = f;
        ss += f * f;
      }
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0 && wave < 4) red[wave] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int wv = 0; wv < 4; ++wv) tot += red[wv];
  __syncthreads();  // red is free for the next row
  const float r = rsqrtf(tot / static_cast<float>(H) + eps);
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int e0 = (c * 256 + static_cast<int>(threadIdx.x)) * 8;
    if (threadIdx.x < 256 && e0 < H) {
      const u32x4 wv = wq[c];
      const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
      uint32_t o[4], ro[4];
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        const float w0 = from_bits<T>(static_cast<uint16_t>(ww[i / 2]));
        const float w1 = from_bits<T>(static_cast<uint16_t>(ww[i / 2] >> 16));
        const float n0 = static_cast<float>(round16<T>(v[c][i] * r));
        const float n1 = static_cast<float>(round16<T>(v[c][i + 1] * r));
        o[i / 2] = pack2<T>(n0 * w0, n1 * w1);
        ro[i / 2] = pack2<T>(v[c][i], v[c][i + 1]);
      }
      store16(out + e0, u32x4{o[0], o[1], o[2], o[3]});
      if (res_out) store16(res_out + e0, u32x4{ro[0], ro[1], ro[2], ro[3]});
    }
  }
}

// One wave, one 128-element head (lane l holds elements l and l + 64 as x0,
// x1): RMSNorm with the weight's elements w0, w1 (has_w false: none; the
// squares summed per lane, then xor steps 32 .. 1), then rotate-half RoPE with
// this lane's cos c and sin s of the position; returns the two outputs' 16-bit
// bits (lo: element l, hi: l + 64). Every operand arrives as a value, so the
// caller issues all of its loads before the reduction.
// Qwen3Attention's q_norm / k_norm then RotaryEmbedding.forward
// (nanovllm/models/qwen3.py:80-88, layers/rotary_embedding.py:6-48), every
// rounding of the eager module kept.
template <typename T>
__device__ __forceinline__ void head_norm_rope(float x0, float x1, bool has_w, float w0, float w1,
                                               float eps, float c, float s, uint16_t& lo,
                                               uint16_t& hi) {
#pragma clang fp contract(off)
  if (has_w) {
    float ss = x0 * x0 + x1 * x1;
    ss = xor_sum_down<32>(ss);  // the xor steps 32 .. 1
    const float r = rsqrtf(ss / 128.f + eps);
    x0 = static_cast<float>(round16<T>(static_cast<float>(round16<T>(x0 * r)) * w0));
    x1 = static_cast<float>(round16<T>(static_cast<float>(round16<T>(x1 * r)) * w1));
  }
  const float a = x0 * c, b = x1 * s;
  const float e = x1 * c, f = x0 * s;
  lo = to_bits<T>(a - b);
  hi = to_bits<T>(e + f);
}

// add_rmsnorm_row by one wave, in two passes over the row (sum of squares,
// then the outputs), with the same bits: the wave plays the 4 waves of the
// 256-thread form one after another (virtual thread 64 vw + lane holds the
// chunks c * 256 + 64 vw + lane, c = 0..3), adds each virtual wave's squares
// with the same xor steps, and the 4 wave sums in order. No LDS and no
// workgroup barrier, so the waves of a workgroup can normalise different rows
// at the same time.
template <typename T>
__device__ __forceinline__ void add_rmsnorm_row_wave(const uint16_t* x, const uint16_t* res,
                                                     const uint16_t* w, int H, float eps,
                                                     uint16_t* out, uint16_t* res_out) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  auto row_val = [&](const u32x4& a, const u32x4& b, int i) {
    const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, bw[4] = {b.x, b.y, b.z, b.w};
    float f = from_bits<T>(static_cast<uint16_t>(aw[i / 2] >> (16 * (i & 1))));
    if (res) f = f + from_bits<T>(static_cast<uint16_t>(bw[i / 2] >> (16 * (i & 1))));
    return f;
  };
  float tot = 0.f;
#pragma unroll
  for (int vw = 0; vw < 4; ++vw) {
    if (vw * 64 * 8 >= H) break;  // wave-uniform: no chunk of this virtual wave is in the row
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int e0 = (c * 256 + vw * 64 + lane) * 8;
      if (e0 < H) {
        const u32x4 a = load16(x + e0);
        const u32x4 b = res ? load16(res + e0) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float f = row_val(a, b, i);
          ss += f * f;
        }
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    tot += ss;
  }
  const float r = rsqrtf(tot / static_cast<float>(H) + eps);
#pragma unroll
  for (int vw = 0; vw < 4; ++vw) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int e0 = (c * 256 + vw * 64 + lane) * 8;
      if (e0 < H) {
        const u32x4 a = load16(x + e0);
        const u32x4 b = res ? load16(res + e0) : u32x4{0u, 0u, 0u, 0u};
        const u32x4 wv = load16(w + e0);
        const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
        uint32_t o[4], ro[4];
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
          const float v0 = row_val(a, b, i), v1 = row_val(a, b, i + 1);
          const float w0 = from_bits<T>(static_cast<uint16_t>(ww[i / 2]));
          const float w1 = from_bits<T>(static_cast<uint16_t>(ww[i / 2] >> 16));
          const float n0 = static_cast<float>(round16<T>(v0 * r));
          const float n1 = static_cast<float>(round16<T>(v1 * r));
          o[i / 2] = pack2<T>(n0 * w0, n1 * w1);
          ro[i / 2] = pack2<T>(v0, v1);
        }
        store16(out + e0, u32x4{o[0], o[1], o[2], o[3]});
        if (res_out) store16(res_out + e0, u32x4{ro[0], ro[1], ro[2], ro[3]});
      }
    }
  }
}

// add_rmsnorm_row_wave for NR rows of H <= 1024 elements at once (H % 8 == 0):
// rows r < nr exist, row r at x + r xs (res + r rs, out + r os, res_out +
// r ros). Lane l holds the 8-element chunks l and 64 + l of each row, the
// RMSNorm kernel's threads l and 64 + l (its waves 0 and 1; its waves 2 and 3
// hold no chunk of such a row and add zeros). Every load goes out before the
// first use, unconditionally (rows and columns clamped into the matrix, zeros
// selected past H), and the row stays in registers between the sum and the
// outputs; the wave sums are xor_sum_down's DPP steps. One round trip for all
// NR rows, where add_rmsnorm_row_wave waits per chunk and reads the row twice.
template <typename T, int NR>
__device__ __forceinline__ void add_rmsnorm_rows_wave(const uint16_t* x, int64_t xs,
                                                      const uint16_t* res, int64_t rs,
                                                      const uint16_t* w, int H, float eps, int nr,
                                                      uint16_t* out, int64_t os,
                                                      uint16_t* res_out, int64_t ros) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  u32x4 a[NR][2], b[NR][2], wq[2];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int64_t rc = min(r, nr - 1);
    const uint16_t* xr = x + rc * xs;
    const uint16_t* br = res ? res + rc * rs : xr;
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      const int e = min((v * 64 + lane) * 8, H - 8);
      a[r][v] = load16(xr + e);
      b[r][v] = load16(br + e);
    }
  }
#pragma unroll
  for (int v = 0; v < 2; ++v) wq[v] = load16(w + min((v * 64 + lane) * 8, H - 8));
  const bool has_res = res != nullptr;
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    float val[2][8];
    float tot = 0.f;
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      const bool ok = (v * 64 + lane) * 8 < H;
      const uint32_t aw[4] = {a[r][v].x, a[r][v].y, a[r][v].z, a[r][v].w};
      const uint32_t bw[4] = {b[r][v].x, b[r][v].y, b[r][v].z, b[r][v].w};
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float f = from_bits<T>(static_cast<uint16_t>(aw[i / 2] >> (16 * (i & 1))));
        const float g = from_bits<T>(static_cast<uint16_t>(bw[i / 2] >> (16 * (i & 1))));
        const float s = has_res ? f + g : f;
        val[v][i] = ok ? s : 0.f;
        ss += val[v][i] * val[v][i];
      }
      tot += xor_sum_down<32>(ss);  // the kernel's wave v
    }
    const float rn = rsqrtf(tot / static_cast<float>(H) + eps);
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      const int e0 = (v * 64 + lane) * 8;
      const uint32_t ww[4] = {wq[v].x, wq[v].y, wq[v].z, wq[v].w};
      uint32_t o[4], ro[4];
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        const float w0 = from_bits<T>(static_cast<uint16_t>(ww[i / 2]));
        const float w1 = from_bits<T>(static_cast<uint16_t>(ww[i / 2] >> 16));
        const float n0 = static_cast<float>(round16<T>(val[v][i] * rn));
        const float n1 = static_cast<float>(round16<T>(val[v][i + 1] * rn));
        o[i / 2] = pack2<T>(n0 * w0, n1 * w1);
        ro[i / 2] = pack2<T>(val[v][i], val[v][i + 1]);
      }
      if (e0 < H && r < nr) {
        store16(out + r * os + e0, u32x4{o[0], o[1], o[2], o[3]});
        if (res_out) store16(res_out + r * ros + e0, u32x4{ro[0], ro[1], ro[2], ro[3]});
      }
    }
  }
}

// SiluAndMul on 8 elements: bf16(bf16(silu(g)) * u) per element (T = the
// activation type), the eager module's roundings; g and u are 8 packed 16-bit
// values each. Shared by the SiLU kernel and the W8A16 activation path that
// fuses it, so both give the same bits.
// One element: the fp32 product before its final rounding to T.
template <typename T>
__device__ __forceinline__ float silu_mul1(float gv, float uv) {
#pragma clang fp contract(off)
  const float sv = static_cast<float>(round16<T>(gv / (1.f + expf(-gv))));
  return sv * uv;
}

template <typename T>
__device__ __forceinline__ u32x4 silu_mul8(u32x4 g, u32x4 u) {
  const uint32_t gw[4] = {g.x, g.y, g.z, g.w}, uw[4] = {u.x, u.y, u.z, u.w};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float r[2];
#pragma unroll
    for (int h = 0; h < 2; ++h)
      r[h] = silu_mul1<T>(from_bits<T>(static_cast<uint16_t>(gw[i] >> (16 * h))),
                          from_bits<T>(static_cast<uint16_t>(uw[i] >> (16 * h))));
    o[i] = pack2<T>(r[0], r[1]);
  }
  return u32x4{o[0], o[1], o[2], o[3]};
}

// LDS transpose read (ds_read_b64_tr_b16): within every 16-lane block, lane
// 4a + c receives 16-bit element c of the 8-byte chunks addressed by lanes
// a, a + 4, a + 8 and a + 12 of that block, in that order.
typedef short s16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint2 lds_read_tr16(const void* p) {
  const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(p));
  return __builtin_bit_cast(uint2, r);
}

// Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy
// as 1, 2, 3", SC 2011): counter (c0..c3), key (k0, k1), ten rounds. The
// fourth counter word names the stream: 0 sampling, 1 verify acceptance,
// 2 verify bonus.
__device__ __forceinline__ void philox(uint32_t c[4], uint32_t k0, uint32_t k1) {
  constexpr uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u;
  constexpr uint32_t W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = static_cast<uint64_t>(M0) * c[0];
    const uint64_t p1 = static_cast<uint64_t>(M1) * c[2];
    const uint32_t n0 = static_cast<uint32_t>(p1 >> 32) ^ c[1] ^ k0;
    const uint32_t n1 = static_cast<uint32_t>(p1);
    const uint32_t n2 = static_cast<uint32_t>(p0 >> 32) ^ c[3] ^ k1;
    const uint32_t n3 = static_cast<uint32_t>(p0);
    c[0] = n0;
    c[1] = n1;
    c[2] = n2;
    c[3] = n3;
    k0 += W0;
    k1 += W1;
  }
}

// --------------------------------------------------------------- host side
// Thread-local message of the last failure (returned by sd_last_error()).
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();
// Maps a pending HIP launch error into SD_ERR_HIP with `what` in the message.
int check_launch(const char* what);

// Compute units / LDS bytes per workgroup of the current device, cached per
// device id (safe to call from several host threads at once).
int device_cus();
int device_lds_per_block();

// Byte range [lo, hi) of a row-major 16-bit matrix (rows x width, row stride
// in elements); empty for a NULL pointer or no rows.
struct Span {
  uintptr_t lo, hi;
  bool overlaps(const Span& o) const { return lo < hi && o.lo < o.hi && lo < o.hi && o.lo < hi; }
};
inline Span span16(const void* p, int64_t rows, int64_t stride, int64_t width) {
  if (!p || rows <= 0 || width <= 0) return Span{0, 0};
  const int64_t st = stride > 0 ? stride : 0;
  const uintptr_t lo = reinterpret_cast<uintptr_t>(p);
  return Span{lo, lo + static_cast<uintptr_t>(((rows - 1) * st + width) * 2)};
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Strides (in elements) the entry points accept: |stride| <= 2^40 keeps every
// offset and product they form from the sizes they accept inside int64.
constexpr int64_t kMaxStride = int64_t(1) << 40;
inline bool strides_ok(std::initializer_list<int64_t> strides) {
  for (const int64_t st : strides)
    if (st < -kMaxStride || st > kMaxStride) return false;
  return true;
}

}  // namespace sd
