// w8a16.hip — W8A16 weight-only linear (int8 weights, fp16/bf16 activations)
// for gfx950.
//
//   y[m, n] = scale[n] * sum_k x[m, k] * w[n, k]  (+ bias[n])      per channel
//   y[m, n] = sum_g scale[n, g] * sum_{k in g} x[m, k] * w[n, k]  (+ bias)  per group
//
// Same contract as `int8_linear` / `_int8_dequant_gemm_kernel`
// (nanovllm/layers/quant.py:165-310): the int8 weight is read once from HBM
// and converted to 16-bit floats in registers (never written back), products
// accumulate in fp32, the per-channel scale multiplies the fp32 accumulator
// after the K loop (quant.py:220-222). Per-group scales multiply each group's
// fp32 partial sum (the reference instead rounds w * scale to bf16 before the
// dot, quant.py:210-214; both are within bf16/fp16 output tolerance of
// dequantize-then-matmul).
//
// Tiling: the weight is the MFMA A operand (16 rows n x 32 k), the activation
// the B operand (32 k x 16 rows m; M < 16 leaves lanes zero), so each lane
// streams 16 contiguous int8 of one weight row per 64-k step — one 16-byte
// load, 1 KB per wave instruction. A workgroup = 4 wave64s sharing NT 16-row
// tiles and splitting K four ways; `sgrid` workgroups split K further for
// narrow layers (N = 1024) and a reduce kernel sums their fp32 partials.
//
// int8 -> fp16: (b ^ 0x80) in the low byte under exponent byte 0x64 is the
// fp16 value 1024 + b + 128, exact; subtracting 1152 (packed fp16) gives b.
// int8 -> bf16: v_cvt_f32_ubyte of (b ^ 0x80) minus 128 is b as fp32, whose
// upper half is the exact bf16 (|b| <= 127 needs 7 mantissa bits).
#include "sd_common.h"

namespace {

using sd::f32x4;
using sd::u32x4;

constexpr int kThreads = 256;
constexpr int kWaves = 4;

struct W8Params {
  const uint16_t* x;
  int64_t xs;
  const int8_t* w;
  int64_t ws;
  const void* scale;
  int32_t scale_dtype;
  int32_t group;  // 0: per channel
  const uint16_t* bias;
  uint16_t* y;
  int64_t ys;
  int32_t M, N, K;
  int32_t nks;    // K / 64
  int32_t sgrid;  // workgroups along K
  float* part;    // [sgrid][M][N] fp32 partial sums when sgrid > 1
};

__device__ __forceinline__ float load_scale(const void* s, int dtype, int64_t i) {
  if (dtype == SD_F32) return static_cast<const float*>(s)[i];
  const uint16_t b = static_cast<const uint16_t*>(s)[i];
  return dtype == SD_BF16 ? sd::from_bits<__bf16>(b) : sd::from_bits<_Float16>(b);
}

// 8 int8 (two dwords) -> 8 x 16-bit floats in MFMA operand order.
template <typename T> __device__ __forceinline__ u32x4 dequant8(uint32_t w0, uint32_t w1);

template <> __device__ __forceinline__ u32x4 dequant8<_Float16>(uint32_t w0, uint32_t w1) {
  const uint32_t u0 = w0 ^ 0x80808080u, u1 = w1 ^ 0x80808080u;
  const sd::f16x2 off = {static_cast<_Float16>(1152.f), static_cast<_Float16>(1152.f)};
  u32x4 r;
  r.x = __builtin_bit_cast(uint32_t,
                           __builtin_bit_cast(sd::f16x2, __builtin_amdgcn_perm(0x64646464u, u0, 0x04010400u)) - off);
  r.y = __builtin_bit_cast(uint32_t,
                           __builtin_bit_cast(sd::f16x2, __builtin_amdgcn_perm(0x64646464u, u0, 0x04030402u)) - off);
  r.z = __builtin_bit_cast(uint32_t,
                           __builtin_bit_cast(sd::f16x2, __builtin_amdgcn_perm(0x64646464u, u1, 0x04010400u)) - off);
  r.w = __builtin_bit_cast(uint32_t,
                           __builtin_bit_cast(sd::f16x2, __builtin_amdgcn_perm(0x64646464u, u1, 0x04030402u)) - off);
  return r;
}

__device__ __forceinline__ uint32_t bf16_pair(uint32_t u, int lo_byte) {
  const float a = static_cast<float>((u >> (8 * lo_byte)) & 0xffu) - 128.f;
  const float b = static_cast<float>((u >> (8 * lo_byte + 8)) & 0xffu) - 128.f;
  return __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, b), __builtin_bit_cast(uint32_t, a),
                               0x07060302u);
}

template <> __device__ __forceinline__ u32x4 dequant8<__bf16>(uint32_t w0, uint32_t w1) {
  const uint32_t u0 = w0 ^ 0x80808080u, u1 = w1 ^ 0x80808080u;
  u32x4 r;
  r.x = bf16_pair(u0, 0);
  r.y = bf16_pair(u0, 2);
  r.z = bf16_pair(u1, 0);
  r.w = bf16_pair(u1, 2);
  return r;
}

template <typename T, int MT, int NT, bool PER_GROUP>
__global__ __launch_bounds__(kThreads) void w8a16_kernel(W8Params p) {
  constexpr int U = MT == 1 ? 4 : (MT == 2 ? 2 : 1);  // 64-k steps loaded per batch
  __shared__ __attribute__((aligned(16))) float red[kWaves - 1][NT * MT * 4][64];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int lr = lane & 15, lg = lane >> 4;
  const int n0 = blockIdx.x * NT * 16;
  const int sg = blockIdx.y;
  const int m0 = blockIdx.z * MT * 16;

  const int parts = kWaves * p.sgrid;
  const int part = sg * kWaves + wave;
  const int ks = static_cast<int>(static_cast<int64_t>(part) * p.nks / parts);
  const int ke = static_cast<int>(static_cast<int64_t>(part + 1) * p.nks / parts);

  const int8_t* wp[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int n = min(n0 + nt * 16 + lr, p.N - 1);  // rows past N: read a valid row, drop result
    wp[nt] = p.w + static_cast<int64_t>(n) * p.ws + lg * 16;
  }
  const uint16_t* xp[MT];
  bool xok[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = m0 + mt * 16 + lr;
    xok[mt] = m < p.M;
    xp[mt] = p.x + static_cast<int64_t>(min(m, p.M - 1)) * p.xs + lg * 16;
  }

  f32x4 acc[NT][MT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto steps = [&](auto nstep, int kk) {
    constexpr int S = decltype(nstep)::value;
    u32x4 wv[S][NT];
    u32x4 xv[S][MT][2];
#pragma unroll
    for (int u = 0; u < S; ++u) {
      const int64_t k0 = static_cast<int64_t>(kk + u) * 64;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) wv[u][nt] = sd::load16(wp[nt] + k0);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if (xok[mt]) {
          xv[u][mt][0] = sd::load16(xp[mt] + k0);
          xv[u][mt][1] = sd::load16(xp[mt] + k0 + 8);
        } else {
          xv[u][mt][0] = u32x4{0u, 0u, 0u, 0u};
          xv[u][mt][1] = u32x4{0u, 0u, 0u, 0u};
        }
      }
    }
#pragma unroll
    for (int u = 0; u < S; ++u) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const u32x4 a0 = dequant8<T>(wv[u][nt].x, wv[u][nt].y);  // k = 16 lg + 0..7
        const u32x4 a1 = dequant8<T>(wv[u][nt].z, wv[u][nt].w);  // k = 16 lg + 8..15
        if constexpr (!PER_GROUP) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            acc[nt][mt] = sd::Elem<T>::mfma(a0, xv[u][mt][0], acc[nt][mt]);
            acc[nt][mt] = sd::Elem<T>::mfma(a1, xv[u][mt][1], acc[nt][mt]);
          }
        } else {
          const int grp = static_cast<int>((static_cast<int64_t>(kk + u) * 64) / p.group);
          const int ng = p.K / p.group;
          float sc[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int n = min(n0 + nt * 16 + lg * 4 + i, p.N - 1);
            sc[i] = load_scale(p.scale, p.scale_dtype, static_cast<int64_t>(n) * ng + grp);
          }
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            f32x4 t = {0.f, 0.f, 0.f, 0.f};
            t = sd::Elem<T>::mfma(a0, xv[u][mt][0], t);
            t = sd::Elem<T>::mfma(a1, xv[u][mt][1], t);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[nt][mt][i] += t[i] * sc[i];
          }
        }
      }
    }
  };

  int kk = ks;
  for (; kk + U <= ke; kk += U) steps(std::integral_constant<int, U>{}, kk);
  for (; kk < ke; ++kk) steps(std::integral_constant<int, 1>{}, kk);

  // ---- reduce the four K slices of this workgroup
  if (wave > 0) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[wave - 1][(nt * MT + mt) * 4 + i][lane] = acc[nt][mt][i];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int w = 0; w < kWaves - 1; ++w) acc[nt][mt][i] += red[w][(nt * MT + mt) * 4 + i][lane];

  // ---- lane holds y^T[n = n0 + 16 nt + 4 lg + i][m = m0 + 16 mt + lr]
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = m0 + mt * 16 + lr;
    if (m >= p.M) continue;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int nb = n0 + nt * 16 + lg * 4;
      if (nb >= p.N) continue;
      if (p.sgrid > 1) {
        float* dst = p.part + (static_cast<int64_t>(sg) * p.M + m) * p.N;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (nb + i < p.N) dst[nb + i] = acc[nt][mt][i];
        continue;
      }
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int n = min(nb + i, p.N - 1);
        float s = PER_GROUP ? 1.f : load_scale(p.scale, p.scale_dtype, n);
        v[i] = acc[nt][mt][i] * s + (p.bias ? sd::from_bits<T>(p.bias[n]) : 0.f);
      }
      uint16_t* dst = p.y + static_cast<int64_t>(m) * p.ys + nb;
      if (nb + 3 < p.N && (reinterpret_cast<uintptr_t>(dst) & 7u) == 0) {
        *reinterpret_cast<uint2*>(dst) = make_uint2(sd::pack2<T>(v[0], v[1]), sd::pack2<T>(v[2], v[3]));
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (nb + i < p.N) dst[i] = sd::to_bits<T>(v[i]);
      }
    }
  }
}

// y[m, n] = T(scale[n] * sum_s part[s, m, n] + bias[n]) (scale = 1 for per group).
template <typename T>
__global__ __launch_bounds__(kThreads) void w8a16_reduce(W8Params p) {
  const int64_t total = static_cast<int64_t>(p.M) * p.N;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * kThreads) {
    const int m = static_cast<int>(i / p.N), n = static_cast<int>(i - static_cast<int64_t>(m) * p.N);
    float a = 0.f;
    for (int s = 0; s < p.sgrid; ++s) a += p.part[static_cast<int64_t>(s) * total + i];
    const float sc = p.group == 0 ? load_scale(p.scale, p.scale_dtype, n) : 1.f;
    const float v = a * sc + (p.bias ? sd::from_bits<T>(p.bias[n]) : 0.f);
    p.y[static_cast<int64_t>(m) * p.ys + n] = sd::to_bits<T>(v);
  }
}

struct W8Plan {
  int MT, NT, sgrid, mblocks;
};

W8Plan make_plan(int64_t M, int64_t N, int64_t K) {
  W8Plan pl;
  pl.MT = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  pl.mblocks = static_cast<int>((M + pl.MT * 16 - 1) / (pl.MT * 16));
  const int64_t nr = (N + 15) / 16;
  pl.NT = nr >= 4 * 1024 ? 4 : (nr >= 2 * 1024 ? 2 : 1);
  const int64_t wgs = (nr + pl.NT - 1) / pl.NT * pl.mblocks;
  const int64_t nks = K / 64;
  int64_t sg = (1024 + wgs - 1) / wgs;
  const int64_t sg_max = nks / kWaves > 0 ? nks / kWaves : 1;  // >= 1 step per wave
  if (sg > sg_max) sg = sg_max;
  if (sg < 1) sg = 1;
  pl.sgrid = static_cast<int>(sg);
  return pl;
}

template <typename T, int MT, int NT, bool PG>
void launch_k(const W8Params& p, dim3 grid, hipStream_t st) {
  hipLaunchKernelGGL((w8a16_kernel<T, MT, NT, PG>), grid, dim3(kThreads), 0, st, p);
}

template <typename T, bool PG>
void launch_mt(const W8Params& p, const W8Plan& pl, dim3 grid, hipStream_t st) {
  switch (pl.MT * 8 + pl.NT) {
    case 1 * 8 + 1: launch_k<T, 1, 1, PG>(p, grid, st); break;
    case 1 * 8 + 2: launch_k<T, 1, 2, PG>(p, grid, st); break;
    case 1 * 8 + 4: launch_k<T, 1, 4, PG>(p, grid, st); break;
    case 2 * 8 + 1: launch_k<T, 2, 1, PG>(p, grid, st); break;
    case 2 * 8 + 2: launch_k<T, 2, 2, PG>(p, grid, st); break;
    case 2 * 8 + 4: launch_k<T, 2, 4, PG>(p, grid, st); break;
    case 4 * 8 + 1: launch_k<T, 4, 1, PG>(p, grid, st); break;
    case 4 * 8 + 2: launch_k<T, 4, 2, PG>(p, grid, st); break;
    default: launch_k<T, 4, 4, PG>(p, grid, st); break;
  }
}

template <typename T>
int launch_all(const W8Params& p, const W8Plan& pl, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>((p.N + pl.NT * 16 - 1) / (pl.NT * 16)), pl.sgrid,
                  pl.mblocks);
  if (p.group == 0) launch_mt<T, false>(p, pl, grid, st);
  else launch_mt<T, true>(p, pl, grid, st);
  int rc = sd::check_launch("w8a16 main");
  if (rc != SD_OK || pl.sgrid <= 1) return rc;
  const int64_t total = static_cast<int64_t>(p.M) * p.N;
  int64_t blocks = (total + kThreads - 1) / kThreads;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL((w8a16_reduce<T>), dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0,
                     st, p);
  return sd::check_launch("w8a16 reduce");
}

}  // namespace

extern "C" size_t sd_w8a16_workspace_size(int64_t M, int64_t N, int64_t K, int32_t group_size) {
  (void)group_size;
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  const W8Plan pl = make_plan(M, N, K);
  if (pl.sgrid <= 1) return 0;
  return static_cast<size_t>(pl.sgrid) * M * N * sizeof(float);
}

extern "C" int sd_w8a16_linear(const void* x, int64_t x_stride_m, const int8_t* w,
                               int64_t w_stride_n, const void* scale, int32_t scale_dtype,
                               int32_t group_size, const void* bias, void* y, int64_t y_stride_m,
                               int64_t M, int64_t N, int64_t K, int32_t dtype, void* workspace,
                               size_t workspace_bytes, void* stream) {
  sd::clear_error();
  if (M < 0 || N <= 0 || K <= 0 || group_size < 0) {
    sd::set_error("w8a16: invalid sizes M=%lld N=%lld K=%lld group=%d", (long long)M,
                  (long long)N, (long long)K, group_size);
    return SD_ERR_VALUE;
  }
  if (M == 0) return SD_OK;
  if (!x || !w || !scale || !y) {
    sd::set_error("w8a16: null pointer argument");
    return SD_ERR_VALUE;
  }
  if (dtype != SD_BF16 && dtype != SD_F16) {
    sd::set_error("w8a16: activation dtype must be bf16 or f16");
    return SD_ERR_UNSUPPORTED;
  }
  if (scale_dtype != SD_BF16 && scale_dtype != SD_F16 && scale_dtype != SD_F32) {
    sd::set_error("w8a16: scale dtype must be bf16, f16 or f32");
    return SD_ERR_UNSUPPORTED;
  }
  if (K % 64 != 0) {
    sd::set_error("w8a16: K must be a multiple of 64, got %lld", (long long)K);
    return SD_ERR_UNSUPPORTED;
  }
  if (group_size != 0 && (group_size % 64 != 0 || K % group_size != 0)) {
    sd::set_error("w8a16: group_size must be a multiple of 64 dividing K (got %d, K=%lld)",
                  group_size, (long long)K);
    return SD_ERR_UNSUPPORTED;
  }
  if (M > (1ll << 30) || N > (1ll << 30) || K > (1ll << 30)) {
    sd::set_error("w8a16: dimensions too large");
    return SD_ERR_UNSUPPORTED;
  }
  if (!sd::aligned16(x) || !sd::aligned16(w) || x_stride_m % 8 != 0 || w_stride_n % 16 != 0) {
    sd::set_error("w8a16: x and w rows must be 16-byte aligned");
    return SD_ERR_UNSUPPORTED;
  }
  const W8Plan pl = make_plan(M, N, K);
  const size_t need = pl.sgrid > 1 ? static_cast<size_t>(pl.sgrid) * M * N * sizeof(float) : 0;
  if (need > 0 && (!workspace || workspace_bytes < need || !sd::aligned16(workspace))) {
    sd::set_error("w8a16: workspace of %zu bytes (16-byte aligned) required, got %zu", need,
                  workspace ? workspace_bytes : (size_t)0);
    return SD_ERR_WORKSPACE;
  }
  W8Params p;
  p.x = static_cast<const uint16_t*>(x);
  p.xs = x_stride_m;
  p.w = w;
  p.ws = w_stride_n;
  p.scale = scale;
  p.scale_dtype = scale_dtype;
  p.group = group_size;
  p.bias = static_cast<const uint16_t*>(bias);
  p.y = static_cast<uint16_t*>(y);
  p.ys = y_stride_m;
  p.M = static_cast<int32_t>(M);
  p.N = static_cast<int32_t>(N);
  p.K = static_cast<int32_t>(K);
  p.nks = static_cast<int32_t>(K / 64);
  p.sgrid = pl.sgrid;
  p.part = need > 0 ? static_cast<float*>(workspace) : nullptr;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == SD_BF16) return launch_all<__bf16>(p, pl, st);
  return launch_all<_Float16>(p, pl, st);
}
