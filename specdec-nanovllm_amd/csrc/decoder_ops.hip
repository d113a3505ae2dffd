// decoder_ops.hip — the draft step's neighbours of the attention and linear
// kernels, for gfx950: the row-wise work of a Qwen3 decoder step that sits
// between the library's paged attention and W8A16 launches.
//
//   rmsnorm_kernel       RMSNorm.forward, with or without the residual add
//                        (nanovllm/layers/layernorm.py:16-47)
//   qk_norm_rope_kernel  per-head q/k RMSNorm then rotate-half RoPE, in place
//                        (models/qwen3.py:80-88, layers/rotary_embedding.py:6-48),
//                        optionally with store_kvcache of the finished k rows
//                        and of v (layers/attention.py:33-40)
//   silu_mul_kernel      SiluAndMul (layers/activation.py:6-11)
//   sample_partial_kernel / sample_merge_kernel
//                        Sampler: temperature + exponential-race (Gumbel-max)
//                        sampling, or greedy argmax (layers/sampler.py:6-12,
//                        spec_decode/draft_proposer.py:505-510), a row split
//                        over 4096-column workgroups and merged per row
//
// Rounding follows the modules' eager torch semantics: fp32 arithmetic, a
// 16-bit rounding wherever the module converts back to the activation dtype
// (`x.to(orig_dtype)`, each elementwise op on 16-bit tensors), and no fused
// multiply-add where the module has separate multiplies and adds.
#include <math.h>

#include "sd_common.h"

namespace {

constexpr int kThreads = 256;

template <typename T> __device__ __forceinline__ float ld(const uint16_t* p, int64_t i) {
  return sd::from_bits<T>(p[i]);
}

// ------------------------------------------------------------------ RMSNorm
// One workgroup per row; thread t holds 8-element chunks t, t + 256, ...
// (up to kChunks of them) in registers between the reduction and the writes,
// so out / residual_out may alias x / residual.
constexpr int kChunks = 4;  // hidden <= 8 * 256 * 4 = 8192

struct NormParams {
  const uint16_t* x;
  int64_t xs;
  const uint16_t* res;  // NULL: no residual add
  int64_t rs;
  const uint16_t* w;
  uint16_t* out;
  int64_t os;
  uint16_t* res_out;
  int64_t ros;
  int32_t H;
  float eps;
};

template <typename T>
__global__ __launch_bounds__(kThreads) void rmsnorm_kernel(NormParams p) {
  __shared__ float red[kThreads / 64];
  const int64_t row = blockIdx.x;
  sd::add_rmsnorm_row<T>(p.x + row * p.xs, p.res ? p.res + row * p.rs : nullptr, p.w, p.H, p.eps,
                         red, p.out + row * p.os,
                         p.res && p.res_out ? p.res_out + row * p.ros : nullptr);
}

// ----------------------------------------------------------- q/k norm + RoPE
// One wave per (token, head); lane l holds dims l and l + 64 of the 128, which
// are exactly the pair rotate-half mixes, so RoPE needs no lane exchange.
struct RopeParams {
  uint16_t* q;
  int64_t q_stok, q_shead;
  uint16_t* k;
  int64_t k_stok, k_shead;
  int64_t tokens;
  int32_t Hq, Hkv;
  const uint16_t* qw;  // (128,) q_norm weight, NULL: no norm
  const uint16_t* kw;
  float eps;
  const int64_t* pos;
  const float* cos_sin;  // (max_position, cs_stride): cos[0:64] | sin[64:128]
  int64_t cs_stride;
  int64_t max_pos;
  // store_kvcache of the finished k rows and of v (kc == NULL: none)
  const uint16_t* v;
  int64_t v_stok, v_shead;
  uint16_t* kc;
  uint16_t* vc;
  int64_t c_sblk, c_spos, c_shead;
  int64_t num_slots;  // num_blocks * block_size
  int32_t block_size;
  const int32_t* slot;
};

template <typename T>
__global__ __launch_bounds__(kThreads) void qk_norm_rope_kernel(RopeParams p) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * (kThreads / 64) +
                       __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int heads = p.Hq + p.Hkv;
  if (item >= p.tokens * heads) return;
  const int64_t t = item / heads;
  const int hd = static_cast<int>(item - t * heads);
  const bool is_q = hd < p.Hq;
  uint16_t* x = is_q ? p.q + t * p.q_stok + static_cast<int64_t>(hd) * p.q_shead
                     : p.k + t * p.k_stok + static_cast<int64_t>(hd - p.Hq) * p.k_shead;
  const uint16_t* w = is_q ? p.qw : p.kw;
  const bool store = p.kc && !is_q;  // k heads of a fused store_kvcache
  // Every load that depends on nothing else goes out first, unconditionally
  // (absent operands read a valid stand-in, never used): the position, the
  // slot, the head's two elements, the norm weight's and the value row's.
  // Then the cos / sin row at the position. Loads under branches or after the
  // reduction cost this small kernel one dependent round trip each.
  const uint16_t* wsrc = w ? w : x;
  const uint16_t* vsrc = store ? p.v + t * p.v_stok + static_cast<int64_t>(hd - p.Hq) * p.v_shead : x;
  // the token index in a VGPR: position and slot become vector loads, counted
  // in order with the rest (scalar loads return out of order, so the first use
  // of any kernel argument after them would wait for them)
  int64_t tv = t;
  asm volatile("" : "+v"(tv));
  const int32_t* ssrc = p.slot ? p.slot + tv : reinterpret_cast<const int32_t*>(p.pos + tv);
  const int64_t pos = p.pos[tv];
  const int64_t sl = *ssrc;
  const uint16_t xb0 = x[lane], xb1 = x[lane + 64];
  const uint16_t wb0 = wsrc[lane], wb1 = wsrc[lane + 64];
  const uint16_t vb0 = vsrc[lane], vb1 = vsrc[lane + 64];
  const bool rope = pos >= 0 && pos < p.max_pos;  // no cos/sin row: the head is left as it is
  const float* cs = p.cos_sin + (rope ? pos : 0) * p.cs_stride;
  const float c = cs[lane], sn = cs[64 + lane];
  // the row's cache slot (-1 or outside the pool: not written, as store_kvcache)
  uint16_t* kdst = nullptr;
  uint16_t* vdst = nullptr;
  if (store && sl >= 0 && sl < p.num_slots) {
    const int64_t blk = sl / p.block_size, off = sl - blk * p.block_size;
    const int64_t row = blk * p.c_sblk + off * p.c_spos + static_cast<int64_t>(hd - p.Hq) * p.c_shead;
    kdst = p.kc + row;
    vdst = p.vc + row;
    vdst[lane] = vb0;
    vdst[lane + 64] = vb1;
  }
  if (!rope) {
    if (kdst) {
      kdst[lane] = xb0;
      kdst[lane + 64] = xb1;
    }
    return;
  }
  uint16_t lo, hi;
  sd::head_norm_rope<T>(sd::from_bits<T>(xb0), sd::from_bits<T>(xb1), w != nullptr,
                        sd::from_bits<T>(wb0), sd::from_bits<T>(wb1), p.eps, c, sn, lo, hi);
  x[lane] = lo;
  x[lane + 64] = hi;
  if (kdst) {
    kdst[lane] = lo;
    kdst[lane + 64] = hi;
  }
}

// ----------------------------------------------------------------- SiLU * up
// out[m, i] = bf16(bf16(silu(g)) * u), g = x[m, i], u = x[m, width + i].
struct SiluParams {
  const uint16_t* x;
  int64_t xs;
  uint16_t* out;
  int64_t os;
  int64_t rows;
  int32_t width;
};

template <typename T>
__global__ __launch_bounds__(kThreads) void silu_mul_kernel(SiluParams p) {
#pragma clang fp contract(off)
  const int64_t chunks = p.width / 8;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (idx >= p.rows * chunks) return;
  const int64_t m = idx / chunks;
  const int e0 = static_cast<int>(idx - m * chunks) * 8;
  const sd::u32x4 g = sd::load16(p.x + m * p.xs + e0);
  const sd::u32x4 u = sd::load16(p.x + m * p.xs + p.width + e0);
  sd::store16(p.out + m * p.os + e0, sd::silu_mul8<T>(g, u));
}

// ------------------------------------------------------------------ sampling
struct SampleParams {
  const void* logits;
  int64_t ls;
  int32_t dtype;  // SD_BF16 / SD_F16 / SD_F32
  int32_t V;
  const float* temp;      // (rows,), NULL: greedy
  const int64_t* state;   // (2,) device: seed, offset; read only
  int64_t* out;
  float2* part;           // [rows][nslices] (best key, its index as int bits)
  int32_t nslices;
};

constexpr int kSampleThreads = 256;
constexpr int kSampleGroups = 4;  // 4-column groups per thread per slice
constexpr int kSampleSlice = 4 * kSampleGroups * kSampleThreads;  // 4096 columns

__device__ __forceinline__ float logit_at(const SampleParams& p, int64_t row, int i) {
  if (p.dtype == SD_F32) return static_cast<const float*>(p.logits)[row * p.ls + i];
  const uint16_t b = static_cast<const uint16_t*>(p.logits)[row * p.ls + i];
  return p.dtype == SD_BF16 ? sd::from_bits<__bf16>(b) : sd::from_bits<_Float16>(b);
}

// Better (key, index): larger key, or the same key at a smaller index (the
// first maximum, as torch.argmax).
__device__ __forceinline__ bool better(float k, int i, float bk, int bi) {
  return k > bk || (k == bk && i < bi);
}

__device__ __forceinline__ void wave_best(float& bk, int& bi) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ok = __shfl_xor(bk, off);
    const int oi = __shfl_xor(bi, off);
    if (better(ok, oi, bk, bi)) {
      bk = ok;
      bi = oi;
    }
  }
}

// Greedy: argmax of the logits. Sampled (T > 0): the reference's
// argmax(softmax(l / T) / E) with E ~ Exp(1) is the argmax of l / T - log(E)
// (log is monotone and the softmax normaliser is common to the row), so one
// pass suffices; the keys are scaled by log2(e) (same argmax). E = -log(U), U
// uniform in (0, 1] from word (column % 4) of the Philox block with key = seed
// and counter = (column / 4, row, offset): a thread takes four consecutive
// columns per Philox call.
// Pass 1, grid (slice, row): the best (key, column) of a 4096-column slice.
__global__ __launch_bounds__(kSampleThreads) void sample_partial_kernel(SampleParams p) {
  __shared__ float sk[kSampleThreads / 64];
  __shared__ int si[kSampleThreads / 64];
  const int64_t row = blockIdx.y;
  const float T = p.temp ? p.temp[row] : 0.f;
  const bool greedy = !(T > 0.f);
  // keys scaled by log2(e) (the argmax is the same): l log2(e) / T - log2(E)
  const float s2 = greedy ? 1.f : 1.4426950408889634f / T;
  uint32_t k0 = 0, k1 = 0, off0 = 0, off1 = 0;
  if (!greedy) {
    const uint64_t seed = static_cast<uint64_t>(p.state[0]);
    const uint64_t off = static_cast<uint64_t>(p.state[1]);
    k0 = static_cast<uint32_t>(seed);
    k1 = static_cast<uint32_t>(seed >> 32);
    off0 = static_cast<uint32_t>(off);
    off1 = static_cast<uint32_t>(off >> 32);
  }
  float bk = -INFINITY;
  int bi = 0x7fffffff;
  const int g0 = blockIdx.x * (kSampleSlice / 4);
#pragma unroll
  for (int j = 0; j < kSampleGroups; ++j) {
    const int g = g0 + j * kSampleThreads + threadIdx.x;
    if (4 * g >= p.V) break;
    uint32_t c[4] = {static_cast<uint32_t>(g), static_cast<uint32_t>(row) ^ off1, off0, 0u};
    if (!greedy) sd::philox(c, k0, k1);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = 4 * g + e;
      if (i >= p.V) break;
      float key = logit_at(p, row, i);
      if (!greedy) {
        const float u = (static_cast<float>(c[e] >> 8) + 1.f) * (1.f / 16777216.f);  // (0, 1]
        // E = max(-ln u, 1e-10); native log2 (v_log_f32)
        const float E = fmaxf(-__builtin_amdgcn_logf(u) * 0.6931471805599453f, 1e-10f);
        key = key * s2 - __builtin_amdgcn_logf(E);
      }
      if (better(key, i, bk, bi)) {
        bk = key;
        bi = i;
      }
    }
  }
  wave_best(bk, bi);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) {
    sk[wave] = bk;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kSampleThreads / 64; ++w)
      if (better(sk[w], si[w], bk, bi)) {
        bk = sk[w];
        bi = si[w];
      }
    p.part[row * p.nslices + blockIdx.x] = make_float2(bk, __int_as_float(bi));
  }
}

// Pass 2, one wave per row: the best of the row's slices.
__global__ __launch_bounds__(64) void sample_merge_kernel(SampleParams p) {
  const int64_t row = blockIdx.x;
  float bk = -INFINITY;
  int bi = 0x7fffffff;
  for (int s = threadIdx.x; s < p.nslices; s += 64) {
    const float2 v = p.part[row * p.nslices + s];
    if (better(v.x, __float_as_int(v.y), bk, bi)) {
      bk = v.x;
      bi = __float_as_int(v.y);
    }
  }
  wave_best(bk, bi);
  if (threadIdx.x == 0) p.out[row] = bi == 0x7fffffff ? 0 : bi;  // an all-NaN row gives token 0
}

constexpr int kSampleMaxRows = 65535;  // grid y

int sample_slices(int32_t vocab) {
  return static_cast<int>((static_cast<int64_t>(vocab) + kSampleSlice - 1) / kSampleSlice);
}

bool is16(int32_t dtype) { return dtype == SD_BF16 || dtype == SD_F16; }

}  // namespace

extern "C" int sd_rmsnorm(const void* x, int64_t x_stride, const void* residual,
                          int64_t residual_stride, const void* weight, void* out,
                          int64_t out_stride, void* residual_out, int64_t residual_out_stride,
                          int64_t rows, int32_t hidden, float eps, int32_t dtype, void* stream) {
  sd::clear_error();
  if (rows < 0 || hidden <= 0 || hidden % 8 != 0 || hidden > 8 * kThreads * kChunks ||
      !is16(dtype)) {
    sd::set_error("rmsnorm: hidden must be a multiple of 8 up to %d, dtype bf16/fp16 "
                  "(rows=%lld hidden=%d dtype=%d)", 8 * kThreads * kChunks, (long long)rows,
                  hidden, dtype);
    return SD_ERR_UNSUPPORTED;
  }
  if (rows == 0) return SD_OK;
  if (!x || !weight || !out || (residual && !residual_out)) {
    sd::set_error("rmsnorm: null pointer argument");
    return SD_ERR_VALUE;
  }
  if (!sd::aligned16(x) || !sd::aligned16(weight) || !sd::aligned16(out) ||
      (residual && (!sd::aligned16(residual) || !sd::aligned16(residual_out))) ||
      x_stride % 8 || out_stride % 8 || (residual && (residual_stride % 8 || residual_out_stride % 8))) {
    sd::set_error("rmsnorm: rows must be 16-byte aligned");
    return SD_ERR_UNSUPPORTED;
  }
  NormParams p{static_cast<const uint16_t*>(x), x_stride, static_cast<const uint16_t*>(residual),
               residual_stride, static_cast<const uint16_t*>(weight), static_cast<uint16_t*>(out),
               out_stride, static_cast<uint16_t*>(residual_out), residual_out_stride, hidden, eps};
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (rows > 0x7fffffff) {
    sd::set_error("rmsnorm: too many rows (%lld)", (long long)rows);
    return SD_ERR_UNSUPPORTED;
  }
  if (dtype == SD_BF16)
    hipLaunchKernelGGL(rmsnorm_kernel<__bf16>, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, st, p);
  else
    hipLaunchKernelGGL(rmsnorm_kernel<_Float16>, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, st, p);
  return sd::check_launch("rmsnorm");
}

namespace {

int run_qk_norm_rope(RopeParams p, int32_t head_dim, int32_t dtype, void* stream) {
  if (head_dim != 128 || !is16(dtype) || p.tokens < 0 || p.tokens > (1ll << 40) || p.Hq < 0 ||
      p.Hkv < 0 || p.Hq > (1 << 20) || p.Hkv > (1 << 20) || p.max_pos <= 0 ||
      p.max_pos > (1ll << 40) || p.cs_stride < 128 || p.cs_stride > (1ll << 40)) {
    sd::set_error("qk_norm_rope: head_dim 128 and bf16/fp16 only, cos_sin rows of >= 128 "
                  "floats (head_dim=%d dtype=%d stride=%lld)", head_dim, dtype,
                  (long long)p.cs_stride);
    return SD_ERR_UNSUPPORTED;
  }
  const int64_t items = p.tokens * (p.Hq + p.Hkv);
  if (items == 0) return SD_OK;
  if ((p.Hq && !p.q) || (p.Hkv && !p.k) || !p.pos || !p.cos_sin) {
    sd::set_error("qk_norm_rope: null pointer argument");
    return SD_ERR_VALUE;
  }
  const int64_t wgs = (items + kThreads / 64 - 1) / (kThreads / 64);
  if (wgs > 0x7fffffff) {
    sd::set_error("qk_norm_rope: too many heads (%lld)", (long long)items);
    return SD_ERR_UNSUPPORTED;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == SD_BF16)
    hipLaunchKernelGGL(qk_norm_rope_kernel<__bf16>, dim3(static_cast<unsigned>(wgs)), dim3(kThreads), 0, st, p);
  else
    hipLaunchKernelGGL(qk_norm_rope_kernel<_Float16>, dim3(static_cast<unsigned>(wgs)), dim3(kThreads), 0, st, p);
  return sd::check_launch("qk_norm_rope");
}

}  // namespace

extern "C" int sd_qk_norm_rope(void* q, int64_t q_stride_tok, int64_t q_stride_head, void* k,
                               int64_t k_stride_tok, int64_t k_stride_head, int64_t num_tokens,
                               int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                               const void* q_weight, const void* k_weight, float eps,
                               const int64_t* positions, const float* cos_sin,
                               int64_t cos_sin_stride, int64_t max_position, int32_t dtype,
                               void* stream) {
  sd::clear_error();
  RopeParams p{};
  p.q = static_cast<uint16_t*>(q);
  p.q_stok = q_stride_tok;
  p.q_shead = q_stride_head;
  p.k = static_cast<uint16_t*>(k);
  p.k_stok = k_stride_tok;
  p.k_shead = k_stride_head;
  p.tokens = num_tokens;
  p.Hq = num_q_heads;
  p.Hkv = num_kv_heads;
  p.qw = static_cast<const uint16_t*>(q_weight);
  p.kw = static_cast<const uint16_t*>(k_weight);
  p.eps = eps;
  p.pos = positions;
  p.cos_sin = cos_sin;
  p.cs_stride = cos_sin_stride;
  p.max_pos = max_position;
  return run_qk_norm_rope(p, head_dim, dtype, stream);
}

extern "C" int sd_qk_norm_rope_store(void* q, int64_t q_stride_tok, int64_t q_stride_head, void* k,
                                     int64_t k_stride_tok, int64_t k_stride_head, const void* v,
                                     int64_t v_stride_tok, int64_t v_stride_head,
                                     int64_t num_tokens, int32_t num_q_heads,
                                     int32_t num_kv_heads, int32_t head_dim, const void* q_weight,
                                     const void* k_weight, float eps, const int64_t* positions,
                                     const float* cos_sin, int64_t cos_sin_stride,
                                     int64_t max_position, void* k_cache, void* v_cache,
                                     int64_t cache_stride_block, int64_t cache_stride_pos,
                                     int64_t cache_stride_head, int64_t num_blocks,
                                     int32_t block_size, const int32_t* slot_mapping,
                                     int32_t dtype, void* stream) {
  sd::clear_error();
  if (num_tokens > 0 && num_kv_heads > 0 &&
      (!v || !k_cache || !v_cache || !slot_mapping || block_size <= 0 || num_blocks <= 0)) {
    sd::set_error("qk_norm_rope_store: v, caches, slot_mapping and a positive pool needed");
    return SD_ERR_VALUE;
  }
  if (block_size > (1 << 20) || num_blocks > (1ll << 32)) {
    sd::set_error("qk_norm_rope_store: pool too large (%lld blocks of %d)", (long long)num_blocks,
                  block_size);
    return SD_ERR_UNSUPPORTED;
  }
  RopeParams p{};
  p.q = static_cast<uint16_t*>(q);
  p.q_stok = q_stride_tok;
  p.q_shead = q_stride_head;
  p.k = static_cast<uint16_t*>(k);
  p.k_stok = k_stride_tok;
  p.k_shead = k_stride_head;
  p.tokens = num_tokens;
  p.Hq = num_q_heads;
  p.Hkv = num_kv_heads;
  p.qw = static_cast<const uint16_t*>(q_weight);
  p.kw = static_cast<const uint16_t*>(k_weight);
  p.eps = eps;
  p.pos = positions;
  p.cos_sin = cos_sin;
  p.cs_stride = cos_sin_stride;
  p.max_pos = max_position;
  p.v = static_cast<const uint16_t*>(v);
  p.v_stok = v_stride_tok;
  p.v_shead = v_stride_head;
  p.kc = static_cast<uint16_t*>(k_cache);
  p.vc = static_cast<uint16_t*>(v_cache);
  p.c_sblk = cache_stride_block;
  p.c_spos = cache_stride_pos;
  p.c_shead = cache_stride_head;
  p.num_slots = num_blocks * block_size;
  p.block_size = block_size;
  p.slot = slot_mapping;
  return run_qk_norm_rope(p, head_dim, dtype, stream);
}

extern "C" int sd_silu_mul(const void* x, int64_t x_stride, void* out, int64_t out_stride,
                           int64_t rows, int32_t width, int32_t dtype, void* stream) {
  sd::clear_error();
  if (rows < 0 || width <= 0 || width % 8 || !is16(dtype)) {
    sd::set_error("silu_mul: width must be a positive multiple of 8, dtype bf16/fp16 "
                  "(width=%d dtype=%d)", width, dtype);
    return SD_ERR_UNSUPPORTED;
  }
  if (rows == 0) return SD_OK;
  if (!x || !out) {
    sd::set_error("silu_mul: null pointer argument");
    return SD_ERR_VALUE;
  }
  if (!sd::aligned16(x) || !sd::aligned16(out) || x_stride % 8 || out_stride % 8) {
    sd::set_error("silu_mul: rows must be 16-byte aligned");
    return SD_ERR_UNSUPPORTED;
  }
  const int64_t wgs = (rows * (width / 8) + kThreads - 1) / kThreads;
  if (wgs > 0x7fffffff) {
    sd::set_error("silu_mul: too large (%lld rows)", (long long)rows);
    return SD_ERR_UNSUPPORTED;
  }
  SiluParams p{static_cast<const uint16_t*>(x), x_stride, static_cast<uint16_t*>(out), out_stride,
               rows, width};
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == SD_BF16)
    hipLaunchKernelGGL(silu_mul_kernel<__bf16>, dim3(static_cast<unsigned>(wgs)), dim3(kThreads), 0, st, p);
  else
    hipLaunchKernelGGL(silu_mul_kernel<_Float16>, dim3(static_cast<unsigned>(wgs)), dim3(kThreads), 0, st, p);
  return sd::check_launch("silu_mul");
}

extern "C" size_t sd_sample_workspace_size(int64_t rows, int32_t vocab) {
  if (rows <= 0 || vocab <= 0) return 0;
  if (rows > kSampleMaxRows) return SIZE_MAX;  // refused by sd_sample
  return static_cast<size_t>(rows) * sample_slices(vocab) * sizeof(float2);
}

extern "C" int sd_sample(const void* logits, int64_t logits_stride, int32_t dtype, int64_t rows,
                         int32_t vocab, const float* temperatures, const int64_t* rng_state,
                         int64_t* out_tokens, void* workspace, size_t workspace_bytes,
                         void* stream) {
  sd::clear_error();
  if (rows < 0 || rows > kSampleMaxRows || vocab <= 0 ||
      (dtype != SD_BF16 && dtype != SD_F16 && dtype != SD_F32)) {
    sd::set_error("sample: up to %d rows, vocab positive, logits bf16/fp16/fp32 (rows=%lld "
                  "vocab=%d dtype=%d)", kSampleMaxRows, (long long)rows, vocab, dtype);
    return SD_ERR_UNSUPPORTED;
  }
  if (rows == 0) return SD_OK;
  if (!logits || !out_tokens || (temperatures && !rng_state)) {
    sd::set_error("sample: null pointer argument (temperatures need rng_state)");
    return SD_ERR_VALUE;
  }
  if (rows > 65535) {
    sd::set_error("sample: at most 65535 rows per call (%lld)", (long long)rows);
    return SD_ERR_UNSUPPORTED;
  }
  const size_t need = sd_sample_workspace_size(rows, vocab);
  if (!workspace || workspace_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 7u)) {
    sd::set_error("sample: workspace of %zu bytes (8-byte aligned) required, got %zu", need,
                  workspace ? workspace_bytes : (size_t)0);
    return SD_ERR_WORKSPACE;
  }
  SampleParams p{logits, logits_stride, dtype, vocab, temperatures, rng_state, out_tokens,
                 static_cast<float2*>(workspace), sample_slices(vocab)};
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(sample_partial_kernel,
                     dim3(static_cast<unsigned>(p.nslices), static_cast<unsigned>(rows)),
                     dim3(kSampleThreads), 0, st, p);
  const int rc = sd::check_launch("sample (slices)");
  if (rc != SD_OK) return rc;
  hipLaunchKernelGGL(sample_merge_kernel, dim3(static_cast<unsigned>(rows)), dim3(64), 0, st, p);
  return sd::check_launch("sample (merge)");
}
