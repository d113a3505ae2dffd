// prefill_attention.hip — variable-length causal attention for gfx950: the
// prefill branch of the engine's attention layer, `flash_attn_varlen_func(q,
// k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, softmax_scale,
// causal=True, block_table)` (nanovllm/layers/attention.py:64-70), with K/V
// either contiguous (total_k, Hkv, D) rows or the paged cache (prefix cache).
//
// Math (sequence b with nq query rows and nk keys, GQA G = Hq / Hkv):
//   o[t, h] = softmax_j( q[t, h] . K[j, h / G] * scale ) . V[.., h / G],
//   j in [0, nk - nq + t]  (bottom-right aligned causal rule)
//
// Work: one workgroup per (128-row tile, kv head, sequence); the 128 rows are
// 128 / G consecutive tokens x the G query heads sharing the kv head, heaviest
// (last) tiles dispatched first. Each of the 4 wave64s owns 32 rows (two
// 16-row MFMA tiles, so every K / V operand read from LDS feeds two MFMAs)
// and its own online softmax. Per step of 64 keys the workgroup stages K and
// V in LDS (double-buffered: one barrier per step; all 256 threads, 16-byte
// loads, the next step's rows in flight in registers meanwhile) and every wave
// computes
//   S^T = K . Q^T      32 x MFMA 16x16x32 (K is the A operand, read from LDS)
//   online softmax     exp2 domain, one row per lane (l % 16)
//   O^T += V^T . P^T   32 x MFMA (P rounded once; 64 with the lo part of P for
//                      waves with rows that see few keys), V^T gathered with
//                      ds_read_b64_tr_b16
// Rows are written normalised at the end (no split over keys: a prefill has
// rows enough to fill the machine).
#include <math.h>

#include <algorithm>

#include "sd_common.h"

namespace {

using sd::f32x4;
using sd::u32x4;

constexpr int kD = 128;
constexpr int kThreads = 256;
constexpr int kRT = 2;                  // 16-row MFMA tiles per wave
constexpr int kRows = 4 * 16 * kRT;     // query rows per workgroup (4 waves x 32)
constexpr int kKeys = 64;               // keys per step
constexpr int kKPitch = 136;   // LDS row pitch of the K tile (16-bit elements)
constexpr int kVPitch = 144;   // LDS row pitch of the V tile

struct PrefillParams {
  const uint16_t* q;
  int64_t q_stok, q_shead;
  const uint16_t* k;  // contiguous (total_k, Hkv, D) rows, or the paged cache
  const uint16_t* v;
  int64_t s_tok;   // contiguous: token stride; paged: position stride within a block
  int64_t s_head;  // head stride
  int64_t s_blk;   // paged: block stride
  int32_t block_size, bs_shift, num_blocks;
  const int32_t* bt;  // (B, bt_stride) block table, NULL: contiguous K/V
  int64_t bt_stride;
  int32_t max_ctx;    // paged: table width x block size
  const int32_t* cu_q;  // (B + 1,)
  const int32_t* cu_k;  // (B + 1,)
  int32_t num_seqs, G, Hkv;
  int64_t total_q;
  float scale_log2;
  uint16_t* out;
  int64_t o_stok, o_shead;
};

// Element offset of key `tok` of sequence b (k0 = cu_k[b] for contiguous K/V).
__device__ __forceinline__ int64_t key_row(const PrefillParams& p, const int32_t* btrow,
                                           int64_t k0, int tok) {
  if (!p.bt) return (k0 + tok) * p.s_tok;
  int pg, off;
  if (p.bs_shift >= 0) {
    pg = tok >> p.bs_shift;
    off = tok & (p.block_size - 1);
  } else {
    pg = tok / p.block_size;
    off = tok - pg * p.block_size;
  }
  const int blk = min(max(btrow[pg], 0), p.num_blocks - 1);
  return static_cast<int64_t>(blk) * p.s_blk + static_cast<int64_t>(off) * p.s_tok;
}

// SPLIT: P enters P.V as hi + lo 16-bit parts (~16 mantissa bits, twice the
// P.V MFMAs), for tiles whose first token sees fewer than kSplitKeys keys:
// with n keys, rounding each P once costs about 2^-9 |v| / sqrt(n_eff) of
// absolute error, which nears the 2e-3 output tolerance when only a handful of
// keys are visible. Other tiles round P once to T, as flash attention does.
// The host launches both instances over the same grid; each workgroup runs in
// the one that matches its tile and exits from the other.
constexpr int kSplitKeys = 128;

template <typename T, bool SPLIT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
void prefill_kernel(PrefillParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t kt[2][kKeys * kKPitch];
  __shared__ __attribute__((aligned(16))) uint16_t vt[2][kKeys * kVPitch];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, lr = lane & 15, lg = lane >> 4;
  const int h = blockIdx.y, b = blockIdx.z;
  const int64_t q0 = p.cu_q[b];
  const int nq = max(p.cu_q[b + 1] - p.cu_q[b], 0);
  const int64_t k0 = p.cu_k[b];
  int nk = max(p.cu_k[b + 1] - p.cu_k[b], 0);
  if (p.bt) nk = min(nk, p.max_ctx);
  const int tpw = kRows / p.G;  // tokens per workgroup
  // SPLIT: the first tiles, in order (a tile's first token sees nk - nq + t0 + 1
  // keys, so only tiles with t0 < kSplitKeys can need it); otherwise the last
  // tiles (the most keys under the causal rule) first
  const int t0 = (SPLIT ? static_cast<int>(blockIdx.x)
                        : static_cast<int>(gridDim.x) - 1 - static_cast<int>(blockIdx.x)) * tpw;
  if (t0 >= nq) return;
  // the split instance covers the first split_tiles tiles; a tile there whose
  // first token sees fewer than kSplitKeys keys is its, every other tile is
  // the single-P instance's (also when nk < nq leaves later tiles short of keys)
  const int split_tiles = (kSplitKeys + tpw - 1) / tpw;
  const bool want_split = t0 < split_tiles * tpw && nk - nq + t0 + 1 < kSplitKeys;
  if (SPLIT != want_split) return;  // the other instance's tile
  const int tl = min(t0 + tpw, nq) - 1;  // last token of the tile
  const int32_t* btrow = p.bt ? p.bt + static_cast<int64_t>(b) * p.bt_stride : nullptr;
  const int64_t hoff = static_cast<int64_t>(h) * p.s_head;

  // ---- this lane's rows (one per row tile): Q operand, causal limit
  int lim[kRT], qi[kRT], gq[kRT];
  bool valid[kRT];
  u32x4 qop[kRT][4];
  int wlast = -1, wfull = 0x7fffffff;
#pragma unroll
  for (int rt = 0; rt < kRT; ++rt) {
    const int row = wave * 16 * kRT + rt * 16 + lr;
    qi[rt] = t0 + row / p.G;
    gq[rt] = row % p.G;
    valid[rt] = row < tpw * p.G && qi[rt] < nq && q0 + qi[rt] < p.total_q;
    lim[rt] = valid[rt] ? nk - nq + qi[rt] : -1;  // last visible key (-1: none)
    const uint16_t* qp =
        p.q + (valid[rt] ? (q0 + qi[rt]) * p.q_stok +
                               static_cast<int64_t>(h * p.G + gq[rt]) * p.q_shead
                         : 0) +
        lg * 8;
#pragma unroll
    for (int s = 0; s < 4; ++s)
      qop[rt][s] = valid[rt] ? sd::load16(qp + s * 32) : u32x4{0u, 0u, 0u, 0u};
    wlast = max(wlast, lim[rt]);
    if (valid[rt]) wfull = min(wfull, lim[rt]);
  }
  // wave-uniform key range of this wave's rows: [0, wlast], and the keys every
  // valid row of the wave sees (no mask needed up to wfull)
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    wlast = max(wlast, __shfl_xor(wlast, off));
    wfull = min(wfull, __shfl_xor(wfull, off));
  }
  wlast = __builtin_amdgcn_readfirstlane(wlast);
  wfull = __builtin_amdgcn_readfirstlane(wfull);
  // workgroup key range: every key any of its rows sees
  const int glast = nk - nq + tl;
  const int nsteps = glast < 0 ? 0 : (glast + kKeys) / kKeys;

  float m_run[kRT], l_run[kRT];
  f32x4 acc[kRT][8];
#pragma unroll
  for (int rt = 0; rt < kRT; ++rt) {
    m_run[rt] = -INFINITY;
    l_run[rt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[rt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // ---- K / V staging: thread t loads key (t / 16) + 16 i, dims 8 (t % 16) .. +8
  const int ld_key = tid >> 4, ld_col = (tid & 15) * 8;
  constexpr int kLd = kKeys / 16;  // rows per thread per step
  u32x4 kr[kLd], vr[kLd];
  auto load = [&](int step) {
#pragma unroll
    for (int i = 0; i < kLd; ++i) {
      const int tok = min(step * kKeys + ld_key + 16 * i, max(nk - 1, 0));
      const int64_t off = key_row(p, btrow, k0, tok) + hoff + ld_col;
      kr[i] = sd::load16_stream(p.k + off);
      vr[i] = sd::load16_stream(p.v + off);
    }
  };
  auto stage = [&](int buf) {
#pragma unroll
    for (int i = 0; i < kLd; ++i) {
      sd::store16(kt[buf] + (ld_key + 16 * i) * kKPitch + ld_col, kr[i]);
      sd::store16(vt[buf] + (ld_key + 16 * i) * kVPitch + ld_col, vr[i]);
    }
  };
  if (nsteps > 0) {
    load(0);
    stage(0);
    if (nsteps > 1) load(1);
    __syncthreads();
  }
  for (int step = 0; step < nsteps; ++step) {
    const int buf = step & 1;
    const uint16_t* kb = kt[buf];
    const uint16_t* vb = vt[buf];
    const int tb = step * kKeys;
    if (tb <= wlast) {  // some row of this wave sees these keys
      // ---- S^T: lane holds S[row lr][key tb + 16 j + 4 lg + i] per row tile
      f32x4 sc[kRT][4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        u32x4 ka[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) ka[s] = sd::load16(kb + (j * 16 + lr) * kKPitch + s * 32 + lg * 8);
#pragma unroll
        for (int rt = 0; rt < kRT; ++rt) {
          f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int s = 0; s < 4; ++s) c = sd::Elem<T>::mfma(ka[s], qop[rt][s], c);
          sc[rt][j] = c;
        }
      }
      // ---- online softmax (exp2 domain), P = hi + lo per 32-key half
      const bool full = tb + kKeys - 1 <= wfull;
      u32x4 phi[kRT][2], plo[SPLIT ? kRT : 1][2];
#pragma unroll
      for (int rt = 0; rt < kRT; ++rt) {
        float mloc = -INFINITY;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float sv = sc[rt][j][i] * p.scale_log2;
            if (!full) sv = (tb + j * 16 + lg * 4 + i <= lim[rt]) ? sv : -INFINITY;
            sc[rt][j][i] = sv;
            mloc = fmaxf(mloc, sv);
          }
        mloc = sd::max_over_groups(mloc);
        const float mnew = fmaxf(m_run[rt], mloc);
        const float mb = mnew == -INFINITY ? 0.f : mnew;
        float ps = 0.f;
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
          float pv[8];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            pv[q] = sd::fast_exp2(sc[rt][2 * kh][q] - mb);
            pv[4 + q] = sd::fast_exp2(sc[rt][2 * kh + 1][q] - mb);
          }
#pragma unroll
          for (int q = 0; q < 8; ++q) ps += pv[q];
          if constexpr (SPLIT) {
            uint32_t hi[4], lo[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) sd::split_pack<T>(pv[2 * q], pv[2 * q + 1], hi[q], lo[q]);
            phi[rt][kh] = u32x4{hi[0], hi[1], hi[2], hi[3]};
            plo[rt][kh] = u32x4{lo[0], lo[1], lo[2], lo[3]};
          } else {
            phi[rt][kh] = u32x4{sd::pack2<T>(pv[0], pv[1]), sd::pack2<T>(pv[2], pv[3]),
                                sd::pack2<T>(pv[4], pv[5]), sd::pack2<T>(pv[6], pv[7])};
          }
        }
        if (__any(mnew > m_run[rt])) {
          const float alpha = sd::fast_exp2(m_run[rt] - mb);
          l_run[rt] *= alpha;
#pragma unroll
          for (int dt = 0; dt < 8; ++dt) acc[rt][dt] *= alpha;
        }
        l_run[rt] += ps;
        m_run[rt] = mnew;
      }
      // ---- O^T += V^T . P^T; in 32-key half kh, k-slot 8 lg + j <-> key
      //      32 kh + 4 lg + j (j < 4) and 32 kh + 16 + 4 lg + j - 4 (j >= 4)
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          const uint16_t* c = vb + (kh * 32 + lg * 4 + (lr >> 2)) * kVPitch + dt * 16 + (lr & 3) * 4;
          const uint2 v0 = sd::lds_read_tr16(c);
          const uint2 v1 = sd::lds_read_tr16(c + 16 * kVPitch);
          const u32x4 vop = {v0.x, v0.y, v1.x, v1.y};
#pragma unroll
          for (int rt = 0; rt < kRT; ++rt) {
            acc[rt][dt] = sd::Elem<T>::mfma(vop, phi[rt][kh], acc[rt][dt]);
            if constexpr (SPLIT) acc[rt][dt] = sd::Elem<T>::mfma(vop, plo[rt][kh], acc[rt][dt]);
          }
        }
    }
    // ---- next step's tile into the other buffer (its readers finished at the
    //      previous barrier), then the one barrier of this step
    if (step + 1 < nsteps) {
      stage(buf ^ 1);
      if (step + 2 < nsteps) load(step + 2);
    }
    __syncthreads();
  }
  // ---- normalised rows: lane holds O[row lr][dims 16 dt + 4 lg .. +4]
#pragma unroll
  for (int rt = 0; rt < kRT; ++rt) {
    const float l = sd::sum_over_groups(l_run[rt]);
    if (!valid[rt]) continue;
    const float inv = l > 0.f ? 1.f / l : 0.f;
    uint16_t* op = p.out + (q0 + qi[rt]) * p.o_stok +
                   static_cast<int64_t>(h * p.G + gq[rt]) * p.o_shead;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      uint2 w;
      w.x = sd::pack2<T>(acc[rt][dt].x * inv, acc[rt][dt].y * inv);
      w.y = sd::pack2<T>(acc[rt][dt].z * inv, acc[rt][dt].w * inv);
      *reinterpret_cast<uint2*>(op + dt * 16 + lg * 4) = w;
    }
  }
}

}  // namespace

extern "C" int sd_prefill_attention(
    const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* k, const void* v,
    int64_t kv_stride_tok, int64_t kv_stride_head, int64_t kv_stride_block, int64_t num_blocks,
    int32_t block_size, const int32_t* block_table, int64_t bt_stride, int32_t max_blocks_per_seq,
    const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int32_t max_seqlen_q,
    int64_t total_q, int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads,
    int32_t head_dim, float scale, int32_t dtype, void* out, int64_t out_stride_tok,
    int64_t out_stride_head, void* stream) {
  sd::clear_error();
  if (num_seqs < 0 || max_seqlen_q < 0 || total_q < 0 || num_q_heads <= 0 || num_kv_heads <= 0 ||
      num_q_heads % num_kv_heads != 0) {
    sd::set_error("prefill_attention: invalid sizes (seqs=%d max_q=%d hq=%d hkv=%d)", num_seqs,
                  max_seqlen_q, num_q_heads, num_kv_heads);
    return SD_ERR_VALUE;
  }
  const int G = num_q_heads / num_kv_heads;
  if (head_dim != kD || G > kRows || kRows % G != 0 || (dtype != SD_BF16 && dtype != SD_F16)) {
    sd::set_error("prefill_attention: head_dim 128, q heads per kv head dividing 128, bf16/fp16 "
                  "only (head_dim=%d G=%d dtype=%d)", head_dim, G, dtype);
    return SD_ERR_UNSUPPORTED;
  }
  if (num_seqs == 0 || total_q == 0 || max_seqlen_q == 0) return SD_OK;
  if (num_seqs > 65535 || num_kv_heads > 65535) {
    sd::set_error("prefill_attention: at most 65535 sequences and kv heads per call");
    return SD_ERR_UNSUPPORTED;
  }
  if (!q || !k || !v || !cu_seqlens_q || !cu_seqlens_k || !out) {
    sd::set_error("prefill_attention: null pointer argument");
    return SD_ERR_VALUE;
  }
  if (block_table && (block_size <= 0 || num_blocks <= 0 || max_blocks_per_seq <= 0)) {
    sd::set_error("prefill_attention: paged K/V needs block_size, num_blocks, table width");
    return SD_ERR_VALUE;
  }
  const int64_t max_ctx = static_cast<int64_t>(max_blocks_per_seq) * block_size;
  if ((block_table && max_ctx > (1ll << 30)) || max_seqlen_q > (1 << 30)) {
    sd::set_error("prefill_attention: context bound %lld or query length %d too large",
                  (long long)max_ctx, max_seqlen_q);
    return SD_ERR_UNSUPPORTED;
  }
  if (!sd::strides_ok({q_stride_tok, q_stride_head, kv_stride_tok, kv_stride_head,
                       kv_stride_block, bt_stride, out_stride_tok, out_stride_head})) {
    sd::set_error("prefill_attention: strides must lie in [-2^40, 2^40] elements");
    return SD_ERR_VALUE;
  }
  if (!sd::aligned16(q) || !sd::aligned16(k) || !sd::aligned16(v) || q_stride_tok % 8 ||
      q_stride_head % 8 || kv_stride_tok % 8 || kv_stride_head % 8 || kv_stride_block % 8 ||
      (reinterpret_cast<uintptr_t>(out) & 7u) || out_stride_tok % 4 || out_stride_head % 4 ||
      kv_stride_tok < 0 || kv_stride_head < 0 || kv_stride_block < 0) {
    sd::set_error("prefill_attention: rows must be 16-byte aligned (output 8-byte)");
    return SD_ERR_UNSUPPORTED;
  }
  PrefillParams p;
  p.q = static_cast<const uint16_t*>(q);
  p.q_stok = q_stride_tok;
  p.q_shead = q_stride_head;
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.s_tok = kv_stride_tok;
  p.s_head = kv_stride_head;
  p.s_blk = kv_stride_block;
  p.block_size = block_size;
  p.bs_shift = block_size > 0 && (block_size & (block_size - 1)) == 0 ? __builtin_ctz(block_size) : -1;
  p.num_blocks = static_cast<int32_t>(num_blocks > 0x7fffffff ? 0x7fffffff : num_blocks);
  p.bt = block_table;
  p.bt_stride = bt_stride;
  p.max_ctx = block_table ? static_cast<int32_t>(max_ctx) : 0x7fffffff;
  p.cu_q = cu_seqlens_q;
  p.cu_k = cu_seqlens_k;
  p.num_seqs = num_seqs;
  p.G = G;
  p.Hkv = num_kv_heads;
  p.total_q = total_q;
  p.scale_log2 = scale * 1.4426950408889634f;
  p.out = static_cast<uint16_t*>(out);
  p.o_stok = out_stride_tok;
  p.o_shead = out_stride_head;
  const int tpw = kRows / G;
  const dim3 grid(static_cast<unsigned>((max_seqlen_q + tpw - 1) / tpw),
                  static_cast<unsigned>(num_kv_heads), static_cast<unsigned>(num_seqs));
  hipStream_t st = static_cast<hipStream_t>(stream);
  // the tiles whose rows see few keys (split P; at most the first
  // ceil(kSplitKeys / tpw) tiles of a sequence), then the rest (P rounded once)
  const dim3 sgrid(std::min(grid.x, static_cast<unsigned>((kSplitKeys + tpw - 1) / tpw)), grid.y,
                   grid.z);
  if (dtype == SD_BF16) {
    hipLaunchKernelGGL((prefill_kernel<__bf16, true>), sgrid, dim3(kThreads), 0, st, p);
    hipLaunchKernelGGL((prefill_kernel<__bf16, false>), grid, dim3(kThreads), 0, st, p);
  } else {
    hipLaunchKernelGGL((prefill_kernel<_Float16, true>), sgrid, dim3(kThreads), 0, st, p);
    hipLaunchKernelGGL((prefill_kernel<_Float16, false>), grid, dim3(kThreads), 0, st, p);
  }
  return sd::check_launch("prefill_attention");
}
