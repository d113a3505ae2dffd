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
// Work: one workgroup per (64-row tile, kv head, sequence); the 64 rows are
// 64 / G consecutive tokens x the G query heads sharing the kv head. Each of
// the 4 wave64s owns 16 rows and its own online softmax. Per step of 32 keys
// the workgroup stages K and V once in LDS (all 256 threads, 16-byte loads;
// the next step's rows are prefetched into registers meanwhile) and every
// wave computes
//   S^T = K . Q^T      8 x MFMA 16x16x32 (K is the A operand, read from LDS)
//   online softmax     exp2 domain, one row per lane (l % 16)
//   O^T += V^T . P^T   16 x MFMA (P split into hi + lo 16-bit parts), V^T
//                      gathered with ds_read_b64_tr_b16
// Rows are written normalised at the end (no split over keys: a prefill has
// rows enough to fill the machine).
#include <math.h>

#include "sd_common.h"

namespace {

using sd::f32x4;
using sd::u32x4;

constexpr int kD = 128;
constexpr int kThreads = 256;
constexpr int kRows = 64;      // query rows per workgroup (4 waves x 16)
constexpr int kKeys = 32;      // keys per step
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

template <typename T>
__global__ __launch_bounds__(kThreads) void prefill_kernel(PrefillParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t kt[kKeys * kKPitch];
  __shared__ __attribute__((aligned(16))) uint16_t vt[kKeys * kVPitch];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, lr = lane & 15, lg = lane >> 4;
  const int h = blockIdx.y, b = blockIdx.z;
  const int64_t q0 = p.cu_q[b];
  const int nq = max(p.cu_q[b + 1] - p.cu_q[b], 0);
  const int64_t k0 = p.cu_k[b];
  int nk = max(p.cu_k[b + 1] - p.cu_k[b], 0);
  if (p.bt) nk = min(nk, p.max_ctx);
  const int tpw = kRows / p.G;  // tokens per workgroup
  const int t0 = blockIdx.x * tpw;
  if (t0 >= nq) return;
  const int tl = min(t0 + tpw, nq) - 1;  // last token of the tile
  const int32_t* btrow = p.bt ? p.bt + static_cast<int64_t>(b) * p.bt_stride : nullptr;
  const int64_t hoff = static_cast<int64_t>(h) * p.s_head;

  // ---- this lane's row: Q operand, causal limit
  const int row = wave * 16 + lr;
  const int qi = t0 + row / p.G, g = row % p.G;
  const bool valid = row < tpw * p.G && qi < nq && q0 + qi < p.total_q;
  const int lim = valid ? nk - nq + qi : -1;  // last visible key (-1: none)
  u32x4 qop[4];
  {
    const uint16_t* qp =
        p.q + (valid ? (q0 + qi) * p.q_stok + static_cast<int64_t>(h * p.G + g) * p.q_shead : 0) +
        lg * 8;
#pragma unroll
    for (int s = 0; s < 4; ++s) qop[s] = valid ? sd::load16(qp + s * 32) : u32x4{0u, 0u, 0u, 0u};
  }
  // wave-uniform key range of this wave's rows: [0, wlast], and the keys
  // every valid row of the wave sees (no mask needed up to wfull)
  int wlast = lim, wfull = valid ? lim : 0x7fffffff;
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

  float m_run = -INFINITY, l_run = 0.f;
  f32x4 acc[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // ---- K / V staging: thread t loads key (t / 16) + 16 i, dims 8 (t % 16) .. +8
  const int ld_key = tid >> 4, ld_col = (tid & 15) * 8;
  u32x4 kr[2], vr[2];
  auto load = [&](int step) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int tok = min(step * kKeys + ld_key + 16 * i, max(nk - 1, 0));
      const int64_t off = key_row(p, btrow, k0, tok) + hoff + ld_col;
      kr[i] = sd::load16_stream(p.k + off);
      vr[i] = sd::load16_stream(p.v + off);
    }
  };
  if (nsteps > 0) load(0);
  for (int step = 0; step < nsteps; ++step) {
    __syncthreads();  // every wave is done reading the previous tiles
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      sd::store16(kt + (ld_key + 16 * i) * kKPitch + ld_col, kr[i]);
      sd::store16(vt + (ld_key + 16 * i) * kVPitch + ld_col, vr[i]);
    }
    __syncthreads();
    if (step + 1 < nsteps) load(step + 1);  // in flight while this step computes
    const int tb = step * kKeys;
    if (tb > wlast) continue;  // no row of this wave sees these keys
    // ---- S^T: lane holds S[row lr][key tb + 16 tt + 4 lg + i]
    f32x4 sc[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s)
        c = sd::Elem<T>::mfma(sd::load16(kt + (tt * 16 + lr) * kKPitch + s * 32 + lg * 8), qop[s],
                              c);
      sc[tt] = c;
    }
    // ---- online softmax (exp2 domain)
    const bool full = tb + kKeys - 1 <= wfull;
    float mloc = -INFINITY;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float sv = sc[tt][i] * p.scale_log2;
        if (!full) sv = (tb + tt * 16 + lg * 4 + i <= lim) ? sv : -INFINITY;
        sc[tt][i] = sv;
        mloc = fmaxf(mloc, sv);
      }
    mloc = sd::max_over_groups(mloc);
    const float mnew = fmaxf(m_run, mloc);
    const float mb = mnew == -INFINITY ? 0.f : mnew;
    float pv[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      pv[q] = sd::fast_exp2(sc[0][q] - mb);
      pv[4 + q] = sd::fast_exp2(sc[1][q] - mb);
    }
    float ps = 0.f;
#pragma unroll
    for (int q = 0; q < 8; ++q) ps += pv[q];
    if (__any(mnew > m_run)) {
      const float alpha = sd::fast_exp2(m_run - mb);
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) acc[dt] *= alpha;
    }
    l_run += ps;
    m_run = mnew;
    uint32_t hi[4], lo[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) sd::split_pack<T>(pv[2 * q], pv[2 * q + 1], hi[q], lo[q]);
    const u32x4 phi = {hi[0], hi[1], hi[2], hi[3]}, plo = {lo[0], lo[1], lo[2], lo[3]};
    // ---- O^T += V^T . P^T; k-slot 8 lg + j <-> key 4 lg + j (j < 4), 16 + 4 lg + j - 4
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const uint16_t* c = vt + (lg * 4 + (lr >> 2)) * kVPitch + dt * 16 + (lr & 3) * 4;
      const uint2 v0 = sd::lds_read_tr16(c);
      const uint2 v1 = sd::lds_read_tr16(c + 16 * kVPitch);
      const u32x4 vop = {v0.x, v0.y, v1.x, v1.y};
      acc[dt] = sd::Elem<T>::mfma(vop, phi, acc[dt]);
      acc[dt] = sd::Elem<T>::mfma(vop, plo, acc[dt]);
    }
  }
  // ---- normalised rows: lane holds O[row lr][dims 16 dt + 4 lg .. +4]
  l_run = sd::sum_over_groups(l_run);
  if (!valid) return;
  const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
  uint16_t* op = p.out + (q0 + qi) * p.o_stok + static_cast<int64_t>(h * p.G + g) * p.o_shead;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
    uint2 w;
    w.x = sd::pack2<T>(acc[dt].x * inv, acc[dt].y * inv);
    w.y = sd::pack2<T>(acc[dt].z * inv, acc[dt].w * inv);
    *reinterpret_cast<uint2*>(op + dt * 16 + lg * 4) = w;
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
    sd::set_error("prefill_attention: head_dim 128, q heads per kv head dividing 64, bf16/fp16 "
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
  p.max_ctx = block_table ? max_blocks_per_seq * block_size : 0x7fffffff;
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
  if (dtype == SD_BF16)
    hipLaunchKernelGGL(prefill_kernel<__bf16>, grid, dim3(kThreads), 0, st, p);
  else
    hipLaunchKernelGGL(prefill_kernel<_Float16>, grid, dim3(kThreads), 0, st, p);
  return sd::check_launch("prefill_attention");
}
