// paged_attention.hip — paged decode / speculative-verify attention for gfx950.
//
// Math (per sequence b, kv head h, query row r = qi * G + g, g < G = Hq / Hkv):
//   o[r] = softmax_j( q[r] . K[j] * scale ) . V,  j in [0, L_b - n_b + qi]
// with K/V row j read from page block_table[b, j / block_size], row
// j % block_size — the paged gather of `paged_decode_attention_ref`
// (nanovllm/kernels/paged_decode_attn.py:472-495) and the bottom-right causal
// rule of the verify forward (nanovllm/layers/attention.py:64-70,
// nanovllm/engine/model_runner.py:522-533).
//
// Work decomposition (split-KV):
//   grid  = (max_splits, Hkv, B); one workgroup = 4 wave64s owns `chunk`
//           tokens of one (sequence, kv head) and walks them in tiles of
//           4 * TPW tokens, every wave taking its own TPW-token slice.
//   wave  : loads its whole slice up front with 16-byte global loads (K in
//           MFMA operand order, V as full 256-byte rows), then per 32 tokens
//             S^T = K . Q^T      4 x MFMA 16x16x32 per 16 tokens per row tile
//             online softmax     exp2 domain, row max over lane groups
//             O^T += V^T . P^T   16 x MFMA per row tile (P split into hi + lo
//                                16-bit parts), V^T gathered from LDS
//           The S^T / O^T orientation puts one query row per lane (l % 16),
//           so the softmax state never moves between lanes.
//   merge : the four waves' (m, l, acc) meet in LDS; a single-split sequence
//           writes the normalised output, otherwise the workgroup writes a
//           partial to the workspace and `paged_attn_combine` merges them.
// G * max_qlen query rows are padded to RT tiles of 16 rows (RT = 1: decode
// with G <= 16 or the 0.6B verify; RT = 2: Qwen3-4B verify with 7 x 4 rows).
#include <math.h>

#include "sd_common.h"

namespace {

using sd::f32x4;
using sd::u32x4;

constexpr int kD = 128;         // head_dim
constexpr int kWaves = 4;       // wave64s per workgroup
constexpr int kThreads = 256;
constexpr int kStep = 32;       // tokens per MFMA step of one wave
constexpr int kVPitch = 136;    // 16-bit elements per LDS row of a V tile (272 B)

struct AttnParams {
  const uint16_t* q;
  int64_t q_stok, q_shead;
  const uint16_t* kc;
  const uint16_t* vc;
  int64_t c_sblk, c_spos, c_shead;
  int32_t num_blocks;
  int32_t block_size;
  int32_t bs_shift;  // log2(block_size), or -1 when block_size is not a power of two
  int32_t max_ctx;   // block_table width * block_size
  const int32_t* bt;
  int64_t bt_stride;
  const int32_t* ctx;   // (B,) keys per sequence, or NULL
  const int32_t* cu_k;  // (B+1,) cumulative keys, used when ctx is NULL
  const int32_t* cu_q;  // (B+1,) cumulative query rows, or NULL (one row per sequence)
  int32_t max_qlen;
  int64_t total_q;
  int32_t G;
  int32_t Hkv;
  float scale_log2;  // softmax scale * log2(e)
  uint16_t* out;
  int64_t o_stok, o_shead;
  float* ws_ml;   // [B][Hkv][max_splits][rmax][2]  (m in log2 units, l)
  float* ws_acc;  // [B][Hkv][max_splits][rmax][kD] unnormalised
  int32_t chunk;  // tokens per split, a multiple of the workgroup tile
  int32_t max_splits;
  int32_t rmax;   // G * max_qlen
};

struct SeqInfo {
  int L;   // keys
  int nq;  // query rows
  int64_t q0;
  int R;   // G * nq
};

__device__ __forceinline__ SeqInfo seq_info(const AttnParams& p, int b) {
  SeqInfo s;
  int L = p.ctx ? p.ctx[b] : (p.cu_k[b + 1] - p.cu_k[b]);
  s.L = min(max(L, 0), p.max_ctx);
  if (p.cu_q) {
    s.q0 = p.cu_q[b];
    s.nq = min(max(p.cu_q[b + 1] - p.cu_q[b], 0), p.max_qlen);
  } else {
    s.q0 = b;
    s.nq = 1;
  }
  s.R = p.G * s.nq;
  return s;
}

// Element offset of key position `tok` (0 <= tok < L) of one sequence.
__device__ __forceinline__ int64_t kv_row(const AttnParams& p, const int32_t* btrow, int tok) {
  int pg, off;
  if (p.bs_shift >= 0) {
    pg = tok >> p.bs_shift;
    off = tok & (p.block_size - 1);
  } else {
    pg = tok / p.block_size;
    off = tok - pg * p.block_size;
  }
  int blk = btrow[pg];
  blk = min(max(blk, 0), p.num_blocks - 1);  // padding ids (-1) never reach here; clamp anyway
  return static_cast<int64_t>(blk) * p.c_sblk + static_cast<int64_t>(off) * p.c_spos;
}

template <typename T>
__device__ __forceinline__ void store4(uint16_t* dst, f32x4 v, float s) {
  uint2 w;
  w.x = sd::pack2<T>(v.x * s, v.y * s);
  w.y = sd::pack2<T>(v.z * s, v.w * s);
  *reinterpret_cast<uint2*>(dst) = w;
}

template <int RT>
constexpr int smem_bytes() {
  constexpr int vtile = kWaves * kStep * kVPitch * 2;
  constexpr int merge = kWaves * RT * 16 * (2 + kD) * 4;
  return vtile > merge ? vtile : merge;
}

// Zero rows of a sequence that has no keys at all (padding rows, L = 0).
template <typename T>
__device__ void write_zero_rows(const AttnParams& p, const SeqInfo& si, int h) {
  for (int idx = threadIdx.x; idx < si.R * 32; idx += kThreads) {
    const int row = idx >> 5, d4 = (idx & 31) * 4;
    const int qi = row / p.G, g = row - qi * p.G;
    const int64_t qt = si.q0 + qi;
    if (qt < 0 || qt >= p.total_q) continue;
    uint16_t* op = p.out + qt * p.o_stok + static_cast<int64_t>(h * p.G + g) * p.o_shead + d4;
    *reinterpret_cast<uint2*>(op) = make_uint2(0u, 0u);
  }
}

// ONE_PAGE: block_size % TPW == 0, so a wave's TPW-token slice never crosses a
// page and one block-table lookup serves the whole slice.
template <typename T, int RT, int TPW, bool ONE_PAGE>
__global__ __launch_bounds__(kThreads) void paged_attn_main(AttnParams p) {
  constexpr int NS = TPW / kStep;
  __shared__ __attribute__((aligned(16))) char smem[smem_bytes<RT>()];

  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const SeqInfo si = seq_info(p, b);
  const int start = split * p.chunk;
  if (start >= si.L) {
    if (split == 0) write_zero_rows<T>(p, si, h);
    return;
  }
  const int end = min(start + p.chunk, si.L);
  const int nsplit = (si.L + p.chunk - 1) / p.chunk;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int lr = lane & 15, lg = lane >> 4;

  // B operand of S^T = K . Q^T: lane holds Q[row = 16 rt + lr][32 s + 8 lg .. +8].
  u32x4 qop[RT][4];
  int lim[RT];  // last key position visible to this lane's row (-1: padding row)
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int row = rt * 16 + lr;
    const int qi = row / p.G, g = row - qi * p.G;
    const int64_t qt = si.q0 + qi;
    const bool valid = row < si.R && qt >= 0 && qt < p.total_q;
    lim[rt] = valid ? si.L - si.nq + qi : -1;
    const uint16_t* qp =
        p.q + (valid ? qt * p.q_stok + static_cast<int64_t>(h * p.G + g) * p.q_shead : 0) + lg * 8;
#pragma unroll
    for (int s = 0; s < 4; ++s) qop[rt][s] = valid ? sd::load16(qp + s * 32) : u32x4{0u, 0u, 0u, 0u};
  }

  float m_run[RT], l_run[RT];
  f32x4 acc[RT][8];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    m_run[rt] = -INFINITY;
    l_run[rt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[rt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  uint16_t* vl = reinterpret_cast<uint16_t*>(smem) + wave * (kStep * kVPitch);
  const int32_t* btrow = p.bt + static_cast<int64_t>(b) * p.bt_stride;
  const int64_t hoff = static_cast<int64_t>(h) * p.c_shead;
  const int last = si.L - 1;

  for (int t0 = __builtin_amdgcn_readfirstlane(start + wave * TPW); t0 < end;
       t0 += kWaves * TPW) {
    // One page lookup per wave slice when the slice cannot cross a page
    // (every clamped token stays in [t0, t0 + TPW)); per-lane lookups otherwise.
    const int64_t base0 = ONE_PAGE ? kv_row(p, btrow, t0) : 0;
    auto row_of = [&](int tok) -> int64_t {
      return ONE_PAGE ? base0 + static_cast<int64_t>(tok - t0) * p.c_spos
                      : kv_row(p, btrow, tok);
    };
    // ---- issue every load of this slice before any math
    u32x4 kr[NS][2][4];
    u32x4 vr[NS][8];
#pragma unroll
    for (int st = 0; st < NS; ++st) {
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const int tok = min(t0 + st * kStep + tt * 16 + lr, last);
        const uint16_t* kp = p.kc + row_of(tok) + hoff + lg * 8;
#pragma unroll
        for (int s = 0; s < 4; ++s) kr[st][tt][s] = sd::load16(kp + s * 32);
      }
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const int tok = min(t0 + st * kStep + r * 4 + lg, last);
        vr[st][r] = sd::load16(p.vc + row_of(tok) + hoff + lr * 8);
      }
    }

#pragma unroll
    for (int st = 0; st < NS; ++st) {
      const int tb = t0 + st * kStep;
      // ---- S^T tiles: lane holds S[row lr][token tb + 16 tt + 4 lg + i]
      f32x4 sc[RT][2];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int s = 0; s < 4; ++s) c = sd::Elem<T>::mfma(kr[st][tt][s], qop[rt][s], c);
          sc[rt][tt] = c;
        }
      }
      // ---- stage the 32 V rows of this step (row-major, padded pitch)
#pragma unroll
      for (int r = 0; r < 8; ++r) sd::store16(vl + (r * 4 + lg) * kVPitch + lr * 8, vr[st][r]);

      // ---- online softmax; P^T operand: k-slot 8 lg + j <-> token 4 lg + j (j < 4)
      //      and token 16 + 4 lg + (j - 4) (j >= 4), the order S^T already holds.
      u32x4 pop[RT], plo[RT];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        float mloc = -INFINITY;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int tok = tb + tt * 16 + lg * 4 + i;
            float s = sc[rt][tt][i] * p.scale_log2;
            s = (tok < end && tok <= lim[rt]) ? s : -INFINITY;
            sc[rt][tt][i] = s;
            mloc = fmaxf(mloc, s);
          }
        }
        mloc = sd::max_over_groups(mloc);
        const float mnew = fmaxf(m_run[rt], mloc);
        const float mb = (mnew == -INFINITY) ? 0.f : mnew;
        const float alpha = exp2f(m_run[rt] - mb);
        float pv[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          pv[j] = exp2f(sc[rt][0][j] - mb);
          pv[4 + j] = exp2f(sc[rt][1][j] - mb);
        }
        float ps = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) ps += pv[j];
        l_run[rt] = l_run[rt] * alpha + ps;
        m_run[rt] = mnew;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) acc[rt][dt] *= alpha;
        // P = hi + lo in two 16-bit operands: P.V keeps ~16 mantissa bits of P
        // instead of the 8 (bf16) a single rounding would leave.
        uint32_t hi[4], lo[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) sd::split_pack<T>(pv[2 * j], pv[2 * j + 1], hi[j], lo[j]);
        pop[rt] = u32x4{hi[0], hi[1], hi[2], hi[3]};
        plo[rt] = u32x4{lo[0], lo[1], lo[2], lo[3]};
      }

      // ---- O^T += V^T . P^T; A operand lane holds V[token slot][dim 16 dt + lr]
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const uint16_t* c0 = vl + (lg * 4) * kVPitch + dt * 16 + lr;
        const uint16_t* c1 = c0 + 16 * kVPitch;
        u32x4 vop;
        vop.x = static_cast<uint32_t>(c0[0]) | (static_cast<uint32_t>(c0[kVPitch]) << 16);
        vop.y = static_cast<uint32_t>(c0[2 * kVPitch]) | (static_cast<uint32_t>(c0[3 * kVPitch]) << 16);
        vop.z = static_cast<uint32_t>(c1[0]) | (static_cast<uint32_t>(c1[kVPitch]) << 16);
        vop.w = static_cast<uint32_t>(c1[2 * kVPitch]) | (static_cast<uint32_t>(c1[3 * kVPitch]) << 16);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          acc[rt][dt] = sd::Elem<T>::mfma(vop, pop[rt], acc[rt][dt]);
          acc[rt][dt] = sd::Elem<T>::mfma(vop, plo[rt], acc[rt][dt]);
        }
      }
    }
  }

  // ---- merge the four waves of this workgroup in LDS
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) l_run[rt] = sd::sum_over_groups(l_run[rt]);
  __syncthreads();  // every wave is done with its V tile; reuse LDS
  float* mm = reinterpret_cast<float*>(smem);
  float* ml = mm + kWaves * RT * 16;
  float* ma = ml + kWaves * RT * 16;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int row = rt * 16 + lr;
    const int slot = wave * RT * 16 + row;
    if (lg == 0) {
      mm[slot] = m_run[rt];
      ml[slot] = l_run[rt];
    }
    if (row < si.R) {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
        sd::store16(ma + slot * kD + dt * 16 + lg * 4, __builtin_bit_cast(u32x4, acc[rt][dt]));
    }
  }
  __syncthreads();

  const int nrows = min(si.R, RT * 16);
  for (int idx = tid; idx < nrows * 32; idx += kThreads) {
    const int row = idx >> 5, d4 = (idx & 31) * 4;
    const int qi = row / p.G, g = row - qi * p.G;
    const int64_t qt = si.q0 + qi;
    if (qt < 0 || qt >= p.total_q) continue;
    float mw[kWaves];
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      mw[w] = mm[w * RT * 16 + row];
      M = fmaxf(M, mw[w]);
    }
    f32x4 o = {0.f, 0.f, 0.f, 0.f};
    float l = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float e = exp2f(mw[w] - M);
        l += e * ml[w * RT * 16 + row];
        o += e * __builtin_bit_cast(f32x4, sd::load16(ma + (w * RT * 16 + row) * kD + d4));
      }
    }
    if (nsplit == 1) {
      uint16_t* op = p.out + qt * p.o_stok + static_cast<int64_t>(h * p.G + g) * p.o_shead + d4;
      store4<T>(op, o, l > 0.f ? 1.f / l : 0.f);
    } else {
      const int64_t e =
          ((static_cast<int64_t>(b) * p.Hkv + h) * p.max_splits + split) * p.rmax + row;
      sd::store16(p.ws_acc + e * kD + d4, __builtin_bit_cast(u32x4, o));
      if ((idx & 31) == 0) {
        p.ws_ml[2 * e] = M;
        p.ws_ml[2 * e + 1] = l;
      }
    }
  }
}

// Log-sum-exp merge of the split partials of one (sequence, kv head). The
// split loops move kUnroll partials per iteration with every load issued
// before any use, so the merge costs a few memory round trips, not one per split.
template <typename T>
__global__ __launch_bounds__(kThreads) void paged_attn_combine(AttnParams p) {
  constexpr int kUnroll = 8;
  const int h = blockIdx.x, b = blockIdx.y;
  const SeqInfo si = seq_info(p, b);
  const int nsplit = (si.L + p.chunk - 1) / p.chunk;
  if (nsplit <= 1) return;
  const int64_t e0 = (static_cast<int64_t>(b) * p.Hkv + h) * p.max_splits * p.rmax;
  const int nrows = min(si.R, p.rmax);
  const float2* ml = reinterpret_cast<const float2*>(p.ws_ml);
  for (int idx = threadIdx.x; idx < nrows * 32; idx += kThreads) {
    const int row = idx >> 5, d4 = (idx & 31) * 4;
    const int qi = row / p.G, g = row - qi * p.G;
    const int64_t qt = si.q0 + qi;
    if (qt < 0 || qt >= p.total_q) continue;
    float M = -INFINITY;
    for (int s0 = 0; s0 < nsplit; s0 += kUnroll) {
      float mv[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u)
        mv[u] = s0 + u < nsplit ? ml[e0 + (s0 + u) * p.rmax + row].x : -INFINITY;
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) M = fmaxf(M, mv[u]);
    }
    f32x4 o = {0.f, 0.f, 0.f, 0.f};
    float l = 0.f;
    if (M != -INFINITY) {
      for (int s0 = 0; s0 < nsplit; s0 += kUnroll) {
        float2 part[kUnroll];
        f32x4 acc[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
          const int64_t e = e0 + (s0 + u) * p.rmax + row;
          if (s0 + u < nsplit) {
            part[u] = ml[e];
            acc[u] = __builtin_bit_cast(f32x4, sd::load16(p.ws_acc + e * kD + d4));
          } else {
            part[u] = make_float2(-INFINITY, 0.f);
            acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
          }
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
          const float w = exp2f(part[u].x - M);
          l += w * part[u].y;
          o += w * acc[u];
        }
      }
    }
    uint16_t* op = p.out + qt * p.o_stok + static_cast<int64_t>(h * p.G + g) * p.o_shead + d4;
    store4<T>(op, o, l > 0.f ? 1.f / l : 0.f);
  }
}

// ------------------------------------------------------------------ host
struct Plan {
  int RT;          // 16-row tiles of query rows
  int TPW;         // tokens per wave per tile
  int chunk;       // tokens per split
  int max_splits;  // grid.x
  int rmax;        // rows per (sequence, kv head) in the workspace
};

Plan make_plan(int num_seqs, int max_qlen, int Hq, int Hkv, int64_t max_ctx, int num_splits) {
  Plan pl;
  const int G = Hq / Hkv;
  pl.rmax = G * max_qlen;
  pl.RT = pl.rmax <= 16 ? 1 : 2;
  pl.TPW = 64;
  if (pl.RT == 2) pl.TPW = 32;
  // Small batches: halve the tile so the grid still covers the 256 CUs.
  const int64_t tiles256 = (max_ctx + 255) / 256;
  if (static_cast<int64_t>(num_seqs) * Hkv * tiles256 < 1024) pl.TPW = 32;
  const int tile = kWaves * pl.TPW;
  int64_t chunk = tile;
  if (num_splits > 0) {
    const int64_t per = (max_ctx + num_splits - 1) / num_splits;
    chunk = (per + tile - 1) / tile * tile;
    if (chunk < tile) chunk = tile;
  }
  pl.chunk = static_cast<int>(chunk);
  int64_t ms = (max_ctx + chunk - 1) / chunk;
  pl.max_splits = static_cast<int>(ms < 1 ? 1 : ms);
  return pl;
}

size_t ws_bytes(const Plan& pl, int num_seqs, int Hkv) {
  if (pl.max_splits <= 1) return 0;
  const size_t entries = static_cast<size_t>(num_seqs) * Hkv * pl.max_splits * pl.rmax;
  const size_t ml = (entries * 2 * sizeof(float) + 255) / 256 * 256;
  return ml + entries * kD * sizeof(float);
}

template <typename T, int RT, int TPW>
void launch_main(const AttnParams& p, dim3 grid, hipStream_t st) {
  if (p.block_size % TPW == 0)
    hipLaunchKernelGGL((paged_attn_main<T, RT, TPW, true>), grid, dim3(kThreads), 0, st, p);
  else
    hipLaunchKernelGGL((paged_attn_main<T, RT, TPW, false>), grid, dim3(kThreads), 0, st, p);
}

template <typename T>
int launch_all(const AttnParams& p, const Plan& pl, int num_seqs, bool combine, hipStream_t st) {
  const dim3 grid(pl.max_splits, p.Hkv, num_seqs);
  if (pl.RT == 1) {
    if (pl.TPW == 64) launch_main<T, 1, 64>(p, grid, st);
    else launch_main<T, 1, 32>(p, grid, st);
  } else {
    launch_main<T, 2, 32>(p, grid, st);
  }
  int rc = sd::check_launch("paged_attention main");
  if (rc != SD_OK || !combine || pl.max_splits <= 1) return rc;
  hipLaunchKernelGGL((paged_attn_combine<T>), dim3(p.Hkv, num_seqs), dim3(kThreads), 0, st, p);
  return sd::check_launch("paged_attention combine");
}

int run_attention(bool combine, const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                  const void* k_cache, const void* v_cache, int64_t cache_stride_block,
                  int64_t cache_stride_pos, int64_t cache_stride_head, int64_t num_blocks,
                  int32_t block_size, const int32_t* block_table, int64_t bt_stride,
                  int32_t max_blocks_per_seq, const int32_t* context_lens,
                  const int32_t* cu_seqlens_k, const int32_t* cu_seqlens_q, int32_t max_qlen,
                  int64_t total_q, int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads,
                  int32_t head_dim, float scale, int32_t dtype, void* out,
                  int64_t out_stride_tok, int64_t out_stride_head, void* workspace,
                  size_t workspace_bytes, int32_t num_splits, void* stream) {
  sd::clear_error();
  if (num_seqs < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 ||
      block_size <= 0 || num_blocks <= 0 || max_blocks_per_seq <= 0 || max_qlen <= 0 ||
      total_q < 0 || num_splits < 0) {
    sd::set_error("paged_attention: invalid sizes (seqs=%d hq=%d hkv=%d d=%d bs=%d blocks=%lld "
                  "maxblk=%d max_qlen=%d total_q=%lld splits=%d)",
                  num_seqs, num_q_heads, num_kv_heads, head_dim, block_size,
                  (long long)num_blocks, max_blocks_per_seq, max_qlen, (long long)total_q,
                  num_splits);
    return SD_ERR_VALUE;
  }
  if (num_q_heads % num_kv_heads != 0) {
    sd::set_error("paged_attention: GQA needs num_q_heads %% num_kv_heads == 0 (%d vs %d)",
                  num_q_heads, num_kv_heads);
    return SD_ERR_VALUE;
  }
  if (num_seqs == 0 || total_q == 0) return SD_OK;
  if (!q || !k_cache || !v_cache || !block_table || !out || (!context_lens && !cu_seqlens_k)) {
    sd::set_error("paged_attention: null pointer argument");
    return SD_ERR_VALUE;
  }
  if (!cu_seqlens_q && max_qlen != 1) {
    sd::set_error("paged_attention: max_qlen must be 1 without cu_seqlens_q");
    return SD_ERR_VALUE;
  }
  if (head_dim != kD) {
    sd::set_error("paged_attention: only head_dim %d is supported, got %d", kD, head_dim);
    return SD_ERR_UNSUPPORTED;
  }
  if (dtype != SD_BF16 && dtype != SD_F16) {
    sd::set_error("paged_attention: dtype must be bf16 or f16");
    return SD_ERR_UNSUPPORTED;
  }
  const int G = num_q_heads / num_kv_heads;
  if (static_cast<int64_t>(G) * max_qlen > 32) {
    sd::set_error("paged_attention: (num_q_heads/num_kv_heads) * max_qlen = %d exceeds 32",
                  G * max_qlen);
    return SD_ERR_UNSUPPORTED;
  }
  const int64_t max_ctx = static_cast<int64_t>(max_blocks_per_seq) * block_size;
  if (max_ctx > (1ll << 30) || num_blocks > (1ll << 31) - 1) {
    sd::set_error("paged_attention: context bound %lld or pool %lld too large",
                  (long long)max_ctx, (long long)num_blocks);
    return SD_ERR_UNSUPPORTED;
  }
  const bool aligned = sd::aligned16(q) && sd::aligned16(k_cache) && sd::aligned16(v_cache) &&
                       (reinterpret_cast<uintptr_t>(out) & 7u) == 0 && q_stride_tok % 8 == 0 &&
                       q_stride_head % 8 == 0 && cache_stride_block % 8 == 0 &&
                       cache_stride_pos % 8 == 0 && cache_stride_head % 8 == 0 &&
                       out_stride_tok % 4 == 0 && out_stride_head % 4 == 0;
  if (!aligned) {
    sd::set_error("paged_attention: q/cache rows must be 16-byte aligned and out rows 8-byte "
                  "aligned");
    return SD_ERR_UNSUPPORTED;
  }
  const Plan pl = make_plan(num_seqs, max_qlen, num_q_heads, num_kv_heads, max_ctx, num_splits);
  const size_t need = ws_bytes(pl, num_seqs, num_kv_heads);
  if (need > 0 && (!workspace || workspace_bytes < need || !sd::aligned16(workspace))) {
    sd::set_error("paged_attention: workspace of %zu bytes (16-byte aligned) required, got %zu",
                  need, workspace ? workspace_bytes : (size_t)0);
    return SD_ERR_WORKSPACE;
  }

  AttnParams p;
  p.q = static_cast<const uint16_t*>(q);
  p.q_stok = q_stride_tok;
  p.q_shead = q_stride_head;
  p.kc = static_cast<const uint16_t*>(k_cache);
  p.vc = static_cast<const uint16_t*>(v_cache);
  p.c_sblk = cache_stride_block;
  p.c_spos = cache_stride_pos;
  p.c_shead = cache_stride_head;
  p.num_blocks = static_cast<int32_t>(num_blocks);
  p.block_size = block_size;
  p.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz(block_size) : -1;
  p.max_ctx = static_cast<int32_t>(max_ctx);
  p.bt = block_table;
  p.bt_stride = bt_stride;
  p.ctx = context_lens;
  p.cu_k = cu_seqlens_k;
  p.cu_q = cu_seqlens_q;
  p.max_qlen = max_qlen;
  p.total_q = total_q;
  p.G = G;
  p.Hkv = num_kv_heads;
  p.scale_log2 = scale * 1.4426950408889634f;
  p.out = static_cast<uint16_t*>(out);
  p.o_stok = out_stride_tok;
  p.o_shead = out_stride_head;
  if (need > 0) {
    const size_t entries =
        static_cast<size_t>(num_seqs) * num_kv_heads * pl.max_splits * pl.rmax;
    p.ws_ml = static_cast<float*>(workspace);
    p.ws_acc = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                        (entries * 2 * sizeof(float) + 255) / 256 * 256);
  } else {
    p.ws_ml = nullptr;
    p.ws_acc = nullptr;
  }
  p.chunk = pl.chunk;
  p.max_splits = pl.max_splits;
  p.rmax = pl.rmax;

  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == SD_BF16) return launch_all<__bf16>(p, pl, num_seqs, combine, st);
  return launch_all<_Float16>(p, pl, num_seqs, combine, st);
}

}  // namespace

extern "C" size_t sd_paged_attention_workspace_size(int32_t num_seqs, int32_t max_qlen,
                                                    int32_t num_q_heads, int32_t num_kv_heads,
                                                    int32_t head_dim, int64_t max_ctx,
                                                    int32_t num_splits) {
  (void)head_dim;
  if (num_seqs <= 0 || max_qlen <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || max_ctx <= 0 ||
      num_q_heads % num_kv_heads != 0 || num_splits < 0)
    return 0;
  const Plan pl = make_plan(num_seqs, max_qlen, num_q_heads, num_kv_heads, max_ctx, num_splits);
  return ws_bytes(pl, num_seqs, num_kv_heads);
}

extern "C" int sd_paged_attention(
    const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* k_cache,
    const void* v_cache, int64_t cache_stride_block, int64_t cache_stride_pos,
    int64_t cache_stride_head, int64_t num_blocks, int32_t block_size,
    const int32_t* block_table, int64_t bt_stride, int32_t max_blocks_per_seq,
    const int32_t* context_lens, const int32_t* cu_seqlens_k, const int32_t* cu_seqlens_q,
    int32_t max_qlen, int64_t total_q, int32_t num_seqs, int32_t num_q_heads,
    int32_t num_kv_heads, int32_t head_dim, float scale, int32_t dtype, void* out,
    int64_t out_stride_tok, int64_t out_stride_head, void* workspace, size_t workspace_bytes,
    int32_t num_splits, void* stream) {
  return run_attention(true, q, q_stride_tok, q_stride_head, k_cache, v_cache,
                       cache_stride_block, cache_stride_pos, cache_stride_head, num_blocks,
                       block_size, block_table, bt_stride, max_blocks_per_seq, context_lens,
                       cu_seqlens_k, cu_seqlens_q, max_qlen, total_q, num_seqs, num_q_heads,
                       num_kv_heads, head_dim, scale, dtype, out, out_stride_tok,
                       out_stride_head, workspace, workspace_bytes, num_splits, stream);
}

extern "C" int sd_paged_attention_partial(
    const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* k_cache,
    const void* v_cache, int64_t cache_stride_block, int64_t cache_stride_pos,
    int64_t cache_stride_head, int64_t num_blocks, int32_t block_size,
    const int32_t* block_table, int64_t bt_stride, int32_t max_blocks_per_seq,
    const int32_t* context_lens, const int32_t* cu_seqlens_k, const int32_t* cu_seqlens_q,
    int32_t max_qlen, int64_t total_q, int32_t num_seqs, int32_t num_q_heads,
    int32_t num_kv_heads, int32_t head_dim, float scale, int32_t dtype, void* out,
    int64_t out_stride_tok, int64_t out_stride_head, void* workspace, size_t workspace_bytes,
    int32_t num_splits, void* stream) {
  return run_attention(false, q, q_stride_tok, q_stride_head, k_cache, v_cache,
                       cache_stride_block, cache_stride_pos, cache_stride_head, num_blocks,
                       block_size, block_table, bt_stride, max_blocks_per_seq, context_lens,
                       cu_seqlens_k, cu_seqlens_q, max_qlen, total_q, num_seqs, num_q_heads,
                       num_kv_heads, head_dim, scale, dtype, out, out_stride_tok,
                       out_stride_head, workspace, workspace_bytes, num_splits, stream);
}
