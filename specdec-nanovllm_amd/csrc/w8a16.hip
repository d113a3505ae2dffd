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
// nontemporal load, 1 KB per wave instruction. One launch per call: a grid of
// resident workgroups walks the row groups (16 NT rows) grid-stride; a row
// group is either one wave's (whole K, when rows are plentiful) or shared by
// the four waves of a workgroup that split K and add their partials in LDS
// (narrow layers such as N = 1024). One or two activation rows on matrices up
// to 32 MiB take the row-streaming kernel instead (w8a16_rows_kernel: whole
// weight rows per load, activations in registers, no MFMA or LDS).
//
// int8 -> fp16: (b ^ 0x80) in the low byte under exponent byte 0x64 is the
// fp16 value 1024 + b + 128, exact; subtracting 1152 (packed fp16) gives b.
// int8 -> bf16: v_cvt_f32_ubyte of (b ^ 0x80) minus 128 is b as fp32, whose
// upper half is the exact bf16 (|b| <= 127 needs 7 mantissa bits).
#include <mutex>

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
  int32_t nks;     // K / 64
  int32_t groups;  // row groups of 16 NT rows
  int32_t xpitch;  // bytes per activation row in LDS (staged activations only)
  int32_t xbytes;  // XL: bytes of staged activation rows; the scale table follows
  int32_t ngmax;   // XL: most row groups one wave owns
  int64_t up;      // SL: elements from a gate_up row's gate half to its up half
  // NM: add + RMSNorm of the activation rows while staging them
  const uint16_t* nw;   // (K,) norm weight
  const uint16_t* nres; // (M, K) residual added first, or NULL
  int64_t nres_s;
  uint16_t* nres_out;   // (M, K) bf16(x + residual), written by workgroup x = 0, or NULL
  int64_t nres_out_s;
  float neps;
  // paired rows (gate_up with the SiluAndMul epilogue): output column i pairs
  // weight rows i and i + pair; N is the number of pairs (output columns)
  int32_t pair;
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

// Row groups of 16 NT rows are spread over the grid (grid-stride). KW waves
// share one row group and split its K (partials meet in LDS); with KW == 1 the
// four waves of a workgroup own four different row groups. Each wave walks its
// (row group, K chunk) items in order and keeps the next D - 1 items' loads
// in flight while it computes item i (a ring of D register buffers), so a
// workgroup streams weights for its whole lifetime instead of loading once
// and exiting.
//
// Weight loads are row-contiguous: a chunk is U 64-k steps (64 U bytes) of
// each of the 16 NT rows, and 4 U lanes read one row's 64 U bytes, so a load
// instruction covers 16 / U whole row segments. The chunk is staged in a
// wave-private LDS tile, 16-byte unit u of row r at position u ^ (r & SWZ)
// (SWZ = min(4 U, 16) - 1), from which each lane reads its MFMA A operand
// (16 int8 of row l % 16 at k = 64 step + 16 (l / 16)) with ds_read_b128; with
// 16 positions per row the 16 lanes of a read hit distinct banks.
// The exception is the staged form with 32 or 64 activation rows (XL, MT >= 2):
// there each lane loads its A operand directly (a load instruction then covers 16
// rows x 64 bytes, half cache lines, which costs the narrower shapes 2-20%),
// because without the weight tile two workgroups fit per CU beside the
// 64 KB of activation rows, and the MFMA work per weight byte is twice that of
// 16 rows.
//
// XL: the workgroup's activation rows (whole K) are staged in LDS once, at
// the start, and each step's B operand is read from there. The only vector
// loads left in the loop are the weight stream's: for M = 1 the activation
// loads were as many instructions per chunk as the weight loads (4 of 64
// lanes active), and every vector load instruction costs the compute unit's
// address path the same time whatever its lane count.
//
// MODE 1 (SL): the activation is SiluAndMul of a gate_up row,
// bf16(bf16(silu(g)) * u) with g = x[m, k] and u = x[m, up + k], formed where
// the activation is loaded (the down projection reads the gate_up projection's
// output directly).
// MODE 2 (NM, staged only): the activation is the add + RMSNorm of the rows
// (sd::add_rmsnorm_row_wave: one wave per row, the RMSNorm kernel's own
// arithmetic and summation order), formed while staging; workgroup x = 0 of
// each activation block writes the new residual.
//
// FLOOR: the measurement twin — the same grid, staging, loads and prefetch, with
// every loaded weight word folded into a register instead of the staging through
// the LDS tile, the MFMAs and the epilogue; no output.
template <typename T, int MT, int NT, int KW, int U, bool PER_GROUP, bool CONTIG = false,
          int D = 2, bool XL = false, int MODE = 0, int NWV = kWaves, bool FLOOR = false>
__global__ __launch_bounds__(NWV * 64) void w8a16_kernel(W8Params p) {
  constexpr bool SL = MODE == 1;
  constexpr bool NM = MODE == 2;
  constexpr int NTH = NWV * 64;  // threads of the workgroup
  static_assert(!NM || XL, "the norm is formed while staging");
  static_assert(U == 2 || U == 4 || U == 8, "a chunk row segment is 64 U bytes");
  constexpr int LPR = 4 * U;         // lanes per row segment (16-byte units per row)
  constexpr int RPI = 64 / LPR;      // row segments per load instruction
  constexpr int NLD = 16 * NT / RPI; // load instructions per chunk
  constexpr int NSUB = NWV / KW;  // row groups a workgroup works on at once
  constexpr int SWZ = (LPR < 16 ? LPR : 16) - 1;  // position swizzle stays inside a row
  // DIRECT: each lane loads its own A operand (row l % 16, 16 bytes at
  // k = 64 step + 16 (l / 16)) straight from HBM, no LDS tile
  constexpr bool DIRECT = XL && MT >= 2;
  constexpr int TILE = DIRECT ? 16 : 16 * NT * LPR * 16;  // bytes of one wave's LDS tile
  __shared__ __attribute__((aligned(16))) char wtile[NWV][TILE];
  __shared__ __attribute__((aligned(16))) float red[KW > 1 ? KW - 1 : 1][NT * MT * 4][64];
  extern __shared__ __attribute__((aligned(16))) char xsm[];  // XL: activation rows

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lg = lane >> 4;
  const int sub = wave / KW, kw = wave - sub * KW;
  const int m0 = blockIdx.y * MT * 16;
  char* tile = wtile[wave];

  // K steps of this wave: [ks, ke); every wave of a row group runs the same
  // number of chunks (so the LDS reduction lines up), short ones skip steps.
  const int ks = static_cast<int>(static_cast<int64_t>(kw) * p.nks / KW);
  const int ke = static_cast<int>(static_cast<int64_t>(kw + 1) * p.nks / KW);
  const int nchunks = ((p.nks + KW - 1) / KW + U - 1) / U;

  // row groups of this wave: g0, g0 + gstride, ... (ngroups of them). Grid-stride
  // over the whole matrix, or (CONTIG) a contiguous range per workgroup whose
  // NSUB waves take alternate groups, so a workgroup reads adjacent rows.
  int g0, gstride, ngroups;
  if constexpr (CONTIG) {
    const int per = (p.groups + gridDim.x * NSUB - 1) / (gridDim.x * NSUB) * NSUB;
    const int gb = blockIdx.x * per, ge = min(gb + per, p.groups);
    g0 = gb + sub;
    gstride = NSUB;
    ngroups = g0 < ge ? (ge - g0 + NSUB - 1) / NSUB : 0;
  } else {
    g0 = blockIdx.x * NSUB + sub;
    gstride = gridDim.x * NSUB;
    ngroups = g0 < p.groups ? (p.groups - g0 + gstride - 1) / gstride : 0;
  }
  const int nit = ngroups * nchunks;
  if (!XL && nit == 0) return;  // uniform over the workgroup when KW > 1 (NSUB == 1)

  // XL: fp32 scale table (and bias) of every row this workgroup's waves own, in
  // LDS after the activation rows: [sub][group of the wave][row][scale column]
  constexpr int RG = NT * 16;  // rows per group
  const int spr = PER_GROUP ? p.K / p.group : 1;
  float* scl = reinterpret_cast<float*>(xsm + p.xbytes);
  float* bis = scl + NSUB * p.ngmax * RG * spr;
  auto srow = [&](int g, int r) {  // scale-table row of row r of group g (this wave's)
    return (sub * p.ngmax + (g - g0) / gstride) * RG + r;
  };
  // pr: gate_up with the SiLU epilogue on the K-split path. Group g is gate tile
  // g (weight rows 16 g ..) and up tile g (rows pair + 16 g ..); its 16 outputs
  // are bf16(bf16(silu(gate)) * up) of the rows the projection would write.
  constexpr bool PRC = KW > 1 && NT == 2 && MODE != 1 && !PER_GROUP;
  const bool pr = PRC && p.pair > 0;
  const int nrows = pr ? 2 * p.pair : p.N;  // weight rows
  auto wrow = [&](int g, int r) {  // weight row of row r (0 .. RG - 1) of group g
    return pr ? (r < 16 ? g * 16 + r : p.pair + g * 16 + (r - 16)) : g * RG + r;
  };

  // Activation rows past M are never loaded from memory: those lanes keep
  // zeros (only the lanes of real rows touch memory, e.g. 4 of 64 at M = 1).
  // Staged rows (XL) are read from LDS with no mask, rows past M reading the
  // last staged row: an MFMA output column depends only on its own activation
  // row, and the columns of rows past M are never written, while the zeros and
  // the mask cost 9 VALU instructions per 16-row tile and step.
  const uint16_t* xp[MT];
  bool xok[MT];
  int xro[MT];  // XL: LDS byte offset of the (clamped) staged row
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = m0 + mt * 16 + lr;
    xok[mt] = m < p.M;
    xp[mt] = p.x + static_cast<int64_t>(min(m, p.M - 1)) * p.xs + lg * 16;
    xro[mt] = (min(m, p.M - 1) - m0) * p.xpitch;
  }

  f32x4 acc[NT][MT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // this lane's place in a load instruction: row segment, 16-byte unit
  const int ld_row = lane / LPR, ld_unit = lane % LPR;
  const int ld_step = ld_unit >> 2;  // 64-k step (within the chunk) of that unit

  struct Regs {
    u32x4 w[NLD];
    u32x4 x[XL ? 1 : U][MT][2];  // activation B operands of the chunk's steps (not XL)
    // SL: the up halves, as loaded; SiluAndMul is applied where the operand is
    // used (applying it here would wait for these loads, queued behind the
    // weight prefetch)
    u32x4 xu[SL && !XL ? U : 1][MT][2];
  };
  // Every call issues the same loads: steps past this wave's K range are
  // clamped into the matrix (loaded, never used), rows past N / M read a valid
  // row whose result is dropped. A load count that never depends on control
  // flow lets the compiler wait for one chunk without waiting for the chunks
  // prefetched after it.
  // `real` false (prefetch past the last item): every lane reads the same 16
  // bytes, one cache line instead of a re-read of streamed weight rows.
  // Weight offsets are 32-bit from the scalar base p.w (the host checks that
  // N x row stride < 4 GiB and the stride < 2^24): one 24-bit multiply-add
  // per load instead of 64-bit address arithmetic.
  const uint32_t ws32 = static_cast<uint32_t>(p.ws);
  auto wload = [&](int n, uint32_t ko, bool real) {
    return sd::load16_stream(p.w + sd::keep_or_zero32(real, __umul24(static_cast<uint32_t>(n), ws32) + ko));
  };
  auto load = [&](Regs& R, int g, int c, bool real) {
    const int s0 = ks + c * U;
    if constexpr (DIRECT) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int n = min(wrow(g, nt * 16 + lr), nrows - 1);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint32_t ko = static_cast<uint32_t>(min(s0 + u, p.nks - 1)) * 64u + lg * 16u;
        R.w[nt * U + u] = wload(n, ko, real);
      }
    }
    } else {
    const uint32_t kw_off = static_cast<uint32_t>(min(s0 + ld_step, p.nks - 1)) * 64u +
                            (ld_unit & 3) * 16u;
#pragma unroll
    for (int i = 0; i < NLD; ++i) R.w[i] = wload(min(wrow(g, i * RPI + ld_row), nrows - 1), kw_off, real);
    }
#pragma unroll
    for (int u = 0; u < (XL ? 0 : U); ++u) {
      const int64_t k0 = static_cast<int64_t>(min(s0 + u, p.nks - 1)) * 64;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if (xok[mt]) {
          R.x[u][mt][0] = sd::load16(xp[mt] + k0);
          R.x[u][mt][1] = sd::load16(xp[mt] + k0 + 8);
          if constexpr (SL) {
            R.xu[u][mt][0] = sd::load16(xp[mt] + p.up + k0);
            R.xu[u][mt][1] = sd::load16(xp[mt] + p.up + k0 + 8);
          }
        } else {
          R.x[u][mt][0] = u32x4{0u, 0u, 0u, 0u};
          R.x[u][mt][1] = u32x4{0u, 0u, 0u, 0u};
          if constexpr (SL) {
            R.xu[u][mt][0] = u32x4{0u, 0u, 0u, 0u};
            R.xu[u][mt][1] = u32x4{0u, 0u, 0u, 0u};
          }
        }
      }
    }
  };

  u32x4 fold = {0u, 0u, 0u, 0u};  // FLOOR: every loaded word is consumed here
  auto compute = [&](Regs& R, int g, int c) {
    if constexpr (FLOOR) {
#pragma unroll
      for (int i = 0; i < NLD; ++i) {
        fold.x ^= R.w[i].x;
        fold.y ^= R.w[i].y;
        fold.z ^= R.w[i].z;
        fold.w ^= R.w[i].w;
      }
#pragma unroll
      for (int u = 0; u < (XL ? 0 : U); ++u)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          fold.x ^= R.x[u][mt][0].x ^ R.x[u][mt][1].y;
          if constexpr (SL) fold.y ^= R.xu[u][mt][0].z ^ R.xu[u][mt][1].w;
        }
      return;
    }
    const int n0 = g * NT * 16;
    const int s0 = ks + c * U;
    // stage: row r = i * RPI + ld_row, unit ld_unit at position ld_unit ^ (r & 15)
    if constexpr (!DIRECT) {
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const int r = i * RPI + ld_row;
      sd::store16(tile + (r * LPR + (ld_unit ^ (r & SWZ))) * 16, R.w[i]);
    }
    sd::wave_lds_sync();
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int step = s0 + u;
      if (step >= ke) break;  // wave-uniform
      const int64_t k0 = static_cast<int64_t>(step) * 64;
      u32x4 xv[MT][2];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if constexpr (XL) {
          const char* xr = xsm + xro[mt] + step * 128 + lg * 32;
          xv[mt][0] = sd::load16(xr);
          xv[mt][1] = sd::load16(xr + 16);
        } else if constexpr (SL) {
          xv[mt][0] = sd::silu_mul8<T>(R.x[u][mt][0], R.xu[u][mt][0]);
          xv[mt][1] = sd::silu_mul8<T>(R.x[u][mt][1], R.xu[u][mt][1]);
        } else {
          xv[mt][0] = R.x[u][mt][0];
          xv[mt][1] = R.x[u][mt][1];
        }
      }
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int r = nt * 16 + lr;
        u32x4 wv;
        if constexpr (DIRECT) wv = R.w[nt * U + u];
        else wv = sd::load16(tile + (r * LPR + ((u * 4 + lg) ^ (r & SWZ))) * 16);
        const u32x4 a0 = dequant8<T>(wv.x, wv.y);  // k = 16 lg + 0..7
        const u32x4 a1 = dequant8<T>(wv.z, wv.w);  // k = 16 lg + 8..15
        if constexpr (!PER_GROUP) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            acc[nt][mt] = sd::Elem<T>::mfma(a0, xv[mt][0], acc[nt][mt]);
            acc[nt][mt] = sd::Elem<T>::mfma(a1, xv[mt][1], acc[nt][mt]);
          }
        } else {
          const int grp = static_cast<int>(k0 / p.group);
          const int ng = p.K / p.group;
          float sc[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if constexpr (XL) {
              sc[i] = scl[srow(g, nt * 16 + lg * 4 + i) * spr + grp];
            } else {
              const int n = min(n0 + nt * 16 + lg * 4 + i, p.N - 1);
              sc[i] = load_scale(p.scale, p.scale_dtype, static_cast<int64_t>(n) * ng + grp);
            }
          }
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            f32x4 t = {0.f, 0.f, 0.f, 0.f};
            t = sd::Elem<T>::mfma(a0, xv[mt][0], t);
            t = sd::Elem<T>::mfma(a1, xv[mt][1], t);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[nt][mt][i] += t[i] * sc[i];
          }
        }
      }
    }
    if constexpr (!DIRECT) sd::wave_lds_sync();  // every lane has read the tile before the next chunk overwrites it
  };

  // lane holds y^T[n = n0 + 16 nt + 4 lg + i][m = m0 + 16 mt + lr]
  auto epilogue = [&](int g) {
    if constexpr (FLOOR) return;
    if constexpr (KW > 1) {
      if (kw > 0) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) red[kw - 1][(nt * MT + mt) * 4 + i][lane] = acc[nt][mt][i];
      }
      __syncthreads();
      if (kw == 0) {
        // partials added in wave order (a few slots per pass: with 16 waves,
        // all 60 in flight would not fit the registers of a 1024-thread group)
#pragma unroll 3
        for (int w = 0; w < KW - 1; ++w)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
              for (int i = 0; i < 4; ++i) acc[nt][mt][i] += red[w][(nt * MT + mt) * 4 + i][lane];
      }
    }
    bool paired = false;
    if constexpr (PRC) {
      if (kw == 0 && pr) {
        paired = true;
        const int nb = g * 16 + lg * 4;  // output column (pair) of this lane's 4 sums
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int m = m0 + mt * 16 + lr;
          if (m >= p.M || nb >= p.N) continue;
          float o[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float v[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {  // gate, up: the projection's rounded output
              const int r = h * 16 + lg * 4 + i;
              float sc, bi;
              if constexpr (XL) {
                sc = scl[srow(g, r)];
                bi = p.bias ? bis[srow(g, r)] : 0.f;
              } else {
                const int n = wrow(g, r);
                sc = load_scale(p.scale, p.scale_dtype, n);
                bi = p.bias ? sd::from_bits<T>(p.bias[n]) : 0.f;
              }
              v[h] = sd::from_bits<T>(sd::to_bits<T>(acc[h][mt][i] * sc + bi));
            }
            o[i] = sd::silu_mul1<T>(v[0], v[1]);
          }
          uint16_t* dst = p.y + static_cast<int64_t>(m) * p.ys + nb;
          if (nb + 3 < p.N && (reinterpret_cast<uintptr_t>(dst) & 7u) == 0) {
            *reinterpret_cast<uint2*>(dst) =
                make_uint2(sd::pack2<T>(o[0], o[1]), sd::pack2<T>(o[2], o[3]));
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (nb + i < p.N) dst[i] = sd::to_bits<T>(o[i]);
          }
        }
      }
    }
    if (kw == 0 && !paired) {
      const int n0 = g * NT * 16;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = m0 + mt * 16 + lr;
        if (m >= p.M) continue;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const int nb = n0 + nt * 16 + lg * 4;
          if (nb >= p.N) continue;
          float v[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int n = min(nb + i, p.N - 1);
            float sc, bi;
            if constexpr (XL) {
              const int sr = srow(g, nt * 16 + lg * 4 + i);
              sc = PER_GROUP ? 1.f : scl[sr];
              bi = p.bias ? bis[sr] : 0.f;
            } else {
              sc = PER_GROUP ? 1.f : load_scale(p.scale, p.scale_dtype, n);
              bi = p.bias ? sd::from_bits<T>(p.bias[n]) : 0.f;
            }
            v[i] = acc[nt][mt][i] * sc + bi;
          }
          uint16_t* dst = p.y + static_cast<int64_t>(m) * p.ys + nb;
          if (nb + 3 < p.N && (reinterpret_cast<uintptr_t>(dst) & 7u) == 0) {
            *reinterpret_cast<uint2*>(dst) =
                make_uint2(sd::pack2<T>(v[0], v[1]), sd::pack2<T>(v[2], v[3]));
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (nb + i < p.N) dst[i] = sd::to_bits<T>(v[i]);
          }
        }
      }
    }
    if constexpr (KW > 1) __syncthreads();  // `red` is free for the next row group
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  };

  // ring of D register buffers: item i + D - 1 is loaded while item i computes
  Regs ring[D];
  // (row group, chunk) of the next item to load and of the next to compute,
  // each advanced one item at a time (uniform selects, no division per item)
  int lgp = g0, lcp = 0, cgp = g0, ccp = 0;
  auto advance = [&](int& g, int& c) {
    const bool wrap = c + 1 == nchunks;
    c = wrap ? 0 : c + 1;
    g = wrap ? g + gstride : g;
  };
  // XL staging: rows m0 .. m0 + rows of x (16-byte units), then the scale table
  // (and bias) of the rows every wave of this workgroup owns; all waves take
  // part. This thread's first SB units and first SC table entries load ahead of
  // the weight prefetch, with no branch (indices clamped into range; entries
  // past the end are loaded but not stored), so that waiting for them leaves
  // the prefetch in flight. A load under a bounds branch or in a loop is waited
  // for together with every load issued before it: the weight prefetch, then
  // one round trip per unit (28 before the first MFMA at 56 rows of K = 1024).
  // HOIST (whole rows per wave, no norm): SB activation units per thread and
  // batch, what K = 1024 asks of a thread (at most 8, 4 with the up halves),
  // and SC table entries per thread in the first batch. The K-split kernels
  // (2 - 4 units per thread) measured slower with it at 56 rows (qkv 6.55 ->
  // 6.91 us) and load one unit per thread and iteration; the norm's rows load
  // after the prefetch anyway.
  constexpr bool HOIST = XL && !NM && KW == 1;
  constexpr int SBK = MT * 16 * 128 / NTH;
  constexpr int SB = HOIST ? (SBK < 1 ? 1 : (SBK > (SL ? 4 : 8) ? (SL ? 4 : 8) : SBK)) : 1;
  constexpr int SC = HOIST ? (NSUB * RG * 2 > NTH ? 2 : 1) : 0;
  const int rows = XL ? min(MT * 16, p.M - m0) : 1;
  const int upr = p.K / 8;  // 16-byte units per row
  const int xtot = rows * upr;
  const int per_sub = p.ngmax * RG;
  const int stot = NSUB * per_sub * spr, btot = NSUB * per_sub;
  auto unit_src = [&](int idx) {
    idx = min(idx, xtot - 1);
    const int r = idx / upr, c = idx - r * upr;
    return p.x + static_cast<int64_t>(m0 + r) * p.xs + c * 8;
  };
  auto unit_dst = [&](int idx) {
    const int r = idx / upr, c = idx - r * upr;
    return xsm + r * p.xpitch + c * 16;
  };
  auto table_row = [&](int t) {  // weight row of table row t (clamped)
    const int sb = t / per_sub, gi = (t - sb * per_sub) / RG, r = t % RG;
    const int g = blockIdx.x * NSUB + sb + gi * gridDim.x * NSUB;
    return min(wrow(g, r), nrows - 1);
  };
  auto scale_elem = [&](int idx) -> int64_t {  // scale element of table entry idx
    idx = min(idx, max(stot, 1) - 1);
    const int j = idx % spr, n = table_row(idx / spr);
    return PER_GROUP ? static_cast<int64_t>(n) * spr + j : n;
  };
  // a scale as 16-bit halves at a uniform shift (fp32: two halves), the bias
  // read from the scale when there is none: one load form, no branch
  const int ssh = p.scale_dtype == SD_F32 ? 1 : 0;
  const uint16_t* s16 = static_cast<const uint16_t*>(p.scale);
  const uint16_t* bsrc = p.bias ? p.bias : s16;
  const int64_t bmask = p.bias ? ~int64_t{0} : int64_t{0};
  auto scale_val = [&](uint32_t h0, uint32_t h1) -> float {
    if (ssh) return __uint_as_float(h0 | (h1 << 16));
    const uint16_t h = static_cast<uint16_t>(h0);
    return p.scale_dtype == SD_BF16 ? sd::from_bits<__bf16>(h) : sd::from_bits<_Float16>(h);
  };
  u32x4 xa[SB], xu[SL ? SB : 1];
  uint32_t sh0[SC > 0 ? SC : 1], sh1[SC > 0 ? SC : 1];
  uint16_t bv[SC > 0 ? SC : 1];
  if constexpr (HOIST) {
#pragma unroll
    for (int j = 0; j < SB; ++j) {
      const uint16_t* src = unit_src(tid + j * NTH);
      xa[j] = sd::load16(src);
      if constexpr (SL) xu[j] = sd::load16(src + p.up);
    }
#pragma unroll
    for (int j = 0; j < SC; ++j) {
      const int64_t e = scale_elem(tid + j * NTH);
      sh0[j] = s16[e << ssh];
      sh1[j] = s16[(e << ssh) + ssh];
      bv[j] = bsrc[static_cast<int64_t>(table_row(min(tid + j * NTH, max(btot, 1) - 1))) & bmask];
    }
  }
#pragma unroll
  for (int d = 0; d < D - 1; ++d) {
    if (XL && nit == 0) break;
    load(ring[d], lgp, lcp, d < nit);
    if (d + 1 < nit) advance(lgp, lcp);  // past the end: the last item again (dummy loads)
  }
  if constexpr (XL) {
    if constexpr (NM) {
      // one wave per row, the waves' rows at the same time (the RMSNorm
      // kernel's bits, sd::add_rmsnorm_row_wave); one workgroup per row block
      // writes the residual sum. Every workgroup repeats this for its block.
      uint16_t* ro = p.nres && p.nres_out && blockIdx.x == 0 ? p.nres_out + m0 * p.nres_out_s : nullptr;
      const uint16_t* res = p.nres ? p.nres + m0 * p.nres_s : nullptr;
      auto row_by_row = [&]() {
        for (int r = wave; r < rows; r += NWV)
          sd::add_rmsnorm_row_wave<T>(p.x + (m0 + r) * p.xs, res ? res + r * p.nres_s : nullptr, p.nw,
                                      p.K, p.neps, reinterpret_cast<uint16_t*>(xsm + r * p.xpitch),
                                      ro ? ro + r * p.nres_out_s : nullptr);
      };
      // up to 4 rows per wave and K <= 1024: each wave's rows in one call,
      // every load of them in one round trip (a loop here would make the
      // compiler wait for the weight prefetch at its head)
      constexpr int NRW = (MT * 16 + NWV - 1) / NWV;
      if constexpr (NRW <= 4) {
        if (p.K <= 1024) {
          const int r0 = wave * NRW;
          if (r0 < rows)
            sd::add_rmsnorm_rows_wave<T, NRW>(
                p.x + (m0 + r0) * p.xs, p.xs, res ? res + r0 * p.nres_s : nullptr, p.nres_s, p.nw,
                p.K, p.neps, min(NRW, rows - r0), reinterpret_cast<uint16_t*>(xsm + r0 * p.xpitch),
                p.xpitch / 2, ro ? ro + r0 * p.nres_out_s : nullptr, p.nres_out_s);
        } else {
          row_by_row();
        }
      } else {
        row_by_row();
      }
    } else {
      // the first batch (loaded above), then SB units per thread at a time
      auto put = [&](int b0) {
#pragma unroll
        for (int j = 0; j < SB; ++j) {
          const int idx = b0 + tid + j * NTH;
          if (idx < xtot) {
            if constexpr (SL) sd::store16(unit_dst(idx), sd::silu_mul8<T>(xa[j], xu[j]));
            else sd::store16(unit_dst(idx), xa[j]);
          }
        }
      };
      if constexpr (HOIST) {
        put(0);
        for (int b0 = SB * NTH; b0 < xtot; b0 += SB * NTH) {
#pragma unroll
          for (int j = 0; j < SB; ++j) {
            const uint16_t* src = unit_src(b0 + tid + j * NTH);
            xa[j] = sd::load16(src);
            if constexpr (SL) xu[j] = sd::load16(src + p.up);
          }
          put(b0);
        }
      } else {
        for (int idx = tid; idx < xtot; idx += NTH) {
          const int r = idx / upr, c = idx - r * upr;
          const uint16_t* src = p.x + static_cast<int64_t>(m0 + r) * p.xs + c * 8;
          if constexpr (SL)
            sd::store16(xsm + r * p.xpitch + c * 16, sd::silu_mul8<T>(sd::load16(src), sd::load16(src + p.up)));
          else
            sd::store16(xsm + r * p.xpitch + c * 16, sd::load16(src));
        }
      }
    }
    if constexpr (HOIST) {
#pragma unroll
      for (int j = 0; j < SC; ++j) {
        const int idx = tid + j * NTH;
        if (idx < stot) scl[idx] = scale_val(sh0[j], sh1[j]);
        if (p.bias && idx < btot) bis[idx] = sd::from_bits<T>(bv[j]);
      }
      // table entries past the first batch (per-group scales, large tables)
      for (int idx = SC * NTH + tid; idx < stot; idx += NTH) {
        const int64_t e = scale_elem(idx);
        scl[idx] = scale_val(s16[e << ssh], s16[(e << ssh) + ssh]);
      }
      if (p.bias) {
        for (int t = SC * NTH + tid; t < btot; t += NTH)
          bis[t] = sd::from_bits<T>(p.bias[table_row(t)]);
      }
    } else {
      for (int idx = tid; idx < stot; idx += NTH) {
        const int j = idx % spr, t = idx / spr;
        const int sb = t / per_sub, gi = (t - sb * per_sub) / RG, r = t % RG;
        const int g = blockIdx.x * NSUB + sb + gi * gridDim.x * NSUB;
        const int n = min(wrow(g, r), nrows - 1);
        scl[idx] = load_scale(p.scale, p.scale_dtype,
                              PER_GROUP ? static_cast<int64_t>(n) * spr + j : n);
      }
      if (p.bias) {
        for (int t = tid; t < btot; t += NTH) {
          const int sb = t / per_sub, gi = (t - sb * per_sub) / RG, r = t % RG;
          const int g = blockIdx.x * NSUB + sb + gi * gridDim.x * NSUB;
          bis[t] = sd::from_bits<T>(p.bias[min(wrow(g, r), nrows - 1)]);
        }
      }
    }
    __syncthreads();
    if (nit == 0) return;
  }
  // Whole rounds of D items, then the last nit % D items (already loaded) after
  // the loop: an exit from inside a round would reach the loop head with this
  // round's loads still in flight, and the compiler then waits for every load
  // at the head, the prefetch of the next item included.
  int it = 0;
  for (; it + D <= nit; it += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int cur = it + d;
      // item cur + D - 1 (past the end: dummy loads)
      load(ring[(d + D - 1) % D], lgp, lcp, cur + D - 1 < nit);
      if (cur + D < nit) advance(lgp, lcp);
      compute(ring[d], cgp, ccp);
      if (ccp + 1 == nchunks) epilogue(cgp);
      advance(cgp, ccp);
    }
  }
#pragma unroll
  for (int d = 0; d < D - 1; ++d) {
    const int cur = it + d;
    if (cur >= nit) break;  // wave-uniform (workgroup-uniform when KW > 1)
    compute(ring[d], cgp, ccp);
    if (ccp + 1 == nchunks) epilogue(cgp);
    advance(cgp, ccp);
  }
  if constexpr (FLOOR) {
    // data-dependent and practically never true: the loads (and, staged, the
    // activation and scale table) cannot be dropped
    uint32_t f = fold.x ^ fold.y ^ fold.z ^ fold.w;
    if constexpr (XL) f ^= *reinterpret_cast<const uint32_t*>(xsm + (lane & 3) * 4) ^ __float_as_uint(scl[lane & 15]);
    if (f == 0x9E3779B9u && lane == 0) p.y[0] = static_cast<uint16_t>(f);
  }
}

// Lane `lane`'s activations of the row-streaming kernels, in two steps so that
// the caller's first weight loads go out between them: act_load issues every
// load the activations need, with no branch (row and column clamped into the
// matrix; K is a multiple of 8), and act_form forms xv[m][c][j], column
// c * 1024 + 16 lane + j of activation row m (zero past K or M), selecting the
// zeros once the data are in. A load under a per-lane bounds branch would be
// waited for where its branch ends, with every load issued before it: one
// round trip per branch. MODE 1 forms SiluAndMul (silu_mul8, the SiLU kernel's
// element function), MODE 2 add + RMSNorm with the RMSNorm kernel's summation
// order; `writer` (one wave of the grid) stores the new residual.
template <int MR, int C, int MODE>
struct RowActs {
  static constexpr int MB = MODE == 0 ? 1 : MR, CB = MODE == 0 ? 1 : C, CN = MODE == 2 ? C : 1;
  u32x4 a[MR][C][2];   // x (MODE 1: the gate half)
  u32x4 b[MB][CB][2];  // MODE 1: the up half; MODE 2: the residual (x again without one)
  u32x4 nw[CN][2];     // MODE 2: the norm weight
};

template <int MR, int C, int MODE>
__device__ __forceinline__ void act_load(const W8Params& p, int lane, RowActs<MR, C, MODE>& r) {
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    const int64_t mc = min(m, p.M - 1);
    const uint16_t* xr = p.x + mc * p.xs;
    const uint16_t* br = xr;
    if constexpr (MODE == 1) br = xr + p.up;
    if constexpr (MODE == 2) br = p.nres ? p.nres + mc * p.nres_s : xr;
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int k = min(c * 1024 + 16 * lane + 8 * e, p.K - 8);
        r.a[m][c][e] = sd::load16(xr + k);
        if constexpr (MODE != 0) r.b[m][c][e] = sd::load16(br + k);
      }
  }
  if constexpr (MODE == 2) {
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
      for (int e = 0; e < 2; ++e) r.nw[c][e] = sd::load16(p.nw + min(c * 1024 + 16 * lane + 8 * e, p.K - 8));
  }
}

template <typename T, int MR, int C, int MODE>
__device__ __forceinline__ void act_form(const W8Params& p, int lane, bool writer,
                                         const RowActs<MR, C, MODE>& r, float (&xv)[MR][C][16]) {
#pragma clang fp contract(off)
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    const bool mok = m < p.M;
    if constexpr (MODE == 2) {
      // s = x (+ residual) in fp32; the RMSNorm kernel's thread t holds the
      // 8-column chunks t, t + 256, ..., so chunk 128 c + 2 lane + e (e = 0, 1)
      // is thread 128 (c % 2) + 2 lane + e: lane halves < 32 / >= 32 are its
      // waves 0 / 1 (even c) and 2 / 3 (odd c), and its xor steps 32 .. 2
      // are lane xor 16 .. 1 here, step 1 the e pair
      const bool res = p.nres != nullptr;
      float ss[2][2] = {{0.f, 0.f}, {0.f, 0.f}};  // [c % 2][e]
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const int k0 = c * 1024 + 16 * lane;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const bool ok = mok && k0 + 8 * e < p.K;
          const u32x4 a = r.a[m][c][e], bq = r.b[m][c][e];
          const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, bw[4] = {bq.x, bq.y, bq.z, bq.w};
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float f = sd::from_bits<T>(static_cast<uint16_t>(aw[i / 2] >> (16 * (i & 1))));
            const float g = sd::from_bits<T>(static_cast<uint16_t>(bw[i / 2] >> (16 * (i & 1))));
            const float s = res ? f + g : f;
            xv[m][c][8 * e + i] = ok ? s : 0.f;
            ss[c & 1][e] += xv[m][c][8 * e + i] * xv[m][c][8 * e + i];  // + 0 past K
          }
          if (p.nres_out && writer && ok) {
            uint32_t ro[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) ro[i] = sd::pack2<T>(xv[m][c][8 * e + 2 * i], xv[m][c][8 * e + 2 * i + 1]);
            sd::store16(p.nres_out + static_cast<int64_t>(m) * p.nres_out_s + k0 + 8 * e,
                        u32x4{ro[0], ro[1], ro[2], ro[3]});
          }
        }
      }
      float wsum[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int e = 0; e < 2; ++e) ss[h][e] = sd::xor_sum_down<16>(ss[h][e]);
        wsum[h] = ss[h][0] + ss[h][1];
      }
      // the RMSNorm kernel's waves 0 - 3, in order
      float tot = 0.f;
      tot += sd::lane_value(wsum[0], 0);
      tot += sd::lane_value(wsum[0], 32);
      tot += sd::lane_value(wsum[1], 0);
      tot += sd::lane_value(wsum[1], 32);
      const float rn = rsqrtf(tot / static_cast<float>(p.K) + p.neps);
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const int k0 = c * 1024 + 16 * lane;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const bool ok = mok && k0 + 8 * e < p.K;
          const u32x4 wq = r.nw[c][e];
          const uint32_t ww[4] = {wq.x, wq.y, wq.z, wq.w};
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float n = static_cast<float>(sd::round16<T>(xv[m][c][8 * e + i] * rn));
            const float wv = sd::from_bits<T>(static_cast<uint16_t>(ww[i / 2] >> (16 * (i & 1))));
            const float o = static_cast<float>(sd::round16<T>(n * wv));
            xv[m][c][8 * e + i] = ok ? o : 0.f;
          }
        }
      }
    } else {
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const int k0 = c * 1024 + 16 * lane;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const bool ok = mok && k0 + 8 * e < p.K;
          u32x4 a = r.a[m][c][e];
          if constexpr (MODE == 1) a = sd::silu_mul8<T>(a, r.b[m][c][e]);
          const uint32_t aw[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float f = sd::from_bits<T>(static_cast<uint16_t>(aw[i / 2] >> (16 * (i & 1))));
            xv[m][c][8 * e + i] = ok ? f : 0.f;
          }
        }
      }
    }
  }
}

// ---- row-streaming GEMV for one or two activation rows (decode)
// Each wave owns a contiguous range of weight rows and streams them whole: a
// load instruction moves 1 KB of one row (lane l: bytes 16 l .. +16 of each
// 1024-column chunk), R rows per batch, two batches in flight. Lane l holds
// the activations of its columns (MR rows x C chunks x 16) in registers for
// the whole launch, formed once per wave: MODE 1 SiluAndMul (silu_mul8, the
// SiLU kernel's element function), MODE 2 add + RMSNorm with the RMSNorm
// kernel's summation order (below), so the fused forms equal their two-launch
// forms bit for bit. Products accumulate in fp32 per lane (one conversion and
// one FMA per weight), then the R x MR sums of a batch reduce across the
// lanes in one reduce-scatter (halving steps, then plain xor steps), so a
// row's result is always summed in the same order. No MFMA, no LDS: at a few
// rows the MFMA form spends its time on operand staging, not on math.
// Per-channel scales only (applied to the reduced sum).
template <int MR, int C, int R>
struct RowsShape {
  static constexpr int V = R * MR;  // sums per lane per batch (R: rows of a batch)
  static constexpr int LV = V == 16 ? 4 : (V == 8 ? 3 : (V == 4 ? 2 : (V == 2 ? 1 : 0)));
  static_assert((1 << LV) == V, "R * MR must be a power of two <= 16");
};

// PAIR (the gate_up projection with SiluAndMul, sd_w8a16_gate_up_silu): a
// wave owns output columns i (weight rows i and i + p.pair); a batch holds
// R / 2 gate rows then the R / 2 matching up rows. After the reduce-scatter
// the gate sum of a pair sits 32 lanes below its up sum, so one xor-32
// shuffle brings them together and the lower lane writes
// bf16(bf16(silu(g)) * u) of the two bf16-rounded sums — the bits that the
// linear followed by the SiLU kernel give.
// FLOOR: the measurement twin — the same grid, loads and prefetch, every
// loaded word folded into a register instead of the math, no output.
template <typename T, int MR, int C, int R, int MODE, bool PAIR = false, bool FLOOR = false>
__global__ __launch_bounds__(kThreads) void w8a16_rows_kernel(W8Params p, int rows_per_wave) {
#pragma clang fp contract(off)
  constexpr int V = RowsShape<MR, C, R>::V, LV = RowsShape<MR, C, R>::LV;
  constexpr int RP = PAIR ? R / 2 : R;  // output rows (pairs) per batch
  static_assert(!PAIR || (R % 2 == 0 && V / 2 * (64 >> LV) == 32), "pairs 32 lanes apart");
  const int lane = threadIdx.x & 63;
  const int gw = blockIdx.x * kWaves + (threadIdx.x >> 6);
  // batches of this wave: nbat of them, the j-th starting at output row base(j);
  // rows at or past r1 are clamped on load and never written
  const int r0 = gw * rows_per_wave;
  const int r1 = min(r0 + rows_per_wave, p.N);
  const int nbat = r0 < p.N ? (r1 - r0 + RP - 1) / RP : 0;
  if (nbat == 0) return;
  auto base = [&](int j) { return r0 + j * RP; };

  // weight row of batch row r for the output rows starting at rb
  auto wrow = [&](int rb, int r) -> int64_t {
    const int64_t o = min(rb + (PAIR ? r % RP : r), r1 - 1);
    return PAIR && r >= RP ? o + p.pair : o;
  };
  // ---- a batch: R weight rows, and the scale (and bias) of the row whose sum
  // this lane holds after the reduce-scatter, loaded together so that using
  // them never waits for the next batch's prefetch (vector loads complete in
  // order). The scale is read as 16-bit halves at a uniform shift (two halves
  // of an fp32 scale, or one 16-bit scale twice) and the bias from the scale
  // when there is none: one load form for every dtype, no branch.
  struct Batch {
    u32x4 w[R][C];
    uint32_t s0, s1, b;
  };
  const int srow = (lane >> (6 - LV)) / MR;  // batch row of this lane's sum
  const int ssh = p.scale_dtype == SD_F32 ? 1 : 0;
  const uint16_t* s16 = static_cast<const uint16_t*>(p.scale);
  const uint16_t* bsrc = p.bias ? p.bias : s16;
  const int64_t bmask = p.bias ? ~int64_t{0} : int64_t{0};
  auto load = [&](Batch& B, int rb) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t row = wrow(rb, r);
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const int k0 = min(c * 1024 + 16 * lane, p.K - 16);  // lanes past K: a valid address, unused
        B.w[r][c] = sd::load16_stream(p.w + row * p.ws + k0);
      }
    }
    const int64_t row = wrow(rb, srow);
    B.s0 = s16[row << ssh];
    B.s1 = s16[(row << ssh) + ssh];
    B.b = bsrc[row & bmask];
  };
  auto scale_of = [&](const Batch& B) -> float {
    if (ssh) return __uint_as_float(B.s0 | (B.s1 << 16));
    const uint16_t h = static_cast<uint16_t>(B.s0);
    return p.scale_dtype == SD_BF16 ? sd::from_bits<__bf16>(h) : sd::from_bits<_Float16>(h);
  };
  // ---- this lane's activations (xv[m][c][j] = column c * 1024 + 16 lane + j),
  // loaded ahead of the first batch and formed while it is in flight
  RowActs<MR, C, MODE> ra;
  act_load<MR, C, MODE>(p, lane, ra);
  Batch ba, bb;
  load(ba, base(0));
  float xv[MR][C][16];
  act_form<T, MR, C, MODE>(p, lane, gw == 0, ra, xv);

  u32x4 fold = {0u, 0u, 0u, 0u};  // FLOOR: every loaded word is consumed here
  auto consume = [&](const Batch& B, int rb) {
    if constexpr (FLOOR) {
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int c = 0; c < C; ++c) {
          fold.x ^= B.w[r][c].x;
          fold.y ^= B.w[r][c].y;
          fold.z ^= B.w[r][c].z;
          fold.w ^= B.w[r][c].w;
        }
      fold.x ^= B.s0 ^ (B.s1 << 8) ^ (B.b << 16);
      return;
    }
    float acc[V];
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int m = 0; m < MR; ++m) acc[r * MR + m] = 0.f;
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const uint32_t ww[4] = {B.w[r][c].x, B.w[r][c].y, B.w[r][c].z, B.w[r][c].w};
        float part[MR];
#pragma unroll
        for (int m = 0; m < MR; ++m) part[m] = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float q = static_cast<float>(static_cast<int8_t>(ww[i >> 2] >> (8 * (i & 3))));
#pragma unroll
          for (int m = 0; m < MR; ++m) part[m] = fmaf(q, xv[m][c][i], part[m]);
        }
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[r * MR + m] += part[m];
      }
    }
    // reduce-scatter: after the halving steps lane l holds sum (l >> (6 - LV))
#pragma unroll
    for (int h = V / 2, off = 32; h >= 1; h >>= 1, off >>= 1) {
      const bool upper = lane & off;
#pragma unroll
      for (int i = 0; i < h; ++i) {
        const float send = upper ? acc[i] : acc[i + h];
        const float keep = upper ? acc[i + h] : acc[i];
        acc[i] = keep + __shfl_xor(send, off);
      }
    }
    float v = acc[0];
#pragma unroll
    for (int off = 32 >> LV; off >= 1; off >>= 1) v += __shfl_xor(v, off);
    if constexpr (PAIR) {
      // every lane scales its sum, the gate half pairs with the up half
      const int idx = lane >> (6 - LV);
      const int r = idx / MR, m = idx - r * MR;
      v = v * scale_of(B);
      if (p.bias) v = v + sd::from_bits<T>(static_cast<uint16_t>(B.b));
      const float vb = sd::from_bits<T>(sd::to_bits<T>(v));  // the linear's rounding
      const float ub = __shfl_xor(vb, 32);
      const int orow = rb + r;
      if ((lane & ((64 >> LV) - 1)) == 0 && r < RP && orow < r1 && m < p.M)
        p.y[static_cast<int64_t>(m) * p.ys + orow] = sd::to_bits<T>(sd::silu_mul1<T>(vb, ub));
    } else if ((lane & ((64 >> LV) - 1)) == 0) {
      const int idx = lane >> (6 - LV);
      const int r = idx / MR, m = idx - r * MR;
      const int row = rb + r;
      if (row < r1 && m < p.M) {
        v = v * scale_of(B);
        if (p.bias) v = v + sd::from_bits<T>(static_cast<uint16_t>(B.b));
        p.y[static_cast<int64_t>(m) * p.ys + row] = sd::to_bits<T>(v);
      }
    }
  };
  for (int j = 0; j < nbat; j += 2) {
    load(bb, base(j + 1 < nbat ? j + 1 : j));
    consume(ba, base(j));
    if (j + 1 >= nbat) break;
    load(ba, base(j + 2 < nbat ? j + 2 : j));
    consume(bb, base(j + 1));
  }
  if constexpr (FLOOR) {
    // data-dependent and practically never true: the loads cannot be dropped
    float xs = 0.f;
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
      for (int c = 0; c < C; ++c)
#pragma unroll
        for (int i = 0; i < 16; ++i) xs += xv[m][c][i];
    const uint32_t f = fold.x ^ fold.y ^ fold.z ^ fold.w ^ __float_as_uint(xs);
    if (f == 0x9E3779B9u && lane == 0) p.y[0] = static_cast<uint16_t>(f);
  }
}

// ---- row-cyclic GEMV for one activation row on wide matrices (the lm_head)
// Weight row n belongs to wave n % W (W waves in the grid), so at any moment the
// grid streams one window of neighbouring rows, and each wave keeps two whole
// rows (C KB each) in flight: the load of row j + 2 is issued once row j has
// arrived (its address takes a zero computed from row j's data), then row j is
// computed. On a 151936 x 1024 matrix one or two 1 KB loads in flight per wave
// at 12 - 24 waves per CU read at the streaming rate (6.9 TB/s); four or more
// per wave (batches of contiguous rows) reached 5.5 - 6.5 TB/s.
// Workgroups are renumbered so that each XCD (hardware blocks b with equal
// b % 8) runs consecutive numbers: the 64 outputs of a 128-byte line of y, and
// the line of scales beside them, then belong to one XCD's L2 instead of
// eight (27.1 -> 25.8 us in the probe that chose this form).
// Four rows' sums reduce across the lanes with two lane-half swaps
// (v_permlane32_swap, v_permlane16_swap) and four DPP adds, without LDS; the
// scales (and bias) of a wave's next 64 rows are gathered once, one row per
// lane, and read back with v_readlane. fp16: each weight byte b becomes the
// exact fp16 value 1152 + b (b ^ 0x80 under exponent byte 0x64), the pairs
// accumulate in fp32 with v_dot2_f32_f16, and 1152 times the lane's activation
// sum comes off once per row (two instructions per 4 weights fewer than
// subtracting 1152 from each; the products stay exact, the larger fp32 partial
// sums add a rounding about 2^-8 of the 16-bit output's); bf16 takes one
// conversion and one FMA per weight. Per-channel scales only (applied to the
// reduced sum).
// FLOOR: the measurement twin: the same grid, loads and chain, every loaded
// word folded into a register instead of the math, no output.
#ifndef SD_W8_CYC_WGS_PER_CU
#define SD_W8_CYC_WGS_PER_CU 3
#endif
constexpr int kCycWgsPerCu = SD_W8_CYC_WGS_PER_CU;

// a[0..3] per lane -> every lane of 16-lane row r holds the wave's sum of a[r]
__device__ __forceinline__ float reduce4_rows(float a0, float a1, float a2, float a3) {
  // lanes 0-31 of a0 meet lanes 32-63 of a0 (and a2's halves the other way)
  auto x = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, a0),
                                            __builtin_bit_cast(uint32_t, a2), false, false);
  auto y = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, a1),
                                            __builtin_bit_cast(uint32_t, a3), false, false);
  const float s02 = __builtin_bit_cast(float, static_cast<uint32_t>(x[0])) +
                    __builtin_bit_cast(float, static_cast<uint32_t>(x[1]));  // a0 | a2
  const float s13 = __builtin_bit_cast(float, static_cast<uint32_t>(y[0])) +
                    __builtin_bit_cast(float, static_cast<uint32_t>(y[1]));  // a1 | a3
  // odd 16-lane rows of s02 meet even rows of s13: rows a0, a1, a2, a3
  auto z = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, s02),
                                            __builtin_bit_cast(uint32_t, s13), false, false);
  float v = __builtin_bit_cast(float, static_cast<uint32_t>(z[0])) +
            __builtin_bit_cast(float, static_cast<uint32_t>(z[1]));
  v = sd::dpp_add<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v = sd::dpp_add<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v = sd::dpp_add<0x141>(v);  // row_half_mirror
  v = sd::dpp_add<0x140>(v);  // row_mirror
  return v;
}

// 4 int8 b -> two pairs of the exact fp16 values 1152 + b (bytes 0, 1 and 2, 3):
// b ^ 0x80 under exponent byte 0x64 is 1024 + (b + 128)
__device__ __forceinline__ void int8x4_to_biased_f16x2(uint32_t w, sd::f16x2& lo, sd::f16x2& hi) {
  const uint32_t u = w ^ 0x80808080u;
  lo = __builtin_bit_cast(sd::f16x2, __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u));
  hi = __builtin_bit_cast(sd::f16x2, __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u));
}

template <typename T, int C, int MODE, bool FLOOR = false>
__global__ __launch_bounds__(kThreads) void w8a16_cyc_kernel(W8Params p) {
#pragma clang fp contract(off)
  constexpr int R = 4;  // rows per reduction
  const int lane = threadIdx.x & 63;
  const int nb = gridDim.x;  // a multiple of 8
  const int blk = (blockIdx.x & 7) * (nb >> 3) + (blockIdx.x >> 3);
  // the wave index in an SGPR: row addresses are scalar (base + j x stride), so a
  // row load is one instruction with a scalar base and the lane's offset
  const int gw = blk * kWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = nb * kWaves;
  const int n = gw < p.N ? (p.N - gw + W - 1) / W : 0;  // rows gw + j W, j < n
  if (n == 0) return;
  const int8_t* const wbase = p.w + static_cast<int64_t>(gw) * p.ws;
  const int64_t wstride = static_cast<int64_t>(W) * p.ws;  // bytes from row j to j + 1
  uint32_t koff[C];  // lanes past K: a valid offset, unused
#pragma unroll
  for (int c = 0; c < C; ++c) koff[c] = static_cast<uint32_t>(min(c * 1024 + 16 * lane, p.K - 16));
  typedef u32x4 Row[C];
  auto load_row = [&](Row& b, int j, uint32_t z) {
    const int8_t* src = wbase + j * wstride;
#pragma unroll
    for (int c = 0; c < C; ++c) b[c] = sd::load16_stream(src + (koff[c] + z));
  };
  // the activations' loads first, formed while the first two rows are in flight
  RowActs<1, C, MODE> ra;
  act_load<1, C, MODE>(p, lane, ra);
  Row buf[2];
  load_row(buf[0], 0, 0);
  load_row(buf[1], n > 1 ? 1 : 0, 0);

  float xv[1][C][16];
  act_form<T, 1, C, MODE>(p, lane, gw == 0, ra, xv);
  // fp16: the activations as exact pairs, and 1152 times their sum (this lane's
  // columns): each weight byte enters the dot products as the exact fp16 value
  // 1152 + b, and the 1152 x sum is taken off once per row
  uint32_t xp[C][8];
  float xoff = 0.f;
  if constexpr (!__is_same(T, __bf16)) {
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
      for (int i = 0; i < 8; ++i) xp[c][i] = sd::pack2<T>(xv[0][c][2 * i], xv[0][c][2 * i + 1]);
    float xs = 0.f;
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
      for (int i = 0; i < 16; ++i) xs += xv[0][c][i];
    xoff = 1152.f * xs;
  }
  auto dot = [&](const Row& b) -> float {
    float a = 0.f;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const uint32_t ww[4] = {b[c].x, b[c].y, b[c].z, b[c].w};
      if constexpr (__is_same(T, __bf16)) {
#pragma unroll
        for (int i = 0; i < 16; ++i)
          a = fmaf(static_cast<float>(static_cast<int8_t>(ww[i >> 2] >> (8 * (i & 3)))), xv[0][c][i], a);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          sd::f16x2 lo, hi;
          int8x4_to_biased_f16x2(ww[i], lo, hi);
          a = __builtin_amdgcn_fdot2(lo, __builtin_bit_cast(sd::f16x2, xp[c][2 * i]), a, false);
          a = __builtin_amdgcn_fdot2(hi, __builtin_bit_cast(sd::f16x2, xp[c][2 * i + 1]), a, false);
        }
      }
    }
    if constexpr (!__is_same(T, __bf16)) a = a - xoff;
    return a;
  };

  // scale / bias bits of row gw + (j0 + lane) W, gathered per 64 rows
  const bool s32 = p.scale_dtype == SD_F32;
  uint32_t sg = 0, bg = 0;
  auto scale_of = [&](uint32_t bits) -> float {
    if (s32) return __uint_as_float(bits);
    const uint16_t h = static_cast<uint16_t>(bits);
    return p.scale_dtype == SD_BF16 ? sd::from_bits<__bf16>(h) : sd::from_bits<_Float16>(h);
  };
  u32x4 fold = {0u, 0u, 0u, 0u};
  for (int j0 = 0; j0 < n; j0 += R) {
    if ((j0 & 63) == 0) {
      const int64_t row = gw + static_cast<int64_t>(min(j0 + lane, n - 1)) * W;
      sg = s32 ? static_cast<const uint32_t*>(p.scale)[row] : static_cast<const uint16_t*>(p.scale)[row];
      if (p.bias) bg = p.bias[row];
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      Row& slot = buf[r & 1];
      Row cur;
#pragma unroll
      for (int c = 0; c < C; ++c) cur[c] = slot[c];
      uint32_t z;  // 0 once row j0 + r has arrived: the next load waits for it
      asm volatile("v_and_b32 %0, 0, %1" : "=v"(z) : "v"(cur[C - 1].x));
      load_row(slot, min(j0 + r + 2, n - 1), z);
      if constexpr (FLOOR) {
#pragma unroll
        for (int c = 0; c < C; ++c) fold ^= cur[c];
        acc[r] = 0.f;
      } else {
        acc[r] = dot(cur);
      }
    }
    if constexpr (FLOOR) {
      fold.x ^= sg ^ (bg << 16);
      continue;
    }
    const float v = reduce4_rows(acc[0], acc[1], acc[2], acc[3]);
    const int r = lane >> 4, jb = j0 & 63;
    const uint32_t sb0 = __builtin_amdgcn_readlane(sg, jb), sb1 = __builtin_amdgcn_readlane(sg, jb + 1),
                   sb2 = __builtin_amdgcn_readlane(sg, jb + 2), sb3 = __builtin_amdgcn_readlane(sg, jb + 3);
    float out = v * scale_of(r == 0 ? sb0 : (r == 1 ? sb1 : (r == 2 ? sb2 : sb3)));
    if (p.bias) {
      const uint32_t bb0 = __builtin_amdgcn_readlane(bg, jb), bb1 = __builtin_amdgcn_readlane(bg, jb + 1),
                     bb2 = __builtin_amdgcn_readlane(bg, jb + 2), bb3 = __builtin_amdgcn_readlane(bg, jb + 3);
      out = out + sd::from_bits<T>(static_cast<uint16_t>(r == 0 ? bb0 : (r == 1 ? bb1 : (r == 2 ? bb2 : bb3))));
    }
    const int j = j0 + r;
    if ((lane & 15) == 0 && j < n)
      p.y[gw + static_cast<int64_t>(j) * W] = sd::to_bits<T>(out);
  }
  if constexpr (FLOOR) {
    // data-dependent and practically never true: the loads cannot be dropped
    float xs = 0.f;
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
      for (int i = 0; i < 16; ++i) xs += xv[0][c][i];
    const uint32_t f = fold.x ^ fold.y ^ fold.z ^ fold.w ^ __float_as_uint(xs);
    if (f == 0x9E3779B9u && lane == 0) p.y[0] = static_cast<uint16_t>(f);
  }
}

// Rows per wave and grid of the row-streaming kernel: about 4 rows per wave,
// at most 8 waves per CU (two per SIMD) over the whole matrix.
struct RowsPlan {
  int blocks, rows_per_wave, R;
};

struct W8Plan {
  int MT, NT, KW, mblocks, groups, grid;
};

W8Plan make_plan(int64_t M, int64_t N, int64_t K) {
  W8Plan pl;
  // Activation rows in blocks of 16 (MT = 1), 32 (MT = 2) or 64 (MT = 4) along
  // grid.y. Every block streams the whole weight matrix, and a second block
  // only hits L2 while it runs in step with the first: with the weight loads
  // pipelined the blocks drift apart (lm_head M = 56 as two 32-row blocks
  // fetched 1.75x the weight bytes from HBM), so up to 64 rows (K <= 1024,
  // staged in one workgroup's LDS) are one block.
  pl.MT = M <= 16 ? 1 : (M <= 32 || K > 1024 || N <= 16 ? 2 : 4);
  pl.mblocks = static_cast<int>((M + pl.MT * 16 - 1) / (pl.MT * 16));
  const int64_t nr = (N + 15) / 16;
  const int cus = sd::device_cus();
  const int64_t nks = K / 64;
  // Enough 16-row tiles for ~8 waves per CU: every wave owns whole rows, two
  // tiles at a time. Otherwise KW waves of one workgroup split K of one tile
  // (16 activation rows) and their partials meet in LDS in wave order: 16 or
  // 8 when that keeps at most about 16 waves per CU busy with whole 2-step
  // chunks each (a narrow layer has too few tiles to fill the GPU with 4:
  // N = 1024 is 64 workgroups), else 4.
  if (nr * pl.mblocks >= 8ll * cus || nks < 4) {
    pl.KW = 1;
    // 16-row groups balance better over the waves (lm_head M = 1: 29.0 vs
    // 30.0 us); from M = 8 up, 32-row groups reuse each activation read twice
    pl.NT = nr < 2 || M <= 4 ? 1 : 2;
  } else {
    pl.NT = 1;
    pl.MT = 1;
    pl.mblocks = static_cast<int>((M + 15) / 16);
    const int64_t tiles = nr * pl.mblocks;
    // (whole 2-step chunks per wave: a partial chunk loads steps nobody uses)
    pl.KW = tiles * 16 <= 16ll * cus && nks % 32 == 0 ? 16
            : (tiles * 8 <= 16ll * cus && nks % 16 == 0 ? 8 : 4);
  }
  pl.groups = static_cast<int>((nr + pl.NT - 1) / pl.NT);
  const int nsub = pl.KW > 1 ? 1 : kWaves;
  const int64_t need = (pl.groups + nsub - 1) / nsub;
  pl.grid = static_cast<int>(need < (1 << 30) ? need : (1 << 30));  // capped at launch
  return pl;
}

// Resident workgroups per CU of one kernel instance (cached per device).
// Resident workgroups per CU of kernel `kern` with `smem` bytes of dynamic
// LDS on the current device, cached per (kernel, device, smem): every
// instance of the kernel template has the same function type, so the key must
// be the kernel's address.
int resident_wgs_of(const void* kern, size_t smem, int threads = kThreads) {
  struct Entry {
    const void* kern;
    int dev;
    size_t smem;
    int n;
  };
  static Entry table[512];
  static int used = 0;
  static std::mutex mu;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  {
    std::lock_guard<std::mutex> lock(mu);
    for (int i = 0; i < used; ++i)
      if (table[i].kern == kern && table[i].dev == dev && table[i].smem == smem) return table[i].n;
  }
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, threads, smem) != hipSuccess || n <= 0)
    n = 1;
  std::lock_guard<std::mutex> lock(mu);
  if (used < 512) table[used++] = Entry{kern, dev, smem, n};
  return n;
}

template <typename Kern>
int resident_wgs(Kern kern, int threads = kThreads) {
  return resident_wgs_of(reinterpret_cast<const void*>(kern), 0, threads);
}

// Activation rows staged in LDS (XL): bytes per row pad and the most a
// workgroup stages (32 rows of K <= 1024).
constexpr int kXPad = 16;
constexpr int kXlMaxBytes = 32 * (1024 * 2 + kXPad);
// 64-row blocks (MT = 4): one workgroup per CU holds the rows.
constexpr int kXlMaxBytes64 = 64 * (1024 * 2 + kXPad);
// K-split kernels (narrow layers, about one row group per workgroup) stage only
// when the activation block is large enough to pay for the staging (M > 16
// rows) and small enough to stage fast (16 rows of K <= 1024), or when the
// SiLU of a fused down projection is computed there (once per workgroup).
constexpr int kXlMaxBytesSplit = 16 * (1024 * 2 + kXPad);
// The most LDS the scale table may take (per group and bias included).
constexpr int kXlScaleBytes = 32 * 1024;

template <typename Kern>
int resident_wgs_xl(Kern kern, size_t smem, int threads = kThreads) {
  return resident_wgs_of(reinterpret_cast<const void*>(kern), smem, threads);
}

// Static LDS of w8a16_kernel<.., MT, NT, KW, U, ..>: the weight tiles and the
// K-split reduction slot, as the kernel declares them.
template <int MT, int NT, int KW, int U, bool XL, int NWV = kWaves>
constexpr size_t w8_static_lds() {
  return static_cast<size_t>(NWV) * (XL && MT >= 2 ? 16 : 16 * NT * 4 * U * 16) +
         static_cast<size_t>(KW > 1 ? KW - 1 : 1) * (NT * MT * 4) * 64 * 4;
}

template <typename T, int MT, int NT, int KW, bool PG, int MODE, bool FLOOR = false>
int launch_k(const W8Params& p, dim3 grid, hipStream_t st) {
  // 64-k steps per chunk: 2 where a wave's K slice is a few steps (8 or 16
  // slices) or the chunk covers 32 rows
  constexpr int U = NT >= 2 || KW >= 8 ? 2 : 4;
  // K-split workgroups have one wave per K slice; whole-row ones four waves
  constexpr int NWV = KW > 1 ? KW : kWaves;
  constexpr int NTH = NWV * 64;
  {
    // activation rows staged in LDS (XL): wide layers up to kXlMaxBytes (their
    // occupancy matters); K-split kernels as kXlMaxBytesSplit says
    const int rows = static_cast<int>(p.M < MT * 16 ? p.M : MT * 16);
    const size_t xbytes = static_cast<size_t>(rows) * p.xpitch;
    const size_t xmax = static_cast<size_t>(KW == 1 ? (MT == 4 ? kXlMaxBytes64 : kXlMaxBytes)
                                                    : kXlMaxBytesSplit);
    if (p.xpitch > 0 && xbytes <= xmax && (KW == 1 || MODE != 0 || p.M > 16)) {
      // 32 or 64 staged rows (MT >= 2) load the weights straight into MFMA
      // operand order, no weight tile: two workgroups per CU fit beside 32
      // rows, one beside 64, and 2-step chunks measured best there (lm_head
      // M = 56, two 32-row blocks before the loads were pipelined: 63.8 us;
      // 8-step chunks through the tile at one workgroup per CU: 77.8 us)
      constexpr int UX = MT >= 2 ? 2 : U;
      constexpr int NSUB = NWV / KW;
      auto kern = w8a16_kernel<T, MT, NT, KW, UX, PG, false, 2, true, MODE, NWV, FLOOR>;
      // occupancy from the activation rows; the scale table adds a few KB (per
      // channel: 16 B per row of the workgroup)
      unsigned cap = static_cast<unsigned>(sd::device_cus() * resident_wgs_xl(kern, xbytes, NTH)) /
                     grid.y;
      cap = cap >= 8 ? cap / 8 * 8 : 1;
      if (grid.x > cap) grid.x = cap;
      W8Params q = p;
      q.xbytes = static_cast<int32_t>((xbytes + 15) / 16 * 16);
      q.ngmax = (p.groups + static_cast<int>(grid.x) * NSUB - 1) / (static_cast<int>(grid.x) * NSUB);
      const size_t spr = PG ? static_cast<size_t>(p.K / p.group) : 1;
      const size_t tbl = static_cast<size_t>(NSUB) * q.ngmax * NT * 16 * (spr + (p.bias ? 1 : 0)) * 4;
      const size_t lds = w8_static_lds<MT, NT, KW, UX, true, NWV>() + q.xbytes + tbl;
      if (tbl <= static_cast<size_t>(kXlScaleBytes) &&
          lds <= static_cast<size_t>(sd::device_lds_per_block())) {
        hipLaunchKernelGGL(kern, grid, dim3(NTH), q.xbytes + tbl, st, q);
        return SD_OK;
      }
    }
  }
  if constexpr (MODE == 2) {
    // the norm needs the rows staged: no register form
    sd::set_error("w8a16_rmsnorm: the activation block (%d rows of K = %d) does not fit the "
                  "staging LDS", static_cast<int>(p.M < MT * 16 ? p.M : MT * 16), p.K);
    return SD_ERR_UNSUPPORTED;
  } else {
    auto kern = w8a16_kernel<T, MT, NT, KW, U, PG, false, 2, false, MODE, NWV, FLOOR>;
    // exactly one resident set of workgroups over all activation blocks (a
    // partial second round would leave most of the GPU idle at the end), grid.x
    // a multiple of 8 so that block (x, y) shares an XCD (and its L2) with (x, 0)
    unsigned cap = static_cast<unsigned>(sd::device_cus() * resident_wgs(kern, NTH)) / grid.y;
    cap = cap >= 8 ? cap / 8 * 8 : 1;
    if (grid.x > cap) grid.x = cap;
    hipLaunchKernelGGL(kern, grid, dim3(NTH), 0, st, p);
    return SD_OK;
  }
}

template <typename T, bool PG, int KW, int MODE, bool FLOOR = false>
int launch_kw(const W8Params& p, const W8Plan& pl, dim3 grid, hipStream_t st) {
  if constexpr (KW == 1) {
    switch (pl.MT * 8 + pl.NT) {
      case 1 * 8 + 1: return launch_k<T, 1, 1, 1, PG, MODE, FLOOR>(p, grid, st);
      case 1 * 8 + 2: return launch_k<T, 1, 2, 1, PG, MODE, FLOOR>(p, grid, st);
      case 2 * 8 + 1: return launch_k<T, 2, 1, 1, PG, MODE, FLOOR>(p, grid, st);
      case 4 * 8 + 2: return launch_k<T, 4, 2, 1, PG, MODE, FLOOR>(p, grid, st);
      default: return launch_k<T, 2, 2, 1, PG, MODE, FLOOR>(p, grid, st);
    }
  } else {
    if (p.pair > 0) {  // gate_up with the SiLU epilogue: gate and up tile per group
      if constexpr (!PG && MODE != 1 && !FLOOR) return launch_k<T, 1, 2, KW, PG, MODE>(p, grid, st);
      else return SD_ERR_UNSUPPORTED;
    }
    return launch_k<T, 1, 1, KW, PG, MODE, FLOOR>(p, grid, st);  // make_plan sets MT = 1 with KW > 1
  }
}

template <typename T, int MODE, bool FLOOR = false>
int launch_all(const W8Params& p, const W8Plan& pl, hipStream_t st) {
  int rc;
  const dim3 grid(static_cast<unsigned>(pl.grid), static_cast<unsigned>(pl.mblocks));
  if (p.group == 0) {
    switch (pl.KW) {
      case 1: rc = launch_kw<T, false, 1, MODE, FLOOR>(p, pl, grid, st); break;
      case 16: rc = launch_kw<T, false, 16, MODE, FLOOR>(p, pl, grid, st); break;
      case 8: rc = launch_kw<T, false, 8, MODE, FLOOR>(p, pl, grid, st); break;
      default: rc = launch_kw<T, false, 4, MODE, FLOOR>(p, pl, grid, st); break;
    }
  } else {
    if constexpr (FLOOR) {
      sd::set_error("w8a16_floor: per-channel scales only");
      return SD_ERR_UNSUPPORTED;
    } else {
      switch (pl.KW) {
        case 1: rc = launch_kw<T, true, 1, MODE>(p, pl, grid, st); break;
        case 16: rc = launch_kw<T, true, 16, MODE>(p, pl, grid, st); break;
        case 8: rc = launch_kw<T, true, 8, MODE>(p, pl, grid, st); break;
        default: rc = launch_kw<T, true, 4, MODE>(p, pl, grid, st); break;
      }
    }
  }
  if (rc != SD_OK) return rc;
  return sd::check_launch(FLOOR ? "w8a16 floor" : "w8a16");
}

// Row-streaming path: one or two activation rows with M * ceil(K / 1024) <= 4
// and a per-channel scale. Up to 32 MiB of weights (the decoder layers' linears,
// where launch latency dominates) each wave owns a contiguous range of about 4
// rows; the tiled kernel is faster from 4 rows up (qkv at M = 7: 4.6 vs 4.9 us
// with 8 rows here). Past 32 MiB (the lm_head) one row takes the row-cyclic
// kernel (w8a16_cyc_kernel); its batch-cyclic predecessor (4-row batches, two
// in flight, 16 waves per CU) took 26.6 - 29.7 us at 151936 x 1024 against
// 29.9 us on the tiled kernel.
// The rule is the same for the plain, SiLU and norm forms, so a fused call and
// its two-launch form always run the same GEMV. Paired rows (gate_up with the
// SiLU epilogue) take it up to 32 MiB only.
constexpr int64_t kRowsNarrowBytes = int64_t{32} << 20;

bool rows_eligible(const W8Params& p, bool pair) {
  const int C = (p.K + 1023) / 1024;
  if (p.M > 2 || p.M * C > 4 || p.group != 0) return false;
  if (static_cast<int64_t>(p.N) * p.K <= kRowsNarrowBytes) return true;
  return p.M == 1 && !pair;
}

template <typename T, int MR, int C, int MODE, bool PAIR = false, bool FLOOR = false>
int launch_rows_c(const W8Params& p, hipStream_t st) {
  if constexpr (MR == 1 && !PAIR) {
    if (static_cast<int64_t>(p.N) * p.K > kRowsNarrowBytes) {
      // row-cyclic (w8a16_cyc_kernel): a grid of a multiple of 8 workgroups
      // (the XCD renumbering), kCycWgsPerCu per CU
      int64_t blocks = static_cast<int64_t>(sd::device_cus()) * kCycWgsPerCu;
      const int64_t need = (static_cast<int64_t>(p.N) + kWaves - 1) / kWaves;
      if (blocks > need) blocks = need;
      blocks = (blocks + 7) / 8 * 8;
      hipLaunchKernelGGL((w8a16_cyc_kernel<T, C, MODE, FLOOR>), dim3(static_cast<unsigned>(blocks)),
                         dim3(kThreads), 0, st, p);
      return SD_OK;
    }
  }
  // One weight row per wave (two output pairs with PAIR) up to two waves per
  // SIMD (8 per CU), more rows per wave beyond; a batch holds the rows a wave
  // owns (1, 2 or 4; 8 for long ranges). At one or two rows these launches are
  // latency-bound, and more waves put more loads in flight at once: against 4
  // rows per wave, the down projection (1024 x 3072) went 4.5 -> 3.2 us and
  // o_proj (1024 x 2048) 3.7 -> 2.9 at M = 1 (1024 waves instead of 256).
  int64_t waves = static_cast<int64_t>(sd::device_cus()) * 8;
  const int64_t want = PAIR ? (static_cast<int64_t>(p.N) + 1) / 2 : static_cast<int64_t>(p.N);
  if (want < waves) waves = want;
  const int blocks = static_cast<int>((waves + kWaves - 1) / kWaves);
  const int rpw = static_cast<int>((p.N + static_cast<int64_t>(blocks) * kWaves - 1) /
                                   (static_cast<int64_t>(blocks) * kWaves));
  if constexpr (PAIR) {
    // 4 weight rows (2 pairs) per batch where a wave owns at most 2 pairs, or
    // from three column chunks up (two batches of 8 rows would fill the
    // register file); 8 rows (4 pairs) otherwise
    if (C >= 3 || rpw <= 2) {
      hipLaunchKernelGGL((w8a16_rows_kernel<T, MR, C, 4, MODE, true, FLOOR>), dim3(blocks),
                         dim3(kThreads), 0, st, p, rpw);
    } else {
      hipLaunchKernelGGL((w8a16_rows_kernel<T, MR, C, C >= 3 ? 4 : 8, MODE, true, FLOOR>),
                         dim3(blocks), dim3(kThreads), 0, st, p, rpw);
    }
    return SD_OK;
  }
  if constexpr (MR == 1 && C == 1) {
    if (rpw >= 32) {
      hipLaunchKernelGGL((w8a16_rows_kernel<T, 1, 1, 8, MODE, false, FLOOR>), dim3(blocks),
                         dim3(kThreads), 0, st, p, rpw);
      return SD_OK;
    }
  }
  if (rpw <= 1) {
    hipLaunchKernelGGL((w8a16_rows_kernel<T, MR, C, 1, MODE, false, FLOOR>), dim3(blocks),
                       dim3(kThreads), 0, st, p, rpw);
  } else if (rpw <= 2) {
    hipLaunchKernelGGL((w8a16_rows_kernel<T, MR, C, 2, MODE, false, FLOOR>), dim3(blocks),
                       dim3(kThreads), 0, st, p, rpw);
  } else {
    hipLaunchKernelGGL((w8a16_rows_kernel<T, MR, C, 4, MODE, false, FLOOR>), dim3(blocks),
                       dim3(kThreads), 0, st, p, rpw);
  }
  return SD_OK;
}

template <typename T, int MODE, bool PAIR = false, bool FLOOR = false>
int launch_rows(const W8Params& p, hipStream_t st) {
  const int C = (p.K + 1023) / 1024;
  int rc;
  if (p.M == 1) {
    switch (C) {
      case 1: rc = launch_rows_c<T, 1, 1, MODE, PAIR, FLOOR>(p, st); break;
      case 2: rc = launch_rows_c<T, 1, 2, MODE, PAIR, FLOOR>(p, st); break;
      case 3: rc = launch_rows_c<T, 1, 3, MODE, PAIR, FLOOR>(p, st); break;
      default: rc = launch_rows_c<T, 1, 4, MODE, PAIR, FLOOR>(p, st); break;
    }
  } else {
    rc = C == 1 ? launch_rows_c<T, 2, 1, MODE, PAIR, FLOOR>(p, st)
                : launch_rows_c<T, 2, 2, MODE, PAIR, FLOOR>(p, st);
  }
  if (rc != SD_OK) return rc;
  return sd::check_launch(FLOOR ? "w8a16 rows floor" : "w8a16 rows");
}

template <typename T>
int launch_rows_any(const W8Params& p, int mode, hipStream_t st) {
  if (p.pair > 0) {  // gate_up with the SiLU epilogue: plain or norm activations
    if (mode == 2) return launch_rows<T, 2, true>(p, st);
    return launch_rows<T, 0, true>(p, st);
  }
  if (mode == 1) return launch_rows<T, 1>(p, st);
  if (mode == 2) return launch_rows<T, 2>(p, st);
  return launch_rows<T, 0>(p, st);
}

}  // namespace

extern "C" size_t sd_w8a16_workspace_size(int64_t M, int64_t N, int64_t K, int32_t group_size) {
  (void)M;
  (void)N;
  (void)K;
  (void)group_size;
  return 0;  // one launch; K splits are reduced inside the workgroup
}

namespace {

// Activation forms of the entry points: plain; SiluAndMul of a gate_up row
// whose up half starts `up` elements after its gate half (up >= 0); add +
// RMSNorm (norm->weight != NULL).
struct NormArgs {
  const void* weight;  // NULL: no norm
  const void* residual;
  int64_t residual_stride;
  void* residual_out;
  int64_t residual_out_stride;
  float eps;
};

// pair: the gate_up projection with the SiLU epilogue (N weight rows, N / 2
// output columns; row-streaming path only)
int run_w8a16(const void* x, int64_t x_stride_m, int64_t up, const NormArgs& norm,
              const int8_t* w, int64_t w_stride_n, const void* scale, int32_t scale_dtype,
              int32_t group_size, const void* bias, void* y, int64_t y_stride_m, int64_t M,
              int64_t N, int64_t K, int32_t dtype, void* stream, bool pair = false,
              bool floor = false) {
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
  if (x_stride_m < 0 || y_stride_m < 0 || w_stride_n < 0 || norm.residual_stride < 0 ||
      norm.residual_out_stride < 0 ||
      !sd::strides_ok({x_stride_m, y_stride_m, w_stride_n, norm.residual_stride,
                       norm.residual_out_stride})) {
    sd::set_error("w8a16: strides must lie in [0, 2^40] elements");
    return SD_ERR_VALUE;
  }
  // the tiled kernel addresses weight bytes with 32-bit offsets formed by one
  // 24 x 24-bit multiply-add (row index x row stride), so both factors must
  // stay below 2^24 and their product below 2^32
  if (N >= (1ll << 24) || w_stride_n >= (1ll << 24) || N * w_stride_n >= (1ll << 32)) {
    sd::set_error("w8a16: the weight matrix must have fewer than 2^24 rows, a row stride below "
                  "2^24 bytes and span less than 4 GiB (N=%lld, stride=%lld)", (long long)N,
                  (long long)w_stride_n);
    return SD_ERR_UNSUPPORTED;
  }
  if (!sd::aligned16(x) || !sd::aligned16(w) || x_stride_m % 8 != 0 || w_stride_n % 16 != 0 ||
      (up >= 0 && up % 8 != 0)) {
    sd::set_error("w8a16: x and w rows (and the up half) must be 16-byte aligned");
    return SD_ERR_UNSUPPORTED;
  }
  // Other workgroups read x / residual while a workgroup writes y and
  // residual_out, so no output may share a byte with an input or with the
  // other output.
  const int64_t xw = up >= 0 ? up + K : K;
  const sd::Span sx = sd::span16(x, M, x_stride_m, xw),
                 sy = sd::span16(y, M, y_stride_m, pair ? N / 2 : N);
  const sd::Span sr = sd::span16(norm.residual, M, norm.residual_stride, K);
  const sd::Span sro = sd::span16(norm.residual_out, M, norm.residual_out_stride, K);
  if (sy.overlaps(sx) || sy.overlaps(sr) || sy.overlaps(sro) || sro.overlaps(sx) ||
      sro.overlaps(sr)) {
    sd::set_error("w8a16: y / residual_out overlap an input or each other (other workgroups "
                  "still read the inputs)");
    return SD_ERR_VALUE;
  }
  const W8Plan pl = make_plan(M, N, K);
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
  p.groups = pl.groups;
  // staged activation rows (wide path): K * 2 bytes + a 16-byte pad per row, so
  // that the 16 rows of a B-operand read start 4 banks apart
  p.xpitch = K <= 16384 ? static_cast<int32_t>(K * 2 + kXPad) : 0;
  p.xbytes = 0;
  p.ngmax = 0;
  p.up = up;
  p.nw = static_cast<const uint16_t*>(norm.weight);
  p.nres = static_cast<const uint16_t*>(norm.residual);
  p.nres_s = norm.residual_stride;
  p.nres_out = static_cast<uint16_t*>(norm.residual_out);
  p.nres_out_s = norm.residual_out_stride;
  p.neps = norm.eps;
  p.pair = 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int mode = up >= 0 ? 1 : (p.nw ? 2 : 0);
  if (pair) {
    // the row-streaming path (one or two rows), or the K-split tiled path with
    // the plain projection's plan (same K split, so the same sums), per-channel
    // scales and whole 16-row tiles of pairs
    const bool rows = N % 2 == 0 && rows_eligible(p, true);
    const bool tiled = N % 32 == 0 && pl.KW > 1 && group_size == 0 && mode != 1;
    if (!rows && !tiled) {
      sd::set_error("w8a16_gate_up_silu: the SiLU epilogue runs on the row-streaming path "
                    "(one or two rows, M * ceil(K / 1024) <= 4, per-channel scales, at most "
                    "32 MiB of weights, N even) or on the K-split path (narrow layers, "
                    "per-channel scales, N a multiple of 32); got M=%lld N=%lld K=%lld group=%d",
                    (long long)M, (long long)N, (long long)K, group_size);
      return SD_ERR_UNSUPPORTED;
    }
    p.pair = static_cast<int32_t>(N / 2);
    p.N = static_cast<int32_t>(N / 2);
    if (rows) {
      if (dtype == SD_BF16) return launch_rows_any<__bf16>(p, mode, st);
      return launch_rows_any<_Float16>(p, mode, st);
    }
    W8Plan pp = pl;
    pp.NT = 2;
    pp.groups = static_cast<int>(N / 32);
    pp.grid = pp.groups;
    p.groups = pp.groups;
    if (mode == 2) {
      if (dtype == SD_BF16) return launch_all<__bf16, 2>(p, pp, st);
      return launch_all<_Float16, 2>(p, pp, st);
    }
    if (dtype == SD_BF16) return launch_all<__bf16, 0>(p, pp, st);
    return launch_all<_Float16, 0>(p, pp, st);
  }
  if (floor) {  // the plain form's plan with the load-only kernels
    if (rows_eligible(p, false)) {
      if (dtype == SD_BF16) return launch_rows<__bf16, 0, false, true>(p, st);
      return launch_rows<_Float16, 0, false, true>(p, st);
    }
    if (dtype == SD_BF16) return launch_all<__bf16, 0, true>(p, pl, st);
    return launch_all<_Float16, 0, true>(p, pl, st);
  }
  if (rows_eligible(p, false)) {
    if (dtype == SD_BF16) return launch_rows_any<__bf16>(p, mode, st);
    return launch_rows_any<_Float16>(p, mode, st);
  }
  if (up >= 0) {
    if (dtype == SD_BF16) return launch_all<__bf16, 1>(p, pl, st);
    return launch_all<_Float16, 1>(p, pl, st);
  }
  if (p.nw) {
    if (dtype == SD_BF16) return launch_all<__bf16, 2>(p, pl, st);
    return launch_all<_Float16, 2>(p, pl, st);
  }
  if (dtype == SD_BF16) return launch_all<__bf16, 0>(p, pl, st);
  return launch_all<_Float16, 0>(p, pl, st);
}

}  // namespace

extern "C" int sd_w8a16_linear(const void* x, int64_t x_stride_m, const int8_t* w,
                               int64_t w_stride_n, const void* scale, int32_t scale_dtype,
                               int32_t group_size, const void* bias, void* y, int64_t y_stride_m,
                               int64_t M, int64_t N, int64_t K, int32_t dtype, void* workspace,
                               size_t workspace_bytes, void* stream) {
  sd::clear_error();
  (void)workspace;
  (void)workspace_bytes;
  return run_w8a16(x, x_stride_m, -1, NormArgs{}, w, w_stride_n, scale, scale_dtype, group_size,
                   bias, y, y_stride_m, M, N, K, dtype, stream);
}

extern "C" int sd_w8a16_floor(const void* x, int64_t x_stride_m, const int8_t* w,
                              int64_t w_stride_n, const void* scale, int32_t scale_dtype,
                              const void* bias, void* y, int64_t y_stride_m, int64_t M, int64_t N,
                              int64_t K, int32_t dtype, void* stream) {
  sd::clear_error();
  return run_w8a16(x, x_stride_m, -1, NormArgs{}, w, w_stride_n, scale, scale_dtype, 0, bias, y,
                   y_stride_m, M, N, K, dtype, stream, false, true);
}

extern "C" int sd_w8a16_silu_linear(const void* gate_up, int64_t gate_up_stride_m,
                                    const int8_t* w, int64_t w_stride_n, const void* scale,
                                    int32_t scale_dtype, int32_t group_size, const void* bias,
                                    void* y, int64_t y_stride_m, int64_t M, int64_t N, int64_t K,
                                    int32_t dtype, void* stream) {
  sd::clear_error();
  if (K > 0 && K <= (1ll << 30) && gate_up_stride_m < 2 * K) {  // other K: refused below
    sd::set_error("w8a16_silu: gate_up rows hold 2 K = %lld elements, stride %lld",
                  (long long)(2 * K), (long long)gate_up_stride_m);
    return SD_ERR_VALUE;
  }
  return run_w8a16(gate_up, gate_up_stride_m, K, NormArgs{}, w, w_stride_n, scale, scale_dtype,
                   group_size, bias, y, y_stride_m, M, N, K, dtype, stream);
}

extern "C" int sd_w8a16_rmsnorm_linear(const void* x, int64_t x_stride_m, const void* residual,
                                       int64_t residual_stride_m, void* residual_out,
                                       int64_t residual_out_stride_m, const void* norm_weight,
                                       float eps, const int8_t* w, int64_t w_stride_n,
                                       const void* scale, int32_t scale_dtype, int32_t group_size,
                                       const void* bias, void* y, int64_t y_stride_m, int64_t M,
                                       int64_t N, int64_t K, int32_t dtype, void* stream) {
  sd::clear_error();
  if (!norm_weight || K % 8 != 0 || K > 8192) {
    sd::set_error("w8a16_rmsnorm: needs the norm weight and K a multiple of 8 up to 8192 (K=%lld)",
                  (long long)K);
    return SD_ERR_UNSUPPORTED;
  }
  if ((residual && (!sd::aligned16(residual) || residual_stride_m % 8)) ||
      (residual_out && (!sd::aligned16(residual_out) || residual_out_stride_m % 8)) ||
      !sd::aligned16(norm_weight)) {
    sd::set_error("w8a16_rmsnorm: residual, residual_out and norm weight rows 16-byte aligned");
    return SD_ERR_UNSUPPORTED;
  }
  const NormArgs norm{norm_weight, residual, residual_stride_m, residual_out,
                      residual_out_stride_m, eps};
  return run_w8a16(x, x_stride_m, -1, norm, w, w_stride_n, scale, scale_dtype, group_size, bias, y,
                   y_stride_m, M, N, K, dtype, stream);
}

extern "C" int sd_w8a16_gate_up_silu(const void* x, int64_t x_stride_m, const void* residual,
                                     int64_t residual_stride_m, void* residual_out,
                                     int64_t residual_out_stride_m, const void* norm_weight,
                                     float eps, const int8_t* w, int64_t w_stride_n,
                                     const void* scale, int32_t scale_dtype, const void* bias,
                                     void* y, int64_t y_stride_m, int64_t M, int64_t N,
                                     int64_t K, int32_t dtype, void* stream) {
  sd::clear_error();
  if (norm_weight && (K % 8 != 0 || K > 8192)) {
    sd::set_error("w8a16_gate_up_silu: the norm needs K a multiple of 8 up to 8192 (K=%lld)",
                  (long long)K);
    return SD_ERR_UNSUPPORTED;
  }
  if ((residual || residual_out) && !norm_weight) {
    sd::set_error("w8a16_gate_up_silu: a residual needs the norm weight");
    return SD_ERR_VALUE;
  }
  if ((residual && (!sd::aligned16(residual) || residual_stride_m % 8)) ||
      (residual_out && (!sd::aligned16(residual_out) || residual_out_stride_m % 8)) ||
      (norm_weight && !sd::aligned16(norm_weight))) {
    sd::set_error("w8a16_gate_up_silu: residual, residual_out and norm weight rows 16-byte "
                  "aligned");
    return SD_ERR_UNSUPPORTED;
  }
  const NormArgs norm{norm_weight, residual, residual_stride_m, residual_out,
                      residual_out_stride_m, eps};
  return run_w8a16(x, x_stride_m, -1, norm, w, w_stride_n, scale, scale_dtype, 0, bias, y,
                   y_stride_m, M, N, K, dtype, stream, true);
}
