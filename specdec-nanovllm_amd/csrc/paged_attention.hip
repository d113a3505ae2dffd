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
// Work decomposition (stream-K over keys, in columns):
//   A "pair" is one (sequence b, kv head h); a "column" is 32 keys of one
//   sequence (all kv heads), so sequence b has ceil(L_b / 32) columns. All
//   columns are laid end to end (b major) and cut into R runs of
//   S = max(ceil(C / R), min_steps) columns. A workgroup has NW wave64s (NW
//   divides Hkv: 4, 2 or 1) and takes heads hg NW .. hg NW + NW - 1 of one run
//   (workgroup w: run w / (Hkv / NW), head group w % (Hkv / NW)): wave i owns
//   head hg NW + i, and all NW waves walk the same columns (two row tiles, or
//   at most 4 sequences: two waves per head take the two halves of 64-key
//   columns and merge in LDS at the flush, KS = 2), so the workgroup
//   reads NW adjacent 256-byte head rows (NW x 256 contiguous bytes) of every
//   key instead of one. Every workgroup streams the same number of bytes
//   whatever the length mix, with no host sync: each workgroup derives C and
//   its start from context_lens itself (a wave-wide scan of the B lengths).
//   The head groups of a run are dispatched together, so a stretch of a page
//   (key rows of all heads side by side) is fetched by neighbouring requests.
//   step  : each wave takes the column's 32 keys of its head. It loads the
//           next step's K and V rows (16-byte loads) while it computes the
//           current one (register double buffer), then per 32 keys
//             S^T = K . Q^T      4 x MFMA 16x16x32 per 16 keys per row tile
//             online softmax     exp2 domain, row max over lane groups
//             O^T += V^T . P^T   16 x MFMA per row tile (P split into hi + lo
//                                16-bit parts), V^T gathered from LDS
//           The S^T / O^T orientation puts one query row per lane (l % 16),
//           so the softmax state never moves between lanes.
//   flush : when a pair ends (or the run does) each wave writes its own head's
//           state straight from registers (no LDS, no barrier): normalised
//           rows if this run saw the whole pair, otherwise a partial to slot
//           (run + b) * Hkv + h of the workspace, which `paged_attn_combine`
//           merges per pair (that slot is unique: a later run can only meet a
//           later sequence).
// G * max_qlen query rows are padded to RT tiles of 16 rows (RT = 1: decode
// with G <= 16 or the 0.6B verify; RT = 2: Qwen3-4B verify with 7 x 4 rows).
//
// Fused store_kvcache (STORE): a sequence's last n_b keys are this launch's new
// rows. The main kernel walks only the cached keys [0, L_b - n_b), which every
// query row of the sequence sees, and always writes partials; the combine
// kernel merges them with the n_b new keys (read from key / value, fp32 dot
// products, bottom-right causal among the new rows) and copies the new rows
// to their slots. The hot loop of the store launch is the plain one.
#include <math.h>

#include <atomic>

#include "sd_common.h"

namespace {

using sd::f32x4;
using sd::u32x4;

constexpr int kD = 128;                // head_dim
constexpr int kCombThreads = 256;      // most threads of a combine workgroup (8 groups of 32)
constexpr int kStep = 32;              // keys of one wave's share of a column
constexpr int kKPitch = 136;  // 16-bit elements per LDS row of a K tile (272 B: b128 reads of
                              // 16 consecutive rows hit distinct banks)
constexpr int kVPitch = 144;  // same for a V tile (288 B: transpose reads of 4 x 4 rows hit
                              // distinct banks)

struct AttnParams {
  const uint16_t* q;
  int64_t q_stok, q_shead;
  const uint16_t* kc;
  const uint16_t* vc;
  int64_t c_sblk, c_spos, c_shead;
  uint32_t c_spos32;  // c_spos, which the host checks fits 32 bits with room for a page
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
  int32_t num_seqs;
  int32_t G;
  int32_t Hkv;
  float scale_log2;  // softmax scale * log2(e)
  uint16_t* out;
  int64_t o_stok, o_shead;
  float* ws_ml;       // [slots][rmax][2]  (m in log2 units, l)
  float* ws_acc;      // [slots][rmax][kD] unnormalised
  int32_t nwg;        // workgroups: runs * (Hkv / NW)
  int32_t runs;
  int32_t min_steps;  // lower bound of columns per run
  int32_t col_keys;   // keys per column: 32 KS (KS waves per kv head)
  int32_t comb_rows;    // query rows per combine workgroup (a power of two)
  int32_t comb_slices;  // groups of 32 threads per row, each merging a share of its partials
  int32_t rmax;       // G * max_qlen
  // Fused store_kvcache (knew == NULL: none). Query row t's key/value row is
  // knew/vnew row t; sequence b's rows are its last n_b keys.
  const uint16_t* knew;
  const uint16_t* vnew;
  int64_t kn_stok, kn_shead, vn_stok, vn_shead;
  const int32_t* slot;  // (total_q,) cache slot of each new row, -1 = not written
  int64_t num_slots;    // num_blocks * block_size
};

struct SeqInfo {
  int L;       // keys the main kernel walks (STORE: cached keys only)
  int causal;  // row qi sees keys <= causal + qi (and < L)
  int nq;      // query rows
  int64_t q0;
  int R;       // G * nq
};

__device__ __forceinline__ int seq_keys(const AttnParams& p, int b) {
  const int L = p.ctx ? p.ctx[b] : (p.cu_k[b + 1] - p.cu_k[b]);
  return min(max(L, 0), p.max_ctx);
}

__device__ __forceinline__ int seq_rows(const AttnParams& p, int b) {
  return p.cu_q ? min(max(p.cu_q[b + 1] - p.cu_q[b], 0), p.max_qlen) : 1;
}

// Keys the main kernel walks: all of them, or (STORE) the cached ones.
template <bool STORE>
__device__ __forceinline__ int walk_keys(const AttnParams& p, int b) {
  const int L = seq_keys(p, b);
  return STORE ? max(L - seq_rows(p, b), 0) : L;
}

// walk_keys for a wave-uniform b (scalar loads).
template <bool STORE>
__device__ __forceinline__ int walk_keys_uniform(const AttnParams& p, int b) {
  int L = p.ctx ? sd::load_scalar_i32(p.ctx + b)
                : sd::load_scalar_i32(p.cu_k + b + 1) - sd::load_scalar_i32(p.cu_k + b);
  L = min(max(L, 0), p.max_ctx);
  if constexpr (STORE) {
    const int nq = p.cu_q ? min(max(sd::load_scalar_i32(p.cu_q + b + 1) -
                                        sd::load_scalar_i32(p.cu_q + b), 0), p.max_qlen)
                          : 1;
    L = max(L - nq, 0);
  }
  return L;
}

__device__ __forceinline__ int steps_of(const AttnParams& p, int L) {
  return (L + p.col_keys - 1) / p.col_keys;
}

template <bool STORE>
__device__ __forceinline__ SeqInfo seq_info(const AttnParams& p, int b) {
  SeqInfo s;
  const int L = seq_keys(p, b);
  if (p.cu_q) {
    s.q0 = p.cu_q[b];
    s.nq = min(max(p.cu_q[b + 1] - p.cu_q[b], 0), p.max_qlen);
  } else {
    s.q0 = b;
    s.nq = 1;
  }
  s.L = STORE ? max(L - s.nq, 0) : L;
  s.causal = L - s.nq;
  s.R = p.G * s.nq;
  return s;
}

// Wave-wide sum of steps(b) (columns) over b in [0, upto) (every lane gets it).
template <bool STORE>
__device__ int cols_before(const AttnParams& p, int upto) {
  const int lane = threadIdx.x & 63;
  int sum = 0;
  for (int c = 0; c < upto; c += 64) {
    const int b = c + lane;
    sum += b < upto ? steps_of(p, walk_keys<STORE>(p, b)) : 0;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
  return sum;
}

// Wave-wide: the sequence holding column s (0 <= s < total) and the index of
// that sequence's first column.
template <bool STORE>
__device__ void locate(const AttnParams& p, int s, int& b_out, int& first_out) {
  const int lane = threadIdx.x & 63;
  int run = 0;
  for (int c = 0; c < p.num_seqs; c += 64) {
    const int b = c + lane;
    const int n = b < p.num_seqs ? steps_of(p, walk_keys<STORE>(p, b)) : 0;
    const int incl = sd::wave_inclusive_sum(n);
    const int excl = run + incl - n;
    const unsigned long long hit = __ballot(n > 0 && excl <= s && s < excl + n);
    if (hit) {
      const int src = __ffsll(static_cast<unsigned long long>(hit)) - 1;
      b_out = c + src;
      first_out = __builtin_amdgcn_readlane(excl, src);
      return;
    }
    run += __builtin_amdgcn_readlane(incl, 63);
  }
  b_out = p.num_seqs - 1;  // s >= total: callers never ask
  first_out = run;
}

// Up to 64 sequences in one pass (lane i holds sequence i): its keys, query
// rows and first query row are loaded once, and everything the prologues need
// comes from shuffles of these registers — one round of global loads instead
// of one per scan.
struct LaneSeq {
  int L;     // keys (clamped)
  int nq;    // query rows
  int q0;    // first query row
  int walk;  // keys the main kernel walks
  int n;     // columns
  int incl;  // columns of sequences [0, lane] (inclusive scan)
};

template <bool STORE>
__device__ __forceinline__ LaneSeq lane_seq(const AttnParams& p) {
  const int lane = threadIdx.x & 63;
  LaneSeq ls{};
  const bool in = lane < p.num_seqs;
  // Every load first, then the arithmetic: the arrays are picked with uniform
  // selects and the index clamped (lanes past num_seqs read the last
  // sequence's words, never used). Loads under the branches on ctx / cu_q made
  // the compiler wait for the key lengths before it issued the query offsets'
  // loads, two round trips.
  const int li = min(lane, p.num_seqs - 1);  // num_seqs >= 1 on every launch
  const int32_t* kp = p.ctx ? p.ctx : p.cu_k;
  const int32_t* qp = p.cu_q ? p.cu_q : kp;
  const int nx = p.ctx ? 0 : 1;  // cu_k: the next offset
  const int nqx = p.cu_q ? 1 : 0;
  const int k0 = kp[li], k1 = kp[li + nx];
  const int q0 = qp[li], q1 = qp[li + nqx];
  const int L = p.ctx ? k0 : k1 - k0;
  ls.L = in ? min(max(L, 0), p.max_ctx) : 0;
  ls.q0 = p.cu_q && in ? q0 : lane;
  ls.nq = p.cu_q ? (in ? min(max(q1 - q0, 0), p.max_qlen) : 1) : 1;
  ls.walk = STORE ? max(ls.L - ls.nq, 0) : ls.L;
  ls.n = in ? steps_of(p, ls.walk) : 0;
  ls.incl = sd::wave_inclusive_sum(ls.n);
  return ls;
}

// SeqInfo of sequence `src` (wave-uniform) from a lane_seq pass, read with
// v_readlane into scalar registers (control flow on them stays uniform).
__device__ __forceinline__ SeqInfo seq_info_of(const AttnParams& p, const LaneSeq& ls, int src) {
  SeqInfo si;
  si.L = __builtin_amdgcn_readlane(ls.walk, src);
  si.nq = __builtin_amdgcn_readlane(ls.nq, src);
  si.q0 = __builtin_amdgcn_readlane(ls.q0, src);
  si.causal = __builtin_amdgcn_readlane(ls.L, src) - si.nq;
  si.R = p.G * si.nq;
  return si;
}

// Start of workgroup run `run`: total columns, columns per run S, the run's
// first column s0, the sequence b holding it, b's first column and b's
// SeqInfo. False when the run has no columns.
template <bool STORE>
__device__ __forceinline__ bool run_start(const AttnParams& p, int run, int& total, int& S,
                                          int& s0, int& b, int& first, SeqInfo& si,
                                          LaneSeq& ls) {
  if (p.num_seqs <= 64) {
    const int lane = threadIdx.x & 63;
    ls = lane_seq<STORE>(p);
    total = __builtin_amdgcn_readlane(ls.incl, 63);
    S = max((total + p.runs - 1) / p.runs, p.min_steps);
    s0 = run * S;
    if (s0 >= total) return false;
    const int excl = ls.incl - ls.n;
    const unsigned long long hit = __ballot(ls.n > 0 && excl <= s0 && s0 < ls.incl);
    b = __ffsll(static_cast<unsigned long long>(hit)) - 1;
    first = __builtin_amdgcn_readlane(excl, b);
    si = seq_info_of(p, ls, b);
    (void)lane;
    return true;
  }
  total = __builtin_amdgcn_readfirstlane(cols_before<STORE>(p, p.num_seqs));
  S = max((total + p.runs - 1) / p.runs, p.min_steps);
  s0 = run * S;
  if (s0 >= total) return false;
  locate<STORE>(p, s0, b, first);
  b = __builtin_amdgcn_readfirstlane(b);
  si = seq_info<STORE>(p, b);
  return true;
}

// Fused store: the 16-byte pieces of the new K and V rows, copied to their
// slots bit for bit (slot -1 or outside the pool: skipped), as store_kvcache
// does. The main kernel reads only cached keys, so the combine kernel, which
// runs after it, does the copies: each thread loads its first piece on entry
// and writes it after its merge. The slot stays the raw 32-bit value until the
// write: widening it where it is loaded would wait for the load right there.
struct StorePiece {
  u32x4 data;
  int32_t slot;
  int64_t tok;
  int head;
  int piece;
  bool is_v;
};

// 32-bit index math: the host caps total_q * Hkv at 2^25 for this launch.
__device__ __forceinline__ void piece_of(const AttnParams& p, uint32_t it, StorePiece& sp) {
  const uint32_t per = static_cast<uint32_t>(p.total_q) * p.Hkv * (kD * 2 / 16);
  sp.is_v = it >= per;
  uint32_t r = sp.is_v ? it - per : it;
  sp.piece = static_cast<int>(r & 15);
  r >>= 4;
  const uint32_t t = r / static_cast<uint32_t>(p.Hkv);
  sp.head = static_cast<int>(r - t * p.Hkv);
  sp.tok = t;
}

__device__ __forceinline__ void load_piece(const AttnParams& p, StorePiece& sp) {
  const uint16_t* src = sp.is_v ? p.vnew + sp.tok * p.vn_stok + sp.head * p.vn_shead
                                : p.knew + sp.tok * p.kn_stok + sp.head * p.kn_shead;
  sp.slot = p.slot[sp.tok];
  sp.data = sd::load16(src + sp.piece * 8);
}

__device__ __forceinline__ void write_piece(const AttnParams& p, const StorePiece& sp) {
  const int64_t slot = sp.slot;
  if (slot < 0 || slot >= p.num_slots) return;
  const int64_t blk = slot / p.block_size, off = slot - blk * p.block_size;
  uint16_t* dst = const_cast<uint16_t*>(sp.is_v ? p.vc : p.kc) + blk * p.c_sblk +
                  off * p.c_spos + sp.head * p.c_shead;
  sd::store16(dst + sp.piece * 8, sp.data);
}

// Element offset of key position `tok` (0 <= tok < L) of one sequence.
// UNIFORM: `btrow` and `tok` are the same on every lane (scalar table load).
template <bool UNIFORM = false>
__device__ __forceinline__ int64_t kv_row(const AttnParams& p, const int32_t* btrow, int tok) {
  int pg, off;
  if (p.bs_shift >= 0) {
    pg = tok >> p.bs_shift;
    off = tok & (p.block_size - 1);
  } else {
    pg = tok / p.block_size;
    off = tok - pg * p.block_size;
  }
  int blk = UNIFORM ? sd::load_scalar_i32(btrow + pg) : btrow[pg];
  blk = min(max(blk, 0), p.num_blocks - 1);  // padding ids (-1) never reach here; clamp anyway
  return static_cast<int64_t>(blk) * p.c_sblk + static_cast<int64_t>(off) * p.c_spos;
}

typedef uint32_t uint2v __attribute__((ext_vector_type(2)));

template <typename T>
__device__ __forceinline__ void store4(uint16_t* dst, f32x4 v, float s) {
  uint2 w;
  w.x = sd::pack2<T>(v.x * s, v.y * s);
  w.y = sd::pack2<T>(v.z * s, v.w * s);
  *reinterpret_cast<uint2*>(dst) = w;
}

// Bytes of one K + V tile of 32 keys (padded pitches).
constexpr int kTileBytes = kStep * (kKPitch + kVPitch) * 2;

// LDS of the main kernel: one K and one V tile per wave (TS = 1), or two
// (double-buffered) shared tiles per pair of waves (TS = 2): NW tiles either way.
template <int NW>
constexpr int smem_bytes() { return NW * kTileBytes; }

// One wave's share of one workgroup step: 32 keys of K and of V, lane l
// holding key 4 r + l/16, dims 8 (l%16) .. +8 of k[r] / v[r] — 16 lanes read one
// whole 256-byte row, so every load instruction moves four full rows. Both
// tiles are then transposed through LDS into MFMA operand order. With TS = 2
// a wave loads one of the two tensors (d: K for its pair's first wave, V for
// the second), in the same lane layout.
template <int TS>
struct StepRegsT {
  u32x4 k[8];
  u32x4 v[8];
};
template <>
struct StepRegsT<2> {
  u32x4 d[8];
};

// ONE_PAGE: block_size % 32 == 0, so a wave's 32-key slice never crosses a
// page and one block-table lookup serves the whole slice.
// Waves per SIMD the main kernel is built for (VGPR budget 512 / this); the
// grid holds this many workgroups per compute unit.
template <int RT>
constexpr int main_occupancy() { return RT == 1 ? 2 : 1; }

// KS = 2: two waves per kv head take the two 32-key halves of a 64-key column
// and merge their states in LDS when a pair ends, so a run covers twice the
// keys and the pairs leave half the partials (verify's two row tiles, small
// batches).
// FLOOR: the measurement twin that issues exactly the loads of the kernel
// (same grid, runs, order and prefetch) with no math and no output — the
// access pattern's own time.
// TS = 2 (tile split, verify's 2 row tiles): two waves share each 32-key step
// of a kv head and take one 16-row tile each (RT = 1 per wave). The first
// loads the step's K rows, the second its V rows; both write them into their
// pair's double-buffered LDS tile, meet at a workgroup barrier, and compute
// their own tile from the shared K and V. A wave then holds half the
// accumulator and half the prefetch of a two-tile wave, so the kernel runs at
// two waves per SIMD without spilling.
template <typename T, int RT, bool ONE_PAGE, bool STORE, int NW, int KS = 1, bool FLOOR = false,
          int TS = 1>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(main_occupancy<RT>())))
void paged_attn_main(AttnParams p) {
  static_assert(TS == 1 || RT == 1, "a tile-split wave holds one row tile");
  using StepRegs = StepRegsT<TS>;
  __shared__ __attribute__((aligned(16))) char smem[smem_bytes<NW>()];

  const int tid = threadIdx.x;
  // wave index held in an SGPR: page lookups and page bases stay scalar
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int lr = lane & 15, lg = lane >> 4;

  // ---- this wave's kv head and the workgroup's run of columns [s0, s1)
  constexpr int HPW = NW / (KS * TS);  // kv heads per workgroup
  const int groups = p.Hkv / HPW;
  const int h = static_cast<int>(blockIdx.x) % groups * HPW + wave / (KS * TS);
  const int ks = wave / TS % KS;  // this wave's 32-key half of a column (KS = 2)
  const int ts = wave % TS;       // TS = 2: this wave's row tile and loaded tensor
  const int tile0 = TS == 2 ? ts : 0;
  const int run = static_cast<int>(blockIdx.x) / groups;
  int total, S, s0, b, first;
  SeqInfo si;
  // up to 64 sequences: every sequence's lengths stay in the lanes of `ls`, so a
  // pair switch reads the next sequence's info from registers, not memory
  LaneSeq ls{};
  if (!run_start<STORE>(p, run, total, S, s0, b, first, si, ls)) return;
  const bool lane_seqs = p.num_seqs <= 64;
  const int s1 = min(s0 + S, total);
  b = __builtin_amdgcn_readfirstlane(b);
  first = __builtin_amdgcn_readfirstlane(first);
  int n = steps_of(p, si.L);  // columns of sequence b
  int j = s0 - first;
  int j_first = j;  // column at which this workgroup entered the current pair

  // ---- per-pair state: Q operand, causal limits, online-softmax state
  u32x4 qop[RT][4];
  int lim[RT];  // last key visible to this lane's row (-1: padding row)
  float m_run[RT], l_run[RT];
  f32x4 acc[RT][8];

  auto begin_pair = [&]() {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int row = (tile0 + rt) * 16 + lr;
      const int qi = row / p.G, g = row - qi * p.G;
      const int64_t qt = si.q0 + qi;
      const bool valid = row < si.R && qt >= 0 && qt < p.total_q;
      lim[rt] = valid ? min(si.causal + qi, si.L - 1) : -1;
      const uint16_t* qp =
          p.q + (valid ? qt * p.q_stok + static_cast<int64_t>(h * p.G + g) * p.q_shead : 0) +
          lg * 8;
#pragma unroll
      for (int s = 0; s < 4; ++s)
        qop[rt][s] = valid ? sd::load16(qp + s * 32) : u32x4{0u, 0u, 0u, 0u};
      m_run[rt] = -INFINITY;
      l_run[rt] = 0.f;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) acc[rt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };

  // Always issues the same 16 loads: a load count that never depends on control
  // flow lets the compiler wait for this step's loads only, not for the
  // prefetch issued after them. Loads nobody uses (`real` false, or a wave
  // without keys in the step) all read one 16-byte location, so they cost one
  // cache line, not a re-read of streamed (nontemporal) rows.
  auto load_step = [&](StepRegs& R, int lb, int lh, int lj, int L, bool real) {
    const int last = L - 1;
    // wave-uniform by construction; readfirstlane lets the compiler prove it, so
    // the block-table lookup is a scalar load (lgkmcnt) and never waits on the
    // vector loads in flight
    const int t0 = __builtin_amdgcn_readfirstlane(min(lj * p.col_keys + ks * kStep, last));
    lb = __builtin_amdgcn_readfirstlane(lb);
    const int32_t* btrow = p.bt + static_cast<int64_t>(lb) * p.bt_stride;
    const int64_t hoff = static_cast<int64_t>(lh) * p.c_shead;
    const bool used = real && lj * p.col_keys + ks * kStep <= last;  // wave-uniform
    if constexpr (ONE_PAGE) {
      // scalar page base + 32-bit lane offsets (key rows of one page)
      const int64_t base = kv_row<true>(p, btrow, t0) + hoff;
      const char* kpg = reinterpret_cast<const char*>(p.kc + base);
      const char* vpg = reinterpret_cast<const char*>(p.vc + base);
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const int tok = min(t0 + r * 4 + lg, last);
        const uint32_t off =  // bytes
            used ? (static_cast<uint32_t>(tok - t0) * p.c_spos32 + lr * 8) * 2u : 0u;
        if constexpr (TS == 2) {
          R.d[r] = sd::load16_stream((ts == 0 ? kpg : vpg) + off);
        } else {
          R.k[r] = sd::load16_stream(kpg + off);
          R.v[r] = sd::load16_stream(vpg + off);
        }
      }
    } else {
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const int tok = min(t0 + r * 4 + lg, last);
        const int64_t off = used ? kv_row(p, btrow, tok) + hoff + lr * 8 : 0;
        if constexpr (TS == 2) {
          R.d[r] = sd::load16_stream((ts == 0 ? p.kc : p.vc) + off);
        } else {
          R.k[r] = sd::load16_stream(p.kc + off);
          R.v[r] = sd::load16_stream(p.vc + off);
        }
      }
    }
  };

  // TS = 1: this wave's own tile. TS = 2: its pair's two tiles (step parity).
  char* const tiles = smem + (TS == 2 ? (wave / 2) * 2 : wave) * kTileBytes;
  uint16_t* kl = reinterpret_cast<uint16_t*>(tiles);
  uint16_t* vl = kl + kStep * kKPitch;
  u32x4 fold = {0u, 0u, 0u, 0u};  // FLOOR: every loaded word is consumed here
  const sd::XorAddr xa = sd::xor_addr();  // lanes of the row-maximum exchanges

  auto compute_step = [&](StepRegs& R, int cj, int par) {
    const int tb = cj * p.col_keys + ks * kStep;
    if constexpr (FLOOR) {
      if (tb >= si.L) return;
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        if constexpr (TS == 2) fold ^= R.d[r];
        else fold ^= R.k[r] ^ R.v[r];
      }
      return;
    }
    if constexpr (TS == 2) {
      // ---- this wave's tensor of the step into the pair's tile `par`; both
      //      waves of every pair reach the barrier on every step
      kl = reinterpret_cast<uint16_t*>(tiles + par * kTileBytes);
      vl = kl + kStep * kKPitch;
      uint16_t* dst = ts == 0 ? kl : vl;
      const int pitch = ts == 0 ? kKPitch : kVPitch;
#pragma unroll
      for (int r = 0; r < 8; ++r) sd::store16(dst + (r * 4 + lg) * pitch + lr * 8, R.d[r]);
      __syncthreads();
      if (tb >= si.L) return;  // wave-uniform (KS = 2: the last half may be empty)
    } else {
      if (tb >= si.L) return;  // wave-uniform (KS = 2: the last half of a column may be empty)
      // ---- stage the 32 K and V rows of this step (row-major, padded pitch)
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        sd::store16(kl + (r * 4 + lg) * kKPitch + lr * 8, R.k[r]);
        sd::store16(vl + (r * 4 + lg) * kVPitch + lr * 8, R.v[r]);
      }
      sd::wave_lds_sync();  // rows written by other lanes of this wave are read below
    }
    // ---- S^T tiles: lane holds S[row lr][key tb + 16 tt + 4 lg + i]; the K
    //      A operand of MFMA s is key 16 tt + lr, dims 32 s + 8 lg .. +8
    f32x4 sc[RT][2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      u32x4 ka[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) ka[s] = sd::load16(kl + (tt * 16 + lr) * kKPitch + s * 32 + lg * 8);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) c = sd::Elem<T>::mfma(ka[s], qop[rt][s], c);
        sc[rt][tt] = c;
      }
    }

    // ---- online softmax; P^T operand: k-slot 8 lg + j <-> key 4 lg + j (j < 4)
    //      and key 16 + 4 lg + (j - 4) (j >= 4), the order S^T already holds.
    u32x4 pop[RT], plo[RT];
    // every row sees every key of this slice: no causal / length mask needed
    // (a wave-uniform branch, so full steps skip the mask's selects)
    const bool full = tb + kStep - 1 <= min(si.causal, si.L - 1);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[rt][tt][i] *= p.scale_log2;
    }
    if (!full) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int tok = tb + tt * 16 + lg * 4 + i;
            // lim < L: also masks keys past the end
            sc[rt][tt][i] = tok <= lim[rt] ? sc[rt][tt][i] : -INFINITY;
          }
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      float mloc = -INFINITY;
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) mloc = fmaxf(mloc, sc[rt][tt][i]);
      // lazy row maximum: exchanged across the row's lanes, and the running
      // sums rescaled, only when some score of the wave exceeds its row's
      // running maximum by more than 8 (log2 units). Otherwise the old maximum
      // stays the reference, so P <= 2^8: well inside the range of the fp32
      // sums and of the hi + lo split below, and acc / l does not depend on the
      // reference chosen (the partials carry it as their m).
      // The vote is wave-wide, so every lane of a row keeps the same maximum.
      if (__any(mloc > m_run[rt] + 8.f)) {
        mloc = sd::max_over_groups(mloc, xa);
        const float mnew = fmaxf(m_run[rt], mloc);
        const float alpha = sd::fast_exp2(m_run[rt] - ((mnew == -INFINITY) ? 0.f : mnew));
        l_run[rt] *= alpha;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) acc[rt][dt] *= alpha;
        m_run[rt] = mnew;
      }
      const float mb = (m_run[rt] == -INFINITY) ? 0.f : m_run[rt];
      float pv[8];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        pv[q] = sd::fast_exp2(sc[rt][0][q] - mb);
        pv[4 + q] = sd::fast_exp2(sc[rt][1][q] - mb);
      }
      float ps = 0.f;
#pragma unroll
      for (int q = 0; q < 8; ++q) ps += pv[q];
      l_run[rt] += ps;
      // P = hi + lo in two 16-bit operands: P.V keeps ~16 mantissa bits of P
      // instead of the 8 (bf16) a single rounding would leave.
      uint32_t hi[4], lo[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) sd::split_pack<T>(pv[2 * q], pv[2 * q + 1], hi[q], lo[q]);
      pop[rt] = u32x4{hi[0], hi[1], hi[2], hi[3]};
      plo[rt] = u32x4{lo[0], lo[1], lo[2], lo[3]};
    }

    // ---- O^T += V^T . P^T; A operand lane holds V[key of slot 8 lg + j][dim 16 dt + lr].
    //      Two transpose reads: lane lr of block lg addresses key 4 lg + lr / 4 (then
    //      16 + 4 lg + lr / 4), dims 16 dt + 4 (lr % 4) .. +4, and receives keys
    //      4 lg .. 4 lg + 3 (then 16 + 4 lg ..) of dim 16 dt + lr.
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const uint16_t* c = vl + (lg * 4 + (lr >> 2)) * kVPitch + dt * 16 + (lr & 3) * 4;
      const uint2 v0 = sd::lds_read_tr16(c);
      const uint2 v1 = sd::lds_read_tr16(c + 16 * kVPitch);
      const u32x4 vop = {v0.x, v0.y, v1.x, v1.y};
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        acc[rt][dt] = sd::Elem<T>::mfma(vop, pop[rt], acc[rt][dt]);
        acc[rt][dt] = sd::Elem<T>::mfma(vop, plo[rt], acc[rt][dt]);
      }
    }
    // every lane has read the tile before the next step overwrites it (TS = 2:
    // the next step writes the other tile, and the barrier orders the one after)
    if constexpr (TS == 1) sd::wave_lds_sync();
  };

  // Write this wave's state of the current pair from registers: normalised
  // rows if this run saw the whole pair, else a partial. Lane (lr, lg) holds
  // row 16 rt + lr, dims 16 dt + 4 lg .. +4 of tile rt.
  auto flush = [&](bool complete) {
    if constexpr (FLOOR) return;
    const int64_t wslot = (static_cast<int64_t>(run) + b) * p.Hkv + h;
    float lsum[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) lsum[rt] = sd::sum_over_groups(l_run[rt]);
    if constexpr (KS == 2) {
      // the second wave of a head hands (m, l, acc) to the first through its
      // own (idle) K/V tile: rows of kD + 4 floats (TS = 2: the second key
      // half's pair of tiles, one state block per row tile)
      constexpr int kPitch = kD + 4;
      static_assert(RT * 16 * kPitch * 4 <= kTileBytes, "state fits the tile");
      __syncthreads();  // every wave is done with its tiles
      float* const xchg = TS == 2
          ? reinterpret_cast<float*>(smem + ((wave / (KS * TS)) * KS * TS + TS) * kTileBytes) +
                ts * 16 * kPitch
          : nullptr;
      if (ks == 1) {
        float* xs = TS == 2 ? xchg : reinterpret_cast<float*>(kl);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          float* xr = xs + (rt * 16 + lr) * kPitch;
#pragma unroll
          for (int dt = 0; dt < 8; ++dt)
            sd::store16(xr + dt * 16 + lg * 4, __builtin_bit_cast(u32x4, acc[rt][dt]));
          if (lg == 0) *reinterpret_cast<float2*>(xr + kD) = make_float2(m_run[rt], lsum[rt]);
        }
      }
      __syncthreads();
      if (ks == 0) {
        const float* ys = TS == 2 ? xchg
                                  : reinterpret_cast<const float*>(kl + kStep * (kKPitch + kVPitch));
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          const float* yr = ys + (rt * 16 + lr) * kPitch;
          const float2 ml = *reinterpret_cast<const float2*>(yr + kD);
          const float M = fmaxf(m_run[rt], ml.x);
          const float a = m_run[rt] == -INFINITY ? 0.f : exp2f(m_run[rt] - M);
          const float c = ml.x == -INFINITY ? 0.f : exp2f(ml.x - M);
          lsum[rt] = lsum[rt] * a + ml.y * c;
#pragma unroll
          for (int dt = 0; dt < 8; ++dt)
            acc[rt][dt] = acc[rt][dt] * a +
                          c * __builtin_bit_cast(f32x4, sd::load16(yr + dt * 16 + lg * 4));
          m_run[rt] = M;
        }
      }
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      if (KS == 2 && ks != 0) break;
      const float l = lsum[rt];
      const int row = (tile0 + rt) * 16 + lr;
      const int qi = row / p.G, g = row - qi * p.G;
      const int64_t qt = si.q0 + qi;
      if (row >= si.R || qt < 0 || qt >= p.total_q) continue;
      if (complete) {
        uint16_t* op = p.out + qt * p.o_stok + static_cast<int64_t>(h * p.G + g) * p.o_shead + lg * 4;
        const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) store4<T>(op + dt * 16, acc[rt][dt], inv);
      } else {
        const int64_t e = wslot * p.rmax + row;
        float* ap = p.ws_acc + e * kD + lg * 4;
        // TS = 2 (verify): nontemporal partial stores (C3 main 19.7 -> 19.0 us); the
        // decode form measured 1 us slower with them
        if constexpr (TS == 2) {
#pragma unroll
          for (int dt = 0; dt < 8; ++dt)
            __builtin_nontemporal_store(__builtin_bit_cast(u32x4, acc[rt][dt]),
                                        reinterpret_cast<u32x4*>(ap + dt * 16));
          if (lg == 0)
            __builtin_nontemporal_store(uint2v{__float_as_uint(m_run[rt]), __float_as_uint(l)},
                                        reinterpret_cast<uint2v*>(p.ws_ml + 2 * e));
        } else {
#pragma unroll
          for (int dt = 0; dt < 8; ++dt) sd::store16(ap + dt * 16, __builtin_bit_cast(u32x4, acc[rt][dt]));
          if (lg == 0) *reinterpret_cast<float2*>(p.ws_ml + 2 * e) = make_float2(m_run[rt], l);
        }
      }
    }
    if constexpr (KS == 2) __syncthreads();  // the tile is read before the next step stages into it
  };

  // ---- walk [s0, s1): load step s + 1 while computing step s
  // the first K/V loads go out before the query rows (needed only at compute)
  StepRegs ra, rb;
  load_step(ra, b, h, j, si.L, true);
  begin_pair();
  int s = s0;
  auto advance = [&](StepRegs& cur, StepRegs& nxt) -> bool {
    // position of step s + 1
    int nb = b, nj = j + 1;
    int nL = si.L;
    const bool more = s + 1 < s1;
    if (more && nj == n) {
      nj = 0;
      do {
        ++nb;
        nL = lane_seqs ? __builtin_amdgcn_readlane(ls.walk, nb) : walk_keys_uniform<STORE>(p, nb);
      } while (nL == 0);  // sequences without keys own no columns; s + 1 < total ends the scan
    }
    // the last step issues a dummy prefetch so that every iteration issues the
    // same loads
    load_step(nxt, more ? nb : b, h, more ? nj : j, more ? nL : si.L, more);
    compute_step(cur, j, s & 1);
    const bool pair_end = j + 1 == n;
    // STORE: partials only; the combine adds the new rows' keys
    if (pair_end || !more) flush(!STORE && pair_end && j_first == 0);
    if (!more) return false;
    if (nb != b) {
      b = nb;
      si = lane_seqs ? seq_info_of(p, ls, b) : seq_info<STORE>(p, b);
      n = steps_of(p, si.L);
      j_first = 0;
      begin_pair();
    }
    j = nj;
    ++s;
    return true;
  };
  for (;;) {
    if (!advance(ra, rb)) break;
    if (!advance(rb, ra)) break;
  }
  if constexpr (FLOOR) {
    // data-dependent and practically never true: the loads cannot be dropped
    const uint32_t f = fold.x ^ fold.y ^ fold.z ^ fold.w;
    if (f == 0x9E3779B9u && lane == 0) p.ws_ml[0] = __uint_as_float(f);
  }
}

// Four consecutive 16-bit elements: their bits, and as fp32.
__device__ __forceinline__ uint2 load_bits4(const uint16_t* src) {
  return *reinterpret_cast<const uint2*>(src);
}

template <typename T>
__device__ __forceinline__ f32x4 to4f(uint2 w) {
  return f32x4{sd::from_bits<T>(static_cast<uint16_t>(w.x)), sd::from_bits<T>(static_cast<uint16_t>(w.x >> 16)),
               sd::from_bits<T>(static_cast<uint16_t>(w.y)), sd::from_bits<T>(static_cast<uint16_t>(w.y >> 16))};
}

template <typename T>
__device__ __forceinline__ f32x4 load4f(const uint16_t* src) {
  return to4f<T>(load_bits4(src));
}

// Wave-wide: the columns of sequences [0, b) and of all sequences, one pass.
template <bool STORE>
__device__ void cols_split(const AttnParams& p, int b, int& before, int& total) {
  const int lane = threadIdx.x & 63;
  int sb = 0, st = 0;
  for (int c = 0; c < p.num_seqs; c += 64) {
    const int s = c + lane;
    const int n = s < p.num_seqs ? steps_of(p, walk_keys<STORE>(p, s)) : 0;
    st += n;
    sb += s < b ? n : 0;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    st += __shfl_xor(st, off);
    sb += __shfl_xor(sb, off);
  }
  before = sb;
  total = st;
}

// Log-sum-exp merge of the partials of pair (b, h) = (blockIdx.z, blockIdx.y),
// rows blockIdx.x * rpw .. + rpw (rpw = comb_rows), zero rows for sequences
// without keys. The workgroup is rpw rows x nsl slices x 32 threads (4 dims per
// thread; one slice where the plan expects at most 16 partials per pair, else
// 8 / rpw): slice s of a row merges its own contiguous share of the row's
// partials, all loads of a batch in flight at once, then (nsl > 1) slice 0
// merges the slices' states (LDS) in slice order. The merge arithmetic runs
// for the partials that exist only (a batch's unrolled steps past the slice's
// count are skipped), in the exp2 domain with the native v_exp_f32: a slice that
// ran all 16 steps under predicates, with the library exp2f, spent about 1 us
// on them. Sequence
// b spans columns [f, f + n); the runs that met it are f / S .. (f + n - 1) / S
// and run r's wave of head h wrote its partial to slot
// (r + b) * Hkv + h. Without STORE a pair met by one run is already final.
// STORE: every run wrote a partial of the cached keys, and the sequence's n_b
// new keys (new row j at position L - n_b + j, seen by query rows qi >= j) are
// merged last: s_j = q . k_j from the 16-bit inputs in fp32, k_j / v_j from
// key / value — or from the cache row when the row's slot is not stored (-1
// or outside the pool), as an unfused store would leave it. The first NK new
// rows' loads go out with the partials' (the rest, rows NK.., one at a time at
// the end; NK = 1 for decode).
template <typename T, bool STORE, int NK = 8>
__device__ __forceinline__ void combine_rows(const AttnParams& p) {
  constexpr int kBatch = 16;   // partial loads in flight per thread
  constexpr int kGroups = kCombThreads / 32;
  __shared__ __attribute__((aligned(16))) float4 s_o[kGroups][32];
  __shared__ float2 s_ml[kGroups];
  const int h = blockIdx.y, b = blockIdx.z;
  // pair b's SeqInfo, its first column f and all columns: one round of loads
  SeqInfo si;
  int f, total;
  if (p.num_seqs <= 64) {
    const LaneSeq ls = lane_seq<STORE>(p);
    si = seq_info_of(p, ls, b);
    total = __builtin_amdgcn_readlane(ls.incl, 63);
    f = __builtin_amdgcn_readlane(ls.incl - ls.n, b);
  } else {
    si = seq_info<STORE>(p, b);
    cols_split<STORE>(p, b, f, total);
  }
  const int grp = threadIdx.x >> 5, d4 = (threadIdx.x & 31) * 4;
  const int rpw = p.comb_rows, nsl = p.comb_slices;
  const int sl = grp / rpw;
  const int row = blockIdx.x * rpw + grp % rpw;
  const int qi = row / p.G, g = row - qi * p.G;
  const int64_t qt = si.q0 + qi;
  const bool live = row < si.R && qt >= 0 && qt < p.total_q;
  const int n = steps_of(p, si.L);

  // STORE: this row's q and the first NK new rows' key / value / slot, loaded
  // now, before the partials. The loads are unconditional, with every index
  // clamped into range, and stay raw bits until they are used: under a per-row
  // branch the compiler waited for each one before the branch joined (one round
  // trip per new row).
  uint2 qb = {0u, 0u}, kb[NK], vb[NK];
  int32_t sn[NK];
  if constexpr (STORE) {
    const int64_t last_q = static_cast<int64_t>(p.total_q) - 1;
    const int64_t qtc = min(max(qt, static_cast<int64_t>(0)), last_q);
    qb = load_bits4(p.q + qtc * p.q_stok + static_cast<int64_t>(h * p.G + g) * p.q_shead + d4);
    const int jl = max(si.nq - 1, 0);
#pragma unroll
    for (int j = 0; j < NK; ++j) {
      const int64_t tr = min(max(si.q0 + min(j, jl), static_cast<int64_t>(0)), last_q);
      sn[j] = p.slot[tr];
      kb[j] = load_bits4(p.knew + tr * p.kn_stok + static_cast<int64_t>(h) * p.kn_shead + d4);
      vb[j] = load_bits4(p.vnew + tr * p.vn_stok + static_cast<int64_t>(h) * p.vn_shead + d4);
    }
  }

  float M = -INFINITY, l = 0.f;
  f32x4 o = {0.f, 0.f, 0.f, 0.f};
  // Sequence b spans columns [f, f + n): runs w0 .. w1 met it (uniform over the
  // workgroup). final_by_main: no keys, or (without STORE) one run, which wrote
  // the output itself.
  const int S = max((total + p.runs - 1) / p.runs, p.min_steps);
  const int w0 = n > 0 ? f / S : 0, w1 = n > 0 ? (f + n - 1) / S : 0;
  const bool final_by_main = !STORE && (n == 0 || w0 == w1);
  const bool parts = n > 0 && !final_by_main;
  const int cnt = w1 - w0 + 1;
  const int per = (cnt + nsl - 1) / nsl;
  const int u0 = sl * per, u1 = min(u0 + per, cnt);  // this slice's share; u1 >= 1
  const float2* ml = reinterpret_cast<const float2*>(p.ws_ml);
  // rows past the pair's (idle) read the last row of the slot
  const int64_t base = ((static_cast<int64_t>(w0) + b) * p.Hkv + h) * p.rmax + min(row, p.rmax - 1);
  const int64_t run_stride = static_cast<int64_t>(p.Hkv) * p.rmax;  // rows between runs
  // One batch of partials: its loads all in flight, then the merge of those
  // that exist. Entries past the slice's count load a partial of the pair again
  // (the last one; never merged): a load under a branch whose other side writes
  // a default into the same registers made the compiler wait for it, and for
  // every load issued before it, at the branch.
  float2 part[kBatch];
  f32x4 a[kBatch];
  auto load_batch = [&](int c0) {
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int cu = max(min(c0 + u, u1 - 1), 0);
      const int64_t e = base + static_cast<int64_t>(cu) * run_stride;
      part[u] = ml[e];
      a[u] = __builtin_bit_cast(f32x4, sd::load16_stream(p.ws_acc + e * kD + d4));
    }
    // all of the batch's loads before any use (left alone, the scheduler
    // interleaved them with the merge and waited after every pair)
    __builtin_amdgcn_sched_barrier(0);
  };
  auto merge_batch = [&](int c0) {
    float mc = M;
#pragma unroll
    for (int u = 0; u < kBatch; ++u) mc = fmaxf(mc, c0 + u < u1 ? part[u].x : -INFINITY);
    // No branch between the loads and their use (the compiler sinks loads past
    // one, a second round trip): entries past the count get weight 0, and with
    // no partial at all (mc = -inf, l = o = 0) the reference point 0 keeps
    // every weight 0 instead of NaN.
    const float mr = mc == -INFINITY ? 0.f : mc;
    const float r = sd::fast_exp2(M - mr);  // rescale what earlier batches summed
    l *= r;
    o *= r;
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const float w = c0 + u < u1 ? sd::fast_exp2(part[u].x - mr) : 0.f;
      l += w * part[u].y;
      o += w * a[u];
    }
    M = mc;
  };
  // STORE: unconditional (the indices are valid without keys too): after a branch
  // around them the compiler could not tell how many loads follow the new rows'
  // and made the dot products below wait for the partials as well.
  if (STORE || parts) load_batch(u0);

  // STORE: while the partials are in flight, the new keys' rows and their dot
  // products with q. The 32 lanes of a row hold 4 dims each and the products
  // reduce over them (every lane of the wave takes part: no row has returned
  // yet). A new row whose slot is not stored keeps the cache row, as an unfused
  // store would leave it: one branch, taken only then. The merges come after the
  // partials', in key order.
  const int L = si.causal + si.nq;  // the sequence's keys, from the scan (no reload)
  const int32_t* btrow = p.bt + static_cast<int64_t>(b) * p.bt_stride;
  auto merge_key = [&](float dot, const f32x4& vv) {
    const float sj = dot * p.scale_log2;
    const float mn = fmaxf(M, sj);
    const float r = sd::fast_exp2(M - mn), w = sd::fast_exp2(sj - mn);
    l = l * r + w;
    o = o * r + w * vv;
    M = mn;
  };
  // new row j is merged into this row when jlo <= j <= jhi (it exists, it is a
  // key position, and the row sees it); bad: its slot is not stored
  const int jhi = min(qi, si.nq - 1), jlo = si.nq - L;  // uniform over the row's lanes
  const uint32_t ns32 =
      static_cast<uint32_t>(p.num_slots < 0x80000000ll ? p.num_slots : 0x80000000ll);
  float dot[NK];
  if constexpr (STORE) {
    uint32_t bad = 0;
#pragma unroll
    for (int j = 0; j < NK; ++j)
      bad |= (static_cast<uint32_t>(sn[j]) >= ns32 && j >= jlo && j <= jhi) ? 1u << j : 0u;
#pragma unroll
    for (int j = 0; j < NK; ++j)
      dot[j] = j >= jlo && j <= jhi ? sd::dot2<T>(qb.y, kb[j].y, sd::dot2<T>(qb.x, kb[j].x, 0.f)) : 0.f;
    // Rows whose slot is not stored: the cache row's bits, and the product
    // recomputed inside the branch. Loads in the branch that wrote registers read
    // after it would make the compiler wait at the join for them, and so for
    // every partial load issued before them.
    if (bad) {
#pragma unroll
      for (int j = 0; j < NK; ++j) {
        if (bad & (1u << j)) {
          const int64_t crow = kv_row(p, btrow, L - si.nq + j) + static_cast<int64_t>(h) * p.c_shead;
          const uint2 kc = load_bits4(p.kc + crow + d4);
          vb[j] = load_bits4(p.vc + crow + d4);
          dot[j] = sd::dot2<T>(qb.y, kc.y, sd::dot2<T>(qb.x, kc.x, 0.f));
          asm volatile("" : "+v"(vb[j].x), "+v"(vb[j].y));  // vb[j] arrives here, not later
        }
      }
    }
#pragma unroll
    for (int j = 0; j < NK; ++j) dot[j] = sd::half_wave_sum(dot[j]);
  }

  if (parts) {
    merge_batch(u0);
    for (int c0 = u0 + kBatch; c0 < u1; c0 += kBatch) {
      load_batch(c0);
      merge_batch(c0);
    }
  }
  if (nsl > 1) {  // workgroup-uniform
    s_o[grp][threadIdx.x & 31] = make_float4(o.x, o.y, o.z, o.w);
    if ((threadIdx.x & 31) == 0) s_ml[grp] = make_float2(M, l);
    __syncthreads();
    if (sl == 0) {
      float mc = M;
      for (int s2 = 1; s2 < nsl; ++s2) mc = fmaxf(mc, s_ml[s2 * rpw + grp].x);
      if (mc != -INFINITY) {
        const float r = sd::fast_exp2(M - mc);
        l *= r;
        o *= r;
        for (int s2 = 1; s2 < nsl; ++s2) {
          const float2 pm = s_ml[s2 * rpw + grp];
          const float4 po = s_o[s2 * rpw + grp][threadIdx.x & 31];
          const float w = sd::fast_exp2(pm.x - mc);
          l += w * pm.y;
          o += w * f32x4{po.x, po.y, po.z, po.w};
        }
        M = mc;
      }
    }
  }
  if (!live || sl != 0) return;
  uint16_t* op = p.out + qt * p.o_stok + static_cast<int64_t>(h * p.G + g) * p.o_shead + d4;
  if (final_by_main) {
    if (n == 0) *reinterpret_cast<uint2*>(op) = make_uint2(0u, 0u);
    return;
  }
  if constexpr (STORE) {
#pragma unroll
    for (int j = 0; j < NK; ++j)
      if (j >= jlo && j <= jhi) merge_key(dot[j], to4f<T>(vb[j]));
    // rows past NK (more new rows per sequence than the launch loads up front;
    // only this row's lanes take part in the reductions from here on)
    for (int j = NK; j < si.nq; ++j) {
      const bool u = j >= jlo && j <= jhi;  // uniform over the row's lanes
      const int64_t tr = si.q0 + j;
      uint2 kj = load_bits4(p.knew + tr * p.kn_stok + static_cast<int64_t>(h) * p.kn_shead + d4);
      uint2 vj = load_bits4(p.vnew + tr * p.vn_stok + static_cast<int64_t>(h) * p.vn_shead + d4);
      if (u && static_cast<uint32_t>(p.slot[tr]) >= ns32) {  // not stored: the cache row stays
        const int64_t crow = kv_row(p, btrow, L - si.nq + j) + static_cast<int64_t>(h) * p.c_shead;
        kj = load_bits4(p.kc + crow + d4);
        vj = load_bits4(p.vc + crow + d4);
      }
      const float dj =
          sd::half_wave_sum(u ? sd::dot2<T>(qb.y, kj.y, sd::dot2<T>(qb.x, kj.x, 0.f)) : 0.f);
      if (u) merge_key(dj, to4f<T>(vj));
    }
  }
  store4<T>(op, o, l > 0.f ? 1.f / l : 0.f);
}

// STORE: the launch's share of the fused store (grid-stride over the pieces;
// the host launches nothing when total_q == 0, so items > 0). Every thread
// loads a piece on entry, threads past the pieces the last one again (one
// cache line), so no branch holds the load.
template <typename T, bool STORE, int NK = 8>
__global__ __launch_bounds__(kCombThreads) void paged_attn_combine(AttnParams p) {
  if constexpr (!STORE) {
    combine_rows<T, false>(p);
  } else {
    const uint32_t items = 2u * static_cast<uint32_t>(p.total_q) * p.Hkv * (kD * 2 / 16);
    const uint32_t nthreads = gridDim.x * gridDim.y * gridDim.z * blockDim.x;
    const uint32_t it0 =
        ((blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x) * blockDim.x + threadIdx.x;
    StorePiece sp;
    piece_of(p, min(it0, items - 1), sp);
    load_piece(p, sp);
    combine_rows<T, true, NK>(p);
    if (it0 < items) write_piece(p, sp);
    for (uint32_t it = it0 + nthreads; it < items; it += nthreads) {
      piece_of(p, it, sp);
      load_piece(p, sp);
      write_piece(p, sp);
    }
  }
}

// ------------------------------------------------------------------ host
struct Plan {
  int RT;         // 16-row tiles of query rows
  int TS;         // 2: the row tiles on two waves that share each step's K/V
  int KS;         // waves per kv head (two 32-key halves of a column when 2)
  int NW;         // waves per main workgroup
  int runs;
  int nwg;        // workgroups of the main grid: runs * Hkv / NW
  int min_steps;  // lower bound of columns per run
  int rmax;       // rows per (sequence, kv head) in the workspace
  int comb_rows;  // combine workgroup: rows x slices x 32 threads
  int comb_slices;
  int64_t slots;  // partial slots: (runs + num_seqs) * Hkv
};

// num_splits == 0: one wave per SIMD (4 per compute unit, one wave per kv
// head of a run, or per half column / row tile) shares all the columns, at
// least one column per run. Against two waves per SIMD (the occupancy the
// kernel is built for) the runs are twice as long and leave half the partials;
// store + attention measured (16 page sets, same process): C2 B = 32 57.1 ->
// 55.8 us, B = 8 28.3 -> 26.1, B = 4 20.9 -> 19.1, B = 2 17.0 -> 14.8, B = 1
// level; C3 verify 26.0 -> 25.3, B = 16 verify 40.7 -> 38.1.
// num_splits > 0: num_splits runs per sequence on average, the meaning of the
// reference's `splits` (KV splits per sequence).
Plan make_plan(int num_seqs, int max_qlen, int Hq, int Hkv, int num_splits) {
  Plan pl;
  const int G = Hq / Hkv;
  pl.rmax = G * max_qlen;
  pl.RT = pl.rmax <= 16 ? 1 : 2;
  // two row tiles: one per wave, two waves sharing each step's loads
  pl.TS = pl.RT == 2 ? 2 : 1;
  // two waves per kv head, half the runs and partials: two row tiles (verify),
  // and small batches, whose pairs each collect a partial from many runs
  pl.KS = (pl.RT == 2 || num_seqs <= 4) && Hkv % 2 == 0 ? 2 : 1;
  // Two key halves: one kv head per workgroup for a single sequence, two heads
  // otherwise. One sequence of 2048 keys fills 33 runs, and two heads per
  // workgroup then left half the CUs without work (C5 draft step B = 1 841 ->
  // 832 us with one head; C2 decode B = 2 13.45 -> 13.75 us the other way).
  pl.NW = pl.TS == 2 ? 2 * pl.KS
                     : (pl.KS == 2 ? (num_seqs == 1 ? 2 : 4)
                                   : (Hkv % 4 == 0 ? 4 : (Hkv % 2 == 0 ? 2 : 1)));
  int64_t runs;
  if (num_splits > 0) {
    runs = static_cast<int64_t>(num_splits) * num_seqs;
    pl.min_steps = 1;
  } else {
    runs = static_cast<int64_t>(sd::device_cus()) * 4 / (Hkv * pl.KS * pl.TS);
    // at least 64 keys per run with two tiles on one wave
    pl.min_steps = pl.RT == 1 || pl.KS == 2 || pl.TS == 2 ? 1 : 2;
  }
  const int groups = Hkv / (pl.NW / (pl.KS * pl.TS));
  const int64_t cap = (1 << 20) / groups > 1 ? (1 << 20) / groups : 1;  // grid of at most 2^20
  runs = runs < 1 ? 1 : (runs > cap ? cap : runs);
  pl.runs = static_cast<int>(runs);
  pl.nwg = static_cast<int>(runs * groups);
  pl.slots = (runs + num_seqs) * Hkv;
  // Combine workgroup: a power of two of rows covering G * max_qlen (at most 8),
  // each row's partials split over the rest of 8 groups of 32 threads. A pair
  // meets about runs / num_seqs + 1 runs; where one slice can merge that many in
  // one batch of 16 (1.5 x the mean, plus 2: decode from about 12 sequences)
  // the row keeps one slice and the workgroup shrinks, with no LDS merge (C2
  // B = 32 combine 4.4 -> 4.1 us; more slices than 8 groups allow measured
  // slower for one sequence and for verify).
  // At least two rows (64 threads, a whole wave; a second row past rmax idles):
  // the length scan runs on all 64 lanes of a wave, one sequence per lane.
  pl.comb_rows = 2;
  while (pl.comb_rows < 8 && pl.comb_rows < pl.rmax) pl.comb_rows *= 2;
  const int64_t ns = num_seqs;
  const int64_t est = (3 * runs + 2 * ns - 1) / (2 * ns) + 2;
  pl.comb_slices = est <= 16 ? 1 : 8 / pl.comb_rows;
  return pl;
}

size_t ml_bytes(const Plan& pl) {
  return (static_cast<size_t>(pl.slots) * pl.rmax * 2 * sizeof(float) + 255) / 256 * 256;
}

size_t ws_bytes(const Plan& pl) {
  return ml_bytes(pl) + static_cast<size_t>(pl.slots) * pl.rmax * kD * sizeof(float);
}

template <typename T, int RT, bool STORE, int NW, int KS = 1, bool FLOOR = false, int TS = 1>
void launch_main(const AttnParams& p, hipStream_t st) {
  if (p.block_size % kStep == 0)
    hipLaunchKernelGGL((paged_attn_main<T, RT, true, STORE, NW, KS, FLOOR, TS>), dim3(p.nwg),
                       dim3(NW * 64), 0, st, p);
  else
    hipLaunchKernelGGL((paged_attn_main<T, RT, false, STORE, NW, KS, FLOOR, TS>), dim3(p.nwg),
                       dim3(NW * 64), 0, st, p);
}

template <typename T, int RT, bool STORE, bool FLOOR = false>
void launch_main(const AttnParams& p, const Plan& pl, hipStream_t st) {
  if constexpr (RT == 2) {  // two row tiles, one per wave (RT = 1 per wave, TS = 2)
    if (pl.KS == 2) launch_main<T, 1, STORE, 4, 2, FLOOR, 2>(p, st);
    else launch_main<T, 1, STORE, 2, 1, FLOOR, 2>(p, st);
  } else {
    if (pl.KS == 2 && pl.NW == 2) launch_main<T, RT, STORE, 2, 2, FLOOR>(p, st);
    else if (pl.KS == 2) launch_main<T, RT, STORE, 4, 2, FLOOR>(p, st);
    else if (pl.NW == 4) launch_main<T, RT, STORE, 4, 1, FLOOR>(p, st);
    else if (pl.NW == 2) launch_main<T, RT, STORE, 2, 1, FLOOR>(p, st);
    else launch_main<T, RT, STORE, 1, 1, FLOOR>(p, st);
  }
}

template <typename T, int RT>
void launch_main(const AttnParams& p, const Plan& pl, hipStream_t st) {
  if (p.knew) launch_main<T, RT, true>(p, pl, st);
  else launch_main<T, RT, false>(p, pl, st);
}

// What a call launches: both kernels, or one of them (measurement twins).
enum RunMode { kRunFull, kRunMain, kRunCombine, kRunFloor };

template <typename T>
int launch_all(const AttnParams& p, const Plan& pl, RunMode mode, hipStream_t st) {
  if (mode == kRunFloor) {  // the loads do not depend on the element type
    if (pl.RT == 1) launch_main<__bf16, 1, false, true>(p, pl, st);
    else launch_main<__bf16, 2, false, true>(p, pl, st);
    return sd::check_launch("paged_attention floor");
  }
  if (mode != kRunCombine) {
    if (pl.RT == 1) launch_main<T, 1>(p, pl, st);
    else launch_main<T, 2>(p, pl, st);
    const int rc = sd::check_launch("paged_attention main");
    if (rc != SD_OK || mode == kRunMain) return rc;
  }
  const dim3 grid((pl.rmax + p.comb_rows - 1) / p.comb_rows, p.Hkv, p.num_seqs);
  const dim3 block(static_cast<unsigned>(p.comb_rows * p.comb_slices * 32));
  if (p.knew && p.max_qlen == 1)  // decode: one new row per sequence
    hipLaunchKernelGGL((paged_attn_combine<T, true, 1>), grid, block, 0, st, p);
  else if (p.knew)
    hipLaunchKernelGGL((paged_attn_combine<T, true>), grid, block, 0, st, p);
  else
    hipLaunchKernelGGL((paged_attn_combine<T, false>), grid, block, 0, st, p);
  return sd::check_launch("paged_attention combine");
}

struct NewRows {  // fused store_kvcache arguments (key == NULL: none)
  const void* key;
  int64_t key_stride_tok, key_stride_head;
  const void* value;
  int64_t value_stride_tok, value_stride_head;
  const int32_t* slot_mapping;
};

// Scratch of sd_paged_attention_noalloc: the split-KV workspace in a static
// device array (each device holds its own copy from the library's load until
// the process ends). Host code never passes `scratch` itself to a kernel: the
// host-side name is a stand-in, not a device address. The per-device address
// comes from hipGetSymbolAddress (scratch_address below).
constexpr size_t kScratchBytes = SD_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) char scratch[kScratchBytes];

constexpr int kMaxScratchDevices = 64;
std::atomic<void*> g_scratch_addr[kMaxScratchDevices];

// Device address of `scratch` on the current device, looked up once per
// device (a racing second lookup stores the same address). A device reset
// reloads the code object and leaves the kept address stale: the entry is
// not for use after hipDeviceReset.
int scratch_address(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices) {
    sd::set_error("paged_attention_noalloc: no current device below %d", kMaxScratchDevices);
    return SD_ERR_HIP;
  }
  void* ptr = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (!ptr) {
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      sd::set_error("paged_attention_noalloc: hipGetSymbolAddress(scratch) failed: %s",
                    hipGetErrorString(e));
      return SD_ERR_HIP;
    }
    g_scratch_addr[dev].store(ptr, std::memory_order_release);
  }
  *out = ptr;
  return SD_OK;
}

// static_scratch: the workspace is this device's `scratch` (sd_paged_attention_noalloc)
int run_attention(RunMode mode, const NewRows& nr, const void* q, int64_t q_stride_tok,
                  int64_t q_stride_head,
                  const void* k_cache, const void* v_cache, int64_t cache_stride_block,
                  int64_t cache_stride_pos, int64_t cache_stride_head, int64_t num_blocks,
                  int32_t block_size, const int32_t* block_table, int64_t bt_stride,
                  int32_t max_blocks_per_seq, const int32_t* context_lens,
                  const int32_t* cu_seqlens_k, const int32_t* cu_seqlens_q, int32_t max_qlen,
                  int64_t total_q, int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads,
                  int32_t head_dim, float scale, int32_t dtype, void* out,
                  int64_t out_stride_tok, int64_t out_stride_head, void* workspace,
                  size_t workspace_bytes, int32_t num_splits, void* stream,
                  bool static_scratch = false) {
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
  if (!sd::strides_ok({q_stride_tok, q_stride_head, cache_stride_block, cache_stride_pos,
                       cache_stride_head, bt_stride, out_stride_tok, out_stride_head})) {
    sd::set_error("paged_attention: strides must lie in [-2^40, 2^40] elements");
    return SD_ERR_VALUE;
  }
  if (cache_stride_block < 0 || cache_stride_pos < 0 || cache_stride_head < 0 ||
      cache_stride_pos > (1ll << 25)) {
    sd::set_error("paged_attention: cache strides must be non-negative and the key-row stride "
                  "at most 2^25 elements");
    return SD_ERR_UNSUPPORTED;
  }
  if (static_cast<int64_t>(num_seqs) * num_kv_heads * ((max_ctx + kStep - 1) / kStep) >
      (1ll << 30)) {
    sd::set_error("paged_attention: %d sequences x %d kv heads x %lld keys is too much work "
                  "for one call", num_seqs, num_kv_heads, (long long)max_ctx);
    return SD_ERR_UNSUPPORTED;
  }
  const Plan pl = make_plan(num_seqs, max_qlen, num_q_heads, num_kv_heads, num_splits);
  const size_t need = ws_bytes(pl);
  if (static_scratch) {
    if (need > kScratchBytes) {
      sd::set_error("paged_attention_noalloc: these sizes need %zu bytes of scratch, more than "
                    "the %zu of the static scratch (call sd_paged_attention with a workspace)",
                    need, kScratchBytes);
      return SD_ERR_UNSUPPORTED;
    }
    const int rc = scratch_address(&workspace);
    if (rc != SD_OK) return rc;
    workspace_bytes = kScratchBytes;
  }
  if (!workspace || workspace_bytes < need || !sd::aligned16(workspace) ||
      reinterpret_cast<uintptr_t>(workspace) > UINTPTR_MAX - workspace_bytes) {
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
  p.c_spos32 = static_cast<uint32_t>(cache_stride_pos);
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
  p.ws_ml = static_cast<float*>(workspace);
  p.ws_acc = reinterpret_cast<float*>(static_cast<char*>(workspace) + ml_bytes(pl));
  p.num_seqs = num_seqs;
  p.nwg = pl.nwg;
  p.runs = pl.runs;
  p.min_steps = pl.min_steps;
  p.col_keys = kStep * pl.KS;
  p.comb_rows = pl.comb_rows;
  p.comb_slices = pl.comb_slices;
  p.knew = static_cast<const uint16_t*>(nr.key);
  p.vnew = static_cast<const uint16_t*>(nr.value);
  p.kn_stok = nr.key_stride_tok;
  p.kn_shead = nr.key_stride_head;
  p.vn_stok = nr.value_stride_tok;
  p.vn_shead = nr.value_stride_head;
  p.slot = nr.slot_mapping;
  p.num_slots = num_blocks * block_size;
  p.rmax = pl.rmax;

  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == SD_BF16) return launch_all<__bf16>(p, pl, mode, st);
  return launch_all<_Float16>(p, pl, mode, st);
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
  const Plan pl = make_plan(num_seqs, max_qlen, num_q_heads, num_kv_heads, num_splits);
  return ws_bytes(pl);
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
  return run_attention(kRunFull, NewRows{}, q, q_stride_tok, q_stride_head, k_cache, v_cache,
                       cache_stride_block, cache_stride_pos, cache_stride_head, num_blocks,
                       block_size, block_table, bt_stride, max_blocks_per_seq, context_lens,
                       cu_seqlens_k, cu_seqlens_q, max_qlen, total_q, num_seqs, num_q_heads,
                       num_kv_heads, head_dim, scale, dtype, out, out_stride_tok,
                       out_stride_head, workspace, workspace_bytes, num_splits, stream);
}

extern "C" int sd_paged_attention_noalloc(
    const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* k_cache,
    const void* v_cache, int64_t cache_stride_block, int64_t cache_stride_pos,
    int64_t cache_stride_head, int64_t num_blocks, int32_t block_size,
    const int32_t* block_table, int64_t bt_stride, int32_t max_blocks_per_seq,
    const int32_t* context_lens, const int32_t* cu_seqlens_k, const int32_t* cu_seqlens_q,
    int32_t max_qlen, int64_t total_q, int32_t num_seqs, int32_t num_q_heads,
    int32_t num_kv_heads, int32_t head_dim, float scale, int32_t dtype, void* out,
    int64_t out_stride_tok, int64_t out_stride_head, int32_t num_splits, void* stream) {
  return run_attention(kRunFull, NewRows{}, q, q_stride_tok, q_stride_head, k_cache, v_cache,
                       cache_stride_block, cache_stride_pos, cache_stride_head, num_blocks,
                       block_size, block_table, bt_stride, max_blocks_per_seq, context_lens,
                       cu_seqlens_k, cu_seqlens_q, max_qlen, total_q, num_seqs, num_q_heads,
                       num_kv_heads, head_dim, scale, dtype, out, out_stride_tok,
                       out_stride_head, nullptr, 0, num_splits, stream, true);
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
  return run_attention(kRunMain, NewRows{}, q, q_stride_tok, q_stride_head, k_cache, v_cache,
                       cache_stride_block, cache_stride_pos, cache_stride_head, num_blocks,
                       block_size, block_table, bt_stride, max_blocks_per_seq, context_lens,
                       cu_seqlens_k, cu_seqlens_q, max_qlen, total_q, num_seqs, num_q_heads,
                       num_kv_heads, head_dim, scale, dtype, out, out_stride_tok,
                       out_stride_head, workspace, workspace_bytes, num_splits, stream);
}

extern "C" int sd_paged_attention_combine(
    const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* k_cache,
    const void* v_cache, int64_t cache_stride_block, int64_t cache_stride_pos,
    int64_t cache_stride_head, int64_t num_blocks, int32_t block_size,
    const int32_t* block_table, int64_t bt_stride, int32_t max_blocks_per_seq,
    const int32_t* context_lens, const int32_t* cu_seqlens_k, const int32_t* cu_seqlens_q,
    int32_t max_qlen, int64_t total_q, int32_t num_seqs, int32_t num_q_heads,
    int32_t num_kv_heads, int32_t head_dim, float scale, int32_t dtype, void* out,
    int64_t out_stride_tok, int64_t out_stride_head, void* workspace, size_t workspace_bytes,
    int32_t num_splits, void* stream) {
  return run_attention(kRunCombine, NewRows{}, q, q_stride_tok, q_stride_head, k_cache, v_cache,
                       cache_stride_block, cache_stride_pos, cache_stride_head, num_blocks,
                       block_size, block_table, bt_stride, max_blocks_per_seq, context_lens,
                       cu_seqlens_k, cu_seqlens_q, max_qlen, total_q, num_seqs, num_q_heads,
                       num_kv_heads, head_dim, scale, dtype, out, out_stride_tok,
                       out_stride_head, workspace, workspace_bytes, num_splits, stream);
}

extern "C" int sd_paged_attention_floor(
    const void* q, int64_t q_stride_tok, int64_t q_stride_head, const void* k_cache,
    const void* v_cache, int64_t cache_stride_block, int64_t cache_stride_pos,
    int64_t cache_stride_head, int64_t num_blocks, int32_t block_size,
    const int32_t* block_table, int64_t bt_stride, int32_t max_blocks_per_seq,
    const int32_t* context_lens, const int32_t* cu_seqlens_k, const int32_t* cu_seqlens_q,
    int32_t max_qlen, int64_t total_q, int32_t num_seqs, int32_t num_q_heads,
    int32_t num_kv_heads, int32_t head_dim, float scale, int32_t dtype, void* out,
    int64_t out_stride_tok, int64_t out_stride_head, void* workspace, size_t workspace_bytes,
    int32_t num_splits, void* stream) {
  return run_attention(kRunFloor, NewRows{}, q, q_stride_tok, q_stride_head, k_cache, v_cache,
                       cache_stride_block, cache_stride_pos, cache_stride_head, num_blocks,
                       block_size, block_table, bt_stride, max_blocks_per_seq, context_lens,
                       cu_seqlens_k, cu_seqlens_q, max_qlen, total_q, num_seqs, num_q_heads,
                       num_kv_heads, head_dim, scale, dtype, out, out_stride_tok,
                       out_stride_head, workspace, workspace_bytes, num_splits, stream);
}

extern "C" int sd_paged_attention_store(
    const void* key, int64_t key_stride_tok, int64_t key_stride_head, const void* value,
    int64_t value_stride_tok, int64_t value_stride_head, const int32_t* slot_mapping,
    const void* q, int64_t q_stride_tok, int64_t q_stride_head, void* k_cache, void* v_cache,
    int64_t cache_stride_block, int64_t cache_stride_pos, int64_t cache_stride_head,
    int64_t num_blocks, int32_t block_size, const int32_t* block_table, int64_t bt_stride,
    int32_t max_blocks_per_seq, const int32_t* context_lens, const int32_t* cu_seqlens_k,
    const int32_t* cu_seqlens_q, int32_t max_qlen, int64_t total_q, int32_t num_seqs,
    int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, float scale, int32_t dtype,
    void* out, int64_t out_stride_tok, int64_t out_stride_head, void* workspace,
    size_t workspace_bytes, int32_t num_splits, void* stream) {
  sd::clear_error();
  if (total_q > 0 && (!key || !value || !slot_mapping)) {
    sd::set_error("paged_attention_store: key, value and slot_mapping are required");
    return SD_ERR_VALUE;
  }
  if (total_q > 0 &&
      (!sd::aligned16(key) || !sd::aligned16(value) || key_stride_tok % 8 != 0 ||
       key_stride_head % 8 != 0 || value_stride_tok % 8 != 0 || value_stride_head % 8 != 0)) {
    sd::set_error("paged_attention_store: key/value rows must be 16-byte aligned");
    return SD_ERR_UNSUPPORTED;
  }
  if (total_q > 0 && num_kv_heads > 0 && total_q > (int64_t{1} << 25) / num_kv_heads) {
    sd::set_error("paged_attention_store: total_q * num_kv_heads above 2^25");
    return SD_ERR_UNSUPPORTED;
  }
  if (num_seqs == 0 && total_q > 0) {  // rows to store but no attention: a plain store
    if (dtype != SD_BF16 && dtype != SD_F16) {
      sd::set_error("paged_attention_store: dtype must be bf16 or fp16");
      return SD_ERR_VALUE;
    }
    return sd_store_kvcache(key, key_stride_tok, key_stride_head, value, value_stride_tok,
                            value_stride_head, k_cache, v_cache, cache_stride_block,
                            cache_stride_pos, cache_stride_head, slot_mapping, total_q,
                            num_kv_heads, head_dim, block_size, num_blocks, 2, stream);
  }
  const NewRows nr{key, key_stride_tok, key_stride_head, value, value_stride_tok,
                   value_stride_head, slot_mapping};
  return run_attention(kRunFull, nr, q, q_stride_tok, q_stride_head, k_cache, v_cache,
                       cache_stride_block, cache_stride_pos, cache_stride_head, num_blocks,
                       block_size, block_table, bt_stride, max_blocks_per_seq, context_lens,
                       cu_seqlens_k, cu_seqlens_q, max_qlen, total_q, num_seqs, num_q_heads,
                       num_kv_heads, head_dim, scale, dtype, out, out_stride_tok,
                       out_stride_head, workspace, workspace_bytes, num_splits, stream);
}
