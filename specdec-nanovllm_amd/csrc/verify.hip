// verify.hip — speculative verification by rejection sampling for gfx950:
// `verify_batch` (nanovllm/spec_decode/verify.py:39-183, Leviathan et al.
// 2023). Per sequence b with k draft tokens x_j:
//   q_j = softmax(draft_j / T) (or the given probabilities for a point-mass
//   draft), p_j = softmax(target_j / T), j <= k;
//   candidate j is accepted when u_j < min(1, p_j[x_j] / q_j[x_j]) (0 when
//   q_j[x_j] == 0), accepted = index of the first rejection (k if none);
//   bonus ~ normalize(max(0, p_a - q_a)) with a = accepted and q_k = 0 (so
//   "all accepted" samples p_k), falling back to p_a when the residual sums
//   to 0, drawn as argmax(resid / E), E ~ Exp(1) (verify.py:171-183,203-209).
//
// Three launches, no host sync:
//   stats_kernel   (m, l) of x log2(e) / T (exp2 domain) over V slices, every
//                  row of every sequence (draft rows 0..k-1, target rows
//                  0..k), one workgroup per
//                  (row, slice of 8192 logits): HBM-bound, reads every logit
//                  once, and records the logit of the row's candidate token;
//   resid_kernel   per (sequence, slice of 2048 logits): merges the row
//                  statistics and runs the k acceptance tests on the recorded
//                  logits (every workgroup of the sequence; a separate launch
//                  cost more), then the residual race over its slice of the
//                  accepted position's rows;
//   finish_kernel  per sequence: merges the slices' races into the bonus.
// Noise: Philox4x32-10 keyed by rng_state[0]; u_j uses counter (j, b ^ off_hi,
// off_lo, 1), u_j = (c0 >> 8) 2^-24 in [0, 1); the bonus noise of element i
// is word i % 4 of the block with counter (i / 4, b ^ off_hi, off_lo, 2) (one
// Philox call per four elements), E = max(-log U, 1e-10), U = ((w >> 8) + 1)
// 2^-24 in (0, 1].
#include <math.h>

#include "sd_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxK = 32;  // draft tokens per sequence
constexpr int kUnroll = 8; // loads a thread has in flight in the scans
constexpr int kMaxParts = 2048;  // (row, slice) statistics one workgroup merges

struct VerifyParams {
  const void* draft;  // (B, k, V): logits, or probabilities when point_mass
  int64_t d_sb, d_sj;
  int32_t d_dtype;
  const void* target;  // (B, k + 1, V) logits
  int64_t t_sb, t_sj;
  int32_t t_dtype;
  const int64_t* tokens;  // (B, k)
  int64_t tok_sb;
  const float* temp;  // (B,), NULL: 1
  const int64_t* state;
  int32_t B, k, V;
  int32_t point_mass;
  int32_t vec4;     // every row starts 4-element aligned and V % 4 == 0
  int32_t nsplit;   // V slices of the row statistics
  int32_t nsplit2;  // V slices of the residual race
  float2* stats;  // [B][2k + 1][nsplit] (m, l) of x log2(e) / T, l = sum 2^(x' - m)
  float* part;    // [B][nsplit2][5] residual sum, key_r, idx_r, key_p, idx_p
  float* gath;    // [B][2k]: logit of candidate x_j in draft row j (slot j) and
                  // target row j (slot k + j), recorded by the statistics pass
  int64_t* accepted;
  int64_t* bonus;
  uint8_t* mask;  // (B, k)
};

// One row of logits of element type DT (SD_F32, SD_BF16 or SD_F16): element
// loads with no run-time type test, so a group of loads issues back to back.
template <int DT>
struct Row {
  const char* base;  // element 0 of the row
  static constexpr int kBytes = DT == SD_F32 ? 4 : 2;
  __device__ __forceinline__ float at(int64_t i) const {
    if constexpr (DT == SD_F32) return reinterpret_cast<const float*>(base)[i];
    const uint16_t h = reinterpret_cast<const uint16_t*>(base)[i];
    if constexpr (DT == SD_BF16) return sd::from_bits<__bf16>(h);
    return sd::from_bits<_Float16>(h);
  }
  // elements i .. i + 3 (i % 4 == 0, rows 4-element aligned): one load
  __device__ __forceinline__ void at4(int64_t i, float out[4]) const {
    if constexpr (DT == SD_F32) {
      const float4 v = *reinterpret_cast<const float4*>(base + i * 4);
      out[0] = v.x;
      out[1] = v.y;
      out[2] = v.z;
      out[3] = v.w;
    } else {
      const uint2 v = *reinterpret_cast<const uint2*>(base + i * 2);
      const uint32_t w[2] = {v.x, v.y};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint16_t h = static_cast<uint16_t>(w[e / 2] >> (16 * (e & 1)));
        out[e] = DT == SD_BF16 ? sd::from_bits<__bf16>(h) : sd::from_bits<_Float16>(h);
      }
    }
  }
};

template <int DT>
__device__ __forceinline__ Row<DT> draft_row(const VerifyParams& p, int b, int j) {
  return Row<DT>{static_cast<const char*>(p.draft) + (b * p.d_sb + j * p.d_sj) * Row<DT>::kBytes};
}
template <int DT>
__device__ __forceinline__ Row<DT> target_row(const VerifyParams& p, int b, int j) {
  return Row<DT>{static_cast<const char*>(p.target) + (b * p.t_sb + j * p.t_sj) * Row<DT>::kBytes};
}

__device__ __forceinline__ float temperature(const VerifyParams& p, int b) {
  const float t = p.temp ? p.temp[b] : 1.f;
  return t > 0.f ? t : 1.f;
}

__device__ __forceinline__ void merge_ml(float& m, float& l, float m2, float l2) {
  const float M = fmaxf(m, m2);
  if (M == -INFINITY) return;
  l = l * sd::fast_exp2(m - M) + l2 * sd::fast_exp2(m2 - M);
  m = M;
}

// Slice `split` of [0, V): ceil(V / nsplit) elements, rounded up to a multiple
// of 4 (so vec4 slices hold whole groups of four).
__device__ __forceinline__ void slice_of(int V, int nsplit, int split, int& v0, int& v1) {
  const int64_t per = ((static_cast<int64_t>(V) + nsplit - 1) / nsplit + 3) / 4 * 4;
  const int64_t a = per * split, e = per * (split + 1);
  v0 = static_cast<int>(a < V ? a : V);
  v1 = static_cast<int>(e < V ? e : V);
}

// (max, sum 2^) of row[v0, v1) * s2 (s2 = log2(e) / T) for this thread's
// elements, in the exp2 domain (a multiply and a native exp2 per logit): groups of
// loads issued together, their maximum, then independent exponentials.
// `want` (or -1): the element whose raw logit is stored to *got by the thread
// that loads it.
template <int DT>
__device__ __forceinline__ void row_stats(const Row<DT>& row, int v0, int v1, float s2, bool vec4,
                                          int64_t want, float* got, float& m, float& l) {
  if (vec4) {
    constexpr int kG = 8;  // 4-element loads a thread has in flight
    for (int i0 = v0 + 4 * threadIdx.x; i0 < v1; i0 += 4 * kG * kThreads) {
      float xs[kG][4];
#pragma unroll
      for (int u = 0; u < kG; ++u) {
        const int i = i0 + 4 * kThreads * u;
        if (i < v1) {
          row.at4(i, xs[u]);
          if (want >= i && want < i + 4) *got = xs[u][want - i];
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) xs[u][e] = -INFINITY;
        }
      }
      float gm = -INFINITY;
#pragma unroll
      for (int u = 0; u < kG; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          xs[u][e] = xs[u][e] * s2;
          gm = fmaxf(gm, xs[u][e]);
        }
      if (gm == -INFINITY) continue;
      float gl = 0.f;
#pragma unroll
      for (int u = 0; u < kG; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) gl += sd::fast_exp2(xs[u][e] - gm);
      merge_ml(m, l, gm, gl);
    }
  } else {
    for (int i0 = v0 + threadIdx.x; i0 < v1; i0 += kThreads * kUnroll) {
      float xs[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int i = i0 + u * kThreads;
        xs[u] = -INFINITY;
        if (i < v1) {
          const float x = row.at(i);
          if (i == want) *got = x;
          xs[u] = x * s2;
        }
      }
      float gm = xs[0];
#pragma unroll
      for (int u = 1; u < kUnroll; ++u) gm = fmaxf(gm, xs[u]);
      if (gm == -INFINITY) continue;
      float gl = 0.f;
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) gl += sd::fast_exp2(xs[u] - gm);
      merge_ml(m, l, gm, gl);
    }
  }
}

template <int DDT, int TDT>
__global__ __launch_bounds__(kThreads) void stats_kernel(VerifyParams p) {
  __shared__ float sm[kThreads / 64], sl[kThreads / 64];
  const int split = static_cast<int>(blockIdx.x % p.nsplit);
  const int b = static_cast<int>(blockIdx.x / p.nsplit);
  const int r = blockIdx.y;
  if (p.point_mass && r < p.k) return;  // probabilities already: no statistics
  const float s2 = 1.4426950408889634f / temperature(p, b);  // log2(e) / T
  int v0, v1;
  slice_of(p.V, p.nsplit, split, v0, v1);
  float m = -INFINITY, l = 0.f;
  // the candidate token of this row: x_r (draft row r) or x_{r-k} (target row
  // r - k < k); the bonus row k has none
  const int j = r < p.k ? r : r - p.k;
  const int64_t want = j < p.k ? p.tokens[b * p.tok_sb + j] : -1;
  float* got = p.gath + static_cast<int64_t>(b) * 2 * p.k + (r < p.k ? j : p.k + j);
  if (r < p.k)
    row_stats(draft_row<DDT>(p, b, r), v0, v1, s2, p.vec4, want, got, m, l);
  else
    row_stats(target_row<TDT>(p, b, r - p.k), v0, v1, s2, p.vec4, want, got, m, l);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) merge_ml(m, l, __shfl_xor(m, off), __shfl_xor(l, off));
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sm[wave] = m;
    sl[wave] = l;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kThreads / 64; ++w) merge_ml(m, l, sm[w], sl[w]);
    p.stats[(static_cast<int64_t>(b) * (2 * p.k + 1) + r) * p.nsplit + split] = make_float2(m, l);
  }
}

__device__ __forceinline__ void philox_words(const VerifyParams& p, uint32_t c0, int b,
                                             uint32_t stream, uint32_t out[4]) {
  const uint64_t seed = static_cast<uint64_t>(p.state[0]);
  const uint64_t off = static_cast<uint64_t>(p.state[1]);
  out[0] = c0;
  out[1] = static_cast<uint32_t>(b) ^ static_cast<uint32_t>(off >> 32);
  out[2] = static_cast<uint32_t>(off);
  out[3] = stream;
  sd::philox(out, static_cast<uint32_t>(seed), static_cast<uint32_t>(seed >> 32));
}

__device__ __forceinline__ bool better(float k, int i, float bk, int bi) {
  return k > bk || (k == bk && i < bi);
}

// The running race state of one thread / wave: residual sum and the two
// (key, index) leaders.
struct Race {
  float rsum = 0.f, kr = -INFINITY, kp = -INFINITY;
  int ir = 0x7fffffff, ip = 0x7fffffff;
  __device__ __forceinline__ void take(float okr, int oir, float okp, int oip) {
    if (better(okr, oir, kr, ir)) {
      kr = okr;
      ir = oir;
    }
    if (better(okp, oip, kp, ip)) {
      kp = okp;
      ip = oip;
    }
  }
  __device__ __forceinline__ void wave_reduce() {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      rsum += __shfl_xor(rsum, off);
      take(__shfl_xor(kr, off), __shfl_xor(ir, off), __shfl_xor(kp, off), __shfl_xor(ip, off));
    }
  }
};

// Acceptance of sequence b, run by every race workgroup of the sequence (a
// separate launch costs more than the repeat): merges the row statistics, runs
// the k tests on the logits the statistics pass recorded, and returns the
// accepted length and the (m, l) of target row a and draft row a; workgroup
// `writer` also stores accepted / mask.
template <int DDT>
__device__ int accept(const VerifyParams& p, int b, bool writer, float4& rec) {
  __shared__ float rm[2 * kMaxK + 1], rz[2 * kMaxK + 1];
  __shared__ float2 parts[kMaxParts];
  __shared__ int acc_s;
  const int rows = 2 * p.k + 1;
  const float s2 = 1.4426950408889634f / temperature(p, b);  // log2(e) / T
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // ---- row statistics: every (row, slice) partial loaded in one round, then
  //      one wave per row merges its slices
  const int nparts = rows * p.nsplit;
  const float2* st = p.stats + static_cast<int64_t>(b) * nparts;
  for (int t = threadIdx.x; t < nparts; t += kThreads) {
    const int r = t / p.nsplit;
    parts[t] = (p.point_mass && r < p.k) ? make_float2(-INFINITY, 0.f) : st[t];
  }
  __syncthreads();
  for (int r = wave; r < rows; r += kThreads / 64) {
    float m = -INFINITY, l = 0.f;
    for (int s = lane; s < p.nsplit; s += 64) {
      const float2 ps = parts[r * p.nsplit + s];
      merge_ml(m, l, ps.x, ps.y);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) merge_ml(m, l, __shfl_xor(m, off), __shfl_xor(l, off));
    if (lane == 0) {
      rm[r] = m;
      rz[r] = l;
    }
  }
  __syncthreads();
  // ---- acceptance: lane j of wave 0 tests candidate j; the first failing lane
  //      is the accepted length
  if (wave == 0) {
    bool ok = true;
    const int j = lane;
    if (j < p.k) {
      const int64_t x = p.tokens[b * p.tok_sb + j];
      float q = 0.f, pt = 0.f;
      if (x >= 0 && x < p.V) {
        const float* g = p.gath + static_cast<int64_t>(b) * 2 * p.k;
        // point-mass drafts skip the statistics pass: their value is read here
        const float dv = p.point_mass ? draft_row<DDT>(p, b, j).at(x) : g[j];
        q = p.point_mass ? dv : sd::fast_exp2(dv * s2 - rm[j]) / rz[j];
        pt = sd::fast_exp2(g[p.k + j] * s2 - rm[p.k + j]) / rz[p.k + j];
      }
      const float ratio = q > 0.f ? fminf(pt / fmaxf(q, 1e-10f), 1.f) : 0.f;
      uint32_t c[4];
      philox_words(p, static_cast<uint32_t>(j), b, 1u, c);
      const float u = static_cast<float>(c[0] >> 8) * (1.f / 16777216.f);  // [0, 1)
      ok = u < ratio;
      if (writer) p.mask[static_cast<int64_t>(b) * p.k + j] = ok ? 1 : 0;
    }
    const unsigned long long fails = __ballot(!ok);
    const int a = fails ? __ffsll(static_cast<long long>(fails)) - 1 : p.k;
    if (lane == 0) {
      acc_s = a;
      if (writer) p.accepted[b] = a;
    }
  }
  __syncthreads();
  const int a = acc_s;
  // (m, l) of target row a and of draft row a (unused when a == k)
  rec = make_float4(rm[p.k + a], rz[p.k + a], a < p.k ? rm[a] : 0.f, a < p.k ? rz[a] : 1.f);
  return a;
}


// Residual race over one slice of the accepted position's rows.
template <int DDT, int TDT>
__global__ __launch_bounds__(kThreads) void resid_kernel(VerifyParams p) {
  __shared__ float red[kThreads / 64][5];
  const int split = static_cast<int>(blockIdx.x % p.nsplit2);
  const int b = static_cast<int>(blockIdx.x / p.nsplit2);
  const float s2 = 1.4426950408889634f / temperature(p, b);  // log2(e) / T
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  float4 rc;
  const int a = accept<DDT>(p, b, split == 0, rc);
  // ---- residual race over this slice: max(0, p_a - q_a) / E and p_a / E
  const bool has_q = a < p.k;
  const Row<TDT> prow = target_row<TDT>(p, b, a);
  const Row<DDT> qrow = draft_row<DDT>(p, b, has_q ? a : 0);
  const float pm = rc.x, pz = rc.y;
  const float qm = rc.z, qz = rc.w;
  int v0, v1;
  slice_of(p.V, p.nsplit2, split, v0, v1);
  Race race;
  // element i's noise is word i % 4 of the Philox block (i / 4, b, offset, 2)
  auto step = [&](int i, float tv, float dv, uint32_t w) {
    const float pv = sd::fast_exp2(tv * s2 - pm) / pz;
    float qv = 0.f;
    if (has_q) qv = p.point_mass ? dv : sd::fast_exp2(dv * s2 - qm) / qz;
    const float r = fmaxf(pv - qv, 0.f);
    race.rsum += r;
    const float U = (static_cast<float>(w >> 8) + 1.f) * (1.f / 16777216.f);  // (0, 1]
    const float E = fmaxf(-__builtin_amdgcn_logf(U) * 0.6931471805599453f, 1e-10f);  // -ln U
    race.take(r / E, i, pv / E, i);
  };
  if (p.vec4) {
    // slices start at multiples of 4: a 4-element group is one Philox block
    for (int i0 = v0 + 4 * threadIdx.x; i0 < v1; i0 += 4 * kThreads) {
      float ts[4], ds[4] = {0.f, 0.f, 0.f, 0.f};
      prow.at4(i0, ts);
      if (has_q) qrow.at4(i0, ds);
      uint32_t c[4];
      philox_words(p, static_cast<uint32_t>(i0 >> 2), b, 2u, c);
#pragma unroll
      for (int e = 0; e < 4; ++e) step(i0 + e, ts[e], ds[e], c[e]);
    }
  } else {
    for (int i0 = v0 + threadIdx.x; i0 < v1; i0 += kThreads * kUnroll) {
      float ts[kUnroll], ds[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int i = min(i0 + u * kThreads, v1 - 1);
        ts[u] = prow.at(i);
        ds[u] = has_q ? qrow.at(i) : 0.f;
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int i = i0 + u * kThreads;
        if (i >= v1) break;
        uint32_t c[4];
        philox_words(p, static_cast<uint32_t>(i >> 2), b, 2u, c);
        step(i, ts[u], ds[u], c[i & 3]);
      }
    }
  }
  race.wave_reduce();
  if (lane == 0) {
    red[wave][0] = race.rsum;
    red[wave][1] = race.kr;
    red[wave][2] = __int_as_float(race.ir);
    red[wave][3] = race.kp;
    red[wave][4] = __int_as_float(race.ip);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kThreads / 64; ++w) {
      race.rsum += red[w][0];
      race.take(red[w][1], __float_as_int(red[w][2]), red[w][3], __float_as_int(red[w][4]));
    }
    float* out = p.part + (static_cast<int64_t>(b) * p.nsplit2 + split) * 5;
    out[0] = race.rsum;
    out[1] = race.kr;
    out[2] = __int_as_float(race.ir);
    out[3] = race.kp;
    out[4] = __int_as_float(race.ip);
  }
}

__global__ __launch_bounds__(64) void finish_kernel(VerifyParams p) {
  const int b = blockIdx.x;
  Race race;
  for (int s = threadIdx.x; s < p.nsplit2; s += 64) {
    const float* in = p.part + (static_cast<int64_t>(b) * p.nsplit2 + s) * 5;
    race.rsum += in[0];
    race.take(in[1], __float_as_int(in[2]), in[3], __float_as_int(in[4]));
  }
  race.wave_reduce();
  if (threadIdx.x == 0) {
    const int t = race.rsum > 0.f ? race.ir : race.ip;
    p.bonus[b] = t == 0x7fffffff ? 0 : t;
  }
}

// Slices of the row statistics: ~8192 logits per workgroup (one round of
// eight 4-element loads per thread; 32K-logit slices were slower), at most
// kMaxParts (row, slice) partials per sequence.
int nsplit_for(int32_t V, int32_t k) {
  const int cap = kMaxParts / (2 * k + 1);
  const int n = static_cast<int>((static_cast<int64_t>(V) + 8191) / 8192);
  return n < 1 ? 1 : (n > cap ? cap : n);
}

// Slices of the residual race: ~2048 logits per workgroup (8 per thread), so
// the per-element work (Philox, log, exp, divides) spreads over many waves.
int nsplit2_for(int32_t V) {
  const int n = static_cast<int>((static_cast<int64_t>(V) + 2047) / 2048);
  return n < 1 ? 1 : (n > 1024 ? 1024 : n);
}

size_t stats_bytes(int64_t B, int32_t k, int ns) {
  return (static_cast<size_t>(B) * (2 * k + 1) * ns * sizeof(float2) + 255) / 256 * 256;
}

size_t parts_bytes(int64_t B, int ns2) {
  return (static_cast<size_t>(B) * ns2 * 5 * sizeof(float) + 255) / 256 * 256;
}

template <int DDT, int TDT>
void launch_two(const VerifyParams& p, dim3 g1, dim3 g2, hipStream_t st) {
  hipLaunchKernelGGL((stats_kernel<DDT, TDT>), g1, dim3(kThreads), 0, st, p);
  hipLaunchKernelGGL((resid_kernel<DDT, TDT>), g2, dim3(kThreads), 0, st, p);
}

template <int DDT>
void launch_t(int32_t tdt, const VerifyParams& p, dim3 g1, dim3 g2, hipStream_t st) {
  if (tdt == SD_F32) launch_two<DDT, SD_F32>(p, g1, g2, st);
  else if (tdt == SD_BF16) launch_two<DDT, SD_BF16>(p, g1, g2, st);
  else launch_two<DDT, SD_F16>(p, g1, g2, st);
}

void launch_pair(int32_t ddt, int32_t tdt, const VerifyParams& p, dim3 g1, dim3 g2,
                 hipStream_t st) {
  if (ddt == SD_F32) launch_t<SD_F32>(tdt, p, g1, g2, st);
  else if (ddt == SD_BF16) launch_t<SD_BF16>(tdt, p, g1, g2, st);
  else launch_t<SD_F16>(tdt, p, g1, g2, st);
}

}  // namespace

extern "C" size_t sd_verify_batch_workspace_size(int64_t batch, int32_t k, int32_t vocab) {
  if (batch <= 0 || k <= 0 || vocab <= 0) return 0;
  if (k > kMaxK || batch > 0x7fffffff) return SIZE_MAX;  // refused by sd_verify_batch
  const int ns = nsplit_for(vocab, k);
  return stats_bytes(batch, k, ns) + parts_bytes(batch, nsplit2_for(vocab)) +
         (static_cast<size_t>(batch) * 2 * k * sizeof(float) + 255) / 256 * 256;
}

extern "C" int sd_verify_batch(const void* draft, int64_t draft_stride_b, int64_t draft_stride_k,
                               int32_t draft_dtype, const void* target, int64_t target_stride_b,
                               int64_t target_stride_k, int32_t target_dtype,
                               const int64_t* draft_tokens, int64_t tokens_stride_b,
                               const float* temperatures, int32_t draft_is_point_mass,
                               const int64_t* rng_state, int64_t batch, int32_t k, int32_t vocab,
                               int64_t* accepted, int64_t* bonus, uint8_t* accept_mask,
                               void* workspace, size_t workspace_bytes, void* stream) {
  sd::clear_error();
  auto ok_dtype = [](int32_t d) { return d == SD_BF16 || d == SD_F16 || d == SD_F32; };
  if (batch < 0 || batch > 0x7fffffff || k <= 0 || k > kMaxK || vocab <= 0 ||
      !ok_dtype(draft_dtype) || !ok_dtype(target_dtype)) {
    sd::set_error("verify_batch: need batch < 2^31, 1 <= k <= %d, vocab > 0, logits "
                  "bf16/fp16/fp32 (batch=%lld k=%d vocab=%d)", kMaxK, (long long)batch, k, vocab);
    return SD_ERR_UNSUPPORTED;
  }
  if (batch == 0) return SD_OK;
  if (!draft || !target || !draft_tokens || !rng_state || !accepted || !bonus || !accept_mask) {
    sd::set_error("verify_batch: null pointer argument");
    return SD_ERR_VALUE;
  }
  const int ns = nsplit_for(vocab, k);
  const size_t need = sd_verify_batch_workspace_size(batch, k, vocab);
  if (!workspace || workspace_bytes < need || !sd::aligned16(workspace)) {
    sd::set_error("verify_batch: workspace of %zu bytes (16-byte aligned) required, got %zu",
                  need, workspace ? workspace_bytes : (size_t)0);
    return SD_ERR_WORKSPACE;
  }
  const int ns2 = nsplit2_for(vocab);
  if (batch * ns2 > 0x7fffffff || batch * ns > 0x7fffffff) {
    sd::set_error("verify_batch: batch too large (%lld)", (long long)batch);
    return SD_ERR_UNSUPPORTED;
  }
  VerifyParams p;
  p.draft = draft;
  p.d_sb = draft_stride_b;
  p.d_sj = draft_stride_k;
  p.d_dtype = draft_dtype;
  p.target = target;
  p.t_sb = target_stride_b;
  p.t_sj = target_stride_k;
  p.t_dtype = target_dtype;
  p.tokens = draft_tokens;
  p.tok_sb = tokens_stride_b;
  p.temp = temperatures;
  p.state = rng_state;
  p.B = static_cast<int32_t>(batch);
  p.k = k;
  p.V = vocab;
  p.point_mass = draft_is_point_mass ? 1 : 0;
  p.nsplit = ns;
  p.nsplit2 = ns2;
  // 4-element groups: V % 4 == 0 and every row start aligned to 4 elements
  // (and the base to 4 elements' bytes)
  auto rows_aligned = [&](const void* base, int32_t dt, int64_t sb, int64_t sj) {
    const int64_t bytes = dt == SD_F32 ? 16 : 8;
    return reinterpret_cast<uintptr_t>(base) % bytes == 0 && sb % 4 == 0 && sj % 4 == 0;
  };
  p.vec4 = vocab % 4 == 0 && rows_aligned(draft, draft_dtype, draft_stride_b, draft_stride_k) &&
           rows_aligned(target, target_dtype, target_stride_b, target_stride_k);
  p.stats = static_cast<float2*>(workspace);
  p.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + stats_bytes(batch, k, ns));
  p.gath = reinterpret_cast<float*>(static_cast<char*>(workspace) + stats_bytes(batch, k, ns) +
                                    parts_bytes(batch, ns2));
  p.accepted = accepted;
  p.bonus = bonus;
  p.mask = accept_mask;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned nb = static_cast<unsigned>(batch * ns);
  launch_pair(draft_dtype, target_dtype, p, dim3(nb, 2 * k + 1),
              dim3(static_cast<unsigned>(batch * ns2)), st);
  int rc = sd::check_launch("verify_batch statistics / acceptance / residual");
  if (rc != SD_OK) return rc;
  hipLaunchKernelGGL(finish_kernel, dim3(static_cast<unsigned>(batch)), dim3(64), 0, st, p);
  return sd::check_launch("verify_batch finish");
}
