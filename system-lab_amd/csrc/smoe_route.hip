// smoe_route.hip — router top-k and the stable expert sort (gfx950).
//
// Router (C1): 16 lanes per token (64 for E > 256).  Softmax over fp32
// logits with the library's exp; the denominator is the fixed reduction tree
// of a 64-lane wave (lane j sums experts j, j+64, ... in order, then an xor
// butterfly 32..1), so the probabilities are bit-reproducible whatever the
// lane mapping.  Top-K by (score desc, id asc).
//
// Sort (C2): three small launches over the R = T*K (token, slot) pairs,
// each wave owning one segment of kSeg consecutive pairs:
//   1. route_hist  — per-segment expert histogram hist[e][seg] (LDS atomics);
//                    router_hist fuses this pass into the router
//   2. route_rowscan — one wave per expert: exclusive scan of hist[e][:] in
//                    place (the expert's rows that earlier segments own) and
//                    counts[e]
//   3. route_rank  — every workgroup scans counts into offsets in LDS; a
//                    wave then walks pairs in order, 64 at a time (ids
//                    prefetched into registers); lanes with equal expert ids
//                    are found with one ballot per id bit, so the rank inside
//                    a chunk is a popcount of lower matching lanes.  The
//                    stand-alone sort gives each 512-pair segment a workgroup
//                    (route_rank_wg: a wave per quarter, combined through
//                    per-wave expert counts in LDS); the fused router path
//                    gives each 128-pair segment a wave (route_rank).
//                    Order is stable and no global atomics are used.
// A pair whose id lies outside [0, E) gets no row: inv_map[p] = -1, and the
// number of such pairs is written to the status word at the head of the
// workspace (0 when every id is valid).
#include <mutex>
#include <type_traits>

#include "smoe_common.h"

namespace smoe {

constexpr int kSeg = 512;  // pairs per segment (one wave)

// ------------------------------------------------------------------ router
// A lane of the same 16-lane row for order-free reductions (max):
// levels 1 and 2 are quad permutes, 4 and 8 the row's half mirror (lane
// i <-> 7-i of each 8) and full mirror (i <-> 15-i), all DPP moves with no
// LDS round trip; after the four levels every lane of the row holds the
// row's result.  Levels 16 and 32 (64-lane groups) are lane swaps.
template <int kO>
__device__ __forceinline__ int red_lanes(int v) {
  // every lane is written (full masks), so the old value is v itself: no
  // register needs clearing first
  if constexpr (kO == 4) return __builtin_amdgcn_update_dpp(v, v, 0x141, 0xF, 0xF, false);
  else if constexpr (kO == 8) return __builtin_amdgcn_update_dpp(v, v, 0x140, 0xF, 0xF, false);
  else return xor_lanes<kO>(v);
}
template <int kO>
__device__ __forceinline__ float red_lanes(float v) {
  return __int_as_float(red_lanes<kO>(__float_as_int(v)));
}

// max(v, partner lane's v) for red_lanes' partners.  Rows of 16 use
// mov_dpp (old value undefined: every lane is written under full masks), so
// the compiler folds the lane move into the max as a DPP operand.
template <int kO>
__device__ __forceinline__ uint32_t max_lanes(uint32_t v) {
  if constexpr (kO == 1) return max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false));
  else if constexpr (kO == 2) return max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false));
  else if constexpr (kO == 4) return max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x141, 0xF, 0xF, false));
  else if constexpr (kO == 8) return max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x140, 0xF, 0xF, false));
  else return max(v, (uint32_t)xor_lanes<kO>((int)v));
}

// Butterfly over the kLPT lanes of a token group, top level first.
template <int kLPT, class F>
__device__ __forceinline__ void group_levels(F&& f) {
  if constexpr (kLPT >= 64) f(std::integral_constant<int, 32>{});
  if constexpr (kLPT >= 32) f(std::integral_constant<int, 16>{});
  f(std::integral_constant<int, 8>{});
  f(std::integral_constant<int, 4>{});
  f(std::integral_constant<int, 2>{});
  f(std::integral_constant<int, 1>{});
}

// Unsigned key of a selection score: larger score -> larger key, NaN (1)
// below every number, 0 for "no expert".  The order of a stable descending
// sort that puts NaN last (the oracle's argsort).  A score is p or p + bias
// with p >= +0, so it is never -0 (+0 + -0 is +0) and equal scores have
// equal keys.
__device__ __forceinline__ uint32_t score_key(float s) {
  const uint32_t u = __float_as_uint(s);
  const uint32_t k = u ^ ((uint32_t)((int32_t)u >> 31) | 0x80000000u);
  return s != s ? 1u : k;
}

// Softmax probabilities of one token's experts e = i + kLPT*q (q < kNV) held
// by lane i of a kLPT-lane group, from the logits already loaded into p[].
//
// Bit-reproducibility: the denominator is the reduction tree of a 64-lane
// wave in which "virtual lane" j (0..63) sums experts j, j+64, ... in order
// and a butterfly at distances 32, 16, ..., 1 combines the lanes.  With 16
// lanes per token, virtual lane j = i + 16a lives in physical lane i
// (a = q mod 4), so distances 32 and 16 are additions between a lane's own
// four partial sums and distances 8..1 are lane exchanges: the same
// operations on the same operands as the 64-lane tree, hence the same bits.
// The quotients p/den are correctly rounded (div_by_recip, or the IEEE
// division when some p is below 2^-100 anywhere in the wave).
template <int kLPT, int kNV, class Red>
__device__ __forceinline__ void token_softmax(float (&p)[kNV], Red red, float& m_out,
                                              float& den_out) {
  constexpr int kVirt = 64 / kLPT;
  float m = -__builtin_inff();
#pragma unroll
  for (int q = 0; q < kNV; ++q) m = fmaxf(m, p[q]);
  group_levels<kLPT>([&](auto o) { m = fmaxf(m, red(o, m)); });
  float vs[kVirt];
#pragma unroll
  for (int a = 0; a < kVirt; ++a) vs[a] = 0.0f;
#pragma unroll
  for (int q = 0; q < kNV; ++q) {
    p[q] = expf32_nonpos(p[q] - m);  // experts past E hold -inf: exp gives exactly 0
    vs[q % kVirt] = vs[q % kVirt] + p[q];
  }
  float den;
  if constexpr (kVirt == 4) den = (vs[0] + vs[2]) + (vs[1] + vs[3]);  // distances 32, 16
  else den = vs[0];
  // the sum keeps the xor partners: its rounding is part of the contract
  group_levels<kLPT>([&](auto o) { den = den + xor_lanes<decltype(o)::value>(den); });
  bool tiny = false;
#pragma unroll
  for (int q = 0; q < kNV; ++q) tiny = tiny | ((p[q] > 0.0f) & (p[q] < 0x1p-100f));
  if (__builtin_amdgcn_ballot_w64(tiny)) {
#pragma unroll
    for (int q = 0; q < kNV; ++q) p[q] = p[q] / den;
  } else {
    const float y = 1.0f / den;
#pragma unroll
    for (int q = 0; q < kNV; ++q) p[q] = div_by_recip(p[q], den, y);
  }
  m_out = m;
  den_out = den;
}

// Routing of one token by a group of kLPT (16 or 64) lanes; lane i of the
// group holds experts e = i + kLPT*q, q < kNV.  ptab is the group's E-float
// LDS table (a wave's LDS accesses complete in order, so no barrier guards
// it within the group).
//
// Top-K is a total order (score desc, id asc), so the arg-max tree shape
// does not change the picks; the K picked probabilities are summed in pick
// order.  Lane (k mod kLPT) returns pick k in slot k / kLPT.
template <int kLPT, int kNV>
struct TokenRoute {
  int id[2];
  float w[2];
};

template <int kLPT, int kNV>
__device__ __forceinline__ TokenRoute<kLPT, kNV> route_token(const float* __restrict__ row,
                                                             const float* __restrict__ bias,
                                                             int E, int K, int i,
                                                             float* __restrict__ ptab) {
  float p[kNV];
  float b[kNV];  // the selection bias
  // every load is unconditional (experts past E re-read expert E-1 and are
  // masked afterwards): a load under a branch would get a vmcnt(0) wait at
  // the branch join, one HBM round trip per load
  if (E == kLPT * kNV) {  // every expert index is valid: constant offsets
#pragma unroll
    for (int q = 0; q < kNV; ++q) p[q] = row[i + kLPT * q];
    if (bias) {
#pragma unroll
      for (int q = 0; q < kNV; ++q) b[q] = bias[i + kLPT * q];
    }
  } else {
#pragma unroll
    for (int q = 0; q < kNV; ++q) p[q] = row[min(i + kLPT * q, E - 1)];
    if (bias) {
#pragma unroll
      for (int q = 0; q < kNV; ++q) b[q] = bias[min(i + kLPT * q, E - 1)];
    }
#pragma unroll
    for (int q = 0; q < kNV; ++q)
      if (i + kLPT * q >= E) p[q] = -__builtin_inff();
  }
  float m, den;
  token_softmax<kLPT, kNV>(p, [](auto o, float v) { return red_lanes<decltype(o)::value>(v); }, m,
                           den);
  uint32_t key[kNV];
#pragma unroll
  for (int q = 0; q < kNV; ++q) {
    const int e = i + kLPT * q;
    ptab[e] = p[q];  // the table has kLPT*kNV entries: no test needed
    key[q] = e < E ? score_key(bias ? p[q] + b[q] : p[q]) : 0u;
  }
  // Each lane offers its best expert not yet picked; the group's arg-max
  // picks one per round.  A lane keeps its three best remaining experts
  // (slot 0 first) and rescans only when all three are gone: the experts a
  // lane gave up are exactly its best ones in the order (score desc, id
  // asc), so the rest are those after the last one it gave up (lk, li).
  uint32_t s0 = 0, s1 = 0, s2 = 0;  // keys; 0 = empty slot
  int i0 = -1, i1 = -1, i2 = -1;
  uint32_t lk = 0;
  int li = -1;
  auto top3 = [&](auto refill) {
    s0 = s1 = s2 = 0;
    i0 = i1 = i2 = -1;
#pragma unroll
    for (int q = 0; q < kNV; ++q) {
      const int id = i + kLPT * q;
      uint32_t u = key[q];
      if constexpr (decltype(refill)::value)
        u = ((u < lk) | ((u == lk) & (id > li))) ? u : 0u;  // experts not yet given up
      // ids ascend with q: a strict > keeps the lower id ahead on equal keys
      const bool c0 = u > s0, c1 = u > s1, c2 = u > s2;
      s2 = c1 ? s1 : (c2 ? u : s2);
      i2 = c1 ? i1 : (c2 ? id : i2);
      s1 = c0 ? s0 : (c1 ? u : s1);
      i1 = c0 ? i0 : (c1 ? id : i1);
      s0 = c0 ? u : s0;
      i0 = c0 ? id : i0;
    }
  };
  top3(std::false_type{});
  bool more = s2 != 0;  // experts beyond the three slots may remain
  TokenRoute<kLPT, kNV> r;
  r.id[0] = r.id[1] = 0;
  r.w[0] = r.w[1] = 0.0f;
  float psum = 0.0f;
  for (int k = 0; k < K; ++k) {
    // arg-max of (key, -id) over the group in two order-free max passes:
    // the largest key, then the largest ~id among the lanes offering it.
    // An empty lane offers key 0 and loses to every expert (K <= E
    // guarantees a real winner).
    uint32_t hi = s0;
    group_levels<kLPT>([&](auto o) { hi = max_lanes<decltype(o)::value>(hi); });
    uint32_t lo = s0 == hi ? ~(uint32_t)i0 : 0u;
    group_levels<kLPT>([&](auto o) { lo = max_lanes<decltype(o)::value>(lo); });
    const int bi = (int)~lo;
    if (bi == i0) {  // this lane gave the winner: advance its slots
      lk = s0;
      li = i0;
      s0 = s1;
      i0 = i1;
      s1 = s2;
      i1 = i2;
      s2 = 0;
      i2 = -1;
    }
    const bool refill = (s0 == 0) & more;
    if (__builtin_amdgcn_ballot_w64(refill)) {
      if (refill) {
        top3(std::true_type{});
        more = s2 != 0;
      }
    }
    const float bp = ptab[bi];
    psum = psum + bp;
    if ((k & (kLPT - 1)) == i) {  // static slot indices keep r in registers
      if (kLPT == 64 || k < kLPT) {
        r.id[0] = bi;
        r.w[0] = bp;
      } else {
        r.id[1] = bi;
        r.w[1] = bp;
      }
    }
  }
  r.w[0] = r.w[0] / psum;
  r.w[1] = r.w[1] / psum;
  return r;
}

// Router only: kLPT lanes per token, 256 threads.
template <int kLPT, int kNV>
__global__ __launch_bounds__(256) void router_topk_kernel(
    const float* __restrict__ logits, const float* __restrict__ bias, int T, int E, int K,
    int32_t* __restrict__ topk_idx, float* __restrict__ topk_w) {
  __shared__ float ptab[256 * kNV];  // E <= kLPT*kNV probabilities per token group
  const int i = threadIdx.x & (kLPT - 1);
  const int g = threadIdx.x / kLPT;
  const int t = blockIdx.x * (256 / kLPT) + g;
  if (t >= T) return;  // whole token groups leave; no workgroup barrier below
  const TokenRoute<kLPT, kNV> r =
      route_token<kLPT, kNV>(logits + (size_t)t * E, bias, E, K, i, ptab + g * kLPT * kNV);
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int k = s * kLPT + i;
    if (k < K) {
      topk_idx[(size_t)t * K + k] = r.id[s];
      topk_w[(size_t)t * K + k] = r.w[s];
    }
  }
}

// Router backward.  With p = softmax(l), the picks s_0..s_{K-1},
// S = sum_k p[s_k] (pick order) and w_k = p[s_k] / S, the gradient g_k of
// w_k gives
//   c = sum_k g_k w_k,  dp[s_k] = (g_k - c) / S  (0 for experts not picked),
//   dl_e = p_e (dp_e - sum_k p[s_k] dp[s_k]).
// The bias only selects, so it has no gradient.  p is recomputed exactly as
// the forward computes it; every lane evaluates the K-term sums itself (the
// picked probabilities from their logits), so no lane exchange is needed
// beyond the softmax reductions.
template <int kLPT, int kNV, int kMaxK>
__global__ __launch_bounds__(256) void router_topk_bwd_kernel(
    const float* __restrict__ logits, const int32_t* __restrict__ topk_idx,
    const float* __restrict__ dtopk_w, int T, int E, int K, float* __restrict__ dlogits) {
  const int i = threadIdx.x & (kLPT - 1);
  const int t = blockIdx.x * (256 / kLPT) + threadIdx.x / kLPT;
  if (t >= T) return;
  const float* row = logits + (size_t)t * E;
  float p[kNV];
#pragma unroll
  for (int q = 0; q < kNV; ++q) p[q] = row[min(i + kLPT * q, E - 1)];  // unconditional loads
#pragma unroll
  for (int q = 0; q < kNV; ++q)
    if (i + kLPT * q >= E) p[q] = -__builtin_inff();
  const int32_t* ids = topk_idx + (size_t)t * K;
  const float* g = dtopk_w + (size_t)t * K;
  // the picked logits, loaded before the softmax so that their latency
  // overlaps it; their probabilities are formed once each.  K <= kMaxK: static indices keep
  // the arrays in registers, and the loads are unconditional (index clamped
  // to K-1, the extra terms masked) so that all of them are in flight at once.
  float pk[kMaxK], gk[kMaxK];
  int ek[kMaxK];
#pragma unroll
  for (int k = 0; k < kMaxK; ++k) {
    ek[k] = min(max(ids[min(k, K - 1)], 0), E - 1);
    gk[k] = g[min(k, K - 1)];
  }
#pragma unroll
  for (int k = 0; k < kMaxK; ++k) pk[k] = row[ek[k]];
  float m, den;
  token_softmax<kLPT, kNV>(p, [](auto o, float v) { return xor_lanes<decltype(o)::value>(v); }, m,
                           den);
  float psum = 0.0f;
#pragma unroll
  for (int k = 0; k < kMaxK; ++k) {
    pk[k] = expf32_nonpos(pk[k] - m) / den;
    psum = k < K ? psum + pk[k] : psum;
  }
  float c = 0.0f;
#pragma unroll
  for (int k = 0; k < kMaxK; ++k) c = k < K ? c + gk[k] * (pk[k] / psum) : c;
  float dot = 0.0f;
  float dp[kNV];
#pragma unroll
  for (int q = 0; q < kNV; ++q) dp[q] = 0.0f;
#pragma unroll
  for (int k = 0; k < kMaxK; ++k) {
    const float d = (gk[k] - c) / psum;
    dot = k < K ? dot + pk[k] * d : dot;
#pragma unroll
    for (int q = 0; q < kNV; ++q) dp[q] = (k < K && i + kLPT * q == ek[k]) ? d : dp[q];
  }
  float* out = dlogits + (size_t)t * E;
#pragma unroll
  for (int q = 0; q < kNV; ++q) {
    const int e = i + kLPT * q;
    if (e < E) out[e] = p[q] * (dp[q] - dot);
  }
}

// Router fused with the sort's first pass: workgroup s routes every token
// that has a pair in segment s (pairs s*kSegR .. +kSegR; a token whose pairs
// straddle two segments is routed by both workgroups, and each writes only
// its own pairs), counts the segment's picks per expert in LDS and writes
// the histogram column hist[e][s] that route_rowscan and route_rank consume.
// A segment of 128 pairs is 16 tokens at top-8, one pass of a 256-thread
// workgroup: as many workgroups as the plain router launches.
constexpr int kSegR = 128;  // pairs per segment of the fused path
constexpr int kHistThreads = 256;
template <int kLPT, int kNV>
__global__ __launch_bounds__(kHistThreads) void router_hist_kernel(
    const float* __restrict__ logits, const float* __restrict__ bias, int T, int E, int K,
    int nseg, int32_t* __restrict__ topk_idx, float* __restrict__ topk_w,
    int32_t* __restrict__ hist) {
  extern __shared__ int32_t hh[];  // [E]
  __shared__ float ptab[kHistThreads * kNV];  // E <= kLPT*kNV probabilities per token group
  const int seg = blockIdx.x;
  const int R = T * K;
  for (int e = threadIdx.x; e < E; e += kHistThreads) hh[e] = 0;
  __syncthreads();
  const int p0 = seg * kSegR, p1 = min(R, p0 + kSegR);
  const int t0 = p0 / K, t1 = (p1 - 1) / K;  // tokens with a pair in [p0, p1)
  const int i = threadIdx.x & (kLPT - 1);
  for (int t = t0 + threadIdx.x / kLPT; t <= t1; t += kHistThreads / kLPT) {
    const TokenRoute<kLPT, kNV> r = route_token<kLPT, kNV>(
        logits + (size_t)t * E, bias, E, K, i, ptab + (threadIdx.x / kLPT) * kLPT * kNV);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int k = s * kLPT + i;
      const int p = t * K + k;
      if (k < K && p >= p0 && p < p1) {
        topk_idx[p] = r.id[s];
        topk_w[p] = r.w[s];
        atomicAdd(&hh[r.id[s]], 1);
      }
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += kHistThreads) hist[(size_t)e * nseg + seg] = hh[e];
}

// ------------------------------------------------------------------- sort
constexpr int kPerLane = kSeg / kWave;

__global__ __launch_bounds__(256) void route_hist_kernel(const int32_t* __restrict__ idx,
                                                         int R, int E, int nseg,
                                                         int32_t* __restrict__ hist) {
  extern __shared__ int32_t h_lds[];  // [4][E]
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int seg = blockIdx.x * 4 + w;
  if (seg >= nseg) return;  // whole wave leaves; no workgroup barrier below
  int32_t* h = h_lds + w * E;
  for (int e = lane; e < E; e += kWave) h[e] = 0;
  const int p0 = seg * kSeg;
  int v[kPerLane];
#pragma unroll
  for (int i = 0; i < kPerLane; ++i) {
    const int p = p0 + i * kWave + lane;
    v[i] = p < R ? idx[p] : -1;
  }
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int i = 0; i < kPerLane; ++i)
    if ((unsigned)v[i] < (unsigned)E) atomicAdd(&h[v[i]], 1);
  __builtin_amdgcn_wave_barrier();
  for (int e = lane; e < E; e += kWave) hist[(size_t)e * nseg + seg] = h[e];
}

__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int u = __shfl_up(v, o, kWave);
    if (lane >= o) v += u;
  }
  return v;
}

// One wave per expert scans its histogram row: each lane takes 16
// consecutive entries per pass of 1024 (one wave-wide scan per pass instead
// of one per 64 entries).  Loads are unconditional (indices clamped to the
// row) so that they are all in flight before the first use.
__global__ __launch_bounds__(256) void route_rowscan_kernel(int32_t* __restrict__ hist, int E,
                                                            int nseg,
                                                            int32_t* __restrict__ counts) {
  constexpr int kPer = 16;
  const int lane = threadIdx.x & 63;
  const int e = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (e >= E) return;
  int32_t* row = hist + (size_t)e * nseg;
  int carry = 0;
  for (int s0 = 0; s0 < nseg; s0 += kWave * kPer) {
    const int b = s0 + lane * kPer;
    int v[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) v[i] = row[min(b + i, nseg - 1)];
    int tot = 0;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      v[i] = b + i < nseg ? v[i] : 0;
      tot += v[i];
    }
    const int inc = wave_incl_scan(tot, lane);
    int run = carry + inc - tot;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      if (b + i < nseg) row[b + i] = run;
      run += v[i];
    }
    carry += __shfl(inc, kWave - 1, kWave);
  }
  if (lane == 0) counts[e] = carry;
}

template <int kSegT>
__global__ __launch_bounds__(256) void route_rank_kernel(const int32_t* __restrict__ idx,
                                                         const int32_t* __restrict__ rowpre,
                                                         const int32_t* __restrict__ counts,
                                                         int R, int E, int nseg, int nbits,
                                                         int32_t* __restrict__ offsets,
                                                         int32_t* __restrict__ row_map,
                                                         int32_t* __restrict__ inv_map,
                                                         int32_t* __restrict__ status) {
  extern __shared__ int32_t c_lds[];  // offs[E] then cur[4][E]
  __shared__ int32_t wtot[4];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  int32_t* offs = c_lds;
  int32_t* cur = c_lds + E + w * E;
  // offsets = exclusive scan of counts (each thread owns up to 4 experts)
  const int per = (E + 255) / 256;
  int loc[4], run = 0;
  for (int i = 0; i < per; ++i) {
    const int e = tid * per + i;
    run += e < E ? counts[e] : 0;
    loc[i] = run;
  }
  const int inc = wave_incl_scan(run, lane);
  if (lane == kWave - 1) wtot[w] = inc;
  __syncthreads();
  int base = inc - run;
  for (int j = 0; j < w; ++j) base += wtot[j];
  for (int i = 0; i < per; ++i) {
    const int e = tid * per + i;
    if (e < E) {
      const int ex = base + (i ? loc[i - 1] : 0);
      offs[e] = ex;
      if (blockIdx.x == 0) offsets[e] = ex;
    }
  }
  if (blockIdx.x == 0 && tid == 0) {
    const int total = wtot[0] + wtot[1] + wtot[2] + wtot[3];
    offsets[E] = total;
    *status = R - total;  // pairs dropped for an id outside [0, E)
  }
  __syncthreads();

  const int seg = blockIdx.x * 4 + w;
  if (seg >= nseg) return;
  constexpr int kPL = kSegT / kWave;
  const int p0 = seg * kSegT;
  int v[kPL];
#pragma unroll
  for (int i = 0; i < kPL; ++i) {
    const int p = p0 + i * kWave + lane;
    v[i] = p < R ? idx[p] : E;  // E is a sentinel id no valid lane has
  }
  for (int e = lane; e < E; e += kWave) cur[e] = offs[e] + rowpre[(size_t)e * nseg + seg];
  __builtin_amdgcn_wave_barrier();
  const uint64_t lt = (1ull << lane) - 1ull;
#pragma unroll
  for (int i = 0; i < kPL; ++i) {
    const int p = p0 + i * kWave + lane;
    const bool valid = (unsigned)v[i] < (unsigned)E;
    const int e = valid ? v[i] : E;  // out-of-range ids rank as the sentinel
    uint64_t m = ~0ull;
    for (int b = 0; b < nbits; ++b) {
      const bool bit = (e >> b) & 1;
      const uint64_t bal = __ballot(bit);
      m &= bit ? bal : ~bal;
    }
    int r = 0;
    if (valid) r = cur[e] + __popcll(m & lt);
    __builtin_amdgcn_wave_barrier();
    if (valid && (m & lt) == 0) cur[e] += __popcll(m);
    __builtin_amdgcn_wave_barrier();
    if (valid) {
      row_map[r] = p;
      inv_map[p] = r;
    } else if (p < R) {
      inv_map[p] = -1;
    }
  }
}

// The rank pass with one workgroup per segment: wave w ranks pairs
// w*kSegT/4 .. +kSegT/4 of the segment in 64-pair chunks as
// route_rank_kernel does, counting per expert in LDS; after a barrier a
// pair's row is offs[e] + rowpre[e][seg] + the counts of expert e in the
// waves before it + its rank inside its wave.  Same rows as
// route_rank_kernel<kSegT> (order by pair index), four times the
// workgroups.
template <int kSegT>
__global__ __launch_bounds__(256) void route_rank_wg_kernel(const int32_t* __restrict__ idx,
                                                            const int32_t* __restrict__ rowpre,
                                                            const int32_t* __restrict__ counts,
                                                            int R, int E, int nseg, int nbits,
                                                            int32_t* __restrict__ offsets,
                                                            int32_t* __restrict__ row_map,
                                                            int32_t* __restrict__ inv_map,
                                                            int32_t* __restrict__ status) {
  extern __shared__ int32_t c_lds[];  // base[E] then cnt[4][E]
  __shared__ int32_t wtot[4];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int seg = blockIdx.x;
  int32_t* base = c_lds;
  int32_t* cnt = c_lds + E;
  constexpr int kPW = kSegT / 4;      // pairs per wave
  constexpr int kPL = kPW / kWave;    // 64-pair chunks per wave
  const int p0 = seg * kSegT + w * kPW;
  // every load issued first: this wave's ids, this thread's experts' counts
  // and segment prefixes
  int v[kPL];
#pragma unroll
  for (int i = 0; i < kPL; ++i) {
    const int p = p0 + i * kWave + lane;
    v[i] = p < R ? idx[p] : E;  // E is a sentinel id no valid lane has
  }
  const int per = (E + 255) / 256;
  int loc[4], pre[4], run = 0;
  for (int i = 0; i < per; ++i) {
    const int e = tid * per + i;
    run += e < E ? counts[e] : 0;
    loc[i] = run;
    pre[i] = e < E ? rowpre[(size_t)e * nseg + seg] : 0;
  }
  for (int e = tid; e < 4 * E; e += 256) cnt[e] = 0;
  // offsets = exclusive scan of counts; base[e] = offsets[e] + rowpre[e][seg]
  const int inc = wave_incl_scan(run, lane);
  if (lane == kWave - 1) wtot[w] = inc;
  __syncthreads();
  int b0 = inc - run;
  for (int j = 0; j < w; ++j) b0 += wtot[j];
  for (int i = 0; i < per; ++i) {
    const int e = tid * per + i;
    if (e < E) {
      const int ex = b0 + (i ? loc[i - 1] : 0);
      base[e] = ex + pre[i];
      if (blockIdx.x == 0) offsets[e] = ex;
    }
  }
  if (blockIdx.x == 0 && tid == 0) {
    const int total = wtot[0] + wtot[1] + wtot[2] + wtot[3];
    offsets[E] = total;
    *status = R - total;  // pairs dropped for an id outside [0, E)
  }
  // ranks inside this wave's pairs
  int32_t* mycnt = cnt + w * E;
  const uint64_t lt = (1ull << lane) - 1ull;
  int rl[kPL];
#pragma unroll
  for (int i = 0; i < kPL; ++i) {
    const bool valid = (unsigned)v[i] < (unsigned)E;
    const int e = valid ? v[i] : E;
    uint64_t m = ~0ull;
    for (int b = 0; b < nbits; ++b) {
      const bool bit = (e >> b) & 1;
      const uint64_t bal = __ballot(bit);
      m &= bit ? bal : ~bal;
    }
    rl[i] = valid ? mycnt[e] + __popcll(m & lt) : 0;
    __builtin_amdgcn_wave_barrier();
    if (valid && (m & lt) == 0) mycnt[e] += __popcll(m);
    __builtin_amdgcn_wave_barrier();
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kPL; ++i) {
    const int p = p0 + i * kWave + lane;
    if ((unsigned)v[i] < (unsigned)E) {
      const int e = v[i];
      int r = base[e] + rl[i];
      for (int j = 0; j < w; ++j) r += cnt[j * E + e];
      row_map[r] = p;
      inv_map[p] = r;
    } else if (p < R) {
      inv_map[p] = -1;
    }
  }
}

static inline int seg_count(int R, int seg = kSeg) { return (R + seg - 1) / seg; }

}  // namespace smoe

using namespace smoe;

// Router instance for E experts: 16 lanes per token up to E = 256, 64 above.
#define SMOE_ROUTE_DISPATCH(E, LAUNCH) \
  do {                                 \
    if ((E) <= 16) LAUNCH(16, 1);      \
    else if ((E) <= 32) LAUNCH(16, 2); \
    else if ((E) <= 64) LAUNCH(16, 4); \
    else if ((E) <= 128) LAUNCH(16, 8); \
    else if ((E) <= 256) LAUNCH(16, 16); \
    else if ((E) <= 512) LAUNCH(64, 8); \
    else LAUNCH(64, 16);               \
  } while (0)

static int check_router_args(const float* logits, const float* bias, int T, int E, int K,
                             const int32_t* topk_idx, const float* topk_w) {
  if (T <= 0) return SMOE_EINVAL_DIM;
  if (E <= 0 || E > SMOE_MAX_EXPERTS) return SMOE_EINVAL_EXPERTS;
  if (K <= 0 || K > E || K > 32) return SMOE_EINVAL_TOPK;
  if ((long long)T * E > 0x7fffffffLL || (long long)T * K > 0x7fffffffLL) return SMOE_EINVAL_DIM;
  if (!logits || !topk_idx || !topk_w) return SMOE_EINVAL_NULL;
  if (((uintptr_t)logits | (uintptr_t)topk_idx | (uintptr_t)topk_w | (uintptr_t)bias) & 3u)
    return SMOE_EINVAL_PTRALIGN;
  return SMOE_OK;
}

extern "C" int smoe_router_topk(const float* logits, const float* bias, int T, int E, int K,
                                int32_t* topk_idx, float* topk_w, void* stream) {
  const int st = check_router_args(logits, bias, T, E, K, topk_idx, topk_w);
  if (st) return st;
  hipStream_t s = (hipStream_t)stream;
#define SMOE_ROUTER(LPT, NV)                                                          \
  router_topk_kernel<LPT, NV><<<dim3((T + 256 / LPT - 1) / (256 / LPT)), dim3(256), 0, s>>>( \
      logits, bias, T, E, K, topk_idx, topk_w)
  SMOE_ROUTE_DISPATCH(E, SMOE_ROUTER);
#undef SMOE_ROUTER
  SMOE_RETURN_LAUNCH();
}

extern "C" int smoe_router_topk_bwd(const float* logits, const int32_t* topk_idx,
                                    const float* dtopk_w, int T, int E, int K, float* dlogits,
                                    void* stream) {
  if (T <= 0) return SMOE_EINVAL_DIM;
  if (E <= 0 || E > SMOE_MAX_EXPERTS) return SMOE_EINVAL_EXPERTS;
  if (K <= 0 || K > E || K > 32) return SMOE_EINVAL_TOPK;
  if ((long long)T * E > 0x7fffffffLL) return SMOE_EINVAL_DIM;
  if (!logits || !topk_idx || !dtopk_w || !dlogits) return SMOE_EINVAL_NULL;
  if (((uintptr_t)logits | (uintptr_t)topk_idx | (uintptr_t)dtopk_w | (uintptr_t)dlogits) & 3u)
    return SMOE_EINVAL_PTRALIGN;
  hipStream_t s = (hipStream_t)stream;
#define SMOE_RBWD_K(LPT, NV, MK)                                                              \
  router_topk_bwd_kernel<LPT, NV, MK><<<dim3((T + 256 / LPT - 1) / (256 / LPT)), dim3(256), 0, s>>>( \
      logits, topk_idx, dtopk_w, T, E, K, dlogits)
#define SMOE_RBWD(LPT, NV)                          \
  do {                                              \
    if (K <= 2) SMOE_RBWD_K(LPT, NV, 2);            \
    else if (K <= 8) SMOE_RBWD_K(LPT, NV, 8);       \
    else SMOE_RBWD_K(LPT, NV, 32);                  \
  } while (0)
  SMOE_ROUTE_DISPATCH(E, SMOE_RBWD);
#undef SMOE_RBWD_K
#undef SMOE_RBWD
  SMOE_RETURN_LAUNCH();
}

// Workspace: a 16-byte status block (int32 dropped-pair count first), then
// the per-segment histogram hist[E][nseg].
constexpr size_t kStatusBytes = 16;

static size_t sort_ws_bytes(int T, int K, int E, int seg) {
  return kStatusBytes + (size_t)E * seg_count(T * K, seg) * sizeof(int32_t);
}

extern "C" size_t smoe_route_sort_workspace_size(int T, int K, int E) {
  if (T <= 0 || K <= 0 || E <= 0 || (long long)T * K > 0x7fffffffLL) return 0;
  // enough for both sorts: the fused router's 128-pair segments need the
  // larger histogram
  return sort_ws_bytes(T, K, E, kSegR);
}

static int check_sort_args(int T, int K, int E, const int32_t* row_map, const int32_t* inv_map,
                           const int32_t* counts, const int32_t* offsets, const void* ws,
                           size_t ws_bytes, int seg) {
  if (T <= 0) return SMOE_EINVAL_DIM;
  if (E <= 0 || E > SMOE_MAX_EXPERTS) return SMOE_EINVAL_EXPERTS;
  if (K <= 0 || K > E || K > 32) return SMOE_EINVAL_TOPK;
  if ((long long)T * K > 0x7fffffffLL) return SMOE_EINVAL_DIM;
  if (!row_map || !inv_map || !counts || !offsets) return SMOE_EINVAL_NULL;
  if (((uintptr_t)row_map | (uintptr_t)inv_map | (uintptr_t)counts | (uintptr_t)offsets) & 3u)
    return SMOE_EINVAL_PTRALIGN;
  if (!ws || ((uintptr_t)ws & 15u)) return ws ? SMOE_EINVAL_PTRALIGN : SMOE_EINVAL_WORKSPACE;
  if (ws_bytes < sort_ws_bytes(T, K, E, seg)) return SMOE_EINVAL_WORKSPACE;
  return SMOE_OK;
}

// Passes 2 and 3 of the sort, from a filled histogram of nseg segments of
// kSegT pairs.
template <int kSegT>
static void sort_tail(const int32_t* topk_idx, int R, int E, int nseg, int32_t* row_map,
                      int32_t* inv_map, int32_t* counts, int32_t* offsets, void* ws,
                      hipStream_t s) {
  int nbits = 1;
  while ((1 << nbits) <= E) ++nbits;  // ids 0..E (E is the sentinel)
  int32_t* status = (int32_t*)ws;
  int32_t* hist = (int32_t*)((char*)ws + kStatusBytes);
  route_rowscan_kernel<<<dim3((E + 3) / 4), dim3(256), 0, s>>>(hist, E, nseg, counts);
  route_rank_kernel<kSegT><<<dim3((nseg + 3) / 4), dim3(256), (size_t)5 * E * sizeof(int32_t), s>>>(
      topk_idx, hist, counts, R, E, nseg, nbits, offsets, row_map, inv_map, status);
}

extern "C" int smoe_route_sort(const int32_t* topk_idx, int T, int K, int E, int32_t* row_map,
                               int32_t* inv_map, int32_t* counts, int32_t* offsets, void* ws,
                               size_t ws_bytes, void* stream) {
  int st = check_sort_args(T, K, E, row_map, inv_map, counts, offsets, ws, ws_bytes, kSeg);
  if (st) return st;
  if (!topk_idx) return SMOE_EINVAL_NULL;
  if ((uintptr_t)topk_idx & 3u) return SMOE_EINVAL_PTRALIGN;
  const int R = T * K;
  const int nseg = seg_count(R);
  int32_t* hist = (int32_t*)((char*)ws + kStatusBytes);
  hipStream_t s = (hipStream_t)stream;
  route_hist_kernel<<<dim3((nseg + 3) / 4), dim3(256), (size_t)4 * E * sizeof(int32_t), s>>>(
      topk_idx, R, E, nseg, hist);
  int nbits = 1;
  while ((1 << nbits) <= E) ++nbits;  // ids 0..E (E is the sentinel)
  route_rowscan_kernel<<<dim3((E + 3) / 4), dim3(256), 0, s>>>(hist, E, nseg, counts);
  route_rank_wg_kernel<kSeg><<<dim3(nseg), dim3(256), (size_t)5 * E * sizeof(int32_t), s>>>(
      topk_idx, hist, counts, R, E, nseg, nbits, offsets, row_map, inv_map, (int32_t*)ws);
  SMOE_RETURN_LAUNCH();
}

extern "C" int smoe_route_topk_sort(const float* logits, const float* bias, int T, int E, int K,
                                    int32_t* topk_idx, float* topk_w, int32_t* row_map,
                                    int32_t* inv_map, int32_t* counts, int32_t* offsets,
                                    void* ws, size_t ws_bytes, void* stream) {
  int st = check_router_args(logits, bias, T, E, K, topk_idx, topk_w);
  if (st) return st;
  st = check_sort_args(T, K, E, row_map, inv_map, counts, offsets, ws, ws_bytes, kSegR);
  if (st) return st;
  const int R = T * K;
  const int nseg = seg_count(R, kSegR);
  int32_t* hist = (int32_t*)((char*)ws + kStatusBytes);
  hipStream_t s = (hipStream_t)stream;
#define SMOE_RHIST(LPT, NV)                                                                \
  router_hist_kernel<LPT, NV><<<dim3(nseg), dim3(kHistThreads), (size_t)E * sizeof(int32_t), s>>>( \
      logits, bias, T, E, K, nseg, topk_idx, topk_w, hist)
  SMOE_ROUTE_DISPATCH(E, SMOE_RHIST);
#undef SMOE_RHIST
  sort_tail<kSegR>(topk_idx, R, E, nseg, row_map, inv_map, counts, offsets, ws, s);
  SMOE_RETURN_LAUNCH();
}

// ---------------------------------------------------- allocation-free sort
// The sort's workspace (status block + histogram) as a file-scope device
// array: callers that cannot allocate (HIP graph capture, serving loops)
// use smoe_route_sort_noalloc.  Each GPU holds its own copy for the life of
// the process; its device address is looked up once per device with
// hipGetSymbolAddress and only that address is passed to kernels.  Every
// call overwrites the whole status block and the histogram columns it uses,
// so nothing needs clearing between calls; calls that overlap on one GPU
// (different streams) share the array and race.
namespace smoe {
constexpr size_t kScratchBytes = kStatusBytes + ((size_t)1 << 22);  // 4 MiB of histogram
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
static void* g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

// The current device's address of `scratch`, or nullptr on a HIP error.
static void* scratch_ptr(hipError_t* err) {
  int dev = 0;
  *err = hipGetDevice(&dev);
  if (*err != hipSuccess) return nullptr;
  if (dev < 0 || dev >= kMaxDevices) {
    *err = hipErrorInvalidDevice;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    *err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (*err != hipSuccess) return nullptr;
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}
}  // namespace smoe

extern "C" size_t smoe_route_sort_noalloc_max_bytes(void) { return smoe::kScratchBytes; }

extern "C" int smoe_route_sort_noalloc(const int32_t* topk_idx, int T, int K, int E,
                                       int32_t* row_map, int32_t* inv_map, int32_t* counts,
                                       int32_t* offsets, void* stream) {
  if (T <= 0 || K <= 0 || E <= 0) return SMOE_EINVAL_DIM;
  if ((long long)T * K > 0x7fffffffLL) return SMOE_EINVAL_DIM;
  // the sort needs E * ceil(T*K / 512) histogram words: reject what the
  // static array cannot hold
  if (sort_ws_bytes(T, K, E, kSeg) > kScratchBytes) return SMOE_EINVAL_WORKSPACE;
  hipError_t err = hipSuccess;
  void* ws = scratch_ptr(&err);
  if (!ws) return err == hipSuccess ? SMOE_EINVAL_WORKSPACE : (int)err;
  return smoe_route_sort(topk_idx, T, K, E, row_map, inv_map, counts, offsets, ws,
                         kScratchBytes, stream);
}
