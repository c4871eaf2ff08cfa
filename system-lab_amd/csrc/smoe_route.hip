// smoe_route.hip — router top-k and the stable expert sort (gfx950).
//
// Router (C1): one wave per token.  Softmax over fp32 logits with the
// library's exp; the denominator is a fixed reduction tree (lane j sums
// experts j, j+64, ... in order, then an xor butterfly 32..1), so the
// probabilities are bit-reproducible.  Top-K by (score desc, id asc).
//
// Sort (C2): three small launches over the R = T*K (token, slot) pairs,
// each wave owning one segment of kSeg consecutive pairs:
//   1. route_hist  — per-segment expert histogram hist[e][seg] (LDS atomics)
//   2. route_rowscan — one wave per expert: exclusive scan of hist[e][:] in
//                    place (the expert's rows that earlier segments own) and
//                    counts[e]
//   3. route_rank  — every workgroup scans counts into offsets in LDS; each
//                    wave then walks its segment in pair order, 64 pairs at a
//                    time (ids prefetched into registers); lanes with equal
//                    expert ids are found with one ballot per id bit, so the
//                    rank inside a chunk is a popcount of lower matching lanes.
//                    Order is stable and no global atomics are used.
#include "smoe_common.h"

namespace smoe {

constexpr int kSeg = 512;  // pairs per segment (one wave)

// ------------------------------------------------------------------ router
// One butterfly level of the wave arg-max: the partner at distance kO wins
// with a larger score, or an equal score and a lower id (0x7fffffff marks a
// lane with no candidate).
template <int kO>
__device__ __forceinline__ void argmax_step(float& bs, int& bi, float& bp) {
  const float os = xor_lanes<kO>(bs);
  const int oi = xor_lanes<kO>(bi);
  const float op = xor_lanes<kO>(bp);
  const bool take = (oi != 0x7fffffff) && (bi == 0x7fffffff || os > bs || (os == bs && oi < bi));
  if (take) {
    bs = os;
    bi = oi;
    bp = op;
  }
}

template <int NC>
__global__ __launch_bounds__(256) void router_topk_kernel(
    const float* __restrict__ logits, const float* __restrict__ bias, int T, int E, int K,
    int32_t* __restrict__ topk_idx, float* __restrict__ topk_w) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const float* row = logits + (size_t)t * E;
  float l[NC];
  bool ok[NC];
  float m = -__builtin_inff();
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    int j = c * kWave + lane;
    ok[c] = j < E;
    l[c] = ok[c] ? row[j] : -__builtin_inff();
    m = fmaxf(m, l[c]);
  }
  m = wave_max(m);
  float p[NC];
  float acc = 0.0f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    p[c] = ok[c] ? expf32(l[c] - m) : 0.0f;
    acc = acc + p[c];
  }
  const float denom = wave_sum_tree(acc);
  float sc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    p[c] = p[c] / denom;
    sc[c] = bias ? p[c] + (ok[c] ? bias[c * kWave + lane] : 0.0f) : p[c];
  }
  float psum = 0.0f;
  float my_p = 0.0f;
  int my_id = 0;
  for (int k = 0; k < K; ++k) {
    // lane-local best among not-yet-taken experts
    float bs = -__builtin_inff();
    int bi = 0x7fffffff;
    float bp = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      if (ok[c] && (sc[c] > bs || bi == 0x7fffffff)) {
        bs = sc[c];
        bi = c * kWave + lane;
        bp = p[c];
      }
    }
    // wave arg-max: larger score wins, equal scores -> lower id
    argmax_step<32>(bs, bi, bp);
    argmax_step<16>(bs, bi, bp);
    argmax_step<8>(bs, bi, bp);
    argmax_step<4>(bs, bi, bp);
    argmax_step<2>(bs, bi, bp);
    argmax_step<1>(bs, bi, bp);
    // owner lane retires the winner
#pragma unroll
    for (int c = 0; c < NC; ++c)
      if (c * kWave + lane == bi) ok[c] = false;
    psum = psum + bp;
    if (lane == k) {
      my_p = bp;
      my_id = bi;
    }
  }
  if (lane < K) {
    topk_idx[(size_t)t * K + lane] = my_id;
    topk_w[(size_t)t * K + lane] = my_p / psum;
  }
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

__global__ __launch_bounds__(256) void route_rowscan_kernel(int32_t* __restrict__ hist, int E,
                                                            int nseg,
                                                            int32_t* __restrict__ counts) {
  const int lane = threadIdx.x & 63;
  const int e = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (e >= E) return;
  int32_t* row = hist + (size_t)e * nseg;
  int carry = 0;
  for (int s0 = 0; s0 < nseg; s0 += kWave) {
    const int s = s0 + lane;
    const int v = s < nseg ? row[s] : 0;
    const int inc = wave_incl_scan(v, lane);
    if (s < nseg) row[s] = carry + inc - v;
    carry += __shfl(inc, kWave - 1, kWave);
  }
  if (lane == 0) counts[e] = carry;
}

__global__ __launch_bounds__(256) void route_rank_kernel(const int32_t* __restrict__ idx,
                                                         const int32_t* __restrict__ rowpre,
                                                         const int32_t* __restrict__ counts,
                                                         int R, int E, int nseg, int nbits,
                                                         int32_t* __restrict__ offsets,
                                                         int32_t* __restrict__ row_map,
                                                         int32_t* __restrict__ inv_map) {
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
  if (blockIdx.x == 0 && tid == 0) offsets[E] = wtot[0] + wtot[1] + wtot[2] + wtot[3];
  __syncthreads();

  const int seg = blockIdx.x * 4 + w;
  if (seg >= nseg) return;
  const int p0 = seg * kSeg;
  int v[kPerLane];
#pragma unroll
  for (int i = 0; i < kPerLane; ++i) {
    const int p = p0 + i * kWave + lane;
    v[i] = p < R ? idx[p] : E;  // E is a sentinel id no valid lane has
  }
  for (int e = lane; e < E; e += kWave) cur[e] = offs[e] + rowpre[(size_t)e * nseg + seg];
  __builtin_amdgcn_wave_barrier();
  const uint64_t lt = (1ull << lane) - 1ull;
#pragma unroll
  for (int i = 0; i < kPerLane; ++i) {
    const int p = p0 + i * kWave + lane;
    const int e = v[i];
    const bool valid = (unsigned)e < (unsigned)E;
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
    }
  }
}

static inline int seg_count(int R) { return (R + kSeg - 1) / kSeg; }

}  // namespace smoe

using namespace smoe;

extern "C" int smoe_router_topk(const float* logits, const float* bias, int T, int E, int K,
                                int32_t* topk_idx, float* topk_w, void* stream) {
  if (T <= 0) return SMOE_EINVAL_DIM;
  if (E <= 0 || E > SMOE_MAX_EXPERTS) return SMOE_EINVAL_EXPERTS;
  if (K <= 0 || K > E || K > 32) return SMOE_EINVAL_TOPK;
  if (!logits || !topk_idx || !topk_w) return SMOE_EINVAL_NULL;
  if (((uintptr_t)logits | (uintptr_t)topk_idx | (uintptr_t)topk_w | (uintptr_t)bias) & 3u)
    return SMOE_EINVAL_PTRALIGN;
  const int nc = (E + kWave - 1) / kWave;
  dim3 grid((T + 3) / 4), block(256);
  hipStream_t s = (hipStream_t)stream;
#define SMOE_ROUTER(NC) \
  router_topk_kernel<NC><<<grid, block, 0, s>>>(logits, bias, T, E, K, topk_idx, topk_w)
  if (nc <= 1) SMOE_ROUTER(1);
  else if (nc <= 2) SMOE_ROUTER(2);
  else if (nc <= 4) SMOE_ROUTER(4);
  else if (nc <= 8) SMOE_ROUTER(8);
  else SMOE_ROUTER(16);
#undef SMOE_ROUTER
  SMOE_RETURN_LAUNCH();
}

extern "C" size_t smoe_route_sort_workspace_size(int T, int K, int E) {
  if (T <= 0 || K <= 0 || E <= 0) return 0;
  const size_t R = (size_t)T * K;
  return (size_t)E * seg_count((int)R) * sizeof(int32_t);
}

extern "C" int smoe_route_sort(const int32_t* topk_idx, int T, int K, int E, int32_t* row_map,
                               int32_t* inv_map, int32_t* counts, int32_t* offsets, void* ws,
                               size_t ws_bytes, void* stream) {
  if (T <= 0) return SMOE_EINVAL_DIM;
  if (E <= 0 || E > SMOE_MAX_EXPERTS) return SMOE_EINVAL_EXPERTS;
  if (K <= 0 || K > E || K > 32) return SMOE_EINVAL_TOPK;
  if ((long long)T * K > 0x7fffffffLL) return SMOE_EINVAL_DIM;
  if (!topk_idx || !row_map || !inv_map || !counts || !offsets) return SMOE_EINVAL_NULL;
  if (((uintptr_t)topk_idx | (uintptr_t)row_map | (uintptr_t)inv_map | (uintptr_t)counts |
       (uintptr_t)offsets) & 3u)
    return SMOE_EINVAL_PTRALIGN;
  if (!ws || ws_bytes < smoe_route_sort_workspace_size(T, K, E)) return SMOE_EINVAL_WORKSPACE;
  const int R = T * K;
  const int nseg = seg_count(R);
  int nbits = 1;
  while ((1 << nbits) <= E) ++nbits;  // ids 0..E (E is the sentinel)
  int32_t* hist = (int32_t*)ws;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((nseg + 3) / 4), block(256);
  route_hist_kernel<<<grid, block, (size_t)4 * E * sizeof(int32_t), s>>>(topk_idx, R, E, nseg,
                                                                        hist);
  route_rowscan_kernel<<<dim3((E + 3) / 4), block, 0, s>>>(hist, E, nseg, counts);
  route_rank_kernel<<<grid, block, (size_t)5 * E * sizeof(int32_t), s>>>(
      topk_idx, hist, counts, R, E, nseg, nbits, offsets, row_map, inv_map);
  SMOE_RETURN_LAUNCH();
}
