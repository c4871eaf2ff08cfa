// smoe_combine.hip — weighted unpermute/combine (gfx950).
//
// One wave per output token.  A lane owns 8 consecutive bf16 columns of a
// 512-column chunk; for each chunk it gathers the K expert-output rows of
// its token (K 128-bit loads in flight), accumulates w[t,k] * y in fp32 in
// k order with separately rounded multiply and add, and writes the bf16
// (round-to-nearest-even) result with one 128-bit non-temporal store.
#include "smoe_common.h"

namespace smoe {

typedef uint32_t v4u __attribute__((ext_vector_type(4)));

template <bool kNT>
__device__ __forceinline__ uint4 load16(const uint16_t* p) {
  if constexpr (kNT) {
    const v4u v = __builtin_nontemporal_load((const v4u*)p);
    return make_uint4(v.x, v.y, v.z, v.w);
  } else {
    return *(const uint4*)p;
  }
}

// kU column chunks of 512 are gathered per iteration, so every lane has
// kU*K 128-bit loads in flight.
template <int kMaxK, int kU, bool kNT>
__global__ __launch_bounds__(256) void combine_kernel(const uint16_t* __restrict__ y,
                                                      const int32_t* __restrict__ inv_map,
                                                      const float* __restrict__ w, int T,
                                                      int K, int H,
                                                      uint16_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int R = T * K;
  int r[kMaxK];
  float wk[kMaxK];
#pragma unroll
  for (int k = 0; k < kMaxK; ++k) {
    if (k < K) {
      r[k] = inv_map[(size_t)t * K + k];
      wk[k] = w[(size_t)t * K + k];
      if ((unsigned)r[k] >= (unsigned)R) {  // malformed map: contribute nothing
        r[k] = 0;
        wk[k] = 0.0f;
      }
    }
  }
  for (int c0 = lane * 8; c0 < H; c0 += kU * kWave * 8) {
    uint4 v[kU][kMaxK];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int col = c0 + u * kWave * 8;
#pragma unroll
      for (int k = 0; k < kMaxK; ++k)
        if (k < K && col < H) v[u][k] = load16<kNT>(y + (size_t)r[k] * H + col);
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int col = c0 + u * kWave * 8;
      if (col >= H) break;
      float acc[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
#pragma unroll
      for (int k = 0; k < kMaxK; ++k) {
        if (k < K) {
          const uint32_t q[4] = {v[u][k].x, v[u][k].y, v[u][k].z, v[u][k].w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            acc[2 * i] = acc[2 * i] + wk[k] * __uint_as_float(q[i] << 16);
            acc[2 * i + 1] = acc[2 * i + 1] + wk[k] * __uint_as_float(q[i] & 0xffff0000u);
          }
        }
      }
      v4u ov;
      ov.x = bf16_pack2(acc[0], acc[1]);
      ov.y = bf16_pack2(acc[2], acc[3]);
      ov.z = bf16_pack2(acc[4], acc[5]);
      ov.w = bf16_pack2(acc[6], acc[7]);
      __builtin_nontemporal_store(ov, (v4u*)(out + (size_t)t * H + col));
    }
  }
}

// One 512-column chunk per iteration with non-temporal loads: the gathered
// rows are read exactly once (measured 5.3 TB/s vs 4.8 TB/s with cached loads
// at the config-2 size; two chunks per iteration gave no further gain).
constexpr int kCombineU = 1;
constexpr bool kCombineNT = true;

}  // namespace smoe

using namespace smoe;

extern "C" int smoe_unpermute_combine(const uint16_t* y, const int32_t* inv_map, const float* w,
                                      int T, int K, int H, uint16_t* out, void* stream) {
  if (T <= 0 || H <= 0) return SMOE_EINVAL_DIM;
  if (H % kLane) return SMOE_EINVAL_ALIGN128;  // whole 16-byte lane pieces
  if (K <= 0 || K > 32) return SMOE_EINVAL_TOPK;
  if ((long long)T * K > 0x7fffffffLL) return SMOE_EINVAL_DIM;
  SMOE_CHECK_PTR(y);
  SMOE_CHECK_PTR(out);
  if (!inv_map || !w) return SMOE_EINVAL_NULL;
  if (((uintptr_t)inv_map | (uintptr_t)w) & 3u) return SMOE_EINVAL_PTRALIGN;
  const dim3 grid((T + 3) / 4), block(256);
  hipStream_t s = (hipStream_t)stream;
#define SMOE_CB(MK) combine_kernel<MK, kCombineU, kCombineNT><<<grid, block, 0, s>>>(y, inv_map, w, T, K, H, out)
  if (K <= 1) SMOE_CB(1);
  else if (K <= 2) SMOE_CB(2);
  else if (K <= 4) SMOE_CB(4);
  else if (K <= 8) SMOE_CB(8);
  else if (K <= 16) SMOE_CB(16);
  else SMOE_CB(32);
#undef SMOE_CB
  SMOE_RETURN_LAUNCH();
}
