// smoe_probe.hip — HBM traffic-mix probe (gfx950), a measurement utility.
//
// Reads n_in bytes once and writes every 16-byte piece it reads to
// `fanout` places of dst (fanout x n_in bytes written), with the access
// pattern of permute_quant: one wave per 1 KiB-wide slab per iteration,
// 128-bit loads, 128-bit non-temporal stores, the fanout copies of a slab
// `stride_out` bytes apart.  fanout = 0 only reads (the loaded words are
// folded into one word per wave so the loads are not dead); fanout >= 1
// with n_in = 0 is not allowed.  It moves the bytes of a dispatch step at a
// chosen read:write ratio without the quantisation, so its rate is the
// ceiling the HBM offers that mix.
#include "smoe_common.h"

namespace smoe {

typedef uint32_t v4u __attribute__((ext_vector_type(4)));

constexpr int kProbeU = 4;  // 16-byte loads in flight per lane

__global__ __launch_bounds__(256) void bw_probe_kernel(const uint4* __restrict__ src,
                                                       uint64_t n16, int fanout,
                                                       uint64_t stride16,
                                                       uint4* __restrict__ dst,
                                                       uint32_t* __restrict__ sink) {
  const uint64_t nthreads = (uint64_t)gridDim.x * blockDim.x;
  uint32_t acc = 0;
  for (uint64_t i0 = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i0 < n16;
       i0 += nthreads * kProbeU) {
    uint4 v[kProbeU];
#pragma unroll
    for (int u = 0; u < kProbeU; ++u) {
      const uint64_t i = i0 + u * nthreads;
      v[u] = i < n16 ? src[i] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < kProbeU; ++u) {
      const uint64_t i = i0 + u * nthreads;
      if (i >= n16) break;
      if (fanout == 0) {
        acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
      } else {
        const v4u o = {v[u].x, v[u].y, v[u].z, v[u].w};
        for (int f = 0; f < fanout; ++f)
          __builtin_nontemporal_store(o, (v4u*)(dst + f * stride16 + i));
      }
    }
  }
  if (fanout == 0 && acc == 0x9e3779b9u) sink[0] = acc;  // keeps the loads live
}

}  // namespace smoe

using namespace smoe;

extern "C" int smoe_bw_probe(const void* src, size_t n_in, int fanout, void* dst,
                             size_t dst_bytes, void* sink, void* stream) {
  if (n_in == 0 || (n_in & 15u) || fanout < 0 || fanout > 64) return SMOE_EINVAL_DIM;
  SMOE_CHECK_PTR(src);
  if (fanout > 0) {
    SMOE_CHECK_PTR(dst);
    if (dst_bytes < n_in * (size_t)fanout) return SMOE_EINVAL_WORKSPACE;
  }
  if (!sink) return SMOE_EINVAL_NULL;
  const uint64_t n16 = n_in / 16;
  // a persistent grid: 16 waves per CU on 256 CUs, each thread striding
  const dim3 grid(256 * 16 / 4), block(256);
  bw_probe_kernel<<<grid, block, 0, (hipStream_t)stream>>>((const uint4*)src, n16, fanout, n16,
                                                           (uint4*)dst, (uint32_t*)sink);
  SMOE_RETURN_LAUNCH();
}
