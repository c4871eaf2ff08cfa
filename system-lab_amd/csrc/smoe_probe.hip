// smoe_probe.hip — HBM traffic-mix probe (gfx950), a measurement utility.
//
// The access pattern of permute_quant without its arithmetic: one wave per
// source row of row_bytes bytes; each lane loads 32 bytes (two 128-bit
// loads) per 2 KiB of the row, four such chunks in flight, and writes one
// 16-byte word derived from them (their xor, standing in for the fp8 bytes
// of 32 bf16 bytes) to each of `fanout` destination rows of row_bytes / 2
// bytes with non-temporal 128-bit stores.  Destination row of (row t, copy
// k) is (t*fanout + k) * 0x9E3779B1 mod (rows*fanout) when rows*fanout is a
// power of two (a scatter like the expert-sorted rows), t*fanout + k
// otherwise.  fanout = 0 only reads.  Bytes moved: rows*row_bytes read,
// rows*fanout*row_bytes/2 written; fanout 8 is the dispatch step's 1:4 mix.
// Its rate is the ceiling the HBM offers that mix to this access pattern.
#include "smoe_common.h"

namespace smoe {

typedef uint32_t v4u __attribute__((ext_vector_type(4)));

constexpr int kProbeU = 4;  // 2 KiB chunks in flight per wave

__global__ __launch_bounds__(256) void bw_probe_kernel(const uint8_t* __restrict__ src, int rows,
                                                       int row_bytes, int fanout,
                                                       uint8_t* __restrict__ dst,
                                                       uint32_t* __restrict__ sink) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= rows) return;
  const int out_bytes = row_bytes / 2;
  const uint32_t nrows_out = (uint32_t)rows * (uint32_t)max(fanout, 1);
  const bool pow2 = (nrows_out & (nrows_out - 1)) == 0;
  const uint8_t* srow = src + (size_t)t * row_bytes;
  uint32_t acc = 0;
  for (int c0 = 0; c0 * 2048 < row_bytes; c0 += kProbeU) {
    uint4 v[kProbeU][2];
#pragma unroll
    for (int u = 0; u < kProbeU; ++u) {
      const int off = (c0 + u) * 2048 + lane * 32;
      if (off < row_bytes) {
        v[u][0] = *(const uint4*)(srow + off);
        v[u][1] = *(const uint4*)(srow + off + 16);
      } else {
        v[u][0] = v[u][1] = make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int u = 0; u < kProbeU; ++u) {
      const int off = (c0 + u) * 2048 + lane * 32;
      const v4u w = {v[u][0].x ^ v[u][1].x, v[u][0].y ^ v[u][1].y, v[u][0].z ^ v[u][1].z,
                     v[u][0].w ^ v[u][1].w};
      if (fanout == 0) {
        acc ^= w.x ^ w.y ^ w.z ^ w.w;
      } else if (off < row_bytes) {
        for (int k = 0; k < fanout; ++k) {
          uint32_t d = (uint32_t)t * (uint32_t)fanout + (uint32_t)k;
          if (pow2) d = (d * 0x9E3779B1u) & (nrows_out - 1);
          __builtin_nontemporal_store(w, (v4u*)(dst + (size_t)d * out_bytes + off / 2));
        }
      }
    }
  }
  if (fanout == 0 && acc == 0x9e3779b9u) sink[0] = acc;  // keeps the loads live
}

}  // namespace smoe

using namespace smoe;

extern "C" int smoe_bw_probe(const void* src, int rows, int row_bytes, int fanout, void* dst,
                             size_t dst_bytes, void* sink, void* stream) {
  if (rows <= 0 || row_bytes <= 0 || row_bytes % 2048 || fanout < 0 || fanout > 32)
    return SMOE_EINVAL_DIM;
  SMOE_CHECK_PTR(src);
  if (fanout > 0) {
    SMOE_CHECK_PTR(dst);
    if (dst_bytes < (size_t)rows * fanout * (row_bytes / 2)) return SMOE_EINVAL_WORKSPACE;
  }
  if (!sink) return SMOE_EINVAL_NULL;
  bw_probe_kernel<<<dim3((rows + 3) / 4), dim3(256), 0, (hipStream_t)stream>>>(
      (const uint8_t*)src, rows, row_bytes, fanout, (uint8_t*)dst, (uint32_t*)sink);
  SMOE_RETURN_LAUNCH();
}
