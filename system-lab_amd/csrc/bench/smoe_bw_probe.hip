// smoe_bw_probe.hip — HBM traffic-mix probe (gfx950), a measurement utility
// for the benchmark only: it is built into its own library,
// libsmoe_probe.so, and is not part of libsmoe.so or its header.
//
//   int smoe_bw_probe(const void* src, int rows, int row_bytes, int fanout,
//                     void* dst, size_t dst_bytes, void* sink, void* stream);
//
// returns 0 or a negative SMOE_EINVAL_* code (row_bytes a multiple of 2048,
// at most 16384; dst must hold rows * fanout * row_bytes / 2 bytes; sink is
// one device word).
//
// The access pattern of permute_quant without its arithmetic: a source row of
// row_bytes (<= 16 KiB) bytes is split over the same number of waves as in
// permute_quant (two for rows of more than 4 chunks of 2 KiB, else one);
// each lane loads 32 bytes (two 128-bit loads) per 2 KiB chunk its wave
// owns, all of them in flight, and writes one 16-byte word derived from them
// (their xor, standing in for the fp8 bytes of 32 bf16 bytes) to each of
// `fanout` destination rows of row_bytes / 2 bytes, its part of each row
// front to back, with cached 128-bit stores.  Destination row of (row t, copy
// k) is (t*fanout + k) * 0x9E3779B1 mod (rows*fanout) when rows*fanout is a
// power of two (a scatter like the expert-sorted rows), t*fanout + k
// otherwise.  fanout = 0 only reads.  Bytes moved: rows*row_bytes read,
// rows*fanout*row_bytes/2 written; fanout 8 is the dispatch step's 1:4 mix.
// Its rate is the ceiling the HBM offers that mix to this access pattern.
#include "../smoe_common.h"

namespace smoe {

typedef uint32_t v4u __attribute__((ext_vector_type(4)));

constexpr int kProbeMaxC = 8;  // 2 KiB chunks per row, all in flight

// The whole-row permute_quant pattern: wave j of a row's kW waves loads
// chunks j*kC .. j*kC + kC - 1 before any store, then writes its part of each
// destination row front to back.
template <int kC, int kW>
__global__ __launch_bounds__(256) void bw_probe_kernel(const uint8_t* __restrict__ src, int rows,
                                                       int row_bytes, int fanout,
                                                       uint8_t* __restrict__ dst,
                                                       uint32_t* __restrict__ sink) {
  const int lane = threadIdx.x & 63;
  const unsigned wv = blockIdx.x * 4u + (threadIdx.x >> 6);
  const int t = (int)(wv / kW), c0 = (int)(wv % kW) * kC;
  if (t >= rows) return;
  const int out_bytes = row_bytes / 2;
  const uint32_t nrows_out = (uint32_t)rows * (uint32_t)max(fanout, 1);
  const bool pow2 = (nrows_out & (nrows_out - 1)) == 0;
  const uint8_t* srow = src + (size_t)t * row_bytes;
  uint4 w[kC];
#pragma unroll
  for (int c = 0; c < kC; ++c) {
    const int off = min((c0 + c) * 2048 + lane * 32, row_bytes - 32);
    const uint4 a = *(const uint4*)(srow + off);
    const uint4 b = *(const uint4*)(srow + off + 16);
    w[c] = make_uint4(a.x ^ b.x, a.y ^ b.y, a.z ^ b.z, a.w ^ b.w);
  }
  if (fanout == 0) {
    uint32_t acc = 0;
#pragma unroll
    for (int c = 0; c < kC; ++c) acc ^= w[c].x ^ w[c].y ^ w[c].z ^ w[c].w;
    if (acc == 0x9e3779b9u) sink[0] = acc;  // keeps the loads live
    return;
  }
  for (int k = 0; k < fanout; ++k) {
    uint32_t d = (uint32_t)t * (uint32_t)fanout + (uint32_t)k;
    if (pow2) d = (d * 0x9E3779B1u) & (nrows_out - 1);
    uint8_t* drow = dst + (size_t)d * out_bytes;
#pragma unroll
    for (int c = 0; c < kC; ++c) {
      const int off = (c0 + c) * 2048 + lane * 32;
      if (off < row_bytes) *(uint4*)(drow + off / 2) = w[c];
    }
  }
}

}  // namespace smoe

using namespace smoe;

extern "C" int smoe_bw_probe(const void* src, int rows, int row_bytes, int fanout, void* dst,
                             size_t dst_bytes, void* sink, void* stream) {
  if (rows <= 0 || row_bytes <= 0 || row_bytes % 2048 || fanout < 0 || fanout > 32)
    return SMOE_EINVAL_DIM;
  if (row_bytes > 2048 * kProbeMaxC) return SMOE_EINVAL_DIM;
  SMOE_CHECK_PTR(src);
  if (fanout > 0) {
    SMOE_CHECK_PTR(dst);
    if (dst_bytes < (size_t)rows * fanout * (row_bytes / 2)) return SMOE_EINVAL_WORKSPACE;
  }
  if (!sink) return SMOE_EINVAL_NULL;
  hipStream_t s = (hipStream_t)stream;
#define SMOE_BP(C, W)                                                                              \
  bw_probe_kernel<C, W><<<dim3((unsigned)(((long long)rows * W + 3) / 4)), dim3(256), 0, s>>>( \
      (const uint8_t*)src, rows, row_bytes, fanout, (uint8_t*)dst, (uint32_t*)sink)
  switch (row_bytes / 2048) {
    case 1: SMOE_BP(1, 1); break; case 2: SMOE_BP(2, 1); break; case 3: SMOE_BP(3, 1); break;
    case 4: SMOE_BP(4, 1); break; case 5: SMOE_BP(3, 2); break; case 6: SMOE_BP(3, 2); break;
    default: SMOE_BP(4, 2); break;
  }
#undef SMOE_BP
  SMOE_RETURN_LAUNCH();
}
