// smoe_quant.hip — fused permute + 1x128 fp8 quantisation, SwiGLU + requant,
// and 128x128 blockwise weight quantisation (gfx950).
//
// Row kernels (permute_quant, swiglu_quant) give one wave to one row.  A lane
// owns 16 consecutive elements, so 8 lanes cover one 128-element group and
// the group amax is a 3-step xor reduction inside those 8 lanes.  A wave
// walks the row 8 groups (1024 elements) at a time; up to kUnroll such chunks
// are loaded with 128-bit loads before any arithmetic so that every lane has
// kUnroll*32 bytes in flight.  Each lane writes its 16 fp8 bytes as one
// 128-bit store, and the first lane of each group writes the group's scale.
//
// A row of H bf16 values whose H is not a multiple of 128 (H % 16 == 0) is
// quantised as the row zero-padded to Hp = pad128(H): lanes past H load
// nothing (a clamped address, zeroed), take part in the group amax as zeros
// and write zero bytes, so the fp8 row has pitch Hp and its last group's
// scale is set by its valid elements.
//
// permute_quant reads a token row once and writes the same bytes to the K
// sorted rows inv_map[t*K + k]: the algorithmic minimum of one read of x and
// K writes of the fp8 row.  Rows of up to 8192 elements use the whole-row
// kernel: all of the row's chunks are loaded before any arithmetic, and each
// destination row is then written front to back.
#include "smoe_common.h"

namespace smoe {

typedef uint32_t v4u __attribute__((ext_vector_type(4)));

// 128-bit store; kNT marks it non-temporal (streamed past the caches)
template <bool kNT>
__device__ __forceinline__ void store16(uint8_t* p, const uint4& q) {
  if constexpr (kNT) {
    v4u v = {q.x, q.y, q.z, q.w};
    __builtin_nontemporal_store(v, (v4u*)p);
  } else {
    *(uint4*)p = q;
  }
}

template <int kUnroll, bool kNT, bool kPow2 = false>
__global__ __launch_bounds__(256) void permute_quant_kernel(
    const uint16_t* __restrict__ x, const int32_t* __restrict__ inv_map, int T, int H, int K,
    uint8_t* __restrict__ xq, float* __restrict__ xs) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int Hp = pad128(H);
  const int G = Hp / kGroup;
  const int R = T * K;
  const int sub = lane & 7, gl = lane >> 3;
  // destination rows: lane k holds inv_map[t*K + k]
  // inv_map == nullptr (K == 1): rows stay in place (plain 1x128 row quant)
  const int my_r = inv_map ? (lane < K ? inv_map[(size_t)t * K + lane] : 0) : t;
  const uint16_t* xrow = x + (size_t)t * H;
  for (int c0 = 0; c0 * 8 < G; c0 += kUnroll) {
    uint4 v[kUnroll][2];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int g = (c0 + u) * 8 + gl;
      const int col = g * kGroup + sub * kLane;
      if (g < G && col < H) {
        const uint4* src = (const uint4*)(xrow + col);
        v[u][0] = src[0];
        v[u][1] = src[1];
      } else {
        v[u][0] = v[u][1] = make_uint4(0, 0, 0, 0);
      }
    }
    Q16 q[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      float f[16];
      unpack_bf16x8(v[u][0], f);
      unpack_bf16x8(v[u][1], f + 8);
      q[u] = quant16_bf16<kPow2>(f);
    }
    for (int k = 0; k < K; ++k) {
      const int r = __shfl(my_r, k, kWave);
      if ((unsigned)r >= (unsigned)R) continue;  // malformed map: never write out of range
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int g = (c0 + u) * 8 + gl;
        if (g < G) {
          store16<kNT>(xq + (size_t)r * Hp + g * kGroup + sub * kLane, q[u].q);
          if (sub == 0) xs[(size_t)r * G + g] = q[u].scale;
        }
      }
    }
  }
}

// Whole-row variant for rows of at most 8 chunks (H <= 8192): a token's row
// is split over kW waves, wave j taking chunks j*kC .. j*kC + kC - 1.  Every
// chunk a wave owns is loaded before any arithmetic, and its part of each
// destination row is then written front to back (kC 1 KiB pieces
// consecutively) before the next.  kW = 2 halves the registers a wave holds
// (88 VGPRs for 4 chunks against 156 for 7 chunks in one wave), so 5 waves
// per SIMD instead of 3 keep loads in flight.
template <int kC, int kW, bool kNT, bool kPow2 = false>
__global__ __launch_bounds__(256) void permute_quant_row_kernel(
    const uint16_t* __restrict__ x, const int32_t* __restrict__ inv_map, int T, int H, int K,
    uint8_t* __restrict__ xq, float* __restrict__ xs) {
  const int lane = threadIdx.x & 63;
  const unsigned wv = blockIdx.x * 4u + (threadIdx.x >> 6);
  const int t = (int)(wv / kW), c0 = (int)(wv % kW) * kC;
  if (t >= T) return;
  const int Hp = pad128(H);
  const int G = Hp / kGroup;
  const int R = T * K;
  const int sub = lane & 7, gl = lane >> 3;
  const int my_r = lane < K ? inv_map[(size_t)t * K + lane] : 0;
  const uint16_t* xrow = x + (size_t)t * H;
  uint4 v[kC][2];
#pragma unroll
  for (int c = 0; c < kC; ++c) {
    // unconditional: every load in flight (a lane past H re-reads column 0
    // and is zeroed below)
    const int col = min((c0 + c) * 8 + gl, G - 1) * kGroup + sub * kLane;
    const uint4* src = (const uint4*)(xrow + (col < H ? col : 0));
    v[c][0] = src[0];
    v[c][1] = src[1];
  }
  if (H != Hp) {
#pragma unroll
    for (int c = 0; c < kC; ++c)
      if (((c0 + c) * 8 + gl) * kGroup + sub * kLane >= H)
        v[c][0] = v[c][1] = make_uint4(0, 0, 0, 0);
  }
  Q16 q[kC];
#pragma unroll
  for (int c = 0; c < kC; ++c) {
    float f[16];
    unpack_bf16x8(v[c][0], f);
    unpack_bf16x8(v[c][1], f + 8);
    q[c] = quant16_bf16<kPow2>(f);
  }
  for (int k = 0; k < K; ++k) {
    const int r = __shfl(my_r, k, kWave);
    if ((unsigned)r >= (unsigned)R) continue;  // malformed map: never write out of range
#pragma unroll
    for (int c = 0; c < kC; ++c) {
      const int g = (c0 + c) * 8 + gl;
      if (g < G) {
        store16<kNT>(xq + (size_t)r * Hp + g * kGroup + sub * kLane, q[c].q);
        if (sub == 0) xs[(size_t)r * G + g] = q[c].scale;
      }
    }
  }
}

// ------------------------------------------------------------ swiglu_quant
// Work is a flat list of (row, 128-column group) slots, slot = r * G + g, so
// every 8-lane group of a wave is busy whatever I is (a row of I = 768 has 6
// groups, which a wave-per-row mapping would leave 2 of 8 lane groups idle
// on).  Wave w takes slots w * 8 * kUnroll .. +8 * kUnroll, 8 at a time; all
// kUnroll batches' loads are issued before any arithmetic.  kSaveH: also
// write h rounded to bf16 (the fc2 wgrad operand of the backward pass),
// saving a recompute from c1.
template <int kUnroll, bool kSaveH, bool kPow2 = false>
__global__ __launch_bounds__(256) void swiglu_quant_kernel(const uint16_t* __restrict__ c1,
                                                           uint32_t nslots, int I,
                                                           uint8_t* __restrict__ hq,
                                                           float* __restrict__ hs,
                                                           uint16_t* __restrict__ hb) {
  const int lane = threadIdx.x & 63;
  const int Ip = pad128(I);  // hq's pitch; columns I .. Ip of h are 0
  const uint32_t G = (uint32_t)(Ip / kGroup);
  const int sub = lane & 7, gl = lane >> 3;
  const uint32_t base = (blockIdx.x * 4u + (threadIdx.x >> 6)) * (8u * kUnroll);
  uint4 vg[kUnroll][2], vu[kUnroll][2];
  uint32_t rr[kUnroll], gg[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const uint32_t slot = base + u * 8 + gl;
    rr[u] = slot / G;
    gg[u] = slot - rr[u] * G;
    if (slot < nslots && (int)gg[u] * kGroup + sub * kLane < I) {
      const uint16_t* gate = c1 + (size_t)rr[u] * 2 * I + gg[u] * kGroup + sub * 16;
      const uint16_t* up = gate + I;
      vg[u][0] = *(const uint4*)gate;
      vg[u][1] = *(const uint4*)(gate + 8);
      vu[u][0] = *(const uint4*)up;
      vu[u][1] = *(const uint4*)(up + 8);
    } else {
      vg[u][0] = vg[u][1] = vu[u][0] = vu[u][1] = make_uint4(0, 0, 0, 0);
    }
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    float fg[16], fu[16], h[16];
    unpack_bf16x8(vg[u][0], fg);
    unpack_bf16x8(vg[u][1], fg + 8);
    unpack_bf16x8(vu[u][0], fu);
    unpack_bf16x8(vu[u][1], fu + 8);
#pragma unroll
    for (int i = 0; i < 16; ++i) h[i] = silu32(fg[i]) * fu[i];
    // the 8 lanes of a group share one slot, so the group's amax shuffle
    // never mixes slots (or a valid slot with padding)
    const Q16 q = quant16<kPow2>(h);
    if (base + u * 8 + gl < nslots) {
      const int col = (int)gg[u] * kGroup + sub * kLane;
      if (kSaveH && col < I) {
        const size_t off = (size_t)rr[u] * I + col;
        uint32_t w[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = bf16_pack2(h[2 * i], h[2 * i + 1]);
        *(uint4*)(hb + off) = make_uint4(w[0], w[1], w[2], w[3]);
        *(uint4*)(hb + off + 8) = make_uint4(w[4], w[5], w[6], w[7]);
      }
      store16<true>(hq + (size_t)rr[u] * Ip + col, q.q);
      if (sub == 0) hs[(size_t)rr[u] * G + gg[u]] = q.scale;
    }
  }
}

// ------------------------------------------------- weight 128x128 blocks
// One 256-thread workgroup per 128x128 block.  Thread t owns 8 chunks of 8
// bf16 (chunk j*256+t -> block row chunk/16, column (chunk%16)*8).  w is
// [E, N, Kd] bf16; wq is [E, N, Kp] with Kp = pad128(Kd), ws [E, NB, Kp/128]
// with NB = ceil(N/128).  Rows past N and columns past Kd of an edge block
// are zeros (not read); padding columns are written as byte 0.
template <bool kPow2 = false>
__global__ __launch_bounds__(256) void quant_weight_kernel(const uint16_t* __restrict__ w,
                                                           int N, int Kd,
                                                           uint8_t* __restrict__ wq,
                                                           float* __restrict__ ws) {
  __shared__ float wmax[4];
  const int Kp = pad128(Kd);
  const int nb = (N + kGroup - 1) / kGroup, kb = Kp / kGroup;
  const int blk = blockIdx.x;
  const int e = blk / (nb * kb);
  const int rem = blk - e * nb * kb;
  const int bn = rem / kb, bk = rem - bn * kb;
  const int r0 = bn * kGroup, k0 = bk * kGroup;
  float f[8][8];
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int ch = j * 256 + threadIdx.x;
    const int row = ch >> 4, col = (ch & 15) * 8;
    const bool ok = r0 + row < N && k0 + col < Kd;
    // unconditional load (an edge chunk re-reads the block's first element)
    const uint16_t* src = w + ((size_t)e * N + r0 + (ok ? row : 0)) * Kd + k0 + (ok ? col : 0);
    uint4 v = *(const uint4*)src;
    if (!ok) v = make_uint4(0, 0, 0, 0);
    unpack_bf16x8(v, f[j]);
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(f[j][i]));
  }
  amax = wave_max(amax);
  if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  const float s = scale_of<kPow2>(amax);
  const QDiv d = qdiv_setup_t<kPow2>(s);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int ch = j * 256 + threadIdx.x;
    const int row = ch >> 4, col = (ch & 15) * 8;
    const uint32_t lo = e4m3_pack4(quot_t<kPow2>(f[j][0], d), quot_t<kPow2>(f[j][1], d),
                                   quot_t<kPow2>(f[j][2], d), quot_t<kPow2>(f[j][3], d));
    const uint32_t hi = e4m3_pack4(quot_t<kPow2>(f[j][4], d), quot_t<kPow2>(f[j][5], d),
                                   quot_t<kPow2>(f[j][6], d), quot_t<kPow2>(f[j][7], d));
    if (r0 + row < N)
      *(uint2*)(wq + ((size_t)e * N + r0 + row) * Kp + k0 + col) = make_uint2(lo, hi);
  }
  if (threadIdx.x == 0) ws[((size_t)e * nb + bn) * kb + bk] = s;
}

// Exhaustive checks of the fast quantisation path against the reference
// rule e4m3_encode_sw(clamp(x / s)) with an IEEE division.
// (1) For every positive finite bf16 amax (blockIdx.y) and every finite bf16
// x with |x| <= amax (both signs), s = group_scale(amax): the byte of the
// division-free quotient converted by v_cvt_pk_fp8_f32.  counts[0] gets the
// mismatches, counts[1] the pairs checked.
__global__ __launch_bounds__(256) void selftest_quant_bf16_kernel(
    unsigned long long* __restrict__ counts) {
  const uint32_t abits = blockIdx.y + 1;  // 0x0001 .. 0x7f7f
  const float amax = __uint_as_float(abits << 16);
  const float s = group_scale(amax);
  const QDiv d = qdiv_setup(s);
  unsigned long long bad = 0, n = 0;
  for (uint32_t xb = blockIdx.x * blockDim.x + threadIdx.x; xb <= abits;
       xb += gridDim.x * blockDim.x) {
#pragma unroll
    for (int sg = 0; sg < 2; ++sg) {
      const float x = __uint_as_float((xb << 16) | (sg ? 0x80000000u : 0u));
      const uint32_t fast = e4m3_pack4(quot_bf16(x, d), 0.0f, 0.0f, 0.0f) & 0xffu;
      bad += quant_one(x, s) != fast;
      ++n;
    }
  }
  for (int o = 32; o > 0; o >>= 1) {
    bad += __shfl_xor(bad, o, kWave);
    n += __shfl_xor(n, o, kWave);
  }
  if ((threadIdx.x & 63) == 0) {
    atomicAdd(&counts[0], bad);
    atomicAdd(&counts[1], n);
  }
}

// (2) For every fp32 v with |v| <= 448 (both signs): the hardware conversion
// against e4m3_encode_sw.  counts[2] gets the mismatches, counts[3] the
// values checked.
__global__ __launch_bounds__(256) void selftest_e4m3_kernel(unsigned long long* __restrict__ counts) {
  const uint32_t lim = __float_as_uint(kE4M3Max);
  unsigned long long bad = 0, n = 0;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i <= lim;
       i += (uint64_t)gridDim.x * blockDim.x) {
#pragma unroll
    for (int sg = 0; sg < 2; ++sg) {
      const float v = __uint_as_float((uint32_t)i | (sg ? 0x80000000u : 0u));
      bad += e4m3_encode_sw(v) != (e4m3_pack4(v, 0.0f, 0.0f, 0.0f) & 0xffu);
      ++n;
    }
  }
  for (int o = 32; o > 0; o >>= 1) {
    bad += __shfl_xor(bad, o, kWave);
    n += __shfl_xor(n, o, kWave);
  }
  if ((threadIdx.x & 63) == 0) {
    atomicAdd(&counts[2], bad);
    atomicAdd(&counts[3], n);
  }
}

// (3) For every fp32 bit pattern: the hardware bf16 conversion (bf16_pack2)
// against f32_to_bf16, in both halves of the pair.  Non-NaN values must give
// the same bits; a NaN must stay a NaN of the same sign.  counts[4] gets the
// mismatches, counts[5] the values checked.
__device__ __forceinline__ bool bf16_same(float v, uint32_t hw) {
  const uint32_t sw = f32_to_bf16(v);
  if (v != v) return (hw & 0x7fffu) > 0x7f80u && (hw & 0x8000u) == (sw & 0x8000u);
  return hw == sw;
}
__global__ __launch_bounds__(256) void selftest_bf16_kernel(unsigned long long* __restrict__ counts) {
  unsigned long long bad = 0, n = 0;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i <= 0xffffffffull;
       i += (uint64_t)gridDim.x * blockDim.x) {
    const float v = __uint_as_float((uint32_t)i);
    // partner for the other half: a different pattern on every lane
    const float w = __uint_as_float((uint32_t)i ^ 0x9e3779b9u);
    const uint32_t p = bf16_pack2(v, w);
    bad += !bf16_same(v, p & 0xffffu);
    bad += !bf16_same(w, p >> 16);
    n += 2;
  }
  for (int o = 32; o > 0; o >>= 1) {
    bad += __shfl_xor(bad, o, kWave);
    n += __shfl_xor(n, o, kWave);
  }
  if ((threadIdx.x & 63) == 0) {
    atomicAdd(&counts[4], bad);
    atomicAdd(&counts[5], n);
  }
}

// recip_rn against the IEEE quotient 1.0f / b for every fp32 b in
// [2^-126, 2^126) (exponent fields 1..252, every significand), and for +inf.
// counts[0] gets the mismatches, counts[1] the values checked.
__global__ __launch_bounds__(256) void selftest_recip_kernel(unsigned long long* __restrict__ counts) {
  constexpr uint64_t kFirst = 1ull << 23, kEnd = 253ull << 23;  // bit patterns
  unsigned long long bad = 0, n = 0;
  for (uint64_t i = kFirst + (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < kEnd;
       i += (uint64_t)gridDim.x * blockDim.x) {
    const float b = __uint_as_float((uint32_t)i);
    bad += __float_as_uint(recip_rn(b)) != __float_as_uint(1.0f / b);
    ++n;
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    const float inf = __builtin_inff();
    bad += __float_as_uint(recip_rn(inf)) != __float_as_uint(1.0f / inf);
    ++n;
  }
  for (int o = 32; o > 0; o >>= 1) {
    bad += __shfl_xor(bad, o, kWave);
    n += __shfl_xor(n, o, kWave);
  }
  if ((threadIdx.x & 63) == 0) {
    atomicAdd(&counts[0], bad);
    atomicAdd(&counts[1], n);
  }
}

}  // namespace smoe

using namespace smoe;

extern "C" int smoe_selftest_quant(unsigned long long* counts, void* stream) {
  if (!counts) return SMOE_EINVAL_NULL;
  if ((uintptr_t)counts & 7u) return SMOE_EINVAL_PTRALIGN;
  hipStream_t st = (hipStream_t)stream;
  selftest_quant_bf16_kernel<<<dim3(64, 0x7f7f), dim3(256), 0, st>>>(counts);
  selftest_e4m3_kernel<<<dim3(4096), dim3(256), 0, st>>>(counts);
  selftest_bf16_kernel<<<dim3(8192), dim3(256), 0, st>>>(counts);
  SMOE_RETURN_LAUNCH();
}

extern "C" int smoe_selftest_recip(unsigned long long* counts, void* stream) {
  if (!counts) return SMOE_EINVAL_NULL;
  if ((uintptr_t)counts & 7u) return SMOE_EINVAL_PTRALIGN;
  selftest_recip_kernel<<<dim3(8192), dim3(256), 0, (hipStream_t)stream>>>(counts);
  SMOE_RETURN_LAUNCH();
}

namespace {
template <bool kPow2>
int permute_quant_launch(const uint16_t* x, const int32_t* inv_map, int T, int H, int K,
                         uint8_t* xq, float* xs, hipStream_t s) {
  const int chunks = (pad128(H) / kGroup + 7) / 8;
  // Rows of up to 8 chunks (H <= 8192): the whole-row kernel with cached
  // stores, rows of 5..8 chunks split over two waves.  Measured with cold
  // caches at config 2 (T=16384, H=7168, top-8) on one box: 0.214 ms for
  // 4 chunks x 2 waves against 0.222 ms for 7 chunks in one wave and
  // 0.214 ms for 2 chunks x 4 waves.  On another box, where one wave per
  // row took 212 us, its non-temporal stores took 229 us and the
  // chunk-interleaved kernel below 232 us.
#define SMOE_PR(C, W) \
  permute_quant_row_kernel<C, W, false, kPow2><<<dim3((unsigned)(((long long)T * W + 3) / 4)), dim3(256), 0, s>>>( \
      x, inv_map, T, H, K, xq, xs)
  if (chunks <= 8) {
    switch (chunks) {
      case 1: SMOE_PR(1, 1); break; case 2: SMOE_PR(2, 1); break; case 3: SMOE_PR(3, 1); break;
      case 4: SMOE_PR(4, 1); break; case 5: SMOE_PR(3, 2); break; case 6: SMOE_PR(3, 2); break;
      default: SMOE_PR(4, 2); break;
    }
    SMOE_RETURN_LAUNCH();
  }
#undef SMOE_PR
  // longer rows: kUnroll = 4 chunks (128 B per lane) in flight keeps 2+
  // waves per SIMD
  permute_quant_kernel<4, true, kPow2><<<dim3((unsigned)(((long long)T + 3) / 4)), dim3(256), 0, s>>>(
      x, inv_map, T, H, K, xq, xs);
  SMOE_RETURN_LAUNCH();
}

template <bool kPow2>
int quant_rows_launch(const uint16_t* x, int M, int C, uint8_t* q, float* s, hipStream_t st) {
  const int chunks = (pad128(C) / kGroup + 7) / 8;
  const dim3 grid((M + 3) / 4), block(256);
#define SMOE_QR(U) permute_quant_kernel<U, true, kPow2><<<grid, block, 0, st>>>(x, nullptr, M, C, 1, q, s)
  switch (chunks) {
    case 1: SMOE_QR(1); break;
    case 2: SMOE_QR(2); break;
    case 3: SMOE_QR(3); break;
    default: SMOE_QR(4); break;
  }
#undef SMOE_QR
  SMOE_RETURN_LAUNCH();
}
}  // namespace

extern "C" int smoe_permute_quant_ex(const uint16_t* x, const int32_t* inv_map, int T, int H,
                                     int K, uint8_t* xq, float* xs, int scale_mode,
                                     void* stream) {
  if (T <= 0 || H <= 0) return SMOE_EINVAL_DIM;
  if (H % kLane) return SMOE_EINVAL_ALIGN128;
  if (K <= 0 || K > 32) return SMOE_EINVAL_TOPK;
  if ((long long)T * K > 0x7fffffffLL) return SMOE_EINVAL_DIM;
  if (scale_mode != SMOE_SCALE_AMAX && scale_mode != SMOE_SCALE_POW2) return SMOE_EINVAL_MODE;
  SMOE_CHECK_PTR(x);
  SMOE_CHECK_PTR(inv_map);
  SMOE_CHECK_PTR(xq);
  SMOE_CHECK_PTR(xs);
  hipStream_t s = (hipStream_t)stream;
  return scale_mode == SMOE_SCALE_POW2 ? permute_quant_launch<true>(x, inv_map, T, H, K, xq, xs, s)
                                       : permute_quant_launch<false>(x, inv_map, T, H, K, xq, xs, s);
}

extern "C" int smoe_permute_quant(const uint16_t* x, const int32_t* inv_map, int T, int H, int K,
                                  uint8_t* xq, float* xs, void* stream) {
  return smoe_permute_quant_ex(x, inv_map, T, H, K, xq, xs, SMOE_SCALE_AMAX, stream);
}

extern "C" int smoe_quant_rows_1x128_ex(const uint16_t* x, int M, int C, uint8_t* q, float* s,
                                        int scale_mode, void* stream) {
  if (M <= 0 || C <= 0) return SMOE_EINVAL_DIM;
  if (C % kLane) return SMOE_EINVAL_ALIGN128;
  if (scale_mode != SMOE_SCALE_AMAX && scale_mode != SMOE_SCALE_POW2) return SMOE_EINVAL_MODE;
  SMOE_CHECK_PTR(x);
  SMOE_CHECK_PTR(q);
  SMOE_CHECK_PTR(s);
  hipStream_t st = (hipStream_t)stream;
  return scale_mode == SMOE_SCALE_POW2 ? quant_rows_launch<true>(x, M, C, q, s, st)
                                       : quant_rows_launch<false>(x, M, C, q, s, st);
}

extern "C" int smoe_quant_rows_1x128(const uint16_t* x, int M, int C, uint8_t* q, float* s,
                                     void* stream) {
  return smoe_quant_rows_1x128_ex(x, M, C, q, s, SMOE_SCALE_AMAX, stream);
}

extern "C" int smoe_dispatch_quant(const uint16_t* x, const int32_t* topk_idx, int T, int H,
                                   int K, int E, int32_t* row_map, int32_t* inv_map,
                                   int32_t* counts, int32_t* offsets, uint8_t* xq, float* xs,
                                   void* ws, size_t ws_bytes, void* stream) {
  if (T <= 0 || H <= 0) return SMOE_EINVAL_DIM;
  if (H % kLane) return SMOE_EINVAL_ALIGN128;
  SMOE_CHECK_PTR(x);
  SMOE_CHECK_PTR(xq);
  SMOE_CHECK_PTR(xs);
  int st = smoe_route_sort(topk_idx, T, K, E, row_map, inv_map, counts, offsets, ws, ws_bytes,
                           stream);
  if (st) return st;
  return smoe_permute_quant(x, inv_map, T, H, K, xq, xs, stream);
}

extern "C" int smoe_swiglu_quant_ex(const uint16_t* c1, int R, int I, uint8_t* hq, float* hs,
                                    uint16_t* h, int scale_mode, void* stream) {
  if (R <= 0 || I <= 0) return SMOE_EINVAL_DIM;
  if (I % kLane) return SMOE_EINVAL_ALIGN128;
  if (scale_mode != SMOE_SCALE_AMAX && scale_mode != SMOE_SCALE_POW2) return SMOE_EINVAL_MODE;
  SMOE_CHECK_PTR(c1);
  SMOE_CHECK_PTR(hq);
  SMOE_CHECK_PTR(hs);
  if (h && ((uintptr_t)h & 15u)) return SMOE_EINVAL_PTRALIGN;
  // slots (row, group) are 32-bit; the grid covers them 32 * kUnroll per block
  const long long nslots = (long long)R * (pad128(I) / kGroup);
  constexpr int kU = 2;
  if (nslots + 32LL * kU > 0xffffffffLL) return SMOE_EINVAL_DIM;
  const dim3 grid((unsigned)((nslots + 32 * kU - 1) / (32 * kU))), block(256);
  hipStream_t s = (hipStream_t)stream;
#define SMOE_SQ(H, P) \
  swiglu_quant_kernel<kU, H, P><<<grid, block, 0, s>>>(c1, (uint32_t)nslots, I, hq, hs, H ? h : nullptr)
  const bool p2 = scale_mode == SMOE_SCALE_POW2;
  if (h) { if (p2) SMOE_SQ(true, true); else SMOE_SQ(true, false); }
  else { if (p2) SMOE_SQ(false, true); else SMOE_SQ(false, false); }
#undef SMOE_SQ
  SMOE_RETURN_LAUNCH();
}

extern "C" int smoe_swiglu_quant_h(const uint16_t* c1, int R, int I, uint8_t* hq, float* hs,
                                   uint16_t* h, void* stream) {
  return smoe_swiglu_quant_ex(c1, R, I, hq, hs, h, SMOE_SCALE_AMAX, stream);
}

extern "C" int smoe_swiglu_quant(const uint16_t* c1, int R, int I, uint8_t* hq, float* hs,
                                 void* stream) {
  return smoe_swiglu_quant_ex(c1, R, I, hq, hs, nullptr, SMOE_SCALE_AMAX, stream);
}

extern "C" int smoe_quantize_weight_blockwise_ex(const uint16_t* w, int E, int N, int Kdim,
                                                 uint8_t* wq, float* ws, int scale_mode,
                                                 void* stream) {
  if (N <= 0 || Kdim <= 0) return SMOE_EINVAL_DIM;
  if (E <= 0 || E > SMOE_MAX_EXPERTS) return SMOE_EINVAL_EXPERTS;
  if (N % kLane || Kdim % kLane) return SMOE_EINVAL_ALIGN128;
  if (scale_mode != SMOE_SCALE_AMAX && scale_mode != SMOE_SCALE_POW2) return SMOE_EINVAL_MODE;
  SMOE_CHECK_PTR(w);
  SMOE_CHECK_PTR(wq);
  SMOE_CHECK_PTR(ws);
  const long long blocks = (long long)E * ((N + kGroup - 1) / kGroup) * (pad128(Kdim) / kGroup);
  if (blocks > 0x7fffffffLL) return SMOE_EINVAL_DIM;
  const dim3 grid((unsigned)blocks), block(256);
  hipStream_t s = (hipStream_t)stream;
  if (scale_mode == SMOE_SCALE_POW2)
    quant_weight_kernel<true><<<grid, block, 0, s>>>(w, N, Kdim, wq, ws);
  else
    quant_weight_kernel<false><<<grid, block, 0, s>>>(w, N, Kdim, wq, ws);
  SMOE_RETURN_LAUNCH();
}

extern "C" int smoe_quantize_weight_blockwise(const uint16_t* w, int E, int N, int Kdim,
                                              uint8_t* wq, float* ws, void* stream) {
  return smoe_quantize_weight_blockwise_ex(w, E, N, Kdim, wq, ws, SMOE_SCALE_AMAX, stream);
}
