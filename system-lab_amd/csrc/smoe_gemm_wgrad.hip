// smoe_gemm_wgrad.hip — variable-K fp8 grouped GEMM for the weight gradient
// of the expert FFN (gfx950):
//
//   dW[e][n][k] = sum_g sa[n,g] * sb[k,g] * sum_{r in g} aT[n,r] * bT[k,r]
//
// over expert e's 128-row groups g in [pad[e], pad[e+1]) of the transposed,
// 128x1-quantised operands aT [N, ld] (e.g. output grads) and bT [K, ld]
// (e.g. activations), both with the reduction index r contiguous.  Output is
// [E, N, K], fp32 or bf16, written (experts without rows get zeros) or added
// into the buffer's contents.
//
// A workgroup of 8 waves owns a 256 (n) x 256 (k) tile of one expert; each
// wave owns 64 n x 128 k, i.e. 4 x 8 blocks of v_mfma_f32_16x16x128_f8f6f4,
// one MFMA per 128-row group.  bT rows feed the MFMA's A operand and aT rows
// its B operand, so an output lane holds one n (lane % 16) and four
// consecutive k, which leave for LDS as one 16-byte write.
// Both scales vary per row and group, so each partial is multiplied by
// sa[n,g]*sb[k,g] before accumulation (the product is formed before the
// MFMA result arrives, leaving one FMA per output after it).  Operands are
// staged by direct global->LDS DMA, two stages deep, as in the forward
// grouped GEMM; both scale vectors are staged 8 row groups at a time.
#include "smoe_mfma.h"

#include <algorithm>
#include <atomic>

namespace smoe {

// Tile: 256 (n, aT rows) x 256 (k, bT rows) per workgroup of 8 waves in a
// 2 (k) x 4 (n) grid; each wave owns 128 k x 64 n = 8 x 4 blocks of the
// 16x16 MFMA.  Stage = aT tile | bT tile.
constexpr int kWN = 256, kWK = 256;
constexpr int kWThreads = 512;
constexpr int kWA = kWN * kRow;  // 32 KiB of aT
constexpr int kWB = kWK * kRow;  // 32 KiB of bT
constexpr int kWStage = kWA + kWB;
// Both operands' 128x1 scales are staged kWChunk row groups at a time:
// [kWN + kWK rows][kWChunk] fp32 per chunk, double-buffered after the stages.
constexpr int kWChunk = 8;
constexpr int kWSC = (kWN + kWK) * kWChunk * 4;  // 16 KiB per chunk
constexpr int kWSmem = 2 * kWStage + 2 * kWSC;
static_assert(kWSmem <= 160 * 1024, "LDS budget");

// Output modes of the weight gradient (SMOE_WGRAD_*): fp32 or
// bf16, written or added into what the buffer holds (a framework's
// gradient-accumulation buffer, "main_grad").
enum WgradOut {
  kOutF32 = SMOE_WGRAD_F32,
  kOutF32Acc = SMOE_WGRAD_F32_ACC,
  kOutBF16 = SMOE_WGRAD_BF16,
  kOutBF16Acc = SMOE_WGRAD_BF16_ACC
};

// One 256 x 256 tile of expert e's weight gradient at (n0, k0).  kE8M0: the
// operands carry power-of-two scales (the optional E8M0 column recipe).
template <int kOut, bool kE8M0>
__device__ __forceinline__ void wgrad_tile(const uint8_t* __restrict__ aT,
                                           const float* __restrict__ aTs,
                                           const uint8_t* __restrict__ bT,
                                           const float* __restrict__ bTs,
                                           const int32_t* __restrict__ pad, int N, int Kd, int ld,
                                           int e, int n0, int k0, uint8_t* smem,
                                           void* __restrict__ dW) {
  // opaque per tile: keeps lane-dependent address arithmetic inside the
  // caller's tile loop instead of live (in VGPRs) across it
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int lane = tid & 63, wid = tid >> 6;
  // operand columns outside [0, ld) are never read, whatever pad[] holds
  const int g0 = max(pad[e], 0), g1 = min(pad[e + 1], ld);
  const int steps = g1 > g0 ? (g1 - g0) / kGroup : 0;
  const int nrows = min(kWN, N - n0), krows = min(kWK, Kd - k0);
  const int sld = ld / kGroup;  // scale row length

  // DMA per wave and stage: aT segments w*4..w*4+3, bT segments w*4..w*4+3
  // (8 rows of 128 bytes each).
  // Lane offsets of segment j: row tile_row((wid*4+j)*8 + lane/8) clamped to
  // the operand's rows, chunk (lane%8) ^ (row%8).  Recomputed at each issue
  // (a few VALU operations) rather than held: the tile body needs the VGPRs.
  auto seg_off = [&](int j, int lim) {
    const int row = tile_row((wid * 4 + j) * 8 + (lane >> 3));
    return (uint32_t)(min(row, lim - 1) * ld + (((lane & 7) ^ (row & 7)) << 4));
  };
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_ptr_t)smem;
  // wave-uniform LDS destinations, computed once into scalar registers
  const uint32_t a_lds = __builtin_amdgcn_readfirstlane(lds0 + wid * 4 * 1024);
  const uint32_t b_lds = __builtin_amdgcn_readfirstlane(lds0 + kWA + wid * 4 * 1024);
  auto issue = [&](int st_idx, int buf) {
    const uint32_t st = buf * kWStage;
    const int r0 = g0 + st_idx * kGroup;
    const uint8_t* ab = aT + (size_t)n0 * ld + r0;
    const uint8_t* bb = bT + (size_t)k0 * ld + r0;
#pragma unroll
    for (int j = 0; j < 4; ++j) dma16(ab, seg_off(j, nrows), a_lds + st + j * 1024);
#pragma unroll
    for (int j = 0; j < 4; ++j) dma16(bb, seg_off(j, krows), b_lds + st + j * 1024);
  };
  // Scale chunk c (row groups g0/128 + 8c .. +8): waves 0-3 take aT rows
  // (wid&3)*64 .., waves 4-7 bT rows; instruction i moves 8 rows x 8
  // consecutive words (lane -> row i*8 + lane/8, group lane%8), so each
  // instruction touches 8 short row segments instead of 64 rows.  Columns
  // past the row end are clamped (their values are never used).
  const float* sbase = uniform_ptr(wid < 4 ? aTs + (size_t)n0 * sld : bTs + (size_t)k0 * sld);
  const int srows = wid < 4 ? nrows : krows;
  const uint32_t sc_lds =
      __builtin_amdgcn_readfirstlane(lds0 + 2 * kWStage + wid * 64 * kWChunk * 4);
  auto issue_sc = [&](int chunk) {
    const int col = min(g0 / kGroup + chunk * kWChunk + (lane & 7), sld - 1);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = min((wid & 3) * 64 + i * 8 + (lane >> 3), srows - 1);
      dma4(sbase, (uint32_t)(row * sld + col) * 4u,
           sc_lds + (chunk & 1) * kWSC + i * 8 * kWChunk * 4);
    }
  };

  const int wk = wid >> 2, wn = wid & 3;  // wave's k half and n quarter
  const int frow = lane & 15;
  const int fch = (lane >> 4) * 2;
  v4f acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

  if (steps > 0) {
    issue_sc(0);
    issue(0, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  }
  for (int st = 0; st < steps; ++st) {
    const int buf = st & 1;
    // the next scale chunk goes out at the first step of the current one,
    // into the half whose chunk was last read before the previous barrier
    if ((st & (kWChunk - 1)) == 0 && st + kWChunk < steps) issue_sc(st / kWChunk + 1);
    if (st + 1 < steps) issue(st + 1, buf ^ 1);
    const uint8_t* sA = smem + buf * kWStage;
    const uint8_t* sB = sA + kWA;
    const float* sSa = (const float*)(smem + 2 * kWStage + ((st / kWChunk) & 1) * kWSC) +
                       (st & (kWChunk - 1));
    const float* sSb = sSa + kWN * kWChunk;
    const int kr0 = wk * 128 + frow;
    if constexpr (kE8M0) {
      // Power-of-two scales (group_scale_pow2): the fp32 exponent field of
      // each scale is its E8M0 byte, and the scaled MFMA applies a row's
      // aT scale and a column's bT scale in hardware, so the 128-row groups
      // accumulate in the MFMA's own fp32 accumulator with no per-output
      // arithmetic.  The MFMA's A rows (and their scales) are indexed by
      // lane % 16, as are its B rows.
      v8i fa[4];
      int ea[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        fa[j] = lds_frag(sA, wn * 64 + j * 16 + frow, fch);
        ea[j] = (int)((__float_as_uint(sSa[(wn * 64 + j * 16 + frow) * kWChunk]) >> 23) & 0xffu);
      }
      v8i fb = lds_frag(sB, kr0, fch);
      int eb = (int)((__float_as_uint(sSb[kr0 * kWChunk]) >> 23) & 0xffu);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        v8i fbn = fb;
        int ebn = eb;
        if (i + 1 < 8) {
          fbn = lds_frag(sB, kr0 + (i + 1) * 16, fch);
          ebn = (int)((__float_as_uint(sSb[(kr0 + (i + 1) * 16) * kWChunk]) >> 23) & 0xffu);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(fb, fa[j], acc[i][j], 0, 0,
                                                                       0, eb, 0, ea[j]);
        fb = fbn;
        eb = ebn;
      }
    } else {
      v8i fa[4];
      float sa[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        fa[j] = lds_frag(sA, wn * 64 + j * 16 + frow, fch);
        sa[j] = sSa[(wn * 64 + j * 16 + frow) * kWChunk];
      }
      // the next row block's fragment and scales are read before this
      // block's MFMAs are issued, so their LDS latency hides behind them;
      // a lane's 4 outputs are 4 consecutive k, each with its own bT scale
      const int kq0 = wk * 128 + (lane >> 4) * 4;
      auto sb_of = [&](int i) {
        v4f r;
#pragma unroll
        for (int v = 0; v < 4; ++v) r[v] = sSb[(kq0 + i * 16 + v) * kWChunk];
        return r;
      };
      v8i fb = lds_frag(sB, kr0, fch);
      v4f sb = sb_of(0);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        v8i fbn = fb;
        v4f sbn = sb;
        if (i + 1 < 8) {
          fbn = lds_frag(sB, kr0 + (i + 1) * 16, fch);
          sbn = sb_of(i + 1);
        }
        // the scale products do not depend on the MFMA results: computing
        // them first leaves one FMA per output after each MFMA
        v4f sab[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) sab[j] = sa[j] * sb;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const v4f p = mfma16(fb, fa[j], v4f{0.0f, 0.0f, 0.0f, 0.0f});
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[i][j][v] = __builtin_fmaf(p[v], sab[j][v], acc[i][j][v]);
        }
        fb = fbn;
        sb = sbn;
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  }

  // An expert without rows adds nothing to an accumulation buffer.
  if ((kOut == kOutF32Acc || kOut == kOutBF16Acc) && steps == 0) return;

  // Epilogue: the fp32 tile leaves through LDS in two 128-row halves (the
  // stage buffers are free after the K loop's last barrier).  Lane (i, j)
  // holds dW row n = wn*64 + j*16 + lane%16, columns k = wk*128 + i*16 +
  // (lane/16)*4 .. +3, written as one 16-byte word; with a row pitch of 260
  // floats the 16 rows of a lane group start 4 banks apart, so each group's
  // 16-byte writes cover all 64 banks once (conflict-free).  Then each
  // wave writes whole rows, 4 columns per lane: fp32 as 16-byte stores,
  // non-temporal (dW is written once here and read by a later kernel), bf16
  // rounded to nearest even as 8-byte stores.  The accumulating modes read
  // the 4 columns first and add the tile's fp32 values to them (one fp32
  // addition per value, then the bf16 rounding for a bf16 buffer: the same
  // result as adding an fp32 gradient to the buffer in a separate pass).
  float* ct = (float*)smem;
  constexpr int kPitch = kWK + 4;
  static_assert(128 * kPitch * 4 <= kWSmem, "epilogue half-tile fits the LDS buffers");
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    if ((wn >> 1) == half) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int row = (wn & 1) * 64 + j * 16 + frow;
          *(v4f*)(ct + row * kPitch + wk * 128 + i * 16 + (lane >> 4) * 4) = acc[i][j];
        }
    }
    __syncthreads();
    for (int r = wid; r < 128; r += 8) {
      const int nl = half * 128 + r;
      if (nl < nrows && lane * 4 < krows) {
        v4f val = *(const v4f*)(ct + r * kPitch + lane * 4);
        const size_t o = ((size_t)e * N + n0 + nl) * Kd + k0 + lane * 4;
        if constexpr (kOut == kOutF32) {
          __builtin_nontemporal_store(val, (v4f*)((float*)dW + o));
        } else if constexpr (kOut == kOutF32Acc) {
          v4f* d = (v4f*)((float*)dW + o);
          const v4f old = *d;
#pragma unroll
          for (int v = 0; v < 4; ++v) val[v] = old[v] + val[v];
          *d = val;
        } else {
          uint2* d = (uint2*)((uint16_t*)dW + o);
          if constexpr (kOut == kOutBF16Acc) {
            const uint2 old = *d;
            val[0] += __uint_as_float(old.x << 16);
            val[1] += __uint_as_float(old.x & 0xffff0000u);
            val[2] += __uint_as_float(old.y << 16);
            val[3] += __uint_as_float(old.y & 0xffff0000u);
          }
          uint2 b;
          b.x = bf16_pack2(val[0], val[1]);
          b.y = bf16_pack2(val[2], val[3]);
          *d = b;
        }
      }
    }
    __syncthreads();
  }
}

// Fixed cost of a tile in row-group steps (zeroing or writing its 256 KiB
// fp32 output and the prologue), so that empty experts' tiles count too.
constexpr int kTileFixed = 4;

template <int kOut, bool kE8M0>
__global__ __launch_bounds__(kWThreads, 1) void grouped_gemm_fp8_wgrad_kernel(
    const uint8_t* __restrict__ aT, const float* __restrict__ aTs, const uint8_t* __restrict__ bT,
    const float* __restrict__ bTs, const int32_t* __restrict__ pad, int E, int N, int Kd, int ld,
    int per_xcd, void* __restrict__ dW) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kWSmem];
  // the cost prefix lives in the stage buffers until the tile range is known
  long long* cpre = (long long*)smem;
  long long* wsum = cpre + SMOE_MAX_EXPERTS + 1;
  static_assert((SMOE_MAX_EXPERTS + 1 + kWThreads / kWave) * 8 <= kWSmem, "cost table fits");
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  // Work-balanced, XCD-aware tile order.  Tiles are numbered expert-major
  // (expert e owns tiles e*NT*KT .. +NT*KT, n-tile major, k-tile minor); a
  // tile of expert e costs steps(e) + kTileFixed.  The tile sequence is cut
  // into 8 contiguous ranges of equal total cost, and XCD x (workgroups are
  // dealt to the 8 XCDs round robin) runs range x in order, block j taking
  // tiles T_x + j, T_x + j + per_xcd, ...  An expert's tiles therefore stay
  // together on one XCD (its L2 serves each aT and bT slice to every tile
  // of the expert that reads it), and a hot expert's tiles are split over
  // as many XCDs as its share of the work needs.
  const int KT = (Kd + kWK - 1) / kWK, NT = (N + kWN - 1) / kWN;
  const int TE = NT * KT;  // tiles per expert
  {
    // cpre[e] = cost of all tiles of experts before e (64-bit: E * TE * steps)
    const int per = (E + kWThreads - 1) / kWThreads;
    long long loc[2], run = 0;
    for (int i = 0; i < per; ++i) {
      const int e = tid * per + i;
      long long c = 0;
      if (e < E) {
        const int a0 = max(pad[e], 0), a1 = min(pad[e + 1], ld);
        c = (long long)TE * ((a1 > a0 ? (a1 - a0) / kGroup : 0) + kTileFixed);
      }
      run += c;
      loc[i] = run;
    }
    long long incl = run;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const long long v = __shfl_up(incl, o, kWave);
      if (lane >= o) incl += v;
    }
    if (lane == kWave - 1) wsum[wid] = incl;
    __syncthreads();
    long long base = 0;
    for (int w = 0; w < wid; ++w) base += wsum[w];
    const long long excl = base + incl - run;
    for (int i = 0; i < per; ++i) {
      const int e = tid * per + i;
      if (e < E) cpre[e + 1] = excl + loc[i];
    }
    if (tid == 0) cpre[0] = 0;
    __syncthreads();
  }
  // first tile whose cost interval starts at or after cost c
  auto first_tile = [&](long long c) -> long long {
    int lo = 0, hi = E;  // largest e with cpre[e] <= c
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (cpre[mid] <= c) lo = mid;
      else hi = mid;
    }
    const long long per_tile = (cpre[lo + 1] - cpre[lo]) / TE;
    const long long r = (c - cpre[lo] + per_tile - 1) / per_tile;
    return (long long)lo * TE + min(r, (long long)TE);
  };
  const long long W = cpre[E];
  const int xcd = blockIdx.x & 7, j = blockIdx.x >> 3;
  // XCD x's range [T_x, T_x+1) starts at the tile where its cost share
  // starts; every workgroup computes it the same way.  Workgroup j of the
  // XCD takes tiles T_x + j, T_x + j + per_xcd, ... (the launch gives each
  // XCD one workgroup per CU, so every workgroup walks its share of the
  // range).  Scalar registers keep the loop off the tile body's VGPRs.
  const int t_begin = __builtin_amdgcn_readfirstlane(xcd == 0 ? 0 : (int)first_tile(W * xcd / 8));
  const int t_end =
      __builtin_amdgcn_readfirstlane(xcd == 7 ? E * TE : (int)first_tile(W * (xcd + 1) / 8));
  __syncthreads();  // the tiles' DMA overwrites the cost table
  for (int t = t_begin + j; t < t_end; t += per_xcd) {
    const int e = t / TE;
    const int rem = t - e * TE;
    wgrad_tile<kOut, kE8M0>(aT, aTs, bT, bTs, pad, N, Kd, ld, e, (rem / KT) * kWN, (rem % KT) * kWK, smem,
                     dW);
    __syncthreads();  // the next tile reuses the LDS
  }
}

// Compute units per XCD of the current device, looked up once per device.
constexpr int kMaxDevices = 64;
static std::atomic<int> g_cus_per_xcd[kMaxDevices];

static int cus_per_xcd(hipError_t* err) {
  int dev = 0;
  *err = hipGetDevice(&dev);
  if (*err != hipSuccess) return 0;
  if (dev < 0 || dev >= kMaxDevices) {
    *err = hipErrorInvalidDevice;
    return 0;
  }
  int n = g_cus_per_xcd[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    int cus = 0;
    *err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (*err != hipSuccess) return 0;
    n = cus / 8 > 0 ? cus / 8 : 1;
    g_cus_per_xcd[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

}  // namespace smoe

using namespace smoe;

extern "C" int smoe_grouped_gemm_fp8_wgrad_ex(const uint8_t* aT, const float* aTs,
                                              const uint8_t* bT, const float* bTs,
                                              const int32_t* pad, int E, int N, int Kdim, int ld,
                                              void* dW, int mode, void* stream) {
  if (N <= 0 || Kdim <= 0 || ld <= 0) return SMOE_EINVAL_DIM;
  if (E <= 0 || E > SMOE_MAX_EXPERTS) return SMOE_EINVAL_EXPERTS;
  // N and Kdim (the operands' rows, dW's edges) need only whole 16-row MFMA
  // blocks: tiles past them are clamped on load and masked on store
  if (N % 16 || Kdim % 16 || ld % kGroup) return SMOE_EINVAL_ALIGN128;
  if ((long long)kWN * ld >= (1LL << 31)) return SMOE_EINVAL_DIM;
  const bool e8m0 = (mode & SMOE_WGRAD_E8M0) != 0;
  mode &= ~SMOE_WGRAD_E8M0;
  if (mode < kOutF32 || mode > kOutBF16Acc) return SMOE_EINVAL_MODE;
  SMOE_CHECK_PTR(aT);
  SMOE_CHECK_PTR(bT);
  SMOE_CHECK_PTR(dW);
  if (!aTs || !bTs || !pad) return SMOE_EINVAL_NULL;
  if (((uintptr_t)aTs | (uintptr_t)bTs | (uintptr_t)pad) & 3u) return SMOE_EINVAL_PTRALIGN;
  // One workgroup per CU (the kernel's LDS allows one), per_xcd of them on
  // each XCD, each walking its XCD's tile range with stride per_xcd: the
  // cost table is built once per workgroup instead of once per tile, and
  // no workgroup is launched per tile.
  const long long tiles = (long long)E * ((Kdim + kWK - 1) / kWK) * ((N + kWN - 1) / kWN);
  if (tiles > 0x7fffffffLL) return SMOE_EINVAL_DIM;  // the kernel numbers tiles in int
  hipError_t herr = hipSuccess;
  const int cus = cus_per_xcd(&herr);
  if (herr != hipSuccess) return (int)herr;
  const long long per_xcd = std::min<long long>((tiles + 7) / 8, cus);
  const dim3 grid((unsigned)(per_xcd * 8)), block(kWThreads);
  hipStream_t s = (hipStream_t)stream;
#define SMOE_WG(M, P2)                                                                   \
  grouped_gemm_fp8_wgrad_kernel<M, P2><<<grid, block, 0, s>>>(aT, aTs, bT, bTs, pad, E, N, Kdim, \
                                                              ld, (int)per_xcd, dW)
#define SMOE_WG2(M) \
  if (e8m0) SMOE_WG(M, true); else SMOE_WG(M, false)
  switch (mode) {
    case kOutF32: SMOE_WG2(kOutF32); break;
    case kOutF32Acc: SMOE_WG2(kOutF32Acc); break;
    case kOutBF16: SMOE_WG2(kOutBF16); break;
    default: SMOE_WG2(kOutBF16Acc); break;
  }
#undef SMOE_WG2
#undef SMOE_WG
  SMOE_RETURN_LAUNCH();
}

extern "C" int smoe_grouped_gemm_fp8_wgrad(const uint8_t* aT, const float* aTs,
                                           const uint8_t* bT, const float* bTs,
                                           const int32_t* pad, int E, int N, int Kdim, int ld,
                                           float* dW, void* stream) {
  return smoe_grouped_gemm_fp8_wgrad_ex(aT, aTs, bT, bTs, pad, E, N, Kdim, ld, dW, kOutF32,
                                        stream);
}
