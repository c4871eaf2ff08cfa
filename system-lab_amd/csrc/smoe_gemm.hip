// smoe_gemm.hip — dropless fp8 (OCP e4m3) grouped GEMM with 1x128 activation
// scales and 128x128 weight-block scales, for gfx950.
//
//   c[r,n] = bf16( sum_kb as[r,kb] * bs[e,n/128,kb] * sum_{k in kb} a[r,k]*b[e,n,k] )
//
// Tiling.  A workgroup of 512 threads (8 waves) owns a 256-row x 256-column
// output tile of one expert; wave w owns rows (w/4)*128 .. +128 and columns
// (w%4)*64 .. +64, i.e. 8 x 4 blocks of the 16x16 fp8 MFMA with K = 128
// (v_mfma_f32_16x16x128_f8f6f4).  One MFMA covers a whole 128-wide scale
// block, so each block's partial sum is scaled by as[r,kb]*bs[e,nb,kb] and
// added to the fp32 accumulator right away (4 FMAs per MFMA).  Weight rows
// feed the MFMA's A operand and activation rows its B operand: an output lane
// holds one activation row (lane % 16), so the activation scale is per lane
// and the weight scale (a wave's 64 columns lie in one 128-column block) is
// wave-uniform.
//
// Data movement.  Each K step stages a 256x128-byte activation tile and a
// 256x128-byte weight tile in LDS with direct global->LDS loads
// (global_load_lds_dwordx4: no VGPR round trip), two stages deep: the loads of
// step kb+1 are issued before the MFMAs of step kb, and the step's single
// barrier waits for them.  The 256 activation scales of a step come either 8
// K steps at a time (K a multiple of 512: one 16-byte DMA per wave per
// chunk, double-buffered) or with each stage (one word from each of 256 rows,
// _dword DMA).  The LDS row layout (lds_row / swz) makes the 128-bit fragment
// reads conflict-free.  The tile's weight-block scales are copied to LDS once,
// before the K loop.
//
// Scheduling.  The grid covers an upper bound of m-tiles (ceil(R/256) + E,
// padded to kChipM) times the n-tiles.  Tiles are taken in chip-wide groups
// of kChipM consecutive m-tiles x all n-tiles; within a group, XCD x (blocks
// are dealt to the 8 XCDs round robin) takes m-tiles x*kChipM/8 .. +kChipM/8
// and sweeps the n-tiles, m fastest, so its 32 CUs run 4 m-tiles x 8 n-tiles
// at once.  All XCDs then stream the same weight slices at once (read from
// HBM once, the other XCDs hit the last-level cache), and each XCD's L2
// serves its own activation rows to all n-tiles.  A last,
// partial group's tiles are split evenly over the 8 XCDs instead.  Every
// workgroup derives the per-expert m-tile prefix sum from offsets[] in LDS
// (no host sync, no workspace) and leaves when its tile index is past the
// real total.  Zero-token experts own no tiles; rows past an expert's end are
// clamped on load and masked on store.
#include "smoe_mfma.h"

namespace smoe {

// m-tiles per chip-wide scheduling group: 4 per XCD, so an XCD's 32 CUs run
// 4 m-tiles x 8 n-tiles at once (12 distinct operand slices per K step)
constexpr int kChipM = 32;

// Tile configuration: waves form a kWR (rows) x kWN (columns) grid; each wave
// owns kRB 16-row blocks x 4 16-column blocks (kRB*16 rows x 64 columns).
// kStages LDS stages of (activation tile | weight tile | activation scales).
template <int kWR_, int kWN_, int kRB_, int kStages_>
struct Cfg {
  static constexpr int kWR = kWR_, kWN = kWN_, kRB = kRB_, kStages = kStages_;
  static constexpr int kWaves = kWR * kWN;
  static constexpr int kThreads = kWaves * kWave;
  static constexpr int kBM = kWR * kRB * 16;
  static constexpr int kBN = kWN * 64;
  static constexpr int kABytes = kBM * kRow;
  static constexpr int kBBytes = kBN * kRow;
  static constexpr int kSBytes = kBM * 4;
  static constexpr int kStage = kABytes + kBBytes + kSBytes;
  static constexpr int kASegs = kABytes / 1024 / kWaves;  // 1 KiB DMA segments per wave
  static constexpr int kBSegs = kBBytes / 1024 / kWaves;
  static constexpr int kSWaves = kBM / 64;                 // waves loading 256 B of scales
  static_assert(kASegs * kWaves * 1024 == kABytes, "A tile split");
  static_assert(kBSegs * kWaves * 1024 == kBBytes, "B tile split");
  static_assert(kSWaves <= kWaves, "scale split");
  static_assert(kStages * kStage + 4200 <= 160 * 1024, "LDS budget");
};

// kSwiGLU: the fc1 GEMM with SwiGLU + 1x128 requantisation fused into the
// epilogue.  b is W1 [E, N = 2I, K] (gate rows [0, I), up rows [I, 2I)); tile
// nt pairs gate columns nt*128 .. +128 with up columns I + nt*128 .. +128, so
// each tile row holds exactly one 128-wide group of h = silu(g)*u.  Outputs
// are hq [R, I] fp8 and hs [R, I/128]; c (c1 [R, 2I] bf16) is written only
// when not null.  h is computed from the bf16-rounded fc1 values exactly as
// the stand-alone SwiGLU kernel does, so the fused path is bit-identical to
// GEMM -> bf16 c1 -> swiglu_quant.
template <class C, bool kSwiGLU, bool kChunkS>
__global__ __launch_bounds__(C::kThreads, 1) void grouped_gemm_fp8_kernel(
    const uint8_t* __restrict__ a, const float* __restrict__ as, const uint8_t* __restrict__ b,
    const float* __restrict__ bs, const int32_t* __restrict__ offsets, int E, int R, int N,
    int Kd, int mt_bound, uint16_t* __restrict__ c, uint8_t* __restrict__ hq,
    float* __restrict__ hs) {
  static_assert(!kSwiGLU || C::kBN == 256, "fused SwiGLU pairs 128 gate with 128 up columns");
  constexpr int kThreads = C::kThreads, kBM = C::kBM, kBN = C::kBN, kStage = C::kStage;
  constexpr int kStages = C::kStages, kABytes = C::kABytes, kBBytes = C::kBBytes;
  constexpr int kASegs = C::kASegs, kBSegs = C::kBSegs, kRB = C::kRB;
  constexpr int kCPitch = kBN * 2 + 16;  // bytes per staged output row (+16: banks)
  // kChunkS (K a multiple of 512): the activation scales are staged kSChunk K
  // steps at a time in a double-buffered area after the stages, instead of
  // 256 words per step.
  constexpr int kSChunk = 8;
  constexpr int kSC0 = kStages * kStage;                 // scale chunk area
  constexpr int kSCBytes = kBM * kSChunk * 4;            // one chunk
  constexpr int kLoop = kSC0 + (kChunkS ? 2 * kSCBytes : 0);
  constexpr int kSmem = kLoop > kBM * kCPitch ? kLoop : kBM * kCPitch;
  static_assert(kSmem + 4200 <= 160 * 1024, "LDS budget");
  static_assert(!kChunkS || kSCBytes == C::kWaves * 1024, "one 1 KiB scale DMA per wave and chunk");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kSmem];
  __shared__ int mstart[SMOE_MAX_EXPERTS + 1];
  __shared__ int wsum[kThreads / kWave];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wid = tid >> 6;

  // ---- per-expert m-tile prefix sum (mstart[e] = first m-tile of e) -----
  const int per = (E + kThreads - 1) / kThreads;
  int loc[4];
  int run = 0;
  for (int i = 0; i < per; ++i) {
    const int e = tid * per + i;
    int t = 0;
    if (e < E) t = (offsets[e + 1] - offsets[e] + kBM - 1) / kBM;
    run += t;
    loc[i] = run;
  }
  int incl = run;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int v = __shfl_up(incl, o, kWave);
    if (lane >= o) incl += v;
  }
  if (lane == kWave - 1) wsum[wid] = incl;
  __syncthreads();
  int wbase = 0;
  for (int w = 0; w < wid; ++w) wbase += wsum[w];
  const int excl = wbase + incl - run;
  for (int i = 0; i < per; ++i) {
    const int e = tid * per + i;
    if (e < E) mstart[e + 1] = excl + loc[i];
  }
  if (tid == 0) mstart[0] = 0;
  __syncthreads();
  const int total_mt = mstart[E];

  // ---- tile index: chip-wide m-groups, kChipM/8 m-tiles per XCD ---------
  const int bid = blockIdx.x;
  const int I = N / 2;
  const int NT = kSwiGLU ? I / kGroup : (N + kBN - 1) / kBN;
  constexpr int kXM = kChipM / 8;  // m-tiles per XCD and group
  const int xcd = bid & 7, kx = bid >> 3;
  const int m_all = min(total_mt, mt_bound);
  const int full = m_all / kChipM;     // complete chip-wide groups
  const int m_last = m_all - full * kChipM;  // m-tiles of the last, partial group
  int mt, nt;
  if (kx < full * kXM * NT) {
    const int g = kx / (kXM * NT), rem = kx - g * (kXM * NT);
    mt = g * kChipM + kXM * xcd + rem % kXM;
    nt = rem / kXM;
  } else {
    // the partial group's m_last x NT tiles, m fastest, split into 8 equal
    // contiguous chunks so that every XCD gets a share
    const int chunk = (m_last * NT + 7) / 8;
    const int j = kx - full * kXM * NT;
    const int tl = xcd * chunk + j;
    if (j >= chunk || tl >= m_last * NT) return;
    mt = full * kChipM + tl % m_last;
    nt = tl / m_last;
  }

  int lo = 0, hi = E;  // largest e with mstart[e] <= mt
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (mstart[mid] <= mt) lo = mid;
    else hi = mid;
  }
  const int e = lo;
  const int row0 = offsets[e] + (mt - mstart[e]) * kBM;
  // rows outside [0, R) are never touched, whatever offsets[] holds
  const int rows = min(kBM, min(offsets[e + 1], R) - row0);
  if (row0 < 0 || rows <= 0) return;  // the whole workgroup leaves together
  const int n0 = nt * kBN;
  const int ksb = Kd / kBK;

  // ---- direct global->LDS loaders ---------------------------------------
  // Wave w fills 1 KiB LDS segments: A segments w*kASegs.., B segments
  // w*kBSegs.. (8 rows each), and (waves below kBM/64) scale rows w*64..+63.
  // Lane i of a segment writes row position p = seg*8 + i/8, chunk slot i%8;
  // that position holds tile row tile_row(p) and the slot holds its global
  // chunk (i%8) ^ (row & 7).  Offsets are per-lane 32-bit byte offsets from
  // wave-uniform (SGPR) base pointers; rows past the expert's end (A) or past
  // N (B) are clamped to the last valid row.
  const uint8_t* a_base = a + (size_t)row0 * Kd;
  const uint8_t* b_base = b + ((size_t)e * N + (kSwiGLU ? 0 : n0)) * Kd;
  const float* s_base = as + (size_t)row0 * ksb;
  const int ncols = kSwiGLU ? kBN : min(kBN, N - n0);
  // weight row of tile column row (fused: gate half, then up half)
  auto wrow = [&](int row) {
    if constexpr (kSwiGLU) return row < kGroup ? nt * kGroup + row : I + nt * kGroup + row - kGroup;
    else return min(row, ncols - 1);
  };
  uint32_t oa[kASegs], ob[kBSegs];
  {
    const int slot = lane & 7;
#pragma unroll
    for (int j = 0; j < kASegs; ++j) {
      const int row = tile_row((wid * kASegs + j) * 8 + (lane >> 3));
      oa[j] = (uint32_t)(min(row, rows - 1) * Kd + ((slot ^ (row & 7)) << 4));
    }
#pragma unroll
    for (int j = 0; j < kBSegs; ++j) {
      const int row = tile_row((wid * kBSegs + j) * 8 + (lane >> 3));
      ob[j] = (uint32_t)(wrow(row) * Kd + ((slot ^ (row & 7)) << 4));
    }
  }
  const uint32_t os = (uint32_t)(min((wid % C::kSWaves) * 64 + lane, rows - 1) * ksb) * 4u;
  // scale chunk DMA: lane l of wave w moves 16 bytes (4 K steps) of tile row
  // w*32 + l/2 into LDS row-major [kBM][kSChunk].  ksb is a multiple of 4, so
  // each 16-byte half of a chunk row lies wholly inside or wholly past the
  // row's end; a half past the end (the last chunk when ksb % 8 == 4) re-reads
  // the first half instead, and its values are never used.
  const uint32_t osc = (uint32_t)(min(wid * 32 + (lane >> 1), rows - 1) * ksb) * 4u;
  const int wr = wid / C::kWN, wn = wid % C::kWN;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_ptr_t)smem;

  // Wave-uniform LDS destinations of this wave's DMA segments, computed once
  // into scalar registers so that issuing a DMA in the K loop costs no
  // VALU -> SGPR round trip.  DMA q of a stage: q = 0 the activation scales
  // (waves below kSWaves), then kASegs A segments, then kBSegs B segments.
  const uint32_t s_lds = __builtin_amdgcn_readfirstlane(lds0 + kABytes + kBBytes + wid * 256);
  const uint32_t a_lds = __builtin_amdgcn_readfirstlane(lds0 + wid * kASegs * 1024);
  const uint32_t b_lds = __builtin_amdgcn_readfirstlane(lds0 + kABytes + wid * kBSegs * 1024);
  constexpr int kDma = 1 + kASegs + kBSegs;
  auto issue_one = [&](int q, int kb, int buf) {
    const uint32_t st = buf * kStage;
    if (q == 0) {
      if (wid < C::kSWaves) dma4(s_base + kb, os, s_lds + st);
    } else if (q <= kASegs) {
      dma16(a_base + (size_t)kb * kBK, oa[q - 1], a_lds + st + (q - 1) * 1024);
    } else {
      dma16(b_base + (size_t)kb * kBK, ob[q - 1 - kASegs], b_lds + st + (q - 1 - kASegs) * 1024);
    }
  };
  auto issue = [&](int kb, int buf) {
#pragma unroll
    for (int q = kChunkS ? 1 : 0; q < kDma; ++q) issue_one(q, kb, buf);
  };
  const uint32_t sc_lds = __builtin_amdgcn_readfirstlane(lds0 + kSC0 + wid * 1024);
  auto issue_sc = [&](int chunk) {
    const bool second = (lane & 1) && (chunk + 1) * kSChunk <= ksb;
    dma16(s_base + chunk * kSChunk, osc + (second ? 16u : 0u), sc_lds + (chunk & 1) * kSCBytes);
  };
  // loads one stage leaves outstanding per wave (waves 0-3 also load scales)
  const bool scale_wave = !kChunkS && wid < C::kSWaves;

  const int frow = lane & 15;
  const int fch = (lane >> 4) * 2;

  v4f acc[kRB][4];
#pragma unroll
  for (int i = 0; i < kRB; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

  // prologue: stages 0 .. kStages-2 in flight, stage 0 landed
  if constexpr (kChunkS) issue_sc(0);
#pragma unroll
  for (int s = 0; s < kStages - 1; ++s)
    if (s < ksb) issue(s, s);
  // While the first stages fly, the tile's weight-block scales (kBN/128
  // blocks x ksb) move to LDS, into the expert table's space (dead from here
  // on): a compiler-visible global load inside the K loop would make the
  // compiler drain vmcnt to zero, i.e. wait for every DMA stage in flight.
  constexpr int kNB128 = kBN / kGroup;
  const int NB = (N + kGroup - 1) / kGroup;  // weight-scale blocks per expert (last may be short)
  float* sbt = (float*)mstart;
  __syncthreads();
  for (int i = tid; i < kNB128 * ksb; i += kThreads) {
    const int nb = i / ksb, kb = i - nb * ksb;
    const int blk = kSwiGLU ? (nb == 0 ? nt : I / kGroup + nt) : min(n0 / kGroup + nb, NB - 1);
    sbt[i] = bs[((size_t)e * NB + blk) * ksb + kb];
  }
  __syncthreads();
  const float* sb_row = sbt + ((wn * 64) / kGroup) * ksb;
  if (kStages > 2 && ksb > 1) {
    if (scale_wave) wait_vm_lgkm0<kASegs + kBSegs + 1>();
    else wait_vm_lgkm0<kASegs + kBSegs>();
  } else {
    wait_vm_lgkm0<0>();
  }
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

  int buf = 0;
  for (int kb = 0; kb < ksb; ++kb) {
    // refill the slot consumed in the previous step (free after its barrier)
    const int nxt = kb + kStages - 1;
    // the next scale chunk goes out at the first step of the current one, into
    // the half whose chunk was last read before the previous barrier
    if (kChunkS && (kb & (kSChunk - 1)) == 0 && kb + kSChunk < ksb) issue_sc(kb / kSChunk + 1);
    if (nxt < ksb) issue(nxt, nxt % kStages);
    const uint8_t* sA = smem + buf * kStage;
    const uint8_t* sB = sA + kABytes;
    const float* sS = (const float*)(sB + kBBytes);
    const float* sC = (const float*)(smem + kSC0 + ((kb / kSChunk) & 1) * kSCBytes) + (kb & (kSChunk - 1));
    const float sb = sb_row[kb];
    v8i fw[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) fw[j] = lds_frag(sB, wn * 64 + j * 16 + frow, fch);
    // the next row block's activation fragment is read before this block's
    // MFMAs are issued, so its LDS latency hides behind them
    const int rbase = wr * kRB * 16 + frow;
    v8i fx = lds_frag(sA, rbase, fch);
#pragma unroll
    for (int i = 0; i < kRB; ++i) {
      v8i fxn = fx;
      if (i + 1 < kRB) fxn = lds_frag(sA, rbase + (i + 1) * 16, fch);
      const float sc = (kChunkS ? sC[(rbase + i * 16) * kSChunk] : sS[rbase + i * 16]) * sb;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const v4f p = mfma16(fw[j], fx, v4f{0.0f, 0.0f, 0.0f, 0.0f});
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[i][j][v] = __builtin_fmaf(p[v], sc, acc[i][j][v]);
      }
      fx = fxn;
    }
    // stage kb+1 must have landed for every wave; later stages may still fly
    if (kStages > 2 && kb + kStages - 1 < ksb) {
      if (scale_wave) wait_vm_lgkm0<kASegs + kBSegs + 1>();
      else wait_vm_lgkm0<kASegs + kBSegs>();
    } else {
      wait_vm_lgkm0<0>();
    }
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    buf = (buf + 1 == kStages) ? 0 : buf + 1;
  }

  // ---- epilogue: the bf16 tile is staged in LDS (the stage buffers are free
  // now: the K loop's last barrier ordered every fragment read before) and
  // written out row by row with 16-byte stores, so each output row segment of
  // kBN columns leaves as whole 128-byte lines.
  uint8_t* ct = smem;
#pragma unroll
  for (int i = 0; i < kRB; ++i) {
    const int rl = wr * kRB * 16 + i * 16 + frow;
    const int cl = wn * 64 + (lane >> 4) * 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint2 o;
      o.x = bf16_pack2(acc[i][j][0], acc[i][j][1]);
      o.y = bf16_pack2(acc[i][j][2], acc[i][j][3]);
      *(uint2*)(ct + rl * kCPitch + (cl + j * 16) * 2) = o;
    }
  }
  __syncthreads();
  if constexpr (kSwiGLU) {
    // 8 lanes per row, 16 columns each: h = silu(g) * u from the staged bf16
    // values, amax over the 8 lanes, 16 fp8 bytes per lane.
    for (int idx = tid; idx < rows * 8; idx += kThreads) {
      const int r = idx >> 3, sub = idx & 7;
      const uint8_t* rowp = ct + r * kCPitch;
      float fg[16], fu[16], h[16];
      unpack_bf16x8(*(const uint4*)(rowp + sub * 32), fg);
      unpack_bf16x8(*(const uint4*)(rowp + sub * 32 + 16), fg + 8);
      unpack_bf16x8(*(const uint4*)(rowp + 256 + sub * 32), fu);
      unpack_bf16x8(*(const uint4*)(rowp + 256 + sub * 32 + 16), fu + 8);
#pragma unroll
      for (int i = 0; i < 16; ++i) h[i] = silu32(fg[i]) * fu[i];
      const Q16 q = quant16(h);
      const size_t gr = (size_t)(row0 + r);
      *(uint4*)(hq + gr * I + nt * kGroup + sub * 16) = q.q;
      if (sub == 0) hs[gr * (I / kGroup) + nt] = q.scale;
      if (c) {
        uint16_t* crow = c + gr * N + nt * kGroup + sub * 16;
        *(uint4*)crow = *(const uint4*)(rowp + sub * 32);
        *(uint4*)(crow + 8) = *(const uint4*)(rowp + sub * 32 + 16);
        *(uint4*)(crow + I) = *(const uint4*)(rowp + 256 + sub * 32);
        *(uint4*)(crow + I + 8) = *(const uint4*)(rowp + 256 + sub * 32 + 16);
      }
    }
  } else {
    store_staged_tile<kThreads, kBM, kBN, kCPitch>(ct, c, row0, rows, N, n0, ncols, tid);
  }
}

#ifndef SMOE_GEMM_CFG
#define SMOE_GEMM_CFG Cfg<2, 4, 8, 2>
#endif
using GemmCfg = SMOE_GEMM_CFG;

}  // namespace smoe

using namespace smoe;

extern "C" size_t smoe_grouped_gemm_fp8_workspace_size(int E, int R, int N, int Kdim) {
  (void)E; (void)R; (void)N; (void)Kdim;
  return 0;
}

extern "C" int smoe_grouped_gemm_fp8(const uint8_t* a, const float* as, const uint8_t* b,
                                     const float* bs, const int32_t* offsets, int E, int R, int N,
                                     int Kdim, uint16_t* c, void* ws, size_t ws_bytes,
                                     void* stream) {
  (void)ws; (void)ws_bytes;
  if (R <= 0 || N <= 0 || Kdim <= 0) return SMOE_EINVAL_DIM;
  if (E <= 0 || E > SMOE_MAX_EXPERTS) return SMOE_EINVAL_EXPERTS;
  // K is the operands' padded pitch; N may end in a partial weight block
  if (N % kLane || Kdim % kGroup) return SMOE_EINVAL_ALIGN128;
  if (Kdim > 65536) return SMOE_EINVAL_DIM;  // weight-scale table fits the LDS expert table
  SMOE_CHECK_PTR(a);
  SMOE_CHECK_PTR(b);
  SMOE_CHECK_PTR(c);
  if (!as || !bs || !offsets) return SMOE_EINVAL_NULL;
  if (((uintptr_t)as | (uintptr_t)bs | (uintptr_t)offsets) & 3u) return SMOE_EINVAL_PTRALIGN;
  using C = GemmCfg;
  const long long mt_bound = (R + C::kBM - 1) / C::kBM + E;
  const long long NT = (N + C::kBN - 1) / C::kBN;
  // pad the m-tile count to whole scheduling groups, the grid to a multiple of 8
  const long long mt_pad = (mt_bound + kChipM - 1) / kChipM * kChipM;
  long long nblk = mt_pad * NT;
  nblk = (nblk + 7) / 8 * 8;
  if (nblk > 0x7fffffffLL) return SMOE_EINVAL_DIM;
  if (Kdim % (kBK * 4) == 0)
    grouped_gemm_fp8_kernel<C, false, true>
        <<<dim3((unsigned)nblk), dim3(C::kThreads), 0, (hipStream_t)stream>>>(
            a, as, b, bs, offsets, E, R, N, Kdim, (int)mt_bound, c, nullptr, nullptr);
  else
    grouped_gemm_fp8_kernel<C, false, false>
        <<<dim3((unsigned)nblk), dim3(C::kThreads), 0, (hipStream_t)stream>>>(
            a, as, b, bs, offsets, E, R, N, Kdim, (int)mt_bound, c, nullptr, nullptr);
  SMOE_RETURN_LAUNCH();
}

extern "C" int smoe_grouped_gemm_fp8_swiglu(const uint8_t* a, const float* as, const uint8_t* w1,
                                            const float* w1s, const int32_t* offsets, int E,
                                            int R, int I, int Kdim, uint8_t* hq, float* hs,
                                            uint16_t* c1, void* stream) {
  if (R <= 0 || I <= 0 || Kdim <= 0) return SMOE_EINVAL_DIM;
  if (E <= 0 || E > SMOE_MAX_EXPERTS) return SMOE_EINVAL_EXPERTS;
  if (I % kGroup || Kdim % kGroup) return SMOE_EINVAL_ALIGN128;
  if (Kdim > 65536) return SMOE_EINVAL_DIM;
  // weight-row offsets are 32-bit from the expert's base
  if (2LL * I * Kdim >= (1LL << 31)) return SMOE_EINVAL_DIM;
  SMOE_CHECK_PTR(a);
  SMOE_CHECK_PTR(w1);
  SMOE_CHECK_PTR(hq);
  if (c1 && ((uintptr_t)c1 & 15u)) return SMOE_EINVAL_PTRALIGN;
  if (!as || !w1s || !offsets || !hs) return SMOE_EINVAL_NULL;
  if (((uintptr_t)as | (uintptr_t)w1s | (uintptr_t)offsets | (uintptr_t)hs) & 3u)
    return SMOE_EINVAL_PTRALIGN;
  using C = GemmCfg;
  const int N = 2 * I;
  const long long mt_bound = (R + C::kBM - 1) / C::kBM + E;
  const long long NT = I / kGroup;
  const long long mt_pad = (mt_bound + kChipM - 1) / kChipM * kChipM;
  long long nblk = mt_pad * NT;
  nblk = (nblk + 7) / 8 * 8;
  if (nblk > 0x7fffffffLL) return SMOE_EINVAL_DIM;
  if (Kdim % (kBK * 4) == 0)
    grouped_gemm_fp8_kernel<C, true, true>
        <<<dim3((unsigned)nblk), dim3(C::kThreads), 0, (hipStream_t)stream>>>(
            a, as, w1, w1s, offsets, E, R, N, Kdim, (int)mt_bound, c1, hq, hs);
  else
    grouped_gemm_fp8_kernel<C, true, false>
        <<<dim3((unsigned)nblk), dim3(C::kThreads), 0, (hipStream_t)stream>>>(
            a, as, w1, w1s, offsets, E, R, N, Kdim, (int)mt_bound, c1, hq, hs);
  SMOE_RETURN_LAUNCH();
}
