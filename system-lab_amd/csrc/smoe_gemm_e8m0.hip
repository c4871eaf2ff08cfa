// smoe_gemm_e8m0.hip — the dropless fp8 grouped GEMM on packed weights for
// operands whose block scales are powers of two (E8M0 values), for gfx950.
//
//   c[r,n] = bf16( sum_kb as[r,kb] * bs[e,n/128,kb] * sum_{k in kb} a[r,k]*b[e,n,k] )
//
// The contract, packed weight layout, expert scan and tile order are those of
// smoe_gemm_packed.hip.  What differs is where the scales are applied: every
// as[r,kb] and bs[e,nb,kb] is a power of two, so the scaled MFMA
// (v_mfma_scale_f32_16x16x128_f8f6f4) applies them in hardware from their
// exponent bytes and accumulates each K block straight into the running sum.
// No VALU instruction touches the accumulators in the K loop, so they can sit
// in the accumulation registers, which frees the architectural ones for a
// wider wave tile:
//
// Tiling.  A workgroup of 4 waves (one per SIMD) owns a 256 x 256 output
// tile; wave w owns all 256 rows and columns w*64 .. +64 (16 row blocks x 4
// column blocks, 256 fp32 accumulators per lane).  Against the 8-wave kernel
// of smoe_gemm_packed.hip each activation fragment read from LDS now feeds 4
// MFMAs instead of 2, which halves the LDS read traffic per step (128 KiB
// per CU instead of 256 KiB).  Activations: a 4-stage LDS ring filled by
// direct global->LDS DMA three K steps ahead, activation scales in
// double-buffered chunks of 8 K steps; weights: four register buffers, step
// kb+3 loaded while step kb computes.
//
// Measured at benchmark config 4 (DeepSeek-V3 local experts, R = 65536, 32
// Zipf-loaded experts) on power-of-two operands: fc1 (N 4096, K 7168)
// 1.53-1.58 ms against 1.77 ms for smoe_gemm_packed.hip, fc2 (N 7168, K 2048)
// 0.92-0.96 against 1.03-1.05 ms; bytes identical.
//
// Scope: K a multiple of 128 from 512 to 65536 (K blocks 4 .. 512), every
// scale a power of two; the ops layer checks the recipe.
#include "smoe_mfma.h"

namespace smoe {
namespace e8m0 {

constexpr int kChipM = 32;              // scheduling group, as in smoe_gemm.hip
constexpr int kThreads = 256, kWaves = 4, kBM = 256, kBN = 256;
constexpr int kRB = 16, kCB = 4;        // row blocks x column blocks per wave
constexpr int kAS = 4;                  // activation stages (DMA three steps ahead)
constexpr int kABytes = kBM * kRow;     // 32 KiB per stage
constexpr int kSegs = kABytes / 1024 / kWaves;  // 1 KiB activation DMAs per wave and stage
constexpr int kSChunk = 8;              // K steps per activation-scale chunk
constexpr int kSCBytes = kBM * kSChunk * 4;
constexpr int kSCDma = kSCBytes / 1024 / kWaves;  // 1 KiB scale DMAs per wave and chunk
constexpr int kCPitch = kBN * 2 + 16;   // bytes per staged bf16 output row
constexpr int kSC0 = kAS * kABytes;     // scale chunk area
constexpr int kLoop = kSC0 + 2 * kSCBytes;
constexpr int kSmem = kLoop > kBM * kCPitch ? kLoop : kBM * kCPitch;
static_assert(kSmem + 4200 <= 160 * 1024, "LDS budget");
static_assert(kSegs == 8 && kSCDma == 2, "DMA split");

typedef v4i WBuf[kCB][2];  // one step's weight operands of a wave

template <int n>
__device__ __forceinline__ void wait_vm() {
  static_assert(n >= 0 && n < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((n & 15) | (7 << 4) | ((n >> 4) << 14));
}

__device__ __forceinline__ v8i lds_frag_p(const uint8_t* base, int row, int g) {
  const v4i lo = *(const v4i*)(base + swz(row, g));
  const v4i hi = *(const v4i*)(base + swz(row, g + 4));
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

__device__ __forceinline__ int e8m0_of(float s) { return (__float_as_uint(s) >> 23) & 0xff; }

// acc += (A scaled by 2^(sa-127) per row) x (B scaled by 2^(sb-127) per
// column), accumulated in place in accumulation registers.  Written as asm
// so that every accumulator keeps one register quad for the whole K loop:
// with 256 of them the compiler's own MFMA form needs a spare quad for a
// fresh destination, which the accumulation file does not have, and it then
// moves accumulators through the architectural registers every step.
// Hazards: the accumulators are written only by these MFMAs (an accumulator
// is reused 64 MFMAs later); a row block's first MFMA starts with two wait
// states after the VALU that may have just written its scale operands; the
// epilogue waits out the last MFMA with explicit s_nops.  Operand loads are waited for by the compiler, which sees
// the asm's register uses.
template <bool kNop>
__device__ __forceinline__ void mfma_scale_acc(v4f& acc, const v8i& a, const v8i& b, int sa,
                                               int sb) {
  if constexpr (kNop)  // the row block's first MFMA: its scale was just computed by VALU
    asm volatile("s_nop 1\n\tv_mfma_scale_f32_16x16x128_f8f6f4 %0, %1, %2, %0, %3, %4 op_sel_hi:[0,0,0]"
                 : "+a"(acc)
                 : "v"(a), "v"(b), "v"(sa), "v"(sb));
  else
    asm volatile("v_mfma_scale_f32_16x16x128_f8f6f4 %0, %1, %2, %0, %3, %4 op_sel_hi:[0,0,0]"
                 : "+a"(acc)
                 : "v"(a), "v"(b), "v"(sa), "v"(sb));
}

// kSwiGLU: bp is W1 packed [E, 2I, K] (N = 2I); tile nt pairs gate columns
// nt*128 .. +128 (waves 0-1) with up columns I + nt*128 .. +128 (waves 2-3),
// and the epilogue writes h = silu(gate) * up requantised 1x128 with
// power-of-two scales into hq [R, I], hs [R, I/128] (and c1 when c is not
// null): the bytes of the SwiGLU quantiser run on this kernel's c.
template <bool kSwiGLU>
__global__ __launch_bounds__(kThreads, 1) void grouped_gemm_fp8_e8m0_kernel(
    const uint8_t* __restrict__ a, const float* __restrict__ as, const uint8_t* __restrict__ bp,
    const float* __restrict__ bs, const int32_t* __restrict__ offsets, int E, int R, int N, int Kd,
    int mt_bound, uint16_t* __restrict__ c, uint8_t* __restrict__ hq, float* __restrict__ hs) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kSmem];
  __shared__ int mstart[SMOE_MAX_EXPERTS + 1];
  __shared__ int wsum[kWaves];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wid = tid >> 6;

  // ---- per-expert m-tile prefix sum ---------------------------------------
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
  constexpr int kXM = kChipM / 8;
  const int xcd = bid & 7, kx = bid >> 3;
  const int m_all = min(total_mt, mt_bound);
  const int full = m_all / kChipM;
  const int m_last = m_all - full * kChipM;
  int mt, nt;
  if (kx < full * kXM * NT) {
    const int g = kx / (kXM * NT), rem = kx - g * (kXM * NT);
    mt = g * kChipM + kXM * xcd + rem % kXM;
    nt = rem / kXM;
  } else {
    const int chunk = (m_last * NT + 7) / 8;
    const int j = kx - full * kXM * NT;
    const int tl = xcd * chunk + j;
    if (j >= chunk || tl >= m_last * NT) return;
    mt = full * kChipM + tl % m_last;
    nt = tl / m_last;
  }
  int lo = 0, hi = E;
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (mstart[mid] <= mt) lo = mid;
    else hi = mid;
  }
  const int e = lo;
  const int row0 = offsets[e] + (mt - mstart[e]) * kBM;
  const int rows = min(kBM, min(offsets[e + 1], R) - row0);
  if (row0 < 0 || rows <= 0) return;  // the whole workgroup leaves together
  const int n0 = nt * kBN;
  const int ksb = Kd / kBK;
  const int ncols = kSwiGLU ? kBN : min(kBN, N - n0);

  // ---- activation DMA: wave w fills 1 KiB segments w*8 .. w*8+7 of a stage
  const uint8_t* a_base = a + (size_t)row0 * Kd;
  const float* s_base = as + (size_t)row0 * ksb;
  uint32_t oa[kSegs];
  {
    const int slot = lane & 7;
#pragma unroll
    for (int j = 0; j < kSegs; ++j) {
      const int row = tile_row((wid * kSegs + j) * 8 + (lane >> 3));
      oa[j] = (uint32_t)(min(row, rows - 1) * Kd + ((slot ^ (row & 7)) << 4));
    }
  }
  // Activation scales travel in chunks of 8 K steps, 32 bytes per tile row:
  // scale DMA h of wave w moves tile rows (w*2+h)*32 + l/2, lane l the 16
  // bytes of half l%2.  Chunk c holds the 8 steps from sc_win(c): 8c, except
  // the last chunk, whose window ends at ksb (so no DMA reads past a row's
  // ksb scales).  With 4 <= ksb < 8 the one chunk's halves hold steps 0..3
  // and ksb-4..ksb-1.  sc_slot maps step kb to its position in its chunk.
  uint32_t osc[kSCDma];
#pragma unroll
  for (int h = 0; h < kSCDma; ++h)
    osc[h] = (uint32_t)(min((wid * kSCDma + h) * 32 + (lane >> 1), rows - 1) * ksb) * 4u;
  auto sc_win = [&](int chunk) { return ksb >= kSChunk ? min(chunk * kSChunk, ksb - kSChunk) : 0; };
  auto sc_src = [&](int chunk) -> uint32_t {  // this lane's first step, in bytes
    const int half = lane & 1;
    const int st = ksb >= kSChunk ? sc_win(chunk) + 4 * half : (half ? ksb - 4 : 0);
    return (uint32_t)st * 4u;
  };
  auto sc_slot = [&](int kb) {
    return ksb >= kSChunk ? kb - sc_win(kb / kSChunk) : (kb < 4 ? kb : kb + kSChunk - ksb);
  };
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_ptr_t)smem;
  const uint32_t a_lds = __builtin_amdgcn_readfirstlane(lds0 + wid * kSegs * 1024);
  const uint32_t sc_lds = __builtin_amdgcn_readfirstlane(lds0 + kSC0 + wid * kSCDma * 1024);
  auto issue_sc = [&](int chunk) __attribute__((always_inline)) {
    const uint32_t src = sc_src(chunk);
#pragma unroll
    for (int h = 0; h < kSCDma; ++h)
      dma16(s_base, osc[h] + src, sc_lds + (chunk & 1) * kSCBytes + h * 1024);
  };
  // The same DMAs issued only when the wave-uniform go is nonzero, with the
  // branch inside one asm statement: a branch the compiler sees in the K loop
  // makes it split the accumulators' live ranges around it.
  auto issue_sc_if = [&](int chunk, int go) __attribute__((always_inline)) {
    const uint32_t src = sc_src(chunk);
    const uint32_t dst = sc_lds + (chunk & 1) * kSCBytes;
    // go is wave-uniform; compared per lane, so that it may sit in either
    // register file
    asm volatile(
        "v_cmp_eq_u32 vcc, 0, %4\n\t"
        "s_cbranch_vccnz 1f\n\t"
        "s_mov_b32 m0, %0\n\t"
        "global_load_lds_dwordx4 %2, %3\n\t"
        "s_mov_b32 m0, %1\n\t"
        "global_load_lds_dwordx4 %5, %3\n\t"
        "1:" ::"s"(dst), "s"(dst + 1024), "v"(osc[0] + src), "s"(s_base), "v"(go),
        "v"(osc[1] + src)
        : "memory", "vcc");
  };
  // ---- packed weights: wave w's four 16-row blocks of weight rows
  const uint8_t* b_base = bp + (size_t)e * ((size_t)N * Kd);
  uint32_t ob[kCB];
#pragma unroll
  for (int j = 0; j < kCB; ++j) {
    int wr0;  // first weight row of this column block
    if constexpr (kSwiGLU)
      wr0 = (wid < 2 ? 0 : I) + nt * kGroup + (wid & 1) * 64 + j * 16;
    else
      wr0 = min(n0 + wid * 64 + j * 16, N - 16);  // columns past N: clamped, never stored
    ob[j] = (uint32_t)(wr0 / 16) * (uint32_t)ksb * 2048u + (uint32_t)lane * 16u;
  }
  auto load_b = [&](int kb, WBuf& f) __attribute__((always_inline)) {
    const uint8_t* base = b_base + (size_t)kb * 2048;
#pragma unroll
    for (int j = 0; j < kCB; ++j) {
      f[j][0] = *(const v4i*)(base + ob[j]);
      f[j][1] = *(const v4i*)(base + ob[j] + 1024);
    }
  };

  const int frow = lane & 15;
  const int fg = lane >> 4;
  v4f acc[kRB][kCB];
#pragma unroll
  for (int i = 0; i < kRB; ++i)
#pragma unroll
    for (int j = 0; j < kCB; ++j) acc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

  // ---- prologue: scale chunk 0, activation stages 0..2, weights of steps 0, 1
  WBuf fA, fB, fC, fD;
  issue_sc(0);
#pragma unroll
  for (int s = 0; s < kAS - 1; ++s) {
    const int ks = min(s, ksb - 1);
#pragma unroll
    for (int q = 0; q < kSegs; ++q)
      dma16(a_base + (size_t)ks * kBK, oa[q], a_lds + s * kABytes + q * 1024);
  }
  load_b(0, fA);
  load_b(min(1, ksb - 1), fB);
  load_b(min(2, ksb - 1), fC);
  // the tile's weight-block scales go to LDS (the expert table's space)
  constexpr int kNB128 = kBN / kGroup;
  const int NB = (N + kGroup - 1) / kGroup;
  float* sbt = (float*)mstart;
  __syncthreads();
  for (int i = tid; i < kNB128 * ksb; i += kThreads) {
    const int nb = i / ksb, kb = i - nb * ksb;
    const int blk = kSwiGLU ? (nb == 0 ? nt : I / kGroup + nt) : min(n0 / kGroup + nb, NB - 1);
    sbt[i] = bs[((size_t)e * NB + blk) * ksb + kb];
  }
  __syncthreads();
  const float* sb_row = sbt + ((wid * 64) / kGroup) * ksb;
  wait_vm<0>();
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

  // ---- one K step: weights of step kb in cur, those of step kb+3 loaded
  // into nxt (the buffer step kb-1 used).  The activation DMAs of a step go
  // out before its first 8 row blocks and the weight loads before the last
  // 8.  The compiler waits for cur itself, counting only its own loads: the
  // 16 loads it sees after cur (steps kb-2 and kb-1) make it wait until at
  // most 16 memory operations are outstanding, which with the DMAs in the
  // same in-order counter retires everything up to step kb-2 (stage kb+1
  // and the weights of step kb+1, both needed within the next step) and
  // leaves step kb-1's loads in flight.  Past the last step the loads repeat
  // step ksb-1's data into buffers and stages no later step reads.
  auto step = [&](int kb, WBuf& cur, WBuf& nxt, bool tail) __attribute__((always_inline)) {
    const int ka = min(kb + kAS - 1, ksb - 1);
    const uint32_t a_dst = a_lds + (uint32_t)((kb + kAS - 1) % kAS) * kABytes;
    const uint8_t* a_src = a_base + (size_t)ka * kBK;
    const uint8_t* b_src = b_base + (size_t)min(kb + 3, ksb - 1) * 2048;
    const uint8_t* sA = smem + (kb % kAS) * kABytes;
    const float* sC = (const float*)(smem + kSC0 + ((kb / kSChunk) & 1) * kSCBytes) + sc_slot(kb);
    const int ew = e8m0_of(sb_row[kb]);
    v8i fw[kCB];
#pragma unroll
    for (int j = 0; j < kCB; ++j)
      fw[j] = __builtin_shufflevector(cur[j][0], cur[j][1], 0, 1, 2, 3, 4, 5, 6, 7);
    asm volatile("" : "+v"(fw[0]), "+v"(fw[1]), "+v"(fw[2]), "+v"(fw[3]));
    // the next scale chunk, after the compiler's wait for cur (which does
    // not count it)
    issue_sc_if(kb / kSChunk + 1, (kb & (kSChunk - 1)) == 0 && kb + kSChunk < ksb);
    v8i fx = lds_frag_p(sA, frow, fg);
    int ex = e8m0_of(sC[frow * kSChunk]);
#pragma unroll
    for (int i = 0; i < kRB; ++i) {
      if (i < 8) {
        dma16(a_src, oa[i], a_dst + i * 1024);
      } else {
        const int q = i - 8;  // weight load q: column block q >> 1, half q & 1
        nxt[q >> 1][q & 1] = *(const v4i*)(b_src + ob[q >> 1] + (q & 1) * 1024);
      }
      v8i fxn = fx;
      int exn = ex;
      if (i + 1 < kRB) {
        fxn = lds_frag_p(sA, (i + 1) * 16 + frow, fg);
        exn = e8m0_of(sC[((i + 1) * 16 + frow) * kSChunk]);
      }
#pragma unroll
      for (int j = 0; j < kCB; ++j) {
        if (j == 0) mfma_scale_acc<true>(acc[i][j], fw[j], fx, ew, ex);
        else mfma_scale_acc<false>(acc[i][j], fw[j], fx, ew, ex);
      }
      fx = fxn;
      ex = exn;
    }
    // Activation stage kb+1 was issued during step kb-2; the 32 loads of
    // steps kb-1 and kb (16 DMAs, 16 weight loads) came after it, so
    // vmcnt(32) covers it and the scale chunks, which are older.  After the
    // loop the compiler may drop weight loads that no step reads, so the
    // steps there count on their 16 DMAs only.  The barrier then makes every
    // wave's stage kb+1 visible and frees stage kb.
    if (tail) wait_vm<16>();
    else wait_vm<32>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  int kb = 0;
  for (; kb + 3 < ksb; kb += 4) {
    step(kb, fA, fD, false);
    step(kb + 1, fB, fA, false);
    step(kb + 2, fC, fB, false);
    step(kb + 3, fD, fC, false);
  }
  if (kb < ksb) step(kb, fA, fD, true);
  if (kb + 1 < ksb) step(kb + 1, fB, fA, true);
  if (kb + 2 < ksb) step(kb + 2, fC, fB, true);
  asm volatile("s_nop 15\n\ts_nop 15" ::: "memory");  // last MFMA results settle
  wait_vm<0>();
  __syncthreads();

  // ---- epilogue: bf16 tile staged in LDS, then written row by row --------
  uint8_t* ct = smem;
#pragma unroll
  for (int i = 0; i < kRB; ++i) {
    const int rl = i * 16 + frow;
    const int cl = wid * 64 + (lane >> 4) * 4;
#pragma unroll
    for (int j = 0; j < kCB; ++j) {
      uint2 o;
      o.x = bf16_pack2(acc[i][j][0], acc[i][j][1]);
      o.y = bf16_pack2(acc[i][j][2], acc[i][j][3]);
      *(uint2*)(ct + rl * kCPitch + (cl + j * 16) * 2) = o;
    }
  }
  __syncthreads();
  if constexpr (kSwiGLU) {
    // 8 lanes per row, 16 columns each: h = silu(g) * u from the staged bf16
    // values, amax over the 8 lanes, 16 fp8 bytes per lane
    for (int idx = tid; idx < rows * 8; idx += kThreads) {
      const int r = idx >> 3, sub = idx & 7;
      const uint8_t* rowp = ct + r * kCPitch;
      float fgt[16], fu[16], h[16];
      unpack_bf16x8(*(const uint4*)(rowp + sub * 32), fgt);
      unpack_bf16x8(*(const uint4*)(rowp + sub * 32 + 16), fgt + 8);
      unpack_bf16x8(*(const uint4*)(rowp + 256 + sub * 32), fu);
      unpack_bf16x8(*(const uint4*)(rowp + 256 + sub * 32 + 16), fu + 8);
#pragma unroll
      for (int i = 0; i < 16; ++i) h[i] = silu32(fgt[i]) * fu[i];
      const Q16 q = quant16<true>(h);
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

}  // namespace e8m0
}  // namespace smoe

using namespace smoe;

namespace {
int e8m0_args(const uint8_t* a, const float* as, const uint8_t* wp, const float* ws,
              const int32_t* offsets, int E, int R, int N, int Kdim) {
  if (R <= 0 || N <= 0 || Kdim <= 0) return SMOE_EINVAL_DIM;
  if (E <= 0 || E > SMOE_MAX_EXPERTS) return SMOE_EINVAL_EXPERTS;
  if (N % kLane || Kdim % kBK) return SMOE_EINVAL_ALIGN128;
  if (Kdim < 4 * kBK || Kdim > 65536) return SMOE_EINVAL_DIM;  // 4 .. 512 K steps
  if ((long long)N * Kdim >= (1LL << 32)) return SMOE_EINVAL_DIM;
  SMOE_CHECK_PTR(a);
  SMOE_CHECK_PTR(wp);
  if (!as || !ws || !offsets) return SMOE_EINVAL_NULL;
  if (((uintptr_t)as | (uintptr_t)ws | (uintptr_t)offsets) & 3u) return SMOE_EINVAL_PTRALIGN;
  return SMOE_OK;
}
long long e8m0_grid(int E, int R, int NT, long long* mt_bound) {
  *mt_bound = (R + e8m0::kBM - 1) / e8m0::kBM + E;
  const long long mt_pad = (*mt_bound + e8m0::kChipM - 1) / e8m0::kChipM * e8m0::kChipM;
  return (mt_pad * NT + 7) / 8 * 8;
}
}  // namespace

extern "C" int smoe_grouped_gemm_fp8_packed_e8m0(const uint8_t* a, const float* as,
                                                 const uint8_t* wp, const float* ws,
                                                 const int32_t* offsets, int E, int R, int N,
                                                 int Kdim, uint16_t* c, void* stream) {
  const int st = e8m0_args(a, as, wp, ws, offsets, E, R, N, Kdim);
  if (st) return st;
  SMOE_CHECK_PTR(c);
  long long mt_bound;
  const long long nblk = e8m0_grid(E, R, (N + e8m0::kBN - 1) / e8m0::kBN, &mt_bound);
  if (nblk > 0x7fffffffLL) return SMOE_EINVAL_DIM;
  e8m0::grouped_gemm_fp8_e8m0_kernel<false>
      <<<dim3((unsigned)nblk), dim3(e8m0::kThreads), 0, (hipStream_t)stream>>>(
          a, as, wp, ws, offsets, E, R, N, Kdim, (int)mt_bound, c, nullptr, nullptr);
  SMOE_RETURN_LAUNCH();
}

extern "C" int smoe_grouped_gemm_fp8_packed_e8m0_swiglu(const uint8_t* a, const float* as,
                                                        const uint8_t* w1p, const float* w1s,
                                                        const int32_t* offsets, int E, int R,
                                                        int I, int Kdim, uint8_t* hq, float* hs,
                                                        uint16_t* c1, void* stream) {
  if (I <= 0) return SMOE_EINVAL_DIM;
  if (I % kGroup) return SMOE_EINVAL_ALIGN128;
  const int st = e8m0_args(a, as, w1p, w1s, offsets, E, R, 2 * I, Kdim);
  if (st) return st;
  SMOE_CHECK_PTR(hq);
  if (c1 && ((uintptr_t)c1 & 15u)) return SMOE_EINVAL_PTRALIGN;
  if (!hs) return SMOE_EINVAL_NULL;
  if ((uintptr_t)hs & 3u) return SMOE_EINVAL_PTRALIGN;
  long long mt_bound;
  const long long nblk = e8m0_grid(E, R, I / kGroup, &mt_bound);
  if (nblk > 0x7fffffffLL) return SMOE_EINVAL_DIM;
  e8m0::grouped_gemm_fp8_e8m0_kernel<true>
      <<<dim3((unsigned)nblk), dim3(e8m0::kThreads), 0, (hipStream_t)stream>>>(
          a, as, w1p, w1s, offsets, E, R, 2 * I, Kdim, (int)mt_bound, c1, hq, hs);
  SMOE_RETURN_LAUNCH();
}
