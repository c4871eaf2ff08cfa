// smoe_gemm_packed.hip — the dropless fp8 grouped GEMM of smoe_gemm.hip on
// weights prepacked in MFMA fragment order, for gfx950.
//
//   c[r,n] = bf16( sum_kb as[r,kb] * bs[e,n/128,kb] * sum_{k in kb} a[r,k]*b[e,n,k] )
//
// Same contract, tile order, expert scan and epilogues as smoe_gemm.hip; what
// differs is where the weights travel.  The outputs equal smoe_gemm.hip's
// whenever each K block's 128 products sum without rounding inside the MFMA
// (the case for every benchmark and layer workload measured); otherwise the
// two K orders below can differ in the last bf16 bit.
//
// Packed weights.  smoe_pack_weight_fp8 rewrites b [E,N,K] once as
// [E][N/16][K/128][2][64 lanes][16 B]: for 16 weight rows and one 128-wide K
// block, half h (0, 1) holds in lane l's 16 bytes row l%16 at K offsets
// h*64 + (l/16)*16 .. +16.  A wave then loads one MFMA operand (16 rows x 128
// K) as two fully coalesced 1 KiB global_load_dwordx4 straight into VGPRs.
// The activation fragment read from LDS uses the same K order (lane group g
// takes bytes 16g.. and 64+16g..), so each MFMA sums the same 128 products,
// in a different order.
//
// Tiling.  A workgroup of 8 waves owns a 256 x 256 output tile; wave w owns
// all 256 rows and columns w*32 .. +32 (16 row blocks x 2 column blocks of
// the 16x16x128 fp8 MFMA), so no two waves need the same weight bytes.  LDS
// holds only activations: a 4-stage ring of 256 x 128-byte tiles filled by
// direct global->LDS DMA three K steps ahead, plus the activation scales in
// double-buffered chunks of 8 K steps.  A wave's weights for step kb+2 are
// loaded into a ring of three register buffers while it computes step kb.
// The four activation DMAs and four weight loads of a step are spread over
// the row blocks, so a wave never waits long on a full load queue at once.
//
// The weight loads are ordinary loads: the compiler places the s_waitcnt
// before each use itself.  It does not count the activation DMAs (inline asm),
// which retire in the same in-order counter, so its waits can only wait
// longer than needed, never too little.  The DMAs are waited for by hand
// (vmcnt(8) at the end of a step, see there).
//
// Scope: K a multiple of 512 (the chunked activation scales); other K use the
// plain kernel (the ops layer and SimpleMoE choose).
#include "smoe_mfma.h"

namespace smoe {
namespace packed {

constexpr int kChipM = 32;              // scheduling group, as in smoe_gemm.hip
constexpr int kThreads = 512, kWaves = 8, kBM = 256, kBN = 256;
constexpr int kRB = 16, kCB = 2;        // row blocks x column blocks per wave
constexpr int kAS = 4;                  // activation stages (DMA three steps ahead)
constexpr int kABytes = kBM * kRow;     // 32 KiB per stage
constexpr int kSChunk = 8;              // K steps per activation-scale chunk
constexpr int kSCBytes = kBM * kSChunk * 4;
constexpr int kCPitch = kBN * 2 + 16;   // bytes per staged bf16 output row
constexpr int kSC0 = kAS * kABytes;     // scale chunk area
constexpr int kLoop = kSC0 + 2 * kSCBytes;
constexpr int kSmem = kLoop > kBM * kCPitch ? kLoop : kBM * kCPitch;
static_assert(kSmem + 4200 <= 160 * 1024, "LDS budget");
static_assert(kSCBytes == kWaves * 1024, "one 1 KiB scale DMA per wave and chunk");

// Packing: one 16-byte slot per thread and iteration, in packed order.
__global__ __launch_bounds__(256) void pack_kernel(const uint8_t* __restrict__ w, int E, int N,
                                                   int Kd, uint8_t* __restrict__ p) {
  const size_t total = (size_t)E * N * Kd / 16;
  const int ksb = Kd / kBK;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const int lane = (int)(i & 63);
    const int h = (int)((i >> 6) & 1);
    size_t rest = i >> 7;  // (e, nb, kb)
    const int kb = (int)(rest % ksb);
    rest /= ksb;
    const int nb = (int)(rest % (N / 16));
    const int e = (int)(rest / (N / 16));
    const int n = nb * 16 + (lane & 15);
    const int k = kb * kBK + h * 64 + (lane >> 4) * 16;
    *(uint4*)(p + i * 16) = *(const uint4*)(w + ((size_t)e * N + n) * Kd + k);
  }
}

typedef v4i WBuf[kCB][2];  // one step's weight operands of a wave

// s_waitcnt vmcnt(n) lgkmcnt(0) (expcnt not waited on); on gfx950 vmcnt's
// low 4 bits sit in [3:0] and its high 2 bits in [15:14].
template <int n>
__device__ __forceinline__ void wait_vm(){
  static_assert(n >= 0 && n < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((n & 15) | (7 << 4) | ((n >> 4) << 14));
}

// activation fragment in the packed weights' K order
__device__ __forceinline__ v8i lds_frag_p(const uint8_t* base, int row, int g) {
  const v4i lo = *(const v4i*)(base + swz(row, g));
  const v4i hi = *(const v4i*)(base + swz(row, g + 4));
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// kSwiGLU: b is W1 packed [E, 2I, K]; tile nt pairs gate columns nt*128 ..
// +128 (waves 0-3) with up columns I + nt*128 .. +128 (waves 4-7) and the
// epilogue writes hq, hs (and c1 when c is not null) exactly as the fused
// epilogue of smoe_gemm.hip does.
template <bool kSwiGLU>
__global__ __launch_bounds__(kThreads, 1) void grouped_gemm_fp8_packed_kernel(
    const uint8_t* __restrict__ a, const float* __restrict__ as, const uint8_t* __restrict__ bp,
    const float* __restrict__ bs, const int32_t* __restrict__ offsets, int E, int R, int N, int Kd,
    int mt_bound, uint16_t* __restrict__ c, uint8_t* __restrict__ hq, float* __restrict__ hs) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kSmem];
  __shared__ int mstart[SMOE_MAX_EXPERTS + 1];
  __shared__ int wsum[kWaves];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wid = tid >> 6;

  // ---- per-expert m-tile prefix sum (as in smoe_gemm.hip) ----------------
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

  // ---- activation DMA: wave w fills 1 KiB segments w*4 .. w*4+3 of a stage
  // (8 rows each, layout and clamping as in smoe_gemm.hip)
  const uint8_t* a_base = a + (size_t)row0 * Kd;
  const float* s_base = as + (size_t)row0 * ksb;
  uint32_t oa[4];
  {
    const int slot = lane & 7;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = tile_row((wid * 4 + j) * 8 + (lane >> 3));
      oa[j] = (uint32_t)(min(row, rows - 1) * Kd + ((slot ^ (row & 7)) << 4));
    }
  }
  // scale chunk DMA: lane l of wave w moves 16 bytes (4 K steps) of tile row
  // w*32 + l/2 (the second half of a chunk past ksb re-reads the first)
  const uint32_t osc = (uint32_t)(min(wid * 32 + (lane >> 1), rows - 1) * ksb) * 4u;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_ptr_t)smem;
  const uint32_t a_lds = __builtin_amdgcn_readfirstlane(lds0 + wid * 4 * 1024);
  const uint32_t sc_lds = __builtin_amdgcn_readfirstlane(lds0 + kSC0 + wid * 1024);
  auto issue_sc = [&](int chunk) __attribute__((always_inline)) {
    const bool second = (lane & 1) && (chunk + 1) * kSChunk <= ksb;
    dma16(s_base + chunk * kSChunk, osc + (second ? 16u : 0u), sc_lds + (chunk & 1) * kSCBytes);
  };
  // ---- packed weights: wave w's two 16-row blocks of weight rows
  const uint8_t* b_base = bp + (size_t)e * ((size_t)N * Kd);
  uint32_t ob[kCB];
#pragma unroll
  for (int j = 0; j < kCB; ++j) {
    int wr0;  // first weight row of this column block
    if constexpr (kSwiGLU)
      wr0 = wid < 4 ? nt * kGroup + wid * 32 + j * 16 : I + nt * kGroup + (wid - 4) * 32 + j * 16;
    else
      wr0 = min(n0 + wid * 32 + j * 16, N - 16);  // columns past N: clamped, never stored
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
  WBuf fA, fB, fC;
  issue_sc(0);
#pragma unroll
  for (int s = 0; s < kAS - 1; ++s) {
    const int ks = min(s, ksb - 1);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      dma16(a_base + (size_t)ks * kBK, oa[q], a_lds + s * kABytes + q * 1024);
  }
  load_b(0, fA);
  load_b(min(1, ksb - 1), fB);
  // the tile's weight-block scales go to LDS (the expert table's space)
  constexpr int kNB128 = kBN / kGroup;
  const int NB = (N + kGroup - 1) / kGroup;  // weight-scale blocks per expert (last may be short)
  float* sbt = (float*)mstart;
  __syncthreads();
  for (int i = tid; i < kNB128 * ksb; i += kThreads) {
    const int nb = i / ksb, kb = i - nb * ksb;
    const int blk = kSwiGLU ? (nb == 0 ? nt : I / kGroup + nt)
                            : min(n0 / kGroup + nb, NB - 1);
    sbt[i] = bs[((size_t)e * NB + blk) * ksb + kb];
  }
  __syncthreads();
  const float* sb_row = sbt + ((wid * 32) / kGroup) * ksb;
  wait_vm<0>();
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

  // ---- one K step: weights of step kb in cur, step kb+1's (loaded during
  // step kb-1) in nx1, step kb+2's loaded into nx2.  Activation DMAs go out
  // before row blocks 0, 4, 8, 12 and weight loads before 1, 5, 9, 13.
  // Past the last step the loads repeat step ksb-1's data into buffers and
  // stages no later step reads, so the count of loads in flight is the same
  // every step (the waits below count on it).
  auto step = [&](int kb, WBuf& cur, WBuf& nx1, WBuf& nx2) __attribute__((always_inline)) {
    if ((kb & (kSChunk - 1)) == 0 && kb + kSChunk < ksb) issue_sc(kb / kSChunk + 1);
    const int ka = min(kb + kAS - 1, ksb - 1);
    const uint32_t a_dst = a_lds + (uint32_t)((kb + kAS - 1) % kAS) * kABytes;
    const uint8_t* a_src = a_base + (size_t)ka * kBK;
    const uint8_t* b_src = b_base + (size_t)min(kb + 2, ksb - 1) * 2048;
    const uint8_t* sA = smem + (kb % kAS) * kABytes;
    const float* sC = (const float*)(smem + kSC0 + ((kb / kSChunk) & 1) * kSCBytes) +
                      (kb & (kSChunk - 1));
    const float sb = sb_row[kb];
    v8i fw[kCB];
#pragma unroll
    for (int j = 0; j < kCB; ++j)
      fw[j] = __builtin_shufflevector(cur[j][0], cur[j][1], 0, 1, 2, 3, 4, 5, 6, 7);
    v8i fx = lds_frag_p(sA, frow, fg);
    // software pipeline over row blocks: block i's MFMAs, then block i-1's
    // scale FMAs.  The empty asm statements order them (the MFMA builtin has
    // no side effects, and without them the compiler hoists every MFMA of
    // the step and holds all 32 results at once).
    v4f pp[kCB];
    float scp = 0.0f;
#pragma unroll
    for (int i = 0; i < kRB; ++i) {
      if ((i & 3) == 0) dma16(a_src, oa[i >> 2], a_dst + (i >> 2) * 1024);
      if ((i & 3) == 1) {
        const int q = i >> 2;  // weight load q: column block q >> 1, half q & 1
        nx2[q >> 1][q & 1] = *(const v4i*)(b_src + ob[q >> 1] + (q & 1) * 1024);
      }
      v8i fxn = fx;
      if (i + 1 < kRB) fxn = lds_frag_p(sA, (i + 1) * 16 + frow, fg);
      const float sc = sC[(i * 16 + frow) * kSChunk] * sb;
      asm volatile("" : "+v"(fx));
      v4f p[kCB];
#pragma unroll
      for (int j = 0; j < kCB; ++j) p[j] = mfma16(fw[j], fx, v4f{0.0f, 0.0f, 0.0f, 0.0f});
      if (i > 0) {
#pragma unroll
        for (int j = 0; j < kCB; ++j)
#pragma unroll
          for (int v = 0; v < 4; ++v)
            acc[i - 1][j][v] = __builtin_fmaf(pp[j][v], scp, acc[i - 1][j][v]);
        asm volatile("" : "+v"(acc[i - 1][0]), "+v"(acc[i - 1][1]));
      }
#pragma unroll
      for (int j = 0; j < kCB; ++j) pp[j] = p[j];
      scp = sc;
      fx = fxn;
    }
#pragma unroll
    for (int j = 0; j < kCB; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[kRB - 1][j][v] = __builtin_fmaf(pp[j][v], scp, acc[kRB - 1][j][v]);
    // Activation stage kb+1 was issued during step kb-2; at least the 8 loads
    // of step kb-1 (4 DMAs, and 4 weight loads the next step reads) came after
    // it, so vmcnt(8) covers it, and the scale chunks, which are older.  (The
    // compiler may drop this step's weight loads in the last steps, where
    // nothing reads them; the count after stage kb+1 stays >= 8.)  The barrier
    // then makes every wave's stage kb+1 visible and frees stage kb.
    wait_vm<8>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  int kb = 0;
  for (; kb + 2 < ksb; kb += 3) {
    step(kb, fA, fB, fC);
    step(kb + 1, fB, fC, fA);
    step(kb + 2, fC, fA, fB);
  }
  if (kb < ksb) step(kb, fA, fB, fC);
  if (kb + 1 < ksb) step(kb + 1, fB, fC, fA);
  // every wave's trailing activation DMAs have landed before any wave writes
  // its output tile over the stage buffers
  wait_vm<0>();
  __syncthreads();

  // ---- epilogue: bf16 tile staged in LDS, then written row by row --------
  uint8_t* ct = smem;
#pragma unroll
  for (int i = 0; i < kRB; ++i) {
    const int rl = i * 16 + frow;
    const int cl = wid * 32 + (lane >> 4) * 4;
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

}  // namespace packed
}  // namespace smoe

using namespace smoe;

extern "C" int smoe_pack_weight_fp8(const uint8_t* wq, int E, int N, int Kdim, uint8_t* wp,
                                    void* stream) {
  if (N <= 0 || Kdim <= 0) return SMOE_EINVAL_DIM;
  if (E <= 0 || E > SMOE_MAX_EXPERTS) return SMOE_EINVAL_EXPERTS;
  if (N % kLane || Kdim % kGroup) return SMOE_EINVAL_ALIGN128;
  SMOE_CHECK_PTR(wq);
  SMOE_CHECK_PTR(wp);
  const long long slots = (long long)E * N * Kdim / 16;
  const int blocks = (int)std::min<long long>((slots + 255) / 256, 8192);
  packed::pack_kernel<<<dim3(blocks), dim3(256), 0, (hipStream_t)stream>>>(wq, E, N, Kdim, wp);
  SMOE_RETURN_LAUNCH();
}

namespace {
int packed_args(const uint8_t* a, const float* as, const uint8_t* wp, const float* ws,
                const int32_t* offsets, int E, int R, int N, int Kdim) {
  if (R <= 0 || N <= 0 || Kdim <= 0) return SMOE_EINVAL_DIM;
  if (E <= 0 || E > SMOE_MAX_EXPERTS) return SMOE_EINVAL_EXPERTS;
  if (N % kLane || Kdim % (4 * kBK)) return SMOE_EINVAL_ALIGN128;  // K: a multiple of 512
  if (Kdim > 65536) return SMOE_EINVAL_DIM;  // weight-scale table fits the LDS expert table
  if ((long long)N * Kdim >= (1LL << 32)) return SMOE_EINVAL_DIM;  // 32-bit weight offsets
  SMOE_CHECK_PTR(a);
  SMOE_CHECK_PTR(wp);
  if (!as || !ws || !offsets) return SMOE_EINVAL_NULL;
  if (((uintptr_t)as | (uintptr_t)ws | (uintptr_t)offsets) & 3u) return SMOE_EINVAL_PTRALIGN;
  return SMOE_OK;
}
long long packed_grid(int E, int R, int NT, long long* mt_bound) {
  *mt_bound = (R + packed::kBM - 1) / packed::kBM + E;
  const long long mt_pad = (*mt_bound + packed::kChipM - 1) / packed::kChipM * packed::kChipM;
  return (mt_pad * NT + 7) / 8 * 8;
}
}  // namespace

extern "C" int smoe_grouped_gemm_fp8_packed(const uint8_t* a, const float* as, const uint8_t* wp,
                                            const float* ws, const int32_t* offsets, int E, int R,
                                            int N, int Kdim, uint16_t* c, void* stream) {
  const int st = packed_args(a, as, wp, ws, offsets, E, R, N, Kdim);
  if (st) return st;
  SMOE_CHECK_PTR(c);
  long long mt_bound;
  const long long nblk = packed_grid(E, R, (N + packed::kBN - 1) / packed::kBN, &mt_bound);
  if (nblk > 0x7fffffffLL) return SMOE_EINVAL_DIM;
  packed::grouped_gemm_fp8_packed_kernel<false>
      <<<dim3((unsigned)nblk), dim3(packed::kThreads), 0, (hipStream_t)stream>>>(
          a, as, wp, ws, offsets, E, R, N, Kdim, (int)mt_bound, c, nullptr, nullptr);
  SMOE_RETURN_LAUNCH();
}

extern "C" int smoe_grouped_gemm_fp8_packed_swiglu(const uint8_t* a, const float* as,
                                                   const uint8_t* w1p, const float* w1s,
                                                   const int32_t* offsets, int E, int R, int I,
                                                   int Kdim, uint8_t* hq, float* hs, uint16_t* c1,
                                                   void* stream) {
  if (I <= 0) return SMOE_EINVAL_DIM;
  if (I % kGroup) return SMOE_EINVAL_ALIGN128;
  const int st = packed_args(a, as, w1p, w1s, offsets, E, R, 2 * I, Kdim);
  if (st) return st;
  SMOE_CHECK_PTR(hq);
  if (c1 && ((uintptr_t)c1 & 15u)) return SMOE_EINVAL_PTRALIGN;
  if (!hs) return SMOE_EINVAL_NULL;
  if ((uintptr_t)hs & 3u) return SMOE_EINVAL_PTRALIGN;
  long long mt_bound;
  const long long nblk = packed_grid(E, R, I / kGroup, &mt_bound);
  if (nblk > 0x7fffffffLL) return SMOE_EINVAL_DIM;
  packed::grouped_gemm_fp8_packed_kernel<true>
      <<<dim3((unsigned)nblk), dim3(packed::kThreads), 0, (hipStream_t)stream>>>(
          a, as, w1p, w1s, offsets, E, R, 2 * I, Kdim, (int)mt_bound, c1, hq, hs);
  SMOE_RETURN_LAUNCH();
}
