// smoe_gemm.hip — dropless fp8 (OCP e4m3) grouped GEMM with 1x128 activation
// scales and 128x128 weight-block scales, for gfx950.
//
//   c[r,n] = bf16( sum_kb as[r,kb] * bs[e,n/128,kb] * sum_{k in kb} a[r,k]*b[e,n,k] )
//
// Tiling.  A workgroup of 256 threads (4 waves, 2x2) owns a 128-row x 128-col
// output tile of one expert; each wave owns 64 rows x 64 cols, i.e. 2x2
// blocks of the 32x32 fp8 MFMA (v_mfma_f32_32x32x64_f8f6f4).  The K loop steps
// one scale block (128) at a time: two MFMAs per 32x32 block produce the
// block's partial sum in fp32, which is then scaled by as[r,kb]*bs[e,nb,kb]
// and added to the fp32 accumulator.  Weight rows feed the MFMA's A operand
// and activation rows its B operand, so an output lane holds one activation
// row r (lane % 32): the activation scale is a per-lane value and the weight
// scale is uniform across the tile.
//
// Data movement.  Each K step loads a 128x128-byte activation tile and a
// 128x128-byte weight tile with 128-bit global loads, stores them to LDS with
// the 16-byte chunk index XOR-swizzled by (row & 7) so the 128-bit fragment
// reads of 8 consecutive rows hit distinct banks, and double-buffers LDS so
// the next step's global loads overlap this step's MFMAs (one barrier per
// step).
//
// Scheduling.  The grid covers an upper bound of m-tiles (ceil(R/128) + E)
// times the n-tiles; each workgroup derives the per-expert m-tile prefix sum
// from offsets[] in LDS (no host sync, no workspace) and leaves when its tile
// index is past the real total.  Zero-token experts own no tiles; rows past
// an expert's end are clamped on load and masked on store.
#include "smoe_common.h"

namespace smoe {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kBM = 128;  // activation rows per tile
constexpr int kBN = 128;  // output columns per tile
constexpr int kBK = 128;  // K per step (= scale block)
constexpr int kThreads = 256;
constexpr int kGroupM = 4;  // m-tiles per scheduling group (L2 reuse of weights)
constexpr int kTileBytes = kBK;                           // bytes per LDS row
constexpr int kStageBytes = (kBM + kBN) * kTileBytes;     // 32 KiB

__device__ __forceinline__ int swz(int row, int chunk) {
  return row * kTileBytes + ((chunk ^ (row & 7)) << 4);
}

__device__ __forceinline__ v16f mfma_f8(v8i a, v8i b, v16f c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

__device__ __forceinline__ v8i lds_frag(const uint8_t* base, int row, int c0) {
  const v4i lo = *(const v4i*)(base + swz(row, c0));
  const v4i hi = *(const v4i*)(base + swz(row, c0 + 1));
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

__global__ __launch_bounds__(kThreads) void grouped_gemm_fp8_kernel(
    const uint8_t* __restrict__ a, const float* __restrict__ as, const uint8_t* __restrict__ b,
    const float* __restrict__ bs, const int32_t* __restrict__ offsets, int E, int N, int Kd,
    int mt_bound, uint16_t* __restrict__ c) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * kStageBytes];
  __shared__ int mstart[SMOE_MAX_EXPERTS + 1];
  __shared__ int wsum[kThreads / kWave];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wid = tid >> 6;

  // ---- per-expert m-tile prefix sum (inclusive, mstart[e+1]) ------------
  // each thread owns experts [tid*per, tid*per+per)
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
  // wave inclusive scan of per-thread totals
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

  // ---- tile index: XCD-contiguous, then grouped-M order -----------------
  const int nblk = gridDim.x;  // multiple of 8
  const int bid = blockIdx.x;
  const int lin = (bid & 7) * (nblk >> 3) + (bid >> 3);
  const int NT = N / kBN;
  const int grp = lin / (kGroupM * NT);
  const int in_g = lin - grp * kGroupM * NT;
  const int mt = grp * kGroupM + (in_g % kGroupM);
  const int nt = in_g / kGroupM;
  if (mt >= total_mt || mt >= mt_bound) return;

  // expert owning m-tile mt: largest e with mstart[e] <= mt (binary search)
  int lo = 0, hi = E;  // mstart[lo] <= mt < mstart[hi]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (mstart[mid] <= mt) lo = mid;
    else hi = mid;
  }
  const int e = lo;
  const int row0 = offsets[e] + (mt - mstart[e]) * kBM;
  const int rows = min(kBM, offsets[e + 1] - row0);
  const int n0 = nt * kBN;
  const int ksb = Kd / kBK;

  // ---- global -> register loaders ---------------------------------------
  // thread t loads 4 chunks of each tile: row = i*32 + t/8, chunk = t%8
  const int lrow = tid >> 3, lch = tid & 7;
  const uint8_t* ga[4];
  const uint8_t* gb[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = min(i * 32 + lrow, rows - 1);
    ga[i] = a + (size_t)(row0 + r) * Kd + lch * 16;
    gb[i] = b + ((size_t)e * N + n0 + i * 32 + lrow) * Kd + lch * 16;
  }
  // per-lane activation scale rows for this wave's two 32-row blocks
  const int wr = wid >> 1, wn = wid & 1;
  const float* sa_ptr[2];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const int r = min(wr * 64 + rb * 32 + (lane & 31), rows - 1);
    sa_ptr[rb] = as + (size_t)(row0 + r) * ksb;
  }
  const float* sb_ptr = bs + ((size_t)e * (N / kGroup) + n0 / kGroup) * ksb;

  uint4 ra[4], rb_[4];
  float sa_n[2], sb_n;
  auto gload = [&](int kb) {
    const size_t ko = (size_t)kb * kBK;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ra[i] = *(const uint4*)(ga[i] + ko);
      rb_[i] = *(const uint4*)(gb[i] + ko);
    }
    sa_n[0] = sa_ptr[0][kb];
    sa_n[1] = sa_ptr[1][kb];
    sb_n = sb_ptr[kb];
  };
  auto lstore = [&](int buf) {
    uint8_t* sA = smem + buf * kStageBytes;
    uint8_t* sB = sA + kBM * kTileBytes;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *(uint4*)(sA + swz(i * 32 + lrow, lch)) = ra[i];
      *(uint4*)(sB + swz(i * 32 + lrow, lch)) = rb_[i];
    }
  };

  v16f acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  gload(0);
  lstore(0);
  float sa_c[2] = {sa_n[0], sa_n[1]};
  float sb_c = sb_n;
  __syncthreads();

  const int frow = lane & 31;
  const int fch = (lane >> 5) * 2;
  for (int kb = 0; kb < ksb; ++kb) {
    const int buf = kb & 1;
    if (kb + 1 < ksb) gload(kb + 1);
    const uint8_t* sA = smem + buf * kStageBytes;
    const uint8_t* sB = sA + kBM * kTileBytes;
    v8i fx[2][2], fw[2][2];
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        fx[i][kh] = lds_frag(sA, wr * 64 + i * 32 + frow, kh * 4 + fch);
        fw[i][kh] = lds_frag(sB, wn * 64 + i * 32 + frow, kh * 4 + fch);
      }
    }
    const v16f zero = {};
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        v16f p = mfma_f8(fw[nb][0], fx[rb][0], zero);
        p = mfma_f8(fw[nb][1], fx[rb][1], p);
        const float sc = sa_c[rb] * sb_c;
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[nb][rb][v] = __builtin_fmaf(p[v], sc, acc[nb][rb][v]);
      }
    }
    if (kb + 1 < ksb) {
      lstore(buf ^ 1);
      sa_c[0] = sa_n[0];
      sa_c[1] = sa_n[1];
      sb_c = sb_n;
    }
    __syncthreads();
  }

  // ---- epilogue: lane holds row (lane%32); v -> col 8*(v/4) + 4*(lane/32) + v%4
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const int rl = wr * 64 + rb * 32 + (lane & 31);
    if (rl >= rows) continue;
    uint16_t* crow = c + (size_t)(row0 + rl) * N + n0 + wn * 64 + (lane >> 5) * 4;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
      for (int vg = 0; vg < 4; ++vg) {
        const v16f& q = acc[nb][rb];
        uint2 o;
        o.x = f32_to_bf16(q[vg * 4 + 0]) | (f32_to_bf16(q[vg * 4 + 1]) << 16);
        o.y = f32_to_bf16(q[vg * 4 + 2]) | (f32_to_bf16(q[vg * 4 + 3]) << 16);
        *(uint2*)(crow + nb * 32 + vg * 8) = o;
      }
    }
  }
}

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
  if (N % kGroup || Kdim % kGroup) return SMOE_EINVAL_ALIGN128;
  SMOE_CHECK_PTR(a);
  SMOE_CHECK_PTR(b);
  SMOE_CHECK_PTR(c);
  if (!as || !bs || !offsets) return SMOE_EINVAL_NULL;
  if (((uintptr_t)as | (uintptr_t)bs | (uintptr_t)offsets) & 3u) return SMOE_EINVAL_PTRALIGN;
  const long long mt_bound = (R + kBM - 1) / kBM + E;
  const long long NT = N / kBN;
  // pad the m-tile count to whole scheduling groups, the grid to a multiple of 8
  const long long mt_pad = (mt_bound + kGroupM - 1) / kGroupM * kGroupM;
  long long nblk = mt_pad * NT;
  nblk = (nblk + 7) / 8 * 8;
  if (nblk > 0x7fffffffLL) return SMOE_EINVAL_DIM;
  grouped_gemm_fp8_kernel<<<dim3((unsigned)nblk), dim3(kThreads), 0, (hipStream_t)stream>>>(
      a, as, b, bs, offsets, E, N, Kdim, (int)mt_bound, c);
  SMOE_RETURN_LAUNCH();
}
