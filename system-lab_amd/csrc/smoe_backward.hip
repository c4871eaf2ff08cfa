// smoe_backward.hip — the backward-pass data kernels of the SimpleMoE expert
// layer on gfx950: blockwise fp8 weight transpose (dgrad operands), 128x1
// column quantisation into transposed, expert-segment-aligned layout (wgrad
// operands), SwiGLU backward and combine backward.
#include "smoe_common.h"

namespace smoe {

typedef uint32_t v4u __attribute__((ext_vector_type(4)));

// ------------------------------------------------------ weight transpose
// [E, N, Kp] fp8 (Kp = pad128(Kd), columns past Kd zero) -> [E, Kd, Np]
// (Np = pad128(N), columns past N zero).  One 256-thread workgroup per
// 64x64-byte tile: each thread loads 16 bytes of a source row into LDS (row
// stride 80 bytes keeps the column reads spread over banks; source rows past
// N read as zeros), then assembles 16 bytes of a destination row from 16 LDS
// bytes of one source column (destination rows past Kd are not written).
__global__ __launch_bounds__(256) void transpose_fp8_kernel(const uint8_t* __restrict__ src,
                                                            int N, int Kd,
                                                            uint8_t* __restrict__ dst) {
  __shared__ uint8_t tile[64][80];
  const int Kp = pad128(Kd), Np = pad128(N);
  const int tk = blockIdx.x, tn = blockIdx.y, e = blockIdx.z;
  const int t = threadIdx.x;
  const int r = t >> 2, c16 = (t & 3) * 16;
  const int n = tn * 64 + r;
  uint4 v = make_uint4(0, 0, 0, 0);
  if (n < N) v = *(const uint4*)(src + ((size_t)e * N + n) * Kp + tk * 64 + c16);
  *(uint4*)&tile[r][c16] = v;
  __syncthreads();
  // destination row k = tk*64 + r, columns n = tn*64 + c16 .. +16
  uint32_t w[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    w[q] = (uint32_t)tile[c16 + 4 * q][r] | ((uint32_t)tile[c16 + 4 * q + 1][r] << 8) |
           ((uint32_t)tile[c16 + 4 * q + 2][r] << 16) | ((uint32_t)tile[c16 + 4 * q + 3][r] << 24);
  }
  const int k = tk * 64 + r;
  if (k < Kd)
    *(uint4*)(dst + ((size_t)e * Kd + k) * Np + tn * 64 + c16) = make_uint4(w[0], w[1], w[2], w[3]);
}

// [E, NB, KB] f32 -> [E, KB, NB]
__global__ __launch_bounds__(256) void transpose_scales_kernel(const float* __restrict__ s,
                                                               int E, int NB, int KB,
                                                               float* __restrict__ d) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long long)E * NB * KB) return;
  const int e = (int)(i / ((long long)NB * KB));
  const int rem = (int)(i - (long long)e * NB * KB);
  const int nb = rem / KB, kb = rem - nb * KB;
  d[((size_t)e * KB + kb) * NB + nb] = s[i];
}

// ---------------------------------------------------- padded segments
// pad[e+1] = pad[e] + ceil(count_e / 128) * 128, one workgroup.
__global__ __launch_bounds__(1024) void pad_offsets_kernel(const int32_t* __restrict__ offsets,
                                                           int E, int32_t* __restrict__ pad) {
  __shared__ int part[1024];
  const int t = threadIdx.x;
  int v = 0;
  if (t < E) v = (offsets[t + 1] - offsets[t] + kGroup - 1) / kGroup * kGroup;
  part[t] = v;
  __syncthreads();
  for (int o = 1; o < 1024; o <<= 1) {
    const int u = t >= o ? part[t - o] : 0;
    __syncthreads();
    part[t] += u;
    __syncthreads();
  }
  if (t < E) pad[t + 1] = part[t];
  if (t == 0) pad[0] = 0;
}

// --------------------------------------------- 128x1 column quantisation
// One 256-thread workgroup per (128-row group, 128-column slab).  The group's
// rows (an expert's rows split into 128-row groups from its first row; short
// last groups are zero-padded) are loaded with non-temporal 128-bit loads,
// optionally gathered through p = gather[r] as row p / gather_div and
// optionally weighted by gather_w[p] (bf16(w * x)).  All 8 loads of a thread
// are issued before any is used.  Thread t owns 8
// columns (t % 16) * 8 .. +8 of the 8 consecutive rows (t / 16) * 8 .. +8, so
// everything stays in registers: the column amax is a local max over the 8
// rows, an xor shuffle over the 4 row groups of a wave, and a 2 KB LDS
// exchange over the 4 waves; one thread per column then derives the scale
// and the quotient set-up for all, and each thread quantises its 64 values
// with the division-free bf16 quantiser and writes, per column, its 8 rows as one
// 8-byte store into the transposed output (ld bytes per column).  The 16
// stores that cover one column's 128 bytes merge in L2.
constexpr int kQcCols = 128;

// kRows: also quantise the same tile 1x128 along rows (the dgrad operand),
// written to qr [R, C] / sr [R, C/128] exactly as smoe_quant_rows_1x128 would,
// so a tensor needed both ways is read once.
// kSwigluBwd: the tiles are not read from x but computed: x is dc1 [R, 2I] =
// [dg | du], the SwiGLU backward of c1 [R, 2I] and dh [R, I], with the same
// fp32 operations and bf16 rounding as swiglu_bwd_kernel (C = 2I).  A
// workgroup takes column block b of both halves, so slabs b (dg) and
// I/128 + b (du) come from one sigmoid evaluation.  dc1 is written only when
// not null.
// kPow2: the 128x1 column scales are group_scale_pow2 (the optional E8M0
// recipe of the wgrad operands) instead of group_scale; kRowPow2 likewise for
// the 1x128 row scales (kRows).
template <bool kRows, bool kSwigluBwd, bool kPow2, bool kRowPow2 = false>
__global__ __launch_bounds__(256) void quant_cols_kernel(
    const uint16_t* __restrict__ x, const int32_t* __restrict__ gather, int gather_div,
    const float* __restrict__ gather_w, int R, int C, const int32_t* __restrict__ offsets, const int32_t* __restrict__ pad, int E, int ld,
    uint8_t* __restrict__ q, float* __restrict__ s, uint8_t* __restrict__ qr,
    float* __restrict__ sr, const uint16_t* __restrict__ c1, const uint16_t* __restrict__ dh,
    uint16_t* __restrict__ dc1) {
  __shared__ int pad_l[SMOE_MAX_EXPERTS + 1];
  __shared__ float wmax[4][kQcCols];
  __shared__ float col_m[kQcCols], col_r[kQcCols];  // per-column quotient set-up
  __shared__ int col_e[kQcCols];
  __shared__ float row_m[kQcCols], row_r[kQcCols];  // per-row set-up (kRows)
  __shared__ int row_e[kQcCols];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  for (int i = t; i <= E; i += 256) pad_l[i] = pad[i];
  __syncthreads();
  const int gpos = blockIdx.y * kGroup;  // position in the padded row space
  if (gpos >= pad_l[E]) return;          // whole workgroup leaves together
  int lo = 0, hi = E;                    // largest e with pad[e] <= gpos
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (pad_l[mid] <= gpos) lo = mid;
    else hi = mid;
  }
  const int e = lo;
  const int row0 = offsets[e] + (gpos - pad_l[e]);
  // rows outside [0, R) are never read, whatever offsets[] holds (the group
  // then quantises as zero padding)
  const int valid = row0 < 0 ? 0 : min(kGroup, min(offsets[e + 1], R) - row0);
  const int cc = (t & 15) * 8;  // this thread's 8 columns
  const int rg = t >> 4;        // this thread's rows rg*8 .. rg*8+7
  // quantise one 128x128 tile (v: this thread's 8 rows x 8 columns) whose
  // columns start at c0, 128x1 along columns and (kRows) 1x128 along rows
  auto quantize = [&](const v4u (&v)[8], const int c0) {
    // column amax: 8 rows here, then the 4 row groups of this wave, then waves
    float cmax[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) cmax[i] = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t wd[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        cmax[2 * i] = fmaxf(cmax[2 * i], fabsf(__uint_as_float(wd[i] << 16)));
        cmax[2 * i + 1] = fmaxf(cmax[2 * i + 1], fabsf(__uint_as_float(wd[i] & 0xffff0000u)));
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      cmax[i] = fmaxf(cmax[i], __shfl_xor(cmax[i], 16, kWave));
      cmax[i] = fmaxf(cmax[i], __shfl_xor(cmax[i], 32, kWave));
    }
    if (lane < 16) {
#pragma unroll
      for (int i = 0; i < 8; ++i) wmax[w][cc + i] = cmax[i];
    }
    if constexpr (kRows) {
      // row amax of each 1x128 group: this thread's 8 columns, then the 16
      // threads that share the row; lane j of the 16 derives row rg*8+j's set-up
      float rmax[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t wd[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
        float m = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          m = fmaxf(m, fabsf(__uint_as_float(wd[i] << 16)));
          m = fmaxf(m, fabsf(__uint_as_float(wd[i] & 0xffff0000u)));
        }
        rmax[j] = row16_max(m);
      }
      const int j = t & 15;
      if (j < 8) {
        float am = rmax[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) am = (j == i) ? rmax[i] : am;
        const float sc = scale_of<kRowPow2>(am);
        const QDiv qd = qdiv_setup_t<kRowPow2>(sc);
        const int r = rg * 8 + j;
        row_m[r] = qd.m;
        row_r[r] = qd.r;
        row_e[r] = qd.e;
        if (r < valid) sr[(size_t)(row0 + r) * (pad128(C) / kGroup) + c0 / kGroup] = sc;
      }
    }
    __syncthreads();
    // one thread per column finishes the amax, derives the scale and the
    // quotient set-up (two IEEE divisions) and shares them: the 16 threads
    // that hold pieces of a column would otherwise repeat the divisions
    if (t < kQcCols) {
      const float am = fmaxf(fmaxf(wmax[0][t], wmax[1][t]), fmaxf(wmax[2][t], wmax[3][t]));
      const float sc = scale_of<kPow2>(am);
      const QDiv qd = qdiv_setup_t<kPow2>(sc);
      col_m[t] = qd.m;
      col_r[t] = qd.r;
      col_e[t] = qd.e;
      if (c0 + t < C) s[(size_t)(c0 + t) * (ld / kGroup) + gpos / kGroup] = sc;
    }
    __syncthreads();
    QDiv d[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      d[i].m = col_m[cc + i];
      d[i].r = col_r[cc + i];
      d[i].e = col_e[cc + i];
    }
    // column c0+cc+i gets bytes for rows gpos + rg*8 .. +8 (columns past C
    // have no output row)
    uint8_t* dst = q + (size_t)(c0 + cc) * ld + gpos + rg * 8;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (c0 + cc >= C) break;
      float qv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t wd = (i & 1) ? (v[j][i >> 1] & 0xffff0000u) : (v[j][i >> 1] << 16);
        qv[j] = quot_t<kPow2>(__uint_as_float(wd), d[i]);
      }
      const uint32_t b[2] = {e4m3_pack4(qv[0], qv[1], qv[2], qv[3]),
                             e4m3_pack4(qv[4], qv[5], qv[6], qv[7])};
      *(uint2*)(dst + (size_t)i * ld) = make_uint2(b[0], b[1]);
    }
    if constexpr (kRows) {
      // row r's 8 bytes at columns c0+cc .. +8 (16 threads cover the group)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int r = rg * 8 + j;
        if (r >= valid) break;
        QDiv rd;
        rd.m = row_m[r];
        rd.r = row_r[r];
        rd.e = row_e[r];
        float qv[8];
        const uint32_t wd[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          qv[2 * i] = quot_t<kRowPow2>(__uint_as_float(wd[i] << 16), rd);
          qv[2 * i + 1] = quot_t<kRowPow2>(__uint_as_float(wd[i] & 0xffff0000u), rd);
        }
        *(uint2*)(qr + (size_t)(row0 + r) * pad128(C) + c0 + cc) =
            make_uint2(e4m3_pack4(qv[0], qv[1], qv[2], qv[3]), e4m3_pack4(qv[4], qv[5], qv[6], qv[7]));
      }
    }
  };

  if constexpr (kSwigluBwd) {
    // column block b of both halves: the sigmoid is computed once per (row,
    // column) and gives dg (slab b) and du (slab I/128 + b)
    const int I = C / 2, nI = I / kGroup;
    const int col = (int)blockIdx.x * kGroup + cc;
    v4u vG[8], vU[8], vD[8];
    // all 24 loads issued before any arithmetic (unconditional; rows outside
    // the group re-read a valid row and are zeroed after)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const size_t row = valid > 0 ? (size_t)(row0 + min(rg * 8 + j, valid - 1)) : 0;
      vG[j] = __builtin_nontemporal_load((const v4u*)(c1 + row * 2 * I + col));
      vU[j] = __builtin_nontemporal_load((const v4u*)(c1 + row * 2 * I + I + col));
      vD[j] = __builtin_nontemporal_load((const v4u*)(dh + row * I + col));
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int r = rg * 8 + j;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float og[2], ou[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float g = h ? __uint_as_float(vG[j][i] & 0xffff0000u) : __uint_as_float(vG[j][i] << 16);
          const float u = h ? __uint_as_float(vU[j][i] & 0xffff0000u) : __uint_as_float(vU[j][i] << 16);
          const float d = h ? __uint_as_float(vD[j][i] & 0xffff0000u) : __uint_as_float(vD[j][i] << 16);
          const float sg = recip_rn(1.0f + expf32(-g));  // = the IEEE 1 / b (smoe_selftest_recip)
          const float silu = g * sg;
          const float ds = sg * (1.0f + g * (1.0f - sg));
          ou[h] = d * silu;
          og[h] = (d * u) * ds;
        }
        vG[j][i] = bf16_pack2(og[0], og[1]);
        vU[j][i] = bf16_pack2(ou[0], ou[1]);
      }
      if (r < valid) {
        if (dc1) {
          const size_t row = (size_t)(row0 + r);
          *(v4u*)(dc1 + row * 2 * I + col) = vG[j];
          *(v4u*)(dc1 + row * 2 * I + I + col) = vU[j];
        }
      } else {
        vG[j] = vU[j] = v4u{0u, 0u, 0u, 0u};
      }
    }
    quantize(vG, (int)blockIdx.x * kGroup);
    __syncthreads();  // the second tile reuses the LDS exchange arrays
    quantize(vU, (nI + (int)blockIdx.x) * kGroup);
  } else {
    v4u v[8];
    float wv[8];
    const int c0 = blockIdx.x * kQcCols;
    // a thread whose 8 columns lie past C (C % 128 != 0) reads column 0 and
    // is zeroed below, like a row outside the group
    const bool col_ok = c0 + cc < C;
    const int ccl = col_ok ? c0 + cc : 0;
    // Loads are unconditional (out-of-group rows re-read the group's last
    // row, or row 0 when the group is empty) and zeroed by selects after, so
    // no control flow separates them and all 8 are in flight at once.
    int src[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int r = rg * 8 + j;
      src[j] = valid > 0 ? row0 + min(r, valid - 1) : 0;
    }
    bool ok[8];
    if (gather) {
      // gathered rows whose map entry lies outside [0, R) stay zero
#pragma unroll
      for (int j = 0; j < 8; ++j) src[j] = gather[src[j]];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        ok[j] = rg * 8 + j < valid && (unsigned)src[j] < (unsigned)R;
        src[j] = (unsigned)src[j] < (unsigned)R ? src[j] : 0;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = *(const v4u*)(x + (size_t)(src[j] / gather_div) * C + ccl);
      if (gather_w) {
#pragma unroll
        for (int j = 0; j < 8; ++j) wv[j] = gather_w[src[j]];
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        ok[j] = rg * 8 + j < valid;
        v[j] = __builtin_nontemporal_load((const v4u*)(x + (size_t)src[j] * C + ccl));
      }
    }
    if (gather && gather_w) {
      // the weighted rows bf16(w[p] * x[p / gather_div]), rounded as
      // combine_bwd_kernel rounds dy
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          v[j][i] = bf16_pack2(wv[j] * __uint_as_float(v[j][i] << 16),
                               wv[j] * __uint_as_float(v[j][i] & 0xffff0000u));
    }
    // rows outside the group and columns past C are +0 (after the weights:
    // w * +0 can be -0)
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (!ok[j] || !col_ok) v[j] = v4u{0u, 0u, 0u, 0u};
    quantize(v, c0);
  }
}

// ------------------------------------------------------- SwiGLU backward
// One wave per row; a lane owns 8 consecutive columns of a 512-column chunk.
// s = 1/(1+exp(-g)); du = dh*(g*s); dg = (dh*u) * (s*(1 + g*(1-s))).
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(const uint16_t* __restrict__ c1,
                                                         const uint16_t* __restrict__ dh, int R,
                                                         int I, uint16_t* __restrict__ dc1) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= R) return;
  const uint16_t* grow = c1 + (size_t)r * 2 * I;
  for (int col = lane * 8; col < I; col += kWave * 8) {
    const uint4 vg = *(const uint4*)(grow + col);
    const uint4 vu = *(const uint4*)(grow + I + col);
    const uint4 vd = *(const uint4*)(dh + (size_t)r * I + col);
    const uint32_t g4[4] = {vg.x, vg.y, vg.z, vg.w};
    const uint32_t u4[4] = {vu.x, vu.y, vu.z, vu.w};
    const uint32_t d4[4] = {vd.x, vd.y, vd.z, vd.w};
    uint32_t og[4], ou[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float gb[2], ub[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float g = h ? __uint_as_float(g4[i] & 0xffff0000u) : __uint_as_float(g4[i] << 16);
        const float u = h ? __uint_as_float(u4[i] & 0xffff0000u) : __uint_as_float(u4[i] << 16);
        const float d = h ? __uint_as_float(d4[i] & 0xffff0000u) : __uint_as_float(d4[i] << 16);
        const float s = recip_rn(1.0f + expf32(-g));  // = the IEEE 1 / b (smoe_selftest_recip)
        const float silu = g * s;
        const float ds = s * (1.0f + g * (1.0f - s));
        ub[h] = d * silu;
        gb[h] = (d * u) * ds;
      }
      og[i] = bf16_pack2(gb[0], gb[1]);
      ou[i] = bf16_pack2(ub[0], ub[1]);
    }
    uint16_t* orow = dc1 + (size_t)r * 2 * I;
    *(uint4*)(orow + col) = make_uint4(og[0], og[1], og[2], og[3]);
    *(uint4*)(orow + I + col) = make_uint4(ou[0], ou[1], ou[2], ou[3]);
  }
}

// ------------------------------------------------------ combine backward
// One wave per token: reads dout[t] once, and for each of its K rows writes
// dy[r] = bf16(w[t,k] * dout[t]) and reduces dw[t,k] = <dout[t], y[r]> in
// fp32 (lane partials over the row, then a wave tree).
// kQuant: dy is not stored; its 1x128 row quantisation goes to dyq [T*K, H]
// / dys [T*K, H/128] instead (the 16 lanes that hold a 128-column group
// share its amax), the bytes smoe_quant_rows_1x128 would write from dy.
template <int kMaxK, bool kQuant, bool kRowPow2 = false>
__global__ __launch_bounds__(256) void combine_bwd_kernel(
    const uint16_t* __restrict__ dout, const uint16_t* __restrict__ y,
    const int32_t* __restrict__ inv_map, const float* __restrict__ w, int T, int K, int H,
    uint16_t* __restrict__ dy, float* __restrict__ dw, uint8_t* __restrict__ dyq,
    float* __restrict__ dys) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int R = T * K;
  int r[kMaxK];
  float wk[kMaxK], part[kMaxK];
#pragma unroll
  for (int k = 0; k < kMaxK; ++k) {
    part[k] = 0.0f;
    if (k < K) {
      r[k] = inv_map[(size_t)t * K + k];
      wk[k] = w[(size_t)t * K + k];
    }
  }
  // kQuant walks the 128-padded row (Hp) so that each 16-lane group covers
  // one whole quantisation group: columns past H read nothing (zeros) and
  // quantise to byte 0
  const int Hp = kQuant ? pad128(H) : H;
  for (int col = lane * 8; col < Hp; col += kWave * 8) {
    const bool in = col < H;
    const uint4 vd = in ? *(const uint4*)(dout + (size_t)t * H + col) : make_uint4(0, 0, 0, 0);
    const uint32_t d4[4] = {vd.x, vd.y, vd.z, vd.w};
    float d[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      d[2 * i] = __uint_as_float(d4[i] << 16);
      d[2 * i + 1] = __uint_as_float(d4[i] & 0xffff0000u);
    }
    // all K rows' loads are issued before any arithmetic or store
    uint4 vyk[kMaxK];
#pragma unroll
    for (int k = 0; k < kMaxK; ++k)
      vyk[k] = (k < K && (unsigned)r[k] < (unsigned)R && in) ? *(const uint4*)(y + (size_t)r[k] * H + col)
                                                             : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int k = 0; k < kMaxK; ++k) {
      if (k >= K || (unsigned)r[k] >= (unsigned)R) continue;
      const uint4 vy = vyk[k];
      const uint32_t y4[4] = {vy.x, vy.y, vy.z, vy.w};
      uint32_t o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float y0 = __uint_as_float(y4[i] << 16);
        const float y1 = __uint_as_float(y4[i] & 0xffff0000u);
        part[k] = part[k] + d[2 * i] * y0;
        part[k] = part[k] + d[2 * i + 1] * y1;
        o[i] = bf16_pack2(wk[k] * d[2 * i], wk[k] * d[2 * i + 1]);
      }
      if (!in) o[0] = o[1] = o[2] = o[3] = 0u;  // padding is +0 (w * +0 can be -0)
      if constexpr (kQuant) {
        float m = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          m = fmaxf(m, fabsf(__uint_as_float(o[i] << 16)));
          m = fmaxf(m, fabsf(__uint_as_float(o[i] & 0xffff0000u)));
        }
        const float sc = scale_of<kRowPow2>(row16_max(m));
        const QDiv qd = qdiv_setup_t<kRowPow2>(sc);
        float qv[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          qv[2 * i] = quot_t<kRowPow2>(__uint_as_float(o[i] << 16), qd);
          qv[2 * i + 1] = quot_t<kRowPow2>(__uint_as_float(o[i] & 0xffff0000u), qd);
        }
        *(uint2*)(dyq + (size_t)r[k] * Hp + col) =
            make_uint2(e4m3_pack4(qv[0], qv[1], qv[2], qv[3]), e4m3_pack4(qv[4], qv[5], qv[6], qv[7]));
        if ((lane & 15) == 0) dys[(size_t)r[k] * (Hp / kGroup) + col / kGroup] = sc;
      } else {
        *(uint4*)(dy + (size_t)r[k] * H + col) = make_uint4(o[0], o[1], o[2], o[3]);
      }
    }
  }
#pragma unroll
  for (int k = 0; k < kMaxK; ++k) {
    if (k >= K) continue;
    const float tot = wave_sum_tree(part[k]);
    if (lane == 0) dw[(size_t)t * K + k] = tot;
  }
}

}  // namespace smoe

using namespace smoe;

extern "C" int smoe_transpose_blockwise_fp8(const uint8_t* wq, const float* ws, int E, int N,
                                            int Kdim, uint8_t* wqT, float* wsT, void* stream) {
  if (N <= 0 || Kdim <= 0) return SMOE_EINVAL_DIM;
  if (E <= 0 || E > SMOE_MAX_EXPERTS) return SMOE_EINVAL_EXPERTS;
  if (N % kLane || Kdim % kLane) return SMOE_EINVAL_ALIGN128;
  SMOE_CHECK_PTR(wq);
  SMOE_CHECK_PTR(wqT);
  if (!ws || !wsT) return SMOE_EINVAL_NULL;
  if (((uintptr_t)ws | (uintptr_t)wsT) & 3u) return SMOE_EINVAL_PTRALIGN;
  hipStream_t s = (hipStream_t)stream;
  const int NB = pad128(N) / kGroup, KB = pad128(Kdim) / kGroup;
  transpose_fp8_kernel<<<dim3(KB * 2, NB * 2, E), dim3(256), 0, s>>>(wq, N, Kdim, wqT);
  const long long ns = (long long)E * NB * KB;
  transpose_scales_kernel<<<dim3((unsigned)((ns + 255) / 256)), dim3(256), 0, s>>>(
      ws, E, NB, KB, wsT);
  SMOE_RETURN_LAUNCH();
}

extern "C" int smoe_quant_cols_ld(int R, int E) {
  if (R < 0 || E <= 0) return 0;
  const long long ld = ((long long)(R + kGroup - 1) / kGroup + E) * kGroup;
  return ld > 0x7fffffffLL ? 0 : (int)ld;
}

extern "C" int smoe_quant_cols_128x1(const uint16_t* x, const int32_t* gather, int gather_div,
                                     int R, int C, const int32_t* offsets, int E, int ld,
                                     uint8_t* xTq, float* xTs, int32_t* pad, int col_scale,
                                     void* stream) {
  if (R <= 0 || C <= 0) return SMOE_EINVAL_DIM;
  if (col_scale != SMOE_COLSCALE_FP32 && col_scale != SMOE_COLSCALE_POW2) return SMOE_EINVAL_MODE;
  if (gather && gather_div <= 0) return SMOE_EINVAL_DIM;
  if (gather && ((uintptr_t)gather & 3u)) return SMOE_EINVAL_PTRALIGN;
  if (E <= 0 || E > SMOE_MAX_EXPERTS) return SMOE_EINVAL_EXPERTS;
  if (C % kLane) return SMOE_EINVAL_ALIGN128;
  if (ld < smoe_quant_cols_ld(R, E) || ld % kGroup) return SMOE_EINVAL_DIM;
  if (ld / kGroup > 65535) return SMOE_EINVAL_DIM;  // 128-row groups are grid.y
  SMOE_CHECK_PTR(x);
  SMOE_CHECK_PTR(xTq);
  if (!offsets || !xTs || !pad) return SMOE_EINVAL_NULL;
  if (((uintptr_t)offsets | (uintptr_t)xTs | (uintptr_t)pad) & 3u) return SMOE_EINVAL_PTRALIGN;
  hipStream_t s = (hipStream_t)stream;
  pad_offsets_kernel<<<1, 1024, 0, s>>>(offsets, E, pad);
  // column slabs vary fastest, so the workgroups in flight read whole rows
#define SMOE_QC(P2)                                                                            \
  quant_cols_kernel<false, false, P2><<<dim3((C + kQcCols - 1) / kQcCols, ld / kGroup), dim3(256), 0, s>>>( \
      x, gather, gather ? gather_div : 1, nullptr, R, C, offsets, pad, E, ld, xTq, xTs, nullptr, nullptr, \
      nullptr, nullptr, nullptr)
  if (col_scale == SMOE_COLSCALE_POW2) SMOE_QC(true);
  else SMOE_QC(false);
#undef SMOE_QC
  SMOE_RETURN_LAUNCH();
}

extern "C" int smoe_quant_rows_cols(const uint16_t* x, int R, int C, const int32_t* offsets, int E,
                                    int ld, uint8_t* xq, float* xs, uint8_t* xTq, float* xTs,
                                    int32_t* pad, int col_scale, void* stream) {
  if (R <= 0 || C <= 0) return SMOE_EINVAL_DIM;
  if (col_scale & ~(SMOE_COLSCALE_POW2 | SMOE_ROWSCALE_POW2)) return SMOE_EINVAL_MODE;
  const bool cp2 = col_scale & SMOE_COLSCALE_POW2, rp2 = col_scale & SMOE_ROWSCALE_POW2;
  if (E <= 0 || E > SMOE_MAX_EXPERTS) return SMOE_EINVAL_EXPERTS;
  if (C % kLane) return SMOE_EINVAL_ALIGN128;
  if (ld < smoe_quant_cols_ld(R, E) || ld % kGroup) return SMOE_EINVAL_DIM;
  if (ld / kGroup > 65535) return SMOE_EINVAL_DIM;
  SMOE_CHECK_PTR(x);
  SMOE_CHECK_PTR(xTq);
  if (!offsets || !xTs || !pad || !xs) return SMOE_EINVAL_NULL;
  if (((uintptr_t)offsets | (uintptr_t)xTs | (uintptr_t)pad | (uintptr_t)xs) & 3u)
    return SMOE_EINVAL_PTRALIGN;
  if (!xq) return SMOE_EINVAL_NULL;
  if ((uintptr_t)xq & 7u) return SMOE_EINVAL_PTRALIGN;
  hipStream_t s = (hipStream_t)stream;
  pad_offsets_kernel<<<1, 1024, 0, s>>>(offsets, E, pad);
#define SMOE_QRC(P2, RP2)                                                                      \
  quant_cols_kernel<true, false, P2, RP2><<<dim3((C + kQcCols - 1) / kQcCols, ld / kGroup), dim3(256), 0, s>>>( \
      x, nullptr, 1, nullptr, R, C, offsets, pad, E, ld, xTq, xTs, xq, xs, nullptr, nullptr, nullptr)
  if (cp2) { if (rp2) SMOE_QRC(true, true); else SMOE_QRC(true, false); }
  else { if (rp2) SMOE_QRC(false, true); else SMOE_QRC(false, false); }
#undef SMOE_QRC
  SMOE_RETURN_LAUNCH();
}

extern "C" int smoe_swiglu_bwd_quant(const uint16_t* c1, const uint16_t* dh, int R, int I,
                                     const int32_t* offsets, int E, int ld, uint8_t* dcq,
                                     float* dcs, uint8_t* dcTq, float* dcTs, int32_t* pad,
                                     uint16_t* dc1, int col_scale, void* stream) {
  if (R <= 0 || I <= 0) return SMOE_EINVAL_DIM;
  if (col_scale & ~(SMOE_COLSCALE_POW2 | SMOE_ROWSCALE_POW2)) return SMOE_EINVAL_MODE;
  const bool cp2 = col_scale & SMOE_COLSCALE_POW2, rp2 = col_scale & SMOE_ROWSCALE_POW2;
  if (E <= 0 || E > SMOE_MAX_EXPERTS) return SMOE_EINVAL_EXPERTS;
  if (I % kGroup) return SMOE_EINVAL_ALIGN128;
  if (ld < smoe_quant_cols_ld(R, E) || ld % kGroup) return SMOE_EINVAL_DIM;
  if (ld / kGroup > 65535) return SMOE_EINVAL_DIM;
  SMOE_CHECK_PTR(c1);
  SMOE_CHECK_PTR(dh);
  SMOE_CHECK_PTR(dcTq);
  if (!offsets || !dcTs || !pad || !dcs || !dcq) return SMOE_EINVAL_NULL;
  if (((uintptr_t)offsets | (uintptr_t)dcTs | (uintptr_t)pad | (uintptr_t)dcs) & 3u)
    return SMOE_EINVAL_PTRALIGN;
  if ((uintptr_t)dcq & 7u) return SMOE_EINVAL_PTRALIGN;
  if (dc1 && ((uintptr_t)dc1 & 15u)) return SMOE_EINVAL_PTRALIGN;
  const int C = 2 * I;
  hipStream_t s = (hipStream_t)stream;
  pad_offsets_kernel<<<1, 1024, 0, s>>>(offsets, E, pad);
  // one workgroup per 128-column block of both halves (dg and du)
#define SMOE_SBQ(P2, RP2)                                                          \
  quant_cols_kernel<true, true, P2, RP2><<<dim3(I / kQcCols, ld / kGroup), dim3(256), 0, s>>>( \
      nullptr, nullptr, 1, nullptr, R, C, offsets, pad, E, ld, dcTq, dcTs, dcq, dcs, c1, dh, dc1)
  if (cp2) { if (rp2) SMOE_SBQ(true, true); else SMOE_SBQ(true, false); }
  else { if (rp2) SMOE_SBQ(false, true); else SMOE_SBQ(false, false); }
#undef SMOE_SBQ
  SMOE_RETURN_LAUNCH();
}

extern "C" int smoe_swiglu_bwd(const uint16_t* c1, const uint16_t* dh, int R, int I,
                               uint16_t* dc1, void* stream) {
  if (R <= 0 || I <= 0) return SMOE_EINVAL_DIM;
  if (I % kLane) return SMOE_EINVAL_ALIGN128;
  SMOE_CHECK_PTR(c1);
  SMOE_CHECK_PTR(dh);
  SMOE_CHECK_PTR(dc1);
  swiglu_bwd_kernel<<<dim3((R + 3) / 4), dim3(256), 0, (hipStream_t)stream>>>(c1, dh, R, I, dc1);
  SMOE_RETURN_LAUNCH();
}

extern "C" int smoe_unpermute_combine_bwd(const uint16_t* dout, const uint16_t* y,
                                          const int32_t* inv_map, const float* w, int T, int K,
                                          int H, uint16_t* dy, float* dw, void* stream) {
  if (T <= 0 || H <= 0) return SMOE_EINVAL_DIM;
  if (H % kLane) return SMOE_EINVAL_ALIGN128;
  if (K <= 0 || K > 32) return SMOE_EINVAL_TOPK;
  if ((long long)T * K > 0x7fffffffLL) return SMOE_EINVAL_DIM;
  SMOE_CHECK_PTR(dout);
  SMOE_CHECK_PTR(y);
  SMOE_CHECK_PTR(dy);
  if (!inv_map || !w || !dw) return SMOE_EINVAL_NULL;
  if (((uintptr_t)inv_map | (uintptr_t)w | (uintptr_t)dw) & 3u) return SMOE_EINVAL_PTRALIGN;
  const dim3 grid((T + 3) / 4), block(256);
  hipStream_t s = (hipStream_t)stream;
#define SMOE_CBB(MK) \
  combine_bwd_kernel<MK, false><<<grid, block, 0, s>>>(dout, y, inv_map, w, T, K, H, dy, dw, \
                                                       nullptr, nullptr)
  if (K <= 2) SMOE_CBB(2);
  else if (K <= 8) SMOE_CBB(8);
  else SMOE_CBB(32);
#undef SMOE_CBB
  SMOE_RETURN_LAUNCH();
}

namespace {
// The 128x1 columns of dy: row r of dy is rebuilt as bf16(w[p] * dout[p / K])
// with p = row_map[r].
void combine_bwd_cols_launch(const uint16_t* dout, const int32_t* row_map, const float* w, int K,
                             int R, int H, const int32_t* offsets, int E, int ld, uint8_t* dyTq,
                             float* dyTs, int32_t* pad, bool p2, hipStream_t s) {
#define SMOE_CQ(P2)                                                                          \
  quant_cols_kernel<false, false, P2><<<dim3((H + kQcCols - 1) / kQcCols, ld / kGroup), dim3(256), \
                                        0, s>>>(dout, row_map, K, w, R, H, offsets, pad, E, ld,  \
                                                dyTq, dyTs, nullptr, nullptr, nullptr, nullptr,  \
                                                nullptr)
  if (p2) SMOE_CQ(true);
  else SMOE_CQ(false);
#undef SMOE_CQ
}
}  // namespace

extern "C" int smoe_unpermute_combine_bwd_quant(const uint16_t* dout, const uint16_t* y,
                                                const int32_t* inv_map, const int32_t* row_map,
                                                const float* w, int T, int K, int H,
                                                const int32_t* offsets, int E, int ld,
                                                uint8_t* dyq, float* dys, uint8_t* dyTq,
                                                float* dyTs, int32_t* pad, float* dw,
                                                int col_scale, void* stream) {
  if (T <= 0 || H <= 0) return SMOE_EINVAL_DIM;
  if (col_scale & ~(SMOE_COLSCALE_POW2 | SMOE_ROWSCALE_POW2)) return SMOE_EINVAL_MODE;
  const bool cp2 = col_scale & SMOE_COLSCALE_POW2, rp2 = col_scale & SMOE_ROWSCALE_POW2;
  if (H % kLane) return SMOE_EINVAL_ALIGN128;
  if (K <= 0 || K > 32) return SMOE_EINVAL_TOPK;
  if ((long long)T * K > 0x7fffffffLL) return SMOE_EINVAL_DIM;
  if (E <= 0 || E > SMOE_MAX_EXPERTS) return SMOE_EINVAL_EXPERTS;
  const int R = T * K;
  if (ld < smoe_quant_cols_ld(R, E) || ld % kGroup) return SMOE_EINVAL_DIM;
  if (ld / kGroup > 65535) return SMOE_EINVAL_DIM;
  SMOE_CHECK_PTR(dout);
  SMOE_CHECK_PTR(y);
  // dyTq and dyTs both NULL: no column pass (smoe_combine_bwd_quant_cols
  // runs it separately)
  const bool cols = dyTq || dyTs;
  if (cols) SMOE_CHECK_PTR(dyTq);
  if (!inv_map || !row_map || !w || !dw || !offsets || !dys || (cols && !dyTs) || !pad || !dyq)
    return SMOE_EINVAL_NULL;
  if (((uintptr_t)inv_map | (uintptr_t)row_map | (uintptr_t)w | (uintptr_t)dw |
       (uintptr_t)offsets | (uintptr_t)dys | (uintptr_t)dyTs | (uintptr_t)pad) & 3u)
    return SMOE_EINVAL_PTRALIGN;
  if ((uintptr_t)dyq & 7u) return SMOE_EINVAL_PTRALIGN;
  hipStream_t s = (hipStream_t)stream;
  // dw and the 1x128 rows of dy; dy itself is never stored
  const dim3 grid((T + 3) / 4), block(256);
#define SMOE_CBB(MK, RP2) \
  combine_bwd_kernel<MK, true, RP2><<<grid, block, 0, s>>>(dout, y, inv_map, w, T, K, H, nullptr, dw, \
                                                           dyq, dys)
  if (rp2) {
    if (K <= 2) SMOE_CBB(2, true);
    else if (K <= 8) SMOE_CBB(8, true);
    else SMOE_CBB(32, true);
  } else {
    if (K <= 2) SMOE_CBB(2, false);
    else if (K <= 8) SMOE_CBB(8, false);
    else SMOE_CBB(32, false);
  }
#undef SMOE_CBB
  pad_offsets_kernel<<<1, 1024, 0, s>>>(offsets, E, pad);
  if (cols) combine_bwd_cols_launch(dout, row_map, w, K, R, H, offsets, E, ld, dyTq, dyTs, pad, cp2, s);
  SMOE_RETURN_LAUNCH();
}

extern "C" int smoe_combine_bwd_quant_cols(const uint16_t* dout, const int32_t* row_map,
                                           const float* w, int T, int K, int H,
                                           const int32_t* offsets, int E, int ld, uint8_t* dyTq,
                                           float* dyTs, int32_t* pad, int col_scale,
                                           void* stream) {
  if (T <= 0 || H <= 0) return SMOE_EINVAL_DIM;
  if (col_scale & ~SMOE_COLSCALE_POW2) return SMOE_EINVAL_MODE;
  if (H % kLane) return SMOE_EINVAL_ALIGN128;
  if (K <= 0 || K > 32) return SMOE_EINVAL_TOPK;
  if ((long long)T * K > 0x7fffffffLL) return SMOE_EINVAL_DIM;
  if (E <= 0 || E > SMOE_MAX_EXPERTS) return SMOE_EINVAL_EXPERTS;
  const int R = T * K;
  if (ld < smoe_quant_cols_ld(R, E) || ld % kGroup) return SMOE_EINVAL_DIM;
  if (ld / kGroup > 65535) return SMOE_EINVAL_DIM;
  SMOE_CHECK_PTR(dout);
  SMOE_CHECK_PTR(dyTq);
  if (!row_map || !w || !offsets || !dyTs || !pad) return SMOE_EINVAL_NULL;
  if (((uintptr_t)row_map | (uintptr_t)w | (uintptr_t)offsets | (uintptr_t)dyTs |
       (uintptr_t)pad) & 3u)
    return SMOE_EINVAL_PTRALIGN;
  hipStream_t s = (hipStream_t)stream;
  pad_offsets_kernel<<<1, 1024, 0, s>>>(offsets, E, pad);
  combine_bwd_cols_launch(dout, row_map, w, K, R, H, offsets, E, ld, dyTq, dyTs, pad,
                          col_scale & SMOE_COLSCALE_POW2, s);
  SMOE_RETURN_LAUNCH();
}
