// smoe_common.h — device helpers shared by the smoe HIP kernels (gfx950).
//
// Everything here is evaluated with separately rounded fp32 operations: the
// library is compiled with -ffp-contract=off so that no multiply/add pair is
// fused behind the source's back, and fp32 division stays IEEE correctly
// rounded (-fhip-fp32-correctly-rounded-divide-sqrt).  This is what makes the
// quantised bytes bit-identical to the CPU restatement of the same rules.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/smoe.h"

namespace smoe {

constexpr int kWave = 64;
constexpr int kGroup = 128;  // quantisation group / weight block edge
constexpr int kLane = 16;    // elements per lane in the row quantisers

// A dimension D that is not a multiple of 128 is quantised as if it were
// zero-padded to pad128(D): the last group's amax is over its valid
// elements (zeros never raise it), its padding quantises to byte 0, and the
// fp8 operand keeps a row pitch of pad128(D).  D must be a multiple of 16.
__host__ __device__ constexpr int pad128(int d) { return (d + kGroup - 1) / kGroup * kGroup; }
constexpr float kE4M3Max = 448.0f;

// ---------------------------------------------------------------- bf16 ----
// Round-to-nearest-even fp32 -> bf16 bits; NaN stays a quiet NaN.  The
// software statement of the rule: kernels use bf16_pack2 below.
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// Two fp32 -> packed bf16 bits (lo in bits 0-15, hi in 16-31) with gfx950's
// conversion instruction (v_cvt_pk_bf16_f32, round to nearest even): one
// instruction per pair where f32_to_bf16's NaN test costs a branch per value.
// smoe_selftest_quant checks it against f32_to_bf16 for every fp32 pattern.
typedef __bf16 bf16x2_hw __attribute__((ext_vector_type(2)));
typedef float f32x2_hw __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t bf16_pack2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_hw{lo, hi}, bf16x2_hw));
}

// ---------------------------------------------------------------- e4m3 ----
// Reference OCP e4m3fn encode of |v| <= 448 with round-to-nearest-even, in
// software.  Subnormal range |v| < 2^-6: code = rint(|v| * 2^9) (the product
// is exact; a result of 8 is the smallest normal, 0x08, which is the correct
// code).  Normal range: RNE to 3 mantissa bits on the fp32 pattern, then
// rebias the exponent 127 -> 7 (subtract 120 << 3 from the combined
// exponent|mantissa).  The kernels use the hardware conversion below; this
// is what smoe_selftest_quant checks it against.
__device__ __forceinline__ uint32_t e4m3_encode_sw(float v) {
  uint32_t u = __float_as_uint(v);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7fffffffu;
  float af = __uint_as_float(a);
  const uint32_t q_sub = (uint32_t)__builtin_rintf(af * 512.0f);
  const uint32_t q_nrm = ((a + 0x7ffffu + ((a >> 20) & 1u)) >> 20) - (120u << 3);
  return (af < 0.015625f ? q_sub : q_nrm) | sign;
}

// Four values (each |v| <= 448) to four e4m3 bytes, a in the low byte, with
// gfx950's v_cvt_pk_fp8_f32 (OCP e4m3fn, round to nearest even): identical
// to e4m3_encode_sw for every fp32 with |v| <= 448, which smoe_selftest_quant
// checks exhaustively.  It does not saturate (464 and above become NaN), so
// its inputs are clamped or bounded by construction.
__device__ __forceinline__ uint32_t e4m3_pack4(float a, float b, float c, float d) {
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);
}

// clamp(x / s, +-448) with an IEEE fp32 division: the quotient the
// quantisation rule is defined on.
__device__ __forceinline__ float quot_ieee(float x, float s) {
  const float y = x / s;
  return fminf(fmaxf(y, -kE4M3Max), kE4M3Max);
}

// Reference rule for one value: e4m3(clamp(x / s)).
__device__ __forceinline__ uint32_t quant_one(float x, float s) {
  return e4m3_encode_sw(quot_ieee(x, s));
}

// s = amax / 448 (fp32 RN), 1 when amax == 0.
__device__ __forceinline__ float group_scale(float amax) {
  return amax == 0.0f ? 1.0f : amax / kE4M3Max;
}

// The power-of-two scale of the optional E8M0 column recipe: the least power
// of two >= RN(amax / 448), at least 2^-127 (the smallest E8M0 value); 1 when
// amax == 0.  Dividing by it is exact, so x / s needs no rounding before the
// e4m3 encoding, and its fp32 exponent field is the E8M0 byte the scaled
// MFMA takes.
__device__ __forceinline__ float group_scale_pow2(float amax) {
  if (amax == 0.0f) return 1.0f;
  const float t = amax / kE4M3Max;
  int e;
  const float m = __builtin_frexpf(t, &e);  // t = m * 2^e, m in [0.5, 1)
  const float s = m == 0.5f ? t : __builtin_ldexpf(1.0f, e);
  return fmaxf(s, 0x1p-127f);
}

// Division-free quotient for bf16 inputs.  With s = m * 2^e (m in [0.5, 1))
// and r = RN(1/m) computed once per group, each element takes
//   xs = x * 2^-e (exact), q0 = RN(xs * r), d = fma(-q0, m, xs),
//   q = fma(d, r, q0) with the sign of x,
// i.e. a reciprocal-based quotient with one residual correction.  The
// quotient can differ from the IEEE quotient x / s in its last bit, but its
// e4m3 byte equals e4m3(clamp(x / s)) for every finite bf16 x and every bf16
// amax >= |x| with s = group_scale(amax), with no clamp needed (|q| stays
// below the 464 rounding boundary): smoe_selftest_quant checks this
// exhaustively over that whole domain on the GPU.  Inputs that are not bf16
// (SwiGLU's fp32 h) use quot_ieee.
struct QDiv {
  float m, r;
  int e;
};
__device__ __forceinline__ QDiv qdiv_setup(float s) {
  QDiv d;
  d.m = __builtin_frexpf(s, &d.e);
  d.r = 1.0f / d.m;
  return d;
}
__device__ __forceinline__ float quot_bf16(float x, const QDiv& d) {
  const float xs = __builtin_ldexpf(x, -d.e);
  const float q0 = xs * d.r;
  const float res = __builtin_fmaf(-q0, d.m, xs);
  const float y = __builtin_fmaf(res, d.r, q0);
  return __uint_as_float((__float_as_uint(y) & 0x7fffffffu) | (__float_as_uint(x) & 0x80000000u));
}

// The same set-up and quotient by scale rule.  A power-of-two scale s
// (kPow2, the E8M0 recipe) has an exact reciprocal 1/s (s in [2^-127,
// 2^127]), so x * (1/s) is the IEEE quotient x / s itself: one multiply.
// Quotients in fp32's subnormal range are far below e4m3's smallest step
// and encode as a signed zero either way.
template <bool kPow2>
__device__ __forceinline__ QDiv qdiv_setup_t(float s) {
  if constexpr (kPow2) {
    QDiv d;
    d.m = 0.0f;
    d.r = 1.0f / s;
    d.e = 0;
    return d;
  } else {
    return qdiv_setup(s);
  }
}
template <bool kPow2>
__device__ __forceinline__ float quot_t(float x, const QDiv& d) {
  if constexpr (kPow2) return x * d.r;
  else return quot_bf16(x, d);
}

// ---------------------------------------------------------------- exp -----
// exp in fp32: Cody-Waite reduction n = rint(x*log2e),
// r = fma(-n, LN2_LO, fma(-n, LN2_HI, x)) with LN2_HI holding 16 significant
// bits, degree-7 Taylor polynomial by Horner in fmas, times 2^n built from
// the exponent field.  x > 88 -> +inf, x < -87 -> 0.  Within 1 ulp of exp
// over [-87, 88] (0.91 ulp at most over 2 M points checked against float64).
// The common part of expf32: xc is x clamped to [-88, 89] (or a subrange
// that holds every x the caller can pass).
__device__ __forceinline__ float expf32_core(float x, float xc) {
  const float kLog2e = 1.4426950408889634f;
  const float kLn2Hi = __uint_as_float(0x3f317200u);
  const float kLn2Lo = __uint_as_float(0x35bfbe8eu);
  float n = __builtin_rintf(xc * kLog2e);
  // Cody-Waite reduction and Horner polynomial in fused multiply-adds (one
  // rounding each, v_fma_f32): the oracle's fma32 reproduces them exactly
  float r = __builtin_fmaf(-n, kLn2Hi, xc);
  r = __builtin_fmaf(-n, kLn2Lo, r);
  float p = (float)(1.0 / 5040.0);
  p = __builtin_fmaf(p, r, (float)(1.0 / 720.0));
  p = __builtin_fmaf(p, r, (float)(1.0 / 120.0));
  p = __builtin_fmaf(p, r, (float)(1.0 / 24.0));
  p = __builtin_fmaf(p, r, (float)(1.0 / 6.0));
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  float two_n = __uint_as_float((uint32_t)((int)n + 127) << 23);
  float y = p * two_n;
  y = x < -87.0f ? 0.0f : y;
  return x != x ? x : y;  // NaN in, NaN out (the range tests are false for NaN)
}

__device__ __forceinline__ float expf32(float x) {
  // evaluated unconditionally and selected at the end (no branches: the
  // range tests would otherwise split the wave's control flow per call)
  const float xc = fminf(fmaxf(x, -88.0f), 89.0f);  // keeps n in int range; result replaced below
  const float y = expf32_core(x, xc);
  return x > 88.0f ? __builtin_inff() : y;
}

// expf32 for x <= 0, -inf or NaN (a softmax's x - max): the upper clamp and
// the overflow select never apply there, so the bits equal expf32(x).
__device__ __forceinline__ float expf32_nonpos(float x) {
  return expf32_core(x, fmaxf(x, -88.0f));
}

// 1/b correctly rounded: v_rcp_f32's approximation y0 and one Newton step
// y0 + y0*(1 - b*y0), both in fmas.  Equal to the IEEE quotient 1.0f / b for
// every fp32 b in [2^-126, 2^126) (smoe_selftest_recip checks each of those
// values on the GPU); +inf gives +0 and NaN gives NaN, as the quotient does.
__device__ __forceinline__ float recip_rn(float b) {
  const float y0 = __builtin_amdgcn_rcpf(b);
  const float e = __builtin_fmaf(-b, y0, 1.0f);
  const float y1 = __builtin_fmaf(e, y0, y0);
  return b == __builtin_inff() ? 0.0f : y1;
}

// a / b correctly rounded, from y = RN(1/b): q0 = RN(a*y), the remainder
// a - q0*b is exact in one fma, and RN(q0 + rem*y) is RN(a/b) whenever the
// quotient and the remainder are normal (Markstein's division theorem; Muller
// et al., Handbook of Floating-Point Arithmetic, the fma-based division
// section).  The callers keep a >= 2^-100 or a == 0 and b in [1, 2048], and
// send any other a to the IEEE division.
__device__ __forceinline__ float div_by_recip(float a, float b, float y) {
  const float q0 = a * y;
  const float rem = __builtin_fmaf(-q0, b, a);
  return __builtin_fmaf(rem, y, q0);
}

__device__ __forceinline__ float silu32(float g) { return g / (1.0f + expf32(-g)); }

// --------------------------------------------------------------- waves ----
template <int kWidth>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int o = kWidth / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWidth));
  return v;
}

// Max over each row of 16 lanes with DPP lane moves (no LDS round trip):
// swap neighbours, swap pairs, mirror within 8, mirror within 16.  Lanes
// that are inactive contribute 0, so the inputs must be >= 0 (amax values).
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false)));
  return v;
}

// The value of lane (l ^ kO) for every lane l of a fully active wave: DPP
// quad permutes for 1 and 2, ds_swizzle's bit mode within 32 lanes for 4, 8
// and 16, ds_bpermute for 32.  The same partner as __shfl_xor(v, kO), with
// shorter exchange latency for the first five levels.
template <int kO>
__device__ __forceinline__ int xor_lanes(int v) {
  static_assert(kO == 1 || kO == 2 || kO == 4 || kO == 8 || kO == 16 || kO == 32, "xor distance");
  if constexpr (kO == 1) return __builtin_amdgcn_update_dpp(v, v, 0xB1, 0xF, 0xF, false);
  else if constexpr (kO == 2) return __builtin_amdgcn_update_dpp(v, v, 0x4E, 0xF, 0xF, false);
  else if constexpr (kO < 32) return __builtin_amdgcn_ds_swizzle(v, (kO << 10) | 0x1F);
  else return __shfl_xor(v, 32, kWave);
}
template <int kO>
__device__ __forceinline__ float xor_lanes(float v) {
  return __int_as_float(xor_lanes<kO>(__float_as_int(v)));
}

// Sum over the wave as a fixed butterfly (partners at distance 32, 16, ...,
// 1), the reduction tree the oracle restates.
__device__ __forceinline__ float wave_sum_tree(float v) {
  v = v + xor_lanes<32>(v);
  v = v + xor_lanes<16>(v);
  v = v + xor_lanes<8>(v);
  v = v + xor_lanes<4>(v);
  v = v + xor_lanes<2>(v);
  v = v + xor_lanes<1>(v);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, xor_lanes<32>(v));
  v = fmaxf(v, xor_lanes<16>(v));
  v = fmaxf(v, xor_lanes<8>(v));
  v = fmaxf(v, xor_lanes<4>(v));
  v = fmaxf(v, xor_lanes<2>(v));
  v = fmaxf(v, xor_lanes<1>(v));
  return v;
}

// ------------------------------------------- 1x128 group quantisation ----
struct Q16 {
  uint4 q;      // 16 fp8 bytes
  float scale;  // group scale (identical in the 8 lanes of a group)
};

// The group scale of a quantiser: amax/448 (group_scale), or with kPow2 the
// least power of two at or above it (group_scale_pow2).
template <bool kPow2>
__device__ __forceinline__ float scale_of(float amax) {
  if constexpr (kPow2) return group_scale_pow2(amax);
  else return group_scale(amax);
}

// Quantise 16 fp32 values owned by this lane whose group spans 8 lanes.
template <bool kPow2 = false>
__device__ __forceinline__ Q16 quant16(const float (&f)[16]) {
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(f[i]));
  amax = group_max<8>(amax);
  const float s = scale_of<kPow2>(amax);
  uint32_t w[4];
  if constexpr (kPow2) {
    // x * (1/s) is the IEEE quotient for a power-of-two s; the clamp keeps
    // quot_ieee's handling of NaN
    const float r = 1.0f / s;
    auto q = [&](float x) { return fminf(fmaxf(x * r, -kE4M3Max), kE4M3Max); };
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = e4m3_pack4(q(f[4 * i]), q(f[4 * i + 1]), q(f[4 * i + 2]), q(f[4 * i + 3]));
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = e4m3_pack4(quot_ieee(f[4 * i], s), quot_ieee(f[4 * i + 1], s),
                        quot_ieee(f[4 * i + 2], s), quot_ieee(f[4 * i + 3], s));
  }
  Q16 r;
  r.q = make_uint4(w[0], w[1], w[2], w[3]);
  r.scale = s;
  return r;
}

// As quant16, for bf16 inputs (the division-free quantiser; with a
// power-of-two scale its quotient is exact).
template <bool kPow2 = false>
__device__ __forceinline__ Q16 quant16_bf16(const float (&f)[16]) {
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(f[i]));
  amax = group_max<8>(amax);
  const float s = scale_of<kPow2>(amax);
  const QDiv d = qdiv_setup_t<kPow2>(s);
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    w[i] = e4m3_pack4(quot_t<kPow2>(f[4 * i], d), quot_t<kPow2>(f[4 * i + 1], d),
                      quot_t<kPow2>(f[4 * i + 2], d), quot_t<kPow2>(f[4 * i + 3], d));
  Q16 r;
  r.q = make_uint4(w[0], w[1], w[2], w[3]);
  r.scale = s;
  return r;
}

__device__ __forceinline__ void unpack_bf16x8(const uint4& v, float* f) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(w[i] << 16);
    f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

}  // namespace smoe

// ------------------------------------------------------ host validation ----
#define SMOE_CHECK_PTR(p)                                   \
  do {                                                      \
    if ((p) == nullptr) return SMOE_EINVAL_NULL;            \
    if (((uintptr_t)(p)) & 15u) return SMOE_EINVAL_PTRALIGN; \
  } while (0)

#define SMOE_RETURN_LAUNCH()                          \
  do {                                                \
    hipError_t err__ = hipGetLastError();             \
    return err__ == hipSuccess ? SMOE_OK : (int)err__; \
  } while (0)
