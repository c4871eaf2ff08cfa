"""CPU oracle for the SimpleMoE expert-layer hot path — TEST INFRASTRUCTURE ONLY.

This module restates, in numpy, the semantics the MI355X kernels must match.
It is the checker: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it.  The product path
(``smoe``) never imports or calls anything here.

The reference (xmpeng-dev/system-lab) holds no code for this path, only
engineering notes describing it; every function below cites the note it
restates.  Where the notes leave a choice open the convention is fixed here
and is binding for the kernels too:

  C1 router: probs = softmax(fp32 logits); score = probs + bias; top-K by
     (score desc, expert id asc); w = probs[sel] / sum(probs[sel]).
  C2 sort:   pair p = t*K + k; stable counting sort by expert id.
  C3 quant:  per 1x128 group: amax = max|x|, s = amax/448 (s = 1 if amax == 0),
     q = e4m3_rne(clamp(x/s, +-448)); s is stored.  The rule is for finite
     inputs: the notes define no bytes for a group holding NaN or +-inf, and
     neither does this oracle (the kernels compute through such a group
     without faulting, its bytes and scale are unspecified).
  C4 weights: C3 over each 128x128 block of W[e] stored [N, K].
  C5 GEMM:   c[r,n] = sum_kb as[r,kb]*bs[e,n/128,kb]*sum_k a[r,k]*b[e,n,k].
  C6 SwiGLU: h = silu(g)*u in fp32, g = c1[:, :I], u = c1[:, I:]; C3 on h.
  C7 combine: out[t] = bf16(sum_k w[t,k]*y[inv_map[t*K+k]]), fp32, k order,
     each product and sum rounded separately.
  C9 short groups: a dimension D that is not a multiple of 128 (D % 16 == 0,
     e.g. GPT-OSS H = I = 2880) is quantised as the operand zero-padded to
     pad128(D): a short last group's amax is over its valid elements, its
     padding is byte 0, fp8 operands keep the padded pitch, and a short last
     weight block (rows or columns) is the zero-padded block.  Blockwise fp8
     GEMMs need dimensions aligned to 16 (moe/MegatronCore_MoE_reading_notes.md:541-543).
  C10 E8M0 scales (opt-in): s = the least power of two >= RN(amax/448), at
     least 2^-127 (1 when amax == 0); x/s is exact.  Either for the wgrad
     operands' 128x1 columns only, or for every quantisation (activation
     rows, weight blocks, gradient rows and columns), the MXFP8 scale format
     at the blockwise recipe's granularity.

Floating-point evaluation order is part of the contract where a kernel is
bit-exact (router softmax reduction tree, exp routine, combine order): the
oracle evaluates those in exactly the order the kernels do, in float32.

Pinning (what checks each function; tests/test_oracle.py):
  e4m3_encode      torch.float8_e4m3fn cast (library RNE) after clamp, over
                   every bf16 pattern and every e4m3 rounding midpoint +-1 ulp.
  fma32            C's fmaf (correctly rounded) on random and cancelling triples.
  expf32           numpy float64 exp (error bound <= 2 ulp), special values.
  router_topk      brute-force python sort on tiny inputs; closed-form softmax.
  route_sort       the reference's worked 16-token routing example
                   (moe/MoE_detailed_computation_dataflow.md:74-122, counts
                   [5,4,5,4,3,4,4,3]); permutation/stability invariants;
                   brute-force python counting sort.
  quant_1x128      closed forms (one-hot, constant, amax==0, +-448 saturation);
                   C9: full groups equal the aligned prefix's bytes, the short
                   group's scale is its valid amax / 448, padding is 0.
  quantize_weight  C9: edge blocks equal the full-width restatement on the
                   aligned part; scales of short blocks from their valid
                   elements; transpose_blockwise against an explicit
                   dequantise-and-transpose.
  grouped_gemm     one-hot rows, identity blocks, single non-zero K block,
                   zero-token experts, float64 dense matmul of the dequantised
                   operands computed per expert independently.
  swiglu_quant     float64 silu; silu(0)=0; silu(x)->x for large x.
  unpermute_combine K=1, w=1 is an exact inverse permutation (bytes equal);
                   python float32 scalar loop on tiny inputs.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32
E4M3_MAX = F32(448.0)
GROUP = 128

# ---------------------------------------------------------------------------
# bit-level helpers
# ---------------------------------------------------------------------------


def bf16_to_f32(u16: np.ndarray) -> np.ndarray:
    """bf16 bits (uint16) -> float32 (exact)."""
    return (np.asarray(u16, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits with round-to-nearest-even (NaN kept quiet)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    rounded = ((u + np.uint32(0x7FFF) + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), rounded)


def e4m3_encode(v: np.ndarray) -> np.ndarray:
    """float32 with |v| <= 448 -> OCP e4m3fn byte, round to nearest even.

    Subnormal range (|v| < 2^-6): the code is rint(|v| * 2^9) (exact scaling,
    RNE), which also yields 0x08 when rounding up to the smallest normal.
    Normal range: RNE on the fp32 bit pattern to 3 mantissa bits, then rebias
    the exponent from 127 to 7 (120 << 3 in the combined field).
    Recipe: E4M3 activations/weights (moe/MegatronCore_MoE_reading_notes.md:498-501),
    OCP e4m3fn with max 448 on gfx950 (summary/fp8_expert_gemm_optimization.md:202-208).
    """
    u = np.ascontiguousarray(v, dtype=np.float32).view(np.uint32)
    sign = ((u >> 24) & 0x80).astype(np.uint32)
    a = u & np.uint32(0x7FFFFFFF)
    af = a.view(np.float32)
    sub = af < F32(2.0 ** -6)
    q_sub = np.rint(af * F32(512.0)).astype(np.uint32)
    rnd = (a + np.uint32(0x7FFFF) + ((a >> 20) & 1)) >> 20
    q_norm = rnd - np.uint32(120 << 3)
    q = np.where(sub, q_sub, q_norm)
    return (q | sign).astype(np.uint8)


def _e4m3_decode_formula(q: np.ndarray) -> np.ndarray:
    """OCP e4m3fn byte -> float32 (0x7f / 0xff -> NaN)."""
    q = np.asarray(q, dtype=np.uint8).astype(np.int32)
    s = np.where(q & 0x80, -1.0, 1.0)
    e = (q >> 3) & 0xF
    m = q & 7
    mag = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    out = (s * mag).astype(np.float32)
    out[(q & 0x7F) == 0x7F] = np.nan
    return out


_E4M3_TABLE = _e4m3_decode_formula(np.arange(256))


def e4m3_decode(q: np.ndarray) -> np.ndarray:
    """OCP e4m3fn byte -> float32 (0x7f / 0xff -> NaN): the formula above,
    tabulated once for all 256 codes and applied by lookup."""
    return _E4M3_TABLE[np.asarray(q, dtype=np.uint8)]


def quant_rule(x: np.ndarray, s: np.ndarray) -> np.ndarray:
    """q = e4m3_rne(clamp(x / s, -448, 448)) in float32 (C3)."""
    y = np.asarray(x, np.float32) / np.asarray(s, np.float32)
    return e4m3_encode(np.clip(y, -E4M3_MAX, E4M3_MAX))


def group_scale(amax: np.ndarray) -> np.ndarray:
    """s = amax / 448 (fp32 RN), or 1 when amax == 0 (C3)."""
    amax = np.asarray(amax, np.float32)
    s = amax / E4M3_MAX
    return np.where(amax == 0, F32(1.0), s).astype(np.float32)


def group_scale_pow2(amax: np.ndarray) -> np.ndarray:
    """C10 (the optional E8M0 recipe): the least power of two
    >= RN(amax / 448), at least 2^-127; 1 when amax == 0.  Powers of
    two are the E8M0 scale format of MXFP8 (moe/MegatronCore_MoE_reading_notes.md:503-504)."""
    amax = np.asarray(amax, np.float32)
    t = (amax / E4M3_MAX).astype(np.float32)
    with np.errstate(divide="ignore"):
        e = np.ceil(np.log2(t.astype(np.float64)))
    s = np.maximum(np.exp2(e), 2.0 ** -127)
    return np.where(amax == 0, 1.0, s).astype(np.float32)


# ---------------------------------------------------------------------------
# fp32 exp shared by the router softmax and SwiGLU
# ---------------------------------------------------------------------------

_LOG2E = F32(1.4426950408889634)
_LN2_HI = np.uint32(0x3F317200).view(np.float32)  # 0.693145751953125, 16 significant bits
_LN2_LO = np.uint32(0x35BFBE8E).view(np.float32)  # ln2 - LN2_HI
_EXP_HI = F32(88.0)
_EXP_LO = F32(-87.0)
_TAYLOR = [F32(1.0 / 5040.0), F32(1.0 / 720.0), F32(1.0 / 120.0), F32(1.0 / 24.0),
           F32(1.0 / 6.0), F32(0.5), F32(1.0), F32(1.0)]


def fma32(a, b, c) -> np.ndarray:
    """Fused multiply-add in float32: RN32(a*b + c) with one rounding, the
    result of the GPU's v_fma_f32.  Emulated in float64: a*b is exact there
    (24 + 24 bits), s = RN64(a*b + c) and its error err = (a*b + c) - s
    come from Knuth's TwoSum, and when err != 0 the last bit of s is forced
    to 1 toward the exact sum (round to odd).  Rounding that 53-bit value to
    24 bits is then the correct rounding of the exact sum (Boldo and
    Melquiond, "Emulation of FMA and correctly rounded sums: proved
    algorithms using rounding to odd", IEEE TC 2008), float32 subnormals
    included since float64 has the exponent range to hold them exactly.
    Finite inputs whose sum stays in float64 range only (the exp routine's
    domain).  Pinned against C's fmaf in tests/test_oracle.py."""
    a = np.asarray(a, np.float32).astype(np.float64)
    b = np.asarray(b, np.float32).astype(np.float64)
    c = np.asarray(c, np.float32).astype(np.float64)
    p = a * b                         # exact
    s = p + c
    bv = s - p
    err = (p - (s - bv)) + (c - bv)   # TwoSum: p + c = s + err exactly
    bits = np.ascontiguousarray(s).view(np.int64)
    even = (bits & 1) == 0
    # one ulp of s toward the exact sum: away from zero when err has the
    # sign of s, toward zero otherwise (s == 0 only when the sum is exact)
    step = np.where(np.signbit(err) == np.signbit(s), 1, -1).astype(np.int64)
    bits = np.where((err != 0) & even, bits + step, bits)
    return bits.view(np.float64).astype(np.float32)


def expf32(x: np.ndarray) -> np.ndarray:
    """exp in float32 by Cody-Waite range reduction and a degree-7 Taylor
    polynomial (Horner), evaluated with fused multiply-adds:
      n = rint(x*log2e); r = fma(-n, LN2_LO, fma(-n, LN2_HI, x));
      p = fma(...fma(1/5040, r, 1/720)..., r, 1); p * 2^n.
    x > 88 -> +inf, x < -87 -> 0, NaN in -> NaN out.  Max error about 1 ulp
    over [-87, 88].  The HIP kernels evaluate the identical sequence (v_fma_f32
    for each fma, everything else separately rounded), so results are
    bit-identical.
    """
    x = np.asarray(x, np.float32)
    xc = np.clip(x, _EXP_LO, _EXP_HI)
    n = np.rint(xc * _LOG2E).astype(np.float32)
    r = fma32(-n, _LN2_HI, xc)
    r = fma32(-n, _LN2_LO, r)
    p = np.full(x.shape, _TAYLOR[0], np.float32)
    for c in _TAYLOR[1:]:
        p = fma32(p, r, np.full(x.shape, c, np.float32))
    ni = np.where(np.isnan(n), F32(0.0), n).astype(np.int32)  # NaN: replaced below
    two_n = ((ni + 127).astype(np.uint32) << 23).view(np.float32)
    out = (p * two_n).astype(np.float32)
    out = np.where(x > _EXP_HI, F32(np.inf), out)
    out = np.where(x < _EXP_LO, F32(0.0), out)
    return np.where(np.isnan(x), x, out).astype(np.float32)


# ---------------------------------------------------------------------------
# R: router
# ---------------------------------------------------------------------------

WAVE = 64


def _wave_tree_sum(vals: np.ndarray) -> np.ndarray:
    """Sum over the last axis in the kernel's order: lane j accumulates
    elements j, j+64, j+128, ... in ascending order, then an xor-butterfly
    over lanes with offsets 32, 16, 8, 4, 2, 1 (all lanes end equal)."""
    T, E = vals.shape
    nchunk = (E + WAVE - 1) // WAVE
    pad = np.zeros((T, nchunk * WAVE), np.float32)
    pad[:, :E] = vals
    lanes = np.zeros((T, WAVE), np.float32)
    for c in range(nchunk):
        lanes = (lanes + pad[:, c * WAVE:(c + 1) * WAVE]).astype(np.float32)
    idx = np.arange(WAVE)
    for off in (32, 16, 8, 4, 2, 1):
        lanes = (lanes + lanes[:, idx ^ off]).astype(np.float32)
    return lanes[:, 0]


def softmax_f32(logits: np.ndarray) -> np.ndarray:
    """probs = exp(l - max) / sum, fp32, sum in the wave-tree order (C1;
    moe/MoE_detailed_computation_dataflow.md:56-58)."""
    logits = np.asarray(logits, np.float32)
    m = logits.max(axis=1, keepdims=True)
    e = expf32((logits - m).astype(np.float32))
    s = _wave_tree_sum(e)
    return (e / s[:, None]).astype(np.float32)


def router_topk(logits: np.ndarray, K: int, bias: np.ndarray | None = None):
    """C1 router: softmax, optional selection bias, top-K with ties toward the
    lower expert id, renormalised weights (sequential fp32 sum in pick order).
    moe/MoE_detailed_computation_dataflow.md:53-66 (gate -> softmax -> top-k,
    renorm); moe/MegatronCore_MoE_reading_notes.md:688-697 (aux-loss-free
    bias used only for selection)."""
    probs = softmax_f32(logits)
    score = probs if bias is None else (probs + np.asarray(bias, np.float32)[None, :]).astype(np.float32)
    order = np.argsort(-score, axis=1, kind="stable")[:, :K]
    picked = np.take_along_axis(probs, order, axis=1)
    ssum = np.zeros(picked.shape[0], np.float32)
    for k in range(K):
        ssum = (ssum + picked[:, k]).astype(np.float32)
    w = (picked / ssum[:, None]).astype(np.float32)
    return order.astype(np.int32), w


def router_topk_bwd(logits: np.ndarray, topk_idx: np.ndarray, dtopk_w: np.ndarray) -> np.ndarray:
    """Gradient of the renormalised top-K weights with respect to the
    logits, in float64 (moe/MoE_detailed_computation_dataflow.md:53-66,
    backward chain :209-226).  With p = softmax(l), picks s_k, S = sum_k
    p[s_k], w_k = p[s_k]/S and g = dL/dw:
        dp[s_k] = (g_k - sum_j g_j w_j) / S   (0 for experts not picked)
        dl = p * (dp - sum_e p_e dp_e).
    The selection bias has no gradient."""
    l = np.asarray(logits, np.float64)
    p = np.exp(l - l.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    idx = np.asarray(topk_idx, np.int64)
    g = np.asarray(dtopk_w, np.float64)
    pk = np.take_along_axis(p, idx, axis=1)
    S = pk.sum(axis=1, keepdims=True)
    w = pk / S
    c = (g * w).sum(axis=1, keepdims=True)
    dp = np.zeros_like(p)
    np.put_along_axis(dp, idx, (g - c) / S, axis=1)
    return p * (dp - (p * dp).sum(axis=1, keepdims=True))


# ---------------------------------------------------------------------------
# K0: expert sort
# ---------------------------------------------------------------------------


def route_sort(topk_idx: np.ndarray, E: int):
    """C2: stable sort of pairs p = t*K + k by expert id.
    row_map[r] = p ("pack_perm: sorted pair index -> original pair index",
    notes/2026-04/2026-04-10_monolithmoe_layout_c_pack_optimization.md:56,80,120),
    inv_map[p] = r, counts[e], offsets = exclusive scan (E+1 entries)."""
    flat = np.asarray(topk_idx, np.int32).reshape(-1)
    row_map = np.argsort(flat, kind="stable").astype(np.int32)
    inv_map = np.empty_like(row_map)
    inv_map[row_map] = np.arange(flat.size, dtype=np.int32)
    counts = np.bincount(flat, minlength=E).astype(np.int32)
    offsets = np.zeros(E + 1, np.int32)
    offsets[1:] = np.cumsum(counts)
    return row_map, inv_map, counts, offsets


# ---------------------------------------------------------------------------
# K1 / W: quantisation
# ---------------------------------------------------------------------------


def pad128(d: int) -> int:
    """C9: a dimension that is not a multiple of 128 is quantised as if
    zero-padded to the next multiple of 128 (zeros never raise an amax and
    quantise to byte 0); fp8 operands keep that padded pitch."""
    return -(-int(d) // GROUP) * GROUP


def quant_1x128(x: np.ndarray, pow2: bool = False):
    """C3 on rows of x [M, H] float32 -> q [M,Hp] u8, s [M,Hp/128] f32 with
    Hp = pad128(H) (C9: a short last group is the zero-padded group).
    1x128 activation tiles: moe/MegatronCore_MoE_reading_notes.md:498-501."""
    x = np.asarray(x, np.float32)
    M, H = x.shape
    if H % GROUP:
        x = np.concatenate([x, np.zeros((M, pad128(H) - H), np.float32)], axis=1)
        H = x.shape[1]
    g = x.reshape(M, H // GROUP, GROUP)
    amax = np.abs(g).max(axis=2)
    s = group_scale_pow2(amax) if pow2 else group_scale(amax)
    q = quant_rule(g, s[:, :, None]).reshape(M, H)
    return q, s


def permute_quant(x_bf16: np.ndarray, inv_map: np.ndarray, K: int, pow2: bool = False):
    """K1: quantise each token row once (C3, or C10 with ``pow2``) and place it
    at the K sorted rows inv_map[t*K+k].  x_bf16 [T,H] uint16 -> xq [T*K,H]
    u8, xs [T*K,H/128] f32."""
    x = bf16_to_f32(x_bf16)
    T, H = x.shape
    q, s = quant_1x128(x, pow2)
    R = T * K
    xq = np.empty((R, q.shape[1]), np.uint8)
    xs = np.empty((R, s.shape[1]), np.float32)
    dst = np.asarray(inv_map, np.int64).reshape(T, K)
    for k in range(K):
        xq[dst[:, k]] = q
        xs[dst[:, k]] = s
    return xq, xs


def quantize_weight_blockwise(w_bf16: np.ndarray, pow2: bool = False):
    """C4: 128x128 blocks of W[e] in [N, K] layout (summary/fp8_expert_gemm_optimization.md:137)
    -> wq [E,N,Kp] u8, ws [E,Np/128,Kp/128] f32 with Np, Kp = pad128(N, K):
    per C9 edge blocks are the zero-padded blocks, and wq keeps N rows.
    ``pow2``: the block scales follow C10."""
    w = bf16_to_f32(w_bf16)
    E, N, Kd = w.shape
    Np, Kp = pad128(N), pad128(Kd)
    if (Np, Kp) != (N, Kd):
        w = np.pad(w, ((0, 0), (0, Np - N), (0, Kp - Kd)))
    b = w.reshape(E, Np // GROUP, GROUP, Kp // GROUP, GROUP)
    amax = np.abs(b).max(axis=(2, 4))
    s = group_scale_pow2(amax) if pow2 else group_scale(amax)
    q = quant_rule(b, s[:, :, None, :, None]).reshape(E, Np, Kp)[:, :N]
    return np.ascontiguousarray(q), s


# ---------------------------------------------------------------------------
# K2: grouped GEMM
# ---------------------------------------------------------------------------


def dequant_rows(q: np.ndarray, s: np.ndarray) -> np.ndarray:
    """[M,K] fp8 with [M,K/128] scales -> float64."""
    M, Kd = q.shape
    v = e4m3_decode(q).astype(np.float64).reshape(M, Kd // GROUP, GROUP)
    return (v * s.astype(np.float64)[:, :, None]).reshape(M, Kd)


def dequant_weight(q: np.ndarray, s: np.ndarray) -> np.ndarray:
    """[N,K] fp8 with [ceil(N/128),K/128] scales -> float64 (K the padded
    pitch; a short last row block uses its block's scale)."""
    N, Kd = q.shape
    Np = pad128(N)
    v = e4m3_decode(q).astype(np.float64)
    if Np != N:
        v = np.concatenate([v, np.zeros((Np - N, Kd))], axis=0)
    v = v.reshape(Np // GROUP, GROUP, Kd // GROUP, GROUP)
    return (v * s.astype(np.float64)[:, None, :, None]).reshape(Np, Kd)[:N]


def grouped_gemm_fp8(a, a_s, b, b_s, offsets) -> np.ndarray:
    """C5 in float64: per expert e, rows [offsets[e], offsets[e+1]) times
    dequantised W[e]^T.  "fp8 dot -> fp32 acc -> dequant -> bf16"
    (summary/fp8_expert_gemm_optimization.md:89-95) applied per 128-K block;
    dropless, zero-token experts produce nothing
    (moe/MegatronCore_MoE_reading_notes.md:695).  Returns float64 [R, N]."""
    R = a.shape[0]
    E, N, _ = b.shape
    out = np.zeros((R, N), np.float64)
    for e in range(E):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if hi <= lo:
            continue
        out[lo:hi] = dequant_rows(a[lo:hi], a_s[lo:hi]) @ dequant_weight(b[e], b_s[e]).T
    return out


# ---------------------------------------------------------------------------
# K3: SwiGLU + requant
# ---------------------------------------------------------------------------


def silu_f32(g: np.ndarray) -> np.ndarray:
    """silu(g) = g / (1 + exp(-g)) in fp32 with expf32."""
    g = np.asarray(g, np.float32)
    return (g / (F32(1.0) + expf32(-g)).astype(np.float32)).astype(np.float32)


def swiglu_quant(c1_bf16: np.ndarray, pow2: bool = False):
    """C6: h = silu(g) * u in fp32 (g = columns [0,I), u = [I,2I);
    moe/MoE_detailed_computation_dataflow.md:172-174), then C3 (C10 with
    ``pow2``) per 1x128."""
    c1 = bf16_to_f32(c1_bf16)
    I = c1.shape[1] // 2
    h = (silu_f32(c1[:, :I]) * c1[:, I:]).astype(np.float32)
    return quant_1x128(h, pow2)


# ---------------------------------------------------------------------------
# K5: combine
# ---------------------------------------------------------------------------


def unpermute_combine(y_bf16: np.ndarray, inv_map: np.ndarray, w: np.ndarray, K: int):
    """C7: out[t] = bf16(sum_k w[t,k] * y[inv_map[t*K+k]]), fp32, k order
    (moe/MoE_detailed_computation_dataflow.md:195; fp32 accumulator per
    notes/2026-04/2026-04-10_monolithmoe_layout_c_pack_optimization.md:67)."""
    y = bf16_to_f32(y_bf16)
    R, H = y.shape
    T = R // K
    dst = np.asarray(inv_map, np.int64).reshape(T, K)
    w = np.asarray(w, np.float32).reshape(T, K)
    acc = np.zeros((T, H), np.float32)
    for k in range(K):
        acc = (acc + (w[:, k:k + 1] * y[dst[:, k]]).astype(np.float32)).astype(np.float32)
    return f32_to_bf16(acc)


# ---------------------------------------------------------------------------
# M: the whole layer
# ---------------------------------------------------------------------------


def moe_forward(x_bf16, logits, w1q, w1s, w2q, w2s, K, bias=None, pow2: bool = False):
    """R -> K0 -> K1 -> K2(fc1) -> K3 -> K2(fc2) -> K5
    (moe/MoE_detailed_computation_dataflow.md:295-317).  GEMM outputs are
    rounded to bf16 between stages as the kernels do.  Returns a dict of every
    intermediate so tests can check stage by stage.  ``pow2``: the activation
    quantisations follow C10 (the weights' scales are whatever w1s, w2s hold)."""
    E = w1q.shape[0]
    idx, w = router_topk(logits, K, bias)
    row_map, inv_map, counts, offsets = route_sort(idx, E)
    xq, xs = permute_quant(x_bf16, inv_map, K, pow2)
    c1 = f32_to_bf16(grouped_gemm_fp8(xq, xs, w1q, w1s, offsets).astype(np.float32))
    hq, hs = swiglu_quant(c1, pow2)
    y = f32_to_bf16(grouped_gemm_fp8(hq, hs, w2q, w2s, offsets).astype(np.float32))
    out = unpermute_combine(y, inv_map, w, K)
    return dict(topk_idx=idx, topk_w=w, row_map=row_map, inv_map=inv_map, counts=counts,
                offsets=offsets, xq=xq, xs=xs, c1=c1, hq=hq, hs=hs, y=y, out=out)


# ---------------------------------------------------------------------------
# Backward (config 5): dgrad / wgrad grouped GEMMs, 128x1 column quantisation,
# SwiGLU and combine backward.  Recipe: E4M3 1x128 activation/grad tiles for
# the row-major (dgrad) operands and transposed 128x1 column tiles for the
# wgrad operands (moe/MegatronCore_MoE_reading_notes.md:498-501); variable-K
# wgrad grouped GEMM (notes/2026-04/2026-04-21_gptoss_10_moe_fp8_grouped_gemm_diagnosis.md:125;
# notes/2026-04/2026-04-25_gptoss_21_turbo_grouped_mlp_trace_evidence.md:95).
# ---------------------------------------------------------------------------


def transpose_blockwise(wq: np.ndarray, ws: np.ndarray, k: int | None = None):
    """[E,N,Kp] fp8 + [E,NB,KB] scales -> [E,K,Np] + [E,KB,NB], with K = k
    (default Kp) and Np = pad128(N) (C9 padding: zero columns past N).
    128x128 block quantisation commutes with the transpose, so the dgrad
    weights are the forward bytes transposed (no requantisation)."""
    E, N, Kp = wq.shape
    Kd = Kp if k is None else int(k)
    full = np.zeros((E, pad128(N), Kp), np.uint8)
    full[:, :N] = wq
    return (np.ascontiguousarray(full.transpose(0, 2, 1)[:, :Kd]),
            np.ascontiguousarray(ws.transpose(0, 2, 1)))


def pad_offsets(offsets: np.ndarray) -> np.ndarray:
    """Per-expert row segments rounded up to whole 128-row groups:
    pad[e+1] = pad[e] + ceil(count_e / 128) * 128."""
    off = np.asarray(offsets, np.int64)
    cnt = np.diff(off)
    pad = np.zeros(off.size, np.int64)
    pad[1:] = np.cumsum((cnt + GROUP - 1) // GROUP * GROUP)
    return pad.astype(np.int32)


def quant_cols_128x1(x: np.ndarray, offsets: np.ndarray, pow2: bool = False):
    """Transposed 128x1 quantisation for the wgrad operands.  x [R, C] float32
    with expert row segments offsets[E+1].  Each expert's rows are split into
    groups of 128 starting at its first row (the last group may be short);
    group g of expert e lands at columns pad[e] + 128*g .. of the transposed
    output, short groups zero-padded.  C3 applies per (column, group), or C10
    (power-of-two scales) with ``pow2``.
    -> xT_q [C, Rp] u8, xT_s [C, Rp/128] f32, pad offsets [E+1] i32."""
    x = np.asarray(x, np.float32)
    R, C = x.shape
    pad = pad_offsets(offsets)
    Rp = int(pad[-1])
    xt = np.zeros((C, Rp), np.float32)
    for e in range(len(offsets) - 1):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        xt[:, pad[e]:pad[e] + (hi - lo)] = x[lo:hi].T
    q, s = quant_1x128(xt, pow2) if Rp else (np.zeros((C, 0), np.uint8), np.zeros((C, 0), np.float32))
    return q, s, pad


def grouped_gemm_fp8_wgrad(aTq, aTs, bTq, bTs, pad, E: int) -> np.ndarray:
    """dW[e] = A_e^T B_e over expert e's rows: aT [N, Rp], bT [K, Rp] (rows
    contiguous, 128x1 scales [*, Rp/128]) -> float64 [E, N, K]; zero for
    experts without rows."""
    N, K = aTq.shape[0], bTq.shape[0]
    out = np.zeros((E, N, K), np.float64)
    for e in range(E):
        lo, hi = int(pad[e]), int(pad[e + 1])
        if hi <= lo:
            continue
        A = dequant_rows(aTq[:, lo:hi], aTs[:, lo // GROUP:hi // GROUP])
        B = dequant_rows(bTq[:, lo:hi], bTs[:, lo // GROUP:hi // GROUP])
        out[e] = A @ B.T
    return out


def swiglu_bwd(c1_bf16: np.ndarray, dh_bf16: np.ndarray) -> np.ndarray:
    """d(silu(g)*u): with s = 1/(1+exp(-g)) (fp32, library exp, IEEE division):
    du = dh*(g*s); dg = (dh*u) * (s*(1 + g*(1 - s))); evaluated in exactly this
    order in fp32, stored as bf16 [R, 2I] = [dg | du]."""
    c1 = bf16_to_f32(c1_bf16)
    dh = bf16_to_f32(dh_bf16)
    I = c1.shape[1] // 2
    g, u = c1[:, :I], c1[:, I:]
    one = F32(1.0)
    s = (one / (one + expf32(-g)).astype(np.float32)).astype(np.float32)
    silu = (g * s).astype(np.float32)
    ds = (s * (one + (g * (one - s).astype(np.float32)).astype(np.float32)).astype(np.float32)).astype(np.float32)
    du = (dh * silu).astype(np.float32)
    dg = ((dh * u).astype(np.float32) * ds).astype(np.float32)
    return f32_to_bf16(np.concatenate([dg, du], axis=1))


def combine_bwd(dout_bf16, y_bf16, inv_map, w, K: int):
    """Backward of C7: dy[inv_map[t*K+k]] = bf16(w[t,k] * dout[t]) and
    dw[t,k] = sum_h dout[t,h] * y[inv_map[t*K+k], h] (float64 here; the kernel
    reduces in fp32).  -> (dy [R,H] bf16, dw [T,K] float64)."""
    dout = bf16_to_f32(dout_bf16)
    y = bf16_to_f32(y_bf16)
    T, H = dout.shape
    dst = np.asarray(inv_map, np.int64).reshape(T, K)
    w = np.asarray(w, np.float32).reshape(T, K)
    dy = np.zeros((T * K, H), np.uint16)
    dw = np.zeros((T, K), np.float64)
    for k in range(K):
        dy[dst[:, k]] = f32_to_bf16((w[:, k:k + 1] * dout).astype(np.float32))
        dw[:, k] = (dout.astype(np.float64) * y[dst[:, k]].astype(np.float64)).sum(1)
    return dy, dw


def moe_backward(fwd: dict, x_bf16, w1q, w1s, w2q, w2s, dout_bf16, K: int, pow2: bool = False,
                 row_pow2: bool = False):
    """Backward of moe_forward given its intermediates and dout [T,H] bf16.
    Stages: combine bwd -> dy quant (1x128) -> fc2 dgrad (W2^T) -> fc2 wgrad
    (128x1 dy, h) -> SwiGLU bwd -> dc1 quant -> fc1 dgrad (W1^T) -> fc1 wgrad
    (128x1 dc1, x) -> un-permute (sum of the K replicas).  GEMM outputs are
    rounded to bf16 between stages like the kernels; wgrads stay float64.
    ``pow2``: the wgrad operands' 128x1 scales follow C10 instead of C3;
    ``row_pow2`` likewise for the dgrad operands' 1x128 scales."""
    E = w1q.shape[0]
    off = fwd["offsets"]
    inv = fwd["inv_map"]
    T = x_bf16.shape[0]
    dy, dw = combine_bwd(dout_bf16, fwd["y"], inv, fwd["topk_w"], K)
    dyq, dys = quant_1x128(bf16_to_f32(dy), row_pow2)
    h = bf16_to_f32(fwd["c1"])
    I = h.shape[1] // 2
    H = x_bf16.shape[1]
    w2tq, w2ts = transpose_blockwise(w2q, w2s, k=I)
    dh = f32_to_bf16(grouped_gemm_fp8(dyq, dys, w2tq, w2ts, off).astype(np.float32))
    # h as the forward saves it: silu(g)*u in fp32, rounded to bf16
    hh = bf16_to_f32(f32_to_bf16((silu_f32(h[:, :I]) * h[:, I:]).astype(np.float32)))
    dyTq, dyTs, pad = quant_cols_128x1(bf16_to_f32(dy), off, pow2)
    hTq, hTs, _ = quant_cols_128x1(hh, off, pow2)
    dW2 = grouped_gemm_fp8_wgrad(dyTq, dyTs, hTq, hTs, pad, E)
    dc1 = swiglu_bwd(fwd["c1"], dh)
    dc1q, dc1s = quant_1x128(bf16_to_f32(dc1), row_pow2)
    w1tq, w1ts = transpose_blockwise(w1q, w1s, k=H)
    dxs = f32_to_bf16(grouped_gemm_fp8(dc1q, dc1s, w1tq, w1ts, off).astype(np.float32))
    xs_sorted = bf16_to_f32(x_bf16)[fwd["row_map"] // K]
    dcTq, dcTs, _ = quant_cols_128x1(bf16_to_f32(dc1), off, pow2)
    xTq, xTs, _ = quant_cols_128x1(xs_sorted, off, pow2)
    dW1 = grouped_gemm_fp8_wgrad(dcTq, dcTs, xTq, xTs, pad, E)
    dx = unpermute_combine(dxs, inv, np.ones((T, K), np.float32), K)
    return dict(dy=dy, dw=dw, dh=dh, dW2=dW2, dc1=dc1, dxs=dxs, dW1=dW1, dx=dx, pad=pad)
