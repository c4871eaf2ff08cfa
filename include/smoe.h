/*
 * smoe.h — C ABI of the MI355X (gfx950) SimpleMoE expert-layer hot path.
 *
 * The reference (xmpeng-dev/system-lab) ships no callable code for this path;
 * its notes quote the call shapes of the external operators it drove on
 * MI355X.  Each entry point below names the reference interface it replaces
 * (file:line under the reference tree).
 *
 * Conventions shared by every entry point:
 *   - returns 0 on success, a negative SMOE_EINVAL_* code on a rejected
 *     argument (checked on the host before anything touches the GPU), or a
 *     positive hipError_t value when a HIP launch fails;
 *   - takes the HIP stream (hipStream_t passed as void*) last, enqueues work on
 *     it and never synchronises, so routing counts stay on the device;
 *   - the caller owns every buffer; the library allocates no device memory;
 *   - bf16 tensors are passed as uint16_t (raw bf16 bits), fp8 tensors as
 *     uint8_t holding OCP float8_e4m3fn bytes (max 448, 0x7f/0xff = NaN);
 *   - every pointer must be 16-byte aligned; E <= SMOE_MAX_EXPERTS;
 *   - H, I, N and C (the row length of a quantised tensor) must be multiples
 *     of 16; a GEMM's K argument is the fp8 operands' row pitch, a multiple
 *     of 128.  A dimension D that is not a multiple of 128 (GPT-OSS:
 *     H = I = 2880) is quantised as if zero-padded to Dp = ceil(D/128)*128:
 *     the short last group's amax is over its valid elements, its padding is
 *     byte 0, and the fp8 tensor keeps the padded pitch Dp (its scales have
 *     Dp/128 groups per row); a weight's short last row or column block is
 *     the zero-padded block.  bf16 tensors keep the tight pitch D.  (Blockwise
 *     fp8 GEMMs align dimensions to 16: moe/MegatronCore_MoE_reading_notes.md:541-543.)
 *
 * Semantics (binding for the kernels and the CPU oracle alike):
 *   pair p = t*K + k; rows are sorted stably by expert id, ties by ascending p;
 *   row_map[r] = p, inv_map[p] = r, offsets = exclusive scan of counts.
 *   1x128 activation quantisation per row and 128-column group g:
 *     amax = max|x|, s = amax/448 (fp32 RN; s = 1 when amax == 0),
 *     q = e4m3_rne(clamp(x/s, -448, 448)); the stored scale is s.
 *   128x128 weight quantisation applies the same rule over each block.
 */
#ifndef SMOE_H_
#define SMOE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SMOE_MAX_EXPERTS 1024

enum {
  SMOE_OK = 0,
  SMOE_EINVAL_NULL = -1,      /* a required pointer is NULL                 */
  SMOE_EINVAL_DIM = -2,       /* a dimension is <= 0 or out of range         */
  SMOE_EINVAL_ALIGN128 = -3,  /* a dimension not a multiple of 16 (128 where
                                 noted, e.g. a GEMM's padded K)              */
  SMOE_EINVAL_EXPERTS = -4,   /* E <= 0 or E > SMOE_MAX_EXPERTS              */
  SMOE_EINVAL_WORKSPACE = -5, /* workspace NULL or smaller than required     */
  SMOE_EINVAL_PTRALIGN = -6,  /* a pointer is not 16-byte aligned            */
  SMOE_EINVAL_TOPK = -7,      /* K <= 0, K > E or K > 32                     */
  SMOE_EINVAL_MODE = -8,      /* an enumerated mode argument is out of range */
};

/* Human-readable text for a status code (never NULL). */
const char* smoe_strerror(int status);

/* Library version string, e.g. "smoe 0.1 gfx950". */
const char* smoe_version(void);

/*
 * Router: softmax over fp32 logits, optional per-expert selection bias,
 * top-K by (score desc, expert id asc), weights renormalised over the K
 * picks.  logits [T,E] f32, bias [E] f32 or NULL -> topk_idx [T,K] i32,
 * topk_w [T,K] f32.
 * Replaces the router "gating linear -> softmax -> top-k -> renorm"
 * (moe/MoE_detailed_computation_dataflow.md:53-66) and the aux-loss-free
 * selection bias (moe/MegatronCore_MoE_reading_notes.md:688-697).
 */
int smoe_router_topk(const float* logits, const float* bias, int T, int E, int K,
                     int32_t* topk_idx, float* topk_w, void* stream);

/*
 * Router backward: dtopk_w [T,K] f32 (gradient of the renormalised weights)
 * -> dlogits [T,E] f32, through the renormalisation and the softmax (the
 * selection bias has no gradient).  topk_idx are the forward's picks.  With
 * S = sum_k p[s_k] and c = sum_k g_k w_k:
 *   dp[s_k] = (g_k - c) / S,  dlogits_e = p_e (dp_e - sum_k p[s_k] dp[s_k]).
 * Replaces the router's autograd backward (gate -> softmax -> top-k ->
 * renorm, moe/MoE_detailed_computation_dataflow.md:53-66, backward chain
 * :209-226).
 */
int smoe_router_topk_bwd(const float* logits, const int32_t* topk_idx, const float* dtopk_w,
                         int T, int E, int K, float* dlogits, void* stream);

/*
 * Expert sort: stable counting sort of the T*K (token, slot) pairs by expert.
 * topk_idx [T,K] i32 -> row_map [T*K], inv_map [T*K], counts [E],
 * offsets [E+1] (all i32).  ws (16-byte aligned) must hold
 * smoe_route_sort_workspace_size() bytes.
 * Ids outside [0, E) are an error the call cannot report synchronously (they
 * live on the device): such a pair gets no row and inv_map[p] = -1, so
 * offsets[E] = T*K minus their number (row_map[offsets[E] ..] is then left
 * unwritten), and the int32 at byte
 * SMOE_ROUTE_STATUS_OFFSET of ws receives that number (0 when every id is
 * valid).  The status word is rewritten by every call.
 * Replaces the pack sort phase that yields pack_perm "sorted pair index ->
 * original pair index" (notes/2026-04/2026-04-10_monolithmoe_layout_c_pack_optimization.md:56,80)
 * and Megatron's tokens_per_expert computation in Dispatcher.permute
 * (moe/MegatronCore_MoE_reading_notes.md:94-99), without the host .tolist()
 * sync (summary/fp8_expert_gemm_optimization.md:190).
 */
#define SMOE_ROUTE_STATUS_OFFSET 0
size_t smoe_route_sort_workspace_size(int T, int K, int E);
int smoe_route_sort(const int32_t* topk_idx, int T, int K, int E, int32_t* row_map,
                    int32_t* inv_map, int32_t* counts, int32_t* offsets, void* ws,
                    size_t ws_bytes, void* stream);

/*
 * Allocation-free variant of smoe_route_sort (no counterpart in the
 * reference: it is for callers that cannot allocate device memory, such as
 * code under HIP graph capture or a serving loop that forbids allocation).
 * Same arguments and bytes as smoe_route_sort without ws / ws_bytes: the
 * workspace is a static device array inside the library (one per GPU,
 * smoe_route_sort_noalloc_max_bytes() bytes, held until the process ends).
 * Sizes whose workspace would exceed it (E * ceil(T*K/512) * 4 + 16 bytes >
 * the maximum, e.g. E = 256 with T*K above 2M pairs) return
 * SMOE_EINVAL_WORKSPACE.  The routing status word is written to the static
 * array and not exposed: offsets[E] < T*K still reports dropped ids.  Every
 * call on one GPU shares the array: calls that overlap on one GPU (other
 * streams or threads) race.  It calls no allocator.
 */
size_t smoe_route_sort_noalloc_max_bytes(void);
int smoe_route_sort_noalloc(const int32_t* topk_idx, int T, int K, int E, int32_t* row_map,
                            int32_t* inv_map, int32_t* counts, int32_t* offsets, void* stream);

/*
 * Router fused with the sort: smoe_router_topk's outputs plus smoe_route_sort's,
 * with the sort's per-segment expert histogram counted inside the router
 * launch (three launches in all, no host sync).  Same bytes as
 * smoe_router_topk followed by smoe_route_sort; ws as for smoe_route_sort.
 * Replaces the fused router kernel with its expert histogram that feeds the
 * permutation ("fused router with aux score", notes/2026-04/2026-04-25_gptoss_22_sync_free_moe_stage_audit.md:25-26,104-124).
 */
int smoe_route_topk_sort(const float* logits, const float* bias, int T, int E, int K,
                         int32_t* topk_idx, float* topk_w, int32_t* row_map, int32_t* inv_map,
                         int32_t* counts, int32_t* offsets, void* ws, size_t ws_bytes,
                         void* stream);

/*
 * Fused permute + 1x128 fp8 quantisation.  Each token row of x [T,H] bf16 is
 * read once, quantised once and its fp8 bytes and scales written to the K
 * sorted rows inv_map[t*K+k]: xq [T*K,Hp] u8, xs [T*K,Hp/128] f32 (Hp =
 * H padded to a multiple of 128, see the conventions above).
 * Replaces Dispatcher.permute(x, routing_map) followed by the separate
 * quantize_fp8 launches (notes/2026-04/2026-04-21_gptoss_10_moe_fp8_grouped_gemm_diagnosis.md:38-46)
 * with the blockwise 1x128 activation recipe
 * (moe/MegatronCore_MoE_reading_notes.md:498-501).
 */
int smoe_permute_quant(const uint16_t* x, const int32_t* inv_map, int T, int H, int K,
                       uint8_t* xq, float* xs, void* stream);

/*
 * Scale rule of the row and weight quantisers' _ex entry points:
 *   SMOE_SCALE_AMAX  s = amax/448 (fp32 RN, 1 when amax == 0): the rule of
 *                    the entry points without _ex;
 *   SMOE_SCALE_POW2  s = the least power of two >= RN(amax/448), at least
 *                    2^-127 (1 when amax == 0).  x/s is then exact and s is
 *                    an E8M0 value: the power-of-two scales of the MXFP8
 *                    recipe (moe/MegatronCore_MoE_reading_notes.md:503-504)
 *                    at the blockwise recipe's 1x128 / 128x128 granularity.
 *                    smoe_grouped_gemm_fp8_packed_e8m0 applies such scales
 *                    in the MFMA.
 * Any other value returns SMOE_EINVAL_MODE.  The bytes for SMOE_SCALE_AMAX
 * equal those of the entry point without _ex.
 */
#define SMOE_SCALE_AMAX 0
#define SMOE_SCALE_POW2 1

/* smoe_permute_quant with a scale rule (SMOE_SCALE_*). */
int smoe_permute_quant_ex(const uint16_t* x, const int32_t* inv_map, int T, int H, int K,
                          uint8_t* xq, float* xs, int scale_mode, void* stream);

/*
 * Dispatch convenience: smoe_route_sort followed by smoe_permute_quant on one
 * stream (no host sync).  ws as for smoe_route_sort.
 */
int smoe_dispatch_quant(const uint16_t* x, const int32_t* topk_idx, int T, int H, int K,
                        int E, int32_t* row_map, int32_t* inv_map, int32_t* counts,
                        int32_t* offsets, uint8_t* xq, float* xs, void* ws,
                        size_t ws_bytes, void* stream);

/*
 * 128x128 blockwise fp8 weight quantisation.  w [E,N,Kdim] bf16 (Kdim
 * contiguous, "NK" layout) -> wq [E,N,Kp] u8, ws [E,ceil(N/128),Kp/128] f32
 * with Kp = Kdim padded to a multiple of 128 (padding columns 0).
 * Replaces the weight-cache refresh (summary/fp8_expert_gemm_optimization.md:135-143)
 * under the 128x128 weight-block recipe (moe/MegatronCore_MoE_reading_notes.md:498-501).
 */
int smoe_quantize_weight_blockwise(const uint16_t* w, int E, int N, int Kdim, uint8_t* wq,
                                   float* ws, void* stream);

/* smoe_quantize_weight_blockwise with a scale rule (SMOE_SCALE_*). */
int smoe_quantize_weight_blockwise_ex(const uint16_t* w, int E, int N, int Kdim, uint8_t* wq,
                                      float* ws, int scale_mode, void* stream);

/*
 * Self-test of the fast quantisation path (no counterpart in the reference:
 * it proves that the faster kernels keep the bit-exact contract).  The
 * contract's rule is e4m3(clamp(x / s)) with an IEEE division and an RNE
 * encoder.  The kernels instead divide bf16 inputs with a reciprocal and one
 * correction, and encode with the hardware conversion.  Checked on the GPU,
 * exhaustively: (1) the bytes of the bf16 path for every finite bf16 x and
 * every positive finite bf16 amax >= |x| (s = amax / 448), about 1.07e9
 * pairs; (2) the hardware encoder for every fp32 with |v| <= 448, about
 * 2.28e9 values; (3) the hardware fp32 -> bf16 conversion the kernels
 * use for bf16 outputs, against the software RNE rule, for every fp32 bit
 * pattern (NaN only needs to stay a NaN of the same sign).  counts [6] u64
 * on the device, zeroed by the caller, receives: mismatches (1), pairs
 * checked (1), mismatches (2), values checked (2), mismatches (3), values
 * checked (3).
 */
int smoe_selftest_quant(unsigned long long* counts, void* stream);

/*
 * No counterpart in the reference: a check of the sigmoid's reciprocal in
 * the SwiGLU backward.  The kernels form 1/b as v_rcp_f32 plus one Newton
 * step instead of the IEEE division; this compares the two, on the GPU, for
 * every fp32 b in [2^-126, 2^126) and for +inf (about 2.11e9 values).
 * counts [2] u64 on the device, zeroed by the caller, receives: mismatches,
 * values checked.
 */
int smoe_selftest_recip(unsigned long long* counts, void* stream);

/*
 * Dropless fp8 grouped GEMM with blockwise scales.  For each expert e and each
 * row r in [offsets[e], offsets[e+1]):
 *   c[r,n] = bf16( sum_kb as[r,kb]*bs[e,n/128,kb] * sum_{k in kb} a[r,k]*b[e,n,k] )
 * a [R,Kdim] u8, as [R,Kdim/128] f32, b [E,N,Kdim] u8, bs [E,ceil(N/128),Kdim/128]
 * f32, offsets [E+1] i32 on the device -> c [R,N] bf16; Kdim is the padded
 * pitch (a multiple of 128), N a multiple of 16.  Zero-token experts
 * produce no tiles.  offsets[] is read on the device only; the kernel clamps
 * every expert's range to rows [0, R), so malformed offsets (decreasing, or
 * past R) never cause an access outside a, as or c.  ws may be NULL
 * (smoe_grouped_gemm_fp8_workspace_size returns 0).
 * Replaces pt.ops.grouped_gemm_fp8(permuted, w1, tokens_per_expert, ...)
 * (notes/2026-04/2026-04-21_gptoss_10_moe_fp8_grouped_gemm_diagnosis.md:39) and
 * _fp8_fused_grouped_fwd(A_fp8, A_si, B_fp8, B_si, tpe)
 * (summary/fp8_expert_gemm_optimization.md:121-131), with blockwise instead
 * of per-tensor scales.
 */
size_t smoe_grouped_gemm_fp8_workspace_size(int E, int R, int N, int Kdim);
int smoe_grouped_gemm_fp8(const uint8_t* a, const float* as, const uint8_t* b,
                          const float* bs, const int32_t* offsets, int E, int R, int N,
                          int Kdim, uint16_t* c, void* ws, size_t ws_bytes, void* stream);

/*
 * fc1 grouped GEMM with the SwiGLU + 1x128 requantisation fused into its
 * epilogue: the result equals smoe_grouped_gemm_fp8(a, as, w1, w1s) -> c1
 * [R,2I] bf16 followed by smoe_swiglu_quant(c1) -> hq [R,I] u8, hs [R,I/128]
 * f32, byte for byte, without the c1 round trip through HBM.  w1 [E,2I,Kdim]
 * u8 holds gate rows [0,I) and up rows [I,2I); w1s [E,2I/128,Kdim/128].  c1
 * may be NULL; when given it also receives the bf16 fc1 output (the backward
 * pass needs it).  Requires I % 128 == 0 (the epilogue pairs 128-column gate
 * and up blocks; other I take the two-kernel path) and 2*I*Kdim < 2^31.
 * Replaces the grouped GEMM + activation_func_with_probs pair of the expert
 * FFN (moe/MoE_detailed_computation_dataflow.md:168-174;
 * notes/2026-04/2026-04-21_gptoss_10_moe_fp8_grouped_gemm_diagnosis.md:39-46).
 */
int smoe_grouped_gemm_fp8_swiglu(const uint8_t* a, const float* as, const uint8_t* w1,
                                 const float* w1s, const int32_t* offsets, int E, int R, int I,
                                 int Kdim, uint8_t* hq, float* hs, uint16_t* c1, void* stream);

/*
 * Weights packed for the register-loaded grouped GEMM: wq [E,N,Kdim] u8 (the
 * output of smoe_quantize_weight_blockwise) -> wp [E,N,Kdim] bytes in MFMA
 * fragment order: [E][N/16][Kdim/128][2][64][16 B], where half h, lane l holds
 * row 16*nb + l%16 at K offsets 128*kb + 64*h + 16*(l/16) .. +16.  The scales
 * are unchanged.  Requires N % 16 == 0 and Kdim % 128 == 0.
 * Replaces the fp8 weight cache refresh that keeps each layout the kernels
 * need (_refresh_fp8_weight_cache caching KN and NK,
 * summary/fp8_expert_gemm_optimization.md:133-137).
 */
int smoe_pack_weight_fp8(const uint8_t* wq, int E, int N, int Kdim, uint8_t* wp, void* stream);

/*
 * smoe_grouped_gemm_fp8 on packed weights (smoe_pack_weight_fp8): the same
 * c [R,N] bf16 (bit for bit whenever each 128-wide K block's products sum
 * exactly in fp32; else within the last bf16 bit), from a kernel that loads each wave's weights
 * straight into registers and keeps activation tiles three K steps ahead in
 * LDS.  Requires Kdim % 512 == 0 and N*Kdim < 2^32 (other shapes use
 * smoe_grouped_gemm_fp8).  Needs no workspace.
 * Replaces fp8_grouped_gemm_forward_prequantized_w(...) on cached weights
 * (summary/fp8_expert_gemm_optimization.md:121-131).
 */
int smoe_grouped_gemm_fp8_packed(const uint8_t* a, const float* as, const uint8_t* wp,
                                 const float* ws, const int32_t* offsets, int E, int R, int N,
                                 int Kdim, uint16_t* c, void* stream);

/*
 * smoe_grouped_gemm_fp8_packed for power-of-two scales (SMOE_SCALE_POW2 on
 * both operands): c within rounding of that kernel's (each K block's sum is
 * added to the accumulator inside the MFMA instead of by an fp32 fma), with
 * the scales applied by the scaled MFMA
 * (v_mfma_scale_f32_16x16x128_f8f6f4) from their exponent bytes and the
 * accumulators kept in the accumulation registers, which lets a workgroup
 * of 4 waves (256 x 64 each) replace the 8 of the packed kernel.  Scales
 * that are not powers of two are read by their exponent only (wrong
 * results).  Requires Kdim % 128 == 0, 512 <= Kdim <= 65536, N % 16 == 0
 * and N*Kdim < 2^32; wp from smoe_pack_weight_fp8.  No
 * counterpart of its own in the reference: the grouped GEMM it replaces is
 * that of smoe_grouped_gemm_fp8, under the MXFP8-style power-of-two scale
 * rule (moe/MegatronCore_MoE_reading_notes.md:503-504).
 */
int smoe_grouped_gemm_fp8_packed_e8m0(const uint8_t* a, const float* as, const uint8_t* wp,
                                      const float* ws, const int32_t* offsets, int E, int R,
                                      int N, int Kdim, uint16_t* c, void* stream);

/*
 * smoe_grouped_gemm_fp8_packed_e8m0 on packed W1 [E,2I,Kdim] with SwiGLU and
 * the power-of-two 1x128 requantisation in its epilogue: hq, hs equal
 * smoe_swiglu_quant_ex(c1, ..., SMOE_SCALE_POW2) of the c1 that
 * smoe_grouped_gemm_fp8_packed_e8m0 writes, and c1 itself is written when
 * not NULL.  Requires I % 128 == 0 and the Kdim range of
 * smoe_grouped_gemm_fp8_packed_e8m0.  Replaces the same grouped GEMM +
 * activation pair as smoe_grouped_gemm_fp8_swiglu
 * (summary/fp8_expert_gemm_optimization.md:121-131) under the MXFP8-style
 * scale rule (moe/MegatronCore_MoE_reading_notes.md:503-504).
 */
int smoe_grouped_gemm_fp8_packed_e8m0_swiglu(const uint8_t* a, const float* as,
                                             const uint8_t* w1p, const float* w1s,
                                             const int32_t* offsets, int E, int R, int I,
                                             int Kdim, uint8_t* hq, float* hs, uint16_t* c1,
                                             void* stream);

/*
 * smoe_grouped_gemm_fp8_swiglu on packed W1 (smoe_pack_weight_fp8 of w1
 * [E,2I,Kdim]): the same hq, hs (and c1 when not NULL) under the same
 * condition as smoe_grouped_gemm_fp8_packed.
 * Requires Kdim % 512 == 0, I % 128 == 0 and 2*I*Kdim < 2^32.
 * Replaces the same grouped GEMM + activation pair as
 * smoe_grouped_gemm_fp8_swiglu, on cached weights
 * (summary/fp8_expert_gemm_optimization.md:121-131).
 */
int smoe_grouped_gemm_fp8_packed_swiglu(const uint8_t* a, const float* as, const uint8_t* w1p,
                                        const float* w1s, const int32_t* offsets, int E, int R,
                                        int I, int Kdim, uint8_t* hq, float* hs, uint16_t* c1,
                                        void* stream);

/*
 * SwiGLU + 1x128 requantisation.  c1 [R,2I] bf16 with gate columns [0,I) and
 * up columns [I,2I): h = silu(g)*u in fp32 -> hq [R,Ip] u8, hs [R,Ip/128] f32
 * (Ip = I padded to a multiple of 128; h's columns past I are 0).
 * silu(g) = g / (1 + exp(-g)) with exp evaluated by the library's own
 * fp32 routine (Cody-Waite reduction + degree-7 Taylor polynomial).
 * Replaces activation_func_with_probs / the SwiGLU elementwise kernel
 * (notes/2026-04/2026-04-21_gptoss_10_moe_fp8_grouped_gemm_diagnosis.md:46;
 * moe/MoE_detailed_computation_dataflow.md:172-174) plus the fc2 input quant.
 */
int smoe_swiglu_quant(const uint16_t* c1, int R, int I, uint8_t* hq, float* hs,
                      void* stream);

/*
 * As smoe_swiglu_quant, and when h is not NULL also writes h rounded to bf16
 * (h [R,I]): the activation the fc2 weight gradient needs in the backward
 * pass (saved by the forward instead of recomputed).
 */
int smoe_swiglu_quant_h(const uint16_t* c1, int R, int I, uint8_t* hq, float* hs, uint16_t* h,
                        void* stream);

/* smoe_swiglu_quant_h with a scale rule (SMOE_SCALE_*) for hs; h may be NULL. */
int smoe_swiglu_quant_ex(const uint16_t* c1, int R, int I, uint8_t* hq, float* hs, uint16_t* h,
                         int scale_mode, void* stream);

/*
 * Weighted unpermute/combine: out[t] = bf16( sum_k w[t,k] * y[inv_map[t*K+k]] )
 * accumulated in fp32 in k order (each product and sum rounded separately).
 * y [T*K,H] bf16, inv_map [T*K] i32, w [T,K] f32 -> out [T,H] bf16.
 * Replaces Dispatcher.unpermute(expert_out, probs) / _unpermute_kernel
 * (notes/2026-04/2026-04-24_gptoss_16_tier1_elementwise_tax_audit.md:69;
 * moe/MoE_detailed_computation_dataflow.md:195).
 */
int smoe_unpermute_combine(const uint16_t* y, const int32_t* inv_map, const float* w,
                           int T, int K, int H, uint16_t* out, void* stream);

/* ---------------------------------------------------------------------------
 * Backward pass of the expert FFN in fp8.  The recipe is
 * the blockwise one: 1x128 row tiles for the dgrad operands, transposed
 * 128x1 column tiles for the wgrad operands, 128x128 weight blocks
 * (moe/MegatronCore_MoE_reading_notes.md:498-501); the wgrad GEMM is the
 * "variable-K" grouped GEMM of the reference's backends
 * (notes/2026-04/2026-04-21_gptoss_10_moe_fp8_grouped_gemm_diagnosis.md:125,
 * notes/2026-04/2026-04-25_gptoss_21_turbo_grouped_mlp_trace_evidence.md:95).
 *
 * The 128x1 column quantisers (the wgrad operands) take col_scale:
 *   SMOE_COLSCALE_FP32  s = amax/448 (fp32 RN, 1 when amax == 0), the rule
 *                       of every other quantiser;
 *   SMOE_COLSCALE_POW2  s = the least power of two >= RN(amax/448), at least
 *                       2^-127 (1 when amax == 0).  x/s is then exact and s is
 *                       an E8M0 value, which the wgrad's scaled MFMA applies
 *                       in hardware (SMOE_WGRAD_E8M0).  This is the
 *                       power-of-two scale of the MXFP8 recipe
 *                       (moe/MegatronCore_MoE_reading_notes.md:503-504) at the
 *                       blockwise recipe's 128-row granularity; it is opt-in.
 * The quantisers that also write 1x128 rows (smoe_quant_rows_cols,
 * smoe_swiglu_bwd_quant, smoe_unpermute_combine_bwd_quant) take in the same
 * argument the bit SMOE_ROWSCALE_POW2, which gives their row scales the
 * SMOE_SCALE_POW2 rule (their row scales follow the FP32 rule without it).
 * Any other value returns SMOE_EINVAL_MODE.
 * ------------------------------------------------------------------------- */
#define SMOE_COLSCALE_FP32 0
#define SMOE_COLSCALE_POW2 1
#define SMOE_ROWSCALE_POW2 2

/*
 * Plain 1x128 row quantisation (no permutation): x [M,C] bf16 ->
 * q [M,Cp] u8, s [M,Cp/128] f32 with the forward rule (Cp = C padded to a
 * multiple of 128).  Used for output grads
 * entering the dgrad GEMM (replaces quantize_fp8 of the grad,
 * notes/2026-04/2026-04-21_gptoss_10_moe_fp8_grouped_gemm_diagnosis.md:99).
 */
int smoe_quant_rows_1x128(const uint16_t* x, int M, int C, uint8_t* q, float* s, void* stream);

/* smoe_quant_rows_1x128 with a scale rule (SMOE_SCALE_*). */
int smoe_quant_rows_1x128_ex(const uint16_t* x, int M, int C, uint8_t* q, float* s,
                             int scale_mode, void* stream);

/*
 * Blockwise weight transpose for dgrad: wq [E,N,Kp] u8 + ws [E,NB,KB]
 * -> wqT [E,Kdim,Np] + wsT [E,KB,NB], with Kdim the weight's true K (Kp its
 * padded pitch), Np = N padded to a multiple of 128 (columns past N are 0),
 * NB = Np/128, KB = Kp/128.  128x128 block quantisation commutes with the
 * transpose, so no requantisation is needed.  Replaces the NK/KN
 * weight cache (summary/fp8_expert_gemm_optimization.md:135-143).
 */
int smoe_transpose_blockwise_fp8(const uint8_t* wq, const float* ws, int E, int N, int Kdim,
                                 uint8_t* wqT, float* wsT, void* stream);

/*
 * Transposed 128x1 column quantisation of x [R,C] bf16 whose rows are the
 * expert segments offsets[E+1].  When gather is not NULL, row r of the
 * operand is x[gather[r] / gather_div] (e.g. row_map and K: the sorted
 * tokens of the forward, gathered on the fly).  Each expert's rows are split
 * into 128-row groups from its first row (short last groups zero-padded);
 * group g of expert e is column block pad[e]/128 + g of the output.
 * C need only be a multiple of 16 (xTq has C rows).
 * -> xTq [C, ld] u8,
 * xTs [C, ld/128] f32, pad [E+1] i32 (pad[e+1] = pad[e] + ceil(count/128)*128).
 * ld must be >= smoe_quant_cols_ld(R, E) (an upper bound known on the host;
 * columns past pad[E] are left untouched) and ld/128 <= 65535.  Rows outside
 * [0, R) are never read, whatever offsets[] holds; gather[] entries are
 * trusted to index rows of x.
 */
int smoe_quant_cols_ld(int R, int E);
int smoe_quant_cols_128x1(const uint16_t* x, const int32_t* gather, int gather_div, int R, int C,
                          const int32_t* offsets, int E, int ld, uint8_t* xTq, float* xTs,
                          int32_t* pad, int col_scale, void* stream);

/*
 * Both quantisations of one tensor from a single read: x [R,C] bf16 ->
 * the 1x128 row quantisation xq [R,Cp] u8 + xs [R,Cp/128] f32 (the bytes of
 * smoe_quant_rows_1x128) and the transposed 128x1 column quantisation
 * xTq / xTs / pad of smoe_quant_cols_128x1 (no gather).  Rows are those of
 * the expert segments offsets[E+1], which must cover [0, R) for every row
 * of xq to be written.  The fp8 recipe quantises activation grads both
 * ways, 1x128 for dgrad and 128x1 for wgrad
 * (moe/MegatronCore_MoE_reading_notes.md:498-501); this replaces the two
 * separate passes of the backward over dy and dc1.
 */
int smoe_quant_rows_cols(const uint16_t* x, int R, int C, const int32_t* offsets, int E, int ld,
                         uint8_t* xq, float* xs, uint8_t* xTq, float* xTs, int32_t* pad,
                         int col_scale, void* stream);

/*
 * SwiGLU backward fused into both quantisations of its output: computes
 * dc1 [R,2I] = [dg | du] from c1 [R,2I] and dh [R,I] exactly as
 * smoe_swiglu_bwd does (bf16-rounded), and writes the
 * smoe_quant_rows_cols outputs of dc1 (dcq [R,2I] u8, dcs [R,2I/128],
 * dcTq [2I,ld] u8, dcTs [2I,ld/128], pad) without storing dc1 itself,
 * unless dc1 is not NULL.  Same bytes as smoe_swiglu_bwd followed by
 * smoe_quant_rows_cols.  Requires I % 128 == 0 (a workgroup takes one
 * 128-column slab of each half; other I take those two calls).  Replaces the "dexpert" activation backward and
 * the requantisation of its gradient
 * (moe/MoE_detailed_computation_dataflow.md:209-226;
 * moe/MegatronCore_MoE_reading_notes.md:498-501).
 */
int smoe_swiglu_bwd_quant(const uint16_t* c1, const uint16_t* dh, int R, int I,
                          const int32_t* offsets, int E, int ld, uint8_t* dcq, float* dcs,
                          uint8_t* dcTq, float* dcTs, int32_t* pad, uint16_t* dc1, int col_scale,
                          void* stream);

/*
 * Variable-K grouped fp8 GEMM for weight gradients:
 *   dW[e][n][k] = sum over expert e's groups g of aTs[n,g]*bTs[k,g]*sum_r aT[n,r]*bT[k,r]
 * aT [N, ld] / bT [Kdim, ld] u8 and scales [*, ld/128] from
 * smoe_quant_cols_128x1, pad [E+1] -> dW [E, N, Kdim] f32 (zeros for experts
 * without rows).  N and Kdim must be multiples of 16.  Replaces the grouped variable-K wgrad
 * (notes/2026-04/2026-04-25_gptoss_21_turbo_grouped_mlp_trace_evidence.md:95).
 */
int smoe_grouped_gemm_fp8_wgrad(const uint8_t* aT, const float* aTs, const uint8_t* bT,
                                const float* bTs, const int32_t* pad, int E, int N, int Kdim,
                                int ld, float* dW, void* stream);

/*
 * smoe_grouped_gemm_fp8_wgrad with a choice of output (the same fp32 tile
 * sums in every mode):
 *   SMOE_WGRAD_F32      dW f32, written (what smoe_grouped_gemm_fp8_wgrad does);
 *   SMOE_WGRAD_F32_ACC  dW f32 += tile (one fp32 addition per value);
 *   SMOE_WGRAD_BF16     dW bf16 = RNE(tile);
 *   SMOE_WGRAD_BF16_ACC dW bf16 = RNE(float(dW) + tile).
 * The accumulating modes add into a framework's gradient-accumulation
 * buffer in the wgrad epilogue (experts without rows leave it untouched), in
 * place of a separate fp32 gradient and an add pass: Megatron's
 * gradient_accumulation_fusion, which writes the weight gradient straight into
 * the fp32 main_grad (notes/mlperf-llama/2026-04-29_nemo_vs_primus_config_diff.md:233-235),
 * and the bf16 main_grads_dtype of the reference's GPT-OSS runs
 * (notes/2026-04/2026-04-20_gptoss_05_borrow_from_deepseek_v3_config.md:23,48).
 * mode may also hold SMOE_WGRAD_E8M0: the operands' scales are powers of two
 * (SMOE_COLSCALE_POW2), read by their exponent only and applied by the
 * scaled MFMA (v_mfma_scale_f32_16x16x128_f8f6f4), so the 128-row groups
 * accumulate in the MFMA with no per-output scale arithmetic.  With scales
 * that are not powers of two this flag gives wrong results.
 * Any other mode returns SMOE_EINVAL_MODE.
 */
#define SMOE_WGRAD_F32 0
#define SMOE_WGRAD_F32_ACC 1
#define SMOE_WGRAD_BF16 2
#define SMOE_WGRAD_BF16_ACC 3
#define SMOE_WGRAD_E8M0 4
int smoe_grouped_gemm_fp8_wgrad_ex(const uint8_t* aT, const float* aTs, const uint8_t* bT,
                                   const float* bTs, const int32_t* pad, int E, int N, int Kdim,
                                   int ld, void* dW, int mode, void* stream);

/*
 * SwiGLU backward: c1 [R,2I] (gate | up) and dh [R,I] bf16 -> dc1 [R,2I]
 * bf16 = [dg | du] with s = 1/(1+exp(-g)), du = dh*(g*s),
 * dg = (dh*u)*(s*(1 + g*(1-s))) in fp32 (library exp).  Replaces the SwiGLU
 * backward (notes/2026-04/2026-04-24_gptoss_16_tier1_elementwise_tax_audit.md:54).
 */
int smoe_swiglu_bwd(const uint16_t* c1, const uint16_t* dh, int R, int I, uint16_t* dc1,
                    void* stream);

/*
 * Combine backward: dy [T*K,H] bf16 with dy[inv_map[t*K+k]] = bf16(w[t,k]*dout[t]),
 * and dw [T,K] f32 = <dout[t], y[inv_map[t*K+k]]> (fp32 reduction).
 * Replaces the unpermute backward (moe/MoE_detailed_computation_dataflow.md:209-226).
 */
int smoe_unpermute_combine_bwd(const uint16_t* dout, const uint16_t* y, const int32_t* inv_map,
                               const float* w, int T, int K, int H, uint16_t* dy, float* dw,
                               void* stream);

/*
 * Combine backward fused with both quantisations of dy: writes dw [T,K] f32
 * as smoe_unpermute_combine_bwd does, and, without storing dy [T*K,H], the
 * smoe_quant_rows_cols outputs of dy (dyq [T*K,Hp] u8, dys [T*K,Hp/128],
 * dyTq [H,ld] u8, dyTs [H,ld/128], pad) over the expert segments offsets:
 * row r of dy is rebuilt inside the quantiser as bf16(w[p]*dout[p/K]) with
 * p = row_map[r] (row_map and inv_map inverse permutations of [0, T*K),
 * as smoe_route_sort writes them).  Same bytes as smoe_unpermute_combine_bwd
 * followed by smoe_quant_rows_cols.  With dyTq and dyTs both NULL the
 * column pass is skipped (pad is still written); smoe_combine_bwd_quant_cols
 * then gives it, e.g. on another stream.  Replaces dmerge and the
 * requantisation of its gradient (moe/MoE_detailed_computation_dataflow.md:209-226;
 * moe/MegatronCore_MoE_reading_notes.md:498-501).
 */
int smoe_unpermute_combine_bwd_quant(const uint16_t* dout, const uint16_t* y,
                                     const int32_t* inv_map, const int32_t* row_map,
                                     const float* w, int T, int K, int H, const int32_t* offsets,
                                     int E, int ld, uint8_t* dyq, float* dys, uint8_t* dyTq,
                                     float* dyTs, int32_t* pad, float* dw, int col_scale,
                                     void* stream);

/*
 * The column pass of smoe_unpermute_combine_bwd_quant alone: dyTq, dyTs and
 * pad, the same bytes, from dout, row_map and w (it does not read y or the
 * row outputs, so it may run beside the row pass).  col_scale is
 * SMOE_COLSCALE_FP32 or SMOE_COLSCALE_POW2.  Replaces the wgrad half of the
 * same requantisation (moe/MegatronCore_MoE_reading_notes.md:498-501).
 */
int smoe_combine_bwd_quant_cols(const uint16_t* dout, const int32_t* row_map, const float* w,
                                int T, int K, int H, const int32_t* offsets, int E, int ld,
                                uint8_t* dyTq, float* dyTs, int32_t* pad, int col_scale,
                                void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SMOE_H_ */
