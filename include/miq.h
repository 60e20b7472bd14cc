/* libmiq -- MI355X (gfx950) quantized-linear hot path, C ABI.
 *
 * Every entry point takes raw device pointers, element counts and a hipStream_t (passed as
 * void*; NULL is the default stream). Work is enqueued on that stream and the call returns
 * without synchronising. The caller owns all memory (inputs, outputs, workspace); the library
 * keeps no pointers between calls. Return value: MIQ_OK (0) or a negative MIQ_ERR_* code, with
 * a message for the calling thread in miq_last_error(). No exception crosses this boundary.
 *
 * Reference interfaces replaced (xnetsc/webpytorch, "webtorch"): each declaration cites the
 * reference function whose work it performs. In the reference those functions dispatch WGSL
 * through `plat.runKernel` (webgpu/wgpy_backends/webgpu/platform.py:39-43) or fall back to
 * numpy; here they are HIP kernels.
 */
#ifndef MIQ_H
#define MIQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MIQ_VERSION 1

/* return codes */
#define MIQ_OK 0
#define MIQ_ERR_INVALID (-1)     /* bad shape or argument (reference: AssertionError/ValueError) */
#define MIQ_ERR_ALIGN (-2)       /* pointer or leading dimension not aligned as required */
#define MIQ_ERR_UNSUPPORTED (-3) /* variant not implemented (reference: NotImplementedError) */
#define MIQ_ERR_HIP (-4)         /* a HIP runtime call or kernel launch failed */

/* element types of activations, outputs and scales */
#define MIQ_F32 0
#define MIQ_F16 1

/* Message describing the last error on the calling thread ("" if none). */
const char* miq_last_error(void);
/* MIQ_VERSION of the built library. */
int miq_version(void);

/* ---------------------------------------------------------------------------------------
 * GPTQ int4/int8 (AutoGPTQ layout)
 *   qweight int32 [K/per][N] (per = 32/bits), qzeros int32 [K/gs][N/per],
 *   scales fp16 or fp32 [K/gs][N], W[k][n] = s[g][n] * (q[k][n] - (z[g][n] + zero_offset)).
 * ------------------------------------------------------------------------------------- */

/* Full fp32 dequant, out [K][N]. g_idx (int32 [K], nullable) maps row -> group (act-order);
 * NULL means g = k / gs. Bit-exact with the reference's float64 product rounded to float32
 * for integer zero offsets.
 * Replaces: `_dequant_full` (webtorch/_core.py:4696-4720) and the dequant step of
 * `_gptq_matmul_np` (webtorch/_core.py:4046-4072). */
int miq_gptq_dequant_f32(const int32_t* qweight, const int32_t* qzeros, const void* scales,
                         int scales_dtype, const int32_t* g_idx, float* out, int K, int N,
                         int gs, int bits, float zero_offset, void* stream);

/* Act-order load-time repack: out row block r holds original rows perm[r*per + j]. With
 * perm = stable argsort(g_idx), groups become consecutive runs of gs rows and the layer runs
 * on the plain kernels with the activation gathered through the same perm.
 * Replaces: nothing in the reference, which ignores g_idx (webtorch/llm.py:569-573,
 * webtorch/_core.py:4420-4430); it is the load step behind `from_autogptq(..., g_idx=)`. */
int miq_gptq_repack_rows(const int32_t* qweight, const int32_t* perm, int32_t* out, int K, int N,
                         int bits, void* stream);

/* Bytes of workspace miq_gptq_gemv needs for this problem (0 if none). The first 4 MiB of a
 * workspace (the counter region) hold arrival counters, fixed-point split-K sums and their
 * escape masks, shared by every split-K entry point, that must be zero before the first call
 * on it; every call leaves them zero again. Partial sums, escape slots and staged activations
 * follow them. One workspace must not serve two calls that run concurrently.
 * Split-K sums are exact for every input: a K-slice partial that is NaN, infinite or of
 * magnitude >= 2^22 (beyond the fixed-point words) reaches the final sum as an fp32 value, so
 * NaN and infinities propagate as in an fp32 sum. (The one-row int4 kernel holds each 64-k step
 * of x in fixed point at the step's own scale, which a non-finite value has not: such a step
 * scales its products by NaN, so an infinite x gives NaN, not +-Inf, in the outputs it
 * reaches.) */
int miq_gptq_gemv_workspace(int M, int K, int N, int gs, int bits, int x_dtype, size_t* bytes);

/* Decode GEMV / skinny GEMM: out[M][N] = x[M][K] (gathered through perm if non-NULL)
 * @ W + bias (nullable, fp32). x fp16|fp32, scales fp16|fp32, out fp16|fp32, fp32
 * accumulation; fp16 x uses fp16 products (exact) with fp32 sums. Requires qweight 16-byte
 * aligned, N % 4 == 0 and gs a multiple of 32 (int4) or 16 (int8); efficient for M <= 8.
 * workspace (256-byte aligned, workspace_bytes >= miq_gptq_gemv_workspace) lets the K
 * dimension be split across workgroups; with NULL the call uses one workgroup per column
 * tile (slower) and fails for K too large to stage. For M == 1, bias may alias out (fp32):
 * out = out + x @ W, an in-place residual add.
 * Replaces: `_gptq_matmul` M == 1 dispatch to `_GPTQ_GEMV_WGSL`
 * (webtorch/_core.py:3926-3978, 4008-4027) and the bias add of `QuantizedLinear.forward`
 * (webtorch/_core.py:4446-4456). */
int miq_gptq_gemv(const void* x, int x_dtype, const int32_t* perm, const int32_t* qweight,
                  const int32_t* qzeros, const void* scales, int scales_dtype, const float* bias,
                  void* out, int out_dtype, int M, int K, int N, int gs, int bits,
                  float zero_offset, void* workspace, size_t workspace_bytes, void* stream);

/* miq_gptq_gemv without a workspace argument, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). It has
 * no counterpart in the reference. The split-K workspace is a fixed array in the library's
 * device memory, miq_gptq_gemv_noalloc_max_bytes() (16 MiB) on each GPU the library runs on,
 * held until the process ends; the first call on a GPU looks its address up and clears its
 * counter region (a fill kernel on `stream`), so that first call must be made outside graph
 * capture: made while `stream` captures, it fails with MIQ_ERR_INVALID and sets nothing up
 * (later calls, captured or not, are fine). The call itself allocates nothing. A problem
 * whose workspace (miq_gptq_gemv_workspace) exceeds the array fails with MIQ_ERR_INVALID
 * before launching anything. Every call on a GPU shares that GPU's array: calls that overlap
 * on one GPU (two streams, two threads) race and may give wrong results; calls issued on one
 * stream are ordered and safe. Arguments and results otherwise as miq_gptq_gemv. */
int miq_gptq_gemv_noalloc(const void* x, int x_dtype, const int32_t* perm, const int32_t* qweight,
                          const int32_t* qzeros, const void* scales, int scales_dtype, const float* bias,
                          void* out, int out_dtype, int M, int K, int N, int gs, int bits, float zero_offset,
                          void* stream);
/* Bytes of the fixed workspace array miq_gptq_gemv_noalloc uses. */
size_t miq_gptq_gemv_noalloc_max_bytes(void);

/* input transforms of miq_gptq_gemv_fused */
#define MIQ_X_PLAIN 0   /* x as given */
#define MIQ_X_RMSNORM 1 /* x[m] / sqrt(mean(x[m]^2) + eps) * norm_w, over the full K */
#define MIQ_X_SWIGLU 2  /* x rows hold [gate | up] (2K values): silu(gate) * up */

/* Decode GEMV with the preceding elementwise step fused into the activation staging:
 * out[M][N] = T(x) @ W + bias for fp32 x and out (M == 1 for the fused modes), with T the
 * x_mode transform. Same weight, workspace and bias rules as miq_gptq_gemv (bias may alias out).
 * Replaces: `_rms` + `_qkv` / `_mlp` of the decode step (webtorch/llm.py:1259-1268, 1489-1519),
 * each an RMSNorm or SwiGLU dispatch followed by a `_gptq_matmul`. */
int miq_gptq_gemv_fused(const float* x, int x_mode, const float* norm_w, float eps, const int32_t* perm,
                        const int32_t* qweight, const int32_t* qzeros, const void* scales,
                        int scales_dtype, const float* bias, float* out, int M, int K, int N, int gs,
                        int bits, float zero_offset, void* workspace, size_t workspace_bytes,
                        void* stream);

/* Bytes of workspace miq_gptq_gemm needs (0 if none); same contract as
 * miq_gptq_gemv_workspace (zeroed counters first, not shared by concurrent calls). */
int miq_gptq_gemm_workspace(int M, int K, int N, int gs, int bits, size_t* bytes);

/* Prefill / batched GEMM on the matrix cores: out[M][N] = x[M][K] (fp16, gathered through perm
 * if non-NULL) @ W + bias (nullable, fp32). W is dequantized exactly to the small integers
 * q - (z + zero_offset) in fp16 (zero_offset must be a small non-negative integer), fp16 x
 * fp16 products accumulate in fp32 and the fp32 group scale multiplies each chunk's sums.
 * scales fp16|fp32, out fp16|fp32. Requires x and qweight 16-byte aligned, N % 4 == 0 and
 * gs in {32, 64} or a multiple of 128. workspace as for miq_gptq_gemv. Up to 16 rows of int4
 * with gs 128 run a kernel that streams the weights like the GEMV (all loads issued up front,
 * K split over waves and workgroups, deterministic fixed-point slice sums); more rows run the
 * tiled LDS-pipelined kernel.
 * Replaces: `_gptq_matmul` M > 1 dispatch to the tiled `_GPTQ_WGSL` kernel
 * (webtorch/_core.py:3833-3888, 3995-4027) and the bias add of `QuantizedLinear.forward`
 * (webtorch/_core.py:4446-4456). */
int miq_gptq_gemm(const void* x, const int32_t* perm, const int32_t* qweight, const int32_t* qzeros,
                  const void* scales, int scales_dtype, const float* bias, void* out, int out_dtype,
                  int M, int K, int N, int gs, int bits, float zero_offset, void* workspace,
                  size_t workspace_bytes, void* stream);

/* Bytes of workspace miq_gptq_gemm_f32x needs; same contract as miq_gptq_gemv_workspace. */
int miq_gptq_gemm_f32x_workspace(int M, int K, int N, int gs, int bits, size_t* bytes);

/* miq_gptq_gemm for fp32 activations (the decoder's prefill): each row of x is scaled by a power
 * of two and split into two fp16 rows, hi = fp16(x 2^s) and lo = fp16(x 2^s - hi) (about 22
 * significant bits relative to the row's largest value, no fp16 range limit; NaN and infinite
 * rows propagate), the tiled matrix-core GEMM runs on the 2M rows, and each output is the sum of
 * its two rows scaled back by 2^-s, + bias. x fp32 16-byte aligned; K <= 32768; otherwise as
 * miq_gptq_gemm.
 * Replaces: `_gptq_matmul` M > 1 (webtorch/_core.py:3833-3888, 3995-4027) on the fp32
 * activations of the prefill `_kv_forward` (webtorch/llm.py:1619-1636). */
int miq_gptq_gemm_f32x(const float* x, const int32_t* perm, const int32_t* qweight, const int32_t* qzeros,
                       const void* scales, int scales_dtype, const float* bias, void* out, int out_dtype,
                       int M, int K, int N, int gs, int bits, float zero_offset, void* workspace,
                       size_t workspace_bytes, void* stream);

/* Asymmetric min-max quantizer to the GPTQ layout (zero_offset 0, fp32 scales), bit-exact
 * with the reference's float32 numpy arithmetic (IEEE division, round-half-even). W is
 * [K][N] or, with from_out_in = 1, [N][K]; fp16 or fp32. Outputs qweight [K/per][N],
 * qzeros [K/gs][N/per], scales [K/gs][N].
 * Replaces: `_gptq_quantize` (webtorch/_core.py:3782-3824) as used by
 * `QuantizedLinear.from_linear` (4433-4444), the tied-head requantization
 * `CausalLM._quantize_head` (webtorch/llm.py:594-602) and `_gquant` (llm.py:835-853). */
int miq_gptq_quantize(const void* W, int w_dtype, int from_out_in, int K, int N, int gs, int bits,
                      int32_t* qweight, int32_t* qzeros, float* scales, void* stream);

/* ---------------------------------------------------------------------------------------
 * GGUF Q4_K (llama.cpp block_q4_K, 144-byte super-blocks of 256 weights)
 * ------------------------------------------------------------------------------------- */

/* Dequant n_blocks super-blocks to fp32 (256 values each). blocks 16-byte aligned.
 * Replaces: `ggufload.dequant` Q4_K (webtorch/ggufload.py:116-130, 188-202). */
int miq_q4k_dequant_f32(const uint8_t* blocks, float* out, int64_t n_blocks, void* stream);

/* out[M][N] = x[M][K] @ W^T + bias, W = N rows of K/256 native super-blocks.
 * Replaces: `ggml_matmul` / `_ggml_run` for Q4_K (webtorch/_core.py:3720-3779) with the
 * decode kernel `_GGML_GEMV_*` + `_Q4K_DEC` (webtorch/_core.py:2985-3044, 3117-3133). */
int miq_q4k_gemv(const void* x, int x_dtype, const uint8_t* w, const float* bias, void* out,
                 int out_dtype, int M, int K, int N, void* stream);

/* out[M][N] = x[M][K] @ W^T + bias on the matrix cores, for prefill rows: W = N rows of K/256
 * native Q4_K super-blocks (K <= 16384), x fp16 or fp32 (fp32 as row-scaled fp16 hi/lo row
 * pairs), each 32-weight sub-block applied exactly as d1 (sum x c) - m1 (sum x). The workspace
 * (miq_q4k_gemm_workspace bytes, 256-byte aligned) holds the staged rows, their sub-block sums
 * and row scales after its first 4 MiB, which it leaves alone (the split-K counter region), so
 * the GEMV's workspace can be shared. Results are deterministic.
 * Replaces: `ggml_matmul` / `_ggml_run` with the batched kernel `_GGML_GEMM_*` + `_Q4K_DEC`
 * (webtorch/_core.py:2908-2975, 3117-3133, 3720-3779). */
int miq_q4k_gemm_workspace(int M, int K, int N, int x_dtype, size_t* bytes);
int miq_q4k_gemm(const void* x, int x_dtype, const uint8_t* w, const float* bias, void* out, int out_dtype,
                 int M, int K, int N, void* workspace, size_t ws_bytes, void* stream);

/* The same matrix-core prefill GEMM for the four types of a Q4_K_M / Q5_K_M file, by ggml type
 * id: 12 Q4_K, 13 Q5_K, 14 Q6_K, 8 Q8_0 (8 consecutive blocks per 256-value step); K a multiple
 * of 256 (<= 16384); miq_q4k_gemm is this call with type 12. Every code enters the fp16 matrix
 * cores as an exact integer: Q5_K as sc c (< 2048), Q6_K as (c - 32) sl and (c - 32) 16 sh with
 * sc = 16 sh + sl (two products into one accumulator), Q8_0 as q with d applied per block. The
 * workspace (miq_ggml_gemm_workspace bytes) is laid out as miq_q4k_gemm's. Other types:
 * MIQ_ERR_UNSUPPORTED.
 * Replaces: `ggml_matmul` / `_ggml_run` with the batched kernel `_GGML_GEMM_*` and the type's
 * decoder (`_Q4K_DEC` 3117, `_Q5K_DEC` 3137, `_Q6K_DEC` 3159, `_Q8_0_DEC` 3072)
 * (webtorch/_core.py:2904-2975, 3720-3779). */
int miq_ggml_gemm_workspace(int M, int K, int N, int x_dtype, int ggml_type, size_t* bytes);
int miq_ggml_gemm(const void* x, int x_dtype, const uint8_t* w, int ggml_type, const float* bias, void* out,
                  int out_dtype, int M, int K, int N, void* workspace, size_t ws_bytes, void* stream);

/* out[M][N] = x[M][K] @ W^T + bias for the native GGUF types, by ggml type id:
 *   32-value blocks: 2 Q4_0, 3 Q4_1, 6 Q5_0, 7 Q5_1, 8 Q8_0, 20 IQ4_NL (18, 20, 22, 24, 34, 18
 *     bytes), 39 MXFP4 (17);
 *   256-value super-blocks: 10 Q2_K, 11 Q3_K, 12 Q4_K, 13 Q5_K, 14 Q6_K, 23 IQ4_XS (84, 110, 144,
 *     176, 210, 136 bytes), 16 IQ2_XXS, 17 IQ2_XS, 22 IQ2_S, 18 IQ3_XXS, 21 IQ3_S, 19 IQ1_S,
 *     29 IQ1_M (66, 74, 82, 98, 110, 50, 56), 34 TQ1_0, 35 TQ2_0 (54, 66);
 *   40 NVFP4 (64 values, 36 bytes), 41 Q1_0 (128, 18), 42 Q2_0 (64, 18);
 *   unquantized matrices: 0 F32, 1 F16, 30 BF16 (any K).
 * W = N rows of K / (values per block) blocks as the file stores them; w and x 16-byte aligned;
 * M <= 65535 (each row a GEMV pass). Q4_K also has miq_q4k_gemv, and Q4_K, Q5_K, Q6_K and Q8_0
 * rows beyond a few run faster through miq_ggml_gemm. Other types: MIQ_ERR_UNSUPPORTED.
 * Replaces: `ggml_matmul` / `_ggml_run` for these types (webtorch/_core.py:3720-3779) with the
 * decode kernel `_GGML_GEMV_*` (webtorch/_core.py:2985-3044) and the type's decoder
 * (`_Q8_0_DEC` 3072, `_IQ4NL_DEC` 3080, `_IQ4XS_DEC` 3094, `_Q5K_DEC` 3137, `_Q6K_DEC` 3159,
 * `_Q3K_DEC` 3182, `_Q2K_DEC` 3214, the i-quant grid decoders 3256-3418, `_Q4_0_DEC` ..
 * `_Q5_1_DEC` 3419-3468, `_F16_DEC` / `_F32_DEC` / `_BF16_DEC`, `_TQ1_0_DEC`, `_TQ2_0_DEC`,
 * `_MXFP4_DEC`, `_NVFP4_DEC`, `_Q1_0_DEC`, `_Q2_0_DEC` 3470-3607; table 3609-3637). */
int miq_ggml_gemv(const void* x, int x_dtype, const uint8_t* w, int ggml_type, const float* bias,
                  void* out, int out_dtype, int M, int K, int N, void* stream);

/* Dequant n_blocks blocks of any type miq_ggml_gemv takes to fp32 (for F32 / F16 / BF16 a
 * block is one value), bit-exact (every value is one fp32 rounding of exact products). blocks
 * 2-byte aligned (16 for Q4_K, 4 for F32). Other types: MIQ_ERR_UNSUPPORTED.
 * Replaces: `ggufload.dequant` / `_dequant_iq` for the same types (webtorch/ggufload.py:133-505). */
int miq_ggml_dequant_f32(const uint8_t* blocks, int ggml_type, float* out, int64_t n_blocks, void* stream);

/* ---------------------------------------------------------------------------------------
 * Sparse MoE MLP (router + experts), all on the device
 *   route buffer: opaque int32 words laid out by (T, E, k), miq_moe_route_bytes long.
 *   expert weights are stacked: qweight [E][K/per][N], qzeros [E][K/gs][N/per], scales [E][K/gs][N].
 * ------------------------------------------------------------------------------------- */

/* Size of the route buffer for T tokens, E experts and top-k (T * k <= 4096, E <= 1024). */
int miq_moe_route_bytes(int T, int E, int k, size_t* bytes);

/* logits fp32 [T][E] -> float64 softmax, top-k (ties to the lower expert index), renormalised
 * over the k picks when norm_topk != 0; per-expert sorted token slots and row tiles.
 * Replaces: the host routing of `moe_mlp` and `_softmax_rows` (webtorch/lm_engine.py:294-307,
 * 331-333), which reads the logits back to the host. */
int miq_moe_route(const float* logits, int T, int E, int k, int norm_topk, void* route,
                  size_t route_bytes, void* stream);

/* h[T*k][I] fp32 = silu(x @ Wgate[e]) * (x @ Wup[e]) for each sorted slot's token and expert;
 * x [T][H] fp16 (x_dtype MIQ_F16) or fp32 (MIQ_F32). fp32 x enters the fp16 matrix cores as two
 * fp16 planes of each row scaled by a power of two (hi = fp16(x 2^s), lo = fp16(x 2^s - hi): about
 * 22 significant bits relative to the row's largest value, no fp16 range limit). Also records
 * each slot row's max |h| in the route buffer for miq_moe_down (route must come from
 * miq_moe_route of the same call sequence). bias_gate / bias_up: the experts' fp32 biases
 * stacked [E][I] (both or neither), added to each projection's product before the SwiGLU.
 * Replaces: the per-expert `silu(exp["gate"](xe)) * exp["up"](xe)` of `moe_mlp`
 * (webtorch/lm_engine.py:310-316). */
int miq_moe_gate_up(const void* x, int x_dtype, void* route, int T, int E, int k, const int32_t* qw_gate,
                    const int32_t* qz_gate, const void* sc_gate, const int32_t* qw_up, const int32_t* qz_up,
                    const void* sc_up, int scales_dtype, const float* bias_gate, const float* bias_up, float* h,
                    int H, int I, int gs, int bits, float zero_offset, void* stream);

/* y[T*k][H] fp32 = routing weight * (h @ Wdown[e] + bias[e]) per sorted slot (bias: fp32 [E][H]
 * or null), h as written by miq_moe_gate_up (fp32, entering the matrix cores as row-scaled fp16
 * hi and lo planes).
 * Replaces: `exp["down"](...)` and `ye * w` of `moe_mlp` (webtorch/lm_engine.py:316-318). */
int miq_moe_down(const float* h, void* route, int T, int E, int k, const int32_t* qw,
                 const int32_t* qz, const void* sc, int scales_dtype, const float* bias, float* y, int I, int H,
                 int gs, int bits, float zero_offset, void* stream);

/* out[T][H] += ys * sigmoid(gate_logits[t]) (gate_logits fp32 [T], or NULL: out += ys), the
 * shared expert's contribution.
 * Replaces: the shared-expert tail of `moe_mlp` (webtorch/lm_engine.py:322-328). */
int miq_moe_shared_add(float* out, const float* ys, const float* gate_logits, int T, int H, void* stream);

/* out[T][H] fp32 = sum of each token's k slot outputs in ascending expert order, from zero.
 * Replaces: the scatter-add `acc[rows] = acc[rows] + ye` of `moe_mlp`
 * (webtorch/lm_engine.py:308-321). */
int miq_moe_combine(const float* y, const void* route, int T, int E, int k, float* out, int H,
                    void* stream);

/* The experts of a GGUF sparse-MoE layer kept in their file encoding: out[slot][N] (fp32) = row
 * @ W_e^T over the T * k slots of a route buffer (miq_moe_route), e the slot's expert, W_e at
 * w + e * expert_stride (N rows of K / (values per block) blocks of ggml_type, any block type
 * miq_ggml_gemv takes). The row is x[token of the slot] (gather = 1: gate / up over x (T, K)) or
 * row `slot` of x (gather = 0: down over h (T * k, K)); weighted = 1 multiplies each result by
 * the slot's routing weight (the down projection, before miq_moe_combine). x, w, route 16-byte
 * aligned; expert_stride >= one expert's bytes, a multiple of 4 (any for MXFP4).
 * Replaces: the per-expert `GGMLLinear` calls of `moe_mlp` for experts `_gexperts` keeps native
 * (webtorch/lm_engine.py:294-329; webtorch/llm.py:731-760). */
int miq_moe_ggml_gemv(const void* x, int x_dtype, const void* route, int T, int E, int k, int gather,
                      int weighted, const uint8_t* w, int ggml_type, size_t expert_stride, float* out,
                      int K, int N, void* stream);

/* ---------------------------------------------------------------------------------------
 * Decode-step operators (fp32 activations). Positions and token ids live in a device
 * "decode state" of miq_decode_state_words() int32 words: [0] position of the next token,
 * [1] tokens generated, [2] zero between calls, [3] last token id; zero it before a sequence.
 * ------------------------------------------------------------------------------------- */
int miq_decode_state_words(void);

/* out[t][:] = embed[ids[t]][:] (fp16 table [V][H] -> fp32); out-of-range ids give zeros.
 * Replaces: `CausalLM._embed_ids` (webtorch/llm.py:1530-1536). */
int miq_embed(const int32_t* ids, const void* embed, float* out, int T, int H, int V, void* stream);

/* miq_embed over an fp32 table [V][H]: the token_embd of a GGUF model, dequantized once at load
 * so that every row is the exact fp32 the file's blocks decode to.
 * Replaces: `_QuantRows` row lookups (webtorch/llm.py:355-375, 1045). */
int miq_embed_f32(const int32_t* ids, const float* embed, float* out, int T, int H, int V, void* stream);

/* out[t] = (x[t] / sqrt(mean(x[t]^2) + eps)) * w, fp32.
 * Replaces: `CausalLM._rms` (webtorch/llm.py:1259-1268) and `rmsnorm` (webtorch/_core.py:2234-2263). */
int miq_rmsnorm(const float* x, const float* w, float* out, int T, int H, float eps, void* stream);

/* Per-head RMSNorm (QK-norm, Qwen3) in place on the fused q|k|v rows qkv [T][(NH + 2 NKV) HD]:
 * each query head x / sqrt(mean(x^2) + eps) * qn (fp32 [HD]), each key head the same with kn;
 * a null weight leaves that part alone; v is untouched. HD <= 256.
 * Replaces: `self._rms(q, lay["qn"])` / `self._rms(k, lay["kn"])` of `CausalLM._qkv`
 * (webtorch/llm.py:1498-1519, 1259-1268), applied before RoPE. */
int miq_head_rmsnorm(float* qkv, const float* qn, const float* kn, int T, int NH, int NKV, int HD, float eps,
                     void* stream);

/* Rotate-half RoPE at positions state[0] + t of the fused q|k|v rows qkv [T][(NH + 2 NKV) HD]
 * with the fp32 tables cos_tab / sin_tab [LMAX][HD/2] (cos/sin of pos * theta^(-2i/HD) in
 * float64, rounded once); q to q_out [T][NH][HD]; k, v written into the caches
 * [NKV][LMAX][HD] at their positions (positions >= LMAX are dropped).
 * Replaces: `_rope_np`, `_rot` and the rope step of `_kv_forward` (webtorch/llm.py:1270-1304,
 * 1626-1627), `rope_decode` (webtorch/_core.py:2302-2330) and `kv_write`
 * (webtorch/_core.py:1504-1540). */
int miq_rope_kv(const float* qkv, const int32_t* state, const float* cos_tab, const float* sin_tab,
                float* q_out, float* kcache, float* vcache, int T, int NH, int NKV, int HD, int LMAX,
                void* stream);

/* One decode token (T = 1): RoPE of q and of the new k from the fused row qkv, the new k and v
 * written into the caches at state[0], and attention over positions 0..state[0]; out [NH][HD].
 * Replaces: the per-token `_rope1` x2 + `kv_write` x2 + `gqa_attention` of `_decode_fwd`
 * (webtorch/llm.py:1591-1616; webtorch/_core.py:1319-1340, 1504-1540, 2302-2330). */
int miq_attention_decode(const float* qkv, const int32_t* state, const float* cos_tab,
                         const float* sin_tab, float* kcache, float* vcache, float* out, int NH,
                         int NKV, int HD, int LMAX, float scale, void* stream);

/* Causal GQA attention: token t (position state[0] + t) of head h attends to cache positions
 * 0..state[0] + t of kv head h / (NH / NKV); out [T][NH][HD] fp32.
 * Replaces: `KVCache.attn` + `gqa_attention` + `softmax` (webtorch/_core.py:1543-1596,
 * 1319-1340, 1764-1787). */
int miq_attention(const float* q, const float* kcache, const float* vcache, const int32_t* state,
                  float* out, int T, int NH, int NKV, int HD, int LMAX, float scale, void* stream);

/* out[t][i] = silu(gu[t][i]) * gu[t][I + i] for the fused gate|up rows.
 * Replaces: `silu(gate(x)) * up(x)` of `CausalLM._mlp` (webtorch/llm.py:1489-1496,
 * webtorch/_core.py:503-504). */
int miq_silu_mul(const float* gu, float* out, int T, int I, void* stream);

/* h[i] += y[i] (residual add). */
int miq_add(float* h, const float* y, int64_t n, void* stream);

/* Greedy pick on the device: argmax of logits[V] (first index on ties) -> ids[0],
 * history[state[1]] (if < hist_len), state[3]; state[1] += 1; state[0] += advance.
 * Replaces: `_head_argmax` / `_pick` greedy branch (webtorch/llm.py:1309-1336), which reads
 * the logits back to the host every token. */
int miq_argmax_advance(const float* logits, int V, int32_t* ids, int32_t* history, int hist_len,
                       int32_t* state, int advance, void* stream);

/* ---------------------------------------------------------------------------------------
 * Persistent decode step: the whole one-token step of an int4 GPTQ Qwen2-style decoder
 * (embedding, L x [RMSNorm, q|k|v + bias, RoPE + KV write + GQA attention, o + residual,
 * RMSNorm, gate|up, SwiGLU, down + residual], final RMSNorm, tied int4 head, greedy argmax
 * and the state advance of miq_argmax_advance) in ONE launch of one 1024-thread workgroup per
 * CU. Workgroups pass activations through tagged device-scope words in the workspace instead
 * of kernel boundaries, and every projection's weights are loaded a layer ahead.
 * Replaces: the captured one-token step `_decode_fwd` (webtorch/llm.py:1591-1616) replayed by
 * capture-replay (webtorch/llm.py:19-20), i.e. the same work as the launch sequence
 * miq_embed, L x (miq_gptq_gemv_fused, miq_attention_decode, miq_gptq_gemv,
 * miq_gptq_gemv_fused x2), miq_gptq_gemv_fused, miq_argmax_advance.
 *
 * miq_decode_persistent_plan: MIQ_OK and the grid (= CU count) and workspace bytes if the
 * shape is supported (bits 4, HD 64, H, (NH + 2 NKV) HD and 2I multiples of 64, H / 8 and
 * NH HD / 8 packed rows within 16 x min(16, gs / 8), LMAX <= 8192, the role workgroups
 * fitting the CU count), else MIQ_ERR_UNSUPPORTED (use the launch sequence above).
 *
 * layer_table: device array [L][20] of uint64 addresses per layer, in this order: q|k|v
 * qweight, qzeros, fp16 scales, fp32 bias (0 if none); o qweight, qzeros, scales; gate|up
 * qweight, qzeros, scales; down qweight, qzeros, scales; input RMSNorm weight, post-attention
 * RMSNorm weight (fp32 [H]); k cache, v cache (fp32 [NKV][LMAX][64]); 3 unused slots.
 * Layers use zero offset zoff, the head (int4, fp32 scales [H/gs][V]) head_zoff; embed is
 * fp16 [V][H]. logits [V] receives the head output. ws: 256-byte aligned, zeroed before the
 * first step and again after any error; uint32 word 0 counts finished steps and word 1 holds
 * error bits (1: a workgroup waited more than 100 ms -- not all workgroups were resident --
 * 2: state[0] >= LMAX), read by the caller after the step. The environment variable
 * MIQ_PD_SPIN_TICKS (wall-clock ticks, read at each call) shortens the 100 ms bound, so that
 * tests can drive the timeout path. After a step that timed out, every later step on the
 * workspace leaves at entry without touching the decode state (its exchange words are dirty)
 * until the workspace is zeroed; the caller then continues the sequence, e.g. with the launch
 * sequence above. Steps on one workspace must not overlap, and the step must not share the
 * GPU with other kernels. */
int miq_decode_persistent_plan(int L, int H, int NH, int NKV, int HD, int I, int V, int LMAX, int gs,
                               int bits, int* grid, size_t* ws_bytes);
int miq_decode_persistent(const uint64_t* layer_table, const void* embed, const int32_t* head_qweight,
                          const int32_t* head_qzeros, const float* head_scales, const float* final_norm,
                          const float* cos_tab, const float* sin_tab, int32_t* ids, int32_t* history,
                          int hist_len, int32_t* state, float* logits, void* ws, size_t ws_bytes, int L,
                          int H, int NH, int NKV, int HD, int I, int V, int LMAX, int gs, int bits,
                          float eps, float zoff, float head_zoff, void* stream);

/* The same step with its phase timeline: thread 0 of every workgroup stores the GPU wall clock
 * (s_memrealtime ticks) at each phase mark into trace[(wg (L + 2) + l) 8 + k] (uint64, 8-byte
 * aligned, at least grid (L + 2) 8 words, zeroed by the caller; unvisited slots stay 0): for
 * layer l < L, k = 0 role weights issued, 1 inputs received, 3 inputs staged, 5 (q|k|v tiles)
 * matrix product done, 4 tile summed (attention: q|k|v staged), 2 result published; l = L the
 * head (0 issued, 1 h(L) received, 2 arg-max published); l = L + 1 the kernel (0 entry,
 * 1 exit). Results are those of miq_decode_persistent. A diagnostic with no counterpart in the
 * reference, for the per-hop latency figures of the step (`python -m webpytorch_amd.pd_trace`). */
int miq_decode_persistent_trace(const uint64_t* layer_table, const void* embed, const int32_t* head_qweight,
                                const int32_t* head_qzeros, const float* head_scales, const float* final_norm,
                                const float* cos_tab, const float* sin_tab, int32_t* ids, int32_t* history,
                                int hist_len, int32_t* state, float* logits, void* ws, size_t ws_bytes, int L,
                                int H, int NH, int NKV, int HD, int I, int V, int LMAX, int gs, int bits,
                                float eps, float zoff, float head_zoff, uint64_t* trace, size_t trace_words,
                                void* stream);

/* ---------------------------------------------------------------------------------------
 * Capture and replay (replaces WebGPUPlatform.beginCapture / endCapture / replay,
 * `webtorch/platform.py:45-56`, which `CausalLM.capture` records one decode step with)
 * ------------------------------------------------------------------------------------- */
/* Starts recording the launches made on `stream` (not the null stream) by the calling thread:
 * nothing recorded runs until it is replayed. Every buffer the recorded launches use must stay
 * allocated while the graph exists. */
int miq_graph_begin(void* stream);
/* Stops recording on `stream` and returns the executable recording in *graph (an opaque
 * handle, hipGraphExec_t). */
int miq_graph_end(void* stream, void** graph);
/* Replays a recording on `stream` (asynchronous, stream-ordered). */
int miq_graph_launch(void* graph, void* stream);
/* Frees a recording (null: nothing). */
int miq_graph_destroy(void* graph);

#ifdef __cplusplus
}
#endif

#endif /* MIQ_H */
