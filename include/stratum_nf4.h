/*
 * stratum_nf4.h -- C ABI of the MI355X (gfx950) NF4 frozen-weight library.
 *
 * One shared library, libstratum_nf4.so, built from the .hip sources in stratum_amd/csrc.
 * Every entry point:
 *   - takes plain device pointers, element counts and a HIP stream handle
 *     (hipStream_t passed as void*, NULL = the null stream);
 *   - is asynchronous on that stream, allocates nothing and keeps no state
 *     between calls (the caller keeps buffers alive until the stream is done);
 *   - never throws; returns STM_OK (0) or a negative STM_ERR_* code, with a
 *     human-readable reason available from stm_last_error() on the same thread.
 *
 * Layout (identical to bitsandbytes' NF4 layout that the reference stores in
 * NF4Payload, stratum/upload.py:70-95):
 *   packed : uint8 [(n + 1) / 2]       two 4-bit codes per byte, element 2i in the
 *                                       high nibble, element 2i+1 in the low nibble
 *   absmax : float [ceil(n / blocksize)] per-block max|x| (fp32), blocks of
 *                                       `blocksize` consecutive row-major elements
 *   code   : the 16 NF4 levels (fixed; the kernels carry them, no code pointer)
 * A weight W[N, K] is flattened row-major, so with K % blocksize == 0 the
 * absmax of element (n, k) is absmax[n * (K / blocksize) + k / blocksize].
 */
#ifndef STRATUM_NF4_H
#define STRATUM_NF4_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define STM_NF4_ABI_VERSION 5

/* return codes */
#define STM_OK 0
#define STM_ERR_INVALID (-1)     /* bad argument (null pointer, size, blocksize, dtype, alignment) */
#define STM_ERR_UNSUPPORTED (-2) /* valid but not handled by this kernel (shape constraint) */
#define STM_ERR_HIP (-3)         /* a HIP runtime call failed (launch error) */

/* element types */
#define STM_F16 0
#define STM_BF16 1
#define STM_F32 2

/* nearest-level rules of the two bitsandbytes NF4 quantizers */
#define STM_NF4_ARGMIN 0    /* torch/CPU backend: clamp, first argmin of fp32 |s - code| */
#define STM_NF4_THRESHOLD 1 /* CUDA kernel: fp32 midpoint comparison tree with strict '>' */

/* Library version (STM_NF4_ABI_VERSION). Host-only, never touches a GPU. */
int stm_nf4_abi_version(void);

/* Reason for the last non-zero return on the calling thread ("" if none). */
const char* stm_last_error(void);

/*
 * Blockwise NF4 quantize + nibble pack.
 * Replaces bitsandbytes.functional.quantize_4bit(A, blocksize=64,
 * compress_statistics=False, quant_type="nf4") as called at
 * stratum/upload.py:367-369 (prepare_nf4) and stratum/upload.py:725-727
 * (stream_load_and_quantize_module).
 *   A        : device, n elements of `dtype` (STM_F16 / STM_BF16 / STM_F32), row-major
 *   blocksize: power of two in [64, 4096]
 *   rounding : STM_NF4_ARGMIN or STM_NF4_THRESHOLD
 *   packed   : device, (n + 1) / 2 bytes        absmax: device, ceil(n / blocksize) floats
 */
int stm_nf4_quantize(const void* A, int dtype, int64_t n, int blocksize, int rounding, uint8_t* packed,
                     float* absmax, void* stream);

/*
 * Blockwise NF4 dequantize: out[i] = dtype(fp32(code[q_i]) * absmax[i / blocksize]),
 * one fp32 product then one round-to-nearest-even conversion.
 * Replaces bitsandbytes.functional.dequantize_4bit(q, QuantState(...)) as called at
 * stratum/upload.py:1038 (ensure_weights), :221 (NF4Prefetch.finalize), :946
 * (upload_stream) and stratum/nf4_linear.py:46 (NF4Linear.forward).
 *   out: device, n elements of out_dtype (STM_F16 / STM_BF16 / STM_F32)
 */
int stm_nf4_dequantize(const uint8_t* packed, const float* absmax, int64_t n, int blocksize, void* out,
                       int out_dtype, void* stream);

/*
 * Many tensors per call: stm_nf4_quantize / stm_nf4_dequantize applied to
 * tensors t = 0 .. count-1 (host arrays of device pointers and sizes; one
 * dtype, blocksize and rule for all), with the whole blocks of up to 32
 * tensors in one launch. Same results, bit for bit, as one call per tensor.
 * Batches the per-parameter loops of stratum/upload.py prepare_nf4
 * (:305-398, quantize) and ensure_weights / NF4Prefetch.finalize (:969-1069,
 * :187-225, dequantize), which call bitsandbytes once per parameter; a
 * layer's projections then cost one launch instead of one each.
 */
int stm_nf4_quantize_many(int count, const void* const* A, const int64_t* n, int dtype, int blocksize, int rounding,
                          uint8_t* const* packed, float* const* absmax, void* stream);
int stm_nf4_dequantize_many(int count, const uint8_t* const* packed, const float* const* absmax, const int64_t* n,
                            int blocksize, void* const* out, int out_dtype, void* stream);

/*
 * Fused NF4 dequant-GEMM, forward of a frozen Linear:
 *   Y[M, N] = X[M, K] . W[N, K]^T  (+ bias[N])  (+ T[M, R] . L[N, R]^T)
 * with W given as NF4 (packed [N*K/2], absmax [N*K/blocksize]) and dequantized
 * tile by tile in LDS with exactly the dequantize rounding above, fp32
 * accumulation on bf16/fp16 MFMA.
 * Replaces F.linear(x, dequantize_4bit(W), bias) at stratum/nf4_linear.py:46-47
 * (and the F.linear that HF/PEFT modules run on the dequantized param.data,
 * stratum/stage.py:135). The optional rank-R term is the LoRA update
 * (T = scale * X . A^T, L = B) that PEFT adds on top of the frozen base.
 *   dtype        : STM_BF16 or STM_F16, for X, Y, bias, T, L and the dequantized W
 *   X, Y         : row-major, leading dimensions K and N
 *   bias         : NULL or [N];  T, L: NULL (lora_rank = 0) or [M, R], [N, R], R % 16 == 0
 *   workspace    : NULL, or device memory of at least
 *                  stm_nf4_gemm_workspace_bytes(M, N, K, 0) bytes (16-byte aligned).
 *                  When the problem has too few output tiles to fill the GPU
 *                  (small M) the reduction is split over several work-groups
 *                  whose fp32 partials go there and are summed (in a fixed
 *                  order) by a second kernel; NULL disables the split. For
 *                  M <= 64 a weight-streaming kernel runs instead of the tiles:
 *                  in one launch with no workspace where its split-free form
 *                  fits (M <= 16 and enough weight rows to fill the GPU), else
 *                  when it has this workspace (or needs none: one range and no
 *                  LoRA term), its split reduce adding bias and the LoRA term.
 *   constraints  : K % 64 == 0, K % blocksize == 0, all pointers 16-byte aligned
 */
int stm_nf4_gemm_fwd(const void* X, const uint8_t* packed, const float* absmax, const void* bias, const void* T,
                     const void* L, int lora_rank, void* Y, int64_t M, int64_t N, int64_t K, int blocksize,
                     int dtype, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * stm_nf4_gemm_fwd without a workspace argument and without any allocation.
 * No counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). The split-reduction partials that stm_nf4_gemm_fwd keeps in
 * the caller's workspace go to a static 16 MiB device array of the library
 * (one per GPU, held until the process ends; its address is looked up once per
 * device on the first call there, on the current device). Problems whose
 * partials need more than 16 MiB (stm_nf4_gemm_workspace_bytes(M, N, K, 0) >
 * 16 MiB) return STM_ERR_UNSUPPORTED. Every call on one GPU shares that array:
 * calls that overlap on one GPU (concurrent streams or threads) race. The
 * partials are fully overwritten by each call (nothing needs clearing).
 * Arguments, constraints and results otherwise as stm_nf4_gemm_fwd.
 */
int stm_nf4_gemm_fwd_noalloc(const void* X, const uint8_t* packed, const float* absmax, const void* bias,
                             const void* T, const void* L, int lora_rank, void* Y, int64_t M, int64_t N, int64_t K,
                             int blocksize, int dtype, void* stream);

/*
 * Fused NF4 dequant-GEMM, input gradient of a frozen Linear (no dW: the base
 * weight has requires_grad=False, stratum/upload.py:328-329):
 *   dX[M, K] = dY[M, N] . W[N, K]  (+ U[M, R] . At[K, R]^T)
 * Replaces the autograd backward of F.linear on the dequantized weight, run by
 * torch.autograd.backward at stratum/runtime.py:340-341. The optional rank-R term
 * is the LoRA input gradient (U = scale * dY . B, At = A^T).
 *   workspace    : as stm_nf4_gemm_fwd, sized by stm_nf4_gemm_workspace_bytes(M, N, K, 1).
 *                  At most 64 rows run a weight-streaming kernel when this
 *                  workspace is given (its ranges of weight rows write fp32
 *                  partials that a second kernel sums with the LoRA term);
 *                  without it the tile kernels run (2-3x slower there).
 *   constraints  : N % 64 == 0, K % 64 == 0, K % blocksize == 0, 16-byte aligned
 */
int stm_nf4_gemm_bwd_dx(const void* dY, const uint8_t* packed, const float* absmax, const void* U, const void* At,
                        int lora_rank, void* dX, int64_t M, int64_t N, int64_t K, int blocksize, int dtype,
                        void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Bytes of fp32 workspace the forward (backward = 0) or input-gradient
 * (backward = 1) GEMM of this size uses to split its reduction: 0 when it does
 * not split. Host-only, never touches a GPU; negative on invalid sizes.
 * No counterpart in the reference (bitsandbytes and cuBLAS size their own
 * scratch); it lets the caller hand in memory from its allocator.
 */
int64_t stm_nf4_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int backward);

/*
 * Tile-shape restriction of the GEMM planner, process-wide: kind 0 = the
 * 256 x 256 tiles, 1 = 128 x 128, 2 = 128 x 256, anything else (e.g. -1) = the
 * cost model (the default). Starts from the environment variable
 * STRATUM_NF4_GEMM_TILE ("big", "small", "mid"), read once when the library
 * loads. A restriction also skips the small-M weight-streaming kernel. Returns
 * the previous setting. Host-only. No counterpart in the reference: it lets
 * tests reach every kernel on the same problem.
 */
int stm_nf4_gemm_set_tile(int kind);

/*
 * Grouped fused NF4 dequant-GEMM over a stacked expert payload, forward:
 *   for each expert e: Y[off[e]:off[e+1], :] = X[off[e]:off[e+1], :] . W_e^T
 * where W is one NF4 payload of the stacked tensor [E, N, K] (the layout
 * prepare_nf4 produces for 3-D MoE weights, stratum/upload.py:365-366) and X/Y
 * rows are grouped by expert. Replaces the per-expert F.linear loop of
 * transformers' Qwen3MoeExperts.forward on the dequantized stacked weight.
 *   offsets: device int32 [E + 1], offsets[0] = 0, non-decreasing, offsets[E] = M_total
 *   host_offsets: NULL, or a host copy of offsets; read before the launch:
 *             validated (offsets[0] = 0, non-decreasing, no expert above
 *             max_rows: else STM_ERR_INVALID, nothing launched) and used to
 *             pick the tile height (stm_nf4_grouped_tile_rows). The kernels
 *             index rows by the device array alone, which is NOT read on the
 *             host: without host_offsets the caller guarantees its contract.
 *   max_rows: an upper bound on offsets[e+1] - offsets[e] (sizes the launch grid);
 *             at most 64 (decode-sized MoE batches): the weight-streaming
 *             kernel runs per (block of weight rows, expert) instead of the
 *             tiles, no workspace
 *   constraints: as stm_nf4_gemm_fwd
 */
int stm_nf4_grouped_gemm_fwd(const void* X, const uint8_t* packed, const float* absmax, const int32_t* offsets,
                             const int32_t* host_offsets, int num_experts, int64_t max_rows, void* Y, int64_t N,
                             int64_t K, int blocksize, int dtype, void* stream);

/*
 * Tile height (192 or 256 rows) the grouped forward uses for these row counts
 * (host int32 [E + 1] offsets): the cheaper by a per-item cost model (a full
 * 256-row item 1, an expert's last 256-row item 0.45 / 0.6 when it holds at
 * most 64 / 128 rows, a 192-row item 0.81). Pure host function; no
 * counterpart in the reference (its per-expert loop has no tiles).
 * Returns 192, 256, or STM_ERR_INVALID (NULL, num_experts <= 0, offsets[0] != 0
 * or decreasing offsets).
 */
int stm_nf4_grouped_tile_rows(const int32_t* host_offsets, int num_experts);

/*
 * Grouped input gradient: for each expert e: dX[rows of e] = dY[rows of e] . W_e.
 * Replaces the autograd backward of the same per-expert F.linear loop.
 *   host_offsets: NULL, or a host copy of offsets, validated as in the forward
 *                 (version 5 added it).
 */
int stm_nf4_grouped_gemm_bwd_dx(const void* dY, const uint8_t* packed, const float* absmax, const int32_t* offsets,
                                const int32_t* host_offsets, int num_experts, int64_t max_rows, void* dX, int64_t N,
                                int64_t K, int blocksize, int dtype, void* stream);

/*
 * SwiGLU gating of a frozen MLP, between the stacked [gate; up] projection and
 * the down projection. Replaces `act_fn(gate_proj(x)) * up_proj(x)` and its
 * autograd backward inside MemoryFlatFrozenMLPFunction
 * (stratum/model/mlp_opt.py:178-180 forward, :203-212 backward recompute),
 * act_fn = SiLU.
 *   gate_up:  [rows, 2 * inter], row = [gate_0 .. gate_{inter-1}, up_0 .. up_{inter-1}]
 *   out:      [rows, inter] = silu(gate) * up
 *   grad_out: [rows, inter] (gradient of out)
 *   grad_gate_up: [rows, 2 * inter] = [d gate | d up], the layout of gate_up
 * fp32 arithmetic, one round-to-nearest-even conversion per output; dtype
 * STM_BF16 or STM_F16. Asynchronous on `stream`.
 */
int stm_swiglu_fwd(const void* gate_up, void* out, int64_t rows, int64_t inter, int dtype, void* stream);
int stm_swiglu_bwd(const void* grad_out, const void* gate_up, void* grad_gate_up, int64_t rows, int64_t inter,
                   int dtype, void* stream);

/*
 * Rank-R side products of a LoRA adapter on the frozen NF4 base. They replace the
 * autograd matmuls of PEFT's lora.Linear (the adapter the reference attaches
 * in scripts/train.py:568-573; forward lora_B(lora_A(x)) * scaling):
 *   stm_lora_down: T[M, R]  = scaling * X[M, K] . A[R, K]^T          (forward, lora_A)
 *   stm_lora_dy:   U[M, R]  = scaling * dY[M, N] . B[N, R]           (backward, into lora_B)
 *                  dB[N, R] = dY^T . T  (skipped when dB is NULL)     (gradient of lora_B)
 *   stm_lora_da:   dA[R, K] = U^T . X                                (gradient of lora_A)
 * T and U are the rank-R tensors the fused GEMMs take as lora_x. stm_lora_dy
 * reads dY once for both U and dB. fp32 accumulation; the fp32 partial sums of
 * the column/row blocks go to the caller's workspace and are added in a fixed
 * order (deterministic), scaled and rounded once; stm_lora_down at M <= 64
 * (decode sizes) is one launch that sums each row's products in a fixed order
 * itself and leaves the workspace unused. R in {8, 16, 24, 32}; the
 * column count of the large operand (K or N) a multiple of 8; all operands
 * 16-byte aligned, row-major and contiguous; dtype STM_BF16 or STM_F16.
 * Workspace: stm_lora_workspace_bytes(rows, cols, R, op) bytes, 16-byte aligned,
 * op 0 = down (rows M, cols K), 1 = dy (M, N) with dB, 2 = da (M, K); for
 * stm_lora_dy without dB, op 1 also suffices. Asynchronous on `stream`.
 */
int64_t stm_lora_workspace_bytes(int64_t rows, int64_t cols, int rank, int op);
int stm_lora_down(const void* X, const void* A, void* T, int64_t M, int64_t K, int rank, float scaling, int dtype,
                  void* workspace, int64_t workspace_bytes, void* stream);
int stm_lora_dy(const void* dY, const void* B, const void* T, void* U, void* dB, int64_t M, int64_t N, int rank,
                float scaling, int dtype, void* workspace, int64_t workspace_bytes, void* stream);
int stm_lora_da(const void* U, const void* X, void* dA, int64_t M, int64_t K, int rank, int dtype, void* workspace,
                int64_t workspace_bytes, void* stream);

/*
 * Host-only introspection used by the CPU test suite (no GPU work):
 * the 15 fp32 decision boundaries of a rounding rule (code > i iff s >= b[i]),
 * and the 65-cell table the quantize kernel indexes with
 * j = (int)(clamp(s, -1, 1) * 32 + 32); code = base[j] + (s >= bound[j]).
 */
int stm_nf4_decision_boundaries(int rounding, float* out15);
int stm_nf4_cell_table(int rounding, float* bound65, uint8_t* base65);

#ifdef __cplusplus
}
#endif

#endif /* STRATUM_NF4_H */
