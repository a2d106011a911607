/*
 * sglang_exl3_amd — C ABI of the MI355X (gfx950) EXL3 quantized-matmul path.
 *
 * Plain pointers, sizes and a HIP stream (passed as void*; NULL = the null
 * stream).  Every device pointer must point into memory of the current HIP
 * device.  Every entry point returns EXL3_OK (0) or a non-zero status, and
 * exl3_last_error() then describes the failure (thread-local string).
 * Kernels are enqueued asynchronously on `stream`; no entry point but
 * exl3_workspace_status synchronises, allocates device memory or copies to
 * the host, so all the others can be captured into a HIP graph.
 *
 * Element types: "f16" = IEEE binary16 bits (uint16_t), "f32" = float,
 * trellis words = int16 as stored by EXL3 ([k/16][n/16][16*K] row-major).
 * Codebook ids follow the reference: 0 = 3INST, 1 = MCG, 2 = mul1.
 *
 * Each declaration names the reference interface it replaces
 * (paths relative to the reference repository).
 */
#ifndef SGLANG_EXL3_AMD_H
#define SGLANG_EXL3_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EXL3_ABI_VERSION 1

#define EXL3_OK 0
#define EXL3_ERR_ARG 1         /* bad shape, size, pointer or parameter */
#define EXL3_ERR_UNSUPPORTED 2 /* valid input outside the implemented set */
#define EXL3_ERR_HIP 3         /* HIP runtime / launch failure */
#define EXL3_ERR_WORKSPACE 4   /* workspace missing or too small */

/* Bits of the workspace status word (exl3_workspace_status): a bounded wait
 * inside a launch gave up, so that launch's output is not valid. */
#define EXL3_WAIT_MOE_FUSED 1 /* one-launch MoE gate/up + down pass: a down item's wait for its h blocks */
#define EXL3_WAIT_FAT_TAIL 2  /* wide-tile GEMM tail split: the second k-half's wait for the first */

/* Element types of exl3_hadamard_fast. */
#define EXL3_DTYPE_F16 0
#define EXL3_DTYPE_BF16 1
#define EXL3_DTYPE_F32 2

#define EXL3_CB_3INST 0
#define EXL3_CB_MCG 1
#define EXL3_CB_MUL1 2

/* Version of this ABI (EXL3_ABI_VERSION).  Replaces the pybind module
 * attribute P2B_MOE_ABI_VERSION (csrc/bindings.cpp:170). */
int exl3_abi_version(void);

/* Message of the last failure on the calling thread ("" if none). */
const char* exl3_last_error(void);

/* Decode a whole EXL3 weight to fp16, bit-identical to the reference host
 * dequant (truncating codebook rounding, two fp32 FWHT passes, RNE store).
 * W: f16 [k][n].  K in 1..8, k and n multiples of 128.
 * Replaces dequant_trellis (csrc/bindings.cpp:117-132; torch op
 * sglang_exl3::dequant_trellis, src/sglang_exl3/ops.py:38-54). */
int exl3_dequant_trellis(const int16_t* trellis, const uint16_t* suh, const uint16_t* svh,
                         uint16_t* W, int k, int n, int K, int codebook, void* stream);

/* Decode `count` raw 16-bit trellis states with a codebook: out[i] = f16 bits
 * of the codebook entry, rounded toward zero (round_toward_zero != 0, the
 * host reference's rounding) or to nearest-even (0, the CUDA kernels' one).
 * Device twin of decode_codebook_bits (csrc/exl3_dequant.cuh:74-93) and
 * decode_3inst (csrc/quant/codebook.cuh:56-90). */
int exl3_decode_states(const uint16_t* states, int count, int codebook, int round_toward_zero,
                       uint16_t* out, void* stream);

/* Decode every 16x16 tile of a trellis into W (f16 [k][n]) without the
 * Hadamard rotations or sign scales: W[16kt+r][16nt+c] = value of tile
 * (kt,nt) at row r, column c.  The per-tile part of dequant_cpu
 * (csrc/bindings.cpp:37-76). */
int exl3_decode_tiles(const int16_t* trellis, uint16_t* W, int k, int n, int K, int codebook,
                      int round_toward_zero, void* stream);

/* Row-wise 128-point Hadamard transform, fp32 inside, fp16 in and out:
 *   y[r][128c + j] = fp16( (H (x[r][128c..128c+127] (.) pre[128c..]))[j] * scale * post[128c + j] )
 * with H the unnormalised Sylvester matrix (scale = 1/sqrt(128) normalises);
 * pre / post may be NULL (no scaling).  x, y: f16 [rows][cols], cols a
 * multiple of 128; y may alias x.  Replaces exllamav3's had_r_128 as called by
 * src/sglang_exl3/exl3.py:1184-1228. */
int exl3_hadamard_rows(const uint16_t* x, uint16_t* y, const uint16_t* pre, const uint16_t* post, float scale,
                       int rows, int cols, void* stream);

/* transform_hadamard_fast in the caller's element type T (EXL3_DTYPE_F16,
 * _BF16 or _F32): per 128-column block,
 *   y[r][128c + j] = T( T( sum_i x[r][128c + i] H[i][j] h ) * post[128c + j] )
 * with H the Sylvester matrix, h = 1/sqrt(128) rounded to fp32 and then to T,
 * the sum in fp32 (here in FWHT order), and post (suh converted to T) may be
 * NULL (then y is the first rounding).  x, y, post: T [rows][cols] / [cols],
 * cols a multiple of 128, y may alias x.  Replaces the fp16 (bf16, fp32)
 * torch.matmul by the cached Hadamard matrix and the suh product of
 * transform_hadamard_fast (src/sglang_exl3/hadamard_cache.py:88-120). */
int exl3_hadamard_fast(const void* x, void* y, const void* post, int rows, int cols, int dtype, void* stream);

/* Scratch bytes exl3_gemv / exl3_gemm / exl3_p2b_gemv_batched need for a
 * problem of `experts` independent GEMVs of [m,k]x[k,n].  The workspace must
 * be zero-filled before its first use; every call leaves it zero-filled again
 * (its counters self-reset).  Concurrent calls must use distinct workspaces. */
size_t exl3_gemv_workspace_size(int m, int k, int n, int K, int experts);

/* Launch shape the gfx950 selector picks for a GEMV problem:
 * out[0] = 16-row blocks, out[1] = steps (4 k-slices) per wave,
 * out[2] = k waves per workgroup, out[3] = k-splits across workgroups,
 * out[4] = LDS bytes per workgroup.  Replaces the per-architecture kernel
 * tables (csrc/exl3_gemv.cu:10-21, 40-48; csrc/quant/exl3_kernel_map.cuh:53-62). */
int exl3_gemv_plan(int m, int k, int n, int K, int experts, int* out);

/* y[m][n] (f16) = x[m][k] (f16) . W, W = the EXL3 weight (suh, trellis, svh).
 * Input rotation, decode, fp32-accumulated MFMA product and output rotation
 * run in one launch.  m in 1..64.
 * Replaces exl3_gemv (csrc/bindings.cpp:134-147 -> csrc/exl3_gemv.cu:23-63;
 * torch op sglang_exl3::exl3_gemv, src/sglang_exl3/ops.py:57-74). */
int exl3_gemv(const uint16_t* x, const int16_t* trellis, const uint16_t* suh, const uint16_t* svh,
              uint16_t* y, int m, int k, int n, int K, int codebook, void* workspace,
              size_t workspace_bytes, void* stream);

/* Bytes of the per-GPU scratch array behind exl3_gemv_noalloc. */
#define EXL3_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)

/* exl3_gemv without a workspace: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  No counterpart in the reference.  The split-k counters,
 * accumulators and partial sums live in a file-scope device array of
 * EXL3_NOALLOC_SCRATCH_BYTES per GPU (allocated with the library's code
 * object, held until the process ends); shapes whose
 * exl3_gemv_workspace_size(m, k, n, K, 1) exceeds it are refused with
 * EXL3_ERR_UNSUPPORTED.  The first call on a GPU enqueues a clear of the
 * array's zeroed regions on `stream`; every call leaves them zero again.
 * All calls on one GPU share the array, so calls that overlap in time on
 * one GPU (other streams, other threads) race; serialise them.
 * Calls no hipMalloc / hipFree and allocates nothing. */
int exl3_gemv_noalloc(const uint16_t* x, const int16_t* trellis, const uint16_t* suh, const uint16_t* svh,
                      uint16_t* y, int m, int k, int n, int K, int codebook, void* stream);

/* Same product for any number of rows m >= 1: the GEMV kernels up to 12 rows
 * (8 from n = 12288 output columns, 7 from 24576; env EXL3_GEMM_GEMV_ROWS);
 * above, the input is rotated once and the MFMA GEMM (exl3_fat_gemm's
 * kernels) runs over it with fp16 output, its k-splits handing partial tiles
 * to the last split (workspace: exl3_gemm_workspace_size).  Deterministic.
 * Replaces exl3_gemm (csrc/bindings.cpp:110-115 -> csrc/exl3_gemm.cu:9-31;
 * torch op sglang_exl3::exl3_gemm, src/sglang_exl3/ops.py:77-93). */
int exl3_gemm(const uint16_t* x, const int16_t* trellis, const uint16_t* suh, const uint16_t* svh,
              uint16_t* y, int m, int k, int n, int K, int codebook, void* workspace,
              size_t workspace_bytes, void* stream);

/* Scratch bytes exl3_gemm needs for m rows: the GEMV workspace where the
 * GEMV kernels run, above that the prefill scratch (rotated input m*k fp16
 * and its per-128 row sums, then the k-splits' fp32 partial tiles or the
 * wide kernel's tail hand-off).  It depends on the current device's CU
 * count.  The workspace must start zero-filled (counters), as for exl3_gemv;
 * every call leaves the counters zero. */
size_t exl3_gemm_workspace_size(int m, int k, int n, int K);

/* Many-row EXL3 GEMM on MFMA with the input already rotated:
 *   out[m][n] (f32) = svh[n] * (H . (a . T)[m][128-block])[n] / sqrt(128)
 * a: f16 [M][k] = fp16(H(x (.) suh) / sqrt(128)) per 128 block; trellis
 * [k/16][n/16][16K]; any K in 1..8 and codebook (the reference: K = 4 MCG
 * only).  `out` is overwritten.
 * Replaces exl3_fat_gemm (csrc/exl3_fat_gemm.cu:275-287; torch op
 * sglang_exl3::exl3_fat_gemm, src/sglang_exl3/ops.py:187-204). */
int exl3_fat_gemm(const uint16_t* a, const int16_t* trellis, float* out, const uint16_t* svh, int M, int k, int n,
                  int K, int codebook, void* stream);

/* As exl3_fat_gemm, but row m is scaled by route_weight[m] (f16) and added
 * into out[token_idx[m]] (int64), atomically (rows may share a destination).
 * Replaces exl3_fat_gemm_scatter (csrc/exl3_fat_gemm.cu:289-305; torch op
 * sglang_exl3::exl3_fat_gemm_scatter, src/sglang_exl3/ops.py:207-226). */
int exl3_fat_gemm_scatter(const uint16_t* a, const int16_t* trellis, float* out, const uint16_t* svh,
                          const int64_t* token_idx, const uint16_t* route_weight, int M, int k, int n, int K,
                          int codebook, void* stream);

/* Scratch bytes exl3_gate_up_swiglu needs for m rows (zero-filled before its
 * first use, left zeroed by every call, like the GEMV workspace). */
size_t exl3_gate_up_workspace_size(int m, int k, int n, int K);

/* Fused gate + up projection with the SwiGLU applied:
 *   out[m][n] (f16) = fp16( silu(min(g, L)) * clamp(u, -L, L) ),
 *   g = x . W_gate, u = x . W_up  (x: f16 [m][k]),
 * where both weights share the input rotation `suh` (f16 [k]), as the
 * reference's fused gate/up path rotates the input once with the gate's suh
 * for both (src/sglang_exl3/exl3.py:1184-1206: exl3_fat_gemm over the
 * concatenated packs, then clamp, sigmoid * gate * up and the fp16 copy in
 * torch).  Trellis [k/16][n/16][16K] and svh f16 [n] per projection, one K
 * and codebook.  L = swiglu_limit; 0 or inf: no clamp.  Up to 3 rows the
 * gate/up GEMV kernel (g and u rounded to fp16 before the SwiGLU, as the
 * reference's batched decode path returns them, exl3.py:1018-1034); above,
 * the input is rotated once and an MFMA kernel computes both projections of
 * a column block and applies the SwiGLU in its epilogue (g and u in fp32):
 * up to 160 rows the narrow kernel in gate/up mode (its k-splits hand fp32
 * partial tiles to the last split of each column block and row tile, or,
 * from 6 to 16 rows, to a finish launch that completes every row), above
 * it the wide-tile kernel, one workgroup holding the gate and up columns.  Replaces the gate/up half of
 * apply_exl3_batched_fat (src/sglang_exl3/exl3.py:1154-1206). */
int exl3_gate_up_swiglu(const uint16_t* x, const uint16_t* suh, const int16_t* gate_trellis,
                        const uint16_t* gate_svh, const int16_t* up_trellis, const uint16_t* up_svh,
                        uint16_t* out, int m, int k, int n, int K, int codebook, float swiglu_limit,
                        void* workspace, size_t workspace_bytes, void* stream);

/* For each active slot e < num_active: out[e] (f16 [m][n]) = x_e . W_{ids[e]}
 * where x_e = x (x_per_expert == 0, x is [m][k]) or x + e*m*k (x_per_expert
 * != 0, x is [num_active][m][k]); weight pointers come from int64 device
 * tables indexed by ids (int32).  One launch for all slots.
 * Replaces p2b_gemv_batched (csrc/bindings.cpp:149-156 ->
 * csrc/p2b_batched.cu:78-101; torch op sglang_exl3::p2b_gemv_batched,
 * src/sglang_exl3/ops.py:96-118). */
int exl3_p2b_gemv_batched(const uint16_t* x, int x_per_expert, const int64_t* trellis_ptrs,
                          const int64_t* suh_ptrs, const int64_t* svh_ptrs, const int32_t* ids,
                          int num_active, uint16_t* out, int m, int k, int n, int K, int codebook,
                          void* workspace, size_t workspace_bytes, void* stream);

/* Scratch bytes exl3_moe_layer / exl3_p2b_fused_moe need for `tokens` tokens
 * routed to `topk` of `num_experts` experts (hidden -> inter -> hidden).
 * Zero-filled before first use; every call leaves its counters zero. */
size_t exl3_moe_workspace_size(int tokens, int topk, int num_experts, int hidden, int inter);

/* Launch shapes the planner picks for a MoE layer: out[0..3] = gate/up
 * (column blocks per work item, steps per wave, k waves, k-splits),
 * out[4..7] = the same for down, out[8] = bound on 16-row work units.  Replaces the occupancy-sized
 * cooperative grid of csrc/p2b_moe.cu:364-378. */
int exl3_moe_plan(int tokens, int topk, int num_experts, int hidden, int inter, int* out);

/* Routed-expert MoE layer for a batch of tokens, one call, no host sync:
 *   out[t] = sum_s w[t][s] * down_e( fp16( silu(min(g, L)) * clamp(u, -L, L) ) ),
 *   e = topk_ids[t][s], g = fp16(gate_e(x[t])), u = fp16(up_e(x[t])),
 * fp16 out [tokens][hidden].  The sum over slots of w * fp16(down) is taken
 * in fp32 in slot order above 48 tokens and in 64-bit fixed point (2^-30
 * resolution) up to 48 tokens; both are deterministic.  Ids outside [0, num_experts) are
 * skipped (weight ignored), like map_topk_to_local's invalid slot.  The nine
 * pointer tables are int64 device arrays of num_experts device addresses.
 * swiglu_limit <= 0 or infinite: no clamp.  K per projection 1..8, one
 * codebook; hidden, inter multiples of 128; num_experts <= 4096, topk <=
 * 16384, any number of tokens (batches above 8192 (token, slot) entries take
 * the prefill path, which runs them in chunks of 16384 entries).
 * Replaces the routed-expert paths of EXL3MoEMethod.apply
 * (src/sglang_exl3/exl3.py:2253-2314 -> apply_exl3_experts :1347-1431 ->
 * apply_exl3_python_loop :520-576 / apply_exl3_batched_moe_gemv :960-1110). */
int exl3_moe_layer(const uint16_t* x, const int32_t* topk_ids, const float* topk_weights,
                   const int64_t* gate_trellis, const int64_t* gate_suh, const int64_t* gate_svh,
                   const int64_t* up_trellis, const int64_t* up_suh, const int64_t* up_svh,
                   const int64_t* down_trellis, const int64_t* down_suh, const int64_t* down_svh,
                   int num_experts, uint16_t* out, int tokens, int topk, int hidden, int inter,
                   int K_gate, int K_up, int K_down, int codebook, float swiglu_limit,
                   void* workspace, size_t workspace_bytes, void* stream);

/* One-token fused MoE: out[0] = fp16( sum_e rw[e] * down_{ids[e]}(...) ) as
 * exl3_moe_layer with tokens = 1, topk = num_ids and fp16 routing weights;
 * `out` [1][hidden] is overwritten.  Any hidden/inter multiple of 128 and any
 * K per projection (the reference: hidden 4096, inter 1024/2048, equal K 2..4).
 * Replaces p2b_fused_moe (csrc/bindings.cpp:158-167 -> csrc/p2b_moe.cu:417-468;
 * torch op sglang_exl3::p2b_fused_moe, src/sglang_exl3/ops.py:121-184). */
int exl3_p2b_fused_moe(const uint16_t* x, uint16_t* out, const int64_t* gate_trellis, const int64_t* gate_suh,
                       const int64_t* gate_svh, const int64_t* up_trellis, const int64_t* up_suh,
                       const int64_t* up_svh, const int64_t* down_trellis, const int64_t* down_suh,
                       const int64_t* down_svh, int num_experts, const int32_t* expert_ids,
                       const uint16_t* routing_weights, int num_ids, int hidden, int inter, int K_gate,
                       int K_up, int K_down, int codebook, float swiglu_limit, void* workspace,
                       size_t workspace_bytes, void* stream);

/* Status word of a workspace: *status_out = the EXL3_WAIT_* bits set by
 * launches on it since the last call (0: none), and the word is cleared.  A
 * set bit means some launch's bounded wait gave up and its output is not
 * valid; the workspace's counters may then be left non-zero, so zero the
 * whole workspace before its next use.  Enqueues a 4-byte copy on `stream`
 * and synchronises it, so it cannot be called during graph capture
 * (EXL3_ERR_ARG).  workspace_bytes must cover the counter region (256 KiB).
 * No counterpart in the reference, whose cooperative kernels wait without a
 * bound (csrc/p2b_moe.cu:166-362, grid.sync) and exit the process on a
 * launch error (csrc/util.cuh:92-100); for callers that need to know that a
 * bounded wait gave up. */
int exl3_workspace_status(void* workspace, size_t workspace_bytes, int32_t* status_out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SGLANG_EXL3_AMD_H */
