/*
 * Operator-level entry points of the FAST path (exported by libqwen_mi355x.so).
 *
 * The reference has no counterpart: its projections are the serial loops of project_tiled
 * (hls/decode_only/qwen_decode_attention_kernel.cpp:62-98, qwen_decode_mlp_kernel.cpp:44-77).
 * These entry points expose, one operator at a time, the integer arithmetic that the FAST model
 * path (QWEN_MODE_FAST of qwen_hip_model.h) runs inside its layers, so that callers and tests can
 * check it on its own:
 *
 *   two-limb activation code of a row x[0, n):
 *     amax = max |x|,  inv = 32512 / amax (fp32; 0 when amax = 0),
 *     X = clip(rint(x * inv), -32512, 32512),  H = floor((X + 128) / 256),  L = X - 256 H,
 *     sx = amax / 32512 (1 when amax = 0),  sums = (sum H, sum L);
 *   projection of token t, output row o (u = q + 8 in [0, 15] for the INT4 weight q):
 *     y = bias[o] + sw[o] * sx[t] * (256 (sum_k u H - 8 sum H) + (sum_k u L - 8 sum L)),
 *     with every integer sum exact (int32 matrix-core accumulators, exact fp32 K-split partials
 *     whenever they are integers below 2^24).
 *
 * All buffers are DEVICE pointers; work is queued on `stream` (a hipStream_t, 0 for the null
 * stream).  Return value: 0, 1 for an invalid argument, 90 for a HIP runtime failure
 * (qwen_hip_last_error() holds the message).
 */
#ifndef QWEN_HIP_OPS_H
#define QWEN_HIP_OPS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Two-limb code of `rows` rows of width n (n a multiple of 128, n <= 8960), as the FAST layers
 * quantize every projection input: xq [rows][n/128][2][128] int8 (K chunk c of a row holds the 128
 * H limbs of inputs 128c.., then their 128 L limbs), sx [rows] fp32, sums [rows][2] int32. */
int qwen_hip_fast_quantize_rows(const float* x, int rows, int n, int8_t* xq, float* sx, int32_t* sums, void* stream);

/* Skip the cross-block K-split workspace: the projection then runs without split partials (for
 * 16 tokens or fewer: the direct-load kernel with an in-block K split). */
#define QWEN_PROJECT_NO_SPLITK 0x1

/* y[t][o] (fp32 [tokens][out_dim]) = the FAST projection of the fp32 rows x [tokens][in_dim] by the
 * INT4 matrix w in the reference layout ([out_dim][in_dim] nibbles, the even flat index in the low
 * nibble; llm_memory_layout.h weight segments) with per-row scales sw [out_dim] and an optional bias
 * [out_dim] (null for none).  out_dim a multiple of 16, in_dim a multiple of 128 and <= 8960.  The
 * kernel is chosen by shape exactly as inside the model (<= 64 tokens: the skinny decode GEMMs; up to
 * 256: the pipelined GEMM with a cross-block K split; more: the pipelined GEMM with two blocks per CU).
 * Allocates its own workspace (repacked weights, activation code, split partials) and synchronizes
 * `stream` before returning. */
int qwen_hip_fast_project(const uint8_t* w, const float* sw, const float* bias, int out_dim, int in_dim,
                          const float* x, int tokens, int flags, float* y, void* stream);

/* Grouped code of the decode of 2..64 sequences (no counterpart in the reference; for tests and callers
 * that check that step on its own).  There the gate/up projection quantizes its SiLU·up rows not per
 * row but per group of 64 rows g (the rows of row tiles 8(g/2) + 2j + g%2, j < 4: the K of one 16x16x64
 * matrix-core product of the down projection), with that group's maximum: for each token t and group
 * g of the 8960 rows, the two-limb code of the 64 values, scale gsx[t][g] = max / 32512 (1 for an
 * all-zero group) and offset term gcorr[t][g] = 256 sum H + sum L, the limbs at the rows' places of
 * xq [tokens][70][2][128].  qwen_hip_fast_silu_mul_grouped runs that projection (INT4 gate and up
 * [8960][1536] in the reference layout with their row scales, on the two-limb code of x [tokens][1536],
 * 1 <= tokens <= 64) twice on the same code: into y [tokens][8960] (fp32 SiLU(gate)·up) and into the
 * grouped code (xq, gsx [tokens][140], gcorr [tokens][140]). */
int qwen_hip_fast_silu_mul_grouped(const uint8_t* gate, const float* sw_gate, const uint8_t* up, const float* sw_up,
                                   const float* x, int tokens, float* y, int8_t* xq, float* gsx, int32_t* gcorr,
                                   void* stream);

/* The down projection of a grouped code (as qwen_hip_fast_silu_mul_grouped writes it; tokens 1..64):
 * y[t][o] = sw[o] * sum_g gsx[t][g] * (sum over the group's K of u X - 8 gcorr[t][g]) for the INT4 matrix w
 * [out_dim][8960] (u = q + 8), out_dim a multiple of 64; each group's integer sum is exact, the sum over
 * groups is fp32.  Allocates its own workspace and synchronizes `stream` before returning. */
int qwen_hip_fast_project_grouped(const uint8_t* w, const float* sw, int out_dim, const int8_t* xq, const float* gsx,
                                  const int32_t* gcorr, int tokens, float* y, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QWEN_HIP_OPS_H */
