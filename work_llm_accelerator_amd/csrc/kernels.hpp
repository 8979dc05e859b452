// Host-side launchers of the HIP kernels (one declaration per kernel family).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace qwen {

// ---- ORDERED (bit-exact) kernels: kernels_ordered.hip ----
void launch_rmsnorm_ordered(const float* x, const float* w, float* y, int tokens, bool prefill, hipStream_t st);
void launch_project_ordered(const float* x, int tokens, int in_dim, const uint8_t* W, const float* scale,
                            const float* bias, int out_dim, float* y, const float* residual, hipStream_t st);
void launch_silu_mul(const float* g, const float* u, float* s, size_t n, bool prefill, hipStream_t st);
void launch_rope_append_decode(float* q, const float* k, const float* v, const int* pos, const float* rope,
                               bool rope_rows_are_tokens, float* k_cache, float* v_cache, size_t cache_stride,
                               int max_keys, int tokens, hipStream_t st);
void launch_rope_prefill(float* q, float* k_rows, const float* rope, int tokens, hipStream_t st);
void launch_rope_table_prefill(float* rope, int first, int count, hipStream_t st);
// prefill: token b is the query at position past + b over keys 0..past+b of one sequence's rows.
void launch_attention_ordered(const float* q, const float* k_cache, const float* v_cache, size_t cache_stride,
                              const int* pos, int max_keys, int tokens, bool prefill, int past, float* ctx,
                              hipStream_t st);

// ---- FAST kernels: kernels_fast.hip ----
constexpr int kKChunk = 128;        // K values per repacked weight chunk
constexpr int kQuantMax = 32512;    // |X| bound of the two-limb activation code (127 * 256)
constexpr int kMaxQuantRow = 8960;  // widest activation row that is quantized
constexpr int kAttnMaxSplits = 64;  // most KV splits of one decode-attention sequence
constexpr int kNormNone = 0, kNormDecode = 1, kNormPrefill = 2;
constexpr int kEpiStore = 0, kEpiSiluMul = 1, kEpiResidual = 2;
// Epilogues fused into the split-K reduce kernel (GEMMs of at most kSplitTokens tokens):
//   kFuseQkvRope:   [q|k|v] rows + bias, decode RoPE of q and k, K/V cache append (kEpiStore);
//   kFuseNormQuant: the finished row (kEpiStore, or kEpiResidual after bf16 rounding) is RMS-normalized
//                   with norm_w and quantized into xq_out / sx_out / sums_out for the next projection.
// Fused into the epilogue of the pipelined GEMM (more than kSplitTokens tokens):
//   kFuseRopePrefill: [q|k|v] rows + bias, prefill RoPE of q (in place in y) and k, K/V cache append;
//                     token t is sequence t / seq_len at position past + t % seq_len.
constexpr int kFuseNone = 0, kFuseQkvRope = 1, kFuseNormQuant = 2, kFuseRopePrefill = 3;

// Bytes of the two-limb code of `rows` activation rows of width n.
inline size_t xq_bytes(size_t rows, size_t n) { return rows * n * 2u; }

// The split-KV decode-attention partials of one sequence (attn_decode_kernel without its merge):
// part[head][split][128] and pml[head][split] = (m, l), merged by the blocks of the O projection.
struct AttnMergeArgs {
  const float* part;
  const float2* pml;
  const int* pos;  // position of the sequence's new token
  int nsplit, chunk, max_keys;
  float* sx_out;  // scale and limb sums of the quantized context row (block 0 writes them)
  int* sums_out;
  // With the attention fused into the Q/K/V projection (AttnFuseArgs), the partials cover the history
  // keys only (keys 0..pos-1 when 0 <= pos < max_keys) and the merge adds the new key's own term from
  // qkv_new, the token's rotated [q | k | v] row (q unscaled; k at + 1536, v at + 1792).
  const float* qkv_new = nullptr;
};

// The decode attention of one sequence fused into its Q/K/V projection: block (query head h, split c)
// computes the head's q row and the attention over history keys [c*chunk, min(end, (c+1)*chunk)),
// end = pos when 0 <= pos < max_keys (the new key is the O projection's merge's own term), else
// min(max(pos, 0) + 1, max_keys), written as partials part[h][c][128], pml[h][c] = (m, l).
struct AttnFuseArgs {
  float* part = nullptr;
  float2* pml = nullptr;
  int nsplit = 0, chunk = 0, max_keys = 0;
};
constexpr int kFusedAttnChunk = 64;      // keys per block of the fused attention (its K/V rows sit in LDS)
constexpr int kFusedAttnMaxSplits = 20;  // at most 248 blocks: one launch wave at one block per CU

struct GemmArgs {
  const uint8_t* wp;    // repacked weights (tile layout)
  const uint8_t* wp2;   // second matrix (gate/up pair) or null
  const float* sw;      // per-row scales
  const float* sw2;
  const float* bias;    // kEpiStore: optional bias
  const int8_t* xq;     // activation limbs [tokens][in/128][2][128]
  const float* sx;      // per-token scale
  const int* sums;      // per-token (sum H, sum L)
  int tokens, in_dim, out_dim;
  float* y;             // output [tokens][y_stride]
  size_t y_stride;
  const float* resid;   // kEpiResidual: residual [tokens][resid_stride]
  size_t resid_stride;
  float* y_raw;         // kEpiResidual: optional copy of the output before bf16 rounding
  int round_bf16;       // kEpiResidual: round the output to bf16 (driver rounding)
  int prefill_silu;     // kEpiSiluMul: 1 = approx_exp SiLU (prefill), 0 = expf SiLU (decode)
  float* part;          // optional fp32 workspace for K splits across blocks: [splits][tokens][out]
  int fuse;             // kFuse*: epilogue of the reduce kernel (needs part; tokens <= kSplitTokens)
  // kFuseQkvRope (token t is sequence t at position pos[t]; positions outside [0, limit) are skipped)
  const int* pos;
  const float* rope;    // [position][cos 64 | sin 64]
  float* k_cache;
  float* v_cache;
  size_t seq_stride;
  int limit;
  // kFuseNormQuant
  const float* norm_w;
  int norm;             // kNormDecode or kNormPrefill
  int8_t* xq_out;
  float* sx_out;
  int* sums_out;
  int defer_reduce;     // kFuseNormQuant, one token: write the partials only; the next projection's
                        // blocks finish the row (launch_gemm_i8_pre)
  int seq_len, past;    // kFuseRopePrefill (with rope, k_cache, v_cache, seq_stride, limit)
  // Grouped two-limb code of the down projection's input (decode batches of 2..64 tokens): every
  // 64-wide K group g of token t has its own scale gsx[t * (n/64) + g] and offset term
  // 256 * sum H + sum L over the group in gcorr[t * (n/64) + g].  The gate/up projection writes it
  // (xq_out, gsx_out, gcorr_out, in place of its fp32 output) and the skinny down projection reads it
  // (gsx, gcorr; its partials then carry the offset correction, so the reduce step gets zero sums).
  float* gsx_out;
  int* gcorr_out;
  const float* gsx;
  const int* gcorr;
  // One token: the K-split gate/up projection writes max |SiLU.up| of each block's 16 rows to
  // amax_out[block]; the down projection's quantization prologue (amax_in, amax_n maxima) then reads
  // only its own K chunks of the row, and one extra block forms the row's scale and limb sums.
  float* amax_out;
  const float* amax_in;
  int amax_n;
};

// K splits across blocks: at most kMaxSplits splits, only for GEMMs of at most kSplitTokens tokens;
// the workspace holds kMaxSplits x kSplitTokens x out floats.
constexpr int kMaxSplits = 16;
constexpr int kSplitTokens = 256;
// K splits of the one-token down projection (8960 = 5 x 14 chunks of 128), whose partials the next
// layer's Q/K/V blocks reduce in their prologue.
constexpr int kPreResidualSplits = 5;
// Head ranges (K ranges of 1536 / kOneTokenOSplits columns) of the one-token O projection: each block
// merges the attention of its range's heads and quantizes them with their own scale, and the gate/up
// projection's prologue adds the kOneTokenOSplits partials.
constexpr int kOneTokenOSplits = 2;
// Decode GEMMs of at most kSkinnyTokens tokens (in_dim 1536 or 8960) run the skinny kernels.
constexpr int kSkinnyTokens = 64;
inline size_t splitk_bytes(size_t out) { return (size_t)kMaxSplits * kSplitTokens * out * 4u; }

void launch_repack_int4(const uint8_t* W, int out_dim, int in_dim, uint8_t* WP, hipStream_t st);
void launch_norm_quant(const float* x, size_t x_stride, int rows, int n, const float* w, int norm, int8_t* xq,
                       float* sx, int* sums, float* xn, hipStream_t st);
void launch_gemm_i8(const GemmArgs& a, int epi, hipStream_t st);
// A projection of one token whose activation row is `pre`'s unfinished reduce step (epilogue
// pre_epi, pre_splits K splits of fp32 partials, kFuseNormQuant on a 1536-wide row): every block
// finishes that row into its own activation slice, block 0 writes it to pre.y.  Shapes: gate/up +
// SiLU·up after the O projection (pre_epi kEpiStore), the fused Q/K/V + RoPE after the down
// projection (pre_epi kEpiResidual).  Returns false (nothing launched) for other shapes.
bool launch_gemm_i8_pre(const GemmArgs& a, const GemmArgs& pre, int pre_epi, int pre_splits, hipStream_t st);
// Row-maxima count that the one-token gate/up projection (launch_gemm_i8_pre with wp2 and amax_out)
// writes for an out_dim-row output: one per block.
int gate_up_maxima_count(int out_dim);
// The down projection (+ residual) of one token whose activation row is the fp32 row pre.y
// (pre.in_dim = 8960 wide): every block quantizes that row for its own K chunks (as norm_quant_kernel
// without a norm), block 0 writes its scale and limb sums to pre.sx_out / pre.sums_out (= a.sx,
// a.sums), followed by the reduce step unless a.defer_reduce.  Returns false for other shapes.
bool launch_gemm_i8_preq(const GemmArgs& a, const GemmArgs& pre, hipStream_t st);
// The O projection of one token whose input row is the attention context of `am`: every block merges
// the attention's split partials (the arithmetic of attn_decode_kernel's merge) and quantizes the row
// into its own slice; block 0 writes the row's scale and limb sums to am.sx_out / am.sums_out (= a.sx,
// a.sums), followed by the reduce step unless a.defer_reduce.  Returns false for other shapes.
bool launch_gemm_i8_prea(const GemmArgs& a, const AttnMergeArgs& am, hipStream_t st);
// The fused [q | k | v] projection + RoPE + K/V append of one token (a.fuse == kFuseQkvRope) with the
// decode attention over the history keys fused in (AttnFuseArgs; af.chunk == kFusedAttnChunk, at most
// kFusedAttnMaxSplits splits): its partials are merged, with the new key's term, by the O projection
// (launch_gemm_i8_prea with am.qkv_new set).  _pre: the activation row is `pre`'s unfinished down-projection
// reduce step (as launch_gemm_i8_pre with kEpiResidual; pre_splits == 0: the row pre.resid itself,
// normalized and quantized, with pre.sums and pre.sx pointing at zeros and pre.y, pre.y_raw null);
// otherwise a.xq holds the quantized row.
// Returns false (nothing launched) for other shapes.
bool launch_gemm_i8_attn(const GemmArgs& a, const AttnFuseArgs& af, hipStream_t st);
bool launch_gemm_i8_pre_attn(const GemmArgs& a, const GemmArgs& pre, int pre_splits, const AttnFuseArgs& af,
                             hipStream_t st);
// Decode (pos given): token t is sequence t at position pos[t].  Prefill (pos null): token t is
// sequence t / seq_len at position past + t % seq_len.  Positions outside [0, limit) are skipped.
void launch_rope_qkv(float* qkv, int qkv_stride, const int* pos, int seq_len, int past, int limit, int tokens,
                     const float* rope, float* k_cache, float* v_cache, size_t seq_stride, hipStream_t st);
// Decode attention split: nsplit blocks of `chunk` keys (a multiple of 16) per sequence and KV
// head, sized so that one launch fills the device once.  Workspace: part [batch][12][nsplit][128]
// floats, pml [batch][12][nsplit] (m, l) pairs.  launch_attn_decode leaves the split partials there,
// then (xq given) merges them into the context row, written to ctx when given, and its two-limb
// code (xq, sx, sums); batch <= 65535 (one grid z index per sequence).
struct AttnDecodePlan {
  int nsplit, chunk;
};
// `cus`: the CUs the launch may use (a CU-masked stream), 0 for all of them.
AttnDecodePlan plan_attn_decode(int batch, int max_keys, int cus = 0);
void launch_zero_u32(unsigned* p, int n, hipStream_t st);
void launch_attn_decode(const float* qkv, int qkv_stride, const float* k_cache, const float* v_cache,
                        size_t seq_stride, const int* pos, int batch, int max_keys, const AttnDecodePlan& plan,
                        float* part, float2* pml, float* ctx, int8_t* xq, float* sx, int* sums, hipStream_t st);
// Prefill attention of S new tokens per sequence at positions past..past+S-1 over the cache rows
// 0..past+S-1: K/V converted once into bf16 hi/lo tiles (workspace of
// attn_prefill_workspace_bytes(past + S, nseq)), then the causal attention over them.
size_t attn_prefill_workspace_bytes(int keys, int nseq);
void launch_attn_prefill(const float* qkv, int qkv_stride, const float* k_cache, const float* v_cache,
                         size_t seq_stride, int S, int past, int nseq, uint8_t* kv_tiles, float* ctx,
                         hipStream_t st);
void launch_round_bf16(float* x, size_t n, hipStream_t st);

}  // namespace qwen

namespace qwen {

// ---- device quantizer, synthetic inputs, embedding: kernels_init.hip ----
uint64_t synth_stream_host(uint64_t seed, uint64_t key);
void launch_quantize_rows(const float* src, int out_dim, int in_dim, uint64_t stream, float sigma, uint8_t* packed,
                          float* scales, hipStream_t st);
void launch_fill_vector(float* dst, size_t n, uint64_t stream, float sigma, int bf16, float constant, hipStream_t st);
void launch_fill_bf16_table(uint16_t* dst, size_t n, uint64_t stream, float sigma, hipStream_t st);
void launch_kv_synthetic(float* cache, uint64_t rows, uint64_t stream, hipStream_t st);
void launch_embed(const uint16_t* table, int vocab, const int* ids, int count, float* hidden, hipStream_t st);
void launch_eval_expf(uint32_t first, uint32_t stride, uint64_t n, float* y, hipStream_t st);

// ---- unquantized layer-0 reference path: kernels_layer0.hip ----
// fp32 weights [out][in] row-major (biases optional), device pointers.
struct Layer0Weights {
  const float *ln, *qw, *qb, *kw, *kb, *vw, *vb, *ow, *ob, *post_ln, *gw, *gb, *uw, *ub, *dw, *db;
};
// Tokens whose attention probabilities are held at once (bounded workspace), of T queries over at
// most nmax keys.
int layer0_attention_chunk(int T, int nmax);
size_t layer0_workspace_bytes(int T, int past, bool decode);
// decode: T = 1 token at position `past`, past_k/past_v head-major [2][past][128], k_out/v_out
// head-major [2][past+1][128].  prefill: T tokens at positions 0..T-1, k_out/v_out (optional)
// head-major [2][T][128].  rope_tab: [T][cos 64 | sin 64] from the host libm (prefill: bf16-rounded).
void run_layer0_reference(const Layer0Weights& W, float eps, bool decode, const float* x, int T, int past,
                          const float* rope_tab, const float* past_k, const float* past_v, float* out, float* k_out,
                          float* v_out, void* workspace, hipStream_t st);

// ---- model head: kernels_head.hip ----
// Final RMSNorm (bf16 weight norm_w[1536]) of `count` hidden rows, tied bf16 lm_head over
// table[vocab][1536] (vocab a multiple of 128), bf16-rounded logits [count][vocab] (when logits is
// not null) and greedy token ids [count] (when ids is not null).  workspace: head_workspace_bytes.
size_t head_workspace_bytes(int count, int vocab);
void launch_head(const float* hidden, int count, const uint16_t* norm_w, const uint16_t* table, int vocab,
                 void* workspace, float* logits, int* ids, hipStream_t st);

}  // namespace qwen
