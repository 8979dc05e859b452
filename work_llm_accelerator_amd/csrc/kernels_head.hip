// Model head of the greedy driver: final RMSNorm, tied bf16 lm_head, greedy argmax.
//
// Semantics of verification/real_host_top_backend.py:138-146 (_finalize_logits) on the bf16 model of
// verification/torch_reference_backend.py:67, and of the greedy step of
// verification/qwen_full_model_validation.py:128,159 (torch.argmax over the last position's logits):
//   x  = bf16(hidden)                                  (the driver's fp32 rows -> model dtype)
//   Qwen2RMSNorm: v = fp32(x); var = sum(v*v) / 1536; r = 1 / sqrt(var + 1e-6);
//                 n = bf16(w * bf16(v * r))            (fp32 math, bf16 results; the squares of
//                                                       bf16 values are summed in double and the
//                                                       sum rounded once to fp32, so var is the
//                                                       correctly rounded value whatever the order)
//   logits = bf16(n . E^T)                             (bf16 Linear, fp32 accumulation; E = the
//                                                       tied embedding table [vocab][1536])
//   token  = first index of the maximal logit (a NaN counts as the maximum, as torch.argmax).
// Built without FMA contraction: every fp32 step of the norm is one IEEE operation.  The lm_head
// runs on the bf16 matrix cores (exact bf16 products, fp32 accumulation in MFMA order).
#include <hip/hip_runtime.h>

#include "kernels.hpp"
#include "qwen_device_math.hpp"

namespace qwen {

typedef __bf16 hbf16x8 __attribute__((ext_vector_type(8)));
typedef float hf32x4 __attribute__((ext_vector_type(4)));

constexpr int kHeadRow = QWEN_HIDDEN + 8;  // bf16 per staged activation row (16-byte pad)
constexpr int kHeadBlockRows = 64;         // vocab rows per lm_head block (4 waves x 16)

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }
// torch's float -> bfloat16 conversion: round to nearest even, NaN kept as a quiet NaN.
__device__ __forceinline__ float to_bf16(float x) {
  return (f32_bits(x) & 0x7FFFFFFFu) > 0x7F800000u ? bits_f32(0x7FC00000u) : round_bf16(x);
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float x) { return (uint16_t)(f32_bits(to_bf16(x)) >> 16); }

// Total order of floats for the argmax key: larger value -> larger key, -0 == +0, NaN above all.
__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t b = f32_bits(f);
  if ((b & 0x7FFFFFFFu) > 0x7F800000u) return 0xFFFFFFFFu;
  if (b == 0x80000000u) b = 0u;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// One block per row (rows_padded, a multiple of 16); rows >= count are written as zeros so the
// lm_head can stage whole 16-row tiles.  block = 256 (6 values per thread).
__global__ void __launch_bounds__(256) head_norm_kernel(const float* __restrict__ x, int count,
                                                        const uint16_t* __restrict__ w, uint16_t* __restrict__ out) {
  __shared__ double red[4];
  const int t = blockIdx.x;
  uint16_t* o = out + (size_t)t * QWEN_HIDDEN;
  if (t >= count) {
    for (int d = threadIdx.x; d < QWEN_HIDDEN; d += 256) o[d] = 0;
    return;
  }
  constexpr int NV = QWEN_HIDDEN / 256;
  float v[NV];
  double ss = 0.0;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    v[j] = to_bf16(x[(size_t)t * QWEN_HIDDEN + threadIdx.x + 256 * j]);
    ss += (double)v[j] * (double)v[j];
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  ss = (red[0] + red[1]) + (red[2] + red[3]);
  const float var = (float)ss / (float)QWEN_HIDDEN;
  const float r = 1.0f / sqrtf(var + QWEN_RMS_EPS);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int d = threadIdx.x + 256 * j;
    const float y = to_bf16(v[j] * r);
    o[d] = f32_to_bf16_bits(bf16_bits_to_f32(w[d]) * y);
  }
}

// K steps [8*kb, 8*kb + 8) of one wave: MFMAs on `cur` while `nxt` receives the next 8 steps.
__device__ __forceinline__ void head_ksteps(const uint4 (&cur)[8], uint4 (&nxt)[8], bool prefetch, const uint4* ap,
                                            int kb, const uint16_t* xrow, hf32x4& acc) {
  if (prefetch) {
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const uint4* p = ap + 4 * (8 * (kb + 1) + s);
      const hf32x4 raw = __builtin_nontemporal_load(reinterpret_cast<const hf32x4*>(p));  // read once per call
      nxt[s] = make_uint4(__float_as_uint(raw[0]), __float_as_uint(raw[1]), __float_as_uint(raw[2]),
                          __float_as_uint(raw[3]));
    }
  }
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const hbf16x8 b = *reinterpret_cast<const hbf16x8*>(xrow + 32 * (8 * kb + s));
    hbf16x8 a;
    __builtin_memcpy(&a, &cur[s], 16);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
  }
}

// grid = (vocab / 64, ceil(count / 16)), block = 256.  Wave w of block (vb, tt) computes the 16 x 16
// logits of vocab rows vb*64 + 16w .. +15 and tokens tt*16 .. +15 over K = 1536 (48 MFMA steps of 32):
//   A = E[row l&15][k = 32s + 8(l>>4) .. +7] straight from HBM (8 steps prefetched),
//   B = n[token l&15][same k] from the LDS copy of the token tile  ->  D[row 4(l>>4)+i][token l&15].
// Each logit is rounded to bf16 (written to `logits` when LOGITS), and the block's best
// (order_key(logit) << 32 | ~row) per token goes to best[token][vb].
template <bool LOGITS>
__global__ void __launch_bounds__(256) lm_head_kernel(const uint16_t* __restrict__ table, int vocab,
                                                      const uint16_t* __restrict__ xn, int count,
                                                      float* __restrict__ logits,
                                                      unsigned long long* __restrict__ best) {
  __shared__ __align__(16) uint16_t xs[16 * kHeadRow];
  __shared__ unsigned long long red[4][16];
  const int tt = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, col = lane & 15, g = lane >> 4;
  const int row0 = blockIdx.x * kHeadBlockRows + wave * 16;
  const uint4* ap = reinterpret_cast<const uint4*>(table + (size_t)(row0 + col) * QWEN_HIDDEN) + g;
  uint4 a0[8], a1[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const hf32x4 raw = __builtin_nontemporal_load(reinterpret_cast<const hf32x4*>(ap + 4 * s));
    a0[s] = make_uint4(__float_as_uint(raw[0]), __float_as_uint(raw[1]), __float_as_uint(raw[2]),
                       __float_as_uint(raw[3]));
  }
  for (int i = threadIdx.x; i < 16 * (QWEN_HIDDEN / 8); i += 256) {
    const int r = i / (QWEN_HIDDEN / 8), c = i % (QWEN_HIDDEN / 8);
    *reinterpret_cast<uint4*>(xs + r * kHeadRow + 8 * c) =
        *reinterpret_cast<const uint4*>(xn + (size_t)(tt * 16 + r) * QWEN_HIDDEN + 8 * c);
  }
  __syncthreads();
  const uint16_t* xrow = xs + col * kHeadRow + 8 * g;
  hf32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  head_ksteps(a0, a1, true, ap, 0, xrow, acc);
  head_ksteps(a1, a0, true, ap, 1, xrow, acc);
  head_ksteps(a0, a1, true, ap, 2, xrow, acc);
  head_ksteps(a1, a0, true, ap, 3, xrow, acc);
  head_ksteps(a0, a1, true, ap, 4, xrow, acc);
  head_ksteps(a1, a0, false, ap, 5, xrow, acc);

  const int tok = tt * 16 + col;
  unsigned long long bk = 0ull;
  float lf[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    lf[i] = to_bf16(acc[i]);
    const uint32_t v = (uint32_t)(row0 + 4 * g + i);
    const unsigned long long key = ((unsigned long long)order_key(lf[i]) << 32) | (unsigned long long)(~v);
    bk = key > bk ? key : bk;
  }
  if (LOGITS && tok < count)
    *reinterpret_cast<float4*>(logits + (size_t)tok * vocab + row0 + 4 * g) = make_float4(lf[0], lf[1], lf[2], lf[3]);
#pragma unroll
  for (int off = 16; off < 64; off <<= 1) {
    const unsigned long long o = __shfl_xor(bk, off, 64);
    bk = o > bk ? o : bk;
  }
  if (g == 0) red[wave][col] = bk;
  __syncthreads();
  if (threadIdx.x < 16) {
    unsigned long long m = red[0][threadIdx.x];
#pragma unroll
    for (int w = 1; w < 4; ++w) m = red[w][threadIdx.x] > m ? red[w][threadIdx.x] : m;
    const int t = tt * 16 + threadIdx.x;
    if (t < count) best[(size_t)t * gridDim.x + blockIdx.x] = m;
  }
}

// ids[t] = the row of the largest key in best[t][0 .. nblk).  grid = count, block = 256.
__global__ void __launch_bounds__(256) argmax_finalize_kernel(const unsigned long long* __restrict__ best, int nblk,
                                                              int* __restrict__ ids) {
  __shared__ unsigned long long red[4];
  const unsigned long long* b = best + (size_t)blockIdx.x * nblk;
  unsigned long long m = 0ull;
  for (int i = threadIdx.x; i < nblk; i += 256) m = b[i] > m ? b[i] : m;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const unsigned long long o = __shfl_xor(m, off, 64);
    m = o > m ? o : m;
  }
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    m = red[0];
    for (int w = 1; w < 4; ++w) m = red[w] > m ? red[w] : m;
    ids[blockIdx.x] = (int)~(uint32_t)(m & 0xFFFFFFFFull);
  }
}

size_t head_workspace_bytes(int count, int vocab) {
  const size_t rows = (size_t)((count + 15) / 16) * 16;
  return rows * QWEN_HIDDEN * 2u + (size_t)count * (size_t)(vocab / kHeadBlockRows) * 8u + 256u;
}

void launch_head(const float* hidden, int count, const uint16_t* norm_w, const uint16_t* table, int vocab,
                 void* workspace, float* logits, int* ids, hipStream_t st) {
  const int tiles = (count + 15) / 16;
  uint16_t* xn = static_cast<uint16_t*>(workspace);
  const size_t xn_bytes = (size_t)tiles * 16 * QWEN_HIDDEN * 2u;
  unsigned long long* best =
      reinterpret_cast<unsigned long long*>(static_cast<char*>(workspace) + ((xn_bytes + 255u) & ~size_t(255u)));
  const int nblk = vocab / kHeadBlockRows;
  hipLaunchKernelGGL(head_norm_kernel, dim3(tiles * 16), dim3(256), 0, st, hidden, count, norm_w, xn);
  if (logits)
    hipLaunchKernelGGL(lm_head_kernel<true>, dim3(nblk, tiles), dim3(256), 0, st, table, vocab, xn, count, logits,
                       best);
  else
    hipLaunchKernelGGL(lm_head_kernel<false>, dim3(nblk, tiles), dim3(256), 0, st, table, vocab, xn, count, logits,
                       best);
  if (ids) hipLaunchKernelGGL(argmax_finalize_kernel, dim3(count), dim3(256), 0, st, best, nblk, ids);
}

}  // namespace qwen
