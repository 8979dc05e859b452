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
constexpr int kHeadBlockRows = 64;         // vocab rows of one tile set of an lm_head block (4 waves x 16)

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

// K steps [4*kb, 4*kb + 4) of one wave for its two row tiles: MFMAs on cur0/cur1 while nxt0/nxt1
// receive the next 4 steps.  B (the token tile's normalized rows) is read from LDS; lanes whose token
// is past the tile's live rows use zeros.
__device__ __forceinline__ void head_ksteps(const uint4 (&cur0)[4], const uint4 (&cur1)[4], uint4 (&nxt0)[4],
                                            uint4 (&nxt1)[4], bool prefetch, const uint4* ap0, const uint4* ap1,
                                            int kb, const uint16_t* xrow, bool live, hf32x4& acc0, hf32x4& acc1) {
  if (prefetch) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int off = 4 * (4 * (kb + 1) + s);
      const hf32x4 r0 = __builtin_nontemporal_load(reinterpret_cast<const hf32x4*>(ap0 + off));  // read once
      const hf32x4 r1 = __builtin_nontemporal_load(reinterpret_cast<const hf32x4*>(ap1 + off));
      nxt0[s] = make_uint4(__float_as_uint(r0[0]), __float_as_uint(r0[1]), __float_as_uint(r0[2]), __float_as_uint(r0[3]));
      nxt1[s] = make_uint4(__float_as_uint(r1[0]), __float_as_uint(r1[1]), __float_as_uint(r1[2]), __float_as_uint(r1[3]));
    }
  }
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    hbf16x8 b = {};
    if (live) b = *reinterpret_cast<const hbf16x8*>(xrow + 32 * (4 * kb + s));
    hbf16x8 a0, a1;
    __builtin_memcpy(&a0, &cur0[s], 16);
    __builtin_memcpy(&a1, &cur1[s], 16);
    acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b, acc0, 0, 0, 0);
    acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b, acc1, 0, 0, 0);
  }
}

// The block's best key per token column from the 4 logits a lane holds for rows rbase + 4g + i.
__device__ __forceinline__ unsigned long long head_best(const hf32x4& acc, int rbase, int g, float (&lf)[4]) {
  unsigned long long bk = 0ull;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    lf[i] = to_bf16(acc[i]);
    const uint32_t v = (uint32_t)(rbase + 4 * g + i);
    const unsigned long long key = ((unsigned long long)order_key(lf[i]) << 32) | (unsigned long long)(~v);
    bk = key > bk ? key : bk;
  }
  return bk;
}

// grid = (vocab / 128, ceil(count / 16)), block = 256, dynamic LDS = live rows x kHeadRow bf16.
// Wave w of block (vb, tt) computes the logits of the two 16-row tiles vb*128 + 16w and vb*128 + 64 +
// 16w for tokens tt*16 .. +15 over K = 1536 (48 MFMA steps of 32, 4 steps prefetched):
//   A = E[row l&15][k = 32s + 8(l>>4) .. +7] straight from HBM,
//   B = n[token l&15][same k] from the LDS copy of the tile's live token rows  ->  D[row 4(l>>4)+i][token l&15].
// One launch over 151936 rows is 1187 blocks of 4 waves: every block is resident at once, and every
// wave streams the same 96 KiB.  Each logit is rounded to bf16 (written to `logits` when LOGITS), and
// the block's best (order_key(logit) << 32 | ~row) per token goes to best[token][vb].
template <bool LOGITS>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(5))) lm_head_kernel(const uint16_t* __restrict__ table, int vocab,
                                                      const uint16_t* __restrict__ xn, int count,
                                                      float* __restrict__ logits,
                                                      unsigned long long* __restrict__ best) {
  extern __shared__ __align__(16) uint16_t xs[];
  __shared__ unsigned long long red[4][16];
  const int tt = blockIdx.y;
  const int live_rows = min(16, count - tt * 16);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, col = lane & 15, g = lane >> 4;
  const int row0 = blockIdx.x * (2 * kHeadBlockRows) + wave * 16;  // second tile: row0 + 64
  const uint4* ap0 = reinterpret_cast<const uint4*>(table + (size_t)(row0 + col) * QWEN_HIDDEN) + g;
  const uint4* ap1 = ap0 + (size_t)kHeadBlockRows * (QWEN_HIDDEN / 8);
  uint4 a0[4], a1[4], b0[4], b1[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const hf32x4 r0 = __builtin_nontemporal_load(reinterpret_cast<const hf32x4*>(ap0 + 4 * s));
    const hf32x4 r1 = __builtin_nontemporal_load(reinterpret_cast<const hf32x4*>(ap1 + 4 * s));
    a0[s] = make_uint4(__float_as_uint(r0[0]), __float_as_uint(r0[1]), __float_as_uint(r0[2]), __float_as_uint(r0[3]));
    a1[s] = make_uint4(__float_as_uint(r1[0]), __float_as_uint(r1[1]), __float_as_uint(r1[2]), __float_as_uint(r1[3]));
  }
  for (int i = threadIdx.x; i < live_rows * (QWEN_HIDDEN / 8); i += 256) {
    const int r = i / (QWEN_HIDDEN / 8), c = i % (QWEN_HIDDEN / 8);
    *reinterpret_cast<uint4*>(xs + r * kHeadRow + 8 * c) =
        *reinterpret_cast<const uint4*>(xn + (size_t)(tt * 16 + r) * QWEN_HIDDEN + 8 * c);
  }
  __syncthreads();
  const bool live = col < live_rows;
  const uint16_t* xrow = xs + (live ? col : 0) * kHeadRow + 8 * g;
  hf32x4 acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int kb = 0; kb < 12; kb += 2) {
    head_ksteps(a0, a1, b0, b1, true, ap0, ap1, kb, xrow, live, acc0, acc1);
    head_ksteps(b0, b1, a0, a1, kb + 2 < 12, ap0, ap1, kb + 1, xrow, live, acc0, acc1);
  }

  const int tok = tt * 16 + col;
  float lf0[4], lf1[4];
  const unsigned long long k0 = head_best(acc0, row0, g, lf0);
  const unsigned long long k1 = head_best(acc1, row0 + kHeadBlockRows, g, lf1);
  unsigned long long bk = k0 > k1 ? k0 : k1;
  if (LOGITS && tok < count) {
    float* lrow = logits + (size_t)tok * vocab + row0 + 4 * g;
    *reinterpret_cast<float4*>(lrow) = make_float4(lf0[0], lf0[1], lf0[2], lf0[3]);
    *reinterpret_cast<float4*>(lrow + kHeadBlockRows) = make_float4(lf1[0], lf1[1], lf1[2], lf1[3]);
  }
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

// One token (greedy decode): each logit as a dot product on the VALU, so that every load reads 1 KiB of
// one table row (lm_head_kernel's MFMA A operand reads 64 B of 16 rows per load: 5.0 TB/s).  grid =
// vocab / 128, block = 256; wave w of block vb takes rows vb*128 + 32w .. + 31, two at a time with the
// next two rows' loads in flight.  Lane l holds x[8l + 512j .. + 7] (j < 3) in fp32 and forms its 24
// products of a row in (j, e) order; the 64 lane sums are added by DPP row steps, then the four rows in
// lane order.  Logits are rounded to bf16 and keyed as in lm_head_kernel (best[0][vb]).
// NORM: the block reads the fp32 row `hidden` and the norm weights instead of the normalized row, and
// every wave forms head_norm_kernel's values for its lanes' 24 columns itself (the sum of squares over
// the whole row by each wave: exact in double, so the same var), with the first table rows in flight.
template <bool LOGITS, bool NORM = false>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(5)))
lm_head_row_kernel(const uint16_t* __restrict__ table, int vocab, const uint16_t* __restrict__ xn,
                   float* __restrict__ logits, unsigned long long* __restrict__ best,
                   const float* __restrict__ hidden = nullptr, const uint16_t* __restrict__ norm_w = nullptr) {
  __shared__ unsigned long long red[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row0 = blockIdx.x * (2 * kHeadBlockRows) + wave * 32;
  constexpr int kRowU4 = QWEN_HIDDEN / 8;  // uint4 per table row
  const uint4* tp = reinterpret_cast<const uint4*>(table) + (size_t)row0 * kRowU4 + lane;
  auto load2 = [&](int r, uint4 (&d)[2][3]) {
#pragma unroll
    for (int rr = 0; rr < 2; ++rr)
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        const hf32x4 v = __builtin_nontemporal_load(reinterpret_cast<const hf32x4*>(tp + (size_t)(r + rr) * kRowU4 + 64 * j));
        d[rr][j] = make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3]));
      }
  };
  uint4 cur[2][3], nxt[2][3];
  load2(0, cur);  // the first two rows in flight while the activation row is formed
  __builtin_amdgcn_sched_barrier(0);
  float x[3][8];
  if constexpr (NORM) {
    float v[3][8];
    uint4 wq[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const float4 a = *reinterpret_cast<const float4*>(hidden + 8 * lane + 512 * j);
      const float4 b = *reinterpret_cast<const float4*>(hidden + 8 * lane + 512 * j + 4);
      wq[j] = *reinterpret_cast<const uint4*>(norm_w + 8 * lane + 512 * j);
      const float h[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) v[j][e] = to_bf16(h[e]);
    }
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < 3; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += (double)v[j][e] * (double)v[j][e];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
    const float var = (float)ss / (float)QWEN_HIDDEN;
    const float r = 1.0f / sqrtf(var + QWEN_RMS_EPS);
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const uint32_t w4[4] = {wq[j].x, wq[j].y, wq[j].z, wq[j].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float w = bits_f32(e & 1 ? (w4[e >> 1] & 0xFFFF0000u) : (w4[e >> 1] << 16));
        x[j][e] = to_bf16(w * to_bf16(v[j][e] * r));
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const uint4 q = *reinterpret_cast<const uint4*>(xn + 8 * lane + 512 * j);
      const uint32_t w4[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x[j][2 * e] = bits_f32(w4[e] << 16);
        x[j][2 * e + 1] = bits_f32(w4[e] & 0xFFFF0000u);
      }
    }
  }
  unsigned long long bk = 0ull;
#pragma unroll 1
  for (int r = 0; r < 32; r += 2) {
    if (r + 2 < 32) load2(r + 2, nxt);
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        const uint32_t w4[4] = {cur[rr][j].x, cur[rr][j].y, cur[rr][j].z, cur[rr][j].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc = fmaf(bits_f32(w4[e] << 16), x[j][2 * e], acc);
          acc = fmaf(bits_f32(w4[e] & 0xFFFF0000u), x[j][2 * e + 1], acc);
        }
      }
      // row sums of 16 lanes (quad_perm [1,0,3,2], [2,3,0,1], row_ror:4, row_ror:8), then the 4 rows
      acc += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(acc), 0xB1, 0xF, 0xF, false));
      acc += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(acc), 0x4E, 0xF, 0xF, false));
      acc += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(acc), 0x124, 0xF, 0xF, false));
      acc += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(acc), 0x128, 0xF, 0xF, false));
      const int ab = __float_as_int(acc);
      const float tot = (__int_as_float(__builtin_amdgcn_readlane(ab, 0)) + __int_as_float(__builtin_amdgcn_readlane(ab, 16))) +
                        (__int_as_float(__builtin_amdgcn_readlane(ab, 32)) + __int_as_float(__builtin_amdgcn_readlane(ab, 48)));
      const float lf = to_bf16(tot);
      const uint32_t v = (uint32_t)(row0 + r + rr);
      const unsigned long long key = ((unsigned long long)order_key(lf) << 32) | (unsigned long long)(~v);
      bk = key > bk ? key : bk;
      if (LOGITS && lane == 0) logits[row0 + r + rr] = lf;
    }
#pragma unroll
    for (int rr = 0; rr < 2; ++rr)
#pragma unroll
      for (int j = 0; j < 3; ++j) cur[rr][j] = nxt[rr][j];
  }
  if (lane == 0) red[wave] = bk;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long m = red[0];
#pragma unroll
    for (int w = 1; w < 4; ++w) m = red[w] > m ? red[w] : m;
    best[blockIdx.x] = m;
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
  return rows * QWEN_HIDDEN * 2u + (size_t)count * (size_t)(vocab / (2 * kHeadBlockRows)) * 8u + 256u;
}

void launch_head(const float* hidden, int count, const uint16_t* norm_w, const uint16_t* table, int vocab,
                 void* workspace, float* logits, int* ids, hipStream_t st) {
  const int tiles = (count + 15) / 16;
  uint16_t* xn = static_cast<uint16_t*>(workspace);
  const size_t xn_bytes = (size_t)tiles * 16 * QWEN_HIDDEN * 2u;
  unsigned long long* best =
      reinterpret_cast<unsigned long long*>(static_cast<char*>(workspace) + ((xn_bytes + 255u) & ~size_t(255u)));
  const int nblk = vocab / (2 * kHeadBlockRows);
  const size_t lds = (size_t)(count < 16 ? count : 16) * kHeadRow * 2u;  // live token rows of a tile
  // one token: the norm runs inside every lm_head block (no launch of its own)
  if (count == 1 && logits)
    hipLaunchKernelGGL((lm_head_row_kernel<true, true>), dim3(nblk), dim3(256), 0, st, table, vocab, xn, logits, best,
                       hidden, norm_w);
  else if (count == 1)
    hipLaunchKernelGGL((lm_head_row_kernel<false, true>), dim3(nblk), dim3(256), 0, st, table, vocab, xn, logits, best,
                       hidden, norm_w);
  else {
    hipLaunchKernelGGL(head_norm_kernel, dim3(tiles * 16), dim3(256), 0, st, hidden, count, norm_w, xn);
    if (logits)
      hipLaunchKernelGGL(lm_head_kernel<true>, dim3(nblk, tiles), dim3(256), lds, st, table, vocab, xn, count, logits,
                         best);
    else
      hipLaunchKernelGGL(lm_head_kernel<false>, dim3(nblk, tiles), dim3(256), lds, st, table, vocab, xn, count, logits,
                         best);
  }
  if (ids) hipLaunchKernelGGL(argmax_finalize_kernel, dim3(count), dim3(256), 0, st, best, nblk, ids);
}

}  // namespace qwen
