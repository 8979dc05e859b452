// ORDERED kernels: bit-exact restatement of the reference host arithmetic on gfx950.
//
// The reference evaluates every output with one serial fp32 chain (qwen_decode_attention_kernel.cpp
// :62-98 and its prefill twins), so these kernels parallelise only across independent outputs
// (rows, tokens, heads, head dims) and keep each chain serial, in the reference order, with no
// FMA contraction (this file is built with -ffp-contract=off).  Weight tiles are staged through
// LDS with coalesced 16-byte loads so that HBM reads stay full-line even though each lane walks
// its own row.
#include <hip/hip_runtime.h>

#include "kernels.hpp"
#include "qwen_device_math.hpp"

namespace qwen {

// ---------------------------------------------------------------------------------------------
// RMSNorm.  decode: double serial sum (qwen_decode_attention_kernel.cpp:13-27);
// prefill: float serial sum + approx_sqrt (qwen_prefill_attention_kernel.cpp:112-126).
// grid.x = tokens, block = 256.
// ---------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) rmsnorm_ordered_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                              float* __restrict__ y, int prefill) {
  __shared__ float xs[QWEN_HIDDEN];
  __shared__ double inv_d;
  __shared__ float inv_f;
  const size_t row = (size_t)blockIdx.x * QWEN_HIDDEN;
  for (int d = threadIdx.x; d < QWEN_HIDDEN; d += blockDim.x) xs[d] = x[row + d];
  __syncthreads();
  if (threadIdx.x == 0) {
    if (prefill) {
      float ms = 0.0f;
      for (int d = 0; d < QWEN_HIDDEN; ++d) ms += xs[d] * xs[d];
      ms /= (float)QWEN_HIDDEN;
      inv_f = 1.0f / approx_sqrt(ms + QWEN_RMS_EPS);
    } else {
      double ms = 0.0;
      for (int d = 0; d < QWEN_HIDDEN; ++d) ms += (double)xs[d] * (double)xs[d];
      ms /= (double)QWEN_HIDDEN;
      inv_d = 1.0 / __dsqrt_rn(ms + (double)QWEN_RMS_EPS);
    }
  }
  __syncthreads();
  if (prefill) {
    const float inv = inv_f;
    for (int d = threadIdx.x; d < QWEN_HIDDEN; d += blockDim.x) y[row + d] = xs[d] * inv * w[d];
  } else {
    const double inv = inv_d;
    for (int d = threadIdx.x; d < QWEN_HIDDEN; d += blockDim.x)
      y[row + d] = (float)((double)xs[d] * inv * (double)w[d]);
  }
}

// ---------------------------------------------------------------------------------------------
// Serial INT4 projection (project_tiled, qwen_decode_attention_kernel.cpp:62-98):
//   y[t][o] = (residual[t][o] +) ( bias[o] + x[t][0]*w(o,0) + x[t][1]*w(o,1) + ... )  left to right,
//   w(o,i) = (float)int4(o,i) * scale[o].
// One thread per output row o; each thread carries TT token chains (independent, so the
// interleaving keeps every chain's order).  The K loop runs in chunks of 256 inputs: the block
// stages its 256 rows x 128 bytes of packed weights and TT x 256 inputs in LDS.
// grid = (out_dim/256, ceil(tokens/TT)), block = 256.  Requires in_dim % 256 == 0.
// ---------------------------------------------------------------------------------------------
constexpr int kOrdRows = 256;
constexpr int kOrdChunk = 256;                  // inputs per chunk
constexpr int kOrdChunkBytes = kOrdChunk / 2;   // 128 bytes of packed weights per row
constexpr int kOrdRowPitch = kOrdChunkBytes + 16;  // LDS row pitch, padded against bank conflicts

template <int TT>
__global__ void __launch_bounds__(256) project_ordered_kernel(const float* __restrict__ x, int tokens, int in_dim,
                                                              const uint8_t* __restrict__ W,
                                                              const float* __restrict__ scale,
                                                              const float* __restrict__ bias, int out_dim,
                                                              float* __restrict__ y, const float* __restrict__ residual) {
  __shared__ __align__(16) uint8_t wt[kOrdRows * kOrdRowPitch];
  __shared__ float xt[TT][kOrdChunk];
  const int tid = threadIdx.x;
  const int row0 = blockIdx.x * kOrdRows;
  const int o = row0 + tid;
  const int t0 = blockIdx.y * TT;
  const bool row_ok = o < out_dim;
  const float s = row_ok ? scale[o] : 0.0f;
  float acc[TT];
  const float b0 = (row_ok && bias) ? bias[o] : 0.0f;
#pragma unroll
  for (int t = 0; t < TT; ++t) acc[t] = b0;
  const size_t row_bytes = (size_t)in_dim / 2;

  for (int k0 = 0; k0 < in_dim; k0 += kOrdChunk) {
    // Stage the weight tile: 256 rows x 128 bytes = 2048 chunks of 16 bytes, 8 per thread.
    // Lane l of a group of 8 reads bytes [16l, 16l+16) of one row: 8 rows per wave-load.
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int c = j * 256 + tid;
      const int r = c >> 3;
      const int part = c & 7;
      uint4 v = make_uint4(0u, 0u, 0u, 0u);
      if (row0 + r < out_dim)
        v = *reinterpret_cast<const uint4*>(W + (size_t)(row0 + r) * row_bytes + (size_t)k0 / 2 + (size_t)part * 16);
      *reinterpret_cast<uint4*>(&wt[r * kOrdRowPitch + part * 16]) = v;
    }
    for (int e = tid; e < TT * kOrdChunk; e += 256) {
      const int t = e / kOrdChunk;
      const int i = e - t * kOrdChunk;
      xt[t][i] = (t0 + t < tokens) ? x[(size_t)(t0 + t) * in_dim + k0 + i] : 0.0f;
    }
    __syncthreads();
    if (row_ok) {
      const uint8_t* my = &wt[tid * kOrdRowPitch];
      for (int b16 = 0; b16 < kOrdChunkBytes; b16 += 16) {
        const uint4 pk = *reinterpret_cast<const uint4*>(my + b16);
        const uint32_t words[4] = {pk.x, pk.y, pk.z, pk.w};
#pragma unroll
        for (int wi = 0; wi < 4; ++wi) {
#pragma unroll
          for (int bi = 0; bi < 4; ++bi) {
            const uint32_t byte = (words[wi] >> (8 * bi)) & 0xFFu;
            const int i = b16 * 2 + wi * 8 + bi * 2;
            const float w_lo = (float)nibble_lo(byte) * s;
            const float w_hi = (float)nibble_hi(byte) * s;
#pragma unroll
            for (int t = 0; t < TT; ++t) {
              acc[t] = acc[t] + xt[t][i] * w_lo;
              acc[t] = acc[t] + xt[t][i + 1] * w_hi;
            }
          }
        }
      }
    }
    __syncthreads();
  }
  if (row_ok) {
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      if (t0 + t < tokens) {
        const size_t idx = (size_t)(t0 + t) * out_dim + o;
        y[idx] = residual ? residual[idx] + acc[t] : acc[t];
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// s = silu(g) * u.  decode silu uses the host-compatible expf (qwen_decode_mlp_kernel.cpp:79-81,
// 113-115), prefill silu uses approx_exp (qwen_prefill_mlp_kernel.cpp:256-258, 318-320).
// ---------------------------------------------------------------------------------------------
__global__ void silu_mul_kernel(const float* __restrict__ g, const float* __restrict__ u, float* __restrict__ s,
                                size_t n, int prefill) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float gv = g[i];
  const float sv = prefill ? silu_prefill(gv) : silu_decode(gv);
  s[i] = sv * u[i];
}

// ---------------------------------------------------------------------------------------------
// RoPE + KV append for decode (qwen_decode_attention_kernel.cpp:29-42, 100-111, 206-213).
// One block of 64 threads per token b: pair p of every Q head and both K heads rotated with the
// host-computed (cos, sin) row of position pos[b]; K (rotated) and V rows written to row pos[b]
// of that token's cache.  rope: [positions][2][64] (cos row then sin row).  Positions outside
// [0, max_keys) are skipped (max_keys = the cache rows the caller sized).
// ---------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(64) rope_append_decode_kernel(float* __restrict__ q, const float* __restrict__ k,
                                                                const float* __restrict__ v, const int* __restrict__ pos,
                                                                const float* __restrict__ rope, int rope_rows_are_tokens,
                                                                float* __restrict__ k_cache, float* __restrict__ v_cache,
                                                                size_t cache_stride, int max_keys) {
  const int b = blockIdx.x;
  const int p = threadIdx.x;
  const int P = pos[b];
  if (P < 0 || P >= max_keys) return;  // position outside the cache rows the caller sized
  const float* cs = rope + (size_t)(rope_rows_are_tokens ? b : P) * 128;
  const float c = cs[p];
  const float sn = cs[64 + p];
  float* qb = q + (size_t)b * QWEN_HIDDEN;
  for (int h = 0; h < QWEN_Q_HEADS; ++h) {
    float* hp = qb + h * QWEN_HEAD_DIM;
    const float e = hp[p], od = hp[p + 64];
    hp[p] = e * c - od * sn;
    hp[p + 64] = od * c + e * sn;
  }
  float* kr = k_cache + (size_t)b * cache_stride + (size_t)P * QWEN_KV_WIDTH;
  float* vr = v_cache + (size_t)b * cache_stride + (size_t)P * QWEN_KV_WIDTH;
  const float* kb = k + (size_t)b * QWEN_KV_WIDTH;
  const float* vb = v + (size_t)b * QWEN_KV_WIDTH;
  for (int h = 0; h < QWEN_KV_HEADS; ++h) {
    const int base = h * QWEN_HEAD_DIM;
    const float e = kb[base + p], od = kb[base + p + 64];
    kr[base + p] = e * c - od * sn;
    kr[base + p + 64] = od * c + e * sn;
    vr[base + p] = vb[base + p];
    vr[base + p + 64] = vb[base + p + 64];
  }
}

// ---------------------------------------------------------------------------------------------
// RoPE for prefill, in place on the Q rows and the K cache rows of every token
// (qwen_prefill_attention_kernel.cpp:2304-2309, 2332-2337).  rope: [positions][2][64].
// grid.x = tokens, block = 64.  Token t has position t.
// ---------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(64) rope_prefill_kernel(float* __restrict__ q, float* __restrict__ k_rows,
                                                          const float* __restrict__ rope) {
  const int t = blockIdx.x;
  const int p = threadIdx.x;
  const float c = rope[(size_t)t * 128 + p];
  const float sn = rope[(size_t)t * 128 + 64 + p];
  float* qt = q + (size_t)t * QWEN_HIDDEN;
  for (int h = 0; h < QWEN_Q_HEADS; ++h) {
    float* hp = qt + h * QWEN_HEAD_DIM;
    const float e = hp[p], od = hp[p + 64];
    hp[p] = e * c - od * sn;
    hp[p + 64] = od * c + e * sn;
  }
  float* kt = k_rows + (size_t)t * QWEN_KV_WIDTH;
  for (int h = 0; h < QWEN_KV_HEADS; ++h) {
    float* hp = kt + h * QWEN_HEAD_DIM;
    const float e = hp[p], od = hp[p + 64];
    hp[p] = e * c - od * sn;
    hp[p + 64] = od * c + e * sn;
  }
}

// Prefill RoPE table (qwen_prefill_attention_kernel.cpp:128-143): inv_freq chain in float,
// angle = (float)pos * inv_freq, approx_sincos.  grid covers positions x 64 pairs.
__global__ void rope_table_prefill_kernel(float* __restrict__ rope, int first, int count) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= count * 64) return;
  const int pos = first + idx / 64;
  const int p = idx % 64;
  float inv_freq = 1.0f;
  for (int j = 0; j < p; ++j) inv_freq *= 0.8058421877614801f;
  const float angle = (float)pos * inv_freq;
  float s, c;
  approx_sincos(angle, &s, &c);
  rope[(size_t)pos * 128 + p] = c;
  rope[(size_t)pos * 128 + 64 + p] = s;
}

// ---------------------------------------------------------------------------------------------
// Two-pass softmax attention, one block of 128 threads per (head, query token).
// decode: decode_attention_context (qwen_decode_attention_kernel.cpp:113-162), keys 0..pos[b],
//         scaling (float)(1/sqrt(128)), host-compatible expf;
// prefill: prefill_attention_context_block (qwen_prefill_attention_kernel.cpp:204-289), keys
//         0..t, scaling 0.08838834764831845f, approx_exp.
// Pass 1 takes the max with the reference's `new > old` rule (any order gives the same value).
// Pass 2 walks the keys in ascending order in chunks of 128: lane j computes e for key base+j,
// lane 0 adds the denominators serially and lane d adds e*v[d] serially, so every sum keeps the
// reference order.  The score is recomputed in pass 2 exactly as the reference does.
// q: [tokens][1536]; cache of token b at k_cache + b*cache_stride (decode) or shared (prefill).
// Decode key counts are clamped to max_keys (the cache rows the caller sized).
// ---------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(128) attention_ordered_kernel(const float* __restrict__ q,
                                                                const float* __restrict__ k_cache,
                                                                const float* __restrict__ v_cache, size_t cache_stride,
                                                                const int* __restrict__ pos, int max_keys, int prefill,
                                                                int past, float* __restrict__ ctx) {
  __shared__ float qs[QWEN_HEAD_DIM];
  __shared__ float es[128];
  __shared__ float red[128];
  __shared__ float den_s;
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int tid = threadIdx.x;
  const int kvh = h / QWEN_GROUPS;
  const int n = prefill ? past + b + 1 : min(max(pos[b], 0) + 1, max_keys);
  // Decode's (float)(1.0/sqrt(128.0)) and prefill's 0.08838834764831845f are the same float
  // (bits 0x3db504f3; checked by tests/test_oracle_math.py).
  const float scaling = 0.08838834764831845f;
  const float* kc = k_cache + (prefill ? 0 : (size_t)b * cache_stride) + kvh * QWEN_HEAD_DIM;
  const float* vc = v_cache + (prefill ? 0 : (size_t)b * cache_stride) + kvh * QWEN_HEAD_DIM;
  qs[tid] = q[(size_t)b * QWEN_HIDDEN + h * QWEN_HEAD_DIM + tid];
  __syncthreads();

  float m = -1.0e30f;
  for (int t = tid; t < n; t += 128) {
    const float* kr = kc + (size_t)t * QWEN_KV_WIDTH;
    float score = 0.0f;
    for (int d = 0; d < QWEN_HEAD_DIM; ++d) score += qs[d] * kr[d];
    const float sc = score * scaling;
    m = sc > m ? sc : m;
  }
  red[tid] = m;
  __syncthreads();
  for (int stride = 64; stride > 0; stride >>= 1) {
    if (tid < stride) {
      const float o = red[tid + stride];
      red[tid] = o > red[tid] ? o : red[tid];
    }
    __syncthreads();
  }
  m = red[0];

  float den = 0.0f;
  float acc = 0.0f;
  for (int base = 0; base < n; base += 128) {
    const int t = base + tid;
    if (t < n) {
      const float* kr = kc + (size_t)t * QWEN_KV_WIDTH;
      float score = 0.0f;
      for (int d = 0; d < QWEN_HEAD_DIM; ++d) score += qs[d] * kr[d];
      const float arg = score * scaling - m;
      es[tid] = prefill ? approx_exp(arg) : glibc_expf(arg);
    }
    __syncthreads();
    const int cnt = min(128, n - base);
    if (tid == 0)
      for (int j = 0; j < cnt; ++j) den += es[j];
    for (int j = 0; j < cnt; ++j) acc += es[j] * vc[(size_t)(base + j) * QWEN_KV_WIDTH + tid];
    __syncthreads();
  }
  if (tid == 0) den_s = den;
  __syncthreads();
  const float dv = den_s;
  const float inv = dv > 0.0f ? 1.0f / dv : 0.0f;
  ctx[(size_t)b * QWEN_HIDDEN + h * QWEN_HEAD_DIM + tid] = acc * inv;
}

// ---------------------------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------------------------
void launch_rmsnorm_ordered(const float* x, const float* w, float* y, int tokens, bool prefill, hipStream_t st) {
  hipLaunchKernelGGL(rmsnorm_ordered_kernel, dim3(tokens), dim3(256), 0, st, x, w, y, prefill ? 1 : 0);
}

void launch_project_ordered(const float* x, int tokens, int in_dim, const uint8_t* W, const float* scale,
                            const float* bias, int out_dim, float* y, const float* residual, hipStream_t st) {
  const unsigned gx = (unsigned)((out_dim + kOrdRows - 1) / kOrdRows);
  if (tokens >= 8) {
    hipLaunchKernelGGL(project_ordered_kernel<8>, dim3(gx, (tokens + 7) / 8), dim3(256), 0, st, x, tokens, in_dim, W,
                       scale, bias, out_dim, y, residual);
  } else {
    hipLaunchKernelGGL(project_ordered_kernel<1>, dim3(gx, tokens), dim3(256), 0, st, x, tokens, in_dim, W, scale,
                       bias, out_dim, y, residual);
  }
}

void launch_silu_mul(const float* g, const float* u, float* s, size_t n, bool prefill, hipStream_t st) {
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, g, u, s, n,
                     prefill ? 1 : 0);
}

void launch_rope_append_decode(float* q, const float* k, const float* v, const int* pos, const float* rope,
                               bool rope_rows_are_tokens, float* k_cache, float* v_cache, size_t cache_stride,
                               int max_keys, int tokens, hipStream_t st) {
  hipLaunchKernelGGL(rope_append_decode_kernel, dim3(tokens), dim3(64), 0, st, q, k, v, pos, rope,
                     rope_rows_are_tokens ? 1 : 0, k_cache, v_cache, cache_stride, max_keys);
}

void launch_rope_prefill(float* q, float* k_rows, const float* rope, int tokens, hipStream_t st) {
  hipLaunchKernelGGL(rope_prefill_kernel, dim3(tokens), dim3(64), 0, st, q, k_rows, rope);
}

void launch_rope_table_prefill(float* rope, int first, int count, hipStream_t st) {
  const int n = count * 64;
  hipLaunchKernelGGL(rope_table_prefill_kernel, dim3((n + 255) / 256), dim3(256), 0, st, rope, first, count);
}

void launch_attention_ordered(const float* q, const float* k_cache, const float* v_cache, size_t cache_stride,
                              const int* pos, int max_keys, int tokens, bool prefill, int past, float* ctx,
                              hipStream_t st) {
  hipLaunchKernelGGL(attention_ordered_kernel, dim3(QWEN_Q_HEADS, tokens), dim3(128), 0, st, q, k_cache, v_cache,
                     cache_stride, pos, max_keys, prefill ? 1 : 0, past, ctx);
}

}  // namespace qwen
