// FAST kernels: the roofline-oriented path (gfx950 / CDNA4).
//
// These kernels compute the same layer as the reference (qwen_decode_*_kernel.cpp,
// qwen_prefill_*_kernel.cpp host branch) but reorder every fp32 reduction, so their results
// agree with the reference to a relative tolerance instead of bit for bit:
//   * INT4 projections run on the int8 matrix cores (v_mfma_i32_16x16x64_i8).  Weights are
//     repacked once into a lane-contiguous tile layout (each wave streams 1 KiB contiguous per
//     128-wide K chunk) and enter the MFMA as q+8 in [0,15].  Activations are quantized per token
//     into two int8 limbs X = 256*H + L with |X| <= 32512 (15 bits), so both limb products are
//     accumulated exactly in int32; the row scale, the token scale and the -8*sum(X) offset
//     correction are applied once after the K reduction.
//   * Decode attention is split over the KV length (flash-decoding): one block per
//     (KV chunk, KV head, sequence) streams each K/V row once for all 6 query heads of its group.
//   * Prefill attention is a causal online-softmax kernel over LDS-staged K/V tiles.
// Elementwise nonlinearities keep the reference's functions (host-compatible expf for decode
// SiLU, approx_exp for prefill softmax and SiLU), so the tolerance only has to absorb reordering
// and the 15-bit activation quantization.
#include <hip/hip_runtime.h>

#include <stdexcept>
#include <type_traits>

#include "kernels.hpp"
#include "qwen_device_math.hpp"

namespace qwen {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Streaming (non-temporal) loads: data read once per launch should not displace reused lines.
__device__ __forceinline__ uint4 ld_stream(const uint4* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ float4 ld_stream(const float4* p) {
  const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
  return make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ float2 ld_stream(const float2* p) {
  const f32x2 v = __builtin_nontemporal_load(reinterpret_cast<const f32x2*>(p));
  return make_float2(v[0], v[1]);
}

// Prefill SiLU for the FAST GEMM epilogue: v / (1 + e(-v)) with the division as v * rcp(1 + e)
// (v_rcp_f32, 1 ulp).  For s = -v >= -1 the reference's approx_exp is its degree-6 Taylor series
// (qwen_prefill_mlp_kernel.cpp:158-181, no halving), kept here in Horner form (a few ulp from the
// term recurrence); below -1 the reference halves s, evaluates the series and squares back, which is
// within 5e-4 x 2^k of exp(s) after k halvings, and the hardware exp (v_exp_f32) replaces that ladder
// (20 VALU operations fewer per output).  SiLU values then differ from silu_prefill by at most
// 1.2e-4 relative (largest near v = 2, where exp(-v) still matters), below 1.3e-6 for v >= 8 and
// below 5e-7 for v < 0 (a sweep of 600,000 inputs over [-40, 40] against the reference form).
__device__ __forceinline__ float silu_prefill_fast(float v) {
  const float s = -v;
  const float t6 = 1.0f + s * (1.0f + s * (0.5f + s * (1.0f / 6.0f + s * (1.0f / 24.0f + s * (1.0f / 120.0f +
                                                                                            s * (1.0f / 720.0f))))));
  // both forms are evaluated and one is selected, so the lanes of a wave do not branch apart (the
  // hardware exp of the other form is finite or +inf and discarded)
  const float ex = __expf(s);
  const float e = s < -1.0f ? ex : t6;
  return v * __builtin_amdgcn_rcpf(1.0f + e);
}

// ---------------------------------------------------------------------------------------------
// Weight repack.  Reference layout: W[o][i] is the nibble at byte (o*in + i)/2, low nibble for
// an even flat index, value q in [-8,7] stored as q & 15 (qwen_decode_attention_kernel.cpp:44-60).
// Tile layout: [out/16 row tiles][in/128 K chunks][64 lanes][16 bytes].  Lane l covers row
// 16*rt + (l & 15) and K = 128*kc + 32*(l >> 4) + [0, 32).  Inside the 16 bytes, 32-bit word w
// covers K 8w..8w+7 of that range: byte b holds K 8w+b in its low nibble and K 8w+4+b in its high
// nibble, each stored as q + 8.  Unpacking word w as (w & 0x0F0F0F0F, (w >> 4) & 0x0F0F0F0F)
// then yields 8 int8 values in natural K order.
// grid = (out/16, in/128), block = 64.
// ---------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(64) repack_int4_kernel(const uint8_t* __restrict__ W, int in_dim,
                                                         uint8_t* __restrict__ WP) {
  const int rt = blockIdx.x;
  const int kc = blockIdx.y;
  const int l = threadIdx.x;
  const int row = rt * 16 + (l & 15);
  const int kbase = kc * kKChunk + 32 * (l >> 4);
  const uint8_t* src = W + (size_t)row * (size_t)(in_dim / 2);
  uint32_t words[4];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    uint32_t word = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int klo = kbase + 8 * w + b;
      const int khi = klo + 4;
      const uint32_t blo = src[klo >> 1];
      const uint32_t bhi = src[khi >> 1];
      const uint32_t nlo = (klo & 1) ? (blo >> 4) : (blo & 0xFu);
      const uint32_t nhi = (khi & 1) ? (bhi >> 4) : (bhi & 0xFu);
      word |= (((nlo ^ 8u) & 0xFu) | (((nhi ^ 8u) & 0xFu) << 4)) << (8 * b);
    }
    words[w] = word;
  }
  const size_t dst = (((size_t)rt * (size_t)(in_dim / kKChunk) + (size_t)kc) * 64u + (size_t)l) * 16u;
  *reinterpret_cast<uint4*>(WP + dst) = make_uint4(words[0], words[1], words[2], words[3]);
}

// ---------------------------------------------------------------------------------------------
// Block reductions (256 threads = 4 waves of 64).
// ---------------------------------------------------------------------------------------------
// Max and integer sum do not depend on the order of the operations, so they reduce each row of 16
// lanes with DPP moves (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_ror:4, row_ror:8: every lane
// ends with its row's result) and combine the four rows from v_readlane, instead of six LDS
// permutes.  Float sums keep the xor butterfly (the prefill norm's rounding follows that order); the
// double sum of the decode RMSNorm takes the DPP order (another rounding of an f64 sum of squares).
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, __int_as_float(dpp_i<0xB1>(__float_as_int(v))));
  v = fmaxf(v, __int_as_float(dpp_i<0x4E>(__float_as_int(v))));
  v = fmaxf(v, __int_as_float(dpp_i<0x124>(__float_as_int(v))));
  v = fmaxf(v, __int_as_float(dpp_i<0x128>(__float_as_int(v))));
  const int b = __float_as_int(v);
  return fmaxf(fmaxf(__int_as_float(__builtin_amdgcn_readlane(b, 0)), __int_as_float(__builtin_amdgcn_readlane(b, 16))),
               fmaxf(__int_as_float(__builtin_amdgcn_readlane(b, 32)), __int_as_float(__builtin_amdgcn_readlane(b, 48))));
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const int lo = dpp_i<CTRL>((int)(uint32_t)u), hi = dpp_i<CTRL>((int)(uint32_t)(u >> 32));
  return __builtin_bit_cast(double, ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}
__device__ __forceinline__ double readlane_d(double v, int l) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)u, l), hi = __builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), l);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
// wave_sum_i's order (pairs, quads, rows of 16 by DPP, then the four rows) on doubles.
__device__ __forceinline__ double wave_sum_d(double v) {
  v += dpp_d<0xB1>(v);
  v += dpp_d<0x4E>(v);
  v += dpp_d<0x124>(v);
  v += dpp_d<0x128>(v);
  return (readlane_d(v, 0) + readlane_d(v, 16)) + (readlane_d(v, 32) + readlane_d(v, 48));
}
__device__ __forceinline__ int wave_sum_i(int v) {
  v += dpp_i<0xB1>(v);
  v += dpp_i<0x4E>(v);
  v += dpp_i<0x124>(v);
  v += dpp_i<0x128>(v);
  return (__builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16)) +
         (__builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48));
}

// Reductions over the 4 waves of a 256-thread block; every thread receives the result.
__device__ __forceinline__ float block_max4(float v, float* s4) {
  v = wave_max(v);
  if ((threadIdx.x & 63) == 0) s4[threadIdx.x >> 6] = v;
  __syncthreads();
  const float r = fmaxf(fmaxf(s4[0], s4[1]), fmaxf(s4[2], s4[3]));
  __syncthreads();
  return r;
}
__device__ __forceinline__ double block_sum4_d(double v, double* s4) {
  v = wave_sum_d(v);
  if ((threadIdx.x & 63) == 0) s4[threadIdx.x >> 6] = v;
  __syncthreads();
  const double r = (s4[0] + s4[1]) + (s4[2] + s4[3]);
  __syncthreads();
  return r;
}
__device__ __forceinline__ float block_sum4(float v, float* s4) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) s4[threadIdx.x >> 6] = v;
  __syncthreads();
  const float r = (s4[0] + s4[1]) + (s4[2] + s4[3]);
  __syncthreads();
  return r;
}
__device__ __forceinline__ int block_sum4_i(int v, int* s4) {
  v = wave_sum_i(v);
  if ((threadIdx.x & 63) == 0) s4[threadIdx.x >> 6] = v;
  __syncthreads();
  const int r = (s4[0] + s4[1]) + (s4[2] + s4[3]);
  __syncthreads();
  return r;
}
// Two integer sums in one round (s8: 8 ints of LDS).
__device__ __forceinline__ void block_sum4_i2(int& a, int& b, int* s8) {
  a = wave_sum_i(a);
  b = wave_sum_i(b);
  if ((threadIdx.x & 63) == 0) {
    s8[threadIdx.x >> 6] = a;
    s8[4 + (threadIdx.x >> 6)] = b;
  }
  __syncthreads();
  a = (s8[0] + s8[1]) + (s8[2] + s8[3]);
  b = (s8[4] + s8[5]) + (s8[6] + s8[7]);
  __syncthreads();
}
// The two sums of a 256-thread block from per-wave partials in LDS (w[2v], w[2v + 1]: wave v's), read
// after a barrier that follows their writes: the one-token prologues leave them so, and the barrier
// that publishes their activation slice also publishes the sums, one barrier fewer on the launch's
// critical path (the sums are first needed in the epilogue).
__device__ __forceinline__ int2 wave_sums_total(const int* w) {
  return make_int2((w[0] + w[2]) + (w[4] + w[6]), (w[1] + w[3]) + (w[5] + w[7]));
}

// ---------------------------------------------------------------------------------------------
// Two-limb activation quantization of one row held in LDS (n values, n % 128 == 0), done by a
// 256-thread block.  Writes the limbs in the GEMM's layout ([K chunk][limb][128 bytes] per row),
// the token scale and the two limb sums.
// ---------------------------------------------------------------------------------------------
__device__ void quantize_row_lds(const float* __restrict__ v, int n, int8_t* __restrict__ xq_row,
                                 float* __restrict__ sx_out, int* __restrict__ sums_out, float* red_f, int* red_i,
                                 int chunk_stride = 256) {
  float amax = 0.0f;
  for (int k = threadIdx.x; k < n; k += 256) amax = fmaxf(amax, fabsf(v[k]));
  amax = block_max4(amax, red_f);
  const float sx = amax > 0.0f ? amax / (float)kQuantMax : 1.0f;
  const float inv = amax > 0.0f ? (float)kQuantMax / amax : 0.0f;
  int sh = 0, sl = 0;
  for (int k = threadIdx.x; k < n; k += 256) {
    float xf = rintf(v[k] * inv);
    xf = fminf(fmaxf(xf, -(float)kQuantMax), (float)kQuantMax);
    const int X = (int)xf;
    const int H = (X + 128) >> 8;
    const int L = X - (H << 8);
    const int chunk = k >> 7;
    const int within = k & 127;
    xq_row[chunk * chunk_stride + within] = (int8_t)H;
    xq_row[chunk * chunk_stride + 128 + within] = (int8_t)L;
    sh += H;
    sl += L;
  }
  block_sum4_i2(sh, sl, red_i);
  if (threadIdx.x == 0) {
    *sx_out = sx;
    sums_out[0] = sh;
    sums_out[1] = sl;
  }
}

// ---------------------------------------------------------------------------------------------
// RMSNorm (optional) + quantization of one token row held by a 256-thread block as float4 v[j] at
// float4 index threadIdx.x + 256*j (n % 128 == 0, n <= 1024*NV):
//   kNormDecode: decode rmsnorm (double mean square, qwen_decode_attention_kernel.cpp:13-27)
//   kNormPrefill: prefill rmsnorm (float, approx_sqrt, qwen_prefill_attention_kernel.cpp:112-126)
//   kNormNone: quantize the row as is.
// Writes the two-limb code ([K chunk][limb][128 bytes]), the token scale and the limb sums, and
// optionally the normalized fp32 row (xn_row).
// ---------------------------------------------------------------------------------------------
template <int NV>
__device__ __forceinline__ void norm_quant_row(float4 (&v)[NV], int n, const float* __restrict__ w, int norm,
                                               int8_t* __restrict__ row, float* __restrict__ sx_out,
                                               int* __restrict__ sums_out, float* __restrict__ xn_row) {
  __shared__ float red_f[4];
  __shared__ double red_d[4];
  __shared__ int red_i[8];
  const int n4 = n >> 2;
  if (norm == kNormDecode) {
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < NV; ++j)
      ss += (double)v[j].x * v[j].x + (double)v[j].y * v[j].y + (double)v[j].z * v[j].z + (double)v[j].w * v[j].w;
    ss = block_sum4_d(ss, red_d);
    const double inv = 1.0 / sqrt(ss / (double)n + (double)QWEN_RMS_EPS);
    const float4* w4 = reinterpret_cast<const float4*>(w);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int k = threadIdx.x + 256 * j;
      if (k < n4) {
        const float4 ww = w4[k];
        v[j] = make_float4((float)((double)v[j].x * inv * ww.x), (float)((double)v[j].y * inv * ww.y),
                           (float)((double)v[j].z * inv * ww.z), (float)((double)v[j].w * inv * ww.w));
      }
    }
  } else if (norm == kNormPrefill) {
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) ss += v[j].x * v[j].x + v[j].y * v[j].y + v[j].z * v[j].z + v[j].w * v[j].w;
    ss = block_sum4(ss, red_f);
    const float inv = 1.0f / approx_sqrt(ss / (float)n + QWEN_RMS_EPS);
    const float4* w4 = reinterpret_cast<const float4*>(w);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int k = threadIdx.x + 256 * j;
      if (k < n4) {
        const float4 ww = w4[k];
        v[j] = make_float4(v[j].x * inv * ww.x, v[j].y * inv * ww.y, v[j].z * inv * ww.z, v[j].w * inv * ww.w);
      }
    }
  }
  if (xn_row) {
    float4* xo = reinterpret_cast<float4*>(xn_row);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int k = threadIdx.x + 256 * j;
      if (k < n4) xo[k] = v[j];
    }
  }
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j)
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
  amax = block_max4(amax, red_f);
  const float inv = amax > 0.0f ? (float)kQuantMax / amax : 0.0f;
  int sh = 0, sl = 0;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int k = threadIdx.x + 256 * j;
    if (k < n4) {
      const float e[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
      uint32_t hw = 0, lw = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float xf = fminf(fmaxf(rintf(e[q] * inv), -(float)kQuantMax), (float)kQuantMax);
        const int X = (int)xf;
        const int H = (X + 128) >> 8;
        const int L = X - (H << 8);
        hw |= (uint32_t)(H & 0xFF) << (8 * q);
        lw |= (uint32_t)(L & 0xFF) << (8 * q);
        sh += H;
        sl += L;
      }
      const int base = ((4 * k) >> 7) * 256 + ((4 * k) & 127);
      *reinterpret_cast<uint32_t*>(row + base) = hw;
      *reinterpret_cast<uint32_t*>(row + base + 128) = lw;
    }
  }
  block_sum4_i2(sh, sl, red_i);
  if (threadIdx.x == 0) {
    *sx_out = amax > 0.0f ? amax / (float)kQuantMax : 1.0f;
    sums_out[0] = sh;
    sums_out[1] = sl;
  }
}

// One block per token row: loads x[t] and runs norm_quant_row.  grid = rows, block = 256.
constexpr int kQuantVecs = (kMaxQuantRow / 4 + 255) / 256;  // float4 per thread for the widest row

template <int NV>
__global__ void __launch_bounds__(256) norm_quant_kernel(const float* __restrict__ x, size_t x_stride, int n,
                                                         const float* __restrict__ w, int norm,
                                                         int8_t* __restrict__ xq, float* __restrict__ sx,
                                                         int* __restrict__ sums, float* __restrict__ xn) {
  const int t = blockIdx.x;
  const int n4 = n >> 2;
  const float4* xr = reinterpret_cast<const float4*>(x + (size_t)t * x_stride);
  float4 v[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int k = threadIdx.x + 256 * j;
    v[j] = k < n4 ? xr[k] : make_float4(0, 0, 0, 0);
  }
  norm_quant_row<NV>(v, n, w, norm, xq + (size_t)t * (size_t)(2 * n), sx + t, sums + 2 * t,
                     xn ? xn + (size_t)t * n : nullptr);
}

// Many-row two-limb quantization (prefill rows of 1,536 or 8,960): one wave per row with NV float4 per
// lane (n = 256*NV), the whole row loaded at once with non-temporal loads (each value is read once),
// wave reductions only (no LDS, no barrier), and each store instruction writing two whole 128-byte
// limb segments.  The values equal norm_quant_row's for kNormNone (the maximum and the integer limb
// sums do not depend on the order of the reduction); for kNormPrefill the sum of squares is added in
// another order, a different fp32 rounding of the same sum.  grid = ceil(rows / 4), block = 256.
template <int NV>
__global__ void __launch_bounds__(256) quant_rows_wave_kernel(const float* __restrict__ x, size_t x_stride,
                                                              int rows, const float* __restrict__ w, int norm,
                                                              int8_t* __restrict__ xq, float* __restrict__ sx,
                                                              int* __restrict__ sums) {
  constexpr int n = 256 * NV;
  const int lane = threadIdx.x & 63;
  const int t = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  if (t >= rows) return;  // wave-uniform
  const float4* xr = reinterpret_cast<const float4*>(x + (size_t)t * x_stride);
  float4 v[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) v[j] = ld_stream(xr + lane + 64 * j);
  if (norm == kNormPrefill) {
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) ss += v[j].x * v[j].x + v[j].y * v[j].y + v[j].z * v[j].z + v[j].w * v[j].w;
    ss = wave_sum(ss);
    const float inv = 1.0f / approx_sqrt(ss / (float)n + QWEN_RMS_EPS);
    const float4* w4 = reinterpret_cast<const float4*>(w);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const float4 ww = w4[lane + 64 * j];
      v[j] = make_float4(v[j].x * inv * ww.x, v[j].y * inv * ww.y, v[j].z * inv * ww.z, v[j].w * inv * ww.w);
    }
  }
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j)
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
  amax = wave_max(amax);
  const float inv = amax > 0.0f ? (float)kQuantMax / amax : 0.0f;
  int8_t* row = xq + (size_t)t * (size_t)(2 * n);
  int sh = 0, sl = 0;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int k = lane + 64 * j;  // float4 index: elements 4k .. 4k+3 of K chunk k / 32
    const float e[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
    uint32_t hw = 0, lw = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float xf = fminf(fmaxf(rintf(e[q] * inv), -(float)kQuantMax), (float)kQuantMax);
      const int X = (int)xf;
      const int H = (X + 128) >> 8;
      const int L = X - (H << 8);
      hw |= (uint32_t)(H & 0xFF) << (8 * q);
      lw |= (uint32_t)(L & 0xFF) << (8 * q);
      sh += H;
      sl += L;
    }
    const int base = (k >> 5) * 256 + (k & 31) * 4;
    *reinterpret_cast<uint32_t*>(row + base) = hw;
    *reinterpret_cast<uint32_t*>(row + base + 128) = lw;
  }
  sh = wave_sum_i(sh);
  sl = wave_sum_i(sl);
  if (lane == 0) {
    sx[t] = amax > 0.0f ? amax / (float)kQuantMax : 1.0f;
    sums[2 * t] = sh;
    sums[2 * t + 1] = sl;
  }
}

// ---------------------------------------------------------------------------------------------
// INT4 x two-limb int8 GEMM on the matrix cores:
//   y[t][o] = sw[o] * sx[t] * ( 256*(sum_k u(o,k) H(t,k) - 8 SH(t)) + (sum_k u(o,k) L(t,k) - 8 SL(t)) )
// with u = q + 8.  A block has 4 waves.  KSPLIT waves share one 16-row tile and split its K
// chunks (their int32 partial sums are added through LDS, exact); 4/KSPLIT row tiles per block.
// Each wave covers NT column tiles of 16 tokens.  DUAL runs a second weight matrix over the same
// activations (gate and up).  grid = (ceil(tokens / (16*NT)), out/16 / (4/KSPLIT)).
// MFMA lane mapping (16x16 output tile): A row = lane & 15, B column = lane & 15, both taking
// the same 16 K values per lane group (lane >> 4); D holds rows 4*(lane>>4)+r, column lane & 15.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ void unpack16(const uint4 w, v4i& a1, v4i& a2) {
  const uint32_t m = 0x0F0F0F0Fu;
  a1[0] = (int)(w.x & m);
  a1[1] = (int)((w.x >> 4) & m);
  a1[2] = (int)(w.y & m);
  a1[3] = (int)((w.y >> 4) & m);
  a2[0] = (int)(w.z & m);
  a2[1] = (int)((w.z >> 4) & m);
  a2[2] = (int)(w.w & m);
  a2[3] = (int)((w.w >> 4) & m);
}

template <int NT, int KSPLIT, bool DUAL>
struct GemmAcc {
  v4i h[NT], l[NT];
  v4i h2[DUAL ? NT : 1], l2[DUAL ? NT : 1];
};

template <int NT, int KSPLIT, int EPI, bool DUAL>
__global__ void __launch_bounds__(256) gemm_i8_kernel(GemmArgs a) {
  constexpr int RTB = 4 / KSPLIT;  // row tiles per block
  constexpr int NACC = NT * 8 * (DUAL ? 2 : 1);  // int32 accumulators per lane
  __shared__ int red[KSPLIT > 1 ? (KSPLIT - 1) * 64 * NACC : 1];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int rt = blockIdx.y * RTB + wave / KSPLIT;
  const int ks = wave % KSPLIT;
  const int row_tiles = a.out_dim / 16;
  const bool rt_ok = rt < row_tiles;
  const int nkc = a.in_dim / kKChunk;
  const int tok0 = blockIdx.x * (16 * NT);
  const int g = lane >> 4;
  const int col = lane & 15;

  v4i accH[NT], accL[NT], accH2[NT], accL2[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    accH[n] = v4i{0, 0, 0, 0};
    accL[n] = v4i{0, 0, 0, 0};
    accH2[n] = v4i{0, 0, 0, 0};
    accL2[n] = v4i{0, 0, 0, 0};
  }

  // K chunks of this wave: [kc_begin, kc_end)
  const int per = (nkc + KSPLIT - 1) / KSPLIT;
  const int kc_begin = min(nkc, ks * per);
  const int kc_end = min(nkc, kc_begin + per);
  const size_t row_stride_x = (size_t)a.in_dim * 2u;  // bytes per token row of limbs

  if (rt_ok) {
    const uint4* wp = reinterpret_cast<const uint4*>(a.wp) + ((size_t)rt * nkc) * 64u + lane;
    const uint4* wp2 = DUAL ? reinterpret_cast<const uint4*>(a.wp2) + ((size_t)rt * nkc) * 64u + lane : nullptr;
    const int8_t* xbase[NT];
    bool tok_ok[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      const int tok = tok0 + n * 16 + col;
      tok_ok[n] = tok < a.tokens;
      xbase[n] = a.xq + (size_t)(tok_ok[n] ? tok : 0) * row_stride_x + 32 * g;
    }
    constexpr int U = 4;
    for (int kc0 = kc_begin; kc0 < kc_end; kc0 += U) {
      uint4 wv[U], wv2[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int kc = kc0 + u;
        wv[u] = kc < kc_end ? ld_stream(wp + (size_t)kc * 64u) : make_uint4(0, 0, 0, 0);
        if (DUAL) wv2[u] = kc < kc_end ? ld_stream(wp2 + (size_t)kc * 64u) : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int kc = kc0 + u;
        if (kc >= kc_end) break;
        v4i a1, a2, c1, c2;
        unpack16(wv[u], a1, a2);
        if (DUAL) unpack16(wv2[u], c1, c2);
#pragma unroll
        for (int n = 0; n < NT; ++n) {
          v4i bh1 = v4i{0, 0, 0, 0}, bh2 = bh1, bl1 = bh1, bl2 = bh1;
          if (tok_ok[n]) {
            const v4i* p = reinterpret_cast<const v4i*>(xbase[n] + (size_t)kc * 256u);
            bh1 = p[0];
            bh2 = p[1];
            bl1 = p[8];
            bl2 = p[9];
          }
          accH[n] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, bh1, accH[n], 0, 0, 0);
          accH[n] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a2, bh2, accH[n], 0, 0, 0);
          accL[n] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, bl1, accL[n], 0, 0, 0);
          accL[n] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a2, bl2, accL[n], 0, 0, 0);
          if (DUAL) {
            accH2[n] = __builtin_amdgcn_mfma_i32_16x16x64_i8(c1, bh1, accH2[n], 0, 0, 0);
            accH2[n] = __builtin_amdgcn_mfma_i32_16x16x64_i8(c2, bh2, accH2[n], 0, 0, 0);
            accL2[n] = __builtin_amdgcn_mfma_i32_16x16x64_i8(c1, bl1, accL2[n], 0, 0, 0);
            accL2[n] = __builtin_amdgcn_mfma_i32_16x16x64_i8(c2, bl2, accL2[n], 0, 0, 0);
          }
        }
      }
    }
  }

  if (KSPLIT > 1) {
    // Waves ks = 1..KSPLIT-1 of each row tile hand their partial sums to wave ks = 0 (exact int32).
    // RTB == 1 whenever KSPLIT > 1, so the block holds one row tile.
    if (ks > 0) {
      int* dst = red + ((ks - 1) * NACC) * 64 + lane;
      int idx = 0;
#pragma unroll
      for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          dst[(idx++) * 64] = accH[n][r];
          dst[(idx++) * 64] = accL[n][r];
          if (DUAL) {
            dst[(idx++) * 64] = accH2[n][r];
            dst[(idx++) * 64] = accL2[n][r];
          }
        }
    }
    __syncthreads();
    if (ks > 0) return;
#pragma unroll
    for (int s = 0; s < KSPLIT - 1; ++s) {
      const int* src = red + (s * NACC) * 64 + lane;
      int idx = 0;
#pragma unroll
      for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          accH[n][r] += src[(idx++) * 64];
          accL[n][r] += src[(idx++) * 64];
          if (DUAL) {
            accH2[n][r] += src[(idx++) * 64];
            accL2[n][r] += src[(idx++) * 64];
          }
        }
    }
  }
  if (!rt_ok) return;

  // Epilogue: lane holds rows row0..row0+3 of token column `col` of each column tile.
  const int row0 = rt * 16 + 4 * g;
  if (!DUAL && a.fuse != kFuseNone) {
    // fused reduce follows: fp32 partials sw*sx*(256*sumH + sumL) into split 0 of a.part
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      const int tok = tok0 + n * 16 + col;
      if (tok >= a.tokens) continue;
      const double sx = (double)a.sx[tok];
      float out[4];
#pragma unroll
      for (int r = 0; r < 4; ++r)
        out[r] = (float)(((double)accH[n][r] * 256.0 + (double)accL[n][r]) * sx) * a.sw[row0 + r];
      *reinterpret_cast<float4*>(a.part + (size_t)tok * a.out_dim + row0) = make_float4(out[0], out[1], out[2], out[3]);
    }
    return;
  }
  float sw[4], sw2[4], bias[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    sw[r] = a.sw[row0 + r];
    sw2[r] = DUAL ? a.sw2[row0 + r] : 0.0f;
    bias[r] = a.bias ? a.bias[row0 + r] : 0.0f;
  }
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const int tok = tok0 + n * 16 + col;
    if (tok >= a.tokens) continue;
    const double sx = (double)a.sx[tok];
    const int sh8 = 8 * a.sums[2 * tok];
    const int sl8 = 8 * a.sums[2 * tok + 1];
    float out[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const double tot = (double)(accH[n][r] - sh8) * 256.0 + (double)(accL[n][r] - sl8);
      const float v = (float)(tot * sx) * sw[r];
      if (EPI == kEpiSiluMul) {
        const double tot2 = (double)(accH2[n][r] - sh8) * 256.0 + (double)(accL2[n][r] - sl8);
        const float u = (float)(tot2 * sx) * sw2[r];
        const float sg = a.prefill_silu ? silu_prefill(v) : silu_decode(v);
        out[r] = sg * u;
      } else if (EPI == kEpiResidual) {
        const float o = a.resid[(size_t)tok * a.resid_stride + row0 + r] + v;
        out[r] = o;
      } else {
        out[r] = v + bias[r];
      }
    }
    float* yp = a.y + (size_t)tok * a.y_stride + row0;
    if (EPI == kEpiResidual && a.y_raw) {
      float* rp = a.y_raw + (size_t)tok * a.y_stride + row0;
      *reinterpret_cast<float4*>(rp) = make_float4(out[0], out[1], out[2], out[3]);
    }
    if (EPI == kEpiResidual && a.round_bf16)
#pragma unroll
      for (int r = 0; r < 4; ++r) out[r] = round_bf16(out[r]);
    *reinterpret_cast<float4*>(yp) = make_float4(out[0], out[1], out[2], out[3]);
  }
}

// ---------------------------------------------------------------------------------------------
// Pipelined many-token GEMM.  Both operands of every K chunk reach LDS through direct
// global->LDS loads (global_load_lds_dwordx4, 16 bytes per lane, no VGPR round trip), NBUF
// chunks deep, so one wave keeps NBUF-1 chunks in flight while the matrix cores consume the
// oldest.  With NBUF = 2 a block's next chunk lands during its current one, and two blocks share
// the CU (WPE = 2 caps a wave at 256 VGPRs, two waves per SIMD): each block's epilogue and load
// waits then run beside the other block's MFMAs.  Per chunk and wave: NT loads of activation rows (the block's TOK rows are split over
// the 4 waves, 4 rows of 256 bytes per load) and RTW*D loads of the wave's own weight tiles.
// Activation rows are XOR-swizzled by 16-byte segment (LDS segment s holds global segment
// s ^ (row & 15)), so the 16 lanes of a lane group read 16 token rows on 16 distinct bank groups.
// Every vector-memory instruction of the loop is one of these loads, issued in chunk order, so
// `s_waitcnt vmcnt(n)` with n = loads issued after chunk i is exactly "chunk i has landed"; a
// barrier then makes every wave's part visible and frees the buffer refilled next.
// gridDim.z > 1 splits the K chunks over blocks: each block writes fp32 partials
// sw*sx*(256*sumH + sumL) of its chunks to a.part[z][tok][row], and gemm_splitk_reduce_kernel adds
// them in z order, applies the -8*sum(X) correction and the epilogue.
// grid = (ceil(tokens/(16*NT)), ceil(row_tiles/(4*RTW)), splits), block = 256.
// ---------------------------------------------------------------------------------------------
template <int VMCNT>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(VMCNT >= 0 && VMCNT < 64, "vmcnt out of range");
  // gfx9 s_waitcnt: vmcnt[3:0] | expcnt[6:4] (7 = no wait) | lgkmcnt[11:8] (15 = no wait) | vmcnt[5:4] << 14
  __builtin_amdgcn_s_waitcnt((VMCNT & 0xF) | (0x7 << 4) | (0xF << 8) | ((VMCNT >> 4) << 14));
}

// A uniform int read through the scalar cache, waited for with lgkmcnt (the vector loads in flight
// are not waited for).  p must be uniform across the wave.
__device__ __forceinline__ int load_uniform_i32(const int* p) {
  int v;
  asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p));
  return v;
}

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
// 16-byte LDS read issued as is: the result may only be used after an lgkm_wait_tie covering it.
__device__ __forceinline__ v4i lds_read_b128(uint32_t addr) {
  v4i r;
  asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(addr) : "memory");
  return r;
}
// Waits until at most N LDS reads are outstanding; the tied registers are the ones this makes valid.
template <int N>
__device__ __forceinline__ void lgkm_wait_tie(v4i& a, v4i& b, v4i& c, v4i& d) {
  asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d) : "i"(N) : "memory");
}
// Orders later uses of r after the preceding waits (no instruction).
__device__ __forceinline__ void reg_tie(v4i& r) { asm volatile("" : "+v"(r)); }

constexpr int kRasterGroup = 8;  // token tiles per raster group of the pipelined GEMM

// Epilogue forms of the pipelined GEMM, fixed per kernel instance by the launcher.
//   kEfPrefillSilu: the SiLU of the gate/up epilogue is the prefill one (silu_prefill_fast); otherwise
//                   the decode one (silu_decode).
//   kEfIntSum:      the two limb sums and their zero-point terms are combined in 32-bit integers,
//                   256 (sum uH - 8 sum H) + (sum uL - 8 sum L) = sum q X, then converted once.  The
//                   result is exact for in_dim <= kIntSumMaxK (|q X| <= 8 * 32512 per term, so the sum fits
//                   in int32 and the modular intermediates do not matter), and its one rounding equals
//                   that of the fp32 form, whose two limb terms are exact before the one fma rounds.
constexpr int kEfPrefillSilu = 1;
constexpr int kEfIntSum = 2;
constexpr int kIntSumMaxK = 8192;

// OWN (one token group of 4 tiles, TW = 1, NT = 4): the token tile a wave loads itself (tile wv) is
// its accumulator slot 0, and the wave runs half of that slot's MFMAs before the chunk's barrier (its
// own loads have landed by its own wait), so waves that reach the barrier late are absorbed by matrix
// work instead of stalling the others.  Slot n holds token tile (wv + n) mod 4.
// ROPE (the fused [q | k | v] projection of a prefill, kFuseRopePrefill): wave w of a block (2 heads,
// 16 row tiles) holds row tiles h*8 + 2*(w & 1) + {0, 1} and the same + 4 of head h = w >> 1, so that
// tiles r and r + 2 hold the rotation pairs (p, p + 64) of one head and the epilogue rotates q and k and
// appends K/V to the cache, as rope_qkv_kernel does after a plain store.
template <int NT, int RTW, int NBUF, int EPI, bool DUAL, int TW, int WPE = 1, bool OWN = false, bool ROPE = false,
          int EF = 0>
__global__ void __launch_bounds__(256 * TW) __attribute__((amdgpu_waves_per_eu(WPE))) gemm_i8_pipe_kernel(GemmArgs a) {
  static_assert(!OWN || (TW == 1 && NT == 4), "own tile first: each of the 4 waves loads one token tile");
  static_assert(!ROPE || (RTW == 4 && TW == 1 && !DUAL && EPI == kEpiStore), "prefill RoPE: 2 heads per block");
  constexpr int D = DUAL ? 2 : 1;
  constexpr int TOK = 16 * NT * TW;        // tokens per block (TW token groups of 16*NT)
  constexpr int XB = TOK * 256;                 // activation bytes per stage
  constexpr int WB = 4 * RTW * D * 1024;        // weight bytes per stage (4 waves)
  constexpr int OPS = NT + RTW * D / TW;        // direct loads per chunk per wave
  static_assert(NBUF >= 2, "at least one chunk in flight");
  static_assert((RTW * D) % TW == 0, "weight tiles split evenly over the token groups");
  static_assert((NBUF - 2) * OPS < 64, "pipeline depth");
  static_assert(D * RTW + 8 <= 15, "LDS reads in flight (weight tiles, token tiles n and n+1) fit lgkmcnt");
  // One LDS object per stage and operand: the compiler tracks direct-load writes per object, so
  // reads of one stage do not wait for loads still landing in the others.
  __shared__ __align__(16) uint8_t smem[NBUF * (XB + WB)];  // stage s: [XB activations][WB weights]
  uint8_t* XS[NBUF];
  uint8_t* WS[NBUF];
#pragma unroll
  for (int st = 0; st < NBUF; ++st) {
    XS[st] = smem + st * (XB + WB);
    WS[st] = XS[st] + XB;
  }
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;  // wave of the block
  const int wave = wv & 3;           // row position of the wave
  const int tw = wv >> 2;            // token group of the wave
  const int g = lane >> 4;
  const int col = lane & 15;
  const int row_tiles = a.out_dim / 16;
  // Block order: block ids are dealt to the 8 XCDs round robin, so XCD x gets the contiguous run
  // [x*per_xcd, (x+1)*per_xcd) of the grid order below; that order walks groups of kRasterGroup
  // token tiles with the token tile fastest, so the blocks an XCD runs together share a few
  // activation tiles and a few weight row groups in its L2.
  const int tiles_t = (a.tokens + TOK - 1) / TOK;
  const int tiles_r = (row_tiles + 4 * RTW - 1) / (4 * RTW);
  const int nblk = tiles_t * tiles_r;
  const int per_xcd = (nblk + 7) / 8;
  const int lin = (int)(blockIdx.x & 7) * per_xcd + (int)(blockIdx.x >> 3);
  if (lin >= nblk) return;  // block-uniform: padding ids of the last XCD run
  const int G = min(kRasterGroup, tiles_t);
  const int group = lin / (G * tiles_r);
  const int first_t = group * G;
  const int gsize = min(tiles_t - first_t, G);
  const int within = lin - group * G * tiles_r;
  const int rt0 = ((within / gsize) * 4 + wave) * RTW;  // the wave's first row tile
  // row tile of the wave's tile r
  auto row_tile = [&](int r) {
    return ROPE ? (within / gsize) * 16 + (wave >> 1) * 8 + (wave & 1) * 2 + (r & 1) + (r >> 1) * 4 : rt0 + r;
  };
  const int tok0 = (first_t + within % gsize) * TOK;   // the block's first token
  const int nkc_all = a.in_dim / kKChunk;
  const int nch = nkc_all / gridDim.z;
  const int kc0 = blockIdx.z * nch;
  const size_t row_stride_x = (size_t)a.in_dim * 2u;

  // per-lane global sources (chunk offsets are added per issue)
  const uint8_t* xsrc[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int r = (wv * NT + j) * 4 + (lane >> 4);    // activation row (token) this lane loads
    const int seg = (lane & 15) ^ (r & 15);
    const int tok = min(tok0 + r, a.tokens - 1);      // rows past the last token reload a valid row
    xsrc[j] = reinterpret_cast<const uint8_t*>(a.xq) + (size_t)tok * row_stride_x + seg * 16;
  }
  const uint8_t* wsrc[D][RTW];
#pragma unroll
  for (int r = 0; r < RTW; ++r) {
    const size_t off = (((size_t)(row_tile(r) < row_tiles ? row_tile(r) : 0) * nkc_all) * 64u + lane) * 16u;
    wsrc[0][r] = a.wp + off;
    if (DUAL) wsrc[D - 1][r] = a.wp2 + off;
  }
  // The next chunk to load.  Past the last chunk the last one is loaded again into a stage nobody
  // reads, which keeps the number of loads per iteration constant (and the waits exact).
  int it_c = 0;
  auto issue = [&](uint8_t* xst, uint8_t* wst) {
    const int kc = kc0 + it_c;
#pragma unroll
    for (int j = 0; j < NT; ++j)
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(xsrc[j] + (size_t)kc * 256u),
                                       (__attribute__((address_space(3))) void*)(xst + (wv * NT + j) * 1024), 16, 0,
                                       0);
#pragma unroll
    for (int d = 0; d < D; ++d)
#pragma unroll
      for (int r = 0; r < RTW; ++r)
        if ((d * RTW + r) % TW == tw)  // the token groups share the row position's weight tiles
          __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(wsrc[d][r] + (size_t)kc * 1024u),
                                           (__attribute__((address_space(3))) void*)(wst + ((wave * D + d) * RTW + r) * 1024),
                                           16, 0, 0);
    if (it_c + 1 < nch) ++it_c;
  };

  v4i accH[D][RTW][NT], accL[D][RTW][NT];
  auto zero_acc = [&]() {
#pragma unroll
    for (int d = 0; d < D; ++d)
#pragma unroll
      for (int r = 0; r < RTW; ++r)
#pragma unroll
        for (int n = 0; n < NT; ++n) accH[d][r][n] = accL[d][r][n] = v4i{0, 0, 0, 0};
  };

  // One chunk: the stage (xst, wst) holds it; (xnx, wnx) is the stage the next issue refills.
  auto chunk = [&](uint8_t* xst, uint8_t* wst, uint8_t* xnx, uint8_t* wnx) {
    // exactly NBUF-2 chunks were issued after this one: waiting for all but their loads means it has
    // landed (this wave's part); the barrier covers the other waves' parts and frees the stage the
    // next issue refills (read in the previous chunk).
    wait_vmcnt<(NBUF - 2) * OPS>();
    if (!OWN) {
      __builtin_amdgcn_s_barrier();
      issue(xnx, wnx);
    }
    // LDS reads of the stage: the weight tiles and token tile 0 first, then tile n+1 while the
    // matrix cores work on tile n.  They are issued as ds_read_b128 with explicit lgkmcnt waits:
    // the compiler cannot tell which stage an in-flight direct load writes, and would otherwise
    // drain every outstanding load (s_waitcnt vmcnt(0)) before each read, i.e. the whole pipeline.
    const uint32_t wa = lds_addr(wst) + (uint32_t)(wave * D * RTW * 1024 + lane * 16);
    const uint32_t xb = lds_addr(xst) + (uint32_t)((tw * 16 * NT + col) * 256);
    const uint32_t xo[4] = {xb + (uint32_t)(((2 * g) ^ col) << 4), xb + (uint32_t)(((2 * g + 1) ^ col) << 4),
                            xb + (uint32_t)(((8 + 2 * g) ^ col) << 4), xb + (uint32_t)(((9 + 2 * g) ^ col) << 4)};
    v4i wr[D][RTW];
#pragma unroll
    for (int d = 0; d < D; ++d)
#pragma unroll
      for (int r = 0; r < RTW; ++r) wr[d][r] = lds_read_b128(wa + (uint32_t)((d * RTW + r) * 1024));
    // LDS offset of the token tile in accumulator slot n
    auto slot_off = [&](int n) { return (uint32_t)((((OWN ? wv : 0) + n) & (NT - 1)) * 16 * 256); };
    v4i bx[2][4];
#pragma unroll
    for (int q = 0; q < 4; ++q) bx[0][q] = lds_read_b128(xo[q] + slot_off(0));
    v4i a1[D][RTW], a2[D][RTW];
    auto mfma_slot = [&](int n, const v4i* cur, int p0, int p1) {  // (d, r) pairs p0 <= p < p1
#pragma unroll
      for (int pr = 0; pr < D * RTW; ++pr) {
        if (pr < p0 || pr >= p1) continue;
        const int d = pr / RTW, r = pr % RTW;
        accH[d][r][n] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1[d][r], cur[0], accH[d][r][n], 0, 0, 0);
        accH[d][r][n] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a2[d][r], cur[1], accH[d][r][n], 0, 0, 0);
        accL[d][r][n] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1[d][r], cur[2], accL[d][r][n], 0, 0, 0);
        accL[d][r][n] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a2[d][r], cur[3], accL[d][r][n], 0, 0, 0);
      }
    };
    auto unpack_weights = [&]() {
#pragma unroll
      for (int d = 0; d < D; ++d)
#pragma unroll
        for (int r = 0; r < RTW; ++r) {
          reg_tie(wr[d][r]);  // landed before token tile 0 (LDS reads complete in order)
          unpack16(make_uint4((uint32_t)wr[d][r][0], (uint32_t)wr[d][r][1], (uint32_t)wr[d][r][2],
                              (uint32_t)wr[d][r][3]),
                   a1[d][r], a2[d][r]);
        }
    };
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      v4i* cur = bx[n & 1];
      if (OWN && n == 0) {
        // own tile and weights: landed by this wave's wait; the other tiles only after the barrier
        lgkm_wait_tie<0>(cur[0], cur[1], cur[2], cur[3]);
        unpack_weights();
        mfma_slot(0, cur, 0, D * RTW / 2);
        __builtin_amdgcn_s_barrier();
        issue(xnx, wnx);
#pragma unroll
        for (int q = 0; q < 4; ++q) bx[1][q] = lds_read_b128(xo[q] + slot_off(1));
        mfma_slot(0, cur, D * RTW / 2, D * RTW);
        continue;
      }
      if (n + 1 < NT) {
#pragma unroll
        for (int q = 0; q < 4; ++q) bx[(n + 1) & 1][q] = lds_read_b128(xo[q] + slot_off(n + 1));
        lgkm_wait_tie<4>(cur[0], cur[1], cur[2], cur[3]);
      } else {
        lgkm_wait_tie<0>(cur[0], cur[1], cur[2], cur[3]);
      }
      if (n == 0) unpack_weights();
      mfma_slot(n, cur, 0, D * RTW);
    }
  };

  const bool partial = gridDim.z > 1 || (!DUAL && a.fuse != kFuseNone);  // a reduce kernel finishes
  // Epilogue.  Every operand load is issued before the first use, so the wave waits for memory once
  // rather than once per (row tile, token tile); token columns past the last token read the last
  // token's values and store nothing.
  auto epilogue = [&]() {
    int tok[NT];
    float sxv[NT];
    int sh8[NT], sl8[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      tok[n] = tok0 + tw * 16 * NT + (((OWN ? wv : 0) + n) & (NT - 1)) * 16 + col;
      const int tc = min(tok[n], a.tokens - 1);
      sxv[n] = a.sx[tc];
      const int2 sm = *reinterpret_cast<const int2*>(a.sums + 2 * tc);
      sh8[n] = 8 * sm.x;
      sl8[n] = 8 * sm.y;
    }
    float sw[RTW][4], sw2[RTW][4], bias[RTW][4];
#pragma unroll
    for (int r = 0; r < RTW; ++r) {
      const int row0 = min(row_tile(r), row_tiles - 1) * 16 + 4 * g;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        sw[r][q] = a.sw[row0 + q];
        sw2[r][q] = DUAL ? a.sw2[row0 + q] : 0.0f;
        bias[r][q] = (EPI == kEpiStore && a.bias) ? a.bias[row0 + q] : 0.0f;
      }
    }
    if constexpr (ROPE) {
      // tiles r and r + 2 (r < 2): dims p .. p + 3 and p + 64 .. p + 67 of head rt / 8; cos/sin of the
      // lane's tokens are loaded per pair, so that one pair's 32 registers are live at a time
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int rt = row_tile(r);
        const int head = rt >> 3;
        const int p = (rt & 7) * 16 + 4 * g;
        int Pn[NT], seqn[NT];
        float4 cs[NT], sn[NT];
#pragma unroll
        for (int n = 0; n < NT; ++n) {
          const int tc = min(tok[n], a.tokens - 1);
          seqn[n] = tc / a.seq_len;
          Pn[n] = a.past + tc % a.seq_len;
          const int Pc = min(max(Pn[n], 0), a.limit - 1);
          cs[n] = *reinterpret_cast<const float4*>(a.rope + (size_t)Pc * 128 + p);
          sn[n] = *reinterpret_cast<const float4*>(a.rope + (size_t)Pc * 128 + 64 + p);
        }
#pragma unroll
        for (int n = 0; n < NT; ++n) {
          if (tok[n] >= a.tokens || Pn[n] < 0 || Pn[n] >= a.limit) continue;
          float e[4], od[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            e[q] = (float)(accH[0][r][n][q] - sh8[n]) * 256.0f + (float)(accL[0][r][n][q] - sl8[n]);
            e[q] = e[q] * sxv[n] * sw[r][q] + bias[r][q];
            od[q] = (float)(accH[0][r + 2][n][q] - sh8[n]) * 256.0f + (float)(accL[0][r + 2][n][q] - sl8[n]);
            od[q] = od[q] * sxv[n] * sw[r + 2][q] + bias[r + 2][q];
          }
          const float c4[4] = {cs[n].x, cs[n].y, cs[n].z, cs[n].w}, s4[4] = {sn[n].x, sn[n].y, sn[n].z, sn[n].w};
          float lo[4], hi[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const bool v_head = head >= QWEN_Q_HEADS + QWEN_KV_HEADS;
            lo[q] = v_head ? e[q] : e[q] * c4[q] - od[q] * s4[q];
            hi[q] = v_head ? od[q] : od[q] * c4[q] + e[q] * s4[q];
          }
          float* dst;
          if (head < QWEN_Q_HEADS) {
            dst = a.y + (size_t)tok[n] * a.y_stride + head * QWEN_HEAD_DIM + p;
          } else {
            const size_t crow = (size_t)seqn[n] * a.seq_stride + (size_t)Pn[n] * QWEN_KV_WIDTH;
            dst = head < QWEN_Q_HEADS + QWEN_KV_HEADS
                      ? a.k_cache + crow + (head - QWEN_Q_HEADS) * QWEN_HEAD_DIM + p
                      : a.v_cache + crow + (head - QWEN_Q_HEADS - QWEN_KV_HEADS) * QWEN_HEAD_DIM + p;
          }
          *reinterpret_cast<float4*>(dst) = make_float4(lo[0], lo[1], lo[2], lo[3]);
          *reinterpret_cast<float4*>(dst + 64) = make_float4(hi[0], hi[1], hi[2], hi[3]);
        }
      }
      return;
    }
    // zero-point term of the int32 form: 256 * (8 sum H) + 8 sum L per token, modulo 2^32
    uint32_t c8[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) c8[n] = ((uint32_t)sh8[n] << 8) + (uint32_t)sl8[n];
    auto dequant = [&](int d, int r, int n, int q) -> float {
      if constexpr ((EF & kEfIntSum) != 0) {
        const uint32_t x = ((uint32_t)accH[d][r][n][q] << 8) + (uint32_t)accL[d][r][n][q] - c8[n];
        return (float)(int32_t)x;
      } else {
        // fp32 dequantization: the int32 sums are exact; fp32 adds ~2^-24 relative, far inside the
        // FAST tolerance, at a quarter of the cost of the fp64 form
        return (float)(accH[d][r][n][q] - sh8[n]) * 256.0f + (float)(accL[d][r][n][q] - sl8[n]);
      }
    };
    // the lane's output rows start at yrow[n] + row0 (one 64-bit product per token, not per store)
    float* yrow[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) yrow[n] = a.y + (size_t)min(tok[n], a.tokens - 1) * a.y_stride;
#pragma unroll
    for (int r = 0; r < RTW; ++r) {
      if (rt0 + r >= row_tiles) continue;
      const int row0 = (rt0 + r) * 16 + 4 * g;
      float4 res[NT];
      if (EPI == kEpiResidual && !partial) {
#pragma unroll
        for (int n = 0; n < NT; ++n)
          res[n] = *reinterpret_cast<const float4*>(a.resid + (size_t)min(tok[n], a.tokens - 1) * a.resid_stride + row0);
      }
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        float out[4];
        if (partial) {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            out[q] = ((float)accH[0][r][n][q] * 256.0f + (float)accL[0][r][n][q]) * sxv[n] * sw[r][q];
          if (tok[n] < a.tokens)
            *reinterpret_cast<float4*>(a.part + ((size_t)blockIdx.z * a.tokens + tok[n]) * a.out_dim + row0) =
                make_float4(out[0], out[1], out[2], out[3]);
          continue;
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float v = dequant(0, r, n, q) * sxv[n] * sw[r][q];
          if (EPI == kEpiSiluMul) {
            const float u = dequant(D - 1, r, n, q) * sxv[n] * sw2[r][q];
            const float sg = (EF & kEfPrefillSilu) != 0 ? silu_prefill_fast(v) : silu_decode(v);
            out[q] = sg * u;
          } else if (EPI == kEpiResidual) {
            out[q] = (&res[n].x)[q] + v;
          } else {
            out[q] = v + bias[r][q];
          }
        }
        if (tok[n] >= a.tokens) continue;
        if (EPI == kEpiResidual && a.y_raw)
          *reinterpret_cast<float4*>(a.y_raw + (size_t)tok[n] * a.y_stride + row0) =
              make_float4(out[0], out[1], out[2], out[3]);
        if (EPI == kEpiResidual && a.round_bf16)
#pragma unroll
          for (int q = 0; q < 4; ++q) out[q] = round_bf16(out[q]);
        *reinterpret_cast<float4*>(yrow[n] + row0) = make_float4(out[0], out[1], out[2], out[3]);
      }
    }
  };

  zero_acc();
#pragma unroll
  for (int i = 0; i < NBUF - 1; ++i) issue(XS[i], WS[i]);
  for (int i0 = 0; i0 < nch; i0 += NBUF) {
#pragma unroll
    for (int sidx = 0; sidx < NBUF; ++sidx) {
      if (i0 + sidx < nch) chunk(XS[sidx], WS[sidx], XS[(sidx + NBUF - 1) % NBUF], WS[(sidx + NBUF - 1) % NBUF]);
    }
  }
  wait_vmcnt<0>();  // the trailing reloads land before the wave moves on
  epilogue();
}

// ---------------------------------------------------------------------------------------------
// Skinny GEMM for decode batches (the same y = W x products as the kernels above, for few tokens).
// A block owns 16 tokens (token tile tt), 4*RTW row tiles (row group rg: wave w holds row tiles
// rg*4*RTW + w + 4r, r < RTW) and NKC K chunks (split z).  Every load of the block is issued at
// once: its activation slice goes to LDS by direct loads ([chunk][token][256 B], 16-byte segments
// XOR-swizzled by token), its weight tiles go straight to registers (RTW*D*NKC x 16 B per lane);
// after one wait the matrix cores run from registers and LDS.  Blocks that share weights (the
// token tiles of one (rg, z)) are given block ids on the same XCD (ids are dealt to the 8 XCDs
// round robin), so the weights come from HBM once and from that XCD's L2 after.
// Epilogues: EPI as in gemm_i8_kernel, or fp32 partials to a.part[z] (K splits, or a fused reduce
// step), or with ROPE the decode RoPE + K/V cache append of the fused [q | k | v] projection (RTW=2:
// wave w holds rows p and p + 64 of head rg, p = 16w + 4g + q).
// grid = 8 * tt_count * ceil(groups / 8) blocks of 256, groups = row groups x splits.
// ---------------------------------------------------------------------------------------------
struct NoIssue {
  __device__ void operator()() const {}
};

// Elementwise pieces of the reduce step: the split sum plus zero-point correction, residual or bias,
// optional y_raw / y stores and bf16 rounding of elements row0 .. row0 + 3; the sum of squares of
// four elements in double; the RMSNorm scaling.
template <int EPI>
__device__ __forceinline__ float4 rnq_combine(const GemmArgs& a, int tok, int row0, float4 acc, float4 sw, float4 ad,
                                              double corr, bool write_y) {
  const float s4[4] = {sw.x, sw.y, sw.z, sw.w};
  const float p4[4] = {acc.x, acc.y, acc.z, acc.w};
  const float d4[4] = {ad.x, ad.y, ad.z, ad.w};
  float out[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float val = p4[q] + (float)(corr * (double)s4[q]);
    out[q] = EPI == kEpiResidual ? d4[q] + val : val + d4[q];
  }
  if (EPI == kEpiResidual && a.y_raw && write_y)
    *reinterpret_cast<float4*>(a.y_raw + (size_t)tok * a.y_stride + row0) = make_float4(out[0], out[1], out[2], out[3]);
  if (EPI == kEpiResidual && a.round_bf16)
#pragma unroll
    for (int q = 0; q < 4; ++q) out[q] = round_bf16(out[q]);
  const float4 v = make_float4(out[0], out[1], out[2], out[3]);
  if (write_y) *reinterpret_cast<float4*>(a.y + (size_t)tok * a.y_stride + row0) = v;
  return v;
}
__device__ __forceinline__ double rnq_sq4(float4 v) {
  return (double)v.x * v.x + (double)v.y * v.y + (double)v.z * v.z + (double)v.w * v.w;
}
__device__ __forceinline__ float4 rnq_norm4(float4 v, double inv, float4 w) {
  return make_float4((float)((double)v.x * inv * w.x), (float)((double)v.y * inv * w.y),
                     (float)((double)v.z * inv * w.z), (float)((double)v.w * inv * w.w));
}
// The operands a one-token prologue's first loads need (and the block mapping's counts), passed as a
// kernel's leading scalar arguments: the hardware preloads those into SGPRs at wave launch (the build
// asks for up to 14 argument dwords), so the prologue issues its loads at once instead of after the
// argument segment's memory round trip (~0.5 us).  The segment's lines are requested at entry all the
// same and waited for once the prologue's loads are issued, before the weights: requested only then,
// behind the prologue's loads, their round trip delayed the weights of the Q/K/V and gate/up launches
// (greedy decode 1.5% slower than without preloading; requested at entry, 5% faster).
// Reduce prologue: p0 partials, p1 residual (bias, or a stand-in), p2 row scales, p3 norm weights (or
// a stand-in), p4 limb sums, p5 scale.  Attention merge: p0 partials, p1 (m, l) pairs, p2 position,
// p3 the [q | k | v] row (or a stand-in), n0 key splits.  Row quantization: p0 the row, p1 its
// per-block maxima, n0 their count.  Fused attention: n0 its key splits.
struct HotArgs {
  const void* p0 = nullptr;
  const void* p1 = nullptr;
  const void* p2 = nullptr;
  const void* p3 = nullptr;
  const void* p4 = nullptr;
  const void* p5 = nullptr;
  int n0 = 0;
};

template <int EPI, class Issue = NoIssue>
__device__ __forceinline__ void reduce_norm_quant_row(const GemmArgs& a, int splits, int tok, int8_t* xq_row,
                                                      int chunk_stride, float* sx_out, int* sums_out, bool write_y,
                                                      Issue&& issue = Issue{});
template <int EPI, int ZB, class Issue, int W = 1, bool HOT = false>
__device__ __forceinline__ void reduce_norm_quant_row_zb(const GemmArgs& a, int splits, int tok, int8_t* xq_row,
                                                         int chunk_stride, float* sx_out, int* sums_out, bool write_y,
                                                         Issue&& issue, const HotArgs& hot = HotArgs{});
template <int EPI, int ZB, bool HOT, class Issue>
__device__ __forceinline__ void reduce_norm_quant_row_w4(const GemmArgs& a, int splits, int8_t* xq_row,
                                                         int chunk_stride, float* sx_out, int* sums_out, bool write_y,
                                                         Issue&& issue, const HotArgs& hot);

// Two-limb quantization of one fp32 row x[0, n) (n % 4 == 0, n <= NV * 1024) by a 256-thread block
// with norm_quant_row's arithmetic and thread mapping (float4 k = t + 256 j): the code of K chunks
// kc0 .. kc0 + nkc - 1 goes to xs (chunk kc0 + i at byte i * chunk_stride), the scale and limb sums of
// the whole row to sx_lds / sums_lds and, when sx_g is given, to sx_g / sums_g.
template <int NV, class Issue>
__device__ __forceinline__ void quant_row_slice(const float* __restrict__ x, int n, int kc0, int nkc, uint8_t* xs,
                                                int chunk_stride, float* sx_lds, int* sums_lds, float* sx_g,
                                                int* sums_g, Issue&& issue) {
  __shared__ float red_f[4];
  __shared__ int red_i[8];
  const int n4 = n >> 2;
  const float4* x4 = reinterpret_cast<const float4*>(x);
  float4 v[NV];
  // branch-free: past the row's end the loads read its last float4 again, zeroed after
#pragma unroll
  for (int j = 0; j < NV; ++j) v[j] = x4[min((int)threadIdx.x + 256 * j, n4 - 1)];
  __builtin_amdgcn_sched_barrier(0);
  issue();  // the caller's loads queue behind the row's
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < NV; ++j)
    if ((int)threadIdx.x + 256 * j >= n4) v[j] = make_float4(0, 0, 0, 0);
  __builtin_amdgcn_sched_barrier(0);
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j)
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
  amax = block_max4(amax, red_f);
  const float inv = amax > 0.0f ? (float)kQuantMax / amax : 0.0f;
  int sh = 0, sl = 0;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int k = threadIdx.x + 256 * j;
    if (k < n4) {
      const float e[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
      uint32_t hw = 0, lw = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float xf = fminf(fmaxf(rintf(e[q] * inv), -(float)kQuantMax), (float)kQuantMax);
        const int X = (int)xf;
        const int H = (X + 128) >> 8;
        const int L = X - (H << 8);
        hw |= (uint32_t)(H & 0xFF) << (8 * q);
        lw |= (uint32_t)(L & 0xFF) << (8 * q);
        sh += H;
        sl += L;
      }
      const int chunk = (4 * k) >> 7;
      if (chunk >= kc0 && chunk < kc0 + nkc) {
        uint8_t* dst = xs + (chunk - kc0) * chunk_stride + ((4 * k) & 127);
        *reinterpret_cast<uint32_t*>(dst) = hw;
        *reinterpret_cast<uint32_t*>(dst + 128) = lw;
      }
    }
  }
  block_sum4_i2(sh, sl, red_i);
  if (threadIdx.x == 0) {
    const float sx = amax > 0.0f ? amax / (float)kQuantMax : 1.0f;
    *sx_lds = sx;
    sums_lds[0] = sh;
    sums_lds[1] = sl;
    if (sx_g) {
      *sx_g = sx;
      sums_g[0] = sh;
      sums_g[1] = sl;
    }
  }
}

// quant_row_slice for a row whose maximum comes as per-block maxima (amax_n of them, a multiple of 4,
// at most 1024): the block reads the maxima and its own K chunks kc0 .. kc0 + nkc - 1 of x (nkc <= 16)
// only, and quantizes those into the slice with the row's scale (the maximum of the maxima, the same
// value as the whole row's: fmaxf is exact).  The row's limb sums are not formed here (sums_lds: 0).
template <class Issue>
__device__ __forceinline__ void quant_chunks_from_maxima(const float* __restrict__ x, const float* __restrict__ amax_in,
                                                         int amax_n, int kc0, int nkc, uint8_t* xs, int chunk_stride,
                                                         float* sx_lds, int* sums_lds, Issue&& issue) {
  __shared__ float red_f[4];
  const int t = threadIdx.x;
  const int n4 = nkc * 32;  // float4s of the block's chunks
  const float4* x4 = reinterpret_cast<const float4*>(x) + kc0 * 32;
  float4 v[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) v[j] = x4[min(t + 256 * j, n4 - 1)];
  const float4 m4 = reinterpret_cast<const float4*>(amax_in)[min(t, amax_n / 4 - 1)];
  __builtin_amdgcn_sched_barrier(0);
  issue();  // the caller's loads queue behind the row's
  __builtin_amdgcn_sched_barrier(0);
  float amax = t < amax_n / 4 ? fmaxf(fmaxf(m4.x, m4.y), fmaxf(m4.z, m4.w)) : 0.0f;
  amax = block_max4(amax, red_f);
  const float inv = amax > 0.0f ? (float)kQuantMax / amax : 0.0f;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int k = t + 256 * j;
    if (k < n4) {
      const float e[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
      uint32_t hw = 0, lw = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float xf = fminf(fmaxf(rintf(e[q] * inv), -(float)kQuantMax), (float)kQuantMax);
        const int X = (int)xf;
        const int H = (X + 128) >> 8;
        const int L = X - (H << 8);
        hw |= (uint32_t)(H & 0xFF) << (8 * q);
        lw |= (uint32_t)(L & 0xFF) << (8 * q);
      }
      uint8_t* dst = xs + ((4 * k) >> 7) * chunk_stride + ((4 * k) & 127);
      *reinterpret_cast<uint32_t*>(dst) = hw;
      *reinterpret_cast<uint32_t*>(dst + 128) = lw;
    }
  }
  if (t == 0) {
    *sx_lds = amax > 0.0f ? amax / (float)kQuantMax : 1.0f;
    sums_lds[0] = 0;
    sums_lds[1] = 0;
  }
}

// Merge weights of one sequence's split-KV decode-attention partials, per head h: M = the maximum of
// the splits' m (and of the new key's score s_new[h] when has_new), f = exp(m - M), L = sum of l * f
// (+ exp(s_new[h] - M)), weight = f / L, written over m in ml ([h][kAttnMaxSplits][2]: m, l) for the
// splits sp < nc (and to s_new[h] for the new key).  Threads 16h + j (h < NH) take splits j, j + 16,
// j + 32, j + 48 of head h; the maximum and the sum meet by DPP row steps (one row of 16 lanes per
// head), each lane's own splits first in ascending order.  Every thread of the block calls it.
template <int NH = QWEN_Q_HEADS>
__device__ __forceinline__ void merge_split_weights(float* ml, int nc, float* s_new, bool has_new) {
  static_assert(kAttnMaxSplits % 16 == 0, "splits in rows of 16 lanes");
  constexpr int kPer = kAttnMaxSplits / 16;
  const int t = threadIdx.x;
  if (t < 16 * NH) {  // wave-uniform for NH a multiple of 4: waves 0..2 for 12 heads
    const int h = t >> 4, j = t & 15;
    float* mh = ml + h * kAttnMaxSplits * 2;
    auto rmax = [](float v) {
      v = fmaxf(v, __int_as_float(dpp_i<0xB1>(__float_as_int(v))));
      v = fmaxf(v, __int_as_float(dpp_i<0x4E>(__float_as_int(v))));
      v = fmaxf(v, __int_as_float(dpp_i<0x124>(__float_as_int(v))));
      return fmaxf(v, __int_as_float(dpp_i<0x128>(__float_as_int(v))));
    };
    auto rsum = [](float v) {
      v += __int_as_float(dpp_i<0xB1>(__float_as_int(v)));
      v += __int_as_float(dpp_i<0x4E>(__float_as_int(v)));
      v += __int_as_float(dpp_i<0x124>(__float_as_int(v)));
      return v + __int_as_float(dpp_i<0x128>(__float_as_int(v)));
    };
    float mv[kPer], lv[kPer];
    float M = -INFINITY;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int sp = j + 16 * k;
      mv[k] = sp < nc ? mh[2 * sp] : -INFINITY;
      lv[k] = sp < nc ? mh[2 * sp + 1] : 0.0f;
      M = fmaxf(M, mv[k]);
    }
    M = rmax(M);
    if (has_new) M = fmaxf(M, s_new[h]);
    float L = 0.0f;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      mv[k] = j + 16 * k < nc ? __expf(mv[k] - M) : 0.0f;
      L += lv[k] * mv[k];
    }
    L = rsum(L);
    const float fn = has_new ? __expf(s_new[h] - M) : 0.0f;
    L += fn;
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
#pragma unroll
    for (int k = 0; k < kPer; ++k)
      if (j + 16 * k < nc) mh[2 * (j + 16 * k)] = mv[k] * inv;  // merge weight of split sp
    if (has_new && j == 0) s_new[h] = fn * inv;                 // merge weight of the new key
  }
}

// The merge of one sequence's split-KV decode-attention partials, in the arithmetic and order of
// attn_decode_kernel's merge (per head: max of the split maxima, exp-weights normalised by the
// weighted sum, then the weighted sum of the split partial rows), followed by quantize_row_lds's
// quantization of the merged rows (from registers) into token 0's row of a skinny-GEMM slice (K
// chunk c at xs + c * chunk_stride).  The block merges query heads h0 .. h0 + HS - 1, i.e. context
// columns 128 h0 .. 128 (h0 + HS) - 1, and quantizes them with their own scale and limb sums (HS = 12:
// the whole row).  The partials come from the previous launch, so plain loads see them.  256 threads.
// NEWKEY (the attention fused into the Q/K/V projection): the partials cover the history keys and the
// new key is a term of its own, read from am.qkv_new: score s = (q / sqrt(128)) . k, weight exp(s - M)
// with M the maximum over the splits and s, added to the sum with l = 1 and to the row with v.
template <bool NEWKEY = false, int KF = 16, int HS = QWEN_Q_HEADS, bool HOT = false, class Issue>
__device__ __forceinline__ void attn_merge_quant_slice(const AttnMergeArgs& am, int h0, uint8_t* xs, int chunk_stride,
                                                       float* sx_lds, int* sums_lds, bool write_global,
                                                       Issue&& issue, const HotArgs& hot = HotArgs{}) {
  static_assert(QWEN_Q_HEADS % HS == 0 && HS * 32 <= 512, "a head range of the context row");
  __shared__ float ml[HS * kAttnMaxSplits * 2];  // (m, l) per head and split, then merge weights
  __shared__ float red_f[4];
  __shared__ int red_i[8];
  // The loads do not wait for the position: the first kFirst splits' partials and every (m, l) pair
  // are loaded whatever the key count; the merge below reads only the splits that hold keys.  Thread
  // t owns float4 f = t and t + 256 (f < kF4) of the block's columns: local head f >> 5, dims 4 (f & 31)
  // .. + 3 (threads past the last float4 load its values again, used by nobody); 16-byte loads keep a
  // wave's outstanding loads (with the caller's weights) under the counter's 63.
  // KF (8, 12 or 16) is the batch of splits loaded at once; with KF < 16 the caller guarantees
  // nsplit <= KF, so one batch and one (m, l) pair per thread cover every split.
  static_assert(KF == 8 || KF == 12 || KF == 16, "merge batch");
  constexpr int kFirst = KF;
  constexpr int kF4 = HS * 32;                // float4s of the block's columns
  constexpr int kU = (kF4 + 255) / 256;       // float4s per thread
  // (HOT: the operands of the first loads from the preloaded HotArgs)
  const int nsplit = HOT ? hot.n0 : am.nsplit;
  const float* m_part = HOT ? static_cast<const float*>(hot.p0) : am.part;
  const float2* m_pml = HOT ? static_cast<const float2*>(hot.p1) : am.pml;
  const int* m_pos = HOT ? static_cast<const int*>(hot.p2) : am.pos;
  const float* m_new = HOT ? static_cast<const float*>(hot.p3) : am.qkv_new;
  float4 pv[kU][kFirst];
  auto fidx = [&](int u) { return min((int)threadIdx.x + 256 * u, kF4 - 1); };
  auto owns = [&](int u) { return (int)threadIdx.x + 256 * u < kF4; };
  auto load_part = [&](int s0) {
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int f = fidx(u);
#pragma unroll
      for (int j = 0; j < kFirst; ++j)
        pv[u][j] = *reinterpret_cast<const float4*>(
            m_part + ((size_t)(h0 + (f >> 5)) * nsplit + min(s0 + j, nsplit - 1)) * QWEN_HEAD_DIM + 4 * (f & 31));
    }
  };
  // the position as a vector load whose register is held until it is needed (read back early, its
  // register was reused and the wait for it held the rest of the loads back by a memory round trip)
  int p0v;
  {
    int lz;
    asm volatile("v_mov_b32 %0, 0" : "=v"(lz));
    p0v = m_pos[lz];
  }
  load_part(0);
  constexpr int kMlPer = (HS * (KF < 16 ? KF : kAttnMaxSplits) + 255) / 256;  // (m, l) pairs per thread
  float2 mlv[kMlPer];
#pragma unroll
  for (int u = 0; u < kMlPer; ++u) {
    const int i = min((int)threadIdx.x + 256 * u, HS * nsplit - 1);
    mlv[u] = m_pml[h0 * nsplit + i];  // pml[h][sp] at h * nsplit + sp
  }
  // NEWKEY: the thread's q, k and v float4s of the new key (head h0 + (f >> 5), its KV head)
  float4 nq[kU], nk[kU], nv[kU];
  if constexpr (NEWKEY) {
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int f = fidx(u), h = h0 + (f >> 5);
      const int d4 = 4 * (f & 31), kvo = (h / QWEN_GROUPS) * QWEN_HEAD_DIM + d4;
      nq[u] = *reinterpret_cast<const float4*>(m_new + h * QWEN_HEAD_DIM + d4);
      nk[u] = *reinterpret_cast<const float4*>(m_new + QWEN_HIDDEN + kvo);
      nv[u] = *reinterpret_cast<const float4*>(m_new + QWEN_HIDDEN + QWEN_KV_WIDTH + kvo);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  issue();  // the caller's loads queue behind the partials
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int u = 0; u < kMlPer; ++u) {
    const int i = threadIdx.x + 256 * u;
    if (i < HS * nsplit) {
      const int h = i / nsplit, sp = i % nsplit;
      ml[(h * kAttnMaxSplits + sp) * 2] = mlv[u].x;
      ml[(h * kAttnMaxSplits + sp) * 2 + 1] = mlv[u].y;
    }
  }
  asm volatile("" : "+v"(p0v));
  const int p0 = __builtin_amdgcn_readfirstlane(p0v);
  const int n = min(max(p0, 0) + 1, am.max_keys);
  // NEWKEY: the history keys end at p0 when the new key is one of the n keys
  const bool has_new = NEWKEY && p0 >= 0 && p0 < am.max_keys;
  const int hist = has_new ? p0 : n;
  const int nc = (hist + am.chunk - 1) / am.chunk;  // splits that hold keys (the rest hold stale values)
  __shared__ float s_new[HS];  // NEWKEY: the new key's score per head, then its merge weight
  if constexpr (NEWKEY) {
    constexpr float kScale = 0.08838834764831845f;  // 1/sqrt(128), the scale of the split partials' q
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      if (u > 0 && !owns(u)) break;  // wave-uniform: the waves without a second float4
      float sc = (nq[u].x * kScale) * nk[u].x + (nq[u].y * kScale) * nk[u].y + (nq[u].z * kScale) * nk[u].z +
                 (nq[u].w * kScale) * nk[u].w;
#pragma unroll
      for (int o = 1; o < 32; o <<= 1) sc += __shfl_xor(sc, o, 64);  // over the head's 32 lanes
      if ((threadIdx.x & 31) == 0 && owns(u)) s_new[(threadIdx.x + 256 * u) >> 5] = sc;
    }
  }
  __syncthreads();
  merge_split_weights<HS>(ml, nc, s_new, has_new);
  __syncthreads();
  float4 out[kU];
#pragma unroll
  for (int u = 0; u < kU; ++u) out[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (int s0 = 0; s0 < nc; s0 += kFirst) {
    if (s0 > 0) load_part(s0);
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int f = threadIdx.x + 256 * u;
      if (f < kF4) {
        // the batch's merge weights read at once (slots past nc hold stale values, not used), then
        // the splits in order as selects: a branch per split waited for its own LDS read
        float w[kFirst];
#pragma unroll
        for (int j = 0; j < kFirst; ++j) w[j] = ml[((f >> 5) * kAttnMaxSplits + s0 + j) * 2];
#pragma unroll
        for (int j = 0; j < kFirst; ++j) {
          const bool live = s0 + j < nc;
          out[u].x = live ? __builtin_fmaf(pv[u][j].x, w[j], out[u].x) : out[u].x;
          out[u].y = live ? __builtin_fmaf(pv[u][j].y, w[j], out[u].y) : out[u].y;
          out[u].z = live ? __builtin_fmaf(pv[u][j].z, w[j], out[u].z) : out[u].z;
          out[u].w = live ? __builtin_fmaf(pv[u][j].w, w[j], out[u].w) : out[u].w;
        }
      }
    }
  }
  if constexpr (NEWKEY) {
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int f = threadIdx.x + 256 * u;
      if (f < kF4) {
        const float w = s_new[f >> 5];
        out[u].x += nv[u].x * w;
        out[u].y += nv[u].y * w;
        out[u].z += nv[u].z * w;
        out[u].w += nv[u].w * w;
      }
    }
  }
  // quantize_row_lds's arithmetic on the thread's own float4s, straight from registers
  float amax = 0.0f;
#pragma unroll
  for (int u = 0; u < kU; ++u)
    if (owns(u))
      amax = fmaxf(amax, fmaxf(fmaxf(fabsf(out[u].x), fabsf(out[u].y)), fmaxf(fabsf(out[u].z), fabsf(out[u].w))));
  amax = block_max4(amax, red_f);
  const float inv = amax > 0.0f ? (float)kQuantMax / amax : 0.0f;
  int sh = 0, sl = 0;
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    const int f = threadIdx.x + 256 * u;
    if (f < kF4) {
      const float e[4] = {out[u].x, out[u].y, out[u].z, out[u].w};
      uint32_t hw = 0, lw = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float xf = fminf(fmaxf(rintf(e[q] * inv), -(float)kQuantMax), (float)kQuantMax);
        const int X = (int)xf;
        const int H = (X + 128) >> 8;
        const int L = X - (H << 8);
        hw |= (uint32_t)(H & 0xFF) << (8 * q);
        lw |= (uint32_t)(L & 0xFF) << (8 * q);
        sh += H;
        sl += L;
      }
      uint8_t* dst = xs + ((4 * f) >> 7) * chunk_stride + ((4 * f) & 127);
      *reinterpret_cast<uint32_t*>(dst) = hw;
      *reinterpret_cast<uint32_t*>(dst + 128) = lw;
    }
  }
  // the limb sums as per-wave partials in sums_lds (8 ints, totals by wave_sums_total after the
  // caller's slice barrier), the scale in *sx_lds; block 0 of a whole-row merge also writes the totals
  const float sx = amax > 0.0f ? amax / (float)kQuantMax : 1.0f;
  if (write_global) {  // block-uniform
    int th = sh, tl = sl;
    block_sum4_i2(th, tl, red_i);
    if (threadIdx.x == 0) {
      *am.sx_out = sx;
      am.sums_out[0] = th;
      am.sums_out[1] = tl;
    }
  }
  sh = wave_sum_i(sh);
  sl = wave_sum_i(sl);
  if ((threadIdx.x & 63) == 0) {
    sums_lds[2 * (threadIdx.x >> 6)] = sh;
    sums_lds[2 * (threadIdx.x >> 6) + 1] = sl;
  }
  if (threadIdx.x == 0) *sx_lds = sx;
}

// PRE (one token, KSW = 1): the activation slice is not loaded but made by the block: its four waves
// redo the reduce step of the previous projection (`pre` with epilogue PRE_EPI, pre_splits K splits,
// kFuseNormQuant on a 1536-wide row) for token 0 straight into the slice, each wave's weight loads
// issued right after its loads of the row; block 0 alone writes the finished row (pre.y, pre.y_raw).  K chunk c of the
// slice is the token's row c.  PRE_QUANT (one token, KSW = 1): the slice is the two-limb code of the
// fp32 row pre.y (pre.in_dim wide, as norm_quant_kernel without a norm), made by every block for its
// own K chunks; block 0 writes the row's scale and limb sums to pre.sx_out / pre.sums_out.  PRE_ATTN
// (one token, KSW = 1, the 1536-wide context row): every block merges the decode attention's split
// partials (am) and quantizes the row into the slice; block 0 writes its scale and limb sums.
//
// ATTN (one token, the fused [q | k | v] projection with RoPE, RTW = 2): the decode attention over the
// history keys runs in the same launch (AttnFuseArgs).  Blocks 0..3 are the k and v heads (rows
// 1536..2047: RoPE, K/V append); from block 8 on, block (query head h, key split c) computes head h's
// rows, rotates them and attends over keys [c*chunk, min(pos, (c+1)*chunk)), whose K/V rows it loads
// into LDS with its weights.  Its partial (m, l, acc[128]) goes to af.part / af.pml; split 0 also stores
// the q row, which the O projection's merge needs for the new key's term.
// Byte size of a kernel's explicit arguments T..., laid out in order at their natural alignments.
template <class... T>
constexpr int kernarg_bytes() {
  int off = 0;
  ((off = (off + (int)alignof(T) - 1) / (int)alignof(T) * (int)alignof(T) + (int)sizeof(T)), ...);
  return off;
}
// Loads one dword of every 64-byte line of the first BYTES bytes of the kernel's argument segment,
// all at once, and waits for them.  The compiler issues the argument loads where each value is first
// needed, in batches with a wait between them, and the segment is written anew for every launch, so
// each batch was a memory round trip of its own before the first global load; after this one round
// trip the later argument loads hit the scalar cache.
template <int BYTES>
__device__ __forceinline__ void touch_kernargs() {
  using KPtr = const __attribute__((address_space(4))) uint32_t*;
  KPtr kp = (KPtr)__builtin_amdgcn_kernarg_segment_ptr();
  constexpr int kLines = (BYTES + 63) / 64;
  uint32_t v[kLines];
#pragma unroll
  for (int i = 0; i < kLines; ++i) v[i] = kp[16 * i];
#pragma unroll
  for (int i = 0; i < kLines; ++i) asm volatile("" ::"s"(v[i]));
}
// The same in two steps, for kernels whose first loads take their operands from preloaded arguments:
// the line loads at the kernel's entry, the wait where the other arguments are first needed.
template <int BYTES>
struct KernargLines {
  uint32_t v[(BYTES + 63) / 64];
};
template <int BYTES>
__device__ __forceinline__ KernargLines<BYTES> kernarg_lines_issue() {
  using KPtr = const __attribute__((address_space(4))) uint32_t*;
  KPtr kp = (KPtr)__builtin_amdgcn_kernarg_segment_ptr();
  KernargLines<BYTES> l;
#pragma unroll
  for (int i = 0; i < (BYTES + 63) / 64; ++i) l.v[i] = kp[16 * i];
  return l;
}
template <int BYTES>
__device__ __forceinline__ void kernarg_lines_wait(const KernargLines<BYTES>& l) {
#pragma unroll
  for (int i = 0; i < (BYTES + 63) / 64; ++i) asm volatile("" ::"s"(l.v[i]));
}

template <int RTW, bool DUAL, int EPI, int NKC, bool ROPE, int KSW, bool PRE, int PRE_EPI = kEpiStore,
          bool PRE_QUANT = false, bool PRE_ATTN = false, bool GRP = false, bool ATTN = false, bool NEWKEY = false,
          bool KW = false, int MKF = 16, int HOT_KB = 0, int HOT_IN = 0, int HOT_OUT = 0>
__device__ __forceinline__ void gemm_skinny_body(const GemmArgs& a, int tt_count, int rg_count, int splits,
                                                 const GemmArgs& pre, int pre_splits,
                                                 const AttnMergeArgs& am = AttnMergeArgs{},
                                                 const AttnFuseArgs& af = AttnFuseArgs{},
                                                 const HotArgs& hot = HotArgs{}) {
  constexpr int D = DUAL ? 2 : 1;
  // (hot: the argument segment's lines are requested at entry and waited for once the prologue's
  // first loads are issued)
  KernargLines<(HOT_KB > 0 ? HOT_KB : 4)> klines;
  if constexpr (HOT_KB > 0) klines = kernarg_lines_issue<HOT_KB>();
  static_assert(!ATTN || (RTW == 2 && !DUAL && ROPE && KSW == 1 && EPI == kEpiStore && !PRE_QUANT && !PRE_ATTN &&
                          !GRP && NKC * kKChunk == QWEN_HIDDEN),
                "ATTN: the one-token [q | k | v] projection with RoPE");
  static_assert(!PRE || (KSW == 1 && NKC * kKChunk == QWEN_HIDDEN), "PRE: one K group over a 1536-wide row");
  static_assert(!PRE_QUANT || (KSW == 1 && !PRE), "PRE_QUANT: one K group");
  static_assert(!PRE_ATTN || (KSW == 1 && !PRE && !PRE_QUANT && QWEN_HIDDEN % (NKC * kKChunk) == 0),
                "PRE_ATTN: one K group over the 1536-wide context row, or over a range of its heads");
  constexpr bool kMade = PRE || PRE_QUANT || PRE_ATTN;  // the slice is made by the block
  // GRP: the activations are the grouped two-limb code (GemmArgs::gsx, gcorr): each 64-wide K group,
  // one MFMA of a K chunk, is dequantized with its own scale, so the block's partials are fp32 sums
  // over groups that already carry the offset correction
  static_assert(!GRP || (!DUAL && !ROPE && KSW == 1 && !kMade), "grouped code: the skinny down projection");
  // KW (one token, a made slice): the block's four waves split the K chunks of the same RTW row tiles
  // instead of taking four row tiles each: a quarter of the weight bytes per block, four times the
  // blocks (a CU streams a few tens of KB at a time; a block's 96 KB of weights was its critical path)
  static_assert(!KW || (KSW == 1 && kMade && !ROPE && !ATTN), "KW: the one-token projections without RoPE");
  constexpr int KG = KW ? 4 : KSW;  // K groups: KSW groups of four waves, or (KW) four groups of one wave
  // K chunks per wave (KW with NKC not a multiple of 4: the last waves take fewer, the wave's chunks
  // past NKC load chunk NKC - 1 again and skip their products)
  constexpr int KC = (NKC + KG - 1) / KG;
  static_assert(KW || NKC % KG == 0, "K chunks split evenly over the wave groups");
  static_assert((KG - 1) * RTW * D * 8 * 256 * (KW ? 1 : 4) <= NKC * 16 * 256 || KG == 1,
                "K-group reduction fits the slice buffer");
  // The activation slice: K chunk c's 16 token rows of 256 bytes at xs + (16 c + row) * 256 (row r's
  // 16-byte segments swizzled by ^ r).  ATTN keeps token 0's row alone (chunk c at xs + c * 256): the
  // MFMAs read it for every column, and the columns of the absent tokens are not stored.  (Its four
  // spare chunk slots take wave 3's load, so that every wave issues one: a load under a wave-dependent
  // branch made the compiler wait for every load in flight at the branch's join.)
  constexpr int kXsRows = ATTN ? 1 : 16;
  constexpr int kXsChunk = kXsRows * 256;
  __shared__ __align__(16) uint8_t xs[(ATTN ? NKC + 4 : NKC) * kXsChunk];
  // ATTN: the split's K rows (16-byte chunks of key row r at slot chunk ^ (r & 7), so that the score
  // reads of 8 consecutive lanes, 8 rows at one chunk, fall in 8 distinct bank groups), then its V rows
  constexpr int kKvRows = ATTN ? kFusedAttnChunk : 1;
  __shared__ __align__(16) float kv_lds[2 * kKvRows * QWEN_HEAD_DIM];
  __shared__ __align__(16) float q_lds[ATTN ? QWEN_HEAD_DIM : 4];  // the head's rotated q row x 1/sqrt(128)
  __shared__ __align__(16) float wacc[ATTN ? 4 * QWEN_HEAD_DIM : 4];  // per wave: acc[128], then m and l
  __shared__ float wml[ATTN ? 8 : 2];
  const int lane = threadIdx.x & 63;
  const int wave = KW ? 0 : ((threadIdx.x >> 6) & 3);        // row position of the wave
  const int kg = KW ? (threadIdx.x >> 6) : (threadIdx.x >> 8);  // K group of the wave
  const int g = lane >> 4;
  const int col = lane & 15;
  if constexpr (PRE_QUANT) {
    // with per-block maxima, the launch's last block forms the row's scale and limb sums (the
    // reduce step's correction) beside the projection blocks, which quantize only their own chunks
    // (the hot form: the block after the 8-rounded projection blocks, from the preloaded counts)
    if (HOT_KB > 0 ? (int)blockIdx.x == 8 * ((rg_count * splits + 7) / 8)
                   : (pre.amax_in && blockIdx.x == gridDim.x - 1)) {
      __shared__ float row_sx;
      __shared__ int row_sums[2];
      quant_row_slice<kQuantVecs>(pre.y, pre.in_dim, 0, 0, xs, 16 * 256, &row_sx, row_sums, pre.sx_out,
                                  pre.sums_out, NoIssue{});
      return;
    }
  }
  int rg_b, z_b, tt_b, ks = -1;  // ks: key split of an ATTN query-head block (-1: none)
  if constexpr (ATTN) {
    // ids 0..3: the k and v heads; 4..7: none; from 8 on, the six query heads of one (KV head, key split)
    // pair at ids 8 + 8 (6 (pair / 8) + j) + pair % 8, so that the blocks reading the same K/V rows share
    // an XCD (block ids are dealt to the 8 XCDs round robin)
    const int b = blockIdx.x;
    if (b < 8) {
      if (b >= 2 * QWEN_KV_HEADS) return;  // block-uniform
      rg_b = QWEN_Q_HEADS + b;
    } else {
      const int id = b - 8, kq = id >> 3;
      const int pair = (kq / QWEN_GROUPS) * 8 + (id & 7);
      if (pair >= QWEN_KV_HEADS * (HOT_KB > 0 ? hot.n0 : af.nsplit)) return;  // block-uniform: past the last pair
      ks = pair / QWEN_KV_HEADS;
      rg_b = (pair % QWEN_KV_HEADS) * QWEN_GROUPS + kq % QWEN_GROUPS;
    }
    z_b = 0;
    tt_b = 0;
  } else {
    const int xcd = blockIdx.x & 7;
    const int j = blockIdx.x >> 3;
    tt_b = j % tt_count;
    const int grp = (j / tt_count) * 8 + xcd;
    if (grp >= rg_count * splits) return;  // block-uniform: ids past the last group
    rg_b = grp % rg_count;
    z_b = grp / rg_count;
  }
  const int rg = rg_b, z = z_b, tt = tt_b;
  // (hot: one token of a fixed shape, so that nothing before the prologue's loads waits for the
  // argument segment)
  constexpr bool kHot = HOT_KB > 0;
  static_assert(!kHot || (HOT_IN > 0 && HOT_OUT > 0), "hot: the shape is fixed");
  const int nkc_all = kHot ? HOT_IN / kKChunk : a.in_dim / kKChunk;
  const int kc0 = z * NKC;
  const int tok0 = tt * 16;
  const int row_tiles = kHot ? HOT_OUT / 16 : a.out_dim / 16;
  const size_t row_stride_x = (size_t)(kHot ? HOT_IN : a.in_dim) * 2u;
  // (hot without a made slice, 1..64 tokens: HotArgs p0 the activation code, p1 the weights, p2 the up
  // matrix (DUAL) or the group scales (GRP), p3 the positions (ROPE), the groups' offset terms (GRP)
  // or the grouped code's scales out (DUAL, null without it), n0 the token count)
  constexpr bool kHotB = kHot && !kMade;
  const int n_tok = kHotB ? hot.n0 : a.tokens;
  const void* xq_p = kHotB ? hot.p0 : a.xq;
  const void* wp_p = kHotB ? hot.p1 : a.wp;
  const void* wp2_p = kHotB && DUAL ? hot.p2 : a.wp2;
  const int* pos_p = kHotB && ROPE ? static_cast<const int*>(hot.p3) : a.pos;
  const float* gsx_p = kHotB && GRP ? static_cast<const float*>(hot.p2) : a.gsx;
  const int* gcorr_p = kHotB && GRP ? static_cast<const int*>(hot.p3) : a.gcorr;
  const bool gsx_out_set = kHotB && DUAL ? hot.p3 != nullptr : a.gsx_out != nullptr;

  // activation slice -> LDS: chunk c, rows 4q..4q+3 per load (1 KiB), wave w takes chunks w, w+4KSW, ..
  // (ATTN: token 0's row of chunks 4j..4j+3 per load, wave w takes j = w, w+4, ..)
  auto issue_slice = [&]() {
    if constexpr (ATTN) {
      static_assert(NKC == 12, "three waves of four 256-byte chunk rows, wave 3 into the spare slots");
      const int j = wave;  // chunks 4j .. 4j + 3 (wave 3: a valid source, the spare slots)
      const uint8_t* src = reinterpret_cast<const uint8_t*>(a.xq) +
                           (size_t)(kc0 + min(4 * j + (lane >> 4), NKC - 1)) * 256u + (lane & 15) * 16;
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(src),
                                       (__attribute__((address_space(3))) void*)(xs + 4 * j * 256), 16, 0, 0);
      return;
    }
    for (int c = threadIdx.x >> 6; c < NKC; c += 4 * KSW) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int row = 4 * q + (lane >> 4);
        const int tok = min(tok0 + row, n_tok - 1);  // rows past the last token reload a valid row
        const int seg = (lane & 15) ^ row;
        const uint8_t* src = reinterpret_cast<const uint8_t*>(xq_p) + (size_t)tok * row_stride_x +
                             (size_t)(kc0 + c) * 256u + seg * 16;
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(src),
                                         (__attribute__((address_space(3))) void*)(xs + (c * 16 + 4 * q) * 256), 16,
                                         0, 0);
      }
    }
  };
  // decode position of this lane's token (RoPE epilogue), loaded with the weights
  // (ATTN, one token: read through the scalar cache once the weights are in flight, in issue_kv: a
  // vector load here made the compiler wait for every load in flight before its first use)
  int P = ROPE && !ATTN ? pos_p[min(tok0 + col, n_tok - 1)] : 0;
  // RoPE cos/sin of pairs p = 16*wave + 4g + q, q < 4, at position P (ATTN: loaded in issue_kv, ahead
  // of the K/V rows; otherwise after the slice barrier, in flight during the MFMAs)
  float4 rc = make_float4(1.0f, 1.0f, 1.0f, 1.0f), rs = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  auto load_rope = [&]() {
    const float* rr = a.rope + (size_t)min(max(P, 0), a.limit - 1) * 128 + 16 * wave + 4 * g;
    rc = *reinterpret_cast<const float4*>(rr);
    rs = *reinterpret_cast<const float4*>(rr + 64);
  };
  // ATTN: end of the history keys (the new key at P joins in the O projection's merge when it is a key
  // of this step, 0 <= P < max_keys; otherwise the keys are min(max(P, 0) + 1, max_keys) cache rows)
  auto hist_end = [&]() {
    const int pu = __builtin_amdgcn_readfirstlane(P);
    return pu >= 0 && pu < af.max_keys ? pu : min(max(pu, 0) + 1, af.max_keys);
  };
  // ATTN: the split's K/V rows of the head's KV head -> LDS, 16 rows per wave, two rows per load.  Every
  // block issues the same number of loads (the k and v heads and empty splits load row 0, which nobody
  // reads), so the wave's load counts stay exact; keys past the split's last one reload it (masked).
  constexpr int kKvLoads = ATTN ? 2 * (kFusedAttnChunk / 4) / 2 : 0;  // per wave: 8 of K, 8 of V
  int pos_v = 0;  // ATTN after a PRE prologue: the position, loaded among the scalars
  auto issue_kv = [&]() {
    if constexpr (ATTN) {
      // after every other load of the wave: the addresses wait for the position
      __builtin_amdgcn_sched_barrier(0);
      P = PRE ? __builtin_amdgcn_readfirstlane(pos_v) : load_uniform_i32(a.pos);
      load_rope();
      const int t0 = ks * kFusedAttnChunk;
      const int t1 = min(hist_end(), t0 + kFusedAttnChunk);
      const bool live = ks >= 0 && t1 > t0;
      const size_t hoff = (size_t)(ks >= 0 ? rg / QWEN_GROUPS : 0) * QWEN_HEAD_DIM;
      const int sl = lane & 31;
#pragma unroll
      for (int i = 0; i < kFusedAttnChunk / 8; ++i) {
        const int r0 = 16 * wave + 2 * i;  // LDS rows r0, r0 + 1 (keys t0 + r0, t0 + r0 + 1)
        const int r = r0 + (lane >> 5);
        const int key = live ? min(t0 + r, t1 - 1) : 0;
        const float* krow = a.k_cache + (size_t)key * QWEN_KV_WIDTH + hoff;
        const float* vrow = a.v_cache + (size_t)key * QWEN_KV_WIDTH + hoff;
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(krow + 4 * (sl ^ (r & 7))),
                                         (__attribute__((address_space(3))) void*)(kv_lds + r0 * QWEN_HEAD_DIM), 16,
                                         0, 0);
        __builtin_amdgcn_global_load_lds(
            reinterpret_cast<const void*>(vrow + 4 * sl),
            (__attribute__((address_space(3))) void*)(kv_lds + (kKvRows + r0) * QWEN_HEAD_DIM), 16, 0, 0);
      }
    }
  };
  uint4 wv[RTW][D][KC];
  bool ok[RTW];
  // Row tile of the wave's tile r: rg*4*RTW + wave + 4r.  A gate/up block writing the grouped code
  // takes instead the four row tiles of one K group of the down projection's input: the down
  // projection's 16x16x64 products cover, per 128-wide K chunk c, the K of row tiles 8c + {0,2,4,6}
  // (one product) and 8c + {1,3,5,7} (the other), so block rg takes tiles 8(rg/2) + 2 wave + rg%2 and
  // its 64 rows are exactly group rg.
  const bool gmap = EPI == kEpiSiluMul && DUAL && !kMade && KSW == 1 && RTW == 1 && gsx_out_set;
  auto row_tile = [&](int r) {
    return KW ? rg * RTW + r : gmap ? 8 * (rg >> 1) + 2 * wave + (rg & 1) : rg * 4 * RTW + wave + 4 * r;
  };
  float swv[RTW][4], sw2v[RTW][4], biasv[RTW][4];
  const int tok_l = kHot && kMade ? 0 : min(tok0 + col, n_tok - 1);
  float sx_l = 0.0f;
  int sh_l = 0, sl_l = 0;
  float gsv[GRP ? 2 * KC : 1];  // GRP: scales and offset terms of the lane's token's 2*KC groups
  int gcv[GRP ? 2 * KC : 1];
  // One token of the gate/up projection with K split over the waves (KW): only column 0 of the
  // products is a token, each tile's 16 rows per matrix four to a lane in lanes 0, 16, 32, 48.  The K
  // groups leave those rows in LDS and lane 16 r + i of wave 0 finishes row i of tile r: one SiLU per
  // lane, not 4 RTW in a row (its row scales loaded per lane, sw_row and sw2_row).
  constexpr bool kRowLane = KW && EPI == kEpiSiluMul && DUAL && RTW <= 4;
  const int rl_r = min(lane >> 4, RTW - 1);  // kRowLane: the lane's tile (lanes past 16 RTW repeat)
  float sw_row = 0.0f, sw2_row = 0.0f;
  // The decode SiLU's exp table, copied to LDS before the epilogue: read from constant memory there,
  // each of a lane's SiLU evaluations waited on one more memory round trip (several tokens; with one
  // token and four SiLUs per lane the copy cost as much as it saved).
  constexpr bool kTab = EPI == kEpiSiluMul && (!kMade || kRowLane);
  __shared__ uint64_t exp_tab[kTab ? 32 : 1];
  uint64_t tab_v = 0;
#pragma unroll
  for (int r = 0; r < RTW; ++r) ok[r] = row_tile(r) < row_tiles;
  // Weight tiles -> registers in K-chunk order (one 16-byte load per chunk and tile, chunk c's loads
  // before chunk c+1's), and the epilogue's per-row scales (and bias) and per-token scale and limb
  // sums: none depends on the MFMAs, and loaded after them they would cost one more round trip.
  // (A made slice waits for every load before its first MFMA, so there the loads go tile by tile:
  // each tile's chunks are one contiguous run of memory.)
  auto issue_weights = [&]() {
    if constexpr (kMade) {
#pragma unroll
      for (int r = 0; r < RTW; ++r) {
        const int rt = row_tile(r);
        const size_t base = ((size_t)(ok[r] ? rt : 0) * nkc_all + kc0) * 64u + lane;
#pragma unroll
        for (int d = 0; d < D; ++d) {
          const uint4* wp = reinterpret_cast<const uint4*>(d ? wp2_p : wp_p) + base;
#pragma unroll
          for (int c = 0; c < KC; ++c) wv[r][d][c] = wp[(size_t)min(kg * KC + c, NKC - 1) * 64u];
        }
      }
    } else {
#pragma unroll
      for (int c = 0; c < KC; ++c)
#pragma unroll
        for (int r = 0; r < RTW; ++r) {
          const int rt = row_tile(r);
          const size_t base = ((size_t)(ok[r] ? rt : 0) * nkc_all + kc0 + kg * KC + c) * 64u + lane;
#pragma unroll
          for (int d = 0; d < D; ++d)  // cached: reused by the XCD's other token tiles
            wv[r][d][c] = reinterpret_cast<const uint4*>(d ? wp2_p : wp_p)[base];
        }
    }
  };
  auto issue_groups = [&]() {
    if constexpr (GRP) {
      static_assert((2 * KC) % 4 == 0, "groups in float4 loads");
      // 16-byte aligned: KC even, in_dim % 256 == 0
      const size_t gb = (size_t)tok_l * ((kHot ? HOT_IN : a.in_dim) / 64) + 2 * (kc0 + kg * KC);
#pragma unroll
      for (int i = 0; i < 2 * KC; i += 4) {
        const float4 s4 = *reinterpret_cast<const float4*>(gsx_p + gb + i);
        const int4 c4 = *reinterpret_cast<const int4*>(gcorr_p + gb + i);
        gsv[i] = s4.x, gsv[i + 1] = s4.y, gsv[i + 2] = s4.z, gsv[i + 3] = s4.w;
        gcv[i] = c4.x, gcv[i + 1] = c4.y, gcv[i + 2] = c4.z, gcv[i + 3] = c4.w;
      }
    }
  };
  auto issue_scalars = [&]() {
    // The bias is loaded unconditionally (the row scales stand in when there is none, masked to +0
    // by their bits, which leaves the epilogue's arithmetic as it is): a load under a run-time
    // condition is a branch, after which the compiler waits for every load in flight, so each of
    // them would be a memory round trip of its own.
    constexpr bool kBias = EPI == kEpiStore && !DUAL;
    const float* bsrc = kBias && a.bias ? a.bias : a.sw;
    const uint32_t bmask = kBias && a.bias ? 0xFFFFFFFFu : 0u;
    if constexpr (kRowLane) {
      const int rt = row_tile(rl_r);
      const int row = (rt < row_tiles ? rt : 0) * 16 + (lane & 15);
      sw_row = a.sw[row];
      sw2_row = a.sw2[row];
    } else {
#pragma unroll
      for (int r = 0; r < RTW; ++r) {
        const int row0 = (ok[r] ? row_tile(r) : 0) * 16 + 4 * g;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          swv[r][q] = a.sw[row0 + q];
          sw2v[r][q] = DUAL ? a.sw2[row0 + q] : 0.0f;
          biasv[r][q] = kBias ? __uint_as_float(__float_as_uint(bsrc[row0 + q]) & bmask) : 0.0f;
        }
      }
    }
    if constexpr (!kMade) {
      sx_l = a.sx[tok_l];
      sh_l = a.sums[2 * tok_l];
      sl_l = a.sums[2 * tok_l + 1];
    }
    if constexpr (GRP && !kHotB) issue_groups();
    if constexpr (kTab) tab_v = kExp2Tab[lane & 31];
    if constexpr (ATTN && PRE) {
      int lz;
      asm volatile("v_mov_b32 %0, 0" : "=v"(lz));  // a vector load: the scalar one waited on lgkmcnt
      pos_v = a.pos[lz];
    }
  };
  // With a made slice (kMade) the weights and scalars are issued inside the prologue, after the
  // prologue's own loads: a wave's loads return in order, so the prologue's few loads must not queue
  // behind the weights.
  // (ATTN after a PRE prologue: the RoPE and K/V rows are issued once the prologue is done and every
  // other load has landed.  The K/V rows are direct loads into LDS, and while one is in flight the
  // compiler waits for every load before any use of a loaded register: issued with the weights, the
  // prologue's first add waited for the whole weight stream, and with it the norm and quantization.)
  auto issue_loads = [&]() {
    if constexpr (HOT_KB > 0) kernarg_lines_wait(klines);  // the prologue's loads are in flight
    issue_weights();
    issue_scalars();
    if constexpr (!(ATTN && PRE)) issue_kv();
  };
  __shared__ float pre_sx;
  __shared__ int pre_sums[8];  // the made slice's limb sums: per-wave partials (wave_sums_total)
  int2 pre_tot = make_int2(0, 0);  // their totals, read after the slice barrier
  if constexpr (PRE_ATTN)
    attn_merge_quant_slice<NEWKEY, MKF, NKC, kHot>(am, z * NKC, xs, kXsChunk, &pre_sx, pre_sums,
                                                   NKC == QWEN_Q_HEADS && blockIdx.x == 0, issue_loads, hot);
  if constexpr (PRE_QUANT) {
    // token 0's row of the slice: K chunks kc0 .. kc0 + NKC - 1 (row 0 of each chunk, unswizzled)
    if constexpr (HOT_KB > 0)  // hot: the row and its per-block maxima (preloaded)
      quant_chunks_from_maxima(static_cast<const float*>(hot.p0), static_cast<const float*>(hot.p1), hot.n0, kc0,
                               NKC, xs, 16 * 256, &pre_sx, pre_sums, issue_loads);
    else if (pre.amax_in)
      quant_chunks_from_maxima(pre.y, pre.amax_in, pre.amax_n, kc0, NKC, xs, 16 * 256, &pre_sx, pre_sums,
                               issue_loads);
    else
      quant_row_slice<kQuantVecs>(pre.y, pre.in_dim, kc0, NKC, xs, 16 * 256, &pre_sx, pre_sums,
                                  blockIdx.x == 0 ? pre.sx_out : nullptr, pre.sums_out, issue_loads);
    if (threadIdx.x < 6) pre_sums[2 + threadIdx.x] = 0;  // the totals in [0], [1] (wave_sums_total)
  }
  if constexpr (PRE) {
    // token 0's row of the slice (K chunk c at xs + c * kXsChunk, row 0 of the chunk, unswizzled), made
    // by the block's four waves together (two block barriers): the O projection's K groups (store
    // epilogue) or the down projection's five splits (residual).  (One wave alone, with the other
    // three issuing their loads, took 2.2 us of arithmetic on the launch's critical path.)
    reduce_norm_quant_row_w4<PRE_EPI, PRE_EPI == kEpiResidual ? kPreResidualSplits : kOneTokenOSplits, kHot>(
        pre, pre_splits, reinterpret_cast<int8_t*>(xs), kXsChunk, &pre_sx, pre_sums, blockIdx.x == 0 && pre.y,
        issue_loads, hot);
  }
  if constexpr (kMade) {
    __builtin_amdgcn_sched_barrier(0);  // every load above is in flight before any use
    if constexpr (ATTN && PRE) {
      wait_vmcnt<0>();  // the weights and the position: the MFMAs then wait for nothing
      issue_kv();       // the RoPE and K/V rows land during the MFMAs
      // the slice's LDS writes are complete before the barrier (a __syncthreads here would also wait
      // for the direct loads into LDS just issued)
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
    } else {
      wait_vmcnt<kKvLoads>();  // ATTN: the K/V rows (the wave's last loads) land during the MFMAs
      __syncthreads();
    }
    pre_tot = wave_sums_total(pre_sums);
  } else {
    // Scalars, then the activation slice, then the weights in chunk order.  A wave's loads return in
    // order, so once at most the weight loads are outstanding its part of the slice has landed, and
    // after the barrier the whole slice has; chunk c's MFMAs then wait only for chunk c's weights
    // (the compiler's own waits on the weight registers), so the MFMAs run under the weight stream.
    if constexpr (kHotB) {
      // hot: the slice, the groups and the weights from the preloaded operands, then (once the
      // argument segment has landed) the epilogue's scalars; at least the weight and K/V loads were
      // issued after the slice
      issue_slice();
      issue_groups();
      issue_weights();
      __builtin_amdgcn_sched_barrier(0);  // (else the wait and the epilogue's addressing move above them)
      kernarg_lines_wait(klines);
      issue_scalars();
      issue_kv();
      __builtin_amdgcn_sched_barrier(0);
      wait_vmcnt<RTW * D * KC + kKvLoads>();
    } else {
      issue_scalars();
      issue_slice();
      issue_weights();
      issue_kv();
      __builtin_amdgcn_sched_barrier(0);  // every load above is in flight before any use
      wait_vmcnt<RTW * D * KC + (ATTN ? 2 : 0) + kKvLoads>();
    }
    if (kTab && threadIdx.x < 32) exp_tab[threadIdx.x] = tab_v;
    if (kTab) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the table store lands before the barrier
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);  // the slice reads below stay after the barrier
  }

  // RoPE cos/sin of pairs p = 16*wave + 4g + q, q < 4, at position P: in flight during the MFMAs.
  // Loaded by every lane at a clamped position (rope_in selects their use): under a run-time
  // condition the load is a branch, whose join waited for every load in flight, the weight stream
  // included, before the first MFMA.
  const bool rope_in = ROPE && P >= 0 && P < a.limit;
  if constexpr (ROPE && !ATTN) load_rope();
  v4i accH[RTW][D], accL[RTW][D];
  constexpr bool kPair = (kMade || ATTN) && !GRP;  // one token
#pragma unroll
  for (int r = 0; r < RTW; ++r)
#pragma unroll
    for (int d = 0; d < D; ++d) accH[r][d] = accL[r][d] = v4i{0, 0, 0, 0};
  float gacc[GRP ? RTW : 1][4] = {};  // GRP: sum over groups of scale * (exact group dot product)
  v4i gprod[2][GRP ? RTW : 1][4];     // GRP: products of two chunks in flight
#pragma unroll
  for (int c = 0; c < KC; ++c) {
    if constexpr (GRP) {
      // chunk c+1's products are issued before chunk c's are consumed, so each conversion works on
      // products that have already left the matrix cores
      auto products = [&](int cc, v4i (&p)[RTW][4]) {
        const uint8_t* xr = xs + ((kg * KC + cc) * 16 + col) * 256;
        const v4i bh1 = *reinterpret_cast<const v4i*>(xr + (((2 * g) ^ col) << 4));
        const v4i bh2 = *reinterpret_cast<const v4i*>(xr + (((2 * g + 1) ^ col) << 4));
        const v4i bl1 = *reinterpret_cast<const v4i*>(xr + (((8 + 2 * g) ^ col) << 4));
        const v4i bl2 = *reinterpret_cast<const v4i*>(xr + (((9 + 2 * g) ^ col) << 4));
#pragma unroll
        for (int r = 0; r < RTW; ++r) {
          v4i a1, a2;
          unpack16(wv[r][0][cc], a1, a2);
          const v4i z = v4i{0, 0, 0, 0};
          p[r][0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, bh1, z, 0, 0, 0);  // group 2cc, H limbs
          p[r][1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, bl1, z, 0, 0, 0);  // group 2cc, L limbs
          p[r][2] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a2, bh2, z, 0, 0, 0);  // group 2cc+1
          p[r][3] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a2, bl2, z, 0, 0, 0);
        }
      };
      if (c == 0) products(0, gprod[0]);
      if (c + 1 < KC) products(c + 1, gprod[(c + 1) & 1]);
      const v4i (&p)[RTW][4] = gprod[c & 1];
#pragma unroll
      for (int r = 0; r < RTW; ++r)
#pragma unroll
        for (int q = 0; q < 4; ++q)  // the group's integer dot product, exact in int32 (< 2^26), then fp32
          gacc[r][q] += gsv[2 * c] * (float)(p[r][0][q] * 256 + p[r][1][q] - 8 * gcv[2 * c]) +
                        gsv[2 * c + 1] * (float)(p[r][2][q] * 256 + p[r][3][q] - 8 * gcv[2 * c + 1]);
      // each chunk's products are consumed in its iteration: without an accumulator chain the compiler
      // would issue every chunk's MFMAs first and hold all their results
#pragma unroll
      for (int r = 0; r < RTW; ++r)
#pragma unroll
        for (int q = 0; q < 4; ++q) asm volatile("" : "+v"(gacc[r][q]));
      __builtin_amdgcn_sched_barrier(0);
      continue;
    }
    if (KW && NKC % KG != 0 && kg * KC + c >= NKC) break;  // wave-uniform: the wave's chunks past NKC
    if constexpr (kPair) {
      // One token (a made slice, or ATTN): its two limbs go in as two columns of one product, the H
      // limbs in the even columns and the L limbs in the odd ones, so a chunk takes two products per
      // tile and matrix instead of four (the 16 columns would otherwise all hold the one token, or
      // nothing).  accH takes the chunk's first 64 K and accL its second 64 (two accumulator chains);
      // their sum's columns 0 and 1 are the token's H and L sums.
      const uint8_t* xr = xs + (kg * KC + c) * kXsChunk;  // row 0 of the chunk, unswizzled
      const int sb = (col & 1) << 3;
      const v4i b1 = *reinterpret_cast<const v4i*>(xr + ((sb + 2 * g) << 4));
      const v4i b2 = *reinterpret_cast<const v4i*>(xr + ((sb + 2 * g + 1) << 4));
#pragma unroll
      for (int r = 0; r < RTW; ++r)
#pragma unroll
        for (int d = 0; d < D; ++d) {
          v4i a1, a2;
          unpack16(wv[r][d][c], a1, a2);
          accH[r][d] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1, accH[r][d], 0, 0, 0);
          accL[r][d] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a2, b2, accL[r][d], 0, 0, 0);
        }
      continue;
    }
    const int colr = ATTN ? 0 : col;  // ATTN: every column reads token 0's row
    const uint8_t* xr = xs + ((kg * KC + c) * kXsRows + colr) * 256;
    const v4i bh1 = *reinterpret_cast<const v4i*>(xr + (((2 * g) ^ colr) << 4));
    const v4i bh2 = *reinterpret_cast<const v4i*>(xr + (((2 * g + 1) ^ colr) << 4));
    const v4i bl1 = *reinterpret_cast<const v4i*>(xr + (((8 + 2 * g) ^ colr) << 4));
    const v4i bl2 = *reinterpret_cast<const v4i*>(xr + (((9 + 2 * g) ^ colr) << 4));
#pragma unroll
    for (int r = 0; r < RTW; ++r)
#pragma unroll
      for (int d = 0; d < D; ++d) {
        v4i a1, a2;
        unpack16(wv[r][d][c], a1, a2);
        accH[r][d] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, bh1, accH[r][d], 0, 0, 0);
        accH[r][d] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a2, bh2, accH[r][d], 0, 0, 0);
        accL[r][d] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, bl1, accL[r][d], 0, 0, 0);
        accL[r][d] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a2, bl2, accL[r][d], 0, 0, 0);
      }
  }
  if constexpr (kPair) {
    // column 0 of the sum: the H sums; column 1 (the lane to the right): the L sums
#pragma unroll
    for (int r = 0; r < RTW; ++r)
#pragma unroll
      for (int d = 0; d < D; ++d)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int t = accH[r][d][q] + accL[r][d][q];
          accH[r][d][q] = t;
          accL[r][d][q] = dpp_i<0xB1>(t);
        }
  }

  if constexpr (kRowLane) {
    __syncthreads();  // every wave's slice reads are done: the slice buffer takes the sums
    // [K group][tile r][matrix d][limb][row 0..15], exact int32
    int* red = reinterpret_cast<int*>(xs);
    constexpr int kPerKg = RTW * D * 2 * 16;
    if (col == 0) {
#pragma unroll
      for (int r = 0; r < RTW; ++r)
#pragma unroll
        for (int d = 0; d < D; ++d) {
          int* dst = red + kg * kPerKg + ((r * D + d) * 2) * 16 + 4 * g;
          *reinterpret_cast<int4*>(dst) = make_int4(accH[r][d][0], accH[r][d][1], accH[r][d][2], accH[r][d][3]);
          *reinterpret_cast<int4*>(dst + 16) = make_int4(accL[r][d][0], accL[r][d][1], accL[r][d][2], accL[r][d][3]);
        }
    }
    if (threadIdx.x < 32) exp_tab[threadIdx.x] = tab_v;
    __syncthreads();
    if (kg > 0) return;
    const int row = lane & 15;  // of tile rl_r; lanes past 16 RTW repeat rows (no stores)
    int hs[2] = {0, 0}, ls[2] = {0, 0};
#pragma unroll
    for (int j = 0; j < KG; ++j)
#pragma unroll
      for (int d = 0; d < D; ++d) {
        const int* src = red + j * kPerKg + ((rl_r * D + d) * 2) * 16 + row;
        hs[d] += src[0];
        ls[d] += src[16];
      }
    const double sx = (double)pre_sx;
    const int sh8 = 8 * pre_tot.x, sl8 = 8 * pre_tot.y;
    const float v = (float)(((double)(hs[0] - sh8) * 256.0 + (double)(ls[0] - sl8)) * sx) * sw_row;
    const float u = (float)(((double)(hs[1] - sh8) * 256.0 + (double)(ls[1] - sl8)) * sx) * sw2_row;
    const float yv = silu_decode(v, exp_tab) * u;
    const bool live = row_tile(rl_r) < row_tiles;
    if (lane < 16 * RTW && live) a.y[(size_t)tok0 * a.y_stride + row_tile(rl_r) * 16 + row] = yv;
    if (a.amax_out) {  // max |SiLU.up| of the block's rows: DPP row maxima of lanes 16 r .. 16 r + 15
      float m = live ? fmaxf(0.0f, fabsf(yv)) : 0.0f;
      m = fmaxf(m, __int_as_float(dpp_i<0xB1>(__float_as_int(m))));
      m = fmaxf(m, __int_as_float(dpp_i<0x4E>(__float_as_int(m))));
      m = fmaxf(m, __int_as_float(dpp_i<0x124>(__float_as_int(m))));
      m = fmaxf(m, __int_as_float(dpp_i<0x128>(__float_as_int(m))));
#pragma unroll
      for (int r = 1; r < RTW; ++r) m = fmaxf(m, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 16 * r)));
      if (lane == 0) a.amax_out[rg] = m;
    }
    return;
  }

  if constexpr (KG > 1 && !kRowLane) {
    // K groups 1.. hand their exact int32 sums to K group 0 through LDS (the slice buffer, now read):
    // region (row wave, or with KW the K group's) of RTW * D * 8 * 64 ints each.
    __syncthreads();
    constexpr int kRegion = RTW * D * 8 * 64;
    int* red = reinterpret_cast<int*>(xs) + lane;
    if (kg > 0) {
      int* mine = red + (KW ? kg - 1 : wave) * kRegion;
#pragma unroll
      for (int r = 0; r < RTW; ++r)
#pragma unroll
        for (int d = 0; d < D; ++d)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            mine[((r * D + d) * 8 + q) * 64] = accH[r][d][q];
            mine[((r * D + d) * 8 + 4 + q) * 64] = accL[r][d][q];
          }
    }
    __syncthreads();
    if (kg > 0) return;
#pragma unroll
    for (int j = 1; j < KG; ++j) {
      const int* theirs = red + (KW ? j - 1 : wave) * kRegion;
#pragma unroll
      for (int r = 0; r < RTW; ++r)
#pragma unroll
        for (int d = 0; d < D; ++d)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            accH[r][d][q] += theirs[((r * D + d) * 8 + q) * 64];
            accL[r][d][q] += theirs[((r * D + d) * 8 + 4 + q) * 64];
          }
    }
  }

  if constexpr (EPI == kEpiSiluMul && DUAL && !kMade && KSW == 1 && RTW == 1) {
    if (a.gsx_out) {
      // Grouped code of the SiLU·up rows for the down projection: the block's 64 rows (rows 64rg..,
      // K group rg of the down projection's input) of each of its tokens are quantized with the group's
      // own maximum, by the row quantizer's arithmetic (X = clip(rint(s * 32512 / max)), limbs
      // H = (X + 128) >> 8 and L = X - 256 H), and written with the group's scale and offset term.
      __shared__ float gq_max[4][16];
      __shared__ int gq_h[4][16], gq_l[4][16];
      const int tok = tok0 + col;
      const bool valid = tok < a.tokens && ok[0];
      const int row0 = row_tile(0) * 16 + 4 * g;
      const int sh8 = 8 * sh_l, sl8 = 8 * sl_l;
      const double sx = (double)sx_l;
      float s[4], m = 0.0f;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const double tot = (double)(accH[0][0][q] - sh8) * 256.0 + (double)(accL[0][0][q] - sl8);
        const double tot2 = (double)(accH[0][1][q] - sh8) * 256.0 + (double)(accL[0][1][q] - sl8);
        const float v = (float)(tot * sx) * swv[0][q];
        const float u = (float)(tot2 * sx) * sw2v[0][q];
        const float sg = a.prefill_silu ? silu_prefill(v) : silu_decode(v, kTab ? exp_tab : kExp2Tab);
        s[q] = valid ? sg * u : 0.0f;
        m = fmaxf(m, fabsf(s[q]));
      }
      m = fmaxf(m, __shfl_xor(m, 16, 64));  // over the wave's 16 rows of the token (g)
      m = fmaxf(m, __shfl_xor(m, 32, 64));
      if (g == 0) gq_max[wave][col] = m;
      __syncthreads();
      const float amax = fmaxf(fmaxf(gq_max[0][col], gq_max[1][col]), fmaxf(gq_max[2][col], gq_max[3][col]));
      const float inv = amax > 0.0f ? (float)kQuantMax / amax : 0.0f;
      uint32_t hw = 0, lw = 0;
      int sh = 0, sl = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float xf = fminf(fmaxf(rintf(s[q] * inv), -(float)kQuantMax), (float)kQuantMax);
        const int X = (int)xf;
        const int H = (X + 128) >> 8;
        const int L = X - (H << 8);
        hw |= (uint32_t)(H & 0xFF) << (8 * q);
        lw |= (uint32_t)(L & 0xFF) << (8 * q);
        sh += H;
        sl += L;
      }
      sh += __shfl_xor(sh, 16, 64);
      sh += __shfl_xor(sh, 32, 64);
      sl += __shfl_xor(sl, 16, 64);
      sl += __shfl_xor(sl, 32, 64);
      if (g == 0) {
        gq_h[wave][col] = sh;
        gq_l[wave][col] = sl;
      }
      __syncthreads();
      if (valid) {  // limbs of K = row0 .. row0+3: chunk row0 / 128, H at +0, L at +128
        int8_t* dst = a.xq_out + (size_t)tok * (2 * (size_t)a.out_dim) + (row0 >> 7) * 256 + (row0 & 127);
        *reinterpret_cast<uint32_t*>(dst) = hw;
        *reinterpret_cast<uint32_t*>(dst + 128) = lw;
      }
      if (wave == 0 && g == 0 && tok < a.tokens) {
        const size_t gi = (size_t)tok * (a.out_dim / 64) + rg;
        a.gsx_out[gi] = amax > 0.0f ? amax / (float)kQuantMax : 1.0f;
        a.gcorr_out[gi] = 256 * (gq_h[0][col] + gq_h[1][col] + gq_h[2][col] + gq_h[3][col]) +
                          (gq_l[0][col] + gq_l[1][col] + gq_l[2][col] + gq_l[3][col]);
      }
      return;
    }
  }

  // epilogue: lane holds rows 16*rt + 4g + q (q < 4) of token tok0 + col
  const int tok = tok0 + col;
  if (!ATTN && tok >= a.tokens) return;  // ATTN: every lane goes on to the attention (stores guarded)
  const double sx = (double)(kMade ? pre_sx : sx_l);
  const bool partial = splits > 1 || (!DUAL && !ROPE && a.fuse != kFuseNone);
  if (partial) {
    // PRE_ATTN over a range of heads: the range has its own scale and limb sums, so its partial takes
    // its own offset correction (the reduce step then adds the partials with a zero correction)
    constexpr bool kOwnCorr = PRE_ATTN && NKC * kKChunk < QWEN_HIDDEN;
    const int ch8 = kOwnCorr ? 8 * pre_tot.x : 0, cl8 = kOwnCorr ? 8 * pre_tot.y : 0;
#pragma unroll
    for (int r = 0; r < RTW; ++r) {
      if (!ok[r]) continue;
      const int row0 = row_tile(r) * 16 + 4 * g;
      float out[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        out[q] = GRP ? gacc[r][q] * swv[r][q]
                     : (float)(((double)(accH[r][0][q] - ch8) * 256.0 + (double)(accL[r][0][q] - cl8)) * sx) *
                           swv[r][q];
      *reinterpret_cast<float4*>(a.part + ((size_t)z * a.tokens + tok) * a.out_dim + row0) =
          make_float4(out[0], out[1], out[2], out[3]);
    }
    return;
  }
  const int sh8 = 8 * (kMade ? pre_tot.x : sh_l);
  const int sl8 = 8 * (kMade ? pre_tot.y : sl_l);
  float y[RTW][4];
#pragma unroll
  for (int r = 0; r < RTW; ++r) {
    const int row0 = row_tile(r) * 16 + 4 * g;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (!ok[r]) {
        y[r][q] = 0.0f;
        continue;
      }
      const double tot = (double)(accH[r][0][q] - sh8) * 256.0 + (double)(accL[r][0][q] - sl8);
      const float v = (float)(tot * sx) * swv[r][q];
      if (EPI == kEpiSiluMul) {
        const double tot2 = (double)(accH[r][D - 1][q] - sh8) * 256.0 + (double)(accL[r][D - 1][q] - sl8);
        const float u = (float)(tot2 * sx) * sw2v[r][q];
        const float sg = a.prefill_silu ? silu_prefill(v) : silu_decode(v, kTab ? exp_tab : kExp2Tab);
        y[r][q] = sg * u;
      } else if (EPI == kEpiResidual) {
        y[r][q] = a.resid[(size_t)tok * a.resid_stride + row0 + q] + v;
      } else {
        y[r][q] = v + biasv[r][q];
      }
    }
  }
  if constexpr (ROPE) {
    // rows p (tile r=0) and p + 64 (tile r=1) of head rg, p = 16*wave + 4g + q: 12 q heads, then 2 k
    // heads, then 2 v heads; each lane writes 4 consecutive p as one float4 per half.
    const int head = rg;
    const float c4[4] = {rc.x, rc.y, rc.z, rc.w}, s4[4] = {rs.x, rs.y, rs.z, rs.w};
    float lo[4], hi[4];
    const bool rotate = head < QWEN_Q_HEADS + QWEN_KV_HEADS && rope_in;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float e = y[0][q], od = y[1][q];
      lo[q] = rotate ? e * c4[q] - od * s4[q] : e;
      hi[q] = rotate ? od * c4[q] + e * s4[q] : od;
    }
    const int p0 = 16 * wave + 4 * g;
    float* dst = nullptr;
    if (head < QWEN_Q_HEADS) {
      dst = a.y + (size_t)tok * a.y_stride + head * QWEN_HEAD_DIM + p0;
    } else if (rope_in) {
      const size_t cache_row = (size_t)tok * a.seq_stride + (size_t)P * QWEN_KV_WIDTH;
      dst = head < QWEN_Q_HEADS + QWEN_KV_HEADS
                ? a.k_cache + cache_row + (head - QWEN_Q_HEADS) * QWEN_HEAD_DIM + p0
                : a.v_cache + cache_row + (head - QWEN_Q_HEADS - QWEN_KV_HEADS) * QWEN_HEAD_DIM + p0;
    }
    if constexpr (ATTN) {
      if (head < QWEN_Q_HEADS && tok < a.tokens) {
        constexpr float kScale = 0.08838834764831845f;  // 1/sqrt(128), as attn_decode_kernel scales q
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          q_lds[p0 + q] = lo[q] * kScale;
          q_lds[p0 + 64 + q] = hi[q] * kScale;
        }
      }
      if (tok >= a.tokens || ks > 0) dst = nullptr;  // split 0 stores the q row (the merge's new-key term)
      if (head >= QWEN_Q_HEADS && tok < a.tokens) {  // the k and v rows also go to the token's row
        float* yr = a.y + (size_t)tok * a.y_stride + head * QWEN_HEAD_DIM + p0;
        *reinterpret_cast<float4*>(yr) = make_float4(lo[0], lo[1], lo[2], lo[3]);
        *reinterpret_cast<float4*>(yr + 64) = make_float4(hi[0], hi[1], hi[2], hi[3]);
      }
    }
    if (dst) {
      *reinterpret_cast<float4*>(dst) = make_float4(lo[0], lo[1], lo[2], lo[3]);
      *reinterpret_cast<float4*>(dst + 64) = make_float4(hi[0], hi[1], hi[2], hi[3]);
    }
    if constexpr (ATTN) {
      // The attention of query head rg over history keys [t0, t1) of this split (the new key joins in
      // the O projection's merge).  Wave w takes keys t0 + 16w .. + 15: lane (key k = lane & 15, dim
      // quarter lane >> 4) forms a quarter of the score, the quarters meet by shuffles; then the wave's
      // online-softmax state over its 16 keys and P.V for dims 2 lane, 2 lane + 1.
      // every wave waits for its K/V loads into LDS before it ends, the blocks without keys included
      wait_vmcnt<0>();
      if (ks < 0) return;  // the k and v heads
      const int t0 = ks * kFusedAttnChunk;
      const int t1 = min(hist_end(), t0 + kFusedAttnChunk);
      if (t1 <= t0) return;  // block-uniform: no history key in this split
      __syncthreads();       // every wave's K/V rows and the q row are visible
      const int kk = lane & 15, qd = lane >> 4;
      const int r = 16 * wave + kk;
      const float* krow = kv_lds + r * QWEN_HEAD_DIM;
      float sc = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int jc = qd * 8 + i;  // 16-byte chunk: dims 4 jc .. 4 jc + 3
        const float4 k4 = *reinterpret_cast<const float4*>(krow + 4 * (jc ^ (r & 7)));
        const float4 q4 = *reinterpret_cast<const float4*>(q_lds + 4 * jc);
        sc += q4.x * k4.x + q4.y * k4.y + q4.z * k4.z + q4.w * k4.w;
      }
      sc += __shfl_xor(sc, 16, 64);
      sc += __shfl_xor(sc, 32, 64);
      if (t0 + r >= t1) sc = -INFINITY;
      // every row of 16 lanes now holds the wave's 16 scores: maximum and sum by DPP row steps, the
      // weights to every lane by readlane (lane k2 holds key k2's)
      auto dppf = [](float v, auto ctrl) { return __int_as_float(dpp_i<decltype(ctrl)::value>(__float_as_int(v))); };
      using C1 = std::integral_constant<int, 0xB1>;   // quad_perm: lanes ^ 1
      using C2 = std::integral_constant<int, 0x4E>;   // quad_perm: lanes ^ 2
      using C4 = std::integral_constant<int, 0x124>;  // row_ror:4
      using C8 = std::integral_constant<int, 0x128>;  // row_ror:8
      float m = sc;
      m = fmaxf(m, dppf(m, C1{}));
      m = fmaxf(m, dppf(m, C2{}));
      m = fmaxf(m, dppf(m, C4{}));
      m = fmaxf(m, dppf(m, C8{}));
      const float pr = m == -INFINITY ? 0.0f : __expf(sc - m);  // a wave without keys: weight 0
      float l = pr;
      l += dppf(l, C1{});
      l += dppf(l, C2{});
      l += dppf(l, C4{});
      l += dppf(l, C8{});
      float a0 = 0.0f, a1 = 0.0f;
      const float* vb = kv_lds + (kKvRows + 16 * wave) * QWEN_HEAD_DIM + 2 * lane;
#pragma unroll
      for (int k2 = 0; k2 < 16; ++k2) {
        const float pk = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pr), k2));
        const float2 v2 = *reinterpret_cast<const float2*>(vb + k2 * QWEN_HEAD_DIM);
        a0 += pk * v2.x;
        a1 += pk * v2.y;
      }
      *reinterpret_cast<float2*>(wacc + wave * QWEN_HEAD_DIM + 2 * lane) = make_float2(a0, a1);
      if (lane == 0) {
        wml[2 * wave] = m;
        wml[2 * wave + 1] = l;
      }
      __syncthreads();
      if (threadIdx.x < QWEN_HEAD_DIM) {
        const int d = threadIdx.x;
        const float M = fmaxf(fmaxf(wml[0], wml[2]), fmaxf(wml[4], wml[6]));  // finite: key t0 is in wave 0
        float L = 0.0f, A = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float f = wml[2 * w] == -INFINITY ? 0.0f : __expf(wml[2 * w] - M);
          L += wml[2 * w + 1] * f;
          A += wacc[w * QWEN_HEAD_DIM + d] * f;
        }
        af.part[((size_t)rg * af.nsplit + ks) * QWEN_HEAD_DIM + d] = A;
        if (d == 0) af.pml[(size_t)rg * af.nsplit + ks] = make_float2(M, L);
      }
    }
  } else {
#pragma unroll
    for (int r = 0; r < RTW; ++r) {
      if (!ok[r]) continue;
      const int row0 = row_tile(r) * 16 + 4 * g;
      float o[4] = {y[r][0], y[r][1], y[r][2], y[r][3]};
      if (EPI == kEpiResidual && a.y_raw)
        *reinterpret_cast<float4*>(a.y_raw + (size_t)tok * a.y_stride + row0) = make_float4(o[0], o[1], o[2], o[3]);
      if (EPI == kEpiResidual && a.round_bf16)
#pragma unroll
        for (int q = 0; q < 4; ++q) o[q] = round_bf16(o[q]);
      *reinterpret_cast<float4*>(a.y + (size_t)tok * a.y_stride + row0) = make_float4(o[0], o[1], o[2], o[3]);
    }
    if constexpr (KW && EPI == kEpiSiluMul && !kRowLane) {
      if (a.amax_out) {  // max |SiLU.up| of the block's rows (lanes 0, 16, 32, 48 hold token 0's)
        float m = 0.0f;
#pragma unroll
        for (int r = 0; r < RTW; ++r)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (ok[r]) m = fmaxf(m, fabsf(y[r][q]));
        m = fmaxf(m, __shfl_xor(m, 16, 64));
        m = fmaxf(m, __shfl_xor(m, 32, 64));
        if (lane == 0) a.amax_out[rg] = m;
      }
    }
  }
}

template <int RTW, bool DUAL, int EPI, int NKC, bool ROPE, int KSW, bool GRP = false>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(3)))
gemm_skinny_kernel(GemmArgs a, int tt_count, int rg_count, int splits) {
  touch_kernargs<kernarg_bytes<GemmArgs, int, int, int>()>();
  gemm_skinny_body<RTW, DUAL, EPI, NKC, ROPE, KSW, false, kEpiStore, false, false, GRP>(a, tt_count, rg_count, splits,
                                                                                      a, 0);
}

// The same for the model's shapes (IN -> OUT) with the operands of the first loads preloaded (HotArgs:
// the activation code, the weights, the up matrix or group scales, the positions, offset terms or
// grouped code's scales out, then the counts).
template <int RTW, bool DUAL, int EPI, int NKC, bool ROPE, int KSW, bool GRP, int IN, int OUT>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(3)))
gemm_skinny_hot_kernel(const void* p0, const void* p1, const void* p2, const void* p3, int tokens, int tt_count,
                       int rg_count, int splits, GemmArgs a) {
  constexpr int kKb = kernarg_bytes<const void*, const void*, const void*, const void*, int, int, int, int, GemmArgs>();
  gemm_skinny_body<RTW, DUAL, EPI, NKC, ROPE, KSW, false, kEpiStore, false, false, GRP, false, false, false, 16, kKb,
                   IN, OUT>(a, tt_count, rg_count, splits, a, 0, AttnMergeArgs{}, AttnFuseArgs{},
                            HotArgs{p0, p1, p2, p3, nullptr, nullptr, tokens});
}

// One token, the activation row quantized by every block for its own K chunks (see PRE_QUANT above;
// KW: the block's waves split K).
template <int RTW, int EPI, int NKC, bool KW = false>
__global__ void __launch_bounds__(256) gemm_skinny_preq_kernel(GemmArgs a, int rg_count, int splits, GemmArgs pre) {
  touch_kernargs<kernarg_bytes<GemmArgs, int, int, GemmArgs>()>();
  gemm_skinny_body<RTW, false, EPI, NKC, false, 1, false, kEpiStore, true, false, false, false, false, KW>(
      a, 1, rg_count, splits, pre, 0);
}

// The same with the operands of the prologue's first loads preloaded: the SiLU·up row, its per-block
// maxima and their count, then the block mapping's counts (HotArgs).
template <int RTW, int EPI, int NKC>
__global__ void __launch_bounds__(256) gemm_skinny_preq_hot_kernel(const float* y, const float* amax_in, int amax_n,
                                                                   int rg_count, int splits, GemmArgs a, GemmArgs pre) {
  constexpr int kKb = kernarg_bytes<const float*, const float*, int, int, int, GemmArgs, GemmArgs>();
  gemm_skinny_body<RTW, false, EPI, NKC, false, 1, false, kEpiStore, true, false, false, false, false, true, 16, kKb,
                   QWEN_INTERMEDIATE, QWEN_HIDDEN>(
      a, 1, rg_count, splits, pre, 0, AttnMergeArgs{}, AttnFuseArgs{}, HotArgs{y, amax_in, nullptr, nullptr, nullptr, nullptr, amax_n});
}

// One token whose activation row is the decode attention's context: every block merges the split
// partials and quantizes the row (see PRE_ATTN above; NEWKEY: with the new key's own term).
// (K split over the block's waves, 1536 x 1536; the merge's operands preloaded, HotArgs: partials,
// (m, l) pairs, position, the [q | k | v] row, then the key splits and the block mapping's count.)
template <int EPI, int NKC, bool NEWKEY, int MKF>
__global__ void __launch_bounds__(256) gemm_skinny_prea_hot_kernel(const void* p0, const void* p1, const void* p2,
                                                                   const void* p3, int nsplit, int rg_count,
                                                                   GemmArgs a, AttnMergeArgs am) {
  constexpr int kKb =
      kernarg_bytes<const void*, const void*, const void*, const void*, int, int, GemmArgs, AttnMergeArgs>();
  gemm_skinny_body<1, false, EPI, NKC, false, 1, false, kEpiStore, false, true, false, false, NEWKEY, true, MKF, kKb,
                   QWEN_HIDDEN, QWEN_HIDDEN>(a, 1, rg_count, QWEN_HIDDEN / (NKC * kKChunk), a, 0, am, AttnFuseArgs{},
                                             HotArgs{p0, p1, p2, p3, nullptr, nullptr, nsplit});
}

// One token's fused [q | k | v] projection + RoPE + K/V append with the decode attention over the
// history keys (see ATTN above); _pre: its activation row is the previous layer's unfinished down
// projection (see PRE above).
__global__ void __launch_bounds__(256) gemm_skinny_attn_kernel(GemmArgs a, AttnFuseArgs af) {
  gemm_skinny_body<2, false, kEpiStore, 12, true, 1, false, kEpiStore, false, false, false, true>(
      a, 1, QWEN_QKV_ROWS / 128, 1, a, 0, AttnMergeArgs{}, af);
}

// (_pre: the prologue's operands preloaded, HotArgs: the reduce step's six pointers, then the key
// splits and the down projection's splits.)
__global__ void __launch_bounds__(256) gemm_skinny_pre_attn_hot_kernel(const void* p0, const void* p1, const void* p2,
                                                                       const void* p3, const void* p4, const void* p5,
                                                                       int nsplit, int pre_splits, GemmArgs a,
                                                                       GemmArgs pre, AttnFuseArgs af) {
  constexpr int kKb = kernarg_bytes<const void*, const void*, const void*, const void*, const void*, const void*, int,
                                    int, GemmArgs, GemmArgs, AttnFuseArgs>();
  gemm_skinny_body<2, false, kEpiStore, 12, true, 1, true, kEpiResidual, false, false, false, true, false, false, 16,
                   kKb, QWEN_HIDDEN, QWEN_QKV_ROWS>(a, 1, QWEN_QKV_ROWS / 128, 1, pre, pre_splits, AttnMergeArgs{},
                                                    af, HotArgs{p0, p1, p2, p3, p4, p5, nsplit});
}

// One token, with the previous projection's reduce step redone by every block (see PRE above).
template <int RTW, bool DUAL, int EPI, int NKC, bool ROPE, int PRE_EPI>
__global__ void __launch_bounds__(256) gemm_skinny_pre_kernel(GemmArgs a, int rg_count, GemmArgs pre, int pre_splits) {
  touch_kernargs<kernarg_bytes<GemmArgs, int, GemmArgs, int>()>();
  gemm_skinny_body<RTW, DUAL, EPI, NKC, ROPE, 1, true, PRE_EPI>(a, 1, rg_count, 1, pre, pre_splits);
}

// The same with the block's four waves splitting K (KW above), three blocks per CU.
template <int RTW, bool DUAL, int EPI, int NKC, int PRE_EPI>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3)))
gemm_skinny_pre_kw_kernel(GemmArgs a, int rg_count, GemmArgs pre, int pre_splits) {
  touch_kernargs<kernarg_bytes<GemmArgs, int, GemmArgs, int>()>();
  gemm_skinny_body<RTW, DUAL, EPI, NKC, false, 1, true, PRE_EPI, false, false, false, false, false, true>(
      a, 1, rg_count, 1, pre, pre_splits);
}

// The same, OUT rows of a 1536-wide row, with the prologue's operands preloaded (HotArgs: the reduce
// step's six pointers), then the block mapping's count and the previous projection's splits.
template <int RTW, bool DUAL, int EPI, int NKC, int PRE_EPI, int OUT>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3)))
gemm_skinny_pre_kw_hot_kernel(const void* p0, const void* p1, const void* p2, const void* p3, const void* p4,
                              const void* p5, int rg_count, int pre_splits, GemmArgs a, GemmArgs pre) {
  constexpr int kKb = kernarg_bytes<const void*, const void*, const void*, const void*, const void*, const void*, int,
                                    int, GemmArgs, GemmArgs>();
  gemm_skinny_body<RTW, DUAL, EPI, NKC, false, 1, true, PRE_EPI, false, false, false, false, false, true, 16, kKb,
                   QWEN_HIDDEN, OUT>(a, 1, rg_count, 1, pre, pre_splits, AttnMergeArgs{}, AttnFuseArgs{},
                                     HotArgs{p0, p1, p2, p3, p4, p5, 0});
}

// Sum over z < splits of part[z * zstride + off .. + 3] in z order.  The loads of 8 splits are all
// issued before the first add, so a reduce costs one memory round trip per 8 splits.
__device__ __forceinline__ float4 sum_splits4(const float* __restrict__ part, size_t zstride, size_t off, int splits) {
  float4 acc = make_float4(0, 0, 0, 0);
  for (int z0 = 0; z0 < splits; z0 += 8) {
    float4 pz[8];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      pz[u] = z0 + u < splits ? *reinterpret_cast<const float4*>(part + (size_t)(z0 + u) * zstride + off)
                              : make_float4(0, 0, 0, 0);
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (z0 + u < splits) {
        acc.x += pz[u].x;
        acc.y += pz[u].y;
        acc.z += pz[u].z;
        acc.w += pz[u].w;
      }
  }
  return acc;
}

// Sums the split partials in z order and applies the offset correction and the epilogue
// (kEpiStore with bias, or kEpiResidual with bf16 rounding).  One thread per 4 outputs.
template <int EPI>
__global__ void __launch_bounds__(256) gemm_splitk_reduce_kernel(GemmArgs a, int splits) {
  const size_t quads = (size_t)a.tokens * (a.out_dim / 4);
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= quads) return;
  const int tok = (int)(i / (a.out_dim / 4));
  const int row0 = (int)(i % (a.out_dim / 4)) * 4;
  const float4 acc = sum_splits4(a.part, (size_t)a.tokens * a.out_dim, (size_t)tok * a.out_dim + row0, splits);
  const double corr = -8.0 * (256.0 * (double)a.sums[2 * tok] + (double)a.sums[2 * tok + 1]) * (double)a.sx[tok];
  float out[4] = {acc.x, acc.y, acc.z, acc.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float v = out[q] + (float)(corr * (double)a.sw[row0 + q]);
    if (EPI == kEpiResidual) {
      const float o = a.resid[(size_t)tok * a.resid_stride + row0 + q] + v;
      out[q] = a.round_bf16 ? round_bf16(o) : o;
    } else {
      out[q] = v + (a.bias ? a.bias[row0 + q] : 0.0f);
    }
  }
  *reinterpret_cast<float4*>(a.y + (size_t)tok * a.y_stride + row0) = make_float4(out[0], out[1], out[2], out[3]);
}

// Finishes output (tok, row) from its split sum: offset correction and bias, the same arithmetic as
// gemm_splitk_reduce_kernel.
__device__ __forceinline__ float finish_one(const GemmArgs& a, float acc, int row, double corr) {
  return acc + (float)(corr * (double)a.sw[row]) + (a.bias ? a.bias[row] : 0.0f);
}

// kFuseQkvRope: reduce of the fused [q | k | v] projection (2048 rows) for decode token t, bias, RoPE
// of the 12 q heads (in place in a.y) and the 2 k heads, and the K/V cache append at position
// pos[t] of sequence t (qwen_decode_attention_kernel.cpp:29-42,100-111 semantics; positions outside
// [0, limit) leave q unrotated and the cache untouched).  Thread t of the block owns rotation pair
// p = t & 63 of heads (t >> 6) + 4k, k < 4 (heads 0-11 q, 12-13 k, 14-15 v).  grid = tokens, block = 256.
__global__ void __launch_bounds__(256) reduce_qkv_rope_kernel(GemmArgs a, int splits) {
  const int tok = blockIdx.x;
  const int p = threadIdx.x & 63;
  const double corr = -8.0 * (256.0 * (double)a.sums[2 * tok] + (double)a.sums[2 * tok + 1]) * (double)a.sx[tok];
  const int P = a.pos[tok];
  const bool in = P >= 0 && P < a.limit;
  float c = 1.0f, sn = 0.0f;
  if (in) {
    c = a.rope[(size_t)P * 128 + p];
    sn = a.rope[(size_t)P * 128 + 64 + p];
  }
  float* yq = a.y + (size_t)tok * a.y_stride;
  float* kc = a.k_cache + (size_t)tok * a.seq_stride + (size_t)(in ? P : 0) * QWEN_KV_WIDTH;
  float* vc = a.v_cache + (size_t)tok * a.seq_stride + (size_t)(in ? P : 0) * QWEN_KV_WIDTH;
  // split sums of the thread's 8 rows (4 pairs), 4 splits per batch of loads, in z order
  const size_t zstride = (size_t)a.tokens * a.out_dim;
  const float* pt = a.part + (size_t)tok * a.out_dim + p;
  float sum[4][2];
#pragma unroll
  for (int k = 0; k < 4; ++k) sum[k][0] = sum[k][1] = 0.0f;
  for (int z0 = 0; z0 < splits; z0 += 4) {
    float pz[4][4][2];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
          pz[u][k][hh] = z0 + u < splits
                             ? pt[(size_t)(z0 + u) * zstride + ((threadIdx.x >> 6) + 4 * k) * QWEN_HEAD_DIM + 64 * hh]
                             : 0.0f;
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (z0 + u < splits)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          sum[k][0] += pz[u][k][0];
          sum[k][1] += pz[u][k][1];
        }
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int head = (threadIdx.x >> 6) + 4 * k;
    const int r0 = head * QWEN_HEAD_DIM + p;
    const float e = finish_one(a, sum[k][0], r0, corr);
    const float od = finish_one(a, sum[k][1], r0 + 64, corr);
    if (head < QWEN_Q_HEADS) {
      yq[r0] = in ? e * c - od * sn : e;
      yq[r0 + 64] = in ? od * c + e * sn : od;
    } else if (!in) {
      continue;
    } else if (head < QWEN_Q_HEADS + QWEN_KV_HEADS) {
      const int base = (head - QWEN_Q_HEADS) * QWEN_HEAD_DIM + p;
      kc[base] = e * c - od * sn;
      kc[base + 64] = od * c + e * sn;
    } else {
      const int base = (head - QWEN_Q_HEADS - QWEN_KV_HEADS) * QWEN_HEAD_DIM + p;
      vc[base] = e;
      vc[base + 64] = od;
    }
  }
}

// kFuseNormQuant: reduce of a 1536-row projection for token t with the EPI epilogue (kEpiStore: bias;
// kEpiResidual: residual, optional raw copy, optional bf16 rounding), the finished row written to
// a.y, then RMSNorm(norm_w) + two-limb quantization of that row into xq_out / sx_out / sums_out.
// Thread t owns float4 columns t and t + 256.  grid = tokens, block = 256.
template <int EPI>
__global__ void __launch_bounds__(256) reduce_norm_quant_kernel(GemmArgs a, int splits) {
  const int tok = blockIdx.x;
  const int n4 = a.out_dim >> 2;
  const double corr = -8.0 * (256.0 * (double)a.sums[2 * tok] + (double)a.sums[2 * tok + 1]) * (double)a.sx[tok];
  float4 v[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int k = threadIdx.x + 256 * j;
    v[j] = make_float4(0, 0, 0, 0);
    if (k >= n4) continue;
    const int row0 = 4 * k;
    const float4 acc = sum_splits4(a.part, (size_t)a.tokens * a.out_dim, (size_t)tok * a.out_dim + row0, splits);
    float out[4] = {acc.x, acc.y, acc.z, acc.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float val = out[q] + (float)(corr * (double)a.sw[row0 + q]);
      if (EPI == kEpiResidual) {
        out[q] = a.resid[(size_t)tok * a.resid_stride + row0 + q] + val;
      } else {
        out[q] = val + (a.bias ? a.bias[row0 + q] : 0.0f);
      }
    }
    if (EPI == kEpiResidual && a.y_raw)
      *reinterpret_cast<float4*>(a.y_raw + (size_t)tok * a.y_stride + row0) = make_float4(out[0], out[1], out[2], out[3]);
    if (EPI == kEpiResidual && a.round_bf16)
#pragma unroll
      for (int q = 0; q < 4; ++q) out[q] = round_bf16(out[q]);
    v[j] = make_float4(out[0], out[1], out[2], out[3]);
    *reinterpret_cast<float4*>(a.y + (size_t)tok * a.y_stride + row0) = v[j];
  }
  norm_quant_row<2>(v, a.out_dim, a.norm_w, a.norm, a.xq_out + (size_t)tok * (size_t)(2 * a.out_dim), a.sx_out + tok,
                    a.sums_out + 2 * tok, nullptr);
}

// kFuseNormQuant for 1536-wide rows, W waves per token row (one in the GEMM prologues, two in
// reduce_norm_quant_pair_kernel): the arithmetic of reduce_norm_quant_kernel with wave reductions
// (and for W = 2 one LDS exchange each) in place of block reductions, and every load of the row (split
// partials, scales, residual or bias, norm weights) issued before the first use, so a row costs one
// memory round trip.  Lane l of the row owns float4 columns l + 64 W j, j < 6 / W.  The two-limb code
// goes to xq_row ([K chunk][limb][128 bytes], K chunk c at byte c * chunk_stride: a row of a.xq_out,
// or a token row of a GEMM's LDS activation slice), the scale and limb sums to sx_out / sums_out;
// the finished row goes to a.y (and a.y_raw) when write_y.
// `issue` runs right after the row's loads are issued (a caller's own loads then queue behind them).
// HOT: the first loads' operands from HotArgs (p0 partials, p1 residual rows of 1536 floats or the
// bias or a stand-in, p2 row scales, p3 norm weights or a stand-in, p4 limb sums, p5 scales, n0 the
// token count), the flags read from `a` after the loads are issued; the outputs are the token's row
// of a.xq_out (chunk_stride 256), a.sx_out and a.sums_out, whatever xq_row, sx_out and sums_out say.
template <int EPI, int ZB, class Issue, int W, bool HOT>
__device__ __forceinline__ void reduce_norm_quant_row_zb(const GemmArgs& a, int splits, int tok, int8_t* xq_row,
                                                         int chunk_stride, float* sx_out, int* sums_out, bool write_y,
                                                         Issue&& issue, const HotArgs& hot) {
  static_assert(W == 1 || W == 2, "one or two waves per row");
  constexpr int NV = QWEN_HIDDEN / (256 * W);
  constexpr int LS = 64 * W;                  // float4 stride between a lane's columns
  const int lane = threadIdx.x & (LS - 1);    // the lane's place among the row's W waves
  // W = 2: the two waves' partial reductions meet in LDS, one slot per reduction (one barrier each)
  __shared__ double x_ss[W > 1 ? 2 : 1];
  __shared__ float x_ssf[W > 1 ? 2 : 1], x_amax[W > 1 ? 2 : 1];
  __shared__ int x_sums[W > 1 ? 4 : 1];
  const int wv = (threadIdx.x >> 6) & (W - 1);
  const size_t zstride4 = (size_t)(HOT ? hot.n0 : a.tokens) * (QWEN_HIDDEN / 4);
  const float* part = HOT ? static_cast<const float*>(hot.p0) : a.part;
  const float4* pt = reinterpret_cast<const float4*>(part + (size_t)tok * QWEN_HIDDEN) + lane;
  const float4* sw4 = reinterpret_cast<const float4*>(HOT ? hot.p2 : a.sw) + lane;
  // Every load in one batch and without branches (a single memory round trip for up to ZB splits): an
  // absent operand (bias, norm weights) is read from the row scales and zeroed after, and the splits of
  // a batch past the last one read the last split again and are not added.
  const float4* r4 =
      HOT ? reinterpret_cast<const float4*>(static_cast<const float*>(hot.p1) +
                                            (EPI == kEpiResidual ? (size_t)tok * QWEN_HIDDEN : 0)) + lane
      : EPI == kEpiResidual ? reinterpret_cast<const float4*>(a.resid + (size_t)tok * a.resid_stride) + lane
                            : (a.bias ? reinterpret_cast<const float4*>(a.bias) + lane : sw4);
  const float4* w4 = HOT                 ? reinterpret_cast<const float4*>(hot.p3) + lane
                     : a.norm != kNormNone ? reinterpret_cast<const float4*>(a.norm_w) + lane
                                           : sw4;
  const int* sums = HOT ? static_cast<const int*>(hot.p4) : a.sums;
  const float* sxs = HOT ? static_cast<const float*>(hot.p5) : a.sx;
  const int sum_h = sums[2 * tok], sum_l = sums[2 * tok + 1];
  const float sx_tok = sxs[tok];
  float4 acc[NV], sw[NV], ad[NV], wn[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    sw[j] = sw4[LS * j];
    ad[j] = r4[LS * j];
    wn[j] = w4[LS * j];
  }
  // split sums in z order
#pragma unroll
  for (int j = 0; j < NV; ++j) acc[j] = make_float4(0, 0, 0, 0);
  if constexpr (HOT) {
    // splits <= ZB (the launcher checks), straight-line: every split's loads issued unconditionally
    // (past the last split the last again, unused; without splits the row scales), `issue`, then the
    // adds as selects (adding +0 leaves a sum that started at +0 unchanged)
    const float4* pt0 = splits > 0 ? pt : sw4;
    const int zlast = max(splits, 1) - 1;
    float4 pz[ZB][NV];
#pragma unroll
    for (int u = 0; u < ZB; ++u)
#pragma unroll
      for (int j = 0; j < NV; ++j) pz[u][j] = pt0[(size_t)min(u, zlast) * zstride4 + LS * j];
    __builtin_amdgcn_sched_barrier(0);
    issue();
    __builtin_amdgcn_sched_barrier(0);
    // the outputs: the token's row of a.xq_out, its scale and limb sums (addressed only now)
    xq_row = a.xq_out + (size_t)tok * (2 * QWEN_HIDDEN);
    sx_out = a.sx_out + tok;
    sums_out = a.sums_out + 2 * tok;
#pragma unroll
    for (int u = 0; u < ZB; ++u) {
      const bool live = u < splits;
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        acc[j].x += live ? pz[u][j].x : 0.0f;
        acc[j].y += live ? pz[u][j].y : 0.0f;
        acc[j].z += live ? pz[u][j].z : 0.0f;
        acc[j].w += live ? pz[u][j].w : 0.0f;
      }
    }
  }
  for (int z0 = 0; !HOT && z0 < splits; z0 += ZB) {
    float4 pz[ZB][NV];
#pragma unroll
    for (int u = 0; u < ZB; ++u)
#pragma unroll
      for (int j = 0; j < NV; ++j) pz[u][j] = pt[(size_t)min(z0 + u, splits - 1) * zstride4 + LS * j];
    if (z0 == 0) {
      __builtin_amdgcn_sched_barrier(0);
      issue();
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int u = 0; u < ZB; ++u)
      if (z0 + u < splits)
#pragma unroll
        for (int j = 0; j < NV; ++j) {
          acc[j].x += pz[u][j].x;
          acc[j].y += pz[u][j].y;
          acc[j].z += pz[u][j].z;
          acc[j].w += pz[u][j].w;
        }
  }
  if (!HOT && splits < 1) issue();  // the caller's loads are issued exactly once, also without splits
  const bool has_add = EPI == kEpiResidual || a.bias != nullptr;
  const bool has_w = a.norm != kNormNone;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    if (!has_add) ad[j] = make_float4(0, 0, 0, 0);
    if (!has_w) wn[j] = make_float4(0, 0, 0, 0);
  }
  const double corr = -8.0 * (256.0 * (double)sum_h + (double)sum_l) * (double)sx_tok;
  float4 v[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j)
    v[j] = rnq_combine<EPI>(a, tok, 4 * (lane + LS * j), acc[j], sw[j], ad[j], corr, write_y);
  // RMSNorm (norm_quant_row's arithmetic, wave reductions)
  if (a.norm == kNormDecode) {
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < NV; ++j) ss += rnq_sq4(v[j]);
    ss = wave_sum_d(ss);
    if constexpr (W > 1) {
      if ((threadIdx.x & 63) == 0) x_ss[wv] = ss;
      __syncthreads();
      ss = x_ss[0] + x_ss[1];
    }
    const double inv = 1.0 / sqrt(ss / (double)QWEN_HIDDEN + (double)QWEN_RMS_EPS);
#pragma unroll
    for (int j = 0; j < NV; ++j) v[j] = rnq_norm4(v[j], inv, wn[j]);
  } else if (a.norm == kNormPrefill) {
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) ss += v[j].x * v[j].x + v[j].y * v[j].y + v[j].z * v[j].z + v[j].w * v[j].w;
    ss = wave_sum(ss);
    if constexpr (W > 1) {
      if ((threadIdx.x & 63) == 0) x_ssf[wv] = ss;
      __syncthreads();
      ss = x_ssf[0] + x_ssf[1];
    }
    const float inv = 1.0f / approx_sqrt(ss / (float)QWEN_HIDDEN + QWEN_RMS_EPS);
#pragma unroll
    for (int j = 0; j < NV; ++j)
      v[j] = make_float4(v[j].x * inv * wn[j].x, v[j].y * inv * wn[j].y, v[j].z * inv * wn[j].z, v[j].w * inv * wn[j].w);
  }
  // two-limb quantization (norm_quant_row's code)
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j)
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
  amax = wave_max(amax);
  if constexpr (W > 1) {
    if ((threadIdx.x & 63) == 0) x_amax[wv] = amax;
    __syncthreads();
    amax = fmaxf(x_amax[0], x_amax[1]);
  }
  const float qinv = amax > 0.0f ? (float)kQuantMax / amax : 0.0f;
  int8_t* row = xq_row;
  int sh = 0, sl = 0;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int k = lane + LS * j;
    const float e[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
    uint32_t hw = 0, lw = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float xf = fminf(fmaxf(rintf(e[q] * qinv), -(float)kQuantMax), (float)kQuantMax);
      const int X = (int)xf;
      const int H = (X + 128) >> 8;
      const int L = X - (H << 8);
      hw |= (uint32_t)(H & 0xFF) << (8 * q);
      lw |= (uint32_t)(L & 0xFF) << (8 * q);
      sh += H;
      sl += L;
    }
    const int base = ((4 * k) >> 7) * chunk_stride + ((4 * k) & 127);
    *reinterpret_cast<uint32_t*>(row + base) = hw;
    *reinterpret_cast<uint32_t*>(row + base + 128) = lw;
  }
  sh = wave_sum_i(sh);
  sl = wave_sum_i(sl);
  if constexpr (W > 1) {
    if ((threadIdx.x & 63) == 0) {
      x_sums[2 * wv] = sh;
      x_sums[2 * wv + 1] = sl;
    }
    __syncthreads();
    sh = x_sums[0] + x_sums[2];
    sl = x_sums[1] + x_sums[3];
  }
  if (lane == 0) {
    *sx_out = amax > 0.0f ? amax / (float)kQuantMax : 1.0f;
    sums_out[0] = sh;
    sums_out[1] = sl;
  }
}

// reduce_norm_quant_row_zb's arithmetic for token 0's 1536-wide row (decode norm or none) by the four
// waves of a 256-thread block: thread t owns float4 t and, for t < 128 (waves 0 and 1), float4 t + 256.
// The sum of squares and the maximum are each a wave reduction (wave_sum's order) and one exchange of
// the four waves' values through LDS (two barriers); the limb sums are left as per-wave partials in
// sums_out (8 ints; see wave_sums_total), and the scale in *sx_out, both published by the caller's
// barrier.  Every wave calls `issue` once, right after its loads of the row.
template <int EPI, int ZB, bool HOT, class Issue>
__device__ __forceinline__ void reduce_norm_quant_row_w4(const GemmArgs& a, int splits, int8_t* xq_row,
                                                         int chunk_stride, float* sx_out, int* sums_out, bool write_y,
                                                         Issue&& issue, const HotArgs& hot) {
  __shared__ double w_ss[4];
  __shared__ float w_max[4];
  constexpr int kF = QWEN_HIDDEN / 4;  // float4s of the row
  const int t = threadIdx.x, wv = t >> 6;
  const bool two = t < kF - 256;  // wave-uniform
  const int f[2] = {t, min(t + 256, kF - 1)};
  // (HOT: the operands of the first loads from the preloaded HotArgs, the stand-ins chosen by the
  // launcher; the flags has_add and has_w are read from `a` after the loads are issued)
  const size_t zstride4 = HOT ? (size_t)kF : (size_t)a.tokens * kF;
  const float4* pt = reinterpret_cast<const float4*>(HOT ? hot.p0 : a.part);
  const float4* sw4 = reinterpret_cast<const float4*>(HOT ? hot.p2 : a.sw);
  const float4* r4 = HOT ? reinterpret_cast<const float4*>(hot.p1)
                         : EPI == kEpiResidual ? reinterpret_cast<const float4*>(a.resid)
                                               : (a.bias ? reinterpret_cast<const float4*>(a.bias) : sw4);
  const float4* w4 = HOT                     ? reinterpret_cast<const float4*>(hot.p3)
                     : a.norm != kNormNone ? reinterpret_cast<const float4*>(a.norm_w)
                                           : sw4;
  float4 acc[2], sw[2], ad[2], wn[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    sw[j] = sw4[f[j]];
    ad[j] = r4[f[j]];
    wn[j] = w4[f[j]];
    acc[j] = make_float4(0, 0, 0, 0);
  }
  // splits <= ZB (the launchers check).  The splits' loads are issued unconditionally (without splits
  // from a valid stand-in, their values unused), then the token's limb sums and scale as vector loads (a lane-varying zero index),
  // then `issue`.  Behind a run-time branch, or with the sums as scalar loads, the partial loads waited
  // for the sums' memory round trip: the wait for the kernel arguments that address the partials
  // counted the scalar loads in flight too.
  const float4* pt0 = splits > 0 ? pt : sw4;
  const int zlast = max(splits, 1) - 1;
  float4 pz[ZB][2];
#pragma unroll
  for (int u = 0; u < ZB; ++u)
#pragma unroll
    for (int j = 0; j < 2; ++j) pz[u][j] = pt0[(size_t)min(u, zlast) * zstride4 + f[j]];
  int lz;
  asm volatile("v_mov_b32 %0, 0" : "=v"(lz));
  const int* sums_p = HOT ? static_cast<const int*>(hot.p4) : a.sums;
  const float* sx_p = HOT ? static_cast<const float*>(hot.p5) : a.sx;
  const int sum_h = sums_p[lz], sum_l = sums_p[lz + 1];
  const float sx_tok = sx_p[lz];
  __builtin_amdgcn_sched_barrier(0);
  issue();
  __builtin_amdgcn_sched_barrier(0);
  const bool has_add = EPI == kEpiResidual || a.bias != nullptr;
  const bool has_w = a.norm != kNormNone;
  // Added as selects, in split order (adding +0 leaves a sum that started at +0 unchanged).  (A loop
  // over further batches, reloading pz, made the compiler wait for every load in flight, `issue`'s
  // weights included, before the first add.)
#pragma unroll
  for (int u = 0; u < ZB; ++u) {
    const bool live = u < splits;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      acc[j].x += live ? pz[u][j].x : 0.0f;
      acc[j].y += live ? pz[u][j].y : 0.0f;
      acc[j].z += live ? pz[u][j].z : 0.0f;
      acc[j].w += live ? pz[u][j].w : 0.0f;
    }
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    if (!has_add) ad[j] = make_float4(0, 0, 0, 0);
    if (!has_w) wn[j] = make_float4(0, 0, 0, 0);
  }
  const double corr = -8.0 * (256.0 * (double)sum_h + (double)sum_l) * (double)sx_tok;
  float4 v[2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
    v[j] = rnq_combine<EPI>(a, 0, 4 * f[j], acc[j], sw[j], ad[j], corr, write_y && (j == 0 || two));
  if (a.norm == kNormDecode) {
    double ss = rnq_sq4(v[0]);
    if (two) ss += rnq_sq4(v[1]);
    ss = wave_sum_d(ss);
    if ((t & 63) == 0) w_ss[wv] = ss;
    __syncthreads();
    ss = (w_ss[0] + w_ss[1]) + (w_ss[2] + w_ss[3]);
    const double inv = 1.0 / sqrt(ss / (double)QWEN_HIDDEN + (double)QWEN_RMS_EPS);
#pragma unroll
    for (int j = 0; j < 2; ++j) v[j] = rnq_norm4(v[j], inv, wn[j]);
  } else if (a.norm == kNormPrefill) {
    float ss = v[0].x * v[0].x + v[0].y * v[0].y + v[0].z * v[0].z + v[0].w * v[0].w;
    if (two) ss += v[1].x * v[1].x + v[1].y * v[1].y + v[1].z * v[1].z + v[1].w * v[1].w;
    ss = wave_sum(ss);
    if ((t & 63) == 0) w_ss[wv] = ss;
    __syncthreads();
    ss = (float)((w_ss[0] + w_ss[1]) + (w_ss[2] + w_ss[3]));
    const float inv = 1.0f / approx_sqrt((float)ss / (float)QWEN_HIDDEN + QWEN_RMS_EPS);
#pragma unroll
    for (int j = 0; j < 2; ++j)
      v[j] = make_float4(v[j].x * inv * wn[j].x, v[j].y * inv * wn[j].y, v[j].z * inv * wn[j].z, v[j].w * inv * wn[j].w);
  }
  float amax = fmaxf(fmaxf(fabsf(v[0].x), fabsf(v[0].y)), fmaxf(fabsf(v[0].z), fabsf(v[0].w)));
  if (two) amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[1].x), fabsf(v[1].y)), fmaxf(fabsf(v[1].z), fabsf(v[1].w))));
  amax = wave_max(amax);
  if ((t & 63) == 0) w_max[wv] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(w_max[0], w_max[1]), fmaxf(w_max[2], w_max[3]));
  const float qinv = amax > 0.0f ? (float)kQuantMax / amax : 0.0f;
  int sh = 0, sl = 0;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    if (j == 1 && !two) break;
    const float e[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
    uint32_t hw = 0, lw = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float xf = fminf(fmaxf(rintf(e[q] * qinv), -(float)kQuantMax), (float)kQuantMax);
      const int X = (int)xf;
      const int H = (X + 128) >> 8;
      const int L = X - (H << 8);
      hw |= (uint32_t)(H & 0xFF) << (8 * q);
      lw |= (uint32_t)(L & 0xFF) << (8 * q);
      sh += H;
      sl += L;
    }
    const int base = ((4 * f[j]) >> 7) * chunk_stride + ((4 * f[j]) & 127);
    *reinterpret_cast<uint32_t*>(xq_row + base) = hw;
    *reinterpret_cast<uint32_t*>(xq_row + base + 128) = lw;
  }
  // the limb sums as per-wave partials (sums_out: 8 ints, totals by wave_sums_total after the
  // caller's slice barrier)
  sh = wave_sum_i(sh);
  sl = wave_sum_i(sl);
  if ((t & 63) == 0) {
    sums_out[2 * wv] = sh;
    sums_out[2 * wv + 1] = sl;
  }
  if (t == 0) *sx_out = amax > 0.0f ? amax / (float)kQuantMax : 1.0f;
}


// One split (the O projection's single K group) or up to five (the down projection's) in one batch.
template <int EPI, class Issue>
__device__ __forceinline__ void reduce_norm_quant_row(const GemmArgs& a, int splits, int tok, int8_t* xq_row,
                                                      int chunk_stride, float* sx_out, int* sums_out, bool write_y,
                                                      Issue&& issue) {
  if (splits == 1)
    reduce_norm_quant_row_zb<EPI, 1>(a, splits, tok, xq_row, chunk_stride, sx_out, sums_out, write_y, issue);
  else
    reduce_norm_quant_row_zb<EPI, 5>(a, splits, tok, xq_row, chunk_stride, sx_out, sums_out, write_y, issue);
}

// grid = tokens, block = 128 (two waves per row: half the per-lane work of the one-wave form, three
// LDS exchanges); the values equal the one-wave form's except the norm's sum of squares, added in
// another order.
template <int EPI>
__global__ void __launch_bounds__(128) reduce_norm_quant_pair_kernel(GemmArgs a, int splits) {
  touch_kernargs<kernarg_bytes<GemmArgs, int>()>();
  const int tok = blockIdx.x;
  int8_t* xq_row = a.xq_out + (size_t)tok * (2 * QWEN_HIDDEN);
  if (splits == 1)
    reduce_norm_quant_row_zb<EPI, 1, NoIssue, 2>(a, splits, tok, xq_row, 256, a.sx_out + tok, a.sums_out + 2 * tok, true,
                                                  NoIssue{});
  else
    reduce_norm_quant_row_zb<EPI, 5, NoIssue, 2>(a, splits, tok, xq_row, 256, a.sx_out + tok, a.sums_out + 2 * tok, true,
                                                  NoIssue{});
}

// The same with the first loads' operands preloaded (HotArgs of reduce_norm_quant_row_zb), residual
// rows 1536 floats apart.
template <int EPI>
__global__ void __launch_bounds__(128) reduce_norm_quant_pair_hot_kernel(const void* p0, const void* p1, const void* p2,
                                                                         const void* p3, const void* p4, const void* p5,
                                                                         int tokens, int splits, GemmArgs a) {
  const auto klines = kernarg_lines_issue<kernarg_bytes<const void*, const void*, const void*, const void*,
                                                        const void*, const void*, int, int, GemmArgs>()>();
  const HotArgs hot{p0, p1, p2, p3, p4, p5, tokens};
  auto issue = [&]() { kernarg_lines_wait(klines); };
  const int tok = blockIdx.x;
  // (the outputs are addressed inside, once the loads are issued)
  if (splits == 1)
    reduce_norm_quant_row_zb<EPI, 1, decltype(issue)&, 2, true>(a, splits, tok, nullptr, 256, nullptr, nullptr, true,
                                                                issue, hot);
  else
    reduce_norm_quant_row_zb<EPI, 5, decltype(issue)&, 2, true>(a, splits, tok, nullptr, 256, nullptr, nullptr, true,
                                                                issue, hot);
}

// ---------------------------------------------------------------------------------------------
// RoPE of q (in place) and k, plus the K/V cache append, for rows of a fused [q | k | v] buffer
// (qkv_stride floats per token).  Decode: token b is sequence b at position pos[b].  Prefill:
// token t is sequence t / seq_len at position t % seq_len.  rope: [position][cos 64 | sin 64].
// Positions outside [0, limit) are skipped (limit = the cache rows the caller sized).
// grid = tokens, block = 64 (one rotation pair per thread).
// ---------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(64) rope_qkv_kernel(float* __restrict__ qkv, int qkv_stride,
                                                      const int* __restrict__ pos, int seq_len, int past, int limit,
                                                      const float* __restrict__ rope, float* __restrict__ k_cache,
                                                      float* __restrict__ v_cache, size_t seq_stride) {
  const int t = blockIdx.x;
  const int p = threadIdx.x;
  const int seq = pos ? t : t / seq_len;
  const int P = pos ? pos[t] : past + t % seq_len;
  if (P < 0 || P >= limit) return;  // position outside the cache rows the caller sized
  const float c = rope[(size_t)P * 128 + p];
  const float sn = rope[(size_t)P * 128 + 64 + p];
  float* row = qkv + (size_t)t * qkv_stride;
#pragma unroll
  for (int h = 0; h < QWEN_Q_HEADS; ++h) {
    float* hp = row + h * QWEN_HEAD_DIM;
    const float e = hp[p], od = hp[p + 64];
    hp[p] = e * c - od * sn;
    hp[p + 64] = od * c + e * sn;
  }
  const float* kr = row + QWEN_HIDDEN;
  const float* vr = row + QWEN_HIDDEN + QWEN_KV_WIDTH;
  float* kc = k_cache + (size_t)seq * seq_stride + (size_t)P * QWEN_KV_WIDTH;
  float* vc = v_cache + (size_t)seq * seq_stride + (size_t)P * QWEN_KV_WIDTH;
#pragma unroll
  for (int h = 0; h < QWEN_KV_HEADS; ++h) {
    const int base = h * QWEN_HEAD_DIM;
    const float e = kr[base + p], od = kr[base + p + 64];
    kc[base + p] = e * c - od * sn;
    kc[base + p + 64] = od * c + e * sn;
    vc[base + p] = vr[base + p];
    vc[base + p + 64] = vr[base + p + 64];
  }
}

// ---------------------------------------------------------------------------------------------
// Decode attention on the fp32 matrix cores, split over the KV length; the split merge and the
// O-projection input quantization follow in attn_decode_merge_kernel (qwen_decode_attention_kernel.cpp:113-162 semantics:
// s_t = (q . k_t) * 0.08838834764831845f over keys 0..pos, softmax, ctx = sum_t p_t v_t; here with
// an online softmax, reordered sums and __expf).
// grid = (nsplit, 2 KV heads, batch), block = 256 (4 waves).  Block (split c, KV head kvh, sequence
// b) takes keys [c*chunk, min(n, c*chunk + chunk)) of sequence b, n = min(pos[b] + 1, max_keys);
// wave w takes the 16-key tiles w, w+4, w+8, ... of that range.  Per tile (lane: col = lane & 15,
// g = lane >> 4):
//   S = K . Q^T:  A = K[key col][dim 4g+16j+e] (streamed from HBM, 64 contiguous bytes per key per
//                 load), B = Q[head col][same dim] (LDS; heads >= 6 are zero rows), 32 MFMAs;
//                 lane gets S[key 4g+r][head col], r = 0..3;
//   online softmax per head col (max over the tile's keys: registers + xor-shuffles 16, 32);
//   O += P . V:   MFMA (r, h, e): A = P[head col][key 4g+r] (the lane's own p[r]),
//                 B = V[key 4g+r][dim 4col+e+64h]; lane holds O[head 4g+r'][dim 4col+e+64h].
// The block merges its 4 waves in LDS and writes (m, l, acc[128]) per query head to
// part[b][head][c][128] and pml[b][head][c] with plain stores (the launch boundary publishes them).
// The splits are merged by the next launch: the merge kernel below, or for one sequence every block
// of the O projection (attn_merge_quant_slice).  (Merged inside this launch by the last-arriving
// block of each sequence, the partials needed device-coherent stores, an arrival count and
// device-coherent reloads, all behind the other blocks' key stream: 95 us per 64 x 4096 launch
// against 85 us for the partials alone plus ~1.2 us of launch hand-off and the merge launch.)
// ---------------------------------------------------------------------------------------------
typedef float v4f __attribute__((ext_vector_type(4)));
constexpr int kQRow = QWEN_HEAD_DIM + 4;  // LDS floats per query row (16-byte pad: no bank aliasing)

// Loads of one 16-key tile of attn_decode_kernel (keys tb..tb+15).  MASK: keys >= t1 read row t1 - 1
// instead, as the first tile does: their scores are masked to -inf, so their weight is exactly 0
// and the finite rows add 0.  (Loads under a per-lane condition were branches, each followed by a
// wait for every load in flight, so the tile's loads went out one round trip at a time.)
template <bool MASK>
__device__ __forceinline__ void attn_decode_tile_load(const float* __restrict__ kb, const float* __restrict__ vb,
                                                      int tb, int t1, int col, int g, float4 (&kr)[8],
                                                      float4 (&vr)[4][2]) {
  const int tk = MASK ? min(tb + col, t1 - 1) : tb + col;
  const float* krow = kb + (size_t)tk * QWEN_KV_WIDTH + 4 * g;
#pragma unroll
  for (int j = 0; j < 8; ++j) kr[j] = ld_stream(reinterpret_cast<const float4*>(krow + 16 * j));
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int tv = MASK ? min(tb + 4 * g + r, t1 - 1) : tb + 4 * g + r;
    const float* vrow = vb + (size_t)tv * QWEN_KV_WIDTH + 4 * col;
#pragma unroll
    for (int h = 0; h < 2; ++h) vr[r][h] = ld_stream(reinterpret_cast<const float4*>(vrow + 64 * h));
  }
  // All 16 loads of the tile are issued before any math (16 KiB in flight per wave): without this
  // fence the register-capped scheduler interleaves each load with its first use.
  __builtin_amdgcn_sched_barrier(0);
}

// Math of one loaded tile: scores, online softmax (MASK: keys >= t1 masked out), P.V.
template <bool MASK>
__device__ __forceinline__ void attn_decode_tile_math(const float* qrow, int tb, int t1, int g, float& m, float& lp,
                                                      v4f (&acc)[8], const float4 (&kr)[8],
                                                      const float4 (&vr)[4][2]) {
  v4f sc = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float4 q4 = *reinterpret_cast<const float4*>(qrow + 16 * j);
    sc = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[j].x, q4.x, sc, 0, 0, 0);
    sc = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[j].y, q4.y, sc, 0, 0, 0);
    sc = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[j].z, q4.z, sc, 0, 0, 0);
    sc = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[j].w, q4.w, sc, 0, 0, 0);
  }
  float mt = -INFINITY;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    if (MASK && tb + 4 * g + r >= t1) sc[r] = -INFINITY;
    mt = fmaxf(mt, sc[r]);
  }
  mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
  mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
  const float mn = fmaxf(m, mt);  // finite: key tb < t1 is in the tile
  const float corr = __expf(m - mn);
  float p[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) p[r] = __expf(sc[r] - mn);
  lp = lp * corr + ((p[0] + p[1]) + (p[2] + p[3]));
  m = mn;
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) {
    const float cr = __shfl(corr, 4 * g + rr, 64);  // lane 4g + rr holds head 4g + rr
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[k][rr] *= cr;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      acc[4 * h + 0] = __builtin_amdgcn_mfma_f32_16x16x4f32(p[r], vr[r][h].x, acc[4 * h + 0], 0, 0, 0);
      acc[4 * h + 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(p[r], vr[r][h].y, acc[4 * h + 1], 0, 0, 0);
      acc[4 * h + 2] = __builtin_amdgcn_mfma_f32_16x16x4f32(p[r], vr[r][h].z, acc[4 * h + 2], 0, 0, 0);
      acc[4 * h + 3] = __builtin_amdgcn_mfma_f32_16x16x4f32(p[r], vr[r][h].w, acc[4 * h + 3], 0, 0, 0);
    }
  }
}

template <bool MASK>
__device__ __forceinline__ void attn_decode_tile(const float* __restrict__ kb, const float* __restrict__ vb,
                                                 const float* qrow, int tb, int t1, int col, int g, float& m,
                                                 float& lp, v4f (&acc)[8]) {
  float4 kr[8], vr[4][2];
  attn_decode_tile_load<MASK>(kb, vb, tb, t1, col, g, kr, vr);
  attn_decode_tile_math<MASK>(qrow, tb, t1, g, m, lp, acc, kr, vr);
}

__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4)))
attn_decode_kernel(const float* __restrict__ qkv, int qkv_stride, const float* __restrict__ k_cache,
                   const float* __restrict__ v_cache, size_t seq_stride, const int* __restrict__ pos, int chunk,
                   int max_keys, float* __restrict__ part, float2* __restrict__ pml) {
  // (the leading 14 argument dwords, through max_keys, are preloaded: the first loads wait for nothing;
  // the segment's other lines are requested at entry and waited for once the first tile is in flight)
  const auto klines = kernarg_lines_issue<
      kernarg_bytes<const float*, int, const float*, const float*, size_t, const int*, int, int, float*, float2*>()>();
  __shared__ __align__(16) float qs[16][kQRow];
  __shared__ __align__(16) float s_acc[4][QWEN_GROUPS][QWEN_HEAD_DIM];
  __shared__ float s_m[4][QWEN_GROUPS], s_l[4][QWEN_GROUPS];
  const int nsplit = gridDim.x;
  const int c = blockIdx.x;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int col = lane & 15;
  const int g = lane >> 4;
  const int n = min(max(pos[b], 0) + 1, max_keys);
  const int t0 = c * chunk;
  const float scaling = 0.08838834764831845f;

  if (t0 < n) {  // block-uniform; splits past the sequence only count themselves in below
    const int t1 = min(n, t0 + chunk);
    // the q rows of the group, then the wave's first K/V tile: both memory round trips overlap
    float qv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = threadIdx.x + 256 * j;
      const int h = i >> 7, d = i & 127;
      const float v = qkv[(size_t)b * qkv_stride + (kvh * QWEN_GROUPS + (h < QWEN_GROUPS ? h : 0)) * QWEN_HEAD_DIM + d];
      qv[j] = h < QWEN_GROUPS ? v : 0.0f;  // rows 6..15 of the MFMA tile are padding
    }
    const float* kb = k_cache + (size_t)b * seq_stride + kvh * QWEN_HEAD_DIM;
    const float* vb = v_cache + (size_t)b * seq_stride + kvh * QWEN_HEAD_DIM;
    int tb = t0 + 16 * wave;
    // Keys past t1 read row t1 - 1 instead (no predicated loads: the 16 loads issue back to back);
    // the masked math gives them score -inf, so their weight is exactly 0 and the finite row adds 0.
    float4 kr0[8], vr0[4][2];
    {
      const float* krow = kb + (size_t)min(tb + col, t1 - 1) * QWEN_KV_WIDTH + 4 * g;
#pragma unroll
      for (int j = 0; j < 8; ++j) kr0[j] = ld_stream(reinterpret_cast<const float4*>(krow + 16 * j));
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float* vrow = vb + (size_t)min(tb + 4 * g + r, t1 - 1) * QWEN_KV_WIDTH + 4 * col;
#pragma unroll
        for (int h = 0; h < 2; ++h) vr0[r][h] = ld_stream(reinterpret_cast<const float4*>(vrow + 64 * h));
      }
    }
    kernarg_lines_wait(klines);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = threadIdx.x + 256 * j;
      qs[i >> 7][i & 127] = qv[j] * scaling;
    }
    __syncthreads();
    const float* qrow = &qs[col][4 * g];
    float m = -INFINITY;
    float lp = 0.0f;
    v4f acc[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[k] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    if (tb < t1) {
      attn_decode_tile_math<true>(qrow, tb, t1, g, m, lp, acc, kr0, vr0);
    } else {
      // a wave without keys still consumes the loads (finite rows: adds exactly 0 to lp = 0), so that
      // the compiler keeps them ahead of the q staging instead of sinking them into the branch above
      float z = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) z += (kr0[j].x + kr0[j].y) + (kr0[j].z + kr0[j].w);
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int h = 0; h < 2; ++h) z += (vr0[r][h].x + vr0[r][h].y) + (vr0[r][h].z + vr0[r][h].w);
      lp += 0.0f * z;
    }
    tb += 64;
#pragma unroll 1
    for (; tb + 16 <= t1; tb += 64) attn_decode_tile<false>(kb, vb, qrow, tb, t1, col, g, m, lp, acc);
    if (tb < t1) attn_decode_tile<true>(kb, vb, qrow, tb, t1, col, g, m, lp, acc);  // the range's last, partial tile
    lp += __shfl_xor(lp, 16, 64);
    lp += __shfl_xor(lp, 32, 64);
    if (g == 0 && col < QWEN_GROUPS) {
      s_m[wave][col] = m;
      s_l[wave][col] = lp;
    }
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int head = 4 * g + rr;
      if (head < QWEN_GROUPS) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int e = 0; e < 4; ++e) s_acc[wave][head][4 * col + e + 64 * h] = acc[4 * h + e][rr];
      }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < QWEN_GROUPS * QWEN_HEAD_DIM; i += 256) {
      const int head = i / QWEN_HEAD_DIM, d = i % QWEN_HEAD_DIM;
      float M = s_m[0][head];
#pragma unroll
      for (int w = 1; w < 4; ++w) M = fmaxf(M, s_m[w][head]);
      float L = 0.0f, A = 0.0f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float f = s_m[w][head] == -INFINITY ? 0.0f : __expf(s_m[w][head] - M);  // waves without keys
        L += s_l[w][head] * f;
        A += s_acc[w][head][d] * f;
      }
      const int qh = kvh * QWEN_GROUPS + head;
      part[(((size_t)b * QWEN_Q_HEADS + qh) * nsplit + c) * QWEN_HEAD_DIM + d] = A;
      if (d == 0) {
        pml[((size_t)b * QWEN_Q_HEADS + qh) * nsplit + c] = make_float2(M, L);
      }
    }
  }
}

// The split merge of attn_decode_kernel's partials, one block per sequence: per head the merge
// weights of the splits that hold keys (merge_split_weights), the weighted sum of their partial rows
// in split order into the context row (written to ctx when given), then the row's two-limb code,
// scale and limb sums for the O projection (quantize_row_lds).  Thread t owns float4 columns t and
// t + 256 (< 384) of the row.  Every load of a batch of 8 splits is issued unconditionally (splits
// past the last one load the last again, unused) together with the (m, l) pairs, so sequences with
// at most 8 splits need one memory round trip.
__global__ void __launch_bounds__(256) attn_decode_merge_kernel(const float* __restrict__ part,
                                                                const float2* __restrict__ pml,
                                                                const int* __restrict__ pos, int nsplit, int chunk,
                                                                int max_keys, float* __restrict__ ctx,
                                                                int8_t* __restrict__ xq, float* __restrict__ sx,
                                                                int* __restrict__ sums) {
  constexpr int kF4 = QWEN_HIDDEN / 4;  // float4 columns of the row
  __shared__ __align__(16) float row[QWEN_HIDDEN];         // the context row
  __shared__ float ml[QWEN_Q_HEADS * kAttnMaxSplits * 2];  // (m, l), then merge weights in place
  __shared__ float red_f[4];
  __shared__ int red_i[8];
  const int b = blockIdx.x;
  const int n = min(max(pos[b], 0) + 1, max_keys);
  const int nc = (n + chunk - 1) / chunk;  // splits that hold keys
  const float2* pb = pml + (size_t)b * QWEN_Q_HEADS * nsplit;
  const float* pa = part + (size_t)b * QWEN_Q_HEADS * nsplit * QWEN_HEAD_DIM;
  const int f[2] = {(int)threadIdx.x, min((int)threadIdx.x + 256, kF4 - 1)};
  const bool two = threadIdx.x + 256 < kF4;  // wave-uniform
  float4 pv[2][8];
  auto load_part = [&](int s0) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int h = f[u] >> 5, d4 = 4 * (f[u] & 31);
#pragma unroll
      for (int j = 0; j < 8; ++j)
        pv[u][j] = *reinterpret_cast<const float4*>(pa + ((size_t)h * nsplit + min(s0 + j, nc - 1)) * QWEN_HEAD_DIM + d4);
    }
  };
  load_part(0);
  for (int i = threadIdx.x; i < QWEN_Q_HEADS * nc; i += 256) {
    const int h = i / nc, sp = i % nc;
    const float2 v = pb[h * nsplit + sp];  // (m, l) in one memory round trip
    ml[(h * kAttnMaxSplits + sp) * 2] = v.x;
    ml[(h * kAttnMaxSplits + sp) * 2 + 1] = v.y;
  }
  __syncthreads();
  merge_split_weights(ml, nc, nullptr, false);
  __syncthreads();
  float4 out[2] = {make_float4(0.0f, 0.0f, 0.0f, 0.0f), make_float4(0.0f, 0.0f, 0.0f, 0.0f)};
  for (int s0 = 0; s0 < nc; s0 += 8) {
    if (s0 > 0) load_part(s0);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int h = f[u] >> 5;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (s0 + j < nc) {  // block-uniform
          const float w = ml[(h * kAttnMaxSplits + s0 + j) * 2];
          out[u].x += pv[u][j].x * w;
          out[u].y += pv[u][j].y * w;
          out[u].z += pv[u][j].z * w;
          out[u].w += pv[u][j].w * w;
        }
    }
  }
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    if (u == 1 && !two) break;
    reinterpret_cast<float4*>(row)[f[u]] = out[u];
    if (ctx) reinterpret_cast<float4*>(ctx + (size_t)b * QWEN_HIDDEN)[f[u]] = out[u];
  }
  __syncthreads();
  quantize_row_lds(row, QWEN_HIDDEN, xq + (size_t)b * (2 * QWEN_HIDDEN), sx + b, sums + 2 * b, red_f, red_i);
}

__global__ void zero_u32_kernel(unsigned* __restrict__ p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// ---------------------------------------------------------------------------------------------
// Prefill attention on the bf16 matrix cores (v_mfma_f32_16x16x32_bf16) with hi/lo splitting:
// every fp32 operand x is carried as hi = bf16(x) and lo = bf16(x - hi), and each product is
// hi*hi + lo*hi + hi*lo (the lo*lo term is below fp32 rounding of the sum), accumulated in fp32.
// ---------------------------------------------------------------------------------------------
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
constexpr int kPfQ = 16;     // queries per block
constexpr int kPfKeys = 32;  // keys per tile

__device__ __forceinline__ bf16x4 bf16_hi4(float4 x) {
  return bf16x4{(__bf16)x.x, (__bf16)x.y, (__bf16)x.z, (__bf16)x.w};
}
__device__ __forceinline__ bf16x4 bf16_lo4(float4 x, bf16x4 h) {
  return bf16x4{(__bf16)(x.x - (float)h[0]), (__bf16)(x.y - (float)h[1]), (__bf16)(x.z - (float)h[2]),
                (__bf16)(x.w - (float)h[3])};
}

// ---------------------------------------------------------------------------------------------
// K/V of one prefill layer in bf16 hi/lo tiles for attn_prefill_tiles_kernel.  Tile (sequence sq,
// KV head kvh, keys 32t..32t+31) is 32 KiB at kvt + ((sq*2 + kvh)*ntile + t) * 32 KiB:
//   [0, 8K)   K hi: row r (key 32t + r) of 256 bytes; 16-byte segment s (dims 8s..8s+7) stored at
//             position s ^ (r & 15)
//   [8K, 16K) K lo, same layout
//   [16K,24K) V^T hi: row d (dim) of 64 bytes; segment s holds keys 4s..4s+3 then 16+4s..16+4s+3
//             (the 8 keys one lane of the P.V product needs, so it reads them with one 16-byte
//             read) at position s ^ ((d>>1)&3)
//   [24K,32K) V^T lo, same layout
// Keys past S repeat key S-1 (masked by the attention).  ds_read_b128 serves 8 consecutive lanes
// at a time from 128 bytes of banks (measured on gfx950: a 2-way conflict in those 8 lanes halves
// the read rate); the swizzles give the 8 lanes of every such group 8 distinct 16-byte bank groups
// (K: rows 256 B apart, segment XOR row; V^T: rows 64 B apart, two rows per 128 B, segment XOR
// (d>>1)&3).  grid = (ntile, 2, nseq), block = 256.
// ---------------------------------------------------------------------------------------------
constexpr int kPfTileBytes = 32768;

__global__ void __launch_bounds__(256) kv_bf16_tiles_kernel(const float* __restrict__ k_cache,
                                                            const float* __restrict__ v_cache, size_t seq_stride,
                                                            int S, uint8_t* __restrict__ kvt) {
  const int t = blockIdx.x, kvh = blockIdx.y, sq = blockIdx.z;
  const int ntile = gridDim.x;
  uint8_t* tile = kvt + ((size_t)(sq * 2 + kvh) * ntile + t) * kPfTileBytes;
  const float* kb = k_cache + (size_t)sq * seq_stride + kvh * QWEN_HEAD_DIM;
  const float* vb = v_cache + (size_t)sq * seq_stride + kvh * QWEN_HEAD_DIM;
  {  // K: thread = (row r, segment pair sp)
    const int r = threadIdx.x >> 3, sp = threadIdx.x & 7;
    const int key = min(t * kPfKeys + r, S - 1);
    const float4* src = reinterpret_cast<const float4*>(kb + (size_t)key * QWEN_KV_WIDTH + 16 * sp);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float4 x0 = src[2 * h], x1 = src[2 * h + 1];
      const bf16x4 h0 = bf16_hi4(x0), h1 = bf16_hi4(x1);
      const bf16x4 l0 = bf16_lo4(x0, h0), l1 = bf16_lo4(x1, h1);
      const int pos = ((2 * sp + h) ^ (r & 15)) * 16;
      *reinterpret_cast<bf16x8*>(tile + r * 256 + pos) = bf16x8{h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
      *reinterpret_cast<bf16x8*>(tile + 8192 + r * 256 + pos) =
          bf16x8{l0[0], l0[1], l0[2], l0[3], l1[0], l1[1], l1[2], l1[3]};
    }
  }
  {  // V^T: thread = (dim d, segment pair sp): segments 2sp and 2sp+1, i.e. keys 8sp..8sp+7 and
     // 16+8sp..16+8sp+7
    const int d = threadIdx.x >> 1, sp = threadIdx.x & 1;
    float x[16];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      x[i] = vb[(size_t)min(t * kPfKeys + 8 * sp + i, S - 1) * QWEN_KV_WIDTH + d];
      x[8 + i] = vb[(size_t)min(t * kPfKeys + 16 + 8 * sp + i, S - 1) * QWEN_KV_WIDTH + d];
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      bf16x8 vh, vl;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float xv = x[(e < 4 ? 0 : 8) + 4 * j + (e & 3)];
        vh[e] = (__bf16)xv;
        vl[e] = (__bf16)(xv - (float)vh[e]);
      }
      const int pos = ((2 * sp + j) ^ ((d >> 1) & 3)) * 16;
      *reinterpret_cast<bf16x8*>(tile + 16384 + d * 64 + pos) = vh;
      *reinterpret_cast<bf16x8*>(tile + 24576 + d * 64 + pos) = vl;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Causal prefill attention over the bf16 hi/lo tiles of kv_bf16_tiles_kernel.  Semantics of
// qwen_prefill_attention_kernel.cpp:204-289 (keys 0..p for the query at position p, scale
// 0.08838834764831845f), for S new queries at positions past..past+S-1 over past+S keys;
// online softmax (exp evaluated with __expf, inside the FAST tolerance).  Per 32-key tile and
// compute wave (lane: col = l & 15, g = l >> 4):
//   S^T = K . Q^T: A = K[key][32m + 8g..+7], B = Q[query][same dims] -> S[key 4g+r][query col];
//   online softmax per query column; P to bf16 hi/lo, keys ordered kt*16 + 4g + r;
//   O += P . V:    A = P[query col][those keys], B = V^T[dim 16n + col][the same keys].
// q rows: qkv + (sq*S + i)*qkv_stride + h*128; ctx: [sq*S + i][1536].
// Warp-specialized: waves 0-5 compute (wave w = query head kvh*6 + w, the block's 16 queries),
// wave 6 only streams tiles into a 2-stage LDS ring (64 KiB) with direct global->LDS loads, one
// tile ahead.  The compute waves never have a load in flight, so nothing drains their work.  One
// barrier per tile hands a landed tile to them and frees the stage of the tile they finished; the
// barrier keeps a block's waves in step (all in the softmax, or all in the MFMAs, at once), so two
// blocks share each CU and their phases interleave.  Measured at 8 x 2048 against one 14-wave block
// of 32 queries with a 3-stage ring per CU: 410 -> 362 us, bit-identical.
// grid = (ceil(S/16), 2, nseq) with query tiles longest first, block = 448.
// ---------------------------------------------------------------------------------------------
constexpr int kPfStages = 2;
constexpr int kPfComputeWaves = QWEN_GROUPS;  // one per query head

__global__ void __launch_bounds__(64 * (kPfComputeWaves + 1)) attn_prefill_tiles_kernel(const float* __restrict__ qkv, int qkv_stride,
                                                                 const uint8_t* __restrict__ kvt, int S, int past,
                                                                 float* __restrict__ ctx) {
  __shared__ __align__(16) uint8_t stages[kPfStages][kPfTileBytes];
  const int nqt = gridDim.x;
  const int qt = nqt - 1 - blockIdx.x;  // longest rows first
  const int kvh = blockIdx.y;
  const int sq = blockIdx.z;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int q0 = qt * kPfQ;                   // local query rows q0.. of the S new tokens
  const int nkeys = past + S;                 // keys of the sequence (past rows, then the new ones)
  const int qlast = past + min(q0 + kPfQ, S) - 1;  // last query position of the block
  const int ntiles = qlast / kPfKeys + 1;     // key tiles 0 .. qlast/32 (causal)
  const int ntile_all = (nkeys + kPfKeys - 1) / kPfKeys;
  const uint8_t* tiles = kvt + (size_t)(sq * 2 + kvh) * ntile_all * kPfTileBytes;

  if (wave >= kPfComputeWaves) {
    // producer: streams each 32 KiB tile, 32 loads of 1 KiB, one tile ahead
    auto issue = [&](int t) {
      const int tt = min(t, ntiles - 1);  // past the last tile: reload it into a stage nobody reads
      const uint8_t* src = tiles + (size_t)tt * kPfTileBytes + lane * 16;
      uint8_t* dst = stages[t % kPfStages];
#pragma unroll
      for (int i = 0; i < 32; ++i)
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(src + i * 1024),
                                         (__attribute__((address_space(3))) void*)(dst + i * 1024), 16, 0, 0);
    };
    issue(0);
    wait_vmcnt<0>();  // tile 0 landed
    __syncthreads();
    for (int t = 0; t < ntiles; ++t) {
      issue(t + 1);     // into the stage of tile t-1, freed by the barrier that ended iteration t-1
      wait_vmcnt<0>();  // tile t+1 landed
      __syncthreads();
    }
    return;
  }

  // compute wave: query head h of the GQA group, the block's 16 queries q0 .. q0+15
  const int col = lane & 15;
  const int g = lane >> 4;
  const int h = kvh * QWEN_GROUPS + wave;
  const float scaling = 0.08838834764831845f;
  bf16x8 qh[4], ql[4];
  {
    const int qi = min(q0 + col, S - 1);
    const float* qp = qkv + ((size_t)sq * S + qi) * qkv_stride + h * QWEN_HEAD_DIM + 8 * g;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const float4 x0 = *reinterpret_cast<const float4*>(qp + 32 * m);
      const float4 x1 = *reinterpret_cast<const float4*>(qp + 32 * m + 4);
      const float4 s0 = make_float4(x0.x * scaling, x0.y * scaling, x0.z * scaling, x0.w * scaling);
      const float4 s1 = make_float4(x1.x * scaling, x1.y * scaling, x1.z * scaling, x1.w * scaling);
      const bf16x4 h0 = bf16_hi4(s0), h1 = bf16_hi4(s1);
      const bf16x4 l0 = bf16_lo4(s0, h0), l1 = bf16_lo4(s1, h1);
      qh[m] = bf16x8{h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
      ql[m] = bf16x8{l0[0], l0[1], l0[2], l0[3], l1[0], l1[1], l1[2], l1[3]};
    }
  }
  const int qpos = past + q0 + col;  // position of this lane's query column
  const int qpos0 = past + q0;       // the wave's first query position
  float m_run = -INFINITY, l_run = 0.0f;
  v4f acc[8];
#pragma unroll
  for (int n = 0; n < 8; ++n) acc[n] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

  __syncthreads();  // tile 0 landed
  for (int t = 0; t < ntiles; ++t) {
    const uint8_t* T = stages[t % kPfStages];
    v4f sc[2] = {v4f{0.0f, 0.0f, 0.0f, 0.0f}, v4f{0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      const int r = kt * 16 + col;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int pos = r * 256 + (((4 * m + g) ^ (r & 15)) << 4);
        const bf16x8 ah = *reinterpret_cast<const bf16x8*>(T + pos);
        const bf16x8 al = *reinterpret_cast<const bf16x8*>(T + 8192 + pos);
        sc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, qh[m], sc[kt], 0, 0, 0);
        sc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, qh[m], sc[kt], 0, 0, 0);
        sc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, ql[m], sc[kt], 0, 0, 0);
      }
    }
    // Only a tile that reaches past the wave's first query or past the last key needs the mask.
    if (t * kPfKeys + kPfKeys - 1 > qpos0 || t * kPfKeys + kPfKeys > nkeys) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = t * kPfKeys + kt * 16 + 4 * g + r;
          if (key > qpos || key >= nkeys) sc[kt][r] = -INFINITY;
        }
    }
    float mt = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 4; ++r) mt = fmaxf(mt, sc[kt][r]);
    mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
    // Tile 0 holds key 0 <= qpos, so m_run is finite from tile 0 on; a later tile with every key
    // past qpos gives mt = -inf, corr = 1 and p = 0, leaving the column's state unchanged.
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const float mn = fmaxf(m_run, mt);
    const float corr = __expf(m_run - mn);
    float p[8];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 4; ++r) p[kt * 4 + r] = __expf(sc[kt][r] - mn);
    l_run = l_run * corr + (((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7])));
    m_run = mn;
    bf16x8 ph, pl;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      ph[e] = (__bf16)p[e];
      pl[e] = (__bf16)(p[e] - (float)ph[e]);
    }
    // The running max of most columns is unchanged by most tiles: corr is then exactly 1 and the
    // rescale is skipped unless some column of the wave needs it.
    if (__ballot(corr != 1.0f) != 0) {
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const float cr = __shfl(corr, 4 * g + rr, 64);  // lane 4g + rr holds query column 4g + rr
#pragma unroll
        for (int n = 0; n < 8; ++n) acc[n][rr] *= cr;
      }
    }
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      const int d = 16 * n + col;
      const int pv = 16384 + d * 64 + ((g ^ ((d >> 1) & 3)) << 4);  // keys 4g..4g+3, 16+4g..16+4g+3
      const bf16x8 vh = *reinterpret_cast<const bf16x8*>(T + pv);
      const bf16x8 vl = *reinterpret_cast<const bf16x8*>(T + 8192 + pv);
      acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ph, vh, acc[n], 0, 0, 0);
      acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pl, vh, acc[n], 0, 0, 0);
      acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ph, vl, acc[n], 0, 0, 0);
    }
    __syncthreads();  // done with tile t; tile t+1 has landed
  }
  float lp = l_run;
  lp += __shfl_xor(lp, 16, 64);
  lp += __shfl_xor(lp, 32, 64);
  const float inv = lp > 0.0f ? 1.0f / lp : 0.0f;  // of query column col
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) {
    const int qi = q0 + 4 * g + rr;
    const float ir = __shfl(inv, 4 * g + rr, 64);
    if (qi < S) {
      float* op = ctx + ((size_t)sq * S + qi) * QWEN_HIDDEN + h * QWEN_HEAD_DIM + col;
#pragma unroll
      for (int n = 0; n < 8; ++n) op[16 * n] = acc[n][rr] * ir;
    }
  }
}

// bf16 rounding of the driver between layers (verification/reference_wrapper_backend.py:40-46).
__global__ void round_bf16_kernel(float* __restrict__ x, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) x[i] = round_bf16(x[i]);
}

// ---------------------------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------------------------
void launch_repack_int4(const uint8_t* W, int out_dim, int in_dim, uint8_t* WP, hipStream_t st) {
  hipLaunchKernelGGL(repack_int4_kernel, dim3(out_dim / 16, in_dim / kKChunk), dim3(64), 0, st, W, in_dim, WP);
}

void launch_norm_quant(const float* x, size_t x_stride, int rows, int n, const float* w, int norm, int8_t* xq,
                       float* sx, int* sums, float* xn, hipStream_t st) {
  // many rows (prefill): one wave per row
  if (rows >= 256 && !xn && norm != kNormDecode && (n == QWEN_HIDDEN || n == QWEN_INTERMEDIATE) && x_stride % 4 == 0) {
    const dim3 grid((unsigned)((rows + 3) / 4));
    if (n == QWEN_HIDDEN)
      hipLaunchKernelGGL(quant_rows_wave_kernel<QWEN_HIDDEN / 256>, grid, dim3(256), 0, st, x, x_stride, rows, w, norm,
                         xq, sx, sums);
    else
      hipLaunchKernelGGL(quant_rows_wave_kernel<QWEN_INTERMEDIATE / 256>, grid, dim3(256), 0, st, x, x_stride, rows,
                         w, norm, xq, sx, sums);
    return;
  }
  if (n <= 2048)
    hipLaunchKernelGGL(norm_quant_kernel<2>, dim3(rows), dim3(256), 0, st, x, x_stride, n, w, norm, xq, sx, sums, xn);
  else
    hipLaunchKernelGGL(norm_quant_kernel<kQuantVecs>, dim3(rows), dim3(256), 0, st, x, x_stride, n, w, norm, xq, sx,
                       sums, xn);
}

template <int NT, int KSPLIT, int EPI, bool DUAL>
static void launch_gemm_t(const GemmArgs& a, hipStream_t st) {
  constexpr int RTB = 4 / KSPLIT;
  const int row_tiles = a.out_dim / 16;
  const dim3 grid((a.tokens + 16 * NT - 1) / (16 * NT), (row_tiles + RTB - 1) / RTB);
  hipLaunchKernelGGL((gemm_i8_kernel<NT, KSPLIT, EPI, DUAL>), grid, dim3(256), 0, st, a);
}

// The reduce step after a GEMM that wrote fp32 partials: plain (bias / residual epilogue) or fused.
template <int EPI>
static void launch_reduce(const GemmArgs& a, int splits, hipStream_t st) {
  if (a.fuse == kFuseQkvRope) {
    hipLaunchKernelGGL(reduce_qkv_rope_kernel, dim3(a.tokens), dim3(256), 0, st, a, splits);
  } else if (a.fuse == kFuseNormQuant) {
    if (a.out_dim == QWEN_HIDDEN && splits <= 5 && (EPI != kEpiResidual || a.resid_stride == QWEN_HIDDEN)) {
      // the first loads' operands preloaded (an absent bias or norm weight read from the row scales)
      const void* add = EPI == kEpiResidual ? (const void*)a.resid : a.bias ? (const void*)a.bias : a.sw;
      const void* nw = a.norm != kNormNone ? (const void*)a.norm_w : a.sw;
      hipLaunchKernelGGL((reduce_norm_quant_pair_hot_kernel<EPI>), dim3(a.tokens), dim3(128), 0, st,
                         (const void*)a.part, add, (const void*)a.sw, nw, (const void*)a.sums, (const void*)a.sx,
                         a.tokens, splits, a);
    } else if (a.out_dim == QWEN_HIDDEN)
      hipLaunchKernelGGL((reduce_norm_quant_pair_kernel<EPI>), dim3(a.tokens), dim3(128), 0, st, a, splits);
    else
      hipLaunchKernelGGL((reduce_norm_quant_kernel<EPI>), dim3(a.tokens), dim3(256), 0, st, a, splits);
  } else {
    const size_t quads = (size_t)a.tokens * (a.out_dim / 4);
    hipLaunchKernelGGL((gemm_splitk_reduce_kernel<EPI>), dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, st, a,
                       splits);
  }
}

template <int NT, int RTW, int NBUF, int EPI, bool DUAL, int TW = 1, int WPE = 1, bool OWN = false, bool ROPE = false>
static void launch_gemm_pipe_t(const GemmArgs& a, int splits, hipStream_t st) {
  const int row_tiles = a.out_dim / 16;
  const int nblk = ((a.tokens + 16 * NT * TW - 1) / (16 * NT * TW)) * ((row_tiles + 4 * RTW - 1) / (4 * RTW));
  const dim3 grid(8 * ((nblk + 7) / 8), 1, splits);
  // epilogue form: the int32 limb combination where in_dim allows it, and the SiLU the call asks for
  const bool int_sum = a.in_dim <= kIntSumMaxK;
  auto go = [&](auto ef) {
    hipLaunchKernelGGL((gemm_i8_pipe_kernel<NT, RTW, NBUF, EPI, DUAL, TW, WPE, OWN, ROPE, decltype(ef)::value>), grid,
                       dim3(256 * TW), 0, st, a);
  };
  if constexpr (EPI == kEpiSiluMul) {
    if (a.prefill_silu)
      int_sum ? go(std::integral_constant<int, kEfPrefillSilu | kEfIntSum>{})
              : go(std::integral_constant<int, kEfPrefillSilu>{});
    else
      int_sum ? go(std::integral_constant<int, kEfIntSum>{}) : go(std::integral_constant<int, 0>{});
  } else if constexpr (ROPE) {
    go(std::integral_constant<int, 0>{});  // the RoPE epilogue has its own dequantization
  } else {
    int_sum ? go(std::integral_constant<int, kEfIntSum>{}) : go(std::integral_constant<int, 0>{});
  }
  // K splits, or an epilogue fused into the reduce step, finish in the reduce kernel; the prefill RoPE
  // epilogue is complete in the GEMM itself
  if (!DUAL && !ROPE && (splits > 1 || a.fuse != kFuseNone)) launch_reduce<EPI>(a, splits, st);
}

// Skinny GEMMs for at most kSkinnyTokens tokens with in_dim 1536 (12 K chunks in one block) or 8960
// (5 splits of 14 chunks, finished by the reduce step).  Returns false for other shapes.

template <int RTW, bool DUAL, int EPI, int NKC, bool ROPE, int KSW = 1, bool GRP = false>
static void launch_skinny_t(const GemmArgs& a, int rg_count, int splits, hipStream_t st) {
  // the grouped code's per-group sums are only finished by the split-K partial epilogue
  if (GRP && splits <= 1) throw std::runtime_error("grouped-code GEMM needs the split-K partial epilogue");
  const int tt = (a.tokens + 15) / 16;
  const int groups = rg_count * splits;
  const int blocks = 8 * tt * ((groups + 7) / 8);
  // the model's shapes: the kernel with the first loads' operands preloaded
  constexpr int kIn = NKC == 12 ? QWEN_HIDDEN : NKC == 14 ? QWEN_INTERMEDIATE : 0;
  constexpr int kOut = NKC == 14 ? QWEN_HIDDEN : ROPE ? QWEN_QKV_ROWS : DUAL ? QWEN_INTERMEDIATE : QWEN_HIDDEN;
  if (kIn > 0 && a.in_dim == kIn && a.out_dim == kOut && splits * NKC * kKChunk == kIn) {
    const void* p2 = GRP ? (const void*)a.gsx : DUAL ? (const void*)a.wp2 : nullptr;
    const void* p3 = GRP ? (const void*)a.gcorr : ROPE ? (const void*)a.pos : DUAL ? (const void*)a.gsx_out : nullptr;
    hipLaunchKernelGGL((gemm_skinny_hot_kernel<RTW, DUAL, EPI, NKC, ROPE, KSW, GRP, kIn, kOut>), dim3(blocks),
                       dim3(256 * KSW), 0, st, (const void*)a.xq, (const void*)a.wp, p2, p3, a.tokens, tt, rg_count,
                       splits, a);
    return;
  }
  hipLaunchKernelGGL((gemm_skinny_kernel<RTW, DUAL, EPI, NKC, ROPE, KSW, GRP>), dim3(blocks), dim3(256 * KSW), 0, st, a,
                     tt, rg_count, splits);
}

template <int EPI, bool DUAL>
static bool launch_skinny(const GemmArgs& a, hipStream_t st) {
  if (a.tokens > kSkinnyTokens || a.out_dim % 64 != 0) return false;
  const int row_tiles = a.out_dim / 16;
  if (a.in_dim == QWEN_HIDDEN) {
    if (!DUAL && EPI == kEpiStore && a.fuse == kFuseQkvRope) {
      if (a.out_dim != QWEN_QKV_ROWS) return false;
      // more than one token tile: two wave groups split K (twice the loads in flight per block;
      // 4.225 -> 4.210 ms per 64-sequence decode step)
      if (a.tokens > 16)
        launch_skinny_t<2, false, kEpiStore, 12, true, 2>(a, row_tiles / 8, 1, st);
      else
        launch_skinny_t<2, false, kEpiStore, 12, true, 1>(a, row_tiles / 8, 1, st);
      return true;
    }
    if (!DUAL && a.fuse != kFuseNone && !a.part) return false;
    // the O shape over more than one token tile: two wave groups split K, as Q/K/V (64 x 4096 decode
    // +0.25%, interleaved; the sums are exact int32, so the bits are the same)
    if (!DUAL && a.tokens > 16 && a.out_dim == QWEN_HIDDEN)
      launch_skinny_t<1, false, EPI, 12, false, 2>(a, row_tiles / 4, 1, st);
    else
      launch_skinny_t<1, DUAL, EPI, 12, false>(a, row_tiles / 4, 1, st);
    if (!DUAL && a.fuse != kFuseNone && !(a.defer_reduce && a.tokens == 1 && a.fuse == kFuseNormQuant))
      launch_reduce<EPI>(a, 1, st);
    return true;
  }
  if constexpr (!DUAL) {
    if (a.in_dim == QWEN_INTERMEDIATE && a.part && a.fuse != kFuseQkvRope) {
      if (a.gsx && a.gcorr)  // the grouped code of the SiLU·up rows
        launch_skinny_t<1, false, EPI, 14, false, 1, true>(a, row_tiles / 4, 5, st);
      else
        launch_skinny_t<1, false, EPI, 14, false>(a, row_tiles / 4, 5, st);
      if (!(a.defer_reduce && a.tokens == 1 && a.fuse == kFuseNormQuant)) launch_reduce<EPI>(a, 5, st);
      return true;
    }
  }
  return false;
}

// Largest divisor of nkc that is <= want (K chunks split evenly over blocks).
static int split_for(int nkc, int want) {
  for (int s = want < kMaxSplits ? want : kMaxSplits; s > 1; --s)
    if (nkc % s == 0) return s;
  return 1;
}

// Shape dispatch (the split-K workspace a.part, when given, holds kMaxSplits x kSplitTokens x
// out_dim floats).  <= 16 tokens: direct-load kernel, 4-way in-block K split per row tile (many
// small blocks, weights streamed once).  More tokens: the pipelined LDS kernel; projections whose
// row tiles alone give fewer than ~256 blocks are also split over K across blocks (needs a.part).
template <int EPI, bool DUAL>
static void launch_gemm_epi(const GemmArgs& a, hipStream_t st) {
  const int nkc = a.in_dim / kKChunk;
  const int row_tiles = a.out_dim / 16;
  // The grouped SiLU·up code (gsx/gcorr read by the down projection, gsx_out/gcorr_out written by
  // gate/up) exists only in the skinny kernels: any other kernel would ignore it, reading the zero
  // limb sums or leaving the code stale.  Such a call either takes the skinny kernel or fails.
  const bool grouped_in = a.gsx != nullptr || a.gcorr != nullptr;
  const bool grouped_out = a.gsx_out != nullptr || a.gcorr_out != nullptr;
  if (grouped_in || grouped_out) {
    const bool in_ok = !grouped_in || (!DUAL && a.gsx && a.gcorr && a.in_dim == QWEN_INTERMEDIATE && a.part &&
                                       a.fuse != kFuseQkvRope);
    const bool out_ok = !grouped_out || (DUAL && EPI == kEpiSiluMul && a.gsx_out && a.gcorr_out && a.xq_out &&
                                         a.in_dim == QWEN_HIDDEN);
    if (!in_ok || !out_ok || !launch_skinny<EPI, DUAL>(a, st))
      throw std::runtime_error("grouped SiLU·up code outside the skinny GEMM shapes (<= 64 tokens, out_dim a "
                               "multiple of 64, gate/up writing it or the split-K down projection reading it)");
    return;
  }
  if (launch_skinny<EPI, DUAL>(a, st)) return;
  if (a.tokens <= 16) {
    launch_gemm_t<1, 4, EPI, DUAL>(a, st);
    if (!DUAL && a.fuse != kFuseNone) launch_reduce<EPI>(a, 1, st);
    return;
  }
  // Many tokens (prefill): 4-wave blocks of 64 tokens with two LDS stages (64 KiB), two blocks per
  // CU.  Measured against one 8-wave block of 128 tokens with three stages (144 KiB) per CU at 16,384
  // tokens: gate/up 0.94-0.98 -> 0.79 ms, down 0.38-0.40 -> 0.34 ms, QKV 111-118 -> 97-100 us.
  if (a.tokens > kSplitTokens && a.fuse == kFuseNone) {
    if constexpr (DUAL)
      launch_gemm_pipe_t<4, 2, 2, EPI, DUAL, 1, 2, true>(a, 1, st);
    else
      launch_gemm_pipe_t<4, 4, 2, EPI, DUAL, 1, 2, true>(a, 1, st);
    return;
  }
  if constexpr (!DUAL && EPI == kEpiStore) {
    if (a.fuse == kFuseRopePrefill) {
      if (a.tokens <= kSplitTokens || a.out_dim != QWEN_QKV_ROWS || a.seq_len <= 0 || a.past < 0 || !a.rope ||
          !a.k_cache || !a.v_cache)
        throw std::runtime_error("prefill RoPE epilogue: more than 256 tokens of the [q | k | v] projection");
      launch_gemm_pipe_t<4, 4, 2, EPI, DUAL, 1, 2, true, true>(a, 1, st);
      return;
    }
  }
  if constexpr (DUAL) {
    if (a.tokens <= 64)
      launch_gemm_pipe_t<4, 1, 4, EPI, DUAL>(a, 1, st);
    else
      launch_gemm_pipe_t<4, 2, 4, EPI, DUAL>(a, 1, st);
  } else {
    if (a.tokens <= 64) {
      const int blocks = (row_tiles + 3) / 4;
      const int splits = a.part ? split_for(nkc, (256 + blocks - 1) / blocks) : 1;
      launch_gemm_pipe_t<4, 1, 4, EPI, DUAL>(a, splits, st);  // a.part holds >= kSplitTokens rows
    } else {
      const int token_tiles = (a.tokens + 63) / 64;
      const int blocks = token_tiles * ((row_tiles + 15) / 16);
      const int splits =
          (a.part && a.tokens <= kSplitTokens && blocks < 256) ? split_for(nkc, (256 + blocks - 1) / blocks) : 1;
      launch_gemm_pipe_t<4, 4, 4, EPI, DUAL>(a, splits, st);
    }
  }
}

// gate/up after O: kGateUpTiles 16-row tiles of both matrices per block, K split over its four waves;
// one block (and one row maximum) per group of tiles, the group count rounded up to a multiple of 4
// for the maxima's float4 reads (the groups past the last tile write a maximum of 0)
constexpr int kGateUpTiles = 3;
int gate_up_maxima_count(int out_dim) {
  const int groups = (out_dim / 16 + kGateUpTiles - 1) / kGateUpTiles;
  return (groups + 3) / 4 * 4;
}

// The operands of a one-token reduce prologue's first loads (HotArgs p0..p5): partials, residual (its
// bias, or the row scales as a stand-in), row scales, norm weights (or the stand-in), limb sums, scale.
struct PreHotPtrs {
  const void* p[6];
};
static PreHotPtrs pre_hot_ptrs(const GemmArgs& pre, int pre_epi) {
  const void* add = pre_epi == kEpiResidual ? (const void*)pre.resid : pre.bias ? (const void*)pre.bias : pre.sw;
  const void* nw = pre.norm != kNormNone ? (const void*)pre.norm_w : pre.sw;
  return PreHotPtrs{{pre.part, add, pre.sw, nw, pre.sums, pre.sx}};
}

bool launch_gemm_i8_pre(const GemmArgs& a, const GemmArgs& pre, int pre_epi, int pre_splits, hipStream_t st) {
  if (a.tokens != 1 || a.in_dim != QWEN_HIDDEN || pre.out_dim != QWEN_HIDDEN || pre.fuse != kFuseNormQuant ||
      pre.tokens != 1 || pre_splits < 1 ||
      pre_splits > (pre_epi == kEpiResidual ? kPreResidualSplits : kOneTokenOSplits))
    return false;
  if (a.wp2 && a.out_dim % 64 == 0 && pre_epi == kEpiStore && !a.prefill_silu) {  // decode gate/up after O
    const int rg_count = gate_up_maxima_count(a.out_dim);
    const dim3 grid(8 * ((rg_count + 7) / 8));
    if (a.out_dim == QWEN_INTERMEDIATE) {
      const PreHotPtrs h = pre_hot_ptrs(pre, pre_epi);
      hipLaunchKernelGGL(
          (gemm_skinny_pre_kw_hot_kernel<kGateUpTiles, true, kEpiSiluMul, 12, kEpiStore, QWEN_INTERMEDIATE>), grid,
          dim3(256), 0, st, h.p[0], h.p[1], h.p[2], h.p[3], h.p[4], h.p[5], rg_count, pre_splits, a, pre);
    } else {
      hipLaunchKernelGGL((gemm_skinny_pre_kw_kernel<kGateUpTiles, true, kEpiSiluMul, 12, kEpiStore>), grid,
                         dim3(256), 0, st, a, rg_count, pre, pre_splits);
    }
    return true;
  }
  if (!a.wp2 && a.fuse == kFuseQkvRope && a.out_dim == QWEN_QKV_ROWS && pre_epi == kEpiResidual) {
    // Q/K/V + RoPE + KV append after the previous layer's down projection
    const int rg_count = a.out_dim / 128;
    hipLaunchKernelGGL((gemm_skinny_pre_kernel<2, false, kEpiStore, 12, true, kEpiResidual>),
                       dim3(8 * ((rg_count + 7) / 8)), dim3(256), 0, st, a, rg_count, pre, pre_splits);
    return true;
  }
  return false;
}

bool launch_gemm_i8_prea(const GemmArgs& a, const AttnMergeArgs& am, hipStream_t st) {
  if (a.tokens != 1 || a.in_dim != QWEN_HIDDEN || a.out_dim != QWEN_HIDDEN || a.wp2 || !a.part ||
      a.fuse != kFuseNormQuant || !am.part || !am.pml || !am.pos || !am.sx_out || !am.sums_out || am.nsplit < 1 ||
      am.nsplit > kAttnMaxSplits || am.chunk < 1)
    return false;
  // one 16-row tile and one of kOneTokenOSplits head ranges (K ranges) per block, K split over its four
  // waves; the merge loads 8, 12 or 16 splits at once.  (With more than one range each range's partial
  // carries its own offset correction, so the reduce step must run with zero limb sums: only the
  // deferred form, whose caller passes them, is offered.)
  constexpr int kSplits = kOneTokenOSplits, kNkc = QWEN_Q_HEADS / kSplits;
  if (kSplits > 1 && !a.defer_reduce) return false;
  const int rg_count = a.out_dim / 16;
  const dim3 grid(8 * ((rg_count * kSplits + 7) / 8));
  // (the merge's operands preloaded; without the new key's row the partials stand in for it, unread)
  const void* qkv_new = am.qkv_new ? (const void*)am.qkv_new : am.part;
  auto go = [&](auto newkey, auto kf) {
    hipLaunchKernelGGL((gemm_skinny_prea_hot_kernel<kEpiStore, kNkc, decltype(newkey)::value, decltype(kf)::value>),
                       grid, dim3(256), 0, st, am.part, am.pml, am.pos, qkv_new, am.nsplit, rg_count, a, am);
  };
  using K8 = std::integral_constant<int, 8>;
  using K12 = std::integral_constant<int, 12>;
  using K16 = std::integral_constant<int, 16>;
  if (am.qkv_new) {
    if (am.nsplit <= 8) go(std::true_type{}, K8{});
    else if (am.nsplit <= 12) go(std::true_type{}, K12{});
    else go(std::true_type{}, K16{});
  } else {
    if (am.nsplit <= 8) go(std::false_type{}, K8{});
    else if (am.nsplit <= 12) go(std::false_type{}, K12{});
    else go(std::false_type{}, K16{});
  }
  if (!a.defer_reduce) launch_reduce<kEpiStore>(a, kSplits, st);
  return true;
}

// Blocks of the fused Q/K/V + attention launch: ids 0..7 (the four k and v heads, four idle), then 8
// per six-head group of 8 (KV head, key split) pairs.
static int fused_attn_blocks(int nsplit) {
  return 8 + 8 * QWEN_GROUPS * ((QWEN_KV_HEADS * nsplit + 7) / 8);
}

static bool fused_attn_ok(const GemmArgs& a, const AttnFuseArgs& af) {
  return a.tokens == 1 && a.in_dim == QWEN_HIDDEN && a.out_dim == QWEN_QKV_ROWS && !a.wp2 &&
         a.fuse == kFuseQkvRope && a.pos && a.rope && a.k_cache && a.v_cache && a.y && af.part && af.pml &&
         af.chunk == kFusedAttnChunk && af.nsplit >= 1 && af.nsplit <= kFusedAttnMaxSplits && af.max_keys >= 1 &&
         af.max_keys <= af.nsplit * af.chunk && a.limit >= 1;
}

bool launch_gemm_i8_attn(const GemmArgs& a, const AttnFuseArgs& af, hipStream_t st) {
  if (!fused_attn_ok(a, af) || !a.xq) return false;
  hipLaunchKernelGGL(gemm_skinny_attn_kernel, dim3(fused_attn_blocks(af.nsplit)), dim3(256), 0, st, a, af);
  return true;
}

bool launch_gemm_i8_pre_attn(const GemmArgs& a, const GemmArgs& pre, int pre_splits, const AttnFuseArgs& af,
                             hipStream_t st) {
  // pre_splits == 0: the row is pre.resid itself (the first layer of a range: RMSNorm and quantization
  // of the input row, pre.sums / pre.sx pointing at zeros, nothing written back)
  if (!fused_attn_ok(a, af) || pre.out_dim != QWEN_HIDDEN || pre.fuse != kFuseNormQuant || pre.tokens != 1 ||
      pre_splits < 0 || pre_splits > kPreResidualSplits || (pre_splits == 0 && (!pre.resid || pre.y || pre.y_raw)))
    return false;
  const PreHotPtrs h = pre_hot_ptrs(pre, kEpiResidual);
  hipLaunchKernelGGL(gemm_skinny_pre_attn_hot_kernel, dim3(fused_attn_blocks(af.nsplit)), dim3(256), 0, st, h.p[0],
                     h.p[1], h.p[2], h.p[3], h.p[4], h.p[5], af.nsplit, pre_splits, a, pre, af);
  return true;
}

bool launch_gemm_i8_preq(const GemmArgs& a, const GemmArgs& pre, hipStream_t st) {
  if (a.tokens != 1 || a.in_dim != QWEN_INTERMEDIATE || a.out_dim != QWEN_HIDDEN || a.wp2 || !a.part ||
      pre.in_dim != a.in_dim || !pre.y || !pre.sx_out || !pre.sums_out)
    return false;
  constexpr int kSplits = kPreResidualSplits;  // 14 K chunks each, as the separate-quantization path
  // two 16-row tiles per block, their 14 K chunks split over the block's four waves (4, 4, 3, 3): 240
  // blocks (every block quantizes the whole 8960-wide row for its scale, so fewer blocks than the other
  // one-token projections: 480 blocks of one tile, or 160 of three, were slower)
  const int rg_count = a.out_dim / 32;
  if (pre.amax_in && (pre.amax_n < 4 || pre.amax_n % 4 != 0 || pre.amax_n > 1024)) return false;
  // (with per-block maxima: one more block, the row's scale and limb sums)
  if (pre.amax_in)
    hipLaunchKernelGGL((gemm_skinny_preq_hot_kernel<2, kEpiResidual, 14>), dim3(8 * ((rg_count * kSplits + 7) / 8) + 1),
                       dim3(256), 0, st, pre.y, pre.amax_in, pre.amax_n, rg_count, kSplits, a, pre);
  else
    hipLaunchKernelGGL((gemm_skinny_preq_kernel<2, kEpiResidual, 14, true>), dim3(8 * ((rg_count * kSplits + 7) / 8)),
                       dim3(256), 0, st, a, rg_count, kSplits, pre);
  if (!(a.defer_reduce && a.fuse == kFuseNormQuant)) launch_reduce<kEpiResidual>(a, kSplits, st);
  return true;
}

void launch_gemm_i8(const GemmArgs& a, int epi, hipStream_t st) {
  switch (epi) {
    case kEpiStore: launch_gemm_epi<kEpiStore, false>(a, st); break;
    case kEpiSiluMul: launch_gemm_epi<kEpiSiluMul, true>(a, st); break;
    case kEpiResidual: launch_gemm_epi<kEpiResidual, false>(a, st); break;
    default: break;
  }
}

void launch_rope_qkv(float* qkv, int qkv_stride, const int* pos, int seq_len, int past, int limit, int tokens,
                     const float* rope, float* k_cache, float* v_cache, size_t seq_stride, hipStream_t st) {
  hipLaunchKernelGGL(rope_qkv_kernel, dim3(tokens), dim3(64), 0, st, qkv, qkv_stride, pos, seq_len, past, limit,
                     rope, k_cache, v_cache, seq_stride);
}

constexpr int kAttnMinChunk = 64;
constexpr int kAttnSoftSplits = 24;

AttnDecodePlan plan_attn_decode(int batch, int max_keys, int cus) {
  // co-resident blocks of attn_decode_kernel on the current device (CUs x blocks per CU)
  static const int2 dev_slots = [] {
    int dev = 0, per_cu = 0;
    hipDeviceProp_t prop;
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess) return int2{256, 4};
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, attn_decode_kernel, 256, 0) != hipSuccess || per_cu < 1)
      per_cu = 1;
    return int2{prop.multiProcessorCount, per_cu};
  }();
  // at most 3 co-resident blocks per CU: the KV stream runs faster at 12 than at 16 waves per CU
  const int slots = (cus > 0 && cus < dev_slots.x ? cus : dev_slots.x) * (dev_slots.y < 3 ? dev_slots.y : 3);
  int nsplit = slots / (QWEN_KV_HEADS * (batch > 0 ? batch : 1));
  nsplit = nsplit < 1 ? 1 : (nsplit > kAttnMaxSplits ? kAttnMaxSplits : nsplit);
  int chunk = (max_keys + nsplit - 1) / nsplit;
  // Small batches cannot fill the device: each extra split then costs more in the merge (one memory
  // round trip per 8 splits) than it saves.  Measured on MI355X (batch 1-16, 544 and 4128 keys):
  // at least 64 keys per split and at most 24 splits.
  chunk = max(chunk, max(kAttnMinChunk, (max_keys + kAttnSoftSplits - 1) / kAttnSoftSplits));
  chunk = (chunk + 15) & ~15;  // whole 16-key tiles
  return AttnDecodePlan{(max_keys + chunk - 1) / chunk, chunk};
}

void launch_zero_u32(unsigned* p, int n, hipStream_t st) {
  hipLaunchKernelGGL(zero_u32_kernel, dim3((n + 255) / 256), dim3(256), 0, st, p, n);
}

void launch_attn_decode(const float* qkv, int qkv_stride, const float* k_cache, const float* v_cache,
                        size_t seq_stride, const int* pos, int batch, int max_keys, const AttnDecodePlan& plan,
                        float* part, float2* pml, float* ctx, int8_t* xq, float* sx, int* sums, hipStream_t st) {
  hipLaunchKernelGGL(attn_decode_kernel, dim3(plan.nsplit, QWEN_KV_HEADS, batch), dim3(256), 0, st, qkv, qkv_stride,
                     k_cache, v_cache, seq_stride, pos, plan.chunk, max_keys, part, pml);
  if (xq)
    hipLaunchKernelGGL(attn_decode_merge_kernel, dim3(batch), dim3(256), 0, st, part, pml, pos, plan.nsplit, plan.chunk,
                       max_keys, ctx, xq, sx, sums);
}

size_t attn_prefill_workspace_bytes(int keys, int nseq) {
  return (size_t)nseq * QWEN_KV_HEADS * ((keys + kPfKeys - 1) / kPfKeys) * kPfTileBytes;
}

void launch_attn_prefill(const float* qkv, int qkv_stride, const float* k_cache, const float* v_cache,
                         size_t seq_stride, int S, int past, int nseq, uint8_t* kv_tiles, float* ctx,
                         hipStream_t st) {
  const int keys = past + S;
  const int ntile = (keys + kPfKeys - 1) / kPfKeys;
  hipLaunchKernelGGL(kv_bf16_tiles_kernel, dim3(ntile, QWEN_KV_HEADS, nseq), dim3(256), 0, st, k_cache, v_cache,
                     seq_stride, keys, kv_tiles);
  hipLaunchKernelGGL(attn_prefill_tiles_kernel, dim3((S + kPfQ - 1) / kPfQ, QWEN_KV_HEADS, nseq),
                     dim3(64 * (kPfComputeWaves + 1)), 0, st,
                     qkv, qkv_stride, kv_tiles, S, past, ctx);
}

void launch_round_bf16(float* x, size_t n, hipStream_t st) {
  hipLaunchKernelGGL(round_bf16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, n);
}

}  // namespace qwen
