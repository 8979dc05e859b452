// Device-side weight quantizer, synthetic-input generators and the embedding gather.
//
// The quantizer restates verification/real_host_top_backend.py:31-41 on the GPU (bit-exact: the
// row max is order-independent, and the fp32 division and rint are IEEE); this file is built
// with -ffp-contract=off like the ORDERED kernels.
#include <hip/hip_runtime.h>

#include "kernels.hpp"
#include "qwen_device_math.hpp"

namespace qwen {

// ---- counter-based normal generator -------------------------------------------------------
QWEN_HD uint64_t splitmix64(uint64_t x) {
  uint64_t z = x + 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// Stream key of one tensor (seed, tensor key).
QWEN_HD uint64_t tensor_stream(uint64_t seed, uint64_t key) { return splitmix64(seed ^ splitmix64(key + 1u)); }

// Irwin-Hall sum of 12 uniforms of 24 bits minus 6: mean 0, variance 1, computed exactly.
QWEN_HD double irwin_hall12(uint64_t stream, uint64_t idx) {
  uint64_t s = 0;
  for (int k = 0; k < 12; ++k) s += splitmix64(stream + idx * 12u + (uint64_t)k) >> 40;
  return (double)s * (1.0 / 16777216.0) - 6.0;
}

QWEN_HD float synth_value(uint64_t stream, uint64_t idx, float sigma, int bf16) {
  const float v = (float)(irwin_hall12(stream, idx) * (double)sigma);
  return bf16 ? round_bf16(v) : v;
}

// ---------------------------------------------------------------------------------------------
// Per-row INT4 quantization, one 256-thread block per row.  Values come from `src` ([out][in]
// fp32) or, when src is null, from the synthetic generator (stream, sigma, bf16 rounding).
// ---------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) quantize_rows_kernel(const float* __restrict__ src, int in_dim,
                                                            uint64_t stream, float sigma, uint8_t* __restrict__ packed,
                                                            float* __restrict__ scales) {
  __shared__ float row[kMaxQuantRow];
  __shared__ float red[4];
  const int o = blockIdx.x;
  const size_t base = (size_t)o * (size_t)in_dim;
  float amax = 0.0f;
  for (int i = threadIdx.x; i < in_dim; i += 256) {
    const float v = src ? src[base + i] : synth_value(stream, base + i, sigma, 1);
    row[i] = v;
    amax = fmaxf(amax, fabsf(v));
  }
  for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float scale = amax > 0.0f ? amax / 7.0f : 1.0f;
  if (threadIdx.x == 0) scales[o] = scale;
  for (int j = threadIdx.x; j < in_dim / 2; j += 256) {
    int q0 = (int)rintf(row[2 * j] / scale);
    int q1 = (int)rintf(row[2 * j + 1] / scale);
    q0 = q0 < -8 ? -8 : (q0 > 7 ? 7 : q0);
    q1 = q1 < -8 ? -8 : (q1 > 7 ? 7 : q1);
    packed[base / 2 + j] = (uint8_t)((q0 & 0xF) | ((q1 & 0xF) << 4));
  }
}

// dst[i] = synthetic value (bf16-rounded when bf16 != 0), or `constant` when sigma == 0.
__global__ void fill_vector_kernel(float* __restrict__ dst, size_t n, uint64_t stream, float sigma, int bf16,
                                   float constant) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  dst[i] = sigma == 0.0f ? constant : synth_value(stream, i, sigma, bf16);
}

// bf16 table rows: bits of bf16(N(0, sigma)).
__global__ void fill_bf16_table_kernel(uint16_t* __restrict__ dst, size_t n, uint64_t stream, float sigma) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  dst[i] = (uint16_t)(f32_bits(synth_value(stream, i, sigma, 1)) >> 16);
}

// KV rows of 256: N(0,1), quantized per row to INT4 (max|x|/7) and dequantized.  One wave per row.
__global__ void __launch_bounds__(256) kv_synthetic_kernel(float* __restrict__ cache, uint64_t rows, uint64_t stream) {
  const uint64_t r = (uint64_t)blockIdx.x * 4u + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int lane = threadIdx.x & 63;
  float v[4];
  float amax = 0.0f;
  for (int j = 0; j < 4; ++j) {
    v[j] = synth_value(stream, r * QWEN_KV_WIDTH + lane + 64 * j, 1.0f, 0);
    amax = fmaxf(amax, fabsf(v[j]));
  }
  for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  const float scale = amax > 0.0f ? amax / 7.0f : 1.0f;
  float* out = cache + r * QWEN_KV_WIDTH;
  for (int j = 0; j < 4; ++j) {
    int q = (int)rintf(v[j] / scale);
    q = q < -8 ? -8 : (q > 7 ? 7 : q);
    out[lane + 64 * j] = (float)q * scale;
  }
}

__global__ void embed_kernel(const uint16_t* __restrict__ table, int vocab, const int* __restrict__ ids, int count,
                             float* __restrict__ hidden) {
  const int t = blockIdx.x;
  const int id = ids[t];
  const size_t row = (size_t)(id >= 0 && id < vocab ? id : 0) * QWEN_HIDDEN;  // out-of-range ids read row 0
  for (int d = threadIdx.x; d < QWEN_HIDDEN; d += blockDim.x)
    hidden[(size_t)t * QWEN_HIDDEN + d] = bits_f32((uint32_t)table[row + d] << 16);
}

// Host-compatible expf over a strided sweep of bit patterns (test hook).
__global__ void eval_expf_kernel(uint32_t first, uint32_t stride, uint64_t n, float* __restrict__ y) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint32_t bits = first + (uint32_t)i * stride;
  y[i] = glibc_expf(bits_f32(bits));
}

// ---------------------------------------------------------------------------------------------
void launch_eval_expf(uint32_t first, uint32_t stride, uint64_t n, float* y, hipStream_t st) {
  hipLaunchKernelGGL(eval_expf_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, first, stride, n, y);
}

void launch_quantize_rows(const float* src, int out_dim, int in_dim, uint64_t stream, float sigma, uint8_t* packed,
                          float* scales, hipStream_t st) {
  hipLaunchKernelGGL(quantize_rows_kernel, dim3(out_dim), dim3(256), 0, st, src, in_dim, stream, sigma, packed, scales);
}

void launch_fill_vector(float* dst, size_t n, uint64_t stream, float sigma, int bf16, float constant, hipStream_t st) {
  hipLaunchKernelGGL(fill_vector_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, dst, n, stream, sigma,
                     bf16, constant);
}

void launch_fill_bf16_table(uint16_t* dst, size_t n, uint64_t stream, float sigma, hipStream_t st) {
  hipLaunchKernelGGL(fill_bf16_table_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, dst, n, stream,
                     sigma);
}

void launch_kv_synthetic(float* cache, uint64_t rows, uint64_t stream, hipStream_t st) {
  hipLaunchKernelGGL(kv_synthetic_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, cache, rows, stream);
}

void launch_embed(const uint16_t* table, int vocab, const int* ids, int count, float* hidden, hipStream_t st) {
  hipLaunchKernelGGL(embed_kernel, dim3(count), dim3(256), 0, st, table, vocab, ids, count, hidden);
}

}  // namespace qwen

namespace qwen {
uint64_t synth_stream_host(uint64_t seed, uint64_t key) { return tensor_stream(seed, key); }
}  // namespace qwen
