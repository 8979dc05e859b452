// Unquantized layer-0 reference path (the reference's model-fidelity wrappers):
//   decode  hls/decode_only/qwen_decode_layer0_reference_wrapper.cpp:75-209
//   prefill hls/prefill_only/qwen_prefill_layer0_reference_wrapper.cpp:60-347
// fp32 weights, every linear output accumulated in double in input order (bias first) and rounded
// to bf16; attention scores, softmax and context in double; the residual stream in fp32.  The two
// wrappers differ in their RMSNorm (decode: double mean square, one rounding; prefill: fp32 mean
// square, input rounded to bf16 before the weight) and RoPE (decode: fp32 rotation; prefill: every
// product and sum rounded to bf16).  The order of every serial sum is the reference's: one thread
// owns each chain.  Built without FMA contraction; double products of fp32 values are exact, so the
// double chains are the reference's sums bit for bit.  RoPE cos/sin come from the host's libm.
#include <hip/hip_runtime.h>

#include "kernels.hpp"
#include "qwen_device_math.hpp"

namespace qwen {

namespace {

constexpr int kL0TokTile = 8;  // tokens per thread of the linear kernel (weights read once per tile)

// RMSNorm of one token row (grid = tokens, block = 64).  Thread 0 forms the serial mean square.
__global__ void l0_rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ w, float eps, int prefill,
                                  float* __restrict__ out) {
  __shared__ double inv_d;
  __shared__ float inv_f;
  const float* xr = x + (size_t)blockIdx.x * QWEN_HIDDEN;
  float* o = out + (size_t)blockIdx.x * QWEN_HIDDEN;
  if (threadIdx.x == 0) {
    if (prefill) {
      float ms = 0.0f;
      for (int d = 0; d < QWEN_HIDDEN; ++d) ms += xr[d] * xr[d];
      ms /= (float)QWEN_HIDDEN;
      inv_f = 1.0f / sqrtf(ms + eps);
    } else {
      double ms = 0.0;
      for (int d = 0; d < QWEN_HIDDEN; ++d) ms += (double)xr[d] * (double)xr[d];
      ms /= (double)QWEN_HIDDEN;
      inv_d = 1.0 / sqrt(ms + (double)eps);
    }
  }
  __syncthreads();
  for (int d = threadIdx.x; d < QWEN_HIDDEN; d += blockDim.x) {
    if (prefill) {
      const float nb = round_bf16(xr[d] * inv_f);
      o[d] = round_bf16(nb * w[d]);
    } else {
      o[d] = round_bf16((float)((double)xr[d] * inv_d * (double)w[d]));
    }
  }
}

// out[t][r] = bf16(fp32(bias[r] + sum_i in[t][i] * W[r][i])), the sum in double in i order.
// Thread = (row r, tile of kL0TokTile tokens).  grid = (ceil(out/128), ceil(T/8)), block = 128.
__global__ void l0_linear_kernel(const float* __restrict__ in, int in_dim, const float* __restrict__ W,
                                 const float* __restrict__ bias, int out_dim, int T, float* __restrict__ out) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= out_dim) return;
  const int t0 = blockIdx.y * kL0TokTile;
  const int nt = min(kL0TokTile, T - t0);
  const float* wr = W + (size_t)r * in_dim;
  const double b = bias ? (double)bias[r] : 0.0;
  double sum[kL0TokTile];
#pragma unroll
  for (int k = 0; k < kL0TokTile; ++k) sum[k] = b;
  const float* x0 = in + (size_t)t0 * in_dim;
  for (int i = 0; i < in_dim; ++i) {
    const double wv = (double)wr[i];
#pragma unroll
    for (int k = 0; k < kL0TokTile; ++k)
      if (k < nt) sum[k] += (double)x0[(size_t)k * in_dim + i] * wv;
  }
#pragma unroll
  for (int k = 0; k < kL0TokTile; ++k)
    if (k < nt) out[(size_t)(t0 + k) * out_dim + r] = round_bf16((float)sum[k]);
}

// RoPE of the 12 q heads and 2 k heads of token t with tab[t] = [cos 64 | sin 64].
// grid = tokens, block = 64 (one rotation pair per thread).
__global__ void l0_rope_kernel(float* __restrict__ q, float* __restrict__ k, const float* __restrict__ tab,
                               int prefill) {
  const int t = blockIdx.x;
  const int p = threadIdx.x;
  const float c = tab[(size_t)t * 128 + p];
  const float s = tab[(size_t)t * 128 + 64 + p];
  for (int h = 0; h < QWEN_Q_HEADS + QWEN_KV_HEADS; ++h) {
    float* hp = h < QWEN_Q_HEADS ? q + (size_t)t * QWEN_HIDDEN + h * QWEN_HEAD_DIM
                                 : k + (size_t)t * QWEN_KV_WIDTH + (h - QWEN_Q_HEADS) * QWEN_HEAD_DIM;
    const float e = hp[p], od = hp[p + 64];
    if (prefill) {
      const float ec = round_bf16(e * c), os = round_bf16(od * s);
      const float oc = round_bf16(od * c), es = round_bf16(e * s);
      hp[p] = round_bf16(ec - os);
      hp[p + 64] = round_bf16(oc + es);
    } else {
      hp[p] = e * c - od * s;
      hp[p + 64] = od * c + e * s;
    }
  }
}

// Head-major caches [kv_head][rows][128] for rows [row0, row0 + T) from token-major k/v [T][256]
// (rounded to bf16 when `round`), and rows [0, row0) copied from head-major past caches
// [kv_head][row0][128] when given.  grid = (row0 + T, 2), block = 128.
__global__ void l0_kv_store_kernel(const float* __restrict__ k, const float* __restrict__ v,
                                   const float* __restrict__ past_k, const float* __restrict__ past_v, int row0, int T,
                                   int round, float* __restrict__ k_out, float* __restrict__ v_out) {
  const int row = blockIdx.x;
  const int kvh = blockIdx.y;
  const int d = threadIdx.x;
  const size_t dst = ((size_t)kvh * (row0 + T) + row) * QWEN_HEAD_DIM + d;
  if (row < row0) {
    const size_t src = ((size_t)kvh * row0 + row) * QWEN_HEAD_DIM + d;
    k_out[dst] = past_k[src];
    v_out[dst] = past_v[src];
  } else {
    const size_t src = (size_t)(row - row0) * QWEN_KV_WIDTH + kvh * QWEN_HEAD_DIM + d;
    k_out[dst] = round ? round_bf16(k[src]) : k[src];
    v_out[dst] = round ? round_bf16(v[src]) : v[src];
  }
}

// Attention of query token t (rows tq0 + t of q) and head h over keys 0 .. n0 + tq0 + t - 1:
// scores = (sum_d q*k in double) * scaling, probs = exp(score - max) in double, sum_exp serial in
// key order, ctx[d] = fp32(sum_src (probs/sum_exp) * v) in key order.  Keys at
// kv + kvh*head_stride + src*key_stride.  probs: [tokens of this launch][12][nmax] doubles.
// grid = (12, tokens of this launch), block = 128.
__global__ void l0_attention_kernel(const float* __restrict__ q, int tq0, const float* __restrict__ k_src,
                                    const float* __restrict__ v_src, size_t key_stride, size_t head_stride, int n0,
                                    int nmax, double* __restrict__ probs, float* __restrict__ ctx) {
  __shared__ float qs[QWEN_HEAD_DIM];
  __shared__ double red[128];
  __shared__ double sum_s;
  const int h = blockIdx.x;
  const int tl = blockIdx.y;
  const int t = tq0 + tl;
  const int kvh = h / QWEN_GROUPS;
  const int n = n0 + t;
  const int tid = threadIdx.x;
  const float scaling = (float)(1.0 / sqrt((double)QWEN_HEAD_DIM));
  const float* kb = k_src + (size_t)kvh * head_stride;
  const float* vb = v_src + (size_t)kvh * head_stride;
  double* pr = probs + ((size_t)tl * QWEN_Q_HEADS + h) * nmax;
  qs[tid] = q[(size_t)t * QWEN_HIDDEN + h * QWEN_HEAD_DIM + tid];
  __syncthreads();
  double m = -1.0e300;
  for (int src = tid; src < n; src += 128) {
    const float* kr = kb + (size_t)src * key_stride;
    double dot = 0.0;
    for (int d = 0; d < QWEN_HEAD_DIM; ++d) dot += (double)qs[d] * (double)kr[d];
    const double sc = dot * (double)scaling;
    pr[src] = sc;
    m = sc > m ? sc : m;
  }
  red[tid] = m;
  __syncthreads();
  for (int s = 64; s > 0; s >>= 1) {
    if (tid < s) red[tid] = red[tid + s] > red[tid] ? red[tid + s] : red[tid];
    __syncthreads();
  }
  m = red[0];
  for (int src = tid; src < n; src += 128) pr[src] = exp(pr[src] - m);
  __syncthreads();
  if (tid == 0) {
    double s = 0.0;
    for (int src = 0; src < n; ++src) s += pr[src];
    sum_s = s;
  }
  __syncthreads();
  const double sum_exp = sum_s;
  for (int src = tid; src < n; src += 128) pr[src] = pr[src] / sum_exp;
  __syncthreads();
  double acc = 0.0;
  for (int src = 0; src < n; ++src) acc += pr[src] * (double)vb[(size_t)src * key_stride + tid];
  ctx[(size_t)t * QWEN_HIDDEN + h * QWEN_HEAD_DIM + tid] = (float)acc;
}

__global__ void l0_add_kernel(const float* __restrict__ a, const float* __restrict__ b, size_t n,
                              float* __restrict__ out) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = a[i] + b[i];
}

// s = silu(g) * u with silu(v) = v / (1 + expf(-v)) (host-compatible expf).
__global__ void l0_silu_mul_kernel(const float* __restrict__ g, const float* __restrict__ u, size_t n,
                                   float* __restrict__ s) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    const float v = g[i];
    s[i] = v / (1.0f + glibc_expf(-v)) * u[i];
  }
}

void linear(const float* in, int in_dim, const float* W, const float* b, int out_dim, int T, float* out,
            hipStream_t st) {
  hipLaunchKernelGGL(l0_linear_kernel, dim3((out_dim + 127) / 128, (T + kL0TokTile - 1) / kL0TokTile), dim3(128), 0,
                     st, in, in_dim, W, b, out_dim, T, out);
}

void add(const float* a, const float* b, size_t n, float* out, hipStream_t st) {
  hipLaunchKernelGGL(l0_add_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a, b, n, out);
}

}  // namespace

size_t layer0_workspace_bytes(int T, int past, bool decode) {
  const size_t t = (size_t)T;
  const size_t floats = t * (5 * QWEN_HIDDEN + 2 * QWEN_KV_WIDTH + 3 * QWEN_INTERMEDIATE) + 16 * 16;  // 10 takes
  const int nmax = decode ? past + 1 : T;
  const size_t probs = (size_t)layer0_attention_chunk(T, nmax) * QWEN_Q_HEADS * nmax * sizeof(double);
  return floats * sizeof(float) + probs + 1024;
}

int layer0_attention_chunk(int T, int nmax) {
  const size_t per_token = (size_t)QWEN_Q_HEADS * (size_t)(nmax > 0 ? nmax : 1) * sizeof(double);
  const size_t budget = (size_t)64 << 20;  // attention probabilities held at once
  size_t c = budget / per_token;
  if (c < 1) c = 1;
  return (int)(c < (size_t)T ? c : (size_t)T);
}

void run_layer0_reference(const Layer0Weights& W, float eps, bool decode, const float* x, int T, int past,
                          const float* rope_tab, const float* past_k, const float* past_v, float* out, float* k_out,
                          float* v_out, void* workspace, hipStream_t st) {
  float* f = static_cast<float*>(workspace);
  auto take = [&](size_t n) {
    float* p = f;
    f += (n + 15) & ~size_t(15);
    return p;
  };
  const size_t th = (size_t)T * QWEN_HIDDEN, tk = (size_t)T * QWEN_KV_WIDTH, ti = (size_t)T * QWEN_INTERMEDIATE;
  float* xn = take(th);
  float* q = take(th);
  float* k = take(tk);
  float* v = take(tk);
  float* ctx = take(th);
  float* o = take(th);
  float* res = take(th);
  float* g = take(ti);
  float* u = take(ti);
  float* s = take(ti);
  float* dn = xn;  // the input norm is dead once q/k/v exist
  float* pn = q;   // so is q once the context exists
  double* probs = reinterpret_cast<double*>(f);

  hipLaunchKernelGGL(l0_rmsnorm_kernel, dim3(T), dim3(64), 0, st, x, W.ln, eps, decode ? 0 : 1, xn);
  linear(xn, QWEN_HIDDEN, W.qw, W.qb, QWEN_HIDDEN, T, q, st);
  linear(xn, QWEN_HIDDEN, W.kw, W.kb, QWEN_KV_WIDTH, T, k, st);
  linear(xn, QWEN_HIDDEN, W.vw, W.vb, QWEN_KV_WIDTH, T, v, st);
  hipLaunchKernelGGL(l0_rope_kernel, dim3(T), dim3(64), 0, st, q, k, rope_tab, decode ? 0 : 1);
  if (decode) {
    // next caches: past rows, then the new row; attention over them (qwen_decode_layer0_reference_wrapper.cpp:136-188)
    hipLaunchKernelGGL(l0_kv_store_kernel, dim3(past + 1, QWEN_KV_HEADS), dim3(128), 0, st, k, v, past_k, past_v, past,
                       1, 0, k_out, v_out);
    hipLaunchKernelGGL(l0_attention_kernel, dim3(QWEN_Q_HEADS, 1), dim3(128), 0, st, q, 0, k_out, v_out,
                       (size_t)QWEN_HEAD_DIM, (size_t)(past + 1) * QWEN_HEAD_DIM, past + 1, past + 1, probs, ctx);
  } else {
    if (k_out)
      hipLaunchKernelGGL(l0_kv_store_kernel, dim3(T, QWEN_KV_HEADS), dim3(128), 0, st, k, v, nullptr, nullptr, 0, T, 1,
                         k_out, v_out);
    const int chunk = layer0_attention_chunk(T, T);
    for (int t0 = 0; t0 < T; t0 += chunk) {
      const int nt = min(chunk, T - t0);
      hipLaunchKernelGGL(l0_attention_kernel, dim3(QWEN_Q_HEADS, nt), dim3(128), 0, st, q, t0, k, v,
                         (size_t)QWEN_KV_WIDTH, (size_t)QWEN_HEAD_DIM, 1, T, probs, ctx);
    }
  }
  linear(ctx, QWEN_HIDDEN, W.ow, W.ob, QWEN_HIDDEN, T, o, st);
  add(x, o, th, res, st);
  hipLaunchKernelGGL(l0_rmsnorm_kernel, dim3(T), dim3(64), 0, st, res, W.post_ln, eps, decode ? 0 : 1, pn);
  linear(pn, QWEN_HIDDEN, W.gw, W.gb, QWEN_INTERMEDIATE, T, g, st);
  linear(pn, QWEN_HIDDEN, W.uw, W.ub, QWEN_INTERMEDIATE, T, u, st);
  hipLaunchKernelGGL(l0_silu_mul_kernel, dim3((unsigned)((ti + 255) / 256)), dim3(256), 0, st, g, u, ti, s);
  linear(s, QWEN_INTERMEDIATE, W.dw, W.db, QWEN_HIDDEN, T, dn, st);
  add(res, dn, th, out, st);
}

}  // namespace qwen
