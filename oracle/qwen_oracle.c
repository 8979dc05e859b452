/*
 * CPU oracle: a C11 restatement of the reference host arithmetic for the quantized
 * Qwen2.5-1.5B decoder layer.  TEST INFRASTRUCTURE ONLY (see qwen_oracle.h for who may call it
 * and how each function is pinned).  Build: gcc -std=c11 -O2 -ffp-contract=off -fPIC -shared.
 *
 * Every function cites the reference file:line it restates.  Tile parameters of the reference
 * only reorder loops that keep the serial accumulation order, so the oracle evaluates each
 * output with one plain serial loop and uses the tile values only for validation.
 */
#include "qwen_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define H QWEN_HIDDEN
#define I QWEN_INTERMEDIATE
#define KVW QWEN_KV_WIDTH
#define HD QWEN_HEAD_DIM

/* Float literals of the prefill kernel (qwen_prefill_attention_kernel.cpp:25-29). */
static const float kPi = 3.14159265358979323846f;
static const float kTwoPi = 6.28318530717958647692f;
static const float kHalfPi = 1.57079632679489661923f;
static const float kAttentionScalingPrefill = 0.08838834764831845f;
static const float kRopeFreqStep = 0.8058421877614801f;

/* ------------------------------------------------------------------------------------------ */
/* elementwise helpers                                                                         */
/* ------------------------------------------------------------------------------------------ */

/* approx_sqrt: qwen_prefill_attention_kernel.cpp:47-57 (= qwen_prefill_mlp_kernel.cpp:146-156). */
float oracle_approx_sqrt(float v) {
  if (v <= 0.0f) return 0.0f;
  float g = v > 1.0f ? v : 1.0f;
  for (int it = 0; it < 6; ++it) g = 0.5f * (g + v / g);
  return g;
}

/* wrap_angle: qwen_prefill_attention_kernel.cpp:59-67. */
float oracle_wrap_angle(float a) {
  while (a > kPi) a -= kTwoPi;
  while (a < -kPi) a += kTwoPi;
  return a;
}

/* approx_sincos: qwen_prefill_attention_kernel.cpp:69-85. */
void oracle_approx_sincos(float a, float* s, float* c) {
  float r = oracle_wrap_angle(a);
  float cs = 1.0f;
  if (r > kHalfPi) {
    r = kPi - r;
    cs = -1.0f;
  } else if (r < -kHalfPi) {
    r = -kPi - r;
    cs = -1.0f;
  }
  const float x2 = r * r;
  const float sp = r * (1.0f + x2 * (-1.0f / 6.0f + x2 * (1.0f / 120.0f + x2 * (-1.0f / 5040.0f))));
  const float cp = 1.0f + x2 * (-0.5f + x2 * (1.0f / 24.0f + x2 * (-1.0f / 720.0f)));
  *s = sp;
  *c = cs * cp;
}

/* approx_exp: qwen_prefill_attention_kernel.cpp:87-110 (= qwen_prefill_mlp_kernel.cpp:158-181).
 * Note `term *= s / deg` divides first, then multiplies. */
float oracle_approx_exp(float v) {
  if (v <= -16.0f) return 0.0f;
  int halves = 0;
  float s = v;
  while (s < -1.0f) {
    s *= 0.5f;
    ++halves;
  }
  float term = 1.0f, series = 1.0f;
  for (int deg = 1; deg <= 6; ++deg) {
    term *= s / (float)deg;
    series += term;
  }
  for (int k = 0; k < halves; ++k) series *= series;
  return series > 0.0f ? series : 0.0f;
}

float oracle_libm_expf(float v) { return expf(v); }

/* decode silu: qwen_decode_mlp_kernel.cpp:79-81 (std::exp(float) -> expf). */
float oracle_silu_decode(float v) { return v / (1.0f + expf(-v)); }

/* prefill silu: qwen_prefill_mlp_kernel.cpp:256-258. */
float oracle_silu_prefill(float v) { return v / (1.0f + oracle_approx_exp(-v)); }

/* round_bfloat16_array: verification/reference_wrapper_backend.py:40-46 (uint32 wrap-around). */
void oracle_round_bf16(float* x, size_t n) {
  for (size_t k = 0; k < n; ++k) {
    uint32_t b;
    memcpy(&b, &x[k], 4);
    b += 0x7FFFu + ((b >> 16) & 1u);
    b &= 0xFFFF0000u;
    memcpy(&x[k], &b, 4);
  }
}

/* quantize_int4_per_channel: verification/real_host_top_backend.py:31-41.
 * numpy semantics: fp32 absmax, fp32 max_abs/7.0, fp32 divide, rint (half to even), clip. */
void oracle_quantize_int4(const float* w, int out_dim, int in_dim, uint8_t* packed, float* scales) {
  const size_t total = (size_t)out_dim * (size_t)in_dim;
  memset(packed, 0, (total + 1) / 2);
  for (int o = 0; o < out_dim; ++o) {
    const float* row = w + (size_t)o * in_dim;
    float m = 0.0f;
    for (int i = 0; i < in_dim; ++i) {
      const float a = fabsf(row[i]);
      if (a > m) m = a;
    }
    const float s = m > 0.0f ? m / 7.0f : 1.0f;
    scales[o] = s;
    for (int i = 0; i < in_dim; ++i) {
      float q = rintf(row[i] / s);
      int qi = (int)q;
      if (qi < -8) qi = -8;
      if (qi > 7) qi = 7;
      const uint8_t nib = (uint8_t)(qi < 0 ? qi + 16 : qi);
      const size_t flat = (size_t)o * in_dim + i;
      if (flat & 1u)
        packed[flat / 2] |= (uint8_t)(nib << 4);
      else
        packed[flat / 2] |= nib;
    }
  }
}

/* apply_rope_inplace tables, decode: qwen_decode_attention_kernel.cpp:29-42 (libm double). */
void oracle_decode_rope_row(int position, float* cos_out, float* sin_out) {
  for (int p = 0; p < HD / 2; ++p) {
    const double angle = (double)position * pow((double)QWEN_ROPE_THETA, -2.0 * (double)p / (double)HD);
    cos_out[p] = (float)cos(angle);
    sin_out[p] = (float)sin(angle);
  }
}

/* apply_rope_inplace tables, prefill: qwen_prefill_attention_kernel.cpp:128-143. */
void oracle_prefill_rope_row(int position, float* cos_out, float* sin_out) {
  float inv_freq = 1.0f;
  for (int p = 0; p < HD / 2; ++p) {
    const float angle = (float)position * inv_freq;
    oracle_approx_sincos(angle, &sin_out[p], &cos_out[p]);
    inv_freq *= kRopeFreqStep;
  }
}

void oracle_layer_offsets(uint64_t o[20]) {
  const uint64_t v[20] = {QWEN_OFF_INPUT_LN, QWEN_OFF_Q_W, QWEN_OFF_K_W, QWEN_OFF_V_W, QWEN_OFF_O_W,
                          QWEN_OFF_POST_LN, QWEN_OFF_GATE_W, QWEN_OFF_UP_W, QWEN_OFF_DOWN_W, QWEN_OFF_Q_B,
                          QWEN_OFF_K_B, QWEN_OFF_V_B, QWEN_OFF_Q_S, QWEN_OFF_K_S, QWEN_OFF_V_S,
                          QWEN_OFF_O_S, QWEN_OFF_GATE_S, QWEN_OFF_UP_S, QWEN_OFF_DOWN_S, QWEN_LAYER_BYTES};
  memcpy(o, v, sizeof(v));
}

/* ------------------------------------------------------------------------------------------ */
/* shared building blocks                                                                      */
/* ------------------------------------------------------------------------------------------ */

/* decode_int4_weight + dequantized_weight: qwen_decode_attention_kernel.cpp:44-60 (the same code
 * is repeated at qwen_decode_mlp_kernel.cpp:10-26, qwen_prefill_attention_kernel.cpp:145-161 and
 * qwen_prefill_mlp_kernel.cpp:183-199).  Row o of an [out][in] matrix, flat index o*in+i, even
 * flat index in the low nibble, nibble >= 8 means nibble-16, times scale[o]. */
static void dequant_row(const uint8_t* packed, const float* scales, int o, int in_dim, float* w) {
  const float s = scales[o];
  for (int i = 0; i < in_dim; ++i) {
    const size_t flat = (size_t)o * (size_t)in_dim + (size_t)i;
    const uint8_t b = packed[flat / 2];
    const int nib = (flat & 1u) ? ((b >> 4) & 0xF) : (b & 0xF);
    const int sv = nib >= 8 ? nib - 16 : nib;
    w[i] = (float)sv * s;
  }
}

/* project_tiled: qwen_decode_attention_kernel.cpp:62-98 / qwen_decode_mlp_kernel.cpp:44-77 /
 * project_tiled_token qwen_prefill_attention_kernel.cpp:163-202 / qwen_prefill_mlp_kernel.cpp:217-254.
 * Per output row: acc = bias (or 0), then acc = acc + x[i]*w(o,i) for i = 0..in-1 in order (the
 * 128/64/256/640-wide tiles only split this loop, the carried partial sum keeps it serial).
 * Applied to `tokens` input vectors at once; each token keeps its own serial chain, so the
 * interleaving does not change any result. */
static void project_serial(const float* x, int tokens, size_t x_stride, const uint8_t* packed, const float* bias,
                           const float* scales, int out_dim, int in_dim, float* y, size_t y_stride) {
  float* w = (float*)malloc(sizeof(float) * (size_t)in_dim);
  for (int o = 0; o < out_dim; ++o) {
    dequant_row(packed, scales, o, in_dim, w);
    const float b0 = bias ? bias[o] : 0.0f;
    int t = 0;
    for (; t + 4 <= tokens; t += 4) {
      const float* x0 = x + (size_t)t * x_stride;
      const float* x1 = x0 + x_stride;
      const float* x2 = x1 + x_stride;
      const float* x3 = x2 + x_stride;
      float a0 = b0, a1 = b0, a2 = b0, a3 = b0;
      for (int i = 0; i < in_dim; ++i) {
        a0 = a0 + x0[i] * w[i];
        a1 = a1 + x1[i] * w[i];
        a2 = a2 + x2[i] * w[i];
        a3 = a3 + x3[i] * w[i];
      }
      y[(size_t)t * y_stride + o] = a0;
      y[(size_t)(t + 1) * y_stride + o] = a1;
      y[(size_t)(t + 2) * y_stride + o] = a2;
      y[(size_t)(t + 3) * y_stride + o] = a3;
    }
    for (; t < tokens; ++t) {
      const float* xt = x + (size_t)t * x_stride;
      float a = b0;
      for (int i = 0; i < in_dim; ++i) a = a + xt[i] * w[i];
      y[(size_t)t * y_stride + o] = a;
    }
  }
  free(w);
}

/* rmsnorm_token, decode: qwen_decode_attention_kernel.cpp:13-27 (= qwen_decode_mlp_kernel.cpp:28-42). */
static void rmsnorm_decode(const float* x, const float* w, float eps, float* out) {
  double ms = 0.0;
  for (int d = 0; d < H; ++d) ms += (double)x[d] * (double)x[d];
  ms /= (double)H;
  const double inv = 1.0 / sqrt(ms + (double)eps);
  for (int d = 0; d < H; ++d) out[d] = (float)((double)x[d] * inv * (double)w[d]);
}

/* rmsnorm_token, prefill: qwen_prefill_attention_kernel.cpp:112-126 (= qwen_prefill_mlp_kernel.cpp:201-215). */
static void rmsnorm_prefill(const float* x, const float* w, float eps, float* out) {
  float ms = 0.0f;
  for (int d = 0; d < H; ++d) ms += x[d] * x[d];
  ms /= (float)H;
  const float inv = 1.0f / oracle_approx_sqrt(ms + eps);
  for (int d = 0; d < H; ++d) out[d] = x[d] * inv * w[d];
}

/* Rotation of pairs (p, p+64): qwen_decode_attention_kernel.cpp:35-40 / prefill :135-140. */
static void rotate_head(float* head, const float* c, const float* s) {
  for (int p = 0; p < HD / 2; ++p) {
    const float e = head[p];
    const float o = head[p + HD / 2];
    head[p] = e * c[p] - o * s[p];
    head[p + HD / 2] = o * c[p] + e * s[p];
  }
}

/* Two-pass softmax attention of one query head over keys 0..n-1 (decode
 * decode_attention_context :113-162 with expf; prefill prefill_attention_context_block :204-289
 * with approx_exp, keys 0..q).  The dot product is recomputed in the second pass like the
 * reference; max uses the reference's "new > old" selection. */
static void attend_head(const float* q, const float* k_rows, const float* v_rows, int n, int kv_head, float scaling,
                        int use_approx_exp, float* ctx) {
  float m = -1.0e30f;
  for (int t = 0; t < n; ++t) {
    const float* k = k_rows + (size_t)t * KVW + kv_head * HD;
    float score = 0.0f;
    for (int d = 0; d < HD; ++d) score += q[d] * k[d];
    const float sc = score * scaling;
    m = sc > m ? sc : m;
  }
  float den = 0.0f;
  float acc[HD];
  for (int d = 0; d < HD; ++d) acc[d] = 0.0f;
  for (int t = 0; t < n; ++t) {
    const float* k = k_rows + (size_t)t * KVW + kv_head * HD;
    const float* v = v_rows + (size_t)t * KVW + kv_head * HD;
    float score = 0.0f;
    for (int d = 0; d < HD; ++d) score += q[d] * k[d];
    const float arg = score * scaling - m;
    const float e = use_approx_exp ? oracle_approx_exp(arg) : expf(arg);
    den += e;
    for (int d = 0; d < HD; ++d) acc[d] += e * v[d];
  }
  const float inv = den > 0.0f ? 1.0f / den : 0.0f;
  for (int d = 0; d < HD; ++d) ctx[d] = acc[d] * inv;
}

/* ------------------------------------------------------------------------------------------ */
/* decode                                                                                      */
/* ------------------------------------------------------------------------------------------ */

/* qwen_decode_attention_kernel: qwen_decode_attention_kernel.cpp:168-218. */
int oracle_decode_attention_smoke_forward(
    const float* x, int past, const float* ln, const uint8_t* qw, const uint8_t* kw, const uint8_t* vw,
    const uint8_t* ow, const float* qb, const float* kb, const float* vb, const float* qs, const float* ks,
    const float* vs, const float* os, float* k_cache, float* v_cache, float* out) {
  if (!x || !out || past < 0 || !ln || !qw || !kw || !vw || !ow || !qb || !kb || !vb || !qs || !ks || !vs || !os ||
      !k_cache || !v_cache)
    return QWEN_ERR_KERNEL;
  float xn[H], q[H], k[KVW], v[KVW], ctx[H], c[HD / 2], s[HD / 2];
  rmsnorm_decode(x, ln, QWEN_RMS_EPS, xn);
  project_serial(xn, 1, H, qw, qb, qs, H, H, q, H);
  project_serial(xn, 1, H, kw, kb, ks, KVW, H, k, KVW);
  project_serial(xn, 1, H, vw, vb, vs, KVW, H, v, KVW);
  oracle_decode_rope_row(past, c, s);
  for (int h = 0; h < QWEN_Q_HEADS; ++h) rotate_head(q + h * HD, c, s);
  for (int h = 0; h < QWEN_KV_HEADS; ++h) rotate_head(k + h * HD, c, s);
  /* append_kv_cache :100-111 */
  const size_t row = (size_t)past * KVW;
  for (int i = 0; i < KVW; ++i) {
    k_cache[row + i] = k[i];
    v_cache[row + i] = v[i];
  }
  /* (float)(1.0 / sqrt((double)128)) :119 */
  const float scaling = (float)(1.0 / sqrt((double)HD));
  for (int h = 0; h < QWEN_Q_HEADS; ++h)
    attend_head(q + h * HD, k_cache, v_cache, past + 1, h / QWEN_GROUPS, scaling, 0, ctx + h * HD);
  project_serial(ctx, 1, H, ow, NULL, os, H, H, out, H);
  return QWEN_OK;
}

/* qwen_decode_mlp_kernel: qwen_decode_mlp_kernel.cpp:87-122. */
int oracle_decode_mlp_smoke_forward(const float* a, const float* post_ln, const uint8_t* gw, const uint8_t* uw,
                                    const uint8_t* dw, const float* gs, const float* us, const float* ds,
                                    float* out) {
  if (!a || !out || !post_ln || !gw || !uw || !dw || !gs || !us || !ds) return QWEN_ERR_KERNEL;
  float pn[H], dn[H];
  float* g = (float*)malloc(sizeof(float) * I * 3);
  float* u = g + I;
  float* sm = u + I;
  rmsnorm_decode(a, post_ln, QWEN_RMS_EPS, pn);
  project_serial(pn, 1, H, gw, NULL, gs, I, H, g, I);
  project_serial(pn, 1, H, uw, NULL, us, I, H, u, I);
  for (int i = 0; i < I; ++i) sm[i] = oracle_silu_decode(g[i]) * u[i];
  project_serial(sm, 1, I, dw, NULL, ds, H, I, dn, H);
  for (int i = 0; i < H; ++i) out[i] = a[i] + dn[i];
  free(g);
  return QWEN_OK;
}

/* qwen_decode_layer_smoke_forward: qwen_decode_host_wrapper.cpp:157-218. */
int oracle_decode_layer_smoke_forward(
    const float* x, int past, const float* ln, const float* post_ln, const uint8_t* qw, const uint8_t* kw,
    const uint8_t* vw, const uint8_t* ow, const uint8_t* gw, const uint8_t* uw, const uint8_t* dw, const float* qb,
    const float* kb, const float* vb, const float* qs, const float* ks, const float* vs, const float* os,
    const float* gs, const float* us, const float* ds, float* k_cache, float* v_cache, float* out) {
  float att[H];
  memset(att, 0, sizeof(att));
  int st = oracle_decode_attention_smoke_forward(x, past, ln, qw, kw, vw, ow, qb, kb, vb, qs, ks, vs, os, k_cache,
                                                 v_cache, att);
  if (st) return st;
  return oracle_decode_mlp_smoke_forward(att, post_ln, gw, uw, dw, gs, us, ds, out);
}

/* qwen_decode_stub_forward: qwen_decode_host_wrapper.cpp:12-71.  Zero weights, unit scales and
 * unit norm weights.  (The reference passes its 1536-row Q/O buffers where the 8960-row gate/up
 * and down buffers belong; every value it could read there multiplies a zero activation, so the
 * oracle uses correctly sized zero buffers.) */
int oracle_decode_stub_forward(const float* x, int past, float* out) {
  if (!x || !out || past < 0) return QWEN_ERR_KERNEL;
  const size_t kv = (size_t)(past + 1) * KVW;
  float* kc = (float*)calloc(kv * 2, sizeof(float));
  uint8_t* zw = (uint8_t*)calloc((size_t)I * H / 2, 1);
  float* ones = (float*)malloc(sizeof(float) * I);
  float* zeros = (float*)calloc(I, sizeof(float));
  for (int i = 0; i < I; ++i) ones[i] = 1.0f;
  int st = oracle_decode_layer_smoke_forward(x, past, ones, ones, zw, zw, zw, zw, zw, zw, zw, zeros, zeros, zeros,
                                             ones, ones, ones, ones, ones, ones, ones, kc, kc + kv, out);
  free(kc);
  free(zw);
  free(ones);
  free(zeros);
  return st;
}

/* Resolve the 19 per-layer pointers from a descriptor: qwen_decode_top_wrapper.cpp:14-26,40-72
 * (weights: base + byte offset; fp32 ports: base + byte_offset / 4, integer division). */
typedef struct {
  const uint8_t *qw, *kw, *vw, *ow, *gw, *uw, *dw;
  const float *ln, *post_ln, *qb, *kb, *vb, *qs, *ks, *vs, *os, *gs, *us, *ds;
} layer_ptrs;

static layer_ptrs resolve_layer(const uint8_t* wd, const float* sd, uint64_t wb, uint64_t sb) {
  layer_ptrs p;
  p.ln = sd + (sb + QWEN_OFF_INPUT_LN) / 4;
  p.post_ln = sd + (sb + QWEN_OFF_POST_LN) / 4;
  p.qw = wd + wb + QWEN_OFF_Q_W;
  p.kw = wd + wb + QWEN_OFF_K_W;
  p.vw = wd + wb + QWEN_OFF_V_W;
  p.ow = wd + wb + QWEN_OFF_O_W;
  p.qb = sd + (sb + QWEN_OFF_Q_B) / 4;
  p.kb = sd + (sb + QWEN_OFF_K_B) / 4;
  p.vb = sd + (sb + QWEN_OFF_V_B) / 4;
  p.qs = sd + (sb + QWEN_OFF_Q_S) / 4;
  p.ks = sd + (sb + QWEN_OFF_K_S) / 4;
  p.vs = sd + (sb + QWEN_OFF_V_S) / 4;
  p.os = sd + (sb + QWEN_OFF_O_S) / 4;
  p.gs = sd + (sb + QWEN_OFF_GATE_S) / 4;
  p.us = sd + (sb + QWEN_OFF_UP_S) / 4;
  p.ds = sd + (sb + QWEN_OFF_DOWN_S) / 4;
  p.gw = wd + wb + QWEN_OFF_GATE_W;
  p.uw = wd + wb + QWEN_OFF_UP_W;
  p.dw = wd + wb + QWEN_OFF_DOWN_W;
  return p;
}

/* qwen_decode_top_wrapper: qwen_decode_top_wrapper.cpp:28-113 (via host wrapper :113-155). */
int oracle_decode_top_smoke_forward(int layer_id, int past, uint64_t in_addr, uint64_t out_addr, uint64_t wb,
                                    uint64_t sb, uint64_t kb_addr, uint64_t vb_addr, const uint8_t* wd,
                                    const float* sd, float* kv, float* act, uint8_t* wsram, float* kvsram,
                                    int32_t* psram, float* smsram, float* csram) {
  if (!qwen_valid_layer_id(layer_id) || past < 0) return QWEN_ERR_DECODE_DESC;
  if (!wd || !sd || !kv || !act || !wsram || !kvsram || !psram || !smsram || !csram) return QWEN_ERR_DECODE_PORT;
  const layer_ptrs p = resolve_layer(wd, sd, wb, sb);
  const float* x = act + in_addr / 4;
  float* out = act + out_addr / 4;
  float* kc = kv + kb_addr / 4;
  float* vc = kv + vb_addr / 4;
  float att[H];
  memset(att, 0, sizeof(att));
  int st = oracle_decode_attention_smoke_forward(x, past, p.ln, p.qw, p.kw, p.vw, p.ow, p.qb, p.kb, p.vb, p.qs, p.ks,
                                                 p.vs, p.os, kc, vc, att);
  if (st) return st;
  return oracle_decode_mlp_smoke_forward(att, p.post_ln, p.gw, p.uw, p.dw, p.gs, p.us, p.ds, out);
}

int oracle_decode_layer_block(const float* x, int past, const uint8_t* wd, const float* sd, float* kc, float* vc,
                              float* out) {
  const layer_ptrs p = resolve_layer(wd, sd, 0, 0);
  return oracle_decode_layer_smoke_forward(x, past, p.ln, p.post_ln, p.qw, p.kw, p.vw, p.ow, p.gw, p.uw, p.dw, p.qb,
                                           p.kb, p.vb, p.qs, p.ks, p.vs, p.os, p.gs, p.us, p.ds, kc, vc, out);
}

/* ------------------------------------------------------------------------------------------ */
/* prefill                                                                                     */
/* ------------------------------------------------------------------------------------------ */

/* Numerics of qwen_prefill_attention_kernel (qwen_prefill_attention_kernel.cpp:2270-2364) without
 * its validation: pass A per token rmsnorm -> K,V (+bias) -> RoPE(K) -> cache row; pass B per
 * query rmsnorm -> Q (+bias) -> RoPE(Q) -> causal context over keys 0..q -> O (no bias). */
static void prefill_attention_math(const float* x, int S, const float* ln, const uint8_t* qw, const uint8_t* kw,
                                   const uint8_t* vw, const uint8_t* ow, const float* qb, const float* kb,
                                   const float* vb, const float* qs, const float* ks, const float* vs,
                                   const float* os, float* kc, float* vc, float* out) {
  float* xn = (float*)malloc(sizeof(float) * (size_t)S * H);
  float* q = (float*)malloc(sizeof(float) * (size_t)S * H);
  float* ctx = (float*)malloc(sizeof(float) * (size_t)S * H);
  float c[HD / 2], s[HD / 2];
  for (int t = 0; t < S; ++t) rmsnorm_prefill(x + (size_t)t * H, ln, QWEN_RMS_EPS, xn + (size_t)t * H);
  project_serial(xn, S, H, kw, kb, ks, KVW, H, kc, KVW);
  project_serial(xn, S, H, vw, vb, vs, KVW, H, vc, KVW);
  project_serial(xn, S, H, qw, qb, qs, H, H, q, H);
  for (int t = 0; t < S; ++t) {
    oracle_prefill_rope_row(t, c, s);
    for (int h = 0; h < QWEN_KV_HEADS; ++h) rotate_head(kc + (size_t)t * KVW + h * HD, c, s);
    for (int h = 0; h < QWEN_Q_HEADS; ++h) rotate_head(q + (size_t)t * H + h * HD, c, s);
  }
  for (int t = 0; t < S; ++t)
    for (int h = 0; h < QWEN_Q_HEADS; ++h)
      attend_head(q + (size_t)t * H + h * HD, kc, vc, t + 1, h / QWEN_GROUPS, kAttentionScalingPrefill, 1,
                  ctx + (size_t)t * H + h * HD);
  project_serial(ctx, S, H, ow, NULL, os, H, H, out, H);
  free(xn);
  free(q);
  free(ctx);
}

/* Numerics of qwen_prefill_mlp_kernel (qwen_prefill_mlp_kernel.cpp:285-334). */
static void prefill_mlp_math(const float* a, int S, const float* post_ln, const uint8_t* gw, const uint8_t* uw,
                             const uint8_t* dw, const float* gs, const float* us, const float* ds, float* out) {
  float* pn = (float*)malloc(sizeof(float) * (size_t)S * H);
  float* g = (float*)malloc(sizeof(float) * (size_t)S * I);
  float* u = (float*)malloc(sizeof(float) * (size_t)S * I);
  float* dn = (float*)malloc(sizeof(float) * (size_t)S * H);
  for (int t = 0; t < S; ++t) rmsnorm_prefill(a + (size_t)t * H, post_ln, QWEN_RMS_EPS, pn + (size_t)t * H);
  project_serial(pn, S, H, gw, NULL, gs, I, H, g, I);
  project_serial(pn, S, H, uw, NULL, us, I, H, u, I);
  for (size_t k = 0; k < (size_t)S * I; ++k) g[k] = oracle_silu_prefill(g[k]) * u[k];
  project_serial(g, S, I, dw, NULL, ds, H, I, dn, H);
  for (size_t k = 0; k < (size_t)S * H; ++k) out[k] = a[k] + dn[k];
  free(pn);
  free(g);
  free(u);
  free(dn);
}

/* Validation of qwen_prefill_attention_kernel: qwen_prefill_attention_kernel.cpp:2252-2268. */
static int prefill_attention_check(const float* x, const float* out, int S, const qwen_prefill_attention_tiles* t,
                                   const void* const* ptrs, int nptrs) {
  if (!x || !out || S <= 0) return QWEN_ERR_KERNEL;
  for (int k = 0; k < nptrs; ++k)
    if (!ptrs[k]) return QWEN_ERR_KERNEL;
  if (t->seq <= 0 || t->query <= 0 || t->key <= 0 || t->hidden_proj <= 0 || t->kv_proj <= 0 || t->head_dim != HD ||
      t->query_heads_parallel <= 0 || t->kv_heads_parallel <= 0)
    return QWEN_ERR_KERNEL;
  if (S > QWEN_PREFILL_CAPACITY || t->seq > QWEN_PREFILL_CAPACITY || t->query > QWEN_PREFILL_QUERY_CAPACITY ||
      t->key > QWEN_PREFILL_KEY_CAPACITY || t->hidden_proj > QWEN_PREFILL_PROJ_CAPACITY ||
      t->kv_proj > QWEN_PREFILL_PROJ_CAPACITY || t->query_heads_parallel > QWEN_Q_HEADS ||
      t->kv_heads_parallel > QWEN_KV_HEADS)
    return QWEN_ERR_CAPACITY;
  return QWEN_OK;
}

/* Validation of qwen_prefill_mlp_kernel: qwen_prefill_mlp_kernel.cpp:277-283. */
static int prefill_mlp_check(const float* a, const float* out, int S, const qwen_prefill_mlp_tiles* t,
                             const void* const* ptrs, int nptrs) {
  if (!a || !out || S <= 0) return QWEN_ERR_KERNEL;
  for (int k = 0; k < nptrs; ++k)
    if (!ptrs[k]) return QWEN_ERR_KERNEL;
  if (t->seq <= 0 || t->hidden <= 0 || t->ff <= 0 || t->hidden > QWEN_PREFILL_MLP_HIDDEN_CAPACITY ||
      t->ff > QWEN_PREFILL_MLP_FF_CAPACITY)
    return QWEN_ERR_KERNEL;
  return QWEN_OK;
}

static qwen_prefill_attention_tiles make_atiles(int a_seq, int a_query, int a_key, int a_hp, int a_kvp, int a_hd,
                                                int a_qhp, int a_kvhp) {
  qwen_prefill_attention_tiles t = {a_seq, a_query, a_key, a_hp, a_kvp, a_hd, a_qhp, a_kvhp};
  return t;
}

/* qwen_prefill_attention_smoke_forward: qwen_prefill_host_wrapper.cpp:300-356. */
int oracle_prefill_attention_smoke_forward(const float* x, int S, int a_seq, int a_query, int a_key, int a_hp,
                                           int a_kvp, int a_hd, int a_qhp, int a_kvhp, const float* ln,
                                           const uint8_t* qw, const uint8_t* kw, const uint8_t* vw,
                                           const uint8_t* ow, const float* qb, const float* kb, const float* vb,
                                           const float* qs, const float* ks, const float* vs, const float* os,
                                           float* kc, float* vc, float* out) {
  const qwen_prefill_attention_tiles t = make_atiles(a_seq, a_query, a_key, a_hp, a_kvp, a_hd, a_qhp, a_kvhp);
  const void* ptrs[] = {ln, qw, kw, vw, ow, qb, kb, vb, qs, ks, vs, os, kc, vc};
  const int st = prefill_attention_check(x, out, S, &t, ptrs, 14);
  if (st) return st;
  prefill_attention_math(x, S, ln, qw, kw, vw, ow, qb, kb, vb, qs, ks, vs, os, kc, vc, out);
  return QWEN_OK;
}

/* qwen_prefill_mlp_smoke_forward: qwen_prefill_host_wrapper.cpp:358-387. */
int oracle_prefill_mlp_smoke_forward(const float* a, int S, int m_seq, int m_hidden, int m_ff, const float* post_ln,
                                     const uint8_t* gw, const uint8_t* uw, const uint8_t* dw, const float* gs,
                                     const float* us, const float* ds, float* out) {
  const qwen_prefill_mlp_tiles t = {m_seq, m_hidden, m_ff};
  const void* ptrs[] = {post_ln, gw, uw, dw, gs, us, ds};
  const int st = prefill_mlp_check(a, out, S, &t, ptrs, 7);
  if (st) return st;
  prefill_mlp_math(a, S, post_ln, gw, uw, dw, gs, us, ds, out);
  return QWEN_OK;
}

/* qwen_prefill_layer_smoke_forward: qwen_prefill_host_wrapper.cpp:389-476. */
int oracle_prefill_layer_smoke_forward(const float* x, int S, int a_seq, int a_query, int a_key, int a_hp, int a_kvp,
                                       int a_hd, int a_qhp, int a_kvhp, int m_seq, int m_hidden, int m_ff,
                                       const float* ln, const float* post_ln, const uint8_t* qw, const uint8_t* kw,
                                       const uint8_t* vw, const uint8_t* ow, const uint8_t* gw, const uint8_t* uw,
                                       const uint8_t* dw, const float* qb, const float* kb, const float* vb,
                                       const float* qs, const float* ks, const float* vs, const float* os,
                                       const float* gs, const float* us, const float* ds, float* kc, float* vc,
                                       float* out) {
  const size_t n = S > 0 ? (size_t)S * H : 1;
  float* att = (float*)calloc(n, sizeof(float));
  int st = oracle_prefill_attention_smoke_forward(x, S, a_seq, a_query, a_key, a_hp, a_kvp, a_hd, a_qhp, a_kvhp, ln,
                                                  qw, kw, vw, ow, qb, kb, vb, qs, ks, vs, os, kc, vc, att);
  if (!st) st = oracle_prefill_mlp_smoke_forward(att, S, m_seq, m_hidden, m_ff, post_ln, gw, uw, dw, gs, us, ds, out);
  free(att);
  return st;
}

/* qwen_prefill_glue_smoke_forward: qwen_prefill_host_wrapper.cpp:478-637.  On the host the glue
 * chain (qwen_prefill_glue_top_v1_catapult.cpp:6-70 -> host shims
 * qwen_prefill_host_catapult_shims.cpp:115-242) calls the same two kernels with the default tiles. */
int oracle_prefill_glue_smoke_forward(const float* x, int S, int a_seq, int a_query, int a_key, int a_hp, int a_kvp,
                                      int a_hd, int a_qhp, int a_kvhp, int m_seq, int m_hidden, int m_ff,
                                      const float* ln, const float* post_ln, const uint8_t* qw, const uint8_t* kw,
                                      const uint8_t* vw, const uint8_t* ow, const uint8_t* gw, const uint8_t* uw,
                                      const uint8_t* dw, const float* qb, const float* kb, const float* vb,
                                      const float* qs, const float* ks, const float* vs, const float* os,
                                      const float* gs, const float* us, const float* ds, float* kc, float* vc,
                                      float* out) {
  const void* ptrs[] = {x, ln, post_ln, qw, kw, vw, ow, gw, uw, dw, qb, kb, vb, qs, ks, vs, os, gs, us, ds, kc, vc, out};
  for (int k = 0; k < 23; ++k)
    if (!ptrs[k]) return QWEN_ERR_KERNEL;
  if (S <= 0) return QWEN_ERR_KERNEL;
  const qwen_prefill_tiles d = qwen_default_prefill_tiles();
  if (a_seq != d.attention.seq || a_query != d.attention.query || a_key != d.attention.key ||
      a_hp != d.attention.hidden_proj || a_kvp != d.attention.kv_proj || a_hd != HD ||
      a_qhp != d.attention.query_heads_parallel || a_kvhp != d.attention.kv_heads_parallel || m_seq != d.mlp.seq ||
      m_hidden != d.mlp.hidden || m_ff != d.mlp.ff)
    return QWEN_ERR_CAPACITY;
  /* valid_attention_stream_config (qwen_prefill_attention_stream_top.cpp:99-101). */
  if (S > QWEN_PREFILL_CAPACITY) return QWEN_ERR_CAPACITY;
  float* att = (float*)malloc(sizeof(float) * (size_t)S * H);
  prefill_attention_math(x, S, ln, qw, kw, vw, ow, qb, kb, vb, qs, ks, vs, os, kc, vc, att);
  prefill_mlp_math(att, S, post_ln, gw, uw, dw, gs, us, ds, out);
  free(att);
  return QWEN_OK;
}

/* qwen_prefill_stub_forward: qwen_prefill_host_wrapper.cpp:205-298. */
int oracle_prefill_stub_forward(const float* x, int S, int a_seq, int a_query, int a_key, int a_hp, int a_kvp,
                                int a_hd, int a_qhp, int a_kvhp, int m_seq, int m_hidden, int m_ff, float* out) {
  if (!x || !out || S <= 0) return QWEN_ERR_KERNEL;
  const size_t kv = (size_t)S * KVW;
  float* kc = (float*)calloc(kv * 2, sizeof(float));
  float* att = (float*)calloc((size_t)S * H, sizeof(float));
  uint8_t* zw = (uint8_t*)calloc((size_t)I * H / 2, 1);
  float* ones = (float*)malloc(sizeof(float) * I);
  float* zeros = (float*)calloc(I, sizeof(float));
  for (int i = 0; i < I; ++i) ones[i] = 1.0f;
  int st = oracle_prefill_attention_smoke_forward(x, S, a_seq, a_query, a_key, a_hp, a_kvp, a_hd, a_qhp, a_kvhp, ones,
                                                  zw, zw, zw, zw, zeros, zeros, zeros, ones, ones, ones, ones, kc,
                                                  kc + kv, att);
  if (!st) st = oracle_prefill_mlp_smoke_forward(att, S, m_seq, m_hidden, m_ff, ones, zw, zw, zw, ones, ones, ones, out);
  free(kc);
  free(att);
  free(zw);
  free(ones);
  free(zeros);
  return st;
}

/* valid_memory_windows: qwen_prefill_top_core.cpp:42-80. */
static int range_fits(uint64_t off, uint64_t count, uint64_t cap) { return off <= cap && count <= cap - off; }
static int ranges_overlap(uint64_t a, uint64_t as, uint64_t b, uint64_t bs) { return a < b + bs && b < a + as; }

static int prefill_windows_ok(const qwen_prefill_descriptor* d) {
  if (d->seq_len <= 0 || d->seq_len > QWEN_PREFILL_CAPACITY) return 0;
  const uint64_t seq_bytes = (uint64_t)d->seq_len * H * 4u;
  const uint64_t kv_bytes = (uint64_t)d->seq_len * KVW * 4u;
  const uint64_t packed = QWEN_OFF_DOWN_W + QWEN_DOWN_WEIGHT_BYTES - QWEN_OFF_Q_W;
  const uint64_t scale_bytes = QWEN_OFF_DOWN_S + 4ull * H;
  if (d->input_sequence_addr % 4 || d->output_sequence_addr % 4 || d->k_cache_base_addr % 4 ||
      d->v_cache_base_addr % 4 || d->scratch_base_addr % 4 || d->layer_scales_base_addr % 4)
    return 0;
  if (!range_fits(d->input_sequence_addr, seq_bytes, QWEN_PREFILL_ACT_WINDOW_BYTES) ||
      !range_fits(d->output_sequence_addr, seq_bytes, QWEN_PREFILL_ACT_WINDOW_BYTES) ||
      !range_fits(d->scratch_base_addr, seq_bytes, QWEN_PREFILL_ACT_WINDOW_BYTES) ||
      !range_fits(d->k_cache_base_addr, kv_bytes, QWEN_PREFILL_KV_WINDOW_BYTES) ||
      !range_fits(d->v_cache_base_addr, kv_bytes, QWEN_PREFILL_KV_WINDOW_BYTES) ||
      !range_fits(d->layer_weights_base_addr + QWEN_OFF_Q_W, packed, QWEN_PREFILL_WEIGHT_WINDOW) ||
      !range_fits(d->layer_scales_base_addr, scale_bytes, QWEN_PREFILL_SCALE_WINDOW_BYTES))
    return 0;
  if (ranges_overlap(d->input_sequence_addr, seq_bytes, d->output_sequence_addr, seq_bytes) ||
      ranges_overlap(d->input_sequence_addr, seq_bytes, d->scratch_base_addr, seq_bytes) ||
      ranges_overlap(d->output_sequence_addr, seq_bytes, d->scratch_base_addr, seq_bytes) ||
      ranges_overlap(d->k_cache_base_addr, kv_bytes, d->v_cache_base_addr, kv_bytes))
    return 0;
  return 1;
}

/* qwen_prefill_top_smoke_forward: qwen_prefill_host_wrapper.cpp:639-705 -> qwen_prefill_top_wrapper
 * (qwen_prefill_top_wrapper.cpp:7-18) -> qwen_prefill_top_core (qwen_prefill_top_core.cpp:84-183). */
int oracle_prefill_top_smoke_forward(int layer_id, int S, int a_seq, int a_query, int a_key, int a_hp, int a_kvp,
                                     int a_hd, int a_qhp, int a_kvhp, int m_seq, int m_hidden, int m_ff,
                                     uint64_t in_addr, uint64_t out_addr, uint64_t wb, uint64_t sb, uint64_t kb_addr,
                                     uint64_t vb_addr, const uint8_t* wd, const float* sd, float* kv, float* act,
                                     uint8_t* wsram, float* kvsram, int32_t* psram, float* smsram, float* csram) {
  qwen_prefill_descriptor d;
  d.layer_id = layer_id;
  d.seq_len = S;
  d.tiles.attention = make_atiles(a_seq, a_query, a_key, a_hp, a_kvp, a_hd, a_qhp, a_kvhp);
  d.tiles.mlp.seq = m_seq;
  d.tiles.mlp.hidden = m_hidden;
  d.tiles.mlp.ff = m_ff;
  d.input_sequence_addr = in_addr;
  d.output_sequence_addr = out_addr;
  d.layer_weights_base_addr = wb;
  d.layer_scales_base_addr = sb;
  d.k_cache_base_addr = kb_addr;
  d.v_cache_base_addr = vb_addr;
  d.scratch_base_addr = out_addr + (uint64_t)(int64_t)S * H * 4u; /* host wrapper :668,:690 */
  /* top wrapper */
  if (S <= 0 || S > QWEN_MAX_SEQ) return QWEN_ERR_PREFILL_DESC;
  if (S > QWEN_PREFILL_CAPACITY) return QWEN_ERR_PREFILL_DESC;
  /* top core */
  if (!qwen_valid_layer_id(layer_id) || S <= 0 || !qwen_valid_prefill_tiles(&d.tiles)) return QWEN_ERR_PREFILL_DESC;
  if (!wd || !sd || !kv || !act || !wsram || !kvsram || !psram || !smsram || !csram) return QWEN_ERR_PREFILL_PORT;
  if (!prefill_windows_ok(&d)) return QWEN_ERR_PREFILL_WINDOW;
  const layer_ptrs p = resolve_layer(wd, sd, wb, sb);
  const float* x = act + in_addr / 4;
  float* out = act + out_addr / 4;
  float* scratch = act + d.scratch_base_addr / 4;
  float* kc = kv + kb_addr / 4;
  float* vc = kv + vb_addr / 4;
  int st = oracle_prefill_attention_smoke_forward(x, S, a_seq, a_query, a_key, a_hp, a_kvp, a_hd, a_qhp, a_kvhp, p.ln,
                                                  p.qw, p.kw, p.vw, p.ow, p.qb, p.kb, p.vb, p.qs, p.ks, p.vs, p.os,
                                                  kc, vc, scratch);
  if (st) return st;
  return oracle_prefill_mlp_smoke_forward(scratch, S, m_seq, m_hidden, m_ff, p.post_ln, p.gw, p.uw, p.dw, p.gs, p.us,
                                          p.ds, out);
}

int oracle_prefill_layer_uncapped(const float* x, int S, const uint8_t* wd, const float* sd, float* kc, float* vc,
                                  float* out) {
  if (!x || !wd || !sd || !kc || !vc || !out || S <= 0 || S > QWEN_MAX_SEQ) return QWEN_ERR_KERNEL;
  const layer_ptrs p = resolve_layer(wd, sd, 0, 0);
  float* att = (float*)malloc(sizeof(float) * (size_t)S * H);
  prefill_attention_math(x, S, p.ln, p.qw, p.kw, p.vw, p.ow, p.qb, p.kb, p.vb, p.qs, p.ks, p.vs, p.os, kc, vc, att);
  prefill_mlp_math(att, S, p.post_ln, p.gw, p.uw, p.dw, p.gs, p.us, p.ds, out);
  free(att);
  return QWEN_OK;
}

/* Compares y[i] with the host expf of the float whose bit pattern is first + i*stride (mod 2^32);
 * NaN results compare equal to NaN.  Returns the number of mismatches; *first_bad receives the
 * first mismatching bit pattern (test infrastructure for the device expf). */
uint64_t oracle_count_expf_mismatches(uint32_t first, uint32_t stride, uint64_t n, const float* y,
                                      uint32_t* first_bad) {
  uint64_t bad = 0;
  for (uint64_t i = 0; i < n; ++i) {
    const uint32_t bits = first + (uint32_t)i * stride;
    float x;
    memcpy(&x, &bits, 4);
    const float r = expf(x);
    uint32_t rb, yb;
    memcpy(&rb, &r, 4);
    memcpy(&yb, &y[i], 4);
    if (rb != yb && !(r != r && y[i] != y[i])) {
      if (bad == 0 && first_bad) *first_bad = bits;
      ++bad;
    }
  }
  return bad;
}

/* ---- model head ---------------------------------------------------------------------------- */

/* torch's float -> bfloat16 conversion: round to nearest even; NaN becomes a quiet NaN. */
static uint16_t head_bf16_bits(float x) {
  uint32_t b;
  memcpy(&b, &x, 4);
  if ((b & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
  b += 0x7FFFu + ((b >> 16) & 1u);
  return (uint16_t)(b >> 16);
}
static float head_bf16_value(uint16_t h) {
  const uint32_t b = (uint32_t)h << 16;
  float f;
  memcpy(&f, &b, 4);
  return f;
}

void oracle_head_norm(const float* x, int count, const uint16_t* w, uint16_t* out) {
  for (int t = 0; t < count; ++t) {
    const float* xr = x + (size_t)t * H;
    float v[H];
    double ss = 0.0;
    for (int d = 0; d < H; ++d) {
      v[d] = head_bf16_value(head_bf16_bits(xr[d]));
      ss += (double)v[d] * (double)v[d];
    }
    const float var = (float)ss / (float)H;
    const float r = 1.0f / sqrtf(var + QWEN_RMS_EPS);
    for (int d = 0; d < H; ++d) {
      const float y = head_bf16_value(head_bf16_bits(v[d] * r));
      out[(size_t)t * H + d] = head_bf16_bits(head_bf16_value(w[d]) * y);
    }
  }
}

void oracle_lm_head(const uint16_t* xn, int count, const uint16_t* table, int vocab, float* logits) {
  for (int t = 0; t < count; ++t) {
    double n[H];
    for (int k = 0; k < H; ++k) n[k] = head_bf16_value(xn[(size_t)t * H + k]);
    for (int j = 0; j < vocab; ++j) {
      const uint16_t* e = table + (size_t)j * H;
      double acc = 0.0;
      for (int k = 0; k < H; ++k) acc += n[k] * (double)head_bf16_value(e[k]);
      logits[(size_t)t * vocab + j] = head_bf16_value(head_bf16_bits((float)acc));
    }
  }
}

void oracle_argmax(const float* logits, int count, int vocab, int* ids) {
  for (int t = 0; t < count; ++t) {
    const float* row = logits + (size_t)t * vocab;
    int best = 0;
    for (int j = 0; j < vocab; ++j) {
      if (row[j] != row[j]) {  /* first NaN wins */
        best = j;
        break;
      }
      if (row[j] > row[best]) best = j;
    }
    ids[t] = best;
  }
}
