// Host runtime: arena, RoPE tables, layer staging and the per-layer executors.
#include "runtime.hpp"

#include <cmath>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>

#include "kernels.hpp"

namespace qwen {

namespace {
thread_local std::string g_last_error;
}
void set_last_error(const std::string& msg) { g_last_error = msg; }
const char* last_error_cstr() { return g_last_error.c_str(); }

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw HipError{e, what};
}

HostLayer resolve_host_layer(const uint8_t* wd, const float* sd, uint64_t wb, uint64_t sb) {
  HostLayer p;
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

// ---------------------------------------------------------------------------------------------
Arena::~Arena() {
  // Process teardown: the HIP runtime may already be gone; leave the block to the driver.
}

void Arena::reserve(size_t bytes) {
  if (bytes <= cap_) return;
  if (used_ != 0) throw std::runtime_error("arena grown while in use");
  if (base_) {
    QWEN_HIP(hipDeviceSynchronize());
    QWEN_HIP(hipFree(base_));
    base_ = nullptr;
    cap_ = 0;
  }
  const size_t want = bytes + (bytes >> 3) + (1u << 20);
  QWEN_HIP(hipMalloc(reinterpret_cast<void**>(&base_), want));
  cap_ = want;
}

void* Arena::alloc(size_t bytes) {
  const size_t off = (used_ + 255u) & ~size_t(255u);
  if (off + bytes > cap_) throw std::runtime_error("arena capacity exceeded");
  used_ = off + bytes;
  return base_ + off;
}

// ---------------------------------------------------------------------------------------------
Runtime& Runtime::get() {
  static Runtime* rt = new Runtime();  // never destroyed: HIP objects outlive static teardown
  return *rt;
}

Runtime::Runtime() {
  // Default-priority stream (no priority other than the default is ever used).
  QWEN_HIP(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
}

void decode_rope_row_host(int position, float* out) {
  // qwen_decode_attention_kernel.cpp:29-42: angle in double with libm pow, cos, sin.
  for (int p = 0; p < QWEN_HEAD_DIM / 2; ++p) {
    const double angle = static_cast<double>(position) *
                         std::pow(static_cast<double>(QWEN_ROPE_THETA),
                                  -2.0 * static_cast<double>(p) / static_cast<double>(QWEN_HEAD_DIM));
    out[p] = static_cast<float>(std::cos(angle));
    out[64 + p] = static_cast<float>(std::sin(angle));
  }
}

const float* Runtime::prefill_rope(int positions) {
  if (positions <= prefill_rope_rows_) return prefill_rope_;
  int rows = 256;
  while (rows < positions) rows *= 2;
  if (rows > QWEN_MAX_SEQ) rows = QWEN_MAX_SEQ;
  float* fresh = nullptr;
  QWEN_HIP(hipMalloc(reinterpret_cast<void**>(&fresh), sizeof(float) * 128u * (size_t)rows));
  launch_rope_table_prefill(fresh, 0, rows, stream);
  QWEN_HIP(hipGetLastError());
  QWEN_HIP(hipStreamSynchronize(stream));
  if (prefill_rope_) QWEN_HIP(hipFree(prefill_rope_));
  prefill_rope_ = fresh;
  prefill_rope_rows_ = rows;
  return prefill_rope_;
}

const float* Runtime::decode_rope(int positions) {
  if (positions <= decode_rope_rows_) return decode_rope_;
  int rows = 256;
  while (rows < positions) rows *= 2;
  if (rows > QWEN_MAX_SEQ) rows = QWEN_MAX_SEQ;
  std::vector<float> host((size_t)rows * 128u);
  for (int r = 0; r < rows; ++r) decode_rope_row_host(r, &host[(size_t)r * 128u]);
  float* fresh = nullptr;
  QWEN_HIP(hipMalloc(reinterpret_cast<void**>(&fresh), sizeof(float) * host.size()));
  QWEN_HIP(hipMemcpy(fresh, host.data(), sizeof(float) * host.size(), hipMemcpyHostToDevice));
  if (decode_rope_) QWEN_HIP(hipFree(decode_rope_));
  decode_rope_ = fresh;
  decode_rope_rows_ = rows;
  return decode_rope_;
}

// ---------------------------------------------------------------------------------------------
size_t staged_layer_bytes() { return QWEN_LAYER_BYTES + 64u * 256u; }

DevLayer stage_layer(Arena& a, const HostLayer& h, hipStream_t st) {
  DevLayer d;
  d.qw = stage_in(a, h.qw, QWEN_Q_WEIGHT_BYTES, st);
  d.kw = stage_in(a, h.kw, QWEN_K_WEIGHT_BYTES, st);
  d.vw = stage_in(a, h.vw, QWEN_V_WEIGHT_BYTES, st);
  d.ow = stage_in(a, h.ow, QWEN_O_WEIGHT_BYTES, st);
  d.gw = stage_in(a, h.gw, QWEN_GATE_WEIGHT_BYTES, st);
  d.uw = stage_in(a, h.uw, QWEN_UP_WEIGHT_BYTES, st);
  d.dw = stage_in(a, h.dw, QWEN_DOWN_WEIGHT_BYTES, st);
  d.ln = stage_in(a, h.ln, QWEN_HIDDEN, st);
  d.post_ln = stage_in(a, h.post_ln, QWEN_HIDDEN, st);
  d.qb = stage_in(a, h.qb, QWEN_HIDDEN, st);
  d.kb = stage_in(a, h.kb, QWEN_KV_WIDTH, st);
  d.vb = stage_in(a, h.vb, QWEN_KV_WIDTH, st);
  d.qs = stage_in(a, h.qs, QWEN_HIDDEN, st);
  d.ks = stage_in(a, h.ks, QWEN_KV_WIDTH, st);
  d.vs = stage_in(a, h.vs, QWEN_KV_WIDTH, st);
  d.os = stage_in(a, h.os, QWEN_HIDDEN, st);
  d.gs = stage_in(a, h.gs, QWEN_INTERMEDIATE, st);
  d.us = stage_in(a, h.us, QWEN_INTERMEDIATE, st);
  d.ds = stage_in(a, h.ds, QWEN_HIDDEN, st);
  return d;
}

// ---------------------------------------------------------------------------------------------
// Executors.  Intermediates come from the arena; sizes in floats per token:
//   xn 1536, q 1536, k 256, v 256, ctx 1536 (attention);  pn 1536, g/u/s 3*8960 (MLP).
// The attention and MLP executors each take their own part, so one token's layer needs the sum.
namespace {
size_t up64(size_t n) { return (n + 63u) & ~size_t(63u); }
size_t decode_attention_floats(size_t T) { return 3u * up64(T * QWEN_HIDDEN) + 2u * up64(T * QWEN_KV_WIDTH); }
size_t decode_mlp_floats(size_t T) { return up64(T * QWEN_HIDDEN) + 3u * up64(T * QWEN_INTERMEDIATE); }

void carve_attention_part(DecodeWorkspace& w, float* p, size_t T) {
  auto take = [&](size_t n) {
    float* r = p;
    p += up64(n);
    return r;
  };
  w.xn = take(T * QWEN_HIDDEN);
  w.q = take(T * QWEN_HIDDEN);
  w.k = take(T * QWEN_KV_WIDTH);
  w.v = take(T * QWEN_KV_WIDTH);
  w.ctx = take(T * QWEN_HIDDEN);
}

void carve_mlp_part(DecodeWorkspace& w, float* p, size_t T) {
  auto take = [&](size_t n) {
    float* r = p;
    p += up64(n);
    return r;
  };
  w.pn = take(T * QWEN_HIDDEN);
  w.g = take(T * QWEN_INTERMEDIATE);
  w.u = take(T * QWEN_INTERMEDIATE);
  w.s = take(T * QWEN_INTERMEDIATE);
}
}  // namespace

// Two arena allocations (attention part, MLP part), each aligned to 256 bytes.
size_t decode_workspace_bytes(int tokens) { return decode_workspace_floats(tokens) * sizeof(float) + 2u * 256u; }
// run_prefill_attention's xn, q, ctx and run_prefill_mlp's pn, g, u, s: seven allocations.
size_t prefill_workspace_bytes(int tokens) {
  const size_t T = (size_t)tokens;
  return (4u * T * QWEN_HIDDEN + 3u * T * QWEN_INTERMEDIATE) * sizeof(float) + 7u * 256u;
}

size_t decode_workspace_floats(int tokens) {
  return decode_attention_floats((size_t)tokens) + decode_mlp_floats((size_t)tokens);
}

DecodeWorkspace carve_decode_workspace(float* base, int tokens) {
  const size_t T = (size_t)tokens;
  DecodeWorkspace w;
  carve_attention_part(w, base, T);
  carve_mlp_part(w, base + decode_attention_floats(T), T);
  return w;
}

void run_decode_attention_ws(const DevLayer& L, const float* x, const DecodeBatch& b, float* att,
                             const DecodeWorkspace& w, hipStream_t st) {
  const int T = b.tokens;
  launch_rmsnorm_ordered(x, L.ln, w.xn, T, false, st);
  launch_project_ordered(w.xn, T, QWEN_HIDDEN, L.qw, L.qs, L.qb, QWEN_HIDDEN, w.q, nullptr, st);
  launch_project_ordered(w.xn, T, QWEN_HIDDEN, L.kw, L.ks, L.kb, QWEN_KV_WIDTH, w.k, nullptr, st);
  launch_project_ordered(w.xn, T, QWEN_HIDDEN, L.vw, L.vs, L.vb, QWEN_KV_WIDTH, w.v, nullptr, st);
  launch_rope_append_decode(w.q, w.k, w.v, b.pos, b.rope, b.rope_per_token, b.k_cache, b.v_cache, b.cache_stride,
                            b.max_keys, T, st);
  launch_attention_ordered(w.q, b.k_cache, b.v_cache, b.cache_stride, b.pos, b.max_keys, T, false, 0, w.ctx, st);
  launch_project_ordered(w.ctx, T, QWEN_HIDDEN, L.ow, L.os, nullptr, QWEN_HIDDEN, att, nullptr, st);
  QWEN_HIP(hipGetLastError());
}

void run_decode_mlp_ws(const DevLayer& L, const float* att, int T, float* out, const DecodeWorkspace& w,
                       hipStream_t st) {
  launch_rmsnorm_ordered(att, L.post_ln, w.pn, T, false, st);
  launch_project_ordered(w.pn, T, QWEN_HIDDEN, L.gw, L.gs, nullptr, QWEN_INTERMEDIATE, w.g, nullptr, st);
  launch_project_ordered(w.pn, T, QWEN_HIDDEN, L.uw, L.us, nullptr, QWEN_INTERMEDIATE, w.u, nullptr, st);
  launch_silu_mul(w.g, w.u, w.s, (size_t)T * QWEN_INTERMEDIATE, false, st);
  launch_project_ordered(w.s, T, QWEN_INTERMEDIATE, L.dw, L.ds, nullptr, QWEN_HIDDEN, out, att, st);
  QWEN_HIP(hipGetLastError());
}

void run_decode_attention(const DevLayer& L, const float* x, const DecodeBatch& b, float* att, Arena& a,
                          hipStream_t st) {
  DecodeWorkspace w{};
  carve_attention_part(w, a.alloc_n<float>(decode_attention_floats((size_t)b.tokens)), (size_t)b.tokens);
  run_decode_attention_ws(L, x, b, att, w, st);
}

void run_decode_mlp(const DevLayer& L, const float* att, int T, float* out, Arena& a, hipStream_t st) {
  DecodeWorkspace w{};
  carve_mlp_part(w, a.alloc_n<float>(decode_mlp_floats((size_t)T)), (size_t)T);
  run_decode_mlp_ws(L, att, T, out, w, st);
}

void run_prefill_attention(const DevLayer& L, const float* x, int T, int past, const float* rope, float* k_rows,
                           float* v_rows, float* att, Arena& a, hipStream_t st) {
  float* k_new = k_rows + (size_t)past * QWEN_KV_WIDTH;
  float* v_new = v_rows + (size_t)past * QWEN_KV_WIDTH;
  float* xn = a.alloc_n<float>((size_t)T * QWEN_HIDDEN);
  float* q = a.alloc_n<float>((size_t)T * QWEN_HIDDEN);
  float* ctx = a.alloc_n<float>((size_t)T * QWEN_HIDDEN);
  launch_rmsnorm_ordered(x, L.ln, xn, T, true, st);
  launch_project_ordered(xn, T, QWEN_HIDDEN, L.kw, L.ks, L.kb, QWEN_KV_WIDTH, k_new, nullptr, st);
  launch_project_ordered(xn, T, QWEN_HIDDEN, L.vw, L.vs, L.vb, QWEN_KV_WIDTH, v_new, nullptr, st);
  launch_project_ordered(xn, T, QWEN_HIDDEN, L.qw, L.qs, L.qb, QWEN_HIDDEN, q, nullptr, st);
  launch_rope_prefill(q, k_new, rope + (size_t)past * 128, T, st);
  launch_attention_ordered(q, k_rows, v_rows, 0, nullptr, past + T, T, true, past, ctx, st);
  launch_project_ordered(ctx, T, QWEN_HIDDEN, L.ow, L.os, nullptr, QWEN_HIDDEN, att, nullptr, st);
  QWEN_HIP(hipGetLastError());
}

void run_prefill_mlp(const DevLayer& L, const float* att, int T, float* out, Arena& a, hipStream_t st) {
  float* pn = a.alloc_n<float>((size_t)T * QWEN_HIDDEN);
  float* g = a.alloc_n<float>((size_t)T * QWEN_INTERMEDIATE);
  float* u = a.alloc_n<float>((size_t)T * QWEN_INTERMEDIATE);
  float* s = a.alloc_n<float>((size_t)T * QWEN_INTERMEDIATE);
  launch_rmsnorm_ordered(att, L.post_ln, pn, T, true, st);
  launch_project_ordered(pn, T, QWEN_HIDDEN, L.gw, L.gs, nullptr, QWEN_INTERMEDIATE, g, nullptr, st);
  launch_project_ordered(pn, T, QWEN_HIDDEN, L.uw, L.us, nullptr, QWEN_INTERMEDIATE, u, nullptr, st);
  launch_silu_mul(g, u, s, (size_t)T * QWEN_INTERMEDIATE, true, st);
  launch_project_ordered(s, T, QWEN_INTERMEDIATE, L.dw, L.ds, nullptr, QWEN_HIDDEN, out, att, st);
  QWEN_HIP(hipGetLastError());
}

}  // namespace qwen
