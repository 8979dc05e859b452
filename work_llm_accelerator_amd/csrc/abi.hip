// The C ABI of the MI355X build: the reference's decode and prefill host-wrapper entry points
// (hls/decode_only/qwen_decode_host_wrapper.h:9-87, hls/prefill_only/qwen_prefill_host_wrapper.h:9-169)
// with identical argument meaning, validation order and status codes.  Every call stages the
// host spans the reference would read onto the GPU, runs the layer executors and copies back
// exactly the spans the reference writes.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <exception>
#include <mutex>
#include <string>
#include <vector>

#include "kernels.hpp"
#include "qwen_decode_host_wrapper.h"
#include "qwen_device_math.hpp"
#include "qwen_prefill_host_wrapper.h"
#include "runtime.hpp"
#include "tops.hpp"

using namespace qwen;

namespace {

template <class Fn>
int guarded(Fn&& fn) {
  try {
    return fn();
  } catch (const HipError& e) {
    set_last_error(std::string(e.what) + ": " + hipGetErrorString(e.code));
  } catch (const std::exception& e) {
    set_last_error(e.what());
  }
  if (std::getenv("QWEN_HIP_VERBOSE")) std::fprintf(stderr, "qwen-mi355x: %s\n", last_error_cstr());
  return QWEN_ERR_DEVICE;
}

struct CallScope {
  Runtime& rt;
  std::lock_guard<std::mutex> lock;
  explicit CallScope(size_t arena_bytes) : rt(Runtime::get()), lock(rt.mu) {
    rt.arena.reset();
    rt.arena.reserve(arena_bytes);
  }
  ~CallScope() { rt.arena.reset(); }
  hipStream_t st() const { return rt.stream; }
  Arena& A() { return rt.arena; }
  void sync() { QWEN_HIP(hipStreamSynchronize(rt.stream)); }
};

bool any_null(std::initializer_list<const void*> ptrs) {
  for (const void* p : ptrs)
    if (!p) return true;
  return false;
}

// Zero weights / unit scales used by the stub entry points (qwen_decode_host_wrapper.cpp:20-35,
// qwen_prefill_host_wrapper.cpp:237-258).
struct StubParams {
  std::vector<uint8_t> zw;
  std::vector<float> ones, zeros;
  HostLayer layer;
  StubParams() : zw((size_t)QWEN_INTERMEDIATE * QWEN_HIDDEN / 2, 0), ones(QWEN_INTERMEDIATE, 1.0f), zeros(QWEN_INTERMEDIATE, 0.0f) {
    const uint8_t* z = zw.data();
    const float* o = ones.data();
    const float* n = zeros.data();
    layer = HostLayer{z, z, z, z, z, z, z, o, o, n, n, n, o, o, o, o, o, o, o};
  }
};
const StubParams& stub_params() {
  static StubParams p;
  return p;
}

size_t act_bytes(int tokens) { return (size_t)tokens * QWEN_HIDDEN * sizeof(float); }
size_t kv_bytes(int rows) { return (size_t)rows * QWEN_KV_WIDTH * sizeof(float); }

// ---------------------------------------------------------------------------------------------
// decode
// ---------------------------------------------------------------------------------------------

size_t decode_call_bytes(int past) {
  return staged_layer_bytes() + decode_workspace_bytes(1) + 2 * kv_bytes(past + 1) + 4 * act_bytes(1) + 64 * 256;
}

// One decode layer for one token (qwen_decode_attention_kernel.cpp:168-218 then
// qwen_decode_mlp_kernel.cpp:87-122).  Host outputs: K/V row `past`, the attention output when
// `att_host` is given, and the layer output when the MLP runs.  When the MLP arguments are
// invalid the attention side effects still happen and status 1 is returned, as in the reference.
int decode_layer_host(const HostLayer& h, const float* x, int past, float* k_cache, float* v_cache, float* att_host,
                      float* out, bool run_mlp, bool mlp_args_ok) {
  return guarded([&]() -> int {
    CallScope cs(decode_call_bytes(past));
    Arena& A = cs.A();
    const hipStream_t st = cs.st();
    const DevLayer d = stage_layer(A, h, st);
    const float* x_d = stage_in(A, x, QWEN_HIDDEN, st);
    const int* pos_d = stage_in(A, &past, 1, st);
    float rope_row[128];
    decode_rope_row_host(past, rope_row);
    const float* rope_d = stage_in(A, rope_row, 128, st);
    const size_t kv_n = (size_t)(past + 1) * QWEN_KV_WIDTH;
    float* kc_d = stage_in(A, k_cache, kv_n, st);
    float* vc_d = stage_in(A, v_cache, kv_n, st);
    float* att_d = A.alloc_n<float>(QWEN_HIDDEN);
    DecodeBatch b{1, pos_d, rope_d, true, kc_d, vc_d, 0, past + 1};
    run_decode_attention(d, x_d, b, att_d, A, st);
    const size_t row = (size_t)past * QWEN_KV_WIDTH;
    copy_out(k_cache + row, kc_d + row, QWEN_KV_WIDTH, st);
    copy_out(v_cache + row, vc_d + row, QWEN_KV_WIDTH, st);
    if (att_host) copy_out(att_host, att_d, QWEN_HIDDEN, st);
    if (!run_mlp || !mlp_args_ok) {
      cs.sync();
      return run_mlp ? QWEN_ERR_KERNEL : QWEN_OK;
    }
    float* out_d = A.alloc_n<float>(QWEN_HIDDEN);
    run_decode_mlp(d, att_d, 1, out_d, A, st);
    copy_out(out, out_d, QWEN_HIDDEN, st);
    cs.sync();
    return QWEN_OK;
  });
}

}  // namespace

extern "C" {

const char* qwen_hip_last_error(void) { return last_error_cstr(); }

int qwen_decode_attention_smoke_forward(const float* x, int past, const float* ln, const uint8_t* qw, const uint8_t* kw,
                                        const uint8_t* vw, const uint8_t* ow, const float* qb, const float* kb,
                                        const float* vb, const float* qs, const float* ks, const float* vs,
                                        const float* os, float* k_cache, float* v_cache, float* out) {
  // qwen_decode_attention_kernel.cpp:187-193
  if (any_null({x, out, ln, qw, kw, vw, ow, qb, kb, vb, qs, ks, vs, os, k_cache, v_cache}) || past < 0)
    return QWEN_ERR_KERNEL;
  const StubParams& z = stub_params();
  HostLayer h = z.layer;  // MLP segments unused here
  h.ln = ln; h.qw = qw; h.kw = kw; h.vw = vw; h.ow = ow;
  h.qb = qb; h.kb = kb; h.vb = vb; h.qs = qs; h.ks = ks; h.vs = vs; h.os = os;
  return decode_layer_host(h, x, past, k_cache, v_cache, out, nullptr, false, true);
}

int qwen_decode_mlp_smoke_forward(const float* a, const float* post_ln, const uint8_t* gw, const uint8_t* uw,
                                  const uint8_t* dw, const float* gs, const float* us, const float* ds, float* out) {
  // qwen_decode_mlp_kernel.cpp:98-102
  if (any_null({a, out, post_ln, gw, uw, dw, gs, us, ds})) return QWEN_ERR_KERNEL;
  HostLayer h = stub_params().layer;
  h.post_ln = post_ln; h.gw = gw; h.uw = uw; h.dw = dw; h.gs = gs; h.us = us; h.ds = ds;
  return guarded([&]() -> int {
    CallScope cs(decode_call_bytes(0));
    const DevLayer d = stage_layer(cs.A(), h, cs.st());
    const float* a_d = stage_in(cs.A(), a, QWEN_HIDDEN, cs.st());
    float* out_d = cs.A().alloc_n<float>(QWEN_HIDDEN);
    run_decode_mlp(d, a_d, 1, out_d, cs.A(), cs.st());
    copy_out(out, out_d, QWEN_HIDDEN, cs.st());
    cs.sync();
    return QWEN_OK;
  });
}

int qwen_decode_layer_smoke_forward(const float* x, int past, const float* ln, const float* post_ln, const uint8_t* qw,
                                    const uint8_t* kw, const uint8_t* vw, const uint8_t* ow, const uint8_t* gw,
                                    const uint8_t* uw, const uint8_t* dw, const float* qb, const float* kb,
                                    const float* vb, const float* qs, const float* ks, const float* vs,
                                    const float* os, const float* gs, const float* us, const float* ds,
                                    float* k_cache, float* v_cache, float* out) {
  // qwen_decode_host_wrapper.cpp:157-218: attention (checks :187-193) then MLP (checks :98-102).
  if (any_null({x, ln, qw, kw, vw, ow, qb, kb, vb, qs, ks, vs, os, k_cache, v_cache}) || past < 0)
    return QWEN_ERR_KERNEL;
  const bool mlp_ok = !any_null({out, post_ln, gw, uw, dw, gs, us, ds});
  const StubParams& z = stub_params();
  HostLayer h{qw, kw, vw, ow, gw ? gw : z.zw.data(), uw ? uw : z.zw.data(), dw ? dw : z.zw.data(),
              ln, post_ln ? post_ln : z.ones.data(), qb, kb, vb, qs, ks, vs, os,
              gs ? gs : z.ones.data(), us ? us : z.ones.data(), ds ? ds : z.ones.data()};
  // The attention kernel checks `out` too (its own output is a local buffer in the reference,
  // so only the MLP sees the caller's output pointer).
  return decode_layer_host(h, x, past, k_cache, v_cache, nullptr, out, true, mlp_ok);
}

int qwen_decode_stub_forward(const float* x, int past, float* out) {
  // qwen_decode_host_wrapper.cpp:12-71
  if (!x || !out || past < 0) return QWEN_ERR_KERNEL;
  std::vector<float> kv((size_t)(past + 1) * QWEN_KV_WIDTH * 2, 0.0f);
  return decode_layer_host(stub_params().layer, x, past, kv.data(), kv.data() + kv.size() / 2, nullptr, out, true, true);
}

static int decode_top(const qwen_decode_descriptor& dsc, const uint8_t* wd, const float* sd, float* kv, float* act,
                      const void* s0, const void* s1, const void* s2, const void* s3, const void* s4) {
  // qwen_decode_top_wrapper.cpp:31-38
  if (const int st = decode_descriptor_status(dsc)) return st;
  if (any_null({wd, sd, kv, act, s0, s1, s2, s3, s4})) return QWEN_ERR_DECODE_PORT;
  const HostLayer h = resolve_host_layer(wd, sd, dsc.layer_weights_base_addr, dsc.layer_scales_base_addr);
  const float* x = act + dsc.input_token_addr / 4;
  float* out = act + dsc.output_token_addr / 4;
  float* kc = kv + dsc.k_cache_base_addr / 4;
  float* vc = kv + dsc.v_cache_base_addr / 4;
  return decode_layer_host(h, x, dsc.past_seq_len, kc, vc, nullptr, out, true, true);
}

int qwen_decode_top_smoke_forward(int layer_id, int past, uint64_t in_addr, uint64_t out_addr, uint64_t wb, uint64_t sb,
                                  uint64_t kb_addr, uint64_t vb_addr, const uint8_t* wd, const float* sd, float* kv,
                                  float* act, uint8_t* wsram, float* kvsram, int32_t* psram, float* smsram,
                                  float* csram) {
  // qwen_decode_host_wrapper.cpp:113-155 (scratch fixed at 0)
  const qwen_decode_descriptor dsc{layer_id, past, in_addr, out_addr, wb, sb, kb_addr, vb_addr, 0};
  return decode_top(dsc, wd, sd, kv, act, wsram, kvsram, psram, smsram, csram);
}

int qwen_decode_dispatch_layers_forward(const qwen_decode_descriptor* dsc, int n, const uint8_t* wd, const float* sd,
                                        float* kv, float* act, uint8_t* wsram, float* kvsram, int32_t* psram,
                                        float* smsram, float* csram, int* completed) {
  // qwen_decode_top_wrapper.cpp:115-130
  if (completed) *completed = 0;
  if (!dsc || n <= 0) return QWEN_ERR_DECODE_DESC;
  for (int i = 0; i < n; ++i) {
    const int st = decode_top(dsc[i], wd, sd, kv, act, wsram, kvsram, psram, smsram, csram);
    if (st) {
      if (completed) *completed = i;
      return st;
    }
  }
  if (completed) *completed = n;
  return QWEN_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------------------------
// prefill
// ---------------------------------------------------------------------------------------------
namespace {

qwen_prefill_attention_tiles atiles(int a_seq, int a_query, int a_key, int a_hp, int a_kvp, int a_hd, int a_qhp,
                                    int a_kvhp) {
  return qwen_prefill_attention_tiles{a_seq, a_query, a_key, a_hp, a_kvp, a_hd, a_qhp, a_kvhp};
}

size_t prefill_call_bytes(int S) {
  return staged_layer_bytes() + prefill_workspace_bytes(S) + 2 * kv_bytes(S) + 4 * act_bytes(S) + 64 * 256;
}

// Attention then (optionally) MLP for one prefill layer.  Host outputs: K/V rows 0..S-1, the
// attention output (`att_host`, may be null) and, when mlp_status == 0, the layer output.
int prefill_layer_host(const HostLayer& h, const float* x, int S, float* k_cache, float* v_cache, float* att_host,
                       float* out, int mlp_status, bool run_mlp) {
  return guarded([&]() -> int {
    CallScope cs(prefill_call_bytes(S));
    Arena& A = cs.A();
    const hipStream_t st = cs.st();
    const float* rope = cs.rt.prefill_rope(S);
    const DevLayer d = stage_layer(A, h, st);
    const float* x_d = stage_in(A, x, (size_t)S * QWEN_HIDDEN, st);
    float* kc_d = A.alloc_n<float>((size_t)S * QWEN_KV_WIDTH);
    float* vc_d = A.alloc_n<float>((size_t)S * QWEN_KV_WIDTH);
    float* att_d = A.alloc_n<float>((size_t)S * QWEN_HIDDEN);
    run_prefill_attention(d, x_d, S, 0, rope, kc_d, vc_d, att_d, A, st);
    copy_out(k_cache, kc_d, (size_t)S * QWEN_KV_WIDTH, st);
    copy_out(v_cache, vc_d, (size_t)S * QWEN_KV_WIDTH, st);
    if (att_host) copy_out(att_host, att_d, (size_t)S * QWEN_HIDDEN, st);
    if (!run_mlp || mlp_status != QWEN_OK) {
      cs.sync();
      return run_mlp ? mlp_status : QWEN_OK;
    }
    float* out_d = A.alloc_n<float>((size_t)S * QWEN_HIDDEN);
    run_prefill_mlp(d, att_d, S, out_d, A, st);
    copy_out(out, out_d, (size_t)S * QWEN_HIDDEN, st);
    cs.sync();
    return QWEN_OK;
  });
}

// qwen_prefill_top_wrapper (qwen_prefill_top_wrapper.cpp:7-18) + qwen_prefill_top_core (:84-183).
int prefill_top(const qwen_prefill_descriptor& d, const uint8_t* wd, const float* sd, float* kv, float* act,
                const void* s0, const void* s1, const void* s2, const void* s3, const void* s4) {
  int mst = QWEN_OK;
  const int st = prefill_top_status(d, any_null({wd, sd, kv, act, s0, s1, s2, s3, s4}), &mst);
  if (st) return st;
  const HostLayer h = resolve_host_layer(wd, sd, d.layer_weights_base_addr, d.layer_scales_base_addr);
  const int S = d.seq_len;
  return prefill_layer_host(h, act + d.input_sequence_addr / 4, S, kv + d.k_cache_base_addr / 4,
                            kv + d.v_cache_base_addr / 4, act + d.scratch_base_addr / 4,
                            act + d.output_sequence_addr / 4, mst, true);
}

}  // namespace

extern "C" {

int qwen_prefill_attention_smoke_forward(const float* x, int S, int a_seq, int a_query, int a_key, int a_hp, int a_kvp,
                                         int a_hd, int a_qhp, int a_kvhp, const float* ln, const uint8_t* qw,
                                         const uint8_t* kw, const uint8_t* vw, const uint8_t* ow, const float* qb,
                                         const float* kb, const float* vb, const float* qs, const float* ks,
                                         const float* vs, const float* os, float* k_cache, float* v_cache,
                                         float* out) {
  if (any_null({x, out, ln, qw, kw, vw, ow, qb, kb, vb, qs, ks, vs, os, k_cache, v_cache})) return QWEN_ERR_KERNEL;
  const int st = check_prefill_attention_tiles(S, atiles(a_seq, a_query, a_key, a_hp, a_kvp, a_hd, a_qhp, a_kvhp));
  if (st) return st;
  HostLayer h = stub_params().layer;
  h.ln = ln; h.qw = qw; h.kw = kw; h.vw = vw; h.ow = ow;
  h.qb = qb; h.kb = kb; h.vb = vb; h.qs = qs; h.ks = ks; h.vs = vs; h.os = os;
  return prefill_layer_host(h, x, S, k_cache, v_cache, out, nullptr, QWEN_OK, false);
}

int qwen_prefill_mlp_smoke_forward(const float* a, int S, int m_seq, int m_hidden, int m_ff, const float* post_ln,
                                   const uint8_t* gw, const uint8_t* uw, const uint8_t* dw, const float* gs,
                                   const float* us, const float* ds, float* out) {
  if (any_null({a, out, post_ln, gw, uw, dw, gs, us, ds})) return QWEN_ERR_KERNEL;
  const int st = check_prefill_mlp_tiles(S, qwen_prefill_mlp_tiles{m_seq, m_hidden, m_ff});
  if (st) return st;
  HostLayer h = stub_params().layer;
  h.post_ln = post_ln; h.gw = gw; h.uw = uw; h.dw = dw; h.gs = gs; h.us = us; h.ds = ds;
  return guarded([&]() -> int {
    CallScope cs(prefill_call_bytes(S));
    const DevLayer d = stage_layer(cs.A(), h, cs.st());
    const float* a_d = stage_in(cs.A(), a, (size_t)S * QWEN_HIDDEN, cs.st());
    float* out_d = cs.A().alloc_n<float>((size_t)S * QWEN_HIDDEN);
    run_prefill_mlp(d, a_d, S, out_d, cs.A(), cs.st());
    copy_out(out, out_d, (size_t)S * QWEN_HIDDEN, cs.st());
    cs.sync();
    return QWEN_OK;
  });
}

int qwen_prefill_layer_smoke_forward(const float* x, int S, int a_seq, int a_query, int a_key, int a_hp, int a_kvp,
                                     int a_hd, int a_qhp, int a_kvhp, int m_seq, int m_hidden, int m_ff,
                                     const float* ln, const float* post_ln, const uint8_t* qw, const uint8_t* kw,
                                     const uint8_t* vw, const uint8_t* ow, const uint8_t* gw, const uint8_t* uw,
                                     const uint8_t* dw, const float* qb, const float* kb, const float* vb,
                                     const float* qs, const float* ks, const float* vs, const float* os,
                                     const float* gs, const float* us, const float* ds, float* k_cache,
                                     float* v_cache, float* out) {
  // qwen_prefill_host_wrapper.cpp:389-476: attention (its output is a local buffer) then MLP.
  if (any_null({x, ln, qw, kw, vw, ow, qb, kb, vb, qs, ks, vs, os, k_cache, v_cache})) return QWEN_ERR_KERNEL;
  const int ast = check_prefill_attention_tiles(S, atiles(a_seq, a_query, a_key, a_hp, a_kvp, a_hd, a_qhp, a_kvhp));
  if (ast) return ast;
  int mst = check_prefill_mlp_tiles(S, qwen_prefill_mlp_tiles{m_seq, m_hidden, m_ff});
  if (any_null({out, post_ln, gw, uw, dw, gs, us, ds})) mst = QWEN_ERR_KERNEL;
  const StubParams& z = stub_params();
  HostLayer h{qw, kw, vw, ow, gw ? gw : z.zw.data(), uw ? uw : z.zw.data(), dw ? dw : z.zw.data(),
              ln, post_ln ? post_ln : z.ones.data(), qb, kb, vb, qs, ks, vs, os,
              gs ? gs : z.ones.data(), us ? us : z.ones.data(), ds ? ds : z.ones.data()};
  return prefill_layer_host(h, x, S, k_cache, v_cache, nullptr, out, mst, true);
}

int qwen_prefill_glue_smoke_forward(const float* x, int S, int a_seq, int a_query, int a_key, int a_hp, int a_kvp,
                                    int a_hd, int a_qhp, int a_kvhp, int m_seq, int m_hidden, int m_ff,
                                    const float* ln, const float* post_ln, const uint8_t* qw, const uint8_t* kw,
                                    const uint8_t* vw, const uint8_t* ow, const uint8_t* gw, const uint8_t* uw,
                                    const uint8_t* dw, const float* qb, const float* kb, const float* vb,
                                    const float* qs, const float* ks, const float* vs, const float* os,
                                    const float* gs, const float* us, const float* ds, float* k_cache,
                                    float* v_cache, float* out) {
  // qwen_prefill_host_wrapper.cpp:514-549
  if (any_null({x, ln, post_ln, qw, kw, vw, ow, gw, uw, dw, qb, kb, vb, qs, ks, vs, os, gs, us, ds, k_cache, v_cache,
                out}) ||
      S <= 0)
    return QWEN_ERR_KERNEL;
  const qwen_prefill_tiles dt = qwen_default_prefill_tiles();
  if (a_seq != dt.attention.seq || a_query != dt.attention.query || a_key != dt.attention.key ||
      a_hp != dt.attention.hidden_proj || a_kvp != dt.attention.kv_proj || a_hd != QWEN_HEAD_DIM ||
      a_qhp != dt.attention.query_heads_parallel || a_kvhp != dt.attention.kv_heads_parallel ||
      m_seq != dt.mlp.seq || m_hidden != dt.mlp.hidden || m_ff != dt.mlp.ff)
    return QWEN_ERR_CAPACITY;
  // valid_attention_stream_config (qwen_prefill_attention_stream_top.cpp:99-101)
  if (S > QWEN_PREFILL_CAPACITY) return QWEN_ERR_CAPACITY;
  const HostLayer h{qw, kw, vw, ow, gw, uw, dw, ln, post_ln, qb, kb, vb, qs, ks, vs, os, gs, us, ds};
  return prefill_layer_host(h, x, S, k_cache, v_cache, nullptr, out, QWEN_OK, true);
}

int qwen_prefill_stub_forward(const float* x, int S, int a_seq, int a_query, int a_key, int a_hp, int a_kvp, int a_hd,
                              int a_qhp, int a_kvhp, int m_seq, int m_hidden, int m_ff, float* out) {
  // qwen_prefill_host_wrapper.cpp:205-298
  if (!x || !out || S <= 0) return QWEN_ERR_KERNEL;
  const int ast = check_prefill_attention_tiles(S, atiles(a_seq, a_query, a_key, a_hp, a_kvp, a_hd, a_qhp, a_kvhp));
  if (ast) return ast;
  const int mst = check_prefill_mlp_tiles(S, qwen_prefill_mlp_tiles{m_seq, m_hidden, m_ff});
  std::vector<float> kv((size_t)S * QWEN_KV_WIDTH * 2, 0.0f);
  return prefill_layer_host(stub_params().layer, x, S, kv.data(), kv.data() + kv.size() / 2, nullptr, out, mst, true);
}

int qwen_prefill_top_smoke_forward(int layer_id, int S, int a_seq, int a_query, int a_key, int a_hp, int a_kvp,
                                   int a_hd, int a_qhp, int a_kvhp, int m_seq, int m_hidden, int m_ff, uint64_t in_addr,
                                   uint64_t out_addr, uint64_t wb, uint64_t sb, uint64_t kb_addr, uint64_t vb_addr,
                                   const uint8_t* wd, const float* sd, float* kv, float* act, uint8_t* wsram,
                                   float* kvsram, int32_t* psram, float* smsram, float* csram) {
  // qwen_prefill_host_wrapper.cpp:639-705: scratch = output + S*1536*4.
  qwen_prefill_descriptor d;
  d.layer_id = layer_id;
  d.seq_len = S;
  d.tiles.attention = atiles(a_seq, a_query, a_key, a_hp, a_kvp, a_hd, a_qhp, a_kvhp);
  d.tiles.mlp = qwen_prefill_mlp_tiles{m_seq, m_hidden, m_ff};
  d.input_sequence_addr = in_addr;
  d.output_sequence_addr = out_addr;
  d.layer_weights_base_addr = wb;
  d.layer_scales_base_addr = sb;
  d.k_cache_base_addr = kb_addr;
  d.v_cache_base_addr = vb_addr;
  d.scratch_base_addr = out_addr + static_cast<uint64_t>(S) * (uint64_t)QWEN_HIDDEN * sizeof(float);
  return prefill_top(d, wd, sd, kv, act, wsram, kvsram, psram, smsram, csram);
}

int qwen_prefill_dispatch_layers_forward(const qwen_prefill_descriptor* dsc, int n, const uint8_t* wd, const float* sd,
                                         float* kv, float* act, uint8_t* wsram, float* kvsram, int32_t* psram,
                                         float* smsram, float* csram, int* completed) {
  // qwen_prefill_top_wrapper.cpp:20-35
  if (completed) *completed = 0;
  if (!dsc || n <= 0) return QWEN_ERR_PREFILL_DESC;
  for (int i = 0; i < n; ++i) {
    const int st = prefill_top(dsc[i], wd, sd, kv, act, wsram, kvsram, psram, smsram, csram);
    if (st) {
      if (completed) *completed = i;
      return st;
    }
  }
  if (completed) *completed = n;
  return QWEN_OK;
}

// ---------------------------------------------------------------------------------------------
// Unquantized layer-0 reference wrappers (qwen_decode_layer0_reference_wrapper.cpp:75-209,
// qwen_prefill_layer0_reference_wrapper.cpp:60-347): fp32 weights, double accumulation, HF
// head-major caches [kv_head][T][128].  Biases may be null (no bias).
// ---------------------------------------------------------------------------------------------
}  // extern "C"

namespace {

struct HostL0 {
  const float *ln, *qw, *qb, *kw, *kb, *vw, *vb, *ow, *ob, *post_ln, *gw, *gb, *uw, *ub, *dw, *db;
  bool weights_present() const { return !any_null({ln, qw, kw, vw, ow, post_ln, gw, uw, dw}); }
};

size_t l0_weight_floats() {
  return (size_t)QWEN_HIDDEN * (2 * QWEN_HIDDEN + 2 * QWEN_KV_WIDTH + 3 * QWEN_INTERMEDIATE) +
         (size_t)(5 * QWEN_HIDDEN + 2 * QWEN_KV_WIDTH + 2 * QWEN_INTERMEDIATE);
}

Layer0Weights stage_l0(Arena& A, const HostL0& h, hipStream_t st) {
  auto opt = [&](const float* p, size_t n) -> const float* { return p ? stage_in(A, p, n, st) : nullptr; };
  const size_t H = QWEN_HIDDEN, KV = QWEN_KV_WIDTH, I = QWEN_INTERMEDIATE;
  Layer0Weights w;
  w.ln = stage_in(A, h.ln, H, st);
  w.qw = stage_in(A, h.qw, H * H, st);
  w.qb = opt(h.qb, H);
  w.kw = stage_in(A, h.kw, KV * H, st);
  w.kb = opt(h.kb, KV);
  w.vw = stage_in(A, h.vw, KV * H, st);
  w.vb = opt(h.vb, KV);
  w.ow = stage_in(A, h.ow, H * H, st);
  w.ob = opt(h.ob, H);
  w.post_ln = stage_in(A, h.post_ln, H, st);
  w.gw = stage_in(A, h.gw, I * H, st);
  w.gb = opt(h.gb, I);
  w.uw = stage_in(A, h.uw, I * H, st);
  w.ub = opt(h.ub, I);
  w.dw = stage_in(A, h.dw, H * I, st);
  w.db = opt(h.db, H);
  return w;
}

// RoPE rows of the layer-0 wrappers: angle = position * pow(1e6, -2p/128) in double with the host libm
// (decode_layer0 :113-116,51-63; prefill_layer0 :107-109,125-160); prefill rounds cos/sin to bf16.
std::vector<float> l0_rope_rows(int first, int count, bool prefill) {
  std::vector<double> inv_freq(QWEN_HEAD_DIM / 2);
  for (int i = 0; i < QWEN_HEAD_DIM / 2; ++i)
    inv_freq[i] = std::pow(1000000.0, -2.0 * static_cast<double>(i) / static_cast<double>(QWEN_HEAD_DIM));
  std::vector<float> tab((size_t)count * 128);
  for (int r = 0; r < count; ++r)
    for (int p = 0; p < QWEN_HEAD_DIM / 2; ++p) {
      const double angle = static_cast<double>(first + r) * inv_freq[p];
      float c = static_cast<float>(std::cos(angle));
      float s = static_cast<float>(std::sin(angle));
      if (prefill) {
        c = round_bf16(c);
        s = round_bf16(s);
      }
      tab[(size_t)r * 128 + p] = c;
      tab[(size_t)r * 128 + 64 + p] = s;
    }
  return tab;
}

int prefill_layer0(const float* x, int S, const HostL0& h, float eps, float* out, float* k_cache, float* v_cache) {
  if (!x || !out || S <= 0 || S > QWEN_MAX_SEQ) return QWEN_ERR_KERNEL;
  if ((k_cache == nullptr) != (v_cache == nullptr)) return QWEN_ERR_KERNEL;
  if (!h.weights_present()) return QWEN_ERR_KERNEL;
  return guarded([&]() -> int {
    const size_t kvn = (size_t)QWEN_KV_HEADS * S * QWEN_HEAD_DIM;
    CallScope cs(l0_weight_floats() * 4 + 64 * 256 + layer0_workspace_bytes(S, 0, false) +
                 ((size_t)S * (2 * QWEN_HIDDEN + 128) + 2 * kvn) * 4);
    Arena& A = cs.A();
    const hipStream_t st = cs.st();
    const Layer0Weights w = stage_l0(A, h, st);
    const float* x_d = stage_in(A, x, (size_t)S * QWEN_HIDDEN, st);
    const std::vector<float> tab = l0_rope_rows(0, S, true);
    const float* tab_d = stage_in(A, tab.data(), tab.size(), st);
    float* out_d = A.alloc_n<float>((size_t)S * QWEN_HIDDEN);
    float* k_d = k_cache ? A.alloc_n<float>(kvn) : nullptr;
    float* v_d = k_cache ? A.alloc_n<float>(kvn) : nullptr;
    void* ws = A.alloc(layer0_workspace_bytes(S, 0, false));
    run_layer0_reference(w, eps, false, x_d, S, 0, tab_d, nullptr, nullptr, out_d, k_d, v_d, ws, st);
    QWEN_HIP(hipGetLastError());
    copy_out(out, out_d, (size_t)S * QWEN_HIDDEN, st);
    if (k_cache) {
      copy_out(k_cache, k_d, kvn, st);
      copy_out(v_cache, v_d, kvn, st);
    }
    cs.sync();
    return QWEN_OK;
  });
}

}  // namespace

extern "C" {

int qwen_decode_layer0_reference_forward(const float* input_token, int past_seq_len, const float* past_k_cache,
                                         const float* past_v_cache, const float* input_layernorm_weight,
                                         const float* q_weight, const float* q_bias, const float* k_weight,
                                         const float* k_bias, const float* v_weight, const float* v_bias,
                                         const float* o_weight, const float* o_bias,
                                         const float* post_attention_layernorm_weight, const float* gate_weight,
                                         const float* gate_bias, const float* up_weight, const float* up_bias,
                                         const float* down_weight, const float* down_bias, float rms_eps,
                                         float* output_token, float* next_k_cache, float* next_v_cache) {
  // qwen_decode_layer0_reference_wrapper.cpp:99-101
  if (!input_token || !output_token || !next_k_cache || !next_v_cache || past_seq_len < 0) return QWEN_ERR_KERNEL;
  const HostL0 h{input_layernorm_weight, q_weight, q_bias, k_weight, k_bias, v_weight, v_bias, o_weight, o_bias,
                 post_attention_layernorm_weight, gate_weight, gate_bias, up_weight, up_bias, down_weight, down_bias};
  if (!h.weights_present() || past_seq_len > QWEN_MAX_SEQ - 1 ||
      (past_seq_len > 0 && (!past_k_cache || !past_v_cache)))
    return QWEN_ERR_KERNEL;
  return guarded([&]() -> int {
    const int past = past_seq_len;
    const size_t past_n = (size_t)QWEN_KV_HEADS * past * QWEN_HEAD_DIM;
    const size_t next_n = (size_t)QWEN_KV_HEADS * (past + 1) * QWEN_HEAD_DIM;
    CallScope cs(l0_weight_floats() * 4 + 64 * 256 + layer0_workspace_bytes(1, past, true) +
                 (2 * QWEN_HIDDEN + 128 + 2 * past_n + 2 * next_n) * 4);
    Arena& A = cs.A();
    const hipStream_t st = cs.st();
    const Layer0Weights w = stage_l0(A, h, st);
    const float* x_d = stage_in(A, input_token, QWEN_HIDDEN, st);
    const std::vector<float> tab = l0_rope_rows(past, 1, false);
    const float* tab_d = stage_in(A, tab.data(), tab.size(), st);
    const float* pk_d = stage_in(A, past_k_cache, past_n, st);
    const float* pv_d = stage_in(A, past_v_cache, past_n, st);
    float* out_d = A.alloc_n<float>(QWEN_HIDDEN);
    float* k_d = A.alloc_n<float>(next_n);
    float* v_d = A.alloc_n<float>(next_n);
    void* ws = A.alloc(layer0_workspace_bytes(1, past, true));
    run_layer0_reference(w, rms_eps, true, x_d, 1, past, tab_d, pk_d, pv_d, out_d, k_d, v_d, ws, st);
    QWEN_HIP(hipGetLastError());
    copy_out(output_token, out_d, QWEN_HIDDEN, st);
    copy_out(next_k_cache, k_d, next_n, st);
    copy_out(next_v_cache, v_d, next_n, st);
    cs.sync();
    return QWEN_OK;
  });
}

int qwen_prefill_layer0_reference_forward(const float* input_sequence, int seq_len,
                                          const float* input_layernorm_weight, const float* q_weight,
                                          const float* q_bias, const float* k_weight, const float* k_bias,
                                          const float* v_weight, const float* v_bias, const float* o_weight,
                                          const float* o_bias, const float* post_attention_layernorm_weight,
                                          const float* gate_weight, const float* gate_bias, const float* up_weight,
                                          const float* up_bias, const float* down_weight, const float* down_bias,
                                          float rms_eps, float* output_sequence) {
  const HostL0 h{input_layernorm_weight, q_weight, q_bias, k_weight, k_bias, v_weight, v_bias, o_weight, o_bias,
                 post_attention_layernorm_weight, gate_weight, gate_bias, up_weight, up_bias, down_weight, down_bias};
  return prefill_layer0(input_sequence, seq_len, h, rms_eps, output_sequence, nullptr, nullptr);
}

int qwen_prefill_layer0_reference_forward_with_cache(
    const float* input_sequence, int seq_len, const float* input_layernorm_weight, const float* q_weight,
    const float* q_bias, const float* k_weight, const float* k_bias, const float* v_weight, const float* v_bias,
    const float* o_weight, const float* o_bias, const float* post_attention_layernorm_weight, const float* gate_weight,
    const float* gate_bias, const float* up_weight, const float* up_bias, const float* down_weight,
    const float* down_bias, float rms_eps, float* output_sequence, float* k_cache, float* v_cache) {
  const HostL0 h{input_layernorm_weight, q_weight, q_bias, k_weight, k_bias, v_weight, v_bias, o_weight, o_bias,
                 post_attention_layernorm_weight, gate_weight, gate_bias, up_weight, up_bias, down_weight, down_bias};
  return prefill_layer0(input_sequence, seq_len, h, rms_eps, output_sequence, k_cache, v_cache);
}

}  // extern "C"
