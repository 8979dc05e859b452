// Host runtime of the MI355X build: device arena, staging helpers and the per-layer executors
// that chain the HIP kernels.  One process-wide Runtime per device; every C-ABI call takes its
// mutex, so concurrent callers (ctypes releases the GIL) are serialised.
#pragma once

#include <hip/hip_runtime.h>

#include <mutex>
#include <string>
#include <vector>

#include "qwen_layout.h"

namespace qwen {


struct HipError {
  hipError_t code;
  const char* what;
};

// Message of the last failure on the calling thread (qwen_hip_last_error).
void set_last_error(const std::string& msg);
const char* last_error_cstr();

// Throws HipError on failure; the C-ABI boundary turns it into status QWEN_ERR_DEVICE.
void hip_check(hipError_t e, const char* what);
#define QWEN_HIP(expr) ::qwen::hip_check((expr), #expr)

// Device pointers of one layer's parameters (the 19 segments of the layer block).
struct DevLayer {
  const uint8_t *qw, *kw, *vw, *ow, *gw, *uw, *dw;
  const float *ln, *post_ln, *qb, *kb, *vb, *qs, *ks, *vs, *os, *gs, *us, *ds;
};

// Host pointers of one layer's parameters, as the reference resolves them.
struct HostLayer {
  const uint8_t *qw, *kw, *vw, *ow, *gw, *uw, *dw;
  const float *ln, *post_ln, *qb, *kb, *vb, *qs, *ks, *vs, *os, *gs, *us, *ds;
};

// Pointer resolution of qwen_decode_top_wrapper.cpp:14-26,40-72 / qwen_prefill_top_core.cpp:
// weights at base + byte offset, fp32 segments at base + byte_offset/4 (integer division).
HostLayer resolve_host_layer(const uint8_t* weight_ddr, const float* scale_ddr, uint64_t w_base, uint64_t s_base);

// Bump allocator over one growable device buffer, reset at the start of every C-ABI call.
class Arena {
 public:
  void reset() { used_ = 0; }
  // Bytes handed out so far, and a return to such a mark (later allocations reuse the space).
  size_t mark() const { return used_; }
  void rewind(size_t mark) { used_ = mark < used_ ? mark : used_; }
  // Reserve capacity before any pointer of this call is handed out (growing frees the old block).
  void reserve(size_t bytes);
  void* alloc(size_t bytes);
  template <class T>
  T* alloc_n(size_t n) {
    return static_cast<T*>(alloc(n * sizeof(T)));
  }
  ~Arena();

 private:
  char* base_ = nullptr;
  size_t cap_ = 0;
  size_t used_ = 0;
};

class Runtime {
 public:
  static Runtime& get();
  std::mutex mu;
  hipStream_t stream = nullptr;
  Arena arena;

  // Prefill RoPE table [positions][cos 64 | sin 64] on the device, extended on demand.
  const float* prefill_rope(int positions);
  // Decode RoPE table (host libm, qwen_decode_attention_kernel.cpp:29-42) for every position up
  // to `positions`, on the device, extended on demand.
  const float* decode_rope(int positions);

 private:
  Runtime();
  float* prefill_rope_ = nullptr;
  int prefill_rope_rows_ = 0;
  float* decode_rope_ = nullptr;
  int decode_rope_rows_ = 0;
};

// Host computation of the decode RoPE row of one position: cos[64] then sin[64].
void decode_rope_row_host(int position, float* out128);

// Copies `n` elements host -> device arena buffer (synchronous with respect to the host).
template <class T>
T* stage_in(Arena& a, const T* host, size_t n, hipStream_t st) {
  T* d = a.alloc_n<T>(n);
  if (n) QWEN_HIP(hipMemcpyAsync(d, host, n * sizeof(T), hipMemcpyHostToDevice, st));
  return d;
}

template <class T>
void copy_out(T* host, const T* dev, size_t n, hipStream_t st) {
  if (n) QWEN_HIP(hipMemcpyAsync(host, dev, n * sizeof(T), hipMemcpyDeviceToHost, st));
}

// Stages all 19 segments of a layer into the arena.
DevLayer stage_layer(Arena& a, const HostLayer& h, hipStream_t st);

// Bytes of arena a staged layer needs (weights + fp32 segments, with alignment slack).
size_t staged_layer_bytes();

// ---- per-layer executors (device pointers; all work queued on `st`) ----
struct DecodeBatch {
  int tokens;              // independent sequences, one new token each
  const int* pos;          // device [tokens]: position (= past length) of each token
  const float* rope;       // device rope rows
  bool rope_per_token;     // true: rope row b belongs to token b; false: indexed by position
  float* k_cache;          // device; sequence b at k_cache + b*cache_stride
  float* v_cache;
  size_t cache_stride;     // floats between sequences
  int max_keys;            // cache rows per sequence the caller sized (key counts are clamped to it)
};

// Arena bytes the executors below need for `tokens` tokens.
size_t decode_workspace_bytes(int tokens);
size_t prefill_workspace_bytes(int tokens);

void run_decode_attention(const DevLayer& L, const float* x, const DecodeBatch& b, float* att, Arena& a,
                          hipStream_t st);
void run_decode_mlp(const DevLayer& L, const float* att, int tokens, float* out, Arena& a, hipStream_t st);

// The same executors over caller-provided intermediates (device memory of `tokens` rows each):
// attention xn, q [tokens][1536], k, v [tokens][256], ctx [tokens][1536]; MLP pn [tokens][1536],
// g, u, s [tokens][8960].
struct DecodeWorkspace {
  float *xn, *q, *k, *v, *ctx, *pn, *g, *u, *s;
};
// Floats of a DecodeWorkspace of `tokens` rows, and its carve-up of `base` (each part 64-float aligned).
size_t decode_workspace_floats(int tokens);
DecodeWorkspace carve_decode_workspace(float* base, int tokens);
void run_decode_attention_ws(const DevLayer& L, const float* x, const DecodeBatch& b, float* att,
                             const DecodeWorkspace& w, hipStream_t st);
void run_decode_mlp_ws(const DevLayer& L, const float* att, int tokens, float* out, const DecodeWorkspace& w,
                       hipStream_t st);
// Prefill attention of `tokens` new tokens at positions past..past+tokens-1 of one sequence whose cache
// rows start at k_rows / v_rows (rows 0..past-1 hold the earlier tokens; the new rows are written).
void run_prefill_attention(const DevLayer& L, const float* x, int tokens, int past, const float* rope, float* k_rows,
                           float* v_rows, float* att, Arena& a, hipStream_t st);
void run_prefill_mlp(const DevLayer& L, const float* att, int tokens, float* out, Arena& a, hipStream_t st);

}  // namespace qwen
