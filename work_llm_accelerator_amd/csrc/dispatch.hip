// Device-resident layer dispatch over the global DDR map (include/qwen_hip_dispatch.h): the
// reference's descriptor loops (qwen_decode_top_wrapper.cpp:115-130, qwen_prefill_top_wrapper.cpp:
// 20-35) with every DDR port a device pointer, so no layer image crosses PCIe.  Each layer runs the
// ORDERED executors (bit-exact with the reference host library) on the caller's stream.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <exception>
#include <mutex>
#include <string>
#include <vector>
#include <stdexcept>

#include "kernels.hpp"
#include "qwen_hip_dispatch.h"
#include "runtime.hpp"
#include "tops.hpp"

using namespace qwen;

// ---------------------------------------------------------------------------------------------
// Scratch of the allocation-free decode dispatch: one token's intermediates (decode_workspace_floats(1))
// plus the RoPE row and position of the descriptor being run.  One copy per GPU, held until the
// process ends; host code reaches it only through the address hipGetSymbolAddress returns for the
// current device (the array's name is a host-side stand-in, not a device address).
// ---------------------------------------------------------------------------------------------
constexpr size_t kNoAllocWorkspaceFloats = 35072;  // decode_workspace_floats(1)
constexpr size_t kNoAllocAttOffset = kNoAllocWorkspaceFloats;             // attention output row
constexpr size_t kNoAllocRopeOffset = kNoAllocAttOffset + QWEN_HIDDEN;    // cos[64] | sin[64]
constexpr size_t kNoAllocPosOffset = kNoAllocRopeOffset + QWEN_HEAD_DIM;  // the position (an int)
constexpr size_t kNoAllocScratchFloats = 36864;                          // 147,456 bytes in all
static_assert(kNoAllocPosOffset < kNoAllocScratchFloats, "scratch layout");
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

namespace {

struct RopeRowArg {
  float cs[128];  // cos[64] then sin[64] of one position (host libm, qwen_decode_attention_kernel.cpp:29-42)
};

// Writes the descriptor's RoPE row and position into the scratch (kernel arguments, so nothing is
// copied from host memory and nothing is allocated).  One block of 128 threads.
__global__ void __launch_bounds__(128) stage_rope_row_kernel(float* __restrict__ rope, int* __restrict__ pos,
                                                              RopeRowArg row, int position) {
  rope[threadIdx.x] = row.cs[threadIdx.x];
  if (threadIdx.x == 0) *pos = position;
}

template <class Fn>
int guarded_dispatch(Fn&& fn) {
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

// Device pointers of one layer at (w_base, s_base) of the global images (the pointer resolution of
// qwen_decode_top_wrapper.cpp:40-72 / qwen_prefill_top_core.cpp:100-135).
DevLayer device_layer(const uint8_t* wd, const float* sd, uint64_t w_base, uint64_t s_base) {
  const HostLayer h = resolve_host_layer(wd, sd, w_base, s_base);
  return DevLayer{h.qw, h.kw, h.vw, h.ow, h.gw, h.uw, h.dw, h.ln, h.post_ln, h.qb, h.kb,
                  h.vb, h.qs, h.ks, h.vs, h.os, h.gs, h.us, h.ds};
}

void set_completed(int* completed, int n) {
  if (completed) *completed = n;
}

// Device address of `scratch` on the current device, looked up once per device.
float* noalloc_scratch() {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static float* addr[kMaxDevices] = {};
  int dev = 0;
  QWEN_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) throw std::runtime_error("device index beyond the scratch table");
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void* p = nullptr;
    QWEN_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    addr[dev] = static_cast<float*>(p);
  }
  return addr[dev];
}

}  // namespace

extern "C" {

int qwen_hip_decode_dispatch_layers(const qwen_decode_descriptor* dsc, int n, const uint8_t* wd, const float* sd,
                                    float* kv, float* act, void* stream, int* completed) {
  set_completed(completed, 0);
  if (!dsc || n <= 0) return QWEN_ERR_DECODE_DESC;  // qwen_decode_top_wrapper.cpp:118-120
  Runtime& rt = Runtime::get();
  std::lock_guard<std::mutex> lock(rt.mu);
  return guarded_dispatch([&]() -> int {
    const hipStream_t st = static_cast<hipStream_t>(stream);
    // Every runnable descriptor's position and RoPE row (host libm, qwen_decode_attention_kernel.cpp:29-42,
    // as the drop-in top wrapper and the allocation-free entry build them: no table, so no bound on the
    // position) staged before the first launch; the arena is sized once (growing it would free memory that
    // queued layers still read), and the layers' intermediates then reuse one workspace in stream order.
    int runnable = 0;
    while (runnable < n && decode_descriptor_status(dsc[runnable]) == QWEN_OK) ++runnable;
    const size_t rows = runnable > 0 ? (size_t)runnable : 1u;
    rt.arena.reset();
    rt.arena.reserve(decode_workspace_bytes(1) + 4u * QWEN_HIDDEN + 4u * rows + 512u * rows + 8192u);
    std::vector<int> pasts(rows, 0);
    std::vector<float> rope_rows(rows * 128u, 0.0f);
    for (int i = 0; i < runnable; ++i) {
      pasts[i] = dsc[i].past_seq_len;
      decode_rope_row_host(dsc[i].past_seq_len, &rope_rows[(size_t)i * 128u]);
    }
    const int* pos_all = stage_in(rt.arena, pasts.data(), rows, st);
    const float* rope_all = stage_in(rt.arena, rope_rows.data(), rope_rows.size(), st);
    float* att = rt.arena.alloc_n<float>(QWEN_HIDDEN);
    const size_t layer_mark = rt.arena.mark();
    int status = QWEN_OK, done = 0;
    for (; done < n; ++done) {
      const qwen_decode_descriptor& d = dsc[done];
      if ((status = decode_descriptor_status(d)) != QWEN_OK) break;
      if (!wd || !sd || !kv || !act) {
        status = QWEN_ERR_DECODE_PORT;
        break;
      }
      const int past = d.past_seq_len;
      rt.arena.rewind(layer_mark);
      const int* pos_d = pos_all + done;
      const DevLayer L = device_layer(wd, sd, d.layer_weights_base_addr, d.layer_scales_base_addr);
      DecodeBatch b{1, pos_d, rope_all + (size_t)done * 128u, true, kv + d.k_cache_base_addr / 4,
                    kv + d.v_cache_base_addr / 4, 0, past + 1};
      run_decode_attention(L, act + d.input_token_addr / 4, b, att, rt.arena, st);
      run_decode_mlp(L, att, 1, act + d.output_token_addr / 4, rt.arena, st);
    }
    QWEN_HIP(hipStreamSynchronize(st));
    rt.arena.reset();
    set_completed(completed, done);
    return status;
  });
}

int qwen_hip_prefill_dispatch_layers(const qwen_prefill_descriptor* dsc, int n, const uint8_t* wd, const float* sd,
                                     float* kv, float* act, void* stream, int* completed) {
  set_completed(completed, 0);
  if (!dsc || n <= 0) return QWEN_ERR_PREFILL_DESC;  // qwen_prefill_top_wrapper.cpp:23-25
  Runtime& rt = Runtime::get();
  std::lock_guard<std::mutex> lock(rt.mu);
  return guarded_dispatch([&]() -> int {
    const hipStream_t st = static_cast<hipStream_t>(stream);
    // a valid descriptor has at most QWEN_PREFILL_CAPACITY tokens: RoPE rows and arena sized once
    const float* rope = rt.prefill_rope(QWEN_PREFILL_CAPACITY);
    rt.arena.reset();
    rt.arena.reserve(prefill_workspace_bytes(QWEN_PREFILL_CAPACITY) + 4096u);
    int status = QWEN_OK, done = 0;
    for (; done < n; ++done) {
      const qwen_prefill_descriptor& d = dsc[done];
      int mlp_status = QWEN_OK;
      if ((status = prefill_top_status(d, !wd || !sd || !kv || !act, &mlp_status)) != QWEN_OK) break;
      const int S = d.seq_len;
      rt.arena.reset();  // reused in stream order by every layer
      const DevLayer L = device_layer(wd, sd, d.layer_weights_base_addr, d.layer_scales_base_addr);
      float* scratch = act + d.scratch_base_addr / 4;  // attention output (qwen_prefill_top_core.cpp:103,155)
      run_prefill_attention(L, act + d.input_sequence_addr / 4, S, 0, rope, kv + d.k_cache_base_addr / 4,
                            kv + d.v_cache_base_addr / 4, scratch, rt.arena, st);
      if ((status = mlp_status) != QWEN_OK) break;  // the attention side effects stay, as in the reference
      run_prefill_mlp(L, scratch, S, act + d.output_sequence_addr / 4, rt.arena, st);
    }
    QWEN_HIP(hipStreamSynchronize(st));
    rt.arena.reset();
    set_completed(completed, done);
    return status;
  });
}

int qwen_hip_decode_dispatch_layers_noalloc(const qwen_decode_descriptor* dsc, int n, const uint8_t* wd,
                                            const float* sd, float* kv, float* act, void* stream, int* completed) {
  set_completed(completed, 0);
  if (!dsc || n <= 0) return QWEN_ERR_DECODE_DESC;  // qwen_decode_top_wrapper.cpp:118-120
  return guarded_dispatch([&]() -> int {
    if (decode_workspace_floats(1) > kNoAllocWorkspaceFloats)
      throw std::runtime_error("one token's decode workspace exceeds the static scratch");
    const hipStream_t st = static_cast<hipStream_t>(stream);
    float* base = noalloc_scratch();
    const DecodeWorkspace w = carve_decode_workspace(base, 1);
    float* att = base + kNoAllocAttOffset;
    float* rope = base + kNoAllocRopeOffset;
    int* pos = reinterpret_cast<int*>(base + kNoAllocPosOffset);
    int status = QWEN_OK, done = 0;
    for (; done < n; ++done) {
      const qwen_decode_descriptor& d = dsc[done];
      if ((status = decode_descriptor_status(d)) != QWEN_OK) break;
      if (!wd || !sd || !kv || !act) {
        status = QWEN_ERR_DECODE_PORT;
        break;
      }
      // every layer reuses the scratch in stream order: its RoPE row and position are written by a kernel
      // queued before its own kernels, after the previous layer's
      RopeRowArg row;
      decode_rope_row_host(d.past_seq_len, row.cs);
      hipLaunchKernelGGL(stage_rope_row_kernel, dim3(1), dim3(128), 0, st, rope, pos, row, d.past_seq_len);
      const DevLayer L = device_layer(wd, sd, d.layer_weights_base_addr, d.layer_scales_base_addr);
      DecodeBatch b{1, pos, rope, true, kv + d.k_cache_base_addr / 4, kv + d.v_cache_base_addr / 4, 0,
                    d.past_seq_len + 1};
      run_decode_attention_ws(L, act + d.input_token_addr / 4, b, att, w, st);
      run_decode_mlp_ws(L, att, 1, act + d.output_token_addr / 4, w, st);
    }
    QWEN_HIP(hipGetLastError());
    set_completed(completed, done);
    return status;
  });
}

}  // extern "C"
