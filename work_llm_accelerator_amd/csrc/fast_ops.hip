// Operator-level entry points of the FAST path (include/qwen_hip_ops.h): the two-limb activation
// code and one INT4 x int8 matrix-core projection, on the same kernels the FAST layers launch.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <exception>
#include <string>

#include "kernels.hpp"
#include "qwen_hip_ops.h"
#include "runtime.hpp"

using namespace qwen;

namespace {

int op_invalid(const char* why) {
  set_last_error(why);
  return QWEN_ERR_KERNEL;
}

template <class Fn>
int guarded_op(Fn&& fn) {
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

// Device buffer freed when the scope ends (after the caller synchronized the stream).
struct ScopedDev {
  void* p = nullptr;
  explicit ScopedDev(size_t bytes) { QWEN_HIP(hipMalloc(&p, bytes)); }
  ~ScopedDev() {
    if (p) (void)hipFree(p);
  }
  template <class T>
  T* as() const {
    return static_cast<T*>(p);
  }
};

}  // namespace

extern "C" {

int qwen_hip_fast_quantize_rows(const float* x, int rows, int n, int8_t* xq, float* sx, int32_t* sums, void* stream) {
  if (!x || !xq || !sx || !sums || rows <= 0 || n <= 0 || n % kKChunk != 0 || n > kMaxQuantRow)
    return op_invalid("invalid quantize arguments (n a multiple of 128, at most 8960)");
  return guarded_op([&]() -> int {
    launch_norm_quant(x, (size_t)n, rows, n, nullptr, kNormNone, xq, sx, reinterpret_cast<int*>(sums), nullptr,
                      static_cast<hipStream_t>(stream));
    QWEN_HIP(hipGetLastError());
    return QWEN_OK;
  });
}

int qwen_hip_fast_project(const uint8_t* w, const float* sw, const float* bias, int out_dim, int in_dim,
                          const float* x, int tokens, int flags, float* y, void* stream) {
  if (!w || !sw || !x || !y || out_dim <= 0 || out_dim % 16 != 0 || in_dim <= 0 || in_dim % kKChunk != 0 ||
      in_dim > kMaxQuantRow || tokens <= 0 || (flags & ~QWEN_PROJECT_NO_SPLITK) != 0)
    return op_invalid("invalid projection arguments (out_dim % 16, in_dim % 128 and <= 8960, tokens > 0)");
  return guarded_op([&]() -> int {
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const bool splitk = (flags & QWEN_PROJECT_NO_SPLITK) == 0;
    ScopedDev wp((size_t)out_dim * in_dim / 2);
    ScopedDev xq(xq_bytes((size_t)tokens, (size_t)in_dim));
    ScopedDev sx((size_t)tokens * 4u);
    ScopedDev sums((size_t)tokens * 8u);
    ScopedDev part(splitk ? splitk_bytes((size_t)out_dim) : 256u);
    launch_repack_int4(w, out_dim, in_dim, wp.as<uint8_t>(), st);
    launch_norm_quant(x, (size_t)in_dim, tokens, in_dim, nullptr, kNormNone, xq.as<int8_t>(), sx.as<float>(),
                      sums.as<int>(), nullptr, st);
    GemmArgs a{};
    a.wp = wp.as<uint8_t>();
    a.sw = sw;
    a.bias = bias;
    a.xq = xq.as<int8_t>();
    a.sx = sx.as<float>();
    a.sums = sums.as<int>();
    a.tokens = tokens;
    a.in_dim = in_dim;
    a.out_dim = out_dim;
    a.y = y;
    a.y_stride = (size_t)out_dim;
    a.part = splitk ? part.as<float>() : nullptr;
    a.fuse = kFuseNone;
    launch_gemm_i8(a, kEpiStore, st);
    QWEN_HIP(hipGetLastError());
    QWEN_HIP(hipStreamSynchronize(st));
    return QWEN_OK;
  });
}

int qwen_hip_fast_silu_mul_grouped(const uint8_t* gate, const float* sw_gate, const uint8_t* up, const float* sw_up,
                                   const float* x, int tokens, float* y, int8_t* xq, float* gsx, int32_t* gcorr,
                                   void* stream) {
  if (!gate || !sw_gate || !up || !sw_up || !x || !y || !xq || !gsx || !gcorr || tokens < 1 || tokens > kSkinnyTokens)
    return op_invalid("invalid grouped SiLU·up arguments (1 to 64 tokens)");
  return guarded_op([&]() -> int {
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const int in = QWEN_HIDDEN, out = QWEN_INTERMEDIATE;
    ScopedDev wg((size_t)out * in / 2), wu((size_t)out * in / 2);
    ScopedDev xc(xq_bytes((size_t)tokens, (size_t)in));
    ScopedDev sx((size_t)tokens * 4u);
    ScopedDev sums((size_t)tokens * 8u);
    launch_repack_int4(gate, out, in, wg.as<uint8_t>(), st);
    launch_repack_int4(up, out, in, wu.as<uint8_t>(), st);
    launch_norm_quant(x, (size_t)in, tokens, in, nullptr, kNormNone, xc.as<int8_t>(), sx.as<float>(), sums.as<int>(),
                      nullptr, st);
    GemmArgs a{};
    a.wp = wg.as<uint8_t>();
    a.wp2 = wu.as<uint8_t>();
    a.sw = sw_gate;
    a.sw2 = sw_up;
    a.xq = xc.as<int8_t>();
    a.sx = sx.as<float>();
    a.sums = sums.as<int>();
    a.tokens = tokens;
    a.in_dim = in;
    a.out_dim = out;
    a.y = y;
    a.y_stride = (size_t)out;
    a.fuse = kFuseNone;
    launch_gemm_i8(a, kEpiSiluMul, st);  // fp32 SiLU(gate)·up
    a.xq_out = xq;
    a.gsx_out = gsx;
    a.gcorr_out = reinterpret_cast<int*>(gcorr);
    launch_gemm_i8(a, kEpiSiluMul, st);  // the grouped code of the same values
    QWEN_HIP(hipGetLastError());
    QWEN_HIP(hipStreamSynchronize(st));
    return QWEN_OK;
  });
}

int qwen_hip_fast_project_grouped(const uint8_t* w, const float* sw, int out_dim, const int8_t* xq, const float* gsx,
                                  const int32_t* gcorr, int tokens, float* y, void* stream) {
  if (!w || !sw || !xq || !gsx || !gcorr || !y || out_dim <= 0 || out_dim % 64 != 0 || tokens < 1 ||
      tokens > kSkinnyTokens)
    return op_invalid("invalid grouped projection arguments (out_dim % 64, 1 to 64 tokens)");
  return guarded_op([&]() -> int {
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const int in = QWEN_INTERMEDIATE;
    ScopedDev wp((size_t)out_dim * in / 2);
    ScopedDev zero((size_t)tokens * 8u);  // limb sums of a code whose offsets are applied per group
    ScopedDev part(splitk_bytes((size_t)out_dim));
    launch_repack_int4(w, out_dim, in, wp.as<uint8_t>(), st);
    launch_zero_u32(zero.as<unsigned>(), 2 * tokens, st);
    GemmArgs a{};
    a.wp = wp.as<uint8_t>();
    a.sw = sw;
    a.xq = xq;
    a.sx = gsx;  // any finite per-token value: multiplied by the zero sums
    a.sums = zero.as<int>();
    a.gsx = gsx;
    a.gcorr = reinterpret_cast<const int*>(gcorr);
    a.tokens = tokens;
    a.in_dim = in;
    a.out_dim = out_dim;
    a.y = y;
    a.y_stride = (size_t)out_dim;
    a.part = part.as<float>();
    a.fuse = kFuseNone;
    launch_gemm_i8(a, kEpiStore, st);
    QWEN_HIP(hipGetLastError());
    QWEN_HIP(hipStreamSynchronize(st));
    return QWEN_OK;
  });
}

}  // extern "C"
