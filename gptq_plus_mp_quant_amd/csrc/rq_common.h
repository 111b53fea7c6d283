// Shared definitions for the gfx950 GPTQ+ hot-path kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <stdint.h>

#include <mutex>

#include "../../include/gptqplus_hip.h"

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef double doublex4 __attribute__((ext_vector_type(4)));

#define RQ_CHECK_LAUNCH()                                   \
  do {                                                      \
    if (hipGetLastError() != hipSuccess) return RQ_EHIP;    \
  } while (0)

// A second stream of the current device for work that overlaps the caller's stream: forked
// from it and joined back through the two events.  Created on first use (non-blocking,
// default priority) and kept until the process ends.  An entry point that uses it holds
// `lock` for the whole call, so calls from several host threads on one device enqueue their
// fork / join pairs one call at a time.
struct RqSide {
  hipStream_t s;
  hipEvent_t fork, join;
};
inline int rq_side_stream(RqSide** out, std::unique_lock<std::mutex>& lock) {
  constexpr int MAXDEV = 64;
  static std::mutex mu[MAXDEV];
  static RqSide side[MAXDEV];
  static bool made[MAXDEV];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAXDEV) return RQ_EHIP;
  lock = std::unique_lock<std::mutex>(mu[dev]);
  if (!made[dev]) {
    if (hipStreamCreateWithFlags(&side[dev].s, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&side[dev].fork, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&side[dev].join, hipEventDisableTiming) != hipSuccess)
      return RQ_EHIP;
    made[dev] = true;
  }
  *out = &side[dev];
  return RQ_OK;
}

// Makes `s` wait for the last work queued on the side stream when it goes out of scope (every
// return path of an entry point that forked work there, errors included), so the caller's
// buffers outlive that work.
struct RqSideJoin {
  RqSide* sd = nullptr;
  hipStream_t s = nullptr;
  bool busy = false;
  ~RqSideJoin() {
    if (busy) (void)hipStreamWaitEvent(s, sd->join, 0);
  }
};

// Workgroup barrier for the direct-to-LDS staging rings: the stage a ring refills after the
// barrier was read before it, so every wave first waits for its own LDS reads to complete
// (lgkmcnt(0): a read only issued before the barrier could otherwise still be pending when
// another wave's direct-to-LDS load lands on the same bytes), then s_barrier, with no wait on
// the vector-memory counter (the loads of later stages stay in flight).  A compiler memory
// barrier on both sides keeps the LDS accesses of a stage on their side of the barrier (the
// builtins alone do not order memory accesses for the compiler).
#define RQ_STAGE_BARRIER()                                                              \
  do {                                                                                  \
    asm volatile("" ::: "memory");                                                      \
    __builtin_amdgcn_s_waitcnt(0xC07F); /* lgkmcnt(0); vmcnt, expcnt not limited */    \
    __builtin_amdgcn_s_barrier();                                                       \
    asm volatile("" ::: "memory");                                                      \
  } while (0)

__device__ __forceinline__ float rq_load_elem(const __half* p) { return __half2float(*p); }
__device__ __forceinline__ float rq_load_elem(const __hip_bfloat16* p) { return __bfloat162float(*p); }
__device__ __forceinline__ float rq_load_elem(const float* p) { return *p; }

// int16 code written for a NaN weight (the reference keeps NaN in its float codes).
constexpr int16_t RQ_CODE_NAN = -32768;

// torch.minimum / torch.maximum semantics: NaN propagates.
__device__ __forceinline__ float rq_nan_min(float a, float b) { return (a != a || a < b) ? a : b; }
__device__ __forceinline__ float rq_nan_max(float a, float b) { return (a != a || a > b) ? a : b; }
// torch.clamp(x, min=lo): NaN stays NaN.
__device__ __forceinline__ float rq_clamp_min(float x, float lo) { return (x < lo) ? lo : x; }

// One element of WeightQuantizer.fake_quantize (utils/quant_utils.py:471-480):
// code = clamp(round_half_even(x / scale), -(maxq+1), maxq); q = scale * code.
// Division is IEEE correctly rounded (hipcc default), no contraction (-ffp-contract=off).
__device__ __forceinline__ float rq_quant_code(float x, float scale, float lo, float hi) {
  float r = __builtin_rintf(x / scale);
  // torch.clamp: NaN propagates; otherwise min/max.
  r = (r < lo) ? lo : r;
  r = (r > hi) ? hi : r;
  return r;
}

// WeightQuantizer.find_params per-channel branch (utils/quant_utils.py:408-421) for one row,
// given the row's NaN-propagating min and max; clip_zero = 0: find_params_weight_groupwise
// (:333-352), whose range is the group's min / max as they are (not widened to include 0).
__device__ __forceinline__ void rq_params_from_minmax(float rmin, float rmax, float maxq, int sym,
                                                      float* scale_out, float* zero_out, int clip_zero = 1) {
  float xmin = clip_zero ? rq_nan_min(rmin, 0.0f) : rmin;
  float xmax = clip_zero ? rq_nan_max(rmax, 0.0f) : rmax;
  if (sym) {
    float m = rq_nan_max(fabsf(xmin), xmax);
    *scale_out = rq_clamp_min(m, 1e-5f) / maxq;
    *zero_out = 0.0f;
  } else {
    if (xmin == 0.0f && xmax == 0.0f) {
      xmin = -1.0f;
      xmax = 1.0f;
    }
    float s = rq_clamp_min(xmax - xmin, 1e-5f) / maxq;
    *scale_out = s;
    *zero_out = __builtin_rintf(-xmin / s);
  }
}

__device__ __forceinline__ int rq_isfinite(float x) { return (x == x) && (fabsf(x) <= 3.402823466e38f); }
__device__ __forceinline__ int rq_isfinite(double x) { return (x == x) && (fabs(x) <= 1.7976931348623157e308); }

// fp32 -> output dtype, round to nearest even (torch's .to(dtype))
template <typename TQ>
__device__ __forceinline__ TQ rq_cast(float v);
template <>
__device__ __forceinline__ __half rq_cast<__half>(float v) { return __float2half_rn(v); }
template <>
__device__ __forceinline__ __hip_bfloat16 rq_cast<__hip_bfloat16>(float v) { return __float2bfloat16(v); }
template <>
__device__ __forceinline__ float rq_cast<float>(float v) { return v; }
