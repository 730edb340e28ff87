// Shared device helpers for the gfx950 KernelIR kernels.
//
// Element types travel through the C ABI as raw 16-bit or 32-bit storage and a
// dtype tag (slc_dtype in include/slc_hip.h).  Conversions are written out here
// so every kernel rounds exactly the same way PyTorch does: float -> bf16 is
// round-to-nearest-even with NaN kept quiet, float -> fp16 uses the hardware
// RNE conversion.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "slc_hip.h"

namespace slc {

struct bf16_t {
  uint16_t bits;
};
struct f16_t {
  uint16_t bits;
};

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16_t x) {
  return __uint_as_float(static_cast<uint32_t>(x.bits) << 16);
}
__device__ __forceinline__ float to_f32(f16_t x) {
  _Float16 h = __builtin_bit_cast(_Float16, x.bits);
  return static_cast<float>(h);
}

// float -> bf16, round to nearest even (v_cvt_pk_bf16_f32 on gfx950; NaN stays
// NaN), the same rounding PyTorch applies.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

template <typename T>
__device__ __forceinline__ T from_f32(float f);
template <>
__device__ __forceinline__ float from_f32<float>(float f) {
  return f;
}
template <>
__device__ __forceinline__ bf16_t from_f32<bf16_t>(float f) {
  return bf16_t{f32_to_bf16_bits(f)};
}
template <>
__device__ __forceinline__ f16_t from_f32<f16_t>(float f) {
  _Float16 h = static_cast<_Float16>(f);
  return f16_t{__builtin_bit_cast(uint16_t, h)};
}

// Round a float to the precision of T and return it as float again.  This is
// the "materialise in dtype" step PyTorch performs between two bf16 ops.
template <typename T>
__device__ __forceinline__ float round_to(float f) {
  return to_f32(from_f32<T>(f));
}

// Wavefront-wide reductions (wave64).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) {
    v += __shfl_xor(v, offset, 64);
  }
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) {
    v = fmaxf(v, __shfl_xor(v, offset, 64));
  }
  return v;
}

__device__ __forceinline__ float load_as_f32(const void* base, int64_t index,
                                             int dtype) {
  if (dtype == SLC_F32) return static_cast<const float*>(base)[index];
  if (dtype == SLC_BF16) return to_f32(static_cast<const bf16_t*>(base)[index]);
  return to_f32(static_cast<const f16_t*>(base)[index]);
}

__device__ __forceinline__ int slc_dtype_bytes(int dtype) {
  return dtype == SLC_F32 ? 4 : 2;
}

__device__ __forceinline__ int64_t load_length(const void* lengths, int64_t b,
                                               int dtype) {
  if (dtype == SLC_I64) return static_cast<const int64_t*>(lengths)[b];
  return static_cast<int64_t>(static_cast<const int32_t*>(lengths)[b]);
}

// Max of x over lanes l and l ^ 16 (and l ^ 32): the gfx950 lane-swap
// instructions exchange rows of 16 (halves of 32) between two registers in the
// VALU, where __shfl_xor goes through LDS (ds_bpermute) and its latency.  With
// x in both operands the two results hold x of each pair of lanes.
__device__ __forceinline__ float max_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

}  // namespace slc

// Host-side helpers shared by the C entry points.
namespace slc_host {

void set_error(const char* fmt, ...);
int check_launch(const char* what);

// Compute units of the current device (cached per device; 256 if the query
// fails).
int device_cu_count();

// Measurement hook: when the caller armed a pair of events on this thread
// (slc_hip_set_timing_events), the entry point brackets its dominant kernel
// with them on the launch stream.  Both are no-ops otherwise.
void mark_kernel_begin(hipStream_t stream);
void mark_kernel_end(hipStream_t stream);
// Launches of the dominant kernel between the two events: the armed repeat
// count (slc_hip_set_timing_repeats) while events are armed, else 1.  The
// kernel must be idempotent for its inputs (it only rewrites its outputs).
int timed_repeats();



inline int dtype_size(int dtype) {
  switch (dtype) {
    case SLC_F32:
      return 4;
    case SLC_F16:
    case SLC_BF16:
      return 2;
    case SLC_I32:
      return 4;
    case SLC_I64:
      return 8;
    default:
      return 0;
  }
}

inline bool is_float_dtype(int dtype) {
  return dtype == SLC_F32 || dtype == SLC_F16 || dtype == SLC_BF16;
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Decode-sized linear shared by slc_hip_linear and the fused decode ops
// (defined with those kernels).
// Prefill-sized linear + residual add (linear.hip); SLC_ERR_UNSUPPORTED when
// its kernel does not take the shape.
int gemm_residual(const void* x, int64_t x_rs, int64_t rows, int64_t K, int64_t N,
                  const void* w, const void* bias, const void* residual, int64_t r_rs, void* y,
                  int64_t y_rs, int dtype, hipStream_t stream);
bool rows_linear_eligible(const void* x, int64_t x_rs, int64_t rows, int64_t K, int64_t N,
                          int dtype);
int rows_linear(const void* x, int64_t x_rs, int64_t rows, int64_t K, int64_t N,
                const void* w, const void* bias, void* y, int64_t y_rs, int dtype,
                hipStream_t stream);

}  // namespace slc_host

#define SLC_REQUIRE(cond, ...)          \
  do {                                  \
    if (!(cond)) {                      \
      slc_host::set_error(__VA_ARGS__); \
      return SLC_ERR_INVALID_ARGUMENT;  \
    }                                   \
  } while (0)
