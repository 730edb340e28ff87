// rms_norm over the last axis (serve.rms_norm).
//
// Semantics: src/stateful_llm_compiler/execution.py:674-692 (reference executor)
// and backends/triton_rmsnorm.py:22-202 (fused kernel):
//   normalized = x * rsqrt(mean(x^2) + eps)   in fp32
//   round_before_weight: out = weight * round(normalized, norm dtype)  (Qwen2)
//   otherwise:           out = round(normalized * weight, out dtype)
//
// One wavefront owns one row: the row is held in registers (16-byte loads),
// the sum of squares is a wave reduction, and the row is written back from the
// registers, so HBM sees exactly one read and one write of every element.
// Rows that do not fit the register plan, or mixed dtypes, use a one-block-
// per-row kernel that re-reads the row (from L2) for the second pass; a
// profile-guided plan may also pick it for few rows, where four waves per row
// shorten the latency of each row.
#include "common.hpp"
#include "op_math.hpp"

namespace {

template <typename T>
struct Vec16 {
  static constexpr int N = 16 / sizeof(T);
};

template <typename T, int NV, bool ROUND>
__global__ __launch_bounds__(256) void rms_norm_wave_kernel(
    const T* __restrict__ x, const T* __restrict__ w, T* __restrict__ y,
    int64_t rows, int hidden, int64_t x_rs, int64_t y_rs, float eps) {
  constexpr int VEC = Vec16<T>::N;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const int nvec = hidden / VEC;
  uint4 out[NV];
  slc::rms_norm_row<T, NV, ROUND>(x + row * x_rs, w, hidden, eps, lane, out);
  T* yr = y + row * y_rs;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = lane + 64 * i;
    if (idx < nvec) *reinterpret_cast<uint4*>(yr + idx * VEC) = out[i];
  }
}

__device__ __forceinline__ void store_dtype(void* base, int64_t i, float v,
                                            int dtype) {
  if (dtype == SLC_F32) {
    static_cast<float*>(base)[i] = v;
  } else if (dtype == SLC_BF16) {
    static_cast<slc::bf16_t*>(base)[i] = slc::from_f32<slc::bf16_t>(v);
  } else {
    static_cast<slc::f16_t*>(base)[i] = slc::from_f32<slc::f16_t>(v);
  }
}

__device__ __forceinline__ float round_dtype(float v, int dtype) {
  if (dtype == SLC_BF16) return slc::round_to<slc::bf16_t>(v);
  if (dtype == SLC_F16) return slc::round_to<slc::f16_t>(v);
  return v;
}

__global__ __launch_bounds__(256) void rms_norm_generic_kernel(
    const void* __restrict__ x, const void* __restrict__ w, void* __restrict__ y,
    int in_dtype, int w_dtype, int out_dtype, int norm_dtype, int hidden,
    int64_t x_rs, int64_t y_rs, float eps, int round_before_weight) {
  __shared__ float partial[4];
  const int64_t row = blockIdx.x;
  float sq = 0.0f;
  for (int i = threadIdx.x; i < hidden; i += 256) {
    const float v = slc::load_as_f32(x, row * x_rs + i, in_dtype);
    sq += v * v;
  }
  sq = slc::wave_sum(sq);
  if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = sq;
  __syncthreads();
  sq = partial[0] + partial[1] + partial[2] + partial[3];
  const float inv = rsqrtf(sq / static_cast<float>(hidden) + eps);
  for (int i = threadIdx.x; i < hidden; i += 256) {
    const float n = slc::load_as_f32(x, row * x_rs + i, in_dtype) * inv;
    const float wv = slc::load_as_f32(w, i, w_dtype);
    const float out = round_before_weight ? round_dtype(n, norm_dtype) * wv : n * wv;
    store_dtype(y, row * y_rs + i, out, out_dtype);
  }
}

template <typename T, bool ROUND>
int launch_wave(const void* x, const void* w, void* y, int64_t rows,
                int64_t hidden, int64_t xs, int64_t ys, float eps,
                hipStream_t stream) {
  constexpr int VEC = Vec16<T>::N;
  const int64_t nvec = hidden / VEC;
  const dim3 grid(static_cast<unsigned>(slc_host::ceil_div(rows, 4)));
#define SLC_RMS(NV)                                                          \
  hipLaunchKernelGGL((rms_norm_wave_kernel<T, NV, ROUND>), grid, dim3(256), 0, \
                     stream, static_cast<const T*>(x),                       \
                     static_cast<const T*>(w), static_cast<T*>(y), rows,     \
                     static_cast<int>(hidden), xs, ys, eps)
  if (nvec <= 64) {
    SLC_RMS(1);
  } else if (nvec <= 128) {
    SLC_RMS(2);
  } else if (nvec <= 256) {
    SLC_RMS(4);
  } else {
    SLC_RMS(8);
  }
#undef SLC_RMS
  return slc_host::check_launch("slc_hip_rms_norm");
}

}  // namespace

extern "C" int slc_hip_rms_norm(const void* input, const void* weight,
                                void* output, int in_dtype, int weight_dtype,
                                int out_dtype, int norm_dtype, int64_t rows,
                                int64_t hidden, int64_t in_stride_row,
                                int64_t out_stride_row, float epsilon,
                                int round_before_weight, int waves_per_row,
                                void* stream) {
  SLC_REQUIRE(slc_host::is_float_dtype(in_dtype) &&
                  slc_host::is_float_dtype(weight_dtype) &&
                  slc_host::is_float_dtype(out_dtype) &&
                  slc_host::is_float_dtype(norm_dtype),
              "slc_hip_rms_norm: bad dtype");
  SLC_REQUIRE(rows >= 0 && hidden > 0 && hidden <= 65536,
              "slc_hip_rms_norm: bad sizes rows=%lld hidden=%lld",
              (long long)rows, (long long)hidden);
  if (rows == 0) return SLC_OK;
  SLC_REQUIRE(input && weight && output, "slc_hip_rms_norm: null pointer");
  SLC_REQUIRE(rows <= 0x7fffffffLL * 4, "slc_hip_rms_norm: too many rows");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool same = in_dtype == weight_dtype && in_dtype == out_dtype &&
                    in_dtype == norm_dtype;
  const int64_t es = slc_host::dtype_size(in_dtype);
  const int64_t vec = 16 / es;
  const uint64_t bits = reinterpret_cast<uintptr_t>(input) |
                        reinterpret_cast<uintptr_t>(weight) |
                        reinterpret_cast<uintptr_t>(output);
  const bool aligned = (bits & 15) == 0 && hidden % vec == 0 &&
                       in_stride_row % vec == 0 && out_stride_row % vec == 0;
  SLC_REQUIRE(waves_per_row == 0 || waves_per_row == 1 || waves_per_row == 4,
              "slc_hip_rms_norm: waves_per_row must be 0, 1 or 4, got %d", waves_per_row);
  if (waves_per_row != 4 && same && aligned && hidden / vec <= 512) {
    const bool r = round_before_weight != 0;
    switch (in_dtype) {
      case SLC_BF16:
        return r ? launch_wave<slc::bf16_t, true>(input, weight, output, rows, hidden,
                                                  in_stride_row, out_stride_row, epsilon, s)
                 : launch_wave<slc::bf16_t, false>(input, weight, output, rows, hidden,
                                                   in_stride_row, out_stride_row, epsilon, s);
      case SLC_F16:
        return r ? launch_wave<slc::f16_t, true>(input, weight, output, rows, hidden,
                                                 in_stride_row, out_stride_row, epsilon, s)
                 : launch_wave<slc::f16_t, false>(input, weight, output, rows, hidden,
                                                  in_stride_row, out_stride_row, epsilon, s);
      default:
        return launch_wave<float, false>(input, weight, output, rows, hidden,
                                         in_stride_row, out_stride_row, epsilon, s);
    }
  }
  SLC_REQUIRE(rows <= 0x7fffffff, "slc_hip_rms_norm: too many rows");
  hipLaunchKernelGGL(rms_norm_generic_kernel, dim3(static_cast<unsigned>(rows)),
                     dim3(256), 0, s, input, weight, output, in_dtype,
                     weight_dtype, out_dtype, norm_dtype,
                     static_cast<int>(hidden), in_stride_row, out_stride_row,
                     epsilon, round_before_weight);
  return slc_host::check_launch("slc_hip_rms_norm(generic)");
}
