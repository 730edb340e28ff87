// Element-level arithmetic shared by the stand-alone kernels and the fused
// decode kernels.  Keeping one definition of each is what makes a fused kernel
// bit-identical to the sequence of kernels it replaces.
#pragma once

#include "common.hpp"

namespace slc {

// One wavefront normalises one row of `hidden` elements held as 16-byte
// vectors (lane owns vectors lane, lane + 64, ...):
//   inv = rsqrt(mean(x^2) + eps) in fp32 (per-lane partial sums, then a
//   wave butterfly), out = round(round(x * inv) * w)  (round_before_weight)
//                       or round(x * inv * w).
// Semantics of src/stateful_llm_compiler/execution.py:674-692.
// The row's and the weight's 16-byte vectors of this lane (rms_norm_row's
// loads), and the normalisation from them: a kernel may request them before
// other loads and normalise later.
template <typename T, int NV>
__device__ __forceinline__ void rms_norm_load(const T* __restrict__ row, int hidden, int lane,
                                              uint4 (&raw)[NV]) {
  constexpr int VEC = 16 / sizeof(T);
  const int nvec = hidden / VEC;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = lane + 64 * i;
    raw[i] = idx < nvec ? *reinterpret_cast<const uint4*>(row + idx * VEC) : make_uint4(0, 0, 0, 0);
  }
}
template <typename T, int NV, bool ROUND>
__device__ __forceinline__ void rms_norm_from(const uint4 (&xraw)[NV], const uint4 (&wraw)[NV],
                                              int hidden, float eps, int lane, uint4 (&out)[NV]) {
  constexpr int VEC = 16 / sizeof(T);
  const int nvec = hidden / VEC;
  float v[NV][VEC];
  float sq = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = lane + 64 * i;
    if (idx < nvec) {
      const T* e = reinterpret_cast<const T*>(&xraw[i]);
#pragma unroll
      for (int k = 0; k < VEC; ++k) {
        v[i][k] = to_f32(e[k]);
        sq += v[i][k] * v[i][k];
      }
    }
  }
  sq = wave_sum(sq);
  const float inv = rsqrtf(sq / static_cast<float>(hidden) + eps);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = lane + 64 * i;
    out[i] = make_uint4(0, 0, 0, 0);
    if (idx < nvec) {
      const T* we = reinterpret_cast<const T*>(&wraw[i]);
      T* oe = reinterpret_cast<T*>(&out[i]);
#pragma unroll
      for (int k = 0; k < VEC; ++k) {
        const float n = v[i][k] * inv;
        const float wk = to_f32(we[k]);
        oe[k] = ROUND ? from_f32<T>(round_to<T>(n) * wk) : from_f32<T>(n * wk);
      }
    }
  }
}
// The weight vectors are requested with the row (they do not depend on it),
// so the sum's reduction does not wait on a second round trip.
template <typename T, int NV, bool ROUND>
__device__ __forceinline__ void rms_norm_row(const T* __restrict__ xr, const T* __restrict__ w,
                                             int hidden, float eps, int lane, uint4 (&out)[NV]) {
  uint4 wraw[NV], xraw[NV];
  rms_norm_load<T, NV>(w, hidden, lane, wraw);
  rms_norm_load<T, NV>(xr, hidden, lane, xraw);
  rms_norm_from<T, NV, ROUND>(xraw, wraw, hidden, eps, lane, out);
}

// SwiGLU of one element: round(silu(g)) * u, silu(g) = g / (1 + exp(-g)),
// with no FMA contraction (PyTorch's eager silu then multiply).
template <typename T>
__device__ __forceinline__ float swiglu_value(float g, float u) {
#pragma clang fp contract(off)
  const float s = g / (1.0f + expf(-g));
  return round_to<T>(s) * u;
}

// Qwen2 half-rotation RoPE of one dim pair (d, d + D/2):
//   o1 = round(x1 * c1) - round(x2 * s1),  o2 = round(x2 * c2) + round(x1 * s2)
// each product rounded to T before the add, as two eager multiplies and an
// add do (execution.py:741-767); rounding is sign-symmetric, so
// round(-x2 * s1) = -round(x2 * s1).
template <typename T>
__device__ __forceinline__ void rope_pair(float x1, float x2, float c1, float c2, float s1,
                                          float s2, float& o1, float& o2) {
#pragma clang fp contract(off)
  const float p1 = x1 * c1;
  const float p2 = x2 * s1;
  const float p3 = x2 * c2;
  const float p4 = x1 * s2;
  o1 = round_to<T>(p1) - round_to<T>(p2);
  o2 = round_to<T>(p3) + round_to<T>(p4);
}

}  // namespace slc
