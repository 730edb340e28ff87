// Fused decode-step kernels (fast numerical mode, decode-sized row counts).
//
// A Qwen2 decode step spends most of its time in launch latency: every layer
// is ~17 small kernels.  These kernels merge neighbours of the KernelIR op
// graph without changing a single rounding step, so each is bit-identical to
// the ops it replaces (the compiler's fusion pass swaps them in):
//
//  * norm_linear_group   rms_norm -> up to three linears reading its output
//                        (Q/K/V).  Every workgroup normalises the <= 32 input
//                        rows into LDS with the rms_norm kernel's own row
//                        routine, then streams its share of the weight rows.
//  * norm_linear_swiglu  rms_norm -> gate and up linears -> swiglu.  A
//                        workgroup owns a run of features of both projections and
//                        applies SwiGLU to the rounded results.
//  * linear_residual     linear -> residual add (O and down projections).
//  * rope_kv_store       rope -> kv_store of the rotated keys and the values;
//                        the rotated queries are written out.
//
// slc_hip_linear runs its decode-sized (<= 32 rows) cases on this same kernel
// (rows_linear), so a fused op and the ops it replaces share the K split over
// the waves, the MFMA order and the partial-sum order, hence the same bits.
// Semantics: src/stateful_llm_compiler/execution.py:674-692 (rms_norm),
// triton_executor.py:159-176 (linear), :741-767 (rope), :743-781 (kv store).

#include "common.hpp"
#include "op_math.hpp"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

template <typename T>
struct Mfma;
template <>
struct Mfma<slc::bf16_t> {
  using vec = bf16x8_t;
  static __device__ __forceinline__ f32x4_t run(vec a, vec b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mfma<slc::f16_t> {
  using vec = f16x8_t;
  static __device__ __forceinline__ f32x4_t run(vec a, vec b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
  const uint64_t address = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(address));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(address >> 32));
  void* uniform = reinterpret_cast<void*>((static_cast<uint64_t>(hi) << 32) | lo);
  const int clamped = bytes > 0x7fffffff ? 0x7fffffff : static_cast<int>(bytes);
  return __builtin_amdgcn_make_buffer_rsrc(uniform, 0, __builtin_amdgcn_readfirstlane(clamped),
                                           0x00020000);
}
__device__ __forceinline__ uint4 buffer_load16(__amdgpu_buffer_rsrc_t rsrc, int offset) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, offset, 0, 0));
}

enum Epilogue { kStore = 0, kResidual = 1, kSwiglu = 2 };

// Waves per workgroup (the K split): 16 from K = 512 (more loads in flight
// per CU: Qwen2 decode SwiGLU 8.1 against 8.9 us with 8, down projection 7.3
// against 8.0), else 8.  It depends on K alone, so the fused ops and the
// single linears they replace split K the same way.
__host__ __device__ constexpr int waves_for(int k) { return k >= 512 ? 16 : 8; }
constexpr int kMaxRows = 32;     // rows (batch x tokens) the fused kernels take
constexpr int kMaxMatrices = 3;

struct FusedArgs {
  const void* x;          // [rows, hidden] input (before the norm when norm_w)
  int64_t x_rs;
  const void* norm_w;     // [hidden] or null
  float eps;
  int rows, hidden;
  const void* w[kMaxMatrices];     // [n_j, hidden] row-major
  const void* bias[kMaxMatrices];  // [n_j] or null
  void* y[kMaxMatrices];           // [rows, n_j] with row stride y_rs_j
  int n[kMaxMatrices];
  int64_t y_rs[kMaxMatrices];
  int feat;                        // features per workgroup (1..32)
  int block_end[kMaxMatrices];     // cumulative workgroups per matrix
  const void* residual;            // [rows, n_0] with row stride r_rs
  int64_t r_rs;
  int alias_partials;              // partial sums reuse the normalised rows' LDS
};

constexpr int kLdsBytes = 160 * 1024;  // LDS per CU (gfx950)

// ---- one round of equal workgroups -------------------------------------------
// A decode-sized projection streams its weights once; every CU should pull an
// equal share, so a call runs about kTargetGroups workgroups of feat =
// ceil(features / kTargetGroups) consecutive features each (one or two MFMA
// tiles of 16 features, the rows past feat masked off by the buffer range).
// Each workgroup's waves split K; a feature's sum (MFMA steps in k order per
// wave, then the wave partials in wave order) does not depend on feat, so the
// fused ops and the single linears they replace agree bit for bit.
constexpr int kTargetGroups = 256;  // MI355X CUs
constexpr int kMaxFeat = 32;
int features_per_group(int64_t features) {
  const int64_t f = (features + kTargetGroups - 1) / kTargetGroups;
  return static_cast<int>(f < 1 ? 1 : (f > kMaxFeat ? kMaxFeat : f));
}
void assign_blocks(FusedArgs& a, int count) {
  int64_t total = 0;
  for (int i = 0; i < count; ++i) total += a.n[i];
  a.feat = features_per_group(total);
  int blocks = 0;
  for (int i = 0; i < kMaxMatrices; ++i) {
    if (i < count) blocks += (a.n[i] + a.feat - 1) / a.feat;
    a.block_end[i] = blocks;
  }
}

// LDS row stride of the normalised input, in elements: 8 extra elements move
// consecutive rows 4 banks apart, so the 16-row operand reads do not collide.
__host__ __device__ constexpr int norm_row(int hidden) { return hidden + 8; }

// NV: 16-byte vectors per lane of the norm prologue (0 = no norm, the input
// rows are read from global memory like the decode linear kernel does).
// TILES: 16-feature MFMA tiles per workgroup (feat <= 16 * TILES).
template <typename T, int MB, int KW, int U, int NV, int EPI, int TILES>
__global__ __launch_bounds__(KW * 64) void fused_rows_kernel(FusedArgs p) {
  constexpr int kWaves = KW;
  using MF = Mfma<T>;
  constexpr int NW = EPI == kSwiglu ? 2 : 1;  // weight streams per workgroup
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int c = lane & 15;
  const int g = lane >> 4;
  const int K = p.hidden;
  const int M = p.rows;
  const int F = p.feat;

  // The matrix and features [n0, n0 + F) of this workgroup.
  const int blk = blockIdx.x;
  const int j = blk < p.block_end[0] ? 0 : (blk < p.block_end[1] ? 1 : 2);
  const int n0 = (blk - (j == 0 ? 0 : p.block_end[j - 1])) * F;
  const int N = p.n[j];
  const int w_rows = min(F, N - n0);

  const int xs_bytes = NV > 0 ? MB * 16 * norm_row(K) * 2 : 0;
  unsigned char* xs = smem;
  // [NW][TILES][kWaves][MB][64][4]; after the normalised rows, or over them
  // when both do not fit (then written only once every wave is done with them).
  float* partial = reinterpret_cast<float*>(smem + (p.alias_partials ? 0 : xs_bytes));

  // K range of this wave.
  const int steps = (K + 31) / 32;             // 32-wide MFMA k-steps
  const int per_wave = (steps + kWaves - 1) / kWaves;
  const int s_begin = wave * per_wave;
  const int s_end = min(s_begin + per_wave, steps);

  __amdgpu_buffer_rsrc_t rw[NW][TILES];
#pragma unroll
  for (int t = 0; t < TILES; ++t) {
    const int rows_t = max(0, min(16, w_rows - 16 * t));
#pragma unroll
    for (int h = 0; h < NW; ++h) {
      const void* base = p.w[NW == 2 ? h : j];
      rw[h][t] = make_rsrc(static_cast<const T*>(base) + static_cast<int64_t>(n0 + 16 * t) * K,
                           static_cast<int64_t>(rows_t) * K * 2);
    }
  }
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(
      p.x, (static_cast<int64_t>(M) - 1) * p.x_rs * 2 + static_cast<int64_t>(K) * 2);
  const int w_off = c * K * 2 + g * 16;
  int x_off[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) {
    x_off[i] = NV > 0 ? ((i * 16 + c) * norm_row(K) + g * 8) * 2
                      : static_cast<int>((i * 16 + c) * p.x_rs * 2) + g * 16;
  }

  f32x4_t acc[NW][TILES][MB];
#pragma unroll
  for (int h = 0; h < NW; ++h)
#pragma unroll
    for (int t = 0; t < TILES; ++t)
#pragma unroll
      for (int i = 0; i < MB; ++i) acc[h][t][i] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // Weight (and, without the norm, input) operands U k-steps at a time, the
  // next batch in flight while the current one is multiplied.
  uint4 wa[U][NW][TILES], wb[U][NW][TILES], xa[U][NV > 0 ? 1 : MB], xb[U][NV > 0 ? 1 : MB];
  auto fetch = [&](int s0, uint4 (&wr)[U][NW][TILES], uint4 (&xr)[U][NV > 0 ? 1 : MB]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int s = s0 + u;
      const bool ok = s < s_end && s * 32 + g * 8 < K;
#pragma unroll
      for (int h = 0; h < NW; ++h)
#pragma unroll
        for (int t = 0; t < TILES; ++t)
          wr[u][h][t] = ok ? buffer_load16(rw[h][t], w_off + s * 64) : make_uint4(0, 0, 0, 0);
      if constexpr (NV == 0) {
#pragma unroll
        for (int i = 0; i < MB; ++i)
          xr[u][i] = ok ? buffer_load16(rx, x_off[i] + s * 64) : make_uint4(0, 0, 0, 0);
      }
    }
  };
  auto multiply = [&](int s0, const uint4 (&wr)[U][NW][TILES],
                      const uint4 (&xr)[U][NV > 0 ? 1 : MB]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int s = s0 + u;
#pragma unroll
      for (int i = 0; i < MB; ++i) {
        uint4 xv;
        if constexpr (NV > 0) {
          const bool ok = s < s_end && s * 32 + g * 8 < K;
          xv = ok ? *reinterpret_cast<const uint4*>(xs + x_off[i] + s * 64) : make_uint4(0, 0, 0, 0);
        } else {
          xv = xr[u][i];
        }
        const auto a = __builtin_bit_cast(typename MF::vec, xv);
#pragma unroll
        for (int h = 0; h < NW; ++h)
#pragma unroll
          for (int t = 0; t < TILES; ++t)
            acc[h][t][i] =
                MF::run(a, __builtin_bit_cast(typename MF::vec, wr[u][h][t]), acc[h][t][i]);
      }
    }
  };

  // Norm prologue: this wave's input rows and the norm weight are requested
  // first, then the first weight batch, and the rows are normalised (exactly
  // as the rms_norm kernel does) while the weights stream: the loads
  // complete in issue order, so waiting for the rows does not wait for the
  // weights.
  constexpr int RPW = (MB * 16 + kWaves - 1) / kWaves;  // rows per wave
  constexpr int NVR = NV > 0 ? NV : 1;
  uint4 xrow[NV > 0 ? RPW : 1][NVR], wnorm[NVR];
  if constexpr (NV > 0) {
    const T* x = static_cast<const T*>(p.x);
    slc::rms_norm_load<T, NV>(static_cast<const T*>(p.norm_w), K, lane, wnorm);
#pragma unroll
    for (int q = 0; q < RPW; ++q) {
      const int m = wave + q * kWaves;
      if (m < M) {
        slc::rms_norm_load<T, NV>(x + m * p.x_rs, K, lane, xrow[q]);
      } else {
#pragma unroll
        for (int i = 0; i < NV; ++i) xrow[q][i] = make_uint4(0, 0, 0, 0);
      }
    }
  }
  int s0 = s_begin;
  fetch(s0, wa, xa);
  // The epilogue's bias and residual elements of this thread, requested
  // behind the first weight batch (so the multiply does not wait for them)
  // instead of after the cross-wave sum (a dependent round trip at the end).
  constexpr int kEpiStride = kWaves * 64;
  constexpr int kEpiIters = (TILES * MB * 256 + kEpiStride - 1) / kEpiStride;
  float pre_bias[kEpiIters], pre_res[kEpiIters];
  auto epi_coords = [&](int idx, int& t, int& i, int& l, int& r, int& f, int& n, int& m) {
    t = idx / (MB * 256);
    const int e = idx % (MB * 256);
    i = e / 256;
    l = (e / 4) % 64;
    r = e % 4;
    f = 16 * t + (l & 15);
    n = n0 + f;
    m = i * 16 + 4 * (l >> 4) + r;
  };
  if constexpr (EPI != kSwiglu) {
#pragma unroll
    for (int k = 0; k < kEpiIters; ++k) {
      const int idx = tid + k * kEpiStride;
      int t, i, l, r, f, n, m;
      epi_coords(idx, t, i, l, r, f, n, m);
      const bool valid = idx < TILES * MB * 256 && f < w_rows && m < M;
      pre_bias[k] = valid && p.bias[j] != nullptr
                        ? slc::to_f32(static_cast<const T*>(p.bias[j])[n]) : 0.0f;
      pre_res[k] = 0.0f;
      if constexpr (EPI == kResidual)
        pre_res[k] = valid ? slc::to_f32(static_cast<const T*>(p.residual)[m * p.r_rs + n]) : 0.0f;
    }
  }
  if constexpr (NV > 0) {
    constexpr int VEC = 16 / sizeof(T);
#pragma unroll
    for (int q = 0; q < RPW; ++q) {
      const int m = wave + q * kWaves;
      if (m >= MB * 16) break;
      uint4 out[NV];
      if (m < M) {
        slc::rms_norm_from<T, NV, true>(xrow[q], wnorm, K, p.eps, lane, out);
      } else {
#pragma unroll
        for (int i = 0; i < NV; ++i) out[i] = make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int idx = lane + 64 * i;
        if (idx < K / VEC)
          *reinterpret_cast<uint4*>(xs + (m * norm_row(K) + idx * VEC) * 2) = out[i];
      }
    }
    __syncthreads();
  }
  while (s0 < s_end) {
    fetch(s0 + U, wb, xb);
    multiply(s0, wa, xa);
    s0 += U;
    if (s0 >= s_end) break;
    fetch(s0 + U, wa, xa);
    multiply(s0, wb, xb);
    s0 += U;
  }

  if (NV > 0 && p.alias_partials) __syncthreads();
  // C layout: lane (col c = feature, rows 4g..4g+3 = input rows of block i).
  auto part = [&](int h, int t, int v, int i, int l, int r) -> float& {
    return partial[(((((h * TILES + t) * kWaves + v) * MB + i) * 64 + l) * 4) + r];
  };
#pragma unroll
  for (int h = 0; h < NW; ++h)
#pragma unroll
    for (int t = 0; t < TILES; ++t)
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) part(h, t, wave, i, lane, r) = acc[h][t][i][r];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < kEpiIters; ++k) {
    const int idx = tid + k * kEpiStride;
    if (idx >= TILES * MB * 256) break;
    int t, i, l, r, f, n, m;
    epi_coords(idx, t, i, l, r, f, n, m);
    if (f >= w_rows || m >= M) continue;
    float sum = 0.0f;
#pragma unroll
    for (int v = 0; v < kWaves; ++v) sum += part(0, t, v, i, l, r);
    if constexpr (EPI == kSwiglu) {
      float up = 0.0f;
#pragma unroll
      for (int v = 0; v < kWaves; ++v) up += part(1, t, v, i, l, r);
      const float gate = slc::round_to<T>(sum);
      static_cast<T*>(p.y[0])[m * p.y_rs[0] + n] =
          slc::from_f32<T>(slc::swiglu_value<T>(gate, slc::round_to<T>(up)));
    } else {
      if (p.bias[j] != nullptr) sum += pre_bias[k];
      if constexpr (EPI == kResidual) sum = pre_res[k] + slc::round_to<T>(sum);
      static_cast<T*>(p.y[j])[m * p.y_rs[j] + n] = slc::from_f32<T>(sum);
    }
  }
}

template <typename T, int NV, int EPI>
int launch_rows(FusedArgs& a, hipStream_t stream) {
  const int blocks = a.block_end[kMaxMatrices - 1];
  const int nw = EPI == kSwiglu ? 2 : 1;
  const int kw = waves_for(a.hidden);
  const int tiles = a.feat > 16 ? 2 : 1;
  auto go = [&](auto kernel, int mb) {
    const int xs_bytes = NV > 0 ? mb * 16 * norm_row(a.hidden) * 2 : 0;
    const int part_bytes = nw * tiles * kw * mb * 64 * 4 * 4;
    a.alias_partials = xs_bytes + part_bytes > kLdsBytes;
    const int bytes = a.alias_partials ? (xs_bytes > part_bytes ? xs_bytes : part_bytes)
                                       : xs_bytes + part_bytes;
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e != hipSuccess) {
      slc_host::set_error("fused decode kernel: LDS size %d rejected: %s", bytes,
                          hipGetErrorString(e));
      return static_cast<int>(e);
    }
    hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(blocks)), dim3(kw * 64),
                       static_cast<unsigned>(bytes), stream, a);
    return slc_host::check_launch("fused decode kernel");
  };
  // Prefetch depth: as deep as the registers allow (two weight streams for
  // SwiGLU, and two tiles, divide it).
  constexpr int U1 = EPI == kSwiglu ? 4 : 8, U2 = EPI == kSwiglu ? 2 : 4;
  // 16 waves: half the k-steps per wave, half the prefetch depth.
  constexpr int V1 = U1 / 2, V2 = U2 / 2;
  if (kw == 16) {
    if (tiles == 2) {
      if (a.rows <= 16) return go(fused_rows_kernel<T, 1, 16, V1 / 2, NV, EPI, 2>, 1);
      return go(fused_rows_kernel<T, 2, 16, (V2 > 1 ? V2 / 2 : 1), NV, EPI, 2>, 2);
    }
    if (a.rows <= 16) return go(fused_rows_kernel<T, 1, 16, V1, NV, EPI, 1>, 1);
    return go(fused_rows_kernel<T, 2, 16, V2, NV, EPI, 1>, 2);
  }
  if (tiles == 2) {
    if (a.rows <= 16) return go(fused_rows_kernel<T, 1, 8, U1 / 2, NV, EPI, 2>, 1);
    return go(fused_rows_kernel<T, 2, 8, U2 / 2, NV, EPI, 2>, 2);
  }
  if (a.rows <= 16) return go(fused_rows_kernel<T, 1, 8, U1, NV, EPI, 1>, 1);
  return go(fused_rows_kernel<T, 2, 8, U2, NV, EPI, 1>, 2);
}

// Wide projections (the vocabulary head): enough 16-feature blocks to fill
// the GPU without splitting K, so each wave owns one block over the whole K
// (no cross-wave reduction, nothing through LDS) and keeps U k-steps of
// weights in flight.
constexpr int kWideBlocks = 1024;
// XL: the input rows are staged in LDS once per workgroup (row stride K + 8
// elements, so the 16 rows of an operand read fall 4 banks apart) instead of
// being re-read from the cache by every wave at every k-step.
// NNV > 0 (with XL): the staged rows are the RMS-normalised input, NNV
// 16-byte vectors per lane, computed by every workgroup with the function
// the rms_norm kernel uses (so the result equals rms_norm then linear bit
// for bit): the vocabulary head and its norm in one launch.
template <typename T, int MB, int U, bool XL = false, int NNV = 0>
__global__ __launch_bounds__(256) void wide_rows_kernel(FusedArgs p) {
  using MF = Mfma<T>;
  const int lane = threadIdx.x & 63;
  const int c = lane & 15;
  const int g = lane >> 4;
  const int K = p.hidden, M = p.rows, N = p.n[0];
  const int n0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 16;
  extern __shared__ uint4 x_lds[];
  const int x_stride = K / 8 + 1;  // 16-byte words per staged row
  if (n0 >= N && !XL) return;
  const T* w = static_cast<const T*>(p.w[0]);
  const int w_rows = min(16, N - n0);
  const __amdgpu_buffer_rsrc_t rw =
      make_rsrc(w + static_cast<int64_t>(n0) * K, static_cast<int64_t>(w_rows) * K * 2);
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(
      p.x, (static_cast<int64_t>(M) - 1) * p.x_rs * 2 + static_cast<int64_t>(K) * 2);
  const int w_off = c * K * 2 + g * 16;
  int x_off[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) x_off[i] = static_cast<int>((i * 16 + c) * p.x_rs * 2) + g * 16;
  const int steps = (K + 31) / 32;
  f32x4_t acc[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  uint4 wa[U], wb[U], xa[U][MB], xb[U][MB];
  auto fetch = [&](int s0, uint4 (&wr)[U], uint4 (&xr)[U][MB]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int s = s0 + u;
      const bool ok = s < steps && s * 32 + g * 8 < K;
      wr[u] = ok ? buffer_load16(rw, w_off + s * 64) : make_uint4(0, 0, 0, 0);
      if constexpr (!XL) {
#pragma unroll
        for (int i = 0; i < MB; ++i)
          xr[u][i] = ok ? buffer_load16(rx, x_off[i] + s * 64) : make_uint4(0, 0, 0, 0);
      }
    }
  };
  auto multiply = [&](int s0, const uint4 (&wr)[U], const uint4 (&xr)[U][MB]) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int i = 0; i < MB; ++i) {
        uint4 xv = xr[u][i];
        if constexpr (XL) {
          const int s = s0 + u;
          const int row = i * 16 + c;
          xv = row < M && s < steps && s * 32 + g * 8 < K ? x_lds[row * x_stride + s * 4 + g]
                                                          : make_uint4(0, 0, 0, 0);
        }
        acc[i] = MF::run(__builtin_bit_cast(typename MF::vec, xv),
                         __builtin_bit_cast(typename MF::vec, wr[u]), acc[i]);
      }
  };
  // XL with NNV: the rows to normalise and the norm weight are requested
  // before the first weight batch and normalised after it is issued: the
  // loads complete in issue order, so the norm waits for the rows only.
  // (The launch keeps M <= 16 rows, 4 per wave.)
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const T* x = static_cast<const T*>(p.x);
  uint4 xrow[NNV > 0 ? 4 : 1][NNV > 0 ? NNV : 1], wnorm[NNV > 0 ? NNV : 1];
  if constexpr (XL && NNV > 0) {
    slc::rms_norm_load<T, NNV>(static_cast<const T*>(p.norm_w), K, lane, wnorm);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int m = wave + 4 * q;
      if (m < M) slc::rms_norm_load<T, NNV>(x + m * p.x_rs, K, lane, xrow[q]);
    }
  }
  int s0 = 0;
  fetch(s0, wa, xa);
  if constexpr (XL) {
    // Every wave passes the barrier (the waves past N leave only after it).
    if constexpr (NNV > 0) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = wave + 4 * q;
        if (m < M) {
          uint4 out[NNV];
          slc::rms_norm_from<T, NNV, true>(xrow[q], wnorm, K, p.eps, lane, out);
#pragma unroll
          for (int i = 0; i < NNV; ++i)
            if (lane + 64 * i < K / 8) x_lds[m * x_stride + lane + 64 * i] = out[i];
        }
      }
    } else {
      // The plain rows: requested here, after the weights (their wait covers
      // the first weight batch; staging them earlier spilled registers).
      for (int idx = threadIdx.x; idx < M * (K / 8); idx += 256) {
        const int r = idx / (K / 8), v = idx % (K / 8);
        x_lds[r * x_stride + v] = *reinterpret_cast<const uint4*>(x + r * p.x_rs + v * 8);
      }
    }
    __syncthreads();
    if (n0 >= N) return;
  }
  while (s0 < steps) {
    fetch(s0 + U, wb, xb);
    multiply(s0, wa, xa);
    s0 += U;
    if (s0 >= steps) break;
    fetch(s0 + U, wa, xa);
    multiply(s0, wb, xb);
    s0 += U;
  }
  // C layout: lane (col c = feature, rows 4g..4g+3 of block i).
  const int n = n0 + c;
  if (n >= N) return;
  const float bias = p.bias[0] != nullptr ? slc::to_f32(static_cast<const T*>(p.bias[0])[n]) : 0.0f;
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = i * 16 + 4 * g + r;
      if (m < M) {
        float v = acc[i][r];
        if (p.bias[0] != nullptr) v += bias;
        static_cast<T*>(p.y[0])[m * p.y_rs[0] + n] = slc::from_f32<T>(v);
      }
    }
}

#ifndef SLC_WIDE_U
#define SLC_WIDE_U 8
#endif
#ifndef SLC_WIDE_XL
#define SLC_WIDE_XL 1
#endif
template <typename T>
int launch_wide(FusedArgs& a, hipStream_t stream) {
  const int blocks = (a.n[0] + 63) / 64;
  const int x_bytes = a.rows * (a.hidden / 8 + 1) * 16;
  const bool x_aligned = reinterpret_cast<uintptr_t>(a.x) % 16 == 0 && a.x_rs % 8 == 0;
  if (a.norm_w != nullptr) {
    // Norm and head in one launch: only with the rows staged in LDS.
    if (a.rows > 16 || a.hidden % 8 != 0 || !x_aligned || x_bytes > 32 * 1024)
      return SLC_ERR_UNSUPPORTED;
    const int nv = (a.hidden / 8 + 63) / 64;
#define SLC_WIDE_NORM(NV)                                                                 \
  hipLaunchKernelGGL((wide_rows_kernel<T, 1, SLC_WIDE_U, true, NV>), dim3(blocks), dim3(256), \
                     static_cast<unsigned>(x_bytes), stream, a)
    if (nv == 1) {
      SLC_WIDE_NORM(1);
    } else if (nv == 2) {
      SLC_WIDE_NORM(2);
    } else if (nv == 3) {
      SLC_WIDE_NORM(3);
    } else if (nv == 4) {
      SLC_WIDE_NORM(4);
    } else {
      return SLC_ERR_UNSUPPORTED;
    }
#undef SLC_WIDE_NORM
    return slc_host::check_launch("decode norm + linear (wide)");
  }
  if (a.rows <= 16 && SLC_WIDE_XL && a.hidden % 8 == 0 && x_aligned && x_bytes <= 32 * 1024) {
    hipLaunchKernelGGL((wide_rows_kernel<T, 1, SLC_WIDE_U, true>), dim3(blocks), dim3(256),
                       static_cast<unsigned>(x_bytes), stream, a);
  } else if (a.rows <= 16) {
    hipLaunchKernelGGL((wide_rows_kernel<T, 1, SLC_WIDE_U>), dim3(blocks), dim3(256), 0, stream, a);
  } else {
    hipLaunchKernelGGL((wide_rows_kernel<T, 2, 4>), dim3(blocks), dim3(256), 0, stream, a);
  }
  return slc_host::check_launch("decode linear (wide)");
}

template <int EPI>
int dispatch_rows(FusedArgs& a, int dtype, hipStream_t stream) {
  const bool norm = a.norm_w != nullptr;
  const int nv = (a.hidden / 8 + 63) / 64;  // 16-byte vectors per lane
#define SLC_ROWS(T)                                             \
  do {                                                          \
    if (!norm) return launch_rows<T, 0, EPI>(a, stream);        \
    if (nv <= 1) return launch_rows<T, 1, EPI>(a, stream);      \
    if (nv <= 2) return launch_rows<T, 2, EPI>(a, stream);      \
    return launch_rows<T, 4, EPI>(a, stream);                   \
  } while (0)
  if (dtype == SLC_BF16) SLC_ROWS(slc::bf16_t);
  SLC_ROWS(slc::f16_t);
#undef SLC_ROWS
}

// Shared argument checks: decode-sized rows, 16-byte aligned contiguous rows.
int check_rows(const char* what, const void* x, int64_t x_rs, int64_t rows, int64_t hidden,
               int dtype, bool norm) {
  SLC_REQUIRE(dtype == SLC_BF16 || dtype == SLC_F16, "%s: dtype must be bf16 or fp16", what);
  SLC_REQUIRE(rows >= 1 && rows <= kMaxRows, "%s: rows must be 1..%d", what, kMaxRows);
  SLC_REQUIRE(hidden >= 8 && hidden % 8 == 0, "%s: hidden must be a positive multiple of 8",
              what);
  SLC_REQUIRE(!norm || hidden <= 64 * 8 * 4, "%s: hidden above 2048 with a norm", what);
  SLC_REQUIRE(x != nullptr && (reinterpret_cast<uintptr_t>(x) & 15) == 0 && x_rs >= hidden &&
                  x_rs % 8 == 0,
              "%s: input rows must be 16-byte aligned", what);
  return SLC_OK;
}

// ---- rope + kv_store ---------------------------------------------------------

struct RopeStoreArgs {
  int64_t q_heads, kv_heads, tokens, half, capacity;
  int64_t q_sb, q_sh, q_st, k_sb, k_sh, k_st, v_sb, v_sh, v_st;
  int64_t c_sb, c_st, s_sb, s_st;
  int64_t qo_sb, qo_sh, qo_st;
};

// One thread owns dims [d, d + VEC) of the first half and the matching dims of
// the second half of one (batch, head, token) row.  Heads [0, QH) are query
// heads (rotated into q_out), [QH, QH + KVH) key heads (rotated into the key
// buffer row positions[b] + t), [QH + KVH, QH + 2 KVH) value heads (copied
// into the value buffer).  Rows past the capacity are skipped and flagged.
// Lengths advance folded into the store: with `lengths_out` set, every
// workgroup counts itself done once all its threads have read their positions
// (the per-stream counter), and the last one writes
// lengths_out[b] = positions[b] + advance (in place is fine: every read
// happened before the count completed), flags an advance past the capacity and
// re-arms the counter.
// The counter is the first int of the caller's counter array (zero between
// calls).

template <typename T, int VEC>
__global__ __launch_bounds__(256) void rope_kv_store_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const T* __restrict__ cosine, const T* __restrict__ sine, T* __restrict__ q_out,
    T* __restrict__ key_buffer, T* __restrict__ value_buffer,
    const int64_t* positions, int* __restrict__ overflow, RopeStoreArgs a,
    int64_t total, int64_t* lengths_out, int64_t batch, int64_t advance, int* counter) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid < total) {
    const int64_t per_row = a.half / VEC;
    const int64_t d = (gid % per_row) * VEC;
    int64_t rest = gid / per_row;
    const int64_t t = rest % a.tokens;
    rest /= a.tokens;
    const int64_t heads = a.q_heads + 2 * a.kv_heads;
    const int64_t h = rest % heads;
    const int64_t b = rest / heads;
    const int64_t D = 2 * a.half;

    const T* src = nullptr;
    T* dst = nullptr;
    if (h < a.q_heads) {
      src = q + b * a.q_sb + h * a.q_sh + t * a.q_st;
      dst = q_out + b * a.qo_sb + h * a.qo_sh + t * a.qo_st;
    } else {
      const int64_t position = positions[b] + t;
      if (position < 0 || position >= a.capacity) {
        if (overflow != nullptr) *overflow = 1;
      } else {
        const bool is_key = h < a.q_heads + a.kv_heads;
        const int64_t kh = is_key ? h - a.q_heads : h - a.q_heads - a.kv_heads;
        const int64_t row = ((b * a.capacity + position) * a.kv_heads + kh) * D;
        if (!is_key) {
          const T* vs = v + b * a.v_sb + kh * a.v_sh + t * a.v_st;
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            value_buffer[row + d + e] = vs[d + e];
            value_buffer[row + d + a.half + e] = vs[d + a.half + e];
          }
        } else {
          src = k + b * a.k_sb + kh * a.k_sh + t * a.k_st;
          dst = key_buffer + row;
        }
      }
    }
    if (src != nullptr) {
      const T* cr = cosine + b * a.c_sb + t * a.c_st;
      const T* sr = sine + b * a.s_sb + t * a.s_st;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        float o1, o2;
        slc::rope_pair<T>(slc::to_f32(src[d + e]), slc::to_f32(src[d + a.half + e]),
                          slc::to_f32(cr[d + e]), slc::to_f32(cr[d + a.half + e]),
                          slc::to_f32(sr[d + e]), slc::to_f32(sr[d + a.half + e]), o1, o2);
        dst[d + e] = slc::from_f32<T>(o1);
        dst[d + a.half + e] = slc::from_f32<T>(o2);
      }
    }
  }
  if (lengths_out == nullptr) return;
  __shared__ int is_last;
  __syncthreads();  // every thread of this workgroup has read its positions
  if (threadIdx.x == 0) {
    // Acquire-release: this workgroup's reads of the positions precede the
    // count, and the last workgroup's length writes follow every arrival.
    const int before =
        __hip_atomic_fetch_add(counter, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    is_last = before == static_cast<int>(gridDim.x) - 1;
    if (is_last) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!is_last) return;
  for (int64_t b = threadIdx.x; b < batch; b += blockDim.x) {
    const int64_t next = positions[b] + advance;
    lengths_out[b] = next;
    if (overflow != nullptr && (next > a.capacity || next < 0)) *overflow = 1;
  }
}

}  // namespace

namespace slc_host {

// Decode-sized plain linear (rows <= 32) for slc_hip_linear: the same kernel
// as the fused ops, so fused and unfused graphs agree bit for bit.
int rows_linear(const void* x, int64_t x_rs, int64_t rows, int64_t K, int64_t N,
                const void* w, const void* bias, void* y, int64_t y_rs, int dtype,
                hipStream_t stream) {
  FusedArgs a{};
  a.x = x;
  a.x_rs = x_rs;
  a.rows = static_cast<int>(rows);
  a.hidden = static_cast<int>(K);
  a.w[0] = w;
  a.bias[0] = bias;
  a.y[0] = y;
  a.n[0] = static_cast<int>(N);
  a.y_rs[0] = y_rs;
  if ((N + 15) / 16 >= kWideBlocks) {
    return dtype == SLC_BF16 ? launch_wide<slc::bf16_t>(a, stream)
                             : launch_wide<slc::f16_t>(a, stream);
  }
  assign_blocks(a, 1);
  return dispatch_rows<kStore>(a, dtype, stream);
}

bool rows_linear_eligible(const void* x, int64_t x_rs, int64_t rows, int64_t K, int64_t N,
                          int dtype) {
  return (dtype == SLC_BF16 || dtype == SLC_F16) && rows >= 1 && rows <= kMaxRows &&
         K % 8 == 0 && K >= 8 && x_rs % 8 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
         N <= (1 << 24);
}

}  // namespace slc_host

extern "C" int slc_hip_norm_linear_group(
    const void* x, int64_t x_rs, const void* norm_weight, float epsilon, int64_t rows,
    int64_t hidden, int count, const void* w0, const void* b0, void* y0, int64_t n0,
    int64_t y0_rs, const void* w1, const void* b1, void* y1, int64_t n1, int64_t y1_rs,
    const void* w2, const void* b2, void* y2, int64_t n2, int64_t y2_rs, int dtype,
    void* stream) {
  const char* what = "slc_hip_norm_linear_group";
  if (int rc = check_rows(what, x, x_rs, rows, hidden, dtype, norm_weight != nullptr)) return rc;
  SLC_REQUIRE(count >= 1 && count <= kMaxMatrices, "%s: 1 to 3 matrices", what);
  FusedArgs a{};
  a.x = x;
  a.x_rs = x_rs;
  a.norm_w = norm_weight;
  a.eps = epsilon;
  a.rows = static_cast<int>(rows);
  a.hidden = static_cast<int>(hidden);
  const void* ws[3] = {w0, w1, w2};
  const void* bs[3] = {b0, b1, b2};
  void* ys[3] = {y0, y1, y2};
  const int64_t ns[3] = {n0, n1, n2};
  const int64_t yrs[3] = {y0_rs, y1_rs, y2_rs};
  for (int i = 0; i < kMaxMatrices; ++i) {
    if (i < count) {
      SLC_REQUIRE(ws[i] && ys[i] && ns[i] >= 1 && ns[i] <= (1 << 24) && yrs[i] >= ns[i],
                  "%s: bad matrix %d", what, i);
      a.w[i] = ws[i];
      a.bias[i] = bs[i];
      a.y[i] = ys[i];
      a.n[i] = static_cast<int>(ns[i]);
      a.y_rs[i] = yrs[i];
    }
  }
  // One vocabulary-width matrix: the wide kernel, normalising in its
  // staging.  The single linear runs such a head on the wide kernel too, so
  // when that kernel cannot take the norm (rows past 16) nothing is launched
  // and the caller runs the norm and the linear: the equal-workgroup kernel
  // would sum K in another order.
  if (count == 1 && (a.n[0] + 15) / 16 >= kWideBlocks && norm_weight != nullptr) {
    return dtype == SLC_BF16 ? launch_wide<slc::bf16_t>(a, static_cast<hipStream_t>(stream))
                             : launch_wide<slc::f16_t>(a, static_cast<hipStream_t>(stream));
  }
  assign_blocks(a, count);
  return dispatch_rows<kStore>(a, dtype, static_cast<hipStream_t>(stream));
}

extern "C" int slc_hip_norm_linear_swiglu(const void* x, int64_t x_rs, const void* norm_weight,
                                          float epsilon, int64_t rows, int64_t hidden,
                                          int64_t features, const void* w_gate,
                                          const void* w_up, void* y, int64_t y_rs, int dtype,
                                          void* stream) {
  const char* what = "slc_hip_norm_linear_swiglu";
  if (int rc = check_rows(what, x, x_rs, rows, hidden, dtype, norm_weight != nullptr)) return rc;
  SLC_REQUIRE(w_gate && w_up && y && features >= 1 && features <= (1 << 24) && y_rs >= features,
              "%s: bad projections", what);
  FusedArgs a{};
  a.x = x;
  a.x_rs = x_rs;
  a.norm_w = norm_weight;
  a.eps = epsilon;
  a.rows = static_cast<int>(rows);
  a.hidden = static_cast<int>(hidden);
  a.w[0] = w_gate;
  a.w[1] = w_up;
  a.y[0] = y;
  a.n[0] = static_cast<int>(features);
  a.y_rs[0] = y_rs;
  assign_blocks(a, 1);
  return dispatch_rows<kSwiglu>(a, dtype, static_cast<hipStream_t>(stream));
}

extern "C" int slc_hip_linear_residual(const void* x, int64_t x_rs, int64_t rows,
                                       int64_t in_features, int64_t out_features,
                                       const void* weight, const void* bias,
                                       const void* residual, int64_t residual_rs, void* y,
                                       int64_t y_rs, int dtype, void* stream) {
  const char* what = "slc_hip_linear_residual";
  if (rows > kMaxRows) {
    // Prefill-sized: the tile kernel with the residual in its store epilogue.
    SLC_REQUIRE(x && weight && residual && y && in_features >= 1 && out_features >= 1,
                "%s: bad operands", what);
    return slc_host::gemm_residual(x, x_rs, rows, in_features, out_features, weight, bias,
                                   residual, residual_rs, y, y_rs, dtype,
                                   static_cast<hipStream_t>(stream));
  }
  if (int rc = check_rows(what, x, x_rs, rows, in_features, dtype, false)) return rc;
  SLC_REQUIRE(weight && residual && y && out_features >= 1 && out_features <= (1 << 24) &&
                  y_rs >= out_features && residual_rs >= out_features,
              "%s: bad operands", what);
  FusedArgs a{};
  a.x = x;
  a.x_rs = x_rs;
  a.rows = static_cast<int>(rows);
  a.hidden = static_cast<int>(in_features);
  a.w[0] = weight;
  a.bias[0] = bias;
  a.y[0] = y;
  a.n[0] = static_cast<int>(out_features);
  a.y_rs[0] = y_rs;
  a.residual = residual;
  a.r_rs = residual_rs;
  assign_blocks(a, 1);
  return dispatch_rows<kResidual>(a, dtype, static_cast<hipStream_t>(stream));
}

extern "C" int slc_hip_rope_kv_store(
    const void* query, const void* key, const void* value, const void* cosine,
    const void* sine, void* query_out, void* key_buffer, void* value_buffer,
    const int64_t* positions, int* overflow, int64_t* lengths_out, int64_t advance, int dtype,
    int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t tokens, int64_t head_dim,
    int64_t capacity, int64_t q_sb, int64_t q_sh, int64_t q_st, int64_t k_sb, int64_t k_sh,
    int64_t k_st, int64_t v_sb, int64_t v_sh, int64_t v_st, int64_t cos_sb, int64_t cos_st,
    int64_t sin_sb, int64_t sin_st, int64_t qo_sb, int64_t qo_sh, int64_t qo_st, int* counters,
    int64_t num_counters, void* stream) {
  const char* what = "slc_hip_rope_kv_store";
  SLC_REQUIRE(slc_host::is_float_dtype(dtype), "%s: bad dtype %d", what, dtype);
  SLC_REQUIRE(batch >= 0 && q_heads >= 0 && kv_heads >= 0 && tokens >= 0 && head_dim > 0 &&
                  head_dim % 2 == 0 && capacity >= 0,
              "%s: bad sizes", what);
  SLC_REQUIRE(lengths_out == nullptr || advance > 0, "%s: advance must be positive", what);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (batch == 0) return SLC_OK;
  if (tokens == 0 || q_heads + kv_heads == 0) {
    if (lengths_out == nullptr) return SLC_OK;
    return slc_hip_kv_advance(positions, lengths_out, batch, advance, capacity, overflow, stream);
  }
  SLC_REQUIRE(query && key && value && cosine && sine && query_out && key_buffer &&
                  value_buffer && positions,
              "%s: null pointer", what);
  RopeStoreArgs a{q_heads, kv_heads, tokens, head_dim / 2, capacity, q_sb, q_sh, q_st,
                  k_sb,    k_sh,     k_st,   v_sb,         v_sh,     v_st, cos_sb, cos_st,
                  sin_sb,  sin_st,   qo_sb,  qo_sh,        qo_st};
  const int64_t per_row = (head_dim / 2) % 4 == 0 ? head_dim / 8 : head_dim / 2;
  const int64_t total = batch * (q_heads + 2 * kv_heads) * tokens * per_row;
  const dim3 grid(static_cast<unsigned>(slc_host::ceil_div(total, 256)));
  const bool vec4 = (head_dim / 2) % 4 == 0;
  // The advance rides on the store kernel when the caller gives a counter
  // for its arrivals; otherwise it is its own launch after the store.
  int* counter = counters != nullptr && num_counters >= 1 ? counters : nullptr;
  int64_t* fused_out = counter != nullptr ? lengths_out : nullptr;
#define SLC_RS(T, V)                                                                      \
  hipLaunchKernelGGL((rope_kv_store_kernel<T, V>), grid, dim3(256), 0, s,                \
                     static_cast<const T*>(query), static_cast<const T*>(key),           \
                     static_cast<const T*>(value), static_cast<const T*>(cosine),        \
                     static_cast<const T*>(sine), static_cast<T*>(query_out),            \
                     static_cast<T*>(key_buffer), static_cast<T*>(value_buffer), positions, \
                     overflow, a, total, fused_out, batch, advance, counter)
  if (dtype == SLC_BF16) {
    if (vec4) SLC_RS(slc::bf16_t, 4); else SLC_RS(slc::bf16_t, 1);
  } else if (dtype == SLC_F16) {
    if (vec4) SLC_RS(slc::f16_t, 4); else SLC_RS(slc::f16_t, 1);
  } else {
    if (vec4) SLC_RS(float, 4); else SLC_RS(float, 1);
  }
#undef SLC_RS
  const int rc = slc_host::check_launch(what);
  if (rc != SLC_OK || lengths_out == nullptr || fused_out != nullptr) return rc;
  return slc_hip_kv_advance(positions, lengths_out, batch, advance, capacity, overflow, stream);
}
