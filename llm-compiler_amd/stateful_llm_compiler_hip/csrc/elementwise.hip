// Small bandwidth-bound device ops that complete the lowering of a Qwen2
// graph, so no op of a compiled step runs as an eager PyTorch kernel:
//   embedding   out[r, :] = table[ids[r], :]          (qwen2.py:427-430)
//   add         out = round(a + b)                    (residual adds)
//   swiglu      out = round(round(silu(gate)) * up)   (qwen2.py:253-256 order)
//   rope_table  cos/sin[b, t, :] = cos/sin(cat(f, f)), f = pos[b, t] * inv_freq
//                                                     (qwen2.py:136-149)
//   kv_advance  lengths_out = lengths_in + delta, overflow flag past capacity
//                                                     (execution.py:421-443)
//   argmax      greedy next token over the vocabulary
// Every op is one launch of 16-byte vector accesses where the layout allows.
#include <algorithm>

#include "common.hpp"
#include "op_math.hpp"

namespace {

template <typename T>
__global__ __launch_bounds__(256) void embedding_kernel(
    const int64_t* __restrict__ ids, const T* __restrict__ table, T* __restrict__ out,
    int64_t rows, int64_t hidden, int64_t vocab, int* __restrict__ bad_index) {
  const int64_t vec = 16 / sizeof(T);
  const int64_t per_row = hidden / vec;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= rows * per_row) return;
  const int64_t r = gid / per_row, u = gid % per_row;
  int64_t id = ids[r];
  if (id < 0 || id >= vocab) {
    if (bad_index != nullptr) *bad_index = 1;
    id = 0;
  }
  reinterpret_cast<uint4*>(out + r * hidden)[u] =
      reinterpret_cast<const uint4*>(table + id * hidden)[u];
}

template <typename T>
__global__ __launch_bounds__(256) void embedding_scalar_kernel(
    const int64_t* __restrict__ ids, const T* __restrict__ table, T* __restrict__ out,
    int64_t rows, int64_t hidden, int64_t vocab, int* __restrict__ bad_index) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= rows * hidden) return;
  const int64_t r = gid / hidden, d = gid % hidden;
  int64_t id = ids[r];
  if (id < 0 || id >= vocab) {
    if (bad_index != nullptr) *bad_index = 1;
    id = 0;
  }
  out[r * hidden + d] = table[id * hidden + d];
}

template <typename T>
__device__ __forceinline__ void load8(const T* p, float (&v)[8]) {
  if constexpr (sizeof(T) == 2) {
    const uint4 raw = *reinterpret_cast<const uint4*>(p);
    const T* e = reinterpret_cast<const T*>(&raw);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = slc::to_f32(e[i]);
  } else {
    const uint4 a = *reinterpret_cast<const uint4*>(p);
    const uint4 b = *reinterpret_cast<const uint4*>(p + 4);
    const float* ea = reinterpret_cast<const float*>(&a);
    const float* eb = reinterpret_cast<const float*>(&b);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = ea[i];
      v[4 + i] = eb[i];
    }
  }
}

template <typename T>
__device__ __forceinline__ void store8(T* p, const float (&v)[8]) {
  if constexpr (sizeof(T) == 2) {
    uint4 raw;
    T* e = reinterpret_cast<T*>(&raw);
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = slc::from_f32<T>(v[i]);
    *reinterpret_cast<uint4*>(p) = raw;
  } else {
    *reinterpret_cast<uint4*>(p) = make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]),
                                              __float_as_uint(v[2]), __float_as_uint(v[3]));
    *reinterpret_cast<uint4*>(p + 4) = make_uint4(__float_as_uint(v[4]), __float_as_uint(v[5]),
                                                  __float_as_uint(v[6]), __float_as_uint(v[7]));
  }
}

// OP 0: add, OP 1: swiglu (silu(a) rounded to T, times b).
template <typename T, int OP, bool VEC>
__global__ __launch_bounds__(256) void binary_kernel(const T* __restrict__ a,
                                                     const T* __restrict__ b,
                                                     T* __restrict__ out, int64_t n) {
#pragma clang fp contract(off)
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  auto apply = [](float x, float y) {
    if constexpr (OP == 0) {
      return x + y;
    } else {
      return slc::swiglu_value<T>(x, y);
    }
  };
  if constexpr (VEC) {
    if (gid * 8 >= n) return;
    float x[8], y[8], z[8];
    load8(a + gid * 8, x);
    load8(b + gid * 8, y);
#pragma unroll
    for (int i = 0; i < 8; ++i) z[i] = apply(x[i], y[i]);
    store8(out + gid * 8, z);
  } else {
    if (gid >= n) return;
    out[gid] = slc::from_f32<T>(apply(slc::to_f32(a[gid]), slc::to_f32(b[gid])));
  }
}

template <typename T>
__global__ __launch_bounds__(256) void rope_table_kernel(
    const int64_t* __restrict__ positions, const float* __restrict__ inv_freq,
    T* __restrict__ cosine, T* __restrict__ sine, int64_t rows, int64_t pos_stride_b,
    int64_t tokens, int head_dim) {
  const int half = head_dim / 2;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= rows * half) return;
  const int64_t r = gid / half;
  const int i = static_cast<int>(gid % half);
  const int64_t b = r / tokens, t = r % tokens;
  const float freq = static_cast<float>(positions[b * pos_stride_b + t]) * inv_freq[i];
  const float cv = cosf(freq), sv = sinf(freq);
  const T c = slc::from_f32<T>(cv), s = slc::from_f32<T>(sv);
  cosine[r * head_dim + i] = c;
  cosine[r * head_dim + i + half] = c;
  sine[r * head_dim + i] = s;
  sine[r * head_dim + i + half] = s;
}

__global__ void kv_advance_kernel(const int64_t* __restrict__ in, int64_t* __restrict__ out,
                                  int64_t batch, int64_t delta, int64_t capacity,
                                  int* __restrict__ overflow) {
  const int64_t b = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (b >= batch) return;
  const int64_t next = in[b] + delta;
  out[b] = next;
  if (overflow != nullptr && (next > capacity || next < 0)) *overflow = 1;
}

// One 1024-thread workgroup per row: 16-byte vector loads, four in flight per
// thread, then a (max, first index) reduction.  NaN ranks above every number
// and ties keep the lowest index, as torch.argmax does.
__device__ __forceinline__ bool argmax_better(float v, int64_t i, float best, int64_t best_i) {
  const bool v_nan = v != v, b_nan = best != best;
  if (v_nan != b_nan) return v_nan;
  if (!v_nan && v != best) return v > best;
  return i < best_i;
}

// Best (value, index) of row[begin, end) over the workgroup: each thread
// scans 16-byte vectors (or elements), then waves and workgroup reduce.
// Returns the result in every thread of wave 0 (thread 0 is authoritative).
template <typename T, int THREADS>
__device__ __forceinline__ void row_segment_best(const T* row, int64_t begin, int64_t end,
                                                 bool vector_ok, float& best, int64_t& best_i) {
  __shared__ float sv[THREADS / 64];
  __shared__ int64_t si[THREADS / 64];
  constexpr int VEC = 16 / sizeof(T);
  best = -INFINITY;
  best_i = INT64_MAX;
  int64_t done = begin;
  if (vector_ok) {
    // begin is a multiple of VEC (the host aligns segments).
    const int64_t v0 = begin / VEC;
    const int64_t v1 = end / VEC;
    const uint4* vrow = reinterpret_cast<const uint4*>(row);
    for (int64_t base = v0 + threadIdx.x; base < v1; base += 4 * THREADS) {
      uint4 raw[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t j = base + u * THREADS;
        raw[u] = j < v1 ? vrow[j] : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t j = base + u * THREADS;
        if (j >= v1) break;
        const T* e = reinterpret_cast<const T*>(&raw[u]);
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
          const float v = slc::to_f32(e[k]);
          if (argmax_better(v, j * VEC + k, best, best_i)) {
            best = v;
            best_i = j * VEC + k;
          }
        }
      }
    }
    done = v1 * VEC;
  }
  for (int64_t i = done + threadIdx.x; i < end; i += THREADS) {
    const float v = slc::to_f32(row[i]);
    if (argmax_better(v, i, best, best_i)) {
      best = v;
      best_i = i;
    }
  }
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(best, off, 64);
    const int64_t oi = __shfl_xor(best_i, off, 64);
    if (argmax_better(ov, oi, best, best_i)) {
      best = ov;
      best_i = oi;
    }
  }
  if ((threadIdx.x & 63) == 0) {
    sv[threadIdx.x >> 6] = best;
    si[threadIdx.x >> 6] = best_i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < THREADS / 64; ++w) {
      if (argmax_better(sv[w], si[w], best, best_i)) {
        best = sv[w];
        best_i = si[w];
      }
    }
  }
}

template <typename T>
__global__ __launch_bounds__(1024) void argmax_kernel(const T* __restrict__ logits,
                                                      int64_t* __restrict__ out, int64_t cols,
                                                      int64_t row_stride, int vector_ok) {
  const int64_t r = blockIdx.x;
  float best;
  int64_t best_i;
  row_segment_best<T, 1024>(logits + r * row_stride, 0, cols, vector_ok != 0, best, best_i);
  if (threadIdx.x == 0) out[r] = best_i < cols ? best_i : 0;
}

// Wide rows: `segs` workgroups per row each reduce one segment and publish
// (value, index) with agent-scope stores; the workgroup that completes the
// row's count combines the segments in order and re-arms the counter.  The
// counters (zero between calls) and the segment results (scratch) are the
// caller's (ArgmaxWorkspace); the add that counts is an agent-scope acquire-release,
// so the publishing thread's stores precede the count and the combining
// workgroup's loads follow every other arrival.  Ties keep the lowest index
// because segments are combined in index order with the same comparison.
constexpr int kArgmaxSegs = 64;
constexpr int kArgmaxThreads = 256;
struct ArgmaxWorkspace {
  int* counters;   // [rows], zero between calls
  float* value;    // [rows * kArgmaxSegs]
  int64_t* index;  // [rows * kArgmaxSegs]
};
int64_t argmax_workspace_bytes(int64_t rows) { return rows * kArgmaxSegs * (4 + 8); }
ArgmaxWorkspace argmax_workspace(void* base, int* counters, int64_t rows) {
  char* p = static_cast<char*>(base);
  ArgmaxWorkspace w;
  w.counters = counters;
  w.index = reinterpret_cast<int64_t*>(p);
  w.value = reinterpret_cast<float*>(p + rows * kArgmaxSegs * 8);
  return w;
}

template <typename T>
__global__ __launch_bounds__(kArgmaxThreads) void argmax_split_kernel(
    const T* __restrict__ logits, int64_t* __restrict__ out, int64_t cols, int64_t row_stride,
    int vector_ok, int64_t seg_len, ArgmaxWorkspace ws) {
  const int seg = blockIdx.x;
  const int segs = gridDim.x;
  const int r = blockIdx.y;
  const int64_t begin = seg * seg_len;
  const int64_t end = begin + seg_len < cols ? begin + seg_len : cols;
  float best;
  int64_t best_i;
  row_segment_best<T, kArgmaxThreads>(logits + r * row_stride, begin, end, vector_ok != 0,
                                      best, best_i);
  __shared__ int is_last;
  if (threadIdx.x == 0) {
    const int slot = r * kArgmaxSegs + seg;
    __hip_atomic_store(&ws.value[slot], best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&ws.index[slot], best_i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // Release per workgroup, acquire only in the one completing the count
    // (an acquire invalidates the XCD's L2, so paying it once per row is
    // cheaper than in every workgroup).  The fence, the barrier below and
    // the completing wave's loads order its reads after every segment's
    // stores.
    const int before = __hip_atomic_fetch_add(&ws.counters[r], 1, __ATOMIC_RELEASE,
                                              __HIP_MEMORY_SCOPE_AGENT);
    is_last = before == segs - 1;
    if (is_last) {
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      __hip_atomic_store(&ws.counters[r], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();
  if (!is_last || threadIdx.x >= 64) return;
  // Wave 0 combines: lane s holds segment s (and s + 64 ...), then a
  // lowest-index-first reduction.
  float v = -INFINITY;
  int64_t i = INT64_MAX;
  for (int s = threadIdx.x; s < segs; s += 64) {
    const int slot = r * kArgmaxSegs + s;
    const float sv = __hip_atomic_load(&ws.value[slot], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int64_t si = __hip_atomic_load(&ws.index[slot], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (argmax_better(sv, si, v, i)) {
      v = sv;
      i = si;
    }
  }
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(v, off, 64);
    const int64_t oi = __shfl_xor(i, off, 64);
    if (argmax_better(ov, oi, v, i)) {
      v = ov;
      i = oi;
    }
  }
  if (threadIdx.x == 0) out[r] = i < cols ? i : 0;
}

template <typename T>
int launch_embedding(const int64_t* ids, const void* table, void* out, int64_t rows,
                     int64_t hidden, int64_t vocab, int* bad, hipStream_t s) {
  const int64_t vec = 16 / sizeof(T);
  const bool vector = hidden % vec == 0 && (reinterpret_cast<uintptr_t>(table) & 15) == 0 &&
                      (reinterpret_cast<uintptr_t>(out) & 15) == 0;
  const int64_t work = vector ? rows * (hidden / vec) : rows * hidden;
  const dim3 grid(static_cast<unsigned>(slc_host::ceil_div(work, 256)));
  if (vector) {
    hipLaunchKernelGGL((embedding_kernel<T>), grid, dim3(256), 0, s, ids,
                       static_cast<const T*>(table), static_cast<T*>(out), rows, hidden, vocab, bad);
  } else {
    hipLaunchKernelGGL((embedding_scalar_kernel<T>), grid, dim3(256), 0, s, ids,
                       static_cast<const T*>(table), static_cast<T*>(out), rows, hidden, vocab, bad);
  }
  return slc_host::check_launch("slc_hip_embedding");
}

template <typename T, int OP>
int launch_binary(const void* a, const void* b, void* out, int64_t n, hipStream_t s) {
  const uint64_t bits = reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
                        reinterpret_cast<uintptr_t>(out);
  const bool vector = n % 8 == 0 && (bits & 15) == 0;
  const int64_t work = vector ? n / 8 : n;
  const dim3 grid(static_cast<unsigned>(slc_host::ceil_div(work, 256)));
  if (vector) {
    hipLaunchKernelGGL((binary_kernel<T, OP, true>), grid, dim3(256), 0, s,
                       static_cast<const T*>(a), static_cast<const T*>(b), static_cast<T*>(out), n);
  } else {
    hipLaunchKernelGGL((binary_kernel<T, OP, false>), grid, dim3(256), 0, s,
                       static_cast<const T*>(a), static_cast<const T*>(b), static_cast<T*>(out), n);
  }
  return slc_host::check_launch(OP == 0 ? "slc_hip_add" : "slc_hip_swiglu");
}

template <int OP>
int binary_entry(const void* a, const void* b, void* out, int dtype, int64_t n, void* stream) {
  SLC_REQUIRE(slc_host::is_float_dtype(dtype), "elementwise op: bad dtype %d", dtype);
  SLC_REQUIRE(n >= 0, "elementwise op: negative size");
  if (n == 0) return SLC_OK;
  SLC_REQUIRE(a && b && out, "elementwise op: null pointer");
  SLC_REQUIRE(slc_host::ceil_div(n, 256) < (1LL << 31), "elementwise op: too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case SLC_BF16:
      return launch_binary<slc::bf16_t, OP>(a, b, out, n, s);
    case SLC_F16:
      return launch_binary<slc::f16_t, OP>(a, b, out, n, s);
    default:
      return launch_binary<float, OP>(a, b, out, n, s);
  }
}

}  // namespace

extern "C" int slc_hip_embedding(const int64_t* ids, const void* table, void* output,
                                 int dtype, int64_t rows, int64_t hidden, int64_t vocab,
                                 int* bad_index, void* stream) {
  SLC_REQUIRE(slc_host::is_float_dtype(dtype), "slc_hip_embedding: bad dtype %d", dtype);
  SLC_REQUIRE(rows >= 0 && hidden > 0 && vocab > 0, "slc_hip_embedding: bad sizes");
  if (rows == 0) return SLC_OK;
  SLC_REQUIRE(ids && table && output, "slc_hip_embedding: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case SLC_BF16:
      return launch_embedding<slc::bf16_t>(ids, table, output, rows, hidden, vocab, bad_index, s);
    case SLC_F16:
      return launch_embedding<slc::f16_t>(ids, table, output, rows, hidden, vocab, bad_index, s);
    default:
      return launch_embedding<float>(ids, table, output, rows, hidden, vocab, bad_index, s);
  }
}

extern "C" int slc_hip_add(const void* a, const void* b, void* output, int dtype,
                           int64_t numel, void* stream) {
  return binary_entry<0>(a, b, output, dtype, numel, stream);
}

extern "C" int slc_hip_swiglu(const void* gate, const void* up, void* output, int dtype,
                              int64_t numel, void* stream) {
  return binary_entry<1>(gate, up, output, dtype, numel, stream);
}

extern "C" int slc_hip_rope_table(const int64_t* positions, const float* inv_freq,
                                  void* cosine, void* sine, int dtype, int64_t batch,
                                  int64_t tokens, int64_t pos_stride_b, int64_t head_dim,
                                  void* stream) {
  SLC_REQUIRE(slc_host::is_float_dtype(dtype), "slc_hip_rope_table: bad dtype %d", dtype);
  SLC_REQUIRE(batch >= 0 && tokens >= 0 && head_dim > 0 && head_dim % 2 == 0,
              "slc_hip_rope_table: bad sizes");
  const int64_t rows = batch * tokens;
  if (rows == 0) return SLC_OK;
  SLC_REQUIRE(positions && inv_freq && cosine && sine, "slc_hip_rope_table: null pointer");
  const dim3 grid(static_cast<unsigned>(slc_host::ceil_div(rows * (head_dim / 2), 256)));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int hd = static_cast<int>(head_dim);
  switch (dtype) {
    case SLC_BF16:
      hipLaunchKernelGGL((rope_table_kernel<slc::bf16_t>), grid, dim3(256), 0, s, positions,
                         inv_freq, static_cast<slc::bf16_t*>(cosine),
                         static_cast<slc::bf16_t*>(sine), rows, pos_stride_b, tokens, hd);
      break;
    case SLC_F16:
      hipLaunchKernelGGL((rope_table_kernel<slc::f16_t>), grid, dim3(256), 0, s, positions,
                         inv_freq, static_cast<slc::f16_t*>(cosine),
                         static_cast<slc::f16_t*>(sine), rows, pos_stride_b, tokens, hd);
      break;
    default:
      hipLaunchKernelGGL((rope_table_kernel<float>), grid, dim3(256), 0, s, positions, inv_freq,
                         static_cast<float*>(cosine), static_cast<float*>(sine), rows,
                         pos_stride_b, tokens, hd);
  }
  return slc_host::check_launch("slc_hip_rope_table");
}

extern "C" int slc_hip_kv_advance(const int64_t* lengths_in, int64_t* lengths_out,
                                  int64_t batch, int64_t delta, int64_t capacity,
                                  int* overflow, void* stream) {
  SLC_REQUIRE(batch >= 0 && capacity > 0, "slc_hip_kv_advance: bad sizes");
  if (batch == 0) return SLC_OK;
  SLC_REQUIRE(lengths_in && lengths_out, "slc_hip_kv_advance: null pointer");
  hipLaunchKernelGGL(kv_advance_kernel, dim3(static_cast<unsigned>(slc_host::ceil_div(batch, 256))),
                     dim3(256), 0, static_cast<hipStream_t>(stream), lengths_in, lengths_out,
                     batch, delta, capacity, overflow);
  return slc_host::check_launch("slc_hip_kv_advance");
}

extern "C" int64_t slc_hip_argmax_workspace_size(int64_t rows) {
  return rows > 0 ? argmax_workspace_bytes(rows) : 0;
}

extern "C" int slc_hip_argmax(const void* logits, int64_t* output, int dtype, int64_t rows,
                              int64_t cols, int64_t row_stride, void* workspace,
                              int64_t workspace_bytes, int* counters, int64_t num_counters,
                              void* stream) {
  SLC_REQUIRE(slc_host::is_float_dtype(dtype), "slc_hip_argmax: bad dtype %d", dtype);
  SLC_REQUIRE(rows >= 0 && cols > 0 && rows <= 0x7fffffff, "slc_hip_argmax: bad sizes");
  if (rows == 0) return SLC_OK;
  SLC_REQUIRE(logits && output, "slc_hip_argmax: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t es = slc_host::dtype_size(dtype);
  const int vector_ok = (reinterpret_cast<uintptr_t>(logits) & 15) == 0 && (row_stride * es) % 16 == 0;
  // Wide rows split over several workgroups per row (about one per CU in
  // total, segments of at least 4096 elements) when the caller gives a
  // workspace and counters; else one 1024-thread workgroup per row.
  const int64_t vec = 16 / es;
  int64_t segs = std::min<int64_t>(kArgmaxSegs, std::max<int64_t>(1, 256 / rows));
  segs = std::min<int64_t>(segs, std::max<int64_t>(1, cols / 4096));
  if (segs > 1 && workspace != nullptr && workspace_bytes >= argmax_workspace_bytes(rows) &&
      counters != nullptr && num_counters >= rows && rows <= 65535) {
    const ArgmaxWorkspace ws = argmax_workspace(workspace, counters, rows);
    const int64_t seg_len = slc_host::ceil_div(slc_host::ceil_div(cols, segs), vec) * vec;
    segs = slc_host::ceil_div(cols, seg_len);
    const dim3 grid(static_cast<unsigned>(segs), static_cast<unsigned>(rows));
#define SLC_ARGMAX_SPLIT(TT)                                                                  \
  hipLaunchKernelGGL((argmax_split_kernel<TT>), grid, dim3(kArgmaxThreads), 0, s,            \
                     static_cast<const TT*>(logits), output, cols, row_stride, vector_ok, seg_len, \
                     ws)
    switch (dtype) {
      case SLC_BF16: SLC_ARGMAX_SPLIT(slc::bf16_t); break;
      case SLC_F16: SLC_ARGMAX_SPLIT(slc::f16_t); break;
      default: SLC_ARGMAX_SPLIT(float);
    }
#undef SLC_ARGMAX_SPLIT
    return slc_host::check_launch("slc_hip_argmax");
  }
  const dim3 grid(static_cast<unsigned>(rows));
  switch (dtype) {
    case SLC_BF16:
      hipLaunchKernelGGL((argmax_kernel<slc::bf16_t>), grid, dim3(1024), 0, s,
                         static_cast<const slc::bf16_t*>(logits), output, cols, row_stride, vector_ok);
      break;
    case SLC_F16:
      hipLaunchKernelGGL((argmax_kernel<slc::f16_t>), grid, dim3(1024), 0, s,
                         static_cast<const slc::f16_t*>(logits), output, cols, row_stride, vector_ok);
      break;
    default:
      hipLaunchKernelGGL((argmax_kernel<float>), grid, dim3(1024), 0, s,
                         static_cast<const float*>(logits), output, cols, row_stride, vector_ok);
  }
  return slc_host::check_launch("slc_hip_argmax");
}
