// rope: dual-output Qwen2 half-rotation rotary embedding (serve.rope).
//
// Semantics: src/stateful_llm_compiler/execution.py:741-767 and
// backends/triton_rope.py:10-133:
//   out = round(x * cos) + round(rotate_half(x) * sin),
//   rotate_half(x) = cat(-x[D/2:], x[:D/2])
// Each product is rounded to the tensor dtype before the add, exactly like two
// separate PyTorch bf16 multiplies followed by a bf16 add, so this kernel is
// bit-identical to the eager composite for every dtype.
//
// One launch covers the query and key heads.  A thread owns VEC consecutive
// dims of the first half and the matching VEC dims of the second half of one
// (batch, head, token) row: it reads each of x, cos and sin once and writes
// both halves, so the kernel moves the algorithmic minimum of bytes.
#include "common.hpp"
#include "op_math.hpp"

namespace {

template <typename T, int VEC>
struct VecOf;
template <typename T>
struct VecOf<T, 1> {
  using type = T;
};
template <>
struct VecOf<slc::bf16_t, 4> {
  using type = uint2;
};
template <>
struct VecOf<slc::f16_t, 4> {
  using type = uint2;
};
template <>
struct VecOf<float, 4> {
  using type = uint4;
};
template <>
struct VecOf<slc::bf16_t, 8> {
  using type = uint4;
};
template <>
struct VecOf<slc::f16_t, 8> {
  using type = uint4;
};

template <typename T, int VEC>
__device__ __forceinline__ void load_vec(const T* p, float (&out)[VEC]) {
  using V = typename VecOf<T, VEC>::type;
  const V raw = *reinterpret_cast<const V*>(p);
  const T* e = reinterpret_cast<const T*>(&raw);
#pragma unroll
  for (int k = 0; k < VEC; ++k) out[k] = slc::to_f32(e[k]);
}

template <typename T, int VEC>
__device__ __forceinline__ void store_vec(T* p, const float (&in)[VEC]) {
  using V = typename VecOf<T, VEC>::type;
  V raw;
  T* e = reinterpret_cast<T*>(&raw);
#pragma unroll
  for (int k = 0; k < VEC; ++k) e[k] = slc::from_f32<T>(in[k]);
  *reinterpret_cast<V*>(p) = raw;
}

struct RopeArgs {
  int64_t q_heads, kv_heads, tokens, half;
  int64_t q_sb, q_sh, q_st, k_sb, k_sh, k_st;
  int64_t c_sb, c_st, s_sb, s_st;
  int64_t qo_sb, qo_sh, qo_st, ko_sb, ko_sh, ko_st;
};

template <typename T, int VEC>
__global__ __launch_bounds__(256) void rope_kernel(
    const T* __restrict__ query, const T* __restrict__ key,
    const T* __restrict__ cosine, const T* __restrict__ sine,
    T* __restrict__ query_out, T* __restrict__ key_out, RopeArgs a,
    int64_t total) {
  // No FMA contraction: fp32 must match a separate multiply and add.
#pragma clang fp contract(off)
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= total) return;
  const int64_t groups_per_row = a.half / VEC;
  const int64_t d = (gid % groups_per_row) * VEC;
  int64_t rest = gid / groups_per_row;
  const int64_t t = rest % a.tokens;
  rest /= a.tokens;
  const int64_t heads = a.q_heads + a.kv_heads;
  const int64_t h = rest % heads;
  const int64_t b = rest / heads;

  const T* src;
  T* dst;
  if (h < a.q_heads) {
    src = query + b * a.q_sb + h * a.q_sh + t * a.q_st;
    dst = query_out + b * a.qo_sb + h * a.qo_sh + t * a.qo_st;
  } else {
    const int64_t kh = h - a.q_heads;
    src = key + b * a.k_sb + kh * a.k_sh + t * a.k_st;
    dst = key_out + b * a.ko_sb + kh * a.ko_sh + t * a.ko_st;
  }
  const T* cr = cosine + b * a.c_sb + t * a.c_st;
  const T* sr = sine + b * a.s_sb + t * a.s_st;

  float x1[VEC], x2[VEC], c1[VEC], c2[VEC], s1[VEC], s2[VEC];
  load_vec<T, VEC>(src + d, x1);
  load_vec<T, VEC>(src + d + a.half, x2);
  load_vec<T, VEC>(cr + d, c1);
  load_vec<T, VEC>(cr + d + a.half, c2);
  load_vec<T, VEC>(sr + d, s1);
  load_vec<T, VEC>(sr + d + a.half, s2);
  float o1[VEC], o2[VEC];
#pragma unroll
  for (int k = 0; k < VEC; ++k) slc::rope_pair<T>(x1[k], x2[k], c1[k], c2[k], s1[k], s2[k], o1[k], o2[k]);
  store_vec<T, VEC>(dst + d, o1);
  store_vec<T, VEC>(dst + d + a.half, o2);
}

template <typename T>
int launch(const void* q, const void* k, const void* c, const void* s,
           void* qo, void* ko, int64_t batch, RopeArgs a, int vec,
           hipStream_t stream) {
  const int64_t total = batch * (a.q_heads + a.kv_heads) * a.tokens * (a.half / vec);
  const dim3 grid(static_cast<unsigned>(slc_host::ceil_div(total, 256)));
  if constexpr (sizeof(T) == 2) {
    if (vec == 8) {
      hipLaunchKernelGGL((rope_kernel<T, 8>), grid, dim3(256), 0, stream,
                         static_cast<const T*>(q), static_cast<const T*>(k),
                         static_cast<const T*>(c), static_cast<const T*>(s),
                         static_cast<T*>(qo), static_cast<T*>(ko), a, total);
      return slc_host::check_launch("slc_hip_rope");
    }
  }
  if (vec == 4) {
    hipLaunchKernelGGL((rope_kernel<T, 4>), grid, dim3(256), 0, stream,
                       static_cast<const T*>(q), static_cast<const T*>(k),
                       static_cast<const T*>(c), static_cast<const T*>(s),
                       static_cast<T*>(qo), static_cast<T*>(ko), a, total);
  } else {
    hipLaunchKernelGGL((rope_kernel<T, 1>), grid, dim3(256), 0, stream,
                       static_cast<const T*>(q), static_cast<const T*>(k),
                       static_cast<const T*>(c), static_cast<const T*>(s),
                       static_cast<T*>(qo), static_cast<T*>(ko), a, total);
  }
  return slc_host::check_launch("slc_hip_rope");
}

}  // namespace

extern "C" int slc_hip_rope(const void* query, const void* key,
                            const void* cosine, const void* sine,
                            void* query_out, void* key_out, int dtype,
                            int64_t batch, int64_t q_heads, int64_t kv_heads,
                            int64_t tokens, int64_t head_dim, int64_t q_sb,
                            int64_t q_sh, int64_t q_st, int64_t k_sb,
                            int64_t k_sh, int64_t k_st, int64_t cos_sb,
                            int64_t cos_st, int64_t sin_sb, int64_t sin_st,
                            int64_t qo_sb, int64_t qo_sh, int64_t qo_st,
                            int64_t ko_sb, int64_t ko_sh, int64_t ko_st,
                            void* stream) {
  SLC_REQUIRE(slc_host::is_float_dtype(dtype), "slc_hip_rope: bad dtype %d", dtype);
  SLC_REQUIRE(batch >= 0 && q_heads >= 0 && kv_heads >= 0 && tokens >= 0 &&
                  head_dim > 0 && head_dim % 2 == 0 && head_dim <= 65536,
              "slc_hip_rope: bad sizes (head_dim must be a positive even number)");
  if (batch == 0 || tokens == 0 || q_heads + kv_heads == 0) return SLC_OK;
  SLC_REQUIRE(query && key && cosine && sine && query_out && key_out,
              "slc_hip_rope: null pointer");
  RopeArgs a{q_heads, kv_heads, tokens, head_dim / 2, q_sb, q_sh, q_st,
             k_sb,    k_sh,     k_st,   cos_sb,       cos_st, sin_sb, sin_st,
             qo_sb,   qo_sh,    qo_st,  ko_sb,        ko_sh,  ko_st};
  const int64_t es = slc_host::dtype_size(dtype);
  const int64_t vbytes = 4 * es;
  uint64_t bits = reinterpret_cast<uintptr_t>(query) |
                  reinterpret_cast<uintptr_t>(key) |
                  reinterpret_cast<uintptr_t>(cosine) |
                  reinterpret_cast<uintptr_t>(sine) |
                  reinterpret_cast<uintptr_t>(query_out) |
                  reinterpret_cast<uintptr_t>(key_out);
  const int64_t strides[] = {q_sb,   q_sh,   q_st,  k_sb,  k_sh,  k_st,
                             cos_sb, cos_st, sin_sb, sin_st, qo_sb, qo_sh,
                             qo_st,  ko_sb,  ko_sh, ko_st, head_dim / 2};
  for (int64_t st : strides) bits |= static_cast<uint64_t>(st * es);
  // 16-byte vectors (8 dims of a 2-byte dtype) when every row start and
  // half allows, else 4 dims, else single elements.
  const int vec = es == 2 && bits % 16 == 0 ? 8 : ((bits % vbytes) == 0 ? 4 : 1);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case SLC_BF16:
      return launch<slc::bf16_t>(query, key, cosine, sine, query_out, key_out,
                                 batch, a, vec, s);
    case SLC_F16:
      return launch<slc::f16_t>(query, key, cosine, sine, query_out, key_out,
                                batch, a, vec, s);
    default:
      return launch<float>(query, key, cosine, sine, query_out, key_out, batch,
                           a, vec, s);
  }
}
