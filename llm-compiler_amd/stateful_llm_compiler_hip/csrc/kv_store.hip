// kv_store: scatter B x H x T x D rows into the preallocated
// B x capacity x H x D buffers (contiguous_bshd).
//
// Follows the reference's runtime contract (src/stateful_llm_compiler/
// execution.py:743-781 native_kv_store, backends/triton_kv.py:10-68): row t of
// batch b goes to buffer row positions[b] + t, rows outside the capacity are
// skipped.  Pure data movement: every thread moves one UNIT-byte chunk of one
// row for both K and V, so a 128-byte bf16 head row is 8 lanes of 16-byte
// loads/stores and a wave covers 8 rows with fully coalesced accesses.
#include "common.hpp"

namespace {

template <typename U>
__global__ __launch_bounds__(256) void kv_store_kernel(
    U* __restrict__ key_buffer, U* __restrict__ value_buffer,
    const U* __restrict__ key, const U* __restrict__ value,
    const int64_t* __restrict__ positions, int* __restrict__ overflow,
    int64_t heads, int64_t tokens, int64_t row_units, int64_t capacity,
    int64_t total, int64_t k_sb,
    int64_t k_sh, int64_t k_st, int64_t v_sb, int64_t v_sh, int64_t v_st) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= total) return;
  const int64_t unit = gid % row_units;
  int64_t rest = gid / row_units;
  const int64_t t = rest % tokens;
  rest /= tokens;
  const int64_t h = rest % heads;
  const int64_t b = rest / heads;
  const int64_t position = positions[b] + t;
  if (position < 0 || position >= capacity) {
    if (overflow != nullptr) *overflow = 1;
    return;
  }
  const int64_t dst = ((b * capacity + position) * heads + h) * row_units + unit;
  key_buffer[dst] = key[b * k_sb + h * k_sh + t * k_st + unit];
  value_buffer[dst] = value[b * v_sb + h * v_sh + t * v_st + unit];
}

template <typename U>
int launch(void* kb, void* vb, const void* k, const void* v,
           const int64_t* pos, int* overflow, int64_t batch, int64_t heads, int64_t tokens,
           int64_t row_bytes, int64_t capacity, const int64_t* ks,
           const int64_t* vs, hipStream_t stream) {
  const int64_t unit = sizeof(U);
  const int64_t row_units = row_bytes / unit;
  const int64_t total = batch * heads * tokens * row_units;
  const int64_t blocks = slc_host::ceil_div(total, 256);
  hipLaunchKernelGGL(kv_store_kernel<U>, dim3(static_cast<unsigned>(blocks)),
                     dim3(256), 0, stream, static_cast<U*>(kb),
                     static_cast<U*>(vb), static_cast<const U*>(k),
                     static_cast<const U*>(v), pos, overflow, heads, tokens, row_units,
                     capacity, total, ks[0] / unit, ks[1] / unit, ks[2] / unit,
                     vs[0] / unit, vs[1] / unit, vs[2] / unit);
  return slc_host::check_launch("slc_hip_kv_store");
}

}  // namespace

extern "C" int slc_hip_kv_store(void* key_buffer, void* value_buffer,
                                const void* key, const void* value,
                                const int64_t* positions, int* overflow,
                                int dtype,
                                int64_t batch, int64_t heads, int64_t tokens,
                                int64_t head_dim, int64_t capacity,
                                int64_t key_stride_b, int64_t key_stride_h,
                                int64_t key_stride_t, int64_t value_stride_b,
                                int64_t value_stride_h, int64_t value_stride_t,
                                void* stream) {
  SLC_REQUIRE(slc_host::is_float_dtype(dtype), "slc_hip_kv_store: bad dtype %d",
              dtype);
  SLC_REQUIRE(batch >= 0 && heads > 0 && tokens >= 0 && head_dim > 0 &&
                  capacity > 0,
              "slc_hip_kv_store: bad sizes B=%lld H=%lld T=%lld D=%lld cap=%lld",
              (long long)batch, (long long)heads, (long long)tokens,
              (long long)head_dim, (long long)capacity);
  if (batch == 0 || tokens == 0) return SLC_OK;
  SLC_REQUIRE(key_buffer && value_buffer && key && value && positions,
              "slc_hip_kv_store: null pointer");
  const int64_t es = slc_host::dtype_size(dtype);
  const int64_t row_bytes = head_dim * es;
  // Strides in bytes; choose the widest unit every address is aligned to.
  const int64_t ks[3] = {key_stride_b * es, key_stride_h * es, key_stride_t * es};
  const int64_t vs[3] = {value_stride_b * es, value_stride_h * es,
                         value_stride_t * es};
  uint64_t bits = static_cast<uint64_t>(row_bytes) |
                  reinterpret_cast<uintptr_t>(key_buffer) |
                  reinterpret_cast<uintptr_t>(value_buffer) |
                  reinterpret_cast<uintptr_t>(key) |
                  reinterpret_cast<uintptr_t>(value);
  for (int i = 0; i < 3; ++i) {
    bits |= static_cast<uint64_t>(ks[i]) | static_cast<uint64_t>(vs[i]);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  if ((bits & 15) == 0)
    return launch<uint4>(key_buffer, value_buffer, key, value, positions, overflow, batch,
                         heads, tokens, row_bytes, capacity, ks, vs, s);
  if ((bits & 7) == 0)
    return launch<uint2>(key_buffer, value_buffer, key, value, positions, overflow, batch,
                         heads, tokens, row_bytes, capacity, ks, vs, s);
  if ((bits & 3) == 0)
    return launch<uint32_t>(key_buffer, value_buffer, key, value, positions, overflow,
                            batch, heads, tokens, row_bytes, capacity, ks, vs,
                            s);
  return launch<uint16_t>(key_buffer, value_buffer, key, value, positions,
                          overflow, batch, heads, tokens, row_bytes, capacity, ks, vs, s);
}
