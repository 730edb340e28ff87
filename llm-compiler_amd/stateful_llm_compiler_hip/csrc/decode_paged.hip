// Paged KV: decode attention and the KV store through a block table.
//
// The reference keeps one contiguous [B, capacity, H, D] buffer per layer and
// names a paged layout with a block table as its next step
// (docs/kv-bufferization.md:317-323; KVStateType.layout, ir.py:87).  Here the
// K and V rows of every sequence live in page pools
// [num_pages, page_tokens, kv_heads, head_dim] shared by the batch, and an
// int32 block table [B, pages_per_seq] maps page t / page_tokens of sequence b
// to its pool page.  Capacity is pages_per_seq * page_tokens.
//
// Attention runs the fixed-chunk MFMA kernel of decode_attention.hip with the
// page lookup in its tile loads (decode_kernel.hpp, PG): the same chunks, the
// same arithmetic, so a paged call equals the contiguous call over the same
// tokens bit for bit.  The store writes each new row at its position's page.
#include "common.hpp"
#include "decode_kernel.hpp"
#include "decode_tiles.hpp"

namespace {

using namespace slc_decode;

int page_shift_of(int64_t page_tokens) {
  if (page_tokens < 16 || page_tokens > (int64_t{1} << 20) ||
      (page_tokens & (page_tokens - 1)) != 0)
    return -1;
  int shift = 0;
  while ((int64_t{1} << shift) < page_tokens) ++shift;
  return shift;
}

// PGM: the kernel's page regime (1: pages hold whole 32-token tiles, 2:
// 16-token pages).
template <typename T, int D, int PGM>
int launch_paged(const void* query, const void* kp, const void* vp, const void* lengths,
                 int lengths_dtype, const void* mask, int mask_dtype, void* output,
                 void* workspace, int* counters, int64_t batch, int64_t q_heads,
                 int64_t kv_heads, int64_t capacity, int64_t mask_len, const int64_t* st,
                 float scale, int64_t chunk, int64_t nchunks, bool exact, const Paging& pg,
                 hipStream_t stream, const RopeStore* rope = nullptr) {
  float* part_o = nullptr;
  float* part_ml = nullptr;
  if (nchunks > 1) {
    part_o = static_cast<float*>(workspace);
    part_ml = part_o + batch * q_heads * nchunks * D;
  }
  const int groups = static_cast<int>(q_heads / kv_heads);
  const dim3 grid(static_cast<unsigned>(nchunks), static_cast<unsigned>(kv_heads),
                  static_cast<unsigned>(batch));
  int* merge = nchunks > 1 && SLC_DECODE_FUSED_MERGE &&
                       (2 * groups * nchunks + groups) * 4 <= SharedLayout<T, D>::kBytes
                   ? counters
                   : nullptr;
  const size_t dyn_lds =
      exact ? static_cast<size_t>(exact_dyn_bytes<T, D>()) : 0;
  RopeStore rs{};
#define SLC_PAGED_K(MK, L64, ROPE, EX)                                                      \
  do {                                                                                      \
    if (EX && exact_lds_limit<T, D, MK, L64, ROPE, EX, PGM>(static_cast<int>(dyn_lds)) !=   \
                  hipSuccess)                                                               \
      return slc_host::check_launch("slc_hip_paged_decode_attention(exact LDS opt-in)");    \
    hipLaunchKernelGGL((decode_attention_mfma_kernel<T, D, MK, L64, ROPE, EX, PGM>), grid,  \
                       dim3(kThreads), dyn_lds, stream, static_cast<const T*>(query),       \
                       static_cast<const T*>(kp), static_cast<const T*>(vp), lengths,       \
                       lengths_dtype, mask, mask_dtype, static_cast<T*>(output), part_o,    \
                       part_ml, static_cast<int>(q_heads), static_cast<int>(kv_heads),      \
                       groups, capacity, mask_len, st[0], st[1], int64_t{0},                \
                       static_cast<int>(st[3]), st[4], st[5], static_cast<int>(st[6]),      \
                       st[7], st[8], scale, static_cast<int>(chunk),                        \
                       static_cast<int>(nchunks), merge, rs, pg);                           \
  } while (0)
#define SLC_PAGED_ORDER(MK, L64, ROPE) \
  if (exact) {                         \
    SLC_PAGED_K(MK, L64, ROPE, true);  \
  } else {                             \
    SLC_PAGED_K(MK, L64, ROPE, false); \
  }
#define SLC_PAGED_MASK(L64, ROPE)              \
  if (mask == nullptr) {                       \
    SLC_PAGED_ORDER(0, L64, ROPE)              \
  } else if (mask_dtype == SLC_BF16) {         \
    SLC_PAGED_ORDER(SLC_BF16 + 1, L64, ROPE)   \
  } else if (mask_dtype == SLC_F16) {          \
    SLC_PAGED_ORDER(SLC_F16 + 1, L64, ROPE)    \
  } else {                                     \
    SLC_PAGED_ORDER(SLC_F32 + 1, L64, ROPE)    \
  }
  if (rope != nullptr) {
    // The RoPE variant: int64 lengths; its length advance rides on the
    // in-kernel merge (or, with one chunk, on the workgroup's end).
    if (lengths_dtype != SLC_I64 || (nchunks > 1 && merge == nullptr)) return kUnsupported;
    rs = *rope;
    rs.counters = counters + batch * kv_heads;
    SLC_PAGED_MASK(true, true)
    return slc_host::check_launch("slc_hip_paged_rope_decode_attention");
  }
  slc_host::mark_kernel_begin(stream);
  for (int rep = slc_host::timed_repeats(); rep > 0; --rep) {
    if (lengths_dtype == SLC_I64) {
      SLC_PAGED_MASK(true, false)
    } else {
      SLC_PAGED_MASK(false, false)
    }
  }
  slc_host::mark_kernel_end(stream);
#undef SLC_PAGED_MASK
#undef SLC_PAGED_ORDER
#undef SLC_PAGED_K
  const int rc = slc_host::check_launch("slc_hip_paged_decode_attention");
  if (rc != SLC_OK || nchunks == 1 || merge != nullptr) return rc;
  hipLaunchKernelGGL((decode_attention_merge_kernel<T, D>),
                     dim3(static_cast<unsigned>(batch * kv_heads)), dim3(256), 0, stream, part_o,
                     part_ml, static_cast<T*>(output), static_cast<int>(q_heads),
                     static_cast<int>(kv_heads), groups, st[7], st[8],
                     static_cast<int>(nchunks));
  return slc_host::check_launch("slc_hip_paged_decode_attention(merge)");
}

// One thread per 16-byte unit of one (b, h, t) row: the row of position
// positions[b] + t goes to its page; positions outside [0, capacity) are
// dropped and flagged, as the contiguous store does.
__global__ __launch_bounds__(256) void paged_kv_store_kernel(
    uint4* __restrict__ key_pool, uint4* __restrict__ value_pool, const int* __restrict__ table,
    int64_t table_sb, int page_shift, int64_t page_stride_u, int64_t row_stride_u,
    int64_t head_stride_u, const uint4* __restrict__ key, const uint4* __restrict__ value,
    const int64_t* __restrict__ positions, int* __restrict__ overflow, int64_t heads,
    int64_t tokens, int64_t row_units, int64_t capacity, int64_t total, int64_t k_sb,
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
  const int64_t page = table[b * table_sb + (position >> page_shift)];
  const int64_t dst = page * page_stride_u +
                      (position & ((int64_t{1} << page_shift) - 1)) * row_stride_u +
                      h * head_stride_u + unit;
  key_pool[dst] = key[b * k_sb + h * k_sh + t * k_st + unit];
  value_pool[dst] = value[b * v_sb + h * v_sh + t * v_st + unit];
}

}  // namespace

extern "C" int slc_hip_paged_decode_attention(
    const void* query, const void* key_pool, const void* value_pool, const int* block_table,
    int64_t table_stride_b, int64_t pages_per_seq, int64_t page_tokens, int64_t page_stride,
    const void* lengths, int lengths_dtype, const void* mask, int mask_dtype, void* output,
    void* workspace, int64_t workspace_bytes, int* counters, int64_t num_counters, int dtype,
    int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t mask_len,
    int64_t q_stride_b, int64_t q_stride_h, int64_t kv_stride_s, int64_t kv_stride_h,
    int64_t mask_stride_b, int64_t mask_stride_s, int64_t out_stride_b, int64_t out_stride_h,
    float scale, int64_t split_tokens, int softmax_order, void* stream) {
  SLC_REQUIRE(dtype == SLC_BF16 || dtype == SLC_F16,
              "slc_hip_paged_decode_attention: bf16 or fp16 only, got dtype %d", dtype);
  SLC_REQUIRE(head_dim == 64 || head_dim == 128,
              "slc_hip_paged_decode_attention: head_dim 64 or 128, got %lld", (long long)head_dim);
  SLC_REQUIRE(lengths_dtype == SLC_I64 || lengths_dtype == SLC_I32,
              "slc_hip_paged_decode_attention: lengths must be int64 or int32");
  SLC_REQUIRE(mask == nullptr || slc_host::is_float_dtype(mask_dtype),
              "slc_hip_paged_decode_attention: bad mask dtype %d", mask_dtype);
  SLC_REQUIRE(softmax_order == SLC_SOFTMAX_ONLINE || softmax_order == SLC_SOFTMAX_EXACT,
              "slc_hip_paged_decode_attention: bad softmax order %d", softmax_order);
  SLC_REQUIRE(batch >= 0 && q_heads > 0 && kv_heads > 0 && q_heads % kv_heads == 0 &&
                  q_heads / kv_heads <= kMaxGroups && pages_per_seq > 0 && mask_len > 0,
              "slc_hip_paged_decode_attention: bad sizes");
  const int shift = page_shift_of(page_tokens);
  SLC_REQUIRE(shift >= 0, "slc_hip_paged_decode_attention: page_tokens must be a power of two "
                          ">= 16, got %lld", (long long)page_tokens);
  const int64_t capacity = pages_per_seq * page_tokens;
  SLC_REQUIRE(batch <= 65535 && kv_heads <= 65535 && capacity < (int64_t{1} << 30) &&
                  page_tokens * kv_stride_s * 2 < (int64_t{1} << 31) &&
                  mask_len * mask_stride_s * (mask == nullptr ? 0 : slc_host::dtype_size(mask_dtype)) <
                      (int64_t{1} << 31),
              "slc_hip_paged_decode_attention: sizes exceed the kernel's index range");
  if (batch == 0) return SLC_OK;
  SLC_REQUIRE(query && key_pool && value_pool && block_table && lengths && output,
              "slc_hip_paged_decode_attention: null pointer");
  const uint64_t bits = reinterpret_cast<uintptr_t>(query) |
                        reinterpret_cast<uintptr_t>(key_pool) |
                        reinterpret_cast<uintptr_t>(value_pool);
  const int64_t strides = q_stride_b | q_stride_h | kv_stride_s | kv_stride_h | page_stride;
  SLC_REQUIRE((bits & 15) == 0 && (strides & 7) == 0 && kv_stride_s > 0 && mask_stride_s >= 0,
              "slc_hip_paged_decode_attention: rows must be 16-byte aligned");
  const bool exact = softmax_order == SLC_SOFTMAX_EXACT;
  SLC_REQUIRE(!exact || std::min(mask_len, capacity) <= exact_max_tokens(head_dim),
              "slc_hip_paged_decode_attention: the exact softmax order takes at most %lld tokens",
              (long long)exact_max_tokens(head_dim));
  int64_t chunk, nchunks;
  if (exact) {
    chunk = mask_len;
    nchunks = 1;
  } else {
    chunk = choose_chunk(batch, kv_heads, mask_len, split_tokens > 0 ? split_tokens : 0);
    nchunks = slc_host::ceil_div(mask_len, chunk);
  }
  const int64_t need = partial_bytes(batch, q_heads, head_dim, nchunks);
  SLC_REQUIRE(need == 0 || (workspace != nullptr && workspace_bytes >= need),
              "slc_hip_paged_decode_attention: workspace of %lld bytes needed, got %lld",
              (long long)need, (long long)workspace_bytes);
  SLC_REQUIRE(counters != nullptr && num_counters >= counter_count(batch, kv_heads),
              "slc_hip_paged_decode_attention: %lld counters needed, got %lld",
              (long long)counter_count(batch, kv_heads), (long long)num_counters);
  // kv_sb has no meaning for pools (the page comes from the table); slot 2 of
  // the stride set is left 0.
  const int64_t st[9] = {q_stride_b,    q_stride_h,    0,            kv_stride_s, kv_stride_h,
                         mask_stride_b, mask_stride_s, out_stride_b, out_stride_h};
  const Paging pg{block_table, table_stride_b, shift, page_stride};
  hipStream_t s = static_cast<hipStream_t>(stream);
#define SLC_PAGED_CALL(TT, DD)                                                              \
  (shift >= 5 ? launch_paged<TT, DD, 1> : launch_paged<TT, DD, 2>)(                          \
      query, key_pool, value_pool, lengths, lengths_dtype, mask, mask_dtype, output, workspace, \
      counters, batch, q_heads, kv_heads, capacity, mask_len, st, scale, chunk, nchunks, exact, \
      pg, s, nullptr)
  if (dtype == SLC_BF16) {
    if (head_dim == 64) return SLC_PAGED_CALL(slc::bf16_t, 64);
    return SLC_PAGED_CALL(slc::bf16_t, 128);
  }
  if (head_dim == 64) return SLC_PAGED_CALL(slc::f16_t, 64);
  return SLC_PAGED_CALL(slc::f16_t, 128);
#undef SLC_PAGED_CALL
}

extern "C" int slc_hip_paged_kv_store(
    void* key_pool, void* value_pool, const int* block_table, int64_t table_stride_b,
    int64_t pages_per_seq, int64_t page_tokens, int64_t page_stride, int64_t kv_stride_s,
    int64_t kv_stride_h, const void* key, const void* value, const int64_t* positions,
    int* overflow, int dtype, int64_t batch, int64_t heads, int64_t tokens, int64_t head_dim,
    int64_t key_stride_b, int64_t key_stride_h, int64_t key_stride_t, int64_t value_stride_b,
    int64_t value_stride_h, int64_t value_stride_t, void* stream) {
  SLC_REQUIRE(slc_host::is_float_dtype(dtype), "slc_hip_paged_kv_store: bad dtype %d", dtype);
  const int shift = page_shift_of(page_tokens);
  SLC_REQUIRE(shift >= 0, "slc_hip_paged_kv_store: page_tokens must be a power of two >= 16");
  SLC_REQUIRE(batch >= 0 && heads > 0 && tokens >= 0 && head_dim > 0 && pages_per_seq > 0,
              "slc_hip_paged_kv_store: bad sizes");
  if (batch == 0 || tokens == 0) return SLC_OK;
  SLC_REQUIRE(key_pool && value_pool && block_table && key && value && positions,
              "slc_hip_paged_kv_store: null pointer");
  const int64_t es = slc_host::dtype_size(dtype);
  const int64_t row_bytes = head_dim * es;
  uint64_t bits = static_cast<uint64_t>(row_bytes) | reinterpret_cast<uintptr_t>(key_pool) |
                  reinterpret_cast<uintptr_t>(value_pool) | reinterpret_cast<uintptr_t>(key) |
                  reinterpret_cast<uintptr_t>(value);
  const int64_t strides[8] = {page_stride, kv_stride_s,   kv_stride_h,    key_stride_b,
                              key_stride_h, key_stride_t, value_stride_b, value_stride_h};
  for (int64_t v : strides) bits |= static_cast<uint64_t>(v * es);
  bits |= static_cast<uint64_t>(value_stride_t * es);
  SLC_REQUIRE((bits & 15) == 0,
              "slc_hip_paged_kv_store: rows, strides and pointers must be 16-byte aligned");
  const int64_t u = 16 / es;  // elements per 16-byte unit
  const int64_t row_units = row_bytes / 16;
  const int64_t total = batch * heads * tokens * row_units;
  SLC_REQUIRE(slc_host::ceil_div(total, 256) <= INT32_MAX,
              "slc_hip_paged_kv_store: %lld rows of 16-byte units exceed one launch's grid",
              (long long)total);
  hipLaunchKernelGGL(paged_kv_store_kernel, dim3(static_cast<unsigned>(slc_host::ceil_div(total, 256))),
                     dim3(256), 0, static_cast<hipStream_t>(stream), static_cast<uint4*>(key_pool),
                     static_cast<uint4*>(value_pool), block_table, table_stride_b, shift,
                     page_stride / u, kv_stride_s / u, kv_stride_h / u,
                     static_cast<const uint4*>(key), static_cast<const uint4*>(value), positions,
                     overflow, heads, tokens, row_units, pages_per_seq * page_tokens, total,
                     key_stride_b / u, key_stride_h / u, key_stride_t / u, value_stride_b / u,
                     value_stride_h / u, value_stride_t / u);
  return slc_host::check_launch("slc_hip_paged_kv_store");
}

extern "C" int slc_hip_paged_rope_decode_attention(
    const void* query, const void* key, const void* value, const void* cosine, const void* sine,
    void* key_pool, void* value_pool, const int* block_table, int64_t table_stride_b,
    int64_t pages_per_seq, int64_t page_tokens, int64_t page_stride, const int64_t* lengths,
    int64_t* lengths_out, int* overflow, const void* mask, int mask_dtype, void* output,
    void* workspace, int64_t workspace_bytes, int* counters, int64_t num_counters, int dtype,
    int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t mask_len,
    int64_t q_stride_b, int64_t q_stride_h, int64_t k_stride_b, int64_t k_stride_h,
    int64_t v_stride_b, int64_t v_stride_h, int64_t cos_stride_b, int64_t sin_stride_b,
    int64_t kv_stride_s, int64_t kv_stride_h, int64_t mask_stride_b, int64_t mask_stride_s,
    int64_t out_stride_b, int64_t out_stride_h, float scale, int softmax_order, void* stream) {
  SLC_REQUIRE(mask == nullptr || slc_host::is_float_dtype(mask_dtype),
              "slc_hip_paged_rope_decode_attention: bad mask dtype %d", mask_dtype);
  SLC_REQUIRE(softmax_order == SLC_SOFTMAX_ONLINE || softmax_order == SLC_SOFTMAX_EXACT,
              "slc_hip_paged_rope_decode_attention: bad softmax order %d", softmax_order);
  SLC_REQUIRE(batch >= 0 && q_heads > 0 && kv_heads > 0 && head_dim > 0 && pages_per_seq > 0 &&
                  mask_len >= 0 && q_heads % kv_heads == 0,
              "slc_hip_paged_rope_decode_attention: bad sizes");
  SLC_REQUIRE(batch <= 65535 && kv_heads <= 65535,
              "slc_hip_paged_rope_decode_attention: batch/kv_heads exceed grid limits");
  const int shift = page_shift_of(page_tokens);
  SLC_REQUIRE(shift >= 0, "slc_hip_paged_rope_decode_attention: page_tokens must be a power of "
                          "two >= 16, got %lld", (long long)page_tokens);
  if (batch == 0) return SLC_OK;
  SLC_REQUIRE(query && key && value && cosine && sine && key_pool && value_pool && block_table &&
                  lengths && lengths_out && output,
              "slc_hip_paged_rope_decode_attention: null pointer");
  const bool exact = softmax_order == SLC_SOFTMAX_EXACT;
  const int64_t groups = q_heads / kv_heads;
  const int64_t capacity = pages_per_seq * page_tokens;
  // The fused kernel's cases; everything else is the caller's three-kernel
  // path (RoPE, paged store, paged attention).
  if (!(dtype == SLC_BF16 || dtype == SLC_F16) || !(head_dim == 64 || head_dim == 128) ||
      groups > kMaxGroups || mask_len <= 0)
    return kUnsupported;
  if (exact && std::min(mask_len, capacity) > exact_max_tokens(head_dim)) return kUnsupported;
  const uint64_t bits =
      reinterpret_cast<uintptr_t>(query) | reinterpret_cast<uintptr_t>(key) |
      reinterpret_cast<uintptr_t>(value) | reinterpret_cast<uintptr_t>(cosine) |
      reinterpret_cast<uintptr_t>(sine) | reinterpret_cast<uintptr_t>(key_pool) |
      reinterpret_cast<uintptr_t>(value_pool);
  const int64_t strides = q_stride_b | q_stride_h | k_stride_b | k_stride_h | v_stride_b |
                          v_stride_h | cos_stride_b | sin_stride_b | kv_stride_s | kv_stride_h |
                          page_stride;
  const int64_t mask_es = mask == nullptr ? 0 : slc_host::dtype_size(mask_dtype);
  if ((bits & 15) != 0 || (strides & 7) != 0 || kv_stride_s <= 0 || mask_stride_s < 0 ||
      page_tokens * kv_stride_s * 2 >= (int64_t{1} << 31) ||
      mask_len * mask_stride_s * mask_es >= (int64_t{1} << 31) || capacity >= (int64_t{1} << 30))
    return kUnsupported;
  int64_t chunk, nchunks;
  if (exact) {
    chunk = mask_len;
    nchunks = 1;
  } else {
    chunk = choose_chunk(batch, kv_heads, mask_len, 0);
    nchunks = slc_host::ceil_div(mask_len, chunk);
  }
  const int64_t need = partial_bytes(batch, q_heads, head_dim, nchunks);
  SLC_REQUIRE(need == 0 || (workspace != nullptr && workspace_bytes >= need),
              "slc_hip_paged_rope_decode_attention: workspace of %lld bytes needed, got %lld",
              (long long)need, (long long)workspace_bytes);
  SLC_REQUIRE(counters != nullptr && num_counters >= counter_count(batch, kv_heads),
              "slc_hip_paged_rope_decode_attention: %lld counters needed, got %lld",
              (long long)counter_count(batch, kv_heads), (long long)num_counters);
  const int64_t st[9] = {q_stride_b,    q_stride_h,    0,            kv_stride_s, kv_stride_h,
                         mask_stride_b, mask_stride_s, out_stride_b, out_stride_h};
  const Paging pg{block_table, table_stride_b, shift, page_stride};
  RopeStore rope{key,          value,        cosine,      sine,         k_stride_b,
                 k_stride_h,   v_stride_b,   v_stride_h,  cos_stride_b, sin_stride_b,
                 key_pool,     value_pool,   lengths_out, overflow,     nullptr};
  hipStream_t s = static_cast<hipStream_t>(stream);
#define SLC_PAGED_ROPE_CALL(TT, DD)                                                              \
  (shift >= 5 ? launch_paged<TT, DD, 1> : launch_paged<TT, DD, 2>)(                              \
      query, key_pool, value_pool, lengths, SLC_I64, mask, mask_dtype, output, workspace,        \
      counters, batch, q_heads, kv_heads, capacity, mask_len, st, scale, chunk, nchunks, exact, \
      pg, s, &rope)
  if (dtype == SLC_BF16) {
    if (head_dim == 64) return SLC_PAGED_ROPE_CALL(slc::bf16_t, 64);
    return SLC_PAGED_ROPE_CALL(slc::bf16_t, 128);
  }
  if (head_dim == 64) return SLC_PAGED_ROPE_CALL(slc::f16_t, 64);
  return SLC_PAGED_ROPE_CALL(slc::f16_t, 128);
#undef SLC_PAGED_ROPE_CALL
}
