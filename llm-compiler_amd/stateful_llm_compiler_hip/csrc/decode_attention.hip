// decode_attention: single-token GQA attention over the preallocated KV buffers.
//
// Semantics follow the reference (src/stateful_llm_compiler/execution.py:281-327
// for the math, backends/triton_attention.py:10-131 for the fast-path contract):
//   out[b,h,:] = sum_s softmax_s(scale * q[b,h].k[b,s,h/g] + mask[b,s]) v[b,s,h/g]
// over s < min(lengths[b], mask_len, capacity), accumulated in fp32.
//
// MI355X design (bf16/fp16, head_dim 64 or 128, up to 16 query heads per KV head):
//  * One workgroup = 4 wavefronts per (batch, kv-head, sequence chunk).  All the
//    query heads of a GQA group are the 16 columns of one MFMA tile, so every
//    K/V byte is read from HBM exactly once (the reference re-reads each KV row
//    once per query head).
//  * Each wave walks 32-token tiles.  S^T[token, head] = K . Q^T is two
//    v_mfma_f32_16x16x32 per 16 tokens with K rows loaded straight from HBM
//    into the A operand (16-byte loads).  The online softmax runs on the MFMA
//    output registers; the max needs two cross-lane shuffles per tile.
//  * O^T[dim, head] += V^T . P^T.  The MFMA reduction index is a permutation of
//    the tile's tokens chosen so that the P operand is exactly the lane's own
//    softmax registers; V is staged through LDS (coalesced 16-byte writes,
//    2-byte transposed reads on a bank-conflict-free padded layout).
//  * Long sequences are split into chunks (split-sequence / flash-decoding) so a
//    batch-32 decode still launches hundreds of workgroups for 256 CUs.  Each
//    chunk writes its (max, sum, acc) partial and a small second kernel merges
//    them.  (Merging inside the first kernel needs an agent-scope release per
//    workgroup -- an L2 write-back -- which measured several times slower than
//    the extra launch.)
//  * Loops stop at the batch's own length, not at the capacity.
// Other dtypes/shapes take a straightforward wave-per-token kernel.
#include <algorithm>
#include <climits>
#include <mutex>
#include <type_traits>

#include "common.hpp"
#include "decode_kernel.hpp"
#include "decode_tiles.hpp"
#include "op_math.hpp"

namespace {

using namespace slc_decode;

template <typename T, int D>
int launch_mfma(const void* query, const void* kb, const void* vb,
                const void* lengths, int lengths_dtype, const void* mask,
                int mask_dtype, void* output, void* workspace, int* counters, int64_t batch,
                int64_t q_heads, int64_t kv_heads, int64_t capacity,
                int64_t mask_len, const int64_t* st, float scale,
                int64_t chunk, int64_t nchunks, bool exact, hipStream_t stream,
                const RopeStore* rope = nullptr) {
  int* advance = counters + batch * kv_heads;
  float* part_o = nullptr;
  float* part_ml = nullptr;
  if (nchunks > 1) {
    part_o = static_cast<float*>(workspace);
    part_ml = part_o + batch * q_heads * nchunks * D;
  }
  const int groups = static_cast<int>(q_heads / kv_heads);
  const dim3 grid(static_cast<unsigned>(nchunks), static_cast<unsigned>(kv_heads),
                  static_cast<unsigned>(batch));
  // Merge inside the split kernel when the chunk weights fit the kernel's
  // LDS; else the separate merge kernel.
  int* merge = nchunks > 1 && SLC_DECODE_FUSED_MERGE &&
                       (2 * groups * nchunks + groups) * 4 <= SharedLayout<T, D>::kBytes
                   ? counters
                   : nullptr;
  const size_t dyn_lds =
      exact ? static_cast<size_t>(exact_dyn_bytes<T, D>()) : 0;
#define SLC_MFMA_K(MK, L64, ROPE, EX)                                                      \
  do {                                                                                     \
    if (EX && exact_lds_limit<T, D, MK, L64, ROPE, EX>(static_cast<int>(dyn_lds)) != hipSuccess) \
      return slc_host::check_launch("slc_hip_decode_attention(exact LDS opt-in)");         \
    hipLaunchKernelGGL((decode_attention_mfma_kernel<T, D, MK, L64, ROPE, EX>), grid,     \
                       dim3(kThreads), dyn_lds, stream, static_cast<const T*>(query),      \
                       static_cast<const T*>(kb), static_cast<const T*>(vb), lengths,      \
                       lengths_dtype, mask, mask_dtype, static_cast<T*>(output), part_o,   \
                       part_ml, static_cast<int>(q_heads), static_cast<int>(kv_heads),     \
                       groups, capacity, mask_len, st[0], st[1], st[2],                    \
                       static_cast<int>(st[3]), st[4], st[5], static_cast<int>(st[6]),     \
                       st[7], st[8], scale, static_cast<int>(chunk),                       \
                       static_cast<int>(nchunks), merge, rs, Paging{});                    \
  } while (0)
#define SLC_MFMA_ORDER(MK, L64, ROPE)     \
  if (exact) {                            \
    SLC_MFMA_K(MK, L64, ROPE, true);      \
  } else {                                \
    SLC_MFMA_K(MK, L64, ROPE, false);     \
  }
  RopeStore rs{};
  if (rope != nullptr) {
    // The advance rides on the in-kernel merge (or, with one chunk, on the
    // workgroup's end); int64 lengths only.
    if (lengths_dtype != SLC_I64 || (nchunks > 1 && merge == nullptr)) return kUnsupported;
    rs = *rope;
    rs.counters = advance;
#define SLC_ROPE(MK) SLC_MFMA_ORDER(MK, true, true)
    if (mask == nullptr) {
      SLC_ROPE(0);
    } else if (mask_dtype == SLC_BF16) {
      SLC_ROPE(SLC_BF16 + 1);
    } else if (mask_dtype == SLC_F16) {
      SLC_ROPE(SLC_F16 + 1);
    } else {
      SLC_ROPE(SLC_F32 + 1);
    }
#undef SLC_ROPE
    return slc_host::check_launch("slc_hip_rope_decode_attention");
  }
  slc_host::mark_kernel_begin(stream);
#define SLC_MFMA(MK)                          \
  if (lengths_dtype == SLC_I64) {             \
    SLC_MFMA_ORDER(MK, true, false);          \
  } else {                                    \
    SLC_MFMA_ORDER(MK, false, false);         \
  }
  for (int rep = slc_host::timed_repeats(); rep > 0; --rep) {
    if (mask == nullptr) {
      SLC_MFMA(0);
    } else if (mask_dtype == SLC_BF16) {
      SLC_MFMA(SLC_BF16 + 1);
    } else if (mask_dtype == SLC_F16) {
      SLC_MFMA(SLC_F16 + 1);
    } else {
      SLC_MFMA(SLC_F32 + 1);
    }
  }
#undef SLC_MFMA
#undef SLC_MFMA_ORDER
#undef SLC_MFMA_K
  slc_host::mark_kernel_end(stream);
  int rc = slc_host::check_launch("slc_hip_decode_attention");
  if (rc != SLC_OK || nchunks == 1 || merge != nullptr) return rc;
  hipLaunchKernelGGL((decode_attention_merge_kernel<T, D>),
                     dim3(static_cast<unsigned>(batch * kv_heads)), dim3(256), 0,
                     stream, part_o, part_ml, static_cast<T*>(output),
                     static_cast<int>(q_heads), static_cast<int>(kv_heads), groups,
                     st[7], st[8], static_cast<int>(nchunks));
  return slc_host::check_launch("slc_hip_decode_attention(merge)");
}

template <typename T>
int launch_generic(const void* query, const void* kb, const void* vb,
                   const void* lengths, int lengths_dtype, const void* mask,
                   int mask_dtype, void* output, int64_t batch, int64_t q_heads,
                   int64_t kv_heads, int64_t head_dim, int64_t capacity,
                   int64_t mask_len, const int64_t* st, float scale, bool exact,
                   hipStream_t stream) {
  const int groups = static_cast<int>(q_heads / kv_heads);
  const dim3 grid(static_cast<unsigned>(batch * q_heads));
#define SLC_GENERIC_K(NI, EX)                                                          \
  hipLaunchKernelGGL((decode_attention_generic_kernel<T, NI, EX>), grid, dim3(256),    \
                     0, stream, static_cast<const T*>(query),                          \
                     static_cast<const T*>(kb), static_cast<const T*>(vb),             \
                     lengths, lengths_dtype, mask, mask_dtype,                         \
                     static_cast<T*>(output), static_cast<int>(q_heads),               \
                     groups, static_cast<int>(head_dim), capacity, mask_len,           \
                     st[0], st[1], st[2], st[3], st[4], st[5], st[6], st[7],           \
                     st[8], scale)
#define SLC_GENERIC(NI)          \
  if (exact) {                   \
    SLC_GENERIC_K(NI, true);     \
  } else {                       \
    SLC_GENERIC_K(NI, false);    \
  }
  if (head_dim <= 64) {
    SLC_GENERIC(1);
  } else if (head_dim <= 128) {
    SLC_GENERIC(2);
  } else {
    SLC_GENERIC(4);
  }
#undef SLC_GENERIC
#undef SLC_GENERIC_K
  return slc_host::check_launch("slc_hip_decode_attention(generic)");
}

// Geometry of one call: which kernel, the split, and the workspace it needs.
struct Plan {
  bool mfma;
  bool stream;       // balanced split (decode_stream.hip)
  int64_t chunk, nchunks;
  int64_t need;      // workspace bytes (partials)
  int64_t counters;  // counter ints, 0 for the generic kernel
};

// split_tokens: 0 = fixed chunk sized for the grid, > 0 = fixed chunk of that
// many tokens, SLC_SPLIT_BALANCED = the length-balanced split (decode_stream.hip;
// online order, where it fits -- else the automatic fixed chunk).
Plan plan_call(int dtype, int64_t batch, int64_t q_heads, int64_t kv_heads,
               int64_t head_dim, int64_t mask_len, int64_t capacity, int64_t split_tokens,
               bool exact, bool allow_stream = true) {
  Plan p{false, false, 0, 1, 0, 0};
  p.mfma = mfma_eligible(dtype, head_dim, q_heads / kv_heads) && mask_len > 0;
  if (!p.mfma) return p;
  if (allow_stream && !exact && split_tokens == SLC_SPLIT_BALANCED &&
      stream_eligible(batch, kv_heads, q_heads / kv_heads, mask_len, capacity)) {
    p.stream = true;
    p.need = stream_workspace_bytes(q_heads, kv_heads, head_dim);
    p.counters = counter_count(batch, kv_heads);
    return p;
  }
  if (exact) {
    p.chunk = mask_len;
    p.nchunks = 1;
  } else {
    p.chunk = choose_chunk(batch, kv_heads, mask_len, split_tokens);
    p.nchunks = slc_host::ceil_div(mask_len, p.chunk);
  }
  p.need = partial_bytes(batch, q_heads, head_dim, p.nchunks);
  p.counters = counter_count(batch, kv_heads);
  return p;
}

}  // namespace

extern "C" int64_t slc_hip_decode_attention_workspace_size(
    int64_t batch, int64_t q_heads, int64_t head_dim, int64_t mask_len,
    int64_t kv_heads, int dtype, int64_t split_tokens) {
  if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || mask_len <= 0 ||
      q_heads % kv_heads != 0) {
    return 0;
  }
  // The online split needs at least what the exact single-chunk form does.
  // Enough for either split (the balanced one may decline at the call's
  // capacity and take the fixed-chunk grid).
  const int64_t fixed =
      plan_call(dtype, batch, q_heads, kv_heads, head_dim, mask_len, mask_len, split_tokens,
                false, false).need;
  const int64_t balanced =
      plan_call(dtype, batch, q_heads, kv_heads, head_dim, mask_len, mask_len, split_tokens,
                false).need;
  return std::max(fixed, balanced);
}

extern "C" int64_t slc_hip_decode_attention_counter_count(int64_t batch, int64_t kv_heads) {
  return batch > 0 && kv_heads > 0 ? counter_count(batch, kv_heads) : 0;
}

extern "C" int64_t slc_hip_decode_attention_exact_max_tokens(int64_t head_dim, int dtype) {
  if (dtype == SLC_BF16 || dtype == SLC_F16) {
    if (head_dim == 64 || head_dim == 128) return exact_max_tokens(head_dim);
  }
  return INT64_MAX;  // the generic kernel takes any length in both orders
}

extern "C" int slc_hip_decode_attention(
    const void* query, const void* key_buffer, const void* value_buffer,
    const void* lengths, int lengths_dtype, const void* mask, int mask_dtype,
    void* output, void* workspace, int64_t workspace_bytes, int* counters,
    int64_t num_counters, int dtype, int64_t batch, int64_t q_heads, int64_t kv_heads,
    int64_t head_dim, int64_t capacity, int64_t mask_len, int64_t q_stride_b,
    int64_t q_stride_h, int64_t kv_stride_b, int64_t kv_stride_s, int64_t kv_stride_h,
    int64_t mask_stride_b, int64_t mask_stride_s, int64_t out_stride_b,
    int64_t out_stride_h, float scale, int64_t split_tokens, int softmax_order,
    void* stream) {
  SLC_REQUIRE(slc_host::is_float_dtype(dtype),
              "slc_hip_decode_attention: bad dtype %d", dtype);
  SLC_REQUIRE(lengths_dtype == SLC_I64 || lengths_dtype == SLC_I32,
              "slc_hip_decode_attention: lengths must be int64 or int32");
  SLC_REQUIRE(mask == nullptr || slc_host::is_float_dtype(mask_dtype),
              "slc_hip_decode_attention: bad mask dtype %d", mask_dtype);
  SLC_REQUIRE(softmax_order == SLC_SOFTMAX_ONLINE || softmax_order == SLC_SOFTMAX_EXACT,
              "slc_hip_decode_attention: bad softmax order %d", softmax_order);
  SLC_REQUIRE(batch >= 0 && q_heads > 0 && kv_heads > 0 && head_dim > 0 &&
                  capacity > 0 && mask_len >= 0,
              "slc_hip_decode_attention: bad sizes");
  SLC_REQUIRE(q_heads % kv_heads == 0,
              "slc_hip_decode_attention: q_heads %lld not a multiple of "
              "kv_heads %lld",
              (long long)q_heads, (long long)kv_heads);
  SLC_REQUIRE(head_dim <= 256, "slc_hip_decode_attention: head_dim > 256");
  SLC_REQUIRE(batch <= 65535 && kv_heads <= 65535,
              "slc_hip_decode_attention: batch/kv_heads exceed grid limits");
  if (batch == 0) return SLC_OK;
  SLC_REQUIRE(query && key_buffer && value_buffer && lengths && output,
              "slc_hip_decode_attention: null pointer");
  const bool exact = softmax_order == SLC_SOFTMAX_EXACT;
  const int64_t st[9] = {q_stride_b,    q_stride_h,    kv_stride_b,
                         kv_stride_s,   kv_stride_h,   mask_stride_b,
                         mask_stride_s, out_stride_b,  out_stride_h};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t ml = mask_len;

  Plan plan =
      plan_call(dtype, batch, q_heads, kv_heads, head_dim, ml, capacity, split_tokens, exact);
  if (plan.mfma) {
    // 16-byte vector loads need 8-element alignment of every row start.
    const uint64_t bits = reinterpret_cast<uintptr_t>(query) |
                          reinterpret_cast<uintptr_t>(key_buffer) |
                          reinterpret_cast<uintptr_t>(value_buffer);
    const int64_t strides = q_stride_b | q_stride_h | kv_stride_b |
                            kv_stride_s | kv_stride_h;
    plan.mfma = (bits & 15) == 0 && (strides & 7) == 0;
    // Per-lane offsets inside one (batch, kv-head) slice are 32-bit.
    const int64_t mask_es = mask == nullptr ? 0 : slc_host::dtype_size(mask_dtype);
    plan.mfma = plan.mfma && kv_stride_s > 0 && mask_stride_s >= 0 &&
                capacity * kv_stride_s * 2 < (int64_t{1} << 31) &&
                mask_len * mask_stride_s * mask_es < (int64_t{1} << 31) &&
                capacity < (int64_t{1} << 30);
  }
  if (plan.mfma) {
    SLC_REQUIRE(!exact || std::min(ml, capacity) <= exact_max_tokens(head_dim),
                "slc_hip_decode_attention: the exact softmax order takes at most %lld tokens "
                "at head_dim %lld, got a mask of %lld",
                (long long)exact_max_tokens(head_dim), (long long)head_dim, (long long)ml);
    SLC_REQUIRE(plan.nchunks <= 0x7fffffff, "slc_hip_decode_attention: too many chunks");
    SLC_REQUIRE(plan.need == 0 || (workspace != nullptr && workspace_bytes >= plan.need),
                "slc_hip_decode_attention: workspace of %lld bytes needed, got "
                "%lld",
                (long long)plan.need, (long long)workspace_bytes);
    SLC_REQUIRE(counters != nullptr && num_counters >= plan.counters,
                "slc_hip_decode_attention: %lld counters needed, got %lld",
                (long long)plan.counters, (long long)num_counters);
    if (plan.stream) {
      StreamCall call{query,   key_buffer, value_buffer, lengths,  lengths_dtype, mask,
                      mask_dtype, output,  workspace,    counters, dtype,         batch,
                      q_heads, kv_heads,  head_dim,     capacity, ml,            {},
                      scale,   s};
      std::copy(st, st + 9, call.st);
      return launch_stream(call);
    }
#define SLC_DA_CALL(TT, DD)                                                                  \
  launch_mfma<TT, DD>(query, key_buffer, value_buffer, lengths, lengths_dtype, mask,         \
                      mask_dtype, output, workspace, counters, batch, q_heads, kv_heads,     \
                      capacity, ml, st, scale, plan.chunk, plan.nchunks, exact, s)
    if (dtype == SLC_BF16) {
      if (head_dim == 64) return SLC_DA_CALL(slc::bf16_t, 64);
      return SLC_DA_CALL(slc::bf16_t, 128);
    }
    if (head_dim == 64) return SLC_DA_CALL(slc::f16_t, 64);
    return SLC_DA_CALL(slc::f16_t, 128);
#undef SLC_DA_CALL
  }
  SLC_REQUIRE(batch * q_heads <= 0x7fffffff,
              "slc_hip_decode_attention: grid too large");
  switch (dtype) {
    case SLC_F32:
      return launch_generic<float>(query, key_buffer, value_buffer, lengths,
                                   lengths_dtype, mask, mask_dtype, output,
                                   batch, q_heads, kv_heads, head_dim, capacity,
                                   ml, st, scale, exact, s);
    case SLC_BF16:
      return launch_generic<slc::bf16_t>(query, key_buffer, value_buffer,
                                         lengths, lengths_dtype, mask,
                                         mask_dtype, output, batch, q_heads,
                                         kv_heads, head_dim, capacity, ml, st,
                                         scale, exact, s);
    default:
      return launch_generic<slc::f16_t>(query, key_buffer, value_buffer,
                                        lengths, lengths_dtype, mask, mask_dtype,
                                        output, batch, q_heads, kv_heads,
                                        head_dim, capacity, ml, st, scale, exact,
                                        s);
  }
}

// ---- decode attention without allocation ------------------------------------
// For callers that cannot allocate device memory (code under HIP graph
// capture, tight serving loops, harnesses that forbid it): the split partials
// and arrival counters live in one file-scope device array instead of a
// caller workspace.  Each GPU holds its own copy until the process ends; the
// host never passes the array's name to a kernel, only the address that
// hipGetSymbolAddress returns for the current device.
namespace {

constexpr int64_t kNoAllocCounterInts = 131072;              // 512 KiB of counters
constexpr int64_t kNoAllocPartialBytes = int64_t{8} << 20;   // 8 MiB of partials
constexpr int64_t kNoAllocBytes = kNoAllocCounterInts * 4 + kNoAllocPartialBytes;

static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

__global__ void zero_ints_kernel(int* p, int64_t n) {
  for (int64_t i = blockIdx.x * int64_t{blockDim.x} + threadIdx.x; i < n;
       i += int64_t{gridDim.x} * blockDim.x)
    p[i] = 0;
}

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
unsigned char* g_scratch_ptr[kMaxDevices] = {};

// The current device's copy of `scratch`, set up on the first call on that
// device: its address, and the counters zeroed by a small kernel on the
// caller's stream (a kernel, not a memset, so that a first call under graph
// capture records nothing a replay mishandles).  Every later call leaves the
// counters zero again.
int noalloc_scratch(hipStream_t stream, unsigned char** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    slc_host::set_error("slc_hip_decode_attention_noalloc: no usable current device");
    return SLC_ERR_INVALID_ARGUMENT;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t rc = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (rc != hipSuccess || ptr == nullptr) {
      slc_host::set_error("slc_hip_decode_attention_noalloc: hipGetSymbolAddress failed: %s",
                          hipGetErrorString(rc));
      return static_cast<int>(rc != hipSuccess ? rc : hipErrorInvalidSymbol);
    }
    hipLaunchKernelGGL(zero_ints_kernel, dim3(128), dim3(256), 0, stream,
                       static_cast<int*>(ptr), kNoAllocCounterInts);
    const int launch = slc_host::check_launch("slc_hip_decode_attention_noalloc(zero counters)");
    if (launch != SLC_OK) return launch;
    g_scratch_ptr[dev] = static_cast<unsigned char*>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return SLC_OK;
}

}  // namespace

extern "C" int slc_hip_decode_attention_noalloc(
    const void* query, const void* key_buffer, const void* value_buffer,
    const void* lengths, int lengths_dtype, const void* mask, int mask_dtype,
    void* output, int dtype, int64_t batch, int64_t q_heads, int64_t kv_heads,
    int64_t head_dim, int64_t capacity, int64_t mask_len, int64_t q_stride_b,
    int64_t q_stride_h, int64_t kv_stride_b, int64_t kv_stride_s, int64_t kv_stride_h,
    int64_t mask_stride_b, int64_t mask_stride_s, int64_t out_stride_b,
    int64_t out_stride_h, float scale, int64_t split_tokens, int softmax_order,
    void* stream) {
  // Sizes first: a call the array cannot hold fails before any device call.
  SLC_REQUIRE(batch >= 0 && q_heads > 0 && kv_heads > 0 && q_heads % kv_heads == 0 &&
                  mask_len >= 0,
              "slc_hip_decode_attention_noalloc: bad sizes");
  const int64_t partials = slc_hip_decode_attention_workspace_size(
      batch, q_heads, head_dim, mask_len, kv_heads, dtype, split_tokens);
  const int64_t counters = slc_hip_decode_attention_counter_count(batch, kv_heads);
  SLC_REQUIRE(partials <= kNoAllocPartialBytes && counters <= kNoAllocCounterInts,
              "slc_hip_decode_attention_noalloc: the call needs %lld bytes of partials and "
              "%lld counters; the no-alloc scratch holds at most %lld and %lld",
              (long long)partials, (long long)counters, (long long)kNoAllocPartialBytes,
              (long long)kNoAllocCounterInts);
  if (batch == 0) return SLC_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  unsigned char* base = nullptr;
  const int rc = noalloc_scratch(s, &base);
  if (rc != SLC_OK) return rc;
  return slc_hip_decode_attention(
      query, key_buffer, value_buffer, lengths, lengths_dtype, mask, mask_dtype, output,
      base + kNoAllocCounterInts * 4, kNoAllocPartialBytes, reinterpret_cast<int*>(base),
      kNoAllocCounterInts, dtype, batch, q_heads, kv_heads, head_dim, capacity, mask_len,
      q_stride_b, q_stride_h, kv_stride_b, kv_stride_s, kv_stride_h, mask_stride_b,
      mask_stride_s, out_stride_b, out_stride_h, scale, split_tokens, softmax_order, stream);
}

extern "C" int slc_hip_rope_decode_attention(
    const void* query, const void* key, const void* value, const void* cosine,
    const void* sine, void* key_buffer, void* value_buffer, const int64_t* lengths,
    int64_t* lengths_out, int* overflow, const void* mask, int mask_dtype, void* output,
    void* workspace, int64_t workspace_bytes, int* counters, int64_t num_counters, int dtype,
    int64_t batch, int64_t q_heads,
    int64_t kv_heads, int64_t head_dim, int64_t capacity, int64_t mask_len, int64_t q_stride_b,
    int64_t q_stride_h, int64_t k_stride_b, int64_t k_stride_h, int64_t v_stride_b,
    int64_t v_stride_h, int64_t cos_stride_b, int64_t sin_stride_b, int64_t kv_stride_b,
    int64_t kv_stride_s, int64_t kv_stride_h, int64_t mask_stride_b, int64_t mask_stride_s,
    int64_t out_stride_b, int64_t out_stride_h, float scale, int softmax_order, void* stream) {
  SLC_REQUIRE(mask == nullptr || slc_host::is_float_dtype(mask_dtype),
              "slc_hip_rope_decode_attention: bad mask dtype %d", mask_dtype);
  SLC_REQUIRE(softmax_order == SLC_SOFTMAX_ONLINE || softmax_order == SLC_SOFTMAX_EXACT,
              "slc_hip_rope_decode_attention: bad softmax order %d", softmax_order);
  SLC_REQUIRE(batch >= 0 && q_heads > 0 && kv_heads > 0 && head_dim > 0 && capacity > 0 &&
                  mask_len >= 0 && q_heads % kv_heads == 0,
              "slc_hip_rope_decode_attention: bad sizes");
  SLC_REQUIRE(batch <= 65535 && kv_heads <= 65535,
              "slc_hip_rope_decode_attention: batch/kv_heads exceed grid limits");
  if (batch == 0) return SLC_OK;
  SLC_REQUIRE(query && key && value && cosine && sine && key_buffer && value_buffer && lengths &&
                  lengths_out && output,
              "slc_hip_rope_decode_attention: null pointer");
  const bool exact = softmax_order == SLC_SOFTMAX_EXACT;
  const int64_t groups = q_heads / kv_heads;
  // The fused kernel's cases; everything else is the caller's two-kernel path.
  if (!mfma_eligible(dtype, head_dim, groups) || mask_len <= 0) return kUnsupported;
  if (exact && std::min(mask_len, capacity) > exact_max_tokens(head_dim)) return kUnsupported;
  const uint64_t bits =
      reinterpret_cast<uintptr_t>(query) | reinterpret_cast<uintptr_t>(key) |
      reinterpret_cast<uintptr_t>(value) | reinterpret_cast<uintptr_t>(cosine) |
      reinterpret_cast<uintptr_t>(sine) | reinterpret_cast<uintptr_t>(key_buffer) |
      reinterpret_cast<uintptr_t>(value_buffer);
  const int64_t strides = q_stride_b | q_stride_h | k_stride_b | k_stride_h | v_stride_b |
                          v_stride_h | cos_stride_b | sin_stride_b | kv_stride_b |
                          kv_stride_s | kv_stride_h;
  const int64_t mask_es = mask == nullptr ? 0 : slc_host::dtype_size(mask_dtype);
  if ((bits & 15) != 0 || (strides & 7) != 0 || kv_stride_s <= 0 || mask_stride_s < 0 ||
      capacity * kv_stride_s * 2 >= (int64_t{1} << 31) ||
      mask_len * mask_stride_s * mask_es >= (int64_t{1} << 31) || capacity >= (int64_t{1} << 30))
    return kUnsupported;
  const Plan plan =
      plan_call(dtype, batch, q_heads, kv_heads, head_dim, mask_len, capacity, 0, exact);
  SLC_REQUIRE(plan.need == 0 || (workspace != nullptr && workspace_bytes >= plan.need),
              "slc_hip_rope_decode_attention: workspace of %lld bytes needed, got %lld",
              (long long)plan.need, (long long)workspace_bytes);
  SLC_REQUIRE(counters != nullptr && num_counters >= plan.counters,
              "slc_hip_rope_decode_attention: %lld counters needed, got %lld",
              (long long)plan.counters, (long long)num_counters);
  const int64_t st[9] = {q_stride_b,    q_stride_h,    kv_stride_b,  kv_stride_s, kv_stride_h,
                         mask_stride_b, mask_stride_s, out_stride_b, out_stride_h};
  RopeStore rope{key,          value,        cosine,       sine,         k_stride_b,
                 k_stride_h,   v_stride_b,   v_stride_h,   cos_stride_b, sin_stride_b,
                 key_buffer,   value_buffer, lengths_out,  overflow,     nullptr};
  hipStream_t s = static_cast<hipStream_t>(stream);
#define SLC_ROPE_CALL(TT, DD)                                                                  \
  launch_mfma<TT, DD>(query, key_buffer, value_buffer, lengths, SLC_I64, mask, mask_dtype,     \
                      output, workspace, counters, batch, q_heads, kv_heads, capacity,         \
                      mask_len, st, scale, plan.chunk, plan.nchunks, exact, s, &rope)
  if (dtype == SLC_BF16) {
    if (head_dim == 64) return SLC_ROPE_CALL(slc::bf16_t, 64);
    return SLC_ROPE_CALL(slc::bf16_t, 128);
  }
  if (head_dim == 64) return SLC_ROPE_CALL(slc::f16_t, 64);
  return SLC_ROPE_CALL(slc::f16_t, 128);
#undef SLC_ROPE_CALL
}
