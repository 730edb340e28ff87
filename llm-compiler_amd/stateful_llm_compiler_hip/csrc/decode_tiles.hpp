// Tile helpers shared by the decode-attention kernels (fixed-chunk and
// balanced split): MFMA operand types, buffer resources, cross-workgroup
// publish/arrival primitives and the in-kernel RoPE of the new token.
#pragma once

#include <type_traits>

#include "common.hpp"
#include "op_math.hpp"

namespace slc_decode {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kTile = 32;   // tokens per wave iteration
#ifndef SLC_DECODE_WAVES
#define SLC_DECODE_WAVES 4
#endif
constexpr int kWaves = SLC_DECODE_WAVES;  // wavefronts per split-kernel workgroup
constexpr int kThreads = kWaves * 64;
#ifndef SLC_DECODE_TILES
#define SLC_DECODE_TILES 2
#endif
constexpr int kTilesInFlight = SLC_DECODE_TILES;  // K/V tiles in flight per wave (split kernel)
constexpr int kGenericWaves = 4;          // wavefronts of the generic kernel
constexpr int kMaxGroups = 16;
constexpr int kMaxChunks = 256;  // split-sequence chunks per (batch, kv-head), merge LDS

struct u16x8 {
  uint16_t v[8];
};

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

template <typename T>
__device__ __forceinline__ typename Mfma<T>::vec as_vec(uint4 raw) {
  return __builtin_bit_cast(typename Mfma<T>::vec, raw);
}

template <typename T>
__device__ __forceinline__ uint16_t bits_of(float f) {
  return slc::from_f32<T>(f).bits;
}

__device__ __forceinline__ float fast_exp2(float x) {
  return __builtin_amdgcn_exp2f(x);
}

// LDS row stride (in 16-bit elements) of a staged V tile row.  The 4-element
// pad makes the four token rows read by one transposed access land on disjoint
// bank groups.
template <int D>
constexpr int v_row() {
  return D + 4;
}

template <typename T, int D>
struct SharedLayout {
  static constexpr int kVTileElems = kTile * v_row<D>();
  static constexpr int kVBytes = kWaves * kVTileElems * 2;
  static constexpr int kCombineBytes =
      kWaves * (2 * kMaxGroups + kMaxGroups * D) * 4;
  static constexpr int kBytes = kVBytes > kCombineBytes ? kVBytes : kCombineBytes;
};

// Dynamic LDS of every EXACT-order launch: 128 KB, or less where the static
// area and the 160 KB of a CU leave less.  (The runtime granted 128 KB here
// and refused the 141 KB that 160 KB minus the static area would allow.)
template <typename T, int D>
constexpr int exact_dyn_bytes() {
  constexpr int room = (160 * 1024 - SharedLayout<T, D>::kBytes - 1024) / 1024 * 1024;
  return room < 128 * 1024 ? room : 128 * 1024;
}

typedef int i32x4_t __attribute__((ext_vector_type(4)));

// Raw buffer resource over [base, base + bytes): loads at or past the end
// return zero without touching memory (the hardware range check), which is how
// rows past the chunk end are handled -- no clamps, no branches.
// Callers pass wave-uniform values; readfirstlane states that to the compiler
// so the resource stays in scalar registers (no per-lane waterfall loop).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int bytes) {
  const uint64_t address = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(address));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(address >> 32));
  void* uniform = reinterpret_cast<void*>((static_cast<uint64_t>(hi) << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(uniform, 0, __builtin_amdgcn_readfirstlane(bytes),
                                           0x00020000);
}
__device__ __forceinline__ uint4 buffer_load16(__amdgpu_buffer_rsrc_t rsrc, int offset) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, offset, 0, 0));
}

// ---- merge inside the split kernel ------------------------------------------
// The caller's counter array holds one counter per (batch, kv-head) (and one
// per batch for the RoPE variant's length advance); it is zero-filled once by
// its owner and every kernel leaves it zero again.
//
// Every split workgroup publishes its partial, meets its waves at a barrier,
// and one thread counts the workgroup's arrival with an agent-scope release
// add: the barrier (a workgroup-scope fence) orders every wave's stores before
// that thread, and the release orders them before the count.  Only the
// workgroup whose add completes the count takes an agent-scope acquire fence
// before its waves, behind a second barrier, load the partials.  Release
// sequence + acquire fence: the HIP memory model's synchronisation, with the
// L2 invalidation of the acquire paid once per (batch, kv-head) instead of
// by every workgroup.  (Relaxed adds with only the hardware ordering of
// completed stores would save the release's L2 write-back too, 1.9 us per
// launch at batch 32 x 8192 tokens, but the model does not order them.)
// The merge weighs the chunks exactly as the separate merge kernel does, so
// both paths give bit-identical outputs.  Two calls that share counters must
// not run concurrently (calls on one stream never do).
__device__ __forceinline__ void publish(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float fetch_partial(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int count_arrival(int* counter) {
  return __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
}
// A count that orders no data: the length advance's last arrival writes the
// new length, which only later kernels read; the add's atomicity suffices.
__device__ __forceinline__ int count_only(int* counter) {
  return __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// The completing workgroup's side of the pairing.
__device__ __forceinline__ void acquire_partials() { __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent"); }
__device__ __forceinline__ void rearm(int* counter) {
  __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

constexpr int kFusedMergeUnroll = 8;
// Length advance folded into the attention kernel: every workgroup of a
// batch bumps the batch's counter once all its waves have read the length
// (the merge's barrier), and the one completing the count writes the new
// length (flagging an advance past the capacity) and re-arms the counter.
struct LenAdvance {
  int* counter;      // nullptr: no advance
  int total;         // workgroups per batch (kv heads x chunks)
  int64_t* out;      // the batch's length
  int64_t next;      // its new value
  int* overflow;
  int64_t capacity;
};

__device__ __forceinline__ void finish_advance(const LenAdvance& adv, int before) {
  if (adv.counter == nullptr || before != adv.total - 1) return;
  rearm(adv.counter);
  *adv.out = adv.next;
  if (adv.overflow != nullptr && (adv.next > adv.capacity || adv.next < 0)) *adv.overflow = 1;
}

// RoPE + KV store of the new token folded into the attention kernel
// (slc_hip_rope_decode_attention).  key/value: the token's projections
// [b, kv_head, D] (key before RoPE); cosine/sine: [b, D] rows of its position.
struct RopeStore {
  const void* key;
  const void* value;
  const void* cosine;
  const void* sine;
  int64_t k_sb, k_sh, v_sb, v_sh, c_sb, s_sb;
  // The KV buffers again, for the new row's write (the kernel's buffer
  // arguments are read-only views; the only row written is one this
  // workgroup does not use from memory, see the tile patch).
  void* key_out;
  void* value_out;
  int64_t* lengths_out;
  int* overflow;
  int* counters;  // per-batch advance counters (caller's counter array)
};

// Qwen2 half rotation of one lane's slices: slice kk pairs with kk + KK/2
// (dims d and d + D/2), rounded exactly as the RoPE kernel rounds.
template <typename T, int KK>
__device__ __forceinline__ void rope_slices(uint4 (&x)[KK], const uint4 (&cs)[KK],
                                            const uint4 (&sn)[KK]) {
  constexpr int H = KK / 2;
  auto f = [](uint16_t bits) {
    T t;
    t.bits = bits;
    return slc::to_f32(t);
  };
#pragma unroll
  for (int kk = 0; kk < H; ++kk) {
    u16x8 a = __builtin_bit_cast(u16x8, x[kk]);
    u16x8 z = __builtin_bit_cast(u16x8, x[kk + H]);
    const u16x8 c1 = __builtin_bit_cast(u16x8, cs[kk]);
    const u16x8 c2 = __builtin_bit_cast(u16x8, cs[kk + H]);
    const u16x8 s1 = __builtin_bit_cast(u16x8, sn[kk]);
    const u16x8 s2 = __builtin_bit_cast(u16x8, sn[kk + H]);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float o1, o2;
      slc::rope_pair<T>(f(a.v[i]), f(z.v[i]), f(c1.v[i]), f(c2.v[i]), f(s1.v[i]), f(s2.v[i]),
                        o1, o2);
      a.v[i] = bits_of<T>(o1);
      z.v[i] = bits_of<T>(o2);
    }
    x[kk] = __builtin_bit_cast(uint4, a);
    x[kk + H] = __builtin_bit_cast(uint4, z);
  }
}

// Paged KV (decode_paged.hip): K/V rows live in page pools
// [num_pages, page_tokens, kv_heads, head_dim]; token t of sequence b is row
// t mod page_tokens of page table[b * table_sb + t / page_tokens].
// page_tokens is a power of two >= 16 (a 16-row MFMA block never straddles
// two pages); page_stride is one page's size in elements.
struct Paging {
  const int* table;
  int64_t table_sb;
  int page_shift;  // log2(page_tokens)
  int64_t page_stride;
};

// ---- balanced split (decode_stream.hip) -------------------------------------
constexpr int kStreamMaxBatch = 2048;  // lengths prefix held in LDS
constexpr int kStreamMaxGrid = 1024;   // workgroups (partial slots) of one call

// One call of the balanced kernel; st[] = q_sb, q_sh, kv_sb, kv_ss, kv_sh,
// m_sb, m_ss, o_sb, o_sh (elements).  counters: batch * kv_heads sequence
// counters, zero between calls.
struct StreamCall {
  const void* query;
  const void* key_buffer;
  const void* value_buffer;
  const void* lengths;
  int lengths_dtype;
  const void* mask;
  int mask_dtype;
  void* output;
  void* workspace;
  int* counters;
  int dtype;
  int64_t batch, q_heads, kv_heads, head_dim, capacity, mask_len;
  int64_t st[9];
  float scale;
  hipStream_t stream;
};
bool stream_eligible(int64_t batch, int64_t kv_heads, int64_t groups, int64_t mask_len,
                     int64_t capacity);
int64_t stream_workspace_bytes(int64_t q_heads, int64_t kv_heads, int64_t head_dim);
int64_t stream_grid(int64_t batch, int64_t segments, int64_t mask_len, int64_t capacity);
int launch_stream(const StreamCall& call);

}  // namespace slc_decode
