// prefill_attention: multi-token GQA attention (serve.prefill_attention).
//
// Semantics: src/stateful_llm_compiler/execution.py:707-739 (reference
// executor) and backends/triton_prefill_attention.py:10-150 (fused kernel):
//   out[b,h,q,:] = sum_k softmax_k(scale * q.k + mask[b,q,k]) v[b,k,h/g,:]
// with keys k > q removed when the op is causal (causal=True); an additive
// mask (B x 1 x T x T) is applied when given.  q.k and its scaling are
// rounded to the I/O dtype as the reference executor's matmul and multiply
// are; fp32 softmax and accumulation.
//
// MI355X design (bf16 / fp16, head_dim 64):
//  * A workgroup is 4 waves x 16 queries of one (batch, query head); K/V tiles
//    of 64 keys are loaded once per workgroup with coalesced 16-byte loads and
//    shared through LDS (double buffered, prefetched into registers).
//  * Each wave computes S^T[key, query] = K . Q^T with v_mfma_f32_16x16x32, so
//    a lane owns one query column: the softmax max needs only two cross-lane
//    shuffles per tile and the exponentials stay in registers.
//  * O^T[dim, query] += V^T . P^T: V is written to LDS transposed, with keys
//    placed in the order of the lanes' P registers, so both MFMA operands are
//    single ds_read_b128 / register reads.
//  * Causal: tiles entirely in a wave's future are skipped (and workgroups
//    are launched heaviest-first); the diagonal tile is masked per element.
// fp32 and other shapes take a simple wave-per-query kernel.
#include <cmath>
#include <type_traits>

#include "common.hpp"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescaleThreshold = 8.0f;

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

struct u16x8 {
  uint16_t v[8];
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

constexpr int kD = 64;       // head dim of the MFMA kernel
#ifndef SLC_PREFILL_GROUPED
#define SLC_PREFILL_GROUPED 1
#endif
constexpr bool kUseGrouped = SLC_PREFILL_GROUPED != 0;
constexpr int kKeys = 64;    // keys per tile
constexpr int kQueries = 64; // queries per workgroup (4 waves x 16)
constexpr int kRowBytes = kD * 2;
constexpr int kTileBytes = kKeys * kRowBytes;  // 8 KB

// K tile: row = key, 16-byte chunks XOR-swizzled by row.
__device__ __forceinline__ int k_offset(int key, int chunk) {
  return key * kRowBytes + ((chunk ^ (key & 7)) << 4);
}
// Position of a key inside its 32-key half in the V^T tile: the order of the
// P operand's k-slots (lane group g holds keys 4g..4g+3 of both 16-key blocks).
__device__ __forceinline__ int key_position(int key) {
  const int half = key >> 5, k = key & 31;
  return half * 32 + ((k & 15) >> 2) * 8 + (k >> 4) * 4 + (k & 3);
}
// V^T tile: row = dim, 64 key positions, 16-byte chunks XOR-swizzled by row.
__device__ __forceinline__ int vt_offset(int dim, int position) {
  return dim * kRowBytes + (((position >> 3) ^ (dim & 7)) << 4) + (position & 7) * 2;
}

template <typename T>
__device__ __forceinline__ uint16_t bits_of(float f) {
  return slc::from_f32<T>(f).bits;
}

// MK: mask element type (0 = none, else slc_dtype + 1).
template <typename T, int MK, bool CAUSAL>
__global__ __launch_bounds__(256) void prefill_attention_mfma_kernel(
    const T* __restrict__ query, const T* __restrict__ key, const T* __restrict__ value,
    const void* __restrict__ mask, T* __restrict__ output, int tokens, int q_heads,
    int groups, int64_t q_sb, int64_t q_sh, int64_t q_st, int64_t k_sb, int64_t k_sh,
    int64_t k_st, int64_t v_sb, int64_t v_sh, int64_t v_st, int64_t m_sb,
    int64_t m_sq, int64_t m_sk, int64_t o_sb, int64_t o_sh, int64_t o_st,
    float scale) {
  using M = Mfma<T>;
  __shared__ __attribute__((aligned(16))) unsigned char smem[2][2][kTileBytes];

  // Grid (heads, batch, query blocks): workgroups dispatch in that order,
  // so with the causal flag every row's heaviest query block goes first.
  const int nqb = gridDim.z;
  const int qb = CAUSAL ? nqb - 1 - static_cast<int>(blockIdx.z) : blockIdx.z;
  const int h = blockIdx.x;
  const int64_t b = blockIdx.y;
  const int kvh = h / groups;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int g = lane >> 4;
  const int c = lane & 15;
  const int q0 = qb * kQueries;
  const int qw = q0 + wave * 16;  // first query of this wave
  const int my_query = qw + c;

  // Q^T as the B operand: lane (query c, k-slice g) holds dims kk*32+8g..+7.
  typename M::vec qv[2];
  {
    const int qrow = my_query < tokens ? my_query : tokens - 1;
    const T* qp = query + b * q_sb + h * q_sh + static_cast<int64_t>(qrow) * q_st;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
      qv[kk] = __builtin_bit_cast(typename M::vec,
                                  *reinterpret_cast<const uint4*>(qp + kk * 32 + 8 * g));
  }

  const int64_t k_rows_bytes = (static_cast<int64_t>(tokens) - 1) * k_st * 2 + kRowBytes;
  const int64_t v_rows_bytes = (static_cast<int64_t>(tokens) - 1) * v_st * 2 + kRowBytes;
  const T* kbase = key + b * k_sb + kvh * k_sh;
  const T* vbase = value + b * v_sb + kvh * v_sh;

  // Keys this workgroup needs: all of them, or up to its last query if causal.
  const int q_last = min(q0 + kQueries, tokens) - 1;
  const int key_end = CAUSAL ? q_last + 1 : tokens;
  const int ntiles = (key_end + kKeys - 1) / kKeys;

  // Cooperative tile fetch: 512 16-byte chunks of K and of V, 2 + 2 per thread.
  uint4 kr[2], vr[2];
  auto fetch = [&](int k0) {
    const __amdgpu_buffer_rsrc_t rk =
        make_rsrc(kbase + static_cast<int64_t>(k0) * k_st,
                  k_rows_bytes - static_cast<int64_t>(k0) * k_st * 2);
    const __amdgpu_buffer_rsrc_t rv =
        make_rsrc(vbase + static_cast<int64_t>(k0) * v_st,
                  v_rows_bytes - static_cast<int64_t>(k0) * v_st * 2);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int ch = tid + 256 * i;
      const int row = ch >> 3, col = (ch & 7) * 8;
      kr[i] = buffer_load16(rk, static_cast<int>((row * k_st + col) * 2));
      vr[i] = buffer_load16(rv, static_cast<int>((row * v_st + col) * 2));
    }
  };
  auto stash = [&](int buf) {
    unsigned char* ks = smem[buf][0];
    unsigned char* vs = smem[buf][1];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int ch = tid + 256 * i;
      const int row = ch >> 3, chunk = ch & 7;
      *reinterpret_cast<uint4*>(ks + k_offset(row, chunk)) = kr[i];
      const uint16_t* e = reinterpret_cast<const uint16_t*>(&vr[i]);
      const int pos = key_position(row);
#pragma unroll
      for (int d = 0; d < 8; ++d)
        *reinterpret_cast<uint16_t*>(vs + vt_offset(chunk * 8 + d, pos)) = e[d];
    }
  };

  float m_run = -INFINITY, l_run = 0.0f;
  f32x4_t acc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) acc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  constexpr int kMaskBytes = MK == SLC_F32 + 1 ? 4 : 2;
  const char* mrow = nullptr;
  if constexpr (MK != 0) {
    const int qrow = my_query < tokens ? my_query : tokens - 1;
    mrow = static_cast<const char*>(mask) + (b * m_sb + static_cast<int64_t>(qrow) * m_sq) * kMaskBytes;
  }

  if (ntiles > 0) {
    fetch(0);
    stash(0);
  }
  __syncthreads();
  for (int kt = 0; kt < ntiles; ++kt) {
    const int buf = kt & 1;
    const int k0 = kt * kKeys;
    if (kt + 1 < ntiles) fetch(k0 + kKeys);
    // A tile wholly in this wave's future contributes nothing.
    const bool active = !CAUSAL || k0 <= qw + 15;
    if (active && qw < tokens) {
      const unsigned char* ks = smem[buf][0];
      const unsigned char* vs = smem[buf][1];
      float s[16];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        f32x4_t st = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const auto a = *reinterpret_cast<const typename M::vec*>(
              ks + k_offset(kb * 16 + c, kk * 4 + g));
          st = M::run(a, qv[kk], st);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int kidx = k0 + kb * 16 + 4 * g + r;
          // q.k and its scaling are materialised in the tensor dtype, as the
          // reference executor's matmul and multiply do; softmax stays fp32.
          float v = slc::round_to<T>(slc::round_to<T>(st[r]) * scale) * kLog2e;
          if constexpr (MK != 0) {
            if (kidx < tokens) {
              const char* p = mrow + static_cast<int64_t>(kidx) * m_sk * kMaskBytes;
              float mv;
              if constexpr (MK == SLC_F32 + 1) {
                mv = *reinterpret_cast<const float*>(p);
              } else if constexpr (MK == SLC_BF16 + 1) {
                mv = slc::to_f32(*reinterpret_cast<const slc::bf16_t*>(p));
              } else {
                mv = slc::to_f32(*reinterpret_cast<const slc::f16_t*>(p));
              }
              v += mv * kLog2e;
            }
          }
          bool valid = kidx < tokens;
          if constexpr (CAUSAL) valid = valid && kidx <= my_query;
          s[kb * 4 + r] = valid ? v : -INFINITY;
        }
      }
      float mx = s[0];
#pragma unroll
      for (int i = 1; i < 16; ++i) mx = fmaxf(mx, s[i]);
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      if (__any(mx > m_run + kRescaleThreshold)) {
        const float m_new = fmaxf(m_run, mx);
        const float alpha = __builtin_amdgcn_exp2f(m_run - (m_new == -INFINITY ? 0.0f : m_new));
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < 4; ++db) acc[db] = acc[db] * alpha;
        m_run = m_new;
      }
      const float m_use = m_run == -INFINITY ? 0.0f : m_run;
      typename M::vec pv[2];
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        u16x8 bits;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float p = __builtin_amdgcn_exp2f(s[(2 * half + (i >> 2)) * 4 + (i & 3)] - m_use);
          l_run += p;
          bits.v[i] = bits_of<T>(p);
        }
        pv[half] = __builtin_bit_cast(typename M::vec, bits);
      }
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const auto a = *reinterpret_cast<const typename M::vec*>(
              vs + vt_offset(db * 16 + c, half * 32 + g * 8));
          acc[db] = M::run(a, pv[half], acc[db]);
        }
    }
    if (kt + 1 < ntiles) stash(buf ^ 1);
    __syncthreads();
  }

  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);
  if (my_query < tokens) {
    const float inv = 1.0f / l_run;
    T* op = output + b * o_sb + h * o_sh + static_cast<int64_t>(my_query) * o_st;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int r = 0; r < 4; ++r) op[db * 16 + 4 * g + r] = slc::from_f32<T>(acc[db][r] * inv);
  }
}

// Generic path: one wave per query row, shuffled dot products, online softmax
// (EXACT: a first pass for the row max and sum, then the normalised
// probabilities rounded to the I/O dtype weigh V, the reference's order).
template <typename T, int NI, bool EXACT>
__global__ __launch_bounds__(256) void prefill_attention_generic_kernel(
    const T* __restrict__ query, const T* __restrict__ key, const T* __restrict__ value,
    const void* __restrict__ mask, int mask_dtype, T* __restrict__ output, int tokens,
    int q_heads, int groups, int head_dim, int causal, int64_t q_sb, int64_t q_sh,
    int64_t q_st, int64_t k_sb, int64_t k_sh, int64_t k_st, int64_t v_sb,
    int64_t v_sh, int64_t v_st, int64_t m_sb, int64_t m_sq, int64_t m_sk,
    int64_t o_sb, int64_t o_sh, int64_t o_st, float scale) {
  const int lane = threadIdx.x & 63;
  const int qi = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int h = blockIdx.y;
  const int64_t b = blockIdx.z;
  if (qi >= tokens) return;
  const int kvh = h / groups;
  float q[NI], acc[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int d = lane + 64 * i;
    q[i] = d < head_dim ? slc::to_f32(query[b * q_sb + h * q_sh + qi * q_st + d]) : 0.0f;
    acc[i] = 0.0f;
  }
  const int key_end = causal ? qi + 1 : tokens;
  auto score = [&](int kidx) {
    float dot = 0.0f;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int d = lane + 64 * i;
      if (d < head_dim) dot += q[i] * slc::to_f32(key[b * k_sb + kvh * k_sh + kidx * k_st + d]);
    }
    dot = slc::wave_sum(dot);
    float s = (sizeof(T) == 2 ? slc::round_to<T>(slc::round_to<T>(dot) * scale) : dot * scale) * kLog2e;
    if (mask != nullptr) s += slc::load_as_f32(mask, b * m_sb + qi * m_sq + kidx * m_sk, mask_dtype) * kLog2e;
    return s;
  };
  float m_run = -INFINITY, l_run = 0.0f;
  for (int kidx = 0; kidx < key_end; ++kidx) {
    const float s = score(kidx);
    const float m_new = fmaxf(m_run, s);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = exp2f(m_run - m_use);
    const float p = exp2f(s - m_use);
    l_run = l_run * alpha + p;
    if constexpr (!EXACT) {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int d = lane + 64 * i;
        const float v = d < head_dim ? slc::to_f32(value[b * v_sb + kvh * v_sh + kidx * v_st + d]) : 0.0f;
        acc[i] = acc[i] * alpha + p * v;
      }
    }
    m_run = m_new;
  }
  float inv = 1.0f / l_run;
  if constexpr (EXACT) {
    const float m_use = m_run == -INFINITY ? 0.0f : m_run;
    const float shift = l_run > 0.0f ? m_use + log2f(l_run) : __builtin_nanf("");
    for (int kidx = 0; kidx < key_end; ++kidx) {
      const float p = slc::round_to<T>(exp2f(score(kidx) - shift));
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int d = lane + 64 * i;
        const float v = d < head_dim ? slc::to_f32(value[b * v_sb + kvh * v_sh + kidx * v_st + d]) : 0.0f;
        acc[i] += p * v;
      }
    }
    inv = l_run > 0.0f ? 1.0f : __builtin_nanf("");
  }
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int d = lane + 64 * i;
    if (d < head_dim) output[b * o_sb + h * o_sh + qi * o_st + d] = slc::from_f32<T>(acc[i] * inv);
  }
}


// ---- mask tile classes ---------------------------------------------------------
// One byte per (batch, 64-query block, 64-key tile) of an explicit [B, 1, T, T]
// mask, so the grouped kernel can leave out what the mask makes trivial:
//   0 (dead)   every entry is -inf: the tile adds nothing to any row (the
//              part of a causal mask past the diagonal); no K/V/mask loads.
//   1 (causal) every entry is +0 where key <= query and -inf where key >
//              query: the causal pattern, applied from the indices, so the
//              tile's mask is not loaded.
//   2          anything else: the mask tile is loaded and added.
// Entries past T (a partial last tile) are not looked at; those keys are
// invalid anyway.  Grid (key tiles, query blocks, batch), 256 threads.
// VEC: unit key stride, 16-byte aligned rows and T a multiple of the 16-byte
// chunk: each thread reads whole 16-byte chunks (2 KB per wave per load).
template <int MK, bool VEC>
__global__ __launch_bounds__(256) void mask_tile_class_kernel(const void* __restrict__ mask,
                                                              unsigned char* __restrict__ classes,
                                                              int tokens, int64_t m_sb, int64_t m_sq,
                                                              int64_t m_sk) {
  constexpr int ME = MK == SLC_F32 + 1 ? 4 : 2;
  constexpr uint32_t kNinf = ME == 4 ? 0xff800000u : (MK == SLC_BF16 + 1 ? 0xff80u : 0xfc00u);
  const int k0 = blockIdx.x * 64, q0 = blockIdx.y * 64;
  const int64_t b = blockIdx.z;
  const unsigned char* base = static_cast<const unsigned char*>(mask) + b * m_sb * ME;
  bool live = false, general = false;
  auto check = [&](uint32_t bits, int q, int key) {
    live |= bits != kNinf;
    general |= key <= q ? bits != 0u : bits != kNinf;
  };
  if constexpr (VEC) {
    constexpr int kPer = 16 / ME;              // elements per chunk
    constexpr int kChunksRow = 64 / kPer;      // chunks per tile row
    for (int id = threadIdx.x; id < 64 * kChunksRow; id += 256) {
      const int r = id / kChunksRow, key = k0 + (id % kChunksRow) * kPer;
      const int q = q0 + r;
      if (q >= tokens || key >= tokens) continue;  // T is a multiple of kPer
      const uint4 v = *reinterpret_cast<const uint4*>(base + (static_cast<int64_t>(q) * m_sq + key) * ME);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int e = 0; e < kPer; ++e) {
        const uint32_t bits = ME == 4 ? w[e] : (w[e >> 1] >> (16 * (e & 1))) & 0xffffu;
        check(bits, q, key + e);
      }
    }
  } else {
    // Thread t: key column k0 + t % 64, query rows q0 + t / 64 + 4i.
    const int key = k0 + (threadIdx.x & 63);
    if (key < tokens) {
      for (int r = threadIdx.x >> 6; r < 64 && q0 + r < tokens; r += 4) {
        const int q = q0 + r;
        const unsigned char* p = base + (static_cast<int64_t>(q) * m_sq + static_cast<int64_t>(key) * m_sk) * ME;
        check(ME == 4 ? *reinterpret_cast<const uint32_t*>(p) : *reinterpret_cast<const uint16_t*>(p), q, key);
      }
    }
  }
  const bool any_live = __syncthreads_or(live);
  const bool any_general = __syncthreads_or(general);
  if (threadIdx.x == 0) {
    const int64_t nqb = gridDim.y, nkt = gridDim.x;
    classes[(b * nqb + blockIdx.y) * nkt + blockIdx.x] = !any_live ? 0 : (any_general ? 2 : 1);
  }
}

// ---- grouped-head kernel (v2) ------------------------------------------------
// A workgroup owns kV2Queries queries of ALL the query heads of one KV head
// (GQA group G): G compute waves (one query head each, kQB MFMA column
// blocks of 16 queries) plus one producer wave that streams the K, V (and mask) tiles of 64
// keys into an LDS ring with direct-to-LDS loads.  K, V and the mask are thus
// read once per workgroup for all G heads (the single-head kernel reads them
// G times), and no VALU work or VGPR goes into staging.
//  * S^T[key, query] = K . Q^T: K rows straight from the XOR-swizzled tile
//    (ds_read_b128), Q^T in registers (kQB query blocks reuse every K read).
//  * O^T[dim, query] += V^T . P^T: V^T operands come from the natural V tile
//    through the LDS transpose read (ds_read_b64_tr_b16), whose lane j of a
//    16-lane group addresses 4 dims of key row T(j/4) and receives dim j of
//    the 4 keys: two reads give the 8 keys in the P operand's slot order.
//  * One barrier per tile: the producer waits for tile i, the barrier hands
//    it to the consumers, then the producer refills the ring slot consumers
//    released at that barrier.
// Query blocks of 16 per consumer wave: 4 (64 queries per workgroup, about
// 214 VGPRs, one workgroup per CU) or 2 (32 queries, at most 128 VGPRs, two
// workgroups per CU whose MFMA and VALU phases need not coincide).
#ifndef SLC_PREFILL_QB
#define SLC_PREFILL_QB 2
#endif
constexpr int kQB = SLC_PREFILL_QB;
constexpr int kV2Queries = 16 * kQB;
// Longest key range (in 64-key tiles) the tile-class list covers: T <= 65536.
constexpr int kMaxClassTiles = 1024;
// Two ring stages: the producer refills one stage while the consumers read
// the other (measured 2-3 % faster than three stages, equal to four).
#ifndef SLC_PREFILL_STAGES
#define SLC_PREFILL_STAGES 2
#endif
constexpr int kV2Stages = SLC_PREFILL_STAGES;
constexpr int kV2TileBytes = kKeys * kRowBytes;                 // 8 KB of K or of V
// Mask tile: kV2Queries query rows x 64 keys of the mask element type (0: no mask).
template <int MK>
constexpr int mask_elem_bytes() { return MK == 0 ? 0 : (MK == SLC_F32 + 1 ? 4 : 2); }
template <int MK>
constexpr int stage_bytes() { return 2 * kV2TileBytes + kV2Queries * kKeys * mask_elem_bytes<MK>(); }

typedef short v4s_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// bf16(a) in the low half, bf16(b) in the high half: one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t round_pair_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}
typedef uint32_t v2u_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t rsrc, unsigned char* lds,
                                          int voffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      rsrc, (__attribute__((address_space(3))) void*)lds, 16, voffset, 0, 0, 0);
}
__device__ __forceinline__ uint2 lds_read_tr(const unsigned char* p) {
  const v4s_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4s_t*)(p));
  return __builtin_bit_cast(uint2, v);
}

// POW2: bf16 with a power-of-two scale (1/8 for head_dim 64): a normal bf16
// value times 2^k is exact and stays a bf16 value (bf16 has fp32's exponent
// range), so bf16(bf16(q.k) * scale) = bf16(q.k) * scale and the second
// rounding goes.  (They differ only for scaled scores below bf16's normal
// range, |score| < 2^-126, where the difference vanishes in score - max.)
// fp16 keeps both roundings: its narrow exponent range makes subnormal
// scaled scores common.
// EXACT: the reference executor's softmax order (execution.py:720-739:
// softmax in fp32, rounded to the I/O dtype, then P.V): two passes over the
// key tiles.  Pass 1 forms each query row's max and sum (K and the mask only;
// the producer's V loads of that pass read a zero-length range, so they move
// no data but keep every tile's load count equal); pass 2 recomputes the
// scores and weighs V with exp(score - max) / sum rounded to the I/O dtype,
// so the rounding applies to the normalised probability as in the reference.
template <typename T, int G, int MK, bool CAUSAL, bool POW2, bool EXACT>
__global__ __launch_bounds__((G + 1) * 64, kQB == 2 ? 4 : 1) void prefill_attention_v2_kernel(
    const T* __restrict__ query, const T* __restrict__ key, const T* __restrict__ value,
    const void* __restrict__ mask, T* __restrict__ output, int tokens, int kv_heads,
    int64_t q_sb, int64_t q_sh, int64_t q_st, int64_t k_sb, int64_t k_sh, int64_t k_st,
    int64_t v_sb, int64_t v_sh, int64_t v_st, int64_t m_sb, int64_t m_sq, int64_t o_sb,
    int64_t o_sh, int64_t o_st, float scale, const unsigned char* __restrict__ tile_class) {
  using M = Mfma<T>;
  constexpr int ME = mask_elem_bytes<MK>();
  constexpr int kMaskRow = kKeys * ME;                 // bytes of one mask tile row
  constexpr int kMaskTile = kV2Queries * kMaskRow;
  __shared__ __attribute__((aligned(16))) unsigned char ring[kV2Stages][stage_bytes<MK>()];
  // With tile classes (MK != 0): the key tiles this query block visits, in
  // order, bit 15 set where the mask tile is loaded (class 2), and their count.
  __shared__ uint16_t live_tiles[MK != 0 ? kMaxClassTiles : 1];
  __shared__ int live_count;

  // Grid (KV heads, batch, query blocks): workgroups dispatch in that
  // order, and the last query blocks go first.  Under the causal flag (or a
  // causal-shaped mask, whose skipped tiles make the work alike) those are
  // the heaviest, so the light ones fill the tail: longest-first list
  // scheduling.  Any other shape is indifferent to the order.
  const int nqb = gridDim.z;
  const int qblk = nqb - 1 - static_cast<int>(blockIdx.z);
  const int kvh = blockIdx.x;
  const int64_t b = blockIdx.y;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int g = lane >> 4;
  const int c = lane & 15;
  const int q0 = qblk * kV2Queries;
  // Factor from the stored score to log2 units: without a mask and with a
  // power-of-two scale the stored score is bf16(q.k), unscaled; otherwise it
  // is the reference's fp32 score itself (scaled, mask added).
  const float c_log2 = POW2 && MK == 0 ? scale * kLog2e : kLog2e;
  const int key_end = CAUSAL ? min(q0 + kV2Queries, tokens) : tokens;
  const int all_tiles = (key_end + kKeys - 1) / kKeys;
  const bool classed = MK != 0 && tile_class != nullptr;
  if (classed && wave == G) {
    // The producer lists the live tiles (class != 0) before the first barrier.
    // The classes are per 64 x 64 tile: a block of kV2Queries rows takes its
    // 64-row block's (the causal pattern and -inf throughout hold for every
    // part of a tile that has them).
    const int64_t key_tiles = (tokens + kKeys - 1) / kKeys;
    const unsigned char* row = tile_class + (b * key_tiles + qblk * kV2Queries / 64) * key_tiles;
    int count = 0;
    for (int base = 0; base < all_tiles; base += 64) {
      const int t = base + lane;
      const int cls = t < all_tiles ? row[t] : 0;
      const uint64_t mask_live = __ballot(cls != 0);
      const int before = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask_live >> 32),
                                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask_live), 0));
      if (cls != 0) live_tiles[count + before] = static_cast<uint16_t>(t | (cls == 2 ? 0x8000 : 0));
      count += __popcll(mask_live);
    }
    if (lane == 0) live_count = count;
  }
  if constexpr (MK != 0) {
    if (classed) __syncthreads();  // the list is ready (the producer matches it)
  }
  const int ntiles = classed ? live_count : all_tiles;
  const int nsteps = EXACT ? 2 * ntiles : ntiles;  // ring steps (tile visits)
  // Key tile of list entry i, and whether its mask tile is loaded.
  auto tile_of = [&](int i) { return classed ? (live_tiles[i] & 0x7fff) : i; };
  auto mask_of = [&](int i) { return !classed || (live_tiles[i] & 0x8000) != 0; };

  if (wave == G) {
    // ---- producer ---------------------------------------------------------
    constexpr int kOps = (2 * kV2TileBytes + kMaskTile) / 1024;  // DMA ops per tile
    const char* kbase = reinterpret_cast<const char*>(key + b * k_sb + kvh * k_sh);
    const char* vbase = reinterpret_cast<const char*>(value + b * v_sb + kvh * v_sh);
    const char* mbase = MK == 0 ? nullptr
                                : static_cast<const char*>(mask) + (b * m_sb + static_cast<int64_t>(q0) * m_sq) * ME;
    const int q_rows = min(kV2Queries, tokens - q0);
    // Lane L of DMA instruction n fills LDS row 8n + L/8, chunk position L%8,
    // with the global 16-byte chunk (L%8) ^ (row & 7) of that row.
    auto issue = [&](int step, int stage) {
      unsigned char* dst = ring[stage];
      const int entry = EXACT && step >= ntiles ? step - ntiles : step;
      const bool in_range = step < nsteps;
      const int tile = in_range ? tile_of(entry) : 0;
      const bool want_v = !EXACT || step >= ntiles;
      const bool want_mask = in_range && mask_of(entry);
      const int k0 = tile * kKeys;
      const int rows = in_range ? min(kKeys, tokens - k0) : 0;
      const __amdgpu_buffer_rsrc_t rk = make_rsrc(kbase + static_cast<int64_t>(k0) * k_st * 2,
                                                  rows > 0 ? (static_cast<int64_t>(rows) - 1) * k_st * 2 + kRowBytes : 0);
      const __amdgpu_buffer_rsrc_t rv = make_rsrc(vbase + static_cast<int64_t>(k0) * v_st * 2,
                                                  rows > 0 && want_v ? (static_cast<int64_t>(rows) - 1) * v_st * 2 + kRowBytes : 0);
#pragma unroll
      for (int n = 0; n < kV2TileBytes / 1024; ++n) {
        const int row = 8 * n + lane / 8;
        const int chunk = (lane % 8) ^ (row & 7);
        lds_dma16(rk, dst + n * 1024, static_cast<int>(row * k_st * 2 + chunk * 16));
        lds_dma16(rv, dst + kV2TileBytes + n * 1024, static_cast<int>(row * v_st * 2 + chunk * 16));
      }
      if constexpr (MK != 0) {
        // Mask rows are queries, chunks 8 keys; whole rows stay inside the
        // [T, T] plane (keys past T are masked as invalid anyway).
        const int64_t bytes = want_mask && q_rows > 0
                                  ? ((static_cast<int64_t>(q_rows) - 1) * m_sq + tokens - k0) * ME
                                  : 0;
        const __amdgpu_buffer_rsrc_t rm = make_rsrc(mbase + static_cast<int64_t>(k0) * ME, bytes);
#pragma unroll
        for (int n = 0; n < kMaskTile / 1024; ++n) {
          const int pos = n * 1024 + 16 * lane;
          const int row = pos / kMaskRow;
          const int chunk = ((pos % kMaskRow) >> 4) ^ (row & 7);
          lds_dma16(rm, dst + 2 * kV2TileBytes + n * 1024, static_cast<int>(row * m_sq * ME + chunk * 16));
        }
      }
    };
#pragma unroll
    for (int t = 0; t < kV2Stages - 1; ++t) issue(t, t);
    for (int t = 0; t < nsteps; ++t) {
      // Tile t landed: kStages - 2 later tiles (kOps each) may still fly.
      asm volatile("s_waitcnt vmcnt(%0)" ::"i"((kV2Stages - 2) * kOps) : "memory");
      __syncthreads();
      issue(t + kV2Stages - 1, (t + kV2Stages - 1) % kV2Stages);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    return;
  }

  // ---- consumers: wave w computes query head kvh * G + w ----------------------
  const int h = kvh * G + wave;
  typename M::vec qv[kQB][2];
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) {
    const int qrow = min(q0 + 16 * qb + c, tokens - 1);
    const T* qp = query + b * q_sb + h * q_sh + static_cast<int64_t>(qrow) * q_st;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
      qv[qb][kk] = __builtin_bit_cast(typename M::vec,
                                      *reinterpret_cast<const uint4*>(qp + kk * 32 + 8 * g));
  }
  // acc[4] is the softmax denominator: the P.V MFMA against a block of ones
  // sums each query's probabilities (all 16 rows of the block hold the
  // same sum), so the matrix cores, not the VALU, do the row sums, and the
  // running rescale applies to it with the outputs.
  float m_run[kQB];
  f32x4_t acc[5][kQB];  // [dim block, then the row-sum block][query block]
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) {
    m_run[qb] = -INFINITY;
#pragma unroll
    for (int db = 0; db < 5; ++db) acc[db][qb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  // Transpose-read lane addresses (bytes within a tile) for V^T blocks:
  // lane j = c of group g reads key row 4g + j/4 (+16 for the second read)
  // of a 32-key half, dims 16db + 4(j%4) .. +3.
  u16x8 one_bits;
#pragma unroll
  for (int i = 0; i < 8; ++i) one_bits.v[i] = bits_of<T>(1.0f);
  const typename M::vec ones = __builtin_bit_cast(typename M::vec, one_bits);
  int tr_off[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) {
    const int row = 4 * g + (c >> 2);
    const int dim = 16 * db + 4 * (c & 3);
    tr_off[db] = row * kRowBytes + (((dim >> 3) ^ (row & 7)) << 4) + (dim & 7) * 2;
  }
  const int kv_off0 = c * kRowBytes;  // K operand row 16kb + c
  // EXACT: per-lane partial row sums of pass 1 (the lane's 16 keys of each
  // tile), then the exponent shift max + log2(sum) of pass 2.
  float l_part[kQB] = {};
  float shift[kQB] = {};

  for (int step = 0; step < nsteps; ++step) {
    __syncthreads();  // tile of this step is in ring[step % kStages]
    const bool pass2 = EXACT && step >= ntiles;
    const int entry = pass2 ? step - ntiles : step;
    const int t = tile_of(entry);
    // A class-1 tile: its mask is the causal pattern, applied from indices.
    const bool tile_mask = MK != 0 && mask_of(entry);
    const bool causal_tile = CAUSAL || (MK != 0 && !tile_mask);
    if (EXACT && step == ntiles) {
      // Pass 1 done: row sums over the 4 lane groups, then the shift.
#pragma unroll
      for (int qb = 0; qb < kQB; ++qb) {
        float l = l_part[qb];
        l += __shfl_xor(l, 16, 64);
        l += __shfl_xor(l, 32, 64);
        const float m_use = m_run[qb] == -INFINITY ? 0.0f : m_run[qb];
        // An empty row (every key masked) gives NaN, as the reference's
        // softmax over an all -inf row does.
        shift[qb] = l > 0.0f ? m_use + __builtin_amdgcn_logf(l) : __builtin_nanf("");
      }
    }
    const unsigned char* kt = ring[step % kV2Stages];
    const unsigned char* vt = kt + kV2TileBytes;
    const unsigned char* mt = kt + 2 * kV2TileBytes;  // mask tile, rows = queries
    const int k0 = t * kKeys;
    if (MK != 0 && tile_mask) {
      // A mask tile that is -inf throughout (the part of a causal mask past
      // the diagonal) adds exp2(-inf) = 0 to every sum and no new maximum:
      // the tile is skipped (for finite scores the result is bit-identical;
      // an infinite or NaN score under such a tile, which would make the
      // reference's row NaN, is not looked at).  Every consumer wave reads
      // the same tile, so all take the same branch; the barrier above is the
      // only one per tile.
      // First the element of the last query row and the first key (the last
      // of a causal tile to become -inf; finite in almost any other mask):
      // only when it is -inf is the whole tile read.
      const unsigned char* corner = mt + (kV2Queries - 1) * kMaskRow + ((0 ^ ((kV2Queries - 1) & 7)) << 4);
      const uint32_t cbits = ME == 4 ? *reinterpret_cast<const uint32_t*>(corner)
                                     : *reinterpret_cast<const uint16_t*>(corner);
      const uint32_t cninf = ME == 4 ? 0xff800000u : (MK == SLC_BF16 + 1 ? 0xff80u : 0xfc00u);
      bool live = cbits != cninf;
#pragma unroll
      for (int off = lane * 16; !__any(live) && off < kMaskTile; off += 64 * 16) {
        const uint4 v = *reinterpret_cast<const uint4*>(mt + off);
        const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (ME == 4) {
            live |= w4[e] != 0xff800000u;
          } else {
            const uint32_t ninf = MK == SLC_BF16 + 1 ? 0xff80ff80u : 0xfc00fc00u;
            live |= w4[e] != ninf;
          }
        }
      }
      if (!__any(live)) continue;
    }

    // S^T blocks: 4 key blocks x 4 query blocks.
    f32x4_t st[4][kQB];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      typename M::vec ka[2];
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
        ka[kk] = *reinterpret_cast<const typename M::vec*>(
            kt + (16 * kb) * kRowBytes + kv_off0 + (((4 * kk + g) ^ (c & 7)) << 4));
#pragma unroll
      for (int qb = 0; qb < kQB; ++qb) {
        f32x4_t a = f32x4_t{0.f, 0.f, 0.f, 0.f};
        a = M::run(ka[0], qv[qb][0], a);
        st[kb][qb] = M::run(ka[1], qv[qb][1], a);
      }
    }

    // Scores with the mask and validity (fp32, as the reference's fused kernel).
    const bool full = !causal_tile ? k0 + kKeys <= tokens : k0 + kKeys <= q0 && k0 + kKeys <= tokens;
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb) {
      const int my_query = q0 + 16 * qb + c;
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        float mv[4] = {0.f, 0.f, 0.f, 0.f};
        if (MK != 0 && tile_mask) {
          // Mask of keys 16kb + 4g .. +3 for this lane's query row.
          const int row = 16 * qb + c;
          const int byte = (16 * kb + 4 * g) * ME;
          const unsigned char* mp = mt + row * kMaskRow + ((((byte >> 4) ^ (row & 7))) << 4) + (byte & 15);
          if constexpr (ME == 4) {
            const uint4 raw = *reinterpret_cast<const uint4*>(mp);
            mv[0] = __uint_as_float(raw.x);
            mv[1] = __uint_as_float(raw.y);
            mv[2] = __uint_as_float(raw.z);
            mv[3] = __uint_as_float(raw.w);
          } else {
            const uint2 raw = *reinterpret_cast<const uint2*>(mp);
            const uint32_t w2[2] = {raw.x, raw.y};
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              if constexpr (MK == SLC_BF16 + 1) {
                // bf16 to fp32: the element moved into the high half.
                mv[r] = __uint_as_float((r & 1) ? (w2[r >> 1] & 0xffff0000u) : (w2[r >> 1] << 16));
              } else {
                const uint16_t bits = static_cast<uint16_t>(w2[r >> 1] >> (16 * (r & 1)));
                mv[r] = slc::to_f32(slc::f16_t{bits});
              }
            }
          }
        }
        if constexpr (std::is_same_v<T, slc::bf16_t>) {
          // Two scores per v_cvt_pk_bf16_f32 (round to nearest even, as
          // round_to), back to fp32 by a shift and a mask.
#pragma unroll
          for (int r = 0; r < 4; r += 2) {
            const uint32_t pk = round_pair_bf16(st[kb][qb][r], st[kb][qb][r + 1]);
            st[kb][qb][r] = __uint_as_float(pk << 16);
            st[kb][qb][r + 1] = __uint_as_float(pk & 0xffff0000u);
          }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          // v = the executor's rounded score: bf16(bf16(q.k) * scale), or
          // bf16(q.k) when the scale is a power of two (POW2; the product is
          // then exact, so without a mask it moves into the exp2 argument).
          // With a mask the stored score is the executor's fp32 score
          // v * scale + mask: one FMA, exact in the product (POW2), so the
          // sum is rounded once as the executor's fp32 add rounds it.  The
          // row max is taken over the stored scores (times the positive
          // factor c_log2 it is the max of the log2-domain scores).
          float v = std::is_same_v<T, slc::bf16_t> ? st[kb][qb][r] : slc::round_to<T>(st[kb][qb][r]);
          if constexpr (!POW2) v = slc::round_to<T>(v * scale);
          if constexpr (MK != 0) v = POW2 ? fmaf(v, scale, mv[r]) : v + mv[r];
          st[kb][qb][r] = v;
        }
      }
      if (!full) {
        // Only the diagonal and the last tile get here (`full` is uniform).
        // The empty asm keeps this block a branch: if-converted, its compares
        // and selects would run on every tile.  Key 16kb + 4g + r of the tile
        // is valid iff it is at most `last` (the last key this query sees,
        // relative to the lane's first key).
        asm volatile("" ::: "memory");
        int last = tokens - 1 - k0 - 4 * g;
        if (causal_tile) last = min(last, my_query - k0 - 4 * g);
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            st[kb][qb][r] = 16 * kb + r <= last ? st[kb][qb][r] : -INFINITY;
      }
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) mx = fmaxf(mx, st[kb][qb][r]);
      if (pass2) continue;
      // The row max spans the 4 lane groups, but it only matters when it
      // moves the running max, i.e. when some lane's own max is past the
      // threshold (times c > 0 commutes with max): the cross-group
      // reduction runs only then.
      mx *= c_log2;
      if (__any(mx > m_run[qb] + kRescaleThreshold)) {
        mx = slc::max_xor32(slc::max_xor16(mx));
        const float m_new = fmaxf(m_run[qb], mx);
        const float alpha = __builtin_amdgcn_exp2f(m_run[qb] - (m_new == -INFINITY ? 0.0f : m_new));
        if constexpr (EXACT) {
          l_part[qb] *= alpha;
        } else {
#pragma unroll
          for (int db = 0; db < 5; ++db) acc[db][qb] = acc[db][qb] * alpha;
        }
        m_run[qb] = m_new;
      }
      if constexpr (EXACT) {
        // Pass 1: this lane's terms of the row sum (fp32, as the reference's
        // softmax sums them).
        const float m_use = m_run[qb] == -INFINITY ? 0.0f : m_run[qb];
        float sum = 0.0f;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float x = st[kb][qb][r];
            sum += __builtin_amdgcn_exp2f(fmaf(x, c_log2, -m_use));
          }
        l_part[qb] += sum;
      }
    }
    if (EXACT && !pass2) continue;

    // P^T operands and O^T += V^T . P^T.
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      typename M::vec pv[kQB];
#pragma unroll
      for (int qb = 0; qb < kQB; ++qb) {
        // Online: exp2 relative to the running max.  EXACT pass 2: relative
        // to max + log2(sum), i.e. the normalised probability, then rounded.
        const float m_use = EXACT ? shift[qb] : (m_run[qb] == -INFINITY ? 0.0f : m_run[qb]);
        u16x8 bits;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float x = st[2 * half + (i >> 2)][qb][i & 3];
          const float p = __builtin_amdgcn_exp2f(fmaf(x, c_log2, -m_use));
          bits.v[i] = bits_of<T>(p);
        }
        pv[qb] = __builtin_bit_cast(typename M::vec, bits);
      }
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const uint2 lo = lds_read_tr(vt + half * 32 * kRowBytes + tr_off[db]);
        const uint2 hi = lds_read_tr(vt + (half * 32 + 16) * kRowBytes + tr_off[db]);
        const typename M::vec va = __builtin_bit_cast(typename M::vec, make_uint4(lo.x, lo.y, hi.x, hi.y));
#pragma unroll
        for (int qb = 0; qb < kQB; ++qb) acc[db][qb] = M::run(va, pv[qb], acc[db][qb]);
      }
      if constexpr (!EXACT) {
#pragma unroll
        for (int qb = 0; qb < kQB; ++qb) acc[4][qb] = M::run(ones, pv[qb], acc[4][qb]);
      }
    }
  }

#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) {
    const int my_query = q0 + 16 * qb + c;
    if (my_query < tokens) {
      // EXACT: the terms were normalised already.  An empty row (every key
      // masked) is NaN, as the reference's softmax over an all -inf row: its
      // shift is NaN, or no tile was visited at all (every tile of the block
      // masked out) -- then even pass 2's terms never ran.
      const bool empty = ntiles == 0 || shift[qb] != shift[qb];
      const float inv = EXACT ? (empty ? __builtin_nanf("") : 1.0f) : 1.0f / acc[4][qb][0];
      T* op = output + b * o_sb + h * o_sh + static_cast<int64_t>(my_query) * o_st;
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        u16x8 e;
#pragma unroll
        for (int r = 0; r < 4; ++r) e.v[r] = bits_of<T>(acc[db][qb][r] * inv);
        uint2 packed;
        packed.x = static_cast<uint32_t>(e.v[0]) | (static_cast<uint32_t>(e.v[1]) << 16);
        packed.y = static_cast<uint32_t>(e.v[2]) | (static_cast<uint32_t>(e.v[3]) << 16);
        *reinterpret_cast<uint2*>(op + 16 * db + 4 * g) = packed;
      }
    }
  }
}

template <typename T, int G, int MK, bool CAUSAL>
int launch_v2(const void* q, const void* k, const void* v, const void* mask, void* out,
              int64_t batch, int tokens, int kv_heads, const int64_t* st, float scale,
              bool exact, const unsigned char* classes, hipStream_t stream) {
  const dim3 grid(kv_heads, static_cast<unsigned>(batch), (tokens + kV2Queries - 1) / kV2Queries);
  int exponent = 0;
  const bool pow2 = std::is_same_v<T, slc::bf16_t> && std::frexp(scale, &exponent) == 0.5f &&
                    exponent > -100;
  auto kernel = exact ? (pow2 ? prefill_attention_v2_kernel<T, G, MK, CAUSAL, true, true>
                              : prefill_attention_v2_kernel<T, G, MK, CAUSAL, false, true>)
                      : (pow2 ? prefill_attention_v2_kernel<T, G, MK, CAUSAL, true, false>
                              : prefill_attention_v2_kernel<T, G, MK, CAUSAL, false, false>);
  hipLaunchKernelGGL(kernel, grid, dim3((G + 1) * 64), 0,
                     stream, static_cast<const T*>(q), static_cast<const T*>(k),
                     static_cast<const T*>(v), mask, static_cast<T*>(out), tokens, kv_heads,
                     st[0], st[1], st[2], st[3], st[4], st[5], st[6], st[7], st[8], st[9], st[10],
                     st[12], st[13], st[14], scale, MK != 0 ? classes : nullptr);
  return slc_host::check_launch("slc_hip_prefill_attention(grouped)");
}

template <typename T, int G>
int dispatch_v2(const void* q, const void* k, const void* v, const void* mask, int mask_dtype,
                void* out, int64_t batch, int tokens, int kv_heads, int causal,
                const int64_t* st, float scale, bool exact, const unsigned char* classes,
                hipStream_t s) {
#define SLC_V2(MKV)                                                                       \
  return causal ? launch_v2<T, G, MKV, true>(q, k, v, mask, out, batch, tokens, kv_heads, st, scale, exact, classes, s) \
                : launch_v2<T, G, MKV, false>(q, k, v, mask, out, batch, tokens, kv_heads, st, scale, exact, classes, s)
  if (mask == nullptr) SLC_V2(0);
  if (mask_dtype == SLC_BF16) SLC_V2(SLC_BF16 + 1);
  if (mask_dtype == SLC_F16) SLC_V2(SLC_F16 + 1);
  SLC_V2(SLC_F32 + 1);
#undef SLC_V2
}

template <typename T>
int try_v2(const void* q, const void* k, const void* v, const void* mask, int mask_dtype,
           void* out, int64_t batch, int tokens, int kv_heads, int groups, int causal,
           const int64_t* st, float scale, bool exact, const unsigned char* c, hipStream_t s) {
  switch (groups) {
    case 1: return dispatch_v2<T, 1>(q, k, v, mask, mask_dtype, out, batch, tokens, kv_heads, causal, st, scale, exact, c, s);
    case 2: return dispatch_v2<T, 2>(q, k, v, mask, mask_dtype, out, batch, tokens, kv_heads, causal, st, scale, exact, c, s);
    case 4: return dispatch_v2<T, 4>(q, k, v, mask, mask_dtype, out, batch, tokens, kv_heads, causal, st, scale, exact, c, s);
    case 7: return dispatch_v2<T, 7>(q, k, v, mask, mask_dtype, out, batch, tokens, kv_heads, causal, st, scale, exact, c, s);
    default: return dispatch_v2<T, 8>(q, k, v, mask, mask_dtype, out, batch, tokens, kv_heads, causal, st, scale, exact, c, s);
  }
}

template <typename T, int MK, bool CAUSAL>
int launch_mfma(const void* q, const void* k, const void* v, const void* mask, void* out,
                int64_t batch, int tokens, int q_heads, int groups, const int64_t* st,
                float scale, hipStream_t stream) {
  const dim3 grid(q_heads, static_cast<unsigned>(batch), (tokens + kQueries - 1) / kQueries);
  hipLaunchKernelGGL((prefill_attention_mfma_kernel<T, MK, CAUSAL>), grid, dim3(256), 0, stream,
                     static_cast<const T*>(q), static_cast<const T*>(k),
                     static_cast<const T*>(v), mask, static_cast<T*>(out), tokens, q_heads,
                     groups, st[0], st[1], st[2], st[3], st[4], st[5], st[6], st[7], st[8],
                     st[9], st[10], st[11], st[12], st[13], st[14], scale);
  return slc_host::check_launch("slc_hip_prefill_attention");
}

template <typename T, bool CAUSAL>
int dispatch_mask(const void* q, const void* k, const void* v, const void* mask,
                  int mask_dtype, void* out, int64_t batch, int tokens, int q_heads,
                  int groups, const int64_t* st, float scale, hipStream_t s) {
  if (mask == nullptr)
    return launch_mfma<T, 0, CAUSAL>(q, k, v, mask, out, batch, tokens, q_heads, groups, st, scale, s);
  if (mask_dtype == SLC_BF16)
    return launch_mfma<T, SLC_BF16 + 1, CAUSAL>(q, k, v, mask, out, batch, tokens, q_heads, groups, st, scale, s);
  if (mask_dtype == SLC_F16)
    return launch_mfma<T, SLC_F16 + 1, CAUSAL>(q, k, v, mask, out, batch, tokens, q_heads, groups, st, scale, s);
  return launch_mfma<T, SLC_F32 + 1, CAUSAL>(q, k, v, mask, out, batch, tokens, q_heads, groups, st, scale, s);
}

template <typename T>
int launch_generic(const void* q, const void* k, const void* v, const void* mask,
                   int mask_dtype, void* out, int64_t batch, int tokens, int q_heads,
                   int groups, int head_dim, int causal, const int64_t* st,
                   float scale, bool exact, hipStream_t stream) {
  const dim3 grid((tokens + 3) / 4, q_heads, static_cast<unsigned>(batch));
#define SLC_GEN_K(NI, EX)                                                                \
  hipLaunchKernelGGL((prefill_attention_generic_kernel<T, NI, EX>), grid, dim3(256), 0, stream, \
                     static_cast<const T*>(q), static_cast<const T*>(k),                 \
                     static_cast<const T*>(v), mask, mask_dtype, static_cast<T*>(out),   \
                     tokens, q_heads, groups, head_dim, causal, st[0], st[1], st[2],     \
                     st[3], st[4], st[5], st[6], st[7], st[8], st[9], st[10], st[11],    \
                     st[12], st[13], st[14], scale)
#define SLC_GEN(NI)           \
  if (exact) {                \
    SLC_GEN_K(NI, true);      \
  } else {                    \
    SLC_GEN_K(NI, false);     \
  }
  if (head_dim <= 64) {
    SLC_GEN(1);
  } else if (head_dim <= 128) {
    SLC_GEN(2);
  } else {
    SLC_GEN(4);
  }
#undef SLC_GEN
#undef SLC_GEN_K
  return slc_host::check_launch("slc_hip_prefill_attention(generic)");
}

}  // namespace

extern "C" int slc_hip_prefill_attention_classes(
    const void* query, const void* key, const void* value, const void* mask,
    int mask_dtype, const unsigned char* mask_tile_classes, void* output, int dtype,
    int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t tokens, int64_t head_dim,
    int causal, int64_t q_sb, int64_t q_sh, int64_t q_st, int64_t k_sb, int64_t k_sh,
    int64_t k_st, int64_t v_sb, int64_t v_sh, int64_t v_st, int64_t m_sb, int64_t m_sq,
    int64_t m_sk, int64_t o_sb, int64_t o_sh, int64_t o_st, float scale,
    int softmax_order, void* stream) {
  SLC_REQUIRE(slc_host::is_float_dtype(dtype), "slc_hip_prefill_attention: bad dtype %d", dtype);
  SLC_REQUIRE(softmax_order == SLC_SOFTMAX_ONLINE || softmax_order == SLC_SOFTMAX_EXACT,
              "slc_hip_prefill_attention: bad softmax order %d", softmax_order);
  const bool exact = softmax_order == SLC_SOFTMAX_EXACT;
  SLC_REQUIRE(mask == nullptr || slc_host::is_float_dtype(mask_dtype),
              "slc_hip_prefill_attention: bad mask dtype %d", mask_dtype);
  SLC_REQUIRE(batch >= 0 && q_heads > 0 && kv_heads > 0 && tokens >= 0 && head_dim > 0 &&
                  head_dim <= 256 && q_heads % kv_heads == 0,
              "slc_hip_prefill_attention: bad sizes");
  SLC_REQUIRE(batch <= 65535 && q_heads <= 65535 && tokens < (1LL << 30),
              "slc_hip_prefill_attention: sizes exceed grid limits");
  if (batch == 0 || tokens == 0) return SLC_OK;
  SLC_REQUIRE(query && key && value && output, "slc_hip_prefill_attention: null pointer");
  const int64_t st[15] = {q_sb, q_sh, q_st, k_sb, k_sh, k_st, v_sb, v_sh,
                          v_st, m_sb, m_sq, m_sk, o_sb, o_sh, o_st};
  const int groups = static_cast<int>(q_heads / kv_heads);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int T_ = static_cast<int>(tokens);
  const uint64_t bits = reinterpret_cast<uintptr_t>(query) | reinterpret_cast<uintptr_t>(key) |
                        reinterpret_cast<uintptr_t>(value);
  const int64_t strides = q_sb | q_sh | q_st | k_sb | k_sh | k_st | v_sb | v_sh | v_st;
  // The MFMA kernel addresses one (batch, kv-head) K/V slice with 32-bit offsets.
  const bool mfma_ok = (dtype == SLC_BF16 || dtype == SLC_F16) && head_dim == kD &&
                       (bits & 15) == 0 && (strides & 7) == 0 && k_st >= kD && v_st >= kD &&
                       tokens * (k_st > v_st ? k_st : v_st) * 2 < (1LL << 31) &&
                       (tokens + kV2Queries - 1) / kV2Queries <= 65535 &&
                       (tokens + kQueries - 1) / kQueries <= 65535;  // grid z: query blocks
  // The grouped kernel: GQA groups of 1, 2, 4, 7 or 8 heads, and a mask (if
  // any) with unit key stride and 16-byte aligned rows.
  const bool group_ok = groups == 1 || groups == 2 || groups == 4 || groups == 7 || groups == 8;
  const int64_t me = mask == nullptr ? 0 : slc_host::dtype_size(mask_dtype);
  const bool mask_ok =
      mask == nullptr ||
      (m_sk == 1 && (m_sq * me) % 16 == 0 && (m_sb * me) % 16 == 0 &&
       (reinterpret_cast<uintptr_t>(mask) & 15) == 0 &&
       ((tokens - 1) * m_sq + tokens) * me < (1LL << 31));
  const bool out_ok = (reinterpret_cast<uintptr_t>(output) & 7) == 0 &&
                      ((o_sb | o_sh | o_st) & 3) == 0;
  // The grouped kernel takes the row max before the scale factor: positive
  // scale.
  if (mfma_ok && group_ok && mask_ok && out_ok && kv_heads <= 65535 && kUseGrouped &&
      scale > 0.0f) {
    // The class list covers up to kMaxClassTiles key tiles.
    const unsigned char* classes =
        mask != nullptr && (tokens + kKeys - 1) / kKeys <= kMaxClassTiles ? mask_tile_classes : nullptr;
    if (dtype == SLC_BF16)
      return try_v2<slc::bf16_t>(query, key, value, mask, mask_dtype, output, batch, T_,
                                 static_cast<int>(kv_heads), groups, causal, st, scale, exact,
                                 classes, s);
    return try_v2<slc::f16_t>(query, key, value, mask, mask_dtype, output, batch, T_,
                              static_cast<int>(kv_heads), groups, causal, st, scale, exact,
                              classes, s);
  }
  // The single-head MFMA kernel has only the online order; the exact order
  // of shapes the grouped kernel does not take runs on the generic kernel.
  if (mfma_ok && !exact) {
    if (dtype == SLC_BF16) {
      return causal ? dispatch_mask<slc::bf16_t, true>(query, key, value, mask, mask_dtype, output, batch, T_, static_cast<int>(q_heads), groups, st, scale, s)
                    : dispatch_mask<slc::bf16_t, false>(query, key, value, mask, mask_dtype, output, batch, T_, static_cast<int>(q_heads), groups, st, scale, s);
    }
    return causal ? dispatch_mask<slc::f16_t, true>(query, key, value, mask, mask_dtype, output, batch, T_, static_cast<int>(q_heads), groups, st, scale, s)
                  : dispatch_mask<slc::f16_t, false>(query, key, value, mask, mask_dtype, output, batch, T_, static_cast<int>(q_heads), groups, st, scale, s);
  }
  switch (dtype) {
    case SLC_F32:
      return launch_generic<float>(query, key, value, mask, mask_dtype, output, batch, T_,
                                   static_cast<int>(q_heads), groups, static_cast<int>(head_dim),
                                   causal, st, scale, exact, s);
    case SLC_BF16:
      return launch_generic<slc::bf16_t>(query, key, value, mask, mask_dtype, output, batch, T_,
                                         static_cast<int>(q_heads), groups,
                                         static_cast<int>(head_dim), causal, st, scale, exact, s);
    default:
      return launch_generic<slc::f16_t>(query, key, value, mask, mask_dtype, output, batch, T_,
                                        static_cast<int>(q_heads), groups,
                                        static_cast<int>(head_dim), causal, st, scale, exact, s);
  }
}

extern "C" int slc_hip_prefill_attention(
    const void* query, const void* key, const void* value, const void* mask,
    int mask_dtype, void* output, int dtype, int64_t batch, int64_t q_heads,
    int64_t kv_heads, int64_t tokens, int64_t head_dim, int causal, int64_t q_sb,
    int64_t q_sh, int64_t q_st, int64_t k_sb, int64_t k_sh, int64_t k_st,
    int64_t v_sb, int64_t v_sh, int64_t v_st, int64_t m_sb, int64_t m_sq,
    int64_t m_sk, int64_t o_sb, int64_t o_sh, int64_t o_st, float scale,
    int softmax_order, void* stream) {
  return slc_hip_prefill_attention_classes(query, key, value, mask, mask_dtype, nullptr, output,
                                           dtype, batch, q_heads, kv_heads, tokens, head_dim,
                                           causal, q_sb, q_sh, q_st, k_sb, k_sh, k_st, v_sb, v_sh,
                                           v_st, m_sb, m_sq, m_sk, o_sb, o_sh, o_st, scale,
                                           softmax_order, stream);
}

extern "C" int64_t slc_hip_prefill_mask_tile_count(int64_t batch, int64_t tokens) {
  if (batch < 0 || tokens < 0) return -1;
  const int64_t tiles = (tokens + kKeys - 1) / kKeys;
  return batch * tiles * tiles;
}

extern "C" int slc_hip_prefill_mask_tiles(const void* mask, int mask_dtype, int64_t batch,
                                          int64_t tokens, int64_t m_sb, int64_t m_sq,
                                          int64_t m_sk, unsigned char* classes, void* stream) {
  SLC_REQUIRE(slc_host::is_float_dtype(mask_dtype), "slc_hip_prefill_mask_tiles: bad mask dtype %d",
              mask_dtype);
  SLC_REQUIRE(batch >= 0 && tokens >= 0 && batch <= 65535 && tokens < (1LL << 30),
              "slc_hip_prefill_mask_tiles: bad sizes");
  if (batch == 0 || tokens == 0) return SLC_OK;
  SLC_REQUIRE(mask != nullptr && classes != nullptr, "slc_hip_prefill_mask_tiles: null pointer");
  const int64_t tiles = (tokens + kKeys - 1) / kKeys;
  SLC_REQUIRE(tiles <= 65535, "slc_hip_prefill_mask_tiles: too many tiles for the grid");
  const dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(tiles), static_cast<unsigned>(batch));
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int T_ = static_cast<int>(tokens);
  const int64_t me = slc_host::dtype_size(mask_dtype);
  const bool vec = m_sk == 1 && (reinterpret_cast<uintptr_t>(mask) & 15) == 0 && (m_sq * me) % 16 == 0 &&
                   (m_sb * me) % 16 == 0 && (tokens * me) % 16 == 0;
#define SLC_CLASSES(MKV)                                                                          \
  if (vec)                                                                                        \
    hipLaunchKernelGGL((mask_tile_class_kernel<MKV, true>), grid, dim3(256), 0, s, mask, classes, \
                       T_, m_sb, m_sq, m_sk);                                                     \
  else                                                                                            \
    hipLaunchKernelGGL((mask_tile_class_kernel<MKV, false>), grid, dim3(256), 0, s, mask, classes, \
                       T_, m_sb, m_sq, m_sk)
  switch (mask_dtype) {
    case SLC_BF16:
      SLC_CLASSES(SLC_BF16 + 1);
      break;
    case SLC_F16:
      SLC_CLASSES(SLC_F16 + 1);
      break;
    default:
      SLC_CLASSES(SLC_F32 + 1);
      break;
  }
#undef SLC_CLASSES
  return slc_host::check_launch("slc_hip_prefill_mask_tiles");
}
