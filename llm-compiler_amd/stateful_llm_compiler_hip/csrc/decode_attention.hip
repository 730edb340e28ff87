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
//    batch-32 decode still launches ~1000 workgroups for 256 CUs.  Each chunk
//    writes its (max, sum, acc) partial; the last chunk of a (batch, kv-head)
//    to finish (an atomic ticket per group) merges them and writes the output,
//    so the whole op is a single launch.
//  * Loops stop at the batch's own length, not at the capacity.
// Other dtypes/shapes take a straightforward wave-per-token kernel.
#include "common.hpp"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kTile = 32;   // tokens per wave iteration
constexpr int kWaves = 4;   // wavefronts per workgroup
constexpr int kMaxGroups = 16;

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

template <typename T, int D>
__global__ __launch_bounds__(256) void decode_attention_mfma_kernel(
    const T* __restrict__ query, const T* __restrict__ key_buffer,
    const T* __restrict__ value_buffer, const void* __restrict__ lengths,
    int lengths_dtype, const void* __restrict__ mask, int mask_dtype,
    T* __restrict__ output, float* __restrict__ part_o,
    float* __restrict__ part_ml, int* __restrict__ tickets, int q_heads,
    int kv_heads, int groups,
    int64_t capacity, int64_t mask_len, int64_t q_sb, int64_t q_sh,
    int64_t kv_sb, int64_t kv_ss, int64_t kv_sh, int64_t m_sb, int64_t m_ss,
    int64_t o_sb, int64_t o_sh, float scale_log2, int chunk_tokens,
    int nchunks) {
  using M = Mfma<T>;
  using Layout = SharedLayout<T, D>;
  constexpr int KK = D / 32;          // MFMA k-steps over head_dim
  constexpr int DB = D / 16;          // 16-dim output blocks
  constexpr int UNITS_PER_ROW = D / 8;  // 16-byte units per V row
  constexpr int V_UNITS = kTile * UNITS_PER_ROW / 64;  // per lane per tile
  constexpr int VR = v_row<D>();

  __shared__ __attribute__((aligned(16))) unsigned char smem[Layout::kBytes];

  const int chunk = blockIdx.x;
  const int kvh = blockIdx.y;
  const int64_t b = blockIdx.z;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int g = lane >> 4;   // lane group: MFMA k-slice / output row block
  const int c = lane & 15;   // MFMA row (A) / column (B, C)

  int64_t end = slc::load_length(lengths, b, lengths_dtype);
  end = end < 0 ? 0 : end;
  end = end < mask_len ? end : mask_len;
  end = end < capacity ? end : capacity;
  const int64_t chunk_start = static_cast<int64_t>(chunk) * chunk_tokens;
  if (nchunks > 1 && chunk_start >= end) {
    // Nothing of this batch in the chunk.  An empty sequence has no chunk to
    // merge, so chunk 0 writes its result (0/0 = NaN, like the reference's
    // softmax over an all -inf row).
    if (chunk == 0 && end == 0) {
      for (int idx = tid; idx < groups * D; idx += 256) {
        const int qh = kvh * groups + idx / D;
        output[b * o_sb + qh * o_sh + idx % D] = slc::from_f32<T>(0.0f / 0.0f);
      }
    }
    return;
  }
  int64_t chunk_end = chunk_start + chunk_tokens;
  chunk_end = chunk_end < end ? chunk_end : end;

  // Q^T as the B operand: lane (head c, k-slice g) holds dims kk*32+8g..+7.
  typename M::vec qv[KK];
  {
    const int head = kvh * groups + c;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      uint4 raw = make_uint4(0, 0, 0, 0);
      if (c < groups) {
        raw = *reinterpret_cast<const uint4*>(query + b * q_sb + head * q_sh +
                                              kk * 32 + 8 * g);
      }
      qv[kk] = as_vec<T>(raw);
    }
  }

  const T* kbase = key_buffer + b * kv_sb + kvh * kv_sh;
  const T* vbase = value_buffer + b * kv_sb + kvh * kv_sh;
  uint16_t* vtile = reinterpret_cast<uint16_t*>(smem) + wave * Layout::kVTileElems;

  float m_run = -INFINITY;
  float l_run = 0.0f;
  f32x4_t acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) acc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int64_t last_row = chunk_end > 0 ? chunk_end - 1 : 0;
  auto load_tile = [&](int64_t t0, uint4 (&kr)[2][KK], uint4 (&vr)[V_UNITS]) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      int64_t tok = t0 + 16 * j + c;
      tok = tok < last_row ? tok : last_row;
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        kr[j][kk] = *reinterpret_cast<const uint4*>(kbase + tok * kv_ss +
                                                    kk * 32 + 8 * g);
      }
    }
#pragma unroll
    for (int i = 0; i < V_UNITS; ++i) {
      const int u = i * 64 + lane;
      int64_t tok = t0 + u / UNITS_PER_ROW;
      tok = tok < last_row ? tok : last_row;
      vr[i] = *reinterpret_cast<const uint4*>(vbase + tok * kv_ss +
                                              (u % UNITS_PER_ROW) * 8);
    }
  };

  int64_t t0 = chunk_start + static_cast<int64_t>(wave) * kTile;
  uint4 kr[2][KK], vr[V_UNITS];
  if (t0 < chunk_end) load_tile(t0, kr, vr);

  for (; t0 < chunk_end; t0 += kWaves * kTile) {
    // Prefetch the wave's next tile while this one is computed.
    const int64_t t_next = t0 + kWaves * kTile;
    uint4 kn[2][KK], vn[V_UNITS];
    if (t_next < chunk_end) load_tile(t_next, kn, vn);

    // Stage V (rows past the chunk end are zeroed so 0 * garbage stays 0).
#pragma unroll
    for (int i = 0; i < V_UNITS; ++i) {
      const int u = i * 64 + lane;
      const int row = u / UNITS_PER_ROW;
      uint4 val = (t0 + row < chunk_end) ? vr[i] : make_uint4(0, 0, 0, 0);
      uint2* dst = reinterpret_cast<uint2*>(vtile + row * VR +
                                            (u % UNITS_PER_ROW) * 8);
      dst[0] = make_uint2(val.x, val.y);
      dst[1] = make_uint2(val.z, val.w);
    }

    // S^T tile: two 16-token MFMA blocks.
    float s[8];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      f32x4_t st = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        st = M::run(as_vec<T>(kr[j][kk]), qv[kk], st);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t tok = t0 + 16 * j + 4 * g + r;
        float v = st[r] * scale_log2;
        if (mask != nullptr && tok < chunk_end) {
          v += slc::load_as_f32(mask, b * m_sb + tok * m_ss, mask_dtype) * kLog2e;
        }
        s[4 * j + r] = tok < chunk_end ? v : -INFINITY;
      }
    }

    float mx = s[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) mx = fmaxf(mx, s[i]);
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = fast_exp2(m_run - m_use);
    u16x8 pbits;
    float psum = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float p = fast_exp2(s[i] - m_use);
      psum += p;
      pbits.v[i] = bits_of<T>(p);
    }
    l_run = l_run * alpha + psum;
    m_run = m_new;
    const typename M::vec pv = __builtin_bit_cast(typename M::vec, pbits);

    // LDS writes above must land before the transposed reads below.
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();

#pragma unroll
    for (int db = 0; db < DB; ++db) {
      u16x8 a;
      const int dim = db * 16 + c;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int row = i < 4 ? 4 * g + i : 16 + 4 * g + (i - 4);
        a.v[i] = vtile[row * VR + dim];
      }
      acc[db] = acc[db] * alpha;
      acc[db] = M::run(__builtin_bit_cast(typename M::vec, a), pv, acc[db]);
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();

#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) kr[j][kk] = kn[j][kk];
#pragma unroll
    for (int i = 0; i < V_UNITS; ++i) vr[i] = vn[i];
  }

  // Finish the per-lane partial sums of l over the 4 lane groups.
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);

  __syncthreads();  // V tiles are dead; reuse LDS for the cross-wave merge.
  float* sm_m = reinterpret_cast<float*>(smem);
  float* sm_l = sm_m + kWaves * kMaxGroups;
  float* sm_o = sm_l + kWaves * kMaxGroups;  // [wave][head][D]
  if (g == 0) {
    sm_m[wave * kMaxGroups + c] = m_run;
    sm_l[wave * kMaxGroups + c] = l_run;
  }
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      sm_o[(wave * kMaxGroups + c) * D + db * 16 + 4 * g + r] = acc[db][r];
  __syncthreads();

  for (int idx = tid; idx < groups * D; idx += 256) {
    const int head = idx / D;
    const int d = idx % D;
    float mmax = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mmax = fmaxf(mmax, sm_m[w * kMaxGroups + head]);
    const float mu = mmax == -INFINITY ? 0.0f : mmax;
    float lsum = 0.0f, osum = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = fast_exp2(sm_m[w * kMaxGroups + head] - mu);
      lsum += f * sm_l[w * kMaxGroups + head];
      osum += f * sm_o[(w * kMaxGroups + head) * D + d];
    }
    const int qh = kvh * groups + head;
    if (nchunks == 1) {
      output[b * o_sb + qh * o_sh + d] = slc::from_f32<T>(osum / lsum);
    } else {
      const int64_t p = (b * q_heads + qh) * nchunks + chunk;
      part_o[p * D + d] = osum;
      if (d == 0) {
        part_ml[2 * p] = mmax;
        part_ml[2 * p + 1] = lsum;
      }
    }
  }
  if (nchunks == 1) return;

  // Split-sequence merge: the last chunk of this (batch, kv-head) to arrive
  // combines every chunk's partial.  Release the partials, take a ticket,
  // acquire the other chunks' partials.
  __shared__ int is_last;
  __threadfence();
  __syncthreads();
  const int nvalid = static_cast<int>((end + chunk_tokens - 1) / chunk_tokens);
  int* ticket = tickets + b * kv_heads + kvh;
  if (tid == 0) is_last = atomicAdd(ticket, 1) == nvalid - 1;
  __syncthreads();
  if (!is_last) return;
  __threadfence();
  for (int idx = tid; idx < groups * D; idx += 256) {
    const int qh = kvh * groups + idx / D;
    const int d = idx % D;
    const int64_t base = (b * q_heads + qh) * nchunks;
    float mmax = -INFINITY;
    for (int i = 0; i < nvalid; ++i) mmax = fmaxf(mmax, part_ml[2 * (base + i)]);
    const float mu = mmax == -INFINITY ? 0.0f : mmax;
    float lsum = 0.0f, osum = 0.0f;
    for (int i = 0; i < nvalid; ++i) {
      const float f = fast_exp2(part_ml[2 * (base + i)] - mu);
      lsum += f * part_ml[2 * (base + i) + 1];
      osum += f * part_o[(base + i) * D + d];
    }
    output[b * o_sb + qh * o_sh + d] = slc::from_f32<T>(osum / lsum);
  }
  // Leave the ticket at zero for the next launch that uses this workspace.
  if (tid == 0) *ticket = 0;
}

// Any dtype / head_dim <= 256 / any group size: one workgroup per
// (batch, query head), each wave takes every 4th token and reduces q.k with
// shuffles.  Used for fp32 and for shapes the MFMA kernel does not cover.
template <typename T, int NI>
__global__ __launch_bounds__(256) void decode_attention_generic_kernel(
    const T* __restrict__ query, const T* __restrict__ key_buffer,
    const T* __restrict__ value_buffer, const void* __restrict__ lengths,
    int lengths_dtype, const void* __restrict__ mask, int mask_dtype,
    T* __restrict__ output, int q_heads, int groups, int head_dim,
    int64_t capacity, int64_t mask_len, int64_t q_sb, int64_t q_sh,
    int64_t kv_sb, int64_t kv_ss, int64_t kv_sh, int64_t m_sb, int64_t m_ss,
    int64_t o_sb, int64_t o_sh, float scale_log2) {
  __shared__ float sm_m[kWaves];
  __shared__ float sm_l[kWaves];
  __shared__ float sm_o[kWaves][NI * 64];
  const int64_t b = blockIdx.x / q_heads;
  const int h = blockIdx.x % q_heads;
  const int kvh = h / groups;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  int64_t end = slc::load_length(lengths, b, lengths_dtype);
  end = end < 0 ? 0 : end;
  end = end < mask_len ? end : mask_len;
  end = end < capacity ? end : capacity;

  float q[NI], acc[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int d = lane + 64 * i;
    q[i] = d < head_dim ? slc::to_f32(query[b * q_sb + h * q_sh + d]) : 0.0f;
    acc[i] = 0.0f;
  }
  float m_run = -INFINITY, l_run = 0.0f;
  const T* kbase = key_buffer + b * kv_sb + kvh * kv_sh;
  const T* vbase = value_buffer + b * kv_sb + kvh * kv_sh;
  for (int64_t t = wave; t < end; t += kWaves) {
    float dot = 0.0f;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int d = lane + 64 * i;
      if (d < head_dim) dot += q[i] * slc::to_f32(kbase[t * kv_ss + d]);
    }
    dot = slc::wave_sum(dot);
    float s = dot * scale_log2;
    if (mask != nullptr) s += slc::load_as_f32(mask, b * m_sb + t * m_ss, mask_dtype) * kLog2e;
    const float m_new = fmaxf(m_run, s);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = exp2f(m_run - m_use);
    const float p = exp2f(s - m_use);
    l_run = l_run * alpha + p;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int d = lane + 64 * i;
      const float v = d < head_dim ? slc::to_f32(vbase[t * kv_ss + d]) : 0.0f;
      acc[i] = acc[i] * alpha + p * v;
    }
    m_run = m_new;
  }
  if (lane == 0) {
    sm_m[wave] = m_run;
    sm_l[wave] = l_run;
  }
#pragma unroll
  for (int i = 0; i < NI; ++i) sm_o[wave][lane + 64 * i] = acc[i];
  __syncthreads();
  for (int d = threadIdx.x; d < head_dim; d += 256) {
    float mmax = -INFINITY;
    for (int w = 0; w < kWaves; ++w) mmax = fmaxf(mmax, sm_m[w]);
    const float mu = mmax == -INFINITY ? 0.0f : mmax;
    float lsum = 0.0f, osum = 0.0f;
    for (int w = 0; w < kWaves; ++w) {
      const float f = exp2f(sm_m[w] - mu);
      lsum += f * sm_l[w];
      osum += f * sm_o[w][d];
    }
    output[b * o_sb + h * o_sh + d] = slc::from_f32<T>(osum / lsum);
  }
}

bool mfma_eligible(int dtype, int64_t head_dim, int64_t groups) {
  return (dtype == SLC_BF16 || dtype == SLC_F16) &&
         (head_dim == 64 || head_dim == 128) && groups <= kMaxGroups;
}

// Sequence chunk of the split-sequence grid: the smallest multiple of the
// workgroup's 128-token sweep that keeps the grid near 4 workgroups per CU
// (256 CUs on MI355X).
int64_t choose_chunk(int64_t batch, int64_t kv_heads, int64_t mask_len,
                     int64_t split_tokens) {
  const int64_t sweep = kWaves * kTile;
  if (split_tokens > 0) {
    return slc_host::ceil_div(split_tokens, sweep) * sweep;
  }
  const int64_t target_groups = 1024;
  int64_t chunk = 2 * sweep;
  while (batch * kv_heads * slc_host::ceil_div(mask_len, chunk) > target_groups) {
    chunk *= 2;
  }
  return chunk;
}

// Workspace layout of the split-sequence path:
//   int   tickets[batch * kv_heads]            (zero between launches)
//   float part_o[batch * q_heads * nchunks * D]
//   float part_ml[batch * q_heads * nchunks * 2]
int64_t tickets_bytes(int64_t batch, int64_t kv_heads) {
  return slc_host::ceil_div(batch * kv_heads * 4, 256) * 256;
}

template <typename T, int D>
int launch_mfma(const void* query, const void* kb, const void* vb,
                const void* lengths, int lengths_dtype, const void* mask,
                int mask_dtype, void* output, void* workspace, int64_t batch,
                int64_t q_heads, int64_t kv_heads, int64_t capacity,
                int64_t mask_len, const int64_t* st, float scale_log2,
                int64_t chunk, int64_t nchunks, hipStream_t stream) {
  int* tickets = nullptr;
  float* part_o = nullptr;
  float* part_ml = nullptr;
  if (nchunks > 1) {
    tickets = static_cast<int*>(workspace);
    part_o = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                      tickets_bytes(batch, kv_heads));
    part_ml = part_o + batch * q_heads * nchunks * D;
  }
  const int groups = static_cast<int>(q_heads / kv_heads);
  hipLaunchKernelGGL(
      (decode_attention_mfma_kernel<T, D>),
      dim3(static_cast<unsigned>(nchunks), static_cast<unsigned>(kv_heads),
           static_cast<unsigned>(batch)),
      dim3(256), 0, stream, static_cast<const T*>(query),
      static_cast<const T*>(kb), static_cast<const T*>(vb), lengths,
      lengths_dtype, mask, mask_dtype, static_cast<T*>(output), part_o, part_ml,
      tickets, static_cast<int>(q_heads), static_cast<int>(kv_heads), groups,
      capacity, mask_len, st[0], st[1], st[2], st[3], st[4], st[5], st[6],
      st[7], st[8], scale_log2, static_cast<int>(chunk),
      static_cast<int>(nchunks));
  return slc_host::check_launch("slc_hip_decode_attention");
}

template <typename T>
int launch_generic(const void* query, const void* kb, const void* vb,
                   const void* lengths, int lengths_dtype, const void* mask,
                   int mask_dtype, void* output, int64_t batch, int64_t q_heads,
                   int64_t kv_heads, int64_t head_dim, int64_t capacity,
                   int64_t mask_len, const int64_t* st, float scale_log2,
                   hipStream_t stream) {
  const int groups = static_cast<int>(q_heads / kv_heads);
  const dim3 grid(static_cast<unsigned>(batch * q_heads));
#define SLC_GENERIC(NI)                                                        \
  hipLaunchKernelGGL((decode_attention_generic_kernel<T, NI>), grid, dim3(256), \
                     0, stream, static_cast<const T*>(query),                  \
                     static_cast<const T*>(kb), static_cast<const T*>(vb),     \
                     lengths, lengths_dtype, mask, mask_dtype,                 \
                     static_cast<T*>(output), static_cast<int>(q_heads),       \
                     groups, static_cast<int>(head_dim), capacity, mask_len,   \
                     st[0], st[1], st[2], st[3], st[4], st[5], st[6], st[7],   \
                     st[8], scale_log2)
  if (head_dim <= 64) {
    SLC_GENERIC(1);
  } else if (head_dim <= 128) {
    SLC_GENERIC(2);
  } else {
    SLC_GENERIC(4);
  }
#undef SLC_GENERIC
  return slc_host::check_launch("slc_hip_decode_attention(generic)");
}

}  // namespace

extern "C" int64_t slc_hip_decode_attention_workspace_size(
    int64_t batch, int64_t q_heads, int64_t head_dim, int64_t mask_len,
    int64_t kv_heads, int dtype, int64_t split_tokens) {
  if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || mask_len <= 0 ||
      q_heads % kv_heads != 0) {
    return 0;
  }
  if (!mfma_eligible(dtype, head_dim, q_heads / kv_heads)) return 0;
  const int64_t chunk = choose_chunk(batch, kv_heads, mask_len, split_tokens);
  const int64_t nchunks = slc_host::ceil_div(mask_len, chunk);
  if (nchunks <= 1) return 0;
  return tickets_bytes(batch, kv_heads) +
         batch * q_heads * nchunks * (head_dim + 2) * static_cast<int64_t>(sizeof(float));
}

extern "C" int slc_hip_decode_attention(
    const void* query, const void* key_buffer, const void* value_buffer,
    const void* lengths, int lengths_dtype, const void* mask, int mask_dtype,
    void* output, void* workspace, int64_t workspace_bytes, int dtype,
    int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
    int64_t capacity, int64_t mask_len, int64_t q_stride_b, int64_t q_stride_h,
    int64_t kv_stride_b, int64_t kv_stride_s, int64_t kv_stride_h,
    int64_t mask_stride_b, int64_t mask_stride_s, int64_t out_stride_b,
    int64_t out_stride_h, float scale, int64_t split_tokens, void* stream) {
  SLC_REQUIRE(slc_host::is_float_dtype(dtype),
              "slc_hip_decode_attention: bad dtype %d", dtype);
  SLC_REQUIRE(lengths_dtype == SLC_I64 || lengths_dtype == SLC_I32,
              "slc_hip_decode_attention: lengths must be int64 or int32");
  SLC_REQUIRE(mask == nullptr || slc_host::is_float_dtype(mask_dtype),
              "slc_hip_decode_attention: bad mask dtype %d", mask_dtype);
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
  const int64_t groups = q_heads / kv_heads;
  const int64_t st[9] = {q_stride_b,    q_stride_h,    kv_stride_b,
                         kv_stride_s,   kv_stride_h,   mask_stride_b,
                         mask_stride_s, out_stride_b,  out_stride_h};
  const float scale_log2 = scale * kLog2e;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t ml = mask_len;

  bool use_mfma = mfma_eligible(dtype, head_dim, groups) && ml > 0;
  if (use_mfma) {
    // 16-byte vector loads need 8-element alignment of every row start.
    const uint64_t bits = reinterpret_cast<uintptr_t>(query) |
                          reinterpret_cast<uintptr_t>(key_buffer) |
                          reinterpret_cast<uintptr_t>(value_buffer);
    const int64_t strides = q_stride_b | q_stride_h | kv_stride_b |
                            kv_stride_s | kv_stride_h;
    use_mfma = (bits & 15) == 0 && (strides & 7) == 0;
  }
  if (use_mfma) {
    const int64_t chunk = choose_chunk(batch, kv_heads, ml, split_tokens);
    const int64_t nchunks = slc_host::ceil_div(ml, chunk);
    const int64_t need =
        nchunks > 1 ? tickets_bytes(batch, kv_heads) +
                          batch * q_heads * nchunks * (head_dim + 2) * 4
                    : 0;
    SLC_REQUIRE(nchunks <= 0x7fffffff, "slc_hip_decode_attention: too many chunks");
    SLC_REQUIRE(need == 0 || (workspace != nullptr && workspace_bytes >= need),
                "slc_hip_decode_attention: workspace of %lld bytes needed, got "
                "%lld",
                (long long)need, (long long)workspace_bytes);
    if (dtype == SLC_BF16) {
      if (head_dim == 64)
        return launch_mfma<slc::bf16_t, 64>(query, key_buffer, value_buffer,
                                            lengths, lengths_dtype, mask,
                                            mask_dtype, output, workspace, batch,
                                            q_heads, kv_heads, capacity, ml, st,
                                            scale_log2, chunk, nchunks, s);
      return launch_mfma<slc::bf16_t, 128>(query, key_buffer, value_buffer,
                                           lengths, lengths_dtype, mask,
                                           mask_dtype, output, workspace, batch,
                                           q_heads, kv_heads, capacity, ml, st,
                                           scale_log2, chunk, nchunks, s);
    }
    if (head_dim == 64)
      return launch_mfma<slc::f16_t, 64>(query, key_buffer, value_buffer,
                                         lengths, lengths_dtype, mask,
                                         mask_dtype, output, workspace, batch,
                                         q_heads, kv_heads, capacity, ml, st,
                                         scale_log2, chunk, nchunks, s);
    return launch_mfma<slc::f16_t, 128>(query, key_buffer, value_buffer,
                                        lengths, lengths_dtype, mask,
                                        mask_dtype, output, workspace, batch,
                                        q_heads, kv_heads, capacity, ml, st,
                                        scale_log2, chunk, nchunks, s);
  }
  SLC_REQUIRE(batch * q_heads <= 0x7fffffff,
              "slc_hip_decode_attention: grid too large");
  switch (dtype) {
    case SLC_F32:
      return launch_generic<float>(query, key_buffer, value_buffer, lengths,
                                   lengths_dtype, mask, mask_dtype, output,
                                   batch, q_heads, kv_heads, head_dim, capacity,
                                   ml, st, scale_log2, s);
    case SLC_BF16:
      return launch_generic<slc::bf16_t>(query, key_buffer, value_buffer,
                                         lengths, lengths_dtype, mask,
                                         mask_dtype, output, batch, q_heads,
                                         kv_heads, head_dim, capacity, ml, st,
                                         scale_log2, s);
    default:
      return launch_generic<slc::f16_t>(query, key_buffer, value_buffer,
                                        lengths, lengths_dtype, mask, mask_dtype,
                                        output, batch, q_heads, kv_heads,
                                        head_dim, capacity, ml, st, scale_log2,
                                        s);
  }
}
