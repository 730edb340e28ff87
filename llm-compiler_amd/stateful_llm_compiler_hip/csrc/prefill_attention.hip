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
#include "prefill_v2.hpp"

namespace {
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


#ifndef SLC_PREFILL_SHORT_ROUNDS
#define SLC_PREFILL_SHORT_ROUNDS 2
#endif

template <typename T, int G>
int dispatch_v2(const void* q, const void* k, const void* v, const void* mask, int mask_dtype,
                void* out, int64_t batch, int tokens, int kv_heads, int causal,
                const int64_t* st, float scale, bool exact, const unsigned char* classes,
                hipStream_t s) {
  // 32-query workgroups (two MFMA column blocks per consumer wave) unless
  // their grid is at most SLC_PREFILL_SHORT_ROUNDS workgroups per CU (two fit
  // on a CU): short sequences then take 16-query workgroups, twice the grid
  // for the same key tiles.  B8 T512 exact with a mask: 31.2 -> 21.6 us;
  // T1024: 64.6 -> 58.3; at T4096 the 32-query form is 8 % faster.
  const int64_t grid32 = int64_t{kv_heads} * batch * ((tokens + 31) / 32);
  const bool short_grid = grid32 <= int64_t{SLC_PREFILL_SHORT_ROUNDS} * slc_host::device_cu_count();
  // One braced statement: each use below sits under an if.
#define SLC_V2(MKV)                                                                                  \
  {                                                                                                   \
    if (short_grid)                                                                                   \
      return causal ? slc_prefill::launch_v2_short<T, G, MKV, true>(q, k, v, mask, out, batch, tokens, \
                                                                    kv_heads, st, scale, exact, classes, s) \
                    : slc_prefill::launch_v2_short<T, G, MKV, false>(q, k, v, mask, out, batch, tokens, \
                                                                     kv_heads, st, scale, exact, classes, s); \
    return causal ? launch_v2<T, G, MKV, true, 2>(q, k, v, mask, out, batch, tokens, kv_heads, st, scale, exact, classes, s) \
                  : launch_v2<T, G, MKV, false, 2>(q, k, v, mask, out, batch, tokens, kv_heads, st, scale, exact, classes, s); \
  }
  if (mask == nullptr) SLC_V2(0)
  if (mask_dtype == SLC_BF16) SLC_V2(SLC_BF16 + 1)
  if (mask_dtype == SLC_F16) SLC_V2(SLC_F16 + 1)
  SLC_V2(SLC_F32 + 1)
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
                       (tokens + 15) / 16 <= 65535 &&
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
