// Balanced split-sequence decode attention (online softmax order).
//
// Same result contract as the fixed-chunk kernel in decode_attention.hip
// (reference: src/stateful_llm_compiler/execution.py:281-327 for the math,
// backends/triton_attention.py:10-131 for the fast-path contract), with a
// different division of the work:
//
//  * A sequence is (batch, head block): with KH = 2 one wave streams whole
//    token rows of two kv heads at once (their 14 query heads share the 16
//    MFMA columns), which halves the softmax work per byte; else KH = 1.
//  * The lengths live on the device, so every workgroup reads them all and
//    sizes the split itself: sequence s of ntb_s 32-token tiles gets
//    k_s = ceil(ntb_s / T) workgroups for the smallest tile budget T with
//    sum k_s <= grid, and its tiles are split evenly over them.  Every
//    workgroup thus streams one contiguous piece of about the same size
//    whatever the spread of the lengths (a fixed chunk per sequence lets the
//    longest sequence set the kernel time; a workgroup whose range crossed
//    into another sequence would refill its load pipeline at loaded-memory
//    latency).  The host sizes the grid from the CU count and the capacity.
//  * A sequence of one piece is written directly.  Otherwise each piece
//    stores its (max, sum, acc) in the workgroup's slot; after one agent-
//    scope release fence per workgroup, the workgroup whose arrival completes
//    the sequence's count takes an acquire fence and folds the pieces in
//    order (deterministic for given lengths).
//  * The fused RoPE + KV store + attention op keeps the fixed-chunk grid, so
//    this variant is the plain op's only.
// One workgroup = 4 wavefronts; the tile math (MFMA scores, lazy-rescale
// online softmax, selector-MFMA P.V) is the fixed-chunk kernel's.
#include <algorithm>
#include <mutex>
#include <unordered_map>

#include "common.hpp"
#include "decode_tiles.hpp"
#include "op_math.hpp"

namespace slc_decode {

namespace {

struct StreamParams {
  const void* query;
  const void* key_buffer;
  const void* value_buffer;
  const void* lengths;
  const void* mask;
  void* output;
  float* part;        // [grid][cols * (D + 2), padded to 16 bytes]
  int* seg_counters;  // [batch * kv_heads], zero between calls
  int batch, q_heads, kv_heads, groups;
  int capacity;  // < 2^30 (host check)
  int limit;     // min(mask_len, capacity)
  int mask_len;
  int64_t q_sb, q_sh, kv_sb, kv_sh, m_sb, o_sb, o_sh;
  int kv_ss, m_ss;
  float scale;
};

constexpr float kRescale = 8.0f;  // lazy-rescale threshold, log2 units
#ifndef SLC_STREAM_TILES
#define SLC_STREAM_TILES 1
#endif
// One tile (16 KB with KH = 2) in flight per wave measured faster than two:
// the grid keeps ~16 MB in flight, which already holds HBM at its sustained
// rate, and more only lengthens the loaded latency every pipeline start pays.
constexpr int NB = SLC_STREAM_TILES;  // K/V tiles in flight per wave

// KH: kv heads per sequence (1, or 2 when both heads' query heads fit the 16
// MFMA columns).  With KH = 2 one wave streams whole token rows of both kv
// heads: the scores of each head come from its own K . Q^T, every lane keeps
// those of its column's head, and P.V runs once per head with the other
// head's columns of P zeroed -- the softmax work per byte halves.
template <typename T, int D, int KH, int MK, bool L64>
__global__ __launch_bounds__(kThreads) void decode_stream_kernel(StreamParams p) {
  using M = Mfma<T>;
  constexpr int KK = D / 32;  // MFMA k-steps over head_dim
  constexpr int DB = D / 16;  // 16-dim output blocks
  constexpr int kCombineBytes = kWaves * (2 * kMaxGroups + kMaxGroups * D) * 4;

  __shared__ __attribute__((aligned(16))) unsigned char smem[kCombineBytes];
  __shared__ int s_lens[kWaves][kStreamMaxBatch];  // each wave's copy of the attended lengths
  __shared__ int s_last;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int g = lane >> 4;  // lane group: MFMA k-slice / output row block
  const int c = lane & 15;  // MFMA row (A) / column (B, C)
  const int B = p.batch;
  const int NS = p.kv_heads / KH;  // segments (head blocks) per batch
  const int cols = KH * p.groups;  // query heads of a segment
  const int w = blockIdx.x;
  const int kc = c < cols ? c / p.groups : 0;  // lane column's kv head in the block

  // ---- attended lengths, the tile budget and the workgroup's piece --------
  // Sequence (b, hb) has ntb = ceil(len_b / 32) tiles.  Every sequence gets
  // k_b = ceil(ntb / T) workgroups for the smallest tile budget T with
  // sum_b NS * k_b <= grid, and its tiles are split evenly over them: each
  // workgroup streams one contiguous piece of one sequence (a workgroup that
  // switched sequences mid-range would refill its load pipeline at loaded-
  // memory latency).  Every wave works the partition out on its own, 64
  // batches per step with lane shuffles and its own LDS copy of the tile
  // counts, so no barrier stands before the first K/V loads.
  int* my_len = s_lens[wave];
  const int nchunk = (B + 63) / 64;
  int N = 0, S = 0, maxntb = 0;
  for (int ch = 0; ch < nchunk; ++ch) {
    const int b = ch * 64 + lane;
    int ntb = 0;
    if (b < B) {
      int64_t len = L64 ? static_cast<const int64_t*>(p.lengths)[b]
                        : static_cast<int64_t>(static_cast<const int32_t*>(p.lengths)[b]);
      len = len < 0 ? 0 : (len < p.limit ? len : p.limit);
      ntb = static_cast<int>((len + kTile - 1) / kTile);
      my_len[b] = static_cast<int>(len);
    }
    N += ntb;
    S += ntb > 0 ? 1 : 0;
    maxntb = max(maxntb, ntb);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    N += __shfl_xor(N, o, 64);
    S += __shfl_xor(S, o, 64);
    maxntb = max(maxntb, __shfl_xor(maxntb, o, 64));
  }
  N *= NS;
  S *= NS;
  const int grid = static_cast<int>(gridDim.x);
  // Smallest feasible budget T: sum ceil(ntb / T) <= sum (ntb / T + 1) =
  // N / T + S, so T = ceil(N / (grid - S)) is feasible when grid > S; search
  // [ceil(N / grid), that].  With as many sequences as workgroups or more,
  // each sequence is one piece (T = longest) and the workgroups loop.
  int budget = maxntb;
  if (N > 0 && grid > S) {
    int tlo = max(1, (N + grid - 1) / grid);
    int thi = min(maxntb, (N + (grid - S) - 1) / (grid - S));
    while (tlo < thi) {
      const int mid = (tlo + thi) >> 1;
      int need = 0;
      for (int b = lane; b < B; b += 64) need += ((my_len[b] + kTile - 1) / kTile + mid - 1) / mid;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) need += __shfl_xor(need, o, 64);
      if (need * NS <= grid) thi = mid; else tlo = mid + 1;
    }
    budget = tlo;
  }
  budget = max(budget, 1);
  // Piece vw: the batch whose workgroup range [W_b, W_b + NS k_b) holds it.
  int V = 0;  // pieces in all
  auto find_piece = [&](int vw, int& pb, int& pk, int& pfirst) {
    int carry = 0;
    pb = -1;
    for (int ch = 0; ch < nchunk; ++ch) {
      const int b = ch * 64 + lane;
      const int kb = b < B ? ((my_len[b] + kTile - 1) / kTile + budget - 1) / budget : 0;
      int incl = kb * NS;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int v = __shfl_up(incl, o, 64);
        if (lane >= o) incl += v;
      }
      const int excl = carry + incl - kb * NS;
      const uint64_t hit = __ballot(b < B && excl <= vw && vw < carry + incl);
      if (pb < 0 && hit != 0) {
        const int src = __builtin_ctzll(hit);
        pb = ch * 64 + src;
        pk = __shfl(kb, src, 64);
        pfirst = __shfl(excl, src, 64);
      }
      carry += __shfl(incl, 63, 64);
    }
    return carry;
  };
  int my_b = -1, my_k = 0, my_first = 0;
  V = find_piece(w, my_b, my_k, my_first);
  T* output = static_cast<T*>(p.output);

  // Loop-invariant lane data of the tile math.
  const int row_bytes = p.kv_ss * 2;
  int koff[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) koff[j] = (16 * j + c) * row_bytes + 16 * g;
  typename M::vec sel[2];  // sel[h][k][n] = (k == n + 16h)
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    u16x8 e;
#pragma unroll
    for (int i = 0; i < 8; ++i) e.v[i] = (8 * g + i == c + 16 * h) ? bits_of<T>(1.0f) : 0;
    sel[h] = __builtin_bit_cast(typename M::vec, e);
  }
  constexpr int kMaskBytes = MK == SLC_F32 + 1 ? 4 : 2;
  const int mask_step = p.m_ss * kMaskBytes;
  // Contiguous mask rows: the lane's 4 consecutive scores of a 16-token block
  // take one 8-byte (2-byte masks) or 16-byte (fp32) load.  A load that
  // crosses the resource's end returns zero as a whole, so these loads are
  // bounded by the mask row's end (a multiple of 4 tokens), not the piece end;
  // the entries past the piece are read but their scores are -inf.
  const bool mask_vec = MK != 0 && p.m_ss == 1 && p.mask_len % 4 == 0 &&
                        (reinterpret_cast<uintptr_t>(p.mask) & 15) == 0 &&
                        (p.m_sb * kMaskBytes) % 16 == 0;
  float* sm_m = reinterpret_cast<float*>(smem);
  float* sm_l = sm_m + kWaves * kMaxGroups;
  float* sm_o = sm_l + kWaves * kMaxGroups;  // [wave][column][D]
  const int slot_floats = (cols * (D + 2) + 3) & ~3;  // 16-byte aligned slots

  struct Tile {
    uint4 k[KH][2][KK];
    uint4 v[KH][2][KK];
    float mk[MK == 0 ? 1 : 8];
  };

  // One piece: tokens [tok_lo, tok_hi) of sequence (b, hb).
  // slot == nullptr: the piece is the whole sequence, written to the output.
  auto run_piece = [&](int b, int hb, int tok_lo, int tok_hi, float* slot) {
    const char* kbase[KH];
    const char* vbase[KH];
#pragma unroll
    for (int k = 0; k < KH; ++k) {
      const int64_t off = b * p.kv_sb + (hb * KH + k) * p.kv_sh;
      kbase[k] = reinterpret_cast<const char*>(static_cast<const T*>(p.key_buffer) + off);
      vbase[k] = reinterpret_cast<const char*>(static_cast<const T*>(p.value_buffer) + off);
    }
    const char* mbase = MK == 0 ? nullptr
                                : static_cast<const char*>(p.mask) + b * p.m_sb * kMaskBytes;
    // Q^T as the B operand: lane (column c, k-slice g) holds dims kk*32+8g..+7
    // of query head hb*cols + c.
    uint4 qraw[KK];
    typename M::vec qv[KK];
    const int head = hb * cols + c;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      qraw[kk] = make_uint4(0, 0, 0, 0);
      if (c < cols)
        qraw[kk] = *reinterpret_cast<const uint4*>(static_cast<const T*>(p.query) +
                                                   b * p.q_sb + head * p.q_sh + kk * 32 + 8 * g);
    }
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) qv[kk] = as_vec<T>(qraw[kk]);

    // 32 token rows of K and V of every head of the block (and the mask
    // entries of the lane's 8 scores) through buffer resources bounded at the
    // piece end: rows past it load zero without touching memory.
    auto load_tile = [&](int t0, Tile& tile) {
      const int rows = tok_hi - t0;
      const int nbytes = rows > 0 ? rows * row_bytes : 0;
      const int64_t shift = static_cast<int64_t>(t0) * row_bytes;
#pragma unroll
      for (int k = 0; k < KH; ++k) {
        const __amdgpu_buffer_rsrc_t rk = make_rsrc(kbase[k] + shift, nbytes);
        const __amdgpu_buffer_rsrc_t rv = make_rsrc(vbase[k] + shift, nbytes);
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int kk = 0; kk < KK; ++kk) {
            tile.k[k][j][kk] = buffer_load16(rk, koff[j] + kk * 64);
            tile.v[k][j][kk] = buffer_load16(rv, koff[j] + kk * 64);
          }
      }
      if constexpr (MK != 0) {
        const int mrows = mask_vec ? p.mask_len - t0 : rows;
        const __amdgpu_buffer_rsrc_t rm =
            make_rsrc(mbase + static_cast<int64_t>(t0) * mask_step, mrows > 0 ? mrows * mask_step : 0);
        if (mask_vec) {
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const int off = (16 * j + 4 * g) * kMaskBytes;
            if constexpr (MK == SLC_F32 + 1) {
              const uint4 q4 = buffer_load16(rm, off);
              tile.mk[4 * j + 0] = __uint_as_float(q4.x) * kLog2e;
              tile.mk[4 * j + 1] = __uint_as_float(q4.y) * kLog2e;
              tile.mk[4 * j + 2] = __uint_as_float(q4.z) * kLog2e;
              tile.mk[4 * j + 3] = __uint_as_float(q4.w) * kLog2e;
            } else {
              const uint2 q2 =
                  __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rm, off, 0, 0));
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const uint32_t word = r < 2 ? q2.x : q2.y;
                const uint16_t bits = static_cast<uint16_t>(word >> (16 * (r & 1)));
                float mv;
                if constexpr (MK == SLC_BF16 + 1) mv = slc::to_f32(slc::bf16_t{bits});
                else mv = slc::to_f32(slc::f16_t{bits});
                tile.mk[4 * j + r] = mv * kLog2e;
              }
            }
          }
        } else {
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int off = (16 * j + 4 * g + r) * mask_step;
              float mv;
              if constexpr (MK == SLC_F32 + 1) {
                mv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rm, off, 0, 0));
              } else if constexpr (MK == SLC_BF16 + 1) {
                mv = slc::to_f32(slc::bf16_t{
                    static_cast<uint16_t>(__builtin_amdgcn_raw_buffer_load_b16(rm, off, 0, 0))});
              } else {
                mv = slc::to_f32(slc::f16_t{
                    static_cast<uint16_t>(__builtin_amdgcn_raw_buffer_load_b16(rm, off, 0, 0))});
              }
              tile.mk[4 * j + r] = mv * kLog2e;
            }
        }
      }
    };

    constexpr int kStride = kWaves * kTile;
    const int t_first = tok_lo + wave * kTile;
    Tile tiles[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) load_tile(t_first + i * kStride, tiles[i]);

    float m_run = -INFINITY;
    float l_run = 0.0f;
    f32x4_t acc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // S_k^T = K_k.Q^T per head of the block (two 16-token MFMA blocks; lane
    // holds tokens 16j+4g+r of column c), the lane keeping its column's head;
    // q.k and its scaling rounded to the tensor dtype as the reference's bf16
    // matmul and multiply do; softmax in fp32, log2 units, lazy rescale;
    // O^T += V_k^T.P_k^T per head, V^T formed by exact selector MFMAs and P_k
    // zero outside head k's columns.
    auto compute_tile = [&](int t0, const Tile& tile) {
      f32x4_t st[KH][2];
#pragma unroll
      for (int k = 0; k < KH; ++k)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          st[k][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kk = 0; kk < KK; ++kk)
            st[k][j] = M::run(as_vec<T>(tile.k[k][j][kk]), qv[kk], st[k][j]);
        }
      float s[8];
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float raw = KH == 1 ? st[0][j][r] : (kc == 0 ? st[0][j][r] : st[KH - 1][j][r]);
          const float rounded = slc::round_to<T>(slc::round_to<T>(raw) * p.scale);
          float v = rounded * kLog2e;
          if constexpr (MK != 0) v += tile.mk[4 * j + r];
          s[4 * j + r] = t0 + 16 * j + 4 * g + r < tok_hi ? v : -INFINITY;
        }
      float mx = s[0];
#pragma unroll
      for (int i = 1; i < 8; ++i) mx = fmaxf(mx, s[i]);
      mx = slc::max_xor32(slc::max_xor16(mx));
      if (__any(mx > m_run + kRescale)) {
        const float m_new = fmaxf(m_run, mx);
        const float alpha = fast_exp2(m_run - (m_new == -INFINITY ? 0.0f : m_new));
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < DB; ++db) acc[db] = acc[db] * alpha;
        m_run = m_new;
      }
      const float m_use = m_run == -INFINITY ? 0.0f : m_run;
      u16x8 pbits;
      float psum = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float pr = fast_exp2(s[i] - m_use);
        psum += pr;
        pbits.v[i] = bits_of<T>(pr);
      }
      l_run += psum;
      const uint4 praw = __builtin_bit_cast(uint4, pbits);
      const uint4 zero4 = make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int k = 0; k < KH; ++k) {
        const typename M::vec pv =
            as_vec<T>(KH == 1 || kc == k ? praw : zero4);
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const f32x4_t zero = f32x4_t{0.f, 0.f, 0.f, 0.f};
          const f32x4_t x0 = M::run(as_vec<T>(tile.v[k][0][db >> 1]), sel[db & 1], zero);
          const f32x4_t x1 = M::run(as_vec<T>(tile.v[k][1][db >> 1]), sel[db & 1], zero);
          u16x8 a;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            a.v[r] = bits_of<T>(x0[r]);
            a.v[4 + r] = bits_of<T>(x1[r]);
          }
          acc[db] = M::run(__builtin_bit_cast(typename M::vec, a), pv, acc[db]);
        }
      }
    };
    // NB tiles in flight per wave: tile i is consumed, then refilled NB
    // sweeps ahead (past the piece end the refill is a zero-length range).
    for (int t0 = t_first; t0 < tok_hi; t0 += NB * kStride) {
      bool done = false;
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        const int tt = t0 + i * kStride;
        if (!done && tt < tok_hi) {
          compute_tile(tt, tiles[i]);
          load_tile(tt + NB * kStride, tiles[i]);
        } else {
          done = true;
        }
      }
    }

    // Cross-wave combine.
    l_run += __shfl_xor(l_run, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);
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
    // One thread per 4 consecutive dims of a column: the partial (or the
    // output) leaves as one 16-byte (8-byte) store.
    for (int idx = tid; idx < cols * (D / 4); idx += kThreads) {
      const int hd = idx / (D / 4);
      const int d0 = (idx % (D / 4)) * 4;
      float mmax = -INFINITY;
#pragma unroll
      for (int v = 0; v < kWaves; ++v) mmax = fmaxf(mmax, sm_m[v * kMaxGroups + hd]);
      const float mu = mmax == -INFINITY ? 0.0f : mmax;
      float lsum = 0.0f;
      float4 osum = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int v = 0; v < kWaves; ++v) {
        const float f = fast_exp2(sm_m[v * kMaxGroups + hd] - mu);
        lsum += f * sm_l[v * kMaxGroups + hd];
        const float4 o = *reinterpret_cast<const float4*>(sm_o + (v * kMaxGroups + hd) * D + d0);
        osum.x += f * o.x;
        osum.y += f * o.y;
        osum.z += f * o.z;
        osum.w += f * o.w;
      }
      if (slot == nullptr) {
        T* out = output + b * p.o_sb + (hb * cols + hd) * p.o_sh + d0;
        out[0] = slc::from_f32<T>(osum.x / lsum);
        out[1] = slc::from_f32<T>(osum.y / lsum);
        out[2] = slc::from_f32<T>(osum.z / lsum);
        out[3] = slc::from_f32<T>(osum.w / lsum);
      } else {
        *reinterpret_cast<float4*>(slot + hd * D + d0) = osum;
        if (d0 == 0) {
          slot[cols * D + hd] = mmax;
          slot[cols * D + cols + hd] = lsum;
        }
      }
    }
    __syncthreads();  // the combine area is reused by the next piece
  };

  // ---- the workgroup's piece(s) ----------------------------------------------
  // Piece vw: sequence (b, hb), share r of its k workgroups.  With more pieces
  // than workgroups (only when every sequence is one piece) the grid loops.
  int part_seg = -1, part_np = 0, part_first = 0;
  for (int vw = w; vw < V; vw += grid) {
    int b = my_b, k = my_k, first = my_first;
    if (vw != w) find_piece(vw, b, k, first);
    const int len = my_len[b];
    const int ntb = (len + kTile - 1) / kTile;
    const int hb = (vw - first) / k;
    const int r = vw - first - hb * k;
    const int t_lo = r * ntb / k;
    const int t_hi = (r + 1) * ntb / k;
    const int tok_hi = min(t_hi * kTile, len);
    float* slot = k == 1 ? nullptr : p.part + static_cast<int64_t>(vw) * slot_floats;
    run_piece(b, hb, t_lo * kTile, tok_hi, slot);
    if (k > 1) {
      part_seg = b * NS + hb;  // k > 1 only when V <= grid: one piece per workgroup
      part_np = k;
      part_first = first + hb * k;
    }
  }

  // ---- sequences with no attended token: NaN rows, as the reference's
  // softmax over an all -inf row gives (batch b's by workgroup b mod grid).
  for (int b = w; b < B; b += grid) {
    if (my_len[b] != 0) continue;
    for (int idx = lane; idx < p.q_heads * D; idx += 64)
      if (wave == 0) output[b * p.o_sb + (idx / D) * p.o_sh + idx % D] = slc::from_f32<T>(__builtin_nanf(""));
  }
  // ---- arrival: merge a completed sequence, advance the lengths -------------
  if (part_seg < 0) return;
  if (tid == 0) {
    // The barrier ending the piece ordered every wave's partial stores before
    // this thread's release.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    int last = 0;
    if (part_seg >= 0) {
      int* counter = p.seg_counters + part_seg;
      const int before = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
      if (before == part_np - 1) {
        rearm(counter);
        last |= 1;
      }
    }
    if (last != 0) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    s_last = last;
  }
  __syncthreads();
  const int last = s_last;
  if (last & 1) {
    // Merge the sequence's pieces in workgroup order: piece r of (b, hb) sits
    // in slot W_b + hb * k + r.
    const int b = part_seg / NS;
    const int hb = part_seg - b * NS;
    const int np = part_np;
    auto slot_of = [&](int r) { return p.part + static_cast<int64_t>(part_first + r) * slot_floats; };
    // One thread per 4 consecutive dims of a column folds the pieces in
    // order with an online rescale; the loads of 16 pieces are issued before
    // any is used (one round trip for up to 16 pieces).
    constexpr int U = 16;
    for (int idx = tid; idx < cols * (D / 4); idx += kThreads) {
      const int hd = idx / (D / 4);
      const int d0 = (idx % (D / 4)) * 4;
      float mrun = -INFINITY, lrun = 0.0f;
      float4 arun = make_float4(0.f, 0.f, 0.f, 0.f);
      for (int k0 = 0; k0 < np; k0 += U) {
        float m[U], l[U];
        float4 a[U];
#pragma unroll
        for (int k = 0; k < U; ++k) {
          const float* sl = slot_of(k0 + k < np ? k0 + k : 0);
          m[k] = sl[cols * D + hd];
          l[k] = sl[cols * D + cols + hd];
          a[k] = *reinterpret_cast<const float4*>(sl + hd * D + d0);
        }
#pragma unroll
        for (int k = 0; k < U; ++k) {
          if (k0 + k >= np) break;
          const float mnew = fmaxf(mrun, m[k]);
          const float base = mnew == -INFINITY ? 0.0f : mnew;
          const float fo = fast_exp2(mrun - base);  // exp2(-inf) = 0: nothing held yet
          const float fk = fast_exp2(m[k] - base);  // an all-masked piece weighs 0
          lrun = lrun * fo + l[k] * fk;
          arun.x = arun.x * fo + a[k].x * fk;
          arun.y = arun.y * fo + a[k].y * fk;
          arun.z = arun.z * fo + a[k].z * fk;
          arun.w = arun.w * fo + a[k].w * fk;
          mrun = mnew;
        }
      }
      const float inv = 1.0f / lrun;
      T* out = output + b * p.o_sb + (hb * cols + hd) * p.o_sh + d0;
      out[0] = slc::from_f32<T>(arun.x * inv);
      out[1] = slc::from_f32<T>(arun.y * inv);
      out[2] = slc::from_f32<T>(arun.z * inv);
      out[3] = slc::from_f32<T>(arun.w * inv);
    }
  }
}

#ifndef SLC_STREAM_ONE_PER_CU
#define SLC_STREAM_ONE_PER_CU 1
#endif

// Dynamic LDS that keeps a second workgroup of `kernel` off its CU (more
// than half of the CU's LDS), so that the grid of one workgroup per CU lands
// one per CU instead of two sharing a CU while another idles.  Cached per
// kernel; 0 when the device or the kernel does not allow it.
size_t one_per_cu_lds(const void* kernel) {
  static std::mutex mu;
  static std::unordered_map<const void*, size_t> cache;
  std::lock_guard<std::mutex> lock(mu);
  const auto it = cache.find(kernel);
  if (it != cache.end()) return it->second;
  size_t dyn = 0;
  int dev = 0, per_cu = 0;
  hipFuncAttributes attr{};
  if (SLC_STREAM_ONE_PER_CU && hipGetDevice(&dev) == hipSuccess &&
      hipDeviceGetAttribute(&per_cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) ==
          hipSuccess &&
      per_cu > 0 && hipFuncGetAttributes(&attr, kernel) == hipSuccess) {
    const size_t target = static_cast<size_t>(per_cu) / 2 + 1024;
    if (attr.sharedSizeBytes < target) {
      dyn = target - attr.sharedSizeBytes;
      if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                              static_cast<int>(dyn)) != hipSuccess) {
        (void)hipGetLastError();
        dyn = 0;
      }
    }
  }
  cache.emplace(kernel, dyn);
  return dyn;
}

#ifndef SLC_STREAM_WGS_PER_CU
#define SLC_STREAM_WGS_PER_CU 1
#endif
#ifndef SLC_STREAM_MIN_TILES
#define SLC_STREAM_MIN_TILES 4
#endif

}  // namespace

bool stream_eligible(int64_t batch, int64_t kv_heads, int64_t groups, int64_t mask_len,
                     int64_t capacity) {
  if (batch <= 0 || batch > kStreamMaxBatch || groups > kMaxGroups) return false;
  const int64_t limit = std::min(mask_len, capacity);
  if (limit <= 0) return false;
  return batch * kv_heads * ((limit + kTile - 1) / kTile) < (int64_t{1} << 31) - 1;
}

// Both kv heads of a block in one wave when their query heads fit the 16
// MFMA columns (head_dim 64: the doubled tile still fits the registers).
bool stream_pair(int64_t head_dim, int64_t kv_heads, int64_t groups) {
  return head_dim == 64 && kv_heads % 2 == 0 && 2 * groups <= kMaxGroups;
}

int64_t stream_workspace_bytes(int64_t q_heads, int64_t kv_heads, int64_t head_dim) {
  const int64_t groups = q_heads / kv_heads;
  const int64_t cols = stream_pair(head_dim, kv_heads, groups) ? 2 * groups : groups;
  return int64_t{kStreamMaxGrid} * ((cols * (head_dim + 2) + 3) & ~int64_t{3}) * 4;
}

int64_t stream_grid(int64_t batch, int64_t segments, int64_t mask_len, int64_t capacity) {
  const int64_t limit = std::min(mask_len, capacity);
  const int64_t tiles = batch * segments * ((limit + kTile - 1) / kTile);
  int64_t grid = int64_t{slc_host::device_cu_count()} * SLC_STREAM_WGS_PER_CU;
  grid = std::min<int64_t>(grid, (tiles + SLC_STREAM_MIN_TILES - 1) / SLC_STREAM_MIN_TILES);
  grid = std::min<int64_t>(grid, kStreamMaxGrid);
  return std::max<int64_t>(grid, 1);
}

int launch_stream(const StreamCall& call) {
  StreamParams p{};
  p.query = call.query;
  p.key_buffer = call.key_buffer;
  p.value_buffer = call.value_buffer;
  p.lengths = call.lengths;
  p.mask = call.mask;
  p.output = call.output;
  SLC_REQUIRE((reinterpret_cast<uintptr_t>(call.workspace) & 15) == 0,
              "slc_hip_decode_attention: workspace must be 16-byte aligned");
  p.part = static_cast<float*>(call.workspace);
  p.seg_counters = call.counters;
  p.batch = static_cast<int>(call.batch);
  p.q_heads = static_cast<int>(call.q_heads);
  p.kv_heads = static_cast<int>(call.kv_heads);
  p.groups = static_cast<int>(call.q_heads / call.kv_heads);
  p.capacity = static_cast<int>(call.capacity);
  p.limit = static_cast<int>(std::min(call.mask_len, call.capacity));
  p.mask_len = static_cast<int>(call.mask_len);
  p.q_sb = call.st[0];
  p.q_sh = call.st[1];
  p.kv_sb = call.st[2];
  p.kv_ss = static_cast<int>(call.st[3]);
  p.kv_sh = call.st[4];
  p.m_sb = call.st[5];
  p.m_ss = static_cast<int>(call.st[6]);
  p.o_sb = call.st[7];
  p.o_sh = call.st[8];
  p.scale = call.scale;
  const bool pair = stream_pair(call.head_dim, call.kv_heads, p.groups);
  const int64_t grid =
      stream_grid(call.batch, call.kv_heads / (pair ? 2 : 1), call.mask_len, call.capacity);
  hipStream_t stream = call.stream;

#define SLC_STREAM_K(TT, DD, KH, MK, L64)                                                     \
  do {                                                                                       \
    const void* fn = reinterpret_cast<const void*>(&decode_stream_kernel<TT, DD, KH, MK, L64>); \
    hipLaunchKernelGGL((decode_stream_kernel<TT, DD, KH, MK, L64>),                         \
                       dim3(static_cast<unsigned>(grid)), dim3(kThreads), one_per_cu_lds(fn), \
                       stream, p);                                                           \
  } while (0)
#define SLC_STREAM_MASK(TT, DD, KH, L64)          \
  if (call.mask == nullptr) {                           \
    SLC_STREAM_K(TT, DD, KH, 0, L64);             \
  } else if (call.mask_dtype == SLC_BF16) {             \
    SLC_STREAM_K(TT, DD, KH, SLC_BF16 + 1, L64);  \
  } else if (call.mask_dtype == SLC_F16) {              \
    SLC_STREAM_K(TT, DD, KH, SLC_F16 + 1, L64);   \
  } else {                                              \
    SLC_STREAM_K(TT, DD, KH, SLC_F32 + 1, L64);   \
  }
#define SLC_STREAM_DIM(TT, L64)          \
  if (pair) {                                  \
    SLC_STREAM_MASK(TT, 64, 2, L64)      \
  } else if (call.head_dim == 64) {            \
    SLC_STREAM_MASK(TT, 64, 1, L64)      \
  } else {                                     \
    SLC_STREAM_MASK(TT, 128, 1, L64)     \
  }
#define SLC_STREAM_DTYPE(L64)               \
  if (call.dtype == SLC_BF16) {                   \
    SLC_STREAM_DIM(slc::bf16_t, L64)        \
  } else {                                        \
    SLC_STREAM_DIM(slc::f16_t, L64)         \
  }

  slc_host::mark_kernel_begin(stream);
  for (int rep = slc_host::timed_repeats(); rep > 0; --rep) {
    if (call.lengths_dtype == SLC_I64) {
      SLC_STREAM_DTYPE(true)
    } else {
      SLC_STREAM_DTYPE(false)
    }
  }
  slc_host::mark_kernel_end(stream);
#undef SLC_STREAM_DTYPE
#undef SLC_STREAM_DIM
#undef SLC_STREAM_MASK
#undef SLC_STREAM_K
  return slc_host::check_launch("slc_hip_decode_attention(balanced)");
}

}  // namespace slc_decode
