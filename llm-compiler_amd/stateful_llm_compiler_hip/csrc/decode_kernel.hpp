// Decode-attention kernel templates shared by the contiguous entry points
// (decode_attention.hip) and the paged ones (decode_paged.hip): each file
// instantiates the variants it launches.  Everything here has internal
// linkage (an anonymous namespace), so every file gets its own copies.
#pragma once

#include <algorithm>
#include <climits>
#include <mutex>
#include <type_traits>

#include "common.hpp"
#include "decode_tiles.hpp"
#include "op_math.hpp"

namespace {

using namespace slc_decode;

template <typename T, int D>
__device__ __forceinline__ void merge_if_last(const float* part_o, const float* part_ml,
                                              T* output, int* counters, unsigned char* smem,
                                              int64_t b, int kvh, int q_heads, int kv_heads,
                                              int groups, int64_t o_sb, int64_t o_sh,
                                              int nchunks, const LenAdvance& adv) {
  const int tid = threadIdx.x;
  __shared__ int is_last;
  __syncthreads();  // every wave's partial stores precede thread 0's release
  if (tid == 0) {
    int* counter = counters + b * kv_heads + kvh;
    const int len_before = adv.counter != nullptr ? count_only(adv.counter) : 0;
    const int before = count_arrival(counter);
    is_last = before == nchunks - 1;
    if (is_last) {
      acquire_partials();
      rearm(counter);
    }
    finish_advance(adv, len_before);
  }
  __syncthreads();
  if (!is_last) return;
  // One round of loads: each thread owns up to two outputs (head, d) and
  // loads every chunk's (max, sum) of their heads and acc of their dims at
  // once, then weighs them in chunk order exactly as the merge kernel does.
  const int64_t head0 = b * q_heads + kvh * groups;
  const int n_out = groups * D;
  for (int base = 0; base < n_out; base += 2 * kThreads) {
    int head[2], dim[2];
    bool valid[2];
#pragma unroll
    for (int o = 0; o < 2; ++o) {
      const int idx = base + tid + o * kThreads;
      valid[o] = idx < n_out;
      head[o] = valid[o] ? idx / D : 0;
      dim[o] = idx % D;
    }
    float mmax[2] = {-INFINITY, -INFINITY};
    float lsum[2] = {0.0f, 0.0f};
    float acc[2] = {0.0f, 0.0f};
    if (nchunks <= kFusedMergeUnroll) {
      // Every chunk's (max, sum, acc) in one batch of loads.
      float m[2][kFusedMergeUnroll], l[2][kFusedMergeUnroll], v[2][kFusedMergeUnroll];
#pragma unroll
      for (int o = 0; o < 2; ++o)
#pragma unroll
        for (int k = 0; k < kFusedMergeUnroll; ++k) {
          const bool ok = valid[o] && k < nchunks;
          const int64_t p = (head0 + head[o]) * nchunks + k;
          m[o][k] = ok ? fetch_partial(part_ml + 2 * p) : -INFINITY;
          l[o][k] = ok ? fetch_partial(part_ml + 2 * p + 1) : 0.0f;
          v[o][k] = ok ? fetch_partial(part_o + p * D + dim[o]) : 0.0f;
        }
#pragma unroll
      for (int o = 0; o < 2; ++o) {
#pragma unroll
        for (int k = 0; k < kFusedMergeUnroll; ++k) mmax[o] = fmaxf(mmax[o], m[o][k]);
        const float mu = mmax[o] == -INFINITY ? 0.0f : mmax[o];
#pragma unroll
        for (int k = 0; k < kFusedMergeUnroll; ++k) {
          if (k < nchunks) {
            const float w = fast_exp2(m[o][k] - mu);  // exp2(-inf) = 0 for empty chunks
            lsum[o] += w * l[o][k];
            acc[o] += w * (w != 0.0f ? v[o][k] : 0.0f);
          }
        }
      }
    }
    // More chunks: pass 1 (max) and pass 2 (weights), the loads of each batch
    // of chunks issued before any is used.
    for (int i0 = 0; nchunks > kFusedMergeUnroll && i0 < nchunks; i0 += kFusedMergeUnroll) {
      float m[2][kFusedMergeUnroll];
#pragma unroll
      for (int o = 0; o < 2; ++o)
#pragma unroll
        for (int k = 0; k < kFusedMergeUnroll; ++k) {
          const int64_t p = (head0 + head[o]) * nchunks + i0 + k;
          m[o][k] = valid[o] && i0 + k < nchunks ? fetch_partial(part_ml + 2 * p) : -INFINITY;
        }
#pragma unroll
      for (int o = 0; o < 2; ++o)
#pragma unroll
        for (int k = 0; k < kFusedMergeUnroll; ++k) mmax[o] = fmaxf(mmax[o], m[o][k]);
    }
    for (int i0 = 0; nchunks > kFusedMergeUnroll && i0 < nchunks; i0 += kFusedMergeUnroll) {
      float m[2][kFusedMergeUnroll], l[2][kFusedMergeUnroll], v[2][kFusedMergeUnroll];
#pragma unroll
      for (int o = 0; o < 2; ++o)
#pragma unroll
        for (int k = 0; k < kFusedMergeUnroll; ++k) {
          const bool ok = valid[o] && i0 + k < nchunks;
          const int64_t p = (head0 + head[o]) * nchunks + i0 + k;
          m[o][k] = ok ? fetch_partial(part_ml + 2 * p) : -INFINITY;
          l[o][k] = ok ? fetch_partial(part_ml + 2 * p + 1) : 0.0f;
          v[o][k] = ok ? fetch_partial(part_o + p * D + dim[o]) : 0.0f;
        }
#pragma unroll
      for (int o = 0; o < 2; ++o) {
        const float mu = mmax[o] == -INFINITY ? 0.0f : mmax[o];
#pragma unroll
        for (int k = 0; k < kFusedMergeUnroll; ++k) {
          if (i0 + k < nchunks) {
            const float w = fast_exp2(m[o][k] - mu);  // exp2(-inf) = 0 for empty chunks
            lsum[o] += w * l[o][k];
            acc[o] += w * (w != 0.0f ? v[o][k] : 0.0f);
          }
        }
      }
    }
#pragma unroll
    for (int o = 0; o < 2; ++o) {
      if (!valid[o]) continue;
      const int qh = kvh * groups + head[o];
      output[b * o_sb + qh * o_sh + dim[o]] = slc::from_f32<T>(acc[o] * (1.0f / lsum[o]));
    }
  }
}

// Rescale the running (max, sum, acc) only when a tile's max exceeds the
// running max by more than this (log2 units): probabilities stay <= 2^8, and
// most tiles skip the accumulator rescale entirely.
constexpr float kRescaleThreshold = 8.0f;

// MK: mask element type (0 = no mask, else an slc_dtype tag + 1), a template
// parameter so the load path has no data-dependent branches.
// EXACT: the reference executor's softmax order -- the probabilities are
// normalised in fp32 and then rounded to the I/O dtype for the P.V product
// (execution.py:319-327: softmax(...).to(query.dtype) then matmul) -- instead
// of rounding the running (unnormalised) probabilities.  One chunk per
// (batch, kv-head): pass 1 streams K, keeps each lane's rounded scores in LDS
// (dynamic shared memory, 1 KB per 32-token tile) and forms the row max and
// sum; pass 2 streams V and weighs it with the normalised, rounded
// probabilities.  K and V are each read once.
// PG: K/V read through a block table (Paging; key_buffer/value_buffer are
// the page pools; with ROPE the new row is written to its position's page).  PG 1: pages of 32 tokens or more
// (one page per 32-row tile); PG 2: 16-token pages (one per 16-row block).
template <typename T, int D, int MK, bool L64, bool ROPE, bool EXACT, int PG = 0>
__global__ __launch_bounds__(kThreads) void decode_attention_mfma_kernel(
    const T* __restrict__ query, const T* __restrict__ key_buffer,
    const T* __restrict__ value_buffer, const void* __restrict__ lengths,
    int lengths_dtype, const void* __restrict__ mask, int mask_dtype,
    T* __restrict__ output, float* __restrict__ part_o,
    float* __restrict__ part_ml, int q_heads, int kv_heads, int groups,
    int64_t capacity, int64_t mask_len, int64_t q_sb, int64_t q_sh,
    int64_t kv_sb, int kv_ss, int64_t kv_sh, int64_t m_sb, int m_ss,
    int64_t o_sb, int64_t o_sh, float scale, int chunk_tokens,
    int nchunks, int* __restrict__ counters, RopeStore rs, Paging pg) {
  using M = Mfma<T>;
  using Layout = SharedLayout<T, D>;
  constexpr int KK = D / 32;            // MFMA k-steps over head_dim
  constexpr int DB = D / 16;            // 16-dim output blocks

  __shared__ __attribute__((aligned(16))) unsigned char smem[Layout::kBytes];
  extern __shared__ uint4 score_lds[];  // EXACT: [tile][lane] rounded scores

  const int chunk = blockIdx.x;
  const int kvh = blockIdx.y;
  const int64_t b = blockIdx.z;
  const int tid = threadIdx.x;
  // readfirstlane: the wave index is wave-uniform, so everything derived from
  // it (tile starts, buffer resources) lives in scalar registers.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int g = lane >> 4;  // lane group: MFMA k-slice / output row block
  const int c = lane & 15;  // MFMA row (A) / column (B, C)

  // Issued first (memory reads complete in issue order, so consuming it
  // later waits only for it), used after the query loads are issued.
  // A vector (buffer) load: a scalar load would share its counter with the
  // kernel-argument loads and be waited for before the tiles are issued.
  // L64: int64 lengths (a template parameter, so no branch separates the load
  // from its use).
  uint32_t length_lo, length_hi = 0;
  {
    constexpr int es = L64 ? 8 : 4;
    const __amdgpu_buffer_rsrc_t rl =
        make_rsrc(static_cast<const char*>(lengths) + b * es, es);
    if constexpr (L64) {
      const auto pair = __builtin_amdgcn_raw_buffer_load_b64(rl, 0, 0, 0);
      length_lo = static_cast<uint32_t>(pair[0]);
      length_hi = static_cast<uint32_t>(pair[1]);
    } else {
      length_lo = static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(rl, 0, 0, 0));
    }
  }
  const int chunk_start = chunk * chunk_tokens;

  // PG: a window of 64 consecutive block-table entries of this sequence, one
  // per lane, from page page_base on, read through a resource bounded at the
  // table's width (entries past it read as 0 and are never used).  A tile
  // picks its page from a register (readlane) instead of waiting on a table
  // read before its K/V loads can issue.  The first window is requested here,
  // beside the length, and covers the first two tiles of every wave; the tile
  // loop moves it (move_window, one table read) before it loads tiles that
  // leave it, so the loads themselves never branch.
  int page_base = PG ? __builtin_amdgcn_readfirstlane(chunk_start >> pg.page_shift) : 0;
  int page_win = 0;
  const int* page_row = PG ? pg.table + b * pg.table_sb : nullptr;
  auto load_window = [&]() {
    const int pages = static_cast<int>(capacity >> pg.page_shift);
    const __amdgpu_buffer_rsrc_t rt =
        make_rsrc(page_row + page_base, page_base < pages ? (pages - page_base) * 4 : 0);
    page_win = static_cast<int>(__builtin_amdgcn_raw_buffer_load_b32(rt, lane * 4, 0, 0));
  };
  if constexpr (PG != 0) load_window();
  // Make the window hold the pages of tokens lo..hi (at most 64 pages apart).
  auto move_window = [&](int lo, int hi) {
    if constexpr (PG != 0) {
      const int lo_page = lo >> pg.page_shift;
      const int hi_page = hi >> pg.page_shift;
      if (static_cast<unsigned>(lo_page - page_base) >= 64u || hi_page - page_base >= 64) {
        page_base = __builtin_amdgcn_readfirstlane(lo_page);
        load_window();
        // Wait for the window here (vmcnt(0)), on this rare path: otherwise
        // the compiler cannot tell at a readlane whether the window is still
        // in flight and drains every tile load before it, on every tile.
        __builtin_amdgcn_s_waitcnt(0x0F70);
      }
    }
  };
  // The pool byte offset of token tok's row (its page from the window).
  auto page_offset = [&](int tok) -> int64_t {
    const int slot = __builtin_amdgcn_readfirstlane((tok >> pg.page_shift) - page_base);
    const int64_t page = __builtin_amdgcn_readlane(page_win, slot);
    return (page * pg.page_stride +
            (tok & ((1 << pg.page_shift) - 1)) * static_cast<int64_t>(kv_ss)) * 2;
  };

  // Q^T as the B operand: lane (head c, k-slice g) holds dims kk*32+8g..+7.
  // ROPE: the query arrives unrotated and is rotated here; every lane also
  // holds its slices of the new token's rotated key and its value (each
  // rotation pair, dims d and d + D/2, is the lane's slices kk and kk + KK/2).
  // (The rotation itself waits until the first tiles are requested: the tile
  // loads must not queue behind these operands.)
  typename M::vec qv[KK];
  uint4 qraw[KK];
  constexpr int KR = ROPE ? KK : 1;
  uint4 knew[KR], vnew[KR], cs[KR], sn[KR];
  {
    const int head = kvh * groups + c;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      qraw[kk] = make_uint4(0, 0, 0, 0);
      if (c < groups) {
        qraw[kk] = *reinterpret_cast<const uint4*>(query + b * q_sb + head * q_sh +
                                                   kk * 32 + 8 * g);
      }
    }
    if constexpr (ROPE) {
      const T* kr = static_cast<const T*>(rs.key) + b * rs.k_sb + kvh * rs.k_sh;
      const T* vr = static_cast<const T*>(rs.value) + b * rs.v_sb + kvh * rs.v_sh;
      const T* cr = static_cast<const T*>(rs.cosine) + b * rs.c_sb;
      const T* sr = static_cast<const T*>(rs.sine) + b * rs.s_sb;
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        const int d = kk * 32 + 8 * g;
        knew[kk] = *reinterpret_cast<const uint4*>(kr + d);
        vnew[kk] = *reinterpret_cast<const uint4*>(vr + d);
        cs[kk] = *reinterpret_cast<const uint4*>(cr + d);
        sn[kk] = *reinterpret_cast<const uint4*>(sr + d);
      }
    } else {
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) qv[kk] = as_vec<T>(qraw[kk]);
    }
  }

  // PG: the pools' kv-head column; the page comes per tile (or 16-row block).
  const int64_t seq_off = PG ? kvh * kv_sh : b * kv_sb + kvh * kv_sh;
  const char* kbase = reinterpret_cast<const char*>(key_buffer + seq_off);
  const char* vbase = reinterpret_cast<const char*>(value_buffer + seq_off);
  constexpr int kMaskBytes = MK == SLC_F32 + 1 ? 4 : 2;
  const char* mbase = MK == 0 ? nullptr
                              : static_cast<const char*>(mask) + b * m_sb * kMaskBytes;
  const int row_bytes = kv_ss * 2;
  const int mask_step = m_ss * kMaskBytes;

  // Loop-invariant per-lane byte offsets inside a tile.
  int koff[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) koff[j] = (16 * j + c) * row_bytes + 16 * g;
  // 0/1 selector B operands: sel[h][k][n] = (k == n + 16h), so that
  // V_block(16 x 32 dims) . sel[h] = the dims 16h..16h+15 of the block.
  typename M::vec sel[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    u16x8 e;
#pragma unroll
    for (int i = 0; i < 8; ++i) e.v[i] = (8 * g + i == c + 16 * h) ? bits_of<T>(1.0f) : 0;
    sel[h] = __builtin_bit_cast(typename M::vec, e);
  }

  float m_run = -INFINITY;
  float l_run = 0.0f;
  f32x4_t acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) acc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  struct Tile {
    uint4 k[2][KK];
    uint4 v[2][KK];
    float mk[MK == 0 ? 1 : 8];
  };
  // One tile = 32 token rows of K and V (and the mask entries of the lane's 8
  // scores) through buffer resources bounded at the chunk end.  K and V use
  // the same lane layout: lane (row c, k-slice g) of 16-row block j holds
  // dims kk*32+8g..+7 of token t0+16j+c.
  // Which: 3 = K and V, 1 = K only, 2 = V only (the EXACT passes).
  auto load_tile = [&](int t0, Tile& tile, int bound, auto which) {
    constexpr int kWhich = decltype(which)::value;
    const int rows = bound - t0;
    if constexpr (PG == 1) {
      // Pages of 32 tokens or more hold a whole tile (tiles start at
      // multiples of 32): one page, one resource per tile, bounded at the
      // chunk end.
      const int nbytes = rows <= 0 ? 0 : (rows < 32 ? rows : 32) * row_bytes;
      const int64_t off = rows > 0 ? page_offset(t0) : 0;
      const __amdgpu_buffer_rsrc_t rk = make_rsrc(kbase + off, nbytes);
      const __amdgpu_buffer_rsrc_t rv = make_rsrc(vbase + off, nbytes);
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
          if constexpr ((kWhich & 1) != 0) tile.k[j][kk] = buffer_load16(rk, koff[j] + kk * 64);
          if constexpr ((kWhich & 2) != 0) tile.v[j][kk] = buffer_load16(rv, koff[j] + kk * 64);
        }
    } else if constexpr (PG == 2) {
      // 16-token pages: each 16-row block from its own page; a block wholly
      // past the chunk end touches no memory.
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int tok = t0 + 16 * j;
        const int brows = rows - 16 * j;
        const int nb = brows <= 0 ? 0 : (brows < 16 ? brows : 16) * row_bytes;
        const int64_t off = brows > 0 ? page_offset(tok) : 0;
        const __amdgpu_buffer_rsrc_t rk = make_rsrc(kbase + off, nb);
        const __amdgpu_buffer_rsrc_t rv = make_rsrc(vbase + off, nb);
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
          const int o = c * row_bytes + 16 * g + kk * 64;
          if constexpr ((kWhich & 1) != 0) tile.k[j][kk] = buffer_load16(rk, o);
          if constexpr ((kWhich & 2) != 0) tile.v[j][kk] = buffer_load16(rv, o);
        }
      }
    } else {
      const int nbytes = rows > 0 ? rows * row_bytes : 0;
      const int64_t shift = static_cast<int64_t>(t0) * row_bytes;
      const __amdgpu_buffer_rsrc_t rk = make_rsrc(kbase + shift, nbytes);
      const __amdgpu_buffer_rsrc_t rv = make_rsrc(vbase + shift, nbytes);
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
          if constexpr ((kWhich & 1) != 0) tile.k[j][kk] = buffer_load16(rk, koff[j] + kk * 64);
          if constexpr ((kWhich & 2) != 0) tile.v[j][kk] = buffer_load16(rv, koff[j] + kk * 64);
        }
    }
    if constexpr (MK != 0) {
      const __amdgpu_buffer_rsrc_t rm =
          make_rsrc(mbase + static_cast<int64_t>(t0) * mask_step,
                    rows > 0 ? rows * mask_step : 0);
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int off = (16 * j + 4 * g + r) * mask_step;
          float mv;
          if constexpr (MK == SLC_F32 + 1) {
            mv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rm, off, 0, 0));
          } else if constexpr (MK == SLC_BF16 + 1) {
            mv = slc::to_f32(slc::bf16_t{static_cast<uint16_t>(
                __builtin_amdgcn_raw_buffer_load_b16(rm, off, 0, 0))});
          } else {
            mv = slc::to_f32(slc::f16_t{static_cast<uint16_t>(
                __builtin_amdgcn_raw_buffer_load_b16(rm, off, 0, 0))});
          }
          tile.mk[4 * j + r] = mv * kLog2e;
        }
    }
  };

  constexpr int kStride = kWaves * kTile;
  const int t_first = chunk_start + wave * kTile;

  // The length is consumed only here, after the query loads were issued
  // (the asm ties its registers to this point; the compiler would otherwise
  // read it into scalars right after the load and wait for it).
  asm volatile("" : "+v"(length_lo), "+v"(length_hi)::"memory");
  int64_t end64 = L64 ? static_cast<int64_t>((static_cast<uint64_t>(length_hi) << 32) | length_lo)
                      : static_cast<int64_t>(static_cast<int32_t>(length_lo));
  // ROPE: the length is the new token's position; attention covers it too.
  const int64_t pos = end64;
  if constexpr (ROPE) end64 = pos + 1;
  end64 = end64 < 0 ? 0 : end64;
  end64 = end64 < mask_len ? end64 : mask_len;
  end64 = end64 < capacity ? end64 : capacity;
  // Host guarantees capacity < 2^30.  The length is one sequence's, so the
  // end is wave-uniform: readfirstlane puts it (and every loop bound derived
  // from it) in scalar registers.  Left in a vector register, the tile loop
  // is compiled as a divergent loop whose exit paths differ in loads issued,
  // and the compiler then waits for every load in flight (vmcnt(0)) at the
  // top of each iteration, draining the tile prefetch.
  const int end = __builtin_amdgcn_readfirstlane(static_cast<int>(end64));
  LenAdvance adv{nullptr, 0, nullptr, 0, nullptr, capacity};
  // ROPE: rotate the new key and write its row (and the value's) from the
  // workgroup of the chunk holding it (the last chunk when it lies past the
  // mask); that workgroup's own tile loads of the row are replaced by the
  // registers (patch below), so no workgroup depends on when the write lands.
  auto store_new_row = [&]() {
    if constexpr (ROPE) {
      rope_slices<T, KK>(knew, cs, sn);
      const bool in_range = pos >= 0 && pos < capacity;
      const int64_t owner =
          in_range ? min(pos / chunk_tokens, static_cast<int64_t>(nchunks) - 1) : 0;
      if (in_range && chunk == owner && wave == 0 && c == 0) {
        // The row's element offset: contiguous, or through the block table.
        int64_t row;
        if constexpr (PG) {
          const int64_t page = pg.table[b * pg.table_sb + (pos >> pg.page_shift)];
          row = page * pg.page_stride + kvh * kv_sh +
                (pos & ((int64_t{1} << pg.page_shift) - 1)) * static_cast<int64_t>(kv_ss);
        } else {
          row = b * kv_sb + kvh * kv_sh + pos * static_cast<int64_t>(kv_ss);
        }
        char* krow = reinterpret_cast<char*>(static_cast<T*>(rs.key_out) + row);
        char* vrow = reinterpret_cast<char*>(static_cast<T*>(rs.value_out) + row);
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
          *reinterpret_cast<uint4*>(krow + kk * 64 + 16 * g) = knew[kk];
          *reinterpret_cast<uint4*>(vrow + kk * 64 + 16 * g) = vnew[kk];
        }
      }
      if (!in_range && chunk == 0 && kvh == 0 && tid == 0 && rs.overflow != nullptr)
        *rs.overflow = 1;
    }
  };
  if constexpr (ROPE) {
    adv = LenAdvance{rs.counters + b, kv_heads * nchunks, rs.lengths_out + b, pos + 1,
                     rs.overflow, capacity};
  }
  if (nchunks > 1 && chunk_start >= end) {
    // Nothing of this batch in the chunk: an empty partial (max -inf, sum 0),
    // which the merge weighs by zero.  A sequence with no token at all thus
    // merges to 0/0 = NaN, like the reference's softmax over an all -inf row.
    store_new_row();
    if (tid < groups) {
      const int64_t p = (b * q_heads + kvh * groups + tid) * nchunks + chunk;
      publish(part_ml + 2 * p, -INFINITY);
      publish(part_ml + 2 * p + 1, 0.0f);
    }
    if (counters != nullptr)
      merge_if_last<T, D>(part_o, part_ml, output, counters, smem, b, kvh, q_heads, kv_heads,
                          groups, o_sb, o_sh, nchunks, adv);
    return;
  }
  const int chunk_end = min(chunk_start + chunk_tokens, end);


  using KV = std::integral_constant<int, 3>;
  using KOnly = std::integral_constant<int, 1>;
  using VOnly = std::integral_constant<int, 2>;
  // kTilesInFlight tiles per wave: tile i is consumed, then refilled
  // kTilesInFlight sweeps ahead.  sched_barrier keeps each prologue tile's
  // loads ahead of the next one's: the loop consumes them in that order, and
  // a later tile issued first would make the first step wait for every load
  // (vmcnt(0)) -- a wait that, sitting in the loop header, would then drain
  // the prefetch on every iteration.  The prologue runs first in each path
  // below (no code precedes it there).
  Tile tiles[kTilesInFlight];
  auto prologue = [&](auto which) {
#pragma unroll
    for (int i = 0; i < kTilesInFlight; ++i) {
      load_tile(t_first + i * kStride, tiles[i], chunk_end, which);
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (ROPE) {
      rope_slices<T, KK>(qraw, cs, sn);
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) qv[kk] = as_vec<T>(qraw[kk]);
      store_new_row();
    }
  };
  // EXACT: when the chunk's tiles fit in the dynamic LDS with their V rows
  // (per 32-token tile: the 8 fp32 log2-domain scores of every lane, 2 KB,
  // and the lanes' V registers, 64 * D bytes), pass 1 loads K and V together
  // and keeps both, and pass 2 reads no memory.  Otherwise pass 1 keeps the
  // rounded scores (1 KB per tile) and pass 2 streams V.
  constexpr int kStashTileBytes = 2048 + 64 * D;
  const int ntiles = (chunk_end - chunk_start + kTile - 1) / kTile;
  const bool stash = EXACT && ntiles * kStashTileBytes <= exact_dyn_bytes<T, D>();

  // S^T tile: two 16-token MFMA blocks; lane holds tokens 16j+4g+r, head c.
  // q.k and its scaling are materialised in the tensor dtype, as the
  // reference's bf16 matmul and multiply do (r); softmax stays fp32, in log2
  // units (s = r * log2 e + mask * log2 e; -inf past the chunk end).
  auto tile_scores = [&](int t0, const Tile& tile, float (&s)[8], u16x8& r_bits) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      f32x4_t st = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) st = M::run(as_vec<T>(tile.k[j][kk]), qv[kk], st);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float rounded = slc::round_to<T>(slc::round_to<T>(st[r]) * scale);
        r_bits.v[4 * j + r] = bits_of<T>(rounded);
        float v = rounded * kLog2e;
        if constexpr (MK != 0) v += tile.mk[4 * j + r];
        s[4 * j + r] = t0 + 16 * j + 4 * g + r < chunk_end ? v : -INFINITY;
      }
    }
  };
  // Running max / sum (and the accumulator, when there is one) with a lazy
  // rescale.
  auto update_max = [&](const float (&s)[8]) {
    float mx = s[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) mx = fmaxf(mx, s[i]);
    mx = slc::max_xor32(slc::max_xor16(mx));
    if (__any(mx > m_run + kRescaleThreshold)) {
      const float m_new = fmaxf(m_run, mx);
      const float alpha = fast_exp2(m_run - (m_new == -INFINITY ? 0.0f : m_new));
      l_run *= alpha;
      if constexpr (!EXACT) {
#pragma unroll
        for (int db = 0; db < DB; ++db) acc[db] = acc[db] * alpha;
      }
      m_run = m_new;
    }
  };
  // O^T[dim, head] += V^T . P^T.  V^T is produced in registers: V rows times
  // a 0/1 selector (one MFMA per 16 tokens x 16 dims) land as lane
  // (dim c, tokens 4g..4g+3) -- exactly the token slots of the P operand.
  // The products are exact (x * 1 + 0), so converting back is lossless.
  auto accumulate_pv = [&](const Tile& tile, const typename M::vec& pv) {
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const f32x4_t zero = f32x4_t{0.f, 0.f, 0.f, 0.f};
      const f32x4_t x0 = M::run(as_vec<T>(tile.v[0][db >> 1]), sel[db & 1], zero);
      const f32x4_t x1 = M::run(as_vec<T>(tile.v[1][db >> 1]), sel[db & 1], zero);
      u16x8 a;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        a.v[r] = bits_of<T>(x0[r]);
        a.v[4 + r] = bits_of<T>(x1[r]);
      }
      acc[db] = M::run(__builtin_bit_cast(typename M::vec, a), pv, acc[db]);
    }
  };

  auto compute_tile = [&](int t0, const Tile& tile) {
    float s[8];
    u16x8 r_bits;
    tile_scores(t0, tile, s, r_bits);
    update_max(s);
    const float m_use = m_run == -INFINITY ? 0.0f : m_run;
    u16x8 pbits;
    float psum = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float p = fast_exp2(s[i] - m_use);
      psum += p;
      pbits.v[i] = bits_of<T>(p);
    }
    l_run += psum;
    accumulate_pv(tile, __builtin_bit_cast(typename M::vec, pbits));
  };
  // EXACT pass 1: scores to LDS, running max and sum (no accumulator).
  auto score_tile = [&](int t0, const Tile& tile) {
    float s[8];
    u16x8 r_bits;
    tile_scores(t0, tile, s, r_bits);
    score_lds[(t0 / kTile) * 64 + lane] = __builtin_bit_cast(uint4, r_bits);
    update_max(s);
    const float m_use = m_run == -INFINITY ? 0.0f : m_run;
    float psum = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) psum += fast_exp2(s[i] - m_use);
    l_run += psum;
  };
  // EXACT pass 2: p = exp2(s - m - log2 l) = exp(score - max) / sum, rounded.
  float norm_shift = 0.0f;
  auto weigh_tile = [&](int t0, const Tile& tile) {
    const u16x8 r_bits = __builtin_bit_cast(u16x8, score_lds[(t0 / kTile) * 64 + lane]);
    u16x8 pbits;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      T rb;
      rb.bits = r_bits.v[i];
      float v = slc::to_f32(rb) * kLog2e;
      if constexpr (MK != 0) v += tile.mk[i];
      const bool valid = t0 + 16 * (i >> 2) + 4 * g + (i & 3) < chunk_end;
      pbits.v[i] = valid ? bits_of<T>(fast_exp2(v - norm_shift)) : 0;
    }
    accumulate_pv(tile, __builtin_bit_cast(typename M::vec, pbits));
  };

  // Two tiles in flight per wave: while tile A is consumed, tile B (issued
  // earlier) and the refill of A stream in.  Prefetches past the chunk end are
  // zero-length buffer ranges and touch no memory.
  // ROPE: the new token's row of a tile comes from the registers.
  auto patch = [&](int t0, Tile& tile) {
    if constexpr (ROPE) {
      if (pos >= t0 && pos < t0 + kTile) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const bool mine = t0 + 16 * j + c == pos;
#pragma unroll
          for (int kk = 0; kk < KK; ++kk) {
            if (mine) {
              tile.k[j][kk] = knew[kk];
              tile.v[j][kk] = vnew[kk];
            }
          }
        }
      }
    }
  };
  constexpr int kAhead = kTilesInFlight * kStride;
  // The exit past the chunk end leaves the whole sweep (not just the inner
  // step): every path back to the loop header then carries the same loads.
  auto sweep = [&](auto body, auto which) {
    for (int t0 = t_first; t0 < chunk_end; t0 += kAhead) {
      if (t0 + kAhead < chunk_end) move_window(t0 + kAhead, t0 + kAhead + kAhead - kStride + kTile - 1);
#pragma unroll
      for (int i = 0; i < kTilesInFlight; ++i) {
        const int tt = t0 + i * kStride;
        if (i > 0 && tt >= chunk_end) goto done;
        patch(tt, tiles[i]);
        body(tt, tiles[i]);
        load_tile(tt + kAhead, tiles[i], chunk_end, which);
      }
    }
  done:;
  };

  float* sm_m = reinterpret_cast<float*>(smem);
  float* sm_l = sm_m + kWaves * kMaxGroups;
  float* sm_o = sm_l + kWaves * kMaxGroups;  // [wave][head][D]
  // EXACT: the row max and sum over the 4 lane groups and the waves, and
  // from them the shift of pass 2.
  auto exact_norm = [&]() {
    l_run += __shfl_xor(l_run, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);
    if (g == 0) {
      sm_m[wave * kMaxGroups + c] = m_run;
      sm_l[wave * kMaxGroups + c] = l_run;
    }
    __syncthreads();
    float mmax = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mmax = fmaxf(mmax, sm_m[w * kMaxGroups + c]);
    const float mu = mmax == -INFINITY ? 0.0f : mmax;
    float lsum = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w)
      lsum += fast_exp2(sm_m[w * kMaxGroups + c] - mu) * sm_l[w * kMaxGroups + c];
    // An empty row (no token, or all of them masked to -inf) has sum 0 and
    // gives NaN, as the reference's softmax over an all -inf row does.
    norm_shift = lsum > 0.0f ? mu + __builtin_amdgcn_logf(lsum) : __builtin_nanf("");
  };
  if constexpr (EXACT) {
    if (stash) {
      // Tile i of the chunk: scores at [2i, 2i + 1][lane], V at [2KK i ..][lane]
      // (16-byte words).
      uint4* s_lds = score_lds;
      uint4* v_lds = score_lds + ntiles * 128;
      auto stash_tile = [&](int t0, const Tile& tile) {
        float s[8];
        u16x8 r_bits;
        tile_scores(t0, tile, s, r_bits);
        const int ti = (t0 - chunk_start) / kTile;
        s_lds[(2 * ti) * 64 + lane] = make_uint4(__float_as_uint(s[0]), __float_as_uint(s[1]),
                                                 __float_as_uint(s[2]), __float_as_uint(s[3]));
        s_lds[(2 * ti + 1) * 64 + lane] = make_uint4(__float_as_uint(s[4]), __float_as_uint(s[5]),
                                                     __float_as_uint(s[6]), __float_as_uint(s[7]));
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int kk = 0; kk < KK; ++kk) v_lds[((2 * ti + j) * KK + kk) * 64 + lane] = tile.v[j][kk];
        update_max(s);
        const float m_use = m_run == -INFINITY ? 0.0f : m_run;
        float psum = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) psum += fast_exp2(s[i] - m_use);
        l_run += psum;
      };
      prologue(KV{});
      sweep(stash_tile, KV{});
      exact_norm();
      // Pass 2 from LDS: each wave weighs its own tiles (the words it wrote).
      for (int t0 = t_first; t0 < chunk_end; t0 += kStride) {
        const int ti = (t0 - chunk_start) / kTile;
        Tile tile;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int kk = 0; kk < KK; ++kk) tile.v[j][kk] = v_lds[((2 * ti + j) * KK + kk) * 64 + lane];
        const uint4 s0 = s_lds[(2 * ti) * 64 + lane];
        const uint4 s1 = s_lds[(2 * ti + 1) * 64 + lane];
        const float s[8] = {__uint_as_float(s0.x), __uint_as_float(s0.y), __uint_as_float(s0.z),
                            __uint_as_float(s0.w), __uint_as_float(s1.x), __uint_as_float(s1.y),
                            __uint_as_float(s1.z), __uint_as_float(s1.w)};
        u16x8 pbits;
#pragma unroll
        for (int i = 0; i < 8; ++i) pbits.v[i] = bits_of<T>(fast_exp2(s[i] - norm_shift));
        accumulate_pv(tile, __builtin_bit_cast(typename M::vec, pbits));
      }
    } else {
      // Pass 1, the norm, then pass 2 streaming V.
      prologue(KOnly{});
      sweep(score_tile, KOnly{});
      move_window(t_first, t_first + kAhead - kStride + kTile - 1);
#pragma unroll
      for (int i = 0; i < kTilesInFlight; ++i) {  // pass 2's first tiles fly during the combine
        load_tile(t_first + i * kStride, tiles[i], chunk_end, VOnly{});
        __builtin_amdgcn_sched_barrier(0);
      }
      exact_norm();
      sweep(weigh_tile, VOnly{});
    }
    __syncthreads();  // the LDS combine area is reused below
  } else {
    prologue(KV{});
    sweep(compute_tile, KV{});
    // Finish the per-lane partial sums of l over the 4 lane groups.
    l_run += __shfl_xor(l_run, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);
    __syncthreads();  // V tiles are dead; reuse LDS for the cross-wave merge.
    if (g == 0) {
      sm_m[wave * kMaxGroups + c] = m_run;
      sm_l[wave * kMaxGroups + c] = l_run;
    }
  }
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      sm_o[(wave * kMaxGroups + c) * D + db * 16 + 4 * g + r] = acc[db][r];
  __syncthreads();

  for (int idx = tid; idx < groups * D; idx += kThreads) {
    const int head = idx / D;
    const int d = idx % D;
    const int qh = kvh * groups + head;
    if constexpr (EXACT) {
      // The waves' sums of normalised terms add up in wave order; a row with
      // no weight at all (sum 0) is NaN, as in the reference's softmax.
      float osum = 0.0f, lsum = 0.0f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        osum += sm_o[(w * kMaxGroups + head) * D + d];
        lsum += sm_l[w * kMaxGroups + head];
      }
      output[b * o_sb + qh * o_sh + d] = slc::from_f32<T>(lsum > 0.0f ? osum : __builtin_nanf(""));
      continue;
    }
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
    if (nchunks == 1) {
      output[b * o_sb + qh * o_sh + d] = slc::from_f32<T>(osum / lsum);
    } else {
      const int64_t p = (b * q_heads + qh) * nchunks + chunk;
      publish(part_o + p * D + d, osum);
      if (d == 0) {
        publish(part_ml + 2 * p, mmax);
        publish(part_ml + 2 * p + 1, lsum);
      }
    }
  }
  if constexpr (ROPE) {
    // One chunk: no merge to carry the advance.  Every wave read the length
    // before the combine's barriers, so the count may be bumped now.
    if (nchunks == 1 && tid == 0) finish_advance(adv, count_only(adv.counter));
  }
  if (nchunks > 1 && counters != nullptr) {
    __syncthreads();  // the merge reuses the LDS
    merge_if_last<T, D>(part_o, part_ml, output, counters, smem, b, kvh, q_heads, kv_heads,
                        groups, o_sb, o_sh, nchunks, adv);
  }
}

// Merge the split-sequence partials: one workgroup per (batch, kv-head).
// Two rounds of independent loads and no length read: every chunk wrote a
// partial (an empty chunk writes max -inf, sum 0).  Round 1 loads every
// (head, chunk) (max, sum) pair at once into LDS; one thread per head turns
// them into weights; round 2 loads each output's values of the chunks with a
// non-zero weight, kMergeUnroll at a time.
constexpr int kMergeUnroll = 8;
template <typename T, int D>
__global__ __launch_bounds__(256) void decode_attention_merge_kernel(
    const float* __restrict__ part_o, const float* __restrict__ part_ml,
    T* __restrict__ output, int q_heads, int kv_heads, int groups, int64_t o_sb,
    int64_t o_sh, int nchunks) {
  __shared__ float sm_w[kMaxGroups * kMaxChunks];
  __shared__ float sm_l[kMaxGroups * kMaxChunks];
  __shared__ float sm_inv[kMaxGroups];
  const int kvh = blockIdx.x % kv_heads;
  const int64_t b = blockIdx.x / kv_heads;
  const int tid = threadIdx.x;
  const int64_t head0 = b * q_heads + kvh * groups;
  for (int idx = tid; idx < groups * nchunks; idx += 256) {
    const int head = idx / nchunks;
    const int i = idx % nchunks;
    const int64_t p = (head0 + head) * nchunks + i;
    sm_w[head * kMaxChunks + i] = part_ml[2 * p];
    sm_l[head * kMaxChunks + i] = part_ml[2 * p + 1];
  }
  __syncthreads();
  if (tid < groups) {
    float* w = sm_w + tid * kMaxChunks;
    const float* l = sm_l + tid * kMaxChunks;
    float mmax = -INFINITY;
    for (int i = 0; i < nchunks; ++i) mmax = fmaxf(mmax, w[i]);
    const float mu = mmax == -INFINITY ? 0.0f : mmax;
    float lsum = 0.0f;
    for (int i = 0; i < nchunks; ++i) {
      const float f = fast_exp2(w[i] - mu);  // exp2(-inf) = 0 for empty chunks
      w[i] = f;
      lsum += f * l[i];
    }
    sm_inv[tid] = 1.0f / lsum;
  }
  __syncthreads();
  for (int idx = tid; idx < groups * D; idx += 256) {
    const int head = idx / D;
    const int d = idx % D;
    const float* po = part_o + (head0 + head) * nchunks * D + d;
    const float* w = sm_w + head * kMaxChunks;
    float acc = 0.0f;
    for (int i0 = 0; i0 < nchunks; i0 += kMergeUnroll) {
      float v[kMergeUnroll];
#pragma unroll
      for (int k = 0; k < kMergeUnroll; ++k) {
        const int i = i0 + k;
        v[k] = i < nchunks && w[i] != 0.0f ? po[i * D] : 0.0f;
      }
#pragma unroll
      for (int k = 0; k < kMergeUnroll; ++k)
        if (i0 + k < nchunks) acc += w[i0 + k] * v[k];
    }
    const int qh = kvh * groups + head;
    output[b * o_sb + qh * o_sh + d] = slc::from_f32<T>(acc * sm_inv[head]);
  }
}

// Any dtype / head_dim <= 256 / any group size: one workgroup per
// (batch, query head), each wave takes every 4th token and reduces q.k with
// shuffles.  Used for fp32 and for shapes the MFMA kernel does not cover.
// EXACT: the reference's softmax order (normalise, round, then P.V) in two
// passes over the keys: the first forms the row max and sum, the second
// recomputes each score and weighs V with its normalised, rounded probability.
template <typename T, int NI, bool EXACT>
__global__ __launch_bounds__(256) void decode_attention_generic_kernel(
    const T* __restrict__ query, const T* __restrict__ key_buffer,
    const T* __restrict__ value_buffer, const void* __restrict__ lengths,
    int lengths_dtype, const void* __restrict__ mask, int mask_dtype,
    T* __restrict__ output, int q_heads, int groups, int head_dim,
    int64_t capacity, int64_t mask_len, int64_t q_sb, int64_t q_sh,
    int64_t kv_sb, int64_t kv_ss, int64_t kv_sh, int64_t m_sb, int64_t m_ss,
    int64_t o_sb, int64_t o_sh, float scale) {
  __shared__ float sm_m[kGenericWaves];
  __shared__ float sm_l[kGenericWaves];
  __shared__ float sm_o[kGenericWaves][NI * 64];
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
  // Score of token t in log2 units.  16-bit dtypes materialise q.k and its
  // scaling like the reference's matmul and multiply; fp32 keeps them exact.
  auto score = [&](int64_t t) {
    float dot = 0.0f;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int d = lane + 64 * i;
      if (d < head_dim) dot += q[i] * slc::to_f32(kbase[t * kv_ss + d]);
    }
    dot = slc::wave_sum(dot);
    float sc = (sizeof(T) == 2 ? slc::round_to<T>(slc::round_to<T>(dot) * scale) : dot * scale) * kLog2e;
    if (mask != nullptr) sc += slc::load_as_f32(mask, b * m_sb + t * m_ss, mask_dtype) * kLog2e;
    return sc;
  };
  for (int64_t t = wave; t < end; t += kGenericWaves) {
    const float sc = score(t);
    const float m_new = fmaxf(m_run, sc);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = exp2f(m_run - m_use);
    const float p = exp2f(sc - m_use);
    l_run = l_run * alpha + p;
    if constexpr (!EXACT) {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int d = lane + 64 * i;
        const float v = d < head_dim ? slc::to_f32(vbase[t * kv_ss + d]) : 0.0f;
        acc[i] = acc[i] * alpha + p * v;
      }
    }
    m_run = m_new;
  }
  if (lane == 0) {
    sm_m[wave] = m_run;
    sm_l[wave] = l_run;
  }
  if constexpr (EXACT) {
    __syncthreads();
    float mmax = -INFINITY;
    for (int w = 0; w < kGenericWaves; ++w) mmax = fmaxf(mmax, sm_m[w]);
    const float mu = mmax == -INFINITY ? 0.0f : mmax;
    float lsum = 0.0f;
    for (int w = 0; w < kGenericWaves; ++w) lsum += exp2f(sm_m[w] - mu) * sm_l[w];
    const float shift = lsum > 0.0f ? mu + log2f(lsum) : __builtin_nanf("");
    for (int64_t t = wave; t < end; t += kGenericWaves) {
      const float p = slc::round_to<T>(exp2f(score(t) - shift));
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int d = lane + 64 * i;
        const float v = d < head_dim ? slc::to_f32(vbase[t * kv_ss + d]) : 0.0f;
        acc[i] += p * v;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < NI; ++i) sm_o[wave][lane + 64 * i] = acc[i];
  __syncthreads();
  for (int d = threadIdx.x; d < head_dim; d += 256) {
    float mmax = -INFINITY;
    for (int w = 0; w < kGenericWaves; ++w) mmax = fmaxf(mmax, sm_m[w]);
    const float mu = mmax == -INFINITY ? 0.0f : mmax;
    float lsum = 0.0f, osum = 0.0f;
    for (int w = 0; w < kGenericWaves; ++w) {
      const float f = exp2f(sm_m[w] - mu);
      lsum += f * sm_l[w];
      osum += EXACT ? sm_o[w][d] : f * sm_o[w][d];
    }
    const float out = EXACT ? (lsum > 0.0f ? osum : __builtin_nanf("")) : osum / lsum;
    output[b * o_sb + h * o_sh + d] = slc::from_f32<T>(out);
  }
}

bool mfma_eligible(int dtype, int64_t head_dim, int64_t groups) {
  return (dtype == SLC_BF16 || dtype == SLC_F16) &&
         (head_dim == 64 || head_dim == 128) && groups <= kMaxGroups;
}

#ifndef SLC_DECODE_MIN_CHUNK
#define SLC_DECODE_MIN_CHUNK 256
#endif

// Sequence chunk of the split-sequence grid: the smallest power-of-two
// multiple of the workgroup's 128-token sweep that keeps the grid at about one
// workgroup per CU (256 CUs on MI355X); longer chunks amortise the per-wave
// pipeline fill and keep the partials small.
int64_t choose_chunk(int64_t batch, int64_t kv_heads, int64_t mask_len,
                     int64_t split_tokens) {
  const int64_t sweep = kWaves * kTile;
  int64_t chunk;
  if (split_tokens > 0) {
    chunk = slc_host::ceil_div(split_tokens, sweep) * sweep;
  } else {
    const int64_t target_groups = 256;
    chunk = SLC_DECODE_MIN_CHUNK;
    // Stop at one chunk per sequence: with more (batch, kv-head) pairs than
    // the target the grid is already that wide.
    while (chunk < mask_len &&
           batch * kv_heads * slc_host::ceil_div(mask_len, chunk) > target_groups) {
      chunk *= 2;
    }
  }
  // The merge keeps every chunk's weight of a (batch, kv-head) in LDS.
  while (slc_host::ceil_div(mask_len, chunk) > kMaxChunks) chunk *= 2;
  return chunk;
}

// Caller-owned device memory of a call:
//   counters (zero before first use; every call leaves them zero again):
//     int merge[batch * kv_heads]       split-merge arrival counters
//     int advance[batch]                RoPE variant's length-advance counters
//   workspace (scratch, no initial contents needed):
//     float part_o[batch * q_heads * nchunks * D]
//     float part_ml[batch * q_heads * nchunks * 2]
// The counters are a separate array so that a call's partials can never land
// where a later call (of another shape) keeps its counters.
int64_t counter_count(int64_t batch, int64_t kv_heads) { return batch * kv_heads + batch; }
int64_t partial_bytes(int64_t batch, int64_t q_heads, int64_t head_dim, int64_t nchunks) {
  return nchunks > 1 ? batch * q_heads * nchunks * (head_dim + 2) * 4 : 0;
}

// Longest sequence (mask length) the EXACT MFMA kernel holds in LDS: 1 KB of
// rounded scores per 32 tokens next to the static combine area (the dynamic
// LDS of every EXACT launch is exact_dyn_bytes).
int64_t exact_max_tokens(int64_t head_dim) {
  return head_dim == 64 ? 4096 : head_dim == 128 ? 2048 : 0;
}

#ifndef SLC_DECODE_FUSED_MERGE
#define SLC_DECODE_FUSED_MERGE 1
#endif

// Status of a fused call the kernels cannot take (nothing was launched).
constexpr int kUnsupported = -2;

template <typename T, int D, int MK, bool L64, bool ROPE, bool EXACT, int PG = 0>
hipError_t exact_lds_limit(int bytes) {
  // Dynamic LDS above the 64 KB default needs the kernel's opt-in (once per
  // instantiation; the attribute is per function).
  static std::once_flag once;
  static hipError_t status = hipSuccess;
  std::call_once(once, [&] {
    status = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&decode_attention_mfma_kernel<T, D, MK, L64, ROPE, EXACT, PG>),
        hipFuncAttributeMaxDynamicSharedMemorySize,
        exact_dyn_bytes<T, D>());
  });
  (void)bytes;
  return status;
}

}  // namespace
