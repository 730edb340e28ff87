// prefill_v2.hpp: the grouped-head prefill attention kernel and the helpers
// it shares with the other prefill kernels.  Its launcher is instantiated for
// 32-query workgroups in prefill_attention.hip and for 16-query workgroups in
// prefill_attention_short.hip (two translation units built in parallel).
#pragma once
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


// ---- grouped-head kernel (v2) ------------------------------------------------
// A workgroup owns 16 * QB queries of ALL the query heads of one KV head
// (GQA group G): G compute waves (one query head each, QB MFMA column
// blocks of 16 queries) plus one producer wave that streams the K, V (and mask) tiles of 64
// keys into an LDS ring with direct-to-LDS loads.  K, V and the mask are thus
// read once per workgroup for all G heads (the single-head kernel reads them
// G times), and no VALU work or VGPR goes into staging.
//  * S^T[key, query] = K . Q^T: K rows straight from the XOR-swizzled tile
//    (ds_read_b128), Q^T in registers (QB query blocks reuse every K read).
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
// Longest key range (in 64-key tiles) the tile-class list covers: T <= 65536.
constexpr int kMaxClassTiles = 1024;
// Two ring stages: the producer refills one stage while the consumers read
// the other (measured 2-3 % faster than three stages, equal to four).
#ifndef SLC_PREFILL_STAGES
#define SLC_PREFILL_STAGES 2
#endif
constexpr int kV2Stages = SLC_PREFILL_STAGES;
constexpr int kV2TileBytes = kKeys * kRowBytes;                 // 8 KB of K or of V
// Mask tile: 16 * QB query rows x 64 keys of the mask element type (0: no mask).
template <int MK>
constexpr int mask_elem_bytes() { return MK == 0 ? 0 : (MK == SLC_F32 + 1 ? 4 : 2); }
template <int MK, int QB>
constexpr int stage_bytes() { return 2 * kV2TileBytes + 16 * QB * kKeys * mask_elem_bytes<MK>(); }

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
template <typename T, int G, int MK, bool CAUSAL, bool POW2, bool EXACT, int QB>
__global__ __launch_bounds__((G + 1) * 64, QB <= 2 ? 4 : 1) void prefill_attention_v2_kernel(
    const T* __restrict__ query, const T* __restrict__ key, const T* __restrict__ value,
    const void* __restrict__ mask, T* __restrict__ output, int tokens, int kv_heads,
    int64_t q_sb, int64_t q_sh, int64_t q_st, int64_t k_sb, int64_t k_sh, int64_t k_st,
    int64_t v_sb, int64_t v_sh, int64_t v_st, int64_t m_sb, int64_t m_sq, int64_t o_sb,
    int64_t o_sh, int64_t o_st, float scale, const unsigned char* __restrict__ tile_class) {
  using M = Mfma<T>;
  constexpr int kQB = QB;                // query blocks of 16 per consumer wave
  constexpr int kV2Queries = 16 * QB;    // queries per workgroup
  constexpr int ME = mask_elem_bytes<MK>();
  constexpr int kMaskRow = kKeys * ME;                 // bytes of one mask tile row
  constexpr int kMaskTile = kV2Queries * kMaskRow;
  __shared__ __attribute__((aligned(16))) unsigned char ring[kV2Stages][stage_bytes<MK, QB>()];
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

template <typename T, int G, int MK, bool CAUSAL, int QB>
int launch_v2(const void* q, const void* k, const void* v, const void* mask, void* out,
              int64_t batch, int tokens, int kv_heads, const int64_t* st, float scale,
              bool exact, const unsigned char* classes, hipStream_t stream) {
  const dim3 grid(kv_heads, static_cast<unsigned>(batch), (tokens + 16 * QB - 1) / (16 * QB));
  int exponent = 0;
  const bool pow2 = std::is_same_v<T, slc::bf16_t> && std::frexp(scale, &exponent) == 0.5f &&
                    exponent > -100;
  auto kernel = exact ? (pow2 ? prefill_attention_v2_kernel<T, G, MK, CAUSAL, true, true, QB>
                              : prefill_attention_v2_kernel<T, G, MK, CAUSAL, false, true, QB>)
                      : (pow2 ? prefill_attention_v2_kernel<T, G, MK, CAUSAL, true, false, QB>
                              : prefill_attention_v2_kernel<T, G, MK, CAUSAL, false, false, QB>);
  hipLaunchKernelGGL(kernel, grid, dim3((G + 1) * 64), 0,
                     stream, static_cast<const T*>(q), static_cast<const T*>(k),
                     static_cast<const T*>(v), mask, static_cast<T*>(out), tokens, kv_heads,
                     st[0], st[1], st[2], st[3], st[4], st[5], st[6], st[7], st[8], st[9], st[10],
                     st[12], st[13], st[14], scale, MK != 0 ? classes : nullptr);
  return slc_host::check_launch("slc_hip_prefill_attention(grouped)");
}

}  // namespace

namespace slc_prefill {
// The grouped kernel with 16-query workgroups (one MFMA column block of
// queries per consumer wave), defined in prefill_attention_short.hip.
template <typename T, int G, int MK, bool CAUSAL>
int launch_v2_short(const void* q, const void* k, const void* v, const void* mask, void* out,
                    int64_t batch, int tokens, int kv_heads, const int64_t* st, float scale,
                    bool exact, const unsigned char* classes, hipStream_t stream);
}  // namespace slc_prefill
