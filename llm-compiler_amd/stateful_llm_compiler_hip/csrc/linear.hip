// linear: Y[M, N] = X[M, K] . W[N, K]^T (+ bias[N]), fp32 accumulation.
//
// Semantics: src/stateful_llm_compiler/backends/triton_linear.py:10-84 (fp32
// accumulate, bias added in fp32, one rounding on store) and the reference
// executor's F.linear (execution.py:694-705).
//
// MI355X design (bf16 / fp16):
//  * X rows and W rows are both K-contiguous, which is exactly the operand
//    layout of v_mfma_f32_16x16x32 (A rows = M, B columns = N, 8 consecutive k
//    per lane), so neither operand needs a transpose.
//  * Global -> LDS with fully coalesced 16-byte loads (8 lanes per 128-byte
//    row segment of a 64-wide K tile), through buffer resources whose range
//    check zero-fills rows past M / N.  LDS rows are XOR-swizzled on 16-byte
//    chunks so the 16-row MFMA operand reads (ds_read_b128) are free of bank
//    conflicts.  Two LDS buffers: tile k+1 is fetched into registers while
//    tile k is multiplied.
//  * Decode-sized M (<= 64) takes a dedicated weight-streaming kernel (split-K
//    across the waves of a workgroup, see linear_skinny_kernel); prefill-sized
//    M uses 128 x 128 tiles (MFMA-bound).
// fp32 (and shapes the vector path cannot take) use a classic LDS-tiled
// FMA kernel.
#include <type_traits>

#include "common.hpp"
#include "op_math.hpp"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x2_t __attribute__((ext_vector_type(2)));

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
// Per-lane offset plus a wave-uniform (scalar) one.
__device__ __forceinline__ uint4 buffer_load16(__amdgpu_buffer_rsrc_t rsrc, int offset,
                                               int uniform) {
  return __builtin_bit_cast(uint4,
                            __builtin_amdgcn_raw_buffer_load_b128(rsrc, offset, uniform, 0));
}

constexpr int kBK = 64;            // K elements per tile (128 bytes of bf16)
constexpr int kChunks = kBK / 8;   // 16-byte chunks per tile row

// Byte offset of (row, 16-byte chunk) inside a swizzled LDS tile.
__device__ __forceinline__ int lds_offset(int row, int chunk) {
  return row * (kBK * 2) + ((chunk ^ (row & 7)) << 4);
}

// KFULL: K is a multiple of the 64-wide k-tile, so no load needs a k check
// (rows past M / N fall outside the buffer ranges and read zero), every
// per-lane offset is fixed for the whole loop and the k-tile offset is a
// scalar: the main loop carries no per-load VALU work (with the checks it ran
// about five VALU instructions per MFMA, as much issue time as the MFMAs).
// VST: N and the output row stride are multiples of 8 (16-byte aligned rows):
// each wave stages its output tile through LDS and writes it with 16-byte
// stores (8 per lane instead of 64 two-byte ones) through a buffer resource
// whose range ends at the workgroup's last valid output element.
// Up to three projections of one input in one launch (GROUP): N-tiles
// [tile_end[j-1], tile_end[j]) belong to matrix j.
struct LinearGroup {
  const void* w[3];
  const void* bias[3];
  void* y[3];
  int n[3];
  int64_t y_rs[3];
  int tile_end[3];
};

template <typename T, int BM, int BN, int WM, int WN, bool KFULL, bool VST>
__global__ __launch_bounds__(WM * WN * 64) void linear_mfma_kernel(
    const T* __restrict__ x, const T* __restrict__ w, const T* __restrict__ bias,
    T* __restrict__ y, int M, int N, int K, int64_t x_rs, int64_t y_rs,
    const T* __restrict__ residual, int64_t r_rs) {
  using MF = Mfma<T>;
  constexpr int NT = WM * WN * 64;  // threads per workgroup
  constexpr int TM = BM / WM;  // rows per wave
  constexpr int TN = BN / WN;  // cols per wave
  constexpr int FM = TM / 16;
  constexpr int FN = TN / 16;
  constexpr int XCH = BM * kChunks;  // 16-byte chunks per X tile
  constexpr int WCH = BN * kChunks;
  constexpr int XPT = (XCH + NT - 1) / NT;  // chunks per thread
  constexpr int WPT = (WCH + NT - 1) / NT;
  constexpr int XB = BM * kBK * 2;  // bytes per X tile
  constexpr int WB = BN * kBK * 2;

  // One LDS tile pair (the next k-tile waits in registers while this one is
  // read), or the epilogue's staging if larger: 40 KB at 128 x 128, so three
  // workgroups share a CU (two with a double-buffered 64 KB ring: the third
  // workgroup hides more load latency than the second barrier per k-tile
  // costs, 362 -> 333 us at M32768 N4864 K896).
  constexpr int kStage = XB + WB;
  constexpr int kEpi = WM * WN * TM * (TN + 8) * 2;
  constexpr int kSmem = kStage > kEpi ? kStage : kEpi;
  __shared__ __attribute__((aligned(16))) unsigned char smem[kSmem];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int c = lane & 15;
  const int g = lane >> 4;
  const int wm = wave / WN;
  const int wn = wave % WN;
  // Tile order for the L2s: workgroup ids go round-robin to the 8 XCDs, each
  // with its own L2, so consecutive ids are first gathered per XCD (id i of
  // the first 8 * floor(tiles / 8) goes to slot (i % 8) * floor(tiles / 8) +
  // i / 8, the rest keep theirs: a bijection), then slots run in groups of
  // kGroupM M-tiles, N-tile-major inside a group, so the workgroups one XCD
  // holds at a time share their X and W tiles in its L2.
  int m_blk, n_blk;
  {
    constexpr int kXcds = 8, kGroupM = 8;
    const int n_tiles = gridDim.x, m_tiles = gridDim.y;
    const int total = n_tiles * m_tiles;
    const int id = blockIdx.y * n_tiles + blockIdx.x;
    const int per = total / kXcds;
    const int t = id < per * kXcds ? (id % kXcds) * per + id / kXcds : id;
    const int span = kGroupM * n_tiles;
    const int first_m = (t / span) * kGroupM;
    const int gm = m_tiles - first_m < kGroupM ? m_tiles - first_m : kGroupM;
    m_blk = first_m + (t % span) % gm;
    n_blk = (t % span) / gm;
  }
  const int n0 = n_blk * BN;
  const int m0 = m_blk * BM;

  // Buffer resources over the workgroup's rows: rows past M / N read zero.
  const int64_t x_rows = M - m0 < BM ? M - m0 : BM;
  const int64_t w_rows = N - n0 < BN ? N - n0 : BN;
  const __amdgpu_buffer_rsrc_t rx =
      make_rsrc(x + m0 * x_rs, x_rows > 0 ? (x_rows - 1) * x_rs * 2 + K * 2 : 0);
  const __amdgpu_buffer_rsrc_t rw =
      make_rsrc(w + static_cast<int64_t>(n0) * K, w_rows > 0 ? w_rows * K * 2 : 0);

  uint4 xr[XPT], wr[WPT];
  static_assert(!KFULL || (XCH % NT == 0 && WCH % NT == 0), "whole chunks per thread");
  int xoff[XPT], woff[WPT];
#pragma unroll
  for (int i = 0; i < XPT; ++i) {
    const int ch = tid + NT * i;
    xoff[i] = static_cast<int>((ch / kChunks) * x_rs + (ch % kChunks) * 8) * 2;
  }
#pragma unroll
  for (int i = 0; i < WPT; ++i) {
    const int ch = tid + NT * i;
    woff[i] = ((ch / kChunks) * K + (ch % kChunks) * 8) * 2;
  }
  auto fetch = [&](int k0) {
    if constexpr (KFULL) {
      const int kb = __builtin_amdgcn_readfirstlane(k0 * 2);
#pragma unroll
      for (int i = 0; i < XPT; ++i) xr[i] = buffer_load16(rx, xoff[i], kb);
#pragma unroll
      for (int i = 0; i < WPT; ++i)
        wr[i] = buffer_load16(rw, woff[i], kb);
      return;
    }
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      const int ch = tid + NT * i;
      const int row = ch / kChunks, col = (ch % kChunks) * 8;
      const bool ok = ch < XCH && row < x_rows && k0 + col < K;
      xr[i] = ok ? buffer_load16(rx, static_cast<int>(row * x_rs + k0 + col) * 2)
                 : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < WPT; ++i) {
      const int ch = tid + NT * i;
      const int row = ch / kChunks, col = (ch % kChunks) * 8;
      const bool ok = ch < WCH && row < w_rows && k0 + col < K;
      wr[i] = ok ? buffer_load16(rw, (row * K + k0 + col) * 2) : make_uint4(0, 0, 0, 0);
    }
  };
  auto stash = [&]() {
    unsigned char* xs = smem;
    unsigned char* ws = xs + XB;
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      const int ch = tid + NT * i;
      if (ch < XCH)
        *reinterpret_cast<uint4*>(xs + lds_offset(ch / kChunks, ch % kChunks)) = xr[i];
    }
#pragma unroll
    for (int i = 0; i < WPT; ++i) {
      const int ch = tid + NT * i;
      if (ch < WCH)
        *reinterpret_cast<uint4*>(ws + lds_offset(ch / kChunks, ch % kChunks)) = wr[i];
    }
  };

  f32x4_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int ktiles = (K + kBK - 1) / kBK;
  fetch(0);
  stash();
  __syncthreads();
  for (int kt = 0; kt < ktiles; ++kt) {
    if (kt + 1 < ktiles) fetch((kt + 1) * kBK);
    const unsigned char* xs = smem;
    const unsigned char* ws = xs + XB;
#pragma unroll
    for (int kk = 0; kk < kBK / 32; ++kk) {
      typename MF::vec a[FM], b[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int row = wm * TM + i * 16 + c;
        a[i] = *reinterpret_cast<const typename MF::vec*>(xs + lds_offset(row, kk * 4 + g));
      }
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int row = wn * TN + j * 16 + c;
        b[j] = *reinterpret_cast<const typename MF::vec*>(ws + lds_offset(row, kk * 4 + g));
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = MF::run(a[i], b[j], acc[i][j]);
    }
    __syncthreads();  // every wave's reads of the tile are done
    if (kt + 1 < ktiles) stash();
    __syncthreads();
  }

  if constexpr (VST) {
    // The loop ended on a barrier, so the LDS is free: wave-private staging
    // of its TM x TN tile as T, rows padded to keep 16-byte alignment.
    constexpr int kCPad = TN + 8;
    static_assert(TM * kCPad * 2 * WM * WN <= kSmem, "staging fits the LDS");
    uint16_t* cs = reinterpret_cast<uint16_t*>(smem) + wave * TM * kCPad;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int n = n0 + wn * TN + j * 16 + c;
      const float bv = bias != nullptr && n < N ? slc::to_f32(bias[n]) : 0.0f;
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          cs[(i * 16 + 4 * g + r) * kCPad + j * 16 + c] =
              slc::from_f32<T>(acc[i][j][r] + bv).bits;
    }
    const int rows = M - m0 < BM ? M - m0 : BM;
    const __amdgpu_buffer_rsrc_t ry =
        make_rsrc(y + m0 * y_rs, (static_cast<int64_t>(rows) - 1) * y_rs * 2 + N * 2);
    // With a residual (VST only): y = residual + round(x.w^T + bias), rounded
    // again, as the separate add does.
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(
        residual != nullptr ? residual + m0 * r_rs : y,
        residual != nullptr ? (static_cast<int64_t>(rows) - 1) * r_rs * 2 + N * 2 : 0);
    constexpr int kPerRow = TN / 8;  // 16-byte chunks per staged row
#pragma unroll
    for (int q = 0; q < TM * kPerRow / 64; ++q) {
      const int id = q * 64 + lane;
      const int row = id / kPerRow, chunk = id % kPerRow;
      const int m_local = wm * TM + row;
      const int n = n0 + wn * TN + chunk * 8;
      uint4 v = *reinterpret_cast<const uint4*>(cs + row * kCPad + chunk * 8);
      if (residual != nullptr) {
        const uint4 rv = buffer_load16(rr, static_cast<int>(m_local * r_rs + n) * 2);
        const uint16_t* lin = reinterpret_cast<const uint16_t*>(&v);
        const uint16_t* res = reinterpret_cast<const uint16_t*>(&rv);
        uint4 o;
        uint16_t* out = reinterpret_cast<uint16_t*>(&o);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          T a, r;
          a.bits = lin[e];
          r.bits = res[e];
          out[e] = slc::from_f32<T>(slc::to_f32(r) + slc::to_f32(a)).bits;
        }
        v = o;
      }
      if (m_local < rows && n < N)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4_t, v), ry,
                                               static_cast<int>(m_local * y_rs + n) * 2, 0, 0);
    }
    return;
  }
  // Epilogue: lane (col c, rows 4g..4g+3) of each 16 x 16 fragment.
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int n = n0 + wn * TN + j * 16 + c;
    if (n >= N) continue;
    const float bv = bias != nullptr ? slc::to_f32(bias[n]) : 0.0f;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * TM + i * 16 + 4 * g + r;
        if (m < M) y[m * y_rs + n] = slc::from_f32<T>(acc[i][j][r] + bv);
      }
  }
}


// ---------------------------------------------------------------------------
// Prefill GEMM with a deep direct-to-LDS ring (KFULL and 16-byte-store shapes).
//
// The register-staged kernel above keeps one k-tile in flight per workgroup:
// each k-tile waits a full memory round trip (~0.7 us under load), so a
// K = 896 GEMM of any size takes >= 14 round trips and the large shapes sit
// near 30 % of MFMA peak.  Here PW producer waves stream X and W k-tiles
// straight into an S-stage LDS ring with buffer_load ... lds (no registers,
// so S - 1 tiles fly at once), and CWM x CWN consumer waves only read LDS
// and issue MFMAs.  One workgroup barrier per k-tile: before it the
// producers wait until their loads of tile kt have landed (vmcnt), after it
// they refill the stage every consumer has just finished reading.  The
// producers' barrier is a bare s_barrier: __syncthreads() would also wait
// for all their in-flight loads and drain the ring.
//
// LDS rows are 128 bytes (64 bf16 of K) with 16-byte chunks XOR-swizzled by
// row, as above: lane L of DMA instruction n fills LDS row 8n + L/8 at chunk
// position L%8 with global chunk (L%8) ^ (row & 7).  Consumer fragment reads
// and the k order of every MFMA chain are those of linear_mfma_kernel, so
// the two kernels give bit-identical outputs.  Past the last k-tile the
// producers keep issuing loads through an empty buffer range (no traffic,
// zeros into a stage nobody reads) so every wait counts the same number of
// loads; they drain them before the epilogue reuses the ring.
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t rsrc, unsigned char* lds,
                                          int voffset, int soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      rsrc, (__attribute__((address_space(3))) void*)lds, 16, voffset, soffset, 0, 0);
}

// Workgroup id -> (m_blk, n_blk): gathered per XCD, then groups of 8 M-tiles
// (see linear_mfma_kernel).
#ifndef SLC_RING_PF
#define SLC_RING_PF 1
#endif

template <int kGroupM>
__device__ __forceinline__ void xcd_tile(int n_tiles, int m_tiles, int& m_blk, int& n_blk) {
  constexpr int kXcds = 8;
  const int total = n_tiles * m_tiles;
  const int id = blockIdx.y * n_tiles + blockIdx.x;
  const int per = total / kXcds;
  const int t = id < per * kXcds ? (id % kXcds) * per + id / kXcds : id;
  const int span = kGroupM * n_tiles;
  const int first_m = (t / span) * kGroupM;
  const int gm = m_tiles - first_m < kGroupM ? m_tiles - first_m : kGroupM;
  m_blk = first_m + (t % span) % gm;
  n_blk = (t % span) / gm;
}

template <typename T, int BM, int BN, int CWM, int CWN, int PW, int S, int GM = 8,
          bool DUAL = false, bool GROUP = false>
__global__ __launch_bounds__((CWM * CWN + PW) * 64) void linear_ring_kernel(
    const T* __restrict__ x, const T* __restrict__ w_arg, const T* __restrict__ bias_arg,
    T* __restrict__ y_arg, int M, int N_arg, int K, int64_t x_rs, int64_t y_rs_arg,
    const T* __restrict__ residual, int64_t r_rs, const T* __restrict__ w2 = nullptr,
    LinearGroup grp = {}) {
  using MF = Mfma<T>;
  constexpr int CW = CWM * CWN;      // consumer waves
  constexpr int CT = CW * 64;        // consumer threads
  constexpr int TM = BM / CWM;
  constexpr int TN = BN / CWN;
  constexpr int FM = TM / 16;
  constexpr int FN = TN / 16;
  constexpr int XB = BM * kBK * 2;   // bytes of an X tile
  constexpr int kStage = (BM + BN) * kBK * 2;
  constexpr int kOps = (BM + BN) / 8 / PW;  // 1 KB DMA instructions per producer wave per tile
  static_assert(((BM + BN) / 8) % PW == 0, "DMA instructions split evenly over the producers");
  // PF: at the barrier of tile kt the producers have landed tile kt + 1 as
  // well, so the consumers read the next tile's first k-step fragments while
  // this tile's MFMAs run, and no LDS latency follows a barrier.  The loads
  // then keep S - 3 tiles in flight at a barrier instead of S - 2, so only
  // rings of four or more stages take it: M4096 N896 K896 12.5 -> 10.8 us,
  // Q/K/V group 30-32 -> 28.5 us; with three stages (256 x 128) the loads
  // lose their lead (vocabulary head 1297 -> 1513 us).
  constexpr bool kPF = SLC_RING_PF != 0 && S >= 4;
  constexpr int kLeadTiles = kPF ? S - 3 : S - 2;
  static_assert(!kPF || kBK == 64, "two k-steps per tile");
  static_assert(kLeadTiles * kOps <= 63, "the wait count fits vmcnt");
  static_assert(TM % 16 == 0 && TN % 16 == 0, "whole MFMA fragments per wave");
  constexpr int kEpiWave = TM * (TN + 8) * 2;
  constexpr int kEpiDual = BM * (BN + 8) * 2;
  static_assert(CW * kEpiWave <= S * kStage && (!DUAL || kEpiDual <= S * kStage),
                "epilogue staging fits in the ring");
  __shared__ __attribute__((aligned(16))) unsigned char ring[S * kStage];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  int m_blk, n_blk;
  xcd_tile<GM>(gridDim.x, gridDim.y, m_blk, n_blk);
  const T* w = w_arg;
  const T* bias = bias_arg;
  T* y = y_arg;
  int N = N_arg;
  int64_t y_rs = y_rs_arg;
  if constexpr (GROUP) {
    const int j = n_blk < grp.tile_end[0] ? 0 : (n_blk < grp.tile_end[1] ? 1 : 2);
    n_blk -= j == 0 ? 0 : grp.tile_end[j - 1];
    w = static_cast<const T*>(grp.w[j]);
    bias = static_cast<const T*>(grp.bias[j]);
    y = static_cast<T*>(grp.y[j]);
    N = grp.n[j];
    y_rs = grp.y_rs[j];
  }
  const int n0 = n_blk * (DUAL ? BN / 2 : BN);
  const int m0 = m_blk * BM;
  const int ktiles = K / kBK;

  if (wave >= CW) {
    // ---- producers ------------------------------------------------------
    const int pw = wave - CW;
    const int64_t x_rows = M - m0 < BM ? M - m0 : BM;
    const int64_t w_rows = DUAL ? (N - n0 < BN / 2 ? N - n0 : BN / 2) : (N - n0 < BN ? N - n0 : BN);
    const __amdgpu_buffer_rsrc_t rx =
        make_rsrc(x + m0 * x_rs, x_rows > 0 ? (x_rows - 1) * x_rs * 2 + K * 2 : 0);
    const __amdgpu_buffer_rsrc_t rw =
        make_rsrc(w + static_cast<int64_t>(n0) * K, w_rows > 0 ? w_rows * K * 2 : 0);
    const __amdgpu_buffer_rsrc_t rw2 = make_rsrc(DUAL ? w2 + static_cast<int64_t>(n0) * K : w,
                                                 DUAL && w_rows > 0 ? w_rows * K * 2 : 0);
    const __amdgpu_buffer_rsrc_t rnone = make_rsrc(x, 0);
    // The X tile's BM / 8 DMA instructions, then the W tile's BN / 8 (gate
    // rows then up rows under DUAL), are dealt round-robin to the producers:
    // instruction i of a wave has a compile-time operand (X, W or up) and
    // covers the ring rows 8 * (pw + PW * i') .. + 7 of that operand.
    constexpr int XO = BM / 8 / PW;
    constexpr int WO = (DUAL ? BN / 2 : BN) / 8 / PW;
    static_assert(XO * PW * 8 == BM && WO * PW * 8 == (DUAL ? BN / 2 : BN) &&
                      XO + WO * (DUAL ? 2 : 1) == kOps,
                  "operands split evenly over the producers");
    int voff[kOps];
#pragma unroll
    for (int i = 0; i < kOps; ++i) {
      const int local = i < XO ? i : (i - XO) % WO;  // instruction index inside its operand
      const int row = 8 * (pw + PW * local) + lane / 8;
      const int chunk = (lane % 8) ^ (row & 7);
      voff[i] = i < XO ? static_cast<int>(row * x_rs * 2) + chunk * 16 : row * K * 2 + chunk * 16;
    }
    auto issue = [&](int kt) {
      unsigned char* dst = ring + (kt % S) * kStage;
      const bool live = kt < ktiles;
      const int kb = __builtin_amdgcn_readfirstlane(live ? kt * kBK * 2 : 0);
      const __amdgpu_buffer_rsrc_t lx = live ? rx : rnone;
      const __amdgpu_buffer_rsrc_t lw = live ? rw : rnone;
      const __amdgpu_buffer_rsrc_t lw2 = live ? rw2 : rnone;
#pragma unroll
      for (int i = 0; i < kOps; ++i) {
        if (i < XO) {
          lds_dma16(lx, dst + (pw + PW * i) * 1024, voff[i], kb);
        } else if (i < XO + WO) {
          lds_dma16(lw, dst + XB + (pw + PW * (i - XO)) * 1024, voff[i], kb);
        } else {
          lds_dma16(lw2, dst + XB + (BN / 2) * 128 + (pw + PW * (i - XO - WO)) * 1024, voff[i], kb);
        }
      }
    };
#pragma unroll
    for (int t = 0; t < S - 1; ++t) issue(t);
    for (int kt = 0; kt < ktiles; ++kt) {
      asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"i"(kLeadTiles * kOps) : "memory");
      issue(kt + S - 1);
    }
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    return;
  }

  // ---- consumers ----------------------------------------------------------
  const int c = lane & 15;
  const int g = lane >> 4;
  const int wm = wave / CWN;
  const int wn = wave % CWN;
  f32x4_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  auto fragments = [&](const unsigned char* xs, int kk, typename MF::vec* a, typename MF::vec* b) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
      a[i] = *reinterpret_cast<const typename MF::vec*>(xs + lds_offset(wm * TM + i * 16 + c, kk * 4 + g));
#pragma unroll
    for (int j = 0; j < FN; ++j)
      b[j] = *reinterpret_cast<const typename MF::vec*>(xs + XB + lds_offset(wn * TN + j * 16 + c, kk * 4 + g));
  };
  typename MF::vec na[FM], nb[FN];  // PF: first k-step fragments of the next tile
  for (int kt = 0; kt < ktiles; ++kt) {
    __syncthreads();  // tile kt is in its stage; the stage of kt - 1 may be refilled
    const unsigned char* xs = ring + (kt % S) * kStage;
    const unsigned char* ws = xs + XB;
    if constexpr (kPF) {
      if (kt == 0) fragments(xs, 0, na, nb);
      typename MF::vec a[FM], b[FN];
      fragments(xs, 1, a, b);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = MF::run(na[i], nb[j], acc[i][j]);
      if (kt + 1 < ktiles) fragments(ring + ((kt + 1) % S) * kStage, 0, na, nb);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = MF::run(a[i], b[j], acc[i][j]);
      continue;
    }
#pragma unroll
    for (int kk = 0; kk < kBK / 32; ++kk) {
      typename MF::vec a[FM], b[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        a[i] = *reinterpret_cast<const typename MF::vec*>(xs + lds_offset(wm * TM + i * 16 + c, kk * 4 + g));
#pragma unroll
      for (int j = 0; j < FN; ++j)
        b[j] = *reinterpret_cast<const typename MF::vec*>(ws + lds_offset(wn * TN + j * 16 + c, kk * 4 + g));
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = MF::run(a[i], b[j], acc[i][j]);
    }
  }
  __syncthreads();  // the producers drained their loads; the ring is free

  if constexpr (DUAL) {
    constexpr int kRow = BN + 8;
    uint16_t* cs = reinterpret_cast<uint16_t*>(ring);
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          cs[(wm * TM + i * 16 + 4 * g + r) * kRow + wn * TN + j * 16 + c] =
              slc::from_f32<T>(acc[i][j][r]).bits;
    __syncthreads();  // consumers only (the producers have ended)
    const int rows = M - m0 < BM ? M - m0 : BM;
    const __amdgpu_buffer_rsrc_t ry =
        make_rsrc(y + m0 * y_rs, (static_cast<int64_t>(rows) - 1) * y_rs * 2 + N * 2);
    constexpr int kPerRow = BN / 2 / 8;
    static_assert((BM * kPerRow) % CT == 0, "whole store rounds");
#pragma unroll
    for (int q = 0; q < BM * kPerRow / CT; ++q) {
      const int id = q * CT + tid;
      const int row = id / kPerRow, chunk = id % kPerRow;
      const uint4 gv = *reinterpret_cast<const uint4*>(cs + row * kRow + chunk * 8);
      const uint4 uv = *reinterpret_cast<const uint4*>(cs + row * kRow + BN / 2 + chunk * 8);
      const uint16_t* gb = reinterpret_cast<const uint16_t*>(&gv);
      const uint16_t* ub = reinterpret_cast<const uint16_t*>(&uv);
      uint4 o;
      uint16_t* ob = reinterpret_cast<uint16_t*>(&o);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        T ge, ue;
        ge.bits = gb[e];
        ue.bits = ub[e];
        ob[e] = slc::from_f32<T>(slc::swiglu_value<T>(slc::to_f32(ge), slc::to_f32(ue))).bits;
      }
      const int n = n0 + chunk * 8;
      if (row < rows && n < N)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4_t, o), ry,
                                               static_cast<int>(row * y_rs + n) * 2, 0, 0);
    }
    return;
  } else {
    constexpr int kCPad = TN + 8;
    uint16_t* cs = reinterpret_cast<uint16_t*>(ring) + wave * TM * kCPad;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int n = n0 + wn * TN + j * 16 + c;
      const float bv = bias != nullptr && n < N ? slc::to_f32(bias[n]) : 0.0f;
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          cs[(i * 16 + 4 * g + r) * kCPad + j * 16 + c] = slc::from_f32<T>(acc[i][j][r] + bv).bits;
    }
    const int rows = M - m0 < BM ? M - m0 : BM;
    const __amdgpu_buffer_rsrc_t ry =
        make_rsrc(y + m0 * y_rs, (static_cast<int64_t>(rows) - 1) * y_rs * 2 + N * 2);
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(
        residual != nullptr ? residual + m0 * r_rs : y,
        residual != nullptr ? (static_cast<int64_t>(rows) - 1) * r_rs * 2 + N * 2 : 0);
    constexpr int kPerRow = TN / 8;
    static_assert((TM * kPerRow) % 64 == 0, "whole store rounds per wave");
#pragma unroll
    for (int q = 0; q < TM * kPerRow / 64; ++q) {
      const int id = q * 64 + lane;
      const int row = id / kPerRow, chunk = id % kPerRow;
      const int m_local = wm * TM + row;
      const int n = n0 + wn * TN + chunk * 8;
      uint4 v = *reinterpret_cast<const uint4*>(cs + row * kCPad + chunk * 8);
      if (residual != nullptr) {
        const uint4 rv = buffer_load16(rr, static_cast<int>(m_local * r_rs + n) * 2);
        const uint16_t* lin = reinterpret_cast<const uint16_t*>(&v);
        const uint16_t* res = reinterpret_cast<const uint16_t*>(&rv);
        uint4 o;
        uint16_t* out = reinterpret_cast<uint16_t*>(&o);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          T a, r;
          a.bits = lin[e];
          r.bits = res[e];
          out[e] = slc::from_f32<T>(slc::to_f32(r) + slc::to_f32(a)).bits;
        }
        v = o;
      }
      if (m_local < rows && n < N)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4_t, v), ry,
                                               static_cast<int>(m_local * y_rs + n) * 2, 0, 0);
    }
  }
}


// Tile id -> (m_blk, n_blk) with the mapping of xcd_tile, for a tile id that
// is not the workgroup id (persistent workgroups).  Tile ids of one residue
// mod 8 run on one XCD when the grid is a multiple of 8 workgroups.
template <int kGroupM>
__device__ __forceinline__ void xcd_tile_of(int id, int n_tiles, int m_tiles, int& m_blk,
                                            int& n_blk) {
  constexpr int kXcds = 8;
  const int per = n_tiles * m_tiles / kXcds;
  const int t = id < per * kXcds ? (id % kXcds) * per + id / kXcds : id;
  const int span = kGroupM * n_tiles;
  const int first_m = (t / span) * kGroupM;
  const int gm = m_tiles - first_m < kGroupM ? m_tiles - first_m : kGroupM;
  m_blk = first_m + (t % span) % gm;
  n_blk = (t % span) / gm;
}

// Persistent form of the 256 x 128 ring tile, for grids several rounds deep.
// One workgroup per CU walks the output tiles id, id + grid, ...; its
// producer waves stream k-tiles into the 3-stage ring without a break at tile
// boundaries, so the first k-tiles of the next output tile land while the
// consumers finish the current one and write it out.  The consumers multiply
// with the operands swapped (W rows as the MFMA A operand, X rows as B): an
// accumulator lane then holds four consecutive output features of one row,
// which it stores with one 8-byte store straight from registers -- the ring
// is never needed for staging the output.  Each output accumulates its k
// range in the ring kernel's order (same fragments, same 32-k MFMA steps; a
// product of two bf16 values does not depend on which operand slot holds
// which), so both kernels give the same bits.
// DUAL: each 128-row W stage holds 64 gate rows then 64 up rows; consumer
// wave wn takes gate and up rows of the same 32 features (fragments 0-1 gate,
// 2-3 up), so the SwiGLU pairs meet in one lane.
template <typename T, bool DUAL>
__global__ __launch_bounds__(12 * 64) void linear_stream_kernel(
    const T* __restrict__ x, const T* __restrict__ w_arg, const T* __restrict__ bias_arg,
    T* __restrict__ y_arg, int M, int N_arg, int K, int64_t x_rs, int64_t y_rs_arg, int n_tiles,
    int m_tiles, const T* __restrict__ w2) {
  using MF = Mfma<T>;
  constexpr int BM = 256, BN = 128, CWN = 2, PW = 4, S = 3, GM = 4;
  constexpr int CW = 8;                      // consumer waves, 4 x 2
  constexpr int TM = 64, TN = 64;            // consumer wave tile
  constexpr int FM = TM / 16, FN = TN / 16;  // fragments
  constexpr int XB = BM * kBK * 2;
  constexpr int kStage = (BM + BN) * kBK * 2;
  constexpr int kOps = (BM + BN) / 8 / PW;
  constexpr int XO = BM / 8 / PW;
  constexpr int WO = (DUAL ? BN / 2 : BN) / 8 / PW;
  static_assert(XO + WO * (DUAL ? 2 : 1) == kOps, "operands split evenly over the producers");
  static_assert((S - 2) * kOps <= 63, "the wait count fits vmcnt");
  __shared__ __attribute__((aligned(16))) unsigned char ring[S * kStage];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int total = n_tiles * m_tiles;
  const int ktiles = K / kBK;
  const int first = blockIdx.x;
  const int step = gridDim.x;

  struct Tile {
    int m0, n0, N;
    const T* w;
    const T* bias;
    T* y;
    int64_t y_rs;
  };
  auto tile_of = [&](int id) {
    int m_blk, n_blk;
    xcd_tile_of<GM>(id, n_tiles, m_tiles, m_blk, n_blk);
    Tile t{0, 0, N_arg, w_arg, bias_arg, y_arg, y_rs_arg};
    t.n0 = n_blk * (DUAL ? BN / 2 : BN);
    t.m0 = m_blk * BM;
    return t;
  };

  if (wave >= CW) {
    // ---- producers: one k-tile per barrier, S - 1 ahead, across tiles -------
    const int pw = wave - CW;
    int voff[kOps];
#pragma unroll
    for (int i = 0; i < kOps; ++i) {
      const int local = i < XO ? i : (i - XO) % WO;
      const int row = 8 * (pw + PW * local) + lane / 8;
      const int chunk = (lane % 8) ^ (row & 7);
      voff[i] = i < XO ? static_cast<int>(row * x_rs * 2) + chunk * 16 : row * K * 2 + chunk * 16;
    }
    // The operand ranges of the tile being loaded, as base + bytes: the
    // resources are rebuilt from them (through readfirstlane) at every issue,
    // so the compiler keeps them scalar; a resource variable reassigned at
    // tile boundaries is taken for divergent, and every load then runs in a
    // waterfall loop.
    const T* xb = x;
    const T* wb = x;
    const T* w2b = x;
    int64_t x_bytes = 0, w_bytes = 0;
    int load_id = first, load_k = 0;
    auto set_tile = [&](int id) {
      x_bytes = w_bytes = 0;
      if (id >= total) return;
      const Tile t = tile_of(id);
      const int64_t x_rows = M - t.m0 < BM ? M - t.m0 : BM;
      const int64_t w_rows =
          DUAL ? (t.N - t.n0 < BN / 2 ? t.N - t.n0 : BN / 2) : (t.N - t.n0 < BN ? t.N - t.n0 : BN);
      xb = x + t.m0 * x_rs;
      x_bytes = x_rows > 0 ? (x_rows - 1) * x_rs * 2 + K * 2 : 0;
      wb = t.w + static_cast<int64_t>(t.n0) * K;
      w2b = DUAL ? w2 + static_cast<int64_t>(t.n0) * K : t.w;
      w_bytes = w_rows > 0 ? w_rows * K * 2 : 0;
    };
    set_tile(load_id);
    int slot = 0;
    auto issue = [&]() {
      unsigned char* dst = ring + __builtin_amdgcn_readfirstlane(slot) * kStage;
      const int kb = __builtin_amdgcn_readfirstlane(load_id < total ? load_k * kBK * 2 : 0);
      const __amdgpu_buffer_rsrc_t lx = make_rsrc(xb, x_bytes);
      const __amdgpu_buffer_rsrc_t lw = make_rsrc(wb, w_bytes);
      const __amdgpu_buffer_rsrc_t lw2 = make_rsrc(w2b, DUAL ? w_bytes : 0);
#pragma unroll
      for (int i = 0; i < kOps; ++i) {
        if (i < XO) {
          lds_dma16(lx, dst + (pw + PW * i) * 1024, voff[i], kb);
        } else if (i < XO + WO) {
          lds_dma16(lw, dst + XB + (pw + PW * (i - XO)) * 1024, voff[i], kb);
        } else {
          lds_dma16(lw2, dst + XB + (BN / 2) * 128 + (pw + PW * (i - XO - WO)) * 1024, voff[i], kb);
        }
      }
      slot = slot == S - 1 ? 0 : slot + 1;
      if (++load_k == ktiles) {
        load_k = 0;
        load_id += step;
        set_tile(load_id);
      }
    };
#pragma unroll
    for (int t = 0; t < S - 1; ++t) issue();
    const int steps = ((total - 1 - first) / step + 1) * ktiles;
    for (int q = 0; q < steps; ++q) {
      asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"i"((S - 2) * kOps) : "memory");
      issue();
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    return;
  }

  // ---- consumers ------------------------------------------------------------
  const int c = lane & 15;
  const int g = lane >> 4;
  const int wm = wave / CWN;
  const int wn = wave % CWN;
  int slot = 0;
  for (int id = first; id < total; id += step) {
    const Tile t = tile_of(id);
    // Bias of this lane's four features per fragment, requested before the
    // k loop so that the epilogue does not wait for it.
    uint32_t braw[FN][2];
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      braw[j][0] = braw[j][1] = 0u;
      const int n = t.n0 + wn * TN + j * 16 + 4 * g;
      if (!DUAL && t.bias != nullptr && n < t.N) {
        const uint16_t* bp = reinterpret_cast<const uint16_t*>(t.bias + n);
        braw[j][0] = bp[0] | (static_cast<uint32_t>(bp[1]) << 16);
        braw[j][1] = bp[2] | (static_cast<uint32_t>(bp[3]) << 16);
      }
    }
    f32x4_t acc[FN][FM];
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int i = 0; i < FM; ++i) acc[j][i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    for (int kt = 0; kt < ktiles; ++kt) {
      // Tile kt is in its stage; the stage read before may be refilled.  No
      // wait on stores: the previous tile's output may still be in flight.
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      const unsigned char* xs = ring + slot * kStage;
      const unsigned char* ws = xs + XB;
      slot = slot == S - 1 ? 0 : slot + 1;
#pragma unroll
      for (int kk = 0; kk < kBK / 32; ++kk) {
        typename MF::vec a[FM], b[FN];
#pragma unroll
        for (int i = 0; i < FM; ++i)
          a[i] = *reinterpret_cast<const typename MF::vec*>(xs + lds_offset(wm * TM + i * 16 + c, kk * 4 + g));
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int wrow = DUAL ? (j < 2 ? wn * 32 + j * 16 : BN / 2 + wn * 32 + (j - 2) * 16)
                                : wn * TN + j * 16;
          b[j] = *reinterpret_cast<const typename MF::vec*>(ws + lds_offset(wrow + c, kk * 4 + g));
        }
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int i = 0; i < FM; ++i) acc[j][i] = MF::run(b[j], a[i], acc[j][i]);
      }
    }
    // Epilogue: lane (c, g) of fragment (j, i) holds features 4g .. 4g + 3 of
    // row c.
    const int rows = M - t.m0 < BM ? M - t.m0 : BM;
    const __amdgpu_buffer_rsrc_t ry =
        make_rsrc(t.y + t.m0 * t.y_rs, (static_cast<int64_t>(rows) - 1) * t.y_rs * 2 + t.N * 2);
    constexpr int kOutFrags = DUAL ? FN / 2 : FN;
#pragma unroll
    for (int j = 0; j < kOutFrags; ++j) {
      const int n = t.n0 + (DUAL ? wn * 32 : wn * TN) + j * 16 + 4 * g;
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int m_local = wm * TM + i * 16 + c;
        uint16_t o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if constexpr (DUAL) {
            const T ge = slc::from_f32<T>(acc[j][i][r]);
            const T ue = slc::from_f32<T>(acc[j + 2][i][r]);
            o[r] = slc::from_f32<T>(slc::swiglu_value<T>(slc::to_f32(ge), slc::to_f32(ue))).bits;
          } else {
            T bt;
            bt.bits = static_cast<uint16_t>(braw[j][r >> 1] >> (16 * (r & 1)));
            o[r] = slc::from_f32<T>(acc[j][i][r] + slc::to_f32(bt)).bits;
          }
        }
        if (m_local < rows && n < t.N) {
          const uint2 packed = make_uint2(o[0] | (static_cast<uint32_t>(o[1]) << 16),
                                          o[2] | (static_cast<uint32_t>(o[3]) << 16));
          __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(i32x2_t, packed), ry,
                                                static_cast<int>(m_local * t.y_rs + n) * 2, 0, 0);
        }
      }
    }
  }
}

// Decode-sized M (<= 64): Y is a handful of rows, W streams from HBM once.
// One workgroup owns 16 output features and all M rows; its KW waves split K
// between them (partial sums meet in LDS at the end), so even a 896-wide
// projection launches N/16 workgroups x KW waves.  Operands are loaded
// straight into MFMA registers -- lane (row c, k-slice g) takes 16 bytes of
// one W row per k-step -- U k-steps per batch, the next batch in flight while
// the current one is multiplied.
template <typename T, int MB, int KW, int U>
__global__ __launch_bounds__(KW * 64) void linear_skinny_kernel(
    const T* __restrict__ x, const T* __restrict__ w, const T* __restrict__ bias,
    T* __restrict__ y, int M, int N, int K, int64_t x_rs, int64_t y_rs) {
  using MF = Mfma<T>;
  __shared__ float partial[KW][MB][64][4];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int c = lane & 15;
  const int g = lane >> 4;
  const int n0 = blockIdx.x * 16;

  const int steps = (K + 31) / 32;               // 32-wide MFMA k-steps
  const int per_wave = (steps + KW - 1) / KW;
  const int s_begin = wave * per_wave;
  const int s_end = min(s_begin + per_wave, steps);

  const int w_rows = min(16, N - n0);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(w + static_cast<int64_t>(n0) * K,
                                              static_cast<int64_t>(w_rows) * K * 2);
  const __amdgpu_buffer_rsrc_t rx =
      make_rsrc(x, (static_cast<int64_t>(M) - 1) * x_rs * 2 + static_cast<int64_t>(K) * 2);
  // Per-lane byte offsets of k-step 0; rows past N / M read zero.
  const int w_off = c * K * 2 + g * 16;
  int x_off[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) x_off[i] = static_cast<int>((i * 16 + c) * x_rs * 2) + g * 16;

  f32x4_t acc[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  uint4 wa[U], xa[U][MB], wb[U], xb[U][MB];
  auto fetch = [&](int s0, uint4 (&wr)[U], uint4 (&xr)[U][MB]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int s = s0 + u;
      const int k = s * 32 + g * 8;
      // k past K (or past this wave's range) contributes zeros; within a row
      // the buffer range check cannot see the end, so this lane test does.
      const bool ok = s < s_end && k < K;
      wr[u] = ok ? buffer_load16(rw, w_off + s * 64) : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < MB; ++i)
        xr[u][i] = ok ? buffer_load16(rx, x_off[i] + s * 64) : make_uint4(0, 0, 0, 0);
    }
  };
  auto multiply = [&](const uint4 (&wr)[U], const uint4 (&xr)[U][MB]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const auto b = __builtin_bit_cast(typename MF::vec, wr[u]);
#pragma unroll
      for (int i = 0; i < MB; ++i)
        acc[i] = MF::run(__builtin_bit_cast(typename MF::vec, xr[u][i]), b, acc[i]);
    }
  };

  int s0 = s_begin;
  fetch(s0, wa, xa);
  while (s0 < s_end) {
    fetch(s0 + U, wb, xb);
    multiply(wa, xa);
    s0 += U;
    if (s0 >= s_end) break;
    fetch(s0 + U, wa, xa);
    multiply(wb, xb);
    s0 += U;
  }

  // C layout: lane (col c = feature, rows 4g..4g+3 = batch rows of block i).
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) partial[wave][i][lane][r] = acc[i][r];
  __syncthreads();
  for (int idx = tid; idx < MB * 64 * 4; idx += KW * 64) {
    const int i = idx / 256, l = (idx / 4) % 64, r = idx % 4;
    float sum = 0.0f;
#pragma unroll
    for (int v = 0; v < KW; ++v) sum += partial[v][i][l][r];
    const int n = n0 + (l & 15);
    const int m = i * 16 + 4 * (l >> 4) + r;
    if (n < N && m < M) {
      if (bias != nullptr) sum += slc::to_f32(bias[n]);
      y[m * y_rs + n] = slc::from_f32<T>(sum);
    }
  }
}

template <typename T, int MB>
int launch_skinny(const void* x, const void* w, const void* bias, void* y, int M, int N,
                  int K, int64_t x_rs, int64_t y_rs, hipStream_t stream) {
  // k-steps per prefetch batch: as deep as the registers allow.
  constexpr int KW = 8, U = MB == 1 ? 8 : (MB == 2 ? 4 : 2);
  hipLaunchKernelGGL((linear_skinny_kernel<T, MB, KW, U>), dim3((N + 15) / 16), dim3(KW * 64), 0,
                     stream, static_cast<const T*>(x), static_cast<const T*>(w),
                     static_cast<const T*>(bias), static_cast<T*>(y), M, N, K, x_rs, y_rs);
  return slc_host::check_launch("slc_hip_linear(skinny)");
}

// Classic 16 x 16 LDS-tiled FMA GEMM for fp32 and unaligned shapes.
template <typename T>
__global__ __launch_bounds__(256) void linear_generic_kernel(
    const T* __restrict__ x, const T* __restrict__ w, const T* __restrict__ bias,
    T* __restrict__ y, int M, int N, int K, int64_t x_rs, int64_t y_rs) {
  __shared__ float xs[16][17];
  __shared__ float ws[16][17];
  const int tx = threadIdx.x & 15;  // n within the tile
  const int ty = threadIdx.x >> 4;  // m within the tile
  const int m = blockIdx.y * 16 + ty;
  const int n = blockIdx.x * 16 + tx;
  float acc = 0.0f;
  for (int k0 = 0; k0 < K; k0 += 16) {
    const int xm = blockIdx.y * 16 + ty, xk = k0 + tx;
    xs[ty][tx] = (xm < M && xk < K) ? slc::to_f32(x[xm * x_rs + xk]) : 0.0f;
    const int wn_ = blockIdx.x * 16 + ty;
    ws[ty][tx] = (wn_ < N && xk < K) ? slc::to_f32(w[static_cast<int64_t>(wn_) * K + xk]) : 0.0f;
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) acc += xs[ty][kk] * ws[tx][kk];
    __syncthreads();
  }
  if (m < M && n < N) {
    if (bias != nullptr) acc += slc::to_f32(bias[n]);
    y[m * y_rs + n] = slc::from_f32<T>(acc);
  }
}

constexpr int kNoResidualPath = -2;  // the residual epilogue needs the 16-byte store path

template <typename T, int BM, int BN, int WM, int WN>
int launch_mfma(const void* x, const void* w, const void* bias, void* y, int M,
                int N, int K, int64_t x_rs, int64_t y_rs, hipStream_t stream,
                const void* residual = nullptr, int64_t r_rs = 0) {
  const dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
  const bool vst = N % 8 == 0 && y_rs % 8 == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0 &&
                   static_cast<int64_t>(BM) * y_rs * 2 < (int64_t{1} << 31);
  if (K % kBK == 0 && vst) {
    hipLaunchKernelGGL((linear_mfma_kernel<T, BM, BN, WM, WN, true, true>), grid, dim3(WM * WN * 64), 0,
                       stream, static_cast<const T*>(x), static_cast<const T*>(w),
                       static_cast<const T*>(bias), static_cast<T*>(y), M, N, K,
                       x_rs, y_rs, static_cast<const T*>(residual), r_rs);
    return slc_host::check_launch("slc_hip_linear");
  }
  if (residual != nullptr) return kNoResidualPath;
  if (K % kBK == 0) {
    hipLaunchKernelGGL((linear_mfma_kernel<T, BM, BN, WM, WN, true, false>), grid, dim3(WM * WN * 64), 0,
                       stream, static_cast<const T*>(x), static_cast<const T*>(w),
                       static_cast<const T*>(bias), static_cast<T*>(y), M, N, K,
                       x_rs, y_rs, static_cast<const T*>(nullptr), int64_t{0});
    return slc_host::check_launch("slc_hip_linear");
  }
  hipLaunchKernelGGL((linear_mfma_kernel<T, BM, BN, WM, WN, false, false>), grid, dim3(WM * WN * 64), 0,
                     stream, static_cast<const T*>(x), static_cast<const T*>(w),
                     static_cast<const T*>(bias), static_cast<T*>(y), M, N, K,
                     x_rs, y_rs, static_cast<const T*>(nullptr), int64_t{0});
  return slc_host::check_launch("slc_hip_linear");
}

// The ring kernel where the shape allows it (K a multiple of the k-tile, the
// 16-byte store path), else the register-staged kernel of the same tile.
template <typename T, int BM, int BN, int CWM, int CWN, int PW, int S, int GM = 8>
int launch_ring(const void* x, const void* w, const void* bias, void* y, int M, int N, int K,
                int64_t x_rs, int64_t y_rs, hipStream_t stream, const void* residual = nullptr,
                int64_t r_rs = 0) {
  const bool vst = N % 8 == 0 && y_rs % 8 == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0 &&
                   static_cast<int64_t>(BM) * y_rs * 2 < (int64_t{1} << 31) &&
                   static_cast<int64_t>(BM) * x_rs * 2 < (int64_t{1} << 31) &&
                   (residual == nullptr || static_cast<int64_t>(BM) * r_rs * 2 < (int64_t{1} << 31));
  if (K % kBK != 0 || !vst) return kNoResidualPath;
  const dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
  hipLaunchKernelGGL((linear_ring_kernel<T, BM, BN, CWM, CWN, PW, S, GM>), grid,
                     dim3((CWM * CWN + PW) * 64), 0, stream, static_cast<const T*>(x),
                     static_cast<const T*>(w), static_cast<const T*>(bias), static_cast<T*>(y), M, N,
                     K, x_rs, y_rs, static_cast<const T*>(residual), r_rs);
  return slc_host::check_launch("slc_hip_linear(ring)");
}

#ifndef SLC_STREAM_MIN_ROUNDS
#define SLC_STREAM_MIN_ROUNDS 2
#endif

// The persistent 256 x 128 form (linear_stream_kernel): one workgroup per CU
// (a multiple of 8, so each one's tiles stay on its XCD), or one per tile
// when there are fewer tiles.  kNoResidualPath where the shape does not fit.
// The library launches it for gate/up + SwiGLU (4-9 % faster there than the
// ring kernel, whose SwiGLU epilogue stages the whole tile in LDS); for plain
// linears it times within 2 % of the ring kernel and is a plan's choice.
template <typename T, bool DUAL>
int launch_stream(const void* x, const void* w, const void* bias, void* y, int M, int N, int K,
                  int64_t x_rs, int64_t y_rs, int n_tiles, hipStream_t stream,
                  const void* w2 = nullptr) {
  const bool fits = K % kBK == 0 && x_rs % 8 == 0 && N % 8 == 0 && y_rs % 8 == 0 &&
                    (reinterpret_cast<uintptr_t>(y) & 15) == 0 &&
                    256 * x_rs * 2 < (int64_t{1} << 31) && 256 * y_rs * 2 < (int64_t{1} << 31);
  if (!fits) return kNoResidualPath;
  const int m_tiles = (M + 255) / 256;
  const int64_t total = int64_t{n_tiles} * m_tiles;
  const int cus = slc_host::device_cu_count() / 8 * 8;
  const int grid = static_cast<int>(total < cus ? total : (cus > 0 ? cus : 8));
  hipLaunchKernelGGL((linear_stream_kernel<T, DUAL>), dim3(grid), dim3(12 * 64), 0, stream,
                     static_cast<const T*>(x), static_cast<const T*>(w),
                     static_cast<const T*>(bias), static_cast<T*>(y), M, N, K, x_rs, y_rs,
                     n_tiles, m_tiles, static_cast<const T*>(w2));
  return slc_host::check_launch("slc_hip_linear(stream)");
}

// Whether the persistent form takes a 256 x 128 grid of `tiles` output tiles:
// from SLC_STREAM_MIN_ROUNDS rounds of one workgroup per CU.
inline bool stream_grid(int64_t tiles) {
  return SLC_STREAM_MIN_ROUNDS > 0 &&
         tiles >= int64_t{SLC_STREAM_MIN_ROUNDS} * slc_host::device_cu_count();
}

// Ring-kernel tile for a shape when the caller leaves it to the library, by
// the number of 128 x 128 tiles the shape has: 256 x 128 from 300 of them
// (the larger tile reads less per flop once the grid is a few rounds deep),
// 128 x 128 from 128 (half a round on 256 CUs), then 128 x 64 while that
// grid has 192 workgroups, else 64 x 64 (small grids: the deep ring hides the
// latency of K's many k-tiles).  The winners measured on MI355X at the
// Qwen2-0.5B projection shapes for M = 128 .. 32768.
inline int auto_ring_tile(int64_t M, int64_t n_tiles128) {
  const int64_t n128 = ((M + 127) / 128) * n_tiles128;
  if (n128 >= 300) return SLC_TILE_R256X128;
  if (n128 >= 128) return SLC_TILE_R128X128;
  if (2 * n128 >= 192) return SLC_TILE_R128X64;
  return SLC_TILE_R64X64;
}

// One of the ring tiles; kNoResidualPath (nothing launched) where the shape
// does not fit the ring kernel.
template <typename T>
int launch_ring_tile(int tile, const void* x, const void* w, const void* bias, void* y, int M,
                     int N, int K, int64_t x_rs, int64_t y_rs, hipStream_t s,
                     const void* residual = nullptr, int64_t r_rs = 0) {
  switch (tile) {
    case SLC_TILE_R128X128:
      return launch_ring<T, 128, 128, 2, 4, 2, 4>(x, w, bias, y, M, N, K, x_rs, y_rs, s, residual, r_rs);
    case SLC_TILE_R256X128:
      // Groups of 4 M-tiles per XCD: eight 256-row X tiles (3.7 MB) would
      // not stay in one XCD's 4 MB L2 beside the W tiles.
      return launch_ring<T, 256, 128, 4, 2, 4, 3, 4>(x, w, bias, y, M, N, K, x_rs, y_rs, s, residual, r_rs);
    case SLC_TILE_R128X64:
      return launch_ring<T, 128, 64, 2, 2, 1, 3>(x, w, bias, y, M, N, K, x_rs, y_rs, s, residual, r_rs);
    case SLC_TILE_S256X128:
      if (residual == nullptr) {
        const int rc = launch_stream<T, false>(x, w, bias, y, M, N, K, x_rs, y_rs,
                                                      (N + 127) / 128, s);
        if (rc != kNoResidualPath) return rc;
      }
      return launch_ring<T, 256, 128, 4, 2, 4, 3, 4>(x, w, bias, y, M, N, K, x_rs, y_rs, s, residual, r_rs);
    default:
      return launch_ring<T, 64, 64, 2, 2, 1, 5>(x, w, bias, y, M, N, K, x_rs, y_rs, s, residual, r_rs);
  }
}

template <typename T>
int dispatch_mfma(const void* x, const void* w, const void* bias, void* y, int M,
                  int N, int K, int64_t x_rs, int64_t y_rs, hipStream_t s, int tile = SLC_TILE_AUTO) {
  // Up to 32 rows: the decode-step linear kernel the fused ops share.
  const int dtype = sizeof(T) == 2 && std::is_same<T, slc::bf16_t>::value ? SLC_BF16 : SLC_F16;
  if (M <= 32 && slc_host::rows_linear_eligible(x, x_rs, M, K, N, dtype))
    return slc_host::rows_linear(x, x_rs, M, K, N, w, bias, y, y_rs, dtype, s);
  if (M <= 16) return launch_skinny<T, 1>(x, w, bias, y, M, N, K, x_rs, y_rs, s);
  if (M <= 32) return launch_skinny<T, 2>(x, w, bias, y, M, N, K, x_rs, y_rs, s);
  if (M <= 64) return launch_skinny<T, 4>(x, w, bias, y, M, N, K, x_rs, y_rs, s);
  // Tile variants (a profile plan picks one): every tile accumulates each
  // output's k range in the same order, 32 k at a time on one MFMA chain, so
  // the variants differ in speed only, never in a bit of the result.
  if (tile == SLC_TILE_AUTO) tile = auto_ring_tile(M, (N + 127) / 128);
  switch (tile) {
    case SLC_TILE_128X64:
      return launch_mfma<T, 128, 64, 2, 2>(x, w, bias, y, M, N, K, x_rs, y_rs, s);
    case SLC_TILE_64X128:
      return launch_mfma<T, 64, 128, 2, 2>(x, w, bias, y, M, N, K, x_rs, y_rs, s);
    case SLC_TILE_64X64:
      return launch_mfma<T, 64, 64, 2, 2>(x, w, bias, y, M, N, K, x_rs, y_rs, s);
    case SLC_TILE_32X64:
      return launch_mfma<T, 32, 64, 2, 2>(x, w, bias, y, M, N, K, x_rs, y_rs, s);
    case SLC_TILE_128X128:
      // Eight waves of 64 x 32 (78 registers, six waves per SIMD): 4-9 %
      // faster than four of 64 x 64 at M 4096, equal at 32768.
      return launch_mfma<T, 128, 128, 2, 4>(x, w, bias, y, M, N, K, x_rs, y_rs, s);
    default: {
      const int rc = launch_ring_tile<T>(tile, x, w, bias, y, M, N, K, x_rs, y_rs, s);
      if (rc != kNoResidualPath) return rc;
      // K not a multiple of the k-tile, or outputs the 16-byte stores cannot
      // take: the register-staged kernel.
      return launch_mfma<T, 128, 128, 2, 4>(x, w, bias, y, M, N, K, x_rs, y_rs, s);
    }
  }
}

template <typename T>
int launch_generic(const void* x, const void* w, const void* bias, void* y, int M,
                   int N, int K, int64_t x_rs, int64_t y_rs, hipStream_t stream) {
  const dim3 grid((N + 15) / 16, (M + 15) / 16);
  hipLaunchKernelGGL((linear_generic_kernel<T>), grid, dim3(256), 0, stream,
                     static_cast<const T*>(x), static_cast<const T*>(w),
                     static_cast<const T*>(bias), static_cast<T*>(y), M, N, K,
                     x_rs, y_rs);
  return slc_host::check_launch("slc_hip_linear(generic)");
}

}  // namespace

namespace slc_host {

// Prefill-sized linear + residual add in one kernel (the tile kernel's
// 16-byte store epilogue adds the residual): y = residual + round(x.w^T +
// bias), rounded again, bit for bit the linear then the add.  Returns
// SLC_ERR_UNSUPPORTED (nothing launched) for shapes that epilogue cannot take.
int gemm_residual(const void* x, int64_t x_rs, int64_t rows, int64_t K, int64_t N,
                  const void* w, const void* bias, const void* residual, int64_t r_rs, void* y,
                  int64_t y_rs, int dtype, hipStream_t stream) {
  const uint64_t bits = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) |
                        reinterpret_cast<uintptr_t>(residual) | reinterpret_cast<uintptr_t>(y);
  const bool ok = (dtype == SLC_BF16 || dtype == SLC_F16) && rows > 64 && (bits & 15) == 0 &&
                  K % kBK == 0 && N % 8 == 0 && x_rs % 8 == 0 && y_rs % 8 == 0 &&
                  r_rs % 8 == 0 && N * K * 2 < (int64_t{1} << 31) &&
                  128 * x_rs * 2 < (int64_t{1} << 31) && 128 * y_rs * 2 < (int64_t{1} << 31) &&
                  128 * r_rs * 2 < (int64_t{1} << 31) && rows < (int64_t{1} << 31);
  if (!ok) return SLC_ERR_UNSUPPORTED;
  const int M = static_cast<int>(rows), n = static_cast<int>(N), k = static_cast<int>(K);
  const int tile = auto_ring_tile(M, (n + 127) / 128);
  int rc = dtype == SLC_BF16
               ? launch_ring_tile<slc::bf16_t>(tile, x, w, bias, y, M, n, k, x_rs, y_rs, stream,
                                               residual, r_rs)
               : launch_ring_tile<slc::f16_t>(tile, x, w, bias, y, M, n, k, x_rs, y_rs, stream,
                                              residual, r_rs);
  if (rc != kNoResidualPath) return rc;
  rc = dtype == SLC_BF16
           ? launch_mfma<slc::bf16_t, 128, 128, 2, 4>(x, w, bias, y, M, n, k, x_rs, y_rs,
                                                      stream, residual, r_rs)
           : launch_mfma<slc::f16_t, 128, 128, 2, 4>(x, w, bias, y, M, n, k, x_rs, y_rs,
                                                     stream, residual, r_rs);
  return rc == kNoResidualPath ? SLC_ERR_UNSUPPORTED : rc;
}

// Prefill-sized gate/up projections with SwiGLU in one kernel: y =
// swiglu(round(x.w_gate^T), round(x.w_up^T)), bit for bit the two linears
// then the elementwise op.  SLC_ERR_UNSUPPORTED (nothing launched) for shapes
// its epilogue cannot take.
int gemm_swiglu(const void* x, int64_t x_rs, int64_t rows, int64_t K, int64_t N,
                const void* w_gate, const void* w_up, void* y, int64_t y_rs, int dtype,
                hipStream_t stream) {
  const uint64_t bits = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w_gate) |
                        reinterpret_cast<uintptr_t>(w_up) | reinterpret_cast<uintptr_t>(y);
  const bool ok = (dtype == SLC_BF16 || dtype == SLC_F16) && rows > 64 && (bits & 15) == 0 &&
                  K % kBK == 0 && N % 8 == 0 && x_rs % 8 == 0 && y_rs % 8 == 0 &&
                  N * K * 2 < (int64_t{1} << 31) && 128 * x_rs * 2 < (int64_t{1} << 31) &&
                  128 * y_rs * 2 < (int64_t{1} << 31) && rows < (int64_t{1} << 31);
  if (!ok) return SLC_ERR_UNSUPPORTED;
  const int M = static_cast<int>(rows), n = static_cast<int>(N), k = static_cast<int>(K);
  // The ring kernel; each 128-wide column tile holds 64 gate and 64 up rows.
  const bool big = auto_ring_tile(M, (n + 63) / 64) == SLC_TILE_R256X128 &&
                   256 * x_rs * 2 < (int64_t{1} << 31) && 256 * y_rs * 2 < (int64_t{1} << 31);
  if (big && stream_grid(int64_t{(M + 255) / 256} * ((n + 63) / 64))) {
    // Several rounds of 256 x 128 tiles: the persistent form, whose
    // SwiGLU pairs meet in registers instead of a staged LDS tile.
    const int rc = dtype == SLC_BF16
                       ? launch_stream<slc::bf16_t, true>(x, w_gate, nullptr, y, M, n, k, x_rs, y_rs,
                                                          (n + 63) / 64, stream, w_up)
                       : launch_stream<slc::f16_t, true>(x, w_gate, nullptr, y, M, n, k, x_rs, y_rs,
                                                         (n + 63) / 64, stream, w_up);
    if (rc != kNoResidualPath) return rc;
  }
#define SLC_DUAL(TT, BM, CWM, PW, S, GM)                                                          \
  hipLaunchKernelGGL((linear_ring_kernel<TT, BM, 128, CWM, 2 * 4 / CWM, PW, S, GM, true>),         \
                     dim3((n + 63) / 64, (M + BM - 1) / BM), dim3((8 + PW) * 64), 0, stream,      \
                     static_cast<const TT*>(x), static_cast<const TT*>(w_gate),                   \
                     static_cast<const TT*>(nullptr), static_cast<TT*>(y), M, n, k, x_rs, y_rs,   \
                     static_cast<const TT*>(nullptr), int64_t{0}, static_cast<const TT*>(w_up))
  if (dtype == SLC_BF16) {
    if (big) SLC_DUAL(slc::bf16_t, 256, 4, 4, 3, 4); else SLC_DUAL(slc::bf16_t, 128, 2, 2, 4, 8);
  } else {
    if (big) SLC_DUAL(slc::f16_t, 256, 4, 4, 3, 4); else SLC_DUAL(slc::f16_t, 128, 2, 2, 4, 8);
  }
#undef SLC_DUAL
  return check_launch("slc_hip_linear_swiglu");
}

// Prefill-sized projections of one input (Q/K/V) in one launch, each matrix
// bit for bit its own linear.  SLC_ERR_UNSUPPORTED (nothing launched) for
// shapes the store epilogue cannot take.
int gemm_group(const void* x, int64_t x_rs, int64_t rows, int64_t K, int count,
               const void* const* w, const void* const* bias, void* const* y,
               const int64_t* n, const int64_t* y_rs, int dtype, hipStream_t stream) {
  bool ok = (dtype == SLC_BF16 || dtype == SLC_F16) && rows > 64 && count >= 1 && count <= 3 &&
            K % kBK == 0 && x_rs % 8 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
            128 * x_rs * 2 < (int64_t{1} << 31) && rows < (int64_t{1} << 31);
  LinearGroup g{};
  int tiles = 0;
  for (int j = 0; j < 3; ++j) {
    if (j < count) {
      ok = ok && w[j] != nullptr && y[j] != nullptr && n[j] >= 1 && n[j] % 8 == 0 &&
           y_rs[j] % 8 == 0 && y_rs[j] >= n[j] && n[j] * K * 2 < (int64_t{1} << 31) &&
           128 * y_rs[j] * 2 < (int64_t{1} << 31) &&
           ((reinterpret_cast<uintptr_t>(w[j]) | reinterpret_cast<uintptr_t>(y[j])) & 15) == 0;
      if (!ok) break;
      g.w[j] = w[j];
      g.bias[j] = bias[j];
      g.y[j] = y[j];
      g.n[j] = static_cast<int>(n[j]);
      g.y_rs[j] = y_rs[j];
      tiles += static_cast<int>((n[j] + 127) / 128);
    }
    g.tile_end[j] = tiles;
  }
  if (!ok) return SLC_ERR_UNSUPPORTED;
  const int M = static_cast<int>(rows), k = static_cast<int>(K);
  bool big = auto_ring_tile(M, tiles) == SLC_TILE_R256X128 && 256 * x_rs * 2 < (int64_t{1} << 31);
  for (int j = 0; j < count; ++j) big = big && 256 * y_rs[j] * 2 < (int64_t{1} << 31);
#define SLC_GROUP(TT, BM, CWM, PW, S, GM)                                                        \
  hipLaunchKernelGGL((linear_ring_kernel<TT, BM, 128, CWM, 2 * 4 / CWM, PW, S, GM, false, true>), \
                     dim3(static_cast<unsigned>(tiles), (M + BM - 1) / BM), dim3((8 + PW) * 64), \
                     0, stream, static_cast<const TT*>(x), static_cast<const TT*>(nullptr),       \
                     static_cast<const TT*>(nullptr), static_cast<TT*>(nullptr), M, 0, k, x_rs,   \
                     int64_t{0}, static_cast<const TT*>(nullptr), int64_t{0},                     \
                     static_cast<const TT*>(nullptr), g)
  if (dtype == SLC_BF16) {
    if (big) SLC_GROUP(slc::bf16_t, 256, 4, 4, 3, 4); else SLC_GROUP(slc::bf16_t, 128, 2, 2, 4, 8);
  } else {
    if (big) SLC_GROUP(slc::f16_t, 256, 4, 4, 3, 4); else SLC_GROUP(slc::f16_t, 128, 2, 2, 4, 8);
  }
#undef SLC_GROUP
  return check_launch("slc_hip_linear_group");
}

}  // namespace slc_host

extern "C" int slc_hip_linear_group(const void* input, int64_t in_stride_row, int64_t rows,
                                    int64_t in_features, int count, const void* w0,
                                    const void* b0, void* y0, int64_t n0, int64_t y0_rs,
                                    const void* w1, const void* b1, void* y1, int64_t n1,
                                    int64_t y1_rs, const void* w2, const void* b2, void* y2,
                                    int64_t n2, int64_t y2_rs, int dtype, void* stream) {
  SLC_REQUIRE(rows >= 0 && in_features > 0 && count >= 1 && count <= 3,
              "slc_hip_linear_group: bad sizes");
  if (rows == 0) return SLC_OK;
  SLC_REQUIRE(input != nullptr, "slc_hip_linear_group: null input");
  const void* ws[3] = {w0, w1, w2};
  const void* bs[3] = {b0, b1, b2};
  void* ys[3] = {y0, y1, y2};
  const int64_t ns[3] = {n0, n1, n2};
  const int64_t rss[3] = {y0_rs, y1_rs, y2_rs};
  return slc_host::gemm_group(input, in_stride_row, rows, in_features, count, ws, bs, ys, ns, rss,
                              dtype, static_cast<hipStream_t>(stream));
}

extern "C" int slc_hip_linear_swiglu(const void* input, int64_t in_stride_row, int64_t rows,
                                     int64_t in_features, int64_t features, const void* w_gate,
                                     const void* w_up, void* output, int64_t out_stride_row,
                                     int dtype, void* stream) {
  SLC_REQUIRE(rows >= 0 && in_features > 0 && features > 0,
              "slc_hip_linear_swiglu: bad sizes");
  if (rows == 0) return SLC_OK;
  SLC_REQUIRE(input && w_gate && w_up && output, "slc_hip_linear_swiglu: null pointer");
  return slc_host::gemm_swiglu(input, in_stride_row, rows, in_features, features, w_gate, w_up,
                               output, out_stride_row, dtype, static_cast<hipStream_t>(stream));
}

extern "C" int slc_hip_linear_tile(const void* input, const void* weight,
                                   const void* bias, void* output, int dtype,
                                   int64_t rows, int64_t out_features,
                                   int64_t in_features, int64_t in_stride_row,
                                   int64_t out_stride_row, int tile, void* stream) {
  SLC_REQUIRE(tile >= SLC_TILE_AUTO && tile <= SLC_TILE_S256X128, "slc_hip_linear_tile: bad tile %d",
              tile);
  SLC_REQUIRE(slc_host::is_float_dtype(dtype), "slc_hip_linear: bad dtype %d", dtype);
  SLC_REQUIRE(rows >= 0 && out_features > 0 && in_features > 0,
              "slc_hip_linear: bad sizes M=%lld N=%lld K=%lld", (long long)rows,
              (long long)out_features, (long long)in_features);
  SLC_REQUIRE(rows < (1LL << 31) && out_features < (1LL << 31) &&
                  in_features < (1LL << 31),
              "slc_hip_linear: sizes exceed 2^31");
  if (rows == 0) return SLC_OK;
  SLC_REQUIRE(input && weight && output, "slc_hip_linear: null pointer");
  const int M = static_cast<int>(rows), N = static_cast<int>(out_features),
            K = static_cast<int>(in_features);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint64_t bits = reinterpret_cast<uintptr_t>(input) |
                        reinterpret_cast<uintptr_t>(weight);
  // The vector path addresses each workgroup's X and W slices with 32-bit
  // offsets and loads 16-byte chunks.
  const bool vec_ok = (bits & 15) == 0 && K % 8 == 0 && in_stride_row % 8 == 0 &&
                      static_cast<int64_t>(N) * K * 2 < (1LL << 31) &&
                      128 * in_stride_row * 2 < (1LL << 31);
  if (vec_ok && dtype == SLC_BF16)
    return dispatch_mfma<slc::bf16_t>(input, weight, bias, output, M, N, K,
                                      in_stride_row, out_stride_row, s, tile);
  if (vec_ok && dtype == SLC_F16)
    return dispatch_mfma<slc::f16_t>(input, weight, bias, output, M, N, K,
                                     in_stride_row, out_stride_row, s, tile);
  switch (dtype) {
    case SLC_F32:
      return launch_generic<float>(input, weight, bias, output, M, N, K,
                                   in_stride_row, out_stride_row, s);
    case SLC_BF16:
      return launch_generic<slc::bf16_t>(input, weight, bias, output, M, N, K,
                                         in_stride_row, out_stride_row, s);
    default:
      return launch_generic<slc::f16_t>(input, weight, bias, output, M, N, K,
                                        in_stride_row, out_stride_row, s);
  }
}

extern "C" int slc_hip_linear(const void* input, const void* weight,
                              const void* bias, void* output, int dtype,
                              int64_t rows, int64_t out_features,
                              int64_t in_features, int64_t in_stride_row,
                              int64_t out_stride_row, void* stream) {
  return slc_hip_linear_tile(input, weight, bias, output, dtype, rows, out_features, in_features,
                             in_stride_row, out_stride_row, SLC_TILE_AUTO, stream);
}
