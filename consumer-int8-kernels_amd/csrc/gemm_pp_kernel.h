// The persistent two-waves-per-SIMD INT8 GEMM kernel (the design is described in
// gemm_pp.hip). It lives in this header so that a measurement build of the same source
// (probe_pp.hip, with per-phase clock stamps) compiles exactly the library's code path.
#pragma once
#include <type_traits>

#include "ci8_device.h"
#include "launch.h"

namespace ci8 {
namespace {

constexpr int kXcds = 8;

// Tiles of 256 (m) x kBN (n), kBN = 224 (the default) or 160 (the narrow tiles that let
// a launch end in whole rounds; see launch_pp_gemm). Group g = wave / 4 owns WN = kBN / 2
// columns of the tile.
template <int kBN>
struct PPConfigT {
  static constexpr int BM = 256, BN = kBN, BK = 128;
  static constexpr int kWaves = 8, kThreads = 512;
  static constexpr int WM = 4;                        // waves along m (per group)
  static constexpr int WN = BN / 2;                   // columns per group (112 or 80)
  static constexpr int TM = BM / WM / 16;             // 4 m blocks per wave
  static constexpr int TN = WN / 16;                  // 7 (or 5) n blocks per wave
  static constexpr int kABlocks = BM * BK / 1024;     // 32 copies of A per stage
  static constexpr int kWBlocks = BN * BK / 1024;     // 28 (or 20) copies of W per stage
  static constexpr int kCopies = kABlocks / WM;       // per A wave per stage (8)
  static constexpr int kWValid = kWBlocks / WM;       // per W wave per stage (7 or 5)
  // Copies a W wave issues per stage: with 7 the eighth reads nothing into a junk KiB, so
  // that both groups' copy sequences are alike; with 5 it issues just those.
  static constexpr int kWCopies = kWValid == kCopies - 1 ? kCopies : kWValid;
  // Copies go out after fragment reads 0, kCopyEvery, 2 kCopyEvery, ... of the memory
  // phase's 2 (TM + TN) reads (22 or 18).
  static constexpr int kCopyEvery = 3 * (kCopies - 1) < 2 * (TM + TN) ? 3 : 2;
  static constexpr int kAStage = BM * BK;             // 32 KB
  static constexpr int kWStage = BN * BK;             // 28 (or 20) KB
  static constexpr int kWBase = 2 * kAStage;          // A ring: 2 slots, W ring: 3 slots
  static constexpr int kJunk = kWBase + 3 * kWStage;  // 148 (or 124) KB
  static constexpr int kRingBytes = kJunk + 1024;
  // Epilogue staging (reuses the ring): each wave's 64 x WN BF16 outputs at a row stride
  // of WN * 2 + 16 bytes (60 or 44 dwords: 16 rows written by one ds_write_b64 start in
  // distinct banks).
  static constexpr int kEpiRowBytes = WN * 2 + 16;
  static constexpr int kEpiPassBytes = 16 * kEpiRowBytes;  // one 16-row block per wave
  // The tile's row scales (256 FP32) and channel scales (BN BF16, copied as 256), copied
  // into LDS at the tile start (waves 0-3 their own 64 rows' scales, waves 4 and 5 128
  // channels each, 4 bytes a lane) and read back by the epilogue, so they take no
  // registers through the K loop.
  static constexpr int kScaleBase = kRingBytes;
  static constexpr int kLdsBytes = kRingBytes + 4 * BM + 2 * 256;
  // m tiles per raster group: each XCD's 32 tiles of a round then cover 4 m x 8 n
  // tiles (measured on MI355X against 2, 8 and 16: configs[2] 277-278 against 280-286
  // us at 8; configs[3] 1,108-1,110 against 1,152-1,154 us).
  static constexpr int GROUP_M = 4;
  static_assert(kCopies * WM == kABlocks && kWValid * WM == kWBlocks && kWCopies <= kCopies,
                "copies");
  static_assert(kCopyEvery * (kCopies - 1) < 2 * (TM + TN), "copies fit between the fragment reads");
  static_assert(WN % 16 == 0 && BN <= 256, "tile width");
  static_assert(kLdsBytes <= 160 * 1024, "LDS");
  static_assert(kWaves * kEpiPassBytes <= kAStage, "epilogue passes fit in A slot 1");
};
using PPConfig = PPConfigT<224>;
using PPConfigNarrow = PPConfigT<160>;

__device__ __forceinline__ i32x4 lds16(const char __attribute__((address_space(3)))* p) {
  return *reinterpret_cast<const __attribute__((address_space(3))) i32x4*>(p);
}
__device__ __forceinline__ void barrier_fenced() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// kStamps (a measurement build only; the library uses 0): 1 records each workgroup's
// shader-clock and wall-clock times at start and end, 2 also sums, per wave, the cycles of
// each phase kind (PhaseStamp) and records those of waves 0 and 4 (one of each group).
// Layout of `stamps`, kStampWords values per workgroup: wave 0's clock start, clock end,
// wall start and wall end; the kStampKinds sums of wave 0, then those of wave 4; wave 4's
// clock start and end; the rest is not written. Each wave's sums add up to its own clock
// end minus its clock start. Reading s_memtime waits for the read, so mode 2 runs slower
// than the kernel it describes.
enum PhaseStamp {
  kStampMemory, kStampWaitW, kStampBarrier1, kStampCompute, kStampWaitA, kStampBarrier2,
  kStampTileStart, kStampDrain, kStampEpilogue, kStampTileEnd, kStampKinds
};
constexpr int kStampWords = 32;
static_assert(6 + 2 * kStampKinds <= kStampWords, "stamp record");

// out[row, col] is written at out + row * ldo + col (ldo >= n): a launch may cover a
// column range of a wider output.
template <bool kExactK, WeightCode kCode, int kStamps = 0, int kBN = 224>
__global__ void __launch_bounds__(PPConfigT<kBN>::kThreads, 1) pp_gemm_kernel(
    const int8_t* __restrict__ a, const int8_t* __restrict__ w, const float* __restrict__ sa,
    const uint16_t* __restrict__ sw, uint16_t* __restrict__ out, int m, int n, int k, int ldo,
    bool out16, int64_t* __restrict__ stamps) {
  using C = PPConfigT<kBN>;
  extern __shared__ __attribute__((aligned(1024))) char lds_raw[];
  auto* lds = (char __attribute__((address_space(3)))*)(lds_raw);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave % C::WM, group = wave / C::WM;
  const bool copies_a = group == 0;

  // Work item -> tile: items are dealt to the 8 XCDs round-robin (workgroup b runs on
  // XCD b % 8 and takes items b, b + grid, ...; the grid is a multiple of 8 when it
  // fills the chip), so map the items of each XCD to a contiguous range of a grouped
  // raster of GROUP_M m tiles: tiles that run together on one XCD share panels in its L2.
  const int tiles_n = (n + C::BN - 1) / C::BN;
  const int tiles_m = (m + C::BM - 1) / C::BM;
  const int tiles = tiles_n * tiles_m;
  const int grid = int(gridDim.x);
  const int my_tiles = (tiles - int(blockIdx.x) + grid - 1) / grid;
  auto tile_of = [&] __device__(int item, int& m0, int& n0) __attribute__((always_inline)) {
    const int per = tiles / kXcds, extra = tiles % kXcds;
    const int xcd = item % kXcds, idx = item / kXcds;
    const int logical =
        (xcd < extra ? xcd * (per + 1) : extra * (per + 1) + (xcd - extra) * per) + idx;
    const int group_span = C::GROUP_M * tiles_n;
    const int first_m = (logical / group_span) * C::GROUP_M;
    const int group_rows = min(tiles_m - first_m, C::GROUP_M);
    m0 = (first_m + (logical % group_span) % group_rows) * C::BM;
    n0 = ((logical % group_span) / group_rows) * C::BN;
  };

  const auto a_rsrc = make_rsrc(a, uint32_t(m) * uint32_t(k));
  const auto w_rsrc = make_rsrc(w, uint32_t(n) * uint32_t(k));
  const auto c_rsrc = copies_a ? a_rsrc : w_rsrc;
  const int ns = (k + C::BK - 1) / C::BK;
  const auto sa_rsrc = make_rsrc(sa, uint32_t(m) * 4u);
  const auto sw_rsrc = make_rsrc(sw, uint32_t(n) * 2u);

  // Copy i of a wave brings block b = 4i + wave % 4 of its operand's stage (8 rows x 128
  // bytes): lane -> row 8b + lane / 8, LDS chunk slot lane % 8 holding logical chunk
  // slot ^ (row % 8). The stage's K offset goes in soffset; the per-lane row offsets
  // depend on the tile and are set when a tile's first copies are issued.
  const int sub = wave % C::WM;
  const int c_row = lane >> 3;
  const int c_chunk = (lane & 7) ^ c_row;
  uint32_t c_off[C::kCopies];
  // K order of a tile: tile (mt, nt) (m0 = 256 mt, n0 = BN nt) copies its K stages in the
  // order t0, t0 + 1, ..., ns - 1, 0, ..., t0 - 1 with t0 = (mt + nt) % 8 (mod ns). The 32
  // tiles an XCD runs together are 4 m x 8 n tiles of the raster, so the 4 that share a W
  // panel and the 8 that share an A panel start at distinct stages and reach each K slice
  // a stage or more apart instead of together: the first to arrive fetches the slice into
  // the XCD's L2, the rest find it there. The INT32 sums are exact in any order, so the
  // output bits are the same. Measured on MI355X at configs[2] (same process, three runs):
  // 272.0-274.9 against 278.1-285.7 us (starting W sharers only 2 stages apart: 272.1-276.0;
  // A sharers only: 288.3-290.4; 2 stages apart or 16 offsets: no gain).
  int c_t0 = 0;
  auto set_copy_tile = [&] __device__(int m0, int n0) __attribute__((always_inline)) {
    c_t0 = (m0 / C::BM + n0 / C::BN) % 8 % ns;
#pragma unroll
    for (int i = 0; i < C::kCopies; ++i) {
      const int row = (copies_a ? m0 : n0) + (i * C::WM + sub) * 8 + c_row;
      const bool valid = (copies_a || i < C::kWValid) && row < (copies_a ? m : n);
      c_off[i] = valid ? uint32_t(row) * uint32_t(k) + uint32_t(c_chunk * 16) : kOutOfRange;
    }
  };
  // LDS destination of copy i into ring slot `slot`: c_dst0 + slot * c_stride + 4096 i
  // (integer arithmetic on wave-uniform values), except a W wave's junk copies.
  const int c_dst0 = (copies_a ? 0 : C::kWBase) + sub * 1024;
  const int c_stride = copies_a ? C::kAStage : C::kWStage;
  auto copy = [&] __device__(int dst, int t, int i) __attribute__((always_inline)) {
    int to = dst + i * C::WM * 1024;
    if (i >= C::kWValid) to = copies_a ? to : C::kJunk;
    const int k0 = (t + c_t0 < ns ? t + c_t0 : t + c_t0 - ns) * C::BK;  // stage t of the tile's order
    uint32_t off = c_off[i];
    if (!kExactK && off != kOutOfRange && k0 + c_chunk * 16 >= k) off = kOutOfRange;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(c_rsrc, reinterpret_cast<lds_void*>(lds + to), 16,
                                             off, k0, 0, 0);
  };
  // A tile's first copies, where the previous tile's last stages did not issue them (the
  // launch's first tile, and every tile when ns == 1): A(0) (group 0) into A slot a_slot,
  // W(0) and W(1) (group 1) into W slots w_slot0 and w_slot1.
  auto first_copies = [&] __device__(int a_slot, int w_slot0, int w_slot1) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < C::kCopies; ++i)
      if (copies_a || i < C::kWCopies) copy(c_dst0 + (copies_a ? a_slot : w_slot0) * c_stride, 0, i);
    if (!copies_a && 1 < ns) {
#pragma unroll
      for (int i = 0; i < C::kWCopies; ++i) copy(c_dst0 + w_slot1 * c_stride, 1, i);
    }
  };

  // Fragments: row (lane % 16) of each 16-row block at logical chunk 4h + lane / 16.
  const int f_row = lane & 15, f_group = lane >> 4;
  int a_base[2], w_base[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int swz = (((4 * h + f_group) ^ (f_row & 7)) * 16);
    a_base[h] = (wm * 64 + f_row) * C::BK + swz;
    w_base[h] = C::kWBase + (group * C::WN + f_row) * C::BK + swz;
  }
  i32x4 af[2][C::TM], wf[2][C::TN];
  // Memory phase: the 2 (TM + TN) fragments of the stage in A slot a_slot and W slot
  // w_slot, with (kCopy) this wave's copies of stage copy_t into `dst` after fragment
  // reads 0, kCopyEvery, ... (224-wide tiles: 22 reads, 8 copies after reads 0, 3, ...,
  // 21). Stages past the end are not copied at all.
  auto memory = [&] __device__(int a_slot, int w_slot, int dst, int copy_t, auto with_copies)
                    __attribute__((always_inline)) {
    constexpr bool kCopy = decltype(with_copies)::value;
    const auto* as = lds + a_slot * C::kAStage;
    const auto* ws = lds + w_slot * C::kWStage;
#pragma unroll
    for (int q = 0; q < 2 * (C::TM + C::TN); ++q) {
      const int h = q / (C::TM + C::TN), r = q % (C::TM + C::TN);
      if (r < C::TM)
        af[h][r] = lds16(as + a_base[h] + r * 16 * C::BK);
      else
        wf[h][r - C::TM] = lds16(ws + w_base[h] + (r - C::TM) * 16 * C::BK);
      if constexpr (kCopy)
        if (q % C::kCopyEvery == 0 && q / C::kCopyEvery < C::kCopies &&
            (copies_a || q / C::kCopyEvery < C::kWCopies))
          copy(dst, copy_t, q / C::kCopyEvery);
    }
    __builtin_amdgcn_s_waitcnt(lgkmcnt0_imm());
    if constexpr (kCode == WeightCode::kBiasedU8) {
      // Biased UINT8 codes (code + 128) -> signed INT8 codes: flip each byte's top bit.
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < C::TN; ++i) wf[h][i] ^= int(0x80808080u);
    }
  };

  i32x4 acc[C::TM][C::TN];
  auto compute = [&] __device__() __attribute__((always_inline)) {
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < C::TN; ++i)
#pragma unroll
        for (int j = 0; j < C::TM; ++j)
          acc[j][i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[h][i], af[h][j], acc[j][i], 0, 0, 0);
    __builtin_amdgcn_s_setprio(0);
  };

  if (my_tiles <= 0) return;  // uniform over the workgroup
  int64_t phase[kStampKinds] = {};
  int64_t last = 0, clock0 = 0, wall0 = 0;
  if constexpr (kStamps > 0) {
    wall0 = __builtin_amdgcn_s_memrealtime();
    clock0 = last = __builtin_amdgcn_s_memtime();
  }
  // Adds the cycles since the previous stamp to phase kind `kind` (mode 2 only).
  auto stamp = [&] __device__(int kind) __attribute__((always_inline)) {
    if constexpr (kStamps > 1) {
      __builtin_amdgcn_sched_barrier(0);
      const int64_t now = __builtin_amdgcn_s_memtime();
      phase[kind] += now - last;
      last = now;
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  int m0, n0;
  tile_of(int(blockIdx.x), m0, n0);
  set_copy_tile(m0, n0);
  first_copies(0, 0, 1);
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  // Ring slots run on across tiles: stage g of the launch's stream (tile r, K stage t,
  // g = r * ns + t) uses A slot g % 2 and W slot g % 3. With ns >= 2 the next tile's
  // first stages are copied by the current tile's last stages like any other stage.
  int a_slot = 0;   // g % 2
  int w_slot = 0;   // g % 3
  int cw_slot = 2;  // (g + 2) % 3
  const bool stream_ok = ns >= 2;
  barrier_fenced();

  for (int r = 0; r < my_tiles; ++r) {
    // This tile's row and channel scales go to LDS now (older than any copy of the tile,
    // so the waits of the K loop cover them).
    if (wave < C::WM + 2) {  // uniform over the wave
      const bool rows = wave < C::WM;
      const int part = rows ? wave : wave - C::WM;
      const uint32_t off = rows ? uint32_t(m0 + part * 64) * 4u + uint32_t(lane) * 4u
                                : uint32_t(n0 + part * 128) * 2u + uint32_t(lane) * 4u;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rows ? sa_rsrc : sw_rsrc,
          reinterpret_cast<lds_void*>(lds + C::kScaleBase + (rows ? 0 : 4 * C::BM) + part * 256),
          4, off, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < C::TM; ++j)
#pragma unroll
      for (int i = 0; i < C::TN; ++i) acc[j][i] = i32x4{0, 0, 0, 0};

    const int tile_m0 = m0, tile_n0 = n0;
    const bool more = r + 1 < my_tiles;
    const int lead = copies_a ? 1 : 2;
    if (group == 1) barrier_fenced();  // phase 0 is group 0's first memory phase
    stamp(kStampTileStart);
    for (int t = 0; t < ns; ++t) {
      int copy_t = t + lead;
      const bool next_tile = copy_t >= ns;
      if (next_tile && more && stream_ok) {
        if (copy_t == ns) {  // this group's first copy of the next tile
          tile_of(int(blockIdx.x) + (r + 1) * grid, m0, n0);
          set_copy_tile(m0, n0);
        }
        copy_t -= ns;
      }
      const bool copies = !next_tile || (more && stream_ok);
      const int dst = c_dst0 + (copies_a ? a_slot ^ 1 : cw_slot) * c_stride;
      if (copies) {  // uniform over the wave
        memory(a_slot, w_slot, dst, copy_t, std::true_type{});
        stamp(kStampMemory);
        // Group 1: W(t + 1) landed (W(t + 2), just issued, may be in flight). In the last
        // stage nothing of this tile is left to wait for.
        if (group == 1 && t + 1 < ns) __builtin_amdgcn_s_waitcnt(vmcnt_imm(C::kWCopies));
      } else {
        memory(a_slot, w_slot, dst, copy_t, std::false_type{});
        stamp(kStampMemory);
        if (group == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
      }
      stamp(kStampWaitW);
      barrier_fenced();
      stamp(kStampBarrier1);
      compute();
      stamp(kStampCompute);
      // Group 0: A(t + 1), issued in the memory phase, landed (in the last stage, the next
      // tile's A(0) is waited for at the tile switch).
      if (group == 0 && (t + 1 < ns || !stream_ok)) __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
      stamp(kStampWaitA);
      barrier_fenced();
      stamp(kStampBarrier2);
      a_slot ^= 1;
      w_slot = w_slot == 2 ? 0 : w_slot + 1;
      cw_slot = cw_slot == 2 ? 0 : cw_slot + 1;
    }
    if (group == 0) barrier_fenced();  // phase 2 ns: group 1's last compute phase
    barrier_fenced();                  // every wave is past its last fragment reads
    stamp(kStampDrain);
    if (more && !stream_ok) {
      tile_of(int(blockIdx.x) + (r + 1) * grid, m0, n0);
      set_copy_tile(m0, n0);
      first_copies(a_slot, w_slot, w_slot == 2 ? 0 : w_slot + 1);
    }
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");

    // Epilogue through LDS, 16 rows of the wave's 64 at a time: the 16 x WN BF16
    // results of row block j go to the wave's region of the A slot the tile's last stage
    // used (the next tile's A(0) is in the other) in the MFMA layout and come back as
    // 16-byte row chunks, so each store instruction writes whole row pieces of 2 WN
    // bytes (224-wide tiles: 224 bytes, 14 lanes per row).
    const int row0 = tile_m0 + wm * 64;
    const int col0 = tile_n0 + group * C::WN;
    auto* region = lds + (a_slot ^ 1) * C::kAStage + wave * C::kEpiPassBytes;
    float rs[C::TM];
    u32x2 s2[C::TN];
#pragma unroll
    for (int j = 0; j < C::TM; ++j)
      rs[j] = *reinterpret_cast<const __attribute__((address_space(3))) float*>(
          lds + C::kScaleBase + (wm * 64 + j * 16 + f_row) * 4);
#pragma unroll
    for (int i = 0; i < C::TN; ++i)
      s2[i] = *reinterpret_cast<const __attribute__((address_space(3))) u32x2*>(
          lds + C::kScaleBase + 4 * C::BM + (group * C::WN + i * 16 + f_group * 4) * 2);
    constexpr int kChunks = C::WN / 8;  // 16-byte chunks per output row piece
    const bool full = out16 && row0 + 64 <= m && col0 + C::WN <= n && (ldo % 8) == 0;
#pragma unroll
    for (int j = 0; j < C::TM; ++j) {
      auto* rbase = region + f_row * C::kEpiRowBytes + f_group * 8;
#pragma unroll
      for (int i = 0; i < C::TN; ++i) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t bits = (s2[i][e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
          v[e] = (float(acc[j][i][e]) * rs[j]) * bf16_to_f32(bits);
        }
        *reinterpret_cast<__attribute__((address_space(3))) u32x2*>(rbase + i * 32) =
            u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
      }
      // One wave's LDS operations complete in order; the wait only orders the reads
      // after every lane's writes for the compiler.
      __builtin_amdgcn_s_waitcnt(lgkmcnt0_imm());
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int it = 0; it < (16 * kChunks + 63) / 64; ++it) {
        const int q = it * 64 + lane;
        if (q >= 16 * kChunks) break;
        const int row = q / kChunks, chunk = q % kChunks;
        const u32x4 v = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(
            region + row * C::kEpiRowBytes + chunk * 16);
        const int grow = row0 + j * 16 + row, gcol = col0 + chunk * 8;
        uint16_t* dst = out + int64_t(grow) * ldo + gcol;
        if (full) {
          *reinterpret_cast<u32x4*>(dst) = v;
        } else if (grow < m) {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (gcol + e < n) dst[e] = uint16_t(v[e >> 1] >> (16 * (e & 1)));
        }
      }
      // The next row block's writes reuse the region after these reads.
      __builtin_amdgcn_s_waitcnt(lgkmcnt0_imm());
      __builtin_amdgcn_wave_barrier();
    }
    stamp(kStampEpilogue);
    if (more) {
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // the next tile's first copies landed
      barrier_fenced();  // every wave's, and the epilogue's LDS (A slot, scales) is free
    }
    stamp(kStampTileEnd);
  }
  if constexpr (kStamps > 0) {
    const int64_t clock1 = __builtin_amdgcn_s_memtime();
    const int64_t wall1 = __builtin_amdgcn_s_memrealtime();
    int64_t* record = stamps + int64_t(blockIdx.x) * kStampWords;
    if (lane == 0 && wave == 0) {
      record[0] = clock0;
      record[1] = clock1;
      record[2] = wall0;
      record[3] = wall1;
    }
    if (lane == 0 && wave == C::WM) {
      record[4 + 2 * kStampKinds] = clock0;
      record[5 + 2 * kStampKinds] = clock1;
    }
    if (lane == 0 && (wave == 0 || wave == C::WM)) {
#pragma unroll
      for (int i = 0; i < kStampKinds; ++i) record[4 + (wave / C::WM) * kStampKinds + i] = phase[i];
    }
  }
}

}  // namespace
}  // namespace ci8
