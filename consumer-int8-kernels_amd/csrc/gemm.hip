// INT8 x INT8 -> INT32 GEMM with the channel-scale epilogue, for gfx950 (CDNA4).
//
//   out[m, n] = bf16_rn( fl( fl( float_rn(acc[m, n]) * sa[m] ) * float(sw[n]) ) )
//   acc[m, n] = sum_k a[m, k] * w[n, k]            (exact INT32)
//
// This is the arithmetic of csrc/fused_mm.cu:24-38 (row scale first, then channel
// scale, then BF16 round-to-nearest) and of csrc/cutlass_mm.cu:30-36, which is also
// the reference test oracle at tests/test_cuda_ops.py:596-600. Biased UINT8 weights
// (csrc/kernels.cu:107) are debiased by an XOR with 0x80 on their way into the MFMA.
//
// Design (MI355X-first, not a translation of the reference's CUTLASS SM80 tiles):
//  * The MFMA computes the transposed tile D[n, m] = W[n, :] . A[m, :] with
//    v_mfma_i32_32x32x32_i8, so each lane ends up with 4 consecutive output columns
//    of one output row and the BF16 epilogue stores 8 bytes per lane.
//  * Both operands are K-contiguous ("TN"). Global -> LDS copies use
//    buffer_load_dwordx4 ... lds (no VGPR staging); rows past M/N and columns past K
//    come back as zeros from the buffer range check, so tails need no branches.
//  * LDS tiles are row-major [rows][BK] with 16-byte chunks XOR-swizzled per row so
//    the ds_read_b128 fragment loads of 16 consecutive rows hit distinct banks.
//  * A multi-stage LDS ring keeps STAGES-1 K-slices in flight behind the MFMAs.
//  * Workgroup ids are remapped so that consecutive tiles of a grouped raster land on
//    the same XCD (the hardware deals workgroups round-robin over the 8 XCDs), which
//    keeps the A and W panels they share in that XCD's L2.
#include <type_traits>
#include <utility>

#include "ci8_device.h"
#include "launch.h"

namespace ci8 {
namespace {

constexpr int kXcds = 8;

template <int BN_, int BM_, int BK_, int WN_, int WM_, int STAGES_, int GROUP_M_>
struct TileConfig {
  static constexpr int BN = BN_;          // W rows (output columns) per workgroup
  static constexpr int BM = BM_;          // A rows (output rows) per workgroup
  static constexpr int BK = BK_;          // K bytes per pipeline stage
  static constexpr int WN = WN_;          // waves along n
  static constexpr int WM = WM_;          // waves along m
  static constexpr int STAGES = STAGES_;  // LDS ring depth
  static constexpr int GROUP_M = GROUP_M_;
  static constexpr int kWaves = WN * WM;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int TN = BN / WN / 32;  // 32x32 MFMA tiles per wave along n
  static constexpr int TM = BM / WM / 32;  // ... along m
  static constexpr int kChunksPerRow = BK / 16;
  static constexpr int kXBytes = BN * BK;  // one stage of the W tile
  static constexpr int kYBytes = BM * BK;  // one stage of the A tile
  static constexpr int kStageBytes = kXBytes + kYBytes;
  static constexpr int kLdsBytes = STAGES * kStageBytes;
  // 1 KiB DMA instructions per wave per stage.
  static constexpr int kXLoads = kXBytes / 1024 / kWaves;
  static constexpr int kYLoads = kYBytes / 1024 / kWaves;
  static constexpr int kLoadsPerStage = kXLoads + kYLoads;
  static_assert(BK == 64 || BK == 128, "BK");
  static_assert(kXLoads * 1024 * kWaves == kXBytes && kYLoads * 1024 * kWaves == kYBytes,
                "stage must split into whole 1 KiB DMA instructions per wave");
  static_assert(TN >= 1 && TM >= 1, "wave tile");
  static_assert(kLdsBytes <= 160 * 1024, "LDS");
};

// 16-byte LDS load (ds_read_b128).
__device__ __forceinline__ i32x4 ld(const char __attribute__((address_space(3)))* p) {
  return *reinterpret_cast<const __attribute__((address_space(3))) i32x4*>(p);
}

// Keeps the instruction scheduler from moving any instruction across this point. The
// epilogues use it to keep every scale load ahead of the first store: stores share the
// vector-memory counter with loads, so a load scheduled after a store makes its wait
// also wait for that store.
__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }

// Chunk slot of logical 16-byte chunk c in LDS row r. A fragment load has 16
// consecutive lanes reading 16 consecutive rows at the same logical chunk; the XOR
// below puts any 8 consecutive rows on distinct 16-byte bank groups of a 128-byte
// window. Measured on gfx950, this makes ds_read_b128 fragment loads as fast as a
// linear 1 KiB read, while leaving them unswizzled or using a 256-byte-window variant
// costs about 12%.
template <class C>
__device__ __forceinline__ int swizzle(int row, int chunk) {
  return chunk ^ ((row / (128 / C::BK)) % C::kChunksPerRow);
}

// Issue this wave's DMA copies of one K-slice of an operand tile (rows x BK) into LDS.
template <class C, int kLoads>
__device__ __forceinline__ void load_tile(__amdgpu_buffer_rsrc_t rsrc, lds_void* lds, int wave,
                                          int lane, int row0, int rows_total, int k0, int k) {
#pragma unroll
  for (int i = 0; i < kLoads; ++i) {
    const int block = i * C::kWaves + wave;  // 1 KiB block of the tile
    const int q = block * 64 + lane;         // chunk index within the tile
    const int row = q / C::kChunksPerRow;
    const int slot = q % C::kChunksPerRow;
    const int chunk = swizzle<C>(row, slot);  // the swizzle is an involution
    const int grow = row0 + row;
    const int gcol = k0 + chunk * 16;
    const uint32_t offset = (grow < rows_total && gcol < k)
                                ? uint32_t(grow) * uint32_t(k) + uint32_t(gcol)
                                : kOutOfRange;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rsrc, reinterpret_cast<lds_void*>(reinterpret_cast<char __attribute__((address_space(3)))*>(lds) + block * 1024),
        16, offset, 0, 0, 0);
  }
}

// K loop of the 32x32 kernel: acc += W[n0:n0+BN, :k] . A[m0:m0+BM, :k]^T (as D[n][m])
// through an STAGES-deep LDS ring. Returns with every vector-memory copy landed; this
// wave's last LDS reads have been consumed by its MFMAs, but other waves may still be
// reading the last stage, so a caller that reuses the ring must barrier first.
template <class C, WeightCode kCode>
__device__ __forceinline__ void gemm_kloop(i32x16 (&acc)[C::TN][C::TM], const int8_t* a,
                                           const void* w,
                                           char __attribute__((address_space(3)))* lds,
                                           int wave, int lane, int wave_n, int wave_m, int m0,
                                           int n0, int m, int n, int k) {
  const auto w_rsrc = make_rsrc(w, uint32_t(n) * uint32_t(k));
  const auto a_rsrc = make_rsrc(a, uint32_t(m) * uint32_t(k));

  const int nk = (k + C::BK - 1) / C::BK;
  auto issue = [&](int kt) {
    auto* stage = lds + (kt % C::STAGES) * C::kStageBytes;
    load_tile<C, C::kXLoads>(w_rsrc, reinterpret_cast<lds_void*>(stage), wave, lane, n0, n,
                             kt * C::BK, k);
    load_tile<C, C::kYLoads>(a_rsrc, reinterpret_cast<lds_void*>(stage + C::kXBytes), wave,
                             lane, m0, m, kt * C::BK, k);
  };
#pragma unroll
  for (int s = 0; s < C::STAGES - 1; ++s)
    if (s < nk) issue(s);

  const int frag_row = lane & 31;
  const int frag_half = lane >> 5;
  const int x_row0 = wave_n * (C::BN / C::WN);
  const int y_row0 = wave_m * (C::BM / C::WM);

  for (int kt = 0; kt < nk; ++kt) {
    // Own copies of stage kt landed; own LDS reads of the previous stage returned.
    if (kt + C::STAGES - 2 < nk)
      __builtin_amdgcn_s_waitcnt(vmcnt_imm((C::STAGES - 2) * C::kLoadsPerStage));
    else
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    __builtin_amdgcn_s_waitcnt(lgkmcnt0_imm());
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (kt + C::STAGES - 1 < nk) issue(kt + C::STAGES - 1);

    const auto* stage = lds + (kt % C::STAGES) * C::kStageBytes;
    const auto* xs = stage;
    const auto* ys = stage + C::kXBytes;
#pragma unroll
    for (int s = 0; s < C::BK / 32; ++s) {
      const int chunk = s * 2 + frag_half;
      i32x4 xf[C::TN], yf[C::TM];
#pragma unroll
      for (int i = 0; i < C::TN; ++i) {
        const int row = x_row0 + i * 32 + frag_row;
        xf[i] = *reinterpret_cast<const __attribute__((address_space(3))) i32x4*>(
            xs + row * C::BK + swizzle<C>(row, chunk) * 16);
        if constexpr (kCode == WeightCode::kBiasedU8) xf[i] ^= int32_t(0x80808080u);
      }
#pragma unroll
      for (int j = 0; j < C::TM; ++j) {
        const int row = y_row0 + j * 32 + frag_row;
        yf[j] = *reinterpret_cast<const __attribute__((address_space(3))) i32x4*>(
            ys + row * C::BK + swizzle<C>(row, chunk) * 16);
      }
#pragma unroll
      for (int i = 0; i < C::TN; ++i)
#pragma unroll
        for (int j = 0; j < C::TM; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(xf[i], yf[j], acc[i][j], 0, 0, 0);
    }
  }

}

template <class C, WeightCode kCode, bool kWorkspace>
__global__ void __launch_bounds__(C::kThreads) channel_gemm_kernel(
    const int8_t* __restrict__ a, const void* __restrict__ w, const float* __restrict__ sa,
    const uint16_t* __restrict__ sw, uint16_t* __restrict__ out, int32_t* __restrict__ ws,
    int m, int n, int k, bool vec_n) {
  extern __shared__ __attribute__((aligned(1024))) char lds_raw[];
  auto* lds = (char __attribute__((address_space(3)))*)(lds_raw);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (SGPR)
  const int wave_n = wave / C::WM;
  const int wave_m = wave % C::WM;

  // Workgroup -> tile: undo the round-robin XCD dealing, then a grouped raster.
  const int tiles_n = (n + C::BN - 1) / C::BN;
  const int tiles_m = (m + C::BM - 1) / C::BM;
  const int blocks = tiles_n * tiles_m;
  int logical = blockIdx.x;
  {
    const int per = blocks / kXcds, extra = blocks % kXcds;
    const int xcd = logical % kXcds, idx = logical / kXcds;
    logical = (xcd < extra ? xcd * (per + 1) : extra * (per + 1) + (xcd - extra) * per) + idx;
  }
  const int group_span = C::GROUP_M * tiles_n;
  const int first_m = (logical / group_span) * C::GROUP_M;
  const int group_rows = min(tiles_m - first_m, C::GROUP_M);
  const int tile_m = first_m + (logical % group_span) % group_rows;
  const int tile_n = (logical % group_span) / group_rows;
  const int n0 = tile_n * C::BN, m0 = tile_m * C::BM;

  i32x16 acc[C::TN][C::TM];
#pragma unroll
  for (int i = 0; i < C::TN; ++i)
#pragma unroll
    for (int j = 0; j < C::TM; ++j) acc[i][j] = i32x16{};
  gemm_kloop<C, kCode>(acc, a, w, lds, wave, lane, wave_n, wave_m, m0, n0, m, n, k);

  // Per-lane fragment geometry: MFMA row/col = lane % 32, K half = lane / 32.
  const int frag_row = lane & 31;
  const int frag_half = lane >> 5;
  const int x_row0 = wave_n * (C::BN / C::WN);
  const int y_row0 = wave_m * (C::BM / C::WM);

  // Epilogue. Lane holds D[n][m] for m = lane % 32 and n = 8*r4 + 4*(lane/32) + e.
  // vec_n: n % 4 == 0 and sw, out (and ws) aligned for 8-byte (16-byte) accesses.
  // All scale loads precede the first store (stores share the vector-memory counter).
  float row_scale[C::TM];
#pragma unroll
  for (int j = 0; j < C::TM; ++j) {
    const int row = m0 + y_row0 + j * 32 + frag_row;
    row_scale[j] = row < m ? sa[row] : 0.f;
  }
  if (vec_n && m0 + C::BM <= m && n0 + C::BN <= n) {
    // Whole block tile in bounds (block-uniform test): unguarded stores after one wait.
    u32x2 s2[C::TN][4];
#pragma unroll
    for (int i = 0; i < C::TN; ++i)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4)
        s2[i][r4] = *reinterpret_cast<const u32x2*>(
            sw + n0 + x_row0 + i * 32 + r4 * 8 + frag_half * 4);
    sched_fence();
#pragma unroll
    for (int j = 0; j < C::TM; ++j) {
      const int64_t row_base =
          int64_t(m0 + y_row0 + j * 32 + frag_row) * n + n0 + x_row0 + frag_half * 4;
#pragma unroll
      for (int i = 0; i < C::TN; ++i) {
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const int64_t base = row_base + i * 32 + r4 * 8;
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t sbits = (s2[i][r4][e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
            v[e] = (float(acc[i][j][r4 * 4 + e]) * row_scale[j]) * bf16_to_f32(sbits);
          }
          *reinterpret_cast<u32x2*>(out + base) = u32x2{pack_bf16x2(v[0], v[1]),
                                                         pack_bf16x2(v[2], v[3])};
          if constexpr (kWorkspace)
            *reinterpret_cast<i32x4*>(ws + base) =
                i32x4{acc[i][j][r4 * 4 + 0], acc[i][j][r4 * 4 + 1], acc[i][j][r4 * 4 + 2],
                      acc[i][j][r4 * 4 + 3]};
        }
      }
    }
  } else if (vec_n) {
    u32x2 s2[C::TN][4];
#pragma unroll
    for (int i = 0; i < C::TN; ++i)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int col = n0 + x_row0 + i * 32 + r4 * 8 + frag_half * 4;
        s2[i][r4] = col < n ? *reinterpret_cast<const u32x2*>(sw + col) : u32x2{0, 0};
      }
    sched_fence();
#pragma unroll
    for (int j = 0; j < C::TM; ++j) {
      const int row = m0 + y_row0 + j * 32 + frag_row;  // output row (m)
      if (row >= m) continue;
#pragma unroll
      for (int i = 0; i < C::TN; ++i) {
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const int col = n0 + x_row0 + i * 32 + r4 * 8 + frag_half * 4;  // output column (n)
          if (col >= n) continue;
          const int64_t base = int64_t(row) * n + col;
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t sbits = (s2[i][r4][e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
            v[e] = (float(acc[i][j][r4 * 4 + e]) * row_scale[j]) * bf16_to_f32(sbits);
          }
          *reinterpret_cast<u32x2*>(out + base) = u32x2{pack_bf16x2(v[0], v[1]),
                                                         pack_bf16x2(v[2], v[3])};
          if constexpr (kWorkspace)
            *reinterpret_cast<i32x4*>(ws + base) =
                i32x4{acc[i][j][r4 * 4 + 0], acc[i][j][r4 * 4 + 1], acc[i][j][r4 * 4 + 2],
                      acc[i][j][r4 * 4 + 3]};
        }
      }
    }
  } else {
    // Element stores, column group by column group (scales loaded before its stores).
#pragma unroll
    for (int i = 0; i < C::TN; ++i)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int col = n0 + x_row0 + i * 32 + r4 * 8 + frag_half * 4;
        float sc[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) sc[e] = col + e < n ? bf16_to_f32(sw[col + e]) : 0.f;
#pragma unroll
        for (int j = 0; j < C::TM; ++j) {
          const int row = m0 + y_row0 + j * 32 + frag_row;
          if (row >= m) continue;
          const int64_t base = int64_t(row) * n + col;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (col + e < n) {
              out[base + e] =
                  uint16_t(f32_to_bf16((float(acc[i][j][r4 * 4 + e]) * row_scale[j]) * sc[e]));
              if constexpr (kWorkspace) ws[base + e] = acc[i][j][r4 * 4 + e];
            }
          }
        }
      }
  }
}

template <class C, WeightCode kCode, bool kWorkspace>
hipError_t run(const int8_t* a, const void* w, const float* sa, const void* sw, void* out,
               int32_t* ws, int m, int n, int k, hipStream_t stream) {
  auto kernel = channel_gemm_kernel<C, kCode, kWorkspace>;
  if (const hipError_t e = prepare_lds<channel_gemm_kernel<C, kCode, kWorkspace>>(C::kLdsBytes); e != hipSuccess)
    return e;
  const int blocks = ((n + C::BN - 1) / C::BN) * ((m + C::BM - 1) / C::BM);
  const bool vec_n = n % 4 == 0 && reinterpret_cast<uintptr_t>(sw) % 8 == 0 &&
                     reinterpret_cast<uintptr_t>(out) % 8 == 0 &&
                     reinterpret_cast<uintptr_t>(ws) % 16 == 0;
  kernel<<<blocks, C::kThreads, C::kLdsBytes, stream>>>(
      a, w, sa, static_cast<const uint16_t*>(sw), static_cast<uint16_t*>(out), ws, m, n, k,
      vec_n);
  return hipGetLastError();
}

// Epilogue for accumulators in the 16x16 MFMA layout: lane holds D[n][m] for
// m = lane % 16 and n = 4 * (lane / 16) + e of each block. All scale loads are issued
// before the first store: on gfx9 stores share the vector-memory counter with loads, so
// a load issued after a store cannot be waited for without also waiting for the store.
template <int TM, int TN, bool kWorkspace>
__device__ __forceinline__ void store_tile16(const i32x4 (&acc)[TM][TN], int row0, int col0,
                                             int m, int n, const float* __restrict__ sa,
                                             const uint16_t* __restrict__ sw,
                                             uint16_t* __restrict__ out, int32_t* __restrict__ ws,
                                             bool vec_n) {
  const int lane = threadIdx.x & 63;
  const int frag_row = lane & 15, frag_group = lane >> 4;
  float row_scale[TM];
#pragma unroll
  for (int j = 0; j < TM; ++j) {
    const int row = row0 + j * 16 + frag_row;
    row_scale[j] = row < m ? sa[row] : 0.f;
  }
  if (vec_n && row0 + TM * 16 <= m && col0 + TN * 16 <= n) {
    // Whole wave tile in bounds (wave-uniform test): no per-element guards, so the
    // stores are issued back to back after a single wait for the scale loads.
    u32x2 s2[TN];
#pragma unroll
    for (int i = 0; i < TN; ++i)
      s2[i] = *reinterpret_cast<const u32x2*>(sw + col0 + i * 16 + frag_group * 4);
    sched_fence();
#pragma unroll
    for (int j = 0; j < TM; ++j) {
      const int64_t row_base = int64_t(row0 + j * 16 + frag_row) * n + col0 + frag_group * 4;
#pragma unroll
      for (int i = 0; i < TN; ++i) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t sbits = (s2[i][e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
          v[e] = (float(acc[j][i][e]) * row_scale[j]) * bf16_to_f32(sbits);
        }
        *reinterpret_cast<u32x2*>(out + row_base + i * 16) =
            u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        if constexpr (kWorkspace) *reinterpret_cast<i32x4*>(ws + row_base + i * 16) = acc[j][i];
      }
    }
  } else if (vec_n) {
    u32x2 s2[TN];
#pragma unroll
    for (int i = 0; i < TN; ++i) {
      const int col = col0 + i * 16 + frag_group * 4;
      s2[i] = col < n ? *reinterpret_cast<const u32x2*>(sw + col) : u32x2{0, 0};
    }
    sched_fence();
#pragma unroll
    for (int j = 0; j < TM; ++j) {
      const int row = row0 + j * 16 + frag_row;
      if (row >= m) continue;
#pragma unroll
      for (int i = 0; i < TN; ++i) {
        const int col = col0 + i * 16 + frag_group * 4;
        if (col >= n) continue;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t sbits = (s2[i][e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
          v[e] = (float(acc[j][i][e]) * row_scale[j]) * bf16_to_f32(sbits);
        }
        const int64_t base = int64_t(row) * n + col;
        *reinterpret_cast<u32x2*>(out + base) =
            u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        if constexpr (kWorkspace) *reinterpret_cast<i32x4*>(ws + base) = acc[j][i];
      }
    }
  } else {
    // Unaligned or n % 4 != 0 (channel_mm accepts any n): element stores, column block
    // by column block, each block's four scales loaded before its stores.
#pragma unroll
    for (int i = 0; i < TN; ++i) {
      const int col = col0 + i * 16 + frag_group * 4;
      float sc[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) sc[e] = col + e < n ? bf16_to_f32(sw[col + e]) : 0.f;
#pragma unroll
      for (int j = 0; j < TM; ++j) {
        const int row = row0 + j * 16 + frag_row;
        if (row >= m) continue;
        const int64_t base = int64_t(row) * n + col;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (col + e < n) {
            out[base + e] = uint16_t(f32_to_bf16((float(acc[j][i][e]) * row_scale[j]) * sc[e]));
            if constexpr (kWorkspace) ws[base + e] = acc[j][i][e];
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------
// Pipelined large-tile kernel (v_mfma_i32_16x16x64_i8), K staged 128 bytes at a time.
//
// Tile 256(m) x 224(n) per workgroup; four waves (one per SIMD) each own 128 x 112 as
// 8 x 7 16x16 INT32 accumulators (224 AGPRs). 256 x 224 suits wave quantization on 256
// CUs: N = 17408 gives 78 n-tiles and M = 4096 gives 16, 1248 tiles = 4.875 rounds
// (97.5% busy), where 256 x 256 gives 1088 tiles = 4.25 rounds (85%).
//
// Feeding: the L2 -> CU path on gfx950 delivers far more when each row segment is a
// full 128-byte line (measured about 14 TB/s aggregate for 64-byte segments through
// buffer_load ... lds, 22 TB/s for 128-byte ones), and a 256 x 224 tile at the MFMA
// rate needs about 17 TB/s. So a stage holds 128 bytes of K per row (60 KB for both
// operands) and two stages fit in LDS. A stage is two K-steps of one 16x16x64 MFMA
// each (56 MFMAs per wave per step). For stage t:
//   step A (K-step 2t):   MFMAs from registers; read the fragments of K-step 2t+1
//                         from slot t%2;
//   barrier:              own copies of stage t+1 landed and own reads of slot t%2
//                         returned (both checked before the barrier), so after it
//                         stage t+1 is visible and slot t%2 is free;
//   step B (K-step 2t+1): issue the copies of stage t+2 into slot t%2, MFMAs from
//                         registers, read the fragments of K-step 2t+2 (stage t+1).
// Stage t+2's copies therefore have two K-steps (about 1800 MFMA cycles) to land.
// W fragments are double-buffered in registers; A fragments 0..5 are reloaded in place
// after their last MFMA, and A fragments 6..7 alternate with a spare pair loaded early,
// so the last LDS read of step A is issued two MFMA groups before the barrier.
template <int BM_, int BN_, int WM_, int WN_, int GROUP_M_>
struct K128Config {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, GROUP_M = GROUP_M_;
  static constexpr int BK = 128;  // K bytes per stage (two 64-deep MFMA steps)
  static constexpr int kWaves = WM * WN;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int TM = BM / WM / 16;  // 16-row m blocks per wave
  static constexpr int TN = BN / WN / 16;  // 16-row n blocks per wave
  static constexpr int kSpare = 2;         // A fragments with a spare register pair
  static constexpr int kChunksPerRow = BK / 16;
  static constexpr int kXBytes = BN * BK;
  static constexpr int kYBytes = BM * BK;
  static constexpr int kStageBytes = kXBytes + kYBytes;
  static constexpr int kXBlocks = kXBytes / 1024;
  static constexpr int kBlocks = kStageBytes / 1024;
  static constexpr int kLoads = (kBlocks + kWaves - 1) / kWaves;  // DMA per wave per stage
  static constexpr int kJunkOffset = 2 * kStageBytes;  // target of padding DMA, if any
  static constexpr int kLdsBytes = kJunkOffset + (kLoads * kWaves > kBlocks ? 1024 : 0);
  static_assert(kXBytes % 1024 == 0 && kYBytes % 1024 == 0, "whole 1 KiB blocks");
  static_assert(TM * 16 * WM == BM && TN * 16 * WN == BN, "wave tiling");
  static_assert(TM > kSpare, "spare A fragments");
  static_assert(kLdsBytes <= 160 * 1024, "LDS");
};

// Wrappers for the target builtins used by the pipelined kernel. Its helper lambdas
// call these rather than the builtins themselves: a builtin written directly inside a
// lambda makes the host compilation pass drop the kernel's launch stub.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, lds_void* dst, uint32_t voffset,
                                      int soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, dst, 16, voffset, soffset, 0, 0);
}
__device__ __forceinline__ u32x4 buffer_load16(__amdgpu_buffer_rsrc_t rsrc, uint32_t voffset,
                                               int soffset) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, voffset, soffset, 0));
}
// XOR `mask` into the 16 bytes at LDS byte address `addr + kOff`.
template <int kOff>
__device__ __forceinline__ void xor_16(uint32_t addr, uint64_t mask) {
  static_assert(kOff >= 0 && kOff + 8 < 65536, "ds offset field");
  asm volatile("ds_xor_b64 %0, %1 offset:%2\n\tds_xor_b64 %0, %1 offset:%3"
               :
               : "v"(addr), "v"(mask), "i"(kOff), "i"(kOff + 8)
               : "memory");
}
// XOR 0x80 into every byte of the 16 bytes at LDS byte address
// wave_base + 16 * lane + i * kStride, for each i in the sequence. The lane address and
// the mask are made here, by volatile assembly the compiler cannot hoist, so that in a
// loop they hold VGPRs only for these few instructions.
template <int kStride, int... I>
__device__ __forceinline__ void xor80_blocks(uint32_t wave_base, std::integer_sequence<int, I...>) {
  uint32_t addr;
  uint64_t mask;
  asm volatile(
      "v_mbcnt_lo_u32_b32 %0, -1, 0\n\t"
      "v_mbcnt_hi_u32_b32 %0, -1, %0\n\t"
      "v_lshl_add_u32 %0, %0, 4, %1"
      : "=v"(addr)
      : "s"(wave_base));
  asm volatile("v_mov_b64 %0, %1" : "=v"(mask) : "s"(0x8080808080808080ull));
  (xor_16<I * kStride>(addr, mask), ...);
}
// ds_write_b128 of v to LDS byte address addr + kOff. Inline assembly, for the same
// reason as the XORs above: the compiler orders a plain LDS store after every
// outstanding LDS copy.
template <int kOff>
__device__ __forceinline__ void ds_write16(uint32_t addr, u32x4 v) {
  static_assert(kOff >= 0 && kOff < 65536, "ds offset field");
  asm volatile("ds_write_b128 %0, %1 offset:%2" : : "v"(addr), "v"(v), "i"(kOff) : "memory");
}
// v[i] to addr + i * kStride for each i in the sequence.
template <int kStride, int... I>
__device__ __forceinline__ void ds_write_blocks(uint32_t addr, const u32x4* v,
                                                std::integer_sequence<int, I...>) {
  (ds_write16<I * kStride>(addr, v[I]), ...);
}
template <int kImm>
__device__ __forceinline__ void waitcnt() {
  __builtin_amdgcn_s_waitcnt(kImm);
}
__device__ __forceinline__ void workgroup_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
__device__ __forceinline__ i32x4 mfma16(i32x4 a, i32x4 b, i32x4 c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}
template <int kMask, int kSize>
__device__ __forceinline__ void sched_group() {
  __builtin_amdgcn_sched_group_barrier(kMask, kSize, 0);
}

// Scheduling-group barriers that place the in-place reload of A fragment J (J < kLast)
// after the last MFMA reading it, MFMA (J+1)*TN - 1; P MFMAs are already placed.
template <int J, int kLast, int TM, int TN, int P>
struct AReloads {
  static __device__ __forceinline__ void run() {
    if constexpr (J < kLast) {
      constexpr int end = (J + 1) * TN;
      if constexpr (end > P) sched_group<0x008, end - P>();
      sched_group<0x100, 1>();
      AReloads<J + 1, kLast, TM, TN, (end > P ? end : P)>::run();
    } else if constexpr (TM * TN > P) {
      sched_group<0x008, TM * TN - P>();
    }
  }
};

template <class C, WeightCode kCode, bool kWorkspace, bool kExactK>
__global__ void __launch_bounds__(C::kThreads, 1) channel_gemm_k128_kernel(
    const int8_t* __restrict__ a, const void* __restrict__ w, const float* __restrict__ sa,
    const uint16_t* __restrict__ sw, uint16_t* __restrict__ out, int32_t* __restrict__ ws,
    int m, int n, int k, bool vec_n) {
  extern __shared__ __attribute__((aligned(1024))) char lds_raw[];
  auto* lds = (char __attribute__((address_space(3)))*)(lds_raw);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (SGPR)
  const int wave_m = wave % C::WM;
  const int wave_n = wave / C::WM;

  const int tiles_n = (n + C::BN - 1) / C::BN;
  const int tiles_m = (m + C::BM - 1) / C::BM;
  const int blocks = tiles_n * tiles_m;
  int logical = blockIdx.x;
  {
    const int per = blocks / kXcds, extra = blocks % kXcds;
    const int xcd = logical % kXcds, idx = logical / kXcds;
    logical = (xcd < extra ? xcd * (per + 1) : extra * (per + 1) + (xcd - extra) * per) + idx;
  }
  const int group_span = C::GROUP_M * tiles_n;
  const int first_m = (logical / group_span) * C::GROUP_M;
  const int group_rows = min(tiles_m - first_m, C::GROUP_M);
  const int tile_m = first_m + (logical % group_span) % group_rows;
  const int tile_n = (logical % group_span) / group_rows;
  const int n0 = tile_n * C::BN, m0 = tile_m * C::BM;

  const auto w_rsrc = make_rsrc(w, uint32_t(n) * uint32_t(k));
  const auto a_rsrc = make_rsrc(a, uint32_t(m) * uint32_t(k));

  // Per-lane DMA sources for this wave's kLoads 1 KiB blocks of a stage: blocks
  // [0, kXBlocks) are W rows, then A rows, then padding (out-of-range source into a
  // scratch KiB). The stage's K offset goes in the scalar soffset.
  uint32_t dma_base[C::kLoads];
  int dma_col[C::kLoads];
#pragma unroll
  for (int i = 0; i < C::kLoads; ++i) {
    const int block = i * C::kWaves + wave;
    const bool is_w = block < C::kXBlocks;
    const int local = is_w ? block : block - C::kXBlocks;
    const int q = local * 64 + lane;
    const int row = q / C::kChunksPerRow;
    const int chunk = swizzle<C>(row, q % C::kChunksPerRow);  // the swizzle is an involution
    const int grow = (is_w ? n0 : m0) + row;
    const bool valid = block < C::kBlocks && grow < (is_w ? n : m);
    dma_col[i] = chunk * 16;
    dma_base[i] = valid ? uint32_t(grow) * uint32_t(k) + uint32_t(chunk * 16) : kOutOfRange;
  }
#define CI8_DMA_RSRC(i) ((i) * C::kWaves + wave < C::kXBlocks ? w_rsrc : a_rsrc)
  auto dma_dst = [&] __device__(int i, int slot) __attribute__((always_inline)) {
    const int block = i * C::kWaves + wave;
    return reinterpret_cast<lds_void*>(
        lds + (block < C::kBlocks ? slot * C::kStageBytes + block * 1024 : C::kJunkOffset));
  };
  const int ns = (k + C::BK - 1) / C::BK;  // stages
  // Copies of stage t into slot t % 2. Stages past the end re-read stage 0 into a slot
  // nobody reads again (keeps the steady loop branch-free).
  auto issue = [&] __device__(int t) __attribute__((always_inline)) {
    const int slot = t & 1;
    const int st = t < ns ? t : 0;
    if constexpr (kExactK) {
#pragma unroll
      for (int i = 0; i < C::kLoads; ++i)
        dma16(CI8_DMA_RSRC(i), dma_dst(i, slot), dma_base[i], st * C::BK);
    } else {
      const int k0 = st * C::BK;
#pragma unroll
      for (int i = 0; i < C::kLoads; ++i) {
        const bool live = dma_base[i] != kOutOfRange && k0 + dma_col[i] < k;
        dma16(CI8_DMA_RSRC(i), dma_dst(i, slot), live ? dma_base[i] + uint32_t(k0) : kOutOfRange,
              0);
      }
    }
  };

  // Fragment addresses. A lane reads row (lane % 16) of each 16-row block at logical
  // chunk 4*h + lane/16 for K-step half h; row % 8 == lane % 8 for every block, so the
  // swizzled chunk depends on the lane only and each half has one base offset.
  const int frag_row = lane & 15;
  const int frag_chunk = lane >> 4;
  int x_base[2], y_base[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int xrow = wave_n * (C::BN / C::WN) + frag_row;
    const int yrow = wave_m * (C::BM / C::WM) + frag_row;
    x_base[h] = xrow * C::BK + swizzle<C>(xrow, 4 * h + frag_chunk) * 16;
    y_base[h] = C::kXBytes + yrow * C::BK + swizzle<C>(yrow, 4 * h + frag_chunk) * 16;
  }
  auto xaddr = [&] __device__(int slot, int h, int i) __attribute__((always_inline)) {
    return lds + slot * C::kStageBytes + x_base[h] + i * 16 * C::BK;
  };
  auto yaddr = [&] __device__(int slot, int h, int j) __attribute__((always_inline)) {
    return lds + slot * C::kStageBytes + y_base[h] + j * 16 * C::BK;
  };

  i32x4 acc[C::TM][C::TN];
#pragma unroll
  for (int j = 0; j < C::TM; ++j)
#pragma unroll
    for (int i = 0; i < C::TN; ++i) acc[j][i] = i32x4{0, 0, 0, 0};

  // Register sets: xf[0] / yf[0..TM-1] hold the fragments of even K-steps (step A),
  // xf[1] / yf[0..TM-kSpare-1] + ysp[*] those of odd K-steps (step B).
  constexpr int kMain = C::TM - C::kSpare;
  i32x4 xf[2][C::TN], yf[C::TM], ysp[C::kSpare];
  auto debias = [&] __device__(int buf) __attribute__((always_inline)) {
    if constexpr (kCode == WeightCode::kBiasedU8) {
#pragma unroll
      for (int i = 0; i < C::TN; ++i) xf[buf][i] ^= int32_t(0x80808080u);
    }
  };
  // Step A: MFMAs of an even K-step; loads the odd K-step (half 1 of `slot`).
  auto step_a = [&] __device__(int slot) __attribute__((always_inline)) {
    debias(0);
#pragma unroll
    for (int i = 0; i < C::TN; ++i) xf[1][i] = ld(xaddr(slot, 1, i));
#pragma unroll
    for (int s2 = 0; s2 < C::kSpare; ++s2) ysp[s2] = ld(yaddr(slot, 1, kMain + s2));
#pragma unroll
    for (int j = 0; j < C::TM; ++j) {
#pragma unroll
      for (int i = 0; i < C::TN; ++i) acc[j][i] = mfma16(xf[0][i], yf[j], acc[j][i]);
      if (j < kMain) yf[j] = ld(yaddr(slot, 1, j));
    }
#pragma unroll
    for (int i = 0; i < C::TN; ++i) {
      sched_group<0x008, 1>();  // MFMA
      sched_group<0x100, 1>();  // DS read (W fragment)
    }
#pragma unroll
    for (int s2 = 0; s2 < C::kSpare; ++s2) {
      sched_group<0x008, 1>();
      sched_group<0x100, 1>();  // DS read (spare A fragment)
    }
    AReloads<0, kMain, C::TM, C::TN, C::TN + C::kSpare>::run();
  };
  // Step B: copies of stage t+2, MFMAs of the odd K-step; loads the next even K-step
  // (half 0 of `next_slot`).
  auto step_b = [&] __device__(int t, int next_slot) __attribute__((always_inline)) {
    issue(t + 2);
    debias(1);
#pragma unroll
    for (int i = 0; i < C::TN; ++i) xf[0][i] = ld(xaddr(next_slot, 0, i));
#pragma unroll
    for (int s2 = 0; s2 < C::kSpare; ++s2) yf[kMain + s2] = ld(yaddr(next_slot, 0, kMain + s2));
#pragma unroll
    for (int j = 0; j < C::TM; ++j) {
#pragma unroll
      for (int i = 0; i < C::TN; ++i)
        acc[j][i] = mfma16(xf[1][i], j < kMain ? yf[j] : ysp[j - kMain], acc[j][i]);
      if (j < kMain) yf[j] = ld(yaddr(next_slot, 0, j));
    }
#pragma unroll
    for (int i = 0; i < C::kLoads; ++i) {
      sched_group<0x008, 1>();  // MFMA
      sched_group<0x010, 1>();  // VMEM (LDS DMA)
    }
#pragma unroll
    for (int i = 0; i < C::TN + C::kSpare; ++i) {
      sched_group<0x008, 1>();
      sched_group<0x100, 1>();  // DS read (W fragment, then A fragments 6..7)
    }
    AReloads<0, kMain, C::TM, C::TN, C::kLoads + C::TN + C::kSpare>::run();
  };
  // Between A and B: own copies of stage t+1 landed, own reads of slot t%2 returned.
  auto sync = [&] __device__() __attribute__((always_inline)) {
    waitcnt<vmcnt_imm(0)>();
    waitcnt<lgkmcnt0_imm()>();
    workgroup_barrier();
  };

  issue(0);
  issue(1);
  waitcnt<vmcnt_imm(C::kLoads)>();  // stage 0 landed (stage 1 may be in flight)
  workgroup_barrier();
#pragma unroll
  for (int i = 0; i < C::TN; ++i) xf[0][i] = ld(xaddr(0, 0, i));
#pragma unroll
  for (int j = 0; j < C::TM; ++j) yf[j] = ld(yaddr(0, 0, j));

  for (int t = 0; t < ns; ++t) {
    const int slot = t & 1;
    step_a(slot);
    sync();
    step_b(t, slot ^ 1);
  }
  waitcnt<vmcnt_imm(0)>();  // padding copies of the last two steps
#undef CI8_DMA_RSRC

  store_tile16<C::TM, C::TN, kWorkspace>(acc, m0 + wave_m * (C::BM / C::WM),
                                        n0 + wave_n * (C::BN / C::WN), m, n, sa, sw, out, ws,
                                        vec_n);
}

// ---------------------------------------------------------------------------------
// Large-tile kernel with W staged in a shared LDS ring and A private to each wave.
//
// Tile 256(m) x 224(n) (or 256-wide); the four waves are stacked along m, each owning
// 64 rows x 224 columns as 4 x 14 16x16 INT32 accumulators (224 AGPRs). The 224 W rows,
// used by all four waves, go through an LDS ring filled by buffer_load ... lds. With only
// W in LDS a stage of 128 K-bytes is 28 KB, so a ring of four slots keeps three stages in
// flight. A wave's A rows are private to it; the A loads of the next two stages are in
// flight in two more register sets (three sets in all). Measured with per-wave clocks on
// MI355X, the main loop is limited by the vector-memory address unit (TA), and A is
// the costly stream: loaded straight into MFMA operand registers, each load touches 16
// rows x 64 bytes, which the unit serves at ~16 B/clk per CU, against ~26 B/clk for 8
// rows x 128 bytes and ~55 B/clk for the W copies. So with the 224-wide tile and K a
// whole number of stages, A takes a detour (kABounce): 8-row x 128-byte loads into
// staging registers, then the wave's own 8 KiB LDS buffer, then fragment reads in the
// operand layout. That is 4% faster at configs[2]; the 256-wide tile has no LDS left for
// the buffers and loads A straight into the operand registers.
//
// K order: within a 128-byte stage, MFMA lane group g (lane / 16) takes physical chunk
// 2g + h in K-step h (0 or 1). A and W use the same order, so the dot products are
// unchanged, and each lane's two 16-byte direct A loads per block cover a whole
// 128-byte line of its row.
//
// For stage t (K-steps h = 0, 1), each wave:
//   h = 0: issue the A loads of stage t+2 (into the set stage t-1 used); 56 MFMAs;
//          reload each W fragment for K-step (t, 1) right after its last MFMA (bounce:
//          and read the A fragments of K-step (t, 1) from the buffer);
//   sync:  own W copies (bounce: and A loads) of stage t+1 landed, then a barrier (all
//          waves' copies landed; every wave finished K-step (t, 0), so nobody reads the
//          slot of stage t-1); bounce: write A of stage t+1 to the buffer, after the
//          reads of stage t's fragments in program order;
//   h = 1: issue the W copies of stage t+3 into the slot of stage t-1; 56 MFMAs;
//          reload the W fragments (bounce: and read the A fragments) for K-step (t+1, 0).
template <int BN_, int GROUP_M_, bool kABounce_>
struct WLdsConfig {
  static constexpr int BM = 256, BN = BN_, GROUP_M = GROUP_M_;
  static constexpr bool kABounce = kABounce_;  // A through a per-wave LDS buffer
  static constexpr int BK = 128;        // K bytes per stage (two 64-deep MFMA steps)
  static constexpr int kWaves = 4;      // stacked along m
  static constexpr int kThreads = 256;
  static constexpr int TM = BM / kWaves / 16;  // 16-row m blocks per wave (4)
  static constexpr int TN = BN / 16;           // 16-row n blocks per wave
  static constexpr int kSlots = 4;             // W ring (a power of two: cheap slot math)
  static constexpr int kAhead = kSlots - 1;    // W stages in flight
  static constexpr int kChunksPerRow = BK / 16;
  static constexpr int kStageBytes = BN * BK;
  static constexpr int kBlocks = kStageBytes / 1024;
  static constexpr int kLoads = kBlocks / kWaves;  // W DMA per wave per stage
  static constexpr int kRingBytes = kSlots * kStageBytes;
  // Epilogue staging, reusing the ring: each wave's 64 x BN BF16 outputs at a row stride
  // of BN*2 + 16 bytes (116 dwords for BN = 224: 116 = 4 x odd mod 64, so the 16 rows a
  // ds_write_b64 covers start in distinct banks).
  static constexpr int kEpiRowBytes = BN * 2 + 16;
  static constexpr int kEpiWaveBytes = (BM / kWaves) * kEpiRowBytes;
  // A bounce buffers: one per wave, its 64 rows x 128 bytes of a stage, after the ring.
  static constexpr int kABytes = (BM / kWaves) * BK;
  static constexpr int kABase = kRingBytes;
  static constexpr int kMainBytes = kRingBytes + (kABounce ? kWaves * kABytes : 0);
  static constexpr int kLdsBytes =
      kMainBytes > kWaves * kEpiWaveBytes ? kMainBytes : kWaves * kEpiWaveBytes;
  static constexpr int kALoads = kABounce ? BM / kWaves / 8 : 2 * TM;  // A loads per stage
  static_assert(kLoads * kWaves == kBlocks, "whole 1 KiB W blocks per wave");
  static_assert((BN * 2) % 16 == 0, "whole 16-byte output chunks per row");
  static_assert(TM * 16 * kWaves == BM && TN * 16 == BN, "wave tiling");
  static_assert(kLdsBytes <= 160 * 1024, "LDS");
};

// Epilogue of one wave's in-bounds 64 x BN tile through LDS. The scale arithmetic and
// rounding are those of store_tile16; the BF16 results go to the wave's LDS region in
// the MFMA layout (8 bytes per lane and block) and come back as 16-byte row chunks, so
// each global store instruction writes whole 128-byte lines (consecutive lanes along a
// row) instead of 16 rows x 32 bytes. Requires n % 8 == 0 and a 16-byte aligned out.
template <class C>
__device__ __forceinline__ void store_tile16_lds(const i32x4 (&acc)[C::TM][C::TN],
                                                 char __attribute__((address_space(3)))* region,
                                                 int row0, int col0, int n,
                                                 const float* __restrict__ sa,
                                                 const uint16_t* __restrict__ sw,
                                                 uint16_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int frag_row = lane & 15, frag_group = lane >> 4;
  float row_scale[C::TM];
#pragma unroll
  for (int j = 0; j < C::TM; ++j) row_scale[j] = sa[row0 + j * 16 + frag_row];
  u32x2 s2[C::TN];
#pragma unroll
  for (int i = 0; i < C::TN; ++i)
    s2[i] = *reinterpret_cast<const u32x2*>(sw + col0 + i * 16 + frag_group * 4);
#pragma unroll
  for (int j = 0; j < C::TM; ++j) {
    auto* row_base = region + (j * 16 + frag_row) * C::kEpiRowBytes + frag_group * 8;
#pragma unroll
    for (int i = 0; i < C::TN; ++i) {
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t sbits = (s2[i][e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
        v[e] = (float(acc[j][i][e]) * row_scale[j]) * bf16_to_f32(sbits);
      }
      *reinterpret_cast<__attribute__((address_space(3))) u32x2*>(row_base + i * 32) =
          u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    }
  }
  // One wave's LDS operations complete in order; the wait only orders the reads after
  // every lane's writes for the compiler.
  __builtin_amdgcn_s_waitcnt(lgkmcnt0_imm());
  __builtin_amdgcn_wave_barrier();
  constexpr int kChunks = C::BN / 8;  // 16-byte chunks per output row
  constexpr int kRows = C::BM / C::kWaves;
#pragma unroll
  for (int it = 0; it < kRows * kChunks / 64; ++it) {
    const int q = it * 64 + lane;
    const int row = q / kChunks, chunk = q % kChunks;
    const u32x4 v = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(
        region + row * C::kEpiRowBytes + chunk * 16);
    *reinterpret_cast<u32x4*>(out + int64_t(row0 + row) * n + col0 + chunk * 8) = v;
  }
}

template <class C, WeightCode kCode, bool kWorkspace, bool kExactK>
__global__ void __launch_bounds__(C::kThreads, 1) channel_gemm_wlds_kernel(
    const int8_t* __restrict__ a, const void* __restrict__ w, const float* __restrict__ sa,
    const uint16_t* __restrict__ sw, uint16_t* __restrict__ out, int32_t* __restrict__ ws,
    int m, int n, int k, bool vec_n) {
  extern __shared__ __attribute__((aligned(1024))) char lds_raw[];
  auto* lds = (char __attribute__((address_space(3)))*)(lds_raw);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (SGPR)

  const int tiles_n = (n + C::BN - 1) / C::BN;
  const int tiles_m = (m + C::BM - 1) / C::BM;
  const int blocks = tiles_n * tiles_m;
  int logical = blockIdx.x;
  {
    const int per = blocks / kXcds, extra = blocks % kXcds;
    const int xcd = logical % kXcds, idx = logical / kXcds;
    logical = (xcd < extra ? xcd * (per + 1) : extra * (per + 1) + (xcd - extra) * per) + idx;
  }
  const int group_span = C::GROUP_M * tiles_n;
  const int first_m = (logical / group_span) * C::GROUP_M;
  const int group_rows = min(tiles_m - first_m, C::GROUP_M);
  const int tile_m = first_m + (logical % group_span) % group_rows;
  const int tile_n = (logical % group_span) / group_rows;
  const int n0 = tile_n * C::BN, m0 = tile_m * C::BM;

  const auto w_rsrc = make_rsrc(w, uint32_t(n) * uint32_t(k));
  const auto a_rsrc = make_rsrc(a, uint32_t(m) * uint32_t(k));
  const int ns = (k + C::BK - 1) / C::BK;  // stages

  // W copies: this wave's kLoads 1 KiB blocks of a stage (8 rows x 128 bytes each).
  uint32_t dma_base[C::kLoads];
  int dma_col[C::kLoads];
#pragma unroll
  for (int i = 0; i < C::kLoads; ++i) {
    const int block = i * C::kWaves + wave;
    const int q = block * 64 + lane;
    const int row = q / C::kChunksPerRow;
    const int chunk = swizzle<C>(row, q % C::kChunksPerRow);  // the swizzle is an involution
    const int grow = n0 + row;
    dma_col[i] = chunk * 16;
    dma_base[i] = grow < n ? uint32_t(grow) * uint32_t(k) + uint32_t(chunk * 16) : kOutOfRange;
  }
  // Stages past the end re-read stage 0 into a slot nobody reads again.
  auto issue_w = [&] __device__(int t) __attribute__((always_inline)) {
    const int st = t < ns ? t : 0;
    auto* slot = lds + (t & (C::kSlots - 1)) * C::kStageBytes;
    if constexpr (kExactK) {
#pragma unroll
      for (int i = 0; i < C::kLoads; ++i)
        dma16(w_rsrc, reinterpret_cast<lds_void*>(slot + (i * C::kWaves + wave) * 1024),
              dma_base[i], st * C::BK);
    } else {
      const int k0 = st * C::BK;
#pragma unroll
      for (int i = 0; i < C::kLoads; ++i) {
        const bool live = dma_base[i] != kOutOfRange && k0 + dma_col[i] < k;
        dma16(w_rsrc, reinterpret_cast<lds_void*>(slot + (i * C::kWaves + wave) * 1024),
              live ? dma_base[i] + uint32_t(k0) : kOutOfRange, 0);
      }
    }
  };
  // Biased UINT8 weights are debiased in LDS, once per stage: each wave XORs the kLoads
  // 1 KiB blocks its own copies wrote with 0x80 in every byte (ds_xor_b64, 14 per lane
  // for BN = 224), after those copies landed and before the barrier that hands the
  // stage to the other waves. Debiasing the fragments in VGPRs instead would cost every
  // wave one v_xor_b32 per fragment dword per K-step, four times the work, and the
  // registers to hold it. Zero bytes from out-of-range copies become -128 codes; they
  // meet zero A bytes (K padding) or feed output columns that are never stored.
  // The XORs are inline assembly: the compiler would otherwise order them after every
  // outstanding LDS copy (s_waitcnt vmcnt(0)), draining the A and W pipelines each
  // stage. The explicit waits below order them instead; they are not counted in the
  // compiler's own LDS waits, which can only make those waits stricter.
  auto debias_w = [&] __device__(int t) __attribute__((always_inline)) {
    if constexpr (kCode == WeightCode::kBiasedU8) {
      const uint32_t wave_base = uint32_t(reinterpret_cast<uintptr_t>(
          lds + (t & (C::kSlots - 1)) * C::kStageBytes + wave * 1024));
      xor80_blocks<C::kWaves * 1024>(wave_base, std::make_integer_sequence<int, C::kLoads>{});
    }
  };

  constexpr bool kBounce = C::kABounce && kExactK;
  const int frag_row = lane & 15;
  const int frag_group = lane >> 4;
  // A operand, K-step h of block j: 16 bytes of row (lane % 16) at chunk
  // 2 * (lane / 16) + h. Two ways to get it there, both loading stage t+2 at the start
  // of stage t into register set (t+2) % 3 (the bounce only where K is a whole number of
  // stages: with the per-load K-tail checks it no longer fits in registers):
  //  * direct (kABounce false): each lane loads its own fragments, 16 rows x 64 bytes
  //    per load, which the vector-memory address unit serves at ~16 B/clk per CU;
  //  * bounce (kABounce true): loads of 8 rows x 128 bytes (lane: row lane / 8, chunk
  //    lane % 8; ~26 B/clk per CU) into staging registers, written at the middle of
  //    stage t-1 to this wave's own LDS buffer (chunks XOR-swizzled by row % 8) and read
  //    back as fragments one K-step ahead. The buffer is private to the wave, whose LDS
  //    operations complete in order, so it needs no barrier.
  // Per-lane voffsets carry the row (the stage's K offset goes in the scalar soffset);
  // rows past m start out of range and stay out of range whatever soffset is added.
  // With K a multiple of 32, a lane's 16- or 32-byte piece of a stage is wholly in range
  // or wholly past K.
  constexpr int kAOff = kBounce ? 8 : C::TM;
  const int a_lrow = kBounce ? (lane >> 3) : frag_row;     // row within a load
  const int a_lcol = kBounce ? (lane & 7) * 16 : frag_group * 32;  // byte within a stage
  const int a_rstep = kBounce ? 8 : 16;                   // rows between loads
  uint32_t a_voff[kAOff];
#pragma unroll
  for (int q = 0; q < kAOff; ++q) {
    const int row = m0 + wave * (C::BM / C::kWaves) + q * a_rstep + a_lrow;
    a_voff[q] = row < m ? uint32_t(row) * uint32_t(k) + uint32_t(a_lcol) : kOutOfRange;
  }
  i32x4 af[kBounce ? 1 : 3][2][C::TM];  // [register set][K-step][m block]
  u32x4 as[kBounce ? 3 : 1][8];          // bounce staging [register set][load]
  auto load_a = [&] __device__(int t, int set) __attribute__((always_inline)) {
    const int st = t < ns ? t : 0;
    const int k0 = st * C::BK;
#pragma unroll
    for (int q = 0; q < kAOff; ++q) {
      uint32_t voff = a_voff[q];
      int soff = k0;
      if constexpr (!kExactK) {
        voff = voff != kOutOfRange && k0 + a_lcol < k ? voff + uint32_t(k0) : kOutOfRange;
        soff = 0;
      }
      if constexpr (kBounce) {
        as[set][q] = buffer_load16(a_rsrc, voff, soff);
      } else {
#pragma unroll
        for (int h = 0; h < 2; ++h)
          af[set][h][q] = __builtin_bit_cast(i32x4, buffer_load16(a_rsrc, voff, soff + h * 16));
      }
    }
  };
  auto* a_buf = lds + C::kABase + wave * C::kABytes;
  const uint32_t a_wr = uint32_t(reinterpret_cast<uintptr_t>(a_buf)) +
                        uint32_t(a_lrow * C::BK + (((lane & 7) ^ a_lrow) * 16));
  auto store_a = [&] __device__(int set) __attribute__((always_inline)) {
    if constexpr (kBounce)
      ds_write_blocks<8 * C::BK>(a_wr, as[set], std::make_integer_sequence<int, 8>{});
  };
  int a_rd[2];
#pragma unroll
  for (int h = 0; h < 2; ++h)
    a_rd[h] = frag_row * C::BK + (((2 * frag_group + h) ^ (frag_row & 7)) * 16);
  auto read_a = [&] __device__(int h) __attribute__((always_inline)) {
    if constexpr (kBounce) {
#pragma unroll
      for (int j = 0; j < C::TM; ++j)
        af[0][h][j] = *reinterpret_cast<const __attribute__((address_space(3))) i32x4*>(
            a_buf + a_rd[h] + j * 16 * C::BK);
    }
  };

  // W fragments: row (lane % 16) of each 16-row block, chunk 2 * (lane / 16) + h; the
  // swizzle depends on row % 8 == lane % 8 only, so each K-step half has one base.
  int x_base[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) x_base[h] = frag_row * C::BK + swizzle<C>(frag_row, 2 * frag_group + h) * 16;
  auto xaddr = [&] __device__(int t, int h, int i) __attribute__((always_inline)) {
    return lds + (t & (C::kSlots - 1)) * C::kStageBytes + x_base[h] + i * 16 * C::BK;
  };

  i32x4 acc[C::TM][C::TN];
#pragma unroll
  for (int j = 0; j < C::TM; ++j)
#pragma unroll
    for (int i = 0; i < C::TN; ++i) acc[j][i] = i32x4{0, 0, 0, 0};
  i32x4 xf[C::TN];

  // One K-step: MFMAs with the W fragments in xf and A set `set`, K-step h; each W
  // fragment is reloaded for K-step (nt, nh) after its last MFMA.
  auto kstep = [&] __device__(int set, int h, int nt, int nh) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < C::TN; ++i) {
#pragma unroll
      for (int j = 0; j < C::TM; ++j)
        acc[j][i] = mfma16(xf[i], af[kBounce ? 0 : set][h][j], acc[j][i]);
      xf[i] = ld(xaddr(nt, nh, i));
      if (i == 0) read_a(nh);  // bounce: the A fragments of K-step (nt, nh)
    }
  };
  // Scheduling: the K-step's VMEM instructions alternate with its first MFMAs (which
  // cover W fragments 0 and 1), then each W fragment reload follows its group of TM
  // MFMAs.
  auto sched_kstep = [&] __device__(auto vmem_mask, auto vmem_count) __attribute__((always_inline)) {
    constexpr int kVmem = decltype(vmem_count)::value;
    static_assert(kVmem <= 2 * C::TM, "VMEM instructions fit in the first two groups");
#pragma unroll
    for (int i = 0; i < kVmem; ++i) {
      sched_group<0x008, 1>();
      sched_group<decltype(vmem_mask)::value, 1>();
    }
    if constexpr (2 * C::TM > kVmem) sched_group<0x008, 2 * C::TM - kVmem>();
    sched_group<0x100, 2 + (kBounce ? C::TM : 0)>();  // W fragments 0, 1 (and A's)
#pragma unroll
    for (int i = 2; i < C::TN; ++i) {
      sched_group<0x008, C::TM>();
      sched_group<0x100, 1>();
    }
  };
  // Before K-step (t, 1): own W copies of stage t+1 landed (and, for the A bounce,
  // own A loads of stage t+1, which go to the LDS buffer right after the barrier).
  // Vector-memory operations are counted in issue order: ..., W(t+1), A(t+1), W(t+2),
  // A(t+2) (stage t-1 issues A(t+1) then W(t+2); the prologue issues W0 A0 W1 A1 W2 so
  // t = 0 follows the same pattern). Allowing A(t+1), W(t+2) and A(t+2) outstanding
  // guarantees W(t+1); allowing only W(t+2) and A(t+2) also guarantees A(t+1). With
  // biased weights, own XORs of stage t+1 (issued at the start of stage t) completed
  // too: LDS operations complete in order, and only the TN W (and, bounce, TM A)
  // fragment reads of K-step (t, 1) follow them (the count field holds at most 15; a
  // smaller count only waits longer).
  auto sync = [&] __device__() __attribute__((always_inline)) {
    constexpr int kVm = (C::kAhead - 2) * C::kLoads + (kBounce ? 1 : 2) * C::kALoads;
    constexpr int kDs = C::TN + (kBounce ? C::TM : 0);
    constexpr int kLgkm = kDs < 15 ? kDs : 15;
    if constexpr (kCode == WeightCode::kBiasedU8)
      waitcnt<vm_lgkm_imm(kVm, kLgkm)>();
    else
      waitcnt<vmcnt_imm(kVm)>();
    workgroup_barrier();
  };
  // A is loaded two stages ahead into three register sets (set = stage % 3): the loads
  // of stage t+2 go into the set stage t-1 used. Biased weights: before those loads,
  // wait for own W copies of stage t+1 (outstanding: A(t+1), W(t+2)) and debias them.
  auto stage = [&] __device__(int t, int set) __attribute__((always_inline)) {
    if constexpr (kCode == WeightCode::kBiasedU8) {
      waitcnt<vmcnt_imm((C::kAhead - 2) * C::kLoads + C::kALoads)>();
      debias_w(t + 1);
    }
    load_a(t + 2, (set + 2) % 3);
    kstep(set, 0, t, 1);
    sched_kstep(std::integral_constant<int, 0x020>{}, std::integral_constant<int, C::kALoads>{});
    sync();
    store_a((set + 1) % 3);  // bounce: A of stage t+1 into the wave's LDS buffer
    issue_w(t + C::kAhead);
    kstep(set, 1, t + 1, 0);
    sched_kstep(std::integral_constant<int, 0x010>{}, std::integral_constant<int, C::kLoads>{});
  };

  // Prologue: W0 A0 W1 A1 W2 (the steady-state order), then the W fragments of K-step
  // (0, 0). The scheduling barriers keep that order.
  static_assert(C::kAhead == 3, "prologue issues W stages 0..2");
  issue_w(0);
  load_a(0, 0);
  __builtin_amdgcn_sched_barrier(0);
  issue_w(1);
  load_a(1, 1);
  __builtin_amdgcn_sched_barrier(0);
  issue_w(2);
  __builtin_amdgcn_sched_barrier(0);
  waitcnt<vmcnt_imm(2 * C::kLoads + C::kALoads)>();  // W(0) and A(0) landed
  store_a(0);
  if constexpr (kCode == WeightCode::kBiasedU8) {
    debias_w(0);
    __builtin_amdgcn_s_waitcnt(lgkmcnt0_imm());
  }
  workgroup_barrier();
#pragma unroll
  for (int i = 0; i < C::TN; ++i) xf[i] = ld(xaddr(0, 0, i));
  read_a(0);

  int t = 0;
  for (; t + 2 < ns; t += 3) {
    stage(t, 0);
    stage(t + 1, 1);
    stage(t + 2, 2);
  }
  if (t < ns) stage(t, 0);
  if (t + 1 < ns) stage(t + 1, 1);
  waitcnt<vmcnt_imm(0)>();  // copies past the last stage

  const int row0 = m0 + wave * (C::BM / C::kWaves);
  if constexpr (!kWorkspace) {
    // Every wave's last ring reads and copies are done before any wave reuses the ring.
    __builtin_amdgcn_s_waitcnt(lgkmcnt0_imm());
    workgroup_barrier();
    const bool lds_path = vec_n && n % 8 == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0 &&
                          row0 + C::TM * 16 <= m && n0 + C::TN * 16 <= n;
    if (lds_path) {
      store_tile16_lds<C>(acc, lds + wave * C::kEpiWaveBytes, row0, n0, n, sa, sw, out);
      return;
    }
  }
  store_tile16<C::TM, C::TN, kWorkspace>(acc, row0, n0, m, n, sa, sw, out, ws, vec_n);
}

template <class C, WeightCode kCode, bool kWorkspace, bool kExactK>
hipError_t run_wlds_exact(const int8_t* a, const void* w, const float* sa, const void* sw,
                          void* out, int32_t* ws, int m, int n, int k, hipStream_t stream) {
  auto kernel = channel_gemm_wlds_kernel<C, kCode, kWorkspace, kExactK>;
  if (const hipError_t e = prepare_lds<channel_gemm_wlds_kernel<C, kCode, kWorkspace, kExactK>>(C::kLdsBytes); e != hipSuccess)
    return e;
  const int blocks = ((n + C::BN - 1) / C::BN) * ((m + C::BM - 1) / C::BM);
  const bool vec_n = n % 4 == 0 && reinterpret_cast<uintptr_t>(sw) % 8 == 0 &&
                     reinterpret_cast<uintptr_t>(out) % 8 == 0 &&
                     reinterpret_cast<uintptr_t>(ws) % 16 == 0;
  kernel<<<blocks, C::kThreads, C::kLdsBytes, stream>>>(
      a, w, sa, static_cast<const uint16_t*>(sw), static_cast<uint16_t*>(out), ws, m, n, k,
      vec_n);
  return hipGetLastError();
}

template <class C, WeightCode kCode, bool kWorkspace>
hipError_t run_wlds(const int8_t* a, const void* w, const float* sa, const void* sw, void* out,
                    int32_t* ws, int m, int n, int k, hipStream_t stream) {
  if (k % C::BK == 0)
    return run_wlds_exact<C, kCode, kWorkspace, true>(a, w, sa, sw, out, ws, m, n, k, stream);
  return run_wlds_exact<C, kCode, kWorkspace, false>(a, w, sa, sw, out, ws, m, n, k, stream);
}

template <class C, WeightCode kCode, bool kWorkspace, bool kExactK>
hipError_t run_k128_exact(const int8_t* a, const void* w, const float* sa, const void* sw,
                          void* out, int32_t* ws, int m, int n, int k, hipStream_t stream) {
  auto kernel = channel_gemm_k128_kernel<C, kCode, kWorkspace, kExactK>;
  if (const hipError_t e = prepare_lds<channel_gemm_k128_kernel<C, kCode, kWorkspace, kExactK>>(C::kLdsBytes); e != hipSuccess)
    return e;
  const int blocks = ((n + C::BN - 1) / C::BN) * ((m + C::BM - 1) / C::BM);
  const bool vec_n = n % 4 == 0 && reinterpret_cast<uintptr_t>(sw) % 8 == 0 &&
                     reinterpret_cast<uintptr_t>(out) % 8 == 0 &&
                     reinterpret_cast<uintptr_t>(ws) % 16 == 0;
  kernel<<<blocks, C::kThreads, C::kLdsBytes, stream>>>(
      a, w, sa, static_cast<const uint16_t*>(sw), static_cast<uint16_t*>(out), ws, m, n, k,
      vec_n);
  return hipGetLastError();
}

template <class C, WeightCode kCode, bool kWorkspace>
hipError_t run_k128(const int8_t* a, const void* w, const float* sa, const void* sw, void* out,
                    int32_t* ws, int m, int n, int k, hipStream_t stream) {
  if (k % C::BK == 0)
    return run_k128_exact<C, kCode, kWorkspace, true>(a, w, sa, sw, out, ws, m, n, k, stream);
  return run_k128_exact<C, kCode, kWorkspace, false>(a, w, sa, sw, out, ws, m, n, k, stream);
}

// Tile configurations. All produce identical bits; they differ only in speed.
using Large = TileConfig<256, 256, 64, 2, 2, 3, 8>;   // 4 waves, 128x128 per wave
using Medium = TileConfig<128, 128, 64, 2, 2, 3, 8>;  // 4 waves, 64x64 per wave
using Small = TileConfig<256, 32, 128, 4, 1, 2, 1>;   // skinny M: 4 waves stacked on n
using Pipe224 = K128Config<256, 224, 2, 2, 8>;        // 4 waves, 128x112 per wave
using WLds224 = WLdsConfig<224, 8, true>;             // 4 waves, 64x224 per wave
using WLds256 = WLdsConfig<256, 8, false>;            // 4 waves, 64x256 per wave

// wide_tiles_pay and pp_beats_wide_tiles (tile_plan.h) choose between the 224-wide,
// 256-wide and persistent kernels.
static_assert(WLds256::BN == kPlanWideBN && WLds224::BN == kPlanBN, "tile_plan.h widths");

template <WeightCode kCode, bool kWorkspace>
hipError_t dispatch(const int8_t* a, const void* w, const float* sa, const void* sw, void* out,
                    int32_t* ws, int m, int n, int k, int schedule, hipStream_t stream) {
  const int cus = device_cu_count();
  int choice = schedule;
  // Schedule 0 up to M = kSmallMaxM (tile_plan.h): the small-M kernel (gemm_small.hip), or
  // above kSmallOnlyMaxM 128 x 128 or 256 x 224 tiles where they finish sooner.
  if (schedule == 0 && m <= kSmallMaxM) {
    choice = mid_m_schedule(m, n, cus);
    if (choice == 0)
      return launch_small_m_gemm(a, w, kCode, sa, sw, out, ws, m, n, k, cus > 0 ? cus : 256,
                                 stream);
  }
  if (choice == 0)
    choice = m < 1024 || medium_tiles_pay(m, n, cus) ? 1 : (wide_tiles_pay(m, n, cus) ? 3 : 4);
  // Without the INT32 copy, M >= 1024: the persistent two-waves-per-SIMD kernel
  // (gemm_pp.hip) for either weight code (its epilogue reads the channel scales 8 bytes
  // at a time) in place of the 224-wide one, and also in place of the 256-wide one
  // unless that needs far fewer rounds: per MFMA it is about 1.2x as fast (configs[3],
  // M = 16384, K = 17408, N = 5120: 5 rounds of 224-wide tiles and one of 160-wide beat 5
  // rounds of 256-wide; M = N = 4096: 2 rounds lose to 1).
  if constexpr (!kWorkspace) {
    if (schedule == 0 && m >= 1024 && choice != 1 && n % 4 == 0 &&
        reinterpret_cast<uintptr_t>(sw) % 8 == 0 && (choice == 4 || pp_beats_wide_tiles(m, n, cus)))
      return launch_pp_gemm(a, w, kCode, sa, sw, out, m, n, k, stream);
  }
  switch (choice) {
    case 5:
      return run<Small, kCode, kWorkspace>(a, w, sa, sw, out, ws, m, n, k, stream);
    case 1:
      return run<Medium, kCode, kWorkspace>(a, w, sa, sw, out, ws, m, n, k, stream);
    case 2:
      return run<Large, kCode, kWorkspace>(a, w, sa, sw, out, ws, m, n, k, stream);
    case 3:
      return run_wlds<WLds256, kCode, kWorkspace>(a, w, sa, sw, out, ws, m, n, k, stream);
    default:
      return run_wlds<WLds224, kCode, kWorkspace>(a, w, sa, sw, out, ws, m, n, k, stream);
    case 6:
      return run_k128<Pipe224, kCode, kWorkspace>(a, w, sa, sw, out, ws, m, n, k, stream);
  }
}

// ---------------------------------------------------------------------------------
// Grouped W8A8 with the per-group partials scaled and summed:
//   out[m, n] = bf16_rn( t_0 + t_1 + ... + t_{G-1} ),  FP32 additions left to right,
//   t_g = fl( fl( float_rn(acc_g[m, n]) * sa[g, m] ) * float(sw[n]) ),
//   acc_g = A_g[m, :] . W_g[n, :]  (exact INT32), A [G, M, K], W [G, N, K], sa [G, M].
// Each term is the fused_channel_mm epilogue of one group; the FP32 sum of scaled INT32
// partials follows benchmarks/cuda/q8_block_int8.cu:54-55 (the reference has no such
// op). The K loop is the 32x32 kernel's, run once per group into fresh INT32
// accumulators; the scaled terms accumulate in FP32 registers next to them, so the
// tiles are the smaller 32x32-kernel shapes (an FP32 copy of the 224-register
// accumulators of the large kernels would not fit).
template <class C>
__global__ void __launch_bounds__(C::kThreads) grouped_summed_kernel(
    const int8_t* __restrict__ a, const int8_t* __restrict__ w, const float* __restrict__ sa,
    const uint16_t* __restrict__ sw, uint16_t* __restrict__ out, int groups, int m, int n,
    int k, bool vec_n) {
  // Every product and sum below is rounded on its own (no FMA contraction of the
  // running sum with the scaled term), as the closed form requires.
#pragma clang fp contract(off)
  extern __shared__ __attribute__((aligned(1024))) char lds_raw[];
  auto* lds = (char __attribute__((address_space(3)))*)(lds_raw);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wave_n = wave / C::WM;
  const int wave_m = wave % C::WM;

  const int tiles_n = (n + C::BN - 1) / C::BN;
  const int tiles_m = (m + C::BM - 1) / C::BM;
  const int blocks = tiles_n * tiles_m;
  int logical = blockIdx.x;
  {
    const int per = blocks / kXcds, extra = blocks % kXcds;
    const int xcd = logical % kXcds, idx = logical / kXcds;
    logical = (xcd < extra ? xcd * (per + 1) : extra * (per + 1) + (xcd - extra) * per) + idx;
  }
  const int group_span = C::GROUP_M * tiles_n;
  const int first_m = (logical / group_span) * C::GROUP_M;
  const int group_rows = min(tiles_m - first_m, C::GROUP_M);
  const int tile_m = first_m + (logical % group_span) % group_rows;
  const int tile_n = (logical % group_span) / group_rows;
  const int n0 = tile_n * C::BN, m0 = tile_m * C::BM;

  // Lane holds D[n][m] for m = lane % 32 and n = 8*r4 + 4*(lane/32) + e.
  const int frag_row = lane & 31;
  const int frag_half = lane >> 5;
  const int x_row0 = wave_n * (C::BN / C::WN);
  const int y_row0 = wave_m * (C::BM / C::WM);

  float chan_scale[C::TN][4][4];
#pragma unroll
  for (int i = 0; i < C::TN; ++i)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int col = n0 + x_row0 + i * 32 + r4 * 8 + frag_half * 4 + e;
        chan_scale[i][r4][e] = col < n ? bf16_to_f32(sw[col]) : 0.f;
      }

  float sum[C::TN][C::TM][16];
  for (int g = 0; g < groups; ++g) {
    i32x16 acc[C::TN][C::TM];
#pragma unroll
    for (int i = 0; i < C::TN; ++i)
#pragma unroll
      for (int j = 0; j < C::TM; ++j) acc[i][j] = i32x16{};
    gemm_kloop<C, WeightCode::kSigned>(acc, a + int64_t(g) * m * k, w + int64_t(g) * n * k,
                                       lds, wave, lane, wave_n, wave_m, m0, n0, m, n, k);
    // Every wave is past its LDS reads before the next group's copies refill the ring.
    __builtin_amdgcn_s_waitcnt(lgkmcnt0_imm());
    __syncthreads();
    float row_scale[C::TM];
#pragma unroll
    for (int j = 0; j < C::TM; ++j) {
      const int row = m0 + y_row0 + j * 32 + frag_row;
      row_scale[j] = row < m ? sa[int64_t(g) * m + row] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < C::TN; ++i)
#pragma unroll
      for (int j = 0; j < C::TM; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float term = (float(acc[i][j][v]) * row_scale[j]) * chan_scale[i][v >> 2][v & 3];
          sum[i][j][v] = g == 0 ? term : sum[i][j][v] + term;
        }
  }

#pragma unroll
  for (int j = 0; j < C::TM; ++j) {
    const int row = m0 + y_row0 + j * 32 + frag_row;
    if (row >= m) continue;
#pragma unroll
    for (int i = 0; i < C::TN; ++i)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int col = n0 + x_row0 + i * 32 + r4 * 8 + frag_half * 4;
        const int64_t base = int64_t(row) * n + col;
        const float* v = &sum[i][j][r4 * 4];
        if (vec_n) {
          if (col < n)
            *reinterpret_cast<u32x2*>(out + base) =
                u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (col + e < n) out[base + e] = uint16_t(f32_to_bf16(v[e]));
        }
      }
  }
}

template <class C>
hipError_t run_grouped(const int8_t* a, const int8_t* w, const float* sa, const void* sw,
                       void* out, int groups, int m, int n, int k, hipStream_t stream) {
  auto kernel = grouped_summed_kernel<C>;
  if (const hipError_t e = prepare_lds<grouped_summed_kernel<C>>(C::kLdsBytes); e != hipSuccess)
    return e;
  const int blocks = ((n + C::BN - 1) / C::BN) * ((m + C::BM - 1) / C::BM);
  const bool vec_n = n % 4 == 0 && reinterpret_cast<uintptr_t>(out) % 8 == 0;
  kernel<<<blocks, C::kThreads, C::kLdsBytes, stream>>>(
      a, w, sa, static_cast<const uint16_t*>(sw), static_cast<uint16_t*>(out), groups, m, n, k,
      vec_n);
  return hipGetLastError();
}

}  // namespace

int device_cu_count() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cached[kMaxDevices];  // 0 until first queried
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices) return 0;
  int cus = cached[device].load(std::memory_order_relaxed);
  if (cus > 0) return cus;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
      cus <= 0)
    return 0;
  cached[device].store(cus, std::memory_order_relaxed);
  return cus;
}

hipError_t launch_channel_gemm(const int8_t* a, const void* w, WeightCode code,
                               const float* sa, const void* sw, void* out,
                               int32_t* workspace, int m, int n, int k, int schedule,
                               hipStream_t stream) {
  if (code == WeightCode::kBiasedU8)
    return dispatch<WeightCode::kBiasedU8, false>(a, w, sa, sw, out, nullptr, m, n, k, 0,
                                                  stream);
  if (workspace)
    return dispatch<WeightCode::kSigned, true>(a, w, sa, sw, out, workspace, m, n, k, 0,
                                               stream);
  return dispatch<WeightCode::kSigned, false>(a, w, sa, sw, out, nullptr, m, n, k, schedule,
                                              stream);
}

hipError_t launch_grouped_summed_gemm(const int8_t* a, const int8_t* w, const float* sa,
                                      const void* sw, void* out, int groups, int m, int n,
                                      int k, hipStream_t stream) {
  if (m <= 32) return run_grouped<Small>(a, w, sa, sw, out, groups, m, n, k, stream);
  // The two-waves-per-SIMD kernel copies the row scales into LDS four rows (16 bytes) at a
  // time at byte offset 4 (g m + row) of a buffer of 4 groups m bytes: that needs m % 4 == 0
  // and a 16-byte aligned sa (so no copy straddles a group boundary, is misaligned or runs
  // past the end of sa), and every offset below the 2^31 out-of-range marker.
  if (m >= 1024 && n % 4 == 0 && reinterpret_cast<uintptr_t>(sw) % 8 == 0 &&
      groups <= grouped_pp_max_groups() && m % 4 == 0 &&
      reinterpret_cast<uintptr_t>(sa) % 16 == 0 &&
      int64_t(groups) * m * 4 < (int64_t(1) << 31))
    return launch_grouped_pp_gemm(a, w, sa, sw, out, groups, m, n, k, stream);
  return run_grouped<Medium>(a, w, sa, sw, out, groups, m, n, k, stream);
}

}  // namespace ci8
