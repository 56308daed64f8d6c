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
  static constexpr int kRowsPer256 = 256 / BK;
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

// Chunk slot of logical 16-byte chunk c in LDS row r.
template <class C>
__device__ __forceinline__ int swizzle(int row, int chunk) {
  return chunk ^ ((row / C::kRowsPer256) % C::kChunksPerRow);
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

template <class C, WeightCode kCode, bool kWorkspace>
__global__ void __launch_bounds__(C::kThreads) channel_gemm_kernel(
    const int8_t* __restrict__ a, const void* __restrict__ w, const float* __restrict__ sa,
    const uint16_t* __restrict__ sw, uint16_t* __restrict__ out, int32_t* __restrict__ ws,
    int m, int n, int k, bool vec_n) {
  extern __shared__ __attribute__((aligned(1024))) char lds_raw[];
  auto* lds = (char __attribute__((address_space(3)))*)(lds_raw);

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
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

  const auto w_rsrc = make_rsrc(w, uint32_t(n) * uint32_t(k));
  const auto a_rsrc = make_rsrc(a, uint32_t(m) * uint32_t(k));

  i32x16 acc[C::TN][C::TM];
#pragma unroll
  for (int i = 0; i < C::TN; ++i)
#pragma unroll
    for (int j = 0; j < C::TM; ++j) acc[i][j] = i32x16{};

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

  // Per-lane fragment geometry: MFMA row/col = lane % 32, K half = lane / 32.
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

  // Epilogue. Lane holds D[n][m] for m = lane % 32 and n = 8*r4 + 4*(lane/32) + j.
  // vec_n: n % 4 == 0 and sw, out (and ws) aligned for 8-byte (16-byte) accesses.
#pragma unroll
  for (int j = 0; j < C::TM; ++j) {
    const int row = m0 + y_row0 + j * 32 + frag_row;  // output row (m)
    if (row >= m) continue;
    const float row_scale = sa[row];
#pragma unroll
    for (int i = 0; i < C::TN; ++i) {
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int col = n0 + x_row0 + i * 32 + r4 * 8 + frag_half * 4;  // output column (n)
        if (col >= n) continue;
        const int64_t base = int64_t(row) * n + col;
        if (vec_n) {
          const u32x2 s2 = *reinterpret_cast<const u32x2*>(sw + col);
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t sbits = (s2[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
            v[e] = (float(acc[i][j][r4 * 4 + e]) * row_scale) * bf16_to_f32(sbits);
          }
          *reinterpret_cast<u32x2*>(out + base) = u32x2{pack_bf16x2(v[0], v[1]),
                                                         pack_bf16x2(v[2], v[3])};
          if constexpr (kWorkspace)
            *reinterpret_cast<i32x4*>(ws + base) =
                i32x4{acc[i][j][r4 * 4 + 0], acc[i][j][r4 * 4 + 1], acc[i][j][r4 * 4 + 2],
                      acc[i][j][r4 * 4 + 3]};
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (col + e < n) {
              const float v = (float(acc[i][j][r4 * 4 + e]) * row_scale) * bf16_to_f32(sw[col + e]);
              out[base + e] = uint16_t(f32_to_bf16(v));
              if constexpr (kWorkspace) ws[base + e] = acc[i][j][r4 * 4 + e];
            }
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
  static bool configured = false;  // benign race: every thread sets the same attribute
  if (!configured) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             C::kLdsBytes);
    if (e != hipSuccess) return e;
    configured = true;
  }
  const int blocks = ((n + C::BN - 1) / C::BN) * ((m + C::BM - 1) / C::BM);
  const bool vec_n = n % 4 == 0 && reinterpret_cast<uintptr_t>(sw) % 8 == 0 &&
                     reinterpret_cast<uintptr_t>(out) % 8 == 0 &&
                     reinterpret_cast<uintptr_t>(ws) % 16 == 0;
  kernel<<<blocks, C::kThreads, C::kLdsBytes, stream>>>(
      a, w, sa, static_cast<const uint16_t*>(sw), static_cast<uint16_t*>(out), ws, m, n, k,
      vec_n);
  return hipGetLastError();
}

// Tile configurations. All produce identical bits; they differ only in speed.
using Large = TileConfig<256, 256, 64, 2, 2, 3, 8>;   // 4 waves, 128x128 per wave
using Medium = TileConfig<128, 128, 64, 2, 2, 3, 8>;  // 4 waves, 64x64 per wave
using Small = TileConfig<256, 32, 128, 4, 1, 2, 1>;   // skinny M: 4 waves stacked on n

template <WeightCode kCode, bool kWorkspace>
hipError_t dispatch(const int8_t* a, const void* w, const float* sa, const void* sw, void* out,
                    int32_t* ws, int m, int n, int k, int schedule, hipStream_t stream) {
  int choice = schedule;
  if (choice == 0) choice = m <= 32 ? 5 : (m < 1024 ? 1 : 4);
  switch (choice) {
    case 5:
      return run<Small, kCode, kWorkspace>(a, w, sa, sw, out, ws, m, n, k, stream);
    case 1:
    case 3:
      return run<Medium, kCode, kWorkspace>(a, w, sa, sw, out, ws, m, n, k, stream);
    default:
      return run<Large, kCode, kWorkspace>(a, w, sa, sw, out, ws, m, n, k, stream);
  }
}

}  // namespace

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

}  // namespace ci8
