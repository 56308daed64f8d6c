// Small-M INT8 GEMM for gfx950: the same product and epilogue as gemm.hip,
//
//   out[m, n] = bf16_rn( fl( fl( float_rn(acc[m, n]) * sa[m] ) * float(sw[n]) ) )
//   acc[m, n] = sum_k a[m, k] * w[n, k]            (exact INT32)
//
// for M up to a few hundred rows (csrc/fused_mm.cu:89-91 shrinks its M tile for the
// same reason). There the GEMM is bound by moving operands, not by the MFMAs: at
// M = 128, K = N = 4096 the 16.8 MB of weights stream from HBM once, and every
// workgroup also reads the activation rows of its tile from L2. The large-tile kernels
// give such a shape 32 workgroups for 256 CUs, so this kernel cuts the output into
// small tiles (BM x BN, 16..64 each) to put a workgroup on every CU, and splits K over
// the workgroup's four waves, which sum their INT32 partials through LDS at the end
// (exact, so the split changes no bit).
//
// Each wave streams its K range through a private 3-slot LDS ring filled by
// buffer_load ... lds (8 rows x 128 bytes per instruction, the pattern the address
// unit serves fastest), so the loop has no workgroup barrier, and reads its MFMA
// fragments from the ring. Rows past M or N and bytes past K come back as zeros from
// the buffer range check. The MFMA is v_mfma_i32_16x16x64_i8 on the transposed tile
// D[n, m] = W . A^T, so a lane ends with 4 consecutive output columns of one row.
#include "ci8_device.h"
#include "launch.h"

namespace ci8 {
namespace {

constexpr int kXcds = 8;

template <int BM_, int BN_, int kWaves_ = 4, int kSlots_ = 3>
struct SmallConfig {
  static constexpr int BM = BM_, BN = BN_;
  static constexpr int kWaves = kWaves_;        // K is split over the waves
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int BK = 128;                // K bytes per stage
  static constexpr int TM = BM / 16, TN = BN / 16;
  static constexpr int kSlots = kSlots_;        // per-wave ring depth
  static constexpr int kALoads = BM / 8;        // 1 KiB copies (8 rows x 128 B) per stage
  static constexpr int kWLoads = BN / 8;
  static constexpr int kLoads = kALoads + kWLoads;
  static constexpr int kStageBytes = kLoads * 1024;
  static constexpr int kWaveBytes = kSlots * kStageBytes;
  static constexpr int kPartialBytes = kWaves * TM * TN * 64 * 16;
  static constexpr int kLdsBytes =
      kWaves * kWaveBytes > kPartialBytes ? kWaves * kWaveBytes : kPartialBytes;
  static_assert(BM % 16 == 0 && BN % 16 == 0, "16-row MFMA blocks");
  static_assert(kLdsBytes <= 160 * 1024, "LDS");
};

__device__ __forceinline__ i32x4 lds_read16(const char __attribute__((address_space(3)))* p) {
  return *reinterpret_cast<const __attribute__((address_space(3))) i32x4*>(p);
}

// Waits until at most `after` stages of this wave's copies are in flight (s_waitcnt
// takes an immediate, so each possible count is its own instruction).
template <class C, int kAfter = C::kSlots - 1>
__device__ __forceinline__ void wait_stages(int after) {
  if constexpr (kAfter == 0) {
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  } else {
    if (after >= kAfter)
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(kAfter * C::kLoads));
    else
      wait_stages<C, kAfter - 1>(after);
  }
}

template <class C, WeightCode kCode, bool kWorkspace>
__global__ void __launch_bounds__(C::kThreads) small_m_gemm_kernel(
    const int8_t* __restrict__ a, const void* __restrict__ w, const float* __restrict__ sa,
    const uint16_t* __restrict__ sw, uint16_t* __restrict__ out, int32_t* __restrict__ ws,
    int m, int n, int k, bool vec_n) {
  extern __shared__ __attribute__((aligned(1024))) char lds_raw[];
  auto* lds = (char __attribute__((address_space(3)))*)(lds_raw);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  // Workgroup -> tile. The hardware deals workgroups round-robin over the 8 XCDs; undo
  // that so each XCD runs a contiguous range of logical tiles, and order the logical
  // tiles m-fastest so the tiles sharing a weight panel run together on one XCD (one
  // HBM read of the panel, the rest from that XCD's L2).
  const int tiles_m = (m + C::BM - 1) / C::BM;
  const int tiles_n = (n + C::BN - 1) / C::BN;
  const int blocks = tiles_m * tiles_n;
  int logical = blockIdx.x;
  {
    const int per = blocks / kXcds, extra = blocks % kXcds;
    const int xcd = logical % kXcds, idx = logical / kXcds;
    logical = (xcd < extra ? xcd * (per + 1) : extra * (per + 1) + (xcd - extra) * per) + idx;
  }
  const int tile_m = logical % tiles_m, tile_n = logical / tiles_m;
  const int m0 = tile_m * C::BM, n0 = tile_n * C::BN;

  // This wave's share of the ns 128-byte K stages: stages wave, wave + kWaves, ...
  // (interleaved, so the waves of a workgroup read neighbouring stretches of each row;
  // measured a few percent faster than contiguous quarters).
  const int ns = (k + C::BK - 1) / C::BK;
  const int count = (ns - wave + C::kWaves - 1) / C::kWaves;
  auto stage_of = [&] __device__(int i) __attribute__((always_inline)) {
    return wave + C::kWaves * i;
  };

  const auto a_rsrc = make_rsrc(a, uint32_t(m) * uint32_t(k));
  const auto w_rsrc = make_rsrc(w, uint32_t(n) * uint32_t(k));

  // Copy q of a stage brings 8 rows x 128 bytes: lane -> row lane / 8, LDS chunk slot
  // lane % 8, which holds logical chunk slot ^ (row % 8) (an involution), so the
  // fragment reads below (16 rows at one logical chunk) spread over all banks. The
  // stage's K offset goes in soffset; per-lane offsets past the matrix stay out of range.
  const int c_row = lane >> 3;
  const int c_chunk = (lane & 7) ^ c_row;
  uint32_t a_off[C::kALoads], w_off[C::kWLoads];
#pragma unroll
  for (int q = 0; q < C::kALoads; ++q) {
    const int row = m0 + q * 8 + c_row;
    a_off[q] = row < m ? uint32_t(row) * uint32_t(k) + uint32_t(c_chunk * 16) : kOutOfRange;
  }
#pragma unroll
  for (int q = 0; q < C::kWLoads; ++q) {
    const int row = n0 + q * 8 + c_row;
    w_off[q] = row < n ? uint32_t(row) * uint32_t(k) + uint32_t(c_chunk * 16) : kOutOfRange;
  }
  auto* ring = lds + wave * C::kWaveBytes;
  const bool exact_k = k % C::BK == 0;
  auto issue = [&] __device__(int it) __attribute__((always_inline)) {
    auto* slot = ring + (it % C::kSlots) * C::kStageBytes;
    const int k0 = stage_of(it) * C::BK;
#pragma unroll
    for (int q = 0; q < C::kLoads; ++q) {
      const bool is_a = q < C::kALoads;
      uint32_t off = is_a ? a_off[q] : w_off[q - C::kALoads];
      // A 16-byte chunk lies wholly inside or wholly past K (k % 32 == 0).
      if (!exact_k && off != kOutOfRange && k0 + c_chunk * 16 >= k) off = kOutOfRange;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(is_a ? a_rsrc : w_rsrc,
                                               reinterpret_cast<lds_void*>(slot + q * 1024), 16,
                                               off, k0, 0, 0);
    }
  };

  // Fragment of 16-row block j, K-step h: row (lane % 16) at logical chunk
  // 2 * (lane / 16) + h of the 128-byte stage (A and W use the same K order, so the
  // dot products are unchanged); the slot of that chunk is chunk ^ (row % 8).
  const int f_row = lane & 15, f_group = lane >> 4;
  int f_off[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) f_off[h] = f_row * 128 + (((2 * f_group + h) ^ (f_row & 7)) * 16);

  i32x4 acc[C::TM][C::TN];
#pragma unroll
  for (int j = 0; j < C::TM; ++j)
#pragma unroll
    for (int i = 0; i < C::TN; ++i) acc[j][i] = i32x4{0, 0, 0, 0};

  // The epilogue's scales, loaded before the K loop so their latency hides behind it.
  // Wave v finishes blocks v, v + kWaves, ... of the tile (block b = m block b / TN,
  // n block b % TN); a lane of block b holds D[n][m] for m = lane % 16 and
  // n = 4 * (lane / 16) + e.
  constexpr int kMine = (C::TM * C::TN + C::kWaves - 1) / C::kWaves;
  float rs[kMine];
  u32x2 s2[kMine];
#pragma unroll
  for (int t = 0; t < kMine; ++t) {
    const int b = wave + t * C::kWaves;
    const int row = m0 + (b / C::TN) * 16 + f_row;
    const int col = n0 + (b % C::TN) * 16 + f_group * 4;
    const bool live = b < C::TM * C::TN && row < m;
    rs[t] = live ? sa[row] : 0.f;
    s2[t] = live && vec_n && col < n ? *reinterpret_cast<const u32x2*>(sw + col) : u32x2{0, 0};
  }

  for (int it = 0; it < C::kSlots - 1 && it < count; ++it) issue(it);
  for (int it = 0; it < count; ++it) {
    if (it + C::kSlots - 1 < count) issue(it + C::kSlots - 1);
    // Own copies of this wave's stage `it` landed: at most the stages issued after it
    // are in flight.
    const int after = min(count - 1 - it, C::kSlots - 1);
    wait_stages<C>(after);
    asm volatile("" ::: "memory");
    const auto* slot = ring + (it % C::kSlots) * C::kStageBytes;
    i32x4 af[2][C::TM], wf[2][C::TN];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int j = 0; j < C::TM; ++j) af[h][j] = lds_read16(slot + j * 2048 + f_off[h]);
#pragma unroll
      for (int i = 0; i < C::TN; ++i) {
        wf[h][i] = lds_read16(slot + C::kALoads * 1024 + i * 2048 + f_off[h]);
        if constexpr (kCode == WeightCode::kBiasedU8) wf[h][i] ^= int32_t(0x80808080u);
      }
    }
    // The slot is refilled two iterations from now, after these reads returned (the
    // MFMAs below consume them first).
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int j = 0; j < C::TM; ++j)
#pragma unroll
        for (int i = 0; i < C::TN; ++i)
          acc[j][i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[h][i], af[h][j], acc[j][i], 0, 0, 0);
  }

  // Sum the waves' partials through LDS (the ring is free once every wave is past its
  // last fragment read), in ascending wave order (INT32 sums are exact in any order).
  __builtin_amdgcn_s_waitcnt(lgkmcnt0_imm());
  __syncthreads();
  auto* part = reinterpret_cast<__attribute__((address_space(3))) i32x4*>(lds);
#pragma unroll
  for (int j = 0; j < C::TM; ++j)
#pragma unroll
    for (int i = 0; i < C::TN; ++i) part[((wave * C::TM + j) * C::TN + i) * 64 + lane] = acc[j][i];
  __syncthreads();

#pragma unroll
  for (int t = 0; t < kMine; ++t) {
    const int b = wave + t * C::kWaves;
    if (b >= C::TM * C::TN) break;
    i32x4 sum = part[b * 64 + lane];
#pragma unroll
    for (int v = 1; v < C::kWaves; ++v) sum += part[(v * C::TM * C::TN + b) * 64 + lane];
    const int row = m0 + (b / C::TN) * 16 + f_row;
    const int col = n0 + (b % C::TN) * 16 + f_group * 4;
    if (row >= m) continue;
    const int64_t base = int64_t(row) * n + col;
    if (vec_n) {
      if (col >= n) continue;
      float v4[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t bits = (s2[t][e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
        v4[e] = (float(sum[e]) * rs[t]) * bf16_to_f32(bits);
      }
      *reinterpret_cast<u32x2*>(out + base) =
          u32x2{pack_bf16x2(v4[0], v4[1]), pack_bf16x2(v4[2], v4[3])};
      if constexpr (kWorkspace) *reinterpret_cast<i32x4*>(ws + base) = sum;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (col + e < n) {
          out[base + e] =
              uint16_t(f32_to_bf16((float(sum[e]) * rs[t]) * bf16_to_f32(sw[col + e])));
          if constexpr (kWorkspace) ws[base + e] = sum[e];
        }
      }
    }
  }
}

template <class C, WeightCode kCode, bool kWorkspace>
hipError_t run_small(const int8_t* a, const void* w, const float* sa, const void* sw, void* out,
                     int32_t* ws, int m, int n, int k, hipStream_t stream) {
  auto kernel = small_m_gemm_kernel<C, kCode, kWorkspace>;
  if (const hipError_t e = prepare_lds<small_m_gemm_kernel<C, kCode, kWorkspace>>(C::kLdsBytes); e != hipSuccess)
    return e;
  const int blocks = ((m + C::BM - 1) / C::BM) * ((n + C::BN - 1) / C::BN);
  const bool vec_n = n % 4 == 0 && reinterpret_cast<uintptr_t>(sw) % 8 == 0 &&
                     reinterpret_cast<uintptr_t>(out) % 8 == 0 &&
                     reinterpret_cast<uintptr_t>(ws) % 16 == 0;
  kernel<<<blocks, C::kThreads, C::kLdsBytes, stream>>>(
      a, w, sa, static_cast<const uint16_t*>(sw), static_cast<uint16_t*>(out), ws, m, n, k,
      vec_n);
  return hipGetLastError();
}

}  // namespace

template <WeightCode kCode, bool kWorkspace>
hipError_t launch_small_m_gemm_t(const int8_t* a, const void* w, const float* sa, const void* sw,
                                 void* out, int32_t* ws, int m, int n, int k, int cus,
                                 hipStream_t stream) {
  const SmallShape best = small_best_shape(m, n, cus);
#define CI8_SMALL(BM_, BN_)                                                                  \
  if (best.bm == BM_ && best.bn == BN_)                                                      \
    return run_small<SmallConfig<BM_, BN_>, kCode, kWorkspace>(a, w, sa, sw, out, ws, m, n, \
                                                               k, stream);
  CI8_SMALL(64, 32) CI8_SMALL(32, 64) CI8_SMALL(16, 64) CI8_SMALL(32, 32) CI8_SMALL(32, 16)
  CI8_SMALL(16, 32)
#undef CI8_SMALL
  return run_small<SmallConfig<16, 16>, kCode, kWorkspace>(a, w, sa, sw, out, ws, m, n, k,
                                                            stream);
}

hipError_t launch_small_m_gemm(const int8_t* a, const void* w, WeightCode code, const float* sa,
                               const void* sw, void* out, int32_t* ws, int m, int n, int k,
                               int cus, hipStream_t stream) {
  if (code == WeightCode::kBiasedU8)
    return launch_small_m_gemm_t<WeightCode::kBiasedU8, false>(a, w, sa, sw, out, nullptr, m, n,
                                                               k, cus, stream);
  if (ws)
    return launch_small_m_gemm_t<WeightCode::kSigned, true>(a, w, sa, sw, out, ws, m, n, k, cus,
                                                            stream);
  return launch_small_m_gemm_t<WeightCode::kSigned, false>(a, w, sa, sw, out, nullptr, m, n, k,
                                                           cus, stream);
}

}  // namespace ci8
