// Small-batch W8A16 (channel_gemv) for gfx950.
//
//   wq[n, k]  = bf16_rn( float(w[n, k]) * float(scale[n]) )       (csrc/gemv.cu:25)
//   out[m, n] = bf16_rn( sum_k float(x[m, k]) * float(wq[n, k]) )  (FP32 accumulation)
//
// The dequantized multiplicand is bit-identical to the reference's. Only the FP32
// summation order differs (the reference uses a per-lane FMA chain and a 32-lane
// butterfly, csrc/gemv.cu:16-45; here the products are summed by the MFMA and the
// partial sums of the K splits are added in a fixed order), so parity is by tolerance
// as in tests/test_gemv.py:24-33.
//
// Design: the op is HBM-bound on the INT8 weights (N*K bytes).
//  * The multiply-accumulate runs on v_mfma_f32_16x16x32_bf16 (rows = 16 channels,
//    columns = up to 16 batch rows, so m <= 16 costs the same as m = 1). The VALU only
//    dequantizes, 2.5 instructions per weight: a sign-extending v_cvt_f32_i32 with SDWA
//    byte select, one multiply by the scale (exact, since code*scale fits in FP32) and
//    half a v_cvt_pk_bf16_f32.
//  * A workgroup owns kCB blocks of 16 channels and splits K into kS contiguous
//    ranges; each of its kCB*kS waves streams one (block, range) pair of W straight
//    from HBM into registers, two stages of kU 64-byte K blocks ahead of its MFMAs.
//  * x is the same for every channel, so it is not loaded per lane: each stage's
//    x[0:m, range] slice is copied once per workgroup into an LDS ring by
//    buffer_load ... lds (1 KiB contiguous per instruction) and shared by the kCB waves
//    of that range. Rows past m are written as zeros by the buffer range check. This
//    cuts the L2 -> CU traffic for x at m = 16 from twice the weight bytes to a small
//    fraction of them.
//  * One barrier per stage. The ring has three slots, held in three separate LDS
//    arrays so the compiler can see that the slot being read is not the slot an
//    in-flight copy is writing.
// At m = 1 with K <= 8192 the MFMA would run 1 useful column of 16, and the weights
// can stream in whole-row order instead: a row kernel (below) gives each wave whole
// weight rows, read as 1 KiB contiguous pieces two rows ahead, and does the dequantize
// and the dot product on the VALU (v_dot2_f32_bf16 on the BF16 products).
// For K <= 8192 and 2 <= m <= 16, a balanced-span kernel (one 16-wave workgroup per
// CU over an equal share of the channels, x fragments held in registers, W streamed one
// block of 16 channels ahead) replaces the kernels below, except where an interleaved
// quad-block kernel is faster (2 <= m <= 4 with K >= 4096, and 5 <= m <= 8 with K >
// 5120): it runs the products on the 4x4x4 MFMA over blocks of 4 channels so that each
// load instruction reads 4 channels x 256 contiguous bytes, and deals the blocks to the
// CUs round-robin so the chip streams one contiguous window. At m = 1 for longer K
// while x[0:m, :] fits in 64 KiB of LDS, a second kernel copies all of x into LDS once
// and then lets every wave stream its W through a rolling window of ten 64-byte blocks
// with no barriers at all, which removes the per-stage lock-step of the ring. Up to
// 160 KiB of LDS, a persistent form of it runs one workgroup per CU that copies x once
// and walks its channel blocks; beyond that, the ring. Weight rows past N and K chunks
// past K read as zero through the buffer range check.
#include "ci8_device.h"
#include "launch.h"

namespace ci8 {
namespace {

template <int kCB_, int kS_, int kU_>
struct GemvConfig {
  static constexpr int kCB = kCB_;                       // channel blocks of 16 per workgroup
  static constexpr int kS = kS_;                         // K ranges per workgroup
  static constexpr int kU = kU_;                         // 64-element K blocks per stage
  static constexpr int kWaves = kCB * kS;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kRowBytes = kU * 128;             // one x row of one stage (BF16)
  static constexpr int kSlotBytes = kS * 16 * kRowBytes;
  static constexpr int kDmaPerStage = kSlotBytes / 1024;  // 1 KiB per copy instruction
  static constexpr int kDmaPerWave = kDmaPerStage / kWaves;
  static_assert(kDmaPerStage % kWaves == 0, "every wave issues the same number of copies");
  static_assert(8 % kU == 0, "a copy instruction covers whole x rows");
};

// Four INT8 codes -> two packed BF16 pairs bf16_rn(code * s). code * s is exact in FP32
// (8-bit by 8-bit significands), so the one rounding is the BF16 one. Each byte is
// sign-extended and converted by one v_cvt_f32_i32 (SDWA byte select).
__device__ __forceinline__ u32x2 dequant4(uint32_t word, float s) {
  return u32x2{pack_bf16x2(float(int8_t(word)) * s, float(int8_t(word >> 8)) * s),
               pack_bf16x2(float(int8_t(word >> 16)) * s, float(int8_t(word >> 24)) * s)};
}

__device__ __forceinline__ f32x4 mfma_bf16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ void copy16(__amdgpu_buffer_rsrc_t rsrc, lds_void* dst,
                                       uint32_t offset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, dst, 16, offset, 0, 0, 0);
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

typedef char __attribute__((address_space(3))) lds_char;

// Per-lane constants of this wave's x copies: copy instruction i writes 16-byte unit
// (wave + i * kWaves) * 64 + lane of a slot laid out as [range][row 0..15][kU][128 B],
// with the 16-byte chunks of each 128-byte block XOR-swizzled by (row & 7).
template <class C>
struct XCopies {
  uint32_t row_base[C::kDmaPerWave];  // row * k * 2, or >= 2^31 for rows >= m
  int range[C::kDmaPerWave], block[C::kDmaPerWave], chunk_byte[C::kDmaPerWave];
};

template <class C>
__device__ __forceinline__ void issue_x(const XCopies<C>& xc, __amdgpu_buffer_rsrc_t x_rsrc,
                                        lds_char* slot, int wave, int stage, int range_len,
                                        int kblocks, int k) {
#pragma unroll
  for (int i = 0; i < C::kDmaPerWave; ++i) {
    const int kb = xc.range[i] * range_len + stage * C::kU + xc.block[i];
    const int kend = min((xc.range[i] + 1) * range_len, kblocks);
    const bool valid = kb < kend && kb * 128 + xc.chunk_byte[i] < k * 2;
    const uint32_t offset =
        valid ? xc.row_base[i] + uint32_t(kb * 128 + xc.chunk_byte[i]) : kOutOfRange;
    copy16(x_rsrc, reinterpret_cast<lds_void*>(slot + (wave + i * C::kWaves) * 1024), offset);
  }
}

template <class C>
__device__ __forceinline__ void issue_w(u32x4 (&wv)[C::kU], __amdgpu_buffer_rsrc_t w_rsrc,
                                        uint32_t w_base, int lane_col, int range, int stage,
                                        int range_len, int kblocks, int k) {
  const int kend = min((range + 1) * range_len, kblocks);
#pragma unroll
  for (int j = 0; j < C::kU; ++j) {
    const int kb = range * range_len + stage * C::kU + j;
    const bool valid = kb < kend && kb * 64 + lane_col < k;
    wv[j] = __builtin_bit_cast(
        u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                   w_rsrc, valid ? w_base + uint32_t(kb * 64) : kOutOfRange, 0, 0));
  }
}

// Stage t (t % 3 == R): wait for x(t) and W(t), barrier, read this stage's x
// fragments, then issue x(t+1) and W(t+2) and run the MFMAs. Copies are issued after
// the LDS reads so the compiler's wait for in-flight LDS copies ahead of those reads
// never has to cover the new ones.
template <class C, int R>
__device__ __forceinline__ void gemv_stage(int t, const XCopies<C>& xc,
                                           __amdgpu_buffer_rsrc_t x_rsrc,
                                           __amdgpu_buffer_rsrc_t w_rsrc,
                                           lds_char* const (&xs)[3], u32x4 (&wv)[3][C::kU],
                                           f32x4& acc, int wave, uint32_t w_base, int group,
                                           int row, int range, int range_len, int kblocks,
                                           int k, float s) {
  waitcnt<vmcnt_imm(C::kU)>();  // everything but W(t+1) has landed, x(t) included
  workgroup_barrier();          // every wave's share of x(t) has landed
  const lds_char* base = xs[R] + (range * 16 + row) * C::kRowBytes;
  u32x4 xf[C::kU][2];
#pragma unroll
  for (int j = 0; j < C::kU; ++j)
#pragma unroll
    for (int h = 0; h < 2; ++h)
      xf[j][h] = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(
          base + j * 128 + (((2 * group + h) ^ (row & 7)) * 16));
  // Slot (R+1)%3 last held stage t-2, which every wave finished before this barrier.
  issue_x<C>(xc, x_rsrc, xs[(R + 1) % 3], wave, t + 1, range_len, kblocks, k);
  issue_w<C>(wv[(R + 2) % 3], w_rsrc, w_base, group * 16, range, t + 2, range_len, kblocks, k);
#pragma unroll
  for (int j = 0; j < C::kU; ++j) {
    const u32x4 wq = wv[R][j];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const u32x2 lo = dequant4(wq[2 * h], s), hi = dequant4(wq[2 * h + 1], s);
      acc = mfma_bf16(u32x4{lo[0], lo[1], hi[0], hi[1]}, xf[j][h], acc);
    }
  }
}

template <class C>
__global__ void __launch_bounds__(C::kThreads) channel_gemv_kernel(
    const uint16_t* __restrict__ x, const int8_t* __restrict__ w,
    const uint16_t* __restrict__ scale, uint16_t* __restrict__ out, int m, int n, int k) {
  __shared__ __attribute__((aligned(16))) char xs0[C::kSlotBytes];
  __shared__ __attribute__((aligned(16))) char xs1[C::kSlotBytes];
  __shared__ __attribute__((aligned(16))) char xs2[C::kSlotBytes];
  __shared__ f32x4 partial[C::kWaves][64];
  lds_char* const xs[3] = {(lds_char*)xs0, (lds_char*)xs1, (lds_char*)xs2};

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int cb = wave % C::kCB, range = wave / C::kCB;
  const int row = lane & 15;   // MFMA row (channel) / column (batch row)
  const int group = lane >> 4; // 16-element K group within a 64-element K block
  const int channel = blockIdx.x * 16 * C::kCB + cb * 16 + row;

  const auto w_rsrc = make_rsrc(w, uint32_t(n) * uint32_t(k));
  const auto x_rsrc = make_rsrc(x, uint32_t(m) * uint32_t(k) * 2u);
  const float s = channel < n ? bf16_to_f32(scale[channel]) : 0.f;
  const uint32_t w_base =
      channel < n ? uint32_t(channel) * uint32_t(k) + uint32_t(group * 16) : kOutOfRange;
  const int kblocks = (k + 63) / 64;
  const int range_len = (kblocks + C::kS - 1) / C::kS;
  const int stages = (range_len + C::kU - 1) / C::kU;

  XCopies<C> xc;
#pragma unroll
  for (int i = 0; i < C::kDmaPerWave; ++i) {
    const int unit = (wave + i * C::kWaves) * 64 + lane;
    const int srow = unit / (C::kRowBytes / 16);
    const int r = srow & 15, within = unit % (C::kRowBytes / 16);
    xc.range[i] = srow >> 4;
    xc.block[i] = within >> 3;
    xc.chunk_byte[i] = ((within & 7) ^ (r & 7)) * 16;
    xc.row_base[i] = r < m ? uint32_t(r) * uint32_t(k) * 2u : kOutOfRange;
  }

  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  u32x4 wv[3][C::kU];
  // Issue order W(0), x(0), W(1): stage 0 then waits with only W(1) outstanding.
  issue_w<C>(wv[0], w_rsrc, w_base, group * 16, range, 0, range_len, kblocks, k);
  issue_x<C>(xc, x_rsrc, xs[0], wave, 0, range_len, kblocks, k);
  issue_w<C>(wv[1], w_rsrc, w_base, group * 16, range, 1, range_len, kblocks, k);
  for (int t = 0; t < stages; t += 3) {
    gemv_stage<C, 0>(t, xc, x_rsrc, w_rsrc, xs, wv, acc, wave, w_base, group, row, range,
                     range_len, kblocks, k, s);
    if (t + 1 >= stages) break;
    gemv_stage<C, 1>(t + 1, xc, x_rsrc, w_rsrc, xs, wv, acc, wave, w_base, group, row, range,
                     range_len, kblocks, k, s);
    if (t + 2 >= stages) break;
    gemv_stage<C, 2>(t + 2, xc, x_rsrc, w_rsrc, xs, wv, acc, wave, w_base, group, row, range,
                     range_len, kblocks, k, s);
  }
  waitcnt<vmcnt_imm(0)>();  // drain the trailing (out-of-range) copies before exit

  // Sum the K ranges' partials in a fixed order, then round once to BF16.
  partial[wave][lane] = acc;
  __syncthreads();
  for (int slot = threadIdx.x; slot < C::kCB * 64 * 4; slot += C::kThreads) {
    const int e = slot & 3, l = (slot >> 2) & 63, b = slot >> 8;
    const int out_row = l & 15;                                       // batch row m
    const int out_col = blockIdx.x * 16 * C::kCB + b * 16 + (l >> 4) * 4 + e;  // channel n
    if (out_row >= m || out_col >= n) continue;
    float sum = partial[b][l][e];
#pragma unroll
    for (int v = 1; v < C::kS; ++v) sum += partial[v * C::kCB + b][l][e];
    out[int64_t(out_row) * n + out_col] = uint16_t(f32_to_bf16(sum));
  }
}


// ---------------------------------------------------------------------------------
// Small-batch variant: x resident in LDS, W streamed with a rolling per-wave window.
//
// A workgroup owns one block of 16 channels and kS waves; wave r sums K range r. The
// LDS holds x[0:m, :] as rows of kblocks 128-byte blocks (16-byte chunks XOR-swizzled
// by row & 7), copied once by buffer_load ... lds. Each wave keeps kAhead 64-byte K
// blocks of its W rows in flight and refills a slot right after its MFMAs, so the
// memory pipe never drains between stages:
//  * every wait is explicit and partial: the x copies are issued before the W
//    prologue and waited for with vmcnt(kAhead), then a bare s_barrier (no fence, so
//    the W loads stay in flight); inside the loop each slot waits for vmcnt(kAhead-1);
//  * the loop has no early exit and a scheduling barrier after each slot, so the
//    compiler neither sinks refills behind a branch nor hoists later slots' MFMAs
//    above earlier slots' refills;
//  * slots past the wave's K range load nothing (range-checked offset) and skip their
//    MFMAs on a wave-uniform branch;
//  * the channel scale is read by a range-checked buffer load (zero past N), so no
//    branch forces a wait before the first W load is issued.
// Batch rows past m read x row m-1 and channels past N re-read row N-1: both feed only
// MFMA output rows/columns that are never stored, so no zero padding is needed. x
// chunks past K are copied as zeros, which also cancels the next row's bytes that a
// K tail (K % 64 != 0) reads into the last block.
template <int kS_, int kAhead_, int kWavesPerEU_>
struct ResidentConfig {
  static constexpr int kS = kS_, kAhead = kAhead_;
  static constexpr int kWavesPerEU = kWavesPerEU_;  // 8: at most 64 VGPRs, 32 waves per CU
  static constexpr int kThreads = 64 * kS;
};

__host__ __device__ inline int resident_lds_bytes(int m, int k) {
  return m * ((k + 63) / 64) * 128 + 1024;  // + one spill KiB for the last copy
}

template <class C>
__global__ void __launch_bounds__(C::kThreads, C::kWavesPerEU) channel_gemv_resident_kernel(
    const uint16_t* __restrict__ x, const int8_t* __restrict__ w,
    const uint16_t* __restrict__ scale, uint16_t* __restrict__ out, int m, int n, int k) {
  extern __shared__ __attribute__((aligned(1024))) char xs_raw[];
  __shared__ f32x4 partial[C::kS][64];
  const lds_char* xs = (const lds_char*)xs_raw;

  const int lane = threadIdx.x & 63;
  const int range = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row = lane & 15, group = lane >> 4;
  const int channel = blockIdx.x * 16 + row;

  const auto w_rsrc = make_rsrc(w, uint32_t(n) * uint32_t(k));
  const auto x_rsrc = make_rsrc(x, uint32_t(m) * uint32_t(k) * 2u);
  const auto s_rsrc = make_rsrc(scale, uint32_t(n) * 2u);
  const uint32_t s_bits = __builtin_amdgcn_raw_buffer_load_b16(s_rsrc, uint32_t(channel) * 2u, 0, 0);
  const uint32_t w_lane = uint32_t(min(channel, n - 1)) * uint32_t(k) + uint32_t(group * 16);
  const int kblocks = (k + 63) / 64;
  const int range_len = (kblocks + C::kS - 1) / C::kS;
  const int kb_first = range * range_len;
  const int kend = min(kb_first + range_len, kblocks);
  const int groups = (range_len + C::kAhead - 1) / C::kAhead;

  // x copy: 16-byte unit u of LDS row r holds global chunk (u % 8) ^ (r & 7) of block
  // u / 8. The last copy may spill up to 1 KiB past the rows, writing zeros.
  const int row_units = kblocks * 8;
  const int units = m * row_units;
  for (int u0 = range * 64; u0 < units; u0 += C::kThreads) {
    const int u = u0 + lane;
    const int r = u / row_units, within = u % row_units;
    const int kb = within >> 3, c = (within & 7) ^ (r & 7);
    const bool valid = u < units && kb * 64 + c * 8 < k;
    copy16(x_rsrc, reinterpret_cast<lds_void*>((lds_char*)xs_raw + u0 * 16),
           valid ? uint32_t(r) * uint32_t(k) * 2u + uint32_t(kb * 128 + c * 16) : kOutOfRange);
  }

  // W prologue: slots 0 .. kAhead-1, in slot order.
  u32x4 wv[C::kAhead];
#pragma unroll
  for (int a = 0; a < C::kAhead; ++a) {
    const int kb = kb_first + a;
    wv[a] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                          w_rsrc, kb < kend ? w_lane + uint32_t(kb * 64) : kOutOfRange, 0, 0));
    __builtin_amdgcn_sched_barrier(0);
  }
  waitcnt<vmcnt_imm(C::kAhead)>();  // the scale and this wave's x copies have landed
  workgroup_barrier();              // every wave's x copies have landed

  const float s = bf16_to_f32(s_bits);
  const int xr = min(row, m - 1);
  const lds_char* x_lane = xs + xr * kblocks * 128 + kb_first * 128;
  const int swz0 = ((2 * group) ^ (xr & 7)) * 16, swz1 = ((2 * group + 1) ^ (xr & 7)) * 16;
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int g = 0; g < groups; ++g) {
#pragma unroll
    for (int a = 0; a < C::kAhead; ++a) {
      const int slot = g * C::kAhead + a;   // wave-uniform
      const int kb = kb_first + slot;
      waitcnt<vmcnt_imm(C::kAhead - 1)>();  // slot a's W has landed
      if (kb < kend) {
        const lds_char* xb = x_lane + slot * 128;
        const u32x4 x0 = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(xb + swz0);
        const u32x4 x1 = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(xb + swz1);
        const u32x4 wq = wv[a];
        const u32x2 d0 = dequant4(wq[0], s), d1 = dequant4(wq[1], s);
        const u32x2 d2 = dequant4(wq[2], s), d3 = dequant4(wq[3], s);
        acc = mfma_bf16(u32x4{d0[0], d0[1], d1[0], d1[1]}, x0, acc);
        acc = mfma_bf16(u32x4{d2[0], d2[1], d3[0], d3[1]}, x1, acc);
      }
      const int next = kb + C::kAhead;
      wv[a] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                            w_rsrc, next < kend ? w_lane + uint32_t(next * 64) : kOutOfRange, 0, 0));
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  waitcnt<vmcnt_imm(0)>();  // drain the trailing (out-of-range) loads before exit

  partial[range][lane] = acc;
  __syncthreads();
  for (int slot = threadIdx.x; slot < 64 * 4; slot += C::kThreads) {
    const int e = slot & 3, l = slot >> 2;
    const int out_row = l & 15;
    const int out_col = blockIdx.x * 16 + (l >> 4) * 4 + e;
    if (out_row >= m || out_col >= n) continue;
    float sum = partial[0][l][e];
#pragma unroll
    for (int v = 1; v < C::kS; ++v) sum += partial[v][l][e];
    out[int64_t(out_row) * n + out_col] = uint16_t(f32_to_bf16(sum));
  }
}

// ---------------------------------------------------------------------------------
// Persistent variant of the resident kernel, for batches whose x fills half the LDS or
// more (one workgroup per CU, so it runs 16 waves, one per K range). Copying x per block of 16 channels would then cost each
// CU a serial x copy per block; here each workgroup copies x once and walks the channel
// blocks blockIdx.x, blockIdx.x + gridDim.x, ... Each wave's W window runs across block
// boundaries: slot f of the flattened sequence (local block f / spb, K slot f % spb, spb
// = the padded slots per block) is refilled with slot f + kAhead, so the loads of the
// next block are in flight while a block's partial sums are reduced. The per-block
// arithmetic and summation order are those of the resident kernel, so the bits are too.
template <class C>
__global__ void __launch_bounds__(C::kThreads, C::kWavesPerEU) channel_gemv_persistent_kernel(
    const uint16_t* __restrict__ x, const int8_t* __restrict__ w,
    const uint16_t* __restrict__ scale, uint16_t* __restrict__ out, int m, int n, int k) {
  extern __shared__ __attribute__((aligned(1024))) char xs_raw[];
  __shared__ f32x4 partial[C::kS][64];
  const lds_char* xs = (const lds_char*)xs_raw;

  const int lane = threadIdx.x & 63;
  const int range = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row = lane & 15, group = lane >> 4;
  const int nblocks = (n + 15) / 16;
  const int nlocal = (nblocks - int(blockIdx.x) + int(gridDim.x) - 1) / int(gridDim.x);

  const auto w_rsrc = make_rsrc(w, uint32_t(n) * uint32_t(k));
  const auto x_rsrc = make_rsrc(x, uint32_t(m) * uint32_t(k) * 2u);
  const auto s_rsrc = make_rsrc(scale, uint32_t(n) * 2u);
  const int kblocks = (k + 63) / 64;
  const int range_len = (kblocks + C::kS - 1) / C::kS;
  const int kb_first = range * range_len;
  const int kend = min(kb_first + range_len, kblocks);
  const int groups = (range_len + C::kAhead - 1) / C::kAhead;
  const int spb = groups * C::kAhead;  // slots per block (wave-uniform)

  // Lane offset of W for local block lb; channels past N re-read row N-1 (their outputs
  // are never stored).
  auto w_lane = [&] __device__(int lb) __attribute__((always_inline)) {
    const int channel = (int(blockIdx.x) + lb * int(gridDim.x)) * 16 + row;
    return uint32_t(min(channel, n - 1)) * uint32_t(k) + uint32_t(group * 16);
  };
  auto w_offset = [&] __device__(int f) __attribute__((always_inline)) {
    const int lb = f / spb;
    const int kb = kb_first + (f - lb * spb);
    return lb < nlocal && kb < kend ? w_lane(lb) + uint32_t(kb * 64) : kOutOfRange;
  };
  auto scale_bits = [&] __device__(int lb) __attribute__((always_inline)) {
    const int channel = (int(blockIdx.x) + lb * int(gridDim.x)) * 16 + row;
    return __builtin_amdgcn_raw_buffer_load_b16(
        s_rsrc, lb < nlocal ? uint32_t(channel) * 2u : kOutOfRange, 0, 0);
  };

  // x copy, as in the resident kernel.
  const int row_units = kblocks * 8;
  const int units = m * row_units;
  for (int u0 = range * 64; u0 < units; u0 += C::kThreads) {
    const int u = u0 + lane;
    const int r = u / row_units, within = u % row_units;
    const int kb = within >> 3, c = (within & 7) ^ (r & 7);
    const bool valid = u < units && kb * 64 + c * 8 < k;
    copy16(x_rsrc, reinterpret_cast<lds_void*>((lds_char*)xs_raw + u0 * 16),
           valid ? uint32_t(r) * uint32_t(k) * 2u + uint32_t(kb * 128 + c * 16) : kOutOfRange);
  }
  uint32_t s_next = scale_bits(0);
  u32x4 wv[C::kAhead];
#pragma unroll
  for (int a = 0; a < C::kAhead; ++a) {
    wv[a] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, w_offset(a), 0, 0));
    __builtin_amdgcn_sched_barrier(0);
  }
  waitcnt<vmcnt_imm(C::kAhead)>();  // the first scale and this wave's x copies have landed
  workgroup_barrier();              // every wave's x copies have landed

  const int xr = min(row, m - 1);
  const lds_char* x_lane = xs + xr * kblocks * 128 + kb_first * 128;
  const int swz0 = ((2 * group) ^ (xr & 7)) * 16, swz1 = ((2 * group + 1) ^ (xr & 7)) * 16;
  for (int lb = 0; lb < nlocal; ++lb) {
    const float s = bf16_to_f32(s_next);
    s_next = scale_bits(lb + 1);  // in flight during this block
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int g = 0; g < groups; ++g) {
#pragma unroll
      for (int a = 0; a < C::kAhead; ++a) {
        const int slot = g * C::kAhead + a;   // wave-uniform
        const int kb = kb_first + slot;
        waitcnt<vmcnt_imm(C::kAhead - 1)>();  // slot a's W has landed
        if (kb < kend) {
          const lds_char* xb = x_lane + slot * 128;
          const u32x4 x0 = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(xb + swz0);
          const u32x4 x1 = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(xb + swz1);
          const u32x4 wq = wv[a];
          const u32x2 d0 = dequant4(wq[0], s), d1 = dequant4(wq[1], s);
          const u32x2 d2 = dequant4(wq[2], s), d3 = dequant4(wq[3], s);
          acc = mfma_bf16(u32x4{d0[0], d0[1], d1[0], d1[1]}, x0, acc);
          acc = mfma_bf16(u32x4{d2[0], d2[1], d3[0], d3[1]}, x1, acc);
        }
        wv[a] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                              w_rsrc, w_offset(lb * spb + slot + C::kAhead), 0, 0));
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // Sum the K ranges' partials of this block in a fixed order; the barrier after the
    // stores keeps the next block's partials from overwriting these early.
    partial[range][lane] = acc;
    __builtin_amdgcn_s_waitcnt(lgkmcnt0_imm());
    workgroup_barrier();
    const int block = int(blockIdx.x) + lb * int(gridDim.x);
    for (int e_slot = threadIdx.x; e_slot < 64 * 4; e_slot += C::kThreads) {
      const int e = e_slot & 3, l = e_slot >> 2;
      const int out_row = l & 15;
      const int out_col = block * 16 + (l >> 4) * 4 + e;
      if (out_row >= m || out_col >= n) continue;
      float sum = partial[0][l][e];
#pragma unroll
      for (int v = 1; v < C::kS; ++v) sum += partial[v][l][e];
      out[int64_t(out_row) * n + out_col] = uint16_t(f32_to_bf16(sum));
    }
    __builtin_amdgcn_s_waitcnt(lgkmcnt0_imm());
    workgroup_barrier();
  }
  waitcnt<vmcnt_imm(0)>();  // drain the trailing (out-of-range) loads before exit
}

// ---------------------------------------------------------------------------------
// Row variant for m = 1: whole weight rows per wave, VALU dot products.
//
// Wave g of the grid (G waves) takes rows g, g + G, g + 2G, ...; a lane holds x[16 c'
// + 0..15] for c' = 64 c + lane (kC = ceil(K / 1024) pieces of 1 KiB per row) in
// registers, and each row arrives as kC 16-byte loads per lane, i.e. whole 1 KiB
// pieces of one row per instruction (the order the memory system streams fastest).
// Two rows are in flight: the loads of row r + 2G are issued right after row r's
// products, so at each row the loads issued after its own are the next row's kC + 1
// (codes and scale), and vmcnt(kC + 1) means row r has landed. A lane dequantizes its
// 16 codes exactly as the MFMA kernels do (bf16_rn(code * scale), packed in pairs) and
// feeds them with x to v_dot2_f32_bf16; the 64 lane sums are added in FP32 (DPP within
// rows of 16 lanes, then the four row sums).
// Rows past N load nothing (range-checked offsets) and store nothing. The weight loads are
// nontemporal: every byte is read once (measured on MI355X at K = 5120, N = 17408: 17.0
// against 17.9 us with plain loads, identical outputs; the balanced-span kernel below
// keeps plain loads, since neighbouring waves read the two halves of a 128-byte line
// there and nontemporal loads made it 18% slower). This kernel also runs M = 2..4
// correctly (one dequantization, M dot products) but loses to the span kernel there:
// 19.1 / 22.2 / 24.0 against 18.7 - 18.9 us at K = 5120, N = 17408.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

// The sum of a float over the 64 lanes, in lane 0 (other lanes hold partial sums): DPP
// adds within each row of 16 lanes (quad swaps, then the half-row and row mirrors), then
// the four row sums read out and added. Measured on MI355X against a ds_bpermute
// butterfly (M = 1, identical inputs): 5.48-5.56 against 5.64-5.68 us at N = K = 4096,
// 14.28-14.40 against 14.90-14.91 us at N = K = 8192, level at K = 5120, N = 17408.
template <int kCtrl>
__device__ __forceinline__ float dpp_move(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), kCtrl, 0xF, 0xF, false));
}
__device__ __forceinline__ float wave_sum_to_lane0(float v) {
  v += dpp_move<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v += dpp_move<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v += dpp_move<0x141>(v);  // row_half_mirror
  v += dpp_move<0x140>(v);  // row_mirror: every lane of a row holds the row's sum
  auto lane_value = [&](int l) __attribute__((always_inline)) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
  };
  return (lane_value(0) + lane_value(16)) + (lane_value(32) + lane_value(48));
}

template <int kC>
__global__ void __launch_bounds__(256) channel_gemv_rows_kernel(
    const uint16_t* __restrict__ x, const int8_t* __restrict__ w,
    const uint16_t* __restrict__ scale, uint16_t* __restrict__ out, int n, int k) {
  constexpr int kAhead = 2;  // rows in flight per wave
  const int lane = threadIdx.x & 63;
  const int first = int(blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int stride = int(gridDim.x) * 4;
  const auto w_rsrc = make_rsrc(w, uint32_t(n) * uint32_t(k));
  const auto x_rsrc = make_rsrc(x, uint32_t(k) * 2u);
  const auto s_rsrc = make_rsrc(scale, uint32_t(n) * 2u);
  u32x4 xv[kC][2];
#pragma unroll
  for (int c = 0; c < kC; ++c) {
    const int col = c * 1024 + lane * 16;
#pragma unroll
    for (int h = 0; h < 2; ++h)
      xv[c][h] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                     x_rsrc, col < k ? uint32_t(col * 2 + h * 16) : kOutOfRange, 0, 0));
  }
  u32x4 wr[kAhead][kC];
  uint32_t sr[kAhead];
  auto issue = [&](int row, int slot) __attribute__((always_inline)) {
#pragma unroll
    for (int c = 0; c < kC; ++c) {
      const int col = c * 1024 + lane * 16;
      wr[slot][c] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                     w_rsrc, row < n && col < k ? uint32_t(row) * uint32_t(k) + uint32_t(col)
                                                : kOutOfRange, 0, kBufferLoadNontemporal));
    }
    sr[slot] = __builtin_amdgcn_raw_buffer_load_b16(s_rsrc, row < n ? uint32_t(row) * 2u
                                                                   : kOutOfRange, 0, 0);
  };
#pragma unroll
  for (int s = 0; s < kAhead; ++s) issue(first + s * stride, s);
  for (int row0 = first; row0 < n; row0 += kAhead * stride) {  // uniform over the wave
#pragma unroll
    for (int s = 0; s < kAhead; ++s) {
      const int row = row0 + s * stride;
      waitcnt<vmcnt_imm((kAhead - 1) * (kC + 1))>();  // row `row` has landed
      const float sc = bf16_to_f32(sr[s]);
      float acc = 0.f;
#pragma unroll
      for (int c = 0; c < kC; ++c)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t word = wr[s][c][j];
          const uint32_t p01 = pack_bf16x2(float(int8_t(word)) * sc, float(int8_t(word >> 8)) * sc);
          const uint32_t p23 =
              pack_bf16x2(float(int8_t(word >> 16)) * sc, float(int8_t(word >> 24)) * sc);
          acc = dot2_bf16(p01, xv[c][j >> 1][2 * (j & 1)], acc);
          acc = dot2_bf16(p23, xv[c][j >> 1][2 * (j & 1) + 1], acc);
        }
      issue(row + kAhead * stride, s);
      __builtin_amdgcn_sched_barrier(0);
      const float total = wave_sum_to_lane0(acc);
      if (lane == 0 && row < n) out[row] = uint16_t(f32_to_bf16(total));
    }
  }
  waitcnt<vmcnt_imm(0)>();  // drain the trailing (out-of-range) loads before exit
}

template <int kC>
hipError_t run_rows(const void* x, const int8_t* w, const void* scale, void* out, int n, int k,
                    int cus, hipStream_t stream) {
  // Two waves per SIMD (measured best at N = 4096 .. 17408, K = 4096 .. 8192).
  const int grid = max(1, min(cus * 2, (n + 3) / 4));
  channel_gemv_rows_kernel<kC><<<grid, 256, 0, stream>>>(
      static_cast<const uint16_t*>(x), w, static_cast<const uint16_t*>(scale),
      static_cast<uint16_t*>(out), n, k);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------
// Balanced-span variant: one 16-wave workgroup per CU, x in registers.
//
// Workgroup b owns the channel span [b * span, (b + 1) * span) with span = ceil(N /
// grid), so every CU streams the same number of weight bytes (N = 17408 on 256 CUs: 68
// channels, 348 KiB each) and no CU waits on a second round. The span is walked in
// blocks of 16 channels; the last block's rows past the span load nothing (range-checked
// offsets) and are not stored. Wave r sums K range r (kSpb 64-element blocks at most);
// its x fragments for that range (x[0:16, range] as MFMA B operands, rows past m zero)
// are loaded once into kSpb * 8 registers and reused for every block, so x needs no
// LDS and M = 16 costs what M = 1 does.
//  * W streams one block ahead: after a slot's MFMAs, the wave issues that slot's load
//    for the next block, and at the start of a block the next block's channel scale.
//    Loads retire in issue order, so at slot s of block lb the loads issued after
//    W(lb, s) are the rest of block lb, the scale of lb + 1 and the first s slots of lb
//    + 1: vmcnt(kSpb) before a slot means its W has landed, and vmcnt(kSpb + 1) at the
//    start of a block, after the next scale is issued, means this block's scale has.
//    The prologue issues x, the scale of block 0 and W(0, *), which gives the same
//    counts. The last block's loads for the block after it are out of range (no
//    memory traffic) and are drained before exit.
//  * Each block's 16 per-range partial sums go to LDS (kBatch blocks' worth); after
//    every kBatch blocks and after the last, one barrier pair adds them in range order,
//    rounds to BF16 and stores, so the waves synchronise once per kBatch blocks.
template <int kSpb_>
struct SpanConfig {
  static constexpr int kS = 16;       // waves, one K range each
  static constexpr int kSpb = kSpb_;  // 64-element K blocks per range
  static constexpr int kBatch = 8;    // blocks per partial-sum reduction (128 KiB of LDS)
  static constexpr int kThreads = 64 * kS;
  static_assert(kSpb + 1 <= 63, "vmcnt holds 6 bits");
};

template <class C>
__global__ void __launch_bounds__(C::kThreads) channel_gemv_span_kernel(
    const uint16_t* __restrict__ x, const int8_t* __restrict__ w,
    const uint16_t* __restrict__ scale, uint16_t* __restrict__ out, int m, int n, int k,
    int span) {
  __shared__ f32x4 partial[C::kBatch][C::kS][64];
  const int c0 = int(blockIdx.x) * span;
  if (c0 >= n) return;  // uniform over the workgroup
  const int c_end = min(c0 + span, n);
  const int nlocal = (c_end - c0 + 15) / 16;

  const int lane = threadIdx.x & 63;
  const int range = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row = lane & 15, group = lane >> 4;
  const int kblocks = (k + 63) / 64;
  const int range_len = (kblocks + C::kS - 1) / C::kS;  // <= kSpb (host-checked)
  const int kb_first = range * range_len;
  const int my_slots = max(0, min(kb_first + range_len, kblocks) - kb_first);

  const auto w_rsrc = make_rsrc(w, uint32_t(n) * uint32_t(k));
  const auto x_rsrc = make_rsrc(x, uint32_t(m) * uint32_t(k) * 2u);
  const auto s_rsrc = make_rsrc(scale, uint32_t(n) * 2u);

  // Byte offset of this lane's 16 codes of block lb, slot s (kOutOfRange: load zeros).
  auto w_offset = [&](int lb, int s) __attribute__((always_inline)) {
    const int channel = c0 + lb * 16 + row;
    const int col = (kb_first + s) * 64 + group * 16;
    const bool valid = channel < c_end && s < my_slots && col < k;
    return valid ? uint32_t(channel) * uint32_t(k) + uint32_t(col) : kOutOfRange;
  };
  auto load_scale = [&](int lb) __attribute__((always_inline)) {
    const int channel = c0 + lb * 16 + row;
    return __builtin_amdgcn_raw_buffer_load_b16(
        s_rsrc, channel < c_end ? uint32_t(channel) * 2u : kOutOfRange, 0, 0);
  };

  // x fragments: lane (row, group) holds x[row, kb * 64 + 16 * group + 8 * h + 0..7].
  u32x4 xf[C::kSpb][2];
#pragma unroll
  for (int s = 0; s < C::kSpb; ++s) {
    const int col = (kb_first + s) * 64 + group * 16;
    const bool valid = row < m && s < my_slots && col < k;
    const uint32_t base = uint32_t(row) * uint32_t(k) * 2u + uint32_t(col) * 2u;
#pragma unroll
    for (int h = 0; h < 2; ++h)
      xf[s][h] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(x_rsrc, valid ? base + 16u * h : kOutOfRange,
                                                       0, 0));
  }
  uint32_t s_next = load_scale(0);
  __builtin_amdgcn_sched_barrier(0);
  u32x4 wv[C::kSpb];
#pragma unroll
  for (int s = 0; s < C::kSpb; ++s) {
    wv[s] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, w_offset(0, s), 0, 0));
    __builtin_amdgcn_sched_barrier(0);
  }

  // Adds the partials of local blocks [lb0, lb0 + count) and stores them.
  auto reduce = [&](int lb0, int count) __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(lgkmcnt0_imm());
    workgroup_barrier();
    for (int i = threadIdx.x; i < count * 256; i += C::kThreads) {
      const int b = i >> 8, e = i & 3, l = (i >> 2) & 63;
      const int out_row = l & 15;
      const int out_col = c0 + (lb0 + b) * 16 + (l >> 4) * 4 + e;
      if (out_row < m && out_col < c_end) {
        float sum = partial[b][0][l][e];
#pragma unroll
        for (int v = 1; v < C::kS; ++v) sum += partial[b][v][l][e];
        out[int64_t(out_row) * n + out_col] = uint16_t(f32_to_bf16(sum));
      }
    }
    __builtin_amdgcn_s_waitcnt(lgkmcnt0_imm());
    workgroup_barrier();
  };

  for (int lb = 0; lb < nlocal; ++lb) {
    const float sc = bf16_to_f32(s_next);
    s_next = load_scale(lb + 1);
    __builtin_amdgcn_sched_barrier(0);
    waitcnt<vmcnt_imm(C::kSpb + 1)>();  // the scale of block lb has landed
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < C::kSpb; ++s) {
      waitcnt<vmcnt_imm(C::kSpb)>();  // W(lb, s) has landed
      if (s < my_slots) {
        const u32x4 wq = wv[s];
        const u32x2 d0 = dequant4(wq[0], sc), d1 = dequant4(wq[1], sc);
        const u32x2 d2 = dequant4(wq[2], sc), d3 = dequant4(wq[3], sc);
        acc = mfma_bf16(u32x4{d0[0], d0[1], d1[0], d1[1]}, xf[s][0], acc);
        acc = mfma_bf16(u32x4{d2[0], d2[1], d3[0], d3[1]}, xf[s][1], acc);
      }
      wv[s] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, w_offset(lb + 1, s), 0, 0));
      __builtin_amdgcn_sched_barrier(0);
    }
    partial[lb % C::kBatch][range][lane] = acc;
    if (lb % C::kBatch == C::kBatch - 1 || lb + 1 == nlocal)  // uniform
      reduce(lb / C::kBatch * C::kBatch, lb % C::kBatch + 1);
  }
  waitcnt<vmcnt_imm(0)>();  // drain the trailing (out-of-range) loads before exit
}

template <class C>
hipError_t run_span(const void* x, const int8_t* w, const void* scale, void* out, int m, int n,
                    int k, int cus, hipStream_t stream) {
  const int grid = min(cus, (n + 15) / 16);
  const int span = (n + grid - 1) / grid;
  channel_gemv_span_kernel<C><<<grid, C::kThreads, 0, stream>>>(
      static_cast<const uint16_t*>(x), w, static_cast<const uint16_t*>(scale),
      static_cast<uint16_t*>(out), m, n, k, span);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------
// Interleaved quad-block variant (K in [4096, 8192], m <= 8): blocks of 4 channels on
// v_mfma_f32_4x4x4bf16_1k.
//
// The 4x4x4 MFMA computes 16 independent 4x4 products. Lane 4q + i supplies row i of
// block q of A and lane 4q + j column j of block q of B; the result of block q lands in
// lane 4q + j, element i. Here A is W (row i = channel i of a 4-channel block) and B is
// x (column j = batch row 4g + j of batch group g), and the 16 MFMA blocks q take 16
// disjoint slices of the K range, so one 16-byte load per lane reads 4 channels x 256
// contiguous bytes. That is a plain weight stream: each instruction fetches whole
// 128-byte lines, where the 16 x 16 MFMA layout needs 16 channels x 64 bytes. The
// price is that every output is a sum over the 16 lane blocks, and that m > 4 needs
// one MFMA per batch group.
//  * Blocks are dealt to workgroups round-robin: workgroup b takes blocks b, b + grid,
//    b + 2 grid, ... (one 16-wave workgroup per CU), so at any time the chip reads one
//    contiguous window of the weights, which measured faster than contiguous per-CU
//    spans (a load-only copy of this layout streamed the configs[1] weights in 14.7
//    against 16.2 us with spans), and N = 17408 gives every CU the same 17 blocks.
//  * Wave r sums K range r (kU units of 64 elements; loads of 16, 8 and 4 bytes per lane
//    cover 4, 2 and 1 units). Its x operands for that range stay in registers.
//  * W streams one block ahead: after a load's MFMAs, the wave issues the same load for
//    its next block, and the next block's channel scale at the start of a block. Loads
//    retire in issue order, so before load e of block t the loads issued after it are
//    the rest of block t, the next scale and the first e loads of block t + 1:
//    vmcnt(kLoads) means it has landed; vmcnt(kLoads + 1) at the start of a block, after
//    the next scale is issued, means this block's scale has.
//  * After a block, two DPP row rotations add the four lane blocks of each 16-lane row;
//    lanes 16R + j (j < 4) then hold the row-R partials of batch row j for the 4
//    channels and store them to LDS. kBatch blocks of partials fit in 128 KiB, so the
//    waves meet at a barrier once per kBatch blocks (at N = 17408 only at the end),
//    where 4 threads per (block, batch row) add the 16 waves' partials of one R each
//    and a quad DPP reduction adds the four R. The order of every sum is fixed.
template <int kU_, int kG_, bool kNt_ = false>
struct QuadConfig {
  static constexpr int kU = kU_;  // 64-element K units per wave
  static constexpr int kG = kG_;  // batch groups of 4 rows
  static constexpr int kS = 16;   // waves, one K range each
  static constexpr int kThreads = 64 * kS;
  static constexpr int kN4 = kU / 4, kHas2 = (kU % 4) >= 2, kHas1 = kU % 2;
  static constexpr int kLoads = kN4 + kHas2 + kHas1;  // W loads per block and wave
  static constexpr int kBatch = 32 / kG;              // blocks of partials in LDS
  // Nontemporal weight loads where every wave's K range and every row are whole 128-byte
  // lines (K % 2048 == 0, so kU is even and rows start on lines). With kU odd (K = 5120:
  // 320-byte ranges) neighbouring waves read the two halves of a line, and a nontemporal
  // first half evicts the line before the second is read. Measured on MI355X (same
  // process, identical outputs), nontemporal against
  // plain: K = 8192, N = 8192: m = 2 / 4 / 8 12.9-13.9 / 13.6-13.7 / 15.9-16.3 against
  // 14.0-14.5 / 14.0-14.4 / 16.6-16.7 us; N = 28672: 35.5-35.7 / 37.4-37.5 / 41.3-43.0
  // against 39.6 / 39.1-39.4 / 44.0-44.8 us; K = 4096 the same within 0.2 us; K = 5120,
  // N = 17408: m = 2 / 4 17.1-17.2 / 17.8-18.1 against 15.8 / 16.4-16.5 us.
  static constexpr bool kNt = kNt_;
  static_assert(kU >= 4 && kU <= 8, "K ranges of 256 to 512 elements");
  static_assert(!kNt || kU % 2 == 0, "nontemporal loads need whole-line K ranges");
  static_assert(kLoads + 1 <= 63, "vmcnt holds 6 bits");
};

typedef short s16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 mfma4x4_bf16(u32x2 a, u32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(s16x4, a),
                                                 __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
}

template <int kCtrl>
__device__ __forceinline__ float dpp_rotate(float x) {  // every lane's source is valid
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), kCtrl, 0xF, 0xF, true));
}

template <class C>
__global__ void __launch_bounds__(C::kThreads) channel_gemv_quad_kernel(
    const uint16_t* __restrict__ x, const int8_t* __restrict__ w,
    const uint16_t* __restrict__ scale, uint16_t* __restrict__ out, int m, int n, int k) {
  __shared__ f32x4 partial[C::kBatch][C::kS][C::kG][16];
  const int nblk = (n + 3) >> 2;
  const int grid = int(gridDim.x), b0 = int(blockIdx.x);
  if (b0 >= nblk) return;  // uniform over the workgroup
  const int nlocal = (nblk - b0 + grid - 1) / grid;

  const int lane = threadIdx.x & 63;
  const int range = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int q = lane >> 2, i = lane & 3;
  const int kc0 = range * C::kU * 64;

  const auto w_rsrc = make_rsrc(w, uint32_t(n) * uint32_t(k));
  const auto x_rsrc = make_rsrc(x, uint32_t(m) * uint32_t(k) * 2u);
  const auto s_rsrc = make_rsrc(scale, uint32_t(n) * 2u);

  // First column of this lane's codes in load e (16, 8 or 4 of them).
  auto col_of = [&](int e) __attribute__((always_inline)) -> int {
    if (e < C::kN4) return kc0 + 256 * e + 16 * q;
    if (C::kHas2 && e == C::kN4) return kc0 + 256 * C::kN4 + 8 * q;
    return kc0 + 256 * C::kN4 + 128 * C::kHas2 + 4 * q;
  };
  // K % 16 == 0, so each load is wholly inside or wholly past its row.
  auto w_offset = [&](int lb, int e) __attribute__((always_inline)) -> uint32_t {
    const int channel = 4 * (b0 + lb * grid) + i, col = col_of(e);
    return lb < nlocal && channel < n && col < k
               ? uint32_t(channel) * uint32_t(k) + uint32_t(col) : kOutOfRange;
  };
  auto load_scale = [&](int lb) __attribute__((always_inline)) -> uint32_t {
    const int channel = 4 * (b0 + lb * grid) + i;
    return __builtin_amdgcn_raw_buffer_load_b16(
        s_rsrc, lb < nlocal && channel < n ? uint32_t(channel) * 2u : kOutOfRange, 0, 0);
  };

  // x operands: xs[g][u] = x[4g + i, the 4 columns lane block q takes of unit u].
  u32x2 xs[C::kG][C::kU];
#pragma unroll
  for (int g = 0; g < C::kG; ++g) {
    const int row = 4 * g + i;
#pragma unroll
    for (int e = 0; e < C::kLoads; ++e) {
      const int col = col_of(e);
      const bool valid = row < m && col < k;
      const uint32_t base = (uint32_t(row) * uint32_t(k) + uint32_t(col)) * 2u;
      auto load16 = [&](uint32_t extra) __attribute__((always_inline)) {
        return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                             x_rsrc, valid ? base + extra : kOutOfRange, 0, 0));
      };
      if (e < C::kN4) {
        const u32x4 lo = load16(0), hi = load16(16);
        xs[g][4 * e] = u32x2{lo[0], lo[1]};
        xs[g][4 * e + 1] = u32x2{lo[2], lo[3]};
        xs[g][4 * e + 2] = u32x2{hi[0], hi[1]};
        xs[g][4 * e + 3] = u32x2{hi[2], hi[3]};
      } else if (C::kHas2 && e == C::kN4) {
        const u32x4 v = load16(0);
        xs[g][4 * C::kN4] = u32x2{v[0], v[1]};
        xs[g][4 * C::kN4 + 1] = u32x2{v[2], v[3]};
      } else {
        xs[g][C::kU - 1] = __builtin_bit_cast(
            u32x2, __builtin_amdgcn_raw_buffer_load_b64(x_rsrc, valid ? base : kOutOfRange, 0, 0));
      }
    }
  }
  uint32_t s_next = load_scale(0);
  __builtin_amdgcn_sched_barrier(0);
  u32x4 w4[C::kN4];
  u32x2 w2;
  uint32_t w1;
  constexpr int kPolicy = C::kNt ? kBufferLoadNontemporal : 0;
  auto issue = [&](int lb, int e) __attribute__((always_inline)) {
    if (e < C::kN4)
      w4[e] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, w_offset(lb, e), 0, kPolicy));
    else if (C::kHas2 && e == C::kN4)
      w2 = __builtin_bit_cast(
          u32x2, __builtin_amdgcn_raw_buffer_load_b64(w_rsrc, w_offset(lb, e), 0, kPolicy));
    else
      w1 = __builtin_amdgcn_raw_buffer_load_b32(w_rsrc, w_offset(lb, e), 0, kPolicy);
  };
#pragma unroll
  for (int e = 0; e < C::kLoads; ++e) {
    issue(0, e);
    __builtin_amdgcn_sched_barrier(0);
  }

  // Adds and stores the partials of local blocks [lb0, lb0 + count). Item (block, batch
  // row, R) adds the 16 ranges' row-R partials (4 channels); the 4 R of an item are the 4
  // lanes of a quad.
  auto reduce = [&](int lb0, int count) __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(lgkmcnt0_imm());
    workgroup_barrier();
    const int items = count * m * 4;  // <= 512
    const int item = int(threadIdx.x), r = item & 3, batch = (item >> 2) % m,
              b = (item >> 2) / m;
    f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
    if (item < items) {
#pragma unroll
      for (int v = 0; v < C::kS; ++v) sum += partial[b][v][batch >> 2][4 * r + (batch & 3)];
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      sum[c] += dpp_rotate<0xB1>(sum[c]);  // quad_perm [1, 0, 3, 2]
      sum[c] += dpp_rotate<0x4E>(sum[c]);  // quad_perm [2, 3, 0, 1]
    }
    if (item < items && r == 0) {
      const int channel = 4 * (b0 + (lb0 + b) * grid);
      uint16_t* o = out + int64_t(batch) * n + channel;
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (channel + c < n) o[c] = uint16_t(f32_to_bf16(sum[c]));
    }
    __builtin_amdgcn_s_waitcnt(lgkmcnt0_imm());
    workgroup_barrier();
  };

  for (int lb = 0; lb < nlocal; ++lb) {
    const float sc = bf16_to_f32(s_next);
    s_next = load_scale(lb + 1);
    __builtin_amdgcn_sched_barrier(0);
    waitcnt<vmcnt_imm(C::kLoads + 1)>();  // the scale of block lb has landed
    f32x4 acc[C::kG];
#pragma unroll
    for (int g = 0; g < C::kG; ++g) acc[g] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int e = 0; e < C::kLoads; ++e) {
      waitcnt<vmcnt_imm(C::kLoads)>();  // W(lb, e) has landed
      auto step = [&](uint32_t word, int unit) __attribute__((always_inline)) {
        const u32x2 a = dequant4(word, sc);
#pragma unroll
        for (int g = 0; g < C::kG; ++g) acc[g] = mfma4x4_bf16(a, xs[g][unit], acc[g]);
      };
      if (e < C::kN4) {
#pragma unroll
        for (int s = 0; s < 4; ++s) step(w4[e][s], 4 * e + s);
      } else if (C::kHas2 && e == C::kN4) {
        step(w2[0], 4 * C::kN4);
        step(w2[1], 4 * C::kN4 + 1);
      } else {
        step(w1, C::kU - 1);
      }
      issue(lb + 1, e);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int g = 0; g < C::kG; ++g)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        acc[g][c] += dpp_rotate<0x128>(acc[g][c]);  // row_ror:8
        acc[g][c] += dpp_rotate<0x124>(acc[g][c]);  // row_ror:4
      }
    if ((lane & 15) < 4) {
#pragma unroll
      for (int g = 0; g < C::kG; ++g)
        partial[lb % C::kBatch][range][g][(lane >> 4) * 4 + (lane & 3)] = acc[g];
    }
    if (lb % C::kBatch == C::kBatch - 1 || lb + 1 == nlocal)  // uniform
      reduce(lb / C::kBatch * C::kBatch, lb % C::kBatch + 1);
  }
  waitcnt<vmcnt_imm(0)>();  // drain the trailing (out-of-range) loads before exit
}

template <int kU, bool kNt = false>
hipError_t run_quad(const void* x, const int8_t* w, const void* scale, void* out, int m, int n,
                    int k, int cus, hipStream_t stream) {
  const int grid = min(cus, (n + 3) / 4);
  auto launch = [&](auto kernel) {
    kernel<<<grid, 1024, 0, stream>>>(static_cast<const uint16_t*>(x), w,
                                      static_cast<const uint16_t*>(scale),
                                      static_cast<uint16_t*>(out), m, n, k);
    return hipGetLastError();
  };
  if (m <= 4) return launch(channel_gemv_quad_kernel<QuadConfig<kU, 1, kNt>>);
  return launch(channel_gemv_quad_kernel<QuadConfig<kU, 2, kNt>>);
}

}  // namespace

hipError_t launch_channel_gemv(const void* x, const int8_t* w, const void* scale, void* out,
                               int m, int n, int k, hipStream_t stream) {
  // K <= 8192 and m >= 2: the balanced-span kernel (measured on MI355X at K = 5120, N =
  // 17408: 20.2 - 22.9 us over m = 2 .. 16, against 20.4 - 30.9 us for the kernels below).
  const int cus = device_cu_count();
  // 2 <= m <= 4 with 4096 <= K <= 8192, and 5 <= m <= 8 with 5120 < K <= 8192: the
  // interleaved quad-block kernel (measured at K = 5120, N = 17408: 16.3 / 17.1 us at
  // m = 2 / 4 against 19.6 / 19.9 us for the span kernel; at N = K = 8192, m = 5 .. 8:
  // 14.3 - 15.5 against 21.0 - 21.4 us). At K = 3072, or m = 5 .. 8 with K <= 5120, or m
  // > 8, it loses to the span kernel (one MFMA per 4 batch rows); at m = 1 the row
  // kernel is as fast or faster at N >= 28672.
  if (cus > 0 && k >= 4096 && k <= 8192 && ((m >= 2 && m <= 4) || (m >= 5 && m <= 8 && k > 5120))) {
    if (k % 2048 == 0) {  // whole-line K ranges and rows: nontemporal weight loads
      if (k == 4096) return run_quad<4, true>(x, w, scale, out, m, n, k, cus, stream);
      if (k == 6144) return run_quad<6, true>(x, w, scale, out, m, n, k, cus, stream);
      return run_quad<8, true>(x, w, scale, out, m, n, k, cus, stream);
    }
    switch (((k + 63) / 64 + 15) / 16) {
      case 4: return run_quad<4>(x, w, scale, out, m, n, k, cus, stream);
      case 5: return run_quad<5>(x, w, scale, out, m, n, k, cus, stream);
      case 6: return run_quad<6>(x, w, scale, out, m, n, k, cus, stream);
      case 7: return run_quad<7>(x, w, scale, out, m, n, k, cus, stream);
      default: return run_quad<8>(x, w, scale, out, m, n, k, cus, stream);
    }
  }
  // m = 1, K <= 8192: whole rows on the VALU (measured at K = 5120, N = 17408: 17.9 us
  // against 21.2 us for the resident MFMA kernel under the same C-side launch loop).
  if (m == 1 && cus > 0 && k <= 8192) {
    switch ((k + 1023) / 1024) {
      case 1: return run_rows<1>(x, w, scale, out, n, k, cus, stream);
      case 2: return run_rows<2>(x, w, scale, out, n, k, cus, stream);
      case 3: return run_rows<3>(x, w, scale, out, n, k, cus, stream);
      case 4: return run_rows<4>(x, w, scale, out, n, k, cus, stream);
      case 5: return run_rows<5>(x, w, scale, out, n, k, cus, stream);
      case 6: return run_rows<6>(x, w, scale, out, n, k, cus, stream);
      case 7: return run_rows<7>(x, w, scale, out, n, k, cus, stream);
      default: return run_rows<8>(x, w, scale, out, n, k, cus, stream);
    }
  }
  const int range_len = ((k + 63) / 64 + 15) / 16;
  if (cus > 0 && range_len <= 8 && m >= 2) {
    if (range_len <= 2) return run_span<SpanConfig<2>>(x, w, scale, out, m, n, k, cus, stream);
    if (range_len <= 4) return run_span<SpanConfig<4>>(x, w, scale, out, m, n, k, cus, stream);
    if (range_len <= 5) return run_span<SpanConfig<5>>(x, w, scale, out, m, n, k, cus, stream);
    return run_span<SpanConfig<8>>(x, w, scale, out, m, n, k, cus, stream);
  }
  // Measured on MI355X at K=5120, N=17408: x resident in LDS with 8 K ranges per block of
  // 16 channels and a 10-block window wins while two workgroups fit on a CU (m <= 6:
  // 23.9 / 24.2 us at m = 5 / 6 against 25.2 / 25.4 us for the ring); with one per CU
  // (m = 8: 30.5 against 26.2 us) the ring with 2 channel blocks x 2 K ranges and
  // 4-block stages is faster.
  const int lds = resident_lds_bytes(m, k);
  // At m = 7 (71 KiB) the resident kernel still fits twice per CU but measures slower
  // than the persistent one (25.7 against 24.6 us at m = 8), so it stops at 64 KiB.
  if (lds <= 64 * 1024) {  // plus 8 KiB of static LDS: two workgroups per CU
    using R = ResidentConfig<8, 10, 8>;
    auto kernel = channel_gemv_resident_kernel<R>;
    if (const hipError_t e = prepare_lds<channel_gemv_resident_kernel<R>>(lds); e != hipSuccess)
      return e;
    const int grid = (n + 15) / 16;
    kernel<<<grid, R::kThreads, lds, stream>>>(
        static_cast<const uint16_t*>(x), w, static_cast<const uint16_t*>(scale),
        static_cast<uint16_t*>(out), m, n, k);
    return hipGetLastError();
  }
  // Larger batches while x still fits (m = 7 .. 14 at K = 5120): the persistent kernel,
  // one 16-wave workgroup per CU copying x once, with 5-block windows (at m = 8, 10,
  // 14: 24.2 - 25.0 us, against 28 - 29 us with 8 waves and 16-block windows, and
  // 26 - 27 us for the ring).
  using P = ResidentConfig<16, 5, 4>;
  constexpr int kStaticLds = P::kS * 64 * 16;  // partial sums
  if (lds + kStaticLds <= 160 * 1024 && cus > 0) {
    auto kernel = channel_gemv_persistent_kernel<P>;
    if (const hipError_t e = prepare_lds<channel_gemv_persistent_kernel<P>>(lds); e != hipSuccess)
      return e;
    const int grid = min((n + 15) / 16, cus);
    kernel<<<grid, P::kThreads, lds, stream>>>(
        static_cast<const uint16_t*>(x), w, static_cast<const uint16_t*>(scale),
        static_cast<uint16_t*>(out), m, n, k);
    return hipGetLastError();
  }
  using C = GemvConfig<2, 2, 4>;
  const int grid = (n + 16 * C::kCB - 1) / (16 * C::kCB);
  channel_gemv_kernel<C><<<grid, C::kThreads, 0, stream>>>(
      static_cast<const uint16_t*>(x), w, static_cast<const uint16_t*>(scale),
      static_cast<uint16_t*>(out), m, n, k);
  return hipGetLastError();
}

}  // namespace ci8
