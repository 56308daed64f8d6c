// Grouped W8A16 with GGUF Q8_0 weights (gguf_q8_packed_mm) for gfx950.
//
//   wq[g, n, k]  = bf16_rn( float(code[g, n, k]) * float(scale[g, n, k / 32]) )
//   out[m, g, n] = bf16_rn( sum_k float(x[m, g, k]) * float(wq[g, n, k]) )   (FP32 sums)
//
// The arithmetic of csrc/gguf_q8_packed.cu:176-183 and :230-244 of the reference: the
// original signed codes and FP16 block scales of each 32-value block are multiplied
// (exactly, in FP32: 8-bit by 11-bit significands), rounded once to BF16, and fed with
// the BF16 activations to a BF16 matrix product with FP32 accumulation. The summation
// order is the hardware's, so parity is by tolerance, as in the reference's test
// (tests/test_gguf_q8.py:20-62).
//
// Layout: x BF16 [M, G, K] with independent row and group strides (K contiguous), codes
// INT8 [G, N, K], scales FP16 [G, N, K / 32], out BF16 [M, G, N] contiguous; K % 64 == 0.
//
// Kernels, all on v_mfma_f32_16x16x32_bf16 with the MFMA computing D[n][m] = Wq . x^T
// (a lane holds 4 consecutive channels of one row and stores 8 bytes):
//  * m <= 16, K <= 8192: the balanced-span kernel (the layout of the W8A16 GEMV).
//  * m > 16: 256 x 128 or 128 x 128 tiles of eight waves with an LDS ring of three K
//    stages, codes dequantized once per tile and stage (gguf_q8_large_kernel).
//  * Otherwise (x or the codes beyond a 2 GiB buffer range, or m <= 16 with K > 8192):
//    a BM x 64 tile of four waves, each owning a 16-channel block and BM / 16 row blocks;
//    K advances 64 at a time through two LDS buffers while the next stage's x and codes
//    wait in registers, and the codes are dequantized on their way into LDS.
// Rows past M or N read as zero and are not stored.
#include <atomic>
#include <climits>
#include <type_traits>

#include "ci8_device.h"
#include "launch.h"

namespace ci8 {
namespace {

constexpr int kBK = 64;  // K per stage
constexpr int kBN = 64;  // channels per workgroup

__device__ __forceinline__ f32x4 mfma_bf16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// FP16 bit pattern -> FP32 (exact).
__device__ __forceinline__ float f16_to_f32(uint32_t bits) {
  return float(__builtin_bit_cast(_Float16, uint16_t(bits)));
}

// LDS tiles are [rows][64 BF16] = 128 bytes per row, 16-byte chunks XOR-swizzled by
// row % 8 so the 16 rows of a fragment read at one chunk fall in distinct banks.
__device__ __forceinline__ int tile_offset(int row, int chunk) {
  return row * 128 + ((chunk ^ (row & 7)) * 16);
}

template <int BM>
__global__ void __launch_bounds__(256) gguf_q8_packed_kernel(
    const uint16_t* __restrict__ x, const int8_t* __restrict__ codes,
    const uint16_t* __restrict__ scales, uint16_t* __restrict__ out, int m, int n, int k,
    int groups, int64_t xs, int64_t xg) {
  constexpr int TM = BM / 16;                  // row blocks per wave
  constexpr int kXChunks = BM * kBK / 8;       // 16-byte x chunks per stage
  constexpr int kXPerThread = (kXChunks + 255) / 256;
  __shared__ __attribute__((aligned(16))) char xs_lds[2][BM * 128];
  __shared__ __attribute__((aligned(16))) char ws_lds[2][kBN * 128];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = blockIdx.z;
  const int n0 = blockIdx.x * kBN, m0 = blockIdx.y * BM;
  const int8_t* gcodes = codes + int64_t(g) * n * k;
  const uint16_t* gscales = scales + int64_t(g) * n * (k / 32);

  // Global -> register staging. x: chunk c of the stage is row c / 8, 16-byte chunk c % 8.
  // Codes: thread t takes row t / 4, 16 codes at k offset (t % 4) * 16, and their scale.
  u32x4 xr[kXPerThread];
  u32x4 cr;
  uint32_t sr;
  const int c_row = tid >> 2, c_col = (tid & 3) * 16;
  const bool c_live = n0 + c_row < n;
  auto load = [&](int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kXPerThread; ++i) {
      const int c = i * 256 + tid;
      const int row = c >> 3, chunk = c & 7;
      xr[i] = u32x4{0, 0, 0, 0};
      if (c < kXChunks && m0 + row < m)
        xr[i] = *reinterpret_cast<const u32x4*>(x + int64_t(m0 + row) * xs + int64_t(g) * xg +
                                                 k0 + chunk * 8);
    }
    cr = u32x4{0, 0, 0, 0};
    sr = 0;
    if (c_live) {
      cr = *reinterpret_cast<const u32x4*>(gcodes + int64_t(n0 + c_row) * k + k0 + c_col);
      sr = gscales[int64_t(n0 + c_row) * (k / 32) + (k0 + c_col) / 32];
    }
  };
  // Registers -> LDS buffer b, dequantizing the codes: 16 codes -> 16 BF16 (2 chunks).
  auto store = [&](int b) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kXPerThread; ++i) {
      const int c = i * 256 + tid;
      if (c < kXChunks)
        *reinterpret_cast<u32x4*>(xs_lds[b] + tile_offset(c >> 3, c & 7)) = xr[i];
    }
    const float s = f16_to_f32(sr);
    uint32_t packed[8];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t word = cr[w];
      packed[2 * w] = pack_bf16x2(float(int8_t(word)) * s, float(int8_t(word >> 8)) * s);
      packed[2 * w + 1] = pack_bf16x2(float(int8_t(word >> 16)) * s, float(int8_t(word >> 24)) * s);
    }
    const int chunk = c_col / 8;
    *reinterpret_cast<u32x4*>(ws_lds[b] + tile_offset(c_row, chunk)) =
        u32x4{packed[0], packed[1], packed[2], packed[3]};
    *reinterpret_cast<u32x4*>(ws_lds[b] + tile_offset(c_row, chunk + 1)) =
        u32x4{packed[4], packed[5], packed[6], packed[7]};
  };

  // Wave w owns channel block w (16 channels) and all TM row blocks. Fragment lane
  // layout (16x16x32 BF16 MFMA): row lane % 16, K elements 8 * (lane / 16) .. + 7 of
  // the 32-wide K-step, i.e. 16-byte chunk 4h + lane / 16 of the 64-wide stage.
  const int f_row = lane & 15, f_chunk = lane >> 4;
  f32x4 acc[TM];
#pragma unroll
  for (int j = 0; j < TM; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};

  load(0);
  store(0);
  __syncthreads();
  const int stages = k / kBK;
  for (int t = 0; t < stages; ++t) {
    const int b = t & 1;
    if (t + 1 < stages) load((t + 1) * kBK);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const u32x4 wfrag = *reinterpret_cast<const u32x4*>(
          ws_lds[b] + tile_offset(wave * 16 + f_row, 4 * h + f_chunk));
#pragma unroll
      for (int j = 0; j < TM; ++j) {
        const u32x4 xfrag = *reinterpret_cast<const u32x4*>(
            xs_lds[b] + tile_offset(j * 16 + f_row, 4 * h + f_chunk));
        acc[j] = mfma_bf16(wfrag, xfrag, acc[j]);
      }
    }
    if (t + 1 < stages) store(b ^ 1);  // buffer b ^ 1 was last read in stage t - 1
    __syncthreads();
  }

  // Lane holds D[n][m] for n = 4 * (lane / 16) + e of the wave's channel block and
  // m = lane % 16 of each row block.
  const int col = n0 + wave * 16 + 4 * f_chunk;
  const bool vec = (n & 3) == 0 && (reinterpret_cast<uintptr_t>(out) & 7) == 0;
#pragma unroll
  for (int j = 0; j < TM; ++j) {
    const int row = m0 + j * 16 + f_row;
    if (row >= m) continue;
    uint16_t* dst = out + (int64_t(row) * groups + g) * n + col;
    if (vec && col + 3 < n) {
      *reinterpret_cast<u32x2*>(dst) =
          u32x2{pack_bf16x2(acc[j][0], acc[j][1]), pack_bf16x2(acc[j][2], acc[j][3])};
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (col + e < n) dst[e] = uint16_t(f32_to_bf16(acc[j][e]));
    }
  }
}

// ---------------------------------------------------------------------------------
// Small batches (m <= 16): the balanced-span layout of the W8A16 GEMV (gemv.hip).
//
// Workgroup (b, g) owns channels [b * span, (b + 1) * span) of group g (span = ceil(N /
// spans), spans chosen so that about one workgroup runs per CU), walked in blocks of 16
// channels. Its 16 waves split K into ranges of at most kSpb 64-element blocks; wave r's
// x fragments for its range (x[0:16, g, range] as MFMA B operands, rows past m zero) are
// loaded once into registers. Lane (row, q) of a slot takes the 16 codes at K offset
// 64 kb + 16 q of channel row `row` and their FP16 block scale (the 16 codes lie in one
// 32-value block), dequantizes them exactly as the tile kernel does and feeds two
// v_mfma_f32_16x16x32_bf16. Each slot's two loads for the next block (codes, scale) are
// issued right after its MFMAs, so at slot s of block lb the loads issued after W(lb, s)
// are its scale, the rest of block lb and the first s slots of block lb + 1: 2 kSpb - 1
// in all, and vmcnt(2 kSpb - 2) means both of the slot's loads have landed (the
// prologue issues x, then W and scale of block 0 slot by slot, which gives the same
// counts). The 16 per-range partial sums of up to 8 blocks go to LDS and are added in
// range order with one barrier pair per 8 blocks; the last block's loads for the block
// after it are out of range and drained before exit.
template <int kSpb_>
struct GgufSpanConfig {
  static constexpr int kS = 16;       // waves, one K range each
  static constexpr int kSpb = kSpb_;  // 64-element K blocks per range
  static constexpr int kBatch = 8;    // blocks per partial-sum reduction (128 KiB of LDS)
  static constexpr int kThreads = 64 * kS;
  // A wave's block scales: with kSpb <= 5 the row's 2 kSpb scales of its K range come in
  // one or two loads per block (one b64 / b128, or b128 + b32); at kSpb = 8 a second copy
  // of all 16 would not fit the 128 registers a lane has at 16 waves per CU, so they come
  // as two 16-byte halves.
  static constexpr bool kBlockScales = kSpb <= 5;
  static constexpr int kSLoads = kSpb == 2 || kSpb == 4 ? 1 : 2;
  static_assert(kSpb == 2 || kSpb == 4 || kSpb == 5 || kSpb == 8, "scale load shapes");
  static_assert(kSpb - 1 + kSLoads <= 63, "vmcnt holds 6 bits");
};

template <int kImm>
__device__ __forceinline__ void waitcnt() {
  __builtin_amdgcn_s_waitcnt(kImm);
}

__device__ __forceinline__ void workgroup_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Four INT8 codes -> two packed BF16 pairs bf16_rn(code * s) (exact product, one rounding).
__device__ __forceinline__ u32x2 dequant4(uint32_t word, float s) {
  return u32x2{pack_bf16x2(float(int8_t(word)) * s, float(int8_t(word >> 8)) * s),
               pack_bf16x2(float(int8_t(word >> 16)) * s, float(int8_t(word >> 24)) * s)};
}

template <class C>
__global__ void __launch_bounds__(C::kThreads) gguf_q8_span_kernel(
    const uint16_t* __restrict__ x, const int8_t* __restrict__ codes,
    const uint16_t* __restrict__ scales, uint16_t* __restrict__ out, int m, int n, int k,
    int groups, int64_t xs, int64_t xg, int span) {
  __shared__ f32x4 partial[C::kBatch][C::kS][64];
  const int g = blockIdx.y;
  const int c0 = int(blockIdx.x) * span;
  if (c0 >= n) return;  // uniform over the workgroup
  const int c_end = min(c0 + span, n);
  const int nlocal = (c_end - c0 + 15) / 16;

  const int lane = threadIdx.x & 63;
  const int range = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row = lane & 15, q = lane >> 4;
  // K is walked in chunks of kS * kSpb blocks of 64 (one chunk unless K > 8192 with
  // kSpb = 8); each chunk splits its blocks into kS ranges, one per wave.
  const int kblocks = k / 64;
  constexpr int kChunkBlocks = C::kS * C::kSpb;
  const int nchunks = (kblocks + kChunkBlocks - 1) / kChunkBlocks;
  int kb_first = 0, my_slots = 0;

  // Group g's codes [n, k] and scales [n, k / 32]; x rows of group g at stride xs.
  const int8_t* gcodes = codes + int64_t(g) * n * k;
  const uint16_t* gscales = scales + int64_t(g) * n * (k / 32);
  const auto w_rsrc = make_rsrc(gcodes, uint32_t(n) * uint32_t(k));
  const auto s_rsrc = make_rsrc(gscales, uint32_t(n) * uint32_t(k / 32) * 2u);
  const auto x_rsrc = make_rsrc(x + int64_t(g) * xg, uint32_t((int64_t(m - 1) * xs + k) * 2));

  auto slot_valid = [&](int lb, int s) __attribute__((always_inline)) {
    return c0 + lb * 16 + row < c_end && s < my_slots;
  };
  auto w_offset = [&](int lb, int s) __attribute__((always_inline)) {
    const int channel = c0 + lb * 16 + row;
    return slot_valid(lb, s)
               ? uint32_t(channel) * uint32_t(k) + uint32_t((kb_first + s) * 64 + q * 16)
               : kOutOfRange;
  };
  // First of the row's block scales of this wave's K range, in block lb.
  auto s_offset = [&](int lb) __attribute__((always_inline)) {
    const int channel = c0 + lb * 16 + row;
    return slot_valid(lb, 0) ? (uint32_t(channel) * uint32_t(k / 32) + uint32_t(kb_first * 2)) * 2u
                             : kOutOfRange;
  };

  // Adds the partials of local blocks [lb0, lb0 + count) in range order and stores them.
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
        out[(int64_t(out_row) * groups + g) * n + out_col] = uint16_t(f32_to_bf16(sum));
      }
    }
    __builtin_amdgcn_s_waitcnt(lgkmcnt0_imm());
    workgroup_barrier();
  };

  for (int chunk = 0; chunk < nchunks; ++chunk) {  // uniform over the workgroup
    const int cb0 = chunk * kChunkBlocks;
    const int cblocks = min(kblocks - cb0, kChunkBlocks);
    const int range_len = (cblocks + C::kS - 1) / C::kS;  // <= kSpb
    kb_first = cb0 + range * range_len;
    my_slots = max(0, min(kb_first + range_len, cb0 + cblocks) - kb_first);

    // x fragments: lane (row, q) holds x[row, g, kb * 64 + 16 q + 8 h + 0..7].
    u32x4 xf[C::kSpb][2];
#pragma unroll
    for (int s = 0; s < C::kSpb; ++s) {
      const bool valid = row < m && s < my_slots;
      const uint32_t base =
          uint32_t((int64_t(row) * xs + (kb_first + s) * 64 + q * 16) * 2);
#pragma unroll
      for (int h = 0; h < 2; ++h)
        xf[s][h] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(x_rsrc, valid ? base + 16u * h : kOutOfRange,
                                                         0, 0));
    }
    u32x4 wv[C::kSpb];
    // The row's 2 kSpb block scales of this wave's K range are kSpb dwords (dword-aligned:
    // K % 64 == 0); slot s of lane group q uses half (q / 2) of dword s. With kSpb <= 5
    // (kBlockScales) they come in C::kSLoads loads per block; with kSpb = 8, as two
    // 16-byte halves (slots 0-3, 4-7), each loaded half a block before its slots, so a
    // lane holds 8 scale registers, as it would with a 2-byte load per slot.
    constexpr int kHeld = C::kBlockScales ? C::kSpb : 4;
    uint32_t sn[kHeld], sd[kHeld];
    auto load_scales = [&](int lb, int half) __attribute__((always_inline)) {
      const uint32_t off = s_offset(lb);
      if constexpr (C::kSpb == 2) {
        const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(s_rsrc, off, 0, 0));
        sn[0] = v[0];
        sn[1] = v[1];
      } else {
        const u32x4 v = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                       s_rsrc, off == kOutOfRange ? off : off + 16u * half, 0, 0));
#pragma unroll
        for (int e = 0; e < 4; ++e) sn[e] = v[e];
        if constexpr (C::kSpb == 5)
          sn[4] = __builtin_amdgcn_raw_buffer_load_b32(s_rsrc, off == kOutOfRange ? off : off + 16u, 0, 0);
      }
    };
    auto take_scales = [&]() __attribute__((always_inline)) {
#pragma unroll
      for (int e = 0; e < kHeld; ++e) sd[e] = sn[e];
      __builtin_amdgcn_sched_barrier(0);
    };
    auto load_w = [&](int lb, int s) __attribute__((always_inline)) {
      wv[s] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, w_offset(lb, s), 0, 0));
      __builtin_amdgcn_sched_barrier(0);
    };
    // Prologue, in the order the loop's waits count on: kBlockScales: S(0), W(0, 0..);
    // halves: W(0, 0..3), S(0, half 0), W(0, 4..7).
    if constexpr (C::kBlockScales) {
      load_scales(0, 0);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int s = 0; s < C::kSpb; ++s) load_w(0, s);
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) load_w(0, s);
      load_scales(0, 0);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int s = 4; s < 8; ++s) load_w(0, s);
    }

    for (int lb = 0; lb < nlocal; ++lb) {
      f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
      // Block lb's scales (kBlockScales) or its first half have landed: the W loads issued
      // after them (all of block lb's, or its slots 4-7) may be in flight. Their successor
      // goes out now.
      waitcnt<vmcnt_imm(C::kBlockScales ? C::kSpb : 4)>();
      take_scales();
      load_scales(C::kBlockScales ? lb + 1 : lb, C::kBlockScales ? 0 : 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int s = 0; s < C::kSpb; ++s) {
        if constexpr (!C::kBlockScales) {
          if (s == 4) {
            // The second half (issued at slot 0, before the first four W loads of block
            // lb + 1) has landed; the next block's first half goes out.
            waitcnt<vmcnt_imm(4)>();
            take_scales();
            load_scales(lb + 1, 0);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
        // W(lb, s) has landed. Loads after it: kBlockScales: the rest of block lb's W, the
        // next scales and the first s W loads of block lb + 1 (kSpb - 1 + kSLoads);
        // halves: the rest of the block's W, two scale halves and W(lb + 1, < s) (9).
        waitcnt<vmcnt_imm(C::kBlockScales ? C::kSpb - 1 + C::kSLoads : 9)>();
        const float sc = f16_to_f32((sd[s % kHeld] >> (16 * (q >> 1))) & 0xFFFFu);
        if (s < my_slots) {
          const u32x4 wq = wv[s];
          const u32x2 d0 = dequant4(wq[0], sc), d1 = dequant4(wq[1], sc);
          const u32x2 d2 = dequant4(wq[2], sc), d3 = dequant4(wq[3], sc);
          acc = mfma_bf16(u32x4{d0[0], d0[1], d1[0], d1[1]}, xf[s][0], acc);
          acc = mfma_bf16(u32x4{d2[0], d2[1], d3[0], d3[1]}, xf[s][1], acc);
        }
        load_w(lb + 1, s);
      }
      if (nchunks == 1) {
        partial[lb % C::kBatch][range][lane] = acc;
        if (lb % C::kBatch == C::kBatch - 1 || lb + 1 == nlocal)  // uniform
          reduce(lb / C::kBatch * C::kBatch, lb % C::kBatch + 1);
      } else {
        // Several chunks: every local block keeps its slot (nlocal <= kBatch, host-checked)
        // and sums its chunks' partials in chunk order.
        if (chunk == 0)
          partial[lb][range][lane] = acc;
        else
          partial[lb][range][lane] += acc;
      }
    }
    waitcnt<vmcnt_imm(0)>();  // drain the trailing (out-of-range) loads of the chunk
  }
  if (nchunks > 1) reduce(0, nlocal);
}

// Channels per span-kernel workgroup: about one workgroup per CU over all groups, each
// over at least 16 channels.
int span_channels(int n, int groups, int cus) {
  const int per_group = max(1, min((cus + groups - 1) / groups, (n + 15) / 16));
  return (n + per_group - 1) / per_group;
}

template <class C>
hipError_t run_span(const void* x, const int8_t* codes, const void* scales, void* out, int m,
                    int n, int k, int groups, int64_t xs, int64_t xg, int cus,
                    hipStream_t stream) {
  const int span = span_channels(n, groups, cus);
  const dim3 grid(unsigned((n + span - 1) / span), unsigned(groups));
  gguf_q8_span_kernel<C><<<grid, C::kThreads, 0, stream>>>(
      static_cast<const uint16_t*>(x), codes, static_cast<const uint16_t*>(scales),
      static_cast<uint16_t*>(out), m, n, k, groups, xs, xg, span);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------
// Large batches: a BM x 128 (rows x channels) tile per workgroup of eight waves.
//
// The BM x 64 tile kernel above dequantizes each weight stage once per 64 rows and runs
// 8 MFMAs a wave per stage between barriers, which leaves it bound by dequantization and
// synchronisation. Here a tile is 256 (or 128) rows by 128 channels: wave w owns 64 rows
// (w % WM) and 128 / WN channels (w / WM) as 4 x TN accumulator blocks, 32 (or 16)
// MFMAs a wave per 64-wide K stage, and each stage's codes are dequantized once for 256
// (128) rows.
//  * LDS holds a ring of three stages, each x [BM][64] BF16 then Wq [128][64] BF16,
//    rows of 128 bytes with 16-byte chunks XOR-swizzled by row % 8.
//  * x goes global -> LDS by buffer_load ... lds (8 rows x 128 bytes a copy; rows past
//    M are out of the buffer's range and arrive as zeros). Each thread loads the 16
//    codes of one channel at one 16-value K offset and their FP16 block scale into
//    registers, two stages ahead, and dequantizes them into the ring one stage ahead.
//  * Stage t: issue stage t + 2's copies and code loads, read stage t's fragments, run
//    the K-step-0 MFMAs, wait for stage t + 1's loads (vmcnt counts the newer copies and
//    loads), dequantize stage t + 1's codes into its slot while the K-step-1 MFMAs run,
//    then one barrier. A slot is refilled two stages after it was read, past a barrier.
// One 16-byte-per-lane LDS DMA copy (a non-template helper: the host pass of a kernel
// template rejects the 16-byte form of the builtin, which only gfx950 has).
__device__ __forceinline__ void copy16_lds(__amdgpu_buffer_rsrc_t rsrc, lds_void* dst,
                                           uint32_t offset, int soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, dst, 16, offset, soffset, 0, 0);
}

template <int BM_>
struct GgufLargeConfig {
  static constexpr int BM = BM_, BN = 128, kWaves = 8, kThreads = 64 * kWaves;
  static constexpr int WM = BM / 64;            // waves along rows (64 rows each)
  static constexpr int WN = kWaves / WM;        // waves along channels
  static constexpr int TM = 4;                  // 16-row blocks per wave
  static constexpr int TN = BN / WN / 16;       // 16-channel blocks per wave
  static constexpr int kXBytes = BM * 128;      // one stage of x: BM rows x 64 BF16
  static constexpr int kWBytes = BN * 128;      // one stage of Wq: 128 channels x 64 BF16
  static constexpr int kStageBytes = kXBytes + kWBytes;
  static constexpr int kLdsBytes = 3 * kStageBytes;
  static constexpr int kXCopies = kXBytes / 1024 / kWaves;  // 1 KiB copies per wave per stage
  // Row tiles per raster group (4 against 8 measured on MI355X, identical outputs: G=1,
  // N=K=4096, M=2048 73.8 against 75.6 us; N=14336: 280.5 against 286.2 us).
  static constexpr int GROUP_M = 4;
  static_assert(WM * WN == kWaves && TN >= 1, "wave grid");
  static_assert(kXCopies * kWaves * 1024 == kXBytes, "x copies");
  static_assert(BN * 4 == kThreads, "one thread per 16 codes of a stage");
  static_assert(kLdsBytes <= 160 * 1024, "LDS");
  static_assert(kXCopies + 2 <= 63, "vmcnt");
};

template <class C>
__global__ void __launch_bounds__(C::kThreads, 1) gguf_q8_large_kernel(
    const uint16_t* __restrict__ x, const int8_t* __restrict__ codes,
    const uint16_t* __restrict__ scales, uint16_t* __restrict__ out, int m, int n, int k,
    int groups, int64_t xs, int64_t xg, int tiles_m, int tiles_n) {
  extern __shared__ __attribute__((aligned(1024))) char lds_raw[];
  auto* lds = (char __attribute__((address_space(3)))*)(lds_raw);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // Workgroup -> (group, tile). The hardware deals workgroups round-robin over the 8
  // XCDs; undo that so each XCD runs a contiguous range of logical tiles, ordered as a
  // raster of GROUP_M row tiles so that tiles sharing a weight panel run together.
  const int tiles = tiles_m * tiles_n;
  const int total = tiles * groups;
  int logical = int(blockIdx.x);
  {
    constexpr int kXcds = 8;
    const int per = total / kXcds, extra = total % kXcds;
    const int xcd = logical % kXcds, idx = logical / kXcds;
    logical = (xcd < extra ? xcd * (per + 1) : extra * (per + 1) + (xcd - extra) * per) + idx;
  }
  const int g = logical / tiles;
  const int tile = logical - g * tiles;
  const int group_span = C::GROUP_M * tiles_n;
  const int first_m = (tile / group_span) * C::GROUP_M;
  const int group_rows = min(tiles_m - first_m, C::GROUP_M);
  const int m0 = (first_m + (tile % group_span) % group_rows) * C::BM;
  const int n0 = ((tile % group_span) / group_rows) * C::BN;

  const auto x_rsrc = make_rsrc(x + int64_t(g) * xg, uint32_t((int64_t(m - 1) * xs + k) * 2));
  const auto c_rsrc = make_rsrc(codes + int64_t(g) * n * k, uint32_t(n) * uint32_t(k));
  const auto s_rsrc = make_rsrc(scales + int64_t(g) * n * (k / 32), uint32_t(n) * uint32_t(k / 32) * 2u);

  // x copy q of this wave brings rows 8 b .. 8 b + 7 (b = wave * kXCopies + q): lane ->
  // row 8 b + lane / 8, LDS chunk slot lane % 8 holding logical chunk slot ^ (row % 8).
  uint32_t x_off[C::kXCopies];
#pragma unroll
  for (int q = 0; q < C::kXCopies; ++q) {
    const int row = (wave * C::kXCopies + q) * 8 + (lane >> 3);
    const int chunk = (lane & 7) ^ (lane >> 3);
    x_off[q] = m0 + row < m ? uint32_t(int64_t(m0 + row) * xs * 2) + uint32_t(chunk * 16)
                            : kOutOfRange;
  }
  // Codes: thread -> channel c_row of the tile, 16 codes at K offset c_col of a stage.
  const int c_row = tid >> 2, c_col = (tid & 3) * 16;
  const bool c_live = n0 + c_row < n;
  const uint32_t c_off = c_live ? uint32_t(n0 + c_row) * uint32_t(k) + uint32_t(c_col) : kOutOfRange;
  const uint32_t s_off =
      c_live ? (uint32_t(n0 + c_row) * uint32_t(k / 32) + uint32_t(c_col / 32)) * 2u : kOutOfRange;

  const int ns = k / 64;
  // Stage t's copies and code loads. Stages past the end issue the same instructions
  // with out-of-range offsets (no memory traffic; the zeros land in a slot no stage
  // reads again), so every path has the same number of loads in flight and each wait
  // below is one constant count.
  auto issue = [&] __device__(int t, u32x4& cr, uint32_t& sr) __attribute__((always_inline)) {
    const bool live = t < ns;  // uniform
    auto* slot = lds + (t % 3) * C::kStageBytes;
#pragma unroll
    for (int q = 0; q < C::kXCopies; ++q)
      copy16_lds(x_rsrc, reinterpret_cast<lds_void*>(slot + (wave * C::kXCopies + q) * 1024),
                 live ? x_off[q] : kOutOfRange, t * 128);
    cr = __builtin_bit_cast(
        u32x4, __builtin_amdgcn_raw_buffer_load_b128(c_rsrc, live ? c_off : kOutOfRange, t * 64, 0));
    sr = __builtin_amdgcn_raw_buffer_load_b16(s_rsrc, live ? s_off : kOutOfRange, t * 4, 0);
  };
  // Dequantized codes of stage t -> its slot's Wq rows (2 chunks of 8 BF16).
  auto dequant = [&] __device__(int t, const u32x4& cr, uint32_t sr) __attribute__((always_inline)) {
    auto* wbase = lds + (t % 3) * C::kStageBytes + C::kXBytes;
    const float s = f16_to_f32(sr);
    uint32_t packed[8];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t word = cr[w];
      packed[2 * w] = pack_bf16x2(float(int8_t(word)) * s, float(int8_t(word >> 8)) * s);
      packed[2 * w + 1] = pack_bf16x2(float(int8_t(word >> 16)) * s, float(int8_t(word >> 24)) * s);
    }
    const int chunk = c_col / 8;
    *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(wbase + tile_offset(c_row, chunk)) =
        u32x4{packed[0], packed[1], packed[2], packed[3]};
    *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(wbase + tile_offset(c_row, chunk + 1)) =
        u32x4{packed[4], packed[5], packed[6], packed[7]};
  };

  // Fragments: row lane % 16 of a 16-row block, K elements 8 (lane / 16) .. + 7 of K-step
  // h, i.e. 16-byte chunk 4 h + lane / 16 of the stage.
  const int f_row = lane & 15, f_chunk = lane >> 4;
  const int wm = wave % C::WM, wn = wave / C::WM;
  f32x4 acc[C::TM][C::TN];
#pragma unroll
  for (int j = 0; j < C::TM; ++j)
#pragma unroll
    for (int i = 0; i < C::TN; ++i) acc[j][i] = f32x4{0.f, 0.f, 0.f, 0.f};

  u32x4 cr[2];
  uint32_t sr[2];
  issue(0, cr[0], sr[0]);
  issue(1, cr[1], sr[1]);
  waitcnt<vmcnt_imm(C::kXCopies + 2)>();  // stage 0's copies and codes landed
  dequant(0, cr[0], sr[0]);
  __builtin_amdgcn_s_waitcnt(lgkmcnt0_imm());
  workgroup_barrier();

  // Stage t's fragments and MFMAs, K-step h.
  u32x4 xf[2][C::TM], wf[2][C::TN];
  auto read_stage = [&] __device__(int t) __attribute__((always_inline)) {
    const auto* slot = lds + (t % 3) * C::kStageBytes;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int i = 0; i < C::TN; ++i)
        wf[h][i] = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(
            slot + C::kXBytes + tile_offset(wn * (C::TN * 16) + i * 16 + f_row, 4 * h + f_chunk));
#pragma unroll
      for (int j = 0; j < C::TM; ++j)
        xf[h][j] = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(
            slot + tile_offset(wm * 64 + j * 16 + f_row, 4 * h + f_chunk));
    }
  };
  auto mfmas = [&] __device__(int h) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < C::TN; ++i)
#pragma unroll
      for (int j = 0; j < C::TM; ++j) acc[j][i] = mfma_bf16(wf[h][i], xf[h][j], acc[j][i]);
  };
  // A stage with a successor; register set R = t % 2 holds the codes of stages t and
  // t + 2. The body is the same for every such stage (no data-dependent branch), so the
  // compiler's own waits see one load pattern.
  auto step = [&] __device__(int t, u32x4& cr_next2, uint32_t& sr_next2, const u32x4& cr_next,
                  uint32_t sr_next) __attribute__((always_inline)) {
    issue(t + 2, cr_next2, sr_next2);
    read_stage(t);
    mfmas(0);
    // Keep the dequantization behind the first MFMAs (the scheduler would otherwise
    // hoist it, and the wait for its codes, to the top of the stage).
    __builtin_amdgcn_sched_barrier(0);
    waitcnt<vmcnt_imm(C::kXCopies + 2)>();  // stage t + 1's copies and codes landed
    dequant(t + 1, cr_next, sr_next);
    mfmas(1);
    __builtin_amdgcn_s_waitcnt(lgkmcnt0_imm());
    workgroup_barrier();
  };
  int t = 0;
  for (; t + 2 < ns; t += 2) {
    step(t, cr[0], sr[0], cr[1], sr[1]);
    step(t + 1, cr[1], sr[1], cr[0], sr[0]);
  }
  if (t + 1 < ns) {  // two stages left
    step(t, cr[0], sr[0], cr[1], sr[1]);
    ++t;
  }
  read_stage(t);  // the last stage
  mfmas(0);
  mfmas(1);
  waitcnt<vmcnt_imm(0)>();  // drain the trailing (out-of-range) copies before exit

  // Lane holds D[n][m] for channels 4 (lane / 16) .. + 3 of each channel block and row
  // lane % 16 of each row block.
  const bool vec = (n & 3) == 0 && (reinterpret_cast<uintptr_t>(out) & 7) == 0;
#pragma unroll
  for (int j = 0; j < C::TM; ++j) {
    const int row = m0 + wm * 64 + j * 16 + f_row;
    if (row >= m) continue;
#pragma unroll
    for (int i = 0; i < C::TN; ++i) {
      const int col = n0 + wn * (C::TN * 16) + i * 16 + 4 * f_chunk;
      uint16_t* dst = out + (int64_t(row) * groups + g) * n + col;
      if (vec && col + 3 < n) {
        *reinterpret_cast<u32x2*>(dst) =
            u32x2{pack_bf16x2(acc[j][i][0], acc[j][i][1]), pack_bf16x2(acc[j][i][2], acc[j][i][3])};
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (col + e < n) dst[e] = uint16_t(f32_to_bf16(acc[j][i][e]));
      }
    }
  }
}

template <class C>
hipError_t run_large(const void* x, const int8_t* codes, const void* scales, void* out, int m,
                     int n, int k, int groups, int64_t xs, int64_t xg, hipStream_t stream) {
  if (const hipError_t e = prepare_lds<gguf_q8_large_kernel<C>>(C::kLdsBytes); e != hipSuccess)
    return e;
  const int tiles_m = (m + C::BM - 1) / C::BM, tiles_n = (n + C::BN - 1) / C::BN;
  gguf_q8_large_kernel<C><<<unsigned(tiles_m * tiles_n * groups), C::kThreads, C::kLdsBytes, stream>>>(
      static_cast<const uint16_t*>(x), codes, static_cast<const uint16_t*>(scales),
      static_cast<uint16_t*>(out), m, n, k, groups, xs, xg, tiles_m, tiles_n);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gguf_q8_packed_mm(const void* x, const int8_t* codes, const void* scales,
                                    void* out, int m, int n, int k, int groups, int64_t xs,
                                    int64_t xg, hipStream_t stream) {
  if (m == 0 || n == 0 || groups == 0) return hipSuccess;
  const auto* xp = static_cast<const uint16_t*>(x);
  const auto* sp = static_cast<const uint16_t*>(scales);
  auto* op = static_cast<uint16_t*>(out);
  const unsigned tiles_n = unsigned((n + kBN - 1) / kBN);
  // m <= 16: the balanced-span kernel while each wave's K range holds its x fragments
  // in registers (K <= 16 ranges x 8 blocks x 64) and x's byte range fits a buffer.
  const int cus = device_cu_count();
  const int range_len = (k / 64 + 15) / 16;
  // K > 8192 runs the span kernel in chunks of 8192 while a workgroup's partial sums of
  // all its channel blocks fit the LDS at once (span <= 8 blocks of 16).
  const int span_blocks = cus > 0 ? (span_channels(n, groups, cus) + 15) / 16 : 0;
  if (m <= 16 && cus > 0 && (range_len <= 8 || span_blocks <= 8) &&
      (int64_t(m - 1) * xs + k) * 2 <= INT32_MAX && int64_t(n) * k <= INT32_MAX) {
    if (range_len <= 2)
      return run_span<GgufSpanConfig<2>>(x, codes, scales, out, m, n, k, groups, xs, xg, cus, stream);
    if (range_len <= 4)
      return run_span<GgufSpanConfig<4>>(x, codes, scales, out, m, n, k, groups, xs, xg, cus, stream);
    if (range_len <= 5)
      return run_span<GgufSpanConfig<5>>(x, codes, scales, out, m, n, k, groups, xs, xg, cus, stream);
    return run_span<GgufSpanConfig<8>>(x, codes, scales, out, m, n, k, groups, xs, xg, cus, stream);
  }
  // m > 16: 128-channel tiles of 256 or 128 rows (while x's and the codes' byte ranges
  // fit a buffer's), whichever takes fewer rounds of one tile per CU, a round of 256-row
  // tiles costing about 1.45 rounds of 128-row ones (measured on MI355X at K = 2048 ..
  // 5120; either beats the 64 x 64 tiles at every M from 64 up).
  const int64_t tiles_n128 = (n + 127) / 128;
  const int64_t tiles256 = (m + 255) / 256 * tiles_n128 * groups;
  const int64_t tiles128 = (m + 127) / 128 * tiles_n128 * groups;
  if (m > 16 && cus > 0 && (int64_t(m - 1) * xs + k) * 2 <= INT32_MAX &&
      int64_t(n) * k <= INT32_MAX && tiles128 <= INT32_MAX) {
    const int64_t rounds256 = (tiles256 + cus - 1) / cus, rounds128 = (tiles128 + cus - 1) / cus;
    if (rounds256 * 29 <= rounds128 * 20)
      return run_large<GgufLargeConfig<256>>(x, codes, scales, out, m, n, k, groups, xs, xg, stream);
    return run_large<GgufLargeConfig<128>>(x, codes, scales, out, m, n, k, groups, xs, xg, stream);
  }
  if (m <= 16) {
    gguf_q8_packed_kernel<16><<<dim3(tiles_n, unsigned(m + 15) / 16, unsigned(groups)), 256, 0,
                                stream>>>(xp, codes, sp, op, m, n, k, groups, xs, xg);
  } else {
    gguf_q8_packed_kernel<64><<<dim3(tiles_n, unsigned(m + 63) / 64, unsigned(groups)), 256, 0,
                                stream>>>(xp, codes, sp, op, m, n, k, groups, xs, xg);
  }
  return hipGetLastError();
}

}  // namespace ci8
