// Grouped W8A8 with the per-group partials scaled and summed (grouped_summed_mm) for
// large M on gfx950: the two-waves-per-SIMD scheme of gemm_pp.hip over the groups' K
// stages in one stream.
//
//   out[m, n] = bf16_rn( t_0 + t_1 + ... + t_{G-1} ),  FP32 additions left to right,
//   t_g = fl( fl( float_rn(acc_g[m, n]) * sa[g, m] ) * float(sw[n]) ),
//   acc_g = A_g[m, :] . W_g[n, :]  (exact INT32), A [G, M, K], W [G, N, K], sa [G, M].
//
// The arithmetic of the grouped kernel in gemm.hip, bit for bit (the reference has no such
// op; each term is the fused_channel_mm epilogue of one group, csrc/fused_mm.cu:24-38, and
// the FP32 sum of scaled INT32 partials follows benchmarks/cuda/q8_block_int8.cu:54-55).
//
// Tile 256 (m) x 128 (n) per workgroup of eight waves; wave w owns rows 64 * (w % 4) and
// columns 64 * (w / 4) as 4 x 4 blocks of v_mfma_i32_16x16x64_i8 accumulators (64
// registers), next to their FP32 running sum (64 more): a wider wave tile would not leave
// room for the sum. Waves w and w + 4 share SIMD w % 4; the waves of group w / 4 alternate
// a memory phase (the stage's 16 fragments from LDS, and this wave's copies of a later
// stage) and a compute phase (32 MFMAs), the two groups one phase apart, with workgroup
// barriers between phases (see gemm_pp.hip). The K stages of all groups form one stream:
// stage s is K stage s % ns of group s / ns, so the copies run across group boundaries
// without a pipeline drain, and after the last stage of a group each wave folds its
// accumulators into the sum and clears them.
// Rings (buffer_load ... lds, 8 rows x 128 bytes per copy; rows past M or N and bytes past
// K come back as zeros):
//   A: two 32 KB slots, group 0 copies A(s + 1) in phase 2s into the slot of A(s - 1) and
//      waits for it at the end of phase 2s + 1 (eight copies per wave per stage);
//   W: three 16 KB slots, group 1 copies W(s + 2) in phase 2s + 1 into the slot of W(s - 1)
//      and waits for W(s + 1) at the end of that phase (four copies per wave per stage).
// Fragments: lane group g (lane / 16) reads logical chunk 4h + g of a row's 128-byte
// stage in K-step h (A and W alike), chunks XOR-swizzled by row % 8.
#include <type_traits>

#include "ci8_device.h"
#include "launch.h"

namespace ci8 {
namespace {

constexpr int kXcds = 8;

struct GroupedConfig {
  static constexpr int BM = 256, BN = 128, BK = 128;
  static constexpr int kWaves = 8, kThreads = 512;
  static constexpr int WM = 4;                     // waves along m (per group of waves)
  static constexpr int TM = BM / WM / 16;          // 4 m blocks per wave
  static constexpr int TN = BN / 2 / 16;           // 4 n blocks per wave
  static constexpr int kACopies = BM * BK / 1024 / WM;  // 8 per A wave per stage
  static constexpr int kWCopies = BN * BK / 1024 / WM;  // 4 per W wave per stage
  static constexpr int kAStage = BM * BK;          // 32 KB
  static constexpr int kWStage = BN * BK;          // 16 KB
  static constexpr int kWBase = 2 * kAStage;       // A ring: 2 slots, W ring: 3 slots
  static constexpr int kRingBytes = kWBase + 3 * kWStage;  // 112 KB
  // Epilogue staging (reuses the ring): each wave's 64 x 64 BF16 sums at a row stride of
  // 144 bytes (36 dwords: 16 rows written by one ds_write_b64 start in distinct banks).
  static constexpr int kEpiRowBytes = (BN / 2) * 2 + 16;
  static constexpr int kEpiWaveBytes = (BM / WM) * kEpiRowBytes;
  static constexpr int kMaxGroups = (160 * 1024 - kRingBytes) / 1024;  // row scales: 48
  // m tiles per raster group (4 against 8 measured on MI355X: configs[4] 118.0-118.1
  // against 119.0-119.6 us).
  static constexpr int GROUP_M = 4;
  static_assert(kWaves * kEpiWaveBytes <= kRingBytes, "epilogue staging fits the ring");
  static_assert(2 * (TM + TN) == 2 * kACopies && 2 * (TM + TN) == 4 * kWCopies,
                "copies go after every second (A) or fourth (W) fragment read");
};

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

template <bool kExactK>
__global__ void __launch_bounds__(GroupedConfig::kThreads, 1) grouped_pp_kernel(
    const int8_t* __restrict__ a, const int8_t* __restrict__ w, const float* __restrict__ sa,
    const uint16_t* __restrict__ sw, uint16_t* __restrict__ out, int groups, int m, int n,
    int k, bool out16) {
  // Every product and sum of the fold is rounded on its own (no FMA contraction of the
  // running sum with the scaled term), as the closed form requires.
#pragma clang fp contract(off)
  using C = GroupedConfig;
  extern __shared__ __attribute__((aligned(1024))) char lds_raw[];
  auto* lds = (char __attribute__((address_space(3)))*)(lds_raw);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave % C::WM, group = wave / C::WM;
  const bool copies_a = group == 0;

  // Workgroup -> tile: undo the round-robin dealing over the 8 XCDs, then a grouped
  // raster of GROUP_M m tiles, so tiles that run together on one XCD share panels.
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
  const int m0 = (first_m + (logical % group_span) % group_rows) * C::BM;
  const int n0 = ((logical % group_span) / group_rows) * C::BN;

  const int ns = (k + C::BK - 1) / C::BK;  // K stages per group
  const int total = groups * ns;           // stages of the stream

  // Copy i of a wave brings block b = 4i + wave % 4 of its operand's stage (8 rows x 128
  // bytes): lane -> row 8b + lane / 8, LDS chunk slot lane % 8 holding logical chunk
  // slot ^ (row % 8). The group's operand base goes in the buffer resource, the stage's
  // K offset in soffset.
  const int sub = wave % C::WM;
  const int c_row = lane >> 3;
  const int c_chunk = (lane & 7) ^ c_row;
  const int c_rows = copies_a ? m : n;
  const int8_t* c_base = copies_a ? a : w;
  const int64_t c_group_bytes = int64_t(c_rows) * k;
  uint32_t c_off[C::kACopies];
#pragma unroll
  for (int i = 0; i < C::kACopies; ++i) {
    const int row = (copies_a ? m0 : n0) + (i * C::WM + sub) * 8 + c_row;
    const bool valid = (copies_a || i < C::kWCopies) && row < c_rows;
    c_off[i] = valid ? uint32_t(row) * uint32_t(k) + uint32_t(c_chunk * 16) : kOutOfRange;
  }
  const int c_dst0 = (copies_a ? 0 : C::kWBase) + sub * 1024;
  const int c_stride = copies_a ? C::kAStage : C::kWStage;
  // Copy i of K stage t of group g into ring slot base `dst`.
  auto copy = [&] __device__(int dst, int g, int t, int i) __attribute__((always_inline)) {
    const auto rsrc = make_rsrc(c_base + int64_t(g) * c_group_bytes, uint32_t(c_group_bytes));
    const int k0 = t * C::BK;
    uint32_t off = c_off[i];
    if (!kExactK && off != kOutOfRange && k0 + c_chunk * 16 >= k) off = kOutOfRange;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, reinterpret_cast<lds_void*>(lds + dst + i * C::WM * 1024),
                                             16, off, k0, 0, 0);
  };
  auto copies = [&] __device__(int dst, int g, int t) __attribute__((always_inline)) {
    const int count = copies_a ? C::kACopies : C::kWCopies;
#pragma unroll
    for (int i = 0; i < C::kACopies; ++i)
      if (i < count) copy(dst, g, t, i);
  };

  // Fragments: row (lane % 16) of each 16-row block at logical chunk 4h + lane / 16.
  const int f_row = lane & 15, f_group = lane >> 4;
  int a_base[2], w_base[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int swz = (((4 * h + f_group) ^ (f_row & 7)) * 16);
    a_base[h] = (wm * 64 + f_row) * C::BK + swz;
    w_base[h] = C::kWBase + (group * 64 + f_row) * C::BK + swz;
  }
  i32x4 af[2][C::TM], wf[2][C::TN];
  // Memory phase: the 16 fragments of stage s (A slot a_slot, W slot w_slot) and, when
  // kCopy, this wave's copies of K stage ct of group cg after every second (A) or fourth
  // (W) fragment read.
  auto memory = [&] __device__(int a_slot, int w_slot, int dst, int cg, int ct, auto role,
                               auto with_copies) __attribute__((always_inline)) {
    constexpr bool kA = decltype(role)::value;
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
      if constexpr (kCopy) {
        if constexpr (kA) {
          if (q % 2 == 0) copy(dst, cg, ct, q / 2);
        } else {
          if (q % 4 == 0) copy(dst, cg, ct, q / 4);
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(lgkmcnt0_imm());
  };

  i32x4 acc[C::TM][C::TN];
  float sum[C::TM][C::TN][4];
#pragma unroll
  for (int j = 0; j < C::TM; ++j)
#pragma unroll
    for (int i = 0; i < C::TN; ++i) acc[j][i] = i32x4{0, 0, 0, 0};
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

  // Channel scales of the wave's 4 x 4 columns (lane: 4 consecutive columns per block),
  // and the row scales of the next group to fold, loaded a whole group ahead.
  const int row0 = m0 + wm * 64, col0 = n0 + group * 64;
  float cs[C::TN][4];
#pragma unroll
  for (int i = 0; i < C::TN; ++i) {
    const int col = col0 + i * 16 + f_group * 4;
    const u32x2 bits = col < n ? *reinterpret_cast<const u32x2*>(sw + col) : u32x2{0, 0};
    cs[i][0] = bf16_lo(bits[0]);
    cs[i][1] = bf16_hi(bits[0]);
    cs[i][2] = bf16_lo(bits[1]);
    cs[i][3] = bf16_hi(bits[1]);
  }
  // Row scales: the tile's 256 rows of every group, copied into LDS (1 KiB per group, after
  // the ring) in the prologue; a fold reads its group's four per lane from there.
  const auto sa_rsrc = make_rsrc(sa, uint32_t(groups) * uint32_t(m) * 4u);
  for (int g = wave; g < groups; g += C::kWaves) {
    const int row = m0 + lane * 4;  // 4 rows per lane; rows past m read as zeros
    const uint32_t off = row < m ? (uint32_t(g) * uint32_t(m) + uint32_t(row)) * 4u : kOutOfRange;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        sa_rsrc, reinterpret_cast<lds_void*>(lds + C::kRingBytes + g * 1024), 16, off, 0, 0, 0);
  }
  // Folds group g's accumulators into the sum and clears them.
  auto fold = [&] __device__(int g) __attribute__((always_inline)) {
    float rs[C::TM];
#pragma unroll
    for (int j = 0; j < C::TM; ++j)
      rs[j] = *reinterpret_cast<const __attribute__((address_space(3))) float*>(
          lds + C::kRingBytes + g * 1024 + (wm * 64 + j * 16 + f_row) * 4);
#pragma unroll
    for (int j = 0; j < C::TM; ++j)
#pragma unroll
      for (int i = 0; i < C::TN; ++i) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float term = (float(acc[j][i][e]) * rs[j]) * cs[i][e];
          sum[j][i][e] = g == 0 ? term : sum[j][i][e] + term;
        }
        acc[j][i] = i32x4{0, 0, 0, 0};
      }
  };

  // Prologue: A(0) (group 0), W(0) and W(1) (group 1) in place for everyone.
  copies(c_dst0, 0, 0);
  if (!copies_a && 1 < total) copies(c_dst0 + c_stride, ns > 1 ? 0 : 1, ns > 1 ? 1 : 0);
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  barrier_fenced();

  // Stage s (group sg, K stage st): group 0 copies A(s + 1) (into A slot (s + 1) % 2),
  // group 1 W(s + 2) (into W slot (s + 2) % 3). The last stages, with nothing left to
  // copy, issue no copies, and group 1 then waits for all of its copies. The loop is
  // compiled once per role, so every copy count and wait count is a constant.
  auto k_loop = [&] __device__(auto role) __attribute__((always_inline)) {
    constexpr bool kA = decltype(role)::value;
    constexpr int lead = kA ? 1 : 2;
    int sg = 0, st = 0;      // stage s
    int cg = 0, ct = lead;   // stage s + lead
    while (ct >= ns) {
      ct -= ns;
      ++cg;
    }
    int w_slot = 0;   // s % 3
    int cw_slot = 2;  // (s + 2) % 3
    if constexpr (!kA) barrier_fenced();  // phase 0 is group 0's first memory phase
    for (int s = 0; s < total; ++s) {
      const int dst = c_dst0 + (kA ? (s + 1) & 1 : cw_slot) * c_stride;
      if (s + lead < total) {  // uniform over the wave
        memory(s & 1, w_slot, dst, cg, ct, role, std::true_type{});
        // W(s + 1) landed (W(s + 2), just issued, may be in flight).
        if constexpr (!kA) __builtin_amdgcn_s_waitcnt(vmcnt_imm(C::kWCopies));
      } else {
        memory(s & 1, w_slot, dst, cg, ct, role, std::false_type{});
        if constexpr (!kA) __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
      }
      barrier_fenced();
      compute();
      if (st == ns - 1) fold(sg);  // uniform: the group's last K stage
      // Group 0: A(s + 1), issued in the memory phase, landed.
      if constexpr (kA) __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
      barrier_fenced();
      w_slot = w_slot == 2 ? 0 : w_slot + 1;
      cw_slot = cw_slot == 2 ? 0 : cw_slot + 1;
      if (++st == ns) {
        st = 0;
        ++sg;
      }
      if (++ct == ns) {
        ct = 0;
        ++cg;
      }
    }
  };
  if (copies_a)
    k_loop(std::true_type{});
  else
    k_loop(std::false_type{});
  if (group == 0) barrier_fenced();  // phase 2 total: group 1's last compute phase
  barrier_fenced();                  // every wave is past its last fragment reads

  // Epilogue through LDS: the wave's 64 x 64 BF16 sums go to its own region in the MFMA
  // layout and come back as 16-byte row chunks, so each store instruction writes whole
  // 128-byte row pieces (8 lanes per row).
  auto* region = lds + wave * C::kEpiWaveBytes;
#pragma unroll
  for (int j = 0; j < C::TM; ++j) {
    auto* rbase = region + (j * 16 + f_row) * C::kEpiRowBytes + f_group * 8;
#pragma unroll
    for (int i = 0; i < C::TN; ++i)
      *reinterpret_cast<__attribute__((address_space(3))) u32x2*>(rbase + i * 32) =
          u32x2{pack_bf16x2(sum[j][i][0], sum[j][i][1]), pack_bf16x2(sum[j][i][2], sum[j][i][3])};
  }
  // One wave's LDS operations complete in order; the wait only orders the reads after
  // every lane's writes for the compiler.
  __builtin_amdgcn_s_waitcnt(lgkmcnt0_imm());
  __builtin_amdgcn_wave_barrier();
  constexpr int kChunks = 64 / 8;  // 16-byte chunks per output row piece
  const bool full = out16 && row0 + 64 <= m && col0 + 64 <= n && (n % 8) == 0;
#pragma unroll
  for (int it = 0; it < kChunks; ++it) {
    const int q = it * 64 + lane;
    const int row = q / kChunks, chunk = q % kChunks;
    const u32x4 v = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(
        region + row * C::kEpiRowBytes + chunk * 16);
    const int grow = row0 + row, gcol = col0 + chunk * 8;
    uint16_t* dst = out + int64_t(grow) * n + gcol;
    if (full) {
      *reinterpret_cast<u32x4*>(dst) = v;
    } else if (grow < m) {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (gcol + e < n) dst[e] = uint16_t(v[e >> 1] >> (16 * (e & 1)));
    }
  }
}

}  // namespace

// Requires a and w 16-byte aligned, sw 8-byte aligned, n % 4 == 0, groups <=
// kMaxGroups (grouped_pp_max_groups()).
int grouped_pp_max_groups() { return GroupedConfig::kMaxGroups; }

hipError_t launch_grouped_pp_gemm(const int8_t* a, const int8_t* w, const float* sa,
                                  const void* sw, void* out, int groups, int m, int n, int k,
                                  hipStream_t stream) {
  using C = GroupedConfig;
  if (groups > C::kMaxGroups) return hipErrorInvalidValue;
  const int blocks = ((n + C::BN - 1) / C::BN) * ((m + C::BM - 1) / C::BM);
  const bool out16 = (reinterpret_cast<uintptr_t>(out) & 15) == 0;
  const int lds = C::kRingBytes + groups * 1024;
  auto launch = [&](auto kernel_constant) {
    constexpr auto kernel = decltype(kernel_constant)::value;
    if (const hipError_t e = prepare_lds<kernel>(lds); e != hipSuccess) return e;
    kernel<<<blocks, C::kThreads, lds, stream>>>(
        a, w, sa, static_cast<const uint16_t*>(sw), static_cast<uint16_t*>(out), groups, m, n, k,
        out16);
    return hipGetLastError();
  };
  return k % C::BK == 0 ? launch(kernel_constant<grouped_pp_kernel<true>>{})
                        : launch(kernel_constant<grouped_pp_kernel<false>>{});
}

}  // namespace ci8
