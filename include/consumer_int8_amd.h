/* consumer_int8_amd.h -- C ABI of the MI355X (gfx950) INT8 linear-layer hot path.
 *
 * Every entry point takes raw device pointers, int64 sizes and a HIP stream passed as
 * `void*` (a hipStream_t; NULL selects the null stream). Calls are asynchronous and
 * stream-ordered, allocate nothing, keep no mutable global state and write only the
 * caller-owned outputs (ci8_cutlass_channel_mm_noalloc also writes the library's own
 * device scratch array), so they can be captured into a HIP graph.
 *
 * Each function validates its arguments before touching the GPU. A rejected call
 * returns a CI8_ERR_* code without launching anything; the message is available from
 * ci8_last_error() on the calling thread. A launch failure returns CI8_ERR_LAUNCH.
 *
 * Reference interfaces each entry point replaces (AppMana/consumer-int8-kernels):
 *   ci8_quantize_rows        csrc/kernels.h:48-49 (host launcher), csrc/bindings.cpp:191-209
 *                            (validation), op schema csrc/bindings.cpp:603
 *   ci8_quantize_grouped4096 csrc/kernels.h:50-51, csrc/bindings.cpp:210-237, schema :604
 *   ci8_fused_channel_mm     csrc/kernels.h:27-28, csrc/bindings.cpp:386-427, schema :598
 *   ci8_cutlass_channel_mm   csrc/kernels.h:63-65, csrc/bindings.cpp:386-424, schema :610
 *   ci8_cutlass_channel_mm_noalloc  no reference counterpart (cutlass_channel_mm without
 *                            the caller's workspace, for callers that cannot allocate)
 *   ci8_channel_mm           csrc/kernels.h:56-58, csrc/bindings.cpp:238-265, schema :605
 *   ci8_grouped_summed_mm    no reference op (configs[4]'s summed grouped W8A8); the
 *                            closest reference code is benchmarks/cuda/q8_block_int8.cu:54-55
 *   ci8_channel_gemv         csrc/kernels.h:54-55, csrc/bindings.cpp:289-310, schema :606
 *   ci8_silu_mul             csrc/silu_quant.h:8, csrc/bindings.cpp:32-44, schema :594
 *   ci8_silu_mul_quantize    csrc/silu_quant.h:6-7, csrc/bindings.cpp:46-64, schema :595
 *   ci8_unpack_allspark      csrc/kernels.h:52-53, csrc/bindings.cpp:266-288,
 *                            schema :607
 *   ci8_q8_block_int8        benchmarks/cuda/q8_block_int8.cu:142-152 (q8_block_int8 and
 *                            its tiled variants :154-174, same contract)
 *   ci8_quantize_block32,    its two stages, benchmarks/cuda/q8_block_int8.cu:11-23 and
 *   ci8_q8_block_mm          :25-63, as separate entry points
 *   ci8_gguf_q8_packed_mm    csrc/gguf_q8_packed.cu:279-285 (host launcher),
 *                            csrc/gguf_bindings.cpp:135-171 (validation), schema :496
 */
#ifndef CONSUMER_INT8_AMD_H
#define CONSUMER_INT8_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. The message of a failed call carries the same wording as the
 * reference's RuntimeError for the same condition. */
enum ci8_status {
  CI8_OK = 0,
  CI8_ERR_GEOMETRY = 1,  /* shapes or sizes the op does not accept */
  CI8_ERR_ALIGNMENT = 2, /* a buffer the kernels read with vector loads is misaligned */
  CI8_ERR_OVERLAP = 3,   /* outputs overlap inputs or each other */
  CI8_ERR_SCHEDULE = 4,  /* fused_channel_mm schedule outside 0..6 */
  CI8_ERR_TOO_LARGE = 5, /* a matrix exceeds INT_MAX elements */
  CI8_ERR_LAUNCH = 6     /* the HIP runtime reported an error at launch */
};

/* Message of the last failed call on this thread ("" after a successful call). */
const char* ci8_last_error(void);

/* Library version string, e.g. "0.1.0". */
const char* ci8_version(void);

/* quantize_rows: x BF16 [m,k] (row-major, any 2-byte alignment) -> codes INT8 [m,k]
 * and scales FP32 [m]. Per row: scale = max(amax/127, 1e-20f) with amax the
 * NaN-ignoring max |x|; code = clamp(rne(x/scale), -127, 127) with IEEE division.
 * Requires m > 0, k > 0, m*k <= INT_MAX.
 * Replaces: quantize_rows(const void*, int8_t*, float*, int m, int k, cudaStream_t),
 *           csrc/kernels.h:48-49; checks of csrc/bindings.cpp:199-203. */
int ci8_quantize_rows(const void* x, int8_t* codes, float* scales, int64_t m, int64_t k,
                      void* stream);

/* quantize_grouped4096: x BF16 [m,groups,4096] -> codes INT8 [groups,m,4096] and
 * scales FP32 [groups,m]; each (row, group) quantized exactly as quantize_rows.
 * m = 0 is a no-op. Requires groups > 0, x 16-byte, codes 8-byte and scales 4-byte
 * aligned, and no overlap between the three buffers.
 * Replaces: quantize_grouped4096(const void*, int8_t*, float*, int m, int groups,
 *           cudaStream_t), csrc/kernels.h:50-51; checks of csrc/bindings.cpp:216-232. */
int ci8_quantize_grouped4096(const void* x, int8_t* codes, float* scales, int64_t m,
                             int64_t groups, void* stream);

/* fused_channel_mm: out BF16 [m,n] = bf16_rn((float(acc) * a_scale[m]) * float(w_scale[n]))
 * with acc = sum_k a[m,k] * w[n,k] exact in INT32; a INT8 [m,k], w INT8 [n,k] (both
 * K-contiguous), a_scale FP32 [m], w_scale BF16 [n]. No workspace.
 * Requires m,n,k > 0, n % 4 == 0, k % 32 == 0, k <= 65536, each matrix <= INT_MAX
 * elements, schedule in 0..6 (a tiling hint; every schedule gives identical bits).
 * Replaces: fused_channel_mm(const int8_t*, const int8_t*, const float*, const void*,
 *           void*, int m, int n, int k, int schedule, cudaStream_t), csrc/kernels.h:27-28;
 *           checks of csrc/bindings.cpp:402-412. */
int ci8_fused_channel_mm(const int8_t* a, const int8_t* w, const float* a_scale,
                         const void* w_scale, void* out, int64_t m, int64_t n, int64_t k,
                         int64_t schedule, void* stream);

/* cutlass_channel_mm: as fused_channel_mm, and also stores the exact INT32
 * accumulators in workspace INT32 [m,n].
 * Replaces: cutlass_channel_mm(..., int32_t* workspace, void* out, int m, int n, int k,
 *           cudaStream_t), csrc/kernels.h:63-65; checks of csrc/bindings.cpp:402-408. */
int ci8_cutlass_channel_mm(const int8_t* a, const int8_t* w, const float* a_scale,
                           const void* w_scale, int32_t* workspace, void* out, int64_t m,
                           int64_t n, int64_t k, void* stream);

/* cutlass_channel_mm_noalloc: cutlass_channel_mm with no workspace argument; the INT32
 * accumulators go to a device array the library holds on each GPU it runs on (32 MiB,
 * kept until the process ends). out is bit-identical to cutlass_channel_mm's. Allocates
 * nothing: no hipMalloc, no allocating library call. Requires what cutlass_channel_mm
 * requires, and m * n <= 8388608 (else CI8_ERR_TOO_LARGE). Calls that overlap in time on
 * one GPU share the array and race on it (their outputs are unaffected: nothing reads
 * the array back). The first call on each GPU looks up that GPU's address of the array
 * and must run outside HIP graph capture (under capture it returns CI8_ERR_LAUNCH and
 * launches nothing); later calls may be captured.
 * No counterpart in the reference: it is for callers that cannot allocate the workspace
 * tensor cutlass_channel_mm needs (code under HIP graph capture, serving loops that
 * forbid allocation). */
int ci8_cutlass_channel_mm_noalloc(const int8_t* a, const int8_t* w, const float* a_scale,
                                   const void* w_scale, void* out, int64_t m, int64_t n,
                                   int64_t k, void* stream);

/* channel_mm: as fused_channel_mm with biased UINT8 weights w_u8 [n,k] holding
 * signed code + 128 (the weight used is w_u8 - 128). Any n > 0.
 * Requires m,n,k > 0, k % 32 == 0, k <= 65536, a and w <= INT_MAX elements; a and w
 * may start at any byte (16-byte aligned operands run the MFMA kernels, others a slower
 * byte-load kernel with the same bits), a_scale 4- and w_scale, out 2-byte aligned.
 * Replaces: channel_mm(const int8_t*, const uint8_t*, const float*, const void*, void*,
 *           int m, int n, int k, cudaStream_t), csrc/kernels.h:56-58;
 *           checks of csrc/bindings.cpp:252-258. */
int ci8_channel_mm(const int8_t* a, const uint8_t* w_u8, const float* a_scale,
                   const void* w_scale, void* out, int64_t m, int64_t n, int64_t k,
                   void* stream);

/* grouped_summed_mm: grouped W8A8 with the per-group partials scaled and summed,
 *   out BF16 [m,n] = bf16_rn( t_0 + t_1 + ... + t_{groups-1} )  (FP32 adds, ascending g),
 *   t_g = fl( fl( float_rn(a[g] . w[g]^T) * a_scale[g,m] ) * float(w_scale[n]) ),
 * with a INT8 [groups,m,k] (the codes quantize_grouped4096 writes for k = 4096),
 * w INT8 [groups,n,k], a_scale FP32 [groups,m], w_scale BF16 [n].
 * Requires groups > 0, m,n,k > 0, k % 32 == 0, k <= 65536, n % 4 == 0, each group's a,
 * w and out <= INT_MAX elements, a and w 16-byte aligned.
 * No reference counterpart: the reference has per-group fused_channel_mm calls with
 * separate outputs (benchmarks/benchmark_grouped_w8a8.py:100-107) and an FP32 sum of
 * scaled INT32 block partials (benchmarks/cuda/q8_block_int8.cu:54-55); this entry point
 * is the build's closed form for configs[4]. */
int ci8_grouped_summed_mm(const int8_t* a, const int8_t* w, const float* a_scale,
                          const void* w_scale, void* out, int64_t groups, int64_t m,
                          int64_t n, int64_t k, void* stream);

/* channel_gemv (W8A16): out BF16 [m,n] = bf16_rn(sum_k float(x[m,k]) * wq[n,k]) with
 * wq[n,k] = bf16_rn(float(w[n,k]) * float(scale[n])) and FP32 accumulation; x BF16
 * [m,k], w INT8 [n,k], scale BF16 [n].
 * Requires 0 < m <= 16 (the reference accepts m <= 8), n > 0, 0 < k <= 65536,
 * k % 16 == 0, w <= INT_MAX elements, w 16-byte and x 4-byte aligned.
 * Replaces: channel_gemv(const void*, const int8_t*, const void*, void*, int m, int n,
 *           int k, cudaStream_t), csrc/kernels.h:54-55; checks of csrc/bindings.cpp:298-305. */
int ci8_channel_gemv(const void* x, const int8_t* w, const void* scale, void* out,
                     int64_t m, int64_t n, int64_t k, void* stream);

/* silu_mul: x BF16 [m,2k] (gate in columns [0,k), up in [k,2k)) -> out BF16 [m,k] =
 * bf16_rn(fl(fl(g / fl(1 + exp(-g))) * u)) in FP32 with IEEE division and an exp within
 * one ULP. Requires k in {8704, 17408}, m >= 0 (0 is a no-op) and 2*m*k <= INT_MAX;
 * any 2-byte alignment; x and out must not overlap.
 * Replaces: silu_mul(const void*, void*, int m, int k, cudaStream_t),
 *           csrc/silu_quant.h:8; checks of csrc/bindings.cpp:36-40. */
int ci8_silu_mul(const void* x, void* out, int64_t m, int64_t k, void* stream);

/* silu_mul_quantize: the silu_mul activations of x BF16 [m,2k], quantized per row as
 * ci8_quantize_rows does, without writing them: codes INT8 [m,k], scales FP32 [m].
 * codes and scales equal ci8_quantize_rows applied to ci8_silu_mul's output, bit for bit.
 * Requires k in {8704, 17408}, m >= 0 (0 is a no-op), 2*m*k <= INT_MAX, x 16-byte,
 * codes 8-byte and scales 4-byte aligned, and no overlap between the three buffers.
 * Replaces: silu_mul_quantize(const void*, int8_t*, float*, int m, int k, cudaStream_t),
 *           csrc/silu_quant.h:6-7; checks of csrc/bindings.cpp:51-59. */
int ci8_silu_mul_quantize(const void* x, int8_t* codes, float* scales, int64_t m, int64_t k,
                          void* stream);

/* unpack_allspark: AllSpark N32K16 packed weights -> row-major signed INT8 weights and
 * channel scales, losslessly. packed UINT8 [padded_n,k] (padded_n = n rounded up to a
 * multiple of 32) holds biased codes (code + 128) in the N32K16 tile order;
 * packed_scales BF16 [padded_n] holds the scales permuted within each group of 32.
 * Writes weight INT8 [n,k] = code and scales BF16 [n]. Padding rows are never read.
 * Requires n > 0, n % 16 == 0, 0 < k <= 65536, k % 16 == 0, padded_n*k <= INT_MAX,
 * packed 4-byte and weight 16-byte aligned, and no overlap between the four buffers.
 * Replaces: unpack_allspark(const uint8_t*, const void*, int8_t*, void*, int n, int k,
 *           cudaStream_t), csrc/allspark_layout.cu:30-35; checks of
 *           csrc/bindings.cpp:276-284. */
int ci8_unpack_allspark(const uint8_t* packed, const void* packed_scales, int8_t* weight,
                        void* scales, int64_t n, int64_t k, void* stream);

/* quantize_block32: x BF16 [m,k] -> a INT8 [m,k] and sa FP32 [m,k/32]; every run of
 * 32 consecutive values is quantized as ci8_quantize_rows quantizes a row. Requires
 * m, k > 0, k % 32 == 0, m*k <= INT_MAX, no overlap; x 2-byte, sa 4-byte aligned.
 * Replaces: the quantize kernel of benchmarks/cuda/q8_block_int8.cu:11-23. */
int ci8_quantize_block32(const void* x, int8_t* a, float* sa, int64_t m, int64_t k,
                         void* stream);

/* q8_block_mm: block-32 W8A8 (GGUF Q8_0 weights with activations quantized per 32):
 * a INT8 [m,k], sa FP32 [m,k/32], w INT8 [n,k] (signed codes), sw FP16 [n,k/32]
 * -> y BF16 [m,n] = bf16_rn(sum), sum over blocks b ascending from +0 of
 * fma(float(acc_b), fl(sa[m,b] * float(sw[n,b])), sum), acc_b the exact INT32 dot
 * product of block b. Requires m, n, k > 0, k % 32 == 0, each of m*k, n*k, m*n <=
 * INT_MAX, a and w 16-byte aligned, y not overlapping an input.
 * Replaces: the matmul kernel of benchmarks/cuda/q8_block_int8.cu:25-63. */
int ci8_q8_block_mm(const int8_t* a, const float* sa, const int8_t* w, const void* sw, void* y,
                    int64_t m, int64_t n, int64_t k, void* stream);

/* q8_block_int8: ci8_quantize_block32 then ci8_q8_block_mm on the caller's a and sa
 * (scratch the caller owns, as in the reference).
 * Replaces: extern "C" int q8_block_int8(const void* x, void* a, float* sa,
 *           const void* w, const void* sw, void* y, int m, int n, int k, cudaStream_t),
 *           benchmarks/cuda/q8_block_int8.cu:142-152. */
int ci8_q8_block_int8(const void* x, int8_t* a, float* sa, const int8_t* w, const void* sw,
                      void* y, int64_t m, int64_t n, int64_t k, void* stream);

/* gguf_q8_packed_mm: grouped W8A16 with GGUF Q8_0 weights kept as their original codes
 * and FP16 block scales. x BF16 [m, groups, k] addressed as x[i*x_row_stride +
 * g*x_group_stride + t] (elements; k contiguous), codes INT8 [groups, n, k], scales
 * FP16 [groups, n, k/32], out BF16 [m, groups, n] contiguous:
 *   out[i, g, j] = bf16_rn(sum_t x[i, g, t] * bf16_rn(codes[g, j, t] * scales[g, j, t/32]))
 * with FP32 accumulation in the kernel's own order. Requires k > 0, k % 64 == 0,
 * m, n, groups >= 0, strides > 0 and multiples of 8, m <= 65535*32, groups <= 65535,
 * k and n <= 2147483584; x and codes 16-byte and scales 4-byte aligned; out not
 * overlapping an input (the reference rejects only identical pointers). An empty
 * output (m, n or groups == 0) returns CI8_OK without a launch.
 * Replaces: void gguf_q8_packed_mm(const void* x, const int8_t* q, const void* scales,
 *           void* y, int m, int n, int k, int groups, int64_t xs, int64_t xg,
 *           cudaStream_t), csrc/gguf_q8_packed.cu:279-285, with the checks of
 *           csrc/gguf_bindings.cpp:135-171. */
int ci8_gguf_q8_packed_mm(const void* x, const int8_t* codes, const void* scales, void* out,
                          int64_t m, int64_t n, int64_t k, int64_t groups,
                          int64_t x_row_stride, int64_t x_group_stride, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CONSUMER_INT8_AMD_H */
