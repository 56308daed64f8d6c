// cutlass_channel_mm without a caller-provided workspace.
//
// cutlass_channel_mm's kernels store the exact INT32 accumulators of the product into a
// workspace [m, n] that the caller allocates (csrc/bindings.cpp:386-424 requires it).
// Callers that cannot allocate (code under HIP graph capture, serving loops that forbid
// hipMalloc) use this variant instead: the same kernels, the accumulators go to
// `scratch`, a file-scope device array that every GPU the library runs on holds until
// the process ends. The BF16 output is bit-identical to cutlass_channel_mm's.
//
// Host code must never pass `scratch` itself to a kernel or a copy: in host code the name
// is a host-side stand-in, not a device address. Each device's address of its own copy
// is looked up once with hipGetSymbolAddress, with that device current, and cached.
//
// The lookup is the one set-up step: the first call on a device must be made outside
// HIP graph capture (under capture it returns hipErrorStreamCaptureUnsupported and
// records nothing); later calls, captured or not, use the cached address.
//
// Every call on one GPU writes the same array, which keeps the last call's values.
// Nothing in it has to start at zero: a call writes every accumulator of its [m, n]
// range before the call ends and reads none. Calls that overlap in time on one GPU (two
// streams) race on the array; their BF16 outputs are unaffected, since no kernel reads
// the array back.
#include <atomic>
#include <mutex>

#include "ci8_device.h"
#include "launch.h"

namespace ci8 {
namespace {

constexpr int64_t kScratchInts = int64_t(1) << 23;  // 32 MiB of INT32 accumulators

__device__ __align__(256) int32_t scratch[kScratchInts];

constexpr int kMaxDevices = 64;
std::atomic<int32_t*> g_scratch[kMaxDevices];
std::mutex g_scratch_mutex;

// The device a launch on `stream` runs on: the stream's own device, or the current one
// for the null stream.
hipError_t stream_device(hipStream_t stream, int* device) {
  if (stream == nullptr) return hipGetDevice(device);
  return hipStreamGetDevice(stream, device);
}

// This device's address of `scratch`, resolved on the first call for the device, which
// must not be under graph capture on `stream`.
hipError_t scratch_on(int device, hipStream_t stream, int32_t** ptr) {
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  int32_t* cached = g_scratch[device].load(std::memory_order_acquire);
  if (cached) {
    *ptr = cached;
    return hipSuccess;
  }
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  if (const hipError_t e = hipStreamIsCapturing(stream, &capture); e != hipSuccess) return e;
  if (capture != hipStreamCaptureStatusNone) return hipErrorStreamCaptureUnsupported;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  cached = g_scratch[device].load(std::memory_order_relaxed);
  if (!cached) {
    int current = 0;
    if (const hipError_t e = hipGetDevice(&current); e != hipSuccess) return e;
    if (current != device)
      if (const hipError_t e = hipSetDevice(device); e != hipSuccess) return e;
    void* address = nullptr;
    const hipError_t e = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
    if (current != device) (void)hipSetDevice(current);
    if (e != hipSuccess) return e;
    if (address == nullptr) return hipErrorInvalidSymbol;
    cached = static_cast<int32_t*>(address);
    g_scratch[device].store(cached, std::memory_order_release);
  }
  *ptr = cached;
  return hipSuccess;
}

}  // namespace

int64_t noalloc_scratch_ints() { return kScratchInts; }

hipError_t launch_cutlass_channel_mm_noalloc(const int8_t* a, const int8_t* w, const float* sa,
                                             const void* sw, void* out, int m, int n, int k,
                                             hipStream_t stream) {
  if (int64_t(m) * n > kScratchInts) return hipErrorInvalidValue;  // the ABI rejects first
  int device = 0;
  if (const hipError_t e = stream_device(stream, &device); e != hipSuccess) return e;
  int32_t* ws = nullptr;
  if (const hipError_t e = scratch_on(device, stream, &ws); e != hipSuccess) return e;
  return launch_channel_gemm(a, w, WeightCode::kSigned, sa, sw, out, ws, m, n, k, 0, stream);
}

}  // namespace ci8
