// LDS budget of one gfx950 workgroup, as pure host arithmetic (no HIP types), so the rule
// every launcher applies can be tested on a machine without a GPU.
//
// A workgroup on gfx950 (MI355X) can hold at most 160 KiB of LDS: the kernel's static LDS
// (its __shared__ variables) plus the dynamic LDS requested at launch. A launch asking for
// more is accepted by the launch call and aborts the queue on the device
// (HSA_STATUS_ERROR_INVALID_ALLOCATION), so launchers check the sum first and return an
// error instead.
#pragma once
#include <stdint.h>

namespace ci8 {

constexpr int64_t kLdsPerWorkgroup = 160 * 1024;  // 163,840 bytes
// Dynamic LDS a kernel may request without raising its attribute.
constexpr int64_t kDefaultDynamicLds = 64 * 1024;

// Whether a launch of a kernel with `static_bytes` of its own LDS and `dynamic_bytes` of
// dynamic LDS fits in one workgroup.
constexpr bool lds_fits(int64_t static_bytes, int64_t dynamic_bytes) {
  return static_bytes >= 0 && dynamic_bytes >= 0 &&
         static_bytes + dynamic_bytes <= kLdsPerWorkgroup;
}

// The dynamic-LDS attribute a kernel with `static_bytes` of its own LDS needs so that
// every launch that fits can run: the rest of the budget.
constexpr int64_t dynamic_lds_limit(int64_t static_bytes) {
  return kLdsPerWorkgroup - static_bytes;
}

}  // namespace ci8
