// Shared helpers of the reelcache HIP library: status reporting and small device utilities.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/reelcache_hip.h"

#define RCH_GLOBAL __attribute__((address_space(1)))

namespace rch {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef double d4 __attribute__((ext_vector_type(4)));
typedef unsigned int u4 __attribute__((ext_vector_type(4)));  // native vectors: promotable to registers
typedef unsigned int u2 __attribute__((ext_vector_type(2)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f2 __attribute__((ext_vector_type(2)));

// Device addresses arrive as int64 descriptor fields; these views make the compiler emit
// global (not flat) memory instructions.
template <typename T>
__device__ __forceinline__ const RCH_GLOBAL T* gin(int64_t address) {
    return reinterpret_cast<const RCH_GLOBAL T*>(address);
}
template <typename T>
__device__ __forceinline__ RCH_GLOBAL T* gout(int64_t address) {
    return reinterpret_cast<RCH_GLOBAL T*>(address);
}

// Raw buffer resources: loads at offsets >= the record count return zero and stores there are
// dropped, so out-of-range lanes need no branches.  kOutOfRange is an offset past any record count.
constexpr int kBufferWord3 = 0x00020000;  // raw buffer resource word 3 for the gfx9 family
constexpr uint32_t kOutOfRange = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(int64_t base, int64_t bytes) {
    const int records = bytes > 0x7fffffff ? 0x7fffffff : static_cast<int>(bytes < 0 ? 0 : bytes);
    return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(base), 0, records, kBufferWord3);
}

// Records `message` as this thread's last error and returns `code`.
int fail(int code, const char* format, ...) __attribute__((format(printf, 2, 3)));

// RCH_OK, or RCH_E_LAUNCH with the HIP error text when the last launch failed.
int check_launch(const char* what);

inline hipStream_t as_stream(void* stream) { return reinterpret_cast<hipStream_t>(stream); }

// Workgroup index -> work unit, so that consecutive units land on the same XCD.
// Workgroups are dispatched round-robin over the 8 XCDs of an MI355X (XCD = b % 8);
// units [x*q + min(x, r), ...) run on XCD x.  A bijection on [0, G).
__device__ __forceinline__ int xcd_unit(int b, int grid) {
    constexpr int kXcds = 8;
    const int q = grid / kXcds, r = grid - q * kXcds;
    const int x = b % kXcds, i = b / kXcds;
    return x * q + (x < r ? x : r) + i;
}

// s_waitcnt vmcnt(0) with expcnt / lgkmcnt unconstrained (gfx9 encoding: vmcnt in bits 3:0 and
// 15:14, expcnt 6:4, lgkmcnt 11:8).  The compiler's wait insertion accounts for it, so registers
// loaded before it are known complete afterwards.
__device__ __forceinline__ void wait_vector_memory() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Exact 2**e as float for e in [-126, 127].
__device__ __forceinline__ float pow2f(int e) { return __int_as_float((e + 127) << 23); }

// ceil(log2(v)) for a finite v > 0, exactly (frexp: v = m * 2**E, m in [0.5, 1)).
__device__ __forceinline__ int ceil_log2(float v) {
    int e;
    const float m = frexpf(v, &e);
    return m == 0.5f ? e - 1 : e;
}

// The reference's power-of-two prescale exponent: max|x| lands in (2**13, 2**14]
// (reelcache/restore_kernels.py:1386-1398), clamped to [-100, 100].
__device__ __forceinline__ int prescale_exponent(float bound) {
    if (!(bound > 0.0f)) return 0;
    int e = 14 - ceil_log2(bound);
    return e < -100 ? -100 : (e > 100 ? 100 : e);
}

}  // namespace rch
