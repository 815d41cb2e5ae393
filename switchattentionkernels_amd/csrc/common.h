// Shared host/device helpers for libswattn.so (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "swattn.h"

namespace swattn {

// Per-thread message for the last failing C-ABI call.
void set_error(const std::string& msg);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Returns a C-ABI status for the last launch on this thread.
inline int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error(std::string(what) + ": " + hipGetErrorString(e));
    return static_cast<int>(e);
  }
  return SWATTN_OK;
}

inline int invalid(const std::string& msg) {
  set_error(msg);
  return SWATTN_EINVAL;
}

// bf16 row tensors (Q, K, V, O and their gradients, caches, partials) move
// in 16-byte pieces, by vector loads and global -> LDS DMAs: their base
// pointers must be 16-byte aligned.
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
// Workspaces hold float4 / int64 records at 256-byte-aligned offsets from
// their start, which must itself be 256-byte aligned (as hipMalloc returns).
inline bool aligned256(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 255u) == 0; }

// popcount(mask & lanes_below_me) without a lane-mask table.
__device__ __forceinline__ int count_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0));
}

__device__ __forceinline__ uint64_t wave_ballot(bool p) { return __builtin_amdgcn_ballot_w64(p); }

}  // namespace swattn
