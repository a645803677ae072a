// sta_api_util.h -- helpers shared by the C ABI translation units: the thread-local error
// message, HIP error wrapping and alignment checks.
#pragma once
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string>

#include <hip/hip_runtime.h>

#include "../../include/sta.h"

namespace sta_api {

extern thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

inline int hip_fail(hipError_t e, const char* what) {
  return fail(STA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

inline int esize(int dtype) { return dtype == STA_DTYPE_F32 ? 4 : 2; }

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// q / k / v pointers and strides: non-NULL, 16-byte aligned rows
int check_qkv_ptrs(int dtype, const void* q, const void* k, const void* v, const int64_t strides[6],
                   bool need_v);

// record stage event i on st when events were given
inline int mark_event(void* const* events, int i, hipStream_t st) {
  if (!events || !events[i]) return STA_OK;   // a NULL entry skips that mark
  hipError_t e = hipEventRecord((hipEvent_t)events[i], st);
  return e == hipSuccess ? STA_OK : hip_fail(e, "stage event record");
}

}  // namespace sta_api
