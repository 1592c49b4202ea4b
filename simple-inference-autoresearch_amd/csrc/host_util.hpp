// Host helpers: error reporting, device facts, occupancy cache, tensor checks.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "sia_attention.h"

namespace sia {

// Records a per-thread message and returns `code` (see sia_last_error_message).
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

struct DeviceInfo {
  int id = -1;
  int cus = 0;
  bool gfx950 = false;
};

// Facts about the current device (cached per device id).
const DeviceInfo& device_info();

// SIA_OK when the current device is a gfx950, else a SIA_ERR_DEVICE failure.
inline int device_ok() {
  const DeviceInfo& dev = device_info();
  if (dev.id < 0) return fail(SIA_ERR_DEVICE, "no HIP device is current");
  if (!dev.gfx950) return fail(SIA_ERR_DEVICE, "this library is built for gfx950 (MI355X) only");
  return SIA_OK;
}

// Launches `kernel` on `stream`.  With timing events it goes through
// hipExtLaunchKernel, which stamps `begin` and `end` with the kernel's own
// start and end times (no marker packets around the dispatch, so short
// kernels are timed as a kernel trace times them).
template <class K, class... Args>
int launch_kernel(K kernel, dim3 grid, dim3 block, size_t lds, hipStream_t stream, hipEvent_t begin,
                  hipEvent_t end, const char* what, Args... args) {
  if (begin || end)
    hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, stream, begin, end, 0u, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, lds, stream, args...);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(SIA_ERR_LAUNCH, "%s launch: %s", what, hipGetErrorString(e));
  return SIA_OK;
}

// Active work-groups per CU for a kernel at a block size and dynamic LDS size
// (cached; computed with hipOccupancyMaxActiveBlocksPerMultiprocessor).
int kernel_occupancy(const void* kernel, int block, size_t lds);

inline int elem_size(int dtype) {
  switch (dtype) {
    case SIA_F16: case SIA_BF16: return 2;
    case SIA_F32: case SIA_I32: return 4;
    case SIA_I8: case SIA_U8: return 1;
    case SIA_I64: return 8;
    default: return 0;
  }
}

inline const char* dtype_name(int dtype) {
  switch (dtype) {
    case SIA_F16: return "float16";
    case SIA_BF16: return "bfloat16";
    case SIA_F32: return "float32";
    case SIA_I8: return "int8";
    case SIA_I32: return "int32";
    case SIA_I64: return "int64";
    case SIA_U8: return "uint8";
    default: return "unknown";
  }
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Byte stride of dimension d.
inline int64_t bstride(const sia_tensor* t, int d) { return t->stride[d] * elem_size(t->dtype); }

}  // namespace sia
