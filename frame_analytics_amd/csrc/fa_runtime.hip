// Library-level entry points: ABI version, status strings, device queries.
#include "fa_common.h"

namespace fa {

int cu_count(int device) {
  constexpr int MAX_DEV = 64;
  static int cache[MAX_DEV] = {0};
  const int d = device < 0 ? 0 : device;
  if (d < MAX_DEV && cache[d] > 0) return cache[d];
  int v = 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, d) !=
          hipSuccess ||
      v <= 0) {
    v = 1;
  }
  if (d < MAX_DEV) cache[d] = v;
  return v;
}

}  // namespace fa

extern "C" {

// reference: fa_cuda.cu:1036 (fa_cuda_abi_version)
FA_API int fa_gpu_abi_version(void) { return FA_ABI_VERSION; }

// reference: fa_cuda.cu:1038-1050 (fa_cuda_error_string)
FA_API const char* fa_gpu_error_string(int code) {
  if (code < 0) return hipGetErrorString(static_cast<hipError_t>(-code));
  switch (code) {
    case FA_OK: return "ok";
    case FA_E_DTYPE: return "unsupported dtype";
    case FA_E_SHAPE: return "unsupported shape";
    case FA_E_WINDOW: return "unsupported window size";
    case FA_E_OP: return "unknown pixel op";
    case FA_E_ARG: return "invalid argument";
    case FA_E_NOGPU: return "no GPU device";
    case FA_E_SCRATCH:
      return "the call needs more partial-sum slots than the no-allocation scratch holds";
    default: return "internal error";
  }
}

// reference: fa_cuda.cu:1052-1062 (fa_cuda_device_count)
FA_API int fa_gpu_device_count(int* out_count) {
  int n = 0;
  const hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) {
    if (out_count) *out_count = 0;
    return -static_cast<int>(e);
  }
  if (out_count) *out_count = n;
  return FA_OK;
}

}  // extern "C"
