// ABI plumbing: version, status strings, stream synchronisation.
#include "common.h"

// Version of this library's C ABI (independent of the reference's libsnowllm ABI numbers:
// this library exports only the verify-step subset and never poses as libsnowllm.so).
#define SNOWVERIFY_ABI_VERSION 1

SV_API int snowllm_abi_version(void) { return SNOWVERIFY_ABI_VERSION; }

SV_API const char* snowllm_error_string(int status) {
  return hipGetErrorString((hipError_t)status);
}

SV_API int snowllm_synchronize(void* stream) {
  return (int)hipStreamSynchronize((hipStream_t)stream);
}
