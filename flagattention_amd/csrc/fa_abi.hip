// C-ABI plumbing: version, thread-local error message, device queries.
#include <stdarg.h>
#include <stdio.h>

#include "fa_common.h"

namespace fa {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

}  // namespace fa

extern "C" int fa_abi_version(void) { return FA_ABI_VERSION; }

extern "C" const char* fa_last_error(void) { return fa::g_last_error; }

extern "C" int64_t fa_mla_decode_args_size(void) {
  return static_cast<int64_t>(sizeof(fa_mla_decode_args));
}

extern "C" int fa_device_cu_count(int device, int32_t* cu_count) {
  FA_CHECK_ARG(cu_count != nullptr, "cu_count is NULL");
  int v = 0;
  FA_CHECK_HIP(hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, device));
  *cu_count = v;
  return FA_OK;
}

extern "C" int64_t fa_gqa_decode_args_size(void) {
  return static_cast<int64_t>(sizeof(fa_gqa_decode_args));
}
