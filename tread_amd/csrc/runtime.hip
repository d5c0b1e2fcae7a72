// Error plumbing, ABI version and the block-tier copy entry point.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"
#include "../../include/tread_hip.h"

namespace tread {

static thread_local char g_err[512];

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail((int)e, "%s: launch failed: %s", what, hipGetErrorString(e));
  return 0;
}

}  // namespace tread

extern "C" const char* tread_last_error(void) { return tread::g_err; }

extern "C" int tread_abi_version(void) { return 10; }

extern "C" int tread_copy_layers_async(void* const* dst, const void* const* src, const size_t* bytes, int per_layer,
                                       int n_layers, tread_stream_t stream, const tread_event_t* layer_done) {
  if (per_layer < 0 || n_layers < 0 || (per_layer > 0 && n_layers > 0 && (!dst || !src || !bytes)))
    return tread::fail(TREAD_EINVAL, "tread_copy_layers_async: bad arguments");
  for (int l = 0; l < n_layers; ++l) {
    for (int i = 0; i < per_layer; ++i) {
      const int64_t k = (int64_t)l * per_layer + i;
      if (bytes[k] == 0) continue;
      if (!dst[k] || !src[k]) return tread::fail(TREAD_EINVAL, "tread_copy_layers_async: null pointer at %lld", (long long)k);
      hipError_t e = hipMemcpyAsync(dst[k], src[k], bytes[k], hipMemcpyDefault, (hipStream_t)stream);
      if (e != hipSuccess) return tread::fail((int)e, "tread_copy_layers_async: copy %lld: %s", (long long)k, hipGetErrorString(e));
    }
    if (layer_done && layer_done[l]) {
      hipError_t e = hipEventRecord((hipEvent_t)layer_done[l], (hipStream_t)stream);
      if (e != hipSuccess) return tread::fail((int)e, "tread_copy_layers_async: event record: %s", hipGetErrorString(e));
    }
  }
  return 0;
}

extern "C" int tread_copy_async(void* dst, const void* src, size_t bytes, tread_stream_t stream,
                                tread_event_t done) {
  if (bytes == 0) return 0;
  if (!dst || !src) return tread::fail(TREAD_EINVAL, "tread_copy_async: null pointer");
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDefault, (hipStream_t)stream);
  if (e != hipSuccess) return tread::fail((int)e, "tread_copy_async: %s", hipGetErrorString(e));
  if (done) {
    e = hipEventRecord((hipEvent_t)done, (hipStream_t)stream);
    if (e != hipSuccess) return tread::fail((int)e, "tread_copy_async: event record: %s", hipGetErrorString(e));
  }
  return 0;
}
