// Error reporting shared by every entry point of libtai_kernels.so.
#include <stdarg.h>

#include "common.h"

namespace tai {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return TAI_ERR_LAUNCH;
  }
  return TAI_OK;
}

// Read-dominated stream (measurement only): every 16 bytes of src read once with the non-temporal
// policy, 4 loads in flight per thread; the first w16 16-byte words of dst are written along the way
// (the value read at the same index, non-temporal stores: the fastest mix measured, 5.4 TB/s against
// 5.0 with plain stores and 4.4 with the writes spread evenly over the reads). The known byte counts of this kernel calibrate achieved HBM
// rates of read-heavy kernels (the grouped GEMMs read 93% of what they move).
namespace {
typedef int v4i_rs __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const v4i_rs gv4i_rs;
typedef __attribute__((address_space(1))) v4i_rs gv4i_rs_w;
__global__ __launch_bounds__(256) void read_stream_kernel(const v4i_rs* src, int64_t n16, v4i_rs* dst, int64_t w16) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const gv4i_rs* s = reinterpret_cast<const gv4i_rs*>(reinterpret_cast<uintptr_t>(src));
  gv4i_rs_w* o = reinterpret_cast<gv4i_rs_w*>(reinterpret_cast<uintptr_t>(dst));
  v4i_rs acc = {0, 0, 0, 0};
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const v4i_rs a = __builtin_nontemporal_load(s + i), b = __builtin_nontemporal_load(s + i + stride);
    const v4i_rs c = __builtin_nontemporal_load(s + i + 2 * stride), d = __builtin_nontemporal_load(s + i + 3 * stride);
    if (i < w16) __builtin_nontemporal_store(a, o + i);
    if (i + stride < w16) __builtin_nontemporal_store(b, o + i + stride);
    if (i + 2 * stride < w16) __builtin_nontemporal_store(c, o + i + 2 * stride);
    if (i + 3 * stride < w16) __builtin_nontemporal_store(d, o + i + 3 * stride);
    acc ^= a ^ b ^ c ^ d;
  }
  for (; i < n16; i += stride) {
    const v4i_rs a = __builtin_nontemporal_load(s + i);
    if (i < w16) __builtin_nontemporal_store(a, o + i);
    acc ^= a;
  }
  // a value that depends on every load (never true for a buffer of ones), so no load is dropped
  if (acc[0] == 0x7fffffff && acc[1] == 0x7fffffff && w16 > 0) dst[0] = acc;
}
}  // namespace
}  // namespace tai

extern "C" int tai_calib_read_stream(const void* src, size_t read_bytes, void* dst, size_t write_bytes, void* stream) {
  using namespace tai;
  TAI_CHECK_ARG(read_bytes % 16 == 0 && write_bytes % 16 == 0, "tai_calib_read_stream: sizes must be multiples of 16");
  TAI_CHECK_ARG(write_bytes <= read_bytes, "tai_calib_read_stream: write_bytes must not exceed read_bytes");
  TAI_CHECK_ARG((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) % 16 == 0,
                "tai_calib_read_stream: buffers must be 16-byte aligned");
  if (read_bytes == 0 && write_bytes == 0) return TAI_OK;
  TAI_CHECK_ARG((src || read_bytes == 0) && (dst || write_bytes == 0), "tai_calib_read_stream: null pointer");
  read_stream_kernel<<<16384, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const v4i_rs*>(src), static_cast<int64_t>(read_bytes / 16), static_cast<v4i_rs*>(dst),
      static_cast<int64_t>(write_bytes / 16));
  return launch_status("tai_calib_read_stream");
}

extern "C" const char* tai_last_error(void) { return tai::g_last_error; }
extern "C" int tai_abi_version(void) { return 1; }

#ifndef TAI_BUILD_ID
#define TAI_BUILD_ID "unversioned"
#endif
// Hash of the sources and flags this library was compiled from (set by the in-tree build).
extern "C" const char* tai_build_id(void) { return TAI_BUILD_ID; }
