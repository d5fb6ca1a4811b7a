// npu_fused_infer_attention_score kernels (placeholder entry points until the kernels land).
#include "common.h"

extern "C" size_t tai_fia_paged_decode_workspace_size(int64_t, int, int, int64_t, int) { return 0; }
extern "C" int tai_fia_paged_decode(const void*, const void*, const void*, int64_t, int64_t, int64_t, const int32_t*,
                                    int64_t, const int64_t*, int64_t, int, int, int, int, float, void*, float*, void*,
                                    size_t, void*) {
  tai::set_error("tai_fia_paged_decode: not implemented yet");
  return TAI_ERR_UNSUPPORTED;
}
extern "C" int tai_fia_prefill(const void*, const void*, const void*, int64_t, int64_t, int64_t, int, int, int,
                               const int64_t*, const int64_t*, const int64_t*, const int64_t*, const int64_t*,
                               const int64_t*, int, float, void*, float*, void*) {
  tai::set_error("tai_fia_prefill: not implemented yet");
  return TAI_ERR_UNSUPPORTED;
}
extern "C" size_t tai_fia_mla_decode_workspace_size(int64_t, int, int, int64_t, int) { return 0; }
extern "C" int tai_fia_mla_decode(const void*, const void*, const int8_t*, const float*, const void*, const int32_t*,
                                  int64_t, const int64_t*, int64_t, int, int, int, int, float, void*, float*, void*,
                                  size_t, void*) {
  tai::set_error("tai_fia_mla_decode: not implemented yet");
  return TAI_ERR_UNSUPPORTED;
}
