// FlashAttention forward / JVP (placeholder until the MFMA kernels land).
#include "kf_common.h"

extern "C" int kf_fa_fwd(const void*, const void*, const void*, void*, float*, int64_t, int64_t,
                         int64_t, int64_t, int64_t, int64_t, float, int, int, kf_stream_t) {
    kf::set_error("kf_fa_fwd: not built yet");
    return KF_E_UNSUPPORTED;
}
extern "C" int kf_fa_jvp(const void*, const void*, const void*, const void*, const void*,
                         const void*, const void*, const float*, void*, int64_t, int64_t, int64_t,
                         int64_t, int64_t, int64_t, float, int, int, kf_stream_t) {
    kf::set_error("kf_fa_jvp: not built yet");
    return KF_E_UNSUPPORTED;
}
extern "C" int kf_fa_fwd_jvp(const void*, const void*, const void*, const void*, const void*,
                             const void*, void*, float*, void*, int64_t, int64_t, int64_t, int64_t,
                             int64_t, int64_t, float, int, int, kf_stream_t) {
    kf::set_error("kf_fa_fwd_jvp: not built yet");
    return KF_E_UNSUPPORTED;
}
