// SANA ReLU linear attention (placeholder until the MFMA kernels land).
#include "kf_common.h"

extern "C" int64_t kf_linattn_default_splits(int64_t, int64_t, int64_t, int64_t) { return 1; }
extern "C" int64_t kf_linattn_workspace_bytes(int64_t, int64_t, int64_t, int64_t) { return 0; }
extern "C" int kf_linattn_fwd(const void*, void*, void*, int64_t, int64_t, int64_t, int64_t,
                              int64_t, int64_t, float, int, int, kf_stream_t) {
    kf::set_error("kf_linattn_fwd: not built yet");
    return KF_E_UNSUPPORTED;
}
