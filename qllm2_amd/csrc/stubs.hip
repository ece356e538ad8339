// Entry points declared in qpam.h whose kernels are not in this build yet:
// they fail loudly with QPAM_ERR_UNSUPPORTED (there is no fallback path).
#include "common.h"

using qpam::fail;

extern "C" int qpam_decay_matrix(int32_t, int32_t, const float *, int64_t, float *, void *) {
    return fail(QPAM_ERR_UNSUPPORTED, "qpam_decay_matrix: not built yet");
}
extern "C" size_t qpam_ce_fwd_workspace_size(const qpam_ce_fwd_args *) { return 0; }
extern "C" int qpam_ce_fwd(const qpam_ce_fwd_args *, void *) {
    return fail(QPAM_ERR_UNSUPPORTED, "qpam_ce_fwd: not built yet");
}
extern "C" size_t qpam_ce_bwd_workspace_size(const qpam_ce_bwd_args *) { return 0; }
extern "C" int qpam_ce_bwd(const qpam_ce_bwd_args *, void *) {
    return fail(QPAM_ERR_UNSUPPORTED, "qpam_ce_bwd: not built yet");
}
