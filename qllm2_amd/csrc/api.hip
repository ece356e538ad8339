// Error plumbing and version of the qpam C ABI.
#include <map>

#include "common.h"

namespace qpam {

std::string &last_error_slot() {
    static thread_local std::string msg;
    return msg;
}

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    last_error_slot() = buf;
    return code;
}

}  // namespace qpam

namespace qpam {
std::mutex &side_stream_mutex() {
    static std::mutex mu;
    return mu;
}

int side_stream(SideStream *&out) {
    static std::map<int, SideStream> streams;  // guarded by side_stream_mutex()
    int dev = 0;
    QPAM_CHECK_HIP(hipGetDevice(&dev));
    auto it = streams.find(dev);
    if (it == streams.end()) {
        SideStream s;
        QPAM_CHECK_HIP(hipStreamCreateWithFlags(&s.side, hipStreamNonBlocking));
        QPAM_CHECK_HIP(hipEventCreateWithFlags(&s.fork, hipEventDisableTiming));
        QPAM_CHECK_HIP(hipEventCreateWithFlags(&s.join, hipEventDisableTiming));
        it = streams.emplace(dev, s).first;
    }
    out = &it->second;
    return QPAM_OK;
}
}  // namespace qpam

extern "C" int qpam_version(void) { return 14; }

extern "C" const char *qpam_last_error(void) { return qpam::last_error_slot().c_str(); }

extern "C" int qpam_event_create(void **ev) {
    QPAM_REQUIRE(ev != nullptr, "qpam_event_create: null out pointer");
    hipEvent_t e;
    QPAM_CHECK_HIP(hipEventCreate(&e));
    *ev = (void *)e;
    return QPAM_OK;
}

extern "C" int qpam_event_destroy(void *ev) {
    if (ev) QPAM_CHECK_HIP(hipEventDestroy((hipEvent_t)ev));
    return QPAM_OK;
}

extern "C" int qpam_event_elapsed_ms(void *ev0, void *ev1, float *ms) {
    QPAM_REQUIRE(ev0 && ev1 && ms, "qpam_event_elapsed_ms: null argument");
    QPAM_CHECK_HIP(hipEventElapsedTime(ms, (hipEvent_t)ev0, (hipEvent_t)ev1));
    return QPAM_OK;
}
