// Library identification and error reporting for the C ABI.
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <set>
#include <utility>

#include "nq_internal.hpp"

namespace nq {

namespace {
thread_local char g_last_error[512] = "";
}

nq_status fail(nq_status st, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return st;
}

nq_status launch_status(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(NQ_HIP_ERROR, "%s: %s", what, hipGetErrorString(e));
    return NQ_OK;
}

nq_status set_dynamic_lds(const void* fn, size_t bytes, const char* who) {
    static std::mutex mu;
    static std::set<std::pair<const void*, int>> done;
    int dev = 0;
    if (hipError_t e = hipGetDevice(&dev); e != hipSuccess)
        return fail(NQ_HIP_ERROR, "%s: hipGetDevice: %s", who, hipGetErrorString(e));
    std::lock_guard<std::mutex> lock(mu);
    if (done.count({fn, dev})) return NQ_OK;
    const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
    if (e != hipSuccess) return fail(NQ_HIP_ERROR, "%s: LDS attribute: %s", who, hipGetErrorString(e));
    done.insert({fn, dev});
    return NQ_OK;
}

}  // namespace nq

extern "C" {

const char* nq_version(void) { return "nq_hip 0.1 gfx950"; }

const char* nq_status_name(int status) {
    switch (status) {
        case NQ_OK: return "NQ_OK";
        case NQ_BAD_SHAPE: return "NQ_BAD_SHAPE";
        case NQ_BAD_ALIGN: return "NQ_BAD_ALIGN";
        case NQ_HIP_ERROR: return "NQ_HIP_ERROR";
        case NQ_BAD_ARG: return "NQ_BAD_ARG";
        case NQ_IO_ERROR: return "NQ_IO_ERROR";
    }
    return "NQ_UNKNOWN";
}

const char* nq_last_error(void) { return nq::g_last_error; }

}  // extern "C"
