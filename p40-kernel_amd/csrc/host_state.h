// host_state.h -- the library's only mutable host state, made safe for
// concurrent callers on any number of devices.
//
//  * Tuning knobs (BONSAI_* environment variables, used by tests and sweeps to
//    pick a kernel variant, and the ggml hook's opt-in switches) are read
//    once, on first use, into atomics; the launch paths then read integers,
//    never the environment.
//    bonsai_p40_reload_tuning() re-reads them (a test that changes a variable
//    calls it).
//  * Device properties (CU count, LDS per workgroup) are cached per device id,
//    each filled exactly once (std::call_once).
//  * Per-kernel attributes (the dynamic-LDS limit) are set once per kernel and
//    device, also under std::call_once.
// It also holds the NULL-pointer check every entry point applies.
// Everything here is host code; inline functions with static locals have one
// instance per process across the library's translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <climits>
#include <cstdlib>
#include <mutex>

namespace pq2host {

enum Knob : int {
    K_GEMV_UNITS_PER_WAVE,
    K_GEMV_XCD_LOG2M,
    K_GEMV_WG_PER_CU,
    K_GEMV_KERNEL,
    K_MFMA4_WG_PER_CU,
    K_MFMA4_WAVES,
    K_MFMA4_MIN_TOK,
    K_FGEMV_WAVES,
    K_FGEMV_OVL,
    K_GEMM_SMALL_GEMV,
    K_GEMM_BD,
    K_GEMM_SMALL,
    K_GEMM_SMALL_CFG,
    K_GEMM_KERNEL,
    K_GEMM_F16_BN,
    K_GEMM_F16_SPLIT,
    K_GEMM_F16_WAVES,
    K_GEMM_WIDE,
    K_GEMM_WIDE_MI,
    K_GEMV_TAIL,
    K_FFN_QUAD,
    K_GGML_ENABLE,
    K_GGML_VERBOSE,
    K_COUNT
};

inline const char * knob_name(int k) {
    static const char * const names[K_COUNT] = {
        "BONSAI_GEMV_UNITS_PER_WAVE", "BONSAI_GEMV_XCD_LOG2M", "BONSAI_GEMV_WG_PER_CU",
        "BONSAI_GEMV_KERNEL",         "BONSAI_MFMA4_WG_PER_CU", "BONSAI_MFMA4_WAVES",
        "BONSAI_MFMA4_MIN_TOK",       "BONSAI_FGEMV_WAVES",     "BONSAI_FGEMV_OVL",
        "BONSAI_GEMM_SMALL_GEMV",     "BONSAI_GEMM_BD",         "BONSAI_GEMM_SMALL",
        "BONSAI_GEMM_SMALL_CFG",      "BONSAI_GEMM_KERNEL",     "BONSAI_GEMM_F16_BN",
        "BONSAI_GEMM_F16_SPLIT",      "BONSAI_GEMM_F16_WAVES",  "BONSAI_GEMM_WIDE",
        "BONSAI_GEMM_WIDE_MI",        "BONSAI_GEMV_TAIL",       "BONSAI_FFN_QUAD",
        "BONSAI_P40",                 "BONSAI_P40_VERBOSE",
    };
    return names[k];
}

constexpr int KNOB_UNSET = INT_MIN;

struct KnobTable {
    std::atomic<int> v[K_COUNT];
    std::once_flag loaded;
    std::mutex reload_mu;
};

inline KnobTable & knob_table() {
    static KnobTable t;
    return t;
}

// one pass over the environment (getenv is not called concurrently with a
// setenv of the caller's own making: the caller owns that race)
inline void read_knobs(KnobTable & t) {
    for (int k = 0; k < K_COUNT; ++k) {
        const char * s = getenv(knob_name(k));
        t.v[k].store((s && *s) ? atoi(s) : KNOB_UNSET, std::memory_order_relaxed);
    }
}

// value of knob k, or dflt when the variable is unset or empty
inline int knob(Knob k, int dflt) {
    KnobTable & t = knob_table();
    std::call_once(t.loaded, [&t] { read_knobs(t); });
    const int v = t.v[k].load(std::memory_order_relaxed);
    return v == KNOB_UNSET ? dflt : v;
}

inline void reload_knobs() {
    KnobTable & t = knob_table();
    std::call_once(t.loaded, [&t] { read_knobs(t); });
    std::lock_guard<std::mutex> g(t.reload_mu);
    read_knobs(t);
}

// ---- per-device caches ------------------------------------------------------
constexpr int MAX_DEVICES = 64;

// the calling thread's current device (0 if the runtime cannot say; the
// launch that follows then reports the runtime's error)
inline int current_device() {
    int d = 0;
    if (hipGetDevice(&d) != hipSuccess) {
        (void)hipGetLastError();
        d = 0;
    }
    return d;
}

struct DeviceInfo {
    int cus = 256;                    // compute units
    int max_lds = 64 * 1024;          // LDS bytes one workgroup may allocate
};

inline DeviceInfo query_device(int dev) {
    DeviceInfo di;
    int x = 0;
    if (hipDeviceGetAttribute(&x, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && x > 0) di.cus = x;
    else (void)hipGetLastError();
    x = 0;
    if (hipDeviceGetAttribute(&x, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess && x > 0)
        di.max_lds = x;
    else (void)hipGetLastError();
    return di;
}

// properties of the calling thread's current device, queried once per device
inline DeviceInfo device_info() {
    static std::once_flag once[MAX_DEVICES];
    static DeviceInfo info[MAX_DEVICES];
    const int d = current_device();
    if (d < 0 || d >= MAX_DEVICES) return query_device(d);
    std::call_once(once[d], [d] { info[d] = query_device(d); });
    return info[d];
}

// One flag per device for a per-kernel, per-device set-up step (a kernel's
// dynamic-LDS limit): declare `static PerDeviceOnce o;` at the launch site.
struct PerDeviceOnce {
    std::once_flag f[MAX_DEVICES];
};

template <class Fn>
inline void once_per_device(PerDeviceOnce & o, Fn && fn) {
    const int d = current_device();
    if (d < 0 || d >= MAX_DEVICES) {
        fn();
        return;
    }
    std::call_once(o.f[d], fn);
}

// Raise a kernel's dynamic-LDS limit; a refused request must not linger as
// the next launch's error.
inline void set_max_dynamic_lds(const void * kern, int bytes) {
    if (hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, bytes) != hipSuccess)
        (void)hipGetLastError();
}

// Argument check shared by the entry points: true if any of the device
// pointers the requested work reads or writes is NULL.
template <class... P>
inline bool any_null(const P *... p) {
    return ((p == nullptr) || ...);
}

}  // namespace pq2host
