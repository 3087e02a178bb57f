// C ABI entry points: argument checking, type dispatch and runtime plumbing.
#include <atomic>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <time.h>

#include "../../include/seedpack_amd.h"
#include "launch.h"

namespace spa {

namespace {
thread_local char g_err[512] = "";

struct TypeInfo { int type, qk, bs; };
// requant.py:21-27 (QFUN): ggml type -> block elements, block bytes.
constexpr TypeInfo kTypes[] = {
    {2, 32, 18},   {3, 32, 20},    {6, 32, 22},    {7, 32, 24},    {8, 32, 34},   {10, 256, 84},  {11, 256, 110},
    {12, 256, 144}, {13, 256, 176}, {14, 256, 210}, {16, 256, 66},  {17, 256, 74}, {18, 256, 98},  {19, 256, 50},
    {20, 32, 18},  {21, 256, 110}, {22, 256, 82},  {23, 256, 136}, {29, 256, 56}, {42, 64, 18},
};

const TypeInfo* find_type(int t) {
    for (const auto& e : kTypes)
        if (e.type == t) return &e;
    return nullptr;
}
}  // namespace

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int type_qk(int t) { const TypeInfo* e = find_type(t); return e ? e->qk : 0; }
int type_bs(int t) { const TypeInfo* e = find_type(t); return e ? e->bs : 0; }

}  // namespace spa

using spa::fail;

extern "C" {

const char* spa_last_error(void) { return spa::g_err; }

int spa_device_count(int* n) {
    SPA_HIP_TRY(hipGetDeviceCount(n));
    return SPA_OK;
}
int spa_set_device(int device) { SPA_HIP_TRY(hipSetDevice(device)); return SPA_OK; }
// How the library's own waits (stream synchronisation, the copies to and from the host) wait. The
// runtime's stream synchronisation spins the calling core until the work is done (an event made with
// hipEventBlockingSync spins as well once the device is in use); blocking waits record an event and
// poll it, sleeping between polls (20 us doubling to 500 us), so the core is free for host work at the
// cost of at most one sleep of latency per wait.
static std::atomic<int> g_blocking{0};

// the event's work done: polled with sleeps between polls when blocking, else the runtime's wait
static hipError_t wait_event(hipEvent_t ev) {
    if (!g_blocking.load(std::memory_order_relaxed)) return hipEventSynchronize(ev);
    for (unsigned us = 20;; us = us < 250 ? 2 * us : 500) {
        const hipError_t e = hipEventQuery(ev);
        if (e != hipErrorNotReady) return e;
        struct timespec ts = {0, (long)us * 1000};
        nanosleep(&ts, nullptr);
    }
}

static hipError_t wait_stream(hipStream_t s) {
    if (!g_blocking.load(std::memory_order_relaxed)) return hipStreamSynchronize(s);
    thread_local hipEvent_t ev = nullptr;   // one per thread and device (kept to the process's end)
    thread_local int ev_dev = -1;
    int d = 0;
    hipError_t e = hipGetDevice(&d);
    if (e != hipSuccess) return e;
    if (!ev || ev_dev != d) {
        e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
        if (e != hipSuccess) { ev = nullptr; return e; }
        ev_dev = d;
    }
    e = hipEventRecord(ev, s);
    return e == hipSuccess ? wait_event(ev) : e;
}

int spa_set_sync_mode(int blocking) {
    if (blocking != 0 && blocking != 1) return fail(SPA_ERR_ARG, "spa_set_sync_mode: %d", blocking);
    g_blocking.store(blocking);
    return SPA_OK;
}
int spa_get_device(int* device) {
    if (!device) return fail(SPA_ERR_ARG, "spa_get_device: null out pointer");
    SPA_HIP_TRY(hipGetDevice(device));
    return SPA_OK;
}
int spa_malloc(void** ptr, size_t nbytes) {
    if (!ptr) return fail(SPA_ERR_ARG, "spa_malloc: null out pointer");
    SPA_HIP_TRY(hipMalloc(ptr, nbytes ? nbytes : 1));
    return SPA_OK;
}
int spa_free(void* ptr) { SPA_HIP_TRY(hipFree(ptr)); return SPA_OK; }
int spa_host_alloc(void** ptr, size_t nbytes) {
    if (!ptr) return fail(SPA_ERR_ARG, "spa_host_alloc: null out pointer");
    SPA_HIP_TRY(hipHostMalloc(ptr, nbytes ? nbytes : 1, hipHostMallocDefault));
    return SPA_OK;
}
int spa_host_free(void* ptr) { SPA_HIP_TRY(hipHostFree(ptr)); return SPA_OK; }
int spa_memcpy_h2d(void* dst, const void* src, size_t n, void* s) {
    SPA_HIP_TRY(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, (hipStream_t)s));
    SPA_HIP_TRY(wait_stream((hipStream_t)s));
    return SPA_OK;
}
int spa_memcpy_d2h(void* dst, const void* src, size_t n, void* s) {
    SPA_HIP_TRY(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, (hipStream_t)s));
    SPA_HIP_TRY(wait_stream((hipStream_t)s));
    return SPA_OK;
}
int spa_memcpy_d2h_async(void* dst, const void* src, size_t n, void* s) {
    SPA_HIP_TRY(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, (hipStream_t)s));
    return SPA_OK;
}
int spa_memcpy_d2d(void* dst, const void* src, size_t n, void* s) {
    SPA_HIP_TRY(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, (hipStream_t)s));
    return SPA_OK;
}
int spa_memset(void* p, int v, size_t n, void* s) { SPA_HIP_TRY(hipMemsetAsync(p, v, n, (hipStream_t)s)); return SPA_OK; }
int spa_stream_create(void** s) { SPA_HIP_TRY(hipStreamCreateWithFlags((hipStream_t*)s, hipStreamNonBlocking)); return SPA_OK; }
int spa_stream_destroy(void* s) { SPA_HIP_TRY(hipStreamDestroy((hipStream_t)s)); return SPA_OK; }
int spa_stream_synchronize(void* s) { SPA_HIP_TRY(wait_stream((hipStream_t)s)); return SPA_OK; }
int spa_device_synchronize(void) { SPA_HIP_TRY(hipDeviceSynchronize()); return SPA_OK; }
int spa_event_create(void** e) { SPA_HIP_TRY(hipEventCreate((hipEvent_t*)e)); return SPA_OK; }
int spa_event_destroy(void* e) { SPA_HIP_TRY(hipEventDestroy((hipEvent_t)e)); return SPA_OK; }
int spa_event_record(void* e, void* s) { SPA_HIP_TRY(hipEventRecord((hipEvent_t)e, (hipStream_t)s)); return SPA_OK; }
int spa_stream_wait_event(void* s, void* e) { SPA_HIP_TRY(hipStreamWaitEvent((hipStream_t)s, (hipEvent_t)e, 0)); return SPA_OK; }
int spa_event_elapsed_ms(float* ms, void* a, void* b) {
    SPA_HIP_TRY(hipEventSynchronize((hipEvent_t)b));
    SPA_HIP_TRY(hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b));
    return SPA_OK;
}
int spa_event_synchronize(void* e) { SPA_HIP_TRY(wait_event((hipEvent_t)e)); return SPA_OK; }
int spa_mem_info(size_t* f, size_t* t) { SPA_HIP_TRY(hipMemGetInfo(f, t)); return SPA_OK; }

uint64_t spa_gguf_strings_bytes(const void* p, uint64_t avail, uint64_t count) {
    // GGUF strings: a little-endian uint64 length, then that many bytes
    const unsigned char* b = static_cast<const unsigned char*>(p);
    uint64_t pos = 0;
    for (uint64_t i = 0; i < count; ++i) {
        if (!b || avail - pos < 8) return UINT64_MAX;
        uint64_t n;
        memcpy(&n, b + pos, 8);
        if (n > avail - pos - 8) return UINT64_MAX;
        pos += 8 + n;
    }
    return pos;
}

size_t spa_row_size(int t, int64_t npr) {
    const int qk = spa::type_qk(t), bs = spa::type_bs(t);
    if (!qk || npr <= 0 || npr % qk) return 0;
    return (size_t)(npr / qk) * (size_t)bs;
}

int spa_type_variants(int t) {
    if (!spa::find_type(t)) return 0;
    return t == 29 ? 2 : 1;
}

uint64_t spa_quantize_work_bytes(int t, int64_t nrows, int64_t n_per_row, int has_imatrix) {
    (void)n_per_row;
    return (uint64_t)spa::quantize_work_bytes(t, nrows, has_imatrix != 0);
}

int spa_quantize(int t, int variant, const void* src, int src_kind, int64_t nrows, int64_t npr, const float* imatrix,
                 void* dst, void* work, void* stream) {
    const int qk = spa::type_qk(t);
    if (!qk) return fail(SPA_ERR_TYPE, "spa_quantize: unknown ggml type %d", t);
    if (variant < 0 || variant >= spa_type_variants(t))
        return fail(SPA_ERR_TYPE, "spa_quantize: type %d has no variant %d", t, variant);
    if (src_kind < SPA_SRC_BF16 || src_kind > SPA_SRC_F32) return fail(SPA_ERR_ARG, "spa_quantize: bad src_kind %d", src_kind);
    if (nrows < 0 || npr <= 0 || npr % qk) return fail(SPA_ERR_ARG, "spa_quantize: n_per_row %lld is not a multiple of %d",
                                                       (long long)npr, qk);
    if (nrows == 0) return SPA_OK;
    if (!src || !dst) return fail(SPA_ERR_ARG, "spa_quantize: null src/dst");
    if ((reinterpret_cast<uintptr_t>(src) & 15u) || (reinterpret_cast<uintptr_t>(dst) & 1u))
        return fail(SPA_ERR_ARG, "spa_quantize: src must be 16-byte and dst 2-byte aligned");
    if (imatrix && (reinterpret_cast<uintptr_t>(imatrix) & 3u)) return fail(SPA_ERR_ARG, "spa_quantize: misaligned imatrix");
    // IQ2_XXS, IQ2_XS, IQ1_S assert an imatrix (ggml-quants.c:3303, :3481, :4528)
    if (!imatrix && (t == 16 || t == 17 || t == 19))
        return fail(SPA_ERR_ASSERT, "spa_quantize: type %d requires an imatrix", t);
    if (work && (reinterpret_cast<uintptr_t>(work) & 3u)) return fail(SPA_ERR_ARG, "spa_quantize: misaligned work");
    spa::QuantArgs a{t, variant, src, src_kind, nrows, npr, imatrix, dst, (hipStream_t)stream, (float*)work};
    switch (t) {
        case 2: case 3: case 6: case 7: case 8: case 42: return spa::launch_legacy(a);
        case 10: case 11: case 12: case 13: case 14: return spa::launch_kquant(a);
        case 20: case 23: return spa::launch_iq4(a);
        default: return spa::launch_iqgrid(a);
    }
}

}  // extern "C"
