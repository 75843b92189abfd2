// C ABI plumbing: error state, device / memory / stream / event calls, and the RNG key.
#include "common.hpp"

#include <cstdio>

namespace mk {

namespace {
thread_local std::string g_error;
}

void set_error(const std::string& msg) { g_error = msg; }

mk_status fail(mk_status s, const std::string& msg)
{
    g_error = msg;
    return s;
}

mk_status hip_check(hipError_t e, const char* what)
{
    g_error = std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")";
    return e == hipErrorOutOfMemory ? MK_ERR_NOMEM : MK_ERR_DEVICE;
}

// FNV-1a of the name mixed with the seed: the per-tensor stream of the counter RNG (the CPU reference keys its
// tensors the same way).
uint64_t tensor_key(uint64_t seed, const char* name)
{
    uint64_t h = 0xcbf29ce484222325ull;
    for (const char* p = name; *p; ++p)
        h = (h ^ uint8_t(*p)) * 0x100000001b3ull;
    return splitmix64(h ^ splitmix64(seed));
}

} // namespace mk

using namespace mk;

extern "C" {

const char* mk_last_error(void) { return g_error.c_str(); }
const char* mk_version(void) { return "mkimage 0.1 gfx950"; }

mk_status mk_device_count(int* n)
{
    if (!n)
        return fail(MK_ERR_ARG, "device_count: null");
    MK_HIP(hipGetDeviceCount(n));
    return MK_OK;
}

mk_status mk_set_device(int dev)
{
    MK_HIP(hipSetDevice(dev));
    return MK_OK;
}

mk_status mk_device_info(int dev, char* name, size_t name_len, int* cus, int* clock_khz, char* arch, size_t arch_len)
{
    hipDeviceProp_t p;
    MK_HIP(hipGetDeviceProperties(&p, dev));
    if (name && name_len) {
        // the marketing name comes from a table the driver package may lack; the architecture name always exists
        std::snprintf(name, name_len, "%s", p.name[0] ? p.name : p.gcnArchName);
    }
    if (arch && arch_len)
        std::snprintf(arch, arch_len, "%s", p.gcnArchName);
    if (cus)
        *cus = p.multiProcessorCount;
    if (clock_khz)
        *clock_khz = p.clockRate;
    return MK_OK;
}

mk_status mk_malloc(void** p, size_t bytes)
{
    if (!p)
        return fail(MK_ERR_ARG, "malloc: null");
    *p = nullptr;
    MK_HIP(hipMalloc(p, bytes ? bytes : 16));
    MK_HIP(hipMemset(*p, 0, bytes ? bytes : 16));
    MK_HIP(hipStreamSynchronize(nullptr)); // zero on return: work on non-blocking streams does not wait for it
    return MK_OK;
}

mk_status mk_free(void* p)
{
    if (p)
        MK_HIP(hipFree(p));
    return MK_OK;
}

mk_status mk_memcpy_h2d(void* dst, const void* src, size_t bytes)
{
    if (bytes && (!dst || !src))
        return fail(MK_ERR_ARG, "memcpy_h2d: null");
    MK_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return MK_OK;
}

mk_status mk_memcpy_d2h(void* dst, const void* src, size_t bytes)
{
    if (bytes && (!dst || !src))
        return fail(MK_ERR_ARG, "memcpy_d2h: null");
    MK_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return MK_OK;
}

mk_status mk_memset(void* p, int v, size_t bytes)
{
    if (bytes && !p)
        return fail(MK_ERR_ARG, "memset: null");
    MK_HIP(hipMemset(p, v, bytes));
    MK_HIP(hipStreamSynchronize(nullptr));
    return MK_OK;
}

mk_status mk_synchronize(void)
{
    MK_HIP(hipDeviceSynchronize());
    return gemm_take_error(nullptr, true);
}

mk_status mk_stream_create(void** s)
{
    if (!s)
        return fail(MK_ERR_ARG, "stream_create: null");
    hipStream_t st;
    MK_HIP(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    *s = st;
    return MK_OK;
}

mk_status mk_stream_destroy(void* s)
{
    if (s)
        MK_HIP(hipStreamDestroy(static_cast<hipStream_t>(s)));
    return MK_OK;
}

mk_status mk_stream_synchronize(void* s)
{
    MK_HIP(hipStreamSynchronize(static_cast<hipStream_t>(s)));
    return gemm_take_error(s);
}

mk_status mk_event_create(void** e)
{
    if (!e)
        return fail(MK_ERR_ARG, "event_create: null");
    hipEvent_t ev;
    MK_HIP(hipEventCreate(&ev));
    *e = ev;
    return MK_OK;
}

mk_status mk_event_destroy(void* e)
{
    if (e)
        MK_HIP(hipEventDestroy(static_cast<hipEvent_t>(e)));
    return MK_OK;
}

mk_status mk_event_record(void* e, void* stream)
{
    if (!e)
        return fail(MK_ERR_ARG, "event_record: null");
    MK_HIP(hipEventRecord(static_cast<hipEvent_t>(e), static_cast<hipStream_t>(stream)));
    return MK_OK;
}

mk_status mk_event_elapsed_ms(void* start, void* stop, float* ms)
{
    if (!start || !stop || !ms)
        return fail(MK_ERR_ARG, "event_elapsed: null");
    MK_HIP(hipEventSynchronize(static_cast<hipEvent_t>(stop)));
    MK_HIP(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)));
    return MK_OK;
}

uint64_t mk_tensor_key(uint64_t seed, const char* name) { return name ? tensor_key(seed, name) : 0; }

} // extern "C"
