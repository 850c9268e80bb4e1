// Device selection and query (the reference's src/device.h:7-13; its CUDA
// implementation is src/cuda/cuda_probe.c). The environment variable names are
// the reference's, so the host's option handling drives this backend unchanged.
#include <hip/hip_runtime.h>
#include "../../include/h3_device.h"
#include <cerrno>
#include <climits>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <sys/sysinfo.h>

extern "C" int h3_device_configure(const char *index, const char *mode, char *error, size_t error_size) {
    if (index) {
        char *end;
        errno = 0;
        long n = strtol(index, &end, 10);
        if (!*index || *end || errno || n < 0 || n > INT_MAX) {
            if (error && error_size) snprintf(error, error_size, "invalid HIP device index: %s", index);
            return 0;
        }
        if (setenv("H3_CUDA_DEVICE", index, 1)) return 0;
    }
    if (mode) {
        if (strcmp(mode, "auto") && strcmp(mode, "resident") && strcmp(mode, "stream")) {
            if (error && error_size) snprintf(error, error_size, "weight mode must be auto, resident or stream");
            return 0;
        }
        if (setenv("H3_CUDA_WEIGHT_MODE", mode, 1)) return 0;
    }
    return 1;
}

extern "C" int h3_device_query(h3_device_info *info, char *error, size_t error_size) {
    if (!info) return 0;
    memset(info, 0, sizeof(*info));
    char index[32] = "0";
    if (const char *env = getenv("H3_CUDA_DEVICE")) {
        if (strlen(env) >= sizeof(index)) {
            if (error && error_size) snprintf(error, error_size, "invalid HIP device index");
            return 0;
        }
        strcpy(index, env);
    }
    if (!h3_device_configure(getenv("H3_CUDA_DEVICE") ? index : nullptr, getenv("H3_CUDA_WEIGHT_MODE"), error, error_size))
        return 0;
    const int device = (int)strtol(index, nullptr, 10);
    auto fail = [&](const char *what, hipError_t e) {
        if (error && error_size) snprintf(error, error_size, "%s: %s", what, hipGetErrorString(e));
        return 0;
    };
    hipError_t e = hipSetDevice(device);
    if (e != hipSuccess) return fail("HIP device", e);
    hipDeviceProp_t prop;
    if ((e = hipGetDeviceProperties(&prop, device)) != hipSuccess) return fail("HIP device properties", e);
    size_t available = 0, total = 0;
    if ((e = hipMemGetInfo(&available, &total)) != hipSuccess) return fail("HIP memory query", e);
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        if (error && error_size) snprintf(error, error_size, "this backend is built for gfx950; device %d is %s", device, prop.gcnArchName);
        return 0;
    }
    snprintf(info->name, sizeof(info->name), "%.*s", (int)sizeof(info->name) - 1, prop.name);
    snprintf(info->backend, sizeof(info->backend), "hip");
    snprintf(info->architecture, sizeof(info->architecture), "%s", prop.gcnArchName);
    info->device_index = device;
    info->cuda_compute_major = prop.major;
    info->cuda_compute_minor = prop.minor;
    info->device_memory = total;
    info->free_device_memory = available;
    info->recommended_working_set = total;
    info->max_buffer_length = total;
    info->multiprocessor_count = prop.multiProcessorCount;
    memcpy(info->cuda_uuid, prop.uuid.bytes, sizeof(info->cuda_uuid));
    hipDriverGetVersion(&info->cuda_driver_version);
    hipRuntimeGetVersion(&info->cuda_runtime_version);
    struct sysinfo host;
    if (!sysinfo(&host)) info->physical_memory = (uint64_t)host.totalram * host.mem_unit;
    return 1;
}

extern "C" int h3_device_memory_fits(uint64_t requested) {
    size_t available = 0, total = 0;
    if (hipMemGetInfo(&available, &total) != hipSuccess) return 0;
    const uint64_t reserve = total / 10;
    return available > reserve && requested <= available - reserve;
}
