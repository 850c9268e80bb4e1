// Process-wide device selection and query behind the reference's src/device.h
// (h3_device_query / h3_device_configure / h3_device_memory_fits). The
// selection travels in the environment variables the host's option handling
// already sets (H3_CUDA_DEVICE, H3_CUDA_WEIGHT_MODE), so `--device` and
// `--weight-mode` reach this backend unchanged; everything else is read from
// the HIP runtime. The backend is built for gfx950 code objects only, so a
// device of another architecture is refused at query time rather than at the
// first kernel launch.
#include <hip/hip_runtime.h>
#include "../../include/h3_device.h"
#include <climits>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <sys/sysinfo.h>

namespace {

const char *const kWeightModes[] = {"auto", "resident", "stream"};

// A device index is a plain decimal ordinal: digits only, no sign, fits an int.
bool parse_ordinal(const char *text, int *out) {
    if (!text || !*text) return false;
    long long value = 0;
    for (const char *p = text; *p; p++) {
        if (*p < '0' || *p > '9') return false;
        value = value * 10 + (*p - '0');
        if (value > INT_MAX) return false;
    }
    *out = (int)value;
    return true;
}

bool known_weight_mode(const char *mode) {
    for (const char *m : kWeightModes)
        if (!strcmp(mode, m)) return true;
    return false;
}

int report(char *error, size_t size, const char *fmt, const char *a = "", const char *b = "") {
    if (error && size) snprintf(error, size, fmt, a, b);
    return 0;
}

// Everything the query reports about one device, read with it current.
struct Snapshot {
    hipDeviceProp_t prop;
    size_t free_bytes = 0, total_bytes = 0;
    int driver = 0, runtime = 0;
};

hipError_t take_snapshot(int device, Snapshot *s) {
    hipError_t e = hipSetDevice(device);
    if (e == hipSuccess) e = hipGetDeviceProperties(&s->prop, device);
    if (e == hipSuccess) e = hipMemGetInfo(&s->free_bytes, &s->total_bytes);
    if (e == hipSuccess) {
        hipDriverGetVersion(&s->driver);
        hipRuntimeGetVersion(&s->runtime);
    }
    return e;
}

}  // namespace

extern "C" int h3_device_configure(const char *index, const char *mode, char *error, size_t error_size) {
    int ordinal = 0;
    if (index && !parse_ordinal(index, &ordinal))
        return report(error, error_size, "invalid HIP device index: %s", index);
    if (mode && !known_weight_mode(mode))
        return report(error, error_size, "weight mode must be auto, resident or stream");
    // Validate both before exporting either.
    if (index && setenv("H3_CUDA_DEVICE", index, 1) != 0) return report(error, error_size, "cannot set H3_CUDA_DEVICE");
    if (mode && setenv("H3_CUDA_WEIGHT_MODE", mode, 1) != 0)
        return report(error, error_size, "cannot set H3_CUDA_WEIGHT_MODE");
    return 1;
}

extern "C" int h3_device_query(h3_device_info *info, char *error, size_t error_size) {
    if (!info) return report(error, error_size, "missing device info");
    memset(info, 0, sizeof(*info));
    const char *selected = getenv("H3_CUDA_DEVICE");
    const char *mode = getenv("H3_CUDA_WEIGHT_MODE");
    int device = 0;
    if (selected && !parse_ordinal(selected, &device))
        return report(error, error_size, "invalid HIP device index: %s", selected);
    if (mode && !known_weight_mode(mode)) return report(error, error_size, "weight mode must be auto, resident or stream");

    Snapshot s;
    hipError_t e = take_snapshot(device, &s);
    if (e != hipSuccess) {
        char ordinal[16];
        snprintf(ordinal, sizeof(ordinal), "%d", device);
        return report(error, error_size, "HIP device %s: %s", ordinal, hipGetErrorString(e));
    }
    if (strncmp(s.prop.gcnArchName, "gfx950", 6) != 0)
        return report(error, error_size, "this backend is built for gfx950 (MI355X); the selected device is %s",
                      s.prop.gcnArchName);

    snprintf(info->name, sizeof(info->name), "%s", s.prop.name);
    snprintf(info->architecture, sizeof(info->architecture), "%s", s.prop.gcnArchName);
    snprintf(info->backend, sizeof(info->backend), "hip");
    info->device_index = device;
    info->cuda_compute_major = s.prop.major;
    info->cuda_compute_minor = s.prop.minor;
    info->cuda_driver_version = s.driver;
    info->cuda_runtime_version = s.runtime;
    info->device_memory = s.total_bytes;
    info->free_device_memory = s.free_bytes;
    // HBM is the working set: no unified memory, one buffer may span it all.
    info->recommended_working_set = s.total_bytes;
    info->max_buffer_length = s.total_bytes;
    info->multiprocessor_count = s.prop.multiProcessorCount;
    static_assert(sizeof(info->cuda_uuid) == sizeof(s.prop.uuid.bytes), "uuid size");
    memcpy(info->cuda_uuid, s.prop.uuid.bytes, sizeof(info->cuda_uuid));
    struct sysinfo host;
    if (sysinfo(&host) == 0) info->physical_memory = (uint64_t)host.totalram * host.mem_unit;
    return 1;
}

// Caches may stay resident while the next component still fits with a tenth
// of the device's memory held back for allocator slack and workspaces.
extern "C" int h3_device_memory_fits(uint64_t requested) {
    size_t free_bytes = 0, total_bytes = 0;
    if (hipMemGetInfo(&free_bytes, &total_bytes) != hipSuccess) return 0;
    const uint64_t held_back = total_bytes / 10;
    return free_bytes > held_back && requested <= free_bytes - held_back;
}
