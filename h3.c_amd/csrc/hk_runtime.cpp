/* Runtime half of the MI355X HIP backend: device context, tensors and their
 * caching allocator, host<->device transfers, batches, errors, stats,
 * per-op event timing.  Kernels live in the hk_*.hip units.
 *
 * Reference counterpart: h3_gpu_cuda.cu (context :81-142, block cache
 * :199-260, transfers :262-430, batches :871-905).  Differences by design:
 *   - one non-default HIP stream per context instead of the legacy default
 *     stream, so the library never serialises against unrelated work in the
 *     host process;
 *   - uploads are enqueued on that stream and the call returns once the
 *     source buffer has been consumed (the caller may reuse it at once, the
 *     same observable contract as the reference's pinned ring);
 *   - no vendor-library handles: every GEMM is a hand-written MFMA kernel.
 */
#include "hk_internal.h"

#include <errno.h>
#include <fcntl.h>
#include <stdlib.h>
#include <sys/stat.h>
#include <time.h>
#include <unistd.h>

#include <mutex>
#include <string>
#include <thread>
#include <vector>

double hk_now(void) {
    struct timespec stamp;
    clock_gettime(CLOCK_MONOTONIC, &stamp);
    return (double)stamp.tv_sec + (double)stamp.tv_nsec * 1e-9;
}

/* ------------------------------------------------------------ allocator */

struct hk_cache_block {
    void *data;
    size_t bytes;
    hk_cache_block *next;
};

static void hk_cache_evict(struct h3_gpu *gpu, size_t keep) {
    while (gpu->cache && gpu->cache_bytes > keep) {
        hk_cache_block *block = gpu->cache;
        gpu->cache = block->next;
        gpu->cache_bytes -= block->bytes;
        (void)hipFree(block->data);
        free(block);
    }
}

/* Blocks are rounded to 256 B so that tensors whose sizes differ by a few
 * elements share cache entries; every kernel may then use 16-byte vector
 * accesses on the tail without leaving the allocation. */
static size_t hk_round_bytes(size_t bytes) {
    if (!bytes) bytes = 1;
    return (bytes + 255) & ~(size_t)255;
}

static void *hk_device_alloc(struct h3_gpu *gpu, size_t bytes) {
    bytes = hk_round_bytes(bytes);
    hk_cache_block **link = &gpu->cache;
    while (*link) {
        if ((*link)->bytes == bytes) {
            hk_cache_block *block = *link;
            *link = block->next;
            gpu->cache_bytes -= bytes;
            void *data = block->data;
            free(block);
            return data;
        }
        link = &(*link)->next;
    }
    void *data = NULL;
    gpu->device_mallocs++;
    hipError_t status = hipMalloc(&data, bytes);
    if (status != hipSuccess) {
        (void)hipGetLastError();
        /* release cached blocks and retry once */
        (void)hipStreamSynchronize(gpu->stream);
        hk_cache_evict(gpu, 0);
        gpu->device_mallocs++;
        status = hipMalloc(&data, bytes);
        if (status != hipSuccess) {
            (void)hipGetLastError();
            hk_fail_hip(gpu, "device allocation", status);
            return NULL;
        }
    }
    return data;
}

static void hk_device_release(struct h3_gpu *gpu, void *data, size_t bytes) {
    bytes = hk_round_bytes(bytes);
    hk_cache_block *block = (hk_cache_block *)malloc(sizeof(*block));
    if (!block) {
        (void)hipStreamSynchronize(gpu->stream);
        (void)hipFree(data);
        return;
    }
    /* Stream order keeps reuse safe: a recycled block is only touched by
     * work enqueued after every kernel that used its previous owner. */
    block->data = data;
    block->bytes = bytes;
    block->next = gpu->cache;
    gpu->cache = block;
    gpu->cache_bytes += bytes;
    if (gpu->cache_bytes > gpu->cache_limit) {
        (void)hipStreamSynchronize(gpu->stream);
        hk_cache_evict(gpu, gpu->cache_limit / 2);
    }
}

static void *hk_grow(struct h3_gpu *gpu, void **buffer, size_t *have,
                     size_t bytes, const char *what) {
    if (!bytes) bytes = 1;
    if (*buffer && bytes <= *have) return *buffer;
    size_t capacity = *have ? *have : 1u << 20;
    while (capacity < bytes) capacity *= 2;
    /* in-flight kernels may still read the old block */
    (void)hipStreamSynchronize(gpu->stream);
    if (*buffer) (void)hipFree(*buffer);
    *buffer = NULL;
    *have = 0;
    void *fresh = NULL;
    gpu->device_mallocs++;
    hipError_t status = hipMalloc(&fresh, capacity);
    if (status != hipSuccess) {
        (void)hipGetLastError();
        hk_fail_hip(gpu, what, status);
        return NULL;
    }
    *buffer = fresh;
    *have = capacity;
    return fresh;
}

void *hk_workspace(struct h3_gpu *gpu, size_t bytes) {
    return hk_grow(gpu, &gpu->workspace, &gpu->workspace_bytes, bytes,
                   "workspace allocation");
}

void *hk_splitk_space(struct h3_gpu *gpu, size_t bytes) {
    return hk_grow(gpu, &gpu->splitk, &gpu->splitk_bytes, bytes,
                   "split-K scratch allocation");
}

/* --------------------------------------------------------------- timing */

struct hk_timed_launch {
    std::string name;
    hipEvent_t start, stop;
};

struct hk_timing {
    int enabled;
    std::vector<hk_timed_launch> launches;
    std::vector<hipEvent_t> pool;
    hipEvent_t pending_start;
    int pending;
};

static hipEvent_t hk_timing_event(hk_timing *timing) {
    if (!timing->pool.empty()) {
        hipEvent_t event = timing->pool.back();
        timing->pool.pop_back();
        return event;
    }
    hipEvent_t event = NULL;
    if (hipEventCreate(&event) != hipSuccess) {
        (void)hipGetLastError();
        return NULL;
    }
    return event;
}

void hk_op_begin(struct h3_gpu *gpu, const char *name) {
    (void)name;
    hk_timing *timing = gpu->timing;
    if (!timing || !timing->enabled) return;
    timing->pending_start = hk_timing_event(timing);
    timing->pending = timing->pending_start != NULL;
    if (timing->pending)
        (void)hipEventRecord(timing->pending_start, gpu->stream);
}

int hk_op_end(struct h3_gpu *gpu, const char *name, int kind) {
    hipError_t status = hipGetLastError();
    hk_timing *timing = gpu->timing;
    if (timing && timing->enabled && timing->pending) {
        hipEvent_t stop = hk_timing_event(timing);
        if (stop) {
            (void)hipEventRecord(stop, gpu->stream);
            timing->launches.push_back(
                hk_timed_launch{name, timing->pending_start, stop});
        } else {
            timing->pool.push_back(timing->pending_start);
        }
        timing->pending = 0;
    }
    if (status != hipSuccess) return hk_fail_hip(gpu, name, status);
    if (kind == HK_KIND_LINEAR) gpu->stats.mps_linear_dispatches++;
    else if (kind == HK_KIND_CONV) gpu->stats.mps_conv_dispatches++;
    else if (kind == HK_KIND_SDPA) gpu->stats.mps_sdpa_dispatches++;
    else gpu->stats.direct_dispatches++;
    return 1;
}

extern "C" int h3_hip_op_timing_enable(h3_gpu *gpu, int enable) {
    if (!gpu) return 0;
    if (!gpu->timing) gpu->timing = new hk_timing();
    gpu->timing->enabled = enable ? 1 : 0;
    return 1;
}

extern "C" int h3_hip_op_timing_reset(h3_gpu *gpu) {
    if (!gpu || !gpu->timing) return 0;
    (void)hipStreamSynchronize(gpu->stream);
    for (auto &launch : gpu->timing->launches) {
        gpu->timing->pool.push_back(launch.start);
        gpu->timing->pool.push_back(launch.stop);
    }
    gpu->timing->launches.clear();
    return 1;
}

extern "C" int h3_hip_op_timing_read(h3_gpu *gpu, const char *prefix,
                                     uint64_t *count, double *milliseconds) {
    if (!gpu || !gpu->timing) return hk_fail(gpu, "op timing is not enabled");
    hipError_t status = hipStreamSynchronize(gpu->stream);
    if (status != hipSuccess) return hk_fail_hip(gpu, "timing wait", status);
    size_t length = prefix ? strlen(prefix) : 0;
    uint64_t n = 0;
    double total = 0.0;
    for (auto &launch : gpu->timing->launches) {
        if (length && launch.name.compare(0, length, prefix) != 0) continue;
        float elapsed = 0.0f;
        if (hipEventElapsedTime(&elapsed, launch.start, launch.stop) !=
            hipSuccess) {
            (void)hipGetLastError();
            continue;
        }
        n++;
        total += elapsed;
    }
    if (count) *count = n;
    if (milliseconds) *milliseconds = total;
    return 1;
}

extern "C" int h3_hip_op_timing_names(h3_gpu *gpu, char *buffer,
                                      size_t buffer_size) {
    if (!gpu || !gpu->timing || !buffer || !buffer_size) return 0;
    std::vector<std::string> names;
    for (auto &launch : gpu->timing->launches) {
        bool seen = false;
        for (auto &name : names) seen = seen || name == launch.name;
        if (!seen) names.push_back(launch.name);
    }
    std::string joined;
    for (auto &name : names) { joined += name; joined += '\n'; }
    snprintf(buffer, buffer_size, "%s", joined.c_str());
    return 1;
}

extern "C" uint64_t h3_hip_device_allocations(const h3_gpu *gpu) {
    return gpu ? gpu->device_mallocs : 0;
}

extern "C" int h3_hip_marker(h3_gpu *gpu, int slot) {
    if (!gpu || slot < 0 || slot >= 16) return 0;
    if (!gpu->marker_valid[slot]) {
        if (hipEventCreate(&gpu->markers[slot]) != hipSuccess)
            return hk_fail(gpu, "cannot create marker event");
        gpu->marker_valid[slot] = 1;
    }
    hipError_t status = hipEventRecord(gpu->markers[slot], gpu->stream);
    if (status != hipSuccess) return hk_fail_hip(gpu, "marker", status);
    return 1;
}

extern "C" int h3_hip_marker_elapsed(h3_gpu *gpu, int from_slot,
                                     int to_slot, double *milliseconds) {
    if (!gpu || from_slot < 0 || from_slot >= 16 || to_slot < 0 ||
        to_slot >= 16 || !gpu->marker_valid[from_slot] ||
        !gpu->marker_valid[to_slot])
        return hk_fail(gpu, "invalid marker slots");
    hipError_t status = hipEventSynchronize(gpu->markers[to_slot]);
    if (status != hipSuccess) return hk_fail_hip(gpu, "marker wait", status);
    float elapsed = 0.0f;
    status = hipEventElapsedTime(&elapsed, gpu->markers[from_slot],
                                 gpu->markers[to_slot]);
    if (status != hipSuccess) return hk_fail_hip(gpu, "marker read", status);
    if (milliseconds) *milliseconds = elapsed;
    return 1;
}

/* -------------------------------------------------------------- context */

extern "C" int h3_hip_probe(struct h3_hip_device_info *info, char *error,
                            size_t error_size) {
    if (!info) return 0;
    memset(info, 0, sizeof(*info));
    int count = 0;
    hipError_t status = hipGetDeviceCount(&count);
    if (status != hipSuccess || count < 1) {
        if (error && error_size)
            snprintf(error, error_size, "no HIP device available: %s",
                     hipGetErrorString(status));
        return 0;
    }
    hipDeviceProp_t properties;
    status = hipGetDeviceProperties(&properties, 0);
    if (status != hipSuccess) {
        if (error && error_size)
            snprintf(error, error_size, "cannot query HIP device: %s",
                     hipGetErrorString(status));
        return 0;
    }
    snprintf(info->name, sizeof(info->name), "%.127s", properties.name);
    snprintf(info->architecture, sizeof(info->architecture), "%.127s",
             properties.gcnArchName);
    long pages = sysconf(_SC_PHYS_PAGES);
    long page_size = sysconf(_SC_PAGESIZE);
    if (pages > 0 && page_size > 0)
        info->physical_memory = (uint64_t)pages * (uint64_t)page_size;
    info->recommended_working_set = properties.totalGlobalMem;
    info->max_buffer_length = properties.totalGlobalMem;
    return 1;
}

static int hk_env_flag(const char *name) {
    const char *value = getenv(name);
    return value && *value && strcmp(value, "0") != 0;
}

static bool hk_loader_new(struct h3_gpu *gpu);
static void hk_loader_free(struct h3_gpu *gpu);

extern "C" h3_gpu *h3_gpu_create(const char *shader_source_path,
                                 char *error, size_t error_size) {
    (void)shader_source_path; /* kernels are compiled into the library */
    int count = 0;
    hipError_t status = hipGetDeviceCount(&count);
    if (status != hipSuccess || count < 1) {
        if (error && error_size)
            snprintf(error, error_size, "no HIP device available: %s",
                     hipGetErrorString(status));
        return NULL;
    }
    struct h3_gpu *gpu = (struct h3_gpu *)calloc(1, sizeof(*gpu));
    if (!gpu) {
        if (error && error_size) snprintf(error, error_size, "out of memory");
        return NULL;
    }
    gpu->device = 0;
    status = hipSetDevice(0);
    if (status == hipSuccess)
        status = hipStreamCreateWithFlags(&gpu->stream, hipStreamNonBlocking);
    if (status != hipSuccess) {
        if (error && error_size)
            snprintf(error, error_size, "cannot initialise HIP device: %s",
                     hipGetErrorString(status));
        free(gpu);
        return NULL;
    }
    size_t available = 0, total = 0;
    if (hipMemGetInfo(&available, &total) == hipSuccess)
        gpu->cache_limit = total / 5;
    else
        gpu->cache_limit = (size_t)8 << 30;
    hipDeviceProp_t properties;
    if (hipGetDeviceProperties(&properties, 0) == hipSuccess)
        gpu->num_cus = properties.multiProcessorCount;
    if (gpu->num_cus <= 0) gpu->num_cus = 256;
    gpu->reference_kernels = hk_env_flag("H3_HIP_REFERENCE");
    gpu->profile_mark_wall = hk_now();
    if (!hk_loader_new(gpu)) {
        if (error && error_size) snprintf(error, error_size, "out of memory");
        (void)hipStreamDestroy(gpu->stream);
        free(gpu);
        return NULL;
    }
    return gpu;
}

extern "C" void h3_gpu_free(h3_gpu *gpu) {
    if (!gpu) return;
    (void)hipStreamSynchronize(gpu->stream);
    if (getenv("H3_PROFILE"))
        fprintf(stderr,
                "h3 hip%s%s: %llu tensors, peak %.3f GiB, %llu dispatches, "
                "%llu GEMM, %llu attention, wait %.3f s\n",
                gpu->profile_label[0] ? " " : "", gpu->profile_label,
                (unsigned long long)gpu->stats.tensor_allocations,
                (double)gpu->stats.peak_live_bytes / (1024.0 * 1024 * 1024),
                (unsigned long long)gpu->stats.direct_dispatches,
                (unsigned long long)gpu->stats.mps_linear_dispatches,
                (unsigned long long)gpu->stats.mps_sdpa_dispatches,
                gpu->stats.command_wait_seconds);
    hk_cache_evict(gpu, 0);
    if (gpu->workspace) (void)hipFree(gpu->workspace);
    if (gpu->splitk) (void)hipFree(gpu->splitk);
    if (gpu->sparse_ptr) (void)hipFree(gpu->sparse_ptr);
    if (gpu->sparse_idx) (void)hipFree(gpu->sparse_idx);
    hk_loader_free(gpu);
    if (gpu->timing) {
        for (auto &launch : gpu->timing->launches) {
            (void)hipEventDestroy(launch.start);
            (void)hipEventDestroy(launch.stop);
        }
        for (auto event : gpu->timing->pool) (void)hipEventDestroy(event);
        delete gpu->timing;
    }
    for (int slot = 0; slot < 16; slot++)
        if (gpu->marker_valid[slot]) (void)hipEventDestroy(gpu->markers[slot]);
    (void)hipStreamDestroy(gpu->stream);
    free(gpu);
}

/* Capability probes: no Apple NAX / int8 MLP; the device-resident Euler
 * sampler is preferred (reference h3_gpu_cuda.cu:334-352). */
extern "C" int h3_gpu_is_m5(const h3_gpu *gpu) { (void)gpu; return 0; }
extern "C" int h3_gpu_has_nax_mlp(const h3_gpu *gpu) { (void)gpu; return 0; }
extern "C" int h3_gpu_has_int8_mlp(const h3_gpu *gpu) { (void)gpu; return 0; }
extern "C" int h3_gpu_prefers_gpu_sampler(const h3_gpu *gpu) {
    return gpu ? 1 : 0;
}

/* Block-sparse joint attention (reference h3_gpu.h:44-52,
 * h3_cuda_attention.cu:1812-1857): validated like the reference (offsets
 * start at 0, end at idx_count, never decrease; every tile index inside the
 * dense 64-row tile count), then each query block's list is sorted so the
 * kernel can walk two neighbouring blocks' lists as one merged sequence. */
static void hk_sparse_clear(struct h3_gpu *gpu) {
    if (gpu->sparse_ptr) (void)hipFree(gpu->sparse_ptr);
    if (gpu->sparse_idx) (void)hipFree(gpu->sparse_idx);
    gpu->sparse_ptr = NULL;
    gpu->sparse_idx = NULL;
    gpu->sparse_rows = 0;
}

static int hk_u32_compare(const void *a, const void *b) {
    uint32_t x = *(const uint32_t *)a, y = *(const uint32_t *)b;
    return x < y ? -1 : x > y;
}

extern "C" int h3_gpu_sdpa_set_sparse(h3_gpu *gpu, const uint32_t *ptr,
                                      size_t ptr_count, const uint32_t *idx,
                                      size_t idx_count, uint32_t rows) {
    if (!gpu) return 0;
    if (gpu->active && hipStreamSynchronize(gpu->stream) != hipSuccess)
        return hk_fail(gpu, "cannot synchronise before replacing the mask");
    hk_sparse_clear(gpu);
    if (!ptr) return 1; /* cleared */
    if (!idx || !ptr_count || !idx_count || !rows)
        return hk_fail(gpu, "invalid block-sparse attention mask");
    const uint32_t ktiles = (rows + 63u) / 64u;
    if (ptr[0] != 0 || ptr[ptr_count - 1] != (uint32_t)idx_count)
        return hk_fail(gpu, "block-sparse mask offsets are inconsistent");
    for (size_t i = 1; i < ptr_count; i++)
        if (ptr[i] < ptr[i - 1])
            return hk_fail(gpu, "block-sparse mask offsets decrease");
    for (size_t i = 0; i < idx_count; i++)
        if (idx[i] >= ktiles)
            return hk_fail(gpu, "block-sparse mask tile %u outside %u tiles",
                           idx[i], ktiles);
    if (ptr_count - 1 < (rows + 127u) / 128u)
        return hk_fail(gpu, "block-sparse mask has %zu query blocks, %u "
                            "rows need %u", ptr_count - 1, rows,
                       (rows + 127u) / 128u);
    uint32_t *sorted = (uint32_t *)malloc(idx_count * sizeof(uint32_t));
    if (!sorted) return hk_fail(gpu, "out of memory");
    memcpy(sorted, idx, idx_count * sizeof(uint32_t));
    for (size_t q = 0; q + 1 < ptr_count; q++)
        qsort(sorted + ptr[q], ptr[q + 1] - ptr[q], sizeof(uint32_t),
              hk_u32_compare);
    gpu->device_mallocs += 2;
    int ok = hipMalloc((void **)&gpu->sparse_ptr,
                       ptr_count * sizeof(uint32_t)) == hipSuccess &&
             hipMalloc((void **)&gpu->sparse_idx,
                       idx_count * sizeof(uint32_t)) == hipSuccess &&
             hipMemcpy(gpu->sparse_ptr, ptr, ptr_count * sizeof(uint32_t),
                       hipMemcpyHostToDevice) == hipSuccess &&
             hipMemcpy(gpu->sparse_idx, sorted, idx_count * sizeof(uint32_t),
                       hipMemcpyHostToDevice) == hipSuccess;
    free(sorted);
    if (!ok) {
        hk_sparse_clear(gpu);
        return hk_fail(gpu, "cannot upload the block-sparse mask");
    }
    gpu->sparse_rows = rows;
    return 1;
}

/* -------------------------------------------------------------- tensors */

static h3_gpu_tensor *hk_tensor_new(struct h3_gpu *gpu, size_t elements,
                                    h3_gpu_dtype dtype) {
    if (!gpu) return NULL;
    size_t item = hk_item_size(dtype);
    if (elements > SIZE_MAX / item) {
        hk_fail(gpu, "tensor size overflow");
        return NULL;
    }
    h3_gpu_tensor *tensor = (h3_gpu_tensor *)calloc(1, sizeof(*tensor));
    if (!tensor) {
        hk_fail(gpu, "out of memory");
        return NULL;
    }
    tensor->elements = elements;
    tensor->bytes = elements * item;
    tensor->dtype = dtype;
    tensor->owner = gpu;
    tensor->data = hk_device_alloc(gpu, tensor->bytes);
    if (!tensor->data) {
        free(tensor);
        return NULL;
    }
    gpu->stats.allocated_bytes += tensor->bytes;
    gpu->stats.live_bytes += tensor->bytes;
    if (gpu->stats.live_bytes > gpu->stats.peak_live_bytes)
        gpu->stats.peak_live_bytes = gpu->stats.live_bytes;
    gpu->stats.tensor_allocations++;
    return tensor;
}

static int hk_upload(struct h3_gpu *gpu, void *device, const void *host,
                     size_t bytes) {
    if (!bytes) return 1;
    hipError_t status = hipMemcpyAsync(device, host, bytes,
                                       hipMemcpyHostToDevice, gpu->stream);
    if (status == hipSuccess) status = hipStreamSynchronize(gpu->stream);
    if (status != hipSuccess) return hk_fail_hip(gpu, "upload", status);
    gpu->stats.blit_copies++;
    return 1;
}

static int hk_download(struct h3_gpu *gpu, void *host, const void *device,
                       size_t bytes) {
    if (!bytes) return 1;
    hipError_t status = hipStreamSynchronize(gpu->stream);
    if (status == hipSuccess)
        status = hipMemcpyAsync(host, device, bytes, hipMemcpyDeviceToHost,
                                gpu->stream);
    if (status == hipSuccess) status = hipStreamSynchronize(gpu->stream);
    if (status != hipSuccess) return hk_fail_hip(gpu, "download", status);
    return 1;
}

static h3_gpu_tensor *hk_tensor_from(struct h3_gpu *gpu, const void *values,
                                     size_t elements, h3_gpu_dtype dtype) {
    h3_gpu_tensor *tensor = hk_tensor_new(gpu, elements, dtype);
    if (!tensor) return NULL;
    if (values && !hk_upload(gpu, tensor->data, values, tensor->bytes)) {
        h3_gpu_tensor_free(tensor);
        return NULL;
    }
    return tensor;
}

extern "C" h3_gpu_tensor *h3_gpu_tensor_new_f32(h3_gpu *gpu, size_t n) {
    return hk_tensor_new(gpu, n, H3_GPU_F32);
}
extern "C" h3_gpu_tensor *h3_gpu_tensor_new_bf16(h3_gpu *gpu, size_t n) {
    return hk_tensor_new(gpu, n, H3_GPU_BF16);
}
extern "C" h3_gpu_tensor *h3_gpu_tensor_new_i8(h3_gpu *gpu, size_t n) {
    return hk_tensor_new(gpu, n, H3_GPU_I8);
}
extern "C" h3_gpu_tensor *h3_gpu_tensor_from_f32(h3_gpu *gpu,
                                                 const float *values,
                                                 size_t n) {
    return hk_tensor_from(gpu, values, n, H3_GPU_F32);
}
extern "C" h3_gpu_tensor *h3_gpu_tensor_from_bf16(h3_gpu *gpu,
                                                  const uint16_t *values,
                                                  size_t n) {
    return hk_tensor_from(gpu, values, n, H3_GPU_BF16);
}
extern "C" h3_gpu_tensor *h3_gpu_tensor_from_u32(h3_gpu *gpu,
                                                 const uint32_t *values,
                                                 size_t n) {
    return hk_tensor_from(gpu, values, n, H3_GPU_U32);
}

/* ---- file payloads -> HBM (reference h3_gpu_cuda.cu:426-703) ------------
 * A pipelined loader instead of the reference's read-all-then-copy: the
 * 4 KiB-aligned superset of the byte range is cut into 8 MiB chunks;
 * up to HK_LOAD_THREADS readers (H3_HIP_LOAD_THREADS, default 16) each pread their chunks (O_DIRECT when the file
 * system allows it, else buffered) into their own two pinned staging slots,
 * and as each chunk lands its payload part is copied to the device on a
 * copy stream while the next chunk is being read.  The kernel cannot pin
 * pages of the driver's pinned mapping for a direct read (EFAULT), so
 * O_DIRECT reads land in a per-thread aligned bounce buffer and the payload
 * is copied on into the pinned slot; buffered reads go straight there.  Disk reads and PCIe
 * transfers overlap, and staging stays bounded at 2 x 16 x 8 MiB
 * whatever the tensor size.  A slot is reused only after the copy out of it
 * has completed (an event per slot). */
enum { HK_LOAD_THREADS = 16, HK_LOAD_SLOTS = 2 * HK_LOAD_THREADS };
static const size_t HK_LOAD_CHUNK = (size_t)8 << 20;
static const size_t HK_LOAD_ALIGN = 4096;

struct hk_loader {
    std::mutex lock;
    unsigned char *slots[HK_LOAD_SLOTS];
    hipEvent_t done[HK_LOAD_SLOTS];
    hipEvent_t after; /* compute-stream work queued before the load */
    unsigned char *bounce[HK_LOAD_THREADS]; /* aligned pageable, O_DIRECT */
    bool pending[HK_LOAD_SLOTS];
    hipStream_t copy;
    bool ready;
};

static bool hk_loader_new(struct h3_gpu *gpu) {
    gpu->loader = new (std::nothrow) hk_loader();
    return gpu->loader != NULL;
}

/* staging and the copy stream are made on the first load; caller holds the
 * loader lock */
static bool hk_loader_init(struct h3_gpu *gpu) {
    hk_loader *l = gpu->loader;
    if (l->ready) return true;
    /* each resource is made once: a failed set-up resumes where it stopped */
    bool ok = (l->copy || hipStreamCreateWithFlags(&l->copy,
                                                   hipStreamNonBlocking) ==
                              hipSuccess) &&
              (l->after || hipEventCreateWithFlags(&l->after,
                                                   hipEventDisableTiming) ==
                               hipSuccess);
    for (int i = 0; ok && i < HK_LOAD_SLOTS; i++) {
        /* hipHostMalloc memory is page aligned, as O_DIRECT needs */
        void *p = l->slots[i];
        ok = (p || hipHostMalloc(&p, HK_LOAD_CHUNK, hipHostMallocDefault) ==
                       hipSuccess) &&
             (l->done[i] || hipEventCreateWithFlags(&l->done[i],
                                                    hipEventDisableTiming) ==
                                hipSuccess);
        if (p) l->slots[i] = (unsigned char *)p;
        l->pending[i] = false;
    }
    if (!ok) (void)hipGetLastError();
    l->ready = ok;
    return ok;
}

static void hk_loader_free(struct h3_gpu *gpu) {
    hk_loader *l = gpu->loader;
    if (!l) return;
    if (l->copy) (void)hipStreamSynchronize(l->copy);
    for (int i = 0; i < HK_LOAD_SLOTS; i++) {
        if (l->slots[i]) (void)hipHostFree(l->slots[i]);
        if (l->done[i]) (void)hipEventDestroy(l->done[i]);
    }
    for (int t = 0; t < HK_LOAD_THREADS; t++) free(l->bounce[t]);
    if (l->after) (void)hipEventDestroy(l->after);
    if (l->copy) (void)hipStreamDestroy(l->copy);
    delete l;
    gpu->loader = NULL;
}

/* pread [offset, +bytes) fully, or until end of file once `need` bytes are
 * in: returns 0, an errno, or -1 for a file that ends early */
static int hk_pread_all(int fd, unsigned char *dst, uint64_t offset,
                        size_t bytes, size_t need) {
    size_t done = 0;
    while (done < bytes) {
        ssize_t got = pread(fd, dst + done, bytes - done,
                            (off_t)(offset + done));
        if (got < 0 && errno == EINTR) continue;
        if (got < 0) return errno;
        if (got == 0) return done >= need ? 0 : -1;
        done += (size_t)got;
    }
    return 0;
}

/* Copy file bytes [offset, +bytes) to device memory `dst`.  Must hold the
 * loader lock.  Returns 1, or 0 with the message in error. */
static int hk_load_range(struct h3_gpu *gpu, const char *path,
                         uint64_t offset, void *dst, size_t bytes,
                         bool try_direct, bool no_reuse, char *error,
                         size_t error_size) {
    hk_loader *l = gpu->loader;
    if (!bytes) return 1;
    int fd = try_direct ? open(path, O_RDONLY | O_CLOEXEC | O_DIRECT) : -1;
    bool direct = fd >= 0;
    if (!direct) fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
        snprintf(error, error_size, "cannot open %s: %s", path,
                 strerror(errno));
        return 0;
    }
    if (no_reuse && !direct)
        (void)posix_fadvise(fd, (off_t)offset, (off_t)bytes,
                            POSIX_FADV_NOREUSE);
    int max_threads = HK_LOAD_THREADS;
    if (const char *env = getenv("H3_HIP_LOAD_THREADS")) {
        int v = atoi(env);
        if (v >= 1 && v <= HK_LOAD_THREADS) max_threads = v;
    }
    const uint64_t end = offset + bytes;
    const uint64_t span0 = direct ? offset & ~(uint64_t)(HK_LOAD_ALIGN - 1)
                                  : offset;
    const uint64_t span1 = direct ? (end + HK_LOAD_ALIGN - 1) &
                                        ~(uint64_t)(HK_LOAD_ALIGN - 1)
                                  : end;
    const size_t chunks = (size_t)((span1 - span0 + HK_LOAD_CHUNK - 1) /
                                   HK_LOAD_CHUNK);
    std::vector<int> status(HK_LOAD_THREADS, 0);
    std::vector<std::thread> readers;
    const int threads = chunks < (size_t)max_threads ? (int)chunks
                                                     : max_threads;
    auto reader = [&](int t) {
        for (size_t c = (size_t)t; c < chunks; c += (size_t)threads) {
            /* thread t owns slots t and t + HK_LOAD_THREADS */
            const int slot = t + (int)((c / (size_t)threads) & 1) *
                                     HK_LOAD_THREADS;
            if (l->pending[slot]) {
                if (hipEventSynchronize(l->done[slot]) != hipSuccess) {
                    status[t] = EIO;
                    return;
                }
                l->pending[slot] = false;
            }
            const uint64_t c0 = span0 + (uint64_t)c * HK_LOAD_CHUNK;
            const uint64_t c1 = c0 + HK_LOAD_CHUNK < span1
                ? c0 + HK_LOAD_CHUNK : span1;
            const uint64_t p0 = c0 > offset ? c0 : offset;
            const uint64_t p1 = c1 < end ? c1 : end;
            unsigned char *land = l->slots[slot];
            if (direct) {
                if (!l->bounce[t]) {
                    void *p = NULL;
                    if (posix_memalign(&p, HK_LOAD_ALIGN, HK_LOAD_CHUNK)) {
                        status[t] = ENOMEM;
                        return;
                    }
                    l->bounce[t] = (unsigned char *)p;
                }
                land = l->bounce[t];
            }
            int rc = hk_pread_all(fd, land, c0, (size_t)(c1 - c0),
                                  (size_t)(p1 - c0));
            if (rc) {
                status[t] = rc;
                return;
            }
            if (direct)
                memcpy(l->slots[slot] + (p0 - c0), land + (p0 - c0),
                       (size_t)(p1 - p0));
            if (hipMemcpyAsync((unsigned char *)dst + (p0 - offset),
                               l->slots[slot] + (p0 - c0), (size_t)(p1 - p0),
                               hipMemcpyHostToDevice, l->copy) != hipSuccess ||
                hipEventRecord(l->done[slot], l->copy) != hipSuccess) {
                status[t] = EIO;
                return;
            }
            l->pending[slot] = true;
        }
    };
    for (int t = 1; t < threads; t++) {
        try {
            readers.emplace_back(reader, t);
        } catch (...) {
            status[t] = -2; /* could not start: read inline below */
        }
    }
    reader(0);
    for (int t = 1; t < threads; t++)
        if (status[t] == -2) {
            status[t] = 0;
            reader(t);
        }
    for (auto &r : readers) r.join();
    close(fd);
    hipError_t sync = hipStreamSynchronize(l->copy);
    for (int i = 0; i < HK_LOAD_SLOTS; i++) l->pending[i] = false;
    for (int t = 0; t < threads; t++) {
        if (!status[t]) continue;
        if (status[t] == EINVAL && direct) {
            /* the file system refused O_DIRECT reads: buffered retry */
            return hk_load_range(gpu, path, offset, dst, bytes, false,
                                 no_reuse, error, error_size);
        }
        snprintf(error, error_size, "cannot read %s: %s", path,
                 status[t] > 0 ? strerror(status[t])
                               : "unexpected end of file");
        return 0;
    }
    if (sync != hipSuccess) {
        snprintf(error, error_size, "file upload failed: %s",
                 hipGetErrorString(sync));
        return 0;
    }
    return 1;
}

/* direct: O_DIRECT first (whole-tensor loads, as the reference does);
 * otherwise buffered reads, with no_reuse asking the page cache not to keep
 * the payload (the reference's stream variant). */
static int hk_load_into(struct h3_gpu *gpu, const char *path, uint64_t offset,
                        void *dst, size_t bytes, bool direct, bool no_reuse,
                        char *error, size_t error_size) {
    if (!path || !*path || offset > (uint64_t)INT64_MAX ||
        (uint64_t)bytes > (uint64_t)INT64_MAX - offset) {
        snprintf(error, error_size, "invalid file range");
        return 0;
    }
    std::lock_guard<std::mutex> guard(gpu->loader->lock);
    if (!hk_loader_init(gpu)) {
        snprintf(error, error_size, "cannot set up pinned staging");
        return 0;
    }
    /* destination memory may be a recycled buffer that work already queued
     * on the compute stream still touches: order the copies after it */
    if (hipEventRecord(gpu->loader->after, gpu->stream) != hipSuccess ||
        hipStreamWaitEvent(gpu->loader->copy, gpu->loader->after, 0) !=
            hipSuccess) {
        snprintf(error, error_size, "device error before file load");
        return 0;
    }
    /* H3_HIP_DIRECT_IO=0 forces buffered reads */
    const char *env = getenv("H3_HIP_DIRECT_IO");
    if (env && strcmp(env, "0") == 0) direct = false;
    return hk_load_range(gpu, path, offset, dst, bytes, direct, no_reuse,
                         error, error_size);
}

static h3_gpu_tensor *hk_tensor_load(struct h3_gpu *gpu, const char *path,
                                     uint64_t offset, size_t elements,
                                     h3_gpu_dtype dtype) {
    if (!gpu || !path) return NULL;
    h3_gpu_tensor *tensor = hk_tensor_new(gpu, elements, dtype);
    if (!tensor) return NULL;
    if (!hk_load_into(gpu, path, offset, tensor->data,
                      elements * hk_item_size(dtype), true, false,
                      gpu->error, sizeof(gpu->error))) {
        h3_gpu_tensor_free(tensor);
        return NULL;
    }
    return tensor;
}

extern "C" h3_gpu_tensor *h3_gpu_tensor_load_bf16(h3_gpu *gpu,
                                                  const char *path,
                                                  uint64_t offset,
                                                  size_t n) {
    return hk_tensor_load(gpu, path, offset, n, H3_GPU_BF16);
}
extern "C" h3_gpu_tensor *h3_gpu_tensor_load_f32(h3_gpu *gpu,
                                                 const char *path,
                                                 uint64_t offset, size_t n) {
    return hk_tensor_load(gpu, path, offset, n, H3_GPU_F32);
}

/* May run on an I/O thread while the calling thread keeps issuing work
 * (reference h3_gpu.h:67-78): the loader lock serialises loads, and the
 * copy stream never touches the context's compute stream. */
static int hk_read_file(h3_gpu_tensor *tensor, const char *path,
                        uint64_t offset, size_t elements, bool no_reuse,
                        char *error, size_t error_size) {
    char local[256];
    if (!error || !error_size) {
        error = local;
        error_size = sizeof(local);
    }
    error[0] = '\0';
    if (!tensor || !tensor->owner || tensor->dtype != H3_GPU_BF16 ||
        elements != tensor->elements) {
        snprintf(error, error_size, "invalid BF16 file read request");
        return 0;
    }
    return hk_load_into(tensor->owner, path, offset, tensor->data,
                        elements * 2, false, no_reuse, error, error_size);
}

extern "C" int h3_gpu_tensor_read_file_bf16(h3_gpu_tensor *tensor,
                                            const char *path,
                                            uint64_t offset, size_t elements,
                                            char *error, size_t error_size) {
    return hk_read_file(tensor, path, offset, elements, false, error,
                        error_size);
}

extern "C" int h3_gpu_tensor_stream_file_bf16(h3_gpu_tensor *tensor,
                                              const char *path,
                                              uint64_t offset,
                                              size_t elements, char *error,
                                              size_t error_size) {
    return hk_read_file(tensor, path, offset, elements, true, error,
                        error_size);
}

extern "C" void h3_gpu_tensor_free(h3_gpu_tensor *tensor) {
    if (!tensor) return;
    struct h3_gpu *gpu = tensor->owner;
    if (gpu && tensor->data) {
        hk_device_release(gpu, tensor->data, tensor->bytes);
        gpu->stats.live_bytes -= tensor->bytes;
    }
    free(tensor);
}

extern "C" size_t h3_gpu_tensor_elements(const h3_gpu_tensor *tensor) {
    return tensor ? tensor->elements : 0;
}

extern "C" h3_gpu_dtype h3_gpu_tensor_dtype(const h3_gpu_tensor *tensor) {
    return tensor ? tensor->dtype : H3_GPU_F32;
}

extern "C" int h3_gpu_tensor_read_f32_range(const h3_gpu_tensor *tensor,
                                            size_t offset, float *values,
                                            size_t n) {
    if (!tensor || !values || tensor->dtype != H3_GPU_F32 ||
        offset > tensor->elements || n > tensor->elements - offset)
        return 0;
    return hk_download(tensor->owner, values,
                       (const float *)tensor->data + offset, n * 4);
}

extern "C" int h3_gpu_tensor_read_f32(const h3_gpu_tensor *tensor,
                                      float *values, size_t n) {
    return h3_gpu_tensor_read_f32_range(tensor, 0, values, n);
}

extern "C" int h3_gpu_tensor_read_bf16(const h3_gpu_tensor *tensor,
                                       uint16_t *values, size_t n) {
    if (!tensor || !values || tensor->dtype != H3_GPU_BF16 ||
        n > tensor->elements)
        return 0;
    return hk_download(tensor->owner, values, tensor->data, n * 2);
}

extern "C" int h3_gpu_tensor_write_f32_range(h3_gpu_tensor *tensor,
                                             size_t offset,
                                             const float *values, size_t n) {
    if (!tensor || !values || tensor->dtype != H3_GPU_F32 ||
        offset > tensor->elements || n > tensor->elements - offset)
        return 0;
    return hk_upload(tensor->owner, (float *)tensor->data + offset, values,
                     n * 4);
}

extern "C" int h3_gpu_tensor_write_f32(h3_gpu_tensor *tensor,
                                       const float *values, size_t n) {
    return h3_gpu_tensor_write_f32_range(tensor, 0, values, n);
}

extern "C" int h3_gpu_tensor_write_bf16_range(h3_gpu_tensor *tensor,
                                              size_t offset,
                                              const uint16_t *values,
                                              size_t n) {
    if (!tensor || !values || tensor->dtype != H3_GPU_BF16 ||
        offset > tensor->elements || n > tensor->elements - offset)
        return 0;
    return hk_upload(tensor->owner, (uint16_t *)tensor->data + offset, values,
                     n * 2);
}

extern "C" int h3_gpu_tensor_write_bf16(h3_gpu_tensor *tensor,
                                        const uint16_t *values, size_t n) {
    return h3_gpu_tensor_write_bf16_range(tensor, 0, values, n);
}

/* -------------------------------------------------------------- batches */

extern "C" int h3_gpu_begin(h3_gpu *gpu) {
    if (!gpu || gpu->active) return 0;
    gpu->error[0] = '\0';
    gpu->active = 1;
    gpu->batch_start = hk_now();
    return 1;
}

extern "C" int h3_gpu_continue(h3_gpu *gpu) {
    if (!gpu || !gpu->active) return 0;
    double now = hk_now();
    gpu->stats.submissions++;
    gpu->stats.command_encode_seconds += now - gpu->batch_start;
    gpu->batch_start = now;
    return 1;
}

extern "C" int h3_gpu_submit(h3_gpu *gpu) {
    if (!gpu || !gpu->active) return 0;
    gpu->active = 0;
    double committed = hk_now();
    hipError_t status = hipStreamSynchronize(gpu->stream);
    double completed = hk_now();
    gpu->stats.submissions++;
    gpu->stats.command_encode_seconds += committed - gpu->batch_start;
    gpu->stats.command_wait_seconds += completed - committed;
    gpu->stats.gpu_seconds += completed - committed;
    if (status != hipSuccess)
        return hk_fail_hip(gpu, "command execution", status);
    return 1;
}

extern "C" const char *h3_gpu_error(const h3_gpu *gpu) {
    if (!gpu || !gpu->error[0]) return "unknown HIP error";
    return gpu->error;
}

extern "C" int h3_gpu_get_stats(const h3_gpu *gpu, h3_gpu_stats *stats) {
    if (!gpu || !stats) return 0;
    *stats = gpu->stats;
    return 1;
}

extern "C" void h3_gpu_profile_set_label(h3_gpu *gpu, const char *label) {
    if (!gpu || !label || !*label) return;
    snprintf(gpu->profile_label, sizeof(gpu->profile_label), "%s", label);
}

extern "C" void h3_gpu_profile_mark(h3_gpu *gpu, const char *phase) {
    if (!gpu || !phase || !*phase || !hk_env_flag("H3_PROFILE")) return;
    (void)hipStreamSynchronize(gpu->stream);
    double now = hk_now();
    fprintf(stderr, "h3 hip %s%s%s: %.3f s wall, %llu dispatches, "
            "%.3f GiB live\n",
            gpu->profile_label, gpu->profile_label[0] ? " " : "", phase,
            now - gpu->profile_mark_wall,
            (unsigned long long)(gpu->stats.direct_dispatches +
                                 gpu->stats.mps_linear_dispatches +
                                 gpu->stats.mps_sdpa_dispatches -
                                 gpu->profile_mark_stats.direct_dispatches -
                                 gpu->profile_mark_stats.mps_linear_dispatches -
                                 gpu->profile_mark_stats.mps_sdpa_dispatches),
            (double)gpu->stats.live_bytes / (1024.0 * 1024 * 1024));
    gpu->profile_mark_stats = gpu->stats;
    gpu->profile_mark_wall = now;
}
