// hip_context.hip -- device context C-ABI: one process-global stream, memory helpers and stream-capture graphs.
//
// Mirrors the reference's device-context boundary (src/backend/cuda/cuda_context.cu:13-126 and
// src/backend/cuda/memory/memory.zig:1-11): every launcher enqueues on one non-blocking stream, launchers never
// synchronise, graphs are recorded on that stream in thread-local capture mode.  hip_set_stream and the
// hip_timer_* helpers have no reference counterpart: the first lets a host that owns its own stream (PyTorch's
// current stream, for example) route the kernels onto it, the second times work on that same stream.
#include "hip_common.h"

#include <stdlib.h>
#include <string.h>

#include <atomic>

hipStream_t g_llmgen_stream = nullptr;
static bool g_own_stream = false;
static hipStream_t g_side_stream = nullptr;
static hipEvent_t g_fork_event = nullptr, g_join_event = nullptr;
static hipGraph_t g_capture_graph = nullptr;
static std::atomic<int> g_own_error{0};

void llmgen_record_error(hipError_t e) {
    int zero = 0;
    g_own_error.compare_exchange_strong(zero, (int)e);
}

#define HIP_WARN(call)                                                                                   \
    do {                                                                                                 \
        hipError_t e_ = (call);                                                                          \
        if (e_ != hipSuccess) fprintf(stderr, "[llmgen-hip] %s failed: %s\n", #call, hipGetErrorString(e_)); \
    } while (0)

// Fork work onto the library's side stream after everything enqueued so far on the launch stream, and join it
// back.  Both are event based, so they are legal inside stream capture (the side stream joins the capture).
// Returns the side stream, or the launch stream itself if the side stream could not be created.
hipStream_t llmgen_fork_side_stream() {
    if (!g_side_stream) {
        if (hipStreamCreateWithFlags(&g_side_stream, hipStreamNonBlocking) != hipSuccess ||
            hipEventCreateWithFlags(&g_fork_event, hipEventDisableTiming) != hipSuccess ||
            hipEventCreateWithFlags(&g_join_event, hipEventDisableTiming) != hipSuccess) {
            g_side_stream = nullptr;
            return g_llmgen_stream;
        }
    }
    if (hipEventRecord(g_fork_event, g_llmgen_stream) != hipSuccess ||
        hipStreamWaitEvent(g_side_stream, g_fork_event, 0) != hipSuccess)
        return g_llmgen_stream;
    return g_side_stream;
}

void llmgen_join_side_stream(hipStream_t side) {
    if (side == g_llmgen_stream) return;
    HIP_WARN(hipEventRecord(g_join_event, side));
    HIP_WARN(hipStreamWaitEvent(g_llmgen_stream, g_join_event, 0));
}

// Run-time options of the launchers (hip_attn_set_option).  Defaults come from the environment on first use:
// SV_ATTN_PART (the reference's switch, attention.cu:219-229: the split-K part length is raised to at least this
// many tokens), LLMGEN_DECODE_ROW_WAVES (4 or 8 waves per workgroup for the decode rows of a prefill step) and
// LLMGEN_DECODE_MERGE (1: merge split-K partials in the separate merge kernel instead of in the decode kernel) and
// LLMGEN_PREFILL_SPLIT_TILES (heavy tiles of a pure prefill step split over two workgroups; -1 = automatic).
static int g_opts[LLMGEN_OPT_COUNT];
static bool g_opts_loaded = false;

static void load_opts() {
    if (g_opts_loaded) return;
    auto env = [](const char *name, int dflt) {
        const char *v = getenv(name);
        return v && *v ? atoi(v) : dflt;
    };
    g_opts[LLMGEN_OPT_ATTN_PART_MIN] = env("SV_ATTN_PART", 0);
    if (g_opts[LLMGEN_OPT_ATTN_PART_MIN] > 0)
        fprintf(stderr, "[llmgen-hip] SV_ATTN_PART=%d: split-K parts of at least that many tokens\n",
                g_opts[LLMGEN_OPT_ATTN_PART_MIN]);
    g_opts[LLMGEN_OPT_DECODE_ROW_WAVES] = env("LLMGEN_DECODE_ROW_WAVES", 4);
    g_opts[LLMGEN_OPT_DECODE_MERGE_KERNEL] = env("LLMGEN_DECODE_MERGE", 0);
    g_opts[LLMGEN_OPT_PREFILL_SPLIT_TILES] = env("LLMGEN_PREFILL_SPLIT_TILES", -1);
    g_opts_loaded = true;
}

int llmgen_opt(int which) {
    load_opts();
    return which >= 0 && which < LLMGEN_OPT_COUNT ? g_opts[which] : 0;
}

int llmgen_num_cus() {
    static int n = 0;
    if (n == 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
    }
    return n;
}

extern "C" {

int hip_attn_set_option(int option, int value) {
    load_opts();
    if (option < 0 || option >= LLMGEN_OPT_COUNT) {
        fprintf(stderr, "[llmgen-hip] hip_attn_set_option: unknown option %d\n", option);
        return -1;
    }
    if (option == LLMGEN_OPT_DECODE_ROW_WAVES && value != 4 && value != 8) {
        fprintf(stderr, "[llmgen-hip] hip_attn_set_option: decode-row waves must be 4 or 8 (got %d)\n", value);
        return -1;
    }
    if (value < 0 && !(option == LLMGEN_OPT_PREFILL_SPLIT_TILES && value == -1)) {
        fprintf(stderr, "[llmgen-hip] hip_attn_set_option: negative value %d\n", value);
        return -1;
    }
    const int prev = g_opts[option];
    g_opts[option] = value;
    return prev;
}

// cuda_context.cu:13-42.  Creates the global stream on device 0.  ws_bytes is accepted for signature parity
// (the reference sizes a cuBLAS workspace with it); the attention path needs no library workspace.
int hip_init(size_t ws_bytes) {
    (void)ws_bytes;
    if (g_llmgen_stream) return 0;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
        fprintf(stderr, "[llmgen-hip] no HIP device\n");
        return 1;
    }
    if (hipSetDevice(0) != hipSuccess) return 1;
    if (hipStreamCreateWithFlags(&g_llmgen_stream, hipStreamNonBlocking) != hipSuccess) {
        fprintf(stderr, "[llmgen-hip] hipStreamCreateWithFlags failed\n");
        g_llmgen_stream = nullptr;
        return 2;
    }
    g_own_stream = true;
    return 0;
}

// Route all launches onto a stream owned by the caller (nullptr = the legacy default stream).
void hip_set_stream(void *stream) {
    if (g_own_stream && g_llmgen_stream) (void)hipStreamDestroy(g_llmgen_stream);
    g_own_stream = false;
    g_llmgen_stream = (hipStream_t)stream;
}

void *hip_get_stream(void) { return (void *)g_llmgen_stream; }

int hip_device_count(void) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess) return 0;
    return count;
}

// cuda_context.cu:50-64; `arch` receives the gcnArch number (e.g. 950) in place of the CUDA SM version.
void hip_device_info(int dev, char *name, int name_cap, size_t *total_mem, int *arch) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) {
        if (name && name_cap > 0) name[0] = '\0';
        if (total_mem) *total_mem = 0;
        if (arch) *arch = 0;
        return;
    }
    if (name && name_cap > 0) {
        strncpy(name, prop.gcnArchName, name_cap - 1);
        name[name_cap - 1] = '\0';
    }
    if (total_mem) *total_mem = prop.totalGlobalMem;
    if (arch) *arch = prop.major * 100 + prop.minor * 10;
}

void hip_mem_info(size_t *free_mem, size_t *total_mem) {
    size_t f = 0, t = 0;
    if (hipMemGetInfo(&f, &t) != hipSuccess) f = t = 0;
    if (free_mem) *free_mem = f;
    if (total_mem) *total_mem = t;
}

// memory.zig:1-11
void *hip_malloc(size_t bytes) {
    void *p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) {
        fprintf(stderr, "[llmgen-hip] hipMalloc(%zu) failed\n", bytes);
        return nullptr;
    }
    return p;
}
void hip_free(void *p) {
    if (p) HIP_WARN(hipFree(p));
}
void *hip_host_alloc(size_t bytes) {
    void *p = nullptr;
    if (hipHostMalloc(&p, bytes, hipHostMallocDefault) != hipSuccess) return nullptr;
    return p;
}
void hip_host_free(void *p) {
    if (p) HIP_WARN(hipHostFree(p));
}
void hip_h2d(void *dst, const void *src, size_t n) { HIP_WARN(hipMemcpy(dst, src, n, hipMemcpyHostToDevice)); }
void hip_d2h(void *dst, const void *src, size_t n) {
    HIP_WARN(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, g_llmgen_stream));
    HIP_WARN(hipStreamSynchronize(g_llmgen_stream));
}
void hip_d2d(void *dst, const void *src, size_t n) { HIP_WARN(hipMemcpy(dst, src, n, hipMemcpyDeviceToDevice)); }
void hip_h2d_async(void *dst, const void *src, size_t n) {
    HIP_WARN(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, g_llmgen_stream));
}
void hip_d2h_async(void *dst, const void *src, size_t n) {
    HIP_WARN(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, g_llmgen_stream));
}

// cuda_context.cu:96-102.  Launches are asynchronous: errors show up after a sync.  An error the library recorded
// itself (a launch it rejected on the host, llmgen_record_error) is returned first, and cleared by the read;
// otherwise the runtime's last error.
int hip_last_error(void) {
    const int own = g_own_error.exchange(0);
    const int rt = (int)hipGetLastError();
    return own ? own : rt;
}
void hip_sync(void) { HIP_WARN(hipStreamSynchronize(g_llmgen_stream)); }

// cuda_context.cu:106-126.  Graph capture on the global stream.
int hip_graph_begin(void) { return (int)hipStreamBeginCapture(g_llmgen_stream, hipStreamCaptureModeThreadLocal); }
void *hip_graph_end(void) {
    if (hipStreamEndCapture(g_llmgen_stream, &g_capture_graph) != hipSuccess || !g_capture_graph) {
        fprintf(stderr, "[llmgen-hip] hipStreamEndCapture failed\n");
        g_capture_graph = nullptr;
        return nullptr;
    }
    hipGraphExec_t exec = nullptr;
    if (hipGraphInstantiate(&exec, g_capture_graph, nullptr, nullptr, 0) != hipSuccess) exec = nullptr;
    (void)hipGraphDestroy(g_capture_graph);
    g_capture_graph = nullptr;
    return (void *)exec;
}
void hip_graph_launch(void *exec) { HIP_WARN(hipGraphLaunch((hipGraphExec_t)exec, g_llmgen_stream)); }
void hip_graph_destroy(void *exec) {
    if (exec) (void)hipGraphExecDestroy((hipGraphExec_t)exec);
}

// ---- timing on the launch stream (measurement helpers; no reference counterpart) ----
void *hip_timer_create(void) {
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return (void *)e;
}
void hip_timer_record(void *ev) { HIP_WARN(hipEventRecord((hipEvent_t)ev, g_llmgen_stream)); }
float hip_timer_elapsed_ms(void *start, void *stop) {
    float ms = -1.f;
    HIP_WARN(hipEventSynchronize((hipEvent_t)stop));
    HIP_WARN(hipEventElapsedTime(&ms, (hipEvent_t)start, (hipEvent_t)stop));
    return ms;
}
void hip_timer_destroy(void *ev) {
    if (ev) (void)hipEventDestroy((hipEvent_t)ev);
}

}  // extern "C"
