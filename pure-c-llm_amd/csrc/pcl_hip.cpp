// pcl_hip.cpp -- the C ABI of libpcl_hip (include/pcl_hip.h): argument
// checks, error reporting, streams, scratch workspaces, kernel dispatch and
// the reference-signature drop-ins.
//
// Error convention: native pcl_* calls return a status (PCL_OK == 0) and
// record a message; void drop-ins record the same and, when
// pcl_set_abort_on_error(1) is in force, print it and exit(1) as the
// reference's CUDA_CHECK does (gpu_kernels.h:34-36). Nothing ever falls back
// to a CPU path: without a usable gfx950 device every call fails loudly.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <algorithm>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "../../include/pcl_hip.h"
#include "internal.h"

namespace {

// Byte ranges [a, a+na) and [b, b+nb) share memory.
bool ranges_overlap(const void *a, size_t na, const void *b, size_t nb) {
    const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
    return x < y + nb && y < x + na;
}


// ----------------------------------------------------------- error state ----
thread_local int t_status = PCL_OK;
thread_local char t_msg[512] = "";
thread_local hipStream_t t_stream = nullptr;
int g_abort_on_error = 0;
int g_d_model = 0, g_vocab = 0;
int g_attn_batch = 0, g_attn_seq = 0, g_attn_heads = 0;

int set_error(int status, const char *fmt, ...) {
    t_status = status;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(t_msg, sizeof t_msg, fmt, ap);
    va_end(ap);
    return status;
}

// Every void drop-in ends here: its own outcome becomes pcl_last_status(),
// so a success clears an earlier failure (the caller's only way to check).
void finish_void(int status) {
    if (status == PCL_OK) {
        t_status = PCL_OK;
        t_msg[0] = 0;
    } else if (g_abort_on_error) {
        fprintf(stderr, "libpcl_hip error %d: %s\n", status, t_msg);
        exit(1);
    }
}

#define HIP_OK(call)                                                                       \
    do {                                                                                   \
        hipError_t e_ = (call);                                                            \
        if (e_ != hipSuccess)                                                              \
            return set_error(PCL_ERR_HIP, "%s failed: %s", #call, hipGetErrorString(e_));  \
    } while (0)

#define CHECK_ARG(cond, ...)                                       \
    do {                                                           \
        if (!(cond)) return set_error(PCL_ERR_INVALID_ARG, __VA_ARGS__); \
    } while (0)

#define PCL_OK_OR_RETURN(expr)      \
    do {                            \
        int s_ = (expr);            \
        if (s_ != PCL_OK) return s_; \
    } while (0)

// -------------------------------------------------------------- device ----
std::mutex g_mu;
bool g_inited = false;
int g_init_status = PCL_OK;
char g_init_msg[256] = "";

void resolve_noalloc_at_init(int dev);

int do_init() {
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_inited) {
        if (g_init_status != PCL_OK) return set_error(g_init_status, "%s", g_init_msg);
        return PCL_OK;
    }
    g_inited = true;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) {
        g_init_status = PCL_ERR_NO_DEVICE;
        snprintf(g_init_msg, sizeof g_init_msg, "no HIP device (%s)",
                 e != hipSuccess ? hipGetErrorString(e) : "count 0");
        return set_error(g_init_status, "%s", g_init_msg);
    }
    int dev = 0;
    (void)hipGetDevice(&dev);
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) {
        g_init_status = PCL_ERR_HIP;
        snprintf(g_init_msg, sizeof g_init_msg, "hipGetDeviceProperties: %s", hipGetErrorString(e));
        return set_error(g_init_status, "%s", g_init_msg);
    }
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        g_init_status = PCL_ERR_NO_DEVICE;
        snprintf(g_init_msg, sizeof g_init_msg,
                 "libpcl_hip is built for gfx950 only; device 0 is %s", prop.gcnArchName);
        return set_error(g_init_status, "%s", g_init_msg);
    }
    resolve_noalloc_at_init(dev);
    return PCL_OK;
}

// ----------------------------------------------------------- workspaces ----
// One scratch set per stream: work on one stream is ordered on the GPU, so
// calls that share a stream may share its scratch. A call holds the stream's
// call lock from taking the scratch until its last launch is enqueued
// (ScratchLease), so a call from another host thread on the same stream (the
// null stream is every thread's default) cannot grow, and so free, a buffer
// the first call has taken but not yet handed to a kernel.
struct StreamScratch {
    std::recursive_mutex call_mu;  // recursive: a call may nest another on the stream
    pcl::Workspace ws;
    void *aux = nullptr;  // padded INT8 activations; head_ce's logits chunk and row losses
    size_t aux_cap = 0;
    // Realigned copies of misaligned FP32 GEMM operands (sgemm_realigned).
    // Kept apart from aux: pcl_head_ce holds its logits chunk in aux while it
    // calls pcl_sgemm, which may realign on the same stream.
    void *realign = nullptr;
    size_t realign_cap = 0;
    unsigned *amax = nullptr;  // per-tensor amax bits
    int *tiles = nullptr;      // the INT8 GEMM's per-XCD tile counters (zero between calls)
    // Set once a graph has been captured on the stream: buffers a graph may
    // reference are never freed before the stream is destroyed.
    bool pinned = false;
    std::vector<void *> retired;
};
std::unordered_map<hipStream_t, StreamScratch> g_scratch;

struct ScratchLease {
    StreamScratch *p = nullptr;
    std::unique_lock<std::recursive_mutex> lk;
    StreamScratch *operator->() const { return p; }
};

int grow(void **p, size_t *cap, size_t need, hipStream_t s, StreamScratch &sc) {
    if (need <= *cap) return PCL_OK;
    size_t sz = need + need / 4 + 4096;
    if (*p) {
        if (sc.pinned) {
            sc.retired.push_back(*p);  // a captured graph may still use it
        } else {
            HIP_OK(hipStreamSynchronize(s));
            HIP_OK(hipFree(*p));
        }
        *p = nullptr;
        *cap = 0;
    }
    if (hipMalloc(p, sz) != hipSuccess) {
        *p = nullptr;
        return set_error(PCL_ERR_OOM, "workspace allocation of %zu bytes failed", sz);
    }
    *cap = sz;
    return PCL_OK;
}

int get_scratch(hipStream_t s, size_t part_bytes, size_t aux_bytes, ScratchLease *out,
                size_t realign_bytes = 0) {
    StreamScratch *entry;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        entry = &g_scratch[s];  // map nodes keep their address
    }
    if (!out->lk.owns_lock()) out->lk = std::unique_lock<std::recursive_mutex>(entry->call_mu);
    std::lock_guard<std::mutex> lk(g_mu);
    StreamScratch &sc = *entry;
    PCL_OK_OR_RETURN(grow(&sc.ws.buf, &sc.ws.bytes_cap, part_bytes, s, sc));
    PCL_OK_OR_RETURN(grow(&sc.aux, &sc.aux_cap, aux_bytes, s, sc));
    PCL_OK_OR_RETURN(grow(&sc.realign, &sc.realign_cap, realign_bytes, s, sc));
    if (!sc.amax) {
        if (hipMalloc((void **)&sc.amax, 256) != hipSuccess)
            return set_error(PCL_ERR_OOM, "amax scratch allocation failed");
    }
    if (!sc.tiles) {
        if (hipMalloc((void **)&sc.tiles, 256) != hipSuccess)
            return set_error(PCL_ERR_OOM, "tile counter allocation failed");
        // zeroed by a kernel on the stream (also inside a capture, where a
        // replay re-zeroes counters that are zero anyway)
        HIP_OK(pcl::launch_igemm_tiles_init(sc.tiles, s));
    }
    out->p = &sc;
    return PCL_OK;
}

// Device address of the static GEMV scratch (gemv.hip), per device, resolved
// once with that device current: by the library's init for its device, else
// by the first pcl_sgemv_noalloc call on another device.
constexpr int NOALLOC_MAX_DEVICES = 64;
void *g_noalloc_ptr[NOALLOC_MAX_DEVICES] = {};
std::mutex g_noalloc_mu;

int noalloc_scratch(int dev, void **out) {
    if (dev < 0 || dev >= NOALLOC_MAX_DEVICES)
        return set_error(PCL_ERR_RANGE, "device %d beyond the static scratch table", dev);
    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    if (!g_noalloc_ptr[dev]) {
        void *p = nullptr;
        const hipError_t e = pcl::gemv_noalloc_scratch(&p);
        if (e != hipSuccess || !p)
            return set_error(PCL_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
        g_noalloc_ptr[dev] = p;
    }
    *out = g_noalloc_ptr[dev];
    return PCL_OK;
}

void resolve_noalloc_at_init(int dev) {
    if (dev < 0 || dev >= NOALLOC_MAX_DEVICES) return;
    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    void *p = nullptr;
    if (pcl::gemv_noalloc_scratch(&p) == hipSuccess && p) g_noalloc_ptr[dev] = p;
    else (void)hipGetLastError();  // not fatal here: the entry point retries and reports it
}

hipStream_t pick(void *stream) { return stream ? (hipStream_t)stream : t_stream; }

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Packed INT8 weight rows: K rounded up to 256 bytes (a multiple of every K
// tile the INT8 GEMM uses), zero padded, so every K-tile read of a weight row
// stays inside that row.
int kpad256(int K) { return ((K + 255) / 256) * 256; }

// ------------------------------------------------------- host staging ----
// Device copies of host operands for the host-pointer drop-ins; one growing
// buffer per slot per thread, freed when the thread exits (its last calls
// ended with a synchronisation, so no kernel still reads them).
struct HostStage {
    void *p[8] = {nullptr};
    size_t cap[8] = {0};
    ~HostStage() {
        for (void *q : p)
            if (q) (void)hipFree(q);
    }
};
thread_local HostStage t_stage;

// This thread's stream is being captured: by pcl_graph_begin, or by the
// caller's own hipStreamBeginCapture on the stream it handed to pcl_set_stream.
thread_local bool t_capturing = false;

// Host-pointer drop-ins copy operands through the staging slots and wait for
// the stream: neither can be recorded into a graph (the copies would read the
// host buffers at replay time, the wait would end the capture). They refuse
// while the stream captures; every one of them stages through here first.
int refuse_capture() {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (!t_capturing && t_stream != nullptr && hipStreamIsCapturing(t_stream, &cs) != hipSuccess) {
        (void)hipGetLastError();
        cs = hipStreamCaptureStatusNone;
    }
    if (t_capturing || cs != hipStreamCaptureStatusNone)
        return set_error(PCL_ERR_INVALID_ARG,
                         "host-pointer drop-ins cannot run while this thread's stream is being captured "
                         "(they copy host operands and wait for the stream); call them outside "
                         "pcl_graph_begin/pcl_graph_end, or capture the device-pointer entry points");
    return PCL_OK;
}

int stage_buf(int slot, size_t bytes, void **out) {
    PCL_OK_OR_RETURN(refuse_capture());
    if (bytes == 0) bytes = 16;
    if (bytes > t_stage.cap[slot]) {
        if (t_stage.p[slot]) {
            HIP_OK(hipStreamSynchronize(t_stream));
            HIP_OK(hipFree(t_stage.p[slot]));
            t_stage.p[slot] = nullptr;
            t_stage.cap[slot] = 0;
        }
        if (hipMalloc(&t_stage.p[slot], bytes) != hipSuccess) {
            t_stage.p[slot] = nullptr;
            return set_error(PCL_ERR_OOM, "staging allocation of %zu bytes failed", bytes);
        }
        t_stage.cap[slot] = bytes;
    }
    *out = t_stage.p[slot];
    return PCL_OK;
}

// Upload `bytes` from host `src` into staging slot `slot` (src may be NULL:
// then *dev is NULL too, for optional operands such as bias).
int upload(int slot, const void *src, size_t bytes, void **dev) {
    PCL_OK_OR_RETURN(refuse_capture());
    if (!src) {
        *dev = nullptr;
        return PCL_OK;
    }
    PCL_OK_OR_RETURN(stage_buf(slot, bytes, dev));
    if (bytes) HIP_OK(hipMemcpyAsync(*dev, src, bytes, hipMemcpyHostToDevice, t_stream));
    return PCL_OK;
}

int download(void *dst, const void *dev, size_t bytes) {
    if (bytes) HIP_OK(hipMemcpyAsync(dst, dev, bytes, hipMemcpyDeviceToHost, t_stream));
    return PCL_OK;
}

int sync_current() {
    HIP_OK(hipStreamSynchronize(t_stream));
    return PCL_OK;
}

}  // namespace

namespace pcl {
int shim_error(int status, const char *msg) { return set_error(status, "%s", msg); }
int shim_init() { return do_init(); }
int sgemv_xf(int xf, int N, int K, const float *X, const float *W, int ldw,
             const float *g, const float *b, const float *bias, int accumulate, float *Y,
             void *stream) {
    PCL_OK_OR_RETURN(do_init());
    hipStream_t s = pick(stream);
    const GemvPlan p = plan_sgemv(1, 1, N, K);
    ScratchLease sc;
    PCL_OK_OR_RETURN(get_scratch(s, p.part_bytes, 0, &sc));
    HIP_OK(launch_sgemv_xf(p, xf, N, K, X, W, ldw, g, b, bias, accumulate, Y, sc->ws, s));
    return PCL_OK;
}
}  // namespace pcl

struct pcl_gemv_group {
    pcl::GgDesc *d_flat = nullptr;  // one descriptor per work item (strip in .strip)
    int n_items = 0, mr = 1;
    bool all_u8s8 = false;
    size_t lds = 0;
};

// =========================================================================
extern "C" {

int pcl_init(void) { return do_init(); }
int pcl_last_status(void) { return t_status; }
const char *pcl_last_error(void) { return t_msg; }
void pcl_clear_error(void) {
    t_status = PCL_OK;
    t_msg[0] = 0;
}
void pcl_set_abort_on_error(int on) { g_abort_on_error = on; }
int pcl_set_stream(void *s) {
    t_stream = (hipStream_t)s;
    return PCL_OK;
}
void *pcl_get_stream(void) { return (void *)t_stream; }
int pcl_stream_synchronize(void) {
    PCL_OK_OR_RETURN(do_init());
    return sync_current();
}

void *pcl_stream_create(void) {
    if (do_init() != PCL_OK) return nullptr;
    hipStream_t st = nullptr;
    if (hipStreamCreateWithFlags(&st, hipStreamNonBlocking) != hipSuccess) {
        set_error(PCL_ERR_HIP, "hipStreamCreateWithFlags failed");
        return nullptr;
    }
    return (void *)st;
}

int pcl_stream_destroy(void *stream) {
    CHECK_ARG(stream != nullptr, "pcl_stream_destroy: the null stream is not destroyed");
    PCL_OK_OR_RETURN(do_init());
    hipStream_t st = (hipStream_t)stream;
    HIP_OK(hipStreamSynchronize(st));
    {
        std::lock_guard<std::mutex> lk(g_mu);
        auto it = g_scratch.find(st);
        if (it != g_scratch.end()) {
            StreamScratch &sc = it->second;
            for (void *q : sc.retired) HIP_OK(hipFree(q));
            if (sc.ws.buf) HIP_OK(hipFree(sc.ws.buf));
            if (sc.aux) HIP_OK(hipFree(sc.aux));
            if (sc.realign) HIP_OK(hipFree(sc.realign));
            if (sc.amax) HIP_OK(hipFree(sc.amax));
            if (sc.tiles) HIP_OK(hipFree(sc.tiles));
            g_scratch.erase(it);
        }
    }
    if (t_stream == st) t_stream = nullptr;
    HIP_OK(hipStreamDestroy(st));
    return PCL_OK;
}

int pcl_release_scratch(void *stream) {
    PCL_OK_OR_RETURN(do_init());
    hipStream_t st = (hipStream_t)stream;
    StreamScratch *entry = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        auto it = g_scratch.find(st);
        if (it == g_scratch.end()) return PCL_OK;
        entry = &it->second;  // map nodes keep their address
    }
    // a call in flight on the stream holds its call lock until its last launch
    std::lock_guard<std::recursive_mutex> call(entry->call_mu);
    std::lock_guard<std::mutex> lk(g_mu);
    if (entry->pinned)
        return set_error(PCL_ERR_INVALID_ARG,
                         "pcl_release_scratch: a graph was captured on this stream and may use its "
                         "scratch; it is freed by pcl_stream_destroy");
    HIP_OK(hipStreamSynchronize(st));
    void **bufs[3] = {&entry->ws.buf, &entry->aux, &entry->realign};
    size_t *caps[3] = {&entry->ws.bytes_cap, &entry->aux_cap, &entry->realign_cap};
    for (int i = 0; i < 3; i++) {
        if (*bufs[i]) HIP_OK(hipFree(*bufs[i]));
        *bufs[i] = nullptr;
        *caps[i] = 0;
    }
    for (void *q : entry->retired) HIP_OK(hipFree(q));
    entry->retired.clear();
    if (entry->amax) HIP_OK(hipFree(entry->amax));
    entry->amax = nullptr;
    if (entry->tiles) HIP_OK(hipFree(entry->tiles));
    entry->tiles = nullptr;
    return PCL_OK;
}

int pcl_graph_begin(void) {
    PCL_OK_OR_RETURN(do_init());
    CHECK_ARG(t_stream != nullptr,
              "pcl_graph_begin: capture needs a stream from pcl_stream_create (pcl_set_stream)");
    {
        std::lock_guard<std::mutex> lk(g_mu);
        g_scratch[t_stream].pinned = true;
    }
    HIP_OK(hipStreamBeginCapture(t_stream, hipStreamCaptureModeRelaxed));
    t_capturing = true;
    return PCL_OK;
}

int pcl_graph_end(void **graph) {
    CHECK_ARG(graph != nullptr, "pcl_graph_end: graph is NULL");
    PCL_OK_OR_RETURN(do_init());
    CHECK_ARG(t_stream != nullptr, "pcl_graph_end: this thread's stream is the null stream");
    hipGraph_t g = nullptr;
    t_capturing = false;
    HIP_OK(hipStreamEndCapture(t_stream, &g));
    hipGraphExec_t ge = nullptr;
    hipError_t e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return set_error(PCL_ERR_HIP, "hipGraphInstantiate: %s", hipGetErrorString(e));
    *graph = (void *)ge;
    return PCL_OK;
}

int pcl_graph_launch(void *graph) {
    CHECK_ARG(graph != nullptr, "pcl_graph_launch: graph is NULL");
    PCL_OK_OR_RETURN(do_init());
    HIP_OK(hipGraphLaunch((hipGraphExec_t)graph, t_stream));
    return PCL_OK;
}

int pcl_graph_destroy(void *graph) {
    CHECK_ARG(graph != nullptr, "pcl_graph_destroy: graph is NULL");
    PCL_OK_OR_RETURN(do_init());
    HIP_OK(hipGraphExecDestroy((hipGraphExec_t)graph));
    return PCL_OK;
}

int pcl_device_info(char *name, int name_len, int *num_cus, int *clock_khz) {
    PCL_OK_OR_RETURN(do_init());
    int dev = 0;
    HIP_OK(hipGetDevice(&dev));
    hipDeviceProp_t prop;
    HIP_OK(hipGetDeviceProperties(&prop, dev));
    if (name && name_len > 0) snprintf(name, name_len, "%s (%s)", prop.name, prop.gcnArchName);
    if (num_cus) *num_cus = prop.multiProcessorCount;
    if (clock_khz) *clock_khz = prop.clockRate;
    return PCL_OK;
}

void *pcl_malloc(size_t bytes) {
    if (do_init() != PCL_OK) return nullptr;
    void *p = nullptr;
    if (hipMalloc(&p, bytes ? bytes : 16) != hipSuccess) {
        set_error(PCL_ERR_OOM, "hipMalloc(%zu) failed", bytes);
        return nullptr;
    }
    return p;
}
int pcl_free(void *p) {
    if (!p) return PCL_OK;
    HIP_OK(hipFree(p));
    return PCL_OK;
}
int pcl_memcpy_h2d(void *dst, const void *src, size_t bytes) {
    PCL_OK_OR_RETURN(do_init());
    HIP_OK(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return PCL_OK;
}
int pcl_memcpy_d2h(void *dst, const void *src, size_t bytes) {
    PCL_OK_OR_RETURN(do_init());
    HIP_OK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return PCL_OK;
}
int pcl_memcpy_d2d(void *dst, const void *src, size_t bytes) {
    PCL_OK_OR_RETURN(do_init());
    HIP_OK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice));
    return PCL_OK;
}
int pcl_memset(void *dst, int value, size_t bytes) {
    PCL_OK_OR_RETURN(do_init());
    HIP_OK(hipMemset(dst, value, bytes));
    return PCL_OK;
}

void *pcl_event_create(void) {
    if (do_init() != PCL_OK) return nullptr;
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) {
        set_error(PCL_ERR_HIP, "hipEventCreate failed");
        return nullptr;
    }
    return (void *)e;
}
int pcl_event_record(void *ev) {
    HIP_OK(hipEventRecord((hipEvent_t)ev, t_stream));
    return PCL_OK;
}
int pcl_event_elapsed_ms(void *start, void *stop, float *ms) {
    HIP_OK(hipEventSynchronize((hipEvent_t)stop));
    HIP_OK(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
    return PCL_OK;
}
int pcl_event_destroy(void *ev) {
    HIP_OK(hipEventDestroy((hipEvent_t)ev));
    return PCL_OK;
}

int pcl_set_model_dims(int d_model, int vocab_size) {
    CHECK_ARG(d_model > 0 && vocab_size > 0, "pcl_set_model_dims: dims must be positive (%d, %d)",
              d_model, vocab_size);
    g_d_model = d_model;
    g_vocab = vocab_size;
    return PCL_OK;
}

int pcl_set_attn_dims(int batch, int seq_len, int n_heads) {
    CHECK_ARG(batch > 0 && seq_len > 0 && n_heads > 0,
              "pcl_set_attn_dims: dims must be positive (%d, %d, %d)", batch, seq_len, n_heads);
    g_attn_batch = batch;
    g_attn_seq = seq_len;
    g_attn_heads = n_heads;
    return PCL_OK;
}

// ----------------------------------------------------------- FP32 native ----
int pcl_sgemv(int opW, int M, int N, int K, const float *X, int ldx, const float *W, int ldw,
              const float *bias, int accumulate, float *Y, int ldy, void *stream) {
    CHECK_ARG(M >= 0 && N >= 0 && K >= 0, "pcl_sgemv: negative dimension (M=%d N=%d K=%d)", M, N, K);
    CHECK_ARG(M <= 8, "pcl_sgemv: M=%d exceeds the decode limit of 8 rows", M);
    CHECK_ARG(opW == PCL_OP_N || opW == PCL_OP_T, "pcl_sgemv: bad opW %d", opW);
    if (M == 0 || N == 0) return PCL_OK;
    CHECK_ARG(Y != nullptr, "pcl_sgemv: Y is NULL");
    CHECK_ARG(ldy >= N, "pcl_sgemv: ldy=%d < N=%d", ldy, N);
    if (K > 0) {
        CHECK_ARG(X && W, "pcl_sgemv: NULL operand");
        CHECK_ARG(ldx >= K, "pcl_sgemv: ldx=%d < K=%d", ldx, K);
        CHECK_ARG(ldw >= (opW == PCL_OP_N ? N : K), "pcl_sgemv: ldw=%d too small", ldw);
    }
    PCL_OK_OR_RETURN(do_init());
    hipStream_t s = pick(stream);
    pcl::GemvPlan p = pcl::plan_sgemv(opW == PCL_OP_T, M, N, K);
    ScratchLease sc;
    PCL_OK_OR_RETURN(get_scratch(s, p.part_bytes, 0, &sc));
    HIP_OK(pcl::launch_sgemv(p, opW == PCL_OP_T, M, N, K, X, ldx, false, W, ldw, bias, accumulate,
                             Y, ldy, sc->ws, s));
    return PCL_OK;
}

// ------------------------------------------------------ measured roofs ----
int pcl_measure_peak_mfma(int data, double *rate) {
    CHECK_ARG(rate != nullptr, "pcl_measure_peak_mfma: rate is NULL");
    CHECK_ARG(data >= 0 && data <= 2, "pcl_measure_peak_mfma: data must be 0, 1 or 2 (got %d)", data);
    PCL_OK_OR_RETURN(do_init());
    int dev = 0, cus = 0;
    HIP_OK(hipGetDevice(&dev));
    HIP_OK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    HIP_OK(pcl::measure_peak_mfma(data, cus, rate, pick(nullptr)));
    return PCL_OK;
}

int pcl_measure_bandwidth(long bytes_per_array, double gbs[4]) {
    CHECK_ARG(gbs != nullptr, "pcl_measure_bandwidth: NULL result pointer");
    CHECK_ARG(bytes_per_array >= (64L << 20), "pcl_measure_bandwidth: arrays of at least 64 MiB (got %ld)",
              bytes_per_array);
    PCL_OK_OR_RETURN(do_init());
    HIP_OK(pcl::measure_bandwidth(bytes_per_array, gbs, pick(nullptr)));
    return PCL_OK;
}

int pcl_measure_lds_feed(int M, int N, int K, double *gbs) {
    CHECK_ARG(gbs != nullptr, "pcl_measure_lds_feed: NULL result pointer");
    CHECK_ARG(M > 0 && N > 0 && K > 0 && M % 128 == 0 && N % 128 == 0 && K % 128 == 0,
              "pcl_measure_lds_feed: M, N, K must be positive multiples of 128 (%d, %d, %d)", M, N, K);
    CHECK_ARG((long)M * K < (1L << 31) && (long)N * K < (1L << 31),
              "pcl_measure_lds_feed: operands of 2^31 bytes or more");
    PCL_OK_OR_RETURN(do_init());
    HIP_OK(pcl::measure_lds_feed(M, N, K, gbs, pick(nullptr)));
    return PCL_OK;
}

int pcl_measure_tile_read(int M, int N, int K, double *gbs) {
    CHECK_ARG(gbs != nullptr, "pcl_measure_tile_read: NULL result pointer");
    CHECK_ARG(M > 0 && N > 0 && K > 0 && M % 128 == 0 && N % 128 == 0 && K % 128 == 0,
              "pcl_measure_tile_read: M, N, K must be positive multiples of 128 (%d, %d, %d)", M, N, K);
    CHECK_ARG((long)M * K < (1L << 31) && (long)N * K < (1L << 31),
              "pcl_measure_tile_read: operands of 2^31 bytes or more");
    PCL_OK_OR_RETURN(do_init());
    HIP_OK(pcl::measure_lds_feed(M, N, K, gbs, pick(nullptr), true));
    return PCL_OK;
}

// ------------------------------------------------------ grouped GEMV ----
int pcl_gemv_group_create(const pcl_gemv_desc *descs, int n, pcl_gemv_group **group) {
    CHECK_ARG(group != nullptr, "pcl_gemv_group_create: group is NULL");
    *group = nullptr;
    CHECK_ARG(descs != nullptr && n > 0, "pcl_gemv_group_create: need n >= 1 products (n=%d)", n);
    std::vector<pcl::GgDesc> dd((size_t)n);
    struct Item {
        long bytes;
        int prod, strip;
    };
    std::vector<Item> items;
    int mr = 1;
    for (int i = 0; i < n; i++) {
        const pcl_gemv_desc &q = descs[i];
        CHECK_ARG(q.kind == PCL_GEMV_F32_N || q.kind == PCL_GEMV_F32_T || q.kind == PCL_GEMV_U8S8,
                  "pcl_gemv_group_create: product %d: unknown kind %d", i, q.kind);
        CHECK_ARG(q.M >= 1 && q.M <= 8 && q.N >= 1 && q.K >= 1,
                  "pcl_gemv_group_create: product %d: need 1 <= M <= 8, N >= 1, K >= 1 (M=%d N=%d K=%d)",
                  i, q.M, q.N, q.K);
        CHECK_ARG(q.X && q.W && q.Y, "pcl_gemv_group_create: product %d: NULL operand", i);
        CHECK_ARG(q.ldy >= q.N, "pcl_gemv_group_create: product %d: ldy=%d < N=%d", i, q.ldy, q.N);
        CHECK_ARG(q.ldx >= q.K, "pcl_gemv_group_create: product %d: ldx=%d < K=%d", i, q.ldx, q.K);
        if (q.kind == PCL_GEMV_F32_N) {
            CHECK_ARG(q.N % 4 == 0 && q.ldw >= q.N && q.ldw % 4 == 0 && aligned16(q.W),
                      "pcl_gemv_group_create: product %d: F32_N needs N %% 4 == 0, ldw >= N, ldw %% 4 "
                      "== 0 and a 16-byte aligned W (N=%d ldw=%d)",
                      i, q.N, q.ldw);
        } else if (q.kind == PCL_GEMV_F32_T) {
            CHECK_ARG(q.K % 4 == 0 && q.ldw >= q.K && q.ldw % 4 == 0 && aligned16(q.W),
                      "pcl_gemv_group_create: product %d: F32_T needs K %% 4 == 0, ldw >= K, ldw %% 4 "
                      "== 0 and a 16-byte aligned W (K=%d ldw=%d)",
                      i, q.K, q.ldw);
        } else {
            CHECK_ARG(q.ldw >= kpad256(q.K) && q.ldw % 16 == 0 && aligned16(q.W),
                      "pcl_gemv_group_create: product %d: U8S8 needs packed rows of ldw >= %d "
                      "(a multiple of 16) and a 16-byte aligned W (ldw=%d)",
                      i, kpad256(q.K), q.ldw);
            CHECK_ARG(q.sb || !q.sa, "pcl_gemv_group_create: product %d: sa without sb", i);
        }
        pcl::GgDesc &g = dd[(size_t)i];
        g.kind = q.kind == PCL_GEMV_F32_N ? pcl::GG_F32_N : (q.kind == PCL_GEMV_F32_T ? pcl::GG_F32_T : pcl::GG_U8S8);
        g.M = q.M, g.N = q.N, g.K = q.K;
        g.X = q.X, g.ldx = q.ldx, g.W = q.W, g.ldw = q.ldw;
        g.bias = q.kind == PCL_GEMV_U8S8 ? nullptr : q.bias;
        g.col_off = q.kind == PCL_GEMV_U8S8 ? q.col_off : nullptr;
        g.sa = q.sa, g.sb = q.sb;
        g.Y = q.Y, g.ldy = q.ldy;
        g.accumulate = q.kind == PCL_GEMV_U8S8 ? 0 : (q.accumulate ? 1 : 0);
        g.out_mode = q.kind != PCL_GEMV_U8S8 ? 0 : (!q.sb ? 0 : (q.sa ? 2 : 1));
        g.xld = pcl::gg_stage_ld(g.kind, q.K);
        g.strip = 0;
        const int m1 = q.M <= 1 ? 1 : (q.M <= 2 ? 2 : (q.M <= 4 ? 4 : 8));
        if (m1 > mr) mr = m1;
        CHECK_ARG((long)q.N * q.ldw < (1L << 31),
                  "pcl_gemv_group_create: product %d: N * ldw must stay below 2^31 bytes", i);
    }
    const bool all_u8s8 =
        std::all_of(dd.begin(), dd.end(), [](const pcl::GgDesc &q) { return q.kind == pcl::GG_U8S8; });
    for (int i = 0; i < n; i++) {
        const pcl::GgDesc &g = dd[(size_t)i];
        const int rows = pcl::gg_strip_rows(g.kind);
        const int strips = (g.N + rows - 1) / rows;
        const long bytes = (long)rows * (g.kind == pcl::GG_U8S8 ? g.ldw : 4L * g.K);
        for (int t = 0; t < strips; t++) items.push_back({bytes, i, t});
        CHECK_ARG(items.size() < (size_t)(1 << 30), "pcl_gemv_group_create: too many work items");
    }
    size_t lds = 0;
    for (int i = 0; i < n; i++) {
        const size_t b = pcl::gg_lds_bytes(dd[(size_t)i].kind, dd[(size_t)i].K, mr);
        if (b > lds) lds = b;
    }
    if (lds > 65536 + 49152)
        return set_error(PCL_ERR_RANGE,
                         "pcl_gemv_group_create: staged operands need %zu bytes of LDS per block (at most "
                         "%d): reduce K or M, or split the group",
                         lds, 65536 + 49152);
    // largest blocks first, so the tail of the launch is short ones
    std::stable_sort(items.begin(), items.end(), [](const Item &a, const Item &b) { return a.bytes > b.bytes; });
    std::vector<pcl::GgDesc> flat(items.size());
    for (size_t t = 0; t < items.size(); t++) {
        flat[t] = dd[(size_t)items[t].prod];
        flat[t].strip = items[t].strip;
    }
    PCL_OK_OR_RETURN(do_init());
    pcl_gemv_group *g = new (std::nothrow) pcl_gemv_group();
    if (!g) return set_error(PCL_ERR_OOM, "pcl_gemv_group_create: out of host memory");
    g->n_items = (int)flat.size();
    g->mr = mr;
    g->lds = lds;
    g->all_u8s8 = all_u8s8;
    if (hipMalloc((void **)&g->d_flat, sizeof(pcl::GgDesc) * flat.size()) != hipSuccess) {
        pcl_gemv_group_free(g);
        return set_error(PCL_ERR_OOM, "pcl_gemv_group_create: device allocation failed");
    }
    if (hipMemcpy(g->d_flat, flat.data(), sizeof(pcl::GgDesc) * flat.size(), hipMemcpyHostToDevice) != hipSuccess) {
        pcl_gemv_group_free(g);
        return set_error(PCL_ERR_HIP, "pcl_gemv_group_create: copying the plan to the device failed");
    }
    *group = g;
    return PCL_OK;
}

int pcl_gemv_group_run(const pcl_gemv_group *group, void *stream) {
    CHECK_ARG(group != nullptr, "pcl_gemv_group_run: group is NULL");
    PCL_OK_OR_RETURN(do_init());
    HIP_OK(pcl::launch_gemv_group(group->d_flat, group->n_items, group->mr, group->lds,
                                  group->all_u8s8, pick(stream)));
    return PCL_OK;
}

void pcl_gemv_group_free(pcl_gemv_group *group) {
    if (!group) return;
    if (group->d_flat) (void)hipFree(group->d_flat);
    delete group;
}

// pcl_sgemv with its split-K partial sums in the static device scratch of
// gemv.hip instead of the per-stream workspace: no allocation of any kind.
// Same kernels, plan and summation order as pcl_sgemv, so the results are
// identical.
int pcl_sgemv_noalloc(int opW, int M, int N, int K, const float *X, int ldx, const float *W,
                      int ldw, const float *bias, int accumulate, float *Y, int ldy, void *stream) {
    CHECK_ARG(M >= 0 && N >= 0 && K >= 0, "pcl_sgemv_noalloc: negative dimension (M=%d N=%d K=%d)",
              M, N, K);
    CHECK_ARG(M <= 8, "pcl_sgemv_noalloc: M=%d exceeds the decode limit of 8 rows", M);
    CHECK_ARG(opW == PCL_OP_N || opW == PCL_OP_T, "pcl_sgemv_noalloc: bad opW %d", opW);
    if (M == 0 || N == 0) return PCL_OK;
    CHECK_ARG(Y != nullptr, "pcl_sgemv_noalloc: Y is NULL");
    CHECK_ARG(ldy >= N, "pcl_sgemv_noalloc: ldy=%d < N=%d", ldy, N);
    if (K > 0) {
        CHECK_ARG(X && W, "pcl_sgemv_noalloc: NULL operand");
        CHECK_ARG(ldx >= K, "pcl_sgemv_noalloc: ldx=%d < K=%d", ldx, K);
        CHECK_ARG(ldw >= (opW == PCL_OP_N ? N : K), "pcl_sgemv_noalloc: ldw=%d too small", ldw);
    }
    PCL_OK_OR_RETURN(do_init());
    const pcl::GemvPlan p = pcl::plan_sgemv(opW == PCL_OP_T, M, N, K);
    if (p.part_bytes > pcl::GEMV_NOALLOC_SCRATCH_BYTES)
        return set_error(PCL_ERR_RANGE,
                         "pcl_sgemv_noalloc: M=%d N=%d K=%d needs %zu bytes of split-K scratch, "
                         "beyond the static %zu",
                         M, N, K, p.part_bytes, pcl::GEMV_NOALLOC_SCRATCH_BYTES);
    int dev = 0;
    HIP_OK(hipGetDevice(&dev));
    void *scr = nullptr;
    PCL_OK_OR_RETURN(noalloc_scratch(dev, &scr));
    pcl::Workspace ws;
    ws.buf = scr;
    ws.bytes_cap = pcl::GEMV_NOALLOC_SCRATCH_BYTES;
    HIP_OK(pcl::launch_sgemv(p, opW == PCL_OP_T, M, N, K, X, ldx, false, W, ldw, bias, accumulate,
                             Y, ldy, ws, pick(stream)));
    return PCL_OK;
}

// A large product whose operands miss the LDS-DMA kernel's requirements
// (16-byte aligned rows, contiguous extents a multiple of 4 floats, K a
// multiple of 32), e.g. the trainer's head backward over 50257-float logits
// rows (train_kaggle.cu:173-174 through gemm_nn / gemm_tn): each misaligned
// operand is copied into rows of a multiple of 64 floats (one pass into the
// stream's workspace, launch_copy_rows), the 64-aligned core (M1 x N1 x K1) runs
// on the LDS-DMA kernel, and the ragged edges -- the K tail of the core,
// added on; the rows past M1 and the columns past N1 at full K -- run on the
// generic kernel with the original operands. Returns 1 when the shape has no
// aligned core (the caller takes the generic kernel instead).
static int sgemm_realigned(int opA, int opB, int M, int N, int K, const float *A, int lda,
                           const float *B, int ldb, const float *bias, int accumulate, float *C,
                           int ldc, hipStream_t s) {
    const bool a_kc = opA == PCL_OP_N, b_kc = opB == PCL_OP_T;  // K-contiguous operands
    const int K1 = K & ~63, M1 = a_kc ? M : (M & ~63), N1 = b_kc ? N : (N & ~63);
    if (K1 == 0 || M1 == 0 || N1 == 0) return 1;
    const long rows_a = a_kc ? M : K, cols_a = a_kc ? K : M;
    const long rows_b = b_kc ? N : K, cols_b = b_kc ? K : N;
    const bool copy_a = !aligned16(A) || lda % 4 != 0, copy_b = !aligned16(B) || ldb % 4 != 0;
    const long lda2 = copy_a ? (cols_a + 63) / 64 * 64 : lda, ldb2 = copy_b ? (cols_b + 63) / 64 * 64 : ldb;
    const size_t abytes = copy_a ? (size_t)rows_a * lda2 * 4 : 0, bbytes = copy_b ? (size_t)rows_b * ldb2 * 4 : 0;
    const pcl::SgemmPlan pc = pcl::plan_sgemm(M1, N1, K1);
    const pcl::SgemmPlan pk = pcl::plan_sgemm(M1, N1, K - K1);
    const pcl::SgemmPlan pm = pcl::plan_sgemm(M - M1, N, K);
    const pcl::SgemmPlan pn = pcl::plan_sgemm(M1, N - N1, K);
    size_t part = pc.part_bytes;
    if (K > K1 && pk.part_bytes > part) part = pk.part_bytes;
    if (M > M1 && pm.part_bytes > part) part = pm.part_bytes;
    if (N > N1 && pn.part_bytes > part) part = pn.part_bytes;
    ScratchLease sc;
    PCL_OK_OR_RETURN(get_scratch(s, part, 0, &sc, abytes + bbytes + 256));
    float *Ac = const_cast<float *>(A), *Bc = const_cast<float *>(B);
    if (copy_a) {
        Ac = static_cast<float *>(sc->realign);
        HIP_OK(pcl::launch_copy_rows(Ac, lda2, A, lda, (int)rows_a, (int)cols_a, s));
    }
    if (copy_b) {
        Bc = reinterpret_cast<float *>(static_cast<char *>(sc->realign) + (abytes + 255) / 256 * 256);
        HIP_OK(pcl::launch_copy_rows(Bc, ldb2, B, ldb, (int)rows_b, (int)cols_b, s));
    }
    // the aligned core, then its K tail added on
    HIP_OK(pcl::launch_sgemm(pc, a_kc, b_kc, M1, N1, K1, Ac, lda2, Bc, ldb2, bias, accumulate, C, ldc, sc->ws, s));
    if (K > K1) {
        const float *Ak = a_kc ? A + K1 : A + (size_t)K1 * lda;
        const float *Bk = b_kc ? B + K1 : B + (size_t)K1 * ldb;
        HIP_OK(pcl::launch_sgemm(pk, a_kc, b_kc, M1, N1, K - K1, Ak, lda, Bk, ldb, nullptr, 1, C, ldc, sc->ws, s));
    }
    if (M > M1) {  // rows M1.. of C, every column, full K
        const float *Am = a_kc ? A + (size_t)M1 * lda : A + M1;
        HIP_OK(pcl::launch_sgemm(pm, a_kc, b_kc, M - M1, N, K, Am, lda, B, ldb, bias, accumulate,
                                 C + (size_t)M1 * ldc, ldc, sc->ws, s));
    }
    if (N > N1) {  // columns N1.. of rows 0 .. M1-1, full K
        const float *Bn = b_kc ? B + (size_t)N1 * ldb : B + N1;
        HIP_OK(pcl::launch_sgemm(pn, a_kc, b_kc, M1, N - N1, K, A, lda, Bn, ldb, bias ? bias + N1 : nullptr,
                                 accumulate, C + N1, ldc, sc->ws, s));
    }
    return PCL_OK;
}

int pcl_sgemm(int opA, int opB, int M, int N, int K, const float *A, int lda, const float *B,
              int ldb, const float *bias, int accumulate, float *C, int ldc, void *stream) {
    CHECK_ARG(M >= 0 && N >= 0 && K >= 0, "pcl_sgemm: negative dimension (M=%d N=%d K=%d)", M, N, K);
    CHECK_ARG((opA == PCL_OP_N || opA == PCL_OP_T) && (opB == PCL_OP_N || opB == PCL_OP_T),
              "pcl_sgemm: bad op (%d, %d)", opA, opB);
    if (M == 0 || N == 0) return PCL_OK;
    CHECK_ARG(C != nullptr, "pcl_sgemm: C is NULL");
    CHECK_ARG(ldc >= N, "pcl_sgemm: ldc=%d < N=%d", ldc, N);
    if (K > 0) {
        CHECK_ARG(A && B, "pcl_sgemm: NULL operand");
        CHECK_ARG(lda >= (opA == PCL_OP_N ? K : M), "pcl_sgemm: lda=%d too small", lda);
        CHECK_ARG(ldb >= (opB == PCL_OP_N ? N : K), "pcl_sgemm: ldb=%d too small", ldb);
    }
    PCL_OK_OR_RETURN(do_init());
    if (M <= 8 && opA == PCL_OP_N)
        return pcl_sgemv(opB, M, N, K, A, lda, B, ldb, bias, accumulate, C, ldc, stream);
    hipStream_t s = pick(stream);
    if (K > 0 && (double)M * N * K >= (double)(1L << 30)) {
        const bool a_kc = opA == PCL_OP_N, b_kc = opB == PCL_OP_T;
        const bool dma_ok = aligned16(A) && aligned16(B) && lda % 4 == 0 && ldb % 4 == 0 &&
                            (a_kc ? K % 4 == 0 : M % 4 == 0) && (b_kc ? K % 4 == 0 : N % 4 == 0) &&
                            K % 32 == 0;
        if (!dma_ok) {
            const int st = sgemm_realigned(opA, opB, M, N, K, A, lda, B, ldb, bias, accumulate, C, ldc, s);
            if (st != 1) return st;
        }
    }
    pcl::SgemmPlan p = pcl::plan_sgemm(M, N, K, opA == PCL_OP_N);
    ScratchLease sc;
    PCL_OK_OR_RETURN(get_scratch(s, p.part_bytes, 0, &sc));
    HIP_OK(pcl::launch_sgemm(p, opA == PCL_OP_N, opB == PCL_OP_T, M, N, K, A, lda, B, ldb, bias,
                             accumulate, C, ldc, sc->ws, s));
    return PCL_OK;
}

int pcl_sgemm_ex(int opA, int opB, int M, int N, int K, const float *A, int lda, const float *B,
                 int ldb, const float *bias, int epilogue, const float *aux_in, float *aux_out,
                 int ld_aux, float *C, int ldc, void *stream) {
    CHECK_ARG(epilogue >= PCL_EPI_NONE && epilogue <= PCL_EPI_GELU_BWD,
              "pcl_sgemm_ex: unknown epilogue %d", epilogue);
    if (epilogue == PCL_EPI_NONE)
        return pcl_sgemm(opA, opB, M, N, K, A, lda, B, ldb, bias, 0, C, ldc, stream);
    CHECK_ARG(M >= 0 && N >= 0 && K >= 0, "pcl_sgemm_ex: negative dimension (M=%d N=%d K=%d)", M, N,
              K);
    CHECK_ARG((opA == PCL_OP_N || opA == PCL_OP_T) && (opB == PCL_OP_N || opB == PCL_OP_T),
              "pcl_sgemm_ex: bad op (%d, %d)", opA, opB);
    if (M == 0 || N == 0) return PCL_OK;
    CHECK_ARG(C != nullptr, "pcl_sgemm_ex: C is NULL");
    CHECK_ARG(ldc >= N, "pcl_sgemm_ex: ldc=%d < N=%d", ldc, N);
    if (K > 0) {
        CHECK_ARG(A && B, "pcl_sgemm_ex: NULL operand");
        CHECK_ARG(lda >= (opA == PCL_OP_N ? K : M), "pcl_sgemm_ex: lda=%d too small", lda);
        CHECK_ARG(ldb >= (opB == PCL_OP_N ? N : K), "pcl_sgemm_ex: ldb=%d too small", ldb);
    }
    CHECK_ARG(epilogue == PCL_EPI_GELU || aux_in != nullptr,
              "pcl_sgemm_ex: the epilogue needs aux_in");
    CHECK_ARG((aux_in == nullptr && aux_out == nullptr) || ld_aux >= N,
              "pcl_sgemm_ex: ld_aux=%d < N=%d", ld_aux, N);
    // The epilogue operands may not share memory with C: depending on the
    // kernel chosen for the shape, C is written before the epilogue reads
    // aux_in (e.g. an in-place residual would add v twice).
    {
        const size_t nc = sizeof(float) * ((size_t)(M - 1) * ldc + N);
        const size_t na = sizeof(float) * ((size_t)(M - 1) * (size_t)(ld_aux > 0 ? ld_aux : N) + N);
        CHECK_ARG(!aux_in || !ranges_overlap(aux_in, na, C, nc),
                  "pcl_sgemm_ex: aux_in overlaps C (write the product to another buffer)");
        CHECK_ARG(!aux_out || epilogue != PCL_EPI_GELU || !ranges_overlap(aux_out, na, C, nc),
                  "pcl_sgemm_ex: aux_out overlaps C");
    }
    PCL_OK_OR_RETURN(do_init());
    hipStream_t s = pick(stream);
    pcl::SgemmPlan p = pcl::plan_sgemm(M, N, K, opA == PCL_OP_N);
    ScratchLease sc;
    PCL_OK_OR_RETURN(get_scratch(s, p.part_bytes, 0, &sc));
    HIP_OK(pcl::launch_sgemm(p, opA == PCL_OP_N, opB == PCL_OP_T, M, N, K, A, lda, B, ldb, bias, 0,
                             C, ldc, sc->ws, s, epilogue, aux_in, epilogue == PCL_EPI_GELU ? aux_out : nullptr,
                             ld_aux));
    return PCL_OK;
}

static int elementwise(const char *who, int op, float *out, const float *a, const float *b,
                       long n, void *stream) {
    CHECK_ARG(n >= 0, "%s: negative length %ld", who, n);
    if (n == 0) return PCL_OK;
    CHECK_ARG(out && a && (op == 0 || b), "%s: NULL operand", who);
    PCL_OK_OR_RETURN(do_init());
    HIP_OK(pcl::launch_elementwise(op, n, out, a, b, pick(stream)));
    return PCL_OK;
}
int pcl_gelu_fwd(float *Y, const float *X, long n, void *stream) {
    return elementwise("pcl_gelu_fwd", 0, Y, X, nullptr, n, stream);
}
int pcl_gelu_bwd(float *dX, const float *dY, const float *X, long n, void *stream) {
    return elementwise("pcl_gelu_bwd", 1, dX, dY, X, n, stream);
}
int pcl_vec_add(float *C, const float *A, const float *B, long n, void *stream) {
    return elementwise("pcl_vec_add", 2, C, A, B, n, stream);
}

int pcl_bias_bwd(float *db, const float *dY, int M, int N, int ld, void *stream) {
    CHECK_ARG(M >= 0 && N >= 0, "pcl_bias_bwd: negative dimension");
    if (N == 0) return PCL_OK;
    CHECK_ARG(db != nullptr, "pcl_bias_bwd: db is NULL");
    if (M > 0) {
        CHECK_ARG(dY != nullptr, "pcl_bias_bwd: dY is NULL");
        CHECK_ARG(ld >= N, "pcl_bias_bwd: ld=%d < N=%d", ld, N);
    }
    PCL_OK_OR_RETURN(do_init());
    hipStream_t s = pick(stream);
    pcl::GemvPlan p = pcl::plan_bias_bwd(N, M);
    ScratchLease sc;
    PCL_OK_OR_RETURN(get_scratch(s, p.part_bytes, 0, &sc));
    HIP_OK(pcl::launch_sgemv(p, 0, 1, N, M, nullptr, 0, true, dY, ld, nullptr, 1, db, N, sc->ws, s));
    return PCL_OK;
}

int pcl_attn_fwd(const float *Q, const float *K, const float *V, int ld, float *att, int ld_att,
                 float *probs, int B, int T, int H, int dh, void *stream) {
    CHECK_ARG(B >= 0 && T >= 0 && H >= 0, "pcl_attn_fwd: negative dimension (B=%d T=%d H=%d)", B,
              T, H);
    CHECK_ARG(dh == 32 || dh == 64 || dh == 128, "pcl_attn_fwd: head size %d is not 32, 64 or 128",
              dh);
    if (B == 0 || T == 0 || H == 0) return PCL_OK;
    CHECK_ARG(Q && K && V && att, "pcl_attn_fwd: NULL operand");
    CHECK_ARG(ld >= H * dh && ld_att >= H * dh, "pcl_attn_fwd: ld=%d / ld_att=%d < H*dh=%d", ld,
              ld_att, H * dh);
    CHECK_ARG(ld % 4 == 0 && ld_att % 4 == 0, "pcl_attn_fwd: ld=%d, ld_att=%d not multiples of 4",
              ld, ld_att);
    CHECK_ARG(aligned16(Q) && aligned16(K) && aligned16(V) && aligned16(att),
              "pcl_attn_fwd: Q, K, V and att must be 16-byte aligned");
    CHECK_ARG((long)B * T <= INT32_MAX && (long)B * H * T <= INT32_MAX,
              "pcl_attn_fwd: B*T or B*H*T beyond 2^31");
    PCL_OK_OR_RETURN(do_init());
    HIP_OK(pcl::launch_attn_fwd(Q, K, V, ld, att, ld_att, probs, B, T, H, dh,
                                1.0f / sqrtf((float)dh), pick(stream)));
    return PCL_OK;
}

int pcl_attn_fwd_lse(const float *Q, const float *K, const float *V, int ld, float *att, int ld_att,
                     float *lse, int B, int T, int H, int dh, void *stream) {
    CHECK_ARG(B >= 0 && T >= 0 && H >= 0, "pcl_attn_fwd_lse: negative dimension (B=%d T=%d H=%d)",
              B, T, H);
    CHECK_ARG(dh == 32 || dh == 64 || dh == 128,
              "pcl_attn_fwd_lse: head size %d is not 32, 64 or 128", dh);
    if (B == 0 || T == 0 || H == 0) return PCL_OK;
    CHECK_ARG(Q && K && V && att, "pcl_attn_fwd_lse: NULL operand");
    CHECK_ARG(ld >= H * dh && ld_att >= H * dh, "pcl_attn_fwd_lse: ld=%d / ld_att=%d < H*dh=%d", ld,
              ld_att, H * dh);
    CHECK_ARG(ld % 4 == 0 && ld_att % 4 == 0,
              "pcl_attn_fwd_lse: ld=%d, ld_att=%d not multiples of 4", ld, ld_att);
    CHECK_ARG(aligned16(Q) && aligned16(K) && aligned16(V) && aligned16(att),
              "pcl_attn_fwd_lse: Q, K, V and att must be 16-byte aligned");
    CHECK_ARG((long)B * T <= INT32_MAX && (long)B * H * T <= INT32_MAX,
              "pcl_attn_fwd_lse: B*T or B*H*T beyond 2^31");
    if (lse) {
        const long n = (long)B * H * T;
        CHECK_ARG(!ranges_overlap(lse, 4 * n, att, 4 * ((long)(B * T - 1) * ld_att + H * dh)),
                  "pcl_attn_fwd_lse: lse overlaps att");
    }
    PCL_OK_OR_RETURN(do_init());
    HIP_OK(pcl::launch_attn_fwd(Q, K, V, ld, att, ld_att, nullptr, B, T, H, dh,
                                1.0f / sqrtf((float)dh), pick(stream), lse));
    return PCL_OK;
}

namespace {
int attn_bwd_common(const char *fn, float *dQ, float *dK, float *dV, int ld_grad, float *scratch,
                    const float *dAtt, int ld_att, const float *Q, const float *K, const float *V,
                    int ld, const float *probs, const float *att, int ld_o, int B, int T, int H,
                    int dh, int accumulate, void *stream) {
    CHECK_ARG(B >= 0 && T >= 0 && H >= 0, "%s: negative dimension (B=%d T=%d H=%d)", fn, B, T, H);
    CHECK_ARG(dh == 32 || dh == 64 || dh == 128, "%s: head size %d is not 32, 64 or 128", fn, dh);
    if (B == 0 || T == 0 || H == 0) return PCL_OK;
    CHECK_ARG(dQ && dK && dV && dAtt && Q && K && V && probs, "%s: NULL operand", fn);
    CHECK_ARG(ld >= H * dh && ld_att >= H * dh && ld_grad >= H * dh,
              "%s: a leading dimension is below H*dh=%d", fn, H * dh);
    CHECK_ARG(ld % 4 == 0 && ld_att % 4 == 0, "%s: ld=%d, ld_att=%d not multiples of 4", fn, ld,
              ld_att);
    CHECK_ARG(aligned16(Q) && aligned16(K) && aligned16(V) && aligned16(dAtt),
              "%s: Q, K, V and dAtt must be 16-byte aligned", fn);
    if (att)
        CHECK_ARG(ld_o >= H * dh && ld_o % 4 == 0 && aligned16(att),
                  "%s: att needs ld_o >= H*dh, a multiple of 4, and 16-byte alignment", fn);
    CHECK_ARG((long)B * T <= INT32_MAX && (long)B * H * T <= INT32_MAX,
              "%s: B*T or B*H*T beyond 2^31", fn);
    PCL_OK_OR_RETURN(do_init());
    hipStream_t s = pick(stream);
    float *dS = scratch;
    if (!dS) {
        ScratchLease sc;
        PCL_OK_OR_RETURN(get_scratch(s, sizeof(float) * (size_t)B * H * T * T, 0, &sc));
        dS = static_cast<float *>(sc->ws.buf);
    }
    HIP_OK(pcl::launch_attn_bwd(dAtt, ld_att, Q, K, V, ld, probs, dS, dQ, dK, dV, ld_grad, B, T, H,
                                dh, 1.0f / sqrtf((float)dh), accumulate, s, att, ld_o));
    return PCL_OK;
}
}  // namespace

int pcl_attn_bwd(float *dQ, float *dK, float *dV, int ld_grad, float *scratch, const float *dAtt,
                 int ld_att, const float *Q, const float *K, const float *V, int ld,
                 const float *probs, int B, int T, int H, int dh, int accumulate, void *stream) {
    return attn_bwd_common("pcl_attn_bwd", dQ, dK, dV, ld_grad, scratch, dAtt, ld_att, Q, K, V, ld,
                           probs, nullptr, 0, B, T, H, dh, accumulate, stream);
}

int pcl_attn_bwd_ex(float *dQ, float *dK, float *dV, int ld_grad, float *scratch,
                    const float *dAtt, int ld_att, const float *Q, const float *K, const float *V,
                    int ld, const float *probs, const float *att, int ld_o, int B, int T, int H,
                    int dh, int accumulate, void *stream) {
    if (!att) return set_error(PCL_ERR_INVALID_ARG, "pcl_attn_bwd_ex: att is NULL");
    return attn_bwd_common("pcl_attn_bwd_ex", dQ, dK, dV, ld_grad, scratch, dAtt, ld_att, Q, K, V,
                           ld, probs, att, ld_o, B, T, H, dh, accumulate, stream);
}

// ----------------------------------------------------------- INT8 native ----
int pcl_s8_kpad(int K) { return kpad256(K < 0 ? 0 : K); }
size_t pcl_s8_packed_bytes(int K, int N) {
    return (size_t)(N < 0 ? 0 : N) * (size_t)pcl_s8_kpad(K);
}

int pcl_pack_b_s8(const int8_t *B, int ldb, int K, int N, int8_t *Bpk, int32_t *colsum,
                  void *stream) {
    CHECK_ARG(K >= 0 && N >= 0, "pcl_pack_b_s8: negative dimension");
    if (N == 0) return PCL_OK;
    CHECK_ARG(Bpk != nullptr && (K == 0 || B != nullptr), "pcl_pack_b_s8: NULL operand");
    CHECK_ARG(K == 0 || ldb >= N, "pcl_pack_b_s8: ldb=%d < N=%d", ldb, N);
    PCL_OK_OR_RETURN(do_init());
    HIP_OK(pcl::launch_pack_b_s8(B, ldb, K, N, Bpk, kpad256(K), colsum, pick(stream)));
    return PCL_OK;
}

int pcl_pack_b_vnni(const int8_t *Bp, int K, int Kpad, int N, int8_t *Bpk, int32_t *colsum,
                    void *stream) {
    CHECK_ARG(K >= 0 && N >= 0 && Kpad >= K && Kpad % 4 == 0,
              "pcl_pack_b_vnni: need 0 <= K <= Kpad, Kpad %% 4 == 0 (K=%d Kpad=%d)", K, Kpad);
    CHECK_ARG(N % 16 == 0, "pcl_pack_b_vnni: N=%d is not a multiple of 16", N);
    if (N == 0) return PCL_OK;
    CHECK_ARG(Bpk != nullptr && (K == 0 || Bp != nullptr), "pcl_pack_b_vnni: NULL operand");
    CHECK_ARG((reinterpret_cast<uintptr_t>(Bp) & 3) == 0, "pcl_pack_b_vnni: Bp not 4-byte aligned");
    PCL_OK_OR_RETURN(do_init());
    HIP_OK(pcl::launch_pack_b_vnni(Bp, K, Kpad, N, Bpk, kpad256(K), colsum, pick(stream)));
    return PCL_OK;
}

static int check_i8_range(int K) {
    // |sum (a-128)*b| <= K * 128 * 128 must fit int32 (K <= 131071).
    if ((long long)K * 128 * 128 > 2147483647LL)
        return set_error(PCL_ERR_RANGE, "K=%d may overflow the int32 accumulator", K);
    return PCL_OK;
}

static int igemm_common(int out_mode, const uint8_t *A, int lda, const int8_t *Bpk,
                        const int32_t *col_off, const float *sa, const float *sb, void *C, int ldc,
                        int M, int N, int K, void *stream, const char *who) {
    CHECK_ARG(M >= 0 && N >= 0 && K >= 0, "%s: negative dimension (M=%d N=%d K=%d)", who, M, N, K);
    PCL_OK_OR_RETURN(check_i8_range(K));
    if (M == 0 || N == 0) return PCL_OK;
    CHECK_ARG(C && Bpk && (K == 0 || A), "%s: NULL operand", who);
    CHECK_ARG(ldc >= N, "%s: ldc=%d < N=%d", who, ldc, N);
    CHECK_ARG(K == 0 || lda >= K, "%s: lda=%d < K=%d", who, lda, K);
    CHECK_ARG(out_mode == 0 || sb, "%s: sb is NULL", who);
    CHECK_ARG(out_mode != 2 || sa, "%s: sa is NULL", who);
    CHECK_ARG(aligned16(Bpk), "%s: packed weights must be 16-byte aligned", who);
    PCL_OK_OR_RETURN(do_init());
    const long ldb = kpad256(K);
    hipStream_t s = pick(stream);
    // Decode rows: with 3-8 rows the matrix-core GEMV (one MFMA per 64 bytes
    // of 16 weight rows, coalesced loads) beats the dot-product kernel, whose
    // per-row work grows with M (3 rows run its 4-row form: +10% on the 350M
    // head); with 1-2 rows the dot-product kernel streams 2-4% faster.
    if (M >= 3 && M <= 8 && K > 0 && pcl::igemv_mfma_fits(M, N, K, ldb)) {
        HIP_OK(pcl::launch_igemv_mfma(out_mode, M, N, K, A, lda, Bpk, ldb, col_off, sa, sb, C, ldc, s));
        return PCL_OK;
    }
    if (M <= 8) {
        pcl::GemvPlan p = pcl::plan_igemv(M, N, K);
        ScratchLease sc;
        PCL_OK_OR_RETURN(get_scratch(s, p.part_bytes, 0, &sc));
        HIP_OK(pcl::launch_igemv(p, out_mode, M, N, K, A, lda, Bpk, ldb, col_off, sa, sb, C, ldc,
                                 sc->ws, s));
        return PCL_OK;
    }
    if (K % 256 == 0 && lda % 16 == 0 && aligned16(A)) {
        ScratchLease sc;  // the stream's tile counters
        PCL_OK_OR_RETURN(get_scratch(s, 0, 0, &sc));
        HIP_OK(pcl::launch_igemm(out_mode, M, N, K, A, lda, Bpk, ldb, col_off, sa, sb, C, ldc, sc->tiles, s));
        return PCL_OK;
    }
    // K not a multiple of 256 (the K tile granularity), or unaligned
    // activations: copy A into a Kp-wide buffer padded with 0x80 (zero after
    // re-centring; the packed weights are zero past K as well).
    const int Kp = (int)ldb;
    ScratchLease sc;
    PCL_OK_OR_RETURN(get_scratch(s, 0, (size_t)M * Kp, &sc));
    uint8_t *Ap = (uint8_t *)sc->aux;
    HIP_OK(pcl::launch_pad_a_u8(A, lda, M, K, Ap, Kp, s));
    HIP_OK(pcl::launch_igemm(out_mode, M, N, Kp, Ap, Kp, Bpk, ldb, col_off, sa, sb, C, ldc, sc->tiles, s));
    return PCL_OK;
}

int pcl_gemm_u8s8_i32(const uint8_t *A, int lda, const int8_t *Bpk, int32_t *C, int ldc, int M,
                      int N, int K, void *stream) {
    return igemm_common(0, A, lda, Bpk, nullptr, nullptr, nullptr, C, ldc, M, N, K, stream,
                        "pcl_gemm_u8s8_i32");
}

int pcl_gemm_u8s8_dq(const uint8_t *A, int lda, const int8_t *Bpk, const int32_t *col_off,
                     const float *sa, const float *sb, float *C, int ldc, int M, int N, int K,
                     void *stream) {
    return igemm_common(sa ? 2 : 1, A, lda, Bpk, col_off, sa, sb, C, ldc, M, N, K, stream,
                        "pcl_gemm_u8s8_dq");
}

int pcl_gemv_u8s8_i32(const uint8_t *X, int ldx, const int8_t *Bpk, int32_t *Y, int ldy, int M,
                      int N, int K, void *stream) {
    if (M > 8) return set_error(PCL_ERR_INVALID_ARG, "pcl_gemv_u8s8_i32: M=%d > 8", M);
    return igemm_common(0, X, ldx, Bpk, nullptr, nullptr, nullptr, Y, ldy, M, N, K, stream,
                        "pcl_gemv_u8s8_i32");
}

int pcl_gemv_u8s8_dq(const uint8_t *X, int ldx, const int8_t *Bpk, const int32_t *col_off,
                     const float *sa, const float *sb, float *Y, int ldy, int M, int N, int K,
                     void *stream) {
    if (M > 8) return set_error(PCL_ERR_INVALID_ARG, "pcl_gemv_u8s8_dq: M=%d > 8", M);
    return igemm_common(sa ? 2 : 1, X, ldx, Bpk, col_off, sa, sb, Y, ldy, M, N, K, stream,
                        "pcl_gemv_u8s8_dq");
}

int pcl_quantize_a_tensor(const float *A, int M, int K, uint8_t *Au, int Kpad, float *scale_dev,
                          void *stream) {
    CHECK_ARG(M >= 0 && K >= 0 && Kpad >= K, "pcl_quantize_a_tensor: bad dims (M=%d K=%d Kpad=%d)",
              M, K, Kpad);
    CHECK_ARG(Au && scale_dev && (M * (long)K == 0 || A), "pcl_quantize_a_tensor: NULL operand");
    PCL_OK_OR_RETURN(do_init());
    hipStream_t s = pick(stream);
    ScratchLease sc;
    PCL_OK_OR_RETURN(get_scratch(s, 0, 0, &sc));
    HIP_OK(pcl::launch_quantize_a_tensor(A, M, K, Au, Kpad, scale_dev, sc->amax, s));
    return PCL_OK;
}

int pcl_quantize_a_rows(const float *A, int M, int K, uint8_t *Au, int Kpad, float *sa,
                        void *stream) {
    CHECK_ARG(M >= 0 && K >= 0 && Kpad >= K, "pcl_quantize_a_rows: bad dims (M=%d K=%d Kpad=%d)",
              M, K, Kpad);
    if (M == 0) return PCL_OK;
    CHECK_ARG(Au && sa && (K == 0 || A), "pcl_quantize_a_rows: NULL operand");
    PCL_OK_OR_RETURN(do_init());
    HIP_OK(pcl::launch_quantize_a_rows(A, M, K, Au, Kpad, sa, pick(stream)));
    return PCL_OK;
}

int pcl_quantize_b_cols(const float *B, int K, int N, int8_t *Bpk, float *bscale, int32_t *colsum,
                        void *stream) {
    CHECK_ARG(K >= 0 && N >= 0, "pcl_quantize_b_cols: negative dimension");
    if (N == 0) return PCL_OK;
    CHECK_ARG(Bpk && bscale && (K == 0 || B), "pcl_quantize_b_cols: NULL operand");
    PCL_OK_OR_RETURN(do_init());
    HIP_OK(pcl::launch_quantize_b_cols(B, K, N, 0, Bpk, kpad256(K), 0, bscale, colsum, pick(stream)));
    return PCL_OK;
}

int pcl_quantize_b_vnni(const float *B, int K, int N, int Kpad, int8_t *Bp, float *bscale,
                        int32_t *colsum, void *stream) {
    CHECK_ARG(K >= 0 && N >= 0 && Kpad >= K && Kpad % 4 == 0,
              "pcl_quantize_b_vnni: need 0 <= K <= Kpad, Kpad %% 4 == 0");
    CHECK_ARG(N % 16 == 0, "pcl_quantize_b_vnni: N=%d is not a multiple of 16", N);
    if (N == 0) return PCL_OK;
    CHECK_ARG(Bp && bscale && (K == 0 || B), "pcl_quantize_b_vnni: NULL operand");
    PCL_OK_OR_RETURN(do_init());
    HIP_OK(pcl::launch_quantize_b_cols(B, K, N, 1, Bp, 0, Kpad, bscale, colsum, pick(stream)));
    return PCL_OK;
}

// ------------------------------------------------- device-pointer drop-ins ----
void gpu_init(void) { finish_void(pcl_init()); }

void gemm_nn(const float *A, const float *B, const float *bias, float *C, int M, int K, int N) {
    finish_void(pcl_sgemm(PCL_OP_N, PCL_OP_N, M, N, K, A, K, B, N, bias, 0, C, N, nullptr));
}
void gemm_nt(const float *A, const float *B, float *C, int M, int K, int N, int accum) {
    finish_void(pcl_sgemm(PCL_OP_N, PCL_OP_T, M, N, K, A, K, B, K, nullptr, accum ? 1 : 0, C, N,
                          nullptr));
}
void gemm_tn(const float *A, const float *B, float *C, int M, int K, int N) {
    finish_void(pcl_sgemm(PCL_OP_T, PCL_OP_N, K, N, M, A, K, B, N, nullptr, 1, C, N, nullptr));
}
void bias_bwd(float *db, const float *dY, int M, int N) {
    finish_void(pcl_bias_bwd(db, dY, M, N, N, nullptr));
}
void gelu_fwd(float *Y, const float *X, long n) { finish_void(pcl_gelu_fwd(Y, X, n, nullptr)); }
void gelu_bwd(float *dX, const float *dY, const float *X, long n) {
    finish_void(pcl_gelu_bwd(dX, dY, X, n, nullptr));
}
void vec_add(float *C, const float *A, const float *B, long n) {
    finish_void(pcl_vec_add(C, A, B, n, nullptr));
}

static int need_attn_dims(const char *who) {
    if (g_d_model <= 0 || g_attn_heads <= 0 || g_attn_batch <= 0)
        return set_error(PCL_ERR_UNSET_DIMS,
                         "%s: call pcl_set_model_dims and pcl_set_attn_dims first", who);
    // the head size is d_model / n_heads; a remainder would leave columns unread
    if (g_d_model % g_attn_heads != 0)
        return set_error(PCL_ERR_INVALID_ARG, "%s: d_model %d is not a multiple of n_heads %d", who,
                         g_d_model, g_attn_heads);
    return PCL_OK;
}

void attn_fwd(const float *Q, const float *K, const float *V, float *att, float *probs) {
    int st = need_attn_dims("attn_fwd");
    if (st == PCL_OK)
        st = pcl_attn_fwd(Q, K, V, g_d_model, att, g_d_model, probs, g_attn_batch, g_attn_seq,
                          g_attn_heads, g_d_model / g_attn_heads, nullptr);
    finish_void(st);
}

void attn_bwd(float *dQ, float *dK, float *dV, float *scratch, const float *dAtt, const float *Q,
              const float *K, const float *V, const float *probs) {
    int st = need_attn_dims("attn_bwd");
    if (st == PCL_OK)
        st = pcl_attn_bwd(dQ, dK, dV, g_d_model, scratch, dAtt, g_d_model, Q, K, V, g_d_model,
                          probs, g_attn_batch, g_attn_seq, g_attn_heads, g_d_model / g_attn_heads,
                          0, nullptr);
    finish_void(st);
}

// --------------------------------------------------- host-pointer drop-ins ----
// Slot numbers name the staging buffer each operand uses.
enum { S_A = 0, S_B, S_C, S_BIAS, S_D, S_E, S_F, S_G };

static int host_sgemm(int opA, int opB, int M, int N, int K, const float *A, const float *B,
                      const float *bias, int accumulate, float *C) {
    CHECK_ARG(M >= 0 && N >= 0 && K >= 0, "negative dimension (M=%d N=%d K=%d)", M, N, K);
    if (M == 0 || N == 0) return PCL_OK;
    CHECK_ARG(C && (K == 0 || (A && B)), "NULL operand");
    PCL_OK_OR_RETURN(do_init());
    void *dA, *dB, *dC, *dbias;
    PCL_OK_OR_RETURN(upload(S_A, K ? A : nullptr, sizeof(float) * (size_t)M * K, &dA));
    PCL_OK_OR_RETURN(upload(S_B, K ? B : nullptr, sizeof(float) * (size_t)K * N, &dB));
    PCL_OK_OR_RETURN(upload(S_BIAS, bias, sizeof(float) * (size_t)N, &dbias));
    if (accumulate) PCL_OK_OR_RETURN(upload(S_C, C, sizeof(float) * (size_t)M * N, &dC));
    else PCL_OK_OR_RETURN(stage_buf(S_C, sizeof(float) * (size_t)M * N, &dC));
    const int lda = opA == PCL_OP_N ? K : M, ldb = opB == PCL_OP_N ? N : K;
    PCL_OK_OR_RETURN(pcl_sgemm(opA, opB, M, N, K, (const float *)dA, lda, (const float *)dB, ldb,
                               (const float *)dbias, accumulate, (float *)dC, N, t_stream));
    PCL_OK_OR_RETURN(download(C, dC, sizeof(float) * (size_t)M * N));
    return sync_current();
}

void matmul(const float *A, const float *B, float *C, int M, int K, int N) {
    finish_void(host_sgemm(PCL_OP_N, PCL_OP_N, M, N, K, A, B, nullptr, 0, C));
}

void matmul_forward(float *out, const float *in, const float *Wt, const float *bias, int M, int K,
                    int N) {
    finish_void(host_sgemm(PCL_OP_N, PCL_OP_N, M, N, K, in, Wt, bias, 0, out));
}

static int host_matmul_backward(const float *dY, const float *X, const float *Wt, float *dX,
                                float *dW, float *db, int M, int K, int N) {
    CHECK_ARG(M >= 0 && N >= 0 && K >= 0, "matmul_backward: negative dimension");
    CHECK_ARG(dY && X && Wt && dX && dW, "matmul_backward: NULL operand");
    PCL_OK_OR_RETURN(do_init());
    void *ddY, *dXin, *dWt, *ddX, *ddW, *ddb;
    PCL_OK_OR_RETURN(upload(S_A, dY, sizeof(float) * (size_t)M * N, &ddY));
    PCL_OK_OR_RETURN(upload(S_B, X, sizeof(float) * (size_t)M * K, &dXin));
    PCL_OK_OR_RETURN(upload(S_D, Wt, sizeof(float) * (size_t)K * N, &dWt));
    PCL_OK_OR_RETURN(upload(S_C, dX, sizeof(float) * (size_t)M * K, &ddX));
    PCL_OK_OR_RETURN(upload(S_E, dW, sizeof(float) * (size_t)K * N, &ddW));
    PCL_OK_OR_RETURN(upload(S_BIAS, db, sizeof(float) * (size_t)N, &ddb));
    // dX(M,K) += dY(M,N) . W(K,N)^T      (train.c:221-232)
    PCL_OK_OR_RETURN(pcl_sgemm(PCL_OP_N, PCL_OP_T, M, K, N, (const float *)ddY, N,
                               (const float *)dWt, N, nullptr, 1, (float *)ddX, K, t_stream));
    // dW(K,N) += X(M,K)^T . dY(M,N)      (train.c:233-242)
    PCL_OK_OR_RETURN(pcl_sgemm(PCL_OP_T, PCL_OP_N, K, N, M, (const float *)dXin, K,
                               (const float *)ddY, N, nullptr, 1, (float *)ddW, N, t_stream));
    // db(N) += colsum(dY)                (train.c:243-251)
    if (db) PCL_OK_OR_RETURN(pcl_bias_bwd((float *)ddb, (const float *)ddY, M, N, N, t_stream));
    PCL_OK_OR_RETURN(download(dX, ddX, sizeof(float) * (size_t)M * K));
    PCL_OK_OR_RETURN(download(dW, ddW, sizeof(float) * (size_t)K * N));
    if (db) PCL_OK_OR_RETURN(download(db, ddb, sizeof(float) * (size_t)N));
    return sync_current();
}

void matmul_backward(const float *dY, const float *X, const float *Wt, float *dX, float *dW,
                     float *db, int M, int K, int N) {
    finish_void(host_matmul_backward(dY, X, Wt, dX, dW, db, M, K, N));
}

static int host_attention_forward(const float *q, const float *k, const float *v, float *att,
                                  float *probs, int B, int T) {
    PCL_OK_OR_RETURN(need_attn_dims("attention_forward"));
    CHECK_ARG(B >= 0 && T >= 0, "attention_forward: negative dimension (B=%d T=%d)", B, T);
    if (B == 0 || T == 0) return PCL_OK;
    CHECK_ARG(q && k && v && att && probs, "attention_forward: NULL operand");
    const int D = g_d_model, H = g_attn_heads;
    CHECK_ARG(D % H == 0, "attention_forward: d_model %d not divisible by %d heads", D, H);
    PCL_OK_OR_RETURN(do_init());
    const size_t act = sizeof(float) * (size_t)B * T * D, pb = sizeof(float) * (size_t)B * H * T * T;
    void *dq, *dk, *dv, *datt, *dp;
    PCL_OK_OR_RETURN(upload(S_A, q, act, &dq));
    PCL_OK_OR_RETURN(upload(S_B, k, act, &dk));
    PCL_OK_OR_RETURN(upload(S_D, v, act, &dv));
    PCL_OK_OR_RETURN(stage_buf(S_C, act, &datt));
    PCL_OK_OR_RETURN(stage_buf(S_E, pb, &dp));
    PCL_OK_OR_RETURN(pcl_attn_fwd((const float *)dq, (const float *)dk, (const float *)dv, D,
                                  (float *)datt, D, (float *)dp, B, T, H, D / H, t_stream));
    PCL_OK_OR_RETURN(download(att, datt, act));
    PCL_OK_OR_RETURN(download(probs, dp, pb));
    return sync_current();
}

void attention_forward(const float *q, const float *k, const float *v, float *att, float *probs,
                       int B, int T) {
    finish_void(host_attention_forward(q, k, v, att, probs, B, T));
}

static int host_attention_backward(float *dq, float *dk, float *dv, const float *d_att,
                                   const float *q, const float *k, const float *v,
                                   const float *probs, int B, int T) {
    PCL_OK_OR_RETURN(need_attn_dims("attention_backward"));
    CHECK_ARG(B >= 0 && T >= 0, "attention_backward: negative dimension (B=%d T=%d)", B, T);
    if (B == 0 || T == 0) return PCL_OK;
    CHECK_ARG(dq && dk && dv && d_att && q && k && v && probs, "attention_backward: NULL operand");
    const int D = g_d_model, H = g_attn_heads;
    CHECK_ARG(D % H == 0, "attention_backward: d_model %d not divisible by %d heads", D, H);
    PCL_OK_OR_RETURN(do_init());
    const size_t act = sizeof(float) * (size_t)B * T * D, pb = sizeof(float) * (size_t)B * H * T * T;
    void *ddq, *ddk, *ddv, *ddo, *dqin, *dkin, *dvin, *dp;
    PCL_OK_OR_RETURN(upload(S_A, q, act, &dqin));
    PCL_OK_OR_RETURN(upload(S_B, k, act, &dkin));
    PCL_OK_OR_RETURN(upload(S_D, v, act, &dvin));
    PCL_OK_OR_RETURN(upload(S_E, probs, pb, &dp));
    PCL_OK_OR_RETURN(upload(S_C, d_att, act, &ddo));
    PCL_OK_OR_RETURN(upload(S_F, dq, act, &ddq));
    PCL_OK_OR_RETURN(upload(S_G, dk, act, &ddk));
    PCL_OK_OR_RETURN(upload(S_BIAS, dv, act, &ddv));
    // train.c:374-407 accumulates into dq, dk, dv; dS goes to the library scratch
    PCL_OK_OR_RETURN(pcl_attn_bwd((float *)ddq, (float *)ddk, (float *)ddv, D, nullptr,
                                  (const float *)ddo, D, (const float *)dqin, (const float *)dkin,
                                  (const float *)dvin, D, (const float *)dp, B, T, H, D / H, 1,
                                  t_stream));
    PCL_OK_OR_RETURN(download(dq, ddq, act));
    PCL_OK_OR_RETURN(download(dk, ddk, act));
    PCL_OK_OR_RETURN(download(dv, ddv, act));
    return sync_current();
}

void attention_backward(float *dq, float *dk, float *dv, const float *d_att, const float *q,
                        const float *k, const float *v, const float *probs, int B, int T) {
    finish_void(host_attention_backward(dq, dk, dv, d_att, q, k, v, probs, B, T));
}

static int need_dims(const char *who) {
    if (g_d_model <= 0 || g_vocab <= 0)
        return set_error(PCL_ERR_UNSET_DIMS, "%s: call pcl_set_model_dims(d_model, vocab) first", who);
    return PCL_OK;
}

void tied_head_forward(float *logits, const float *lnf, const float *wte, int M) {
    int st = need_dims("tied_head_forward");
    if (st == PCL_OK) st = host_sgemm(PCL_OP_N, PCL_OP_T, M, g_vocab, g_d_model, lnf, wte, nullptr, 0, logits);
    finish_void(st);
}

static int host_tied_head_backward(float *d_lnf, float *dwte, const float *d_logits,
                                   const float *lnf, const float *wte, int M) {
    PCL_OK_OR_RETURN(need_dims("tied_head_backward"));
    PCL_OK_OR_RETURN(do_init());
    const int D = g_d_model, V = g_vocab;
    CHECK_ARG(M >= 0, "tied_head_backward: negative M");
    CHECK_ARG(d_lnf && dwte && d_logits && lnf && wte, "tied_head_backward: NULL operand");
    void *ddl, *dlnf, *dwt, *ddlnf, *ddwte;
    PCL_OK_OR_RETURN(upload(S_A, d_logits, sizeof(float) * (size_t)M * V, &ddl));
    PCL_OK_OR_RETURN(upload(S_B, lnf, sizeof(float) * (size_t)M * D, &dlnf));
    PCL_OK_OR_RETURN(upload(S_D, wte, sizeof(float) * (size_t)V * D, &dwt));
    PCL_OK_OR_RETURN(stage_buf(S_C, sizeof(float) * (size_t)M * D, &ddlnf));
    PCL_OK_OR_RETURN(upload(S_E, dwte, sizeof(float) * (size_t)V * D, &ddwte));
    // d_lnf(M,D) = d_logits(M,V) . wte(V,D)        (train.c:426-435, SET)
    PCL_OK_OR_RETURN(pcl_sgemm(PCL_OP_N, PCL_OP_N, M, D, V, (const float *)ddl, V,
                               (const float *)dwt, D, nullptr, 0, (float *)ddlnf, D, t_stream));
    // dwte(V,D) += d_logits(M,V)^T . lnf(M,D)      (train.c:436-446)
    PCL_OK_OR_RETURN(pcl_sgemm(PCL_OP_T, PCL_OP_N, V, D, M, (const float *)ddl, V,
                               (const float *)dlnf, D, nullptr, 1, (float *)ddwte, D, t_stream));
    PCL_OK_OR_RETURN(download(d_lnf, ddlnf, sizeof(float) * (size_t)M * D));
    PCL_OK_OR_RETURN(download(dwte, ddwte, sizeof(float) * (size_t)V * D));
    return sync_current();
}

void tied_head_backward(float *d_lnf, float *dwte, const float *d_logits, const float *lnf,
                        const float *wte, int M) {
    finish_void(host_tied_head_backward(d_lnf, dwte, d_logits, lnf, wte, M));
}

void lm_head(float *logits, const float *x, const float *wte, int num_tokens) {
    int st = need_dims("lm_head");
    if (st == PCL_OK)
        st = host_sgemm(PCL_OP_N, PCL_OP_T, num_tokens, g_vocab, g_d_model, x, wte, nullptr, 0, logits);
    finish_void(st);
}

void proj_token(float *out, const float *in, const float *W, const float *bias, int K, int N) {
    finish_void(host_sgemm(PCL_OP_N, PCL_OP_N, 1, N, K, in, W, bias, 0, out));
}

void matvec(float *out, const float *x, const float *W, const float *b, int K, int N) {
    finish_void(host_sgemm(PCL_OP_N, PCL_OP_N, 1, N, K, x, W, b, 0, out));
}

static int host_quantize_A(const float *A, uint8_t *Au, int M, int K, int Kpad, float *scale) {
    CHECK_ARG(M >= 0 && K >= 0 && Kpad >= K, "quantize_A: bad dims (M=%d K=%d Kpad=%d)", M, K, Kpad);
    CHECK_ARG(Au && (M * (long)K == 0 || A), "quantize_A: NULL operand");
    PCL_OK_OR_RETURN(do_init());
    void *dA, *dAu, *dS;
    PCL_OK_OR_RETURN(upload(S_A, A, sizeof(float) * (size_t)M * K, &dA));
    PCL_OK_OR_RETURN(stage_buf(S_B, (size_t)M * Kpad, &dAu));
    PCL_OK_OR_RETURN(stage_buf(S_D, sizeof(float), &dS));
    PCL_OK_OR_RETURN(pcl_quantize_a_tensor((const float *)dA, M, K, (uint8_t *)dAu, Kpad,
                                           (float *)dS, t_stream));
    PCL_OK_OR_RETURN(download(Au, dAu, (size_t)M * Kpad));
    PCL_OK_OR_RETURN(download(scale, dS, sizeof(float)));
    return sync_current();
}

float quantize_A(const float *A, uint8_t *Au, int M, int K, int Kpad) {
    float scale = NAN;
    finish_void(host_quantize_A(A, Au, M, K, Kpad, &scale));
    return scale;
}

static int host_quantize_B_pack(const float *B, int8_t *Bp, float *bscale, int32_t *colsum, int K,
                                int N, int Kpad) {
    CHECK_ARG(B && Bp && bscale && colsum, "quantize_B_pack: NULL operand");
    CHECK_ARG(N >= 0 && N % 16 == 0, "quantize_B_pack: N=%d is not a multiple of 16", N);
    CHECK_ARG(K >= 0 && Kpad >= K && Kpad % 4 == 0, "quantize_B_pack: bad K=%d Kpad=%d", K, Kpad);
    PCL_OK_OR_RETURN(do_init());
    const size_t bp_bytes = (size_t)(N / 16) * (Kpad / 4) * 64;
    void *dB, *dBp, *dsc, *dcs;
    PCL_OK_OR_RETURN(upload(S_A, B, sizeof(float) * (size_t)K * N, &dB));
    PCL_OK_OR_RETURN(stage_buf(S_B, bp_bytes, &dBp));
    PCL_OK_OR_RETURN(stage_buf(S_D, sizeof(float) * (size_t)N, &dsc));
    PCL_OK_OR_RETURN(stage_buf(S_E, sizeof(int32_t) * (size_t)N, &dcs));
    PCL_OK_OR_RETURN(pcl_quantize_b_vnni((const float *)dB, K, N, Kpad, (int8_t *)dBp,
                                         (float *)dsc, (int32_t *)dcs, t_stream));
    PCL_OK_OR_RETURN(download(Bp, dBp, bp_bytes));
    PCL_OK_OR_RETURN(download(bscale, dsc, sizeof(float) * (size_t)N));
    PCL_OK_OR_RETURN(download(colsum, dcs, sizeof(int32_t) * (size_t)N));
    return sync_current();
}

void quantize_B_pack(const float *B, int8_t *Bp, float *bscale, int32_t *colsum, int K, int N,
                     int Kpad) {
    finish_void(host_quantize_B_pack(B, Bp, bscale, colsum, K, N, Kpad));
}

static int host_gemm_int8_kernel(const uint8_t *Au, int Kpad, const int8_t *Bp,
                                 const int32_t *corr, const float *dq, float *C, int M, int N) {
    CHECK_ARG(M >= 0 && N >= 0 && Kpad >= 0 && Kpad % 4 == 0,
              "gemm_int8_kernel: bad dims (M=%d N=%d Kpad=%d)", M, N, Kpad);
    CHECK_ARG(N % 16 == 0, "gemm_int8_kernel: N=%d is not a multiple of 16", N);
    if (M == 0 || N == 0) return PCL_OK;
    CHECK_ARG(Au && Bp && corr && dq && C, "gemm_int8_kernel: NULL operand");
    PCL_OK_OR_RETURN(do_init());
    const int K = Kpad;  // the reference kernel runs over all Kpad bytes
    const size_t bp_bytes = (size_t)(N / 16) * (Kpad / 4) * 64;
    void *dAu, *dBp, *dcorr, *ddq, *dC, *dBpk, *dcs, *doff;
    PCL_OK_OR_RETURN(upload(S_A, Au, (size_t)M * Kpad, &dAu));
    PCL_OK_OR_RETURN(upload(S_B, Bp, bp_bytes, &dBp));
    PCL_OK_OR_RETURN(upload(S_D, corr, sizeof(int32_t) * (size_t)N, &dcorr));
    PCL_OK_OR_RETURN(upload(S_BIAS, dq, sizeof(float) * (size_t)N, &ddq));
    PCL_OK_OR_RETURN(stage_buf(S_C, sizeof(float) * (size_t)M * N, &dC));
    PCL_OK_OR_RETURN(stage_buf(S_E, pcl_s8_packed_bytes(K, N), &dBpk));
    PCL_OK_OR_RETURN(stage_buf(S_F, sizeof(int32_t) * (size_t)N, &dcs));
    PCL_OK_OR_RETURN(stage_buf(S_G, sizeof(int32_t) * (size_t)N, &doff));
    PCL_OK_OR_RETURN(pcl_pack_b_vnni((const int8_t *)dBp, K, Kpad, N, (int8_t *)dBpk,
                                     (int32_t *)dcs, t_stream));
    HIP_OK(pcl::launch_corr_to_offset((const int32_t *)dcs, (const int32_t *)dcorr,
                                      (int32_t *)doff, N, t_stream));
    PCL_OK_OR_RETURN(pcl_gemm_u8s8_dq((const uint8_t *)dAu, Kpad, (const int8_t *)dBpk,
                                      (const int32_t *)doff, nullptr, (const float *)ddq,
                                      (float *)dC, N, M, N, K, t_stream));
    PCL_OK_OR_RETURN(download(C, dC, sizeof(float) * (size_t)M * N));
    return sync_current();
}

void gemm_int8_kernel(const uint8_t *Au, int Kpad, const int8_t *Bp, const int32_t *corr,
                      const float *dq, float *C, int M, int N) {
    finish_void(host_gemm_int8_kernel(Au, Kpad, Bp, corr, dq, C, M, N));
}

// ------------------------------------------------------ cross-entropy ----
int pcl_cross_entropy(const float *logits, int ld, const int *targets, float *dlogits, int ldd,
                      int M, int V, float *loss, void *stream) {
    CHECK_ARG(M >= 0 && V > 0, "pcl_cross_entropy: bad dims (M=%d V=%d)", M, V);
    if (M == 0) return PCL_OK;
    CHECK_ARG(logits && targets && dlogits && loss, "pcl_cross_entropy: NULL operand");
    CHECK_ARG(ld >= V && ldd >= V, "pcl_cross_entropy: ld=%d, ldd=%d below V=%d", ld, ldd, V);
    const size_t nl = sizeof(float) * ((size_t)(M - 1) * ld + V);
    const size_t nd = sizeof(float) * ((size_t)(M - 1) * ldd + V);
    CHECK_ARG(!ranges_overlap(logits, nl, dlogits, nd) || (logits == dlogits && ld == ldd),
              "pcl_cross_entropy: dlogits overlaps logits other than in place");
    PCL_OK_OR_RETURN(do_init());
    hipStream_t s = pick(stream);
    ScratchLease sc;
    PCL_OK_OR_RETURN(get_scratch(s, 0, sizeof(double) * (size_t)M, &sc));
    double *rl = static_cast<double *>(sc->aux);
    HIP_OK(pcl::launch_cross_entropy(logits, ld, targets, dlogits, ldd, M, V, V, M, rl, s));
    HIP_OK(pcl::launch_ce_loss(rl, M, M, loss, s));
    return PCL_OK;
}

int pcl_head_ce(const float *lnf, const float *wte, const int *targets, int M, int D, int V,
                float *loss, float *d_lnf, float *dwte, long chunk_bytes, void *stream) {
    CHECK_ARG(M >= 0 && D > 0 && V > 0, "pcl_head_ce: bad dims (M=%d D=%d V=%d)", M, D, V);
    if (M == 0) return PCL_OK;
    CHECK_ARG(lnf && wte && targets && loss, "pcl_head_ce: NULL operand");
    PCL_OK_OR_RETURN(do_init());
    hipStream_t s = pick(stream);
    // logits rows padded to 64 floats: 256-byte aligned rows, and a product
    // over the first V - V % 64 vocabulary entries has K (or M) a multiple of 64
    const long ldp = (V + 63) / 64 * 64, row_bytes = ldp * (long)sizeof(float);
    const long cap = chunk_bytes > 0 ? chunk_bytes : (1L << 30);
    long mc = cap / row_bytes;
    if (mc < 1) mc = 1;
    if (mc > M) mc = M;
    if (mc > 128) mc = mc / 128 * 128;
    const size_t loss_off = ((size_t)mc * row_bytes + 255) / 256 * 256;
    ScratchLease sc;
    PCL_OK_OR_RETURN(get_scratch(s, 0, loss_off + sizeof(double) * (size_t)M, &sc));
    float *lg = static_cast<float *>(sc->aux);
    double *rl = reinterpret_cast<double *>(static_cast<char *>(sc->aux) + loss_off);
    const int Vm = V / 64 * 64, Vr = V - Vm, L = (int)ldp;
    for (int m0 = 0; m0 < M; m0 += (int)mc) {
        const int mm = (int)(M - m0 < mc ? M - m0 : mc);
        const float *x = lnf + (size_t)m0 * D;
        // train.c:412-423 on the chunk, then :449-465 in place
        PCL_OK_OR_RETURN(pcl_sgemm(PCL_OP_N, PCL_OP_T, mm, V, D, x, D, wte, D, nullptr, 0, lg, L, s));
        HIP_OK(pcl::launch_cross_entropy(lg, ldp, targets + m0, lg, ldp, mm, V, L, M, rl + m0, s));
        if (d_lnf) {  // train.c:426-435 (set): K = V in two parts
            float *dx = d_lnf + (size_t)m0 * D;
            PCL_OK_OR_RETURN(pcl_sgemm(PCL_OP_N, PCL_OP_N, mm, D, Vm, lg, L, wte, D, nullptr, 0, dx, D, s));
            if (Vr)
                PCL_OK_OR_RETURN(pcl_sgemm(PCL_OP_N, PCL_OP_N, mm, D, Vr, lg + Vm, L, wte + (size_t)Vm * D,
                                           D, nullptr, 1, dx, D, s));
        }
        if (dwte) {  // train.c:436-446 (accumulate): vocabulary rows in two parts
            if (Vm)
                PCL_OK_OR_RETURN(pcl_sgemm(PCL_OP_T, PCL_OP_N, Vm, D, mm, lg, L, x, D, nullptr, 1, dwte, D, s));
            if (Vr)
                PCL_OK_OR_RETURN(pcl_sgemm(PCL_OP_T, PCL_OP_N, Vr, D, mm, lg + Vm, L, x, D, nullptr, 1,
                                           dwte + (size_t)Vm * D, D, s));
        }
    }
    HIP_OK(pcl::launch_ce_loss(rl, M, M, loss, s));
    return PCL_OK;
}

// gpu_kernels.h:78-81: M_ROWS = B_SIZE * T_SIZE rows of VOCAB_SIZE logits
void ce_fwd_bwd(const float *logits, const int *targets, float *dlogits, float *loss_dev) {
    int st = PCL_OK;
    if (g_vocab <= 0 || g_attn_batch <= 0 || g_attn_seq <= 0)
        st = set_error(PCL_ERR_UNSET_DIMS,
                       "ce_fwd_bwd: call pcl_set_model_dims and pcl_set_attn_dims first");
    if (st == PCL_OK)
        st = pcl_cross_entropy(logits, g_vocab, targets, dlogits, g_vocab, g_attn_batch * g_attn_seq,
                               g_vocab, loss_dev, nullptr);
    finish_void(st);
}

// train.c:449-465 on host buffers: returns the mean loss, fills d_logits
static int host_cross_entropy(const float *logits, const int *targets, float *d_logits, int M,
                              float *out) {
    if (g_vocab <= 0)
        return set_error(PCL_ERR_UNSET_DIMS, "cross_entropy: call pcl_set_model_dims first");
    CHECK_ARG(M >= 0, "cross_entropy: negative M=%d", M);
    *out = 0.f;
    if (M == 0) return PCL_OK;
    CHECK_ARG(logits && targets && d_logits, "cross_entropy: NULL operand");
    PCL_OK_OR_RETURN(do_init());
    const int V = g_vocab;
    const size_t lb = sizeof(float) * (size_t)M * V;
    void *dl, *dt, *dd, *dloss;
    PCL_OK_OR_RETURN(upload(S_A, logits, lb, &dl));
    PCL_OK_OR_RETURN(upload(S_B, targets, sizeof(int) * (size_t)M, &dt));
    PCL_OK_OR_RETURN(stage_buf(S_C, lb, &dd));
    static const float zero = 0.f;  // the loss is added into this slot
    PCL_OK_OR_RETURN(upload(S_D, &zero, sizeof(float), &dloss));
    PCL_OK_OR_RETURN(pcl_cross_entropy((const float *)dl, V, (const int *)dt, (float *)dd, V, M, V,
                                       (float *)dloss, t_stream));
    PCL_OK_OR_RETURN(download(d_logits, dd, lb));
    PCL_OK_OR_RETURN(download(out, dloss, sizeof(float)));
    return sync_current();
}

float cross_entropy(const float *logits, const int *targets, float *d_logits, int M) {
    float loss = 0.f;
    finish_void(host_cross_entropy(logits, targets, d_logits, M, &loss));
    return loss;
}

}  // extern "C"
