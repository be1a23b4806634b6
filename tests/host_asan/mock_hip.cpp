// mock_hip.cpp -- a host-only stand-in for the HIP runtime and for the
// library's kernel launchers, so the C-ABI shim (pcl_hip.cpp) and the bench
// harness run on a CPU under AddressSanitizer / UndefinedBehaviorSanitizer.
// Test infrastructure only: it computes nothing. "Device" memory is host heap
// memory (malloc/free, so the sanitizer sees every buffer), copies are memcpy,
// streams and graphs are small heap objects, and each launcher writes every
// byte of the buffers it is handed (outputs, workspaces, realigned copies),
// so a buffer that is freed, or smaller than the launch needs, is reported.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <set>

#include "../../pure-c-llm_amd/csrc/internal.h"

namespace {
std::mutex mu;
std::set<void *> live;  // hipMalloc'd blocks
struct Stream { int capturing = 0; };
struct Graph { int nodes = 0; };
void touch(void *p, size_t n) {
    if (p && n) memset(p, 0x5a, n);
}
}  // namespace

extern "C" {
hipError_t hipMalloc(void **p, size_t n) {
    *p = malloc(n ? n : 1);
    if (!*p) return hipErrorOutOfMemory;
    std::lock_guard<std::mutex> lk(mu);
    live.insert(*p);
    return hipSuccess;
}
hipError_t hipFree(void *p) {
    if (!p) return hipSuccess;
    {
        std::lock_guard<std::mutex> lk(mu);
        if (!live.erase(p)) {
            fprintf(stderr, "mock hipFree: %p is not a live allocation\n", p);
            abort();
        }
    }
    free(p);
    return hipSuccess;
}
hipError_t hipMemcpy(void *d, const void *s, size_t n, hipMemcpyKind) { memmove(d, s, n); return hipSuccess; }
hipError_t hipMemcpyAsync(void *d, const void *s, size_t n, hipMemcpyKind, hipStream_t) { memmove(d, s, n); return hipSuccess; }
hipError_t hipMemset(void *d, int v, size_t n) { memset(d, v, n); return hipSuccess; }
hipError_t hipGetDeviceCount(int *n) { *n = 1; return hipSuccess; }
hipError_t hipGetDevice(int *d) { *d = 0; return hipSuccess; }
hipError_t hipGetDevicePropertiesR0600(hipDeviceProp_tR0600 *p, int) {
    memset(p, 0, sizeof *p);
    strcpy(p->name, "mock");
    strcpy(p->gcnArchName, "gfx950:sramecc+:xnack-");
    p->multiProcessorCount = 256;
    p->clockRate = 2400000;
    return hipSuccess;
}
hipError_t hipDeviceGetAttribute(int *v, hipDeviceAttribute_t, int) { *v = 256; return hipSuccess; }
const char *hipGetErrorString(hipError_t) { return "mock error"; }
hipError_t hipGetLastError(void) { return hipSuccess; }
hipError_t hipStreamCreateWithFlags(hipStream_t *s, unsigned) {
    *s = reinterpret_cast<hipStream_t>(new Stream);
    return hipSuccess;
}
hipError_t hipStreamDestroy(hipStream_t s) { delete reinterpret_cast<Stream *>(s); return hipSuccess; }
hipError_t hipStreamSynchronize(hipStream_t) { return hipSuccess; }
hipError_t hipStreamBeginCapture(hipStream_t s, hipStreamCaptureMode) {
    if (!s) return hipErrorInvalidValue;
    reinterpret_cast<Stream *>(s)->capturing = 1;
    return hipSuccess;
}
hipError_t hipStreamEndCapture(hipStream_t s, hipGraph_t *g) {
    if (!s || !reinterpret_cast<Stream *>(s)->capturing) return hipErrorInvalidValue;
    reinterpret_cast<Stream *>(s)->capturing = 0;
    *g = reinterpret_cast<hipGraph_t>(new Graph);
    return hipSuccess;
}
hipError_t hipStreamIsCapturing(hipStream_t s, hipStreamCaptureStatus *cs) {
    *cs = s && reinterpret_cast<Stream *>(s)->capturing ? hipStreamCaptureStatusActive : hipStreamCaptureStatusNone;
    return hipSuccess;
}
hipError_t hipGraphInstantiate(hipGraphExec_t *e, hipGraph_t, hipGraphNode_t *, char *, size_t) {
    *e = reinterpret_cast<hipGraphExec_t>(new Graph);
    return hipSuccess;
}
hipError_t hipGraphDestroy(hipGraph_t g) { delete reinterpret_cast<Graph *>(g); return hipSuccess; }
hipError_t hipGraphExecDestroy(hipGraphExec_t g) { delete reinterpret_cast<Graph *>(g); return hipSuccess; }
hipError_t hipGraphLaunch(hipGraphExec_t, hipStream_t) { return hipSuccess; }
hipError_t hipEventCreate(hipEvent_t *e) { *e = reinterpret_cast<hipEvent_t>(new int(0)); return hipSuccess; }
hipError_t hipEventDestroy(hipEvent_t e) { delete reinterpret_cast<int *>(e); return hipSuccess; }
hipError_t hipEventRecord(hipEvent_t, hipStream_t) { return hipSuccess; }
hipError_t hipEventSynchronize(hipEvent_t) { return hipSuccess; }
hipError_t hipEventElapsedTime(float *ms, hipEvent_t, hipEvent_t) { *ms = 1.0f; return hipSuccess; }
}  // extern "C"

// ---- the library's launchers: plans of plausible size, buffers written whole
namespace pcl {
namespace {
size_t cdiv(size_t a, size_t b) { return (a + b - 1) / b; }
void out2(void *C, long ld, int rows, int cols, size_t esz) {
    if (rows > 0 && cols > 0) touch(C, ((size_t)(rows - 1) * ld + cols) * esz);
}
}  // namespace
SgemmPlan plan_sgemm(int M, int N, int K, bool) {
    SgemmPlan p{0, 1, K, 0};
    if ((long)M * N < 65536 && K >= 1024) {  // small grids split K
        p.splits = 4;
        p.kchunk = (int)cdiv(K, 4);
        p.part_bytes = (size_t)4 * M * N * 4;
    }
    return p;
}
hipError_t launch_sgemm(const SgemmPlan &p, bool, bool, int M, int N, int, const float *, long, const float *,
                        long, const float *, int, float *C, long ldc, const Workspace &ws, hipStream_t, int,
                        const float *, float *aux_out, long ld_aux) {
    if (p.part_bytes > ws.bytes_cap) return hipErrorInvalidValue;
    touch(ws.buf, p.part_bytes);
    out2(C, ldc, M, N, 4);
    if (aux_out) out2(aux_out, ld_aux, M, N, 4);
    return hipSuccess;
}
hipError_t launch_copy_rows(float *dst, long ldd, const float *, long, int rows, int cols, hipStream_t) {
    out2(dst, ldd, rows, cols, 4);
    return hipSuccess;
}
hipError_t launch_elementwise(int, long n, float *out, const float *, const float *, hipStream_t) {
    touch(out, (size_t)n * 4);
    return hipSuccess;
}
hipError_t launch_igemm(int out_mode, int M, int N, int, const uint8_t *, long, const int8_t *, long,
                        const int32_t *, const float *, const float *, void *C, long ldc, int *tile_ctr,
                        hipStream_t) {
    (void)out_mode;
    if (tile_ctr) touch(tile_ctr, IGEMM_TILE_CTRS * sizeof(int));
    out2(C, ldc, M, N, 4);
    return hipSuccess;
}
hipError_t launch_igemm_tiles_init(int *ctr, hipStream_t) {
    touch(ctr, IGEMM_TILE_CTRS * sizeof(int));
    return hipSuccess;
}
hipError_t launch_pad_a_u8(const uint8_t *, long, int M, int, uint8_t *dst, int Kd, hipStream_t) {
    touch(dst, (size_t)M * Kd);
    return hipSuccess;
}
hipError_t launch_attn_fwd(const float *, const float *, const float *, long, float *O, long ldo, float *P, int B,
                           int T, int H, int dh, float, hipStream_t, float *lse) {
    out2(O, ldo, B * T, H * dh, 4);
    if (P) touch(P, (size_t)B * H * T * T * 4);
    if (lse) touch(lse, (size_t)B * H * T * 4);
    return hipSuccess;
}
hipError_t launch_attn_bwd(const float *, long, const float *, const float *, const float *, long, const float *,
                           float *dS, float *dQ, float *dK, float *dV, long ldg, int B, int T, int H, int dh, float,
                           int, hipStream_t, const float *, long) {
    touch(dS, (size_t)B * H * T * T * 4);
    out2(dQ, ldg, B * T, H * dh, 4);
    out2(dK, ldg, B * T, H * dh, 4);
    out2(dV, ldg, B * T, H * dh, 4);
    return hipSuccess;
}
hipError_t launch_cross_entropy(const float *, long, const int *, float *dl, long ldd, int M, int, int pad, int,
                                double *row_loss, hipStream_t) {
    out2(dl, ldd, M, pad, 4);
    touch(row_loss, (size_t)M * 8);
    return hipSuccess;
}
hipError_t launch_ce_loss(const double *, int, int, float *loss, hipStream_t) {
    *loss += 1.0f;
    return hipSuccess;
}
hipError_t measure_peak_mfma(int, int, double *rate, hipStream_t) { *rate = 1; return hipSuccess; }
hipError_t measure_bandwidth(long, double gbs[4], hipStream_t) { gbs[0] = gbs[1] = gbs[2] = gbs[3] = 1; return hipSuccess; }
hipError_t measure_lds_feed(int, int, int, double *gbs, hipStream_t, bool) { *gbs = 1; return hipSuccess; }
GemvPlan plan_sgemv(int, int M, int N, int K) {
    GemvPlan p{(int)cdiv(N, 64), 1, K, 0, 64};
    if (K > 1024) {
        p.splits = (int)cdiv(K, 1024);
        p.kchunk = 1024;
        p.part_bytes = (size_t)p.splits * M * N * 4;
    }
    return p;
}
int gg_strip_rows(int kind) { return kind == GG_U8S8 ? 64 : 32; }
int gg_stage_ld(int, int K) { return (K + 255) / 256 * 256 + 16; }
size_t gg_lds_bytes(int, int K, int mr) { return (size_t)mr * ((K + 63) / 64 * 64) * 4; }
hipError_t launch_gemv_group(const GgDesc *, int, int, size_t, bool, hipStream_t) { return hipSuccess; }
bool igemv_mfma_fits(int M, int, int, long) { return M >= 3; }
hipError_t launch_igemv_mfma(int, int M, int N, int, const uint8_t *, long, const int8_t *, long, const int32_t *,
                             const float *, const float *, void *Y, long ldy, hipStream_t) {
    out2(Y, ldy, M, N, 4);
    return hipSuccess;
}
hipError_t gemv_noalloc_scratch(void **p) {
    static char *buf = (char *)malloc(GEMV_NOALLOC_SCRATCH_BYTES);
    *p = buf;
    return hipSuccess;
}
GemvPlan plan_bias_bwd(int N, int K) { return plan_sgemv(0, 1, N, K); }
GemvPlan plan_igemv(int M, int N, int K) { return plan_sgemv(0, M, N, K); }
hipError_t launch_sgemv(const GemvPlan &p, int, int M, int N, int, const float *, long, bool, const float *, long,
                        const float *, int, float *Y, long ldy, const Workspace &ws, hipStream_t) {
    if (p.part_bytes > ws.bytes_cap) return hipErrorInvalidValue;
    touch(ws.buf, p.part_bytes);
    out2(Y, ldy, M, N, 4);
    return hipSuccess;
}
hipError_t launch_sgemv_xf(const GemvPlan &p, int, int N, int, const float *, const float *, long, const float *,
                           const float *, const float *, int, float *Y, const Workspace &ws, hipStream_t) {
    if (p.part_bytes > ws.bytes_cap) return hipErrorInvalidValue;
    touch(ws.buf, p.part_bytes);
    touch(Y, (size_t)N * 4);
    return hipSuccess;
}
hipError_t launch_igemv(const GemvPlan &p, int, int M, int N, int, const uint8_t *, long, const int8_t *, long,
                        const int32_t *, const float *, const float *, void *Y, long ldy, const Workspace &ws,
                        hipStream_t) {
    if (p.part_bytes > ws.bytes_cap) return hipErrorInvalidValue;
    touch(ws.buf, p.part_bytes);
    out2(Y, ldy, M, N, 4);
    return hipSuccess;
}
hipError_t launch_quantize_a_tensor(const float *, int M, int, uint8_t *Au, int Kpad, float *scale, unsigned *amax,
                                    hipStream_t) {
    touch(Au, (size_t)M * Kpad);
    *scale = 1.0f;
    *amax = 0;
    return hipSuccess;
}
hipError_t launch_quantize_a_rows(const float *, int M, int, uint8_t *Au, int Kpad, float *sa, hipStream_t) {
    touch(Au, (size_t)M * Kpad);
    touch(sa, (size_t)M * 4);
    return hipSuccess;
}
hipError_t launch_quantize_b_cols(const float *, int, int N, int, int8_t *dst, long ldb, int Kpad, float *bscale,
                                  int32_t *colsum, hipStream_t) {
    touch(dst, (size_t)N * (ldb > Kpad ? ldb : Kpad));
    touch(bscale, (size_t)N * 4);
    if (colsum) touch(colsum, (size_t)N * 4);
    return hipSuccess;
}
hipError_t launch_pack_b_s8(const int8_t *, long, int, int N, int8_t *Bpk, long ldb, int32_t *colsum, hipStream_t) {
    touch(Bpk, (size_t)N * ldb);
    if (colsum) touch(colsum, (size_t)N * 4);
    return hipSuccess;
}
hipError_t launch_pack_b_vnni(const int8_t *, int, int, int N, int8_t *Bpk, long ldb, int32_t *colsum, hipStream_t) {
    touch(Bpk, (size_t)N * ldb);
    if (colsum) touch(colsum, (size_t)N * 4);
    return hipSuccess;
}
hipError_t launch_corr_to_offset(const int32_t *, const int32_t *, int32_t *off, int N, hipStream_t) {
    touch(off, (size_t)N * 4);
    return hipSuccess;
}
}  // namespace pcl
