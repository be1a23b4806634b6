// ce.hip -- softmax cross-entropy over rows of logits (train.c:449-465,
// gpu_kernels.cu:518-547): per row m with target t,
//   p[v] = expf(l[v] - max) * (1 / sum_v expf(l[v] - max)),
//   loss_m = -log((double)p[t] + 1e-30),  dl[v] = (p[v] - [v == t]) / M.
//
// One workgroup per row, two passes over the row in HBM (16-byte accesses over
// the row's aligned middle): the first keeps a
// running (max, sum) per thread (the sum rescaled whenever the max grows), the
// second writes dl. dl may alias the logits (each element is read before the
// same thread overwrites it). Row losses go to a double array; a second kernel
// adds their mean, summed in a fixed order, into *loss. Columns [V, pad) of dl
// are written as zeros so a padded dl can feed K-padded products.
#include "internal.h"

namespace pcl {
namespace {

constexpr int CE_NT = 512;  // 8 waves per row

// (m, s) += x: s holds sum exp(x_i - m). NaN logits propagate into s; -inf
// logits add nothing.
__device__ __forceinline__ void ce_push(float &m, float &s, float x) {
    const float d = x - m;
    if (d > 0.f) {
        s = s * expf(-d) + 1.f;
        m = x;
    } else if (x != -INFINITY) {
        s += expf(d);
    }
}

__device__ __forceinline__ void ce_merge(float &m, float &s, float m2, float s2) {
    if (s2 == 0.f) return;
    if (s == 0.f) {
        m = m2, s = s2;
        return;
    }
    if (m2 > m) {
        s = s * expf(m - m2) + s2;
        m = m2;
    } else {
        s += s2 * expf(m2 - m);
    }
}

__global__ __launch_bounds__(CE_NT) void ce_rows_kernel(const float *logits, long ld,
                                                        const int *__restrict__ targets, float *dl,
                                                        long ldd, int V, int pad, float rows,
                                                        double *__restrict__ row_loss) {
    typedef float v4f_t __attribute__((ext_vector_type(4)));
    __shared__ float sm_m[CE_NT / 64], sm_s[CE_NT / 64];
    const int tid = threadIdx.x, row = blockIdx.x;
    const float *x = logits + (long)row * ld;
    float *o = dl + (long)row * ldd;
    // Rows are read (and written) as 16-byte vectors between a scalar head (up
    // to the first 16-byte boundary) and a scalar tail, when the dlogits row
    // has the same alignment as the logits row; otherwise element by element.
    const bool vec = ((reinterpret_cast<uintptr_t>(x) ^ reinterpret_cast<uintptr_t>(o)) & 15) == 0;
    const int head = vec ? min(V, (int)((16 - (reinterpret_cast<uintptr_t>(x) & 15)) & 15) / 4) : V;
    const int nv = vec ? (V - head) / 4 : 0;
    const int tail0 = head + 4 * nv;
    const v4f_t *x4 = reinterpret_cast<const v4f_t *>(x + head);
    float m = -INFINITY, s = 0.f;
    if (vec) {
        if (tid < head) ce_push(m, s, x[tid]);
        int c = tid;
        for (; c + CE_NT < nv; c += 2 * CE_NT) {
            const v4f_t a = x4[c], b = x4[c + CE_NT];
            ce_push(m, s, a[0]), ce_push(m, s, a[1]), ce_push(m, s, a[2]), ce_push(m, s, a[3]);
            ce_push(m, s, b[0]), ce_push(m, s, b[1]), ce_push(m, s, b[2]), ce_push(m, s, b[3]);
        }
        for (; c < nv; c += CE_NT) {
            const v4f_t a = x4[c];
            ce_push(m, s, a[0]), ce_push(m, s, a[1]), ce_push(m, s, a[2]), ce_push(m, s, a[3]);
        }
        for (int v = tail0 + tid; v < V; v += CE_NT) ce_push(m, s, x[v]);
    } else {
        int v = tid;
        for (; v + 3 * CE_NT < V; v += 4 * CE_NT) {
            const float x0 = x[v], x1 = x[v + CE_NT], x2 = x[v + 2 * CE_NT], x3 = x[v + 3 * CE_NT];
            ce_push(m, s, x0);
            ce_push(m, s, x1);
            ce_push(m, s, x2);
            ce_push(m, s, x3);
        }
        for (; v < V; v += CE_NT) ce_push(m, s, x[v]);
    }
#pragma unroll
    for (int sh = 32; sh > 0; sh >>= 1) {
        const float m2 = __shfl_xor(m, sh), s2 = __shfl_xor(s, sh);
        ce_merge(m, s, m2, s2);
    }
    if ((tid & 63) == 0) sm_m[tid >> 6] = m, sm_s[tid >> 6] = s;
    __syncthreads();
    m = sm_m[0], s = sm_s[0];
#pragma unroll
    for (int w = 1; w < CE_NT / 64; w++) ce_merge(m, s, sm_m[w], sm_s[w]);
    const float inv = 1.0f / s;
    const int t = targets[row];
    if (tid == 0 && (t < 0 || t >= V)) row_loss[row] = __longlong_as_double(0x7ff8000000000000LL);
    // p = expf(x - m) * inv; dl = (p - [v == t]) / rows; the target's loss term
    auto one = [&](int v, float xv) {
        const float p = expf(xv - m) * inv;
        if (v == t) row_loss[row] = -log((double)p + 1e-30);
        return (p - (v == t ? 1.0f : 0.0f)) / rows;
    };
    if (vec) {
        if (tid < head) o[tid] = one(tid, x[tid]);
        v4f_t *o4 = reinterpret_cast<v4f_t *>(o + head);
        for (int c = tid; c < nv; c += CE_NT) {
            const v4f_t a = x4[c];
            const int v0 = head + 4 * c;
            o4[c] = v4f_t{one(v0, a[0]), one(v0 + 1, a[1]), one(v0 + 2, a[2]), one(v0 + 3, a[3])};
        }
        for (int v = tail0 + tid; v < V; v += CE_NT) o[v] = one(v, x[v]);
        for (int v = V + tid; v < pad; v += CE_NT) o[v] = 0.f;
        return;
    }
    int v = tid;
    for (; v + 3 * CE_NT < V; v += 4 * CE_NT) {
        float p[4];
#pragma unroll
        for (int u = 0; u < 4; u++) p[u] = expf(x[v + u * CE_NT] - m) * inv;
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int vv = v + u * CE_NT;
            if (vv == t) row_loss[row] = -log((double)p[u] + 1e-30);
            o[vv] = (p[u] - (vv == t ? 1.0f : 0.0f)) / rows;
        }
    }
    for (; v < V; v += CE_NT) {
        const float p = expf(x[v] - m) * inv;
        if (v == t) row_loss[row] = -log((double)p + 1e-30);
        o[v] = (p - (v == t ? 1.0f : 0.0f)) / rows;
    }
    for (v = V + tid; v < pad; v += CE_NT) o[v] = 0.f;
}

// *loss += (float)(sum_m row_loss[m] / rows), the sum in a fixed order.
__global__ __launch_bounds__(256) void ce_loss_kernel(const double *__restrict__ row_loss, int M,
                                                      double rows, float *__restrict__ loss) {
    __shared__ double red[4];
    double a = 0.0;
    for (int i = threadIdx.x; i < M; i += 256) a += row_loss[i];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) a += __shfl_xor(a, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = a;
    __syncthreads();
    if (threadIdx.x == 0) loss[0] += (float)((((red[0] + red[1]) + red[2]) + red[3]) / rows);
}

}  // namespace

hipError_t launch_cross_entropy(const float *logits, long ld, const int *targets, float *dl,
                                long ldd, int M, int V, int pad, int rows, double *row_loss,
                                hipStream_t s) {
    if (M <= 0) return hipSuccess;
    hipLaunchKernelGGL(ce_rows_kernel, dim3((unsigned)M), dim3(CE_NT), 0, s, logits, ld, targets,
                       dl, ldd, V, pad, (float)rows, row_loss);
    return hipGetLastError();
}

hipError_t launch_ce_loss(const double *row_loss, int M, int rows, float *loss, hipStream_t s) {
    if (M <= 0) return hipSuccess;
    hipLaunchKernelGGL(ce_loss_kernel, dim3(1), dim3(256), 0, s, row_loss, M, (double)rows, loss);
    return hipGetLastError();
}

}  // namespace pcl
