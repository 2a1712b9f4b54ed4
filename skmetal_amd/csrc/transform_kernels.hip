// transform_kernels.hip -- KMeans.transform on the device (gfx950): the
// n x k matrix of Euclidean distances from each row to each centre.
//
// scikit-learn's KMeans.transform is euclidean_distances(X, cluster_centers_)
// (sklearn/cluster/_kmeans.py:1124-1148); for float32 inputs that upcasts to
// fp64 (_euclidean_distances_upcast, sklearn/metrics/pairwise.py:582-652):
// d = (-2 x.c + ||x||^2) + ||c||^2 in fp64 (:647-649), cast to fp32 (:651),
// negatives set to 0 (:428-431), then np.sqrt in fp32 (:441).  The kernel computes the same expression with
// exact fp64 products of the fp32 inputs, so the fp32 results round alike.
// The fp32 square root is taken as the fp64 root rounded to fp32, which is the
// correctly rounded fp32 root (53 >= 2 * 24 + 2 bits).
//
// A block owns a 128-row x 64-centre tile: thread (rg, cg) accumulates rows
// rg + 32 i (i < 4) against centres cg + 8 j (j < 8) in fp64 registers, the
// rows and centres staged through LDS (as fp64) 32 features at a time
// (coalesced 128-byte row runs).  The reference computed ||x||^2 + ||c||^2 - 2 x.c in fp32 around
// skmetal_gemm (skmetal/estimators/cluster.py:135-146).
#include "device.h"

namespace skm {

namespace {

constexpr int kTR = 128;  // rows per tile (4 per thread)
constexpr int kTC = 64;   // centres per tile
constexpr int kTF = 32;   // features per LDS segment

__global__ __launch_bounds__(256) void k_cnorm64(TransformArgs a)
{
    const int j = blockIdx.x * 256 + threadIdx.x;
    if (j >= a.k) return;
    const float* c = a.C + (long)j * a.ld;
    double acc = 0.0;
    // the loads of 8 features in flight at once, the sum in feature order
    int f = 0;
    for (; f + 8 <= a.ld; f += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = c[f + u];
#pragma unroll
        for (int u = 0; u < 8; ++u) acc = fma((double)v[u], (double)v[u], acc);
    }
    for (; f < a.ld; ++f) acc = fma((double)c[f], (double)c[f], acc);
    a.cc[j] = acc;
}

__global__ __launch_bounds__(256) void k_transform(TransformArgs a)
{
    // x is staged as fp64 (converted once, not at every use)
    // rows of kTF + 2 doubles: 16-byte aligned for the two-feature reads
    __shared__ __attribute__((aligned(16))) double xs[kTR][kTF + 2];
    __shared__ __attribute__((aligned(16))) double cs[kTC][kTF + 2];
    constexpr int RI = kTR / 32;  // rows per thread
    const int tid = threadIdx.x;
    const int rg = tid >> 3, cg = tid & 7;
    const long r0 = (long)blockIdx.x * kTR;
    const int c0 = blockIdx.y * kTC;
    double acc[RI][8];
#pragma unroll
    for (int i = 0; i < RI; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = 0.0;
    double xx[RI];
#pragma unroll
    for (int i = 0; i < RI; ++i) xx[i] = 0.0;

    for (int f0 = 0; f0 < a.ld; f0 += kTF) {
        const int fl = min(kTF, a.ld - f0);  // a multiple of 4 (ld is)
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kTR * kTF / 4 / 256; ++i) {
            const int e = tid + 256 * i;
            const int r = e >> 3, q = e & 7;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (4 * q < fl && r0 + r < a.n) v = *reinterpret_cast<const float4*>(a.X + (r0 + r) * a.ld + f0 + 4 * q);
            xs[r][4 * q] = v.x;
            xs[r][4 * q + 1] = v.y;
            xs[r][4 * q + 2] = v.z;
            xs[r][4 * q + 3] = v.w;
        }
#pragma unroll
        for (int i = 0; i < kTC * kTF / 4 / 256; ++i) {
            const int e = tid + 256 * i;
            const int r = e >> 3, q = e & 7;
            float4 w = make_float4(0.f, 0.f, 0.f, 0.f);
            if (4 * q < fl && c0 + r < a.k) w = *reinterpret_cast<const float4*>(a.C + (long)(c0 + r) * a.ld + f0 + 4 * q);
            cs[r][4 * q] = w.x;
            cs[r][4 * q + 1] = w.y;
            cs[r][4 * q + 2] = w.z;
            cs[r][4 * q + 3] = w.w;
        }
        __syncthreads();
        for (int f = 0; f < fl; f += 2) {  // fl is even: features f, f + 1 per read
            double2 x[RI];
#pragma unroll
            for (int i = 0; i < RI; ++i) {
                x[i] = *reinterpret_cast<const double2*>(&xs[rg + 32 * i][f]);
                xx[i] = fma(x[i].x, x[i].x, xx[i]);
                xx[i] = fma(x[i].y, x[i].y, xx[i]);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const double2 c = *reinterpret_cast<const double2*>(&cs[cg + 8 * j][f]);
#pragma unroll
                for (int i = 0; i < RI; ++i) {
                    acc[i][j] = fma(x[i].x, c.x, acc[i][j]);
                    acc[i][j] = fma(x[i].y, c.y, acc[i][j]);
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < RI; ++i) {
        const long row = r0 + rg + 32 * i;
        if (row >= a.n) continue;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int col = c0 + cg + 8 * j;
            if (col < a.k) {
                float d32 = (float)((-2.0 * acc[i][j] + xx[i]) + a.cc[col]);
                if (d32 < 0.f) d32 = 0.f;
                a.out[row * a.k + col] = (float)sqrt((double)d32);
            }
        }
    }
}

}  // namespace

hipError_t launch_transform(const TransformArgs& a, hipStream_t s)
{
    hipLaunchKernelGGL(k_cnorm64, dim3((unsigned)((a.k + 255) / 256)), dim3(256), 0, s, a);
    const dim3 grid((unsigned)((a.n + kTR - 1) / kTR), (unsigned)((a.k + kTC - 1) / kTC));
    hipLaunchKernelGGL(k_transform, grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace skm
