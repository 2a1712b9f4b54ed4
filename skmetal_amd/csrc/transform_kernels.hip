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
// Rows of at most 128 floats (k_transform_mm): the dot products on the fp64
// matrix cores, v_mfma_f64_16x16x4_f64 chained over the features, which adds
// the exact products one at a time in feature order (the sums of a
// sequential fma chain).  Wider rows (k_transform): a block owns a 128-row x
// 64-centre tile: thread (rg, cg) accumulates rows rg + 32 i (i < 4) against
// centres cg + 8 j (j < 8) in fp64 registers, the rows and centres staged
// through LDS (as fp64) 32 features at a time (coalesced 128-byte row runs),
// the same chains.  The reference computed ||x||^2 + ||c||^2 - 2 x.c in fp32
// around skmetal_gemm (skmetal/estimators/cluster.py:135-146).
#include "device.h"

namespace skm {

namespace {

constexpr int kTR = 128;  // rows per tile (4 per thread)
constexpr int kTC = 64;   // centres per tile
constexpr int kTF = 32;   // features per LDS segment

// ||c||^2 in fp64 (feature order), and with a.cfrag the centres as the B
// operands of v_mfma_f64_16x16x4_f64 in 16-centre groups:
// cfrag[(g ld/4 + j) 64 + l] = centre 16 g + l % 16 (the last one past k),
// feature 4 j + l / 16.
__global__ __launch_bounds__(256) void k_cnorm64(TransformArgs a)
{
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    const int c4 = a.ld / 4, G = (a.k + 15) / 16;
    if (a.cfrag != nullptr && i < (long)G * c4 * 64) {
        const int l = (int)(i & 63);
        const long gj = i >> 6;
        const int g = (int)(gj / c4), jj = (int)(gj - (long)g * c4);
        a.cfrag[i] = (double)a.C[(long)min(16 * g + (l & 15), a.k - 1) * a.ld + 4 * jj + (l >> 4)];
    }
    const int j = (int)i;
    if (i >= a.k) return;
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

// Rows of at most LDM floats: 64-row sub-groups through LDS (each a
// contiguous span of X loaded whole, the next one in flight), wave w taking
// rows 16 w .. 16 w + 15 and, per 16-centre group, a chain of ld / 4
// v_mfma_f64_16x16x4_f64 (A: the rows, B: a.cfrag).  Lane l then holds
// rows l / 16 + 4 r against centre l % 16.
template <int LDM>
__global__ __launch_bounds__(256, 4) void k_transform_mm(TransformArgs a)
{
    typedef double v4d __attribute__((ext_vector_type(4)));
    constexpr int SMAX = ctg_stride(LDM);
    constexpr int NV = (16 * LDM + 255) / 256;
    constexpr int NJ = LDM / 4;
    __shared__ __attribute__((aligned(16))) float tile[64 * SMAX];
    __shared__ double sxx[64];  // ||x||^2 of the sub-group's rows
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ld = a.ld, c4 = ld / 4, S = ctg_stride(ld), k = a.k;
    const long n = a.n;
    const long nsg = (n + 63) / 64;
    const f4v* X4 = reinterpret_cast<const f4v*>(a.X);
    const int G = (k + 15) / 16;
    const int q = lane >> 4, cj = lane & 15;

    int off[NV];
    const float inv_c4 = 1.0f / (float)c4;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int qq = tid + 256 * i;
        const int r = (int)(((float)qq + 0.5f) * inv_c4);
        off[i] = r * S + 4 * (qq - r * c4);
    }
    f4v P[NV];
    auto load = [&](long sg) {
        const long r0 = 64 * sg;
        const int e4 = (int)(min(64L, n - r0) * c4);
        const f4v* base = X4 + r0 * c4;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int qq = tid + 256 * i;
            if (qq < e4) P[i] = base[qq];
        }
    };
    long sg = blockIdx.x;
    if (sg < nsg) load(sg);
    for (; sg < nsg; sg += gridDim.x) {
        const long r0 = 64 * sg;
        const int e4 = (int)(min(64L, n - r0) * c4);
        __syncthreads();  // every wave is done with the tile
#pragma unroll
        for (int i = 0; i < NV; ++i)
            if (tid + 256 * i < e4) *reinterpret_cast<f4v*>(tile + off[i]) = P[i];
        if (sg + gridDim.x < nsg) load(sg + gridDim.x);  // in flight while this one is worked on
        __syncthreads();

        // ||x||^2 of the wave's 16 rows in feature order (lanes 0..15)
        if (lane < 16) {
            const float* xr = tile + (16 * w + lane) * S;
            double xx = 0.0;
#pragma unroll
            for (int j = 0; j < NJ; ++j)
                if (j < c4) {
                    const f4v xv = *reinterpret_cast<const f4v*>(xr + 4 * j);
                    xx = fma((double)xv.x, (double)xv.x, xx);
                    xx = fma((double)xv.y, (double)xv.y, xx);
                    xx = fma((double)xv.z, (double)xv.z, xx);
                    xx = fma((double)xv.w, (double)xv.w, xx);
                }
            sxx[16 * w + lane] = xx;
        }
        __builtin_amdgcn_wave_barrier();  // (a wave's LDS accesses complete in order)
        double xxr[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) xxr[r] = sxx[16 * w + q + 4 * r];

        const float* ar = tile + (16 * w + cj) * S + q;  // A: row cj, feature 4 j + q
        // two groups at a time: two independent chains share the A values
        for (int g = 0; g < G; g += 2) {
            const bool two = g + 1 < G;  // wave-uniform
            const double* bf = a.cfrag + ((long)g * c4 << 6) + lane;
            const double* bf2 = two ? bf + ((long)c4 << 6) : bf;  // (in bounds either way)
            v4d acc = {0.0, 0.0, 0.0, 0.0}, acc2 = {0.0, 0.0, 0.0, 0.0};
            for (int j0 = 0; j0 < c4; j0 += 4) {  // four K steps' operands loaded together
                double bv[4], bv2[4];
                float av[4];
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    if (j0 + u < c4) {
                        bv[u] = bf[(long)(j0 + u) << 6];
                        bv2[u] = bf2[(long)(j0 + u) << 6];
                        av[u] = ar[4 * (j0 + u)];
                    }
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    if (j0 + u < c4) {
                        const double x = (double)av[u];
                        acc = __builtin_amdgcn_mfma_f64_16x16x4f64(x, bv[u], acc, 0, 0, 0);
                        if (two) acc2 = __builtin_amdgcn_mfma_f64_16x16x4f64(x, bv2[u], acc2, 0, 0, 0);
                    }
            }
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const int col = 16 * (g + p) + cj;
                if (col < k && (p == 0 || two)) {
                    const double cn = a.cc[col];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const long row = r0 + 16 * w + q + 4 * r;
                        if (row < n) {
                            float d32 = (float)((-2.0 * (p == 0 ? acc[r] : acc2[r]) + xxr[r]) + cn);
                            if (d32 < 0.f) d32 = 0.f;
                            a.out[row * k + col] = (float)sqrt((double)d32);
                        }
                    }
                }
            }
        }
        __builtin_amdgcn_wave_barrier();  // sxx is rewritten only after the next block barrier
    }
}

typedef void (*transform_fn)(TransformArgs);

int transform_occupancy(transform_fn f)
{
    static transform_fn keys[8];
    static int vals[8];
    static int used = 0;
    for (int i = 0; i < used; ++i)
        if (keys[i] == f) return vals[i];
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, reinterpret_cast<const void*>(f), 256, 0) != hipSuccess ||
        nb < 1)
        nb = 1;
    if (used < 8) {
        keys[used] = f;
        vals[used] = nb;
        ++used;
    }
    return nb;
}

}  // namespace

hipError_t launch_transform(const TransformArgs& a, hipStream_t s)
{
    const long nf = a.cfrag != nullptr ? (long)(a.k + 15) / 16 * 16 * a.ld : 0;  // fragment elements
    const long ne = nf > a.k ? nf : a.k;
    hipLaunchKernelGGL(k_cnorm64, dim3((unsigned)((ne + 255) / 256)), dim3(256), 0, s, a);
    if (a.cfrag != nullptr && transform_mm_path(a.ld)) {
        const transform_fn f = a.ld <= 32 ? &k_transform_mm<32>
                               : a.ld <= 64 ? &k_transform_mm<64>
                               : a.ld <= 104 ? &k_transform_mm<104>
                                             : &k_transform_mm<128>;
        const long nsg = (a.n + 63) / 64;
        const long cap = (long)(a.cus > 0 ? a.cus : 256) * transform_occupancy(f);
        hipLaunchKernelGGL(f, dim3((unsigned)(nsg < cap ? nsg : cap)), dim3(256), 0, s, a);
        return hipGetLastError();
    }
    const dim3 grid((unsigned)((a.n + kTR - 1) / kTR), (unsigned)((a.k + kTC - 1) / kTC));
    hipLaunchKernelGGL(k_transform, grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace skm
