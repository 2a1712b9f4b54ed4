// kmeans_kernels.hip -- gfx950 (MI355X, CDNA4) kernels of the KMeans Lloyd path.
//
//   assign    fused E-step: x.c on fp32 MFMA (v_mfma_f32_4x4x1_16b_f32), the
//             ||c||^2 - 2 x.c epilogue and the running argmin stay in
//             registers; the n x k distance matrix never exists.
//   update    per-(row range, cluster group) sums and counts of X rows by
//             label in LDS, each column owned by one thread (deterministic).
//   finalize  fixed-order fp64 reduction of the partials, new centres,
//             ||c||^2 (centroid norms) and centre shift, then the loop's
//             convergence / empty-cluster decision in the last block.
//   rowdist   ||x_i - c_{label_i}||^2 per row (inertia, k-means|| mindists)
//             with a fixed-order fp64 reduction.
//   colsum / colmean / center / cnorm   set-up kernels.
//
// Semantics follow scikit-learn 1.7.2's Lloyd step:
//   sklearn/cluster/_k_means_lloyd.pyx:196-218 (E-step, strict '<' argmin)
//   sklearn/cluster/_k_means_common.pyx:94-124, :274-311 (inertia, average,
//   shift); the relocation of empty clusters runs on the host.
#include <math.h>

#include "internal.h"

namespace skm {

typedef float v4f __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// assign
// ---------------------------------------------------------------------------
//
// A wave owns 64 consecutive rows, one per lane.  For feature f, lane l feeds
// B = x_{row l}[f]; lane l also holds A = c_{chunk, l}[f] (cluster l of a
// 64-cluster chunk).  v_mfma_f32_4x4x1_16b_f32 with CBSZ=4, ABID=g broadcasts
// lanes 4g..4g+3 of A to all 16 blocks, so one instruction adds
// x_{row l}[f] * c_{4g+r}[f] into lane l, register r, for all 64 rows: each
// lane ends with its own row's dot products against 4*KG clusters and the
// argmin needs no cross-lane traffic.  k pads only to a multiple of 4.
//
// Centres are staged through LDS per (chunk, feature segment); X rows are read
// straight from HBM into registers (one row per lane, 16-byte loads).

template <int KG, int G = 0>
__device__ __forceinline__ void mfma_groups(v4f* acc, float a, float b)
{
    if constexpr (G < KG) {
        acc[G] = __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, acc[G], 4, G, 0);
        mfma_groups<KG, G + 1>(acc, a, b);
    }
}

template <int KG, int NQ>
__global__ __launch_bounds__(256, 2) void k_assign(const float* __restrict__ X, long n, int ld,
                                                   const float* __restrict__ C,
                                                   const float* __restrict__ cnorm, int k,
                                                   int* __restrict__ labels, LoopState* st,
                                                   int count_changes)
{
    if (st != nullptr && st->done != 0) return;
    constexpr int CPC = 4 * KG;   // clusters per chunk
    constexpr int SEG = 4 * NQ;   // features per segment
    constexpr int LS = SEG + 4;   // LDS row stride (floats): conflict-free b128 reads
    __shared__ __attribute__((aligned(16))) float sC[CPC * LS];
    __shared__ float sN[CPC];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int nchunk = (k + CPC - 1) / CPC;
    const int nseg = (ld + SEG - 1) / SEG;
    const bool single = (nchunk == 1) && (nseg == 1);
    const int crow = lane < CPC ? lane : CPC - 1;

    auto stage = [&](int ch, int sg) {
        const int f0 = sg * SEG;
        const int nq = min(NQ, (ld - f0) >> 2);
        for (int idx = tid; idx < CPC * NQ; idx += 256) {
            const int cl = idx / NQ;
            const int q = idx - cl * NQ;
            const int j = ch * CPC + cl;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (j < k && q < nq) v = *reinterpret_cast<const float4*>(C + (long)j * ld + f0 + 4 * q);
            *reinterpret_cast<float4*>(&sC[cl * LS + 4 * q]) = v;
        }
        if (sg == 0) {
            for (int i = tid; i < CPC; i += 256) {
                const int j = ch * CPC + i;
                sN[i] = j < k ? cnorm[j] : 0.f;
            }
        }
    };

    if (single) {
        stage(0, 0);
        __syncthreads();
    }

    const long stride = (long)gridDim.x * 256;
    for (long base = (long)blockIdx.x * 256; base < n; base += stride) {
        const long row = base + wave * 64 + lane;
        const long rr = row < n ? row : n - 1;
        const float* xrow = X + rr * ld;
        float best = INFINITY;
        int bidx = 0;
        for (int ch = 0; ch < nchunk; ++ch) {
            v4f acc[KG];
#pragma unroll
            for (int g = 0; g < KG; ++g) acc[g] = v4f{0.f, 0.f, 0.f, 0.f};
            for (int sg = 0; sg < nseg; ++sg) {
                if (!single) {
                    __syncthreads();
                    stage(ch, sg);
                    __syncthreads();
                }
                const int f0 = sg * SEG;
                const int nq = min(NQ, (ld - f0) >> 2);
                float4 xv[NQ];
#pragma unroll
                for (int q = 0; q < NQ; ++q)
                    if (q < nq) xv[q] = *reinterpret_cast<const float4*>(xrow + f0 + 4 * q);
#pragma unroll
                for (int q = 0; q < NQ; ++q) {
                    if (q < nq) {
                        const float4 cv = *reinterpret_cast<const float4*>(&sC[crow * LS + 4 * q]);
                        mfma_groups<KG>(acc, cv.x, xv[q].x);
                        mfma_groups<KG>(acc, cv.y, xv[q].y);
                        mfma_groups<KG>(acc, cv.z, xv[q].z);
                        mfma_groups<KG>(acc, cv.w, xv[q].w);
                    }
                }
            }
            // ||c||^2 - 2 x.c, first minimum wins (_k_means_lloyd.pyx:196-212)
#pragma unroll
            for (int g = 0; g < KG; ++g) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int jl = 4 * g + r;
                    const int j = ch * CPC + jl;
                    const float dist = fmaf(-2.0f, acc[g][r], sN[jl]);
                    if (j < k && dist < best) {
                        best = dist;
                        bidx = j;
                    }
                }
            }
        }
        if (row < n) {
            int moved = 0;
            if (count_changes) moved = labels[row] != bidx;
            labels[row] = bidx;
            if (count_changes) {
                const unsigned long long m = __ballot(moved);
                if (lane == 0 && m != 0ull) atomicAdd(&st->changed, (int)__popcll(m));
            }
        }
    }
}

typedef void (*assign_fn)(const float*, long, int, const float*, const float*, int, int*, LoopState*, int);

template <int NQ, int... KGs>
struct AssignTable {
    static assign_fn get(int kg)
    {
        assign_fn f = nullptr;
        ((kg == KGs ? (f = &k_assign<KGs, NQ>, 0) : 0), ...);
        return f;
    }
};

template <int NQ>
static assign_fn pick_kg(int kg)
{
    return AssignTable<NQ, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16>::get(kg);
}

static int occupancy_blocks(assign_fn f)
{
    // cached per kernel instance
    static assign_fn keys[80];
    static int vals[80];
    static int used = 0;
    for (int i = 0; i < used; ++i)
        if (keys[i] == f) return vals[i];
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, reinterpret_cast<const void*>(f), 256, 0) != hipSuccess ||
        nb < 1)
        nb = 1;
    if (used < 80) {
        keys[used] = f;
        vals[used] = nb;
        ++used;
    }
    return nb;
}

hipError_t launch_assign(const AssignArgs& a, int num_cu, hipStream_t s)
{
    if (a.n <= 0) return hipSuccess;
    const int nchunk = (a.k + 63) / 64;
    const int per = (a.k + nchunk - 1) / nchunk;
    const int kg = (per + 3) / 4;
    const int q = a.ld / 4;
    assign_fn f = q <= 4 ? pick_kg<4>(kg) : q <= 8 ? pick_kg<8>(kg) : q <= 16 ? pick_kg<16>(kg) : pick_kg<32>(kg);
    if (f == nullptr) return hipErrorInvalidValue;
    const long tiles = (a.n + 255) / 256;
    long blocks = (long)num_cu * occupancy_blocks(f);
    if (blocks > tiles) blocks = tiles;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(f, dim3((unsigned)blocks), dim3(256), 0, s, a.X, a.n, a.ld, a.C, a.cnorm, a.k, a.labels,
                       a.state, a.count_changes);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// update: per-(row range, cluster group) sums and counts
// ---------------------------------------------------------------------------
//
// Block (r, g) walks rows [r*rpr, (r+1)*rpr) in order and adds every row whose
// label falls in cluster group g into an LDS table S[cg x d].  Column c of S is
// only ever touched by thread c mod blockDim, so every partial sum is formed
// in row order: bitwise reproducible.  X is read once overall (each row is
// used by the one group owning its label); labels are read once per group.

__global__ __launch_bounds__(256) void k_update(const float* __restrict__ X, long n, int ld, int d,
                                                const int* __restrict__ labels, int k, int cg, long rpr,
                                                float* __restrict__ psum, int* __restrict__ pcnt,
                                                const LoopState* st)
{
    if (st != nullptr && st->done != 0) return;
    extern __shared__ float sS[];
    constexpr int LCH = 256;
    __shared__ int sLab[LCH];
    int* sCnt = reinterpret_cast<int*>(sS + (long)cg * d);
    const int r = blockIdx.x;
    const int g = blockIdx.y;
    const int j0 = g * cg;
    const int j1 = min(k, j0 + cg);
    const long row0 = (long)r * rpr;
    const long row1 = min(n, row0 + rpr);
    const int T = blockDim.x;
    for (int i = threadIdx.x; i < cg * d; i += T) sS[i] = 0.f;
    for (int i = threadIdx.x; i < cg; i += T) sCnt[i] = 0;
    for (long c0 = row0; c0 < row1; c0 += LCH) {
        const int m = (int)min((long)LCH, row1 - c0);
        __syncthreads();
        for (int i = threadIdx.x; i < m; i += T) sLab[i] = labels[c0 + i];
        __syncthreads();
        for (int i = 0; i < m; ++i) {
            const int lab = sLab[i];
            if (lab >= j0 && lab < j1) {
                float* srow = sS + (long)(lab - j0) * d;
                const float* xr = X + (c0 + i) * ld;
                for (int c = threadIdx.x; c < d; c += T) srow[c] += xr[c];
                if (threadIdx.x == 0) sCnt[lab - j0] += 1;
            }
        }
    }
    __syncthreads();
    for (int jl = 0; jl < j1 - j0; ++jl) {
        float* dst = psum + ((long)r * k + j0 + jl) * ld;
        for (int c = threadIdx.x; c < d; c += T) dst[c] = sS[(long)jl * d + c];
    }
    for (int jl = threadIdx.x; jl < j1 - j0; jl += T) pcnt[(long)r * k + j0 + jl] = sCnt[jl];
}

UpdateGeom update_geometry(long n, int d, int k, int num_cu)
{
    UpdateGeom g{};
    const long lds_words = 12 * 1024;  // 48 KB of sums + counts per block
    g.cg = (int)max(1L, min((long)k, lds_words / (long)(d + 1)));
    g.G = (k + g.cg - 1) / g.cg;
    g.threads = d >= 256 ? 256 : ((d + 63) / 64) * 64;
    const long target = (long)num_cu * 8;
    long R = target / g.G;
    if (R < 1) R = 1;
    const long max_r = (n + 255) / 256;
    if (R > max_r) R = max_r;
    if (R > 4096) R = 4096;
    g.R = (int)R;
    g.rows_per_range = (n + R - 1) / R;
    g.lds = (size_t)g.cg * d * sizeof(float) + (size_t)g.cg * sizeof(int);
    return g;
}

hipError_t launch_update(const UpdateArgs& a, const UpdateGeom& g, hipStream_t s)
{
    if (a.n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_update, dim3(g.R, g.G), dim3(g.threads), g.lds, s, a.X, a.n, a.ld, a.d, a.labels, a.k,
                       g.cg, g.rows_per_range, a.psum, a.pcnt, a.state);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// finalize
// ---------------------------------------------------------------------------
//
// Block (j, cc) reduces the R partial sums of cluster j, columns
// [32cc, 32cc+32), in a fixed order (8 interleaved fp64 lanes per column, then
// those 8 in order).  The last block to finish cluster j folds the per-chunk
// shift^2 and ||c||^2 partials; the last cluster to finish evaluates the
// loop's stopping rules (_kmeans.py:717-732) and flags empty clusters.

template <typename T>
__device__ __forceinline__ T coherent_load(const T* p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ __launch_bounds__(256) void k_finalize(FinalizeArgs a)
{
    LoopState* st = a.state;
    if (st->done != 0) return;
    const int j = blockIdx.x;
    const int cc = blockIdx.y;
    const int nch = gridDim.y;
    const int tid = threadIdx.x;
    const int cl = tid & 31;
    const int rs = tid >> 5;
    const int col = cc * 32 + cl;
    __shared__ double red[8][33];
    __shared__ int cred[256];
    __shared__ double pr[2][32];

    int cnt = 0;
    for (int r = tid; r < a.R; r += 256) cnt += a.pcnt[(long)r * a.k + j];
    cred[tid] = cnt;
    double s = 0.0;
    if (col < a.d)
        for (int r = rs; r < a.R; r += 8) s += (double)a.psum[((long)r * a.k + j) * a.ld + col];
    red[rs][cl] = s;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (tid < w) cred[tid] += cred[tid + w];
        __syncthreads();
    }
    const int count = cred[0];
    if (rs == 0) {
        double sq = 0.0, nrm = 0.0;
        if (col < a.d) {
            double tot = 0.0;
            for (int t = 0; t < 8; ++t) tot += red[t][cl];
            a.sums[(long)j * a.ld + col] = tot;
            if (count > 0) {
                const float cn = (float)(tot / (double)count);
                a.C_new[(long)j * a.ld + col] = cn;
                const double df = (double)cn - (double)a.C_old[(long)j * a.ld + col];
                sq = df * df;
                nrm = (double)cn * (double)cn;
            }
        }
        pr[0][cl] = sq;
        pr[1][cl] = nrm;
    }
    __syncthreads();
    if (tid == 0) {
        double ssq = 0.0, snr = 0.0;
        for (int t = 0; t < 32; ++t) {
            ssq += pr[0][t];
            snr += pr[1][t];
        }
        a.part[((long)j * nch + cc) * 2 + 0] = ssq;
        a.part[((long)j * nch + cc) * 2 + 1] = snr;
        __threadfence();
        const unsigned prev = atomicAdd(&a.cluster_ctr[j], 1u);
        if (prev == (unsigned)(nch - 1)) {
            __threadfence();
            double tsq = 0.0, tnr = 0.0;
            for (int c2 = 0; c2 < nch; ++c2) {
                tsq += coherent_load(&a.part[((long)j * nch + c2) * 2 + 0]);
                tnr += coherent_load(&a.part[((long)j * nch + c2) * 2 + 1]);
            }
            a.shift_sq[j] = (float)tsq;
            if (count > 0) a.cnorm[j] = (float)tnr;
            a.counts[j] = count;
            a.cluster_ctr[j] = 0u;
            __threadfence();
            const unsigned done_clusters = atomicAdd(&st->global_ctr, 1u);
            if (done_clusters == (unsigned)(a.k - 1)) {
                __threadfence();
                int n_empty = 0;
                double tot = 0.0;
                for (int jj = 0; jj < a.k; ++jj) {
                    n_empty += coherent_load(&a.counts[jj]) == 0;
                    tot += (double)coherent_load(&a.shift_sq[jj]);
                }
                const int changed = coherent_load(&st->changed);
                st->n_empty = n_empty;
                st->shift_tot = tot;
                st->last_changed = changed;
                st->changed = 0;
                st->global_ctr = 0u;
                st->n_iter = a.iter + 1;
                int done = 0;
                if (n_empty > 0)
                    done = 3;
                else if ((a.flags & kStopStrict) && changed == 0)
                    done = 1;
                else if (a.tol > 0.0 && tot <= a.tol)
                    done = 2;
                if (done != 0) st->halt_iter = a.iter;
                __threadfence();
                st->done = done;
            }
        }
    }
}

hipError_t launch_finalize(const FinalizeArgs& a, hipStream_t s)
{
    hipLaunchKernelGGL(k_finalize, dim3(a.k, finalize_col_chunks(a.d)), dim3(256), 0, s, a);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// rowdist: ||x_i - c_{label_i}||^2 and its fp64 total
// ---------------------------------------------------------------------------
//
// Per row in fp32, in the association order of sklearn's
// _euclidean_dense_dense (_k_means_common.pyx:16-43): groups of four squared
// differences summed left to right, each group added to the running sum.

__global__ __launch_bounds__(256) void k_rowdist(RowDistArgs a)
{
#pragma clang fp contract(off)
    const long row = (long)blockIdx.x * 256 + threadIdx.x;
    double v = 0.0;
    const int lab = row < a.n ? a.labels[row] : -1;
    if (lab >= 0 && lab < a.k) {
        const float* x = a.X + row * a.ld;
        const float* c = a.C + (long)lab * a.ld;
        float res = 0.f;
        int f = 0;
        for (; f + 4 <= a.d; f += 4) {
            const float4 xv = *reinterpret_cast<const float4*>(x + f);
            const float4 cv = *reinterpret_cast<const float4*>(c + f);
            const float t0 = xv.x - cv.x, t1 = xv.y - cv.y, t2 = xv.z - cv.z, t3 = xv.w - cv.w;
            res += ((t0 * t0 + t1 * t1) + t2 * t2) + t3 * t3;
        }
        for (; f < a.d; ++f) {
            const float t = x[f] - c[f];
            res += t * t;
        }
        if (a.out_rows != nullptr) a.out_rows[row] = res;
        v = (double)res;
    }
    __shared__ double red[256];
    red[threadIdx.x] = v;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    __shared__ bool last;
    if (threadIdx.x == 0) {
        a.block_part[blockIdx.x] = red[0];
        __threadfence();
        last = atomicAdd(&a.state->rowdist_ctr, 1u) == gridDim.x - 1;
    }
    __syncthreads();
    if (!last) return;
    __threadfence();
    double t = 0.0;
    for (int b = threadIdx.x; b < (int)gridDim.x; b += 256) t += coherent_load(&a.block_part[b]);
    red[threadIdx.x] = t;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        a.state->inertia = red[0];
        a.state->rowdist_ctr = 0u;
    }
}

int rowdist_grid(long n) { return (int)max(1L, (n + 255) / 256); }

hipError_t launch_rowdist(const RowDistArgs& a, hipStream_t s)
{
    hipLaunchKernelGGL(k_rowdist, dim3(rowdist_grid(a.n)), dim3(256), 0, s, a);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// set-up kernels
// ---------------------------------------------------------------------------

constexpr long kColsumRows = 4096;

int colsum_grid(long n) { return (int)max(1L, (n + kColsumRows - 1) / kColsumRows); }

__global__ __launch_bounds__(256) void k_colsum(const float* __restrict__ X, long n, int ld, int d,
                                                double* __restrict__ part)
{
    const long r0 = (long)blockIdx.x * kColsumRows;
    const long r1 = min(n, r0 + kColsumRows);
    for (int c = threadIdx.x; c < d; c += blockDim.x) {
        double s = 0.0;
        for (long r = r0; r < r1; ++r) s += (double)X[r * ld + c];
        part[(long)blockIdx.x * d + c] = s;
    }
}

hipError_t launch_colsum(const float* X, long n, int ld, int d, double* part, int nblk, hipStream_t s)
{
    hipLaunchKernelGGL(k_colsum, dim3(nblk), dim3(256), 0, s, X, n, ld, d, part);
    return hipGetLastError();
}

__global__ void k_colmean(const double* __restrict__ part, int nblk, long n, int d, float* __restrict__ mean)
{
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= d) return;
    double s = 0.0;
    for (int b = 0; b < nblk; ++b) s += part[(long)b * d + c];
    mean[c] = (float)(s / (double)n);
}

hipError_t launch_colmean(const double* part, int nblk, long n, int d, float* mean, hipStream_t s)
{
    hipLaunchKernelGGL(k_colmean, dim3((d + 255) / 256), dim3(256), 0, s, part, nblk, n, d, mean);
    return hipGetLastError();
}

__global__ void k_center(float* __restrict__ X, long n, int ld, int d, const float* __restrict__ mean)
{
    const long total = n * (long)ld;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (long)gridDim.x * blockDim.x) {
        const int c = (int)(i % ld);
        if (c < d) X[i] = X[i] - mean[c];
    }
}

hipError_t launch_center(float* X, long n, int ld, int d, const float* mean, hipStream_t s)
{
    const long total = n * (long)ld;
    long blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(k_center, dim3((unsigned)blocks), dim3(256), 0, s, X, n, ld, d, mean);
    return hipGetLastError();
}

__global__ void k_cnorm(const float* __restrict__ C, int k, int ld, float* __restrict__ cnorm)
{
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= k) return;
    double s = 0.0;
    for (int c = 0; c < ld; ++c) {
        const double v = (double)C[(long)j * ld + c];
        s += v * v;
    }
    cnorm[j] = (float)s;
}

hipError_t launch_cnorm(const float* C, int k, int ld, float* cnorm, hipStream_t s)
{
    hipLaunchKernelGGL(k_cnorm, dim3((k + 255) / 256), dim3(256), 0, s, C, k, ld, cnorm);
    return hipGetLastError();
}

}  // namespace skm
