// plusplus_kernels.hip -- greedy k-means++ seeding on the device (gfx950).
//
// scikit-learn's _kmeans_plusplus (sklearn/cluster/_kmeans.py:174-260), unit
// sample weights, with X resident in HBM.  The caller draws the random numbers
// from its RandomState in sklearn's order (the first row, then T uniforms per
// further centre) and passes them in, so a seeded run picks the rows sklearn
// picks.  Per centre c:
//
//   k_pp_select(c)  one block: the potential of each of centre c-1's
//                   candidates (fixed-order fp64 sum of its block partials),
//                   first minimum wins -> centre c-1 = that candidate's row
//                   (gathered into `centers`); then the draws of centre c:
//                   r_t = u_t * fp32(potential) (sklearn's potential is an
//                   fp32 dot product), candidate_t = the first row whose
//                   running sum of closest distances reaches r_t (searchsorted
//                   over stable_cumsum, :247-250), clipped to n - 1;
//   k_pp_dist(c)    one thread per row (rows staged through LDS in
//                   coalesced 128-byte runs): the distance to each candidate in
//                   sklearn's form for fp32 data (_euclidean_distances_upcast:
//                   fp64 -2 x.c + ||c||^2 + ||x||^2, cast to fp32, negatives
//                   to 0), min with the row's closest distance so far, and
//                   per-block fp64 sums of those minima.
//
// The running sum is a two-level fp64 scan (block sums, then the rows of the
// block the draw falls in), so its rounding differs from numpy's sequential
// cumsum only at the last bits of fp64.  Everything is fixed-order:
// identical inputs give identical picks.
#include <climits>

#include "device.h"

namespace skm {

namespace {

constexpr int kFS = 32;         // features per LDS segment (one 128-byte run per row)
constexpr int kXS = kFS + 4;    // LDS row stride (floats): 144 bytes keeps 8 lanes' float4 reads on distinct banks

// Centre c's candidate distances, TP candidates per pass (Tc in all).  The
// block's 256 rows go through LDS one 32-feature segment at a time: eight
// lanes load one row's 128-byte run (coalesced), then thread r works on row r.
// ||x||^2 and the candidates' ||c||^2 come from the same staged values.
template <int TP>
__global__ __launch_bounds__(256) void k_pp_dist(PPArgs a, int c, int Tc)
{
    __shared__ float4 xs4[kPPRows * kXS / 4];
    __shared__ double cs[TP][kFS];
    __shared__ double ccs[TP];
    __shared__ double red[4][TP];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const long r0 = (long)blockIdx.x * kPPRows;
    const long row = r0 + tid;
    const bool live = row < a.n;
    const int p = c & 1;
    float closest = INFINITY;
    if (c > 0 && live) closest = a.D[p ^ 1][(long)a.best[c - 1] * a.n + row];

    for (int t0 = 0; t0 < Tc; t0 += TP) {
        const int tn = min(TP, Tc - t0);
        double acc[TP];
#pragma unroll
        for (int t = 0; t < TP; ++t) acc[t] = 0.0;
        double xx = 0.0, cc = 0.0;
        // segment f0's runs: lane group tid >> 3 loads rows (tid >> 3) + 32 i
        const int q = tid & 7;
        float4 pre[8];
        auto load_seg = [&](int f0) {
            const int fl = min(kFS, a.ld - f0);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int lr = (tid >> 3) + 32 * i;
                pre[i] = make_float4(0.f, 0.f, 0.f, 0.f);
                if (4 * q < fl && r0 + lr < a.n) pre[i] = *reinterpret_cast<const float4*>(a.X + (r0 + lr) * a.ld + f0 + 4 * q);
            }
        };
        load_seg(0);
        for (int f0 = 0; f0 < a.ld; f0 += kFS) {
            const int fl = min(kFS, a.ld - f0);  // a multiple of 4 (ld is)
            __syncthreads();
#pragma unroll
            for (int i = 0; i < 8; ++i) xs4[(((tid >> 3) + 32 * i) * kXS) / 4 + q] = pre[i];
            for (int e = tid; e < TP * kFS; e += 256) {
                const int t = e / kFS, f = e % kFS;
                double v = 0.0;
                if (t < tn && f < fl) v = (double)a.X[a.cand[t0 + t] * a.ld + f0 + f];
                cs[t][f] = v;
            }
            __syncthreads();
            if (f0 + kFS < a.ld) load_seg(f0 + kFS);  // in flight during this segment's work
            if (tid < TP)
                for (int f = 0; f < kFS; ++f) cc = fma(cs[tid][f], cs[tid][f], cc);
#pragma unroll
            for (int j = 0; j < kFS / 4; ++j) {
                if (4 * j < fl) {
                    const float4 xv = xs4[(tid * kXS) / 4 + j];
                    const double x0 = xv.x, x1 = xv.y, x2 = xv.z, x3 = xv.w;
                    xx = fma(x0, x0, xx);
                    xx = fma(x1, x1, xx);
                    xx = fma(x2, x2, xx);
                    xx = fma(x3, x3, xx);
#pragma unroll
                    for (int t = 0; t < TP; ++t) {
                        double v = acc[t];
                        v = fma(x0, cs[t][4 * j], v);
                        v = fma(x1, cs[t][4 * j + 1], v);
                        v = fma(x2, cs[t][4 * j + 2], v);
                        v = fma(x3, cs[t][4 * j + 3], v);
                        acc[t] = v;
                    }
                }
            }
        }
        if (tid < TP) ccs[tid] = cc;
        __syncthreads();
        // distances, minima with the closest so far, block sums
#pragma unroll
        for (int t = 0; t < TP; ++t) {
            double part = 0.0;
            if (t < tn) {
                float m = 0.f;
                if (live) {
                    float d32 = (float)((-2.0 * acc[t] + ccs[t]) + xx);
                    if (d32 < 0.f) d32 = 0.f;
                    m = d32 < closest ? d32 : closest;
                    a.D[p][(long)(t0 + t) * a.n + row] = m;
                }
                part = wave_sum((double)m);
            }
            if (lane == 0) red[wv][t] = part;
        }
        __syncthreads();
        if (tid < tn)
            a.P[p][(long)(t0 + tid) * a.nb + blockIdx.x] = ((red[0][tid] + red[1][tid]) + red[2][tid]) + red[3][tid];
    }
}

// Inclusive scan over the 64 lanes of a wave (fixed order).
__device__ __forceinline__ double wave_scan(double v, int lane)
{
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const double u = __shfl_up(v, off, 64);
        if (lane >= off) v += u;
    }
    return v;
}

__global__ __launch_bounds__(1024) void k_pp_select(PPArgs a, int c)
{
    __shared__ double wpot[16][kPPMaxTrials];
    __shared__ double wsum[16];
    __shared__ double rv[kPPMaxTrials];
    __shared__ int found[kPPMaxTrials];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int q = (c - 1) & 1;
    const int Tq = c == 1 ? 1 : a.T;

    // centre c - 1: the candidate of least potential (first one on ties);
    // each potential is a fixed-order sum of the block partials
    for (int t = 0; t < Tq; ++t) {
        double v = 0.0;
        for (int b = tid; b < a.nb; b += 1024) v += a.P[q][(long)t * a.nb + b];
        v = wave_sum(v);
        if (lane == 0) wpot[wv][t] = v;
    }
    __syncthreads();
    if (tid < Tq) {
        double v = 0.0;
        for (int w = 0; w < 16; ++w) v += wpot[w][tid];
        rv[tid] = v;
    }
    __syncthreads();
    double bestpot = rv[0];
    int best = 0;
    for (int t = 1; t < Tq; ++t)
        if (rv[t] < bestpot) {
            bestpot = rv[t];
            best = t;
        }
    __syncthreads();
    const long crow = a.cand[best];
    if (tid == 0) {
        a.idx[c - 1] = crow;
        a.best[c - 1] = best;
        a.pot[c - 1] = bestpot;
    }
    for (int f = tid; f < a.ld; f += 1024) a.centers[(long)(c - 1) * a.ld + f] = a.X[crow * a.ld + f];
    if (c >= a.k) return;

    // centre c's draws
    const double pot32 = (double)(float)bestpot;
    for (int t = tid; t < a.T; t += 1024) {
        rv[t] = a.U[(long)(c - 1) * a.T + t] * pot32;
        found[t] = INT_MAX;
    }
    __syncthreads();

    // running sum over the blocks' sums; found[t] = first block reaching r_t
    const double* S = a.P[q] + (long)best * a.nb;
    double carry = 0.0;
    for (int b0 = 0; b0 < a.nb; b0 += 1024) {
        const int b = b0 + tid;
        const double v = wave_scan(b < a.nb ? S[b] : 0.0, lane);
        if (lane == 63) wsum[wv] = v;
        __syncthreads();
        double off = carry;
        for (int w = 0; w < wv; ++w) off += wsum[w];
        const double incl = off + v;
        if (b < a.nb) {
            a.pfx[b] = incl;
            for (int t = 0; t < a.T; ++t)
                if (incl >= rv[t]) atomicMin(&found[t], b);
        }
        for (int w = 0; w < 16; ++w) carry += wsum[w];
        __syncthreads();
    }

    // within that block: the first row whose running sum reaches r_t
    const float* Dq = a.D[q] + (long)best * a.n;
    for (int t = wv; t < a.T; t += 16) {
        const int b = found[t];
        long pick = a.n - 1;
        if (b != INT_MAX) {
            double base = b > 0 ? a.pfx[b - 1] : 0.0;
            const long r0 = (long)b * kPPRows, r1 = min(a.n, r0 + (long)kPPRows);
            pick = r1 - 1;
            for (long r = r0; r < r1; r += 64) {
                const long i = r + lane;
                const double v = wave_scan(i < r1 ? (double)Dq[i] : 0.0, lane);
                const unsigned long long m = __ballot(i < r1 && base + v >= rv[t]);
                if (m != 0ull) {
                    pick = r + __ffsll((long long)m) - 1;
                    break;
                }
                base += __shfl(v, 63, 64);
            }
        }
        if (lane == 0) a.cand[t] = pick;
    }
}

}  // namespace

hipError_t launch_pp_dist(const PPArgs& a, int c, hipStream_t s)
{
    const dim3 grid((unsigned)a.nb), block(256);
    if (c == 0)
        hipLaunchKernelGGL(k_pp_dist<1>, grid, block, 0, s, a, 0, 1);
    else if (a.T <= 4)
        hipLaunchKernelGGL(k_pp_dist<4>, grid, block, 0, s, a, c, a.T);
    else if (a.T <= 8)
        hipLaunchKernelGGL(k_pp_dist<8>, grid, block, 0, s, a, c, a.T);
    else
        hipLaunchKernelGGL(k_pp_dist<16>, grid, block, 0, s, a, c, a.T);
    return hipGetLastError();
}

hipError_t launch_pp_select(const PPArgs& a, int c, hipStream_t s)
{
    hipLaunchKernelGGL(k_pp_select, dim3(1), dim3(1024), 0, s, a, c);
    return hipGetLastError();
}

}  // namespace skm
