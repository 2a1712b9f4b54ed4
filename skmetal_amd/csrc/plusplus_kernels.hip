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
//   k_pp_rows(c)    (rows of at most 128 floats, at most 8 candidates; else
//   k_pp_dist(c))   one lane per row: the distance to each candidate in
//                   sklearn's form for fp32 data (_euclidean_distances_upcast:
//                   fp64 -2 x.c + ||c||^2 + ||x||^2, cast to fp32, negatives
//                   to 0), min with the row's closest distance so far, and
//                   per-block fp64 sums of those minima.  k_pp_select also
//                   leaves the drawn candidates' values as fp64 for k_pp_rows.
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
// block's kPPRows rows go through LDS one 32-feature segment at a time: eight
// lanes load one row's 128-byte run (coalesced), then thread r works on row r.
// ||x||^2 and the candidates' ||c||^2 come from the same staged values.
//
// MIN = true (k-means||): the row's running minimum over every candidate so
// far, a.mind[row], is updated with the Tc candidates (started from +inf when
// a.mind_reset); no per-candidate minima or block sums are written.
template <int TP, bool MIN = false>
__global__ __launch_bounds__(kPPRows) void k_pp_dist(PPArgs a, int c, int Tc)
{
    __shared__ float4 xs4[kPPRows * kXS / 4];
    __shared__ double cs[TP][kFS];
    __shared__ double ccs[TP];
    constexpr int NW = kPPRows / 64;  // waves
    constexpr int RG = kPPRows / 8;   // rows loaded per instruction (8 lanes a row)
    __shared__ double red[NW][TP];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const long r0 = (long)blockIdx.x * kPPRows;
    const long row = r0 + tid;
    const bool live = row < a.n;
    const int p = c & 1;
    float closest = INFINITY;
    if (MIN) {
        if (!a.mind_reset && live) closest = a.mind[row];
    } else if (c > 0 && live) {
        closest = a.D[p ^ 1][(long)a.best[c - 1] * a.n + row];
    }

    for (int t0 = 0; t0 < Tc; t0 += TP) {
        const int tn = min(TP, Tc - t0);
        double acc[TP];
#pragma unroll
        for (int t = 0; t < TP; ++t) acc[t] = 0.0;
        double xx = 0.0, cc = 0.0;
        // segment f0's runs: lane group tid >> 3 loads rows (tid >> 3) + RG i
        const int q = tid & 7;
        float4 pre[8];
        auto load_seg = [&](int f0) {
            const int fl = min(kFS, a.ld - f0);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int lr = (tid >> 3) + RG * i;
                pre[i] = make_float4(0.f, 0.f, 0.f, 0.f);
                if (4 * q < fl && r0 + lr < a.n) pre[i] = *reinterpret_cast<const float4*>(a.X + (r0 + lr) * a.ld + f0 + 4 * q);
            }
        };
        // the candidates' values of a segment: element e = tid + kPPRows j is
        // feature e % kFS (= tid % kFS) of candidate e / kFS; they are loaded
        // with the segment's rows, so no dependent load waits between barriers
        constexpr int CE = (TP * kFS + kPPRows - 1) / kPPRows;
        long coff[CE];
        float cpre[CE];
#pragma unroll
        for (int j = 0; j < CE; ++j) {
            const int t = (tid + kPPRows * j) / kFS;
            coff[j] = t < tn ? a.cand[t0 + t] * a.ld : -1;
        }
        auto load_cand = [&](int f0) {
            const int f = tid % kFS;
#pragma unroll
            for (int j = 0; j < CE; ++j) {
                cpre[j] = 0.f;
                if (coff[j] >= 0 && f < a.ld - f0) cpre[j] = a.X[coff[j] + f0 + f];
            }
        };
        load_seg(0);
        load_cand(0);
        for (int f0 = 0; f0 < a.ld; f0 += kFS) {
            const int fl = min(kFS, a.ld - f0);  // a multiple of 4 (ld is)
            __syncthreads();
#pragma unroll
            for (int i = 0; i < 8; ++i) xs4[(((tid >> 3) + RG * i) * kXS) / 4 + q] = pre[i];
#pragma unroll
            for (int j = 0; j < CE; ++j) {
                const int e = tid + kPPRows * j;
                if (e < TP * kFS) (&cs[0][0])[e] = (double)cpre[j];
            }
            __syncthreads();
            if (f0 + kFS < a.ld) {  // in flight during this segment's work
                load_seg(f0 + kFS);
                load_cand(f0 + kFS);
            }
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
        if (MIN) {
            // the next pass rewrites ccs only after its first segment barrier
#pragma unroll
            for (int t = 0; t < TP; ++t)
                if (t < tn && live) {
                    float d32 = (float)((-2.0 * acc[t] + ccs[t]) + xx);
                    if (d32 < 0.f) d32 = 0.f;
                    closest = d32 < closest ? d32 : closest;
                }
            continue;
        }
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
        {
            double v = red[0][tid];
#pragma unroll
            for (int w = 1; w < NW; ++w) v += red[w][tid];
            a.P[p][(long)(t0 + tid) * a.nb + blockIdx.x] = v;
        }
    }
    if (MIN && live) a.mind[row] = closest;
}

// Rows of at most LDM floats, exactly TP candidates, one pass.  The block's
// 256-row range (the unit of the block sums) is read as four 64-row
// sub-groups, each a contiguous span of X loaded whole by the block (a float4
// a thread per instruction, every cache line once) and staged in LDS with
// row stride ctg_stride(ld); the next sub-group's loads are in flight while
// one is worked on.  Lane l of every wave takes row l of the sub-group; wave
// w takes its float4 chunks w, w + 4, ..., so the candidates' values a wave
// needs at a step are the same for all its lanes: they come through the
// scalar cache straight from X.  The four waves' partial sums meet in LDS
// and are added in wave order; wave 3 - w then finishes candidates w, w + 4,
// ... (wave 0 has the most chunks when ld / 4 is not a multiple of 4).
// Blocks are persistent over the 256-row ranges (b, b + gridDim.x, ...).
//
// TAB: the candidates' values as fp64 from a.ctab ([ld / 4][TP][4], written
// by k_pp_select), not converted from X by every wave, and each row's ||x||^2
// from a.xxn, which the launch without TAB (the first centre) writes.
template <int TP, int LDM, bool TAB>
__global__ __launch_bounds__(256) void k_pp_rows(PPArgs a, int c)
{
    typedef const __attribute__((address_space(4))) f4v sf4v;  // uniform loads: scalar cache
    typedef const __attribute__((address_space(4))) double sdbl;
    constexpr int SMAX = ctg_stride(LDM);
    constexpr int NV = (16 * LDM + 255) / 256;  // float4s a thread loads per sub-group
    constexpr int NU = (TP + 3) / 4;            // candidates a wave finishes
    constexpr int NJ = (LDM / 4 + 3) / 4;       // chunks a wave works on
    __shared__ __attribute__((aligned(16))) float tile[64 * SMAX];
    constexpr int NR = TAB ? TP : TP + 1;        // partial sums per lane (+ ||x||^2)
    __shared__ double red[4][NR][64];
    __shared__ double ccs[TP];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tw = 3 - w;  // this wave finishes candidates tw, tw + 4, ...
    const int ld = a.ld, c4 = ld / 4, S = ctg_stride(ld);
    const long n = a.n;
    const long nsg = (n + 63) / 64;
    const int p = c & 1;
    sf4v* Xs = (sf4v*)a.X;
    sdbl* Cs = (sdbl*)a.ctab;
    const f4v* X4 = reinterpret_cast<const f4v*>(a.X);
    long coff[TP];  // candidate t's row, in float4s
#pragma unroll
    for (int t = 0; t < TP; ++t) coff[t] = a.cand[t] * c4;
    const float* Dprev = c > 0 ? a.D[p ^ 1] + (long)a.best[c - 1] * n : nullptr;

    // ||c_t||^2 in feature order, one lane a candidate
    if (w == 0 && lane < TP) {
        long o = 0;
#pragma unroll
        for (int t = 0; t < TP; ++t)
            if (t == lane) o = coff[t];
        double cc = 0.0;
#pragma unroll 4
        for (int j = 0; j < c4; ++j) {
            const f4v v = X4[o + j];
            cc = fma((double)v.x, (double)v.x, cc);
            cc = fma((double)v.y, (double)v.y, cc);
            cc = fma((double)v.z, (double)v.z, cc);
            cc = fma((double)v.w, (double)v.w, cc);
        }
        ccs[lane] = cc;
    }

    // thread tid's float4s q = tid + 256 i of a full sub-group: tile offsets
    int off[NV];
    const float inv_c4 = 1.0f / (float)c4;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int q = tid + 256 * i;
        const int r = (int)(((float)q + 0.5f) * inv_c4);
        off[i] = r * S + 4 * (q - r * c4);
    }
    f4v P[NV];
    float pclose = INFINITY;
    double pxx = 0.0;
    auto load = [&](long sg) {
        const long r0 = 64 * sg;
        const int e4 = (int)(min(64L, n - r0) * c4);
        const f4v* base = X4 + r0 * c4;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int q = tid + 256 * i;
            if (q < e4) P[i] = base[q];
        }
        if (tw < TP) {
            const long rr = min(r0 + lane, n - 1);
            if (Dprev != nullptr) pclose = Dprev[rr];
            if constexpr (TAB) pxx = a.xxn[rr];
        }
    };

    double lsum[NU];  // the lane's minima over the 256-row range's sub-groups
#pragma unroll
    for (int u = 0; u < NU; ++u) lsum[u] = 0.0;
    long blk = blockIdx.x;
    int s = 0;
    if (4 * blk < nsg) load(4 * blk);
    while (blk < a.nb) {
        const long sg = 4 * blk + s;
        const long r0 = 64 * sg;
        const int e4 = (int)max(0L, min(64L, n - r0) * c4);
        __syncthreads();  // every wave is done with the tile and red
#pragma unroll
        for (int i = 0; i < NV; ++i)
            if (tid + 256 * i < e4) *reinterpret_cast<f4v*>(tile + off[i]) = P[i];
        const float closest = pclose;
        const double rxx = pxx;
        const long nxt = s == 3 ? 4 * (blk + gridDim.x) : sg + 1;
        if (nxt < nsg) load(nxt);  // in flight while this sub-group is worked on
        __syncthreads();

        double acc[TP], xx = 0.0;
#pragma unroll
        for (int t = 0; t < TP; ++t) acc[t] = 0.0;
        const float* xr = tile + lane * S;
#pragma unroll
        for (int i = 0; i < NJ; ++i) {
            const int j = w + 4 * i;
            if (j < c4) {
                const f4v xv = *reinterpret_cast<const f4v*>(xr + 4 * j);
                const double x0 = xv.x, x1 = xv.y, x2 = xv.z, x3 = xv.w;
                if constexpr (!TAB) {
                    xx = fma(x0, x0, xx);
                    xx = fma(x1, x1, xx);
                    xx = fma(x2, x2, xx);
                    xx = fma(x3, x3, xx);
                }
#pragma unroll
                for (int t = 0; t < TP; ++t) {
                    double c0, c1, c2, c3;
                    if constexpr (TAB) {
                        sdbl* cp = Cs + 4 * (j * TP + t);
                        c0 = cp[0];
                        c1 = cp[1];
                        c2 = cp[2];
                        c3 = cp[3];
                    } else {
                        const f4v cv = Xs[coff[t] + j];
                        c0 = cv.x;
                        c1 = cv.y;
                        c2 = cv.z;
                        c3 = cv.w;
                    }
                    double v = acc[t];
                    v = fma(x0, c0, v);
                    v = fma(x1, c1, v);
                    v = fma(x2, c2, v);
                    v = fma(x3, c3, v);
                    acc[t] = v;
                }
            }
        }
#pragma unroll
        for (int t = 0; t < TP; ++t) red[w][t][lane] = acc[t];
        if constexpr (!TAB) red[w][NR - 1][lane] = xx;
        __syncthreads();

        // wave 3 - tw finishes candidates tw, tw + 4, ...: sums in wave
        // order, the distance in sklearn's fp32-data form, min with the
        // closest so far
        const long row = r0 + lane;
        const bool live = row < n;
        if (tw < TP) {
            double x2 = rxx;
            if constexpr (!TAB) {
                x2 = ((red[0][NR - 1][lane] + red[1][NR - 1][lane]) + red[2][NR - 1][lane]) + red[3][NR - 1][lane];
                if (tw == 0 && live && a.xxn != nullptr) a.xxn[row] = x2;
            }
#pragma unroll
            for (int u = 0; u < NU; ++u) {
                const int t = tw + 4 * u;
                if (t < TP) {
                    const double dot = ((red[0][t][lane] + red[1][t][lane]) + red[2][t][lane]) + red[3][t][lane];
                    float m = 0.f;
                    if (live) {
                        float d32 = (float)((-2.0 * dot + ccs[t]) + x2);
                        if (d32 < 0.f) d32 = 0.f;
                        m = d32 < closest ? d32 : closest;
                        a.D[p][(long)t * n + row] = m;
                    }
                    lsum[u] += (double)m;
                }
            }
        }
        if (++s == 4) {  // the range's sums: each lane's four rows, then the lanes
#pragma unroll
            for (int u = 0; u < NU; ++u) {
                const int t = tw + 4 * u;
                if (t < TP) {
                    const double v = wave_sum(lsum[u]);
                    if (lane == 0) a.P[p][(long)t * a.nb + blk] = v;
                }
                lsum[u] = 0.0;
            }
            s = 0;
            blk += gridDim.x;
        }
    }
}

// k-means|| rounds on the fp64 matrix cores: the m candidates as the B
// operands of v_mfma_f64_16x16x4_f64 in 16-candidate groups,
// bfrag[(g ld/4 + j) 64 + l] = candidate 16 g + l % 16, feature 4 j + l / 16
// (fp64; candidates past m - 1 repeat it, which leaves every minimum as it
// is), and ||c_t||^2 (fp64 fmas in feature order), ccn[t], t < 16 G.
__global__ __launch_bounds__(256) void k_pp_bfrag(PPArgs a, int m)
{
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    const int ld = a.ld, c4 = ld / 4;
    const int G = (m + 15) / 16;
    if (i < (long)G * c4 * 64) {
        const int l = (int)(i & 63);
        const long gj = i >> 6;
        const int g = (int)(gj / c4), j = (int)(gj - (long)g * c4);
        const int t = min(16 * g + (l & 15), m - 1);
        a.ctab[i] = (double)a.X[a.cand[t] * ld + 4 * j + (l >> 4)];
    }
    if (i < 16L * G) {  // rows of at most 128 floats: the row's loads all in flight, then the fmas
        const f4v* x = reinterpret_cast<const f4v*>(a.X + a.cand[min((int)i, m - 1)] * ld);
        f4v v[32];
#pragma unroll
        for (int j = 0; j < 32; ++j)
            if (4 * j < ld) v[j] = x[j];
        double cc = 0.0;
#pragma unroll
        for (int j = 0; j < 32; ++j)
            if (4 * j < ld) {
                cc = fma((double)v[j].x, (double)v[j].x, cc);
                cc = fma((double)v[j].y, (double)v[j].y, cc);
                cc = fma((double)v[j].z, (double)v[j].z, cc);
                cc = fma((double)v[j].w, (double)v[j].w, cc);
            }
        a.ccn[i] = cc;
    }
}

// k-means||: a.mind[row] = min(a.mind[row] (+inf with a.mind_reset), the
// distance to each of the m candidates), rows of at most LDM floats.  The
// rows go through LDS in 64-row sub-groups as in k_pp_rows; wave w takes
// rows 16 w .. 16 w + 15 of a sub-group and, per 16-candidate group, chains
// ld / 4 v_mfma_f64_16x16x4_f64 over the features: the fp64 matrix cores
// add the exact products x_f c_f one at a time in feature order, the same
// sums as a sequential fma chain.  Lane l then holds rows l / 16 + 4 r,
// candidate l % 16.
template <int LDM>
__global__ __launch_bounds__(256, 4) void k_pp_mm_min(PPArgs a, int m)
{
    typedef double v4d __attribute__((ext_vector_type(4)));
    constexpr int SMAX = ctg_stride(LDM);
    constexpr int NV = (16 * LDM + 255) / 256;
    constexpr int NJ = LDM / 4;
    __shared__ __attribute__((aligned(16))) float tile[64 * SMAX];
    __shared__ double sxx[64];  // ||x||^2 of the sub-group's rows
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ld = a.ld, c4 = ld / 4, S = ctg_stride(ld);
    const long n = a.n;
    const long nsg = (n + 63) / 64;
    const f4v* X4 = reinterpret_cast<const f4v*>(a.X);
    const int G = (m + 15) / 16;
    const int q = lane >> 4, cj = lane & 15;
    // the row this lane writes (lanes with cj < 4): 16 w + q + 4 cj
    const int orow = 16 * w + q + 4 * cj;

    int off[NV];
    const float inv_c4 = 1.0f / (float)c4;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int qq = tid + 256 * i;
        const int r = (int)(((float)qq + 0.5f) * inv_c4);
        off[i] = r * S + 4 * (qq - r * c4);
    }
    f4v P[NV];
    float pclose = INFINITY;
    auto load = [&](long sg) {
        const long r0 = 64 * sg;
        const int e4 = (int)(min(64L, n - r0) * c4);
        const f4v* base = X4 + r0 * c4;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int qq = tid + 256 * i;
            if (qq < e4) P[i] = base[qq];
        }
        if (cj < 4 && !a.mind_reset) pclose = a.mind[min(r0 + orow, n - 1)];
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
        const float closest = pclose;
        if (sg + gridDim.x < nsg) load(sg + gridDim.x);  // in flight while this one is worked on
        __syncthreads();

        // ||x||^2 of the wave's 16 rows in feature order (lanes 0..15), then
        // each lane takes its four rows' values
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

        float best[4] = {INFINITY, INFINITY, INFINITY, INFINITY};
        const float* ar = tile + (16 * w + cj) * S + q;  // A: row cj, feature 4 j + q
        // two groups at a time: two independent chains share the A values
        for (int g = 0; g < G; g += 2) {
            const bool two = g + 1 < G;  // wave-uniform
            const double* bf = a.ctab + ((long)g * c4 << 6) + lane;
            const double* bf2 = two ? bf + ((long)c4 << 6) : bf;  // (in bounds either way)
            v4d acc = {0.0, 0.0, 0.0, 0.0}, acc2 = {0.0, 0.0, 0.0, 0.0};
            // four K steps at a time: their B fragments and A values loaded together
            for (int j0 = 0; j0 < c4; j0 += 4) {
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
                if (p == 1 && !two) break;
                const double cn = a.ccn[16 * (g + p) + cj];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float d32 = (float)((-2.0 * (p == 0 ? acc[r] : acc2[r]) + cn) + xxr[r]);
                    if (d32 < 0.f) d32 = 0.f;
                    best[r] = d32 < best[r] ? d32 : best[r];
                }
            }
        }
        // min over the 16 candidate lanes of each row (lanes 16 q .. 16 q + 15)
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) {
                const float u = __shfl_xor(best[r], o, 64);
                best[r] = u < best[r] ? u : best[r];
            }
        if (cj < 4 && r0 + orow < n) {
            const float b = cj == 0 ? best[0] : cj == 1 ? best[1] : cj == 2 ? best[2] : best[3];
            a.mind[r0 + orow] = b < closest ? b : closest;
        }
        __builtin_amdgcn_wave_barrier();  // sxx is rewritten only after the next block barrier
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
    constexpr int RPL = kPPRows / 64;  // rows per lane in the row search
    static_assert(kPPRows % 64 == 0, "the row search gives each lane whole rows");
    constexpr int TB = 8;  // candidates whose partials are summed together
    __shared__ double wsum[16];
    __shared__ double wpot[16][TB];
    __shared__ double rv[kPPMaxTrials];
    __shared__ int found[kPPMaxTrials];
    __shared__ long picks[kPPMaxTrials];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int q = (c - 1) & 1;
    const int Tq = c == 1 ? 1 : a.T;

    // centre c - 1: the candidate of least potential (first one on ties).
    // Each potential is a fixed-order sum of the block partials: thread i adds
    // its blocks (the loads of TB candidates in flight together), then a
    // butterfly per wave, then the 16 waves in order.  With at most TB
    // candidates and 2048 blocks, thread i owns blocks [m i, m i + m), the
    // same blocks as in the running sum below, which then takes the chosen
    // candidate's values from these registers instead of loading them again;
    // otherwise thread i adds blocks i, i + 1024, ...
    const int m = (a.nb + 1023) / 1024;
    const int b0 = m * tid, b1 = min(a.nb, b0 + m);
    const bool regs = Tq <= TB && m <= 2;  // block-uniform
    double pv[TB][2];
    for (int t0 = 0; t0 < Tq; t0 += TB) {
        double v[TB];
#pragma unroll
        for (int t = 0; t < TB; ++t) v[t] = 0.0;
        if (regs) {
#pragma unroll
            for (int t = 0; t < TB; ++t)
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    pv[t][i] = t < Tq && b0 + i < b1 ? a.P[q][(long)t * a.nb + b0 + i] : 0.0;
#pragma unroll
            for (int t = 0; t < TB; ++t)
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    if (b0 + i < b1) v[t] += pv[t][i];
        } else {
            for (int b = tid; b < a.nb; b += 1024) {
#pragma unroll
                for (int t = 0; t < TB; ++t)
                    if (t0 + t < Tq) v[t] += a.P[q][(long)(t0 + t) * a.nb + b];
            }
        }
#pragma unroll
        for (int t = 0; t < TB; ++t) {
            const double w = wave_sum(v[t]);
            if (lane == 0) wpot[wv][t] = w;
        }
        __syncthreads();
        if (tid < TB && t0 + tid < Tq) {
            double w = 0.0;
            for (int i = 0; i < 16; ++i) w += wpot[i][tid];
            rv[t0 + tid] = w;
        }
        __syncthreads();
    }
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

    // running sum over the blocks' sums in one pass: thread i owns blocks
    // [m i, m i + m); its start is the scan of the thread totals before it.
    // found[t] = the first block whose running sum reaches r_t.
    const double* S = a.P[q] + (long)best * a.nb;
    double sv0 = 0.0, sv1 = 0.0;  // the register path's values of S[b0], S[b0 + 1]
    if (regs) {
#pragma unroll
        for (int t = 0; t < TB; ++t)
            if (t == best) {
                sv0 = pv[t][0];
                sv1 = pv[t][1];
            }
    }
    auto sval = [&](int b) { return regs ? (b == b0 ? sv0 : sv1) : S[b]; };
    double own = 0.0;
    for (int b = b0; b < b1; ++b) own += sval(b);
    const double incl = wave_scan(own, lane);
    if (lane == 63) wsum[wv] = incl;
    double excl = __shfl_up(incl, 1, 64);
    if (lane == 0) excl = 0.0;
    __syncthreads();  // wsum, rv and found
    double run0 = 0.0;
    for (int w = 0; w < wv; ++w) run0 += wsum[w];
    run0 += excl;
    double run = run0;
    for (int b = b0; b < b1; ++b) {
        run += sval(b);
        a.pfx[b] = run;
    }
    // a thread's running sum only grows, so the first lane of a wave whose last
    // value reaches r_t holds the wave's first such block: it alone finds it
    // (the same additions again) and posts it
    for (int t = 0; t < a.T; ++t) {
        const unsigned long long msk = __ballot(b0 < b1 && run >= rv[t]);
        if (msk != 0ull && lane == __ffsll((long long)msk) - 1) {
            double r = run0;
            int bf = b1 - 1;
            for (int b = b0; b < b1; ++b) {
                r += sval(b);
                if (r >= rv[t]) {
                    bf = b;
                    break;
                }
            }
            atomicMin(&found[t], bf);
        }
    }
    __syncthreads();

    // within that block: the first row whose running sum reaches r_t; lane l
    // holds rows RPL l .. RPL l + RPL - 1 of the block, all loaded at once
    const float* Dq = a.D[q] + (long)best * a.n;
    for (int t = wv; t < a.T; t += 16) {
        const int b = found[t];
        long pick = a.n - 1;
        if (b != INT_MAX) {
            const double base = b > 0 ? a.pfx[b - 1] : 0.0;
            const long r0 = (long)b * kPPRows, r1 = min(a.n, r0 + (long)kPPRows);
            const long i0 = r0 + RPL * lane;
            float dv[RPL];
#pragma unroll
            for (int j = 0; j < RPL; ++j) dv[j] = i0 + j < r1 ? Dq[i0 + j] : 0.f;
            double sj[RPL], acc = 0.0;
#pragma unroll
            for (int j = 0; j < RPL; ++j) {
                acc += (double)dv[j];
                sj[j] = acc;
            }
            const double inc = wave_scan(acc, lane);
            double ex = __shfl_up(inc, 1, 64);
            if (lane == 0) ex = 0.0;
            const double lb = base + ex;
            int jf = RPL;
#pragma unroll
            for (int j = RPL - 1; j >= 0; --j)
                if (i0 + j < r1 && lb + sj[j] >= rv[t]) jf = j;
            const unsigned long long msk = __ballot(jf < RPL);
            pick = r1 - 1;
            if (msk != 0ull) {
                const int L = __ffsll((long long)msk) - 1;
                pick = r0 + RPL * L + __shfl(jf, L, 64);
            }
        }
        if (lane == 0) {
            a.cand[t] = pick;
            picks[t] = pick;
        }
    }
    // the candidates' values as fp64 for k_pp_rows: ctab[f / 4][t][f % 4]
    if (a.ctab != nullptr) {
        __syncthreads();
        const int e = a.T * a.ld;
        for (int i = tid; i < e; i += 1024) {
            const int t = i / a.ld, f = i - t * a.ld;
            a.ctab[((f >> 2) * a.T + t) * 4 + (f & 3)] = (double)a.X[picks[t] * a.ld + f];
        }
    }
}

typedef void (*pp_rows_fn)(PPArgs, int);

template <int LDM, int... TPs>
struct PPRowsTable {
    static pp_rows_fn get(int T, bool tab)
    {
        pp_rows_fn f = nullptr;
        ((T == TPs ? (f = tab ? &k_pp_rows<TPs, LDM, true> : &k_pp_rows<TPs, LDM, false>, 0) : 0), ...);
        return f;
    }
};

template <int LDM>
pp_rows_fn pp_rows_for(int T, bool tab)
{
    return PPRowsTable<LDM, 1, 2, 3, 4, 5, 6, 7, 8>::get(T, tab);
}

// Resident blocks per CU of a k_pp_rows instance (cached).
int pp_rows_occupancy(pp_rows_fn f)
{
    static pp_rows_fn keys[32];
    static int vals[32];
    static int used = 0;
    for (int i = 0; i < used; ++i)
        if (keys[i] == f) return vals[i];
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, reinterpret_cast<const void*>(f), 256, 0) != hipSuccess ||
        nb < 1)
        nb = 1;
    if (used < 32) {
        keys[used] = f;
        vals[used] = nb;
        ++used;
    }
    return nb;
}

}  // namespace

hipError_t launch_pp_dist(const PPArgs& a, int c, hipStream_t s)
{
    const dim3 grid((unsigned)a.nb), block(kPPRows);
    // one pass over X for T <= 16 (the candidate count exactly for T <= 8,
    // the usual 2 + ln k), passes of 16 beyond
    const int T = c == 0 ? 1 : a.T;
    if (pp_rows_path(T, a.ld)) {  // whole rows through LDS, candidates through the scalar cache
        const bool tab = c > 0 && a.ctab != nullptr;  // k_pp_select wrote centre c's table; launch 0 wrote xxn
        const pp_rows_fn f = a.ld <= 32 ? pp_rows_for<32>(T, tab)
                             : a.ld <= 64 ? pp_rows_for<64>(T, tab)
                             : a.ld <= 104 ? pp_rows_for<104>(T, tab)
                                           : pp_rows_for<128>(T, tab);
        const long cap = (long)(a.cus > 0 ? a.cus : 256) * pp_rows_occupancy(f);
        const unsigned g = (unsigned)(a.nb < cap ? a.nb : cap);
        hipLaunchKernelGGL(f, dim3(g), dim3(256), 0, s, a, c);
        return hipGetLastError();
    }
    switch (T) {
    case 1: hipLaunchKernelGGL(k_pp_dist<1>, grid, block, 0, s, a, c, T); break;
    case 2: hipLaunchKernelGGL(k_pp_dist<2>, grid, block, 0, s, a, c, T); break;
    case 3: hipLaunchKernelGGL(k_pp_dist<3>, grid, block, 0, s, a, c, T); break;
    case 4: hipLaunchKernelGGL(k_pp_dist<4>, grid, block, 0, s, a, c, T); break;
    case 5: hipLaunchKernelGGL(k_pp_dist<5>, grid, block, 0, s, a, c, T); break;
    case 6: hipLaunchKernelGGL(k_pp_dist<6>, grid, block, 0, s, a, c, T); break;
    case 7: hipLaunchKernelGGL(k_pp_dist<7>, grid, block, 0, s, a, c, T); break;
    case 8: hipLaunchKernelGGL(k_pp_dist<8>, grid, block, 0, s, a, c, T); break;
    default:
        if (T <= 12) hipLaunchKernelGGL(k_pp_dist<12>, grid, block, 0, s, a, c, T);
        else hipLaunchKernelGGL(k_pp_dist<16>, grid, block, 0, s, a, c, T);
    }
    return hipGetLastError();
}

hipError_t launch_pp_mindist(const PPArgs& a, int m, hipStream_t s)
{
    // a round of at most 4 candidates (the first, against the first row) on
    // the VALU kernel: the matrix cores would pad it to 16 (62 against 77 us at
    // 500000 x 100); the sums are the same fma chains in feature order
    if (m > 4 && pp_rows_min_path(a.ld) && a.ctab != nullptr && a.ccn != nullptr) {
        if (m > 0) {
            const long e = (long)(m + 15) / 16 * 16 * a.ld;  // G ld/4 64 fragments
            hipLaunchKernelGGL(k_pp_bfrag, dim3((unsigned)((e + 255) / 256)), dim3(256), 0, s, a, m);
        }
        const pp_rows_fn f = a.ld <= 32 ? &k_pp_mm_min<32>
                             : a.ld <= 64 ? &k_pp_mm_min<64>
                             : a.ld <= 104 ? &k_pp_mm_min<104>
                                           : &k_pp_mm_min<128>;
        const long nsg = (a.n + 63) / 64;
        const long cap = (long)(a.cus > 0 ? a.cus : 256) * pp_rows_occupancy(f);
        const unsigned g = (unsigned)(nsg < cap ? nsg : cap);
        hipLaunchKernelGGL(f, dim3(g), dim3(256), 0, s, a, m);
        return hipGetLastError();
    }
    const dim3 grid((unsigned)a.nb), block(kPPRows);
    if (m <= 8)
        hipLaunchKernelGGL((k_pp_dist<8, true>), grid, block, 0, s, a, 0, m);
    else if (m <= 16)
        hipLaunchKernelGGL((k_pp_dist<16, true>), grid, block, 0, s, a, 0, m);
    else  // passes of 32 (64 at once holds one wave per SIMD: twice the time)
        hipLaunchKernelGGL((k_pp_dist<32, true>), grid, block, 0, s, a, 0, m);
    return hipGetLastError();
}

hipError_t launch_pp_select(const PPArgs& a, int c, hipStream_t s)
{
    hipLaunchKernelGGL(k_pp_select, dim3(1), dim3(1024), 0, s, a, c);
    return hipGetLastError();
}

}  // namespace skm
