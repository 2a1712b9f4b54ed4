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
#include <stdlib.h>

#include "device.h"

namespace skm {

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

template <int KG, int NQ>
__global__ __launch_bounds__(256, 1) void k_assign(const float* __restrict__ X, long n, int ld,
                                                   const float* __restrict__ C,
                                                   const float* __restrict__ cnorm, int k,
                                                   int* __restrict__ labels, LoopState* st,
                                                   int* changed)
{
    if (st != nullptr && st->done != 0) return;
    constexpr int CPC = 4 * KG;   // clusters per chunk
    constexpr int SEG = 4 * NQ;   // features per segment
    constexpr int LS = SEG + 4;   // LDS row stride (floats): conflict-free b128 reads
    __shared__ __attribute__((aligned(16))) float sC[CPC * LS];
    __shared__ float sN[CPC];
    __shared__ int sChg;  // labels the block changed

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: keeps descriptors scalar
    if (tid == 0) sChg = 0;  // (published by the first staging barrier, or read back by this thread)
    int nchg = 0;            // lane 0: labels this wave changed
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
        const long row0 = base + wave * 64;
        const long row = row0 + lane;
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
                load_row_quads<NQ>(xv, X, row0, n, ld, f0, nq, lane);
                // past nq both operands are 0 (zero-filled stage, zero loads)
#pragma unroll
                for (int q = 0; q < NQ; ++q) {
                    const float4 cv = *reinterpret_cast<const float4*>(&sC[crow * LS + 4 * q]);
                    mfma_groups<KG>(acc, cv.x, xv[q].x);
                    mfma_groups<KG>(acc, cv.y, xv[q].y);
                    mfma_groups<KG>(acc, cv.z, xv[q].z);
                    mfma_groups<KG>(acc, cv.w, xv[q].w);
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
        int moved = 0;
        if (row < n) {
            if (changed != nullptr) moved = labels[row] != bidx;
            labels[row] = bidx;
        }
        if (changed != nullptr) nchg += (int)__popcll(__ballot(moved));
    }
    // one global atomic per block: a wave-level atomic per 64 rows on one
    // address serialises thousands of them while labels move
    if (changed != nullptr) {
        if (lane == 0 && nchg != 0) atomicAdd(&sChg, nchg);
        __syncthreads();
        if (tid == 0 && sChg != 0) atomicAdd(changed, sChg);
    }
}

typedef void (*assign_fn)(const float*, long, int, const float*, const float*, int, int*, LoopState*, int*);

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
                       a.state, a.changed);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// update: per-(row range, cluster group, column tile) sums and counts
// ---------------------------------------------------------------------------
//
// Block (r, g, z) handles rows [r*rpr, (r+1)*rpr), clusters [g*cg, (g+1)*cg)
// and columns [z*W, (z+1)*W).  Its threads form `nslots` row slots of `ct`
// column threads; slot s owns a contiguous half/quarter of the rows and its
// own LDS table S_s[cg x dt].  A slot walks its rows in batches of kUB: the
// batch's labels are uniform across the slot, so duplicates inside a batch are
// folded in registers first (in row order) and every distinct label then costs
// one LDS read-modify-write -- one LDS round trip per batch instead of per row,
// and the kUB row loads of a batch are all in flight together.  Column c of
// S_s is only touched by one thread, and the slots are summed in slot order at
// the end, so each partial is bitwise reproducible.  Rows outside the group
// are skipped without loading X, so X is read once overall.

constexpr int kUB = 8;     // rows per batch
constexpr int kLCH = 256;  // labels staged per slot and chunk

template <int NCP>
__global__ __launch_bounds__(256) void k_update(const float* __restrict__ X, long n, int ld, int d,
                                                const int* __restrict__ labels, int k, int cg, long rpr,
                                                int nslots, int W, float* __restrict__ psum,
                                                int* __restrict__ pcnt, const LoopState* st)
{
    if (st != nullptr && st->done != 0) return;
    extern __shared__ float smem[];
    const int T = blockDim.x;
    const int ct = T / nslots;
    const int slot = threadIdx.x / ct;
    const int lt = threadIdx.x - slot * ct;
    const int r = blockIdx.x;
    const int j0 = blockIdx.y * cg;
    const int j1 = min(k, j0 + cg);
    const int col0 = blockIdx.z * W;
    const int dt = min(d - col0, W);
    const long row0 = (long)r * rpr;
    const long row1 = min(n, row0 + rpr);
    const long per = (row1 - row0 + nslots - 1) / nslots;
    const long a = min(row1, row0 + (long)slot * per);
    const long b = min(row1, a + per);
    float* S = smem + (long)slot * cg * dt;
    int* cnt_all = reinterpret_cast<int*>(smem + (long)nslots * cg * dt);
    int* cnt = cnt_all + slot * cg;
    int* sLab = cnt_all + nslots * cg + slot * kLCH;
    for (int i = threadIdx.x; i < nslots * cg * dt; i += T) smem[i] = 0.f;
    for (int i = threadIdx.x; i < nslots * cg; i += T) cnt_all[i] = 0;

    for (long base = 0; base < per; base += kLCH) {
        __syncthreads();
        for (int i = lt; i < kLCH; i += ct) {
            const long row = a + base + i;
            int lab = -1;
            if (row < b) {
                lab = labels[row];
                lab = (lab >= j0 && lab < j1) ? lab - j0 : -1;
            }
            sLab[i] = lab;
        }
        __syncthreads();
        const int m = (int)min((long)kLCH, max(0L, b - a - base));
        for (int i0 = 0; i0 < m; i0 += kUB) {
            int lj[kUB], dup[kUB];
#pragma unroll
            for (int u = 0; u < kUB; ++u) lj[u] = __builtin_amdgcn_readfirstlane(i0 + u < m ? sLab[i0 + u] : -1);
#pragma unroll
            for (int u = 0; u < kUB; ++u) {
                dup[u] = -1;
#pragma unroll
                for (int v = 0; v < u; ++v)
                    if (dup[u] < 0 && lj[u] >= 0 && dup[v] < 0 && lj[v] == lj[u]) dup[u] = v;
            }
            if (lt == 0) {
#pragma unroll
                for (int u = 0; u < kUB; ++u)
                    if (lj[u] >= 0) cnt[lj[u]] += 1;
            }
            const float* xb = X + (a + base + i0) * ld + col0;
#pragma unroll
            for (int p = 0; p < NCP; ++p) {
                const int c = lt + p * ct;
                if (c < dt) {
                    float v[kUB];
#pragma unroll
                    for (int u = 0; u < kUB; ++u) v[u] = lj[u] >= 0 ? xb[(long)u * ld + c] : 0.f;
#pragma unroll
                    for (int u = 1; u < kUB; ++u) {
#pragma unroll
                        for (int w = 0; w < u; ++w)
                            if (dup[u] == w) v[w] += v[u];
                    }
                    float o[kUB];
#pragma unroll
                    for (int u = 0; u < kUB; ++u)
                        if (lj[u] >= 0 && dup[u] < 0) o[u] = S[lj[u] * dt + c];
#pragma unroll
                    for (int u = 0; u < kUB; ++u)
                        if (lj[u] >= 0 && dup[u] < 0) S[lj[u] * dt + c] = o[u] + v[u];
                }
            }
        }
    }
    __syncthreads();
    const int ncl = j1 - j0;
    for (int idx = threadIdx.x; idx < ncl * dt; idx += T) {
        const int jl = idx / dt;
        const int c = idx - jl * dt;
        float acc = 0.f;
        for (int q = 0; q < nslots; ++q) acc += smem[(long)q * cg * dt + idx];
        psum[((long)r * k + j0 + jl) * ld + col0 + c] = acc;
    }
    if (blockIdx.z == 0) {
        for (int jl = threadIdx.x; jl < ncl; jl += T) {
            int c2 = 0;
            for (int q = 0; q < nslots; ++q) c2 += cnt_all[q * cg + jl];
            pcnt[(long)r * k + j0 + jl] = c2;
        }
    }
}

UpdateGeom update_geometry(long n, int d, int k, int num_cu)
{
    UpdateGeom g{};
    const int ct = d >= 256 ? 256 : ((d + 63) / 64) * 64;
    g.nslots = 256 / ct;
    g.ncp = d <= ct ? 1 : d <= 2 * ct ? 2 : 4;
    g.W = ct * g.ncp;
    g.Z = (d + g.W - 1) / g.W;
    const long words = 16 * 1024 - (long)g.nslots * kLCH;  // 64 KB of LDS per block
    g.cg = (int)max(1L, min((long)k, words / ((long)g.nslots * (min(d, g.W) + 1))));
    g.G = (k + g.cg - 1) / g.cg;
    g.threads = 256;
    long R = (2L * num_cu) / ((long)g.G * g.Z);
    const long min_r = (n + 32767) / 32768;  // bound the label scan of one block
    if (R < min_r) R = min_r;
    if (R < 1) R = 1;
    const long max_r = (n + 255) / 256;
    if (R > max_r) R = max_r;
    g.R = (int)R;
    g.rows_per_range = (n + R - 1) / R;
    const int dt = min(d, g.W);
    g.lds = ((size_t)g.nslots * g.cg * dt + (size_t)g.nslots * g.cg + (size_t)g.nslots * kLCH) * 4;
    return g;
}

hipError_t launch_update(const UpdateArgs& a, const UpdateGeom& g, hipStream_t s)
{
    if (a.n <= 0) return hipSuccess;
    const dim3 grid(g.R, g.G, g.Z);
    if (g.ncp == 1)
        hipLaunchKernelGGL(k_update<1>, grid, dim3(g.threads), g.lds, s, a.X, a.n, a.ld, a.d, a.labels, a.k, g.cg,
                           g.rows_per_range, g.nslots, g.W, a.psum, a.pcnt, a.state);
    else if (g.ncp == 2)
        hipLaunchKernelGGL(k_update<2>, grid, dim3(g.threads), g.lds, s, a.X, a.n, a.ld, a.d, a.labels, a.k, g.cg,
                           g.rows_per_range, g.nslots, g.W, a.psum, a.pcnt, a.state);
    else
        hipLaunchKernelGGL(k_update<4>, grid, dim3(g.threads), g.lds, s, a.X, a.n, a.ld, a.d, a.labels, a.k, g.cg,
                           g.rows_per_range, g.nslots, g.W, a.psum, a.pcnt, a.state);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// sorted update (generic path): counting sort by label + segmented sums
// ---------------------------------------------------------------------------
//
// 1. k_label_hist   a block per range of wr rows: LDS histogram of labels.
// 2. k_label_segs   column sums of the range histograms per segment of
//                   kSortSeg ranges.
// 3. k_label_scan   one block: per-cluster counts, exclusive scan over
//                   clusters (first sorted position), chunk spans and record
//                   offsets, and per-segment bases.
// 4. k_label_offs   range offsets: start_j + rows of cluster j in earlier
//                   ranges.
// 5. k_label_scatter_lds  a block of four waves per range (k_label_scatter,
//                   one wave, when its LDS does not fit): row ids and labels
//                   to their sorted positions (ranges in order, rows in order
//                   inside a cluster; inside a wave instruction the LDS
//                   atomic hands out the positions).
// 6. k_segsum       a group of G threads sums one chunk of B sorted rows,
//                   segment by segment (the rows of one cluster are
//                   consecutive), gathering each X row once; a segment's sum
//                   is the record (cluster, chunk).
// The finalize then folds cluster j's records in chunk order.  X is read
// once; labels a few times (4 bytes per row).

// Exclusive prefix sum over a 256-thread block; *total gets the block's sum.
// sh: 4 ints.  Ends with a barrier.
__device__ int block_excl_scan(int v, int* sh, int* total)
{
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int x = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
    }
    if (lane == 63) sh[w] = x;
    __syncthreads();
    int base = 0, tot = 0;
    for (int i = 0; i < 4; ++i) {
        base += i < w ? sh[i] : 0;
        tot += sh[i];
    }
    __syncthreads();
    *total = tot;
    return base + x - v;
}

// The sort kernels read the halt flag beside their first loads and test it
// once those are in flight (a test first put a memory round trip before
// every kernel's work).
__global__ __launch_bounds__(256) void k_label_hist(SortArgs a, int wr)
{
    const int done = a.state->done;
    extern __shared__ int h[];
    const int tid = threadIdx.x;
    for (int j = tid; j < a.k; j += 256) h[j] = 0;
    const long r0 = (long)blockIdx.x * wr;
    const int nr = (int)(min(a.n, r0 + wr) - r0);
    // the labels 16 rows a thread at a time, all in flight before the
    // first is counted (integer adds: any order gives the same counts)
    constexpr int U = 16;
    int lv[U];
    auto load = [&](int q0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int q = q0 + 256 * u + tid;
            lv[u] = q < nr ? a.labels[r0 + q] : -1;
        }
    };
    load(0);
    if (done != 0) return;
    __syncthreads();  // h cleared
    for (int q0 = 0; q0 < nr; q0 += 256 * U) {
        if (q0 > 0) load(q0);
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (lv[u] >= 0) atomicAdd(&h[lv[u]], 1);
    }
    __syncthreads();
    int* out = a.hist + (long)blockIdx.x * a.k;
    for (int j = tid; j < a.k; j += 256) out[j] = h[j];
}

__global__ __launch_bounds__(256) void k_label_segs(SortArgs a, int nw)
{
    const int done = a.state->done;
    const int j = blockIdx.x * 256 + threadIdx.x;
    if (j >= a.k) return;
    const int w0 = blockIdx.y * kSortSeg;
    const int w1 = min(nw, w0 + kSortSeg);
    int v[kSortSeg];
#pragma unroll
    for (int i = 0; i < kSortSeg; ++i) v[i] = a.hist[(long)min(w0 + i, w1 - 1) * a.k + j];  // all in flight
    if (done != 0) return;
    int s = 0;
#pragma unroll
    for (int i = 0; i < kSortSeg; ++i) s += w0 + i < w1 ? v[i] : 0;
    a.segsum[(long)blockIdx.y * a.k + j] = s;
}

// Exclusive scan of v over the 1024 threads of the block (v per thread).
__device__ int block_exclusive_scan(int v, int* sh)
{
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    int x = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
    }
    if (lane == 63) sh[tid >> 6] = x;
    __syncthreads();
    if (tid < 16) {
        int w = sh[tid];
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) {
            const int y = __shfl_up(w, off, 16);
            if (tid >= off) w += y;
        }
        sh[16 + tid] = w;
    }
    __syncthreads();
    const int base = (tid >> 6) > 0 ? sh[16 + (tid >> 6) - 1] : 0;
    __syncthreads();
    return base + x - v;
}

__global__ __launch_bounds__(1024) void k_label_scan(SortArgs a, int nseg, int B)
{
    const int done = a.state->done;
    __shared__ int sh[32];
    __shared__ int sc[16384];  // cluster j's count, then its span of chunks (k <= 16384)
    const int tid = threadIdx.x;
    const int per = (a.k + 1023) / 1024;  // clusters per thread, contiguous
    const int j0 = tid * per;
    const int j1 = min(a.k, j0 + per);
    // counts, and per-segment bases relative to the cluster's start; the
    // first cluster's loads go out before the halt flag is tested
    int v[kSortSeg];
    auto load = [&](int j) {
#pragma unroll
        for (int s = 0; s < kSortSeg; ++s) v[s] = a.segsum[(long)min(s, nseg - 1) * a.k + j];  // all in flight
    };
    if (j0 < j1) load(j0);
    if (done != 0) return;
    int tot = 0;
    for (int j = j0; j < j1; ++j) {
        if (j > j0) load(j);
        int run = 0;
#pragma unroll
        for (int s = 0; s < kSortSeg; ++s) {
            if (s < nseg) {
                a.segsum[(long)s * a.k + j] = run;
                run += v[s];
            }
        }
        a.counts[j] = run;
        sc[j] = run;
        tot += run;
    }
    int pos = block_exclusive_scan(tot, sh);
    int spans = 0;
    for (int j = j0; j < j1; ++j) {
        a.start[j] = pos;
        const int c = sc[j];
        const int span = c > 0 ? (pos + c - 1) / B - pos / B + 1 : 0;
        a.rec_cnt[j] = span;
        sc[j] = span;
        spans += span;
        pos += c;
    }
    int rec = block_exclusive_scan(spans, sh);
    for (int j = j0; j < j1; ++j) {
        a.rec_off[j] = rec;
        rec += sc[j];
    }
}

__global__ __launch_bounds__(256) void k_label_offs(SortArgs a, int nw)
{
    const int done = a.state->done;
    const int j = blockIdx.x * 256 + threadIdx.x;
    if (j >= a.k) return;
    const int w0 = blockIdx.y * kSortSeg;
    const int w1 = min(nw, w0 + kSortSeg);
    int v[kSortSeg];
#pragma unroll
    for (int i = 0; i < kSortSeg; ++i) v[i] = a.hist[(long)min(w0 + i, w1 - 1) * a.k + j];  // all in flight
    const int st = a.start[j], sb = a.segsum[(long)blockIdx.y * a.k + j];
    if (done != 0) return;
    int run = st + sb;
#pragma unroll
    for (int i = 0; i < kSortSeg; ++i) {
        if (w0 + i < w1) a.hist[(long)(w0 + i) * a.k + j] = run;
        run += v[i];
    }
}

// Range w of the nw: blocks are dealt to the 8 XCDs in turn (block b on XCD
// b % 8), and XCD x takes ranges [x per, (x + 1) per), per = ceil(nw / 8):
// consecutive ranges fill consecutive positions of every cluster's run, so
// a cache line two neighbouring ranges share is completed in one L2.
__device__ __forceinline__ int scatter_range(int nw)
{
    const int per = (nw + 7) / 8, w = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
    return (int)(blockIdx.x >> 3) < per && w < nw ? w : -1;
}

// One wave per range: each row's sorted position from an LDS counter per
// cluster (inside a wave instruction the LDS atomic hands out the positions
// in lane order), the row id and label stored there.
__global__ __launch_bounds__(64) void k_label_scatter(SortArgs a, int wr, int nw)
{
    if (a.state->done != 0) return;
    const int w = scatter_range(nw);
    if (w < 0) return;
    extern __shared__ int ctr[];
    const int* off = a.hist + (long)w * a.k;
    for (int j = threadIdx.x; j < a.k; j += 64) ctr[j] = off[j];
    __syncthreads();
    const long r0 = (long)w * wr;
    const long r1 = min(a.n, r0 + wr);
    for (long r = r0 + threadIdx.x; r < r1; r += 64) {
        const int l = a.labels[r];
        const int p = atomicAdd(&ctr[l], 1);
        a.perm[p] = (int)r;
        a.slab[p] = l;
    }
}

// As k_label_scatter, with the range's output staged in LDS: the rows are
// first placed in the range's own cluster order, then written out in that
// order, so that each cluster's run of the range goes out in one pass of
// consecutive stores instead of a few entries at a time over the whole
// kernel (lines written in pieces and evicted in between: 7x the bytes at
// 4M rows and 1024 clusters).  A block of four waves per range, wave s
// taking the s-th quarter of its rows: (1) each wave counts its quarter's
// rows per cluster, (2) the range's staged layout -- cluster j's run starts
// at lst[j], the exclusive prefix over j of its rows, and quarter s's rows
// of j follow quarters 0 .. s-1's -- (3) each wave places its rows with an
// LDS counter per (quarter, cluster): inside a wave instruction the LDS
// atomic hands out positions in lane order, so every cluster's rows stay in
// row order, the order a single wave over the range gives; (4) the staged
// entries go to their sorted positions.  (One wave per range left a SIMD
// with one wave at 4M rows: 41 us.)  Dynamic LDS: cnt (4 k ints, the counts
// and then the counters), off and lst (k each), the staged row ids and
// labels (wr each).
__global__ __launch_bounds__(256) void k_label_scatter_lds(SortArgs a, int wr, int nw)
{
    const int done = a.state->done;
    const int w = scatter_range(nw);
    if (w < 0) return;
    extern __shared__ int sl[];
    const int k = a.k;
    int* cnt = sl;            // [4][k] rows of cluster j in quarter s, then quarter s's next staged position
    int* off = sl + 4 * k;    // [k] first sorted position of the range's rows of cluster j
    int* lst = off + k;       // [k] first staged position of those rows
    int* sperm = lst + k;     // [wr]
    int* slab = sperm + wr;   // [wr]
    __shared__ int shi[4];
    const int tid = threadIdx.x, lane = tid & 63, s = tid >> 6;
    const long r0 = (long)w * wr;
    const int nr = (int)(min(a.n, r0 + wr) - r0);
    const int qs = (nr + 3) / 4;  // rows per quarter
    const int q0 = min(nr, s * qs), q1 = min(nr, q0 + qs);
    for (int i = tid; i < 4 * k; i += 256) cnt[i] = 0;
    // this thread's contiguous clusters for (2); the range's offsets are
    // requested now
    const int per = (k + 255) / 256;
    const int j0 = min(k, tid * per), j1 = min(k, j0 + per);
    const int* o = a.hist + (long)w * k;
    for (int jb = 0; jb < k; jb += 1024) {
        int v[4];
#pragma unroll
        for (int f = 0; f < 4; ++f) {
            const int j = jb + 256 * f + tid;
            v[f] = j < k ? o[j] : 0;
        }
#pragma unroll
        for (int f = 0; f < 4; ++f) {
            const int j = jb + 256 * f + tid;
            if (j < k) off[j] = v[f];
        }
    }
    if (done != 0) return;
    __syncthreads();
    // (1) the labels 16 rows a lane at a time, all in flight before the
    // first is counted
    constexpr int U = 16;
    for (int qb = q0; qb < q1; qb += 64 * U) {
        int lv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int q = qb + 64 * u + lane;
            lv[u] = q < q1 ? a.labels[r0 + q] : -1;
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (lv[u] >= 0) atomicAdd(&cnt[s * k + lv[u]], 1);
    }
    __syncthreads();
    // (2) the staged layout
    int mine = 0;
    for (int j = j0; j < j1; ++j) mine += (cnt[j] + cnt[k + j]) + (cnt[2 * k + j] + cnt[3 * k + j]);
    int tot;
    int run = block_excl_scan(mine, shi, &tot);
    for (int j = j0; j < j1; ++j) {
        lst[j] = run;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int c = cnt[t * k + j];
            cnt[t * k + j] = run;
            run += c;
        }
    }
    __syncthreads();
    // (3) the rows placed, quarter by quarter (labels read again: the L2)
    for (int qb = q0; qb < q1; qb += 64 * U) {
        int lv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int q = qb + 64 * u + lane;
            lv[u] = q < q1 ? a.labels[r0 + q] : 0;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int q = qb + 64 * u + lane;
            if (q < q1) {
                const int p = atomicAdd(&cnt[s * k + lv[u]], 1);
                sperm[p] = (int)(r0 + q);
                slab[p] = lv[u];
            }
        }
    }
    __syncthreads();
    // (4) four entries a thread at a time: their LDS reads overlap
    constexpr int F = 4;
    for (int qb = 0; qb < nr; qb += 256 * F) {
        int l[F], pr[F];
#pragma unroll
        for (int f = 0; f < F; ++f) {
            const int q = min(qb + 256 * f + tid, nr - 1);
            l[f] = slab[q];
            pr[f] = sperm[q];
        }
#pragma unroll
        for (int f = 0; f < F; ++f) {
            const int q = qb + 256 * f + tid;
            if (q < nr) {
                const int p = off[l[f]] + (q - lst[l[f]]);
                a.perm[p] = pr[f];
                a.slab[p] = l[f];
            }
        }
    }
}

// LDS of k_label_scatter_lds (0: it does not fit; k_label_scatter then).
constexpr size_t kScatterLdsMax = 150 * 1024;
static size_t scatter_lds_bytes(int k, int wr)
{
    const size_t b = ((size_t)6 * k + (size_t)2 * wr) * sizeof(int);
    return b <= kScatterLdsMax ? b : 0;
}

// Columns per thread: CPT * G >= the tile's columns (<= 1024 per grid row).
template <int CPT>
__global__ __launch_bounds__(256) void k_segsum(SortArgs a, int B, int G)
{
    const int done = a.state->done;
    constexpr int U = 64 / CPT;  // sorted rows per batch: 64 loads in flight per thread
    const int groups = 256 / G;  // G >= 64: a wave lies in one group
    const int grp = threadIdx.x / G;
    const int t = threadIdx.x - grp * G;
    const int lane = threadIdx.x & 63;
    const long c = (long)blockIdx.x * groups + grp;
    const long p0 = c * B;
    if (p0 >= a.n) return;
    const long p1 = min(a.n, p0 + B);
    const int col0 = blockIdx.y * 1024;
    int cols[CPT];
    bool on[CPT];
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
        cols[i] = col0 + t + i * G;
        on[i] = cols[i] < a.d && t + i * G < 1024;
    }
    float acc[CPT];
#pragma unroll
    for (int i = 0; i < CPT; ++i) acc[i] = 0.f;
    int cur = a.slab[p0];
    auto flush = [&](int j) {
        const long rec = a.rec_off[j] + (c - a.start[j] / B);
        float* dst = a.rec + rec * a.ld;
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            if (on[i]) dst[cols[i]] = acc[i];
            acc[i] = 0.f;
        }
    };
    // lane u holds the label and row id of sorted row p + u (clamped to the
    // chunk); a batch's ids are loaded one batch ahead, and each row's id is
    // read out of its lane, so the row loads have a scalar base
    int labv, ridv;
    auto load_ids = [&](long p) {
        const long q = min(p + lane, p1 - 1);
        labv = a.slab[q];
        ridv = a.perm[q];
    };
    load_ids(p0);
    if (done != 0) return;
    for (long p = p0; p < p1; p += U) {
        float v[U][CPT];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const float* row = a.X + (long)__builtin_amdgcn_readlane(ridv, u) * a.ld;
#pragma unroll
            for (int i = 0; i < CPT; ++i) v[u][i] = on[i] ? row[cols[i]] : 0.f;
        }
        const int labb = labv;
        if (p + U < p1) load_ids(p + U);
        const int nb = (int)min((long)U, p1 - p);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (u < nb) {
                const int lb = __builtin_amdgcn_readlane(labb, u);
                if (lb != cur) {
                    flush(cur);
                    cur = lb;
                }
#pragma unroll
                for (int i = 0; i < CPT; ++i) acc[i] += v[u][i];
            }
        }
    }
    flush(cur);
}

SortGeom sort_geometry(long n, int d, int ld, int k)
{
    SortGeom g;
    if (k > 16384 || n < 1) return g;  // LDS histogram of one wave: 64 KB
    long wr = (n + 1023) / 1024;
    wr = ((wr + 63) / 64) * 64;
    if (wr < 256) wr = 256;
    g.wr = (int)wr;
    g.nw = (int)((n + wr - 1) / wr);
    if ((long)g.nw * k > (64L << 20)) return g;
    g.nseg = (g.nw + kSortSeg - 1) / kSortSeg;
    const int dcols = ld < 1024 ? ld : 1024;
    g.G = dcols <= 64 ? 64 : dcols <= 128 ? 128 : 256;
    // chunks of B sorted rows (a multiple of 64), a group of G threads each:
    // about 8192 waves in all, 32 per CU, so that enough row gathers are in
    // flight (4M rows of 64 floats: 2,017 single-wave chunks summed at 4.9
    // TB/s, 7,813 at 5.3)
    const long wpc = g.G / 64;  // waves per chunk
    long B = (n * wpc + 8191) / 8192;
    B = ((B + 63) / 64) * 64;
    if (B < 64) B = 64;
    g.B = (int)B;
    g.nchunks = (n + B - 1) / B;
    g.max_records = k + g.nchunks;
    g.on = true;
    return g;
}

hipError_t launch_sorted_update(const SortArgs& a, const SortGeom& g, hipStream_t s)
{
    if (!g.on) return hipErrorInvalidValue;
    const size_t hlds = (size_t)a.k * sizeof(int);
    const unsigned kb = (unsigned)((a.k + 255) / 256);
    hipLaunchKernelGGL(k_label_hist, dim3(g.nw), dim3(256), hlds, s, a, g.wr);
    hipLaunchKernelGGL(k_label_segs, dim3(kb, g.nseg), dim3(256), 0, s, a, g.nw);
    hipLaunchKernelGGL(k_label_scan, dim3(1), dim3(1024), 0, s, a, g.nseg, g.B);
    hipLaunchKernelGGL(k_label_offs, dim3(kb, g.nseg), dim3(256), 0, s, a, g.nw);
    const size_t slds = scatter_lds_bytes(a.k, g.wr);
    if (slds > 0) {
        static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(k_label_scatter_lds),
                                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                                           (int)kScatterLdsMax);
        if (attr != hipSuccess) return attr;
        hipLaunchKernelGGL(k_label_scatter_lds, dim3(8 * ((g.nw + 7) / 8)), dim3(256), slds, s, a, g.wr, g.nw);
    } else {
        hipLaunchKernelGGL(k_label_scatter, dim3(8 * ((g.nw + 7) / 8)), dim3(64), hlds, s, a, g.wr, g.nw);
    }
    const int groups = 256 / g.G;
    const int dcols = a.d < 1024 ? a.d : 1024;
    const int cpt = (dcols + g.G - 1) / g.G;
    const dim3 grid((unsigned)((g.nchunks + groups - 1) / groups), (unsigned)((a.d + 1023) / 1024));
    if (cpt <= 1)
        hipLaunchKernelGGL(k_segsum<1>, grid, dim3(256), 0, s, a, g.B, g.G);
    else if (cpt == 2)
        hipLaunchKernelGGL(k_segsum<2>, grid, dim3(256), 0, s, a, g.B, g.G);
    else
        hipLaunchKernelGGL(k_segsum<4>, grid, dim3(256), 0, s, a, g.B, g.G);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// finalize: two kernels, no cross-block atomics or fences
// ---------------------------------------------------------------------------
//
// k_finalize_cols, block (j, cc): the R partial sums of cluster j, columns
// [32 cc, 32 cc + 32), reduced in a fixed order -- thread (rs, q) adds the
// float4 of columns 32 cc + 4q.. of partials rs, rs + 32, ... in fp64 (eight
// threads read one 128-byte run of a partial), the eight rs lanes of a wave
// are combined by an xor butterfly (every lane ends with bitwise the same
// value) and the four waves in wave order -- then the new centre, and the
// chunk's shift^2 and ||c||^2 partials.
// k_finalize_loop, one block: folds each cluster's chunk partials in chunk
// order and evaluates the loop's stopping rules (_kmeans.py:717-732).
// The kernel boundary makes the first kernel's stores visible to the second;
// agent-scope fences inside one kernel would write back and invalidate the
// L2 of every XCD for each block.

// Sum over a 256-thread block in a fixed order (wave butterflies, then waves
// 0..3); every thread gets the total.  `sh` holds 4 elements; the call ends
// with a barrier, so it may be reused right after.
template <typename T>
__device__ __forceinline__ T block_sum(T v, T* sh)
{
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    const T t = (sh[0] + sh[1]) + (sh[2] + sh[3]);
    __syncthreads();
    return t;
}

// Largest value over a 256-thread block (every thread gets it), as block_sum.
__device__ __forceinline__ float block_max(float v, float* sh)
{
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    const float t = fmaxf(fmaxf(sh[0], sh[1]), fmaxf(sh[2], sh[3]));
    __syncthreads();
    return t;
}

constexpr int kFinUnroll = 8;  // partials in flight per thread

// One (cluster j, column chunk cc of nch) of the finalize over R per-block
// partials (partial r of cluster j at r k + j); a whole block.  Lane (rs,
// q) = (thread / 8, thread % 8) adds the float4 of columns 32 cc + 4q of
// partials rs, rs + 32, .. in fp64.
__device__ __forceinline__ void finalize_cols_block(const FinalizeArgs& a, int j, int cc, int nch)
{
    const int tid = threadIdx.x;
    const int q = tid & 7;          // float4 column of the block
    const int rs = tid >> 3;        // partial lane, 0..31
    const int c4 = cc * 32 + 4 * q; // first column of this thread
    __shared__ double red[4][8][4];
    __shared__ int rcnt[4];

    // the halt flag, the old centres, each lane's first kFinUnroll partials
    // and the counts are all requested before any of them is used: one
    // memory round trip (a count loop that waited before the partials were
    // requested made it four)
    const int done = a.state->done;
    const int ccol = cc * 32 + tid;  // threads 0..31: one column each for the centre update
    const float c_old = tid < 32 && ccol < a.d ? a.C_old[(long)j * a.ld + ccol] : 0.f;
    const int R = a.R;
    const float* src = a.psum + (long)j * a.ld + c4;
    const long step = (long)a.k * a.ld;
    const bool live = c4 < a.ld && R > 0;  // ld is a multiple of 4: the float4 is in or out
    float4 v[kFinUnroll];
    if (live) {
#pragma unroll
        for (int u = 0; u < kFinUnroll; ++u) {
            const int r = rs + u * 32;
            v[u] = *reinterpret_cast<const float4*>(src + (long)(r < R ? r : R - 1) * step);
        }
    }
    int cnt = 0;
    for (int r = tid; r < R; r += 256) cnt += a.pcnt[(long)r * a.k + j];
    double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
    if (live) {
#pragma unroll
        for (int u = 0; u < kFinUnroll; ++u) {
            if (rs + u * 32 < R) {
                s0 += (double)v[u].x;
                s1 += (double)v[u].y;
                s2 += (double)v[u].z;
                s3 += (double)v[u].w;
            }
        }
        // R > 256 partials: further rounds in the same order
        for (int r0 = rs + kFinUnroll * 32; r0 < R; r0 += kFinUnroll * 32) {
#pragma unroll
            for (int u = 0; u < kFinUnroll; ++u) {
                const int r = r0 + u * 32;
                v[u] = *reinterpret_cast<const float4*>(src + (long)(r < R ? r : R - 1) * step);
            }
#pragma unroll
            for (int u = 0; u < kFinUnroll; ++u) {
                if (r0 + u * 32 < R) {
                    s0 += (double)v[u].x;
                    s1 += (double)v[u].y;
                    s2 += (double)v[u].z;
                    s3 += (double)v[u].w;
                }
            }
        }
    }
    if (done != 0) return;  // the loop has halted: nothing is written
    // the eight partial lanes of a wave (lane bits 3..5), then the waves
    for (int off = 8; off < 64; off <<= 1) {
        s0 += __shfl_xor(s0, off, 64);
        s1 += __shfl_xor(s1, off, 64);
        s2 += __shfl_xor(s2, off, 64);
        s3 += __shfl_xor(s3, off, 64);
    }
    cnt = wave_sum(cnt);
    if ((tid & 63) < 8) {
        red[tid >> 6][q][0] = s0;
        red[tid >> 6][q][1] = s1;
        red[tid >> 6][q][2] = s2;
        red[tid >> 6][q][3] = s3;
    }
    if ((tid & 63) == 0) rcnt[tid >> 6] = cnt;
    __syncthreads();  // red[] and rcnt[] from every wave
    if (tid >= 64) return;
    // wave 0: the count, then the new centres of the chunk's columns and
    // their shift^2 and ||c||^2 partials (fp64 sums over lanes 0..31 in a
    // fixed butterfly order; lanes 32..63 add zeros)
    const int count = (rcnt[0] + rcnt[1]) + (rcnt[2] + rcnt[3]);
    double sq = 0.0, nrm = 0.0;
    if (tid < 32 && ccol < a.d) {
        const int qq = tid >> 2, e = tid & 3;
        const double tot = ((red[0][qq][e] + red[1][qq][e]) + red[2][qq][e]) + red[3][qq][e];
        a.sums[(long)j * a.ld + ccol] = tot;
        if (count > 0) {
            const float cn = (float)(tot / (double)count);
            a.C_new[(long)j * a.ld + ccol] = cn;
            const double df = (double)cn - (double)c_old;
            sq = df * df;
            nrm = (double)cn * (double)cn;
        }
    }
    sq = wave_sum(sq);
    nrm = wave_sum(nrm);
    if (tid == 0) {
        a.part[((long)j * nch + cc) * 2 + 0] = sq;
        a.part[((long)j * nch + cc) * 2 + 1] = nrm;
        if (cc == 0) a.counts[j] = count;
        if (cc == 0 && count == 0) atomicAdd(&a.state->empty_cnt[a.iter & 1], 1);  // for k_reloc
        if (j == 0 && cc == 0) {
            if (a.chg_next != nullptr) *a.chg_next = 0;
            a.state->empty_cnt[(a.iter + 1) & 1] = 0;  // read by k_reloc of iteration iter - 1, which has run
        }
    }
}

__global__ __launch_bounds__(256) void k_finalize_cols(FinalizeArgs a)
{
    finalize_cols_block(a, blockIdx.x, blockIdx.y, gridDim.y);
}

// Record mode (the sorted update: a cluster has a few records, one per
// chunk of sorted rows it touches): one wave per (cluster j, column chunk
// cc), item 4 blockIdx.x + wave of k nch.  Lane (rs, q) = (lane / 8, lane %
// 8) adds the float4 of columns 32 cc + 4q of records rs, rs + 8, .. in
// fp64, and the eight rs lanes are combined by an xor butterfly.  A block
// per item made 98,304 blocks at 4096 clusters of 768 floats, each waiting
// on one round trip.
__global__ __launch_bounds__(256) void k_finalize_recs(FinalizeArgs a, int nch)
{
    const int lane = threadIdx.x & 63;
    const long item = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (item >= (long)a.k * nch) return;
    const int j = (int)(item / nch), cc = (int)(item - (long)j * nch);
    const int done = a.state->done;
    const int q = lane & 7, rs = lane >> 3;
    const int c4 = cc * 32 + 4 * q;
    const int ccol = cc * 32 + lane;  // lanes 0..31: one column each
    const float c_old = lane < 32 && ccol < a.d ? a.C_old[(long)j * a.ld + ccol] : 0.f;
    const int R = a.rec_cnt[j];
    const int count = a.cnt_in[j];
    const float* src = a.psum + (long)a.rec_off[j] * a.ld + c4;
    if (done != 0) return;  // tested once the loads above are in flight
    double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
    if (c4 < a.ld) {  // ld is a multiple of 4: the float4 is in or out
        for (int r = rs; r < R; r += 8) {
            const float4 v = *reinterpret_cast<const float4*>(src + (long)r * a.ld);
            s0 += (double)v.x;
            s1 += (double)v.y;
            s2 += (double)v.z;
            s3 += (double)v.w;
        }
    }
    for (int off = 8; off < 64; off <<= 1) {
        s0 += __shfl_xor(s0, off, 64);
        s1 += __shfl_xor(s1, off, 64);
        s2 += __shfl_xor(s2, off, 64);
        s3 += __shfl_xor(s3, off, 64);
    }
    // lane c < 32 takes column 32 cc + c: component c % 4 of lane c / 4
    const int e = lane & 3, src_lane = (lane >> 2) & 7;
    const double t0 = __shfl(s0, src_lane, 64), t1 = __shfl(s1, src_lane, 64);
    const double t2 = __shfl(s2, src_lane, 64), t3 = __shfl(s3, src_lane, 64);
    const double tot = e == 0 ? t0 : e == 1 ? t1 : e == 2 ? t2 : t3;
    double sq = 0.0, nrm = 0.0;
    if (lane < 32 && ccol < a.d) {
        a.sums[(long)j * a.ld + ccol] = tot;
        if (count > 0) {
            const float cn = (float)(tot / (double)count);
            a.C_new[(long)j * a.ld + ccol] = cn;
            const double df = (double)cn - (double)c_old;
            sq = df * df;
            nrm = (double)cn * (double)cn;
        }
    }
    sq = wave_sum(sq);
    nrm = wave_sum(nrm);
    if (lane == 0) {
        a.part[((long)j * nch + cc) * 2 + 0] = sq;
        a.part[((long)j * nch + cc) * 2 + 1] = nrm;
        if (cc == 0) a.counts[j] = count;
        if (cc == 0 && count == 0) atomicAdd(&a.state->empty_cnt[a.iter & 1], 1);  // for k_reloc
        if (j == 0 && cc == 0) {
            if (a.chg_next != nullptr) *a.chg_next = 0;
            a.state->empty_cnt[(a.iter + 1) & 1] = 0;  // read by k_reloc of iteration iter - 1, which has run
        }
    }
}

__global__ __launch_bounds__(256) void k_finalize_loop(FinalizeArgs a, int nch)
{
    LoopState* st = a.state;
    if (st->done != 0) return;
    const int tid = threadIdx.x;
    __shared__ double shd[4];
    __shared__ int shi[4];
    __shared__ float shm[4];
    int n_empty = 0;
    double tot = 0.0;
    float mx = 0.f;
    for (int j = tid; j < a.k; j += 256) {
        double tsq = 0.0, tnr = 0.0;
        for (int c = 0; c < nch; ++c) {
            tsq += a.part[((long)j * nch + c) * 2 + 0];
            tnr += a.part[((long)j * nch + c) * 2 + 1];
        }
        const int count = a.counts[j];
        a.shift_sq[j] = (float)tsq;
        if (count > 0 || a.after_reloc) a.cnorm[j] = (float)tnr;
        n_empty += count == 0;
        tot += (double)(float)tsq;
        mx = fmaxf(mx, (float)tsq);
    }
    n_empty = block_sum(n_empty, shi);
    tot = block_sum(tot, shd);
    mx = block_max(mx, shm);
    if (tid == 0) {
        const int changed = *a.chg_cur;
        st->n_empty = n_empty;
        st->shift_tot = tot;
        st->last_changed = changed;
        st->n_iter = a.iter + 1;
        int done = 0;
        if (n_empty > 0 && !a.after_reloc && st->reloc_iter != a.iter)
            done = 3;
        else if ((a.flags & kStopStrict) && changed == 0)
            done = 1;
        else if (shift_rule_stops(a.flags, a.tol, tot, mx))
            done = 2;
        if (done != 0) st->halt_iter = a.iter;
        st->done = done;
    }
}

hipError_t launch_finalize(const FinalizeArgs& a, hipStream_t s, bool with_loop)
{
    const int nch = finalize_col_chunks(a.d, a.R);
    if (a.rec_off != nullptr)
        hipLaunchKernelGGL(k_finalize_recs, dim3((unsigned)(((long)a.k * nch + 3) / 4)), dim3(256), 0, s, a, nch);
    else
        hipLaunchKernelGGL(k_finalize_cols, dim3(a.k, nch), dim3(256), 0, s, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || !with_loop) return e;
    return launch_finalize_loop(a, s);
}

hipError_t launch_finalize_loop(const FinalizeArgs& a, hipStream_t s, int nch)
{
    hipLaunchKernelGGL(k_finalize_loop, dim3(1), dim3(256), 0, s, a, nch > 0 ? nch : finalize_col_chunks(a.d, a.R));
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// rowdist: ||x_i - c_{label_i}||^2 and its fp64 total
// ---------------------------------------------------------------------------
//
// Per row in fp32, in the association order of sklearn's
// _euclidean_dense_dense (_k_means_common.pyx:16-43): groups of four squared
// differences summed left to right, each group added to the running sum, the
// remainder one by one.  Rows longer than 128 floats (rows_dist): a block
// takes a contiguous share of the rows, a wave 64 consecutive rows at a time;
// their features come in slabs of 32 columns, loaded coalesced (8 lanes per
// 128-byte piece of a row) into the wave's LDS tile, and lane l carries row
// l's running sum from slab to slab.  Shorter rows take the contiguous path
// (rows_dist_ctg) below.  The total is summed in fp64: each lane over its
// rows, then the lanes and waves of a block, then the blocks in order.

constexpr int kRowSlab = 32;                  // columns per slab
constexpr int kRowPiece = kRowSlab / 4;       // float4s per row of a slab = lanes per row in a load
constexpr int kRowVec = kRowSlab / 4;         // float4s per lane per slab (64 rows x kRowSlab / 64 lanes / 4)
constexpr int kRowTileStride = kRowSlab + 1;  // floats per tile row: lane l's column reads spread over the banks
constexpr int kRowTileFloats = 64 * kRowTileStride;

// Squared distances of rows [r0, r1) to their centres into dist (nullable);
// returns the lane's fp64 total over its rows.  Wave w takes the 64-row
// chunks r0 + 64 w + 256 t, lane l row l of a chunk, a 32-column slab at a
// time; the slab's float4 q = 64 i + lane (row q / 8, columns 4 (q % 8)..)
// is loaded coalesced into the wave's LDS tile, and each slab's loads are
// issued before the previous slab is summed.  Out-of-range parts of a slab
// load clamped addresses and are never summed.  A row whose label is
// outside [0, k) counts 0.
__device__ __forceinline__ double rows_dist(const float* __restrict__ X, int ld, int d, const float* __restrict__ C,
                            const int* __restrict__ labels, int k, long r0, long r1, float* __restrict__ dist,
                            float* tile)
{
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int ns = (d + kRowSlab - 1) / kRowSlab;
    long c0 = r0 + 64L * w;
    double total = 0.0;
    if (c0 >= r1) return total;
    float4 v[kRowVec];
    auto load = [&](long cc, int sl) {
        const int f0 = sl * kRowSlab;
        const int wd4 = ((min(kRowSlab, d - f0) + 3) & ~3) - 4;  // last float4 of the slab in the row
        const int last = (int)min(64L, r1 - cc) - 1;
#pragma unroll
        for (int i = 0; i < kRowVec; ++i) {
            const int q = 64 * i + lane;
            const int r = min(q / kRowPiece, last), c4 = min(4 * (q % kRowPiece), wd4);
            v[i] = *reinterpret_cast<const float4*>(X + (cc + r) * ld + f0 + c4);
        }
    };
    load(c0, 0);
    int sl = 0;
    float res = 0.f;
    bool ok = false;
    const float* crow = C;
    while (c0 < r1) {
        const long row = c0 + lane;
        if (sl == 0) {
            const int lab = row < r1 ? labels[row] : -1;
            ok = lab >= 0 && lab < k;
            crow = C + (long)(ok ? lab : 0) * ld;
            res = 0.f;
        }
        const int f0 = sl * kRowSlab, wd = min(kRowSlab, d - f0);
        const int wd4 = ((wd + 3) & ~3) - 4;
        float4 cv[kRowVec];
#pragma unroll
        for (int i = 0; i < kRowVec; ++i) cv[i] = *reinterpret_cast<const float4*>(crow + f0 + min(4 * i, wd4));
        // the centre loads go out before the next slab's (the sums then wait
        // for them alone)
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < kRowVec; ++i) {
            const int q = 64 * i + lane;
            float* t = tile + (q / kRowPiece) * kRowTileStride + 4 * (q % kRowPiece);
            t[0] = v[i].x;
            t[1] = v[i].y;
            t[2] = v[i].z;
            t[3] = v[i].w;
        }
        // (a wave's LDS accesses complete in order: the tile is written
        // before any lane reads it)
        __builtin_amdgcn_wave_barrier();
        long nc0 = c0;
        int nsl = sl + 1;
        if (nsl == ns) {
            nsl = 0;
            nc0 += 256;
        }
        // in flight while this slab is summed; past the last job the current
        // slab loads again, so every pass issues the same loads (the wait
        // counts before the sums then cover only the centre loads)
        load(nc0 < r1 ? nc0 : c0, nc0 < r1 ? nsl : sl);
        {  // every lane sums (a row without a valid label uses centre 0 and is dropped below)
            const float* t = tile + lane * kRowTileStride;
#pragma unroll
            for (int i = 0; i < kRowVec; ++i) {
                if (4 * i + 4 <= wd) {
                    const float t0 = t[4 * i] - cv[i].x, t1 = t[4 * i + 1] - cv[i].y;
                    const float t2 = t[4 * i + 2] - cv[i].z, t3 = t[4 * i + 3] - cv[i].w;
                    res += ((t0 * t0 + t1 * t1) + t2 * t2) + t3 * t3;
                } else if (4 * i < wd) {  // the row's last features, one by one
                    float tt = t[4 * i] - cv[i].x;
                    res += tt * tt;
                    if (4 * i + 1 < wd) {
                        tt = t[4 * i + 1] - cv[i].y;
                        res += tt * tt;
                    }
                    if (4 * i + 2 < wd) {
                        tt = t[4 * i + 2] - cv[i].z;
                        res += tt * tt;
                    }
                }
            }
        }
        __builtin_amdgcn_wave_barrier();  // every lane is done with the tile
        if (sl == ns - 1 && row < r1) {
            if (dist != nullptr) dist[row] = ok ? res : 0.f;
            total += ok ? (double)res : 0.0;
        }
        c0 = nc0;
        sl = nsl;
    }
    return total;
}

// Rows of at most LDM floats (ld <= LDM, a multiple of 4) take a contiguous
// path: a wave takes the ROWS-row chunks (ROWS = 32 or 64) r0 + ROWS w +
// wstep t; a chunk's rows are one span of ROWS ld floats, loaded as
// lane-linear float4s (whole cache lines) and stored as float4s into the
// wave's LDS tile with row stride S = ctg_stride(ld), an odd number of
// 16-byte units, so that the row-per-lane float4 reads of the sums fall in
// distinct bank groups; lane l < ROWS sums row l of the chunk in the
// association order above.  The column slabs of rows_dist read 128-byte
// pieces of rows that need not start on a cache line, and fetch such lines
// twice when their neighbours have left the L2 in between.
// The centre rows come from Cs, row stride cs: with CL the block's LDS copy
// of C, read group by group in a loop over the row's whole float4s; else C
// itself, each chunk's centre float4s loaded into registers before the next
// chunk's loads are issued, so the sums wait for the centres alone.
template <int LDM, int ROWS>
struct CtgGeom {
    static constexpr int NV = ROWS * LDM / 256;       // float4 loads per lane per chunk, at most
    static constexpr int NG = LDM / 4;                // float4 groups per row, at most
    static constexpr int SMAX = 4 * ((LDM / 4) | 1);  // largest tile row stride
    static constexpr int TILE = ROWS * SMAX;          // floats per wave tile
};

struct NoPrologue {
    __device__ void operator()() const {}
};

// ld: the row stride, a multiple of 4 (<= LDM); row r's distance goes to
// dist[r - dbase] (nullable); tile: the wave's ROWS ctg_stride(ld) floats;
// pro: block-wide set-up run by every wave once its first chunk's loads are
// in flight.  As rows_dist otherwise.
template <int LDM, int ROWS, bool CL, typename Pro = NoPrologue>
__device__ __forceinline__ double rows_dist_ctg(const float* __restrict__ X, int ld, int d,
                                                const float* __restrict__ Cs, int cs,
                                                const int* __restrict__ labels, int k, long r0, long r1,
                                                long wstep, float* __restrict__ dist, long dbase, float* tile,
                                                Pro pro = Pro())
{
#pragma clang fp contract(off)
    using G = CtgGeom<LDM, ROWS>;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int S = ctg_stride(ld);
    const float inv_ld = 1.0f / (float)ld;
    long c0 = r0 + (long)ROWS * w;
    double total = 0.0;
    f4v P[G::NV];
    int plab = -1;
    // loads past a chunk's span repeat its last float4 (NV covers LDM)
    auto load = [&](long cc) {
        const int nrows = (int)min((long)ROWS, r1 - cc);
        const int e4 = nrows * ld / 4;  // float4s of the chunk's rows
        const f4v* base = reinterpret_cast<const f4v*>(X + cc * ld);
#pragma unroll
        for (int i = 0; i < G::NV; ++i) P[i] = base[min(64 * i + lane, e4 - 1)];
        plab = labels[cc + min(lane, nrows - 1)];
    };
    // float p = 4 q of a span: row p / ld (p + 1/2 keeps the float quotient
    // clear of integers), column p % ld; a repeated float4 goes where the
    // span's last one goes (same value)
    auto tile_off = [&](int i, int e4) {
        const int p = 4 * min(64 * i + lane, e4 - 1);
        const int r = (int)(((float)p + 0.5f) * inv_ld);
        return r * S + (p - r * ld);
    };
    int off[G::NV];  // a whole chunk's tile offsets
#pragma unroll
    for (int i = 0; i < G::NV; ++i) off[i] = tile_off(i, ROWS * ld / 4);
    if (c0 < r1) load(c0);
    pro();
    while (c0 < r1) {
        const int nrows = (int)min((long)ROWS, r1 - c0);
        if (nrows == ROWS) {
#pragma unroll
            for (int i = 0; i < G::NV; ++i) *reinterpret_cast<f4v*>(tile + off[i]) = P[i];
        } else {
            const int e4 = nrows * ld / 4;
#pragma unroll
            for (int i = 0; i < G::NV; ++i) *reinterpret_cast<f4v*>(tile + tile_off(i, e4)) = P[i];
        }
        const int lab = plab;
        const bool ok = lane < nrows && lab >= 0 && lab < k;
        const float* crow = Cs + (long)(ok ? lab : 0) * cs;
        f4v cv[CL ? 1 : G::NG];
        if constexpr (!CL) {
#pragma unroll
            for (int g = 0; g < G::NG; ++g)
                if (4 * g < d) cv[g] = *reinterpret_cast<const f4v*>(crow + 4 * g);
        }
        __builtin_amdgcn_sched_barrier(0);
        const long nc0 = c0 + wstep;
        // in flight while this chunk is summed; past the last chunk the
        // current one loads again, so every pass issues the same loads
        load(nc0 < r1 ? nc0 : c0);
        // (a wave's LDS accesses complete in order: the tile is written
        // before any lane reads it)
        __builtin_amdgcn_wave_barrier();
        float res = 0.f;
        const float* t = tile + min(lane, ROWS - 1) * S;
        auto group = [&](const f4v& x4, const f4v& c4) {
            const float t0 = x4.x - c4.x, t1 = x4.y - c4.y;
            const float t2 = x4.z - c4.z, t3 = x4.w - c4.w;
            res += ((t0 * t0 + t1 * t1) + t2 * t2) + t3 * t3;
        };
        auto last = [&](const f4v& x4, const f4v& c4, int m) {  // the row's last m < 4 features, one by one
            float tt = x4.x - c4.x;
            res += tt * tt;
            if (m > 1) {
                tt = x4.y - c4.y;
                res += tt * tt;
            }
            if (m > 2) {
                tt = x4.z - c4.z;
                res += tt * tt;
            }
        };
        if constexpr (CL) {
            const f4v* t4 = reinterpret_cast<const f4v*>(t);
            const f4v* c4 = reinterpret_cast<const f4v*>(crow);
            const int nfull = d >> 2;
#pragma unroll 5
            for (int g = 0; g < nfull; ++g) group(t4[g], c4[g]);
            if (d & 3) last(t4[nfull], c4[nfull], d & 3);
        } else {
#pragma unroll
            for (int g = 0; g < G::NG; ++g) {
                if (4 * g + 4 <= d)
                    group(*reinterpret_cast<const f4v*>(t + 4 * g), cv[g]);
                else if (4 * g < d)
                    last(*reinterpret_cast<const f4v*>(t + 4 * g), cv[g], d - 4 * g);
            }
        }
        __builtin_amdgcn_wave_barrier();  // every lane is done with the tile
        if (lane < nrows) {
            if (dist != nullptr) dist[c0 + lane - dbase] = ok ? res : 0.f;
            total += ok ? (double)res : 0.0;
        }
        c0 = nc0;
    }
    return total;
}

// The path for rows of stride ld: the narrowest contiguous one that holds
// them, else the column slabs.
int row_path(int ld) { return ld <= 32 ? 32 : ld <= 64 ? 64 : ld <= 104 ? 104 : ld <= 128 ? 128 : 0; }

// The relocation's row distances, rows [r0, r1) of a 256-thread block:
// 64-row chunks (kRelocTileFloats per wave tile), the centres from sC (CL:
// the block's LDS copy, which pro writes) or from C.
template <int LDM, bool CL>
struct RelocGeom {
    static constexpr int TF = LDM == 0 ? kRowTileFloats : CtgGeom<LDM == 0 ? 32 : LDM, 64>::TILE;  // wave tile
    static constexpr int CF = CL ? 64 * CtgGeom<LDM == 0 ? 32 : LDM, 64>::SMAX : 1;                   // centres, k <= 64
};

template <int LDM, bool CL, typename Pro>
__device__ __forceinline__ void reloc_rows_dist(const float* __restrict__ X, int ld, int d, const float* __restrict__ C,
                                                const float* sC, const int* __restrict__ labels, int k, long r0,
                                                long r1, float* dist, long dbase, float* tile, Pro pro)
{
    if constexpr (LDM == 0) {
        pro();
        (void)rows_dist(X, ld, d, C, labels, k, r0, r1, dist, tile);
    } else {
        (void)rows_dist_ctg<LDM, 64, CL>(X, ld, d, CL ? sC : C, CL ? ctg_stride(ld) : ld, labels, k, r0, r1, 256,
                                         dist, dbase, tile, pro);
    }
}

// k_rowdist, 64-row chunks dealt round-robin to the grid's waves (wave w of
// block b takes chunks b 4 + w + 4 gridDim t); dynamic LDS holds the four
// wave tiles (64 ctg_stride(ld) floats each) and, with CL, the centres (k
// rows of stride ctg_stride(ld)), copied in while the first chunks load.
// Each block's fp64 total (lanes, then waves in order) goes to
// block_part[b]; k_rowdist_total adds them.
template <int LDM, bool CL>
__global__ __launch_bounds__(256) void k_rowdist(RowDistArgs a)
{
    extern __shared__ __attribute__((aligned(16))) float rd_lds[];
    __shared__ double sh[4];
    const int S = ctg_stride(a.ld);
    float* sC = rd_lds + 4 * 64 * S;
    auto copy_centres = [&]() {
        if constexpr (CL) {
            const int e4 = a.k * a.ld / 4;
            const f4v* c4 = reinterpret_cast<const f4v*>(a.C);
            for (int q = threadIdx.x; q < e4; q += 256) {
                const int p = 4 * q, r = p / a.ld;
                *reinterpret_cast<f4v*>(sC + r * S + (p - r * a.ld)) = c4[q];
            }
            __syncthreads();
        }
    };
    const double v = rows_dist_ctg<LDM, 64, CL>(a.X, a.ld, a.d, CL ? sC : a.C, CL ? S : a.ld, a.labels, a.k,
                                                (long)blockIdx.x * 256, a.n, (long)gridDim.x * 256, a.out_rows, 0,
                                                rd_lds + (threadIdx.x >> 6) * 64 * S, copy_centres);
    const double t = block_sum(v, sh);
    if (threadIdx.x == 0) a.block_part[blockIdx.x] = t;
}

// Rows longer than 128 floats: the column slabs, block b taking rows
// [b rpb, (b + 1) rpb).
__global__ __launch_bounds__(256) void k_rowdist_slab(RowDistArgs a)
{
    __shared__ float tiles[4 * kRowTileFloats];
    __shared__ double sh[4];
    const long rpb = (a.n + gridDim.x - 1) / gridDim.x;
    const long r0 = min(a.n, (long)blockIdx.x * rpb), r1 = min(a.n, r0 + rpb);
    const double v = rows_dist(a.X, a.ld, a.d, a.C, a.labels, a.k, r0, r1, a.out_rows,
                               tiles + (threadIdx.x >> 6) * kRowTileFloats);
    const double t = block_sum(v, sh);
    if (threadIdx.x == 0) a.block_part[blockIdx.x] = t;
}

// The inertia: the nb block totals added in block order (each thread its
// strided share, then the block's fixed-order sum).  The kernel boundary
// makes k_rowdist's totals visible without a device-scope fence in every
// block, which cost 5 us of k_rowdist's 42 at 500000 x 100.
__global__ __launch_bounds__(256) void k_rowdist_total(RowDistArgs a, int nb)
{
    __shared__ double sh[4];
    double s = 0.0;
    for (int b = threadIdx.x; b < nb; b += 256) s += a.block_part[b];
    s = block_sum(s, sh);
    if (threadIdx.x == 0) a.state->inertia = s;
}

hipError_t launch_inertia_total(const double* parts, int nb, LoopState* state, hipStream_t s)
{
    RowDistArgs a{};
    a.block_part = const_cast<double*>(parts);
    a.state = state;
    hipLaunchKernelGGL(k_rowdist_total, dim3(1), dim3(256), 0, s, a, nb);
    return hipGetLastError();
}

int rowdist_grid(long n) { return (int)max(1L, min((long)kRowDistBlocks, (n + 255) / 256)); }

// LDS of k_rowdist for rows of stride ld: the tiles, and the centres when
// they fit beside them (*cl).
static size_t rowdist_lds(int ld, int k, bool* cl)
{
    constexpr size_t kBudget = 150 * 1024;
    const size_t S = (size_t)ctg_stride(ld), tiles = 4 * 64 * S * sizeof(float);
    const size_t cen = (size_t)k * S * sizeof(float);
    *cl = tiles + cen <= kBudget;
    return *cl ? tiles + cen : tiles;
}

template <int LDM>
static hipError_t launch_rowdist_ctg(const RowDistArgs& a, hipStream_t s, int* nb)
{
    bool cl = false;
    const size_t lds = rowdist_lds(a.ld, a.k, &cl);
    auto f = cl ? k_rowdist<LDM, true> : k_rowdist<LDM, false>;
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(f),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    // one block per CU (the LDS allows no more), at most one per 256 rows
    *nb = (int)max(1L, min((long)min(kRowDistBlocks, 256), (a.n + 255) / 256));
    hipLaunchKernelGGL(f, dim3(*nb), dim3(256), lds, s, a);
    return hipGetLastError();
}

hipError_t launch_rowdist(const RowDistArgs& a, hipStream_t s)
{
    int nb = rowdist_grid(a.n);
    hipError_t e = hipSuccess;
    switch (row_path(a.ld)) {
    case 32: e = launch_rowdist_ctg<32>(a, s, &nb); break;
    case 64: e = launch_rowdist_ctg<64>(a, s, &nb); break;
    case 104: e = launch_rowdist_ctg<104>(a, s, &nb); break;
    case 128: e = launch_rowdist_ctg<128>(a, s, &nb); break;
    default:
        hipLaunchKernelGGL(k_rowdist_slab, dim3(nb), dim3(256), 0, s, a);
        e = hipGetLastError();
    }
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_rowdist_total, dim3(1), dim3(256), 0, s, a, nb);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// relocation of empty clusters on the device
// ---------------------------------------------------------------------------
//
// sklearn's _relocate_empty_clusters_dense (_k_means_common.pyx:167-211):
// the n_empty rows farthest from their centre (fp32 direct-form distances from
// k_rowdist; descending distance, lower row index first on ties) move, in
// that order, to the empty clusters in ascending cluster order; each moves its
// row out of its old cluster's sums.  Then the centres are re-averaged from
// the fp64 sums with _average_centers' handling of still-empty clusters
// (:274-295) and the shift / ||c||^2 partials feed k_finalize_loop.

// (d, row) order: larger distance first, then lower row index.
__device__ __forceinline__ bool far_before(float d1, long i1, float d2, long i2)
{
    return d1 > d2 || (d1 == d2 && i1 < i2);
}

// One step of a selection: the best candidate strictly after (dl, il).
__device__ __forceinline__ void far_pick(float& bd, long& bi, float d, long i, float dl, long il)
{
    if (far_before(dl, il, d, i) && (bi < 0 || far_before(d, i, bd, bi))) {
        bd = d;
        bi = i;
    }
}

// The first of the block's candidates in far_before order (bi < 0: none);
// every thread gets it.  The order is total on rows, so the xor butterflies
// leave the same candidate in every lane.  sd / si: 4 entries each.
__device__ void far_block_reduce(float& bd, long& bi, float* sd, long* si)
{
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const float d2 = __shfl_xor(bd, off, 64);
        const long i2 = __shfl_xor(bi, off, 64);
        if (i2 >= 0 && (bi < 0 || far_before(d2, i2, bd, bi))) {
            bd = d2;
            bi = i2;
        }
    }
    if ((threadIdx.x & 63) == 0) {
        sd[threadIdx.x >> 6] = bd;
        si[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    bd = sd[0];
    bi = si[0];
    for (int w = 1; w < 4; ++w) {
        if (si[w] >= 0 && (bi < 0 || far_before(sd[w], si[w], bd, bi))) {
            bd = sd[w];
            bi = si[w];
        }
    }
    __syncthreads();
}

// Block b: its E farthest rows, in order, among rows [b*rpb, (b+1)*rpb).
__global__ __launch_bounds__(256) void k_far_select(RelocArgs a, int E, long rpb)
{
    __shared__ float sd[256];
    __shared__ long si[256];
    const long r0 = (long)blockIdx.x * rpb;
    const long r1 = min(a.n, r0 + rpb);
    float dl = INFINITY;
    long il = -1;
    for (int e = 0; e < E; ++e) {
        float bd = 0.f;
        long bi = -1;
        for (long r = r0 + threadIdx.x; r < r1; r += 256) far_pick(bd, bi, a.dist[r], r, dl, il);
        far_block_reduce(bd, bi, sd, si);
        if (threadIdx.x == 0) {
            a.cand_d[(long)blockIdx.x * E + e] = bd;
            a.cand_i[(long)blockIdx.x * E + e] = bi;
        }
        if (bi < 0) {
            // this block has no more rows: pad the rest
            for (int e2 = e + 1 + threadIdx.x; e2 < E; e2 += 256) {
                a.cand_d[(long)blockIdx.x * E + e2] = 0.f;
                a.cand_i[(long)blockIdx.x * E + e2] = -1;
            }
            return;
        }
        dl = bd;
        il = bi;
    }
}

// One block: merge the candidates, move the rows, then the heaviest cluster.
__global__ __launch_bounds__(256) void k_far_apply(RelocArgs a, int E, int nb)
{
    __shared__ float sd[256];
    __shared__ long si[256];
    __shared__ long far[kMaxReloc];
    __shared__ int empt[kMaxReloc];
    __shared__ int ne_s;
    const int tid = threadIdx.x;
    if (tid == 0) {
        int ne = 0;
        for (int j = 0; j < a.k && ne < E; ++j)
            if (a.counts[j] == 0) empt[ne++] = j;
        ne_s = ne;
    }
    float dl = INFINITY;
    long il = -1;
    for (int e = 0; e < E; ++e) {
        float bd = 0.f;
        long bi = -1;
        for (int c = tid; c < nb * E; c += 256) {
            const long i = a.cand_i[c];
            if (i >= 0) far_pick(bd, bi, a.cand_d[c], i, dl, il);
        }
        far_block_reduce(bd, bi, sd, si);
        if (tid == 0) far[e] = bi;
        dl = bd;
        il = bi;
        // the farthest distance decides whether anything moves (all zero: no)
        if (e == 0 && tid == 0 && (bi < 0 || bd <= 0.f)) ne_s = 0;
    }
    __syncthreads();
    const int ne = ne_s;
    for (int e = 0; e < ne; ++e) {
        const long fr = far[e];
        const int j = empt[e];
        const int o = a.labels[fr];
        const float* x = a.X + fr * a.ld;
        for (int c = tid; c < a.d; c += 256) {
            a.sums[(long)o * a.ld + c] -= (double)x[c];
            a.sums[(long)j * a.ld + c] = (double)x[c];
        }
        __syncthreads();
        if (tid == 0) {
            a.counts[j] = 1;
            a.counts[o] -= 1;
        }
        __syncthreads();
    }
    if (tid == 0) {
        int amax = 0;
        for (int j = 1; j < a.k; ++j)
            if (a.counts[j] > a.counts[amax]) amax = j;
        *a.amax = amax;
    }
}

// Centres from the fp64 sums (block (j, cc): columns [cc*CW, cc*CW + CW)),
// and the shift^2 / ||c||^2 chunk partials, as k_finalize_cols.
__global__ __launch_bounds__(256) void k_finalize_sums(RelocArgs a, int CW)
{
    const int j = blockIdx.x;
    const int cc = blockIdx.y;
    const int nch = gridDim.y;
    const int tid = threadIdx.x;
    __shared__ double shd[2][4];
    const int col = cc * CW + tid;
    const int cnt = a.counts[j];
    const int amax = *a.amax;
    double sq = 0.0, nrm = 0.0;
    if (tid < CW && col < a.d) {
        double v;
        if (cnt > 0) {
            v = a.sums[(long)j * a.ld + col] / (double)cnt;
        } else {
            // _average_centers: the heaviest cluster's row as the loop has it
            // -- already divided when it comes before j, still a sum after
            const double sa = a.sums[(long)amax * a.ld + col];
            v = amax < j ? sa / (double)a.counts[amax] : sa;
        }
        const float cn = (float)v;
        a.C_new[(long)j * a.ld + col] = cn;
        const double df = (double)cn - (double)a.C_old[(long)j * a.ld + col];
        sq = df * df;
        nrm = (double)cn * (double)cn;
    }
    sq = block_sum(sq, shd[0]);
    nrm = block_sum(nrm, shd[1]);
    if (tid == 0) {
        a.part[((long)j * nch + cc) * 2 + 0] = sq;
        a.part[((long)j * nch + cc) * 2 + 1] = nrm;
    }
}

hipError_t launch_relocate(const RelocArgs& a, int E, hipStream_t s)
{
    if (E < 1 || E > kMaxReloc) return hipErrorInvalidValue;
    const int nb = kRelocBlocks;
    const long rpb = (a.n + nb - 1) / nb;
    hipLaunchKernelGGL(k_far_select, dim3(nb), dim3(256), 0, s, a, E, rpb);
    hipLaunchKernelGGL(k_far_apply, dim3(1), dim3(256), 0, s, a, E, nb);
    hipLaunchKernelGGL(k_finalize_sums, dim3(a.k, (a.d + kRelocCW - 1) / kRelocCW), dim3(256), 0, s, a, kRelocCW);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// in-stream relocation: k_reloc
// ---------------------------------------------------------------------------
//
// Launched after every step's k_finalize_cols, which counts the clusters it
// finds empty in state->empty_cnt[iter & 1]; with none the kernel returns at
// its first load.  Otherwise, as the device path above but in one kernel:
// (A) each block takes the distances of its contiguous share of the rows and
// its E farthest, in order, and counts itself done; (B) the last block to
// finish merges the blocks' lists, moves the rows in the fp64 sums and
// counts, and (C) redoes the centres and chunk partials (the finalize's
// 32-column chunks) of the clusters involved -- the filled ones, those that
// gave a row, and any still empty -- as k_finalize_sums does; every other
// cluster keeps what k_finalize_cols wrote.  state->reloc_iter = iter then
// tells the loop decision that this step's empty clusters were handled.  No
// block waits for another.

// ||x - c||^2 of one row in fp32 with rows_dist_ctg's operations in its
// order (whole float4 groups, then the last d % 4 features one by one), so
// that a row gets the same value either way.
template <int LDM>
struct RowRegs {
    f4v v[LDM / 4];
};
template <int LDM>
__device__ __forceinline__ void load_row(RowRegs<LDM>& xv, const float* __restrict__ x, int d)
{
    const f4v* x4 = reinterpret_cast<const f4v*>(x);
#pragma unroll
    for (int g = 0; g < LDM / 4; ++g)
        if (4 * g < d) xv.v[g] = x4[g];  // all in flight
}
template <int LDM>
__device__ __forceinline__ float direct_dist(const RowRegs<LDM>& xr, const float* c, int d)
{
#pragma clang fp contract(off)
    constexpr int NG = LDM / 4;
    const f4v* c4 = reinterpret_cast<const f4v*>(c);
    const f4v* xv = xr.v;
    float res = 0.f;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        if (4 * g >= d) break;
        const f4v cv = c4[g];
        if (4 * g + 4 <= d) {
            const float t0 = xv[g].x - cv.x, t1 = xv[g].y - cv.y;
            const float t2 = xv[g].z - cv.z, t3 = xv[g].w - cv.w;
            res += ((t0 * t0 + t1 * t1) + t2 * t2) + t3 * t3;
        } else {
            const int m = d - 4 * g;
            float tt = xv[g].x - cv.x;
            res += tt * tt;
            if (m > 1) {
                tt = xv[g].y - cv.y;
                res += tt * tt;
            }
            if (m > 2) {
                tt = xv[g].z - cv.z;
                res += tt * tt;
            }
        }
    }
    return res;
}

constexpr int kRelocCand = 256;  // candidate rows per block, at most (one per thread)

// The relocation of E (1..kMaxReloc) empty clusters by every block of the
// grid (gridDim.x <= kRelocCandBlocks): phases A, B and C above.
template <int LDM, bool CL>
__device__ __forceinline__ void reloc_body(const InRelocArgs& a, int E)
{
    using RG = RelocGeom<LDM, CL>;
    __shared__ __attribute__((aligned(16))) float tiles[4 * RG::TF];
    __shared__ __attribute__((aligned(16))) float sC[RG::CF];
    __shared__ float sdist[kRelocLdsRows];
    __shared__ float sd[4];
    __shared__ long si[4];
    __shared__ int shi[4];
    __shared__ int last_s;
    LoopState* st = a.state;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;

    // (A) distances of rows [r0, r1), into LDS when they fit (a.dist
    // otherwise), then this block's E farthest, in order.  Distances left
    // in the L2 would make the device-scope fence below write back 2 MB at
    // 500000 rows: 29 of the step's 95 us.
    const long rpb = (a.n + gridDim.x - 1) / gridDim.x;
    const long r0 = min(a.n, (long)blockIdx.x * rpb), r1 = min(a.n, r0 + rpb);
    const bool in_lds = LDM != 0 && r1 - r0 <= kRelocLdsRows;
    float* dist = in_lds ? sdist : a.dist;
    const long dbase = in_lds ? r0 : 0;
    auto copy_centres = [&]() {
        if constexpr (CL) {
            const int S = ctg_stride(a.ld), e4 = a.k * a.ld / 4;
            const f4v* c4 = reinterpret_cast<const f4v*>(a.C_old);
            for (int q = tid; q < e4; q += 256) {
                const int p = 4 * q, r = p / a.ld;
                *reinterpret_cast<f4v*>(sC + r * S + (p - r * a.ld)) = c4[q];
            }
            __syncthreads();
        }
    };
    // (A') With the E-step's row minima: the approximate distance xnorm[r]
    // + emin[r] (= ||x||^2 + ||c||^2 - 2 x.c, c the row's centre) of every
    // row, the block's E-th largest of them, T, and as candidates the rows
    // within 2M of T, M = 2^-10 (max ||x||^2 + max ||c||^2): for rows of
    // at most 128 floats the approximation and the direct form each lie
    // within 2^-13 of that sum of the true distance (fp32 norms, the split's
    // dropped terms, the fp32 accumulation of at most 768 part products, and
    // the direct form's rounding), so every row of the block's E
    // farthest by direct-form distance is a candidate.  Only the candidates
    // get that distance, and the selection runs over them: the same rows as
    // (A), for 8 bytes a row instead of the row.  More than kRelocCand
    // candidates (wide ties at the top), or a bound that is not finite: (A).
    bool exact = true;  // block-uniform
    int ncand = 0;
    long* const ccl = reinterpret_cast<long*>(tiles);  // (the tiles are free until (A))
    float* const ccd = tiles + 2 * kRelocCand;
    if constexpr (LDM != 0) {
        if (a.emin != nullptr && a.xnorm != nullptr && in_lds) {
            const int nr = (int)(r1 - r0);
            float xm = 0.f;
            constexpr int U = 8;
            float xv[U], ev[U];
            auto load = [&](int q0) {
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int q = q0 + 256 * u + tid;
                    xv[u] = q < nr ? a.xnorm[r0 + q] : 0.f;
                    ev[u] = q < nr ? a.emin[r0 + q] : 0.f;
                }
            };
            auto put = [&](int q0) {
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int q = q0 + 256 * u + tid;
                    if (q < nr) {
                        sdist[q] = xv[u] + ev[u];
                        xm = fmaxf(xm, xv[u]);
                    }
                }
            };
            // the first rows' values and the centres in one round trip
            load(0);
            copy_centres();
            put(0);
            for (int q0 = 256 * U; q0 < nr; q0 += 256 * U) {
                load(q0);
                put(q0);
            }
            // the largest ||c||^2: four threads a centre, a quarter of its
            // float4s each (the four lanes of a quad run the same trips)
            float cm = 0.f;
            for (int j = tid >> 2; j < (a.k + 63) / 64 * 64; j += 64) {
                const int qq = tid & 3;
                const int g4 = a.ld >> 2;  // float4s a row (its pad is zero)
                float s2 = 0.f;
                if (j < a.k) {
                    const f4v* cr = reinterpret_cast<const f4v*>(CL ? sC + j * ctg_stride(a.ld) : a.C_old + (long)j * a.ld);
                    for (int g = qq; g < g4; g += 4) {
                        const f4v v = cr[g];
                        s2 = fmaf(v.x, v.x, fmaf(v.y, v.y, fmaf(v.z, v.z, fmaf(v.w, v.w, s2))));
                    }
                }
                s2 += __shfl_xor(s2, 1, 64);
                s2 += __shfl_xor(s2, 2, 64);
                cm = fmaxf(cm, s2);
            }
            __syncthreads();  // sdist from every thread
            const float M = 0x1p-10f * (block_max(xm, sd) + block_max(cm, sd));
            float dl = INFINITY;
            long il = -1;
            for (int e = 0; e < E; ++e) {
                float bd = 0.f;
                long bi = -1;
                for (int q = tid; q < nr; q += 256) far_pick(bd, bi, sdist[q], r0 + q, dl, il);
                far_block_reduce(bd, bi, sd, si);
                dl = bd;
                il = bi;
            }
            const float thr = il < 0 ? -INFINITY : dl - 2.f * M;  // fewer than E rows: all
            int mine = 0;
            for (int q = tid; q < nr; q += 256) mine += sdist[q] >= thr;
            int tot;
            int pos = block_excl_scan(mine, shi, &tot);
            if (M < INFINITY && tot <= kRelocCand) {
                for (int q = tid; q < nr; q += 256)
                    if (sdist[q] >= thr) ccl[pos++] = r0 + q;
                __syncthreads();
                if (tid < tot) {
                    const long r = ccl[tid];
                    RowRegs<LDM == 0 ? 4 : LDM> xr;
                    load_row(xr, a.X + r * a.ld, a.d);  // the row and its label: one round trip
                    const int lab = a.labels[r];
                    const bool ok = lab >= 0 && lab < a.k;
                    const float* cr = CL ? sC + (ok ? lab : 0) * ctg_stride(a.ld) : a.C_old + (long)(ok ? lab : 0) * a.ld;
                    const float dd = direct_dist(xr, cr, a.d);
                    ccd[tid] = ok ? dd : 0.f;
                }
                __syncthreads();
                exact = false;
                ncand = tot;
            }
        }
    }
    if (exact) {
        reloc_rows_dist<LDM, CL>(a.X, a.ld, a.d, a.C_old, sC, a.labels, a.k, r0, r1, dist, dbase,
                                 tiles + w * RG::TF, copy_centres);
        __threadfence_block();
        __syncthreads();
    }
    {
        float dl = INFINITY;
        long il = -1;
        for (int e = 0; e < E; ++e) {
            float bd = 0.f;
            long bi = -1;
            if (exact) {
                for (long r = r0 + tid; r < r1; r += 256) far_pick(bd, bi, dist[r - dbase], r, dl, il);
            } else if (tid < ncand) {
                far_pick(bd, bi, ccd[tid], ccl[tid], dl, il);
            }
            far_block_reduce(bd, bi, sd, si);
            if (tid == 0) {
                a.cand_d[(long)blockIdx.x * kMaxReloc + e] = bd;
                a.cand_i[(long)blockIdx.x * kMaxReloc + e] = bi;
            }
            dl = bd;
            il = bi;
        }
    }
    // the last block to get here takes (B) and (C).  The block's stores (the
    // candidates, and in k_finalize_reloc the finalize chunk's sums, counts,
    // centres and partials, written by several waves) are done once its
    // waves pass the barrier; thread 0's ticket is an agent-scope release
    // RMW (the L2's dirty lines written back first), and the last block's
    // thread 0 acquires after it, before the barrier its other waves wait
    // at.  One write-back per block and one invalidation in all: a
    // __threadfence in every wave (write-back and L2 invalidation each) cost
    // 14.6 us of the relocating step at 500000 rows.
    __syncthreads();
    if (tid == 0)
        last_s = __hip_atomic_fetch_add(&st->reloc_ctr, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT) ==
                 gridDim.x - 1;
    __syncthreads();
    if (!last_s) return;
    if (tid == 0) {
        st->reloc_ctr = 0u;
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");  // every block's stores
    }
    __syncthreads();

    // each thread's contiguous share of the clusters
    const int per = (a.k + 255) / 256;
    const int j0 = min(a.k, tid * per), j1 = min(a.k, j0 + per);

    // (B) the first E empty clusters in ascending order
    __shared__ long far[kMaxReloc];
    __shared__ int empt[kMaxReloc];
    __shared__ int donor[kMaxReloc];
    __shared__ int still[kMaxReloc];
    __shared__ int ne_s;
    {
        int mine = 0;
        for (int j = j0; j < j1; ++j) mine += a.counts[j] == 0;
        int tot;
        int pos = block_excl_scan(mine, shi, &tot);
        for (int j = j0; j < j1 && pos < E; ++j)
            if (a.counts[j] == 0) empt[pos++] = j;
        if (tid == 0) ne_s = min(tot, E);
    }
    // the E farthest rows overall: a merge of the blocks' ordered lists,
    // thread t holding the heads of blocks t + 256 j
    {
        constexpr int HPT = (kRelocInlineBlocks + 255) / 256;  // list heads per thread
        const int nb = (int)gridDim.x;  // <= 256 HPT
        int h[HPT];
        float hd[HPT];
        long hi[HPT];
#pragma unroll
        for (int j = 0; j < HPT; ++j) {
            const int b = tid + 256 * j;
            h[j] = 0;
            hd[j] = 0.f;
            hi[j] = -1;
            if (b < nb) {
                hd[j] = a.cand_d[(long)b * kMaxReloc];
                hi[j] = a.cand_i[(long)b * kMaxReloc];
            }
        }
        for (int e = 0; e < E; ++e) {
            float bd = hd[0];
            long bi = hi[0];
#pragma unroll
            for (int j = 1; j < HPT; ++j) {
                if (hi[j] >= 0 && (bi < 0 || far_before(hd[j], hi[j], bd, bi))) {
                    bd = hd[j];
                    bi = hi[j];
                }
            }
            far_block_reduce(bd, bi, sd, si);
            if (tid == 0) {
                far[e] = bi;
                // the farthest distance decides whether anything moves (all zero: no)
                if (e == 0 && (bi < 0 || bd <= 0.f)) ne_s = 0;
            }
#pragma unroll
            for (int j = 0; j < HPT; ++j) {
                if (bi >= 0 && hi[j] == bi) {
                    const long b = tid + 256 * j;
                    ++h[j];
                    hd[j] = 0.f;
                    hi[j] = -1;
                    if (h[j] < E) {
                        hd[j] = a.cand_d[b * kMaxReloc + h[j]];
                        hi[j] = a.cand_i[b * kMaxReloc + h[j]];
                    }
                }
            }
        }
    }
    __syncthreads();
    const int nm = ne_s;
    // move far[e] to empt[e], in order: each thread owns columns of the sums
    if (tid < nm) donor[tid] = a.labels[far[tid]];
    __syncthreads();
    for (int c = tid; c < a.d; c += 256) {
        for (int e = 0; e < nm; ++e) {
            const double xv = (double)a.X[far[e] * a.ld + c];
            a.sums[(long)donor[e] * a.ld + c] -= xv;
            a.sums[(long)empt[e] * a.ld + c] = xv;
        }
    }
    if (tid < nm) {
        a.counts[empt[tid]] = 1;
        // a donor's first move takes all of its moves off its count
        int m = 0;
        bool first = true;
        for (int e = 0; e < nm; ++e) {
            if (donor[e] == donor[tid]) {
                ++m;
                first = first && e >= tid;
            }
        }
        if (first) a.counts[donor[tid]] -= m;
    }
    __threadfence_block();
    __syncthreads();

    // the largest cluster (lowest index on ties) and the clusters still empty
    __shared__ int amax_s, nstill_s;
    {
        int bc = -1, bj = a.k, mine = 0;
        for (int j = j0; j < j1; ++j) {
            const int c = a.counts[j];
            if (c > bc) {
                bc = c;
                bj = j;
            }
            mine += c == 0;
        }
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int oc = __shfl_xor(bc, off, 64), oj = __shfl_xor(bj, off, 64);
            if (oc > bc || (oc == bc && oj < bj)) {
                bc = oc;
                bj = oj;
            }
        }
        __shared__ int mc[4], mj[4];
        if (lane == 0) {
            mc[w] = bc;
            mj[w] = bj;
        }
        int tot;
        int pos = block_excl_scan(mine, shi, &tot);  // (its first barrier publishes mc, mj)
        for (int j = j0; j < j1 && pos < kMaxReloc; ++j)
            if (a.counts[j] == 0) still[pos++] = j;
        if (tid == 0) {
            int c = mc[0], jj = mj[0];
            for (int q = 1; q < 4; ++q) {
                if (mc[q] > c || (mc[q] == c && mj[q] < jj)) {
                    c = mc[q];
                    jj = mj[q];
                }
            }
            amax_s = jj;
            nstill_s = min(tot, kMaxReloc);
        }
    }
    __syncthreads();
    const int amax = amax_s;

    // (C) centres and chunk partials of the clusters involved, one (cluster,
    // chunk) per wave at a time: entries q < nm the filled clusters, nm <= q
    // < 2 nm the donors, then the clusters still empty (repeats write the
    // same values).  The chunk sums are the wave sums k_finalize_cols forms.
    constexpr int CW = 32;
    const int nitems = 2 * nm + nstill_s;
    for (int p = w; p < nitems * a.nch; p += 4) {
        const int q = p / a.nch, cc = p - q * a.nch;
        const int j = q < nm ? empt[q] : q < 2 * nm ? donor[q - nm] : still[q - 2 * nm];
        const int cnt = a.counts[j];
        const int col = cc * CW + lane;
        double sq = 0.0, nrm = 0.0;
        if (lane < CW && col < a.d) {
            double v;
            if (cnt > 0) {
                v = a.sums[(long)j * a.ld + col] / (double)cnt;
            } else {
                const double sa = a.sums[(long)amax * a.ld + col];
                v = amax < j ? sa / (double)a.counts[amax] : sa;
            }
            const float cn = (float)v;
            a.C_new[(long)j * a.ld + col] = cn;
            const double df = (double)cn - (double)a.C_old[(long)j * a.ld + col];
            sq = df * df;
            nrm = (double)cn * (double)cn;
        }
        sq = wave_sum(sq);
        nrm = wave_sum(nrm);
        if (lane == 0) {
            a.part[((long)j * a.nch + cc) * 2 + 0] = sq;
            a.part[((long)j * a.nch + cc) * 2 + 1] = nrm;
        }
    }
    if (tid == 0) st->reloc_iter = a.iter;
}

// After k_finalize_cols: the clusters it counted empty.
template <int LDM>
__global__ __launch_bounds__(256) void k_reloc(InRelocArgs a)
{
    if (a.state->done != 0) return;
    const int E = a.state->empty_cnt[a.iter & 1];
    if (E == 0 || E > kMaxReloc) return;
    reloc_body<LDM, false>(a, E);
}

// The fused step's finalize and relocation in one launch.  The F = k nch
// finalize chunks (cluster j, column chunk cc) are numbered j nch + cc, the
// order of their columns in memory; blocks are dealt to the 8 XCDs in turn
// (block b on XCD b % 8), and the blocks of XCD x take chunks
// [x per, (x + 1) per), per = ceil(F / 8), so that a cache line two
// neighbouring chunks share is fetched into one XCD's L2 (the partials'
// rows of d floats need not start on a line).  Then, when some cluster
// received no row (the fused kernel's presence bits, so every block knows
// at once), every block joins the relocation.  The last block to finish its
// rows finds every finalize chunk written.
template <int LDM>
__global__ __launch_bounds__(256) void k_finalize_reloc(FinalizeArgs f, InRelocArgs a, int nch)
{
    const int b = blockIdx.x;
    LoopState* st = f.state;
    const unsigned long long pres = st->present[f.iter & 1];
    const int per = (f.k * nch + 7) / 8, item = (b & 7) * per + (b >> 3);
    if ((b >> 3) < per && item < f.k * nch) finalize_cols_block(f, item / nch, item % nch, nch);
    if (b == 0 && threadIdx.x == 0) st->present[(f.iter + 1) & 1] = 0ull;  // for the next fused kernel
    if (st->done != 0) return;
    const unsigned long long all = f.k >= 64 ? ~0ull : (1ull << f.k) - 1ull;
    const int E = __popcll(all & ~pres);
    if (E == 0 || E > kMaxReloc) return;
    // k <= 64: the centres fit in LDS beside the tiles up to 104 floats a row
    reloc_body<LDM, LDM != 0 && LDM <= 104>(a, E);
}

hipError_t launch_finalize_reloc(const FinalizeArgs& f, const InRelocArgs& a, hipStream_t s)
{
    const int nch = finalize_col_chunks(f.d, f.R);
    if (f.k > 64 || 8 * ((f.k * nch + 7) / 8) > kRelocInlineBlocks || f.rec_off != nullptr) return hipErrorInvalidValue;
    const dim3 g(kRelocInlineBlocks);
    switch (row_path(a.ld)) {
    case 32: hipLaunchKernelGGL(k_finalize_reloc<32>, g, dim3(256), 0, s, f, a, nch); break;
    case 64: hipLaunchKernelGGL(k_finalize_reloc<64>, g, dim3(256), 0, s, f, a, nch); break;
    case 104: hipLaunchKernelGGL(k_finalize_reloc<104>, g, dim3(256), 0, s, f, a, nch); break;
    case 128: hipLaunchKernelGGL(k_finalize_reloc<128>, g, dim3(256), 0, s, f, a, nch); break;
    default: hipLaunchKernelGGL(k_finalize_reloc<0>, g, dim3(256), 0, s, f, a, nch); break;
    }
    return hipGetLastError();
}

hipError_t launch_reloc_inline(const InRelocArgs& a, hipStream_t s)
{
    const dim3 g(kRelocInlineBlocks);
    switch (row_path(a.ld)) {
    case 32: hipLaunchKernelGGL(k_reloc<32>, g, dim3(256), 0, s, a); break;
    case 64: hipLaunchKernelGGL(k_reloc<64>, g, dim3(256), 0, s, a); break;
    case 104: hipLaunchKernelGGL(k_reloc<104>, g, dim3(256), 0, s, a); break;
    case 128: hipLaunchKernelGGL(k_reloc<128>, g, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL(k_reloc<0>, g, dim3(256), 0, s, a); break;
    }
    return hipGetLastError();
}

__global__ void k_state_reset(LoopState* st, LoopState v)
{
    if (threadIdx.x == 0) *st = v;
}

hipError_t launch_state_reset(LoopState* st, const LoopState& v, hipStream_t s)
{
    hipLaunchKernelGGL(k_state_reset, dim3(1), dim3(64), 0, s, st, v);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// set-up kernels
// ---------------------------------------------------------------------------

constexpr long kColsumRows = 512;

int colsum_grid(long n) { return (int)max(1L, (n + kColsumRows - 1) / kColsumRows); }

// Block b sums rows [512 b, 512 b + 512) of every column in fp64: thread
// (slot, q) adds the float4 of columns 4q.. (plus 128 per pass) of rows
// slot, slot + 8, ... (eight slots, all loads of a batch in flight), then the
// slots are added in slot order -- a fixed order, so the mean is bitwise
// reproducible.
__global__ __launch_bounds__(256) void k_colsum(const float* __restrict__ X, long n, int ld, int d,
                                                double* __restrict__ part)
{
    const long r0 = (long)blockIdx.x * kColsumRows;
    const long r1 = min(n, r0 + kColsumRows);
    const int q = threadIdx.x & 31;
    const int slot = threadIdx.x >> 5;
    __shared__ double red[8][128];
    for (int c0 = 0; c0 < ld; c0 += 128) {
        const int c = c0 + 4 * q;
        double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
        if (c < ld) {  // ld is a multiple of 4
            for (long r = r0 + slot; r < r1; r += 8 * 8) {
                float4 v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const long rr = r + 8 * u;
                    v[u] = rr < r1 ? *reinterpret_cast<const float4*>(X + rr * ld + c) : make_float4(0.f, 0.f, 0.f, 0.f);
                }
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    s0 += (double)v[u].x;
                    s1 += (double)v[u].y;
                    s2 += (double)v[u].z;
                    s3 += (double)v[u].w;
                }
            }
        }
        red[slot][4 * q + 0] = s0;
        red[slot][4 * q + 1] = s1;
        red[slot][4 * q + 2] = s2;
        red[slot][4 * q + 3] = s3;
        __syncthreads();
        if (threadIdx.x < 128 && c0 + (int)threadIdx.x < d) {
            double t = 0.0;
#pragma unroll
            for (int k8 = 0; k8 < 8; ++k8) t += red[k8][threadIdx.x];
            part[(long)blockIdx.x * d + c0 + threadIdx.x] = t;
        }
        __syncthreads();
    }
}

hipError_t launch_colsum(const float* X, long n, int ld, int d, double* part, int nblk, hipStream_t s)
{
    hipLaunchKernelGGL(k_colsum, dim3(nblk), dim3(256), 0, s, X, n, ld, d, part);
    return hipGetLastError();
}

// Block c: column c's mean from the nblk block sums -- thread t adds sums t,
// t + 256, ... and the block adds its threads in a fixed order.
__global__ __launch_bounds__(256) void k_colmean(const double* __restrict__ part, int nblk, long n, int d,
                                                 float* __restrict__ mean)
{
    __shared__ double sh[4];
    const int c = blockIdx.x;
    double s = 0.0;
    for (int b = threadIdx.x; b < nblk; b += 256) s += part[(long)b * d + c];
    s = block_sum(s, sh);
    if (threadIdx.x == 0) mean[c] = (float)(s / (double)n);
}

hipError_t launch_colmean(const double* part, int nblk, long n, int d, float* mean, hipStream_t s)
{
    hipLaunchKernelGGL(k_colmean, dim3(d), dim3(256), 0, s, part, nblk, n, d, mean);
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

// Largest |x| over `count` floats (NaN counts as +inf) into *out as float
// bits: non-negative floats order like their bit patterns, so an unsigned
// atomic max per wave combines them.
__global__ __launch_bounds__(256) void k_absmax(const float* __restrict__ X, long count, unsigned* out)
{
    float m = 0.f;
    const long stride = (long)gridDim.x * 256;
    const long c4 = count >> 2;  // 16-byte loads over the multiple-of-4 part
    const float4* X4 = reinterpret_cast<const float4*>(X);
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < c4; i += stride) {
        const float4 v4 = X4[i];
        const float e[4] = {fabsf(v4.x), fabsf(v4.y), fabsf(v4.z), fabsf(v4.w)};
#pragma unroll
        for (int u = 0; u < 4; ++u) m = e[u] != e[u] ? INFINITY : fmaxf(m, e[u]);
    }
    for (long i = 4 * c4 + (long)blockIdx.x * 256 + threadIdx.x; i < count; i += stride) {
        const float v = fabsf(X[i]);
        m = v != v ? INFINITY : fmaxf(m, v);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    __shared__ float wm[4];
    if ((threadIdx.x & 63) == 0) wm[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) atomicMax(out, __float_as_uint(fmaxf(fmaxf(wm[0], wm[1]), fmaxf(wm[2], wm[3]))));
}

hipError_t launch_absmax(const float* X, long count, unsigned* out, hipStream_t s)
{
    const hipError_t e = hipMemsetAsync(out, 0, sizeof(unsigned), s);
    if (e != hipSuccess) return e;
    long blocks = (count / 4 + 255) / 256;
    if (blocks > 1024) blocks = 1024;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(k_absmax, dim3((unsigned)blocks), dim3(256), 0, s, X, count, out);
    return hipGetLastError();
}

// ||x_r||^2 in fp32, one thread per row (the relocation's approximate
// distances; their candidate margin covers its rounding).
__global__ __launch_bounds__(256) void k_rownorm(const float* __restrict__ X, long n, int ld, int d,
                                                 float* __restrict__ out)
{
    const long r = (long)blockIdx.x * 256 + threadIdx.x;
    if (r >= n) return;
    const float4* x4 = reinterpret_cast<const float4*>(X + r * ld);
    float s = 0.f;
    const int nfull = d >> 2;
    for (int g = 0; g < nfull; ++g) {
        const float4 v = x4[g];
        s = fmaf(v.x, v.x, s);
        s = fmaf(v.y, v.y, s);
        s = fmaf(v.z, v.z, s);
        s = fmaf(v.w, v.w, s);
    }
    for (int c = 4 * nfull; c < d; ++c) s = fmaf(X[r * ld + c], X[r * ld + c], s);
    out[r] = s;
}

hipError_t launch_rownorm(const float* X, long n, int ld, int d, float* out, hipStream_t s)
{
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_rownorm, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, X, n, ld, d, out);
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
