// sample_kernels.hip -- weighted draws without replacement on the device (gfx950).
//
// numpy's legacy RandomState.choice(n, size, replace=False, p=w / w.sum()) for
// fp32 weights w (the k-means|| rounds of skmetal's MetalKMeans,
// skmetal/estimators/cluster.py:92-98, with w = maximum(dists, 1e-30); and
// scikit-learn's init="random", sklearn/cluster/_kmeans.py:1010-1013, with unit
// weights), picking the rows numpy picks for the same uniforms.  The caller
// draws the uniforms from its RandomState (rand(size - found) per pass) and
// runs numpy's pass loop (drop repeated picks, zero the found rows, draw
// again); the device does everything that is O(n):
//
//   k_ws_block    fp32 sum of each 8192-weight block in numpy's pairwise
//                 order (leaves of <= 128 weights on eight accumulators,
//                 halves split at a multiple of 8) -- numpy reduces a
//                 contiguous fp32 array one 8192-element buffer at a time; a
//                 whole block is a perfect tree of 64 leaves (one lane each,
//                 then a butterfly), the last one is walked by one thread;
//   k_ws_total    the block sums added in order (numpy's running total);
//   k_ws_prob     p_i = fp64(fp32(w_i / total)) (choice converts the fp32
//                 probabilities to fp64), per-2048-row chunk fp64 sums and
//                 non-zero counts;
//   k_ws_prefix   the chunk sums' running total (fixed order);
//   k_ws_search   one block per uniform u: the row r with cdf[r-1] <= u <
//                 cdf[r] (searchsorted side="right"), where numpy's cdf is the
//                 sequential fp64 cumsum of p divided by its last element.
//                 The block forms the cumsum of its chunk from the chunk
//                 prefix in another order; a sum of non-negative terms whose
//                 every term passes through at most h roundings is within
//                 gamma_h = h 2^-53 / (1 - h 2^-53) of the exact sum relative
//                 to the total, so numpy's cdf and this one differ by at most
//                 Delta (below) at every row.  r is certified when
//                 cdf~[r-1] < u - Delta and cdf~[r] > u + Delta; otherwise
//                 the draw is marked unsure;
//   k_ws_chain    (only for unsure draws) numpy's cumsum itself, exactly,
//                 chunk by chunk: inside one binade of the running sum the
//                 additions are exact integer sums on that binade's grid;
//   k_ws_exact_search  the draw's chunk, then its row, on those sums.
//
// An unsure draw needs u within Delta ~ 4 n 2^-53 of one of the n cdf values:
// at n = 500,000 about 2e-4 of the draws.
#include <cfloat>

#include "device.h"

namespace skm {

namespace {

constexpr int kWSThreads = 256;
constexpr int kLeaf = 128;     // numpy's PW_BLOCKSIZE
constexpr int kMaxLeaves = 72; // a block of <= 8192 has at most 65 leaves

__device__ __forceinline__ int pw_half(int l)
{
    const int h = l / 2;
    return h - h % 8;
}

// LDS index of weight i of the block: one pad float per 128 keeps the leaves'
// reads (leaf starts 128 apart for a full block) on distinct banks.
__device__ __forceinline__ int pad_idx(int i) { return i + (i >> 7); }

// numpy's maximum(w, floor): NaN stays NaN
__device__ __forceinline__ float floored(float w, float floor) { return (w >= floor || w != w) ? w : floor; }

// The fp32 sum of the block's weights in numpy's pairwise order.
__global__ __launch_bounds__(kWSThreads) void k_ws_block(WSArgs a)
{
    __shared__ float wv[kWSBlock + kWSBlock / kLeaf];
    __shared__ int leaf_s[kMaxLeaves], leaf_l[kMaxLeaves];
    __shared__ float leaf_v[kMaxLeaves];
    __shared__ int snl;
    const int tid = threadIdx.x;
    const long b0 = (long)blockIdx.x * kWSBlock;
    const int L = (int)min((long)kWSBlock, a.n - b0);
    if (L == kWSBlock) {
        // a whole block is a perfect tree: 64 leaves of 128 (halves of 8192,
        // 4096, .., 256), so lane t sums leaf t and a butterfly down the
        // wave adds the subtrees in tree order
        if (tid >= 64) return;
        const float* src = a.w != nullptr ? a.w + b0 + kLeaf * tid : nullptr;
        auto get8 = [&](int i, float* v) {
            if (src == nullptr) {
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] = 1.0f;
                return;
            }
            const float4 p = *reinterpret_cast<const float4*>(src + i);
            const float4 q = *reinterpret_cast<const float4*>(src + i + 4);
            v[0] = floored(p.x, a.floor);
            v[1] = floored(p.y, a.floor);
            v[2] = floored(p.z, a.floor);
            v[3] = floored(p.w, a.floor);
            v[4] = floored(q.x, a.floor);
            v[5] = floored(q.y, a.floor);
            v[6] = floored(q.z, a.floor);
            v[7] = floored(q.w, a.floor);
        };
        float r[8];
        get8(0, r);
#pragma unroll
        for (int i = 8; i < kLeaf; i += 8) {
            float v[8];
            get8(i, v);
#pragma unroll
            for (int j = 0; j < 8; ++j) r[j] += v[j];
        }
        float t = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const float o = __shfl_down(t, off, 64);
            t = t + o;
        }
        if (tid == 0) a.bsum[blockIdx.x] = t;
        return;
    }
    // the last, partial block: the tree of its length, walked by one thread
    for (int i = tid; i < L; i += kWSThreads) wv[pad_idx(i)] = a.w != nullptr ? floored(a.w[b0 + i], a.floor) : 1.0f;
    if (tid == 0) {
        // leaves in order: depth-first, left half first
        int st_s[16], st_l[16], sp = 1, nl = 0;
        st_s[0] = 0;
        st_l[0] = L;
        while (sp > 0) {
            --sp;
            const int s = st_s[sp], l = st_l[sp];
            if (l <= kLeaf) {
                leaf_s[nl] = s;
                leaf_l[nl] = l;
                ++nl;
            } else {
                const int h = pw_half(l);
                st_s[sp] = s + h;
                st_l[sp] = l - h;
                ++sp;
                st_s[sp] = s;
                st_l[sp] = h;
                ++sp;
            }
        }
        snl = nl;
    }
    __syncthreads();
    if (tid < snl) {
        const int s = leaf_s[tid], l = leaf_l[tid];
        float res;
        if (l < 8) {
            res = 0.0f;
            for (int i = 0; i < l; ++i) res += wv[pad_idx(s + i)];
        } else {
            float r[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) r[j] = wv[pad_idx(s + j)];
            int i = 8;
            for (; i < l - l % 8; i += 8) {
#pragma unroll
                for (int j = 0; j < 8; ++j) r[j] += wv[pad_idx(s + i + j)];
            }
            res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
            for (; i < l; ++i) res += wv[pad_idx(s + i)];
        }
        leaf_v[tid] = res;
    }
    __syncthreads();
    if (tid == 0) {
        // post-order over the same tree: a node's value is left + right
        int len[10], ph[10];
        float lv[10];
        int d = 0, next = 0;
        len[0] = L;
        ph[0] = 0;
        float ret = 0.0f;
        for (;;) {
            if (len[d] <= kLeaf) {
                ret = leaf_v[next++];
                bool up = true;
                while (up) {
                    if (d == 0) {
                        a.bsum[blockIdx.x] = ret;
                        return;
                    }
                    --d;
                    if (ph[d] == 0) {
                        lv[d] = ret;
                        ph[d] = 1;
                        len[d + 1] = len[d] - pw_half(len[d]);
                        ph[d + 1] = 0;
                        ++d;
                        up = false;
                    } else {
                        ret = lv[d] + ret;
                    }
                }
            } else {
                len[d + 1] = pw_half(len[d]);
                ph[d + 1] = 0;
                ++d;
            }
        }
    }
}

constexpr int kSeqTile = 1024;  // values per LDS tile of a sequential running sum

// Running sum of v[0 .. m) in order, by thread 0 over LDS tiles the block
// fills: out[i] (nullable) = sum of v[0 .. i]; returns the total in thread 0.
template <typename T>
__device__ T seq_running_sum(const T* v, int m, T* out, T* tile)
{
    const int tid = threadIdx.x;
    T s = T(0);
    for (int c0 = 0; c0 < m; c0 += kSeqTile) {
        const int len = min(kSeqTile, m - c0);
        for (int i = tid; i < len; i += blockDim.x) tile[i] = v[c0 + i];
        __syncthreads();
        if (tid == 0) {
            int i = 0;
            for (; i + 8 <= len; i += 8) {
                T u[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) u[j] = tile[i + j];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    s += u[j];
                    tile[i + j] = s;
                }
            }
            for (; i < len; ++i) {
                s += tile[i];
                tile[i] = s;
            }
        }
        __syncthreads();
        if (out != nullptr)
            for (int i = tid; i < len; i += blockDim.x) out[c0 + i] = tile[i];
        __syncthreads();
    }
    return s;
}

// numpy's running total over the blocks, in block order.
__global__ __launch_bounds__(kWSThreads) void k_ws_total(WSArgs a, int nb)
{
    __shared__ float tile[kSeqTile];
    const float r = seq_running_sum<float>(a.bsum, nb, nullptr, tile);
    if (threadIdx.x == 0) *a.total = r;
}

// fp64 sum of this block's 8 values per thread, in a fixed order (thread,
// then wave butterfly, then the four waves in order); valid in thread 0.
__device__ __forceinline__ double block_sum4(double v, double* red)
{
    const int tid = threadIdx.x;
    v = wave_sum(v);
    if ((tid & 63) == 0) red[tid >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// p_i = fp64(fp32(floored(w_i) / total)); chunk sums of p and counts of p > 0.
__global__ __launch_bounds__(kWSThreads) void k_ws_prob(WSArgs a)
{
    __shared__ double red[4];
    __shared__ int redc[4];
    const int tid = threadIdx.x;
    const long c0 = (long)blockIdx.x * kWSChunk;
    const float tot = *a.total;
    double s = 0.0;
    int nz = 0;
#pragma unroll
    for (int j = 0; j < kWSChunk / kWSThreads; ++j) {
        const long i = c0 + tid + j * kWSThreads;
        if (i < a.n) {
            const float w = a.w != nullptr ? floored(a.w[i], a.floor) : 1.0f;
            const double p = (double)__fdiv_rn(w, tot);
            a.p[i] = p;
            s += p;
            nz += p > 0.0;
        }
    }
    const double cs = block_sum4(s, red);
    int c = nz;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) c += __shfl_xor(c, off, 64);
    if ((tid & 63) == 0) redc[tid >> 6] = c;
    __syncthreads();
    if (tid == 0) {
        a.ctot[blockIdx.x] = cs;
        a.cnz[blockIdx.x] = redc[0] + redc[1] + redc[2] + redc[3];
    }
}

// p[zero[t]] = 0 (numpy's p[found] = 0 before a further pass).
__global__ void k_ws_zero(WSArgs a)
{
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t < a.nz) a.p[a.zero[t]] = 0.0;
}

// Chunk sums of p again (after zeroing), same order as k_ws_prob.
__global__ __launch_bounds__(kWSThreads) void k_ws_ctot(WSArgs a)
{
    __shared__ double red[4];
    const int tid = threadIdx.x;
    const long c0 = (long)blockIdx.x * kWSChunk;
    double s = 0.0;
#pragma unroll
    for (int j = 0; j < kWSChunk / kWSThreads; ++j) {
        const long i = c0 + tid + j * kWSThreads;
        if (i < a.n) s += a.p[i];
    }
    const double cs = block_sum4(s, red);
    if (tid == 0) a.ctot[blockIdx.x] = cs;
}

// pfx[c] = sum of chunks 0 .. c-1 in chunk order (non-decreasing), pfx[nc] =
// the total; with counts: nnz = number of p > 0.
__global__ __launch_bounds__(kWSThreads) void k_ws_prefix(WSArgs a, int nc, int counts)
{
    __shared__ double tile[kSeqTile];
    __shared__ long long zs[kWSThreads / 64];
    const int tid = threadIdx.x;
    if (tid == 0) a.pfx[0] = 0.0;
    (void)seq_running_sum<double>(a.ctot, nc, a.pfx + 1, tile);
    if (!counts) return;
    long long z = 0;
    for (int c = tid; c < nc; c += kWSThreads) z += a.cnz[c];
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) z += __shfl_xor(z, off, 64);
    if ((tid & 63) == 0) zs[tid >> 6] = z;
    __syncthreads();
    if (tid == 0) *a.nnz = zs[0] + zs[1] + zs[2] + zs[3];
}

// Certified searchsorted of u[t] (one block per draw).
__global__ __launch_bounds__(kWSThreads) void k_ws_search(WSArgs a, int nc)
{
    __shared__ int sb;
    __shared__ double red[4];
    __shared__ int redc[4];
    __shared__ double nb_lo, nb_hi;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const double u = a.u[blockIdx.x];
    const double T = a.pfx[nc];
    constexpr double eps = 0x1p-53;
    // numpy's sum has n - 1 additions on every path; this block's has at most
    // nc + 64 (chunk prefix, chunk tree, wave scan and the subtraction that
    // turns it exclusive, each within a unit roundoff per level)
    const double ne = (double)(a.n + nc + 64) * eps;
    const double gam = ne / (1.0 - ne);
    const double B = 2.0 * gam * (T / (1.0 - gam));  // |cdf sums, either order - exact| summed
    const bool ok = T > 0.0 && B <= 0.01 * T;        // false for a NaN total
    const double Dl = fmax(2.1 * B / (T - B) + 8.0 * eps, a.dmin);
    if (tid == 0) {
        // the last chunk whose prefix / T <= u (pfx[0] = 0)
        int lo = 1, hi = nc;
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (a.pfx[mid] / T <= u) lo = mid + 1;
            else hi = mid;
        }
        sb = lo - 1;
    }
    __syncthreads();
    const int b = sb;
    const long c0 = (long)b * kWSChunk;
    const int len = (int)min((long)kWSChunk, a.n - c0);
    constexpr int PT = kWSChunk / kWSThreads;  // 8 consecutive rows per thread
    double loc[PT];
    double run = 0.0;
#pragma unroll
    for (int j = 0; j < PT; ++j) {
        const int i = tid * PT + j;
        run += i < len ? a.p[c0 + i] : 0.0;
        loc[j] = run;
    }
    // exclusive scan of the thread totals: wave inclusive scan, then wave bases
    double inc = run;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const double o = __shfl_up(inc, off, 64);
        if (lane >= off) inc += o;
    }
    if (lane == 63) red[wv] = inc;
    __syncthreads();
    double wb = 0.0;
    for (int w = 0; w < wv; ++w) wb += red[w];
    const double ex = wb + (inc - run);
    const double base = a.pfx[b];
    double cv[PT];
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < PT; ++j) {
        cv[j] = (base + (ex + loc[j])) / T;
        cnt += (tid * PT + j < len && cv[j] <= u) ? 1 : 0;
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) cnt += __shfl_xor(cnt, off, 64);
    if (lane == 0) redc[wv] = cnt;
    __syncthreads();
    const int count = redc[0] + redc[1] + redc[2] + redc[3];
    const long r = c0 + count;
    // the approximations of cdf[r - 1] and cdf[r]
    if (tid == 0) {
        nb_lo = count == 0 ? (b == 0 ? -DBL_MAX : base / T) : 0.0;
        nb_hi = DBL_MAX;
        if (count == len) nb_hi = r < a.n ? (a.pfx[b + 1] + a.p[r]) / T : -DBL_MAX;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < PT; ++j) {
        const int i = tid * PT + j;
        if (count > 0 && i == count - 1) nb_lo = cv[j];
        if (count < len && i == count) nb_hi = cv[j];
    }
    __syncthreads();
    if (tid == 0) {
        const bool sure = ok && (nb_lo == -DBL_MAX || u - nb_lo > Dl) && nb_hi - u > Dl;
        a.out[blockIdx.x] = r;
        a.unsure[blockIdx.x] = sure ? 0 : 1;
    }
}

// numpy's cumsum of p, exactly, chunk by chunk (one block): s = the sum before
// chunk c.  While the running sum stays in one binade [2^e, 2^(e+1)), every
// double there is a multiple of g = 2^(e-52), so fl(s + p) = s + g RN(p / g):
// the chunk's sums are s + g Q_i with Q_i an exact int64 prefix of q_j =
// RN(p_j / g).  A chunk is walked in row order by one thread instead when s is
// 0, when its sum leaves the binade, or when some p_j / g ends in exactly .5
// (a tie, whose rounding depends on the running sum's last bit).  cst[c] = s
// before chunk c (cst[nc] = the total), cseq[c] = 1 for a walked chunk.
__device__ __forceinline__ bool grid_q(double v, int e, long long& q)
{
    const double w = ldexp(v, 52 - e);  // exact
    if (w >= 0x1p52) return false;
    const double fl = floor(w), fr = w - fl;  // exact
    if (fr == 0.5) return false;
    q = (long long)fl + (fr > 0.5 ? 1 : 0);
    return true;
}

__global__ __launch_bounds__(kWSThreads) void k_ws_chain(WSArgs a, int nc)
{
    constexpr int PT = kWSChunk / kWSThreads;
    __shared__ double tile[kWSChunk];
    __shared__ long long qred[kWSThreads / 64];
    __shared__ int bred[kWSThreads / 64];
    __shared__ double walked;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    double s = 0.0;
    for (int c = 0; c < nc; ++c) {
        const long c0 = (long)c * kWSChunk;
        const int len = (int)min((long)kWSChunk, a.n - c0);
        double v[PT];
#pragma unroll
        for (int j = 0; j < PT; ++j) {
            const int i = tid + kWSThreads * j;
            v[j] = i < len ? a.p[c0 + i] : 0.0;
            tile[i] = v[j];
        }
        long long q = 0;
        int bad = s > 0.0 ? 0 : 1;
        const int e = s > 0.0 ? ilogb(s) : 0;
        if (!bad) {
#pragma unroll
            for (int j = 0; j < PT; ++j) {
                long long qj = 0;
                if (!grid_q(v[j], e, qj)) bad = 1;
                q += qj;
            }
        }
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            q += __shfl_xor(q, off, 64);
            bad |= __shfl_xor(bad, off, 64);
        }
        if (lane == 0) {
            qred[wv] = q;
            bred[wv] = bad;
        }
        __syncthreads();
        const long long Q = (qred[0] + qred[1]) + (qred[2] + qred[3]);
        bool ok = (bred[0] | bred[1] | bred[2] | bred[3]) == 0 && Q < (1LL << 53);
        double next = s;
        if (ok) {
            next = s + ldexp((double)Q, e - 52);  // a multiple of g: exact while below 2^(e+1)
            ok = next < ldexp(1.0, e + 1);
        }
        if (tid == 0) {
            a.cst[c] = s;
            a.cseq[c] = ok ? 0 : 1;
        }
        if (!ok) {
            if (tid == 0) {
                double r = s;
                for (int i = 0; i < len; ++i) r += tile[i];
                walked = r;
            }
            __syncthreads();
            next = walked;
        }
        s = next;
        __syncthreads();  // the tile and the reductions are reused
    }
    if (tid == 0) a.cst[nc] = s;
}

// searchsorted(cumsum / cumsum[n - 1], u, side="right") for the unsure draws
// (every draw with all != 0), one block per draw: the chunk whose end is the
// first above u, then its sums rebuilt as k_ws_chain formed them.
__global__ __launch_bounds__(kWSThreads) void k_ws_exact_search(WSArgs a, int nc, int all)
{
    constexpr int PT = kWSChunk / kWSThreads;
    __shared__ int csh;
    __shared__ long long qex[kWSThreads / 64];
    __shared__ int cred[kWSThreads / 64];
    const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    if (!(all || a.unsure[t])) return;
    const double u = a.u[t];
    const double T = a.cst[nc];
    if (tid == 0) {
        int lo = 0, hi = nc - 1;  // cst[nc] / T = 1 > u: the last chunk qualifies
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (a.cst[mid + 1] / T <= u) lo = mid + 1;
            else hi = mid;
        }
        csh = lo;
    }
    __syncthreads();
    const int c = csh;
    const long c0 = (long)c * kWSChunk;
    const int len = (int)min((long)kWSChunk, a.n - c0);
    const double s0 = a.cst[c];
    int count = 0;
    if (a.cseq[c] != 0) {
        if (tid == 0) {
            double r = s0;
            for (int i = 0; i < len; ++i) {
                r += a.p[c0 + i];
                if (r / T > u) break;
                ++count;
            }
            cred[0] = count;
        }
        __syncthreads();
        count = cred[0];
    } else {
        // thread tid holds rows PT tid .. PT tid + PT - 1: local prefixes, then
        // an exclusive scan of the thread totals (int64, exact)
        const int e = ilogb(s0);
        long long loc[PT], run = 0;
#pragma unroll
        for (int j = 0; j < PT; ++j) {
            const int i = PT * tid + j;
            long long qj = 0;
            if (i < len) (void)grid_q(a.p[c0 + i], e, qj);  // the chain checked every q_j
            run += qj;
            loc[j] = run;
        }
        long long inc = run;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const long long o = __shfl_up(inc, off, 64);
            if (lane >= off) inc += o;
        }
        if (lane == 63) qex[wv] = inc;
        __syncthreads();
        long long base = inc - run;
        for (int w = 0; w < wv; ++w) base += qex[w];
        int cnt = 0;
#pragma unroll
        for (int j = 0; j < PT; ++j) {
            const int i = PT * tid + j;
            const double si = s0 + ldexp((double)(base + loc[j]), e - 52);
            cnt += (i < len && si / T <= u) ? 1 : 0;
        }
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) cnt += __shfl_xor(cnt, off, 64);
        if (lane == 0) cred[wv] = cnt;
        __syncthreads();
        count = cred[0] + cred[1] + cred[2] + cred[3];
    }
    if (tid == 0) a.out[t] = c0 + count;
}

}  // namespace

int ws_blocks(long n) { return (int)((n + kWSBlock - 1) / kWSBlock); }
int ws_chunks(long n) { return (int)((n + kWSChunk - 1) / kWSChunk); }

hipError_t launch_ws_prepare(const WSArgs& a, hipStream_t s)
{
    const int nb = ws_blocks(a.n), nc = ws_chunks(a.n);
    hipLaunchKernelGGL(k_ws_block, dim3(nb), dim3(kWSThreads), 0, s, a);
    hipLaunchKernelGGL(k_ws_total, dim3(1), dim3(kWSThreads), 0, s, a, nb);
    hipLaunchKernelGGL(k_ws_prob, dim3(nc), dim3(kWSThreads), 0, s, a);
    hipLaunchKernelGGL(k_ws_prefix, dim3(1), dim3(kWSThreads), 0, s, a, nc, 1);
    return hipGetLastError();
}

hipError_t launch_ws_zero(const WSArgs& a, hipStream_t s)
{
    const int nc = ws_chunks(a.n);
    hipLaunchKernelGGL(k_ws_zero, dim3((a.nz + 255) / 256), dim3(256), 0, s, a);
    hipLaunchKernelGGL(k_ws_ctot, dim3(nc), dim3(kWSThreads), 0, s, a);
    hipLaunchKernelGGL(k_ws_prefix, dim3(1), dim3(kWSThreads), 0, s, a, nc, 0);
    return hipGetLastError();
}

hipError_t launch_ws_search(const WSArgs& a, hipStream_t s)
{
    hipLaunchKernelGGL(k_ws_search, dim3(a.m), dim3(kWSThreads), 0, s, a, ws_chunks(a.n));
    return hipGetLastError();
}

hipError_t launch_ws_exact(const WSArgs& a, int all, hipStream_t s)
{
    const int nc = ws_chunks(a.n);
    hipLaunchKernelGGL(k_ws_chain, dim3(1), dim3(kWSThreads), 0, s, a, nc);
    hipLaunchKernelGGL(k_ws_exact_search, dim3(a.m), dim3(kWSThreads), 0, s, a, nc, all);
    return hipGetLastError();
}

}  // namespace skm
