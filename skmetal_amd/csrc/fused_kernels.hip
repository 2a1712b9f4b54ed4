// fused_kernels.hip -- one-pass Lloyd step for small k*d on gfx950 (MI355X):
// the E-step (sklearn/cluster/_k_means_lloyd.pyx:196-212) and the
// per-cluster sums and counts of the M-step (:214-218) in one kernel that
// reads X from HBM once per step, plus the split E-step for any k.
//
//   k_fused3    E-step and per-cluster sums on bf16 MFMAs over an exact
//               three-part bf16 split of x and c (fp32 accumulation);
//               12 waves per block (d >= 17).
//   k_fused     E-step on fp32 MFMA, per-cluster sums by a VALU walker; 8
//               waves per block (d <= 16, data outside the split's range, or
//               the fp32 switch).
//   k_assign3   E-step alone for any k over the same split (the generic path).
//
// The fused kernels are used when k <= 64 and d <= 100; X's row stride ld is
// then padded (with zeros) to 4*NQ floats for one of the compiled NQ, so the
// kernels' loops over the row's float4s have no bounds.  The separate assign
// / update kernels cover every other shape.
//
// Built without -amdgpu-mfma-vgpr-form (the register allocator places the
// MFMA accumulators).
#include <math.h>
#include <stdlib.h>

#include "device.h"

namespace skm {

// A block is 8 waves, two per SIMD: MFMA waves 0-3 and walker waves 4-7.
// MFMA wave p and walker wave 4+p form pair p and share one 64-row LDS tile;
// pair p of block b handles tiles t = 4b + p + r*P (P = 4 * blocks) in
// rounds r.  A wave cannot issue VALU work while its own MFMAs run, but the
// other wave on the same SIMD can, so the walker's adds overlap the MFMA
// wave's E-step.  The two waves of a pair hand tiles over through LDS flags;
// there is no block barrier until the end.
//
//   MFMA wave  holds tile t's row in registers (one row per lane) and runs
//              the E-step as k_assign does: x.c on v_mfma_f32_4x4x1_16b_f32
//              (B = this lane's row, A = centres from LDS, lane j = cluster
//              j), ||c||^2 - 2 x.c and the first minimum in the lane.  From
//              chunk K on, each chunk is written to the pair's LDS tile right
//              after its MFMAs (once the walker has read that chunk of tile
//              t - P: it publishes its progress per chunk) and its registers
//              are reloaded with tile t + P, so the HBM reads spread over the
//              E-step.  Chunks [0, K) are held in one
//              of two register sets (by round parity), written out after the
//              argmin and reloaded with tile t + 2P.  Then the tile's rows of
//              each cluster go to LDS as bit masks (an LDS atomic OR of
//              1 << lane into mask[label]; OR does not depend on the order the
//              lanes land in) and the tile is flagged ready.
//   walker     lane j adds the ready tile's rows of cluster j to its running
//              sums of every column, in registers: the lowest WS bits of its
//              mask become LDS row offsets (unused ones point at a row of
//              zeros, so the walk is a fixed sequence), rows past the first
//              WS by a loop; it flags each chunk as soon as its reads are
//              issued.
//
// Rows are added in ascending row order per cluster (the first WS rows after
// the others), tiles in round order, and the four walkers are combined in
// wave order: bitwise reproducible.

// Rows per (cluster, tile) walked without a loop: about the mean 64/k plus
// three standard deviations for balanced clusters.
template <int KG>
__host__ __device__ constexpr int walk_steps()
{
    return KG >= 12 ? 6 : KG >= 8 ? 8 : KG >= 4 ? 12 : 16;
}

// Floats per LDS row for a row of NQ float4s: an odd number of float4s, so
// 16-byte accesses of different rows at the same column fall in different
// bank groups.
__host__ __device__ constexpr int fused_stride(int nq) { return 4 * (nq | 1); }

// Buffer descriptor over the rows of tile t (none past the last row: loads
// there return 0 without a memory access).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const float* X, long t, long n, int ld)
{
    const long r0 = t * 64;
    const long rows = n - r0 < 64 ? (n - r0 > 0 ? n - r0 : 0) : 64;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(X + (rows > 0 ? r0 * ld : 0)), (short)0,
                                             (int)(rows * ld * 4), 0x00020000);
}

__device__ __forceinline__ float4 load_quad(__amdgpu_buffer_rsrc_t rs, int off)
{
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
    return *reinterpret_cast<const float4*>(&v);
}

// Waits (polling LDS) until *flag >= v and returns the value seen.  Flags are
// written by the other wave of the pair; LDS operations of one wave are
// performed in issue order, so a wave that sees a flag value also sees the
// LDS writes issued before it, and LDS reads issued before it are done.
__device__ __forceinline__ int wait_flag(int* flag, int v)
{
    int seen;
    while ((seen = __hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) < v)
        __builtin_amdgcn_s_sleep(1);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);  // no LDS access moves above the wait
    return seen;
}

__device__ __forceinline__ void set_flag(int* flag, int v)
{
    __atomic_signal_fence(__ATOMIC_SEQ_CST);  // every LDS access above stays above
    __hip_atomic_store(flag, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// First minimum of d[0..N) with its index, as a pairwise tree in which the
// lower-index side wins ties -- the same result as scanning j upward with a
// strict '<' from +inf (NaN never wins: leaves are clamped to +inf first).
template <int N>
__device__ __forceinline__ int argmin_tree(float* d)
{
    int ix[N];
#pragma unroll
    for (int j = 0; j < N; ++j) {
        d[j] = fminf(d[j], INFINITY);
        ix[j] = j;
    }
#pragma unroll
    for (int w = 1; w < N; w *= 2) {
#pragma unroll
        for (int j = 0; j + w < N; j += 2 * w) {
            const bool take = d[j + w] < d[j];
            d[j] = take ? d[j + w] : d[j];
            ix[j] = take ? ix[j + w] : ix[j];
        }
    }
    return ix[0];
}

// Wave 4 of every block: the previous step's stopping rules when a.decide
// (evaluated identically by every block: same loads, same order as
// k_finalize_loop for k <= 64; block 0 records the decision), else nothing
// to decide.  Writes ||c||^2 of this step's centres to sN (padding clusters
// j >= k get +inf: their distance never wins) and the decision to *sDone.
template <int CPC>
__device__ __forceinline__ void step_norms(const FusedArgs& a, int lane, float* sN, int* sDone)
{
    const int k = a.k;
    const int j = lane;
    if (a.decide) {
        double tsq = 0.0, tnr = 0.0;
        int count = 1;
        if (j < k) {
            // all chunk partials in flight at once (the sum order is the
            // finalize's: chunk 0, 1, ...)
            const double* pj = a.part + (long)j * a.nch * 2;
            constexpr int NB = 16;
            for (int c0 = 0; c0 < a.nch; c0 += NB) {
                double v[2 * NB];
#pragma unroll
                for (int u = 0; u < NB; ++u) {
                    const int c = min(c0 + u, a.nch - 1);
                    v[2 * u] = pj[2 * c];
                    v[2 * u + 1] = pj[2 * c + 1];
                }
#pragma unroll
                for (int u = 0; u < NB; ++u) {
                    if (c0 + u < a.nch) {
                        tsq += v[2 * u];
                        tnr += v[2 * u + 1];
                    }
                }
            }
            count = a.counts[j];
        }
        const int n_empty = wave_sum(j < k && count == 0 ? 1 : 0);
        const double tot = wave_sum(j < k ? (double)(float)tsq : 0.0);
        const int chg = *a.prev_changed;
        int done = 0;
        if (n_empty > 0)
            done = 3;
        else if ((a.flags & kStopStrict) && chg == 0)
            done = 1;
        else if (a.tol >= 0.0 && tot <= a.tol)  // tol < 0: no shift rule (fixed iterations)
            done = 2;
        if (blockIdx.x == 0) {
            LoopState* st = a.state;
            if (j < k) {
                a.shift_sq[j] = (float)tsq;
                if (count > 0) a.cnorm_out[j] = (float)tnr;
            }
            if (lane == 0) {
                st->n_empty = n_empty;
                st->shift_tot = tot;
                st->last_changed = chg;
                st->n_iter = a.iter;
                if (done != 0) st->halt_iter = a.iter - 1;
                st->done = done;
            }
        }
        if (j < CPC) sN[j] = j < k ? (float)tnr : INFINITY;
        if (lane == 0) *sDone = done;
    } else {
        if (j < CPC) sN[j] = j < k ? a.cnorm[j] : INFINITY;
        if (lane == 0) *sDone = 0;
    }
}

// The walker wave of a pair: for every round, waits for the tile, then lane j
// adds the tile's rows of cluster j (its mask) to S, publishing its progress
// per chunk; cnt counts the rows.
template <int CPC, int WS, int NQ, int XS>
__device__ __forceinline__ void walk_tiles(float4 (&S)[NQ], int& cnt, int rounds, int lane, int* ready, int* prog,
                                           const unsigned long long* mask, const char* lbase, int toff, int zoff)
{
#pragma unroll
    for (int q = 0; q < NQ; ++q) S[q] = make_float4(0.f, 0.f, 0.f, 0.f);
    cnt = 0;
    for (int r = 0; r < rounds; ++r) {
        wait_flag(ready, r + 1);
        unsigned long long m = lane < CPC ? mask[lane] : 0ull;
        cnt += (int)__popcll(m);
        int ro[WS];
#pragma unroll
        for (int s = 0; s < WS; ++s) {
            const int rr = __ffsll((long long)m) - 1;
            ro[s] = m != 0ull ? toff + rr * XS * 4 : zoff;
            m &= m - 1ull;
        }
        // rows past the first WS (ascending) first, then the first WS: a
        // fixed order either way
        if (__ballot(m != 0ull) != 0ull) {
            while (m != 0ull) {
                const int rr = __ffsll((long long)m) - 1;
                m &= m - 1ull;
                const char* src = lbase + toff + rr * XS * 4;
#pragma unroll
                for (int q = 0; q < NQ; ++q) {
                    const float4 v = *reinterpret_cast<const float4*>(src + 16 * q);
                    S[q].x += v.x;
                    S[q].y += v.y;
                    S[q].z += v.z;
                    S[q].w += v.w;
                }
            }
        }
        float4 wv[WS];
#pragma unroll
        for (int s = 0; s < WS; ++s) wv[s] = *reinterpret_cast<const float4*>(lbase + ro[s]);
        set_flag(prog, r * NQ + 1);
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            float4 wn[WS];
            if (q + 1 < NQ) {
#pragma unroll
                for (int s = 0; s < WS; ++s) wn[s] = *reinterpret_cast<const float4*>(lbase + ro[s] + 16 * (q + 1));
                set_flag(prog, r * NQ + q + 2);  // reads issued: LDS keeps their order
            }
#pragma unroll
            for (int s = 0; s < WS; ++s) {
                S[q].x += wv[s].x;
                S[q].y += wv[s].y;
                S[q].z += wv[s].z;
                S[q].w += wv[s].w;
            }
            if (q + 1 < NQ) {
#pragma unroll
                for (int s = 0; s < WS; ++s) wv[s] = wn[s];
            }
        }
    }
}

// After the tiles: every walker's sums into red = [4][CPC][ld] (over the tile
// area, once every pair is done with it), then the block's partial sums and
// counts, the four walkers combined in wave order.
template <int CPC, int NQ>
__device__ __forceinline__ void publish_sums(const float4 (&S)[NQ], int cnt, float* red, int ld, int pair, int lane,
                                             int (*sCnt)[64])
{
    if (lane < CPC) {
        float* dst = red + (pair * CPC + lane) * ld;
#pragma unroll
        for (int q = 0; q < NQ; ++q) *reinterpret_cast<float4*>(dst + 4 * q) = S[q];
        sCnt[pair][lane] = cnt;
    }
}

template <int CPC, int NT = 512>
__device__ __forceinline__ void combine_sums(const float* red, int ld, int k, float* psum, int* pcnt, int (*sCnt)[64],
                                             int tid)
{
    const int kl = k * ld;
    float* out = psum + (long)blockIdx.x * kl;
    for (int i = tid; i < kl; i += NT) {
        const int j = i / ld;
        const int col = i - j * ld;
        const float* p = red + j * ld + col;
        out[i] = ((p[0] + p[CPC * ld]) + p[2 * CPC * ld]) + p[3 * CPC * ld];
    }
    if (tid < k) pcnt[(long)blockIdx.x * k + tid] = ((sCnt[0][tid] + sCnt[1][tid]) + sCnt[2][tid]) + sCnt[3][tid];
}

template <int KG, int NQ>
__global__ __launch_bounds__(512, 1) void k_fused(FusedArgs a)
{
    const float* __restrict__ X = a.X;
    const long n = a.n;
    const int ld = a.ld;
    const float* __restrict__ C = a.C;
    const int k = a.k;
    int* __restrict__ labels = a.labels;
    float* __restrict__ psum = a.psum;
    int* __restrict__ pcnt = a.pcnt;
    LoopState* st = a.state;
    constexpr int CPC = 4 * KG;
    constexpr int WS = walk_steps<KG>();
    constexpr int XS = fused_stride(NQ);      // ld == 4 * NQ
    constexpr int K = NQ >= 8 ? 3 : NQ / 2;  // chunks computed before the LDS tile is reused
    constexpr int KA = K > 0 ? K : 1;
    constexpr int LB = 8;                     // chunks per burst of HBM loads
    // LDS: centres [CPC x XS] | zero row [XS] | 4 pair tiles [64 x XS]
    extern __shared__ __attribute__((aligned(16))) float lds[];
    __shared__ unsigned long long sMask[4][64];
    __shared__ int sCnt[4][64];
    __shared__ __attribute__((aligned(16))) float sN[CPC];
    __shared__ int sReady[4];  // tiles the MFMA wave has put in LDS
    __shared__ int sProg[4];   // chunks the walker has read: tile * NQ + chunk
    __shared__ int sDone;      // nonzero: the loop has halted, nothing to do
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: keeps descriptors scalar
    const int pair = wave & 3;

    float* sC = lds;
    float* zrow = lds + CPC * XS;
    float* tile = zrow + XS + pair * 64 * XS;
    const int zoff = CPC * XS * 4;  // byte offsets from `lds`
    const int toff = (CPC + 1 + pair * 64) * XS * 4;
    const char* lbase = reinterpret_cast<const char*>(lds);

    const long ntiles = (n + 63) >> 6;
    const long P = (long)gridDim.x * 4;
    const long t0 = (long)blockIdx.x * 4 + pair;
    const int rounds = t0 < ntiles ? (int)((ntiles - t0 + P - 1) / P) : 0;  // this pair's tiles
    const int xoff = lane * ld * 4;  // this lane's row inside a tile of X

    if (wave < 4) {
        // MFMA wave.  Tile t's row: chunks [0, K) in pre (two sets, one per
        // round parity, loaded a round ahead), chunks [K, NQ) in xv.  The
        // first tiles are requested before anything else: their HBM latency
        // overlaps the walkers' set-up.
        float4 preA[KA], preB[KA], xv[NQ - K];
        const __amdgpu_buffer_rsrc_t r0 = tile_rsrc(X, t0, n, ld);
        const __amdgpu_buffer_rsrc_t r1 = tile_rsrc(X, t0 + P, n, ld);
#pragma unroll
        for (int q = 0; q < K; ++q) preA[q] = load_quad(r0, xoff + 16 * q);
#pragma unroll
        for (int q = K; q < NQ; ++q) xv[q - K] = load_quad(r0, xoff + 16 * q);
#pragma unroll
        for (int q = 0; q < K; ++q) preB[q] = load_quad(r1, xoff + 16 * q);
        __syncthreads();  // LDS set up by the walkers
        if (sDone != 0) return;
        const char* cbase = reinterpret_cast<const char*>(sC + (lane < CPC ? lane : CPC - 1) * XS);
        float* myrow = tile + lane * XS;
        int changed = 0;

        auto round = [&](int r, float4* pre) {
            const long t = t0 + (long)r * P;
            const long nrow = n - t * 64 < 64 ? n - t * 64 : 64;
            const bool valid = lane < nrow;
            // the tile's labels; lanes past the last row fall outside the
            // descriptor (the load returns 0, the store is dropped)
            const __amdgpu_buffer_rsrc_t rl =
                __builtin_amdgcn_make_buffer_rsrc(labels + t * 64, (short)0, (int)(nrow * 4), 0x00020000);
            const int old = __builtin_amdgcn_raw_buffer_load_b32(rl, lane * 4, 0, 0);
            const __amdgpu_buffer_rsrc_t rn = tile_rsrc(X, t + P, n, ld);
            v4f acc[KG];
#pragma unroll
            for (int g = 0; g < KG; ++g) acc[g] = v4f{0.f, 0.f, 0.f, 0.f};
            float4 cv = *reinterpret_cast<const float4*>(cbase);
            int seen = 0;  // walker progress last read
#pragma unroll
            for (int q = 0; q < NQ; ++q) {
                // chunk q of the LDS tile is rewritten below once the walker
                // has read it for tile t - P (it runs well ahead: few polls)
                if (q >= K && r > 0) {
                    const int need = (r - 1) * NQ + q + 1;
                    if (seen < need) seen = wait_flag(&sProg[pair], need);
                }
                const float4 cvn = *reinterpret_cast<const float4*>(cbase + 16 * (q + 1 < NQ ? q + 1 : 0));
                const float4 x = q < K ? pre[q < K ? q : 0] : xv[q < K ? 0 : q - K];
                mfma_groups<KG>(acc, cv.x, x.x);
                mfma_groups<KG>(acc, cv.y, x.y);
                mfma_groups<KG>(acc, cv.z, x.z);
                mfma_groups<KG>(acc, cv.w, x.w);
                if (q >= K) {
                    *reinterpret_cast<float4*>(myrow + 4 * q) = x;
                    // tile t + P into the registers of the last LB chunks,
                    // back to back: the loads of one row's 16-byte pieces
                    // then meet the same cache lines together
                    if ((q - K) % LB == LB - 1 || q == NQ - 1) {
#pragma unroll
                        for (int qq = q - (q - K) % LB; qq <= q; ++qq) xv[qq - K] = load_quad(rn, xoff + 16 * qq);
                    }
                }
                cv = cvn;
                // one chunk per scheduling region: keeps each chunk's load
                // in its chunk, spreading the HBM reads over the E-step
                __builtin_amdgcn_sched_barrier(0);
            }
            // ||c||^2 - 2 x.c, first minimum wins (_k_means_lloyd.pyx:196-212)
            float d[CPC];
#pragma unroll
            for (int g = 0; g < KG; ++g) {
#pragma unroll
                for (int i = 0; i < 4; ++i) d[4 * g + i] = fmaf(-2.0f, acc[g][i], sN[4 * g + i]);
            }
            const int bidx = argmin_tree<CPC>(d);
            __builtin_amdgcn_raw_buffer_store_b32(bidx, rl, lane * 4, 0, 0);
            changed += (int)__popcll(__ballot(valid && old != bidx));
            // held chunks to LDS, then their registers take tile t + 2P
            const __amdgpu_buffer_rsrc_t rn2 = tile_rsrc(X, t + 2 * P, n, ld);
#pragma unroll
            for (int q = 0; q < K; ++q) {
                *reinterpret_cast<float4*>(myrow + 4 * q) = pre[q];
                pre[q] = load_quad(rn2, xoff + 16 * q);
            }
            // the tile's rows of each cluster
            if (lane < CPC) sMask[pair][lane] = 0ull;
            if (valid) atomicOr(&sMask[pair][bidx], 1ull << lane);
            set_flag(&sReady[pair], r + 1);
        };

        int r = 0;
        for (; r + 1 < rounds; r += 2) {
            round(r, preA);
            round(r + 1, preB);
        }
        if (r < rounds) round(r, preA);
        if (lane == 0 && changed != 0) atomicAdd(a.changed, changed);
        __syncthreads();  // every pair's walker is done: the tile area is free
        __syncthreads();  // the walkers' sums are in LDS
    } else {
        // walker waves: the halt test, then centres and the zero row into
        // LDS (all loads in flight at once) and ||c||^2
        const int prev = st->done;  // an earlier step halted the loop
        if (prev != 0) {
            if (tid == 256) sDone = prev;
            __syncthreads();
            return;
        }
        const int wt = tid - 256;
        constexpr int NF = (CPC * NQ + 255) / 256;
        float4 cf[NF];
#pragma unroll
        for (int u = 0; u < NF; ++u) {
            const int idx = wt + 256 * u;
            const int cl = idx / NQ;
            const int q = idx - cl * NQ;
            cf[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (idx < CPC * NQ && cl < k) cf[u] = *reinterpret_cast<const float4*>(C + (long)cl * ld + 4 * q);
        }
#pragma unroll
        for (int u = 0; u < NF; ++u) {
            const int idx = wt + 256 * u;
            const int cl = idx / NQ;
            const int q = idx - cl * NQ;
            if (idx < CPC * NQ) *reinterpret_cast<float4*>(&sC[cl * XS + 4 * q]) = cf[u];
        }
        for (int i = wt; i < XS; i += 256) zrow[i] = 0.f;
        if (wt < 4) {
            sReady[wt] = 0;
            sProg[wt] = 0;
        }
        if (wave == 4) step_norms<CPC>(a, lane, sN, &sDone);
        __syncthreads();
        if (sDone != 0) return;
        // walker
        float4 S[NQ];
        int cnt;
        walk_tiles<CPC, WS, NQ, XS>(S, cnt, rounds, lane, &sReady[pair], &sProg[pair], sMask[pair], lbase, toff,
                                    zoff);
        __syncthreads();  // every pair is done with its tile
        publish_sums<CPC, NQ>(S, cnt, zrow + XS, ld, pair, lane, sCnt);
        __syncthreads();
    }
    combine_sums<CPC>(zrow + XS, ld, k, psum, pcnt, sCnt, tid);
}

// ---------------------------------------------------------------------------
// Three-part bf16 split.  bf16 keeps fp32's exponent range with 8 significant
// bits, so every finite fp32 v with |v| >= 2^-103 is the exact sum of three
// bf16 values, each rounded to nearest:
//   hi = bf16(v),  mid = bf16(v - hi),  lo = (v - hi) - mid.
// v - hi is a multiple of v's fp32 ulp no larger than 2^16 of them, so the fp32
// subtraction is exact; likewise (v - hi) - mid, which is at most 2^8 ulps and
// therefore exactly a bf16.  |mid| <= 2^-8 |v|, |lo| <= 2^-16 |v|.
// A product of two bf16 values is exact in fp32, and the MFMAs accumulate in
// fp32, so
//  - the per-cluster sums (one-hot x hi, x mid, x lo) add every x exactly as
//    given, in fp32 (the one-hot operand is exact);
//  - the E-step takes 6 of the 9 part products of x.c (hh, hm, mh, hl, lh, mm):
//    the three left out (ml, lm, ll) total at most (2^-23 + 2^-32) |x_i c_i|
//    per feature, two units of fp32 roundoff, against the one unit by which an
//    fp32 product of x_i and c_i is itself rounded.

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef unsigned v2u __attribute__((ext_vector_type(2)));
typedef float v2f __attribute__((ext_vector_type(2)));

// (a, b) rounded to nearest even bf16, a in the low half: v_cvt_pk_bf16_f32
__device__ __forceinline__ unsigned pack_bf16(float a, float b)
{
    return __builtin_bit_cast(unsigned, __builtin_convertvector(v2f{a, b}, v2bf));
}
__device__ __forceinline__ float bf16_lo(unsigned p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float bf16_hi(unsigned p) { return __uint_as_float(p & 0xffff0000u); }

// The parts of a and b, as bf16 pairs (a's part in the low half).
__device__ __forceinline__ void split3(float a, float b, unsigned& hi, unsigned& mid, unsigned& lo)
{
    hi = pack_bf16(a, b);
    const float ra = a - bf16_lo(hi), rb = b - bf16_hi(hi);  // exact
    mid = pack_bf16(ra, rb);
    lo = pack_bf16(ra - bf16_lo(mid), rb - bf16_hi(mid));   // exact, and exactly bf16
}

struct Parts8 {
    v8bf h, m, l;
};
struct Parts4 {
    v4s h, m, l;  // 16x16x16 bf16 operands are passed as shorts
};

__device__ __forceinline__ Parts8 split8(float4 u, float4 v)
{
    unsigned h0, h1, h2, h3, m0, m1, m2, m3, l0, l1, l2, l3;
    split3(u.x, u.y, h0, m0, l0);
    split3(u.z, u.w, h1, m1, l1);
    split3(v.x, v.y, h2, m2, l2);
    split3(v.z, v.w, h3, m3, l3);
    return Parts8{__builtin_bit_cast(v8bf, v4u{h0, h1, h2, h3}), __builtin_bit_cast(v8bf, v4u{m0, m1, m2, m3}),
                  __builtin_bit_cast(v8bf, v4u{l0, l1, l2, l3})};
}

__device__ __forceinline__ Parts4 split4(float4 u)
{
    unsigned h0, h1, m0, m1, l0, l1;
    split3(u.x, u.y, h0, m0, l0);
    split3(u.z, u.w, h1, m1, l1);
    return Parts4{__builtin_bit_cast(v4s, v2u{h0, h1}), __builtin_bit_cast(v4s, v2u{m0, m1}),
                  __builtin_bit_cast(v4s, v2u{l0, l1})};
}

// D += A B on bf16: 16x16x32 (8 values per lane) and 16x16x16 (4)
__device__ __forceinline__ v4f mfma_bf16(v8bf a, v8bf b, v4f c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v4f mfma_bf16(v4s a, v4s b, v4f c)
{
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

// acc += the six kept part products of a.b (smaller terms first)
template <typename P>
__device__ __forceinline__ v4f dot6(const P& a, const P& b, v4f acc)
{
    acc = mfma_bf16(a.m, b.m, acc);
    acc = mfma_bf16(a.l, b.h, acc);
    acc = mfma_bf16(a.h, b.l, acc);
    acc = mfma_bf16(a.m, b.h, acc);
    acc = mfma_bf16(a.h, b.m, acc);
    return mfma_bf16(a.h, b.h, acc);
}

// ---------------------------------------------------------------------------
// k_fused3: the fused step with the E-step and the per-cluster sums on bf16
// MFMAs over the three-part split (v_mfma_f32_16x16x32_bf16, and
// v_mfma_f32_16x16x16_bf16 for a last 4-, 8- or 16-feature slice).
//
// MFMA operand layout (16x16x32, checked on the device): lane l holds A[m =
// l%16][kk = 8(l/16) + j] and B[kk = 8(l/16) + j][n = l%16], j < 8, and
// receives D[m = 4(l/16) + i][n = l%16], i < 4; 16x16x16 the same with 4
// values per lane.  In the E-step A = 16 centres (block cb, parts from LDS)
// and B = 16 rows of the tile (group g, from registers), so lane l ends with
// the x.c of row 16g + l%16 and centres 16cb + 4(l/16) + i: the first minimum
// over the lane's 4 CB centres, then over the four lanes l%16 + 16h (lower
// index wins ties: the first minimum over all centres), and lane 16g + r
// keeps row 16g + r's label -- lane = row for the labels and counts.
//
// A block is 12 waves, three per SIMD.  E-step waves e = 0..7 (two per SIMD)
// each work on their own 32-row tiles t = 8b + e + r P, with their own LDS
// tile; sums wave 8 + m serves the two E-step waves m and m + 4 of its SIMD,
// taking their tiles in turn.  Each lane loads its 8 (K32 step) or 4 (tail)
// features of its rows straight from HBM into registers, writes them to the
// wave's LDS tile for the sums wave and reloads them with tile t + P once the
// sums wave has read those columns of the previous tile.  The waves hand over
// work through LDS flags; there is no block barrier until the end.

// The sums wave of SIMD m serves E-step waves m and m + 4 (the same SIMD),
// taking their 32-row tiles in turn: round r of wave m, then round r of wave
// m + 4.  The per-cluster sums of a tile are onehot^T x on
// v_mfma_f32_16x16x32_bf16, once for each part of x.  A = one-hot (16
// clusters x the tile's 32 rows: lane l holds rows 8(l/16) + j for cluster
// 16cb + l%16), B = a part of x (the 32 rows x 16 features of block fb, read
// transposed from the LDS tile); D lane l: clusters 16cb + 4(l/16) + i,
// feature 16fb + l%16.  Progress is published per 16-feature block (all rows
// read).  Columns at and past ld hold whatever the LDS has there (the next
// row's values, never-written padding): their sums are never published.
template <int CB, int NQ, int XS, int NFB>
__device__ __forceinline__ void msum_tiles3(v4f (&S)[CB][NFB], int rounds0, int rounds1, int* ready0, int* ready1,
                                            int* prog0, int* prog1, unsigned* mask0, unsigned* mask1,
                                            const v8bf* onehot, const float* tile0, const float* tile1, int lane)
{
    const int h = lane >> 4, r16 = lane & 15;
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
#pragma unroll
        for (int fb = 0; fb < NFB; ++fb) S[cb][fb] = v4f{0.f, 0.f, 0.f, 0.f};
    }
    const int rmax = rounds0 > rounds1 ? rounds0 : rounds1;
    for (int r = 0; r < rmax; ++r) {
        for (int u = 0; u < 2; ++u) {
            // (selects, not an indexed array: the pointers stay in registers)
            if (r >= (u == 0 ? rounds0 : rounds1)) continue;
            int* const ready = u == 0 ? ready0 : ready1;
            int* const prog = u == 0 ? prog0 : prog1;
            unsigned* const mask = u == 0 ? mask0 : mask1;
            const float* const tile = u == 0 ? tile0 : tile1;
            wait_flag(ready, r + 1);
            // A[cb][j] = 1 when row 8h + j has label 16 cb + r16: byte h of that
            // cluster's row mask, through the one-hot table; then the masks
            // are cleared for the next round (the E-step wave sets the next
            // bits only after this tile's progress flags, which follow)
            v8bf A[CB];
            {
                unsigned mw[CB];
#pragma unroll
                for (int cb = 0; cb < CB; ++cb) mw[cb] = mask[16 * cb + r16];
#pragma unroll
                for (int cb = 0; cb < CB; ++cb) A[cb] = onehot[(mw[cb] >> (8 * h)) & 0xffu];
                if (h == 0) {
#pragma unroll
                    for (int cb = 0; cb < CB; ++cb) mask[16 * cb + r16] = 0u;
                }
            }
            const float* col = tile + 8 * h * XS + 16 * h + r16;  // rows 8h .. 8h + 7 sit 16 h floats further
#pragma unroll
            for (int fb = 0; fb < NFB; ++fb) {
                float cur[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) cur[j] = col[j * XS + 16 * fb];
                // columns of feature block fb have been read for every row
                set_flag(prog, r * NQ + (4 * fb + 4 < NQ ? 4 * fb + 4 : NQ));
                const Parts8 b = split8(make_float4(cur[0], cur[1], cur[2], cur[3]),
                                        make_float4(cur[4], cur[5], cur[6], cur[7]));
#pragma unroll
                for (int cb = 0; cb < CB; ++cb) {
                    S[cb][fb] = mfma_bf16(A[cb], b.l, S[cb][fb]);
                    S[cb][fb] = mfma_bf16(A[cb], b.m, S[cb][fb]);
                    S[cb][fb] = mfma_bf16(A[cb], b.h, S[cb][fb]);
                }
            }
        }
    }
}

// M-step sums into red = [4][CPC][ld], once every pair is done.
template <int CB, int NFB>
__device__ __forceinline__ void publish_msums(const v4f (&S)[CB][NFB], float* red, int ld, int pair, int lane)
{
    const int h = lane >> 4, r16 = lane & 15;
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
#pragma unroll
        for (int fb = 0; fb < NFB; ++fb) {
            const int f = 16 * fb + r16;
            if (f < ld) {
#pragma unroll
                for (int i = 0; i < 4; ++i) red[(pair * 16 * CB + 16 * cb + 4 * h + i) * ld + f] = S[cb][fb][i];
            }
        }
    }
}

// Geometry of k_fused3 for a row of NQ float4s.
template <int NQ>
struct Fused3Geom {
    static constexpr int LDX = 4 * NQ;                       // == ld
    static constexpr int NK = LDX / 32;                      // 32-feature K steps
    static constexpr int TAIL = LDX - 32 * NK;               // features of the last, 16-wide step (0: none)
    static constexpr int NS = NK + (TAIL > 0 ? 1 : 0);       // K steps
    static constexpr int QG = 2 * NK + (TAIL > 0 ? 1 : 0);   // float4s per lane per 16-row group
    static constexpr int TQ = TAIL > 0 ? 2 * NK : 0;         // the tail's float4 (dead code without a tail)
    static constexpr int KP = 32 * NK + (TAIL > 0 ? 16 : 0); // features the MFMAs cover
    static constexpr int CSTR = KP + 8;                      // bf16 per centre row: an odd number of 16-byte units
    static constexpr int XS = fused_stride(NQ);              // LDS row: >= ld floats
    static constexpr int NFB = KP / 16;                      // 16-feature blocks of the sums
    // a wave's tile: row rho at rho * XS + 16 (rho >> 3).  XS is 4 x odd, so
    // 8 XS = 32 (mod 64): without the shift the sums wave's column reads of
    // rows 8h + j (lanes h = 0..3) fall on the same banks in pairs; with it
    // the four h start 48 h (mod 64) apart, distinct in every 32-lane pass.
    // The sums wave reads KP columns of every row: rows past XS floats run
    // into the next row (KP - XS floats of padding after the last one).
    static constexpr int TS = 32 * XS + 48 + (KP > XS ? KP - XS : 0);
    static_assert(TAIL == 0 || TAIL == 4 || TAIL == 8 || TAIL == 16, "one 16-wide step covers the tail");
    static_assert(TS % 4 == 0, "16-byte aligned tiles");
};

template <int CB, int NQ>
__global__ __launch_bounds__(768, 1) void k_fused3(FusedArgs a)
{
    using G = Fused3Geom<NQ>;
    const float* __restrict__ X = a.X;
    const long n = a.n;
    const int ld = a.ld;
    const float* __restrict__ C = a.C;
    const int k = a.k;
    int* __restrict__ labels = a.labels;
    LoopState* st = a.state;
    constexpr int CPC = 16 * CB;  // clusters padded to 16-centre blocks
    constexpr int LDX = G::LDX, NK = G::NK, TAIL = G::TAIL, NS = G::NS, QG = G::QG, TQ = G::TQ, KP = G::KP;
    constexpr int CSTR = G::CSTR, XS = G::XS, NFB = G::NFB, TS = G::TS;
    constexpr int CPART = CPC * CSTR;  // bf16 from one centre part to the next
    // LDS: 8 wave tiles [TS floats] | centre parts hi, mid, lo [CPC x CSTR] bf16
    extern __shared__ __attribute__((aligned(16))) float lds[];
    __shared__ unsigned sMask[8][64];                           // a tile's rows of each cluster (bit = row)
    __shared__ __attribute__((aligned(16))) v8bf sOneHot[256];  // byte b -> its 8 bits as bf16 0 / 1
    __shared__ int sCnt[4][64];                                 // rows per cluster, per SIMD
    __shared__ __attribute__((aligned(16))) float sN[CPC];
    __shared__ int sReady[8];  // tiles E-step wave e has labelled
    __shared__ int sProg[8];   // columns of e's tile the sums wave has read: tile * NQ + chunk
    __shared__ int sDone;      // nonzero: the loop has halted, nothing to do
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 4;    // this lane's K slice / centre quad in the MFMA layout
    const int r16 = lane & 15;  // this lane's row of a 16-row group / centre of a block

    float* tiles = lds;
    __bf16* sCP = reinterpret_cast<__bf16*>(tiles + 8 * TS);

    // 32-row tiles: E-step wave e of block b handles t = 8b + e + r*P
    const long ntiles = (n + 31) >> 5;
    const long P = (long)gridDim.x * 8;
    auto rounds_of = [&](int e) {
        const long t0 = (long)blockIdx.x * 8 + e;
        return t0 < ntiles ? (int)((ntiles - t0 + P - 1) / P) : 0;
    };

    if (wave < 8) {
        // E-step wave e (SIMD e % 4).  xr[g] holds this lane's features of
        // row 16g + l%16 of the tile: K32 step s in xr[g][2s], xr[g][2s + 1]
        // (features 32s + 8h + 0..7), the tail in xr[g][2NK] (features 32NK +
        // 4h + 0..3; lanes past the row's last feature load nothing: zeros)
        const int e = wave;
        const long t0 = (long)blockIdx.x * 8 + e;
        const int rounds = rounds_of(e);
        float4 xr[2][QG];
        auto rsrc32 = [&](long t) {
            const long r0 = t * 32;
            const long rows = n - r0 < 32 ? (n - r0 > 0 ? n - r0 : 0) : 32;
            return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(X + (rows > 0 ? r0 * ld : 0)), (short)0,
                                                     (int)(rows * ld * 4), 0x00020000);
        };
        auto load_step = [&](__amdgpu_buffer_rsrc_t rs, int g, int s) {
            if (s < NK) {
                const int o = ((16 * g + r16) * LDX + 32 * s + 8 * h) * 4;
                xr[g][2 * s] = load_quad(rs, o);
                xr[g][2 * s + 1] = load_quad(rs, o + 16);
            } else {
                const int o = ((16 * g + r16) * LDX + 32 * NK + 4 * h) * 4;
                xr[g][TQ] = load_quad(rs, 4 * h < TAIL ? o : 0x40000000);
            }
        };
        {
            // in the order of the reloads in the rounds below (the waits at
            // the top of a round then count the same loads either way)
            const __amdgpu_buffer_rsrc_t r0 = rsrc32(t0);
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                load_step(r0, 0, s);
                load_step(r0, 1, s);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        __syncthreads();  // LDS set up by the sums waves
        if (sDone != 0) return;
        float* const trow = tiles + e * TS + r16 * XS + 16 * (r16 >> 3);  // group 0's row; group g's: + g * GS
        constexpr int GS = 16 * XS + 32;
        // this lane's centre operands: one base address, the block, step and
        // part as constant offsets (no per-block address registers)
        const __bf16* const cbase = sCP + r16 * CSTR + 8 * h;
        int changed = 0;
        for (int r = 0; r < rounds; ++r) {
            const long t = t0 + (long)r * P;
            const long nrow = n - t * 32 < 32 ? n - t * 32 : 32;
            const bool valid = lane < nrow;
            const __amdgpu_buffer_rsrc_t rl =
                __builtin_amdgcn_make_buffer_rsrc(labels + t * 32, (short)0, (int)(nrow * 4), 0x00020000);
            const int old = __builtin_amdgcn_raw_buffer_load_b32(rl, lane * 4, 0, 0);
            const __amdgpu_buffer_rsrc_t rn = rsrc32(t + P);
            int seen = 0;  // sums-wave progress last read
            v4f acc[2][CB];
#pragma unroll
            for (int g = 0; g < 2; ++g) {
#pragma unroll
                for (int cb = 0; cb < CB; ++cb) acc[g][cb] = v4f{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                // the columns of step s are rewritten below once the sums
                // wave has read them for tile t - P
                if (r > 0) {
                    const int need = (r - 1) * NQ + (s < NK ? min(NQ, 8 * s + 8) : NQ);
                    if (seen < need) seen = wait_flag(&sProg[e], need);
                }
                if (s < NK) {
                    Parts8 xp[2];
#pragma unroll
                    for (int g = 0; g < 2; ++g) {
                        float* dst = trow + g * GS + 32 * s + 8 * h;
                        *reinterpret_cast<float4*>(dst) = xr[g][2 * s];
                        *reinterpret_cast<float4*>(dst + 4) = xr[g][2 * s + 1];
                        xp[g] = split8(xr[g][2 * s], xr[g][2 * s + 1]);
                        load_step(rn, g, s);
                    }
#pragma unroll
                    for (int cb = 0; cb < CB; ++cb) {
                        const __bf16* cp = cbase + 16 * cb * CSTR + 32 * s;
                        const Parts8 cpt{*reinterpret_cast<const v8bf*>(cp),
                                         *reinterpret_cast<const v8bf*>(cp + CPART),
                                         *reinterpret_cast<const v8bf*>(cp + 2 * CPART)};
#pragma unroll
                        for (int g = 0; g < 2; ++g) acc[g][cb] = dot6(cpt, xp[g], acc[g][cb]);
                    }
                } else {
                    Parts4 xp[2];
#pragma unroll
                    for (int g = 0; g < 2; ++g) {
                        // lanes past the row's last feature hold zeros and
                        // store nothing: the LDS row may be shorter than KP
                        if (4 * h < TAIL)
                            *reinterpret_cast<float4*>(trow + g * GS + 32 * NK + 4 * h) = xr[g][TQ];
                        xp[g] = split4(xr[g][TQ]);
                        load_step(rn, g, s);
                    }
#pragma unroll
                    for (int cb = 0; cb < CB; ++cb) {
                        const __bf16* cp = cbase - 4 * h + 16 * cb * CSTR + 32 * NK;  // features 32 NK + 4h ..
                        const Parts4 cpt{*reinterpret_cast<const v4s*>(cp),
                                         *reinterpret_cast<const v4s*>(cp + CPART),
                                         *reinterpret_cast<const v4s*>(cp + 2 * CPART)};
#pragma unroll
                        for (int g = 0; g < 2; ++g) acc[g][cb] = dot6(cpt, xp[g], acc[g][cb]);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            // ||c||^2 - 2 x.c, first minimum wins (_k_means_lloyd.pyx:196-212)
            int mylab = 0;
#pragma unroll
            for (int g = 0; g < 2; ++g) {
                float bd = INFINITY;
                int bi = 4 * h;
#pragma unroll
                for (int cb = 0; cb < CB; ++cb) {
                    const float4 c4 = *reinterpret_cast<const float4*>(&sN[16 * cb + 4 * h]);
                    const float cn[4] = {c4.x, c4.y, c4.z, c4.w};
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        // a NaN distance compares false: it never wins
                        const float dd = fmaf(-2.0f, acc[g][cb][i], cn[i]);
                        const bool take = dd < bd;
                        bd = take ? dd : bd;
                        bi = take ? 16 * cb + 4 * h + i : bi;
                    }
                }
#pragma unroll
                for (int m = 16; m <= 32; m *= 2) {
                    const float od = __shfl_xor(bd, m);
                    const int oi = __shfl_xor(bi, m);
                    const bool take = (od < bd) | ((od == bd) & (oi < bi));  // no branch
                    bd = take ? od : bd;
                    bi = take ? oi : bi;
                }
                if (h == g) mylab = bi;  // lanes 0..31: row = lane
            }
            __builtin_amdgcn_raw_buffer_store_b32(mylab, rl, lane * 4, 0, 0);
            changed += (int)__popcll(__ballot(valid && old != mylab));
            // the tile's rows per cluster for the sums wave (an OR of bits:
            // any order gives the same mask); the counts (integer adds)
            if (valid) atomicOr(&sMask[e][mylab], 1u << lane);
            if (valid) atomicAdd(&sCnt[e & 3][mylab], 1);
            set_flag(&sReady[e], r + 1);
        }
        if (lane == 0 && changed != 0) atomicAdd(a.changed, changed);
        __syncthreads();  // every sums wave is done: the tile area is free
        __syncthreads();  // the sums are in LDS
    } else {
        // the E-step waves wait on the sums wave's progress before rewriting
        // their tile: issue priority for the sums wave
        __builtin_amdgcn_s_setprio(2);
        // sums waves 8..11: the halt test, then the centres' three parts
        // (rows >= k and columns >= ld zero) and ||c||^2
        const int prev = st->done;
        if (prev != 0) {
            if (tid == 512) sDone = prev;
            __syncthreads();
            return;
        }
        const int wt = tid - 512;
        constexpr int CQ = KP / 4;
        constexpr int NF = (CPC * CQ + 255) / 256;
        float4 cf[NF];
#pragma unroll
        for (int u = 0; u < NF; ++u) {
            const int idx = wt + 256 * u;
            const int cl = idx / CQ;
            const int q = idx - cl * CQ;
            cf[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (idx < CPC * CQ && cl < k && 4 * q < LDX)
                cf[u] = *reinterpret_cast<const float4*>(C + (long)cl * ld + 4 * q);
        }
#pragma unroll
        for (int u = 0; u < NF; ++u) {
            const int idx = wt + 256 * u;
            const int cl = idx / CQ;
            const int q = idx - cl * CQ;
            if (idx < CPC * CQ) {
                const Parts4 p = split4(cf[u]);
                __bf16* dst = sCP + cl * CSTR + 4 * q;
                *reinterpret_cast<v4s*>(dst) = p.h;
                *reinterpret_cast<v4s*>(dst + CPART) = p.m;
                *reinterpret_cast<v4s*>(dst + 2 * CPART) = p.l;
            }
        }
        if (wt < 8) {
            sReady[wt] = 0;
            sProg[wt] = 0;
        }
        sCnt[wt >> 6][wt & 63] = 0;
        sMask[wt >> 6][wt & 63] = 0u;
        sMask[4 + (wt >> 6)][wt & 63] = 0u;
        {
            unsigned w[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                w[j] = ((wt >> (2 * j)) & 1 ? 0x3f80u : 0u) | ((wt >> (2 * j + 1)) & 1 ? 0x3f800000u : 0u);
            sOneHot[wt] = __builtin_bit_cast(v8bf, v4u{w[0], w[1], w[2], w[3]});
        }
        if (wave == 8) step_norms<CPC>(a, lane, sN, &sDone);
        __syncthreads();
        if (sDone != 0) return;
        // the sums wave of SIMD m serves E-step waves m and m + 4
        const int m = wave - 8;
        v4f S[CB][NFB];
        msum_tiles3<CB, NQ, XS, NFB>(S, rounds_of(m), rounds_of(m + 4), &sReady[m], &sReady[m + 4], &sProg[m],
                                     &sProg[m + 4], sMask[m], sMask[m + 4], sOneHot, tiles + m * TS,
                                     tiles + (m + 4) * TS, lane);
        __syncthreads();  // every wave is done with its tile
        publish_msums<CB, NFB>(S, tiles, ld, m, lane);
        __syncthreads();
    }
    combine_sums<CPC, 768>(tiles, ld, k, a.psum, a.pcnt, sCnt, tid);
}

// ---------------------------------------------------------------------------
// k_assign3: the E-step for any k (the generic path and the assign entry
// point) on bf16 MFMA over the three-part split, with k_fused3's operand
// layout.  A block of 8 waves owns 256 rows (32 per wave: two 16-row groups);
// it takes the centres in passes of 16*CB (A operands from LDS, the three
// parts staged per SEG-feature segment by the whole block) and keeps per lane
// the first minimum over its centres 16cb + 4(l/16) + i, in ascending order
// across passes; the four lanes of a row are combined after the last pass.
// X is read once per pass (k/(16 CB) times), the centres once per 256 rows.
template <int CB>
struct Assign3Geom {
    static constexpr int CPC = 16 * CB;               // centres per pass
    static constexpr int SEG = CB >= 16 ? 64 : 128;   // features per staged segment
    static constexpr int NKS = SEG / 32;              // K32 steps per segment
    static constexpr int CSTR = SEG + 8;              // bf16 per centre row: an odd number of 16-byte units
    static constexpr int CPART = CPC * CSTR;          // bf16 from one part to the next
    static constexpr size_t LDS = size_t(3) * CPART * sizeof(__bf16);
};

template <int CB>
__global__ __launch_bounds__(512, 1) void k_assign3(const float* __restrict__ X, long n, int ld,
                                                   const float* __restrict__ C, const float* __restrict__ cnorm,
                                                   int k, int* __restrict__ labels, LoopState* st, int* changed)
{
    if (st != nullptr && st->done != 0) return;
    using G = Assign3Geom<CB>;
    constexpr int CPC = G::CPC, SEG = G::SEG, NKS = G::NKS, CSTR = G::CSTR, CPART = G::CPART;
    extern __shared__ __attribute__((aligned(16))) __bf16 cs[];  // [3][CPC][CSTR]
    __shared__ __attribute__((aligned(16))) float sN[CPC];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 4, r16 = lane & 15;
    const int npass = (k + CPC - 1) / CPC;
    const int nseg = (ld + SEG - 1) / SEG;
    const __bf16* const cbase = cs + r16 * CSTR + 8 * h;
    // one pass of one segment (k <= 16 CB, ld <= SEG): the staged operands
    // are the same for every row block, so they are staged once
    const bool once = npass == 1 && nseg == 1;

    for (long base = (long)blockIdx.x * 256; base < n; base += (long)gridDim.x * 256) {
        const long wrow = base + 32 * wave;  // this wave's first row
        const long nrow = n - wrow < 32 ? (n - wrow > 0 ? n - wrow : 0) : 32;
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(X + (nrow > 0 ? wrow * ld : 0)), (short)0, (int)(nrow * ld * 4), 0x00020000);
        float bd[2] = {INFINITY, INFINITY};
        int bi[2] = {0, 0};
        for (int p = 0; p < npass; ++p) {
            v4f acc[2][CB];
#pragma unroll
            for (int g = 0; g < 2; ++g) {
#pragma unroll
                for (int cb = 0; cb < CB; ++cb) acc[g][cb] = v4f{0.f, 0.f, 0.f, 0.f};
            }
            for (int sg = 0; sg < nseg; ++sg) {
                const int f0 = sg * SEG;
                if (!once || base == (long)blockIdx.x * 256) {  // (uniform across the block)
                __syncthreads();  // the previous segment's operands are consumed
                // stage centres p*CPC.. x the features f0.. of the K steps this
                // segment has (32 each; centres >= k and features >= ld zero),
                // as the three bf16 parts: eight threads per (centre, K step),
                // two K steps' loads in flight before the first split
                constexpr int UPK = CPC * 8 / 512;  // float4s per thread per K step
                const int nks_s = min(NKS, (ld - f0 + 31) / 32);
                for (int ks0 = 0; ks0 < nks_s; ks0 += 2) {
                    float4 v[2][UPK];
#pragma unroll
                    for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
                        for (int u = 0; u < UPK; ++u) {
                            const int idx = tid + 512 * u;
                            const int j = p * CPC + (idx >> 3);
                            const int f = f0 + 4 * (8 * (ks0 + kk) + (idx & 7));
                            v[kk][u] = make_float4(0.f, 0.f, 0.f, 0.f);
                            if (ks0 + kk < nks_s && j < k && f < ld)
                                v[kk][u] = *reinterpret_cast<const float4*>(C + (long)j * ld + f);
                        }
                    }
#pragma unroll
                    for (int kk = 0; kk < 2; ++kk) {
                        if (ks0 + kk >= nks_s) break;
#pragma unroll
                        for (int u = 0; u < UPK; ++u) {
                            const int idx = tid + 512 * u;
                            const int cl = idx >> 3;
                            const int q = 8 * (ks0 + kk) + (idx & 7);
                            const Parts4 pt = split4(v[kk][u]);
                            __bf16* dst = cs + cl * CSTR + 4 * q;
                            *reinterpret_cast<v4s*>(dst) = pt.h;
                            *reinterpret_cast<v4s*>(dst + CPART) = pt.m;
                            *reinterpret_cast<v4s*>(dst + 2 * CPART) = pt.l;
                        }
                    }
                }
                if (sg == 0) {
                    for (int i = tid; i < CPC; i += 512) {
                        const int j = p * CPC + i;
                        sN[i] = j < k ? cnorm[j] : INFINITY;  // padding centres never win
                    }
                }
                __syncthreads();
                }
                const int nks = min(NKS, (ld - f0 + 31) / 32);
                for (int ks = 0; ks < nks; ++ks) {
                    // rows 16g + l%16, features f0 + 32ks + 8h..: past the
                    // row's end the next row's (finite) values meet zero
                    // centre parts; past the last row the loads return 0
                    Parts8 xp[2];
#pragma unroll
                    for (int g = 0; g < 2; ++g) {
                        const int o = ((16 * g + r16) * ld + f0 + 32 * ks + 8 * h) * 4;
                        xp[g] = split8(load_quad(rs, o), load_quad(rs, o + 16));
                    }
#pragma unroll
                    for (int cb = 0; cb < CB; ++cb) {
                        const __bf16* cp = cbase + 16 * cb * CSTR + 32 * ks;
                        const Parts8 cpt{*reinterpret_cast<const v8bf*>(cp),
                                         *reinterpret_cast<const v8bf*>(cp + CPART),
                                         *reinterpret_cast<const v8bf*>(cp + 2 * CPART)};
#pragma unroll
                        for (int g = 0; g < 2; ++g) acc[g][cb] = dot6(cpt, xp[g], acc[g][cb]);
                    }
                }
            }
            // ||c||^2 - 2 x.c, first minimum wins (_k_means_lloyd.pyx:196-212);
            // the lane's centres come in ascending order, passes too
#pragma unroll
            for (int g = 0; g < 2; ++g) {
#pragma unroll
                for (int cb = 0; cb < CB; ++cb) {
                    const float4 c4 = *reinterpret_cast<const float4*>(&sN[16 * cb + 4 * h]);
                    const float cn[4] = {c4.x, c4.y, c4.z, c4.w};
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float dd = fmaf(-2.0f, acc[g][cb][i], cn[i]);  // NaN compares false
                        const bool take = dd < bd[g];
                        bd[g] = take ? dd : bd[g];
                        bi[g] = take ? p * CPC + 16 * cb + 4 * h + i : bi[g];
                    }
                }
            }
        }
        int mylab = 0;
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            float d0 = bd[g];
            int i0 = bi[g];
#pragma unroll
            for (int m = 16; m <= 32; m *= 2) {
                const float od = __shfl_xor(d0, m);
                const int oi = __shfl_xor(i0, m);
                const bool take = (od < d0) | ((od == d0) & (oi < i0));
                d0 = take ? od : d0;
                i0 = take ? oi : i0;
            }
            if (h == g) mylab = i0;  // lanes 0..31: row = lane
        }
        const bool valid = lane < nrow;
        const long row = wrow + lane;
        int moved = 0;
        if (valid) {
            if (changed != nullptr) moved = labels[row] != mylab;
            labels[row] = mylab;
        }
        if (changed != nullptr) {
            const unsigned long long mm = __ballot(moved);
            if (lane == 0 && mm != 0ull) atomicAdd(changed, (int)__popcll(mm));
        }
    }
}

typedef void (*assign3_fn)(const float*, long, int, const float*, const float*, int, int*, LoopState*, int*);

static int assign3_cb(int k) { return k <= 64 ? 4 : k <= 128 ? 8 : 16; }

static assign3_fn assign3_kernel(int k)
{
    const int cb = assign3_cb(k);
    return cb == 4 ? &k_assign3<4> : cb == 8 ? &k_assign3<8> : &k_assign3<16>;
}

static size_t assign3_lds(int k)
{
    const int cb = assign3_cb(k);
    return cb == 4 ? Assign3Geom<4>::LDS : cb == 8 ? Assign3Geom<8>::LDS : Assign3Geom<16>::LDS;
}

// SKMETAL_HIP_SPLIT=0 keeps the fp32 MFMA E-step for every shape
static bool split_disabled()
{
    const char* env = getenv("SKMETAL_HIP_SPLIT");
    return env != nullptr && env[0] == '0';
}

int assign3_ready(int d, int k)
{
    if (split_disabled() || d < 17 || k < 1) return 0;
    for (const int kk : {64, 128, 129}) {
        assign3_fn f = assign3_kernel(kk);
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(f), hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)assign3_lds(kk)) != hipSuccess) {
            (void)hipGetLastError();
            return 0;
        }
    }
    return 1;
}

hipError_t launch_assign3(const AssignArgs& a, int num_cu, hipStream_t s)
{
    if (a.n <= 0) return hipSuccess;
    long blocks = (a.n + 255) / 256;
    if (blocks > num_cu) blocks = num_cu;
    hipLaunchKernelGGL(assign3_kernel(a.k), dim3((unsigned)blocks), dim3(512), assign3_lds(a.k), s, a.X, a.n, a.ld,
                       a.C, a.cnorm, a.k, a.labels, a.state, a.changed);
    return hipGetLastError();
}

typedef void (*fused_fn)(FusedArgs);

template <int NQ, int... KGs>
struct FusedTable {
    static fused_fn get(int kg)
    {
        fused_fn f = nullptr;
        ((kg == KGs ? (f = &k_fused<KGs, NQ>, 0) : 0), ...);
        return f;
    }
};

template <int NQ>
static fused_fn pick_fused(int kg)
{
    return FusedTable<NQ, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16>::get(kg);
}

// Compiled row sizes (float4s); ld = 4 * NQ.
static fused_fn fused_kernel(int k, int ld)
{
    if (k < 1 || k > 64) return nullptr;
    const int kg = (k + 3) / 4;
    switch (ld) {
    case 4: return pick_fused<1>(kg);
    case 8: return pick_fused<2>(kg);
    case 16: return pick_fused<4>(kg);
    case 32: return pick_fused<8>(kg);
    case 48: return pick_fused<12>(kg);
    case 64: return pick_fused<16>(kg);
    case 80: return pick_fused<20>(kg);
    case 100: return pick_fused<25>(kg);
    default: return nullptr;
    }
}

template <int NQ, int... CBs>
struct Fused3Table {
    static fused_fn get(int cb)
    {
        fused_fn f = nullptr;
        ((cb == CBs ? (f = &k_fused3<CBs, NQ>, 0) : 0), ...);
        return f;
    }
    static size_t dyn_lds(int cb)
    {
        using G = Fused3Geom<NQ>;
        return (size_t)8 * G::TS * sizeof(float) + (size_t)3 * 16 * cb * G::CSTR * sizeof(__bf16);
    }
};

// The split kernel for row strides of 32 floats and more (below that the K
// steps would be mostly padding).
static fused_fn fused3_kernel(int k, int ld, size_t* dyn)
{
    if (k < 1 || k > 64) return nullptr;
    const int cb = (k + 15) / 16;
    switch (ld) {
    case 32: *dyn = Fused3Table<8, 1, 2, 3, 4>::dyn_lds(cb); return Fused3Table<8, 1, 2, 3, 4>::get(cb);
    case 48: *dyn = Fused3Table<12, 1, 2, 3, 4>::dyn_lds(cb); return Fused3Table<12, 1, 2, 3, 4>::get(cb);
    case 64: *dyn = Fused3Table<16, 1, 2, 3, 4>::dyn_lds(cb); return Fused3Table<16, 1, 2, 3, 4>::get(cb);
    case 80: *dyn = Fused3Table<20, 1, 2, 3, 4>::dyn_lds(cb); return Fused3Table<20, 1, 2, 3, 4>::get(cb);
    case 100: *dyn = Fused3Table<25, 1, 2, 3, 4>::dyn_lds(cb); return Fused3Table<25, 1, 2, 3, 4>::get(cb);
    default: return nullptr;
    }
}

int fused3_ready(int k, int ld)
{
    if (split_disabled()) return 0;
    size_t dyn = 0;
    fused_fn f = fused3_kernel(k, ld, &dyn);
    // sMask, sOneHot, sCnt, sN, flags
    const size_t stat = 8 * 64 * sizeof(unsigned) + 256 * 16 + 4 * 64 * sizeof(int) + 64 * sizeof(float) + 128;
    if (f == nullptr || dyn + stat > 160 * 1024) return 0;
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(f), hipFuncAttributeMaxDynamicSharedMemorySize, (int)dyn) !=
        hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return 1;
}

static size_t fused_dyn_lds(int k, int ld)
{
    const int cpc = 4 * ((k + 3) / 4);
    return (size_t)(cpc + 1 + 4 * 64) * fused_stride(ld / 4) * sizeof(float);
}

int fused_ld(int d, int k)
{
    // SKMETAL_HIP_FUSED=0 selects the separate assign/update kernels for every shape
    const char* env = getenv("SKMETAL_HIP_FUSED");
    if (env != nullptr && env[0] == '0') return 0;
    if (d < 1 || k < 1 || k > 64) return 0;
    static const int kLds[] = {4, 8, 16, 32, 48, 64, 80, 100};
    for (int ld : kLds) {
        if (ld < d) continue;
        fused_fn f = fused_kernel(k, ld);
        const size_t dyn = fused_dyn_lds(k, ld);
        const size_t stat = 4 * 64 * (sizeof(unsigned long long) + sizeof(int)) + 64 * sizeof(float);  // sMask, sCnt, sN
        if (f == nullptr || dyn + stat > 160 * 1024) return 0;
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(f), hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)dyn) != hipSuccess) {
            (void)hipGetLastError();
            return 0;
        }
        return ld;
    }
    return 0;
}

int fused_blocks(long n, int ld, int k, int num_cu)
{
    if (fused_kernel(k, ld) == nullptr) return 0;
    const long tiles = (n + 63) / 64;
    long blocks = (tiles + 3) / 4;
    if (blocks > num_cu) blocks = num_cu;
    return (int)(blocks < 1 ? 1 : blocks);
}

hipError_t launch_fused(const FusedArgs& a, hipStream_t s)
{
    size_t dyn = 0;
    fused_fn f = a.split ? fused3_kernel(a.k, a.ld, &dyn) : fused_kernel(a.k, a.ld);
    if (!a.split) dyn = fused_dyn_lds(a.k, a.ld);
    if (f == nullptr || a.blocks < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(f, dim3(a.blocks), dim3(a.split ? 768 : 512), dyn, s, a);
    return hipGetLastError();
}

}  // namespace skm
