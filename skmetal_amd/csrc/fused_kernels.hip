// fused_kernels.hip -- one-pass Lloyd step for small k*d on gfx950 (MI355X):
// the E-step (sklearn/cluster/_k_means_lloyd.pyx:196-212) and the
// per-cluster sums and counts of the M-step (:214-218) in one kernel that
// reads X from HBM once per step.
//
//   k_fused     E-step on fp32 MFMA, per-cluster sums by a VALU walker; 8
//               waves per block (d <= 16, data outside the split's range of
//               split_kernels.hip's k_fused3, or the fp32 switch).
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

#include "fused_common.h"

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
// Buffer descriptor over the rows of tile t (none past the last row: loads
// there return 0 without a memory access).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const float* X, long t, long n, int ld)
{
    const long r0 = t * 64;
    const long rows = n - r0 < 64 ? (n - r0 > 0 ? n - r0 : 0) : 64;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(X + (rows > 0 ? r0 * ld : 0)), (short)0,
                                             (int)(rows * ld * 4), 0x00020000);
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
    __shared__ int sChg;       // labels the block's MFMA waves changed
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
        // one global atomic per block (below), not one per wave
        if (lane == 0 && changed != 0) atomicAdd(&sChg, changed);
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
        if (wt == 0) sChg = 0;
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
    if (tid == 0 && sChg != 0) atomicAdd(a.changed, sChg);
    combine_sums<CPC>(zrow + XS, ld, k, psum, pcnt, sCnt, tid, &st->present[a.iter & 1]);
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
    if (a.split) return launch_fused3(a, s);
    fused_fn f = fused_kernel(a.k, a.ld);
    if (f == nullptr || a.blocks < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(f, dim3(a.blocks), dim3(512), fused_dyn_lds(a.k, a.ld), s, a);
    return hipGetLastError();
}
}  // namespace skm
