// split_kernels.hip -- the Lloyd step's E-step and per-cluster sums on bf16
// MFMAs (gfx950) over an exact three-part bf16 split of x and c, with fp32
// accumulation: the E-step of sklearn/cluster/_k_means_lloyd.pyx:196-212 and
// the sums and counts of :214-218.
//
//   k_fused3    E-step + per-cluster sums in one pass over X (k <= 64,
//               17 <= d <= 100); 12 waves per block.
//   k_assign3   E-step alone for any k (the generic path, the final E-step
//               and the assign entry point).
//
// Built without -amdgpu-mfma-vgpr-form (the register allocator places the
// MFMA accumulators).
#include <stdlib.h>

#include "fused_common.h"

namespace skm {

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

hipError_t launch_fused3(const FusedArgs& a, hipStream_t s)
{
    size_t dyn = 0;
    fused_fn f = fused3_kernel(a.k, a.ld, &dyn);
    if (f == nullptr || a.blocks < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(f, dim3(a.blocks), dim3(768), dyn, s, a);
    return hipGetLastError();
}

}  // namespace skm
