// split_kernels.hip -- the Lloyd step's E-step and per-cluster sums on bf16
// MFMAs (gfx950) over an exact three-part bf16 split of x and c, with fp32
// accumulation: the E-step of sklearn/cluster/_k_means_lloyd.pyx:196-212 and
// the sums and counts of :214-218.
//
//   k_fused3    E-step + per-cluster sums in one pass over X (k <= 64,
//               17 <= d <= 100); 16 waves per block.
//   k_assign3   E-step alone for any k (the generic path, the final E-step
//               and the assign entry point), its centres staged from the
//               per-step image that k_centre_image writes.
//
// Built without -amdgpu-mfma-vgpr-form (the register allocator places the
// MFMA accumulators).
#include <stdlib.h>

#include <type_traits>

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
// MFMAs over the three-part split (v_mfma_f32_16x16x32_bf16).
//
// MFMA operand layout (16x16x32, checked on the device): lane l holds A[m =
// l%16][kk = 8(l/16) + j] and B[kk = 8(l/16) + j][n = l%16], j < 8, and
// receives D[m = 4(l/16) + i][n = l%16], i < 4.
//
// A block is 16 waves, four per SIMD: E-step waves m and m + 4 and sums waves
// 8 + m and 12 + m on SIMD m share the 32-row tiles t = 4b + m + r P (P = 4 x
// blocks), E-step wave m taking rows 0..15 of each and wave m + 4 rows
// 16..31.  An E-step wave loads its 16 rows straight from HBM into registers
// (one tile ahead), splits each value once, takes the E-step's MFMAs with the
// parts as B (its 16 rows as the columns n) against 16-centre blocks of the
// centre parts as A, and writes the parts to the SIMD's LDS tile, row-major.
// Lane l then holds x.c of row l%16 and centres 16cb + 4(l/16) + i: the first
// minimum over the lane's centres, then over the four lanes l%16 + 16h (lower
// index wins ties: the first minimum over all centres); lane r < 16 keeps row
// r's label.
//
// The centre operands sit in LDS in fragment order -- 1 KB per MFMA operand,
// lane l's 16 bytes at 16 l -- so every A read is one contiguous block.
//
// The sums waves read the 32-row tile back transposed (ds_read_b64_tr_b16
// returns the B operand with K = the tile's rows) and add onehot^T x once per
// part, wave 8 + m over the first half of the 16-feature blocks and 12 + m
// over the rest.  The waves hand over through LDS flags: ready (half tiles
// labelled, their row masks set) and progress (blocks of a tile read, per
// sums wave); there is no block barrier until the end.
//
// Features past the last 32-feature K step (a tail of TAIL = 4 or 16): the
// six products of the E-step are laid side by side along K, block b (TAIL
// values) pairing centre part PC[b] with x part PX[b] for (PC, PX) = (h, h),
// (m, h), (l, h), (h, m), (m, m), (h, l).  One MFMA (TAIL = 4) or three (TAIL
// = 16) take the six products in place of six each.
//
// When the last 16-centre block holds at most 4 real centres (STK), its A
// rows m = 4 slot + p carry part p of centre 16(CB-1) + slot (p = 3: zero)
// and the B operands are the three x parts in turn: three MFMAs per K step
// give all nine part products, and lane l's D[0..2] are the parts of the dot
// product with centre 16(CB-1) + l/16.

// Geometry of k_fused3 for a row of NQ float4s.
template <int NQ>
struct Fused3Geom {
    static constexpr int LDX = 4 * NQ;                        // == ld
    static constexpr int NK = LDX / 32;                       // 32-feature K steps
    static constexpr int TAIL = LDX - 32 * NK;                // features after them: 0, 4 or 16
    static constexpr int KP = 32 * NK + (TAIL > 0 ? 16 : 0);  // features per part in a tile row
    static constexpr int NFB = KP / 16;                       // 16-feature blocks of the sums
    static constexpr int QG = 2 * NK + TAIL / 8 + (TAIL == 4 ? 1 : 0);  // float4s per lane
    static constexpr int NT = TAIL == 4 ? 1 : TAIL == 16 ? 3 : 0;      // tail MFMAs per block
    static constexpr int NTS = TAIL == 4 ? 1 : TAIL == 16 ? 2 : 0;     // tail MFMAs of a stacked block
    // a tile row is hi | mid | lo, KP bf16 each: 6 KP bytes (a multiple of 32),
    // padded to an odd number of 16-byte units: the E-step waves' 16-byte
    // stores of 16 rows at one column then fall in distinct banks (a stride of
    // 32 mod 128 bytes costs 8 conflict cycles per store), and the transposed
    // reads cost the same as at any other stride
    static constexpr int RSB = 6 * KP + 16;
    static constexpr int TILEB = 32 * RSB;
    // centre fragments (1 KB each): [cb][s][part], then [cb][tail MFMA], then
    // the stacked block's [s] and [tail MFMA]
    static constexpr int frags(int cb) { return cb * (3 * NK + NT) + NK + NTS; }
    static constexpr size_t lds(int cb)
    {
        const size_t work = (size_t)4 * TILEB + (size_t)1024 * frags(cb);
        const size_t red = (size_t)4 * 16 * cb * LDX * sizeof(float);  // the sums of the four sums waves
        return work > red ? work : red;
    }
    static_assert(TAIL == 0 || TAIL == 4 || TAIL == 16, "tails of 4 or 16 features");
    static_assert(RSB % 32 == 16 && (2 * KP) % 16 == 0, "rows of an odd number of 16-byte units, aligned parts");
};

__device__ __forceinline__ v4s lds_tr16(const char* p)
{
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(p));
}

__device__ __forceinline__ v8bf cat8(v4s a, v4s b)
{
    return __builtin_bit_cast(v8bf, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
}

// part p (0 hi, 1 mid, 2 lo) of a split
__device__ __forceinline__ v8bf part_of(const Parts8& x, int p) { return p == 0 ? x.h : p == 1 ? x.m : x.l; }
__device__ __forceinline__ v4s part_of(const Parts4& x, int p) { return p == 0 ? x.h : p == 1 ? x.m : x.l; }

// centre part (0 hi, 1 mid, 2 lo) of tail block b: (h, m, l, h, m, h)
__device__ __forceinline__ int tail_cpart(int b) { return b == 1 || b == 4 ? 1 : b == 2 ? 2 : 0; }

// (a & ma) | (b & mb) per 32-bit word: a lane-dependent choice between
// operands, or zero, without a branch (ma, mb are all-ones or zero).
__device__ __forceinline__ v4s pick2(v4s a, unsigned ma, v4s b, unsigned mb)
{
    const v2u ua = __builtin_bit_cast(v2u, a), ub = __builtin_bit_cast(v2u, b);
    return __builtin_bit_cast(v4s, (ua & ma) | (ub & mb));
}
__device__ __forceinline__ v8bf pick2(v8bf a, unsigned ma, v8bf b, unsigned mb)
{
    const v4u ua = __builtin_bit_cast(v4u, a), ub = __builtin_bit_cast(v4u, b);
    return __builtin_bit_cast(v8bf, (ua & ma) | (ub & mb));
}

// The first minimum of (d, i) over lanes l and l ^ 16 (X = 16) or l ^ 32 (X =
// 32), lower index first on ties, in both lanes.  v_permlane16_swap_b32 /
// v_permlane32_swap_b32 of a register with itself leave lane l's value in one
// result and lane l ^ X's in the other (which is which depends on the lane);
// the lexicographic minimum of the two pairs is the same either way.  Plain
// VALU: no LDS round trip.
template <int X>
__device__ __forceinline__ void argmin_swap(float& d, int& i)
{
    const unsigned du = __float_as_uint(d), iu = (unsigned)i;
    v2u pd, pi;
    if constexpr (X == 16) {
        pd = __builtin_amdgcn_permlane16_swap(du, du, false, false);
        pi = __builtin_amdgcn_permlane16_swap(iu, iu, false, false);
    } else {
        pd = __builtin_amdgcn_permlane32_swap(du, du, false, false);
        pi = __builtin_amdgcn_permlane32_swap(iu, iu, false, false);
    }
    const float d0 = __uint_as_float(pd[0]), d1 = __uint_as_float(pd[1]);
    const int i0 = (int)pi[0], i1 = (int)pi[1];
    const bool take1 = (d1 < d0) | ((d1 == d0) & (i1 < i0));  // no branch
    d = take1 ? d1 : d0;
    i = take1 ? i1 : i0;
}

template <int CB, int NQ, bool STK>
__global__ __launch_bounds__(1024, 1) void k_fused3(FusedArgs a)
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
    constexpr int LDX = G::LDX, NK = G::NK, TAIL = G::TAIL, KP = G::KP, NFB = G::NFB, QG = G::QG, NT = G::NT;
    constexpr int RSB = G::RSB, TILEB = G::TILEB;
    constexpr int CBF = STK ? CB - 1 : CB;  // blocks taken as 16 centres
    constexpr int NFA = (NFB + 1) / 2;      // feature blocks of the first sums wave of a SIMD
    constexpr int NFZ = NFB - NFA;          // and of the second
    // fragment indices (units of 64 v8bf)
    constexpr int FT = CB * 3 * NK;         // tail fragments
    constexpr int FS = CB * (3 * NK + NT);  // stacked block: K steps, then its tail
    // LDS: 4 SIMD tiles [32 x RSB bytes] | centre fragments [frags x 1 KB]
    extern __shared__ __attribute__((aligned(16))) float lds[];
    // rows of each cluster in E-step wave e's half of a tile (bit = row), by
    // round parity
    __shared__ unsigned sMask[2][8][64];
    __shared__ __attribute__((aligned(16))) v8bf sOneHot[256];  // byte b -> its 8 bits as bf16 0 / 1
    __shared__ int sCnt[4][64];                                 // rows per cluster, per SIMD (its first sums wave)
    __shared__ __attribute__((aligned(16))) float sN[CPC];
    __shared__ int sReady[8];  // half tiles E-step wave e has labelled
    __shared__ int sProg[8];   // feature blocks sums wave w has read: tile * (its blocks) + blocks
    __shared__ int sDone;      // nonzero: the loop has halted, nothing to do
    __shared__ int sChg;       // labels the block's E-step waves changed
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 4;    // this lane's K slice / centre quad in the MFMA layout
    const int r16 = lane & 15;  // this lane's row / centre of a block

    char* const tiles = reinterpret_cast<char*>(lds);
    v8bf* const sFr = reinterpret_cast<v8bf*>(tiles + 4 * TILEB);

    // 32-row tiles: SIMD slot t0 = 4b + m (of P = 4 x blocks) takes tile t0
    // + r P in each of the Rf rounds in which every slot has a whole tile;
    // the rem rows after them go out in 16-row halves, half h to slot h % P
    // as its half h / P, so that the last round is at most one half tile for
    // every slot when rem <= 16 P (500,000 rows on 1,024 slots: 530 halves
    // instead of 265 whole tiles, and the last round costs one E-step wave
    // instead of two)
    const long P = (long)gridDim.x * 4;
    const long Rf = n / (32 * P);
    const long rem = n - Rf * P * 32;
    auto rounds_of = [&](int m) {
        const long t0 = (long)blockIdx.x * 4 + m;
        return (int)Rf + (16 * t0 < rem ? 1 : 0);
    };

    if (wave < 8) {
        // E-step wave e: SIMD m = e & 3, rows 16 hf .. 16 hf + 15 of the
        // tiles.  xr holds this lane's features of row l%16: K32 step s in
        // xr[2s], xr[2s + 1] (features 32s + 8h + 0..7); the tail in xr[2NK]
        // (TAIL = 4: features 32NK + 0..3 in every h) or xr[2NK], xr[2NK + 1]
        // (TAIL = 16: features 32NK + 8(h&1) + 0..7)
        const int e = wave, m = wave & 3, hf = wave >> 2;
        const long t0 = (long)blockIdx.x * 4 + m;
        const int rounds = rounds_of(m);
        float4 xr[QG];
        // the first row of this wave's half in round r
        auto rowbase = [&](int r) -> long {
            return r < Rf ? (t0 + (long)r * P) * 32 + 16 * hf : Rf * P * 32 + 16 * (t0 + (long)hf * P);
        };
        auto rows_at = [&](long r0) { return n - r0 < 16 ? (n - r0 > 0 ? n - r0 : 0) : 16; };
        auto rsrc16 = [&](int r) {
            const long r0 = rowbase(r);
            const long rows = r < rounds ? rows_at(r0) : 0;
            return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(X + (rows > 0 ? r0 * ld : 0)), (short)0,
                                                     (int)(rows * ld * 4), 0x00020000);
        };
        auto load_step = [&](__amdgpu_buffer_rsrc_t rs, int s) {
            const int row = r16 * LDX;
            if (s < NK) {
                const int o = (row + 32 * s + 8 * h) * 4;
                xr[2 * s] = load_quad(rs, o);
                xr[2 * s + 1] = load_quad(rs, o + 16);
            } else if constexpr (TAIL == 4) {
                xr[2 * NK] = load_quad(rs, (row + 32 * NK) * 4);
            } else if constexpr (TAIL == 16) {
                const int o = (row + 32 * NK + 8 * (h & 1)) * 4;
                xr[2 * NK] = load_quad(rs, o);
                xr[QG - 1] = load_quad(rs, o + 16);
            }
        };
        constexpr int NS = NK + (TAIL > 0 ? 1 : 0);
        {
            // in the order of the reloads in the rounds below (the waits at
            // the top of a step then count the same loads either way)
            const __amdgpu_buffer_rsrc_t r0 = rsrc16(0);
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                load_step(r0, s);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        __syncthreads();  // LDS set up by the sums waves
        if (sDone != 0) return;
        char* const trow = tiles + m * TILEB + (16 * hf + r16) * RSB;  // this lane's row of the tile
        const v8bf* const fr = sFr + lane;                            // this lane's 16 bytes of fragment f: fr[64 f]
        // before feature blocks f0 .. f1 of the tile are rewritten for round r,
        // the sums waves have read them for round r - 1
        auto wait_blocks = [&](int r, int f0, int f1) {
            if (r == 0) return;
            if (f0 < NFA) wait_flag(&sProg[m], (r - 1) * NFA + (f1 + 1 < NFA ? f1 + 1 : NFA));
            if (f1 >= NFA) wait_flag(&sProg[4 + m], (r - 1) * NFZ + (f1 + 1 - NFA));
        };
        // lane masks of the tail's operands (all ones when the lane's h matches)
        const unsigned mh0 = h == 0 ? ~0u : 0u, mh1 = h == 1 ? ~0u : 0u, mh2 = h == 2 ? ~0u : 0u;
        const unsigned mlt2 = h < 2 ? ~0u : 0u, mge2 = ~mlt2;
        int changed = 0;
        // only the last round's half can lie past the rows: this wave then
        // skips it (below) instead of computing on zeros
        const int rounds_e = rounds > 0 && rows_at(rowbase(rounds - 1)) <= 0 ? rounds - 1 : rounds;
        for (int r = 0; r < rounds_e; ++r) {
            const long rb = rowbase(r);
            const long nrow = rows_at(rb);
            const bool valid = lane < nrow;
            const __amdgpu_buffer_rsrc_t rl = __builtin_amdgcn_make_buffer_rsrc(
                labels + rb, (short)0, (int)(nrow > 0 ? nrow * 4 : 0), 0x00020000);
            const int old = __builtin_amdgcn_raw_buffer_load_b32(rl, lane * 4, 0, 0);
            const __amdgpu_buffer_rsrc_t rn = rsrc16(r + 1);
            v4f acc[CB];
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) acc[cb] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < NK; ++s) {
                // the step's centre fragments first: their LDS latency runs
                // under the split
                Parts8 cpt[CBF > 0 ? CBF : 1];
#pragma unroll
                for (int cb = 0; cb < CBF; ++cb) {
                    const int f = (cb * NK + s) * 3;
                    cpt[cb] = Parts8{fr[64 * f], fr[64 * (f + 1)], fr[64 * (f + 2)]};
                }
                v8bf cs;
                if constexpr (STK) cs = fr[64 * (FS + s)];
                const Parts8 xp = split8(xr[2 * s], xr[2 * s + 1]);
                wait_blocks(r, 2 * s, 2 * s + 1);
                {
                    char* dst = trow + (32 * s + 8 * h) * 2;
                    *reinterpret_cast<v8bf*>(dst) = xp.h;
                    *reinterpret_cast<v8bf*>(dst + 2 * KP) = xp.m;
                    *reinterpret_cast<v8bf*>(dst + 4 * KP) = xp.l;
                }
                load_step(rn, s);
                // product-major: consecutive MFMAs write different accumulators
#pragma unroll
                for (int pr = 0; pr < 6; ++pr) {
#pragma unroll
                    for (int cb = 0; cb < CBF; ++cb) {
                        const Parts8& c = cpt[cb];
                        const v8bf ca = pr == 0 ? c.m : pr == 1 ? c.l : pr == 2 ? c.h : pr == 3 ? c.m : c.h;
                        const v8bf xb = pr == 0 ? xp.m : pr == 1 ? xp.h : pr == 2 ? xp.l : pr == 3 ? xp.h
                                                                                                 : pr == 4 ? xp.m : xp.h;
                        acc[cb] = mfma_bf16(ca, xb, acc[cb]);
                    }
                    if constexpr (STK) {
                        if (pr < 3) acc[CB - 1] = mfma_bf16(cs, pr == 0 ? xp.l : pr == 1 ? xp.m : xp.h, acc[CB - 1]);
                    }
                }
            }
            if constexpr (TAIL > 0) {
                const v4s z4 = v4s{0, 0, 0, 0};
                if constexpr (TAIL == 4) {
                    const Parts4 xt = split4(xr[2 * NK]);
                    wait_blocks(r, NFB - 1, NFB - 1);
                    {
                        // every lane holds the same four features: lane h
                        // writes them at features 32NK + 4h of the tail block,
                        // whose features past 32NK + 3 are padding the sums
                        // never read (no branch)
                        char* dst = trow + (32 * NK + 4 * h) * 2;
                        *reinterpret_cast<v4s*>(dst) = xt.h;
                        *reinterpret_cast<v4s*>(dst + 2 * KP) = xt.m;
                        *reinterpret_cast<v4s*>(dst + 4 * KP) = xt.l;
                    }
                    load_step(rn, NK);
                    // blocks 2h, 2h + 1 of (x_h, x_h, x_h, x_m, x_m, x_l, 0, 0)
                    const v8bf bt = cat8(pick2(xt.h, mlt2, xt.m, mh2),
                                         pick2(pick2(xt.h, mh0, xt.m, mh1), ~0u, xt.l, mh2));
#pragma unroll
                    for (int cb = 0; cb < CBF; ++cb) acc[cb] = mfma_bf16(fr[64 * (FT + cb)], bt, acc[cb]);
                    if constexpr (STK) {
                        // blocks 2h, 2h + 1 of (x_h, x_m, x_l, 0, ...)
                        const v8bf bs = cat8(pick2(xt.h, mh0, xt.l, mh1), pick2(xt.m, mh0, z4, 0u));
                        acc[CB - 1] = mfma_bf16(fr[64 * (FS + NK)], bs, acc[CB - 1]);
                    }
                } else {
                    const Parts8 xt = split8(xr[2 * NK], xr[QG - 1]);
                    wait_blocks(r, NFB - 1, NFB - 1);
                    {
                        // lanes h and h + 2 hold the same eight features
                        // 32NK + 8(h&1): both write them (the same values)
                        char* dst = trow + (32 * NK + 8 * (h & 1)) * 2;
                        *reinterpret_cast<v8bf*>(dst) = xt.h;
                        *reinterpret_cast<v8bf*>(dst + 2 * KP) = xt.m;
                        *reinterpret_cast<v8bf*>(dst + 4 * KP) = xt.l;
                    }
                    load_step(rn, NK);
                    // MFMA q, lane h: block 2q + h/2 of (x_h, x_h, x_h, x_m, x_m, x_l)
                    const v8bf b1 = pick2(xt.h, mlt2, xt.m, mge2), b2 = pick2(xt.m, mlt2, xt.l, mge2);
#pragma unroll
                    for (int q = 0; q < 3; ++q) {
#pragma unroll
                        for (int cb = 0; cb < CBF; ++cb)
                            acc[cb] = mfma_bf16(fr[64 * (FT + cb * NT + q)], q == 0 ? xt.h : q == 1 ? b1 : b2, acc[cb]);
                    }
                    if constexpr (STK) {
                        // blocks of (x_h, x_m, x_l, 0): lanes h < 2 take the
                        // first of each MFMA's two, h >= 2 the second
                        acc[CB - 1] = mfma_bf16(fr[64 * (FS + NK)], b1, acc[CB - 1]);
                        acc[CB - 1] = mfma_bf16(fr[64 * (FS + NK + 1)], pick2(xt.l, mlt2, xt.l, 0u), acc[CB - 1]);
                    }
                }
            }
            // ||c||^2 - 2 x.c, first minimum wins (_k_means_lloyd.pyx:196-212)
            float bd = INFINITY;
            int bi = 4 * h;
#pragma unroll
            for (int cb = 0; cb < CBF; ++cb) {
                const float4 c4 = *reinterpret_cast<const float4*>(&sN[16 * cb + 4 * h]);
                const float cn[4] = {c4.x, c4.y, c4.z, c4.w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    // a NaN distance compares false: it never wins
                    const float dd = fmaf(-2.0f, acc[cb][i], cn[i]);
                    const bool take = dd < bd;
                    bd = take ? dd : bd;
                    bi = take ? 16 * cb + 4 * h + i : bi;
                }
            }
            if constexpr (STK) {
                // centre 16(CB-1) + h: the sum of its three parts' products
                const float dot = (acc[CB - 1][2] + acc[CB - 1][1]) + acc[CB - 1][0];
                const float dd = fmaf(-2.0f, dot, sN[16 * (CB - 1) + h]);
                const bool take = dd < bd;
                bd = take ? dd : bd;
                bi = take ? 16 * (CB - 1) + h : bi;
            }
            argmin_swap<16>(bd, bi);
            argmin_swap<32>(bd, bi);
            // lanes 0..15: row = lane
            __builtin_amdgcn_raw_buffer_store_b32(bi, rl, lane * 4, 0, 0);
            if (a.emin != nullptr) {
                const __amdgpu_buffer_rsrc_t re = __builtin_amdgcn_make_buffer_rsrc(
                    a.emin + rb, (short)0, (int)(nrow > 0 ? nrow * 4 : 0), 0x00020000);
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(bd), re, lane * 4, 0, 0);
            }
            changed += (int)__popcll(__ballot(valid && old != bi));
            // this half tile's rows per cluster: the words of round r - 2, read
            // by both sums waves before they read any block of round r - 1
            // (waited on above), are cleared, then the bits set (an OR: any
            // order gives the same mask)
            unsigned* const mw = sMask[r & 1][e];
            mw[lane] = 0u;
            if (valid) atomicOr(&mw[bi], 1u << lane);
            set_flag(&sReady[e], r + 1);
        }
        if (rounds_e < rounds) {
            // the skipped half's round: once the sums waves are past the round
            // before (as in the loop), its tile rows zeroed (they meet zero
            // masks, but LDS a first round never wrote may hold NaN bit
            // patterns) and its mask words cleared, then the half declared
            // labelled: no row of it counts
            const int r = rounds_e;
            wait_blocks(r, 0, NFB - 1);
            char* const half = tiles + m * TILEB + 16 * hf * RSB;  // the half tile, 16 RSB bytes
#pragma unroll
            for (int i = 0; i < (RSB + 63) / 64; ++i) {
                const int c = lane + 64 * i;  // 16-byte units
                if (c < RSB) *reinterpret_cast<v4u*>(half + 16 * c) = v4u{0u, 0u, 0u, 0u};
            }
            sMask[r & 1][e][lane] = 0u;
            set_flag(&sReady[e], r + 1);
        }
        // one global atomic per block (below): 2,048 waves adding to one
        // address at the end of a step cost up to 16 us while labels move
        if (lane == 0 && changed != 0) atomicAdd(&sChg, changed);
        __syncthreads();  // every sums wave is done: the tile area is free
        __syncthreads();  // the sums are in LDS
    } else {
        // (every wave at the same issue priority: raising the sums waves',
        // whose progress the E-step waves wait on, was no faster)
        // sums waves 8..15: the centre fragments (centres >= k and features
        // >= ld zero), ||c||^2 and the halt test.  Every set-up load goes out
        // at once, before any is used (one memory round trip): the halt flag,
        // the centre values of every fragment (out-of-range items read centre
        // 0 and are zeroed), and wave 8's loop state.
        const int wt = tid - 512;  // 0 .. 511
        const int prev = st->done;
        // full blocks: fragment (cb, s, part), item idx = 64 (cb NK + s) + lane
        constexpr int NE = CB * NK * 64;
        constexpr int NU = (NE + 511) / 512;
        float4 cf[NU][2];
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            const int idx = wt + 512 * u;
            const int l = idx & 63, cs = idx >> 6;  // cs = cb * NK + s
            const int cb = cs / NK, sk = cs - cb * NK;
            const int cl = 16 * cb + (l & 15);
            const bool ok = idx < NE && cl < k;
            const float* p = C + (ok ? (long)cl * ld + 32 * sk + 8 * (l >> 4) : 0L);
            cf[u][0] = *reinterpret_cast<const float4*>(p);
            cf[u][1] = *reinterpret_cast<const float4*>(p + 4);
        }
        // full blocks' tail: fragment (cb, q), item wt = 64 cb + lane
        float4 ct[2];
        if constexpr (TAIL > 0) {
            const int l = wt & 63, cb = wt >> 6, hh = l >> 4;
            const int cl = 16 * cb + (l & 15);
            const bool ok = wt < CB * 64 && cl < k;
            const float* p = C + (ok ? (long)cl * ld + 32 * NK + (TAIL == 16 ? 8 * (hh & 1) : 0) : 0L);
            ct[0] = *reinterpret_cast<const float4*>(p);
            ct[1] = TAIL == 16 ? *reinterpret_cast<const float4*>(p + 4) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        // stacked block: K-step fragment s, item wt = 64 s + lane (lane = 16h
        // + 4 slot + p: part p of centre 16(CB-1) + slot, p = 3 zero); its
        // tail fragments, item wt = 64 NK + lane
        float4 cs4[2], cst[2];
        if constexpr (STK) {
            {
                const int l = wt & 63, sk = wt >> 6;
                const int pp = l & 3, cl = 16 * (CB - 1) + ((l & 15) >> 2);
                const bool ok = wt < 64 * NK && pp < 3 && cl < k;
                const float* q = C + (ok ? (long)cl * ld + 32 * sk + 8 * (l >> 4) : 0L);
                cs4[0] = *reinterpret_cast<const float4*>(q);
                cs4[1] = *reinterpret_cast<const float4*>(q + 4);
            }
            if constexpr (TAIL > 0) {
                const int l = (wt - 64 * NK) & 63, hh = l >> 4;
                const int pp = l & 3, cl = 16 * (CB - 1) + ((l & 15) >> 2);
                const bool ok = wt >= 64 * NK && wt < 64 * NK + 64 && pp < 3 && cl < k;
                const float* q = C + (ok ? (long)cl * ld + 32 * NK + (TAIL == 16 ? 8 * (hh & 1) : 0) : 0L);
                cst[0] = *reinterpret_cast<const float4*>(q);
                cst[1] = TAIL == 16 ? *reinterpret_cast<const float4*>(q + 4) : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
        StepNormsIn sni;
        if (wave == 8) sni = step_norms_load(a, lane);
        if (prev != 0) {
            if (tid == 512) sDone = prev;
            __syncthreads();
            return;
        }
        const float4 z4f = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            const int idx = wt + 512 * u;
            const int l = idx & 63, cs = idx >> 6;
            const int cl = 16 * (cs / NK) + (l & 15);
            if (idx < NE) {
                const bool ok = cl < k;
                const Parts8 p = split8(ok ? cf[u][0] : z4f, ok ? cf[u][1] : z4f);
                sFr[64 * (3 * cs) + l] = p.h;
                sFr[64 * (3 * cs + 1) + l] = p.m;
                sFr[64 * (3 * cs + 2) + l] = p.l;
            }
        }
        if constexpr (TAIL > 0) {
            // tail fragments (cb, q): lane l = 16h + r holds values 32q + 8h ..
            // of centre 16cb + r's tail row (blocks of TAIL values: parts (h,
            // m, l, h, m, h) of its features 32NK .., zeros after them)
            if (wt < CB * 64) {
                const int l = wt & 63, cb = wt >> 6, hh = l >> 4;
                const bool ok = 16 * cb + (l & 15) < k;
                if constexpr (TAIL == 4) {
                    const Parts4 p = split4(ok ? ct[0] : z4f);
                    const v4s z4 = v4s{0, 0, 0, 0};
                    // blocks 2hh, 2hh + 1
                    const v4s q0 = hh < 3 ? part_of(p, tail_cpart(2 * hh)) : z4;
                    const v4s q1 = hh < 3 ? part_of(p, tail_cpart(2 * hh + 1)) : z4;
                    sFr[64 * (FT + cb) + l] = cat8(q0, q1);
                } else {
                    const Parts8 p = split8(ok ? ct[0] : z4f, ok ? ct[1] : z4f);
#pragma unroll
                    for (int q = 0; q < 3; ++q) sFr[64 * (FT + cb * NT + q) + l] = part_of(p, tail_cpart(2 * q + (hh >> 1)));
                }
            }
        }
        if constexpr (STK) {
            if (wt < 64 * NK) {
                const int l = wt & 63, sk = wt >> 6;
                const int pp = l & 3, cl = 16 * (CB - 1) + ((l & 15) >> 2);
                const bool ok = pp < 3 && cl < k;
                sFr[64 * (FS + sk) + l] = part_of(split8(ok ? cs4[0] : z4f, ok ? cs4[1] : z4f), pp < 3 ? pp : 0);
            }
            if constexpr (TAIL > 0) {
                if (wt >= 64 * NK && wt < 64 * NK + 64) {
                    const int l = wt - 64 * NK, hh = l >> 4;
                    const int pp = l & 3, cl = 16 * (CB - 1) + ((l & 15) >> 2);
                    const bool ok = pp < 3 && cl < k;
                    const v4s z4 = v4s{0, 0, 0, 0};
                    if constexpr (TAIL == 4) {
                        const v4s cp = part_of(split4(ok ? cst[0] : z4f), pp < 3 ? pp : 0);
                        // blocks 2hh, 2hh + 1 of (c_p, c_p, c_p, 0, ...)
                        sFr[64 * (FS + NK) + l] = cat8(hh < 2 ? cp : z4, hh == 0 ? cp : z4);
                    } else {
                        const v8bf cp = part_of(split8(ok ? cst[0] : z4f, ok ? cst[1] : z4f), pp < 3 ? pp : 0);
                        sFr[64 * (FS + NK) + l] = cp;
                        sFr[64 * (FS + NK + 1) + l] = hh < 2 ? cp : cat8(z4, z4);
                    }
                }
            }
        }
        if (wt < 8) {
            sReady[wt] = 0;
            sProg[wt] = 0;
        }
        if (wt == 0) sChg = 0;
        if (wt < 256) {
            sCnt[wt >> 6][wt & 63] = 0;
            unsigned w[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                w[j] = ((wt >> (2 * j)) & 1 ? 0x3f80u : 0u) | ((wt >> (2 * j + 1)) & 1 ? 0x3f800000u : 0u);
            sOneHot[wt] = __builtin_bit_cast(v8bf, v4u{w[0], w[1], w[2], w[3]});
        }
        (&sMask[0][0][0])[wt] = 0u;
        (&sMask[0][0][0])[512 + wt] = 0u;
        if (wave == 8) {
            step_norms_apply<CPC>(a, lane, sni, sN, &sDone);
            if constexpr (STK) {
                // The stacked block's distances take all nine part products,
                // the full blocks' six: an exact copy of an earlier centre
                // would not tie with it, and could take rows that scikit-learn
                // gives the lower index (the copy then never gets one).  A
                // stacked centre equal to an earlier one, feature for feature,
                // gets +inf here (its norm equal first: one compare a lane).
                const int s0 = 16 * (CB - 1);
                for (int s = 0; s < 4 && s0 + s < k; ++s) {
                    const float ns = sN[s0 + s];
                    unsigned long long m = __ballot(lane < s0 && sN[lane] == ns);
                    while (m != 0ull) {
                        const int j = __ffsll((long long)m) - 1;
                        m &= m - 1ull;
                        bool same = true;
                        for (int f = lane; f < ld; f += 64) same = same && C[(long)j * ld + f] == C[(long)(s0 + s) * ld + f];
                        if (__ballot(!same) == 0ull) {
                            if (lane == 0) sN[s0 + s] = INFINITY;
                            break;
                        }
                    }
                }
            }
        }
        __syncthreads();
        if (sDone != 0) return;
        // sums wave 8 + w: SIMD m = w & 3, feature blocks [0, NFA) (w < 4) or
        // [NFA, NFB) of its tiles
        const int w = wave - 8, m = w & 3;
        const int rounds = rounds_of(m);
        const char* const tile = tiles + m * TILEB;
        // transposed reads: lane 16h + 4q + jr supplies the address of row 8h
        // + jr (+ 4 for the second read), features 4q .. 4q + 3 of a block, and
        // receives rows 8h .. 8h + 3 (+ 4) of feature 4(l%16/4) + l%4 = l%16
        const int q4 = r16 & 3, jr = r16 >> 2;
        const char* const src = tile + (8 * h + jr) * RSB + 8 * q4;
        // TAIL = 4, the last block: column n = 4p + f is part p of feature
        // 32NK + f (p = 3: part 0 again, never published)
        const char* const srct = tile + (8 * h + jr) * RSB + (q4 < 3 ? q4 : 0) * 2 * KP + 64 * NK;
        auto sums = [&](auto fb0c, auto nfc) {
            constexpr int FB0 = decltype(fb0c)::value, NF = decltype(nfc)::value;
            v4f S[CB][NF];
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) {
#pragma unroll
                for (int j = 0; j < NF; ++j) S[cb][j] = v4f{0.f, 0.f, 0.f, 0.f};
            }
            // the first sums wave of the SIMD also counts the rows per
            // cluster: lane (r16, h) adds the bits of the mask byte it reads
            // (cluster 16 cb + r16, rows 8h .. 8h + 7); integer adds, so the
            // counts are exact and order-free.  (An LDS atomic per row by the
            // E-step waves cost up to 5 us per launch: same-address adds.)
            int cnt[CB];
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) cnt[cb] = 0;
            for (int r = 0; r < rounds; ++r) {
                wait_flag(&sReady[m], r + 1);
                wait_flag(&sReady[m + 4], r + 1);
                // A[cb][j] = 1 when row 8h + j has label 16 cb + r16: byte h of
                // that cluster's row mask (rows 0..15 from E-step wave m, 16..31
                // from wave m + 4), through the one-hot table
                v8bf A[CB];
                {
                    const unsigned* mw = sMask[r & 1][h < 2 ? m : m + 4];
                    const int sft = 8 * (h & 1);
                    unsigned mv[CB];
#pragma unroll
                    for (int cb = 0; cb < CB; ++cb) mv[cb] = mw[16 * cb + r16];
#pragma unroll
                    for (int cb = 0; cb < CB; ++cb) A[cb] = sOneHot[(mv[cb] >> sft) & 0xffu];
                    if constexpr (FB0 == 0) {
#pragma unroll
                        for (int cb = 0; cb < CB; ++cb) cnt[cb] += __builtin_popcount((mv[cb] >> sft) & 0xffu);
                    }
                }
                // the B operands of block j + 1 are read before block j's MFMAs
                auto read_block = [&](int j, v8bf (&b)[3]) {
                    const int fb = FB0 + j;
                    if (TAIL == 4 && fb == NFB - 1) {
                        b[0] = cat8(lds_tr16(srct), lds_tr16(srct + 4 * RSB));
                    } else {
#pragma unroll
                        for (int p = 0; p < 3; ++p) {
                            const char* s0 = src + p * 2 * KP + 32 * fb;
                            b[p] = cat8(lds_tr16(s0), lds_tr16(s0 + 4 * RSB));
                        }
                    }
                    // feature block fb of the tile has been read
                    set_flag(&sProg[w], r * NF + j + 1);
                };
                v8bf bc[3], bn[3];
                read_block(0, bc);
#pragma unroll
                for (int j = 0; j < NF; ++j) {
                    if (j + 1 < NF) read_block(j + 1, bn);
                    if (TAIL == 4 && FB0 + j == NFB - 1) {
#pragma unroll
                        for (int cb = 0; cb < CB; ++cb) S[cb][j] = mfma_bf16(A[cb], bc[0], S[cb][j]);
                    } else {
                        // lo, mid, hi; consecutive MFMAs write different accumulators
#pragma unroll
                        for (int p = 2; p >= 0; --p) {
#pragma unroll
                            for (int cb = 0; cb < CB; ++cb) S[cb][j] = mfma_bf16(A[cb], bc[p], S[cb][j]);
                        }
                    }
#pragma unroll
                    for (int p = 0; p < 3; ++p) bc[p] = bn[p];
                }
            }
            if constexpr (FB0 == 0) {
                // the SIMD's counts: the four row groups of each cluster
#pragma unroll
                for (int cb = 0; cb < CB; ++cb) {
                    int c = cnt[cb];
                    c += __shfl_xor(c, 16, 64);
                    c += __shfl_xor(c, 32, 64);
                    if (h == 0) sCnt[m][16 * cb + r16] = c;
                }
            }
            __syncthreads();  // every wave is done with its tile
            // the sums into red = [4][CPC][ld] (D lane l: clusters 16cb +
            // 4(l/16) + i, column l%16 of block fb)
            float* const red = lds;
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) {
#pragma unroll
                for (int j = 0; j < NF; ++j) {
                    const int fb = FB0 + j;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int row = (m * CPC + 16 * cb + 4 * h + i) * ld;
                        const float v = S[cb][j][i];
                        if (TAIL == 4 && fb == NFB - 1) {
                            // columns f, 4 + f, 8 + f: parts h, m, l of feature 32NK + f
                            const float vm = __shfl_down(v, 4, 16);
                            const float vl = __shfl_down(v, 8, 16);
                            if (r16 < 4) red[row + 32 * NK + r16] = (vl + vm) + v;
                        } else {
                            const int f = 16 * fb + r16;
                            if (f < ld) red[row + f] = v;
                        }
                    }
                }
            }
        };
        if (w < 4)
            sums(std::integral_constant<int, 0>{}, std::integral_constant<int, NFA>{});
        else
            sums(std::integral_constant<int, NFA>{}, std::integral_constant<int, NFZ>{});
        __syncthreads();
    }
    if (tid == 0 && sChg != 0) atomicAdd(a.changed, sChg);
    combine_sums<CPC, 1024>(lds, ld, k, a.psum, a.pcnt, sCnt, tid, &a.state->present[a.iter & 1]);
}

// ---------------------------------------------------------------------------
// k_assign3: the E-step for any k (the generic path and the assign entry
// point) on bf16 MFMA over the three-part split, with k_fused3's operand
// layout.  A block of 8 waves owns 256 rows (32 per wave: two 16-row groups);
// it takes the centres in passes of 16*CB (A operands from LDS) and keeps per
// lane the first minimum over its centres 16cb + 4(l/16) + i, in ascending
// order across passes; the four lanes of a row are combined after the last
// pass.  X is read once per pass (k/(16 CB) times).
//
// The centres' parts come from an image that k_centre_image writes once per
// step: per stage (pass p, SEG-feature segment sg) the three bf16 parts of
// centres 16 CB p.. as rows of CSTR bf16 (zeros past k and ld), then the
// pass's ||c||^2 (+inf past k), padded to whole KB -- the LDS layout itself.
// Two LDS stages alternate: while the MFMAs of one run, the next stage's
// image is copied in with direct-to-LDS loads (1 KB per wave instruction).
template <int CB>
struct Assign3Geom {
    static constexpr int CPC = 16 * CB;                             // centres per pass
    static constexpr int SEG = CB >= 16 ? 32 : CB >= 8 ? 64 : 128;  // features per stage
    static constexpr int NKS = SEG / 32;                            // K32 steps per stage
    static constexpr int CSTR = SEG + 8;                            // bf16 per centre row: an odd number of 16-byte units
    static constexpr int CPART = CPC * CSTR;                        // bf16 from one part to the next
    static constexpr int PBYTES = 3 * CPART * 2;                    // the three parts
    // + ||c||^2 of the stage's pass and of the pass before it (cyclically),
    // whole KB
    static constexpr int STAGE = (PBYTES + 2 * CPC * 4 + 1023) / 1024 * 1024;
    static constexpr size_t LDS = size_t(2) * STAGE;
};

template <int CB>
__global__ __launch_bounds__(256) void k_centre_image(const float* __restrict__ C, const float* __restrict__ cnorm,
                                                      int k, int ld, int nseg, char* __restrict__ img)
{
    using G = Assign3Geom<CB>;
    const int stg = blockIdx.x, p = stg / nseg, sg = stg - p * nseg;
    char* const out = img + (size_t)stg * G::STAGE;
    __bf16* const parts = reinterpret_cast<__bf16*>(out);
    constexpr int Q = G::CSTR / 4;  // 4-feature groups per row, padding included
    for (int e = threadIdx.x; e < G::CPC * Q; e += 256) {
        const int c = e / Q, q = e - c * Q;
        const int j = p * G::CPC + c, f = sg * G::SEG + 4 * q;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (4 * q < G::SEG && j < k && f < ld) v = *reinterpret_cast<const float4*>(C + (long)j * ld + f);
        const Parts4 pt = split4(v);
        __bf16* dst = parts + c * G::CSTR + 4 * q;
        *reinterpret_cast<v4s*>(dst) = pt.h;
        *reinterpret_cast<v4s*>(dst + G::CPART) = pt.m;
        *reinterpret_cast<v4s*>(dst + 2 * G::CPART) = pt.l;
    }
    // ||c||^2 of pass p, then of pass p - 1 (the last pass for p = 0): the
    // assign kernel reads the norms of the pass it has just finished from the
    // stage that follows it
    const int npass = (k + G::CPC - 1) / G::CPC, pp = (p + npass - 1) % npass;
    float* const sn = reinterpret_cast<float*>(out + G::PBYTES);
    for (int c = threadIdx.x; c < G::STAGE / 4 - G::PBYTES / 4; c += 256) {
        const int j = (c < G::CPC ? p : pp) * G::CPC + c % G::CPC;
        sn[c] = c < 2 * G::CPC ? (j < k ? cnorm[j] : INFINITY) : 0.f;  // padding centres never win
    }
}

template <int CB>
__global__ __launch_bounds__(512, 1) void k_assign3(const float* __restrict__ X, long n, int ld,
                                                   const char* __restrict__ img, int k, int* __restrict__ labels,
                                                   LoopState* st, int* changed, const float* __restrict__ C, int d,
                                                   double* __restrict__ inert, float* __restrict__ emin)
{
    if (st != nullptr && st->done != 0) return;
    using G = Assign3Geom<CB>;
    constexpr int CPC = G::CPC, SEG = G::SEG, NKS = G::NKS, CSTR = G::CSTR, CPART = G::CPART;
    extern __shared__ __attribute__((aligned(1024))) char smem[];  // two stages
    __shared__ int sChg;  // labels the block changed
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 4, r16 = lane & 15;
    if (tid == 0) sChg = 0;  // (published by the first barrier)
    int nchg = 0;            // lane 0: labels this wave changed
    double itot = 0.0;       // lanes 0..31: the inertia of their rows
    const int npass = (k + CPC - 1) / CPC;
    const int nseg = (ld + SEG - 1) / SEG;
    const int nst = npass * nseg;
    // stage stg's image into LDS stage b: wave w copies KB w, w + 8, .. (the
    // buffer descriptor spans the whole image)
    const __amdgpu_buffer_rsrc_t irs = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(img), (short)0,
                                                                         nst * G::STAGE, 0x00020000);
    // (the offsets go through plain ints: a template-dependent argument of the
    // builtin leaves the host side without the kernel's launch stub)
    const int stage_bytes = G::STAGE;
    auto copy_stage = [&](int stg, int b) {
        char* dst = smem + b * stage_bytes;
        for (int i = wave; i < stage_bytes / 1024; i += 8) {
            const int soff = stg * stage_bytes + i * 1024;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(irs, (__attribute__((address_space(3))) void*)(dst + i * 1024), 16,
                                                     lane * 16, soff, 0, 0);
        }
    };
    // this wave's 32 rows of the row block at base (past the last row the
    // descriptor is empty: loads return 0)
    auto rows_rsrc = [&](long base) {
        const long wrow = base + 32 * wave;
        const long nrow = n - wrow < 32 ? (n - wrow > 0 ? n - wrow : 0) : 32;
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(X + (nrow > 0 ? wrow * ld : 0)), (short)0,
                                                 (int)(nrow * ld * 4), 0x00020000);
    };
    // rows 16g + l%16, features f + 8h..: past the row's end the next row's
    // (finite) values meet zero centre parts.  The K step after the current
    // one is loaded while the current one's MFMAs run.
    float4 xr[2][2];
    auto xload = [&](__amdgpu_buffer_rsrc_t r, int f) {
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            const int o = ((16 * g + r16) * ld + f + 8 * h) * 4;
            xr[g][0] = load_quad(r, o);
            xr[g][1] = load_quad(r, o + 16);
        }
    };
    xload(rows_rsrc((long)blockIdx.x * 256), 0);
    copy_stage(0, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    int cur = 0;  // the LDS stage holding the current stage

    for (long base = (long)blockIdx.x * 256; base < n; base += (long)gridDim.x * 256) {
        const long wrow = base + 32 * wave;  // this wave's first row
        const long nrow = n - wrow < 32 ? (n - wrow > 0 ? n - wrow : 0) : 32;
        const __amdgpu_buffer_rsrc_t rs = rows_rsrc(base);
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
                const int stg = p * nseg + sg;
                const int f0 = sg * SEG;
                const __bf16* const cbase = reinterpret_cast<const __bf16*>(smem + cur * G::STAGE) + r16 * CSTR + 8 * h;
                const int nks = min(NKS, (ld - f0 + 31) / 32);
                for (int ks = 0; ks < nks; ++ks) {
                    Parts8 xp[2];
#pragma unroll
                    for (int g = 0; g < 2; ++g) xp[g] = split8(xr[g][0], xr[g][1]);
                    // the next K step's rows: this stage's next, the next
                    // segment's or pass's first (same rows), or the next row
                    // block's first
                    if (ks + 1 < nks) {
                        xload(rs, f0 + 32 * (ks + 1));
                    } else if (sg + 1 < nseg) {
                        xload(rs, f0 + SEG);
                    } else if (p + 1 < npass) {
                        xload(rs, 0);
                    } else if (base + (long)gridDim.x * 256 < n) {
                        xload(rows_rsrc(base + (long)gridDim.x * 256), 0);
                    }
                    // the next stage's copy goes out behind the X loads that
                    // this stage still waits on (loads complete in order)
                    if (ks == nks - 1 && nst > 1) copy_stage(stg + 1 < nst ? stg + 1 : 0, cur ^ 1);
                    // four centre blocks at a time, product-major over their
                    // eight accumulators: consecutive MFMAs write different
                    // accumulators (a block's six products back to back wait
                    // on each other).  Each accumulator takes dot6's products
                    // in dot6's order.
                    constexpr int CG = 4;
#pragma unroll
                    for (int cb0 = 0; cb0 < CB; cb0 += CG) {
                        Parts8 cpt[CG];
#pragma unroll
                        for (int c = 0; c < CG; ++c) {
                            const __bf16* cp = cbase + 16 * (cb0 + c) * CSTR + 32 * ks;
                            cpt[c] = Parts8{*reinterpret_cast<const v8bf*>(cp),
                                            *reinterpret_cast<const v8bf*>(cp + CPART),
                                            *reinterpret_cast<const v8bf*>(cp + 2 * CPART)};
                        }
#pragma unroll
                        for (int pr = 0; pr < 6; ++pr) {
#pragma unroll
                            for (int c = 0; c < CG; ++c) {
                                const Parts8& cc = cpt[c];
                                const v8bf ca = pr == 0 ? cc.m : pr == 1 ? cc.l : pr == 2 ? cc.h : pr == 3 ? cc.m : cc.h;
#pragma unroll
                                for (int g = 0; g < 2; ++g) {
                                    const Parts8& x = xp[g];
                                    const v8bf xb = pr == 0 ? x.m : pr == 1 ? x.h : pr == 2 ? x.l : pr == 3 ? x.h
                                                                                               : pr == 4 ? x.m : x.h;
                                    acc[g][cb0 + c] = mfma_bf16(ca, xb, acc[g][cb0 + c]);
                                }
                            }
                        }
                    }
                }
                if (nst > 1) {
                    // the next stage is in (every wave's copies) and this one
                    // is read: swap
                    __builtin_amdgcn_s_waitcnt(0);
                    __syncthreads();
                    cur ^= 1;
                }
            }
            // ||c||^2 - 2 x.c, first minimum wins (_k_means_lloyd.pyx:196-212);
            // the lane's centres come in ascending order, passes too.  With
            // one stage, the pass's ||c||^2 are in it; else they are read as
            // the previous pass's norms of the stage now current, which the
            // stage copies rewrite only after the next barrier (a wave past
            // that barrier has every wave's reads of this behind it).
            const float* sN = reinterpret_cast<const float*>(smem + cur * G::STAGE + G::PBYTES) + (nst > 1 ? CPC : 0);
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) {
                const float4 c4 = *reinterpret_cast<const float4*>(&sN[16 * cb + 4 * h]);
                const float cn[4] = {c4.x, c4.y, c4.z, c4.w};
#pragma unroll
                for (int g = 0; g < 2; ++g) {
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
        float mymin = 0.f;
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
            if (h == g) {  // lanes 0..31: row = lane
                mylab = i0;
                mymin = d0;
            }
        }
        const bool valid = lane < nrow;
        const long row = wrow + lane;
        int moved = 0;
        if (valid) {
            if (changed != nullptr) moved = labels[row] != mylab;
            labels[row] = mylab;
            // the row's minimum ||c||^2 - 2 x.c, for the relocation's
            // candidate search (as k_fused3 writes it)
            if (emin != nullptr) emin[row] = mymin;
        }
        if (changed != nullptr) nchg += (int)__popcll(__ballot(moved));
        // the inertia term of the row: ||x - c_label||^2 in fp32, in the
        // association order of sklearn's _euclidean_dense_dense
        // (_k_means_common.pyx:16-43; the same sums as k_rowdist), from the
        // row just read (in the L2) and the fp32 centre; lane l < 32 takes
        // row l.  (The centre's exact parts from the LDS image instead of C
        // took 121 us instead of 87 at 500000 x 100, k = 50: bank conflicts
        // of 32 random centre rows; each row split over lanes l and l + 32,
        // 118 us.)
        if (inert != nullptr && valid) {
#pragma clang fp contract(off)
            const float4* x4 = reinterpret_cast<const float4*>(X + row * ld);
            const float4* c4 = reinterpret_cast<const float4*>(C + (long)mylab * ld);
            float res = 0.f;
            const int nfull = d >> 2;
#pragma unroll 5
            for (int g = 0; g < nfull; ++g) {
                const float4 xv = x4[g], cv = c4[g];
                const float t0 = xv.x - cv.x, t1 = xv.y - cv.y, t2 = xv.z - cv.z, t3 = xv.w - cv.w;
                res += ((t0 * t0 + t1 * t1) + t2 * t2) + t3 * t3;
            }
            if (d & 3) {  // the row's last features, one by one
                const float4 xv = x4[nfull], cv = c4[nfull];
                float tt = xv.x - cv.x;
                res += tt * tt;
                if ((d & 3) > 1) {
                    tt = xv.y - cv.y;
                    res += tt * tt;
                }
                if ((d & 3) > 2) {
                    tt = xv.z - cv.z;
                    res += tt * tt;
                }
            }
            itot += (double)res;
        }
    }
    // one global atomic per block: a wave-level atomic per 32 rows on one
    // address serialises thousands of them while labels move
    if (changed != nullptr) {
        if (lane == 0 && nchg != 0) atomicAdd(&sChg, nchg);
        __syncthreads();
        if (tid == 0 && sChg != 0) atomicAdd(changed, sChg);
    }
    // the block's inertia total: lanes (butterfly), then waves in order
    if (inert != nullptr) {
        __shared__ double sI[8];
        itot = wave_sum(itot);
        if (lane == 0) sI[wave] = itot;
        __syncthreads();
        if (tid == 0) {
            double t = 0.0;
            for (int w = 0; w < 8; ++w) t += sI[w];
            inert[blockIdx.x] = t;
        }
    }
}

typedef void (*assign3_fn)(const float*, long, int, const char*, int, int*, LoopState*, int*, const float*, int,
                           double*, float*);
typedef void (*image_fn)(const float*, const float*, int, int, int, char*);

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

// (stages, bytes per stage) of k_assign3's centre image for (k, ld)
static void assign3_stages(int k, int ld, int* nst, int* nseg, size_t* stage)
{
    const int cb = assign3_cb(k);
    const int cpc = 16 * cb;
    const int seg = cb == 4 ? Assign3Geom<4>::SEG : cb == 8 ? Assign3Geom<8>::SEG : Assign3Geom<16>::SEG;
    *stage = cb == 4 ? Assign3Geom<4>::STAGE : cb == 8 ? Assign3Geom<8>::STAGE : Assign3Geom<16>::STAGE;
    *nseg = (ld + seg - 1) / seg;
    *nst = ((k + cpc - 1) / cpc) * *nseg;
}

size_t assign3_image_bytes(int k, int ld)
{
    int nst = 0, nseg = 0;
    size_t stage = 0;
    assign3_stages(k, ld, &nst, &nseg, &stage);
    return size_t(nst) * stage;
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
    if (a.img == nullptr) return hipErrorInvalidValue;
    int nst = 0, nseg = 0;
    size_t stage = 0;
    assign3_stages(a.k, a.ld, &nst, &nseg, &stage);
    const int cb = assign3_cb(a.k);
    const image_fn img = cb == 4 ? &k_centre_image<4> : cb == 8 ? &k_centre_image<8> : &k_centre_image<16>;
    hipLaunchKernelGGL(img, dim3((unsigned)nst), dim3(256), 0, s, a.C, a.cnorm, a.k, a.ld, nseg, a.img);
    long blocks = (a.n + 255) / 256;
    if (blocks > num_cu) blocks = num_cu;
    hipLaunchKernelGGL(assign3_kernel(a.k), dim3((unsigned)blocks), dim3(512), assign3_lds(a.k), s, a.X, a.n, a.ld,
                       a.img, a.k, a.labels, a.state, a.changed, a.C, a.d, a.inert, a.emin);
    if (a.inert_blocks != nullptr) *a.inert_blocks = (int)blocks;
    return hipGetLastError();
}
typedef void (*fused_fn)(FusedArgs);

template <int NQ, int... CBs>
struct Fused3Table {
    static fused_fn get(int cb, bool stk)
    {
        fused_fn f = nullptr;
        ((cb == CBs ? (f = stk ? &k_fused3<CBs, NQ, true> : &k_fused3<CBs, NQ, false>, 0) : 0), ...);
        return f;
    }
    static size_t dyn_lds(int cb) { return Fused3Geom<NQ>::lds(cb); }
};

// The split kernel for row strides of 32 floats and more (below that the K
// steps would be mostly padding).  The last 16-centre block is stacked when
// it holds at most 4 centres.
static fused_fn fused3_kernel(int k, int ld, size_t* dyn)
{
    if (k < 1 || k > 64) return nullptr;
    const int cb = (k + 15) / 16;
    const bool stk = k - 16 * (cb - 1) <= 4;
    switch (ld) {
    case 32: *dyn = Fused3Table<8, 1, 2, 3, 4>::dyn_lds(cb); return Fused3Table<8, 1, 2, 3, 4>::get(cb, stk);
    case 48: *dyn = Fused3Table<12, 1, 2, 3, 4>::dyn_lds(cb); return Fused3Table<12, 1, 2, 3, 4>::get(cb, stk);
    case 64: *dyn = Fused3Table<16, 1, 2, 3, 4>::dyn_lds(cb); return Fused3Table<16, 1, 2, 3, 4>::get(cb, stk);
    case 80: *dyn = Fused3Table<20, 1, 2, 3, 4>::dyn_lds(cb); return Fused3Table<20, 1, 2, 3, 4>::get(cb, stk);
    case 100: *dyn = Fused3Table<25, 1, 2, 3, 4>::dyn_lds(cb); return Fused3Table<25, 1, 2, 3, 4>::get(cb, stk);
    default: return nullptr;
    }
}

int fused3_ready(int k, int ld)
{
    if (split_disabled()) return 0;
    size_t dyn = 0;
    fused_fn f = fused3_kernel(k, ld, &dyn);
    // sMask, sOneHot, sCnt, sN, flags
    const size_t stat = 2 * 8 * 64 * sizeof(unsigned) + 256 * 16 + 4 * 64 * sizeof(int) + 64 * sizeof(float) + 80;
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
    hipLaunchKernelGGL(f, dim3(a.blocks), dim3(1024), dyn, s, a);
    return hipGetLastError();
}

}  // namespace skm
