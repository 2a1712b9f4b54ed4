// fused_common.h -- device helpers shared by the fused Lloyd-step kernels
// (fused_kernels.hip: k_fused; split_kernels.hip: k_fused3, k_assign3).
#pragma once

#include <math.h>

#include "device.h"

namespace skm {

// Floats per LDS row for a row of NQ float4s: an odd number of float4s, so
// 16-byte accesses of different rows at the same column fall in different
// bank groups.
__host__ __device__ constexpr int fused_stride(int nq) { return 4 * (nq | 1); }

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

// The loads of step_norms, issued together (one memory round trip) so that a
// kernel can put them in flight beside its other set-up loads: the first
// kNormChunks chunk partials of the lane's cluster (further chunks, if any,
// are read by step_norms_apply).
constexpr int kNormChunks = 4;
struct StepNormsIn {
    double v[2 * kNormChunks];  // lane j < k: chunk c's shift^2 and ||c||^2 in v[2c], v[2c + 1]
    int count;                  // lane j < k: cluster j's count
    int chg;                    // rows the previous step's E-step relabelled
    int reloc_iter;             // the last step k_reloc relocated in
    float cnorm;                // lane j < k: ||c||^2 from a.cnorm (no decision to take)
};

__device__ __forceinline__ StepNormsIn step_norms_load(const FusedArgs& a, int lane)
{
    StepNormsIn in;
    in.count = 1;
    in.chg = 0;
    in.reloc_iter = 0;
    in.cnorm = INFINITY;
    const int j = lane;
    if (a.decide) {
        in.chg = *a.prev_changed;
        in.reloc_iter = a.state->reloc_iter;
        const double* pj = a.part + (long)(j < a.k ? j : 0) * a.nch * 2;
#pragma unroll
        for (int u = 0; u < kNormChunks; ++u) {
            const int c = min(u, a.nch - 1);
            in.v[2 * u] = pj[2 * c];
            in.v[2 * u + 1] = pj[2 * c + 1];
        }
        if (j < a.k) in.count = a.counts[j];
    } else if (j < a.k) {
        in.cnorm = a.cnorm[j];
    }
    return in;
}

// Wave 4 of every block: the previous step's stopping rules when a.decide
// (evaluated identically by every block: same loads, same order as
// k_finalize_loop for k <= 64; block 0 records the decision), else nothing
// to decide.  Writes ||c||^2 of this step's centres to sN (padding clusters
// j >= k get +inf: their distance never wins) and the decision to *sDone.
template <int CPC>
__device__ __forceinline__ void step_norms_apply(const FusedArgs& a, int lane, const StepNormsIn& in, float* sN,
                                                 int* sDone)
{
    const int k = a.k;
    const int j = lane;
    if (a.decide) {
        // the chunk partials in chunk order (the finalize's order)
        double tsq = 0.0, tnr = 0.0;
        if (j < k) {
#pragma unroll
            for (int u = 0; u < kNormChunks; ++u) {
                if (u < a.nch) {
                    tsq += in.v[2 * u];
                    tnr += in.v[2 * u + 1];
                }
            }
            const double* pj = a.part + (long)j * a.nch * 2;
            for (int c = kNormChunks; c < a.nch; ++c) {
                tsq += pj[2 * c];
                tnr += pj[2 * c + 1];
            }
        }
        const int count = in.count;
        const int n_empty = wave_sum(j < k && count == 0 ? 1 : 0);
        const double tot = wave_sum(j < k ? (double)(float)tsq : 0.0);
        float mx = j < k ? (float)tsq : 0.f;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
        const int chg = in.chg;
        int done = 0;
        // (empty clusters k_reloc has already relocated do not stop the loop)
        if (n_empty > 0 && in.reloc_iter != a.iter - 1)
            done = 3;
        else if ((a.flags & kStopStrict) && chg == 0)
            done = 1;
        else if (shift_rule_stops(a.flags, a.tol, tot, mx))
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
        if (j < CPC) sN[j] = j < k ? in.cnorm : INFINITY;
        if (lane == 0) *sDone = 0;
    }
}

template <int CPC>
__device__ __forceinline__ void step_norms(const FusedArgs& a, int lane, float* sN, int* sDone)
{
    step_norms_apply<CPC>(a, lane, step_norms_load(a, lane), sN, sDone);
}

// The block's partial sums and counts; its clusters with a row go into the
// presence bits (*present, k <= 64).
template <int CPC, int NT = 512>
__device__ __forceinline__ void combine_sums(const float* red, int ld, int k, float* psum, int* pcnt, int (*sCnt)[64],
                                             int tid, unsigned long long* present)
{
    const int kl = k * ld;
    float* out = psum + (long)blockIdx.x * kl;
    for (int i = tid; i < kl; i += NT) {
        const int j = i / ld;
        const int col = i - j * ld;
        const float* p = red + j * ld + col;
        out[i] = ((p[0] + p[CPC * ld]) + p[2 * CPC * ld]) + p[3 * CPC * ld];
    }
    if (tid < 64) {
        const int c = tid < k ? ((sCnt[0][tid] + sCnt[1][tid]) + sCnt[2][tid]) + sCnt[3][tid] : 0;
        if (tid < k) pcnt[(long)blockIdx.x * k + tid] = c;
        const unsigned long long m = __ballot(c > 0);
        if (tid == 0 && m != 0ull) atomicOr(present, m);
    }
}

}  // namespace skm
