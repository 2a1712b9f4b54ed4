// device.h -- device helpers shared by the KMeans kernels (gfx950).
#pragma once

#include "internal.h"

namespace skm {

typedef float v4f __attribute__((ext_vector_type(4)));

// Native 4-float vector for staging registers: arrays of it stay in
// registers (an array of HIP's float4 struct copied whole went to scratch
// memory).
typedef float f4v __attribute__((ext_vector_type(4)));

// LDS row stride for rows of ld floats (ld a multiple of 4): an odd number of
// 16-byte units, so that row-per-lane float4 reads fall in distinct bank
// groups.
__host__ __device__ constexpr int ctg_stride(int ld) { return 4 * ((ld / 4) | 1); }

// Loads NQ float4s of this lane's row (row0 + lane) starting at feature f0,
// with no branches: the buffer descriptor covers exactly the valid rows, so a
// lane past the last row, and any float4 at or past `nq`, reads 0 without a
// memory access.  All NQ loads stay in flight together.
template <int NQ>
__device__ __forceinline__ void load_row_quads(float4* xv, const float* X, long row0, long n, int ld, int f0,
                                               int nq, int lane)
{
    const long rows = n - row0 < 64 ? (n - row0 > 0 ? n - row0 : 0) : 64;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(X + (rows > 0 ? row0 * ld + f0 : 0)), (short)0, (int)(rows * ld * 4), 0x00020000);
    const int base = lane * ld * 4;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        const int off = q < nq ? base + 16 * q : 0x7ffffff0;
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
        xv[q] = *reinterpret_cast<const float4*>(&v);
    }
}

// acc[g] += (lanes 4g..4g+3 of a, broadcast to all 16 blocks) x b, for g < KG:
// v_mfma_f32_4x4x1_16b_f32 with CBSZ=4 (broadcast one 4-lane block of A), ABID=g.
template <int KG, int G = 0>
__device__ __forceinline__ void mfma_groups(v4f* acc, float a, float b)
{
    if constexpr (G < KG) {
        acc[G] = __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, acc[G], 4, G, 0);
        mfma_groups<KG, G + 1>(acc, a, b);
    }
}

// Sum over the 64 lanes of a wave by xor butterfly; all lanes get the total.
template <typename T>
__device__ __forceinline__ T wave_sum(T v)
{
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Load that sees stores other blocks made visible with __threadfence().
template <typename T>
__device__ __forceinline__ T coherent_load(const T* p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace skm
