// mh_device.h — device helpers prepended to every generated layer source (gfx950, wave64, hipRTC).
//
// Kept free of #includes so that hipRTC can compile it without a header search path.
#pragma once

#define MH_WAVE 64
#define MH_NXCD 8

// Workgroups are dispatched round-robin over the MI355X's 8 XCDs (block b runs on XCD b % 8), and each XCD has its
// own L2.  Map the hardware block index to a logical one so that every XCD walks one contiguous range of logical
// blocks: rows that are close in index (atoms of the same structure, whose neighbour features overlap) then share
// one L2.  Bijective on [0, nblocks).
__device__ __forceinline__ int mh_xcd_block(int b, int nblocks) {
    const int xcd = b % MH_NXCD, local = b / MH_NXCD;
    const int per = nblocks / MH_NXCD, rem = nblocks % MH_NXCD;
    return xcd < rem ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
}

// Value of `v` in lane `j` (j wave-uniform) as a scalar.
__device__ __forceinline__ int mh_bcast(int v, int j) { return __builtin_amdgcn_readlane(v, j); }

// Sum each of NV per-lane values over the 64 lanes of the wave, NV a power of two <= 64.  Transpose reduction: every
// exchange step halves the number of values a lane carries, so the cost is NV-1 + log2(64/NV) shuffles instead of
// 6*NV.  On return every lane L holds the wave total of component (L >> (6 - log2 NV)) in v[0].  The summation
// order is fixed, so results are bitwise reproducible.
template <int NV>
__device__ __forceinline__ float mh_wave_transpose_sum(float (&v)[NV]) {
    const int lane = threadIdx.x & (MH_WAVE - 1);
    int n = NV;
    int m = MH_WAVE / 2;
#pragma unroll
    for (int step = 0; step < 6; ++step) {
        if (n > 1) {
            n >>= 1;
            const bool hi = (lane & m) != 0;
#pragma unroll
            for (int k = 0; k < NV / 2; ++k) {
                if (k < n) {
                    const float send = hi ? v[k] : v[k + n];
                    const float keep = hi ? v[k + n] : v[k];
                    v[k] = keep + __shfl_xor(send, m, MH_WAVE);
                }
            }
        } else {
            v[0] += __shfl_xor(v[0], m, MH_WAVE);
        }
        m >>= 1;
    }
    return v[0];
}
