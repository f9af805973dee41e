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

// Load / store at a wave-uniform base pointer plus a 32-bit unsigned per-lane byte offset.  Written this way the
// compiler keeps the 64-bit base in SGPRs and issues global_load/store with a 32-bit VGPR offset (saddr form), so
// a gather from a different row costs scalar arithmetic only, no 64-bit VALU address computation per access.
__device__ __forceinline__ float mh_ld(const float* __restrict__ base, unsigned boff) {
    return *reinterpret_cast<const float*>(reinterpret_cast<const char*>(base) + boff);
}
__device__ __forceinline__ void mh_st(float* __restrict__ base, unsigned boff, float v) {
    *reinterpret_cast<float*>(reinterpret_cast<char*>(base) + boff) = v;
}
// Streaming (non-temporal) variants for data touched once per call (edge weights in, weight gradients out): they
// do not displace the node rows that the edge loop gathers repeatedly from L2.
__device__ __forceinline__ float mh_ld_nt(const float* __restrict__ base, unsigned boff) {
    return __builtin_nontemporal_load(reinterpret_cast<const float*>(reinterpret_cast<const char*>(base) + boff));
}
__device__ __forceinline__ void mh_st_nt(float* __restrict__ base, unsigned boff, float v) {
    __builtin_nontemporal_store(v, reinterpret_cast<float*>(reinterpret_cast<char*>(base) + boff));
}

// Sum each of NV per-lane values over the 64 lanes of the wave, NV a power of two <= 64.  Transpose reduction: every
// exchange step halves the number of values a lane carries, so the cost is NV-1 + log2(64/NV) shuffles instead of
// 6*NV.  On return every lane L holds the wave total of component (L >> (6 - log2 NV)) in v[0].  The summation
// order is fixed, so results are bitwise reproducible.
// One step exchanges with lane ^ M: N values per lane become N/2 (lanes with bit M set keep the upper half).  The
// recursion is resolved at compile time so every register index is a constant (a runtime index would turn the
// array into compare/select chains).
template <int N, int M, int NV>
struct MhTransposeStep {
    static __device__ __forceinline__ void run(float (&v)[NV], int lane) {
        const bool hi = (lane & M) != 0;
#pragma unroll
        for (int k = 0; k < N / 2; ++k) {
            const float send = hi ? v[k] : v[k + N / 2];
            const float keep = hi ? v[k + N / 2] : v[k];
            v[k] = keep + __shfl_xor(send, M, MH_WAVE);
        }
        MhTransposeStep<N / 2, M / 2, NV>::run(v, lane);
    }
};

template <int M, int NV>
struct MhTransposeStep<1, M, NV> {
    static __device__ __forceinline__ void run(float (&v)[NV], int lane) {
        v[0] += __shfl_xor(v[0], M, MH_WAVE);
        MhTransposeStep<1, M / 2, NV>::run(v, lane);
    }
};

template <int NV>
struct MhTransposeStep<1, 0, NV> {
    static __device__ __forceinline__ void run(float (&)[NV], int) {}
};

template <int NV>
__device__ __forceinline__ float mh_wave_transpose_sum(float (&v)[NV]) {
    static_assert(NV >= 1 && NV <= MH_WAVE && (NV & (NV - 1)) == 0, "NV must be a power of two <= 64");
    MhTransposeStep<NV, MH_WAVE / 2, NV>::run(v, threadIdx.x & (MH_WAVE - 1));
    return v[0];
}
