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

// index of the k-th set bit (k from 0) of a wave-uniform mask
__device__ __forceinline__ int mh_kth_bit(unsigned m, int k) {
  for (; k > 0; --k) m &= m - 1u;
  return __builtin_ctz(m);
}

// Exclusive prefix sum of v over the workgroup (NW waves of 64, every thread calling), in a fixed order: an inclusive
// scan inside each wave by shuffles, then the wave totals (through LDS `wsum`, NW entries) added in wave order.
// `total` receives the workgroup's sum.  Two barriers; `wsum` may be reused after the call.
template <typename T, int NW>
__device__ __forceinline__ T mh_block_excl_scan(T v, T& total, T* wsum) {
    const int lane = threadIdx.x & (MH_WAVE - 1), wave = threadIdx.x >> 6;
    T inc = v;
#pragma unroll
    for (int off = 1; off < MH_WAVE; off <<= 1) {
        const T t = __shfl_up(inc, off, MH_WAVE);
        if (lane >= off) inc += t;
    }
    if (lane == MH_WAVE - 1) wsum[wave] = inc;
    __syncthreads();
    T before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        const T sw = wsum[w];
        before += w < wave ? sw : T(0);
        all += sw;
    }
    __syncthreads();
    total = all;
    return before + inc - v;
}

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

// fp32 at fp32 accuracy on the bf16 matrix cores: a float splits exactly into three bf16 parts v = hi + mid + lo
// (truncation at every step: hi keeps the top 8 significant bits, mid the next 8, lo the last 8), and a product
// a·b is then the sum of the six partial products hi·hi, hi·mid, mid·hi, hi·lo, mid·mid, lo·hi up to terms below
// 2^-24 of |a·b| — as accurate as an fp32 multiply.  mh_split8 splits eight floats into the three bf16x8 MFMA
// operands (v_mfma_f32_16x16x32_bf16 takes eight K values per lane).
typedef float mh_f4 __attribute__((ext_vector_type(4)));
typedef __bf16 mh_bf8 __attribute__((ext_vector_type(8)));
typedef unsigned int mh_u4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void mh_split8(const float (&v)[8], mh_bf8 (&s)[3]) {
    unsigned p[3][4];
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
        unsigned b[2][3];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const unsigned hb = __float_as_uint(v[j + e]) & 0xFFFF0000u;
            const float r1 = v[j + e] - __uint_as_float(hb);
            const unsigned mb = __float_as_uint(r1) & 0xFFFF0000u;
            const float r2 = r1 - __uint_as_float(mb);
            b[e][0] = hb >> 16;
            b[e][1] = mb >> 16;
            b[e][2] = __float_as_uint(r2) >> 16;
        }
#pragma unroll
        for (int k = 0; k < 3; ++k) p[k][j / 2] = b[0][k] | (b[1][k] << 16);
    }
#pragma unroll
    for (int k = 0; k < 3; ++k) s[k] = __builtin_bit_cast(mh_bf8, mh_u4{p[k][0], p[k][1], p[k][2], p[k][3]});
}
