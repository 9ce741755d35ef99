// Softmax / top-8 / renormalise of one token on one wave, in the declared
// order (see routing.hip).  Each lane sorts its four probabilities; eight
// rounds then take the wave-wide maximum of the lane heads (fp32 bit
// patterns, all non-negative, so integer order is value order); exact ties
// between lane heads go to the lowest expert id.  The picks come out in
// descending order and are renormalised by their slot-order sum.
#pragma once
#include "common.hpp"

namespace ornith {

__device__ __forceinline__ void cswap(uint32_t& ka, int& ia, uint32_t& kb, int& ib) {
    // keep (ka, ia) ahead of (kb, ib): larger key first, then lower id
    const bool swap = kb > ka || (kb == ka && ib < ia);
    const uint32_t tk = swap ? kb : ka, tk2 = swap ? ka : kb;
    const int ti = swap ? ib : ia, ti2 = swap ? ia : ib;
    ka = tk; kb = tk2; ia = ti; ib = ti2;
}

// v: lane l holds the logits of experts l, l+64, l+128, l+192.  Writes the
// eight weights and ids (identical on every lane).
__device__ __forceinline__ void softmax_top8(const float v[4], float* w_out, int* id_out) {
    const int lane = threadIdx.x & 63;
    const float m = wave_max(fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])));
    float e[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) e[i] = portable_exp(v[i] - m);
    float part = e[0];
#pragma unroll
    for (int i = 1; i < 4; ++i) part = part + e[i];
    const float sum = wave_butterfly_sum(part);
    uint32_t k[4];
    int id[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        k[i] = __float_as_uint(fdiv_rn(e[i], sum));
        id[i] = lane + 64 * i;
    }
    // sorting network for four (key desc, id asc)
    cswap(k[0], id[0], k[1], id[1]);
    cswap(k[2], id[2], k[3], id[3]);
    cswap(k[0], id[0], k[2], id[2]);
    cswap(k[1], id[1], k[3], id[3]);
    cswap(k[1], id[1], k[2], id[2]);
    int head = 0;
    uint32_t pk[kTop];
    int pid[kTop];
#pragma unroll
    for (int j = 0; j < kTop; ++j) {
        const uint32_t hk = head == 0 ? k[0] : head == 1 ? k[1] : head == 2 ? k[2] : head == 3 ? k[3] : 0u;
        const int hid = head == 0 ? id[0] : head == 1 ? id[1] : head == 2 ? id[2] : head == 3 ? id[3] : 0x7fffffff;
        const bool live = head < 4;
        const uint32_t best = wave_max_u(live ? hk : 0u);
        const uint64_t tied = __ballot(live && hk == best);
        int win;
        if (__popcll(tied) == 1) win = __builtin_amdgcn_readlane(hid, __ffsll((long long)tied) - 1);
        else win = wave_min_i((live && hk == best) ? hid : 0x7fffffff);
        pk[j] = best;
        pid[j] = win;
        if (live && hid == win) ++head;
    }
    float tot = 0.f;
#pragma unroll
    for (int j = 0; j < kTop; ++j) tot = tot + __uint_as_float(pk[j]);
#pragma unroll
    for (int j = 0; j < kTop; ++j) { w_out[j] = fdiv_rn(__uint_as_float(pk[j]), tot); id_out[j] = pid[j]; }
}

}  // namespace ornith
