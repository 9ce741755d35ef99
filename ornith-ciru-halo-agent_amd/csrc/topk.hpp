// Softmax / top-8 / renormalise of one token on one wave, in the declared
// order (see routing.hip).  Each lane sorts its four probabilities; eight
// rounds then take the wave-wide maximum of the lane heads (fp32 bit
// patterns, all non-negative, so integer order is value order); exact ties
// between lane heads go to the lowest expert id.  The picks come out in
// descending order and are renormalised by their slot-order sum.
// top8_rank_lds makes the same picks with a threshold and a rank count (for
// kernels where the selection latency is on the critical path).
#pragma once
#include "common.hpp"
#include "handoff.hpp"

namespace ornith {

__device__ __forceinline__ void cswap(uint32_t& ka, int& ia, uint32_t& kb, int& ib) {
    // keep (ka, ia) ahead of (kb, ib): larger key first, then lower id
    const bool swap = kb > ka || (kb == ka && ib < ia);
    const uint32_t tk = swap ? kb : ka, tk2 = swap ? ka : kb;
    const int ti = swap ? ib : ia, ti2 = swap ? ia : ib;
    ka = tk; kb = tk2; ia = ti; ib = ti2;
}

// Router logits of one router row for up to 8 consecutive tokens t0.. on one
// wave, in the declared order (routing.hip): lane l forms the fma chain over
// chunks l, l+64, l+128, l+192, then the butterfly; + bias.  Every token row
// is loaded before the first fma (rows past T repeat the last token and are
// not written), so the loads overlap.  With `words`, token t0 + t's logit is
// also published as tagged word word0 + t (handoff.hpp), by lane t.
__device__ __forceinline__ void router_rows_wave(const uint16_t* __restrict__ x, int64_t stride, int T, int t0,
                                                 const uint16_t* __restrict__ wrow, float bias, bool has_bias,
                                                 float* __restrict__ logits, int64_t logit_stride, int row,
                                                 uint64_t* words = nullptr, uint32_t seq = 0, uint32_t word0 = 0) {
    constexpr int kBatch = 8;
    const int lane = threadIdx.x & 63, nt = min(kBatch, T - t0);
    uint4 wv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) wv[i] = *reinterpret_cast<const uint4*>(wrow + (i * 64 + lane) * 8);
    u32x4 xv[kBatch][4];
#pragma unroll
    for (int t = 0; t < kBatch; ++t) {
        const uint16_t* xrow = x + size_t(min(t0 + t, T - 1)) * stride;
#pragma unroll
        for (int i = 0; i < 4; ++i) xv[t][i] = *reinterpret_cast<const u32x4*>(xrow + (i * 64 + lane) * 8);
    }
    float acc[kBatch];
#pragma unroll
    for (int t = 0; t < kBatch; ++t) {
        acc[t] = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t ww[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t xw = xv[t][i][j];
                acc[t] = __builtin_fmaf(bf16_bits_to_f32(xw & 0xffffu), bf16_bits_to_f32(ww[j] & 0xffffu), acc[t]);
                acc[t] = __builtin_fmaf(bf16_bits_to_f32(xw >> 16), bf16_bits_to_f32(ww[j] >> 16), acc[t]);
            }
        }
    }
    float pub = 0.f;
#pragma unroll
    for (int t = 0; t < kBatch; ++t) {
        if (t < nt) {
            float v = wave_butterfly_sum(acc[t]);
            if (has_bias) v = v + bias;
            if (lane == 0) logits[size_t(t0 + t) * logit_stride + row] = v;
            if (lane == t) pub = v;
        }
    }
    if (words) {
        // the call's sequence number is taken only now: its load was issued
        // before the rows', and converting it earlier made the compiler wait
        // for it before issuing them
        asm volatile("" : "+v"(seq));
        const uint32_t sq = __builtin_amdgcn_readfirstlane(seq);
        if (lane < nt) l1_put(words, word0 + lane, sq, __float_as_uint(pub));
    }
}

// Order key of an fp32 value: unsigned order of keys = numeric order of the
// values (-0 and +0 differ; NaNs sort beyond the infinities by sign).
__device__ __forceinline__ uint32_t f32_order_key(float v) {
    const uint32_t b = __float_as_uint(v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Softmax probabilities of one token as order keys: lane l holds experts l,
// l+64, l+128, l+192; k[i] is the fp32 bit pattern of the probability (all
// non-negative, so integer order is value order).
__device__ __forceinline__ void softmax_keys(const float v[4], uint32_t k[4]) {
    const float m = wave_max(fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])));
    float e[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) e[i] = portable_exp(v[i] - m);
    float part = e[0];
#pragma unroll
    for (int i = 1; i < 4; ++i) part = part + e[i];
    const float sum = wave_butterfly_sum(part);
#pragma unroll
    for (int i = 0; i < 4; ++i) k[i] = __float_as_uint(fdiv_rn(e[i], sum));
}

// Top-8 of the keys by eight wave-wide rounds.  Each lane sorts its four
// (key desc, id asc); eight rounds then take the wave-wide maximum of the lane
// heads, exact ties between lane heads going to the lowest expert id.  pk/pid
// come out in descending order, identical on every lane.
__device__ __forceinline__ void top8_rounds(const uint32_t keys[4], uint32_t pk[kTop], int pid[kTop]) {
    const int lane = threadIdx.x & 63;
    uint32_t k[4];
    int id[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        k[i] = keys[i];
        id[i] = lane + 64 * i;
    }
    // sorting network for four (key desc, id asc)
    cswap(k[0], id[0], k[1], id[1]);
    cswap(k[2], id[2], k[3], id[3]);
    cswap(k[0], id[0], k[2], id[2]);
    cswap(k[1], id[1], k[3], id[3]);
    cswap(k[1], id[1], k[2], id[2]);
    // Each lane's four form a queue: the head is k[0]/id[0]; a pop shifts the
    // rest up and appends the sentinel id 0x7fffffff (a lane is exhausted
    // when its head id is the sentinel).  All selects, no lane branches.
    constexpr int kNone = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < kTop; ++j) {
        const bool live = id[0] != kNone;
        const uint32_t best = wave_max_u(live ? k[0] : 0u);
        const bool cand = live && k[0] == best;
        const uint64_t tied = __ballot(cand);
        int win;
        if (__popcll(tied) == 1) win = __builtin_amdgcn_readlane(id[0], __ffsll((long long)tied) - 1);
        else win = wave_min_i(cand ? id[0] : kNone);
        pk[j] = best;
        pid[j] = win;
        const bool pop = cand && id[0] == win;
        k[0] = pop ? k[1] : k[0];
        k[1] = pop ? k[2] : k[1];
        k[2] = pop ? k[3] : k[2];
        k[3] = pop ? 0u : k[3];
        id[0] = pop ? id[1] : id[0];
        id[1] = pop ? id[2] : id[1];
        id[2] = pop ? id[3] : id[2];
        id[3] = pop ? kNone : id[3];
    }
}

// v: lane l holds the logits of experts l, l+64, l+128, l+192.  Returns the
// eight selected ids (identical on every lane) in pid, and on lane j < 8 the
// weight and id of slot j (the renormalisation runs lane-parallel).
__device__ __forceinline__ void softmax_top8(const float v[4], float& w_lane, int& id_lane, int pid[kTop]) {
    const int lane = threadIdx.x & 63;
    uint32_t k[4], pk[kTop];
    softmax_keys(v, k);
    top8_rounds(k, pk, pid);
    float tot = 0.f;
#pragma unroll
    for (int j = 0; j < kTop; ++j) tot = tot + __uint_as_float(pk[j]);
    uint32_t mk = pk[0];
    int mi = pid[0];
#pragma unroll
    for (int j = 1; j < kTop; ++j)
        if (lane == j) { mk = pk[j]; mi = pid[j]; }
    w_lane = fdiv_rn(__uint_as_float(mk), tot);
    id_lane = mi;
}

// Top-8 of the keys by a threshold and a rank count, on one wave:
//  1. Threshold t: the largest quad maximum (quad = 4 lanes, 16 keys) that
//     at least eight quad maxima reach.  Those eight belong to distinct
//     experts, so every key below t is beaten by eight keys and the top
//     eight lie among the candidates {key >= t} (t itself is a key; about
//     ten candidates for router-like logits).
//  2. The candidates are compacted into LDS as (key << 32 | ~id); candidate c
//     (lane c) counts the candidates ahead of it in (key desc, id asc) order
//     -- one 64-bit compare each -- and ranks 0..7 write themselves to
//     sel[rank].
// More than 64 candidates (many equal keys) take top8_rounds instead; both
// give the same picks.  cand: 65 entries of LDS (the last one takes the
// writes of non-candidates), 16-byte aligned; sel: 8.  sel[r] = {key bits,
// id}; visible to the wave when this returns.
__device__ __forceinline__ void top8_rank_lds(const uint32_t k[4], uint64_t* cand, uint2* sel) {
    const int lane = threadIdx.x & 63;
    uint32_t q = max(max(k[0], k[1]), max(k[2], k[3]));
    q = max(q, uint32_t(dpp_i<kDppXor1>(int(q))));
    q = max(q, uint32_t(dpp_i<kDppXor2>(int(q))));           // the quad's maximum
    int ge = 0;                                               // quad maxima >= this quad's
#pragma unroll
    for (int j = 0; j < 16; ++j) ge += uint32_t(__builtin_amdgcn_readlane(int(q), 4 * j)) >= q ? 1 : 0;
    const uint32_t t = wave_max_u(ge >= kTop ? q : 0u);
    uint64_t b[4];
    int base[4], C = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        b[i] = __ballot(k[i] >= t);
        base[i] = C;
        C += __popcll(b[i]);
    }
    if (C <= 64) {
        // zero padding (a zero entry is ahead of no candidate: every candidate
        // has ~id > 0), then the candidates; others write entry 64
        cand[lane] = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int pos = base[i] + int(__builtin_amdgcn_mbcnt_hi(uint32_t(b[i] >> 32),
                                                                    __builtin_amdgcn_mbcnt_lo(uint32_t(b[i]), 0u)));
            cand[k[i] >= t ? pos : 64] = (uint64_t(k[i]) << 32) | ~uint32_t(lane + 64 * i);
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        const uint64_t me = cand[lane];
        int rank = 0;
        for (int j = 0; j < C; j += 16) {
            const ulonglong2* p = reinterpret_cast<const ulonglong2*>(cand + j);
            ulonglong2 e[8];
#pragma unroll
            for (int r = 0; r < 8; ++r) e[r] = p[r];
#pragma unroll
            for (int r = 0; r < 8; ++r) rank += (e[r].x > me ? 1 : 0) + (e[r].y > me ? 1 : 0);
        }
        if (lane < C && rank < kTop) sel[rank] = make_uint2(uint32_t(me >> 32), ~uint32_t(me));
    } else {
        uint32_t pk[kTop];
        int pid[kTop];
        top8_rounds(k, pk, pid);
        uint32_t mk = pk[0];
        int mi = pid[0];
#pragma unroll
        for (int j = 1; j < kTop; ++j)
            if (lane == j) { mk = pk[j]; mi = pid[j]; }
        if (lane < kTop) sel[lane] = make_uint2(mk, uint32_t(mi));
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

}  // namespace ornith
