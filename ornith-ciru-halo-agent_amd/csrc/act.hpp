// Activation preparation of bf16 rows (H128 + group-256 quantisation), as a
// per-block device function shared by act.hip and the fused router launch.
#pragma once
#include "common.hpp"

namespace ornith {

// Quarter-wave groups (common.hpp): each 16-lane quarter owns one 256-group,
// lane l holding its 16 values k = quarter_base(l) + i; four groups per wave
// (flattened (row, group) index 4 * wave + quarter).
// Block `block` of the grid (four waves); also run by trailing blocks of the
// permutation's bank-scan launch (routing.hip).
template <int QMAX>
__device__ __forceinline__ void act_bf16_block(int block, const uint16_t* __restrict__ x, int64_t stride, int rows,
                                               int groups, const int32_t* __restrict__ ids,
                                               uint32_t* __restrict__ words, uint16_t* __restrict__ scales,
                                               int32_t* __restrict__ sums, uint32_t* sticky, uint32_t flag_input,
                                               uint32_t flag_act) {
    const int wave = (block * 4) + ((threadIdx.x >> 6) & 3);     // 4 waves per block index
    const int lane = threadIdx.x & 63, l = lane & 15;
    const int total = rows * groups;
    const int g = 4 * wave + (lane >> 4);
    if (4 * wave >= total) return;
    // groups past the end repeat the last one (loaded, never written)
    const int gl = min(g, total - 1);
    const int row = gl / groups, group = gl - row * groups, k0 = quarter_base(l);
    const uint16_t* src = x + row * stride + group * kGroup + k0;
    const uint4 r0 = *reinterpret_cast<const uint4*>(src), r1 = *reinterpret_cast<const uint4*>(src + 8);
    bool live = true;
    if (ids) {
        live = false;
#pragma unroll
        for (int s = 0; s < kTop; ++s) {
            const int id = ids[row * kTop + s];
            live |= id >= 0 && id < kExperts;
        }
    }
    float v[16];
    const uint32_t u[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        v[2 * e] = bf16_bits_to_f32(u[e] & 0xffffu);
        v[2 * e + 1] = bf16_bits_to_f32(u[e] >> 16);
    }
    uint32_t flags = 0;
    if (live) {
#pragma unroll
        for (int e = 0; e < 16; ++e) if (!isfinite(v[e])) flags |= flag_input;
        h128_quarter(v);
    } else {
#pragma unroll
        for (int e = 0; e < 16; ++e) v[e] = 0.f;
    }
    uint32_t w4[4];
    uint16_t sbits;
    int sum;
    // a non-finite transformed value raises both flags (as the separate check
    // and the quantiser's own did)
    quantize_quarter_fast<QMAX>(v, w4, sbits, sum, flags, flag_input | flag_act, flag_act);
    if (g < total) {
        *reinterpret_cast<uint4*>(words + size_t(g) * 64 + k0 / 4) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
        if (l == 0) { scales[g] = sbits; sums[g] = sum; }
    } else {
        flags = 0;
    }
    flag_or(sticky, flags);
}

}  // namespace ornith
