// Activation preparation: 128-point Hadamard transform + group-256
// quantisation into the int8 layout described in common.hpp.
//   act_bf16   - routed gate / dense input (routed_storage_n32_consumer.cpp:22-76,
//                dense_g256_consumer.cpp:27-73, dense_n32 :276-322)
//   act_middle - SiLU(gate)*up, then transform + quantise of the down input
//                (routed_storage_n32_consumer.cpp:168-175, 231-295)
// One wave owns one (row, 256-group); four waves per block.
#include "kernels.hpp"
#include "timing.hpp"
#include "act.hpp"

namespace ornith {

template <int QMAX>
__global__ __launch_bounds__(256) void act_bf16_kernel(const uint16_t* __restrict__ x, int64_t stride, int rows,
                                                       int groups, const int32_t* __restrict__ ids,
                                                       uint32_t* __restrict__ words, uint16_t* __restrict__ scales,
                                                       int32_t* __restrict__ sums, uint32_t* sticky,
                                                       uint32_t flag_input, uint32_t flag_act) {
    act_bf16_block<QMAX>(int(blockIdx.x), x, stride, rows, groups, ids, words, scales, sums, sticky, flag_input,
                         flag_act);
}

template <int QMAX>
__global__ __launch_bounds__(256) void act_middle_kernel(const float* __restrict__ gate_y, int RS, int R,
                                                         const int32_t* __restrict__ ids,
                                                         const float* __restrict__ silu_table,
                                                         uint32_t* __restrict__ words, uint16_t* __restrict__ scales,
                                                         int32_t* __restrict__ sums, uint32_t* sticky) {
    constexpr int groups = kInter / kGroup;
    const int wave = (blockIdx.x * 4) + (threadIdx.x >> 6);
    if (wave >= RS * groups) return;
    const int lane = threadIdx.x & 63;
    const int route = wave / groups, group = wave % groups;
    uint32_t flags = 0;
    const bool shared = route >= R;
    float v[4];
    if (!shared && (ids[route] < 0 || ids[route] >= kExperts)) {
        v[0] = v[1] = v[2] = v[3] = 0.f;
    } else {
        const float4 g = *reinterpret_cast<const float4*>(gate_y + size_t(route) * (2 * kInter) + group * kGroup + lane * 4);
        const float4 u = *reinterpret_cast<const float4*>(gate_y + size_t(route) * (2 * kInter) + kInter + group * kGroup + lane * 4);
        const float gg[4] = {g.x, g.y, g.z, g.w}, uu[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float value;
            if (shared) {
                // Shared rows: tabulated SiLU of the bf16 gate value, product
                // rounded to bf16 (routed_storage_n32_consumer.cpp:246-250).
                const float silu = silu_table[__float_as_uint(gg[i]) >> 16];
                value = bf16_round(silu * uu[i]);
            } else {
                const float silu = silu_portable(gg[i]);
                value = silu * uu[i];
            }
            if (!isfinite(value)) flags |= kFlagNonfiniteMiddle | kFlagNonfiniteInput;
            v[i] = value;
        }
    }
    h128_wave(v);
#pragma unroll
    for (int i = 0; i < 4; ++i) if (!isfinite(v[i])) flags |= kFlagNonfiniteInput;
    quantize_group_wave<QMAX>(v, words + (size_t(route) * groups + group) * 64, scales + size_t(route) * groups + group,
                              sums + size_t(route) * groups + group, flags, kFlagInvalidActivation);
    flag_or(sticky, flags);
}

hipError_t launch_act_bf16(const uint16_t* x, int64_t stride, int rows, int K, int qmax, const int32_t* ids,
                           uint32_t* words, uint16_t* scales, int32_t* sums, uint32_t* sticky,
                           uint32_t flag_input, uint32_t flag_act, hipStream_t s) {
    const int groups = K / kGroup;
    const int waves = (rows * groups + 3) / 4;
    const dim3 grid((waves + 3) / 4), block(256);
    if (qmax == 127)
        timed_launch("act", act_bf16_kernel<127>, dim3(grid), dim3(block), 0, s, x, stride, rows, groups, ids, words, scales, sums, sticky,
                                                     flag_input, flag_act);
    else
        timed_launch("act", act_bf16_kernel<7>, dim3(grid), dim3(block), 0, s, x, stride, rows, groups, ids, words, scales, sums, sticky,
                                                   flag_input, flag_act);
    return hipGetLastError();
}

hipError_t launch_act_middle(const float* gate_y, int RS, int R, const int32_t* ids, int qmax,
                             const float* silu_table, uint32_t* words, uint16_t* scales, int32_t* sums,
                             uint32_t* sticky, hipStream_t s) {
    const int waves = RS * (kInter / kGroup);
    const dim3 grid((waves + 3) / 4), block(256);
    if (qmax == 127)
        timed_launch("act_middle", act_middle_kernel<127>, dim3(grid), dim3(block), 0, s, gate_y, RS, R, ids, silu_table, words, scales, sums, sticky);
    else
        timed_launch("act_middle", act_middle_kernel<7>, dim3(grid), dim3(block), 0, s, gate_y, RS, R, ids, silu_table, words, scales, sums, sticky);
    return hipGetLastError();
}

// ---- dense bf16 prefill operands (dense_g256_consumer.cpp:192-229) ----------
__global__ __launch_bounds__(256) void transform_bf16_kernel(const uint16_t* __restrict__ x, int M, int groups,
                                                             uint16_t* __restrict__ y, uint32_t* sticky) {
    const int wave = (blockIdx.x * 4) + (threadIdx.x >> 6);
    if (wave >= M * groups) return;
    const int lane = threadIdx.x & 63;
    const size_t base = size_t(wave) * kGroup + lane * 4;
    uint32_t flags = 0;
    const uint2 raw = *reinterpret_cast<const uint2*>(x + base);
    float v[4] = {bf16_bits_to_f32(raw.x & 0xffffu), bf16_bits_to_f32(raw.x >> 16),
                  bf16_bits_to_f32(raw.y & 0xffffu), bf16_bits_to_f32(raw.y >> 16)};
#pragma unroll
    for (int i = 0; i < 4; ++i) if (!isfinite(v[i])) flags |= kDenseNonfiniteInput;
    h128_wave(v);
    uint16_t r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (!isfinite(v[i])) flags |= kDenseNonfiniteInput;
        r[i] = f32_to_bf16_bits(v[i]);
        if ((r[i] & 0x7f80u) == 0x7f80u) flags |= kDenseNonfiniteBf16;
    }
    *reinterpret_cast<uint2*>(y + base) = make_uint2(r[0] | (uint32_t(r[1]) << 16), r[2] | (uint32_t(r[3]) << 16));
    flag_or(sticky, flags);
}

// Four packed code words per thread (32 bf16 weights RN(RN(s*code)+off)).
// Threads walk the code words in storage order ([N/tile, K/256, 32, tile]:
// column fastest), four adjacent columns each, so a wave reads one contiguous
// 1 KiB run; each word becomes its column's 16-byte run of eight weights
// (tile / 4 lanes per chunk j, so every row gets 64 / (tile / 4) adjacent
// runs per wave).
__global__ __launch_bounds__(256) void dequantize_bf16_kernel(const uint32_t* __restrict__ codes,
                                                              const uint32_t* __restrict__ meta, int N, int K,
                                                              int tile, uint16_t* __restrict__ w, uint32_t* sticky) {
    const size_t idx = (size_t(blockIdx.x) * 256 + threadIdx.x) * 4;   // first of four words, storage order
    const size_t total = size_t(N) * (K / 8);
    if (idx >= total) return;
    const int groups = K / kGroup;
    const int c = int(idx % tile);                               // columns c .. c+3 of the tile
    const size_t rest = idx / tile;                              // (column tile, group, chunk j)
    const int j = int(rest % 32);
    const size_t tg = rest / 32;                                 // column tile * groups + group
    const int g = int(tg % groups), nt = int(tg / groups);
    const int kw = g * 32 + j;
    // codes and metadata carry 4-byte alignment only (prepare_bf16's contract)
    const uint32_t* cp = codes + idx;
    const uint32_t* mp = meta + tg * tile + c;
    const uint32_t wv[4] = {cp[0], cp[1], cp[2], cp[3]}, mv[4] = {mp[0], mp[1], mp[2], mp[3]};
    uint32_t flags = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float scale = f16_bits_to_f32(mv[e] & 0xffffu), offset = f16_bits_to_f32(mv[e] >> 16);
        uint32_t out[4];
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
            const float a = scale * float((wv[e] >> (4 * i)) & 15u) + offset;
            const float b = scale * float((wv[e] >> (4 * i + 4)) & 15u) + offset;
            const uint16_t ra = f32_to_bf16_bits(a), rb = f32_to_bf16_bits(b);
            if ((ra & 0x7f80u) == 0x7f80u || (rb & 0x7f80u) == 0x7f80u) flags |= kDenseNonfiniteBf16;
            out[i / 2] = ra | (uint32_t(rb) << 16);
        }
        const int n = nt * tile + c + e;
        *reinterpret_cast<uint4*>(w + size_t(n) * K + size_t(kw) * 8) = make_uint4(out[0], out[1], out[2], out[3]);
    }
    flag_or(sticky, flags);
}

hipError_t launch_transform_bf16(const uint16_t* x, int M, int K, uint16_t* y, uint32_t* sticky, hipStream_t s) {
    const int waves = M * (K / kGroup);
    timed_launch("transform", transform_bf16_kernel, dim3((waves + 3) / 4), dim3(256), 0, s, x, M, K / kGroup, y, sticky);
    return hipGetLastError();
}

hipError_t launch_dequantize_bf16(const uint32_t* codes, const uint32_t* meta, int N, int K, int tile, uint16_t* w,
                                  uint32_t* sticky, hipStream_t s) {
    const size_t threads = size_t(N) * (K / 8) / 4;    // tile >= 16: four words never straddle a tile row
    timed_launch("dequantize", dequantize_bf16_kernel, dim3((threads + 255) / 256), dim3(256), 0, s, codes, meta, N, K, tile, w, sticky);
    return hipGetLastError();
}

__global__ void fill_u32_kernel(uint32_t* p, size_t n, uint32_t v) {
    const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

hipError_t launch_fill_u32(uint32_t* p, size_t n, uint32_t v, hipStream_t s) {
    if (!n) return hipSuccess;
    timed_launch("fill", fill_u32_kernel, dim3((n + 255) / 256), dim3(256), 0, s, p, n, v);
    return hipGetLastError();
}

}  // namespace ornith
