// W8 G128 LM head (kernels/head/head_i8_tile_consumer.cpp:30-291).
//
// Arithmetic (bit-exact): fp32 H128 of each 128 block, per-128 A8 encoding
// (absmax/127, fp16 scale, round-even, clamp), exact int8 dot per group, then
// acc = acc + RN(sw * RN(sa * dot)) over the 16 groups in ascending order.
// Weights keep the reference's tile layout uint32 [N/16, 128, 4, 16]: the
// (n16 tile, group) block of 512 words (2 KiB) is contiguous.
#include "kernels.hpp"
#include "timing.hpp"
#include "validate.hpp"
#include "../../include/ornith_head.h"

namespace ornith {
namespace {

constexpr int kHeadK = 2048, kHeadGroups = 16;

template <int M> __device__ __forceinline__ void head_step(float& v0, float& v1, int lane) {
    const bool upper = lane & M;
    const float p0 = xor_perm_f<M>(v0), p1 = xor_perm_f<M>(v1);
    v0 = upper ? (p0 - v0) : (v0 + p0);
    v1 = upper ? (p1 - v1) : (v1 + p1);
}

// One wave per (row, 128-group): lane l holds k = 2l, 2l+1.
__global__ __launch_bounds__(256) void head_encode_kernel(const uint16_t* __restrict__ x, int M,
                                                          uint32_t* __restrict__ words, uint16_t* __restrict__ scales,
                                                          uint32_t* sticky) {
    const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (wave >= M * kHeadGroups) return;
    const int lane = threadIdx.x & 63;
    const uint32_t raw = *reinterpret_cast<const uint32_t*>(x + size_t(wave) * 128 + lane * 2);
    float a = bf16_bits_to_f32(raw & 0xffffu), b = bf16_bits_to_f32(raw >> 16);
    uint32_t flags = 0;
    if (!isfinite(a) || !isfinite(b)) flags |= kDenseNonfiniteInput;
    float v0 = a + b, v1 = a - b;                 // butterfly step 1
    head_step<1>(v0, v1, lane);                   // steps 2..64 = lane bits 0..5
    head_step<2>(v0, v1, lane);
    head_step<4>(v0, v1, lane);
    head_step<8>(v0, v1, lane);
    head_step<16>(v0, v1, lane);
    head_step<32>(v0, v1, lane);
    v0 = v0 * kInvSqrt128;
    v1 = v1 * kInvSqrt128;
    if (!isfinite(v0) || !isfinite(v1)) flags |= kDenseNonfiniteInput;
    if (!isfinite(v0)) { flags |= kDenseInvalidActivation; v0 = 0.f; }
    if (!isfinite(v1)) { flags |= kDenseInvalidActivation; v1 = 0.f; }
    const float maximum = wave_max(fmaxf(fabsf(v0), fabsf(v1)));
    const float rawscale = fdiv_rn(maximum, 127.f);
    const bool valid = isfinite(rawscale) && rawscale <= 65504.f;
    if (!valid) flags |= kDenseInvalidActivation;
    const bool zero = maximum == 0.f || !valid;
    const uint16_t sbits = f32_to_f16_bits(zero ? 1.f : fmaxf(rawscale, 0x1p-14f));
    const float scale = f16_bits_to_f32(sbits);
    int q0 = zero ? 0 : __float2int_rn(fdiv_rn(v0, scale));
    int q1 = zero ? 0 : __float2int_rn(fdiv_rn(v1, scale));
    q0 = q0 < -127 ? -127 : (q0 > 127 ? 127 : q0);
    q1 = q1 < -127 ? -127 : (q1 > 127 ? 127 : q1);
    const uint32_t half = (uint32_t(q0) & 255u) | ((uint32_t(q1) & 255u) << 8);
    const uint32_t other = uint32_t(xor_perm_i<1>(int(half)));
    if (!(lane & 1)) words[size_t(wave) * 32 + lane / 2] = half | (other << 16);
    if (lane == 0) scales[wave] = sbits;
    flag_or(sticky, flags);
}

// One block per n16 tile: the 16 group blocks (32 KiB) are staged in LDS,
// thread (group g, column n) forms the integer dot of every row.
template <bool DOTS>
__global__ __launch_bounds__(256) void head_project_kernel(const uint32_t* __restrict__ w,
                                                           const uint16_t* __restrict__ wscale,
                                                           const uint32_t* __restrict__ act,
                                                           const uint16_t* __restrict__ ascale, int M, int N,
                                                           float* __restrict__ diag, uint16_t* __restrict__ out,
                                                           int32_t* __restrict__ group_dots, uint32_t* sticky) {
    __shared__ uint32_t lw[kHeadGroups * 528];    // 512 words + 16 pad per group
    __shared__ uint32_t la[512];
    __shared__ float lterm[kHeadGroups][16];
    const int tid = threadIdx.x, tile = blockIdx.x;
    const uint32_t* src = w + size_t(tile) * (kHeadGroups * 512);
    for (int q = tid; q < kHeadGroups * 128; q += 256) {
        const int g = q >> 7, within = (q & 127) * 4;
        *reinterpret_cast<uint4*>(&lw[g * 528 + within]) = *reinterpret_cast<const uint4*>(src + g * 512 + within);
    }
    const int g = tid >> 4, n = tid & 15;
    const int col = tile * 16 + n;
    const float sw = f16_bits_to_f32(wscale[size_t(col) * kHeadGroups + g]);
    uint32_t flags = 0;
    for (int row = 0; row < M; ++row) {
        __syncthreads();
        for (int q = tid; q < 512; q += 256) la[q] = act[size_t(row) * 512 + q];
        __syncthreads();
        // block word (kword/4 - 8g)*64 + (kword&3)*16 + n, kword = 32g + i
        const uint32_t* wb = &lw[g * 528 + n];
        const uint32_t* ab = &la[g * 32];
        int dot = 0;
#pragma unroll 8
        for (int i = 0; i < 32; ++i) dot = dot4(int(wb[(i >> 2) * 64 + (i & 3) * 16]), int(ab[i]), dot);
        if (DOTS) group_dots[(size_t(row) * N + col) * kHeadGroups + g] = dot;
        const float sa = f16_bits_to_f32(ascale[size_t(row) * kHeadGroups + g]);
        const float scaled = sa * float(dot);
        lterm[g][n] = sw * scaled;
        __syncthreads();
        if (tid < 16) {
            float v = 0.f;
#pragma unroll
            for (int gg = 0; gg < kHeadGroups; ++gg) v = v + lterm[gg][tid];
            const size_t o = size_t(row) * N + tile * 16 + tid;
            const uint16_t b = f32_to_bf16_bits(v);
            if (!isfinite(v)) flags |= kDenseNonfiniteProjection;
            if ((b & 0x7f80u) == 0x7f80u) flags |= kDenseNonfiniteBf16;
            diag[o] = v;
            out[o] = b;
        }
    }
    flag_or(sticky, flags);
}

bool head_shape(int N) { return N == 256 || N == 1024 || N == 4096 || N == 65536 || N == 248320; }

OrnithHeadI8Layout head_layout(int Mcap, int N) {
    OrnithHeadI8Layout l{};
    size_t cursor = 0;
    const size_t m = size_t(Mcap);
    auto add = [&](size_t& field, size_t bytes) { field = cursor; cursor = align256(cursor + bytes); };
    add(l.transformed, 0);
    add(l.activation_words, m * kHeadK);
    add(l.activation_scales, m * kHeadGroups * 2);
    add(l.projection, m * size_t(N) * 4);
    l.workspace_bytes = cursor;
    return l;
}

}  // namespace
}  // namespace ornith

using namespace ornith;

extern "C" uint32_t ornith_head_i8_tile_abi_version(void) { return 1; }

extern "C" hipError_t ornith_head_i8_tile_get_layout(int Mcap, int N, OrnithHeadI8Layout* out) {
    if (!out || Mcap < 0 || Mcap > 64 || !head_shape(N)) return hipErrorInvalidValue;
    *out = head_layout(Mcap, N);
    return hipSuccess;
}

extern "C" hipError_t ornith_head_i8_tile_launch(const void* input, const void* weights, const void* scales,
                                                 void* workspace, size_t workspace_bytes, void* output,
                                                 void* group_dots, size_t group_dots_bytes, void* flags, int M,
                                                 int Mcap, int N, int geometry, hipStream_t stream) {
    OrnithHeadI8Layout l{};
    if (ornith_head_i8_tile_get_layout(Mcap, N, &l) != hipSuccess || M < 0 || M > Mcap || geometry < 0 || geometry > 2)
        return hipErrorInvalidValue;
    if ((group_dots == nullptr) != (group_dots_bytes == 0) ||
        (group_dots && group_dots_bytes < size_t(M) * N * kHeadGroups * 4))
        return hipErrorInvalidValue;
    if (M == 0) return hipSuccess;
    if (workspace_bytes < l.workspace_bytes) return hipErrorInvalidValue;
    // inputs first, then the buffers this call writes (none may overlap another)
    const Buffer buffers[] = {{input, size_t(M) * kHeadK * 2, 4, false, false},
                              {weights, size_t(N) * kHeadK, 16, false, false},
                              {scales, size_t(N) * kHeadGroups * 2, 2, false, false},
                              {workspace, workspace_bytes, 256, true, false},
                              {output, size_t(M) * N * 2, 2, true, false},
                              {group_dots, group_dots_bytes, 4, true, true},
                              {flags, 4, 4, true, false}};
    if (!check_buffers(buffers)) return hipErrorInvalidValue;
    auto sticky = static_cast<uint32_t*>(flags);
    auto words = at<uint32_t>(workspace, l.activation_words);
    auto ascale = at<uint16_t>(workspace, l.activation_scales);
    const int waves = M * kHeadGroups;
    timed_launch("head_encode", head_encode_kernel, dim3((waves + 3) / 4), dim3(256), 0, stream, static_cast<const uint16_t*>(input), M, words, ascale,
                                                            sticky);
    hipError_t st = hipGetLastError();
    if (st != hipSuccess) return st;
    auto diag = at<float>(workspace, l.projection);
    if (group_dots)
        timed_launch("head_project", head_project_kernel<true>, dim3(N / 16), dim3(256), 0, stream,
            static_cast<const uint32_t*>(weights), static_cast<const uint16_t*>(scales), words, ascale, M, N, diag,
            static_cast<uint16_t*>(output), static_cast<int32_t*>(group_dots), sticky);
    else
        timed_launch("head_project", head_project_kernel<false>, dim3(N / 16), dim3(256), 0, stream,
            static_cast<const uint32_t*>(weights), static_cast<const uint16_t*>(scales), words, ascale, M, N, diag,
            static_cast<uint16_t*>(output), nullptr, sticky);
    return hipGetLastError();
}
