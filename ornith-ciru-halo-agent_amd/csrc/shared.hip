// Shared expert with the reference's fixed8 semantics
// (plugin-site/ornith_g256/iu4_correctness/shared_kernel.py:33-62): the two
// dense A8 projections run through the dense kernels; these two kernels are
// the steps between and after them.
//
//   act[m, c]  = bf16( f32(bf16(silu(g))) * f32(up) ),  g, up = bf16 gate/up
//                outputs, silu from the reference's SiLU table (fp32 SiLU of
//                every bf16 input), i.e. vLLM silu_and_mul's bf16 SiLU then
//                bf16 product;
//   logit[m]   = bf16(x[m] . w_gate) in the library's declared row-dot order
//                (the router's order for the shared gate row);
//   out[m, n]  = bf16( f32(sigmoid_bf16[logit]) * f32(down[m, n]) ).
#include "kernels.hpp"
#include "timing.hpp"

namespace ornith {
namespace {

// Block = one row: 256 threads make the 512 activations; wave 0 also forms
// the gate logit (lane partials over k = 8c .. 8c + 7, c = lane + 64 i, then
// the 64-lane butterfly).
__global__ __launch_bounds__(256) void fixed8_act_kernel(const uint16_t* __restrict__ gu,
                                                         const uint16_t* __restrict__ x,
                                                         const uint16_t* __restrict__ gate_w,
                                                         const float* __restrict__ silu_table,
                                                         uint16_t* __restrict__ act, uint16_t* __restrict__ logit) {
    const int row = blockIdx.x, tid = threadIdx.x;
    const uint16_t* g = gu + size_t(row) * 1024;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int c = tid + 256 * h;
        const uint16_t gb = g[c], ub = g[kInter + c];
        const float s = bf16_round(silu_table[gb]);
        act[size_t(row) * kInter + c] = f32_to_bf16_bits(s * bf16_bits_to_f32(ub));
    }
    if (tid >= 64) return;
    const int lane = tid;
    const uint16_t* xr = x + size_t(row) * kHidden;
    uint4 xv[4], wv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        xv[i] = *reinterpret_cast<const uint4*>(xr + (i * 64 + lane) * 8);
        wv[i] = *reinterpret_cast<const uint4*>(gate_w + (i * 64 + lane) * 8);
    }
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t xw[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
        const uint32_t ww[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            acc = __builtin_fmaf(bf16_bits_to_f32(xw[j] & 0xffffu), bf16_bits_to_f32(ww[j] & 0xffffu), acc);
            acc = __builtin_fmaf(bf16_bits_to_f32(xw[j] >> 16), bf16_bits_to_f32(ww[j] >> 16), acc);
        }
    }
    const float v = wave_butterfly_sum(acc);
    if (lane == 0) logit[row] = f32_to_bf16_bits(v);
}

// out = bf16(sigmoid(logit) * down): eight values per thread.
__global__ __launch_bounds__(256) void fixed8_gate_kernel(const uint16_t* __restrict__ down,
                                                          const uint16_t* __restrict__ logit,
                                                          const uint16_t* __restrict__ sigmoid_table,
                                                          uint16_t* __restrict__ out, size_t chunks,
                                                          uint32_t* sticky) {
    const size_t q = size_t(blockIdx.x) * 256 + threadIdx.x;        // chunk of 8 values
    if (q >= chunks) return;
    const size_t row = q / (kHidden / 8);
    const float gate = bf16_bits_to_f32(sigmoid_table[logit[row]]);
    const uint4 d = reinterpret_cast<const uint4*>(down)[q];
    const uint32_t w[4] = {d.x, d.y, d.z, d.w};
    uint32_t o[4];
    uint32_t flags = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint16_t lo = f32_to_bf16_bits(gate * bf16_bits_to_f32(w[e] & 0xffffu));
        const uint16_t hi = f32_to_bf16_bits(gate * bf16_bits_to_f32(w[e] >> 16));
        if ((lo & 0x7f80u) == 0x7f80u || (hi & 0x7f80u) == 0x7f80u) flags |= kDenseNonfiniteBf16;
        o[e] = uint32_t(lo) | (uint32_t(hi) << 16);
    }
    reinterpret_cast<uint4*>(out)[q] = make_uint4(o[0], o[1], o[2], o[3]);
    flag_or(sticky, flags);
}

}  // namespace

hipError_t launch_fixed8_act(const uint16_t* gu, const uint16_t* x, const uint16_t* gate_w, const float* silu,
                             uint16_t* act, uint16_t* logit, int M, hipStream_t s) {
    if (M <= 0) return hipSuccess;
    timed_launch("fixed8_act", fixed8_act_kernel, dim3(M), dim3(256), 0, s, gu, x, gate_w, silu, act, logit);
    return hipGetLastError();
}

hipError_t launch_fixed8_gate(const uint16_t* down, const uint16_t* logit, const uint16_t* sigmoid, uint16_t* out,
                              int M, uint32_t* sticky, hipStream_t s) {
    if (M <= 0) return hipSuccess;
    const size_t chunks = size_t(M) * (kHidden / 8);
    timed_launch("fixed8_gate", fixed8_gate_kernel, dim3(unsigned((chunks + 255) / 256)), dim3(256), 0, s, down,
                 logit, sigmoid, out, chunks, sticky);
    return hipGetLastError();
}

}  // namespace ornith
