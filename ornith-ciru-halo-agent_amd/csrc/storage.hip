// One-time storage conversion: N16 tile banks -> N32 tile banks.
//
// The checkpoint stores 4-bit codes as [N/16, K/256, 32, 16] uint32 words and
// metadata as [N/16, K/256, 16] per bank; the N32 consumers read
// [N/32, K/256, 32, 32] and [N/32, K/256, 32], where 32-column tile t is the
// pair of 16-column tiles 2t (columns 0..15) and 2t+1 (columns 16..31)
// (plugin-site/ornith_g256/method.py:143-147, dense_n32.py:32-33).
// Every output row of 32 words is two 64-byte input rows; one thread moves 16
// bytes.
#include "kernels.hpp"
#include "timing.hpp"
#include "validate.hpp"
#include "../../include/ornith_storage.h"

namespace ornith {
namespace {

// codes: out word ((b * T32 + t) * G + g) * 1024 + j * 32 + n, n = 16 h + c,
// from in word ((b * 2 T32 + 2 t + h) * G + g) * 512 + j * 16 + c.
__global__ __launch_bounds__(256) void repack_codes_kernel(const uint4* __restrict__ in, uint4* __restrict__ out,
                                                           size_t quads, int G) {
    const size_t q = size_t(blockIdx.x) * 256 + threadIdx.x;     // output uint4 index
    if (q >= quads) return;
    const size_t w = q * 4;                                       // first output word
    const int n = int(w & 31), j = int((w >> 5) & 31);
    const size_t tg = w >> 10;                                    // (b * T32 + t) * G + g
    const size_t g = tg % size_t(G), bt = tg / size_t(G);         // b * T32 + t
    const int h = n >> 4, c = n & 15;
    const size_t src = (((2 * bt + size_t(h)) * G + g) * 512) + size_t(j) * 16 + size_t(c);
    out[q] = in[src / 4];
}

// meta: out word ((b * T32 + t) * G + g) * 32 + n from in word
// ((b * 2 T32 + 2 t + h) * G + g) * 16 + c.
__global__ __launch_bounds__(256) void repack_meta_kernel(const uint4* __restrict__ in, uint4* __restrict__ out,
                                                          size_t quads, int G) {
    const size_t q = size_t(blockIdx.x) * 256 + threadIdx.x;
    if (q >= quads) return;
    const size_t w = q * 4;
    const int n = int(w & 31);
    const size_t tg = w >> 5;
    const size_t g = tg % size_t(G), bt = tg / size_t(G);
    const int h = n >> 4, c = n & 15;
    const size_t src = ((2 * bt + size_t(h)) * G + g) * 16 + size_t(c);
    out[q] = in[src / 4];
}

}  // namespace
}  // namespace ornith

using namespace ornith;

extern "C" hipError_t ornith_repack_n16_to_n32(const void* codes16, const void* meta16, void* codes32, void* meta32,
                                               int banks, int N, int K, hipStream_t stream) {
    if (banks < 0 || N < 0 || K < 0 || N % 32 || K % kGroup) return hipErrorInvalidValue;
    if (!banks || !N || !K) return hipSuccess;
    const size_t code_bytes = size_t(banks) * N * (K / 2), meta_bytes = size_t(banks) * N * (K / kGroup) * 4;
    const Buffer buffers[] = {{codes16, code_bytes, 16, false, false},
                              {meta16, meta_bytes, 16, false, false},
                              {codes32, code_bytes, 16, true, false},
                              {meta32, meta_bytes, 16, true, false}};
    if (!check_buffers(buffers)) return hipErrorInvalidValue;
    const int G = K / kGroup;
    const size_t cq = code_bytes / 16, mq = meta_bytes / 16;
    timed_launch("repack_codes", repack_codes_kernel, dim3(unsigned((cq + 255) / 256)), dim3(256), 0, stream,
                 static_cast<const uint4*>(codes16), static_cast<uint4*>(codes32), cq, G);
    hipError_t st = hipGetLastError();
    if (st != hipSuccess) return st;
    timed_launch("repack_meta", repack_meta_kernel, dim3(unsigned((mq + 255) / 256)), dim3(256), 0, stream,
                 static_cast<const uint4*>(meta16), static_cast<uint4*>(meta32), mq, G);
    return hipGetLastError();
}
