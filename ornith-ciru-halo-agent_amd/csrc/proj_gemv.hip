// Grouped G256 projection for small row counts (decode GEMV path).
//
// Arithmetic: routed_storage_n32_consumer.cpp:124-161 (projection_n32_job) and
// dense_g256_consumer.cpp:116-143 (compact_projection): per output column an
// exact integer dot per 256-group, then the fp32 group tree in ascending
// group order.  The dot uses v_dot4_i32_i8 on the int8 activation layout and
// codes split into even/odd bytes (common.hpp).
//
// Work split: one block (4 waves) owns one segment (one weight bank and its
// routes) and NT consecutive 32-column tiles.  The block stages the code
// blocks of GC groups (NT*GC <= 8 blocks of 4 KiB) into LDS with 128-bit
// coalesced loads, then every thread computes one (tile, group, column)
// integer dot for each route; the group tree runs in a second pass.
#include "kernels.hpp"
#include "timing.hpp"

namespace ornith {

constexpr int kPad = 1056;          // LDS words per (tile, group) block: 32x32 + 32 (bank spread)
constexpr int kRouteBatch = 16;     // routes whose running sums are kept in LDS

template <int TILE, Out MODE>
__global__ __launch_bounds__(256) void project_gemv_kernel(ProjArgs a, int NT, int GC) {
    __shared__ uint32_t lw[8 * kPad];
    __shared__ uint32_t lm[8 * 32];
    __shared__ uint32_t la[8 * 64];
    __shared__ float lsa[8], lss[8];
    __shared__ float lterm[8][32];
    __shared__ float lrun[kRouteBatch][256];
    __shared__ int lrow[kRouteBatch], lroute[kRouteBatch];

    const int tid = threadIdx.x;
    if (a.nseg && int(blockIdx.x) >= *a.nseg) return;
    const Segment sg = a.segments ? a.segments[blockIdx.x] : Segment{0, 0, a.dense_rows, 0};
    const bool shared = sg.bank == kShared;
    const uint32_t* codes = shared ? a.shared_codes : a.codes + size_t(sg.bank) * a.bank_words;
    const uint32_t* meta = shared ? a.shared_meta : a.meta + size_t(sg.bank) * a.bank_meta_words;
    const int GS = a.K / kGroup;
    const int ntiles = (a.N + 31) / 32;
    const int tile0 = blockIdx.y * NT;
    const int pairs = NT * GC * 32;
    const int cols = NT * 32;

    for (int rb = 0; rb < sg.count; rb += kRouteBatch) {
        const int nr = min(kRouteBatch, sg.count - rb);
        if (tid < nr) {
            const int route = a.routes ? a.routes[sg.first + rb + tid] : rb + tid;
            lroute[tid] = route;
            lrow[tid] = a.row_mode == 0 ? route : (route < a.R ? route / kTop : route - a.R);
        }
        for (int g0 = 0; g0 < GS; g0 += GC) {
            const int gc = min(GC, GS - g0);
            __syncthreads();
            // ---- stage code blocks (tile tl, group gl) and metadata ----
            for (int q = tid; q < NT * gc * 256; q += 256) {
                const int blk = q >> 8, within = (q & 255) * 4;     // word offset inside 1024-word block
                const int tl = blk / gc, gl = blk % gc;
                const int t = tile0 + tl, g = g0 + gl;
                uint4 v = make_uint4(0, 0, 0, 0);
                if (t < ntiles) {
                    if (TILE == 32) {
                        v = *reinterpret_cast<const uint4*>(codes + ((size_t(t) * GS + g) * 32) * 32 + within);
                    } else {
                        const int j = within >> 5, n32 = within & 31, h = n32 >> 4, n16 = n32 & 15;
                        if ((2 * t + h) * 16 < a.N)
                            v = *reinterpret_cast<const uint4*>(codes + ((size_t(2 * t + h) * GS + g) * 32 + j) * 16 + n16);
                    }
                }
                *reinterpret_cast<uint4*>(&lw[(tl * gc + gl) * kPad + within]) = v;
            }
            for (int q = tid; q < NT * gc * 32; q += 256) {
                const int blk = q >> 5, n = q & 31, tl = blk / gc, gl = blk % gc;
                const int t = tile0 + tl, g = g0 + gl, col = t * 32 + n;
                uint32_t m = 0;
                if (col < a.N) {
                    if (TILE == 32) m = meta[(size_t(t) * GS + g) * 32 + n];
                    else m = meta[(size_t(col / 16) * GS + g) * 16 + (col & 15)];
                }
                lm[blk * 32 + n] = m;
            }
            for (int r = 0; r < nr; ++r) {
                const int row = lrow[r];
                // ---- stage this route's activation words for the chunk ----
                for (int q = tid; q < gc * 64; q += 256)
                    la[q] = a.act_words[size_t(row) * (a.K / 4) + size_t(g0) * 64 + q];
                if (tid < gc) {
                    const float sa = f16_bits_to_f32(a.act_scales[size_t(row) * GS + g0 + tid]);
                    lsa[tid] = sa;
                    lss[tid] = sa * float(a.act_sums[size_t(row) * GS + g0 + tid]);
                }
                __syncthreads();
                if (tid < NT * gc * 32) {
                    const int blk = tid >> 5, n = tid & 31, gl = blk % gc;
                    const uint32_t* wb = &lw[blk * kPad + n];
                    const uint32_t* ab = &la[gl * 64];
                    int dot = 0;
#pragma unroll 8
                    for (int c = 0; c < 32; ++c) {
                        const uint32_t w = wb[c * 32];
                        dot = dot4(code_even(w), int(ab[2 * c]), dot);
                        dot = dot4(code_odd(w), int(ab[2 * c + 1]), dot);
                    }
                    lterm[blk][n] = tree_term(dot, lsa[gl], lss[gl], lm[blk * 32 + n]);
                }
                __syncthreads();
                if (tid < cols) {
                    const int tl = tid >> 5, n = tid & 31;
                    float v = g0 == 0 ? 0.f : lrun[r][tid];
                    for (int gl = 0; gl < gc; ++gl) v = v + lterm[tl * gc + gl][n];
                    lrun[r][tid] = v;
                }
            }
        }
        __syncthreads();
        // ---- write the finished rows ----
        for (int q = tid; q < nr * cols; q += 256) {
            const int r = q / cols, cidx = q % cols;
            const int col = tile0 * 32 + cidx;
            if (col >= a.N) continue;
            float v = lrun[r][cidx];
            if (MODE == Out::Routed) {
                if (shared) v = bf16_round(v);   // shared linear outputs are bf16 (:226-227)
                a.out[size_t(lroute[r]) * a.N + col] = v;
                if (!isfinite(v)) atomicOr(a.sticky, a.flag_projection);
            } else {
                const size_t o = size_t(lroute[r]) * a.N + col;
                const uint16_t b = f32_to_bf16_bits(v);
                uint32_t f = 0;
                if (!isfinite(v)) f |= a.flag_projection;
                if ((b & 0x7f80u) == 0x7f80u) f |= a.flag_bf16;
                if (a.out) a.out[o] = v;
                if (a.out_bf16) a.out_bf16[o] = b;
                flag_or(a.sticky, f);
            }
        }
        __syncthreads();
    }
}

hipError_t launch_project_gemv(const ProjArgs& a, int max_segments, Out mode, hipStream_t s) {
    const int GS = a.K / kGroup;
    const int GC = GS < 8 ? GS : 8;
    const int NT = 8 / GC;
    const int ntiles = (a.N + 31) / 32;
    const dim3 grid(max_segments, (ntiles + NT - 1) / NT);
    if (max_segments <= 0) return hipSuccess;
    if (a.tile == 32) {
        if (mode == Out::Routed) timed_launch("dense_gemv", project_gemv_kernel<32, Out::Routed>, dim3(grid), dim3(256), 0, s, a, NT, GC);
        else timed_launch("dense_gemv", project_gemv_kernel<32, Out::Dense>, dim3(grid), dim3(256), 0, s, a, NT, GC);
    } else {
        if (mode == Out::Routed) timed_launch("dense_gemv", project_gemv_kernel<16, Out::Routed>, dim3(grid), dim3(256), 0, s, a, NT, GC);
        else timed_launch("dense_gemv", project_gemv_kernel<16, Out::Dense>, dim3(grid), dim3(256), 0, s, a, NT, GC);
    }
    return hipGetLastError();
}

}  // namespace ornith
