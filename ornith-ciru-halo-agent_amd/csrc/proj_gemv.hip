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
#include "act.hpp"

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

// Dense weight-streaming projection for up to kStreamRows rows (decode and
// small batches).  One block of 4 waves owns COLS (32, or 16 on tile-16
// banks above kDenseNarrowRows rows) consecutive output columns;
// half-wave h of the block owns group g0 + h of the current 8-group pass.
// Each lane keeps its 32 code words of that group in registers (every load of
// the block is issued before the first dot), so one pass over the bank moves
// the whole weight through HBM once however many rows there are.
//   tile 32: lane L holds column L, words j*32 + L of block (tile, g).
//   tile 16: lane L = 16*jp + n holds words (2i+jp)*16 + n (i < 16) of the two
//            16-column blocks of the 32-column unit; the two half-dots of a
//            column meet across lanes L and L^16, after which lane L keeps
//            column L of the unit.  With 16 columns a lane holds the words
//            of its one block and lanes L, L^16 both end with column n.
// FUSED (a.dense_x set, up to kDenseFusedRows rows): the block also prepares
// its activations from the bf16 input: the H128 +
// group-256 int8 recipe of act_bf16_block, 16 lanes per (row, group), written
// to LDS instead of the workspace.  Every block repeats this small amount of
// work; the first chunk's inputs are loaded before the code words, so it runs
// while the weights are in flight and the separate activation launch goes.
// Otherwise the activations come from the workspace (act_words/scales/sums).
// Terms go through LDS; one thread per (row, column) adds them in group order
// (the fp32 tree of dense_g256_consumer.cpp:116-143), so results equal
// project_gemv_kernel's bit for bit.
constexpr int kStreamRows = kDenseStreamRows;   // rows whose running sums stay in LDS
constexpr int kStreamChunk = 8;     // rows per term pass (8 rows x 32 columns = 256 threads)
// Tile-16 banks above this many rows (the activations read from the
// workspace) run 16-column blocks: twice the blocks, each lane streaming one
// 16-column tile.  One-row-per-block latency favours 32 columns below it
// (graph-timed per call, 16 against 32 columns: 1 row 6.0 / 5.55 us, 8 rows
// 15.8 / 12.6, 16 rows 15.8 / 16.1, 32 rows 24.5 / 25.6, 64 rows 40.9 / 44.1).
constexpr int kDenseNarrowRows = 16;

template <int TILE, bool FUSED, int COLS = 32>
__global__ __launch_bounds__(256) void dense_stream_kernel(ProjArgs a) {
    static_assert(COLS == 32 || TILE == 16, "16-column blocks read the N16 layout");
    __shared__ uint32_t la[kStreamChunk][8 * 64];
    __shared__ float lsa[kStreamChunk][8], lss[kStreamChunk][8];
    __shared__ float lterm[kStreamChunk][8][32];
    __shared__ float lrun[kStreamRows][32];

    const int tid = threadIdx.x, hw = tid >> 5, L = tid & 31, jp = L >> 4, n16 = L & 15;
    const int GS = a.K / kGroup, M = a.dense_rows;
    const int col0 = blockIdx.x * COLS, col = col0 + (COLS == 16 ? n16 : L);
    for (int g0 = 0; g0 < GS; g0 += 8) {
        const int g = g0 + hw, gc = min(8, GS - g0);
        const bool gv = g < GS;
        // Loads are unconditional (a predicated load would drain the queue):
        // a half-wave past the last group reads group GS-1 and writes no term;
        // a missing second 16-column block reads the first one, whose dots
        // only reach columns >= N, which are never written.
        const int gq = gv ? g : GS - 1;
        // input words of the first chunk's first pair pass (fused activations)
        auto xsrc = [&](int r0, int nr, int p0) {
            const int pc = min(p0 + (tid >> 4), nr * gc - 1);
            return a.dense_x + size_t(r0 + pc / gc) * a.K + (g0 + pc % gc) * kGroup + quarter_base(tid & 15);
        };
        uint4 px0 = make_uint4(0, 0, 0, 0), px1 = px0;
        if constexpr (FUSED) {
            const uint16_t* xp0 = xsrc(0, min(kStreamChunk, M), 0);
            px0 = *reinterpret_cast<const uint4*>(xp0);
            px1 = *reinterpret_cast<const uint4*>(xp0 + 8);
        }
        uint32_t wr[32];
        uint32_t mw;
        if (TILE == 32) {
            const uint32_t* wp = a.codes + (size_t(blockIdx.x) * GS + gq) * 1024 + L;
#pragma unroll
            for (int j = 0; j < 32; ++j) wr[j] = load_once(wp + j * 32);
            mw = a.meta[(size_t(blockIdx.x) * GS + gq) * 32 + L];
        } else {
            const int tA = COLS == 16 ? int(blockIdx.x) : 2 * int(blockIdx.x);
            const int tB = (tA + 1) * 16 < a.N ? tA + 1 : tA;
            const uint32_t* pa = a.codes + (size_t(tA) * GS + gq) * 512 + jp * 16 + n16;
            const uint32_t* pb = a.codes + (size_t(tB) * GS + gq) * 512 + jp * 16 + n16;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                wr[i] = load_once(pa + i * 32);
                if (COLS == 32) wr[16 + i] = load_once(pb + i * 32);
            }
            const int cq = min(col, a.N - 1);
            mw = a.meta[(size_t(cq >> 4) * GS + gq) * 16 + (cq & 15)];
        }
        // the input's first use stays behind the weight loads (its wait would
        // otherwise come before they are issued)
        asm volatile("" : "+v"(px0.x), "+v"(px0.y), "+v"(px0.z), "+v"(px0.w), "+v"(px1.x), "+v"(px1.y), "+v"(px1.z),
                     "+v"(px1.w));
        for (int r0 = 0; r0 < M; r0 += kStreamChunk) {
            const int nr = min(kStreamChunk, M - r0);
            __syncthreads();
            // ---- this chunk's activation words, scales and scaled sums ----
            if constexpr (!FUSED) {
                for (int q = tid; q < nr * gc * 16; q += 256) {
                    const int r = q / (gc * 16), w4 = q % (gc * 16);
                    *reinterpret_cast<uint4*>(&la[r][w4 * 4]) = *reinterpret_cast<const uint4*>(
                        a.act_words + size_t(r0 + r) * (a.K / 4) + size_t(g0) * 64 + w4 * 4);
                }
                if (tid < nr * gc) {
                    const int r = tid / gc, gl = tid % gc;
                    const float sa = f16_bits_to_f32(a.act_scales[size_t(r0 + r) * GS + g0 + gl]);
                    lsa[r][gl] = sa;
                    lss[r][gl] = sa * float(a.act_sums[size_t(r0 + r) * GS + g0 + gl]);
                }
            }
            const int pairs = FUSED ? nr * gc : 0, l = tid & 15;
            for (int p0 = 0; p0 < pairs; p0 += 16) {
                uint4 x0 = px0, x1 = px1;
                if (r0 != 0 || p0 != 0) {
                    const uint16_t* xp = xsrc(r0, nr, p0);
                    x0 = *reinterpret_cast<const uint4*>(xp);
                    x1 = *reinterpret_cast<const uint4*>(xp + 8);
                }
                const uint32_t u[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
                float v[16];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    v[2 * e] = bf16_bits_to_f32(u[e] & 0xffffu);
                    v[2 * e + 1] = bf16_bits_to_f32(u[e] >> 16);
                }
                uint32_t flags = 0;
#pragma unroll
                for (int e = 0; e < 16; ++e) if (!isfinite(v[e])) flags |= a.flag_input;
                h128_quarter(v);
                uint32_t w4[4];
                uint16_t sbits;
                int sum;
                quantize_quarter_fast<127>(v, w4, sbits, sum, flags, a.flag_input | a.flag_act, a.flag_act);
                const int pi = p0 + (tid >> 4);
                if (pi < pairs) {
                    const int r = pi / gc, gl = pi % gc;
                    *reinterpret_cast<uint4*>(&la[r][gl * 64 + quarter_base(l) / 4]) =
                        make_uint4(w4[0], w4[1], w4[2], w4[3]);
                    if (l == 0) {
                        const float sa = f16_bits_to_f32(sbits);
                        lsa[r][gl] = sa;
                        lss[r][gl] = sa * float(sum);
                    }
                    flag_or(a.sticky, flags);
                }
            }
            __syncthreads();
            for (int r = 0; r < nr; ++r) {
                const uint32_t* ab = &la[r][hw * 64];
                int dot;
                if (TILE == 32) {
                    int d = 0;
#pragma unroll
                    for (int c4 = 0; c4 < 16; ++c4) {
                        const uint4 av = reinterpret_cast<const uint4*>(ab)[c4];
                        d = dot4(code_even(wr[2 * c4]), int(av.x), d);
                        d = dot4(code_odd(wr[2 * c4]), int(av.y), d);
                        d = dot4(code_even(wr[2 * c4 + 1]), int(av.z), d);
                        d = dot4(code_odd(wr[2 * c4 + 1]), int(av.w), d);
                    }
                    dot = d;
                } else {
                    int d0 = 0, d1 = 0;
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const uint2 av = *reinterpret_cast<const uint2*>(&ab[4 * i + 2 * jp]);
                        d0 = dot4(code_even(wr[i]), int(av.x), d0);
                        d0 = dot4(code_odd(wr[i]), int(av.y), d0);
                        if (COLS == 32) {
                            d1 = dot4(code_even(wr[16 + i]), int(av.x), d1);
                            d1 = dot4(code_odd(wr[16 + i]), int(av.y), d1);
                        }
                    }
                    const int sA = d0 + xor_perm_i<16>(d0), sB = COLS == 32 ? d1 + xor_perm_i<16>(d1) : sA;
                    dot = jp ? sB : sA;
                }
                // 16-column blocks: lanes L and L ^ 16 hold the same column
                if (gv && (COLS == 32 || jp == 0)) lterm[r][hw][L] = tree_term(dot, lsa[r][hw], lss[r][hw], mw);
            }
            __syncthreads();
            const int r = tid >> 5;
            if (r < nr && (COLS == 32 || L < 16)) {
                float v = g0 == 0 ? 0.f : lrun[r0 + r][L];
                for (int gl = 0; gl < gc; ++gl) v = v + lterm[r][gl][L];
                lrun[r0 + r][L] = v;
            }
        }
    }
    __syncthreads();
    for (int q = tid; q < M * COLS; q += 256) {
        const int r = q / COLS, c = col0 + q % COLS;
        if (c >= a.N) continue;
        const float v = lrun[r][q % COLS];
        const size_t o = size_t(r) * a.N + c;
        const uint16_t b = f32_to_bf16_bits(v);
        uint32_t f = 0;
        if (!isfinite(v)) f |= a.flag_projection;
        if ((b & 0x7f80u) == 0x7f80u) f |= a.flag_bf16;
        if (a.out) a.out[o] = v;
        if (a.out_bf16) a.out_bf16[o] = b;
        flag_or(a.sticky, f);
    }
}

hipError_t launch_project_gemv(const ProjArgs& a, int max_segments, Out mode, hipStream_t s) {
    const int GS = a.K / kGroup;
    const int GC = GS < 8 ? GS : 8;
    const int NT = 8 / GC;
    const int ntiles = (a.N + 31) / 32;
    const dim3 grid(max_segments, (ntiles + NT - 1) / NT);
    if (max_segments <= 0) return hipSuccess;
    if (mode == Out::Dense && !a.segments && a.dense_rows <= kStreamRows) {
        const dim3 g((a.N + 31) / 32);
        if (a.dense_x) {
            if (a.tile == 32) timed_launch("dense_stream", dense_stream_kernel<32, true>, g, dim3(256), 0, s, a);
            else timed_launch("dense_stream", dense_stream_kernel<16, true>, g, dim3(256), 0, s, a);
        } else {
            if (a.tile == 32) timed_launch("dense_stream", dense_stream_kernel<32, false>, g, dim3(256), 0, s, a);
            else if (a.dense_rows > kDenseNarrowRows)
                timed_launch("dense_stream", dense_stream_kernel<16, false, 16>, dim3((a.N + 15) / 16), dim3(256), 0, s,
                             a);
            else timed_launch("dense_stream", dense_stream_kernel<16, false>, g, dim3(256), 0, s, a);
        }
        return hipGetLastError();
    }
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
