// W8 G128 LM head (kernels/head/head_i8_tile_consumer.cpp:30-291).
//
// Arithmetic (bit-exact): fp32 H128 of each 128 block, per-128 A8 encoding
// (absmax/127, fp16 scale, round-even, clamp), exact int8 dot per group, then
// acc = acc + RN(sw * RN(sa * dot)) over the 16 groups in ascending order.
// Weights keep the reference's tile layout uint32 [N/16, 128, 4, 16]: the
// (n16 tile, group) block of 512 words (2 KiB) is contiguous.
#include <algorithm>
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

// ---------------------------------------------------------------------------
// Projection on the int8 matrix cores (v_mfma_i32_16x16x64_i8).
//
// A block of 8 waves copies the M rows' A8 words (MT tiles of 16 rows, rows
// past M repeating row M - 1) and their group scales into LDS once; each
// wave then streams its own contiguous range of 16-column tiles (the N / 16
// tiles split evenly over all waves of the grid), D groups of weights in
// flight, the ring running across tiles.
//  - Weights of one (tile, group) are 2 KiB: words [kq 0..7][kr 0..3][n 0..15],
//    word (kq, kr, n) = the four K bytes 16 kq + 4 kr .. +3 of column n.  For
//    k-step s (64 K) lane n + 16q needs words (4s + q, 0..3, n): the 16
//    contiguous K bytes 64 s + 16 q .. +15 of column n, its B operand.  Those
//    words lie 64 bytes apart, so (LB, the path without group dots) each lane
//    loads 16 contiguous bytes instead (two non-temporal loads per block:
//    1 row 96 -> 81 us, 64 rows 154 -> 141 us against dword loads) and the
//    wave passes the block through 2 KiB of LDS to regroup it per column;
//    the group-dot path keeps the dword loads into registers.
//  - A: lane r + 16q reads row r's same 16 bytes from LDS; 16-byte piece p of
//    row r sits at slot (p & ~15) | ((p ^ r) & 15).
//  - C: register k of lane n + 16q is row 4q + k, column n.  Dots start from
//    the bits of kDotBias (|dot| <= 128 * 127 * 127 < 2^22), so
//    fma(sa, acc, -sa * kDotBias) is RN(sa * dot); term = RN(sw * that);
//    value = value + term, ascending groups (head_i8_tile_consumer.cpp:96-104).
// ---------------------------------------------------------------------------
constexpr float kW8DotBias = 12582912.0f;          // 1.5 * 2^23
constexpr int kW8DotBiasBits = 0x4B400000;
constexpr int kW8Waves = 8;
typedef int w8_i32x4 __attribute__((ext_vector_type(4)));

template <int MT, int D, bool DOTS, bool LB = false>
__global__ __launch_bounds__(64 * kW8Waves, 1) void head_w8_mfma_kernel(
    const uint32_t* __restrict__ w, const uint16_t* __restrict__ wscale, const uint32_t* __restrict__ act,
    const uint16_t* __restrict__ ascale, int M, int N, int nwaves, float* __restrict__ diag,
    uint16_t* __restrict__ out, int32_t* __restrict__ group_dots, uint32_t* sticky) {
    constexpr int ROWS = 16 * MT, RW = kHeadK / 4, NT = 64 * kW8Waves;
    static_assert(kHeadGroups % D == 0, "ring slots repeat every tile");
    __shared__ __attribute__((aligned(16))) uint32_t sA[ROWS * RW];
    __shared__ __attribute__((aligned(16))) float s_sa[kHeadGroups][ROWS];
    __shared__ __attribute__((aligned(16))) float s_nb[kHeadGroups][ROWS];
    // LB: each wave's (tile, group) block passes through 2 KiB of LDS: 16-byte
    // loads in (chunk c of a 1 KiB half from lane c), chunk c stored at
    // position c ^ 4 ((c >> 4) & 3), B words read back per column
    // (conflict-free both ways)
    __shared__ __attribute__((aligned(16))) uint32_t sB[LB ? kW8Waves * 512 : 4];
    // LB up to 32 rows: each wave's logits of a four-tile group (rows of 68 floats)
    __shared__ __attribute__((aligned(16))) float sO[LB && MT <= 2 ? kW8Waves * ROWS * 68 : 4];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, li = lane & 15, q = lane >> 4;

    for (int i = tid; i < ROWS * (RW / 4); i += NT) {
        const int r = i / (RW / 4), pc = i % (RW / 4);
        const u32x4 v = *reinterpret_cast<const u32x4*>(act + size_t(min(r, M - 1)) * RW + 4 * pc);
        *reinterpret_cast<u32x4*>(&sA[r * RW + 4 * ((pc & ~15) | ((pc ^ r) & 15))]) = v;
    }
    for (int i = tid; i < ROWS * kHeadGroups; i += NT) {
        const int r = i / kHeadGroups, g = i % kHeadGroups;
        const float sa = f16_bits_to_f32(ascale[min(r, M - 1) * kHeadGroups + g]);
        s_sa[g][r] = sa;
        s_nb[g][r] = -sa * kW8DotBias;
    }
    __syncthreads();

    const int gw = wv * int(gridDim.x) + int(blockIdx.x);
    if (gw >= nwaves) return;                         // no barrier follows
    const int ntiles = N >> 4;
    const int base = ntiles / nwaves, extra = ntiles % nwaves;
    const int t0 = gw * base + min(gw, extra), cnt = base + (gw < extra ? 1 : 0);
    if (cnt == 0) return;

    // step st = 16 * (tile - t0) + group: 512 weight words and the lane
    // column's scale per step
    const uint32_t* wbase = w + size_t(t0) * (kHeadGroups * 512) + 64 * q + li;
    const uint16_t* sbase = wscale + size_t(16 * t0 + li) * kHeadGroups;
    uint32_t bw[D][8];
    uint16_t bs[D];
    uint32_t* stg = sB + (LB ? wv * 512 : 0);
    const int pos = lane ^ (((lane >> 4) & 3) << 2);
    const uint32_t* wx = w + size_t(t0) * (kHeadGroups * 512) + 4 * lane;
    auto load_b = [&](int st, int slot) {
        if constexpr (LB) {
            const uint32_t* src = wx + size_t(st) * 512;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                // non-temporal at every row count (1 row 95 -> 81 us, 8 rows 110 -> 99)
                const uint4 v = load_once4(src + 256 * h);
                bw[slot][4 * h] = v.x;
                bw[slot][4 * h + 1] = v.y;
                bw[slot][4 * h + 2] = v.z;
                bw[slot][4 * h + 3] = v.w;
            }
        } else {
            const uint32_t* src = wbase + size_t(st) * 512;
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const uint32_t* pu = src + 256 * (u >> 2) + 16 * (u & 3);
                bw[slot][u] = MT >= 4 ? load_once(pu) : *pu;   // non-temporal only for the 64-row tiles (measured)
            }
        }
        bs[slot] = sbase[size_t(st >> 4) * (16 * kHeadGroups) + (st & 15)];
    };
#pragma unroll
    for (int st = 0; st < D; ++st) load_b(st, st);
    uint32_t flags = 0;
    constexpr w8_i32x4 kInit = {kW8DotBiasBits, kW8DotBiasBits, kW8DotBiasBits, kW8DotBiasBits};

    // one tile's values (t: the wave's tile number)
    auto tile = [&](int t, float (&val)[MT][4]) {
        const int col = 16 * (t0 + t) + li;
        (void)col;
#pragma unroll
        for (int rt = 0; rt < MT; ++rt)
#pragma unroll
            for (int k = 0; k < 4; ++k) val[rt][k] = 0.f;
        const bool refill = t + 1 < cnt;
        // D groups per pass (compile-time ring slots); the passes stay a loop so
        // the A fragments of one pass only are live
#pragma unroll 1
        for (int g0 = 0; g0 < kHeadGroups; g0 += D) {
#pragma unroll
            for (int slot = 0; slot < D; ++slot) {
                const int g = g0 + slot;
                w8_i32x4 acc[MT];
                uint32_t bl[8];
                if constexpr (LB) {
#pragma unroll
                    for (int h = 0; h < 2; ++h)
                        *reinterpret_cast<uint4*>(&stg[256 * h + 4 * pos]) =
                            make_uint4(bw[slot][4 * h], bw[slot][4 * h + 1], bw[slot][4 * h + 2], bw[slot][4 * h + 3]);
#pragma unroll
                    for (int u = 0; u < 8; ++u) bl[u] = stg[256 * (u >> 2) + 64 * q + 16 * ((u & 3) ^ q) + li];
                } else {
#pragma unroll
                    for (int u = 0; u < 8; ++u) bl[u] = bw[slot][u];
                }
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    const w8_i32x4 fb = {int(bl[4 * s]), int(bl[4 * s + 1]), int(bl[4 * s + 2]), int(bl[4 * s + 3])};
#pragma unroll
                    for (int rt = 0; rt < MT; ++rt) {
                        const int r = 16 * rt + li, p = 8 * g + 4 * s + q;
                        const u32x4 av =
                            *reinterpret_cast<const u32x4*>(&sA[r * RW + 4 * ((p & ~15) | ((p ^ r) & 15))]);
                        const w8_i32x4 fa = {int(av.x), int(av.y), int(av.z), int(av.w)};
                        acc[rt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa, fb, s ? acc[rt] : kInit, 0, 0, 0);
                    }
                }
                // the scale is taken at its use: converted early, every slot's
                // scale (the last load of its refill) was waited for at the top
                // of a pass, which emptied the ring
                uint32_t sbits = bs[slot];
                asm volatile("" : "+v"(sbits));
                const float sw = f16_bits_to_f32(uint16_t(sbits));
                // always refill (the wave's last steps reload the current one:
                // a predicated load would make every later wait drain the queue)
                load_b(g + D < kHeadGroups || refill ? 16 * t + g + D : 16 * t + g, slot);
#pragma unroll
                for (int rt = 0; rt < MT; ++rt) {
                    const float4 sa4 = *reinterpret_cast<const float4*>(&s_sa[g][16 * rt + 4 * q]);
                    const float4 nb4 = *reinterpret_cast<const float4*>(&s_nb[g][16 * rt + 4 * q]);
                    const float sa[4] = {sa4.x, sa4.y, sa4.z, sa4.w}, nb[4] = {nb4.x, nb4.y, nb4.z, nb4.w};
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const float scaled = __builtin_fmaf(sa[k], __int_as_float(acc[rt][k]), nb[k]);
                        const float term = sw * scaled;
                        val[rt][k] = val[rt][k] + term;
                        if constexpr (DOTS) {
                            const int row = 16 * rt + 4 * q + k;
                            if (row < M)
                                group_dots[(size_t(row) * N + col) * kHeadGroups + g] = acc[rt][k] - kW8DotBiasBits;
                        }
                    }
                }
            }
        }
    };
    // LB: tiles go in aligned groups of GT = 4 (64 columns) and a group's
    // logits are stored together: up to 32 rows they pass through LDS
    // (rows of 64 values, padded to 68 words) and leave as 16-byte fp32 and
    // 8-byte bf16 pieces, four whole rows of the group per store; above, each
    // tile's 4-row pieces are stored back to back.  Measured at 8 rows: the
    // head without any logit store (a timing probe) 83 us, stored a tile at
    // a time (64- and 32-byte pieces) 99.5 us, this way 92.5 us.
    constexpr int GT = LB ? 4 : 1;
    const int tend = t0 + cnt;
    for (int g4 = t0 & ~(GT - 1); g4 < tend; g4 += GT) {
        float ov[GT][MT][4];
#pragma unroll
        for (int u = 0; u < GT; ++u) {
            const int tt = g4 + u;
            if (tt >= t0 && tt < tend) tile(tt - t0, ov[u]);
        }
        if constexpr (LB && MT <= 2) {
            float* so = sO + wv * (ROWS * 68);
#pragma unroll
            for (int u = 0; u < GT; ++u)
#pragma unroll
                for (int rt = 0; rt < MT; ++rt)
#pragma unroll
                    for (int k = 0; k < 4; ++k) so[(16 * rt + 4 * q + k) * 68 + 16 * u + li] = ov[u][rt][k];
            const int c = lane & 15, tt = g4 + (c >> 2);
            const bool live = tt >= t0 && tt < tend;
            const int col = 16 * g4 + 4 * c;
            for (int r0 = 0; r0 < M; r0 += 4) {
                const int row = r0 + (lane >> 4);
                if (!live || row >= M) continue;
                const float4 v4 = *reinterpret_cast<const float4*>(&so[row * 68 + 4 * c]);
                const float v[4] = {v4.x, v4.y, v4.z, v4.w};
                uint16_t b[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    b[e] = f32_to_bf16_bits(v[e]);
                    if (!isfinite(v[e])) flags |= kDenseNonfiniteProjection;
                    if ((b[e] & 0x7f80u) == 0x7f80u) flags |= kDenseNonfiniteBf16;
                }
                const size_t o = size_t(row) * N + col;
                *reinterpret_cast<float4*>(diag + o) = v4;
                *reinterpret_cast<uint2*>(out + o) =
                    make_uint2(uint32_t(b[0]) | (uint32_t(b[1]) << 16), uint32_t(b[2]) | (uint32_t(b[3]) << 16));
            }
        } else {
#pragma unroll
            for (int u = 0; u < GT; ++u) {
                const int tt = g4 + u;
                if (tt < t0 || tt >= tend) continue;
                const int col = 16 * tt + li;
#pragma unroll
                for (int rt = 0; rt < MT; ++rt)
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const int row = 16 * rt + 4 * q + k;
                        if (row >= M) continue;
                        const float v = ov[u][rt][k];
                        const uint16_t b = f32_to_bf16_bits(v);
                        if (!isfinite(v)) flags |= kDenseNonfiniteProjection;
                        if ((b & 0x7f80u) == 0x7f80u) flags |= kDenseNonfiniteBf16;
                        const size_t o = size_t(row) * N + col;
                        diag[o] = v;
                        out[o] = b;
                    }
            }
        }
    }
    flag_or(sticky, flags);
}

// Per-row argmax of bf16 logits [M, N] (row stride ld): the first NaN if any,
// else the first maximum (torch.argmax / numpy).  One block per row; every
// thread scans a strided slice, keys are order-preserving images of the value
// over the complemented column, so the unsigned maximum is the answer.
__global__ __launch_bounds__(256) void logits_argmax_kernel(const uint16_t* __restrict__ logits, int N, int64_t ld,
                                                            int64_t* __restrict__ argmax) {
    __shared__ uint64_t s_best[256];
    const int row = blockIdx.x, tid = threadIdx.x;
    const uint16_t* src = logits + size_t(row) * size_t(ld);
    uint64_t best = 0;
    for (int c = tid; c < N; c += 256) {
        const uint32_t b = src[c];
        const bool nan = (b & 0x7fffu) > 0x7f80u;
        const uint32_t mag = (b & 0x8000u) ? ((b & 0x7fffu) ? (~b & 0xffffu) : 0x8000u) : (b | 0x8000u);
        const uint32_t ord = nan ? 0x1ffffu : mag;        // every NaN above +inf
        const uint64_t key = (uint64_t(ord) << 32) | uint32_t(~c);
        best = key > best ? key : best;
    }
    s_best[tid] = best;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (tid < s) s_best[tid] = s_best[tid] > s_best[tid + s] ? s_best[tid] : s_best[tid + s];
        __syncthreads();
    }
    if (tid == 0) argmax[row] = int64_t(~uint32_t(s_best[0]));
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
extern "C" int ornith_head_i8_tile_shortlist(void) { return 1; }

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
    timed_launch("head_encode", head_encode_kernel, dim3((waves + 3) / 4), dim3(256), 0, stream,
                 static_cast<const uint16_t*>(input), M, words, ascale, sticky);
    hipError_t st = hipGetLastError();
    if (st != hipSuccess) return st;
    auto diag = at<float>(workspace, l.projection);
    const int cus = device_cu_count();
    const int ntiles = N / 16;
    const int blocks = std::min(cus, (ntiles + kW8Waves - 1) / kW8Waves);
    const int nwaves = std::min(blocks * kW8Waves, ntiles);
    const auto W = static_cast<const uint32_t*>(weights);
    const auto S = static_cast<const uint16_t*>(scales);
    auto out = static_cast<uint16_t*>(output);
    auto dots = static_cast<int32_t*>(group_dots);
    auto go = [&](auto kernel) {
        timed_launch("head_w8_mfma", kernel, dim3(blocks), dim3(64 * kW8Waves), 0, stream, W, S, words, ascale, M, N,
                     nwaves, diag, out, dots, sticky);
    };
    const int mt = (M + 15) / 16;
    if (group_dots) {
        if (mt == 1) go(head_w8_mfma_kernel<1, 4, true>);
        else if (mt == 2) go(head_w8_mfma_kernel<2, 4, true>);
        else if (mt == 3) go(head_w8_mfma_kernel<3, 2, true>);
        else go(head_w8_mfma_kernel<4, 2, true>);
    } else {
        if (mt == 1) go(head_w8_mfma_kernel<1, 4, false, true>);
        else if (mt == 2) go(head_w8_mfma_kernel<2, 4, false, true>);
        else if (mt == 3) go(head_w8_mfma_kernel<3, 4, false, true>);
        else go(head_w8_mfma_kernel<4, 4, false, true>);
    }
    return hipGetLastError();
}

extern "C" hipError_t ornith_logits_argmax_launch(const void* logits_bf16, int M, int N, int64_t ld,
                                                  void* argmax_i64, hipStream_t stream) {
    if (M < 0 || N < 0 || ld < N) return hipErrorInvalidValue;
    if (!M || !N) return hipSuccess;
    const Buffer buffers[] = {{logits_bf16, (size_t(M - 1) * size_t(ld) + size_t(N)) * 2, 2, false, false},
                              {argmax_i64, size_t(M) * 8, 8, true, false}};
    if (!check_buffers(buffers)) return hipErrorInvalidValue;
    timed_launch("logits_argmax", logits_argmax_kernel, dim3(M), dim3(256), 0, stream,
                 static_cast<const uint16_t*>(logits_bf16), N, ld, static_cast<int64_t*>(argmax_i64));
    return hipGetLastError();
}
