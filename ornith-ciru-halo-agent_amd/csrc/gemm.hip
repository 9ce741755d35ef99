// Dense G256 linear for many rows on the bf16 matrix cores, reading the 4-bit
// codes directly.
//
// Semantics (the reference's prefill path, dense_g256_consumer.cpp:192-246
// with the torch.mm of native.py:140-150):
//   out[m, n] = bf16( sum_k bf16(H128 x)[m, k] * bf16(RN(RN(s * code) + off))[n, k] )
// with fp32 accumulation.  s * code is exact (4-bit code, 11-bit scale), so
// one fma per weight gives RN(RN(s * code) + off).  The summation order is
// this kernel's own (the reference's is hipBLASLt's), so results are checked
// by tolerance.
//
// Two kernels:
//  - transform: bf16(H128 x) of every 128-block, one wave per (8 rows, 128
//    k), the butterflies in registers and by DPP, written in matrix-core
//    fragment order so that every A operand is one contiguous 1 KiB load (a
//    row-major operand puts the 16 rows of a fragment in 16 cache lines per
//    instruction, and the L1 tag lookups become the limit);
//  - gemm: block tile 256 rows x 64 columns, 4 waves of 64 x 64 rows, two
//    blocks per CU (one block's barrier wait is covered by the other's
//    products), v_mfma_f32_16x16x32_bf16 on 32-k steps.  Per step every
//    thread dequantises one code word (8 weights of one column) into a 4-deep
//    LDS ring of bf16 [64 columns][32 k] tiles, two steps ahead, so each
//    weight is dequantised once per block; the B fragments are read from LDS
//    one step ahead; the A fragments come straight into registers, kRing
//    steps ahead; meta words once per 256-group.  The products are
//    (weights x activations), so each lane ends with 4 consecutive columns of
//    one row, staged through LDS into whole-row stores.
//    Lane l of a 16x16x32 product holds row / column l % 16, k chunk l / 16
//    (8 values); its four outputs are rows 4 (l / 16) + 0..3 of column l % 16.
#include "kernels.hpp"
#include "timing.hpp"

namespace ornith {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// ---- bf16(H128 x), in matrix-core fragment order -------------------------------
// Fragment layout of the transformed activations (rows padded to Mp, a
// multiple of 16, with zero rows): block (row group rg = r / 16, step
// s = k / 32) is 512 bf16 at ((rg * (K / 32)) + s) * 512, and holds value
// (r, k) at (16 * ((k % 32) / 8) + r % 16) * 8 + k % 8 - lane l's operand of a
// 16x16x32 product (row l % 16, k chunk l / 16) is its 16 bytes at 16 l, so
// one fragment is one contiguous 1 KiB load.

// Row-major [M, K] bf16(H128 x) (the activation operand of prepare_bf16):
// a quarter-wave per (row, 256-group).
__global__ __launch_bounds__(256) void transform_bf16_kernel(const uint16_t* __restrict__ x, int M, int K,
                                                             uint16_t* __restrict__ y, uint32_t* sticky) {
    const int G = K / kGroup, wave = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, l = lane & 15;
    const int g = 4 * wave + (lane >> 4);                  // (row, group)
    if (4 * wave >= M * G) return;
    const bool real = g < M * G;
    const uint16_t* src = x + size_t(min(g, M * G - 1)) * kGroup + quarter_base(l);
    const uint4 r0 = *reinterpret_cast<const uint4*>(src), r1 = *reinterpret_cast<const uint4*>(src + 8);
    const uint32_t u[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
    float v[16];
    uint32_t flags = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        v[2 * e] = bf16_bits_to_f32(u[e] & 0xffffu);
        v[2 * e + 1] = bf16_bits_to_f32(u[e] >> 16);
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) if (!isfinite(v[e])) flags |= kDenseNonfiniteInput;
    h128_quarter(v);
    uint32_t o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        if (!isfinite(v[2 * e]) || !isfinite(v[2 * e + 1])) flags |= kDenseNonfiniteInput;
        const uint16_t a = f32_to_bf16_bits(v[2 * e]), b = f32_to_bf16_bits(v[2 * e + 1]);
        if ((a & 0x7f80u) == 0x7f80u || (b & 0x7f80u) == 0x7f80u) flags |= kDenseNonfiniteBf16;
        o[e] = real ? uint32_t(a) | (uint32_t(b) << 16) : 0u;
    }
    if (real) {
        uint16_t* d = y + size_t(g) * kGroup + quarter_base(l);
        *reinterpret_cast<uint4*>(d) = make_uint4(o[0], o[1], o[2], o[3]);
        *reinterpret_cast<uint4*>(d + 8) = make_uint4(o[4], o[5], o[6], o[7]);
    }
    flag_or(sticky, real ? flags : 0u);
}

// Fragment order, one wave per (8-row half rg8 of a 16-row group, 128-k
// block kb): lane l is row 8 rg8 + l / 8 and k chunks c = q + 8 i (q = l % 8,
// i = 0, 1), i.e. k = 128 kb + 64 i + 8 q + 0..7, so the eight lanes of a row
// read 128 contiguous bytes per load.  Butterflies on k bits 0..2 in
// registers, bits 3, 4 and 5 across the lanes of a row (xor 1, 2, 4), bit 6
// in registers again: the ascending order of the reference.  Chunk c lands
// in fragment 4 kb + c / 4 at rows (16 (c % 4) + 8 (rg8 % 2) + l / 8) * 8:
// two 16-byte stores per lane.  Two waves per 16-row group keep two or more
// waves on a SIMD (one wave alone issues its vector work at half rate).
__global__ __launch_bounds__(256) void transform_frag_kernel(const uint16_t* __restrict__ x, int M, int Mp, int K,
                                                             uint16_t* __restrict__ y, uint32_t* sticky) {
    const int KB = K / 128, S = K / 32;
    const int wave = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int rg8 = wave / KB, kb = wave - rg8 * KB;
    if (8 * rg8 >= Mp) return;
    const int r = lane >> 3, q = lane & 7, row = 8 * rg8 + r;
    const bool real = row < M;
    const uint16_t* src = x + size_t(min(row, M - 1)) * K + 128 * kb + 8 * q;
    uint4 raw[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) raw[i] = *reinterpret_cast<const uint4*>(src + 64 * i);
    float v[16];                                            // v[8 i + e]: k = 64 i + 8 q + e
    uint32_t flags = 0;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t u[4] = {raw[i].x, raw[i].y, raw[i].z, raw[i].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[8 * i + 2 * e] = bf16_bits_to_f32(u[e] & 0xffffu);
            v[8 * i + 2 * e + 1] = bf16_bits_to_f32(u[e] >> 16);
        }
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) if (!isfinite(v[e])) flags |= kDenseNonfiniteInput;
#pragma unroll
    for (int b = 1; b < 8; b <<= 1) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            if (i & b) continue;
            const float lo = v[i], hi = v[i + b];
            v[i] = lo + hi;
            v[i + b] = lo - hi;
        }
    }
    // k bits 3, 4, 5 (lane bits 0, 1, 2): the lane with the bit set keeps
    // partner - own, the other own + partner
    {
        const uint32_t flip = (lane & 1) ? 0x80000000u : 0u;
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = xor_perm_f<1>(v[i]) + __uint_as_float(__float_as_uint(v[i]) ^ flip);
    }
    {
        const uint32_t flip = (lane & 2) ? 0x80000000u : 0u;
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = xor_perm_f<2>(v[i]) + __uint_as_float(__float_as_uint(v[i]) ^ flip);
    }
    {
        const uint32_t flip = (lane & 4) ? 0x80000000u : 0u;
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = xor_perm_f<4>(v[i]) + __uint_as_float(__float_as_uint(v[i]) ^ flip);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float lo = v[i], hi = v[i + 8];
        v[i] = lo + hi;
        v[i + 8] = lo - hi;
    }
    uint32_t o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float a = v[2 * e] * kInvSqrt128, b = v[2 * e + 1] * kInvSqrt128;
        if (!isfinite(a) || !isfinite(b)) flags |= kDenseNonfiniteInput;
        const uint16_t ha = f32_to_bf16_bits(a), hb = f32_to_bf16_bits(b);
        if ((ha & 0x7f80u) == 0x7f80u || (hb & 0x7f80u) == 0x7f80u) flags |= kDenseNonfiniteBf16;
        o[e] = real ? uint32_t(ha) | (uint32_t(hb) << 16) : 0u;
    }
    const int rg = rg8 >> 1, r16 = 8 * (rg8 & 1) + r;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = q + 8 * i;
        uint16_t* frag = y + (size_t(rg) * S + 4 * kb + c / 4) * 512 + (16 * (c % 4) + r16) * 8;
        *reinterpret_cast<uint4*>(frag) = make_uint4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
    }
    flag_or(sticky, real ? flags : 0u);
}

// ---- GEMM ---------------------------------------------------------------------
constexpr int kBM = 256, kBN = 64, kBK = 32, kRing = 4;

// 16-byte chunk `chunk` (0..3) of column c's 64-byte LDS row, rotated by the
// column so that any 8 consecutive columns at one chunk fill the 8 slots of a
// 128-byte bank line (a 16-byte access serves 8 lanes per LDS cycle)
__device__ __forceinline__ int b_slot(int c, int chunk) { return c * 64 + ((chunk ^ ((c >> 1) & 3)) << 4); }

// kslices > 1 (split K, for grids that fill few of the chip's block slots):
// tile = (slice, row block, column block); slice ks takes 256-groups
// [ks G / kslices, (ks + 1) G / kslices) and writes its fp32 sums to
// partial[ks] ([M, N]); dense_slices_kernel adds the slices in order.
__global__ __launch_bounds__(256, 2) void dense_gemm_bf16_kernel(const uint16_t* __restrict__ xt,
                                                                 const uint32_t* __restrict__ codes,
                                                                 const uint32_t* __restrict__ meta, int M, int N,
                                                                 int K, int nblocks_m, int nblocks_n, int kslices,
                                                                 uint16_t* __restrict__ out,
                                                                 float* __restrict__ partial, uint32_t* sticky) {
    __shared__ __attribute__((aligned(16))) uint8_t sB[kRing][kBN * 64];  // bf16 [64 columns][32 k], a ring
    __shared__ __attribute__((aligned(16))) uint8_t sC[4 * 16 * 136];     // output staging, 16 rows per wave
    const int tid = threadIdx.x, lane = tid & 63;
    const int wm = __builtin_amdgcn_readfirstlane(tid >> 6), w = wm;      // wave-uniform
    const int li = lane & 15, q = lane >> 4;
    // Workgroups go to the 8 XCDs round-robin: XCD x = L % 8 takes the
    // contiguous tile range [x * per, (x + 1) * per) of the row-major
    // (row block, column block) order, so its concurrent blocks share one or
    // two row blocks of A in its L2 instead of every row block.
    const int L = int(blockIdx.x), per = int(gridDim.x) / 8;
    const int tile = (L & 7) * per + (L >> 3), mn = nblocks_m * nblocks_n;
    if (tile >= mn * kslices) return;
    const int ks = tile / mn, nb = tile % nblocks_n, mb = (tile - ks * mn) / nblocks_n;
    const int row0 = mb * kBM, col0 = nb * kBN;
    const bool wave_live = row0 + 64 * wm < M;
    const int G = K / kGroup, S = K / kBK;
    const int g0 = ks * G / kslices, g1 = (ks + 1) * G / kslices;   // this slice's groups (at least one)
    const int st0 = 8 * g0, st1 = 8 * g1;

    // ---- B: column c = lane, word jw = wave of the step's four (32 k) ----
    // Addresses are a wave-uniform part (scalar registers) plus one 32-bit
    // byte offset per lane: the 64-bit per-lane address arithmetic would cost
    // the vector registers that the load rings need.
    const int c = lane, jw = w;
    const int colc = min(col0 + c, N - 1);
    const uint32_t cw_lane = (uint32_t(colc >> 4) * G * 512 + (colc & 15)) * 4;      // bytes
    const uint32_t mw_lane = (uint32_t(colc >> 4) * G * 16 + (colc & 15)) * 4;
    const char* cw_wave = reinterpret_cast<const char*>(codes) + jw * 64;
    const char* mw_wave = reinterpret_cast<const char*>(meta);
    // rings of kRing steps (code words, A chunks) in registers; the meta word
    // of a column is one per 256-group (8 steps), loaded a group ahead
    uint32_t cw[kRing];
    auto load_codes = [&](int st, int slot) {                 // step st: group st / 8, word 4 (st % 8) + jw
        cw[slot] = *reinterpret_cast<const uint32_t*>(cw_wave + size_t(st >> 3) * 2048 + (st & 7) * 256 + cw_lane);
    };
    auto load_meta = [&](int g) { return *reinterpret_cast<const uint32_t*>(mw_wave + size_t(g) * 64 + mw_lane); };
    uint32_t flags = 0;
    struct Affine { float s, off; };
    auto affine = [&](uint32_t m) {
        const Affine a{f16_bits_to_f32(m & 0xffffu), f16_bits_to_f32(m >> 16)};
        if (!isfinite(a.s) || !isfinite(a.off)) flags |= kDenseNonfiniteBf16;
        return a;
    };
    // bf16(RN(s * code + off)), nibble i of a word being k = 8 j + i.  s * code
    // + off is finite and within bf16 range whenever s and off are finite
    // (|s * 15 + off| < 2^21), so only the meta word needs checking, and the
    // hardware's round-to-nearest-even pair conversion gives the bits of the
    // scalar bf16 rounding.
    auto dequant = [&](int slot, int buf, Affine a) {
        const uint32_t lo = cw[slot] & 0x0F0F0F0Fu, hi = (cw[slot] >> 4) & 0x0F0F0F0Fu;
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const f32x2 v = {__builtin_fmaf(a.s, float((lo >> (8 * e)) & 0xffu), a.off),
                             __builtin_fmaf(a.s, float((hi >> (8 * e)) & 0xffu), a.off)};
            o[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
        }
        *reinterpret_cast<uint4*>(&sB[buf][b_slot(c, jw)]) = make_uint4(o[0], o[1], o[2], o[3]);
    };
    // the wave's B fragments of one step: column tile ct is columns 16 ct + 0..15
    auto read_b = [&](int buf, bf16x8 (&fb)[4]) {
#pragma unroll
        for (int ct = 0; ct < 4; ++ct)
            fb[ct] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(&sB[buf][b_slot(16 * ct + li, q)]));
    };

    // ---- A: row tile rt is fragment row group (row0 + 64 wm + 16 rt) / 16; lane l's 16 bytes at 16 l ----
    const char* a_frag[4];                                  // wave-uniform
    const int last_group = (M + 15) / 16 - 1;
    const uint32_t a_lane = lane * 16;
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)   // row groups past the padded rows repeat the last (never stored)
        a_frag[rt] = reinterpret_cast<const char*>(xt) +
                     size_t(min((row0 + 64 * wm + 16 * rt) >> 4, last_group)) * S * 1024;
    uint4 ra[kRing][4];
    auto load_a = [&](int st, int slot) {
#pragma unroll
        for (int rt = 0; rt < 4; ++rt)
            ra[slot][rt] = *reinterpret_cast<const uint4*>(a_frag[rt] + size_t(st) * 1024 + a_lane);
    };

    // Pipeline (steps st0 .. st1 - 1 of the slice, at least 8): at step st the products of st run on B
    // fragments read from LDS during step st - 1, the fragments of st + 1 are
    // read, and the B tile of st + 2 is dequantised into LDS buffer
    // (st + 2) % kRing, then one barrier.  A buffer is rewritten two barriers
    // after its last read.  Code words are loaded kRing steps before their
    // dequantisation, A fragments kRing steps before their products, meta
    // words a group before their group.
#pragma unroll
    for (int d = 0; d < kRing; ++d) {
        load_codes(st0 + d, d);
        load_a(st0 + d, d);
    }
    Affine acur = affine(load_meta(g0));
    uint32_t mnext = load_meta(min(g0 + 1, g1 - 1));
    dequant(0, 0, acur);
    load_codes(st0 + kRing, 0);
    dequant(1, 1, acur);
    load_codes(st0 + kRing + 1, 1);
    __syncthreads();
    bf16x8 fb[4];
    read_b(0, fb);

    f32x4 acc[4][4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) acc[rt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int g = g0; g < g1; ++g) {                            // one 256-group (8 steps) per iteration
        // the next group's scale and offset (for the tiles of its first two
        // steps, dequantised at steps 6 and 7), its successor's word loaded
        const Affine anext = g + 1 < g1 ? affine(mnext) : acur;
        mnext = load_meta(min(g + 2, g1 - 1));
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int st = 8 * g + u, slot = u % kRing, nslot = (u + 2) % kRing;
            // one scheduling region per step: the B fragments of st + 1 read,
            // the B tile of st + 2 dequantised into LDS, the products of st
            __builtin_amdgcn_sched_barrier(0);
            bf16x8 fn[4];
            read_b((u + 1) % kRing, fn);
            dequant(nslot, nslot, u < 6 ? acur : anext);
            // products (weights x activations): lane (li, q) gets row li, columns 4 q + 0..3;
            // a wave whose 64 rows all lie past M only dequantises its share of B
            if (wave_live) {
#pragma unroll
                for (int rt = 0; rt < 4; ++rt) {
                    const bf16x8 fa = __builtin_bit_cast(bf16x8, ra[slot][rt]);
#pragma unroll
                    for (int ct = 0; ct < 4; ++ct)
                        acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[ct], fa, acc[rt][ct], 0, 0, 0);
                }
            }
            // refills issued here, kRing steps ahead of their use (the scheduler
            // may not sink them towards their uses): A slot with step
            // st + kRing, code slot nslot with step st + 2 + kRing (clamped:
            // unconditional loads)
            __builtin_amdgcn_sched_barrier(0);
            load_a(min(st + kRing, st1 - 1), slot);
            load_codes(min(st + 2 + kRing, st1 - 1), nslot);
            __builtin_amdgcn_sched_barrier(0);
            __syncthreads();
#pragma unroll
            for (int ct = 0; ct < 4; ++ct) fb[ct] = fn[ct];
        }
        acur = anext;
    }

    if (kslices > 1) {
        // fp32 sums of this slice straight from the product layout: lane
        // (li, q) of row tile rt and column tile ct holds row 16 rt + li,
        // columns 16 ct + 4 q + 0..3 (N % 16 == 0: all four or none in range)
        float* dst = partial + size_t(ks) * M * N;
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) {
            const int row = row0 + 64 * wm + 16 * rt + li;
#pragma unroll
            for (int ct = 0; ct < 4; ++ct) {
                const int col = col0 + 16 * ct + 4 * q;
                if (row < M && col < N)
                    *reinterpret_cast<f32x4*>(dst + size_t(row) * N + col) = acc[rt][ct];
            }
        }
        flag_or(sticky, flags);
        return;
    }
    // ---- epilogue: bf16 RNE of the fp32 sums, through LDS to whole-row stores ----
    // The products are (weights x activations), so lane (li, q) of row tile rt
    // and column tile ct holds row 16 rt + li, columns 16 ct + 4 q + 0..3 of its
    // wave's 64 x 64 tile.  Per row tile each wave stages its 16 x 64 bf16 in
    // its own LDS rows (136 bytes apart against bank conflicts), then stores
    // 8 rows x 128 bytes per instruction.
    constexpr int kStage = 136;
    uint8_t* stage = sC + w * 16 * kStage;
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
            const f32x2 lo = {acc[rt][ct][0], acc[rt][ct][1]}, hi = {acc[rt][ct][2], acc[rt][ct][3]};
            const uint2 v = make_uint2(__builtin_bit_cast(uint32_t, __builtin_convertvector(lo, bf16x2)),
                                       __builtin_bit_cast(uint32_t, __builtin_convertvector(hi, bf16x2)));
            *reinterpret_cast<uint2*>(stage + li * kStage + (16 * ct + 4 * q) * 2) = v;
        }
        __syncthreads();
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int r = 8 * h + (lane >> 3), chunk = lane & 7;          // 8 columns per lane
            const uint4 v = *reinterpret_cast<const uint4*>(stage + r * kStage + chunk * 16);
            const int row = row0 + 64 * wm + 16 * rt + r, col = col0 + 8 * chunk;
            if (row < M && col < N) *reinterpret_cast<uint4*>(out + size_t(row) * N + col) = v;
        }
        __syncthreads();
    }
    flag_or(sticky, flags);
}

// out = bf16(((partial[0] + partial[1]) + ...) + partial[kslices - 1]), four
// columns per thread.
__global__ __launch_bounds__(256) void dense_slices_kernel(const float* __restrict__ partial, int kslices,
                                                           size_t count4, uint16_t* __restrict__ out) {
    const size_t i = size_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= count4) return;
    const f32x4* p = reinterpret_cast<const f32x4*>(partial) + i;
    f32x4 s = p[0];
    for (int k = 1; k < kslices; ++k) {
        const f32x4 v = p[size_t(k) * count4];
#pragma unroll
        for (int e = 0; e < 4; ++e) s[e] = s[e] + v[e];
    }
    const f32x2 lo = {s[0], s[1]}, hi = {s[2], s[3]};
    reinterpret_cast<uint2*>(out)[i] = make_uint2(__builtin_bit_cast(uint32_t, __builtin_convertvector(lo, bf16x2)),
                                                  __builtin_bit_cast(uint32_t, __builtin_convertvector(hi, bf16x2)));
}

}  // namespace

hipError_t launch_transform_bf16_fast(const uint16_t* x, int M, int K, uint16_t* y, uint32_t* sticky, hipStream_t s) {
    const int waves = (M * (K / kGroup) + 3) / 4;
    timed_launch("transform_bf16", transform_bf16_kernel, dim3((waves + 3) / 4), dim3(256), 0, s, x, M, K, y, sticky);
    return hipGetLastError();
}

hipError_t launch_transform_bf16_frag(const uint16_t* x, int M, int K, uint16_t* y, uint32_t* sticky, hipStream_t s) {
    const int Mp = (M + 15) / 16 * 16;
    const int waves = Mp / 8 * (K / 128);
    timed_launch("transform_bf16_frag", transform_frag_kernel, dim3((waves + 3) / 4), dim3(256), 0, s, x, M, Mp, K, y,
                 sticky);
    return hipGetLastError();
}

int dense_gemm_slices(int M, int N, int K, size_t partial_bytes) {
    // the GEMM runs two blocks per CU: a grid of fewer tiles than block slots
    // splits K, up to kMaxDenseSlices ways with at least two 256-groups per
    // slice (one-group slices measured slower: 1120 x 2048 x 512, 11.1 us
    // unsplit against 16.1 + 4.6 split), as far as the partial sums fit
    const int tiles = ((N + kBN - 1) / kBN) * ((M + kBM - 1) / kBM);
    const int slots = 2 * device_cu_count();
    int k = min(min(slots / max(tiles, 1), K / kGroup / 2), kMaxDenseSlices);
    while (k > 1 && size_t(k) * M * N * 4 > partial_bytes) --k;
    return max(k, 1);
}

hipError_t launch_dense_gemm_bf16(const uint16_t* xt, const uint32_t* codes, const uint32_t* meta, int M, int N, int K,
                                  uint16_t* out, float* partial, size_t partial_bytes, uint32_t* sticky,
                                  hipStream_t s) {
    const int nbn = (N + kBN - 1) / kBN, nbm = (M + kBM - 1) / kBM;
    const int kslices = dense_gemm_slices(M, N, K, partial ? partial_bytes : 0);
    const int per = (nbn * nbm * kslices + 7) / 8;       // tiles per XCD
    timed_launch("dense_gemm", dense_gemm_bf16_kernel, dim3(8 * per), dim3(256), 0, s, xt, codes, meta, M, N, K, nbm,
                 nbn, kslices, out, partial, sticky);
    hipError_t st = hipGetLastError();
    if (st != hipSuccess || kslices == 1) return st;
    const size_t count4 = size_t(M) * N / 4;
    timed_launch("dense_slices", dense_slices_kernel, dim3((count4 + 255) / 256), dim3(256), 0, s,
                 static_cast<const float*>(partial), kslices, count4, out);
    return hipGetLastError();
}

}  // namespace ornith
