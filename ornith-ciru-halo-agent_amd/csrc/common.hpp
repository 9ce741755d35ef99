// Shared device helpers for the MI355X (gfx950, wave64) Ornith G256 kernels.
//
// Numerics contract (restated from kernels/dense/dense_g256_api.h:32-38 and
// kernels/routed_storage/routed_storage_n32_consumer.cpp:12-21): fp32
// arithmetic is evaluated operation by operation (the library is compiled
// with -ffp-contract=off), fp32 division is correctly rounded, bf16 and fp16
// conversions round to nearest even.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stddef.h>

namespace ornith {

// native 4 x u32 vector: array elements of this type stay in registers
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kExperts = 256, kTop = 8, kHidden = 2048, kInter = 512, kGroup = 256;
constexpr int kShared = kExperts;            // bank id of the always-on shared expert
constexpr int kWave = 64;

// 1/sqrt(128) with the bit pattern 0x3db504f3 (routed_storage_n32_consumer.cpp:12).
constexpr float kInvSqrt128 = 0x1.6a09e6p-4f;

// Sticky flag bits of the routed ABI (routed_storage_n32_consumer.cpp:33-183).
enum : uint32_t {
    kFlagNonfiniteInput = 1, kFlagInvalidActivation = 2, kFlagInvalidExpert = 4,
    kFlagNonfiniteProjection = 8, kFlagNonfiniteMiddle = 16, kFlagNonfiniteOutput = 32,
};
// Dense/head flag bits (dense_g256_api.h:14-19, head_i8_tile_api.h:16-21).
enum : uint32_t {
    kDenseNonfiniteInput = 1, kDenseInvalidActivation = 2,
    kDenseNonfiniteProjection = 4, kDenseNonfiniteBf16 = 8,
};

// Routed expert banks come in tiles of ORNITH_ROUTED_TILE output columns:
// 32 is the N32 storage (routed_storage_n32_consumer.cpp:1-2), 16 the
// checkpoint's N16 storage read by the parent routed library
// (routed_direct_api.h:7).  The library is built once per tile width.
// Shared-expert banks are dense N32 banks in both builds.
#ifndef ORNITH_ROUTED_TILE
#define ORNITH_ROUTED_TILE 32
#endif
static_assert(ORNITH_ROUTED_TILE == 16 || ORNITH_ROUTED_TILE == 32, "routed tile must be 16 or 32");
constexpr int kRoutedTile = ORNITH_ROUTED_TILE;
constexpr int kRoutedTileLog2 = kRoutedTile == 16 ? 4 : 5;

// Addressing inside one bank of `groups` 256-groups: codes [N/TW, groups, 32, TW]
// (word j of column n, group g at word(n, g) + j * stride()), meta [N/TW, groups, TW].
struct BankView {
    int log2;   // log2 of the tile width TW
    __device__ __forceinline__ size_t word(int n, int g, int groups) const {
        return ((size_t(n >> log2) * groups + g) << (5 + log2)) + (n & ((1 << log2) - 1));
    }
    __device__ __forceinline__ size_t meta(int n, int g, int groups) const {
        return ((size_t(n >> log2) * groups + g) << log2) + (n & ((1 << log2) - 1));
    }
    __device__ __forceinline__ int stride() const { return 1 << log2; }
};
// the view of a routed bank, or (shared) of a shared-expert bank
__device__ __forceinline__ BankView bank_view(bool shared) { return BankView{shared ? 5 : kRoutedTileLog2}; }

__host__ __device__ inline size_t align256(size_t n) { return (n + 255) & ~size_t(255); }
template <class T> __host__ __device__ inline T* at(void* base, size_t offset) {
    return reinterpret_cast<T*>(static_cast<uint8_t*>(base) + offset);
}

__device__ __forceinline__ float fdiv_rn(float a, float b) { return __fdiv_rn(a, b); }
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits) { return __uint_as_float(bits << 16); }
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float v) {
    uint32_t b = __float_as_uint(v);
    if ((b & 0x7fffffffu) > 0x7f800000u) return uint16_t((b >> 16) | 0x40u);
    return uint16_t((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ float bf16_round(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }
__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits) {
    return __half2float(__ushort_as_half(uint16_t(bits)));
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float v) { return __half_as_ushort(__float2half_rn(v)); }

// Deterministic exp with the reference's Taylor coefficients and step order
// (kernels/routed_storage/portable_exp.h:6-26): n = rint(x log2 e), the
// reduced argument r in two steps, the degree-9 polynomial, 2^n.
__device__ __forceinline__ float portable_exp_poly(float x, float n_float) {
    const float high = n_float * 0x1.62e400p-1f;
    const float low = n_float * 0x1.7f7d1cp-20f;
    const float r = (x - high) - low;
    float p = 0x1.a01a02p-16f;
    p = p * r + 0x1.a01a02p-13f;
    p = p * r + 0x1.6c16c2p-10f;
    p = p * r + 0x1.111112p-7f;
    p = p * r + 0x1.555556p-5f;
    p = p * r + 0x1.555556p-3f;
    p = p * r + 0x1p-1f;
    p = p * r + 0x1p+0f;
    p = p * r + 0x1p+0f;
    return p;
}
// The special cases are applied by selects after the polynomial (the GPU's
// float ops do not trap and the conversion saturates), so no lane branches.
__device__ __forceinline__ float portable_exp(float x) {
    const float n_float = __builtin_rintf(x * 0x1.715476p+0f);
    // in range for every x the result keeps (-104 < x < 89); the clamp keeps the
    // conversion defined for the special cases, whose results are discarded
    const int n = static_cast<int>(fminf(fmaxf(n_float, -200.f), 200.f));
    float y = __builtin_ldexpf(portable_exp_poly(x, n_float), n);
    asm volatile("" : "+v"(y));               // keep the polynomial unconditional (no per-lane branch)
    // special cases as three selects, innermost first
    y = x >= 89.f ? __builtin_huge_valf() : y;
    y = x <= -104.f ? 0.f : y;
    return x != x ? x : y;
}
__device__ __forceinline__ float silu_portable(float g) { return fdiv_rn(g, 1.f + portable_exp(-g)); }

// silu_portable for 2^-60 <= |g| <= 80 (silu_fast_domain).  There no special
// case of portable_exp applies and |n| < 128, and the divisor d = 1 + e lies
// in [1, 2^116] with every quotient and remainder a normal number, so the
// division takes its short correctly rounded form: y0 = v_rcp_f32(d), one
// Newton step y = y0 + y0 (1 - d y0), q0 = RN(g y), the exact remainder
// g - d q0 (fma), and q = RN(q0 + remainder y) (Markstein's final step).
// Bit-identical to silu_portable on this domain: checked on the MI355X for
// every fp32 value in it.
__device__ __forceinline__ bool silu_fast_domain(float g) {
    const float a = __builtin_fabsf(g);
    return a <= 80.f && a >= 0x1p-60f;
}
__device__ __forceinline__ float silu_portable_fast(float g) {
    const float x = -g;
    const float n_float = __builtin_rintf(x * 0x1.715476p+0f);
    const float e = __builtin_ldexpf(portable_exp_poly(x, n_float), static_cast<int>(n_float));
    const float d = 1.f + e;
    const float y0 = __builtin_amdgcn_rcpf(d);
    const float y = __builtin_fmaf(y0, __builtin_fmaf(-d, y0, 1.f), y0);
    const float q0 = g * y;
    return __builtin_fmaf(__builtin_fmaf(-d, q0, g), y, q0);
}
// silu_portable of one value per lane, the short form when every active
// lane's value is in its domain (a wave-uniform choice; same bits either way).
__device__ __forceinline__ float silu_portable_wave(float g) {
    return __builtin_amdgcn_ballot_w64(!silu_fast_domain(g)) == 0 ? silu_portable_fast(g) : silu_portable(g);
}

// ---- wave64 cross-lane helpers --------------------------------------------
// Exact lane permutation l -> l ^ M, M in {1,2,4,8,16,32}, with no LDS-pipe
// instruction: DPP quad_perm for 1 and 2; DPP row_ror for 4 and 8 (row_ror:n
// gives lane i the value of lane (i - n) mod 16, so xor 8 is row_ror:8 and
// xor 4 is row_ror:4 on lanes with bit 2 set, row_ror:12 on the others);
// v_permlane16_swap / v_permlane32_swap for 16 and 32 (swapping a value with
// itself returns rows (0,0,2,2) and (1,1,3,3), resp. halves (lo,lo) and
// (hi,hi)).  Lanes are threadIdx.x & 63 of a one-dimensional block.
template <int M> __device__ __forceinline__ int xor_perm_i(int v) {
    if constexpr (M == 1) return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
    else if constexpr (M == 2) return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
    else if constexpr (M == 4) {
        const int down = __builtin_amdgcn_update_dpp(0, v, 0x124, 0xF, 0xF, false);
        const int up = __builtin_amdgcn_update_dpp(0, v, 0x12C, 0xF, 0xF, false);
        return (threadIdx.x & 4) ? down : up;
    } else if constexpr (M == 8) return __builtin_amdgcn_update_dpp(0, v, 0x128, 0xF, 0xF, false);
    else if constexpr (M == 16) {
        const auto s = __builtin_amdgcn_permlane16_swap(uint32_t(v), uint32_t(v), false, false);
        return int((threadIdx.x & 16) ? s[0] : s[1]);
    } else {
        static_assert(M == 32, "xor_perm: M must be a power of two up to 32");
        const auto s = __builtin_amdgcn_permlane32_swap(uint32_t(v), uint32_t(v), false, false);
        return int((threadIdx.x & 32) ? s[0] : s[1]);
    }
}
template <int M> __device__ __forceinline__ float xor_perm_f(float v) {
    return __int_as_float(xor_perm_i<M>(__float_as_int(v)));
}
__device__ __forceinline__ float readlane_f(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
// Row-uniform reductions with DPP only: after xor 1 and xor 2 (quad_perm)
// each quad is uniform, so row_half_mirror pairs whole quads (== xor 4) and
// row_mirror pairs whole half-rows (== xor 8).  The four 16-lane rows are then
// combined through readlane in the xor-16 / xor-32 pairing.  For the fp32
// butterfly this gives exactly the bits of the xor butterfly with masks
// 1, 2, 4, 8, 16, 32 (each step adds two identical-per-lane operands, and
// fp32 addition is commutative).
template <int CTRL> __device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL> __device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(dpp_i<CTRL>(__float_as_int(v)));
}
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<kDppXor1>(v));
    v = fmaxf(v, dpp_f<kDppXor2>(v));
    v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
    v = fmaxf(v, dpp_f<kDppMirror>(v));
    return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}
__device__ __forceinline__ uint32_t wave_max_u(uint32_t v) {
    v = max(v, uint32_t(dpp_i<kDppXor1>(int(v))));
    v = max(v, uint32_t(dpp_i<kDppXor2>(int(v))));
    v = max(v, uint32_t(dpp_i<kDppHalfMirror>(int(v))));
    v = max(v, uint32_t(dpp_i<kDppMirror>(int(v))));
    const uint32_t r0 = uint32_t(__builtin_amdgcn_readlane(int(v), 0)), r1 = uint32_t(__builtin_amdgcn_readlane(int(v), 16));
    const uint32_t r2 = uint32_t(__builtin_amdgcn_readlane(int(v), 32)), r3 = uint32_t(__builtin_amdgcn_readlane(int(v), 48));
    return max(max(r0, r1), max(r2, r3));
}
__device__ __forceinline__ int wave_min_i(int v) {
    v = min(v, dpp_i<kDppXor1>(v));
    v = min(v, dpp_i<kDppXor2>(v));
    v = min(v, dpp_i<kDppHalfMirror>(v));
    v = min(v, dpp_i<kDppMirror>(v));
    return min(min(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
               min(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}
__device__ __forceinline__ int wave_sum_i(int v) {
    v += dpp_i<kDppXor1>(v);
    v += dpp_i<kDppXor2>(v);
    v += dpp_i<kDppHalfMirror>(v);
    v += dpp_i<kDppMirror>(v);
    return (__builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16)) +
           (__builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48));
}
// Butterfly sum over the 64 lanes: lane l adds lane l^m for m = 1, 2, 4, 8,
// 16, 32 (see above); the result is the same in every lane.
__device__ __forceinline__ float wave_butterfly_sum(float v) {
    v = v + dpp_f<kDppXor1>(v);
    v = v + dpp_f<kDppXor2>(v);
    v = v + dpp_f<kDppHalfMirror>(v);
    v = v + dpp_f<kDppMirror>(v);
    const float r0 = readlane_f(v, 0), r1 = readlane_f(v, 16), r2 = readlane_f(v, 32), r3 = readlane_f(v, 48);
    return (r0 + r1) + (r2 + r3);
}

// Inclusive prefix sum over the 64 lanes by DPP (no LDS): Hillis-Steele
// within each row of 16 (row_shr 1, 2, 4, 8; lanes shifted in from outside
// the row add 0), then row_bcast 15 into rows 1 and 3 and row_bcast 31 into
// rows 2 and 3.
__device__ __forceinline__ int wave_prefix_sum(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);
    return v;
}

__device__ __forceinline__ void flag_or(uint32_t* sticky, uint32_t bits) {
    if (bits) atomicOr(sticky, bits);
}

// A code word of a weight stream that one launch reads once: a non-temporal
// load, so the stream does not displace the lines other blocks still use
// (measured on the decode paths: N=32 gate-up 33.3 -> 32.0 us and down 20.6
// -> 19.4 us, the single-token layer 12.5 -> 12.1 us and its router rows
// (load_once4) 11.85 -> 11.55 us more, the one-row dense linear 5.9 -> 5.45
// us; the W8 head at 1-8 rows got slower and keeps plain loads there).
__device__ __forceinline__ uint32_t load_once(const uint32_t* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ uint4 load_once4(const void* p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v[0], v[1], v[2], v[3]);
}

// ---- 4-bit weight unpacking -----------------------------------------------
// A packed code word holds K values 8c..8c+7, low nibble first
// (dense_g256_api.h:25).  Even codes (k = 8c, 8c+2, 8c+4, 8c+6) go to the
// bytes of the first word and odd codes to the bytes of the second: this is
// the byte order the A8 activation layout uses, so both feed v_dot4 and the
// i8 MFMA directly.
__device__ __forceinline__ int code_even(uint32_t w) { return int(w & 0x0f0f0f0fu); }
__device__ __forceinline__ int code_odd(uint32_t w) { return int((w >> 4) & 0x0f0f0f0fu); }
__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// ---- Layout of quantized activations (this library's own format) ------------
// For row r and K chunk c (8 values k = 8c..8c+7) two int32 words are stored
// at word index r*(K/4) + 2c and 2c+1: bytes (q[8c], q[8c+2], q[8c+4], q[8c+6])
// and (q[8c+1], q[8c+3], q[8c+5], q[8c+7]).  Per 256-group: fp16 scale and
// int32 sum of q, as in the reference (routed_storage_n32_consumer.cpp:75).

// Group-256 activation quantisation on one wave.  Lane l holds the four
// transformed values k = 4l..4l+3 of the group in v[0..3].  Implements the
// absmax / fp16 scale / round-even / clamp recipe of
// routed_storage_n32_consumer.cpp:44-76 with any qmax, writes this library's
// int8 layout (64 words), the scale and the sum.
template <int QMAX>
__device__ __forceinline__ void quantize_group_wave(float v[4], uint32_t* words, uint16_t* scale_out,
                                                    int32_t* sum_out, uint32_t& flags, uint32_t invalid_flag) {
    const int lane = threadIdx.x & 63;
    float absmax = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (!isfinite(v[i])) { flags |= invalid_flag; v[i] = 0.f; }
        absmax = fmaxf(absmax, fabsf(v[i]));
    }
    absmax = wave_max(absmax);
    const float raw = fdiv_rn(absmax, float(QMAX));
    const bool valid = isfinite(raw) && raw <= 65504.f;
    if (!valid) flags |= invalid_flag;
    const bool zero = absmax == 0.f || !valid;
    const uint16_t sbits = f32_to_f16_bits(zero ? 1.f : fmaxf(raw, 0x1p-14f));
    const float scale = f16_bits_to_f32(sbits);
    int q[4], sum = 0;
    const int keep = zero ? 0 : -1;            // scale is 1 when zero: the division is harmless
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // v is finite and |v / scale| <= QMAX + 1/2 unless the group is zero (scale 1):
        // round, clamp in float, then convert (always in range)
        const float qf = fminf(fmaxf(__builtin_rintf(fdiv_rn(v[i], scale)), -float(QMAX)), float(QMAX));
        const int t = int(qf) & keep;
        q[i] = t;
        sum += t;
    }
    sum = wave_sum_i(sum);
    // lane 2c holds q[8c..8c+3], lane 2c+1 holds q[8c+4..8c+7].
    const uint32_t ev = (uint32_t(q[0]) & 255u) | ((uint32_t(q[2]) & 255u) << 8);
    const uint32_t od = (uint32_t(q[1]) & 255u) | ((uint32_t(q[3]) & 255u) << 8);
    const uint32_t pev = uint32_t(xor_perm_i<1>(int(ev)));
    const uint32_t pod = uint32_t(xor_perm_i<1>(int(od)));
    const uint32_t word = (lane & 1) ? (pod | (od << 16)) : (ev | (pev << 16));
    words[lane] = word;
    if (lane == 0) { *scale_out = sbits; *sum_out = sum; }
}

// One cross-lane butterfly step: pairs lanes l and l^M; the lane with the
// bit set keeps partner - own (src[lo] - src[hi]), the other own + partner.
template <int M> __device__ __forceinline__ void h128_lane_step(float v[4], int lane) {
    const bool upper = lane & M;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float p = xor_perm_f<M>(v[i]);
        v[i] = upper ? (p - v[i]) : (v[i] + p);
    }
}

// 128-point Hadamard transform of two blocks held by one wave: lane l holds
// k = 4l..4l+3 of a 256-value group (block = l/32).  Seven ascending
// butterflies exactly as routed_storage_n32_consumer.cpp:34-41, then the
// 0x3db504f3 scale.
__device__ __forceinline__ void h128_wave(float v[4]) {
    const int lane = threadIdx.x & 63;
    // step 1 (k bit 0)
    float a0 = v[0] + v[1], a1 = v[0] - v[1], a2 = v[2] + v[3], a3 = v[2] - v[3];
    // step 2 (k bit 1)
    v[0] = a0 + a2; v[2] = a0 - a2; v[1] = a1 + a3; v[3] = a1 - a3;
    // steps 4..64 (k bits 2..6 = lane bits 0..4)
    h128_lane_step<1>(v, lane);
    h128_lane_step<2>(v, lane);
    h128_lane_step<4>(v, lane);
    h128_lane_step<8>(v, lane);
    h128_lane_step<16>(v, lane);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = v[i] * kInvSqrt128;
}

// ---- half-wave group layout ------------------------------------------------
// One 256-value group on 32 lanes: lane l' = lane & 31 holds k = 8l'..8l'+7,
// so a wave holds two groups (lanes 0-31 and 32-63).  Every cross-lane step
// of the H128 stays inside a 16-lane row (DPP only).

// 128-point Hadamard of the two 128-blocks of a group (k bit 7 = lane bit 4):
// seven ascending butterflies exactly as routed_storage_n32_consumer.cpp:34-41
// (k bits 0..2 in registers, 3..6 = lane bits 0..3), then 0x3db504f3.
__device__ __forceinline__ void h128_half(float v[8]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int b = 1; b < 8; b <<= 1) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (i & b) continue;
            const float lo = v[i], hi = v[i + b];
            v[i] = lo + hi;
            v[i + b] = lo - hi;
        }
    }
    h128_lane_step<1>(v, lane);
    h128_lane_step<1>(v + 4, lane);
    h128_lane_step<2>(v, lane);
    h128_lane_step<2>(v + 4, lane);
    h128_lane_step<4>(v, lane);
    h128_lane_step<4>(v + 4, lane);
    h128_lane_step<8>(v, lane);
    h128_lane_step<8>(v + 4, lane);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = v[i] * kInvSqrt128;
}

// ---- Quarter-wave groups: 16 lanes, 16 values per lane ------------------------
// Lane l (= threadIdx.x & 15) of a 16-lane quarter (one DPP row) holds the 16
// consecutive values k = quarter_base(l) + i of its 256-group.  Lane bits 0, 1
// and 3 are k bits 4, 5 and 6, lane bit 2 is k bit 7: every H128 butterfly is
// in-register (k bits 0..3) or a single DPP lane exchange (xor 1, 2, 8), and
// the two 128-blocks (k bit 7) never exchange.
__device__ __forceinline__ int quarter_base(int l) {
    return 16 * ((l & 3) | (((l >> 3) & 1) << 2) | (((l >> 2) & 1) << 3));
}
template <int N> __device__ __forceinline__ float row_ror_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + N, 0xF, 0xF, false));
}
template <int N> __device__ __forceinline__ int row_ror_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, 0x120 + N, 0xF, 0xF, false);
}
// Cross-lane butterfly on lane bit M: the lane with the bit clear keeps
// lo + hi, the other lo - hi.  partner + (+-v), the sign flipped on the upper
// lane, is exactly both (a + (-b) == a - b in IEEE arithmetic).
template <int M> __device__ __forceinline__ void h128_quarter_step(float v[16]) {
    const uint32_t flip = (threadIdx.x & M) ? 0x80000000u : 0u;
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = xor_perm_f<M>(v[i]) + __uint_as_float(__float_as_uint(v[i]) ^ flip);
}
// H128 of both 128-blocks of the quarter's group (butterflies on k bits 0..6
// in ascending order), then x 1/sqrt(128).
__device__ __forceinline__ void h128_quarter(float v[16]) {
#pragma unroll
    for (int b = 1; b < 16; b <<= 1) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            if (i & b) continue;
            const float lo = v[i], hi = v[i + b];
            v[i] = lo + hi;
            v[i + b] = lo - hi;
        }
    }
    h128_quarter_step<1>(v);
    h128_quarter_step<2>(v);
    h128_quarter_step<8>(v);
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = v[i] * kInvSqrt128;
}
// Group-256 quantisation of a quarter (the recipe of quantize_group_wave).
// Every lane gets the group's fp16 scale bits and the sum of q; words[0..3]
// are activation words 2c..2c+3 of its chunks c = quarter_base(l) / 8 + 0, 1.
template <int QMAX>
__device__ __forceinline__ void quantize_quarter(float v[16], uint32_t words[4], uint16_t& sbits_out, int& sum_out,
                                                 uint32_t& flags, uint32_t invalid_flag) {
    float absmax = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        if (!isfinite(v[i])) { flags |= invalid_flag; v[i] = 0.f; }
        absmax = fmaxf(absmax, fabsf(v[i]));
    }
    // lanes i, i-4, i-8, i-12 of the row, then xor 1, 2: all 16 lanes
    absmax = fmaxf(absmax, row_ror_f<4>(absmax));
    absmax = fmaxf(absmax, row_ror_f<8>(absmax));
    absmax = fmaxf(absmax, xor_perm_f<1>(absmax));
    absmax = fmaxf(absmax, xor_perm_f<2>(absmax));
    const float raw = fdiv_rn(absmax, float(QMAX));
    const bool valid = isfinite(raw) && raw <= 65504.f;
    if (!valid) flags |= invalid_flag;
    const bool zero = absmax == 0.f || !valid;
    const uint16_t sbits = f32_to_f16_bits(zero ? 1.f : fmaxf(raw, 0x1p-14f));
    const float scale = f16_bits_to_f32(sbits);
    int q[16], sum = 0;
    const int keep = zero ? 0 : -1;            // scale is 1 when zero: the division is harmless
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        // v is finite and |v / scale| <= QMAX + 1/2 unless the group is zero (scale 1):
        // round, clamp in float, then convert (always in range)
        const float qf = fminf(fmaxf(__builtin_rintf(fdiv_rn(v[i], scale)), -float(QMAX)), float(QMAX));
        const int t = int(qf) & keep;
        q[i] = t;
        sum += t;
    }
    sum += row_ror_i<4>(sum);
    sum += row_ror_i<8>(sum);
    sum += xor_perm_i<1>(sum);
    sum += xor_perm_i<2>(sum);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const int* qc = q + 8 * c;
        words[2 * c] = (uint32_t(qc[0]) & 255u) | ((uint32_t(qc[2]) & 255u) << 8) | ((uint32_t(qc[4]) & 255u) << 16) |
                       ((uint32_t(qc[6]) & 255u) << 24);
        words[2 * c + 1] = (uint32_t(qc[1]) & 255u) | ((uint32_t(qc[3]) & 255u) << 8) |
                           ((uint32_t(qc[5]) & 255u) << 16) | ((uint32_t(qc[7]) & 255u) << 24);
    }
    sbits_out = sbits;
    sum_out = sum;
}

// quantize_quarter with the arithmetic of quantize_half_fast (one fma per
// value detects non-finite values, which OR nonfinite_flags and are zeroed;
// q = rint(v * RN(1/scale)) with the exact fallback near half-integers):
// the same words, scale and sum.
template <int QMAX>
__device__ __forceinline__ void quantize_quarter_fast(float v[16], uint32_t words[4], uint16_t& sbits_out,
                                                      int& sum_out, uint32_t& flags, uint32_t nonfinite_flags,
                                                      uint32_t invalid_flag) {
    float fin = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) fin = __builtin_fmaf(v[i], 0.f, fin);
    if (fin != fin) {
        flags |= nonfinite_flags;
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = isfinite(v[i]) ? v[i] : 0.f;
    }
    float absmax = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) absmax = fmaxf(absmax, fabsf(v[i]));
    absmax = fmaxf(absmax, row_ror_f<4>(absmax));
    absmax = fmaxf(absmax, row_ror_f<8>(absmax));
    absmax = fmaxf(absmax, xor_perm_f<1>(absmax));
    absmax = fmaxf(absmax, xor_perm_f<2>(absmax));
    const float raw = fdiv_rn(absmax, float(QMAX));
    const bool valid = isfinite(raw) && raw <= 65504.f;
    if (!valid) flags |= invalid_flag;
    const bool zero = absmax == 0.f || !valid;
    const uint16_t sbits = f32_to_f16_bits(zero ? 1.f : fmaxf(raw, 0x1p-14f));
    const float scale = f16_bits_to_f32(sbits);
    const float rs = fdiv_rn(1.f, scale);
    float qf[16];
    bool near = false;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float r = v[i] * rs;
        const float n = __builtin_rintf(r);
        near |= 0.5f - fabsf(r - n) <= 0x1p-14f;
        qf[i] = n;
    }
    if (near) {
#pragma unroll
        for (int i = 0; i < 16; ++i) qf[i] = __builtin_rintf(fdiv_rn(v[i], scale));
    }
    int q[16], sum = 0;
    const int keep = zero ? 0 : -1;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        q[i] = int(fminf(fmaxf(qf[i], -float(QMAX)), float(QMAX))) & keep;
        sum += q[i];
    }
    sum += row_ror_i<4>(sum);
    sum += row_ror_i<8>(sum);
    sum += xor_perm_i<1>(sum);
    sum += xor_perm_i<2>(sum);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const int* qc = q + 8 * c;
        words[2 * c] = (uint32_t(qc[0]) & 255u) | ((uint32_t(qc[2]) & 255u) << 8) | ((uint32_t(qc[4]) & 255u) << 16) |
                       ((uint32_t(qc[6]) & 255u) << 24);
        words[2 * c + 1] = (uint32_t(qc[1]) & 255u) | ((uint32_t(qc[3]) & 255u) << 8) |
                           ((uint32_t(qc[5]) & 255u) << 16) | ((uint32_t(qc[7]) & 255u) << 24);
    }
    sbits_out = sbits;
    sum_out = sum;
}

// Group quantisation of the half-wave layout (same arithmetic as
// quantize_group_wave).  Every lane of the half gets the group's fp16 scale
// bits and Σq; lane l' gets its two activation words 2l' = (q0,q2,q4,q6) and
// 2l'+1 = (q1,q3,q5,q7) of its chunk.
template <int QMAX>
__device__ __forceinline__ void quantize_half(float v[8], uint32_t words[2], uint16_t& sbits_out, int& sum_out,
                                              uint32_t& flags, uint32_t invalid_flag) {
    float absmax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        if (!isfinite(v[i])) { flags |= invalid_flag; v[i] = 0.f; }
        absmax = fmaxf(absmax, fabsf(v[i]));
    }
    absmax = fmaxf(absmax, xor_perm_f<1>(absmax));
    absmax = fmaxf(absmax, xor_perm_f<2>(absmax));
    absmax = fmaxf(absmax, xor_perm_f<4>(absmax));
    absmax = fmaxf(absmax, xor_perm_f<8>(absmax));
    absmax = fmaxf(absmax, xor_perm_f<16>(absmax));
    const float raw = fdiv_rn(absmax, float(QMAX));
    const bool valid = isfinite(raw) && raw <= 65504.f;
    if (!valid) flags |= invalid_flag;
    const bool zero = absmax == 0.f || !valid;
    const uint16_t sbits = f32_to_f16_bits(zero ? 1.f : fmaxf(raw, 0x1p-14f));
    const float scale = f16_bits_to_f32(sbits);
    int q[8], sum = 0;
    const int keep = zero ? 0 : -1;            // scale is 1 when zero: the division is harmless
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        // v is finite and |v / scale| <= QMAX + 1/2 unless the group is zero (scale 1):
        // round, clamp in float, then convert (always in range)
        const float qf = fminf(fmaxf(__builtin_rintf(fdiv_rn(v[i], scale)), -float(QMAX)), float(QMAX));
        const int t = int(qf) & keep;
        q[i] = t;
        sum += t;
    }
    sum += xor_perm_i<1>(sum);
    sum += xor_perm_i<2>(sum);
    sum += xor_perm_i<4>(sum);
    sum += xor_perm_i<8>(sum);
    sum += xor_perm_i<16>(sum);
    words[0] = (uint32_t(q[0]) & 255u) | ((uint32_t(q[2]) & 255u) << 8) | ((uint32_t(q[4]) & 255u) << 16) |
               ((uint32_t(q[6]) & 255u) << 24);
    words[1] = (uint32_t(q[1]) & 255u) | ((uint32_t(q[3]) & 255u) << 8) | ((uint32_t(q[5]) & 255u) << 16) |
               ((uint32_t(q[7]) & 255u) << 24);
    sbits_out = sbits;
    sum_out = sum;
}

// One cross-lane H128 butterfly on lane bit M for a single value: the lane
// with the bit clear keeps lo + hi, the other lo - hi (partner + (+-own), the
// sign flipped on the upper lane; a + (-b) == a - b in IEEE arithmetic).
template <int M> __device__ __forceinline__ float butterfly_lane(float v) {
    const uint32_t flip = (threadIdx.x & M) ? 0x80000000u : 0u;
    return xor_perm_f<M>(v) + __uint_as_float(__float_as_uint(v) ^ flip);
}

// quantize_half with the same results and fewer operations:
//  - one fma(v, 0, acc) per value detects a non-finite value (the product is
//    NaN exactly for inf and NaN); such lanes OR nonfinite_flags and zero
//    those values, as quantize_half does with its invalid flag;
//  - q = rint(RN(v / scale)) is taken as rint(v * RN(1 / scale)).  In a valid
//    group |v / scale| <= QMAX * (1 + 2^-10) < 128, so the product lies within
//    2^-16 of v / scale and the correctly rounded quotient within 2^-17 of
//    it: both round to the same integer unless the product lies within 2^-14
//    of a half-integer (0.5 - |r - rint(r)| is exact).  Lanes holding such a
//    value (rare) redo their eight with the correctly rounded division.  An
//    invalid or zero group uses scale 1 and masks q to 0 as before.
template <int QMAX>
__device__ __forceinline__ void quantize_half_fast(float v[8], uint32_t words[2], uint16_t& sbits_out, int& sum_out,
                                                   uint32_t& flags, uint32_t nonfinite_flags, uint32_t invalid_flag) {
    float fin = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) fin = __builtin_fmaf(v[i], 0.f, fin);
    if (fin != fin) {
        flags |= nonfinite_flags;
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = isfinite(v[i]) ? v[i] : 0.f;
    }
    float absmax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) absmax = fmaxf(absmax, fabsf(v[i]));
    absmax = fmaxf(absmax, xor_perm_f<1>(absmax));
    absmax = fmaxf(absmax, xor_perm_f<2>(absmax));
    absmax = fmaxf(absmax, xor_perm_f<4>(absmax));
    absmax = fmaxf(absmax, xor_perm_f<8>(absmax));
    absmax = fmaxf(absmax, xor_perm_f<16>(absmax));
    const float raw = fdiv_rn(absmax, float(QMAX));
    const bool valid = isfinite(raw) && raw <= 65504.f;
    if (!valid) flags |= invalid_flag;
    const bool zero = absmax == 0.f || !valid;
    const uint16_t sbits = f32_to_f16_bits(zero ? 1.f : fmaxf(raw, 0x1p-14f));
    const float scale = f16_bits_to_f32(sbits);
    const float rs = fdiv_rn(1.f, scale);
    float qf[8];
    bool near = false;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float r = v[i] * rs;
        const float n = __builtin_rintf(r);
        near |= 0.5f - fabsf(r - n) <= 0x1p-14f;
        qf[i] = n;
    }
    if (near) {
#pragma unroll
        for (int i = 0; i < 8; ++i) qf[i] = __builtin_rintf(fdiv_rn(v[i], scale));
    }
    int q[8], sum = 0;
    const int keep = zero ? 0 : -1;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int t = int(fminf(fmaxf(qf[i], -float(QMAX)), float(QMAX))) & keep;
        q[i] = t;
        sum += t;
    }
    sum += xor_perm_i<1>(sum);
    sum += xor_perm_i<2>(sum);
    sum += xor_perm_i<4>(sum);
    sum += xor_perm_i<8>(sum);
    sum += xor_perm_i<16>(sum);
    words[0] = (uint32_t(q[0]) & 255u) | ((uint32_t(q[2]) & 255u) << 8) | ((uint32_t(q[4]) & 255u) << 16) |
               ((uint32_t(q[6]) & 255u) << 24);
    words[1] = (uint32_t(q[1]) & 255u) | ((uint32_t(q[3]) & 255u) << 8) | ((uint32_t(q[5]) & 255u) << 16) |
               ((uint32_t(q[7]) & 255u) << 24);
    sbits_out = sbits;
    sum_out = sum;
}

// ---- strided half-wave layout of the single-token middle row ---------------
// Lane l' = lane & 31 of a 256-group holds k = strided_base(l') + 16 j,
// j = 0..7: k bits 0..3 and 7 come from the lane, k bits 4..6 from j, so the
// H128 butterflies left after the producer's k bits 0..3 are in-register.
__device__ __forceinline__ int strided_base(int l) { return (l & 15) | ((l >> 4) << 7); }
__device__ __forceinline__ void h128_tail_strided(float v[8]) {
#pragma unroll
    for (int b = 1; b < 8; b <<= 1) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (i & b) continue;
            const float lo = v[i], hi = v[i + b];
            v[i] = lo + hi;
            v[i + b] = lo - hi;
        }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = v[i] * kInvSqrt128;
}
// quantize_half_fast's arithmetic on the strided layout: q[j] of value j (the
// caller places the bytes), fp16 scale bits and the group's sum of q.
template <int QMAX>
__device__ __forceinline__ void quantize_strided(float v[8], int q[8], uint16_t& sbits_out, int& sum_out,
                                                 uint32_t& flags, uint32_t nonfinite_flags, uint32_t invalid_flag) {
    float fin = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) fin = __builtin_fmaf(v[i], 0.f, fin);
    if (fin != fin) {
        flags |= nonfinite_flags;
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = isfinite(v[i]) ? v[i] : 0.f;
    }
    float absmax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) absmax = fmaxf(absmax, fabsf(v[i]));
    absmax = fmaxf(absmax, xor_perm_f<1>(absmax));
    absmax = fmaxf(absmax, xor_perm_f<2>(absmax));
    absmax = fmaxf(absmax, xor_perm_f<4>(absmax));
    absmax = fmaxf(absmax, xor_perm_f<8>(absmax));
    absmax = fmaxf(absmax, xor_perm_f<16>(absmax));
    const float raw = fdiv_rn(absmax, float(QMAX));
    const bool valid = isfinite(raw) && raw <= 65504.f;
    if (!valid) flags |= invalid_flag;
    const bool zero = absmax == 0.f || !valid;
    const uint16_t sbits = f32_to_f16_bits(zero ? 1.f : fmaxf(raw, 0x1p-14f));
    const float scale = f16_bits_to_f32(sbits);
    const float rs = fdiv_rn(1.f, scale);
    float qf[8];
    bool near = false;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float r = v[i] * rs;
        const float n = __builtin_rintf(r);
        near |= 0.5f - fabsf(r - n) <= 0x1p-14f;
        qf[i] = n;
    }
    if (near) {
#pragma unroll
        for (int i = 0; i < 8; ++i) qf[i] = __builtin_rintf(fdiv_rn(v[i], scale));
    }
    int sum = 0;
    const int keep = zero ? 0 : -1;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        q[i] = int(fminf(fmaxf(qf[i], -float(QMAX)), float(QMAX))) & keep;
        sum += q[i];
    }
    sum += xor_perm_i<1>(sum);
    sum += xor_perm_i<2>(sum);
    sum += xor_perm_i<4>(sum);
    sum += xor_perm_i<8>(sum);
    sum += xor_perm_i<16>(sum);
    sbits_out = sbits;
    sum_out = sum;
}

// fp32 group tree term of one (row, column, group) (dense_g256_api.h:35-37):
// RN(sw*RN(sa*dot)) + RN(off*RN(sa*sum)), returned unrounded-sum-ready.
__device__ __forceinline__ float tree_term(int dot, float sa, float scaled_sum, uint32_t meta) {
    const float sw = f16_bits_to_f32(meta & 0xffffu), off = f16_bits_to_f32(meta >> 16);
    const float scaled_dot = sa * float(dot);
    const float product = sw * scaled_dot;
    const float correction = off * scaled_sum;
    return product + correction;
}

}  // namespace ornith
