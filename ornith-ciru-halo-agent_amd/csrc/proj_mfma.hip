// Grouped G256 projection on the int8 matrix cores (prefill path, T > 32).
//
// Arithmetic is the reference's A8/A4 routed math, exactly
// (routed_storage_n32_prefill.h:43-149 computes the same per-group integer
// dots with WMMA-iu4, routed_storage_n32_consumer.cpp:152-157 the tree):
// per (route, column, 256-group) the integer dot sum_k code*q is formed by
// v_mfma_i32_16x16x64_i8 (exact: |dot| < 2^19), then the fp32 group tree
// value = value + (RN(sw*RN(sa*dot)) + RN(off*RN(sa*sum))) runs in ascending
// group order on the VALU.
//
// MFMA operand layout (verified on gfx950): lane i+16q supplies the 16 bytes
// of row/column i for k-group q, A and B bytes pair positionally, and output
// register r of lane l is C[4*(l/16)+r][l%16].  Both operands use this
// build's byte order (even codes then odd codes per 8-value chunk), so the
// logical k pairing matches and the integer dot is exact.
//
// The same kernel body serves the routed gate/up and down projections of the
// permuted routes and the quantised LM head (one row tile of up to 64 rows
// over the whole vocabulary, logits and per-block argmax partials out).
#include "kernels.hpp"
#include "timing.hpp"
#include "decode.hpp"
#include <algorithm>
#include <utility>

namespace ornith {

constexpr int kMT = 64, kNT = 128;   // routes per m-tile, columns per column block

// Integer dots start from the bits of kDotBias = 1.5 * 2^23, so the int32
// result read as fp32 is kDotBias + dot exactly (|dot| < 2^19 << 2^22); with
// nb = -sa * kDotBias (exact: sa is an fp16 value, 11 significant bits, and
// kDotBias = 3 * 2^22) fma(sa, kDotBias + dot, nb) rounds sa * dot once:
// RN(sa * dot) without an integer-to-float conversion.
constexpr float kDotBias = 12582912.0f;
constexpr int kDotBiasBits = 0x4B400000;

typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kModeGateUp = 0, kModeDown = 1, kModeHead = 2;

// Top-1 order of numpy's argmax: the first NaN if any, else the first maximum.
__device__ __forceinline__ bool arg_better(float a, int ia, float b, int ib) {
    const bool na = isnan(a), nb = isnan(b);
    if (na != nb) return na;
    if (na) return ia < ib;
    return a > b || (a == b && ia < ib);
}
// The same order without branches (lane masks combined bitwise), for
// reductions across lanes.
__device__ __forceinline__ bool arg_better_select(float a, int ia, float b, int ib) {
    const bool na = a != a, nb = b != b, first = ia < ib;
    return (na & (!nb | first)) | (!na & !nb & ((a > b) | ((a == b) & first)));
}

// Per-row combination of the head's block partials (numpy argmax rule).
__global__ __launch_bounds__(256) void head_argmax_kernel(const float* __restrict__ val, const int32_t* __restrict__ idx,
                                                          int nblk, int64_t* __restrict__ out) {
    __shared__ float bv[256];
    __shared__ int bi[256];
    const int row = blockIdx.x, t = threadIdx.x;
    float v = 0.f;
    int i = 0x7fffffff;
    // eight independent loads per thread per round (2048 partials per round)
    for (int b0 = 0; b0 < nblk; b0 += 8 * 256) {
        float ov[8];
        int oi[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int b = b0 + 256 * u + t;
            ov[u] = b < nblk ? val[size_t(row) * nblk + b] : 0.f;
            oi[u] = b < nblk ? idx[size_t(row) * nblk + b] : 0x7fffffff;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (oi[u] != 0x7fffffff && (i == 0x7fffffff || arg_better(ov[u], oi[u], v, i))) { v = ov[u]; i = oi[u]; }
    }
    bv[t] = v;
    bi[t] = i;
    __syncthreads();
    for (int m = 128; m > 0; m >>= 1) {
        if (t < m) {
            const int o = t + m;
            if (bi[o] != 0x7fffffff && (bi[t] == 0x7fffffff || arg_better(bv[o], bi[o], bv[t], bi[t]))) {
                bv[t] = bv[o];
                bi[t] = bi[o];
            }
        }
        __syncthreads();
    }
    if (t == 0) out[row] = bi[0];
}

// ---------------------------------------------------------------------------
// Prefill projections with column-owning waves.
//
// Block = (64-route m-tile, column block).  Wave w owns two 16-column tiles
// over all 64 rows, so every code word is fetched and unpacked once per block:
//  - B: each lane loads its own packed code words straight into registers.
//    Lane i+16q of column tile ct takes, for k-step s (64 k), the words
//    j = 8s+2q and 8s+2q+1 (chunks of 8 codes) of its column; unpacked
//    (even codes, odd codes) they are the 16 operand bytes of that lane.
//  - A: the tile's activation rows of one 256-group per step are staged in
//    LDS through registers; 16-byte piece p of row r sits at slot p ^ (r & 15),
//    so the 16 rows read by one k-group of lanes hit distinct banks.  Lane
//    i+16q reads activation words 2j..2j+3 of row i, the same chunks j.
// Gate/up: block nt covers middle columns 64nt..64nt+63; wave w's tiles are
// gate and up of columns 64nt+16w+i, so a lane forms SiLU(gate)*up itself and
// writes the middle row of the route's position in the permuted order.
// Down: a block covers NSUB x 128 output columns of its m-tile; both groups of
// A (K = 512) stay in LDS while the column blocks are walked.
//
// Steps (one 256-group of one column block each) are unrolled, so the
// register rings have compile-time slots and every load wait is exact.  A
// moves global -> registers (loaded one step before its store) -> LDS
// (stored two steps before its dots, three stages) -> MFMA; codes are DB
// steps ahead.  Matrix-core and VALU work of one SIMD do not overlap on
// gfx950 (measured), so a step runs its dots and then its tree, and the
// register budget goes to occupancy instead: gate/up holds two blocks per
// CU, down (one code slot) three.  The step body is instantiated for 1, 2
// and 4 row tiles of 16 rows, so partial tiles skip dead row tiles without
// branches.
// ---------------------------------------------------------------------------
template <int MODE, int GS, int NSUB, int DB, int MAXL = 4>
__global__ __launch_bounds__(256, MODE == kModeDown ? 3 : 2) void prefill_mfma_kernel(MfmaArgs a) {
    constexpr bool GATEUP = MODE == kModeGateUp, HEAD = MODE == kModeHead;
    constexpr bool BIAS = GATEUP || HEAD;                     // dots start from kDotBias
    constexpr int NSTEP = GS * NSUB;
    constexpr int KW = GS * 64;                               // activation words per row
    constexpr int NCB = GATEUP ? (2 * kInter) / kNT : kHidden / (kNT * NSUB);
    constexpr int NSTAGE = GS < 3 ? GS : 3;                   // A stages in LDS
    constexpr int NSC = NSTAGE;                               // scale stages (with their A words)
    static_assert(GS >= 2, "two A stages are filled in the prologue");
    __shared__ __attribute__((aligned(16))) uint32_t sA[NSTAGE][kMT * 64];
    __shared__ __attribute__((aligned(16))) float s_sa[NSC][kMT];
    __shared__ __attribute__((aligned(16))) float s_ss[NSC][kMT];
    __shared__ __attribute__((aligned(16))) float s_nb[BIAS ? NSC : 1][kMT];   // -sa * kDotBias (exact)
    __shared__ int s_route[kMT];
    __shared__ float s_bv[HEAD ? 4 : 1][kMT];                 // head: per-wave row best
    __shared__ int s_bi[HEAD ? 4 : 1][kMT];

    // Workgroups go to the 8 XCDs round-robin (linear block L runs on XCD
    // L % 8).  Three block orders:
    //  - column-block major (a.tile_xcd == 0): nt = L % NCB.  Every XCD runs
    //    one column slice of every tile (even load; each XCD streams all the
    //    tiles' activation rows);
    //  - tile per XCD (a.tile_xcd == 1): L = 8 * NCB * q + 8 * nt + x runs
    //    m-tile 8q + x, so all column blocks of a tile share one L2 (its
    //    activation rows are fetched once) and each XCD walks every 8th tile.
    //    At large T (full tiles, heavy experts) this cuts the L2 misses ~3x.
    //  - tile ranges per XCD (a.tile_xcd == 2): the same L, XCD x runs the
    //    contiguous m-tiles [x per, (x + 1) per), per = ceil(ntiles / 8), so
    //    an expert's consecutive m-tiles also share its weights in one L2.
    //    Measured: down at 1120 tokens 38.7 -> 36.8 us; at 8192 tokens down
    //    200.7 -> 204.6 and gate-up 352 -> 368 us, which keep orders 0 and 1.
    // Head: one m-tile of the a.R input rows, block L = column block L.
    const int L = int(blockIdx.x);
    int nt, mtile;
    Segment td;
    if constexpr (HEAD) {
        nt = L;
        mtile = 0;
        td = Segment{0, 0, a.R, 0};
    } else {
        const int ntiles = a.ntiles[0];
        if (a.tile_xcd == 2) {
            const int per = (ntiles + 7) >> 3, q = L / (8 * NCB);
            nt = (L >> 3) % NCB;
            mtile = (L & 7) * per + q;
            if (q >= per) return;
        } else {
            nt = a.tile_xcd ? (L >> 3) % NCB : L % NCB;
            mtile = a.tile_xcd ? 8 * (L / (8 * NCB)) + (L & 7) : L / NCB;
        }
        if (mtile >= ntiles) return;
        td = a.tiles[mtile];
    }
    const int bank = td.bank, first = td.first, nrows = td.count;
    const bool shared = !HEAD && bank == kShared;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, li = lane & 15, q = lane >> 4;
    const uint32_t* codes = shared ? a.shared_codes : a.codes + size_t(bank) * a.bank_words;
    const uint32_t* meta = shared ? a.shared_meta : a.meta + size_t(bank) * a.bank_meta_words;
    // the head and the shared expert read dense N32 banks
    const BankView bv = bank_view(HEAD || shared);

    // routes of this lane's A row (tid / 4) and scale row (tid % 64), first:
    // later waits on them must not wait on the code loads
    // (clamped to the route range: a malformed list gives wrong rows, never
    // an access outside the activation / output buffers)
    const int a_r = tid >> 2, a_part = tid & 3;
    const int rmax = a.R + (a.shared_codes ? a.R / kTop : 0) - 1;
    const int route_a = HEAD ? 0 : min(max(a.routes[first + min(a_r, nrows - 1)], 0), rmax);
    const int route_s = HEAD ? 0 : min(max(a.routes[first + min(tid & 63, nrows - 1)], 0), rmax);

    // ---- B: code words of step st for this lane ----
    // column tile ct of step st: 32-column code tile and the column in it
    auto b_tile = [&](int st, int ct, int& ntile, int& n) {
        if (GATEUP) {
            const int c = 64 * nt + 16 * w + li;
            ntile = (ct ? kInter / 32 : 0) + (c >> 5);
            n = c & 31;
        } else {
            // down / head: 32 columns per wave (the head's last block may
            // reach past N: its tiles repeat the last one, never stored)
            const int base = kNT * (nt * NSUB + st / GS);
            ntile = HEAD ? min((base >> 5) + w, a.N / 32 - 1) : (base >> 5) + w;
            n = 16 * ct + li;
        }
    };
    uint32_t bw[DB][2][8];          // [slot][ct][2s + e]
    uint32_t bm[DB][2];             // meta word (sw | off << 16) per column tile
    auto load_b = [&](int st, int slot) {
        const int g = st % GS;
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
            int ntile, n;
            b_tile(st, ct, ntile, n);
            const int col = 32 * ntile + n;
            const uint32_t* src = codes + bv.word(col, g, GS) + (2 * q) * bv.stride();
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                bw[slot][ct][2 * s] = src[(8 * s) * bv.stride()];
                bw[slot][ct][2 * s + 1] = src[(8 * s + 1) * bv.stride()];
            }
            bm[slot][ct] = meta[bv.meta(col, g, GS)];
        }
    };
#pragma unroll
    for (int st = 0; st < DB; ++st) load_b(st, st);

    // ---- rows of the tile (dead rows repeat the last live row; never written) ----
    // gate/up: activation row = token of the route; down: the permuted position
    auto act_row = [&](int r, int route) {
        return GATEUP ? (route < a.R ? route / kTop : route - a.R) : first + min(r, nrows - 1);
    };

    // ---- A: activation words of group g, 64 bytes per lane ----
    const uint32_t* a_src = a.act_words + size_t(act_row(a_r, route_a)) * KW + 16 * a_part;
    // register k of the staging thread holds piece 4 a_part + (k + a_part) % 4
    // of its row: the 8 lanes of each LDS store phase (2 rows x 4 parts) then
    // hit 8 distinct 16-byte bank groups
    auto a_piece = [&](int k) { return (k + a_part) & 3; };
    const size_t sa_base = size_t(act_row(tid & 63, route_s)) * GS;
    u32x4 ra[1][4];                 // one register slot: A(g) is loaded one step before its LDS store
    uint32_t rsa[1];
    int rsum[1];
    auto load_a = [&](int g, int slot) {
#pragma unroll
        for (int k = 0; k < 4; ++k) ra[slot][k] = *reinterpret_cast<const u32x4*>(a_src + g * 64 + 4 * a_piece(k));
        rsa[slot] = a.act_scales[sa_base + g];
        rsum[slot] = a.act_sums[sa_base + g];
    };
    auto store_a = [&](int slot, int stage, int g) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int piece = (4 * a_part + a_piece(k)) ^ (a_r & 15);
            *reinterpret_cast<u32x4*>(&sA[stage][a_r * 64 + 4 * piece]) = ra[slot][k];
        }
        if (tid < kMT) {
            const int sc = g % NSC;
            const float sa = f16_bits_to_f32(uint16_t(rsa[slot]));
            s_sa[sc][tid] = sa;
            s_ss[sc][tid] = sa * float(rsum[slot]);
            if constexpr (BIAS) s_nb[sc][tid] = -sa * kDotBias;
        }
    };
    // A(0) and A(1) in flight together (A(1) through prologue-only registers)
    u32x4 ra1[4];
    uint32_t rsa1;
    int rsum1;
    load_a(0, 0);
#pragma unroll
    for (int k = 0; k < 4; ++k) ra1[k] = *reinterpret_cast<const u32x4*>(a_src + 64 + 4 * a_piece(k));
    rsa1 = a.act_scales[sa_base + 1];
    rsum1 = a.act_sums[sa_base + 1];
    store_a(0, 0, 0);
#pragma unroll
    for (int k = 0; k < 4; ++k) ra[0][k] = ra1[k];
    rsa[0] = rsa1;
    rsum[0] = rsum1;
    store_a(0, 1, 1);
    if (!GATEUP && tid < kMT) s_route[tid] = tid < nrows ? route_s : -1;   // read after the first barrier
    if (GS > 2) load_a(2, 0);
    __syncthreads();

    uint32_t flags = 0;
    // L = row tiles with a live row (compile time, so the step body is branch-free)
    auto run = [&]<int L>() {
        float val[4][2][4];
#pragma unroll
        for (int rt = 0; rt < 4; ++rt)
#pragma unroll
            for (int ct = 0; ct < 2; ++ct)
#pragma unroll
                for (int r = 0; r < 4; ++r) val[rt][ct][r] = 0.f;
        i32x4 acc[1][4][2];
        float swv[1][2], offv[1][2];
        // gate/up and head dots start from kDotBias (see kDotBias); the down
        // kernel keeps the conversion (measured: the bias costs it more than it
        // saves there)
        constexpr i32x4 kAccInit = BIAS ? i32x4{kDotBiasBits, kDotBiasBits, kDotBiasBits, kDotBiasBits}
                                        : i32x4{0, 0, 0, 0};

        // matrix-core dots of step ST for the L live row tiles (rows past
        // nrows in them hold copies of a live row)
        auto mfma_step = [&]<int ST>() {
            constexpr int g = ST % GS, stage = g % NSTAGE, bslot = ST % DB, ab = 0;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                i32x4 fa[4], fb[2];
#pragma unroll
                for (int rt = 0; rt < L; ++rt) {
                    const int row = 16 * rt + li;
                    const u32x4 v = *reinterpret_cast<const u32x4*>(&sA[stage][row * 64 + 4 * ((4 * s + q) ^ li)]);
                    fa[rt] = i32x4{int(v.x), int(v.y), int(v.z), int(v.w)};
                }
#pragma unroll
                for (int ct = 0; ct < 2; ++ct) {
                    const uint32_t w0 = bw[bslot][ct][2 * s], w1 = bw[bslot][ct][2 * s + 1];
                    fb[ct] = i32x4{code_even(w0), code_odd(w0), code_even(w1), code_odd(w1)};
                }
#pragma unroll
                for (int rt = 0; rt < L; ++rt)
#pragma unroll
                    for (int ct = 0; ct < 2; ++ct)
                        acc[ab][rt][ct] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                            fa[rt], fb[ct], s ? acc[ab][rt][ct] : kAccInit, 0, 0, 0);
            }
            // the slot's scales are taken before the slot is refilled
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
                swv[ab][ct] = f16_bits_to_f32(uint16_t(bm[bslot][ct] & 0xffffu));
                offv[ab][ct] = f16_bits_to_f32(uint16_t(bm[bslot][ct] >> 16));
            }
            if constexpr (ST + DB < NSTEP) load_b(ST + DB, bslot);
        };

        // fp32 group tree of step ST (dense_g256_api.h:35-37), ascending groups
        auto tree_step = [&]<int ST>() {
            constexpr int g = ST % GS, sub = ST / GS, sc = g % NSC, ab = 0;
#pragma unroll
            for (int rt = 0; rt < L; ++rt) {
                const float4 sa4 = *reinterpret_cast<const float4*>(&s_sa[sc][16 * rt + 4 * q]);
                const float4 ss4 = *reinterpret_cast<const float4*>(&s_ss[sc][16 * rt + 4 * q]);
                const float4 nb4 = BIAS ? *reinterpret_cast<const float4*>(&s_nb[BIAS ? sc : 0][16 * rt + 4 * q])
                                        : float4{0.f, 0.f, 0.f, 0.f};
                const float sa[4] = {sa4.x, sa4.y, sa4.z, sa4.w}, ss[4] = {ss4.x, ss4.y, ss4.z, ss4.w};
                const float nb[4] = {nb4.x, nb4.y, nb4.z, nb4.w};
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int ct = 0; ct < 2; ++ct) {
                        // gate/up: acc holds the bits of kDotBias + dot, one fma gives RN(sa * dot)
                        const float scaled_dot = BIAS ? __builtin_fmaf(sa[r], __int_as_float(acc[ab][rt][ct][r]), nb[r])
                                                      : sa[r] * float(acc[ab][rt][ct][r]);
                        const float product = swv[ab][ct] * scaled_dot;
                        const float correction = offv[ab][ct] * ss[r];
                        val[rt][ct][r] = val[rt][ct][r] + (product + correction);
                    }
            }
            // keep each step's tree in its step: sinking it would keep every
            // step's accumulators alive at once
#pragma unroll
            for (int rt = 0; rt < L; ++rt)
#pragma unroll
                for (int ct = 0; ct < 2; ++ct)
#pragma unroll
                    for (int r = 0; r < 4; ++r) asm volatile("" : "+v"(val[rt][ct][r]));
            if constexpr (g == GS - 1) {
                // ---- epilogue of one column block ----
                if constexpr (GATEUP) {
                    // every row's SiLU(gate) * up unconditionally (dead rows
                    // repeat the last live row's inputs, so their values and
                    // flags equal that row's; they are not stored), one
                    // straight-line loop per path so the chains interleave
                    float mid[L][4];
                    bool finite = true;
                    if (shared) {
#pragma unroll
                        for (int rt = 0; rt < L; ++rt)
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                const float vg = bf16_round(val[rt][0][r]), vu = bf16_round(val[rt][1][r]);
                                mid[rt][r] = bf16_round(a.silu_table[__float_as_uint(vg) >> 16] * vu);
                                finite = finite && isfinite(vg) && isfinite(vu) && isfinite(mid[rt][r]);
                            }
                    } else {
                        // a non-finite gate or up value always gives a
                        // non-finite middle value here (NaN, inf * x, x / inf
                        // or 0 * inf; in the fast domain silu(g) is finite and
                        // nonzero), so the middle value alone decides.  The
                        // short form when every gate value of the wave is in
                        // its domain (common.hpp), the full one otherwise.
                        bool fast = true;
#pragma unroll
                        for (int rt = 0; rt < L; ++rt)
#pragma unroll
                            for (int r = 0; r < 4; ++r) fast = fast && silu_fast_domain(val[rt][0][r]);
                        if (__builtin_amdgcn_ballot_w64(!fast) == 0) {
#pragma unroll
                            for (int rt = 0; rt < L; ++rt)
#pragma unroll
                                for (int r = 0; r < 4; ++r) {
                                    mid[rt][r] = silu_portable_fast(val[rt][0][r]) * val[rt][1][r];
                                    finite = finite && isfinite(mid[rt][r]);
                                }
                        } else {
#pragma unroll
                            for (int rt = 0; rt < L; ++rt)
#pragma unroll
                                for (int r = 0; r < 4; ++r) {
                                    mid[rt][r] = silu_portable(val[rt][0][r]) * val[rt][1][r];
                                    finite = finite && isfinite(mid[rt][r]);
                                }
                        }
                    }
                    if (__builtin_amdgcn_ballot_w64(!finite) != 0) {
                        // the exact flags of this lane's live rows (rare)
#pragma unroll
                        for (int rt = 0; rt < L; ++rt)
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                float vg = val[rt][0][r], vu = val[rt][1][r];
                                if (shared) {
                                    vg = bf16_round(vg);
                                    vu = bf16_round(vu);
                                }
                                uint32_t f = (!isfinite(vg) || !isfinite(vu)) ? kFlagNonfiniteProjection : 0u;
                                f |= !isfinite(mid[rt][r]) ? (kFlagNonfiniteMiddle | kFlagNonfiniteInput) : 0u;
                                flags |= 16 * rt + 4 * q + r < nrows ? f : 0u;
                            }
                    }
                    // byte offsets from a.out fit 32 bits (rows < 2^22), so each
                    // store is one add from this lane's first row
                    const uint32_t obase = (uint32_t(first + 4 * q) * kInter + 64 * nt + 16 * w + li) * 4u;
                    const int live = nrows - 4 * q;       // rows 4q + j of the tile are live for j < live
#pragma unroll
                    for (int rt = 0; rt < L; ++rt)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            if (16 * rt + r < live)
                                *reinterpret_cast<float*>(reinterpret_cast<char*>(a.out) + obase +
                                                          uint32_t(16 * rt + r) * (kInter * 4u)) = mid[rt][r];
#pragma unroll
                            for (int ct = 0; ct < 2; ++ct) val[rt][ct][r] = 0.f;
                        }
                } else if constexpr (HEAD) {
                    // Logits go through LDS (the A ring is free once every
                    // wave is past its last dots) and leave as whole 16-byte
                    // row pieces; per row, the best of this block's 128
                    // columns (numpy argmax rule): lane (2 columns), 16 lanes
                    // (xor 1..8), 4 waves in LDS.
                    constexpr int kLS = kNT + 4;                  // padded row stride (floats)
                    static_assert(kMT * kLS <= NSTAGE * kMT * 64, "logit staging fits the A ring");
                    float* sL = reinterpret_cast<float*>(&sA[0][0]);
                    const int nblk = (a.N + kNT - 1) / kNT;
                    __syncthreads();
#pragma unroll
                    for (int rt = 0; rt < L; ++rt)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int row = 16 * rt + 4 * q + r;
                            float bv = 0.f;
                            int bi = 0x7fffffff;
#pragma unroll
                            for (int ct = 0; ct < 2; ++ct) {
                                const int cl = 32 * w + 16 * ct + li, col = kNT * nt + cl;
                                const float v = val[rt][ct][r];
                                sL[row * kLS + cl] = v;
                                if (col < a.N && (bi == 0x7fffffff || arg_better(v, col, bv, bi))) {
                                    bv = v;
                                    bi = col;
                                }
                                val[rt][ct][r] = 0.f;
                            }
#pragma unroll
                            for (int m = 1; m < 16; m <<= 1) {
                                float ov;
                                int oi;
                                if (m == 1) { ov = xor_perm_f<1>(bv); oi = xor_perm_i<1>(bi); }
                                else if (m == 2) { ov = xor_perm_f<2>(bv); oi = xor_perm_i<2>(bi); }
                                else if (m == 4) { ov = xor_perm_f<4>(bv); oi = xor_perm_i<4>(bi); }
                                else { ov = xor_perm_f<8>(bv); oi = xor_perm_i<8>(bi); }
                                if (oi != 0x7fffffff && (bi == 0x7fffffff || arg_better(ov, oi, bv, bi))) {
                                    bv = ov;
                                    bi = oi;
                                }
                            }
                            if (li == 0) { s_bv[w][row] = bv; s_bi[w][row] = bi; }
                        }
                    __syncthreads();
                    // rows of 32 float4 pieces: thread -> (row, piece), 8 rows per pass
                    const int cols = min(kNT, a.N - kNT * nt);
                    for (int row = tid >> 5; row < nrows; row += 8) {
                        const int c4 = 4 * (tid & 31);
                        if (c4 < cols) {
                            const float4 v = *reinterpret_cast<const float4*>(&sL[row * kLS + c4]);
                            const size_t o = size_t(row) * a.N + kNT * nt + c4;
                            *reinterpret_cast<float4*>(a.out + o) = v;
                            const float vv[4] = {v.x, v.y, v.z, v.w};
                            uint16_t b16[4];
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                b16[e] = f32_to_bf16_bits(vv[e]);
                                if (!isfinite(vv[e])) flags |= a.flag_projection;
                                if ((b16[e] & 0x7f80u) == 0x7f80u) flags |= a.flag_bf16;
                            }
                            if (a.out_bf16)
                                *reinterpret_cast<uint2*>(a.out_bf16 + o) =
                                    make_uint2(b16[0] | (uint32_t(b16[1]) << 16), b16[2] | (uint32_t(b16[3]) << 16));
                        }
                    }
                    if (tid < nrows) {
                        float bv = s_bv[0][tid];
                        int bi = s_bi[0][tid];
#pragma unroll
                        for (int ww = 1; ww < 4; ++ww) {
                            const float ov = s_bv[ww][tid];
                            const int oi = s_bi[ww][tid];
                            if (oi != 0x7fffffff && (bi == 0x7fffffff || arg_better(ov, oi, bv, bi))) {
                                bv = ov;
                                bi = oi;
                            }
                        }
                        a.arg_val[size_t(tid) * nblk + nt] = bv;
                        a.arg_idx[size_t(tid) * nblk + nt] = bi;
                    }
                } else {
#pragma unroll
                for (int rt = 0; rt < L; ++rt) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int row = 16 * rt + 4 * q + r;
                        if (row < nrows) {
                            {
                                const int route = s_route[row];
                                const int col0 = kNT * (nt * NSUB + sub) + 32 * w + li;
#pragma unroll
                                for (int ct = 0; ct < 2; ++ct) {
                                    float v = val[rt][ct][r];
                                    if (shared) v = bf16_round(v);
                                    if (!isfinite(v)) flags |= kFlagNonfiniteProjection;
                                    a.out[size_t(route) * kHidden + col0 + 16 * ct] = v;
                                }
                            }
                        }
#pragma unroll
                        for (int ct = 0; ct < 2; ++ct) val[rt][ct][r] = 0.f;
                    }
                }
                }
            }
        };

        [&]<int... S>(std::integer_sequence<int, S...>) {
            ([&] {
                constexpr int ST = S;
                __syncthreads();            // A of step ST visible; stage (ST+2)%3 free
                if constexpr (ST + 2 < GS) {
                    store_a(0, (ST + 2) % NSTAGE, ST + 2);
                    if constexpr (ST + 3 < GS) load_a(ST + 3, 0);
                }
                mfma_step.template operator()<ST>();
                tree_step.template operator()<ST>();
            }(), ...);
        }(std::make_integer_sequence<int, NSTEP>{});
    };
    // gate/up: 33..48 rows run a three-tile body; down: the four-tile one (a
    // fourth instantiation there costs it registers and 5 % of its time)
    if constexpr (MAXL >= 4 && GATEUP) {
        if (nrows > 48) run.template operator()<4>();
        else if (nrows > 32) run.template operator()<3>();
        else if (nrows > 16) run.template operator()<2>();
        else run.template operator()<1>();
    } else if constexpr (MAXL >= 4) {
        if (nrows > 32) run.template operator()<4>();
        else if (nrows > 16) run.template operator()<2>();
        else run.template operator()<1>();
    } else {
        if (nrows > 16) run.template operator()<2>();
        else run.template operator()<1>();
    }
    flag_or(a.sticky, flags);
}

// Every fp32 bit pattern (64 per thread): silu_portable_fast against
// silu_portable wherever silu_fast_domain holds.
__global__ __launch_bounds__(256) void silu_selfcheck_kernel(unsigned long long* checked, uint32_t* mismatches) {
    const uint64_t base = (uint64_t(blockIdx.x) * 256u + threadIdx.x) * 64u;
    unsigned long long n = 0;
    uint32_t bad = 0;
    for (int i = 0; i < 64; ++i) {
        const float g = __uint_as_float(uint32_t(base + i));
        if (!silu_fast_domain(g)) continue;
        ++n;
        bad += __float_as_uint(silu_portable(g)) != __float_as_uint(silu_portable_fast(g)) ? 1u : 0u;
    }
    atomicAdd(checked, n);
    if (bad) atomicAdd(mismatches, bad);
}

hipError_t launch_silu_selfcheck(unsigned long long* checked, uint32_t* mismatches, hipStream_t s) {
    // the counters are cleared by a kernel (graph-safe, no memset node)
    hipError_t st = launch_fill_u32(reinterpret_cast<uint32_t*>(checked), 2, 0u, s);
    if (st == hipSuccess) st = launch_fill_u32(mismatches, 1, 0u, s);
    if (st != hipSuccess) return st;
    timed_launch("silu_selfcheck", silu_selfcheck_kernel, dim3((1u << 26) / 256), dim3(256), 0, s, checked,
                 mismatches);
    return hipGetLastError();
}

hipError_t launch_grouped_mfma(const MfmaArgs& a, bool gateup, int max_tiles, hipStream_t s) {
    if (max_tiles <= 0) return hipSuccess;
    const int tiles8 = (max_tiles + 7) / 8 * 8;   // m-tiles rounded up to the 8 XCDs
    if (gateup) {
        timed_launch("gateup_mfma", prefill_mfma_kernel<kModeGateUp, kHidden / kGroup, 1, 2>,
                     dim3(tiles8 * ((2 * kInter) / kNT)), dim3(256), 0, s, a);
        return hipGetLastError();
    }
    // down: 4 column blocks (512 columns) per block, or 2 when that grid would
    // fill fewer than three rounds of the chip's block slots (three blocks
    // per CU): the second of ~1.3 rounds ran mostly empty (1120 tokens:
    // 41.5 -> 39.3 us; 8192 tokens, 7 rounds: 195.5 with 4 against 202 with 2)
    if (tiles8 * (kHidden / (kNT * 4)) < 3 * 3 * device_cu_count())
        timed_launch("down_mfma", prefill_mfma_kernel<kModeDown, kInter / kGroup, 2, 1>,
                     dim3(tiles8 * (kHidden / (kNT * 2))), dim3(256), 0, s, a);
    else
        timed_launch("down_mfma", prefill_mfma_kernel<kModeDown, kInter / kGroup, 4, 1>,
                     dim3(tiles8 * (kHidden / (kNT * 4))), dim3(256), 0, s, a);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// G256 LM head for up to 32 rows on the 32x32x32 int8 matrix cores.
//
// A block of WPB waves copies the rows' A8 activations (32 rows x 2048 int8,
// rows past R repeating row R - 1) and per-group scales into LDS once; then
// every wave streams its own contiguous range of 32-column code tiles (the
// N / 32 tiles split evenly over the grid's waves) with D group-steps of
// codes in flight, the ring running across tiles.
//  - Codes of one (tile, group) are 32 rows j of 32 words (word (j, n): the 8
//    codes of column n for k = 8j .. 8j + 7).  Load u (0..15) of lane
//    n + 32h takes word (4 (u / 2) + 2h + u % 2, n): the 32 lanes of a half
//    read one whole 128-byte row, and lane n + 32h ends up holding column n,
//    rows 4i + 2h and 4i + 2h + 1 for MFMA i (0..7): its 16 operand bytes
//    (even codes, odd codes per word) of k-half h.
//  - A: lane r + 32h of MFMA i reads the matching activation words (chunks
//    4i + 2h, 4i + 2h + 1 of the group: 16-byte piece 2i + h); row r's piece
//    p sits at LDS slot (p & ~15) | ((p ^ r) & 15).
//  - Output register k of lane l is C[8 (k / 4) + 4 (l / 32) + k % 4][l % 32]:
//    the fp32 group tree (dense_g256_api.h:35-37) runs per lane over its 16
//    rows of one column, ascending groups.
// Logits leave straight from that layout (two 128-byte rows per store).  A
// lane meets its columns in ascending order, so its running argmax candidate
// per row changes only on a strictly larger value or a first NaN (numpy
// rule); the wave writes one partial per row at the end.
// ---------------------------------------------------------------------------
typedef int i32x16 __attribute__((ext_vector_type(16)));

template <int WPB, int D>
__global__ __launch_bounds__(64 * WPB, 1) void head_tile_kernel(MfmaArgs a, int nwaves) {
    constexpr int GS = kHidden / kGroup;          // 8 groups of 256
    constexpr int RW = kHidden / 4;               // activation words per row
    constexpr int ROWS = 32, NT = 64 * WPB;
    static_assert(GS % D == 0, "ring slots repeat every tile");
    __shared__ __attribute__((aligned(16))) uint32_t sA[ROWS * RW];
    __shared__ __attribute__((aligned(16))) float s_sa[GS][ROWS];
    __shared__ __attribute__((aligned(16))) float s_ss[GS][ROWS];
    __shared__ __attribute__((aligned(16))) float s_nb[GS][ROWS];   // -sa * kDotBias (exact)
    __shared__ uint64_t s_key[WPB][16][65];       // per-wave argmax keys (padded rows)
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int cl = lane & 31, h = lane >> 5;
    const int R = a.R;

    constexpr int APASS = ROWS * 128 / NT;        // 16-byte pieces per thread
    static_assert(APASS % 4 == 0, "pieces move in batches of four");
#pragma unroll
    for (int b = 0; b < APASS; b += 4) {
        u32x4 v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int i = (b + k) * NT + tid, r = i >> 7, pc = i & 127;
            v[k] = *reinterpret_cast<const u32x4*>(a.act_words + size_t(min(r, R - 1)) * RW + 4 * pc);
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int i = (b + k) * NT + tid, r = i >> 7, pc = i & 127;
            *reinterpret_cast<u32x4*>(&sA[r * RW + 4 * ((pc & ~15) | ((pc ^ r) & 15))]) = v[k];
        }
    }
    for (int i = tid; i < ROWS * GS; i += NT) {
        const int r = i / GS, g = i % GS, sr = min(r, R - 1);
        const float sa = f16_bits_to_f32(a.act_scales[sr * GS + g]);
        s_sa[g][r] = sa;
        s_ss[g][r] = sa * float(a.act_sums[sr * GS + g]);
        s_nb[g][r] = -sa * kDotBias;
    }
    __syncthreads();

    // wave rank w * blocks + block: the ranks holding one tile more than the
    // rest (the lowest ones) spread over every CU, not a few whole blocks
    const int gw = w * int(gridDim.x) + int(blockIdx.x);
    if (gw >= nwaves) return;                     // no barrier follows
    const int ntiles = a.N >> 5;
    const int base = ntiles / nwaves, extra = ntiles % nwaves;
    const int c0 = gw * base + min(gw, extra), cnt = base + (gw < extra ? 1 : 0);

    // step st = 8 * (tile - c0) + group: 1024 code words and 32 meta words on
    const uint32_t* cbase = a.codes + size_t(c0) * GS * 1024 + 64 * h + cl;
    const uint32_t* mbase = a.meta + size_t(c0) * GS * 32 + cl;
    uint32_t bw[D][16];
    uint32_t bm[D];
    auto load_b = [&](int st, int slot) {
        const uint32_t* src = cbase + size_t(st) * 1024;
#pragma unroll
        for (int u = 0; u < 16; ++u) bw[slot][u] = load_once(src + 128 * (u >> 1) + 32 * (u & 1));
        bm[slot] = mbase[size_t(st) * 32];
    };
#pragma unroll
    for (int st = 0; st < D; ++st) load_b(st, st);

    // candidate per row: value and tile (t < 256: one byte each, packed);
    // all -inf keeps the first tile (the first column)
    float bv[16];
    uint32_t bt[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int k = 0; k < 16; ++k) bv[k] = -__builtin_inff();
    float nonfinite = 0.f, nonfinite_bf16 = 0.f;  // NaN once a logit (resp. its bf16) is inf or NaN
    constexpr i32x16 kAccInit = {kDotBiasBits, kDotBiasBits, kDotBiasBits, kDotBiasBits, kDotBiasBits, kDotBiasBits,
                                 kDotBiasBits, kDotBiasBits, kDotBiasBits, kDotBiasBits, kDotBiasBits, kDotBiasBits,
                                 kDotBiasBits, kDotBiasBits, kDotBiasBits, kDotBiasBits};

    // one code tile: 8 groups; REFILL = a next tile exists
    auto tile_body = [&]<bool REFILL>(int t) {
        float val[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) val[k] = 0.f;
#pragma unroll
        for (int g = 0; g < GS; ++g) {
            const int slot = g % D;
            i32x16 acc;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t w0 = bw[slot][2 * i], w1 = bw[slot][2 * i + 1];
                const i32x4 fb = {code_even(w0), code_odd(w0), code_even(w1), code_odd(w1)};
                const u32x4 av =
                    *reinterpret_cast<const u32x4*>(&sA[cl * RW + 4 * ((16 * g) | ((2 * i + h) ^ (cl & 15)))]);
                const i32x4 fa = {int(av.x), int(av.y), int(av.z), int(av.w)};
                acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa, fb, i ? acc : kAccInit, 0, 0, 0);
            }
            // pin the meta word here: left free, its conversion is hoisted
            // next to the load and waits out the whole ring
            asm volatile("" : "+v"(bm[slot]));
            const float sw = f16_bits_to_f32(uint16_t(bm[slot] & 0xffffu));
            const float off = f16_bits_to_f32(uint16_t(bm[slot] >> 16));
            if (g + D < GS) load_b(8 * t + g + D, slot);
            else if constexpr (REFILL) load_b(8 * t + g + D, slot);
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const float4 sa4 = *reinterpret_cast<const float4*>(&s_sa[g][8 * b + 4 * h]);
                const float4 ss4 = *reinterpret_cast<const float4*>(&s_ss[g][8 * b + 4 * h]);
                const float4 nb4 = *reinterpret_cast<const float4*>(&s_nb[g][8 * b + 4 * h]);
                const float sa[4] = {sa4.x, sa4.y, sa4.z, sa4.w}, ss[4] = {ss4.x, ss4.y, ss4.z, ss4.w};
                const float nb[4] = {nb4.x, nb4.y, nb4.z, nb4.w};
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int k = 4 * b + c;
                    const float scaled_dot = __builtin_fmaf(sa[c], __int_as_float(acc[k]), nb[c]);
                    const float product = sw * scaled_dot;
                    const float correction = off * ss[c];
                    val[k] = val[k] + (product + correction);
                }
            }
#pragma unroll
            for (int k = 0; k < 16; ++k) asm volatile("" : "+v"(val[k]));
        }
        // rows past R repeat row R - 1 bit for bit, so every lane's values
        // may feed the flags and the candidates
        const int col = 32 * (c0 + t) + cl;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const int row = 8 * (k >> 2) + 4 * h + (k & 3);
            const float v = val[k];
            const uint16_t b16 = f32_to_bf16_bits(v);
            if (row < R) {
                const size_t o = size_t(row) * a.N + col;
                a.out[o] = v;
                if (a.out_bf16) a.out_bf16[o] = b16;
            }
            nonfinite = __builtin_fmaf(v, 0.f, nonfinite);
            nonfinite_bf16 = __builtin_fmaf(bf16_bits_to_f32(b16), 0.f, nonfinite_bf16);
            const bool take = (v > bv[k]) | ((v != v) & (bv[k] == bv[k]));
            bv[k] = take ? v : bv[k];
            const uint32_t mask = 0xffu << (8 * (k & 3));
            bt[k >> 2] = take ? ((bt[k >> 2] & ~mask) | (uint32_t(t) << (8 * (k & 3)))) : bt[k >> 2];
        }
    };
    for (int t = 0; t + 1 < cnt; ++t) tile_body.template operator()<true>(t);
    tile_body.template operator()<false>(cnt - 1);

    // ---- per-row best of the wave, then one partial per row.  Key: an
    // order-preserving image of the value (-0 as +0, every NaN above +inf)
    // over the complemented column, so the unsigned maximum is the numpy
    // argmax candidate (first NaN, else first maximum).  The 16 keys of each
    // lane go through LDS; lane r (and r + 32) takes row r's 32 candidates
    // (columns cl of its half), 16 each, and the two halves meet by xor 32.
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const float v = bv[k] + 0.f;
        const uint32_t u = __float_as_uint(v);
        const uint32_t ord = v != v ? 0xffffffffu : ((u & 0x80000000u) ? ~u : (u | 0x80000000u));
        const int colk = 32 * (c0 + int((bt[k >> 2] >> (8 * (k & 3))) & 0xffu)) + cl;
        s_key[w][k][lane] = (uint64_t(ord) << 32) | uint32_t(~colk);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    {
        const int r = lane & 31, rh = (r >> 2) & 1, rk = 4 * (r >> 3) + (r & 3), c0h = 16 * (lane >> 5);
        uint64_t key = s_key[w][rk][32 * rh + c0h];
#pragma unroll
        for (int c = 1; c < 16; ++c) {
            const uint64_t o = s_key[w][rk][32 * rh + c0h + c];
            key = o > key ? o : key;
        }
        const int hi = xor_perm_i<32>(int(key >> 32)), lo = xor_perm_i<32>(int(uint32_t(key)));
        const uint64_t other = (uint64_t(uint32_t(hi)) << 32) | uint32_t(lo);
        key = other > key ? other : key;
        if (lane < 32 && r < R) {
            const uint32_t o = uint32_t(key >> 32);
            const float v = o == 0xffffffffu ? __builtin_nanf("") : __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
            a.arg_idx[size_t(r) * nwaves + gw] = int(~uint32_t(key));
            a.arg_val[size_t(r) * nwaves + gw] = v;
        }
    }
    uint32_t flags = 0;
    if (nonfinite != nonfinite) flags |= a.flag_projection;
    if (nonfinite_bf16 != nonfinite_bf16) flags |= a.flag_bf16;
    flag_or(a.sticky, flags);
}

// Head waves: WPB-wave blocks (one per CU), at least two code tiles per wave
// (so the partial count per row, nwaves, stays within ceil(N / 64)).
constexpr int kHeadWaves = 8, kHeadRing = 2;
static int head_waves(int N) { return std::max(1, std::min(kHeadWaves * device_cu_count(), (N / 32) / 2)); }

hipError_t launch_head_mfma(const MfmaArgs& a, int64_t* argmax, hipStream_t s) {
    if (a.R <= 0 || a.R > kMT || a.N <= 0 || a.N % 32 != 0 || a.K != kHidden) return hipErrorInvalidValue;
    int nparts;
    if (a.R <= 32) {
        // up to 32 rows (the decode-side head): streaming waves
        nparts = head_waves(a.N);
        timed_launch("head_mfma", head_tile_kernel<kHeadWaves, kHeadRing>,
                     dim3((nparts + kHeadWaves - 1) / kHeadWaves), dim3(64 * kHeadWaves), 0, s, a, nparts);
    } else {
        nparts = (a.N + kNT - 1) / kNT;
        timed_launch("head_mfma", prefill_mfma_kernel<kModeHead, kHidden / kGroup, 1, 2>, dim3(nparts), dim3(256), 0,
                     s, a);
    }
    hipError_t st = hipGetLastError();
    if (st != hipSuccess) return st;
    timed_launch("argmax", head_argmax_kernel, dim3(a.R), dim3(256), 0, s, a.arg_val, a.arg_idx, nparts, argmax);
    return hipGetLastError();
}

// H128 + quantisation of the middle rows in permuted route order: rows 0 ..
// *nrows - 1, on quarter-wave groups (common.hpp), four groups (two rows) per
// wave.
template <int QMAX>
__global__ __launch_bounds__(256) void quant_middle_permuted_kernel(const float* __restrict__ middle, int RS,
                                                                    const int32_t* __restrict__ nrows,
                                                                    uint32_t* __restrict__ words,
                                                                    uint16_t* __restrict__ scales,
                                                                    int32_t* __restrict__ sums, uint32_t* sticky) {
    const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, l = lane & 15;
    const int total = min(nrows[0], RS) * 2;                  // two groups per 512-wide row
    if (4 * wave >= total) return;
    const int g = 4 * wave + (lane >> 4), k0 = quarter_base(l);
    const float* src = middle + size_t(min(g, total - 1)) * kGroup + k0;   // row g / 2, group g % 2
    float v[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 m = *reinterpret_cast<const float4*>(src + 4 * i);
        v[4 * i] = m.x; v[4 * i + 1] = m.y; v[4 * i + 2] = m.z; v[4 * i + 3] = m.w;
    }
    uint32_t flags = 0;
    h128_quarter(v);
    uint32_t w4[4];
    uint16_t sbits;
    int sum;
    quantize_quarter_fast<QMAX>(v, w4, sbits, sum, flags, kFlagNonfiniteInput | kFlagInvalidActivation,
                                kFlagInvalidActivation);
    if (g < total) {
        *reinterpret_cast<uint4*>(words + size_t(g) * 64 + k0 / 4) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
        if (l == 0) { scales[g] = sbits; sums[g] = sum; }
    } else {
        flags = 0;
    }
    flag_or(sticky, flags);
}

hipError_t launch_quant_middle_permuted(const float* middle, int RS, const int32_t* nrows, int qmax, uint32_t* words,
                                        uint16_t* scales, int32_t* sums, uint32_t* sticky, hipStream_t s) {
    const int waves = (RS * 2 + 3) / 4;
    if (qmax == 127)
        timed_launch("quant_middle", quant_middle_permuted_kernel<127>, dim3((waves + 3) / 4), dim3(256), 0, s, middle, RS, nrows, words, scales, sums, sticky);
    else
        timed_launch("quant_middle", quant_middle_permuted_kernel<7>, dim3((waves + 3) / 4), dim3(256), 0, s, middle, RS, nrows, words, scales, sums, sticky);
    return hipGetLastError();
}

}  // namespace ornith
