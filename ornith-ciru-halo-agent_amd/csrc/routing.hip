// Router logits, softmax/top-8/renormalise, token permutation and the
// slot-order unpermute.
//
// Router and top-k replace the reference's Triton row-dot
// (iu4_correctness/gates_projection.py:18-26,36-42) and vLLM's topk_softmax
// (contract moe_base.py:57-64, dtypes :53-54).  Both reduction orders are
// declared by this library (the reference's are compiler/library chosen):
//   logit[t,e] = bias[e] + butterfly (masks 1,2,...,32) over 64 lanes of lane partials, lane l
//   accumulating fma(x[k], w[k], acc) over k = 8c..8c+7 for
//   c = l, l+64, l+128, l+192 (bf16*bf16 products are exact in fp32, so the
//   fma equals a separate multiply and add).
// Permute replaces histogram/scan_routes/scatter/partition
// (routed_storage_n32_prefill.h:19-42) with a deterministic stable order.
#include "kernels.hpp"
#include "timing.hpp"
#include "topk.hpp"
#include "act.hpp"

namespace ornith {

__device__ __forceinline__ void bf16x8_to_f32(const uint4 v, float f[8]) {
    const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        f[2 * e] = __uint_as_float(u[e] << 16);
        f[2 * e + 1] = __uint_as_float(u[e] & 0xffff0000u);
    }
}

constexpr int kPermTokens = 16;                      // tokens per permutation count / scatter block
constexpr int kPermRoutes = kPermTokens * kTop;      // routed routes per block

// ---------------------------------------------------------------------------
// Router logits for large T on the matrix cores (declared order above).  A
// K = 1 fp32 matrix-core step d = RN(a * b + c) equals v_fma_f32 bit for bit
// (measured for v_mfma_f32_32x32x1_2b_f32 on every operand class: normal,
// denormal, zero, inf, NaN), and a product of two bf16 values is exact in
// fp32, so one step per k advances the fma chains of two partials (its two
// blocks) for a whole 32-expert x 32-token tile.  The 32 x 32 form does
// twice the multiply-adds per converted operand of the 16 x 16 one; the
// bf16 -> fp32 conversions are vector-ALU work that the fp32 matrix steps
// wait for, so that halves their cost.
// The butterfly is a balanced tree over the 64 lane partials (every pair sum
// is formed once and fp32 addition commutes).  Block = 16 waves on one tile;
// wave q carries partials 4q..4q+3 (chunk p + 64j, j = quarter of K, k
// ascending) in two steps per k (blocks b = partials 4q + b and 4q + 2 + b)
// and sums them as (P0 + P1) + (P2 + P3); the 16 wave sums meet in LDS in
// the balanced 16-leaf tree.
// Lane layout of a step: block b takes expert row i and token row i from lane
// 32 b + i; its output (i, j) lands in lane 32 ((i / 4) % 2) + j, register
// 16 b + 4 (i / 8) + i % 4.
// The shared-expert gate row (row 256) runs on the vector ALUs beside the
// tiles: the eight expert-group blocks of a token group each take 4 of its
// tokens, lane p forming partial p from the staged rows, then the butterfly.
// ---------------------------------------------------------------------------
typedef float f32x32 __attribute__((ext_vector_type(32)));
typedef __attribute__((address_space(3))) void lds_void;
constexpr int kRmTile = 32, kRmWaves = 16;
constexpr int kRmGroups = kExperts / kRmTile;              // expert groups (tiles) per token group
constexpr int kRmQuarter = kHidden / 4;                    // k per staged quarter
constexpr int kRmRowBytes = 2 * kRmQuarter + 16;           // staged row + a 16-byte pad (conflict-free columns)

// Token groups past full_tg (the tiles that would otherwise make a short last
// round on a few CUs) are split into units of one eighth of a tile: unit
// (tile, j) forms lane partials 8j..8j+7 of the tile's 32 x 32 logits and
// sums them as ((P0 + P1) + (P2 + P3)) + ((P4 + P5) + (P6 + P7)) -- levels 1-3
// of the balanced tree -- into split_sums[tile][j][token][expert]; the top-k
// kernel adds levels 4-6 in the same order, then the bias.  Units spread over
// every block (unit u = blk, blk + nblk, ...).  The unit's rows are staged
// whole (its 32 chunks of each of the 64 rows, 32 KB) piece-major, so the
// column reads are conflict-free; waves 0-3 carry the partials (two per
// step, as in the tiles), and for j == 0 waves 4-7 form the shared-gate
// logits of tokens 4 eg .. 4 eg + 3 of the tile straight from memory.
__device__ __forceinline__ void router_split_units(int blk, int nblk, const uint16_t* __restrict__ x, int64_t stride,
                                                   int T, const uint16_t* __restrict__ w,
                                                   const uint16_t* __restrict__ shared_w,
                                                   float* __restrict__ logits, int64_t logit_stride, int ntg,
                                                   int full_tg, float* __restrict__ split_sums, uint8_t* lds0,
                                                   uint8_t* lds1) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int q = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int b = lane >> 5, i = lane & 31;
    const int nunits = 64 * (ntg - full_tg);
    for (int u = blk; u < nunits; u += nblk) {
        const int tile = u >> 3, j = u & 7;                // tile = 8 (tg - full_tg) + eg
        const int tg = full_tg + (tile >> 3), eg = tile & 7, e0 = eg * kRmTile, t0 = tg * kRmTile;
        // piece p = 8 jq + c (chunk 8j + c of quarter jq) of row r at (64 p + r) * 16;
        // wave q stages pieces 2q, 2q + 1, lane = row
        {
            const uint16_t* row = lane < kRmTile ? w + size_t(e0 + lane) * kHidden
                                                 : x + size_t(min(t0 + lane - kRmTile, T - 1)) * stride;
#pragma unroll
            for (int n = 0; n < 2; ++n) {
                const int p = 2 * q + n, jq = p >> 3, cc = p & 7;
                __builtin_amdgcn_global_load_lds(row + kRmQuarter * jq + 8 * (8 * j + cc),
                                                 (lds_void*)(lds0 + 1024 * p), 16, 0, 0);
            }
        }
        __syncthreads();
        if (q < 4) {
            // wave q: partials 8j + 2q + b, chunk 2q + b of each quarter
            f32x32 acc = f32x32{};
#pragma unroll
            for (int jq = 0; jq < 4; ++jq) {
                const int p = 8 * jq + 2 * q + b;
                const uint4 wv = *reinterpret_cast<const uint4*>(lds0 + (64 * p + i) * 16);
                const uint4 xv = *reinterpret_cast<const uint4*>(lds0 + (64 * p + kRmTile + i) * 16);
                const uint32_t uw[4] = {wv.x, wv.y, wv.z, wv.w};
                const uint32_t ux[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    acc = __builtin_amdgcn_mfma_f32_32x32x1f32(__uint_as_float(uw[h] << 16),
                                                               __uint_as_float(ux[h] << 16), acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_32x32x1f32(__uint_as_float(uw[h] & 0xffff0000u),
                                                               __uint_as_float(ux[h] & 0xffff0000u), acc, 0, 0, 0);
                }
            }
            // level 1 (the step's two blocks), then the [wave][token][expert] exchange
            float* sS = reinterpret_cast<float*>(lds1);
            const int jt = lane & 31;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int grp = 2 * g + b;
                *reinterpret_cast<float4*>(sS + (q * kRmTile + jt) * kRmTile + 4 * (grp ^ (jt & 7))) =
                    make_float4(acc[4 * g] + acc[16 + 4 * g], acc[4 * g + 1] + acc[17 + 4 * g],
                                acc[4 * g + 2] + acc[18 + 4 * g], acc[4 * g + 3] + acc[19 + 4 * g]);
            }
        } else if (q < 8 && j == 0 && shared_w) {
            // shared-gate logit of token 4 eg + (q - 4) of the tile, lane = partial
            const int t = t0 + 4 * eg + (q - 4);
            const uint16_t* xr = x + size_t(min(t, T - 1)) * stride;
            float sacc = 0.f;
#pragma unroll
            for (int jq = 0; jq < 4; ++jq) {
                float xf[8], wf[8];
                bf16x8_to_f32(*reinterpret_cast<const uint4*>(xr + kRmQuarter * jq + 8 * lane), xf);
                bf16x8_to_f32(*reinterpret_cast<const uint4*>(shared_w + kRmQuarter * jq + 8 * lane), wf);
#pragma unroll
                for (int k = 0; k < 8; ++k) sacc = __builtin_fmaf(xf[k], wf[k], sacc);
            }
            const float v = wave_butterfly_sum(sacc);
            if (lane == 0 && t < T) logits[size_t(t) * logit_stride + kExperts] = v;
        }
        __syncthreads();
        {
            // levels 2-3 over the four waves; thread = (expert er, token tc)
            const float* sS = reinterpret_cast<const float*>(lds1);
            const int er = tid & 31, tc = (tid >> 5) & 31;
            const int off = tc * kRmTile + 4 * ((er >> 2) ^ (tc & 7)) + (er & 3);
            if (tid < kRmTile * kRmTile) {
                const float v = (sS[off] + sS[kRmTile * kRmTile + off]) +
                                (sS[2 * kRmTile * kRmTile + off] + sS[3 * kRmTile * kRmTile + off]);
                split_sums[(size_t(tile) * 8 + j) * (kRmTile * kRmTile) + tc * kRmTile + er] = v;
            }
        }
        __syncthreads();                                  // both buffers free for the next unit
    }
}

// Persistent: block b runs on XCD b % 8 and walks that XCD's tiles (token
// groups tg = x (mod 8), all eight expert groups, so a token group's x rows
// stay in the XCD's L2), tile c, c + B, c + 2B, ... of the XCD's list for
// c = b / 8 and B = blocks / 8.  The next tile's first quarter is staged
// during the last quarter of the current one, and the Sq exchange uses the
// buffer that quarter leaves free, so a tile boundary costs only the exchange.
__device__ __forceinline__ void router_mfma_run(int blk, int nblk, const uint16_t* __restrict__ x, int64_t stride,
                                                int T, const uint16_t* __restrict__ w,
                                                const uint16_t* __restrict__ shared_w, const float* __restrict__ bias,
                                                float* __restrict__ logits, int64_t logit_stride, int ntg, int full_tg,
                                                float* __restrict__ split_sums) {
    // two buffers (separate arrays, so the compiler sees that loads into one
    // do not alias reads of the other) of one K quarter of a tile's 32
    // expert rows (rows 0..31) and 32 token rows (rows 32..63), bf16, rows
    // kRmRowBytes apart; the shared-expert row whole
    constexpr int kBuf = 2 * kRmTile * kRmRowBytes;
    __shared__ __align__(16) uint8_t lds0[kBuf];
    __shared__ __align__(16) uint8_t lds1[kBuf];
    __shared__ __align__(16) uint8_t lshared[2 * kHidden];
    static_assert(kRmWaves * kRmTile * kRmTile * 4 <= kBuf, "Sq exchange fits a buffer");
    const int xcd = blk & 7, c = blk >> 3, B = nblk >> 3;
    const int ntiles = 8 * ((full_tg - xcd + 7) / 8);          // this XCD's whole tiles: 8 per token group
    const int tid = threadIdx.x, lane = tid & 63;
    const int q = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: row pointers stay scalar
    const int b = lane >> 5, i = lane & 31;
    const bool has_shared = shared_w != nullptr;
    // staging straight into LDS: wave q loads rows q, q + 16 (experts) and
    // q + 32, q + 48 (tokens; past the end they repeat the last one), lane =
    // 16-byte chunk of the quarter
    auto stage = [&](int u, int jq, uint8_t* dst) __attribute__((always_inline)) {
        const int tg = 8 * (u >> 3) + xcd, e0 = (u & 7) * kRmTile, t0 = tg * kRmTile;
#pragma unroll
        for (int n = 0; n < 4; ++n) {
            const int r = q + 16 * n;
            const uint16_t* row = n < 2 ? w + size_t(e0 + r) * kHidden
                                        : x + size_t(min(t0 + r - kRmTile, T - 1)) * stride;
            __builtin_amdgcn_global_load_lds(row + kRmQuarter * jq + 8 * lane,
                                             (lds_void*)(dst + (q + 16 * n) * kRmRowBytes), 16, 0, 0);
        }
    };
    // this lane's operands: expert row i and token row i, chunk 4q + b (first
    // step) and 4q + 2 + b (second step) of the quarter
    const int abase = i * kRmRowBytes + 16 * (4 * q + b), bbase = (kRmTile + i) * kRmRowBytes + 16 * (4 * q + b);
    if (c < ntiles) stage(c, 0, lds0);
    if (has_shared && q < 4)
        __builtin_amdgcn_global_load_lds(shared_w + kRmQuarter * q + 8 * lane, (lds_void*)(lshared + 1024 * q), 16, 0,
                                         0);
    __syncthreads();
    for (int u = c; u < ntiles; u += B) {
        const int tg = 8 * (u >> 3) + xcd, eg = u & 7, e0 = eg * kRmTile, t0 = tg * kRmTile;
        const bool next = u + B < ntiles;
        // shared row: waves eg and eg + 8 of the tile take token rows q and
        // 16 + q (4 tokens per tile), lane = partial
        const bool mine = has_shared && (q & 7) == eg;
        float sacc[2] = {0.f, 0.f};
        f32x32 acc[2] = {f32x32{}, f32x32{}};
#pragma unroll
        for (int jq = 0; jq < 4; ++jq) {
            const uint8_t* sb = jq & 1 ? lds1 : lds0;
            // the target buffer's last readers passed the previous barrier
            if (jq < 3) stage(u, jq + 1, jq & 1 ? lds0 : lds1);
            else if (next) stage(u + B, 0, lds0);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const uint4 wv = *reinterpret_cast<const uint4*>(sb + abase + 32 * s);
                const uint4 xv = *reinterpret_cast<const uint4*>(sb + bbase + 32 * s);
                const uint32_t uw[4] = {wv.x, wv.y, wv.z, wv.w};
                const uint32_t ux[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    acc[s] = __builtin_amdgcn_mfma_f32_32x32x1f32(__uint_as_float(uw[h] << 16),
                                                                  __uint_as_float(ux[h] << 16), acc[s], 0, 0, 0);
                    acc[s] = __builtin_amdgcn_mfma_f32_32x32x1f32(__uint_as_float(uw[h] & 0xffff0000u),
                                                                  __uint_as_float(ux[h] & 0xffff0000u), acc[s], 0, 0,
                                                                  0);
                }
            }
            if (mine) {
                float wf[8], xf[8];
                bf16x8_to_f32(*reinterpret_cast<const uint4*>(lshared + 2 * kRmQuarter * jq + 16 * lane), wf);
#pragma unroll
                for (int v = 0; v < 2; ++v) {
                    bf16x8_to_f32(*reinterpret_cast<const uint4*>(sb + (kRmTile + q + 16 * v) * kRmRowBytes + 16 * lane),
                                  xf);
#pragma unroll
                    for (int k = 0; k < 8; ++k) sacc[v] = __builtin_fmaf(xf[k], wf[k], sacc[v]);
                }
            }
            __syncthreads();                              // (waits for this wave's staging loads first)
        }
        if (mine) {
#pragma unroll
            for (int v = 0; v < 2; ++v) {
                const float sv = wave_butterfly_sum(sacc[v]);
                const int t = t0 + 16 * v + q;
                if (lane == 0 && t < T) logits[size_t(t) * logit_stride + kExperts] = sv;
            }
        }
        // (P0 + P1) + (P2 + P3): the two blocks of each step hold the same
        // (i, j) in registers r and 16 + r
        float sq[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) sq[r] = (acc[0][r] + acc[0][16 + r]) + (acc[1][r] + acc[1][16 + r]);
        // exchange in buffer 1 (free after the last quarter) as [wave][token j]
        // [expert i], 16-byte group i / 4 stored at group (i / 4) ^ (j & 7):
        // registers 4g..4g+3 are rows 8g + 4 (lane / 32) + 0..3, one 16-byte
        // store each, conflict-free, and so are the reads
        float* sS = reinterpret_cast<float*>(lds1);
        const int j = lane & 31;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int grp = 2 * g + b;                    // rows 4 grp .. 4 grp + 3
            *reinterpret_cast<float4*>(sS + (q * kRmTile + j) * kRmTile + 4 * (grp ^ (j & 7))) =
                make_float4(sq[4 * g], sq[4 * g + 1], sq[4 * g + 2], sq[4 * g + 3]);
        }
        __syncthreads();
        {
            const int er = tid & 31, tc = tid >> 5, e = e0 + er, t = t0 + tc;
            const int off = tc * kRmTile + 4 * ((er >> 2) ^ (tc & 7)) + (er & 3);
            float lv[kRmWaves];
#pragma unroll
            for (int v = 0; v < kRmWaves; ++v) lv[v] = sS[v * kRmTile * kRmTile + off];
#pragma unroll
            for (int step = 1; step < kRmWaves; step *= 2)
#pragma unroll
                for (int v = 0; v < kRmWaves; v += 2 * step) lv[v] = lv[v] + lv[v + step];
            if (t < T) logits[size_t(t) * logit_stride + e] = bias ? lv[0] + bias[e] : lv[0];
        }
        __syncthreads();                                  // buffer 1 free for the next tile's second quarter
    }
    if (split_sums) router_split_units(blk, nblk, x, stride, T, w, shared_w, logits, logit_stride, ntg, full_tg,
                                       split_sums, lds0, lds1);
}

// full_tg < ntg: token groups full_tg .. ntg - 1 run as eighth-tile units
// into split_sums.
__global__ __launch_bounds__(kRmWaves * 64) void router_mfma_kernel(const uint16_t* __restrict__ x, int64_t stride, int T,
                                                                     const uint16_t* __restrict__ w,
                                                                     const uint16_t* __restrict__ shared_w,
                                                                     const float* __restrict__ bias,
                                                                     float* __restrict__ logits, int64_t logit_stride,
                                                                     int ntg, int full_tg,
                                                                     float* __restrict__ split_sums) {
    router_mfma_run(int(blockIdx.x), int(gridDim.x), x, stride, T, w, shared_w, bias, logits, logit_stride, ntg,
                    full_tg, split_sums);
}

// One wave per (router row, batch of 8 tokens): the choice for small and
// medium T, where the tiled kernel has too few blocks to fill the chip.
__global__ __launch_bounds__(256) void router_rows_kernel(const uint16_t* __restrict__ x, int64_t stride, int T,
                                                          const uint16_t* __restrict__ w,
                                                          const uint16_t* __restrict__ shared_w,
                                                          const float* __restrict__ bias, float* __restrict__ logits,
                                                          int64_t logit_stride, int nrows) {
    const int gw = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int nb = (T + 7) / 8;
    if (gw >= nrows * nb) return;
    const int row = gw / nb, t0 = (gw % nb) * 8;
    const uint16_t* wrow = row < kExperts ? w + size_t(row) * kHidden : shared_w;
    const bool has_bias = bias && row < kExperts;
    router_rows_wave(x, stride, T, t0, wrow, has_bias ? bias[row] : 0.f, has_bias, logits, logit_stride, row);
}

// Persistent tile blocks: 8 B (B per XCD), at most one per CU and at most the
// tiles an XCD has (8 per token group).
static int router_mfma_blocks(int ntg) {
    const int per_xcd = std::max(1, std::min(device_cu_count() / 8, 8 * ((ntg + 7) / 8)));
    return 8 * per_xcd;
}

hipError_t launch_router(const uint16_t* x, int64_t stride, int T, const uint16_t* w, const uint16_t* shared_w,
                         const float* bias, float* logits, int64_t logit_stride, hipStream_t s, float* split_sums) {
    if (T <= 0) return hipSuccess;
    if (T <= kRouterRowsMaxTokens) {
        const int nrows = kExperts + (shared_w ? 1 : 0);
        const int waves = nrows * ((T + 7) / 8);
        timed_launch("router", router_rows_kernel, dim3((waves + 3) / 4), dim3(256), 0, s, x, stride, T, w, shared_w,
                     bias, logits, logit_stride, nrows);
        return hipGetLastError();
    }
    const int ntg = (T + kRmTile - 1) / kRmTile;
    const int full_tg = ntg - (split_sums ? router_split_groups(T) : 0);
    timed_launch("router", router_mfma_kernel, dim3(router_mfma_blocks(ntg)), dim3(kRmWaves * 64), 0, s, x, stride, T,
                 w, shared_w, bias, logits, logit_stride, ntg, full_tg, full_tg < ntg ? split_sums : nullptr);
    return hipGetLastError();
}

// The tile kernel holds one block per CU (its LDS), each walking its share of
// the tiles.  When the token groups past the last whole round are few (at
// most 2 eighth-tile units per block), they go to units over every block,
// so the launch ends about a unit after its last whole round (a unit costs
// its loads' latency besides an eighth of a tile's products, so larger
// remainders stay whole tiles).
int router_split_groups(int T) {
    if (T <= kRouterRowsMaxTokens) return 0;
    const int cus = device_cu_count(), per = cus / 8, ntg = (T + kRmTile - 1) / kRmTile;
    if (per <= 0 || ntg < per) return 0;
    const int left = ntg % per;
    return 64 * left <= 2 * cus ? left : 0;
}

size_t router_split_bytes(int Tcap) {
    if (Tcap <= kRouterRowsMaxTokens) return 0;
    const int groups = std::max(1, 2 * device_cu_count() / 64);
    return size_t(groups) * 64 * kRmTile * kRmTile * sizeof(float);
}

// ---------------------------------------------------------------------------
// Softmax / top-8 / renormalise, one wave per token (topk.hpp: threshold and
// rank count, LDS scratch per wave).  Declared
// order: m = max; e = pexp(l - m); s = butterfly (masks 1..32) over lanes of
// ((e[l] + e[l+64]) + e[l+128]) + e[l+192]; p = e / s; the eight largest p
// (ties to the lower id) in descending order; weights p / (slot-order sum of
// the picked p).
// ---------------------------------------------------------------------------
// WAVES tokens per block; COUNT adds the routed-bank histogram of the block's
// tokens (block_counts[blockIdx.x][bank], the count step of the permutation;
// WAVES is then its 16-token block).
template <int WAVES, bool COUNT>
__global__ __launch_bounds__(64 * WAVES) void topk_kernel(float* __restrict__ logits, int64_t logit_stride, int T,
                                                          float* __restrict__ weights, int32_t* __restrict__ ids,
                                                          const float* __restrict__ shared_logit, int64_t shared_stride,
                                                          uint16_t* __restrict__ shared_bf16,
                                                          int32_t* __restrict__ block_counts,
                                                          const float* __restrict__ split, int split_t0,
                                                          const float* __restrict__ bias) {
    __shared__ __align__(16) uint64_t s_cand[WAVES][66];
    __shared__ uint2 s_sel[WAVES][kTop];
    __shared__ int s_hist[COUNT ? kExperts : 1];
    const int w = threadIdx.x >> 6, t = blockIdx.x * WAVES + w;
    const int lane = threadIdx.x & 63;
    if (COUNT) {
        for (int i = threadIdx.x; i < kExperts; i += 64 * WAVES) s_hist[i] = 0;
        __syncthreads();
    }
    if (t < T) {
        float v[4];
        if (split && t >= split_t0) {
            // levels 4-6 of the router's balanced tree over its eighth-tile sums, then the bias
            // (all 32 sums and the bias loaded before any is used: one round trip)
            const int tile0 = 8 * ((t - split_t0) / kRmTile), tl = t % kRmTile;
            float p[4][8], bv[4] = {};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int e = lane + 64 * i;
                const float* S = split + size_t(tile0 + e / kRmTile) * 8 * (kRmTile * kRmTile) +
                                 tl * kRmTile + e % kRmTile;
#pragma unroll
                for (int j = 0; j < 8; ++j) p[i][j] = S[j * (kRmTile * kRmTile)];
            }
            if (bias) {
#pragma unroll
                for (int i = 0; i < 4; ++i) bv[i] = bias[lane + 64 * i];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float lv = ((p[i][0] + p[i][1]) + (p[i][2] + p[i][3])) + ((p[i][4] + p[i][5]) + (p[i][6] + p[i][7]));
                if (bias) lv = lv + bv[i];
                v[i] = lv;
                logits[size_t(t) * logit_stride + lane + 64 * i] = lv;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = logits[size_t(t) * logit_stride + lane + 64 * i];
        }
        uint32_t k[4];
        softmax_keys(v, k);
        top8_rank_lds(k, s_cand[w], s_sel[w]);
        float tot = 0.f;
#pragma unroll
        for (int j = 0; j < kTop; ++j) tot = tot + __uint_as_float(s_sel[w][j].x);
        if (lane < kTop) {
            const uint2 pick = s_sel[w][lane];
            weights[size_t(t) * kTop + lane] = fdiv_rn(__uint_as_float(pick.x), tot);
            ids[size_t(t) * kTop + lane] = int(pick.y);
            if (COUNT) atomicAdd(&s_hist[pick.y], 1);
        }
        if (lane == 0 && shared_bf16) shared_bf16[t] = f32_to_bf16_bits(shared_logit[size_t(t) * shared_stride]);
    }
    if (COUNT) {
        __syncthreads();
        for (int i = threadIdx.x; i < kExperts; i += 64 * WAVES)
            block_counts[size_t(blockIdx.x) * kExperts + i] = s_hist[i];
    }
}

hipError_t launch_topk(const float* logits, int64_t logit_stride, int T, float* weights, int32_t* ids,
                       const float* shared_logit, int64_t shared_stride, uint16_t* shared_bf16, hipStream_t s,
                       int32_t* block_counts, const float* split_sums, const float* bias) {
    if (T <= 0) return hipSuccess;
    const int split_groups = split_sums ? router_split_groups(T) : 0;
    const float* split = split_groups ? split_sums : nullptr;
    const int split_t0 = ((T + kRmTile - 1) / kRmTile - split_groups) * kRmTile;
    float* lg = const_cast<float*>(logits);        // written back only for the split tokens
    if (block_counts)
        timed_launch("topk", topk_kernel<kPermTokens, true>, dim3((T + kPermTokens - 1) / kPermTokens),
                     dim3(64 * kPermTokens), 0, s, lg, logit_stride, T, weights, ids, shared_logit, shared_stride,
                     shared_bf16, block_counts, split, split_t0, bias);
    else
        timed_launch("topk", topk_kernel<4, false>, dim3((T + 3) / 4), dim3(256), 0, s, lg, logit_stride, T,
                     weights, ids, shared_logit, shared_stride, shared_bf16, block_counts, split, split_t0, bias);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Permutation: stable counting sort of routes by bank.
// banks: 0..255 routed experts, 256 = shared expert (routes R..R+T-1).
// Produces counts, exclusive offsets, the permuted route list, one Segment
// per non-empty bank (ascending bank order) and the MFMA tile list.
// ---------------------------------------------------------------------------
constexpr int kBanks = kExperts + 1;

__device__ __forceinline__ int route_bank(const int32_t* ids, int r, int R, uint32_t& flags) {
    if (r >= R) return kShared;
    const int id = ids[r];
    if (id >= 0 && id < kExperts) return id;
    if (id != -1) flags |= kFlagInvalidExpert;
    return -1;
}

__device__ __forceinline__ int wave_inclusive_scan(int v) { return wave_prefix_sum(v); }

size_t permute_scratch_bytes(int Rcap, int Tcap) {
    const size_t rall = size_t(Rcap) + size_t(Tcap);
    const size_t blocks = (size_t(Rcap / kTop) + kPermTokens - 1) / kPermTokens;
    size_t bytes = 0;
    bytes += align256(blocks * kExperts * 4);
    bytes += align256(kBanks * 4);
    bytes += align256((kBanks + 1) * 4);
    bytes += align256(rall * 4);
    bytes += align256(kBanks * sizeof(Segment));
    bytes += align256(4 * 4);
    // one per 64-route m-tile, plus the launch's rounding up to a multiple of 8 tiles
    bytes += align256((rall / 64 + kBanks + 10) * sizeof(Segment));
    return bytes;
}

PermuteScratch carve_permute(void* base, int Rcap, int Tcap) {
    const size_t rall = size_t(Rcap) + size_t(Tcap);
    const size_t blocks = (size_t(Rcap / kTop) + kPermTokens - 1) / kPermTokens;
    PermuteScratch p{};
    size_t off = 0;
    auto take = [&](size_t bytes) { void* q = at<void>(base, off); off += align256(bytes); return q; };
    p.block_counts = static_cast<int32_t*>(take(blocks * kExperts * 4));
    p.counts = static_cast<int32_t*>(take(kBanks * 4));
    p.offsets = static_cast<int32_t*>(take((kBanks + 1) * 4));
    p.routes = static_cast<int32_t*>(take(rall * 4));
    p.segments = static_cast<Segment*>(take(kBanks * sizeof(Segment)));
    p.meta = static_cast<int32_t*>(take(4 * 4));
    p.tiles = static_cast<Segment*>(take((rall / 64 + kBanks + 10) * sizeof(Segment)));
    return p;
}

// Stable counting sort of routes by bank (ascending route within a bank; the
// shared expert's routes R + t are bank 256, in token order):
//   count      per 16-token block, the routed banks' route counts (LDS
//              histogram; fused into topk_kernel on the layer path)
//   bank scan  one wave per routed bank: exclusive running sums over blocks
//              (in place) and the bank total
//   scatter    every block scans the 257 bank totals into offsets; block 0
//              also writes offsets, segments, the MFMA tile list and meta; a
//              route's slot is offset + running sum + its rank in the block.
__global__ __launch_bounds__(kPermRoutes) void permute_count_kernel(const int32_t* __restrict__ ids, int T,
                                                                    int32_t* __restrict__ block_counts,
                                                                    uint32_t* sticky) {
    __shared__ int cnt[kExperts];
    for (int i = threadIdx.x; i < kExperts; i += kPermRoutes) cnt[i] = 0;
    __syncthreads();
    const int r = blockIdx.x * kPermRoutes + threadIdx.x;
    uint32_t flags = 0;
    if (r < T * kTop) {
        const int b = route_bank(ids, r, T * kTop, flags);
        if (b >= 0) atomicAdd(&cnt[b], 1);
    }
    flag_or(sticky, flags);
    __syncthreads();
    for (int i = threadIdx.x; i < kExperts; i += kPermRoutes) block_counts[size_t(blockIdx.x) * kExperts + i] = cnt[i];
}

__device__ __forceinline__ void permute_bank_scan_block(int blk, int nblocks, int32_t* __restrict__ block_counts,
                                                        int32_t* __restrict__ counts) {
    const int bank = blk * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (bank >= kExperts) return;
    constexpr int kRounds = 8;                       // 8 x 64 blocks = 8192 tokens
    int v[kRounds];
#pragma unroll
    for (int i = 0; i < kRounds; ++i) {
        const int b = 64 * i + lane;
        v[i] = b < nblocks ? block_counts[size_t(b) * kExperts + bank] : 0;
    }
    int run = 0;
#pragma unroll
    for (int i = 0; i < kRounds; ++i) {
        const int incl = wave_inclusive_scan(v[i]);
        const int b = 64 * i + lane;
        if (b < nblocks) block_counts[size_t(b) * kExperts + bank] = run + incl - v[i];
        run += __shfl(incl, 63, 64);
    }
    if (lane == 0) counts[bank] = run;
}

__global__ __launch_bounds__(256) void permute_bank_scan_kernel(int nblocks, int32_t* __restrict__ block_counts,
                                                                int32_t* __restrict__ counts) {
    permute_bank_scan_block(int(blockIdx.x), nblocks, block_counts, counts);
}

// The bank scan's kExperts / 4 blocks, then the activation quantisation's
// (act_bf16_block indices 0, 1, ...; neither part waits on the other).
__global__ __launch_bounds__(256) void permute_bank_scan_act_kernel(int nblocks, int32_t* __restrict__ block_counts,
                                                                    int32_t* __restrict__ counts, ActJob act,
                                                                    uint32_t* sticky) {
    const int b = int(blockIdx.x);
    if (b < kExperts / 4)
        permute_bank_scan_block(b, nblocks, block_counts, counts);
    else
        act_bf16_block<127>(b - kExperts / 4, act.x, kHidden, act.rows, kHidden / kGroup, act.ids, act.words,
                            act.scales, act.sums, sticky, kFlagNonfiniteInput, kFlagInvalidActivation);
}

__global__ __launch_bounds__(256) void permute_scatter_kernel(const int32_t* __restrict__ ids, int T, int shared_routes,
                                                              const int32_t* __restrict__ block_counts,
                                                              int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
                                                              int32_t* __restrict__ routes, Segment* __restrict__ segments,
                                                              int32_t* __restrict__ meta, Segment* __restrict__ tiles,
                                                              int mfma_rows) {
    __shared__ int s_off[kBanks + 1];        // exclusive route offsets (s_off[257] = live routes)
    __shared__ int s_tile[kBanks + 1];       // exclusive m-tile offsets (s_tile[257] = tiles)
    __shared__ __align__(16) int bank_of[kPermRoutes];
    const int tid = threadIdx.x, lane = tid & 63, R = T * kTop;
    // this thread's route, its bank and the running count of earlier blocks
    // (loaded before the offsets are ready)
    const int r = blockIdx.x * kPermRoutes + tid;
    uint32_t dummy = 0;
    int b = -1, before = 0;
    if (tid < kPermRoutes) {
        b = r < R ? route_bank(ids, r, R, dummy) : -1;
        if (b >= 0) before = block_counts[size_t(blockIdx.x) * kExperts + b];
        bank_of[tid] = b;
    }
    if (tid < 64) {
        // bank totals -> offsets, non-empty ranks and m-tile offsets (lane holds
        // banks 4 lane .. 4 lane + 3; the shared bank 256 follows)
        int tot[4], nt[4], ne[4], part = 0, ntp = 0, nep = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            tot[i] = counts[4 * lane + i];
            nt[i] = (tot[i] + mfma_rows - 1) / mfma_rows;
            ne[i] = tot[i] > 0 ? 1 : 0;
            part += tot[i];
            ntp += nt[i];
            nep += ne[i];
        }
        const int incl = wave_inclusive_scan(part), nt_incl = wave_inclusive_scan(ntp);
        const int ne_incl = wave_inclusive_scan(nep);
        int off = incl - part, tb = nt_incl - ntp, seg = ne_incl - nep;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = 4 * lane + i;
            s_off[e] = off;
            s_tile[e] = tb;
            if (blockIdx.x == 0) {
                offsets[e] = off;
                if (tot[i] > 0) segments[seg] = Segment{e, off, tot[i], tb};
            }
            off += tot[i];
            tb += nt[i];
            seg += ne[i];
        }
        if (lane == 63) {
            const int snt = (shared_routes + mfma_rows - 1) / mfma_rows;
            s_off[kExperts] = off;
            s_off[kBanks] = off + shared_routes;
            s_tile[kExperts] = tb;
            s_tile[kBanks] = tb + snt;
            if (blockIdx.x == 0) {
                offsets[kExperts] = off;
                offsets[kBanks] = off + shared_routes;
                counts[kExperts] = shared_routes;
                if (shared_routes > 0) segments[seg] = Segment{kExperts, off, shared_routes, tb};
                meta[0] = seg + (shared_routes > 0 ? 1 : 0);
                meta[1] = tb + snt;
            }
        }
    }
    __syncthreads();
    // m-tiles, spread over the grid: tile i belongs to the bank e with
    // s_tile[e] <= i < s_tile[e + 1] (binary search; empty banks have no tiles)
    const int ntiles = s_tile[kBanks];
    for (int i = blockIdx.x * 256 + tid; i < ntiles; i += gridDim.x * 256) {
        int lo = 0, hi = kBanks;                    // s_tile[lo] <= i < s_tile[hi]
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (s_tile[mid] <= i) lo = mid; else hi = mid;
        }
        const int k = i - s_tile[lo], total = s_off[lo + 1] - s_off[lo];
        tiles[i] = Segment{lo, s_off[lo] + k * mfma_rows, min(mfma_rows, total - k * mfma_rows), k};
    }
    if (tid < kPermRoutes && b >= 0) {
        // rank in the block = earlier routes of the block with bank b: all of
        // an earlier token's eight, the first `slot` of this token's (a token
        // may name one expert twice); all 16 tokens' ids read at once
        const int tok = tid >> 3, slot = tid & 7;
        int rank = 0;
#pragma unroll
        for (int u = 0; u < kPermTokens; ++u) {
            const int4 lo = *reinterpret_cast<const int4*>(&bank_of[8 * u]);
            const int4 hi = *reinterpret_cast<const int4*>(&bank_of[8 * u + 4]);
            const int n = u < tok ? 8 : (u == tok ? slot : 0);
            const int hit = (n > 0 && lo.x == b) + (n > 1 && lo.y == b) + (n > 2 && lo.z == b) + (n > 3 && lo.w == b) +
                            (n > 4 && hi.x == b) + (n > 5 && hi.y == b) + (n > 6 && hi.z == b) + (n > 7 && hi.w == b);
            rank += hit;
        }
        routes[s_off[b] + before + rank] = r;
    } else if (tid >= kPermRoutes && tid < kPermRoutes + kPermTokens) {
        const int t = blockIdx.x * kPermTokens + (tid - kPermRoutes);
        if (t < shared_routes) routes[s_off[kExperts] + t] = R + t;
    }
}

hipError_t launch_permute(const int32_t* ids, int R, int T, bool with_shared, const PermuteScratch& p,
                          uint32_t* sticky, int mfma_rows, hipStream_t s, bool counted, const ActJob* act) {
    if (R != T * kTop) return hipErrorInvalidValue;
    const int nblocks = (T + kPermTokens - 1) / kPermTokens;
    if (nblocks > 8 * 64) return hipErrorInvalidValue;
    if (!counted) {
        timed_launch("permute_count", permute_count_kernel, dim3(nblocks), dim3(kPermRoutes), 0, s, ids, T,
                     p.block_counts, sticky);
        const hipError_t st = hipGetLastError();
        if (st != hipSuccess) return st;
    }
    if (act) {
        // act_bf16_block: four 4-group waves per block index
        const int act_blocks = (act->rows * (kHidden / kGroup) + 15) / 16;
        timed_launch("permute_scan_act", permute_bank_scan_act_kernel, dim3(kExperts / 4 + act_blocks), dim3(256), 0,
                     s, nblocks, p.block_counts, p.counts, *act, sticky);
    } else {
        timed_launch("permute_scan", permute_bank_scan_kernel, dim3(kExperts / 4), dim3(256), 0, s, nblocks,
                     p.block_counts, p.counts);
    }
    hipError_t st = hipGetLastError();
    if (st != hipSuccess) return st;
    timed_launch("permute_scatter", permute_scatter_kernel, dim3(nblocks), dim3(256), 0, s, ids, T,
                 with_shared ? T : 0, p.block_counts, p.counts, p.offsets, p.routes, p.segments, p.meta, p.tiles,
                 mfma_rows);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Unpermute: slot-order reduction (routed_storage_n32_consumer.cpp:176-184,
// 296-307).
// ---------------------------------------------------------------------------
// Eight columns per thread, four in each half of the row (thread j of a
// token: columns 4j.. and 1024 + 4j.., so every load instruction of a wave
// reads 1 KB contiguous); every slot's row is loaded unconditionally (rows
// of slots without a live id hold stale data and are dropped by the select),
// so all 18 row loads of a thread are in flight together.
template <bool STREAM>
__global__ __launch_bounds__(256) void reduce_kernel(const float* __restrict__ route_out,
                                                     const float* __restrict__ weights,
                                                     const int32_t* __restrict__ ids, int T,
                                                     float* __restrict__ final_f32, uint16_t* __restrict__ out,
                                                     const uint16_t* __restrict__ shared_logit,
                                                     const uint16_t* __restrict__ sigmoid_table,
                                                     uint16_t* __restrict__ shared_out, uint16_t* __restrict__ layer_out,
                                                     uint32_t* sticky) {
    constexpr int kCols = 8, kThreadsPerToken = kHidden / kCols;
    const size_t idx = size_t(blockIdx.x) * 256 + threadIdx.x;   // over T * H/8
    if (idx >= size_t(T) * kThreadsPerToken) return;
    const int t = int(idx / kThreadsPerToken);
    const int c = int(idx % kThreadsPerToken) * 4, c1 = c + kHidden / 2;
    int idv[kTop];
    float wv[kTop];
#pragma unroll
    for (int s = 0; s < kTop; ++s) { idv[s] = ids[t * kTop + s]; wv[s] = weights[t * kTop + s]; }
    float4 rv[kTop][2];
    // Route rows are read exactly once.  When they exceed what the caches
    // hold (STREAM), non-temporal loads keep them from displacing other
    // lines: 8192 tokens, 604 MB of rows, 156 -> 112 us; at 1120 tokens the
    // 82 MB are mostly still cached from the down projection and plain loads
    // are faster.
    auto stream4 = [](const float* p) {
        if constexpr (STREAM) {
            const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
            return make_float4(v[0], v[1], v[2], v[3]);
        } else {
            return *reinterpret_cast<const float4*>(p);
        }
    };
#pragma unroll
    for (int s = 0; s < kTop; ++s) {
        const float* row = route_out + size_t(t * kTop + s) * kHidden;
        rv[s][0] = stream4(row + c);
        rv[s][1] = stream4(row + c1);
    }
    const bool shared = sigmoid_table != nullptr;
    float4 sh[2] = {};
    float gate = 0.f;
    if (shared) {
        const float* row = route_out + size_t(T * kTop + t) * kHidden;
        sh[0] = stream4(row + c);
        sh[1] = stream4(row + c1);
        gate = bf16_bits_to_f32(sigmoid_table[shared_logit[t]]);
    }
    // slot-order fp32 sum (routed_storage_n32_consumer.cpp:176-184)
    float sum[kCols];
#pragma unroll
    for (int i = 0; i < kCols; ++i) sum[i] = 0.f;
#pragma unroll
    for (int s = 0; s < kTop; ++s) {
        const bool live = idv[s] >= 0 && idv[s] < kExperts;
        const float v[kCols] = {rv[s][0].x, rv[s][0].y, rv[s][0].z, rv[s][0].w,
                                rv[s][1].x, rv[s][1].y, rv[s][1].z, rv[s][1].w};
#pragma unroll
        for (int i = 0; i < kCols; ++i) sum[i] = live ? sum[i] + v[i] * wv[s] : sum[i];
    }
    uint32_t flags = 0;
    uint16_t o[kCols];
#pragma unroll
    for (int i = 0; i < kCols; ++i) {
        o[i] = f32_to_bf16_bits(sum[i]);
        if (!isfinite(sum[i]) || (o[i] & 0x7f80u) == 0x7f80u) flags |= kFlagNonfiniteOutput;
    }
    // bf16 columns 0-3 to row offset c, 4-7 to c1
    auto put = [](uint16_t* dst, const uint16_t h[kCols]) {
        *reinterpret_cast<uint2*>(dst) = make_uint2(h[0] | (uint32_t(h[1]) << 16), h[2] | (uint32_t(h[3]) << 16));
        *reinterpret_cast<uint2*>(dst + kHidden / 2) =
            make_uint2(h[4] | (uint32_t(h[5]) << 16), h[6] | (uint32_t(h[7]) << 16));
    };
    const size_t base = size_t(t) * kHidden + c;
    if (final_f32) {
        *reinterpret_cast<float4*>(final_f32 + base) = make_float4(sum[0], sum[1], sum[2], sum[3]);
        *reinterpret_cast<float4*>(final_f32 + base + kHidden / 2) = make_float4(sum[4], sum[5], sum[6], sum[7]);
    }
    if (out) put(out + base, o);
    if (shared) {
        const float sv[kCols] = {sh[0].x * gate, sh[0].y * gate, sh[0].z * gate, sh[0].w * gate,
                                 sh[1].x * gate, sh[1].y * gate, sh[1].z * gate, sh[1].w * gate};
        uint16_t so[kCols], lo[kCols];
#pragma unroll
        for (int i = 0; i < kCols; ++i) {
            if (!isfinite(sv[i])) flags |= kFlagNonfiniteOutput;
            so[i] = f32_to_bf16_bits(sv[i]);
            lo[i] = f32_to_bf16_bits(bf16_bits_to_f32(o[i]) + bf16_bits_to_f32(so[i]));
        }
        if (shared_out) put(shared_out + base, so);
        if (layer_out) put(layer_out + base, lo);
    }
    flag_or(sticky, flags);
}

hipError_t launch_reduce(const float* route_out, const float* weights, const int32_t* ids, int T, float* final_f32,
                         uint16_t* out, const uint16_t* shared_logit, const uint16_t* sigmoid_table,
                         uint16_t* shared_out, uint16_t* layer_out, uint32_t* sticky, hipStream_t s) {
    const size_t n = size_t(T) * (kHidden / 8);
    const size_t route_bytes = size_t(T) * (kTop + 1) * kHidden * 4;
    auto kernel = route_bytes > (size_t(128) << 20) ? reduce_kernel<true> : reduce_kernel<false>;
    timed_launch("reduce", kernel, dim3((n + 255) / 256), dim3(256), 0, s, route_out, weights, ids, T, final_f32, out,
                 shared_logit, sigmoid_table, shared_out, layer_out, sticky);
    return hipGetLastError();
}

}  // namespace ornith
