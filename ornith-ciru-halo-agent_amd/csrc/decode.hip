// Decode path for 2..32 tokens: the routed MoE layer as seven kernels, none of
// which waits on another block (kernel boundaries carry every hand-off), or,
// with the router, five, the first of which hands values between its blocks.
//
//   S1 decode_route_kernel     router logits, one wave per (router row, batch
//                              of 8 tokens), and the quantised gate input
//                              (H128 + A8/A4, half-wave layout).
//   S2 topk                    softmax/top-8, one wave per token (routing.hip),
//      decode_sort_kernel      then one block: stable counting sort of the
//                              routes into per-bank segments.
//   (With the router, S1 and S2 run by default as one launch whose blocks
//   hand logits and ids to each other: decode_route_select_kernel.)
//   S3 decode_gateup_kernel    block (segment, 16 gate + 16 up columns): the
//                              codes stay in registers while the segment's
//                              routes stream through four at a time; exact
//                              int8 dots, fp32 group tree, SiLU(gate)*up.
//   S5 decode_down_kernel      block (segment, 128 output columns), same
//                              scheme, writing route_out; its prologue runs
//                              H128 + quantisation of the segment's fp32
//                              middle rows (every block of a segment, as
//                              each needs all 512 values of its routes).
//   S6 reduce                  slot-order combination (+ shared expert).
//
// Arithmetic is the reference's (routed_storage_n32_consumer.cpp:22-307); the
// decomposition into kernels is this library's.  A single token takes
// decode1.hip.
#include "kernels.hpp"
#include "timing.hpp"
#include "topk.hpp"
#include "decode.hpp"
#include "handoff.hpp"

namespace ornith {

constexpr int kDecodeBanks = kExperts + 1;
constexpr int kMaxRoutes = kDecodeMaxTokens * (kTop + 1);
constexpr int kRouteChunk = 4;
constexpr int kTokenBatch = 8;

// Router wave gw's job: the four waves of a block take four consecutive
// router rows of one batch of 8 tokens, so they load the same token rows (L1
// hits after the first) and different weight rows; rows run to a multiple of
// 4 (waves past the last row have no job).
__device__ __forceinline__ void router_wave_job(int gw, int T, int& row, int& t0) {
    const int nb = (T + kTokenBatch - 1) / kTokenBatch, grp = gw >> 2;
    row = 4 * (grp / nb) + (gw & 3);
    t0 = (grp % nb) * kTokenBatch;
}
constexpr int router_waves_for(bool shared, int T) {
    return ((shared ? kExperts + 1 : kExperts) + 3) / 4 * 4 * ((T + kTokenBatch - 1) / kTokenBatch);
}

// ---------------------------------------------------------------------------
// S1
// ---------------------------------------------------------------------------
template <bool ROUTER, bool SHARED, int QMAX>
__global__ __launch_bounds__(256) void decode_route_kernel(DecodeArgs a, int router_waves) {
    const int T = a.T, lane = threadIdx.x & 63;
    const int gw = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (ROUTER && gw < router_waves) {
        int row, t0;
        router_wave_job(gw, T, row, t0);
        if (row > (SHARED ? kExperts : kExperts - 1)) return;
        const uint16_t* wrow = row < kExperts ? a.router_w + size_t(row) * kHidden : a.shared_gate_w;
        const bool has_bias = a.bias && row < kExperts;
        router_rows_wave(a.x, kHidden, T, t0, wrow, has_bias ? a.bias[row] : 0.f, has_bias, a.logits, kLogitStride,
                         row);
        return;
    }
    // quantised gate input: wave q handles groups 2(q%4), 2(q%4)+1 of token q/4
    const int q = gw - (ROUTER ? router_waves : 0);
    if (q >= T * 4) return;
    const int tok = q >> 2, job = (q & 3) * 2 + (lane >> 5), lp = lane & 31;
    uint32_t flags = 0;
    bool live = true;
    if (!ROUTER && !SHARED) {
        live = false;
#pragma unroll
        for (int s = 0; s < kTop; ++s) {
            const int id = a.ids_in[tok * kTop + s];
            live |= id >= 0 && id < kExperts;
        }
    }
    const uint4 raw = *reinterpret_cast<const uint4*>(a.x + size_t(tok) * kHidden + job * kGroup + lp * 8);
    const uint32_t rw[4] = {raw.x, raw.y, raw.z, raw.w};
    float v[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        v[2 * e] = bf16_bits_to_f32(rw[e] & 0xffffu);
        v[2 * e + 1] = bf16_bits_to_f32(rw[e] >> 16);
    }
    if (live) {
#pragma unroll
        for (int e = 0; e < 8; ++e) if (!isfinite(v[e])) flags |= kFlagNonfiniteInput;
        h128_half(v);
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = 0.f;
    }
    uint32_t w2[2];
    uint16_t sb;
    int sum;
    quantize_half_fast<QMAX>(v, w2, sb, sum, flags, kFlagNonfiniteInput | kFlagInvalidActivation,
                             kFlagInvalidActivation);
    const size_t g = size_t(tok) * 8 + job;
    *reinterpret_cast<uint2*>(a.x_words + g * 64 + 2 * lp) = make_uint2(w2[0], w2[1]);
    if (lp == 0) {
        a.x_scales[g] = sb;
        a.x_sums[g] = sum;
    }
    flag_or(a.sticky, flags);
}

// ---------------------------------------------------------------------------
// S2b (after the top-k kernel): one block.  Segments are the non-empty banks
// in bank order (0..255, 256 = shared); inside a segment routes keep their
// index order (route r = 8t + slot, shared route R + t).  Route r is thread
// r: its stable rank = routes of its bank in earlier 64-route chunks (chunk
// histograms, prefixed per bank) + earlier lanes of its own chunk (readlane
// scan inside the wave).
// ---------------------------------------------------------------------------
constexpr int kSegRoutes = 8;          // a segment longer than this is split into pieces of 8 routes
constexpr int kMaxSegments = kDecodeBanks + kMaxRoutes / kSegRoutes;

// NT threads, route r = tid + NT j (j < ceil(routes / NT)) in chunk r / 64,
// so a wave's lanes hold one chunk at a time.  ids: the token-major expert
// ids, global or LDS.
template <bool SHARED, int NT>
__device__ __forceinline__ void sort_routes_block(const DecodeArgs& a, const int32_t* ids) {
    constexpr int kRounds = (kMaxRoutes + NT - 1) / NT, kChunks = kRounds * NT / 64;
    __shared__ int s_hist[kChunks][kDecodeBanks];
    __shared__ int s_total[kDecodeBanks], s_off[kDecodeBanks];
    const int T = a.T, R = T * kTop, Rall = R + (SHARED ? T : 0);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int i = tid; i < kChunks * kDecodeBanks; i += NT) (&s_hist[0][0])[i] = 0;
    uint32_t flags = 0;
    int bank[kRounds], rank_in[kRounds];
#pragma unroll
    for (int j = 0; j < kRounds; ++j) {
        const int r = tid + NT * j;
        bank[j] = -1;
        if (r < R) {
            const int id = ids[r];
            bank[j] = (id >= 0 && id < kExperts) ? id : -1;
            if (bank[j] < 0 && id != -1) flags |= kFlagInvalidExpert;
        } else if (r < Rall) {
            bank[j] = kShared;
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kRounds; ++j) {
        if (bank[j] >= 0) atomicAdd(&s_hist[wave + (NT / 64) * j][bank[j]], 1);
        rank_in[j] = 0;
#pragma unroll 8
        for (int l = 0; l < 64; ++l) {
            const int bl = __builtin_amdgcn_readlane(bank[j], l);
            rank_in[j] += (l < lane && bl == bank[j]) ? 1 : 0;
        }
    }
    __syncthreads();
    for (int bk = tid; bk < kDecodeBanks; bk += NT) {
        int run = 0;
#pragma unroll
        for (int k = 0; k < kChunks; ++k) {
            const int c = s_hist[k][bk];
            s_hist[k][bk] = run;
            run += c;
        }
        s_total[bk] = run;
    }
    __syncthreads();
    if (wave == 0) {
        // exclusive scans of counts and of non-empty flags over 257 banks,
        // 5 banks per lane (lane-serial) then a wave scan of the lane totals
        int c[5], nz[5], tc = 0, tn = 0;
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            const int b = lane * 5 + i;
            c[i] = b < kDecodeBanks ? s_total[b] : 0;
            nz[i] = (c[i] + kSegRoutes - 1) / kSegRoutes;      // pieces of this bank
            tc += c[i];
            tn += nz[i];
        }
        const int ic = wave_prefix_sum(tc), in = wave_prefix_sum(tn);
        int runc = ic - tc, runn = in - tn;
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            const int b = lane * 5 + i;
            if (b < kDecodeBanks) {
                s_off[b] = runc;
                for (int k = 0; k < nz[i]; ++k)
                    a.segments[runn + k] = Segment{b, runc + k * kSegRoutes, min(kSegRoutes, c[i] - k * kSegRoutes), 0};
            }
            runc += c[i];
            runn += nz[i];
        }
        if (lane == 63) { a.nseg[0] = in; a.nseg[1] = ic; }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kRounds; ++j)
        if (bank[j] >= 0)
            a.routes[s_off[bank[j]] + s_hist[wave + (NT / 64) * j][bank[j]] + rank_in[j]] = tid + NT * j;
    flag_or(a.sticky, flags);
}

// The same order when every token's ids are distinct (the router's top-8):
// a route's rank in its bank is the number of earlier tokens that chose the
// bank, so one 32-bit token mask per bank (T <= 32) replaces the chunk
// histograms and the in-wave rank loops.
template <bool SHARED, int NT>
__device__ __forceinline__ void sort_routes_masks(const DecodeArgs& a, const int32_t* ids) {
    __shared__ uint32_t s_mask[kDecodeBanks];
    __shared__ int s_off[kDecodeBanks];
    const int T = a.T, R = T * kTop, Rall = R + (SHARED ? T : 0);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t all = T >= 32 ? 0xffffffffu : (1u << T) - 1u;
    for (int i = tid; i < kDecodeBanks; i += NT) s_mask[i] = (SHARED && i == kShared) ? all : 0u;
    uint32_t flags = 0;
    __syncthreads();
    for (int r = tid; r < R; r += NT) {
        const int id = ids[r];
        if (id >= 0 && id < kExperts) atomicOr(&s_mask[id], 1u << (r >> 3));
        else if (id != -1) flags |= kFlagInvalidExpert;
    }
    __syncthreads();
    if (wave == 0) {
        // exclusive scans of counts and of segment pieces over 257 banks,
        // 5 banks per lane (lane-serial) then a wave scan of the lane totals
        int c[5], nz[5], tc = 0, tn = 0;
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            const int b = lane * 5 + i;
            c[i] = b < kDecodeBanks ? __popc(s_mask[b]) : 0;
            nz[i] = (c[i] + kSegRoutes - 1) / kSegRoutes;
            tc += c[i];
            tn += nz[i];
        }
        const int ic = wave_prefix_sum(tc), in = wave_prefix_sum(tn);
        int runc = ic - tc, runn = in - tn;
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            const int b = lane * 5 + i;
            if (b < kDecodeBanks) {
                s_off[b] = runc;
                for (int k = 0; k < nz[i]; ++k)
                    a.segments[runn + k] = Segment{b, runc + k * kSegRoutes, min(kSegRoutes, c[i] - k * kSegRoutes), 0};
            }
            runc += c[i];
            runn += nz[i];
        }
        if (lane == 63) { a.nseg[0] = in; a.nseg[1] = ic; }
    }
    __syncthreads();
    for (int r = tid; r < Rall; r += NT) {
        int bank = kShared, t = r - R;
        if (r < R) {
            const int id = ids[r];
            bank = (id >= 0 && id < kExperts) ? id : -1;
            t = r >> 3;
        }
        if (bank >= 0) a.routes[s_off[bank] + __popc(s_mask[bank] & ((1u << t) - 1u))] = r;
    }
    flag_or(a.sticky, flags);
}

// DISTINCT: the ids are the router's top-8 (distinct within a token)
template <bool SHARED, bool DISTINCT>
__global__ __launch_bounds__(512) void decode_sort_kernel(DecodeArgs a, const int32_t* __restrict__ ids) {
    if constexpr (DISTINCT) sort_routes_masks<SHARED, 512>(a, ids);
    else sort_routes_block<SHARED, 512>(a, ids);
}

// ---------------------------------------------------------------------------
// S1 + S2 in one launch (router and shared expert, 2..32 tokens).  Blocks of
// 4 waves take the waves of S1 (router row waves, then the gate-input waves);
// each router wave also publishes its logits as tagged words (handoff.hpp).
// Wave w of block L < ceil(T / 4) then selects token 4L + w from the tagged
// logits (the per-token selection of routing.hip's top-k) and publishes its
// eight ids; block 0 gathers the ids and runs the sort above.  Every block
// publishes an arrival word after its first barrier (by then every wave has
// read the sequence number); block 0 advances the number once all have
// arrived.  Waits are bounded (kFlagHandoffTimeout); the launcher uses this
// kernel only when the whole grid is resident at once.
// ---------------------------------------------------------------------------
template <bool SHARED, int QMAX>
__global__ __launch_bounds__(256) void decode_route_select_kernel(DecodeArgs a, int router_waves) {
    __shared__ __align__(16) uint64_t s_cand[4][66];
    __shared__ uint2 s_sel[4][kTop];
    __shared__ int32_t s_ids[kDecodeMaxTokens * kTop];
    const int T = a.T, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int L = int(blockIdx.x), gw = L * 4 + wave;
    uint64_t* W = a.l1_words;
    // the call's sequence number: loaded first, its value taken only after
    // each wave's own loads (router rows, x) are issued and used
    uint32_t seq_v = __hip_atomic_load(a.l1_seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint32_t flags = 0;
    int row = 0, t0 = 0;
    if (gw < router_waves) router_wave_job(gw, T, row, t0);
    if (gw < router_waves && row <= (SHARED ? kExperts : kExperts - 1)) {
        const uint16_t* wrow = row < kExperts ? a.router_w + size_t(row) * kHidden : a.shared_gate_w;
        const bool has_bias = a.bias && row < kExperts;
        router_rows_wave(a.x, kHidden, T, t0, wrow, has_bias ? a.bias[row] : 0.f, has_bias, a.logits, kLogitStride,
                         row, W, seq_v, uint32_t(kDecodeRouteLogit + kDecodeMaxTokens * row + t0));
    } else if (gw < router_waves) {
        // a padding wave of the last row group: no router row
    } else if (gw - router_waves < T * 4) {
        // quantised gate input: wave q handles groups 2(q%4), 2(q%4)+1 of token q/4
        const int q = gw - router_waves;
        const int tok = q >> 2, job = (q & 3) * 2 + (lane >> 5), lp = lane & 31;
        const uint4 raw = *reinterpret_cast<const uint4*>(a.x + size_t(tok) * kHidden + job * kGroup + lp * 8);
        const uint32_t rw[4] = {raw.x, raw.y, raw.z, raw.w};
        float v[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[2 * e] = bf16_bits_to_f32(rw[e] & 0xffffu);
            v[2 * e + 1] = bf16_bits_to_f32(rw[e] >> 16);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) if (!isfinite(v[e])) flags |= kFlagNonfiniteInput;
        h128_half(v);
        uint32_t w2[2];
        uint16_t sb;
        int sum;
        quantize_half_fast<QMAX>(v, w2, sb, sum, flags, kFlagNonfiniteInput | kFlagInvalidActivation,
                                 kFlagInvalidActivation);
        const size_t g = size_t(tok) * 8 + job;
        *reinterpret_cast<uint2*>(a.x_words + g * 64 + 2 * lp) = make_uint2(w2[0], w2[1]);
        if (lp == 0) {
            a.x_scales[g] = sb;
            a.x_sums[g] = sum;
        }
    }
    // every wave has its sequence number before the barrier, so before the
    // block's arrival word (waves with loads have long had it: their loads
    // were issued after it and are done)
    asm volatile("" : "+v"(seq_v));
    const uint32_t seq = __builtin_amdgcn_readfirstlane(seq_v);
    const int limit = l1_limit(seq, a.handoff_spins);
    __syncthreads();
    if (threadIdx.x == 0) l1_put(W, kDecodeRouteArrive + 8 * L, seq, 1u);

    // ---- selection of token 4L + wave ----
    const int t = L * 4 + wave;
    if (t < T) {
        uint32_t idx[5], got[5];
#pragma unroll
        for (int i = 0; i < 4; ++i) idx[i] = kDecodeRouteLogit + kDecodeMaxTokens * (lane + 64 * i) + t;
        idx[4] = SHARED ? kDecodeRouteLogit + kDecodeMaxTokens * kExperts + t : idx[3];   // the shared gate row
        if (!l1_wait<5, 0>(W, idx, seq, got, limit)) flags |= kFlagHandoffTimeout;
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = __uint_as_float(got[i]);
        uint32_t k[4];
        softmax_keys(v, k);
        top8_rank_lds(k, s_cand[wave], s_sel[wave]);
        float tot = 0.f;
#pragma unroll
        for (int j = 0; j < kTop; ++j) tot = tot + __uint_as_float(s_sel[wave][j].x);
        if (lane < kTop) {
            const uint2 pick = s_sel[wave][lane];
            a.topk_w[size_t(t) * kTop + lane] = fdiv_rn(__uint_as_float(pick.x), tot);
            a.topk_ids[size_t(t) * kTop + lane] = int(pick.y);
            l1_put(W, kDecodeRouteIds + kTop * t + lane, seq, pick.y);
        }
        if (SHARED && lane == 0) a.shared_logit[t] = f32_to_bf16_bits(__uint_as_float(got[4]));
    }

    // ---- block 0: gather the ids, sort, advance the sequence number ----
    if (L == 0) {
        const int R = T * kTop;
        if (wave * 64 < R) {                           // R <= 256: one id word per thread
            const int r = min(wave * 64 + lane, R - 1);
            uint32_t idx[1] = {uint32_t(kDecodeRouteIds + r)}, got[1];
            if (!l1_wait<1, 0>(W, idx, seq, got, limit)) flags |= kFlagHandoffTimeout;
            if (wave * 64 + lane < R) s_ids[wave * 64 + lane] = int32_t(got[0]);
        }
        __syncthreads();
        sort_routes_masks<SHARED, 256>(a, s_ids);
        if (wave == 0) {
            const int nblocks = int(gridDim.x);
            uint32_t idx[5], got[5];
#pragma unroll
            for (int i = 0; i < 5; ++i) idx[i] = kDecodeRouteArrive + 8 * min(lane + 64 * i, nblocks - 1);
            // advance only once every block has read `seq` (see handoff.hpp)
            const bool arrived = l1_wait<5, 1>(W, idx, seq, got, limit);
            if (!arrived) flags |= kFlagHandoffTimeout;
            if (lane == 0)
                __hip_atomic_store(a.l1_seq, arrived ? l1_next_seq(seq) : kSeqPoisoned, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    flag_or(a.sticky, flags);
}

// ---------------------------------------------------------------------------
// S3: block (segment, p): gate columns 32p..32p+31 and up columns 512+32p..
// (one whole 32-column tile each).  Wave g = group g; lane = local column
// (0..31 gate, 32..63 up), so every load instruction reads two whole 128-byte
// rows.  Each thread keeps its 32 code words in registers while the
// segment's routes stream through four at a time; the next chunk's
// activations load while the current one computes.
// ---------------------------------------------------------------------------
template <bool SHARED>
__global__ __launch_bounds__(512) void decode_gateup_kernel(DecodeArgs a) {
    __shared__ __align__(16) uint32_t la[kRouteChunk][512];
    __shared__ float lsa[kRouteChunk][8], lss[kRouteChunk][8];
    __shared__ float lterm[kRouteChunk][8][64];
    __shared__ int lr[256];
    // segments in reverse bank order: the shared expert's (longest, last)
    // segment is dispatched first
    const int nseg = a.nseg[0];
    if (int(blockIdx.y) >= nseg) return;
    const Segment sg = a.segments[nseg - 1 - int(blockIdx.y)];
    const int tid = threadIdx.x, lane = tid & 63, g = tid >> 6, p = blockIdx.x, R = a.T * kTop;
    const bool shared = SHARED && sg.bank == kShared;
    const uint32_t* codes = shared ? a.s13_codes : a.w13_codes + size_t(sg.bank) * kGateBankWords;
    const uint32_t* meta = shared ? a.s13_meta : a.w13_meta + size_t(sg.bank) * kGateBankMeta;
    // route list first (waiting for it must not wait for the codes)
    const int route_in = a.routes[sg.first + min(tid, sg.count - 1)];
    __builtin_amdgcn_sched_barrier(0);
    const int col = (lane < 32 ? 0 : kInter) + 32 * p + (lane & 31);
    const BankView bv = bank_view(shared);
    const uint32_t* wp = codes + bv.word(col, g, 8);
    uint32_t wr[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) wr[j] = load_once(wp + j * bv.stride());
    const uint32_t mw = meta[bv.meta(col, g, 8)];
    if (tid < sg.count) lr[tid] = route_in;
    __syncthreads();
    // staging registers for one chunk: route rr = tid / 128 holds words
    // (tid % 128) * 4 .. + 3 of its row; threads tid < 32 also hold the
    // (route tid / 8, group tid % 8) scale and sum
    u32x4 areg;
    uint32_t sreg = 0;
    int sumreg = 0;
    auto load_chunk = [&](int r0) {
        const int k = min(r0 + (tid >> 7), sg.count - 1);
        const int route = lr[k];
        const int row = route < R ? route / kTop : route - R;
        areg = *reinterpret_cast<const u32x4*>(a.x_words + size_t(row) * 512 + (tid & 127) * 4);
        const int k2 = min(r0 + ((tid & 31) >> 3), sg.count - 1);
        const int route2 = lr[k2];
        const int row2 = route2 < R ? route2 / kTop : route2 - R;
        sreg = a.x_scales[size_t(row2) * 8 + (tid & 7)];
        sumreg = a.x_sums[size_t(row2) * 8 + (tid & 7)];
    };
    uint32_t flags = 0;
    load_chunk(0);
    for (int r0 = 0; r0 < sg.count; r0 += kRouteChunk) {
        const int nr = min(kRouteChunk, sg.count - r0);
        __syncthreads();                                   // previous chunk's readers are done
        *reinterpret_cast<u32x4*>(&la[tid >> 7][(tid & 127) * 4]) = areg;
        if (tid < 32) {
            const float sc = f16_bits_to_f32(uint16_t(sreg));
            lsa[tid >> 3][tid & 7] = sc;
            lss[tid >> 3][tid & 7] = sc * float(sumreg);
        }
        __syncthreads();
        if (r0 + kRouteChunk < sg.count) load_chunk(r0 + kRouteChunk);
        for (int rr = 0; rr < nr; ++rr) {
            const uint4* ab = reinterpret_cast<const uint4*>(&la[rr][g * 64]);
            int dot = 0;
#pragma unroll
            for (int c4 = 0; c4 < 16; ++c4) {
                const uint4 av = ab[c4];
                dot = dot4(code_even(wr[2 * c4]), int(av.x), dot);
                dot = dot4(code_odd(wr[2 * c4]), int(av.y), dot);
                dot = dot4(code_even(wr[2 * c4 + 1]), int(av.z), dot);
                dot = dot4(code_odd(wr[2 * c4 + 1]), int(av.w), dot);
            }
            lterm[rr][g][lane] = tree_term(dot, lsa[rr][g], lss[rr][g], mw);
        }
        __syncthreads();
        if (tid < nr * 32) {
            const int rr = tid >> 5, c = tid & 31;
            float vg = 0.f, vu = 0.f;
#pragma unroll
            for (int gg = 0; gg < 8; ++gg) vg = vg + lterm[rr][gg][c];
#pragma unroll
            for (int gg = 0; gg < 8; ++gg) vu = vu + lterm[rr][gg][32 + c];
            float mid;
            if (shared) {
                // shared linear outputs are bf16; tabulated SiLU; bf16 product
                // (routed_storage_n32_consumer.cpp:226-227, 246-250)
                vg = bf16_round(vg);
                vu = bf16_round(vu);
                if (!isfinite(vg) || !isfinite(vu)) flags |= kFlagNonfiniteProjection;
                mid = bf16_round(a.silu_table[__float_as_uint(vg) >> 16] * vu);
            } else {
                if (!isfinite(vg) || !isfinite(vu)) flags |= kFlagNonfiniteProjection;
                mid = silu_portable_wave(vg) * vu;
            }
            if (!isfinite(mid)) flags |= kFlagNonfiniteMiddle | kFlagNonfiniteInput;
            a.middle[size_t(lr[r0 + rr]) * kInter + p * 32 + c] = mid;
        }
    }
    flag_or(a.sticky, flags);
}

// ---------------------------------------------------------------------------
// S5: block (segment, CPB 32-column tiles c).  Wave q = chunk quarter (chunks
// 8q..8q+7); lane = (group lane / 32, column lane % 32), so every load
// instruction reads two whole 128-byte rows.  The quarters' exact integer
// partial dots meet in LDS; the two groups' terms follow in group order.  The
// segment's routes and activations are loaded once for the block's tiles.
// The activations are the fp32 middle rows: wave rr of a chunk takes route
// rr, lane half = group, 8 consecutive values per lane (the half-wave layout
// of the gate input), and runs H128 + A8/A4 quantisation itself (the
// arithmetic of the reference's down input, routed_storage_n32_consumer.cpp:
// 231-295) before the words go to LDS.
// Measured alternatives (2..32 tokens): a separate quantisation kernel (4.6 us
// at 32 tokens against +3.5 us here); quantising waves apart from the code
// loads in 8-wave blocks (half the resident blocks: 38 us); a fixed grid of
// 1024 blocks walking the items (items run serially per block: 29 us).
// ---------------------------------------------------------------------------
template <bool SHARED, int CPB, int QMAX>
__global__ __launch_bounds__(256) void decode_down_kernel(DecodeArgs a) {
    __shared__ __align__(16) uint32_t la[kRouteChunk][128];
    __shared__ float lsa[kRouteChunk][2], lss[kRouteChunk][2];
    __shared__ int lpart[CPB][kRouteChunk][4][64];
    __shared__ int lr[kSegRoutes];
    const int nseg = a.nseg[0];
    if (int(blockIdx.y) >= nseg) return;
    const Segment sg = a.segments[nseg - 1 - int(blockIdx.y)];    // shared expert's segments first
    const int tid = threadIdx.x, lane = tid & 63, q = tid >> 6, c0 = blockIdx.x * CPB;
    const bool shared = SHARED && sg.bank == kShared;
    const uint32_t* codes = shared ? a.s2_codes : a.w2_codes + size_t(sg.bank) * kDownBankWords;
    const uint32_t* meta = shared ? a.s2_meta : a.w2_meta + size_t(sg.bank) * kDownBankMeta;
    const int route_in = a.routes[sg.first + min(tid, sg.count - 1)];
    __builtin_amdgcn_sched_barrier(0);
    const int g = lane >> 5, n = lane & 31;
    uint32_t wr[CPB][8], mw[CPB];
    const BankView bv = bank_view(shared);
#pragma unroll
    for (int cc = 0; cc < CPB; ++cc) {
        const uint32_t* wp = codes + bv.word(32 * (c0 + cc) + n, g, 2) + 8 * q * bv.stride();
#pragma unroll
        for (int j = 0; j < 8; ++j) wr[cc][j] = load_once(wp + j * bv.stride());
    }
#pragma unroll
    for (int cc = 0; cc < CPB; ++cc) mw[cc] = meta[bv.meta(32 * (c0 + cc) + n, g, 2)];   // epilogue thread (g, n)
    if (tid < sg.count) lr[tid] = route_in;
    __syncthreads();
    float4 m0, m1;
    auto load_chunk = [&](int r0) {
        // route rr = tid / 64: values 8 (lane % 32) .. + 7 of group lane / 32
        // of its fp32 middle row (dead routes of a chunk repeat the last one)
        const float* src = a.middle + size_t(lr[min(r0 + q, sg.count - 1)]) * kInter + 8 * lane;
        m0 = *reinterpret_cast<const float4*>(src);
        m1 = *reinterpret_cast<const float4*>(src + 4);
    };
    uint32_t flags = 0;
    load_chunk(0);
    for (int r0 = 0; r0 < sg.count; r0 += kRouteChunk) {
        const int nr = min(kRouteChunk, sg.count - r0);
        float v[8] = {m0.x, m0.y, m0.z, m0.w, m1.x, m1.y, m1.z, m1.w};
        h128_half(v);
        uint32_t w2[2];
        uint16_t sb;
        int sum;
        quantize_half_fast<QMAX>(v, w2, sb, sum, flags, kFlagNonfiniteInput | kFlagInvalidActivation,
                                 kFlagInvalidActivation);
        __syncthreads();                                   // previous chunk's readers are done
        *reinterpret_cast<uint2*>(&la[q][2 * lane]) = make_uint2(w2[0], w2[1]);
        if ((lane & 31) == 0) {
            const float sc = f16_bits_to_f32(sb);
            lsa[q][g] = sc;
            lss[q][g] = sc * float(sum);
        }
        __syncthreads();
        if (r0 + kRouteChunk < sg.count) load_chunk(r0 + kRouteChunk);
        for (int rr = 0; rr < nr; ++rr) {
            const uint4* ab = reinterpret_cast<const uint4*>(&la[rr][g * 64 + 16 * q]);
            uint4 av[4];
#pragma unroll
            for (int c4 = 0; c4 < 4; ++c4) av[c4] = ab[c4];
#pragma unroll
            for (int cc = 0; cc < CPB; ++cc) {
                int dot = 0;
#pragma unroll
                for (int c4 = 0; c4 < 4; ++c4) {
                    dot = dot4(code_even(wr[cc][2 * c4]), int(av[c4].x), dot);
                    dot = dot4(code_odd(wr[cc][2 * c4]), int(av[c4].y), dot);
                    dot = dot4(code_even(wr[cc][2 * c4 + 1]), int(av[c4].z), dot);
                    dot = dot4(code_odd(wr[cc][2 * c4 + 1]), int(av[c4].w), dot);
                }
                lpart[cc][rr][q][lane] = dot;
            }
        }
        __syncthreads();
        if (tid < nr * 64) {
            // thread (route rr, group, column): the exact dot, then the group term
            const int rr = tid >> 6;
#pragma unroll
            for (int cc = 0; cc < CPB; ++cc) {
                const int dot = lpart[cc][rr][0][lane] + lpart[cc][rr][1][lane] + lpart[cc][rr][2][lane] +
                                lpart[cc][rr][3][lane];
                const float term = tree_term(dot, lsa[rr][g], lss[rr][g], mw[cc]);
                const float term1 = xor_perm_f<32>(term);       // group 1 of the same column
                if (g == 0) {
                    float v = 0.f;
                    v = v + term;
                    v = v + term1;
                    if (shared) v = bf16_round(v);
                    if (!isfinite(v)) flags |= kFlagNonfiniteProjection;
                    a.route_out[size_t(lr[r0 + rr]) * kHidden + (c0 + cc) * 32 + n] = v;
                }
            }
        }
    }
    flag_or(a.sticky, flags);
}

// ---------------------------------------------------------------------------
size_t decode_scratch_bytes() {
    return align256(size_t(kDecodeMaxTokens) * kLogitStride * 4) + align256(kMaxSegments * sizeof(Segment)) +
           align256(kMaxRoutes * 4) + align256(8) + align256(4) + align256(size_t(kHandoffWords) * 8);
}

void carve_decode(void* base, DecodeArgs& a) {
    size_t off = 0;
    auto take = [&](size_t bytes) { void* q = at<void>(base, off); off += align256(bytes); return q; };
    a.logits = static_cast<float*>(take(size_t(kDecodeMaxTokens) * kLogitStride * 4));
    a.segments = static_cast<Segment*>(take(kMaxSegments * sizeof(Segment)));
    a.routes = static_cast<int32_t*>(take(kMaxRoutes * 4));
    a.nseg = static_cast<int32_t*>(take(8));
    a.l1_seq = static_cast<uint32_t*>(take(4));
    a.l1_words = static_cast<uint64_t*>(take(size_t(kHandoffWords) * 8));
}

constexpr int kDownTilesPerBlock = 4;    // 32-column down tiles per block (2048 / 32 / 4 = 16 blocks per segment)

// Whether `blocks` blocks of the one-launch route kernel are resident at once
// on the device that runs stream `s` (occupancy checked once per device).
template <bool SHARED, int QMAX>
static bool route_select_fits(int blocks, hipStream_t s) {
    constexpr int kMaxDevices = 64;
    static std::atomic<int> capacity[kMaxDevices];   // resident blocks; 0 unknown, -1 query failed
    const int dev = stream_device(s);
    if (dev < 0 || dev >= kMaxDevices) return false;
    int cap = capacity[dev].load(std::memory_order_relaxed);
    if (cap == 0) {
        cap = resident_blocks(decode_route_select_kernel<SHARED, QMAX>, 256, dev);
        capacity[dev].store(cap, std::memory_order_relaxed);
    }
    return cap >= blocks;
}

std::atomic<int> g_route_select_mode{0};   // 0 automatic, 1 separate route / top-k / sort kernels

template <bool ROUTER, bool SHARED, int QMAX>
static hipError_t run(const DecodeArgs& a, hipStream_t s) {
    const int T = a.T, R = T * kTop;
    const int router_waves = ROUTER ? router_waves_for(SHARED, T) : 0;
    const int s1_waves = router_waves + T * 4;
    hipError_t st;
    bool fused = false;
    if constexpr (ROUTER) {
        const int fused_blocks = (s1_waves + 3) / 4;
        if (fused_blocks <= kDecodeRouteMaxBlocks && g_route_select_mode.load(std::memory_order_relaxed) == 0 &&
            route_select_fits<SHARED, QMAX>(fused_blocks, s)) {
            DecodeArgs b = a;
            b.handoff_spins = g_handoff_spins.load(std::memory_order_relaxed);
            timed_launch("route_select", decode_route_select_kernel<SHARED, QMAX>, dim3(fused_blocks), dim3(256), 0, s,
                         b, router_waves);
            st = hipGetLastError();
            if (st != hipSuccess) return st;
            fused = true;
        }
    }
    if (!fused) {
        timed_launch("route", decode_route_kernel<ROUTER, SHARED, QMAX>, dim3((s1_waves + 3) / 4), dim3(256), 0, s, a,
                     router_waves);
        st = hipGetLastError();
        if (st != hipSuccess) return st;
        if (ROUTER) {
            st = launch_topk(a.logits, kLogitStride, T, a.topk_w, a.topk_ids, SHARED ? a.logits + kExperts : nullptr,
                             kLogitStride, SHARED ? a.shared_logit : nullptr, s);
            if (st != hipSuccess) return st;
        }
        timed_launch("sort", decode_sort_kernel<SHARED, ROUTER>, dim3(1), dim3(512), 0, s, a, ROUTER ? a.topk_ids : a.ids_in);
        st = hipGetLastError();
        if (st != hipSuccess) return st;
    }
    // segments: at most one per non-empty bank plus one per extra 8 routes
    const int maxseg = min(R, kExperts) + (SHARED ? 1 : 0) + (R + (SHARED ? T : 0)) / kSegRoutes;
    timed_launch("gateup", decode_gateup_kernel<SHARED>, dim3(kInter / 32, maxseg), dim3(512), 0, s, a);
    st = hipGetLastError();
    if (st != hipSuccess) return st;
    timed_launch("down", decode_down_kernel<SHARED, kDownTilesPerBlock, QMAX>,
                 dim3(kHidden / (32 * kDownTilesPerBlock), maxseg), dim3(256), 0, s, a);
    st = hipGetLastError();
    if (st != hipSuccess) return st;
    return launch_reduce(a.route_out, a.reduce_w, a.reduce_ids, T, a.final_f32, a.out, a.shared_logit,
                         SHARED ? a.sigmoid_table : nullptr, a.shared_out, a.layer_out, a.sticky, s);
}

hipError_t launch_decode(const DecodeArgs& a, bool router, bool shared, int qmax, hipStream_t s) {
    if (a.T <= 0 || a.T > kDecodeMaxTokens) return hipErrorInvalidValue;
    if (a.T == 1) return launch_decode1(a, router, shared, qmax, s);
    if (router && shared) return run<true, true, 127>(a, s);
    if (router) return run<true, false, 127>(a, s);
    if (shared) return run<false, true, 127>(a, s);
    if (qmax == 127) return run<false, false, 127>(a, s);
    return run<false, false, 7>(a, s);
}

}  // namespace ornith
