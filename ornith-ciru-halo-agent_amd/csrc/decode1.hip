// Single-token decode (T == 1): three kernels with one global-load level of
// routing latency each.
//
//   D1 decode1_route_kernel    router logits (257 waves, one row each) and
//                              the quantised gate input (8 more waves).
//   D2 decode1_gateup_kernel   block (slot s, p): 16 gate + 16 up columns of
//                              slot s (slots 0..7 routed, 8 the shared
//                              expert), 288 blocks.  The activation loads
//                              (and, for the shared slot, the weights) start
//                              at once; routed blocks derive their expert
//                              with an in-block softmax/top-8 of the 257
//                              logits (threshold + rank count, topk.hpp).
//                              Codes go straight to registers.  The middle
//                              row leaves with the first four H128
//                              butterflies of the down input applied.
//   D3 decode1_down_kernel     block = 16 output columns over all slots (128
//                              blocks, one wave per slot): the last three
//                              H128 butterflies + A8 of the slot's middle
//                              row, exact dots, fp32 tree and the
//                              slot-order reduction.
//
// One token has no expert reuse, so slots are processed as they come (no
// permutation); a slot repeated by the caller simply loads its weights twice.
// Arithmetic: routed_storage_n32_consumer.cpp:22-307.
#include "kernels.hpp"
#include "timing.hpp"
#include "topk.hpp"
#include "decode.hpp"
#include "handoff.hpp"
#include <atomic>

namespace ornith {

constexpr int kSlots = kTop + 1;

// Blocks 2m and 2m+1 of a kernel read the two 64-byte halves of the same
// 128-byte code rows.  Workgroups go to the 8 XCDs round-robin, so linear
// block L = 16q + 8h + x is mapped to pair 8q + x, half h: both halves of a
// row then come through one XCD's L2 and each row is fetched once.
__device__ __forceinline__ int xcd_paired_block(int L) {
    const int x = L & 7, h = (L >> 3) & 1, q = L >> 4;
    return 2 * (8 * q + x) + h;
}

// ---------------------------------------------------------------------------
template <bool ROUTER, bool SHARED, int QMAX>
__global__ __launch_bounds__(64) void decode1_route_kernel(DecodeArgs a) {
    const int lane = threadIdx.x;
    const int gw = blockIdx.x;                       // one wave per block
    uint32_t flags = 0;
    const int nrows = ROUTER ? (SHARED ? kExperts + 1 : kExperts) : 0;
    if (gw < nrows) {
        const uint16_t* wrow = gw < kExperts ? a.router_w + size_t(gw) * kHidden : a.shared_gate_w;
        uint4 wv[4], xv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            wv[i] = *reinterpret_cast<const uint4*>(wrow + (i * 64 + lane) * 8);
            xv[i] = *reinterpret_cast<const uint4*>(a.x + (i * 64 + lane) * 8);
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
        float v = wave_butterfly_sum(acc);
        if (a.bias && gw < kExperts) v = v + a.bias[gw];
        if (lane == 0) a.logits[gw] = v;
        return;
    }
    // quantised gate input: two groups per wave (half-wave layout)
    const int job = 2 * (gw - nrows) + (lane >> 5), lp = lane & 31;
    bool live = true;
    if (!ROUTER && !SHARED) {
        live = false;
#pragma unroll
        for (int s = 0; s < kTop; ++s) {
            const int id = a.ids_in[s];
            live |= id >= 0 && id < kExperts;
        }
    }
    const uint4 raw = *reinterpret_cast<const uint4*>(a.x + job * kGroup + lp * 8);
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
    // a non-finite transformed value raises both flags (as the separate check
    // and the quantiser's own did)
    quantize_half_fast<QMAX>(v, w2, sb, sum, flags, kFlagNonfiniteInput | kFlagInvalidActivation,
                             kFlagInvalidActivation);
    *reinterpret_cast<uint2*>(a.x_words + job * 64 + 2 * lp) = make_uint2(w2[0], w2[1]);
    if (lp == 0) {
        a.x_scales[job] = sb;
        a.x_sums[job] = sum;
    }
    flag_or(a.sticky, flags);
}

// ---------------------------------------------------------------------------
// D2: block (slot s, p) computes gate columns 16p..16p+15 and the matching up
// columns 512+16p.. over all 8 groups.  Thread (n, g): local column n (0..15
// gate, 16..31 up), group g; it loads its 32 code words (stride 32, so each
// half-wave reads two contiguous 64-byte runs) straight into registers.
// Wave 0 finishes the 16 middle values and applies the H128 butterflies on
// k bits 0..3 (the 16 values of a block are one run of k), so the consumer
// only does k bits 4..6; the order of the butterflies is unchanged.
template <bool ROUTER, bool SHARED>
__global__ __launch_bounds__(256) void decode1_gateup_kernel(DecodeArgs a) {
    __shared__ __align__(16) uint32_t la[8 * 64];
    __shared__ float lsa[8], lss[8];
    __shared__ float lterm[8][32];
    __shared__ __align__(16) uint64_t s_cand[65];
    __shared__ uint2 s_sel[kTop];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // (slot, column pair) from the XCD-paired block index: 32 blocks per slot
    const int bi = xcd_paired_block(int(blockIdx.x)), s = bi >> 5, p = bi & 31;
    const bool shared = SHARED && s == kTop;
    // activations of the token: no dependency, issue first
    const uint32_t a0 = a.x_words[tid], a1 = a.x_words[256 + tid];
    const uint32_t sbits = a.x_scales[tid & 7];
    const int sum = a.x_sums[tid & 7];
    int bank = kShared;
    if (!shared) {
        if (ROUTER) {
            if (wave == 0) {
                float v[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = a.logits[lane + 64 * i];
                uint32_t k[4];
                softmax_keys(v, k);
                top8_rank_lds(k, s_cand, s_sel);
                if (s == 0 && p == 0) {
                    // slot weights renormalised by the slot-order sum of the picks
                    float tot = 0.f;
#pragma unroll
                    for (int j = 0; j < kTop; ++j) tot = tot + __uint_as_float(s_sel[j].x);
                    if (lane < kTop) {
                        const uint2 pick = s_sel[lane];
                        a.topk_w[lane] = fdiv_rn(__uint_as_float(pick.x), tot);
                        a.topk_ids[lane] = int(pick.y);
                    }
                    if (SHARED && lane == 0) a.shared_logit[0] = f32_to_bf16_bits(a.logits[kExperts]);
                }
            }
            __syncthreads();
            bank = int(s_sel[s].y);
        } else {
            bank = a.ids_in[s];
            if (bank < 0 || bank >= kExperts) {
                if (bank != -1 && p == 0 && tid == 0) atomicOr(a.sticky, kFlagInvalidExpert);
                return;
            }
        }
    }
    const uint32_t* codes = shared ? a.s13_codes : a.w13_codes + size_t(bank) * kGateBankWords;
    const uint32_t* meta = shared ? a.s13_meta : a.w13_meta + size_t(bank) * kGateBankMeta;
    const int n = lane & 31, g = 2 * wave + (lane >> 5);
    const int col = n < 16 ? 16 * p + n : kInter + 16 * p + (n - 16);
    const BankView bv = bank_view(shared);
    const uint32_t* wp = codes + bv.word(col, g, 8);
    uint32_t wr[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) wr[j] = load_once(wp + j * bv.stride());
    const uint32_t mw = meta[bv.meta(col, g, 8)];
    la[tid] = a0;
    la[tid + 256] = a1;
    if (tid < 8) {
        const float sc = f16_bits_to_f32(uint16_t(sbits));
        lsa[tid] = sc;
        lss[tid] = sc * float(sum);
    }
    __syncthreads();
    const uint4* ab = reinterpret_cast<const uint4*>(&la[g * 64]);
    int dot = 0;
#pragma unroll
    for (int c4 = 0; c4 < 16; ++c4) {
        const uint4 av = ab[c4];
        dot = dot4(code_even(wr[2 * c4]), int(av.x), dot);
        dot = dot4(code_odd(wr[2 * c4]), int(av.y), dot);
        dot = dot4(code_even(wr[2 * c4 + 1]), int(av.z), dot);
        dot = dot4(code_odd(wr[2 * c4 + 1]), int(av.w), dot);
    }
    lterm[g][n] = tree_term(dot, lsa[g], lss[g], mw);
    __syncthreads();
    if (wave == 0) {
        // lanes 16..63 repeat lanes 0..15 so the butterflies see a full row
        const int c = lane & 15;
        uint32_t flags = 0;
        float vg = 0.f, vu = 0.f;
#pragma unroll
        for (int gg = 0; gg < 8; ++gg) vg = vg + lterm[gg][c];
#pragma unroll
        for (int gg = 0; gg < 8; ++gg) vu = vu + lterm[gg][16 + c];
        float mid;
        if (shared) {
            vg = bf16_round(vg);
            vu = bf16_round(vu);
            if (!isfinite(vg) || !isfinite(vu)) flags |= kFlagNonfiniteProjection;
            mid = bf16_round(a.silu_table[__float_as_uint(vg) >> 16] * vu);
        } else {
            if (!isfinite(vg) || !isfinite(vu)) flags |= kFlagNonfiniteProjection;
            mid = silu_portable_wave(vg) * vu;
        }
        if (!isfinite(mid)) flags |= kFlagNonfiniteMiddle | kFlagNonfiniteInput;
        // the first four H128 butterflies of the down input (k bits 0..3 =
        // column bits 0..3 = lane bits 0..3), in ascending order
        mid = butterfly_lane<1>(mid);
        mid = butterfly_lane<2>(mid);
        mid = butterfly_lane<4>(mid);
        mid = butterfly_lane<8>(mid);
        if (lane < 16) {
            a.middle[size_t(s) * kInter + p * 16 + lane] = mid;
            flag_or(a.sticky, flags);
        }
    }
}

// ---------------------------------------------------------------------------
// D3: block = 16 output columns over all slots (9 waves).  Wave w quantises
// slot w's middle row (H128 butterflies on k bits 4..6 + A8/A4 of both
// groups, strided half-wave layout: lane values 16 apart in k, so the
// butterflies are in-register and each q is stored as a byte) while every
// thread's down-code loads are in flight.  Thread: (slot i, group g) =
// tid / 64 and lane / 32, chunk half h = (lane / 16) & 1, column n = lane & 15,
// 16 code words in registers; the two halves' integer dots are added exactly,
// the two groups' terms meet through xor 32, and the slots are reduced in
// slot order (routed_storage_n32_consumer.cpp:176-184, 296-307).
template <bool SHARED, int QMAX>
__global__ __launch_bounds__(576) void decode1_down_kernel(DecodeArgs a) {
    __shared__ __align__(16) uint32_t la[kSlots * 2 * 64];
    __shared__ float lsa[kSlots * 2], lss[kSlots * 2];
    __shared__ float lro[kSlots][16];
    __shared__ int lbank[kSlots];
    __shared__ float lw8[kTop];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, c = xcd_paired_block(int(blockIdx.x));
    const int nslots = SHARED ? kSlots : kTop;
    // Every load below is unconditional (unused lanes read a valid address and
    // drop the value), so the in-order load counter stays exact and each wait
    // leaves the younger loads in flight.
    // Load order = wait order: routing first, then the middle row of slot
    // `wave` (lanes 0-31 group 0, 32-63 group 1), then the shared logit.
    const int id_in = a.reduce_ids[tid & 7];
    const float w_in = a.reduce_w[tid & 7];
    __builtin_amdgcn_sched_barrier(0);                 // keep the routing loads oldest
    const int lp = lane & 31, gm = lane >> 5, kb = strided_base(lp);
    const float* mrow = a.middle + size_t(wave < nslots ? wave : nslots - 1) * kInter + gm * kGroup + kb;
    float mv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) mv[j] = mrow[16 * j];
    const uint16_t shared_logit = SHARED ? a.shared_logit[0] : 0;
    if (tid < kTop) {
        lbank[tid] = (id_in >= 0 && id_in < kExperts) ? id_in : -1;
        lw8[tid] = w_in;
    }
    if (tid == kTop) lbank[kTop] = SHARED ? kShared : -1;
    __syncthreads();
    // ---- down codes of (slot i, group g, column n, chunks 16h..16h+15) ----
    const int i = wave, g = gm, h = (lane >> 4) & 1, n = lane & 15;
    const int bank = i < nslots ? lbank[i] : -1;
    const int col = 16 * c + n;
    const int lb = bank >= 0 ? bank : 0;
    const uint32_t* base = lb == kShared ? a.s2_codes : a.w2_codes + size_t(lb) * kDownBankWords;
    const uint32_t* mbase = lb == kShared ? a.s2_meta : a.w2_meta + size_t(lb) * kDownBankMeta;
    const BankView bv = bank_view(lb == kShared);
    const uint32_t* wp = base + bv.word(col, g, 2) + 16 * h * bv.stride();
    uint32_t wr[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) wr[j] = load_once(wp + j * bv.stride());
    const uint32_t mw = mbase[bv.meta(col, g, 2)];
    // shared-expert gate: its table load goes out behind the codes, used at the end
    const uint16_t gate_bits = SHARED ? a.sigmoid_table[shared_logit] : 0;
    // ---- middle quantisation, one slot per wave ----
    uint32_t flags = 0;
    if (bank >= 0) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = mv[j];
        h128_tail_strided(v);
        int qv[8];
        uint16_t sb;
        int sum;
        quantize_strided<QMAX>(v, qv, sb, sum, flags, kFlagNonfiniteInput | kFlagInvalidActivation,
                               kFlagInvalidActivation);
        // value j (k = kb + 16 j) is byte (k & 7) >> 1 of word 2 (k >> 3) + (k & 1)
        uint8_t* lb = reinterpret_cast<uint8_t*>(&la[(2 * i + gm) * 64]);
#pragma unroll
        for (int j = 0; j < 8; ++j)
            lb[4 * (2 * ((kb >> 3) + 2 * j) + (kb & 1)) + ((kb & 7) >> 1)] = uint8_t(qv[j]);
        if (lp == 0) {
            const float sc = f16_bits_to_f32(sb);
            lsa[2 * i + gm] = sc;
            lss[2 * i + gm] = sc * float(sum);
        }
    }
    __syncthreads();
    // ---- dots and the two-group tree ----
    float term = 0.f;
    if (bank >= 0) {
        const uint4* ab = reinterpret_cast<const uint4*>(&la[(2 * i + g) * 64 + 32 * h]);
        int dot = 0;
#pragma unroll
        for (int c4 = 0; c4 < 8; ++c4) {
            const uint4 av = ab[c4];
            dot = dot4(code_even(wr[2 * c4]), int(av.x), dot);
            dot = dot4(code_odd(wr[2 * c4]), int(av.y), dot);
            dot = dot4(code_even(wr[2 * c4 + 1]), int(av.z), dot);
            dot = dot4(code_odd(wr[2 * c4 + 1]), int(av.w), dot);
        }
        dot += xor_perm_i<16>(dot);
        term = tree_term(dot, lsa[2 * i + g], lss[2 * i + g], mw);
    }
    const float term1 = xor_perm_f<32>(term);          // group 1 of the same (slot, column)
    if (bank >= 0 && lane < 16) {
        float v = 0.f;
        v = v + term;
        v = v + term1;
        if (i == kTop) v = bf16_round(v);
        if (!isfinite(v)) flags |= kFlagNonfiniteProjection;
        lro[i][n] = v;
    }
    __syncthreads();
    if (tid < 16) {
        const int col = c * 16 + tid;
        // every LDS read first, then the slot-order sum over live slots
        int lb8[kTop];
        float ro[kTop], w8[kTop];
#pragma unroll
        for (int sl = 0; sl < kTop; ++sl) {
            lb8[sl] = lbank[sl];
            ro[sl] = lro[sl][tid];
            w8[sl] = lw8[sl];
        }
        float sum = 0.f;
#pragma unroll
        for (int sl = 0; sl < kTop; ++sl) {
            const float t = sum + ro[sl] * w8[sl];
            sum = lb8[sl] >= 0 ? t : sum;
        }
        const uint16_t o = f32_to_bf16_bits(sum);
        if (!isfinite(sum) || (o & 0x7f80u) == 0x7f80u) flags |= kFlagNonfiniteOutput;
        if (a.final_f32) a.final_f32[col] = sum;
        if (a.out) a.out[col] = o;
        if (SHARED) {
            const float gate = bf16_bits_to_f32(gate_bits);
            const float sv = lro[kTop][tid] * gate;
            if (!isfinite(sv)) flags |= kFlagNonfiniteOutput;
            const uint16_t so = f32_to_bf16_bits(sv);
            if (a.shared_out) a.shared_out[col] = so;
            if (a.layer_out) a.layer_out[col] = f32_to_bf16_bits(bf16_bits_to_f32(o) + bf16_bits_to_f32(so));
        }
    }
    flag_or(a.sticky, flags);
}

// ---------------------------------------------------------------------------
// The whole single-token layer in one launch: 256 blocks of 9 waves, all
// resident at once (the launcher checks the occupancy; otherwise the three
// kernels above run).  Values that cross blocks -- the 257 router logits and
// the nine middle rows -- travel as 64-bit words (tag << 32 | value bits),
// each written and read with one agent-scope atomic access.  The tag hashes
// the call's sequence number with the word's index, so a reader knows a word
// belongs to this call once its tag matches: no fence, counter or kernel
// boundary sits between producer and consumer, and a stale word (an earlier
// call, another workspace) does not match.  Every wait is bounded; a block
// that gives up raises kFlagHandoffTimeout and finishes on what it has.
//
// Block L (linear launch index; XCDs take blocks round-robin):
//   wave 8    router row L (block 0 also the shared gate row), published as
//             a tagged logit as soon as it is formed;
//   waves 4-7 H128 + A8 quantisation of x into LDS (every block its own);
//             then wave 4 waits for the 257 logits and selects the experts;
//   waves 0-3 gate-up: 16 gate + 16 up columns of routed slot s (XCD-paired
//             as decode1_gateup_kernel); blocks of slot 0 also do the same
//             columns of the shared expert, whose codes load at once; waves
//             0 and 1 publish the 16 middle values of the routed and shared
//             unit;
//   blocks L < 128 then finish 16 output columns as decode1_down_kernel:
//             wave i's down codes of slot i load as soon as the experts are
//             known (behind the gate-up codes on waves 0-3), so a wave's
//             loads have landed before it waits for slot i's middle row (a
//             wave's loads complete in order: a wait for a hand-off word
//             queued behind a weight load would wait for the weights);
//             then the H128 tail and A8 of the middle row, the dots, the
//             tree and the slot-order sum.
// Every wave reads the sequence number at its start and has it before the
// block's first barrier, after which the block publishes an arrival word;
// block 0 advances the number once every block has arrived.  The arithmetic
// is that of the three kernels above, operation for operation.
namespace {
// Waits until an LDS counter of this block reaches n (bounded; the waves
// that count it are this block's own and wait for nothing else).
__device__ __forceinline__ void lds_wait(uint32_t* counter, uint32_t n) {
    for (int spin = 0; spin < (1 << 22); ++spin) {
        if (__hip_atomic_load(counter, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) >= n) return;
        __builtin_amdgcn_s_sleep(1);
    }
}
constexpr int kLayer1DownBlocks = kHidden / 16;
// Waves of a block: 0-3 gate-up (wave 1 also its epilogue), 4 routing, 4-7 x
// quantisation, 8 router row, 4-12 the down slots 0-8 (slot = wave - 4).  The
// gate-up waves load nothing for the down part, so each down wave's poll for
// its middle row queues behind its own down codes only, issued right after
// the experts are known.
constexpr int kLayer1Waves = 13, kLayer1DownWave0 = 4;
// The routed gate-up epilogue runs on wave 1: the shared slot's down wave (12)
// works at the same time and waves are dealt to the four SIMDs in turn
// (wave w on SIMD w % 4), so the two do not share a SIMD.
constexpr int kLayer1EpilogueWave = 1;
}  // namespace

// Stage trace (measurement builds only, -DORNITH_STAGE_TRACE): lane 0 of the
// named wave stores the steady clock (100 MHz) when a block reaches a stage,
// into slot (call sequence number % kStageCalls) of g_layer1_stages, so the
// calls of a captured graph land in distinct slots.  Ordinary builds compile
// every stage point to nothing.
#ifdef ORNITH_STAGE_TRACE
__device__ uint64_t g_layer1_stages[kStageCalls * kLayer1Blocks * kStageSlots];
#define L1_STAGE_AT(i, t)                                                                             \
    do {                                                                                              \
        if ((threadIdx.x & 63) == 0)                                                                  \
            g_layer1_stages[(size_t(seq % kStageCalls) * kLayer1Blocks + blockIdx.x) * kStageSlots + (i)] = \
                (t) | (uint64_t(seq & 0xFFFu) << 52);                                                 \
    } while (0)
#define L1_STAGE(i) L1_STAGE_AT(i, uint64_t(wall_clock64()))
#else
#define L1_STAGE_AT(i, t) do {} while (0)
#define L1_STAGE(i) do {} while (0)
#endif

template <bool ROUTER, bool SHARED, int QMAX>
__global__ __launch_bounds__(64 * kLayer1Waves) void layer1_kernel(DecodeArgs a) {
    __shared__ __align__(16) uint32_t lx[8 * 64];               // A8 words of x
    __shared__ float lxa[8], lxs[8];                            // group scale, scale * sum
    __shared__ float lterm[2][8][32];                           // gate-up terms: shared unit, routed unit
    __shared__ __align__(16) uint64_t s_cand[65];
    __shared__ uint2 s_sel[kTop], s_spec[kTop];
    __shared__ int lbank[kSlots], lspec[kTop];
    __shared__ float lw8[kTop];
    __shared__ __align__(16) uint32_t lm[kSlots * 2 * 64];      // A8 words of the middle rows
    __shared__ float lma[kSlots * 2], lms[kSlots * 2];
    __shared__ float lro[kSlots][16];
    __shared__ uint32_t lseq[kLayer1Waves];
    __shared__ uint32_t lgate;                                  // bf16 sigmoid gate of the shared expert
    // waves done: x quantisation (4), shared-unit dots (4); speculative picks
    // published (1); routed gate-up dots (4)
    __shared__ uint32_t lsync[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, L = int(blockIdx.x);
    uint64_t* W = a.l1_words;
    // the call's sequence number: its load is issued first and its value is
    // used only after the independent loads below are issued (a wave's loads
    // complete in order, so the first use waits for nothing issued later)
    uint32_t seq_v = __hip_atomic_load(a.l1_seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#ifdef ORNITH_STAGE_TRACE
    const uint64_t t_start = uint64_t(wall_clock64());
#endif
    const int gu = xcd_paired_block(L), s = gu >> 5, p = gu & 31;   // routed gate-up unit (slot s, pair p)
    const bool down_block = L < kLayer1DownBlocks;
    const int c = xcd_paired_block(L & (kLayer1DownBlocks - 1));   // down columns 16c..16c+15
    const bool shared_unit = SHARED && s == 0;
    uint32_t flags = 0;
    // gate-up thread (n, g): column n of the pair (0..15 gate, 16..31 up), group g
    const int n = lane & 31, g = 2 * (wave & 3) + (lane >> 5);
    const int gcol = n < 16 ? 16 * p + n : kInter + 16 * p + (n - 16);
    // down thread (decode1_down_kernel's): slot = wave, group dg, chunk half dh, column dn
    const int lp = lane & 31;
    const int dg = lane >> 5, dh = (lane >> 4) & 1, dn = lane & 15, dcol = 16 * c + dn;

    // ---- loads with no dependency: router row(s), shared-unit codes, x ----
    uint4 rv[4], rv2[4], xv[4];
    if (ROUTER && wave == 8) {
        const uint16_t* wrow = a.router_w + size_t(L) * kHidden;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            rv[i] = load_once4(wrow + (i * 64 + lane) * 8);
            xv[i] = *reinterpret_cast<const uint4*>(a.x + (i * 64 + lane) * 8);
        }
        if (SHARED && L == 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i) rv2[i] = load_once4(a.shared_gate_w + (i * 64 + lane) * 8);
        }
    }
    uint32_t ws[32], wd[16], mws = 0, mwd = 0;
    const int job = 2 * (wave - 4) + (lane >> 5);
    uint4 raw{};
    if (wave >= 4 && wave < 8) raw = *reinterpret_cast<const uint4*>(a.x + job * kGroup + lp * 8);
    if (tid == 0) {
        lsync[0] = 0;
        lsync[1] = 0;
        lsync[2] = 0;
        lsync[3] = 0;
    }
    __syncthreads();
    // The sequence number is taken only here, where every wave needs the
    // loads it issued above anyway (without the asm the compiler converts it
    // to a scalar right after its load and waits for it before issuing them).
    // Each wave has it before barrier A, so before the block's arrival word.
    asm volatile("" : "+v"(seq_v));
    const uint32_t seq = __builtin_amdgcn_readfirstlane(seq_v);
    const int limit = l1_limit(seq, a.handoff_spins);
    if (lane == 0) lseq[wave] = seq;
    if (wave == 0) L1_STAGE_AT(0, t_start);                      // block started
    // shared-unit codes (slot-0 blocks), issued after the router rows so the
    // two do not share the first HBM burst; the shared middle row has slack
    if (shared_unit && wave < 4) {
        const BankView bv = bank_view(true);
        const uint32_t* wp = a.s13_codes + bv.word(gcol, g, 8);
#pragma unroll
        for (int j = 0; j < 32; ++j) ws[j] = load_once(wp + j * bv.stride());
        mws = a.s13_meta[bv.meta(gcol, g, 8)];
    }
    // ---- router row(s) in the declared order of decode1_route_kernel, published at once ----
    if (ROUTER && wave == 8) {
        auto row = [&](const uint4 (&wv)[4]) {
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
            return wave_butterfly_sum(acc);
        };
        float v = row(rv);
        if (a.bias) v = v + a.bias[L];
        if (lane == 0) l1_put(W, kLayer1Spread * L, seq, __float_as_uint(v));
        L1_STAGE(1);                                                  // router row published
        if (SHARED && L == 0) {
            const float v2 = row(rv2);
            if (lane == 0) l1_put(W, kLayer1Spread * kExperts, seq, __float_as_uint(v2));
        }
    }
    int id_in = -1;
    float w_in = 0.f;
    if (!ROUTER && wave == 4) {
        id_in = a.ids_in[lane & 7];
        w_in = a.reduce_w[lane & 7];
    }
    // gate-up dots of one unit from codes in registers, into lterm[u]
    auto gate_dots = [&](const uint32_t (&wr)[32], uint32_t mw, int u) {
        const uint4* ab = reinterpret_cast<const uint4*>(&lx[g * 64]);
        int dot = 0;
#pragma unroll
        for (int c4 = 0; c4 < 16; ++c4) {
            const uint4 av = ab[c4];
            dot = dot4(code_even(wr[2 * c4]), int(av.x), dot);
            dot = dot4(code_odd(wr[2 * c4]), int(av.y), dot);
            dot = dot4(code_even(wr[2 * c4 + 1]), int(av.z), dot);
            dot = dot4(code_odd(wr[2 * c4 + 1]), int(av.w), dot);
        }
        lterm[u][g][n] = tree_term(dot, lxa[g], lxs[g], mw);
    };
    // gate-up epilogue of one unit on one wave (decode1_gateup_kernel's wave
    // 0), then the 16 middle values are published
    auto gate_epilogue = [&](int u, int slot, bool table) {
        // lane c < 32 sums column c over the groups in ascending order (gate
        // columns 0..15, up 16..31); lane l < 16 takes up from lane l + 16
        float v = 0.f;
#pragma unroll
        for (int gg = 0; gg < 8; ++gg) v = v + lterm[u][gg][lane & 31];
        float vg = v, vu = xor_perm_f<16>(v);
        float mid;
        uint32_t f = 0;
        if (table) {
            vg = bf16_round(vg);
            vu = bf16_round(vu);
            if (!isfinite(vg) || !isfinite(vu)) f |= kFlagNonfiniteProjection;
            mid = bf16_round(a.silu_table[__float_as_uint(vg) >> 16] * vu);
        } else {
            if (!isfinite(vg) || !isfinite(vu)) f |= kFlagNonfiniteProjection;
            mid = silu_portable_wave(vg) * vu;
        }
        if (!isfinite(mid)) f |= kFlagNonfiniteMiddle | kFlagNonfiniteInput;
        mid = butterfly_lane<1>(mid);
        mid = butterfly_lane<2>(mid);
        mid = butterfly_lane<4>(mid);
        mid = butterfly_lane<8>(mid);
        if (lane < 16) {
            l1_put(W, kLayer1Middle + slot * kInter + p * 16 + lane, seq, __float_as_uint(mid));
            flags |= f;
        }
    };
    // ---- quantised gate input (decode1_route_kernel's second part) ----
    if (wave >= 4 && wave < 8) {
        bool live = true;
        if (!ROUTER && !SHARED) {
            live = false;
#pragma unroll
            for (int j = 0; j < kTop; ++j) {
                const int id = a.ids_in[j];
                live |= id >= 0 && id < kExperts;
            }
        }
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
        // only block 0 reports the input's flags (every block sees the same x)
        if (L != 0) flags = 0;
        lx[job * 64 + 2 * lp] = w2[0];
        lx[job * 64 + 2 * lp + 1] = w2[1];
        if (lp == 0) {
            const float sc = f16_bits_to_f32(sb);
            lxa[job] = sc;
            lxs[job] = sc * float(sum);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        if (lane == 0) __hip_atomic_fetch_add(&lsync[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    // ---- shared unit (blocks of slot 0) as soon as x is quantised: its
    // middle row leaves long before the routed ones ----
    if (shared_unit && wave < 4) {
        lds_wait(&lsync[0], 4u);
        gate_dots(ws, mws, 0);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        if (lane == 0) __hip_atomic_fetch_add(&lsync[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (wave == 1) {
            lds_wait(&lsync[1], 4u);
            gate_epilogue(0, kTop, true);
            L1_STAGE(11);                                             // shared middle published
        }
    }
    // ---- routing on wave 4 ----
    if (wave == 4) {
        if (ROUTER) {
            // the 256 expert logits (the shared gate logit is read later, by
            // the shared slot's down wave)
            uint32_t idx[4], got[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) idx[i] = uint32_t(kLayer1Spread * (lane + 64 * i));
            if (!l1_wait<4, 0>(W, idx, seq, got, limit)) flags |= kFlagHandoffTimeout;
            L1_STAGE(2);                                              // 256 logits seen
            float lg[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) lg[i] = __uint_as_float(got[i]);
            // speculative picks: the eight largest logits (ties to the lower
            // id), published at once so waves 0-3 start loading their codes.
            // The softmax is monotone, so these are the exact picks unless
            // rounding makes two probabilities equal; waves 0-3 check them
            // against the exact picks below and reload on a difference.
            uint32_t lk[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) lk[i] = f32_order_key(lg[i] + 0.f);   // -0 -> +0
            top8_rank_lds(lk, s_cand, s_spec);
            if (lane < kTop) lspec[lane] = int(s_spec[lane].y);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            if (lane == 0) __hip_atomic_fetch_add(&lsync[2], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            L1_STAGE(12);                                             // speculative picks published
            uint32_t k[4];
            softmax_keys(lg, k);
            top8_rank_lds(k, s_cand, s_sel);
            float tot = 0.f;
#pragma unroll
            for (int j = 0; j < kTop; ++j) tot = tot + __uint_as_float(s_sel[j].x);
            if (lane < kTop) {
                const uint2 pick = s_sel[lane];
                const float wgt = fdiv_rn(__uint_as_float(pick.x), tot);
                lbank[lane] = int(pick.y);
                lw8[lane] = wgt;
                if (L == 0) {
                    a.topk_w[lane] = wgt;
                    a.topk_ids[lane] = int(pick.y);
                }
            }
        } else {
            if (lane < kTop) {
                lbank[lane] = (id_in >= 0 && id_in < kExperts) ? id_in : -1;
                lw8[lane] = w_in;
            }
        }
        if (lane == kTop) lbank[kTop] = SHARED ? kShared : -1;
        L1_STAGE(3);                                                  // experts selected
    }
    // ---- the shared slot's down wave, idle until here: the shared expert's
    // bf16 sigmoid gate (used by the last step only) from the gate logit
    // (block 0's second row) and the table, then the shared down codes, which
    // need no routing, so the shared slot's down work runs as soon as its
    // middle row (formed before the routing) arrives ----
    uint32_t gate_bits = 0;
    if (SHARED && down_block && wave == kLayer1DownWave0 + kTop) {
        uint32_t sl;
        if (ROUTER) {
            uint32_t idx1[1] = {uint32_t(kLayer1Spread * kExperts)}, got1[1];
            if (!l1_wait<1, 1>(W, idx1, seq, got1, limit)) flags |= kFlagHandoffTimeout;
            sl = f32_to_bf16_bits(__uint_as_float(got1[0]));
            if (L == 0 && lane == 0) a.shared_logit[0] = uint16_t(sl);
            L1_STAGE(13);                                             // shared gate logit seen
        } else {
            sl = a.shared_logit[0];
        }
        gate_bits = a.sigmoid_table[sl];
        const BankView bv = bank_view(true);
        const uint32_t* wp = a.s2_codes + bv.word(dcol, dg, 2) + 16 * dh * bv.stride();
#pragma unroll
        for (int j = 0; j < 16; ++j) wd[j] = load_once(wp + j * bv.stride());
        mwd = a.s2_meta[bv.meta(dcol, dg, 2)];
    }
    // ---- routed gate-up codes (waves 0-3), loaded from the speculative pick
    // of slot s as soon as it is published (the caller's id without the
    // router); the exact pick is checked after the barrier ----
    uint32_t wr[32], mw = 0;
    int sbank = -1;
    auto load_gate = [&](int b) {
        const BankView bv = bank_view(false);
        const uint32_t* wp = a.w13_codes + size_t(b) * kGateBankWords + bv.word(gcol, g, 8);
#pragma unroll
        for (int j = 0; j < 32; ++j) wr[j] = load_once(wp + j * bv.stride());
        mw = a.w13_meta[size_t(b) * kGateBankMeta + bv.meta(gcol, g, 8)];
    };
    if (wave < 4) {
        if (ROUTER) {
            lds_wait(&lsync[2], 1u);
            sbank = lspec[s];
        } else {
            const int id = a.ids_in[s];
            sbank = id >= 0 && id < kExperts ? id : -1;
        }
        load_gate(sbank >= 0 ? sbank : 0);
    }
    __syncthreads();
    if (tid == 0) l1_put(W, kLayer1Arrive + kLayer1Spread * L, seq, lseq[0]);

    // the down codes of slot `dslot`
    const int dslot = wave - kLayer1DownWave0;
    const int dbank = down_block && dslot >= 0 && dslot < kSlots ? lbank[dslot] : -1;
    auto load_down = [&]() {
        const int lb = dbank >= 0 ? dbank : 0;
        const bool sh = lb == kShared;
        const BankView bv = bank_view(sh);
        const uint32_t* wp = (sh ? a.s2_codes : a.w2_codes + size_t(lb) * kDownBankWords) + bv.word(dcol, dg, 2) +
                             16 * dh * bv.stride();
#pragma unroll
        for (int j = 0; j < 16; ++j) wd[j] = load_once(wp + j * bv.stride());
        mwd = (sh ? a.s2_meta : a.w2_meta + size_t(lb) * kDownBankMeta)[bv.meta(dcol, dg, 2)];
    };

    // ---- routed gate-up dots (waves 0-3) ----
    int bank = -1;
    if (wave < 4) {
        bank = lbank[s];
        if (!ROUTER && bank < 0) {
            const int id = a.ids_in[s];
            if (id != -1 && p == 0 && tid == 0) flags |= kFlagInvalidExpert;
        }
        // the exact pick differs from the speculative one only when two
        // softmax values tie after rounding: load the right codes
        if (bank != sbank) load_gate(bank >= 0 ? bank : 0);
        // the routed dots always run (an empty slot's are not used), so no
        // load is left pending past this branch
        gate_dots(wr, mw, 1);
        if (wave == 0) L1_STAGE(4);                                   // routed gate-up dots done
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        if (lane == 0) __hip_atomic_fetch_add(&lsync[3], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    // routed down codes: issued as soon as the experts are known (barrier A),
    // behind the block's gate-up codes.  With both streams non-temporal this
    // measured 11.88 -> 11.76 us per layer in graph replays against issuing
    // them after the block's gate-up dots (without the hint the early issue
    // had slowed the gate-up codes); issued after the epilogue they land
    // after the middle rows.  The shared slot's wave loaded its codes before
    // barrier A.
    if (down_block && dslot >= 0 && dslot < kTop) load_down();
    uint64_t arrival[4] = {0, 0, 0, 0};
    if (wave == kLayer1EpilogueWave) {
        lds_wait(&lsync[3], 4u);
        L1_STAGE(14);                                                 // gate-up dots of all four waves done
        if (bank >= 0) {
            gate_epilogue(1, s, false);
            L1_STAGE(5);                                              // routed middle published
        }
    }
    if (L == 0 && wave == 0) {
        // every block published its arrival after barrier A: read the words
        // now, check them at the end
#pragma unroll
        for (int i = 0; i < 4; ++i) arrival[i] = l1_get(W, uint32_t(kLayer1Arrive + kLayer1Spread * (lane + 64 * i)));
    }
    if (!down_block) {
        flag_or(a.sticky, flags);
        return;
    }

    // ---- middle row of slot `dslot`: wait, H128 tail, A8 (decode1_down_kernel) ----
    const int gm = lane >> 5, kb = strided_base(lp);
    if (dbank >= 0) {
        uint32_t idx[8], val[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) idx[j] = uint32_t(kLayer1Middle + dslot * kInter + gm * kGroup + kb + 16 * j);
        if (!l1_wait<8, 1>(W, idx, seq, val, limit)) flags |= kFlagHandoffTimeout;
        if (dslot == 0) L1_STAGE(6);                                  // middle of slot 0 seen
        if (dslot == 7) L1_STAGE(7);                                  // middle of slot 7 seen
        if (dslot == 8) L1_STAGE(8);                                  // shared middle seen
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = __uint_as_float(val[j]);
        h128_tail_strided(v);
        int qv[8];
        uint16_t sb;
        int sum;
        quantize_strided<QMAX>(v, qv, sb, sum, flags, kFlagNonfiniteInput | kFlagInvalidActivation,
                               kFlagInvalidActivation);
        uint8_t* lb = reinterpret_cast<uint8_t*>(&lm[(2 * dslot + gm) * 64]);
#pragma unroll
        for (int j = 0; j < 8; ++j)
            lb[4 * (2 * ((kb >> 3) + 2 * j) + (kb & 1)) + ((kb & 7) >> 1)] = uint8_t(qv[j]);
        if (lp == 0) {
            const float sc = f16_bits_to_f32(sb);
            lma[2 * dslot + gm] = sc;
            lms[2 * dslot + gm] = sc * float(sum);
        }
    }
    // the quantised row is this wave's own: no block barrier before its dots
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    // ---- down dots: the two chunk halves joined exactly, then the two-group tree ----
    float term = 0.f;
    if (dbank >= 0) {
        const uint4* ab = reinterpret_cast<const uint4*>(&lm[(2 * dslot + dg) * 64 + 32 * dh]);
        int dot = 0;
#pragma unroll
        for (int c4 = 0; c4 < 8; ++c4) {
            const uint4 av = ab[c4];
            dot = dot4(code_even(wd[2 * c4]), int(av.x), dot);
            dot = dot4(code_odd(wd[2 * c4]), int(av.y), dot);
            dot = dot4(code_even(wd[2 * c4 + 1]), int(av.z), dot);
            dot = dot4(code_odd(wd[2 * c4 + 1]), int(av.w), dot);
        }
        dot += xor_perm_i<16>(dot);
        term = tree_term(dot, lma[2 * dslot + dg], lms[2 * dslot + dg], mwd);
    }
    const float term1 = xor_perm_f<32>(term);
    if (dbank >= 0 && lane < 16) {
        float v = 0.f;
        v = v + term;
        v = v + term1;
        if (dslot == kTop) v = bf16_round(v);
        if (!isfinite(v)) flags |= kFlagNonfiniteProjection;
        lro[dslot][dn] = v;
    }
    if (dslot == 0) L1_STAGE(9);                                      // down dots of slot 0 done
    if (SHARED && dslot == kTop && lane == 0) lgate = gate_bits;
    __syncthreads();
    if (tid < 16) {
        const int col = 16 * c + tid;
        int lb8[kTop];
        float ro[kTop], w8[kTop];
#pragma unroll
        for (int sl = 0; sl < kTop; ++sl) {
            lb8[sl] = lbank[sl];
            ro[sl] = lro[sl][tid];
            w8[sl] = lw8[sl];
        }
        float sum = 0.f;
#pragma unroll
        for (int sl = 0; sl < kTop; ++sl) {
            const float t = sum + ro[sl] * w8[sl];
            sum = lb8[sl] >= 0 ? t : sum;
        }
        const uint16_t o = f32_to_bf16_bits(sum);
        if (!isfinite(sum) || (o & 0x7f80u) == 0x7f80u) flags |= kFlagNonfiniteOutput;
        if (a.final_f32) a.final_f32[col] = sum;
        if (a.out) a.out[col] = o;
        if (SHARED) {
            const float gate = bf16_bits_to_f32(lgate);
            const float sv = lro[kTop][tid] * gate;
            if (!isfinite(sv)) flags |= kFlagNonfiniteOutput;
            const uint16_t so = f32_to_bf16_bits(sv);
            if (a.shared_out) a.shared_out[col] = so;
            if (a.layer_out) a.layer_out[col] = f32_to_bf16_bits(bf16_bits_to_f32(o) + bf16_bits_to_f32(so));
        }
    }
    if (wave == 0) L1_STAGE(10);                                      // output columns stored
    // ---- block 0 advances the sequence number once every block has arrived ----
    if (L == 0 && wave == 0) {
        uint32_t idx[4], val[4];
        bool ok = true;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            idx[i] = uint32_t(kLayer1Arrive + kLayer1Spread * (lane + 64 * i));
            ok = ok && uint32_t(arrival[i] >> 32) == l1_tag(seq, idx[i]);
        }
        // every block has read `seq` once all arrival words carry its tag;
        // otherwise a late block could publish under the next number's tags,
        // so the workspace is marked poisoned instead of advanced
        const bool arrived =
            limit > 0 && (__builtin_amdgcn_ballot_w64(!ok) == 0 || l1_wait<4, 1>(W, idx, seq, val, limit));
        if (!arrived) flags |= kFlagHandoffTimeout;
        if (lane == 0)
            __hip_atomic_store(a.l1_seq, arrived ? l1_next_seq(seq) : kSeqPoisoned, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
    flag_or(a.sticky, flags);
}

template <bool ROUTER, bool SHARED, int QMAX>
static hipError_t run1(const DecodeArgs& a, hipStream_t s) {
    const int rows = ROUTER ? (SHARED ? kExperts + 1 : kExperts) : 0;
    const int waves = rows + kHidden / kGroup / 2;
    timed_launch("route1", decode1_route_kernel<ROUTER, SHARED, QMAX>, dim3(waves), dim3(64), 0, s, a);
    hipError_t st = hipGetLastError();
    if (st != hipSuccess) return st;
    timed_launch("gateup1", decode1_gateup_kernel<ROUTER, SHARED>, dim3((SHARED ? kSlots : kTop) * (kInter / 16)), dim3(256), 0, s, a);
    st = hipGetLastError();
    if (st != hipSuccess) return st;
    timed_launch("down1", decode1_down_kernel<SHARED, QMAX>, dim3(kHidden / 16), dim3(64 * kSlots), 0, s, a);
    return hipGetLastError();
}

// Whether 256 blocks of the one-launch kernel are resident at once on the
// device that runs stream `s` (checked once per device).
template <bool ROUTER, bool SHARED, int QMAX>
static bool layer1_fits(hipStream_t s) {
    constexpr int kMaxDevices = 64;
    static std::atomic<int> state[kMaxDevices];   // 0 unknown, 1 fits, 2 does not
    const int dev = stream_device(s);
    if (dev < 0 || dev >= kMaxDevices) return false;
    int st = state[dev].load(std::memory_order_relaxed);
    if (st == 0) {
        st = resident_blocks(layer1_kernel<ROUTER, SHARED, QMAX>, 64 * kLayer1Waves, dev) >= kLayer1Blocks ? 1 : 2;
        state[dev].store(st, std::memory_order_relaxed);
    }
    return st == 1;
}

std::atomic<int> g_single_token_mode{0};   // 0 automatic, 1 three kernels
std::atomic<int> g_handoff_spins{kHandoffSpins};

template <bool ROUTER, bool SHARED, int QMAX>
static hipError_t run1_any(const DecodeArgs& a, hipStream_t s) {
    const int mode = g_single_token_mode.load(std::memory_order_relaxed);
    if (mode == 1 || !layer1_fits<ROUTER, SHARED, QMAX>(s)) return run1<ROUTER, SHARED, QMAX>(a, s);
    DecodeArgs b = a;
    b.handoff_spins = g_handoff_spins.load(std::memory_order_relaxed);
    timed_launch("layer1", layer1_kernel<ROUTER, SHARED, QMAX>, dim3(kLayer1Blocks), dim3(64 * kLayer1Waves), 0, s,
                 b);
    return hipGetLastError();
}

hipError_t layer1_stage_trace(uint64_t* out, size_t entries, hipStream_t s) {
#ifdef ORNITH_STAGE_TRACE
    const size_t n = size_t(kStageCalls) * kLayer1Blocks * kStageSlots;
    if (!out || entries < n) return hipErrorInvalidValue;
    return hipMemcpyFromSymbolAsync(out, HIP_SYMBOL(g_layer1_stages), n * sizeof(uint64_t), 0,
                                    hipMemcpyDeviceToDevice, s);
#else
    (void)out; (void)entries; (void)s;
    return hipErrorNotSupported;
#endif
}

hipError_t launch_decode1(const DecodeArgs& a, bool router, bool shared, int qmax, hipStream_t s) {
    if (a.T != 1) return hipErrorInvalidValue;
    if (router && shared) return run1_any<true, true, 127>(a, s);
    if (router) return run1_any<true, false, 127>(a, s);
    if (shared) return run1_any<false, true, 127>(a, s);
    if (qmax == 127) return run1_any<false, false, 127>(a, s);
    return run1_any<false, false, 7>(a, s);
}

}  // namespace ornith
