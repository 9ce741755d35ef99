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
    for (int j = 0; j < 32; ++j) wr[j] = wp[j * bv.stride()];
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
            mid = silu_portable(vg) * vu;
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
    for (int j = 0; j < 16; ++j) wr[j] = wp[j * bv.stride()];
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

hipError_t launch_decode1(const DecodeArgs& a, bool router, bool shared, int qmax, hipStream_t s) {
    if (a.T != 1) return hipErrorInvalidValue;
    if (router && shared) return run1<true, true, 127>(a, s);
    if (router) return run1<true, false, 127>(a, s);
    if (shared) return run1<false, true, 127>(a, s);
    if (qmax == 127) return run1<false, false, 127>(a, s);
    return run1<false, false, 7>(a, s);
}

}  // namespace ornith
