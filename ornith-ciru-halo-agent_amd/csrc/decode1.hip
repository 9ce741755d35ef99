// Single-token decode (T == 1): three kernels with one global-load level of
// routing latency each.
//
//   D1 decode1_route_kernel    router logits (257 waves, one row each) and
//                              the quantised gate input (8 more waves).
//   D2 decode1_gateup_kernel   block (slot s, tile pair p): slots 0..7 are
//                              the routed slots, slot 8 the shared expert.
//                              The activation loads (and, for the shared
//                              slot, the weights) start at once; routed
//                              blocks derive their expert with an in-block
//                              softmax/top-8 of the 257 logits.
//   D3 decode1_down_kernel     block = 32-column tile over all slots: H128 +
//                              A8 of the middles, exact dots, fp32 tree and
//                              the slot-order reduction.
//
// One token has no expert reuse, so slots are processed as they come (no
// permutation); a slot repeated by the caller simply loads its weights twice.
// Arithmetic: routed_storage_n32_consumer.cpp:22-307.
#include "kernels.hpp"
#include "timing.hpp"
#include "topk.hpp"
#include "decode.hpp"

namespace ornith {

constexpr int kPad1 = 1056;
constexpr int kSlots = kTop + 1;

// ---------------------------------------------------------------------------
template <bool ROUTER, bool SHARED, int QMAX>
__global__ __launch_bounds__(1024) void decode1_route_kernel(DecodeArgs a) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int gw = blockIdx.x * 16 + wave;
    uint32_t flags = 0;
    const int nrows = ROUTER ? (SHARED ? kExperts + 1 : kExperts) : 0;
    if (gw < nrows) {
        const uint16_t* wrow = gw < kExperts ? a.router_w + size_t(gw) * kHidden : a.shared_gate_w;
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint4 wv = *reinterpret_cast<const uint4*>(wrow + (i * 64 + lane) * 8);
            const uint4 xv = *reinterpret_cast<const uint4*>(a.x + (i * 64 + lane) * 8);
            const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
            const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc = __builtin_fmaf(bf16_bits_to_f32(xw[j] & 0xffffu), bf16_bits_to_f32(ww[j] & 0xffffu), acc);
                acc = __builtin_fmaf(bf16_bits_to_f32(xw[j] >> 16), bf16_bits_to_f32(ww[j] >> 16), acc);
            }
        }
        float v = wave_butterfly_sum(acc);
        if (a.bias && gw < kExperts) v = v + a.bias[gw];
        if (lane == 0) a.logits[gw] = v;
    }
    // quantised gate input on the waves after the router rows
    const int job = gw - (ROUTER ? kExperts + 1 : 0);
    if (job >= 0 && job < kHidden / kGroup) {
        bool live = true;
        if (!ROUTER && !SHARED) {
            live = false;
#pragma unroll
            for (int s = 0; s < kTop; ++s) {
                const int id = a.ids_in[s];
                live |= id >= 0 && id < kExperts;
            }
        }
        const uint2 raw = *reinterpret_cast<const uint2*>(a.x + job * kGroup + lane * 4);
        float v[4] = {bf16_bits_to_f32(raw.x & 0xffffu), bf16_bits_to_f32(raw.x >> 16),
                      bf16_bits_to_f32(raw.y & 0xffffu), bf16_bits_to_f32(raw.y >> 16)};
        if (live) {
#pragma unroll
            for (int i = 0; i < 4; ++i) if (!isfinite(v[i])) flags |= kFlagNonfiniteInput;
            h128_wave(v);
#pragma unroll
            for (int i = 0; i < 4; ++i) if (!isfinite(v[i])) flags |= kFlagNonfiniteInput;
        } else {
            v[0] = v[1] = v[2] = v[3] = 0.f;
        }
        quantize_group_wave<QMAX>(v, a.x_words + job * 64, a.x_scales + job, a.x_sums + job, flags,
                                  kFlagInvalidActivation);
    }
    flag_or(a.sticky, flags);
}

// ---------------------------------------------------------------------------
template <bool ROUTER, bool SHARED>
__global__ __launch_bounds__(256) void decode1_gateup_kernel(DecodeArgs a) {
    __shared__ uint32_t lw[16 * kPad1];
    __shared__ uint32_t lm[16 * 32];
    __shared__ uint32_t la[8 * 64];
    __shared__ float lsa[8], lss[8];
    __shared__ float lterm[16][32];
    __shared__ int s_bank;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int s = blockIdx.x, p = blockIdx.y;
    const bool shared = SHARED && s == kTop;
    // activations of the token: no dependency, issue first
    const uint32_t a0 = a.x_words[tid], a1 = a.x_words[256 + tid];
    float sreg = 0.f, ssum = 0.f;
    if (tid < 8) {
        sreg = f16_bits_to_f32(a.x_scales[tid]);
        ssum = sreg * float(a.x_sums[tid]);
    }
    int bank = kShared;
    if (!shared) {
        if (ROUTER) {
            if (wave == 0) {
                float v[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = a.logits[lane + 64 * i];
                float w8[kTop];
                int i8[kTop];
                softmax_top8(v, w8, i8);
                int mine = i8[0];
#pragma unroll
                for (int j = 1; j < kTop; ++j) if (s == j) mine = i8[j];
                if (lane == 0) s_bank = mine;
                if (s == 0 && p == 0 && lane < kTop) {
                    float wv = w8[0];
                    int iv = i8[0];
#pragma unroll
                    for (int j = 1; j < kTop; ++j) if (lane == j) { wv = w8[j]; iv = i8[j]; }
                    a.topk_w[lane] = wv;
                    a.topk_ids[lane] = iv;
                }
                if (SHARED && s == 0 && p == 0 && lane == 0) a.shared_logit[0] = f32_to_bf16_bits(a.logits[kExperts]);
            }
            __syncthreads();
            bank = s_bank;
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
    uint4 stage[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int h = i >> 3, g = i & 7;
        stage[i] = *reinterpret_cast<const uint4*>(codes + (size_t(p + 16 * h) * 8 + g) * 1024 + tid * 4);
    }
    uint32_t mreg[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int q = tid + 256 * k, blk = q >> 5, n = q & 31, h = blk >> 3, g = blk & 7;
        mreg[k] = meta[(size_t(p + 16 * h) * 8 + g) * 32 + n];
    }
    la[tid] = a0;
    la[tid + 256] = a1;
    if (tid < 8) { lsa[tid] = sreg; lss[tid] = ssum; }
#pragma unroll
    for (int i = 0; i < 16; ++i) *reinterpret_cast<uint4*>(&lw[i * kPad1 + tid * 4]) = stage[i];
    lm[tid] = mreg[0];
    lm[tid + 256] = mreg[1];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int blk = (tid >> 5) + 8 * k, n = tid & 31, g = blk & 7;
        const uint32_t* wb = &lw[blk * kPad1 + n];
        const uint32_t* ab = &la[g * 64];
        int dot = 0;
#pragma unroll 8
        for (int c = 0; c < 32; ++c) {
            const uint32_t w = wb[c * 32];
            dot = dot4(code_even(w), int(ab[2 * c]), dot);
            dot = dot4(code_odd(w), int(ab[2 * c + 1]), dot);
        }
        lterm[blk][n] = tree_term(dot, lsa[g], lss[g], lm[blk * 32 + n]);
    }
    __syncthreads();
    if (tid < 32) {
        uint32_t flags = 0;
        float vg = 0.f, vu = 0.f;
#pragma unroll
        for (int g = 0; g < 8; ++g) vg = vg + lterm[g][tid];
#pragma unroll
        for (int g = 0; g < 8; ++g) vu = vu + lterm[8 + g][tid];
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
        a.middle[size_t(s) * kInter + p * 32 + tid] = mid;
        flag_or(a.sticky, flags);
    }
}

// ---------------------------------------------------------------------------
template <bool SHARED, int QMAX>
__global__ __launch_bounds__(512) void decode1_down_kernel(DecodeArgs a) {
    __shared__ uint32_t lw[kSlots * 2 * kPad1];
    __shared__ uint32_t lm[kSlots * 2 * 32];
    __shared__ uint32_t la[kSlots * 2 * 64];
    __shared__ float lsa[kSlots * 2], lss[kSlots * 2];
    __shared__ float lterm[kSlots * 2][32];
    __shared__ float lro[kSlots][32];
    __shared__ int lbank[kSlots];
    __shared__ float lw8[kTop];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, c = blockIdx.x;
    const int nslots = SHARED ? kSlots : kTop;
    if (tid < kTop) {
        const int id = a.reduce_ids[tid];
        lbank[tid] = (id >= 0 && id < kExperts) ? id : -1;
        lw8[tid] = a.reduce_w[tid];
    }
    if (tid == kTop) lbank[kTop] = SHARED ? kShared : -1;
    __syncthreads();
    // ---- middle rows: job (i, g) = 2i + g on wave job % 8 ----
    uint32_t flags = 0;
    float4 mid[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const int job = wave + 8 * k, i = job >> 1, g = job & 1;
        mid[k] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (i < nslots && lbank[i] >= 0)
            mid[k] = *reinterpret_cast<const float4*>(a.middle + size_t(i) * kInter + g * kGroup + lane * 4);
    }
    // ---- weights: slot i, group g, tile c ----
    uint4 stage[kSlots * 2 / 2];
#pragma unroll
    for (int k = 0; k < kSlots; ++k) {
        // 18 (slot, group) blocks of 256 uint4 over 512 threads: thread half h takes blocks 2k+h
        const int blk = 2 * k + (tid >> 8), i = blk >> 1, g = blk & 1;
        const int bank = lbank[i];
        stage[k] = make_uint4(0, 0, 0, 0);
        if (i < nslots && bank >= 0) {
            const uint32_t* base = bank == kShared ? a.s2_codes : a.w2_codes + size_t(bank) * kDownBankWords;
            stage[k] = *reinterpret_cast<const uint4*>(base + (size_t(c) * 2 + g) * 1024 + (tid & 255) * 4);
        }
    }
    uint32_t mreg[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int q = tid + 512 * k, i = q >> 6, g = (q >> 5) & 1, n = q & 31;
        mreg[k] = 0;
        if (i < nslots && lbank[i] >= 0) {
            const int bank = lbank[i];
            const uint32_t* meta = bank == kShared ? a.s2_meta : a.w2_meta + size_t(bank) * kDownBankMeta;
            mreg[k] = meta[(size_t(c) * 2 + g) * 32 + n];
        }
    }
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const int job = wave + 8 * k, i = job >> 1;
        if (i < nslots && lbank[i] >= 0) {
            float v[4] = {mid[k].x, mid[k].y, mid[k].z, mid[k].w};
            h128_wave(v);
#pragma unroll
            for (int e = 0; e < 4; ++e) if (!isfinite(v[e])) flags |= kFlagNonfiniteInput;
            uint16_t sb;
            int32_t sum;
            quantize_group_wave<QMAX>(v, &la[job * 64], &sb, &sum, flags, kFlagInvalidActivation);
            if (lane == 0) {
                const float sc = f16_bits_to_f32(sb);
                lsa[job] = sc;
                lss[job] = sc * float(sum);
            }
        }
    }
#pragma unroll
    for (int k = 0; k < kSlots; ++k) {
        const int blk = 2 * k + (tid >> 8);
        *reinterpret_cast<uint4*>(&lw[blk * kPad1 + (tid & 255) * 4]) = stage[k];
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) if (tid + 512 * k < kSlots * 64) lm[tid + 512 * k] = mreg[k];
    __syncthreads();
    // ---- dots: term (i, g, n) ----
    for (int q = tid; q < nslots * 64; q += 512) {
        const int blk = q >> 5, n = q & 31;
        if (lbank[blk >> 1] < 0) continue;
        const uint32_t* wb = &lw[blk * kPad1 + n];
        const uint32_t* ab = &la[blk * 64];
        int dot = 0;
#pragma unroll 8
        for (int cc = 0; cc < 32; ++cc) {
            const uint32_t w = wb[cc * 32];
            dot = dot4(code_even(w), int(ab[2 * cc]), dot);
            dot = dot4(code_odd(w), int(ab[2 * cc + 1]), dot);
        }
        lterm[blk][n] = tree_term(dot, lsa[blk], lss[blk], lm[blk * 32 + n]);
    }
    __syncthreads();
    if (tid < nslots * 32) {
        const int i = tid >> 5, n = tid & 31;
        if (lbank[i] >= 0) {
            float v = 0.f;
            v = v + lterm[2 * i][n];
            v = v + lterm[2 * i + 1][n];
            if (i == kTop) v = bf16_round(v);
            if (!isfinite(v)) flags |= kFlagNonfiniteProjection;
            lro[i][n] = v;
        }
    }
    __syncthreads();
    // ---- slot-order reduction (routed_storage_n32_consumer.cpp:176-184, 296-307) ----
    if (tid < 32) {
        const int col = c * 32 + tid;
        float sum = 0.f;
#pragma unroll
        for (int s = 0; s < kTop; ++s)
            if (lbank[s] >= 0) sum = sum + lro[s][tid] * lw8[s];
        const uint16_t o = f32_to_bf16_bits(sum);
        if (!isfinite(sum) || (o & 0x7f80u) == 0x7f80u) flags |= kFlagNonfiniteOutput;
        if (a.final_f32) a.final_f32[col] = sum;
        if (a.out) a.out[col] = o;
        if (SHARED) {
            const float gate = bf16_bits_to_f32(a.sigmoid_table[a.shared_logit[0]]);
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
    const int waves = rows + kHidden / kGroup;
    timed_launch("route1", decode1_route_kernel<ROUTER, SHARED, QMAX>, dim3((waves + 15) / 16), dim3(1024), 0, s, a);
    hipError_t st = hipGetLastError();
    if (st != hipSuccess) return st;
    timed_launch("gateup1", decode1_gateup_kernel<ROUTER, SHARED>, dim3(SHARED ? kSlots : kTop, 16), dim3(256), 0, s, a);
    st = hipGetLastError();
    if (st != hipSuccess) return st;
    timed_launch("down1", decode1_down_kernel<SHARED, QMAX>, dim3(kHidden / 32), dim3(512), 0, s, a);
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
