// Decode path (T <= 32 tokens): the routed MoE layer in three or four kernels.
//
//   K1 decode_route_kernel       router logits (fp32, declared order) and the
//                                quantised gate input; the last block to
//                                arrive runs softmax/top-8 and the stable
//                                permutation into per-bank segments.
//   K2 decode_gateup_kernel      one block per (segment, gate/up tile pair):
//                                64 KiB of codes staged in LDS, exact int8
//                                dots, fp32 group tree, then SiLU(gate)*up.
//   K3 decode_down_tile_kernel   T == 1: one block per 32-column tile over all
//                                routes; H128 + A8 of the middles, exact dots,
//                                fp32 tree and the slot reduction in-block.
//      decode_down_kernel        T > 1: one block per (segment, 128 columns),
//                                then reduce_kernel combines the slots.
//
// Arithmetic is the reference's (routed_storage_n32_consumer.cpp:22-307); the
// decomposition into kernels is this build's.  The only cross-block hand-off
// inside a kernel is K1's last-block election (one release fence per block,
// one acquire); kernel boundaries carry everything else.  Nothing waits on
// another block, so no launch can dead-lock.
#include "kernels.hpp"
#include "timing.hpp"
#include "topk.hpp"
#include "decode.hpp"

namespace ornith {

// Arrival counter of K1's last-block election.  It lives in this library's
// own device memory (not the caller's arena, which other ops overwrite
// between calls) and is reset by the last block, so every launch starts at 0.
// Launches on one device must therefore not overlap (the same single-stream
// use the reference's shared arena requires).
static __device__ uint32_t g_route_arrivals;

constexpr int kDecodeBanks = kExperts + 1;
constexpr int kMaxRoutes = kDecodeMaxTokens * (kTop + 1);
constexpr int kPadWords = 1056;

// ---------------------------------------------------------------------------
// K1
// ---------------------------------------------------------------------------
template <bool ROUTER, bool SHARED, int QMAX>
__global__ __launch_bounds__(1024) void decode_route_kernel(DecodeArgs a) {
    __shared__ uint4 xs[8][256];                  // 8 tokens x 2048 bf16
    __shared__ int s_last;
    __shared__ int s_bank[kMaxRoutes];
    __shared__ int s_cnt[kDecodeBanks], s_off[kDecodeBanks + 1];
    __shared__ int s_segidx[kDecodeBanks];
    __shared__ int s_ids[kDecodeMaxTokens * kTop];
    const int T = a.T, R = T * kTop;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int gw = blockIdx.x * 16 + wave, nwaves = gridDim.x * 16;
    uint32_t flags = 0;

    // ---- router logits: wave gw owns router row gw (256 = shared gate) ----
    if (ROUTER) {
        const bool has_row = gw < (SHARED ? kExperts + 1 : kExperts);
        const uint16_t* wrow = gw < kExperts ? a.router_w + size_t(gw) * kHidden : a.shared_gate_w;
        uint4 wr[4];
        if (has_row) {
#pragma unroll
            for (int i = 0; i < 4; ++i) wr[i] = *reinterpret_cast<const uint4*>(wrow + (i * 64 + lane) * 8);
        }
        const float b = (has_row && a.bias && gw < kExperts) ? a.bias[gw] : 0.f;
        for (int t0 = 0; t0 < T; t0 += 8) {
            const int nt = min(8, T - t0);
            __syncthreads();
            for (int q = tid; q < nt * 256; q += 1024)
                xs[q >> 8][q & 255] = *reinterpret_cast<const uint4*>(a.x + size_t(t0 + (q >> 8)) * kHidden + (q & 255) * 8);
            __syncthreads();
            if (has_row) {
                // lane partials of up to eight tokens first (independent chains), then the butterflies
                float acc[8];
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    acc[t] = 0.f;
                    if (t < nt) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const uint4 xv = xs[t][i * 64 + lane];
                            const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
                            const uint32_t ww[4] = {wr[i].x, wr[i].y, wr[i].z, wr[i].w};
#pragma unroll
                            for (int j = 0; j < 4; ++j) {
                                acc[t] = __builtin_fmaf(bf16_bits_to_f32(xw[j] & 0xffffu), bf16_bits_to_f32(ww[j] & 0xffffu), acc[t]);
                                acc[t] = __builtin_fmaf(bf16_bits_to_f32(xw[j] >> 16), bf16_bits_to_f32(ww[j] >> 16), acc[t]);
                            }
                        }
                    }
                }
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    if (t < nt) {
                        float v = wave_butterfly_sum(acc[t]);
                        if (a.bias && gw < kExperts) v = v + b;
                        if (lane == 0) a.logits[size_t(t0 + t) * kLogitStride + gw] = v;
                    }
                }
            }
        }
    }

    // ---- quantised gate input: one wave per (token, 256-group) ----
    for (int job = gw; job < T * (kHidden / kGroup); job += nwaves) {
        const int row = job >> 3, group = job & 7;
        bool live = true;
        if (!ROUTER && !SHARED) {
            live = false;
#pragma unroll
            for (int s = 0; s < kTop; ++s) {
                const int id = a.ids_in[row * kTop + s];
                live |= id >= 0 && id < kExperts;
            }
        }
        const uint2 raw = *reinterpret_cast<const uint2*>(a.x + size_t(row) * kHidden + group * kGroup + lane * 4);
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
        const size_t g = size_t(row) * 8 + group;
        quantize_group_wave<QMAX>(v, a.x_words + g * 64, a.x_scales + g, a.x_sums + g, flags,
                                  kFlagInvalidActivation);
    }

    // ---- K3's column-group counters (stream order makes these visible) ----
    if (blockIdx.x == 0 && tid < kDownGroups) a.counters[tid] = 0;

    // ---- last-block election ----
    // Every wave waits for its own stores, one release fence per block makes
    // them visible device-wide, and only the last block acquires.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        const uint32_t old = atomicAdd(&g_route_arrivals, 1u);
        s_last = old == gridDim.x - 1;
        if (s_last) {
            g_route_arrivals = 0;
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        }
    }
    __syncthreads();
    if (!s_last) { flag_or(a.sticky, flags); return; }

    // ---- top-8 (router) or the caller's ids ----
    if (ROUTER) {
        for (int t = wave; t < T; t += 16) {
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = a.logits[size_t(t) * kLogitStride + lane + 64 * i];
            float wv;
            int iv, i8[kTop];
            softmax_top8(v, wv, iv, i8);
            if (lane < kTop) {
                a.topk_w[t * kTop + lane] = wv;
                a.topk_ids[t * kTop + lane] = iv;
                s_ids[t * kTop + lane] = iv;
            }
            if (SHARED && lane == 0) a.shared_logit[t] = f32_to_bf16_bits(a.logits[size_t(t) * kLogitStride + kExperts]);
        }
    } else {
        for (int r = tid; r < R; r += 1024) s_ids[r] = a.ids_in[r];
    }
    for (int b = tid; b < kDecodeBanks; b += 1024) s_cnt[b] = 0;
    __syncthreads();

    // ---- stable counting sort of routes by bank ----
    const int Rall = R + (SHARED ? T : 0);
    for (int r = tid; r < Rall; r += 1024) {
        int bank = kShared;
        if (r < R) {
            const int id = s_ids[r];
            bank = (id >= 0 && id < kExperts) ? id : -1;
            if (bank < 0 && id != -1) flags |= kFlagInvalidExpert;
        }
        s_bank[r] = bank;
        if (bank >= 0) atomicAdd(&s_cnt[bank], 1);
    }
    __syncthreads();
    if (wave == 0) {
        // exclusive scans of counts and of non-empty flags over 257 banks,
        // 5 banks per lane (lane-serial) then a wave scan of the lane totals
        int c[5], nz[5], tc = 0, tn = 0;
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            const int b = lane * 5 + i;
            c[i] = b < kDecodeBanks ? s_cnt[b] : 0;
            nz[i] = c[i] > 0;
            tc += c[i];
            tn += nz[i];
        }
        int ic = tc, in = tn;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int oc = __shfl_up(ic, d, 64), on = __shfl_up(in, d, 64);
            if (lane >= d) { ic += oc; in += on; }
        }
        int runc = ic - tc, runn = in - tn;
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            const int b = lane * 5 + i;
            if (b < kDecodeBanks) {
                s_off[b] = runc;
                s_segidx[b] = nz[i] ? runn : -1;
                if (nz[i]) a.segments[runn] = Segment{b, runc, c[i], 0};
            }
            runc += c[i];
            runn += nz[i];
        }
        if (lane == 63) { s_off[kDecodeBanks] = ic; a.nseg[0] = in; a.nseg[1] = ic; }
    }
    __syncthreads();
    for (int r = tid; r < Rall; r += 1024) {
        const int bank = s_bank[r];
        if (bank < 0) continue;
        int rank = 0;
        for (int j = 0; j < r; ++j) rank += s_bank[j] == bank;
        a.routes[s_off[bank] + rank] = r;
    }
    flag_or(a.sticky, flags);
}

// ---------------------------------------------------------------------------
// K2: gate/up for one (segment, tile pair p): gate columns 32p..32p+31 and the
// matching up columns 512+32p..; writes middle[route, 32p..32p+31].
// Every global load that depends only on the segment is issued before the
// first wait: the 64 KiB of codes, the metadata, and the first route's
// quantised activations.
// ---------------------------------------------------------------------------
template <bool SHARED>
__global__ __launch_bounds__(256) void decode_gateup_kernel(DecodeArgs a) {
    __shared__ uint32_t lw[16 * kPadWords];
    __shared__ uint32_t lm[16 * 32];
    __shared__ uint32_t la[8 * 64];
    __shared__ float lsa[8], lss[8];
    __shared__ float lterm[16][32];
    if (int(blockIdx.x) >= a.nseg[0]) return;
    const Segment sg = a.segments[blockIdx.x];
    const int tid = threadIdx.x, p = blockIdx.y, R = a.T * kTop;
    const bool shared = SHARED && sg.bank == kShared;
    const uint32_t* codes = shared ? a.s13_codes : a.w13_codes + size_t(sg.bank) * kGateBankWords;
    const uint32_t* meta = shared ? a.s13_meta : a.w13_meta + size_t(sg.bank) * kGateBankMeta;
    uint4 stage[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        // block i = (h, g): tile p + 16h, group g; thread tid owns words 4tid..4tid+3
        const int h = i >> 3, g = i & 7;
        stage[i] = *reinterpret_cast<const uint4*>(codes + (size_t(p + 16 * h) * 8 + g) * 1024 + tid * 4);
    }
    uint32_t mreg[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int q = tid + 256 * k, blk = q >> 5, n = q & 31, h = blk >> 3, g = blk & 7;
        mreg[k] = meta[(size_t(p + 16 * h) * 8 + g) * 32 + n];
    }
    int route = a.routes[sg.first];
    int row = route < R ? route / kTop : route - R;
    uint32_t areg[2];
    areg[0] = a.x_words[size_t(row) * 512 + tid];
    areg[1] = a.x_words[size_t(row) * 512 + 256 + tid];
    float sreg = 0.f, ssum = 0.f;
    if (tid < 8) {
        sreg = f16_bits_to_f32(a.x_scales[row * 8 + tid]);
        ssum = sreg * float(a.x_sums[row * 8 + tid]);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) *reinterpret_cast<uint4*>(&lw[i * kPadWords + tid * 4]) = stage[i];
    lm[tid] = mreg[0];
    lm[tid + 256] = mreg[1];
    uint32_t flags = 0;
    for (int r = 0; r < sg.count; ++r) {
        if (r > 0) {
            __syncthreads();
            route = a.routes[sg.first + r];
            row = route < R ? route / kTop : route - R;
            areg[0] = a.x_words[size_t(row) * 512 + tid];
            areg[1] = a.x_words[size_t(row) * 512 + 256 + tid];
            if (tid < 8) {
                sreg = f16_bits_to_f32(a.x_scales[row * 8 + tid]);
                ssum = sreg * float(a.x_sums[row * 8 + tid]);
            }
        }
        la[tid] = areg[0];
        la[tid + 256] = areg[1];
        if (tid < 8) { lsa[tid] = sreg; lss[tid] = ssum; }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int blk = (tid >> 5) + 8 * k, n = tid & 31, g = blk & 7;
            const uint32_t* wb = &lw[blk * kPadWords + n];
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
            float vg = 0.f, vu = 0.f;
#pragma unroll
            for (int g = 0; g < 8; ++g) vg = vg + lterm[g][tid];
#pragma unroll
            for (int g = 0; g < 8; ++g) vu = vu + lterm[8 + g][tid];
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
                mid = silu_portable(vg) * vu;
            }
            if (!isfinite(mid)) flags |= kFlagNonfiniteMiddle | kFlagNonfiniteInput;
            a.middle[size_t(route) * kInter + p * 32 + tid] = mid;
        }
    }
    flag_or(a.sticky, flags);
}

// H128 + quantisation of one 256-group of a middle row, held as float4 per lane.
template <int QMAX>
__device__ __forceinline__ void quantize_middle(float4 m4, uint32_t* words, float* sa, float* ss, uint32_t& flags) {
    float v[4] = {m4.x, m4.y, m4.z, m4.w};
    h128_wave(v);
#pragma unroll
    for (int i = 0; i < 4; ++i) if (!isfinite(v[i])) flags |= kFlagNonfiniteInput;
    uint16_t sb;
    int32_t sum;
    quantize_group_wave<QMAX>(v, words, &sb, &sum, flags, kFlagInvalidActivation);
    if ((threadIdx.x & 63) == 0) {
        const float s = f16_bits_to_f32(sb);
        *sa = s;
        *ss = s * float(sum);
    }
}

// ---------------------------------------------------------------------------
// K3 (T == 1): one block per 32-column tile over every route (at most 8
// routed + 1 shared), so the slot reduction needs no other block.  Each block
// quantises the (at most 9) middle rows itself.
// ---------------------------------------------------------------------------
template <bool SHARED, int QMAX>
__global__ __launch_bounds__(256) void decode_down_tile_kernel(DecodeArgs a) {
    constexpr int MR = kTop + 1;
    __shared__ uint32_t lw[MR * 2 * kPadWords];
    __shared__ uint32_t lm[MR * 2 * 32];
    __shared__ uint32_t la[MR * 2 * 64];
    __shared__ float lsa[MR * 2], lss[MR * 2];
    __shared__ float lterm[MR * 2][32];
    __shared__ float lro[MR][32];
    __shared__ int lroute[MR], lslot[kTop + 1];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, c = blockIdx.x;
    const int nr = a.nseg[1];                      // valid routes in permuted order
    if (tid < MR) {
        const int route = tid < nr ? a.routes[tid] : -1;
        lroute[tid] = route;
    }
    if (tid < kTop + 1) lslot[tid] = -1;
    __syncthreads();
    if (tid < nr) lslot[lroute[tid] < kTop ? lroute[tid] : kTop] = tid;    // route -> row in this block
    // ---- weights: route i, group g, tile c (2 KiB-aligned 4 KiB blocks) ----
    uint4 stage[2 * MR];
#pragma unroll
    for (int k = 0; k < 2 * MR; ++k) {
        const int i = k >> 1, g = k & 1;
        stage[k] = make_uint4(0, 0, 0, 0);
        if (i < nr) {
            const int route = lroute[i];
            const int id = route < kTop ? a.reduce_ids[route] : kShared;
            const bool sh = SHARED && route >= kTop;
            const uint32_t* bank = sh ? a.s2_codes : a.w2_codes + size_t(id) * kDownBankWords;
            stage[k] = *reinterpret_cast<const uint4*>(bank + (size_t(c) * 2 + g) * 1024 + tid * 4);
        }
    }
    uint32_t mreg[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const int q = tid + 256 * k, i = q >> 6, g = (q >> 5) & 1, n = q & 31;
        mreg[k] = 0;
        if (i < nr) {
            const int route = lroute[i];
            const int id = route < kTop ? a.reduce_ids[route] : kShared;
            const bool sh = SHARED && route >= kTop;
            const uint32_t* meta = sh ? a.s2_meta : a.w2_meta + size_t(id) * kDownBankMeta;
            mreg[k] = meta[(size_t(c) * 2 + g) * 32 + n];
        }
    }
    // ---- middle rows: job (i, g) on wave (2i + g) % 4 ----
    uint32_t flags = 0;
    float4 mid[5];
#pragma unroll
    for (int k = 0; k < 5; ++k) {
        const int job = wave + 4 * k, i = job >> 1, g = job & 1;
        mid[k] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (i < nr) mid[k] = *reinterpret_cast<const float4*>(a.middle + size_t(lroute[i]) * kInter + g * kGroup + lane * 4);
    }
#pragma unroll
    for (int k = 0; k < 5; ++k) {
        const int job = wave + 4 * k, i = job >> 1;
        if (i < nr) quantize_middle<QMAX>(mid[k], &la[job * 64], &lsa[job], &lss[job], flags);
    }
#pragma unroll
    for (int k = 0; k < 2 * MR; ++k) *reinterpret_cast<uint4*>(&lw[k * kPadWords + tid * 4]) = stage[k];
#pragma unroll
    for (int k = 0; k < 3; ++k) if (tid + 256 * k < MR * 64) lm[tid + 256 * k] = mreg[k];
    __syncthreads();
    // ---- dots: term (i, g, n) ----
    for (int q = tid; q < nr * 64; q += 256) {
        const int blk = q >> 5, n = q & 31;
        const uint32_t* wb = &lw[blk * kPadWords + n];
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
    for (int q = tid; q < nr * 32; q += 256) {
        const int i = q >> 5, n = q & 31;
        float v = 0.f;
        v = v + lterm[2 * i][n];
        v = v + lterm[2 * i + 1][n];
        if (SHARED && lroute[i] >= kTop) v = bf16_round(v);
        if (!isfinite(v)) flags |= kFlagNonfiniteProjection;
        lro[i][n] = v;
    }
    __syncthreads();
    // ---- slot-order reduction of token 0 (routed_storage_n32_consumer.cpp:176-184, 296-307) ----
    if (tid < 32) {
        const int col = c * 32 + tid;
        float sum = 0.f;
#pragma unroll
        for (int s = 0; s < kTop; ++s) {
            const int id = a.reduce_ids[s];
            if (id >= 0 && id < kExperts) sum = sum + lro[lslot[s]][tid] * a.reduce_w[s];
        }
        const uint16_t o = f32_to_bf16_bits(sum);
        if (!isfinite(sum) || (o & 0x7f80u) == 0x7f80u) flags |= kFlagNonfiniteOutput;
        if (a.final_f32) a.final_f32[col] = sum;
        if (a.out) a.out[col] = o;
        if (SHARED) {
            const float gate = bf16_bits_to_f32(a.sigmoid_table[a.shared_logit[0]]);
            const float sv = lro[lslot[kTop]][tid] * gate;
            if (!isfinite(sv)) flags |= kFlagNonfiniteOutput;
            const uint16_t so = f32_to_bf16_bits(sv);
            if (a.shared_out) a.shared_out[col] = so;
            if (a.layer_out) a.layer_out[col] = f32_to_bf16_bits(bf16_bits_to_f32(o) + bf16_bits_to_f32(so));
        }
    }
    flag_or(a.sticky, flags);
}

// ---------------------------------------------------------------------------
// K3 (T > 1): down projection for one (segment, 128-column group), writing
// route_out; the slot reduction runs in its own kernel afterwards.
// ---------------------------------------------------------------------------
template <bool SHARED, int QMAX>
__global__ __launch_bounds__(256) void decode_down_kernel(DecodeArgs a) {
    __shared__ uint32_t lw[8 * kPadWords];
    __shared__ uint32_t lm[8 * 32];
    __shared__ uint32_t la[2 * 64];
    __shared__ float lsa[2], lss[2];
    __shared__ float lterm[8][32];
    if (int(blockIdx.x) >= a.nseg[0]) return;
    const Segment sg = a.segments[blockIdx.x];
    const int tid = threadIdx.x, cg = blockIdx.y, lane = tid & 63, wave = tid >> 6;
    const bool shared = SHARED && sg.bank == kShared;
    const uint32_t* codes = shared ? a.s2_codes : a.w2_codes + size_t(sg.bank) * kDownBankWords;
    const uint32_t* meta = shared ? a.s2_meta : a.w2_meta + size_t(sg.bank) * kDownBankMeta;
    uint4 stage[8];
    const uint32_t* src = codes + size_t(4 * cg) * 2 * 1024;
#pragma unroll
    for (int i = 0; i < 8; ++i) stage[i] = *reinterpret_cast<const uint4*>(src + size_t(i * 256 + tid) * 4);
    const uint32_t mreg = meta[size_t(4 * cg) * 2 * 32 + tid];
    int route = a.routes[sg.first];
    float4 m4 = make_float4(0.f, 0.f, 0.f, 0.f);
    if (wave < 2) m4 = *reinterpret_cast<const float4*>(a.middle + size_t(route) * kInter + wave * kGroup + lane * 4);
#pragma unroll
    for (int i = 0; i < 8; ++i) *reinterpret_cast<uint4*>(&lw[i * kPadWords + tid * 4]) = stage[i];
    lm[tid] = mreg;
    uint32_t flags = 0;
    for (int r = 0; r < sg.count; ++r) {
        if (r > 0) {
            __syncthreads();
            route = a.routes[sg.first + r];
            if (wave < 2) m4 = *reinterpret_cast<const float4*>(a.middle + size_t(route) * kInter + wave * kGroup + lane * 4);
        }
        if (wave < 2) quantize_middle<QMAX>(m4, &la[wave * 64], &lsa[wave], &lss[wave], flags);
        __syncthreads();
        {
            const int blk = tid >> 5, n = tid & 31, g = blk & 1;
            const uint32_t* wb = &lw[blk * kPadWords + n];
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
        if (tid < 128) {
            const int tl = tid >> 5, n = tid & 31;
            float v = 0.f;
            v = v + lterm[2 * tl][n];
            v = v + lterm[2 * tl + 1][n];
            if (shared) v = bf16_round(v);
            if (!isfinite(v)) flags |= kFlagNonfiniteProjection;
            a.route_out[size_t(route) * kHidden + cg * 128 + tid] = v;
        }
    }
    flag_or(a.sticky, flags);
}

// ---------------------------------------------------------------------------
size_t decode_scratch_bytes() {
    return align256(size_t(kDecodeMaxTokens) * kLogitStride * 4) + align256(kDecodeBanks * sizeof(Segment)) +
           align256(kMaxRoutes * 4) + align256(kDownGroups * 4) + align256(8);
}

void carve_decode(void* base, DecodeArgs& a) {
    size_t off = 0;
    auto take = [&](size_t bytes) { void* q = at<void>(base, off); off += align256(bytes); return q; };
    a.logits = static_cast<float*>(take(size_t(kDecodeMaxTokens) * kLogitStride * 4));
    a.segments = static_cast<Segment*>(take(kDecodeBanks * sizeof(Segment)));
    a.routes = static_cast<int32_t*>(take(kMaxRoutes * 4));
    a.counters = static_cast<uint32_t*>(take(kDownGroups * 4));
    a.nseg = static_cast<int32_t*>(take(8));
}

template <bool ROUTER, bool SHARED, int QMAX>
static hipError_t run(const DecodeArgs& a, hipStream_t s) {
    const int T = a.T, R = T * kTop;
    const int k1_blocks = ROUTER ? (SHARED ? 17 : 16) : max(1, (T * 8 + 15) / 16);
    timed_launch("route", decode_route_kernel<ROUTER, SHARED, QMAX>, dim3(k1_blocks), dim3(1024), 0, s, a);
    hipError_t st = hipGetLastError();
    if (st != hipSuccess) return st;
    const int maxseg = min(R, kExperts) + (SHARED ? 1 : 0);
    timed_launch("gateup", decode_gateup_kernel<SHARED>, dim3(maxseg, 16), dim3(256), 0, s, a);
    st = hipGetLastError();
    if (st != hipSuccess) return st;
    if (T == 1) {
        timed_launch("down", decode_down_tile_kernel<SHARED, QMAX>, dim3(kHidden / 32), dim3(256), 0, s, a);
        return hipGetLastError();
    }
    timed_launch("down", decode_down_kernel<SHARED, QMAX>, dim3(maxseg, kDownGroups), dim3(256), 0, s, a);
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
