// Decode-path (T <= 32) arguments and launcher.
#pragma once
#include "kernels.hpp"

namespace ornith {

constexpr int kDecodeMaxTokens = 32;
constexpr int kLogitStride = kExperts + 1;
constexpr int64_t kGateBankWords = int64_t(2 * kInter) * kHidden / 8;
constexpr int64_t kGateBankMeta = int64_t(2 * kInter) * (kHidden / kGroup);
constexpr int64_t kDownBankWords = int64_t(kHidden) * kInter / 8;
constexpr int64_t kDownBankMeta = int64_t(kHidden) * (kInter / kGroup);

struct DecodeArgs {
    int T;
    const uint16_t* x;                 // [T, 2048] bf16
    // router (layer entry)
    const uint16_t* router_w;          // [256, 2048] bf16
    const float* bias;                 // [256] or null
    const uint16_t* shared_gate_w;     // [2048] bf16
    float* topk_w; int32_t* topk_ids;  // outputs [T, 8]
    // caller routing (routed entries)
    const int32_t* ids_in;
    // routing used by the reduce (= topk outputs or the caller's)
    const float* reduce_w; const int32_t* reduce_ids;
    // banks
    const uint32_t *w13_codes, *w13_meta, *w2_codes, *w2_meta;
    const uint32_t *s13_codes, *s13_meta, *s2_codes, *s2_meta;
    const float* silu_table; const uint16_t* sigmoid_table;
    uint16_t* shared_logit;            // bf16 [T]: written by the router, else read
    // workspace
    uint32_t* x_words; uint16_t* x_scales; int32_t* x_sums;
    float* middle;                     // [RS, 512]
    uint32_t* m_words; uint16_t* m_scales; int32_t* m_sums;   // quantised middle rows (2..32 tokens)
    float* route_out;                  // [RS, 2048]
    float* logits; Segment* segments; int32_t* routes; int32_t* nseg;
    // outputs
    float* final_f32; uint16_t* out; uint16_t* shared_out; uint16_t* layer_out;
    uint32_t* sticky;
};

size_t decode_scratch_bytes();
void carve_decode(void* base, DecodeArgs& a);
hipError_t launch_decode(const DecodeArgs& a, bool router, bool shared, int qmax, hipStream_t s);
hipError_t launch_decode1(const DecodeArgs& a, bool router, bool shared, int qmax, hipStream_t s);

}  // namespace ornith
