// Internal launch wrappers shared by the C-ABI translation units.  Every
// wrapper enqueues on the caller's stream and returns hipGetLastError().
#pragma once
#include "common.hpp"
#include <atomic>

namespace ornith {

// Compute units of the current device, queried once per device (256 on
// MI355X; `fallback` if the query fails).
inline int device_cu_count(int fallback = 256) {
    constexpr int kMaxDevices = 64;
    static std::atomic<int> cached[kMaxDevices];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return fallback;
    int n = cached[dev].load(std::memory_order_relaxed);
    if (n <= 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return fallback;
        cached[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

// The device that runs stream `s` (for HIP's null stream, the current
// device); -1 if the query fails.
inline int stream_device(hipStream_t s) {
    int dev = -1;
    if (hipStreamGetDevice(s, &dev) != hipSuccess) return -1;
    return dev;
}

// Blocks of `kernel` (`threads` threads, no dynamic LDS) that can be resident
// at once on device `dev`, all CUs together; -1 if a query fails.  The
// occupancy query runs with `dev` current (restored afterwards).
template <class Kernel>
int resident_blocks(Kernel kernel, int threads, int dev) {
    int current = -1, per_cu = 0, cus = 0;
    if (dev < 0 || hipGetDevice(&current) != hipSuccess) return -1;
    if (current != dev && hipSetDevice(dev) != hipSuccess) return -1;
    const bool ok = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) == hipSuccess &&
                    hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess;
    if (current != dev && hipSetDevice(current) != hipSuccess) return -1;
    return ok && per_cu > 0 && cus > 0 ? per_cu * cus : -1;
}

// A run of consecutive entries of the permuted route list that all use one
// weight bank (expert id 0..255, or kShared for the shared expert).
struct Segment { int32_t bank, first, count, tile_base; };

// Scratch used by the permutation step, carved out of the caller's workspace.
struct PermuteScratch {
    int32_t* block_counts;   // [blocks, banks]
    int32_t* counts;         // [banks]
    int32_t* offsets;        // [banks + 1]
    int32_t* routes;         // [routes] permuted route ids
    Segment* segments;       // [banks]
    int32_t* meta;           // [4]: segment count, mfma tile count, ...
    Segment* tiles;          // [max tiles] per m-tile: bank, first permuted route, rows, tile-in-segment
};

// ---- activations -----------------------------------------------------------
// H128 + group quantisation of bf16 rows [rows, K] (row stride in elements).
// ids != nullptr: routed gate input, tokens without a live id are zeroed
// (routed_storage_n32_consumer.cpp:24-29).
hipError_t launch_act_bf16(const uint16_t* x, int64_t stride, int rows, int K, int qmax,
                           const int32_t* ids, uint32_t* words, uint16_t* scales, int32_t* sums,
                           uint32_t* sticky, uint32_t flag_input, uint32_t flag_act, hipStream_t s);
// Middle (SiLU(gate) * up) + H128 + quantisation for RS route rows of
// gate_y [RS, 1024].  Rows >= R are shared-expert rows (table SiLU, bf16
// rounding) when silu_table != nullptr.
hipError_t launch_act_middle(const float* gate_y, int RS, int R, const int32_t* ids, int qmax,
                             const float* silu_table, uint32_t* words, uint16_t* scales,
                             int32_t* sums, uint32_t* sticky, hipStream_t s);

// ---- routing ---------------------------------------------------------------
constexpr int kRouterRowsMaxTokens = 256;      // wave-per-row router up to here, token-tiled beyond
// Router logits [T, 256 (+1)] in the declared order; shared_w (nullable) adds
// column 256, the shared-expert gate logit.  split_sums (nullable,
// router_split_bytes): for T > kRouterRowsMaxTokens the last
// router_split_groups(T) token groups run as eighth-tile units whose partial
// sums launch_topk completes (their logits are final only after it).
hipError_t launch_router(const uint16_t* x, int64_t stride, int T, const uint16_t* w, const uint16_t* shared_w,
                         const float* bias, float* logits, int64_t logit_stride, hipStream_t s,
                         float* split_sums = nullptr);
int router_split_groups(int T);
size_t router_split_bytes(int Tcap);
// block_counts != nullptr (the layer path) also does the permutation's count
// step: launch_permute(..., counted = true) then skips it.
// split_sums (with bias): the logits of the last router_split_groups(T) token
// groups are completed here from the router's eighth-tile sums (and written
// back to logits).
hipError_t launch_topk(const float* logits, int64_t logit_stride, int T, float* weights, int32_t* ids,
                       const float* shared_logit_f32, int64_t shared_stride, uint16_t* shared_logit_bf16,
                       hipStream_t s, int32_t* block_counts = nullptr, const float* split_sums = nullptr,
                       const float* bias = nullptr);
// The A8 gate-input quantisation of contiguous bf16 rows (launch_act_bf16 with
// K = stride = kHidden, qmax 127): rows with no live id are skipped when ids
// is given.
struct ActJob {
    const uint16_t* x; int rows; const int32_t* ids;
    uint32_t* words; uint16_t* scales; int32_t* sums;
};
// Stable counting sort of route ids by bank.  Routes 0..R-1 use ids[r];
// when with_shared, routes R..R+T-1 use the shared bank.  act (nullable):
// that quantisation runs as trailing blocks of the bank-scan launch (its 64
// blocks leave the rest of the chip idle).
size_t permute_scratch_bytes(int Rcap, int Tcap);
PermuteScratch carve_permute(void* base, int Rcap, int Tcap);
hipError_t launch_permute(const int32_t* ids, int R, int T, bool with_shared, const PermuteScratch& p,
                          uint32_t* sticky, int mfma_rows, hipStream_t s, bool counted = false,
                          const ActJob* act = nullptr);

// ---- projections -----------------------------------------------------------
enum class Out { Routed, Dense };
struct ProjArgs {
    const uint32_t* codes; const uint32_t* meta;             // routed or dense bank
    const uint32_t* shared_codes; const uint32_t* shared_meta;
    int64_t bank_words, bank_meta_words;                       // per-expert strides
    const Segment* segments; const int32_t* nseg;             // device segment table
    const int32_t* routes;                                      // permuted route ids
    int row_mode;                                               // 0: row = route, 1: gate row (route/8 or route-R)
    int R;
    int dense_rows;            // rows when segments == nullptr (dense: one bank, rows 0..M-1)
    const uint32_t* act_words; const uint16_t* act_scales; const int32_t* act_sums;
    float* out;               // f32 [rows, N]
    uint16_t* out_bf16;       // dense: bf16 [rows, N]
    int N, K, tile;           // tile: 16 or 32 (bank layout)
    uint32_t* sticky;
    uint32_t flag_projection, flag_bf16;
    // dense, rows <= kDenseFusedRows: bf16 input [rows, K]; the projection
    // kernel then prepares the activations itself (act_words unused)
    const uint16_t* dense_x;
    uint32_t flag_input, flag_act;
};
constexpr int kDenseStreamRows = 64;   // weight-streaming projection up to this many rows
constexpr int kDenseFusedRows = 8;     // ... with activations prepared in the same kernel
hipError_t launch_project_gemv(const ProjArgs& a, int max_segments, Out mode, hipStream_t s);

// Grouped int8-MFMA projection over the permuted routes (prefill path).
struct MfmaArgs {
    const Segment* segments; const Segment* tiles; const int32_t* ntiles; const int32_t* routes;
    int R;                                       // routed routes; rows >= R are shared-expert rows
    const uint32_t* codes; const uint32_t* meta; const uint32_t* shared_codes; const uint32_t* shared_meta;
    int64_t bank_words, bank_meta_words;
    const uint32_t* act_words; const uint16_t* act_scales; const int32_t* act_sums;
    int K;
    float* out;                                  // gate/up: middle [RS, 512]; down: route_out [RS, 2048]
    const float* silu_table;
    uint32_t* sticky;
    // dense head (rows = R, identity; columns N): fp32 and bf16 logits [R, N],
    // argmax partials [R, partials] (one per wave of the <= 32-row kernel or per
    // 128-column block of the 33..64-row kernel), the dense flag bits
    int N;
    uint16_t* out_bf16;
    float* arg_val; int32_t* arg_idx;
    uint32_t flag_projection, flag_bf16;
    int tile_xcd;                                // prefill block order: 0 column-block major, 1 tile per XCD, 2 tile ranges per XCD
};
hipError_t launch_grouped_mfma(const MfmaArgs& a, bool gateup, int max_tiles, hipStream_t s);
// Dense G256 head on the matrix cores: M <= 64 rows of A8 activations against
// N32 codes, then the per-row argmax (numpy rule) into argmax[M].
hipError_t launch_head_mfma(const MfmaArgs& a, int64_t* argmax, hipStream_t s);
// H128 + quantisation of middle rows stored in permuted route order: rows 0 .. *nrows - 1
// (the permuted routes, all with a valid bank), RS rows at most.
hipError_t launch_quant_middle_permuted(const float* middle, int RS, const int32_t* nrows, int qmax, uint32_t* words,
                                        uint16_t* scales, int32_t* sums, uint32_t* sticky, hipStream_t s);

// ---- combination -------------------------------------------------------------
// out[t] = bf16(sum over valid slots of route_out[8t+s] * w[8t+s]); optional
// fp32 diagnostic; optional shared output and layer sum.
hipError_t launch_reduce(const float* route_out, const float* weights, const int32_t* ids, int T,
                         float* final_f32, uint16_t* out, const uint16_t* shared_logit,
                         const uint16_t* sigmoid_table, uint16_t* shared_out, uint16_t* layer_out,
                         uint32_t* sticky, hipStream_t s);

// ---- dense bf16 preparation (dense_g256_consumer.cpp:192-246) ---------------
hipError_t launch_transform_bf16(const uint16_t* x, int M, int K, uint16_t* y, uint32_t* sticky, hipStream_t s);
hipError_t launch_dequantize_bf16(const uint32_t* codes, const uint32_t* meta, int N, int K, int tile,
                                  uint16_t* w, uint32_t* sticky, hipStream_t s);

// ---- dense bf16 GEMM reading 4-bit codes (gemm.hip) ---------------------------
// y = bf16(H128 x) [M, K] row-major (flags: 1 non-finite input/transform, 8 non-finite bf16)
hipError_t launch_transform_bf16_fast(const uint16_t* x, int M, int K, uint16_t* y, uint32_t* sticky, hipStream_t s);
// the same values in matrix-core fragment order over round_up(M, 16) rows
// (padding rows zero): (r, k) at ((r / 16 * K / 32 + k / 32) * 64 + 16 (k % 32 / 8) + r % 16) * 8 + k % 8
hipError_t launch_transform_bf16_frag(const uint16_t* x, int M, int K, uint16_t* y, uint32_t* sticky, hipStream_t s);
// out bf16 [M, N] = y @ bf16(dequant(N16 codes, meta))^T, fp32 accumulation; y in fragment order.
// A grid that fills few block slots splits K into slices (dense_gemm_slices)
// whose fp32 sums go to `partial` (up to partial_bytes; null: no split) and
// are added in slice order.
constexpr int kMaxDenseSlices = 8;
int dense_gemm_slices(int M, int N, int K, size_t partial_bytes);
hipError_t launch_dense_gemm_bf16(const uint16_t* xt, const uint32_t* codes, const uint32_t* meta, int M, int N, int K,
                                  uint16_t* out, float* partial, size_t partial_bytes, uint32_t* sticky,
                                  hipStream_t s);

// ---- shared expert, fixed8 semantics (shared.hip) ------------------------------
// act [M, 512] bf16 from the bf16 gate/up projection gu [M, 1024] (tabulated
// SiLU rounded to bf16, bf16 product) and the bf16 gate logit x . gate_w [M].
hipError_t launch_fixed8_act(const uint16_t* gu, const uint16_t* x, const uint16_t* gate_w, const float* silu,
                             uint16_t* act, uint16_t* logit, int M, hipStream_t s);
// out [M, 2048] = bf16(sigmoid_table[logit] * down)
hipError_t launch_fixed8_gate(const uint16_t* down, const uint16_t* logit, const uint16_t* sigmoid, uint16_t* out,
                              int M, uint32_t* sticky, hipStream_t s);

// ---- fill (graph-capture safe replacement for hipMemsetAsync) -------------------
hipError_t launch_fill_u32(uint32_t* p, size_t n, uint32_t v, hipStream_t s);
// Both SiLU forms of the gate/up epilogue over every fp32 value of the short
// form's domain: values compared and mismatching bit patterns.
hipError_t launch_silu_selfcheck(unsigned long long* checked, uint32_t* mismatches, hipStream_t s);

}  // namespace ornith
