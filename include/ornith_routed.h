/* Routed G256 MoE C ABI of the MI355X (gfx950) Ornith library.
 *
 * Drop-in for the reference's routed libraries: same symbol names, argument
 * order and meaning, return codes and sticky-flag bits.  Each declaration
 * cites the reference interface it replaces.  The library is built twice
 * from the same sources, one build per routed bank layout:
 *   libornith_g256_mi355x_n16.so - N16 banks, for libornith_routed_direct.so
 *                                  (routed_direct_api.h:7; ornith_routed_storage_n32 returns 16);
 *   libornith_g256_mi355x.so     - N32 banks, for libornith_routed_storage_n32.so
 *                                  (routed_storage_n32_consumer.cpp:1-2; returns 32).
 *
 * Storage (unchanged from the reference; T = 32 for the N32 build, 16 for the N16 build):
 *   codes    uint32 [E=256, N/T, K/256, 32, T]; word ((e*N/T + n/T)*K/256 + g)*32*T + j*T + n%T
 *            packs K values 256g+8j .. +7 of row n, low nibble first (unsigned 4-bit).
 *   metadata uint32 [E, N/T, K/256, T] = fp16 scale | fp16 offset << 16; w = scale*code + offset.
 *   The shared-expert banks of the *_shared_tables and layer entries are N32 in both builds.
 *   gate_up: N=1024 (gate rows 0..511, up rows 512..1023), K=2048; down: N=2048, K=512.
 *
 * Arithmetic (bit-exact with the reference A8/A4 paths): fp32 H128 of each
 * 128 block, group-256 activation quantisation (qmax 127 for A8, 7 for A4),
 * exact integer dot per group, the fp32 group tree in ascending group order,
 * SiLU via the reference's portable exp, slot-order fp32 reduction, bf16 RNE.
 *
 * Contract differences (all stricter, none in arithmetic):
 *   - workspace internals are this library's own; OrnithRoutedDirectLayout keeps
 *     the reference field names and order but fields this library does not use
 *     have size zero, so workspace_bytes differs from the reference's;
 *   - alignment: input 16 bytes, codes 16 bytes, workspace 256 bytes;
 *   - Tcap <= 8192 for every entry (the reference's N16 parent allowed 2048).
 * Sticky flags (uint32, OR-ed, never cleared): 1 non-finite input/transform,
 * 2 invalid activation scale, 4 invalid expert id (other than -1), 8 non-finite
 * projection, 16 non-finite middle, 32 non-finite/overflowed output.
 * Every launch is asynchronous on `stream`, allocates nothing and reads no host
 * data; T == 0 returns hipSuccess after scalar validation without touching any
 * pointer; bad arguments return hipErrorInvalidValue before any launch.
 */
#ifndef ORNITH_MI355X_ROUTED_H
#define ORNITH_MI355X_ROUTED_H
#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>
#ifdef __cplusplus
extern "C" {
#endif
#ifndef ORNITH_EXPORT
#define ORNITH_EXPORT __attribute__((visibility("default")))
#endif

/* kernels/routed_storage/routed_direct_api.h:13-16 */
typedef struct OrnithRoutedDirectLayout {
    size_t workspace_bytes, gate_x, gate_low, gate_high, gate_scales, gate_sums, gate_y;
    size_t middle, down_x, down_low, down_high, down_scales, down_sums, route_out, final_f32;
} OrnithRoutedDirectLayout;

/* routed_direct_api.h:18; routed_storage_n32_consumer.cpp:309-318.  0 <= Tcap <= 8192. */
ORNITH_EXPORT hipError_t ornith_routed_direct_get_layout(int Tcap, OrnithRoutedDirectLayout* out);

/* routed_direct_api.h:19-22; routed_storage_n32_consumer.cpp:319-359.  A8 activations. */
ORNITH_EXPORT hipError_t ornith_routed_direct_launch(
    const void* input_bf16, const void* route_weights_f32, const void* ids_i32,
    const void* gate_codes, const void* gate_meta, const void* down_codes, const void* down_meta,
    void* workspace, size_t bytes, void* output_bf16, void* flags_u32, int T, int Tcap, hipStream_t stream);

/* routed_direct_api.h:23-28; routed_storage_n32_consumer.cpp:360.  Signed A4 activations. */
ORNITH_EXPORT hipError_t ornith_routed_direct_launch_a4(
    const void* input_bf16, const void* route_weights_f32, const void* ids_i32,
    const void* gate_codes, const void* gate_meta, const void* down_codes, const void* down_meta,
    void* workspace, size_t bytes, void* output_bf16, void* flags_u32, int T, int Tcap, hipStream_t stream);

/* routed_direct_api.h:29-33; routed_storage_n32_consumer.cpp:362-370.  A4 iff T > 64, else A8. */
ORNITH_EXPORT hipError_t ornith_routed_direct_launch_a4_prefill(
    const void* input_bf16, const void* route_weights_f32, const void* ids_i32,
    const void* gate_codes, const void* gate_meta, const void* down_codes, const void* down_meta,
    void* workspace, size_t bytes, void* output_bf16, void* flags_u32, int T, int Tcap, hipStream_t stream);

/* routed_storage_n32_consumer.cpp:372-373 (storage marker, returns 32; prefill output tile, returns 32). */
ORNITH_EXPORT int ornith_routed_storage_n32(void);
ORNITH_EXPORT int ornith_routed_prefill_output_tile(void);

/* routed_storage_n32_consumer.cpp:375-384.  Shared-expert-as-ninth-slot layout, 0 <= Tcap <= 16. */
ORNITH_EXPORT hipError_t ornith_routed_shared_get_layout(int Tcap, OrnithRoutedDirectLayout* out);

/* routed_storage_n32_consumer.cpp:385-401.  Routed A8 + shared expert (dense N32
 * banks gate_up [1024,2048], down [2048,512]); shared linear outputs bf16,
 * SiLU from silu_f32[65536], gate sigmoid_bf16[65536] indexed by raw bf16 bits of
 * shared_logit_bf16[T].  output = routed bf16 [T,2048]; shared_output = shared bf16 [T,2048]. */
ORNITH_EXPORT hipError_t ornith_routed_direct_launch_shared_tables(
    const void* input_bf16, const void* route_weights_f32, const void* ids_i32,
    const void* gate_codes, const void* gate_meta, const void* down_codes, const void* down_meta,
    const void* shared_gate_codes, const void* shared_gate_meta,
    const void* shared_down_codes, const void* shared_down_meta,
    const void* shared_logit_bf16, const void* silu_f32, const void* sigmoid_bf16,
    void* workspace, size_t bytes, void* output_bf16, void* shared_output_bf16, void* flags_u32,
    int T, int Tcap, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif
