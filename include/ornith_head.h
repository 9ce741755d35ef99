/* W8 G128 LM-head C ABI of the MI355X (gfx950) Ornith library.
 *
 * Drop-in for libornith_head_i8_tile.so (kernels/head/head_i8_tile_api.h).
 * Weights keep the reference's physical layout: uint32 [N/16, K/16, 4, 16],
 * each word four signed K bytes, lowest K first; scales fp16 [N, 16].
 * K = 2048, G = 128, N in {256, 1024, 4096, 65536, 248320}, 0 <= M <= Mcap <= 64.
 * Arithmetic (bit-exact): fp32 H128, per-128 A8 encoding (absmax/127, fp16
 * scale floor 2^-14, round-even, clamp +-127), exact int8 group dots,
 * acc = acc + RN(sw * RN(sa * dot)) over groups 0..15, bf16 RNE output with the
 * fp32 projection kept in the workspace (head_i8_tile_api.h:22-42).
 * Contract differences: workspace internals are this library's own (the
 * layout struct keeps the reference field names, `transformed` has size 0);
 * weights must be 16-byte aligned.  `geometry` 0..2 is accepted and does not
 * change results: every row count runs on the int8 matrix cores
 * (v_mfma_i32_16x16x64_i8, rows in tiles of 16, each weight byte read once).
 * Flags: 1 non-finite input/transform, 2 invalid activation, 4 non-finite
 * projection, 8 non-finite bf16 (head_i8_tile_api.h:16-21).
 */
#ifndef ORNITH_MI355X_HEAD_H
#define ORNITH_MI355X_HEAD_H
#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>
#ifdef __cplusplus
extern "C" {
#endif
#ifndef ORNITH_EXPORT
#ifndef ORNITH_EXPORT
#define ORNITH_EXPORT __attribute__((visibility("default")))
#endif
#endif

/* head_i8_tile_api.h:13-15 */
typedef struct OrnithHeadI8Layout {
    size_t workspace_bytes, transformed, activation_words, activation_scales, projection;
} OrnithHeadI8Layout;

/* head_i8_tile_api.h:43 (returns 1) */
ORNITH_EXPORT uint32_t ornith_head_i8_tile_abi_version(void);
/* head_i8_tile_consumer.cpp:293 (returns 1): the build's capability marker
 * that the launch below takes the optional per-group dots (the raw 16 group
 * dots of every logit a shortlist re-scoring reads). */
ORNITH_EXPORT int ornith_head_i8_tile_shortlist(void);
/* head_i8_tile_api.h:44; head_i8_tile_consumer.cpp:248-256 */
ORNITH_EXPORT hipError_t ornith_head_i8_tile_get_layout(int Mcap, int N, OrnithHeadI8Layout* out);
/* head_i8_tile_api.h:45-49; head_i8_tile_consumer.cpp:257-291.  group_dots int32 [M,N,16]
 * (raw group dots) is optional: NULL iff group_dots_bytes == 0. */
ORNITH_EXPORT hipError_t ornith_head_i8_tile_launch(
    const void* input_bf16, const void* weights_i8, const void* scales_f16,
    void* workspace, size_t workspace_bytes, void* output_bf16,
    void* group_dots_i32, size_t group_dots_bytes, void* flags_u32,
    int M, int Mcap, int N, int geometry, hipStream_t stream);

/* Greedy sampling hand-off after a head (no C counterpart in the reference,
 * which takes torch.argmax of the bf16 logits downstream): argmax_i64[m] =
 * the column of row m's maximum bf16 logit (the first NaN if the row has
 * one, else the first maximum, as torch.argmax / numpy.argmax).  logits
 * bf16 [M, N] with row stride ld >= N elements; M == 0 or N == 0 returns
 * hipSuccess without touching memory. */
ORNITH_EXPORT hipError_t ornith_logits_argmax_launch(const void* logits_bf16, int M, int N, int64_t ld,
                                                     void* argmax_i64, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif
