/* Dense G256 linear C ABI of the MI355X (gfx950) Ornith library.
 *
 * Drop-in for libornith_dense_g256.so and libornith_dense_g256_n32.so
 * (kernels/dense/dense_g256_api.h, kernels/dense_n32/dense_g256_consumer.cpp).
 * Storage is the reference's: codes uint32 [N/16, K/256, 32, 16] (N16 entries)
 * or [N/32, K/256, 32, 32] (N32 entries), eight low-first 4-bit K values per
 * word; metadata uint32 [N/16, K/256, 16] or [N/32, K/256, 32] = fp16 scale |
 * fp16 offset << 16.
 *
 * Arithmetic (bit-exact): fp32 H128, A8 group quantisation, exact integer
 * dot, fp32 group tree, bf16 RNE output with the fp32 projection kept in the
 * workspace (dense_g256_api.h:32-38).
 * Contract differences: workspace internals are this library's own
 * (OrnithDenseG256Layout keeps the field names; unused fields have size 0);
 * input alignment 16 bytes, codes 16 bytes.
 * Flags: 1 non-finite input/transform, 2 invalid activation, 4 non-finite
 * projection, 8 non-finite bf16 (dense_g256_api.h:14-19).
 */
#ifndef ORNITH_MI355X_DENSE_H
#define ORNITH_MI355X_DENSE_H
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

/* dense_g256_api.h:11-13 */
typedef struct OrnithDenseG256Layout {
    size_t workspace_bytes, transformed, low, high, scales, sums, projection;
} OrnithDenseG256Layout;

/* dense_g256_api.h:45 (returns 1) */
ORNITH_EXPORT uint32_t ornith_dense_g256_abi_version(void);

/* dense_g256_api.h:46; dense_g256_consumer.cpp:162-171.  0<=Mcap<=8192, N%16==0,
 * 0<N<=12288 or N==248320, K%256==0, 0<K<=8192, bits==8. */
ORNITH_EXPORT hipError_t ornith_dense_g256_get_layout(int Mcap, int N, int K, int bits, OrnithDenseG256Layout* out);

/* dense_g256_api.h:47-50; dense_g256_consumer.cpp:172-189.  N16 codes.  transform==128,
 * geometry 0..2 (accepted; this library has one kernel family for every geometry).
 * The workspace's fp32 projection is always written; its activation words, scales
 * and sums only for M > 8 (up to 8 rows the projection kernel prepares them itself). */
ORNITH_EXPORT hipError_t ornith_dense_g256_launch(
    const void* input_bf16, const void* codes, const void* metadata,
    void* workspace, size_t workspace_bytes, void* output_bf16, void* flags_u32,
    int M, int Mcap, int N, int K, int bits, int transform, int geometry, hipStream_t stream);

/* dense_g256_api.h:51-59; dense_g256_consumer.cpp:231-246.  bf16(H128 x) [M,K] and
 * bf16(RN(RN(scale*code)+offset)) [N,K] from N16 codes, for a bf16 GEMM. */
ORNITH_EXPORT hipError_t ornith_dense_g256_prepare_bf16(
    const void* input_bf16, const void* codes, const void* metadata,
    void* transformed_bf16, void* weights_bf16, void* flags_u32,
    int M, int N, int K, hipStream_t stream);

/* dense_g256_consumer.cpp:192-246 + the torch.mm that follows it (plugin-site/
 * ornith_g256/native.py:140-150) as one operation: out bf16 [M,N] =
 * bf16(H128 x) @ bf16(RN(RN(scale*code)+offset))^T with fp32 accumulation,
 * reading the N16 codes directly (no dequantised weight copy).  The
 * summation order is this library's (the reference's is hipBLASLt's), so the
 * product agrees with it within fp32-accumulation tolerance.  Workspace: at
 * least round_up(M,16)*K*2 bytes (the transformed activations, in the
 * library's matrix-core fragment order), 256-byte aligned; output 16-byte
 * aligned.  Bytes beyond that (up to 32 MiB are used) let a product whose
 * grid fills few of the chip's block slots split K: the slices' fp32 sums are
 * kept there and added in slice order (deterministic; same tolerance).
 * Flags: 1 non-finite input/transform, 8 non-finite bf16 operand. */
ORNITH_EXPORT hipError_t ornith_dense_g256_gemm_bf16(
    const void* input_bf16, const void* codes, const void* metadata, void* workspace, size_t workspace_bytes,
    void* output_bf16, void* flags_u32, int M, int N, int K, hipStream_t stream);

/* dense_n32/dense_g256_consumer.cpp:360-378.  N32 codes, 1<=M<=16, N%32==0, geometry==2.
 * Workspace regions as for ornith_dense_g256_launch. */
ORNITH_EXPORT hipError_t ornith_dense_g256_launch_n32(
    const void* input_bf16, const void* codes, const void* metadata, void* workspace, size_t bytes,
    void* output_bf16, void* flags_u32, int M, int Mcap, int N, int K, int bits, int transform,
    int geometry, hipStream_t stream);

/* dense_n32/dense_g256_consumer.cpp:380 (returns 16). */
ORNITH_EXPORT int ornith_dense_g256_n32_rows(void);

/* No reference counterpart: the G256 4-bit LM head of the 8192-token prefill
 * benchmark (vocabulary 151936 is outside every reference shape check).  Same
 * arithmetic as ornith_dense_g256_launch_n32 (N32 codes, K=2048), widened to
 * 1<=M<=64 and any N%32==0 up to 262144; writes fp32 logits [M,N], bf16 logits
 * [M,N] (nullable) and the top-1 index int64 [M] (numpy's argmax rule: the
 * first NaN if any, else the first maximum).  Runs on the int8 matrix cores.
 * Alignment: input 16 bytes, logits_f32 16, logits_bf16 8, argmax 8, codes 16.
 * Workspace: ornith_dense_g256_head_workspace_bytes(Mcap, N). */
ORNITH_EXPORT size_t ornith_dense_g256_head_workspace_bytes(int Mcap, int N);
ORNITH_EXPORT hipError_t ornith_dense_g256_head_launch(
    const void* input_bf16, const void* codes, const void* metadata, void* workspace, size_t bytes,
    void* logits_f32, void* logits_bf16, void* argmax_i64, void* flags_u32,
    int M, int Mcap, int N, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif
