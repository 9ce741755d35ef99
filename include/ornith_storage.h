/* Storage conversion C ABI of the MI355X (gfx950) Ornith library.
 *
 * The reference converts N16 checkpoint banks to the N32 tile order with a
 * torch permute on the GPU, once at start-up
 * (plugin-site/ornith_g256/method.py:124-158 for routed experts,
 * dense_n32.py:32-33 for dense banks); it has no C entry for it.  This entry
 * does the same conversion with a HIP kernel.
 */
#ifndef ORNITH_MI355X_STORAGE_H
#define ORNITH_MI355X_STORAGE_H
#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>
#ifdef __cplusplus
extern "C" {
#endif
#ifndef ORNITH_EXPORT
#define ORNITH_EXPORT __attribute__((visibility("default")))
#endif

/* method.py:143-147.  `banks` consecutive banks of N x K 4-bit weights:
 *   codes16 uint32 [banks, N/16, K/256, 32, 16] -> codes32 [banks, N/32, K/256, 32, 32]
 *   meta16  uint32 [banks, N/16, K/256, 16]     -> meta32  [banks, N/32, K/256, 32]
 * (32-column tile t = 16-column tiles 2t then 2t+1).  N % 32 == 0, K % 256 == 0;
 * all four buffers 16-byte aligned; the outputs must not overlap anything.
 * banks, N or K == 0 returns hipSuccess without touching memory. */
ORNITH_EXPORT hipError_t ornith_repack_n16_to_n32(const void* codes16, const void* meta16, void* codes32,
                                                  void* meta32, int banks, int N, int K, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif
