// Tagged hand-off words between blocks of one launch: a 64-bit word holds
// (tag << 32) | value bits and is written and read with one relaxed
// agent-scope atomic access (these bypass the non-coherent caches).  The tag
// hashes the call's sequence number (one per workspace, advanced once per
// call after every block has read it) with the word's index, so a reader
// knows a word belongs to this call once its tag matches, and words of
// earlier calls or other data never match.  Every wait is bounded.
#pragma once
#include "common.hpp"

namespace ornith {

__device__ __forceinline__ uint32_t l1_tag(uint32_t seq, uint32_t idx) {
    uint32_t h = seq * 0x9E3779B9u ^ (idx + 0x7F4A7C15u) * 0x85EBCA77u;
    h ^= h >> 16;
    h *= 0x7FEB352Du;
    h ^= h >> 15;
    h *= 0x846CA68Bu;
    h ^= h >> 16;
    return h;
}
__device__ __forceinline__ void l1_put(uint64_t* w, uint32_t idx, uint32_t seq, uint32_t bits) {
    __hip_atomic_store(w + idx, (uint64_t(l1_tag(seq, idx)) << 32) | bits, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t l1_get(uint64_t* w, uint32_t idx) {
    return __hip_atomic_load(w + idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
constexpr int kHandoffSpins = 1 << 15;      // default poll rounds before a wait gives up
// Sequence value that marks a workspace whose last call could not confirm
// that every block had read its sequence number (an arrival wait gave up):
// words of that call may still be published under a tag a later call would
// accept.  A call that reads it gives up every wait at once (raising the
// time-out flag) and leaves the mark; zeroing the workspace clears it.  The
// running number skips this value.
constexpr uint32_t kSeqPoisoned = 0xFFFFFFFFu;
__device__ __forceinline__ uint32_t l1_next_seq(uint32_t seq) { return seq + 1 == kSeqPoisoned ? 0u : seq + 1; }
// Poll rounds of this call's waits: `spins` (the host's setting), or 0 on a
// poisoned workspace.
__device__ __forceinline__ int l1_limit(uint32_t seq, int spins) { return seq == kSeqPoisoned ? 0 : spins; }
// Waits until this wave's N words idx[] carry this call's tags; val[] gets
// their value bits.  One round of N loads at a time, all issued before any is
// checked; PAUSE (s_sleep units of 64 clocks) between rounds.  Wave-uniform.
// At most `limit` rounds, then false; limit 0 reads the words once and
// reports a time-out whatever they hold (val[] is always assigned).
template <int N, int PAUSE>
__device__ __forceinline__ bool l1_wait(uint64_t* w, const uint32_t (&idx)[N], uint32_t seq, uint32_t (&val)[N],
                                        int limit) {
    uint32_t want[N];
#pragma unroll
    for (int i = 0; i < N; ++i) want[i] = l1_tag(seq, idx[i]);
    for (int spin = 0;; ++spin) {
        uint64_t r[N];
#pragma unroll
        for (int i = 0; i < N; ++i) r[i] = l1_get(w, idx[i]);
        bool ok = true;
#pragma unroll
        for (int i = 0; i < N; ++i) {
            val[i] = uint32_t(r[i]);
            ok = ok && uint32_t(r[i] >> 32) == want[i];
        }
        if (limit > 0 && __builtin_amdgcn_ballot_w64(!ok) == 0) return true;
        if (spin + 1 >= limit) return false;
        if (PAUSE) __builtin_amdgcn_s_sleep(PAUSE);
    }
}

}  // namespace ornith
