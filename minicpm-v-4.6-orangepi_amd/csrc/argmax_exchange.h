// argmax_exchange.h -- the device-token lm_head's cross-workgroup argmax,
// shared by the W4A16 and W8A8 lm_head kernels (w4a16_gemv.hip,
// w8a8_tiled.hip).
#pragma once

#include "common.h"

namespace mcv {

// Cross-workgroup argmax without fences or counters (the L2s of the eight
// XCDs are not coherent with each other).  Every workgroup publishes its best
// key as one call-tagged 64-bit word (bits 63..40 tag, 39..24 the fp16 key,
// 23..0 the complement of the column index) with a device-scope store, which
// goes through to the coherent point; the grid's last workgroup polls all the
// words with device-scope loads until each carries this call's tag, takes
// the maximum and writes the token -- one store's visibility plus one poll
// after the last workgroup.  The tag comes from the workspace's generation
// word: every workgroup reads it at its start, and the poller advances it
// once it has seen every key of the call (so no workgroup of the call can
// still be about to read it).  The next call is stream-ordered after this
// kernel and reads the advanced value; a graph replay reads it afresh from
// device memory.  The key words sit at a fixed offset whatever the grid, so
// calls over different V may share one workspace (one at a time).
// Workspace (zero-filled once): u32 give-up flag at word 0, u32 generation
// at word 1, the u64 keys from byte kLmKeysByte, one per workgroup.
// Measured on MI355X with the lm_head's workgroups: 3877 atomics on one
// address serialise to 45 us, a __threadfence per workgroup adds ~30 us,
// CAS-combined (key, count) words 22-39 us, and the fence-free 64-slot
// arrival tree this replaces (atomicMax, then slot and global counts, then a
// read of the slot maxima) ~1.8 us: four device round trips.
constexpr int kLmGen = 1;                                     // u32 index of the generation word
constexpr int kLmKeysByte = 128;                              // byte offset of the key words
constexpr int kLmPollVec = 8;                                 // key words per lane per poll
constexpr int kLmSpinLimit = 1 << 18;

// The call's tag from a generation: 1 .. 2^24 - 1 (a zero-filled key, tag 0,
// never matches).
__device__ __forceinline__ unsigned long long lm_tag(unsigned gen) { return (gen % 0xffffffu) + 1u; }

// Run by one full wave of each workgroup after its columns are final; `key`
// is the workgroup's best argmax_key64 (wave-uniform), `gen` the generation
// word as read at the start of the kernel.  `skew` is 0 except under
// mcv_testing_lm_head_skew_poll, where the poller expects a tag no key
// carries, so its bounded wait gives up (the give-up path's test).
__device__ __forceinline__ void argmax_publish(unsigned long long* __restrict__ ws, unsigned long long key,
                                               unsigned gen, unsigned skew, int b, int nblk, int lane,
                                               int64_t* __restrict__ token, unsigned* status) {
    unsigned* ws32 = reinterpret_cast<unsigned*>(ws);
    unsigned long long* keys = ws + kLmKeysByte / 8;
    const unsigned long long tag = lm_tag(gen);
    const unsigned long long want = (tag + skew) & 0xffffffull;
    if (lane == 0) {
        const unsigned long long k16 = key >> 32, idx = key & 0xffffffull;
        __hip_atomic_store(keys + b, (tag << 40) | (k16 << 24) | (k16 ? idx : 0ull), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
    if (b != nblk - 1) return;
    unsigned long long best = 0ull;
    bool gave_up = false;
    for (int base = 0; base < nblk; base += 64 * kLmPollVec) {
        unsigned long long v[kLmPollVec];
        for (int spins = 0;; ++spins) {
#pragma unroll
            for (int i = 0; i < kLmPollVec; ++i) {
                const int j = base + lane + 64 * i;
                v[i] = __hip_atomic_load(keys + (j < nblk ? j : b), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            unsigned long long bad = 0;
#pragma unroll
            for (int i = 0; i < kLmPollVec; ++i) bad |= (v[i] >> 40) ^ want;
            if (__all(bad == 0)) break;
            if (spins > kLmSpinLimit) {
                if (lane == 0) flag_gave_up(ws32, status);
                gave_up = true;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
#pragma unroll
        for (int i = 0; i < kLmPollVec; ++i) {
            const unsigned long long k = v[i] & 0xffffffffffull;
            best = k > best ? k : best;
        }
    }
    best = wave_max_u64(best);
    if (lane == 0) {
        // -1: the keys of this call never all arrived, so no token is known
        *token = gave_up ? int64_t(-1)
                 : (best >> 24) ? static_cast<int64_t>(0xffffffu - static_cast<uint32_t>(best & 0xffffffu)) : 0;
        // the next call's tag (also after a give-up: this call's late keys
        // then carry a tag the next call does not accept)
        __hip_atomic_store(ws32 + kLmGen, gen + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

}  // namespace mcv
