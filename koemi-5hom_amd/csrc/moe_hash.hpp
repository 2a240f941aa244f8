// The content hash of the MoE hash route (model/experts.py:30-38, 283-289),
// shared by the route kernel and the permutation that routes pairs itself.
#pragma once

#include <cstdint>

namespace koemi {

// mix32 of experts.py:30-38. The product tok * 1000003 + prev * 97409 is taken
// modulo 2^64 (the int64 tensor arithmetic of the reference) and only its low
// 32 bits are used, so unsigned 64-bit arithmetic gives the same bits.
__device__ __forceinline__ uint32_t content_hash(int64_t token, int64_t previous) {
    const uint64_t mixed = static_cast<uint64_t>(token) * 1000003ull + static_cast<uint64_t>(previous) * 97409ull;
    uint32_t v = static_cast<uint32_t>(mixed);
    v ^= v >> 16;
    v *= 0x45D9F3Bu;
    v ^= v >> 16;
    v *= 0x45D9F3Bu;
    return v ^ (v >> 16);
}

// Expert of slot s for hash h (experts.py:288): the int64 sum h + s * 0x9E3779B9
// (no 32-bit wraparound: h < 2^32, s * 0x9E3779B9 < 2^40) modulo E.
__device__ __forceinline__ int64_t hash_slot_expert(uint64_t h, int64_t s, int64_t E) {
    return static_cast<int64_t>((h + static_cast<uint64_t>(s) * 0x9E3779B9ull) % static_cast<uint64_t>(E));
}

}  // namespace koemi
