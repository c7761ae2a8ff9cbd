// XXH3 64-bit hash with a seed, written from the published XXH3 algorithm
// (xxHash, Yann Collet, specification 0.8).  PagedBlockPool.ComputePrefixHash
// (PagedBlockPool.cs:168-172) hashes the little-endian bytes of a block's token
// ids with System.IO.Hashing.XxHash3.HashToUInt64, seeded with the parent
// block's hash; this is the same function.  The prime constants and the
// 192-byte default secret are the algorithm's own and must match it bit for
// bit.  Host code only.
#pragma once

#include <cstdint>
#include <cstring>

namespace gsp {
namespace xxh3 {

constexpr uint32_t kP32_1 = 0x9E3779B1u;
constexpr uint32_t kP32_2 = 0x85EBCA77u;
constexpr uint32_t kP32_3 = 0xC2B2AE3Du;
constexpr uint64_t kP64_1 = 0x9E3779B185EBCA87ull;
constexpr uint64_t kP64_2 = 0xC2B2AE3D27D4EB4Full;
constexpr uint64_t kP64_3 = 0x165667B19E3779F9ull;
constexpr uint64_t kP64_4 = 0x85EBCA77C2B2AE63ull;
constexpr uint64_t kP64_5 = 0x27D4EB2F165667C5ull;
constexpr uint64_t kMx1 = 0x165667919E3779F9ull;
constexpr uint64_t kMx2 = 0x9FB21C651E98DF25ull;

constexpr int kSecretSize = 192;
constexpr int kStripe = 64;
constexpr int kConsume = 8;  // secret bytes consumed per stripe

alignas(64) constexpr uint8_t kSecret[kSecretSize] = {
    0xb8, 0xfe, 0x6c, 0x39, 0x23, 0xa4, 0x4b, 0xbe, 0x7c, 0x01, 0x81, 0x2c, 0xf7, 0x21, 0xad, 0x1c,
    0xde, 0xd4, 0x6d, 0xe9, 0x83, 0x90, 0x97, 0xdb, 0x72, 0x40, 0xa4, 0xa4, 0xb7, 0xb3, 0x67, 0x1f,
    0xcb, 0x79, 0xe6, 0x4e, 0xcc, 0xc0, 0xe5, 0x78, 0x82, 0x5a, 0xd0, 0x7d, 0xcc, 0xff, 0x72, 0x21,
    0xb8, 0x08, 0x46, 0x74, 0xf7, 0x43, 0x24, 0x8e, 0xe0, 0x35, 0x90, 0xe6, 0x81, 0x3a, 0x26, 0x4c,
    0x3c, 0x28, 0x52, 0xbb, 0x91, 0xc3, 0x00, 0xcb, 0x88, 0xd0, 0x65, 0x8b, 0x1b, 0x53, 0x2e, 0xa3,
    0x71, 0x64, 0x48, 0x97, 0xa2, 0x0d, 0xf9, 0x4e, 0x38, 0x19, 0xef, 0x46, 0xa9, 0xde, 0xac, 0xd8,
    0xa8, 0xfa, 0x76, 0x3f, 0xe3, 0x9c, 0x34, 0x3f, 0xf9, 0xdc, 0xbb, 0xc7, 0xc7, 0x0b, 0x4f, 0x1d,
    0x8a, 0x51, 0xe0, 0x4b, 0xcd, 0xb4, 0x59, 0x31, 0xc8, 0x9f, 0x7e, 0xc9, 0xd9, 0x78, 0x73, 0x64,
    0xea, 0xc5, 0xac, 0x83, 0x34, 0xd3, 0xeb, 0xc3, 0xc5, 0x81, 0xa0, 0xff, 0xfa, 0x13, 0x63, 0xeb,
    0x17, 0x0d, 0xdd, 0x51, 0xb7, 0xf0, 0xda, 0x49, 0xd3, 0x16, 0x55, 0x26, 0x29, 0xd4, 0x68, 0x9e,
    0x2b, 0x16, 0xbe, 0x58, 0x7d, 0x47, 0xa1, 0xfc, 0x8f, 0xf8, 0xb8, 0xd1, 0x7a, 0xd0, 0x31, 0xce,
    0x45, 0xcb, 0x3a, 0x8f, 0x95, 0x16, 0x04, 0x28, 0xaf, 0xd7, 0xfb, 0xca, 0xbb, 0x4b, 0x40, 0x7e,
};

inline uint64_t rd64(const uint8_t* p) {
    uint64_t v;
    std::memcpy(&v, p, 8);  // x86-64 and gfx hosts are little-endian
    return v;
}
inline uint32_t rd32(const uint8_t* p) {
    uint32_t v;
    std::memcpy(&v, p, 4);
    return v;
}
inline void wr64(uint8_t* p, uint64_t v) { std::memcpy(p, &v, 8); }
inline uint64_t rotl64(uint64_t x, int r) { return (x << r) | (x >> (64 - r)); }
inline uint64_t swap64(uint64_t x) { return __builtin_bswap64(x); }
inline uint32_t swap32(uint32_t x) { return __builtin_bswap32(x); }

// Low and high halves of the 128-bit product, xor-folded.
inline uint64_t mul_fold(uint64_t a, uint64_t b) {
    const unsigned __int128 p = (unsigned __int128)a * b;
    return (uint64_t)p ^ (uint64_t)(p >> 64);
}

inline uint64_t avalanche64(uint64_t h) {  // the XXH64 finaliser
    h ^= h >> 33;
    h *= kP64_2;
    h ^= h >> 29;
    h *= kP64_3;
    h ^= h >> 32;
    return h;
}

inline uint64_t avalanche3(uint64_t h) {
    h ^= h >> 37;
    h *= kMx1;
    h ^= h >> 32;
    return h;
}

inline uint64_t rrmxmx(uint64_t h, uint64_t len) {
    h ^= rotl64(h, 49) ^ rotl64(h, 24);
    h *= kMx2;
    h ^= (h >> 35) + len;
    h *= kMx2;
    h ^= h >> 28;
    return h;
}

inline uint64_t mix16(const uint8_t* in, const uint8_t* sec, uint64_t seed) {
    return mul_fold(rd64(in) ^ (rd64(sec) + seed), rd64(in + 8) ^ (rd64(sec + 8) - seed));
}

inline uint64_t len_0to16(const uint8_t* in, size_t len, uint64_t seed) {
    const uint8_t* s = kSecret;
    if (len > 8) {
        const uint64_t flip1 = (rd64(s + 24) ^ rd64(s + 32)) + seed;
        const uint64_t flip2 = (rd64(s + 40) ^ rd64(s + 48)) - seed;
        const uint64_t lo = rd64(in) ^ flip1;
        const uint64_t hi = rd64(in + len - 8) ^ flip2;
        return avalanche3(len + swap64(lo) + hi + mul_fold(lo, hi));
    }
    if (len >= 4) {
        seed ^= (uint64_t)swap32((uint32_t)seed) << 32;
        const uint32_t a = rd32(in), b = rd32(in + len - 4);
        const uint64_t flip = (rd64(s + 8) ^ rd64(s + 16)) - seed;
        return rrmxmx(((uint64_t)b + ((uint64_t)a << 32)) ^ flip, len);
    }
    if (len > 0) {
        const uint32_t c1 = in[0], c2 = in[len >> 1], c3 = in[len - 1];
        const uint32_t combined = (c1 << 16) | (c2 << 24) | c3 | ((uint32_t)len << 8);
        const uint64_t flip = (uint64_t)(rd32(s) ^ rd32(s + 4)) + seed;
        return avalanche64((uint64_t)combined ^ flip);
    }
    return avalanche64(seed ^ (rd64(s + 56) ^ rd64(s + 64)));
}

inline uint64_t len_17to128(const uint8_t* in, size_t len, uint64_t seed) {
    const uint8_t* s = kSecret;
    uint64_t acc = len * kP64_1;
    if (len > 32) {
        if (len > 64) {
            if (len > 96) {
                acc += mix16(in + 48, s + 96, seed);
                acc += mix16(in + len - 64, s + 112, seed);
            }
            acc += mix16(in + 32, s + 64, seed);
            acc += mix16(in + len - 48, s + 80, seed);
        }
        acc += mix16(in + 16, s + 32, seed);
        acc += mix16(in + len - 32, s + 48, seed);
    }
    acc += mix16(in, s, seed);
    acc += mix16(in + len - 16, s + 16, seed);
    return avalanche3(acc);
}

inline uint64_t len_129to240(const uint8_t* in, size_t len, uint64_t seed) {
    const uint8_t* s = kSecret;
    constexpr int kStartOffset = 3, kLastOffset = 17, kSecretMin = 136;
    uint64_t acc = len * kP64_1;
    const int rounds = (int)(len / 16);
    for (int i = 0; i < 8; ++i) acc += mix16(in + 16 * i, s + 16 * i, seed);
    acc = avalanche3(acc);
    for (int i = 8; i < rounds; ++i) acc += mix16(in + 16 * i, s + 16 * (i - 8) + kStartOffset, seed);
    acc += mix16(in + len - 16, s + kSecretMin - kLastOffset, seed);
    return avalanche3(acc);
}

inline void accumulate_stripe(uint64_t acc[8], const uint8_t* in, const uint8_t* sec) {
    for (int i = 0; i < 8; ++i) {
        const uint64_t v = rd64(in + 8 * i);
        const uint64_t k = v ^ rd64(sec + 8 * i);
        acc[i ^ 1] += v;
        acc[i] += (uint64_t)(uint32_t)k * (k >> 32);
    }
}

inline void scramble(uint64_t acc[8], const uint8_t* sec) {
    for (int i = 0; i < 8; ++i) {
        uint64_t a = acc[i];
        a ^= a >> 47;
        a ^= rd64(sec + 8 * i);
        a *= kP32_1;
        acc[i] = a;
    }
}

inline uint64_t hash_long(const uint8_t* in, size_t len, const uint8_t* sec) {
    constexpr int kLastAccStart = 7, kMergeStart = 11;
    uint64_t acc[8] = {kP32_3, kP64_1, kP64_2, kP64_3, kP64_4, kP32_2, kP64_5, kP32_1};
    const size_t stripes_per_block = (kSecretSize - kStripe) / kConsume;
    const size_t block_len = kStripe * stripes_per_block;
    const size_t blocks = (len - 1) / block_len;
    for (size_t b = 0; b < blocks; ++b) {
        for (size_t n = 0; n < stripes_per_block; ++n)
            accumulate_stripe(acc, in + b * block_len + n * kStripe, sec + n * kConsume);
        scramble(acc, sec + kSecretSize - kStripe);
    }
    const size_t stripes = ((len - 1) - block_len * blocks) / kStripe;
    for (size_t n = 0; n < stripes; ++n) accumulate_stripe(acc, in + blocks * block_len + n * kStripe, sec + n * kConsume);
    accumulate_stripe(acc, in + len - kStripe, sec + kSecretSize - kStripe - kLastAccStart);
    uint64_t h = len * kP64_1;
    for (int i = 0; i < 4; ++i)
        h += mul_fold(acc[2 * i] ^ rd64(sec + kMergeStart + 16 * i), acc[2 * i + 1] ^ rd64(sec + kMergeStart + 16 * i + 8));
    return avalanche3(h);
}

// XXH3_64bits_withSeed(data, len, seed).
inline uint64_t hash64(const void* data, size_t len, uint64_t seed) {
    const uint8_t* in = static_cast<const uint8_t*>(data);
    if (len <= 16) return len_0to16(in, len, seed);
    if (len <= 128) return len_17to128(in, len, seed);
    if (len <= 240) return len_129to240(in, len, seed);
    if (seed == 0) return hash_long(in, len, kSecret);
    alignas(64) uint8_t custom[kSecretSize];  // the default secret with the seed folded in
    for (int i = 0; i < kSecretSize / 16; ++i) {
        wr64(custom + 16 * i, rd64(kSecret + 16 * i) + seed);
        wr64(custom + 16 * i + 8, rd64(kSecret + 16 * i + 8) - seed);
    }
    return hash_long(in, len, custom);
}

}  // namespace xxh3
}  // namespace gsp
