// SHA-256 as FIPS 180-4 specifies it, for per-layer checkpoint hashes: the
// compression function in plain C, and with the x86 SHA extensions where the
// host CPU has them (the instruction sequence of Intel's SHA extensions
// reference: state kept as ABEF/CDGH, four rounds per two sha256rnds2, the
// message schedule by sha256msg1/msg2).
#include <immintrin.h>

#include <cstring>

#include "runtime_internal.h"

namespace {

const uint32_t K[64] = {
    0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
    0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
    0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
    0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
    0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
    0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
    0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
    0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};

inline uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

void compress(uint32_t h[8], const uint8_t* p) {
    uint32_t w[64];
    for (int i = 0; i < 16; i++)
        w[i] = ((uint32_t)p[4 * i] << 24) | ((uint32_t)p[4 * i + 1] << 16) | ((uint32_t)p[4 * i + 2] << 8) | p[4 * i + 3];
    for (int i = 16; i < 64; i++) {
        uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
        uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
        w[i] = w[i - 16] + s0 + w[i - 7] + s1;
    }
    uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
    for (int i = 0; i < 64; i++) {
        uint32_t S1 = rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25);
        uint32_t ch = (e & f) ^ (~e & g);
        uint32_t t1 = hh + S1 + ch + K[i] + w[i];
        uint32_t S0 = rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22);
        uint32_t mj = (a & b) ^ (a & c) ^ (b & c);
        uint32_t t2 = S0 + mj;
        hh = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
    }
    h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
}

__attribute__((target("sha,sse4.1,ssse3"))) void compress_sha_ext(uint32_t h[8], const uint8_t* p, size_t blocks) {
    const __m128i bswap = _mm_set_epi64x(0x0c0d0e0f08090a0bULL, 0x0405060700010203ULL);
    __m128i tmp = _mm_shuffle_epi32(_mm_loadu_si128((const __m128i*)&h[0]), 0xB1);  // CDAB
    __m128i st1 = _mm_shuffle_epi32(_mm_loadu_si128((const __m128i*)&h[4]), 0x1B);  // EFGH
    __m128i st0 = _mm_alignr_epi8(tmp, st1, 8);                                       // ABEF
    st1 = _mm_blend_epi16(st1, tmp, 0xF0);                                            // CDGH
    for (; blocks; blocks--, p += 64) {
        const __m128i save0 = st0, save1 = st1;
        __m128i x[16];
        for (int j = 0; j < 4; j++) x[j] = _mm_shuffle_epi8(_mm_loadu_si128((const __m128i*)(p + 16 * j)), bswap);
        for (int j = 4; j < 16; j++)
            x[j] = _mm_sha256msg2_epu32(
                _mm_add_epi32(_mm_sha256msg1_epu32(x[j - 4], x[j - 3]), _mm_alignr_epi8(x[j - 1], x[j - 2], 4)),
                x[j - 1]);
        for (int j = 0; j < 16; j++) {
            __m128i msg = _mm_add_epi32(x[j], _mm_loadu_si128((const __m128i*)&K[4 * j]));
            st1 = _mm_sha256rnds2_epu32(st1, st0, msg);
            msg = _mm_shuffle_epi32(msg, 0x0E);
            st0 = _mm_sha256rnds2_epu32(st0, st1, msg);
        }
        st0 = _mm_add_epi32(st0, save0);
        st1 = _mm_add_epi32(st1, save1);
    }
    tmp = _mm_shuffle_epi32(st0, 0x1B);      // FEBA
    st1 = _mm_shuffle_epi32(st1, 0xB1);      // DCHG
    st0 = _mm_blend_epi16(tmp, st1, 0xF0);   // DCBA
    st1 = _mm_alignr_epi8(st1, tmp, 8);      // HGFE
    _mm_storeu_si128((__m128i*)&h[0], st0);
    _mm_storeu_si128((__m128i*)&h[4], st1);
}

bool have_sha_ext() {
    static const bool yes = __builtin_cpu_supports("sha");
    return yes;
}

void compress_blocks(uint32_t h[8], const uint8_t* p, size_t blocks) {
    if (have_sha_ext()) {
        compress_sha_ext(h, p, blocks);
        return;
    }
    for (; blocks; blocks--, p += 64) compress(h, p);
}

}  // namespace

void iris_sha256(const uint8_t* data, size_t len, uint8_t out[32]) {
    uint32_t h[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a, 0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    const size_t i = len / 64 * 64;
    compress_blocks(h, data, len / 64);
    uint8_t tail[128] = {0};
    const size_t rem = len - i;
    std::memcpy(tail, data + i, rem);
    tail[rem] = 0x80;
    const size_t tl = rem + 9 <= 64 ? 64 : 128;
    const uint64_t bits = (uint64_t)len * 8;
    for (int k = 0; k < 8; k++) tail[tl - 1 - k] = (uint8_t)(bits >> (8 * k));
    compress_blocks(h, tail, tl / 64);
    for (int k = 0; k < 8; k++) {
        out[4 * k] = (uint8_t)(h[k] >> 24);
        out[4 * k + 1] = (uint8_t)(h[k] >> 16);
        out[4 * k + 2] = (uint8_t)(h[k] >> 8);
        out[4 * k + 3] = (uint8_t)h[k];
    }
}

extern "C" int iris_sha256_bytes(const uint8_t* data, uint64_t len, uint8_t* out) {
    if (!out || (!data && len)) return -1;
    iris_sha256(data, (size_t)len, out);
    return 0;
}
