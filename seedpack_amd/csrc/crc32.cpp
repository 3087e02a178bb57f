// CRC-32 as zlib computes it (polynomial 0x04C11DB7 bit-reflected, initial and final value ~0) on the
// host, for the container's chunk checksums. Blocks of 16 bytes are folded with carry-less
// multiplication (PCLMULQDQ; the folding method of Gopal et al., "Fast CRC Computation for Generic
// Polynomials Using PCLMULQDQ Instruction", Intel, 2009): sixteen 128-bit accumulators in four
// 512-bit registers (VPCLMULQDQ) over the bulk where the CPU has it, then four 128-bit accumulators
// 64 bytes apart, combined into one, whose CRC and the tail bytes' are taken a byte at a time from a
// table.
//
// A 128-bit register holds 128 message bits in order (bit k = message bit k, least significant bit of
// each byte first), i.e. a polynomial R with bit k the coefficient of x^(127-k); its low quadword H
// holds the high-degree half, so R = H x^64 + L. Moving R by D bits, R x^D = H x^(D+64) + L x^D, is
// congruent mod P to H (x^(D+63) mod P) x + L (x^(D-1) mod P) x, and the carry-less product of two
// such bit-reflected operands carries exactly that extra factor x. The constants are computed from
// the polynomial when the library loads.
#include <immintrin.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#include "../../include/seedpack_amd.h"

namespace {

constexpr uint64_t kPoly = 0x104C11DB7ull;   // x^32 + ... + 1, bit d = coefficient of x^d

uint32_t xpow_mod(unsigned k) {              // x^k mod P, same bit order
    uint64_t r = 1;
    for (unsigned i = 0; i < k; ++i) {
        r <<= 1;
        if (r >> 32) r ^= kPoly;
    }
    return (uint32_t)r;
}

uint64_t reflect64(uint32_t v) {             // coefficient of x^d at bit 63 - d
    uint64_t out = 0;
    for (int d = 0; d < 32; ++d)
        if (v >> d & 1) out |= 1ull << (63 - d);
    return out;
}

struct Tables {
    uint32_t byte[256];
    uint64_t k512[2], k384[2], k256[2], k128[2];   // {for H, for L} of a move by 512, 384, 256, 128 bits
    uint64_t k2048[2];                              // the same for 2048 bits (four 512-bit registers)
    bool clmul, wide;
    Tables() {
        for (uint32_t i = 0; i < 256; ++i) {
            uint32_t c = i;
            for (int j = 0; j < 8; ++j) c = (c & 1) ? (c >> 1) ^ 0xEDB88320u : c >> 1;
            byte[i] = c;
        }
        const unsigned D[4] = {512, 384, 256, 128};
        uint64_t* K[4] = {k512, k384, k256, k128};
        for (int i = 0; i < 4; ++i) {
            K[i][0] = reflect64(xpow_mod(D[i] + 63));
            K[i][1] = reflect64(xpow_mod(D[i] - 1));
        }
        k2048[0] = reflect64(xpow_mod(2048 + 63));
        k2048[1] = reflect64(xpow_mod(2048 - 1));
        __builtin_cpu_init();
        clmul = __builtin_cpu_supports("pclmul") && __builtin_cpu_supports("sse4.1");
        wide = clmul && __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("vpclmulqdq");
    }
};

const Tables& tables() {
    static const Tables t;
    return t;
}

// the raw register (no inversions) over n bytes, a byte at a time
uint32_t by_table(uint32_t s, const uint8_t* p, size_t n, const uint32_t* T) {
    for (size_t i = 0; i < n; ++i) s = T[(s ^ p[i]) & 0xFF] ^ (s >> 8);
    return s;
}

__attribute__((target("pclmul,sse4.1"))) inline __m128i move(__m128i r, __m128i k) {
    return _mm_xor_si128(_mm_clmulepi64_si128(r, k, 0x00), _mm_clmulepi64_si128(r, k, 0x11));
}

// the raw register after n >= 64 bytes, starting from register s
__attribute__((target("pclmul,sse4.1"))) uint32_t by_folding(uint32_t s, const uint8_t* p, size_t n, const Tables& T) {
    auto ld = [](const uint8_t* q) { return _mm_loadu_si128(reinterpret_cast<const __m128i*>(q)); };
    auto kk = [](const uint64_t* k) { return _mm_set_epi64x((long long)k[1], (long long)k[0]); };
    __m128i x0 = _mm_xor_si128(ld(p), _mm_cvtsi32_si128((int)s)), x1 = ld(p + 16), x2 = ld(p + 32), x3 = ld(p + 48);
    size_t at = 64;
    const __m128i k512 = kk(T.k512);
    for (; n - at >= 64; at += 64) {
        x0 = _mm_xor_si128(move(x0, k512), ld(p + at));
        x1 = _mm_xor_si128(move(x1, k512), ld(p + at + 16));
        x2 = _mm_xor_si128(move(x2, k512), ld(p + at + 32));
        x3 = _mm_xor_si128(move(x3, k512), ld(p + at + 48));
    }
    const __m128i k128 = kk(T.k128);
    __m128i x = _mm_xor_si128(_mm_xor_si128(move(x0, kk(T.k384)), move(x1, kk(T.k256))),
                              _mm_xor_si128(move(x2, k128), x3));
    for (; n - at >= 16; at += 16) x = _mm_xor_si128(move(x, k128), ld(p + at));
    uint8_t last[16];
    _mm_storeu_si128(reinterpret_cast<__m128i*>(last), x);
    return by_table(by_table(0, last, 16, T.byte), p + at, n - at, T.byte);
}

#define SPA_WIDE __attribute__((target("avx512f,vpclmulqdq,pclmul,sse4.1")))

SPA_WIDE inline __m512i ld512(const uint8_t* q) { return _mm512_loadu_si512(reinterpret_cast<const void*>(q)); }

SPA_WIDE inline __m512i move512(__m512i r, __m512i k) {
    return _mm512_xor_si512(_mm512_clmulepi64_epi128(r, k, 0x00), _mm512_clmulepi64_epi128(r, k, 0x11));
}

// the raw register after the largest multiple of 256 bytes (n >= 512) of p, from register s: four
// 512-bit registers, each four 128-bit accumulators, folded 2048 bits at a time with VPCLMULQDQ; their
// 16 accumulators (256 bytes, in message order) are then taken by the 128-bit path; `used` = the bytes
SPA_WIDE uint32_t by_folding512(uint32_t s, const uint8_t* p, size_t n, size_t& used, const Tables& T) {
    const __m512i k = _mm512_set_epi64((long long)T.k2048[1], (long long)T.k2048[0], (long long)T.k2048[1],
                                       (long long)T.k2048[0], (long long)T.k2048[1], (long long)T.k2048[0],
                                       (long long)T.k2048[1], (long long)T.k2048[0]);
    __m512i x0 = _mm512_xor_si512(ld512(p), _mm512_castsi128_si512(_mm_cvtsi32_si128((int)s)));
    __m512i x1 = ld512(p + 64), x2 = ld512(p + 128), x3 = ld512(p + 192);
    size_t at = 256;
    for (; n - at >= 256; at += 256) {
        x0 = _mm512_xor_si512(move512(x0, k), ld512(p + at));
        x1 = _mm512_xor_si512(move512(x1, k), ld512(p + at + 64));
        x2 = _mm512_xor_si512(move512(x2, k), ld512(p + at + 128));
        x3 = _mm512_xor_si512(move512(x3, k), ld512(p + at + 192));
    }
    alignas(64) uint8_t acc[256];
    _mm512_store_si512(reinterpret_cast<void*>(acc), x0);
    _mm512_store_si512(reinterpret_cast<void*>(acc + 64), x1);
    _mm512_store_si512(reinterpret_cast<void*>(acc + 128), x2);
    _mm512_store_si512(reinterpret_cast<void*>(acc + 192), x3);
    used = at;
    return by_folding(0, acc, 256, T);
}

}  // namespace

extern "C" uint32_t spa_crc32(uint32_t crc, const void* data, size_t n) {
    const Tables& T = tables();
    const uint8_t* p = static_cast<const uint8_t*>(data);
    if (!p || n == 0) return crc;
    uint32_t s = ~crc;
    if (n >= 512 && T.wide) {
        size_t used = 0;
        s = by_folding512(s, p, n, used, T);
        p += used;
        n -= used;
    }
    return ~(n >= 64 && T.clmul ? by_folding(s, p, n, T) : by_table(s, p, n, T.byte));
}
