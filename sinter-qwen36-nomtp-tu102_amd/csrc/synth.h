// Deterministic synthetic tensors, identical bytes on host and device.
//
// Random bits come from a counter-based SplitMix64 hash of (tensor seed,
// element index); floats are formed with exactly rounded fp32 operations
// (int->float conversion, one multiply, one add) and f16/bf16 conversions
// round to nearest even, so the host build (g++, -ffp-contract=off) and the
// gfx950 build produce the same bits.  "Normal" values use an Irwin-Hall(4)
// sum of 16-bit uniforms scaled to unit variance: bounded at +-3.46 sigma,
// which is adequate for random-init weights, caches and states.
#pragma once
#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define SX_HD __host__ __device__
#else
#define SX_HD
#endif

namespace sinter {

SX_HD inline uint64_t sx_mix(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
SX_HD inline uint64_t sx_u64(uint64_t seed, uint64_t idx) { return sx_mix(seed ^ sx_mix(idx)); }

// ~N(0,1): (sum of four U{0..65535} - 131070) / sqrt(4 * (65536^2 - 1) / 12)
SX_HD inline float sx_normal(uint64_t seed, uint64_t idx) {
    const uint64_t u = sx_u64(seed, idx);
    const int32_t s = (int32_t)(u & 0xffff) + (int32_t)((u >> 16) & 0xffff) +
                      (int32_t)((u >> 32) & 0xffff) + (int32_t)(u >> 48) - 131070;
    return (float)s * 2.64289234e-05f;
}
// U[0,1) with 24 random bits (exact)
SX_HD inline float sx_unit(uint64_t seed, uint64_t idx) {
    return (float)(uint32_t)(sx_u64(seed, idx) >> 40) * 5.9604644775390625e-08f;
}

// f32 -> f16 bits, round to nearest even (software; same result as
// __float2half_rn)
SX_HD inline uint16_t sx_f2h(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return sign | 0x7c00 | (ax > 0x7f800000u ? 0x200 : 0);
    if (ax >= 0x477ff000u) return sign | 0x7c00;
    if (ax < 0x38800000u) {
        // subnormal: value * 2^24, rounded half to even, done in integers
        const uint32_t e = ax >> 23;             // biased exponent, < 113
        if (e < 102) return sign;                // below half the smallest subnormal
        const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        const uint32_t sh = 126 - e;             // value*2^24 = m >> sh
        const uint32_t q = m >> sh, rem = m & ((1u << sh) - 1), half = 1u << (sh - 1);
        const uint32_t r = (rem > half || (rem == half && (q & 1u))) ? q + 1 : q;
        return sign | (uint16_t)r;
    }
    const uint32_t mant = ax + 0xfffu + ((ax >> 13) & 1u);
    return sign | (uint16_t)((mant - 0x38000000u) >> 13);
}
SX_HD inline uint16_t sx_f2bf(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 64);
    return (uint16_t)((u + (0x7fffu + ((u >> 16) & 1u))) >> 16);
}

// ----------------------------------------------------------------- blocks
// Each generator writes one 256-element group of a weight row (block index b
// counts groups over the whole tensor).  Target: dequantised values with
// mean ~0 and standard deviation ~0.02.

// Q4_K: codes U{0..15}, sub-block scales U{32..63}, mins U{0..63},
// d ~ 9.13e-5 * U(0.8,1.2), dmin ~ 1.03e-3 * U(0.8,1.2).
SX_HD inline void sx_q4k_block(uint64_t seed, uint64_t b, uint8_t *out /*144*/) {
    const uint64_t base = b * 32;
    const uint64_t us = sx_u64(seed, base + 16), um = sx_u64(seed, base + 17);
    int sc[8], mn[8];
    for (int j = 0; j < 8; j++) {
        sc[j] = 32 + (int)((us >> (5 * j)) & 31);
        mn[j] = (int)((um >> (6 * j)) & 63);
    }
    const float d = 9.13e-05f * (0.8f + 0.4f * sx_unit(seed, base + 18));
    const float dm = 1.03e-03f * (0.8f + 0.4f * sx_unit(seed, base + 19));
    const uint16_t dh = sx_f2h(d), dmh = sx_f2h(dm);
    out[0] = (uint8_t)(dh & 0xff); out[1] = (uint8_t)(dh >> 8);
    out[2] = (uint8_t)(dmh & 0xff); out[3] = (uint8_t)(dmh >> 8);
    uint8_t *q = out + 4;
    for (int j = 0; j < 4; j++) {
        q[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        q[j + 4] = (uint8_t)((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
        q[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4));
    }
    for (int i = 0; i < 16; i++) {
        const uint64_t u = sx_u64(seed, base + (uint64_t)i);
        for (int k = 0; k < 8; k++) out[16 + 8 * i + k] = (uint8_t)(u >> (8 * k));
    }
}

// Q6_K: codes U{0..63} (stored value q-32), int8 scales U{-127..127},
// d ~ 1.48e-5 * U(0.8,1.2) (an f16 subnormal, as real Q6_K tensors have).
SX_HD inline void sx_q6k_block(uint64_t seed, uint64_t b, uint8_t *out /*210*/) {
    const uint64_t base = b * 32;
    for (int i = 0; i < 24; i++) {  // ql[128] + qh[64] = 192 random bytes
        const uint64_t u = sx_u64(seed, base + (uint64_t)i);
        for (int k = 0; k < 8; k++) out[8 * i + k] = (uint8_t)(u >> (8 * k));
    }
    for (int j = 0; j < 16; j++) {  // 16 random bits per scale: U{-127..127}
        const uint32_t r = (uint32_t)((sx_u64(seed, base + 24 + (uint64_t)(j >> 2)) >> (16 * (j & 3))) & 0xffff);
        out[192 + j] = (uint8_t)(int8_t)((int)((r * 255u) >> 16) - 127);
    }
    const float d = 1.48e-05f * (0.8f + 0.4f * sx_unit(seed, base + 28));
    const uint16_t dh = sx_f2h(d);
    out[208] = (uint8_t)(dh & 0xff);
    out[209] = (uint8_t)(dh >> 8);
}

// Q8_0 (8 blocks = 256 elements): codes U{-127..127}; cfg1 = true draws
// d = f16(|N(0,0.02)|), otherwise d ~ 2.73e-4 * U(0.8,1.2).
SX_HD inline void sx_q80_group(uint64_t seed, uint64_t b, bool cfg1, uint8_t *out /*272*/) {
    for (int blk = 0; blk < 8; blk++) {
        const uint64_t base = (b * 8 + (uint64_t)blk) * 16;
        float d;
        if (cfg1) {
            const float n = sx_normal(seed, base + 5) * 0.02f;
            d = n < 0.0f ? -n : n;
        } else {
            d = 2.73e-04f * (0.8f + 0.4f * sx_unit(seed, base + 5));
        }
        const uint16_t dh = sx_f2h(d);
        uint8_t *o = out + 34 * blk;
        o[0] = (uint8_t)(dh & 0xff);
        o[1] = (uint8_t)(dh >> 8);
        for (int i = 0; i < 8; i++) {  // 16 random bits per code: U{-127..127}
            const uint64_t u = sx_u64(seed, base + 8 + (uint64_t)i);
            for (int k = 0; k < 4; k++) {
                const uint32_t r = (uint32_t)((u >> (16 * k)) & 0xffff);
                o[2 + 4 * i + k] = (uint8_t)(int8_t)((int)((r * 255u) >> 16) - 127);
            }
        }
    }
}

// type ids as include/sinter.h
enum { SX_F32 = 0, SX_F16 = 1, SX_Q8_0 = 8, SX_Q4_K = 12, SX_Q6_K = 14, SX_BF16 = 30 };

SX_HD inline uint32_t sx_group_bytes(int type) {
    switch (type) {
    case SX_Q4_K: return 144;
    case SX_Q6_K: return 210;
    case SX_Q8_0: return 272;
    case SX_BF16: case SX_F16: return 512;
    default: return 1024;
    }
}

// Q8_0 block b of std * N(0,1) values (elements 32b .. 32b+31), quantised
// as ggml's quantize_row_q8_0_ref: d = amax / 127, id = d ? 1/d : 0,
// q = roundf(x * id), d stored as f16.  34 bytes.
SX_HD inline void sx_q8_0_normal_block(uint64_t seed, uint64_t b, float std, uint8_t *out /*34*/) {
    float x[32], amax = 0.0f;
    for (int l = 0; l < 32; l++) {
        x[l] = std * sx_normal(seed, b * 32 + (uint64_t)l);
        amax = fmaxf(amax, fabsf(x[l]));
    }
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const uint16_t dh = sx_f2h(d);
    out[0] = (uint8_t)(dh & 0xff);
    out[1] = (uint8_t)(dh >> 8);
    for (int l = 0; l < 32; l++) out[2 + l] = (uint8_t)(int8_t)roundf(x[l] * id);
}

// Fill weight group b (256 elements) of a tensor of `type`.
SX_HD inline void sx_weight_group(uint64_t seed, uint64_t b, int type, bool cfg1, uint8_t *out) {
    switch (type) {
    case SX_Q4_K: sx_q4k_block(seed, b, out); break;
    case SX_Q6_K: sx_q6k_block(seed, b, out); break;
    case SX_Q8_0: sx_q80_group(seed, b, cfg1, out); break;
    case SX_BF16: case SX_F16:
        for (int i = 0; i < 256; i++) {
            const float v = sx_normal(seed, b * 256 + (uint64_t)i) * 0.02f;
            const uint16_t h = type == SX_BF16 ? sx_f2bf(v) : sx_f2h(v);
            out[2 * i] = (uint8_t)(h & 0xff);
            out[2 * i + 1] = (uint8_t)(h >> 8);
        }
        break;
    default:
        for (int i = 0; i < 256; i++) {
            const float v = sx_normal(seed, b * 256 + (uint64_t)i) * 0.02f;
            memcpy(out + 4 * i, &v, 4);
        }
        break;
    }
}

}  // namespace sinter
