/*
 * thvm_gen.h - portable synthetic input generator shared by the fixture
 * capture, the replayer and the CPU baseline, so that every side sees
 * bit-identical inputs without shipping them.
 *
 * Element i of a tensor with seed s uses SplitMix64 outputs, which are
 * counter based: output n (n >= 1) = mix(s + n * 0x9E3779B97F4A7C15).
 *   uniform U(lo,hi): u = (out(i+1) >> 40) * 2^-24, value = (f32)(lo + (hi-lo)*u)
 *   normal N(m,sd):   u1 = ((out(2i+1) >> 11) + 1) * 2^-53, u2 = (out(2i+2) >> 11) * 2^-53,
 *                     value = (f32)(m + sd * sqrt(-2 ln u1) * cos(2 pi u2))   (f64 math)
 *   int [lo,hi):      value = lo + ((out(i+1) >> 32) * (hi-lo)) >> 32
 *   const:            value = lo
 * Storage: f32 and i32/u32 elements take 4 bytes; f16 elements take 2, the
 * f32 value encoded with the engine's own f32 -> f16 rounding (round half up
 * on the first dropped mantissa bit, src/tinyhvm.h:433-457), so an f16 tensor
 * holds exactly what the engine would store for those values.
 */
#ifndef THVM_GEN_H
#define THVM_GEN_H

#include <stdint.h>
#include <math.h>
#include <string.h>

#define THVM_GEN_GAMMA 0x9E3779B97F4A7C15ULL

static inline uint64_t thvm_gen_mix(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

static inline uint64_t thvm_gen_out(uint64_t seed, uint64_t n) {
    return thvm_gen_mix(seed + n * THVM_GEN_GAMMA);
}

/* dist codes match TRC_GEN_* in thvm_trace.h */
static inline float thvm_gen_f32(uint32_t dist, uint64_t seed, uint64_t i, float p0, float p1) {
    switch (dist) {
    case 1: {
        double u = (double)(thvm_gen_out(seed, i + 1) >> 40) * (1.0 / 16777216.0);
        return (float)((double)p0 + ((double)p1 - (double)p0) * u);
    }
    case 2: {
        double u1 = ((double)(thvm_gen_out(seed, 2 * i + 1) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
        double u2 = (double)(thvm_gen_out(seed, 2 * i + 2) >> 11) * (1.0 / 9007199254740992.0);
        double r = sqrt(-2.0 * log(u1));
        return (float)((double)p0 + (double)p1 * r * cos(6.283185307179586 * u2));
    }
    case 3: {
        int64_t lo = (int64_t)p0, hi = (int64_t)p1;
        uint64_t span = (uint64_t)(hi - lo);
        uint64_t v = ((thvm_gen_out(seed, i + 1) >> 32) * span) >> 32;
        return (float)(lo + (int64_t)v);
    }
    case 4:
    default:
        return p0;
    }
}

static inline int32_t thvm_gen_i32(uint32_t dist, uint64_t seed, uint64_t i, float p0, float p1) {
    if (dist == 3) {
        int64_t lo = (int64_t)p0, hi = (int64_t)p1;
        uint64_t span = (uint64_t)(hi - lo);
        uint64_t v = ((thvm_gen_out(seed, i + 1) >> 32) * span) >> 32;
        return (int32_t)(lo + (int64_t)v);
    }
    return (int32_t)thvm_gen_f32(dist, seed, i, p0, p1);
}

/* f32 -> f16 bits with round half up on bit 12 of the mantissa; subnormal
 * results shift the implicit bit in first; overflow goes to infinity; NaN
 * keeps a quiet payload bit. */
static inline uint16_t thvm_gen_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u, man = x & 0x7FFFFFu;
    int32_t ex = (int32_t)((x >> 23) & 0xFFu) - 112;
    if (ex <= 0) {
        if (ex < -10) return (uint16_t)sign;
        man = (man | 0x800000u) >> (1 - ex);
        if (man & 0x1000u) man += 0x2000u;
        return (uint16_t)(sign | (man >> 13));
    }
    if (ex >= 31) return (uint16_t)(sign | 0x7C00u | (man ? 0x200u : 0u));
    if (man & 0x1000u) {
        man += 0x2000u;
        if (man & 0x800000u) {
            man = 0;
            ex += 1;
            if (ex >= 31) return (uint16_t)(sign | 0x7C00u);
        }
    }
    return (uint16_t)(sign | ((uint32_t)ex << 10) | (man >> 13));
}

/* Bytes per element of a storage dtype. */
static inline uint32_t thvm_gen_esize(uint32_t dtype) { return dtype == 1 ? 2u : 4u; }

/* Fill [begin, end) of a buffer of the given storage dtype (0 f32, 1 f16, 2 i32, 3 u32). */
static inline void thvm_gen_fill(void *dst, uint32_t dtype, uint32_t dist, uint64_t seed,
                                 float p0, float p1, uint64_t begin, uint64_t end) {
    for (uint64_t i = begin; i < end; i++) {
        if (dtype == 2 || dtype == 3) {
            int32_t v = thvm_gen_i32(dist, seed, i, p0, p1);
            memcpy((char *)dst + 4 * i, &v, 4);
        } else if (dtype == 1) {
            uint16_t h = thvm_gen_f16(thvm_gen_f32(dist, seed, i, p0, p1));
            memcpy((char *)dst + 2 * i, &h, 2);
        } else {
            float v = thvm_gen_f32(dist, seed, i, p0, p1);
            memcpy((char *)dst + 4 * i, &v, 4);
        }
    }
}

#endif /* THVM_GEN_H */
