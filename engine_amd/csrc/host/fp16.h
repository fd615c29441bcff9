// Host-side IEEE binary16 / bfloat16 conversions with round-to-nearest-even,
// the semantics of the reference's CPU codecs (backends/cpu/cpu_backend.cpp:
// 8-97): subnormals kept, overflow to infinity, NaN stays NaN.
#pragma once

#include <cmath>
#include <cstdint>
#include <cstring>

namespace lyk {

inline uint32_t float_bits(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}
inline float bits_float(uint32_t u) {
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

inline float f16_to_f32(uint16_t h) {
    const uint32_t sign = uint32_t(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 0x1F) return bits_float(sign | 0x7F800000u | (m << 13));
    if (e != 0) return bits_float(sign | ((e + 112u) << 23) | (m << 13));
    if (m == 0) return bits_float(sign);
    // subnormal: value m * 2^-24, exact in fp32
    const float v = float(m) * 5.9604644775390625e-08f;
    return sign ? -v : v;
}

inline uint16_t f32_to_f16(float f) {
    const uint32_t u = float_bits(f);
    const uint16_t sign = uint16_t((u >> 16) & 0x8000u);
    const uint32_t abs = u & 0x7FFFFFFFu;
    if (abs >= 0x7F800000u)  // inf / nan
        return uint16_t(sign | 0x7C00u | (abs > 0x7F800000u ? 0x200u : 0u));
    if (abs >= 0x477FF000u) return uint16_t(sign | 0x7C00u);  // rounds past 65504
    if (abs < 0x38800000u) {
        // result subnormal or zero: round abs * 2^24 to an integer, RNE
        if (abs < 0x33000000u) return sign;  // below half the smallest subnormal
        const uint32_t e = abs >> 23;
        const uint32_t mant = (abs & 0x7FFFFFu) | 0x800000u;
        const uint32_t shift = 126u - e;  // 14 - (e - 112)
        uint32_t q = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return uint16_t(sign | q);
    }
    // normal: rebias and round the low 13 mantissa bits to nearest even
    const uint32_t r = abs - (112u << 23);
    const uint32_t q = (r + 0x0FFFu + ((r >> 13) & 1u)) >> 13;
    return uint16_t(sign | q);
}

inline float bf16_to_f32(uint16_t b) { return bits_float(uint32_t(b) << 16); }

inline uint16_t f32_to_bf16(float f) {
    const uint32_t u = float_bits(f);
    if (std::isnan(f)) return uint16_t((u >> 16) | 0x0040u);
    return uint16_t((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// fp16 scale for symmetric quantization with codes in [-qmax, qmax]:
// fp16(absmax / qmax); 1.0 for an all-zero group or an fp16 underflow, the
// largest finite half on overflow.
inline uint16_t quant_scale_f16(float absmax, float qmax) {
    if (!(absmax > 0.0f)) return 0x3C00u;
    const uint16_t h = f32_to_f16(absmax / qmax);
    if ((h & 0x7FFFu) == 0) return 0x3C00u;
    if ((h & 0x7C00u) == 0x7C00u) return 0x7BFFu;
    return h;
}

}  // namespace lyk
