/*
 * Oracle: independent C restatement of the weight-only int8 format.
 * TEST INFRASTRUCTURE ONLY - linked by tests through oracle/int8_quant_c.py,
 * never by the product library.
 *
 * The format is build-defined (the reference's quantized-linear slot is the
 * third-party autoawq int4 WQLinear, runtime/phase2/worker_server.py:194-205).
 * It restates oracle/int8_quant.py without numpy: the fp32 -> fp16
 * round-to-nearest-even conversion is written from the IEEE 754 bit layout, so
 * agreement between the two restatements pins numpy's conversion, division and
 * rint as well as the formula.
 *
 *   amax = max_k |w[n,k]|
 *   s    = fp16_rne(min(amax / 127, 65504)); amax == 0 -> 1.0; s == 0 -> 2^-24
 *   q    = clamp(rint(w / float(s)), -127, 127)
 *
 * Build: oracle/Makefile (gcc, no fast-math, SSE float arithmetic).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static uint16_t f32_to_f16_rne(float f) {
    uint32_t x;
    memcpy(&x, &f, sizeof x);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) { /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x0200u : 0u));
    }
    if (ax >= 0x477ff000u) { /* >= 65520 rounds to infinity */
        return (uint16_t)(sign | 0x7c00u);
    }
    if (ax < 0x38800000u) { /* below 2^-14: fp16 subnormal or zero */
        if (ax < 0x33000000u) { /* below 2^-25: rounds to zero */
            return (uint16_t)sign;
        }
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - e; /* value / 2^-24 = m * 2^(e - 126) */
        uint32_t qv = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (qv & 1u))) qv++;
        return (uint16_t)(sign | qv);
    }
    uint32_t e = (ax >> 23) - 127u + 15u;
    uint32_t m = ax & 0x7fffffu;
    uint32_t h = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

static float f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t m = (uint32_t)h & 0x3ffu;
    float out;
    if (e == 0) {
        out = ldexpf((float)m, -24);
        if (sign) out = -out;
        return out;
    }
    uint32_t bits;
    if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e - 15u + 127u) << 23) | (m << 13);
    }
    memcpy(&out, &bits, sizeof out);
    return out;
}

uint16_t oracle_f32_to_f16(float f) { return f32_to_f16_rne(f); }

float oracle_f16_to_f32(uint16_t h) { return f16_to_f32(h); }

/* Returns 0 on success, -1 on a non-finite weight. */
int oracle_quantize_int8(const float* w, int64_t n, int64_t k, int8_t* q, uint16_t* s_bits) {
    for (int64_t row = 0; row < n; ++row) {
        const float* wr = w + row * k;
        float amax = 0.0f;
        for (int64_t j = 0; j < k; ++j) {
            if (!isfinite(wr[j])) return -1;
            float a = fabsf(wr[j]);
            if (a > amax) amax = a;
        }
        float s32 = amax / 127.0f;
        if (s32 > 65504.0f) s32 = 65504.0f;
        uint16_t sb = f32_to_f16_rne(s32);
        if (amax == 0.0f) {
            sb = 0x3c00u;
        } else if ((sb & 0x7fffu) == 0) {
            sb = 0x0001u;
        }
        s_bits[row] = sb;
        float s = f16_to_f32(sb);
        for (int64_t j = 0; j < k; ++j) {
            float v = rintf(wr[j] / s);
            if (v > 127.0f) v = 127.0f;
            if (v < -127.0f) v = -127.0f;
            q[row * k + j] = (int8_t)v;
        }
    }
    return 0;
}

/* Tile pack: see oracle/int8_quant.py. Returns -1 on a bad shape. */
int oracle_pack_tiles(const int8_t* q, int64_t n, int64_t k, uint8_t* packed) {
    if (n % 16 != 0 || k % 64 != 0) return -1;
    int64_t nt_count = n / 16;
    for (int64_t row = 0; row < n; ++row) {
        int64_t nt = row / 16, r = row % 16;
        for (int64_t col = 0; col < k; ++col) {
            int64_t kt = col / 64, g = (col % 64) / 16, j = col % 16;
            int64_t lane = g * 16 + r;
            int64_t off = (kt * nt_count + nt) * 1024 + lane * 16 + j;
            packed[off] = (uint8_t)((uint8_t)q[row * k + col] ^ 0x80u);
        }
    }
    return 0;
}
