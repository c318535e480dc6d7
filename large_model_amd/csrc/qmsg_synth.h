/* qmsg_synth.h - seeded synthetic Qwen3-MoE layer data, bit-identical on host and device.
 *
 * Every tensor element is a pure function of (seed, layer, kind, expert, element index), so a
 * weight block can be produced anywhere - on the GPU straight into HBM for the large stacks,
 * on the host for the CPU checks - without moving data. Only integer arithmetic, IEEE
 * multiply/divide and round-to-nearest-even conversions are used, so a C compiler and hipcc
 * produce the same bits (build with -ffp-contract=off on both sides).
 *
 * Normal samples: Irwin-Hall sum of twelve 16-bit uniforms (three 64-bit hashes), centred and
 * scaled by 2^-16, which is N(0,1) up to the Irwin-Hall approximation (support +-6).
 * Q4_0 blocks use the usual ggml rounding (scale = signed max / -8, codes (x/d + 8.5) truncated,
 * capped at 15); Q4_1 blocks take the block's min as m and (max - min) / 15 as d. Q6_K super-blocks use per-16 scales (max|x|/31) requantised to int8 against
 * one fp16 super-scale; only the block format matters for the layer, not this rounding rule. */
#ifndef QMSG_SYNTH_H
#define QMSG_SYNTH_H

#include <stdint.h>

#if defined(__HIPCC__)
#define QMSG_HD __host__ __device__
#else
#define QMSG_HD
#endif

enum {                    /* tensor kinds, the third coordinate of an element's key */
    QMSG_KIND_X = 0,      /* layer input rows [T][E]                                   */
    QMSG_KIND_ROUTER = 1, /* ffn_gate_inp [X][E], F32                                   */
    QMSG_KIND_GATE = 2,   /* ffn_gate_exps [X][F][E]                                    */
    QMSG_KIND_UP = 3,     /* ffn_up_exps   [X][F][E]                                    */
    QMSG_KIND_DOWN = 4    /* ffn_down_exps [X][E][F]                                    */
};

QMSG_HD static inline uint64_t qmsg_mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

/* Key of one tensor slice (an expert's matrix, the router, the input). */
QMSG_HD static inline uint64_t qmsg_tensor_key(uint64_t seed, uint32_t layer, uint32_t kind,
                                               uint32_t expert)
{
    const uint64_t tag = ((uint64_t)layer << 40) ^ ((uint64_t)kind << 32) ^ (uint64_t)expert;
    return qmsg_mix64(seed ^ qmsg_mix64(tag + 0x632be59bd9b4e019ULL));
}

QMSG_HD static inline uint64_t qmsg_hash(uint64_t key, uint64_t i)
{
    return qmsg_mix64(key + (i + 1) * 0x9e3779b97f4a7c15ULL);
}

/* Approximately standard-normal sample number i of the slice `key`. */
QMSG_HD static inline float qmsg_normal(uint64_t key, uint64_t i)
{
    int32_t s = 0;
    for (int h = 0; h < 3; h++) {
        const uint64_t r = qmsg_hash(key, 3 * i + (uint64_t)h);
        s += (int32_t)(r & 0xFFFF) + (int32_t)((r >> 16) & 0xFFFF) + (int32_t)((r >> 32) & 0xFFFF) +
             (int32_t)(r >> 48);
    }
    return (float)(s - 393210) * (1.0f / 65536.0f);
}

union qmsg_f32_bits { float f; uint32_t u; };

/* fp32 -> fp16, round to nearest even, including subnormal results and overflow to inf. */
QMSG_HD static inline uint16_t qmsg_f32_to_f16(float f)
{
    union qmsg_f32_bits v;
    v.f = f;
    const uint32_t sign = (v.u >> 16) & 0x8000u;
    const uint32_t a = v.u & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (a > 0x7F800000u ? 0x200u : 0u));
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);          /* rounds past 65504 */
    if (a < 0x38800000u) {                                            /* fp16 subnormal or 0 */
        if (a < 0x33000000u) return (uint16_t)sign;                   /* below half of 2^-24 */
        const uint32_t e = a >> 23, m = (a & 0x7FFFFFu) | 0x800000u;
        const uint32_t shift = 126u - e;                              /* 14..24 */
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((a >> 13) - (112u << 10));                          /* rebias 127 -> 15 */
    const uint32_t rem = a & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

/* fp16 -> fp32, exact for every finite half. */
QMSG_HD static inline float qmsg_f16_to_f32(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu, bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            e = 113;
            while (!(m & 0x400u)) { m <<= 1; e--; }
            bits = sign | (e << 23) | ((m & 0x3FFu) << 13);
        }
    } else if (e == 0x1F) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    union qmsg_f32_bits v;
    v.u = bits;
    return v.f;
}

/* One Q4_0 block {f16 d; u8 qs[16]} from 32 values: element j < 16 in the low nibble of qs[j],
 * element j >= 16 in the high nibble of qs[j - 16]; w = (q - 8) * d. */
QMSG_HD static inline void qmsg_quant_q4_0_block(const float *v, uint8_t *out)
{
    float amax = 0.0f, mx = 0.0f;
    for (int j = 0; j < 32; j++) {
        const float a = v[j] < 0.0f ? -v[j] : v[j];
        if (a > amax) { amax = a; mx = v[j]; }
    }
    const float d = mx / -8.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const uint16_t dh = qmsg_f32_to_f16(d);
    out[0] = (uint8_t)(dh & 0xFF);
    out[1] = (uint8_t)(dh >> 8);
    for (int j = 0; j < 16; j++) {
        const float x0 = v[j] * id, x1 = v[j + 16] * id;
        int q0 = (int)(x0 + 8.5f), q1 = (int)(x1 + 8.5f);
        q0 = q0 < 0 ? 0 : (q0 > 15 ? 15 : q0);
        q1 = q1 < 0 ? 0 : (q1 > 15 ? 15 : q1);
        out[2 + j] = (uint8_t)(q0 | (q1 << 4));
    }
}

/* Q4_0 block b of row r of a [rows][cols] slice drawn from N(0, sigma). */
QMSG_HD static inline void qmsg_synth_q4_0_block(uint64_t key, uint64_t cols, uint64_t r, uint64_t b,
                                                 float sigma, uint8_t *out)
{
    float v[32];
    const uint64_t i0 = r * cols + b * 32;
    for (int j = 0; j < 32; j++) v[j] = qmsg_normal(key, i0 + (uint64_t)j) * sigma;
    qmsg_quant_q4_0_block(v, out);
}

/* One Q4_1 block {f16 d; f16 m; u8 qs[16]} from 32 values, nibbles as in Q4_0; w = q * d + m
 * with m = min, d = (max - min) / 15, codes (x - m) / d rounded half up, capped at 15. */
QMSG_HD static inline void qmsg_quant_q4_1_block(const float *v, uint8_t *out)
{
    float lo = v[0], hi = v[0];
    for (int j = 1; j < 32; j++) {
        lo = v[j] < lo ? v[j] : lo;
        hi = v[j] > hi ? v[j] : hi;
    }
    const float d = (hi - lo) / 15.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const uint16_t dh = qmsg_f32_to_f16(d), mh = qmsg_f32_to_f16(lo);
    out[0] = (uint8_t)(dh & 0xFF);
    out[1] = (uint8_t)(dh >> 8);
    out[2] = (uint8_t)(mh & 0xFF);
    out[3] = (uint8_t)(mh >> 8);
    for (int j = 0; j < 16; j++) {
        const float x0 = (v[j] - lo) * id, x1 = (v[j + 16] - lo) * id;
        int q0 = (int)(x0 + 0.5f), q1 = (int)(x1 + 0.5f);
        q0 = q0 > 15 ? 15 : q0;
        q1 = q1 > 15 ? 15 : q1;
        out[4 + j] = (uint8_t)(q0 | (q1 << 4));
    }
}

/* Q4_1 block b of row r of a [rows][cols] slice drawn from N(0, sigma). */
QMSG_HD static inline void qmsg_synth_q4_1_block(uint64_t key, uint64_t cols, uint64_t r, uint64_t b,
                                                 float sigma, uint8_t *out)
{
    float v[32];
    const uint64_t i0 = r * cols + b * 32;
    for (int j = 0; j < 32; j++) v[j] = qmsg_normal(key, i0 + (uint64_t)j) * sigma;
    qmsg_quant_q4_1_block(v, out);
}

/* One Q6_K super-block {u8 ql[128]; u8 qh[64]; i8 sc[16]; f16 d} = 210 bytes for 256 values
 * drawn from N(0, sigma) at elements i0 .. i0+255 of the slice `key`. Element i of the
 * super-block (half h = i/128, m = i%128, g = m/32, l = m%32) stores its 6-bit code q+32 in
 * ql[64h + 32(g&1) + l] (low nibble for g < 2, high for g >= 2) and qh[32h + l] bits 2g..2g+1,
 * with sub-scale sc[i/16]; w = d * sc * q. Values are regenerated instead of held (the
 * device version runs one super-block per thread). */
QMSG_HD static inline void qmsg_synth_q6_k_block(uint64_t key, uint64_t i0, float sigma, uint8_t *out)
{
    float scale[16];
    float smax = 0.0f;
    for (int s = 0; s < 16; s++) {
        float amax = 0.0f;
        for (int j = 0; j < 16; j++) {
            const float x = qmsg_normal(key, i0 + (uint64_t)(16 * s + j)) * sigma;
            const float a = x < 0.0f ? -x : x;
            if (a > amax) amax = a;
        }
        scale[s] = amax / 31.0f;
        if (scale[s] > smax) smax = scale[s];
    }
    const float d = smax / 127.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    const uint16_t dh = qmsg_f32_to_f16(d);
    const float dq = qmsg_f16_to_f32(dh);
    for (int i = 0; i < 208; i++) out[i] = 0;
    int8_t sc[16];
    for (int s = 0; s < 16; s++) {
        float r = scale[s] * id;
        int q = (int)(r + 0.5f);                  /* r >= 0 */
        q = q > 127 ? 127 : q;
        sc[s] = (int8_t)q;
        out[192 + s] = (uint8_t)sc[s];
    }
    out[208] = (uint8_t)(dh & 0xFF);
    out[209] = (uint8_t)(dh >> 8);
    for (int i = 0; i < 256; i++) {
        const float x = qmsg_normal(key, i0 + (uint64_t)i) * sigma;
        const float st = dq * (float)sc[i / 16];
        int q = 0;
        if (st != 0.0f) {
            const float r = x / st;
            q = (int)(r < 0.0f ? r - 0.5f : r + 0.5f);
            q = q < -32 ? -32 : (q > 31 ? 31 : q);
        }
        const int c = q + 32, h = i / 128, m = i % 128, g = m / 32, l = m % 32;
        out[64 * h + 32 * (g & 1) + l] |= (uint8_t)((c & 15) << (g < 2 ? 0 : 4));
        out[128 + 32 * h + l] |= (uint8_t)(((c >> 4) & 3) << (2 * g));
    }
}

#endif /* QMSG_SYNTH_H */
