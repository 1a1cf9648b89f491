/*
 * lb_oracle.c — scalar CPU restatement of LightBridge-Engine's quantized-dot
 * path.  TEST INFRASTRUCTURE ONLY (the checker and CPU baseline, never the
 * product).  Citations are to /root/reference paths (file:line).
 *
 * Built with -O2 -ffp-contract=off -fno-fast-math: every f32 expression below
 * is evaluated as written (x86-64 SSE, FLT_EVAL_METHOD == 0), matching Rust's
 * non-contracting f32 semantics.
 */
#include "lb_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

#include "../lightbridge-engine_amd/csrc/lbh_iq_grids.inc"

static const uint64_t IQ2S_GRID[1024] = {LBH_IQ2S_GRID_VALUES};
static const uint32_t IQ3S_GRID[512] = {LBH_IQ3S_GRID_VALUES};

/* ---------------------------------------------------------------- helpers */

static inline int set_err(lbo_error *err, int status, int ty, uint64_t index, uint64_t expected,
                          uint64_t actual, uint32_t bits, uint32_t field) {
    if (err) {
        err->status = status;
        err->ty = ty;
        err->index = index;
        err->expected = expected;
        err->actual = actual;
        err->bits = bits;
        err->field = field;
    }
    return status;
}

static inline uint16_t rd_u16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline int16_t rd_i16(const uint8_t *p) { return (int16_t)rd_u16(p); }
static inline uint32_t rd_u32(const uint8_t *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
static inline float bits_f32(uint32_t b) {
    float f;
    memcpy(&f, &b, 4);
    return f;
}
static inline uint32_t f32_bits(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    return b;
}
static inline int f32_finite(float f) { return (f32_bits(f) & 0x7f800000u) != 0x7f800000u; }
static inline int f16_finite(uint16_t h) { return (h & 0x7c00u) != 0x7c00u; }

/* IEEE binary16 -> binary32, exact for every finite input including
 * subnormals; the reference uses half 2.7.1 `f16::to_f32` (q8_k.rs:230-232). */
float lbo_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            int e = -14;
            while (!(man & 0x400)) {
                man <<= 1;
                e -= 1;
            }
            man &= 0x3ff;
            bits = sign | ((uint32_t)(e + 127) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man ? (0x00400000u | (man << 13)) : 0);
    } else {
        bits = sign | ((exp - 15 + 127) << 23) | (man << 13);
    }
    return bits_f32(bits);
}

static inline float rd_f16(const uint8_t *p) { return lbo_f16_to_f32(rd_u16(p)); }
static inline float rd_f32(const uint8_t *p) { return bits_f32(rd_u32(p)); }

float lbo_expf(float x) { return expf(x); }

void lbo_expf_array(const float *x, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = expf(x[i]);
}

size_t lbo_block_bytes(int ty) {
    switch (ty) {
    case LBO_F32: return 4;
    case LBO_Q4_K: return 144;
    case LBO_Q5_K: return 176;
    case LBO_IQ2_S: return 82;
    case LBO_IQ3_S: return 110;
    case LBO_Q8_K: return 292;
    default: return 0;
    }
}

static size_t block_elems(int ty) { return ty == LBO_F32 ? 1 : 256; }

static int is_dot_type(int ty) {
    return ty == LBO_Q4_K || ty == LBO_Q5_K || ty == LBO_IQ2_S || ty == LBO_IQ3_S;
}

/* ------------------------------------------------------------- Q8_K quant */

/* nearest_int (q8_k.rs:224-228): magic-number round-to-nearest-even. */
static inline int32_t nearest_int(float v) {
    float s = v + 12582912.0f;
    int32_t b = (int32_t)f32_bits(s);
    return (b & 0x007fffff) - 0x00400000;
}

/* validate_logical_elements (q8_k.rs:188-200). */
static int check_elements(int ty, size_t n, size_t *blocks, lbo_error *err) {
    if (n == 0) return set_err(err, LBO_ZERO_LOGICAL_ELEMENTS, ty, 0, 0, 0, 0, 0);
    if (n % 256 != 0) return set_err(err, LBO_LOGICAL_ELEMENTS_NOT_DIVISIBLE, ty, 0, 256, n, 0, 0);
    *blocks = n / 256;
    return LBO_OK;
}

/* quantize_row_q8_k_into (q8_k.rs:16-76). */
int lbo_quantize_row_q8_k(const float *input, size_t n, uint8_t *encoded, size_t encoded_len,
                          lbo_error *err) {
    size_t blocks;
    int st = check_elements(LBO_Q8_K, n, &blocks, err);
    if (st) return st;
    size_t expected = blocks * 292;
    if (encoded_len != expected)
        return set_err(err, LBO_ENCODED_LENGTH_MISMATCH, LBO_Q8_K, 0, expected, encoded_len, 0, 0);
    for (size_t i = 0; i < n; ++i)
        if (!f32_finite(input[i]))
            return set_err(err, LBO_NON_FINITE_ACTIVATION, LBO_Q8_K, i, 0, 0, f32_bits(input[i]), 0);

    for (size_t b = 0; b < blocks; ++b) {
        const float *x = input + b * 256;
        uint8_t *out = encoded + b * 292;
        float max = 0.0f, amax = 0.0f;
        for (int i = 0; i < 256; ++i) {
            float a = fabsf(x[i]);
            if (a > amax) { /* strict: the first index wins a tie (q8_k.rs:43-49) */
                amax = a;
                max = x[i];
            }
        }
        if (amax == 0.0f) {
            memset(out, 0, 292);
            continue;
        }
        float iscale = -127.0f / max;
        for (int i = 0; i < 256; ++i) {
            int32_t q = nearest_int(iscale * x[i]);
            if (q > 127) q = 127;
            out[4 + i] = (uint8_t)(int8_t)q;
        }
        for (int g = 0; g < 16; ++g) {
            int32_t s = 0;
            for (int l = 0; l < 16; ++l) s += (int8_t)out[4 + 16 * g + l];
            uint16_t u = (uint16_t)(int16_t)s;
            out[260 + 2 * g] = (uint8_t)(u & 0xff);
            out[261 + 2 * g] = (uint8_t)(u >> 8);
        }
        uint32_t db = f32_bits(1.0f / iscale);
        out[0] = (uint8_t)db;
        out[1] = (uint8_t)(db >> 8);
        out[2] = (uint8_t)(db >> 16);
        out[3] = (uint8_t)(db >> 24);
    }
    return LBO_OK;
}

/* ------------------------------------------------------------ validation */

/* validate_scales (k_quants.rs:178-208): d then dmin, block by block. */
static int validate_scales(int ty, const uint8_t *w, size_t blocks, lbo_error *err) {
    size_t bb = lbo_block_bytes(ty);
    int two = (ty == LBO_Q4_K || ty == LBO_Q5_K);
    for (size_t b = 0; b < blocks; ++b) {
        uint16_t d = rd_u16(w + b * bb);
        if (!f16_finite(d)) return set_err(err, LBO_NON_FINITE_SCALE, ty, b, 0, 0, d, 0);
        if (two) {
            uint16_t m = rd_u16(w + b * bb + 2);
            if (!f16_finite(m)) return set_err(err, LBO_NON_FINITE_SCALE, ty, b, 0, 0, m, 1);
        }
    }
    return LBO_OK;
}

/* validate_q8_scales (q8_k.rs:208-222). */
static int validate_q8_scales(const uint8_t *q8, size_t blocks, lbo_error *err) {
    for (size_t b = 0; b < blocks; ++b) {
        uint32_t bits = rd_u32(q8 + b * 292);
        if (!f32_finite(bits_f32(bits)))
            return set_err(err, LBO_NON_FINITE_Q8_SCALE, LBO_Q8_K, b, 0, 0, bits, 0);
    }
    return LBO_OK;
}

/* validate_vec_dot_q8_k_inner (q8_k.rs:121-161). */
static int validate_dot(int ty, size_t w_len, const uint8_t *w, size_t q8_len, const uint8_t *q8,
                        size_t n, size_t *blocks, lbo_error *err) {
    if (!is_dot_type(ty)) return set_err(err, LBO_UNSUPPORTED_TYPE, ty, 0, 0, 0, 0, 0);
    int st = check_elements(ty, n, blocks, err);
    if (st) return st;
    size_t ew = *blocks * lbo_block_bytes(ty);
    if (w_len != ew) return set_err(err, LBO_ENCODED_LENGTH_MISMATCH, ty, 0, ew, w_len, 0, 0);
    size_t eq = *blocks * 292;
    if (q8_len != eq) return set_err(err, LBO_ENCODED_LENGTH_MISMATCH, LBO_Q8_K, 0, eq, q8_len, 0, 0);
    st = validate_scales(ty, w, *blocks, err);
    if (st) return st;
    return validate_q8_scales(q8, *blocks, err);
}

/* ------------------------------------------------------------ scalar dots */

/* scale_min (k_quants.rs:231-240): 6-bit (scale, min) of sub-block j. */
static inline void scale_min(const uint8_t *sc, int j, uint8_t *s, uint8_t *m) {
    if (j < 4) {
        *s = sc[j] & 63;
        *m = sc[j + 4] & 63;
    } else {
        *s = (uint8_t)((sc[j + 4] & 0x0f) | ((sc[j - 4] >> 6) << 4));
        *m = (uint8_t)((sc[j + 4] >> 4) | ((sc[j] >> 6) << 4));
    }
}

/* Unpack one Q4_K / Q5_K block into 256 unsigned quants (q8_k.rs:259-286). */
static void kquant_unpack(int ty, const uint8_t *blk, int8_t q[256]) {
    if (ty == LBO_Q4_K) {
        for (int g = 0; g < 4; ++g)
            for (int l = 0; l < 32; ++l) {
                uint8_t p = blk[16 + 32 * g + l];
                q[64 * g + l] = (int8_t)(p & 0x0f);
                q[64 * g + 32 + l] = (int8_t)(p >> 4);
            }
    } else {
        for (int g = 0; g < 4; ++g)
            for (int l = 0; l < 32; ++l) {
                uint8_t p = blk[48 + 32 * g + l];
                uint8_t h = blk[16 + l];
                q[64 * g + l] = (int8_t)((p & 0x0f) + (((h >> (2 * g)) & 1) ? 16 : 0));
                q[64 * g + 32 + l] = (int8_t)((p >> 4) + (((h >> (2 * g + 1)) & 1) ? 16 : 0));
            }
    }
}

/* Integer stage of dot_q4_or_q5_k (q8_k.rs:288-312): 8 lane sums keyed by
 * element index mod 8, plus minimum_sum. */
static void kquant_block_ints(int ty, const uint8_t *blk, const uint8_t *a, int32_t lanes[8],
                              int32_t *minsum) {
    int8_t q[256];
    kquant_unpack(ty, blk, q);
    uint8_t sc[8], mn[8];
    for (int j = 0; j < 8; ++j) scale_min(blk + 4, j, &sc[j], &mn[j]);
    int32_t ms = 0;
    for (int g = 0; g < 16; ++g) ms += (int32_t)rd_i16(a + 260 + 2 * g) * (int32_t)mn[g / 2];
    *minsum = ms;
    for (int l = 0; l < 8; ++l) lanes[l] = 0;
    int off = 0;
    for (int j = 0; j < 8; ++j)
        for (int k = 0; k < 4; ++k) {
            for (int l = 0; l < 8; ++l)
                lanes[l] += (int32_t)sc[j] * (int32_t)(int8_t)a[4 + off + l] * (int32_t)q[off + l];
            off += 8;
        }
}

/* dot_q4_or_q5_k (q8_k.rs:247-327). */
static float dot_kquant(int ty, const uint8_t *w, const uint8_t *q8, size_t blocks) {
    size_t bb = lbo_block_bytes(ty);
    float sums[8] = {0};
    float sum = 0.0f;
    for (size_t b = 0; b < blocks; ++b) {
        const uint8_t *blk = w + b * bb;
        const uint8_t *a = q8 + b * 292;
        int32_t lanes[8], ms;
        kquant_block_ints(ty, blk, a, lanes, &ms);
        float d8 = rd_f32(a);
        float scale = rd_f16(blk) * d8;
        for (int l = 0; l < 8; ++l) sums[l] += scale * (float)lanes[l];
        float mscale = rd_f16(blk + 2) * d8;
        sum -= mscale * (float)ms;
    }
    for (int l = 0; l < 8; ++l) sum += sums[l];
    return sum;
}

/* Integer block sum of dot_iq2_s (q8_k.rs:337-364). */
static int32_t iq2s_block_int(const uint8_t *blk, const uint8_t *a) {
    int32_t bsum = 0;
    for (int g = 0; g < 8; ++g) {
        uint8_t ps = blk[74 + g];
        int32_t s1 = 1 + 2 * (ps & 0x0f), s2 = 1 + 2 * (ps >> 4);
        uint32_t hi = blk[66 + g];
        int32_t part[2] = {0, 0};
        for (int lg = 0; lg < 4; ++lg) {
            uint32_t idx = blk[2 + 4 * g + lg] | ((hi << (8 - 2 * lg)) & 0x300);
            uint64_t grid = IQ2S_GRID[idx];
            uint8_t signs = blk[34 + 4 * g + lg];
            const int8_t *av = (const int8_t *)(a + 4 + 32 * g + 8 * lg);
            for (int l = 0; l < 8; ++l) {
                int32_t mag = (int32_t)((grid >> (8 * l)) & 0xff);
                int32_t sg = (signs >> l) & 1 ? -1 : 1;
                part[lg / 2] += (int32_t)av[l] * mag * sg;
            }
        }
        bsum += s1 * part[0] + s2 * part[1];
    }
    return bsum;
}

/* dot_iq2_s (q8_k.rs:329-370). */
static float dot_iq2s(const uint8_t *w, const uint8_t *q8, size_t blocks) {
    float sum = 0.0f;
    for (size_t b = 0; b < blocks; ++b) {
        const uint8_t *blk = w + b * 82;
        const uint8_t *a = q8 + b * 292;
        float scale = rd_f16(blk) * rd_f32(a);
        sum += scale * (float)iq2s_block_int(blk, a);
    }
    return 0.125f * sum;
}

/* Integer block sum of dot_iq3_s (q8_k.rs:380-428). */
static int32_t iq3s_block_int(const uint8_t *blk, const uint8_t *a) {
    int32_t bsum = 0;
    for (int p = 0; p < 4; ++p) {
        uint8_t ps = blk[106 + p];
        int32_t pscale[2] = {2 * (ps & 0x0f) + 1, 2 * (ps >> 4) + 1};
        for (int h = 0; h < 2; ++h) {
            int g = 2 * p + h;
            uint32_t hi = blk[66 + g];
            int32_t gs = 0;
            for (int lg = 0; lg < 4; ++lg) {
                uint32_t i1 = blk[2 + 8 * g + 2 * lg] | ((hi << (8 - 2 * lg)) & 0x100);
                uint32_t i2 = blk[2 + 8 * g + 2 * lg + 1] | ((hi << (7 - 2 * lg)) & 0x100);
                uint32_t g1 = IQ3S_GRID[i1], g2 = IQ3S_GRID[i2];
                uint8_t signs = blk[74 + 4 * g + lg];
                const int8_t *av = (const int8_t *)(a + 4 + 32 * g + 8 * lg);
                for (int l = 0; l < 4; ++l) {
                    int32_t m1 = (int32_t)((g1 >> (8 * l)) & 0xff);
                    int32_t m2 = (int32_t)((g2 >> (8 * l)) & 0xff);
                    int32_t s1 = (signs >> l) & 1 ? -1 : 1;
                    int32_t s2 = (signs >> (l + 4)) & 1 ? -1 : 1;
                    gs += (int32_t)av[l] * m1 * s1;
                    gs += (int32_t)av[l + 4] * m2 * s2;
                }
            }
            bsum += gs * pscale[h];
        }
    }
    return bsum;
}

/* dot_iq3_s (q8_k.rs:372-434). */
static float dot_iq3s(const uint8_t *w, const uint8_t *q8, size_t blocks) {
    float sum = 0.0f;
    for (size_t b = 0; b < blocks; ++b) {
        const uint8_t *blk = w + b * 110;
        const uint8_t *a = q8 + b * 292;
        float scale = rd_f16(blk) * rd_f32(a);
        sum += scale * (float)iq3s_block_int(blk, a);
    }
    return sum;
}

/* dot_scalar (q8_k.rs:163-170). */
float lbo_dot_scalar(int ty, const uint8_t *w, const uint8_t *q8, size_t blocks) {
    switch (ty) {
    case LBO_Q4_K:
    case LBO_Q5_K: return dot_kquant(ty, w, q8, blocks);
    case LBO_IQ2_S: return dot_iq2s(w, q8, blocks);
    case LBO_IQ3_S: return dot_iq3s(w, q8, blocks);
    default: return NAN;
    }
}

int lbo_block_sums(int ty, const uint8_t *w, const uint8_t *q8, size_t blocks, int32_t *out) {
    size_t bb = lbo_block_bytes(ty);
    for (size_t b = 0; b < blocks; ++b) {
        const uint8_t *blk = w + b * bb;
        const uint8_t *a = q8 + b * 292;
        switch (ty) {
        case LBO_Q4_K:
        case LBO_Q5_K: kquant_block_ints(ty, blk, a, out + 9 * b, out + 9 * b + 8); break;
        case LBO_IQ2_S: out[b] = iq2s_block_int(blk, a); break;
        case LBO_IQ3_S: out[b] = iq3s_block_int(blk, a); break;
        default: return LBO_UNSUPPORTED_TYPE;
        }
    }
    return LBO_OK;
}

/* vec_dot_q8_k (q8_k.rs:80-89). */
int lbo_vec_dot_q8_k(int ty, const uint8_t *w, size_t w_len, const uint8_t *q8, size_t q8_len,
                     size_t n, float *out, lbo_error *err) {
    size_t blocks;
    int st = validate_dot(ty, w_len, w, q8_len, q8, n, &blocks, err);
    if (st) return st;
    *out = lbo_dot_scalar(ty, w, q8, blocks);
    return LBO_OK;
}

/* vec_dot_q8_k_cpu (q8_k.rs:103-119) with the AVX2 branch taken. */
int lbo_vec_dot_q8_k_avx2(int ty, const uint8_t *w, size_t w_len, const uint8_t *q8, size_t q8_len,
                          size_t n, float *out, lbo_error *err) {
    size_t blocks;
    int st = validate_dot(ty, w_len, w, q8_len, q8, n, &blocks, err);
    if (st) return st;
    *out = lbo_dot_avx2(ty, w, q8, blocks);
    return LBO_OK;
}

/* --------------------------------------------------------------- decoders */

/* decode_q4_k_validated / decode_q5_k_validated (k_quants.rs:242-300). */
static void decode_kquant(int ty, const uint8_t *blk, float *o) {
    float d = rd_f16(blk), dmin = rd_f16(blk + 2);
    const uint8_t *sc = blk + 4;
    const uint8_t *qs = blk + (ty == LBO_Q4_K ? 16 : 48);
    for (int g = 0; g < 4; ++g) {
        uint8_t s1, m1, s2, m2;
        scale_min(sc, 2 * g, &s1, &m1);
        scale_min(sc, 2 * g + 1, &s2, &m2);
        float d1 = d * (float)s1, mm1 = dmin * (float)m1;
        float d2 = d * (float)s2, mm2 = dmin * (float)m2;
        for (int l = 0; l < 32; ++l) {
            uint8_t q = qs[32 * g + l] & 0x0f;
            if (ty == LBO_Q5_K && ((blk[16 + l] >> (2 * g)) & 1)) q += 16;
            o[64 * g + l] = d1 * (float)q - mm1;
        }
        for (int l = 0; l < 32; ++l) {
            uint8_t q = qs[32 * g + l] >> 4;
            if (ty == LBO_Q5_K && ((blk[16 + l] >> (2 * g + 1)) & 1)) q += 16;
            o[64 * g + 32 + l] = d2 * (float)q - mm2;
        }
    }
}

/* decode_iq2_s_validated (iq2_s.rs:9-39). */
static void decode_iq2s(const uint8_t *blk, float *o) {
    float d = rd_f16(blk);
    for (int g = 0; g < 8; ++g) {
        uint8_t s = blk[74 + g];
        float bs[2] = {d * (0.5f + (float)(s & 0x0f)) * 0.25f, d * (0.5f + (float)(s >> 4)) * 0.25f};
        uint32_t hi = blk[66 + g];
        for (int lg = 0; lg < 4; ++lg) {
            uint32_t idx = blk[2 + 4 * g + lg] | ((hi << (8 - 2 * lg)) & 0x300);
            uint64_t grid = IQ2S_GRID[idx];
            uint8_t signs = blk[34 + 4 * g + lg];
            for (int l = 0; l < 8; ++l) {
                float sg = (signs >> l) & 1 ? -1.0f : 1.0f;
                o[32 * g + 8 * lg + l] = bs[lg / 2] * (float)((grid >> (8 * l)) & 0xff) * sg;
            }
        }
    }
}

/* decode_iq3_s_validated (iq3_s.rs:9-53). */
static void decode_iq3s(const uint8_t *blk, float *o) {
    float d = rd_f16(blk);
    for (int p = 0; p < 4; ++p) {
        uint8_t ps = blk[106 + p];
        float sc[2] = {d * (float)(1 + 2 * (ps & 0x0f)), d * (float)(1 + 2 * (ps >> 4))};
        for (int h = 0; h < 2; ++h) {
            int g = 2 * p + h;
            uint32_t hi = blk[66 + g];
            for (int lg = 0; lg < 4; ++lg) {
                uint32_t i1 = blk[2 + 8 * g + 2 * lg] | ((hi << (8 - 2 * lg)) & 0x100);
                uint32_t i2 = blk[2 + 8 * g + 2 * lg + 1] | ((hi << (7 - 2 * lg)) & 0x100);
                uint32_t g1 = IQ3S_GRID[i1], g2 = IQ3S_GRID[i2];
                uint8_t signs = blk[74 + 4 * g + lg];
                for (int l = 0; l < 4; ++l) {
                    float s1 = (signs >> l) & 1 ? -1.0f : 1.0f;
                    float s2 = (signs >> (l + 4)) & 1 ? -1.0f : 1.0f;
                    o[32 * g + 8 * lg + l] = sc[h] * (float)((g1 >> (8 * l)) & 0xff) * s1;
                    o[32 * g + 8 * lg + l + 4] = sc[h] * (float)((g2 >> (8 * l)) & 0xff) * s2;
                }
            }
        }
    }
}

static void decode_block(int ty, const uint8_t *blk, float *o) {
    switch (ty) {
    case LBO_F32: o[0] = rd_f32(blk); break;
    case LBO_Q4_K:
    case LBO_Q5_K: decode_kquant(ty, blk, o); break;
    case LBO_IQ2_S: decode_iq2s(blk, o); break;
    case LBO_IQ3_S: decode_iq3s(blk, o); break;
    }
}

/* decode_row_into (k_quants.rs:71-105). */
int lbo_decode_row(int ty, const uint8_t *w, size_t w_len, size_t n, float *out, size_t out_len,
                   lbo_error *err) {
    size_t bb = lbo_block_bytes(ty);
    if (bb == 0 || ty == LBO_Q8_K) return set_err(err, LBO_UNSUPPORTED_TYPE, ty, 0, 0, 0, 0, 0);
    size_t be = block_elems(ty);
    if (n == 0) return set_err(err, LBO_ZERO_LOGICAL_ELEMENTS, ty, 0, 0, 0, 0, 0);
    if (n % be) return set_err(err, LBO_LOGICAL_ELEMENTS_NOT_DIVISIBLE, ty, 0, be, n, 0, 0);
    size_t blocks = n / be;
    if (w_len != blocks * bb)
        return set_err(err, LBO_ENCODED_LENGTH_MISMATCH, ty, 0, blocks * bb, w_len, 0, 0);
    if (out_len != n) return set_err(err, LBO_OUTPUT_LENGTH_MISMATCH, ty, 0, n, out_len, 0, 0);
    if (ty != LBO_F32) {
        int st = validate_scales(ty, w, blocks, err);
        if (st) return st;
    }
    for (size_t b = 0; b < blocks; ++b) decode_block(ty, w + b * bb, out + b * be);
    return LBO_OK;
}

/* ------------------------------------------------------------ thread pool */

/* A persistent fork-join pool standing in for the reference's bounded rayon
 * pool (crates/bridge-kernels-cpu/src/lib.rs:76-118); rows are claimed in small
 * chunks, like par_iter_mut's splitting.  Rows are independent, so scheduling
 * has no arithmetic effect. */
typedef void (*row_fn)(void *ctx, size_t r0, size_t r1);

typedef struct pool {
    int threads;
    pthread_t tids[256];
    pthread_mutex_t mu;
    pthread_cond_t cv_start, cv_done;
    uint64_t generation;
    int pending;
    int shutdown;
    row_fn fn;
    void *ctx;
    size_t rows, chunk;
    atomic_size_t next;
} pool;

static pool *g_pool;
static pthread_mutex_t g_pool_mu = PTHREAD_MUTEX_INITIALIZER;

static void pool_run_rows(pool *p) {
    for (;;) {
        size_t r0 = atomic_fetch_add(&p->next, p->chunk);
        if (r0 >= p->rows) break;
        size_t r1 = r0 + p->chunk < p->rows ? r0 + p->chunk : p->rows;
        p->fn(p->ctx, r0, r1);
    }
}

static void *pool_worker(void *arg) {
    pool *p = (pool *)arg;
    uint64_t seen = 0;
    pthread_mutex_lock(&p->mu);
    for (;;) {
        while (p->generation == seen && !p->shutdown) pthread_cond_wait(&p->cv_start, &p->mu);
        if (p->shutdown) break;
        seen = p->generation;
        pthread_mutex_unlock(&p->mu);
        pool_run_rows(p);
        pthread_mutex_lock(&p->mu);
        if (--p->pending == 0) pthread_cond_signal(&p->cv_done);
    }
    pthread_mutex_unlock(&p->mu);
    return NULL;
}

static void pool_destroy(pool *p) {
    pthread_mutex_lock(&p->mu);
    p->shutdown = 1;
    pthread_cond_broadcast(&p->cv_start);
    pthread_mutex_unlock(&p->mu);
    for (int i = 0; i < p->threads - 1; ++i) pthread_join(p->tids[i], NULL);
    free(p);
}

static pool *pool_get(int threads) {
    if (threads > 256) threads = 256;
    pthread_mutex_lock(&g_pool_mu);
    if (g_pool && g_pool->threads != threads) {
        pool_destroy(g_pool);
        g_pool = NULL;
    }
    if (!g_pool) {
        pool *p = (pool *)calloc(1, sizeof(pool));
        p->threads = threads;
        pthread_mutex_init(&p->mu, NULL);
        pthread_cond_init(&p->cv_start, NULL);
        pthread_cond_init(&p->cv_done, NULL);
        for (int i = 0; i < threads - 1; ++i) pthread_create(&p->tids[i], NULL, pool_worker, p);
        g_pool = p;
    }
    pthread_mutex_unlock(&g_pool_mu);
    return g_pool;
}

static void parallel_rows(int threads, size_t rows, row_fn fn, void *ctx) {
    if (threads <= 1 || rows < 2) {
        fn(ctx, 0, rows);
        return;
    }
    pool *p = pool_get(threads);
    size_t chunk = rows / (size_t)(threads * 8);
    if (chunk < 1) chunk = 1;
    pthread_mutex_lock(&p->mu);
    p->fn = fn;
    p->ctx = ctx;
    p->rows = rows;
    p->chunk = chunk;
    atomic_store(&p->next, 0);
    p->pending = threads - 1;
    p->generation++;
    pthread_cond_broadcast(&p->cv_start);
    pthread_mutex_unlock(&p->mu);
    pool_run_rows(p);
    pthread_mutex_lock(&p->mu);
    while (p->pending) pthread_cond_wait(&p->cv_done, &p->mu);
    pthread_mutex_unlock(&p->mu);
}

/* ------------------------------------------------------------------ gemv */

static size_t row_bytes(const lbo_matrix *m) { return (size_t)(m->k / block_elems(m->ty)) * lbo_block_bytes(m->ty); }

typedef struct gemv_ctx {
    const lbo_matrix *m;
    const uint8_t *q8;
    float *out;
    float scale;
    int accumulate;
    int avx2;
} gemv_ctx;

static void gemv_rows(void *vctx, size_t r0, size_t r1) {
    gemv_ctx *c = (gemv_ctx *)vctx;
    size_t rb = row_bytes(c->m), blocks = c->m->k / 256;
    for (size_t r = r0; r < r1; ++r) {
        const uint8_t *row = c->m->bytes + r * rb;
        float v = c->avx2 ? lbo_dot_avx2(c->m->ty, row, c->q8, blocks)
                          : lbo_dot_scalar(c->m->ty, row, c->q8, blocks);
        if (c->accumulate)
            c->out[r] += c->scale * v;
        else
            c->out[r] = v;
    }
}

int lbo_gemv_prequantized(const lbo_exec *ex, const lbo_matrix *m, const uint8_t *q8, float *y) {
    gemv_ctx c = {m, q8, y, 0.0f, 0, ex->avx2};
    int threads = ex->mode == LBO_MODE_CPU_PARALLEL_Q8K ? ex->threads : 1;
    parallel_rows(threads, m->rows, gemv_rows, &c);
    return LBO_OK;
}

/* dot_f32_row (gemv.rs:286-303). */
static float dot_f32_row(const lbo_matrix *m, size_t r, const float *x) {
    const uint8_t *row = m->bytes + r * m->k * 4;
    float sum = 0.0f;
    for (size_t i = 0; i < m->k; ++i) sum += rd_f32(row + 4 * i) * x[i];
    return sum;
}

/* dot_dequant_row (gemv.rs:305-328). */
static float dot_dequant_row(const lbo_matrix *m, size_t r, const float *x) {
    size_t bb = lbo_block_bytes(m->ty), be = block_elems(m->ty), rb = row_bytes(m);
    float dec[256];
    float sum = 0.0f;
    for (size_t b = 0; b < m->k / be; ++b) {
        decode_block(m->ty, m->bytes + r * rb + b * bb, dec);
        for (size_t l = 0; l < be; ++l) sum += dec[l] * x[b * be + l];
    }
    return sum;
}

void lbo_router_logits_f32(const float *w, size_t n_experts, size_t k, const float *x, float *logits) {
    for (size_t e = 0; e < n_experts; ++e) {
        float sum = 0.0f;
        for (size_t i = 0; i < k; ++i) sum += w[e * k + i] * x[i];
        logits[e] = sum;
    }
}

/* validate_dimensions (gemv.rs:195-211). */
static int validate_dimensions(const lbo_matrix *m, const float *input, size_t input_len,
                               size_t output_len, lbo_error *err) {
    if (input_len != m->k) return set_err(err, LBO_DIMENSION_MISMATCH, m->ty, 0, m->k, input_len, 0, 0);
    if (output_len != m->rows)
        return set_err(err, LBO_DIMENSION_MISMATCH, m->ty, 1, m->rows, output_len, 0, 0);
    for (size_t i = 0; i < input_len; ++i)
        if (!f32_finite(input[i]))
            return set_err(err, LBO_NON_FINITE_VALUE, m->ty, i, 0, 0, f32_bits(input[i]), 0);
    return LBO_OK;
}

/* prepare_dequant (gemv.rs:213-243): decode every block and require finite weights. */
static int prepare_dequant(const lbo_matrix *m, const float *input, size_t input_len,
                           size_t output_len, lbo_error *err) {
    int st = validate_dimensions(m, input, input_len, output_len, err);
    if (st) return st;
    size_t bb = lbo_block_bytes(m->ty), be = block_elems(m->ty), rb = row_bytes(m);
    if (bb == 0 || m->ty == LBO_Q8_K) return set_err(err, LBO_UNSUPPORTED_TYPE, m->ty, 0, 0, 0, 0, 0);
    float dec[256];
    for (size_t r = 0; r < m->rows; ++r)
        for (size_t b = 0; b < m->k / be; ++b) {
            const uint8_t *blk = m->bytes + r * rb + b * bb;
            if (m->ty != LBO_F32) {
                st = validate_scales(m->ty, blk, 1, err);
                if (st) return st;
            }
            decode_block(m->ty, blk, dec);
            for (size_t l = 0; l < be; ++l)
                if (!f32_finite(dec[l]))
                    return set_err(err, LBO_NON_FINITE_VALUE, m->ty, l, 0, 0, f32_bits(dec[l]), 1);
        }
    return LBO_OK;
}

/* prepare_llama_q8k (gemv.rs:245-272). */
static int prepare_q8k(const lbo_matrix *m, const float *input, size_t input_len, size_t output_len,
                       uint8_t *q8, size_t q8_len, lbo_error *err) {
    int st = validate_dimensions(m, input, input_len, output_len, err);
    if (st) return st;
    if (!is_dot_type(m->ty)) return set_err(err, LBO_UNSUPPORTED_TYPE, m->ty, 0, 0, 0, 0, 0);
    if (m->k == 0 || m->k % 256)
        return set_err(err, LBO_DIMENSION_MISMATCH, LBO_Q8_K, 2, 256, m->k, 0, 0);
    size_t need = m->k / 256 * 292;
    if (q8_len < need) return set_err(err, LBO_SCRATCH_TOO_SMALL, LBO_Q8_K, 0, need, q8_len, 0, 0);
    st = lbo_quantize_row_q8_k(input, input_len, q8, need, err);
    if (st) return st;
    size_t rb = row_bytes(m), blocks = m->k / 256;
    for (size_t r = 0; r < m->rows; ++r) {
        size_t nb;
        st = validate_dot(m->ty, rb, m->bytes + r * rb, need, q8, m->k, &nb, err);
        if (st) return st; /* err->index is the block index within the failing row */
    }
    (void)blocks;
    return LBO_OK;
}

int lbo_gemv(const lbo_exec *ex, const lbo_matrix *m, const float *input, size_t input_len,
             float *output, size_t output_len, uint8_t *q8_scratch, size_t q8_len, lbo_error *err) {
    int st;
    if (m->ty == LBO_F32 || ex->mode == LBO_MODE_DEQUANT_F32) {
        st = prepare_dequant(m, input, input_len, output_len, err);
        if (st) return st;
        for (size_t r = 0; r < m->rows; ++r)
            output[r] = m->ty == LBO_F32 ? dot_f32_row(m, r, input) : dot_dequant_row(m, r, input);
        return LBO_OK;
    }
    st = prepare_q8k(m, input, input_len, output_len, q8_scratch, q8_len, err);
    if (st) return st;
    gemv_ctx c = {m, q8_scratch, output, 0.0f, 0, ex->mode == LBO_MODE_CPU_PARALLEL_Q8K && ex->avx2};
    parallel_rows(ex->mode == LBO_MODE_CPU_PARALLEL_Q8K ? ex->threads : 1, m->rows, gemv_rows, &c);
    return LBO_OK;
}

int lbo_gemv_accumulate(const lbo_exec *ex, const lbo_matrix *m, const float *input,
                        size_t input_len, float *dest, size_t dest_len, float scale,
                        uint8_t *q8_scratch, size_t q8_len, lbo_error *err) {
    if (!f32_finite(scale)) return set_err(err, LBO_NON_FINITE_VALUE, m->ty, 0, 0, 0, f32_bits(scale), 2);
    for (size_t i = 0; i < dest_len; ++i)
        if (!f32_finite(dest[i])) return set_err(err, LBO_NON_FINITE_VALUE, m->ty, i, 0, 0, f32_bits(dest[i]), 3);
    int st;
    if (m->ty == LBO_F32 || ex->mode == LBO_MODE_DEQUANT_F32) {
        st = prepare_dequant(m, input, input_len, dest_len, err);
        if (st) return st;
        for (size_t r = 0; r < m->rows; ++r)
            dest[r] += scale * (m->ty == LBO_F32 ? dot_f32_row(m, r, input) : dot_dequant_row(m, r, input));
        return LBO_OK;
    }
    st = prepare_q8k(m, input, input_len, dest_len, q8_scratch, q8_len, err);
    if (st) return st;
    gemv_ctx c = {m, q8_scratch, dest, scale, 1, ex->mode == LBO_MODE_CPU_PARALLEL_Q8K && ex->avx2};
    parallel_rows(ex->mode == LBO_MODE_CPU_PARALLEL_Q8K ? ex->threads : 1, m->rows, gemv_rows, &c);
    return LBO_OK;
}

/* residual_add_in_place (crates/bridge-kernels-reference/src/norm.rs:83-98):
 * lengths, then a finite destination, a finite source and every sum finite
 * (field 0 destination, 1 source, 2 output; index = lane), all before the
 * first write; then destination[i] += residual[i]. */
int lbo_residual_add_in_place(float *destination, size_t dest_len, const float *residual, size_t residual_len,
                              lbo_error *err) {
    if (dest_len != residual_len)
        return set_err(err, LBO_DIMENSION_MISMATCH, LBO_F32, 0, dest_len, residual_len, 0, 0);
    for (size_t i = 0; i < dest_len; ++i)
        if (!f32_finite(destination[i]))
            return set_err(err, LBO_NON_FINITE_VALUE, LBO_F32, i, 0, 0, f32_bits(destination[i]), 0);
    for (size_t i = 0; i < dest_len; ++i)
        if (!f32_finite(residual[i]))
            return set_err(err, LBO_NON_FINITE_VALUE, LBO_F32, i, 0, 0, f32_bits(residual[i]), 1);
    for (size_t i = 0; i < dest_len; ++i) {
        float v = destination[i] + residual[i];
        if (!f32_finite(v)) return set_err(err, LBO_NON_FINITE_VALUE, LBO_F32, i, 0, 0, f32_bits(v), 2);
    }
    for (size_t i = 0; i < dest_len; ++i) destination[i] += residual[i];
    return LBO_OK;
}

/* --------------------------------------------------------------- SwiGLU */

/* apply_swiglu (activation.rs:170-178).  On a non-finite product the
 * reference returns NonFiniteValue carrying that product's bits
 * (validate_finite_value, gemv.rs); it is left in gate[i] so the caller can
 * report them (the reference's scratch is not observable otherwise). */
int64_t lbo_apply_swiglu(float *gate, const float *up, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        float g = gate[i];
        float act = g / (1.0f + expf(-g));
        float v = act * up[i];
        gate[i] = v;
        if (!f32_finite(v)) return (int64_t)i;
    }
    return -1;
}

typedef struct swiglu_scratch {
    float *act;      /* 2 * hidden */
    uint8_t *q8;
    size_t q8_len;
} swiglu_scratch;

/* swiglu_project_into / expert_swiglu_accumulate_into (activation.rs:65-144). */
static int swiglu_expert(const lbo_exec *ex, const lbo_expert *e, const float *input, float *out,
                         int accumulate, float coef, swiglu_scratch *s, lbo_error *err) {
    if (accumulate && !f32_finite(coef))
        return set_err(err, LBO_NON_FINITE_VALUE, 0, 0, 0, 0, f32_bits(coef), 4);
    size_t hidden = e->gate.rows;
    float *g = s->act, *u = s->act + hidden;
    int st = lbo_gemv(ex, &e->gate, input, e->gate.k, g, hidden, s->q8, s->q8_len, err);
    if (st) return st;
    st = lbo_gemv(ex, &e->up, input, e->up.k, u, hidden, s->q8, s->q8_len, err);
    if (st) return st;
    int64_t bad = lbo_apply_swiglu(g, u, hidden);
    if (bad >= 0) return set_err(err, LBO_NON_FINITE_VALUE, 0, (uint64_t)bad, 0, 0, f32_bits(g[bad]), 5);
    if (accumulate)
        return lbo_gemv_accumulate(ex, &e->down, g, hidden, out, e->down.rows, coef, s->q8, s->q8_len, err);
    return lbo_gemv(ex, &e->down, g, hidden, out, e->down.rows, s->q8, s->q8_len, err);
}

/* moe_routed_by_id_into (moe.rs:64-147). */
int lbo_moe_routed_by_id(const lbo_exec *ex, const uint32_t *ids, const float *coefs,
                         size_t n_routed, const lbo_expert *experts, size_t n_experts,
                         const lbo_expert *shared, const float *input, float *output, int preflight,
                         lbo_error *err) {
    if (n_routed == 0) return set_err(err, LBO_DIMENSION_MISMATCH, 0, 3, 1, 0, 0, 0);
    size_t width = shared->gate.k, out_w = shared->down.rows;
    size_t max_hidden = shared->gate.rows;
    for (size_t i = 0; i < n_routed; ++i)
        if (ids[i] < n_experts && experts[ids[i]].gate.rows > max_hidden) max_hidden = experts[ids[i]].gate.rows;
    size_t max_k = width > max_hidden ? width : max_hidden;
    swiglu_scratch s;
    s.act = (float *)malloc(sizeof(float) * 2 * max_hidden);
    s.q8_len = max_k / 256 * 292;
    s.q8 = (uint8_t *)malloc(s.q8_len ? s.q8_len : 1);
    float *pre = (float *)malloc(sizeof(float) * out_w);
    int st = LBO_OK;
    int64_t prev = -1;
    for (size_t i = 0; i < n_routed && !st; ++i) {
        if (!f32_finite(coefs[i])) {
            st = set_err(err, LBO_NON_FINITE_VALUE, 0, 0, 0, 0, f32_bits(coefs[i]), 6);
            break;
        }
        if (prev >= 0 && ids[i] == (uint32_t)prev) {
            st = set_err(err, LBO_DUPLICATE_ROUTED_EXPERT, 0, ids[i], 0, 0, 0, 0);
            break;
        }
        if (prev >= 0 && ids[i] < (uint32_t)prev) {
            st = set_err(err, LBO_ROUTED_EXPERT_ORDER, 0, ids[i], (uint64_t)prev, ids[i], 0, 0);
            break;
        }
        prev = ids[i];
        if (ids[i] >= n_experts) {
            st = set_err(err, LBO_INVALID_PARAMETER, 0, ids[i], 0, 0, 0, 0);
            break;
        }
        const lbo_expert *e = &experts[ids[i]];
        if (e->gate.k != width || e->down.rows != out_w) {
            st = set_err(err, LBO_DIMENSION_MISMATCH, 0, 4, width, e->gate.k, 0, 0);
            break;
        }
        if (preflight) st = swiglu_expert(ex, e, input, pre, 0, 0.0f, &s, err);
    }
    if (!st && preflight) st = swiglu_expert(ex, shared, input, pre, 0, 0.0f, &s, err);
    if (!st) {
        for (size_t r = 0; r < out_w; ++r) output[r] = 0.0f;
        for (size_t i = 0; i < n_routed && !st; ++i)
            st = swiglu_expert(ex, &experts[ids[i]], input, output, 1, coefs[i], &s, err);
        if (!st) st = swiglu_expert(ex, shared, input, output, 1, 1.0f, &s, err);
    }
    free(s.act);
    free(s.q8);
    free(pre);
    return st;
}

/* --------------------------------------------------------------- routers */

typedef struct cand {
    uint32_t id;
    float score;
    float weight;
} cand;

static int cand_cmp(const void *a, const void *b) {
    const cand *x = (const cand *)a, *y = (const cand *)b;
    if (x->score > y->score) return -1;
    if (x->score < y->score) return 1;
    return x->id < y->id ? -1 : (x->id > y->id ? 1 : 0);
}

static int id_cmp(const void *a, const void *b) {
    const cand *x = (const cand *)a, *y = (const cand *)b;
    return x->id < y->id ? -1 : (x->id > y->id ? 1 : 0);
}

static inline float sigmoidf_ref(float v) { return 1.0f / (1.0f + expf(-v)); }

/* route_experts_into (routing.rs:25-107) and sigmoid (routing.rs:109-111). */
int lbo_route_sigmoid_bias(const float *logits, const float *bias, size_t n, size_t k, float wscale,
                           uint32_t *ids, float *coefs, lbo_error *err) {
    if (k == 0 || k > n) return set_err(err, LBO_INVALID_PARAMETER, 0, k, n, k, 0, 0);
    if (!f32_finite(wscale)) return set_err(err, LBO_NON_FINITE_VALUE, 0, 0, 0, 0, f32_bits(wscale), 7);
    for (size_t i = 0; i < n; ++i) {
        if (!f32_finite(logits[i])) return set_err(err, LBO_NON_FINITE_VALUE, 0, i, 0, 0, f32_bits(logits[i]), 8);
        if (!f32_finite(bias[i])) return set_err(err, LBO_NON_FINITE_VALUE, 0, i, 0, 0, f32_bits(bias[i]), 9);
        float sc = sigmoidf_ref(logits[i]) + bias[i];
        if (!f32_finite(sc)) return set_err(err, LBO_NON_FINITE_VALUE, 0, i, 0, 0, f32_bits(sc), 10);
    }
    cand *c = (cand *)malloc(sizeof(cand) * n);
    for (size_t i = 0; i < n; ++i) {
        float w = sigmoidf_ref(logits[i]);
        c[i].id = (uint32_t)i;
        c[i].weight = w;
        c[i].score = w + bias[i];
    }
    qsort(c, n, sizeof(cand), cand_cmp);
    float sum = 0.0f;
    for (size_t i = 0; i < k; ++i) sum += c[i].weight;
    const float floor_ = 0.000061035156f; /* 2^-14, routing.rs:5 */
    if (!(sum >= floor_)) sum = floor_;
    for (size_t i = 0; i < k; ++i) c[i].score = c[i].weight / sum * wscale;
    qsort(c, k, sizeof(cand), id_cmp);
    for (size_t i = 0; i < k; ++i) {
        ids[i] = c[i].id;
        coefs[i] = c[i].score;
    }
    free(c);
    return LBO_OK;
}

int lbo_route_softmax_topk(const float *logits, size_t n, size_t k, uint32_t *ids, float *coefs,
                           lbo_error *err) {
    if (k == 0 || k > n) return set_err(err, LBO_INVALID_PARAMETER, 0, k, n, k, 0, 0);
    for (size_t i = 0; i < n; ++i)
        if (!f32_finite(logits[i])) return set_err(err, LBO_NON_FINITE_VALUE, 0, i, 0, 0, f32_bits(logits[i]), 8);
    cand *c = (cand *)malloc(sizeof(cand) * n);
    for (size_t i = 0; i < n; ++i) {
        c[i].id = (uint32_t)i;
        c[i].score = logits[i];
    }
    qsort(c, n, sizeof(cand), cand_cmp);
    float m = c[0].score;
    float sum = 0.0f;
    for (size_t i = 0; i < k; ++i) {
        c[i].weight = expf(c[i].score - m);
        sum += c[i].weight;
    }
    for (size_t i = 0; i < k; ++i) c[i].score = c[i].weight / sum;
    qsort(c, k, sizeof(cand), id_cmp);
    for (size_t i = 0; i < k; ++i) {
        ids[i] = c[i].id;
        coefs[i] = c[i].score;
    }
    free(c);
    return LBO_OK;
}
