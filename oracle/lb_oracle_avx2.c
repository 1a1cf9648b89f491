/*
 * lb_oracle_avx2.c — restatement of the reference's AVX2 dot kernels
 * (crates/bridge-quant-layout/src/q8_k.rs:436-731), used as the timed CPU
 * baseline.  TEST INFRASTRUCTURE ONLY.
 *
 * Same integer decomposition as the scalar path (lane l of lane_sums_i8_32
 * accumulates products p[l], p[8+l], p[16+l], p[24+l]) and the same f32 fold,
 * so results are bit-identical to lb_oracle.c's scalar dots; the tests assert
 * that on seeded random rows.  Built with -mavx2 -mfma -ffp-contract=off.
 */
#include <immintrin.h>
#include <string.h>

#include "lb_oracle.h"
#include "../lightbridge-engine_amd/csrc/lbh_iq_grids.inc"

static const uint64_t IQ2S_GRID_A[1024] = {LBH_IQ2S_GRID_VALUES};
static const uint32_t IQ3S_GRID_A[512] = {LBH_IQ3S_GRID_VALUES};

float lbo_f16_to_f32(uint16_t h);

static inline uint16_t rd_u16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline float rd_f32(const uint8_t *p) {
    float f;
    memcpy(&f, p, 4);
    return f;
}
static inline float rd_f16(const uint8_t *p) { return lbo_f16_to_f32(rd_u16(p)); }

/* lane_sums_i8_32 (q8_k.rs:668-699). */
static inline void lane_sums_i8_32(const int8_t *w, const uint8_t *a, int32_t out[8]) {
    __m256i acc = _mm256_setzero_si256();
    for (int off = 0; off < 32; off += 16) {
        __m128i w8 = _mm_loadu_si128((const __m128i *)(w + off));
        __m128i a8 = _mm_loadu_si128((const __m128i *)(a + off));
        __m256i p16 = _mm256_mullo_epi16(_mm256_cvtepi8_epi16(w8), _mm256_cvtepi8_epi16(a8));
        acc = _mm256_add_epi32(acc, _mm256_cvtepi16_epi32(_mm256_castsi256_si128(p16)));
        acc = _mm256_add_epi32(acc, _mm256_cvtepi16_epi32(_mm256_extracti128_si256(p16, 1)));
    }
    _mm256_storeu_si256((__m256i *)out, acc);
}

/* dot_i8_32 (q8_k.rs:701-706). */
static inline int32_t dot_i8_32(const int8_t *w, const uint8_t *a) {
    int32_t l[8];
    lane_sums_i8_32(w, a, l);
    return l[0] + l[1] + l[2] + l[3] + l[4] + l[5] + l[6] + l[7];
}

/* dot_i8_16 (q8_k.rs:708-731). */
static inline int32_t dot_i8_16(const int8_t *w, const uint8_t *a) {
    __m128i w8 = _mm_loadu_si128((const __m128i *)w);
    __m128i a8 = _mm_loadu_si128((const __m128i *)a);
    __m256i p16 = _mm256_mullo_epi16(_mm256_cvtepi8_epi16(w8), _mm256_cvtepi8_epi16(a8));
    __m256i pairs = _mm256_madd_epi16(p16, _mm256_set1_epi16(1));
    int32_t l[8];
    _mm256_storeu_si256((__m256i *)l, pairs);
    return l[0] + l[1] + l[2] + l[3] + l[4] + l[5] + l[6] + l[7];
}

static inline void scale_min(const uint8_t *sc, int j, uint8_t *s, uint8_t *m) {
    if (j < 4) {
        *s = sc[j] & 63;
        *m = sc[j + 4] & 63;
    } else {
        *s = (uint8_t)((sc[j + 4] & 0x0f) | ((sc[j - 4] >> 6) << 4));
        *m = (uint8_t)((sc[j + 4] >> 4) | ((sc[j] >> 6) << 4));
    }
}

/* dot_q4_or_q5_k_avx2 (q8_k.rs:457-542). */
static float dot_kquant_avx2(int ty, const uint8_t *w, const uint8_t *q8, size_t blocks) {
    size_t bb = ty == LBO_Q4_K ? 144 : 176;
    float sums[8] = {0};
    float sum = 0.0f;
    for (size_t b = 0; b < blocks; ++b) {
        const uint8_t *blk = w + b * bb;
        const uint8_t *a = q8 + b * 292;
        int8_t q[256];
        if (ty == LBO_Q4_K) {
            for (int g = 0; g < 4; ++g)
                for (int l = 0; l < 32; ++l) {
                    uint8_t p = blk[16 + 32 * g + l];
                    q[64 * g + l] = (int8_t)(p & 0x0f);
                    q[64 * g + 32 + l] = (int8_t)(p >> 4);
                }
        } else {
            uint8_t lo = 1, hi = 2;
            for (int g = 0; g < 4; ++g) {
                for (int l = 0; l < 32; ++l) {
                    uint8_t p = blk[48 + 32 * g + l];
                    uint8_t h = blk[16 + l];
                    q[64 * g + l] = (int8_t)((p & 0x0f) + ((h & lo) ? 16 : 0));
                    q[64 * g + 32 + l] = (int8_t)((p >> 4) + ((h & hi) ? 16 : 0));
                }
                lo <<= 2;
                hi <<= 2;
            }
        }
        uint8_t sc[8], mn[8];
        for (int j = 0; j < 8; ++j) scale_min(blk + 4, j, &sc[j], &mn[j]);
        int32_t ms = 0;
        for (int g = 0; g < 16; ++g) ms += (int32_t)(int16_t)rd_u16(a + 260 + 2 * g) * (int32_t)mn[g / 2];
        int32_t lanes[8] = {0};
        for (int j = 0; j < 8; ++j) {
            int32_t raw[8];
            lane_sums_i8_32(q + 32 * j, a + 4 + 32 * j, raw);
            for (int l = 0; l < 8; ++l) lanes[l] += (int32_t)sc[j] * raw[l];
        }
        float d8 = rd_f32(a);
        float scale = rd_f16(blk) * d8;
        for (int l = 0; l < 8; ++l) sums[l] += scale * (float)lanes[l];
        float mscale = rd_f16(blk + 2) * d8;
        sum -= mscale * (float)ms;
    }
    for (int l = 0; l < 8; ++l) sum += sums[l];
    return sum;
}

/* dot_iq2_s_avx2 (q8_k.rs:544-601). */
static float dot_iq2s_avx2(const uint8_t *w, const uint8_t *q8, size_t blocks) {
    float sum = 0.0f;
    for (size_t b = 0; b < blocks; ++b) {
        const uint8_t *blk = w + b * 82;
        const uint8_t *a = q8 + b * 292;
        float scale = rd_f16(blk) * rd_f32(a);
        int32_t bsum = 0;
        for (int g = 0; g < 8; ++g) {
            uint8_t ps = blk[74 + g];
            int32_t s1 = 1 + 2 * (ps & 0x0f), s2 = 1 + 2 * (ps >> 4);
            uint32_t hi = blk[66 + g];
            int8_t sg[32];
            for (int lg = 0; lg < 4; ++lg) {
                uint32_t idx = blk[2 + 4 * g + lg] | ((hi << (8 - 2 * lg)) & 0x300);
                uint64_t grid = IQ2S_GRID_A[idx];
                uint8_t signs = blk[34 + 4 * g + lg];
                for (int l = 0; l < 8; ++l) {
                    int8_t mag = (int8_t)((grid >> (8 * l)) & 0xff);
                    sg[8 * lg + l] = ((signs >> l) & 1) ? (int8_t)-mag : mag;
                }
            }
            const uint8_t *ag = a + 4 + 32 * g;
            bsum += s1 * dot_i8_16(sg, ag) + s2 * dot_i8_16(sg + 16, ag + 16);
        }
        sum += scale * (float)bsum;
    }
    return 0.125f * sum;
}

/* dot_iq3_s_avx2 (q8_k.rs:603-666). */
static float dot_iq3s_avx2(const uint8_t *w, const uint8_t *q8, size_t blocks) {
    float sum = 0.0f;
    for (size_t b = 0; b < blocks; ++b) {
        const uint8_t *blk = w + b * 110;
        const uint8_t *a = q8 + b * 292;
        float scale = rd_f16(blk) * rd_f32(a);
        int32_t bsum = 0;
        for (int p = 0; p < 4; ++p) {
            uint8_t ps = blk[106 + p];
            int32_t pscale[2] = {2 * (ps & 0x0f) + 1, 2 * (ps >> 4) + 1};
            for (int h = 0; h < 2; ++h) {
                int g = 2 * p + h;
                uint32_t hi = blk[66 + g];
                int8_t sg[32];
                for (int lg = 0; lg < 4; ++lg) {
                    uint32_t i1 = blk[2 + 8 * g + 2 * lg] | ((hi << (8 - 2 * lg)) & 0x100);
                    uint32_t i2 = blk[2 + 8 * g + 2 * lg + 1] | ((hi << (7 - 2 * lg)) & 0x100);
                    uint32_t g1 = IQ3S_GRID_A[i1], g2 = IQ3S_GRID_A[i2];
                    uint8_t signs = blk[74 + 4 * g + lg];
                    for (int l = 0; l < 4; ++l) {
                        int8_t m1 = (int8_t)((g1 >> (8 * l)) & 0xff);
                        int8_t m2 = (int8_t)((g2 >> (8 * l)) & 0xff);
                        sg[8 * lg + l] = ((signs >> l) & 1) ? (int8_t)-m1 : m1;
                        sg[8 * lg + l + 4] = ((signs >> (l + 4)) & 1) ? (int8_t)-m2 : m2;
                    }
                }
                bsum += dot_i8_32(sg, a + 4 + 32 * g) * pscale[h];
            }
        }
        sum += scale * (float)bsum;
    }
    return sum;
}

/* dot_avx2 (q8_k.rs:436-455). */
float lbo_dot_avx2(int ty, const uint8_t *w, const uint8_t *q8, size_t blocks) {
    switch (ty) {
    case LBO_Q4_K:
    case LBO_Q5_K: return dot_kquant_avx2(ty, w, q8, blocks);
    case LBO_IQ2_S: return dot_iq2s_avx2(w, q8, blocks);
    case LBO_IQ3_S: return dot_iq3s_avx2(w, q8, blocks);
    default: return 0.0f;
    }
}
