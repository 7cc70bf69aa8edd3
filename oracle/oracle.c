/*
 * CPU oracle for the whisper.go decoder token loop — TEST INFRASTRUCTURE ONLY.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it,
 * to check and time against. Restates the reference (github.com/whispergo/whisper.go);
 * every function cites the file:line it follows. See oracle.h for what pins
 * each part and what stays "parity unpinned".
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no -ffast-math).
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <ctype.h>

static __thread char g_err[512];
static void set_err(const char *msg) { snprintf(g_err, sizeof g_err, "%s", msg); }
const char *or_last_error(void) { return g_err; }

static float bits_f32(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static uint32_t f32_bits(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }

/* gguf/dequant.go:15-44 (identical to ml/matmul_q8.go:759-781) */
float or_f16_to_f32(uint16_t h) {
    uint32_t s = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 0x1F;
    uint32_t m = h & 0x3FF;
    if (e == 0) {
        if (m == 0) return bits_f32(s);
        uint32_t k = 1;
        m <<= 1;
        while ((m & 0x400) == 0) { m <<= 1; k++; }
        m &= 0x3FF;
        return bits_f32(s | ((113 - k) << 23) | (m << 13));
    }
    if (e == 31) return bits_f32(s | 0x7F800000u | (m << 13));
    return bits_f32(s | ((e + 112) << 23) | (m << 13));
}

/* gguf/quant.go:11-55: round half-up on mantissa bit 12, subnormal f32 -> 0 */
uint16_t or_f32_to_f16(float f) {
    uint32_t bits = f32_bits(f);
    uint16_t sign = (uint16_t)(bits >> 31);
    int exp = (int)(bits >> 23) & 0xFF;
    uint32_t mant = bits & 0x7FFFFF;
    if (exp == 255) return mant != 0 ? (uint16_t)(sign << 15 | 0x7E00) : (uint16_t)(sign << 15 | 0x7C00);
    if (exp == 0) return (uint16_t)(sign << 15);
    int exp16 = exp - 127 + 15;
    if (exp16 >= 31) return (uint16_t)(sign << 15 | 0x7C00);
    if (exp16 <= 0) {
        if (exp16 < -10) return (uint16_t)(sign << 15);
        unsigned shift = (unsigned)(1 - exp16);
        uint16_t mant16 = (uint16_t)((mant | 0x800000) >> (13 + shift));
        return (uint16_t)(sign << 15 | mant16);
    }
    uint16_t mant16 = (uint16_t)(mant >> 13);
    if ((mant >> 12) & 1) mant16++;
    if (mant16 >= 0x400) {
        mant16 = 0;
        exp16++;
        if (exp16 >= 31) return (uint16_t)(sign << 15 | 0x7C00);
    }
    return (uint16_t)(sign << 15 | (uint16_t)exp16 << 10 | mant16);
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static uint32_t rd32(const uint8_t *p) {
    return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
}

/* gguf/tensor.go:60-85 */
size_t or_row_bytes(uint32_t type, size_t n) {
    size_t b = (n + 31) / 32;
    switch (type) {
    case 0: return n * 4;
    case 1: return n * 2;
    case 2: return b * 18;
    case 3: return b * 20;
    case 6: return b * 22;
    case 7: return b * 24;
    case 8: return b * 34;
    default: return 0;
    }
}

/* gguf/dequant.go:47-201 */
int or_dequantize(const uint8_t *raw, uint32_t type, size_t n, float *out) {
    size_t nb = (n + 31) / 32;
    switch (type) {
    case 0:
        for (size_t i = 0; i < n; i++) out[i] = bits_f32(rd32(raw + 4 * i));
        return 0;
    case 1:
        for (size_t i = 0; i < n; i++) out[i] = or_f16_to_f32(rd16(raw + 2 * i));
        return 0;
    case 2: /* dequant.go:92-108 */
        for (size_t b = 0; b < nb; b++) {
            const uint8_t *blk = raw + b * 18;
            float scale = or_f16_to_f32(rd16(blk));
            const uint8_t *qs = blk + 2;
            size_t base = b * 32;
            for (int i = 0; i < 16; i++) {
                size_t j = base + 2 * i;
                if (j < n) out[j] = scale * (float)((int32_t)(qs[i] & 0xF) - 8);
                if (j + 1 < n) out[j + 1] = scale * (float)((int32_t)(qs[i] >> 4) - 8);
            }
        }
        return 0;
    case 3: /* dequant.go:113-130 */
        for (size_t b = 0; b < nb; b++) {
            const uint8_t *blk = raw + b * 20;
            float d = or_f16_to_f32(rd16(blk));
            float m = or_f16_to_f32(rd16(blk + 2));
            const uint8_t *qs = blk + 4;
            size_t base = b * 32;
            for (int i = 0; i < 16; i++) {
                size_t j = base + 2 * i;
                if (j < n) out[j] = d * (float)(qs[i] & 0xF) + m;
                if (j + 1 < n) out[j + 1] = d * (float)(qs[i] >> 4) + m;
            }
        }
        return 0;
    case 6: /* dequant.go:135-156 */
        for (size_t b = 0; b < nb; b++) {
            const uint8_t *blk = raw + b * 22;
            float scale = or_f16_to_f32(rd16(blk));
            uint32_t qh = rd32(blk + 2);
            const uint8_t *qs = blk + 6;
            size_t base = b * 32;
            for (int i = 0; i < 16; i++) {
                uint32_t hi0 = (qh >> (2 * i)) & 1, hi1 = (qh >> (2 * i + 1)) & 1;
                int32_t v0 = (int32_t)((uint32_t)(qs[i] & 0xF) | (hi0 << 4)) - 16;
                int32_t v1 = (int32_t)((uint32_t)(qs[i] >> 4) | (hi1 << 4)) - 16;
                size_t j = base + 2 * i;
                if (j < n) out[j] = scale * (float)v0;
                if (j + 1 < n) out[j + 1] = scale * (float)v1;
            }
        }
        return 0;
    case 7: /* dequant.go:161-183 */
        for (size_t b = 0; b < nb; b++) {
            const uint8_t *blk = raw + b * 24;
            float d = or_f16_to_f32(rd16(blk));
            float m = or_f16_to_f32(rd16(blk + 2));
            uint32_t qh = rd32(blk + 4);
            const uint8_t *qs = blk + 8;
            size_t base = b * 32;
            for (int i = 0; i < 16; i++) {
                uint32_t hi0 = (qh >> (2 * i)) & 1, hi1 = (qh >> (2 * i + 1)) & 1;
                float v0 = (float)((uint32_t)(qs[i] & 0xF) | (hi0 << 4));
                float v1 = (float)((uint32_t)(qs[i] >> 4) | (hi1 << 4));
                size_t j = base + 2 * i;
                if (j < n) out[j] = d * v0 + m;
                if (j + 1 < n) out[j + 1] = d * v1 + m;
            }
        }
        return 0;
    case 8: /* dequant.go:188-201 */
        for (size_t b = 0; b < nb; b++) {
            const uint8_t *blk = raw + b * 34;
            float scale = or_f16_to_f32(rd16(blk));
            size_t base = b * 32;
            for (int i = 0; i < 32; i++)
                if (base + i < n) out[base + i] = scale * (float)(int8_t)blk[2 + i];
        }
        return 0;
    default:
        set_err("oracle: dequantize: unsupported dtype");
        return -1;
    }
}

/* ---- quantizers: gguf/quant.go:87-232 and helpers :252-376 ---------------- */
static void put_f16(uint8_t *dst, float f) {
    uint16_t h = or_f32_to_f16(f);
    dst[0] = (uint8_t)h;
    dst[1] = (uint8_t)(h >> 8);
}
static float blk_at(const float *blk, int len, int i) { return i < len ? blk[i] : 0.0f; }
static int32_t go_round_i32(float q) { return (int32_t)round((double)q); } /* math.Round: half away from zero */

static uint8_t quant_nibble(const float *blk, int len, int i, float scale, int32_t bias) { /* :284-299 */
    float v = blk_at(blk, len, i);
    int32_t q = bias;
    if (scale != 0) q = go_round_i32(v / scale) + bias;
    if (q < 0) q = 0;
    if (q > 15) q = 15;
    return (uint8_t)q;
}
static uint8_t quant_nibble_unsigned(const float *blk, int len, int i, float scale, float mn) { /* :302-317 */
    float v = blk_at(blk, len, i);
    int32_t q = 0;
    if (scale != 0) q = go_round_i32((v - mn) / scale);
    if (q < 0) q = 0;
    if (q > 15) q = 15;
    return (uint8_t)q;
}
static uint8_t quant5_signed(const float *blk, int len, int i, float scale, int32_t bias) { /* :320-335 */
    float v = blk_at(blk, len, i);
    int32_t q = bias;
    if (scale != 0) q = go_round_i32(v / scale) + bias;
    if (q < 0) q = 0;
    if (q > 31) q = 31;
    return (uint8_t)q;
}
static uint8_t quant5_unsigned(const float *blk, int len, int i, float scale, float mn) { /* :338-353 */
    float v = blk_at(blk, len, i);
    int32_t q = 0;
    if (scale != 0) q = go_round_i32((v - mn) / scale);
    if (q < 0) q = 0;
    if (q > 31) q = 31;
    return (uint8_t)q;
}
static void nibble_set(uint8_t *dst, int i, uint8_t v) { /* :356-362 */
    if (i % 2 == 0) dst[i / 2] = (uint8_t)((dst[i / 2] & 0xF0) | (v & 0xF));
    else dst[i / 2] = (uint8_t)((dst[i / 2] & 0x0F) | ((v & 0xF) << 4));
}
static float block_absmax(const float *blk, int len) {
    float a = 0;
    for (int i = 0; i < len; i++) {
        float v = fabsf(blk[i]);
        if (v > a) a = v;
    }
    return a;
}
static void block_minmax(const float *blk, int len, float *mn, float *mx) { /* :261-276 */
    if (len == 0) { *mn = 0; *mx = 0; return; }
    *mn = blk[0]; *mx = blk[0];
    for (int i = 1; i < len; i++) {
        if (blk[i] < *mn) *mn = blk[i];
        if (blk[i] > *mx) *mx = blk[i];
    }
}

size_t or_quantize(const float *src, size_t n, uint32_t type, uint8_t *dst) {
    size_t nb = (n + 31) / 32;
    size_t bytes = or_row_bytes(type, n);
    if (bytes == 0) { set_err("oracle: quantize: unsupported type"); return 0; }
    memset(dst, 0, bytes);
    if (type == 0) { memcpy(dst, src, n * 4); return bytes; }
    if (type == 1) { for (size_t i = 0; i < n; i++) put_f16(dst + 2 * i, src[i]); return bytes; }
    for (size_t b = 0; b < nb; b++) {
        const float *blk = src + b * 32;
        int len = (int)((n - b * 32) < 32 ? (n - b * 32) : 32);
        if (type == 2) { /* QuantizeQ4_0 :87-109 */
            float scale = block_absmax(blk, len) / 7.0f;
            uint8_t *ob = dst + b * 18;
            put_f16(ob, scale);
            for (int i = 0; i < 16; i++) {
                uint8_t lo = quant_nibble(blk, len, 2 * i, scale, 8);
                uint8_t hi = quant_nibble(blk, len, 2 * i + 1, scale, 8);
                ob[2 + i] = (uint8_t)(lo | (hi << 4));
            }
        } else if (type == 3) { /* QuantizeQ4_1 :113-131 */
            float mn, mx;
            block_minmax(blk, len, &mn, &mx);
            float scale = (mx - mn) / 15.0f;
            uint8_t *ob = dst + b * 20;
            put_f16(ob, scale);
            put_f16(ob + 2, mn);
            for (int i = 0; i < 16; i++) {
                uint8_t lo = quant_nibble_unsigned(blk, len, 2 * i, scale, mn);
                uint8_t hi = quant_nibble_unsigned(blk, len, 2 * i + 1, scale, mn);
                ob[4 + i] = (uint8_t)(lo | (hi << 4));
            }
        } else if (type == 6) { /* QuantizeQ5_0 :135-168 */
            float scale = block_absmax(blk, len) / 15.0f;
            uint8_t *ob = dst + b * 22;
            put_f16(ob, scale);
            uint32_t qh = 0;
            for (int i = 0; i < 32; i++) {
                uint8_t q = quant5_signed(blk, len, i, scale, 16);
                if ((q >> 4) & 1) qh |= 1u << i;
                nibble_set(ob + 6, i, (uint8_t)(q & 0xF));
            }
            ob[2] = (uint8_t)qh; ob[3] = (uint8_t)(qh >> 8); ob[4] = (uint8_t)(qh >> 16); ob[5] = (uint8_t)(qh >> 24);
        } else if (type == 7) { /* QuantizeQ5_1 :172-198 */
            float mn, mx;
            block_minmax(blk, len, &mn, &mx);
            float scale = (mx - mn) / 31.0f;
            uint8_t *ob = dst + b * 24;
            put_f16(ob, scale);
            put_f16(ob + 2, mn);
            uint32_t qh = 0;
            for (int i = 0; i < 32; i++) {
                uint8_t q = quant5_unsigned(blk, len, i, scale, mn);
                if ((q >> 4) & 1) qh |= 1u << i;
                nibble_set(ob + 8, i, (uint8_t)(q & 0xF));
            }
            ob[4] = (uint8_t)qh; ob[5] = (uint8_t)(qh >> 8); ob[6] = (uint8_t)(qh >> 16); ob[7] = (uint8_t)(qh >> 24);
        } else if (type == 8) { /* QuantizeQ8_0 :202-232 */
            float scale = block_absmax(blk, len) / 127.0f;
            uint8_t *ob = dst + b * 34;
            put_f16(ob, scale);
            for (int i = 0; i < 32; i++) {
                float v = blk_at(blk, len, i);
                int32_t q = 0;
                if (scale != 0) {
                    q = go_round_i32(v / scale);
                    if (q < -127) q = -127; /* clampI8 :368-376 */
                    if (q > 127) q = 127;
                }
                ob[2 + i] = (uint8_t)(int8_t)q;
            }
        }
    }
    return bytes;
}

/* gguf/quant.go:236-248 */
int or_should_quantize(const char *name) {
    size_t n = strlen(name);
    char *lower = (char *)malloc(n + 1);
    for (size_t i = 0; i <= n; i++) lower[i] = (char)tolower((unsigned char)name[i]);
    int r;
    if (strstr(lower, "norm") || strstr(lower, ".ln")) r = 0;
    else if (n >= 5 && strcmp(lower + n - 5, ".bias") == 0) r = 0;
    else r = (n >= 7 && strcmp(lower + n - 7, ".weight") == 0);
    free(lower);
    return r;
}

/* ---- dot kernels ----------------------------------------------------------- */
/* ml/dot_int8_f32_avx2_amd64.s:4-45: 8 lanes x 4 products, fold, 2x hadd */
static float avx2_dot32(const int8_t *q, const float *f) {
    float acc[8];
    for (int l = 0; l < 8; l++) acc[l] = 0.0f + (float)q[l] * f[l];
    for (int c = 1; c < 4; c++)
        for (int l = 0; l < 8; l++) acc[l] = acc[l] + (float)q[8 * c + l] * f[8 * c + l];
    float t0 = acc[0] + acc[4], t1 = acc[1] + acc[5], t2 = acc[2] + acc[6], t3 = acc[3] + acc[7];
    return (t0 + t1) + (t2 + t3);
}

/* ml/matmul_q8.go:679-744 */
static float gen_q8_block(float scale, const uint8_t *q, const float *f) {
    float s0 = 0, s1 = 0, s2 = 0, s3 = 0;
    for (int i = 0; i < 32; i += 8) {
        s0 += (float)(int8_t)q[i + 0] * f[i + 0];
        s1 += (float)(int8_t)q[i + 1] * f[i + 1];
        s2 += (float)(int8_t)q[i + 2] * f[i + 2];
        s3 += (float)(int8_t)q[i + 3] * f[i + 3];
        s0 += (float)(int8_t)q[i + 4] * f[i + 4];
        s1 += (float)(int8_t)q[i + 5] * f[i + 5];
        s2 += (float)(int8_t)q[i + 6] * f[i + 6];
        s3 += (float)(int8_t)q[i + 7] * f[i + 7];
    }
    return scale * (s0 + s1 + s2 + s3);
}

static float dot_f32(const float *w, const float *x, int n) {
    float s = 0;
    for (int i = 0; i < n; i++) s += w[i] * x[i];
    return s;
}

float or_dot(uint32_t type, const uint8_t *q, const float *f, int n, int variant) {
    float sum = 0;
    if (n <= 0) return 0;
    int nb = (n + 31) / 32;
    if (type == 0) return dot_f32((const float *)q, f, n);
    for (int b = 0; b < nb; b++) {
        int base = b * 32, rem = n - base;
        if (type == 8) { /* matmul_q8.go:395-429 ; kernels_amd64.go:15-42 */
            const uint8_t *blk = q + b * 34;
            float scale = or_f16_to_f32(rd16(blk));
            if (rem >= 32) {
                if (variant) sum += scale * avx2_dot32((const int8_t *)(blk + 2), f + base);
                else sum += gen_q8_block(scale, blk + 2, f + base);
                continue;
            }
            for (int i = 0; i < rem; i++) sum += scale * (float)(int8_t)blk[2 + i] * f[base + i];
        } else if (type == 2) { /* matmul_q8.go:237-268 ; kernels_amd64.go:44-82 */
            const uint8_t *blk = q + b * 18;
            float d = or_f16_to_f32(rd16(blk));
            const uint8_t *qs = blk + 2;
            if (rem >= 32) {
                if (variant) {
                    int8_t tmp[32];
                    for (int i = 0; i < 16; i++) {
                        tmp[2 * i] = (int8_t)(uint8_t)((qs[i] & 0x0F) - 8);
                        tmp[2 * i + 1] = (int8_t)(uint8_t)((qs[i] >> 4) - 8);
                    }
                    sum += d * avx2_dot32(tmp, f + base);
                } else {
                    float s = 0; /* dotQ40Block32 :693-702 */
                    for (int i = 0; i < 16; i++) {
                        s += (float)((int32_t)(qs[i] & 0xF) - 8) * f[base + 2 * i];
                        s += (float)((int32_t)(qs[i] >> 4) - 8) * f[base + 2 * i + 1];
                    }
                    sum += d * s;
                }
                continue;
            }
            for (int i = 0; i < rem; i++) {
                int32_t qv = (i & 1) ? (int32_t)(qs[i >> 1] >> 4) - 8 : (int32_t)(qs[i >> 1] & 0xF) - 8;
                sum += d * (float)qv * f[base + i];
            }
        } else if (type == 3) { /* matmul_q8.go:274-306 ; kernels_amd64.go:84-128 */
            const uint8_t *blk = q + b * 20;
            float d = or_f16_to_f32(rd16(blk)), m = or_f16_to_f32(rd16(blk + 2));
            const uint8_t *qs = blk + 4;
            if (rem >= 32) {
                if (variant) {
                    int8_t tmp[32];
                    for (int i = 0; i < 16; i++) { tmp[2 * i] = (int8_t)(qs[i] & 0x0F); tmp[2 * i + 1] = (int8_t)(qs[i] >> 4); }
                    float s = avx2_dot32(tmp, f + base), fsum = 0;
                    for (int i = 0; i < 32; i++) fsum += f[base + i];
                    sum += d * s + m * fsum;
                } else {
                    float s = 0; /* dotQ41Block32 :704-713 */
                    for (int i = 0; i < 16; i++) {
                        s += (d * (float)(qs[i] & 0xF) + m) * f[base + 2 * i];
                        s += (d * (float)(qs[i] >> 4) + m) * f[base + 2 * i + 1];
                    }
                    sum += s;
                }
                continue;
            }
            for (int i = 0; i < rem; i++) {
                float qv = (i & 1) ? (float)(qs[i >> 1] >> 4) : (float)(qs[i >> 1] & 0xF);
                sum += (d * qv + m) * f[base + i];
            }
        } else if (type == 6) { /* matmul_q8.go:312-349 ; kernels_amd64.go:130-177 */
            const uint8_t *blk = q + b * 22;
            float d = or_f16_to_f32(rd16(blk));
            uint32_t qh = rd32(blk + 2);
            const uint8_t *qs = blk + 6;
            if (rem >= 32) {
                if (variant) {
                    int8_t tmp[32];
                    for (int i = 0; i < 16; i++) {
                        tmp[2 * i] = (int8_t)(uint8_t)(((qs[i] & 0x0F) | (uint8_t)(((qh >> (2 * i)) & 1) << 4)) - 16);
                        tmp[2 * i + 1] = (int8_t)(uint8_t)(((qs[i] >> 4) | (uint8_t)(((qh >> (2 * i + 1)) & 1) << 4)) - 16);
                    }
                    sum += d * avx2_dot32(tmp, f + base);
                } else {
                    float s = 0; /* dotQ50Block32 :715-728 */
                    for (int i = 0; i < 16; i++) {
                        uint32_t hi0 = (qh >> (2 * i)) & 1, hi1 = (qh >> (2 * i + 1)) & 1;
                        float v0 = (float)((int32_t)((uint32_t)(qs[i] & 0xF) | (hi0 << 4)) - 16);
                        float v1 = (float)((int32_t)((uint32_t)(qs[i] >> 4) | (hi1 << 4)) - 16);
                        s += d * v0 * f[base + 2 * i];
                        s += d * v1 * f[base + 2 * i + 1];
                    }
                    sum += s;
                }
                continue;
            }
            for (int i = 0; i < rem; i++) {
                uint32_t hi = (qh >> i) & 1;
                uint32_t low = (i & 1) ? (uint32_t)(qs[i >> 1] >> 4) : (uint32_t)(qs[i >> 1] & 0xF);
                float v = (float)((int32_t)(low | (hi << 4)) - 16);
                sum += d * v * f[base + i];
            }
        } else if (type == 7) { /* matmul_q8.go:355-391 ; kernels_amd64.go:179-224 */
            const uint8_t *blk = q + b * 24;
            float d = or_f16_to_f32(rd16(blk)), m = or_f16_to_f32(rd16(blk + 2));
            uint32_t qh = rd32(blk + 4);
            const uint8_t *qs = blk + 8;
            if (rem >= 32) {
                if (variant) {
                    int8_t tmp[32];
                    for (int i = 0; i < 16; i++) {
                        tmp[2 * i] = (int8_t)((qs[i] & 0x0F) | (uint8_t)(((qh >> (2 * i)) & 1) << 4));
                        tmp[2 * i + 1] = (int8_t)((qs[i] >> 4) | (uint8_t)(((qh >> (2 * i + 1)) & 1) << 4));
                    }
                    float s = avx2_dot32(tmp, f + base), fsum = 0;
                    for (int i = 0; i < 32; i++) fsum += f[base + i];
                    sum += d * s + m * fsum;
                } else {
                    float s = 0; /* dotQ51Block32 :730-743 */
                    for (int i = 0; i < 16; i++) {
                        uint32_t hi0 = (qh >> (2 * i)) & 1, hi1 = (qh >> (2 * i + 1)) & 1;
                        float v0 = (float)((uint32_t)(qs[i] & 0xF) | (hi0 << 4));
                        float v1 = (float)((uint32_t)(qs[i] >> 4) | (hi1 << 4));
                        s += (d * v0 + m) * f[base + 2 * i];
                        s += (d * v1 + m) * f[base + 2 * i + 1];
                    }
                    sum += s;
                }
                continue;
            }
            for (int i = 0; i < rem; i++) {
                uint32_t hi = (qh >> i) & 1;
                uint32_t low = (i & 1) ? (uint32_t)(qs[i >> 1] >> 4) : (uint32_t)(qs[i >> 1] & 0xF);
                float v = (float)(low | (hi << 4));
                sum += (d * v + m) * f[base + i];
            }
        } else {
            return NAN;
        }
    }
    return sum;
}

/* ---- GEMV with optional row-parallelism: ml/matmul_q8.go:93-196 ------------ */
typedef struct {
    uint32_t type; const uint8_t *w; int rows, cols; const float *a; float *out;
    int m0, m1, variant; size_t row_bytes;
} gemv_job;

static void *gemv_worker(void *p) {
    gemv_job *j = (gemv_job *)p;
    for (int i = j->m0; i < j->m1; i++)
        for (int r = 0; r < j->rows; r++)
            j->out[(size_t)i * j->rows + r] =
                or_dot(j->type, j->w + (size_t)r * j->row_bytes, j->a + (size_t)i * j->cols, j->cols, j->variant);
    return NULL;
}

/* One input row, output rows [m0, m1) of the matrix: the same dot per output
 * element as the serial loop, so the result does not depend on the split. Used
 * only to generate test fixtures faster (the reference's batch-1 GEMV is serial,
 * internal/ml/matmul_q8.go:110-118). */
static void *gemv_rows_worker(void *p) {
    gemv_job *j = (gemv_job *)p;
    for (int r = j->m0; r < j->m1; r++)
        j->out[r] = or_dot(j->type, j->w + (size_t)r * j->row_bytes, j->a, j->cols, j->variant);
    return NULL;
}

static void gemv1_split(uint32_t type, const uint8_t *w, int rows, int cols, const float *a, float *out, int variant,
                        int threads) {
    size_t rb = or_row_bytes(type, (size_t)cols);
    if (threads > 64) threads = 64;
    gemv_job jobs[64];
    pthread_t th[64];
    for (int t = 0; t < threads; t++)
        jobs[t] = (gemv_job){type, w, rows, cols, a, out, (t * rows) / threads, ((t + 1) * rows) / threads, variant, rb};
    for (int t = 0; t < threads; t++) pthread_create(&th[t], NULL, gemv_rows_worker, &jobs[t]);
    for (int t = 0; t < threads; t++) pthread_join(th[t], NULL);
}

int or_gemv(uint32_t type, const uint8_t *w, int rows, int cols, const float *a, int m, float *out,
            int variant, int threads) {
    size_t rb = or_row_bytes(type, (size_t)cols);
    if (rb == 0 && type != 0) { set_err("oracle: gemv: unsupported type"); return -1; }
    if (threads > m) threads = m;
    if (threads < 1) threads = 1;
    gemv_job jobs[256];
    pthread_t th[256];
    if (threads > 256) threads = 256;
    for (int t = 0; t < threads; t++) {
        jobs[t] = (gemv_job){type, w, rows, cols, a, out, (t * m) / threads, ((t + 1) * m) / threads, variant, rb};
    }
    if (threads == 1) { gemv_worker(&jobs[0]); return 0; }
    for (int t = 0; t < threads; t++) pthread_create(&th[t], NULL, gemv_worker, &jobs[t]);
    for (int t = 0; t < threads; t++) pthread_join(th[t], NULL);
    return 0;
}

/* ---- LayerNorm: ml/ops.go:153-202 ------------------------------------------ */
void or_layernorm(float *dst, const float *src, const float *w, const float *b, int rows, int c, float eps) {
    for (int r = 0; r < rows; r++) {
        const float *s = src + (size_t)r * c;
        float *d = dst + (size_t)r * c;
        float mean = 0;
        int i = 0;
        for (; i + 3 < c; i += 4) mean += s[i] + s[i + 1] + s[i + 2] + s[i + 3];
        for (; i < c; i++) mean += s[i];
        mean /= (float)c;
        float vari = 0;
        i = 0;
        for (; i + 3 < c; i += 4) {
            float d0 = s[i] - mean, d1 = s[i + 1] - mean, d2 = s[i + 2] - mean, d3 = s[i + 3] - mean;
            vari += d0 * d0 + d1 * d1 + d2 * d2 + d3 * d3;
        }
        for (; i < c; i++) { float dd = s[i] - mean; vari += dd * dd; }
        vari /= (float)c;
        float std = (float)sqrt((double)(vari + eps));
        for (i = 0; i < c; i++) {
            float v = s[i];
            d[i] = w[i] * (v - mean) / std + b[i];
        }
    }
}

/* ---- GELU (tanh form, tanh in float64): ml/ops.go:102-122 ------------------ */
void or_gelu(float *t, int n) {
    const float k = 0.7978845608028654f;
    for (int i = 0; i < n; i++) {
        float x = t[i];
        float inner = k * (x + 0.044715f * x * x * x);
        t[i] = x * 0.5f * (float)(1 + tanh((double)inner));
    }
}

/* ---- fast exp: ml/attention.go:34-61 --------------------------------------- */
float or_fast_exp(float x) {
    const float inv_ln2 = 1.4426950408889634f, ln2 = 0.6931471805599453f;
    if (x <= -20) return 0;
    float y = x * inv_ln2;
    int k = (int)y;
    if ((float)k > y) k--;
    float r = x - (float)k * ln2;
    float r2 = r * r, r3 = r2 * r, r4 = r3 * r;
    float poly = 1 + r + 0.5f * r2 + (float)(1.0 / 6.0) * r3 + (float)(1.0 / 24.0) * r4;
    if (k < -126) return 0;
    if (k > 127) return 3.40282346638528859811704183484516925440e+38f;
    float two_pow_k = bits_f32((uint32_t)(k + 127) << 23);
    return poly * two_pow_k;
}

/* ml/attention.go:63-91 */
static float row_max(const float *row, int n) {
    float m = row[0];
    for (int i = 1; i < n; i++) if (row[i] > m) m = row[i];
    return m;
}

/* ml/attention.go:93-131 */
void or_softmax_fast(float *row, int n) {
    float mx = row_max(row, n), sum = 0;
    int i = 0;
    for (; i + 3 < n; i += 4) {
        float x0 = or_fast_exp(row[i] - mx), x1 = or_fast_exp(row[i + 1] - mx);
        float x2 = or_fast_exp(row[i + 2] - mx), x3 = or_fast_exp(row[i + 3] - mx);
        row[i] = x0; row[i + 1] = x1; row[i + 2] = x2; row[i + 3] = x3;
        sum += x0 + x1 + x2 + x3;
    }
    for (; i < n; i++) { float x = or_fast_exp(row[i] - mx); row[i] = x; sum += x; }
    if (sum == 0) { float inv = 1.0f / (float)n; for (i = 0; i < n; i++) row[i] = inv; return; }
    float inv = 1 / sum;
    for (i = 0; i < n; i++) row[i] *= inv;
}

/* ml/attention.go:133-171 */
void or_softmax_exact(float *row, int n) {
    float mx = row_max(row, n), sum = 0;
    int i = 0;
    for (; i + 3 < n; i += 4) {
        float x0 = (float)exp((double)(row[i] - mx)), x1 = (float)exp((double)(row[i + 1] - mx));
        float x2 = (float)exp((double)(row[i + 2] - mx)), x3 = (float)exp((double)(row[i + 3] - mx));
        row[i] = x0; row[i + 1] = x1; row[i + 2] = x2; row[i + 3] = x3;
        sum += x0 + x1 + x2 + x3;
    }
    for (; i < n; i++) { float x = (float)exp((double)(row[i] - mx)); row[i] = x; sum += x; }
    if (sum == 0) { float inv = 1.0f / (float)n; for (i = 0; i < n; i++) row[i] = inv; return; }
    float inv = 1 / sum;
    for (i = 0; i < n; i++) row[i] *= inv;
}

/* ml/attention.go:193-281 (sgemm summation order is sequential here: unpinned) */
void or_sdpa(const float *q, const float *k, const float *v, int heads, int tq, int tk, int hd, int causal,
             int fast_exp, float *out, float *weights) {
    float scale = (float)(1.0 / sqrt((double)hd));
    float *scores = (float *)malloc(sizeof(float) * (size_t)tq * tk);
    for (int h = 0; h < heads; h++) {
        const float *qh = q + (size_t)h * tq * hd, *kh = k + (size_t)h * tk * hd, *vh = v + (size_t)h * tk * hd;
        for (int i = 0; i < tq; i++)
            for (int j = 0; j < tk; j++) scores[i * tk + j] = dot_f32(qh + (size_t)i * hd, kh + (size_t)j * hd, hd);
        for (int i = 0; i < tq * tk; i++) scores[i] *= scale;
        if (causal)
            for (int i = 0; i < tq; i++)
                for (int j = i + 1; j < tk; j++) scores[i * tk + j] = -INFINITY;
        for (int i = 0; i < tq; i++) {
            if (fast_exp) or_softmax_fast(scores + (size_t)i * tk, tk);
            else or_softmax_exact(scores + (size_t)i * tk, tk);
        }
        if (weights) memcpy(weights + (size_t)h * tq * tk, scores, sizeof(float) * (size_t)tq * tk);
        float *oh = out + (size_t)h * tq * hd;
        for (int i = 0; i < tq; i++)
            for (int c = 0; c < hd; c++) {
                float s = 0;
                for (int j = 0; j < tk; j++) s += scores[i * tk + j] * vh[(size_t)j * hd + c];
                oh[(size_t)i * hd + c] = s;
            }
    }
    free(scores);
}

/* ---- sampling --------------------------------------------------------------- */
/* model/decoder.go:1140-1167 */
void or_repetition_penalty(const float *logits, int n, const int32_t *hist, int hist_len, float penalty,
                           int window, float *out) {
    memcpy(out, logits, sizeof(float) * (size_t)n);
    if (penalty <= 0 || hist_len == 0 || window <= 0) return;
    int start = hist_len > window ? hist_len - window : 0;
    int *cnt = (int *)calloc((size_t)n, sizeof(int));
    for (int i = start; i < hist_len; i++) {
        int id = hist[i];
        if (id >= 0 && id < n) cnt[id]++;
    }
    for (int id = 0; id < n; id++)
        if (cnt[id] > 0) out[id] -= penalty * (float)cnt[id];
    free(cnt);
}

/* model/decoder.go:996-1034 (top-p fallback :1036-1056 excluded: unseeded RNG) */
int32_t or_sample_greedy(const float *logits, int n, float temperature, int suppress_nst, float no_speech_thold,
                         int32_t eot) {
    float inv = 1.0f;
    if (temperature > 0) inv = 1 / temperature;
    int mi = 0;
    float ms = logits[0] * inv;
    for (int i = 1; i < n; i++) {
        float s = logits[i] * inv;
        if (s > ms) { ms = s; mi = i; }
    }
    if (suppress_nst && eot >= 0 && eot < n) {
        if (logits[eot] < -no_speech_thold && mi == eot) {
            mi = -1;
            ms = -INFINITY;
            for (int i = 0; i < n; i++) {
                if (i == eot) continue;
                float s = logits[i] * inv;
                if (s > ms) { ms = s; mi = i; }
            }
            if (mi < 0) mi = eot;
        }
    }
    return mi;
}

/* model/decoder.go:1068-1136. sort.Slice is unstable in Go; here ties keep
 * their position in the replace-min buffer (stable insertion sort). */
int or_topk(const float *vals, int n, int k, float temperature, int32_t *tok, float *logprob) {
    if (k <= 0 || n <= 0) return 0;
    if (k > n) k = n;
    float inv = 1.0f;
    if (temperature > 0) inv = 1 / temperature;
    int len = 0, min_pos = -1;
    float min_val = 0, smax = -INFINITY;
    for (int i = 0; i < n; i++) {
        float s = vals[i] * inv;
        if (s > smax) smax = s;
        if (len < k) {
            tok[len] = i; logprob[len] = s; len++;
            if (min_pos < 0 || s < min_val) { min_pos = len - 1; min_val = s; }
            continue;
        }
        if (s <= min_val) continue;
        tok[min_pos] = i; logprob[min_pos] = s;
        min_pos = 0; min_val = logprob[0];
        for (int j = 1; j < len; j++) if (logprob[j] < min_val) { min_val = logprob[j]; min_pos = j; }
    }
    float es = 0;
    for (int i = 0; i < n; i++) es += (float)exp((double)(vals[i] * inv - smax));
    float logz = (float)log((double)es) + smax;
    for (int i = 0; i < len; i++) logprob[i] -= logz;
    for (int i = 1; i < len; i++) { /* stable descending insertion sort */
        float lp = logprob[i]; int32_t t = tok[i]; int j = i - 1;
        while (j >= 0 && logprob[j] < lp) { logprob[j + 1] = logprob[j]; tok[j + 1] = tok[j]; j--; }
        logprob[j + 1] = lp; tok[j + 1] = t;
    }
    return len;
}

/* ---- decoder model: model/decoder.go:19-303, model/compat.go ---------------- */
typedef struct {
    uint32_t type; /* 0 => float matrix in f32 (F32/F16/transposed loads), else raw quant */
    int rows, cols;
    const uint8_t *q; /* raw GGUF blocks (borrowed from caller) */
    float *f;         /* owned float data for type 0 */
    size_t row_bytes;
} omat;

typedef struct {
    float *ln1w, *ln1b, *sqb, *svb, *sob, *ln2w, *ln2b, *cqb, *cvb, *cob, *ln3w, *ln3b, *fc1b, *fc2b;
    omat sq, sk, sv, so, cq, ck, cv, co, fc1, fc2;
} olayer;

struct or_model {
    int n_vocab, n_state, n_head, n_layer, n_ctx;
    int32_t eot;
    int dot_variant, threads, fast_exp;
    int fwd_threads; /* > 1: split the forward's GEMV rows over threads (fixture generation only) */
    omat tok; /* type!=0: tokenEmbQ (row lookups dequantize, the documented extension of P4) */
    float *pos;
    float *lnw, *lnb;
    olayer *layers;
};

struct or_state {
    int n_layer;
    int32_t *tokens;
    int n_tokens, cap;
    float *kv;          /* [L,2,H,ctx,hd] */
    float **cross_k, **cross_v;
    int *cross_ready;
    float *x, *xln, *q, *k, *v, *attn, *out, *mlp, *kfull, *vfull, *logits_scratch;
};

/* model/compat.go:31-148 */
static int map_encoder_name(const char *name, char *out, size_t cap);
static int map_tensor_name(const char *name, char *out, size_t cap) {
    if (strncmp(name, "encoder.", 8) == 0) return map_encoder_name(name, out, cap);
    static const char *simple[][2] = {
        {"decoder.token_embedding.weight", "model.decoder.embed_tokens.weight"},
        {"decoder.positional_embedding", "model.decoder.embed_positions.weight"},
        {"decoder.ln.weight", "model.decoder.layer_norm.weight"},
        {"decoder.ln.bias", "model.decoder.layer_norm.bias"},
    };
    for (size_t i = 0; i < sizeof simple / sizeof simple[0]; i++)
        if (strcmp(name, simple[i][0]) == 0) { snprintf(out, cap, "%s", simple[i][1]); return 1; }
    const char *pre = "decoder.blocks.";
    if (strncmp(name, pre, strlen(pre)) != 0) return 0;
    const char *rest = name + strlen(pre);
    char *end;
    long idx = strtol(rest, &end, 10);
    if (end == rest || *end != '.') return 0;
    const char *suf = end + 1;
    static const char *sm[][2] = {
        {"self_attn_ln.weight", "self_attn_layer_norm.weight"}, {"self_attn_ln.bias", "self_attn_layer_norm.bias"},
        {"self_attn.query.weight", "self_attn.q_proj.weight"}, {"self_attn.query.bias", "self_attn.q_proj.bias"},
        {"self_attn.key.weight", "self_attn.k_proj.weight"}, {"self_attn.value.weight", "self_attn.v_proj.weight"},
        {"self_attn.value.bias", "self_attn.v_proj.bias"}, {"self_attn.out.weight", "self_attn.out_proj.weight"},
        {"self_attn.out.bias", "self_attn.out_proj.bias"},
        {"cross_attn_ln.weight", "encoder_attn_layer_norm.weight"}, {"cross_attn_ln.bias", "encoder_attn_layer_norm.bias"},
        {"cross_attn.query.weight", "encoder_attn.q_proj.weight"}, {"cross_attn.query.bias", "encoder_attn.q_proj.bias"},
        {"cross_attn.key.weight", "encoder_attn.k_proj.weight"}, {"cross_attn.value.weight", "encoder_attn.v_proj.weight"},
        {"cross_attn.value.bias", "encoder_attn.v_proj.bias"}, {"cross_attn.out.weight", "encoder_attn.out_proj.weight"},
        {"cross_attn.out.bias", "encoder_attn.out_proj.bias"},
        {"mlp_ln.weight", "final_layer_norm.weight"}, {"mlp_ln.bias", "final_layer_norm.bias"},
        {"mlp.0.weight", "fc1.weight"}, {"mlp.0.bias", "fc1.bias"}, {"mlp.2.weight", "fc2.weight"}, {"mlp.2.bias", "fc2.bias"},
    };
    for (size_t i = 0; i < sizeof sm / sizeof sm[0]; i++)
        if (strcmp(suf, sm[i][0]) == 0) { snprintf(out, cap, "model.decoder.layers.%ld.%s", idx, sm[i][1]); return 1; }
    return 0;
}

static const or_tensor *find_exact(const or_tensor *t, int n, const char *name) {
    for (int i = 0; i < n; i++) if (strcmp(t[i].name, name) == 0) return &t[i];
    return NULL;
}
/* model/compat.go:15-29 */
static const or_tensor *resolve(const or_tensor *t, int n, const char *name) {
    const or_tensor *r = find_exact(t, n, name);
    if (r) return r;
    char alt[256];
    if (!map_tensor_name(name, alt, sizeof alt)) return NULL;
    return find_exact(t, n, alt);
}
static uint64_t numel(const or_tensor *t) {
    uint64_t e = 1;
    for (uint32_t i = 0; i < t->ndim; i++) e *= t->shape[i];
    return e;
}
/* gguf.go:203-222 Tensor(): dequantize everything to f32 */
static float *load_f32(const or_tensor *t) {
    uint64_t ne = numel(t);
    float *o = (float *)malloc(sizeof(float) * (ne ? ne : 1));
    if (or_dequantize((const uint8_t *)t->data, t->type, ne, o) != 0) { free(o); return NULL; }
    return o;
}
static int is_quant(uint32_t type) { return type == 2 || type == 3 || type == 6 || type == 7 || type == 8; }

static float *transpose(const float *src, int r, int c) { /* src [r,c] -> [c,r] */
    float *o = (float *)malloc(sizeof(float) * (size_t)r * c);
    for (int i = 0; i < r; i++)
        for (int j = 0; j < c; j++) o[(size_t)j * r + i] = src[(size_t)i * c + j];
    return o;
}

/* model/compat.go:199-270 loadMatWeightAuto */
static int load_mat(const or_tensor *t, int n, const char *name, int want_rows, int want_cols, omat *m) {
    const or_tensor *tt = resolve(t, n, name);
    char msg[300];
    if (!tt) { snprintf(msg, sizeof msg, "model: load tensor \"%s\": not found", name); set_err(msg); return -1; }
    memset(m, 0, sizeof *m);
    if (tt->ndim == 2 && is_quant(tt->type) && (int)tt->shape[0] == want_rows && (int)tt->shape[1] == want_cols) {
        m->type = tt->type; m->rows = want_rows; m->cols = want_cols; m->q = (const uint8_t *)tt->data;
        m->row_bytes = or_row_bytes(tt->type, (size_t)want_cols);
        return 0;
    }
    if (tt->ndim != 2) { snprintf(msg, sizeof msg, "model: invalid %s shape", name); set_err(msg); return -1; }
    float *f = load_f32(tt);
    if (!f) return -1;
    if ((int)tt->shape[0] == want_rows && (int)tt->shape[1] == want_cols) {
        m->f = f;
    } else if ((int)tt->shape[0] == want_cols && (int)tt->shape[1] == want_rows) {
        m->f = transpose(f, want_cols, want_rows);
        free(f);
    } else {
        free(f);
        snprintf(msg, sizeof msg, "model: unsupported %s shape", name); set_err(msg); return -1;
    }
    m->type = 0; m->rows = want_rows; m->cols = want_cols; m->row_bytes = (size_t)want_cols * 4;
    return 0;
}
static float *load_vec(const or_tensor *t, int n, const char *name) {
    const or_tensor *tt = resolve(t, n, name);
    if (!tt) { char msg[300]; snprintf(msg, sizeof msg, "model: load tensor \"%s\": not found", name); set_err(msg); return NULL; }
    return load_f32(tt);
}
static const uint8_t *mat_rowptr(const omat *m, int r) {
    return m->type == 0 ? (const uint8_t *)(m->f + (size_t)r * m->cols) : m->q + (size_t)r * m->row_bytes;
}

void or_model_destroy(or_model *m) {
    if (!m) return;
    free(m->tok.f); free(m->pos); free(m->lnw); free(m->lnb);
    if (m->layers) {
        for (int i = 0; i < m->n_layer; i++) {
            olayer *l = &m->layers[i];
            float *v[] = {l->ln1w, l->ln1b, l->sqb, l->svb, l->sob, l->ln2w, l->ln2b, l->cqb, l->cvb, l->cob, l->ln3w, l->ln3b, l->fc1b, l->fc2b};
            for (size_t j = 0; j < sizeof v / sizeof v[0]; j++) free(v[j]);
            omat *ms[] = {&l->sq, &l->sk, &l->sv, &l->so, &l->cq, &l->ck, &l->cv, &l->co, &l->fc1, &l->fc2};
            for (size_t j = 0; j < sizeof ms / sizeof ms[0]; j++) free(ms[j]->f);
        }
        free(m->layers);
    }
    free(m);
}

/* model/decoder.go:97-303 */
or_model *or_model_create(const or_tensor *t, int n, const or_meta *meta, int dot_variant, int threads) {
    uint32_t n_head = meta ? meta->n_head : 0, n_layer = meta ? meta->n_layer : 0;
    uint32_t n_ctx = meta ? meta->n_ctx : 0, n_state = meta ? meta->n_state : 0, n_vocab = meta ? meta->n_vocab : 0;
    char name[256], msg[300];
    if (n_layer == 0) { /* compat.go:167-181 inferLayerCount */
        int c = 0;
        for (;;) {
            snprintf(name, sizeof name, "decoder.blocks.%d.self_attn.query.weight", c);
            if (!resolve(t, n, name)) break;
            c++;
        }
        n_layer = (uint32_t)c;
    }
    const or_tensor *aq = resolve(t, n, "decoder.blocks.0.self_attn.query.weight");
    if (aq && aq->ndim == 2 && aq->shape[0] == aq->shape[1] && aq->shape[0] > 0) n_state = (uint32_t)aq->shape[0];
    if (n_ctx == 0 || n_state == 0) {
        const or_tensor *p = resolve(t, n, "decoder.positional_embedding");
        if (!p) { set_err("model: load tensor \"decoder.positional_embedding\": not found"); return NULL; }
        if (p->ndim != 2) { set_err("model: decoder: invalid positional embedding shape"); return NULL; }
        if (n_state > 0) {
            if (p->shape[0] == n_state && p->shape[1] != n_state) n_ctx = (uint32_t)p->shape[1];
            else if (p->shape[1] == n_state) n_ctx = (uint32_t)p->shape[0];
        } else {
            n_ctx = (uint32_t)p->shape[0];
            n_state = (uint32_t)p->shape[1];
        }
    }
    if (n_vocab == 0) {
        const or_tensor *e = resolve(t, n, "decoder.token_embedding.weight");
        if (!e) { set_err("model: load tensor \"decoder.token_embedding.weight\": not found"); return NULL; }
        if (e->ndim != 2) { set_err("model: decoder: invalid token embedding shape"); return NULL; }
        if (n_state > 0) {
            if (e->shape[1] == n_state) n_vocab = (uint32_t)e->shape[0];
            else if (e->shape[0] == n_state) n_vocab = (uint32_t)e->shape[1];
        } else {
            n_vocab = (uint32_t)e->shape[0];
            n_state = (uint32_t)e->shape[1];
        }
    }
    if (n_head == 0) {
        if (n_state % 64 != 0) {
            snprintf(msg, sizeof msg, "model: decoder: cannot infer head count from embedding length %u", n_state);
            set_err(msg); return NULL;
        }
        n_head = n_state / 64;
    }
    or_model *m = (or_model *)calloc(1, sizeof *m);
    m->n_vocab = (int)n_vocab; m->n_state = (int)n_state; m->n_head = (int)n_head; m->n_layer = (int)n_layer;
    m->n_ctx = (int)n_ctx; m->eot = 50256; m->dot_variant = dot_variant; m->threads = threads > 0 ? threads : 1;
    m->fast_exp = 1;
    int d = m->n_state;
    /* token embedding :176-189 */
    const or_tensor *te = resolve(t, n, "decoder.token_embedding.weight");
    if (!te) { set_err("model: load tensor \"decoder.token_embedding.weight\": not found"); goto fail; }
    if (te->ndim == 2 && is_quant(te->type) && (int)te->shape[0] == m->n_vocab && (int)te->shape[1] == d) {
        m->tok.type = te->type; m->tok.rows = m->n_vocab; m->tok.cols = d; m->tok.q = (const uint8_t *)te->data;
        m->tok.row_bytes = or_row_bytes(te->type, (size_t)d);
    } else {
        if (te->ndim != 2) { set_err("model: decoder: invalid token embedding shape"); goto fail; }
        float *f = load_f32(te);
        if (!f) goto fail;
        if ((int)te->shape[0] == d && (int)te->shape[1] == m->n_vocab) { m->tok.f = transpose(f, d, m->n_vocab); free(f); }
        else m->tok.f = f;
        m->tok.type = 0; m->tok.rows = m->n_vocab; m->tok.cols = d; m->tok.row_bytes = (size_t)d * 4;
    }
    /* positional embedding :191-200 */
    const or_tensor *pe = resolve(t, n, "decoder.positional_embedding");
    if (!pe) { set_err("model: load tensor \"decoder.positional_embedding\": not found"); goto fail; }
    if (pe->ndim != 2) { set_err("model: decoder: invalid positional embedding shape"); goto fail; }
    {
        float *f = load_f32(pe);
        if (!f) goto fail;
        if ((int)pe->shape[0] == d && (int)pe->shape[1] == m->n_ctx) { m->pos = transpose(f, d, m->n_ctx); free(f); }
        else m->pos = f;
    }
    m->layers = (olayer *)calloc((size_t)m->n_layer, sizeof(olayer));
    for (int i = 0; i < m->n_layer; i++) {
        olayer *l = &m->layers[i];
        char p[64];
        snprintf(p, sizeof p, "decoder.blocks.%d", i);
#define VEC(field, suffix) do { snprintf(name, sizeof name, "%s.%s", p, suffix); if (!(l->field = load_vec(t, n, name))) goto fail; } while (0)
#define MAT(field, suffix, r, c) do { snprintf(name, sizeof name, "%s.%s", p, suffix); if (load_mat(t, n, name, r, c, &l->field)) goto fail; } while (0)
        VEC(ln1w, "self_attn_ln.weight"); VEC(ln1b, "self_attn_ln.bias");
        MAT(sq, "self_attn.query.weight", d, d); VEC(sqb, "self_attn.query.bias");
        MAT(sk, "self_attn.key.weight", d, d);
        MAT(sv, "self_attn.value.weight", d, d); VEC(svb, "self_attn.value.bias");
        MAT(so, "self_attn.out.weight", d, d); VEC(sob, "self_attn.out.bias");
        VEC(ln2w, "cross_attn_ln.weight"); VEC(ln2b, "cross_attn_ln.bias");
        MAT(cq, "cross_attn.query.weight", d, d); VEC(cqb, "cross_attn.query.bias");
        MAT(ck, "cross_attn.key.weight", d, d);
        MAT(cv, "cross_attn.value.weight", d, d); VEC(cvb, "cross_attn.value.bias");
        MAT(co, "cross_attn.out.weight", d, d); VEC(cob, "cross_attn.out.bias");
        VEC(ln3w, "mlp_ln.weight"); VEC(ln3b, "mlp_ln.bias");
        MAT(fc1, "mlp.0.weight", 4 * d, d); VEC(fc1b, "mlp.0.bias");
        MAT(fc2, "mlp.2.weight", d, 4 * d); VEC(fc2b, "mlp.2.bias");
#undef VEC
#undef MAT
    }
    if (!(m->lnw = load_vec(t, n, "decoder.ln.weight"))) goto fail;
    if (!(m->lnb = load_vec(t, n, "decoder.ln.bias"))) goto fail;
    return m;
fail:
    or_model_destroy(m);
    return NULL;
}

void or_model_hparams(const or_model *m, int32_t *o) {
    o[0] = m->n_vocab; o[1] = m->n_state; o[2] = m->n_head; o[3] = m->n_layer; o[4] = m->n_ctx;
}
void or_model_set_eot(or_model *m, int32_t eot) { m->eot = eot; }
void or_model_set_fast_exp(or_model *m, int on) { m->fast_exp = on; }
void or_model_set_forward_threads(or_model *m, int n) { m->fwd_threads = n; }

/* model/decoder.go:330-365 */
or_state *or_state_create(const or_model *m, const int32_t *prompt, int plen) {
    or_state *s = (or_state *)calloc(1, sizeof *s);
    int d = m->n_state, hd = d / m->n_head;
    s->n_layer = m->n_layer;
    s->cap = m->n_ctx + plen + 8;
    s->tokens = (int32_t *)malloc(sizeof(int32_t) * (size_t)s->cap);
    if (plen) memcpy(s->tokens, prompt, sizeof(int32_t) * (size_t)plen);
    s->n_tokens = plen;
    s->kv = (float *)calloc((size_t)m->n_layer * 2 * m->n_head * m->n_ctx * hd, sizeof(float));
    s->cross_k = (float **)calloc((size_t)m->n_layer, sizeof(float *));
    s->cross_v = (float **)calloc((size_t)m->n_layer, sizeof(float *));
    s->cross_ready = (int *)calloc((size_t)m->n_layer, sizeof(int));
    s->x = (float *)calloc((size_t)d, 4); s->xln = (float *)calloc((size_t)d, 4);
    s->q = (float *)calloc((size_t)d, 4); s->k = (float *)calloc((size_t)d, 4); s->v = (float *)calloc((size_t)d, 4);
    s->attn = (float *)calloc((size_t)d, 4); s->out = (float *)calloc((size_t)d, 4);
    s->mlp = (float *)calloc((size_t)4 * d, 4);
    s->kfull = (float *)calloc((size_t)m->n_head * m->n_ctx * hd, 4);
    s->vfull = (float *)calloc((size_t)m->n_head * m->n_ctx * hd, 4);
    return s;
}
void or_state_destroy(or_state *s) {
    if (!s) return;
    free(s->tokens); free(s->kv);
    for (int i = 0; i < s->n_layer; i++) { free(s->cross_k[i]); free(s->cross_v[i]); }
    free(s->cross_ready);
    free(s->x); free(s->xln); free(s->q); free(s->k); free(s->v); free(s->attn); free(s->out); free(s->mlp);
    free(s->kfull); free(s->vfull);
    free(s->cross_k); free(s->cross_v);
    free(s);
}
static void state_free_cross(const or_model *m, or_state *s) {
    for (int i = 0; i < m->n_layer; i++) {
        free(s->cross_k[i]); free(s->cross_v[i]);
        s->cross_k[i] = s->cross_v[i] = NULL; s->cross_ready[i] = 0;
    }
}
/* model/decoder.go:367-386 */
void or_state_reset(const or_model *m, or_state *s, const int32_t *tokens, int n) {
    if (n + 8 > s->cap) { s->cap = n + m->n_ctx + 8; s->tokens = (int32_t *)realloc(s->tokens, sizeof(int32_t) * (size_t)s->cap); }
    memmove(s->tokens, tokens, sizeof(int32_t) * (size_t)n);
    s->n_tokens = n;
    int hd = m->n_state / m->n_head;
    memset(s->kv, 0, sizeof(float) * (size_t)m->n_layer * 2 * m->n_head * m->n_ctx * hd);
    /* crossReady=false: the recompute yields identical values (deterministic
     * function of the encoder output), so the cached K/V are kept. */
}
int or_state_push(or_state *s, int32_t tok) {
    if (s->n_tokens + 1 > s->cap) { s->cap *= 2; s->tokens = (int32_t *)realloc(s->tokens, sizeof(int32_t) * (size_t)s->cap); }
    s->tokens[s->n_tokens++] = tok;
    return 0;
}

static void mat_gemv(const or_model *m, const omat *w, const float *a, int rows_a, float *out, int threads) {
    if (rows_a == 1 && m->fwd_threads > 1 && (size_t)w->rows * w->cols >= (1u << 16)) {
        gemv1_split(w->type, w->type == 0 ? (const uint8_t *)w->f : w->q, w->rows, w->cols, a, out, m->dot_variant,
                    m->fwd_threads);
        return;
    }
    or_gemv(w->type, w->type == 0 ? (const uint8_t *)w->f : w->q, w->rows, w->cols, a, rows_a, out, m->dot_variant, threads);
}

/* model/decoder.go:923-940 */
static void prepare_cross_layer(const or_model *m, or_state *s, int li, const float *enc, int enc_len) {
    const olayer *l = &m->layers[li];
    int d = m->n_state;
    s->cross_k[li] = (float *)malloc(sizeof(float) * (size_t)enc_len * d);
    s->cross_v[li] = (float *)malloc(sizeof(float) * (size_t)enc_len * d);
    mat_gemv(m, &l->ck, enc, enc_len, s->cross_k[li], m->threads);
    mat_gemv(m, &l->cv, enc, enc_len, s->cross_v[li], m->threads);
    for (int i = 0; i < enc_len; i++)
        for (int j = 0; j < d; j++) s->cross_v[li][(size_t)i * d + j] += l->cvb[j];
    s->cross_ready[li] = 1;
}
int or_state_prepare_cross(const or_model *m, or_state *s, const float *enc, int enc_len) {
    for (int i = 0; i < m->n_layer; i++) if (!s->cross_ready[i]) prepare_cross_layer(m, s, i, enc, enc_len);
    return 0;
}

/* model/decoder.go:745-833 (+ :836-993) */
int or_forward(const or_model *m, or_state *s, const float *enc, int enc_len, float *logits) {
    if (s->n_tokens == 0) { set_err("model: decode: forward: no tokens in state"); return -1; }
    int pos = s->n_tokens - 1;
    if (pos >= m->n_ctx) { set_err("model: decode: forward: position >= context length"); return -1; }
    int32_t id = s->tokens[pos];
    if (id < 0 || id >= m->n_vocab) { set_err("model: decode: forward: invalid token ID"); return -1; }
    int d = m->n_state, H = m->n_head, hd = d / H, ctx = m->n_ctx;
    float *x = s->x;
    if (m->tok.type == 0) memcpy(x, m->tok.f + (size_t)id * d, sizeof(float) * (size_t)d);
    else or_dequantize(mat_rowptr(&m->tok, id), m->tok.type, (size_t)d, x); /* P4 extension */
    for (int i = 0; i < d; i++) x[i] += m->pos[(size_t)pos * d + i];
    for (int li = 0; li < m->n_layer; li++) {
        const olayer *l = &m->layers[li];
        /* self-attention :836-908 */
        or_layernorm(s->xln, x, l->ln1w, l->ln1b, 1, d, 1e-5f);
        mat_gemv(m, &l->sq, s->xln, 1, s->q, 1);
        for (int i = 0; i < d; i++) s->q[i] += l->sqb[i];
        mat_gemv(m, &l->sk, s->xln, 1, s->k, 1);
        mat_gemv(m, &l->sv, s->xln, 1, s->v, 1);
        for (int i = 0; i < d; i++) s->v[i] += l->svb[i];
        size_t hb = (size_t)ctx * hd, base = (size_t)li * 2 * H * hb;
        for (int h = 0; h < H; h++) {
            memcpy(s->kv + base + h * hb + (size_t)pos * hd, s->k + h * hd, sizeof(float) * (size_t)hd);
            memcpy(s->kv + base + H * hb + h * hb + (size_t)pos * hd, s->v + h * hd, sizeof(float) * (size_t)hd);
        }
        int seq = pos + 1;
        for (int h = 0; h < H; h++) {
            memcpy(s->kfull + (size_t)h * seq * hd, s->kv + base + h * hb, sizeof(float) * (size_t)seq * hd);
            memcpy(s->vfull + (size_t)h * seq * hd, s->kv + base + H * hb + h * hb, sizeof(float) * (size_t)seq * hd);
        }
        or_sdpa(s->q, s->kfull, s->vfull, H, 1, seq, hd, 1, m->fast_exp, s->attn, NULL);
        mat_gemv(m, &l->so, s->attn, 1, s->out, 1);
        for (int i = 0; i < d; i++) x[i] += s->out[i] + l->sob[i];
        /* cross-attention :911-971 */
        or_layernorm(s->xln, x, l->ln2w, l->ln2b, 1, d, 1e-5f);
        mat_gemv(m, &l->cq, s->xln, 1, s->q, 1);
        for (int i = 0; i < d; i++) s->q[i] += l->cqb[i];
        if (!s->cross_ready[li]) prepare_cross_layer(m, s, li, enc, enc_len);
        /* P3: [encLen, d] row-major viewed as [H, encLen, hd] without transpose */
        or_sdpa(s->q, s->cross_k[li], s->cross_v[li], H, 1, enc_len, hd, 0, m->fast_exp, s->attn, NULL);
        mat_gemv(m, &l->co, s->attn, 1, s->out, 1);
        for (int i = 0; i < d; i++) x[i] += s->out[i] + l->cob[i];
        /* MLP :974-993 */
        or_layernorm(s->xln, x, l->ln3w, l->ln3b, 1, d, 1e-5f);
        mat_gemv(m, &l->fc1, s->xln, 1, s->mlp, 1);
        for (int i = 0; i < 4 * d; i++) s->mlp[i] += l->fc1b[i];
        or_gelu(s->mlp, 4 * d);
        mat_gemv(m, &l->fc2, s->mlp, 1, s->out, 1);
        for (int i = 0; i < d; i++) x[i] += s->out[i] + l->fc2b[i];
    }
    or_layernorm(x, x, m->lnw, m->lnb, 1, d, 1e-5f);
    mat_gemv(m, &m->tok, x, 1, logits, 1);
    return 0;
}

/* ---- Decode: model/decoder.go:401-726 -------------------------------------- */
typedef struct { int32_t *tokens; int len; float score; } obeam;
typedef struct { int parent; float score; int32_t token; float logprob; float norm; } ocand;

static int cap_max_tokens(const or_model *m, const or_decode_params *p) { /* :420-430 */
    int mt = p->max_tokens;
    if (mt <= 0) mt = m->n_ctx;
    if (m->n_ctx - p->prompt_len < mt) mt = m->n_ctx - p->prompt_len;
    if (mt < 0) mt = 0;
    return mt;
}

static int decode_greedy(const or_model *m, const float *enc, int enc_len, const or_decode_params *p, int32_t *out,
                         int cap, int32_t *out_len) {
    float base = p->temperature == 0 ? 1.0f : p->temperature;
    int mt = cap_max_tokens(m, p);
    if (p->logprob_thold > 0 && !p->no_fallback && base > 0) {
        set_err("model: decode: top-p fallback is non-deterministic in the reference and not supported");
        return -1;
    }
    or_state *s = or_state_create(m, p->prompt, p->prompt_len);
    float *logits = (float *)malloc(sizeof(float) * (size_t)m->n_vocab);
    float *cur = (float *)malloc(sizeof(float) * (size_t)m->n_vocab);
    int streak = 0, rc = 0;
    int32_t prev = -1;
    while (s->n_tokens < p->prompt_len + mt) {
        if (or_forward(m, s, enc, enc_len, logits)) { rc = -1; break; }
        or_repetition_penalty(logits, m->n_vocab, s->tokens, s->n_tokens, 2.0f, 128, cur);
        int32_t next = or_sample_greedy(cur, m->n_vocab, base, p->suppress_nst, p->no_speech_thold, m->eot);
        or_state_push(s, next);
        if (next == m->eot) break;
        if (prev == next) streak++;
        else { streak = 1; prev = next; }
        if (streak > 20) break;
    }
    if (rc == 0) {
        if (s->n_tokens > cap) { set_err("oracle: output capacity too small"); rc = -1; }
        else { memcpy(out, s->tokens, sizeof(int32_t) * (size_t)s->n_tokens); *out_len = s->n_tokens; }
    }
    state_free_cross(m, s);
    or_state_destroy(s);
    free(logits); free(cur);
    return rc;
}

/* ---- Go's sort.Slice (third-party: the Go 1.25 standard library, src/sort/slice.go
 * + zsortfunc.go, pattern-defeating quicksort "pdqsort_func"), restated for the
 * beam candidates with the reference's less(i, j) = norm[i] > norm[j]
 * (decoder.go:1462-1475). sort.Slice is not stable; the order it leaves equal
 * candidates in decides which parent lands in which slot, so the algorithm is
 * restated step by step: insertion sort up to 12 elements, median-of-three /
 * Tukey-ninther pivots, partial insertion sort on presorted input, partition on
 * duplicates, xorshift pattern breaking, heapsort fallback. */
typedef struct { ocand *v; } gosort;
static int gs_less(const gosort *d, int i, int j) { return d->v[i].norm > d->v[j].norm; }
static void gs_swap(gosort *d, int i, int j) { ocand t = d->v[i]; d->v[i] = d->v[j]; d->v[j] = t; }
static int go_bits_len(unsigned long x) { int n = 0; while (x) { n++; x >>= 1; } return n; }

static void gs_insertion(gosort *d, int a, int b) {
    for (int i = a + 1; i < b; i++)
        for (int j = i; j > a && gs_less(d, j, j - 1); j--) gs_swap(d, j, j - 1);
}
static void gs_sift_down(gosort *d, int lo, int hi, int first) {
    int root = lo;
    for (;;) {
        int child = 2 * root + 1;
        if (child >= hi) return;
        if (child + 1 < hi && gs_less(d, first + child, first + child + 1)) child++;
        if (!gs_less(d, first + root, first + child)) return;
        gs_swap(d, first + root, first + child);
        root = child;
    }
}
static void gs_heapsort(gosort *d, int a, int b) {
    int first = a, lo = 0, hi = b - a;
    for (int i = (hi - 1) / 2; i >= 0; i--) gs_sift_down(d, i, hi, first);
    for (int i = hi - 1; i >= 0; i--) { gs_swap(d, first, first + i); gs_sift_down(d, lo, i, first); }
}
static int gs_order2(gosort *d, int a, int b, int *swaps, int *lo) {
    if (gs_less(d, b, a)) { (*swaps)++; *lo = b; return a; }
    *lo = a; return b;
}
static int gs_median(gosort *d, int a, int b, int c, int *swaps) {
    int x, y;
    y = gs_order2(d, a, b, swaps, &x); a = x; b = y;
    y = gs_order2(d, b, c, swaps, &x); b = x; c = y;
    y = gs_order2(d, a, b, swaps, &x); a = x; b = y;
    (void)c;
    return b;
}
enum { GS_UNKNOWN = 0, GS_INCREASING = 1, GS_DECREASING = 2 };
static int gs_choose_pivot(gosort *d, int a, int b, int *hint) {
    const int l = b - a;
    int swaps = 0, i = a + l / 4 * 1, j = a + l / 4 * 2, k = a + l / 4 * 3;
    if (l >= 8) {
        if (l >= 50) { /* Tukey ninther */
            i = gs_median(d, i - 1, i, i + 1, &swaps);
            j = gs_median(d, j - 1, j, j + 1, &swaps);
            k = gs_median(d, k - 1, k, k + 1, &swaps);
        }
        j = gs_median(d, i, j, k, &swaps);
    }
    *hint = swaps == 0 ? GS_INCREASING : swaps == 12 ? GS_DECREASING : GS_UNKNOWN;
    return j;
}
static void gs_reverse(gosort *d, int a, int b) {
    for (int i = a, j = b - 1; i < j; i++, j--) gs_swap(d, i, j);
}
static int gs_partial_insertion(gosort *d, int a, int b) {
    int i = a + 1;
    for (int step = 0; step < 5; step++) {
        while (i < b && !gs_less(d, i, i - 1)) i++;
        if (i == b) return 1;
        if (b - a < 50) return 0;
        gs_swap(d, i, i - 1);
        if (i - a >= 2)
            for (int j = i - 1; j >= 1; j--) { if (!gs_less(d, j, j - 1)) break; gs_swap(d, j, j - 1); }
        if (b - i >= 2)
            for (int j = i + 1; j < b; j++) { if (!gs_less(d, j, j - 1)) break; gs_swap(d, j, j - 1); }
    }
    return 0;
}
static void gs_break_patterns(gosort *d, int a, int b) {
    const int length = b - a;
    if (length >= 8) {
        uint64_t r = (uint64_t)length; /* xorshift seeded with the length */
        const unsigned long modulus = 1ul << go_bits_len((unsigned long)length);
        const int idx = a + (length / 4) * 2 - 1;
        for (int i = 0; i < 3; i++) {
            r ^= r << 13; r ^= r >> 7; r ^= r << 17;
            int other = (int)((unsigned long)r & (modulus - 1));
            if (other >= length) other -= length;
            gs_swap(d, idx - 1 + i, a + other);
        }
    }
}
static int gs_partition_equal(gosort *d, int a, int b, int pivot) {
    gs_swap(d, a, pivot);
    int i = a + 1, j = b - 1;
    for (;;) {
        while (i <= j && !gs_less(d, a, i)) i++;
        while (i <= j && gs_less(d, a, j)) j--;
        if (i > j) break;
        gs_swap(d, i, j); i++; j--;
    }
    return i;
}
static int gs_partition(gosort *d, int a, int b, int pivot, int *already) {
    gs_swap(d, a, pivot);
    int i = a + 1, j = b - 1;
    while (i <= j && gs_less(d, i, a)) i++;
    while (i <= j && !gs_less(d, j, a)) j--;
    if (i > j) { gs_swap(d, j, a); *already = 1; return j; }
    gs_swap(d, i, j); i++; j--;
    for (;;) {
        while (i <= j && gs_less(d, i, a)) i++;
        while (i <= j && !gs_less(d, j, a)) j--;
        if (i > j) break;
        gs_swap(d, i, j); i++; j--;
    }
    gs_swap(d, j, a);
    *already = 0;
    return j;
}
static void gs_pdqsort(gosort *d, int a, int b, int limit) {
    int was_balanced = 1, was_partitioned = 1;
    for (;;) {
        const int length = b - a;
        if (length <= 12) { gs_insertion(d, a, b); return; }
        if (limit == 0) { gs_heapsort(d, a, b); return; }
        if (!was_balanced) { gs_break_patterns(d, a, b); limit--; }
        int hint;
        int pivot = gs_choose_pivot(d, a, b, &hint);
        if (hint == GS_DECREASING) {
            gs_reverse(d, a, b);
            pivot = (b - 1) - (pivot - a);
            hint = GS_INCREASING;
        }
        if (was_balanced && was_partitioned && hint == GS_INCREASING && gs_partial_insertion(d, a, b)) return;
        if (a > 0 && !gs_less(d, a - 1, pivot)) { a = gs_partition_equal(d, a, b, pivot); continue; }
        int already;
        const int mid = gs_partition(d, a, b, pivot, &already);
        was_partitioned = already;
        const int left = mid - a, right = b - mid, thr = length / 8;
        if (left < right) { was_balanced = left >= thr; gs_pdqsort(d, a, mid, limit); a = mid + 1; }
        else { was_balanced = right >= thr; gs_pdqsort(d, mid + 1, b, limit); b = mid; }
    }
}
/* sort.Slice(c, func(i, j) bool { return c[i].norm > c[j].norm }) */
static void go_sort_cands(ocand *c, int n) {
    gosort d = {c};
    gs_pdqsort(&d, 0, n, go_bits_len((unsigned long)n));
}
void or_go_sort_norm(float *norm, int32_t *id, int n) {
    ocand *c = (ocand *)calloc((size_t)(n > 0 ? n : 1), sizeof(ocand));
    for (int i = 0; i < n; i++) { c[i].norm = norm[i]; c[i].parent = id[i]; }
    go_sort_cands(c, n);
    for (int i = 0; i < n; i++) { norm[i] = c[i].norm; id[i] = c[i].parent; }
    free(c);
}

/* A Go `*beam` whose token slice has Go's length and capacity: make([]int32, n)
 * has capacity n, reslicing within the capacity keeps the backing array
 * (decoder.go:545-553, :636-658). Every beam owns its backing array. */
typedef struct { int32_t *buf; int len, cap; float score; } gobeam;

/* Beam search, decoder.go:528-726 (one attempt: no vocabulary, so no retry).
 * The next hypotheses are built inside the beam objects of the current step,
 * taken from the end of reusableBeams (:627-660): slot i reuses the object of
 * beams[nbeams-1-i] while later candidates may still name it as their parent,
 * so a parent is read as earlier slots left it; an object that is its own
 * parent and must grow gets a fresh zeroed slice first, which is also what the
 * copy then reads. Results for every beam object are exposed to tests through
 * or_beam_run. */
/* Per-step selection margins of the last beam_loop on this thread (test hook):
 * the smallest gap between two different normalised scores among the first
 * keep + 1 sorted candidates, i.e. how far the step's choice is from a reorder. */
static __thread float *g_margin_out;
static __thread int g_margin_cap;

static int beam_loop(const or_model *m, const float *enc, int enc_len, const or_decode_params *p, gobeam **out_obj,
                     int **out_order, int *out_nbeams, int *out_tcap) {
    float temp = p->temperature == 0 ? 1.0f : p->temperature;
    int bs = p->beam_size <= 0 ? 1 : p->beam_size;
    int mt = cap_max_tokens(m, p);
    int tcap = p->prompt_len + bs * (mt + 1) + 2; /* a slot grows by at most one per earlier slot and step */
    gobeam *obj = (gobeam *)calloc((size_t)bs, sizeof(gobeam));
    int *order = (int *)malloc(sizeof(int) * (size_t)bs), *reuse = (int *)malloc(sizeof(int) * (size_t)bs);
    int *next = (int *)malloc(sizeof(int) * (size_t)bs);
    for (int i = 0; i < bs; i++) {
        obj[i].buf = (int32_t *)calloc((size_t)tcap, sizeof(int32_t));
        memcpy(obj[i].buf, p->prompt, sizeof(int32_t) * (size_t)p->prompt_len);
        obj[i].len = obj[i].cap = p->prompt_len;
        obj[i].score = 0;
        order[i] = i;
    }
    int nbeams = bs;
    or_state *s = or_state_create(m, p->prompt, p->prompt_len);
    float *logits = (float *)malloc(sizeof(float) * (size_t)m->n_vocab);
    float *cur = (float *)malloc(sizeof(float) * (size_t)m->n_vocab);
    ocand *cands = (ocand *)malloc(sizeof(ocand) * (size_t)bs * 6);
    int rc = 0;
    for (int step = 0; step < mt; step++) {
        int nc = 0, nreuse = 0;
        for (int b = 0; b < nbeams; b++) {
            gobeam *h = &obj[order[b]];
            reuse[nreuse++] = order[b];
            if (h->len > 0 && h->buf[h->len - 1] == m->eot) {
                float norm = h->score / (float)pow((double)h->len, 0.6);
                cands[nc++] = (ocand){order[b], h->score, m->eot, 0, norm};
                continue;
            }
            or_state_reset(m, s, h->buf, h->len);
            if (or_forward(m, s, enc, enc_len, logits)) { rc = -1; goto done; }
            or_repetition_penalty(logits, m->n_vocab, h->buf, h->len, 2.0f, 128, cur);
            int32_t tk[5]; float lp[5];
            int k = or_topk(cur, m->n_vocab, 5, temp, tk, lp);
            for (int c = 0; c < k; c++) {
                int nl = h->len + 1;
                float ns = h->score + lp[c];
                float norm = ns / (float)pow((double)nl, 0.6);
                cands[nc++] = (ocand){order[b], ns, tk[c], lp[c], norm};
            }
        }
        go_sort_cands(cands, nc);
        int keep = nc < bs ? nc : bs;
        if (g_margin_out && step < g_margin_cap) {
            float gap = INFINITY;
            for (int i = 0; i < keep && i + 1 < nc; i++)
                if (cands[i].norm != cands[i + 1].norm && cands[i].norm - cands[i + 1].norm < gap)
                    gap = cands[i].norm - cands[i + 1].norm;
            g_margin_out[step] = gap;
        }
        for (int i = 0; i < keep; i++) {
            const ocand *c = &cands[i];
            if (nreuse == 0) { set_err("oracle: beam object pool exhausted"); rc = -1; goto done; }
            const int nbi = reuse[--nreuse];
            gobeam *nb = &obj[nbi], *par = &obj[c->parent];
            const int carry = par->len > 0 && par->buf[par->len - 1] == m->eot && c->token == m->eot && c->logprob == 0;
            const int need = carry ? par->len : par->len + 1;
            if (nb->cap < need) { /* nb.tokens = make([]int32, need) */
                memset(nb->buf, 0, sizeof(int32_t) * (size_t)need);
                nb->cap = need;
            }
            nb->len = need; /* or nb.tokens = nb.tokens[:need] */
            if (nb != par) memcpy(nb->buf, par->buf, sizeof(int32_t) * (size_t)(carry ? need : need - 1));
            if (!carry) nb->buf[need - 1] = c->token;
            nb->score = c->score;
            next[i] = nbi;
        }
        memcpy(order, next, sizeof(int) * (size_t)keep);
        nbeams = keep;
        int all_eot = 1;
        for (int b = 0; b < nbeams; b++) {
            const gobeam *h = &obj[order[b]];
            if (h->len == 0 || h->buf[h->len - 1] != m->eot) { all_eot = 0; break; }
        }
        if (all_eot) break;
        if (nbeams > 0 && obj[order[0]].len >= 2) {
            const gobeam *h = &obj[order[0]];
            int32_t last = h->buf[h->len - 1];
            int streak = 1, stop = 0;
            for (int i = h->len - 2; i >= 0 && h->buf[i] == last; i--) {
                streak++;
                if (streak > 20) { stop = 1; break; }
            }
            if (stop) break;
        }
    }
done:
    state_free_cross(m, s);
    or_state_destroy(s);
    free(logits); free(cur); free(cands); free(reuse); free(next);
    *out_obj = obj; *out_order = order; *out_nbeams = nbeams; *out_tcap = tcap;
    return rc;
}

static void beams_free(gobeam *obj, int *order, int bs) {
    for (int i = 0; i < bs; i++) free(obj[i].buf);
    free(obj); free(order);
}

static int decode_beam(const or_model *m, const float *enc, int enc_len, const or_decode_params *p, int32_t *out,
                       int cap, int32_t *out_len) {
    gobeam *obj; int *order, nbeams, tcap;
    const int bs = p->beam_size <= 0 ? 1 : p->beam_size;
    int rc = beam_loop(m, enc, enc_len, p, &obj, &order, &nbeams, &tcap);
    if (rc == 0) {
        if (nbeams == 0) *out_len = 0;
        else if (obj[order[0]].len > cap) { set_err("oracle: output capacity too small"); rc = -1; }
        else {
            memcpy(out, obj[order[0]].buf, sizeof(int32_t) * (size_t)obj[order[0]].len);
            *out_len = obj[order[0]].len;
        }
    }
    beams_free(obj, order, bs);
    return rc;
}

/* Every beam after the search, in beams order: lens[i], scores[i] and the
 * tokens of beam i at out + i * cap. Test hook for the in-place reuse. */
int or_beam_run(const or_model *m, const float *enc, int enc_len, const or_decode_params *p, int32_t *out, int cap,
                int32_t *lens, float *scores, int32_t *nbeams_out, float *step_margin, int margin_cap) {
    gobeam *obj; int *order, nbeams, tcap;
    const int bs = p->beam_size <= 0 ? 1 : p->beam_size;
    g_margin_out = step_margin;
    g_margin_cap = step_margin ? margin_cap : 0;
    int rc = beam_loop(m, enc, enc_len, p, &obj, &order, &nbeams, &tcap);
    g_margin_out = NULL;
    g_margin_cap = 0;
    if (rc == 0) {
        for (int i = 0; i < nbeams && rc == 0; i++) {
            const gobeam *h = &obj[order[i]];
            if (h->len > cap) { set_err("oracle: output capacity too small"); rc = -1; break; }
            memcpy(out + (size_t)i * cap, h->buf, sizeof(int32_t) * (size_t)h->len);
            lens[i] = h->len;
            scores[i] = h->score;
        }
        *nbeams_out = nbeams;
    }
    beams_free(obj, order, bs);
    return rc;
}

/* model/decoder.go:401-410 */
int or_decode(const or_model *m, const float *enc, int enc_len, const or_decode_params *p, int32_t *out, int cap,
              int32_t *out_len) {
    *out_len = 0;
    if (p->beam_size > 1) return decode_beam(m, enc, enc_len, p, out, cap, out_len);
    return decode_greedy(m, enc, enc_len, p, out, cap, out_len);
}


/* ---- encoder (model/encoder.go) --------------------------------------------- */

/* model/compat.go:31-83, the encoder half of mapTensorName */
static int map_encoder_name(const char *name, char *out, size_t cap) {
    static const char *simple[][2] = {
        {"encoder.conv1.weight", "model.encoder.conv1.weight"},
        {"encoder.conv1.bias", "model.encoder.conv1.bias"},
        {"encoder.conv2.weight", "model.encoder.conv2.weight"},
        {"encoder.conv2.bias", "model.encoder.conv2.bias"},
        {"encoder.positional_embedding", "model.encoder.embed_positions.weight"},
        {"encoder.ln_post.weight", "model.encoder.layer_norm.weight"},
        {"encoder.ln_post.bias", "model.encoder.layer_norm.bias"},
    };
    for (size_t i = 0; i < sizeof simple / sizeof simple[0]; i++)
        if (strcmp(name, simple[i][0]) == 0) { snprintf(out, cap, "%s", simple[i][1]); return 1; }
    const char *pre = "encoder.blocks.";
    if (strncmp(name, pre, strlen(pre)) != 0) return 0;
    const char *rest = name + strlen(pre);
    char *end;
    long idx = strtol(rest, &end, 10);
    if (end == rest || *end != '.') return 0;
    const char *suf = end + 1;
    static const char *sm[][2] = {
        {"attn_ln.weight", "self_attn_layer_norm.weight"}, {"attn_ln.bias", "self_attn_layer_norm.bias"},
        {"attn.query.weight", "self_attn.q_proj.weight"}, {"attn.query.bias", "self_attn.q_proj.bias"},
        {"attn.key.weight", "self_attn.k_proj.weight"}, {"attn.value.weight", "self_attn.v_proj.weight"},
        {"attn.value.bias", "self_attn.v_proj.bias"}, {"attn.out.weight", "self_attn.out_proj.weight"},
        {"attn.out.bias", "self_attn.out_proj.bias"}, {"mlp_ln.weight", "final_layer_norm.weight"},
        {"mlp_ln.bias", "final_layer_norm.bias"}, {"mlp.0.weight", "fc1.weight"}, {"mlp.0.bias", "fc1.bias"},
        {"mlp.2.weight", "fc2.weight"}, {"mlp.2.bias", "fc2.bias"},
    };
    for (size_t i = 0; i < sizeof sm / sizeof sm[0]; i++)
        if (strcmp(suf, sm[i][0]) == 0) { snprintf(out, cap, "model.encoder.layers.%ld.%s", idx, sm[i][1]); return 1; }
    return 0;
}

typedef struct {
    float *attn_lnw, *attn_lnb, *qb, *vb, *ob, *mlp_lnw, *mlp_lnb, *fc1b, *fc2b;
    omat q, k, v, o, fc1, fc2;
} oeblock;

struct or_encoder {
    int n_mels, n_state, n_head, n_layer, n_ctx;
    int dot_variant, threads, fast_exp;
    float *conv1w, *conv1b; /* [d, n_mels, 3] */
    float *conv2w, *conv2b; /* [d, d, 3] */
    float *pos;             /* [n_ctx, d] */
    oeblock *blocks;
    float *ln_postw, *ln_postb;
};

/* ml/conv.go:19-70: pad = kernel / 2, T' = (T + 2 pad - kernel) / stride + 1;
 * out[oc, t] = bias[oc] + sum over ic, then k, of in[ic, t stride - pad + k] w[oc, ic, k]
 * (zero padding), accumulated in that order in float32. Returns T'. */
int or_conv1d(const float *in, int in_c, int t, const float *w, const float *bias, int out_c, int kernel, int stride,
              float *out) {
    const int pad = kernel / 2, tp = (t + 2 * pad - kernel) / stride + 1;
    for (int oc = 0; oc < out_c; oc++)
        for (int j = 0; j < tp; j++) {
            float sum = bias[oc];
            for (int ic = 0; ic < in_c; ic++)
                for (int k = 0; k < kernel; k++) {
                    const int it = j * stride - pad + k;
                    if (it < 0 || it >= t) continue;
                    sum += in[(size_t)ic * t + it] * w[((size_t)oc * in_c + ic) * kernel + k];
                }
            out[(size_t)oc * tp + j] = sum;
        }
    return tp;
}

/* ml.Transpose of a [a, b, c] tensor by the permutation (i0, i1, i2). */
static float *transpose3(const float *src, const uint64_t *sh, int i0, int i1, int i2) {
    const uint64_t n[3] = {sh[0], sh[1], sh[2]};
    const uint64_t o1 = n[i1], o2 = n[i2];
    float *o = (float *)malloc(sizeof(float) * (size_t)(n[0] * n[1] * n[2]));
    for (uint64_t a = 0; a < n[0]; a++)
        for (uint64_t b = 0; b < n[1]; b++)
            for (uint64_t c = 0; c < n[2]; c++) {
                const uint64_t idx[3] = {a, b, c};
                o[(idx[i0] * o1 + idx[i1]) * o2 + idx[i2]] = src[(a * n[1] + b) * n[2] + c];
            }
    return o;
}

void or_encoder_destroy(or_encoder *e) {
    if (!e) return;
    free(e->conv1w); free(e->conv1b); free(e->conv2w); free(e->conv2b); free(e->pos);
    free(e->ln_postw); free(e->ln_postb);
    if (e->blocks) {
        for (int i = 0; i < e->n_layer; i++) {
            oeblock *b = &e->blocks[i];
            float *v[] = {b->attn_lnw, b->attn_lnb, b->qb, b->vb, b->ob, b->mlp_lnw, b->mlp_lnb, b->fc1b, b->fc2b};
            for (size_t j = 0; j < sizeof v / sizeof v[0]; j++) free(v[j]);
            omat *ms[] = {&b->q, &b->k, &b->v, &b->o, &b->fc1, &b->fc2};
            for (size_t j = 0; j < sizeof ms / sizeof ms[0]; j++) free(ms[j]->f);
        }
        free(e->blocks);
    }
    free(e);
}

/* model/encoder.go:58-263 NewEncoder: hyper-parameters from metadata, else
 * inferred from the tensors; conv weights in any of the stored orders the
 * reference accepts; the positional embedding transposed when stored [d, ctx]. */
or_encoder *or_encoder_create(const or_tensor *t, int n, const or_enc_meta *meta, int dot_variant, int threads) {
    char msg[300];
    uint32_t n_head = meta ? meta->n_head : 0, n_layer = meta ? meta->n_layer : 0, n_ctx = meta ? meta->n_ctx : 0;
    uint32_t n_state = meta ? meta->n_state : 0, n_mels = meta ? meta->n_mels : 0;
    if (n_layer == 0) {
        char nm[96];
        while (1) {
            snprintf(nm, sizeof nm, "encoder.blocks.%u.attn.query.weight", n_layer);
            if (!resolve(t, n, nm)) break;
            n_layer++;
        }
    }
    if (n_state == 0) {
        const or_tensor *b = resolve(t, n, "encoder.conv1.bias");
        if (!b) { set_err("model: load tensor \"encoder.conv1.bias\": not found"); return NULL; }
        if (b->ndim != 1 || b->shape[0] == 0) { set_err("model: encoder: invalid conv1.bias shape"); return NULL; }
        n_state = (uint32_t)b->shape[0];
    }
    const or_tensor *aq = resolve(t, n, "encoder.blocks.0.attn.query.weight");
    if (aq && aq->ndim == 2 && aq->shape[0] == aq->shape[1] && aq->shape[0] > 0) n_state = (uint32_t)aq->shape[0];
    const or_tensor *pe = resolve(t, n, "encoder.positional_embedding");
    if (n_ctx == 0) {
        if (!pe) { set_err("model: load tensor \"encoder.positional_embedding\": not found"); return NULL; }
        if (pe->ndim != 2) { set_err("model: encoder: invalid positional embedding shape"); return NULL; }
        if (pe->shape[0] == n_state && pe->shape[1] != n_state) n_ctx = (uint32_t)pe->shape[1];
        else n_ctx = (uint32_t)pe->shape[0];
    }
    if (n_head == 0) {
        if (n_state % 64 != 0) {
            snprintf(msg, sizeof msg, "model: encoder: cannot infer head count from embedding length %u", n_state);
            set_err(msg);
            return NULL;
        }
        n_head = n_state / 64;
    }
    or_encoder *e = (or_encoder *)calloc(1, sizeof *e);
    e->n_state = (int)n_state; e->n_head = (int)n_head; e->n_layer = (int)n_layer; e->n_ctx = (int)n_ctx;
    e->dot_variant = dot_variant; e->threads = threads > 0 ? threads : 1; e->fast_exp = 1;
    const int d = e->n_state;
    /* conv1: [d, n_mels, 3], or [n_mels, d, 3] (legacy), or [3, n_mels, d] */
    const or_tensor *c1 = resolve(t, n, "encoder.conv1.weight");
    if (!c1) { set_err("model: load tensor \"encoder.conv1.weight\": not found"); goto fail; }
    if (c1->ndim != 3) { set_err("model: encoder: invalid conv1.weight shape"); goto fail; }
    {
        float *f = load_f32(c1);
        if (!f) goto fail;
        if ((int)c1->shape[0] == d && c1->shape[1] > 0 && c1->shape[2] == 3) {
            e->conv1w = f;
            if (n_mels == 0) n_mels = (uint32_t)c1->shape[1];
        } else if ((int)c1->shape[1] == d && c1->shape[0] > 0 && c1->shape[2] == 3) {
            e->conv1w = transpose3(f, c1->shape, 1, 0, 2); free(f);
            if (n_mels == 0) n_mels = (uint32_t)c1->shape[0];
        } else if (c1->shape[0] == 3 && (int)c1->shape[2] == d && c1->shape[1] > 0) {
            e->conv1w = transpose3(f, c1->shape, 2, 1, 0); free(f);
            if (n_mels == 0) n_mels = (uint32_t)c1->shape[1];
        } else {
            free(f);
            set_err("model: encoder: unsupported conv1.weight shape");
            goto fail;
        }
    }
    e->n_mels = (int)n_mels;
    if (!(e->conv1b = load_vec(t, n, "encoder.conv1.bias"))) goto fail;
    {
        const or_tensor *c2 = resolve(t, n, "encoder.conv2.weight");
        if (!c2) { set_err("model: load tensor \"encoder.conv2.weight\": not found"); goto fail; }
        if (c2->ndim != 3) { set_err("model: encoder: invalid conv2.weight shape"); goto fail; }
        float *f = load_f32(c2);
        if (!f) goto fail;
        if ((int)c2->shape[0] == d && (int)c2->shape[1] == d && c2->shape[2] == 3) e->conv2w = f;
        else if (c2->shape[0] == 3 && (int)c2->shape[1] == d && (int)c2->shape[2] == d) {
            e->conv2w = transpose3(f, c2->shape, 2, 1, 0); free(f);
        } else {
            e->conv2w = transpose3(f, c2->shape, 1, 0, 2); free(f);
        }
    }
    if (!(e->conv2b = load_vec(t, n, "encoder.conv2.bias"))) goto fail;
    {
        if (!pe) { set_err("model: load tensor \"encoder.positional_embedding\": not found"); goto fail; }
        if (pe->ndim != 2) { set_err("model: encoder: invalid positional embedding shape"); goto fail; }
        float *f = load_f32(pe);
        if (!f) goto fail;
        if ((int)pe->shape[0] == d && (int)pe->shape[1] == e->n_ctx) { e->pos = transpose(f, d, e->n_ctx); free(f); }
        else e->pos = f;
    }
    e->blocks = (oeblock *)calloc((size_t)(n_layer ? n_layer : 1), sizeof(oeblock));
    for (int i = 0; i < e->n_layer; i++) {
        oeblock *b = &e->blocks[i];
        char nm[160];
#define EVEC(field, suf) do { snprintf(nm, sizeof nm, "encoder.blocks.%d." suf, i); if (!(b->field = load_vec(t, n, nm))) goto fail; } while (0)
#define EMAT(field, suf, r, c) do { snprintf(nm, sizeof nm, "encoder.blocks.%d." suf, i); if (load_mat(t, n, nm, r, c, &b->field)) goto fail; } while (0)
        EVEC(attn_lnw, "attn_ln.weight"); EVEC(attn_lnb, "attn_ln.bias");
        EMAT(q, "attn.query.weight", d, d); EVEC(qb, "attn.query.bias");
        EMAT(k, "attn.key.weight", d, d);
        EMAT(v, "attn.value.weight", d, d); EVEC(vb, "attn.value.bias");
        EMAT(o, "attn.out.weight", d, d); EVEC(ob, "attn.out.bias");
        EVEC(mlp_lnw, "mlp_ln.weight"); EVEC(mlp_lnb, "mlp_ln.bias");
        EMAT(fc1, "mlp.0.weight", 4 * d, d); EVEC(fc1b, "mlp.0.bias");
        EMAT(fc2, "mlp.2.weight", d, 4 * d); EVEC(fc2b, "mlp.2.bias");
#undef EVEC
#undef EMAT
    }
    if (!(e->ln_postw = load_vec(t, n, "encoder.ln_post.weight"))) goto fail;
    if (!(e->ln_postb = load_vec(t, n, "encoder.ln_post.bias"))) goto fail;
    return e;
fail:
    or_encoder_destroy(e);
    return NULL;
}

void or_encoder_set_fast_exp(or_encoder *e, int on) { e->fast_exp = on; }

void or_encoder_hparams(const or_encoder *e, int32_t *o) {
    o[0] = e->n_mels; o[1] = e->n_state; o[2] = e->n_head; o[3] = e->n_layer; o[4] = e->n_ctx;
}

static void enc_gemv(const or_encoder *e, const omat *w, const float *a, int rows_a, float *out) {
    or_gemv(w->type, w->type == 0 ? (const uint8_t *)w->f : w->q, w->rows, w->cols, a, rows_a, out, e->dot_variant,
            e->threads);
}
static void add_bias(float *x, const float *b, int rows, int c) {
    for (int r = 0; r < rows; r++)
        for (int j = 0; j < c; j++) x[(size_t)r * c + j] += b[j];
}

/* model/encoder.go:340-379 runSelfAttn: Q = x Wq^T + bq, K = x Wk^T, V = x Wv^T + bv,
 * heads [T, H, hd] -> [H, T, hd], SDPA without a mask, back to [T, d], out projection. */
static void enc_self_attn(const or_encoder *e, const oeblock *b, const float *x, int T, float *out) {
    const int d = e->n_state, H = e->n_head, hd = d / H;
    const size_t n = (size_t)T * d;
    float *Q = (float *)malloc(sizeof(float) * n), *K = (float *)malloc(sizeof(float) * n);
    float *V = (float *)malloc(sizeof(float) * n), *A = (float *)malloc(sizeof(float) * n);
    float *qh = (float *)malloc(sizeof(float) * n), *kh = (float *)malloc(sizeof(float) * n);
    float *vh = (float *)malloc(sizeof(float) * n), *ah = (float *)malloc(sizeof(float) * n);
    enc_gemv(e, &b->q, x, T, Q); add_bias(Q, b->qb, T, d);
    enc_gemv(e, &b->k, x, T, K);
    enc_gemv(e, &b->v, x, T, V); add_bias(V, b->vb, T, d);
    for (int t = 0; t < T; t++)
        for (int h = 0; h < H; h++)
            for (int c = 0; c < hd; c++) {
                const size_t src = (size_t)t * d + h * hd + c, dst = ((size_t)h * T + t) * hd + c;
                qh[dst] = Q[src]; kh[dst] = K[src]; vh[dst] = V[src];
            }
    or_sdpa(qh, kh, vh, H, T, T, hd, 0, e->fast_exp, ah, NULL);
    for (int t = 0; t < T; t++)
        for (int h = 0; h < H; h++)
            for (int c = 0; c < hd; c++) A[(size_t)t * d + h * hd + c] = ah[((size_t)h * T + t) * hd + c];
    enc_gemv(e, &b->o, A, T, out); add_bias(out, b->ob, T, d);
    free(Q); free(K); free(V); free(A); free(qh); free(kh); free(vh); free(ah);
}

/* model/encoder.go:265-338 Encode: conv stem with GELU, positional embedding,
 * pre-LN blocks (self-attention, MLP with GELU), final LayerNorm. mel is
 * [n_mels, T]; out receives [T', d] with T' = T / 2 (T even). Returns T' or -1. */
int or_encode(const or_encoder *e, const float *mel, int n_mels, int T, float *out) {
    char msg[200];
    if (n_mels != e->n_mels) {
        snprintf(msg, sizeof msg, "model: encoder: mel must be [%d, T], got [%d %d]", e->n_mels, n_mels, T);
        set_err(msg);
        return -1;
    }
    if (T == 2 * e->n_ctx + 1) T = 2 * e->n_ctx; /* one extra STFT frame: the first 2 n_ctx frames */
    if (T > 2 * e->n_ctx) {
        snprintf(msg, sizeof msg, "model: encoder: T=%d > 2*n_audio_ctx=%d", T, 2 * e->n_ctx);
        set_err(msg);
        return -1;
    }
    const int d = e->n_state;
    float *c1 = (float *)malloc(sizeof(float) * (size_t)d * (T > 0 ? T : 1));
    const int t1 = or_conv1d(mel, n_mels, T, e->conv1w, e->conv1b, d, 3, 1, c1);
    or_gelu(c1, d * t1);
    const int tp = (t1 + 2 - 3) / 2 + 1;
    float *c2 = (float *)malloc(sizeof(float) * (size_t)d * (tp > 0 ? tp : 1));
    or_conv1d(c1, d, t1, e->conv2w, e->conv2b, d, 3, 2, c2);
    or_gelu(c2, d * tp);
    float *x = (float *)malloc(sizeof(float) * (size_t)tp * d);
    for (int t = 0; t < tp; t++)
        for (int c = 0; c < d; c++) x[(size_t)t * d + c] = c2[(size_t)c * tp + t] + e->pos[(size_t)t * d + c];
    float *xln = (float *)malloc(sizeof(float) * (size_t)tp * d);
    float *o = (float *)malloc(sizeof(float) * (size_t)tp * d);
    float *h = (float *)malloc(sizeof(float) * (size_t)tp * 4 * d);
    for (int i = 0; i < e->n_layer; i++) {
        const oeblock *b = &e->blocks[i];
        or_layernorm(xln, x, b->attn_lnw, b->attn_lnb, tp, d, 1e-5f);
        enc_self_attn(e, b, xln, tp, o);
        for (size_t j = 0; j < (size_t)tp * d; j++) x[j] = x[j] + o[j];
        or_layernorm(xln, x, b->mlp_lnw, b->mlp_lnb, tp, d, 1e-5f);
        enc_gemv(e, &b->fc1, xln, tp, h); add_bias(h, b->fc1b, tp, 4 * d);
        or_gelu(h, tp * 4 * d);
        enc_gemv(e, &b->fc2, h, tp, o); add_bias(o, b->fc2b, tp, d);
        for (size_t j = 0; j < (size_t)tp * d; j++) x[j] = x[j] + o[j];
    }
    or_layernorm(out, x, e->ln_postw, e->ln_postb, tp, d, 1e-5f);
    free(c1); free(c2); free(x); free(xln); free(o); free(h);
    return tp;
}
