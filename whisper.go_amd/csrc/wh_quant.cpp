// Host-side GGUF block quantisation (bit-exact with internal/gguf/quant.go)
// and the re-layout of GGUF rows into the device planes used by the kernels.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cctype>
#include <cmath>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "wh_internal.h"

namespace wh {

static inline float bits_to_f32(uint32_t b) {
    float f;
    std::memcpy(&f, &b, 4);
    return f;
}
static inline uint32_t f32_to_bits(float f) {
    uint32_t b;
    std::memcpy(&b, &f, 4);
    return b;
}

// internal/gguf/quant.go:11-55 — mantissa rounded half-up on bit 12, float32
// subnormals flush to signed zero, overflow saturates to Inf.
uint16_t f32_to_f16(float f) {
    const uint32_t bits = f32_to_bits(f);
    const uint16_t sign = (uint16_t)((bits >> 31) << 15);
    const int exp = (int)((bits >> 23) & 0xFF);
    const uint32_t mant = bits & 0x7FFFFFu;
    if (exp == 255) return (uint16_t)(sign | (mant ? 0x7E00 : 0x7C00));
    if (exp == 0) return sign;
    int e16 = exp - 112;
    if (e16 >= 31) return (uint16_t)(sign | 0x7C00);
    if (e16 <= 0) {
        if (e16 < -10) return sign;
        return (uint16_t)(sign | ((mant | 0x800000u) >> (14 - e16)));
    }
    uint32_t m16 = (mant >> 13) + ((mant >> 12) & 1u);
    if (m16 >= 0x400) {
        m16 = 0;
        if (++e16 >= 31) return (uint16_t)(sign | 0x7C00);
    }
    return (uint16_t)(sign | ((uint32_t)e16 << 10) | m16);
}

// internal/gguf/dequant.go:15-44.
float f16_to_f32(uint16_t h) {
    const uint32_t s = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    if (e == 0) {
        if (m == 0) return bits_to_f32(s);
        uint32_t k = 0;
        while ((m & 0x400u) == 0) { m <<= 1; k++; }
        return bits_to_f32(s | ((113u - k) << 23) | ((m & 0x3FFu) << 13));
    }
    if (e == 31) return bits_to_f32(s | 0x7F800000u | (m << 13));
    return bits_to_f32(s | ((e + 112u) << 23) | (m << 13));
}

uint64_t gguf_row_bytes(uint32_t type, uint64_t n) {
    const uint64_t b = (n + 31) / 32;
    switch (type) {
    case WH_TYPE_F32: return n * 4;
    case WH_TYPE_F16: return n * 2;
    case WH_TYPE_Q4_0: return b * 18;
    case WH_TYPE_Q4_1: return b * 20;
    case WH_TYPE_Q5_0: return b * 22;
    case WH_TYPE_Q5_1: return b * 24;
    case WH_TYPE_Q8_0: return b * 34;
    default: return 0;
    }
}

bool is_quant_type(uint32_t t) {
    return t == WH_TYPE_Q4_0 || t == WH_TYPE_Q4_1 || t == WH_TYPE_Q5_0 || t == WH_TYPE_Q5_1 || t == WH_TYPE_Q8_0;
}

// math.Round semantics (half away from zero) applied to float64(v), then int32.
static inline int32_t round_half_away(float v) { return (int32_t)std::round((double)v); }

static inline void store_f16(uint8_t *p, float f) {
    const uint16_t h = f32_to_f16(f);
    p[0] = (uint8_t)h;
    p[1] = (uint8_t)(h >> 8);
}

// One 32-element block (len <= 32 live values, the rest read as 0) of each
// format; internal/gguf/quant.go:87-232 with helpers :252-376.
static void quant_block(uint32_t type, const float *v, int len, uint8_t *out) {
    float x[32];
    for (int i = 0; i < 32; i++) x[i] = i < len ? v[i] : 0.0f;
    float amax = 0.0f, mn = 0.0f, mx = 0.0f;
    for (int i = 0; i < len; i++) amax = std::max(amax, std::fabs(x[i]));
    if (len > 0) {
        mn = mx = x[0];
        for (int i = 1; i < len; i++) {
            if (x[i] < mn) mn = x[i];
            if (x[i] > mx) mx = x[i];
        }
    }
    auto clampi = [](int32_t q, int32_t lo, int32_t hi) { return q < lo ? lo : (q > hi ? hi : q); };
    switch (type) {
    case WH_TYPE_Q4_0: {
        const float d = amax / 7.0f;
        store_f16(out, d);
        for (int i = 0; i < 16; i++) {
            int32_t lo = d != 0 ? round_half_away(x[2 * i] / d) + 8 : 8;
            int32_t hi = d != 0 ? round_half_away(x[2 * i + 1] / d) + 8 : 8;
            out[2 + i] = (uint8_t)(clampi(lo, 0, 15) | (clampi(hi, 0, 15) << 4));
        }
        break;
    }
    case WH_TYPE_Q4_1: {
        const float d = (mx - mn) / 15.0f;
        store_f16(out, d);
        store_f16(out + 2, mn);
        for (int i = 0; i < 16; i++) {
            int32_t lo = d != 0 ? round_half_away((x[2 * i] - mn) / d) : 0;
            int32_t hi = d != 0 ? round_half_away((x[2 * i + 1] - mn) / d) : 0;
            out[4 + i] = (uint8_t)(clampi(lo, 0, 15) | (clampi(hi, 0, 15) << 4));
        }
        break;
    }
    case WH_TYPE_Q5_0: {
        const float d = amax / 15.0f;
        store_f16(out, d);
        uint32_t qh = 0;
        for (int i = 0; i < 32; i++) {
            int32_t q = clampi(d != 0 ? round_half_away(x[i] / d) + 16 : 16, 0, 31);
            qh |= (uint32_t)((q >> 4) & 1) << i;
            uint8_t &byte = out[6 + i / 2];
            byte = (i & 1) ? (uint8_t)((byte & 0x0F) | ((q & 0xF) << 4)) : (uint8_t)((byte & 0xF0) | (q & 0xF));
        }
        std::memcpy(out + 2, &qh, 4);
        break;
    }
    case WH_TYPE_Q5_1: {
        const float d = (mx - mn) / 31.0f;
        store_f16(out, d);
        store_f16(out + 2, mn);
        uint32_t qh = 0;
        for (int i = 0; i < 32; i++) {
            int32_t q = clampi(d != 0 ? round_half_away((x[i] - mn) / d) : 0, 0, 31);
            qh |= (uint32_t)((q >> 4) & 1) << i;
            uint8_t &byte = out[8 + i / 2];
            byte = (i & 1) ? (uint8_t)((byte & 0x0F) | ((q & 0xF) << 4)) : (uint8_t)((byte & 0xF0) | (q & 0xF));
        }
        std::memcpy(out + 4, &qh, 4);
        break;
    }
    case WH_TYPE_Q8_0: {
        const float d = amax / 127.0f;
        store_f16(out, d);
        for (int i = 0; i < 32; i++) {
            int32_t q = d != 0 ? clampi(round_half_away(x[i] / d), -127, 127) : 0;
            out[2 + i] = (uint8_t)(int8_t)q;
        }
        break;
    }
    default: break;
    }
}

int quantize(uint32_t type, const float *src, uint64_t n, uint8_t *dst, uint64_t dst_bytes, int threads) {
    const uint64_t need = gguf_row_bytes(type, n);
    if (need == 0 && n != 0) return fail(WH_ERR_UNSUPPORTED, "gguf: quantize: unsupported quant type");
    if (dst_bytes < need) return fail(WH_ERR_INVALID, "gguf: quantize: destination too small");
    if (type == WH_TYPE_F32) {
        std::memcpy(dst, src, n * 4);
        return WH_OK;
    }
    const uint64_t nblk = (n + 31) / 32;
    const uint64_t bbytes = type == WH_TYPE_F16 ? 0 : need / (nblk ? nblk : 1);
    auto work = [&](uint64_t b0, uint64_t b1) {
        if (type == WH_TYPE_F16) {
            for (uint64_t i = b0 * 32; i < std::min(n, b1 * 32); i++) store_f16(dst + 2 * i, src[i]);
            return;
        }
        for (uint64_t b = b0; b < b1; b++) {
            std::memset(dst + b * bbytes, 0, bbytes);
            const uint64_t base = b * 32;
            quant_block(type, src + base, (int)std::min<uint64_t>(32, n - base), dst + b * bbytes);
        }
    };
    int nt = std::max(1, threads);
    if ((uint64_t)nt > nblk / 4096 + 1) nt = (int)(nblk / 4096 + 1);
    if (nt <= 1) {
        work(0, nblk);
        return WH_OK;
    }
    std::vector<std::thread> th;
    for (int t = 0; t < nt; t++) th.emplace_back(work, nblk * t / nt, nblk * (t + 1) / nt);
    for (auto &x : th) x.join();
    return WH_OK;
}

// internal/gguf/quant.go:236-248.
int should_quantize(const char *name) {
    std::string s(name ? name : "");
    for (auto &c : s) c = (char)std::tolower((unsigned char)c);
    auto ends = [&](const char *suf) {
        size_t k = std::strlen(suf);
        return s.size() >= k && s.compare(s.size() - k, k, suf) == 0;
    };
    if (s.find("norm") != std::string::npos || s.find(".ln") != std::string::npos) return 0;
    if (ends(".bias")) return 0;
    return ends(".weight") ? 1 : 0;
}

// ---- device planes ----------------------------------------------------------
static uint64_t align256(uint64_t x) { return (x + 255) & ~uint64_t(255); }

struct Plan {
    uint64_t qs_bytes, qh_bytes, sc_bytes, qh_off, sc_off, total;
};

static Plan plan_of(uint32_t type, int32_t rows, int32_t nb) {
    Plan p{};
    const uint64_t blocks = (uint64_t)rows * nb;
    if (type == WH_TYPE_F32 || type == WH_TYPE_F16) {
        p.qs_bytes = blocks * 32 * 4;
    } else if (type == WH_TYPE_Q8_0) {
        p.qs_bytes = blocks * 32;
        p.sc_bytes = blocks * 2;
    } else {
        p.qs_bytes = blocks * 16;
        p.sc_bytes = blocks * ((type == WH_TYPE_Q4_1 || type == WH_TYPE_Q5_1) ? 4 : 2);
        if (type == WH_TYPE_Q5_0 || type == WH_TYPE_Q5_1) p.qh_bytes = blocks * 4;
    }
    p.qh_off = align256(p.qs_bytes);
    p.sc_off = align256(p.qh_off + p.qh_bytes);
    p.total = align256(p.sc_off + p.sc_bytes);
    return p;
}

int devmat_plan(DevMat &m, uint32_t type, int32_t rows, int32_t cols) {
    if (rows <= 0 || cols <= 0) return fail(WH_ERR_INVALID, "NewQuantizedMatrix: invalid dims");
    if (!(type == WH_TYPE_F32 || type == WH_TYPE_F16 || is_quant_type(type)))
        return fail(WH_ERR_UNSUPPORTED, "unsupported quant type " + std::to_string(type));
    m.type = (type == WH_TYPE_F16) ? WH_TYPE_F32 : type;  // F16 is widened exactly at upload
    m.rows = rows;
    m.cols = cols;
    m.nb = (cols + 31) / 32;
    m.algo_bytes = (uint64_t)rows * gguf_row_bytes(type, (uint64_t)cols);
    m.dev_bytes = plan_of(type, rows, m.nb).total;
    return WH_OK;
}

// Scatter the raw GGUF rows (source type `src_type`) into the staging image of
// the device allocation.
static void pack_rows(uint32_t src_type, int32_t r0, int32_t r1, int32_t cols, int32_t nb, const uint8_t *raw,
                      uint8_t *img, const Plan &p) {
    const uint64_t rb = gguf_row_bytes(src_type, (uint64_t)cols);
    for (int32_t r = r0; r < r1; r++) {
        const uint8_t *row = raw + (uint64_t)r * rb;
        if (src_type == WH_TYPE_F32 || src_type == WH_TYPE_F16) {
            float *o = (float *)img + (uint64_t)r * nb * 32;
            for (int32_t c = 0; c < nb * 32; c++) {
                float v = 0.0f;
                if (c < cols) {
                    if (src_type == WH_TYPE_F32) std::memcpy(&v, row + 4 * (uint64_t)c, 4);
                    else v = f16_to_f32((uint16_t)(row[2 * c] | (row[2 * c + 1] << 8)));
                }
                o[c] = v;
            }
            continue;
        }
        for (int32_t b = 0; b < nb; b++) {
            const uint64_t blk = (uint64_t)r * nb + b;
            switch (src_type) {
            case WH_TYPE_Q8_0: {
                const uint8_t *s = row + (uint64_t)b * 34;
                std::memcpy(img + p.sc_off + blk * 2, s, 2);
                std::memcpy(img + blk * 32, s + 2, 32);
                break;
            }
            case WH_TYPE_Q4_0: {
                const uint8_t *s = row + (uint64_t)b * 18;
                std::memcpy(img + p.sc_off + blk * 2, s, 2);
                std::memcpy(img + blk * 16, s + 2, 16);
                break;
            }
            case WH_TYPE_Q4_1: {
                const uint8_t *s = row + (uint64_t)b * 20;
                std::memcpy(img + p.sc_off + blk * 4, s, 4);
                std::memcpy(img + blk * 16, s + 4, 16);
                break;
            }
            case WH_TYPE_Q5_0: {
                const uint8_t *s = row + (uint64_t)b * 22;
                std::memcpy(img + p.sc_off + blk * 2, s, 2);
                std::memcpy(img + p.qh_off + blk * 4, s + 2, 4);
                std::memcpy(img + blk * 16, s + 6, 16);
                break;
            }
            case WH_TYPE_Q5_1: {
                const uint8_t *s = row + (uint64_t)b * 24;
                std::memcpy(img + p.sc_off + blk * 4, s, 4);
                std::memcpy(img + p.qh_off + blk * 4, s + 4, 4);
                std::memcpy(img + blk * 16, s + 8, 16);
                break;
            }
            default: break;
            }
        }
    }
}

int devmat_upload_typed(DevMat &m, uint32_t src_type, const uint8_t *raw, uint64_t nbytes) {
    const uint64_t need = (uint64_t)m.rows * gguf_row_bytes(src_type, (uint64_t)m.cols);
    if (nbytes < need)
        return fail(WH_ERR_INVALID, "NewQuantizedMatrix: short data got=" + std::to_string(nbytes) +
                                        " need=" + std::to_string(need));
    const Plan p = plan_of(src_type, m.rows, m.nb);
    std::vector<uint8_t> img(p.total, 0);
    const int nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    if (m.rows >= 256 && nt > 1) {
        std::vector<std::thread> th;
        for (int t = 0; t < nt; t++)
            th.emplace_back(pack_rows, src_type, (int32_t)((int64_t)m.rows * t / nt),
                            (int32_t)((int64_t)m.rows * (t + 1) / nt), m.cols, m.nb, raw, img.data(), std::cref(p));
        for (auto &x : th) x.join();
    } else {
        pack_rows(src_type, 0, m.rows, m.cols, m.nb, raw, img.data(), p);
    }
    void *d = nullptr;
    WH_HIP(hipMalloc(&d, p.total));
    hipError_t e = hipMemcpy(d, img.data(), p.total, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(d);
        return fail(WH_ERR_HIP, std::string("hip: upload: ") + hipGetErrorString(e));
    }
    m.alloc = d;
    m.qs = d;
    m.qh = p.qh_bytes ? (uint32_t *)((uint8_t *)d + p.qh_off) : nullptr;
    m.sc = p.sc_bytes ? (void *)((uint8_t *)d + p.sc_off) : nullptr;
    m.dev_bytes = p.total;
    return WH_OK;
}

int devmat_stack(std::vector<DevMat *> parts, DevMat &out) {
    if (parts.empty()) return fail(WH_ERR_INVALID, "stack: no matrices");
    const uint32_t type = parts[0]->type;
    const int32_t cols = parts[0]->cols;
    int32_t rows = 0;
    for (DevMat *p : parts) {
        if (p->type != type || p->cols != cols || !p->alloc) return fail(WH_ERR_INVALID, "stack: incompatible matrices");
        rows += p->rows;
    }
    DevMat m;
    int rc = devmat_plan(m, type, rows, cols);
    if (rc) return rc;
    const Plan pl = plan_of(type, rows, m.nb);
    void *d = nullptr;
    WH_HIP(hipMalloc(&d, pl.total));
    const uint64_t qs_row = pl.qs_bytes / (uint64_t)rows, sc_row = pl.sc_bytes / (uint64_t)rows,
                   qh_row = pl.qh_bytes / (uint64_t)rows;
    uint64_t r0 = 0;
    for (DevMat *p : parts) {
        const uint64_t n = (uint64_t)p->rows;
        hipError_t e = hipMemcpy((uint8_t *)d + r0 * qs_row, p->qs, n * qs_row, hipMemcpyDeviceToDevice);
        if (e == hipSuccess && sc_row)
            e = hipMemcpy((uint8_t *)d + pl.sc_off + r0 * sc_row, p->sc, n * sc_row, hipMemcpyDeviceToDevice);
        if (e == hipSuccess && qh_row)
            e = hipMemcpy((uint8_t *)d + pl.qh_off + r0 * qh_row, p->qh, n * qh_row, hipMemcpyDeviceToDevice);
        if (e != hipSuccess) {
            (void)hipFree(d);
            return fail(WH_ERR_HIP, std::string("hip: stack copy: ") + hipGetErrorString(e));
        }
        r0 += n;
    }
    m.alloc = d;
    m.qs = d;
    m.sc = pl.sc_bytes ? (void *)((uint8_t *)d + pl.sc_off) : nullptr;
    m.qh = pl.qh_bytes ? (uint32_t *)((uint8_t *)d + pl.qh_off) : nullptr;
    m.dev_bytes = pl.total;
    r0 = 0;
    for (DevMat *p : parts) {
        devmat_free(*p);
        p->qs = (uint8_t *)d + r0 * qs_row;
        p->sc = sc_row ? (void *)((uint8_t *)m.sc + r0 * sc_row) : nullptr;
        p->qh = qh_row ? (uint32_t *)((uint8_t *)m.qh + r0 * qh_row) : nullptr;
        r0 += (uint64_t)p->rows;
    }
    out = m;
    return WH_OK;
}

void devmat_free(DevMat &m) {
    if (m.alloc) (void)hipFree(m.alloc);
    m.alloc = m.qs = m.sc = nullptr;
    m.qh = nullptr;
}

}  // namespace wh

namespace wh {

// internal/gguf/dequant.go:47-201 on the host (used for the float vectors and
// float-path matrices of a model, which the reference dequantises at load).
int dequantize_host(uint32_t type, const uint8_t *raw, uint64_t n, float *out) {
    const uint64_t nb = (n + 31) / 32;
    auto rd16 = [](const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); };
    switch (type) {
    case WH_TYPE_F32: std::memcpy(out, raw, n * 4); return WH_OK;
    case WH_TYPE_F16:
        for (uint64_t i = 0; i < n; i++) out[i] = f16_to_f32(rd16(raw + 2 * i));
        return WH_OK;
    default: break;
    }
    if (!is_quant_type(type)) return fail(WH_ERR_UNSUPPORTED, "unsupported dtype: " + std::to_string(type));
    const uint64_t bb = gguf_row_bytes(type, 32);
    for (uint64_t b = 0; b < nb; b++) {
        const uint8_t *blk = raw + b * bb;
        const uint64_t base = b * 32;
        for (int j = 0; j < 32 && base + j < n; j++) {
            float v = 0.0f;
            if (type == WH_TYPE_Q8_0) {
                v = f16_to_f32(rd16(blk)) * (float)(int8_t)blk[2 + j];
            } else {
                const uint8_t *qs = blk + (type == WH_TYPE_Q4_0 ? 2 : type == WH_TYPE_Q4_1 ? 4 : type == WH_TYPE_Q5_0 ? 6 : 8);
                uint32_t nib = (j & 1) ? (qs[j >> 1] >> 4) : (qs[j >> 1] & 0xF);
                if (type == WH_TYPE_Q5_0 || type == WH_TYPE_Q5_1) {
                    uint32_t qh;
                    std::memcpy(&qh, blk + (type == WH_TYPE_Q5_0 ? 2 : 4), 4);
                    nib |= ((qh >> j) & 1u) << 4;
                }
                const float d = f16_to_f32(rd16(blk));
                if (type == WH_TYPE_Q4_0) v = d * (float)((int32_t)nib - 8);
                else if (type == WH_TYPE_Q5_0) v = d * (float)((int32_t)nib - 16);
                else {
                    volatile float t = d * (float)nib;  // two rounded ops, never fused
                    v = t + f16_to_f32(rd16(blk + 2));
                }
            }
            out[base + j] = v;
        }
    }
    return WH_OK;
}

}  // namespace wh
