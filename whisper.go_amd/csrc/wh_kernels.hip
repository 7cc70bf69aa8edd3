// gfx950 kernels for the whisper.go decoder token loop (multi-kernel path).
//
// Each kernel cites the reference function whose arithmetic it carries out
// (paths relative to the reference repository). Accumulation is fp32; the
// summation order differs from the Go code's sequential sums (parity is
// tolerance-based there), except where noted as bit-exact.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>

#include "wh_device.h"
#include "wh_internal.h"

namespace wh {

// ---------------------------------------------------------------------------
// Quantised GEMV: y[m, r] = sum_c x[m, c] * W[r, c]
// (internal/ml/matmul_q8.go:93-139 with the per-block dot kernels :237-429).
// A group of LG lanes owns one row; lane g of the group walks blocks
// g, g+LG, ... so a wavefront streams 64 consecutive 32-weight blocks per
// step with 16-byte loads. Per block the integer codes are formed exactly,
// s = sum q_i x_i is accumulated in fp32 and scaled once by d (plus m*sum x
// for the _1 formats), as the reference AVX2 kernels do
// (internal/ml/matmul_q8_kernels_amd64.go:15-224).
// ---------------------------------------------------------------------------
struct GemvOpDev {
    const uint8_t *qs;
    const void *sc;
    const uint32_t *qh;
    int32_t rows, cols, nb;
    const float *x;
    int32_t ldx;
    float *y;
    int32_t ldy;
    const float *bias;
    const float *res;
    int32_t ldres;
    int32_t gelu;
    int32_t row_begin;
    int32_t tile_begin;  // first 16-row tile of this op in the split-K workspace
};
struct GemvArgs {
    GemvOpDev op[3];
    int32_t nop, batch, total_rows;
    int32_t nsplit;       // k_gemv_mfma: K ranges per row tile (1 = no split)
    uint32_t seq;         // launch number of the workspace (the tag of this launch's partials)
    uint64_t *part;       // [tile][nsplit][256] {tag, value} partial tiles when nsplit > 1
    uint32_t *cnt;        // [tile] arrivals, zero between launches
};

// Decode block `blk` of a row into integer-valued floats q[32] and return the
// scale d (and, for _1 formats, m).
template <int TYPE>
__device__ __forceinline__ void load_block(const GemvOpDev &op, size_t blk, float q[32], float &d, float &mm) {
    mm = 0.0f;
    if constexpr (TYPE == 0) {
        const float4 *p = (const float4 *)((const float *)op.qs + blk * 32);
#pragma unroll
        for (int t = 0; t < 8; t++) {
            float4 v = p[t];
            q[4 * t] = v.x; q[4 * t + 1] = v.y; q[4 * t + 2] = v.z; q[4 * t + 3] = v.w;
        }
        d = 1.0f;
    } else if constexpr (TYPE == 8) {
        const uint4 *p = (const uint4 *)(op.qs + blk * 32);
        uint4 a = p[0], b = p[1];
        uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int t = 0; t < 8; t++) {
            int v = (int)w[t];
            q[4 * t + 0] = (float)((v << 24) >> 24);
            q[4 * t + 1] = (float)((v << 16) >> 24);
            q[4 * t + 2] = (float)((v << 8) >> 24);
            q[4 * t + 3] = (float)(v >> 24);
        }
        d = h2f(((const uint16_t *)op.sc)[blk]);
    } else {
        uint4 a = *(const uint4 *)(op.qs + blk * 16);
        uint32_t w[4] = {a.x, a.y, a.z, a.w};
        uint32_t hbits = 0;
        if constexpr (TYPE == 6 || TYPE == 7) hbits = op.qh[blk];
        const float off = (TYPE == 2) ? 8.0f : (TYPE == 6 ? 16.0f : 0.0f);
#pragma unroll
        for (int t = 0; t < 4; t++) {
#pragma unroll
            for (int k = 0; k < 4; k++) {
                uint32_t byte = (w[t] >> (8 * k)) & 0xFFu;
                uint32_t lo = byte & 0xFu, hi = byte >> 4;
                int e0 = 8 * t + 2 * k, e1 = e0 + 1;
                if constexpr (TYPE == 6 || TYPE == 7) {
                    lo |= ((hbits >> e0) & 1u) << 4;
                    hi |= ((hbits >> e1) & 1u) << 4;
                }
                q[e0] = (float)lo - off;
                q[e1] = (float)hi - off;
            }
        }
        if constexpr (TYPE == 3 || TYPE == 7) {
            uint32_t s = ((const uint32_t *)op.sc)[blk];
            d = h2f(s & 0xFFFFu);
            mm = h2f(s >> 16);
        } else {
            d = h2f(((const uint16_t *)op.sc)[blk]);
        }
    }
}

template <int TYPE, int LG, int MAXB, bool SAFE>
__global__ __launch_bounds__(256) void k_gemv(GemvArgs a) {
    constexpr int GPW = 64 / LG;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int gl = lane % LG;
    const int grow = (blockIdx.x * 4 + wave) * GPW + lane / LG;
    if (grow >= a.total_rows) return;
    int oi = 0;
    if (a.nop > 1 && grow >= a.op[1].row_begin) oi = 1;
    if (a.nop > 2 && grow >= a.op[2].row_begin) oi = 2;
    const GemvOpDev &op = a.op[oi];
    const int r = grow - op.row_begin;
    const int batch = a.batch;

    float acc[MAXB];
#pragma unroll
    for (int m = 0; m < MAXB; m++) acc[m] = 0.0f;

    for (int b = gl; b < op.nb; b += LG) {
        float q[32], d, mm;
        size_t blk = (size_t)r * op.nb + b;
        load_block<TYPE>(op, blk, q, d, mm);
        const int c0 = b * 32;
#pragma unroll
        for (int m = 0; m < MAXB; m++) {
            if (m < batch) {
                const float *xp = op.x + (size_t)m * op.ldx + c0;
                float s = 0.0f, sx = 0.0f;
                if (!SAFE) {
                    const float4 *x4 = (const float4 *)xp;
#pragma unroll
                    for (int t = 0; t < 8; t++) {
                        float4 v = x4[t];
                        s += q[4 * t] * v.x + q[4 * t + 1] * v.y + q[4 * t + 2] * v.z + q[4 * t + 3] * v.w;
                        if constexpr (TYPE == 3 || TYPE == 7) sx += (v.x + v.y) + (v.z + v.w);
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < 32; i++) {
                        float v = (c0 + i < op.cols) ? xp[i] : 0.0f;
                        s += q[i] * v;
                        if constexpr (TYPE == 3 || TYPE == 7) sx += v;
                    }
                }
                if constexpr (TYPE == 3 || TYPE == 7) acc[m] += d * s + mm * sx;
                else acc[m] += d * s;
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MAXB; m++) acc[m] = group_sum<LG>(acc[m]);

    // epilogue: lane m of the group writes batch row m
    for (int m = gl; m < batch && m < MAXB; m += LG) {
        float v = 0.0f;
#pragma unroll
        for (int j = 0; j < MAXB; j++)
            if (j == m) v = acc[j];
        if (op.bias) v = v + op.bias[r];
        if (op.gelu) v = gelu_ref(v);
        if (op.res) v = op.res[(size_t)m * op.ldres + r] + v;
        op.y[(size_t)m * op.ldy + r] = v;
    }
}

// ---------------------------------------------------------------------------
// Raw blocks for the LDS-staged GEMVs below: a lane loads a block's code bytes,
// scale word(s) and Q5 high bits as they sit in the device layout (16-byte loads
// for the codes) and decodes them where it multiplies.
// ---------------------------------------------------------------------------
struct RawBlk {
    uint4 a, b;  // 32 code bytes (Q8_0), or 16 (a) for the 4/5-bit formats
    uint32_t s, h;  // scale word(s), Q5 high bits
};

template <int TYPE>
__device__ __forceinline__ void raw_load(const GemvOpDev &op, size_t blk, RawBlk &r) {
    if constexpr (TYPE == 8) {
        const uint4 *p = (const uint4 *)(op.qs + blk * 32);
        r.a = p[0];
        r.b = p[1];
        r.s = ((const uint16_t *)op.sc)[blk];
        r.h = 0u;
    } else {
        r.a = *(const uint4 *)(op.qs + blk * 16);
        r.b = make_uint4(0u, 0u, 0u, 0u);
        if constexpr (TYPE == 3 || TYPE == 7) r.s = ((const uint32_t *)op.sc)[blk];
        else r.s = ((const uint16_t *)op.sc)[blk];
        if constexpr (TYPE == 6 || TYPE == 7) r.h = op.qh[blk];
        else r.h = 0u;
    }
}

// ---- quantised GEMV with x staged in LDS ----
// A workgroup stages each batch row of x once as float4 chunks, chunk k (elements
// 32b+4k..32b+4k+3) of block b at slot 8b + ((k + b) & 7): the LG lanes of a row read
// LG consecutive blocks at the same k, which fall in distinct banks, and the other
// rows of the wave read the same slots. LG lanes per weight row, up to KB blocks per
// lane, one weight row per lane group; its raw blocks are loaded once for the batch.
constexpr int GEMV2_KB = 5;

__device__ __forceinline__ int xslot(int b, int k) { return 8 * b + ((k + b) & 7); }

// Codes are taken as floats: signed for Q8_0, unsigned for the 4/5-bit formats (the
// offset, 8 or 16, and the _1 formats' m are applied through sx, the sum of the
// block's 32 x, by block_scale).
// the block's contribution from qx = sum q_i x_i and sx = sum x_i
template <int TYPE>
__device__ __forceinline__ float block_scale(const RawBlk &r, float qx, float sx) {
    if constexpr (TYPE == 8) return h2f(r.s) * qx;
    else if constexpr (TYPE == 2) return h2f(r.s) * __builtin_fmaf(-8.0f, sx, qx);
    else if constexpr (TYPE == 6) return h2f(r.s) * __builtin_fmaf(-16.0f, sx, qx);
    else return __builtin_fmaf(h2f(r.s & 0xFFFFu), qx, h2f(r.s >> 16) * sx);
}

// batch 1: codes made chunk by chunk inside the FMA chains
template <int TYPE>
__device__ __forceinline__ float lds_dot(const RawBlk &r, const float4 *xs, int b, float sx) {
    float acc = 0.0f, acc1 = 0.0f;
    if constexpr (TYPE == 8) {
        const uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const float4 xv = xs[xslot(b, t)];
            const int v = (int)w[t];
            float &c = (t & 1) ? acc1 : acc;
            c = __builtin_fmaf((float)((v << 24) >> 24), xv.x, c);
            c = __builtin_fmaf((float)((v << 16) >> 24), xv.y, c);
            c = __builtin_fmaf((float)((v << 8) >> 24), xv.z, c);
            c = __builtin_fmaf((float)(v >> 24), xv.w, c);
        }
    } else {
        const uint32_t w[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const float4 xa = xs[xslot(b, 2 * t)], xb = xs[xslot(b, 2 * t + 1)];
            uint32_t lo = w[t] & 0x0F0F0F0Fu, hi = (w[t] >> 4) & 0x0F0F0F0Fu;
            if constexpr (TYPE == 6 || TYPE == 7) {
                const uint32_t hb = (r.h >> (8 * t)) & 0xFFu;
                lo |= ((hb & 0x55u) * 0x00410410u) & 0x10101010u;
                hi |= (((hb >> 1) & 0x55u) * 0x00410410u) & 0x10101010u;
            }
            float &c = (t & 1) ? acc1 : acc;
            c = __builtin_fmaf((float)(lo & 0xFFu), xa.x, c);
            c = __builtin_fmaf((float)(hi & 0xFFu), xa.y, c);
            c = __builtin_fmaf((float)((lo >> 8) & 0xFFu), xa.z, c);
            c = __builtin_fmaf((float)((hi >> 8) & 0xFFu), xa.w, c);
            c = __builtin_fmaf((float)((lo >> 16) & 0xFFu), xb.x, c);
            c = __builtin_fmaf((float)((hi >> 16) & 0xFFu), xb.y, c);
            c = __builtin_fmaf((float)(lo >> 24), xb.z, c);
            c = __builtin_fmaf((float)(hi >> 24), xb.w, c);
        }
    }
    return block_scale<TYPE>(r, acc + acc1, sx);
}

// Batch 1: one weight row per lane group, all of x staged (nb * 132 bytes of LDS).
template <int TYPE, int LG>
__global__ __launch_bounds__(256) void k_gemv1(GemvArgs a) {
    constexpr int KB = GEMV2_KB, GPW = 64 / LG;
    extern __shared__ float4 xs[];  // 8 * nb chunks, then the nb block sums
    const GemvOpDev &op = a.op[blockIdx.y];
    const int nb = op.nb;
    const int row0 = blockIdx.x * 4 * GPW;
    if (row0 >= op.rows) return;  // the whole workgroup: past this op's rows
    const int lane = threadIdx.x & 63, gl = lane % LG;
    const int row = row0 + (threadIdx.x >> 6) * GPW + lane / LG;
    const int r = min(row, op.rows - 1);  // past the last row: re-read it, drop it
    // the weights first: their loads are in flight while x is staged
    RawBlk blk[KB];
#pragma unroll
    for (int k = 0; k < KB; k++)
        if (LG * k < nb) raw_load<TYPE>(op, (size_t)r * nb + min(gl + LG * k, nb - 1), blk[k]);
    const int nch = 8 * nb;
    float *sxs = (float *)(xs + nch);
    const bool vec = (((uintptr_t)op.x) & 15) == 0;
    for (int c = threadIdx.x; c < nch; c += 256) {
        const int e = 4 * c;
        float4 v;
        if (vec && e + 3 < op.cols) {
            v = ((const float4 *)op.x)[c];
        } else {
            v.x = e < op.cols ? op.x[e] : 0.0f;
            v.y = e + 1 < op.cols ? op.x[e + 1] : 0.0f;
            v.z = e + 2 < op.cols ? op.x[e + 2] : 0.0f;
            v.w = e + 3 < op.cols ? op.x[e + 3] : 0.0f;
        }
        xs[xslot(c >> 3, c & 7)] = v;
    }
    __syncthreads();
    if constexpr (TYPE != 8) {
        for (int b = threadIdx.x; b < nb; b += 256) {
            float s = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const float4 v = xs[xslot(b, k)];
                s += (v.x + v.y) + (v.z + v.w);
            }
            sxs[b] = s;
        }
        __syncthreads();
    }
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < KB; k++) {
        const int b = gl + LG * k;
        if (b < nb) acc += lds_dot<TYPE>(blk[k], xs, b, TYPE == 8 ? 0.0f : sxs[b]);
    }
    acc = group_sum<LG>(acc);
    if (gl == 0 && row < op.rows) {
        float v = acc;
        if (op.bias) v = v + op.bias[row];
        if (op.gelu) v = gelu_ref(v);
        if (op.res) v = op.res[row] + v;
        op.y[row] = v;
    }
}

// codes of elements 4c..4c+3 of one raw block (c = 0..7), as block_codes makes them
template <int TYPE>
__device__ __forceinline__ void chunk_codes(const RawBlk &r, int c, float (&q)[4]) {
    if constexpr (TYPE == 8) {
        const uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
        const int v = (int)w[c];
        q[0] = (float)((v << 24) >> 24);
        q[1] = (float)((v << 16) >> 24);
        q[2] = (float)((v << 8) >> 24);
        q[3] = (float)(v >> 24);
    } else {
        const uint32_t w[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
        const int t = c >> 1, sh = 16 * (c & 1);  // bytes 2c, 2c + 1: word c / 2
        uint32_t lo = w[t] & 0x0F0F0F0Fu, hi = (w[t] >> 4) & 0x0F0F0F0Fu;
        if constexpr (TYPE == 6 || TYPE == 7) {
            const uint32_t hb = (r.h >> (8 * t)) & 0xFFu;
            lo |= ((hb & 0x55u) * 0x00410410u) & 0x10101010u;
            hi |= (((hb >> 1) & 0x55u) * 0x00410410u) & 0x10101010u;
        }
        q[0] = (float)((lo >> sh) & 0xFFu);
        q[1] = (float)((hi >> sh) & 0xFFu);
        q[2] = (float)((lo >> (sh + 8)) & 0xFFu);
        q[3] = (float)((hi >> (sh + 8)) & 0xFFu);
    }
}

// the raw words through an empty asm statement: codes made from the copy are made
// where they are used, not hoisted out of the chunk loop for all blocks at once
template <int TYPE>
__device__ __forceinline__ RawBlk opaque_blk(const RawBlk &b) {
    RawBlk r = b;
    asm volatile("" : "+v"(r.a.x), "+v"(r.a.y), "+v"(r.a.z), "+v"(r.a.w));
    if constexpr (TYPE == 8) asm volatile("" : "+v"(r.b.x), "+v"(r.b.y), "+v"(r.b.z), "+v"(r.b.w));
    if constexpr (TYPE == 6 || TYPE == 7) asm volatile("" : "+v"(r.h));
    return r;
}

// A batch of up to NB rows of x (the rows from batch to NB staged as zeros): two
// adjacent weight rows per lane group, so each x chunk read from LDS feeds both.
template <int TYPE, int LG, int NB>
__global__ __launch_bounds__(256) void k_gemv2(GemvArgs a, int ch) {
    constexpr int KB = GEMV2_KB, GPW = 64 / LG, RW = 2, XR = 4;
    // per batch row m: 8 * ch chunks of x, then ch block sums
    extern __shared__ float4 xs[];
    const GemvOpDev &op = a.op[blockIdx.y];
    const int nb = op.nb, batch = a.batch;
    const int row0 = blockIdx.x * 4 * GPW * RW;
    if (row0 >= op.rows) return;  // the whole workgroup: past this op's rows
    const int lane = threadIdx.x & 63, gl = lane % LG;
    const int row = row0 + ((threadIdx.x >> 6) * GPW + lane / LG) * RW;
    const int stride = 8 * ch + ch / 4;  // float4s per batch row (ch is a multiple of 4)
    const bool vec = (((uintptr_t)op.x) & 15) == 0 && (op.ldx & 3) == 0 && (op.cols & 3) == 0;
    // x is staged in rounds of up to XR float4 chunks per thread, all of a round's
    // loads before its stores; the first round is loaded before the weights (x is
    // small and cached, and no wait for the weights stands before its loads). x not
    // 16-byte aligned, or cols not a multiple of 4: a plain loop (x_slow) instead.
    float4 xv[XR];
    auto x_round = [&](int cb, int i0) {
        if (!vec) return;
        const int nch = 8 * min(ch, nb - cb), nall = NB * nch;
#pragma unroll
        for (int j = 0; j < XR; j++) {
            const int i = i0 + 256 * j + threadIdx.x;
            const int m = i / nch, c = i - m * nch;
            const int e = 32 * cb + 4 * c;
            xv[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (i < nall && m < batch && e < op.cols) xv[j] = *(const float4 *)(op.x + (size_t)m * op.ldx + e);
        }
    };
    x_round(0, 0);
    // the weights: in flight while x is staged
    RawBlk blk[RW][KB];
#pragma unroll
    for (int u = 0; u < RW; u++) {
        const int r = min(row + u, op.rows - 1);  // past the last row: re-read it, drop it
#pragma unroll
        for (int k = 0; k < KB; k++)
            if (LG * k < nb) raw_load<TYPE>(op, (size_t)r * nb + min(gl + LG * k, nb - 1), blk[u][k]);
    }
    float acc[RW][NB];
#pragma unroll
    for (int u = 0; u < RW; u++)
#pragma unroll
        for (int m = 0; m < NB; m++) acc[u][m] = 0.0f;
    // column chunks of ch blocks (one chunk whenever x fits): ch is a multiple of LG,
    // so block gl + LG * k of every lane lies in the same chunk
    for (int cb = 0; cb < nb; cb += ch) {
        const int nbc = min(ch, nb - cb), nch = 8 * nbc, nall = NB * nch;
        if (vec) {
            for (int i0 = 0; i0 < nall; i0 += 256 * XR) {
                if (cb > 0 || i0 > 0) x_round(cb, i0);
#pragma unroll
                for (int j = 0; j < XR; j++) {
                    const int i = i0 + 256 * j + threadIdx.x;
                    const int m = i / nch, c = i - m * nch;
                    if (i < nall) xs[m * stride + xslot(c >> 3, c & 7)] = xv[j];
                }
            }
        } else {
            for (int i = threadIdx.x; i < 4 * nall; i += 256) {  // x_slow: one float each
                const int q = i >> 2, m = q / nch, c = q - m * nch, e = 32 * cb + 4 * c + (i & 3);
                const float v = (m < batch && e < op.cols) ? op.x[(size_t)m * op.ldx + e] : 0.0f;
                ((float *)(xs + m * stride + xslot(c >> 3, c & 7)))[i & 3] = v;
            }
        }
        __syncthreads();
        if constexpr (TYPE != 8) {
            for (int i = threadIdx.x; i < NB * nbc; i += 256) {
                const int m = i / nbc, b = i - m * nbc;
                float s = 0.0f;
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const float4 v = xs[m * stride + xslot(b, k)];
                    s += (v.x + v.y) + (v.z + v.w);
                }
                ((float *)(xs + m * stride + 8 * ch))[b] = s;
            }
            __syncthreads();
        }
#pragma unroll
        for (int k = 0; k < KB; k++) {
            const int b = gl + LG * k;
            if (LG * k >= cb && LG * k < cb + ch && b < nb) {
                const int bl = b - cb;
                // the sums pass through an empty asm statement that also clobbers
                // memory: the FMAs of block k - 1 come before it and the LDS reads of
                // block k after it (likewise per chunk below); the reads of all blocks
                // and chunks issued together would not fit the registers
#pragma unroll
                for (int m = 0; m < NB; m++) asm volatile("" : "+v"(acc[0][m]), "+v"(acc[1][m])::"memory");
                const RawBlk ra = opaque_blk<TYPE>(blk[0][k]), rb = opaque_blk<TYPE>(blk[1][k]);
                float pa[NB], pb[NB];
#pragma unroll
                for (int m = 0; m < NB; m++) pa[m] = pb[m] = 0.0f;
#pragma unroll
                for (int c = 0; c < 8; c++) {
#pragma unroll
                    for (int m = 0; m < NB; m++) asm volatile("" : "+v"(pa[m]), "+v"(pb[m])::"memory");
                    float qa[4], qb[4];
                    chunk_codes<TYPE>(ra, c, qa);
                    chunk_codes<TYPE>(rb, c, qb);
#pragma unroll
                    for (int m = 0; m < NB; m++) {
                        const float4 xv = xs[m * stride + xslot(bl, c)];
                        pa[m] = __builtin_fmaf(qa[0], xv.x, pa[m]);
                        pb[m] = __builtin_fmaf(qb[0], xv.x, pb[m]);
                        pa[m] = __builtin_fmaf(qa[1], xv.y, pa[m]);
                        pb[m] = __builtin_fmaf(qb[1], xv.y, pb[m]);
                        pa[m] = __builtin_fmaf(qa[2], xv.z, pa[m]);
                        pb[m] = __builtin_fmaf(qb[2], xv.z, pb[m]);
                        pa[m] = __builtin_fmaf(qa[3], xv.w, pa[m]);
                        pb[m] = __builtin_fmaf(qb[3], xv.w, pb[m]);
                    }
                }
#pragma unroll
                for (int m = 0; m < NB; m++) {
                    const float sx = TYPE == 8 ? 0.0f : ((const float *)(xs + m * stride + 8 * ch))[bl];
                    acc[0][m] += block_scale<TYPE>(ra, pa[m], sx);
                    acc[1][m] += block_scale<TYPE>(rb, pb[m], sx);
                }
            }
        }
        if (cb + ch < nb) __syncthreads();  // the next chunk overwrites x
    }
    // every lane of a group holds every sum after the butterfly; the group's lanes
    // share the RW * NB outputs (one lane doing them all serialised ten float64 tanh
    // evaluations of the GELU)
    constexpr int NO = RW * NB;
    float sums[NO];
#pragma unroll
    for (int u = 0; u < RW; u++)
#pragma unroll
        for (int m = 0; m < NB; m++) sums[u * NB + m] = group_sum<LG>(acc[u][m]);
#pragma unroll
    for (int p0 = 0; p0 < NO; p0 += LG) {
        const int p = p0 + gl;
        float v = 0.0f;
#pragma unroll
        for (int q = 0; q < NO; q++)
            if (q == p) v = sums[q];
        const int u = p / NB, m = p - u * NB, rr = row + u;
        if (p < NO && m < batch && rr < op.rows) {
            if (op.bias) v = v + op.bias[rr];
            if (op.gelu) v = gelu_ref(v);
            if (op.res) v = op.res[(size_t)m * op.ldres + rr] + v;
            op.y[(size_t)m * op.ldy + rr] = v;
        }
    }
}

// ---- batches up to 16 on the matrix cores ----
// D (16 batch rows x 16 weight rows) += A (16 x 4: x) x B (4 x 16: codes) with
// v_mfma_f32_16x16x4f32: fp32 operands (the codes are small exact integers), fp32
// accumulation. Lane l: batch row / weight row l % 16, k slot kq = l / 16; the j-th
// of a block's 8 products covers columns 4j .. 4j + 3, so the lane takes element
// 4j + kq of its x row and of its weight row; D register i of lane l is batch row
// 4 kq + i, weight row l % 16. Each block's 8 products go to a fresh tile that is
// scaled (d, and the offset or m through the block sums of x) into the total. A
// workgroup takes 16 weight rows; its NW waves take the blocks in turn and their
// tiles are summed through LDS at the end (NW = 4, or 16 for matrices of at most
// 2048 rows, whose 16-row workgroups are too few to fill the chip). x is staged per chunk of CH blocks as
// [block][kq][batch row][j] (two float4 reads per lane per block), rows past the
// batch as zeros: CH = 20 (42 KiB of LDS), or 40 (84 KiB, one workgroup per CU)
// for matrices of at most 2048 rows, whose grid is below the CU count anyway and
// whose time goes to staging rounds (1280x5120 at batch 16: 8 rounds of 20 blocks).
#ifndef GEMVM_MIN_BATCH
#define GEMVM_MIN_BATCH 6
#endif
#ifndef GEMVM_NW_SMALL
#define GEMVM_NW_SMALL 16  // waves per workgroup for matrices of at most 2048 rows
#endif
#ifndef GEMVM_CH_SMALL
#define GEMVM_CH_SMALL 56  // blocks staged per round for matrices of at most 2048 rows
#endif
#ifndef GEMVM_SMALL_ROWS
#define GEMVM_SMALL_ROWS 2048  // matrices up to this many rows use the CH_SMALL, NW_SMALL kernel
#endif
#ifndef GEMVM_CH_TALL
#define GEMVM_CH_TALL 20
#endif
#ifndef GEMVM_NW_TALL
#define GEMVM_NW_TALL 10
#endif
#ifndef GEMVM_WG_TARGET_TALL
#define GEMVM_WG_TARGET_TALL 640  // the same for taller matrices (three 42 KiB workgroups fit a CU)
#endif
#ifndef GEMVM_WG_TARGET
#define GEMVM_WG_TARGET 256  // split K up to this many workgroups
#endif

typedef float gemvm_f4 __attribute__((ext_vector_type(4)));

// element 4j + kq (j = 0..7) of a raw block as a float code (signed for Q8_0)
template <int TYPE>
__device__ __forceinline__ void mfma_codes(const RawBlk &r, int kq, float (&q)[8]) {
    if constexpr (TYPE == 8) {
        const uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
        for (int j = 0; j < 8; j++) q[j] = (float)(int)__builtin_amdgcn_sbfe((int)w[j], 8 * kq, 8);  // the builtin's type is unsigned
    } else {
        const uint32_t w[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
        // element e = 4j + kq: byte 2j + kq / 2, nibble kq & 1
        const int sh0 = 8 * (kq >> 1) + 4 * (kq & 1);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            uint32_t c = (w[j >> 1] >> (16 * (j & 1) + sh0)) & 0xFu;
            if constexpr (TYPE == 6 || TYPE == 7) c |= ((r.h >> (4 * j + kq)) & 1u) << 4;
            q[j] = (float)c;
        }
    }
}

template <int TYPE, int CH, int NW>
__global__ __launch_bounds__(64 * NW) void k_gemv_mfma(GemvArgs a) {
    constexpr int NT = 64 * NW, NBW = (CH + NW - 1) / NW;  // threads; blocks per wave per chunk
    extern __shared__ float xm[];  // CH * 512 floats of x, then CH * 16 block sums
    const GemvOpDev &op = a.op[blockIdx.y];
    const int nb = op.nb, batch = a.batch;
    const int r0 = blockIdx.x * 16;
    if (r0 >= op.rows) return;  // the whole workgroup: past this op's rows
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lr = lane & 15, kq = lane >> 4;
    const int row = min(r0 + lr, op.rows - 1);  // past the last row: re-read it, drop it
    float *sxs = xm + CH * 512;
    const bool vec = (((uintptr_t)op.x) & 15) == 0 && (op.ldx & 3) == 0 && (op.cols & 3) == 0;
    // this workgroup's blocks: split z of a.nsplit equal runs of the row
    const int nsplit = a.nsplit, split = blockIdx.z, per = (nb + nsplit - 1) / nsplit;
    const int kb0 = min(nb, split * per), kb1 = min(nb, kb0 + per);
    gemvm_f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int cb = kb0; cb < kb1; cb += CH) {
        const int nbc = min(CH, kb1 - cb);
        // this wave's blocks of the chunk (cb + wave + NW u): raw loads first
        RawBlk rb[NBW];
#pragma unroll
        for (int u = 0; u < NBW; u++)
            if (wave + NW * u < nbc) raw_load<TYPE>(op, (size_t)row * nb + cb + wave + NW * u, rb[u]);
        // x: 16 batch rows x nbc blocks x 8 float4 (columns 4j .. 4j + 3 of a block)
        const int nall = 16 * nbc * 8;
        if (vec) {
            for (int i0 = 0; i0 < nall; i0 += NT * 4) {
                float4 v[4];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int i = i0 + NT * u + tid, b = i / (nbc * 8), f = i - b * (nbc * 8);
                    const int e = 32 * (cb + (f >> 3)) + 4 * (f & 7);
                    v[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                    if (i < nall && b < batch && e < op.cols) v[u] = *(const float4 *)(op.x + (size_t)b * op.ldx + e);
                }
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int i = i0 + NT * u + tid, b = i / (nbc * 8), f = i - b * (nbc * 8);
                    if (i < nall) {
                        float *o = xm + (((f >> 3) * 4) * 16 + b) * 8 + (f & 7);  // kq = 0
                        o[0] = v[u].x; o[128] = v[u].y; o[256] = v[u].z; o[384] = v[u].w;
                    }
                }
            }
        } else {
            for (int i = tid; i < 4 * nall; i += NT) {
                const int q4 = i >> 2, b = q4 / (nbc * 8), f = q4 - b * (nbc * 8), k = i & 3;
                const int e = 32 * (cb + (f >> 3)) + 4 * (f & 7) + k;
                xm[(((f >> 3) * 4 + k) * 16 + b) * 8 + (f & 7)] =
                    (b < batch && e < op.cols) ? op.x[(size_t)b * op.ldx + e] : 0.0f;
            }
        }
        __syncthreads();
        if constexpr (TYPE != 8) {
            for (int i = tid; i < 16 * nbc; i += NT) {
                const int bl = i >> 4, b = i & 15;
                float sum = 0.0f;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const float4 *p = (const float4 *)(xm + ((bl * 4 + k) * 16 + b) * 8);
                    const float4 p0 = p[0], p1 = p[1];
                    sum += ((p0.x + p0.y) + (p0.z + p0.w)) + ((p1.x + p1.y) + (p1.z + p1.w));
                }
                sxs[bl * 16 + b] = sum;
            }
            __syncthreads();
        }
#pragma unroll
        for (int u = 0; u < NBW; u++) {
            const int bl = wave + NW * u;
            if (bl < nbc) {
                const float4 *xp = (const float4 *)(xm + ((bl * 4 + kq) * 16 + lr) * 8);
                const float4 x0 = xp[0], x1 = xp[1];
                float q[8];
                mfma_codes<TYPE>(rb[u], kq, q);
                gemvm_f4 t = {0.0f, 0.0f, 0.0f, 0.0f};
                t = __builtin_amdgcn_mfma_f32_16x16x4f32(x0.x, q[0], t, 0, 0, 0);
                t = __builtin_amdgcn_mfma_f32_16x16x4f32(x0.y, q[1], t, 0, 0, 0);
                t = __builtin_amdgcn_mfma_f32_16x16x4f32(x0.z, q[2], t, 0, 0, 0);
                t = __builtin_amdgcn_mfma_f32_16x16x4f32(x0.w, q[3], t, 0, 0, 0);
                t = __builtin_amdgcn_mfma_f32_16x16x4f32(x1.x, q[4], t, 0, 0, 0);
                t = __builtin_amdgcn_mfma_f32_16x16x4f32(x1.y, q[5], t, 0, 0, 0);
                t = __builtin_amdgcn_mfma_f32_16x16x4f32(x1.z, q[6], t, 0, 0, 0);
                t = __builtin_amdgcn_mfma_f32_16x16x4f32(x1.w, q[7], t, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float sx = TYPE == 8 ? 0.0f : sxs[bl * 16 + 4 * kq + i];
                    acc[i] += block_scale<TYPE>(rb[u], t[i], sx);
                }
            }
        }
        __syncthreads();  // x and the sums are restaged (or reused for the tiles below)
    }
    // the waves' tiles (NW KiB of LDS), summed in wave order; then one output per
    // thread of the first 256 (batch row t / 16, weight row t % 16) for the epilogue
    gemvm_f4 *red = (gemvm_f4 *)xm;
    float *outs = xm + NW * 64 * 4;
    red[wave * 64 + lane] = acc;
    __syncthreads();
    if (wave == 0) {
        gemvm_f4 sum = red[lane];
#pragma unroll
        for (int w = 1; w < NW; w++) sum += red[w * 64 + lane];
#pragma unroll
        for (int i = 0; i < 4; i++) outs[(4 * kq + i) * 16 + lr] = sum[i];
    }
    __syncthreads();
    float v = tid < 256 ? outs[tid] : 0.0f;
    if (nsplit > 1) {
        // Split K: every split stores its tile as {launch number, value} pairs and
        // counts itself in; the workgroup that arrives last sums the nsplit tiles
        // in split order (the same sum whatever the arrival order) and runs the
        // epilogue. No fences (on this chip they write back or drop the whole L2):
        // the pairs are stored and read at agent scope, and the last workgroup
        // reads each pair until it carries this launch's number (a pair from a
        // workgroup already counted is in flight, so the bounded wait ends at
        // once; a pair that never arrives gives NaN). The counter goes back to 0.
        __shared__ int last;
        const int tile = op.tile_begin + blockIdx.x;
        uint64_t *pt = a.part + (size_t)tile * nsplit * 256;
        const uint64_t tag = (uint64_t)a.seq << 32;
        if (tid < 256)
            __hip_atomic_store(pt + split * 256 + tid, tag | __float_as_uint(v), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (tid == 0)
            last = __hip_atomic_fetch_add(a.cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                   (uint32_t)(nsplit - 1);
        __syncthreads();
        if (!last) return;
        if (tid < 256) {
            // all the other splits' pairs are loaded at once, then any pair not yet
            // carrying this launch's number is read again
            uint64_t pr[GEMVM_MAX_SPLIT];
#pragma unroll
            for (int j = 0; j < GEMVM_MAX_SPLIT; j++)
                if (j < nsplit && j != split)
                    pr[j] = __hip_atomic_load(pt + j * 256 + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            float sum = 0.0f;
#pragma unroll
            for (int j = 0; j < GEMVM_MAX_SPLIT; j++) {
                if (j >= nsplit) break;
                float pj = v;
                if (j != split) {
                    uint64_t q = pr[j];
                    for (int spin = 0; (q & 0xffffffff00000000ull) != tag; spin++) {
                        if (spin >= (1 << 20)) {
                            q = tag | 0x7fc00000u;  // NaN
                            break;
                        }
                        __builtin_amdgcn_s_sleep(1);
                        q = __hip_atomic_load(pt + j * 256 + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
                    pj = __uint_as_float((uint32_t)q);
                }
                sum += pj;
            }
            v = sum;
        }
        if (tid == 0) __hip_atomic_store(a.cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (tid < 256) {
        const int b = tid >> 4, r = r0 + (tid & 15);
        if (b < batch && r < op.rows) {
            if (op.bias) v = v + op.bias[r];
            if (op.gelu) v = gelu_ref(v);
            if (op.res) v = op.res[(size_t)b * op.ldres + r] + v;
            op.y[(size_t)b * op.ldy + r] = v;
        }
    }
}

// Dynamic LDS above the default 64 KiB for one kernel, asked once per device and
// remembered per (weight type, kernel slot K, device) in a bit set; true when granted.
template <int TYPE, int K>
static bool gemvm_lds_granted(const void *kern, size_t lds) {
    if (lds <= 65536) return true;
    static std::atomic<uint32_t> granted{0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 32) return false;
    if ((granted.load() >> dev) & 1u) return true;
    if (hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) return false;
    granted.fetch_or(1u << dev);
    return true;
}

template <int TYPE>
static bool gemvm_launch(GemvArgs &a, int maxrows, GemvWork *work, hipStream_t st) {
    if (a.batch < GEMVM_MIN_BATCH || a.batch > 16) return false;
    // split K while the row tiles of the launch are too few to give every CU a
    // workgroup (matrices of at most 2048 rows, with a workspace)
    int tiles = 0;
    for (int i = 0; i < a.nop; i++) tiles += (a.op[i].rows + 15) / 16;
    a.nsplit = 1;
    if (work && work->part && tiles <= work->tiles) {
        int nsplit = (maxrows <= GEMVM_SMALL_ROWS ? GEMVM_WG_TARGET : GEMVM_WG_TARGET_TALL) / tiles;
        int nbmin = a.op[0].nb;
        for (int i = 1; i < a.nop; i++) nbmin = std::min(nbmin, a.op[i].nb);
        nsplit = std::min(std::min(nsplit, GEMVM_MAX_SPLIT), std::max(1, nbmin / 8));
        if (nsplit > 1) {
            a.nsplit = nsplit;
            a.part = work->part;
            a.cnt = work->cnt;
            a.seq = ++work->seq;
            if (a.seq == 0) a.seq = ++work->seq;  // 0 is the tag of the zeroed buffer
        }
    }
    const dim3 grid((maxrows + 15) / 16, a.nop, a.nsplit);
    if (maxrows <= GEMVM_SMALL_ROWS) {
        constexpr size_t lds = (size_t)GEMVM_CH_SMALL * (512 + 16) * 4;
        if (gemvm_lds_granted<TYPE, 0>((const void *)k_gemv_mfma<TYPE, GEMVM_CH_SMALL, GEMVM_NW_SMALL>, lds)) {
            hipLaunchKernelGGL((k_gemv_mfma<TYPE, GEMVM_CH_SMALL, GEMVM_NW_SMALL>), grid, dim3(64 * GEMVM_NW_SMALL),
                               lds, st, a);
            return true;
        }
    } else {
        constexpr size_t lds = (size_t)GEMVM_CH_TALL * (512 + 16) * 4;
        if (gemvm_lds_granted<TYPE, 1>((const void *)k_gemv_mfma<TYPE, GEMVM_CH_TALL, GEMVM_NW_TALL>, lds)) {
            hipLaunchKernelGGL((k_gemv_mfma<TYPE, GEMVM_CH_TALL, GEMVM_NW_TALL>), grid, dim3(64 * GEMVM_NW_TALL), lds,
                               st, a);
            return true;
        }
    }
    // LDS above 64 KiB refused: 20-block chunks
    hipLaunchKernelGGL((k_gemv_mfma<TYPE, 20, 4>), grid, dim3(256), (size_t)20 * (512 + 16) * 4, st, a);
    return true;
}

constexpr int GEMV2_LDS = 64 * 1024;

// Lanes per row: the fewest (a power of two, at least 4) whose GEMV2_KB blocks each
// cover the row, doubled while the launch would have fewer workgroups than CUs
// (rows_per_group weight rows per lane group).
static int gemv2_lanes(int nbmax, int total_rows, int rows_per_group) {
    int lg = 4;
    while (lg * GEMV2_KB < nbmax) lg *= 2;
    while (lg < 64 && (total_rows + 4 * (64 / lg) * rows_per_group - 1) / (4 * (64 / lg) * rows_per_group) < 256) lg *= 2;
    return lg;
}

template <int TYPE, int LG>
static void gemv1_launch_t(const GemvArgs &a, int maxrows, int nbmax, hipStream_t st) {
    constexpr int rows_per_wg = 4 * (64 / LG);
    const dim3 grid((maxrows + rows_per_wg - 1) / rows_per_wg, a.nop);
    hipLaunchKernelGGL((k_gemv1<TYPE, LG>), grid, dim3(256), (size_t)nbmax * (8 * 16 + 4), st, a);
}

template <int TYPE, int LG, int NB>
static void gemv2_launch_t(const GemvArgs &a, int maxrows, int ch, hipStream_t st) {
    constexpr int rows_per_wg = 4 * (64 / LG) * 2;
    const dim3 grid((maxrows + rows_per_wg - 1) / rows_per_wg, a.nop);
    const size_t lds = (size_t)NB * (8 * ch + ch / 4) * 16;
    hipLaunchKernelGGL((k_gemv2<TYPE, LG, NB>), grid, dim3(256), lds, st, a, ch);
}

template <int TYPE, int NB>
static void gemv2_launch_nb(const GemvArgs &a, int lg, int maxrows, int ch, hipStream_t st) {
    switch (lg) {
    case 4: gemv2_launch_t<TYPE, 4, NB>(a, maxrows, ch, st); break;
    case 8: gemv2_launch_t<TYPE, 8, NB>(a, maxrows, ch, st); break;
    case 16: gemv2_launch_t<TYPE, 16, NB>(a, maxrows, ch, st); break;
    case 32: gemv2_launch_t<TYPE, 32, NB>(a, maxrows, ch, st); break;
    default: gemv2_launch_t<TYPE, 64, NB>(a, maxrows, ch, st); break;
    }
}

// Quantised GEMV with x staged in LDS: batch 1 (x up to 64 * GEMV2_KB blocks) and
// batches 2..5 of matrices with at least 1024 rows; anything else is not handled
// here (k_gemv takes it). Below 1024 rows the batched kernel stages five rows of x
// per workgroup for a few weight rows and k_gemv is faster (768x768 at batch 5:
// 6.7 against 10.2 us; 1280x1280: equal; 5120x1280: 22 against 13 us).
template <int TYPE>
static bool gemv2_launch(const GemvArgs &a, int maxrows, int nbmax, hipStream_t st) {
    if (nbmax > 64 * GEMV2_KB || a.batch > 5 || (a.batch > 1 && maxrows < 1024)) return false;
    if (a.batch == 1) {
        switch (gemv2_lanes(nbmax, a.total_rows, 1)) {
        case 4: gemv1_launch_t<TYPE, 4>(a, maxrows, nbmax, st); break;
        case 8: gemv1_launch_t<TYPE, 8>(a, maxrows, nbmax, st); break;
        case 16: gemv1_launch_t<TYPE, 16>(a, maxrows, nbmax, st); break;
        case 32: gemv1_launch_t<TYPE, 32>(a, maxrows, nbmax, st); break;
        default: gemv1_launch_t<TYPE, 64>(a, maxrows, nbmax, st); break;
        }
        return true;
    }
    const int nb_rows = a.batch == 2 ? 2 : 5;  // rows past the batch are staged as zeros
    const int lg = gemv2_lanes(nbmax, a.total_rows, 2);
    const int per_block = nb_rows * (8 * 16 + 4);  // LDS bytes per block of x
    int ch = ((nbmax + 3) / 4) * 4;
    if (ch * per_block > GEMV2_LDS) {
        // several chunks: each a multiple of LG blocks (one chunk may be any width)
        ch = (GEMV2_LDS / per_block) / lg * lg;
        if (ch < lg) return false;
    }
    if (nb_rows == 2) gemv2_launch_nb<TYPE, 2>(a, lg, maxrows, ch, st);
    else gemv2_launch_nb<TYPE, 5>(a, lg, maxrows, ch, st);
    return true;
}

template <int TYPE, int LG, int MAXB>
static void gemv_launch_t(const GemvArgs &a, bool safe, hipStream_t st) {
    constexpr int rows_per_block = 4 * (64 / LG);
    dim3 grid((a.total_rows + rows_per_block - 1) / rows_per_block);
    if (safe) hipLaunchKernelGGL((k_gemv<TYPE, LG, MAXB, true>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((k_gemv<TYPE, LG, MAXB, false>), grid, dim3(256), 0, st, a);
}

template <int TYPE>
static void gemv_launch_type(const GemvArgs &a, int nb, bool safe, hipStream_t st) {
    const int b = a.batch;
    if (nb <= 16) {
        if (b <= 1) gemv_launch_t<TYPE, 16, 1>(a, safe, st);
        else if (b <= 8) gemv_launch_t<TYPE, 16, 8>(a, safe, st);
        else gemv_launch_t<TYPE, 16, 16>(a, safe, st);
    } else {
        if (b <= 1) gemv_launch_t<TYPE, 64, 1>(a, safe, st);
        else if (b <= 8) gemv_launch_t<TYPE, 64, 8>(a, safe, st);
        else gemv_launch_t<TYPE, 64, 16>(a, safe, st);
    }
}

int launch_gemv(const DevMat *const *mats, const GemvIn *in, const GemvOut *out, int nmat, int batch,
                hipStream_t st, GemvWork *work) {
    if (nmat < 1 || nmat > 3) return fail(WH_ERR_INVALID, "gemv: 1..3 matrices per launch");
    if (batch < 1 || batch > 16) return fail(WH_ERR_INVALID, "gemv: batch must be in [1,16]");
    GemvArgs a;
    memset(&a, 0, sizeof a);
    a.nop = nmat;
    a.batch = batch;
    int total = 0, nbmax = 0, maxrows = 0;
    bool safe = false;
    const uint32_t type = mats[0]->type;
    for (int i = 0; i < nmat; i++) {
        const DevMat &m = *mats[i];
        if (m.type != type) return fail(WH_ERR_INVALID, "gemv: mixed matrix types in one launch");
        GemvOpDev &o = a.op[i];
        o.qs = (const uint8_t *)m.qs;
        o.sc = m.sc;
        o.qh = m.qh;
        o.rows = m.rows;
        o.cols = m.cols;
        o.nb = m.nb;
        o.x = in[i].x;
        o.ldx = in[i].ldx;
        o.y = out[i].y;
        o.ldy = out[i].ldy;
        o.bias = out[i].bias;
        o.res = out[i].res;
        o.ldres = out[i].ldres;
        o.gelu = out[i].gelu;
        o.row_begin = total;
        o.tile_begin = i == 0 ? 0 : a.op[i - 1].tile_begin + (a.op[i - 1].rows + 15) / 16;
        total += m.rows;
        if (m.nb > nbmax) nbmax = m.nb;
        if (m.rows > maxrows) maxrows = m.rows;
        if ((m.cols % 32) != 0 || (in[i].ldx % 4) != 0 || (((uintptr_t)in[i].x) & 15) != 0) safe = true;
    }
    a.total_rows = total;
    bool done = false;
    switch (type) {
    case 2: done = gemv2_launch<2>(a, maxrows, nbmax, st) || gemvm_launch<2>(a, maxrows, work, st); break;
    case 3: done = gemv2_launch<3>(a, maxrows, nbmax, st) || gemvm_launch<3>(a, maxrows, work, st); break;
    case 6: done = gemv2_launch<6>(a, maxrows, nbmax, st) || gemvm_launch<6>(a, maxrows, work, st); break;
    case 7: done = gemv2_launch<7>(a, maxrows, nbmax, st) || gemvm_launch<7>(a, maxrows, work, st); break;
    case 8: done = gemv2_launch<8>(a, maxrows, nbmax, st) || gemvm_launch<8>(a, maxrows, work, st); break;
    default: break;
    }
    if (!done) {
        switch (type) {
        case 0: gemv_launch_type<0>(a, nbmax, safe, st); break;
        case 2: gemv_launch_type<2>(a, nbmax, safe, st); break;
        case 3: gemv_launch_type<3>(a, nbmax, safe, st); break;
        case 6: gemv_launch_type<6>(a, nbmax, safe, st); break;
        case 7: gemv_launch_type<7>(a, nbmax, safe, st); break;
        case 8: gemv_launch_type<8>(a, nbmax, safe, st); break;
        default: return fail(WH_ERR_UNSUPPORTED, "gemv: unsupported matrix type");
        }
    }
    WH_HIP(hipGetLastError());
    return WH_OK;
}

// ---------------------------------------------------------------------------
// Bit-exact row dequantisation (internal/gguf/dequant.go:47-201).
// ---------------------------------------------------------------------------
template <int TYPE>
__global__ void k_dequant_rows(MatView m, int32_t row0, int32_t nrows, float *out) {
    size_t n = (size_t)nrows * m.cols;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        int r = row0 + (int)(i / m.cols);
        int c = (int)(i % m.cols);
        out[i] = dequant_elem<TYPE>(m, r, c >> 5, c & 31);
    }
}

static MatView view_of(const DevMat &d) {
    MatView v;
    v.qs = (const uint8_t *)d.qs;
    v.sc = d.sc;
    v.qh = d.qh;
    v.rows = d.rows;
    v.cols = d.cols;
    v.nb = d.nb;
    return v;
}

int launch_dequant_rows(const DevMat &m, int32_t row0, int32_t nrows, float *out, hipStream_t st) {
    MatView v = view_of(m);
    size_t n = (size_t)nrows * m.cols;
    int grid = (int)((n + 255) / 256);
    if (grid > 65535) grid = 65535;
    if (grid < 1) grid = 1;
    switch (m.type) {
    case 0: hipLaunchKernelGGL(k_dequant_rows<0>, dim3(grid), dim3(256), 0, st, v, row0, nrows, out); break;
    case 2: hipLaunchKernelGGL(k_dequant_rows<2>, dim3(grid), dim3(256), 0, st, v, row0, nrows, out); break;
    case 3: hipLaunchKernelGGL(k_dequant_rows<3>, dim3(grid), dim3(256), 0, st, v, row0, nrows, out); break;
    case 6: hipLaunchKernelGGL(k_dequant_rows<6>, dim3(grid), dim3(256), 0, st, v, row0, nrows, out); break;
    case 7: hipLaunchKernelGGL(k_dequant_rows<7>, dim3(grid), dim3(256), 0, st, v, row0, nrows, out); break;
    case 8: hipLaunchKernelGGL(k_dequant_rows<8>, dim3(grid), dim3(256), 0, st, v, row0, nrows, out); break;
    default: return fail(WH_ERR_UNSUPPORTED, "dequant: unsupported type");
    }
    WH_HIP(hipGetLastError());
    return WH_OK;
}

// ---------------------------------------------------------------------------
// Token + positional embedding (internal/model/decoder.go:756-773). A
// quantised token embedding row is dequantised bit-exactly (the documented
// extension for P4: the reference reads an empty float table there).
// ---------------------------------------------------------------------------
template <int TYPE>
__global__ void k_embed(MatView tok, const float *pos_emb, const int32_t *tokv, const int32_t *posv,
                        const int32_t *active, float *x, int d) {
    int s = blockIdx.x;
    if (active && !active[s]) return;
    int id = tokv[s], p = posv[s];
    for (int i = threadIdx.x; i < d; i += blockDim.x) {
        float e = dequant_elem<TYPE>(tok, id, i >> 5, i & 31);
        x[(size_t)s * d + i] = e + pos_emb[(size_t)p * d + i];
    }
}

int launch_embed(const wh_model &m, const int32_t *tok, const int32_t *pos, const int32_t *active, float *x,
                 int S, hipStream_t st) {
    MatView v = view_of(m.tok);
    int d = m.n_state;
    switch (m.tok.type) {
    case 0: hipLaunchKernelGGL(k_embed<0>, dim3(S), dim3(256), 0, st, v, m.pos, tok, pos, active, x, d); break;
    case 2: hipLaunchKernelGGL(k_embed<2>, dim3(S), dim3(256), 0, st, v, m.pos, tok, pos, active, x, d); break;
    case 3: hipLaunchKernelGGL(k_embed<3>, dim3(S), dim3(256), 0, st, v, m.pos, tok, pos, active, x, d); break;
    case 6: hipLaunchKernelGGL(k_embed<6>, dim3(S), dim3(256), 0, st, v, m.pos, tok, pos, active, x, d); break;
    case 7: hipLaunchKernelGGL(k_embed<7>, dim3(S), dim3(256), 0, st, v, m.pos, tok, pos, active, x, d); break;
    case 8: hipLaunchKernelGGL(k_embed<8>, dim3(S), dim3(256), 0, st, v, m.pos, tok, pos, active, x, d); break;
    default: return fail(WH_ERR_UNSUPPORTED, "embed: unsupported type");
    }
    WH_HIP(hipGetLastError());
    return WH_OK;
}

// ---------------------------------------------------------------------------
// LayerNorm over d (internal/ml/ops.go:153-202): y = w*(x-mean)/std + b with
// std = float32(sqrt(float64(var+eps))), eps = 1e-5. One block per row.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float block_sum256(float v, float *red) {
    v = group_sum<64>(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.0f;
    const int nw = blockDim.x >> 6;
    for (int i = 0; i < nw; i++) t += red[i];
    return t;
}

constexpr int LN_KEEP = 8;  // values of x a thread keeps in registers (rows up to 2048)

__global__ __launch_bounds__(256) void k_layernorm(const float *x, const float *w, const float *b, float *y,
                                                   int d) {
    __shared__ float red[8];
    const float *xr = x + (size_t)blockIdx.x * d;
    float *yr = y + (size_t)blockIdx.x * d;
    if (d <= 256 * LN_KEEP) {
        // the row read once: a thread keeps its values (elements t, t + 256, ...) for
        // the three passes, in the same order and arithmetic as below
        float xv[LN_KEEP];
#pragma unroll
        for (int j = 0; j < LN_KEEP; j++) {
            const int i = threadIdx.x + 256 * j;
            xv[j] = i < d ? xr[i] : 0.0f;
        }
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < LN_KEEP; j++)
            if (threadIdx.x + 256 * j < d) s += xv[j];
        const float mean = block_sum256(s, red) / (float)d;
        float v = 0.0f;
#pragma unroll
        for (int j = 0; j < LN_KEEP; j++)
            if (threadIdx.x + 256 * j < d) {
                const float t = xv[j] - mean;
                v += t * t;
            }
        const float var = block_sum256(v, red) / (float)d;
        const float sd = (float)sqrt((double)(var + 1e-5f));
#pragma unroll
        for (int j = 0; j < LN_KEEP; j++) {
            const int i = threadIdx.x + 256 * j;
            if (i < d) yr[i] = w[i] * (xv[j] - mean) / sd + b[i];
        }
        return;
    }
    float s = 0.0f;
    for (int i = threadIdx.x; i < d; i += blockDim.x) s += xr[i];
    float mean = block_sum256(s, red) / (float)d;
    float v = 0.0f;
    for (int i = threadIdx.x; i < d; i += blockDim.x) {
        float t = xr[i] - mean;
        v += t * t;
    }
    float var = block_sum256(v, red) / (float)d;
    float sd = (float)sqrt((double)(var + 1e-5f));
    __syncthreads();
    for (int i = threadIdx.x; i < d; i += blockDim.x) yr[i] = w[i] * (xr[i] - mean) / sd + b[i];
}

// Loads this file's code object (the runtime does it on first use otherwise).
int warm_kernels() {
    hipFuncAttributes attr;
    WH_HIP(hipFuncGetAttributes(&attr, (const void *)k_layernorm));
    return WH_OK;
}

int launch_layernorm(const float *x, const float *w, const float *b, float *y, int S, int d, hipStream_t st) {
    hipLaunchKernelGGL(k_layernorm, dim3(S), dim3(256), 0, st, x, w, b, y, d);
    WH_HIP(hipGetLastError());
    return WH_OK;
}

// ---------------------------------------------------------------------------
// Decoder self-attention with the persistent KV cache
// (internal/model/decoder.go:836-908 + internal/ml/attention.go:193-281).
// KV layout per stream and layer: [2][H][ctx][hd] (K plane, then V plane).
// mode 0 reproduces the reference mask: with Tq = 1 every key j > 0 is masked
// (attention.go:250-256), so only cache row 0 is attended. mode 1 attends to
// rows 0..pos (textbook causal decoding). One wavefront per (stream, head); mode 1
// runs k_self_attn_tiled below instead where the head size allows.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void k_self_attn(const float *q, const float *k, const float *v, float *kv_layer,
                                                  size_t kv_stream_stride, const int32_t *posv,
                                                  const int32_t *active, float *out, int H, int hd, int ctx,
                                                  int mode, float scale) {
    extern __shared__ float sc[];
    const int s = blockIdx.x / H, h = blockIdx.x % H, lane = threadIdx.x;
    if (active && !active[s]) return;
    const int d = H * hd;
    const int p = posv[s];
    float *Kc = kv_layer + (size_t)s * kv_stream_stride + (size_t)h * ctx * hd;
    float *Vc = Kc + (size_t)H * ctx * hd;
    const float *qh = q + (size_t)s * d + (size_t)h * hd;
    const float *kh = k + (size_t)s * d + (size_t)h * hd;
    const float *vh = v + (size_t)s * d + (size_t)h * hd;
    for (int j = lane; j < hd; j += 64) {
        Kc[(size_t)p * hd + j] = kh[j];
        Vc[(size_t)p * hd + j] = vh[j];
    }
    const int n = (mode == 0) ? 1 : p + 1;
    float mx = -INFINITY;
    for (int t = 0; t < n; t++) {
        const float *kr = (t == p) ? kh : Kc + (size_t)t * hd;
        float part = 0.0f;
        for (int j = lane; j < hd; j += 64) part += qh[j] * kr[j];
        float sco = group_sum<64>(part) * scale;
        if (lane == 0) sc[t] = sco;
        mx = fmaxf(mx, sco);
    }
    __syncthreads();
    float sum = 0.0f;
    for (int t = lane; t < n; t += 64) {
        float e = fast_exp(sc[t] - mx);
        sc[t] = e;
        sum += e;
    }
    sum = group_sum<64>(sum);
    __syncthreads();
    const bool uniform = (sum == 0.0f);
    const float inv = uniform ? 1.0f / (float)n : 1.0f / sum;
    for (int j = lane; j < hd; j += 64) {
        float o = 0.0f;
        for (int t = 0; t < n; t++) {
            const float *vr = (t == p) ? vh : Vc + (size_t)t * hd;
            float pt = uniform ? inv : sc[t] * inv;
            o += pt * vr[j];
        }
        out[(size_t)s * d + (size_t)h * hd + j] = o;
    }
}

// mode 1 when hd % 4 == 0 and hd <= 128: one 256-thread block per (stream,
// head). Keys pass through LDS in tiles of 64 rows with a row stride of hd + 1,
// so the four lanes of a key (quarters of hd) and the 16 keys of a wave read
// different banks; a key's quarter sums meet in two butterfly steps. Weights . V:
// a thread owns one column and every (256 / hd)-th key, and the column partials
// are summed through LDS. Row pos of the cache is written here and read from the
// fresh k, v instead.
constexpr int SA_TILE = 64;

__host__ __device__ constexpr size_t self_attn_tiled_lds(int hd, int ctx) {
    return sizeof(float) * ((size_t)hd + (size_t)SA_TILE * (hd + 1) + (size_t)ctx + 8 + 256);
}

__global__ __launch_bounds__(256) void k_self_attn_tiled(const float *q, const float *k, const float *v,
                                                         float *kv_layer, size_t kv_stream_stride,
                                                         const int32_t *posv, const int32_t *active, float *out,
                                                         int H, int hd, int ctx, float scale) {
    extern __shared__ float sm[];
    const int s = blockIdx.x / H, h = blockIdx.x % H, t = threadIdx.x;
    if (active && !active[s]) return;
    const int d = H * hd, p = posv[s], n = p + 1;
    float *Kc = kv_layer + (size_t)s * kv_stream_stride + (size_t)h * ctx * hd;
    float *Vc = Kc + (size_t)H * ctx * hd;
    const float *qh = q + (size_t)s * d + (size_t)h * hd;
    const float *kh = k + (size_t)s * d + (size_t)h * hd;
    const float *vh = v + (size_t)s * d + (size_t)h * hd;
    float *qs = sm, *tile = qs + hd, *sc = tile + SA_TILE * (hd + 1), *red = sc + ctx, *part = red + 8;
    for (int j = t; j < hd; j += 256) {
        Kc[(size_t)p * hd + j] = kh[j];
        Vc[(size_t)p * hd + j] = vh[j];
        qs[j] = qh[j];
    }
    const int r = t >> 2, qt = t & 3, qlen = hd >> 2;
    float mx = -INFINITY;
    for (int t0 = 0; t0 < n; t0 += SA_TILE) {
        const int nk = min(SA_TILE, n - t0);
        __syncthreads();  // the previous tile is consumed (and qs is written)
        for (int e = t; e < nk * qlen; e += 256) {
            const int rr = e / qlen, c4 = e - rr * qlen, key = t0 + rr;
            const float4 x = *reinterpret_cast<const float4 *>((key == p ? kh : Kc + (size_t)key * hd) + 4 * c4);
            float *dst = tile + rr * (hd + 1) + 4 * c4;
            dst[0] = x.x;
            dst[1] = x.y;
            dst[2] = x.z;
            dst[3] = x.w;
        }
        __syncthreads();
        float acc = 0.0f;
        if (r < nk) {
            const float *row = tile + r * (hd + 1) + qt * qlen;
            const float *qq = qs + qt * qlen;
            for (int c = 0; c < qlen; c++) acc += qq[c] * row[c];
        }
        acc = group_sum<4>(acc);
        if (r < nk && qt == 0) {
            const float sco = acc * scale;
            sc[t0 + r] = sco;
            mx = fmaxf(mx, sco);
        }
    }
    mx = group_max<64>(mx);
    __syncthreads();
    if ((t & 63) == 0) red[t >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float sum = 0.0f;
    for (int i = t; i < n; i += 256) {
        const float e = fast_exp(sc[i] - mx);
        sc[i] = e;
        sum += e;
    }
    sum = block_sum256(sum, red + 4);
    const bool uniform = (sum == 0.0f);
    const float inv = uniform ? 1.0f / (float)n : 1.0f / sum;
    const int G = 256 / hd, g = t / hd, c = t - g * hd;
    if (g < G) {
        float o = 0.0f;
        for (int i = g; i < n; i += G) {
            const float *vr = (i == p) ? vh : Vc + (size_t)i * hd;
            o += (uniform ? inv : sc[i] * inv) * vr[c];
        }
        part[g * hd + c] = o;
    }
    __syncthreads();
    if (t < hd) {
        float o = 0.0f;
        for (int i = 0; i < G; i++) o += part[i * hd + t];
        out[(size_t)s * d + (size_t)h * hd + t] = o;
    }
}

int launch_self_attn(const float *q, const float *k, const float *v, float *kv_layer, size_t kv_stream_stride,
                     const int32_t *pos, const int32_t *active, float *out, int S, int H, int hd, int ctx, int mode,
                     hipStream_t st) {
    float scale = (float)(1.0 / sqrt((double)hd));
    if (mode == 1 && hd % 4 == 0 && hd <= 128 && self_attn_tiled_lds(hd, ctx) <= 65536) {
        hipLaunchKernelGGL(k_self_attn_tiled, dim3(S * H), dim3(256), self_attn_tiled_lds(hd, ctx), st, q, k, v,
                           kv_layer, kv_stream_stride, pos, active, out, H, hd, ctx, scale);
        WH_HIP(hipGetLastError());
        return WH_OK;
    }
    size_t shmem = sizeof(float) * (size_t)(mode == 0 ? 1 : ctx);
    hipLaunchKernelGGL(k_self_attn, dim3(S * H), dim3(64), shmem, st, q, k, v, kv_layer, kv_stream_stride, pos,
                       active, out, H, hd, ctx, mode, scale);
    WH_HIP(hipGetLastError());
    return WH_OK;
}

// ---------------------------------------------------------------------------
// Cross-attention over the cached encoder K/V
// (internal/model/decoder.go:911-971, P3 addressing :949-951): the [enc_len, d]
// row-major projection is viewed as [H, enc_len, hd] without a transpose, so
// head h reads the contiguous slab [h*enc_len*hd, (h+1)*enc_len*hd).
// hd == 64: split over key chunks in two kernels (the last chunk of a head
// combines it); the softmax subtracts the exact global maximum before the fast
// exp, as the reference does (attention.go:93-131). Other head sizes: one block
// per (stream, head).
// ---------------------------------------------------------------------------
constexpr int CROSS_CHUNK = 128;
constexpr int CROSS_MAXC = 16;  // key chunks per head (encoder lengths up to 2048)

__global__ __launch_bounds__(256) void k_cross_scores64(const float *q, const float *const *kbase,
                                                        const int32_t *active, float *scores, float *cmax, int H,
                                                        int enc_len, int chunks, float scale) {
    __shared__ float red[4];
    const int c = blockIdx.x % chunks, sh = blockIdx.x / chunks, h = sh % H, s = sh / H;
    if (active && !active[s]) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, slot = lane & 15;
    const int d = H * 64;
    const float4 q4 = ((const float4 *)(q + (size_t)s * d + h * 64))[slot];
    const float *K = kbase[s] + (size_t)h * enc_len * 64;
    const int t0 = c * CROSS_CHUNK, t1 = min(t0 + CROSS_CHUNK, enc_len);
    // each 16-lane group takes keys tb, tb + 16, ...: all CROSS_CHUNK / 16 key rows
    // are loaded before the first dot product, so a wave keeps 8 KiB in flight
    constexpr int U = CROSS_CHUNK / 16;
    const int tb = t0 + wave * 4 + (lane >> 4);
    float4 k4[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int t = tb + 16 * u;
        k4[u] = t < t1 ? ((const float4 *)(K + (size_t)t * 64))[slot] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int t = tb + 16 * u;
        float part = q4.x * k4[u].x + q4.y * k4[u].y + q4.z * k4[u].z + q4.w * k4[u].w;
        float dot = group_sum<16>(part);
        if (t < t1) {
            float sco = dot * scale;
            if (slot == 0) scores[((size_t)s * H + h) * enc_len + t] = sco;
            mx = fmaxf(mx, sco);
        }
    }
    mx = group_max<64>(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    if (threadIdx.x == 0) cmax[((size_t)s * H + h) * chunks + c] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// Weights . V of one chunk; the chunk workgroup that arrives last for its
// (stream, head) then combines the head: the chunks' weight sums and partial
// products summed in chunk order, times the reciprocal of the sum. The partials
// travel as {launch number, value} pairs stored and read at agent scope (no
// fences: on this chip they write back or drop the whole L2); the last workgroup
// reads each pair until it carries this launch's number (a counted chunk's pairs
// are in flight, so the bounded wait ends at once; one that never arrives gives
// NaN). The counter goes back to zero.
__global__ __launch_bounds__(256) void k_cross_pv64(const float *const *vbase, const int32_t *active,
                                                    const float *scores, const float *cmax, uint64_t *pvt,
                                                    uint32_t *cnt, uint32_t seq, float *out, int H, int enc_len,
                                                    int chunks) {
    __shared__ float4 red4[4][16];
    __shared__ float reds[4];
    __shared__ int last;
    const int c = blockIdx.x % chunks, sh = blockIdx.x / chunks, h = sh % H, s = sh / H;
    if (active && !active[s]) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, slot = lane & 15;
    float M = -INFINITY;
    const float *cm = cmax + ((size_t)s * H + h) * chunks;
    for (int i = 0; i < chunks; i++) M = fmaxf(M, cm[i]);
    const float *V = vbase[s] + (size_t)h * enc_len * 64;
    const float *sc = scores + ((size_t)s * H + h) * enc_len;
    const int t0 = c * CROSS_CHUNK, t1 = min(t0 + CROSS_CHUNK, enc_len);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    float es = 0.0f;
    // all of a lane's V rows and scores are loaded first (8 KiB in flight per
    // wave), then summed in key order
    constexpr int U = CROSS_CHUNK / 16;
    const int tb = t0 + wave * 4 + (lane >> 4);
    float4 v4[U];
    float sv[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int t = tb + 16 * u;
        v4[u] = t < t1 ? ((const float4 *)(V + (size_t)t * 64))[slot] : make_float4(0.f, 0.f, 0.f, 0.f);
        sv[u] = t < t1 ? sc[t] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
        if (tb + 16 * u < t1) {
            float e = fast_exp(sv[u] - M);
            acc.x += e * v4[u].x; acc.y += e * v4[u].y; acc.z += e * v4[u].z; acc.w += e * v4[u].w;
            if (slot == 0) es += e;
        }
    }
    // reduce the 4 key groups of the wave (lanes differing in bits 4,5)
#pragma unroll
    for (int o = 16; o < 64; o <<= 1) {
        acc.x += __shfl_xor(acc.x, o, 64);
        acc.y += __shfl_xor(acc.y, o, 64);
        acc.z += __shfl_xor(acc.z, o, 64);
        acc.w += __shfl_xor(acc.w, o, 64);
    }
    es = group_sum<64>(es);
    if (lane < 16) red4[wave][lane] = acc;
    if (lane == 0) reds[wave] = es;
    __syncthreads();
    const uint64_t tag = (uint64_t)seq << 32;
    uint64_t *pt = pvt + (size_t)sh * chunks * 65;
    if (threadIdx.x < 16) {
        float4 r = red4[0][threadIdx.x];
        for (int w = 1; w < 4; w++) {
            float4 t = red4[w][threadIdx.x];
            r.x += t.x; r.y += t.y; r.z += t.z; r.w += t.w;
        }
        uint64_t *p = pt + (size_t)c * 65 + 4 * threadIdx.x;
        __hip_atomic_store(p, tag | __float_as_uint(r.x), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(p + 1, tag | __float_as_uint(r.y), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(p + 2, tag | __float_as_uint(r.z), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(p + 3, tag | __float_as_uint(r.w), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (threadIdx.x == 16)
        __hip_atomic_store(pt + (size_t)c * 65 + 64, tag | __float_as_uint((reds[0] + reds[1]) + (reds[2] + reds[3])),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (threadIdx.x == 0)
        last = __hip_atomic_fetch_add(cnt + sh, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(chunks - 1);
    __syncthreads();
    if (!last || threadIdx.x >= 64) return;
    // every chunk's pairs are loaded at once; a pair not yet carrying this
    // launch's number is read again
    const int j = threadIdx.x;
    uint64_t ps[CROSS_MAXC], pj[CROSS_MAXC];
#pragma unroll
    for (int i = 0; i < CROSS_MAXC; i++)
        if (i < chunks) {
            ps[i] = __hip_atomic_load(pt + (size_t)i * 65 + 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            pj[i] = __hip_atomic_load(pt + (size_t)i * 65 + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    auto settle = [&](uint64_t v, const uint64_t *p) {
        for (int spin = 0; (v & 0xffffffff00000000ull) != tag; spin++) {
            if (spin >= (1 << 20)) return __uint_as_float(0x7fc00000u);  // NaN
            __builtin_amdgcn_s_sleep(1);
            v = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return __uint_as_float((uint32_t)v);
    };
    float sum = 0.0f, o = 0.0f;
#pragma unroll
    for (int i = 0; i < CROSS_MAXC; i++)
        if (i < chunks) sum += settle(ps[i], pt + (size_t)i * 65 + 64);
    const float inv = 1.0f / sum;  // sum >= 1: the maximum key contributes fast_exp(0) = 1
#pragma unroll
    for (int i = 0; i < CROSS_MAXC; i++)
        if (i < chunks) o += settle(pj[i], pt + (size_t)i * 65 + j);
    out[(size_t)s * H * 64 + h * 64 + j] = o * inv;
    if (j == 0) __hip_atomic_store(cnt + sh, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ __launch_bounds__(256) void k_cross_generic(const float *q, const float *const *kbase,
                                                       const float *const *vbase, const int32_t *active, float *out,
                                                       int H, int hd, int enc_len, float scale) {
    extern __shared__ float sc[];
    __shared__ float red[8];
    const int s = blockIdx.x / H, h = blockIdx.x % H;
    if (active && !active[s]) return;
    const int d = H * hd;
    const float *qh = q + (size_t)s * d + (size_t)h * hd;
    const float *K = kbase[s] + (size_t)h * enc_len * hd;
    const float *V = vbase[s] + (size_t)h * enc_len * hd;
    float mx = -INFINITY;
    for (int t = threadIdx.x; t < enc_len; t += blockDim.x) {
        float dot = 0.0f;
        for (int j = 0; j < hd; j++) dot += qh[j] * K[(size_t)t * hd + j];
        float sco = dot * scale;
        sc[t] = sco;
        mx = fmaxf(mx, sco);
    }
    mx = group_max<64>(mx);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = red[0];
    for (int i = 1; i < (int)(blockDim.x >> 6); i++) mx = fmaxf(mx, red[i]);
    __syncthreads();
    float es = 0.0f;
    for (int t = threadIdx.x; t < enc_len; t += blockDim.x) {
        float e = fast_exp(sc[t] - mx);
        sc[t] = e;
        es += e;
    }
    float sum = block_sum256(es, red);
    __syncthreads();
    const float inv = 1.0f / sum;
    for (int j = threadIdx.x; j < hd; j += blockDim.x) {
        float o = 0.0f;
        for (int t = 0; t < enc_len; t++) o += sc[t] * V[(size_t)t * hd + j];
        out[(size_t)s * d + (size_t)h * hd + j] = o * inv;
    }
}

int launch_cross_attn(const float *q, const float *const *kbase, const float *const *vbase, const int32_t *active,
                      float *out, int S, int H, int hd, int enc_len, CrossBufs &b, hipStream_t st) {
    float scale = (float)(1.0 / sqrt((double)hd));
    if (hd == 64 && b.chunks <= CROSS_MAXC) {
        int chunks = b.chunks;
        if (++b.seq == 0) ++b.seq;  // 0 is the tag of the zeroed buffer
        hipLaunchKernelGGL(k_cross_scores64, dim3(S * H * chunks), dim3(256), 0, st, q, kbase, active, b.scores,
                           b.cmax, H, enc_len, chunks, scale);
        hipLaunchKernelGGL(k_cross_pv64, dim3(S * H * chunks), dim3(256), 0, st, vbase, active, b.scores, b.cmax,
                           b.pvt, b.cnt, b.seq, out, H, enc_len, chunks);
    } else {
        size_t shmem = sizeof(float) * (size_t)enc_len;
        if (shmem > 64 * 1024) return fail(WH_ERR_UNSUPPORTED, "cross-attention: encoder length too large for head size");
        hipLaunchKernelGGL(k_cross_generic, dim3(S * H), dim3(256), shmem, st, q, kbase, vbase, active, out, H, hd,
                           enc_len, scale);
    }
    WH_HIP(hipGetLastError());
    return WH_OK;
}

// ---------------------------------------------------------------------------
// Cross K/V projection: C[t, r] = sum_c E[t, c] * W[r, c] (+ bias[r]) for all
// encoder frames (internal/model/decoder.go:923-940 via
// internal/ml/matmul_q8.go:141-196), on the fp32 matrix cores. A 64 (frames) x
// 64 (rows) output tile per workgroup of 4 waves, each wave a 32x32 quarter
// accumulated by v_mfma_f32_32x32x2_f32; K-steps of one 32-weight block: the
// E tile and the weight tile (dequantised bit-exactly, 8 weights per thread)
// go through LDS.
// ---------------------------------------------------------------------------
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Weights 8g .. 8g+7 of block b of row r, dequantised exactly as dequant_elem.
// The raw bytes behind elements 8g .. 8g+7 of block b of row r, and their
// bit-exact conversion (split so a loop can load the next tile's raw bytes while it
// works on the current one).
struct Raw8 {
    float4 x, y;       // F32
    uint32_t w0, w1;   // code bytes (Q8_0: 8, the 4/5-bit formats: 4 in w0)
    uint32_t sc, hb;   // scale word(s), Q5 high bits of these 8 elements
};

template <int TYPE>
__device__ __forceinline__ void dq8_load(const MatView &m, int r, int b, int g, Raw8 &q) {
    const size_t blk = (size_t)r * m.nb + b;
    if constexpr (TYPE == 0) {
        const float4 *p = (const float4 *)((const float *)m.qs + blk * 32 + 8 * g);
        q.x = p[0];
        q.y = p[1];
    } else if constexpr (TYPE == 8) {
        q.sc = ((const uint16_t *)m.sc)[blk];
        const uint2 c = *(const uint2 *)(m.qs + blk * 32 + 8 * g);
        q.w0 = c.x;
        q.w1 = c.y;
    } else {
        q.w0 = *(const uint32_t *)(m.qs + blk * 16 + 4 * g);  // weights 8g .. 8g+7
        if constexpr (TYPE == 3 || TYPE == 7) q.sc = ((const uint32_t *)m.sc)[blk];
        else q.sc = ((const uint16_t *)m.sc)[blk];
        if constexpr (TYPE == 6 || TYPE == 7) q.hb = (m.qh[blk] >> (8 * g)) & 0xFFu;
    }
}

template <int TYPE>
__device__ __forceinline__ void dq8_convert(const Raw8 &q, float (&o)[8]) {
#pragma clang fp contract(off)
    if constexpr (TYPE == 0) {
        o[0] = q.x.x; o[1] = q.x.y; o[2] = q.x.z; o[3] = q.x.w; o[4] = q.y.x; o[5] = q.y.y; o[6] = q.y.z; o[7] = q.y.w;
    } else if constexpr (TYPE == 8) {
        const float d = h2f(q.sc);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t w = j < 4 ? q.w0 : q.w1;
            o[j] = d * (float)(int)(int8_t)(w >> (8 * (j & 3)));
        }
    } else {
        float d, mn = 0.0f;
        if constexpr (TYPE == 3 || TYPE == 7) {
            d = h2f(q.sc & 0xFFFFu);
            mn = h2f(q.sc >> 16);
        } else {
            d = h2f(q.sc);
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t byte = (q.w0 >> (8 * (j >> 1))) & 0xFFu;
            uint32_t nib = (j & 1) ? (byte >> 4) : (byte & 0xFu);
            if constexpr (TYPE == 6 || TYPE == 7) nib |= ((q.hb >> j) & 1u) << 4;
            if constexpr (TYPE == 2) o[j] = d * (float)((int32_t)nib - 8);
            else if constexpr (TYPE == 3) o[j] = mul_add_nofma(d, (float)nib, mn);
            else if constexpr (TYPE == 6) o[j] = d * (float)((int32_t)nib - 16);
            else o[j] = mul_add_nofma(d, (float)nib, mn);
        }
    }
}

template <int TYPE>
__device__ __forceinline__ void dequant8(const MatView &m, int r, int b, int g, float (&o)[8]) {
    Raw8 q;
    dq8_load<TYPE>(m, r, b, g, q);
    dq8_convert<TYPE>(q, o);
}

// Epilogue: v = acc + bias; gelu: C = gelu(v); res: C = res + v (res may alias C).
// BK blocks of 32 columns per K-step (one LDS stage and two barriers per step);
// a row's last step with fewer blocks left stages zeros in their place.
// Up to three products of the same frames in one launch (grid z), e.g. the cross
// K and V of a layer or the encoder's q, k and v; res and gelu apply to every one.
struct XGemmOps {
    MatView w[3];
    const float *bias[3];
    float *C[3];
    const float *res;
    int gelu;
};

template <int TYPE, int BK>
__global__ __launch_bounds__(256) void k_cross_gemm(XGemmOps ops, const float *E, int T) {
    constexpr int KW = 32 * BK, KP = KW + 1;  // columns per step; LDS row stride (conflict-free operand reads)
    __shared__ float Es[64][KP];  // [frame][k]
    __shared__ float Ws[64][KP];  // [row][k]
    // this workgroup's matrix: grid z picks one of ops.n products of the same frames
    const int z = blockIdx.z;
    const MatView w = z == 0 ? ops.w[0] : z == 1 ? ops.w[1] : ops.w[2];
    const float *bias = z == 0 ? ops.bias[0] : z == 1 ? ops.bias[1] : ops.bias[2];
    float *C = z == 0 ? ops.C[0] : z == 1 ? ops.C[1] : ops.C[2];
    const int gelu = ops.gelu;
    const float *res = ops.res;
    const int t0 = blockIdx.y * 64, r0 = blockIdx.x * 64;
    if (r0 >= w.rows) return;  // the whole workgroup: past this matrix's rows
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wt = (wave >> 1) * 32, wr = (wave & 1) * 32;  // this wave's quarter of the tile
    const int K = w.cols;
    const int lr = tid >> 2, lg = tid & 3;  // tile loads: row (frame) lr, elements 8 lg .. 8 lg + 7 of each block
    f32x16 acc = {};
    // the next K-step in registers: its loads are in flight while the current step's
    // matrix-core products run
    float4 ex[BK], ey[BK];
    Raw8 wq[BK];
    auto load_step = [&](int b0) {
        const int t = t0 + lr;
#pragma unroll
        for (int u = 0; u < BK; u++) {
            const int b = b0 + u;
            ex[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            ey[u] = ex[u];
            wq[u] = {};
            if (b < w.nb) {
                if (t < T) {
                    const float4 *p = (const float4 *)(E + (size_t)t * K + b * 32 + 8 * lg);
                    ex[u] = p[0];
                    ey[u] = p[1];
                }
                if (r0 + lr < w.rows) dq8_load<TYPE>(w, r0 + lr, b, lg, wq[u]);
            }
        }
    };
    load_step(0);
    for (int b0 = 0; b0 < w.nb; b0 += BK) {
#pragma unroll
        for (int u = 0; u < BK; u++) {
            float *e = &Es[lr][32 * u + 8 * lg];
            e[0] = ex[u].x; e[1] = ex[u].y; e[2] = ex[u].z; e[3] = ex[u].w;
            e[4] = ey[u].x; e[5] = ey[u].y; e[6] = ey[u].z; e[7] = ey[u].w;
            float o[8];
            if (r0 + lr < w.rows && b0 + u < w.nb) {
                dq8_convert<TYPE>(wq[u], o);
            } else {
#pragma unroll
                for (int j = 0; j < 8; j++) o[j] = 0.0f;
            }
#pragma unroll
            for (int j = 0; j < 8; j++) Ws[lr][32 * u + 8 * lg + j] = o[j];
        }
        __syncthreads();
        if (b0 + BK < w.nb) load_step(b0 + BK);
        // A (32 frames x 2 k): lane -> frame lane % 32, k lane / 32; B (2 k x 32 rows) likewise
#pragma unroll
        for (int kk = 0; kk < KW; kk += 2) {
            const float av = Es[wt + (lane & 31)][kk + (lane >> 5)];
            const float bv = Ws[wr + (lane & 31)][kk + (lane >> 5)];
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, acc, 0, 0, 0);
        }
        __syncthreads();
    }
    // D (32 x 32): lane l, register i -> frame 8 (i / 4) + 4 (l / 32) + i % 4, row l % 32
    const int r = r0 + wr + (lane & 31);
    const float bb = (bias && r < w.rows) ? bias[r] : 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int t = t0 + wt + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
        if (t < T && r < w.rows) {
            const size_t o = (size_t)t * w.rows + r;
            const float v = bias ? acc[i] + bb : acc[i];
            C[o] = gelu ? gelu_ref(v) : res ? res[o] + v : v;
        }
    }
}

// The same product on the vector units for a row length that is not a whole
// number of blocks (small test models): one 32-column block per K-step,
// element-wise dequantisation, columns past the row end read as zero.
template <int TYPE>
__global__ __launch_bounds__(256) void k_cross_gemm_simt(MatView w, const float *E, int T, const float *bias, float *C,
                                                         int gelu, const float *res) {
    __shared__ float Es[32][64 + 4];
    __shared__ float Ws[32][64 + 4];
    const int t0 = blockIdx.y * 64, r0 = blockIdx.x * 64;
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int K = w.cols;
    float acc[4][4] = {};
    for (int b = 0; b < w.nb; b++) {
        const int c0 = b * 32;
        // E tile: 64 frames x 32 columns
        for (int i = threadIdx.x; i < 64 * 32; i += 256) {
            int tt = i / 32, cc = i % 32;
            int t = t0 + tt, c = c0 + cc;
            Es[cc][tt] = (t < T && c < K) ? E[(size_t)t * K + c] : 0.0f;
        }
        for (int i = threadIdx.x; i < 64 * 32; i += 256) {
            int rr = i / 32, cc = i % 32;
            int r = r0 + rr;
            Ws[cc][rr] = (r < w.rows && c0 + cc < K) ? dequant_elem<TYPE>(w, r, b, cc) : 0.0f;
        }
        __syncthreads();
#pragma unroll 8
        for (int kk = 0; kk < 32; kk++) {
            float av[4], bv[4];
#pragma unroll
            for (int i = 0; i < 4; i++) av[i] = Es[kk][ty * 4 + i];
#pragma unroll
            for (int j = 0; j < 4; j++) bv[j] = Ws[kk][tx * 4 + j];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] += av[i] * bv[j];
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        int t = t0 + ty * 4 + i;
        if (t >= T) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            int r = r0 + tx * 4 + j;
            if (r < w.rows) {
                const size_t o = (size_t)t * w.rows + r;
                const float v = bias ? acc[i][j] + bias[r] : acc[i][j];
                C[o] = gelu ? gelu_ref(v) : res ? res[o] + v : v;
            }
        }
    }
}

int launch_cross_gemm_n(const DevMat *const *ws, int n, const float *enc, int enc_len, const float *const *bias,
                        float *const *out, hipStream_t st, int gelu, const float *res) {
    if (n < 1 || n > 3) return fail(WH_ERR_INVALID, "cross gemm: 1..3 matrices per launch");
    bool same = true;
    for (int i = 1; i < n; i++) same &= ws[i]->type == ws[0]->type && ws[i]->cols == ws[0]->cols;
    if (!same || ws[0]->cols % 32 != 0 || (((uintptr_t)enc) & 15) != 0) {
        // mixed matrices, a partial last block or unaligned frame rows: one
        // vector-unit GEMM per matrix
        for (int i = 0; i < n; i++) {
            const DevMat &w = *ws[i];
            MatView v = view_of(w);
            dim3 grid((w.rows + 63) / 64, (enc_len + 63) / 64);
            const float *b = bias[i];
            float *o = out[i];
            switch (w.type) {
            case 0: hipLaunchKernelGGL(k_cross_gemm_simt<0>, grid, dim3(256), 0, st, v, enc, enc_len, b, o, gelu, res); break;
            case 2: hipLaunchKernelGGL(k_cross_gemm_simt<2>, grid, dim3(256), 0, st, v, enc, enc_len, b, o, gelu, res); break;
            case 3: hipLaunchKernelGGL(k_cross_gemm_simt<3>, grid, dim3(256), 0, st, v, enc, enc_len, b, o, gelu, res); break;
            case 6: hipLaunchKernelGGL(k_cross_gemm_simt<6>, grid, dim3(256), 0, st, v, enc, enc_len, b, o, gelu, res); break;
            case 7: hipLaunchKernelGGL(k_cross_gemm_simt<7>, grid, dim3(256), 0, st, v, enc, enc_len, b, o, gelu, res); break;
            case 8: hipLaunchKernelGGL(k_cross_gemm_simt<8>, grid, dim3(256), 0, st, v, enc, enc_len, b, o, gelu, res); break;
            default: return fail(WH_ERR_UNSUPPORTED, "cross gemm: unsupported type");
            }
            WH_HIP(hipGetLastError());
        }
        return WH_OK;
    }
    XGemmOps ops{};
    int rows = 0;
    for (int i = 0; i < n; i++) {
        ops.w[i] = view_of(*ws[i]);
        ops.bias[i] = bias[i];
        ops.C[i] = out[i];
        rows = std::max(rows, ws[i]->rows);
    }
    ops.res = res;
    ops.gelu = gelu;
    dim3 grid((rows + 63) / 64, (enc_len + 63) / 64, n);
    switch (ws[0]->type) {
    case 0: hipLaunchKernelGGL((k_cross_gemm<0, 2>), grid, dim3(256), 0, st, ops, enc, enc_len); break;
    case 2: hipLaunchKernelGGL((k_cross_gemm<2, 2>), grid, dim3(256), 0, st, ops, enc, enc_len); break;
    case 3: hipLaunchKernelGGL((k_cross_gemm<3, 2>), grid, dim3(256), 0, st, ops, enc, enc_len); break;
    case 6: hipLaunchKernelGGL((k_cross_gemm<6, 2>), grid, dim3(256), 0, st, ops, enc, enc_len); break;
    case 7: hipLaunchKernelGGL((k_cross_gemm<7, 2>), grid, dim3(256), 0, st, ops, enc, enc_len); break;
    case 8: hipLaunchKernelGGL((k_cross_gemm<8, 2>), grid, dim3(256), 0, st, ops, enc, enc_len); break;
    default: return fail(WH_ERR_UNSUPPORTED, "cross gemm: unsupported type");
    }
    WH_HIP(hipGetLastError());
    return WH_OK;
}

int launch_cross_gemm(const DevMat &w, const float *enc, int enc_len, const float *bias, float *out, hipStream_t st,
                      int gelu, const float *res) {
    const DevMat *ws[1] = {&w};
    return launch_cross_gemm_n(ws, 1, enc, enc_len, &bias, &out, st, gelu, res);
}

// ---------------------------------------------------------------------------
// Repetition penalty + greedy argmax on device
// (internal/model/decoder.go:1140-1167 and :996-1034). The penalty subtracts
// 2.0*count over the last 128 history ids (prompt included) from a copy of
// the logits; selection is the first index of the maximum of logit*invTemp.
// Stage 1: per-part maxima; stage 2: ordered reduction + SuppressNST + append.
// ---------------------------------------------------------------------------
constexpr int PEN_WINDOW = 128;

__device__ __forceinline__ void better(float v, int i, float &bv, int &bi) {
    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
}

__global__ __launch_bounds__(256) void k_penalty_argmax(const float *logits, const int32_t *hist,
                                                        const int32_t *hist_len, int hist_cap, const int32_t *active,
                                                        int V, const float *inv_temps, int eot, float *cur, float *pval,
                                                        int32_t *pidx, float *pval2, int32_t *pidx2, int parts) {
    __shared__ int32_t win[PEN_WINDOW];
    __shared__ float rv[4], rv2[4];
    __shared__ int ri[4], ri2[4];
    const int s = blockIdx.y, part = blockIdx.x;
    if (active && !active[s]) return;
    const float inv_temp = inv_temps[s];
    const int len = hist_len[s];
    const int start = len > PEN_WINDOW ? len - PEN_WINDOW : 0;
    const int nwin = len - start;
    for (int i = threadIdx.x; i < nwin; i += blockDim.x) win[i] = hist[(size_t)s * hist_cap + start + i];
    __syncthreads();
    const int per = (V + parts - 1) / parts;
    const int i0 = part * per, i1 = min(V, i0 + per);
    float bv = -INFINITY, bv2 = -INFINITY;
    int bi = 0x7FFFFFFF, bi2 = 0x7FFFFFFF;
    const float *lg = logits + (size_t)s * V;
    float *cu = cur + (size_t)s * V;
    for (int i = i0 + threadIdx.x; i < i1; i += blockDim.x) {
        int cnt = 0;
        for (int w = 0; w < nwin; w++) cnt += (win[w] == i);
        float v = lg[i];
        if (cnt > 0) v -= 2.0f * (float)cnt;
        cu[i] = v;
        float sc = v * inv_temp;
        better(sc, i, bv, bi);
        if (i != eot) better(sc, i, bv2, bi2);
    }
    // wave reduce (value, index) pairs
    for (int o = 32; o > 0; o >>= 1) {
        float ov = __shfl_xor(bv, o, 64);
        int oi = __shfl_xor(bi, o, 64);
        better(ov, oi, bv, bi);
        float ov2 = __shfl_xor(bv2, o, 64);
        int oi2 = __shfl_xor(bi2, o, 64);
        better(ov2, oi2, bv2, bi2);
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) { rv[wave] = bv; ri[wave] = bi; rv2[wave] = bv2; ri2[wave] = bi2; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; w++) { better(rv[w], ri[w], rv[0], ri[0]); better(rv2[w], ri2[w], rv2[0], ri2[0]); }
        pval[(size_t)s * parts + part] = rv[0];
        pidx[(size_t)s * parts + part] = ri[0];
        pval2[(size_t)s * parts + part] = rv2[0];
        pidx2[(size_t)s * parts + part] = ri2[0];
    }
}

__global__ void k_argmax_final(const float *pval, const int32_t *pidx, const float *pval2, const int32_t *pidx2,
                               int parts, const float *cur, int V, int eot, const int32_t *suppress_nsts,
                               const float *nsts, const int32_t *active, int32_t *hist, int32_t *hist_len,
                               int hist_cap, int32_t *tok, int32_t *pos, int32_t *out_ids) {
    const int s = blockIdx.x;
    if (threadIdx.x != 0) return;
    if (active && !active[s]) { if (out_ids) out_ids[s] = -1; return; }
    float bv = -INFINITY, bv2 = -INFINITY;
    int bi = 0x7FFFFFFF, bi2 = 0x7FFFFFFF;
    for (int p = 0; p < parts; p++) {
        better(pval[(size_t)s * parts + p], pidx[(size_t)s * parts + p], bv, bi);
        better(pval2[(size_t)s * parts + p], pidx2[(size_t)s * parts + p], bv2, bi2);
    }
    if (bi == 0x7FFFFFFF) bi = 0;  // all values NaN: the reference keeps index 0
    int id = bi;
    // SuppressNST (decoder.go:1016-1034): an EOT below -NoSpeechThold is replaced by
    // the best other token
    if (suppress_nsts[s] && eot >= 0 && eot < V) {
        if (cur[(size_t)s * V + eot] < -nsts[s] && id == eot) id = (bi2 == 0x7FFFFFFF) ? eot : bi2;
    }
    int len = hist_len[s];
    if (len < hist_cap) hist[(size_t)s * hist_cap + len] = id;
    hist_len[s] = len + 1;
    tok[s] = id;
    pos[s] = len;
    if (out_ids) out_ids[s] = id;
}

int launch_penalty_argmax(const float *logits, const int32_t *hist, const int32_t *hist_len, int hist_cap,
                          const int32_t *active, int S, int V, int eot, const SampleBufs &b, hipStream_t st) {
    hipLaunchKernelGGL(k_penalty_argmax, dim3(b.parts, S), dim3(256), 0, st, logits, hist, hist_len, hist_cap,
                       active, V, b.inv_temp, eot, b.cur, b.part_val, b.part_idx, b.part_val2, b.part_idx2, b.parts);
    WH_HIP(hipGetLastError());
    return WH_OK;
}

int launch_argmax_final(const SampleBufs &b, const float *cur, int S, int V, int eot, const int32_t *active,
                        int32_t *hist, int32_t *hist_len, int hist_cap, int32_t *tok, int32_t *pos, int32_t *out_ids,
                        hipStream_t st) {
    hipLaunchKernelGGL(k_argmax_final, dim3(S), dim3(64), 0, st, b.part_val, b.part_idx, b.part_val2, b.part_idx2,
                       b.parts, cur, V, eot, b.supp, b.nst, active, hist, hist_len, hist_cap, tok, pos, out_ids);
    WH_HIP(hipGetLastError());
    return WH_OK;
}

// ---------------------------------------------------------------------------
// Top-k with log-normaliser for beam search (internal/model/decoder.go:1068-1136):
// s_i = v_i*invTemp; keep the k largest (value desc, index asc); logZ =
// log(sum float32(exp(float64(s_i - max)))) + max; logprob = s - logZ.
// One block per stream.
// ---------------------------------------------------------------------------
constexpr int TOPK_MAX = 8;
constexpr int BEAM_MAX = 16;

// Top-k of each row of cur * inv_temp by (value desc, index asc), with
// logZ = log(sum_i exp(x_i - max)) + max (each exp in float64, summed in float32).
// Three launches over P partitions of each row (grid P x S): k_topk_part keeps each
// partition's max and its top-k (every entry of the row's top-k is in its
// partition's top-k), k_topk_sum adds the partition's exp terms against the row's
// max, and k_topk_merge picks the row's top-k from the P * k candidates and forms
// logZ. Scratch per (row, partition): TOPK_PART floats (max, sum, k values, k
// indices).
constexpr int TOPK_PART = 2 + 2 * TOPK_MAX;

__device__ __forceinline__ bool topk_before(float v, int i, float w, int j) { return v > w || (v == w && i < j); }

// Block-wide: the best (value desc, index asc) over one candidate per thread, k
// rounds; the chosen are written to outv/outi[0..k) in order. Candidates already
// chosen are masked by index. All 256 threads call it.
__device__ void topk_block_select(float v, int i, int k, float *outv, int *outi, float *redv, int *redi) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int r = 0; r < k; r++) {
        float bv = v;
        int bi = i;
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const int oi = __shfl_xor(bi, o, 64);
            if (oi != 0x7FFFFFFF && (bi == 0x7FFFFFFF || topk_before(ov, oi, bv, bi))) { bv = ov; bi = oi; }
        }
        if (lane == 0) { redv[wave] = bv; redi[wave] = bi; }
        __syncthreads();
        float b0 = redv[0];
        int i0 = redi[0];
        for (int w = 1; w < 4; w++)
            if (redi[w] != 0x7FFFFFFF && (i0 == 0x7FFFFFFF || topk_before(redv[w], redi[w], b0, i0))) { b0 = redv[w]; i0 = redi[w]; }
        if (threadIdx.x == 0) { outv[r] = b0; outi[r] = i0; }
        if (i == i0) i = 0x7FFFFFFF;  // indices are distinct: only the chosen one drops out
        __syncthreads();
    }
}

__global__ __launch_bounds__(256) void k_topk_part(const float *cur, const int32_t *active, int V, int k,
                                                   float inv_temp, int P, float *part) {
    __shared__ float redv[4], selv[TOPK_MAX];
    __shared__ int redi[4], seli[TOPK_MAX];
    const int s = blockIdx.y, p = blockIdx.x;
    if (active && !active[s]) return;
    const float *x = cur + (size_t)s * V;
    const int chunk = (V + P - 1) / P, lo = p * chunk, hi = min(V, lo + chunk);
    // this thread's top TOPK_MAX (constant indices: registers), then the max
    float tv[TOPK_MAX];
    int ti[TOPK_MAX];
#pragma unroll
    for (int j = 0; j < TOPK_MAX; j++) { tv[j] = -INFINITY; ti[j] = 0x7FFFFFFF; }
    float mx = -INFINITY;
    for (int i = lo + threadIdx.x; i < hi; i += 256) {
        const float v = x[i] * inv_temp;
        mx = fmaxf(mx, v);
        if (ti[TOPK_MAX - 1] == 0x7FFFFFFF || topk_before(v, i, tv[TOPK_MAX - 1], ti[TOPK_MAX - 1])) {
            tv[TOPK_MAX - 1] = v;
            ti[TOPK_MAX - 1] = i;
#pragma unroll
            for (int j = TOPK_MAX - 1; j > 0; j--) {
                if (ti[j - 1] == 0x7FFFFFFF || topk_before(tv[j], ti[j], tv[j - 1], ti[j - 1])) {
                    const float fv = tv[j]; tv[j] = tv[j - 1]; tv[j - 1] = fv;
                    const int fi = ti[j]; ti[j] = ti[j - 1]; ti[j - 1] = fi;
                }
            }
        }
    }
    mx = group_max<64>(mx);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) redv[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(redv[0], redv[1]), fmaxf(redv[2], redv[3]));
    __syncthreads();
    // the partition's top k: k rounds, each thread offering the best of its own list
    // not yet taken (its list is in order, so that is its next entry)
    int head = 0;
    float *o = part + ((size_t)s * P + p) * TOPK_PART;
    for (int r = 0; r < k; r++) {
        float v = -INFINITY;
        int i = 0x7FFFFFFF;
#pragma unroll
        for (int j = 0; j < TOPK_MAX; j++)
            if (j == head) { v = tv[j]; i = ti[j]; }
        topk_block_select(v, i, 1, selv + r, seli + r, redv, redi);
        if (i != 0x7FFFFFFF && i == seli[r]) head++;
        __syncthreads();
    }
    if (threadIdx.x == 0) o[0] = mx;
    if (threadIdx.x < k) {
        o[2 + threadIdx.x] = selv[threadIdx.x];
        o[2 + TOPK_MAX + threadIdx.x] = __int_as_float(seli[threadIdx.x]);
    }
}

__global__ __launch_bounds__(256) void k_topk_sum(const float *cur, const int32_t *active, int V, float inv_temp,
                                                  int P, float *part) {
    __shared__ float red[8];
    const int s = blockIdx.y, p = blockIdx.x;
    if (active && !active[s]) return;
    const float *x = cur + (size_t)s * V;
    float mx = -INFINITY;
    for (int q = 0; q < P; q++) mx = fmaxf(mx, part[((size_t)s * P + q) * TOPK_PART]);
    const int chunk = (V + P - 1) / P, lo = p * chunk, hi = min(V, lo + chunk);
    float es = 0.0f;
    for (int i = lo + threadIdx.x; i < hi; i += 256) es += (float)exp((double)(x[i] * inv_temp - mx));
    const float sum = block_sum256(es, red);
    if (threadIdx.x == 0) part[((size_t)s * P + p) * TOPK_PART + 1] = sum;
}

__global__ __launch_bounds__(256) void k_topk_merge(const int32_t *active, int k, int P, const float *part,
                                                    int32_t *out_tok, float *out_lp, float *out_logz) {
    __shared__ float redv[4], selv[TOPK_MAX];
    __shared__ int redi[4], seli[TOPK_MAX];
    const int s = blockIdx.x;
    if (active && !active[s]) return;
    const float *ps = part + (size_t)s * P * TOPK_PART;
    // candidate t = (partition t / k, place t % k); P * k <= 256
    const int t = threadIdx.x;
    float v = -INFINITY;
    int i = 0x7FFFFFFF;
    if (t < P * k) {
        v = ps[(t / k) * TOPK_PART + 2 + t % k];
        i = __float_as_int(ps[(t / k) * TOPK_PART + 2 + TOPK_MAX + t % k]);
    }
    topk_block_select(v, i, k, selv, seli, redv, redi);
    if (threadIdx.x == 0) {
        float mx = -INFINITY, sum = 0.0f;
        for (int q = 0; q < P; q++) mx = fmaxf(mx, ps[q * TOPK_PART]);
        for (int q = 0; q < P; q++) sum += ps[q * TOPK_PART + 1];
        redv[0] = (float)log((double)sum) + mx;
    }
    __syncthreads();
    const float logz = redv[0];
    if (threadIdx.x < k) {
        out_tok[(size_t)s * k + threadIdx.x] = seli[threadIdx.x];
        out_lp[(size_t)s * k + threadIdx.x] = selv[threadIdx.x] - logz;
    }
    if (threadIdx.x == 0) out_logz[s] = logz;
}

// Rows of the top-k ([S][kk], kk = k + 1) with equal values at or inside the k-th
// place: the kept set and its order are those of the reference's streaming
// replace-min scan (decoder.go:1089-1121) followed by a stable sort by value
// (decoder.go:1123-1127), so one thread reruns that scan over the penalised row
// and rewrites the first k entries. Other rows keep the top-k's (value desc, index
// asc) result, which is the same when no values tie.
__global__ __launch_bounds__(64) void k_topk_ties(const float *cur, const int32_t *active, int V, int k, int kk,
                                                  float inv_temp, const float *logz, int32_t *tok, float *lp) {
    const int s = blockIdx.x;
    if (threadIdx.x != 0 || (active && !active[s])) return;
    float *l = lp + (size_t)s * kk;
    bool tie = false;
    for (int j = 0; j + 1 < kk; j++) tie |= (l[j] == l[j + 1]);
    if (!tie) return;
    const float *x = cur + (size_t)s * V;
    int bt[TOPK_MAX], order[TOPK_MAX];
    float bv[TOPK_MAX];
    int n = 0, minpos = -1;
    float minval = 0.0f;
    for (int i = 0; i < V; i++) {
        const float sc = x[i] * inv_temp;
        if (n < k) {
            bt[n] = i;
            bv[n] = sc;
            if (minpos < 0 || sc < minval) { minpos = n; minval = sc; }
            n++;
            continue;
        }
        if (sc <= minval) continue;
        bt[minpos] = i;
        bv[minpos] = sc;
        minpos = 0;
        minval = bv[0];
        for (int j = 1; j < n; j++)
            if (bv[j] < minval) { minval = bv[j]; minpos = j; }
    }
    const float lz = logz[s];
    for (int j = 0; j < n; j++) {
        bv[j] -= lz;
        order[j] = j;
    }
    for (int a = 1; a < n; a++) {  // stable insertion sort, value descending
        const int o = order[a];
        int b = a - 1;
        while (b >= 0 && bv[order[b]] < bv[o]) {
            order[b + 1] = order[b];
            b--;
        }
        order[b + 1] = o;
    }
    int32_t *t = tok + (size_t)s * kk;
    for (int j = 0; j < k; j++) {
        t[j] = j < n ? bt[order[j]] : -1;
        l[j] = j < n ? bv[order[j]] : 0.0f;
    }
}

// ---- Go's sort.Slice on the device (one lane) ---------------------------------------
// The beam prune sorts its candidates with Go's sort.Slice (decoder.go:1462-1475),
// which is pdqsort (Go 1.25 src/sort/zsortfunc.go) and not stable: the order it
// leaves equal normalised scores in decides which parent lands in which slot.
// This is that algorithm step by step over an index permutation ix of LDS keys,
// less(i, j) = key[ix[i]] > key[ix[j]]. Sorting disjoint ranges in another order
// gives the same result (a range only ever compares with its fixed left
// neighbour), so the recursion runs from an explicit stack.
struct GoSort {
    const float *key;
    int *ix;
    __device__ bool less(int i, int j) const { return key[ix[i]] > key[ix[j]]; }
    __device__ void swap(int i, int j) const { const int t = ix[i]; ix[i] = ix[j]; ix[j] = t; }
    __device__ void insertion(int a, int b) const {
        for (int i = a + 1; i < b; i++)
            for (int j = i; j > a && less(j, j - 1); j--) swap(j, j - 1);
    }
    __device__ void sift_down(int lo, int hi, int first) const {
        int root = lo;
        for (;;) {
            int child = 2 * root + 1;
            if (child >= hi) return;
            if (child + 1 < hi && less(first + child, first + child + 1)) child++;
            if (!less(first + root, first + child)) return;
            swap(first + root, first + child);
            root = child;
        }
    }
    __device__ void heapsort(int a, int b) const {
        const int hi = b - a;
        for (int i = (hi - 1) / 2; i >= 0; i--) sift_down(i, hi, a);
        for (int i = hi - 1; i >= 0; i--) { swap(a, a + i); sift_down(0, i, a); }
    }
    // median of three by three order-2 steps, counting swaps
    __device__ int median(int a, int b, int c, int &swaps) const {
        if (less(b, a)) { swaps++; const int t = a; a = b; b = t; }
        if (less(c, b)) { swaps++; const int t = b; b = c; c = t; }
        if (less(b, a)) { swaps++; const int t = a; a = b; b = t; }
        return b;
    }
    // hint: 0 unknown, 1 increasing, 2 decreasing
    __device__ int choose_pivot(int a, int b, int &hint) const {
        const int l = b - a;
        int swaps = 0, i = a + l / 4, j = a + l / 4 * 2, k = a + l / 4 * 3;
        if (l >= 8) {
            if (l >= 50) {
                i = median(i - 1, i, i + 1, swaps);
                j = median(j - 1, j, j + 1, swaps);
                k = median(k - 1, k, k + 1, swaps);
            }
            j = median(i, j, k, swaps);
        }
        hint = swaps == 0 ? 1 : (swaps == 12 ? 2 : 0);
        return j;
    }
    __device__ bool partial_insertion(int a, int b) const {
        int i = a + 1;
        for (int step = 0; step < 5; step++) {
            while (i < b && !less(i, i - 1)) i++;
            if (i == b) return true;
            if (b - a < 50) return false;
            swap(i, i - 1);
            if (i - a >= 2)
                for (int j = i - 1; j >= 1; j--) {
                    if (!less(j, j - 1)) break;
                    swap(j, j - 1);
                }
            if (b - i >= 2)
                for (int j = i + 1; j < b; j++) {
                    if (!less(j, j - 1)) break;
                    swap(j, j - 1);
                }
        }
        return false;
    }
    __device__ void break_patterns(int a, int b) const {
        const int length = b - a;
        if (length < 8) return;
        uint64_t r = (uint64_t)length;
        const unsigned modulus = 1u << (32 - __clz(length));
        const int idx = a + (length / 4) * 2 - 1;
        for (int i = 0; i < 3; i++) {
            r ^= r << 13;
            r ^= r >> 7;
            r ^= r << 17;
            int other = (int)((unsigned)r & (modulus - 1));
            if (other >= length) other -= length;
            swap(idx - 1 + i, a + other);
        }
    }
    __device__ int partition_equal(int a, int b, int pivot) const {
        swap(a, pivot);
        int i = a + 1, j = b - 1;
        for (;;) {
            while (i <= j && !less(a, i)) i++;
            while (i <= j && less(a, j)) j--;
            if (i > j) break;
            swap(i, j);
            i++;
            j--;
        }
        return i;
    }
    __device__ int partition(int a, int b, int pivot, bool &already) const {
        swap(a, pivot);
        int i = a + 1, j = b - 1;
        while (i <= j && less(i, a)) i++;
        while (i <= j && !less(j, a)) j--;
        if (i > j) {
            swap(j, a);
            already = true;
            return j;
        }
        swap(i, j);
        i++;
        j--;
        for (;;) {
            while (i <= j && less(i, a)) i++;
            while (i <= j && !less(j, a)) j--;
            if (i > j) break;
            swap(i, j);
            i++;
            j--;
        }
        swap(j, a);
        already = false;
        return j;
    }
    // Returns false if the frame stack would overflow (cannot happen below 2^16 items).
    __device__ bool sort(int n) const {
        constexpr int STACK = 48;
        int sa[STACK], sb[STACK], sl[STACK];
        int sp = 0;
        sa[sp] = 0; sb[sp] = n; sl[sp] = n > 0 ? 32 - __clz(n) : 0; sp++;
        while (sp > 0) {
            sp--;
            int a = sa[sp], b = sb[sp], limit = sl[sp];
            bool balanced = true, partitioned = true;
            for (;;) {
                const int length = b - a;
                if (length <= 12) { insertion(a, b); break; }
                if (limit == 0) { heapsort(a, b); break; }
                if (!balanced) { break_patterns(a, b); limit--; }
                int hint;
                int pivot = choose_pivot(a, b, hint);
                if (hint == 2) {
                    for (int i = a, j = b - 1; i < j; i++, j--) swap(i, j);
                    pivot = (b - 1) - (pivot - a);
                    hint = 1;
                }
                if (balanced && partitioned && hint == 1 && partial_insertion(a, b)) break;
                if (a > 0 && !less(a - 1, pivot)) { a = partition_equal(a, b, pivot); continue; }
                bool already;
                const int mid = partition(a, b, pivot, already);
                partitioned = already;
                const int left = mid - a, right = b - mid, thr = length / 8;
                if (sp == STACK) return false;
                if (left < right) {
                    balanced = left >= thr;
                    sa[sp] = a; sb[sp] = mid; sl[sp] = limit; sp++;
                    a = mid + 1;
                } else {
                    balanced = right >= thr;
                    sa[sp] = mid + 1; sb[sp] = b; sl[sp] = limit; sp++;
                    b = mid;
                }
            }
        }
        return true;
    }
};

// One beam step's prune and next hypotheses (decoder.go:575-718). The hypotheses
// are beam objects: object o has its own token history hist[o][0..len[o]) with
// Go's slice capacity gcap[o], and a score; order[0..*nbeams) is the beams slice.
// Each live object in that order proposes its k candidates (its top-k rows of
// ttok/tlp, normalised by (len+1)^0.6), a finished one (last token EOT) proposes
// itself. Candidates are sorted with Go's sort.Slice (above); the first bs are
// applied in slot order exactly as the reference's loop does: slot i reuses the
// object of beams[nbeams-1-i] (popped from the end of reusableBeams), reads its
// parent as earlier slots left it, and an object too small for the new length
// gets a fresh zeroed slice (make) first, which a self-parent then copies onto
// itself. Then tok, pos and active of every object are set for the next forward,
// and stop[0] = 1 when every hypothesis has finished or the first repeats its
// last token more than 20 times (decoder.go:690-718). stop[1] is the position
// of the first live hypothesis at or past n_ctx (the reference's forward fails
// there on the next step), else -1; such a hypothesis is not made active.
// powtab[n] = float(pow(n, 0.6)) as the host computes it. stop[3] is the step
// (the host's loop index `step`) that set stop[0] or stop[1]. A stopped state,
// or one with stop[1] set, is left as it is, so the host may queue several steps
// before it reads the flags.
__global__ __launch_bounds__(256) void k_beam_select(const int32_t *ttok, const float *tlp, int k, int kk,
                                                     int32_t *hist, int32_t *len, int32_t *gcap, int cap,
                                                     float *score, int32_t *order, int32_t *nbeams, int32_t *active,
                                                     int32_t *tok, int32_t *pos, int32_t *stop, const float *powtab,
                                                     int bs, int eot, int n_ctx, int step) {
    constexpr int NCAND = BEAM_MAX * (TOPK_MAX - 1);
    __shared__ float cnorm[NCAND], cscore[NCAND], clp[NCAND];
    __shared__ int cpar[NCAND], ctok[NCAND], cix[NCAND];
    __shared__ int reuse[BEAM_MAX], next[BEAM_MAX];
    // the beam objects' state, read once by as many threads: length, capacity,
    // last token (kept current as the slots below are applied in place), score,
    // and the candidates of the top-k
    __shared__ int blen[BEAM_MAX], bcap[BEAM_MAX], blast[BEAM_MAX], border[BEAM_MAX];
    __shared__ float bscore[BEAM_MAX];
    __shared__ float tlps[BEAM_MAX * TOPK_MAX];
    __shared__ int ttoks[BEAM_MAX * TOPK_MAX];
    __shared__ int nkeep, nbin, s_nb, s_par, s_cpy, s_zero, s_bad;
    const int t = threadIdx.x;
    if (stop[0] || stop[1] >= 0) return;
    if (t < bs) {
        blen[t] = len[t];
        bcap[t] = gcap[t];
        bscore[t] = score[t];
        border[t] = order[t];
    }
    for (int i = t; i < bs * kk; i += blockDim.x) {
        tlps[i] = tlp[i];
        ttoks[i] = ttok[i];
    }
    __syncthreads();
    if (t < bs) blast[t] = blen[t] > 0 ? hist[(size_t)t * cap + blen[t] - 1] : -1;
    __syncthreads();
    if (t == 0) {
        const int nb = *nbeams;
        int n = 0;
        for (int b = 0; b < nb; b++) {
            const int o = border[b];
            reuse[b] = o;
            const int L = blen[o];
            const float sc = bscore[o];
            if (blast[o] == eot) {
                cpar[n] = o; cscore[n] = sc; ctok[n] = eot; clp[n] = 0.0f; cnorm[n] = sc / powtab[L];
                n++;
            } else {
                for (int c = 0; c < k; c++) {
                    const float lpc = tlps[o * kk + c];
                    const float ns = sc + lpc;
                    cpar[n] = o; cscore[n] = ns; ctok[n] = ttoks[o * kk + c]; clp[n] = lpc;
                    cnorm[n] = ns / powtab[L + 1];
                    n++;
                }
            }
        }
        for (int i = 0; i < n; i++) cix[i] = i;
        const GoSort gs{cnorm, cix};
        s_bad = gs.sort(n) ? 0 : 1;
        nbin = nb;
        nkeep = min(min(n, bs), nb);
    }
    __syncthreads();
    const int keep = nkeep;
    for (int i = 0; i < keep; i++) {
        if (t == 0) {
            const int c = cix[i];
            const int o = reuse[nbin - 1 - i];  // reusableBeams[n-1], popped
            const int par = cpar[c];
            const int L = blen[par];
            const bool carry = blast[par] == eot && ctok[c] == eot && clp[c] == 0.0f;
            const int need = carry ? L : L + 1;
            // make([]int32, need) when the capacity is short; a self-parent then copies the zeros
            s_zero = (bcap[o] < need && o == par) ? need : 0;
            if (bcap[o] < need) bcap[o] = need;
            s_cpy = (o != par) ? (carry ? need : need - 1) : 0;
            s_nb = o;
            s_par = par;
            next[i] = o;
            blen[o] = need;
            bscore[o] = cscore[c];
            blast[o] = carry ? eot : ctok[c];
            // the appended token (written after the copy below)
            cix[i] = carry ? -1 : ctok[c];
        }
        __syncthreads();
        const int o = s_nb, par = s_par, nz = s_zero, nc = s_cpy;
        for (int j = t; j < nz; j += blockDim.x) hist[(size_t)o * cap + j] = 0;
        for (int j = t; j < nc; j += blockDim.x) hist[(size_t)o * cap + j] = hist[(size_t)par * cap + j];
        __syncthreads();
        if (t == 0 && cix[i] >= 0) hist[(size_t)o * cap + blen[o] - 1] = cix[i];
        __syncthreads();
    }
    if (t < bs) {
        len[t] = blen[t];
        gcap[t] = bcap[t];
        score[t] = bscore[t];
    }
    if (t == 0) {
        int bad_pos = -1;
        for (int i = 0; i < keep; i++) {
            const int o = next[i];
            order[i] = o;
            const int L = blen[o];
            const int lt = L > 0 ? blast[o] : -1;
            tok[o] = lt;
            pos[o] = L - 1;
            const bool live = lt != eot;
            if (live && L - 1 >= n_ctx && bad_pos < 0) bad_pos = L - 1;
            active[o] = live && L - 1 < n_ctx;
        }
        // objects left out of the beams slice (never with at least one candidate per hypothesis)
        for (int i = keep; i < nbin; i++) active[reuse[nbin - 1 - i]] = 0;
        *nbeams = keep;
        bool all = true;
        for (int i = 0; i < keep; i++) all &= (blast[next[i]] == eot);
        bool halt = all || keep == 0;
        if (!halt && keep > 0) {
            const int o = next[0], L0 = blen[o];
            const int32_t *h0 = hist + (size_t)o * cap;
            if (L0 >= 2) {
                int streak = 1;
                for (int i = L0 - 2; i >= 0 && h0[i] == blast[o]; i--)
                    if (++streak > 20) { halt = true; break; }
            }
        }
        stop[0] = halt ? 1 : (s_bad ? 1 : 0);
        stop[1] = bad_pos;
        stop[2] = s_bad;
        if (halt || s_bad || bad_pos >= 0) stop[3] = step;
    }
}

int launch_topk_ties(const float *cur, const int32_t *active, int S, int V, int k, int kk, float inv_temp,
                     const float *logz, int32_t *tok, float *lp, hipStream_t st) {
    if (k < 1 || kk > TOPK_MAX || k >= kk) return fail(WH_ERR_INVALID, "topk: bad k");
    hipLaunchKernelGGL(k_topk_ties, dim3(S), dim3(64), 0, st, cur, active, V, k, kk, inv_temp, logz, tok, lp);
    WH_HIP(hipGetLastError());
    return WH_OK;
}

int launch_beam_select(const int32_t *ttok, const float *tlp, int k, int kk, int32_t *hist, int32_t *len,
                       int32_t *gcap, int cap, float *score, int32_t *order, int32_t *nbeams, int32_t *active,
                       int32_t *tok, int32_t *pos, int32_t *stop, const float *powtab, int bs, int eot, int n_ctx,
                       int step, hipStream_t st) {
    if (bs < 1 || bs > BEAM_MAX || k < 1 || k >= kk || kk > TOPK_MAX)
        return fail(WH_ERR_INVALID, "beam: unsupported beam size");
    hipLaunchKernelGGL(k_beam_select, dim3(1), dim3(256), 0, st, ttok, tlp, k, kk, hist, len, gcap, cap, score, order,
                       nbeams, active, tok, pos, stop, powtab, bs, eot, n_ctx, step);
    WH_HIP(hipGetLastError());
    return WH_OK;
}

int launch_topk(const float *cur, const int32_t *active, int S, int V, int k, float inv_temp, int32_t *out_tok,
                float *out_lp, float *out_logz, float *part, hipStream_t st) {
    if (k < 1 || k > TOPK_MAX) return fail(WH_ERR_INVALID, "topk: k must be in [1,8]");
    if (S < 1 || S > TOPK_ROWS_MAX) return fail(WH_ERR_INVALID, "topk: 1..16 rows");
    // partitions of ~2048 entries, at most TOPK_PARTS (P * k <= 256 candidates to merge)
    const int P = std::max(1, std::min(TOPK_PARTS, (V + 2047) / 2048));
    hipLaunchKernelGGL(k_topk_part, dim3(P, S), dim3(256), 0, st, cur, active, V, k, inv_temp, P, part);
    hipLaunchKernelGGL(k_topk_sum, dim3(P, S), dim3(256), 0, st, cur, active, V, inv_temp, P, part);
    hipLaunchKernelGGL(k_topk_merge, dim3(S), dim3(256), 0, st, active, k, P, part, out_tok, out_lp, out_logz);
    WH_HIP(hipGetLastError());
    return WH_OK;
}

}  // namespace wh
