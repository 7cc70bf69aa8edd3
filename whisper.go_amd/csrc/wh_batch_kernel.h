// Persistent forward of S decoder states (beam hypotheses or independent
// streams, 2 <= S <= 8) in one cooperative launch per token step
// (internal/model/decoder.go:745-993 for every state, reference attention mask).
//
// The multi-kernel path runs a step as ~13 launches per layer; each launch costs
// a dispatch and a drain of the whole chip. Here one workgroup per CU walks the
// phases of the step and the phases meet at grid barriers:
//   embed                x = token row + positional row                 (once)
//   per layer l:
//     A   LN1(x); q,k,v rows (k, v -> KV cache at pos); self-attention out rows
//         on V cache row 0 (the reference mask attends row 0 only,
//         internal/ml/attention.go:250-256): x1 = x + (Wo.V0 + bo). When a
//         state is at position 0 its row 0 is written in this phase, so the
//         out rows then wait for a barrier of their own.
//     B   LN2(x1); cross query rows -> q
//     C   cross scores of (state, head, key chunk) items, chunk maxima
//     D   fast-exp weights against the head maximum, partial P.V per chunk
//     E   head combine -> attn
//     F   cross out rows: x2 = x1 + (Wo_c.attn + b)
//     G   LN3(x2); fc1 rows + GELU -> h
//     H   fc2 rows: x = x2 + (W2.h + b2)
//   final LN; tied logits rows -> logits
// Each phase splits the rows of its matrix evenly over the workgroups; a
// workgroup stages the phase's input activations of all S states in LDS once
// (LayerNorm computed on the way, one wave per state) and every decoded weight
// block feeds the S states. The arithmetic is that of the multi-kernel kernels
// (exact integer codes, fp32 FMA accumulation, LayerNorm in two passes with a
// float64 sqrt, GELU with a float64 tanh, the reference's fast exp); only the
// summation order differs.
//
// Barrier: every workgroup releases its stores at agent scope, publishes its
// phase number, and waits until all workgroups have published it, then
// acquires. Every wait is bounded: on expiry the error word is set, later waits
// return at once, and the host reports a failure.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "wh_batch.h"
#include "wh_internal.h"

namespace wh {
namespace batch {

constexpr int NWV = NT / 64;
constexpr int XBLK = XBUDGET / 128;  // staged 32-float blocks, over all states
constexpr unsigned SPIN_MAX = 1u << 22;
constexpr int CHUNK = 128;           // keys per cross-attention item

// ---- cross-lane sums ---------------------------------------------------------------
__device__ __forceinline__ float wsum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wmax(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// ---- grid barrier -------------------------------------------------------------------
__device__ __forceinline__ bool failed(unsigned *err) {
    return __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}

__device__ void gbar(unsigned *flags, unsigned *err, unsigned &g) {
    ++g;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __syncthreads();
    if (threadIdx.x < 64) {
        if (threadIdx.x == 0) __hip_atomic_store(flags + blockIdx.x, g, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int W = (int)gridDim.x;
        for (unsigned spins = 0;; spins++) {
            bool ok = true;
            for (int w = threadIdx.x; w < W; w += 64)
                ok &= (int)(__hip_atomic_load(flags + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - g) >= 0;
            if (__all(ok)) break;
            if (__any(failed(err) || spins > SPIN_MAX)) {
                if (threadIdx.x == 0) atomicOr(err, 1u);
                break;
            }
        }
    }
    __syncthreads();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
}

// ---- weight blocks ------------------------------------------------------------------
struct Blk {
    uint4 a, b;
    uint32_t s, h;
};

template <int TYPE>
__device__ __forceinline__ void blk_load(const MatView &m, size_t blk, Blk &r) {
    if constexpr (TYPE == 8) {
        const uint4 *p = (const uint4 *)(m.qs + blk * 32);
        r.a = p[0];
        r.b = p[1];
        r.s = ((const uint16_t *)m.sc)[blk];
        r.h = 0u;
    } else {
        r.a = *(const uint4 *)(m.qs + blk * 16);
        r.b = make_uint4(0u, 0u, 0u, 0u);
        if constexpr (TYPE == 3 || TYPE == 7) r.s = ((const uint32_t *)m.sc)[blk];
        else r.s = ((const uint16_t *)m.sc)[blk];
        if constexpr (TYPE == 6 || TYPE == 7) r.h = m.qh[blk];
        else r.h = 0u;
    }
}

// Codes of elements 4c..4c+3 of a block as floats: signed for Q8_0, unsigned for
// the 4/5-bit formats (their offset and the _1 formats' m enter through the
// block's sum of x in bscale).
template <int TYPE>
__device__ __forceinline__ void codes4(const Blk &r, int c, float (&q)[4]) {
    if constexpr (TYPE == 8) {
        const uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
        const int v = (int)w[c];
        q[0] = (float)((v << 24) >> 24);
        q[1] = (float)((v << 16) >> 24);
        q[2] = (float)((v << 8) >> 24);
        q[3] = (float)(v >> 24);
    } else {
        const uint32_t w[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
        const int t = c >> 1, sh = 16 * (c & 1);
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

// A block's contribution from qx = sum q_i x_i and sx = sum x_i.
template <int TYPE>
__device__ __forceinline__ float bscale(const Blk &r, float qx, float sx) {
    if constexpr (TYPE == 8) return h2f(r.s) * qx;
    else if constexpr (TYPE == 2) return h2f(r.s) * __builtin_fmaf(-8.0f, sx, qx);
    else if constexpr (TYPE == 6) return h2f(r.s) * __builtin_fmaf(-16.0f, sx, qx);
    else return __builtin_fmaf(h2f(r.s & 0xFFFFu), qx, h2f(r.s >> 16) * sx);
}

// ---- staged activations in LDS -------------------------------------------------------
// State s, block b (of nbc staged blocks), chunk k (elements 4k..4k+3) at float4
// slot (s * nbc + b) * 8 + ((k + b) & 7): the lanes of a wave read consecutive
// blocks at one k and hit distinct banks. Block sums (4/5-bit formats) at
// sx[s * nbc + b].
__device__ __forceinline__ int slot(int s, int nbc, int b, int k) { return (s * nbc + b) * 8 + ((k + b) & 7); }

// Block sums of the staged blocks, in the order the multi-kernel GEMV uses.
__device__ void stage_sums(int S, int nbc, const float4 *xs, float *sx) {
    for (int i = threadIdx.x; i < S * nbc; i += NT) {
        const int s = i / nbc, b = i % nbc;
        float t = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float4 v = xs[slot(s, nbc, b, k)];
            t += (v.x + v.y) + (v.z + v.w);
        }
        sx[i] = t;
    }
}

// Blocks [c0, c0 + nbc) of rows src(s, col) of the S states (zero past cols).
template <class Src>
__device__ void stage_cols(int S, int cols, int c0, int nbc, Src src, float4 *xs, float *sx, bool sums) {
    for (int i = threadIdx.x; i < S * nbc * 8; i += NT) {
        const int s = i / (nbc * 8), r = i % (nbc * 8), b = r >> 3, k = r & 7;
        const int col = (c0 + b) * 32 + 4 * k;
        float4 v;
        v.x = col < cols ? src(s, col) : 0.0f;
        v.y = col + 1 < cols ? src(s, col + 1) : 0.0f;
        v.z = col + 2 < cols ? src(s, col + 2) : 0.0f;
        v.w = col + 3 < cols ? src(s, col + 3) : 0.0f;
        xs[slot(s, nbc, b, k)] = v;
    }
    __syncthreads();
    if (sums) {
        stage_sums(S, nbc, xs, sx);
        __syncthreads();
    }
}

// LayerNorm (internal/ml/ops.go:153-202) of the d-element rows x[s] of the S
// states into the staged layout, one wave per state: the mean, then the mean of
// squared deviations, std = float32(sqrt(float64(var + eps))), w*(x-mean)/std + b.
// A lane keeps its elements (lane + 64 j) in their LDS slots between the passes.
__device__ void stage_ln(int S, int d, const float *x, const float *w, const float *bb, float4 *xs, float *sx,
                         bool sums) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int nbc = (d + 31) / 32;
    float *xf = (float *)xs;
    for (int s = wv; s < S; s += NWV) {
        const float *xr = x + (size_t)s * d;
        float t = 0.0f;
        for (int i = lane; i < nbc * 32; i += 64) {
            const float v = i < d ? xr[i] : 0.0f;  // the tail of the last block stays zero
            xf[slot(s, nbc, i >> 5, (i & 31) >> 2) * 4 + (i & 3)] = v;
            t += v;
        }
        const float mean = wsum(t) / (float)d;
        float q = 0.0f;
        for (int i = lane; i < d; i += 64) {
            const float u = xf[slot(s, nbc, i >> 5, (i & 31) >> 2) * 4 + (i & 3)] - mean;
            q += u * u;
        }
        const float var = wsum(q) / (float)d;
        const float sd = (float)sqrt((double)(var + 1e-5f));
        for (int i = lane; i < d; i += 64) {
            float &e = xf[slot(s, nbc, i >> 5, (i & 31) >> 2) * 4 + (i & 3)];
            e = w[i] * (e - mean) / sd + bb[i];
        }
    }
    __syncthreads();
    if (sums) {
        stage_sums(S, nbc, xs, sx);
        __syncthreads();
    }
}

// ---- GEMV over a row range, all states at once ----------------------------------------
// Rows [rg, rg + RW) of w (clamped to row1 - 1; the extra rows' results are
// dropped), staged blocks [0, nbc) = matrix blocks [c0, c0 + nbc): lane l takes
// blocks l, l + 64, ...; every decoded chunk of codes feeds the S states.
template <int TYPE, int RW>
__device__ __forceinline__ void dots(const MatView &w, int rg, int row1, int S, int c0, int nbc, const float4 *xs,
                                     const float *sx, float (&acc)[RW][SMAX]) {
    const int lane = threadIdx.x & 63;
    for (int b = lane; b < nbc; b += 64) {
        Blk rb[RW];
#pragma unroll
        for (int r = 0; r < RW; r++) blk_load<TYPE>(w, (size_t)min(rg + r, row1 - 1) * w.nb + c0 + b, rb[r]);
        float qx[RW][SMAX];
#pragma unroll
        for (int r = 0; r < RW; r++)
#pragma unroll
            for (int s = 0; s < SMAX; s++) qx[r][s] = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            // the chunk's codes, made from copies of the raw words that the compiler
            // cannot see through, so they are not hoisted out for all eight chunks
            float q[RW][4];
#pragma unroll
            for (int r = 0; r < RW; r++) {
                Blk cur = rb[r];
                asm volatile("" : "+v"(cur.a.x), "+v"(cur.a.y), "+v"(cur.a.z), "+v"(cur.a.w));
                if constexpr (TYPE == 8) asm volatile("" : "+v"(cur.b.x), "+v"(cur.b.y), "+v"(cur.b.z), "+v"(cur.b.w));
                if constexpr (TYPE == 6 || TYPE == 7) asm volatile("" : "+v"(cur.h));
                codes4<TYPE>(cur, k, q[r]);
            }
#pragma unroll
            for (int s = 0; s < SMAX; s++)
                if (s < S) {
                    const float4 xv = xs[slot(s, nbc, b, k)];
#pragma unroll
                    for (int r = 0; r < RW; r++) {
                        float &c = qx[r][s];
                        c = __builtin_fmaf(q[r][0], xv.x, c);
                        c = __builtin_fmaf(q[r][1], xv.y, c);
                        c = __builtin_fmaf(q[r][2], xv.z, c);
                        c = __builtin_fmaf(q[r][3], xv.w, c);
                    }
                }
            // keep the next chunk's LDS reads after these FMAs
            asm volatile("" ::: "memory");
        }
#pragma unroll
        for (int s = 0; s < SMAX; s++)
            if (s < S) {
                const float bsum = TYPE == 8 ? 0.0f : sx[s * nbc + b];
#pragma unroll
                for (int r = 0; r < RW; r++) acc[r][s] += bscale<TYPE>(rb[r], qx[r][s], bsum);
            }
    }
}

template <int RW, class Epi>
__device__ __forceinline__ void finish(int rg, int row1, int S, const int32_t *active, float (&acc)[RW][SMAX],
                                       Epi epi) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int r = 0; r < RW; r++)
#pragma unroll
        for (int s = 0; s < SMAX; s++)
            if (s < S) {
                const float v = wsum(acc[r][s]);
                if (lane == 0 && rg + r < row1 && active[s]) epi(s, rg + r, v);
            }
}

// Rows [row0, row1) of w against the staged input (already in LDS when `staged`,
// else staged here from src in passes of as many blocks as fit).
template <int TYPE, int RW, class Src, class Epi>
__device__ void gemv(const MatView &w, int row0, int row1, int S, const int32_t *active, bool staged, Src src,
                     float4 *xs, float *sx, Epi epi) {
    const int wv = threadIdx.x >> 6, nb = w.nb, per = XBLK / S;
    if (staged || nb <= per) {
        if (!staged) stage_cols(S, w.cols, 0, nb, src, xs, sx, TYPE != 8);
        for (int rg = row0 + wv * RW; rg < row1; rg += NWV * RW) {
            float acc[RW][SMAX];
#pragma unroll
            for (int r = 0; r < RW; r++)
#pragma unroll
                for (int s = 0; s < SMAX; s++) acc[r][s] = 0.0f;
            dots<TYPE, RW>(w, rg, row1, S, 0, nb, xs, sx, acc);
            finish<RW>(rg, row1, S, active, acc, epi);
        }
    } else {
        // passes over the columns; each wave keeps its RW rows' sums across the passes
        // (the host sizes the grid so a workgroup has at most NWV * RW rows here)
        const int rg = row0 + wv * RW;
        float acc[RW][SMAX];
#pragma unroll
        for (int r = 0; r < RW; r++)
#pragma unroll
            for (int s = 0; s < SMAX; s++) acc[r][s] = 0.0f;
        for (int c0 = 0; c0 < nb; c0 += per) {
            const int nbc = min(per, nb - c0);
            stage_cols(S, w.cols, c0, nbc, src, xs, sx, TYPE != 8);
            if (rg < row1) dots<TYPE, RW>(w, rg, row1, S, c0, nbc, xs, sx, acc);
            __syncthreads();
        }
        if (rg < row1) finish<RW>(rg, row1, S, active, acc, epi);
    }
    __syncthreads();
}

__device__ __forceinline__ int split(int n, int w, int W) { return (int)((long)n * w / W); }

// ---- the step ------------------------------------------------------------------------------
template <int TYPE>
__global__ __launch_bounds__(NT) void k_fwd_batch(BArgs a) {
    extern __shared__ float4 lds4[];
    float4 *xs = lds4;
    float *sx = (float *)(lds4 + XBLK * 8);
    float *red = sx + XBLK;  // reduction area (1024 floats)
    const int W = (int)gridDim.x, w = (int)blockIdx.x;
    const int S = a.S, d = a.d, H = a.H, L = a.L, C = a.chunks;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    // the phase counter continues from this workgroup's last published phase (every
    // workgroup passes the same barriers, so all start from the same value)
    unsigned *const flags = a.flags, *const errw = a.err;
    unsigned g = __hip_atomic_load(flags + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    bool pos0 = false;
    for (int s = 0; s < S; s++) pos0 |= a.active[s] && a.posv[s] == 0;

    // embedding (decoder.go:756-773): the quantised row is dequantised bit-exactly
    for (int i = split(S * d, w, W) + threadIdx.x; i < split(S * d, w + 1, W); i += NT) {
        const int s = i / d, e = i % d;
        if (!a.active[s]) continue;
        a.x[i] = dequant_elem<TYPE>(a.tok, a.tokv[s], e >> 5, e & 31) + a.pos_emb[(size_t)a.posv[s] * d + e];
    }
    gbar(flags, errw, g);

    // after a failed wait every barrier returns at once: the launch runs out and the
    // host reports the failure
    const int32_t *act = a.active, *posv = a.posv;
    float *xg = a.x, *x1g = a.x1, *x2g = a.x2, *qg = a.q, *attng = a.attn, *hg = a.h;
    const int ctx = a.ctx, enc_len = a.enc_len;
    const size_t kvs = a.kv_stream, plane = (size_t)H * ctx * 64;
    for (int l = 0; l < L; l++) {
        const BLayer *ly = a.layers + l;
        // ---- A: LN1, q,k,v rows; self-attention out rows on V row 0 ----
        stage_ln(S, d, xg, ly->ln1w, ly->ln1b, xs, sx, TYPE != 8);
        {
            float *kv = ly->kv;
            const float *svb = ly->svb;
            gemv<TYPE, 2>(ly->sqkv, split(3 * d, w, W), split(3 * d, w + 1, W), S, act, true,
                          [](int, int) { return 0.0f; }, xs, sx, [=](int s, int r, float v) {
                              // rows [0,d) q (unread under the reference mask), [d,2d) k, [2d,3d) v + b
                              if (r < d) return;
                              const int j = r % d;
                              float *dst = kv + (size_t)s * kvs + (r >= 2 * d ? plane : 0) +
                                           (size_t)(j >> 6) * ctx * 64 + (size_t)posv[s] * 64 + (j & 63);
                              *dst = r >= 2 * d ? v + svb[j] : v;
                          });
        }
        if (pos0) gbar(flags, errw, g);  // a state at position 0 attends the row it just wrote
        {
            const float *vp = ly->kv + plane;
            const float *sob = ly->sob;
            gemv<TYPE, 2>(ly->so, split(d, w, W), split(d, w + 1, W), S, act, false,
                          [=](int s, int c) { return vp[(size_t)s * kvs + (size_t)(c >> 6) * ctx * 64 + (c & 63)]; },
                          xs, sx, [=](int s, int r, float v) {
                              x1g[(size_t)s * d + r] = xg[(size_t)s * d + r] + (v + sob[r]);
                          });
        }
        gbar(flags, errw, g);
        // ---- B: LN2, cross query rows ----
        stage_ln(S, d, x1g, ly->ln2w, ly->ln2b, xs, sx, TYPE != 8);
        {
            const float *cqb = ly->cqb;
            gemv<TYPE, 2>(ly->cq, split(d, w, W), split(d, w + 1, W), S, act, true, [](int, int) { return 0.0f; },
                          xs, sx, [=](int s, int r, float v) { qg[(size_t)s * d + r] = v + cqb[r]; });
        }
        gbar(flags, errw, g);
        // ---- C: scores of (state, head, chunk) items and chunk maxima ----
        for (int it = w; it < S * H * C; it += W) {
            const int s = it / (H * C), h = (it / C) % H, c = it % C;
            if (!act[s]) continue;
            const int slot16 = lane & 15;
            const float4 q4 = ((const float4 *)(qg + (size_t)s * d + h * 64))[slot16];
            const float *K = ly->kbase[s] + (size_t)h * enc_len * 64;
            const int t0 = c * CHUNK, t1 = min(t0 + CHUNK, enc_len);
            float mx = -INFINITY;
            for (int t = t0 + wv * 4 + (lane >> 4); t - (lane >> 4) < t1; t += 4 * NWV) {
                float part = 0.0f;
                if (t < t1) {
                    const float4 k4 = ((const float4 *)(K + (size_t)t * 64))[slot16];
                    part = q4.x * k4.x + q4.y * k4.y + q4.z * k4.z + q4.w * k4.w;
                }
                float dot = part;
#pragma unroll
                for (int o = 8; o > 0; o >>= 1) dot += __shfl_xor(dot, o, 64);
                if (t < t1) {
                    const float sco = dot * a.scale;
                    if (slot16 == 0) a.scores[((size_t)s * H + h) * enc_len + t] = sco;
                    mx = fmaxf(mx, sco);
                }
            }
            mx = wmax(mx);
            if (lane == 0) red[wv] = mx;
            __syncthreads();
            if (threadIdx.x == 0) {
                float m = red[0];
                for (int i = 1; i < NWV; i++) m = fmaxf(m, red[i]);
                a.cmax[((size_t)s * H + h) * C + c] = m;
            }
            __syncthreads();
        }
        gbar(flags, errw, g);
        // ---- D: fast-exp weights against the head maximum, partial P.V ----
        for (int it = w; it < S * H * C; it += W) {
            const int s = it / (H * C), h = (it / C) % H, c = it % C;
            if (!act[s]) continue;
            const int slot16 = lane & 15;
            float M = -INFINITY;
            const float *cm = a.cmax + ((size_t)s * H + h) * C;
            for (int i = 0; i < C; i++) M = fmaxf(M, cm[i]);
            const float *V = ly->vbase[s] + (size_t)h * enc_len * 64;
            const float *sc = a.scores + ((size_t)s * H + h) * enc_len;
            const int t0 = c * CHUNK, t1 = min(t0 + CHUNK, enc_len);
            float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
            float es = 0.0f;
            for (int t = t0 + wv * 4 + (lane >> 4); t < t1; t += 4 * NWV) {
                const float e = fast_exp(sc[t] - M);
                const float4 v4 = ((const float4 *)(V + (size_t)t * 64))[slot16];
                acc.x += e * v4.x; acc.y += e * v4.y; acc.z += e * v4.z; acc.w += e * v4.w;
                if (slot16 == 0) es += e;
            }
#pragma unroll
            for (int o = 16; o < 64; o <<= 1) {
                acc.x += __shfl_xor(acc.x, o, 64);
                acc.y += __shfl_xor(acc.y, o, 64);
                acc.z += __shfl_xor(acc.z, o, 64);
                acc.w += __shfl_xor(acc.w, o, 64);
            }
            es = wsum(es);
            float4 *red4 = (float4 *)red;  // [NWV][16]
            if (lane < 16) red4[wv * 16 + lane] = acc;
            if (lane == 0) red[512 + wv] = es;
            __syncthreads();
            const size_t item = ((size_t)s * H + h) * C + c;
            if (threadIdx.x < 16) {
                float4 r = red4[threadIdx.x];
                for (int i = 1; i < NWV; i++) {
                    const float4 t4 = red4[i * 16 + threadIdx.x];
                    r.x += t4.x; r.y += t4.y; r.z += t4.z; r.w += t4.w;
                }
                ((float4 *)(a.pv + item * 64))[threadIdx.x] = r;
            }
            if (threadIdx.x == 0) {
                float t = 0.0f;
                for (int i = 0; i < NWV; i++) t += red[512 + i];
                a.psum[item] = t;
            }
            __syncthreads();
        }
        gbar(flags, errw, g);
        // ---- E: head combine, one wave per (state, head) ----
        for (int it = w * NWV + wv; it < S * H; it += W * NWV) {
            const int s = it / H, h = it % H;
            if (!act[s]) continue;
            const float *ps = a.psum + (size_t)it * C;
            float sum = 0.0f;
            for (int i = 0; i < C; i++) sum += ps[i];
            float o = 0.0f;
            for (int i = 0; i < C; i++) o += a.pv[((size_t)it * C + i) * 64 + lane];
            attng[(size_t)s * d + h * 64 + lane] = o * (1.0f / sum);
        }
        gbar(flags, errw, g);
        // ---- F: cross out rows ----
        {
            const float *cob = ly->cob;
            gemv<TYPE, 2>(ly->co, split(d, w, W), split(d, w + 1, W), S, act, false,
                          [=](int s, int c) { return attng[(size_t)s * d + c]; }, xs, sx, [=](int s, int r, float v) {
                              x2g[(size_t)s * d + r] = x1g[(size_t)s * d + r] + (v + cob[r]);
                          });
        }
        gbar(flags, errw, g);
        // ---- G: LN3, fc1 rows + GELU ----
        stage_ln(S, d, x2g, ly->ln3w, ly->ln3b, xs, sx, TYPE != 8);
        {
            const float *fc1b = ly->fc1b;
            gemv<TYPE, 2>(ly->fc1, split(4 * d, w, W), split(4 * d, w + 1, W), S, act, true,
                          [](int, int) { return 0.0f; }, xs, sx,
                          [=](int s, int r, float v) { hg[(size_t)s * 4 * d + r] = gelu_ref(v + fc1b[r]); });
        }
        gbar(flags, errw, g);
        // ---- H: fc2 rows ----
        {
            const float *fc2b = ly->fc2b;
            gemv<TYPE, 2>(ly->fc2, split(d, w, W), split(d, w + 1, W), S, act, false,
                          [=](int s, int c) { return hg[(size_t)s * 4 * d + c]; }, xs, sx, [=](int s, int r, float v) {
                              xg[(size_t)s * d + r] = x2g[(size_t)s * d + r] + (v + fc2b[r]);
                          });
        }
        gbar(flags, errw, g);
    }
    // ---- final LayerNorm and tied logits rows (decoder.go:817-832) ----
    stage_ln(S, d, xg, a.lnw, a.lnb, xs, sx, TYPE != 8);
    {
        float *lg = a.logits;
        const int V = a.V;
        gemv<TYPE, 2>(a.tok, split(V, w, W), split(V, w + 1, W), S, act, true, [](int, int) { return 0.0f; }, xs, sx,
                      [=](int s, int r, float v) { lg[(size_t)s * V + r] = v; });
    }
}

int launch(uint32_t type, int grid, const BArgs &a, hipStream_t st) {
    void *args[] = {(void *)&a};
    const void *fn = nullptr;
    switch (type) {
    case 2: fn = (const void *)k_fwd_batch<2>; break;
    case 3: fn = (const void *)k_fwd_batch<3>; break;
    case 6: fn = (const void *)k_fwd_batch<6>; break;
    case 7: fn = (const void *)k_fwd_batch<7>; break;
    case 8: fn = (const void *)k_fwd_batch<8>; break;
    default: return fail(WH_ERR_UNSUPPORTED, "batched persistent forward: unsupported weight type");
    }
    WH_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)LDS_BYTES));
    WH_HIP(hipLaunchCooperativeKernel(fn, dim3(grid), dim3(NT), args, LDS_BYTES, st));
    return WH_OK;
}


}  // namespace batch
}  // namespace wh
