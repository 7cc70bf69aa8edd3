// Persistent forward of S decoder states (beam hypotheses or independent
// streams, 2 <= S <= 16) in one cooperative launch per token step
// (internal/model/decoder.go:745-993 for every state, reference attention mask).
//
// The multi-kernel path runs a step as ~13 launches per layer; each launch costs
// a dispatch and a drain of the whole chip. Here one workgroup per CU walks the
// phases of the step and the phases meet at grid barriers.
//
// Under the reference mask a state past position 0 attends KV row 0 only
// (internal/ml/attention.go:250-256), so its self-attention output
// sa_l = Wo_l . V0_l + bo_l depends on no activation of the step: all layers'
// sa_l are computed in the first phase, together with the embedding. A layer is
// then five phases:
//   B   LN1(x) -> k,v rows into the KV cache at pos (two thirds of the
//       workgroups); LN2(x + sa_l) -> cross query rows (the other third)
//   X   cross attention: workgroup w takes key chunk c of head h of state s
//       (the host picks the chunk count so that every item has a workgroup, or
//       one chunk per head and several heads per workgroup when S * H exceeds
//       the grid);
//       scores into LDS, the head maximum from the chunk maxima of the head's
//       workgroups, fast-exp weights against it and the chunk's partial P.V;
//       the head's first chunk then forms attn = (sum of the chunks' P.V) /
//       (sum of their weight sums)
//   F   cross out rows: x2 = (x + sa_l) + (Wo_c.attn + b)
//   G   LN3(x2); fc1 rows + GELU -> h
//   H   fc2 rows: x = x2 + (W2.h + b2)
// and the step ends with the final LN and the tied logits rows. When a state is
// at position 0 its V0_l is written within the step, so each layer runs the k,v
// rows, the sa_l rows and the query rows as three phases instead.
//
// Each GEMV phase splits the rows of its matrix evenly over the workgroups; a
// workgroup stages the phase's input activations of all S states in LDS once
// (LayerNorm computed on the way) and every decoded weight block feeds the S
// states. The arithmetic is that of the multi-kernel kernels (exact integer
// codes, fp32 FMA accumulation, LayerNorm in two passes with a float64 sqrt, GELU
// with a float64 tanh, the reference's fast exp); only the summation order
// differs.
//
// Exchange between workgroups: every value another workgroup reads within the
// launch travels as a {tag, value} pair, stored and loaded with one relaxed
// agent-scope 64-bit atomic (past the per-XCD caches). The tag is the phase
// that wrote it (a counter every workgroup advances alike, continued across
// launches); a reader polls the pairs themselves until they carry the phase it
// needs, so a phase waits only for the values it reads, with no grid barrier,
// store-completion wait or separate flag. A buffer is rewritten only after every
// reader of its previous value has published a later value that the writer
// waited for. Only the KV rows at position 0, read by the next phase as plain
// floats, are followed by a grid barrier. Every wait is bounded: on expiry the
// error word is set, the values are taken as they are, and the host reports a
// failure.
#pragma once
// Included by the per-format sources wh_batch_q*.hip, each of which
// instantiates the kernel for one weight type (the instantiations compile in
// parallel).
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
constexpr int PU = 4, PU2 = 2;  // pair slots per thread loaded before a wait (one vector, two vectors)

// ---- cross-lane sums ---------------------------------------------------------------
// DPP lane exchange within rows of 16 lanes
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// Wave sum and maximum, left in every lane: quad exchanges, half-row and row
// mirrors (DPP), then lane swaps across the four rows.
__device__ __forceinline__ float wsum(float v) {
    v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp<0x141>(v);  // row_half_mirror
    v += dpp<0x140>(v);  // row_mirror
    v += __shfl_xor(v, 16, 64);
    return v + __shfl_xor(v, 32, 64);
}
__device__ __forceinline__ float wmax(float v) {
    v = fmaxf(v, dpp<0xB1>(v));
    v = fmaxf(v, dpp<0x4E>(v));
    v = fmaxf(v, dpp<0x141>(v));
    v = fmaxf(v, dpp<0x140>(v));
    v = fmaxf(v, __shfl_xor(v, 16, 64));
    return fmaxf(v, __shfl_xor(v, 32, 64));
}
// sum over aligned groups of G lanes (G = 32 or 64), left in every lane of the
// group: quad exchanges, half-row and row mirrors (DPP), then lane swaps across
// rows
template <int G>
__device__ __forceinline__ float gsum(float v) {
    v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp<0x141>(v);  // row_half_mirror
    v += dpp<0x140>(v);  // row_mirror
    v += __shfl_xor(v, 16, 64);
    if constexpr (G == 64) v += __shfl_xor(v, 32, 64);
    return v;
}
// the wave's index, known to be uniform
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// ---- global memory ---------------------------------------------------------------------
// Pointers read from descriptors are generic; typed as global memory, their loads
// are global_load (vector memory counter only) instead of flat_load, which would
// also hold up every LDS wait.
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const float gcf;
typedef __attribute__((address_space(1))) const f32x4 gcf4;
typedef __attribute__((address_space(1))) const u32x4 gcu4;
typedef __attribute__((address_space(1))) const uint16_t gcu16;
typedef __attribute__((address_space(1))) const uint32_t gcu32;
typedef __attribute__((address_space(1))) const uint64_t gcu64;
typedef __attribute__((address_space(1))) uint32_t gu32;
typedef __attribute__((address_space(1))) uint64_t gu64;
typedef __attribute__((address_space(1))) float gf;

__device__ __forceinline__ float ldg(const float *p) { return *(gcf *)p; }
__device__ __forceinline__ float4 ldg4(const float *p) {
    const f32x4 v = *(gcf4 *)p;
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void stg(float *p, float v) { *(gf *)p = v; }

// ---- exchanged values ----------------------------------------------------------------
__device__ __forceinline__ float ldx(const float *p) {
    return __uint_as_float(__hip_atomic_load((gcu32 *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}
// four consecutive floats at a 16-byte aligned address
__device__ __forceinline__ float4 ldx4(const float *p) {
    const uint64_t a = __hip_atomic_load((gcu64 *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t b = __hip_atomic_load((gcu64 *)p + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return make_float4(__uint_as_float((uint32_t)a), __uint_as_float((uint32_t)(a >> 32)),
                       __uint_as_float((uint32_t)b), __uint_as_float((uint32_t)(b >> 32)));
}
__device__ __forceinline__ void stx(float *p, float v) {
    __hip_atomic_store((gu32 *)p, __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// this wave's stores (and loads) have completed
__device__ __forceinline__ void stores_done() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// ---- {tag, value} pairs ------------------------------------------------------------
__device__ __forceinline__ uint64_t ldp(const uint64_t *p) {
    return __hip_atomic_load((gcu64 *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stp(uint64_t *p, float v, unsigned t) {
    __hip_atomic_store((gu64 *)p, ((uint64_t)t << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool ready(uint64_t v, unsigned t) { return (unsigned)(v >> 32) >= t; }
__device__ __forceinline__ float val(uint64_t v) { return __uint_as_float((uint32_t)v); }

// ---- grid barrier -------------------------------------------------------------------
__device__ __forceinline__ bool failed(unsigned *err) {
    return __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}

// The value of pair p, v as already loaded, once its tag reaches t.
__device__ __forceinline__ float waitp(const uint64_t *p, uint64_t v, unsigned t, unsigned *err) {
    for (unsigned spins = 0; !ready(v, t); spins++) {
        if (spins > SPIN_MAX || failed(err)) {
            atomicOr(err, 1u);
            break;
        }
        v = ldp(p);
    }
    return val(v);
}

__device__ __forceinline__ void gbar(unsigned *flags, unsigned *err, unsigned &g) {
    ++g;
    stores_done();
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
}

// ---- weight blocks ------------------------------------------------------------------
struct Blk {
    uint4 a, b;
    uint32_t s, h;
};

template <int TYPE>
__device__ __forceinline__ void blk_load(const MatView &m, size_t blk, Blk &r) {
    if constexpr (TYPE == 8) {
        gcu4 *p = (gcu4 *)(m.qs + blk * 32);
        const u32x4 a = p[0], b = p[1];
        r.a = make_uint4(a.x, a.y, a.z, a.w);
        r.b = make_uint4(b.x, b.y, b.z, b.w);
        r.s = ((gcu16 *)m.sc)[blk];
        r.h = 0u;
    } else {
        const u32x4 a = *(gcu4 *)(m.qs + blk * 16);
        r.a = make_uint4(a.x, a.y, a.z, a.w);
        r.b = make_uint4(0u, 0u, 0u, 0u);
        if constexpr (TYPE == 3 || TYPE == 7) r.s = ((gcu32 *)m.sc)[blk];
        else r.s = ((gcu16 *)m.sc)[blk];
        if constexpr (TYPE == 6 || TYPE == 7) r.h = ((gcu32 *)m.qh)[blk];
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

// ---- LDS --------------------------------------------------------------------------------
struct Lds {
    float4 *xs;   // staged blocks
    float *sx;    // their sums
    float *lw, *lb;  // LayerNorm weight and bias
    int *pos;     // [SMAX] positions
    float *stat;  // [2][SMAX] LayerNorm mean and std
    float *red;   // reduction area (1024 floats)
};

// State s, block b (of nbc staged blocks), chunk k (elements 4k..4k+3) at float4
// slot (s * nbc + b) * 8 + ((k + b) & 7): the lanes of a wave read consecutive
// blocks at one k and hit distinct banks. Block sums (4/5-bit formats) at
// sx[s * nbc + b].
__device__ __forceinline__ int slot(int s, int nbc, int b, int k) { return (s * nbc + b) * 8 + ((k + b) & 7); }

// Block sums of the staged blocks, in the order the multi-kernel GEMV uses.
__device__ __forceinline__ void stage_sums(int S, int nbc, const float4 *xs, float *sx) {
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

// Columns [32 c0, 32 (c0 + nbc)) of the S states' rows into the staged layout:
// src(s, col) gives elements col..col+3 (col a multiple of 4; zero past cols).
// Eight loads per thread are in flight before the first LDS store.
template <class Src>
__device__ __forceinline__ void burst(int S, int cols, int c0, int nbc, Src src, float4 *xs) {
    const int n = S * nbc * 8;
    for (int i0 = threadIdx.x; i0 < n; i0 += NT * 8) {
        float4 v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = i0 + u * NT;
            v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (i < n) {
                const int s = i / (nbc * 8), r = i % (nbc * 8);
                const int col = (c0 + (r >> 3)) * 32 + 4 * (r & 7);
                if (col < cols) v[u] = src(s, col);
            }
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = i0 + u * NT;
            if (i < n) {
                const int s = i / (nbc * 8), r = i % (nbc * 8);
                xs[slot(s, nbc, r >> 3, r & 7)] = v[u];
            }
        }
    }
}

// The same from the pair vector a (plus b, element by element, when TWO), rows
// ld pairs apart, once the pairs' tags reach ta (tb); rows of inactive states
// stage as zeros and are not waited for. Each thread loads U slots (4 pairs each)
// before it waits for any, then re-reads only the pending pairs.
template <int U, bool TWO>
__device__ __forceinline__ void burst_pairs(int S, unsigned amask, int cols, int c0, int nbc, const uint64_t *a,
                                            unsigned ta, const uint64_t *b, unsigned tb, size_t ld, float4 *xs,
                                            unsigned *err) {
    const int n = S * nbc * 8;
    for (int i0 = threadIdx.x; i0 < n; i0 += NT * U) {
        uint64_t va[U][4], vb[U][TWO ? 4 : 1];
        size_t off[U];
        bool on[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = i0 + u * NT, s = i / (nbc * 8), r = i - s * (nbc * 8);
            const int col = (c0 + (r >> 3)) * 32 + 4 * (r & 7);
            on[u] = i < n && col < cols && ((amask >> s) & 1u);
            off[u] = on[u] ? (size_t)s * ld + col : 0;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                va[u][k] = on[u] ? ldp(a + off[u] + k) : 0;
                if constexpr (TWO) vb[u][k] = on[u] ? ldp(b + off[u] + k) : 0;
            }
        }
        for (unsigned spins = 0;; spins++) {
            bool ok = true;
#pragma unroll
            for (int u = 0; u < U; u++)
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    ok = ok && (!on[u] || ready(va[u][k], ta));
                    if constexpr (TWO) ok = ok && (!on[u] || ready(vb[u][k], tb));
                }
            if (ok) break;
            if (spins > SPIN_MAX || failed(err)) {
                atomicOr(err, 1u);
                break;
            }
#pragma unroll
            for (int u = 0; u < U; u++)
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    if (on[u] && !ready(va[u][k], ta)) va[u][k] = ldp(a + off[u] + k);
                    if constexpr (TWO)
                        if (on[u] && !ready(vb[u][k], tb)) vb[u][k] = ldp(b + off[u] + k);
                }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = i0 + u * NT;
            if (i < n) {
                const int s = i / (nbc * 8), r = i - s * (nbc * 8);
                float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                if (on[u]) {
                    if constexpr (TWO)
                        v = make_float4(val(va[u][0]) + val(vb[u][0]), val(va[u][1]) + val(vb[u][1]),
                                        val(va[u][2]) + val(vb[u][2]), val(va[u][3]) + val(vb[u][3]));
                    else
                        v = make_float4(val(va[u][0]), val(va[u][1]), val(va[u][2]), val(va[u][3]));
                }
                xs[slot(s, nbc, r >> 3, r & 7)] = v;
            }
        }
    }
}

// fill() stages the columns, then their block sums when asked.
template <class Fill>
__device__ __forceinline__ void stage_cols(int S, int nbc, Fill fill, float4 *xs, float *sx, bool sums) {
    fill();
    __syncthreads();
    if (sums) {
        stage_sums(S, nbc, xs, sx);
        __syncthreads();
    }
}

// LayerNorm (internal/ml/ops.go:153-202) of the d-element rows of the S states,
// which fill() stages, in the staged layout: the mean, then the mean of squared
// deviations, std = float32(sqrt(float64(var + eps))), w*(x-mean)/std + b. The
// weights are loaded before the rows; the statistics take one wave per state,
// the normalisation every thread.
template <class Fill>
__device__ __forceinline__ void stage_ln(int S, int d, Fill fill, const float *w, const float *bb, const Lds &L, bool sums) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int nbc = d / 32, dq = d / 4;
    const int iw = min((int)threadIdx.x, dq - 1);  // d <= 4 NT
    const float4 wr = ldg4(w + 4 * iw), br = ldg4(bb + 4 * iw);
    fill();
    if ((int)threadIdx.x < dq) {
        ((float4 *)L.lw)[threadIdx.x] = wr;
        ((float4 *)L.lb)[threadIdx.x] = br;
    }
    __syncthreads();
    float *xf = (float *)L.xs;
    float *mean_l = L.stat, *sd_l = L.stat + SMAX;
    for (int s = wv; s < S; s += NWV) {
        float t = 0.0f;
#pragma unroll 8
        for (int i = lane; i < d; i += 64) t += xf[slot(s, nbc, i >> 5, (i & 31) >> 2) * 4 + (i & 3)];
        const float mean = wsum(t) / (float)d;
        float q = 0.0f;
#pragma unroll 8
        for (int i = lane; i < d; i += 64) {
            const float u = xf[slot(s, nbc, i >> 5, (i & 31) >> 2) * 4 + (i & 3)] - mean;
            q += u * u;
        }
        const float var = wsum(q) / (float)d;
        if (lane == 0) {
            mean_l[s] = mean;
            sd_l[s] = (float)sqrt((double)(var + 1e-5f));
        }
    }
    __syncthreads();
    // four consecutive elements per thread and step
    for (int i = threadIdx.x; i < S * dq; i += NT) {
        const int s = i / dq, e = (i - s * dq) * 4;
        float4 &v = L.xs[slot(s, nbc, e >> 5, (e & 31) >> 2)];
        const float4 g4 = ((const float4 *)L.lw)[e >> 2], b4 = ((const float4 *)L.lb)[e >> 2];
        const float m = mean_l[s], sd = sd_l[s];
        v.x = g4.x * (v.x - m) / sd + b4.x;
        v.y = g4.y * (v.y - m) / sd + b4.y;
        v.z = g4.z * (v.z - m) / sd + b4.z;
        v.w = g4.w * (v.w - m) / sd + b4.w;
    }
    __syncthreads();
    if (sums) {
        stage_sums(S, nbc, L.xs, L.sx);
        __syncthreads();
    }
}

// ---- GEMV over a row range, all states at once ----------------------------------------
// A pass covers NWV * RW * (64 / G) rows from P, interleaved over the waves so
// that every wave has work when a workgroup has few rows: lanes form groups of G
// and lane l of wave v works on row P + (r * (64 / G) + l / G) * NWV + v for the
// wave's first nr slots r (uniform; rows past row1 - 1 are clamped and their
// results dropped). A lane takes staged blocks l % G, l % G + G, ... of the row.
template <int G>
__device__ __forceinline__ int prow(int P, int r) {
    return P + (r * (64 / G) + (int)(threadIdx.x & 63) / G) * NWV + wave_id();
}
template <int G>
__device__ __forceinline__ int pslots(int P, int row1) {
    constexpr int step = (64 / G) * NWV;
    const int left = row1 - P - wave_id();
    return left <= 0 ? 0 : min(RW, (left + step - 1) / step);
}

// Every slot is loaded (rows clamped to row1 - 1), so the compiler's wait counts
// stay exact across the pipelined units.
template <int TYPE, int G>
__device__ __forceinline__ void load_blks(const MatView &w, int P, int row1, int c0, int b, Blk (&rb)[RW]) {
#pragma unroll
    for (int r = 0; r < RW; r++) blk_load<TYPE>(w, (size_t)min(prow<G>(P, r), row1 - 1) * w.nb + c0 + b, rb[r]);
}

// The staged block b of every state against the decoded blocks rb of the lane's
// rows: the rows' 32 codes are decoded once, then the states follow one another,
// each state's eight staged chunks read from LDS together; four partial sums per
// row keep the FMA chains short. `valid` false (a lane past the row's
// last block) leaves acc unchanged.
template <int TYPE>
__device__ __forceinline__ void dot_blk(const Blk (&rb)[RW], int nr, int S, int b, int nbc, bool valid,
                                        const float4 *xs, const float *sx, float (&acc)[RW][SMAX]) {
    float q[RW][32];
#pragma unroll
    for (int r = 0; r < RW; r++)
#pragma unroll
        for (int k = 0; k < 8; k++) {
            float c4[4];
            codes4<TYPE>(rb[r], k, c4);
            q[r][4 * k] = c4[0];
            q[r][4 * k + 1] = c4[1];
            q[r][4 * k + 2] = c4[2];
            q[r][4 * k + 3] = c4[3];
        }
#pragma unroll
    for (int s = 0; s < SMAX; s++) {
        if (s >= S) break;
        float4 xv[8];
#pragma unroll
        for (int k = 0; k < 8; k++) xv[k] = xs[slot(s, nbc, b, k)];
        const float bsum = TYPE == 8 ? 0.0f : sx[s * nbc + b];
#pragma unroll
        for (int r = 0; r < RW; r++) {
            if (r >= nr) continue;
            float p[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const float4 x = xv[k];
                float &c = p[k & 3];
                c = __builtin_fmaf(q[r][4 * k], x.x, c);
                c = __builtin_fmaf(q[r][4 * k + 1], x.y, c);
                c = __builtin_fmaf(q[r][4 * k + 2], x.z, c);
                c = __builtin_fmaf(q[r][4 * k + 3], x.w, c);
            }
            const float v = bscale<TYPE>(rb[r], (p[0] + p[1]) + (p[2] + p[3]), bsum);
            acc[r][s] += valid ? v : 0.0f;
        }
        // keep the next state's LDS reads after these FMAs
        asm volatile("" ::: "memory");
    }
}

// The epilogue operand pre(s, row) of each of the lane's rows for the state the
// lane finishes (lane % G), loaded before the dot products so that its latency
// overlaps the weight loads.
template <int G, class Pre, class PV>
__device__ __forceinline__ void load_pre(int P, int row1, int S, Pre pre, PV (&ad)[RW]) {
    const int st = min((int)(threadIdx.x & 63) % G, S - 1);
#pragma unroll
    for (int r = 0; r < RW; r++) ad[r] = pre(st, min(prow<G>(P, r), row1 - 1));
}

// Row sums over the lane groups; lane s of a group runs the epilogue of state s.
template <int G, class PV, class Epi>
__device__ __forceinline__ void finish(int P, int nr, int row1, int S, unsigned amask, float (&acc)[RW][SMAX],
                                       const PV (&ad)[RW], Epi epi) {
    const int gl = (int)(threadIdx.x & 63) % G;
#pragma unroll
    for (int r = 0; r < RW; r++) {
        if (r >= nr) continue;
        const int row = prow<G>(P, r);
        float mine = 0.0f;
#pragma unroll
        for (int s = 0; s < SMAX; s++)
            if (s < S) {
                const float v = gsum<G>(acc[r][s]);
                mine = gl == s ? v : mine;
            }
        if (gl < S && row < row1 && ((amask >> gl) & 1u)) epi(gl, row, mine, ad[r]);
    }
}

// ---- GEMV on the matrix cores ---------------------------------------------------------
// 16 weight rows x up to 16 states per tile with v_mfma_f32_16x16x4f32 (fp32
// operands: the codes are exact small integers). Lane l (r = l % 16, kq = l / 16)
// supplies, for the block's j-th product, element 8 kq + j of state r's staged
// row (chunks 2 kq and 2 kq + 1 of the block, two LDS reads) and of weight row r
// (its code: Q8_0 byte 8 kq + j; 4/5-bit nibble j of the word of bytes 4 kq ..,
// the nibbles interleaved in the device layout, plus high bit 8 kq + j); D register
// i of lane l is state 4 kq + i, row r, scaled per block (d, and the offset or m
// through the staged block sums) into the total. Each staged value is read by one
// lane per block instead of one per row, the lanes' dot products become 8 matrix
// instructions. The waves take the blocks of a tile in turn; their tiles are summed
// in wave order through LDS and thread t < 256 runs the epilogue of state t / 16,
// row t % 16.
struct MBlk {
    uint32_t a, b;  // the lane's code bytes (Q8_0: 8 in a, b; 4/5-bit: 4 in a)
    uint32_t s, h;  // scale word(s), Q5 high bits
};

template <int TYPE>
__device__ __forceinline__ void mblk_load(const MatView &m, int row, int b, int kq, MBlk &k) {
    const size_t blk = (size_t)row * m.nb + b;
    if constexpr (TYPE == 8) {
        k.a = *(gcu32 *)(m.qs + blk * 32 + 8 * kq);
        k.b = *(gcu32 *)(m.qs + blk * 32 + 8 * kq + 4);
        k.s = ((gcu16 *)m.sc)[blk];
        k.h = 0u;
    } else {
        k.a = *(gcu32 *)(m.qs + blk * 16 + 4 * kq);
        k.b = 0u;
        if constexpr (TYPE == 3 || TYPE == 7) k.s = ((gcu32 *)m.sc)[blk];
        else k.s = ((gcu16 *)m.sc)[blk];
        if constexpr (TYPE == 6 || TYPE == 7) k.h = ((gcu32 *)m.qh)[blk];
        else k.h = 0u;
    }
}

// code of element 8 kq + j of the lane's block
template <int TYPE>
__device__ __forceinline__ float mcode(const MBlk &k, int kq, int j) {
    if constexpr (TYPE == 8) {
        const uint32_t w = j < 4 ? k.a : k.b;
        return (float)(int)__builtin_amdgcn_sbfe((int)w, 8 * (j & 3), 8);  // the builtin's type is unsigned
    } else {
        uint32_t c = (k.a >> (4 * j)) & 0xFu;
        if constexpr (TYPE == 6 || TYPE == 7) c |= ((k.h >> (8 * kq + j)) & 1u) << 4;
        return (float)c;
    }
}

// staged block b (of nbc) against the lane's codes k; adds the block's terms to acc
template <int TYPE>
__device__ __forceinline__ void mdot(const MBlk &k, int S, int nbc, int b, const Lds &L, f32x4 &acc) {
    const int lane = threadIdx.x & 63, lr = lane & 15, kq = lane >> 4;
    float4 x0 = make_float4(0.f, 0.f, 0.f, 0.f), x1 = x0;
    if (lr < S) {
        x0 = L.xs[slot(lr, nbc, b, 2 * kq)];
        x1 = L.xs[slot(lr, nbc, b, 2 * kq + 1)];
    }
    const float xa[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    f32x4 t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 8; j++) t = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[j], mcode<TYPE>(k, kq, j), t, 0, 0, 0);
    Blk sb;
    sb.s = k.s;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int st = 4 * kq + i;
        const float sxv = (TYPE != 8 && st < S) ? L.sx[st * nbc + b] : 0.0f;
        acc[i] += bscale<TYPE>(sb, t[i], sxv);
    }
}

// The waves' tiles summed in wave order (in the LayerNorm weight area, free once
// the inputs are staged); out[t] for t < 256 is state t / 16, row t % 16.
__device__ __forceinline__ void mreduce(const f32x4 &acc, const Lds &L) {
    const int lane = threadIdx.x & 63, wv = wave_id(), lr = lane & 15, kq = lane >> 4;
    f32x4 *red = (f32x4 *)L.lw;  // [NWV][64]
    red[wv * 64 + lane] = acc;
    __syncthreads();
    if (wv == 0) {
        f32x4 sum = red[lane];
#pragma unroll
        for (int w = 1; w < NWV; w++) sum += red[w * 64 + lane];
#pragma unroll
        for (int i = 0; i < 4; i++) L.red[(4 * kq + i) * 16 + lr] = sum[i];
    }
    __syncthreads();
}

template <int TYPE, class Stage, class Pre, class Epi>
__device__ __forceinline__ void gemv_mf(const MatView &w, int row0, int row1, int S, unsigned amask, Stage stage,
                                        const Lds &L, Pre pre, Epi epi) {
    constexpr int U = 4;  // blocks of a wave per group
    const int nb = w.nb, lane = threadIdx.x & 63, wv = wave_id(), lr = lane & 15, kq = lane >> 4;
    const int ntile = (row1 - row0 + 15) / 16;
    const int ng = ((nb + NWV - 1) / NWV + U - 1) / U;  // groups of a tile (the same for every wave)
    const int NUn = ntile * ng;
    const int et = threadIdx.x, es = et >> 4, er = et & 15;  // epilogue: state es, row er of a tile
    decltype(pre(0, 0)) ep;
    const auto load_ep = [&](int tile) __attribute__((always_inline)) {
        if (et < 256) ep = pre(min(es, S - 1), min(row0 + 16 * tile + er, row1 - 1));
    };
    const auto load_unit = [&](int u, MBlk (&k)[U]) __attribute__((always_inline)) {
        const int tile = u / ng, g = u - tile * ng;
        const int row = min(row0 + 16 * tile + lr, row1 - 1);
#pragma unroll
        for (int v = 0; v < U; v++) mblk_load<TYPE>(w, row, min(wv + NWV * (g * U + v), nb - 1), kq, k[v]);
    };
    MBlk cur[U], nxt[U];
    load_unit(0, cur);
    load_ep(0);
    stage();
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int u = 0; u < NUn; u++) {
        const int tile = u / ng, g = u - tile * ng;
        if (u + 1 < NUn) load_unit(u + 1, nxt);
#pragma unroll
        for (int v = 0; v < U; v++) {
            const int b = wv + NWV * (g * U + v);
            if (b < nb) mdot<TYPE>(cur[v], S, nb, b, L, acc);
        }
#pragma unroll
        for (int v = 0; v < U; v++) cur[v] = nxt[v];
        if (g == ng - 1) {
            mreduce(acc, L);
            const int row = row0 + 16 * tile + er;
            if (et < 256 && es < S && row < row1 && ((amask >> es) & 1u)) epi(es, row, L.red[et], ep);
            if (tile + 1 < ntile) load_ep(tile + 1);
            acc = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }
    __syncthreads();
}

template <int TYPE, class FillC, class Pre, class Epi>
__device__ __forceinline__ void gemv_cols_mf(const MatView &w, int row0, int row1, int S, unsigned amask, FillC fillc,
                                             const Lds &L, Pre pre, Epi epi) {
    // one tile: the host sizes the grid so a workgroup has at most 16 rows here
    const int nb = w.nb, per = XBLK / S, lane = threadIdx.x & 63, wv = wave_id(), lr = lane & 15, kq = lane >> 4;
    const int et = threadIdx.x, es = et >> 4, er = et & 15;
    const int row = min(row0 + lr, row1 - 1);
    decltype(pre(0, 0)) ep;
    if (et < 256) ep = pre(min(es, S - 1), min(row0 + er, row1 - 1));
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int c0 = 0; c0 < nb; c0 += per) {
        const int nbc = min(per, nb - c0);
        stage_cols(S, nbc, [&]() __attribute__((always_inline)) { fillc(c0, nbc); }, L.xs, L.sx, TYPE != 8);
        for (int b = wv; b < nbc; b += NWV) {
            MBlk k;
            mblk_load<TYPE>(w, row, c0 + b, kq, k);
            mdot<TYPE>(k, S, nbc, b, L, acc);
        }
        __syncthreads();
    }
    mreduce(acc, L);
    if (et < 256 && es < S && row0 + er < row1 && ((amask >> es) & 1u)) epi(es, row0 + er, L.red[et], ep);
    __syncthreads();
}

// Rows [row0, row1) of w against inputs that stage() puts in LDS (all columns).
// A workgroup without rows returns at once (uniformly). The work is a sequence
// of units (row pass, block step); the first two units' weight blocks and the
// first pass's epilogue operands are loaded before stage() runs, and every unit
// loads the blocks of the unit two ahead while it computes.
template <int TYPE, int G, bool MF, class Stage, class Pre, class Epi>
__device__ __forceinline__ void gemv(const MatView &w, int row0, int row1, int S, unsigned amask, Stage stage,
                                     const Lds &L, Pre pre, Epi epi) {
    if (row0 >= row1) return;
    if constexpr (MF) {
        gemv_mf<TYPE>(w, row0, row1, S, amask, stage, L, pre, epi);
        return;
    }
    constexpr int PR = NWV * RW * (64 / G);  // rows of a workgroup's pass
    const int nb = w.nb, gl = (int)(threadIdx.x & 63) % G;
    const int NBJ = (nb + G - 1) / G, NU = (row1 - row0 + PR - 1) / PR * NBJ;
    const auto unit = [&](int u, Blk (&rb)[RW]) __attribute__((always_inline)) {
        const int p = u / NBJ, j = u - p * NBJ;
        load_blks<TYPE, G>(w, row0 + p * PR, row1, 0, min(gl + j * G, nb - 1), rb);
    };
    Blk b0[RW], b1[RW], b2[RW];
    float acc[RW][SMAX];
    decltype(pre(0, 0)) ad[RW];
    unit(0, b0);
    unit(min(1, NU - 1), b1);
    load_pre<G>(row0, row1, S, pre, ad);
    stage();
    for (int u = 0; u < NU; u++) {
        const int p = u / NBJ, j = u - p * NBJ, P = row0 + p * PR, nr = pslots<G>(P, row1);
        if (j == 0) {
#pragma unroll
            for (int r = 0; r < RW; r++)
#pragma unroll
                for (int s = 0; s < SMAX; s++) acc[r][s] = 0.0f;
            if (u > 0) load_pre<G>(P, row1, S, pre, ad);
        }
        unit(min(u + 2, NU - 1), b2);
        const int b = gl + j * G;
        dot_blk<TYPE>(b0, nr, S, min(b, nb - 1), nb, b < nb, L.xs, L.sx, acc);
        if (j == NBJ - 1) finish<G>(P, nr, row1, S, amask, acc, ad, epi);
#pragma unroll
        for (int r = 0; r < RW; r++) {
            b0[r] = b1[r];
            b1[r] = b2[r];
        }
    }
    __syncthreads();
}

// Rows [row0, row1) of w when the S states' input rows do not fit in LDS: passes
// over the columns, staged by fillc(c0, nbc); each wave keeps its rows' sums
// across the passes (the host sizes the grid so a workgroup has at most one pass
// of rows).
template <int TYPE, int G, bool MF, class FillC, class Pre, class Epi>
__device__ __forceinline__ void gemv_cols(const MatView &w, int row0, int row1, int S, unsigned amask, FillC fillc,
                                          const Lds &L, Pre pre, Epi epi) {
    if (row0 >= row1) return;
    if constexpr (MF) {
        gemv_cols_mf<TYPE>(w, row0, row1, S, amask, fillc, L, pre, epi);
        return;
    }
    const int nb = w.nb, per = XBLK / S, gl = (int)(threadIdx.x & 63) % G;
    const int nr = pslots<G>(row0, row1);
    decltype(pre(0, 0)) ad[RW];
    load_pre<G>(row0, row1, S, pre, ad);
    float acc[RW][SMAX];
#pragma unroll
    for (int r = 0; r < RW; r++)
#pragma unroll
        for (int s = 0; s < SMAX; s++) acc[r][s] = 0.0f;
    for (int c0 = 0; c0 < nb; c0 += per) {
        const int nbc = min(per, nb - c0);
        stage_cols(S, nbc, [&]() __attribute__((always_inline)) { fillc(c0, nbc); }, L.xs, L.sx, TYPE != 8);
        if (nr > 0)
            for (int b = gl; b < nbc; b += G) {
                Blk rb[RW];
                load_blks<TYPE, G>(w, row0, row1, c0, b, rb);
                dot_blk<TYPE>(rb, nr, S, b, nbc, true, L.xs, L.sx, acc);
            }
        __syncthreads();
    }
    if (nr > 0) finish<G>(row0, nr, row1, S, amask, acc, ad, epi);
    __syncthreads();
}

// All columns staged by fillc when they fit, else column passes.
template <int TYPE, int G, bool MF, class FillC, class Pre, class Epi>
__device__ __forceinline__ void gemv_src(const MatView &w, int row0, int row1, int S, unsigned amask, FillC fillc,
                                         const Lds &L, Pre pre, Epi epi) {
    if (w.nb <= XBLK / S)
        gemv<TYPE, G, MF>(
            w, row0, row1, S, amask,
            [&]() __attribute__((always_inline)) {
                stage_cols(S, w.nb, [&]() __attribute__((always_inline)) { fillc(0, w.nb); }, L.xs, L.sx, TYPE != 8);
            },
            L, pre, epi);
    else
        gemv_cols<TYPE, G, MF>(w, row0, row1, S, amask, fillc, L, pre, epi);
}

__device__ __forceinline__ int split(int n, int w, int W) { return (int)((long)n * w / W); }

// ---- the step ------------------------------------------------------------------------------
// epilogue operands: pairs already loaded, checked for their tag when used
struct PreXS {  // x and sa_l of the row, the bias
    uint64_t x, sa;
    float b;
};
struct PreX2 {  // x2 of the row, the bias
    uint64_t x2;
    float b;
};

// G: lanes per row group, 32 for models of width <= 1024, else 64; MF: GEMV rows on
// the matrix cores (gemv_mf) instead of the lanes' dot products
template <int TYPE, int G, bool MF>
__global__ __launch_bounds__(NT) void k_fwd_batch(BArgs a) {
    extern __shared__ float4 lds4[];
    Lds L;
    L.xs = lds4;
    L.sx = (float *)(lds4 + XBLK * 8);
    L.lw = L.sx + XBLK;
    L.lb = L.lw + LNMAX;
    L.pos = (int *)(L.lb + LNMAX);
    L.stat = (float *)(L.pos + 16);
    L.red = (float *)(L.pos + 64);
    BLayer *lyl = (BLayer *)(L.red + 1024);  // the layer descriptors, copied once
    const int W = (int)gridDim.x, w = (int)blockIdx.x;
    const int S = a.S, d = a.d, H = a.H, Ln = a.L;
    {
        const int n = Ln * (int)(sizeof(BLayer) / 8);
        for (int i = threadIdx.x; i < n; i += NT) ((uint64_t *)lyl)[i] = ((gcu64 *)a.layers)[i];
    }
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    // the phase counter continues from this workgroup's last published phase (every
    // workgroup advances it alike, so all start from the same value)
    unsigned *const flags = a.flags, *const errw = a.err;
    unsigned g = __hip_atomic_load(flags + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    unsigned amask = 0;
    bool pos0 = false;
    for (int s = 0; s < S; s++) {
        const bool on = a.active[s] != 0;
        amask |= (unsigned)on << s;
        pos0 |= on && a.posv[s] == 0;
    }
    if (threadIdx.x < S) L.pos[threadIdx.x] = a.posv[threadIdx.x];
    __syncthreads();

    const int ctx = a.ctx, enc_len = a.enc_len;
    const size_t kvs = a.kv_stream, plane = (size_t)H * ctx * 64;
    uint64_t *const xg = a.x, *const x2g = a.x2, *const qg = a.q, *const hg = a.h, *const atg = a.attn;
    uint64_t *const sag = a.sa;
    const int *posl = L.pos;
    const auto nopre = [](int, int) { return make_float2(0.f, 0.f); };
    // staging of [S][cols] pair vectors (rows ld apart), tags >= t
    const auto fill_pairs = [&](const uint64_t *v, unsigned t, size_t ld, int cols) __attribute__((always_inline)) {
        return [=](int c0, int nbc) __attribute__((always_inline)) {
            burst_pairs<PU, false>(S, amask, cols, c0, nbc, v, t, nullptr, 0, ld, L.xs, errw);
        };
    };
    // rows of this layer's self-attention output sa_l = Wo V0 + bo (V0: KV row 0), tag t
    const auto sa_rows = [&](const BLayer *ly, uint64_t *sal, int r0, int r1, unsigned t) __attribute__((always_inline)) {
        const float *vp = ly->kv + plane;
        const float *sob = ly->sob;
        gemv_src<TYPE, G, MF>(
            ly->so, r0, r1, S, amask,
            [&](int c0, int nbc) __attribute__((always_inline)) {
                burst(S, d, c0, nbc,
                      [=](int s, int c) { return ldx4(vp + (size_t)s * kvs + (size_t)(c >> 6) * ctx * 64 + (c & 63)); },
                      L.xs);
            },
            L, [=](int, int r) { return make_float2(0.f, ldg(sob + r)); },
            [=](int s, int r, float v, float2 p) { stp(sal + (size_t)s * d + r, v + p.y, t); });
    };
    // k,v rows [d + r0, d + r1) of the stacked q,k,v matrix into the KV cache at pos,
    // from LN1 of x (tag tx)
    const auto kv_rows = [&](const BLayer *ly, int r0, int r1, unsigned tx) __attribute__((always_inline)) {
        const float *lw = ly->ln1w, *lb = ly->ln1b;
        float *kv = ly->kv;
        const float *svb = ly->svb;
        gemv<TYPE, G, MF>(ly->sqkv, d + r0, d + r1, S, amask,
                   [&]() __attribute__((always_inline)) {
                       stage_ln(S, d,
                                [&]() __attribute__((always_inline)) {
                                    burst_pairs<PU, false>(S, amask, d, 0, d / 32, xg, tx, nullptr, 0, d, L.xs, errw);
                                },
                                lw, lb, L, TYPE != 8);
                   }, L,
                   [=](int, int r) { return make_float2(0.f, r >= 2 * d ? ldg(svb + r - 2 * d) : 0.0f); },
                   [=](int s, int r, float v, float2 p) {
                       const int j = r % d;
                       stx(kv + (size_t)s * kvs + (r >= 2 * d ? plane : 0) + (size_t)(j >> 6) * ctx * 64 +
                               (size_t)posl[s] * 64 + (j & 63),
                           v + p.y);
                   });
    };
    // cross query rows [r0, r1) from LN2(x + sa_l) (tags tx, tsa) into q (tag t)
    const auto cq_rows = [&](const BLayer *ly, const uint64_t *sal, int r0, int r1, unsigned tx, unsigned tsa,
                             unsigned t) __attribute__((always_inline)) {
        const float *lw = ly->ln2w, *lb = ly->ln2b;
        const float *cqb = ly->cqb;
        gemv<TYPE, G, MF>(ly->cq, r0, r1, S, amask,
                   [&]() __attribute__((always_inline)) {
                       stage_ln(S, d,
                                [&]() __attribute__((always_inline)) {
                                    burst_pairs<PU2, true>(S, amask, d, 0, d / 32, xg, tx, sal, tsa, d, L.xs, errw);
                                },
                                lw, lb, L, TYPE != 8);
                   }, L, [=](int, int r) { return make_float2(0.f, ldg(cqb + r)); },
                   [=](int s, int r, float v, float2 p) { stp(qg + (size_t)s * d + r, v + p.y, t); });
    };

    // embedding (decoder.go:756-773): the quantised row is dequantised bit-exactly
    const unsigned tE = ++g;
    for (int i = split(S * d, w, W) + threadIdx.x; i < split(S * d, w + 1, W); i += NT) {
        const int s = i / d, e = i % d;
        if (!((amask >> s) & 1u)) continue;
        stp(xg + i, dequant_elem<TYPE>(a.tok, a.tokv[s], e >> 5, e & 31) + ldg(a.pos_emb + (size_t)posl[s] * d + e),
            tE);
    }
    // past position 0 every layer's sa_l is known now: its rows for all layers
    if (!pos0) {
        const int r0 = split(Ln * d, w, W), r1 = split(Ln * d, w + 1, W);
        for (int l = r0 / d; l < Ln && l * d < r1; l++)
            sa_rows(lyl + l, sag + (size_t)l * S * d, max(r0, l * d) - l * d, min(r1, (l + 1) * d) - l * d, tE);
    }
    __syncthreads();

    // after a failed wait every wait returns at once: the launch runs out and the
    // host reports the failure
    const int Wk = W - W / 3;  // k,v workgroups of phase B
    unsigned tx = tE;          // tag of the current x
    for (int l = 0; l < Ln; l++) {
        const BLayer *ly = lyl + l;
        uint64_t *sal = sag + (size_t)l * S * d;
        // ---- B: k,v rows; cross query rows ----
        unsigned tsa = tE, tq;
        if (pos0) {
            kv_rows(ly, split(2 * d, w, W), split(2 * d, w + 1, W), tx);
            gbar(flags, errw, g);  // V0 is read as plain floats next
            tsa = ++g;
            sa_rows(ly, sal, split(d, w, W), split(d, w + 1, W), tsa);
            tq = ++g;
            cq_rows(ly, sal, split(d, w, W), split(d, w + 1, W), tx, tsa, tq);
        } else {
            tq = ++g;
            if (w < Wk)
                kv_rows(ly, split(2 * d, w, Wk), split(2 * d, w + 1, Wk), tx);
            else
                cq_rows(ly, sal, split(d, w - Wk, W - Wk), split(d, w + 1 - Wk, W - Wk), tx, tsa, tq);
        }
        // ---- X: cross attention; item (state, head, key chunk) on workgroup w ----
        const unsigned tX = ++g;
        {
            // one item per workgroup when they fit the grid; else XC is 1 and a
            // workgroup takes whole heads one after another (no exchange to wait on)
            const int XC = a.xchunks, klen = (enc_len + XC - 1) / XC;
            for (int it = w; it < S * H * XC; it += W) {
            const int s = it / (H * XC), h = (it / XC) % H, c = it % XC;
            if ((amask >> s) & 1u) {
                constexpr int KG = 4 * NWV;  // keys per step: 16 lanes per key
                constexpr int XS = 12;       // steps per batch
                const int q16 = lane & 15, kq = wv * 4 + (lane >> 4);  // the lane's key of a step
                const size_t sh = (size_t)s * H + h;
                float4 q4;
                {
                    const uint64_t *qp = qg + (size_t)s * d + h * 64 + q16 * 4;
                    const uint64_t v0 = ldp(qp), v1 = ldp(qp + 1), v2 = ldp(qp + 2), v3 = ldp(qp + 3);
                    q4 = make_float4(waitp(qp, v0, tq, errw), waitp(qp + 1, v1, tq, errw), waitp(qp + 2, v2, tq, errw),
                                     waitp(qp + 3, v3, tq, errw));
                }
                const float *K = (const float *)((gcu64 *)ly->kbase)[s] + (size_t)h * enc_len * 64;
                const float *V = (const float *)((gcu64 *)ly->vbase)[s] + (size_t)h * enc_len * 64;
                const int t0 = c * klen, t1 = min(t0 + klen, enc_len);
                float *scl = (float *)L.xs;  // the chunk's scores
                // scores, XS steps per batch, the next batch's K loads in flight
                float mx = -INFINITY;
                float4 kb[XS];
#pragma unroll
                for (int j = 0; j < XS; j++) {
                    const int t = t0 + j * KG + kq;
                    kb[j] = t < t1 ? ldg4(K + (size_t)t * 64 + q16 * 4) : make_float4(0.f, 0.f, 0.f, 0.f);
                }
                for (int tb = t0; tb < t1; tb += XS * KG) {
                    float4 kn[XS];
#pragma unroll
                    for (int j = 0; j < XS; j++) {
                        const int t = tb + XS * KG + j * KG + kq;
                        kn[j] = t < t1 ? ldg4(K + (size_t)t * 64 + q16 * 4) : make_float4(0.f, 0.f, 0.f, 0.f);
                    }
#pragma unroll
                    for (int j = 0; j < XS; j++) {
                        const int t = tb + j * KG + kq;
                        float dot = q4.x * kb[j].x + q4.y * kb[j].y + q4.z * kb[j].z + q4.w * kb[j].w;
#pragma unroll
                        for (int o = 8; o > 0; o >>= 1) dot += __shfl_xor(dot, o, 64);
                        if (t < t1) {
                            const float sco = dot * a.scale;
                            if (q16 == 0) scl[t - t0] = sco;
                            mx = fmaxf(mx, sco);
                        }
                    }
#pragma unroll
                    for (int j = 0; j < XS; j++) kb[j] = kn[j];
                }
                // the first V batch loads, independent of the maximum, go out now
                float4 vb[XS];
#pragma unroll
                for (int j = 0; j < XS; j++) {
                    const int t = t0 + j * KG + kq;
                    vb[j] = t < t1 ? ldg4(V + (size_t)t * 64 + q16 * 4) : make_float4(0.f, 0.f, 0.f, 0.f);
                }
                mx = wmax(mx);
                if (lane == 0) L.red[wv] = mx;
                __syncthreads();
                float M = L.red[0];
                for (int i = 1; i < NWV; i++) M = fmaxf(M, L.red[i]);
                // the head maximum: the chunk maxima of the head's workgroups
                if (XC > 1) {
                    if (threadIdx.x == 0) stp(a.xmax + it, M, tX);
                    if (threadIdx.x < 64) {
                        const uint64_t *src = a.xmax + sh * XC;
                        const int li = min(lane, XC - 1);
                        const float m = wmax(waitp(src + li, ldp(src + li), tX, errw));
                        if (lane == 0) L.red[8] = m;
                    }
                    __syncthreads();
                    M = L.red[8];
                }
                // fast-exp weights against the head maximum and the chunk's P.V
                float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
                float es = 0.0f;
                for (int tb = t0; tb < t1; tb += XS * KG) {
                    float4 vn[XS];
#pragma unroll
                    for (int j = 0; j < XS; j++) {
                        const int t = tb + XS * KG + j * KG + kq;
                        vn[j] = t < t1 ? ldg4(V + (size_t)t * 64 + q16 * 4) : make_float4(0.f, 0.f, 0.f, 0.f);
                    }
#pragma unroll
                    for (int j = 0; j < XS; j++) {
                        const int t = tb + j * KG + kq;
                        if (t < t1) {
                            const float e = fast_exp(scl[t - t0] - M);
                            acc.x += e * vb[j].x; acc.y += e * vb[j].y; acc.z += e * vb[j].z; acc.w += e * vb[j].w;
                            if (q16 == 0) es += e;
                        }
                    }
#pragma unroll
                    for (int j = 0; j < XS; j++) vb[j] = vn[j];
                }
#pragma unroll
                for (int o = 16; o < 64; o <<= 1) {
                    acc.x += __shfl_xor(acc.x, o, 64);
                    acc.y += __shfl_xor(acc.y, o, 64);
                    acc.z += __shfl_xor(acc.z, o, 64);
                    acc.w += __shfl_xor(acc.w, o, 64);
                }
                es = wsum(es);
                float4 *red4 = (float4 *)(L.red + 64);  // [NWV][16]
                float *own = L.red + 640;              // the chunk's P.V [64] and weight sum [64]
                if (lane < 16) red4[wv * 16 + lane] = acc;
                if (lane == 0) L.red[16 + wv] = es;
                __syncthreads();
                if (threadIdx.x < 16) {
                    float4 r = red4[threadIdx.x];
                    for (int i = 1; i < NWV; i++) {
                        const float4 t4 = red4[i * 16 + threadIdx.x];
                        r.x += t4.x; r.y += t4.y; r.z += t4.z; r.w += t4.w;
                    }
                    *(float4 *)(own + 4 * threadIdx.x) = r;
                }
                if (threadIdx.x == 0) {
                    float t = 0.0f;
                    for (int i = 0; i < NWV; i++) t += L.red[16 + i];
                    own[64] = t;
                }
                __syncthreads();
                uint64_t *at = atg + (size_t)s * d + h * 64;
                if (XC == 1) {
                    if (threadIdx.x < 64) stp(at + threadIdx.x, own[threadIdx.x] * (1.0f / own[64]), tX);
                } else {
                    // the chunk's P.V and weight sum; the head's first chunk adds the
                    // others' in chunk order: attn = sum P.V * (1 / sum of weight sums)
                    if (threadIdx.x < 65) stp(a.pv + (size_t)it * 65 + threadIdx.x, own[threadIdx.x], tX);
                    if (c == 0) {
                        // thread t: element t % 65 (P.V columns, then the weight sum) of
                        // chunk 1 + t / 65, into LDS; then lane j adds column j in chunk order
                        float *oth = scl;  // [XC - 1][65], over the chunk's scores (used up)
                        const int t = threadIdx.x;
                        if (t < (XC - 1) * 65) {
                            const uint64_t *pp = a.pv + ((size_t)it + 1) * 65 + t;
                            oth[t] = waitp(pp, ldp(pp), tX, errw);
                        }
                        __syncthreads();
                        if (t < 64) {
                            float o = own[t], sum = own[64];
                            for (int i = 1; i < XC; i++) {
                                o += oth[(i - 1) * 65 + t];
                                sum += oth[(i - 1) * 65 + 64];
                            }
                            stp(at + t, o * (1.0f / sum), tX);
                        }
                    }
                }
                __syncthreads();  // LDS scores and reduction area free for the next item
            }
            }
        }
        // ---- F: cross out rows; x2 = (x + sa_l) + (Wo_c.attn + b) ----
        const unsigned tF = ++g;
        {
            const float *cob = ly->cob;
            gemv_src<TYPE, G, MF>(
                ly->co, split(d, w, W), split(d, w + 1, W), S, amask, fill_pairs(atg, tX, d, d), L,
                [=](int s, int r) {
                    return PreXS{ldp(xg + (size_t)s * d + r), ldp(sal + (size_t)s * d + r), ldg(cob + r)};
                },
                [=](int s, int r, float v, PreXS p) {
                    const float xv = waitp(xg + (size_t)s * d + r, p.x, tx, errw);
                    const float sv = waitp(sal + (size_t)s * d + r, p.sa, tsa, errw);
                    stp(x2g + (size_t)s * d + r, (xv + sv) + (v + p.b), tF);
                });
        }
        // ---- G: LN3, fc1 rows + GELU ----
        const unsigned tG = ++g;
        {
            const int r0 = split(4 * d, w, W), r1 = split(4 * d, w + 1, W);
            if (r0 < r1) {
                const float *fc1b = ly->fc1b, *lw = ly->ln3w, *lb = ly->ln3b;
                gemv<TYPE, G, MF>(ly->fc1, r0, r1, S, amask,
                           [&]() __attribute__((always_inline)) {
                               stage_ln(S, d,
                                        [&]() __attribute__((always_inline)) {
                                            burst_pairs<PU, false>(S, amask, d, 0, d / 32, x2g, tF, nullptr, 0, d, L.xs,
                                                                  errw);
                                        },
                                        lw, lb, L, TYPE != 8);
                           }, L,
                           [=](int, int r) { return make_float2(0.f, ldg(fc1b + r)); },
                           [=](int s, int r, float v, float2 p) {
                               stp(hg + (size_t)s * 4 * d + r, gelu_ref(v + p.y), tG);
                           });
            }
        }
        // ---- H: fc2 rows; x = x2 + (W2.h + b2) ----
        const unsigned tH = ++g;
        {
            const float *fc2b = ly->fc2b;
            gemv_src<TYPE, G, MF>(
                ly->fc2, split(d, w, W), split(d, w + 1, W), S, amask, fill_pairs(hg, tG, (size_t)4 * d, 4 * d), L,
                [=](int s, int r) { return PreX2{ldp(x2g + (size_t)s * d + r), ldg(fc2b + r)}; },
                [=](int s, int r, float v, PreX2 p) {
                    stp(xg + (size_t)s * d + r, waitp(x2g + (size_t)s * d + r, p.x2, tF, errw) + (v + p.b), tH);
                });
        }
        tx = tH;
    }
    // ---- final LayerNorm and tied logits rows (decoder.go:817-832) ----
    {
        const int r0 = split(a.V, w, W), r1 = split(a.V, w + 1, W);
        if (r0 < r1) {
            const float *lw = a.lnw, *lb = a.lnb;
            float *lg = a.logits;
            const int V = a.V;
            gemv<TYPE, G, MF>(a.tok, r0, r1, S, amask,
                       [&]() __attribute__((always_inline)) {
                           stage_ln(S, d,
                                    [&]() __attribute__((always_inline)) {
                                        burst_pairs<PU, false>(S, amask, d, 0, d / 32, xg, tx, nullptr, 0, d, L.xs,
                                                              errw);
                                    },
                                    lw, lb, L, TYPE != 8);
                       }, L, nopre,
                       [=](int s, int r, float v, float2) { stg(lg + (size_t)s * V + r, v); });
        }
    }
    // the next launch continues from this phase
    if (threadIdx.x == 0) __hip_atomic_store(flags + w, g, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Loads the code objects of the instantiations a model of width d launches (the
// runtime loads them on first use otherwise, in the first step).
template <int TYPE>
int warm_type(int d) {
    hipFuncAttributes attr;
    const void *fns[2] = {d <= 1024 ? (const void *)k_fwd_batch<TYPE, 32, false> : (const void *)k_fwd_batch<TYPE, 64, false>,
                          d <= 1024 ? (const void *)k_fwd_batch<TYPE, 32, true> : (const void *)k_fwd_batch<TYPE, 64, true>};
    for (const void *fn : fns) WH_HIP(hipFuncGetAttributes(&attr, fn));
    return WH_OK;
}

// Launch of the kernel for weight type TYPE; G from the model width.
template <int TYPE>
int launch_type(int grid, const BArgs &a, hipStream_t st) {
    void *args[] = {(void *)&a};
    const void *fn = a.mfma ? (a.d <= 1024 ? (const void *)k_fwd_batch<TYPE, 32, true> : (const void *)k_fwd_batch<TYPE, 64, true>)
                            : (a.d <= 1024 ? (const void *)k_fwd_batch<TYPE, 32, false> : (const void *)k_fwd_batch<TYPE, 64, false>);
    WH_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)LDS_BYTES));
    WH_HIP(hipLaunchCooperativeKernel(fn, dim3(grid), dim3(NT), args, LDS_BYTES, st));
    return WH_OK;
}

}  // namespace batch
}  // namespace wh
