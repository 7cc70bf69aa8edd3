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
//       workgroups (a {phase, value} exchange among them, no grid barrier),
//       fast-exp weights against it and the chunk's partial P.V
//   F   cross out rows on attn = (sum of the head's partial P.V) / (sum of its
//       weight sums), combined while staging: x2 = (x + sa_l) + (Wo_c.attn + b)
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
// launch is stored and loaded with relaxed agent-scope atomics, which bypass
// the per-XCD caches, so the barrier needs no cache writeback or invalidation:
// each wave waits for its stores to complete, the workgroup publishes its phase
// number and waits until all workgroups have published it. Every wait is
// bounded: on expiry the error word is set, later waits return at once, and the
// host reports a failure.
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

// ---- grid barrier -------------------------------------------------------------------
__device__ __forceinline__ bool failed(unsigned *err) {
    return __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
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

template <class Src>
__device__ __forceinline__ void stage_cols(int S, int cols, int c0, int nbc, Src src, float4 *xs, float *sx, bool sums) {
    burst(S, cols, c0, nbc, src, xs);
    __syncthreads();
    if (sums) {
        stage_sums(S, nbc, xs, sx);
        __syncthreads();
    }
}

// LayerNorm (internal/ml/ops.go:153-202) of the d-element rows src(s, .) of the
// S states into the staged layout: the mean, then the mean of squared
// deviations, std = float32(sqrt(float64(var + eps))), w*(x-mean)/std + b. The
// rows and the weights are loaded in one burst; the statistics take one wave per
// state, the normalisation every thread.
template <class Src>
__device__ __forceinline__ void stage_ln(int S, int d, Src src, const float *w, const float *bb, const Lds &L, bool sums) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int nbc = d / 32, dq = d / 4;
    const int iw = min((int)threadIdx.x, dq - 1);  // d <= 4 NT
    const float4 wr = ldg4(w + 4 * iw), br = ldg4(bb + 4 * iw);
    burst(S, d, 0, nbc, src, L.xs);
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
template <int G, class Pre>
__device__ __forceinline__ void load_pre(int P, int row1, int S, Pre pre, float2 (&ad)[RW]) {
    const int st = min((int)(threadIdx.x & 63) % G, S - 1);
#pragma unroll
    for (int r = 0; r < RW; r++) ad[r] = pre(st, min(prow<G>(P, r), row1 - 1));
}

// Row sums over the lane groups; lane s of a group runs the epilogue of state s.
template <int G, class Epi>
__device__ __forceinline__ void finish(int P, int nr, int row1, int S, unsigned amask, float (&acc)[RW][SMAX],
                                       const float2 (&ad)[RW], Epi epi) {
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

// Rows [row0, row1) of w against inputs that stage() puts in LDS (all columns).
// A workgroup without rows returns at once (uniformly). The work is a sequence
// of units (row pass, block step); the first two units' weight blocks and the
// first pass's epilogue operands are loaded before stage() runs, and every unit
// loads the blocks of the unit two ahead while it computes.
template <int TYPE, int G, class Stage, class Pre, class Epi>
__device__ __forceinline__ void gemv(const MatView &w, int row0, int row1, int S, unsigned amask, Stage stage,
                                     const Lds &L, Pre pre, Epi epi) {
    if (row0 >= row1) return;
    constexpr int PR = NWV * RW * (64 / G);  // rows of a workgroup's pass
    const int nb = w.nb, gl = (int)(threadIdx.x & 63) % G;
    const int NBJ = (nb + G - 1) / G, NU = (row1 - row0 + PR - 1) / PR * NBJ;
    const auto unit = [&](int u, Blk (&rb)[RW]) __attribute__((always_inline)) {
        const int p = u / NBJ, j = u - p * NBJ;
        load_blks<TYPE, G>(w, row0 + p * PR, row1, 0, min(gl + j * G, nb - 1), rb);
    };
    Blk b0[RW], b1[RW], b2[RW];
    float acc[RW][SMAX];
    float2 ad[RW];
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
// over the columns, staged from src; each wave keeps its rows' sums across the
// passes (the host sizes the grid so a workgroup has at most one pass of rows).
template <int TYPE, int G, class Src, class Pre, class Epi>
__device__ __forceinline__ void gemv_cols(const MatView &w, int row0, int row1, int S, unsigned amask, Src src,
                                          const Lds &L, Pre pre, Epi epi) {
    if (row0 >= row1) return;
    const int nb = w.nb, per = XBLK / S, gl = (int)(threadIdx.x & 63) % G;
    const int nr = pslots<G>(row0, row1);
    float2 ad[RW];
    load_pre<G>(row0, row1, S, pre, ad);
    float acc[RW][SMAX];
#pragma unroll
    for (int r = 0; r < RW; r++)
#pragma unroll
        for (int s = 0; s < SMAX; s++) acc[r][s] = 0.0f;
    for (int c0 = 0; c0 < nb; c0 += per) {
        const int nbc = min(per, nb - c0);
        stage_cols(S, w.cols, c0, nbc, src, L.xs, L.sx, TYPE != 8);
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

// All columns staged from src when they fit, else column passes.
template <int TYPE, int G, class Src, class Pre, class Epi>
__device__ __forceinline__ void gemv_src(const MatView &w, int row0, int row1, int S, unsigned amask, Src src,
                                         const Lds &L, Pre pre, Epi epi) {
    if (w.nb <= XBLK / S)
        gemv<TYPE, G>(
            w, row0, row1, S, amask,
            [&]() __attribute__((always_inline)) { stage_cols(S, w.cols, 0, w.nb, src, L.xs, L.sx, TYPE != 8); }, L,
            pre, epi);
    else
        gemv_cols<TYPE, G>(w, row0, row1, S, amask, src, L, pre, epi);
}

__device__ __forceinline__ int split(int n, int w, int W) { return (int)((long)n * w / W); }

// ---- the step ------------------------------------------------------------------------------
// G: lanes per row group, 32 for models of width <= 1024, else 64
template <int TYPE, int G>
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
    // workgroup passes the same barriers, so all start from the same value)
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
    float *xg = a.x, *x2g = a.x2, *qg = a.q, *hg = a.h, *sag = a.sa;
    const int *posl = L.pos;
    const auto nopre = [](int, int) { return make_float2(0.f, 0.f); };
    // rows of this layer's self-attention output sa_l = Wo V0 + bo (V0: KV row 0)
    const auto sa_rows = [&](const BLayer *ly, float *sal, int r0, int r1) __attribute__((always_inline)) {
        const float *vp = ly->kv + plane;
        const float *sob = ly->sob;
        gemv_src<TYPE, G>(
            ly->so, r0, r1, S, amask,
            [=](int s, int c) { return ldx4(vp + (size_t)s * kvs + (size_t)(c >> 6) * ctx * 64 + (c & 63)); }, L,
            [=](int, int r) { return make_float2(0.f, ldg(sob + r)); },
            [=](int s, int r, float v, float2 p) { stx(sal + (size_t)s * d + r, v + p.y); });
    };
    // k,v rows [d + r0, d + r1) of the stacked q,k,v matrix into the KV cache at pos
    const auto kv_rows = [&](const BLayer *ly, int r0, int r1) __attribute__((always_inline)) {
        const float *xr = xg, *lw = ly->ln1w, *lb = ly->ln1b;
        float *kv = ly->kv;
        const float *svb = ly->svb;
        gemv<TYPE, G>(ly->sqkv, d + r0, d + r1, S, amask,
                   [&]() __attribute__((always_inline)) {
                       stage_ln(S, d, [=](int s, int c) { return ldx4(xr + (size_t)s * d + c); }, lw, lb, L, TYPE != 8);
                   }, L,
                   [=](int, int r) { return make_float2(0.f, r >= 2 * d ? ldg(svb + r - 2 * d) : 0.0f); },
                   [=](int s, int r, float v, float2 p) {
                       const int j = r % d;
                       stx(kv + (size_t)s * kvs + (r >= 2 * d ? plane : 0) + (size_t)(j >> 6) * ctx * 64 +
                               (size_t)posl[s] * 64 + (j & 63),
                           v + p.y);
                   });
    };
    // cross query rows [r0, r1) from LN2(x + sa_l)
    const auto cq_rows = [&](const BLayer *ly, const float *sal, int r0, int r1) __attribute__((always_inline)) {
        const float *xr = xg, *lw = ly->ln2w, *lb = ly->ln2b;
        const float *cqb = ly->cqb;
        float *qw = qg;
        gemv<TYPE, G>(ly->cq, r0, r1, S, amask,
                   [&]() __attribute__((always_inline)) {
                       stage_ln(
                           S, d,
                           [=](int s, int c) {
                               const float4 u = ldx4(xr + (size_t)s * d + c), v = ldx4(sal + (size_t)s * d + c);
                               return make_float4(u.x + v.x, u.y + v.y, u.z + v.z, u.w + v.w);
                           },
                           lw, lb, L, TYPE != 8);
                   }, L, [=](int, int r) { return make_float2(0.f, ldg(cqb + r)); },
                   [=](int s, int r, float v, float2 p) { stx(qw + (size_t)s * d + r, v + p.y); });
    };

    // embedding (decoder.go:756-773): the quantised row is dequantised bit-exactly
    for (int i = split(S * d, w, W) + threadIdx.x; i < split(S * d, w + 1, W); i += NT) {
        const int s = i / d, e = i % d;
        if (!((amask >> s) & 1u)) continue;
        stx(xg + i, dequant_elem<TYPE>(a.tok, a.tokv[s], e >> 5, e & 31) + ldg(a.pos_emb + (size_t)posl[s] * d + e));
    }
    // past position 0 every layer's sa_l is known now: its rows for all layers
    if (!pos0) {
        const int r0 = split(Ln * d, w, W), r1 = split(Ln * d, w + 1, W);
        for (int l = r0 / d; l < Ln && l * d < r1; l++)
            sa_rows(lyl + l, sag + (size_t)l * S * d, max(r0, l * d) - l * d, min(r1, (l + 1) * d) - l * d);
    }
    gbar(flags, errw, g);

    // after a failed wait every barrier returns at once: the launch runs out and the
    // host reports the failure
    const int Wk = W - W / 3;  // k,v workgroups of phase B
    for (int l = 0; l < Ln; l++) {
        const BLayer *ly = lyl + l;
        float *sal = sag + (size_t)l * S * d;
        // ---- B: k,v rows; cross query rows ----
        if (pos0) {
            kv_rows(ly, split(2 * d, w, W), split(2 * d, w + 1, W));
            gbar(flags, errw, g);
            sa_rows(ly, sal, split(d, w, W), split(d, w + 1, W));
            gbar(flags, errw, g);
            cq_rows(ly, sal, split(d, w, W), split(d, w + 1, W));
        } else if (w < Wk) {
            kv_rows(ly, split(2 * d, w, Wk), split(2 * d, w + 1, Wk));
        } else {
            cq_rows(ly, sal, split(d, w - Wk, W - Wk), split(d, w + 1 - Wk, W - Wk));
        }
        gbar(flags, errw, g);
        // ---- X: cross attention; item (state, head, key chunk) on workgroup w ----
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
                const float4 q4 = ldx4(qg + (size_t)s * d + h * 64 + q16 * 4);
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
                // the head maximum: the chunk maxima of the head's workgroups, exchanged as
                // {phase, value} pairs (no grid barrier)
                if (XC > 1) {
                    if (threadIdx.x == 0)
                        __hip_atomic_store((gu64 *)(a.xmax + it), ((uint64_t)g << 32) | __float_as_uint(M),
                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if (threadIdx.x < 64) {
                        gcu64 *src = (gcu64 *)(a.xmax + sh * XC);
                        const int li = min(lane, XC - 1);
                        uint64_t v = __hip_atomic_load(src + li, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        for (unsigned spins = 0;; spins++) {
                            if (__all((unsigned)(v >> 32) >= g)) break;
                            if (__any(failed(errw) || spins > SPIN_MAX)) {
                                if (lane == 0) atomicOr(errw, 1u);
                                break;
                            }
                            if ((unsigned)(v >> 32) < g)
                                v = __hip_atomic_load(src + li, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        }
                        const float m = wmax(__uint_as_float((uint32_t)v));
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
                if (lane < 16) red4[wv * 16 + lane] = acc;
                if (lane == 0) L.red[16 + wv] = es;
                __syncthreads();
                if (threadIdx.x < 16) {
                    float4 r = red4[threadIdx.x];
                    for (int i = 1; i < NWV; i++) {
                        const float4 t4 = red4[i * 16 + threadIdx.x];
                        r.x += t4.x; r.y += t4.y; r.z += t4.z; r.w += t4.w;
                    }
                    float *dst = a.pv + (size_t)it * 64 + threadIdx.x * 4;
                    stx(dst, r.x); stx(dst + 1, r.y); stx(dst + 2, r.z); stx(dst + 3, r.w);
                }
                if (threadIdx.x == 0) {
                    float t = 0.0f;
                    for (int i = 0; i < NWV; i++) t += L.red[16 + i];
                    stx(a.psum + it, t);
                }
                __syncthreads();  // LDS scores and reduction area free for the next item
            }
            }
        }
        gbar(flags, errw, g);
        // ---- F: cross out rows on the combined heads; x2 = (x + sa_l) + (Wo_c.attn + b) ----
        {
            const float *cob = ly->cob, *xr = xg, *pvr = a.pv, *psr = a.psum;
            float *x2w = x2g;
            const int XC = a.xchunks;
            gemv_src<TYPE, G>(
                ly->co, split(d, w, W), split(d, w + 1, W), S, amask,
                [=](int s, int c) {
                    // head h of state s: its chunks' P.V over their weight sums
                    const size_t b = ((size_t)s * H + (c >> 6)) * XC;
                    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
                    float sum = 0.0f;
                    // the chunks' loads go out together, then the sums
                    float4 p4[CMAX];
                    float ps[CMAX];
#pragma unroll
                    for (int i = 0; i < CMAX; i++)
                        if (i < XC) {
                            p4[i] = ldx4(pvr + (b + i) * 64 + (c & 63));
                            ps[i] = ldx(psr + b + i);
                        }
#pragma unroll
                    for (int i = 0; i < CMAX; i++)
                        if (i < XC) {
                            o.x += p4[i].x; o.y += p4[i].y; o.z += p4[i].z; o.w += p4[i].w;
                            sum += ps[i];
                        }
                    const float inv = 1.0f / sum;
                    return make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
                },
                L,
                [=](int s, int r) {
                    return make_float2(ldx(xr + (size_t)s * d + r) + ldx(sal + (size_t)s * d + r), ldg(cob + r));
                },
                [=](int s, int r, float v, float2 p) { stx(x2w + (size_t)s * d + r, p.x + (v + p.y)); });
        }
        gbar(flags, errw, g);
        // ---- G: LN3, fc1 rows + GELU ----
        {
            const int r0 = split(4 * d, w, W), r1 = split(4 * d, w + 1, W);
            if (r0 < r1) {
                const float *x2r = x2g, *fc1b = ly->fc1b, *lw = ly->ln3w, *lb = ly->ln3b;
                float *hw = hg;
                gemv<TYPE, G>(ly->fc1, r0, r1, S, amask,
                           [&]() __attribute__((always_inline)) {
                               stage_ln(S, d, [=](int s, int c) { return ldx4(x2r + (size_t)s * d + c); }, lw, lb, L,
                                        TYPE != 8);
                           }, L,
                           [=](int, int r) { return make_float2(0.f, ldg(fc1b + r)); },
                           [=](int s, int r, float v, float2 p) { stx(hw + (size_t)s * 4 * d + r, gelu_ref(v + p.y)); });
            }
        }
        gbar(flags, errw, g);
        // ---- H: fc2 rows; x = x2 + (W2.h + b2) ----
        {
            const float *fc2b = ly->fc2b, *hr = hg, *x2r = x2g;
            float *xw = xg;
            gemv_src<TYPE, G>(
                ly->fc2, split(d, w, W), split(d, w + 1, W), S, amask,
                [=](int s, int c) { return ldx4(hr + (size_t)s * 4 * d + c); }, L,
                [=](int s, int r) { return make_float2(ldx(x2r + (size_t)s * d + r), ldg(fc2b + r)); },
                [=](int s, int r, float v, float2 p) { stx(xw + (size_t)s * d + r, p.x + (v + p.y)); });
        }
        gbar(flags, errw, g);
    }
    // ---- final LayerNorm and tied logits rows (decoder.go:817-832) ----
    {
        const int r0 = split(a.V, w, W), r1 = split(a.V, w + 1, W);
        if (r0 < r1) {
            const float *xr = xg, *lw = a.lnw, *lb = a.lnb;
            float *lg = a.logits;
            const int V = a.V;
            gemv<TYPE, G>(a.tok, r0, r1, S, amask,
                       [&]() __attribute__((always_inline)) {
                           stage_ln(S, d, [=](int s, int c) { return ldx4(xr + (size_t)s * d + c); }, lw, lb, L,
                                    TYPE != 8);
                       }, L, nopre,
                       [=](int s, int r, float v, float2) { stg(lg + (size_t)s * V + r, v); });
        }
    }
}

// Launch of the kernel for weight type TYPE; G from the model width.
template <int TYPE>
int launch_type(int grid, const BArgs &a, hipStream_t st) {
    void *args[] = {(void *)&a};
    const void *fn = a.d <= 1024 ? (const void *)k_fwd_batch<TYPE, 32> : (const void *)k_fwd_batch<TYPE, 64>;
    WH_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)LDS_BYTES));
    WH_HIP(hipLaunchCooperativeKernel(fn, dim3(grid), dim3(NT), args, LDS_BYTES, st));
    return WH_OK;
}

}  // namespace batch
}  // namespace wh
