// Persistent decode kernel: whole greedy token steps of one stream in a single
// cooperative launch on gfx950 (internal/model/decoder.go:413-525 loop,
// :745-993 forward, reference-compatible attention mask).
//
// Under the reference mask the self-attention of a step past position 0
// attends KV row 0 only (internal/ml/attention.go:250-256), so its output
// sa_l = Wo_l . V0_l + ob_l does not depend on the step's activations, and the
// q,k,v rows the step adds to the cache are read by nobody within the step.
// Both are computed off the critical path by "side" workgroups while the
// cross-attention runs. One workgroup of 512 threads per CU walks these
// phases; each boundary is a data dependency between workgroups:
//   S   (once per step) embedding; side workgroups: sa_0 rows
//   B1  item workgroups (one per (head, key chunk)): x1 = x_l + sa_l, LN2 and
//       the chunk's share of the head's cross-query rows. Side workgroups:
//       LN1(x_l), q,k,v rows -> KV cache, and the rows of sa_{l+1}.
//   B2  items: the head's q (head-local exchange), scores of the chunk
//       against its K rows (staged in LDS a layer ahead), chunk maximum
//   C   items: head maximum, fast-exp weights, partial sum and P.V; the last
//       chunk of a head to finish combines the head
//   D   cross output rows: x2 = x1 + (Wo_c . attn + ob_c)
//   E   LN3 + fc1 rows + GELU
//   F   fc2 rows: x_{l+1} = x2 + (W2 . h + b2)
//   T   final LN + tied logits rows + repetition penalty + partial argmax;
//       every workgroup reduces the partials and takes the same next token.
//
// Roles of the 8 waves of a workgroup. The vector memory counter of a wave
// retires in order, so a wave that waits for one load waits for every older
// one. Waves 1..7 (compute waves) hold all weight rows: right after the dot
// products of a phase they issue the loads of the next phase's rows, which
// then stream while the flags travel. Wave 0 (communication wave) never has a
// weight load in flight: it polls the flags, loads the exchanged vectors into
// LDS, stores the results the compute waves post in an LDS outbox, retires
// those stores with s_waitcnt and publishes the phase flag. LDS-only work
// (scores) is shared by all waves.
//
// Cross-workgroup data moves through relaxed agent-scope atomic loads and
// stores, which bypass the non-coherent caches. Every wait is bounded: on timeout the
// error word is set, later waits return at once, the token loop stops and the
// host reports a failure.
//
// Addressing: the layer descriptors are copied into LDS once per launch; each
// phase reads the pointers it needs from there into scalar registers
// (readfirstlane) as global-address-space pointers, so weight loads are
// `global_load ... v_offset, s[base]`.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#include "wh_device.h"
#include "wh_internal.h"
#include "wh_mega.h"

namespace wh {
namespace mega {

constexpr int NT = THREADS;
constexpr int NW = WAVES;
constexpr int NC = CWAVES;    // compute waves 1..NC
constexpr int NCT = NC * 64;  // compute threads
constexpr int OUTBOX = 64;    // posted (row, value) pairs per phase
constexpr unsigned SPIN_MAX = 1u << 22;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const uint8_t gu8;
typedef __attribute__((address_space(1))) const u32x4 gu4;
typedef __attribute__((address_space(1))) const uint16_t gu16;
typedef __attribute__((address_space(1))) const uint32_t gu32;
typedef __attribute__((address_space(1))) const float gf;
typedef __attribute__((address_space(1))) const f32x4 gf4;
typedef __attribute__((address_space(1))) float gfw;

__device__ __forceinline__ uint4 ld16(gu8 *p) {
    const u32x4 v = *(gu4 *)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float4 ld16f(gf *p) {
    const f32x4 v = *(gf4 *)p;
    return make_float4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ unsigned ld_u(const unsigned *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_u(unsigned *p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_f(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_f(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// threadIdx.x hidden from loop-invariant code motion. Every per-thread index
// and address below derives from it, so the compiler recomputes them inside
// each phase instead of hoisting them out of the token and layer loops, where
// the offsets of all phases would stay live at once and spill.
__device__ __forceinline__ int tid() {
    int t = (int)threadIdx.x;
    __asm__ volatile("" : "+v"(t));
    return t;
}

// A value that is the same on every lane, kept in a scalar register.
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Compute-wave index 0..NC-1 of this wave, or -1 for the communication wave.
__device__ __forceinline__ int cwave() { return uni(tid() >> 6) - 1; }
__device__ __forceinline__ bool comm() { return uni(tid() >> 6) == 0; }
// Compute-thread index 0..NCT-1 (0 in the communication wave).
__device__ __forceinline__ int ctid() { return max(tid() - 64, 0); }

// A pointer that is the same on every lane, moved to scalar registers and
// typed as global memory.
template <typename G, typename T>
__device__ __forceinline__ G *glob(T *p) {
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (G *)(((uint64_t)hi << 32) | lo);
}

// A matrix as scalar global pointers to its planes (block counts come from d).
struct UView {
    gu8 *qs, *sc, *qh;
};
__device__ __forceinline__ UView uview(const MatView &m) {
    return UView{glob<gu8>(m.qs), glob<gu8>((const uint8_t *)m.sc), glob<gu8>((const uint8_t *)m.qh)};
}

// ---- cross-lane reductions: DPP within 16-lane rows, readlane across rows -------
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
// Sum over each 16-lane row (xor 1, xor 2, half-row mirror, row mirror); every
// lane of the row ends with the same value.
__device__ __forceinline__ float row_sum16(float v) {
    v += dpp<0xB1>(v);
    v += dpp<0x4E>(v);
    v += dpp<0x141>(v);
    v += dpp<0x140>(v);
    return v;
}
__device__ __forceinline__ float row_max16(float v) {
    v = fmaxf(v, dpp<0xB1>(v));
    v = fmaxf(v, dpp<0x4E>(v));
    v = fmaxf(v, dpp<0x141>(v));
    v = fmaxf(v, dpp<0x140>(v));
    return v;
}
__device__ __forceinline__ float lane_f(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
// Sum over the wave in a fixed order, (row0 + row1) + (row2 + row3); uniform.
__device__ __forceinline__ float wave_sum(float v) {
    v = row_sum16(v);
    return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}
__device__ __forceinline__ float wave_max(float v) {
    v = row_max16(v);
    return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

#ifdef WH_MEGA_TRACE
// Diagnostic build only: thread 0 of every workgroup stamps the constant
// 100 MHz clock at each phase's start (point 0), after its wait (1) and before
// its publish (2), for the first TR_STEPS steps of a launch; points 3.. split
// a phase's work. Phase 0 is B2, 6 is T, 7 the step-start phase S.
constexpr int TR_STEPS = 2, TR_MAXL = 33, TR_PTS = 8, TR_MAXW = 256;
#ifdef WH_MEGA_TRACE_CYCLES
#define WH_STAMP() clock64()
#else
#define WH_STAMP() wall_clock64()
#endif
__device__ long long g_trace[TR_STEPS * TR_MAXL * 8 * TR_PTS * TR_MAXW];
#define TRACE(step, l, ph, pt)                                                                                        \
    do {                                                                                                              \
        if ((step) < TR_STEPS && (l) < TR_MAXL && blockIdx.x < TR_MAXW && tid() == 0)                                 \
            g_trace[((((step) * TR_MAXL + (l)) * 8 + (ph)) * TR_PTS + (pt)) * TR_MAXW + blockIdx.x] = WH_STAMP(); \
    } while (0)
// the same stamp from the first compute wave
#define TRACEC(step, l, ph, pt)                                                                                       \
    do {                                                                                                              \
        if ((step) < TR_STEPS && (l) < TR_MAXL && blockIdx.x < TR_MAXW && tid() == 64)                                \
            g_trace[((((step) * TR_MAXL + (l)) * 8 + (ph)) * TR_PTS + (pt)) * TR_MAXW + blockIdx.x] = WH_STAMP(); \
    } while (0)
#else
#define TRACE(step, l, ph, pt) \
    do {                       \
    } while (0)
#define TRACEC(step, l, ph, pt) \
    do {                        \
    } while (0)
#endif

// ---- exchange: {value, phase} pairs ------------------------------------------------
__device__ __forceinline__ void st_pair(uint64_t *p, float v, unsigned g) {
    __hip_atomic_store(p, ((uint64_t)g << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// LDS vectors keep each 32-element block in 36 slots: a lane reading its whole
// block then hits 4 banks no other lane of its 16-lane group uses.
__device__ __forceinline__ int pad(int i) { return i + ((i >> 5) << 2); }

// One wave: wait until the pairs src[first + 64k + lane] (k < K, below n;
// 1 <= n) carry phase >= g; their values are left in v. Every pair is loaded
// up front; later rounds re-read only the pending ones. Lanes past n re-read
// the last pair and do not wait for it. On timeout, or when another workgroup
// gave up, the error word is set and the (stale) values are returned anyway;
// the token loop then stops.
template <int K>
__device__ __forceinline__ void ll_poll(uint64_t (&v)[K], const uint64_t *src, int n, unsigned g, unsigned *err,
                                        int first = 0) {
    typedef __attribute__((address_space(1))) const uint64_t gcu64;
    typedef __attribute__((address_space(1))) const unsigned gcu;
    const int lane = first + (tid() & 63);
    gcu64 *s8 = glob<gcu64>(src);
    gcu *perr = glob<gcu>(err);
#pragma unroll
    for (int k = 0; k < K; k++)
        v[k] = __hip_atomic_load(s8 + min(lane + 64 * k, n - 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    unsigned e = __hip_atomic_load(perr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (unsigned spins = 0;; spins++) {
        bool ok = true;
#pragma unroll
        for (int k = 0; k < K; k++) ok &= (lane + 64 * k >= n) || (unsigned)(v[k] >> 32) >= g;
        if (__all(ok)) break;
        if (e != 0 || spins > SPIN_MAX) {  // another workgroup gave up, or this wait expired
            if ((tid() & 63) == 0) atomicOr(err, 1u);
            break;
        }
#pragma unroll
        for (int k = 0; k < K; k++)
            if ((unsigned)(v[k] >> 32) < g)
                v[k] = __hip_atomic_load(s8 + min(lane + 64 * k, n - 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        e = __hip_atomic_load(perr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// ll_poll, then the values into LDS dst at the same indices (padded when PAD).
template <int K, bool PAD>
__device__ __forceinline__ void ll_load(float *dst, const uint64_t *src, int n, unsigned g, unsigned *err,
                                        int first = 0) {
    uint64_t v[K];
    ll_poll<K>(v, src, n, g, err, first);
    const int lane = first + (tid() & 63);
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int i = lane + 64 * k;
        if (i < n) dst[PAD ? pad(i) : i] = __uint_as_float((uint32_t)v[k]);
    }
}

// ll_load of two vectors in one wait: src1 (n1 pairs of phase g1 from first1,
// into dst1, padded when PAD1) and src2 (n2 pairs of phase g2 from first2, into
// plain dst2). Both are loaded up front, so a vector that is already there costs
// no round trip of its own.
template <int K1, bool PAD1, int K2>
__device__ __forceinline__ void ll_load2(float *dst1, const uint64_t *src1, int n1, unsigned g1, int first1,
                                         float *dst2, const uint64_t *src2, int n2, unsigned g2, int first2,
                                         unsigned *err) {
    typedef __attribute__((address_space(1))) const uint64_t gcu64;
    typedef __attribute__((address_space(1))) const unsigned gcu;
    const int l1 = first1 + (tid() & 63), l2 = first2 + (tid() & 63);
    gcu64 *a8 = glob<gcu64>(src1), *b8 = glob<gcu64>(src2);
    gcu *perr = glob<gcu>(err);
    uint64_t v[K1], u[K2];
#pragma unroll
    for (int k = 0; k < K1; k++)
        v[k] = __hip_atomic_load(a8 + min(l1 + 64 * k, n1 - 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
    for (int k = 0; k < K2; k++)
        u[k] = __hip_atomic_load(b8 + min(l2 + 64 * k, n2 - 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    unsigned e = __hip_atomic_load(perr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (unsigned spins = 0;; spins++) {
        bool ok = true;
#pragma unroll
        for (int k = 0; k < K1; k++) ok &= (l1 + 64 * k >= n1) || (unsigned)(v[k] >> 32) >= g1;
#pragma unroll
        for (int k = 0; k < K2; k++) ok &= (l2 + 64 * k >= n2) || (unsigned)(u[k] >> 32) >= g2;
        if (__all(ok)) break;
        if (e != 0 || spins > SPIN_MAX) {
            if ((tid() & 63) == 0) atomicOr(err, 1u);
            break;
        }
#pragma unroll
        for (int k = 0; k < K1; k++)
            if ((unsigned)(v[k] >> 32) < g1)
                v[k] = __hip_atomic_load(a8 + min(l1 + 64 * k, n1 - 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int k = 0; k < K2; k++)
            if ((unsigned)(u[k] >> 32) < g2)
                u[k] = __hip_atomic_load(b8 + min(l2 + 64 * k, n2 - 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        e = __hip_atomic_load(perr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int k = 0; k < K1; k++) {
        const int i = l1 + 64 * k;
        if (i < n1) dst1[PAD1 ? pad(i) : i] = __uint_as_float((uint32_t)v[k]);
    }
#pragma unroll
    for (int k = 0; k < K2; k++) {
        const int i = l2 + 64 * k;
        if (i < n2) dst2[i] = __uint_as_float((uint32_t)u[k]);
    }
}

// LayerNorm parameters of one wave's elements lane + 64k (k < K).
template <int K>
struct LnW {
    float w[K], b[K];
};
template <int K>
__device__ __forceinline__ void ln_params(LnW<K> &p, gf *w, gf *b, int n) {
    const int lane = tid() & 63;
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int i = min(lane + 64 * k, n - 1);
        p.w[k] = w[i];
        p.b[k] = b[i];
    }
}

// Sum of v[0..K) as a balanced binary tree (a fixed order, short dependency
// chains).
template <int K>
__device__ __forceinline__ float tree_sum(const float (&v)[K]) {
    float t[K];
#pragma unroll
    for (int k = 0; k < K; k++) t[k] = v[k];
#pragma unroll
    for (int w = 1; w < K; w *= 2) {
#pragma unroll
        for (int k = 0; k + w < K; k += 2 * w) t[k] += t[k + w];
    }
    return t[0];
}

// LayerNorm (internal/ml/ops.go:153-202) by one wave of the n values
// x[k] = element lane + 64k, into padded LDS xo: the mean, then the mean of
// squared deviations, sqrt in float64, each element w * (x - mean) * (1/sd) + b
// (one reciprocal instead of a division per element: they differ by at most
// an ulp). No barrier: the sums are wave reductions.
template <int K>
__device__ __forceinline__ void ln_wave(const float (&x)[K], int n, const LnW<K> &p, float *xo) {
    const int lane = tid() & 63;
    float t[K];
#pragma unroll
    for (int k = 0; k < K; k++) t[k] = (lane + 64 * k < n) ? x[k] : 0.0f;
    const float mean = wave_sum(tree_sum<K>(t)) / (float)n;
#pragma unroll
    for (int k = 0; k < K; k++) {
        const float u = x[k] - mean;
        t[k] = (lane + 64 * k < n) ? u * u : 0.0f;
    }
    const float var = wave_sum(tree_sum<K>(t)) / (float)n;
    const float rsd = 1.0f / (float)sqrt((double)(var + 1e-5f));
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int i = lane + 64 * k;
        if (i < n) xo[pad(i)] = p.w[k] * (x[k] - mean) * rsd + p.b[k];
    }
}

// Communication wave: wait for the exchanged vector src (n pairs of phase g),
// add the plain LDS vector add when ADD (the residual x + sa), LayerNorm it
// into padded LDS xo.
template <int K, bool ADD>
__device__ __forceinline__ void ll_load_ln(float *xo, const uint64_t *src, int n, unsigned g, unsigned *err,
                                           const LnW<K> &p, const float *add) {
    uint64_t v[K];
    ll_poll<K>(v, src, n, g, err);
    const int lane = tid() & 63;
    float x[K];
#pragma unroll
    for (int k = 0; k < K; k++) {
        x[k] = __uint_as_float((uint32_t)v[k]);
        if (ADD) x[k] += add[min(lane + 64 * k, n - 1)];
    }
    ln_wave<K>(x, n, p, xo);
}

// ll_load_ln with the LayerNorm weight and bias read from LDS (wl, bl [n]).
template <int K>
__device__ __forceinline__ void ll_load_ln_lds(float *xo, const uint64_t *src, int n, unsigned g, unsigned *err,
                                               const float *wl, const float *bl) {
    uint64_t v[K];
    ll_poll<K>(v, src, n, g, err);
    const int lane = tid() & 63;
    float x[K], t[K];
#pragma unroll
    for (int k = 0; k < K; k++) {
        x[k] = __uint_as_float((uint32_t)v[k]);
        t[k] = (lane + 64 * k < n) ? x[k] : 0.0f;
    }
    const float mean = wave_sum(tree_sum<K>(t)) / (float)n;
#pragma unroll
    for (int k = 0; k < K; k++) {
        const float u = x[k] - mean;
        t[k] = (lane + 64 * k < n) ? u * u : 0.0f;
    }
    const float var = wave_sum(tree_sum<K>(t)) / (float)n;
    const float rsd = 1.0f / (float)sqrt((double)(var + 1e-5f));
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int i = lane + 64 * k;
        if (i < n) xo[pad(i)] = wl[i] * (x[k] - mean) * rsd + bl[i];
    }
}

// ---- LayerNorm folded into the rows that read it --------------------------------
// For a row W of the next matrix, W·LN(x) = rsd*(W·(w*x) - mean*(W·w)) + W·b:
// the communication wave stores w*x into the padded LDS vector as soon as x has
// arrived, the compute waves start their dots on it, and the communication wave
// computes mean and rsd while they run; the per-row constants W·w and W·b (+
// the row bias) come from the host.

// LayerNorm weights of one wave's elements lane + 64k.
template <int K>
__device__ __forceinline__ void ln_gain(float (&w)[K], gf *g, int n) {
    const int lane = tid() & 63;
#pragma unroll
    for (int k = 0; k < K; k++) w[k] = g[min(lane + 64 * k, n - 1)];
}

// x[k] (element lane + 64k) into padded LDS xo as w[k] * x[k].
template <int K>
__device__ __forceinline__ void store_scaled(const float (&x)[K], const float (&w)[K], int n, float *xo) {
    const int lane = tid() & 63;
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int i = lane + 64 * k;
        if (i < n) xo[pad(i)] = w[k] * x[k];
    }
}

// Communication wave: wait for the exchanged vector src (n pairs of phase g),
// plus the plain LDS vector add when ADD, into x (kept for ln_stats), and store w*x.
template <int K, bool ADD>
__device__ __forceinline__ void ll_load_scaled(float (&x)[K], float *xo, const uint64_t *src, int n, unsigned g,
                                               unsigned *err, const float (&w)[K], const float *add) {
    uint64_t v[K];
    ll_poll<K>(v, src, n, g, err);
    const int lane = tid() & 63;
#pragma unroll
    for (int k = 0; k < K; k++) {
        x[k] = __uint_as_float((uint32_t)v[k]);
        if (ADD) x[k] += add[min(lane + 64 * k, n - 1)];
    }
    store_scaled<K>(x, w, n, xo);
}

// Mean and 1/sd of the n values x[k] = element lane + 64k, in two passes as the
// reference computes them (internal/ml/ops.go:166-193): the mean, then the mean
// of squared deviations, sqrt in float64. A one-pass E[x^2] - mean^2 loses the
// variance to cancellation once |mean| is ~100x the spread. The communication
// wave computes them while the compute waves run the folded dots.
template <int K>
__device__ __forceinline__ void ln_stats(const float (&x)[K], int n, float &mean, float &rsd) {
    const int lane = tid() & 63;
    float t[K];
#pragma unroll
    for (int k = 0; k < K; k++) t[k] = (lane + 64 * k < n) ? x[k] : 0.0f;
    mean = wave_sum(tree_sum<K>(t)) / (float)n;
#pragma unroll
    for (int k = 0; k < K; k++) {
        const float u = x[k] - mean;
        t[k] = (lane + 64 * k < n) ? u * u : 0.0f;
    }
    const float var = wave_sum(tree_sum<K>(t)) / (float)n;
    rsd = 1.0f / (float)sqrt((double)(var + 1e-5f));
}

// A folded row's value from its dot with w*x.
__device__ __forceinline__ float ln_fold(float dot, float mean, float rsd, float c, float e) {
    return rsd * (dot - mean * c) + e;
}

// ---- outbox: compute lanes post (row, value); the communication wave stores ----
// Lane k < K of compute wave c posts into slot c*K + k; r < 0 posts nothing.
template <int K>
__device__ __forceinline__ void post(int *obi, float *obv, int r, float v) {
    static_assert(NC * K <= OUTBOX, "outbox too small");
    const int lane = tid() & 63, cw = cwave();
    if (cw >= 0 && lane < K) {
        obi[cw * K + lane] = r;
        obv[cw * K + lane] = v;
    }
}
// Communication wave only, after a barrier that follows the posts: store the
// posted values as pairs of phase g into dst. Nothing waits for the stores:
// readers poll the pairs.
template <int K>
__device__ __forceinline__ void flush(const int *obi, const float *obv, uint64_t *dst, unsigned g) {
    const int t = tid() & 63;
    if (t < NC * K) {
        const int r = obi[t];
        if (r >= 0) st_pair(&dst[r], obv[t], g);
    }
}

// ---- weight rows prefetched into registers ----------------------------------------
// Rows [r0, r1) of a workgroup; compute wave c takes rows r0+c, r0+c+NC, ...;
// lane l takes blocks l, l+64, ... of each row (PASSES passes). Slot s holds
// row k = s / PASSES of this wave and pass p = s % PASSES.
template <int TYPE, int MAXS>
struct Pre {
    uint4 a[MAXS];
    uint4 b[MAXS];  // second 16 bytes of a Q8_0 block
    uint32_t s[MAXS];
    uint32_t h[MAXS];
};

// Byte offsets stay 32-bit (the host checks every plane is below 4 GiB).
template <int TYPE>
__device__ __forceinline__ void load_blk(const UView &m, unsigned blk, uint4 &a, uint4 &b, uint32_t &s, uint32_t &h) {
    if constexpr (TYPE == 8) {
        a = ld16(m.qs + blk * 32u);
        b = ld16(m.qs + blk * 32u + 16u);
        s = *(gu16 *)(m.sc + blk * 2u);
    } else {
        a = ld16(m.qs + blk * 16u);
        if constexpr (TYPE == 3 || TYPE == 7) s = *(gu32 *)(m.sc + blk * 4u);
        else s = *(gu16 *)(m.sc + blk * 2u);
        if constexpr (TYPE == 6 || TYPE == 7) h = *(gu32 *)(m.qh + blk * 4u);
    }
}

// Slots [0, NS) load; slots [NS, MAXS) and every slot of the communication
// wave hold zeros. Loads are unconditional: a slot past the range re-reads the
// last valid row or block (row 0 for an empty range; a cache hit) and the dot
// products drop it, so no slot is ever undefined (undefined slots become
// loop-carried live ranges and spill) and no branch surrounds the loads.
template <int TYPE, int MAXS, int PASSES, int NS = MAXS>
__device__ __forceinline__ void prefetch(Pre<TYPE, MAXS> &P, const UView &m, int nb, int r0, int r1) {
    const int lane = tid() & 63, cw = cwave();
#pragma unroll
    for (int s = 0; s < MAXS; s++) {
        if (s >= NS || cw < 0) {
            P.a[s] = make_uint4(0u, 0u, 0u, 0u);
            P.b[s] = make_uint4(0u, 0u, 0u, 0u);
            P.s[s] = 0u;
            P.h[s] = 0u;
        } else {
            const int r = max(min(r0 + cw + NC * (s / PASSES), r1 - 1), 0);
            const int b = min(lane + 64 * (s % PASSES), nb - 1);
            load_blk<TYPE>(m, (unsigned)r * (unsigned)nb + (unsigned)b, P.a[s], P.b[s], P.s[s], P.h[s]);
        }
    }
}

// f16 scale to f32 by the hardware conversion (exact for every finite value).
__device__ __forceinline__ float hf(uint32_t bits) { return (float)__builtin_bit_cast(_Float16, (uint16_t)bits); }

// dot of one prefetched block with 32 activations in registers
template <int TYPE>
__device__ __forceinline__ float block_dot(const uint4 &a, const uint4 &b, uint32_t s, uint32_t h, const float *x) {
    float acc = 0.0f;
    if constexpr (TYPE == 8) {
        // one convert and one fused multiply-add per weight, in two chains (even and odd words)
        const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        float acc1 = 0.0f;
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const int v = (int)w[t];
            float &c = (t & 1) ? acc1 : acc;
            c = __builtin_fmaf((float)((v << 24) >> 24), x[4 * t], c);
            c = __builtin_fmaf((float)((v << 16) >> 24), x[4 * t + 1], c);
            c = __builtin_fmaf((float)((v << 8) >> 24), x[4 * t + 2], c);
            c = __builtin_fmaf((float)(v >> 24), x[4 * t + 3], c);
        }
        return hf(s) * (acc + acc1);
    } else {
        const uint32_t w[4] = {a.x, a.y, a.z, a.w};
        const float off = (TYPE == 2) ? 8.0f : (TYPE == 6 ? 16.0f : 0.0f);
        float sx = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; t++) {
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t byte = (w[t] >> (8 * k)) & 0xFFu;
                uint32_t lo = byte & 0xFu, hi = byte >> 4;
                const int e0 = 8 * t + 2 * k;
                if constexpr (TYPE == 6 || TYPE == 7) {
                    lo |= ((h >> e0) & 1u) << 4;
                    hi |= ((h >> (e0 + 1)) & 1u) << 4;
                }
                acc += ((float)lo - off) * x[e0] + ((float)hi - off) * x[e0 + 1];
                if constexpr (TYPE == 3 || TYPE == 7) sx += x[e0] + x[e0 + 1];
            }
        }
        if constexpr (TYPE == 3 || TYPE == 7) return hf(s & 0xFFFFu) * acc + hf(s >> 16) * sx;
        else return hf(s) * acc;
    }
}

// Activation block b of a padded LDS vector (16-byte aligned) into registers.
__device__ __forceinline__ void lds_block(const float *xs, int b, float (&xr)[32]) {
    const float4 *x4 = (const float4 *)(xs + b * 36);
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const float4 v = x4[j];
        xr[4 * j] = v.x;
        xr[4 * j + 1] = v.y;
        xr[4 * j + 2] = v.z;
        xr[4 * j + 3] = v.w;
    }
}

// A prefetched slot made opaque right before its use: otherwise the compiler
// moves the first operations on it (the f16 scale conversion, byte extracts)
// up into the prefetch, right behind the loads, and has to wait for each load
// there, which makes the prefetch synchronous.
template <int TYPE>
__device__ __forceinline__ void opaque_slot(uint4 &a, uint4 &b, uint32_t &s, uint32_t &h) {
    __asm__ volatile("" : "+v"(a.x), "+v"(a.y), "+v"(a.z), "+v"(a.w), "+v"(s));
    if constexpr (TYPE == 8) __asm__ volatile("" : "+v"(b.x), "+v"(b.y), "+v"(b.z), "+v"(b.w));
    if constexpr (TYPE == 6 || TYPE == 7) __asm__ volatile("" : "+v"(h));
}

// Row dots of the prefetched slots: out[k] (same on every lane) is the dot of
// row r0 + cw + NC*k (cw = cwave()) with the padded LDS vector xs of nb
// blocks. Lanes past the last block and rows past r1 compute on duplicate
// data and add zero; the communication wave returns zeros.
template <int TYPE, int MAXS, int PASSES, int NK = MAXS / PASSES>
__device__ __forceinline__ void row_dots(Pre<TYPE, MAXS> &P, int nb, int r0, int r1, const float *xs,
                                         float (&out)[MAXS / PASSES]) {
    const int lane = tid() & 63, cw = cwave();
    constexpr int K = MAXS / PASSES;
#pragma unroll
    for (int k = 0; k < K; k++) out[k] = 0.0f;
    if (cw < 0) return;
#pragma unroll
    for (int p = 0; p < PASSES; p++) {
        const int b = lane + 64 * p;
        float xr[32];
        lds_block(xs, min(b, nb - 1), xr);
#pragma unroll
        for (int k = 0; k < NK; k++) {  // rows past NK per wave are known empty
            const int s = k * PASSES + p;
            const int r = r0 + cw + NC * k;
            // in place: the slot is dead after its dot, so no copy is made
            opaque_slot<TYPE>(P.a[s], P.b[s], P.s[s], P.h[s]);
            const float v = block_dot<TYPE>(P.a[s], P.b[s], P.s[s], P.h[s], xr);
            out[k] += (r < r1 && b < nb) ? v : 0.0f;
        }
    }
#pragma unroll
    for (int k = 0; k < NK; k++) out[k] = wave_sum(out[k]);
}

// out[lane] for lane < K (the row a lane finishes in an epilogue). out[] is
// wave-uniform, so each value is written into its lane with v_writelane; a
// select chain on the lane index is turned into a private (scratch) array.
template <int K>
__device__ __forceinline__ float pick(const float (&out)[K]) {
    float v = 0.0f;
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int s = uni(__builtin_bit_cast(int, out[k]));
        __asm__ volatile("v_writelane_b32 %0, %1, %2" : "+v"(v) : "s"(s), "i"(k));
    }
    return v;
}

// Per-lane bias of row r0 + cw + NC*lane (lane < K), clamped into [r0, r1);
// the communication wave loads nothing.
template <int K>
__device__ __forceinline__ float lane_bias(gf *bias, int r0, int r1) {
    const int lane = tid() & 63, cw = cwave();
    if (cw < 0) return 0.0f;
    return bias[max(min(r0 + cw + NC * min(lane, K - 1), r1 - 1), 0)];
}

// Row finished by this lane in an epilogue (lane < K of a compute wave), or -1.
template <int K>
__device__ __forceinline__ int lane_row(int r0, int r1) {
    const int lane = tid() & 63, cw = cwave();
    const int r = r0 + cw + NC * lane;
    return (cw >= 0 && lane < K && r < r1) ? r : -1;
}

// ---- flat split of a workgroup's rows ---------------------------------------------
// The (row, block) items of rows [r0, r0 + nrows), nb blocks each, in row-major
// order: item i is block r0*nb + i of the matrix, whose rows are contiguous.
// Compute wave c < A takes items [c*N/A, (c+1)*N/A) (N = nrows*nb, A =
// min(NC, 2 nrows) waves, so a wave holds at least half a row) and its lane l
// the items i0 + l + 64p, p < P: every compute wave gets the same number of
// blocks whatever the row count (a row per wave leaves lanes idle when nb is not
// a multiple of 64 and loads some SIMDs twice as much as others), and a wave's
// loads are consecutive blocks. A wave sums its items by row (at most RS rows,
// counted from the row of its first item); a row can straddle two or three
// waves, and the communication wave adds its wave sums in wave order.
__device__ __forceinline__ int flat_i0(int c, int nrows, int nb) {
    const int A = min(NC, max(1, 2 * nrows)), n = nrows * nb;
    return c >= A ? n : c * n / A;
}

// Per-launch constants of a flat split for this lane. Compute lanes: pass p's
// block within its row (bits 12p..12p+7) and wave-relative row (bits
// 12p+8..12p+11; 15 marks a lane past the wave's items), p < 2. Communication
// lanes t < nrows: the outbox slots of row t's wave sums in wave order (bits
// 0-7, 8-15, 16-23) and their count (bits 24-25). The host checks the limits
// (nb <= 255, at most 64P items and RS rows per wave, 3 waves per row).
template <int P, int RS>
__device__ __forceinline__ uint32_t flat_info(int nb, int nrows) {
    static_assert(P <= 2 && RS <= 15 && NC * RS <= OUTBOX, "flat split limits");
    const int lane = tid() & 63, cw = cwave();
    const int n = nrows * nb;
    uint32_t r = 0;
    if (n <= 0) return cw >= 0 ? 0xF00F00u : 0u;
    if (cw >= 0) {
        const int i0 = flat_i0(cw, nrows, nb), i1 = flat_i0(cw + 1, nrows, nb), ra = i0 / nb;
        for (int p = 0; p < P; p++) {
            const int i = i0 + lane + 64 * p;
            const int ic = min(i, max(i1 - 1, 0));
            const int row = ic / nb;
            const uint32_t rel = i < i1 ? (uint32_t)(row - ra) : 15u;
            r |= ((uint32_t)(ic - row * nb) | rel << 8) << (12 * p);
        }
        if (P < 2) r |= 0xF00u << 12;
    } else if (lane < nrows) {
        uint32_t cnt = 0;
        for (int c = 0; c < NC; c++) {
            const int i0 = flat_i0(c, nrows, nb), i1 = flat_i0(c + 1, nrows, nb);
            if (i1 <= i0) continue;
            const int ra = i0 / nb, rb = (i1 - 1) / nb;
            if (lane >= ra && lane <= rb && cnt < 3) {
                r |= (uint32_t)(c * RS + lane - ra) << (8 * cnt);
                cnt++;
            }
        }
        r |= cnt << 24;
    }
    return r;
}

// Items of this compute lane into its P slots (zeros when !on and on the
// communication wave). Past the wave's items a slot re-reads its last item
// (a cache hit); with no items at all, block 0.
template <int TYPE, int P>
__device__ __forceinline__ void flat_prefetch(Pre<TYPE, P> &F, const UView &m, int nb, int r0, int nrows, bool on) {
    const int lane = tid() & 63, cw = cwave();
    const int n = nrows * nb, c = max(cw, 0);
    const int i0 = flat_i0(c, nrows, nb), last = max(flat_i0(c + 1, nrows, nb) - 1, 0);
    const unsigned base = n > 0 ? (unsigned)r0 * (unsigned)nb : 0u;
#pragma unroll
    for (int p = 0; p < P; p++) {
        if (cw < 0 || !on) {
            F.a[p] = make_uint4(0u, 0u, 0u, 0u);
            F.b[p] = make_uint4(0u, 0u, 0u, 0u);
            F.s[p] = 0u;
            F.h[p] = 0u;
        } else {
            load_blk<TYPE>(m, base + (unsigned)min(i0 + lane + 64 * p, last), F.a[p], F.b[p], F.s[p], F.h[p]);
        }
    }
}

// Wave sums by row of this compute wave's items: out[j] (same on every lane) is
// the sum over its items of wave-relative row j. The communication wave returns zeros.
template <int TYPE, int P, int RS>
__device__ __forceinline__ void flat_dots(Pre<TYPE, P> &F, uint32_t info, const float *xs, float (&out)[RS]) {
#pragma unroll
    for (int j = 0; j < RS; j++) out[j] = 0.0f;
    if (cwave() < 0) return;
    float acc[RS];
#pragma unroll
    for (int j = 0; j < RS; j++) acc[j] = 0.0f;
#pragma unroll
    for (int p = 0; p < P; p++) {
        const uint32_t f = info >> (12 * p);
        const uint32_t rel = (f >> 8) & 0xFu;
        float xr[32];
        lds_block(xs, (int)(f & 0xFFu), xr);
        opaque_slot<TYPE>(F.a[p], F.b[p], F.s[p], F.h[p]);
        const float v = block_dot<TYPE>(F.a[p], F.b[p], F.s[p], F.h[p], xr);
#pragma unroll
        for (int j = 0; j < RS; j++) acc[j] += rel == (uint32_t)j ? v : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < RS; j++) out[j] = wave_sum(acc[j]);
}

// Compute wave c posts its row sums into outbox slots c*RS + j.
template <int RS>
__device__ __forceinline__ void flat_post(float *obv, const float (&out)[RS]) {
    const int lane = tid() & 63, cw = cwave();
    const float v = pick<RS>(out);
    if (cw >= 0 && lane < RS) obv[cw * RS + lane] = v;
}

// Communication lane t < nrows, after the barrier that follows the posts: row t's sum.
__device__ __forceinline__ float flat_sum(const float *obv, uint32_t slots) {
    const uint32_t n = slots >> 24;
    float s = obv[slots & 0xFFu];
    if (n > 1) s += obv[(slots >> 8) & 0xFFu];
    if (n > 2) s += obv[(slots >> 16) & 0xFFu];
    return s;
}

// Bias of row r0 + lane on the communication wave (clamped into [r0, r1)); zero elsewhere.
__device__ __forceinline__ float comm_bias(gf *bias, int r0, int r1) {
    const int lane = tid() & 63;
    return (comm() && r1 > r0) ? bias[min(r0 + lane, r1 - 1)] : 0.0f;
}

// The tanh-form GELU of internal/ml/ops.go:102-122 with tanh in float32 (the
// reference takes tanh in float64; the two differ by about one float32 ulp of
// 1 + tanh, far inside the logits tolerance). The float64 tanh is a long
// dependent chain on the critical path of every layer.
__device__ __forceinline__ float gelu_f32(float x) {
#pragma clang fp contract(off)
    const float k = 0.7978845608028654f;
    const float inner = k * (x + 0.044715f * x * x * x);
    return x * 0.5f * (1.0f + tanhf(inner));
}

__device__ __forceinline__ void better(float v, int i, float &bv, int &bi) {
    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
}

// Logits rows of one chunk (<= NC*TS rows) with penalty and running argmax.
// pen[r - rv0] is the window count of row r. The raw logit of the EOT row is
// posted to LDS (*eotv) for the communication wave to publish.
template <int TYPE>
__device__ __forceinline__ void logits_chunk(const MegaArgs &a, Pre<TYPE, TS> &P, int nb, int base, int end,
                                             const float *xn, const int *pen, int rv0, float &bv, int &bi,
                                             float &bv2, int &bi2, float *eotv) {
    const int lane = tid() & 63, cw = cwave();
    float out[TS];
    row_dots<TYPE, TS, 1>(P, nb, base, end, xn, out);
    if (cw < 0) return;
#pragma unroll
    for (int k = 0; k < TS; k++) {
        const int r = base + cw + NC * k;
        if (r < end) {
            float v = out[k];
            if (a.out_logits && lane == 0) a.out_logits[r] = v;
            const int cnt = pen[r - rv0];
            if (cnt > 0) v -= 2.0f * (float)cnt;
            const float s = v * a.inv_temp;
            better(s, r, bv, bi);
            if (r != a.eot) better(s, r, bv2, bi2);
            if (r == a.eot && lane == 0) *eotv = v;
        }
    }
}

// LDS layout (floats): layer descriptors, then the vectors of k_decode.
__host__ __device__ inline int layer_floats(int L) { return (int)((L * sizeof(MegaLayer) + 15) / 16 * 4); }
__host__ __device__ inline int pen_floats(int V, int W) { return ((V + W - 1) / W + 3) / 4 * 4; }

// Rows of phase B1 of one layer. Item workgroups load their share of the
// head's cross-query rows and the query bias a phase ahead (loop carried).
// Side workgroups (decoder.go:780-790 under the reference mask) load their q,k,v
// rows with the v bias and the next layer's self-attention output rows with
// their bias and that layer's V0 (3 elements per compute thread) only once x_l
// has arrived: their work has slack, and a prefetch at the end of F would
// contend with the exchange polls for the memory pipeline. The communication
// wave loads the LN parameters.
template <int TYPE>
struct B1Item {
    Pre<TYPE, FQ> pc;
    float qc, qe;  // communication lanes: their row's folded LN2 constants (bias in qe)
};
template <int TYPE>
struct B1Side {
    Pre<TYPE, SQ> pq;
    Pre<TYPE, SO> po;
    float qb, ob;
    float v0r[3];
};

template <int TYPE>
__device__ __forceinline__ void v0_load(float (&v0r)[3], const MegaArgs &a, const MegaLayer &Ly) {
    gf *kv = glob<gf>(Ly.kv) + (size_t)a.H * a.ctx * 64;  // V plane, row 0 of each head
    const int c = ctid();
    const bool cw = cwave() >= 0;
#pragma unroll
    for (int j = 0; j < 3; j++) {
        const int i = min(c + NCT * j, a.d - 1);
        v0r[j] = cw ? kv[(size_t)(i / 64) * a.ctx * 64 + (i % 64)] : 0.0f;
    }
}
__device__ __forceinline__ void v0_store(const float (&v0r)[3], float *v0, int d) {
    const int c = ctid();
    if (cwave() < 0) return;
#pragma unroll
    for (int j = 0; j < 3; j++)
        if (c + NCT * j < d) v0[pad(c + NCT * j)] = v0r[j];
}

// Item rows of B1 (zeros for side workgroups).
template <int TYPE>
__device__ __forceinline__ void b1_item_prefetch(B1Item<TYPE> &S, const MegaLayer *ls, int l, bool item, int cq0,
                                                 int cq1, int nbd) {
    const MegaLayer &Ly = ls[l];
    S.qc = item ? comm_bias(glob<gf>(Ly.cqc), cq0, cq1) : 0.0f;
    S.qe = item ? comm_bias(glob<gf>(Ly.cqe), cq0, cq1) : 0.0f;
    flat_prefetch<TYPE, FQ>(S.pc, uview(Ly.cq), nbd, cq0, cq1 - cq0, item);
}

template <int TYPE>
__device__ __forceinline__ void b1_side_load(B1Side<TYPE> &S, const MegaArgs &a, const MegaLayer *ls, int l, int q0,
                                             int q1, int o0, int o1, int nbd) {
    const MegaLayer &Ly = ls[l];
    {
        // v rows take the v bias; k rows have none; q rows are not used
        const int lane = tid() & 63, cw = max(cwave(), 0);
        const int r = max(min(q0 + cw + NC * min(lane, SQ - 1), q1 - 1), 0);
        S.qb = cwave() >= 0 ? glob<gf>(Ly.svb)[max(r - 2 * a.d, 0)] : 0.0f;
    }
    // the last layer has no next layer: its own rows are loaded and not used
    const MegaLayer &Ln = ls[min(l + 1, a.L - 1)];
    S.ob = lane_bias<SO>(glob<gf>(Ln.sob), o0, o1);
    v0_load<TYPE>(S.v0r, a, Ln);
    prefetch<TYPE, SQ, 1>(S.pq, uview(Ly.sqkv), nbd, q0, q1);
    prefetch<TYPE, SO, 1>(S.po, uview(Ln.so), nbd, o0, o1);
}

// Direct global->LDS load of 16 bytes per lane (lane l writes lds + 16 l bytes;
// lds wave-uniform), in inline assembly: for the builtin form the compiler makes
// every later LDS read of the wave wait for all of its outstanding loads, which
// would hold the next phase's dots until the V rows and weight rows issued with
// K have arrived. Here the issuing wave waits explicitly (k_wait) before the
// barrier that precedes the first read. M0 is otherwise unused by this kernel.
__device__ __forceinline__ void dma16(const float *g, float *lds) {
    const uint32_t m0v = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) float *)lds;
    __asm__ volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(m0v)
                     : "memory", "m0");
}

// Stage K rows [t0, t1) of head ih (a [enc_len][64] block of crossK) into LDS
// kst in the same layout, 1 KiB per instruction, by the compute waves; issued
// before the next phase's weight rows, so the first wait for those rows also
// covers K.
__device__ __forceinline__ void stage_k(const float *crossK, int enc_len, int ih, int t0, int t1, float *kst) {
    const int cw = cwave(), lane = tid() & 63;
    if (cw < 0) return;
    const float *src = crossK + ((size_t)ih * enc_len + t0) * 64;
    const int nvec = (t1 - t0) * 16;  // 16-byte vectors
    const int nblk = (nvec + 63) / 64;
    for (int b = cw; b < nblk; b += NC) {
        const int v = b * 64 + lane;
        if (v < nvec) dma16(src + 4 * v, kst + b * 256);
    }
}
// The compute waves' wait for their staged K rows (before the barrier that
// precedes the first read).
__device__ __forceinline__ void k_wait() {
    if (!comm()) __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// Rows [t0, t1) of head ih of a [enc_len][64] block (cross K or V of one
// layer) into registers of the compute waves: compute thread c holds elements
// 4(c & 15) .. +3 of keys t0 + 28 j + (c >> 4), j < PVK. Keys past the chunk
// re-read its last key; the communication wave holds zeros.
__device__ __forceinline__ void chunk_rows(float4 (&r)[PVK], const float *base, int enc_len, int ih, int t0, int t1) {
    gf *src = glob<gf>(base) + ((size_t)ih * enc_len + t0) * 64;
    const unsigned c = (unsigned)ctid(), n = (unsigned)(t1 - t0);
    const bool cwv = cwave() >= 0;
#pragma unroll
    for (int j = 0; j < PVK; j++) {
        const unsigned t = min((unsigned)j * (NCT / 16) + (c >> 4), n - 1u);
        r[j] = cwv ? ld16f(src + t * 64u + 4u * (c & 15u)) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

// An item's V rows for C (chunk_rows), zeros for other workgroups.
__device__ __forceinline__ void v_rows(float4 (&r)[PVK], bool item, const float *base, int enc_len, int ih, int t0,
                                       int t1) {
    if (item) {
        chunk_rows(r, base, enc_len, ih, t0, t1);
    } else {
#pragma unroll
        for (int j = 0; j < PVK; j++) r[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

template <int TYPE>
__global__ __launch_bounds__(NT, 1) void k_decode(MegaArgs a) {
    extern __shared__ __align__(16) float lds[];
    const int d = a.d, H = a.H, L = a.L, W = gridDim.x, w = blockIdx.x;
    const int nbd = d / 32, nbf = 4 * d / 32;  // d is a multiple of 64
    const int d36 = nbd * 36;
    MegaLayer *ls = (MegaLayer *)lds;     // [L] layer descriptors
    float *xs = lds + layer_floats(L);    // [d36] x_l, later x2 (padded)
    float *v0 = xs + d36;                 // [d36] V0 of the next layer (side workgroups)
    float *xn = v0 + d36;                 // [4 d36] normalised / exchanged vectors (padded)
    float *sav = xn + 4 * d36;            // [d] sa_l (plain)
    float *xl_own = sav + d;              // [64] own rows of x_l
    float *x2_own = xl_own + 64;          // [64] own rows of x2
    float *red = x2_own + 64;             // [64]
    float *qh = red + 64;                 // [64] q of this workgroup's head
    float *obv = qh + 64;                 // [OUTBOX] posted values
    int *obi = (int *)(obv + OUTBOX);     // [OUTBOX] posted rows
    float *xp = (float *)(obi + OUTBOX);  // [64 * XT] a head's chunk sums (leader), argmax partials
    int *hl = (int *)(xp + 64 * XT);      // [128] the last 128 tokens of the history, by position mod 128
    float *sc = (float *)(hl + 128);      // [SC_FLOATS] scores of this workgroup's chunk
    int *pen = (int *)(sc + SC_FLOATS);   // [pen_floats] window counts of this workgroup's vocabulary rows
    float *kst = (float *)pen + pen_floats(a.V, gridDim.x);  // [chunk_len * 64] K rows of this item's chunk
    uint32_t *fil = (uint32_t *)(kst + a.chunk_len * 64);     // [3][NT] flat-split constants by thread
    float *lnf = (float *)(fil + 3 * NT);                      // [2][d] final LayerNorm weight, bias
    __shared__ float eotv;
    __shared__ int eotf;

    {
        const uint32_t *src = (const uint32_t *)a.layers;
        uint32_t *dst = (uint32_t *)ls;
        const int nw = L * (int)(sizeof(MegaLayer) / 4);
        for (int i = tid(); i < nw; i += NT) dst[i] = src[i];
        // the history the host wrote before the launch; later tokens are appended here
        for (int i = tid(); i < 128; i += NT) {
            const int p = a.len0 - 128 + i;
            if (p >= 0) hl[p & 127] = a.hist[p];
        }
        __syncthreads();
    }
    const Role &rl = a.roles[w];
    const int item = uni(rl.item), q0 = uni(rl.q0), q1 = uni(rl.q1), o0 = uni(rl.o0), o1 = uni(rl.o1);
    const bool has_item = item >= 0;
    const int ih = has_item ? item / a.C : 0, ic = has_item ? item % a.C : 0;
    const int t0 = ic * a.chunk_len, t1 = min(t0 + a.chunk_len, a.enc_len);
    // this item's share of its head's cross-query rows
    const int cq0 = ih * 64 + ic * 64 / a.C, cq1 = ih * 64 + (ic + 1) * 64 / a.C;
    const int rd0 = (int)((long)w * d / W), rd1 = (int)((long)(w + 1) * d / W);
    const int rf0 = (int)((long)w * 4 * d / W), rf1 = (int)((long)(w + 1) * 4 * d / W);
    const int rv0 = (int)((long)w * a.V / W), rv1 = (int)((long)(w + 1) * a.V / W);
    // flat splits of the cross-query (items), fc1 and fc2 rows
    // (kept in LDS: registers are short in the logits phase)
    fil[tid()] = flat_info<FQ, RQ>(nbd, has_item ? cq1 - cq0 : 0);
    fil[NT + tid()] = flat_info<FE, RE>(nbd, rf1 - rf0);
    fil[2 * NT + tid()] = flat_info<FF, RF>(nbf, rd1 - rd0);
    for (int i = tid(); i < d; i += NT) {
        lnf[i] = a.lnw[i];
        lnf[d + i] = a.lnb[i];
    }

    unsigned g = a.g0;
    int tok = a.tok0, len = a.len0, prev = a.prev0, streak = a.streak0;
    int produced = 0;

    // Rows loaded a phase ahead by the compute waves: the S rows (this layer-0
    // self-attention output rows and V0) and the B1 rows of layer 0.
    Pre<TYPE, SO> pS;
    float obS, v0S[3];
    B1Item<TYPE> nb1;
    v0_load<TYPE>(v0S, a, ls[0]);
    obS = lane_bias<SO>(glob<gf>(ls[0].sob), o0, o1);
    prefetch<TYPE, SO, 1>(pS, uview(ls[0].so), nbd, o0, o1);
    if (has_item) stage_k(ls[0].crossK, a.enc_len, ih, t0, t1, kst);
    b1_item_prefetch<TYPE>(nb1, ls, 0, has_item, cq0, cq1, nbd);
    // V rows of this item's chunk for C (zeros elsewhere), issued a layer ahead with
    // the K rows: issued later, the wait before the score phase's LDS reads (which the
    // K rows' direct-to-LDS loads impose) would cover them too
    float4 vr[PVK];
    v_rows(vr, has_item, ls[0].crossV, a.enc_len, ih, t0, t1);

    for (int step = 0; step < a.n_steps; step++) {
        const int pos = len - 1;
        // ---------------- S: embedding, sa_0 rows ----------------
        {
            TRACE(step, 0, 7, 0);
            v0_store(v0S, v0, d);
            // token + positional embedding (decoder.go:756-773; quantised rows dequantised bit-exactly)
            for (int i = tid(); i < d; i += NT)
                xs[pad(i)] = dequant_elem<TYPE>(a.tok, tok, i >> 5, i & 31) + a.pos_emb[(size_t)pos * d + i];
            __syncthreads();
            for (int i = rd0 + tid(); i < rd1; i += NT) xl_own[i - rd0] = xs[pad(i)];
            {
                float out[SO];
                row_dots<TYPE, SO, 1>(pS, nbd, o0, o1, v0, out);
                post<SO>(obi, obv, lane_row<SO>(o0, o1), pick<SO>(out) + obS);
            }
            __syncthreads();
            TRACE(step, 0, 7, 2);
            ++g;
            if (comm()) flush<SO>(obi, obv, a.sa, g);
        }
        for (int l = 0; l < L; l++) {
            // layer 0: sa_0 carries phase gin (x_0 is local); later layers: x_l carries gin
            const unsigned gin = g;
            const MegaLayer &Ly = ls[l];
            Pre<TYPE, SD> pd;        // D's rows, loaded after C (items) or B1 (side)
            float cb;
            // ---------------- B1: cross q rows (items) / side rows ----------------
            TRACE(step, l, 1, 0);
            // items: x1 = x_l + sa_l (x_0 is local) for LN2, folded into the cross-query
            // rows (w2*x1 into xn; the statistics during the dots); side workgroups: x_l
            // LayerNormed (LN1) into xn
            float x1[XD];
            if (comm()) {
                if (has_item) {
                    float w2[XD];
                    ln_gain<XD>(w2, glob<gf>(Ly.ln2w), d);
                    if (l > 0) {
                        ll_load_scaled<XD, true>(x1, xn, a.xg, d, gin, a.err, w2, sav);
                    } else {
                        ll_load<XD, false>(sav, a.sa, d, gin, a.err);
                        const int lane = tid() & 63;
#pragma unroll
                        for (int k = 0; k < XD; k++) {
                            const int i = min(lane + 64 * k, d - 1);
                            x1[k] = xs[pad(i)] + sav[i];
                        }
                        store_scaled<XD>(x1, w2, d, xn);
                    }
                } else {
                    LnW<XD> lp;
                    ln_params<XD>(lp, glob<gf>(Ly.ln1w), glob<gf>(Ly.ln1b), d);
                    if (l > 0) {
                        ll_load_ln<XD, false>(xn, a.xg, d, gin, a.err, lp, nullptr);
                    } else {
                        const int lane = tid() & 63;
#pragma unroll
                        for (int k = 0; k < XD; k++) x1[k] = xs[pad(min(lane + 64 * k, d - 1))];
                        ln_wave<XD>(x1, d, lp, xn);
                        ll_load<XD, false>(sav, a.sa, d, gin, a.err);  // sa_0 for D
                    }
                }
                TRACE(step, l, 1, 1);
            }
            __syncthreads();
            ++g;
            const unsigned gB1 = g;  // items' cross-query rows; side workgroups' sa_{l+1} rows
            if (has_item) {
                float mean = 0.0f, rsd = 0.0f;
                {
                    float out[RQ];
                    flat_dots<TYPE, FQ, RQ>(nb1.pc, fil[tid()], xn, out);
                    if (comm()) ln_stats<XD>(x1, d, mean, rsd);
                    flat_post<RQ>(obv, out);
                }

                __syncthreads();
                TRACE(step, l, 1, 2);
                if (comm()) {
                    const int t = tid();
                    if (t < cq1 - cq0)
                        st_pair(&a.qx[cq0 + t], ln_fold(flat_sum(obv, fil[t]), mean, rsd, nb1.qc, nb1.qe), gB1);
                }
                prefetch<TYPE, SD, 1, 0>(pd, uview(Ly.co), nbd, 0, 0);  // zeros until C
                cb = 0.0f;
            } else {
                B1Side<TYPE> sp;
                b1_side_load<TYPE>(sp, a, ls, l, q0, q1, o0, o1, nbd);
                v0_store(sp.v0r, v0, d);
                __syncthreads();
                {
                    float out[SQ];
                    row_dots<TYPE, SQ, 1>(sp.pq, nbd, q0, q1, xn, out);
                    const float v = pick<SQ>(out);
                    const int r = lane_row<SQ>(q0, q1);
                    // rows [0,d) q (unused under the reference mask), [d,2d) k, [2d,3d) v; the
                    // cache rows are read only after the launch, so the compute lanes store them
                    if (r >= d) {
                        const int j = r % d, hh = j / 64, cidx = j % 64;
                        const bool isv = r >= 2 * d;  // sp.qb holds this lane's v bias then
                        gfw *kv = glob<gfw>(Ly.kv);
                        kv[(isv ? (size_t)H * a.ctx * 64 : 0) + (size_t)hh * a.ctx * 64 + (size_t)pos * 64 + cidx] =
                            isv ? v + sp.qb : v;
                    }
                }
                {
                    float out[SO];
                    row_dots<TYPE, SO, 1>(sp.po, nbd, o0, o1, v0, out);
                    post<SO>(obi, obv, l + 1 < L ? lane_row<SO>(o0, o1) : -1, pick<SO>(out) + sp.ob);
                }
                __syncthreads();
                TRACE(step, l, 1, 2);
                // sa_{l+1}, read in F of this layer
                if (comm()) flush<SO>(obi, obv, a.sa + (size_t)((l + 1) & 1) * d, gB1);
                // D's rows (B2 and C are item work)
                prefetch<TYPE, SD, 1>(pd, uview(Ly.co), nbd, rd0, rd1);
                cb = lane_bias<SD>(glob<gf>(Ly.cob), rd0, rd1);
            }
            // ---------------- B2: scores of the chunk against the head's q ----------------
            ++g;
            const unsigned gB = g;
            if (has_item) {
                const int lane = tid() & 63, wave = tid() >> 6;
                TRACE(step, l, 0, 0);
                if (comm()) {
                    ll_load<1, false>(qh, a.qx + ih * 64, 64, gB1, a.err);
                    TRACE(step, l, 0, 1);
                }
                k_wait();  // K rows staged in F
                __syncthreads();
                TRACEC(step, l, 0, 3);
                // 4 lanes per key, 16 elements each (four float4 chunks); key k of the chunk is
                // 128 j + (thread >> 2). A lane reads its chunks rotated by its quarter and by
                // the key's parity, so the 8 lanes of each LDS cycle (two keys) hit disjoint
                // banks; q is loaded in the same rotation. Keys past the chunk re-read its last
                // key: they rewrite that key's score and add nothing new to the maximum.
                {
                    const int tt = tid();
                    const int n = t1 - t0, kq = tt >> 2, e = tt & 3, rot = e + (kq & 1);
                    const float4 *q4 = (const float4 *)qh;
                    const float4 *k4 = (const float4 *)kst;
                    float4 qv[4];
#pragma unroll
                    for (int m = 0; m < 4; m++) qv[m] = q4[e * 4 + ((m + rot) & 3)];
                    float part[PKQ];
#pragma unroll
                    for (int j = 0; j < PKQ; j++) {
                        const int key = min(kq + 128 * j, n - 1);
                        float acc = 0.0f;
#pragma unroll
                        for (int m = 0; m < 4; m++) {
                            const float4 kr = k4[key * 16 + e * 4 + ((m + rot) & 3)];
                            acc += qv[m].x * kr.x + qv[m].y * kr.y + qv[m].z * kr.z + qv[m].w * kr.w;
                        }
                        part[j] = acc;
                    }
                    float mx = -INFINITY;
#pragma unroll
                    for (int j = 0; j < PKQ; j++) {
                        float v = part[j];
                        v += dpp<0xB1>(v);  // quad_perm [1,0,3,2]
                        v += dpp<0x4E>(v);  // quad_perm [2,3,0,1]
                        const float sj = v * a.scale;
                        if (e == 0) sc[min(kq + 128 * j, n - 1)] = sj;
                        mx = fmaxf(mx, sj);
                    }
                    mx = wave_max(mx);
                    if (lane == 0) red[wave] = mx;
                }
                TRACEC(step, l, 0, 4);
                __syncthreads();
                TRACE(step, l, 0, 2);
                if (comm() && tid() == 0) {
                    float m = red[0];
                    for (int i = 1; i < NW; i++) m = fmaxf(m, red[i]);
                    st_pair(&a.cmax[item], m, gB);
                }
                TRACEC(step, l, 0, 5);
            }
            // ---------------- C: softmax weights, partial P.V, head combine ----------------
            ++g;
            const unsigned gC = g;
            if (has_item) {
                const int lane = tid() & 63, cw = cwave();
                TRACE(step, l, 2, 0);
                if (comm()) {
                    // chunk maxima of the head
                    ll_load<1, false>(red + 40, a.cmax + ih * a.C, a.C, gB, a.err);
                    TRACE(step, l, 2, 1);
                    float M = red[40];
                    for (int i = 1; i < a.C; i++) M = fmaxf(M, red[40 + i]);
                    if (lane == 0) red[32] = M;
                }
                __syncthreads();
                {
                    // fast-exp weight of each key once (internal/ml/attention.go:34-131), in place of its score
                    const float M = red[32];
                    float es = 0.0f;
                    for (int t = tid(); t < t1 - t0; t += NT) {
                        const float e = fast_exp(sc[t] - M);
                        sc[t] = e;
                        es += e;
                    }
                    es = wave_sum(es);
                    if ((tid() & 63) == 0) red[48 + (tid() >> 6)] = es;
                }
                __syncthreads();
                if (cw >= 0) {
                    const unsigned c = (unsigned)ctid(), n = (unsigned)(t1 - t0);
                    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                    for (int j = 0; j < PVK; j++) {
                        // keys past the chunk (their V rows re-read the last key) add zero
                        const unsigned t = (unsigned)j * (NCT / 16) + (c >> 4);
                        const float e = t < n ? sc[min(t, n - 1u)] : 0.0f;
                        acc.x += e * vr[j].x; acc.y += e * vr[j].y; acc.z += e * vr[j].z; acc.w += e * vr[j].w;
                    }
#pragma unroll
                    for (int o = 16; o < 64; o <<= 1) {
                        acc.x += __shfl_xor(acc.x, o, 64);
                        acc.y += __shfl_xor(acc.y, o, 64);
                        acc.z += __shfl_xor(acc.z, o, 64);
                        acc.w += __shfl_xor(acc.w, o, 64);
                    }
                    float4 *red4 = (float4 *)xn;  // [NC][16]
                    if (lane < 16) red4[cw * 16 + lane] = acc;
                }
                __syncthreads();
                if (cw >= 0) {
                    // D's rows, while the communication wave combines
                    prefetch<TYPE, SD, 1>(pd, uview(Ly.co), nbd, rd0, rd1);
                    cb = lane_bias<SD>(glob<gf>(Ly.cob), rd0, rd1);
                } else {
                    const float4 *red4 = (const float4 *)xn;
                    uint64_t *pv = a.parts + (size_t)item * 65;
                    if (lane < 16) {
                        float4 r = red4[lane];
                        for (int v2 = 1; v2 < NC; v2++) {
                            const float4 t4 = red4[v2 * 16 + lane];
                            r.x += t4.x; r.y += t4.y; r.z += t4.z; r.w += t4.w;
                        }
                        st_pair(&pv[4 * lane], r.x, gC);
                        st_pair(&pv[4 * lane + 1], r.y, gC);
                        st_pair(&pv[4 * lane + 2], r.z, gC);
                        st_pair(&pv[4 * lane + 3], r.w, gC);
                    }
                    if (lane == 0) {
                        float s = 0.0f;
                        for (int v2 = 0; v2 < NW; v2++) s += red[48 + v2];
                        st_pair(&pv[64], s, gC);
                    }
                    if (ic == 0) {
                        // the head's first chunk combines the head: sum of the chunks' weight sums and P.V
                        ll_load<XP, false>(xp, a.parts + (size_t)ih * a.C * 65, a.C * 65, gC, a.err);
                        float sum = 0.0f, o = 0.0f;
                        for (int i = 0; i < a.C; i++) {
                            sum += xp[i * 65 + 64];
                            o += xp[i * 65 + lane];
                        }
                        st_pair(&a.attn[ih * 64 + lane], o * (1.0f / sum), gC);
                    }
                    TRACE(step, l, 2, 2);
                }
            }
            // ---------------- D: cross out rows -> x2 ----------------
            Pre<TYPE, FE> pe;
            float fcE, feE;
            {
                TRACE(step, l, 3, 0);
                if (comm()) {
                    ll_load<XD, true>(xn, a.attn, d, gC, a.err);
                    TRACE(step, l, 3, 1);
                }
                __syncthreads();
                {
                    float out[SD];
                    row_dots<TYPE, SD, 1>(pd, nbd, rd0, rd1, xn, out);
                    const float v = pick<SD>(out);
                    const int r = lane_row<SD>(rd0, rd1);
                    float x2 = 0.0f;
                    if (r >= 0) {
                        const float x1 = xl_own[r - rd0] + sav[r];
                        x2 = x1 + (v + cb);
                        x2_own[r - rd0] = x2;
                    }
                    post<SD>(obi, obv, r, x2);
                }
                __syncthreads();
                TRACE(step, l, 3, 2);
                ++g;
                if (comm()) flush<SD>(obi, obv, a.x2, g);
                // E's bias and rows
                fcE = comm_bias(glob<gf>(Ly.f1c), rf0, rf1);
                feE = comm_bias(glob<gf>(Ly.f1e), rf0, rf1);
                flat_prefetch<TYPE, FE>(pe, uview(Ly.fc1), nbd, rf0, rf1 - rf0, true);
            }
            const unsigned gD = g;
            // ---------------- E: LN3 + fc1 + GELU ----------------
            Pre<TYPE, FF> pf;
            float fbF;
            {
                TRACE(step, l, 4, 0);
                // x2 for LN3, folded into the fc1 rows (w3*x2 into xn; the statistics during the dots)
                float x2v[XD];
                if (comm()) {
                    float w3[XD];
                    ln_gain<XD>(w3, glob<gf>(Ly.ln3w), d);
                    ll_load_scaled<XD, false>(x2v, xn, a.x2, d, gD, a.err, w3, nullptr);
                    TRACE(step, l, 4, 1);
                }
                __syncthreads();
                TRACE(step, l, 4, 3);
                TRACE(step, l, 4, 4);
                TRACEC(step, l, 4, 7);
                float mean = 0.0f, rsd = 0.0f;
                {
                    float out[RE];
                    flat_dots<TYPE, FE, RE>(pe, fil[NT + tid()], xn, out);
                    TRACEC(step, l, 4, 5);
                    if (comm()) ln_stats<XD>(x2v, d, mean, rsd);
                    flat_post<RE>(obv, out);
                }
                __syncthreads();
                TRACE(step, l, 4, 2);
                ++g;
                if (comm()) {
                    const int t = tid();
                    if (t < rf1 - rf0)
                        st_pair(&a.hbuf[rf0 + t], gelu_f32(ln_fold(flat_sum(obv, fil[NT + t]), mean, rsd, fcE, feE)), g);
                }
                TRACE(step, l, 4, 6);
                // F's bias and rows
                fbF = comm_bias(glob<gf>(Ly.fc2b), rd0, rd1);
                flat_prefetch<TYPE, FF>(pf, uview(Ly.fc2), nbf, rd0, rd1 - rd0, true);
            }
            const unsigned gE = g;
            // ---------------- F: fc2 rows -> x_{l+1} ----------------
            {
                TRACE(step, l, 5, 0);
                // h (12 pairs per lane) and sa_{l+1} (3 per lane; published long ago, its
                // loads ride along) by the compute waves
                if (!comm()) {
                    if (l + 1 < L)
                        ll_load2<XH, true, XS>(xn, a.hbuf, 4 * d, gE, cwave() * 64 * XH, sav,
                                               a.sa + (size_t)((l + 1) & 1) * d, d, gB1, cwave() * 64 * XS, a.err);
                    else
                        ll_load<XH, true>(xn, a.hbuf, 4 * d, gE, a.err, cwave() * 64 * XH);
                    TRACEC(step, l, 5, 4);
                }
                TRACE(step, l, 5, 1);
                __syncthreads();
                TRACE(step, l, 5, 3);
                {
                    float out[RF];
                    flat_dots<TYPE, FF, RF>(pf, fil[2 * NT + tid()], xn, out);
                    TRACEC(step, l, 5, 5);
                    flat_post<RF>(obv, out);
                }
                __syncthreads();
                TRACE(step, l, 5, 2);
                ++g;
                if (comm()) {
                    // x_{l+1} = x2 + (fc2 + b); D of the next layer reads the own rows
                    const int t = tid();
                    if (t < rd1 - rd0) {
                        const float x = x2_own[t] + (flat_sum(obv, fil[2 * NT + t]) + fbF);
                        xl_own[t] = x;
                        st_pair(&a.xg[rd0 + t], x, g);
                    }
                }
                TRACE(step, l, 5, 6);
                if (l + 1 < L) {
                    // the next layer's K rows (this layer's were consumed in B2), its B1 rows,
                    // then its V rows (C)
                    if (has_item) stage_k(ls[l + 1].crossK, a.enc_len, ih, t0, t1, kst);
                    b1_item_prefetch<TYPE>(nb1, ls, l + 1, has_item, cq0, cq1, nbd);
                    v_rows(vr, has_item, ls[l + 1].crossV, a.enc_len, ih, t0, t1);
                }
            }
        }
        const unsigned gF = g;
        // ---------------- T: final LN, logits rows, penalty, argmax ----------------
        {
            const int lane = tid() & 63, cw = cwave();
            TRACE(step, L, 6, 0);
            const UView vt = uview(a.tok);
            Pre<TYPE, TS> p0, p1;
            const int CH = NC * TS;
            prefetch<TYPE, TS, 1>(p0, vt, nbd, rv0, min(rv0 + CH, rv1));
            if (comm()) {
                for (int i = tid(); i < rv1 - rv0; i += 64) pen[i] = 0;
                if (tid() == 0) eotf = 0;
                // repetition window (decoder.go:1000-1016): counts of this workgroup's rows
                const int start = len > 128 ? len - 128 : 0, nwin = len - start;
                for (int i = tid(); i < nwin; i += 64) {
                    const int id = hl[(start + i) & 127];
                    if (id >= rv0 && id < rv1) atomicAdd(&pen[id - rv0], 1);
                }
                // the final LayerNorm's parameters come from LDS: registers are short here
                ll_load_ln_lds<XD>(xn, a.xg, d, gF, a.err, lnf, lnf + d);
                TRACE(step, L, 6, 1);
            }
            __syncthreads();
            TRACE(step, L, 6, 3);
            TRACE(step, L, 6, 4);
            float bv = -INFINITY, bv2 = -INFINITY;
            int bi = 0x7FFFFFFF, bi2 = 0x7FFFFFFF;
            float ev = -INFINITY;
            for (int base = rv0; base < rv1; base += 2 * CH) {
                const int b1 = base + CH;
                prefetch<TYPE, TS, 1>(p1, vt, nbd, min(b1, rv1 - 1), min(b1 + CH, rv1));
                logits_chunk<TYPE>(a, p0, nbd, base, min(base + CH, rv1), xn, pen, rv0, bv, bi, bv2, bi2, &ev);
                if (b1 < rv1) {
                    const int b2 = b1 + CH;
                    prefetch<TYPE, TS, 1>(p0, vt, nbd, min(b2, rv1 - 1), min(b2 + CH, rv1));
                    logits_chunk<TYPE>(a, p1, nbd, b1, min(b1 + CH, rv1), xn, pen, rv0, bv, bi, bv2, bi2, &ev);
                }
            }
            TRACE(step, L, 6, 5);
            float *rv = red;
            float *rv2 = red + NC;
            int *ri = (int *)(red + 2 * NC), *ri2 = (int *)(red + 3 * NC);
            if (cw >= 0 && lane == 0) {
                rv[cw] = bv; ri[cw] = bi; rv2[cw] = bv2; ri2[cw] = bi2;
                if (ev != -INFINITY) {
                    eotv = ev;
                    eotf = 1;
                }
            }
            __syncthreads();
            const unsigned gT = g + 1;
            if (comm()) {
                if (tid() == 0) {
                    for (int i = 1; i < NC; i++) {
                        better(rv[i], ri[i], rv[0], ri[0]);
                        better(rv2[i], ri2[i], rv2[0], ri2[0]);
                    }
                    st_pair(&a.part[4 * w], rv[0], gT);
                    st_pair(&a.part[4 * w + 1], __int_as_float(ri[0]), gT);
                    st_pair(&a.part[4 * w + 2], rv2[0], gT);
                    st_pair(&a.part[4 * w + 3], __int_as_float(ri2[0]), gT);
                    if (eotf) st_pair(a.eot_logit, eotv, gT);
                }
                TRACE(step, L, 6, 2);
                ll_load<XT, false>(xp, a.part, 4 * W, gT, a.err);
                TRACE(step, L, 6, 6);
                // every workgroup reduces the partials the same way
                float b1 = -INFINITY, b2 = -INFINITY;
                int i1 = 0x7FFFFFFF, i2 = 0x7FFFFFFF;
                for (int i = tid(); i < W; i += 64) {
                    better(xp[4 * i], __float_as_int(xp[4 * i + 1]), b1, i1);
                    better(xp[4 * i + 2], __float_as_int(xp[4 * i + 3]), b2, i2);
                }
                for (int o = 32; o > 0; o >>= 1) {
                    float ov = __shfl_xor(b1, o, 64);
                    int oi = __shfl_xor(i1, o, 64);
                    better(ov, oi, b1, i1);
                    ov = __shfl_xor(b2, o, 64);
                    oi = __shfl_xor(i2, o, 64);
                    better(ov, oi, b2, i2);
                }
                int id = (i1 == 0x7FFFFFFF) ? 0 : i1;
                if (a.suppress_nst && a.eot >= 0 && a.eot < a.V && id == a.eot) {
                    ll_load<1, false>(xp, a.eot_logit, 1, gT, a.err);
                    if (xp[0] < -a.nst) id = (i2 == 0x7FFFFFFF) ? a.eot : i2;
                }
                if (tid() == 0) red[63] = __int_as_float(id);
            }
            // the next step's S and B1 rows and its first K rows (the communication wave, done
            // with its part, fills zeros)
            v0_load<TYPE>(v0S, a, ls[0]);
            obS = lane_bias<SO>(glob<gf>(ls[0].sob), o0, o1);
            prefetch<TYPE, SO, 1>(pS, uview(ls[0].so), nbd, o0, o1);
            if (has_item) stage_k(ls[0].crossK, a.enc_len, ih, t0, t1, kst);
            b1_item_prefetch<TYPE>(nb1, ls, 0, has_item, cq0, cq1, nbd);
            v_rows(vr, has_item, ls[0].crossV, a.enc_len, ih, t0, t1);
            g = gT;
            __syncthreads();
            tok = __float_as_int(red[63]);
            __syncthreads();
        }
        // history append and the reference's stop rules (decoder.go:462-484)
        if (tid() == 0) hl[len & 127] = tok;
        if (w == 0 && tid() == 0) {
            a.hist[len] = tok;
            a.out_tokens[produced] = tok;
        }
        len++;
        produced++;
        bool stop = (tok == a.eot) || (len >= a.max_len);
        if (prev == tok) streak++;
        else { streak = 1; prev = tok; }
        if (streak > 20) stop = true;
        if (stop || ld_u(a.err)) break;
    }
    if (w == 0 && tid() == 0) {
        a.state_out[0] = produced;
        a.state_out[1] = prev;
        a.state_out[2] = streak;
        a.state_out[3] = (int)g;
    }
}

#ifdef WH_MEGA_TRACE
extern "C" int wh_mega_trace_read(void *out, size_t bytes) {
    if (bytes > sizeof(g_trace)) bytes = sizeof(g_trace);
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(g_trace), bytes, 0, hipMemcpyDeviceToHost) == hipSuccess ? 0 : -2;
}
#endif

size_t lds_bytes(int d, int L, int V, int W, int chunk_len) {
    const int d36 = ((d + 31) / 32) * 36;
    return sizeof(float) * (size_t)(layer_floats(L) + 6 * d36 + d + 64 * 4 + 2 * OUTBOX + 64 * XT + 128 +
                                    SC_FLOATS + pen_floats(V, W) + chunk_len * 64 + 3 * NT + 2 * d);
}

__global__ void k_coop_warm() {}

// The runtime loads a kernel's code object on its first use and sets up its
// cooperative launches on the first one, which the first token would otherwise
// pay for (~6 ms): asking for the kernel's attributes and one empty cooperative
// launch at model creation do both there. Unsupported types are left alone.
int warm_decode(uint32_t type) {
    const void *fn = nullptr;
    switch (type) {
    case 2: fn = (const void *)k_decode<2>; break;
    case 3: fn = (const void *)k_decode<3>; break;
    case 6: fn = (const void *)k_decode<6>; break;
    case 7: fn = (const void *)k_decode<7>; break;
    case 8: fn = (const void *)k_decode<8>; break;
    default: return WH_OK;
    }
    hipFuncAttributes attr;
    WH_HIP(hipFuncGetAttributes(&attr, fn));
    WH_HIP(hipLaunchCooperativeKernel((const void *)k_coop_warm, dim3(1), dim3(64), nullptr, 0, nullptr));
    WH_HIP(hipDeviceSynchronize());
    return WH_OK;
}

int launch_decode(uint32_t type, int grid, const MegaArgs &a, hipStream_t st) {
    void *args[] = {(void *)&a};
    const size_t shmem = lds_bytes(a.d, a.L, a.V, grid, a.chunk_len);
    const void *fn = nullptr;
    switch (type) {
    case 2: fn = (const void *)k_decode<2>; break;
    case 3: fn = (const void *)k_decode<3>; break;
    case 6: fn = (const void *)k_decode<6>; break;
    case 7: fn = (const void *)k_decode<7>; break;
    case 8: fn = (const void *)k_decode<8>; break;
    default: return fail(WH_ERR_UNSUPPORTED, "persistent decode: unsupported weight type");
    }
    WH_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shmem));
    WH_HIP(hipLaunchCooperativeKernel(fn, dim3(grid), dim3(NT), args, shmem, st));
    return WH_OK;
}

}  // namespace mega
}  // namespace wh
